"""Size-independent properties at the full sequence lengths of configs C
(131072 keys, causal, GQA, chunks of 32768) and E (119056 keys, non-causal,
one group per row, two-pass split selection), on a subset of heads (heads are
independent: one kv group of C, two heads of E).  Run on an MI355X.

- gap 1e6 selects every selectable key: counts equal the closed form, through
  the split (segmented) selection that VecAttention_prefill runs;
- sampled rows of the full prefill: selection bit-exact and attention within
  the north-star tolerance of the oracle;
- the certified split selection equals the exact fp64 kernel on every row of
  a chunk;
- chunk-size invariance where the reference's rule makes it hold.
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from vecattention_amd import VecAttention_prefill
from vecattention_amd import _native as nat
from vecattention_amd import stages
from vecattention_amd.synth import make_inputs

pytestmark = pytest.mark.gpu

ATOL_MAX, ATOL_MEAN = 2e-2, 2e-3
DEV = "cuda:0"


def note(*a):
    print("[case]", *a, flush=True)


def segment_totals(counts):
    return counts.sum(dim=-1)


@pytest.fixture(scope="module")
def config_c():
    # one kv group of C: 7 q heads over 1 kv head, 131072 keys
    q, k, v = make_inputs(1, 7, 1, 131072, 128, torch.bfloat16, seed=0)
    return q, k, v, q.to(DEV), k.to(DEV), v.to(DEV)


@pytest.fixture(scope="module")
def config_e():
    # two heads of E: 119056 keys, text tokens last, 33 frames of 3600 tokens
    q, k, v = make_inputs(1, 2, 2, 119056, 128, torch.bfloat16, seed=0, sinks="text_last",
                          frames=(33, 3600), text_tokens=256)
    return q, k, v, q.to(DEV), k.to(DEV), v.to(DEV)


def test_c_large_gap_selects_every_selectable_key(config_c):
    note("C all selectable")
    _, _, _, qd, kd, _ = config_c
    qps, S = 64, 131072
    qs, _ = stages.pool_scaled(qd, qps)
    segk = stages.segment_keys(S, 16, 16)
    for J0 in (0, 1536):  # first and last 32K chunk
        cnt, _ = stages.select_segments(qs[:, :, J0:J0 + 512], kd, J0, 1e6, None, True, qps, 16,
                                        16, True, segk)
        J = torch.arange(J0, J0 + 512)
        # every key before the row's q-block except [0, qps), minus the 48 keys
        # the first row of each 64-row program rejects
        want = torch.clamp((J - 1) * qps, min=0) - torch.where((J % 64 == 0) & (J >= 2), 48, 0)
        assert torch.equal(segment_totals(cnt).cpu(), want.to(torch.int64).expand(1, 7, 512))


def test_c_sampled_rows_match_oracle(config_c):
    note("C sampled rows")
    q, k, v, qd, kd, vd = config_c
    qps, S, th = 64, 131072, 0.84
    out = VecAttention_prefill(qd, kd, vd, th, qps, 16, 16, True, 32768)
    torch.cuda.synchronize()
    out_cpu = out.float().cpu().numpy()
    gaps = orc.gap_from_threshold(th, 1, 1)
    rng = np.random.default_rng(1)
    for h in (0, 6):
        qh = q[:, h:h + 1]
        _, qs = orc.pool(qh, qps, "bfloat16")
        for J in sorted(rng.choice(np.arange(1536, 2048), 3, replace=False).tolist()) + [2047]:
            _, lists = orc.select(qs, k, 1536, 512, gaps, qps, 16, 16, True, True, 64,
                                  rows=(J - 1536, J - 1535))
            bc, bi = orc.local_blocks(1, 1, S, qps, True)
            row = lists[0][0][J - 1536]
            want = orc.attention(qh, k, v, qps, True, bc, bi, [[[row]]], J0=J, nc=1)
            err = np.abs(out_cpu[0, h, J * qps:(J + 1) * qps] - want[0, 0])
            assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN, (h, J, err.max())


def test_c_chunking_invariant(config_c):
    # 16K and 32K chunks both start programs at multiples of 64 q-blocks
    note("C chunk invariance")
    _, _, _, qd, kd, vd = config_c
    a = VecAttention_prefill(qd, kd, vd, 0.84, 64, 16, 16, True, 32768)
    b = VecAttention_prefill(qd, kd, vd, 0.84, 64, 16, 16, True, 16384)
    assert torch.equal(a, b)


def test_e_large_gap_selects_every_key(config_e):
    note("E all keys")
    _, _, _, qd, kd, _ = config_e
    qps, S = 64, 119056
    qs, _ = stages.pool_scaled(qd, qps)
    segk = stages.segment_keys(S, 16, 8192)
    nqb = qs.shape[2]
    for J0 in (0, 1536):  # the first chunk and the partial last one
        nc = min(512, nqb - J0)
        cnt, _ = stages.select_segments(qs[:, :, J0:J0 + nc], kd, J0, 1e6, None, False, qps, 16,
                                        8192, False, segk)
        assert torch.equal(segment_totals(cnt).cpu(), torch.full((1, 2, nc), S, dtype=torch.int64))


def test_e_split_selection_equals_exact_kernel(config_e):
    # the two-pass split selection (maxima pass + carry pass) against the fp64
    # kernel on every row of the last chunk, as index sets per row
    note("E split == exact")
    _, _, _, qd, kd, _ = config_e
    qps, S = 64, 119056
    qs, _ = stages.pool_scaled(qd, qps)
    nqb = qs.shape[2]
    J0 = 3 * 512
    nc = nqb - J0
    gap = -math.log(0.43 + 1e-9)
    segk = stages.segment_keys(S, 16, 8192)
    c1, i1 = stages.select_rows(qs[:, :, J0:], kd, J0, gap, None, False, qps, 16, 8192, False,
                                kernel=nat.VA_SEL_EXACT)
    c2, i2 = stages.select_segments(qs[:, :, J0:], kd, J0, gap, None, False, qps, 16, 8192, False,
                                    segk)
    c1n, c2n = c1.cpu().numpy(), c2.cpu().numpy()
    assert np.array_equal(c1n, c2n.sum(axis=-1))
    a, b = i1.cpu().numpy(), i2.cpu().numpy()
    nseg = c2n.shape[-1]
    for h in range(2):
        for jr in range(nc):
            o = stages.row_offset(S, qps, False, False, J0, nc, h, jr)
            exact = a[o:o + c1n[0, h, jr]]
            split = np.concatenate([b[o + s * segk:o + s * segk + c2n[0, h, jr, s]]
                                    for s in range(nseg)])
            assert np.array_equal(exact, split), (h, jr)


def test_e_sampled_rows_match_oracle(config_e):
    note("E sampled rows")
    q, k, v, qd, kd, vd = config_e
    qps, S, th = 64, 119056, 0.43
    out = VecAttention_prefill(qd, kd, vd, th, qps, 16, 8192, False, 32768)
    torch.cuda.synchronize()
    out_cpu = out.float().cpu().numpy()
    gaps = orc.gap_from_threshold(th, 1, 1)
    nqb = -(-S // qps)
    bc, bi = orc.local_blocks(1, 1, S, qps, False)
    for h in (0, 1):
        qh, kh, vh = q[:, h:h + 1], k[:, h:h + 1], v[:, h:h + 1]
        _, qs = orc.pool(qh, qps, "bfloat16")
        for J in (0, 700, 1537, nqb - 1):
            J0 = (J // 512) * 512
            nc = min(512, nqb - J0)
            _, lists = orc.select(qs, kh, J0, nc, gaps, qps, 16, 8192, False, False, 64,
                                  rows=(J - J0, J - J0 + 1))
            row = lists[0][0][J - J0]
            want = orc.attention(qh, kh, vh, qps, False, bc, bi, [[[row]]], J0=J, nc=1)
            r0, r1 = J * qps, min(S, (J + 1) * qps)
            err = np.abs(out_cpu[0, h, r0:r1] - want[0, 0])
            assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN, (h, J, err.max())
