"""Parity at the full sequence lengths of configs C (131072 keys, causal, GQA,
chunks of 32768), D (32760 keys, non-causal, one group per row, two-pass split
selection, a 56-row last q-block) and E (119056 keys, non-causal, two-pass
split selection), on a subset of heads (heads are independent: one kv group
of C, two heads of D and of E).  Run on an MI355X.

- gap 1e6 selects every selectable key: counts equal the closed form, through
  the split (segmented) selection that VecAttention_prefill runs;
- sampled rows: the split selection's lists (the ones the prefill's attention
  reads) equal the oracle's bit for bit, at the threshold calibrated to the
  workload's keep ratio and at a fixed one, and the prefill output of those
  rows is within the north-star tolerance of the oracle;
- the two-pass split selection equals the exact fp64 kernel on every row of a
  chunk;
- every row of one chunk (all heads of the subset) equals the oracle's list;
- chunk-size invariance where the reference's rule makes it hold;
- with all 28 heads of C, the prefill's causal row groups (the index buffer
  holds one group of a chunk at a time) give the same output as whole chunks.
"""
import math
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from seglists import calibrate_threshold, check_rows, pooled_oracle, select_chunk
from vecattention_amd import VecAttention_prefill
from vecattention_amd import _native as nat
from vecattention_amd import stages
from vecattention_amd.synth import WORKLOADS, make_inputs

pytestmark = pytest.mark.gpu

ATOL_MAX, ATOL_MEAN = 2e-2, 2e-3
DEV = "cuda:0"


def note(*a):
    print("[case]", *a, flush=True)


def segment_totals(counts):
    return counts.sum(dim=-1)


def check_every_row(q, k, qs_dev, kd, J0, nc, th, causal, G, heads, rep=1, qps=64, bk=16):
    """Every row J0..J0+nc-1 of every head in `heads`: the split selection's
    list equals the oracle's bit for bit (heads in parallel threads; the
    oracle's C selection releases the interpreter lock)."""
    gap = -math.log(th + 1e-9)
    gaps = orc.gap_from_threshold(th, 1, 1)
    gpu = select_chunk(qs_dev, kd, J0, nc, gap, causal, qps, bk, G)

    def head(h):
        qs = pooled_oracle(q[:, h:h + 1], qps)
        cnt, lists = orc.select(qs, k[:, h // rep:h // rep + 1], J0, nc, gaps, qps, bk, G,
                                causal, causal, 64)
        bad = [J for J in range(nc) if not np.array_equal(gpu.row(0, h, J), lists[0][0][J])]
        return h, int(cnt.sum()), bad

    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as ex:
        results = list(ex.map(head, heads))
    for h, total, bad in results:
        assert total > 0, h
        assert not bad, f"h={h}: rows {[J0 + J for J in bad[:10]]} differ"
    return sum(t for _, t, _ in results)


# ------------------------------------------------------------------ config C --

@pytest.fixture(scope="module")
def config_c():
    # one kv group of C: 7 q heads over 1 kv head, 131072 keys
    q, k, v = make_inputs(1, 7, 1, 131072, 128, torch.bfloat16, seed=0)
    qd = q.to(DEV)
    qs, _ = stages.pool_scaled(qd, 64)
    return q, k, v, qd, k.to(DEV), v.to(DEV), qs


def test_c_large_gap_selects_every_selectable_key(config_c):
    note("C all selectable")
    _, _, _, qd, kd, _, qs = config_c
    qps, S = 64, 131072
    segk = stages.segment_keys(S, 16, 16)
    for J0 in (0, 1536):  # first and last 32K chunk
        cnt, _ = stages.select_segments(qs[:, :, J0:J0 + 512], kd, J0, 1e6, None, True, qps, 16,
                                        16, True, segk)
        J = torch.arange(J0, J0 + 512)
        # every key before the row's q-block except [0, qps), minus the 48 keys
        # the first row of each 64-row program rejects
        want = torch.clamp((J - 1) * qps, min=0) - torch.where((J % 64 == 0) & (J >= 2), 48, 0)
        assert torch.equal(segment_totals(cnt).cpu(), want.to(torch.int64).expand(1, 7, 512))


@pytest.mark.parametrize("th", ["calibrated", 0.84])
def test_c_sampled_rows_match_oracle(config_c, th):
    q, k, v, qd, kd, vd, qs = config_c
    if th == "calibrated":
        th = calibrate_threshold(qs, kd, True, 64, 16, 16, WORKLOADS["C"].keep)
    note("C sampled rows, threshold", th)
    out = VecAttention_prefill(qd, kd, vd, th, 64, 16, 16, True, 32768)
    torch.cuda.synchronize()
    out_cpu = out.float().cpu().numpy()
    rng = np.random.default_rng(1)
    # rows of the first and the last chunk; 0 and 64 are first rows of a
    # program (the causal first-row rule), 2047 is the longest row
    rows = [1, 64] + sorted(rng.choice(np.arange(1536, 2048), 3, replace=False).tolist()) + [2047]
    check_rows(q, k, v, qs, kd, out_cpu, (0, 6), rows, th, True, 16, rep=7)


def test_c_last_chunk_every_row_matches_oracle(config_c):
    # the longest rows (96K..128K keys), all 7 heads of the kv group
    q, k, _, _, kd, _, qs = config_c
    note("C every row of the last chunk")
    check_every_row(q, k, qs, kd, 1536, 512, 0.84, True, 16, range(7), rep=7)


def test_c_chunking_invariant(config_c):
    # 16K and 32K chunks both start programs at multiples of 64 q-blocks
    note("C chunk invariance")
    _, _, _, qd, kd, vd, _ = config_c
    a = VecAttention_prefill(qd, kd, vd, 0.84, 64, 16, 16, True, 32768)
    b = VecAttention_prefill(qd, kd, vd, 0.84, 64, 16, 16, True, 16384)
    assert torch.equal(a, b)


def test_c_all_heads_row_groups_equal_whole_chunks():
    # All 28 q heads of C: VecAttention_prefill holds the lists of one row
    # group of a chunk at a time (the last chunk's whole index capacity, 6.2
    # GiB, exceeds its budget), the stage path below selects and attends whole
    # chunks.  Groups start at multiples of BLOCK_SIZE_Q from the chunk origin,
    # so the lists and therefore the outputs are identical.
    note("C all heads: row groups == whole chunks")
    wl = WORKLOADS["C"]
    q, k, v = make_inputs(1, 28, 4, 131072, 128, torch.bfloat16, seed=1)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    del q, k, v
    th = 0.8385383879401624
    out = VecAttention_prefill(qd, kd, vd, th, 64, 16, 16, True, wl.chunk_size)
    ref = torch.empty_like(qd)
    qs, _ = stages.pool_scaled(qd, 64)
    segk = stages.segment_keys(131072, 16, 16)
    gap = -math.log(th + 1e-9)
    for J0 in range(0, 2048, 512):
        cnt, idx = stages.select_segments(qs[:, :, J0:J0 + 512], kd, J0, gap, None, True, 64, 16, 16,
                                          True, segk)
        stages.sparse_attention(qd, kd, vd, ref, J0, 512, cnt, idx, True, 64, segk=segk)
        del cnt, idx
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


# ------------------------------------------------------------------ config D --

@pytest.fixture(scope="module")
def config_d():
    # two heads of D: 32760 keys (21 frames of 1560 tokens), 512 q-blocks, the
    # last of 56 rows
    q, k, v = make_inputs(1, 2, 2, 32760, 128, torch.bfloat16, seed=0, frames=(21, 1560))
    qd = q.to(DEV)
    qs, _ = stages.pool_scaled(qd, 64)
    return q, k, v, qd, k.to(DEV), v.to(DEV), qs


def test_d_runs_two_pass_split():
    # one group per row (G*BK >= Sk): the segments carry the running maximum
    segk = stages.segment_keys(32760, 16, 8192)
    assert segk == 2048
    assert 16 * 8192 >= 32760


def test_d_large_gap_selects_every_key(config_d):
    note("D all keys")
    _, _, _, _, kd, _, qs = config_d
    S = 32760
    segk = stages.segment_keys(S, 16, 8192)
    cnt, _ = stages.select_segments(qs, kd, 0, 1e6, None, False, 64, 16, 8192, False, segk)
    assert torch.equal(segment_totals(cnt).cpu(), torch.full((1, 2, 512), S, dtype=torch.int64))


@pytest.mark.parametrize("th", ["calibrated", 0.3])
def test_d_sampled_rows_match_oracle(config_d, th):
    q, k, v, qd, kd, vd, qs = config_d
    if th == "calibrated":
        th = calibrate_threshold(qs, kd, False, 64, 16, 8192, WORKLOADS["D"].keep)
    note("D sampled rows, threshold", th)
    out = VecAttention_prefill(qd, kd, vd, th, 64, 16, 8192, False, 32768)
    torch.cuda.synchronize()
    out_cpu = out.float().cpu().numpy()
    rng = np.random.default_rng(2)
    rows = [0] + sorted(rng.choice(np.arange(1, 511), 5, replace=False).tolist()) + [511]
    check_rows(q, k, v, qs, kd, out_cpu, (0, 1), rows, th, False, 8192)


def test_d_every_row_matches_oracle(config_d):
    q, k, _, _, kd, _, qs = config_d
    note("D every row")
    check_every_row(q, k, qs, kd, 0, 512, 0.3, False, 8192, range(2))


def test_d_split_selection_equals_exact_kernel(config_d):
    note("D split == exact")
    _, _, _, _, kd, _, qs = config_d
    S = 32760
    gap = -math.log(0.3 + 1e-9)
    segk = stages.segment_keys(S, 16, 8192)
    c1, i1 = stages.select_rows(qs, kd, 0, gap, None, False, 64, 16, 8192, False,
                                kernel=nat.VA_SEL_EXACT)
    c2, i2 = stages.select_segments(qs, kd, 0, gap, None, False, 64, 16, 8192, False, segk)
    c1n, c2n = c1.cpu().numpy(), c2.cpu().numpy()
    assert np.array_equal(c1n, c2n.sum(axis=-1))
    a, b = i1.cpu().numpy(), i2.cpu().numpy()
    nseg = c2n.shape[-1]
    for h in range(2):
        for jr in range(512):
            o = stages.row_offset(S, 64, False, False, 0, 512, h, jr)
            split = np.concatenate([b[o + s * segk:o + s * segk + c2n[0, h, jr, s]]
                                    for s in range(nseg)])
            assert np.array_equal(a[o:o + c1n[0, h, jr]], split), (h, jr)


# ------------------------------------------------------------------ config E --

@pytest.fixture(scope="module")
def config_e():
    # two heads of E: 119056 keys, text tokens last, 33 frames of 3600 tokens
    q, k, v = make_inputs(1, 2, 2, 119056, 128, torch.bfloat16, seed=0, sinks="text_last",
                          frames=(33, 3600), text_tokens=256)
    qd = q.to(DEV)
    qs, _ = stages.pool_scaled(qd, 64)
    return q, k, v, qd, k.to(DEV), v.to(DEV), qs


def test_e_large_gap_selects_every_key(config_e):
    note("E all keys")
    _, _, _, _, kd, _, qs = config_e
    qps, S = 64, 119056
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
    _, _, _, _, kd, _, qs = config_e
    qps, S = 64, 119056
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


@pytest.mark.parametrize("th", ["calibrated", 0.43])
def test_e_sampled_rows_match_oracle(config_e, th):
    q, k, v, qd, kd, vd, qs = config_e
    if th == "calibrated":
        th = calibrate_threshold(qs, kd, False, 64, 16, 8192, WORKLOADS["E"].keep)
    note("E sampled rows, threshold", th)
    out = VecAttention_prefill(qd, kd, vd, th, 64, 16, 8192, False, 32768)
    torch.cuda.synchronize()
    out_cpu = out.float().cpu().numpy()
    nqb = qs.shape[2]
    check_rows(q, k, v, qs, kd, out_cpu, (0, 1), [0, 700, 1537, nqb - 1], th, False, 8192)


def test_e_last_chunk_every_row_matches_oracle(config_e):
    q, k, _, _, kd, _, qs = config_e
    note("E every row of the last chunk")
    nqb = qs.shape[2]
    check_every_row(q, k, qs, kd, 1536, nqb - 1536, 0.43, False, 8192, range(2))
