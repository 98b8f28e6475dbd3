"""GPU parity of the paired lists and the attention's pair form (the layout
va_prefill runs for bf16/fp16, head_dim 128, q_pooling_size 64).

- va_select_segments_paired: within each key segment, row A = chunk row 2i
  holds the keys both rows of the pair selected (ascending from the segment's
  first slot) and its own keys (descending from the segment's last slot), row
  B = 2i+1 its own keys (ascending); pair_common counts the shared keys.  The
  lists are cut here with the oracle's own capacity arithmetic and must give
  back each row's list bit for bit (the oracle's), with the shared keys
  exactly the intersection.
- va_sparse_attn_segments_paired: within the north-star tolerance of the
  oracle's float64 attention on the same lists.
Every call goes through the C ABI of libvecattn.so.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from vecattention_amd import VecAttention_prefill
from vecattention_amd import stages
from vecattention_amd.synth import make_inputs

pytestmark = pytest.mark.gpu

ATOL_MAX, ATOL_MEAN = 2e-2, 2e-3
DTN = {torch.bfloat16: "bfloat16", torch.float16: "float16"}


def note(*a):
    print("[case]", *a, flush=True)


def paired_rows(counts, indices, pair_common, J0, nc, qps, Sk, causal, wo_init, segk, b, h, Hq):
    """Per-row lists of one (b, h) decoded from the paired layout, with checks
    of the layout itself (runs inside their segment's slots and key range,
    run orders, shared keys in both rows only once)."""
    cnt = counts.cpu().numpy()
    pc = pair_common.cpu().numpy()
    idx = indices.cpu().numpy().reshape(-1)
    nseg = cnt.shape[-1]
    smin = (qps if causal else min(qps, Sk)) if wo_init else 0
    caps = [orc.row_capacity(J0 + jr, qps, Sk, causal, wo_init) for jr in range(nc)]
    block = sum(caps)
    starts = np.concatenate([[0], np.cumsum(caps)[:-1]]).astype(np.int64)
    base = (b * Hq + h) * block

    def seg_first(s):
        return max(s * segk, smin) - smin

    rows = [None] * nc
    for p in range((nc + 1) // 2):
        ja, jb = 2 * p, 2 * p + 1
        oa = base + int(starts[ja])
        ob = base + int(starts[jb]) if jb < nc else None
        ra, rb = [], []
        for s in range(nseg):
            lo, hi = s * segk, min((s + 1) * segk, Sk)
            s0 = seg_first(s)
            nxt = seg_first(s + 1) if s + 1 < nseg else 1 << 40
            end_a = min(nxt, caps[ja])
            ca = int(cnt[b, h, ja, s])
            c = int(pc[b, h, p, s])
            assert 0 <= c <= ca and s0 + ca <= max(end_a, s0), (p, s, c, ca)
            common = idx[oa + s0:oa + s0 + c]
            a_only = idx[oa + end_a - (ca - c):oa + end_a][::-1]  # written descending
            assert np.all(np.diff(common) > 0) and np.all(np.diff(a_only) > 0), (p, s)
            both = np.concatenate([common, a_only])
            assert both.size == 0 or (both.min() >= lo and both.max() < hi), (p, s)
            ra.append(np.sort(both))
            if ob is not None:
                cb = int(cnt[b, h, jb, s])
                end_b = min(nxt, caps[jb])
                assert c <= cb and s0 + (cb - c) <= max(end_b, s0), (p, s, c, cb)
                b_only = idx[ob + s0:ob + s0 + (cb - c)]
                assert np.all(np.diff(b_only) > 0)
                assert np.intersect1d(b_only, a_only).size == 0
                assert b_only.size == 0 or (b_only.min() >= lo and b_only.max() < hi)
                rb.append(np.sort(np.concatenate([common, b_only])))
            else:
                assert c == 0
        rows[ja] = np.concatenate(ra) if ra else np.zeros(0, np.int32)
        if ob is not None:
            rows[jb] = np.concatenate(rb) if rb else np.zeros(0, np.int32)
    return rows


PAIR_CASES = [
    # name, Hq, Hk, S, D, dtype, causal, bk, G, gap (None: calibrated ~10%), segk, chunk_rows
    ("causal-G16-seg256", 4, 2, 2048, 128, torch.bfloat16, True, 16, 16, None, 256, None),
    # odd chunk rows: the last row of each chunk has no partner
    ("causal-G16-seg512-chunked-odd", 2, 1, 3000, 128, torch.bfloat16, True, 16, 16, None, 512,
     13),
    ("noncausal-bk32-G4-seg128-fp16", 2, 2, 1500, 128, torch.float16, False, 32, 4, None, 128,
     None),
    ("causal-gap0-seg256", 2, 1, 2048, 128, torch.bfloat16, True, 16, 16, 0.0, 256, None),
    ("noncausal-G8192-2pass-seg2048", 2, 2, 9000, 128, torch.bfloat16, False, 16, 8192, None,
     2048, None),
    ("noncausal-2pass-gap0-seg1024-chunked", 2, 1, 4100, 128, torch.bfloat16, False, 16, 8192,
     0.0, 1024, 23),
]


def _gap(q, k, bk, G, causal, gap):
    if gap is not None:
        return gap
    _, qs = orc.pool(q, 64, DTN[q.dtype])
    nqb = qs.shape[2]
    allc, _ = orc.select(qs, k, 0, nqb, np.full(q.shape[1], 1e6, np.float32), 64, bk, G, causal,
                         causal, 64)
    lo, hi = 1e-6, 1.0
    for _ in range(14):
        th = (lo * hi) ** 0.5
        c, _ = orc.select(qs, k, 0, nqb, orc.gap_from_threshold(th, 1, q.shape[1]), 64, bk, G,
                          causal, causal, 64)
        if c.sum() > 0.1 * allc.sum():
            lo = th
        else:
            hi = th
    return float(orc.gap_from_threshold((lo * hi) ** 0.5, 1, 1)[0])


@pytest.mark.parametrize("case", PAIR_CASES, ids=[c[0] for c in PAIR_CASES])
def test_paired_lists_and_attention(device, case):
    name, Hq, Hk, S, D, dtype, causal, bk, G, gap, segk, chunk_rows = case
    note("paired", name)
    q, k, v = make_inputs(1, Hq, Hk, S, D, dtype, seed=S + segk + 3)
    gap = _gap(q, k, bk, G, causal, gap)
    gaps = np.full(Hq, gap, np.float32)
    _, qs_cpu = orc.pool(q, 64, DTN[dtype])
    nqb = qs_cpu.shape[2]
    qs, _ = stages.pool_scaled(q.to(device), 64)
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    step = chunk_rows or nqb
    out = torch.zeros_like(qd)
    want_out = np.zeros(q.shape, np.float64)
    bc, bi = orc.local_blocks(1, Hq, S, 64, causal)
    shared = total = 0
    for J0 in range(0, nqb, step):
        nc = min(step, nqb - J0)
        want_c, want = orc.select(qs_cpu, k, J0, nc, gaps, 64, bk, G, causal, causal, 64)
        cnt, idx, pc = stages.select_segments(qs[:, :, J0:J0 + nc], kd, J0, gap, None, causal, 64,
                                              bk, G, causal, segk, paired=True)
        pcc = pc.cpu().numpy()
        for h in range(Hq):
            rows = paired_rows(cnt, idx, pc, J0, nc, 64, S, causal, causal, segk, 0, h, Hq)
            for jr in range(nc):
                assert np.array_equal(rows[jr], want[0][h][jr]), (name, h, J0 + jr)
            for p in range(nc // 2):  # shared keys: exactly the intersection
                inter = np.intersect1d(want[0][h][2 * p], want[0][h][2 * p + 1]).size
                assert int(pcc[0, h, p].sum()) == inter, (name, h, p)
                shared += inter
                total += want[0][h][2 * p].size
        stages.sparse_attention(qd, kd, vd, out, J0, nc, cnt, idx, causal, 64, segk=segk,
                                pair_common=pc)
        r0, r1 = J0 * 64, min(S, (J0 + nc) * 64)
        want_out[:, :, r0:r1] = orc.attention(q, k, v, 64, causal, bc, bi, want, J0=J0, nc=nc)
    torch.cuda.synchronize()
    err = np.abs(out.float().cpu().numpy() - want_out)
    assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN, (name, err.max(), err.mean())
    note("paired", name, f"shared {shared} of {total} row-A keys, max err {err.max():.2e}")


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_pair_form_matches_per_row_form(device, causal):
    # The prefill (pair form) against the per-row form of the same stages on
    # the same lists: same keys, different order, so equal within rounding.
    B, Hq, Hk, S, D = 1, 4, 2, 4096, 128
    note("prefill pair vs per-row", causal)
    q, k, v = make_inputs(B, Hq, Hk, S, D, torch.bfloat16, seed=5 + causal)
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    G = 16 if causal else 8192
    th = 0.8 if causal else 0.5
    out = VecAttention_prefill(qd, kd, vd, threshold=th, q_pooling_size=64, k_local_size=16,
                               group_k_block=G, causal=causal, chunk_size=2048)
    segk = stages.segment_keys(S, 16, G)
    qs, _ = stages.pool_scaled(qd, 64)
    gap = float(orc.gap_from_threshold(th, 1, 1)[0])
    ref = torch.zeros_like(qd)
    nqb = S // 64
    for J0 in range(0, nqb, 32):
        cnt, idx = stages.select_segments(qs[:, :, J0:J0 + 32], kd, J0, gap, None, causal, 64, 16,
                                          G, causal, segk)
        stages.sparse_attention(qd, kd, vd, ref, J0, 32, cnt, idx, causal, 64, segk=segk)
    torch.cuda.synchronize()
    err = (out.float() - ref.float()).abs()
    assert err.max().item() <= 1e-2 and err.mean().item() <= 5e-4, (err.max(), err.mean())
