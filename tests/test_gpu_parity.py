"""GPU parity of the HIP path against the CPU oracle (run on an MI355X).

Bar: pooling and selected index sets bit-exact; attention outputs within
max-abs 2e-2 and mean-abs 2e-3 of the oracle's float64 result (bf16/fp16
inputs), 1e-4 / 1e-5 for fp32 inputs.  Every call goes through the C ABI of
libvecattn.so.
"""
import math
import os

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from vecattention_amd import VecAttention_prefill
from vecattention_amd import _native as nat
from vecattention_amd import stages
from seglists import SegmentedLists, calibrate_threshold, select_chunk
from vecattention_amd.synth import WORKLOADS, make_inputs

pytestmark = pytest.mark.gpu

ATOL_MAX, ATOL_MEAN = 2e-2, 2e-3          # north-star tolerance, bf16/fp16
ATOL_MAX_F32, ATOL_MEAN_F32 = 1e-4, 1e-5
DTN = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}


def note(*a):
    print("[case]", *a, flush=True)


def gpu_lists(counts, indices, B, Hq, J0, nc, qps, Sk, causal, wo_init, dense_stride=0):
    """Per-row index lists from the GPU output, cut with the oracle's own
    capacity arithmetic (independent of the library's layout code)."""
    counts = counts.cpu().numpy().reshape(B, Hq, nc)
    idx = indices.cpu().numpy().reshape(-1)
    if dense_stride:
        caps = [dense_stride] * nc
    else:
        caps = [orc.row_capacity(J0 + jr, qps, Sk, causal, wo_init) for jr in range(nc)]
    out, base = [], 0
    for b in range(B):
        out.append([])
        for h in range(Hq):
            rows = []
            for jr in range(nc):
                c = int(counts[b, h, jr])
                assert 0 <= c <= caps[jr]
                rows.append(idx[base:base + c].copy())
                base += caps[jr]
            out[-1].append(rows)
    return counts, out


def assert_lists_equal(got, want, ctx=""):
    for b in range(len(want)):
        for h in range(len(want[b])):
            for jr in range(len(want[b][h])):
                g, w = got[b][h][jr], want[b][h][jr]
                if not np.array_equal(g, w):
                    extra = sorted(set(g.tolist()) ^ set(w.tolist()))[:10]
                    raise AssertionError(f"{ctx} b={b} h={h} jr={jr}: {len(g)} vs {len(w)} keys, "
                                         f"differ at {extra}")


def calibrated_threshold(keep, q, k, qps, bk, G, causal):
    """A threshold giving roughly `keep` of the selectable keys on these inputs (oracle)."""
    _, qs = orc.pool(q, qps, DTN[q.dtype])
    B, Hq = q.shape[:2]
    nqb = qs.shape[2]
    all_cnt, _ = orc.select(qs, k, 0, nqb, np.full(B * Hq, 1e6, np.float32), qps, bk, G, causal,
                            causal, 64)
    lo, hi = 1e-6, 1.0
    for _ in range(18):
        th = math.sqrt(lo * hi)
        c, _ = orc.select(qs, k, 0, nqb, orc.gap_from_threshold(th, B, Hq), qps, bk, G, causal,
                          causal, 64)
        if c.sum() > keep * all_cnt.sum():
            lo = th
        else:
            hi = th
    return math.sqrt(lo * hi)


# ------------------------------------------------------------------ pooling --

@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("S,qps", [(1000, 64), (4096, 128), (77, 64)])
def test_pool_bit_exact(device, dtype, S, qps):
    note("pool", dtype, S, qps)
    q, _, _ = make_inputs(2, 3, 3, S, 128 if dtype != torch.float32 else 64, dtype, seed=S)
    scaled, pooled = stages.pool_scaled(q.to(device), qps, want_pooled=True)
    want_p, want_s = orc.pool(q, qps, DTN[dtype])
    assert np.array_equal(pooled.float().cpu().numpy(), want_p)
    assert np.array_equal(scaled.float().cpu().numpy(), want_s)


@pytest.mark.parametrize("dtype,D,offset", [(torch.bfloat16, 256, 0), (torch.float32, 256, 0),
                                            (torch.float32, 36, 0), (torch.bfloat16, 200, 1),
                                            (torch.float16, 24, 0)])
def test_pool_head_dims_and_alignment(device, dtype, D, offset):
    """Vectorised rows (16-byte loads, up to 64 lanes per row) and the
    per-feature form (rows not 16-byte aligned: a one-element offset into the
    buffer), at head dims up to 256."""
    note("pool D", dtype, D, offset)
    q, _, _ = make_inputs(1, 3, 3, 700, D, dtype, seed=D)
    buf = torch.empty(q.numel() + offset, dtype=dtype, device=device)
    qd = buf[offset:].view(q.shape)
    qd.copy_(q.to(device))
    scaled, pooled = stages.pool_scaled(qd, 64, want_pooled=True)
    want_p, want_s = orc.pool(q, 64, DTN[dtype])
    assert np.array_equal(pooled.float().cpu().numpy(), want_p)
    assert np.array_equal(scaled.float().cpu().numpy(), want_s)


def test_pool_strided_bshd_view(device):
    note("pool strided")
    q, _, _ = make_inputs(1, 4, 4, 640, 128, torch.bfloat16, seed=11)
    bshd = q.transpose(1, 2).contiguous().to(device)        # memory (B, S, H, D)
    view = bshd.transpose(1, 2)                              # shape (B, H, S, D)
    scaled, pooled = stages.pool_scaled(view, 64, want_pooled=True)
    want_p, want_s = orc.pool(q, 64, "bfloat16")
    assert np.array_equal(pooled.float().cpu().numpy(), want_p)
    assert np.array_equal(scaled.float().cpu().numpy(), want_s)
    avg = stages.average_vector(view, 64)
    assert np.array_equal(avg.float().cpu().numpy(), want_p)


# ---------------------------------------------------------------- selection --

SELECT_CASES = [
    # name, B, Hq, Hk, S, D, dtype, causal, qps, bk, G, keep, chunk_rows
    ("A-fp32-noncausal", 1, 4, 4, 4096, 64, torch.float32, False, 64, 16, 16, 0.10, None),
    ("bf16-gqa-causal-G16", 1, 8, 2, 2048, 128, torch.bfloat16, True, 64, 16, 16, 0.10, None),
    ("bf16-gqa-causal-chunked", 1, 4, 1, 2048, 128, torch.bfloat16, True, 64, 16, 16, 0.10, 8),
    ("bf16-noncausal-G8192-tail", 1, 4, 4, 3000, 128, torch.bfloat16, False, 64, 16, 8192, 0.15, None),
    ("fp16-causal-qps128-bk32", 2, 4, 2, 1536, 64, torch.float16, True, 128, 32, 4, 0.10, None),
    ("bf16-noncausal-G1-bk64", 1, 2, 1, 1100, 128, torch.bfloat16, False, 64, 64, 1, 0.2, None),
    # groups of 16 and 32 keys (the reference models' group_k_block 1): the
    # wave kernel restarts the running maximum inside its 64-key chunks
    ("bf16-causal-bk16-G1", 1, 4, 2, 2048, 128, torch.bfloat16, True, 64, 16, 1, 0.10, None),
    ("fp16-noncausal-bk16-G2-tail", 1, 4, 2, 1500, 64, torch.float16, False, 64, 16, 2, 0.15,
     None),
    ("bf16-causal-qps128-bk32-G1-chunked", 2, 4, 1, 1800, 128, torch.bfloat16, True, 128, 32, 1,
     0.10, 6),
    # tiny key ranges: groups wholly past Sk inside the last chunk
    ("bf16-causal-bk16-G1-S200", 1, 2, 1, 200, 64, torch.bfloat16, True, 64, 16, 1, 0.30, None),
    ("fp16-noncausal-bk16-G2-S130", 1, 2, 2, 130, 64, torch.float16, False, 64, 16, 2, 0.50,
     None),
]


SEL_KERNELS = [nat.VA_SEL_EXACT, nat.VA_SEL_AUTO, nat.VA_SEL_MFMA, nat.VA_SEL_WAVE]
SEL_IDS = ["exact", "auto", "mfma", "wave"]


def select_or_skip(*args, **kw):
    """stages.select_rows, skipping the test when a forced kernel does not
    support the configuration (the library reports VA_ERR_UNSUPPORTED)."""
    try:
        return stages.select_rows(*args, **kw)
    except NotImplementedError as e:
        pytest.skip(f"kernel does not support this configuration: {e}")


@pytest.mark.parametrize("kernel", SEL_KERNELS, ids=SEL_IDS)
@pytest.mark.parametrize("case", SELECT_CASES, ids=[c[0] for c in SELECT_CASES])
def test_select_bit_exact(device, case, kernel):
    _select_case(device, case, kernel)


# A q_pooling_size that is not a multiple of 64 (the tuner API takes any):
# with the initial block excluded the first selectable key does not start a
# 64-key chunk, so the wave kernel refuses it and AUTO takes another kernel.
UNALIGNED_CASE = ("bf16-causal-qps96-bk16-G4", 1, 4, 2, 1536, 128, torch.bfloat16, True, 96,
                  16, 4, 0.10, None)


@pytest.mark.parametrize("kernel", [nat.VA_SEL_AUTO, nat.VA_SEL_MFMA], ids=["auto", "mfma"])
def test_select_unaligned_first_key(device, kernel):
    _select_case(device, UNALIGNED_CASE, kernel)


def test_select_unaligned_first_key_refuses_wave_kernel(device):
    name, B, Hq, Hk, S, D, dtype, causal, qps, bk, G, _, _ = UNALIGNED_CASE
    note("select refuses wave", name)
    q, k, _ = make_inputs(B, Hq, Hk, S, D, dtype, seed=1)
    qs, _ = stages.pool_scaled(q.to(device), qps)
    with pytest.raises(NotImplementedError):
        stages.select_rows(qs, k.to(device), 0, 0.2, None, causal, qps, bk, G, causal,
                           kernel=nat.VA_SEL_WAVE)


# Tiles of 128 and 256 keys (the reference signature's default k_local_size is
# 128): the 64-row MFMA kernel takes them (a tile is 8 or 16 of its 16-key
# segments, one or two per 256-key chunk); the wave kernel does not.
BIG_TILE_CASES = [
    # name, B, Hq, Hk, S, D, dtype, causal, qps, bk, G, keep, chunk_rows
    ("bf16-causal-qps128-bk128-G1", 1, 4, 2, 2048, 128, torch.bfloat16, True, 128, 128, 1, 0.10,
     None),
    ("bf16-causal-qps128-bk128-G4-chunked", 1, 4, 1, 3000, 128, torch.bfloat16, True, 128, 128,
     4, 0.10, 8),
    ("fp16-noncausal-bk256-G2-tail", 2, 4, 2, 1800, 64, torch.float16, False, 64, 256, 2, 0.15,
     None),
    ("bf16-noncausal-bk128-G8192", 1, 2, 2, 2500, 128, torch.bfloat16, False, 64, 128, 8192, 0.10,
     None),
]


@pytest.mark.parametrize("kernel", [nat.VA_SEL_EXACT, nat.VA_SEL_AUTO, nat.VA_SEL_MFMA],
                         ids=["exact", "auto", "mfma"])
@pytest.mark.parametrize("case", BIG_TILE_CASES, ids=[c[0] for c in BIG_TILE_CASES])
def test_select_big_tiles_bit_exact(device, case, kernel):
    _select_case(device, case, kernel)


# Small grids on the exact kernel: B*Hq*ceil(nc/R) < 256 work-groups for R = 4
# takes 2 rows (R=2: 1 x 4 heads x 128 rows) or 1 row per work-group (A's 64
# rows, and a causal chunked case).
EXACT_SMALL_GRID_CASES = [
    # name, B, Hq, Hk, S, D, dtype, causal, qps, bk, G, keep, chunk_rows
    ("fp32-noncausal-2rows", 1, 4, 4, 8192, 64, torch.float32, False, 64, 16, 16, 0.10, None),
    ("fp32-causal-1row-chunked", 1, 2, 1, 2500, 64, torch.float32, True, 64, 16, 16, 0.10, 13),
    ("bf16-noncausal-1row-G8192", 1, 2, 2, 1900, 128, torch.bfloat16, False, 64, 16, 8192, 0.15,
     None),
]


@pytest.mark.parametrize("case", EXACT_SMALL_GRID_CASES, ids=[c[0] for c in EXACT_SMALL_GRID_CASES])
def test_select_exact_small_grids(device, case):
    _select_case(device, case, nat.VA_SEL_EXACT)


def _select_case(device, case, kernel):
    name, B, Hq, Hk, S, D, dtype, causal, qps, bk, G, keep, chunk_rows = case
    note("select", name, kernel)
    q, k, _ = make_inputs(B, Hq, Hk, S, D, dtype, seed=len(name))
    th = calibrated_threshold(keep, q, k, qps, bk, G, causal)
    gaps = orc.gap_from_threshold(th, B, Hq)
    _, qs_cpu = orc.pool(q, qps, DTN[dtype])
    nqb = qs_cpu.shape[2]
    qs, _ = stages.pool_scaled(q.to(device), qps)
    kd = k.to(device)
    step = chunk_rows or nqb
    total_sel = 0
    for J0 in range(0, nqb, step):
        nc = min(step, nqb - J0)
        want_c, want = orc.select(qs_cpu, k, J0, nc, gaps, qps, bk, G, causal, causal, 64)
        cnt, idx = select_or_skip(qs[:, :, J0:J0 + nc], kd, J0, float(gaps[0]), None, causal,
                                  qps, bk, G, causal, kernel=kernel)
        got_c, got = gpu_lists(cnt, idx, B, Hq, J0, nc, qps, S, causal, causal)
        assert np.array_equal(got_c, want_c)
        assert_lists_equal(got, want, name)
        total_sel += int(want_c.sum())
    assert total_sel > 0


SEGMENT_CASES = [
    # name, Hq, Hk, S, D, dtype, causal, bk, G, keep, segk, chunk_rows
    ("causal-G16-seg256", 4, 2, 2048, 128, torch.bfloat16, True, 16, 16, 0.10, 256, None),
    ("causal-G16-seg512-chunked", 4, 1, 3000, 128, torch.bfloat16, True, 16, 16, 0.10, 512, 12),
    ("noncausal-bk32-G4-seg128", 2, 2, 1500, 64, torch.float16, False, 32, 4, 0.15, 128, None),
    ("causal-gap0-seg256", 2, 1, 2048, 128, torch.bfloat16, True, 16, 16, None, 256, None),
    # one group per row (DiT-style G): maxima pass, then the carry pass
    ("noncausal-G8192-2pass-seg2048", 2, 2, 9000, 128, torch.bfloat16, False, 16, 8192, 0.15,
     2048, None),
    ("noncausal-G8192-2pass-seg512-chunked", 2, 1, 5000, 64, torch.float16, False, 16, 8192,
     0.10, 512, 40),
    ("causal-Glong-2pass-seg1024", 2, 1, 4096, 128, torch.bfloat16, True, 16, 1024, 0.10, 1024,
     None),
    ("noncausal-2pass-gap0-seg1024", 2, 2, 4100, 128, torch.bfloat16, False, 16, 8192, None,
     1024, None),
    # groups of 16 and 32 keys: segments of whole 64-key chunks
    ("causal-bk16-G1-seg512-chunked", 4, 2, 3000, 128, torch.bfloat16, True, 16, 1, 0.10, 512,
     20),
    ("noncausal-bk16-G2-seg192-gap0", 2, 2, 2000, 64, torch.float16, False, 16, 2, None, 192,
     None),
]


@pytest.mark.parametrize("case", SEGMENT_CASES, ids=[c[0] for c in SEGMENT_CASES])
def test_select_segments_bit_exact(device, case):
    # The split selection that VecAttention_prefill runs: per-segment lists,
    # concatenated, equal the oracle's rows.
    name, Hq, Hk, S, D, dtype, causal, bk, G, keep, segk, chunk_rows = case
    note("select segments", name)
    q, k, _ = make_inputs(1, Hq, Hk, S, D, dtype, seed=S + segk)
    if keep is None:
        gaps = np.zeros(Hq, np.float32)
    else:
        gaps = orc.gap_from_threshold(calibrated_threshold(keep, q, k, 64, bk, G, causal), 1, Hq)
    _, qs_cpu = orc.pool(q, 64, DTN[dtype])
    nqb = qs_cpu.shape[2]
    qs, _ = stages.pool_scaled(q.to(device), 64)
    kd = k.to(device)
    smin = 64 if causal else 0
    step = chunk_rows or nqb
    for J0 in range(0, nqb, step):
        nc = min(step, nqb - J0)
        want_c, want = orc.select(qs_cpu, k, J0, nc, gaps, 64, bk, G, causal, causal, 64)
        cnt, idx = stages.select_segments(qs[:, :, J0:J0 + nc], kd, J0, float(gaps[0]), None,
                                          causal, 64, bk, G, causal, segk)
        cnt = cnt.cpu().numpy()
        idx = idx.cpu().numpy()
        nseg = cnt.shape[-1]
        for h in range(Hq):
            for jr in range(nc):
                o = stages.row_offset(S, 64, causal, causal, J0, nc, h, jr)
                parts = []
                for sg in range(nseg):
                    slot = max(sg * segk, smin) - smin
                    parts.append(idx[o + slot:o + slot + cnt[0, h, jr, sg]])
                got = np.concatenate(parts)
                assert np.array_equal(got, want[0][h][jr]), (name, h, J0 + jr)


def test_select_per_head_gaps_and_dense_layout(device):
    note("select per-head dense")
    B, Hq, Hk, S, D = 2, 4, 2, 1024, 128
    q, k, _ = make_inputs(B, Hq, Hk, S, D, torch.bfloat16, seed=21)
    th = torch.tensor([0.9, 0.5, 0.2, 0.05], dtype=torch.float32)
    gaps = (-torch.log(th + 1e-9)).float()
    gaps_bh = gaps.expand(B, Hq).contiguous()
    _, qs_cpu = orc.pool(q, 64, "bfloat16")
    nqb = qs_cpu.shape[2]
    want_c, want = orc.select(qs_cpu, k, 0, nqb, gaps_bh.numpy().reshape(-1), 64, 16, 16, True,
                              True, 64)
    pooled = stages.average_vector(q.to(device), 64)
    cnt, index = stages.fuse_qk_softmax_minp_wo_causal(pooled, k.to(device), 0, gaps.to(device),
                                                       True, 64, 16, True, 16)
    assert np.array_equal(cnt.cpu().numpy(), want_c)
    assert index.shape[-1] == max(min(S, int(want_c.max())), 1)
    idx = index.cpu().numpy()
    for b in range(B):
        for h in range(Hq):
            for J in range(nqb):
                c = want_c[b, h, J]
                assert np.array_equal(idx[b, h, J, :c], want[b][h][J])
                assert np.all(idx[b, h, J, c:] == 0)


MFMA_STRESS = [
    # name, Hq, Hk, S, D, causal, bk, G, gap   (gap 0: every running maximum is in the band)
    ("causal-G16-gap0", 4, 1, 2048, 128, True, 16, 16, 0.0),
    ("noncausal-G8192-gap0", 2, 2, 3000, 128, False, 16, 8192, 0.0),
    ("noncausal-G8192-bk32", 2, 1, 2500, 128, False, 32, 8192, 0.12),
    ("noncausal-G3-bk64-gap0", 2, 2, 1500, 64, False, 64, 3, 0.0),
    ("causal-G5-bk16", 2, 2, 2048, 64, True, 16, 5, 0.05),
    # groups of 16 and 32 keys: every tile's maximum key is ambiguous at gap 0
    ("causal-G1-bk16-gap0", 2, 1, 2048, 128, True, 16, 1, 0.0),
    ("noncausal-G2-bk16-gap0-tail", 2, 2, 1500, 64, False, 16, 2, 0.0),
    ("noncausal-G1-bk32-gap0", 2, 1, 1300, 128, False, 32, 1, 0.0),
    # tiles of 128 / 256 keys (MFMA kernel only): exact ties, groups over chunks
    ("noncausal-G2-bk128-gap0", 2, 2, 1500, 128, False, 128, 2, 0.0),
    ("noncausal-G3-bk256-gap0", 2, 1, 1300, 64, False, 256, 3, 0.0),
]


MFMA_SPLIT_CASES = [
    # name, Hq, Hk, S, D, dtype, causal, qps, bk, G, keep, segk, chunk_rows
    ("causal-qps128-bk128-G1-seg512", 4, 2, 3000, 128, torch.bfloat16, True, 128, 128, 1, 0.10,
     512, None),
    ("causal-qps128-bk128-G2-seg1024-chunked", 2, 1, 4500, 128, torch.bfloat16, True, 128, 128,
     2, 0.10, 1024, 9),
    ("noncausal-bk256-G2-seg512-gap0", 2, 2, 2300, 64, torch.float16, False, 64, 256, 2, None,
     512, None),
    # groups of 16 keys with a first selectable key (q_pooling_size 32) that
    # does not start a 64-key chunk, and groups of 48 keys: spans the wave
    # kernel does not take
    ("causal-qps32-bk16-G1-seg512-chunked", 4, 2, 3000, 128, torch.bfloat16, True, 32, 16, 1,
     0.10, 512, 40),
    ("noncausal-bk16-G3-seg768-gap0", 2, 2, 2500, 128, torch.bfloat16, False, 64, 16, 3, None,
     768, None),
]


@pytest.mark.parametrize("case", MFMA_SPLIT_CASES, ids=[c[0] for c in MFMA_SPLIT_CASES])
def test_select_segments_mfma_kernel_bit_exact(device, case):
    # Tiles of 128 / 256 keys split into key segments (whole 256-key chunks)
    # on the 64-row MFMA kernel: per-segment lists, concatenated, equal the
    # oracle's rows; the plan query reports the split.
    name, Hq, Hk, S, D, dtype, causal, qps, bk, G, keep, segk, chunk_rows = case
    note("select segments mfma", name)
    q, k, v = make_inputs(1, Hq, Hk, S, D, dtype, seed=S + segk + bk)
    if keep is None:
        gaps = np.zeros(Hq, np.float32)
    else:
        gaps = orc.gap_from_threshold(calibrated_threshold(keep, q, k, qps, bk, G, causal), 1, Hq)
    _, qs_cpu = orc.pool(q, qps, DTN[dtype])
    nqb = qs_cpu.shape[2]
    qs, _ = stages.pool_scaled(q.to(device), qps)
    kd = k.to(device)
    step = chunk_rows or nqb
    for J0 in range(0, nqb, step):
        nc = min(step, nqb - J0)
        want_c, want = orc.select(qs_cpu, k, J0, nc, gaps, qps, bk, G, causal, causal, 64)
        cnt, idx = stages.select_segments(qs[:, :, J0:J0 + nc], kd, J0, float(gaps[0]), None,
                                          causal, qps, bk, G, causal, segk)
        lists = SegmentedLists(cnt, idx, J0, nc, qps, S, causal, causal, segk)
        for h in range(Hq):
            for jr in range(nc):
                assert np.array_equal(lists.row(0, h, jr), want[0][h][jr]), (name, h, J0 + jr)
    assert want_c.sum() > 0


# fp32 inputs (and head dims the MFMA kernels do not take) select on the
# exact kernel; va_prefill splits it into key segments (one pass: every
# segment starts a group) when the fp32 matrix-core attention reads the lists.
EXACT_SPLIT_CASES = [
    # name, B, Hq, Hk, S, D, dtype, causal, qps, bk, G, keep, segk, chunk_rows
    ("A-fp32-noncausal-seg256", 1, 4, 4, 4096, 64, torch.float32, False, 64, 16, 16, 0.10, 256,
     None),
    ("fp32-causal-gqa-bk32-G4-seg384-chunked", 2, 4, 2, 2500, 64, torch.float32, True, 64, 32, 4,
     0.10, 384, 13),
    ("fp32-noncausal-qps128-d128-seg512-gap0", 1, 2, 1, 1800, 128, torch.float32, False, 128, 16,
     16, None, 512, None),
    ("fp32-causal-seg256-gap0", 1, 2, 1, 2048, 64, torch.float32, True, 64, 16, 16, None, 256,
     None),
    # segments that are not whole 256-key chunks
    ("bf16-d96-noncausal-bk16-G2-seg320", 1, 2, 2, 1900, 96, torch.bfloat16, False, 64, 16, 2,
     0.15, 320, None),
    # one group spans the row: maxima pass, then carry pass
    ("fp32-noncausal-G8192-2pass-seg512", 1, 2, 2, 2300, 64, torch.float32, False, 64, 16, 8192,
     0.15, 512, None),
    ("fp32-causal-Glong-2pass-seg256-chunked", 1, 4, 2, 2048, 64, torch.float32, True, 64, 16,
     1024, 0.10, 256, 9),
    ("fp32-noncausal-2pass-gap0-seg768-d128", 1, 2, 1, 2000, 128, torch.float32, False, 64, 16,
     8192, None, 768, None),
    ("bf16-d96-noncausal-G8192-2pass-seg256", 1, 2, 2, 1100, 96, torch.bfloat16, False, 64, 16,
     8192, 0.15, 256, None),
]


@pytest.mark.parametrize("case", EXACT_SPLIT_CASES, ids=[c[0] for c in EXACT_SPLIT_CASES])
def test_select_segments_exact_kernel_bit_exact(device, case):
    # The exact kernel's split: per-segment lists, concatenated, equal the
    # oracle's rows (every segment's keys inside the segment, within the row's
    # capacity).
    name, B, Hq, Hk, S, D, dtype, causal, qps, bk, G, keep, segk, chunk_rows = case
    note("select segments exact", name)
    q, k, _ = make_inputs(B, Hq, Hk, S, D, dtype, seed=S + segk + D)
    if keep is None:
        gaps = np.zeros(B * Hq, np.float32)
    else:
        gaps = orc.gap_from_threshold(calibrated_threshold(keep, q, k, qps, bk, G, causal), B, Hq)
    _, qs_cpu = orc.pool(q, qps, DTN[dtype])
    nqb = qs_cpu.shape[2]
    qs, _ = stages.pool_scaled(q.to(device), qps)
    kd = k.to(device)
    step = chunk_rows or nqb
    total = 0
    for J0 in range(0, nqb, step):
        nc = min(step, nqb - J0)
        want_c, want = orc.select(qs_cpu, k, J0, nc, gaps, qps, bk, G, causal, causal, 64)
        cnt, idx = stages.select_segments(qs[:, :, J0:J0 + nc], kd, J0, float(gaps[0]), None,
                                          causal, qps, bk, G, causal, segk, bsq=64)
        lists = SegmentedLists(cnt, idx, J0, nc, qps, S, causal, causal, segk)
        for b in range(B):
            for h in range(Hq):
                for jr in range(nc):
                    assert np.array_equal(lists.row(b, h, jr), want[b][h][jr]), (name, b, h,
                                                                                  J0 + jr)
        total += int(want_c.sum())
    assert total > 0


@pytest.mark.parametrize("causal,qps,D", [(True, 64, 64), (False, 128, 128)],
                         ids=["causal-qps64-d64", "noncausal-qps128-d128"])
def test_fp32_attention_on_segmented_lists_equals_unsplit(device, causal, qps, D):
    # The fp32 matrix-core attention on a split selection's segmented lists
    # (va_prefill's fp32 form) gives the output of the unsplit lists bit for
    # bit: the concatenated lists hold the same keys in the same order, so
    # every tile holds the same keys.
    B, Hq, Hk, S, bk, G = 2, 4, 2, 1700, 16, 16
    note("attn fp32 segmented", causal, qps, D)
    q, k, v = make_inputs(B, Hq, Hk, S, D, torch.float32, seed=D + qps)
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    qs, _ = stages.pool_scaled(qd, qps)
    nqb = qs.shape[2]
    segk = stages.segment_keys(S, bk, G, exact=True)
    assert segk > 0 and -(-S // segk) > 1
    gap = -math.log(0.3)
    cnt1, idx1 = stages.select_rows(qs, kd, 0, gap, None, causal, qps, bk, G, causal)
    cnt2, idx2 = stages.select_segments(qs, kd, 0, gap, None, causal, qps, bk, G, causal, segk)
    assert torch.equal(cnt2.sum(-1), cnt1) and int(cnt1.sum()) > 0
    outs = []
    for cnt, idx, sk in ((cnt1, idx1, 0), (cnt2, idx2, segk)):
        out = torch.zeros(B, Hq, S, D, dtype=torch.float32, device=device)
        stages.sparse_attention(qd, kd, vd, out, 0, nqb, cnt, idx, causal, qps, segk=sk)
        outs.append(out.cpu())
    assert torch.equal(outs[0], outs[1])


# (the wave kernel takes tiles of at most 64 keys)
STRESS_PARAMS = [pytest.param(case, kern, id=f"{case[0]}-{kid}") for case in MFMA_STRESS
                 for kern, kid in ((nat.VA_SEL_MFMA, "mfma"), (nat.VA_SEL_WAVE, "wave"))
                 if not (kern == nat.VA_SEL_WAVE and case[6] > 64)]


@pytest.mark.parametrize("case,kernel", STRESS_PARAMS)
def test_select_mfma_exact_fallback(device, case, kernel):
    # Exact ties at gap 0 and groups straddling chunks drive the certified
    # kernels through their exact paths (ambiguous pairs, carried maxima).
    name, Hq, Hk, S, D, causal, bk, G, gap = case
    note("select certified stress", name, kernel)
    q, k, _ = make_inputs(1, Hq, Hk, S, D, torch.bfloat16, seed=S + bk)
    _, qs_cpu = orc.pool(q, 64, "bfloat16")
    nqb = qs_cpu.shape[2]
    gaps = np.full(Hq, gap, np.float32)
    want_c, want = orc.select(qs_cpu, k, 0, nqb, gaps, 64, bk, G, causal, causal, 64)
    qs, _ = stages.pool_scaled(q.to(device), 64)
    cnt, idx = select_or_skip(qs, k.to(device), 0, gap, None, causal, 64, bk, G, causal,
                              kernel=kernel)
    got_c, got = gpu_lists(cnt, idx, 1, Hq, 0, nqb, 64, S, causal, causal)
    assert np.array_equal(got_c, want_c)
    assert_lists_equal(got, want, name)


@pytest.mark.parametrize("G", [1, 2, 4, 64])
@pytest.mark.parametrize("kernel", SEL_KERNELS, ids=SEL_IDS)
def test_select_ties_from_duplicate_keys(device, kernel, G):
    # Repeated key rows give exactly equal scores: selection at equality.
    note("select ties", kernel, G)
    q, k, _ = make_inputs(1, 2, 1, 1024, 64, torch.bfloat16, seed=5)
    k[:, :, 512:] = k[:, :, :512]
    _, qs_cpu = orc.pool(q, 64, "bfloat16")
    qs, _ = stages.pool_scaled(q.to(device), 64)
    for gap in (0.0, 0.05, 0.3):
        gaps = np.full(2, gap, np.float32)
        want_c, want = orc.select(qs_cpu, k, 0, 16, gaps, 64, 16, G, False, False, 64)
        cnt, idx = select_or_skip(qs, k.to(device), 0, gap, None, False, 64, 16, G, False,
                                  kernel=kernel)
        got_c, got = gpu_lists(cnt, idx, 1, 2, 0, 16, 64, 1024, False, False)
        assert np.array_equal(got_c, want_c)
        assert_lists_equal(got, want, f"ties gap={gap}")


# ---------------------------------------------------------------- attention --

ATTN_CASES = [
    # name, B, Hq, Hk, Sq, Sk, D, dtype, causal, qps, keep
    ("bf16-causal-gqa-d128", 1, 8, 2, 1536, 1536, 128, torch.bfloat16, True, 64, 0.1),
    ("bf16-causal-tail-d64-qps128", 1, 4, 4, 1000, 1000, 64, torch.bfloat16, True, 128, 0.1),
    ("fp16-noncausal-d128", 2, 4, 2, 1100, 1100, 128, torch.float16, False, 64, 0.15),
    ("bf16-noncausal-sq-ne-sk", 1, 4, 4, 700, 1300, 128, torch.bfloat16, False, 64, 0.2),
    ("fp32-noncausal-d64", 1, 4, 4, 1024, 1024, 64, torch.float32, False, 64, 0.1),
    # fp32 on the fp32 matrix-core kernel (auto) and the per-row kernel (simple)
    ("fp32-causal-gqa-d128-qps128", 1, 4, 2, 1000, 1000, 128, torch.float32, True, 128, 0.1),
    ("fp32-causal-batch2-tail-d64", 2, 4, 2, 1100, 1100, 64, torch.float32, True, 64, 0.1),
    ("fp32-noncausal-sq-ne-sk-d128", 1, 2, 2, 700, 1300, 128, torch.float32, False, 64, 0.2),
]


ATTN_KERNELS = [nat.VA_ATTN_AUTO, nat.VA_ATTN_SIMPLE, nat.VA_ATTN_MFMA_STAGED,
                nat.VA_ATTN_MFMA_RING]


def _oracle_lists_as_layout(q, k, case):
    # The oracle's selection of the case, laid out as the index workspace.
    name, B, Hq, Hk, Sq, Sk, D, dtype, causal, qps, keep = case
    th = calibrated_threshold(keep, q, k, qps, 16, 16, causal) if Sq == Sk else 0.3
    _, qs_cpu = orc.pool(q, qps, DTN[dtype])
    nqb = qs_cpu.shape[2]
    gaps = orc.gap_from_threshold(th, B, Hq)
    _, lists = orc.select(qs_cpu, k, 0, nqb, gaps, qps, 16, 16, causal, causal, 64)
    caps = [orc.row_capacity(J, qps, Sk, causal, causal) for J in range(nqb)]
    idx = np.zeros(max(sum(caps) * B * Hq, 1), np.int32)
    cnt = np.zeros((B, Hq, nqb), np.int32)
    base = 0
    for b in range(B):
        for h in range(Hq):
            for J in range(nqb):
                l = lists[b][h][J]
                idx[base:base + len(l)] = l
                cnt[b, h, J] = len(l)
                base += caps[J]
    return nqb, lists, torch.from_numpy(cnt), torch.from_numpy(idx)


@pytest.mark.parametrize("kernel", ATTN_KERNELS, ids=["auto", "simple", "staged", "ring"])
@pytest.mark.parametrize("case", ATTN_CASES, ids=[c[0] for c in ATTN_CASES])
def test_sparse_attention_matches_oracle(device, case, kernel):
    name, B, Hq, Hk, Sq, Sk, D, dtype, causal, qps, keep = case
    note("attn", name, kernel)
    q, k, v = make_inputs(B, Hq, Hk, max(Sq, Sk), D, dtype, seed=len(name) + 1)
    q = q[:, :, :Sq].contiguous()
    k, v = k[:, :, :Sk].contiguous(), v[:, :, :Sk].contiguous()
    nqb, lists, cnt, idx = _oracle_lists_as_layout(q, k, case)
    out = torch.zeros(B, Hq, Sq, D, dtype=dtype, device=device)
    run = lambda: stages.sparse_attention(q.to(device), k.to(device), v.to(device), out, 0, nqb,
                                          cnt.to(device), idx.to(device), causal, qps,
                                          kernel=kernel)
    mfma_ok = dtype != torch.float32
    ring_ok = mfma_ok and D == 128 and qps == 64
    if (kernel == nat.VA_ATTN_MFMA_RING and not ring_ok) or (
            kernel == nat.VA_ATTN_MFMA_STAGED and not mfma_ok):
        with pytest.raises(NotImplementedError):  # the form does not exist for this shape
            run()
        return
    run()
    bc, bi = orc.local_blocks(B, Hq, Sq, qps, causal)
    want = orc.attention(q, k, v, qps, causal, bc, bi, lists)
    err = np.abs(out.float().cpu().numpy() - want)
    tol = (ATOL_MAX_F32, ATOL_MEAN_F32) if dtype == torch.float32 else (ATOL_MAX, ATOL_MEAN)
    assert err.max() <= tol[0] and err.mean() <= tol[1], (err.max(), err.mean())


def test_fp32_matrix_core_attention_equals_per_row_kernel(device):
    # fp32 inputs: the fp32 matrix-core kernel (VA_ATTN_MFMA) and the per-row
    # kernel agree to fp32 rounding on the same lists, and the prefill plan
    # reports the matrix-core kernel.
    case = ("fp32-causal-gqa-d64", 1, 4, 2, 1536, 1536, 64, torch.float32, True, 64, 0.1)
    name, B, Hq, Hk, Sq, Sk, D, dtype, causal, qps, keep = case
    note("attn fp32 mfma vs per-row")
    q, k, v = make_inputs(B, Hq, Hk, Sq, D, dtype, seed=17)
    nqb, lists, cnt, idx = _oracle_lists_as_layout(q, k, case)
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    outs = []
    for kernel in (nat.VA_ATTN_MFMA, nat.VA_ATTN_SIMPLE):
        out = torch.zeros(B, Hq, Sq, D, dtype=dtype, device=device)
        stages.sparse_attention(qd, kd, vd, out, 0, nqb, cnt.to(device), idx.to(device), causal,
                                qps, kernel=kernel)
        outs.append(out.cpu())
    d = (outs[0] - outs[1]).abs()
    assert float(d.max()) <= 2e-5 and float(d.mean()) <= 2e-6, (float(d.max()), float(d.mean()))
    flags = nat.lib().va_prefill_kernels(
        nat.VA_F32, nat.ptr(qd), qd.stride(0), qd.stride(1), qd.stride(2), nat.ptr(kd),
        kd.stride(0), kd.stride(1), kd.stride(2), nat.ptr(vd), vd.stride(0), vd.stride(1),
        vd.stride(2), nat.ptr(qd), qd.stride(0), qd.stride(1), qd.stride(2), Hq, Hk, Sk, D, qps,
        16, 16)
    assert flags & nat.VA_KERNELS_ATTN_F32 and not flags & nat.VA_KERNELS_ATTN_ROW


@pytest.mark.parametrize("case", [c for c in ATTN_CASES if c[6] == 128 and c[9] == 64 and
                                  c[7] != torch.float32], ids=lambda c: c[0])
def test_attention_forms_are_bit_identical(device, case):
    # The staged and ring forms of the MFMA loop run the same arithmetic in
    # the same order.
    name, B, Hq, Hk, Sq, Sk, D, dtype, causal, qps, keep = case
    note("attn forms", name)
    q, k, v = make_inputs(B, Hq, Hk, max(Sq, Sk), D, dtype, seed=len(name) + 7)
    q = q[:, :, :Sq].contiguous()
    k, v = k[:, :, :Sk].contiguous(), v[:, :, :Sk].contiguous()
    nqb, _, cnt, idx = _oracle_lists_as_layout(q, k, case)
    outs = []
    for kernel in (nat.VA_ATTN_MFMA_STAGED, nat.VA_ATTN_MFMA_RING):
        out = torch.full((B, Hq, Sq, D), 7.0, dtype=dtype, device=device)
        stages.sparse_attention(q.to(device), k.to(device), v.to(device), out, 0, nqb,
                                cnt.to(device), idx.to(device), causal, qps, kernel=kernel)
        outs.append(out)
    assert torch.equal(outs[0], outs[1])


def test_mfma_all_keys_equals_dense_sdpa(device):
    # Non-causal, every key selected: the sparse kernel is dense attention.
    note("attn dense equivalence")
    B, Hq, Hk, S, D = 1, 4, 2, 2048, 128
    q, k, v = make_inputs(B, Hq, Hk, S, D, torch.bfloat16, seed=9)
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    nqb = S // 64
    cnt = torch.full((B, Hq, nqb), S, dtype=torch.int32, device=device)
    idx = torch.arange(S, dtype=torch.int32, device=device).repeat(B * Hq * nqb)
    out = torch.empty_like(qd)
    stages.sparse_attention(qd, kd, vd, out, 0, nqb, cnt, idx, False, 64, kernel=nat.VA_ATTN_MFMA)
    ref = torch.nn.functional.scaled_dot_product_attention(
        qd.float(), kd.float().repeat_interleave(2, 1).contiguous(),
        vd.float().repeat_interleave(2, 1).contiguous())
    err = (out.float() - ref).abs()
    assert err.max().item() <= ATOL_MAX and err.mean().item() <= ATOL_MEAN


@pytest.mark.parametrize("kernel", [nat.VA_ATTN_MFMA_STAGED, nat.VA_ATTN_MFMA_RING],
                         ids=["staged", "ring"])
def test_attention_scores_far_below_zero(device, kernel):
    # Every score is about -150 (q = -c, k = +c, every key selected): the
    # softmax is uniform and each output row is the mean of V.  A walk step
    # past the end of a row's list (zero K rows, score 0) that escaped its
    # mask would move the running maximum to 0 and underflow the row's sums.
    # 1000 keys: every row ends in a partial tile, and rows start their walk
    # at different tiles.
    note("attn scores far below zero", kernel)
    B, H, S, D = 1, 2, 1000, 128
    c = 3.65  # q.k / sqrt(D) = -sqrt(128) * c^2 = -150.7
    q = torch.full((B, H, S, D), -c, dtype=torch.bfloat16)
    k = torch.full((B, H, S, D), c, dtype=torch.bfloat16)
    v = torch.randn(B, H, S, D, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    nqb = -(-S // 64)
    cnt = torch.full((B, H, nqb), S, dtype=torch.int32, device=device)
    idx = torch.arange(S, dtype=torch.int32, device=device).repeat(B * H * nqb)
    out = torch.empty(B, H, S, D, dtype=torch.bfloat16, device=device)
    stages.sparse_attention(q.to(device), k.to(device), v.to(device), out, 0, nqb, cnt, idx, False,
                            64, kernel=kernel)
    got = out.float().cpu()
    assert torch.isfinite(got).all()
    want = v.float().mean(dim=2, keepdim=True).expand(B, H, S, D)
    err = (got - want).abs()
    assert err.max().item() <= ATOL_MAX and err.mean().item() <= ATOL_MEAN


# -------------------------------------------------------------- end to end --

E2E_CASES = [
    # name, B, Hq, Hk, S, D, dtype, causal, qps, bk, G, chunk, threshold
    ("vlm-like-causal", 1, 8, 2, 2048, 128, torch.bfloat16, True, 64, 16, 16, 1024, 0.5),
    ("dit-like-noncausal", 1, 4, 4, 2000, 128, torch.bfloat16, False, 64, 16, 8192, 1024, 0.3),
    # long enough for the two-pass split selection (segments of 2048 keys)
    ("dit-like-2pass", 1, 2, 2, 9000, 128, torch.bfloat16, False, 64, 16, 8192, 4608, 0.3),
    ("causal-qps128-bk16", 1, 4, 4, 1300, 64, torch.bfloat16, True, 128, 16, 4, 512, 0.6),
    # the reference models' defaults (k_local_size 16, group_k_block 1)
    ("model-defaults-causal-G1", 1, 4, 2, 3000, 128, torch.bfloat16, True, 64, 16, 1, 1024, 0.9),
    ("A-fp32-noncausal", 1, 4, 4, 4096, 64, torch.float32, False, 64, 16, 16, 4096, 0.35),
    # fp32 split selection under the causal rule, over chunks
    ("fp32-causal-gqa-chunked", 1, 4, 2, 2500, 64, torch.float32, True, 64, 16, 16, 1024, 0.5),
    # fp32 with one group per row: the exact kernel's two-pass split
    ("fp32-dit-like-2pass", 1, 2, 2, 3000, 64, torch.float32, False, 64, 16, 8192, 1024, 0.3),
    ("fp32-noncausal-qps128-d128", 2, 2, 1, 1500, 128, torch.float32, False, 128, 32, 4, 1024,
     0.4),
    # batches: every (b, h) work item, strides over the batch dimension
    ("batch2-causal-gqa", 2, 8, 2, 1536, 128, torch.bfloat16, True, 64, 16, 16, 1024, 0.5),
    ("batch3-noncausal-fp16-d64", 3, 4, 2, 1100, 64, torch.float16, False, 64, 16, 8192, 1024, 0.3),
]


@pytest.mark.parametrize("case", E2E_CASES, ids=[c[0] for c in E2E_CASES])
def test_vecattention_prefill_matches_oracle(device, case):
    name, B, Hq, Hk, S, D, dtype, causal, qps, bk, G, chunk, th = case
    note("e2e", name)
    q, k, v = make_inputs(B, Hq, Hk, S, D, dtype, seed=3)
    # Queries arrive as a (B, H, S, D) view of (B, S, H, D) memory, as in the VLM caller.
    qv = q.transpose(1, 2).contiguous().to(device).transpose(1, 2)
    out = VecAttention_prefill(qv, k.to(device), v.to(device), threshold=th, q_pooling_size=qps,
                               k_local_size=bk, group_k_block=G, causal=causal, chunk_size=chunk)
    torch.cuda.synchronize()
    assert out.shape == (B, Hq, S, D) and out.dtype == dtype and out.is_contiguous()
    want, _ = orc.prefill(q, k, v, th, qps, bk, G, causal, chunk, 64, DTN[dtype])
    err = np.abs(out.float().cpu().numpy() - want)
    tol = (ATOL_MAX_F32, ATOL_MEAN_F32) if dtype == torch.float32 else (ATOL_MAX, ATOL_MEAN)
    assert err.max() <= tol[0] and err.mean() <= tol[1], (err.max(), err.mean())


def test_reference_default_tiles_take_the_mfma_kernels(device):
    # The reference signature's defaults (q_pooling_size 128, k_local_size 128,
    # group_k_block 1) run on the MFMA selection and attention without a
    # warning, and match the oracle.
    import warnings
    note("default tiles")
    B, Hq, Hk, S, D = 1, 4, 2, 1300, 128
    q, k, v = make_inputs(B, Hq, Hk, S, D, torch.bfloat16, seed=4)
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    with warnings.catch_warnings():
        warnings.simplefilter("error", RuntimeWarning)
        out = VecAttention_prefill(qd, kd, vd, threshold=0.5)
    torch.cuda.synchronize()
    want, _ = orc.prefill(q, k, v, 0.5, 128, 128, 1, True, 16 * 1024, 64, "bfloat16")
    err = np.abs(out.float().cpu().numpy() - want)
    assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN, (err.max(), err.mean())


def test_slow_path_is_announced_and_matches_oracle(device):
    # head_dim 96 has no MFMA kernel: the exact selection and the per-row
    # attention run, the prefill warns once, and the result matches the oracle.
    from vecattention_amd import vecattention as va_mod
    note("slow path")
    B, Hq, Hk, S, D = 1, 2, 1, 700, 96
    q, k, v = make_inputs(B, Hq, Hk, S, D, torch.bfloat16, seed=5)
    va_mod._warned_paths.clear()
    with pytest.warns(RuntimeWarning, match="exact fp64 kernel"):
        out = VecAttention_prefill(q.to(device), k.to(device), v.to(device), threshold=0.5,
                                   q_pooling_size=64, k_local_size=16, group_k_block=16)
    torch.cuda.synchronize()
    want, _ = orc.prefill(q, k, v, 0.5, 64, 16, 16, True, 16 * 1024, 64, "bfloat16")
    err = np.abs(out.float().cpu().numpy() - want)
    assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN, (err.max(), err.mean())


def _device_gaps(th, B, Hq, device):
    """The fp32 gaps VecAttention_prefill computes on the device for a
    threshold tensor (-torch.log(th + 1e-9) there), as a host array."""
    from vecattention_amd.vecattention import threshold_to_gap
    _, g = threshold_to_gap(th.to(device), B, Hq, device)
    return g.reshape(-1).cpu().numpy()


def _ulps(a, b):
    return np.abs(a.view(np.int32).astype(np.int64) - b.view(np.int32).astype(np.int64))


def test_device_gaps_equal_oracle(device):
    # The gaps the prefill computes on the device for a threshold tensor are
    # the oracle's (the correctly rounded fp32 of -log(th + 1e-9)) bit for bit.
    th = torch.cat([torch.rand(4096, generator=torch.Generator().manual_seed(0)),
                    torch.logspace(-7, 0, 4096)]).reshape(-1, 8)
    g_dev = _device_gaps(th, th.shape[0], 8, device)
    g_orc = orc.gap_from_threshold(th.numpy(), th.shape[0], 8)
    d = _ulps(g_dev, g_orc)
    note(f"device gaps: {int((d > 0).sum())} of {d.size} differ from the oracle "
         f"(max {int(d.max())} ulp)")
    assert d.max() == 0


@pytest.mark.parametrize("causal", [False, True])
def test_per_head_gaps_select_bit_exact(device, causal):
    # Per-head thresholds through the prefill's split selection: lists equal
    # the oracle's, fed the gaps the product computed on the device.
    note("per-head lists", causal)
    B, Hq, Hk, S, D = 1, 4, 2, 9000, 128
    q, k, v = make_inputs(B, Hq, Hk, S, D, torch.bfloat16, seed=6)
    th = torch.tensor([0.9, 0.5, 0.1, 0.01])
    gaps = _device_gaps(th, B, Hq, device)
    G = 16 if causal else 8192
    qd, kd = q.to(device), k.to(device)
    qs_gpu, _ = stages.pool_scaled(qd, 64)
    segk = stages.segment_keys(S, 16, G)
    assert segk > 0
    nqb = qs_gpu.shape[2]
    _, qs = orc.pool(q, 64, "bfloat16")
    for J0 in (0, 128):
        nc = min(128, nqb - J0)
        cnt, idx = stages.select_segments(qs_gpu[:, :, J0:J0 + nc], kd, J0, 0.0,
                                          torch.from_numpy(gaps).to(device), causal, 64, 16, G,
                                          causal, segk)
        got = SegmentedLists(cnt, idx, J0, nc, 64, S, causal, causal, segk)
        _, want = orc.select(qs, k, J0, nc, gaps, 64, 16, G, causal, causal, 64)
        for h in range(Hq):
            for jr in range(nc):
                assert np.array_equal(got.row(0, h, jr), want[0][h][jr]), (J0, h, jr)


def test_prefill_per_head_threshold_tensor(device):
    note("e2e per-head")
    B, Hq, S, D = 1, 4, 1024, 128
    q, k, v = make_inputs(B, Hq, Hq, S, D, torch.bfloat16, seed=4)
    th = torch.tensor([0.9, 0.5, 0.1, 0.01])
    out = VecAttention_prefill(q.to(device), k.to(device), v.to(device), th.to(device), 64, 16, 16,
                               False, 512)
    want, _ = orc.prefill(q, k, v, th.numpy(), 64, 16, 16, False, 512, 64, "bfloat16",
                          gaps=_device_gaps(th, B, Hq, device))
    err = np.abs(out.float().cpu().numpy() - want)
    assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN


def test_prefill_per_batch_and_head_threshold_tensor(device):
    # a (B, H) threshold tensor: every (b, h) its own gap
    note("e2e per-(b,h)")
    B, Hq, S, D = 2, 3, 900, 128
    q, k, v = make_inputs(B, Hq, Hq, S, D, torch.bfloat16, seed=5)
    th = torch.tensor([[0.9, 0.5, 0.1], [0.05, 0.3, 0.7]])
    out = VecAttention_prefill(q.to(device), k.to(device), v.to(device), th.to(device), 64, 16, 16,
                               True, 512)
    want, _ = orc.prefill(q, k, v, th.numpy(), 64, 16, 16, True, 512, 64, "bfloat16",
                          gaps=_device_gaps(th, B, Hq, device))
    err = np.abs(out.float().cpu().numpy() - want)
    assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN


# --------------------------------------------- full-size properties (config B) --

@pytest.fixture(scope="module")
def config_b(device):
    q, k, v = make_inputs(1, 28, 4, 32768, 128, torch.bfloat16, seed=0)
    return q, k, v, q.to(device), k.to(device), v.to(device)


def test_full_size_large_gap_selects_every_selectable_key(config_b):
    note("full-size all selectable")
    q, k, v, qd, kd, vd = config_b
    qps, nqb = 64, 512
    qs, _ = stages.pool_scaled(qd, qps)
    cnt, _ = stages.select_rows(qs, kd, 0, 1e6, None, True, qps, 16, 16, True)
    J = torch.arange(nqb)
    want = torch.clamp((J - 1) * qps, min=0) - torch.where((J % 64 == 0) & (J >= 2), 48, 0)
    assert torch.equal(cnt.cpu(), want.to(torch.int32).expand(1, 28, nqb))


@pytest.mark.parametrize("th", ["calibrated", 0.35])
def test_full_size_rows_match_oracle(config_b, th):
    # Sampled rows of the full 32K config: the split selection's lists (the
    # ones VecAttention_prefill's attention reads: 16 segments of 2048 keys)
    # equal the oracle's bit for bit, and the prefill output is within tolerance.
    q, k, v, qd, kd, vd = config_b
    qps = 64
    qs_gpu, _ = stages.pool_scaled(qd, qps)
    if th == "calibrated":
        th = calibrate_threshold(qs_gpu, kd, True, qps, 16, 16, WORKLOADS["B"].keep)
    note("full-size sampled rows, threshold", th)
    out = VecAttention_prefill(qd, kd, vd, th, qps, 16, 16, True, 32768)
    gpu = select_chunk(qs_gpu, kd, 0, 512, -math.log(th + 1e-9), True, qps, 16, 16)
    torch.cuda.synchronize()
    out_cpu = out.float().cpu().numpy()
    gaps = orc.gap_from_threshold(th, 1, 28)
    bc, bi = orc.local_blocks(1, 1, 32768, qps, True)
    rng = np.random.default_rng(0)
    for h in (0, 13, 27):
        qh, kh, vh = q[:, h:h + 1], k[:, h // 7:h // 7 + 1], v[:, h // 7:h // 7 + 1]
        _, qs = orc.pool(qh, qps, "bfloat16")
        for J in [64] + sorted(rng.choice(np.arange(1, 512), 4, replace=False).tolist()) + [511]:
            _, lists = orc.select(qs, kh, 0, 512, gaps[:1], qps, 16, 16, True, True, 64,
                                  rows=(J, J + 1))
            assert np.array_equal(gpu.row(0, h, J), lists[0][0][J]), (h, J)
            want = orc.attention(qh, kh, vh, qps, True, bc, bi, [[lists[0][0][J:J + 1]]], J0=J,
                                 nc=1)
            err = np.abs(out_cpu[0, h, J * qps:(J + 1) * qps] - want[0, 0])
            assert err.max() <= ATOL_MAX and err.mean() <= ATOL_MEAN, (h, J, err.max())


def test_full_size_every_row_matches_oracle(config_b):
    # Every row of every head of the 32K config at the benchmark's calibrated
    # threshold: the split selection's lists (16 segments of 2048 keys, as the
    # prefill runs them) equal the CPU oracle's bit for bit.  The oracle runs
    # per head in threads (its C loop releases the interpreter lock).
    from concurrent.futures import ThreadPoolExecutor
    q, k, _, qd, kd, _ = config_b
    qps, nqb, th = 64, 512, 0.7550760976531293
    note("full-size every row, threshold", th)
    qs_gpu, _ = stages.pool_scaled(qd, qps)
    gpu = select_chunk(qs_gpu, kd, 0, nqb, -math.log(th + 1e-9), True, qps, 16, 16)
    gaps = orc.gap_from_threshold(th, 1, 1)

    def head(h):
        _, qs = orc.pool(q[:, h:h + 1], qps, "bfloat16")
        cnt, lists = orc.select(qs, k[:, h // 7:h // 7 + 1], 0, nqb, gaps, qps, 16, 16, True,
                                True, 64)
        bad = [J for J in range(nqb) if not np.array_equal(gpu.row(0, h, J), lists[0][0][J])]
        return h, int(cnt.sum()), bad

    with ThreadPoolExecutor(max_workers=min(16, os.cpu_count() or 1)) as ex:
        results = list(ex.map(head, range(28)))
    total = sum(n for _, n, _ in results)
    assert total > 0
    for h, _, bad in results:
        assert not bad, (h, bad[:8])


def test_full_size_chunking_invariant(config_b):
    # Chunks of 16K and 32K start q-block programs at multiples of 64 rows
    # either way, so the selection and therefore the output are identical.
    note("full-size chunk invariance")
    _, _, _, qd, kd, vd = config_b
    a = VecAttention_prefill(qd, kd, vd, 0.35, 64, 16, 16, True, 32768)
    b = VecAttention_prefill(qd, kd, vd, 0.35, 64, 16, 16, True, 16384)
    assert torch.equal(a, b)


@pytest.mark.parametrize("kernel", [nat.VA_SEL_MFMA, nat.VA_SEL_WAVE], ids=["mfma", "wave"])
def test_full_size_mfma_selection_equals_exact_kernel(config_b, kernel):
    # Every row of the 32K config: a certified MFMA kernel and the fp64 kernel
    # (independent implementations of the canonical rule) agree bit for bit.
    note("full-size certified == exact", kernel)
    _, _, _, qd, kd, vd = config_b
    qs, _ = stages.pool_scaled(qd, 64)
    gap = -math.log(0.75 + 1e-9)
    c1, i1 = stages.select_rows(qs, kd, 0, gap, None, True, 64, 16, 16, True,
                                kernel=nat.VA_SEL_EXACT)
    c2, i2 = stages.select_rows(qs, kd, 0, gap, None, True, 64, 16, 16, True,
                                kernel=kernel)
    assert torch.equal(c1, c2)
    # compare only the written slots of every row
    lay_c = c1.cpu().numpy().reshape(-1)
    a, b = i1.cpu().numpy(), i2.cpu().numpy()
    for bh in range(28):
        for J in range(512):
            o = stages.row_offset(32768, 64, True, True, 0, 512, bh, J)
            n = lay_c[bh * 512 + J]
            assert np.array_equal(a[o:o + n], b[o:o + n]), (bh, J)
