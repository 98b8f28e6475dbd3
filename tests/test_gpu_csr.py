"""The compact (CSR) selection output, va_select_csr, on an MI355X.

Bar: every row's keys at indices[offsets[r]:offsets[r+1]] equal the oracle's
list bit for bit, offsets[0] = 0 and the offsets step by the per-row counts
(summed over key segments), and the total equals the oracle's.  Cases cover
the three selection kernels (wave: one pass, split, two-pass split; 64-row
MFMA: split and unsplit; exact fp32), batches, ragged tails and chunked rows.
At the full 32K size of workload B the compact lists equal the capacity
layout's lists of the split selection (itself pinned to the oracle row by row
in test_gpu_parity.py).
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from vecattention_amd import stages
from vecattention_amd.synth import make_inputs
from seglists import select_chunk
from test_gpu_parity import DTN, calibrated_threshold, note

pytestmark = pytest.mark.gpu

CSR_CASES = [
    # name, B, Hq, Hk, S, D, dtype, causal, qps, bk, G, keep, segk, chunk_rows
    ("wave-causal-G16", 1, 4, 2, 2048, 128, torch.bfloat16, True, 64, 16, 16, 0.10, 0, None),
    ("wave-causal-bk16-G1-seg512-chunked", 1, 4, 2, 3000, 128, torch.bfloat16, True, 64, 16, 1,
     0.10, 512, 20),
    ("wave-noncausal-G8192-2pass-seg1024", 1, 2, 2, 4100, 128, torch.bfloat16, False, 64, 16,
     8192, 0.15, 1024, None),
    ("wave-batch2-fp16-noncausal-G2-tail", 2, 4, 2, 1500, 64, torch.float16, False, 64, 16, 2,
     0.15, 0, None),
    ("mfma-causal-qps128-bk128-seg512", 1, 4, 2, 3000, 128, torch.bfloat16, True, 128, 128, 1,
     0.10, 512, None),
    ("mfma-causal-qps96-unaligned", 1, 4, 2, 1536, 128, torch.bfloat16, True, 96, 16, 4, 0.10, 0,
     None),
    ("exact-fp32-noncausal", 1, 4, 4, 2048, 64, torch.float32, False, 64, 16, 16, 0.10, 0, None),
    # the exact kernel's one-pass split (segments of whole groups)
    ("exact-fp32-causal-seg256-chunked", 1, 4, 2, 2500, 64, torch.float32, True, 64, 16, 16,
     0.10, 256, 13),
    ("exact-fp32-noncausal-G8192-2pass-seg512", 1, 2, 2, 2300, 64, torch.float32, False, 64, 16,
     8192, 0.15, 512, None),
]


def check_csr(cnt, off, idx, want_c, want, B, Hq, nc, ctx):
    off = off.cpu().numpy()
    idx = idx.cpu().numpy()
    cnt = cnt.cpu().numpy().reshape(B * Hq * nc, -1)
    assert off[0] == 0 and np.array_equal(np.diff(off), cnt.sum(axis=1)), ctx
    assert off[-1] == want_c.sum() == idx.size, ctx
    for b in range(B):
        for h in range(Hq):
            for jr in range(nc):
                r = (b * Hq + h) * nc + jr
                assert np.array_equal(idx[off[r]:off[r + 1]], want[b][h][jr]), (ctx, b, h, jr)


@pytest.mark.parametrize("case", CSR_CASES, ids=[c[0] for c in CSR_CASES])
def test_select_csr_matches_oracle(device, case):
    name, B, Hq, Hk, S, D, dtype, causal, qps, bk, G, keep, segk, chunk_rows = case
    note("select csr", name)
    q, k, _ = make_inputs(B, Hq, Hk, S, D, dtype, seed=S + bk + segk)
    th = calibrated_threshold(keep, q, k, qps, bk, G, causal)
    gaps = orc.gap_from_threshold(th, B, Hq)
    _, qs_cpu = orc.pool(q, qps, DTN[dtype])
    nqb = qs_cpu.shape[2]
    qs, _ = stages.pool_scaled(q.to(device), qps)
    kd = k.to(device)
    step = chunk_rows or nqb
    for J0 in range(0, nqb, step):
        nc = min(step, nqb - J0)
        want_c, want = orc.select(qs_cpu, k, J0, nc, gaps, qps, bk, G, causal, causal, 64)
        cnt, off, idx = stages.select_csr(qs[:, :, J0:J0 + nc], kd, J0, float(gaps[0]), None,
                                          causal, qps, bk, G, causal, segk)
        check_csr(cnt, off, idx, want_c, want, B, Hq, nc, (name, J0))


def test_select_csr_gap_extremes(device):
    # gap 0 (only keys at their running maximum) and a huge gap (every
    # selectable key): the compact rows are exactly the oracle's.
    note("select csr extremes")
    B, Hq, Hk, S, D = 1, 2, 1, 1100, 128
    q, k, _ = make_inputs(B, Hq, Hk, S, D, torch.bfloat16, seed=9)
    _, qs_cpu = orc.pool(q, 64, "bfloat16")
    nqb = qs_cpu.shape[2]
    qs, _ = stages.pool_scaled(q.to(device), 64)
    kd = k.to(device)
    for gap in (0.0, 1e6):
        gaps = np.full(B * Hq, gap, np.float32)
        want_c, want = orc.select(qs_cpu, k, 0, nqb, gaps, 64, 16, 16, True, True, 64)
        cnt, off, idx = stages.select_csr(qs, kd, 0, gap, None, True, 64, 16, 16, True)
        check_csr(cnt, off, idx, want_c, want, B, Hq, nqb, ("extremes", gap))


def test_select_csr_full_size_equals_capacity_layout(device):
    # Workload B's shape (28 q heads, 4 kv heads, 32K keys, causal, G 16) at
    # its benchmark threshold, all 512 rows, both with the split of the
    # prefill (16 segments of 2048 keys) and unsplit: the compact rows equal
    # the capacity layout's rows of the split selection.
    note("select csr full size")
    q, k, _ = make_inputs(1, 28, 4, 32768, 128, torch.bfloat16, seed=0)
    qd, kd = q.to(device), k.to(device)
    th, qps, nqb = 0.7550760976531293, 64, 512
    gap = -math.log(th + 1e-9)
    qs, _ = stages.pool_scaled(qd, qps)
    lists = select_chunk(qs, kd, 0, nqb, gap, True, qps, 16, 16)
    for segk in (stages.segment_keys(32768, 16, 16), 0):
        cnt, off, idx = stages.select_csr(qs, kd, 0, gap, None, True, qps, 16, 16, True, segk)
        off = off.cpu().numpy()
        idx = idx.cpu().numpy()
        assert off[0] == 0 and np.all(np.diff(off) >= 0)
        for h in range(28):
            for J in range(nqb):
                r = h * nqb + J
                assert np.array_equal(idx[off[r]:off[r + 1]], lists.row(0, h, J)), (segk, h, J)
