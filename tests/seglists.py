"""Helpers of the GPU parity tests: per-row key lists cut out of the split
(segmented) selection output, and a threshold calibrated to a keep ratio.

The lists are cut with the oracle's own capacity arithmetic
(oracle.row_capacity), not with the library's layout code: row J of a chunk
owns row_capacity(J) int32 slots, the rows of one (b, h) follow each other and
the (b, h) blocks follow each other; segment s of a row writes its keys from
slot max(s * segk, smin) - smin, smin being the first key the rule can select
(q_pooling_size for causal rows without the initial block, else 0).
"""
import math

import numpy as np
import torch

from oracle import oracle as orc
from vecattention_amd import stages


def _smin(qps, Sk, causal, wo_init):
    if not wo_init:
        return 0
    return qps if causal else min(qps, Sk)


class SegmentedLists:
    """Per-row lists of one chunk's split selection, copied to the host once."""

    def __init__(self, counts, indices, J0, nc, qps, Sk, causal, wo_init, segk):
        self.counts = counts.cpu().numpy()          # (B, Hq, nc, nseg)
        self.idx = indices.cpu().numpy().reshape(-1)
        B, Hq, nc_, nseg = self.counts.shape
        assert nc_ == nc and nseg == -(-Sk // segk)
        self.caps = np.array([orc.row_capacity(J0 + jr, qps, Sk, causal, wo_init)
                              for jr in range(nc)], np.int64)
        self.starts = np.concatenate([[0], np.cumsum(self.caps)[:-1]]).astype(np.int64)
        self.block = int(self.caps.sum())
        self.Hq, self.nseg, self.segk, self.Sk = Hq, nseg, segk, Sk
        self.smin = _smin(qps, Sk, causal, wo_init)

    def row(self, b, h, jr):
        """Ascending keys of chunk row jr; checks that every segment's keys lie
        inside that segment and fit the row's capacity."""
        base = (b * self.Hq + h) * self.block + int(self.starts[jr])
        cap = int(self.caps[jr])
        parts = []
        for s in range(self.nseg):
            c = int(self.counts[b, h, jr, s])
            lo, hi = s * self.segk, min((s + 1) * self.segk, self.Sk)
            slot = max(lo, self.smin) - self.smin
            assert c >= 0 and (c == 0 or slot + c <= cap), (b, h, jr, s, c, slot, cap)
            keys = self.idx[base + slot:base + slot + c]
            assert c == 0 or (keys[0] >= lo and keys[-1] < hi), (b, h, jr, s)
            parts.append(keys)
        return np.concatenate(parts) if parts else np.zeros(0, np.int32)

    def total(self):
        return self.counts.sum(axis=-1)


def select_chunk(qs, kd, J0, nc, gap, causal, qps, bk, G, bsq=64):
    """The split selection VecAttention_prefill runs for chunk rows [J0, J0+nc),
    as a SegmentedLists."""
    Sk = kd.shape[2]
    segk = stages.segment_keys(Sk, bk, G)
    assert segk > 0, "this shape does not run the split selection"
    cnt, idx = stages.select_segments(qs[:, :, J0:J0 + nc], kd, J0, gap, None, causal, qps, bk,
                                      G, causal, segk, bsq=bsq)
    return SegmentedLists(cnt, idx, J0, nc, qps, Sk, causal, causal, segk)


def calibrate_threshold(qs, kd, causal, qps, bk, G, keep, chunk_rows=512, iters=14):
    """A threshold whose selection keeps about `keep` of the selectable keys of
    these heads (bisection on the GPU selection counts, as the benchmark
    calibrates its workloads)."""
    nqb = qs.shape[2]
    Sk = kd.shape[2]
    segk = stages.segment_keys(Sk, bk, G)

    def total(gap):
        t = 0
        for J0 in range(0, nqb, chunk_rows):
            nc = min(chunk_rows, nqb - J0)
            cnt, _ = stages.select_segments(qs[:, :, J0:J0 + nc], kd, J0, gap, None, causal, qps,
                                            bk, G, causal, segk)
            t += int(cnt.sum().item())
        return t

    target = keep * total(1e6)
    lo, hi = 1e-6, 1.0
    for _ in range(iters):
        th = math.sqrt(lo * hi)
        if total(-math.log(th + 1e-9)) > target:
            lo = th
        else:
            hi = th
    return math.sqrt(lo * hi)


def pooled_oracle(q_head, qps, dtype=torch.bfloat16):
    name = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}[dtype]
    return orc.pool(q_head, qps, name)[1]


def check_rows(q, k, v, qs_dev, kd, out_cpu, heads, rows, th, causal, G, chunk_rows=512,
               qps=64, bk=16, rep=1):
    """For each sampled (head, q-block J): the split selection's list equals
    the oracle's, and the prefill output rows are within tolerance."""
    S, Sk = q.shape[2], k.shape[2]
    nqb = -(-S // qps)
    gap = -math.log(th + 1e-9)
    gaps = orc.gap_from_threshold(th, 1, 1)
    bc, bi = orc.local_blocks(1, 1, S, qps, causal)
    by_chunk = {}
    for J in rows:
        by_chunk.setdefault(J // chunk_rows * chunk_rows, []).append(J)
    for J0, Js in sorted(by_chunk.items()):
        nc = min(chunk_rows, nqb - J0)
        gpu = select_chunk(qs_dev, kd, J0, nc, gap, causal, qps, bk, G)
        for h in heads:
            hk = h // rep
            qh, kh, vh = q[:, h:h + 1], k[:, hk:hk + 1], v[:, hk:hk + 1]
            qs = pooled_oracle(qh, qps)
            for J in Js:
                _, lists = orc.select(qs, kh, J0, nc, gaps, qps, bk, G, causal, causal, 64,
                                      rows=(J - J0, J - J0 + 1))
                want_list = lists[0][0][J - J0]
                got_list = gpu.row(0, h, J - J0)
                if not np.array_equal(got_list, want_list):
                    diff = sorted(set(got_list.tolist()) ^ set(want_list.tolist()))[:10]
                    raise AssertionError(f"h={h} J={J}: {len(got_list)} vs {len(want_list)} "
                                         f"keys, differ at {diff}")
                if out_cpu is not None:
                    want = orc.attention(qh, kh, vh, qps, causal, bc, bi, [[[want_list]]], J0=J,
                                         nc=1)
                    r0, r1 = J * qps, min(S, (J + 1) * qps)
                    err = np.abs(out_cpu[0, h, r0:r1] - want[0, 0])
                    assert err.max() <= 2e-2 and err.mean() <= 2e-3, (h, J, err.max())
