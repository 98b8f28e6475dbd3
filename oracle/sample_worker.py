"""CPU baseline worker — TEST INFRASTRUCTURE ONLY.

Run by bench.py's cpu_baseline leg as a child process (one per host core):
it times the CPU oracle (C selection + numpy fp32 attention, one thread) on
its share of the sampled q-blocks of a workload and prints one JSON line.
It imports numpy and the oracle only (no torch, no GPU).

    python -m oracle.sample_worker DATA_DIR WORKER_ID N_WORKERS SECONDS

DATA_DIR holds meta.json (shapes, rule parameters, threshold and the sample
list of (q head, q-block) pairs) and, per sampled q head h, q_h.npy (the
head's queries), qs_h.npy (its scaled pooled rows) and, per kv head g,
k_g.npy / v_g.npy, all float32.  Worker w takes samples w, w + n, w + 2n, ...
until SECONDS have passed.
"""
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import oracle as orc  # noqa: E402


def local_keys(J, qps, Sk, causal):
    """Keys of the initial and diagonal 64-key blocks of q-block J (counted whole)."""
    if not causal:
        return 0
    if J == 0:
        return min(qps, Sk)
    return qps + min(qps, Sk - J * qps)


def main():
    data_dir, wid, nw, seconds = sys.argv[1], int(sys.argv[2]), int(sys.argv[3]), float(sys.argv[4])
    with open(os.path.join(data_dir, "meta.json")) as f:
        meta = json.load(f)
    qps, bk, G = meta["qps"], meta["bk"], meta["G"]
    causal, chunk, S, Sk, D, rep = (meta["causal"], meta["chunk"], meta["S"], meta["Sk"], meta["D"],
                                    meta["rep"])
    nqb = math.ceil(S / qps)
    gaps = orc.gap_from_threshold(meta["threshold"], 1, 1)
    bc, bi = orc.local_blocks(1, 1, S, qps, causal)
    arrays = {}

    def head(name):
        if name not in arrays:
            arrays[name] = np.load(os.path.join(data_dir, name + ".npy"), mmap_mode="r")
        return arrays[name]

    orc.lib()
    samples = meta["samples"][wid::nw]
    flops = t_sel = t_attn = 0.0
    done = 0
    t0 = time.perf_counter()
    for h, J in samples:
        g = h // rep
        qh, qs = head(f"q_{h}"), head(f"qs_{h}")
        kh, vh = head(f"k_{g}"), head(f"v_{g}")
        c0 = (J * qps) // chunk * (chunk // qps)
        ncc = min(chunk // qps, nqb - c0)
        a = time.perf_counter()
        cnt, lists = orc.select(qs[None, None], kh[None, None], c0, ncc, gaps, qps, bk, G, causal,
                                causal, 64, rows=(J - c0, J - c0 + 1))
        b = time.perf_counter()
        orc.attention(qh[None, None], kh[None, None], vh[None, None], qps, causal, bc, bi,
                      [[lists[0][0][J - c0:J - c0 + 1]]], J0=J, nc=1, acc=np.float32)
        c = time.perf_counter()
        t_sel += b - a
        t_attn += c - b
        rows = min(qps, S - J * qps)
        flops += 4.0 * D * rows * (int(cnt[0, 0, J - c0]) + local_keys(J, qps, Sk, causal))
        done += 1
        if c - t0 > seconds:
            break
    print(json.dumps({"worker": wid, "flops": flops, "blocks": done, "t_sel": t_sel,
                      "t_attn": t_attn, "elapsed": time.perf_counter() - t0}), flush=True)


if __name__ == "__main__":
    main()
