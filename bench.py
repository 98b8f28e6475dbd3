"""Benchmark of the VecAttention prefill hot path on one MI355X.

A step is one VecAttention_prefill call (pooling + TilingSelect selection +
vector-sparse attention) on the seeded synthetic input of the workload, with
inputs resident in HBM.  Default workload: C (Qwen2.5-VL-shaped 128K causal
prefill, GQA 28/4, bf16, keep ~5%), the north-star shape; the same line
carries workload B (the 32K prefill) under "extra_workloads".

Prints ONE JSON line.  `value` is the end-to-end sparse-effective throughput
F_attn / t_step in TFLOP/s, where t_step is the timed VecAttention_prefill
step (ms_per_step) and F_attn counts the attention FLOPs actually executed
(4*D per query row per gathered key, local diagonal blocks counted whole).
Extra fields: per-stage latencies (the same kernels, timed stage by stage with
events on the launch stream), selection GB/s, the dense latencies on the
same GPU (PyTorch SDPA and this library's va_dense_attn) and the speedups of
the step over both, the roofline of the dominant kernel, and the CPU oracle
timed on a bounded sample over every host core.

Other modes (one JSON line each): --decode L (decode attention over an
L-token KV cache), --tuner (the threshold tuner's recall/sparsity evaluation).
"""
import argparse
import json
import math
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3  # MI355X fp32: dense matrix cores (and packed vector fp32)
FP64_PEAK_TFLOPS = 78.6   # MI355X fp64 (the exact selection kernel)
METRIC = "prefill attn latency (ms) + effective TFLOPS at 32k/128k; speedup vs dense"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="C", help="workload key A..E")
    ap.add_argument("--extra", default=None,
                    help="comma-separated workload keys measured after the headline and "
                         "reported under extra_workloads (default: B,D,E,A when the headline "
                         "is C; 'none' for none)")
    ap.add_argument("--no-dense", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--cpu-workers", type=int, default=None,
                    help="CPU baseline processes (default: every core of the affinity set)")
    ap.add_argument("--stage-reps", type=int, default=5)
    ap.add_argument("--extra-json", default=None, help="append the result line to this file too")
    ap.add_argument("--threshold", type=float, default=None,
                    help="use this threshold instead of calibrating one to the keep ratio")
    ap.add_argument("--decode", type=int, default=None, metavar="L",
                    help="time decode attention (single_decode_with_kv_cache) over a KV cache "
                         "of L tokens with the workload's heads instead of the prefill")
    ap.add_argument("--tuner", action="store_true",
                    help="time the threshold tuner's recall/sparsity evaluation "
                         "(seg_pr_perHead) on the workload's shapes instead of the prefill")
    return ap.parse_args()


# ------------------------------------------------------------ workload math --

def local_keys(J, qps, S, causal):
    if not causal:
        return 0
    if J == 0:
        return min(qps, S)
    return qps + min(qps, S - J * qps)


def attn_flops(counts_per_chunk, wl, S, Sk):
    """Executed attention FLOPs: 4*D * sum rows(J) * (count + local keys)."""
    qps, D = wl.q_pooling_size, wl.D
    total = 0
    for J0, cnt in counts_per_chunk:
        nc = cnt.shape[-1]
        J = torch.arange(J0, J0 + nc)
        rows = torch.clamp(S - J * qps, max=qps).double()
        loc = torch.tensor([local_keys(int(j), qps, Sk, wl.causal) for j in J], dtype=torch.float64)
        total += float((rows * (cnt.detach().cpu().double() + loc)).sum())
    return 4.0 * D * total


def dense_flops(wl, S, Sk):
    if wl.causal:
        return 4.0 * wl.D * wl.B * wl.Hq * S * (S + 1) / 2
    return 4.0 * wl.D * wl.B * wl.Hq * S * Sk


def selection_bytes(wl, S, Sk, sum_count, nqb):
    e = 2 if wl.dtype != torch.float32 else 4
    return (e * wl.B * wl.Hq * S * wl.D + e * wl.B * wl.Hk * Sk * wl.D + 4 * sum_count
            + 4 * wl.B * wl.Hq * nqb)


def selectable(wl, S):
    """Keys the rule can select (gap -> infinity), summed over rows."""
    qps = wl.q_pooling_size
    nqb = math.ceil(S / qps)
    if not wl.causal:
        return wl.B * wl.Hq * nqb * S
    bsq = 64
    tot = 0
    for i in range(0, S, wl.chunk_size):
        J0 = i // qps
        for jr in range(math.ceil(min(wl.chunk_size, S - i) / qps)):
            J = J0 + jr
            n = max(0, (J - 1) * qps)
            if jr % bsq == 0 and J >= 2:
                n -= qps - wl.k_local_size
            tot += n
    return wl.B * wl.Hq * tot


# ------------------------------------------------------------------ traffic --

def kernel_source_hash():
    """sha256 (first 16 hex digits) over the HIP sources and headers of the
    library, in name order: the key that ties a traffic profile to the
    kernels it measured."""
    import hashlib
    csrc = os.path.join(ROOT, "vecattention_amd", "csrc")
    h = hashlib.sha256()
    for name in sorted(os.listdir(csrc)):
        if name.endswith((".hip", ".h")):
            h.update(name.encode())
            with open(os.path.join(csrc, name), "rb") as f:
                h.update(f.read())
    return h.hexdigest()[:16]


def profiled_record(workload, kernel):
    """The record of `kernel` on `workload` in profiles/hbm_traffic.json, or None
    when not profiled or profiled on other kernel sources than the ones built now."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            doc = json.load(f)
        rec = doc["workloads"][workload][kernel]
    except (OSError, KeyError, ValueError):
        return None
    return rec if doc.get("source_hash") == kernel_source_hash() else None


def gather_ceiling(dev, work_groups=256 * 12, steps=512, reps=5):
    """Rate (TB/s) of the attention kernel's K/V copy instruction on its own
    (va_probe_gather: 256-byte rows at hashed ids into LDS, 8 copies in flight
    per wave), from a 2 MiB table (L2 hits) and a 64 MiB one (L2 misses served
    over the data fabric by the Infinity Cache)."""
    sys.path.insert(0, os.path.join(ROOT, "tests", "numerics"))
    import gather_probe
    from vecattention_amd import _native as nat
    sink = torch.empty(work_groups, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    moved = work_groups * 4 * steps * 1024
    rates = {}
    for name, mib in (("l2", 2), ("fabric", 64)):
        rows = (mib << 20) // 256
        table = torch.ones(rows * 256, dtype=torch.uint8, device=dev)
        call = lambda: gather_probe.gather(nat.ptr(table), rows, work_groups, steps, 0,
                                           nat.ptr(sink), stream)
        call()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            call()
        b.record()
        torch.cuda.synchronize()
        rates[name] = moved / (a.elapsed_time(b) / reps * 1e-3) / 1e12
        del table
    return rates


def profiled_traffic(workload, kernel):
    """Bytes per launch of `kernel` on `workload` crossing between L2 and the
    data fabric (reads + writes; fabric reads include those the Infinity
    Cache serves), counted exactly from the TCC_EA0 request-size counters in
    the rocprofv3 --pmc runs summarised in profiles/hbm_traffic.json, and the
    compulsory bytes of that launch (None where not recorded).  (None, None)
    when not profiled, or when the profile was taken on other kernel sources
    than the ones built now (its source_hash differs)."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    try:
        with open(path) as f:
            doc = json.load(f)
        rec = doc["workloads"][workload][kernel]
    except (OSError, KeyError, ValueError):
        return None, None
    if doc.get("source_hash") != kernel_source_hash():
        return None, None
    return int(round(rec["fetch_bytes"] + rec["write_bytes"])), rec.get("compulsory_bytes")


# ------------------------------------------------------------------- stages --

def prefill_plan(wl, q, k, v, out):
    """va_prefill_kernels' bit set for these tensors: the kernels the prefill runs."""
    from vecattention_amd import _native as nat
    return nat.check_flags("va_prefill_kernels", nat.lib().va_prefill_kernels(
        nat.dtype_code(q), nat.ptr(q), q.stride(0), q.stride(1), q.stride(2), nat.ptr(k),
        k.stride(0), k.stride(1), k.stride(2), nat.ptr(v), v.stride(0), v.stride(1), v.stride(2),
        nat.ptr(out), out.stride(0), out.stride(1), out.stride(2), q.shape[1], k.shape[1],
        k.shape[2], q.shape[3], wl.q_pooling_size, wl.k_local_size, wl.group_k_block))


def run_stages(wl, q, k, v, gap, out, events=None):
    """Pool + per-chunk select/attention through the stage API (same kernels
    as VecAttention_prefill).  Returns per-chunk counts; records events."""
    from vecattention_amd import _native as nat
    from vecattention_amd import stages
    qps, S = wl.q_pooling_size, q.shape[2]
    # the key segments the prefill uses, when its plan splits the selection
    plan = prefill_plan(wl, q, k, v, out)
    exact = bool(plan & nat.VA_KERNELS_SELECT_EXACT)
    segk = (stages.segment_keys(k.shape[2], wl.k_local_size, wl.group_k_block, exact=exact)
            if plan & nat.VA_KERNELS_SPLIT else 0)
    ev = events
    if ev is not None:
        ev["p0"].record()
    qs, _ = stages.pool_scaled(q, qps)
    if ev is not None:
        ev["p1"].record()
    res = []
    nqb = qs.shape[2]
    idx_buf = scr_buf = None
    if segk:  # buffers for the largest chunk, reused (as the prefill's workspace is)
        B, Hq, Hk, Sk = q.shape[0], q.shape[1], k.shape[1], k.shape[2]
        caps, scrs = [], []
        for i in range(0, S, wl.chunk_size):
            J0, nc = i // qps, math.ceil(min(wl.chunk_size, S - i) / qps)
            caps.append(stages.index_capacity(B, Hq, Sk, qps, wl.causal, wl.causal, J0, nc))
            scrs.append(int(stages.nat.lib().va_select_segments_scratch_floats(
                B, Hq, Hk, Sk, nc, segk, wl.k_local_size, wl.group_k_block)))
        idx_buf = torch.empty(max(max(caps), 1), dtype=torch.int32, device=q.device)
        scr_buf = torch.empty(max(max(scrs), 1), dtype=torch.float32, device=q.device)
    for ci, i in enumerate(range(0, S, wl.chunk_size)):
        J0 = i // qps
        nc = math.ceil(min(wl.chunk_size, S - i) / qps)
        if ev is not None:
            ev[f"s0_{ci}"].record()
        if segk:
            cnt, idx = stages.select_segments(qs[:, :, J0:J0 + nc], k, J0, gap, None, wl.causal,
                                              qps, wl.k_local_size, wl.group_k_block, wl.causal,
                                              segk, indices=idx_buf, scratch=scr_buf)
        else:
            cnt, idx = stages.select_rows(qs[:, :, J0:J0 + nc], k, J0, gap, None, wl.causal, qps,
                                          wl.k_local_size, wl.group_k_block, wl.causal)
        if ev is not None:
            ev[f"s1_{ci}"].record()
        stages.sparse_attention(q, k, v, out, J0, nc, cnt, idx, wl.causal, qps, segk=segk)
        if ev is not None:
            ev[f"a1_{ci}"].record()
        res.append((J0, cnt.sum(-1) if segk else cnt))
    return res


class StreamHold:
    """Holds the current stream with torch's spin kernel while the host
    enqueues work behind it, so that events recorded between those launches
    time the kernels and not the host's launch gaps (at the small
    configurations a launch from Python takes longer than its kernel)."""

    def __init__(self):
        self.ms_per_cycle = None
        try:
            cyc = 2_000_000
            torch.cuda._sleep(cyc)  # first launch (module load) outside the calibration
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            torch.cuda._sleep(cyc)
            b.record()
            torch.cuda.synchronize()
            self.ms_per_cycle = a.elapsed_time(b) / cyc
        except (AttributeError, RuntimeError) as e:  # no spin kernel: events time the gaps too
            print(f"[bench] no stream hold ({e})", file=sys.stderr, flush=True)

    def __call__(self, ms):
        if self.ms_per_cycle and ms > 0:
            torch.cuda._sleep(int(min(ms, 200.0) / self.ms_per_cycle))


def calibrate_threshold(wl, q, k, v, out):
    """Bisection on the threshold for the workload's keep ratio (GPU selection)."""
    target = wl.keep * selectable(wl, q.shape[2])
    lo, hi = 1e-8, 1.0
    for _ in range(16):
        th = math.sqrt(lo * hi)
        gap = -math.log(th + 1e-9)
        counts = count_only(wl, q, k, gap)
        if counts > target:
            lo = th
        else:
            hi = th
    return math.sqrt(lo * hi)


def count_only(wl, q, k, gap):
    from vecattention_amd import stages
    qps, S = wl.q_pooling_size, q.shape[2]
    qs, _ = stages.pool_scaled(q, qps)
    tot = 0
    for i in range(0, S, wl.chunk_size):
        J0 = i // qps
        nc = math.ceil(min(wl.chunk_size, S - i) / qps)
        cnt, _ = stages.select_rows(qs[:, :, J0:J0 + nc], k, J0, gap, None, wl.causal, qps,
                                    wl.k_local_size, wl.group_k_block, wl.causal)
        tot += int(cnt.sum().item())
    return tot


def time_dense(wl, q, k, v, reps=10, warmup=3):
    """PyTorch SDPA (flash backend only; never the bf16 math path) on the same GPU."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    for backend in (SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION):
        try:
            with sdpa_kernel([backend]):
                kk, vv = k, v
                if wl.Hq != wl.Hk:
                    kk = k.repeat_interleave(wl.Hq // wl.Hk, dim=1).contiguous()
                    vv = v.repeat_interleave(wl.Hq // wl.Hk, dim=1).contiguous()
                f = lambda: torch.nn.functional.scaled_dot_product_attention(  # noqa: E731
                    q, kk, vv, is_causal=wl.causal)
                for _ in range(warmup):
                    f()
                torch.cuda.synchronize()
                ts = []
                for _ in range(reps):
                    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    a.record()
                    f()
                    b.record()
                    torch.cuda.synchronize()
                    ts.append(a.elapsed_time(b))
                del kk, vv
                return statistics.median(ts), str(backend).split(".")[-1]
        except RuntimeError as e:  # backend unavailable for this shape
            last = str(e)
            continue
    return None, f"unavailable: {last[:80]}"


def time_dense_va(wl, q, k, v, reps=5, warmup=2):
    """This library's dense attention (va_dense_attn, the Full_prefill path) on
    the same tensors: every key, causal rows bottom-right aligned, GQA read in
    place."""
    from vecattention_amd import stages
    out = torch.empty_like(q)
    f = lambda: stages.dense_attention(q, k, v, out, causal=wl.causal)  # noqa: E731
    for _ in range(warmup):
        f()
    torch.cuda.synchronize()
    ts = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        f()
        b.record()
        torch.cuda.synchronize()
        ts.append(a.elapsed_time(b))
    del out
    return statistics.median(ts)


# --------------------------------------------------------------- CPU oracle --

def host_cpu_model():
    """The CPU model named by /proc/cpuinfo (else the machine type)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_baseline(wl, q_cpu, k_cpu, v_cpu, threshold, seconds, workers=None):
    """The CPU oracle (C selection + numpy fp32 attention, one thread per
    process) on q-blocks sampled uniformly over the workload's (q head,
    q-block) pairs, spread over one child process per host core in the
    process's affinity set (oracle/sample_worker.py; the children never touch
    the GPU).  Each child works through its share of the sample for `seconds`;
    the value is the sample's executed attention FLOPs over the slowest
    child's time, in TFLOP/s, with selection and attention times reported
    separately."""
    import json as _json
    import shutil
    import subprocess
    import tempfile

    import numpy as np

    from oracle import oracle as orc
    qps, S, D = wl.q_pooling_size, q_cpu.shape[2], wl.D
    rep = wl.Hq // wl.Hk
    dt = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}[wl.dtype]
    nqb = math.ceil(S / qps)
    n = workers or len(os.sched_getaffinity(0))
    rng = np.random.default_rng(0)
    # one q head per kv group (heads cost the same), q-blocks uniform over the
    # sequence; enough samples that no child runs out before its time is up
    heads = [g * rep for g in range(wl.Hk)][:4]
    samples = [(int(rng.choice(heads)), int(rng.integers(0, nqb))) for _ in range(4000 * n)]
    base = "/dev/shm" if os.path.isdir("/dev/shm") else None
    tmp = tempfile.mkdtemp(prefix="va_cpu_", dir=base)
    try:
        for h in heads:
            qh = q_cpu[:, h:h + 1].float().numpy()
            np.save(os.path.join(tmp, f"q_{h}.npy"), qh[0, 0])
            np.save(os.path.join(tmp, f"qs_{h}.npy"), orc.pool(qh, qps, dt)[1][0, 0])
        for g in sorted({h // rep for h in heads}):
            np.save(os.path.join(tmp, f"k_{g}.npy"), k_cpu[0, g].float().numpy())
            np.save(os.path.join(tmp, f"v_{g}.npy"), v_cpu[0, g].float().numpy())
        meta = {"qps": qps, "bk": wl.k_local_size, "G": wl.group_k_block, "causal": wl.causal,
                "chunk": wl.chunk_size, "S": S, "Sk": k_cpu.shape[2], "D": D, "rep": rep,
                "threshold": threshold, "samples": samples}
        with open(os.path.join(tmp, "meta.json"), "w") as f:
            _json.dump(meta, f)
        env = dict(os.environ, OMP_NUM_THREADS="1", OPENBLAS_NUM_THREADS="1",
                   MKL_NUM_THREADS="1", HIP_VISIBLE_DEVICES="", CUDA_VISIBLE_DEVICES="")
        procs = [subprocess.Popen([sys.executable, "-m", "oracle.sample_worker", tmp, str(w), str(n),
                                   str(seconds)], cwd=ROOT, env=env, stdout=subprocess.PIPE,
                                  text=True) for w in range(n)]
        res = []
        for p in procs:
            out, _ = p.communicate()
            if p.returncode != 0:
                raise RuntimeError(f"cpu baseline worker exited with {p.returncode}")
            res.append(_json.loads(out.strip().splitlines()[-1]))
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    flops = sum(r["flops"] for r in res)
    blocks = sum(r["blocks"] for r in res)
    el = max(r["elapsed"] for r in res)
    t_sel = sum(r["t_sel"] for r in res)
    t_attn = sum(r["t_attn"] for r in res)
    return {"value": flops / el / 1e12, "unit": "TFLOP/s", "cores": n, "kind": "port",
            "sample": f"oracle (C selection, numpy fp32 attention) on {blocks} q-blocks drawn "
                      f"uniformly over q heads {heads} and all {nqb} q-blocks of workload "
                      f"{wl.name}, {n} processes x {el:.1f} s",
            "selection_s_per_qblock": round(t_sel / max(blocks, 1), 5),
            "attention_s_per_qblock": round(t_attn / max(blocks, 1), 5),
            "host_cpu": host_cpu_model(),
            "host_threads_available": len(os.sched_getaffinity(0))}


def cpu_full_run(wl, q_cpu, k_cpu, v_cpu, threshold, F_attn, reps=3):
    """The whole prefill on the CPU oracle (oracle.prefill: C selection, numpy
    attention) in fp32 arithmetic for the attention, on the host cores of this
    box: 1 warmup + `reps` timed runs, median.  The C selection is single
    threaded; numpy's BLAS uses the threads its environment allows."""
    import numpy as np

    from oracle import oracle as orc
    dt = {torch.bfloat16: "bfloat16", torch.float16: "float16", torch.float32: "float32"}[wl.dtype]
    run = lambda: orc.prefill(q_cpu, k_cpu, v_cpu, threshold, wl.q_pooling_size,
                              wl.k_local_size, wl.group_k_block, wl.causal, wl.chunk_size, 64, dt,
                              acc=np.float32)
    run()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    return {"ms": round(med * 1e3, 2), "value": F_attn / med / 1e12, "unit": "TFLOP/s",
            "reps": reps, "warmup": 1, "kind": "port",
            "threads": {"blas": os.environ.get("OMP_NUM_THREADS", "unset"), "selection": 1},
            "host_cpu": host_cpu_model(),
            "host_threads_available": len(os.sched_getaffinity(0)),
            "sample": f"whole workload {wl.name}: oracle.prefill (fp32 attention), median of "
                      f"{reps} runs after 1 warmup"}


# -------------------------------------------------------------------- tuner --

def bench_tuner(args, wl, dev):
    """One seg_pr_perHead call (spattn/threshold/model_tuner.py:118-226) per
    step on the workload's shapes: fp32 Q/K holding bf16 values (the tuner's
    load_tensor copies of the dumped states), K expanded to the q heads (the
    dumps follow repeat_kv), a per-head threshold vector around the first
    bisection midpoint, chunk 8192 (the reference's default).  Beside it: the
    dense-statistics kernel alone (its MFMA roofline) and the reference's
    dense step (matmul + mask + fp32 softmax of model_tuner.py:193-199) timed
    in torch on the same GPU for one (head, chunk) and scaled to the call, a
    lower bound of the reference's evaluation (its mask loops excluded)."""
    from vecattention_amd import stages, tuner
    from vecattention_amd.synth import workload_inputs
    q_cpu, k_cpu, _ = workload_inputs(wl, seed=0)
    rep = wl.Hq // wl.Hk
    q = q_cpu.float().to(dev)
    k = k_cpu.repeat_interleave(rep, dim=1).float().to(dev)
    B, H, S, D = q.shape
    base = args.threshold if args.threshold is not None else 0.25
    th = (base * torch.linspace(0.8, 1.2, H)).clamp(max=0.999).to(dev)
    chunk = 8 * 1024

    def call():
        return tuner.seg_pr_perHead(q, k, wl.q_pooling_size, wl.k_local_size, wl.group_k_block,
                                    threshold=th, chunk_size=chunk, causal=wl.causal)

    def timed(fn, reps, warm):
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(reps):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b))
        return statistics.median(ts)

    for _ in range(args.warmup):
        r, sp = call()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        r, sp = call()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / max(args.steps, 1)
    print(f"[bench] tuner: {ms:.3f} ms per seg_pr_perHead; recall {r.mean().item():.4f} "
          f"sparsity {sp.mean().item():.4f}", file=sys.stderr, flush=True)

    qb, kb = q.to(torch.bfloat16), k.to(torch.bfloat16)
    stats = torch.empty(B, H, S, 2, dtype=torch.float32, device=dev)
    t_dense = timed(lambda: stages.dense_row_stats(qb, kb, wl.causal, stats=stats), 5, 2)
    visible = S * (S + 1) // 2 if wl.causal else S * S
    F_dense = 2 * D * B * H * visible
    dense_tflops = F_dense / (t_dense * 1e-3) / 1e12

    rows = min(chunk, S)
    mask = None
    if wl.causal:
        mask = torch.triu(torch.full((rows, S), float("-inf"), device=dev), diagonal=1)

    def ref_dense():
        a = torch.matmul(q[0, 0, :rows], k[0, 0].transpose(-2, -1)) / math.sqrt(D)
        if mask is not None:
            a = a + mask
        return torch.softmax(a, dim=-1, dtype=torch.float32)
    t_ref = timed(ref_dense, 3, 1) * B * H * math.ceil(S / chunk)
    result = {
        "metric": "tuner seg_pr_perHead latency (ms)",
        "value": round(ms, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32 inputs (bf16 values), bf16 MFMA scores, fp32 sums",
        "data": "synthetic (the workload's seeded inputs as fp32 copies)",
        "config": {"workload": "tuner-" + wl.name, "B": B, "H": H, "S": S, "D": D,
                   "causal": wl.causal, "block_size_q": wl.q_pooling_size,
                   "block_size_k": wl.k_local_size, "group_size_k": wl.group_k_block,
                   "chunk_size": chunk, "threshold_base": base},
        "dense_stats_ms": round(t_dense, 4),
        "reference_dense_step_ms_lower_bound": round(t_ref, 2),
        "speedup_vs_reference_dense_step": round(t_ref / ms, 2),
        "roofline": {"bound": "mfma", "kernel": "attn_mfma_kernel (dense statistics form)",
                     "achieved": round(dense_tflops, 3), "peak": BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(dense_tflops / BF16_PEAK_TFLOPS, 4),
                     "traffic": None},
        "recall_mean": round(r.mean().item(), 6),
        "sparsity_mean": round(sp.mean().item(), 6),
    }
    line = json.dumps(result)
    print(line, flush=True)
    if args.extra_json:
        with open(args.extra_json, "a") as f:
            f.write(line + "\n")


# ------------------------------------------------------------------- decode --

def bench_decode(args, wl, dev):
    """Decode attention of one token over an L-token KV cache with the
    workload's heads (q (Hq, D), K/V NHD (L, Hk, D), bf16), as the reference's
    decode branch calls flashinfer (load_qwen2p5_vl.py:61-66), but on the
    unexpanded kv heads.  HBM roofline: K and V are read once (2 * L * Hk * D
    elements); q and the output are negligible.  Baseline: torch SDPA
    (enable_gqa) on the same GPU and tensors."""
    from vecattention_amd.decode import single_decode_with_kv_cache
    L, Hq, Hk, D = args.decode, wl.Hq, wl.Hk, wl.D
    g = torch.Generator().manual_seed(0)
    q = torch.randn(Hq, D, generator=g).to(wl.dtype).to(dev)
    k = torch.randn(L, Hk, D, generator=g).to(wl.dtype).to(dev)
    v = torch.randn(L, Hk, D, generator=g).to(wl.dtype).to(dev)
    esz = torch.tensor([], dtype=wl.dtype).element_size()
    kv_bytes = 2 * L * Hk * D * esz

    def timed(fn, reps, warm):
        for _ in range(warm):
            fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    call = lambda: single_decode_with_kv_cache(q, k, v, kv_layout="NHD")  # noqa: E731
    steps = max(args.steps, 1) * 20
    ms = timed(call, steps, max(args.warmup, 1) * 5)
    gbs = kv_bytes / (ms * 1e-3) / 1e9
    print(f"[bench] decode L={L}: {ms * 1e3:.1f} us per call, {gbs:.0f} GB/s", file=sys.stderr,
          flush=True)
    qs, ks, vs = q[None, :, None, :], k.permute(1, 0, 2)[None], v.permute(1, 0, 2)[None]
    sdpa_ms = None
    try:
        sdpa = lambda: torch.nn.functional.scaled_dot_product_attention(  # noqa: E731
            qs, ks, vs, enable_gqa=True)
        sdpa_ms = timed(sdpa, steps, 5)
    except RuntimeError as e:
        print(f"[bench] SDPA unavailable: {str(e)[:80]}", file=sys.stderr, flush=True)
    result = {
        "metric": "decode attention latency (us)",
        "value": round(ms * 1e3, 2),
        "unit": "us",
        "n_gpus": 1,
        "steps": steps,
        "warmup": max(args.warmup, 1) * 5,
        "ms_per_step": round(ms, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float16: "fp16"}.get(wl.dtype, "fp32"),
        "data": "synthetic (seeded N(0,1) q, K and V)",
        "config": {"workload": f"decode-{wl.name}-L{L}", "Hq": Hq, "Hk": Hk, "D": D, "L": L,
                   "kv_layout": "NHD"},
        "sdpa_us": None if sdpa_ms is None else round(sdpa_ms * 1e3, 2),
        "speedup_vs_sdpa": None if sdpa_ms is None else round(sdpa_ms / ms, 2),
        "roofline": {"bound": "hbm", "kernel": "attn_mfma_kernel (split form) + decode_merge_kernel",
                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
    }
    line = json.dumps(result)
    print(line, flush=True)
    if args.extra_json:
        with open(args.extra_json, "a") as f:
            f.write(line + "\n")


# --------------------------------------------------------------------- main --

def measure_prefill(args, wl, dev, with_cpu):
    """Measure one workload: calibrated threshold, stage timing, the timed
    VecAttention_prefill steps, the dense baselines and (optionally) the CPU
    baseline.  Returns the result dictionary of the JSON line."""
    from vecattention_amd import VecAttention_prefill
    from vecattention_amd.synth import workload_inputs

    t_gen = time.perf_counter()
    q_cpu, k_cpu, v_cpu = workload_inputs(wl, seed=0)
    q, k, v = q_cpu.to(dev), k_cpu.to(dev), v_cpu.to(dev)
    print(f"[bench] {wl.name}: inputs ready in {time.perf_counter() - t_gen:.1f}s", file=sys.stderr,
          flush=True)
    S, Sk = q.shape[2], k.shape[2]
    out = torch.empty_like(q)

    th = args.threshold if args.threshold is not None else calibrate_threshold(wl, q, k, v, out)
    gap = -math.log(th + 1e-9)
    print(f"[bench] threshold {th:.6g} (gap {gap:.6g})", file=sys.stderr, flush=True)

    # ---- per-stage timing through the stage API ----
    nch = math.ceil(S / wl.chunk_size)
    names = ["p0", "p1"] + [f"{p}_{c}" for c in range(nch) for p in ("s0", "s1", "a1")]
    t_pool, t_sel, t_attn = [], [], []
    counts = None
    hold = StreamHold()
    hold_ms = 0.0
    for r in range(max(args.stage_reps, 1) + 1):
        ev = {n: torch.cuda.Event(enable_timing=True) for n in names}
        hold(hold_ms)
        h0 = time.perf_counter()
        counts = run_stages(wl, q, k, v, gap, out, ev)
        host_ms = (time.perf_counter() - h0) * 1e3  # the host's time to enqueue the pass
        torch.cuda.synchronize()
        if r == 0:
            gpu_ms = ev["p0"].elapsed_time(ev[f"a1_{nch - 1}"])
            # Short passes (A, B, D: a few ms or less) are held: launches
            # that reach an idle GPU there add tens of microseconds of gaps
            # and dispatch latency inside the stages (B's attention measured
            # 6-11% slower unheld than its kernel trace), and so are passes
            # the host takes long to enqueue (a tracer's launch overhead).
            # Long passes (C, E) are not: the GPU idles through the hold and
            # starts the pass at a lower clock (C's stages 5% slower held).
            if gpu_ms < 5.0 or host_ms > 0.5 * gpu_ms:
                hold_ms = 2.0 * host_ms + 1.0
            print(f"[bench] stage pass: host enqueue {host_ms:.3f} ms, GPU {gpu_ms:.3f} ms; "
                  f"stream hold {hold_ms:.3f} ms", file=sys.stderr, flush=True)
            continue
        t_pool.append(ev["p0"].elapsed_time(ev["p1"]))
        t_sel.append(sum(ev[f"s0_{c}"].elapsed_time(ev[f"s1_{c}"]) for c in range(nch)))
        t_attn.append(sum(ev[f"s1_{c}"].elapsed_time(ev[f"a1_{c}"]) for c in range(nch)))
    t_pool, t_sel, t_attn = (statistics.median(x) for x in (t_pool, t_sel, t_attn))
    F_attn = attn_flops(counts, wl, S, Sk)
    F_dense = dense_flops(wl, S, Sk)
    sum_count = sum(int(c.sum().item()) for _, c in counts)
    nqb = math.ceil(S / wl.q_pooling_size)
    sel_bytes = selection_bytes(wl, S, Sk, sum_count, nqb)
    keep = sum_count / selectable(wl, S)
    print(f"[bench] stages: pool {t_pool:.3f} ms, select {t_sel:.3f} ms, attn {t_attn:.3f} ms; "
          f"keep {keep:.4f}", file=sys.stderr, flush=True)

    # ---- the timed steps: whole VecAttention_prefill calls ----
    def step():
        return VecAttention_prefill(q, k, v, threshold=th, q_pooling_size=wl.q_pooling_size,
                                    k_local_size=wl.k_local_size, group_k_block=wl.group_k_block,
                                    causal=wl.causal, chunk_size=wl.chunk_size)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / max(args.steps, 1)
    print(f"[bench] {args.steps} steps: {ms_per_step:.3f} ms/step", file=sys.stderr, flush=True)

    dense_ms, dense_backend, dense_va_ms = (None, "skipped", None)
    if not args.no_dense:
        dense_ms, dense_backend = time_dense(wl, q, k, v)
        print(f"[bench] dense SDPA ({dense_backend}): {dense_ms} ms", file=sys.stderr, flush=True)
        dense_va_ms = time_dense_va(wl, q, k, v)
        print(f"[bench] dense va_dense_attn: {dense_va_ms:.3f} ms", file=sys.stderr, flush=True)

    t_sel_total = t_pool + t_sel
    # value: the whole VecAttention_prefill step, as timed above
    e2e_tflops = F_attn / (ms_per_step * 1e-3) / 1e12
    attn_tflops = F_attn / (t_attn * 1e-3) / 1e12
    from vecattention_amd import _native as nat
    plan = prefill_plan(wl, q, k, v, out)
    attn_mfma = bool(plan & nat.VA_KERNELS_ATTN_MFMA)
    attn_f32 = bool(plan & nat.VA_KERNELS_ATTN_F32)
    attn_kernel = ("attn_mfma_kernel" if attn_mfma else "attn_f32_kernel" if attn_f32
                   else "attn_simple_kernel")
    attn_peak = BF16_PEAK_TFLOPS if attn_mfma else FP32_PEAK_TFLOPS
    attn_bound = "mfma" if attn_mfma else "mfma-fp32" if attn_f32 else "valu-fp32"
    # Selection (pooling + TilingSelect) against max(Bytes_sel / HBM peak,
    # F_sel / the scoring kernel's peak): F_sel = 2*D per selectable (row, key).
    F_sel = 2.0 * wl.D * selectable(wl, S)
    sel_peak = FP64_PEAK_TFLOPS if plan & nat.VA_KERNELS_SELECT_EXACT else BF16_PEAK_TFLOPS
    t_bytes = sel_bytes / (HBM_PEAK_GBS * 1e9) * 1e3
    t_flops = F_sel / (sel_peak * 1e12) * 1e3
    sel_roof = {"bound": "hbm" if t_bytes >= t_flops else "mfma" if sel_peak == BF16_PEAK_TFLOPS
                else "fp64", "bytes": sel_bytes, "flops": F_sel,
                "t_bound_ms": round(max(t_bytes, t_flops), 4), "t_ms": round(t_sel_total, 4),
                "frac": round(max(t_bytes, t_flops) / t_sel_total, 4)}
    traffic, compulsory = profiled_traffic(wl.name, "attn_mfma_kernel")
    # The attention's K/V gathers against the copy instruction's own rate: K and
    # V rows of every (q-block, key) pair, F_attn * elem / (2 * qps) bytes.
    es = q.element_size()
    gathered = F_attn * es / (2 * wl.q_pooling_size)
    gather_rate = gathered / (t_attn * 1e-3) / 1e12
    ceil = gather_ceiling(dev) if attn_mfma else {"l2": float("nan"), "fabric": float("nan")}
    rec = profiled_record(wl.name, "attn_mfma_kernel")
    l2_share = None if rec is None or "fabric_over_gathered" not in rec else \
        max(0.0, 1.0 - rec["fabric_over_gathered"])
    mix = None if l2_share is None else \
        1.0 / (l2_share / ceil["l2"] + (1.0 - l2_share) / ceil["fabric"])
    if attn_mfma:  # the per-row kernel gathers through L1 loads, not the copy instruction
        print(f"[bench] gathers {gather_rate:.2f} TB/s; copy-instruction ceiling {ceil['l2']:.2f} "
              f"(L2) / {ceil['fabric']:.2f} (fabric) TB/s", file=sys.stderr, flush=True)
    result = {
        "metric": METRIC,
        "value": round(e2e_tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[wl.dtype],
        "data": "synthetic (seeded N(0,1) + vertical-column and frame structure; threshold "
                "calibrated to the keep ratio)",
        "config": {"workload": wl.name, "B": wl.B, "Hq": wl.Hq, "Hk": wl.Hk, "S": S, "D": wl.D,
                   "causal": wl.causal, "q_pooling_size": wl.q_pooling_size,
                   "k_local_size": wl.k_local_size, "group_k_block": wl.group_k_block,
                   "chunk_size": wl.chunk_size, "threshold": th, "keep": round(keep, 5),
                   "parallelism": "single GPU"},
        "latency_ms": {"pool": round(t_pool, 4), "select": round(t_sel, 4),
                       "attn": round(t_attn, 4), "total": round(t_sel_total + t_attn, 4)},
        "sparse_attn_tflops": round(attn_tflops, 3),
        "selection_gbs": round(sel_bytes / (t_sel_total * 1e-3) / 1e9, 1),
        "selection_hbm_frac": round(sel_bytes / (t_sel_total * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "selection_roofline": sel_roof,
        "dense_ms": None if dense_ms is None else round(dense_ms, 4),
        "dense_backend": dense_backend,
        "speedup_vs_dense": None if dense_ms is None else round(dense_ms / ms_per_step, 3),
        "dense_va_ms": None if dense_va_ms is None else round(dense_va_ms, 4),
        "dense_va_tflops": None if dense_va_ms is None else round(F_dense / (dense_va_ms * 1e-3) / 1e12, 1),
        "speedup_vs_dense_va": None if dense_va_ms is None else round(dense_va_ms / ms_per_step, 3),
        "roofline": {"bound": attn_bound, "kernel": attn_kernel,
                     "achieved": round(attn_tflops, 3), "peak": attn_peak,
                     "unit": "TFLOP/s", "frac": round(attn_tflops / attn_peak, 4),
                     "traffic": traffic,
                     "traffic_kind": "L2<->fabric bytes per launch (exact, from the TCC_EA0 "
                                     "request-size counters; Infinity Cache hits included)",
                     "traffic_over_compulsory": (round(traffic / compulsory, 2)
                                                 if traffic and compulsory else None),
                     "gather": None if not attn_mfma else {
                         "achieved_TBps": round(gather_rate, 3),
                         "ceiling_l2_TBps": round(ceil["l2"], 3),
                         "ceiling_fabric_TBps": round(ceil["fabric"], 3),
                         "l2_share_profiled": None if l2_share is None else round(l2_share, 3),
                         "ceiling_at_l2_share_TBps": None if mix is None else round(mix, 3),
                         "frac_of_ceiling_at_l2_share": None if mix is None else
                         round(gather_rate / mix, 3),
                         "frac_of_l2_ceiling": round(gather_rate / ceil["l2"], 3)}},
        "flops": {"attn_executed": F_attn, "dense": F_dense},
    }
    if with_cpu:
        result["cpu_baseline"] = cpu_baseline(wl, q_cpu, k_cpu, v_cpu, th, args.cpu_seconds,
                                              args.cpu_workers)
    if wl.dtype == torch.float32 and not args.no_cpu:
        # the workload small enough for the whole CPU path (the fp32 CPU
        # reference configuration): 1 warmup + 3 reps, median
        result["cpu_full"] = cpu_full_run(wl, q_cpu, k_cpu, v_cpu, th, F_attn)
    del q, k, v, out
    torch.cuda.empty_cache()
    return result


EXTRA_KEYS = ("ms_per_step", "value", "config", "latency_ms", "sparse_attn_tflops", "selection_gbs",
              "selection_hbm_frac", "selection_roofline", "dense_ms", "dense_backend",
              "speedup_vs_dense", "dense_va_ms", "dense_va_tflops", "speedup_vs_dense_va",
              "roofline", "flops", "cpu_full")


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for "
              f"--gpus {args.gpus}); per-GPU sharding is by (batch, kv head) and needs no "
              f"collective (see DESIGN.md).", file=sys.stderr)
        sys.exit(2)
    from vecattention_amd.synth import WORKLOADS

    wl = WORKLOADS[args.config]
    dev = torch.device("cuda:0")
    if args.tuner:
        bench_tuner(args, wl, dev)
        return
    if args.decode:
        bench_decode(args, wl, dev)
        return
    extra = args.extra if args.extra is not None else ("B,D,E,A" if args.config == "C" else "none")
    extra = [] if extra.lower() == "none" else [x for x in extra.split(",") if x]
    result = measure_prefill(args, wl, dev, with_cpu=not args.no_cpu)
    if extra:
        saved_th = args.threshold
        args.threshold = None  # each extra workload calibrates its own threshold
        result["extra_workloads"] = {}
        for key in extra:
            r = measure_prefill(args, WORKLOADS[key], dev, with_cpu=False)
            result["extra_workloads"][r["config"]["workload"]] = {k: r[k] for k in EXTRA_KEYS
                                                                  if k in r}
        args.threshold = saved_th
    line = json.dumps(result)
    print(line, flush=True)
    if args.extra_json:
        with open(args.extra_json, "a") as f:
            f.write(line + "\n")


if __name__ == "__main__":
    main()
