"""Seeded synthetic inputs with vertical (column) structure, for parity tests
and benchmarks.  No dataset or checkpoint is needed.

Per KV head hk: q, k, v ~ N(0, 1); a random unit vector u[hk]; key rows at the
sink positions and at 2% random positions get +4*u[hk]; every query row of a
q head h gets +1.5*u[h // n_rep].  DiT configs add per-frame locality: a unit
vector w[hk, f] per latent frame f is added to that frame's keys and (x1.0) to
its queries.  Softmax scale 1/sqrt(D).
"""
from dataclasses import dataclass, field
from typing import Optional, Tuple

import torch


@dataclass(frozen=True)
class Workload:
    name: str
    B: int
    Hq: int
    Hk: int
    S: int
    D: int
    dtype: torch.dtype
    causal: bool
    keep: float                      # target fraction of selectable keys
    group_k_block: int
    q_pooling_size: int = 64
    k_local_size: int = 16
    chunk_size: int = 32768
    sinks: str = "first64"           # "first64" | "text_last"
    frames: Optional[Tuple[int, int]] = None   # (num frames, tokens per frame)
    text_tokens: int = 0


# The five configurations of the benchmark plan (A is the CPU-reference case).
WORKLOADS = {
    "A": Workload("A-cpu-ref", 1, 4, 4, 4096, 64, torch.float32, False, 0.10, 16),
    "B": Workload("B-qwen2.5vl-32k", 1, 28, 4, 32768, 128, torch.bfloat16, True, 0.10, 16),
    "C": Workload("C-qwen2.5vl-128k", 1, 28, 4, 131072, 128, torch.bfloat16, True, 0.05, 16),
    "D": Workload("D-wan2.1-32760", 1, 12, 12, 32760, 128, torch.bfloat16, False, 0.15, 8192,
                  frames=(21, 1560)),
    "E": Workload("E-hunyuan-119056", 1, 24, 24, 119056, 128, torch.bfloat16, False, 0.10, 8192,
                  sinks="text_last", frames=(33, 3600), text_tokens=256),
}


def make_inputs(B, Hq, Hk, S, D, dtype=torch.bfloat16, seed=0, sinks="first64", frames=None,
                text_tokens=0, device="cpu"):
    """q (B,Hq,S,D), k, v (B,Hk,S,D) in `dtype` on `device` (generated on CPU)."""
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn(B, Hq, S, D, generator=g)
    k = torch.randn(B, Hk, S, D, generator=g)
    v = torch.randn(B, Hk, S, D, generator=g)
    rep = Hq // Hk
    u = torch.randn(Hk, D, generator=g)
    u = u / u.norm(dim=-1, keepdim=True)
    if sinks == "first64":
        sink_idx = torch.arange(min(64, S))
    elif sinks == "text_last":
        sink_idx = torch.arange(max(S - text_tokens, 0), S)
    else:
        raise ValueError(f"unknown sinks mode {sinks!r}")
    n_rand = int(round(0.02 * S))
    for hk in range(Hk):
        rnd = torch.randperm(S, generator=g)[:n_rand]
        idx = torch.unique(torch.cat([sink_idx, rnd]))
        k[:, hk, idx] += 4.0 * u[hk]
    q += 1.5 * u.repeat_interleave(rep, dim=0)[None, :, None, :]
    if frames is not None:
        nf, tpf = frames
        w = torch.randn(Hk, nf, D, generator=g)
        w = w / w.norm(dim=-1, keepdim=True)
        for f in range(nf):
            lo, hi = f * tpf, min((f + 1) * tpf, S)
            if lo >= hi:
                break
            k[:, :, lo:hi] += w[None, :, f, None, :]
            q[:, :, lo:hi] += w.repeat_interleave(rep, dim=0)[None, :, f, None, :]
    return (q.to(dtype).to(device), k.to(dtype).to(device), v.to(dtype).to(device))


def workload_inputs(wl: Workload, seed=0, device="cpu", S=None):
    """Inputs of a named workload; `S` overrides the length (parity-sized cases)."""
    S = S or wl.S
    frames = wl.frames
    return make_inputs(wl.B, wl.Hq, wl.Hk, S, wl.D, wl.dtype, seed, wl.sinks, frames,
                       wl.text_tokens, device)
