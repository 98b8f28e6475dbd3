"""CPU oracle of the VecAttention prefill path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker (or, for the baseline, the thing timed on
the host).  The product path (vecattention_amd/) never imports it.

Pieces and the reference lines they restate:
  pool / select       oracle/vecattn_oracle.c (pooling: spattn/src/utils.py:
                      8-83,340-360; selection: spattn/src/kernels/
                      vecattention_kernels.py:59-181,206-345)
  local_blocks        spattn/src/VecAttention.py:63-92 (also
                      spattn/threshold/model_tuner.py:144-176)
  attention           spattn/threshold/model_tuner.py:193-216 (the dense-mask
                      statement of sparse_attn_func: local blocks of 64 keys
                      clipped to S_k, union selected columns, causal mask,
                      softmax scale 1/sqrt(D)); an empty key set gives 0
  prefill             spattn/src/VecAttention.py:43-123 (gap, chunk loop)
  decode              flashinfer.single_decode_with_kv_cache as called at
                      spattn/src/models/load_qwen2p5_vl.py:61-66 (NHD) and
                      spattn/src/models/load_llama.py:183-188 (HND): one
                      query row per head, softmax over every cached key
  seg_pr_perhead      spattn/threshold/model_tuner.py:118-226 (the tuner's
                      recall / sparsity evaluation: dense softmax per head,
                      boolean mask of local blocks and selected columns)

Pinning (tests/test_oracle.py): closed forms for pooling and gap (the tensor
branch against torch's evaluation of the reference expression); hand-derived
known answers for the selection rule (prefix maximum updated before the
compare, group restarts, causal first-row tile rule, key tail); a brute force
written from the reference kernel's program structure (grid of BLOCK_SIZE_Q
rows x groups, per-program tile range, running maximum per row, truncating
causal division) on small-integer inputs whose scores are exact, over random
tile sizes, groups, chunk origins, BLOCK_SIZE_Q and key tails; invariants
(large gap selects every selectable key; larger gap selects a superset;
chunk-size invariance; single-group equivalence); attention against torch's
dense SDPA in float64 where the sparse set is all keys.
"""
import ctypes
import math
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
SPATTN_BLOCK_SIZE_K = 64  # spattn/src/VecAttention.py:45-46

ORC_F32, ORC_BF16, ORC_F16 = 0, 1, 2
_lib = None


def build():
    """Compile the C restatement (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        h = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        I = ctypes.c_int64
        h.orc_pool.restype = ctypes.c_int
        h.orc_pool.argtypes = [P, I, I, I, I, I, ctypes.c_int, P, P]
        h.orc_select.restype = ctypes.c_int
        h.orc_select.argtypes = [P, I, P, I, I, I, I, I, I, I, I, ctypes.c_int, ctypes.c_int, I, I,
                                 I, I, I, P, P, P, P, P]
        h.orc_dot.restype = ctypes.c_float
        h.orc_dot.argtypes = [P, P, I]
        h.orc_round.restype = ctypes.c_float
        h.orc_round.argtypes = [ctypes.c_float, ctypes.c_int]
        _lib = h
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def dtype_code(name):
    return {"float32": ORC_F32, "bfloat16": ORC_BF16, "float16": ORC_F16}[name]


def as_f32(x):
    """torch tensor or array -> contiguous float32 numpy array (exact for bf16/fp16).
    A torch tensor can only come from a caller that imported torch, so torch is
    looked up, not imported (numpy-only callers stay free of it)."""
    torch = sys.modules.get("torch")
    if torch is not None and isinstance(x, torch.Tensor):
        return np.ascontiguousarray(x.detach().float().cpu().numpy())
    return np.ascontiguousarray(np.asarray(x, dtype=np.float32))


def pool(q, qps, dtype):
    """(pooled, scaled) for q (B,H,S,D) float32 values of element type `dtype`."""
    q = as_f32(q)
    B, H, S, D = q.shape
    nqb = math.ceil(S / qps)
    pooled = np.empty((B, H, nqb, D), np.float32)
    scaled = np.empty((B, H, nqb, D), np.float32)
    rc = lib().orc_pool(_p(q), B, H, S, D, qps, dtype_code(dtype), _p(pooled), _p(scaled))
    assert rc == 0, rc
    return pooled, scaled


def gap_from_threshold(threshold, B, H):
    """fp32 gap per (b, h) as spattn/src/VecAttention.py:48-52.

    Float branch: -ln(th + 1e-9) in double, then fp32 (the reference passes a
    Python float).  Tensor branch, -log(threshold + 1e-9) on an fp32 tensor:
    the fp32 sum, then the correctly rounded fp32 value of its logarithm (fp64
    log, one rounding).  The reference evaluates the logarithm in fp32 on its
    GPU, whose result is within one unit in the last place of this value; the
    last bit of a per-head gap is therefore not pinned by the reference.
    (numpy's float32 log is not correctly rounded: it is off by one unit for
    about one threshold in six, so it is not used.)
    """
    if np.ndim(threshold) == 0:
        return np.full(B * H, np.float32(-math.log(float(threshold) + 1e-9)), np.float32)
    t = np.asarray(threshold, np.float32)
    s = (t + np.float32(1e-9)).astype(np.float32)
    g = (-np.log(s.astype(np.float64))).astype(np.float32)
    return np.ascontiguousarray(np.broadcast_to(g, (B, H)).reshape(-1))


def row_capacity(J, qps, Sk, causal, wo_init):
    smin = (qps if causal else min(qps, Sk)) if wo_init else 0
    if causal:
        return max(0, min(Sk, J * qps) - smin)
    return Sk - smin


def select(qs, k, J0, nc, gaps, qps, bk, group, causal, wo_init, bsq, rows=None):
    """Selected key lists for rows [J0, J0+nc) of every (b, h).

    qs: scaled pooled queries (B,Hq,nqb_total,D); k: (B,Hk,Sk,D); gaps: fp32 B*Hq.
    rows: optional (jr_begin, jr_end) subset of the chunk [J0, J0+nc) to compute
    (the chunk start still fixes the causal program tiling); others count 0.
    Returns (counts (B,Hq,nc) int32, lists: nested list [b][h][jr] of int32 arrays).
    """
    qs = as_f32(qs)
    k = as_f32(k)
    B, Hq, nqb_total, D = qs.shape
    Hk, Sk = k.shape[1], k.shape[2]
    caps = np.array([[row_capacity(J0 + jr, qps, Sk, causal, wo_init) for jr in range(nc)]] * (B * Hq),
                    np.int64).reshape(-1)
    base = np.zeros_like(caps)
    base[1:] = np.cumsum(caps)[:-1]
    idx = np.zeros(max(int(caps.sum()), 1), np.int32)
    counts = np.zeros(B * Hq * nc, np.int32)
    gaps = np.ascontiguousarray(gaps, np.float32)
    jb, je = rows if rows is not None else (0, nc)
    rc = lib().orc_select(_p(qs), nqb_total, _p(k), B, Hq, Hk, Sk, D, qps, bk, group, int(causal),
                          int(wo_init), J0, nc, jb, je, bsq, _p(gaps), _p(counts), _p(idx), _p(base),
                          _p(caps))
    assert rc == 0, rc
    lists = [[[idx[base[(b * Hq + h) * nc + jr]: base[(b * Hq + h) * nc + jr] + counts[(b * Hq + h) * nc + jr]].copy()
               for jr in range(nc)] for h in range(Hq)] for b in range(B)]
    return counts.reshape(B, Hq, nc), lists


def local_blocks(B, H, S, qps, causal):
    """(blk_count (B,H,nqb) int32, blk_idx (B,H,nqb,2n|1) int32), as
    spattn/src/VecAttention.py:63-92."""
    nqb = math.ceil(S / qps)
    if causal:
        n = qps // SPATTN_BLOCK_SIZE_K
        cnt = np.full((B, H, nqb), 2 * n, np.int32)
        cnt[..., 0] = math.ceil(min(S, qps) / SPATTN_BLOCK_SIZE_K)
        if S > qps and S % qps != 0:
            cnt[..., -1] = n + math.ceil((S - (S // qps) * qps) / SPATTN_BLOCK_SIZE_K)
        idx = np.zeros((B, H, nqb, 2 * n), np.int32)
        offs = np.arange(n, dtype=np.int32) * SPATTN_BLOCK_SIZE_K
        idx[..., :n] = offs
        idx[..., n:] = (np.arange(nqb, dtype=np.int32) * qps)[:, None] + offs
    else:
        cnt = np.zeros((B, H, nqb), np.int32)
        idx = np.zeros((B, H, nqb, 1), np.int32)
    return cnt, idx


def key_set(J, blk_count, blk_idx, cols, Sk):
    """Sorted key positions of q-block J: blocks of 64 clipped to [0, Sk) ∪ columns."""
    parts = [np.arange(int(o), min(int(o) + SPATTN_BLOCK_SIZE_K, Sk)) for o in blk_idx[:blk_count]]
    parts.append(np.asarray(cols, np.int64))
    return np.unique(np.concatenate(parts).astype(np.int64)) if parts else np.zeros(0, np.int64)


def attention(q, k, v, qps, causal, blk_count, blk_idx, lists, J0=0, nc=None, acc=np.float64):
    """Masked softmax attention for q-blocks [J0, J0+nc): out rows (B,Hq,rows,D) in `acc`.

    q (B,Hq,Sq,D), k/v (B,Hk,Sk,D) as float arrays; lists[b][h][jr] selected columns.
    Causal alignment is bottom-right (row i of the query sequence sees keys
    <= i + Sk - Sq), as for each chunk of the reference.
    """
    q = as_f32(q).astype(acc, copy=False)
    k = as_f32(k).astype(acc, copy=False)
    v = as_f32(v).astype(acc, copy=False)
    B, Hq, Sq, D = q.shape
    Hk, Sk = k.shape[1], k.shape[2]
    rep = Hq // Hk
    nqb = math.ceil(Sq / qps)
    nc = nqb - J0 if nc is None else nc
    r0, r1 = J0 * qps, min(Sq, (J0 + nc) * qps)
    out = np.zeros((B, Hq, r1 - r0, D), acc)
    scale = 1.0 / math.sqrt(D)
    for b in range(B):
        for h in range(Hq):
            kh, vh = k[b, h // rep], v[b, h // rep]
            for jr in range(nc):
                J = J0 + jr
                keys = key_set(J, blk_count[b, h, J], blk_idx[b, h, J], lists[b][h][jr], Sk)
                a, e = J * qps, min(Sq, (J + 1) * qps)
                if keys.size == 0:
                    continue
                s = (q[b, h, a:e] @ kh[keys].T) * scale
                if causal:
                    pos = np.arange(a, e)[:, None] + (Sk - Sq)
                    s = np.where(keys[None, :] <= pos, s, -np.inf)
                m = s.max(axis=1, keepdims=True)
                m = np.where(np.isfinite(m), m, 0.0)
                p = np.exp(s - m)
                l = p.sum(axis=1, keepdims=True)
                o = (p @ vh[keys]) / np.where(l > 0, l, 1.0)
                out[b, h, a - r0:e - r0] = np.where(l > 0, o, 0.0)
    return out


def prefill(q, k, v, threshold, q_pooling_size=128, k_local_size=128, group_k_block=1,
            causal=True, chunk_size=16 * 1024, bsq=64, dtype="bfloat16", acc=np.float64,
            gaps=None):
    """Whole-path oracle: returns (out (B,Hq,S,D) in `acc`, per-chunk (counts, lists)).
    `gaps` (fp32, B*Hq) replaces the gaps derived from `threshold` when given."""
    q, k, v = as_f32(q), as_f32(k), as_f32(v)
    B, Hq, S, D = q.shape
    Sk = k.shape[2]
    if gaps is None:
        gaps = gap_from_threshold(threshold, B, Hq)
    gaps = np.ascontiguousarray(np.asarray(gaps, np.float32).reshape(-1))
    _, qs = pool(q, q_pooling_size, dtype)
    blk_count, blk_idx = local_blocks(B, Hq, S, q_pooling_size, causal)
    out = np.zeros((B, Hq, S, D), acc)
    chunks = []
    for i in range(0, S, chunk_size):
        J0 = i // q_pooling_size
        nc = math.ceil(min(chunk_size, S - i) / q_pooling_size)
        counts, lists = select(qs, k, J0, nc, gaps, q_pooling_size, k_local_size, group_k_block,
                               causal, causal, bsq)
        chunks.append((counts, lists))
        kc = k[:, :, :i + chunk_size] if causal else k
        vc = v[:, :, :i + chunk_size] if causal else v
        qc = q[:, :, :min(S, i + chunk_size)]
        o = attention(qc, kc, vc, q_pooling_size, causal, blk_count, blk_idx, lists, J0=J0, nc=nc,
                      acc=acc)
        out[:, :, i:i + o.shape[2]] = o
    return out, chunks


def seg_pr_perhead(q, k, block_size_q, block_size_k=16, group_size_k=16, threshold=None,
                   chunk_size=8 * 1024, causal=False, dtype="float32", bsq=64):
    """(recall (H,), sparsity (H,)) in float64, restating model_tuner.py:118-226.

    q (B,H,S,D), k (B,Hk,Sk,D) float values of element type `dtype`;
    threshold: per-head (H,) values.  gap = -log(th + 1e-50) (model_tuner.py:150;
    1e-50 is 0 in fp32): the fp32 sum, its log in fp64, rounded once to fp32.
    Per chunk: pooled rows, selection with wo_initial=causal (:183-187), then
    per (b, h) the dense
    softmax with the top-left causal mask (:139-143,193-199), the boolean mask
    of the blocks [off, min(off+64, Sk)) and the selected columns (:201-216),
    recall = masked row sums (:216,220) and sparsity += (1 - mean(mask count /
    visible count)) * chunk_len (:218-219), divided by B and S (:222-223).
    """
    q = as_f32(q).astype(np.float64)
    k = as_f32(k).astype(np.float64)
    B, H, S, D = q.shape
    Hk, Sk = k.shape[1], k.shape[2]
    rep = H // Hk
    th = np.asarray(threshold, np.float32)
    with np.errstate(divide="ignore"):
        summed = (th + np.float32(1e-50)).astype(np.float32)
        gap = (-np.log(summed.astype(np.float64))).astype(np.float32)
    gaps = np.ascontiguousarray(np.broadcast_to(gap, (B, H)).reshape(-1), np.float32)
    _, qs = pool(q.astype(np.float32), block_size_q, dtype)
    blk_count, blk_idx = local_blocks(B, H, S, block_size_q, causal)
    recalls = np.zeros((B, H, S))
    sparsity = np.zeros(H)
    scale = 1.0 / math.sqrt(D)
    for c0 in range(0, S, chunk_size):
        rows = min(chunk_size, S - c0)
        J0, nc = c0 // block_size_q, math.ceil(rows / block_size_q)
        _, lists = select(qs, k.astype(np.float32), J0, nc, gaps, block_size_q, block_size_k,
                          group_size_k, causal, causal, bsq)
        pos = np.arange(c0, c0 + rows)
        allowed = (np.arange(Sk)[None, :] <= pos[:, None]) if causal else np.ones((rows, Sk), bool)
        for b in range(B):
            for h in range(H):
                s = (q[b, h, c0:c0 + rows] @ k[b, h // rep].T) * scale
                s = np.where(allowed, s, -np.inf)
                p = np.exp(s - s.max(axis=1, keepdims=True))
                p /= p.sum(axis=1, keepdims=True)
                mask = np.zeros((rows, Sk), bool)
                for jr in range(nc):
                    J = J0 + jr
                    r0, r1 = jr * block_size_q, min((jr + 1) * block_size_q, rows)
                    for off in blk_idx[b, h, J, :blk_count[b, h, J]]:
                        mask[r0:r1, int(off):min(int(off) + SPATTN_BLOCK_SIZE_K, Sk)] = True
                    mask[r0:r1, lists[b][h][jr]] = True
                sparsity[h] += (1.0 - (mask.sum(axis=1) / allowed.sum(axis=1)).mean()) * rows
                recalls[b, h, c0:c0 + rows] = (p * mask).sum(axis=1)
    sparsity /= B
    sparsity /= S
    return recalls.sum(axis=(0, 2)) / (B * S), sparsity


def decode(q, k, v, kv_layout="NHD", sm_scale=None):
    """(Hq, D) float64: out[h] = softmax(q[h] . K_g^T * sm_scale) V_g with
    g = h // (Hq / Hk), every key visible (flashinfer-python 0.5.2
    single_decode_with_kv_cache semantics: default sm_scale 1/sqrt(D), GQA
    by integer division of the head index)."""
    q = as_f32(q).astype(np.float64)
    k = as_f32(k).astype(np.float64)
    v = as_f32(v).astype(np.float64)
    if kv_layout == "NHD":
        k, v = k.transpose(1, 0, 2), v.transpose(1, 0, 2)
    Hq, D = q.shape
    Hk = k.shape[0]
    scale = 1.0 / math.sqrt(D) if sm_scale is None else float(sm_scale)
    out = np.zeros((Hq, D))
    for h in range(Hq):
        g = h // (Hq // Hk)
        s = (k[g] @ q[h]) * scale
        p = np.exp(s - s.max())
        out[h] = (p @ v[g]) / p.sum()
    return out
