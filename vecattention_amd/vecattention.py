"""VecAttention prefill on MI355X: the drop-in for
``spattn.src.VecAttention.VecAttention_prefill`` (spattn/src/VecAttention.py:10-123).

Same signature, defaults, argument meaning, assertions and return layout as the
reference.  The work runs in libvecattn.so (HIP kernels for gfx950): query
pooling, TilingSelect selection and vector-sparse attention, chunk by chunk on
the current stream with no host synchronisation.
"""
import math
import warnings
from typing import Union

import torch

from . import _native as nat

# BLOCK_SIZE_Q of the reference's selection launch.  The reference reads it
# from pickled Triton configs keyed (qps, BK, G, D, causal)
# (spattn/src/kernels/vecattention_kernels.py:24-56,101-102); every causal key
# in the shipped vlm/dit caches maps to 64, and so does the fallback (:51-53).
# It matters only for the causal first-row tile rule, which is tied to the
# program tiling.  Non-causal entries (128 for G=16 in the dit cache) have no
# effect on results.
REFERENCE_BLOCK_SIZE_Q = 64


def reference_block_size_q(q_pooling_size, k_local_size, group_k_block, head_dim, causal):
    """BLOCK_SIZE_Q the reference would launch with for this configuration."""
    return REFERENCE_BLOCK_SIZE_Q


def threshold_to_gap(threshold, batch_size, num_heads, device):
    """MinP threshold -> minS gap, as spattn/src/VecAttention.py:48-52.

    Returns (gap_scalar: float, gaps: fp32 device tensor of B*H or None).
    A float threshold gives gap = -ln(threshold + 1e-9) in double precision,
    consumed as fp32 by the kernel (the reference passes it as a Triton
    constexpr).  A tensor threshold gives -log(threshold + 1e-9): the sum in
    the tensor's dtype, as the reference's expression, and the logarithm of
    that sum in fp64, rounded once to fp32.  The reference evaluates the
    logarithm in fp32 on its GPU; an fp32 logarithm is at best this correctly
    rounded value, and the device's fp32 logarithm here is not always it (up
    to two units in the last place off), so the gap is not taken from it.  A
    (H,) tensor is shared by every batch row and a (B, H) tensor is used as is.
    """
    if isinstance(threshold, torch.Tensor):
        gap = -torch.log((threshold + 1e-9).to(torch.float64))
        gap = gap.to(device=device, dtype=torch.float32)
        if gap.dim() == 0:
            gap = gap.expand(batch_size, num_heads)
        elif gap.dim() == 1:
            if gap.numel() != num_heads:
                raise AssertionError(f"per-head threshold has {gap.numel()} entries for {num_heads} heads")
            gap = gap.unsqueeze(0).expand(batch_size, num_heads)
        elif gap.dim() == 2:
            if tuple(gap.shape) != (batch_size, num_heads):
                raise AssertionError(f"threshold shape {tuple(gap.shape)} != (B, H) = {(batch_size, num_heads)}")
        else:
            raise AssertionError(f"threshold must be a float, (H,) or (B, H) tensor; got {tuple(gap.shape)}")
        return 0.0, gap.contiguous()
    # Same expression (and the same TypeError for None) as the reference.
    gap = -math.log(threshold + 1e-9, math.e)
    return float(gap), None


def _check_inputs(q, k, v):
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise AssertionError("query/key/value must be (batch, heads, seq, head_dim)")
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise RuntimeError("VecAttention_prefill runs on the GPU: query/key/value must be device tensors")
    if not (q.device == k.device == v.device):
        raise RuntimeError("query/key/value must be on one device")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("query/key/value must share a dtype")
    if k.shape != v.shape:
        raise AssertionError(f"key {tuple(k.shape)} and value {tuple(v.shape)} shapes differ")
    B, Hq, S, D = q.shape
    if k.shape[0] != B or k.shape[3] != D:
        raise AssertionError("key batch/head_dim differ from query")
    if Hq % k.shape[1]:
        raise AssertionError(f"query heads {Hq} not a multiple of key heads {k.shape[1]}")


_warned_paths = set()


def _warn_slow_path(flags, dtype, head_dim, q_pooling_size, k_local_size):
    """Warn once per configuration when va_prefill leaves the MFMA kernels."""
    reasons = []
    if flags & nat.VA_KERNELS_SELECT_EXACT:
        reasons.append("the selection runs on the exact fp64 kernel (the MFMA selection takes "
                       "bf16/fp16, head_dim 64 or 128, k_local_size 16 to 256 and 16-byte "
                       "aligned keys)")
    if flags & nat.VA_KERNELS_ATTN_ROW:
        reasons.append("the attention runs on the per-row kernel (the MFMA attention takes "
                       "bf16/fp16, head_dim and q_pooling_size 64 or 128, aligned tensors and "
                       "key/value row strides under 16 KiB)")
    key = (flags, str(dtype), head_dim, q_pooling_size, k_local_size)
    if reasons and key not in _warned_paths:
        _warned_paths.add(key)
        warnings.warn("VecAttention_prefill: " + "; ".join(reasons) +
                      "; expect several times the time of the MFMA path", RuntimeWarning,
                      stacklevel=3)


def _feature_contiguous(t):
    return t if t.stride(-1) == 1 else t.contiguous()


def VecAttention_prefill(
    query_states: torch.Tensor,
    key_states: torch.Tensor,
    value_states: torch.Tensor,
    threshold: Union[float, torch.Tensor] = None,
    q_pooling_size: int = 128,
    k_local_size: int = 128,
    group_k_block: int = 1,
    causal: bool = True,
    chunk_size: int = 16 * 1024,
):
    """Vectorized sparse attention prefill (VecAttention).

    Args (as spattn/src/VecAttention.py:10-42):
        query_states: (batch, num_heads, seq_len, head_dim); any outer strides.
        key_states:   (batch, num_kv_heads, seq_len, head_dim).  num_kv_heads
            may divide num_heads (GQA is handled natively, no repeat_kv).
        value_states: (batch, num_kv_heads, seq_len, head_dim)
        threshold: MinP threshold; float, or a per-head (H,) / (B, H) tensor.
        q_pooling_size: query block size (64 or 128).
        k_local_size: key tile size of the selection (power of two, 16..256).
        group_k_block: key tiles sharing one running maximum.
        causal: causal masking (then key and query lengths must match).
        chunk_size: query chunk size, a multiple of q_pooling_size.

    Returns:
        attn_output: (batch, num_heads, seq_len, head_dim), dtype of query.
    """
    assert chunk_size % q_pooling_size == 0, "chunk_size must be a multiple of q_pooling_size"
    assert q_pooling_size in [64, 128], "q_pooling_size must be 64 or 128"
    gap, gaps = threshold_to_gap(threshold, query_states.shape[0], query_states.shape[1],
                                 query_states.device)
    _check_inputs(query_states, key_states, value_states)
    if causal:
        assert q_pooling_size % k_local_size == 0, "causal requires q_pooling_size % k_local_size == 0"
        if key_states.shape[2] != query_states.shape[2]:
            raise NotImplementedError("causal VecAttention_prefill needs equal query and key lengths")

    q = _feature_contiguous(query_states)
    k = _feature_contiguous(key_states)
    v = _feature_contiguous(value_states)
    B, Hq, S, D = q.shape
    Hk, Sk = k.shape[1], k.shape[2]
    dt = nat.dtype_code(q)
    L = nat.lib()
    attn_output = torch.empty(B, Hq, S, D, dtype=q.dtype, device=q.device)
    flags = L.va_prefill_kernels(
        dt, nat.ptr(q), q.stride(0), q.stride(1), q.stride(2), nat.ptr(k), k.stride(0),
        k.stride(1), k.stride(2), nat.ptr(v), v.stride(0), v.stride(1), v.stride(2),
        nat.ptr(attn_output), attn_output.stride(0), attn_output.stride(1), attn_output.stride(2),
        Hq, Hk, Sk, D, q_pooling_size, k_local_size, group_k_block)
    if flags < 0:
        nat.check("va_prefill_kernels", flags)
    _warn_slow_path(flags, q.dtype, D, q_pooling_size, k_local_size)
    bsq = reference_block_size_q(q_pooling_size, k_local_size, group_k_block, D, causal)
    ws_bytes = L.va_prefill_workspace_size(dt, B, Hq, S, Sk, D, q_pooling_size, int(causal),
                                           chunk_size, bsq)
    if ws_bytes < 0:
        raise AssertionError("invalid VecAttention_prefill sizes")
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        rc = L.va_prefill(
            dt, nat.ptr(q), q.stride(0), q.stride(1), q.stride(2),
            nat.ptr(k), k.stride(0), k.stride(1), k.stride(2),
            nat.ptr(v), v.stride(0), v.stride(1), v.stride(2),
            nat.ptr(attn_output), attn_output.stride(0), attn_output.stride(1), attn_output.stride(2),
            B, Hq, Hk, S, Sk, D, gap, nat.ptr(gaps), q_pooling_size, k_local_size, group_k_block,
            int(causal), chunk_size, bsq, nat.ptr(workspace), ws_bytes, nat.stream_ptr(q.device))
    nat.check("va_prefill", rc)
    return attn_output
