"""Decode attention (one new token per sequence) on the MI355X kernels.

Mirrors ``flashinfer.single_decode_with_kv_cache`` (flashinfer-python 0.5.2,
git 4aed50cf, the reference's pin at uv.lock:1407-1409) as the reference's
patched forwards call it in their decode branch
(spattn/src/models/load_qwen2p5_vl.py:61-66 with kv_layout "NHD",
spattn/src/models/load_llama.py:183-188 with "HND"): for each query head h,
softmax(q[h] . K_g^T * sm_scale) V_g over every cached key of kv head
g = h // (num_qo_heads // num_kv_heads), no mask, output in q's dtype.

The reference expands K/V with repeat_kv and copies them to NHD/HND before the
call; here the kv heads may be shared (GQA) and any strides with contiguous
features are read in place.
"""
import math

import torch

from . import _native as nat


def single_decode_with_kv_cache(q, k, v, kv_layout="NHD", pos_encoding_mode="NONE",
                                use_tensor_cores=False, q_scale=None, k_scale=None, v_scale=None,
                                window_left=-1, logits_soft_cap=None, sm_scale=None,
                                rope_scale=None, rope_theta=None, return_lse=False):
    """q: (num_qo_heads, head_dim); k, v: (kv_len, num_kv_heads, head_dim) for
    "NHD" or (num_kv_heads, kv_len, head_dim) for "HND".  Returns
    (num_qo_heads, head_dim) in q's dtype.

    Supported: the arguments the reference passes (q, k, v, kv_layout) and
    sm_scale (default 1/sqrt(head_dim)); `use_tensor_cores` picks an
    implementation in flashinfer and is ignored.  RoPE, sliding windows, soft
    caps, fp8 scales and the LSE output raise NotImplementedError.
    """
    if pos_encoding_mode != "NONE" or rope_scale is not None or rope_theta is not None:
        raise NotImplementedError("decode: positional encoding inside attention is not supported")
    if window_left != -1 or logits_soft_cap is not None:
        raise NotImplementedError("decode: sliding windows and logit soft caps are not supported")
    if q_scale is not None or k_scale is not None or v_scale is not None:
        raise NotImplementedError("decode: fp8 scales are not supported")
    if return_lse:
        raise NotImplementedError("decode: the log-sum-exp output is not supported")
    if q.dim() != 2 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q must be (num_qo_heads, head_dim) and k, v 3-dimensional")
    if k.shape != v.shape:
        raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} differ")
    if kv_layout == "NHD":
        L, Hk, D = k.shape
        kh, kn, vh, vn = k.stride(1), k.stride(0), v.stride(1), v.stride(0)
    elif kv_layout == "HND":
        Hk, L, D = k.shape
        kh, kn, vh, vn = k.stride(0), k.stride(1), v.stride(0), v.stride(1)
    else:
        raise KeyError(f"Invalid kv_layout {kv_layout}")
    Hq = q.shape[0]
    if q.shape[1] != D:
        raise ValueError(f"head_dim of q ({q.shape[1]}) and k ({D}) differ")
    if Hq % Hk:
        raise ValueError(f"num_qo_heads {Hq} is not a multiple of num_kv_heads {Hk}")
    if q.dtype != k.dtype or v.dtype != k.dtype:
        raise ValueError("q, k and v must share a dtype")
    if not q.is_cuda:
        raise RuntimeError("decode attention runs on the GPU")
    if q.stride(1) != 1:
        q = q.contiguous()
    if k.stride(2) != 1 or v.stride(2) != 1:
        raise ValueError("k and v need contiguous head_dim")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    out = torch.empty(Hq, D, dtype=q.dtype, device=q.device)
    L_ = nat.lib()
    ws_bytes = int(L_.va_decode_workspace_size(Hq, Hk, L, D))
    work = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=q.device)
    with torch.cuda.device(q.device):
        rc = L_.va_decode_attn(nat.dtype_code(q), nat.ptr(q), q.stride(0), nat.ptr(k), kh, kn,
                               nat.ptr(v), vh, vn, nat.ptr(out), out.stride(0), Hq, Hk, L, D,
                               float(sm_scale), nat.VA_ATTN_AUTO, nat.ptr(work), work.numel(),
                               nat.stream_ptr(q.device))
    nat.check("va_decode_attn", rc)
    return out


__all__ = ["single_decode_with_kv_cache"]
