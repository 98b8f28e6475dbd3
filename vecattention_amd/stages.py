"""Stage-level entry points of the prefill path, and the reference's
second-level API used by its threshold tuner.

* ``average_vector``                 spattn/src/utils.py:340-360
* ``fuse_qk_softmax_minp_wo_causal`` spattn/src/kernels/vecattention_kernels.py:59-181
* ``pool_scaled`` / ``select_rows`` / ``sparse_attention``: the three stages of
  VecAttention_prefill (spattn/src/VecAttention.py:94-121) on the packed
  "index layout" of include/vecattn.h, for callers that drive the stages
  themselves (tests, benchmarks, tuners).
"""
import math

import torch

from . import _native as nat
from .vecattention import reference_block_size_q, threshold_to_gap


def _stream(t):
    return nat.stream_ptr(t.device)


def pool_scaled(q, q_pooling_size, want_pooled=False):
    """Pooled queries scaled by fp32(1/sqrt(D)) and rounded to q's dtype.

    Returns (scaled, pooled-or-None), both contiguous (B, H, ceil(S/qps), D).
    """
    if q.stride(-1) != 1:
        q = q.contiguous()
    B, H, S, D = q.shape
    nqb = math.ceil(S / q_pooling_size)
    scaled = torch.empty(B, H, nqb, D, dtype=q.dtype, device=q.device)
    pooled = torch.empty_like(scaled) if want_pooled else None
    with torch.cuda.device(q.device):
        rc = nat.lib().va_pool(nat.dtype_code(q), nat.ptr(q), B, H, S, D, q.stride(0), q.stride(1),
                               q.stride(2), q_pooling_size, nat.ptr(pooled), nat.ptr(scaled),
                               _stream(q))
    nat.check("va_pool", rc)
    return scaled, pooled


def average_vector(q, block_size, use_triton=True):
    """Block means of q over `block_size` rows (fp32 accumulation, the last
    block divided by its real row count), returned in q's dtype.
    Mirrors spattn/src/utils.py:340-360; `use_triton` is accepted and ignored.
    """
    if q.stride(-1) != 1:
        q = q.contiguous()
    B, H, S, D = q.shape
    nqb = math.ceil(S / block_size)
    pooled = torch.empty(B, H, nqb, D, dtype=q.dtype, device=q.device)
    with torch.cuda.device(q.device):
        rc = nat.lib().va_pool(nat.dtype_code(q), nat.ptr(q), B, H, S, D, q.stride(0), q.stride(1),
                               q.stride(2), block_size, nat.ptr(pooled), None, _stream(q))
    nat.check("va_pool", rc)
    return pooled


def index_capacity(B, Hq, Sk, qps, causal, wo_init, J0, nc, dense_stride=0):
    return int(nat.lib().va_select_index_capacity(B, Hq, Sk, qps, int(causal), int(wo_init), J0,
                                                  nc, dense_stride))


def row_offset(Sk, qps, causal, wo_init, J0, nc, bh, jr, dense_stride=0):
    return int(nat.lib().va_select_row_offset(Sk, qps, int(causal), int(wo_init), J0, nc,
                                              dense_stride, bh, jr))


def select_rows(qs_chunk, k, J0, gap, gaps, causal, q_pooling_size, k_local_size, group_k_block,
                wo_init, bsq=None, dense_stride=0, indices=None, counts=None,
                kernel=nat.VA_SEL_AUTO):
    """TilingSelect for the pooled rows of one chunk.

    qs_chunk: (B, Hq, nc, D) scaled pooled rows J0 .. J0+nc-1 (any strides,
    features contiguous); k: (B, Hk, Sk, D).  `kernel`: VA_SEL_AUTO (a certified
    MFMA kernel when supported), VA_SEL_EXACT, VA_SEL_MFMA or VA_SEL_WAVE.
    Returns (counts (B, Hq, nc) int32, indices int32 in the index layout).
    """
    if qs_chunk.stride(-1) != 1:
        qs_chunk = qs_chunk.contiguous()
    if k.stride(-1) != 1:
        k = k.contiguous()
    B, Hq, nc, D = qs_chunk.shape
    Hk, Sk = k.shape[1], k.shape[2]
    if bsq is None:
        bsq = reference_block_size_q(q_pooling_size, k_local_size, group_k_block, D, causal)
    cap = index_capacity(B, Hq, Sk, q_pooling_size, causal, wo_init, J0, nc, dense_stride)
    if counts is None:
        counts = torch.empty(B, Hq, nc, dtype=torch.int32, device=k.device)
    if indices is None:
        indices = torch.empty(max(cap, 1), dtype=torch.int32, device=k.device)
    nscr = int(nat.lib().va_select_scratch_floats(B, Hk))
    scratch = torch.empty(max(nscr, 1), dtype=torch.float32, device=k.device)
    with torch.cuda.device(k.device):
        rc = nat.lib().va_select(
            nat.dtype_code(k), nat.ptr(qs_chunk), qs_chunk.stride(0), qs_chunk.stride(1),
            qs_chunk.stride(2), nat.ptr(k), k.stride(0), k.stride(1), k.stride(2), B, Hq, Hk, Sk, D,
            q_pooling_size, k_local_size, group_k_block, int(causal), int(wo_init), J0, nc, bsq,
            float(gap), nat.ptr(gaps), dense_stride, nat.ptr(counts), nat.ptr(indices), int(kernel),
            nat.ptr(scratch), nscr, _stream(k))
    nat.check("va_select", rc)
    return counts, indices


def segment_keys(Sk, k_local_size, group_k_block, exact=False):
    """Segment length of the split selection va_prefill uses (0: not split):
    the wave/MFMA kernels' for bf16/fp16, the exact kernel's (`exact`) for
    fp32 inputs on the fp32 matrix-core attention."""
    fn = nat.lib().va_select_exact_segment_keys if exact else nat.lib().va_select_segment_keys
    return int(fn(Sk, k_local_size, group_k_block))


def select_segments(qs_chunk, k, J0, gap, gaps, causal, q_pooling_size, k_local_size,
                    group_k_block, wo_init, segk, bsq=None, dense_stride=0, indices=None,
                    scratch=None):
    """Split TilingSelect (the form VecAttention_prefill runs): keys cut into
    segments of `segk` keys selected in parallel.  Returns (counts
    (B, Hq, nc, nseg) int32, indices int32): segment s of a row writes from slot
    max(s*segk, smin) - smin of the row in the index layout.  `indices` and
    `scratch` may be passed in (int32 / fp32 device buffers at least as large as
    the index layout and va_select_segments_scratch_floats) to reuse them.
    """
    if qs_chunk.stride(-1) != 1:
        qs_chunk = qs_chunk.contiguous()
    if k.stride(-1) != 1:
        k = k.contiguous()
    B, Hq, nc, D = qs_chunk.shape
    Hk, Sk = k.shape[1], k.shape[2]
    if bsq is None:
        bsq = reference_block_size_q(q_pooling_size, k_local_size, group_k_block, D, causal)
    nseg = -(-Sk // segk)
    cap = index_capacity(B, Hq, Sk, q_pooling_size, causal, wo_init, J0, nc, dense_stride)
    counts = torch.empty(B, Hq, nc, nseg, dtype=torch.int32, device=k.device)
    if indices is None:
        indices = torch.empty(max(cap, 1), dtype=torch.int32, device=k.device)
    elif indices.dtype != torch.int32 or indices.numel() < cap:
        raise AssertionError(f"indices: need {cap} int32 slots")
    nscr = int(nat.lib().va_select_segments_scratch_floats(B, Hq, Hk, Sk, nc, segk, k_local_size,
                                                            group_k_block))
    if nscr < 0:
        raise AssertionError("va_select_segments_scratch_floats: invalid sizes")
    if scratch is None:
        scratch = torch.empty(max(nscr, 1), dtype=torch.float32, device=k.device)
    elif scratch.dtype != torch.float32 or scratch.numel() < nscr:
        raise AssertionError(f"scratch: need {nscr} fp32 slots")
    else:
        nscr = scratch.numel()
    with torch.cuda.device(k.device):
        rc = nat.lib().va_select_segments(
            nat.dtype_code(k), nat.ptr(qs_chunk), qs_chunk.stride(0), qs_chunk.stride(1),
            qs_chunk.stride(2), nat.ptr(k), k.stride(0), k.stride(1), k.stride(2), B, Hq, Hk, Sk, D,
            q_pooling_size, k_local_size, group_k_block, int(causal), int(wo_init), J0, nc, bsq,
            float(gap), nat.ptr(gaps), dense_stride, segk, nat.ptr(counts), nat.ptr(indices),
            nat.ptr(scratch), nscr, _stream(k))
    nat.check("va_select_segments", rc)
    return counts, indices


def select_csr(qs_chunk, k, J0, gap, gaps, causal, q_pooling_size, k_local_size, group_k_block,
               wo_init, segk=0, bsq=None):
    """TilingSelect into the compact (CSR) layout: returns (counts, offsets,
    indices) with offsets (B*Hq*nc + 1,) int64 and row r = (b*Hq + h)*nc + jr
    holding its keys, ascending, at indices[offsets[r]:offsets[r+1]].  counts
    is (B, Hq, nc) int32, or (B, Hq, nc, nseg) with segk > 0 (the split of
    select_segments).  Two library calls: the counting one, a read of the
    total (one host synchronisation, to size `indices`), the writing one.
    """
    if qs_chunk.stride(-1) != 1:
        qs_chunk = qs_chunk.contiguous()
    if k.stride(-1) != 1:
        k = k.contiguous()
    B, Hq, nc, D = qs_chunk.shape
    Hk, Sk = k.shape[1], k.shape[2]
    if bsq is None:
        bsq = reference_block_size_q(q_pooling_size, k_local_size, group_k_block, D, causal)
    if segk:
        counts = torch.empty(B, Hq, nc, -(-Sk // segk), dtype=torch.int32, device=k.device)
        nscr = int(nat.lib().va_select_segments_scratch_floats(B, Hq, Hk, Sk, nc, segk,
                                                                k_local_size, group_k_block))
    else:
        counts = torch.empty(B, Hq, nc, dtype=torch.int32, device=k.device)
        nscr = int(nat.lib().va_select_scratch_floats(B, Hk))
    if nscr < 0:
        raise AssertionError("scratch size query: invalid sizes")
    scratch = torch.empty(max(nscr, 1), dtype=torch.float32, device=k.device)
    offsets = torch.empty(B * Hq * nc + 1, dtype=torch.int64, device=k.device)

    def call(indices):
        with torch.cuda.device(k.device):
            rc = nat.lib().va_select_csr(
                nat.dtype_code(k), nat.ptr(qs_chunk), qs_chunk.stride(0), qs_chunk.stride(1),
                qs_chunk.stride(2), nat.ptr(k), k.stride(0), k.stride(1), k.stride(2), B, Hq, Hk,
                Sk, D, q_pooling_size, k_local_size, group_k_block, int(causal), int(wo_init), J0,
                nc, bsq, float(gap), nat.ptr(gaps), segk, nat.ptr(counts), nat.ptr(offsets),
                nat.ptr(indices), nat.ptr(scratch), nscr, _stream(k))
        nat.check("va_select_csr", rc)

    call(None)
    total = int(offsets[-1].item())
    indices = torch.empty(max(total, 1), dtype=torch.int32, device=k.device)
    call(indices)
    return counts, offsets, indices[:total]


def sparse_attention(q, k, v, out, J0, nc, counts, indices, causal, q_pooling_size, wo_init=None,
                     dense_stride=0, softmax_scale=None, kernel=nat.VA_ATTN_AUTO, segk=0):
    """Vector-sparse attention of q-block rows [J0, J0+nc) into `out` (B, Hq, Sq, D).
    With segk > 0, (counts, indices) are the segmented lists of select_segments."""
    q = q if q.stride(-1) == 1 else q.contiguous()
    k = k if k.stride(-1) == 1 else k.contiguous()
    v = v if v.stride(-1) == 1 else v.contiguous()
    B, Hq, Sq, D = q.shape
    Hk, Sk = k.shape[1], k.shape[2]
    if wo_init is None:
        wo_init = causal
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    if segk:
        with torch.cuda.device(q.device):
            rc = nat.lib().va_sparse_attn_segments(
                nat.dtype_code(q), nat.ptr(q), q.stride(0), q.stride(1), q.stride(2), nat.ptr(k),
                k.stride(0), k.stride(1), k.stride(2), nat.ptr(v), v.stride(0), v.stride(1),
                v.stride(2), nat.ptr(out), out.stride(0), out.stride(1), out.stride(2), B, Hq, Hk,
                Sq, Sk, D, q_pooling_size, int(causal), int(wo_init), J0, nc, dense_stride, segk,
                nat.ptr(counts), nat.ptr(indices), float(softmax_scale), _stream(q))
        nat.check("va_sparse_attn_segments", rc)
        return out
    with torch.cuda.device(q.device):
        rc = nat.lib().va_sparse_attn(
            nat.dtype_code(q), nat.ptr(q), q.stride(0), q.stride(1), q.stride(2), nat.ptr(k),
            k.stride(0), k.stride(1), k.stride(2), nat.ptr(v), v.stride(0), v.stride(1), v.stride(2),
            nat.ptr(out), out.stride(0), out.stride(1), out.stride(2), B, Hq, Hk, Sq, Sk, D,
            q_pooling_size, int(causal), int(wo_init), J0, nc, dense_stride, nat.ptr(counts),
            nat.ptr(indices), float(softmax_scale), int(kernel), _stream(q))
    nat.check("va_sparse_attn", rc)
    return out


def dense_attention(q, k, v, out=None, causal=True, softmax_scale=None):
    """Attention over every key (va_dense_attn): (B, Hq, Sq, D) q, (B, Hk, Sk, D)
    k/v; causal rows see keys up to i + Sk - Sq."""
    q = q if q.stride(-1) == 1 else q.contiguous()
    k = k if k.stride(-1) == 1 else k.contiguous()
    v = v if v.stride(-1) == 1 else v.contiguous()
    B, Hq, Sq, D = q.shape
    Hk, Sk = k.shape[1], k.shape[2]
    if out is None:
        out = torch.empty_like(q)
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    with torch.cuda.device(q.device):
        rc = nat.lib().va_dense_attn(
            nat.dtype_code(q), nat.ptr(q), q.stride(0), q.stride(1), q.stride(2), nat.ptr(k),
            k.stride(0), k.stride(1), k.stride(2), nat.ptr(v), v.stride(0), v.stride(1), v.stride(2),
            nat.ptr(out), out.stride(0), out.stride(1), out.stride(2), B, Hq, Hk, Sq, Sk, D,
            int(causal), float(softmax_scale), _stream(q))
    nat.check("va_dense_attn", rc)
    return out


def _stats_out(stats, B, Hq, Sq, device):
    if stats is None:
        return torch.empty(B, Hq, Sq, 2, dtype=torch.float32, device=device)
    if stats.dtype != torch.float32 or tuple(stats.shape) != (B, Hq, Sq, 2) or not stats.is_contiguous():
        raise AssertionError(f"stats must be a contiguous float32 ({B}, {Hq}, {Sq}, 2) tensor")
    return stats


def dense_row_stats(q, k, causal, softmax_scale=None, kernel=nat.VA_ATTN_AUTO, stats=None):
    """Softmax statistics of every query row over every key (va_dense_row_stats).

    Returns stats (B, Hq, Sq, 2) float32: (m, l) with l = sum_j 2^(s_ij - m),
    s_ij = q_i.k_j * scale * log2(e); causal rows see keys <= i + Sk - Sq.
    """
    q = q if q.stride(-1) == 1 else q.contiguous()
    k = k if k.stride(-1) == 1 else k.contiguous()
    B, Hq, Sq, D = q.shape
    Hk, Sk = k.shape[1], k.shape[2]
    stats = _stats_out(stats, B, Hq, Sq, q.device)
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    with torch.cuda.device(q.device):
        rc = nat.lib().va_dense_row_stats(
            nat.dtype_code(q), nat.ptr(q), q.stride(0), q.stride(1), q.stride(2), nat.ptr(k),
            k.stride(0), k.stride(1), k.stride(2), B, Hq, Hk, Sq, Sk, D, int(causal),
            float(softmax_scale), int(kernel), nat.ptr(stats), _stream(q))
    nat.check("va_dense_row_stats", rc)
    return stats


def sparse_row_stats(q, k, J0, nc, counts, indices, causal, q_pooling_size, wo_init=None,
                     dense_stride=0, softmax_scale=None, kernel=nat.VA_ATTN_AUTO, stats=None,
                     segk=0):
    """Softmax statistics of the rows of q-blocks [J0, J0+nc) over their
    vector-sparse key sets (va_sparse_row_stats); other rows of `stats` are
    left as they are.  Same (m, l) convention as dense_row_stats.  With
    segk > 0, (counts, indices) are the segmented lists of select_segments
    (va_sparse_row_stats_segments, MFMA kernel)."""
    q = q if q.stride(-1) == 1 else q.contiguous()
    k = k if k.stride(-1) == 1 else k.contiguous()
    B, Hq, Sq, D = q.shape
    Hk, Sk = k.shape[1], k.shape[2]
    stats = _stats_out(stats, B, Hq, Sq, q.device)
    if wo_init is None:
        wo_init = causal
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    with torch.cuda.device(q.device):
        if segk:
            rc = nat.lib().va_sparse_row_stats_segments(
                nat.dtype_code(q), nat.ptr(q), q.stride(0), q.stride(1), q.stride(2), nat.ptr(k),
                k.stride(0), k.stride(1), k.stride(2), B, Hq, Hk, Sq, Sk, D, q_pooling_size,
                int(causal), int(wo_init), J0, nc, dense_stride, segk, nat.ptr(counts),
                nat.ptr(indices), float(softmax_scale), nat.ptr(stats), _stream(q))
            nat.check("va_sparse_row_stats_segments", rc)
            return stats
        rc = nat.lib().va_sparse_row_stats(
            nat.dtype_code(q), nat.ptr(q), q.stride(0), q.stride(1), q.stride(2), nat.ptr(k),
            k.stride(0), k.stride(1), k.stride(2), B, Hq, Hk, Sq, Sk, D, q_pooling_size,
            int(causal), int(wo_init), J0, nc, dense_stride, nat.ptr(counts), nat.ptr(indices),
            float(softmax_scale), int(kernel), nat.ptr(stats), _stream(q))
    nat.check("va_sparse_row_stats", rc)
    return stats


def fuse_qk_softmax_minp_wo_causal(
    avg_q_chunk,
    k,
    avg_q_chunk_offset,
    gap,
    causal=True,
    q_pooling_size=128,
    k_local_size=128,
    wo_initial=False,
    group_k_block=1,
):
    """Q.K^T scoring of pooled query blocks with MinP column selection.

    Mirrors spattn/src/kernels/vecattention_kernels.py:59-181: `avg_q_chunk`
    holds the pooled (unscaled) rows of a chunk starting at q-block
    `avg_q_chunk_offset`; `gap` is a float or a per-(b, h) tensor.  Returns
    column_count (B, H, nqb) int32 and column_index (B, H, nqb, max_count)
    int32, zero beyond each row's count, trimmed to max(min(k_len, max_count), 1)
    columns (a host synchronisation, as in the reference).  Index order within a
    row is ascending (the reference's order is that of its atomic appends).
    """
    B, H, nqb, D = avg_q_chunk.shape
    assert avg_q_chunk.shape[1] % k.shape[1] == 0
    assert not causal or q_pooling_size % k_local_size == 0
    k_len = k.shape[-2]
    sm = torch.tensor(1.0 / math.sqrt(D), dtype=torch.float32)
    qs = (avg_q_chunk.float() * sm.to(avg_q_chunk.device)).to(avg_q_chunk.dtype)
    if isinstance(gap, torch.Tensor):
        gaps = gap.to(device=k.device, dtype=torch.float32)
        gaps = (gaps.expand(B, H) if gaps.dim() <= 1 else gaps).contiguous()
        gap_scalar = 0.0
    else:
        gaps, gap_scalar = None, float(gap)
    padded_k = math.ceil(k_len / k_local_size) * k_local_size
    index = torch.zeros(B, H, nqb, padded_k, dtype=torch.int32, device=k.device)
    count, index = select_rows(qs, k, avg_q_chunk_offset, gap_scalar, gaps, causal, q_pooling_size,
                               k_local_size, group_k_block, wo_initial, dense_stride=padded_k,
                               indices=index)
    max_count = int(count.max().item()) if count.numel() else 0
    return count, index[:, :, :, :max(min(k_len, max_count), 1)].contiguous()


__all__ = [
    "average_vector", "fuse_qk_softmax_minp_wo_causal", "pool_scaled", "select_rows",
    "sparse_attention", "index_capacity", "row_offset", "threshold_to_gap", "segment_keys",
    "select_segments", "dense_row_stats", "sparse_row_stats",
]
