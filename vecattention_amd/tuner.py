"""Recall / sparsity evaluation of the threshold tuner, on the GPU kernels.

Mirrors ``seg_pr_perHead`` (spattn/threshold/model_tuner.py:118-226), the
function the tuner's bisection (``tune_per_layer_coop_bisect``,
model_tuner.py:295-507) calls once per iteration with a per-head threshold
vector.  For every query row it measures how much of the row's dense softmax
mass falls on the keys VecAttention would keep (recall), and how many of the
causally visible keys those are (sparsity), averaged per head.

The reference materialises the dense S x S softmax per head and a boolean
mask.  Here nothing quadratic is stored: two passes of the attention kernel
in its statistics form give, per row, the dense (m_d, l_d) over every visible
key and the sparse (m_s, l_s) over the selected key set, and

    recall_i = l_s * 2^(m_s - m_d) / l_d

is the masked softmax sum of model_tuner.py:202-219 (probabilities of keys
outside the causal window are 0 there and absent here).  The mask size of a
row is a closed form of the selection counts: the local blocks of its q-block
(causal: [0, qps) for J >= 1 and the whole diagonal block, clipped to S_k,
as blk_count/blk_idx at model_tuner.py:155-176 build them) plus its selected
columns, so sparsity needs no mask either.  As in the reference, the mask
counts the whole diagonal block while a row sees only the keys up to itself,
so causal sparsity falls below 0 when short sequences make those rows weigh.
"""
import math

import torch

from . import stages


def _bf16_exact(t):
    return t.dtype == torch.float32 and bool(torch.equal(t.to(torch.bfloat16).float(), t))


def _gaps(threshold, B, H, device):
    """gap = -log(threshold + 1e-50) as model_tuner.py:150: the sum in the
    threshold's dtype (for fp32, 1e-50 rounds to 0), its logarithm in fp64
    rounded once to fp32 (the correctly rounded value of the reference's fp32
    logarithm), as fp32 per (b, h) for the selection."""
    gap = -torch.log((threshold + 1e-50).to(torch.float64))
    gap = gap.to(device=device, dtype=torch.float32)
    if gap.dim() == 0:
        gap = gap.expand(B, H)
    elif gap.dim() == 1:
        if gap.numel() != H:
            raise AssertionError(f"per-head threshold has {gap.numel()} entries for {H} heads")
        gap = gap.unsqueeze(0).expand(B, H)
    elif tuple(gap.shape) != (B, H):
        raise AssertionError(f"threshold shape {tuple(threshold.shape)} is not (H,) or (B, H)")
    return gap.contiguous()


def local_keys(nqb, block_size_q, Sk, causal, device):
    """Keys in the local blocks of each q-block (B/H-independent), int64 (nqb,)."""
    J = torch.arange(nqb, device=device, dtype=torch.int64)
    if not causal:
        return torch.zeros_like(J)
    n_init = torch.where(J >= 1, block_size_q, 0)
    n_diag = (Sk - J * block_size_q).clamp(min=0, max=block_size_q)
    return n_init + n_diag


def recall_from_stats(dense, sparse):
    """Per-row recall l_s 2^(m_s - m_d) / l_d from two (..., 2) statistics tensors."""
    m_d, l_d = dense[..., 0], dense[..., 1]
    m_s, l_s = sparse[..., 0], sparse[..., 1]
    r = l_s * torch.exp2(m_s - m_d) / l_d
    return torch.where(l_s > 0, r, torch.zeros_like(r))


def seg_pr_perHead(q, k, block_size_q, block_size_k=16, group_size_k=16, threshold=None,
                   chunk_size=8 * 1024, causal=False):
    """(recall (H,), sparsity (H,)) in q's dtype, as model_tuner.py:118-226.

    q: (B, H, S, D), k: (B, Hk, S_k, D) on the GPU (Hk dividing H; the
    reference needs Hk == H); threshold: per-head tensor (H,) (or (B, H), or a
    0-dim tensor).  The tuner passes fp32 copies of the model's bf16 Q/K
    (model_tuner.py:53-77); such values are exactly representable in bf16, so
    the score passes run on the bf16 MFMA kernels without changing a score.
    Other fp32 inputs take the per-row fp32 kernel.  The selection runs on the
    inputs as given (pooled per chunk, scaled, selected as
    fuse_qk_softmax_minp_wo_causal with wo_initial=causal).
    """
    if q.dim() != 4 or k.dim() != 4:
        raise AssertionError("q and k must be (batch, heads, seq, head_dim)")
    B, H, S, D = q.shape
    Sk = k.shape[2]
    if k.shape[0] != B or k.shape[3] != D or H % k.shape[1]:
        raise AssertionError(f"query and key shape mismatch, query: {tuple(q.shape)}, key: {tuple(k.shape)}")
    if not q.is_cuda:
        raise RuntimeError("seg_pr_perHead runs on the GPU")
    if causal and S != Sk:
        raise NotImplementedError("causal evaluation needs equal query and key lengths")
    if chunk_size % block_size_q:
        raise AssertionError("chunk_size must be a multiple of block_size_q")
    gaps = _gaps(threshold, B, H, q.device)

    qa, ka = q, k
    if q.dtype == torch.float32 and _bf16_exact(q) and _bf16_exact(k):
        qa, ka = q.to(torch.bfloat16), k.to(torch.bfloat16)
    dense = stages.dense_row_stats(qa, ka, causal)
    sparse = torch.zeros_like(dense)
    nqb = math.ceil(S / block_size_q)
    counts_all = torch.empty(B, H, nqb, dtype=torch.int32, device=q.device)
    # fp32 queries select on the exact kernel; when the statistics run on the
    # MFMA kernel (bf16-exact inputs) that selection is split into key
    # segments (the lists are the same keys in the same order)
    segk = 0
    if (q.dtype == torch.float32 and qa.dtype != torch.float32 and D in (64, 128)
            and block_size_q in (64, 128)):
        segk = stages.segment_keys(Sk, block_size_k, group_size_k, exact=True)
    for c0 in range(0, S, chunk_size):
        rows = min(chunk_size, S - c0)
        J0, nc = c0 // block_size_q, math.ceil(rows / block_size_q)
        scaled, _ = stages.pool_scaled(q[:, :, c0:c0 + rows], block_size_q)
        if segk:
            counts, indices = stages.select_segments(scaled, k, J0, 0.0, gaps, causal,
                                                     block_size_q, block_size_k, group_size_k,
                                                     causal, segk)
            stages.sparse_row_stats(qa, ka, J0, nc, counts, indices, causal, block_size_q,
                                    wo_init=causal, stats=sparse, segk=segk)
            counts = counts.sum(-1, dtype=torch.int32)
        else:
            counts, indices = stages.select_rows(scaled, k, J0, 0.0, gaps, causal, block_size_q,
                                                 block_size_k, group_size_k, causal)
            stages.sparse_row_stats(qa, ka, J0, nc, counts, indices, causal, block_size_q,
                                    wo_init=causal, stats=sparse)
        counts_all[:, :, J0:J0 + nc] = counts

    recall = recall_from_stats(dense, sparse)  # (B, H, S)
    overall_recall = recall.sum(dim=(0, 2)) / (B * S)

    # mask size / visible keys per row (model_tuner.py:218-219)
    mask_rows = (local_keys(nqb, block_size_q, Sk, causal, q.device).view(1, 1, nqb) +
                 counts_all.to(torch.int64))
    mask_rows = mask_rows.repeat_interleave(block_size_q, dim=2)[:, :, :S].to(torch.float64)
    i = torch.arange(S, device=q.device, dtype=torch.float64)
    visible = torch.clamp(i + 1, max=Sk) if causal else torch.full_like(i, Sk)
    ratio_sum = (mask_rows / visible).sum(dim=(0, 2))
    sparsity = 1.0 - ratio_sum / (B * S)
    return overall_recall.to(q.dtype), sparsity.to(q.dtype)


__all__ = ["seg_pr_perHead", "recall_from_stats", "local_keys"]
