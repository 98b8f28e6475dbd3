"""GPU parity of the tuner's recall/sparsity evaluation (run on an MI355X).

- Row statistics (va_dense_row_stats / va_sparse_row_stats): the row's
  log-sum-exp, (m + log2 l) * ln 2, against float64 on the CPU over the same
  key set; tolerance 2e-5 relative (fp32 accumulation of exact products).
- seg_pr_perHead against the oracle's restatement of model_tuner.py:118-226:
  recall within 1e-5 absolute for fp32 inputs (probabilities summed in fp32
  here and in float64 there), sparsity within 1e-6 (the selection is exact,
  so the mask counts are equal).
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from vecattention_amd import _native as nat
from vecattention_amd import stages, tuner

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
LN2 = math.log(2.0)


def note(*a):
    print("[case]", *a, flush=True)


def _qk(B, Hq, Hk, Sq, Sk, D, dtype, seed, bf16_values=True):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Hq, Sq, D, generator=g)
    k = torch.randn(B, Hk, Sk, D, generator=g)
    k[:, :, 7] *= 3.0
    if bf16_values:
        q, k = q.bfloat16().float(), k.bfloat16().float()
    return q.to(dtype), k.to(dtype)


def _lse(stats):
    s = stats.double().cpu().numpy()
    with np.errstate(divide="ignore"):
        return (s[..., 0] + np.log2(s[..., 1])) * LN2


def _lse_ref(q, k, keys_of, causal_off=None):
    """float64 log-sum-exp of every row over keys_of(b, h, i) (or all keys with
    the bottom-right causal offset)."""
    qn = q.double().cpu().numpy()
    kn = k.double().cpu().numpy()
    B, Hq, Sq, D = qn.shape
    rep = Hq // kn.shape[1]
    out = np.full((B, Hq, Sq), -np.inf)
    for b in range(B):
        for h in range(Hq):
            s = qn[b, h] @ kn[b, h // rep].T / math.sqrt(D)
            for i in range(Sq):
                keys = keys_of(b, h, i)
                if len(keys):
                    x = s[i, keys]
                    m = x.max()
                    out[b, h, i] = m + math.log(np.exp(x - m).sum())
    return out


@pytest.mark.parametrize("dtype,kernel", [(torch.bfloat16, nat.VA_ATTN_MFMA),
                                          (torch.float16, nat.VA_ATTN_MFMA),
                                          (torch.float32, nat.VA_ATTN_SIMPLE)])
@pytest.mark.parametrize("causal,Sq,Sk", [(True, 200, 200), (True, 130, 300), (False, 150, 333)])
def test_dense_row_stats(dtype, kernel, causal, Sq, Sk):
    note("dense stats", dtype, kernel, causal, Sq, Sk)
    q, k = _qk(1, 4, 2, Sq, Sk, 128 if dtype != torch.float32 else 64, dtype, 11)
    st = stages.dense_row_stats(q.to(DEV), k.to(DEV), causal, kernel=kernel)
    torch.cuda.synchronize()
    off = Sk - Sq
    want = _lse_ref(q, k, lambda b, h, i: np.arange(i + off + 1 if causal else Sk))
    np.testing.assert_allclose(_lse(st), want, rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize("dtype,kernel", [(torch.bfloat16, nat.VA_ATTN_MFMA),
                                          (torch.float32, nat.VA_ATTN_SIMPLE)])
@pytest.mark.parametrize("causal,qps", [(True, 64), (True, 128), (False, 64)])
def test_sparse_row_stats(dtype, kernel, causal, qps):
    note("sparse stats", dtype, kernel, causal, qps)
    B, Hq, Hk, S, D = 1, 4, 2, 448, 64
    q, k = _qk(B, Hq, Hk, S, S, D, dtype, 12)
    nqb = math.ceil(S / qps)
    gaps = np.full(B * Hq, 1.5, np.float32)
    _, qs = orc.pool(q.float(), qps, "bfloat16" if dtype == torch.bfloat16 else "float32")
    cnt, lists = orc.select(qs, k.float(), 0, nqb, gaps, qps, 16, 4, causal, causal, 64)
    # the oracle's lists in the index layout of the library
    cap = stages.index_capacity(B, Hq, S, qps, causal, causal, 0, nqb)
    idx = np.zeros(max(cap, 1), np.int32)
    for h in range(Hq):
        for jr in range(nqb):
            o = stages.row_offset(S, qps, causal, causal, 0, nqb, h, jr)
            idx[o:o + len(lists[0][h][jr])] = lists[0][h][jr]
    counts = torch.from_numpy(cnt.astype(np.int32)).to(DEV)
    indices = torch.from_numpy(idx).to(DEV)
    st = stages.sparse_row_stats(q.to(DEV), k.to(DEV), 0, nqb, counts, indices, causal, qps,
                                 kernel=kernel)
    torch.cuda.synchronize()
    blk_count, blk_idx = orc.local_blocks(B, Hq, S, qps, causal)

    def keys_of(b, h, i):
        J = i // qps
        ks = orc.key_set(J, blk_count[b, h, J], blk_idx[b, h, J], lists[b][h][J], S)
        return ks[ks <= i] if causal else ks
    np.testing.assert_allclose(_lse(st), _lse_ref(q, k, keys_of), rtol=2e-5, atol=2e-5)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("bf16_values", [True, False])
def test_seg_pr_perhead_matches_oracle(causal, bf16_values):
    note("seg_pr", causal, bf16_values)
    B, H, S, D = 2, 3, 384, 64
    q, k = _qk(B, H, H, S, S, D, torch.float32, 13, bf16_values=bf16_values)
    th = torch.tensor([0.97, 0.9, 0.75])  # pooled scores spread ~0.1-0.3: partial selections
    r, s = tuner.seg_pr_perHead(q.to(DEV), k.to(DEV), 64, 16, 8, threshold=th.to(DEV),
                                chunk_size=128, causal=causal)
    torch.cuda.synchronize()
    rr, ss = orc.seg_pr_perhead(q, k, 64, 16, 8, th.numpy(), chunk_size=128, causal=causal)
    assert r.dtype == torch.float32 and s.dtype == torch.float32
    np.testing.assert_allclose(r.cpu().numpy(), rr, atol=1e-5)
    np.testing.assert_allclose(s.cpu().numpy(), ss, atol=1e-6)
    assert float(r.min()) > 0.0 and (causal or float(s.max()) > 0.05)


def test_seg_pr_perhead_gqa_and_long_keys():
    """Non-causal, Sq != Sk (the Hunyuan shape), kv heads shared by two q heads."""
    note("seg_pr gqa")
    q, _ = _qk(1, 4, 4, 320, 320, 64, torch.float32, 14)
    _, k = _qk(1, 2, 2, 520, 520, 64, torch.float32, 15)
    th = torch.tensor([0.97, 0.9, 0.9, 0.8])
    r, s = tuner.seg_pr_perHead(q.to(DEV), k.to(DEV), 64, 16, 16, threshold=th.to(DEV),
                                causal=False)
    torch.cuda.synchronize()
    rr, ss = orc.seg_pr_perhead(q, k, 64, 16, 16, th.numpy(), causal=False)
    np.testing.assert_allclose(r.cpu().numpy(), rr, atol=1e-5)
    np.testing.assert_allclose(s.cpu().numpy(), ss, atol=1e-6)


@pytest.mark.parametrize("causal,qps,D", [(True, 64, 128), (False, 128, 64)],
                         ids=["causal-qps64-d128", "noncausal-qps128-d64"])
def test_sparse_row_stats_on_segmented_lists_equal_unsplit(causal, qps, D):
    # The split exact selection (fp32 pooled queries, the tuner's form) and the
    # MFMA statistics over its segmented lists give the statistics of the
    # unsplit lists bit for bit: the concatenated lists are the same keys in
    # the same order.
    note("sparse stats segmented", causal, qps, D)
    B, Hq, Hk, S, bk, G = 1, 4, 2, 2300, 16, 16
    q, k = _qk(B, Hq, Hk, S, S, D, torch.float32, 16)
    qd, kd = q.to(DEV), k.to(DEV)
    qb, kb = qd.to(torch.bfloat16), kd.to(torch.bfloat16)
    qs, _ = stages.pool_scaled(qd, qps)
    nqb = qs.shape[2]
    segk = stages.segment_keys(S, bk, G, exact=True)
    assert segk > 0 and -(-S // segk) > 1
    gaps = torch.full((B, Hq), 1.0, dtype=torch.float32, device=DEV)
    c1, i1 = stages.select_rows(qs, kd, 0, 0.0, gaps, causal, qps, bk, G, causal)
    c2, i2 = stages.select_segments(qs, kd, 0, 0.0, gaps, causal, qps, bk, G, causal, segk)
    assert torch.equal(c2.sum(-1, dtype=torch.int32), c1) and int(c1.sum()) > 0
    s1 = stages.sparse_row_stats(qb, kb, 0, nqb, c1, i1, causal, qps)
    s2 = stages.sparse_row_stats(qb, kb, 0, nqb, c2, i2, causal, qps, segk=segk)
    torch.cuda.synchronize()
    assert torch.equal(s1, s2)
