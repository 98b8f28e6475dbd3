"""Pins of the oracle's restatement of the tuner's recall/sparsity evaluation
(oracle.seg_pr_perhead, spattn/threshold/model_tuner.py:118-226): closed forms
where the selection is empty or takes every selectable key, monotonicity in
the threshold, and chunk-size invariance where the selection has no
chunk-relative rule (non-causal)."""
import math

import numpy as np
import pytest

from oracle import oracle as orc


def _inputs(B, H, S, D, seed, Sk=None):
    rng = np.random.default_rng(seed)
    Sk = S if Sk is None else Sk
    q = rng.standard_normal((B, H, S, D)).astype(np.float32)
    k = rng.standard_normal((B, H, Sk, D)).astype(np.float32)
    k[:, :, 5] *= 3.0  # a heavy column, so that the selection is not trivial
    return q, k


def _dense_softmax(q, k, causal):
    s = (q.astype(np.float64) @ k.astype(np.float64).T) / math.sqrt(q.shape[-1])
    if causal:
        i = np.arange(q.shape[0])[:, None]
        s = np.where(np.arange(k.shape[0])[None, :] <= i, s, -np.inf)
    p = np.exp(s - s.max(axis=1, keepdims=True))
    return p / p.sum(axis=1, keepdims=True)


def _local_counts(S, qps):
    """(n_init, n_diag) of each q-block under the causal local-block rule."""
    nqb = math.ceil(S / qps)
    return [((qps if J >= 1 else 0), min(qps, S - J * qps)) for J in range(nqb)]


@pytest.mark.parametrize("th,recall,sparsity", [(0.0, 1.0, 0.0), (2.0, 0.0, 1.0)])
def test_noncausal_every_key_or_none(th, recall, sparsity):
    """th = 0: gap = +inf selects every key (recall 1, sparsity 0); th > 1:
    gap < 0 selects nothing, not even the maximum (recall 0, sparsity 1)."""
    q, k = _inputs(1, 2, 192, 16, 0)
    r, s = orc.seg_pr_perhead(q, k, 64, 16, 16, np.full(2, th, np.float32), causal=False)
    np.testing.assert_allclose(r, recall, atol=1e-12)
    np.testing.assert_allclose(s, sparsity, atol=1e-12)


def test_causal_local_blocks_only():
    """No columns (th > 1): recall is the softmax mass on [0, qps) and the
    diagonal block, sparsity 1 - mean((n_init + n_diag) / (i + 1))."""
    qps, S, D = 64, 200, 16
    q, k = _inputs(1, 2, S, D, 1)
    r, s = orc.seg_pr_perhead(q, k, qps, 16, 16, np.full(2, 2.0, np.float32), causal=True)
    loc = _local_counts(S, qps)
    for h in range(2):
        p = _dense_softmax(q[0, h], k[0, h], True)
        rec, ratio = [], []
        for i in range(S):
            J = i // qps
            n_init, n_diag = loc[J]
            keys = list(range(n_init)) + list(range(J * qps, J * qps + n_diag))
            rec.append(p[i, keys].sum())
            ratio.append((n_init + n_diag) / (i + 1))
        np.testing.assert_allclose(r[h], np.mean(rec), rtol=1e-12)
        np.testing.assert_allclose(s[h], 1.0 - np.mean(ratio), rtol=1e-12)


def test_causal_every_selectable_key():
    """th = 0 with fewer q-blocks than BSQ (no first-row tile rule applies
    past block 0): rows see every visible key (recall 1); mask J*qps +
    n_diag keys."""
    qps, S = 64, 256
    q, k = _inputs(1, 1, S, 16, 2)
    r, s = orc.seg_pr_perhead(q, k, qps, 16, 16, np.zeros(1, np.float32), causal=True)
    loc = _local_counts(S, qps)
    ratio = [((i // qps) * qps + loc[i // qps][1]) / (i + 1) for i in range(S)]
    np.testing.assert_allclose(r, 1.0, atol=1e-12)
    np.testing.assert_allclose(s, 1.0 - np.mean(ratio), rtol=1e-12)


@pytest.mark.parametrize("causal", [False, True])
def test_monotone_in_threshold(causal):
    """A smaller threshold (larger gap) selects a superset: recall does not
    fall and sparsity does not rise."""
    q, k = _inputs(1, 2, 256, 16, 3)
    prev = None
    for th in (0.3, 0.1, 0.02, 0.001):
        r, s = orc.seg_pr_perhead(q, k, 64, 16, 4, np.full(2, th, np.float32), causal=causal)
        if prev is not None:
            assert np.all(r >= prev[0] - 1e-12) and np.all(s <= prev[1] + 1e-12)
        prev = (r, s)
    assert prev[0].min() > 0.5


def test_noncausal_chunk_invariance():
    q, k = _inputs(2, 2, 320, 16, 4, Sk=384)
    th = np.array([0.05, 0.2], np.float32)
    a = orc.seg_pr_perhead(q, k, 64, 16, 8, th, chunk_size=128, causal=False)
    b = orc.seg_pr_perhead(q, k, 64, 16, 8, th, chunk_size=8192, causal=False)
    np.testing.assert_allclose(a[0], b[0], rtol=1e-12)
    np.testing.assert_allclose(a[1], b[1], rtol=1e-12)
