"""Brute-force check of the oracle's selection (orc.select) — CPU only.

The brute force below is written from the reference kernel's program
structure, not from the oracle's code
(spattn/src/kernels/vecattention_kernels.py:91-181,206-272):

- a grid of programs (q-tile p of BLOCK_SIZE_Q pooled rows, key group g of
  group_k_block tiles), over the padded row and key ranges;
- per program the key range [start, end): start = g*G*BK, raised to
  q_pooling_size when the initial block is skipped; end = g*G*BK + G*BK, capped
  at the key length and, when causal, at the program's last row's causal limit
  (chunk_off + (p+1)*BSQ)*qps - qps;
- per row, a running maximum over the whole tiles of its program, updated with
  the tile's maximum before the tile's keys are compared; key c is selected iff
  fp32(s_c + gap) >= m and, when causal, the row index r inside the program
  satisfies r > trunc((k_offset - offset_at_causal) / qps);
- keys past the key length (the NaN pad) never count and never move m.

Inputs are small integers (queries in [-3, 3], keys in [-3, 3]) and gaps are
multiples of 1/2, so every score and every fp32(s + gap) is exact and the
check does not depend on rounding: it pins the rule (tile order, group starts,
the prefix maximum, ties at equality, the causal tile rule and its first-row
quirk, chunk origins, BLOCK_SIZE_Q and key tails).
"""
import math

import numpy as np
import pytest

from oracle import oracle as orc


def trunc_div(a, b):
    q = abs(a) // b
    return q if a >= 0 else -q


def brute_select(qs, k, J0, nc, gap, qps, bk, G, causal, wo_init, bsq):
    """Lists for chunk rows [J0, J0+nc) of one head; qs (nqb_total, D), k (Sk, D)."""
    Sk = k.shape[0]
    lists = [[] for _ in range(nc)]
    n_prog = math.ceil(nc / bsq)
    padded_k = math.ceil(Sk / bk) * bk
    n_groups = math.ceil(padded_k / (bk * G))
    scores = qs[J0:J0 + nc].astype(np.int64) @ k.astype(np.int64).T  # exact integers
    for p in range(n_prog):
        off_causal = (J0 + p * bsq) * qps
        for g in range(n_groups):
            start = g * G * bk if not wo_init else max(qps, g * G * bk)
            limit = Sk if not causal else min(Sk, (J0 + (p + 1) * bsq) * qps - qps)
            end = min(limit, g * G * bk + bk * G)
            if end <= start:
                continue
            for r in range(bsq):
                jr = p * bsq + r
                if jr >= nc:
                    break  # padded rows: trimmed by the reference
                m = -math.inf
                for ko in range(start, end, bk):
                    tile = [c for c in range(ko, ko + bk) if c < Sk]
                    if tile:
                        m = max(m, max(float(scores[jr, c]) for c in tile))
                    allowed = (not causal) or r > trunc_div(ko - off_causal, qps)
                    if not allowed:
                        continue
                    for c in tile:
                        if np.float32(float(scores[jr, c]) + gap) >= m:
                            lists[jr].append(c)
    return [np.array(sorted(x), np.int64) for x in lists]


CASES = []
_rng = np.random.default_rng(1234)
for _i in range(48):
    _bk = int(_rng.choice([16, 32, 64]))
    _qps = int(_rng.choice([64, 128]))
    _causal = bool(_rng.integers(2))
    _G = int(_rng.choice([1, 2, 3, 4, 5, 16, 1000]))
    _bsq = int(_rng.choice([1, 2, 3, 4, 64]))
    _nqb = int(_rng.integers(2, 13))
    if _causal:
        _S = _nqb * _qps - int(_rng.integers(0, _qps))          # Sq == Sk, partial last block
        _Sk = _S
        _wo = True
    else:
        _S = _nqb * _qps - int(_rng.integers(0, _qps))
        _Sk = int(_rng.integers(40, 700))                       # Sq != Sk, key tails
        _wo = bool(_rng.integers(2)) and _qps % _bk == 0
    _nqb = math.ceil(_S / _qps)
    _J0 = int(_rng.integers(0, _nqb))
    _nc = int(_rng.integers(1, _nqb - _J0 + 1))
    _gap = float(_rng.choice([0.0, 0.5, 1.5, 3.0, 6.0, 1e6]))
    CASES.append((_i, _bk, _qps, _causal, _G, _bsq, _S, _Sk, _wo, _J0, _nc, _gap))


@pytest.mark.parametrize("case", CASES, ids=[f"c{c[0]}" for c in CASES])
def test_oracle_select_equals_brute_force(case):
    i, bk, qps, causal, G, bsq, S, Sk, wo, J0, nc, gap = case
    rng = np.random.default_rng(100 + i)
    D = 8
    nqb = math.ceil(S / qps)
    qs = rng.integers(-3, 4, size=(nqb, D)).astype(np.float32)
    k = rng.integers(-3, 4, size=(Sk, D)).astype(np.float32)
    # a few columns that dominate every row (vertical structure), so running
    # maxima both rise and stay flat across tiles
    for c in rng.choice(Sk, size=min(4, Sk), replace=False):
        k[c] = 3.0
    want = brute_select(qs, k, J0, nc, np.float32(gap), qps, bk, G, causal, wo, bsq)
    counts, lists = orc.select(qs[None, None], k[None, None], J0, nc,
                               np.full(1, gap, np.float32), qps, bk, G, causal, wo, bsq)
    for jr in range(nc):
        got = np.asarray(lists[0][0][jr], np.int64)
        assert int(counts[0, 0, jr]) == len(want[jr]), (jr, counts[0, 0, jr], len(want[jr]))
        assert np.array_equal(got, want[jr]), (jr, sorted(set(got) ^ set(want[jr]))[:8])


def test_brute_force_detects_a_planted_mistake():
    # The brute force is sensitive to the order of "update the maximum" and
    # "compare": comparing against the maximum of the earlier tiles only (a
    # plausible mistake) selects a different set on these inputs.
    rng = np.random.default_rng(7)
    qs = rng.integers(-3, 4, size=(4, 8)).astype(np.float32)
    k = rng.integers(-3, 4, size=(256, 8)).astype(np.float32)
    right = brute_select(qs, k, 0, 4, np.float32(1.5), 64, 16, 16, False, False, 64)

    def stale_max(qs, k, gap, bk, G):
        out = []
        s = qs.astype(np.int64) @ k.astype(np.int64).T
        for jr in range(qs.shape[0]):
            sel = []
            for g0 in range(0, k.shape[0], bk * G):
                m = -math.inf
                for ko in range(g0, min(g0 + bk * G, k.shape[0]), bk):
                    for c in range(ko, min(ko + bk, k.shape[0])):
                        if np.float32(float(s[jr, c]) + gap) >= m:
                            sel.append(c)
                    m = max(m, max(float(s[jr, c]) for c in range(ko, min(ko + bk, k.shape[0]))))
            out.append(np.array(sel))
        return out
    wrong = stale_max(qs, k, np.float32(1.5), 16, 16)
    assert any(not np.array_equal(a, b) for a, b in zip(right, wrong))
    _, lists = orc.select(qs[None, None], k[None, None], 0, 4, np.full(1, 1.5, np.float32), 64, 16,
                          16, False, False, 64)
    assert all(np.array_equal(np.asarray(lists[0][0][j], np.int64), right[j]) for j in range(4))
