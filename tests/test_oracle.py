"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

The reference ships no tests, fixtures or golden vectors for this path, and it
cannot run here (Triton + an absent CUDA extension).  Each oracle function is
therefore checked against facts fixed independently of its own code:
closed forms, hand-derived known answers, torch library routines, invariants
of the rule, and the reference's own PyTorch twin of pooling.
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc


def bf16(x):
    return torch.as_tensor(x, dtype=torch.float32).to(torch.bfloat16).float().numpy()


# ---------------------------------------------------------------- pooling ----

def test_pool_constant_rows_partial_last_block():
    # Every row equal to c: each block mean is c, including a 16-row tail block
    # (a divide by qps instead of the real row count would give c/4 there).
    S, qps, D = 208, 64, 8
    q = np.broadcast_to(np.float32(1.5), (1, 2, S, D)).copy()
    pooled, scaled = orc.pool(q, qps, "bfloat16")
    assert pooled.shape == (1, 2, 4, D)
    assert np.all(pooled == 1.5)
    # scaled = bf16(1.5 * fp32(1/sqrt(8))) = bf16(0.53033006...) = 0.53125
    assert np.all(scaled == np.float32(0.53125))


def test_pool_row_index_closed_form():
    # Row r holds the value r (exact in fp32): block J mean = J*qps + (rows-1)/2.
    S, qps = 200, 64
    q = np.arange(S, dtype=np.float32)[None, None, :, None].repeat(2, axis=3)
    pooled, _ = orc.pool(q, qps, "float32")
    assert list(pooled[0, 0, :, 0]) == [31.5, 95.5, 159.5, 195.5]


def test_pool_matches_reference_pytorch_twin():
    # spattn/threshold/model_tuner.py:79-95 (and utils.py:352-360): pad with
    # zeros, fp32 mean over the padded block, rescale the last block, cast.
    g = torch.Generator().manual_seed(3)
    for S, qps in [(4096, 64), (1000, 128), (333, 64)]:
        x = torch.randn(1, 3, S, 64, generator=g).to(torch.bfloat16)
        xf = x.float()
        nb = math.ceil(S / qps)
        pad = nb * qps - S
        twin = torch.nn.functional.pad(xf, (0, 0, 0, pad)).view(1, 3, nb, qps, 64).mean(-2)
        twin[:, :, -1] = twin[:, :, -1] * qps / (qps - pad)
        twin = twin.to(torch.bfloat16).float().numpy()
        pooled, _ = orc.pool(x, qps, "bfloat16")
        # The twin sums in fp32 in torch's order: equal up to one bf16 ulp.
        ulp = np.abs(twin) * 2.0 ** -7 + 1e-30
        assert np.all(np.abs(pooled - twin) <= ulp)
        assert np.mean(pooled == twin) > 0.97


def test_pool_scale_is_fp32_product_then_rne():
    # scaled = T(fp32(p) * fp32(1/sqrt(D))); for D=128 fp32(1/sqrt(128)) = 0.0883883461356163.
    assert np.float32(1 / math.sqrt(128)) == np.float32(0.0883883461356163)
    q = np.full((1, 1, 64, 128), 3.0, np.float32)
    _, scaled = orc.pool(q, 64, "bfloat16")
    # 3 * 0.0883883461... = 0.26516503... -> bf16 0.265625
    assert np.all(scaled == np.float32(0.265625))


def test_rounding_helpers():
    L = orc.lib()
    # bf16 RNE: 1 + 2^-8 is a tie -> even (1.0); 1 + 3*2^-8 -> 1 + 2^-6... (ties up)
    assert L.orc_round(1.0 + 2 ** -8, orc.ORC_BF16) == 1.0
    assert L.orc_round(1.0 + 3 * 2 ** -8, orc.ORC_BF16) == 1.0 + 2 ** -6
    # fp16 RNE, subnormal and overflow edges.
    assert L.orc_round(1.0 + 2 ** -11, orc.ORC_F16) == 1.0
    assert L.orc_round(2 ** -25 * 3, orc.ORC_F16) == 2 ** -24 * 2
    assert L.orc_round(65520.0, orc.ORC_F16) == float("inf")
    assert L.orc_round(65519.0, orc.ORC_F16) == 65504.0
    vals = np.array([0.1, -2.7, 1e-6, 3.3e4, 7.77e-5], np.float32)
    ref = torch.tensor(vals).to(torch.float16).float().numpy()
    assert [L.orc_round(float(v), orc.ORC_F16) for v in vals] == list(ref)
    ref = torch.tensor(vals).to(torch.bfloat16).float().numpy()
    assert [L.orc_round(float(v), orc.ORC_BF16) for v in vals] == list(ref)


# -------------------------------------------------------------------- gap ----

def test_gap_closed_form():
    g = orc.gap_from_threshold(0.8, 1, 2)
    assert g.dtype == np.float32 and np.all(g == np.float32(0.2231435477733612))
    g = orc.gap_from_threshold(0.9, 1, 1)
    assert g[0] == np.float32(0.10536051541566849)


def test_gap_tensor_branch_correctly_rounded():
    # spattn/src/VecAttention.py:50: gap = -torch.log(threshold + 1e-9) on an
    # fp32 tensor.  The oracle's per-head gaps are the correctly rounded fp32
    # values of that expression: the fp32 sum, then ln in fp64 rounded once.
    # Checked against an fp64 log of the sum computed with math.log (an
    # independent libm path) and against torch's fp32 evaluation of the
    # reference expression, which is faithful (within one unit in the last
    # place).  (B, H) and (H,) shapes broadcast as in the kernel.
    rng = np.random.default_rng(0)
    th = np.concatenate([rng.random(4000), np.geomspace(1e-7, 1.0, 4000)]).astype(np.float32)
    th = th.reshape(-1, 8)
    g = orc.gap_from_threshold(th, th.shape[0], 8).reshape(th.shape)
    s = (th + np.float32(1e-9)).astype(np.float32)
    want = np.array([[np.float32(-math.log(float(x))) for x in row] for row in s], np.float32)
    assert g.dtype == np.float32 and np.array_equal(g, want)
    torch32 = (-torch.log(torch.from_numpy(th) + 1e-9)).numpy()
    ulp = np.abs(g.view(np.int32).astype(np.int64) - torch32.view(np.int32).astype(np.int64))
    assert ulp.max() <= 1
    g1 = orc.gap_from_threshold(th[0], 3, 8).reshape(3, 8)
    assert np.array_equal(g1, np.broadcast_to(want[0], (3, 8)))


# -------------------------------------------------------- selection KATs ----

def _select_scores(scores, gap, bk, group, causal=False, wo_init=False, qps=64, J0=0, bsq=64,
                   nc=None):
    """Run the oracle on rows whose scores against every key are given by hand:
    qs = e_0, k[c, 0] = scores[row][c] is impossible for several rows, so each
    row r gets its own feature: qs[r] = e_r, k[c, r] = scores[r][c]."""
    scores = np.asarray(scores, np.float32)
    R, Sk = scores.shape
    D = max(R, 2)
    nc = nc or R
    qs = np.zeros((1, 1, J0 + nc, D), np.float32)
    for r in range(nc):
        qs[0, 0, J0 + r, r % R] = 1.0
    k = np.zeros((1, 1, Sk, D), np.float32)
    k[0, 0, :, :R] = scores.T
    gaps = np.full(1, gap, np.float32)
    counts, lists = orc.select(qs, k, J0, nc, gaps, qps, bk, group, causal, wo_init, bsq)
    return [list(map(int, lists[0][0][jr])) for jr in range(nc)]


def test_kat_prefix_max_updated_before_compare():
    # One group of 4 tiles.  tile0: 1.0 except key 3 = 2.0; tile1: 1.5 except
    # key 20 = 5.0; tile2: -1; tile3: -1 except key 60 = 2.5; gap 1.
    s = np.full(64, -1.0, np.float32)
    s[:16] = 1.0
    s[3] = 2.0
    s[16:32] = 1.5
    s[20] = 5.0
    s[60] = 2.5
    got = _select_scores([s], 1.0, 16, 4)[0]
    # tile0: m=2 -> all 16; tile1: m=5 -> only key 20; tiles 2,3: m=5 -> none.
    # (A maximum updated after the compare would also take the 1.5s of tile1;
    # a row-global maximum would take nothing from tile0.)
    assert got == list(range(16)) + [20]


def test_kat_group_restarts_running_max():
    s = np.full(64, -1.0, np.float32)
    s[:16] = 1.0
    s[3] = 2.0
    s[16:32] = 1.5
    s[20] = 5.0
    s[60] = 2.5
    got = _select_scores([s], 1.0, 16, 1)[0]
    # Every tile is its own group: tile1 -> {20}; tile2 -> all (m=-1); tile3 -> {60}.
    assert got == list(range(16)) + [20] + list(range(32, 48)) + [60]
    got = _select_scores([s], 1.0, 16, 2)[0]
    # Groups {0,1}, {2,3}: tile2 m=-1 -> all; tile3 m=2.5 -> {60}.
    assert got == list(range(16)) + [20] + list(range(32, 48)) + [60]


def test_kat_ties_select_at_equality():
    s = np.zeros(32, np.float32)
    s[5] = 1.0
    s[7] = 1.0
    got = _select_scores([s], 0.0, 16, 2)[0]
    assert got == [5, 7]


def test_kat_key_tail_not_multiple_of_tile():
    s = np.zeros(40, np.float32)
    s[39] = 3.0
    got = _select_scores([s], 1.0, 16, 16)[0]
    assert got == list(range(32)) + [39]


def test_kat_causal_first_row_tile_rule():
    # All scores equal, gap 0.5: every allowed key is selected.  qps=64, BK=16,
    # BLOCK_SIZE_Q=4, rows J0..J0+7.  Allowed keys: [64, J*64), except the first
    # row of each 4-row program (J - J0 = 0, 4), which stops at (J-1)*64 + 16.
    Sk = 1024
    s = np.zeros((1, Sk), np.float32)
    for J0 in (0, 8):
        got = _select_scores(np.repeat(s, 8, 0), 0.5, 16, 1024, causal=True, wo_init=True,
                             qps=64, J0=J0, bsq=4, nc=8)
        for jr in range(8):
            J = J0 + jr
            if jr % 4 == 0:
                want = list(range(64, max(64, (J - 1) * 64 + 16)))
            else:
                want = list(range(64, max(64, J * 64)))
            assert got[jr] == want, (J0, jr)


def test_selectable_count_closed_form_large_gap():
    # gap = 1e6 selects every selectable key: non-causal S_k per row; causal
    # (J-1)*qps, minus 48 on the first row of each BLOCK_SIZE_Q program (J>=2).
    g = torch.Generator().manual_seed(0)
    S, qps, bk, bsq = 1024, 64, 16, 4
    q = torch.randn(1, 2, S, 32, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 2, S, 32, generator=g).to(torch.bfloat16)
    _, qs = orc.pool(q, qps, "bfloat16")
    gaps = np.full(2, 1e6, np.float32)
    counts, _ = orc.select(qs, k, 0, 16, gaps, qps, bk, 16, False, False, bsq)
    assert np.all(counts == S)
    counts, lists = orc.select(qs, k, 0, 16, gaps, qps, bk, 16, True, True, bsq)
    for J in range(16):
        want = max(0, (J - 1) * qps) - (48 if (J % bsq == 0 and J >= 2) else 0)
        assert np.all(counts[:, :, J] == want), J


# ------------------------------------------------------------- invariants ----

def _random_select(seed, causal, gap, group, S=512, qps=64, bk=16, J0=0, nc=None, bsq=64, Hq=2, Hk=1):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, Hq, S, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(1, Hk, S, 64, generator=g)
    k[:, :, torch.randperm(S, generator=g)[:S // 20]] += 2.0
    k = k.to(torch.bfloat16)
    _, qs = orc.pool(q, qps, "bfloat16")
    nc = nc or math.ceil(S / qps) - J0
    gaps = np.full(Hq, gap, np.float32)
    return orc.select(qs, k, J0, nc, gaps, qps, bk, group, causal, causal, bsq)


@pytest.mark.parametrize("causal", [False, True])
def test_larger_gap_gives_superset(causal):
    _, small = _random_select(1, causal, 0.3, 4)
    _, large = _random_select(1, causal, 0.6, 4)
    for h in range(2):
        for a, b in zip(small[0][h], large[0][h]):
            assert set(a.tolist()) <= set(b.tolist())


def test_chunked_rows_equal_whole():
    _, whole = _random_select(2, False, 0.4, 8, S=1024)
    _, part = _random_select(2, False, 0.4, 8, S=1024, J0=5, nc=7)
    for h in range(2):
        for jr in range(7):
            assert np.array_equal(whole[0][h][5 + jr], part[0][h][jr])


def test_group_covering_all_keys_is_single_group():
    _, a = _random_select(3, False, 0.5, 64, S=1024)       # 64*16 = 1024 keys
    _, b = _random_select(3, False, 0.5, 100000, S=1024)
    for h in range(2):
        for x, y in zip(a[0][h], b[0][h]):
            assert np.array_equal(x, y)


def test_block_size_q_only_moves_first_row_rule():
    _, a = _random_select(4, True, 0.5, 16, S=2048, bsq=4)
    _, b = _random_select(4, True, 0.5, 16, S=2048, bsq=8)
    for h in range(2):
        for J in range(32):
            if J % 4 != 0:  # not a first row under either tiling
                assert np.array_equal(a[0][h][J], b[0][h][J]), J


def test_gqa_head_mapping():
    # q heads 0..3 share kv head 0, heads 4..7 kv head 1 (repeat_interleave).
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, 8, 256, 32, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 2, 256, 32, generator=g).to(torch.bfloat16)
    _, qs = orc.pool(q, 64, "bfloat16")
    gaps = np.full(8, 0.5, np.float32)
    c1, l1 = orc.select(qs, k, 0, 4, gaps, 64, 16, 4, False, False, 64)
    krep = k.repeat_interleave(4, dim=1)
    c2, l2 = orc.select(qs, krep, 0, 4, gaps, 64, 16, 4, False, False, 64)
    assert np.array_equal(c1, c2)


# -------------------------------------------------------------- attention ----

def test_local_blocks_closed_form():
    cnt, idx = orc.local_blocks(1, 1, 200, 64, True)
    assert cnt[0, 0].tolist() == [1, 2, 2, 2]
    assert idx[0, 0].tolist() == [[0, 0], [0, 64], [0, 128], [0, 192]]
    cnt, idx = orc.local_blocks(1, 1, 300, 128, True)
    assert cnt[0, 0].tolist() == [2, 4, 3]
    assert idx[0, 0, 2].tolist() == [0, 64, 256, 320]


def test_attention_all_keys_equals_dense_sdpa():
    g = torch.Generator().manual_seed(6)
    B, H, S, D = 1, 2, 300, 32
    # The oracle takes float32 values; SDPA runs on the same values in float64.
    q = torch.randn(B, H, S, D, generator=g).double()
    k = torch.randn(B, H, S, D, generator=g).double()
    v = torch.randn(B, H, S, D, generator=g).double()
    cnt, idx = orc.local_blocks(B, H, S, 64, False)
    lists = [[[np.arange(S)] * 5 for _ in range(H)]]
    out = orc.attention(q.numpy(), k.numpy(), v.numpy(), 64, False, cnt, idx, lists)
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v).numpy()
    assert np.max(np.abs(out - ref)) < 1e-12


def test_attention_causal_large_gap_is_dense_causal_minus_first_row_rule():
    g = torch.Generator().manual_seed(7)
    B, H, S, D, qps = 1, 1, 640, 32, 64
    q = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    out, _ = orc.prefill(q, k, v, 1e-300, q_pooling_size=qps, k_local_size=16, group_k_block=16,
                         causal=True, chunk_size=256, bsq=4)
    # threshold 1e-300 -> gap = -ln(1e-9) ~ 20.7: every selectable key.  The
    # first row of each BLOCK_SIZE_Q program loses keys [(J-1)*64+16, J*64)
    # (programs restart at chunk starts: 256/64 = 4 rows per chunk).
    mask = torch.ones(S, S, dtype=torch.bool).tril()
    for J in range(S // qps):
        if (J % 4) == 0 and J >= 2:
            mask[J * qps:(J + 1) * qps, (J - 1) * qps + 16:J * qps] = False
    ref = torch.nn.functional.scaled_dot_product_attention(
        q.double(), k.double(), v.double(), attn_mask=mask).numpy()
    assert np.max(np.abs(out - ref)) < 1e-10


def test_attention_uniform_values_closed_form():
    B, H, S, D = 1, 1, 256, 16
    g = torch.Generator().manual_seed(8)
    q = torch.randn(B, H, S, D, generator=g)
    k = torch.randn(B, H, S, D, generator=g)
    v = torch.ones(B, H, S, D) * torch.arange(D)
    out, _ = orc.prefill(q, k, v, 0.5, q_pooling_size=64, k_local_size=16, group_k_block=4,
                         causal=False, chunk_size=128, dtype="float32")
    assert np.allclose(out, np.arange(D)[None, None, None, :], atol=1e-12)


def test_attention_empty_key_set_is_zero():
    B, H, S, D = 1, 1, 64, 8
    q = np.ones((B, H, S, D), np.float32)
    cnt, idx = orc.local_blocks(B, H, S, 64, False)
    out = orc.attention(q, q, q, 64, False, cnt, idx, [[[np.zeros(0, np.int64)]]])
    assert np.all(out == 0)


# ---- decode (flashinfer single_decode_with_kv_cache semantics) ----

@pytest.mark.parametrize("layout", ["NHD", "HND"])
def test_decode_matches_sdpa_float64(layout):
    """Against torch's SDPA in float64 with the kv heads expanded
    (repeat_interleave, the repeat_kv convention) and one query row per head."""
    import torch
    g = torch.Generator().manual_seed(5)
    Hq, Hk, L, D = 8, 2, 77, 32
    q = torch.randn(Hq, D, generator=g).double()  # fp32 values: the oracle reads fp32
    k = torch.randn(Hk, L, D, generator=g).double()
    v = torch.randn(Hk, L, D, generator=g).double()
    kk = k.repeat_interleave(Hq // Hk, dim=0)
    vv = v.repeat_interleave(Hq // Hk, dim=0)
    want = torch.nn.functional.scaled_dot_product_attention(
        q[:, None, :], kk, vv, scale=0.3)[:, 0, :].numpy()
    kl, vl = (k.transpose(0, 1), v.transpose(0, 1)) if layout == "NHD" else (k, v)
    got = orc.decode(q.numpy(), kl.numpy(), vl.numpy(), layout, sm_scale=0.3)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_decode_closed_forms():
    """One key: the output is that key's value row.  Equal keys: the mean of
    the value rows."""
    rng = np.random.default_rng(6)
    f32 = lambda *shape: rng.standard_normal(shape).astype(np.float32)  # noqa: E731
    q = f32(4, 16)
    v1 = f32(1, 2, 16)
    k1 = f32(1, 2, 16)
    out = orc.decode(q, k1, v1, "NHD")
    np.testing.assert_allclose(out, np.repeat(v1[0], 2, axis=0), rtol=1e-12)
    kq = np.repeat(f32(1, 1, 16), 9, axis=0)
    vq = f32(9, 1, 16)
    out = orc.decode(q, kq, vq, "NHD")
    np.testing.assert_allclose(out, np.repeat(vq[:, 0].astype(np.float64).mean(0, keepdims=True),
                                              4, axis=0), rtol=1e-12)
