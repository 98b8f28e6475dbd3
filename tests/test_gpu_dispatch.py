"""GPU parity of the caller glue: dense prefill (va_dense_attn, the reference's
Full_prefill), the dispatcher's vision-span slicing, and the DiT call with
Sq != Sk and per-head thresholds, against the CPU oracle (run on an MI355X).
Tolerance: max-abs 2e-2, mean-abs 2e-3 (bf16/fp16 inputs)."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from vecattention_amd import (FastPrefillConfig, Full_prefill, VecAttention_prefill,
                              customize_prefill_attention)
from vecattention_amd.synth import make_inputs

pytestmark = pytest.mark.gpu

ATOL_MAX, ATOL_MEAN = 2e-2, 2e-3
DTN = {torch.bfloat16: "bfloat16", torch.float16: "float16"}


def note(*a):
    print("[case]", *a, flush=True)


def dense_oracle(q, k, v, causal, qps=64):
    """Every key for every q-block (the oracle's masked attention with all
    columns selected); causal alignment is bottom-right."""
    B, Hq, Sq, _ = q.shape
    Sk = k.shape[2]
    nqb = -(-Sq // qps)
    allk = np.arange(Sk, dtype=np.int64)
    lists = [[[allk for _ in range(nqb)] for _ in range(Hq)] for _ in range(B)]
    zc = np.zeros((B, Hq, nqb), np.int64)
    zi = np.zeros((B, Hq, nqb, 0), np.int64)
    return orc.attention(q, k, v, qps, causal, zc, zi, lists)


def check(out, want):
    err = np.abs(out.float().cpu().numpy() - want)
    tol = (1e-4, 1e-5) if out.dtype == torch.float32 else (ATOL_MAX, ATOL_MEAN)
    assert err.max() <= tol[0] and err.mean() <= tol[1], (err.max(), err.mean())


DENSE_CASES = [
    # name, B, Hq, Hk, Sq, Sk, D, dtype, causal
    ("causal-square-gqa", 1, 4, 2, 1000, 1000, 128, torch.bfloat16, True),
    ("causal-bottom-right", 1, 2, 2, 300, 1000, 64, torch.float16, True),
    ("causal-one-row", 2, 2, 1, 1, 777, 128, torch.bfloat16, True),
    ("noncausal-sq-lt-sk", 1, 3, 3, 500, 1200, 128, torch.bfloat16, False),
    ("noncausal-ragged", 2, 2, 2, 197, 197, 64, torch.float16, False),
    # fp32 on the fp32 matrix-core kernel
    ("fp32-causal-bottom-right-gqa", 1, 4, 2, 300, 1000, 64, torch.float32, True),
    ("fp32-noncausal-ragged-d128", 2, 2, 2, 197, 450, 128, torch.float32, False),
]


@pytest.mark.parametrize("case", DENSE_CASES, ids=[c[0] for c in DENSE_CASES])
def test_full_prefill_matches_oracle(device, case):
    name, B, Hq, Hk, Sq, Sk, D, dtype, causal = case
    note("dense", name)
    q, _, _ = make_inputs(B, Hq, Hk, Sq, D, dtype, seed=11)
    _, k, v = make_inputs(B, Hq, Hk, Sk, D, dtype, seed=12)
    out = Full_prefill(q.to(device), k.to(device), v.to(device), causal=causal)
    torch.cuda.synchronize()
    assert out.shape == q.shape and out.dtype == dtype
    check(out, dense_oracle(q, k, v, causal))


def test_full_prefill_rejects_causal_sq_gt_sk(device):
    q = torch.zeros(1, 2, 100, 64, dtype=torch.bfloat16, device=device)
    k = torch.zeros(1, 2, 50, 64, dtype=torch.bfloat16, device=device)
    with pytest.raises(AssertionError):
        Full_prefill(q, k, k, causal=True)


class _Layer:
    def __init__(self, idx):
        self.layer_idx = idx


def test_dispatcher_vision_span(device):
    # Text before the vision span and after it in dense attention, the span
    # [0, vision_end) in VecAttention (spattn/src/models/utils.py:99-128).
    note("dispatch vision span")
    B, Hq, Hk, S, D, dt = 1, 4, 2, 1500, 128, torch.bfloat16
    vs, ve, th = 200, 1300, 0.5
    q, k, v = make_inputs(B, Hq, Hk, S, D, dt, seed=13)
    cfg = FastPrefillConfig(metric="vecattention", threshold=th, block_size_q=64, block_size_k=16,
                            group_k_block=16, chunk_size=1024, vision_start_position=vs,
                            vision_end_position=ve)
    out = customize_prefill_attention(_Layer(3), q.to(device), k.to(device), v.to(device),
                                      causal=True, config=cfg)
    torch.cuda.synchronize()
    assert out.shape == (B, Hq, S, D)
    span, _ = orc.prefill(q[:, :, :ve], k[:, :, :ve], v[:, :, :ve], th, 64, 16, 16, True, 1024, 64,
                          "bfloat16")
    want = np.zeros((B, Hq, S, D))
    want[:, :, :ve] = span
    want[:, :, :vs] = dense_oracle(q[:, :, :vs], k[:, :, :vs], v[:, :, :vs], True)
    want[:, :, ve:] = dense_oracle(q[:, :, ve:], k, v, True)
    check(out, want)


def test_dispatcher_layer_threshold_and_full_metric(device):
    note("dispatch layer threshold")
    B, H, S, D, dt = 1, 4, 1024, 128, torch.bfloat16
    q, k, v = make_inputs(B, H, H, S, D, dt, seed=14)
    thr = torch.tensor([[0.9, 0.9, 0.9, 0.9], [0.9, 0.5, 0.1, 0.01]], device=device)
    cfg = FastPrefillConfig(metric="vecattention", threshold=thr, block_size_q=64, block_size_k=16,
                            group_k_block=8192, chunk_size=512)
    out = customize_prefill_attention(_Layer(1), q.to(device), k.to(device), v.to(device),
                                      causal=False, config=cfg)
    want, _ = orc.prefill(q, k, v, thr[1].cpu().numpy(), 64, 16, 8192, False, 512, 64, "bfloat16")
    check(out, want)
    full = customize_prefill_attention(_Layer(0), q.to(device), k.to(device), v.to(device),
                                       causal=False, config=FastPrefillConfig(metric="full"))
    check(full, dense_oracle(q, k, v, False))


def test_dit_image_queries_over_image_and_text_keys(device):
    # The Hunyuan call (hyvideo/attention.py:1030-1042): non-causal VecAttention
    # of the image queries over image + text keys (Sq < Sk), per-head thresholds.
    note("dit sq<sk")
    B, H, D, img, txt = 1, 3, 128, 1100, 157
    q, _, _ = make_inputs(B, H, H, img, D, torch.bfloat16, seed=15)
    _, k, v = make_inputs(B, H, H, img + txt, D, torch.bfloat16, seed=16)
    th = torch.tensor([0.6, 0.3, 0.05])
    out = VecAttention_prefill(q.to(device), k.to(device), v.to(device), th.to(device), 64, 16, 8192,
                               False, 512)
    want, _ = orc.prefill(q, k, v, th.numpy(), 64, 16, 8192, False, 512, 64, "bfloat16")
    check(out, want)
