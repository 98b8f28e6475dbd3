"""The MFMA accumulation error the certified selection kernel relies on.

select_mfma.hip takes decisions on MFMA scores outside a band built from
|s_mfma - s| <= 2*(D/16 + 2) * 2^-23 * sum_d |q_d k_d|.  This test runs chains
of v_mfma_f32_32x32x16 (bf16 and fp16) on random and adversarial operands —
wide exponent spreads, large accumulators, exact cancellation — and checks the
error against exact sums (math.fsum) with half of that allowance, so a change
of the hardware's accumulation behaviour fails here before it can flip a
selection decision.
"""
import ctypes
import math
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "numerics", "libmfmaprobe.so")


@pytest.fixture(scope="module")
def probe(device):
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} missing: run __graft_entry__.build()")
    lib = ctypes.CDLL(LIB)
    lib.mfma_chain_run.restype = ctypes.c_int
    return lib


def _bits(x, f16):
    t = torch.as_tensor(x, dtype=torch.float32).to(torch.float16 if f16 else torch.bfloat16)
    return t.view(torch.int16), t.float().numpy()


def _run(lib, a, b, acc0, f16):
    steps = a.shape[0]
    ab, av = _bits(a.reshape(-1), f16)
    bb, bv = _bits(b.reshape(-1), f16)
    dev = torch.device("cuda:0")
    A, Bt = ab.to(dev), bb.to(dev)
    C0 = torch.as_tensor(acc0, dtype=torch.float32).to(dev)
    C = torch.zeros(32, 32, dtype=torch.float32, device=dev)
    rc = lib.mfma_chain_run(int(f16), ctypes.c_void_p(A.data_ptr()), ctypes.c_void_p(Bt.data_ptr()),
                            ctypes.c_void_p(C0.data_ptr()), ctypes.c_void_p(C.data_ptr()), steps)
    assert rc == 0
    return C.cpu().numpy().astype(np.float64), av.reshape(steps, 32, 16).astype(np.float64), \
        bv.reshape(steps, 16, 32).astype(np.float64)


def _check(lib, a, b, acc0, f16, allow_units):
    c, A, B = _run(lib, a, b, acc0, f16)
    acc0 = np.asarray(acc0, np.float32).astype(np.float64)
    worst = 0.0
    for m in range(32):
        for n in range(32):
            terms = (A[:, m, :] * B[:, :, n]).reshape(-1)  # exact products
            exact = math.fsum(list(terms) + [acc0[m, n]])
            scale = math.fsum(np.abs(terms)) + abs(acc0[m, n])
            if scale == 0:
                assert c[m, n] == 0
                continue
            worst = max(worst, abs(c[m, n] - exact) / (scale * 2.0 ** -24))
    assert worst <= allow_units, worst
    return worst


CASES = ["normal", "wide_exponents", "large_accumulator", "cancellation"]


@pytest.mark.parametrize("f16", [False, True], ids=["bf16", "f16"])
@pytest.mark.parametrize("case", CASES)
def test_mfma_error_within_selection_bound(probe, case, f16):
    rng = np.random.default_rng(CASES.index(case) + 10 * f16)
    steps = 8                                   # D = 128
    allow = 2 * (steps + 2) / 2                 # half the kernel's 2*(D/16+2) ulps (units 2^-23)
    allow_units = allow * 2                     # in units of 2^-24
    a = rng.standard_normal((steps, 32, 16))
    b = rng.standard_normal((steps, 16, 32))
    acc0 = np.zeros((32, 32))
    spread = 6 if f16 else 20                   # keep fp16 operands in range
    if case == "wide_exponents":
        a *= 2.0 ** rng.integers(-spread, spread, a.shape)
        b *= 2.0 ** rng.integers(-spread, spread, b.shape)
    elif case == "large_accumulator":
        acc0 = rng.standard_normal((32, 32)) * 2.0 ** rng.integers(-10, 10, (32, 32))
    elif case == "cancellation":
        a[:, :, 1::2] = -a[:, :, 0::2]
        b[:, 1::2, :] = b[:, 0::2, :]
        a[:, :, 15] *= 2.0 ** -10
    print(f"[case] mfma numerics {case} {'f16' if f16 else 'bf16'}", flush=True)
    _check(probe, a, b, acc0, f16, allow_units)


def test_mfma_rounds_to_nearest_even(probe):
    # 1 + k*2^-23 plus exactly half an ulp: ties go to even.
    a = np.zeros((1, 32, 16))
    b = np.zeros((1, 16, 32))
    a[0, :, 0] = 2.0 ** -12
    b[0, 0, :] = 2.0 ** -12
    acc0 = 1.0 + (np.arange(32)[:, None] % 4) * 2.0 ** -23 + np.zeros((32, 32))
    c, _, _ = _run(probe, a, b, acc0, False)
    want = np.where(np.arange(32)[:, None] % 2 == 1, acc0 + 2.0 ** -23, acc0) + np.zeros((32, 32))
    assert np.array_equal(c, want.astype(np.float32).astype(np.float64))
