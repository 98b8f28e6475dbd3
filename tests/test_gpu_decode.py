"""GPU parity of decode attention (single_decode_with_kv_cache ->
va_decode_attn) against the float64 oracle (run on an MI355X).
Tolerance: max-abs 2e-2, mean-abs 2e-3 for bf16/fp16 inputs (as the prefill
attention), 1e-4 for fp32 (the per-row kernel)."""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from vecattention_amd import _native as nat
from vecattention_amd.decode import single_decode_with_kv_cache

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def note(*a):
    print("[case]", *a, flush=True)


def _kv(layout, Hk, L, D, dtype, g):
    shape = (L, Hk, D) if layout == "NHD" else (Hk, L, D)
    k = torch.randn(*shape, generator=g)
    v = torch.randn(*shape, generator=g)
    return k.to(dtype), v.to(dtype)


def _check(out, want, dtype):
    err = np.abs(out.float().cpu().numpy() - want)
    if dtype == torch.float32:
        assert err.max() <= 1e-4, err.max()
    else:
        assert err.max() <= 2e-2 and err.mean() <= 2e-3, (err.max(), err.mean())


@pytest.mark.parametrize("layout", ["NHD", "HND"])
@pytest.mark.parametrize("Hq,Hk,L,D", [(28, 4, 5000, 128), (28, 28, 777, 128), (8, 2, 64, 64),
                                       (12, 12, 33, 128), (16, 1, 70001, 64), (4, 4, 1, 128)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_decode_matches_oracle(layout, Hq, Hk, L, D, dtype):
    note("decode", layout, Hq, Hk, L, D, dtype)
    g = torch.Generator().manual_seed(L + Hq)
    q = torch.randn(Hq, D, generator=g).to(dtype)
    k, v = _kv(layout, Hk, L, D, dtype, g)
    out = single_decode_with_kv_cache(q.to(DEV), k.to(DEV), v.to(DEV), kv_layout=layout)
    torch.cuda.synchronize()
    assert out.dtype == dtype and tuple(out.shape) == (Hq, D)
    _check(out, orc.decode(q.float(), k.float(), v.float(), layout), dtype)


def test_decode_peaked_and_scaled():
    """A few keys carry most of the mass (scores far apart) across split
    boundaries, and a custom sm_scale."""
    note("decode peaked")
    g = torch.Generator().manual_seed(3)
    Hq, Hk, L, D = 14, 2, 9000, 128
    q = torch.randn(Hq, D, generator=g)
    k = torch.randn(L, Hk, D, generator=g)
    for pos in (5, 4097, 8999):
        k[pos] = q.view(Hk, Hq // Hk, D).mean(1) * 4.0
    v = torch.randn(L, Hk, D, generator=g)
    q, k, v = q.bfloat16(), k.bfloat16(), v.bfloat16()
    out = single_decode_with_kv_cache(q.to(DEV), k.to(DEV), v.to(DEV), sm_scale=0.2)
    torch.cuda.synchronize()
    _check(out, orc.decode(q.float(), k.float(), v.float(), "NHD", sm_scale=0.2), torch.bfloat16)


def test_decode_fp32_per_row_kernel():
    note("decode fp32")
    g = torch.Generator().manual_seed(4)
    q = torch.randn(8, 64, generator=g)
    k, v = _kv("HND", 2, 1500, 64, torch.float32, g)
    out = single_decode_with_kv_cache(q.to(DEV), k.to(DEV), v.to(DEV), kv_layout="HND")
    torch.cuda.synchronize()
    _check(out, orc.decode(q, k, v, "HND"), torch.float32)


def test_decode_strided_cache_views():
    """K/V as views into a larger cache (token stride past the live heads), as
    a paged or preallocated cache hands them over."""
    note("decode strided")
    g = torch.Generator().manual_seed(5)
    Hq, Hk, L, D, cap = 28, 4, 3000, 128, 4096
    kc = torch.randn(cap, Hk + 2, D, generator=g).bfloat16()
    vc = torch.randn(cap, Hk + 2, D, generator=g).bfloat16()
    q = torch.randn(Hq, D, generator=g).bfloat16()
    kd, vd = kc.to(DEV), vc.to(DEV)
    out = single_decode_with_kv_cache(q.to(DEV), kd[:L, 1:1 + Hk], vd[:L, 1:1 + Hk])
    torch.cuda.synchronize()
    _check(out, orc.decode(q.float(), kc[:L, 1:1 + Hk].float(), vc[:L, 1:1 + Hk].float(), "NHD"),
           torch.bfloat16)


def test_decode_mfma_equals_per_row_kernel():
    """The split MFMA path and the per-row kernel agree (independent code)."""
    note("decode mfma vs simple")
    g = torch.Generator().manual_seed(6)
    Hq, Hk, L, D = 28, 4, 20000, 128
    q = torch.randn(Hq, D, generator=g).bfloat16().to(DEV)
    k = torch.randn(L, Hk, D, generator=g).bfloat16().to(DEV)
    v = torch.randn(L, Hk, D, generator=g).bfloat16().to(DEV)
    L_ = nat.lib()
    outs = []
    for kernel in (nat.VA_ATTN_MFMA, nat.VA_ATTN_SIMPLE):
        out = torch.empty(Hq, D, dtype=torch.bfloat16, device=DEV)
        ws = torch.empty(int(L_.va_decode_workspace_size(Hq, Hk, L, D)), dtype=torch.uint8,
                         device=DEV)
        rc = L_.va_decode_attn(nat.VA_BF16, nat.ptr(q), q.stride(0), nat.ptr(k), k.stride(1),
                               k.stride(0), nat.ptr(v), v.stride(1), v.stride(0), nat.ptr(out),
                               out.stride(0), Hq, Hk, L, D, 1.0 / math.sqrt(D), kernel,
                               nat.ptr(ws), ws.numel(), nat.stream_ptr(q.device))
        nat.check("va_decode_attn", rc)
        outs.append(out.float())
    torch.cuda.synchronize()
    d = (outs[0] - outs[1]).abs()
    assert float(d.max()) <= 1e-2 and float(d.mean()) <= 1e-3
