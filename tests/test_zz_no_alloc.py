"""The allocation-free decode entry point (va_decode_attn_noalloc) against
va_decode_attn, through the C ABI, on an MI355X.

Both run the same kernels, so the outputs must be identical bit for bit (and
therefore within the decode tolerance of the float64 oracle, checked once).
Two calls in a row share the library's device array: the second, with a
smaller cache and fewer heads, must not see anything of the first.  Sizes
beyond the array are rejected on the host before any launch.
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from vecattention_amd import _native as nat

pytestmark = pytest.mark.gpu


def _case(Hq, Hk, L, D, seed, dtype=torch.bfloat16, dev="cuda:0"):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(Hq, D, generator=g).to(dtype).to(dev)
    k = torch.randn(L, Hk, D, generator=g).to(dtype).to(dev)   # NHD
    v = torch.randn(L, Hk, D, generator=g).to(dtype).to(dev)
    return q, k, v


def _noalloc(q, k, v, out, kernel=nat.VA_ATTN_AUTO):
    L, Hk, D = k.shape
    Hq = q.shape[0]
    return nat.lib().va_decode_attn_noalloc(
        nat.dtype_code(q), nat.ptr(q), q.stride(0), nat.ptr(k), k.stride(1), k.stride(0),
        nat.ptr(v), v.stride(1), v.stride(0), nat.ptr(out), out.stride(0), Hq, Hk, L, D,
        1.0 / math.sqrt(D), kernel, nat.stream_ptr(q.device))


def _with_workspace(q, k, v, out, kernel=nat.VA_ATTN_AUTO):
    L, Hk, D = k.shape
    Hq = q.shape[0]
    ws = int(nat.lib().va_decode_workspace_size(Hq, Hk, L, D))
    work = torch.empty(max(ws, 16), dtype=torch.uint8, device=q.device)
    rc = nat.lib().va_decode_attn(
        nat.dtype_code(q), nat.ptr(q), q.stride(0), nat.ptr(k), k.stride(1), k.stride(0),
        nat.ptr(v), v.stride(1), v.stride(0), nat.ptr(out), out.stride(0), Hq, Hk, L, D,
        1.0 / math.sqrt(D), kernel, nat.ptr(work), work.numel(), nat.stream_ptr(q.device))
    nat.check("va_decode_attn", rc)
    return out


def test_noalloc_decode_equals_workspace_decode_twice(device):
    # First call: Qwen2.5-VL heads over a 50000-token cache (many key spans);
    # second call, right after on the same stream: fewer heads and a short
    # cache, so fewer partial states than the first call left in the array.
    for (Hq, Hk, L, D, seed) in [(28, 4, 50000, 128, 0), (8, 2, 3000, 64, 1)]:
        print(f"[case] noalloc decode Hq={Hq} Hk={Hk} L={L} D={D}", flush=True)
        need = int(nat.lib().va_decode_workspace_size(Hq, Hk, L, D))
        assert 0 < need <= int(nat.lib().va_decode_noalloc_scratch_bytes())
        q, k, v = _case(Hq, Hk, L, D, seed)
        got = torch.full((Hq, D), float("nan"), dtype=q.dtype, device=q.device)
        nat.check("va_decode_attn_noalloc", _noalloc(q, k, v, got))
        want = _with_workspace(q, k, v, torch.empty_like(got))
        torch.cuda.synchronize()
        assert torch.equal(got, want), (Hq, L)
        ref = orc.decode(q.float().cpu(), k.float().cpu(), v.float().cpu(), "NHD")
        err = np.abs(got.float().cpu().numpy() - ref)
        assert err.max() <= 2e-2 and err.mean() <= 2e-3


def test_noalloc_decode_rejects_sizes_beyond_its_array(device):
    # 64 q heads over one kv head and a long cache need more partial states
    # than the array holds: rejected before any launch, nothing written.  K/V
    # have their full size (256 MiB each), so that if the size check ever
    # regressed the launch would read in bounds and fail the assertions below
    # instead of reading past the allocation.
    Hq, Hk, L, D = 64, 1, 1 << 20, 128
    need = int(nat.lib().va_decode_workspace_size(Hq, Hk, L, D))
    assert need > int(nat.lib().va_decode_noalloc_scratch_bytes())
    q = torch.zeros(Hq, D, dtype=torch.bfloat16, device=device)
    kv = torch.zeros(L, Hk, D, dtype=torch.bfloat16, device=device)  # NHD, never read
    out = torch.full((Hq, D), 7.0, dtype=torch.bfloat16, device=device)
    rc = nat.lib().va_decode_attn_noalloc(
        nat.VA_BF16, nat.ptr(q), q.stride(0), nat.ptr(kv), kv.stride(1), kv.stride(0),
        nat.ptr(kv), kv.stride(1), kv.stride(0), nat.ptr(out), out.stride(0), Hq, Hk, L, D,
        1.0 / math.sqrt(D), nat.VA_ATTN_AUTO, nat.stream_ptr(q.device))
    assert rc == nat.VA_ERR_UNSUPPORTED
    assert b"at most" in nat.lib().va_last_error()
    torch.cuda.synchronize()
    assert torch.all(out == 7.0)


def test_noalloc_decode_per_row_kernel(device):
    # fp32 runs the per-row kernel, which needs no partial states
    Hq, Hk, L, D = 8, 2, 777, 128
    q, k, v = _case(Hq, Hk, L, D, 3, dtype=torch.float32)
    got = torch.empty(Hq, D, dtype=q.dtype, device=q.device)
    nat.check("va_decode_attn_noalloc", _noalloc(q, k, v, got))
    want = _with_workspace(q, k, v, torch.empty_like(got))
    torch.cuda.synchronize()
    assert torch.equal(got, want)
