"""libvecattn.so on a machine without a GPU: it loads, exports every symbol
include/vecattn.h declares, answers its pure-host queries, and turns invalid
arguments into error codes before any device work."""
import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from vecattention_amd import _native as nat

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def L():
    if not os.path.exists(nat.LIB_PATH):
        from vecattention_amd import build
        build.build()
    return nat.lib()


def header_functions():
    text = open(os.path.join(ROOT, "include", "vecattn.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(va_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(L):
    names = header_functions()
    assert len(names) >= 9
    for name in names:
        assert hasattr(L, name), name
        assert name in nat.SIGNATURES, name
    assert sorted(nat.SIGNATURES) == names


def test_version_and_error_string(L):
    assert L.va_version() == 100
    assert isinstance(L.va_last_error(), bytes)


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-device path")
def test_no_device_is_an_error(L):
    rc = L.va_device_count()
    assert rc == nat.VA_ERR_HIP
    assert L.va_last_error()


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("wo_init", [False, True])
def test_index_layout_matches_capacities(L, causal, wo_init):
    B, Hq, Sk, qps = 2, 3, 1000, 64
    for J0, nc in [(0, 16), (5, 7), (3, 1)]:
        caps = [orc.row_capacity(J0 + jr, qps, Sk, causal, wo_init) for jr in range(nc)]
        total = L.va_select_index_capacity(B, Hq, Sk, qps, int(causal), int(wo_init), J0, nc, 0)
        assert total == B * Hq * sum(caps)
        off = [L.va_select_row_offset(Sk, qps, int(causal), int(wo_init), J0, nc, 0, bh, jr)
               for bh in range(B * Hq) for jr in range(nc)]
        want = np.concatenate([[0], np.cumsum(caps * (B * Hq))[:-1]])
        assert off == want.tolist()
    # dense rows
    assert L.va_select_row_offset(Sk, qps, 1, 1, 0, 4, 1008, 2, 3) == (2 * 4 + 3) * 1008


def _null_select(L, **over):
    args = dict(dtype=nat.VA_BF16, qs=256, sqb=0, sqh=0, sqn=0, k=256, skb=0, skh=0, sks=128, B=1, Hq=4,
                Hk=2, Sk=1024, D=128, qps=64, bk=16, G=16, causal=1, wo_init=1, J0=0, nc=16, bsq=64,
                gap=0.2, gaps=None, dense=0, counts=1, indices=1, kernel=0, scratch=None,
                scratch_floats=0, stream=None)
    args.update(over)
    return L.va_select(*args.values())


def test_select_argument_errors_before_launch(L):
    assert _null_select(L, bk=48) == nat.VA_ERR_UNSUPPORTED
    assert b"k_local_size" in L.va_last_error()
    assert _null_select(L, Hk=3) == nat.VA_ERR_ARG
    assert _null_select(L, qps=64, bk=128) == nat.VA_ERR_ARG   # the reference's causal assert
    assert _null_select(L, qps=64, bk=128, causal=0) == nat.VA_ERR_UNSUPPORTED  # wo_init tiling
    assert _null_select(L, dtype=7) == nat.VA_ERR_ARG
    assert _null_select(L, counts=None) == nat.VA_ERR_ARG
    assert _null_select(L, D=512) == nat.VA_ERR_UNSUPPORTED
    assert _null_select(L, kernel=nat.VA_SEL_MFMA) == nat.VA_ERR_ARG            # no scratch
    assert _null_select(L, kernel=nat.VA_SEL_MFMA, dtype=nat.VA_F32) == nat.VA_ERR_UNSUPPORTED
    assert _null_select(L, kernel=nat.VA_SEL_WAVE) == nat.VA_ERR_ARG            # no scratch
    assert _null_select(L, kernel=nat.VA_SEL_WAVE, G=5) == nat.VA_ERR_UNSUPPORTED  # span 80 keys
    assert _null_select(L, kernel=9) == nat.VA_ERR_ARG


def _null_csr(L, **over):
    args = dict(dtype=nat.VA_BF16, qs=256, sqb=0, sqh=0, sqn=0, k=256, skb=0, skh=0, sks=128, B=1,
                Hq=4, Hk=2, Sk=1024, D=128, qps=64, bk=16, G=16, causal=1, wo_init=1, J0=0, nc=16,
                bsq=64, gap=0.2, gaps=None, segk=0, counts=1, offsets=1, indices=None,
                scratch=None, scratch_floats=0, stream=None)
    args.update(over)
    return L.va_select_csr(*args.values())


def test_select_csr_argument_errors_before_launch(L):
    assert _null_csr(L, counts=None) == nat.VA_ERR_ARG
    assert _null_csr(L, offsets=None) == nat.VA_ERR_ARG
    assert _null_csr(L, segk=-64) == nat.VA_ERR_ARG
    assert _null_csr(L, Hk=3) == nat.VA_ERR_ARG
    assert _null_csr(L, bk=48) == nat.VA_ERR_UNSUPPORTED
    # split: segment length rules and scratch as va_select_segments
    assert _null_csr(L, segk=100) == nat.VA_ERR_ARG                 # not a multiple of 64
    assert _null_csr(L, segk=512) == nat.VA_ERR_ARG                 # no scratch
    assert b"scratch" in L.va_last_error()
    # the exact kernel (fp32) also takes the two-pass split (a group spans the
    # row), with its carry records in scratch
    assert _null_csr(L, dtype=nat.VA_F32, G=8192, segk=512) == nat.VA_ERR_ARG
    assert b"scratch" in L.va_last_error()
    assert _null_csr(L, dtype=nat.VA_F32, segk=320) == nat.VA_ERR_ARG  # not whole 256-key groups


def test_prefill_argument_errors_before_launch(L):
    f = L.va_prefill
    base = [nat.VA_BF16, 1, 0, 0, 128, 1, 0, 0, 128, 1, 0, 0, 128, 1, 0, 0, 128,
            1, 4, 2, 1024, 1024, 128, 0.2, None, 64, 16, 16, 1, 1000, 64, 1, 1 << 30, None]
    a = list(base)
    assert f(*a) == nat.VA_ERR_ARG            # chunk 1000 not a multiple of 64
    a = list(base); a[29] = 1024; a[25] = 96
    assert f(*a) == nat.VA_ERR_ARG            # q_pooling_size not 64/128
    a = list(base); a[29] = 1024; a[32] = 16
    assert f(*a) == nat.VA_ERR_WORKSPACE      # workspace too small
    a = list(base); a[29] = 1024; a[21] = 512
    assert f(*a) == nat.VA_ERR_UNSUPPORTED    # causal with Sq != Sk


def test_workspace_size_covers_largest_row_group(L):
    # causal 128K: the index buffer holds one row group of the last chunk at a
    # time (128 q-block rows, a multiple of BLOCK_SIZE_Q = 64, at most 2 GiB of
    # slots or one group), not the whole 32K chunk.
    B, Hq, S, D, qps, chunk = 1, 28, 131072, 128, 64, 32768
    qs_bytes = B * Hq * (S // qps) * D * 2
    ws = L.va_prefill_workspace_size(nat.VA_BF16, B, Hq, S, S, D, qps, 1, chunk, 64)
    whole = L.va_select_index_capacity(B, Hq, S, qps, 1, 1, (S - chunk) // qps, chunk // qps, 0)
    group = L.va_select_index_capacity(B, Hq, S, qps, 1, 1, S // qps - 128, 128, 0)
    assert group * 4 <= 2 << 30
    assert ws >= group * 4 + qs_bytes
    assert ws < whole * 4
    assert ws < 2 * 2 ** 30 + qs_bytes + (64 << 20)
    # non-causal chunks are not split: every row sees every key
    S2, H2 = 119056, 24
    ws2 = L.va_prefill_workspace_size(nat.VA_BF16, B, H2, S2, S2, D, qps, 0, chunk, 64)
    full = L.va_select_index_capacity(B, H2, S2, qps, 0, 0, 0, chunk // qps, 0)
    assert ws2 >= full * 4 + B * H2 * (-(-S2 // qps)) * D * 2


def test_workspace_size_follows_bsq(L):
    # Causal row groups are runs of units of ceil(128 / bsq) * bsq rows from the
    # chunk origin: the query sizes them for the bsq va_prefill is given.
    B, Hq, S, D, qps, chunk = 1, 28, 131072, 128, 64, 32768
    for bsq in (3, 5, 64, 100, 256):
        unit = -(-128 // bsq) * bsq
        ws = L.va_prefill_workspace_size(nat.VA_BF16, B, Hq, S, S, D, qps, 1, chunk, bsq)
        # the last unit of the last chunk, the one with the longest rows, fits
        nqb, J0 = S // qps, (S - chunk) // qps
        last = J0 + (chunk // qps - 1) // unit * unit
        cap = L.va_select_index_capacity(B, Hq, S, qps, 1, 1, last, nqb - last, 0)
        assert ws >= cap * 4
    assert L.va_prefill_workspace_size(nat.VA_BF16, B, Hq, S, S, D, qps, 1, chunk, 0) == -1


def _dense(L, **over):
    args = dict(dtype=nat.VA_BF16, q=256, sqb=0, sqh=0, sqs=128, k=256, skb=0, skh=0, sks=128,
                v=256, svb=0, svh=0, svs=128, out=256, sob=0, soh=0, sos=128, B=1, Hq=4, Hk=2,
                Sq=100, Sk=300, D=128, causal=1, scale=0.088, stream=None)
    args.update(over)
    return L.va_dense_attn(*args.values())


def test_dense_attn_argument_errors_before_launch(L):
    assert _dense(L, q=None) == nat.VA_ERR_ARG
    assert _dense(L, Sq=400) == nat.VA_ERR_ARG                 # causal needs Sq <= Sk
    assert _dense(L, Hk=3) == nat.VA_ERR_ARG
    assert _dense(L, Sk=0) == nat.VA_ERR_ARG
    # fp32 runs on the fp32 matrix-core kernel: D 64 or 128, 16-byte aligned rows
    assert _dense(L, dtype=nat.VA_F32, D=96) == nat.VA_ERR_UNSUPPORTED
    assert _dense(L, dtype=nat.VA_F32, sks=130) == nat.VA_ERR_UNSUPPORTED
    assert _dense(L, dtype=nat.VA_F32, out=260) == nat.VA_ERR_UNSUPPORTED
    assert _dense(L, D=256) == nat.VA_ERR_UNSUPPORTED
    assert _dense(L, sks=1 << 14) == nat.VA_ERR_UNSUPPORTED   # row stride past the 14-bit field
    assert _dense(L, scale=-1.0) == nat.VA_ERR_UNSUPPORTED
    assert _dense(L, dtype=9) == nat.VA_ERR_ARG


def _dense_stats(L, **over):
    args = dict(dtype=nat.VA_BF16, q=256, sqb=0, sqh=0, sqs=128, k=256, skb=0, skh=0, sks=128,
                B=1, Hq=4, Hk=2, Sq=100, Sk=300, D=128, causal=1, scale=0.088,
                kernel=nat.VA_ATTN_MFMA, stats=256, stream=None)
    args.update(over)
    return L.va_dense_row_stats(*args.values())


def _sparse_stats(L, **over):
    args = dict(dtype=nat.VA_BF16, q=256, sqb=0, sqh=0, sqs=128, k=256, skb=0, skh=0, sks=128,
                B=1, Hq=4, Hk=2, Sq=256, Sk=256, D=128, qps=64, causal=1, wo_init=1, J0=0,
                nc=4, dense_stride=0, counts=256, indices=256, scale=0.088,
                kernel=nat.VA_ATTN_MFMA, stats=256, stream=None)
    args.update(over)
    return L.va_sparse_row_stats(*args.values())


def test_row_stats_argument_errors_before_launch(L):
    assert _dense_stats(L, stats=None) == nat.VA_ERR_ARG
    assert _dense_stats(L, q=None) == nat.VA_ERR_ARG
    assert _dense_stats(L, Sq=400) == nat.VA_ERR_ARG            # causal needs Sq <= Sk
    assert _dense_stats(L, Hk=3) == nat.VA_ERR_ARG
    assert _dense_stats(L, dtype=nat.VA_F32) == nat.VA_ERR_UNSUPPORTED  # MFMA asked for fp32
    assert _dense_stats(L, D=96) == nat.VA_ERR_UNSUPPORTED
    assert _dense_stats(L, scale=-1.0) == nat.VA_ERR_UNSUPPORTED
    assert _dense_stats(L, kernel=7) == nat.VA_ERR_ARG
    assert _sparse_stats(L, stats=None) == nat.VA_ERR_ARG
    assert _sparse_stats(L, counts=None) == nat.VA_ERR_ARG      # counts without indices
    assert _sparse_stats(L, Sq=300) == nat.VA_ERR_UNSUPPORTED   # causal needs Sq == Sk
    assert _sparse_stats(L, nc=5) == nat.VA_ERR_ARG             # rows past the q-blocks
    assert _sparse_stats(L, dtype=nat.VA_F32) == nat.VA_ERR_UNSUPPORTED


def _decode(lib, **over):
    args = dict(dtype=nat.VA_BF16, q=256, sqh=128, k=256, skh=128, sks=512, v=256, svh=128,
                svs=512, out=256, soh=128, Hq=28, Hk=4, L=1000, D=128, scale=0.088,
                kernel=nat.VA_ATTN_MFMA, ws=256, ws_bytes=1 << 30, stream=None)
    args.update(over)
    return lib.va_decode_attn(*args.values())


def test_decode_argument_errors_before_launch(L):
    assert L.va_decode_workspace_size(28, 3, 1000, 128) == -1
    need = L.va_decode_workspace_size(28, 4, 1000, 128)
    assert need > 0 and need % 256 == 0
    assert _decode(L, q=None) == nat.VA_ERR_ARG
    assert _decode(L, Hk=3) == nat.VA_ERR_ARG
    assert _decode(L, L=0) == nat.VA_ERR_ARG
    assert _decode(L, dtype=nat.VA_F32) == nat.VA_ERR_UNSUPPORTED   # MFMA asked for fp32
    assert _decode(L, D=96, sqh=96, skh=96, svh=96, soh=96) == nat.VA_ERR_UNSUPPORTED
    assert _decode(L, Hq=4 * 65, Hk=4) == nat.VA_ERR_UNSUPPORTED    # > 64 q heads per kv head
    assert _decode(L, sks=1 << 14) == nat.VA_ERR_UNSUPPORTED        # row stride past 14 bits
    assert _decode(L, ws=None) == nat.VA_ERR_WORKSPACE
    assert _decode(L, ws_bytes=need - 256) == nat.VA_ERR_WORKSPACE
    assert _decode(L, kernel=9) == nat.VA_ERR_ARG


def _plan(L, dtype=nat.VA_BF16, D=128, qps=64, bk=16, G=16, Sk=32768, kv_row=None, align=256,
          Hq=28, Hk=4):
    # va_prefill_kernels only inspects addresses and strides (no device access):
    # plain integers stand for the tensors' addresses.
    row = D if kv_row is None else kv_row
    q, k, v, out = align, 2 * align, 3 * align, 4 * align
    return L.va_prefill_kernels(dtype, q, 8 * Sk * D, Sk * D, D, k, 8 * Sk * row, Sk * row, row,
                                v, 8 * Sk * row, Sk * row, row, out, 8 * Sk * D, Sk * D, D, Hq,
                                Hk, Sk, D, qps, bk, G)


def test_prefill_kernels_reports_the_mfma_path(L):
    fast = nat.VA_KERNELS_SELECT_WAVE | nat.VA_KERNELS_ATTN_MFMA | nat.VA_KERNELS_SPLIT
    ring = nat.VA_KERNELS_ATTN_RING
    assert _plan(L) == fast | ring                            # 32K causal GQA
    assert _plan(L, Sk=131072) == fast | ring                 # 128K: 7 q heads per kv head
    # one group per row (DiT group_k_block): the two-pass split
    assert _plan(L, G=8192, Sk=32760, Hq=12, Hk=12) == fast | ring
    # unshared kv heads whose K and V pass 32 MiB a head: the staged form
    assert _plan(L, G=8192, Sk=119056, Hq=24, Hk=24) == fast
    # the ring form exists for D = 128 and 64-row blocks only
    assert not _plan(L, D=64) & ring and not _plan(L, qps=128) & ring
    assert _plan(L, Hq=6, Hk=4) == nat.VA_ERR_ARG             # q heads not a multiple
    # va_prefill takes q_pooling_size 64 or 128 only, and so does its plan
    assert _plan(L, qps=96) == nat.VA_ERR_ARG
    # the reference models' default group_k_block 1: groups of 16 or 32 keys
    # divide the wave kernel's 64-key chunk, so it takes them, in segments of
    # whole chunks
    assert _plan(L, G=1) == fast | ring
    assert _plan(L, G=1, Sk=131072) == fast | ring
    assert _plan(L, G=2) == fast | ring and _plan(L, bk=32, G=1) == fast | ring
    assert L.va_select_segment_keys(131072, 16, 1) == 4096
    assert L.va_select_segment_keys(32768, 16, 1) == 2048
    assert L.va_select_segment_keys(3000, 32, 1) % 64 == 0
    # a 48-key span neither divides nor is a multiple of the chunk: the 64-row
    # MFMA kernel, split into key segments of whole 256-key chunks
    split_mfma = nat.VA_KERNELS_SELECT_MFMA | nat.VA_KERNELS_ATTN_MFMA | nat.VA_KERNELS_SPLIT
    assert _plan(L, G=3) == split_mfma | ring
    assert L.va_select_segment_keys(3000, 16, 3) % 768 == 0


def test_prefill_kernels_reports_the_slow_paths(L):
    # the reference signature's default tiles (q_pooling_size and k_local_size
    # 128): the 64-row MFMA selection (the wave kernel takes tiles up to 64)
    # in key segments of whole 256-key chunks
    mfma = nat.VA_KERNELS_SELECT_MFMA | nat.VA_KERNELS_ATTN_MFMA | nat.VA_KERNELS_SPLIT
    assert _plan(L, qps=128, bk=128, G=1) == mfma
    assert _plan(L, bk=256, G=2) == mfma | nat.VA_KERNELS_ATTN_RING
    # one group per row: no carry pass on this kernel, so no split
    assert _plan(L, bk=128, G=8192) == (nat.VA_KERNELS_SELECT_MFMA | nat.VA_KERNELS_ATTN_MFMA |
                                        nat.VA_KERNELS_ATTN_RING)
    assert _plan(L, bk=512, G=1) & nat.VA_KERNELS_SELECT_EXACT
    # fp32 inputs: exact selection and the fp32 matrix-core attention; the
    # per-row attention for a head_dim that kernel does not take
    # (in key segments the exact kernel splits at in one pass)
    f = _plan(L, dtype=nat.VA_F32)
    f32 = nat.VA_KERNELS_SELECT_EXACT | nat.VA_KERNELS_ATTN_F32
    assert f == f32 | nat.VA_KERNELS_SPLIT
    # one group per row: the exact kernel's two-pass split
    assert _plan(L, dtype=nat.VA_F32, G=8192, Sk=32760, Hq=12, Hk=12) == f32 | nat.VA_KERNELS_SPLIT
    # segments of 256 keys or more, multiples of 256 and of the group span,
    # at most 64 of them
    assert L.va_select_exact_segment_keys(4096, 16, 16) == 256
    assert L.va_select_exact_segment_keys(32768, 16, 16) == 512
    assert L.va_select_exact_segment_keys(131072, 16, 1) == 2048
    assert L.va_select_exact_segment_keys(4096, 16, 3) == 768       # span 48: lcm 768
    assert L.va_select_exact_segment_keys(4096, 16, 8192) == 256    # one group per row: 2 passes
    assert L.va_select_exact_segment_keys(32760, 16, 8192) == 512
    assert L.va_select_exact_segment_keys(200, 16, 16) == 0         # one group covers Sk
    assert L.va_select_exact_segment_keys(0, 16, 16) == -1
    assert _plan(L, dtype=nat.VA_F32, D=96) == nat.VA_KERNELS_SELECT_EXACT | nat.VA_KERNELS_ATTN_ROW
    # head_dim 96: neither MFMA kernel
    f = _plan(L, D=96)
    assert f & nat.VA_KERNELS_SELECT_EXACT and f & nat.VA_KERNELS_ATTN_ROW
    # K/V rows 16 KiB apart: the attention's buffer record stride no longer fits
    f = _plan(L, kv_row=8192)
    assert f & nat.VA_KERNELS_ATTN_ROW
    # unaligned keys
    f = _plan(L, align=258)
    assert f & nat.VA_KERNELS_SELECT_EXACT and f & nat.VA_KERNELS_ATTN_ROW
    assert _plan(L, D=0) < 0


def test_probe_rejects_bad_sizes():
    # The helper library (not the product): checked before any launch, so fake
    # addresses are never dereferenced.
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "numerics"))
    import gather_probe
    P = gather_probe.lib()
    t, sink = 256, 512
    assert P.va_probe_gather(t, 1024, 8, 15, 0, sink, None) == nat.VA_ERR_ARG   # steps % 16
    assert P.va_probe_gather(t, 0, 8, 16, 0, sink, None) == nat.VA_ERR_ARG      # no rows
    assert P.va_probe_gather(t, (1 << 23) + 1, 8, 16, 0, sink, None) == nat.VA_ERR_ARG
    assert P.va_probe_gather(None, 1024, 8, 16, 0, sink, None) == nat.VA_ERR_ARG
    assert P.va_probe_gather(t, 1024, 1 << 20, 1 << 12, 0, sink, None) == nat.VA_ERR_ARG  # ids


def test_product_exports_no_probe():
    L = nat.lib()
    assert not hasattr(L, "va_probe_gather")


@pytest.mark.parametrize("src", ["attn_mfma.hip", "select_wave.hip"])
def test_m0_is_only_set_by_the_lds_copies(src, tmp_path):
    # The LDS-DMA copies set M0 inside inline assembly (lanes.h).  M0 is
    # reserved to the compiler, which ignores it as a clobber, so the copies
    # are only safe while no compiler-generated instruction reads or writes
    # M0: check the device assembly outside the inline-asm blocks.
    from vecattention_amd import build as vbuild
    out = tmp_path / (src + ".s")
    subprocess.run([vbuild.hipcc(), *vbuild.FLAGS, "--cuda-device-only", "-S",
                    os.path.join(vbuild.CSRC, src), "-o", str(out)],
                   check=True, capture_output=True)
    inside, outside, sets = False, [], 0
    for line in out.read_text().splitlines():
        if "ASMSTART" in line:
            inside = True
        elif "ASMEND" in line:
            inside = False
        elif not line.lstrip().startswith(";") and re.search(r"\bm0\b", line):
            if inside:
                sets += 1
            else:
                outside.append(line.strip())
    assert sets > 0
    assert outside == []


def _stats_seg(L, **over):
    args = dict(dtype=nat.VA_BF16, q=256, sqb=0, sqh=0, sqs=128, k=256, skb=0, skh=0, sks=128,
                B=1, Hq=4, Hk=2, Sq=1024, Sk=1024, D=128, qps=64, causal=1, wo_init=1, J0=0,
                nc=16, dense_stride=0, segk=256, counts=256, indices=256, scale=0.088,
                stats=256, stream=None)
    args.update(over)
    return L.va_sparse_row_stats_segments(*args.values())


def test_sparse_row_stats_segments_argument_errors_before_launch(L):
    assert _stats_seg(L, stats=None) == nat.VA_ERR_ARG
    assert _stats_seg(L, counts=None) == nat.VA_ERR_ARG
    assert _stats_seg(L, segk=100) == nat.VA_ERR_ARG                 # not a multiple of 64
    assert _stats_seg(L, segk=0) == nat.VA_ERR_ARG
    assert _stats_seg(L, Sk=8192, Sq=8192, nc=128, segk=64) == nat.VA_ERR_ARG  # 128 segments
    # segmented lists run on the MFMA kernel only: not fp32, not D = 96
    assert _stats_seg(L, dtype=nat.VA_F32) == nat.VA_ERR_UNSUPPORTED
    assert _stats_seg(L, D=96, sqs=96, sks=96) == nat.VA_ERR_UNSUPPORTED
