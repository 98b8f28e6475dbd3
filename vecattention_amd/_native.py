"""ctypes binding of libvecattn.so (the C ABI declared in include/vecattn.h).

The library is built in-tree by ``python -m vecattention_amd.build`` (or
``__graft_entry__.build()``).  There is no fallback: if the library is missing
or fails to load, every entry point raises.
"""
import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libvecattn.so")

VA_F32, VA_BF16, VA_F16 = 0, 1, 2
VA_OK, VA_ERR_ARG, VA_ERR_UNSUPPORTED, VA_ERR_HIP, VA_ERR_WORKSPACE = 0, -1, -2, -3, -4
VA_ATTN_AUTO, VA_ATTN_MFMA, VA_ATTN_SIMPLE = 0, 1, 2
VA_ATTN_MFMA_STAGED, VA_ATTN_MFMA_RING = 3, 4  # forms of the MFMA kernel's loop
VA_SEL_AUTO, VA_SEL_EXACT, VA_SEL_MFMA, VA_SEL_WAVE = 0, 1, 2, 3
VA_KERNELS_SELECT_WAVE, VA_KERNELS_SELECT_MFMA, VA_KERNELS_SELECT_EXACT = 1, 2, 4
VA_KERNELS_ATTN_MFMA, VA_KERNELS_ATTN_ROW, VA_KERNELS_SPLIT = 16, 32, 64
VA_KERNELS_ATTN_RING, VA_KERNELS_ATTN_F32 = 128, 256

_DTYPES = {torch.float32: VA_F32, torch.bfloat16: VA_BF16, torch.float16: VA_F16}

_lock = threading.Lock()
_lib = None

_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p
_f32 = ctypes.c_float

# name -> (restype, argtypes); the exported surface of include/vecattn.h.
SIGNATURES = {
    "va_version": (_int, []),
    "va_last_error": (ctypes.c_char_p, []),
    "va_device_count": (_int, []),
    "va_pool": (_int, [_int, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp]),
    "va_select": (_int, [_int, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                         _i64, _i64, _i64, _i64, _i64, _int, _int, _i64, _i64, _i64, _f32, _vp,
                         _i64, _vp, _vp, _int, _vp, _i64, _vp]),
    "va_select_segment_keys": (_i64, [_i64, _i64, _i64]),
    "va_select_exact_segment_keys": (_i64, [_i64, _i64, _i64]),
    "va_select_segments": (_int, [_int, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64,
                                  _i64, _i64, _i64, _i64, _i64, _i64, _int, _int, _i64, _i64, _i64,
                                  _f32, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _vp]),
    "va_select_csr": (_int, [_int, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                             _i64, _i64, _i64, _i64, _i64, _int, _int, _i64, _i64, _i64, _f32, _vp,
                             _i64, _vp, _vp, _vp, _vp, _i64, _vp]),
    "va_select_scratch_floats": (_i64, [_i64, _i64]),
    "va_select_segments_scratch_floats": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64]),
    "va_select_index_capacity": (_i64, [_i64, _i64, _i64, _i64, _int, _int, _i64, _i64, _i64]),
    "va_select_row_offset": (_i64, [_i64, _i64, _int, _int, _i64, _i64, _i64, _i64, _i64]),
    "va_sparse_attn": (_int, [_int, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64,
                              _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                              _i64, _int, _int, _i64, _i64, _i64, _vp, _vp, _f32, _int, _vp]),
    "va_dense_attn": (_int, [_int, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64,
                             _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                             _int, _f32, _vp]),
    "va_sparse_attn_segments": (_int, [_int, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp,
                                       _i64, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                                       _i64, _i64, _i64, _i64, _int, _int, _i64, _i64, _i64, _i64,
                                       _vp, _vp, _f32, _vp]),
    "va_sparse_row_stats": (_int, [_int, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64,
                                   _i64, _i64, _i64, _i64, _i64, _int, _int, _i64, _i64, _i64, _vp,
                                   _vp, _f32, _int, _vp, _vp]),
    "va_sparse_row_stats_segments": (_int, [_int, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64,
                                            _i64, _i64, _i64, _i64, _i64, _i64, _i64, _int, _int,
                                            _i64, _i64, _i64, _i64, _vp, _vp, _f32, _vp, _vp]),
    "va_dense_row_stats": (_int, [_int, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64,
                                  _i64, _i64, _i64, _i64, _int, _f32, _int, _vp, _vp]),
    "va_decode_workspace_size": (_i64, [_i64, _i64, _i64, _i64]),
    "va_decode_attn": (_int, [_int, _vp, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64,
                              _i64, _i64, _i64, _f32, _int, _vp, _i64, _vp]),
    "va_decode_noalloc_scratch_bytes": (_i64, []),
    "va_decode_attn_noalloc": (_int, [_int, _vp, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp,
                                      _i64, _i64, _i64, _i64, _i64, _f32, _int, _vp]),
    "va_prefill_workspace_size": (_i64, [_int, _i64, _i64, _i64, _i64, _i64, _i64, _int, _i64,
                                         _i64]),
    "va_prefill_kernels": (_int, [_int, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64,
                                  _i64, _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                  _i64, _i64, _i64]),
    "va_prefill": (_int, [_int, _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _i64,
                          _i64, _vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _f32,
                          _vp, _i64, _i64, _i64, _int, _i64, _i64, _vp, _i64, _vp]),
}


class NativeError(RuntimeError):
    """A libvecattn call returned an error code."""

    def __init__(self, fn, code, msg):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


def lib():
    """Load (once) and return the ctypes handle; raises if the library is absent."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m vecattention_amd.build` "
                    "(the HIP path has no CPU fallback)")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
        return _lib


def check(fn, code):
    if code != VA_OK:
        msg = lib().va_last_error().decode(errors="replace")
        if code == VA_ERR_ARG:
            raise AssertionError(f"{fn}: {msg}")
        if code == VA_ERR_UNSUPPORTED:
            raise NotImplementedError(f"{fn}: {msg}")
        raise NativeError(fn, code, msg)
    return code


def check_flags(fn, flags):
    """A bit-set result (va_prefill_kernels): raise on a negative error code."""
    if flags < 0:
        check(fn, flags)
    return flags


def dtype_code(t):
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32, bfloat16 or float16")


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def stream_ptr(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
