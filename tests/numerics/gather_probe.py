"""ctypes binding of libgatherprobe.so (gather_probe.hip): the L2 -> LDS
row-gather rate that bench.py reports beside the attention kernel's gathers.
A measurement helper built by __graft_entry__.build(), not part of the
product library."""
import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libgatherprobe.so")
_lib = None


def lib():
    """The loaded helper library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        L.va_probe_gather.restype = ctypes.c_int
        L.va_probe_gather.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                                      ctypes.c_int64, ctypes.c_int, ctypes.c_void_p,
                                      ctypes.c_void_p]
        _lib = L
    return _lib


def gather(table_ptr, rows, work_groups, steps, sequential, sink_ptr, stream):
    """Run the probe (see gather_probe.hip); raises on a nonzero status."""
    rc = lib().va_probe_gather(table_ptr, rows, work_groups, steps, sequential, sink_ptr, stream)
    if rc != 0:
        raise RuntimeError(f"va_probe_gather failed with status {rc}")
