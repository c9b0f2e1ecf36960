"""The benchmark's measurement kernels (libq8bench.so, include/q8bench.h):
what one MI355X sustains at the path's shapes -- plain reads, MFMA, VALU,
their mixes and co-resident splits -- so bench.py can quote each hot-path
kernel against a ceiling.  Bench-only: nothing of the product path imports
this module, and the product library does not contain these kernels."""
from __future__ import annotations

import ctypes
import os

from . import q8

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libq8bench.so")

EMPTY, MFMA, VALU, MIX, MIX_F16, SPLIT_I8_VALU, SPLIT_I8_FMA, SPLIT_F32_VALU = range(8)
EXPORTS = ("q8bench_open", "q8bench_close", "q8bench_last_error", "q8bench_build_info", "q8bench_read",
           "q8bench_probe")

_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m llm_amd.build`")
    L = ctypes.CDLL(LIB_PATH)
    c_int, vp = ctypes.c_int, ctypes.c_void_p
    sig = {
        "q8bench_open": (c_int, [vp, ctypes.POINTER(vp)]),
        "q8bench_close": (None, [vp]),
        "q8bench_last_error": (ctypes.c_char_p, []),
        "q8bench_build_info": (ctypes.c_char_p, []),
        "q8bench_read": (c_int, [vp, ctypes.c_uint64, ctypes.c_size_t, c_int, c_int, c_int]),
        "q8bench_probe": (c_int, [vp, c_int, c_int, c_int, c_int]),
    }
    assert set(sig) == set(EXPORTS)
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def _check(status: int):
    if status != q8.Q8_OK:
        raise q8.Q8Error(status, lib().q8bench_last_error().decode())


class Probes:
    """Measurement kernels on a matmul context's stream (so they can be
    captured into its graphs and timed with its events)."""

    def __init__(self, gpu: "q8.Gpu"):
        h = ctypes.c_void_p()
        _check(lib().q8bench_open(gpu.stream(), ctypes.byref(h)))
        self.handle = h.value

    def close(self):
        if self.handle:
            lib().q8bench_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def read(self, src: "q8.DeviceBuffer", nbytes: int, loads: int, nontemporal: bool = False, threads: int = 256,
             src_offset: int = 0):
        _check(lib().q8bench_read(self.handle, src.ptr + src_offset, nbytes, loads, 1 if nontemporal else 0, threads))

    def probe(self, which: int, iters: int = 0, workgroups: int = 0, mask: int = 3):
        _check(lib().q8bench_probe(self.handle, which, iters, workgroups, mask))
