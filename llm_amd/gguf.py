"""GGUF reader: the reference's ``GgufFile`` (apps/engine/src/gguf.rs) over the
C-ABI of include/q8gguf.h, plus the model loader's shape-checked ``weight``
lookup (apps/engine/src/model.rs:1670-1684).

The file is memory-mapped by the native library; ``data(name)`` is a read-only
numpy view of the map (no copy), and a ``Weight`` built on it carries the
map address as its identity, so the device residency cache uploads it once,
as the reference's ``Gpu::quantized`` does for its mmap slices.  A view keeps
its file mapped for as long as the view lives.

    gguf = GgufFile.open(path)
    wq = weight(gguf, "blk.0.attn_q.weight", k, out)
    compute.matmul(wq, x, 0, 1, y, 0)
"""
from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass

import numpy as np

from . import q8
from .q8 import GgufTensorInfo, Q8Error, Weight, _check, lib


class DType(enum.IntEnum):
    """gguf.rs:19-56."""
    F32 = 0
    F16 = 1
    Q8_0 = 8

    def block_elements(self) -> int:
        return 32 if self is DType.Q8_0 else 1

    def block_bytes(self) -> int:
        return {DType.Q8_0: 34, DType.F32: 4, DType.F16: 2}[self]

    def byte_len(self, elements: int) -> int:
        return elements // self.block_elements() * self.block_bytes()


@dataclass(frozen=True)
class TensorInfo:
    """gguf.rs:58-71."""
    name: str
    dims: tuple
    dtype: DType
    offset: int
    byte_len: int

    def elements(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n


class _MapView:
    """Array interface over bytes of the map; holds the file open."""

    def __init__(self, owner: "GgufFile", address: int, length: int):
        self._owner = owner
        self.__array_interface__ = {"shape": (length,), "typestr": "|u1", "data": (address, True),
                                    "version": 3}


class GgufFile:
    """GgufFile (gguf.rs:88-311).  Errors raise ``Q8Error`` with the status of
    the reference's error kind: Q8_ERR_FORMAT (Format), Q8_ERR_MISSING
    (MissingTensor / MissingMetadata), Q8_ERR_UNSUPPORTED, Q8_ERR_IO."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        _check(lib().q8_gguf_open(str(path).encode(), ctypes.byref(h)))
        self.handle = h.value
        self.path = str(path)

    @classmethod
    def open(cls, path) -> "GgufFile":
        return cls(path)

    def __del__(self):
        h, self.handle = getattr(self, "handle", None), None
        if h:
            lib().q8_gguf_close(h)

    # ---- header ----
    def layout(self) -> dict:
        v, a, d, f = ctypes.c_uint32(), ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        _check(lib().q8_gguf_layout(self.handle, ctypes.byref(v), ctypes.byref(a), ctypes.byref(d),
                                    ctypes.byref(f)))
        return {"version": v.value, "alignment": a.value, "data_start": d.value, "file_bytes": f.value}

    # ---- tensors ----
    @staticmethod
    def _info(t: GgufTensorInfo) -> TensorInfo:
        name = ctypes.string_at(t.name, t.name_len).decode()
        return TensorInfo(name, tuple(t.dims[i] for i in range(t.n_dims)), DType(t.dtype), t.offset, t.byte_len)

    def tensors(self) -> list[TensorInfo]:
        n = ctypes.c_uint64()
        _check(lib().q8_gguf_tensor_count(self.handle, ctypes.byref(n)))
        out = []
        for i in range(n.value):
            t = GgufTensorInfo()
            _check(lib().q8_gguf_tensor_at(self.handle, i, ctypes.byref(t)))
            out.append(self._info(t))
        return out

    def _raw(self, name: str) -> GgufTensorInfo:
        t = GgufTensorInfo()
        _check(lib().q8_gguf_tensor(self.handle, name.encode(), ctypes.byref(t)))
        return t

    def tensor(self, name: str) -> TensorInfo:
        return self._info(self._raw(name))

    def data_address(self, name: str) -> int:
        return self._raw(name).data or 0

    def data(self, name: str) -> np.ndarray:
        """Raw little-endian bytes of a tensor, a read-only view of the map."""
        t = self._raw(name)
        if t.byte_len == 0:
            return np.zeros(0, dtype=np.uint8)
        return np.asarray(_MapView(self, t.data, t.byte_len))

    # ---- metadata ----
    def keys(self) -> list[str]:
        n = ctypes.c_uint64()
        _check(lib().q8_gguf_meta_count(self.handle, ctypes.byref(n)))
        out = []
        for i in range(n.value):
            k = ctypes.c_char_p()
            _check(lib().q8_gguf_meta_key_at(self.handle, i, ctypes.byref(k)))
            out.append(k.value.decode())
        return out

    def meta_type(self, key: str) -> tuple[int, int, int]:
        t, e, n = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint64()
        _check(lib().q8_gguf_meta_type(self.handle, key.encode(), ctypes.byref(t), ctypes.byref(e),
                                       ctypes.byref(n)))
        return t.value, e.value, n.value

    def meta_u64(self, key: str) -> int:
        v = ctypes.c_uint64()
        _check(lib().q8_gguf_meta_u64(self.handle, key.encode(), ctypes.byref(v)))
        return v.value

    def meta_f32(self, key: str) -> np.float32:
        v = ctypes.c_float()
        _check(lib().q8_gguf_meta_f32(self.handle, key.encode(), ctypes.byref(v)))
        return np.float32(v.value)

    def meta_bool(self, key: str) -> bool:
        v = ctypes.c_int()
        _check(lib().q8_gguf_meta_bool(self.handle, key.encode(), ctypes.byref(v)))
        return bool(v.value)

    def meta_u64_opt(self, key: str) -> int | None:
        """gguf.rs:220-228: None for a missing key or a value of another kind."""
        try:
            return self.meta_u64(key)
        except Q8Error as e:
            if e.status in (q8.Q8_ERR_MISSING, q8.Q8_ERR_FORMAT):
                return None
            raise

    def meta_f32_opt(self, key: str) -> np.float32 | None:
        """gguf.rs:230-235."""
        try:
            return self.meta_f32(key)
        except Q8Error as e:
            if e.status in (q8.Q8_ERR_MISSING, q8.Q8_ERR_FORMAT):
                return None
            raise

    def has_key_prefix(self, prefix: str) -> bool:
        return bool(lib().q8_gguf_has_key_prefix(self.handle, prefix.encode()))

    def meta_str(self, key: str) -> str:
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        _check(lib().q8_gguf_meta_str(self.handle, key.encode(), ctypes.byref(p), ctypes.byref(n)))
        return ctypes.string_at(p.value, n.value).decode() if n.value else ""

    def _array_len(self, fn, key: str) -> int:
        n = ctypes.c_uint64()
        _check(fn(self.handle, key.encode(), None, 0, ctypes.byref(n)))
        return n.value

    def meta_i32_array(self, key: str) -> np.ndarray:
        n = self._array_len(lib().q8_gguf_meta_i32_array, key)
        out = np.empty(n, dtype=np.int32)
        got = ctypes.c_uint64()
        _check(lib().q8_gguf_meta_i32_array(self.handle, key.encode(), out.ctypes.data, n, ctypes.byref(got)))
        return out

    def meta_f32_array(self, key: str) -> np.ndarray:
        n = self._array_len(lib().q8_gguf_meta_f32_array, key)
        out = np.empty(n, dtype=np.float32)
        got = ctypes.c_uint64()
        _check(lib().q8_gguf_meta_f32_array(self.handle, key.encode(), out.ctypes.data, n, ctypes.byref(got)))
        return out

    def meta_str_array(self, key: str) -> list[str]:
        got = ctypes.c_uint64()
        _check(lib().q8_gguf_meta_str_array(self.handle, key.encode(), None, None, 0, ctypes.byref(got)))
        n = got.value
        ptrs = (ctypes.c_void_p * max(n, 1))()
        lens = (ctypes.c_uint64 * max(n, 1))()
        _check(lib().q8_gguf_meta_str_array(self.handle, key.encode(), ptrs, lens, n, ctypes.byref(got)))
        return [ctypes.string_at(ptrs[i], lens[i]).decode() if lens[i] else "" for i in range(n)]


def weight(gguf: GgufFile, name: str, k: int, out: int) -> Weight:
    """model.rs:1670-1684: the tensor must have dims exactly [k, out].  The
    device path takes Q8_0 only (Compute::matmul, compute.rs:475-529)."""
    info = gguf.tensor(name)
    if info.dims != (k, out):
        raise Q8Error(q8.Q8_ERR_FORMAT, f"malformed gguf: {name} has shape {list(info.dims)}, expected [{k}, {out}]")
    if info.dtype != DType.Q8_0:
        raise Q8Error(q8.Q8_ERR_UNSUPPORTED, f"unsupported: {name} is {info.dtype.name}, the device path takes Q8_0")
    return Weight(gguf.data(name), k, out)
