"""A small GGUF writer for the tests: well-formed files of any metadata type
and tensor type, and deliberately malformed ones (every field can be
overridden).  The layout rules are the GGUF format's as the reference reads
them (apps/engine/src/gguf.rs:95-175): header, key/value pairs, tensor
table, padding to the alignment, tensor data at 32-aligned offsets (or the
alignment in force) from the data start.
"""
from __future__ import annotations

import struct

import numpy as np

MAGIC = 0x46554747
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
T_F32, T_F16, T_Q8_0 = 0, 1, 8

_FIXED = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
          U64: "<Q", I64: "<q", F64: "<d"}


def enc_str(s) -> bytes:
    b = s if isinstance(s, bytes) else s.encode()
    return struct.pack("<Q", len(b)) + b


def enc_value(kind: int, value) -> bytes:
    """Payload of one value of type `kind` (without the type id).  Arrays are
    (elem_type, [values]); nested arrays are (ARRAY, [(elem_type, [..]), ..])."""
    if kind in _FIXED:
        return struct.pack(_FIXED[kind], value)
    if kind == STRING:
        return enc_str(value)
    if kind == ARRAY:
        elem, items = value
        out = struct.pack("<IQ", elem, len(items))
        return out + b"".join(enc_value(elem, v) for v in items)
    raise ValueError(kind)


def q8_bytes(rows: int, k: int, rng: np.random.Generator) -> np.ndarray:
    """Q8_0 rows x k: random quants in [-127, 127] and f16 scales (normal and
    subnormal), row-major blocks of [f16 d][32 x i8]."""
    nb = k // 32
    blk = np.zeros((rows, nb, 34), np.uint8)
    d = (np.abs(rng.normal(0.0, 0.02, (rows, nb))) / 127).astype(np.float16)
    blk[:, :, 0:2] = d.view(np.uint8).reshape(rows, nb, 2)
    blk[:, :, 2:] = rng.integers(-127, 128, (rows, nb, 32), dtype=np.int8).view(np.uint8)
    return blk.reshape(-1)


def build(metadata=(), tensors=(), *, magic=MAGIC, version=3, tensor_count=None, kv_count=None,
          alignment=32, trailing=b"") -> bytes:
    """metadata: (key, kind, value) or (key, kind, raw_payload_bytes) when
    kind is given as ('raw', type_id).  tensors: dicts with name, dims, dtype,
    data (bytes) and optional offset / n_dims overrides."""
    head = bytearray(struct.pack("<II", magic, version))
    head += struct.pack("<Q", len(tensors) if tensor_count is None else tensor_count)
    head += struct.pack("<Q", len(metadata) if kv_count is None else kv_count)
    for key, kind, value in metadata:
        head += enc_str(key)
        if isinstance(kind, tuple):
            head += struct.pack("<I", kind[1]) + value
        else:
            head += struct.pack("<I", kind) + enc_value(kind, value)
    offset = 0
    blobs = []
    for t in tensors:
        dims = t["dims"]
        head += enc_str(t["name"])
        head += struct.pack("<I", t.get("n_dims", len(dims)))
        head += b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<I", t["dtype"])
        off = t.get("offset", offset)
        head += struct.pack("<Q", off)
        data = bytes(t.get("data", b""))
        blobs.append((off, data))
        offset = off + len(data)
        offset = (offset + alignment - 1) // alignment * alignment
    data_start = (len(head) + alignment - 1) // alignment * alignment
    body = bytearray(head) + b"\0" * (data_start - len(head))
    for off, data in blobs:
        if not data:  # a tensor written without bytes (for malformed files)
            continue
        end = data_start + off + len(data)
        if len(body) < end:
            body += b"\0" * (end - len(body))
        body[data_start + off:end] = data
    pad = (len(body) + alignment - 1) // alignment * alignment - len(body)
    return bytes(body) + b"\0" * pad + trailing


def write(path, *args, **kw) -> str:
    with open(path, "wb") as f:
        f.write(build(*args, **kw))
    return str(path)
