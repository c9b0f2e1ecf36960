"""CPU oracle for the Q8_0 matmul path -- TEST INFRASTRUCTURE ONLY.

This package is the checker the HIP path is compared against.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it; nothing under ``llm_amd/`` does, and the product path never falls back to it.

``q8_oracle.c`` restates the reference's CPU kernels in the same floating-point
order (``apps/engine/src/quant.rs:8-203``, ``apps/engine/src/tensor.rs:92-149``,
``apps/engine/src/ops.rs:5-35``, ``apps/engine/src/sampler.rs:167-175``).  This
module wraps it with numpy and adds the seeded synthetic-input generators that
the parity tests and the benchmark share.

How each function is pinned (and where the pin lives):

* ``f16_to_f32`` / ``dequant_q8_0`` -- closed form (IEEE binary16 decode,
  including every subnormal ``m * 2**-24``) and the reference KATs of
  ``apps/engine/tests/quant_q8.rs:13-63``; ``tests/test_oracle.py``.
* ``dot_q8_0`` (AVX2 and scalar orders) -- the KATs of ``quant_q8.rs:14-44`` and
  ``matmul.rs:139-152`` (f64 references, 1e-4 / 1e-3), exact-arithmetic cases
  (``tests/test_oracle.py``), and an independent exact-order restatement in
  Python with each f32 operation rounded once (FMAs rounded from the exact
  rational) that must agree bit for bit on random rows, in both orders
  (``tests/test_oracle_order.py``).
* ``quantize_q8_0`` -- closed form: scale = peak/127, half-away rounding,
  saturation, NaN and all-zero blocks; ``tests/test_oracle.py``.
* ``dot_q8_0_q8_0`` -- the int32 block dot by brute force in int64, the KATs of
  ``matmul.rs:154-168`` and ``matmul.rs:170-198``, and the same exact-order
  restatement of both the scalar and the AVX2 lane order
  (``tests/test_oracle_order.py``).
* ``matmul`` -- ``matmul.rs:139-198`` and the row/thread independence the
  reference relies on (``tensor.rs:127-148``).
* ``silu`` / ``rmsnorm`` / ``argmax`` -- ``ops.rs``'s hand values
  (``apps/engine/tests/ops.rs``) and closed forms.
* ``rope`` -- closed forms: position 0 is the identity, each pair keeps its
  norm, rotations compose (angle(p) = p * angle(1) within f32 rounding), pairs
  past ``n_rot`` are untouched, and a hand-computed pair; ``tests/test_oracle.py``.
* ``attention`` -- closed forms: one visible key returns its value, equal keys
  return the mean of the values, a key far above the rest returns its value,
  shifting every score changes nothing, and later keys never change earlier
  rows (causality); ``tests/test_oracle.py``.  It computes the exact (f64)
  value of the reference's formula; the device is held to the f32 bar against
  it rather than to one f32 summation order.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libq8oracle.so")

BLOCK_ELEMS = 32
BLOCK_BYTES = 34

_lib = None


def build() -> str:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        u8p = ctypes.POINTER(ctypes.c_uint8)
        i8p = ctypes.POINTER(ctypes.c_int8)
        f32p = ctypes.POINTER(ctypes.c_float)
        sz = ctypes.c_size_t
        L.q8o_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.q8o_f16_to_f32.restype = ctypes.c_float
        for name in ("q8o_dot_q8_0", "q8o_dot_q8_0_scalar", "q8o_dot_q8_0_avx2"):
            f = getattr(L, name)
            f.argtypes = [u8p, f32p, sz]
            f.restype = ctypes.c_float
        for name in ("q8o_dot_q8_0_q8_0", "q8o_dot_q8_0_q8_0_scalar", "q8o_dot_q8_0_q8_0_avx2"):
            f = getattr(L, name)
            f.argtypes = [u8p, i8p, f32p, sz]
            f.restype = ctypes.c_float
        L.q8o_block_dot_i64.argtypes = [u8p, i8p, sz]
        L.q8o_block_dot_i64.restype = ctypes.c_int64
        L.q8o_quantize_q8_0.argtypes = [f32p, sz, i8p, f32p]
        L.q8o_quantize_q8_0.restype = None
        L.q8o_dequant_q8_0.argtypes = [u8p, f32p, sz]
        L.q8o_dequant_q8_0.restype = None
        L.q8o_matmul.argtypes = [u8p, sz, sz, f32p, sz, f32p, ctypes.c_int]
        L.q8o_matmul.restype = ctypes.c_int
        L.q8o_silu.argtypes = [ctypes.c_float]
        L.q8o_silu.restype = ctypes.c_float
        L.q8o_silu_mul.argtypes = [f32p, f32p, f32p, sz]
        L.q8o_silu_mul.restype = None
        L.q8o_rms_scale.argtypes = [f32p, sz, ctypes.c_float]
        L.q8o_rms_scale.restype = ctypes.c_float
        L.q8o_rmsnorm.argtypes = [f32p, f32p, sz, ctypes.c_float, f32p]
        L.q8o_rmsnorm.restype = None
        L.q8o_argmax.argtypes = [f32p, sz]
        L.q8o_argmax.restype = ctypes.c_uint32
        L.q8o_simd_path.argtypes = []
        L.q8o_simd_path.restype = ctypes.c_int
        _lib = L
    return _lib


def _p(a: np.ndarray, ctype):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def simd_path() -> str:
    """Which order ``dot_q8_0`` dispatches to on this host (quant.rs:25-31)."""
    return "avx2+fma" if lib().q8o_simd_path() else "scalar"


def f16_to_f32(bits: int) -> float:
    return float(lib().q8o_f16_to_f32(int(bits) & 0xFFFF))


def dot_q8_0(row: np.ndarray, x: np.ndarray, order: str = "dispatch") -> np.float32:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    blocks = x.size // BLOCK_ELEMS
    assert x.size % BLOCK_ELEMS == 0 and row.size == blocks * BLOCK_BYTES
    f = {"dispatch": lib().q8o_dot_q8_0, "scalar": lib().q8o_dot_q8_0_scalar,
         "avx2": lib().q8o_dot_q8_0_avx2}[order]
    return np.float32(f(_p(row, ctypes.c_uint8), _p(x, ctypes.c_float), blocks))


def dot_q8_0_q8_0(row: np.ndarray, quants: np.ndarray, scales: np.ndarray,
                  order: str = "dispatch") -> np.float32:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    quants = np.ascontiguousarray(quants, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    blocks = quants.size // BLOCK_ELEMS
    assert row.size == blocks * BLOCK_BYTES and scales.size == blocks
    f = {"dispatch": lib().q8o_dot_q8_0_q8_0, "scalar": lib().q8o_dot_q8_0_q8_0_scalar,
         "avx2": lib().q8o_dot_q8_0_q8_0_avx2}[order]
    return np.float32(f(_p(row, ctypes.c_uint8), _p(quants, ctypes.c_int8),
                        _p(scales, ctypes.c_float), blocks))


def block_dot_i64(row: np.ndarray, quants: np.ndarray, block: int) -> int:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    quants = np.ascontiguousarray(quants, dtype=np.int8)
    return int(lib().q8o_block_dot_i64(_p(row, ctypes.c_uint8), _p(quants, ctypes.c_int8), block))


def quantize_q8_0(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    assert x.size % BLOCK_ELEMS == 0
    quants = np.zeros(x.size, dtype=np.int8)
    scales = np.zeros(x.size // BLOCK_ELEMS, dtype=np.float32)
    lib().q8o_quantize_q8_0(_p(x, ctypes.c_float), x.size, _p(quants, ctypes.c_int8),
                            _p(scales, ctypes.c_float))
    return quants, scales


def dequant_q8_0(row: np.ndarray, k: int) -> np.ndarray:
    row = np.ascontiguousarray(row, dtype=np.uint8)
    out = np.zeros(k, dtype=np.float32)
    lib().q8o_dequant_q8_0(_p(row, ctypes.c_uint8), _p(out, ctypes.c_float), k)
    return out


def matmul(data: np.ndarray, k: int, out: int, x: np.ndarray, n: int,
           threads: int | None = None) -> np.ndarray:
    """``tensor::matmul`` (tensor.rs:92-149): y[t, o] over GGUF Q8_0 bytes."""
    data = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    assert data.size == out * (k // BLOCK_ELEMS) * BLOCK_BYTES, "weight byte length mismatch"
    assert x.size == n * k, "activation shape mismatch"
    y = np.zeros(n * out, dtype=np.float32)
    if threads is None:
        threads = os.cpu_count() or 1
    rc = lib().q8o_matmul(_p(data, ctypes.c_uint8), k, out, _p(x, ctypes.c_float), n,
                          _p(y, ctypes.c_float), int(threads))
    if rc != 0:
        raise RuntimeError(f"oracle matmul failed ({rc})")
    return y.reshape(n, out)


def silu(v: float) -> np.float32:
    return np.float32(lib().q8o_silu(float(v)))


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    gate = np.ascontiguousarray(gate, dtype=np.float32).reshape(-1)
    up = np.ascontiguousarray(up, dtype=np.float32).reshape(-1)
    act = np.zeros_like(gate)
    lib().q8o_silu_mul(_p(gate, ctypes.c_float), _p(up, ctypes.c_float), _p(act, ctypes.c_float),
                       gate.size)
    return act


def rmsnorm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    weight = np.ascontiguousarray(weight, dtype=np.float32).reshape(-1)
    out = np.zeros_like(x)
    lib().q8o_rmsnorm(_p(x, ctypes.c_float), _p(weight, ctypes.c_float), x.size,
                      ctypes.c_float(eps), _p(out, ctypes.c_float))
    return out


def argmax(values: np.ndarray) -> int:
    values = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    return int(lib().q8o_argmax(_p(values, ctypes.c_float), values.size))


# ---------------------------------------------------------------------------
# Seeded synthetic inputs (the shapes and distributions of the benchmark configs).
# ---------------------------------------------------------------------------

def make_q8_weight(rng: np.random.Generator, out: int, k: int, scale_std: float = 0.02,
                   scales=None) -> np.ndarray:
    """GGUF Q8_0 bytes for an ``out x k`` matrix: q uniform in [-127, 127],
    d = f16(|N(0, scale_std)| / 127) (about 30% of them f16 subnormals)."""
    assert k % BLOCK_ELEMS == 0
    blocks = out * (k // BLOCK_ELEMS)
    raw = np.empty((blocks, BLOCK_BYTES), dtype=np.uint8)
    if scales is None:
        scales = (np.abs(rng.standard_normal(blocks, dtype=np.float32)) * scale_std / 127.0)
    d16 = np.asarray(scales, dtype=np.float32).astype(np.float16)
    raw[:, 0:2] = d16.view(np.uint8).reshape(blocks, 2)
    q = rng.integers(-127, 128, size=(blocks, 32), dtype=np.int16).astype(np.int8)
    raw[:, 2:] = q.view(np.uint8)
    return raw.reshape(-1)


def make_activations(rng: np.random.Generator, n: int, k: int,
                     outlier_rate: float = 0.0, outlier: float = 20.0) -> np.ndarray:
    """f32 [n, k] from N(0, 1); with ``outlier_rate`` each element is replaced
    by +-``outlier`` (random sign) with that probability."""
    x = rng.standard_normal((n, k), dtype=np.float32)
    if outlier_rate > 0:
        mask = rng.random((n, k)) < outlier_rate
        signs = np.where(rng.random((n, k)) < 0.5, -outlier, outlier).astype(np.float32)
        x = np.where(mask, signs, x).astype(np.float32)
    return np.ascontiguousarray(x)


# ---------------------------------------------------------------------------
# Decoder support: rotary embedding, f16 KV cache, attention (numpy).
# ---------------------------------------------------------------------------

def rope(x: np.ndarray, start: int, n_rot: int, base: float) -> np.ndarray:
    """RopeTable::new + apply (apps/engine/src/ops.rs:120-166) for rows at
    positions start, start+1, ...: ``x`` is [n, heads, head_dim] f32; pair i of
    every head (dims 2i, 2i+1) for i < n_rot/2 rotates by
    angle = position * base.powf(-2 * i / n_rot), all in f32 and without
    contraction (low*cos - high*sin, low*sin + high*cos); other dims are kept.
    powf, cos and sin are the correctly rounded values of their f32 operands."""
    x = np.array(x, dtype=np.float32, copy=True)
    n = x.shape[0]
    half = n_rot // 2
    if half == 0:
        return x
    pair = np.arange(half, dtype=np.float32)
    exponent = (np.float32(-2.0) * pair) / np.float32(n_rot)
    # f32::powf is the C library's powf, correctly rounded here; numpy's float32
    # power is not (it is an ulp off at base 1e4, exponent -1/32), so take the
    # f64 power of the same f32 operands and round once
    freq = np.power(np.float64(np.float32(base)), exponent.astype(np.float64)).astype(np.float32)
    pos = (np.arange(n, dtype=np.float32) + np.float32(start)).astype(np.float32)
    angle = (pos[:, None] * freq[None, :]).astype(np.float32)          # [n, half]
    cos = np.cos(angle.astype(np.float64)).astype(np.float32)[:, None, :]
    sin = np.sin(angle.astype(np.float64)).astype(np.float32)[:, None, :]
    low = x[:, :, 0:2 * half:2].copy()
    high = x[:, :, 1:2 * half:2].copy()
    x[:, :, 0:2 * half:2] = (low * cos).astype(np.float32) - (high * sin).astype(np.float32)
    x[:, :, 1:2 * half:2] = (low * sin).astype(np.float32) + (high * cos).astype(np.float32)
    return x


def to_f16(x: np.ndarray) -> np.ndarray:
    """The device cache's f32 -> f16 narrowing, nearest even (gpu.cu:506-519)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16)


def attention(q: np.ndarray, keys: np.ndarray, values: np.ndarray, start: int, scale: float) -> np.ndarray:
    """attend_host (apps/engine/src/compute.rs:1075-1126): q [n, n_head, hd]
    for tokens at positions start + t, keys/values [L, n_kv, hd] (the cache,
    L >= start + n); token t sees positions 0 ..= start + t.  Query head h uses
    kv head h // (n_head / n_kv).  scores = dot(q, k) * scale, softmax with the
    max subtracted, output = sum of weight * value.  Computed in f64 (the exact
    value of that formula on the given inputs), returned as f32."""
    q = np.asarray(q, dtype=np.float64)
    keys = np.asarray(keys, dtype=np.float64)
    values = np.asarray(values, dtype=np.float64)
    n, n_head, hd = q.shape
    n_kv = keys.shape[1]
    group = n_head // n_kv
    out = np.zeros((n, n_head, hd))
    for t in range(n):
        vis = start + t + 1
        for h in range(n_head):
            kv = h // group
            s = keys[:vis, kv, :] @ q[t, h] * float(scale)
            w = np.exp(s - s.max())
            out[t, h] = (w / w.sum()) @ values[:vis, kv, :]
    return out.astype(np.float32)
