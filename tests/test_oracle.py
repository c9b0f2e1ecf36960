"""Pins the CPU oracle (oracle/q8_oracle.c) before it is trusted as the checker.

Every check here is independent of the oracle's own formula: the reference's
known-answer tests (apps/engine/tests/quant_q8.rs, matmul.rs, ops.rs), closed
forms (IEEE binary16 decode, exact integer arithmetic with power-of-two
scales), brute force in Python integers, and invariants (round-to-nearest
reconstruction bound, thread-count independence).
"""
import math

import numpy as np
import pytest

import oracle

RNG_SEED = 0x5EED


def block(scale: float, quants) -> np.ndarray:
    """quant_q8_q8.rs:6-11: [f16 LE scale][32 x i8]."""
    out = np.zeros(34, dtype=np.uint8)
    out[0:2] = np.array([scale], dtype=np.float16).view(np.uint8)
    out[2:] = np.asarray(quants, dtype=np.int8).view(np.uint8)
    return out


# ---- f16 decode: all 65536 patterns against numpy's IEEE conversion ----

def test_f16_decode_is_exact_for_every_bit_pattern():
    bits = np.arange(65536, dtype=np.uint32)
    expected = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(expected)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), expected[~nan].view(np.uint32))


def test_f16_subnormal_scales_decode_to_mantissa_times_2_pow_minus_24():
    for m in (1, 2, 3, 511, 1023):
        assert oracle.f16_to_f32(m) == m * 2.0 ** -24
        assert oracle.f16_to_f32(0x8000 | m) == -m * 2.0 ** -24


# ---- quant_q8.rs KATs, for both summation orders ----

@pytest.mark.parametrize("order", ["scalar", "avx2"])
def test_dot_matches_f64_reference(order):
    """quant_q8.rs:13-33."""
    if order == "avx2" and oracle.simd_path() != "avx2+fma":
        pytest.skip("host has no AVX2+FMA")
    quants = [i - 16 for i in range(32)]
    row = block(0.5, quants)
    x = np.array([i * 0.125 - 1.0 for i in range(32)], dtype=np.float32)
    expected = sum(q * float(v) for q, v in zip(quants, x)) * 0.5
    actual = oracle.dot_q8_0(row, x, order)
    assert abs(float(actual) - expected) < 1e-4


@pytest.mark.parametrize("order", ["scalar", "avx2", "dispatch"])
def test_dot_spans_multiple_blocks_with_per_block_scale(order):
    """quant_q8.rs:35-44: 0.25*32 + 2.0*32 = 72."""
    if order == "avx2" and oracle.simd_path() != "avx2+fma":
        pytest.skip("host has no AVX2+FMA")
    row = np.concatenate([block(0.25, [1] * 32), block(2.0, [1] * 32)])
    x = np.ones(64, dtype=np.float32)
    assert abs(float(oracle.dot_q8_0(row, x, order)) - 72.0) < 1e-4
    # every partial sum is an exact small binary fraction, so all orders are exact
    assert float(oracle.dot_q8_0(row, x, order)) == 72.0


def test_dequant_row_round_trips_through_dot():
    """quant_q8.rs:46-63."""
    quants = [3 if i % 2 == 0 else -7 for i in range(32)]
    row = block(1.5, quants)
    values = oracle.dequant_q8_0(row, 32)
    expected = np.float32(sum(np.float32(q * 1.5) for q in quants))
    assert abs(float(values.sum(dtype=np.float32)) - float(expected)) < 1e-4
    assert abs(float(oracle.dot_q8_0(row, values)) - float((values * values).sum())) < 1e-2


@pytest.mark.parametrize("order", ["scalar", "avx2"])
def test_dot_is_exact_on_exactly_representable_data(order):
    """Power-of-two scales and small integer activations make every product
    and partial sum exact, so any correct order equals the integer closed form;
    a dropped term, a sign slip or a transposed operand does not."""
    if order == "avx2" and oracle.simd_path() != "avx2+fma":
        pytest.skip("host has no AVX2+FMA")
    rng = np.random.default_rng(RNG_SEED)
    blocks = 9
    qs = rng.integers(-127, 128, size=(blocks, 32))
    exps = rng.integers(-12, 3, size=blocks)
    row = np.concatenate([block(2.0 ** int(e), q) for e, q in zip(exps, qs)])
    x = rng.integers(-8, 9, size=blocks * 32).astype(np.float32)
    exact = sum(2.0 ** int(exps[b]) * int(np.dot(qs[b], x[b * 32:(b + 1) * 32].astype(np.int64)))
                for b in range(blocks))
    assert float(oracle.dot_q8_0(row, x, order)) == exact


def test_dot_orders_agree_with_f64_on_random_rows():
    rng = np.random.default_rng(RNG_SEED + 1)
    k = 2304
    row = oracle.make_q8_weight(rng, 1, k)
    x = rng.standard_normal(k, dtype=np.float32)
    deq = oracle.dequant_q8_0(row, k).astype(np.float64)
    ref = float(np.dot(deq, x.astype(np.float64)))
    mag = float(np.abs(deq * x).sum())
    for order in ("scalar", "avx2"):
        if order == "avx2" and oracle.simd_path() != "avx2+fma":
            continue
        assert abs(float(oracle.dot_q8_0(row, x, order)) - ref) <= 1e-6 * mag


# ---- quantize_q8_0 closed forms ----

def test_quantize_all_zero_block_gives_zero_scale_and_quants():
    q, s = oracle.quantize_q8_0(np.zeros(64, dtype=np.float32))
    assert np.all(q == 0) and np.all(s == 0)


def test_quantize_rounds_half_away_from_zero():
    """peak = 127 makes inverse exactly 1.0, so v*inverse = v: 2.5 -> 3,
    -2.5 -> -3, 0.5 -> 1, -0.5 -> -1 (banker's rounding would give 2, -2, 0, 0)."""
    x = np.zeros(32, dtype=np.float32)
    x[0] = 127.0
    x[1:5] = [2.5, -2.5, 0.5, -0.5]
    x[5:8] = [1.49999988, -126.5, 126.5]
    q, s = oracle.quantize_q8_0(x)
    assert s[0] == np.float32(1.0)
    assert list(q[:8]) == [127, 3, -3, 1, -1, 1, -127, 127]


def test_quantize_peak_maps_to_127_and_reconstructs_within_half_a_step():
    rng = np.random.default_rng(RNG_SEED + 2)
    x = oracle.make_activations(rng, 4, 2304, outlier_rate=0.01)
    q, s = oracle.quantize_q8_0(x)
    xb = x.reshape(-1, 32)
    qb = q.reshape(-1, 32).astype(np.float64)
    peak = np.abs(xb).max(axis=1)
    assert np.array_equal(s, (peak / np.float32(127.0)).astype(np.float32))
    arg = np.abs(xb).argmax(axis=1)
    assert np.all(np.abs(qb[np.arange(len(arg)), arg]) == 127)
    step = s.astype(np.float64)[:, None]
    assert np.all(np.abs(xb - qb * step) <= 0.5 * step * (1 + 1e-5) + 1e-30)


def test_quantize_ignores_nan_in_the_peak_and_maps_it_to_zero():
    x = np.zeros(32, dtype=np.float32)
    x[0] = np.nan
    x[1] = -4.0
    x[2] = 2.0
    q, s = oracle.quantize_q8_0(x)
    assert s[0] == np.float32(4.0) / np.float32(127.0)
    assert q[0] == 0 and q[1] == -127 and q[2] == 64  # 2*127/4 = 63.5 -> 64


# ---- dot_q8_0_q8_0: the int32 block dot and the f32 epilogue ----

def test_block_dot_is_the_brute_force_integer_sum():
    rng = np.random.default_rng(RNG_SEED + 3)
    row = oracle.make_q8_weight(rng, 1, 32 * 6)
    quants = rng.integers(-128, 128, size=32 * 6).astype(np.int8)
    w = row.reshape(6, 34)[:, 2:].view(np.int8).astype(np.int64)
    for b in range(6):
        expect = int(sum(int(a) * int(c) for a, c in zip(w[b], quants[b * 32:(b + 1) * 32])))
        assert oracle.block_dot_i64(row, quants, b) == expect
        assert abs(expect) <= 32 * 128 * 127  # fits i32 with room


@pytest.mark.parametrize("order", ["scalar", "avx2"])
def test_int8_dot_is_exact_on_power_of_two_scales(order):
    if order == "avx2" and oracle.simd_path() != "avx2+fma":
        pytest.skip("host has no AVX2+FMA")
    rng = np.random.default_rng(RNG_SEED + 4)
    blocks = 7
    qw = rng.integers(-127, 128, size=(blocks, 32))
    ew = rng.integers(-10, 2, size=blocks)
    row = np.concatenate([block(2.0 ** int(e), q) for e, q in zip(ew, qw)])
    qx = rng.integers(-127, 128, size=blocks * 32).astype(np.int8)
    ex = rng.integers(-8, 1, size=blocks)
    sx = np.array([2.0 ** int(e) for e in ex], dtype=np.float32)
    exact = sum(2.0 ** int(ew[b] + ex[b]) * int(np.dot(qw[b], qx[b * 32:(b + 1) * 32].astype(np.int64)))
                for b in range(blocks))
    assert float(oracle.dot_q8_0_q8_0(row, qx, sx, order)) == exact


def test_int8_dot_orders_agree_with_f64():
    rng = np.random.default_rng(RNG_SEED + 5)
    k = 5760
    row = oracle.make_q8_weight(rng, 1, k)
    x = oracle.make_activations(rng, 1, k, outlier_rate=0.01)
    qx, sx = oracle.quantize_q8_0(x)
    w = row.reshape(-1, 34)
    d = w[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(-1)
    iq = np.array([oracle.block_dot_i64(row, qx, b) for b in range(k // 32)], dtype=np.float64)
    ref = float(np.sum(d * sx.astype(np.float64) * iq))
    mag = float(np.sum(np.abs(d * sx.astype(np.float64) * iq)))
    for order in ("scalar", "avx2"):
        if order == "avx2" and oracle.simd_path() != "avx2+fma":
            continue
        assert abs(float(oracle.dot_q8_0_q8_0(row, qx, sx, order)) - ref) <= 1e-6 * mag


# ---- tensor::matmul (matmul.rs KATs) ----

K, OUT = 32, 4


def quantized_matrix() -> np.ndarray:
    """matmul.rs:74-88."""
    rows = []
    for o in range(OUT):
        q = [((o * 7 + i * 3) % 21) - 10 for i in range(K)]
        rows.append(block(0.125 * (o + 1.0), q))
    return np.concatenate(rows)


def activations(n: int) -> np.ndarray:
    """matmul.rs:107-109: sin(0.017 i) in f32."""
    return np.sin(np.arange(n * K, dtype=np.float32) * np.float32(0.017)).astype(np.float32)


def reference(data, x, n):
    """matmul.rs:90-105 (f64 naive on f32 activations)."""
    y = np.zeros(n * OUT, dtype=np.float32)
    for t in range(n):
        for o in range(OUT):
            base = o * 34
            scale = float(data[base:base + 2].copy().view(np.float16)[0])
            s = sum(float(np.int8(data[base + 2 + i].astype(np.int8))) * float(x[t * K + i]) for i in range(K))
            y[t * OUT + o] = np.float32(scale * s)
    return y


def quantized_reference(data, x, n):
    """matmul.rs:114-137 (f64 over the quantized activations)."""
    y = np.zeros(n * OUT, dtype=np.float32)
    for t in range(n):
        quants, scales = oracle.quantize_q8_0(x[t * K:(t + 1) * K])
        for o in range(OUT):
            base = o * 34
            scale = float(data[base:base + 2].copy().view(np.float16)[0])
            inner = sum(int(data[base + 2 + i].astype(np.int8)) * int(quants[i]) for i in range(K))
            y[t * OUT + o] = np.float32(scale * inner * float(scales[0]))
    return y


def test_decode_step_matches_reference():
    """matmul.rs:139-152."""
    data = quantized_matrix()
    x = activations(1)
    y = oracle.matmul(data, K, OUT, x, 1).reshape(-1)
    assert np.all(np.abs(y - reference(data, x, 1)) < 1e-3)


def test_prefill_batch_matches_reference():
    """matmul.rs:154-168."""
    data = quantized_matrix()
    n = 5
    x = activations(n)
    y = oracle.matmul(data, K, OUT, x, n).reshape(-1)
    assert np.all(np.abs(y - quantized_reference(data, x, n)) < 1e-3)


def test_batch_and_single_agree_up_to_activation_quantization():
    """matmul.rs:170-198."""
    data = quantized_matrix()
    n = 3
    x = activations(n)
    batched = oracle.matmul(data, K, OUT, x, n)
    for t in range(n):
        single = oracle.matmul(data, K, OUT, x[t * K:(t + 1) * K], 1).reshape(-1)
        tol = 0.02 * max(float(np.abs(single).max()), 1.0)
        assert np.all(np.abs(single - batched[t]) < tol)


@pytest.mark.parametrize("n", [1, 2, 9])
def test_matmul_is_independent_of_the_thread_count(n):
    """tensor.rs:127-148: every element is computed by one thread, no
    cross-thread reduction, so results are bit-identical for any split."""
    rng = np.random.default_rng(RNG_SEED + 6)
    k, out = 256, 37
    data = oracle.make_q8_weight(rng, out, k)
    x = oracle.make_activations(rng, n, k)
    a = oracle.matmul(data, k, out, x, n, threads=1)
    b = oracle.matmul(data, k, out, x, n, threads=7)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_matmul_rows_match_the_row_dot():
    rng = np.random.default_rng(RNG_SEED + 7)
    k, out, n = 128, 5, 3
    data = oracle.make_q8_weight(rng, out, k)
    x = oracle.make_activations(rng, n, k)
    y = oracle.matmul(data, k, out, x, n)
    rows = data.reshape(out, -1)
    for t in range(n):
        qx, sx = oracle.quantize_q8_0(x[t])
        for o in range(out):
            assert y[t, o] == oracle.dot_q8_0_q8_0(rows[o], qx, sx)
    y1 = oracle.matmul(data, k, out, x[0], 1).reshape(-1)
    for o in range(out):
        assert y1[o] == oracle.dot_q8_0(rows[o], x[0])


# ---- ops and argmax ----

def test_silu_matches_reference_points():
    """ops.rs tests: silu(0)=0, silu(1)=0.7310586, silu(-1)=-0.2689414."""
    assert abs(float(oracle.silu(0.0))) < 1e-6
    assert abs(float(oracle.silu(1.0)) - 0.7310586) < 1e-6
    assert abs(float(oracle.silu(-1.0)) + 0.2689414) < 1e-6
    for v in (-20.0, -3.0, 0.5, 7.0):
        assert abs(float(oracle.silu(v)) - v / (1 + math.exp(-v))) <= 2e-7 * max(1.0, abs(v))


def test_rmsnorm_matches_reference_points():
    """ops.rs tests: mean square 7.5, and the weight applied after the norm."""
    out = oracle.rmsnorm(np.array([1, 2, 3, 4], np.float32), np.ones(4, np.float32), 0.0)
    scale = 1.0 / math.sqrt(7.5)
    assert np.all(np.abs(out - np.array([1, 2, 3, 4]) * scale) < 1e-6)
    out = oracle.rmsnorm(np.array([2, 2], np.float32), np.array([3, 0.5], np.float32), 0.0)
    assert abs(out[0] - 3.0) < 1e-6 and abs(out[1] - 0.5) < 1e-6


def test_argmax_takes_the_first_strictly_greatest():
    assert oracle.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    assert oracle.argmax(np.array([-1, -1], np.float32)) == 0
    assert oracle.argmax(np.array([0, np.nan, 5, 5], np.float32)) == 2
    assert oracle.argmax(np.array([np.nan, 1, 9], np.float32)) == 0


# ---- rope (ops.rs:120-166) ----

def test_rope_position_zero_is_identity_and_pairs_keep_their_norm():
    rng = np.random.default_rng(RNG_SEED)
    x = rng.standard_normal((5, 3, 64)).astype(np.float32)
    y = oracle.rope(x, 0, 64, 10000.0)
    assert np.array_equal(y[0], x[0])  # angle 0: cos 1, sin 0 exactly
    norm_x = np.hypot(x[..., 0::2].astype(np.float64), x[..., 1::2])
    norm_y = np.hypot(y[..., 0::2].astype(np.float64), y[..., 1::2])
    assert np.allclose(norm_x, norm_y, rtol=1e-6, atol=1e-7)


def test_rope_hand_value_and_partial_rotation():
    # pair 0 rotates by exactly `position` radians (base^0 = 1); pair 1 of a
    # 4-dim rotary span by position * base^(-1/2)
    x = np.zeros((1, 1, 8), np.float32)
    x[0, 0, :] = [1, 0, 0, 1, 5, 6, 7, 8]
    y = oracle.rope(x, 3, 4, 100.0)
    assert np.allclose(y[0, 0, 0:2], [np.cos(3.0), np.sin(3.0)], atol=1e-6)
    a = 3.0 * 100.0 ** -0.5
    assert np.allclose(y[0, 0, 2:4], [-np.sin(a), np.cos(a)], atol=1e-6)
    assert np.array_equal(y[0, 0, 4:], x[0, 0, 4:])  # past n_rot: untouched


def test_rope_rotations_compose():
    rng = np.random.default_rng(RNG_SEED + 1)
    x = rng.standard_normal((1, 2, 64)).astype(np.float32)
    once = oracle.rope(x, 7, 64, 10000.0)
    # rotating position 3 then by 4 more equals position 7, to f32 rounding
    twice = oracle.rope(oracle.rope(x, 3, 64, 10000.0), 4, 64, 10000.0)
    assert np.allclose(once, twice, atol=2e-5)
    with pytest.raises(AssertionError):  # a sign slip in the rotation fails this
        bad = x.copy()
        bad[..., 1::2] *= -1
        assert np.allclose(oracle.rope(bad, 7, 64, 10000.0), once, atol=2e-5)


# ---- attention (compute.rs:1075-1126) ----

def test_attention_single_key_returns_its_value():
    rng = np.random.default_rng(RNG_SEED + 2)
    q = rng.standard_normal((1, 4, 64)).astype(np.float32)
    k = rng.standard_normal((1, 2, 64)).astype(np.float32)
    v = rng.standard_normal((1, 2, 64)).astype(np.float32)
    out = oracle.attention(q, k, v, 0, 0.125)
    for h in range(4):
        assert np.allclose(out[0, h], v[0, h // 2], atol=1e-7)


def test_attention_equal_keys_average_and_dominant_key_wins():
    rng = np.random.default_rng(RNG_SEED + 3)
    L = 9
    q = rng.standard_normal((1, 1, 64)).astype(np.float32)
    k = np.repeat(rng.standard_normal((1, 1, 64)).astype(np.float32), L, axis=0)
    v = rng.standard_normal((L, 1, 64)).astype(np.float32)
    out = oracle.attention(q, k, v, L - 1, 0.125)
    assert np.allclose(out[0, 0], v[:, 0].astype(np.float64).mean(axis=0), atol=1e-6)
    k2 = rng.standard_normal((L, 1, 64)).astype(np.float32) * 0.01
    k2[4, 0] = q[0, 0] * 100.0  # score ~ 100 * |q|^2 * 0.125 above the rest
    out2 = oracle.attention(q, k2, v, L - 1, 0.125)
    assert np.allclose(out2[0, 0], v[4, 0], atol=1e-6)


def test_attention_is_causal_and_convex():
    rng = np.random.default_rng(RNG_SEED + 4)
    n, L = 6, 6
    q = rng.standard_normal((n, 2, 64)).astype(np.float32)
    k = rng.standard_normal((L, 2, 64)).astype(np.float32)
    v = rng.standard_normal((L, 2, 64)).astype(np.float32)
    full = oracle.attention(q, k, v, 0, 0.125)
    for t in range(n):  # row t only sees keys 0..t
        part = oracle.attention(q[t:t + 1], k[:t + 1], v[:t + 1], t, 0.125)
        assert np.allclose(full[t], part[0], atol=1e-6)
    # a larger scale sharpens but the row still sums the same values convexly
    sharp = oracle.attention(q, k, v, 0, 10.0)
    lo, hi = v.min(axis=0), v.max(axis=0)
    assert np.all(sharp >= lo[None] - 1e-5) and np.all(sharp <= hi[None] + 1e-5)


def test_rope_frequency_is_the_correctly_rounded_powf():
    # the frequency of pair 1 at base 1e4 over 64 dims: 10000^(-1/32) =
    # 0.74989420933..., whose nearest f32 is 0.7498942 (numpy's float32 power
    # returns the next one up, 0.74989426; a position of 511 turns that ulp
    # into a 3e-5 error in the rotated value)
    import math
    exact = math.exp(-math.log(10000.0) / 32)
    nearest = np.float32(exact)
    assert abs(float(nearest) - exact) < abs(float(np.nextafter(nearest, np.float32(1))) - exact)
    x = np.zeros((512, 1, 64), np.float32)
    x[:, 0, 2] = 1.0
    y = oracle.rope(x, 0, 64, 10000.0)
    angle = np.float32(511) * nearest
    assert y[511, 0, 2] == np.float32(np.cos(np.float64(angle)))
