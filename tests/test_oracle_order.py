"""Pins the oracle's two summation orders bit for bit.

An independent restatement of the reference's CPU dot products in Python,
with every f32 operation rounded exactly once:

* mul and add are numpy float32 operations (IEEE single, correctly rounded);
* the FMA of ``_mm256_fmadd_ps`` is formed exactly as a rational number and
  rounded to the nearest f32 (ties to even) by integer arithmetic, so there is
  no double rounding through f64.

The orders restated (apps/engine/src/quant.rs):
* ``dot_q8_0_avx2`` (54-78): per block, eight lane accumulators; chunk c adds
  fma(q[8c+j], x[8c+j], acc[j]); ``horizontal_sum`` (80-91) is
  ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)); total += d * hsum;
* ``dot_q8_0_scalar`` (39-52): sum += q_i * x_i left to right; total += d * sum;
* ``dot_q8_0_q8_0_avx2`` (156-181): lane i holds the exact integer sum of
  products 4i..4i+3 (maddubs, then madd with ones); acc[i] = fma(d_w * s_x,
  f32(lane_i), acc[i]) over all blocks; one final horizontal_sum;
* the scalar q8 x q8 loop (142-153): total += (d_w * s_x) * f32(isum).

Random inputs make every rounding matter, so a swapped lane pairing, a
transposed chunk order, a contracted multiply-add or a dropped term changes
the bits and fails here.
"""
from fractions import Fraction

import numpy as np
import pytest

import oracle

F32 = np.float32


def round_f32(v: Fraction) -> F32:
    """Nearest f32 to an exact rational (ties to even, gradual underflow)."""
    if v == 0:
        return F32(0.0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    # now 2**e <= a < 2**(e+1); f32 keeps 24 bits, subnormals a fixed 2**-149 step
    ulp_exp = max(e - 23, -149)
    scaled = a / (Fraction(2) ** ulp_exp)
    m = scaled.numerator // scaled.denominator
    rem = scaled - m
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and m % 2 == 1):
        m += 1
    return F32(sign * m * 2.0 ** ulp_exp)


def fma(a, b, c) -> F32:
    return round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def hsum(lanes):
    """horizontal_sum: low + high, then two hadds."""
    s = [F32(lanes[j]) + F32(lanes[j + 4]) for j in range(4)]
    return (s[0] + s[1]) + (s[2] + s[3])


def split(row: np.ndarray):
    blocks = row.reshape(-1, 34)
    d = blocks[:, 0:2].copy().view(np.float16).astype(np.float32).reshape(-1)
    q = blocks[:, 2:].copy().view(np.int8).astype(np.int64)
    return d, q


def dot_avx2(row, x, lane_sum=hsum):
    d, q = split(row)
    total = F32(0.0)
    for b in range(len(d)):
        acc = [F32(0.0)] * 8
        for c in range(4):
            for j in range(8):
                acc[j] = fma(F32(q[b, 8 * c + j]), x[32 * b + 8 * c + j], acc[j])
        total = total + F32(d[b]) * lane_sum(acc)
    return total


def dot_scalar(row, x):
    d, q = split(row)
    total = F32(0.0)
    for b in range(len(d)):
        s = F32(0.0)
        for i in range(32):
            s = s + F32(q[b, i]) * x[32 * b + i]
        total = total + F32(d[b]) * s
    return total


def dot_q8q8_avx2(row, quants, scales):
    d, q = split(row)
    acc = [F32(0.0)] * 8
    for b in range(len(d)):
        prod = q[b] * quants[32 * b:32 * b + 32].astype(np.int64)
        combined = F32(d[b]) * F32(scales[b])
        for i in range(8):
            lane = int(prod[4 * i:4 * i + 4].sum())
            acc[i] = fma(combined, F32(lane), acc[i])
    return hsum(acc)


def dot_q8q8_scalar(row, quants, scales):
    d, q = split(row)
    total = F32(0.0)
    for b in range(len(d)):
        isum = int((q[b] * quants[32 * b:32 * b + 32].astype(np.int64)).sum())
        total = total + (F32(d[b]) * F32(scales[b])) * F32(isum)
    return total


def bits(v) -> int:
    return int(np.array([v], np.float32).view(np.uint32)[0])


def needs_avx2(order):
    if order == "avx2" and oracle.simd_path() != "avx2+fma":
        pytest.skip("host has no AVX2+FMA: the reference dispatches to the scalar order")


def test_round_f32_matches_numpy_where_f64_is_exact():
    r = np.random.default_rng(7)
    for v in r.standard_normal(200) * 10.0 ** r.integers(-40, 30, 200):
        assert bits(round_f32(Fraction(float(v)))) == bits(F32(v))
    # a tie rounds to even, and the smallest subnormal survives
    assert float(round_f32(Fraction(1) + Fraction(1, 2 ** 24))) == 1.0
    assert float(round_f32(Fraction(1) + Fraction(3, 2 ** 24))) == 1.0 + 2.0 ** -22
    assert float(round_f32(Fraction(1, 2 ** 149))) == 2.0 ** -149


@pytest.mark.parametrize("order", ["avx2", "scalar"])
@pytest.mark.parametrize("k,seed", [(32, 0), (256, 1), (2304, 2)])
def test_dot_q8_0_order_is_bit_exact(order, k, seed):
    needs_avx2(order)
    r = np.random.default_rng(0x5EED + seed)
    rows = 4 if k == 2304 else 12
    data = oracle.make_q8_weight(r, rows, k).reshape(rows, -1)
    x = r.standard_normal(k).astype(np.float32) * np.float32(3.0)
    restated = dot_avx2 if order == "avx2" else dot_scalar
    for o in range(rows):
        got = oracle.dot_q8_0(data[o], x, order)
        assert bits(got) == bits(restated(data[o], x)), f"row {o}"


@pytest.mark.parametrize("order", ["avx2", "scalar"])
@pytest.mark.parametrize("k,seed", [(64, 3), (2304, 4)])
def test_dot_q8_0_q8_0_order_is_bit_exact(order, k, seed):
    needs_avx2(order)
    r = np.random.default_rng(0x5EED + seed)
    rows = 6
    data = oracle.make_q8_weight(r, rows, k).reshape(rows, -1)
    x = oracle.make_activations(r, 1, k, outlier_rate=0.01).reshape(-1)
    quants, scales = oracle.quantize_q8_0(x)
    restated = dot_q8q8_avx2 if order == "avx2" else dot_q8q8_scalar
    for o in range(rows):
        got = oracle.dot_q8_0_q8_0(data[o], quants, scales, order)
        assert bits(got) == bits(restated(data[o], quants, scales)), f"row {o}"


def test_a_planted_order_change_is_caught():
    """The restatement is sensitive: pairing the lanes (l0+l1)+(l2+l3) instead
    of the hadd order changes the bits on random data, so the bit-exact tests
    above would see such a slip in the oracle."""
    r = np.random.default_rng(0x5EED + 9)
    data = oracle.make_q8_weight(r, 8, 256).reshape(8, -1)
    x = r.standard_normal(256).astype(np.float32)

    def paired(lanes):
        return ((F32(lanes[0]) + F32(lanes[1])) + (F32(lanes[2]) + F32(lanes[3]))) + \
               ((F32(lanes[4]) + F32(lanes[5])) + (F32(lanes[6]) + F32(lanes[7])))

    assert sum(bits(dot_avx2(data[o], x, paired)) != bits(dot_avx2(data[o], x)) for o in range(8)) > 0
