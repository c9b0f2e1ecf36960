"""GPU parity of the HIP Q8_0 path against the CPU oracle, through the C-ABI.

Bars (the path's parity targets):
  * integer/byte work bit-exact: the device weight layout (round trip), the
    quantized activations (q and scales), the int32 block dot;
  * f32 outputs within |d| <= 2e-6 + 1e-5*|ref| (TOL_ABS, TOL_REL below);
  * n = 1 with gemv.exact = 1: bit-identical to the reference's AVX2 order
    when the host oracle takes that order (it does on AVX2+FMA hosts);
  * lm_head: identical argmax.
"""
import ctypes
import math

import numpy as np
import pytest

import oracle
from llm_amd import q8

pytestmark = pytest.mark.gpu

TOL_ABS = 2e-6
TOL_REL = 1e-5
SEED = 0x5EED
J = [[0, 4, 1, 5], [2, 6, 3, 7]]
OPTIONS = ("gemv.exact", "gemv.waves", "gemv.pairs", "gemv.slices", "gemv.rows", "gemv.loads", "gemv.xcd_order", "gemm.smode", "gemm.tpw", "gemm.twaves",
           "gemm.xcd_remap", "gemm.kwaves", "gemm.slices", "gemm.rwaves", "gemm.f16", "gemm.pipe", "gemm.lds",
           "gemm.silu", "gemm.small_gemv", "gemm.stream", "gemv.slice_copy")


def assert_close(got, ref, what):
    got = np.asarray(got, np.float32)
    ref = np.asarray(ref, np.float32)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} vs {ref.shape}"
    d = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bound = TOL_ABS + TOL_REL * np.abs(ref.astype(np.float64))
    bad = ~(d <= bound)
    if bad.any():
        i = int(np.flatnonzero(bad.reshape(-1))[0])
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outside tolerance; max|d| = "
                             f"{float(np.nanmax(d)):.3e}; first at {i}: got {got.reshape(-1)[i]!r} "
                             f"ref {ref.reshape(-1)[i]!r}")


def exact_matmul(wdata, k, out, x, n):
    """The exact value of the n >= 2 product the reference rounds: the
    reference quantization of x (oracle), integer block dots, and the f32
    scale product d_w*s_x, all summed in f64 (tensor.rs:104-140)."""
    nb = k // 32
    raw = np.asarray(wdata, np.uint8).reshape(out, nb, 34)
    d = raw[:, :, 0:2].copy().view(np.float16).astype(np.float32).reshape(out, nb)
    qw = raw[:, :, 2:].copy().view(np.int8).astype(np.float64)
    x = np.asarray(x, np.float32).reshape(n, k)
    y = np.zeros((n, out))
    for t in range(n):
        qx, sx = oracle.quantize_q8_0(x[t])
        blk = np.einsum("onk,nk->on", qw, qx.reshape(nb, 32).astype(np.float64))
        comb = (d * sx[None, :]).astype(np.float32).astype(np.float64)  # d_w*s_x rounded to f32, as the reference
        y[t] = (blk * comb).sum(axis=1)
    return y


CLAUSE_LOG = []  # (what, outputs that used the accuracy clause, outputs checked); printed in the summary


def exact_at(wdata, k, out, x=None, n=None, quants=None, scales=None):
    """A function of flat output indices t*out + o giving the exact value of
    the n >= 2 product there (f64 sum of the integer block dots times the f32
    scale products d_w*s_x) and the sum of the block terms' magnitudes, for
    assert_parity on shapes where the whole exact product is too slow in
    numpy.  The activations come as f32 x (the
    reference quantization is applied, quantize_q8_0) or already quantized
    (quants [n, k] int8, scales [n, k/32] f32)."""
    nb = k // 32
    raw = np.asarray(wdata, np.uint8).reshape(out, nb, 34)
    if quants is None:
        x = np.asarray(x, np.float32).reshape(n, k)

    def token(t):
        if quants is not None:
            return np.asarray(quants[t], np.int64).reshape(nb, 32), np.asarray(scales[t], np.float32)
        qx, sx = oracle.quantize_q8_0(x[t])
        return qx.astype(np.int64).reshape(nb, 32), sx

    def at(flat):
        flat = np.asarray(flat, np.int64).reshape(-1)
        res = np.empty(flat.size)
        mag = np.empty(flat.size)
        tok, row = flat // out, flat % out
        for t in np.unique(tok):
            sel = np.flatnonzero(tok == t)
            o = row[sel]
            qx, sx = token(int(t))
            d = raw[o, :, 0:2].copy().view(np.float16).astype(np.float32).reshape(o.size, nb)
            qw = raw[o, :, 2:].copy().view(np.int8).astype(np.int64)
            blk = (qw * qx[None]).sum(axis=2)
            comb = (d * sx[None, :]).astype(np.float32).astype(np.float64)  # d_w*s_x rounded to f32
            terms = blk * comb
            res[sel] = terms.sum(axis=1)
            mag[sel] = np.abs(terms).sum(axis=1)
        return res, mag
    return at


U32 = 2.0 ** -24  # f32 unit roundoff


def assert_parity(got, ref, exact, what, max_frac=1e-3):
    """n >= 2 bar: |got - ref| <= 2e-6 + 1e-5|ref|.  Where two f32 sums of the
    same block terms in different orders differ by more than that (the
    reference's own error reaches 2.9e-6 at K = 5760 with outliers, and sums
    that cancel -- terms adding up to 15.8 in magnitude for a result of 0.02
    -- carry errors of a few roundings at the scale of the terms), an output
    passes the accuracy clause instead if its error against the exact value is
    at most twice the reference's own, or at most 4 u T, where T is the sum of
    the block terms' magnitudes and u = 2^-24: the error of four f32 roundings
    at the size of the terms (the textbook bound for a sum of nb terms is
    (nb - 1) u T).  At most `max_frac` of the outputs may need the clause.
    `exact` is the exact product (array; T is then not used) or a function of
    flat indices returning (exact, T) (exact_at), evaluated only where the
    first clause fails."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float32).astype(np.float64)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} vs {ref.shape}"
    within = np.abs(got - ref) <= TOL_ABS + TOL_REL * np.abs(ref)
    idx = np.flatnonzero(~within.reshape(-1))
    if idx.size:
        g, r = got.reshape(-1)[idx], ref.reshape(-1)[idx]
        if callable(exact):
            e, mag = exact(idx)
        else:
            e, mag = np.asarray(exact, np.float64).reshape(-1)[idx], np.zeros(idx.size)
        err = np.abs(g - e)
        no_worse = (err <= 2.0 * np.abs(r - e)) | (err <= 4.0 * U32 * mag)
        if not no_worse.all():
            i = int(np.flatnonzero(~no_worse)[0])
            raise AssertionError(f"{what}: {int((~no_worse).sum())} of {ref.size} outside tolerance and less "
                                 f"accurate than the reference; first at {int(idx[i])}: got {g[i]!r} ref {r[i]!r} "
                                 f"exact {e[i]!r} (term magnitudes {mag[i]:.4g})")
        print(f"{what}: {idx.size} outputs beyond the bar, each within the accuracy clause "
              f"(max error {float(err.max()):.3e}, max of 2|ref - exact| {float(2 * np.abs(r - e).max()):.3e})",
              flush=True)
    CLAUSE_LOG.append((what, int(idx.size), int(ref.size)))
    frac = idx.size / ref.size
    assert frac <= max_frac, f"{what}: {frac:.2e} of outputs needed the accuracy clause"


def assert_bits(got, ref, what):
    got = np.ascontiguousarray(got, np.float32)
    ref = np.ascontiguousarray(ref, np.float32)
    diff = got.view(np.uint32) != ref.view(np.uint32)
    if diff.any():
        i = int(np.flatnonzero(diff.reshape(-1))[0])
        raise AssertionError(f"{what}: {int(diff.sum())} of {diff.size} not bit-identical; first at {i}: "
                             f"got {got.reshape(-1)[i]!r} ref {ref.reshape(-1)[i]!r}")


@pytest.fixture(scope="module")
def gpu():
    g = q8.Gpu(0)
    print(f"\ndevice: {g.name}", flush=True)
    yield g
    g.close()


@pytest.fixture(autouse=True)
def default_options(gpu):
    """Each test starts from the defaults except gemv.exact = 1: the n = 1
    tests assert the reference's AVX2 bits, which the exact block order gives
    (the default sums blocks in a tree; tests that take `exact` set it, and
    test_gemv_default_order_is_within_the_bar covers the default)."""
    gpu.set_option("gemv.exact", 1)
    yield
    for name in OPTIONS:
        gpu.set_option(name, -1)


def rng(i=0):
    return np.random.default_rng(SEED + i)


def weight(r, out, k, **kw):
    return q8.Weight(oracle.make_q8_weight(r, out, k, **kw), k, out)


def run_matmul(gpu, w, x, n, bias=None):
    k, out = w.k, w.out
    xb = gpu.alloc(4 * n * k)
    yb = gpu.alloc(4 * n * out)
    xb.upload(x.astype(np.float32))
    bb = None
    if bias is not None:
        yb.upload(bias.astype(np.float32))
        bb = yb
    gpu.matmul(w, xb, 0, n, yb, 0, bias=bb)
    y = yb.download(np.float32, n * out).reshape(n, out)
    xb.free()
    yb.free()
    return y


def unpack_prepared(gpu, p, n, k):
    """Download a prepared buffer and undo the lane-order layout
    (llm_amd/csrc/q8_layout.h) into [n][k] int8 and [n][k/32] f32.  The f16
    format holds the same integers as f16: unit half u, lane L = bytes
    8u..8u+7 of lane L's 16-byte int8 slot."""
    nb = k // 32
    tt = (n + 31) // 32
    sraw = np.empty(tt * nb * 32, np.float32)
    q8._check(q8.lib().q8_download(gpu.handle, sraw.ctypes.data, p.scales, sraw.nbytes))
    if p.format == q8.PREPARED_F16:
        hraw = np.empty(tt * nb * 1024, np.float16)
        q8._check(q8.lib().q8_download(gpu.handle, hraw.ctypes.data, p.quants, hraw.nbytes))
        hv = hraw.astype(np.float32).reshape(tt, nb, 2, 64, 8)          # [tt][b][u][lane][8]
        assert np.array_equal(hv, np.round(hv)) and np.abs(hv).max(initial=0) <= 127, "f16 quants are integers"
        qraw = hv.transpose(0, 1, 3, 2, 4).reshape(tt, nb, 64, 16).astype(np.int8).view(np.uint8).reshape(-1)
    else:
        assert p.format == q8.PREPARED_I8
        qraw = np.empty(tt * nb * 1024, np.uint8)
        q8._check(q8.lib().q8_download(gpu.handle, qraw.ctypes.data, p.quants, qraw.nbytes))
    qv = qraw.view(np.int8).reshape(tt, nb, 2, 32, 16)
    out = np.zeros((tt, 32, nb, 32), np.int8)
    for h in range(2):
        for pp in range(16):
            e = 8 * (pp % 4) + J[h][pp // 4]
            out[:, :, :, e] = qv[:, :, h, :, pp].transpose(0, 2, 1)
    q = out.reshape(tt * 32, nb * 32)
    s = sraw.reshape(tt, nb, 32).transpose(0, 2, 1).reshape(tt * 32, nb)
    return q, s


# ---------------------------------------------------------------------------
# weight residency: the device tile layout is a byte-exact re-arrangement
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("out,k", [(1, 32), (4, 64), (33, 96), (100, 2304), (2304, 5760), (5760, 2304)])
def test_weight_layout_round_trips_byte_exact(gpu, out, k):
    w = weight(rng(1), out, k)
    back = gpu.export(w)
    assert np.array_equal(back, w.data)
    gpu.release(w)


@pytest.mark.parametrize("out,k", [(5760, 2304), (2304, 2304), (2304, 5760), (6912, 2304), (122880, 2304),
                                   (33, 96)])
def test_gemv_default_order_is_within_the_bar(gpu, out, k):
    """The default n = 1 path (the tactic's kernel, blocks summed in a fixed
    tree): within 2e-6 + 1e-5|ref| of the reference, the same bits run to run,
    and each row within a few roundings of the exact sum of its block values."""
    gpu.set_option("gemv.exact", -1)
    r = rng(20 + out % 97)
    w = weight(r, out, k)
    x = r.standard_normal(k, dtype=np.float32)
    ref = oracle.matmul(w.data, k, out, x, 1).reshape(-1)
    got = run_matmul(gpu, w, x, 1).reshape(-1)
    assert_close(got, ref, f"default gemv {out}x{k}")
    assert_bits(run_matmul(gpu, w, x, 1).reshape(-1), got, f"default gemv {out}x{k} rerun")
    gpu.release(w)


def test_weight_cache_is_keyed_by_identity(gpu):
    w = weight(rng(2), 64, 64)
    a = gpu.resident(w)
    b = gpu.resident(w)
    assert a == b
    w2 = q8.Weight(w.data.copy(), 64, 64)
    assert gpu.resident(w2) != a
    gpu.release(w)
    gpu.release(w2)


# ---------------------------------------------------------------------------
# n = 1 GEMV (tensor.rs:96-101)
# ---------------------------------------------------------------------------

def test_gemv_configs0_matches_the_reference_bit_for_bit(gpu):
    """W 5760 x 2304, x ~ N(0,1), y f32[5760]."""
    r = rng(10)
    w = weight(r, 5760, 2304)
    x = r.standard_normal(2304, dtype=np.float32)
    ref = oracle.matmul(w.data, 2304, 5760, x, 1).reshape(-1)
    got = run_matmul(gpu, w, x, 1).reshape(-1)
    assert_close(got, ref, "gemv configs[0]")
    if oracle.simd_path() == "avx2+fma":
        assert_bits(got, ref, "gemv configs[0] (AVX2 order)")
    gpu.release(w)


@pytest.mark.parametrize("out,k", [(1, 32), (4, 32), (33, 96), (64, 64), (100, 1056), (257, 2304),
                                   (2304, 5760), (96, 224)])
@pytest.mark.parametrize("exact", [1, 0])
def test_gemv_shapes(gpu, out, k, exact):
    gpu.set_option("gemv.exact", exact)
    r = rng(11 + out + k)
    w = weight(r, out, k)
    x = r.standard_normal(k, dtype=np.float32)
    ref = oracle.matmul(w.data, k, out, x, 1).reshape(-1)
    got = run_matmul(gpu, w, x, 1).reshape(-1)
    assert_close(got, ref, f"gemv {out}x{k} exact={exact}")
    if exact and oracle.simd_path() == "avx2+fma":
        assert_bits(got, ref, f"gemv {out}x{k}")
    gpu.release(w)


@pytest.mark.parametrize("slices,waves,pairs", [(1, 1, 9), (1, 2, 5), (1, 3, 3), (1, 4, 2), (1, 6, 2), (1, 8, 5),
                                                (2, 2, 3), (3, 1, 5), (5, 2, 2), (12, 1, 2), (7, 3, 9)])
@pytest.mark.parametrize("exact", [1, 0])
def test_gemv_launch_shapes_agree(gpu, slices, waves, pairs, exact):
    """Every (K slices, waves per slice, pairs per batch) split gives the same
    bits in exact mode, and stays within tolerance otherwise."""
    gpu.set_option("gemv.exact", exact)
    gpu.set_option("gemv.slices", slices)
    gpu.set_option("gemv.waves", waves)
    gpu.set_option("gemv.pairs", pairs)
    r = rng(12)
    w = weight(r, 320, 768)
    x = r.standard_normal(768, dtype=np.float32)
    ref = oracle.matmul(w.data, 768, 320, x, 1).reshape(-1)
    got = run_matmul(gpu, w, x, 1).reshape(-1)
    what = f"gemv slices={slices} waves={waves} pairs={pairs} exact={exact}"
    assert_close(got, ref, what)
    if exact and oracle.simd_path() == "avx2+fma":
        assert_bits(got, ref, what)
    gpu.release(w)


ROW_SLICES = [(8, 2), (8, 3), (8, 6), (16, 3), (16, 6)]


@pytest.mark.parametrize("exact", [1, 0])
@pytest.mark.parametrize("rows,loads", ROW_SLICES)
@pytest.mark.parametrize("out,k", [(1, 32), (33, 96), (100, 1056), (257, 2304), (5760, 2304), (2304, 5760),
                                   (96, 224), (40, 12288)])
def test_gemv_row_slices_match_the_reference(gpu, rows, loads, out, k, exact):
    """The row-slice GEMV (a workgroup per 8 or 16 rows of a tile, whole K).
    exact = 1 keeps the exact block order: bit-identical to dot_q8_0's AVX2
    path.  exact = 0 (q8_gemv_r*_e0) sums the same block values in a fixed
    tree: within the f32 bar, and equal run to run.  K = 12288 needs more
    than 16 waves at 8 rows x 3 loads, where the tile kernel takes over."""
    gpu.set_option("gemv.rows", rows)
    gpu.set_option("gemv.loads", loads)
    gpu.set_option("gemv.exact", exact)
    r = rng(40 + out + k)
    w = weight(r, out, k)
    x = r.standard_normal(k, dtype=np.float32)
    ref = oracle.matmul(w.data, k, out, x, 1).reshape(-1)
    got = run_matmul(gpu, w, x, 1).reshape(-1)
    what = f"gemv rows={rows} loads={loads} {out}x{k} exact={exact}"
    assert_close(got, ref, what)
    if exact and oracle.simd_path() == "avx2+fma":
        assert_bits(got, ref, what)
    if not exact:
        assert_bits(run_matmul(gpu, w, x, 1).reshape(-1), got, what + " rerun")
    gpu.release(w)


def device_bytes(gpu, w):
    k, out, nbytes = ctypes.c_int(), ctypes.c_int(), ctypes.c_size_t()
    handle = gpu.resident(w)
    assert q8.lib().q8_weight_shape(ctypes.c_void_p(handle), ctypes.byref(k), ctypes.byref(out),
                                    ctypes.byref(nbytes)) == q8.Q8_OK
    return nbytes.value


@pytest.mark.parametrize("exact", [1, 0])
@pytest.mark.parametrize("out,k,rows", [(5760, 2304, 8), (4096, 2304, 8), (2304, 5760, 16), (2304, 2304, 16),
                                        (257, 2304, 16)])
def test_gemv_slice_major_copy_matches_the_unit_layout(gpu, out, k, rows, exact):
    """A weight whose one-token GEMV runs in row slices keeps a slice-major
    copy of its quants (each slice's bytes in one run); the row-slice kernels
    read it by default and the unit layout with option gemv.slice_copy = 0, and
    give the same bits either way (residual included), within the bar of the
    oracle.  A weight made resident with the option at 0 has no copy: its
    device bytes are one copy of the quants fewer."""
    r = rng(70 + out + k)
    w = weight(r, out, k)
    x = r.standard_normal(k, dtype=np.float32)
    bias = r.standard_normal(out).astype(np.float32)
    assert q8.plan(1, out, k, gpu)["row_slice"] == rows
    gpu.set_option("gemv.exact", exact)
    try:
        got = run_matmul(gpu, w, x, 1, bias=bias).reshape(-1)
        ref = oracle.matmul(w.data, k, out, x, 1).reshape(-1) + bias
        assert_close(got, ref, f"slice-major {out}x{k} exact={exact}")
        gpu.set_option("gemv.slice_copy", 0)
        unit = run_matmul(gpu, w, x, 1, bias=bias).reshape(-1)
        assert_bits(got, unit, f"slice-major against unit layout {out}x{k} exact={exact}")
        with_copy = device_bytes(gpu, w)
        bare = weight(r, out, k)  # resident while the option is 0
        without = device_bytes(gpu, bare)
        assert_bits(run_matmul(gpu, bare, x, 1, bias=bias).reshape(-1),
                    run_matmul(gpu, bare, x, 1, bias=bias).reshape(-1), "no copy, rerun")
        quants = (out + 31) // 32 * (k // 32) * 1024
        assert quants <= with_copy - without < quants + 256, (with_copy, without, quants)
        gpu.release(bare)
    finally:
        gpu.set_option("gemv.slice_copy", -1)
        gpu.set_option("gemv.exact", -1)
        gpu.release(w)


@pytest.mark.parametrize("order,exact", [(0, 1), (1, 1), (1, 0)])
@pytest.mark.parametrize("rows,loads", ROW_SLICES)
@pytest.mark.parametrize("out", [1, 200, 520])
def test_gemv_row_slices_residual_subnormals_and_offsets(gpu, rows, loads, out, order, exact):
    """Residual epilogue (compute.rs:537-581), all-subnormal and zero scales,
    and x at a 4-byte offset, through the row-slice kernels (exact block order
    and the tree-sum variant)."""
    gpu.set_option("gemv.rows", rows)
    gpu.set_option("gemv.loads", loads)
    gpu.set_option("gemv.xcd_order", order)
    gpu.set_option("gemv.exact", exact)
    r = rng(60 + rows + loads + out)
    k = 2304
    scales = np.abs(r.standard_normal(out * k // 32)).astype(np.float32) * 1e-6
    scales[::7] = 0.0
    w = weight(r, out, k, scales=scales)
    x = r.standard_normal(k, dtype=np.float32)
    y0 = r.standard_normal(out, dtype=np.float32)
    xb, yb = gpu.alloc(4 * (k + 1)), gpu.alloc(4 * out)
    xb.upload(np.concatenate([np.full(1, np.nan, np.float32), x]))
    yb.upload(y0)
    gpu.matmul(w, xb, 1, 1, yb, 0, bias=yb)
    got = yb.download(np.float32, out)
    ref = y0 + oracle.matmul(w.data, k, out, x, 1).reshape(-1)
    what = f"gemv rows={rows} loads={loads} out={out} xcd_order={order} exact={exact} residual"
    assert_close(got, ref, what)
    if exact and oracle.simd_path() == "avx2+fma":
        assert_bits(got, ref, what)
    xb.free()
    yb.free()
    gpu.release(w)


def test_gemv_subnormal_and_special_scales(gpu):
    r = rng(13)
    out, k = 64, 256
    blocks = out * k // 32
    scales = np.abs(r.standard_normal(blocks)).astype(np.float32) * 1e-6  # all f16 subnormal
    scales[::7] = 0.0
    scales[1::11] = 6e-8  # the smallest subnormal
    w = weight(r, out, k, scales=scales)
    x = r.standard_normal(k, dtype=np.float32)
    ref = oracle.matmul(w.data, k, out, x, 1).reshape(-1)
    got = run_matmul(gpu, w, x, 1).reshape(-1)
    assert_close(got, ref, "gemv subnormal scales")
    if oracle.simd_path() == "avx2+fma":
        assert_bits(got, ref, "gemv subnormal scales")
    gpu.release(w)


def test_gemv_residual_epilogue_is_matmul_add(gpu):
    """compute.rs:537-581: y += W x, the add fused in the epilogue."""
    r = rng(14)
    w = weight(r, 2304, 2304)
    x = r.standard_normal(2304, dtype=np.float32)
    y0 = r.standard_normal(2304, dtype=np.float32)
    ref = y0 + oracle.matmul(w.data, 2304, 2304, x, 1).reshape(-1)
    got = run_matmul(gpu, w, x, 1, bias=y0).reshape(-1)
    assert_close(got, ref, "gemv residual")
    if oracle.simd_path() == "avx2+fma":
        assert_bits(got, ref, "gemv residual")
    gpu.release(w)


@pytest.mark.parametrize("x_off", [1, 2, 3, 4])
def test_gemv_x_offsets_of_any_alignment(gpu, x_off):
    """Offsets are in f32 elements (compute.rs:421-431); x at a 4-, 8- or
    12-byte offset takes the kernel's dword path, 16 bytes its dwordx4 path."""
    r = rng(16 + x_off)
    out, k = 96, 2304
    w = weight(r, out, k)
    x = r.standard_normal(k, dtype=np.float32)
    xb, yb = gpu.alloc(4 * (k + x_off)), gpu.alloc(4 * out)
    xb.upload(np.concatenate([np.full(x_off, np.nan, np.float32), x]))
    gpu.matmul(w, xb, x_off, 1, yb, 0)
    got = yb.download(np.float32, out)
    ref = oracle.matmul(w.data, k, out, x, 1).reshape(-1)
    assert_close(got, ref, f"gemv x_off={x_off}")
    if oracle.simd_path() == "avx2+fma":
        assert_bits(got, ref, f"gemv x_off={x_off}")
    xb.free()
    yb.free()
    gpu.release(w)


def test_decode_group_matches_separate_matmuls(gpu):
    """cuda/mod.rs:1482-1543: QKV-like group sharing x in one launch."""
    r = rng(15)
    k = 2304
    ws = [weight(r, o, k) for o in (2304, 512, 768)]
    x = r.standard_normal(k, dtype=np.float32)
    xb = gpu.alloc(4 * k)
    xb.upload(x)
    ys = [gpu.alloc(4 * (w.out + 8)) for w in ws]
    gpu.matmul_decode_group([(w, y, 8) for w, y in zip(ws, ys)], xb, 0, k)
    for w, y in zip(ws, ys):
        got = y.download(np.float32, w.out, offset_bytes=32)
        ref = oracle.matmul(w.data, k, w.out, x, 1).reshape(-1)
        assert_close(got, ref, f"group member {w.out}")
        if oracle.simd_path() == "avx2+fma":
            assert_bits(got, ref, f"group member {w.out}")
        gpu.release(w)
        y.free()
    xb.free()


# ---------------------------------------------------------------------------
# activation quantization (quant.rs:98-121), byte-exact
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n,k", [(1, 32), (2, 64), (31, 2304), (33, 2304), (65, 5760), (130, 2304)])
@pytest.mark.parametrize("f16", [-1, 0, 1])
def test_quantized_activations_are_bit_exact(gpu, n, k, f16):
    """Both prepared formats (int8 units, and the same integers as f16 for
    the f16-MFMA GEMM) hold the reference's quantize_q8_0 bit for bit."""
    gpu.set_option("gemm.f16", f16)
    r = rng(20 + n)
    x = oracle.make_activations(r, n, k, outlier_rate=0.01)
    x[0, :32] = 0.0                                   # all-zero block
    if k >= 64:
        x[0, 32:64] = np.arange(32, dtype=np.float32) - 16.0
        x[0, 32] = 127.0                              # inverse exactly 1: ties
        x[0, 33:37] = [2.5, -2.5, 0.5, -0.5]
    if n > 1:
        x[1, 5] = np.nan                              # ignored by the peak, q = 0
        x[1, 40 % k] = np.inf if k > 40 else x[1, 40 % k]
    xb = gpu.alloc(4 * n * k)
    xb.upload(x)
    p = gpu.prepare(xb, 0, n, k)
    planned_f16 = n >= 2 and gpu.plan(n, 64, k)["kernel"] == q8.KERNEL_GEMM_F16
    assert p.format == (q8.PREPARED_F16 if planned_f16 else q8.PREPARED_I8)
    if f16 == 1:
        assert planned_f16 == (n >= 2)
    if f16 == 0:
        assert not planned_f16
    q, s = unpack_prepared(gpu, p, n, k)
    for t in range(n):
        rq, rs = oracle.quantize_q8_0(x[t])
        assert np.array_equal(q[t], rq), f"token {t}: quants differ"
        assert np.array_equal(s[t].view(np.uint32), rs.view(np.uint32)), f"token {t}: scales differ"
    tt = (n + 31) // 32
    assert not q[n:tt * 32].any() and not s[n:tt * 32].any(), "padding tokens must be zero"
    xb.free()


# ---------------------------------------------------------------------------
# n >= 2 MFMA GEMM (tensor.rs:104-148)
# ---------------------------------------------------------------------------

def exact_problem(r, out, k, n):
    """Power-of-two scales, one per weight row and one per token, and
    activations whose block peak is exactly 127 * s_x, so d_w*s_x is a power
    of two, every quantized value is the integer itself, and (with k <= 1024,
    |sum| < 2^24) every f32 step is exact: y must equal the integer sum."""
    assert k <= 1024
    nb = k // 32
    qw = r.integers(-127, 128, size=(out, nb, 32))
    ew = r.integers(-12, 0, size=out)
    raw = np.zeros((out, nb, 34), np.uint8)
    d16 = np.repeat((2.0 ** ew)[:, None], nb, axis=1).astype(np.float16)
    raw[:, :, 0:2] = d16.view(np.uint8).reshape(out, nb, 2)
    raw[:, :, 2:] = qw.astype(np.int8).view(np.uint8)
    qx = r.integers(-127, 128, size=(n, nb, 32))
    qx[:, :, 0] = 127
    ex = r.integers(-6, 1, size=n)
    x = (qx * (2.0 ** ex)[:, None, None]).reshape(n, k).astype(np.float32)
    isum = np.einsum("onk,tnk->to", qw.astype(np.int64), qx.astype(np.int64))
    y = isum.astype(np.float64) * (2.0 ** ew)[None, :] * (2.0 ** ex)[:, None]
    return q8.Weight(raw.reshape(-1), k, out), x, y.astype(np.float32)


@pytest.mark.parametrize("n,k", [(2, 32), (5, 64), (33, 96), (64, 1024), (160, 1024)])
@pytest.mark.parametrize("path", ["i8_smode1", "i8_smode0", "f16"])
def test_gemm_int32_block_dot_is_exact(gpu, n, k, path):
    gpu.set_option("gemm.f16", 1 if path == "f16" else 0)
    gpu.set_option("gemm.smode", 0 if path == "i8_smode0" else 1)
    r = rng(30 + n)
    w, x, y = exact_problem(r, 40, k, n)
    got = run_matmul(gpu, w, x, n)
    assert_bits(got, y, f"exact gemm n={n} k={k}")
    gpu.release(w)


@pytest.mark.parametrize("n", [2, 7, 8, 9, 33, 64, 65, 128, 129, 172, 193, 512, 1024])
def test_gemm_matches_the_reference(gpu, n):
    r = rng(40 + n)
    out, k = 392, 2304
    w = weight(r, out, k)
    x = oracle.make_activations(r, n, k, outlier_rate=0.01)
    ref = oracle.matmul(w.data, k, out, x, n)
    got = run_matmul(gpu, w, x, n)
    assert_parity(got, ref, exact_matmul(w.data, k, out, x, n), f"gemm n={n}")
    gpu.release(w)


@pytest.mark.parametrize("n", [8, 64])
def test_gemm_configs1(gpu, n):
    """same W as configs[0], X [n, 2304] N(0,1) with ~1% +-20."""
    r = rng(50 + n)
    w = weight(r, 5760, 2304)
    x = oracle.make_activations(r, n, 2304, outlier_rate=0.01)
    ref = oracle.matmul(w.data, 2304, 5760, x, n)
    got = run_matmul(gpu, w, x, n)
    assert_parity(got, ref, exact_matmul(w.data, 2304, 5760, x, n), f"configs[1] n={n}")
    gpu.release(w)


@pytest.mark.parametrize("smode,tpw,twaves,remap,kwaves,slices", [
    (0, 1, 1, 0, 1, 1), (0, 1, 4, 1, 1, 1), (1, 1, 2, 0, 1, 1), (1, 1, 3, 1, 1, 1), (1, 1, 1, 1, 8, 1),
    (1, 2, 2, 0, 3, 1), (1, 2, 1, 1, 2, 4), (1, 4, 1, 0, 1, 7), (1, 4, 2, 1, 4, 1), (1, 4, 1, 1, 8, 3),
    (0, 1, 2, 1, 4, 3), (1, 1, 1, 1, 6, 15), (1, 2, 3, 0, 2, 2), (1, 4, 2, 0, 1, 1)])
def test_gemm_variants_agree(gpu, smode, tpw, twaves, remap, kwaves, slices):
    gpu.set_option("gemm.f16", 0)  # the int8-MFMA family's launch variants
    gpu.set_option("gemm.smode", smode)
    gpu.set_option("gemm.tpw", tpw)
    gpu.set_option("gemm.twaves", twaves)
    gpu.set_option("gemm.xcd_remap", remap)
    gpu.set_option("gemm.kwaves", kwaves)
    gpu.set_option("gemm.slices", slices)
    r = rng(60)
    n, out, k = 200, 256, 5760
    w = weight(r, out, k)
    x = oracle.make_activations(r, n, k, outlier_rate=0.01)
    ref = oracle.matmul(w.data, k, out, x, n)
    got = run_matmul(gpu, w, x, n)
    assert_parity(got, ref, exact_matmul(w.data, k, out, x, n),
                  f"gemm smode={smode} tpw={tpw} twaves={twaves} remap={remap} kwaves={kwaves} slices={slices}")
    gpu.release(w)


@pytest.mark.parametrize("n,out,k", [(200, 256, 5760), (64, 96, 2304), (512, 320, 2304), (33, 40, 96),
                                     (130, 64, 32)])
@pytest.mark.parametrize("tpw,rwaves,kwaves", [(2, 4, 1), (2, 2, 1), (2, 2, 3), (2, 4, 2), (1, 4, 2), (2, 2, 4)])
def test_gemm_f16_equals_int8_bit_for_bit(gpu, n, out, k, tpw, rwaves, kwaves):
    """The f16-MFMA GEMM computes each block's integer dot exactly and then
    the int8 kernel's arithmetic in its order, so with the same K split the
    two families agree to the bit (and both meet the reference bar)."""
    r = rng(61 + n + out)
    w = weight(r, out, k)
    x = oracle.make_activations(r, n, k, outlier_rate=0.01)
    gpu.set_option("gemm.f16", 1)
    gpu.set_option("gemm.tpw", tpw)
    gpu.set_option("gemm.rwaves", rwaves)
    gpu.set_option("gemm.kwaves", kwaves)
    t = gpu.plan(n, out, k)
    assert t["kernel"] == q8.KERNEL_GEMM_F16
    kw = t["kwaves"]                              # the K split the runtime settles on (LDS, pairs)
    got = run_matmul(gpu, w, x, n)
    gpu.set_option("gemm.f16", 0)
    gpu.set_option("gemm.tpw", 1)
    gpu.set_option("gemm.twaves", 1)
    gpu.set_option("gemm.slices", 1)
    gpu.set_option("gemm.kwaves", kw)
    assert gpu.plan(n, out, k)["kwaves"] == kw
    want = run_matmul(gpu, w, x, n)
    what = f"f16 gemm n={n} out={out} k={k} tpw={tpw} rwaves={rwaves} kwaves={kw}"
    assert_bits(got, want, what)
    ref = oracle.matmul(w.data, k, out, x, n)
    assert_parity(got, ref, exact_matmul(w.data, k, out, x, n), what)
    gpu.release(w)


@pytest.mark.parametrize("n,out,k", [(200, 256, 5760), (64, 96, 2304), (512, 320, 2304), (33, 40, 96),
                                     (2, 64, 32), (130, 64, 160)])
@pytest.mark.parametrize("tpw,kwaves", [(1, 1), (1, 3), (1, 8), (2, 1), (2, 2), (2, 5)])
def test_gemm_pipelined_equals_unpipelined(gpu, n, out, k, tpw, kwaves):
    """The pipelined int8 kernel reorders instructions only: with the same K
    split its outputs equal the plain kernel's bit for bit, including the
    zero-scaled padding pair and an odd last block."""
    r = rng(63 + n + out + k)
    w = weight(r, out, k)
    x = oracle.make_activations(r, n, k, outlier_rate=0.01)
    gpu.set_option("gemm.f16", 0)
    gpu.set_option("gemm.tpw", tpw)
    gpu.set_option("gemm.twaves", 1)
    gpu.set_option("gemm.slices", 1)
    gpu.set_option("gemm.kwaves", kwaves)
    gpu.set_option("gemm.pipe", 1)
    t = gpu.plan(n, out, k)
    assert t["pipe"] == 1 and t["kslices"] == 1
    got = run_matmul(gpu, w, x, n)
    gpu.set_option("gemm.pipe", 0)
    gpu.set_option("gemm.kwaves", t["kwaves"])
    assert gpu.plan(n, out, k)["kwaves"] == t["kwaves"]
    want = run_matmul(gpu, w, x, n)
    what = f"pipelined gemm n={n} out={out} k={k} tpw={tpw} kwaves={t['kwaves']}"
    assert_bits(got, want, what)
    assert_parity(got, oracle.matmul(w.data, k, out, x, n), exact_matmul(w.data, k, out, x, n), what)
    gpu.release(w)


@pytest.mark.parametrize("n,out,k", [(200, 256, 5760), (64, 96, 2304), (512, 320, 2304), (33, 40, 96),
                                     (2, 64, 32), (130, 64, 160)])
@pytest.mark.parametrize("tpw,rwaves,kwaves", [(2, 4, 1), (2, 2, 1), (2, 2, 3), (2, 4, 2), (1, 2, 2), (1, 2, 4)])
def test_gemm_lds_staged_equals_plain(gpu, n, out, k, tpw, rwaves, kwaves):
    """q8_gemm_l (int8 activation units staged in LDS, shared by row-tile
    waves) and the plain int8 kernel agree to the bit at the same K split,
    residual epilogue included."""
    r = rng(65 + n + out + k)
    w = weight(r, out, k)
    x = oracle.make_activations(r, n, k, outlier_rate=0.01)
    y0 = r.standard_normal((n, out)).astype(np.float32)
    gpu.set_option("gemm.f16", 0)
    gpu.set_option("gemm.lds", 1)
    gpu.set_option("gemm.tpw", tpw)
    gpu.set_option("gemm.rwaves", rwaves)
    gpu.set_option("gemm.kwaves", kwaves)
    t = gpu.plan(n, out, k)
    assert t["kernel"] == q8.KERNEL_GEMM and t["rwaves"] in (2, 4)
    got = run_matmul(gpu, w, x, n, bias=y0)
    gpu.set_option("gemm.lds", 0)
    gpu.set_option("gemm.tpw", 1)
    gpu.set_option("gemm.twaves", 1)
    gpu.set_option("gemm.slices", 1)
    gpu.set_option("gemm.kwaves", t["kwaves"])
    assert gpu.plan(n, out, k)["kwaves"] == t["kwaves"]
    want = run_matmul(gpu, w, x, n, bias=y0)
    what = f"lds gemm n={n} out={out} k={k} tpw={t['tpw']} rwaves={t['rwaves']} kwaves={t['kwaves']}"
    assert_bits(got, want, what)
    gpu.release(w)


def test_gemm_residual_and_prompt_group(gpu):
    r = rng(61)
    n, k = 96, 2304
    ws = [weight(r, o, k) for o in (256, 128, 320)]
    x = oracle.make_activations(r, n, k, outlier_rate=0.01)
    xb = gpu.alloc(4 * n * k)
    xb.upload(x)
    p = gpu.prepare(xb, 0, n, k)
    ys = [gpu.alloc(4 * n * w.out) for w in ws]
    gpu.matmul_prompt_group([(w, y, 0) for w, y in zip(ws, ys)], p, n, k)
    for w, y in zip(ws, ys):
        ref = oracle.matmul(w.data, k, w.out, x, n)
        assert_parity(y.download(np.float32, n * w.out).reshape(n, w.out), ref,
                      exact_matmul(w.data, k, w.out, x, n), f"prompt group {w.out}")
    # residual: y += W x on the first member
    y0 = r.standard_normal((n, ws[0].out), dtype=np.float32)
    ys[0].upload(y0)
    gpu.matmul(ws[0], xb, 0, n, ys[0], 0, prepared=p, bias=ys[0])
    ref = y0 + oracle.matmul(ws[0].data, k, ws[0].out, x, n)
    exact = y0.astype(np.float64) + exact_matmul(ws[0].data, k, ws[0].out, x, n)
    assert_parity(ys[0].download(np.float32, n * ws[0].out).reshape(n, -1), ref, exact, "prompt residual")
    for w, y in zip(ws, ys):
        gpu.release(w)
        y.free()
    xb.free()


def test_reference_gpu_vs_cpu_protocol(gpu):
    """gpu_matmul.rs:32-80 on synthetic weights of attn_q / ffn_down shape:
    x = 0.5 sin(0.017 i + n), n in {1, 8, 65, 128, 129, 172, 193},
    max|d| <= 1e-3 * max(max|y|, 1); plus this build's tighter bar."""
    r = rng(70)
    for out, k in ((2304, 2304), (2304, 5760)):
        w = weight(r, out, k)
        for n in (1, 8, 65, 128, 129, 172, 193):
            x = (np.sin(np.arange(n * k, dtype=np.float32) * np.float32(0.017) + np.float32(n))
                 * np.float32(0.5)).astype(np.float32)
            ref = oracle.matmul(w.data, k, out, x, n)
            got = run_matmul(gpu, w, x, n)
            md = float(np.max(np.abs(got - ref)))
            scale = float(np.max(np.abs(ref)))
            print(f"{out}x{k} n={n}: max|d| = {md:.3e} (values up to {scale:.3f})", flush=True)
            assert md <= 1e-3 * max(scale, 1.0)
            if n == 1:
                assert_close(got, ref, f"protocol {out}x{k} n={n}")
            else:
                assert_parity(got, ref, exact_matmul(w.data, k, out, x, n), f"protocol {out}x{k} n={n}")
        gpu.release(w)


# ---------------------------------------------------------------------------
# gate/up + SiLU, silu_mul_prepare, lm_head argmax
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n,ffn", [(1, 5760), (3, 5760), (64, 5760), (130, 640)])
def test_gate_up_silu(gpu, n, ffn):
    r = rng(80 + n)
    k = 2304
    gw, uw = weight(r, ffn, k), weight(r, ffn, k)
    x = oracle.make_activations(r, n, k)
    xb = gpu.alloc(4 * n * k)
    xb.upload(x)
    act = gpu.alloc(4 * n * ffn)
    gpu.gate_up_silu(gw, uw, xb, 0, n, act, 0)
    g = oracle.matmul(gw.data, k, ffn, x, n)
    u = oracle.matmul(uw.data, k, ffn, x, n)
    ref = oracle.silu_mul(g, u).reshape(n, ffn)
    got = act.download(np.float32, n * ffn).reshape(n, ffn)
    if n == 1:
        assert_close(got, ref, f"gate_up_silu n={n}")
    else:
        ge, ue = exact_matmul(gw.data, k, ffn, x, n), exact_matmul(uw.data, k, ffn, x, n)
        assert_parity(got, ref, ge / (1.0 + np.exp(-ge)) * ue, f"gate_up_silu n={n}")
    for b in (xb, act):
        b.free()
    gpu.release(gw)
    gpu.release(uw)


@pytest.mark.parametrize("n,ffn,k", [(2, 640, 2304), (33, 96, 96), (130, 5760, 2304), (512, 320, 5760),
                                     (64, 64, 32)])
@pytest.mark.parametrize("kw", [1, 2, 3, 8])
@pytest.mark.parametrize("entry", ["x", "prepared", "prepared_f16_out"])
def test_gate_up_silu_fused_epilogue_equals_unfused(gpu, n, ffn, k, kw, entry):
    """q8_gemm_silu (gate and up accumulated by one wave, silu(g) * u
    quantized to Q8_0 in the epilogue) writes the same prepared bytes as the
    int8 GEMM into f32 workspace followed by the SiLU-product quantization,
    at the same K split; odd block counts and an f16 output plane included."""
    r = rng(95 + n + ffn + k)
    gw, uw = weight(r, ffn, k), weight(r, ffn, k)
    x = oracle.make_activations(r, n, k, outlier_rate=0.01)
    xb = gpu.alloc(4 * n * k)
    xb.upload(x)
    act = gpu.alloc(4 * n * ffn)
    for name, value in (("gemm.f16", 0), ("gemm.tpw", 1), ("gemm.twaves", 1), ("gemm.slices", 1),
                        ("gemm.pipe", 0), ("gemm.lds", 0), ("gemm.kwaves", kw)):
        gpu.set_option(name, value)

    def run(fused):
        gpu.set_option("gemm.silu", fused)
        if entry == "x":
            p = gpu.gate_up_silu(gw, uw, xb, 0, n, act, 0, want_prepared=True)
        else:
            gpu.set_option("gemm.f16", 0)
            px = gpu.prepare(xb, 0, n, k)
            assert px.format == q8.PREPARED_I8
            if entry == "prepared_f16_out":
                gpu.set_option("gemm.f16", 1)   # int8 input, f16 output plane
            p = gpu.gate_up_silu_prepared(gw, uw, px)
        want_fmt = q8.PREPARED_F16 if entry == "prepared_f16_out" else q8.PREPARED_I8
        assert p.format == want_fmt and p.n == n and p.k == ffn
        return unpack_prepared(gpu, p, n, ffn)

    q1, s1 = run(1)
    q0, s0 = run(0)
    what = f"gate_up_silu fused n={n} ffn={ffn} k={k} kw={kw} {entry}"
    assert np.array_equal(s1, s0), f"{what}: scales differ"
    assert np.array_equal(q1, q0), f"{what}: {int((q1 != q0).sum())} quants differ"
    # and the bytes quantize the reference's product
    g = oracle.matmul(gw.data, k, ffn, x, n)
    u = oracle.matmul(uw.data, k, ffn, x, n)
    ref = oracle.silu_mul(g, u).reshape(n, ffn)
    deq = q1[:n].astype(np.float32).reshape(n, ffn // 32, 32) * s1[:n, :, None]
    bound = 0.5 * s1[:n, :, None] * 1.001 + 1e-4 * np.abs(ref.reshape(n, ffn // 32, 32)) + 1e-5
    assert np.all(np.abs(deq - ref.reshape(n, ffn // 32, 32)) <= bound), what
    for b in (xb, act):
        b.free()
    gpu.release(gw)
    gpu.release(uw)


@pytest.mark.parametrize("n,k", [(40, 5760), (130, 1024)])
def test_silu_mul_and_its_quantization(gpu, n, k):
    r = rng(90 + n)
    g = (r.standard_normal((n, k)) * 3).astype(np.float32)
    u = r.standard_normal((n, k)).astype(np.float32)
    gb, ub, ab = gpu.alloc(4 * n * k), gpu.alloc(4 * n * k), gpu.alloc(4 * n * k)
    gb.upload(g)
    ub.upload(u)
    gpu.silu_mul(ab, gb, ub, n * k)
    act_ref = oracle.silu_mul(g, u).reshape(n, k)
    act = ab.download(np.float32, n * k).reshape(n, k)
    assert_close(act, act_ref, "silu_mul")
    ulp = np.abs(act.view(np.int32).astype(np.int64) - act_ref.view(np.int32).astype(np.int64))
    assert int(ulp.max()) <= 2, f"silu_mul differs by {int(ulp.max())} ulp"
    p = gpu.silu_mul_prepare(gb, ub, n, k)
    q, s = unpack_prepared(gpu, p, n, k)
    for t in range(n):
        # quantize exactly what the device computed: bit-exact
        rq, rs = oracle.quantize_q8_0(act[t])
        assert np.array_equal(q[t], rq) and np.array_equal(s[t], rs), f"token {t}"
    for b in (gb, ub, ab):
        b.free()


# ---------------------------------------------------------------------------
# RMSNorm and the fused norm -> Q8_0 prepare (ops.rs:5-30, compute.rs:584-614, 959-984)
# ---------------------------------------------------------------------------

EPS = 1e-6  # configs[4]'s RMSNorm epsilon


def norm_rows(r, rows, k):
    x = (r.standard_normal((rows, k)) * 3.0).astype(np.float32)
    x[0, :] = 0.0                                     # all-zero row: scale = 1 / sqrt(eps)
    if rows > 2:
        x[2, :] *= 1e4                                # large row
        x[2, 7] = -3e5
    if rows > 3:
        x[3, :] *= 1e-5                               # tiny row (the eps term dominates)
    w = (1.0 + 0.1 * r.standard_normal(k)).astype(np.float32)
    return x, w


def test_norm_weight_cache_is_keyed_by_host_identity_until_released(gpu):
    """Norm weights are made resident by (pointer, length) like weights: new
    contents at the same address are not seen until q8_vector_release drops
    the device copy (the decoder releases its vectors when destroyed)."""
    import ctypes
    r = rng(77)
    k = 256
    x = r.standard_normal((1, k)).astype(np.float32)
    w = (1.0 + 0.1 * r.standard_normal(k)).astype(np.float32)
    xb, ob = gpu.alloc(4 * k), gpu.alloc(4 * k)
    xb.upload(x)
    q8._check(q8.lib().q8_rmsnorm(gpu.handle, xb.ptr, 0, w.ctypes.data, k, ctypes.c_float(EPS), 1, ob.ptr, 0))
    first = ob.download(np.float32, k)
    assert_bits(first, oracle.rmsnorm(x[0], w, EPS), "first norm")
    w *= 2.0  # same address, new contents
    q8._check(q8.lib().q8_rmsnorm(gpu.handle, xb.ptr, 0, w.ctypes.data, k, ctypes.c_float(EPS), 1, ob.ptr, 0))
    assert_bits(ob.download(np.float32, k), first, "cached copy (identity key)")
    q8._check(q8.lib().q8_vector_release(gpu.handle, w.ctypes.data, k))
    q8._check(q8.lib().q8_vector_release(gpu.handle, w.ctypes.data, k))  # not resident: a no-op
    q8._check(q8.lib().q8_rmsnorm(gpu.handle, xb.ptr, 0, w.ctypes.data, k, ctypes.c_float(EPS), 1, ob.ptr, 0))
    assert_bits(ob.download(np.float32, k), oracle.rmsnorm(x[0], w, EPS), "after release")
    q8._check(q8.lib().q8_vector_release(gpu.handle, w.ctypes.data, k))
    xb.free()
    ob.free()


@pytest.mark.parametrize("rows,k", [(1, 2304), (3, 32), (5, 5760), (40, 2304), (67, 64)])
def test_rmsnorm_rows_match_the_reference_bit_for_bit(gpu, rows, k):
    """f32 squares summed in f64, then 1 / sqrt(ms + eps) and (x * s) * w in
    f32; the device's f64 sum is a tree, the reference's left to right, which
    round to the same f32 mean square unless it lies within ~1e-12 of an f32
    rounding boundary -- not the case on these seeded rows."""
    r = rng(100 + rows + k)
    x, w = norm_rows(r, rows, k)
    xb, ob = gpu.alloc(4 * rows * k), gpu.alloc(4 * rows * k)
    xb.upload(x)
    gpu.rmsnorm(xb, 0, w, EPS, rows, ob, 0)
    got = ob.download(np.float32, rows * k).reshape(rows, k)
    ref = np.stack([oracle.rmsnorm(x[t], w, EPS) for t in range(rows)])
    assert_bits(got, ref, f"rmsnorm {rows}x{k}")
    xb.free()
    ob.free()


@pytest.mark.parametrize("rows,k", [(1, 2304), (2, 64), (33, 2304), (130, 5760), (512, 2304), (3, 8192)])
@pytest.mark.parametrize("f16", [-1, 1])
def test_norm_prepare_is_quantize_of_rmsnorm(gpu, rows, k, f16):
    """Gpu::rmsnorm_prepare: the quantized bytes and scales are the
    reference's quantize_q8_0(rmsnorm(x)) exactly, padding tokens zero."""
    gpu.set_option("gemm.f16", f16)
    r = rng(110 + rows + k)
    x, w = norm_rows(r, rows, k)
    xb = gpu.alloc(4 * rows * k)
    xb.upload(x)
    p = gpu.norm_prepare(xb, 0, w, EPS, rows)
    assert p.n == rows and p.k == k
    q, sc = unpack_prepared(gpu, p, rows, k)
    for t in range(rows):
        rq, rs = oracle.quantize_q8_0(oracle.rmsnorm(x[t], w, EPS))
        assert np.array_equal(q[t], rq), f"token {t}: quants differ"
        assert np.array_equal(sc[t].view(np.uint32), rs.view(np.uint32)), f"token {t}: scales differ"
    tt = (rows + 31) // 32
    assert not q[rows:tt * 32].any() and not sc[rows:tt * 32].any(), "padding tokens must be zero"
    xb.free()


def test_norm_prepare_feeds_the_gemm_and_compute_threshold(gpu):
    """The layer's norm -> QKV chain (model.rs:887-954): norm_prepare's
    operand through the GEMM equals the reference's matmul of the normed rows;
    Compute.norm_prepare below prepare_min_tokens writes the f32 norm instead."""
    r = rng(120)
    n, k, out = 96, 2304, 320
    x, wn = norm_rows(r, n, k)
    wm = weight(r, out, k)
    xb, yb = gpu.alloc(4 * n * k), gpu.alloc(4 * n * out)
    xb.upload(x)
    p = gpu.norm_prepare(xb, 0, wn, EPS, n)
    gpu.matmul(wm, xb, 0, n, yb, 0, prepared=p)
    got = yb.download(np.float32, n * out).reshape(n, out)
    normed = np.stack([oracle.rmsnorm(x[t], wn, EPS) for t in range(n)])
    ref = oracle.matmul(wm.data, k, out, normed, n)
    assert_parity(got, ref, exact_matmul(wm.data, k, out, normed, n), "norm_prepare -> gemm")
    comp = q8.Compute(gpu)
    ob = gpu.alloc(4 * k)
    assert comp.norm_prepare(xb, k, wn, EPS, 1, ob, 0) is None
    assert_bits(ob.download(np.float32, k), oracle.rmsnorm(x[1], wn, EPS), "Compute.norm_prepare n=1")
    for b in (xb, yb, ob):
        b.free()
    gpu.release(wm)


def test_lm_head_argmax(gpu):
    """lm_head 122880 x 2304 with the greedy argmax."""
    r = rng(100)
    vocab, k = 122880, 2304
    w = weight(r, vocab, k)
    x = r.standard_normal(k, dtype=np.float32)
    ref = oracle.matmul(w.data, k, vocab, x, 1).reshape(-1)
    xb, lb = gpu.alloc(4 * k), gpu.alloc(4 * vocab)
    xb.upload(x)
    best = gpu.lm_head_argmax(w, xb, 0, lb, 0)
    got = lb.download(np.float32, vocab)
    assert_close(got, ref, "lm_head logits")
    if oracle.simd_path() == "avx2+fma":
        assert_bits(got, ref, "lm_head logits")
    assert best == oracle.argmax(ref)
    top2 = np.sort(ref)[-2:]
    print(f"argmax {best}, top-2 gap {float(top2[1] - top2[0]):.3e}", flush=True)
    xb.free()
    lb.free()
    gpu.release(w)


@pytest.mark.parametrize("seed", [100, 101, 102])
def test_lm_head_default_order_argmax(gpu, seed):
    """The lm_head at the default block order (the tree sum, not the exact
    AVX2 order): logits within the bar and the token the GEMV's folded argmax
    returns equal to the greedy argmax of the oracle's logits
    (sampler.rs:167-175, first index of the strictly greatest value)."""
    gpu.set_option("gemv.exact", -1)
    r = rng(seed)
    vocab, k = 122880, 2304
    w = weight(r, vocab, k)
    x = r.standard_normal(k, dtype=np.float32)
    ref = oracle.matmul(w.data, k, vocab, x, 1).reshape(-1)
    xb, lb = gpu.alloc(4 * k), gpu.alloc(4 * vocab)
    xb.upload(x)
    best = gpu.lm_head_argmax(w, xb, 0, lb, 0)
    got = lb.download(np.float32, vocab)
    assert_close(got, ref, f"default-order lm_head logits seed {seed}")
    top2 = np.sort(ref)[-2:]
    gap = float(top2[1] - top2[0])
    print(f"default order: argmax {best}, oracle {oracle.argmax(ref)}, top-2 gap {gap:.3e}", flush=True)
    assert best == oracle.argmax(ref), f"seed {seed}: token {best} vs oracle {oracle.argmax(ref)} (gap {gap:.3e})"
    assert best == oracle.argmax(got), "the folded argmax is the argmax of the logits it wrote"
    xb.free()
    lb.free()
    gpu.release(w)


@pytest.mark.parametrize("exact", [1, 0])
@pytest.mark.parametrize("out", [1000, 40, 8])
def test_gemv_tile_kernel_residual_at_ragged_rows(gpu, out, exact):
    """The 32-row tile kernel (gemv.rows = 32) with a residual whose row count
    is not a multiple of 32: the padding lanes of the last tile read no
    residual (the bias buffer holds `out` floats) and write nothing."""
    gpu.set_option("gemv.rows", 32)
    gpu.set_option("gemv.exact", exact)
    r = rng(110 + out + exact)
    k = 2304
    w = weight(r, out, k)
    x = r.standard_normal(k, dtype=np.float32)
    y0 = r.standard_normal(out, dtype=np.float32)
    ref = y0 + oracle.matmul(w.data, k, out, x, 1).reshape(-1)
    got = run_matmul(gpu, w, x, 1, bias=y0).reshape(-1)
    what = f"tile gemv residual out={out} exact={exact}"
    assert_close(got, ref, what)
    if exact and oracle.simd_path() == "avx2+fma":
        assert_bits(got, ref, what)
    gpu.release(w)


@pytest.mark.parametrize("values,expect", [
    ([1, 3, 3, 2], 1), ([-1, -1], 0), ([0, float("nan"), 5, 5], 2), ([float("nan"), 1, 9], 0),
    ([-0.0, 0.0], 0), ([float("-inf"), float("-inf")], 0), ([1, float("inf"), float("inf")], 1),
])
def test_argmax_semantics(gpu, values, expect):
    v = np.array(values, np.float32)
    b = gpu.alloc(4 * v.size)
    b.upload(v)
    assert gpu.argmax(b, 0, v.size) == expect == oracle.argmax(v)
    b.free()


def test_argmax_large_with_ties_across_workgroups(gpu):
    r = rng(101)
    v = r.standard_normal(1_000_003).astype(np.float32)
    v[[123_456, 654_321, 999_999]] = 50.0
    b = gpu.alloc(4 * v.size)
    b.upload(v)
    assert gpu.argmax(b, 0, v.size) == 123_456 == oracle.argmax(v)
    b.free()


# ---------------------------------------------------------------------------
# error paths: rejected on the host, nothing launched
# ---------------------------------------------------------------------------

def test_errors_are_reported_not_launched(gpu):
    r = rng(110)
    w = weight(r, 64, 64)
    xb = gpu.alloc(4 * 64 * 2000)
    small = gpu.alloc(4 * 10)
    with pytest.raises(q8.Q8Error) as e:
        gpu.matmul(w, xb, 0, 1025, xb, 0)
    assert e.value.status == q8.Q8_ERR_UNSUPPORTED
    with pytest.raises(q8.Q8Error) as e:
        gpu.matmul(w, xb, 0, 1, small, 0)            # y too small
    assert e.value.status == q8.Q8_ERR_INVALID
    with pytest.raises(q8.Q8Error) as e:
        gpu.matmul(w, small, 0, 2, xb, 0)            # x too small
    assert e.value.status == q8.Q8_ERR_INVALID
    with pytest.raises(q8.Q8Error) as e:
        gpu.matmul_decode_group([(w, xb, 0)] * 5, xb, 0, 64)
    assert e.value.status == q8.Q8_ERR_INVALID
    with pytest.raises(q8.Q8Error) as e:
        gpu.matmul_decode_group([(w, xb, 0), (w, xb, 64)], xb, 0, 64, bias=xb)
    assert e.value.status == q8.Q8_ERR_INVALID
    p = gpu.prepare(xb, 0, 4, 64)
    with pytest.raises(q8.Q8Error) as e:
        gpu.matmul(w, xb, 0, 5, xb, 4096, prepared=p)  # prepared for another n
    assert e.value.status == q8.Q8_ERR_INVALID
    raw = np.zeros(34 * 3, np.uint8)
    import ctypes
    h = ctypes.c_void_p()
    assert q8.lib().q8_weight_resident(gpu.handle, raw.ctypes.data, 100, 96, 1,
                                       ctypes.byref(h)) == q8.Q8_ERR_INVALID
    assert q8.lib().q8_weight_resident(gpu.handle, raw.ctypes.data, raw.nbytes, 95, 1,
                                       ctypes.byref(h)) == q8.Q8_ERR_INVALID
    gpu.sync()
    xb.free()
    small.free()
    gpu.release(w)


# ---------------------------------------------------------------------------
# graph capture: replays match eager results (no memset nodes are recorded)
# ---------------------------------------------------------------------------

def test_graph_replay_matches_eager(gpu):
    r = rng(120)
    k, out, n = 2304, 640, 48
    w = weight(r, out, k)
    x1 = r.standard_normal(k, dtype=np.float32)
    xn = oracle.make_activations(r, n, k)
    b1, bn = gpu.alloc(4 * k), gpu.alloc(4 * n * k)
    y1, yn = gpu.alloc(4 * out), gpu.alloc(4 * n * out)
    b1.upload(x1)
    bn.upload(xn)
    gpu.matmul(w, b1, 0, 1, y1, 0)
    gpu.matmul(w, bn, 0, n, yn, 0)
    e1 = y1.download(np.float32, out)
    en = yn.download(np.float32, n * out)
    gpu.graph_begin()
    gpu.matmul(w, b1, 0, 1, y1, 0)
    gpu.matmul(w, bn, 0, n, yn, 0)
    graph = gpu.graph_end()
    try:
        for i in range(3):
            y1.upload(np.zeros(out, np.float32))
            yn.upload(np.zeros(n * out, np.float32))
            gpu.graph_launch(graph)
            gpu.sync()
            assert_bits(y1.download(np.float32, out), e1, f"replay {i} gemv")
            assert_bits(yn.download(np.float32, n * out), en, f"replay {i} gemm")
    finally:
        gpu.graph_destroy(graph)
    for b in (b1, bn, y1, yn):
        b.free()
    gpu.release(w)


@pytest.mark.parametrize("n,out,k", [(8, 5760, 2304), (1 + 31, 200, 96), (3, 64, 5760), (33, 2304, 2304)])
def test_gemm_streamed_weights_are_the_same_bits(gpu, n, out, k):
    """One token tile (n <= 32): the GEMM reads its weights non-temporally
    (q8_gemm_s1_t1s); option gemm.stream = 0 keeps the default cache policy.
    Same bits either way (the policy is not arithmetic), within the n >= 2
    bar of the reference; n = 33 (two token tiles) is the plain kernel."""
    r = rng(900 + n + out + k)
    w = weight(r, out, k)
    x = oracle.make_activations(r, n, k, outlier_rate=0.01)
    try:
        got = run_matmul(gpu, w, x, n).reshape(n, out)
        gpu.set_option("gemm.stream", 0)
        plain = run_matmul(gpu, w, x, n).reshape(n, out)
    finally:
        gpu.set_option("gemm.stream", -1)
    assert_bits(got, plain, f"streamed weights n={n} {out}x{k}")
    assert_parity(got, oracle.matmul(w.data, k, out, x, n), exact_at(w.data, k, out, x, n),
                  f"streamed weights n={n} {out}x{k}")
    gpu.release(w)
