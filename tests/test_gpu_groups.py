"""GPU tests of contiguous weight groups (q8_weight_group_resident), through the
C-ABI: a decode group or gate/up pair whose members lie back to back in one
allocation runs the preloaded-head row-slice kernels (q8_gemv_hg*,
q8_gemv_hp16_*), and must give what the same weights made resident one by one
give (the tile kernels, or the two-slot row slices with gemv.group_pair = 0):

  * exact mode ("gemv.exact" = 1): every output and cache half bit-identical;
  * the default tree order: within 2e-6 + 1e-5 |ref| of the separate weights'
    exact result, the appended cache row within one f16 step, and within the
    same bar of the oracle (rmsnorm, matmul, silu_mul of oracle/q8_oracle.c).
    Where two orders of the same nb block values legitimately differ by more
    (K = 5760 with an outlier: sums that cancel), an output passes if the
    difference is within the reordering bound 2 nb u T (T the row's sum of
    |w x| in f64, u = 2^-24; for the SiLU product that bound carried through
    silu(g) * u, for a rotated q through the pair it mixes);
  * a second launch repeats the first bit for bit.

Shapes cover the configs[4] projections, grouped kv heads, member row counts
that leave padding rows inside the group (40 rows: a tile and a partial one),
K that takes six loads a lane, and K too long for the folded norm's register
budget (the launch then takes another kernel, with the same results).
"""
import numpy as np
import pytest

import oracle
from llm_amd import q8
from test_gpu_q8 import assert_bits

pytestmark = pytest.mark.gpu
SEED = 0x6A0
U = 2.0 ** -24


def reorder_bounds(datas, outs, k, xin):
    """Per member, the bound 2 nb u T on the difference between two summation
    orders of a row's nb block values (T = sum |w x| in f64)."""
    xa = np.abs(np.asarray(xin, np.float64))
    out = []
    for d, o in zip(datas, outs):
        rows = d.reshape(o, -1)
        t = np.array([np.abs(oracle.dequant_q8_0(rows[i], k).astype(np.float64)) @ xa for i in range(o)])
        out.append(2.0 * (k // 32) * U * t)
    return out


def assert_reordered(got, ref, allowance, what):
    """Within the f32 bar, or (another order of the same terms) within
    `allowance` per element."""
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    bar = 2e-6 + 1e-5 * np.abs(ref)
    bad = ~((d <= bar) | (d <= allowance))
    if bad.any():
        i = int(np.flatnonzero(bad)[0])
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} beyond the bar and the reordering bound; "
                             f"first at {i}: got {got[i]!r} ref {ref[i]!r} bound {allowance[i]:.3e}")


@pytest.fixture(scope="module")
def gpu():
    g = q8.Gpu(0)
    yield g
    g.close()


def f16_buffer(gpu, rows, kv_dim):
    host = np.full(rows * kv_dim, np.float16(-7.0), np.float16)
    b = gpu.alloc(host.nbytes)
    b.upload(host)
    return b


def run(gpu, kind, ws, xb, nw, ys, caches, pos, geom):
    eps = 1e-6
    k = ws[0].k
    if kind == "group":
        gpu.matmul_decode_group([(w, y, 0) for w, y in zip(ws, ys)], xb, 0, k)
    elif kind == "norm_group":
        gpu.norm_matmul_decode_group(nw, eps, [(w, y, 0) for w, y in zip(ws, ys)], xb, 0, k)
    elif kind == "qkv_rope":
        n_head, n_kv, n_rot, cap = geom
        gpu.norm_qkv_rope(nw, eps, ws[0], ws[1], ws[2], xb, 0, ys[0], 0, caches[0], caches[1], n_head, n_kv, 64,
                          n_rot, 10000.0, cap, pos)
    elif kind == "gate_up":
        gpu.gate_up_silu(ws[0], ws[1], xb, 0, 1, ys[0], 0)
    else:
        gpu.norm_gate_up_silu(nw, eps, ws[0], ws[1], xb, 0, ys[0], 0)
    gpu.sync()


CASES = [("qkv_rope", (2304, 2304, 2304), 2304), ("qkv_rope", (256, 128, 128), 256),
         ("group", (2304, 512, 768), 2304), ("group", (40, 72, 40), 96), ("norm_group", (1024, 256, 256), 1024),
         ("norm_group", (320, 40), 5760), ("norm_group", (40, 2304), 2304),
         ("gate_up", (5760, 5760), 2304), ("gate_up", (40, 40), 96), ("gate_up", (2304, 2304), 5760),
         ("norm_gate_up", (5760, 5760), 2304), ("norm_gate_up", (640, 640), 2304), ("norm_gate_up", (72, 72), 2304),
         ("norm_gate_up", (2304, 2304), 5760)]


# no_pair and pair_l6 / pair_l3 concern gate/up pairs only
VARIANTS = [(kind, outs, k, v) for kind, outs, k in CASES
            for v in ("default", "unit_layout", "no_pair", "pair_l6", "pair_l3")
            if v in ("default", "unit_layout") or kind in ("gate_up", "norm_gate_up")]


@pytest.mark.parametrize("kind,outs,k,variant", VARIANTS)
@pytest.mark.parametrize("exact", [1, 0])
def test_contiguous_group_equals_separate_weights(gpu, kind, outs, k, variant, exact):
    """unit_layout: the group built with gemv.slice_copy = 0 (its kernels read
    the unit layout); no_pair: a gate/up pair with gemv.group_pair = 0 (the
    two-slot row slices); pair_l6 / pair_l3: the paired slices with six or
    three loads a lane (gemv.pair_loads; three where K needs no more than 16
    waves, else the default)."""
    r = np.random.default_rng(SEED + sum(outs) + k + len(kind))
    datas = [oracle.make_q8_weight(r, o, k) for o in outs]
    sep = [q8.Weight(d.copy(), k, o) for d, o in zip(datas, outs)]
    grp = [q8.Weight(d.copy(), k, o) for d, o in zip(datas, outs)]
    pair = kind in ("gate_up", "norm_gate_up")
    x = (r.standard_normal(k) * 2.0).astype(np.float32)
    x[3] = 25.0
    nw = (1.0 + 0.1 * r.standard_normal(k)).astype(np.float32)
    xb = gpu.alloc(4 * k)
    xb.upload(x)
    geom, caches, pos = None, [None, None], None
    if kind == "qkv_rope":
        geom = (outs[0] // 64, outs[1] // 64, 64, 64)
        caches = [f16_buffer(gpu, 64, outs[1]) for _ in range(2)]
        pos = gpu.alloc(256)
        pos.upload(np.array([37, 0], np.int32))
    ny = 1 if kind in ("qkv_rope", "gate_up", "norm_gate_up") else len(outs)
    ys = [gpu.alloc(4 * outs[i]) for i in range(ny)]
    try:
        print(f"\n{kind} outs={outs} k={k} {variant} exact={exact}", flush=True)
        gpu.set_option("gemv.exact", 1)
        for w in sep:
            gpu.resident(w)
        run(gpu, kind, sep, xb, nw, ys, caches, pos, geom)
        want = [y.download(np.float32, outs[i]) for i, y in enumerate(ys)]
        want_c = [c.download(np.uint16, 64 * outs[1]).copy() for c in caches if c is not None]
        for c in caches:
            if c is not None:
                c.upload(np.full(64 * outs[1], np.float16(-7.0), np.float16))
        if variant == "unit_layout":
            gpu.set_option("gemv.slice_copy", 0)
        gpu.resident_group(grp, pair=pair)
        gpu.set_option("gemv.slice_copy", -1)
        if variant == "no_pair":
            gpu.set_option("gemv.group_pair", 0)
        if variant.startswith("pair_l"):
            gpu.set_option("gemv.pair_loads", int(variant[-1]))
        gpu.set_option("gemv.exact", exact)
        runs = []
        for _ in range(2):
            run(gpu, kind, grp, xb, nw, ys, caches, pos, geom)
            runs.append(([y.download(np.float32, outs[i]) for i, y in enumerate(ys)],
                         [c.download(np.uint16, 64 * outs[1]).copy() for c in caches if c is not None]))
        xo = oracle.rmsnorm(x, nw, 1e-6) if kind.startswith("norm") or kind == "qkv_rope" else x
        bounds = reorder_bounds(datas, outs, k, xo)
        if pair:  # carried through silu(g) * u (|silu'| < 1.1)
            g = oracle.matmul(datas[0], k, outs[0], xo, 1).reshape(-1).astype(np.float64)
            u = oracle.matmul(datas[1], k, outs[1], xo, 1).reshape(-1).astype(np.float64)
            bounds = [1.1 * np.abs(u) * bounds[0] + np.abs(g / (1.0 + np.exp(-g))) * bounds[1]]
        elif kind == "qkv_rope":  # a rotated q row mixes its pair
            bounds = [bounds[0] + bounds[0].reshape(-1, 2)[:, ::-1].reshape(-1)]
        for i, (g0, g1) in enumerate(zip(runs[0][0], runs[1][0])):
            assert_bits(g1, g0, f"{kind} output {i}: a second launch")
            if exact:
                assert_bits(g0, want[i], f"{kind} output {i} vs separate weights")
            else:
                assert_reordered(g0, want[i], bounds[i], f"{kind} output {i} (tree order) vs separate weights")
        for ci, (cg, cw) in enumerate(zip(runs[0][1], want_c)):
            cg, cw = cg.reshape(64, -1), cw.reshape(64, -1)
            if exact:
                assert np.array_equal(cg, cw), f"cache {ci}: {int((cg != cw).sum())} halves differ"
            else:
                others = [t for t in range(64) if t != 37]
                assert np.array_equal(cg[others], cw[others]), f"cache {ci}: rows off the position changed"
                a32 = cg[37].view(np.float16).astype(np.float32)
                b32 = cw[37].view(np.float16).astype(np.float32)
                assert (np.abs(a32 - b32) <= 2e-3 * np.abs(b32) + 1e-4).all(), f"cache {ci} position row"
        # the oracle on the same bytes (the un-rotated members only: rotation
        # has its own oracle tests)
        if pair:
            og = oracle.matmul(datas[0], k, outs[0], xo, 1)
            ou = oracle.matmul(datas[1], k, outs[1], xo, 1)
            assert_reordered(runs[0][0][0], oracle.silu_mul(og, ou).reshape(-1), bounds[0], f"{kind} vs oracle")
        elif kind != "qkv_rope":
            for i, (d, o) in enumerate(zip(datas, outs)):
                assert_reordered(runs[0][0][i], oracle.matmul(d, k, o, xo, 1).reshape(-1), bounds[i],
                                 f"{kind} member {i} vs oracle")
    finally:
        for name in ("gemv.exact", "gemv.group_pair", "gemv.slice_copy", "gemv.pair_loads"):
            gpu.set_option(name, -1)
        for b in [xb] + ys + [c for c in caches if c is not None] + ([pos] if pos else []):
            b.free()
        for w in sep + grp:
            gpu.release(w)


def test_group_members_stand_alone_and_release_in_any_order(gpu):
    """Members of a group are weights of their own: each exports its own GGUF
    bytes, runs alone (q8_matmul, the single-matrix row slices over its part
    of the group's allocation) bit-identical to a separately resident copy,
    stays usable after another member is released, and the allocation is
    returned when the last member goes (device free bytes back within 64 MiB
    over repeated cycles)."""
    r = np.random.default_rng(SEED)
    k, outs = 2304, (2304, 576, 576)
    datas = [oracle.make_q8_weight(r, o, k) for o in outs]
    x = r.standard_normal(k).astype(np.float32)
    xb, y1, y2 = gpu.alloc(4 * k), gpu.alloc(4 * 2304), gpu.alloc(4 * 2304)
    xb.upload(x)
    free0 = gpu.info()["free_bytes"]
    try:
        for cycle in range(3):
            grp = [q8.Weight(d.copy(), k, o) for d, o in zip(datas, outs)]
            gpu.resident_group(grp)
            for d, w in zip(datas, grp):
                assert np.array_equal(gpu.export(w), d.view(np.uint8).reshape(-1)), "member export"
            order = [1, 0, 2] if cycle % 2 == 0 else [2, 1, 0]
            for i in order:
                alone = q8.Weight(datas[i].copy(), k, outs[i])
                gpu.matmul(grp[i], xb, 0, 1, y1, 0)
                gpu.matmul(alone, xb, 0, 1, y2, 0)
                assert_bits(y1.download(np.float32, outs[i]), y2.download(np.float32, outs[i]), f"member {i} alone")
                gpu.release(alone)
                gpu.release(grp[i])
        gpu.sync()
        assert gpu.info()["free_bytes"] >= free0 - (64 << 20), "group allocations not returned"
    finally:
        for b in (xb, y1, y2):
            b.free()


def test_group_residency_errors(gpu):
    """A member already resident, a pair of two shapes, more than four members
    and a byte count that does not match the shape are refused with
    Q8_ERR_INVALID before anything is allocated; a refused call leaves no
    member resident."""
    r = np.random.default_rng(SEED + 1)
    k = 256
    a, b = q8.Weight(oracle.make_q8_weight(r, 64, k), k, 64), q8.Weight(oracle.make_q8_weight(r, 96, k), k, 96)
    gpu.resident(a)
    try:
        with pytest.raises(q8.Q8Error) as e:
            gpu.resident_group([a, b])
        assert e.value.status == q8.Q8_ERR_INVALID
        c = q8.Weight(oracle.make_q8_weight(r, 64, k), k, 64)
        with pytest.raises(q8.Q8Error) as e:
            gpu.resident_group([c, b], pair=True)
        assert e.value.status == q8.Q8_ERR_INVALID
        many = [q8.Weight(oracle.make_q8_weight(r, 32, k), k, 32) for _ in range(5)]
        with pytest.raises(q8.Q8Error) as e:
            gpu.resident_group(many)
        assert e.value.status == q8.Q8_ERR_INVALID
        # a byte count that is not outs x k Q8_0, through the C-ABI directly
        import ctypes
        d2 = oracle.make_q8_weight(r, 64, k)
        ptrs = (ctypes.c_void_p * 2)(c.data.ctypes.data, d2.ctypes.data)
        sizes = (ctypes.c_size_t * 2)(c.data.nbytes, d2.nbytes)
        outs = (ctypes.c_int * 2)(64, 63)
        hs = (ctypes.c_void_p * 2)()
        assert q8.lib().q8_weight_group_resident(gpu.handle, 2, ptrs, sizes, k, outs, 0, hs) == q8.Q8_ERR_INVALID
        assert "byte length" in q8.lib().q8_last_error().decode()
        # nothing of the refused calls stayed resident: c groups now
        gpu.resident_group([c, b])
        gpu.release(c)
        gpu.release(b)
    finally:
        gpu.release(a)
