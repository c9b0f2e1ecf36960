"""GPU tests of the decoder support kernels and the synthetic decoder, through
the C-ABI (include/q8decoder.h), against the CPU oracle.

Bars:
  * rope_append: rotated q within 2e-6 + 1e-5|ref| of oracle.rope (device
    powf/sincosf vs correctly rounded host values); the f16 value cache
    bit-exact (a pure narrowing); the f16 key cache equal to the narrowed
    oracle keys except where the f32 rotation differs in its last bit at an
    f16 rounding boundary (at most one f16 ulp, on at most 1% of elements);
    rows outside [position, position + n) and at or past capacity untouched;
  * attention (decode with 1..7 splits, prefill tiles): within 2e-6 + 1e-5|ref|
    of the exact value of the reference formula over the same f16 cache;
  * embeddings/argmax/advance on device memory: bit-exact / exact;
  * the decoder: logits of a prompt and of greedy decode steps against the
    oracle's composition of the reference ops on the same (exported) weights,
    within a whole-model tolerance (1e-3 relative to the logit scale: f16
    cache rounding and int8 activation rounding both flip on last-bit
    differences), identical greedy tokens wherever the oracle's top-2 gap
    exceeds that tolerance, and bit-identical replays of the captured graphs.
"""
from types import SimpleNamespace

import numpy as np
import pytest

import oracle
from llm_amd import decoder as dm
from llm_amd import q8
from test_gpu_q8 import assert_bits, assert_close

pytestmark = pytest.mark.gpu
SEED = 0x5EED


@pytest.fixture(scope="module")
def gpu():
    g = q8.Gpu(0)
    yield g
    g.close()


def f16_buffer(gpu, rows, kv_dim, fill=np.float16(-7.0)):
    host = np.full(rows * kv_dim, fill, np.float16)
    b = gpu.alloc(host.nbytes)
    b.upload(host)
    return b


def read_f16(buf, rows, kv_dim):
    return buf.download(np.uint16, rows * kv_dim).view(np.float16).reshape(rows, kv_dim)


def int_buffer(gpu, value):
    b = gpu.alloc(256)
    b.upload(np.array([value, 0], np.int32))
    return b


def q8w(r, out, k):
    return q8.Weight(oracle.make_q8_weight(r, out, k), k, out)


@pytest.mark.parametrize("outs,k", [((2304, 2304, 2304), 2304), ((2304,), 5760), ((320,), 768), ((96, 64), 32),
                                    ((1024, 256, 256), 1024), ((64,), 2304)])
@pytest.mark.parametrize("exact", [1, 0])
def test_norm_folded_decode_group_equals_norm_then_group(gpu, outs, k, exact):
    """q8_norm_matmul_decode_group: the fold (or, where the GEMV needs a K
    split or has fewer than 256 threads, the two-step path it takes instead)
    is bit-identical to q8_rmsnorm followed by q8_matmul_decode_group in exact
    mode, within the f32 bar of it in the tree order (the norm's scale then
    multiplies the row sums), and within the f32 bar of the oracle's
    rmsnorm + matmul in both."""
    gpu.set_option("gemv.exact", exact)
    r = np.random.default_rng(SEED + k + len(outs))
    ws = [q8w(r, o, k) for o in outs]
    x = (r.standard_normal(k) * 3.0).astype(np.float32)
    x[7] = -40.0
    nw = (1.0 + 0.1 * r.standard_normal(k)).astype(np.float32)
    eps = 1e-6
    xb, xn = gpu.alloc(4 * k), gpu.alloc(4 * k)
    xb.upload(x)
    ys = [gpu.alloc(4 * o) for o in outs]
    refs = [gpu.alloc(4 * o) for o in outs]
    try:
        gpu.rmsnorm(xb, 0, nw, eps, 1, xn)
        gpu.matmul_decode_group([(w, y, 0) for w, y in zip(ws, refs)], xn, 0, k)
        gpu.norm_matmul_decode_group(nw, eps, [(w, y, 0) for w, y in zip(ws, ys)], xb, 0, k)
        xo = oracle.rmsnorm(x, nw, eps)
        for i, (w, o) in enumerate(zip(ws, outs)):
            got = ys[i].download(np.float32, o)
            if exact:
                assert_bits(got, refs[i].download(np.float32, o), f"member {i} of {outs} k={k}")
            else:
                assert_close(got, refs[i].download(np.float32, o), f"member {i} of {outs} k={k} (tree order)")
            assert_close(got, oracle.matmul(w.data, k, o, xo, 1).reshape(-1), f"member {i} vs oracle")
    finally:
        gpu.set_option("gemv.exact", -1)
        for b in [xb, xn] + ys + refs:
            b.free()
        for w in ws:
            gpu.release(w)


@pytest.mark.parametrize("E,n_head,n_kv,n_rot,position,capacity", [(2304, 36, 36, 64, 511, 1024),
                                                                 (256, 4, 2, 64, 7, 32), (256, 4, 2, 32, 0, 16),
                                                                 (512, 8, 2, 64, 3, 8), (256, 4, 4, 64, 16, 16),
                                                                 (1024, 16, 4, 16, 4095, 4096)])
@pytest.mark.parametrize("exact", [1, 0])
def test_norm_qkv_rope_equals_norm_group_then_rope_append(gpu, E, n_head, n_kv, n_rot, position, capacity, exact):
    """q8_norm_qkv_rope (norm folded into the q/k/v GEMV, rotation and KV
    append in its epilogue) against q8_rmsnorm + q8_matmul_decode_group +
    q8_rope_append: the rotated q and both caches bit-identical in exact mode
    (in the tree order q within the f32 bar and the appended cache row within
    one f16 step), including partial rotation, grouped kv heads, a position
    at capacity (nothing appended, q unrotated) and the last cache row; cache
    rows elsewhere keep their fill."""
    gpu.set_option("gemv.exact", exact)
    r = np.random.default_rng(SEED + E + n_head + position)
    hd, base, eps = 64, 10000.0, 1e-6
    kv_dim = n_kv * hd
    wq, wk, wv = q8w(r, n_head * hd, E), q8w(r, kv_dim, E), q8w(r, kv_dim, E)
    x = (r.standard_normal(E) * 2.0).astype(np.float32)
    nw = (1.0 + 0.1 * r.standard_normal(E)).astype(np.float32)
    xb, xn = gpu.alloc(4 * E), gpu.alloc(4 * E)
    xb.upload(x)
    q1, k1, v1, q2 = gpu.alloc(4 * n_head * hd), gpu.alloc(4 * kv_dim), gpu.alloc(4 * kv_dim), gpu.alloc(4 * n_head * hd)
    kc1, vc1 = f16_buffer(gpu, capacity, kv_dim), f16_buffer(gpu, capacity, kv_dim)
    kc2, vc2 = f16_buffer(gpu, capacity, kv_dim), f16_buffer(gpu, capacity, kv_dim)
    pos = int_buffer(gpu, position)
    try:
        print(f"\nnorm_qkv_rope E={E} heads={n_head}/{n_kv} rot={n_rot} pos={position} cap={capacity}", flush=True)
        gpu.rmsnorm(xb, 0, nw, eps, 1, xn)
        gpu.matmul_decode_group([(wq, q1, 0), (wk, k1, 0), (wv, v1, 0)], xn, 0, E)
        gpu.rope_append(q1, k1, v1, kc1, vc1, 1, n_head, n_kv, hd, n_rot, base, capacity, pos)
        gpu.norm_qkv_rope(nw, eps, wq, wk, wv, xb, 0, q2, 0, kc2, vc2, n_head, n_kv, hd, n_rot, base, capacity, pos)
        gpu.sync()
        qg, qw = q2.download(np.float32, n_head * hd), q1.download(np.float32, n_head * hd)
        if exact:
            assert_bits(qg, qw, "rotated q")
        else:
            assert_close(qg, qw, "rotated q (tree order)")
        for name, a, b in (("key", kc2, kc1), ("value", vc2, vc1)):
            got = read_f16(a, capacity, kv_dim).view(np.uint16)
            want = read_f16(b, capacity, kv_dim).view(np.uint16)
            if exact:
                assert np.array_equal(got, want), f"{name} cache: {int((got != want).sum())} halves differ"
            else:
                g32, w32 = got.view(np.float16).astype(np.float32), want.view(np.float16).astype(np.float32)
                assert (np.abs(g32 - w32) <= 2e-3 * np.abs(w32) + 1e-4).all(), f"{name} cache beyond one f16 step"
        kg = read_f16(kc2, capacity, kv_dim)
        others = [t for t in range(capacity) if t != position]
        assert (kg[others] == np.float16(-7.0)).all(), "rows other than the position keep their fill"
    finally:
        gpu.set_option("gemv.exact", -1)
        for b in (xb, xn, q1, k1, v1, q2, kc1, vc1, kc2, vc2, pos):
            b.free()
        for w in (wq, wk, wv):
            gpu.release(w)


@pytest.mark.parametrize("E,n_head,n_kv,n_rot,n,position,capacity,option", [
    (2304, 36, 36, 64, 512, 0, 4096, None), (256, 4, 2, 32, 70, 37, 128, None), (512, 8, 2, 64, 40, 100, 128, None),
    (256, 4, 4, 64, 33, 0, 64, ("gemm.f16", 1)), (1024, 16, 4, 16, 64, 5, 256, ("gemm.pipe", 1)),
    (2304, 36, 36, 64, 48, 7, 256, ("gemm.slices", 3)), (256, 4, 2, 64, 2, 126, 128, None)])
def test_prompt_qkv_rope_equals_group_then_rope_append(gpu, E, n_head, n_kv, n_rot, n, position, capacity, option):
    """q8_prompt_qkv_rope (RoPE + KV append in the q/k/v GEMM's epilogue)
    against q8_matmul_prompt_group + q8_rope_append on the same prepared
    activations: the rotated q and both whole caches bit-identical, on the
    int8, f16-MFMA, pipelined and K-split GEMM paths, with partial rotation,
    grouped kv heads, and tokens past the cache's end (q unrotated, nothing
    appended)."""
    if option:
        gpu.set_option(*option)
    r = np.random.default_rng(SEED + E + n + position)
    hd, base = 64, 10000.0
    kv_dim = n_kv * hd
    wq, wk, wv = q8w(r, n_head * hd, E), q8w(r, kv_dim, E), q8w(r, kv_dim, E)
    x = oracle.make_activations(r, n, E)
    xb = gpu.alloc(4 * n * E)
    xb.upload(x)
    q1, q2 = gpu.alloc(4 * n * n_head * hd), gpu.alloc(4 * n * n_head * hd)
    k1, v1 = gpu.alloc(4 * n * kv_dim), gpu.alloc(4 * n * kv_dim)
    kc1, vc1 = f16_buffer(gpu, capacity, kv_dim), f16_buffer(gpu, capacity, kv_dim)
    kc2, vc2 = f16_buffer(gpu, capacity, kv_dim), f16_buffer(gpu, capacity, kv_dim)
    pos = int_buffer(gpu, position)
    try:
        print(f"\nprompt_qkv_rope E={E} heads={n_head}/{n_kv} rot={n_rot} n={n} pos={position} cap={capacity} "
              f"{option}", flush=True)
        p = gpu.prepare(xb, 0, n, E)
        gpu.matmul_prompt_group([(wq, q1, 0), (wk, k1, 0), (wv, v1, 0)], p, n, E)
        gpu.rope_append(q1, k1, v1, kc1, vc1, n, n_head, n_kv, hd, n_rot, base, capacity, pos)
        gpu.prompt_qkv_rope(wq, wk, wv, p, n, q2, kc2, vc2, n_head, n_kv, hd, n_rot, base, capacity, pos)
        gpu.sync()
        assert_bits(q2.download(np.float32, n * n_head * hd), q1.download(np.float32, n * n_head * hd), "rotated q")
        for name, a, b in (("key", kc2, kc1), ("value", vc2, vc1)):
            got = read_f16(a, capacity, kv_dim).view(np.uint16)
            want = read_f16(b, capacity, kv_dim).view(np.uint16)
            assert np.array_equal(got, want), f"{name} cache: {int((got != want).sum())} halves differ"
    finally:
        if option:
            gpu.set_option(option[0], -1)
        for b in (xb, q1, q2, k1, v1, kc1, vc1, kc2, vc2, pos):
            b.free()
        for w in (wq, wk, wv):
            gpu.release(w)


@pytest.mark.parametrize("ffn,k", [(5760, 2304), (640, 2304), (64, 2304), (2304, 5760)])
@pytest.mark.parametrize("exact", [1, 0])
def test_norm_folded_gate_up_silu_equals_norm_then_gate_up(gpu, ffn, k, exact):
    """q8_norm_gate_up_silu against q8_rmsnorm + q8_gate_up_silu: bit-identical
    in exact mode, within the f32 bar in the tree order; both within the bar
    of the oracle."""
    gpu.set_option("gemv.exact", exact)
    r = np.random.default_rng(SEED + ffn + k)
    gw, uw = q8w(r, ffn, k), q8w(r, ffn, k)
    x = (r.standard_normal(k) * 2.0).astype(np.float32)
    nw = (1.0 + 0.1 * r.standard_normal(k)).astype(np.float32)
    eps = 1e-6
    xb, xn, act, ref = gpu.alloc(4 * k), gpu.alloc(4 * k), gpu.alloc(4 * ffn), gpu.alloc(4 * ffn)
    xb.upload(x)
    try:
        gpu.rmsnorm(xb, 0, nw, eps, 1, xn)
        gpu.gate_up_silu(gw, uw, xn, 0, 1, ref, 0)
        gpu.norm_gate_up_silu(nw, eps, gw, uw, xb, 0, act, 0)
        got = act.download(np.float32, ffn)
        if exact:
            assert_bits(got, ref.download(np.float32, ffn), f"norm gate_up_silu ffn={ffn} k={k}")
        else:
            assert_close(got, ref.download(np.float32, ffn), f"norm gate_up_silu ffn={ffn} k={k} (tree order)")
        xo = oracle.rmsnorm(x, nw, eps)
        g = oracle.matmul(gw.data, k, ffn, xo, 1)
        u = oracle.matmul(uw.data, k, ffn, xo, 1)
        assert_close(got, oracle.silu_mul(g, u).reshape(-1), "norm gate_up_silu vs oracle")
    finally:
        gpu.set_option("gemv.exact", -1)
        for b in (xb, xn, act, ref):
            b.free()
        gpu.release(gw)
        gpu.release(uw)


def _run_decode_multi(gpu, kind, ws, xb, nw, ys, caches, pos, geom):
    """One multi-matrix decode launch of `kind` into ys (and the caches)."""
    eps = 1e-6
    if kind == "group":
        gpu.matmul_decode_group([(w, y, 0) for w, y in zip(ws, ys)], xb, 0, ws[0].k)
    elif kind == "norm_group":
        gpu.norm_matmul_decode_group(nw, eps, [(w, y, 0) for w, y in zip(ws, ys)], xb, 0, ws[0].k)
    elif kind == "qkv_rope":
        n_head, n_kv, n_rot, cap = geom
        gpu.norm_qkv_rope(nw, eps, ws[0], ws[1], ws[2], xb, 0, ys[0], 0, caches[0], caches[1], n_head, n_kv, 64,
                          n_rot, 10000.0, cap, pos)
    elif kind == "gate_up":
        gpu.gate_up_silu(ws[0], ws[1], xb, 0, 1, ys[0], 0)
    else:
        gpu.norm_gate_up_silu(nw, eps, ws[0], ws[1], xb, 0, ys[0], 0)


@pytest.mark.parametrize("kind,outs,k", [
    ("qkv_rope", (2304, 2304, 2304), 2304), ("qkv_rope", (256, 128, 128), 256), ("group", (2304, 512, 768), 2304),
    ("group", (96, 64), 32), ("norm_group", (1024, 256, 256), 1024), ("norm_group", (320, 40), 5760),
    ("gate_up", (5760, 5760), 2304), ("gate_up", (72, 72), 96), ("norm_gate_up", (5760, 5760), 2304),
    ("norm_gate_up", (2304, 2304), 5760), ("norm_gate_up", (640, 640), 2304)])
@pytest.mark.parametrize("rows,loads", [(8, 3), (16, 3), (16, 6)])
@pytest.mark.parametrize("exact", [1, 0])
def test_group_row_slices_equal_the_tile_kernel(gpu, kind, outs, k, rows, loads, exact):
    """The row-slice kernels over a decode group or the gate/up pair
    (q8_gemv_g*, q8_gemv_s*; options gemv.group_rows / gemv.group_loads),
    with the folded norm and the RoPE + KV append epilogue, against the
    multi-matrix tile kernel (gemv.group_rows = 0) in exact mode: every
    output and cache half bit-identical.  The tree order (exact = 0) stays
    within the f32 bar of the tile kernel's exact result and repeats bit for
    bit.  Shapes no built variant fits (K needing more than 16 waves, a
    folded norm on fewer than 256 threads) fall back to the tile kernel."""
    r = np.random.default_rng(SEED + sum(outs) + k + rows)
    ws = [q8w(r, o, k) for o in outs]
    x = (r.standard_normal(k) * 2.0).astype(np.float32)
    x[3] = 25.0
    nw = (1.0 + 0.1 * r.standard_normal(k)).astype(np.float32)
    xb = gpu.alloc(4 * k)
    xb.upload(x)
    geom, caches, pos = None, [None, None], None
    if kind == "qkv_rope":
        n_head, n_kv = outs[0] // 64, outs[1] // 64
        geom = (n_head, n_kv, 64, 64)
        caches = [f16_buffer(gpu, 64, outs[1]) for _ in range(2)]
        pos = int_buffer(gpu, 37)
    ny = 1 if kind in ("qkv_rope", "gate_up", "norm_gate_up") else len(outs)
    ys = [gpu.alloc(4 * outs[i]) for i in range(ny)]
    try:
        print(f"\n{kind} outs={outs} k={k} rows={rows} loads={loads} exact={exact}", flush=True)
        gpu.set_option("gemv.exact", 1)
        gpu.set_option("gemv.group_rows", 0)
        _run_decode_multi(gpu, kind, ws, xb, nw, ys, caches, pos, geom)
        want = [y.download(np.float32, outs[i]) for i, y in enumerate(ys)]
        want_c = [read_f16(c, 64, outs[1]).view(np.uint16).copy() for c in caches if c is not None]
        for c in caches:
            if c is not None:
                c.upload(np.full(64 * outs[1], np.float16(-7.0), np.float16))
        gpu.set_option("gemv.exact", exact)
        gpu.set_option("gemv.group_rows", rows)
        gpu.set_option("gemv.group_loads", loads)
        runs = []
        for _ in range(2):
            _run_decode_multi(gpu, kind, ws, xb, nw, ys, caches, pos, geom)
            runs.append(([y.download(np.float32, outs[i]) for i, y in enumerate(ys)],
                         [read_f16(c, 64, outs[1]).view(np.uint16).copy() for c in caches if c is not None]))
        for i, (g0, g1) in enumerate(zip(runs[0][0], runs[1][0])):
            assert_bits(g1, g0, f"{kind} output {i}: a second run")
            if exact:
                assert_bits(g0, want[i], f"{kind} output {i} vs the tile kernel")
            else:
                assert_close(g0, want[i], f"{kind} output {i} (tree order) vs the tile kernel")
        for ci, (cg, cw) in enumerate(zip(runs[0][1], want_c)):
            if exact:
                assert np.array_equal(cg, cw), f"cache {ci}: {int((cg != cw).sum())} halves differ"
            else:  # the rows other than the position keep their fill; the position row is close
                others = [t for t in range(64) if t != 37]
                assert np.array_equal(cg[others], cw[others])
                a32 = cg[37].view(np.float16).astype(np.float32)
                b32 = cw[37].view(np.float16).astype(np.float32)
                # one f16 ulp: the f32 values differ in their last bits and may
                # round to neighbouring halves
                assert (np.abs(a32 - b32) <= 2e-3 * np.abs(b32) + 1e-4).all(), f"cache {ci} position row"

    finally:
        gpu.set_option("gemv.exact", -1)
        gpu.set_option("gemv.group_rows", -1)
        gpu.set_option("gemv.group_loads", -1)
        for b in [xb] + ys + [c for c in caches if c is not None] + ([pos] if pos else []):
            b.free()
        for w in ws:
            gpu.release(w)


@pytest.mark.parametrize("n,n_head,n_kv,n_rot,position,capacity", [(5, 4, 2, 64, 7, 32), (1, 36, 36, 64, 511, 1024),
                                                                   (40, 4, 4, 32, 3, 64), (6, 2, 1, 64, 30, 32)])
def test_rope_append_matches_the_oracle(gpu, n, n_head, n_kv, n_rot, position, capacity):
    """The last case runs past the capacity: rows from there on are not
    written (and their queries not rotated: the host reports the full context
    before such a call)."""
    r = np.random.default_rng(SEED + n)
    hd, base = 64, 10000.0
    kv_dim = n_kv * hd
    q = r.standard_normal((n, n_head, hd)).astype(np.float32)
    k = r.standard_normal((n, n_kv, hd)).astype(np.float32)
    v = r.standard_normal((n, n_kv, hd)).astype(np.float32)
    qb, kb, vb = (gpu.alloc(a.nbytes) for a in (q, k, v))
    qb.upload(q)
    kb.upload(k)
    vb.upload(v)
    extra = 8  # rows past capacity that must stay untouched
    kc, vc = f16_buffer(gpu, capacity + extra, kv_dim), f16_buffer(gpu, capacity + extra, kv_dim)
    pos = int_buffer(gpu, position)
    print(f"\nrope n={n} heads={n_head}/{n_kv} rot={n_rot} pos={position}", flush=True)
    gpu.rope_append(qb, kb, vb, kc, vc, n, n_head, n_kv, hd, n_rot, base, capacity, pos)
    gpu.sync()
    q_ref = oracle.rope(q, position, n_rot, base)
    k_ref = oracle.to_f16(oracle.rope(k, position, n_rot, base)).reshape(n, kv_dim)
    v_ref = oracle.to_f16(v).reshape(n, kv_dim)
    live = min(n, capacity - position)
    assert_close(qb.download(np.float32, q.size).reshape(q.shape)[:live], q_ref[:live], "rotated q")
    kg, vg = read_f16(kc, capacity + extra, kv_dim), read_f16(vc, capacity + extra, kv_dim)
    rows = slice(position, position + live)
    assert np.array_equal(vg[rows].view(np.uint16), v_ref[:live].view(np.uint16)), "value cache not bit-exact"
    diff = kg[rows].view(np.uint16).astype(np.int32) - k_ref[:live].view(np.uint16).astype(np.int32)
    assert np.abs(diff).max() <= 1 and (diff != 0).mean() <= 0.01, f"key cache: {int((diff != 0).sum())} differ"
    untouched = np.ones(capacity + extra, bool)
    untouched[rows] = False
    assert (kg[untouched] == np.float16(-7.0)).all() and (vg[untouched] == np.float16(-7.0)).all()


def cache_pair(gpu, r, L, capacity, n_kv, hd=64):
    k = oracle.to_f16(r.standard_normal((capacity, n_kv, hd)))
    v = oracle.to_f16(r.standard_normal((capacity, n_kv, hd)))
    kc, vc = gpu.alloc(k.nbytes), gpu.alloc(v.nbytes)
    kc.upload(k.view(np.uint16))
    vc.upload(v.view(np.uint16))
    return k.astype(np.float32), v.astype(np.float32), kc, vc


ATTN_CASES = [(1, 1, 4, 2), (200, 1, 4, 2), (200, 3, 4, 4), (200, 7, 8, 2), (640, 10, 36, 36), (4096, 16, 4, 1),
              (600, 3, 36, 36), (2400, 5, 36, 36)]


# waves: option attn.waves (-1 the default choice; 4 or 8 forced on the split kernel)
@pytest.mark.parametrize("visible,splits,n_head,n_kv,waves",
                         [c + (w,) for c in ATTN_CASES for w in (-1, 4, 8) if w < 0 or c[1] > 1])
def test_decode_attention_matches_the_oracle(gpu, visible, splits, n_head, n_kv, waves):
    """The split kernel's 256-row chunks over four or eight waves (by default
    eight while heads x splits workgroups fit one per CU) and the one-split
    16-wave kernel, against the exact attention formula."""
    gpu.set_option("attn.waves", waves)
    r = np.random.default_rng(SEED + visible + splits)
    capacity = max(visible, 256)
    kf, vf, kc, vc = cache_pair(gpu, r, visible, capacity, n_kv)
    q = (r.standard_normal((1, n_head, 64)) * 2).astype(np.float32)
    qb, out = gpu.alloc(q.nbytes), gpu.alloc(q.nbytes)
    qb.upload(q)
    pos = int_buffer(gpu, visible - 1)
    print(f"\ndecode attention visible={visible} splits={splits} heads={n_head}/{n_kv}", flush=True)
    try:
        gpu.attention(qb, kc, vc, out, 1, n_head, n_kv, 64, capacity, 0.125, pos, splits)
        got = out.download(np.float32, q.size).reshape(q.shape)
    finally:
        gpu.set_option("attn.waves", -1)
    assert_close(got, oracle.attention(q, kf, vf, visible - 1, 0.125), f"decode attention L={visible} s={splits}")


@pytest.mark.parametrize("visible,splits,n_head,n_kv", [(1, 1, 4, 2), (200, 1, 36, 36), (600, 3, 36, 36),
                                                        (640, 8, 36, 36), (4096, 8, 4, 1), (3000, 5, 8, 2),
                                                        (2000, 12, 8, 8), (300, 2, 32, 8)])
@pytest.mark.parametrize("exact,rows,loads", [(1, -1, -1), (1, 8, 2), (1, 8, 3), (1, 8, 6), (1, 16, 6), (1, 32, -1),
                                               (0, -1, -1), (0, 8, 2)])
def test_attention_matmul_add_equals_attention_then_matmul(gpu, visible, splits, n_head, n_kv, exact, rows, loads):
    """q8_attention_matmul_add: the partials combined in the output
    projection's GEMV prologue (or, past eight splits, the two calls it makes
    instead) give y bit-identical to q8_attention with the same splits then
    q8_matmul with y as the residual; and the attention alone is within the
    f32 bar of the oracle.  rows/loads: the row-slice kernels q8_gemv_rc8_l{2,3,6}
    and q8_gemv_rc16_l{3,6} (-1: the tactic's choice), where fewer threads than x has float4s
    build the rest of x in turn, or the tile kernel (32).  Only splits > 8
    (the 12-split case) leave the folded combine for the two calls."""
    gpu.set_option("gemv.exact", exact)
    gpu.set_option("gemv.rows", rows)
    gpu.set_option("gemv.loads", loads)
    r = np.random.default_rng(SEED + 7 * visible + splits)
    capacity = max(visible, 256)
    kf, vf, kc, vc = cache_pair(gpu, r, visible, capacity, n_kv)
    E = n_head * 64
    q = (r.standard_normal((1, n_head, 64)) * 2).astype(np.float32)
    wo = q8w(r, E, E)
    y0 = r.standard_normal(E).astype(np.float32)
    qb, att, yref, yf = gpu.alloc(q.nbytes), gpu.alloc(q.nbytes), gpu.alloc(4 * E), gpu.alloc(4 * E)
    qb.upload(q)
    yref.upload(y0)
    yf.upload(y0)
    pos = int_buffer(gpu, visible - 1)
    try:
        print(f"\nattention + O visible={visible} splits={splits} heads={n_head}/{n_kv} exact={exact} rows={rows} "
              f"loads={loads}", flush=True)
        gpu.attention(qb, kc, vc, att, 1, n_head, n_kv, 64, capacity, 0.125, pos, splits)
        gpu.matmul(wo, att, 0, 1, yref, 0, bias=yref)
        gpu.attention_matmul_add(qb, kc, vc, n_head, n_kv, 64, capacity, 0.125, pos, splits, wo, yf)
        assert_bits(yf.download(np.float32, E), yref.download(np.float32, E), "fused attention + O projection")
        a_ref = oracle.attention(q, kf, vf, visible - 1, 0.125)
        assert_close(att.download(np.float32, q.size).reshape(q.shape), a_ref, "attention vs oracle")
    finally:
        gpu.set_option("gemv.exact", -1)
        gpu.set_option("gemv.rows", -1)
        gpu.set_option("gemv.loads", -1)
        for b in (qb, att, yref, yf, kc, vc, pos):
            b.free()
        gpu.release(wo)


@pytest.mark.parametrize("n,start,n_head,n_kv,f16", [(512, 0, 36, 36, -1), (70, 37, 4, 2, -1), (33, 0, 8, 8, 1),
                                                     (2, 100, 4, 1, -1), (200, 5, 16, 4, 1)])
def test_attention_prepare_equals_attention_then_prepare(gpu, n, start, n_head, n_kv, f16):
    """q8_attention_prepare (each prompt-attention workgroup quantizing its
    own heads' blocks) against q8_attention + q8_prepare of its f32 rows: the
    prepared quants and scales bit-identical, padding tokens of the last tile
    included, in the int8 and f16 unit formats."""
    gpu.set_option("gemm.f16", f16)
    r = np.random.default_rng(SEED + 3 * n + start)
    capacity = start + n + 16
    kf, vf, kc, vc = cache_pair(gpu, r, start + n, capacity, n_kv)
    q = (r.standard_normal((n, n_head, 64)) * 2).astype(np.float32)
    qb, out = gpu.alloc(q.nbytes), gpu.alloc(q.nbytes)
    qb.upload(q)
    pos = int_buffer(gpu, start)
    try:
        print(f"\nattention_prepare n={n} start={start} heads={n_head}/{n_kv} f16={f16}", flush=True)
        gpu.attention(qb, kc, vc, out, n, n_head, n_kv, 64, capacity, 0.125, pos)
        ref = gpu.prepare(out, 0, n, n_head * 64)
        unit = 2048 if ref.format == q8.PREPARED_F16 else 1024
        nb, tt = n_head * 2, (n + 31) // 32

        def raw(ptr, nbytes):
            host = np.empty(nbytes, np.uint8)
            q8._check(q8.lib().q8_download(gpu.handle, host.ctypes.data, ptr, nbytes))
            return host
        want_q, want_s = raw(ref.quants, tt * nb * unit), raw(ref.scales, 4 * tt * nb * 32)
        # the same workspace receives both: fill it with other activations first
        out.upload((r.standard_normal(q.size) * 5).astype(np.float32))
        other = gpu.prepare(out, 0, n, n_head * 64)
        assert not np.array_equal(raw(other.scales, 4 * tt * nb * 32), want_s)
        got = gpu.attention_prepare(qb, kc, vc, n, n_head, n_kv, 64, capacity, 0.125, pos)
        assert got.format == ref.format and got.n == n and got.k == n_head * 64
        assert np.array_equal(raw(got.quants, tt * nb * unit), want_q), "prepared quants differ"
        assert np.array_equal(raw(got.scales, 4 * tt * nb * 32), want_s), "prepared scales differ"
    finally:
        gpu.set_option("gemm.f16", -1)
        for b in (qb, out, kc, vc, pos):
            b.free()


@pytest.mark.parametrize("n,start,n_head,n_kv", [(2, 0, 4, 2), (64, 0, 4, 4), (100, 0, 2, 1), (130, 37, 4, 2),
                                                 (512, 0, 36, 36)])
def test_prefill_attention_matches_the_oracle(gpu, n, start, n_head, n_kv):
    r = np.random.default_rng(SEED + n + start)
    capacity = start + n + 16
    kf, vf, kc, vc = cache_pair(gpu, r, start + n, capacity, n_kv)
    q = (r.standard_normal((n, n_head, 64)) * 2).astype(np.float32)
    qb, out = gpu.alloc(q.nbytes), gpu.alloc(q.nbytes)
    qb.upload(q)
    pos = int_buffer(gpu, start)
    print(f"\nprefill attention n={n} start={start} heads={n_head}/{n_kv}", flush=True)
    gpu.attention(qb, kc, vc, out, n, n_head, n_kv, 64, capacity, 0.125, pos)
    got = out.download(np.float32, q.size).reshape(q.shape)
    ref = oracle.attention(q, kf, vf, start, 0.125) if n <= 130 else None
    if ref is None:  # the large case: check a sample of rows against the oracle
        rows = [0, 1, 63, 64, 255, 511]
        ref = np.stack([oracle.attention(q[t:t + 1], kf, vf, start + t, 0.125)[0] for t in rows])
        got = got[rows]
    assert_close(got, ref, f"prefill attention n={n} start={start}")


def test_device_token_ops(gpu):
    r = np.random.default_rng(SEED)
    data = oracle.make_q8_weight(r, 300, 96)
    w = q8.Weight(data, 96, 300)
    ids = np.array([5, 299, 0, 1000], np.uint32)  # 1000: outside the vocabulary -> zero row
    tb = gpu.alloc(16)
    tb.upload(ids)
    out = gpu.alloc(4 * 4 * 96)
    gpu.embeddings_device(w, tb, 4, out, 0)
    got = out.download(np.float32, 4 * 96).reshape(4, 96)
    rows = data.reshape(300, -1)
    for i, t in enumerate(ids[:3]):
        assert_bits(got[i], oracle.dequant_q8_0(rows[t], 96), f"row {t}")
    assert (got[3].view(np.uint32) == 0).all()
    vals = r.standard_normal(5000).astype(np.float32)
    vb = gpu.alloc(vals.nbytes)
    vb.upload(vals)
    gpu.argmax_device(vb, 0, vals.size, tb)
    pos = int_buffer(gpu, 10)
    gpu.advance_position(pos, 7)
    gpu.advance_position(pos, 1)
    assert int(tb.download(np.uint32, 1)[0]) == oracle.argmax(vals)
    assert int(pos.download(np.int32, 1)[0]) == 18


@pytest.mark.parametrize("vocab,k,ties,nan,norm", [(122880, 2304, False, False, True), (1000, 256, False, False, True),
                                                   (4096, 512, True, False, True), (4096, 512, True, False, False),
                                                   (333, 96, False, True, True), (70000, 2304, True, False, False)])
@pytest.mark.parametrize("exact", [1, 0])
def test_norm_lm_head_argmax_equals_norm_matmul_argmax(gpu, vocab, k, ties, nan, norm, exact):
    """q8_norm_lm_head_argmax (the lm_head GEMV leaving each tile's best
    candidate, then one workgroup choosing) against q8_rmsnorm + q8_matmul +
    q8_argmax_device: the same token, including equal maxima in different
    tiles and inside a tile (the lowest index wins), a NaN input (every logit
    NaN: token 0), a vocabulary that ends inside a tile, and no norm; the
    logits bit-identical in exact mode (in the tree order within the f32 bar:
    the partials need the tile kernel, where a small matmul takes row
    slices); the token always equals the oracle's argmax over the device's
    own logits."""
    gpu.set_option("gemv.exact", exact)
    r = np.random.default_rng(SEED + vocab + k)
    data = oracle.make_q8_weight(r, vocab, k)
    x = (r.standard_normal(k) * 2).astype(np.float32)
    if nan:
        x[5] = np.nan
    nw = (1.0 + 0.1 * r.standard_normal(k)).astype(np.float32)
    copies = (3, 17, 40, vocab // 2, vocab - 1)
    if ties:  # the oracle's top row, its scales doubled (a clear maximum), copied: equal maxima across tiles
        src = oracle.argmax(oracle.matmul(data, k, vocab, oracle.rmsnorm(x, nw, 1e-6) if norm else x, 1))
        rows = data.reshape(vocab, -1)
        blocks = rows[src].reshape(k // 32, 34)
        d = blocks[:, :2].copy().view(np.float16)
        blocks[:, :2] = (d.astype(np.float32) * 2).astype(np.float16).view(np.uint8).reshape(-1, 2)
        rows[src] = blocks.reshape(-1)
        for dst in copies:
            rows[dst] = rows[src]
    w = q8.Weight(data, k, vocab)
    xb, xn, la, lb = gpu.alloc(4 * k), gpu.alloc(4 * k), gpu.alloc(4 * vocab), gpu.alloc(4 * vocab)
    ta, tb = gpu.alloc(256), gpu.alloc(256)
    xb.upload(x)
    try:
        print(f"\nlm_head argmax vocab={vocab} k={k} ties={ties} nan={nan} norm={norm} exact={exact}", flush=True)
        if norm:
            gpu.rmsnorm(xb, 0, nw, 1e-6, 1, xn, 0)
            gpu.matmul(w, xn, 0, 1, la, 0)
        else:
            gpu.matmul(w, xb, 0, 1, la, 0)
        gpu.argmax_device(la, 0, vocab, ta)
        gpu.norm_lm_head_argmax(nw if norm else None, 1e-6, w, xb, 0, lb, 0, tb)
        want, got = int(ta.download(np.uint32, 1)[0]), int(tb.download(np.uint32, 1)[0])
        ga, gb = la.download(np.float32, vocab), lb.download(np.float32, vocab)
        if exact:
            assert_bits(gb, ga, "logits")
            assert got == want
        elif not nan:  # the tile kernel's block tree, where the plain matmul may take row slices
            assert_close(gb, ga, "logits (tree order)")
        assert got == oracle.argmax(gb), f"token {got}, oracle argmax of the same logits {oracle.argmax(gb)}"
        if nan:
            assert got == 0
        if ties:
            assert got == min(min(copies), src), f"token {got}: the lowest of the equal maxima is {min(min(copies), src)}"
    finally:
        gpu.set_option("gemv.exact", -1)
        for b in (xb, xn, la, lb, ta, tb):
            b.free()
        gpu.release(w)


def test_synthetic_weights_are_valid_q8_0_and_seeded(gpu):
    a = gpu.weight_synthetic(2304, 96, seed=7)
    b = gpu.weight_synthetic(2304, 96, seed=7)
    c = gpu.weight_synthetic(2304, 96, seed=8)
    ea, eb, ec = gpu.export(a), gpu.export(b), gpu.export(c)
    assert np.array_equal(ea, eb) and not np.array_equal(ea, ec)
    blk = ea.reshape(-1, 34)
    qv = blk[:, 2:].view(np.int8)
    d = blk[:, :2].copy().view(np.float16).astype(np.float32)
    assert qv.min() >= -127 and qv.max() <= 127 and abs(float(qv.mean())) < 1.0
    assert (d >= 0).all() and np.isfinite(d).all() and 0.5e-4 < float(np.median(d)) < 2e-4
    x = np.random.default_rng(SEED).standard_normal(2304).astype(np.float32)
    xb, yb = gpu.alloc(x.nbytes), gpu.alloc(96 * 4)
    xb.upload(x)
    gpu.matmul(a, xb, 0, 1, yb, 0)
    assert_close(yb.download(np.float32, 96), oracle.matmul(ea, 2304, 96, x, 1)[0], "GEMV on a synthetic weight")
    for w in (a, b, c):
        gpu.release_device(w)


# ---- the decoder against the oracle's composition of the reference ops ----

def small_config():
    return dm.config(n_layer=2, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, head_dim=64, n_vocab=1000,
                     capacity=96, max_batch=80)


class OracleDecoder:
    """Model::body (model.rs:755-826) composed from the oracle's restatements of
    the reference ops, over the decoder's exported weights."""

    def __init__(self, gpu, dec, perturb=0.0):
        """perturb: scale every embedded row by (1 + perturb) -- with 2**-23,
        a change of the input's last bit, which measures how far the model
        itself moves under one-ulp differences (the whole-model bar)."""
        c = self.cfg = dec.cfg
        self.perturb = perturb
        if gpu is not None:
            self.embd = gpu.export(dec.weight(-1))
            self.out = gpu.export(dec.weight(-1, dm.OUTPUT))  # the embedding itself when tied
            self.w = {(l, i): gpu.export(dec.weight(l, i)) for l in range(c.n_layer) for i in range(7)}
            self.norms = {(l, i): dec.norm(l, i) for l in range(c.n_layer) for i in range(2)}
            self.out_norm = dec.norm(-1)
        self.kc = [np.zeros((c.capacity, c.n_head_kv, c.head_dim), np.float32) for _ in range(c.n_layer)]
        self.vc = [np.zeros((c.capacity, c.n_head_kv, c.head_dim), np.float32) for _ in range(c.n_layer)]
        self.kv_dim = c.n_head_kv * c.head_dim
        self.pos = 0

    def twin(self, perturb):
        """A fresh oracle over the same weights (empty cache, position 0)."""
        t = OracleDecoder(None, SimpleNamespace(cfg=self.cfg), perturb)
        t.embd, t.out, t.w, t.norms, t.out_norm = self.embd, self.out, self.w, self.norms, self.out_norm
        return t

    def mm(self, data, k, out, x):
        x = np.asarray(x, np.float32)
        return oracle.matmul(data, k, out, x.reshape(-1), x.shape[0]).reshape(x.shape[0], out)

    def norm_rows(self, x, w):
        return np.stack([oracle.rmsnorm(row, w, self.cfg.eps) for row in x])

    def forward(self, tokens):
        c, E = self.cfg, self.cfg.n_embd
        n = len(tokens)
        rows = self.embd.reshape(c.n_vocab, -1)
        x = np.stack([oracle.dequant_q8_0(rows[t], E) for t in tokens]).astype(np.float32)
        if self.perturb:
            x = (x * np.float32(1.0 + self.perturb)).astype(np.float32)
        H, KV, hd = c.n_head, c.n_head_kv, c.head_dim
        for l in range(c.n_layer):
            h = self.norm_rows(x, self.norms[(l, 0)])
            q = self.mm(self.w[(l, dm.Q)], E, H * hd, h).reshape(n, H, hd)
            k = self.mm(self.w[(l, dm.K)], E, KV * hd, h).reshape(n, KV, hd)
            v = self.mm(self.w[(l, dm.V)], E, KV * hd, h).reshape(n, KV, hd)
            q = oracle.rope(q, self.pos, c.n_rot, c.rope_base)
            k = oracle.rope(k, self.pos, c.n_rot, c.rope_base)
            self.kc[l][self.pos:self.pos + n] = oracle.to_f16(k).astype(np.float32)
            self.vc[l][self.pos:self.pos + n] = oracle.to_f16(v).astype(np.float32)
            a = oracle.attention(q, self.kc[l], self.vc[l], self.pos, 1.0 / np.sqrt(np.float32(hd)))
            x = (x + self.mm(self.w[(l, dm.O)], H * hd, E, a.reshape(n, -1))).astype(np.float32)
            h = self.norm_rows(x, self.norms[(l, 1)])
            g = self.mm(self.w[(l, dm.GATE)], E, c.n_ff, h)
            u = self.mm(self.w[(l, dm.UP)], E, c.n_ff, h)
            act = oracle.silu_mul(g, u).reshape(n, c.n_ff)
            x = (x + self.mm(self.w[(l, dm.DOWN)], c.n_ff, E, act)).astype(np.float32)
        self.pos += n
        last = oracle.rmsnorm(x[-1], self.out_norm, c.eps)
        return self.mm(self.out, E, c.n_vocab, last[None])[0]


def check_logits(got, ref, what, tol=None):
    """Whole-model bar: max |d| <= tol (default 1e-3 of the logit scale), and
    the same greedy token wherever the oracle's top-2 gap exceeds 2 tol."""
    if tol is None:
        tol = 1e-3 * float(np.abs(ref).max())
    d = np.abs(got.astype(np.float64) - ref)
    print(f"{what}: max |d| {d.max():.3e} (bar {tol:.3e}, logit scale {float(np.abs(ref).max()):.3e})", flush=True)
    assert d.max() <= tol, f"{what}: max |d| {d.max():.3e} > {tol:.3e}"
    top2 = np.sort(ref)[-2:]
    if top2[1] - top2[0] > 2 * tol:
        assert int(np.argmax(got)) == oracle.argmax(ref), f"{what}: greedy token differs"


def model_bar(ref_logits, twin_logits):
    """The bar for a model whose own logits move by max|ref - twin| when its
    input changes in the last bit: twice that, and at least 1e-3 of the logit
    scale.  Activation quantization (round half away at a .5 boundary) and the
    f16 cache narrowing turn last-bit differences into whole quantization
    steps, so a deep or wide model amplifies them; the device's own last-bit
    differences from the reference's summation order do the same."""
    sens = float(np.abs(ref_logits.astype(np.float64) - twin_logits).max())
    return max(1e-3 * float(np.abs(ref_logits).max()), 2.0 * sens), sens


def test_decoder_prompt_and_decode_steps_match_the_oracle(gpu):
    dec = dm.Decoder(gpu, small_config(), seed=11)
    try:
        ref = OracleDecoder(gpu, dec)
        prompt = np.random.default_rng(SEED).integers(0, 1000, 70).astype(np.uint32)
        print("\ndecoder prompt of 70", flush=True)
        nxt = dec.forward(prompt)
        ref_logits = ref.forward(prompt)
        got = dec.logits()
        check_logits(got, ref_logits, "prompt logits")
        assert nxt == int(np.argmax(got))
        steps = dec.generate(4)  # eager step, then captured replays
        assert dec.position == 74
        feed = [nxt] + [int(t) for t in steps[:-1]]
        for i, tok in enumerate(feed):
            logits = ref.forward([tok])
            top2 = np.sort(logits)[-2:]
            if top2[1] - top2[0] > 2e-3 * np.abs(logits).max():
                assert int(steps[i]) == oracle.argmax(logits), f"decode step {i}"
        check_logits(dec.logits(), logits, "last decode step logits")
    finally:
        dec.close()


@pytest.mark.parametrize("embd_std", [1.0, 4.0])
def test_decoder_greedy_feedback_varies_through_the_captured_graph(gpu, embd_std):
    """Greedy decode whose tokens change from step to step, fed back on the
    device through the captured step graph: a model with its own output head
    (a GGUF with output.weight, model.rs:519-524) and an embedding scale at
    which the current token shows in the last hidden state.  Each step's
    logits against the oracle decoder fed the same tokens; the device's token
    is the argmax of its logits, and the oracle's wherever the oracle's top-2
    gap clears the bar; at least two distinct tokens over the steps."""
    cfg = small_config()
    cfg.untied_output = 1
    cfg.embd_std = embd_std
    dec = dm.Decoder(gpu, cfg, seed=21)
    try:
        ref = OracleDecoder(gpu, dec)
        assert not np.array_equal(ref.out, ref.embd), "the output head is a matrix of its own"
        prompt = np.random.default_rng(SEED + 5).integers(0, cfg.n_vocab, 24).astype(np.uint32)
        print(f"\nuntied decoder, embd_std {embd_std}: prompt of 24, then 10 steps", flush=True)
        tokens = [dec.forward(prompt)]
        check_logits(dec.logits(), ref.forward(prompt), "untied prompt logits")
        for i in range(10):  # one step a call: eager, then captured, then graph replays
            t = int(dec.generate(1)[0])
            got = dec.logits()
            want = ref.forward([tokens[-1]])
            check_logits(got, want, f"untied step {i}")
            assert t == int(np.argmax(got)), f"step {i}: the token is the argmax of the step's logits"
            tokens.append(t)
        stats = dec.graph_stats()
        print(f"tokens {tokens}, graphs {stats}", flush=True)
        assert stats["captured"] >= 1 and stats["graphs"] >= 1, stats
        assert len(set(tokens)) >= 2, f"greedy decode repeated one token: {tokens}"
    finally:
        dec.close()


def test_decoder_graph_replays_are_bit_identical(gpu):
    dec = dm.Decoder(gpu, small_config(), seed=12)
    try:
        prompt = np.arange(1, 41, dtype=np.uint32)
        runs = []
        for _ in range(3):  # eager, capture + replay, replay
            dec.reset()
            first = dec.forward(prompt)
            toks = dec.generate(6)
            runs.append((first, toks.copy(), dec.logits()))
        for first, toks, logits in runs[1:]:
            assert first == runs[0][0] and np.array_equal(toks, runs[0][1])
            assert_bits(logits, runs[0][2], "replayed logits")
    finally:
        dec.close()


def test_prompt_weight_announcements_change_no_bits(gpu):
    """A prompt pass announces each next projection's weights
    (q8_gemm_prefetch: cache riders in the launch before); with the
    announcements switched off (option gemm.prefetch = 0) the prompt's token
    and logits are the same bits, eagerly and through the captured graph."""
    prompt = np.arange(1, 41, dtype=np.uint32)
    runs = []
    try:
        for pf in (0, 1):
            gpu.set_option("gemm.prefetch", pf)
            dec = dm.Decoder(gpu, small_config(), seed=12)
            try:
                for _ in range(3):  # eager, capture + replay, replay
                    dec.reset()
                    runs.append((pf, dec.forward(prompt), dec.logits()))
                assert dec.graph_stats()["captured"] >= 1
            finally:
                dec.close()
    finally:
        gpu.set_option("gemm.prefetch", -1)
    for pf, token, logits in runs[1:]:
        assert token == runs[0][1], f"announcements {pf}: token {token} against {runs[0][1]}"
        assert_bits(logits, runs[0][2], f"prompt logits, announcements {pf}")


def test_decoders_in_turn_on_one_context_agree(gpu):
    """Two decoders with the same seed, one after the other on one context,
    give bit-identical tokens and logits (eager and replayed): the first one's
    norm vectors, cached by host address, are released with it and cannot be
    found again at a reused address."""
    cfg = dm.config(n_layer=3, n_embd=256, n_ff=512, n_head=4, n_head_kv=2, head_dim=64, n_vocab=1000,
                    capacity=128, max_batch=64)
    results = []
    for _ in range(2):
        dec = dm.Decoder(gpu, cfg, seed=21)
        try:
            prompt = np.arange(3, 27, dtype=np.uint32)
            for _ in range(3):  # eager, capture + replay, replay
                dec.reset()
                first = dec.forward(prompt)
                toks = dec.generate(5)
                results.append((first, toks.copy(), dec.logits()))
        finally:
            dec.close()
    for first, toks, logits in results[1:]:
        assert first == results[0][0] and np.array_equal(toks, results[0][1])
        assert_bits(logits, results[0][2], "logits of the second decoder")


def test_decoder_errors(gpu):
    dec = dm.Decoder(gpu, small_config(), seed=13)
    try:
        with pytest.raises(q8.Q8Error) as e:
            dec.forward([1, 1000])
        assert e.value.status == q8.Q8_ERR_INVALID and "outside vocabulary" in e.value.message
        with pytest.raises(q8.Q8Error) as e:
            dec.forward([])
        assert e.value.status == q8.Q8_ERR_INVALID
        with pytest.raises(q8.Q8Error) as e:
            dec.generate(1)  # nothing to feed yet
        assert e.value.status == q8.Q8_ERR_INVALID
        dec.forward(np.zeros(80, np.uint32))
        with pytest.raises(q8.Q8Error) as e:
            dec.generate(17)  # 80 + 17 > capacity 96
        assert e.value.status == q8.Q8_ERR_UNSUPPORTED and "context full" in e.value.message
        assert dec.position == 80
        assert len(dec.generate(16)) == 16 and dec.position == 96
    finally:
        dec.close()
