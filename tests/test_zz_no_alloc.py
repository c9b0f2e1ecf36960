"""q8_matmul_noalloc (include/q8mi.h) through the C-ABI against q8_matmul on
the same inputs: two calls in a row, the second with a smaller input (the
static scratch keeps the first call's bytes, which the second must not see),
to the n >= 2 parity bar, bit-identical where q8_matmul keeps every block of
a row tile in one workgroup; the n = 1 GEMV bit-identical; sizes beyond the
scratch rejected before any launch."""
import numpy as np
import pytest

import oracle
from llm_amd import q8
from test_gpu_q8 import assert_bits, assert_close, assert_parity, exact_at

pytestmark = pytest.mark.gpu
SEED = 0x5EED


@pytest.fixture(scope="module")
def gpu():
    g = q8.Gpu(0)
    yield g
    g.close()


def noalloc(gpu, w, xb, n, yb, bias=None):
    h = gpu.resident(w)
    q8._check(q8.lib().q8_matmul_noalloc(gpu.handle, h, xb.ptr, 0, n, yb.ptr, 0,
                                         bias.ptr if bias is not None else 0, 0))


def run_both(gpu, w, x, n, residual=None):
    k, out = w.k, w.out
    xb = gpu.alloc(4 * n * k)
    xb.upload(x)
    ya, yb = gpu.alloc(4 * n * out), gpu.alloc(4 * n * out)
    if residual is not None:
        ya.upload(residual)
        yb.upload(residual)
    gpu.matmul(w, xb, 0, n, ya, 0, bias=ya if residual is not None else None)
    noalloc(gpu, w, xb, n, yb, bias=yb if residual is not None else None)
    want = ya.download(np.float32, n * out).reshape(n, out)
    got = yb.download(np.float32, n * out).reshape(n, out)
    for b in (xb, ya, yb):
        b.free()
    return got, want


def test_a_refused_call_does_not_take_the_scratch():
    """First in this module, before its shared context uses the array: a
    call refused for its size holds nothing, so another context's call then
    takes the array, and the refused context's next call is the one turned
    away."""
    r = np.random.default_rng(SEED + 4)
    a, b = q8.Gpu(0), q8.Gpu(0)
    try:
        nb_, kb_, ob_ = 1024, 8192, 64  # 32 x 256 x 1152 bytes > 8 MiB
        wbig = q8.Weight(oracle.make_q8_weight(r, ob_, kb_), kb_, ob_)
        xa, ya = a.alloc(4 * nb_ * kb_), a.alloc(4 * nb_ * ob_)
        print("\ncontext A: an oversized noalloc call (refused)", flush=True)
        with pytest.raises(q8.Q8Error) as e:
            noalloc(a, wbig, xa, nb_, ya)
        assert e.value.status == q8.Q8_ERR_UNSUPPORTED and "more than" in e.value.message
        n, k, out = 64, 2304, 256
        w = q8.Weight(oracle.make_q8_weight(r, out, k), k, out)
        x = oracle.make_activations(r, n, k, outlier_rate=0.01)
        xb, yb = b.alloc(4 * n * k), b.alloc(4 * n * out)
        xb.upload(x)
        print("context B: noalloc n=64 (takes the array)", flush=True)
        noalloc(b, w, xb, n, yb)
        b.sync()
        got = yb.download(np.float32, n * out).reshape(n, out)
        assert_parity(got, oracle.matmul(w.data, k, out, x, n), exact_at(w.data, k, out, x, n), "context B noalloc")
        xa2, ya2 = a.alloc(4 * n * k), a.alloc(4 * n * out)
        xa2.upload(x)
        print("context A: noalloc n=64 (refused: B holds the array)", flush=True)
        with pytest.raises(q8.Q8Error) as e:
            noalloc(a, w, xa2, n, ya2)
        assert e.value.status == q8.Q8_ERR_UNSUPPORTED and "held by another context" in e.value.message
        for buf in (xa, ya, xa2, ya2, xb, yb):
            buf.free()
        a.release(wbig)
        a.release(w)
        b.release(w)
    finally:
        b.close()
        a.close()


@pytest.mark.parametrize("first,second", [((512, 2304, 2304), (40, 2304, 576)), ((300, 5760, 2304), (33, 5760, 64)),
                                          ((1024, 2304, 1024), (2, 2304, 256))])
def test_noalloc_matches_matmul_twice_second_smaller(gpu, first, second):
    r = np.random.default_rng(SEED + first[0] + second[0])
    for i, (n, k, out) in enumerate((first, second)):
        w = q8.Weight(oracle.make_q8_weight(r, out, k), k, out)
        x = oracle.make_activations(r, n, k, outlier_rate=0.01)
        res = r.standard_normal((n, out)).astype(np.float32) if i == 1 else None
        print(f"\nnoalloc call {i}: n={n} k={k} out={out} residual={res is not None}", flush=True)
        got, want = run_both(gpu, w, x, n, res)
        what = f"noalloc call {i} n={n} k={k} out={out}"
        # the existing entry point's output is the reference, to the n >= 2 bar
        ref = oracle.matmul(w.data, k, out, x, n)
        if res is not None:
            ref = (ref + res).astype(np.float32)
        ex = exact_at(w.data, k, out, x, n)
        exact = (lambda idx, ex=ex, res=res: ex(idx)) if res is None else \
            (lambda idx, ex=ex, res=res: (res.reshape(-1)[idx].astype(np.float64) + ex(idx)[0], ex(idx)[1]))
        assert_parity(want, ref, exact, what + " (q8_matmul)")
        assert_parity(got, ref, exact, what)
        if gpu.plan(n, out, k)["kslices"] == 1:
            assert_bits(got, want, what + " vs q8_matmul")
        else:
            assert_close(got, want, what + " vs q8_matmul")
        gpu.release(w)


def test_noalloc_gemv_is_the_gemv(gpu):
    r = np.random.default_rng(SEED + 1)
    for out, k in ((5760, 2304), (64, 256)):  # a large one, then a smaller one
        w = q8.Weight(oracle.make_q8_weight(r, out, k), k, out)
        x = r.standard_normal(k).astype(np.float32)
        got, want = run_both(gpu, w, x, 1)
        assert_bits(got, want, f"noalloc gemv {out}x{k}")
        assert_close(got.reshape(-1), oracle.matmul(w.data, k, out, x, 1).reshape(-1), f"noalloc gemv {out}x{k}")
        gpu.release(w)


def test_noalloc_rejects_what_the_scratch_cannot_hold(gpu):
    n, k, out = 1024, 8192, 64  # 32 x 256 x 1152 bytes > 8 MiB
    r = np.random.default_rng(SEED + 2)
    w = q8.Weight(oracle.make_q8_weight(r, out, k), k, out)
    xb, yb = gpu.alloc(4 * n * k), gpu.alloc(4 * n * out)
    yb.upload(np.zeros(n * out, np.float32))
    with pytest.raises(q8.Q8Error) as e:
        noalloc(gpu, w, xb, n, yb)
    assert e.value.status == q8.Q8_ERR_UNSUPPORTED and "scratch" in e.value.message
    gpu.sync()
    assert not yb.download(np.float32, n * out).any()  # nothing was launched
    xb.free()
    yb.free()
    gpu.release(w)


def test_noalloc_scratch_is_held_by_one_context(gpu):
    """Two contexts on one GPU each have a stream of their own, so their calls
    could overlap on the one static array: the first context to use it holds
    it until q8_close and a second context is refused (Q8_ERR_UNSUPPORTED,
    nothing launched); calls that need no scratch (n = 1, the two-token GEMV)
    still run.  The hand-over after q8_close is tested on the CPU
    (tests/test_abi.py, q8_noalloc_owner.h)."""
    r = np.random.default_rng(SEED + 3)
    n, k, out = 64, 2304, 256
    w = q8.Weight(oracle.make_q8_weight(r, out, k), k, out)
    x = oracle.make_activations(r, n, k, outlier_rate=0.01)
    xb, yb = gpu.alloc(4 * n * k), gpu.alloc(4 * n * out)
    xb.upload(x)
    noalloc(gpu, w, xb, n, yb)  # this module's context holds the scratch (if it did not already)
    gpu.sync()
    held = yb.download(np.float32, n * out)
    other = q8.Gpu(0)
    try:
        xo, yo = other.alloc(4 * n * k), other.alloc(4 * n * out)
        xo.upload(x)
        yo.upload(np.zeros(n * out, np.float32))
        print("\nsecond context on device 0: noalloc n=64 (refused), n=1 and n=2 (no scratch)", flush=True)
        with pytest.raises(q8.Q8Error) as e:
            noalloc(other, w, xo, n, yo)
        assert e.value.status == q8.Q8_ERR_UNSUPPORTED and "held by another context" in e.value.message
        other.sync()
        assert not yo.download(np.float32, n * out).any()  # nothing was launched
        for m in (1, 2):
            noalloc(other, w, xo, m, yo)
            other.sync()
            want = oracle.matmul(w.data, k, out, x[:m], m)
            got = yo.download(np.float32, m * out).reshape(m, out)
            if m == 1:  # the GEMV on f32 x
                assert_close(got, want, "second context noalloc n=1")
            else:
                assert_parity(got, want, exact_at(w.data, k, out, x[:m], m), f"second context noalloc n={m}")
        xo.free()
        yo.free()
        other.release(w)
    finally:
        other.close()
    # the holder's scratch was not touched by the refused call
    noalloc(gpu, w, xb, n, yb)
    gpu.sync()
    assert_bits(yb.download(np.float32, n * out), held, "holder after the refusal")
    xb.free()
    yb.free()
    gpu.release(w)
