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
