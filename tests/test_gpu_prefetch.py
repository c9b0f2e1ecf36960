"""Cache riders: workgroups appended to an n >= 2 GEMM launch that only read
weights into the device caches (q8_gemm_prefetch announces the next GEMM's
weights; option gemm.riders reads the launch's own).  They change no result:
every GEMM kernel that carries them (the int8 GEMM at one, two and four token
tiles per wave, VALU scale products, split K, one token tile, the prompt group
and the fused gate/up) gives the same bits with and without them, with the
riders first or last in the grid and either load policy, and the result
without them meets the oracle.  An announcement is consumed by one launch and
dropped with its weight."""
import ctypes

import numpy as np
import pytest

import oracle
from llm_amd import q8
from test_gpu_q8 import assert_bits, assert_parity, exact_at, unpack_prepared

pytestmark = pytest.mark.gpu

SEED = 0x5EED + 0x9F

RIDER_OPTIONS = ("gemm.riders", "gemm.rider_first", "gemm.rider_nt", "gemm.next_riders", "gemm.next_rider_first",
                 "gemm.rider_wave_kib", "gemm.prefetch")


@pytest.fixture(scope="module")
def gpu():
    g = q8.Gpu(0)
    yield g
    g.close()


def rng(i):
    return np.random.default_rng(SEED + i)


def weight(r, out, k):
    return q8.Weight(oracle.make_q8_weight(r, out, k), k, out)


def reset(gpu, extra=()):
    for name in RIDER_OPTIONS + tuple(extra):
        gpu.set_option(name, -1)


# (announce another weight?, options): riders last / first, own riders first,
# own riders last with the non-temporal policy, small rider share per wave
VARIANTS = [
    ("announced, last", True, {}),
    ("announced, first", True, {"gemm.next_rider_first": 1}),
    ("announced, 8 KiB a rider wave", True, {"gemm.rider_wave_kib": 8}),
    ("announced, 40 riders", True, {"gemm.next_riders": 40}),
    ("own, first", False, {"gemm.riders": 64}),
    ("own, last, nt", False, {"gemm.riders": 64, "gemm.rider_first": 0, "gemm.rider_nt": 1}),
]

# (n, out, k, options selecting the kernel)
CASES = [
    (256, 1024, 2304, {}),                               # q8_gemm_s1_t1, K split over waves
    (8, 1024, 1024, {}),                                 # one token tile: q8_gemm_s1_t1s
    (128, 2304, 2304, {"gemm.tpw": 2}),                  # q8_gemm_s1_t2
    (96, 1024, 2304, {"gemm.tpw": 4}),                   # q8_gemm_s1_t4
    (64, 1024, 2304, {"gemm.smode": 0}),                 # q8_gemm_s0_t1
    (64, 1024, 5760, {"gemm.slices": 2}),                # split K over workgroups (arrival counters)
]


@pytest.mark.parametrize("n,out,k,opts", CASES)
def test_riders_change_no_bits(gpu, n, out, k, opts):
    r = rng(n + out + k + len(opts))
    w = weight(r, out, k)
    other = weight(r, 2304, 5760)  # 14 MB to announce
    x = oracle.make_activations(r, n, k, outlier_rate=0.01)
    xb, yb = gpu.alloc(4 * n * k), gpu.alloc(4 * n * out)
    xb.upload(x)
    try:
        reset(gpu, opts)
        for name, value in opts.items():
            gpu.set_option(name, value)
        gpu.matmul(w, xb, 0, n, yb, 0)
        base = yb.download(np.float32, n * out).reshape(n, out)
        assert_parity(base, oracle.matmul(w.data, k, out, x, n).reshape(n, out), exact_at(w.data, k, out, x=x, n=n),
                      f"riders off n={n} {out}x{k} {opts}")
        for label, announce, vopts in VARIANTS:
            print(f"\nn={n} {out}x{k} {opts}: {label}", flush=True)
            for name, value in vopts.items():
                gpu.set_option(name, value)
            if announce:
                gpu.gemm_prefetch([other])
            yb.upload(np.full(n * out, np.nan, np.float32))
            gpu.matmul(w, xb, 0, n, yb, 0)
            assert_bits(yb.download(np.float32, n * out).reshape(n, out), base, f"{label} n={n} {out}x{k} {opts}")
            for name in vopts:
                gpu.set_option(name, -1)
    finally:
        reset(gpu, opts)
        xb.free()
        yb.free()
        gpu.release(w)
        gpu.release(other)


def test_prompt_group_and_fused_gate_up_with_riders(gpu):
    """The q/k/v prompt group and the fused gate/up (q8_gemm_silu, its Q8_0
    epilogue bytes) with an announcement of three and two weights, riders
    last and first."""
    r = rng(7)
    n, k, ffn = 160, 2304, 1536
    ws = [weight(r, 1024, k) for _ in range(3)]
    gate, up = weight(r, ffn, k), weight(r, ffn, k)
    x = oracle.make_activations(r, n, k, outlier_rate=0.01)
    xb, yb, act = gpu.alloc(4 * n * k), gpu.alloc(4 * n * 3 * 1024), gpu.alloc(4 * n * ffn)
    xb.upload(x)
    try:
        reset(gpu)

        def group(announce, first):
            gpu.set_option("gemm.next_rider_first", first)
            if announce:
                gpu.gemm_prefetch([gate, up])
            p = gpu.prepare(xb, 0, n, k)
            yb.upload(np.full(n * 3 * 1024, np.nan, np.float32))
            gpu.matmul_prompt_group([(ws[i], yb, i * n * 1024) for i in range(3)], p, n, k)
            return yb.download(np.float32, n * 3 * 1024)

        def fused(announce, first):
            gpu.set_option("gemm.next_rider_first", first)
            if announce:
                gpu.gemm_prefetch(ws)
            p = gpu.gate_up_silu(gate, up, xb, 0, n, act, 0, want_prepared=True)
            return unpack_prepared(gpu, p, n, ffn)

        g0 = group(False, 0)
        for i in range(3):
            ref = oracle.matmul(ws[i].data, k, 1024, x, n).reshape(n, 1024)
            assert_parity(g0[i * n * 1024:(i + 1) * n * 1024].reshape(n, 1024), ref,
                          exact_at(ws[i].data, k, 1024, x=x, n=n), f"group member {i}")
        q0, s0 = fused(False, 0)
        for first in (0, 1):
            print(f"\nprompt group and fused gate/up, riders first={first}", flush=True)
            assert_bits(group(True, first), g0, f"prompt group, riders first={first}")
            q1, s1 = fused(True, first)
            assert np.array_equal(s1, s0) and np.array_equal(q1, q0), f"fused gate/up bytes, riders first={first}"
    finally:
        reset(gpu)
        for b in (xb, yb, act):
            b.free()
        for w in ws + [gate, up]:
            gpu.release(w)


def test_announcement_rules(gpu):
    """At most four weights, each of this context; count 0 withdraws; a
    released weight's announcement is dropped before any launch reads it."""
    r = rng(11)
    n, k = 64, 1024
    w, a, b = weight(r, 1024, k), weight(r, 2048, k), weight(r, 512, k)
    x = oracle.make_activations(r, n, k)
    xb, yb = gpu.alloc(4 * n * k), gpu.alloc(4 * n * 1024)
    xb.upload(x)
    other = q8.Gpu(0)
    try:
        reset(gpu)
        with pytest.raises(q8.Q8Error, match="at most 4"):
            gpu.gemm_prefetch([w, a, b, w, a])
        foreign = other.resident(weight(r, 256, k))
        arr = (ctypes.c_void_p * 1)(foreign)
        rc = q8.lib().q8_gemm_prefetch(gpu.handle, arr, 1)
        assert rc == q8.Q8_ERR_INVALID and "does not belong" in q8.lib().q8_last_error().decode()
        gpu.matmul(w, xb, 0, n, yb, 0)
        base = yb.download(np.float32, n * 1024)
        gpu.gemm_prefetch([a, b])
        gpu.gemm_prefetch([])  # withdrawn
        gpu.matmul(w, xb, 0, n, yb, 0)
        assert_bits(yb.download(np.float32, n * 1024), base, "after a withdrawn announcement")
        print("\nannounce, release, then launch", flush=True)
        gpu.gemm_prefetch([a, b])
        gpu.release(a)  # a leaves the announcement; b stays announced
        yb.upload(np.full(n * 1024, np.nan, np.float32))
        gpu.matmul(w, xb, 0, n, yb, 0)
        assert_bits(yb.download(np.float32, n * 1024), base, "after releasing an announced weight")
    finally:
        reset(gpu)
        other.close()
        xb.free()
        yb.free()
        gpu.release(w)
        gpu.release(b)
