"""Concurrent use of the C-ABI from several host threads (the reference's Gpu
is Send + Sync, apps/engine/src/cuda/mod.rs:1975-1979, and re-binds its
context on every entry point).  ctypes releases the GIL for the length of
each library call, so the calls below overlap inside the library.

  * threads sharing one context: its mutex orders their calls, and every
    result equals the single-threaded one bit for bit;
  * threads with a context each (a stream each): independent, and again every
    result equals the single-threaded one bit for bit.
"""
import threading

import numpy as np
import pytest

import oracle
from llm_amd import q8

pytestmark = pytest.mark.gpu

SEED = 0x5EED + 0x7E
K, OUT = 2304, 2304


def inputs():
    r = np.random.default_rng(SEED)
    w = q8.Weight(oracle.make_q8_weight(r, OUT, K), K, OUT)
    xs = {n: oracle.make_activations(r, n, K, outlier_rate=0.01) for n in (1, 64)}
    return w, xs


def run_once(gpu, w, x, n):
    xb, yb = gpu.alloc(4 * n * K), gpu.alloc(4 * n * OUT)
    try:
        xb.upload(x)
        gpu.matmul(w, xb, 0, n, yb, 0)
        gpu.sync()
        return yb.download(np.float32, n * OUT)
    finally:
        xb.free()
        yb.free()


def hammer(make_gpu, w, xs, want, threads=4, iters=8):
    errors = []

    def work(tid):
        try:
            gpu = make_gpu(tid)
            for i in range(iters):
                n = 1 if (tid + i) % 2 else 64
                got = run_once(gpu, w, xs[n], n)
                if not np.array_equal(got.view(np.uint32), want[n].view(np.uint32)):
                    errors.append(f"thread {tid} iteration {i} n={n}: result differs")
        except Exception as e:  # reported below, in the main thread
            errors.append(f"thread {tid}: {type(e).__name__}: {e}")

    ts = [threading.Thread(target=work, args=(t,)) for t in range(threads)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in ts), "a worker thread did not finish"
    assert not errors, errors


def test_threads_sharing_one_context():
    w, xs = inputs()
    gpu = q8.Gpu(0)
    try:
        want = {n: run_once(gpu, w, xs[n], n) for n in (1, 64)}
        assert np.isfinite(want[64]).all()
        print("\n4 threads x 8 calls on one context", flush=True)
        hammer(lambda tid: gpu, w, xs, want)
    finally:
        gpu.close()


def test_threads_with_a_context_each():
    w, xs = inputs()
    ref = q8.Gpu(0)
    try:
        want = {n: run_once(ref, w, xs[n], n) for n in (1, 64)}
    finally:
        ref.close()
    gpus = {}
    lock = threading.Lock()

    def make(tid):
        g = q8.Gpu(0)
        with lock:
            gpus[tid] = g
        return g

    print("\n4 threads x 8 calls, a context each", flush=True)
    try:
        hammer(make, w, xs, want)
    finally:
        for g in gpus.values():
            g.close()
