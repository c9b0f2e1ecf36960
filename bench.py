"""Benchmark of the Q8_0 matmul hot path on one MI355X (BASELINE.json metric:
"Q8_0 n=1 GEMV HBM GB/s (%peak); n=512 GEMM int8 TOPS (%MFMA peak)").

A step is one n = 1 Q8_0 GEMV of configs[0] (W 5760 x 2304, x f32[2304]),
each step on the next of R weight copies whose total (> 600 MB) exceeds the
256 MB Infinity Cache, so every step streams its weights from HBM.  Steps are
captured into one HIP graph of exactly --steps launches and timed with HIP
events on the library's own stream.  `value` is that GEMV's HBM throughput:
algorithmic bytes (M*K/32*34 + 4K + 4M per step) / time per step.

Also reported (own fixed repetition counts, graphs, events):
  gemm_n512   configs[3]: the layer's projections at n = 512 (QKV 6912, O 2304,
              gate|up 2x5760, down 2304x5760) with their activation
              quantization, in int8 TOPS (2*M*N*K) vs the 5.0 POPS dense peak;
  extras      configs[1] n = 8 / 64 (GB/s), configs[2] decode layer set and
              the 122880 x 2304 lm_head GEMV + argmax (GB/s, us);
  decoder     configs[4]: the 42-layer synthetic decoder (hidden 2304, FFN
              5760, 36 heads x 64, vocab 122880, f16 KV cache of 4096) with
              random-init Q8_0 weights generated on the device: a 512-token
              prefill of random ids, then 128 greedy decode steps (tok/s);
  cpu_baseline the oracle's C restatement of the reference rayon CPU path
              (oracle/q8_oracle.c) on this host's cores, on a bounded sample.

Prints ONE JSON line.  N > 1 GPUs is not part of this build.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
MALL_BYTES = 256 << 20
METRIC = "Q8_0 n=1 GEMV HBM GB/s (%peak); n=512 GEMM int8 TOPS (%MFMA peak)"


def log(msg: str):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gemv_bytes(m: int, k: int) -> int:
    return m * k // 32 * 34 + 4 * k + 4 * m


def make_weight(rng, out, k):
    import oracle
    from llm_amd import q8
    return q8.Weight(oracle.make_q8_weight(rng, out, k), k, out)


def timed_graph(gpu, record, reps: int, warmup: int) -> float:
    """Capture `record()` once into a graph, replay `warmup` times untimed,
    then `reps` times between HIP events; returns ms per replay."""
    record()  # eager run: grows workspaces outside the capture
    gpu.sync()
    gpu.graph_begin()
    record()
    graph = gpu.graph_end()
    try:
        for _ in range(warmup):
            gpu.graph_launch(graph)
        gpu.sync()
        e0, e1 = gpu.event(), gpu.event()
        gpu.record(e0)
        for _ in range(reps):
            gpu.graph_launch(graph)
        gpu.record(e1)
        ms = gpu.elapsed_ms(e0, e1)
        gpu.sync()
        gpu.destroy_event(e0)
        gpu.destroy_event(e1)
    finally:
        gpu.graph_destroy(graph)
    return ms / reps


def bench_gemv_rotating(gpu, m, k, steps, warmup, rng, label):
    """n = 1 GEMV over rotating weight copies (MALL-cold)."""
    base = make_weight(rng, m, k)
    per = gemv_bytes(m, k)
    copies = max(2, math.ceil(600e6 / per))
    from llm_amd import q8
    weights = [base] + [q8.Weight(base.data.copy(), k, m) for _ in range(copies - 1)]
    for w in weights:
        gpu.resident(w)
    x = rng.standard_normal(k, dtype=np.float32)
    xb, yb = gpu.alloc(4 * k), gpu.alloc(4 * m)
    xb.upload(x)

    def record_n(count):
        def rec():
            for i in range(count):
                gpu.matmul(weights[i % copies], xb, 0, 1, yb, 0)
        return rec

    # warmup graph, then one graph of exactly `steps` launches
    if warmup:
        timed_graph(gpu, record_n(min(warmup, 4 * copies)), 1, 0)
    ms_total = timed_graph(gpu, record_n(steps), 1, 1)
    ms = ms_total / steps
    gbs = per / (ms * 1e-3) / 1e9
    log(f"{label}: {ms * 1e3:.2f} us/step, {gbs:.0f} GB/s over {copies} copies ({copies * per / 1e6:.0f} MB)")
    for w in weights:
        gpu.release(w)
    xb.free()
    yb.free()
    return {"us_per_step": ms * 1e3, "gbs": gbs, "bytes_per_step": per, "copies": copies,
            "total_ms": ms_total}


def bench_gemv_hot(gpu, m, k, rng, steps=2000):
    """The same GEMV on one weight copy (14 MB, resident in the 256 MB
    Infinity Cache after the first launch): the MALL-hot figure."""
    w = make_weight(rng, m, k)
    gpu.resident(w)
    xb, yb = gpu.alloc(4 * k), gpu.alloc(4 * m)
    xb.upload(rng.standard_normal(k, dtype=np.float32))

    def rec():
        for _ in range(steps):
            gpu.matmul(w, xb, 0, 1, yb, 0)
    ms = timed_graph(gpu, rec, 1, 1) / steps
    gbs = gemv_bytes(m, k) / (ms * 1e-3) / 1e9
    log(f"configs[0] GEMV MALL-hot: {ms * 1e3:.2f} us/step, {gbs:.0f} GB/s")
    gpu.release(w)
    xb.free()
    yb.free()
    return round(gbs, 1)


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "q8_gemv_configs0_traffic.md")


def traffic_from_profile():
    """HBM bytes per configs[0] GEMV launch from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary, if it was measured on the code object
    loaded now (its sha256 is recorded in the summary); otherwise None."""
    from llm_amd import q8
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None
    fields = {}
    for line in text.splitlines():
        if line.startswith("- ") and ": " in line:
            key, val = line[2:].split(": ", 1)
            fields[key.strip("` ")] = val.strip("` ")
    if fields.get("code_object_sha256") != json.loads(q8.build_info())["code_object_sha256"]:
        return None
    try:
        return int(fields["traffic_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def bench_gemm_rotating(gpu, m, k, n, reps, rng, label):
    """n tokens over rotating weight copies, quantization included."""
    import oracle
    from llm_amd import q8
    base = make_weight(rng, m, k)
    per = m * k // 32 * 34 + n * k * 4 + 4 * n * m
    copies = max(2, math.ceil(600e6 / (m * k // 32 * 34)))
    weights = [base] + [q8.Weight(base.data.copy(), k, m) for _ in range(copies - 1)]
    for w in weights:
        gpu.resident(w)
    x = oracle.make_activations(rng, n, k, outlier_rate=0.01)
    xb, yb = gpu.alloc(4 * n * k), gpu.alloc(4 * n * m)
    xb.upload(x)

    def rec():
        for w in weights:
            gpu.matmul(w, xb, 0, n, yb, 0)

    ms = timed_graph(gpu, rec, reps, 2) / copies
    gbs = per / (ms * 1e-3) / 1e9
    tops = 2 * m * n * k / (ms * 1e-3) / 1e12
    log(f"{label}: {ms * 1e3:.2f} us/matmul, {gbs:.0f} GB/s, {tops:.1f} TOPS")
    for w in weights:
        gpu.release(w)
    xb.free()
    yb.free()
    return {"us": ms * 1e3, "gbs": gbs, "tops": tops, "bytes": per}


def own_prepared(gpu, prep, n, k):
    """Copy a prepared operand (quants in either format, then f32 scales) into
    a buffer we own; returns (Prepared, buffer)."""
    from llm_amd import q8
    qbytes, sbytes = prep.quant_bytes(), prep.scale_bytes()
    buf = gpu.alloc(qbytes + sbytes)
    q8._check(q8.lib().q8_copy_device(gpu.handle, buf.ptr, prep.quants, qbytes))
    q8._check(q8.lib().q8_copy_device(gpu.handle, buf.ptr + qbytes, prep.scales, sbytes))
    return q8.Prepared(buf.ptr, buf.ptr + qbytes, n, k, prep.format), buf


def bench_layer_n512(gpu, reps, rng, n=512):
    """the four projections at n tokens on the int8 MFMA path."""
    import oracle
    from llm_amd import q8
    hid, ffn = 2304, 5760
    wq, wk, wv = (make_weight(rng, hid, hid) for _ in range(3))
    wo = make_weight(rng, hid, hid)
    wg, wu = make_weight(rng, ffn, hid), make_weight(rng, ffn, hid)
    wd = make_weight(rng, hid, ffn)
    for w in (wq, wk, wv, wo, wg, wu, wd):
        gpu.resident(w)
    x = oracle.make_activations(rng, n, hid)
    xb = gpu.alloc(4 * n * hid)
    xb.upload(x)
    qkv = gpu.alloc(4 * n * 3 * hid)
    hb = gpu.alloc(4 * n * hid)
    hb.upload(x)
    act = gpu.alloc(4 * n * ffn)
    ops = {
        "qkv": 2 * n * 3 * hid * hid,
        "o": 2 * n * hid * hid,
        "gate_up": 2 * n * 2 * ffn * hid,
        "down": 2 * n * hid * ffn,
    }

    def rec():
        p = gpu.prepare(xb, 0, n, hid)
        gpu.matmul_prompt_group([(wq, qkv, 0), (wk, qkv, n * hid), (wv, qkv, 2 * n * hid)], p, n, hid)
        gpu.matmul(wo, qkv, 0, n, hb, 0, bias=hb)           # O with its residual
        pd = gpu.gate_up_silu(wg, wu, hb, 0, n, act, 0, want_prepared=True)
        gpu.matmul(wd, act, 0, n, hb, 0, prepared=pd, bias=hb)  # down with its residual

    ms = timed_graph(gpu, rec, reps, 3)
    total_ops = sum(ops.values())
    tops = total_ops / (ms * 1e-3) / 1e12
    log(f"n={n} layer set: {ms * 1e3:.1f} us, {tops:.1f} TOPS ({tops / INT8_PEAK_TOPS * 100:.1f}% of int8 peak)")

    # the same work piece by piece (each its own graph): quantization alone and
    # each projection on already-prepared activations
    gu = gpu.alloc(4 * n * 2 * ffn)
    norm_w = (1.0 + 0.1 * rng.standard_normal(hid)).astype(np.float32)  # the fused rmsnorm -> Q8_0 prologue
    # A Prepared points into the library's one activation workspace (valid
    # until the next prepare, as the reference's); keep copies in buffers of
    # our own so both operands stay valid side by side.
    p, pbuf = own_prepared(gpu, gpu.prepare(xb, 0, n, hid), n, hid)
    pf, pfbuf = own_prepared(gpu, gpu.prepare(act, 0, n, ffn), n, ffn)
    pieces = {
        "quantize_x": lambda: gpu.prepare(xb, 0, n, hid),
        "quantize_act": lambda: gpu.prepare(act, 0, n, ffn),
        "norm_prepare_x": lambda: gpu.norm_prepare(xb, 0, norm_w, 1e-6, n),
        "qkv": lambda: gpu.matmul_prompt_group([(wq, qkv, 0), (wk, qkv, n * hid), (wv, qkv, 2 * n * hid)],
                                               p, n, hid),
        "o": lambda: gpu.matmul(wo, qkv, 0, n, hb, 0, prepared=p),
        "gate_up": lambda: gpu.matmul_prompt_group([(wg, gu, 0), (wu, gu, n * ffn)], p, n, hid),
        "gate_up_silu": lambda: gpu.gate_up_silu(wg, wu, hb, 0, n, act, 0, want_prepared=True),
        "down": lambda: gpu.matmul(wd, act, 0, n, hb, 0, prepared=pf),
    }
    piece_us = {}
    per_graph = 10  # one graph launch costs more than a kernel: record each piece 10 times per graph

    def repeat(fn):
        return lambda: [fn() for _ in range(per_graph)]
    for name, fn in pieces.items():
        piece_us[name] = round(timed_graph(gpu, repeat(fn), reps, 3) / per_graph * 1e3, 2)
    log("n=512 pieces (us): " + ", ".join(f"{k} {v}" for k, v in piece_us.items()))
    for w in (wq, wk, wv, wo, wg, wu, wd):
        gpu.release(w)
    for b in (xb, qkv, hb, act, gu, pbuf, pfbuf):
        b.free()
    return {"us": ms * 1e3, "tops": tops, "ops": total_ops, "frac": tops / INT8_PEAK_TOPS,
            "ops_by_projection": ops, "quantize_us": piece_us["quantize_x"], "projections_us": piece_us}


def bench_decode_layer(gpu, reps, rng):
    """decode n = 1 layer set and the lm_head GEMV + argmax."""
    hid, ffn, vocab = 2304, 5760, 122880
    wq, wk, wv, wo = (make_weight(rng, hid, hid) for _ in range(4))
    wg, wu = make_weight(rng, ffn, hid), make_weight(rng, ffn, hid)
    wd = make_weight(rng, hid, ffn)
    for w in (wq, wk, wv, wo, wg, wu, wd):
        gpu.resident(w)
    x = rng.standard_normal(hid, dtype=np.float32)
    xb, qkv, hb, act = gpu.alloc(4 * hid), gpu.alloc(4 * 3 * hid), gpu.alloc(4 * hid), gpu.alloc(4 * ffn)
    xb.upload(x)
    hb.upload(x)

    def rec():
        gpu.matmul_decode_group([(wq, qkv, 0), (wk, qkv, hid), (wv, qkv, 2 * hid)], xb, 0, hid)
        gpu.matmul(wo, qkv, 0, 1, hb, 0, bias=hb)
        gpu.gate_up_silu(wg, wu, hb, 0, 1, act, 0)
        gpu.matmul(wd, act, 0, 1, hb, 0, bias=hb)

    ms = timed_graph(gpu, rec, reps, 3)
    wbytes = (4 * hid * hid + 2 * ffn * hid + hid * ffn) // 32 * 34
    layer = {"us": ms * 1e3, "weight_bytes": wbytes, "gbs": wbytes / (ms * 1e-3) / 1e9}
    log(f"decode layer set: {ms * 1e3:.1f} us, {layer['gbs']:.0f} GB/s (weights, L2/MALL-warm)")
    for w in (wq, wk, wv, wo, wg, wu, wd):
        gpu.release(w)

    wl = make_weight(rng, vocab, hid)
    gpu.resident(wl)
    logits = gpu.alloc(4 * vocab)

    def rec_head():
        gpu.matmul(wl, xb, 0, 1, logits, 0)

    ms_h = timed_graph(gpu, rec_head, reps, 3)
    per = gemv_bytes(vocab, hid)
    t0 = time.perf_counter()
    best = gpu.lm_head_argmax(wl, xb, 0, logits, 0)
    head = {"us": ms_h * 1e3, "gbs": per / (ms_h * 1e-3) / 1e9, "bytes": per, "argmax": best,
            "argmax_call_us_host": (time.perf_counter() - t0) * 1e6}
    log(f"lm_head 122880x2304: {ms_h * 1e3:.1f} us, {head['gbs']:.0f} GB/s")
    gpu.release(wl)
    for b in (xb, qkv, hb, act, logits):
        b.free()
    return layer, head


def bench_decoder(gpu, rng, prompt=512, steps=128, reps=3):
    """prefill `prompt` random ids, then `steps` greedy decode
    steps, on the 42-layer synthetic decoder.  Each phase runs once untimed
    (the eager pass, then the capture of its graph) before the timed runs;
    times are host wall-clock around the calls (which end in a wait), the
    median of `reps`."""
    from llm_amd import decoder as dm
    cfg = dm.config(n_layer=42, n_embd=2304, n_ff=5760, n_head=36, n_head_kv=36, head_dim=64, n_vocab=122880,
                    capacity=4096, max_batch=prompt)
    t0 = time.perf_counter()
    dec = dm.Decoder(gpu, cfg, seed=0x5EED)
    log(f"decoder: 42 layers generated on the device in {time.perf_counter() - t0:.1f} s")
    ids = rng.integers(0, cfg.n_vocab, prompt).astype(np.uint32)
    try:
        for _ in range(2):  # eager pass, then capture
            dec.reset()
            dec.forward(ids)
            dec.generate(steps)
        pre, gen = [], []
        tokens = None
        for _ in range(reps):
            dec.reset()
            t0 = time.perf_counter()
            first = dec.forward(ids)
            pre.append(time.perf_counter() - t0)
            t0 = time.perf_counter()
            toks = dec.generate(steps)
            gen.append(time.perf_counter() - t0)
            cur = [first] + toks.tolist()
            assert tokens is None or tokens == cur, "greedy tokens differ between identical runs"
            tokens = cur
    finally:
        dec.close()
    t_pre, t_gen = float(np.median(pre)), float(np.median(gen))
    layer_w = (2304 * 3 * 2304 + 2304 * 2304 + 2 * 5760 * 2304 + 2304 * 5760) // 32 * 34
    head_w = 122880 * 2304 // 32 * 34
    per_token = 42 * layer_w + head_w
    out = {"prefill_tokens": prompt, "prefill_ms": round(t_pre * 1e3, 2),
           "prefill_tok_s": round(prompt / t_pre, 1),
           "decode_steps": steps, "decode_ms_per_token": round(t_gen / steps * 1e3, 3),
           "decode_tok_s": round(steps / t_gen, 1),
           "decode_weight_bytes_per_token": per_token,
           "decode_weight_gbs": round(per_token * steps / t_gen / 1e9, 1),
           "decode_floor_ms_per_token_at_8tbs": round(per_token / 8e12 * 1e3, 3),
           "first_tokens": tokens[:8]}
    log(f"decoder: prefill {prompt} in {t_pre * 1e3:.1f} ms ({out['prefill_tok_s']} tok/s); decode "
        f"{out['decode_ms_per_token']} ms/token ({out['decode_tok_s']} tok/s, {out['decode_weight_gbs']} GB/s of "
        f"weights)")
    return out


CALIBRATION_BYTES = 64 << 20


def calibration_copy(gpu, reps=3):
    """A plain q8_copy of CALIBRATION_BYTES, the known-size kernel the
    rocprofv3 FETCH_SIZE / WRITE_SIZE counters are scaled against."""
    src, dst = gpu.alloc(CALIBRATION_BYTES), gpu.alloc(CALIBRATION_BYTES)
    for _ in range(reps):
        gpu.copy(dst, src, CALIBRATION_BYTES)
    gpu.sync()
    src.free()
    dst.free()


def cpu_baseline(seconds: float = 10.0):
    """The oracle (C restatement of tensor::matmul, rayon-style row split) on
    this host's cores: configs[0] GEMV for ~`seconds` of wall time."""
    import oracle
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    threads = max(1, min(cores, 16))
    rng = np.random.default_rng(0x5EED)
    m, k = 5760, 2304
    data = oracle.make_q8_weight(rng, m, k)
    x = rng.standard_normal(k, dtype=np.float32)
    oracle.matmul(data, k, m, x, 1, threads=threads)
    reps = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        oracle.matmul(data, k, m, x, 1, threads=threads)
        reps += 1
    dt = time.perf_counter() - t0
    gbs = gemv_bytes(m, k) * reps / dt / 1e9
    log(f"cpu baseline: {gbs:.1f} GB/s with {threads} threads ({oracle.simd_path()}), {reps} GEMVs")
    return {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{reps} configs[0] GEMVs (5760x2304, n=1, f32 x) in {dt:.1f} s, "
                      f"{oracle.simd_path()} order, threads={threads}, cache-warm 14 MB matrix"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--sections", default="all",
                    help="comma list of gemv,gemm,extras,decoder,cpu (default all); a profiler run names "
                         "one so each kernel's average covers one workload")
    args = ap.parse_args()
    known = {"gemv", "gemm", "extras", "decoder", "cpu"}
    sections = set(known) if args.sections == "all" else set(args.sections.split(","))
    unknown = sections - known
    if unknown:
        ap.error(f"unknown sections {sorted(unknown)}")
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus "
              f"{args.gpus}); the sharding design is described in DESIGN.md", file=sys.stderr)
        sys.exit(2)

    from llm_amd import q8
    rng = np.random.default_rng(0x5EED)
    gpu = q8.Gpu(0)
    log(f"device {gpu.name}")
    calibration_copy(gpu)
    m, k = 5760, 2304
    gemv = {"gbs": None, "us_per_step": None, "bytes_per_step": gemv_bytes(m, k), "copies": None}
    if "gemv" in sections:
        gemv = bench_gemv_rotating(gpu, m, k, args.steps, args.warmup, rng, "configs[0] GEMV")
    gemm = {"tops": None, "frac": None, "us": None, "ops": None}
    if "gemm" in sections:
        gemm = bench_layer_n512(gpu, 20, rng)
    extras = {}
    if "extras" in sections:
        gemv["mall_hot"] = bench_gemv_hot(gpu, m, k, rng)
        extras["configs1_n8"] = bench_gemm_rotating(gpu, m, k, 8, 5, rng, "configs[1] n=8")
        extras["configs1_n64"] = bench_gemm_rotating(gpu, m, k, 64, 5, rng, "configs[1] n=64")
        layer, head = bench_decode_layer(gpu, 50, rng)
        extras["configs2_decode_layer"] = layer
        extras["configs2_lm_head"] = head
    decoder = bench_decoder(gpu, rng) if "decoder" in sections else None
    cpu = cpu_baseline(args.cpu_seconds) if "cpu" in sections and args.cpu_seconds > 0 else None
    # the kernel the tactic table runs for configs[0] (the one `value` times)
    t = gpu.plan(1, m, k)
    gemv_kernel = (f"q8_gemv_r{t['row_slice']}_l{t['slice_loads']}" if t["row_slice"] in (8, 16)
                   else f"q8_gemv1_pb{t['pairs_per_batch']}_e{t['exact']}")
    gpu.close()

    value = gemv["gbs"]
    line = {
        "metric": METRIC,
        "value": round(value, 1) if value is not None else None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": gemv["us_per_step"] / 1e3 if gemv["us_per_step"] is not None else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 weights x f32 activations (n=1); int8 x int8 -> int32, f32 scales (n>=2)",
        "data": "synthetic: seeded random Q8_0 weights (q ~ U[-127,127], d = f16(|N(0,0.02)|/127)), x ~ N(0,1)",
        "config": {"workload": "configs[0] Q8_0 GEMV n=1, W 5760x2304, MALL-cold (rotating copies); "
                               "plus configs[3] n=512 layer projections",
                   "M": m, "K": k, "n": 1, "rotating_copies": gemv["copies"]},
        "roofline": {"bound": "hbm", "achieved": round(value, 1) if value is not None else None,
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4) if value is not None else None,
                     "traffic": traffic_from_profile(),
                     "kernel": gemv_kernel, "bytes_per_launch": gemv["bytes_per_step"],
                     "mall_hot_gbs": gemv.get("mall_hot")},
        "gemm_n512": {"value": round(gemm["tops"], 2) if gemm["tops"] is not None else None, "unit": "TOPS",
                      "peak": INT8_PEAK_TOPS,
                      "frac": round(gemm["frac"], 4) if gemm["frac"] is not None else None,
                      "us_per_layer": round(gemm["us"], 2) if gemm["us"] is not None else None,
                      "ops_per_layer": gemm["ops"],
                      "quantize_us": gemm.get("quantize_us"),
                      "projections_us": gemm.get("projections_us")},
        "extras": extras,
        "decoder_configs4": decoder,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
