"""Benchmark of the Q8_0 matmul hot path on one MI355X (the benchmark's metric:
"Q8_0 n=1 GEMV HBM GB/s (%peak); n=512 GEMM int8 TOPS (%MFMA peak)").

A step is one n = 1 Q8_0 GEMV of configs[0] (W 5760 x 2304, x f32[2304]).
Every step reads the next of R weight copies (R x 14.1 MB > 600 MB, more
than twice the 256 MB Infinity Cache), in one rotation that runs on across
the warmup and every trial, so whatever --steps is, a copy is read again only
after all the others: every step streams its weights from HBM.

Protocol (the same for every rotating figure below):
  * an eager pass over all copies, then one graph of --warmup steps;
  * T >= 5 trials; each captures into one graph an untimed "filler" (the
    next max(steps, R) launches of the rotation), then exactly --steps
    launches between two event nodes, and times those steps with the events
    (HIP events on the library's stream, recorded inside the graph): the
    timed kernels run back to back in the middle of one graph, so neither
    host submission nor a graph boundary shows in the timed region;
  * the figure is the median over the trials (all trials are reported).
`value` is the GEMV's HBM throughput: algorithmic bytes (M*K/32*34 + 4K + 4M
per step) / median time per step.

Also reported, each on its own rotation:
  configs0_quantized_x  the same GEMV with x quantized to Q8_0 per 32-block
                first, as configs[0]'s wording reads (q8_matmul_q8: the
                n >= 2 arithmetic of tensor::matmul at n = 1, quantization
                and int8 block dots in one launch);
  configs0_sustained  the same rotation replayed back to back for
                --sustained-seconds (default 6): GB/s over every replay and
                the slowest replay against the fastest, i.e. whether the
                figure holds under continuous load;
  ceilings      what one kernel of this size can do on this box: the best
                plain streaming read of the configs[0] byte count (the
                GEMV's achievable ceiling), an empty kernel's cost per graph
                launch, the sustained int8 MFMA rate (v_mfma_i32_32x32x32_i8
                only), VALU rate, and the GEMM's per-tile-block instruction
                mix with operands in registers (its own ceiling), for the
                int8 and the f16-MFMA families;
  reads         the same plain-read ceiling at the byte counts of the decode
                step's launches (reported under ceilings);
  gemm_n512     configs[3]: the layer's projections at n = 512 (QKV 6912,
                O 2304 + residual, gate|up 2x5760 -> SiLU -> Q8_0, down
                2304x5760 + residual) with the activation quantization, on
                rotating copies of the layer (MALL-cold), int8 TOPS
                (2*M*N*K) vs the 5.0 POPS dense peak, each GEMM announcing
                the next one's weights (q8_gemm_prefetch) as the decoder's
                prefill does; the same layer without announcements, and
                each piece alone, beside it;
  extras        configs[1] n = 8 / 64, configs[2] decode layer set (rotating
                layer copies) and the 122880 x 2304 lm_head GEMV + argmax;
  decoder       configs[4]: the 42-layer synthetic decoder (hidden 2304, FFN
                5760, 36 heads x 64, vocab 122880, f16 KV cache of 4096),
                random-init Q8_0 weights generated on the device, reported as
                llama-bench does (apps/cli/src/bench.rs:83-229): pp512 and
                tg128 tok/s, mean +- sample std over r = 5 repeats, with the
                build's code object hash and the tactics its shapes run;
  chain         (named only, not in the default set) the decoder's decode
                step as its op chain launched eagerly, no graphs: 42 layers
                of norm + q/k/v + RoPE, attention + O, norm + gate/up + SiLU,
                down, then the head, 20 steps at 600 visible positions, for a
                kernel trace of the launches the captured step replays;
  cpu_baseline  the oracle's C restatement of the reference rayon CPU path
                (oracle/q8_oracle.c, AVX2 order) on this host's cores: the
                configs[0] GEMV in GB/s and the configs[3] layer set in TOPS,
                each on a bounded sample.

Prints ONE JSON line.  N > 1 GPUs is not part of this build.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
MALL_BYTES = 256 << 20
ROTATE_BYTES = 600e6
TRIALS = 5
METRIC = "Q8_0 n=1 GEMV HBM GB/s (%peak); n=512 GEMM int8 TOPS (%MFMA peak)"
HID, FFN, VOCAB = 2304, 5760, 122880


def log(msg: str):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gemv_bytes(m: int, k: int) -> int:
    return m * k // 32 * 34 + 4 * k + 4 * m


def make_weight(rng, out, k):
    import oracle
    from llm_amd import q8
    return q8.Weight(oracle.make_q8_weight(rng, out, k), k, out)


def copies_for(nbytes: float) -> int:
    return max(2, math.ceil(ROTATE_BYTES / nbytes))


def rotating_trials(gpu, launch, copies: int, steps: int, warmup: int, trials: int = TRIALS) -> list[float]:
    """The protocol of the module docstring: `launch(i)` enqueues step i on
    copy i (mod copies).  Returns ms per step of each trial."""
    pos = 0

    def record(count):
        nonlocal pos
        for _ in range(count):
            launch(pos % copies)
            pos += 1

    for i in range(copies):  # eager: workspaces grown, every copy touched once
        launch(i)
    gpu.sync()
    if warmup:
        gpu.graph_begin()
        record(warmup)
        g = gpu.graph_end()
        gpu.graph_launch(g)
        gpu.sync()
        gpu.graph_destroy(g)
    filler = max(steps, copies)
    out = []
    e0, e1 = gpu.event(), gpu.event()
    for _ in range(trials):
        # one graph: the filler launches, then the timed steps between two
        # event nodes, so no graph boundary or host submission is timed
        gpu.graph_begin()
        record(filler)
        gpu.record(e0)
        record(steps)
        gpu.record(e1)
        g = gpu.graph_end()
        gpu.graph_launch(g)
        ms = gpu.elapsed_ms(e0, e1)
        gpu.sync()
        gpu.graph_destroy(g)
        out.append(ms / steps)
    gpu.destroy_event(e0)
    gpu.destroy_event(e1)
    return out


def summary(ms_list, work, unit_scale):
    """Median over trials and the per-trial figures (work / ms * unit_scale)."""
    med = statistics.median(ms_list)
    return {"median_us": round(med * 1e3, 3), "value": work / (med * 1e-3) * unit_scale,
            "trials": [round(work / (m * 1e-3) * unit_scale, 1) for m in ms_list]}


# ---------------------------------------------------------------------------
# configs[0] GEMV (the headline) and its ceiling
# ---------------------------------------------------------------------------

def sustained_gemv(gpu, launch, copies, per, seconds, steps=2000):
    """The same rotation replayed back to back for about `seconds`: one graph
    of `steps` launches between two event nodes, replayed until the host
    clock passes `seconds`; GB/s over every replay's event time, and the
    slowest replay against the fastest (a throttling GPU would show it)."""
    if seconds <= 0:
        return None
    pos = 0
    e0, e1 = gpu.event(), gpu.event()
    gpu.graph_begin()
    gpu.record(e0)
    for _ in range(steps):
        launch(pos % copies)
        pos += 1
    gpu.record(e1)
    g = gpu.graph_end()
    per_replay = []
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        gpu.graph_launch(g)
        per_replay.append(gpu.elapsed_ms(e0, e1))  # waits for the replay
    wall = time.perf_counter() - t0
    gpu.graph_destroy(g)
    gpu.destroy_event(e0)
    gpu.destroy_event(e1)
    total_ms = sum(per_replay)
    out = {"seconds": round(wall, 2), "replays": len(per_replay), "steps": steps * len(per_replay),
           "gbs": round(per * steps * len(per_replay) / (total_ms * 1e-3) / 1e9, 1),
           "us_per_step": round(total_ms * 1e3 / (steps * len(per_replay)), 3),
           "slowest_over_fastest": round(max(per_replay) / min(per_replay), 3)}
    log(f"configs[0] GEMV sustained: {out['gbs']:.0f} GB/s over {out['steps']} steps in {out['seconds']} s "
        f"(slowest / fastest replay {out['slowest_over_fastest']})")
    return out


def bench_gemv(gpu, m, k, steps, warmup, rng, sustained_s=6.0):
    from llm_amd import q8
    base = make_weight(rng, m, k)
    per = gemv_bytes(m, k)
    copies = copies_for(per)
    weights = [base] + [q8.Weight(base.data.copy(), k, m) for _ in range(copies - 1)]
    for w in weights:
        gpu.resident(w)
    xb, yb = gpu.alloc(4 * k), gpu.alloc(4 * m)
    xb.upload(rng.standard_normal(k, dtype=np.float32))
    ms = rotating_trials(gpu, lambda i: gpu.matmul(weights[i], xb, 0, 1, yb, 0), copies, steps, warmup)
    s = summary(ms, per, 1e-9)
    log(f"configs[0] GEMV: {s['median_us']:.2f} us/step, {s['value']:.0f} GB/s (median of {len(ms)} trials of "
        f"{steps} steps; trials {s['trials']}) over {copies} copies ({copies * per / 1e6:.0f} MB)")
    # MALL-hot: one copy, re-read every step
    hot = rotating_trials(gpu, lambda i: gpu.matmul(base, xb, 0, 1, yb, 0), 1, max(steps, 50), warmup)
    hs = summary(hot, per, 1e-9)
    log(f"configs[0] GEMV MALL-hot: {hs['median_us']:.2f} us/step, {hs['value']:.0f} GB/s")
    sustained = sustained_gemv(gpu, lambda i: gpu.matmul(weights[i], xb, 0, 1, yb, 0), copies, per, sustained_s)
    # x quantized to Q8_0 first, as the n >= 2 path does (q8_matmul_q8: one
    # launch quantizes x and takes the int8 block dots), same rotation
    q8x = rotating_trials(gpu, lambda i: gpu.matmul_q8(weights[i], xb, 0, 1, yb, 0), copies, steps, warmup)
    qs = summary(q8x, per, 1e-9)
    log(f"configs[0] GEMV on Q8_0-quantized x: {qs['median_us']:.2f} us/step, {qs['value']:.0f} GB/s "
        f"(trials {qs['trials']})")
    for w in weights:
        gpu.release(w)
    xb.free()
    yb.free()
    return {"us_per_step": s["median_us"], "gbs": s["value"], "trials_gbs": s["trials"], "bytes_per_step": per,
            "copies": copies, "mall_hot_gbs": round(hs["value"], 1), "mall_hot_us": hs["median_us"],
            "q8x_gbs": round(qs["value"], 1), "q8x_us": qs["median_us"], "q8x_trials_gbs": qs["trials"],
            "sustained": sustained}


# the read probe's shapes: 16-byte loads per lane, cache policy, threads per
# workgroup (576 = nine waves, the configs[0] GEMV's row-slice workgroups,
# whose weight loads are non-temporal)
READ_SHAPES = [(loads, nt, threads) for threads in (256, 576, 1024) for nt in (False, True) for loads in (2, 4, 8, 16)]


def best_read(gpu, pr, nbytes, copies, steps, warmup):
    """The fastest plain read of nbytes over `copies` rotating copies, over
    READ_SHAPES: (us, shape name, {shape: us})."""
    nb = (nbytes + 15) // 16 * 16
    stride = (nb + 4095) // 4096 * 4096
    buf = gpu.alloc(stride * copies)
    table = {}
    for loads, nt, threads in READ_SHAPES:
        name = f"l{loads}{'_nt' if nt else ''}_t{threads}"
        ms = rotating_trials(gpu, lambda i, l=loads, n=nt, t=threads: pr.read(buf, nb, l, n, t, src_offset=i * stride),
                             copies, steps, warmup)
        table[name] = statistics.median(ms) * 1e3
    buf.free()
    best = min(table, key=table.get)
    return table[best], best, table


def bench_ceilings(gpu, steps, warmup, read_bytes):
    """The plain-read ceiling at the GEMV's byte count (best of the read
    shapes, the GEMV's own non-temporal nine-wave shape among them), an empty
    kernel, the MFMA / VALU / tile-block-mix rates, and the co-resident split
    probes: an int8-MFMA role and a VALU role on the same SIMDs, timed alone
    and together (together = the larger of the two if their pipes overlap,
    the sum if they share one)."""
    from llm_amd import probes
    pr = probes.Probes(gpu)
    copies = copies_for(read_bytes)
    best_us, best_name, table = best_read(gpu, pr, read_bytes, copies, steps, warmup)
    log(f"plain read of {read_bytes} B, MALL-cold: best {best_name} {best_us:.2f} us "
        f"({read_bytes / (best_us * 1e-6) / 1e9:.0f} GB/s); " +
        ", ".join(f"{n} {u:.2f}" for n, u in sorted(table.items(), key=lambda kv: kv[1])[:6]))
    empty = rotating_trials(gpu, lambda i: pr.probe(probes.EMPTY), 1, 200, 20)
    empty_us = statistics.median(empty) * 1e3
    cus = gpu.info()["cu_count"]
    wgs = 4 * cus  # four 4-wave workgroups a CU: four waves a SIMD
    rates = {}
    for which, name, per_iter in ((probes.MFMA, "mfma", 4), (probes.VALU, "valu", 1), (probes.MIX, "mix", 2),
                                  (probes.MIX_F16, "mix_f16", 2)):
        iters = 2048 if which != probes.VALU else 8192
        ms = rotating_trials(gpu, lambda i, w=which, it=iters: pr.probe(w, iters=it, workgroups=wgs), 1, 3, 1)
        t = statistics.median(ms) * 1e-3
        units = wgs * 4 * iters * per_iter  # per wave: MFMAs (mfma), 32-VALU groups (valu), tile-blocks (mix)
        rates[name] = {"units_per_s": units / t, "seconds": t}
    mfma_tops = rates["mfma"]["units_per_s"] * 65536 / 1e12
    simds = 4 * cus
    valu_ns = simds / (rates["valu"]["units_per_s"] * 32) * 1e9  # ns per wave64 VALU op per SIMD
    mix_ns = simds / rates["mix"]["units_per_s"] * 1e9            # ns per tile-block per SIMD
    mix_tops = rates["mix"]["units_per_s"] * 65536 / 1e12
    mix16_ns = simds / rates["mix_f16"]["units_per_s"] * 1e9
    # co-resident roles: 2 eight-wave workgroups a CU = one wave of each role on every SIMD, twice
    split = {}
    for which, name in ((probes.SPLIT_I8_VALU, "i8_mfma|cvt+fma"), (probes.SPLIT_I8_FMA, "i8_mfma|fma"),
                        (probes.SPLIT_F32_VALU, "f32_outer_mfma|cvt+fma")):
        t = {}
        for mask, part in ((1, "a"), (2, "b"), (3, "both")):
            ms = rotating_trials(gpu, lambda i, w=which, m=mask: pr.probe(w, iters=4096, workgroups=2 * cus, mask=m),
                                 1, 3, 1)
            t[part] = statistics.median(ms) * 1e3
        lo, hi = min(t["a"], t["b"]), max(t["a"], t["b"])
        split[name] = {"a_us": round(t["a"], 1), "b_us": round(t["b"], 1), "both_us": round(t["both"], 1),
                       "both_over_sum": round(t["both"] / (t["a"] + t["b"]), 3),
                       "overlapped_frac_of_shorter": round((t["a"] + t["b"] - t["both"]) / lo, 3),
                       "both_over_max": round(t["both"] / hi, 3)}
    pr.close()
    log(f"empty kernel {empty_us:.2f} us/launch; int8 MFMA only {mfma_tops:.0f} TOPS; VALU {valu_ns:.2f} ns/op/SIMD; "
        f"GEMM tile-block mix {mix_ns:.1f} ns/SIMD = {mix_tops:.0f} TOPS (f16-MFMA family's mix {mix16_ns:.1f} ns); "
        "co-resident split (both / sum): " + ", ".join(f"{k} {v['both_over_sum']}" for k, v in split.items()))
    return {"read_bytes": read_bytes, "read_copies": copies,
            "read_us_by_shape": {n: round(u, 3) for n, u in table.items()},
            "ceiling_gbs": round(read_bytes / (best_us * 1e-6) / 1e9, 1), "ceiling_us": round(best_us, 3),
            "ceiling_kernel": f"q8_probe_read ({best_name})",
            "empty_kernel_us_per_launch": round(empty_us, 3),
            "mfma_i8_tops": round(mfma_tops, 1),
            # the nominal 5.03 POPS is 8192 int8 ops per clock per CU at 2.4 GHz:
            # the clock at which the measured MFMA-only rate is that per-CU rate
            "mfma_implied_sclk_ghz": round(mfma_tops * 1e12 / (cus * 8192) / 1e9, 3),
            "valu_ns_per_op_per_simd": round(valu_ns, 3),
            "tile_block_mix_ns_per_simd": round(mix_ns, 2), "tile_block_mix_tops": round(mix_tops, 1),
            "tile_block_mix_f16_ns_per_simd": round(mix16_ns, 2),
            "coresident_split": split}


def bench_launch_reads(gpu, steps, warmup):
    """The plain-read ceiling at the byte counts of the decode step's
    launches (weights only): what one launch of that size can read on this
    box, best of the read shapes.  Its own section: a rocprofv3 kernel trace
    of it died on the host inside hipGraphLaunch, so traced runs leave it out."""
    from llm_amd import probes
    pr = probes.Probes(gpu)
    decode_reads = {}
    for name, nb in (("o", HID * HID // 32 * 34), ("qkv", 3 * HID * HID // 32 * 34),
                     ("down", FFN * HID // 32 * 34), ("gate_up", 2 * FFN * HID // 32 * 34),
                     ("lm_head", VOCAB * HID // 32 * 34)):
        cp = copies_for(nb)
        us, shape, _ = best_read(gpu, pr, nb, cp, max(cp, min(steps, 100)), min(warmup, 10))
        decode_reads[name] = {"bytes": nb, "us": round(us, 3), "gbs": round(nb / (us * 1e-6) / 1e9, 1),
                              "shape": shape}
    pr.close()
    log("plain reads at the decode launches' sizes, MALL-cold: " +
        ", ".join(f"{n} {v['bytes'] / 1e6:.1f} MB {v['us']:.2f} us ({v['shape']})" for n, v in decode_reads.items()))
    return decode_reads


# ---------------------------------------------------------------------------
# n = 512 layer projections
# ---------------------------------------------------------------------------

def own_prepared(gpu, prep, n, k):
    """Copy a prepared operand (quants, then f32 scales) into a buffer we own."""
    from llm_amd import q8
    qbytes, sbytes = prep.quant_bytes(), prep.scale_bytes()
    buf = gpu.alloc(qbytes + sbytes)
    q8._check(q8.lib().q8_copy_device(gpu.handle, buf.ptr, prep.quants, qbytes))
    q8._check(q8.lib().q8_copy_device(gpu.handle, buf.ptr + qbytes, prep.scales, sbytes))
    return q8.Prepared(buf.ptr, buf.ptr + qbytes, n, k, prep.format), buf


def bench_layer_n512(gpu, steps, warmup, rng, n=512):
    """configs[3] on rotating copies of the layer's seven weights."""
    import oracle
    from llm_amd import q8
    names = ("q", "k", "v", "o", "gate", "up", "down")
    shapes = {"q": (HID, HID), "k": (HID, HID), "v": (HID, HID), "o": (HID, HID), "gate": (FFN, HID),
              "up": (FFN, HID), "down": (HID, FFN)}
    base = {nm: make_weight(rng, *shapes[nm]) for nm in names}
    layer_bytes = sum(w.data.size for w in base.values())
    copies = copies_for(layer_bytes)
    layers = [base] + [{nm: q8.Weight(base[nm].data.copy(), base[nm].k, base[nm].out) for nm in names}
                       for _ in range(copies - 1)]
    for L in layers:
        for w in L.values():
            gpu.resident(w)
    x = oracle.make_activations(rng, n, HID)
    xb, hb = gpu.alloc(4 * n * HID), gpu.alloc(4 * n * HID)
    xb.upload(x)
    hb.upload(x)
    qkv, act, gu = gpu.alloc(4 * n * 3 * HID), gpu.alloc(4 * n * FFN), gpu.alloc(4 * n * 2 * FFN)
    ops = {"qkv": 2 * n * 3 * HID * HID, "o": 2 * n * HID * HID, "gate_up": 2 * n * 2 * FFN * HID,
           "down": 2 * n * HID * FFN}
    total_ops = sum(ops.values())

    def make_layer_set(announce):
        def layer_set(i):
            L, N = layers[i], layers[(i + 1) % copies]
            hint = gpu.gemm_prefetch if announce else (lambda ws: None)
            p = gpu.prepare(xb, 0, n, HID)
            hint([L["o"]])  # read by the next GEMM launch's cache riders
            gpu.matmul_prompt_group([(L["q"], qkv, 0), (L["k"], qkv, n * HID), (L["v"], qkv, 2 * n * HID)], p, n,
                                    HID)
            hint([L["gate"], L["up"]])
            gpu.matmul(L["o"], qkv, 0, n, hb, 0, bias=hb)                  # O with its residual
            hint([L["down"]])
            pd = gpu.gate_up_silu(L["gate"], L["up"], hb, 0, n, act, 0, want_prepared=True)
            hint([N["q"], N["k"], N["v"]])                                 # the next layer's
            gpu.matmul(L["down"], act, 0, n, hb, 0, prepared=pd, bias=hb)  # down with its residual
        return layer_set

    ms = rotating_trials(gpu, make_layer_set(True), copies, max(steps // 4, copies), warmup)
    s = summary(ms, total_ops, 1e-12)
    log(f"n={n} layer set (MALL-cold, {copies} layer copies): {s['median_us']:.1f} us, {s['value']:.1f} TOPS "
        f"({s['value'] / INT8_PEAK_TOPS * 100:.1f}% of int8 peak); trials {s['trials']}")
    ms_plain = rotating_trials(gpu, make_layer_set(False), copies, max(steps // 4, copies), warmup)
    plain_us = statistics.median(ms_plain) * 1e3
    log(f"n={n} layer set without weight announcements: {plain_us:.1f} us")

    # each piece alone on the same rotation; prepared operands copied into
    # buffers of our own (a Prepared views the one activation workspace)
    norm_w = (1.0 + 0.1 * rng.standard_normal(HID)).astype(np.float32)
    p, pbuf = own_prepared(gpu, gpu.prepare(xb, 0, n, HID), n, HID)
    pf, pfbuf = own_prepared(gpu, gpu.prepare(act, 0, n, FFN), n, FFN)
    pieces = {
        "quantize_x": lambda i: gpu.prepare(xb, 0, n, HID),
        "quantize_act": lambda i: gpu.prepare(act, 0, n, FFN),
        "norm_prepare_x": lambda i: gpu.norm_prepare(xb, 0, norm_w, 1e-6, n),
        "qkv": lambda i: gpu.matmul_prompt_group([(layers[i]["q"], qkv, 0), (layers[i]["k"], qkv, n * HID),
                                                  (layers[i]["v"], qkv, 2 * n * HID)], p, n, HID),
        "o": lambda i: gpu.matmul(layers[i]["o"], qkv, 0, n, hb, 0, prepared=p),
        "gate_up": lambda i: gpu.matmul_prompt_group([(layers[i]["gate"], gu, 0), (layers[i]["up"], gu, n * FFN)],
                                                     p, n, HID),
        "gate_up_silu": lambda i: gpu.gate_up_silu(layers[i]["gate"], layers[i]["up"], hb, 0, n, act, 0,
                                                   want_prepared=True),
        "down": lambda i: gpu.matmul(layers[i]["down"], act, 0, n, hb, 0, prepared=pf),
    }
    piece_us = {}
    for name, fn in pieces.items():
        piece_us[name] = round(statistics.median(rotating_trials(gpu, fn, copies, max(steps // 2, copies), 2)) * 1e3,
                               2)
    piece_tops = {nm: round(ops[nm] / (piece_us[nm] * 1e-6) / 1e12, 1) for nm in ("qkv", "o", "gate_up", "down")}
    # a piece rotates only its own weights over the copies: where those are
    # smaller than the Infinity Cache, the piece runs MALL-warm, the layer set not
    piece_w = {"qkv": ("q", "k", "v"), "o": ("o",), "gate_up": ("gate", "up"), "gate_up_silu": ("gate", "up"),
               "down": ("down",)}
    piece_mall = {nm: ("warm" if copies * sum(base[w].data.size for w in ws) < MALL_BYTES else "cold")
                  for nm, ws in piece_w.items()}
    # the compulsory-traffic bound of each projection: weights + Q8_0 X + f32 Y
    # once each, at 8 TB/s, against its ops at the 5.0 POPS int8 peak
    dims = {"qkv": (3 * HID, HID), "o": (HID, HID), "gate_up": (2 * FFN, HID), "down": (HID, FFN)}
    bound = {}
    for nm, (m_, k_) in dims.items():
        nbytes = m_ * k_ // 32 * 34 + n * k_ * 9 // 8 + 4 * n * m_
        t_hbm, t_mfma = nbytes / (HBM_PEAK_GBS * 1e3), ops[nm] / (INT8_PEAK_TOPS * 1e6)
        bound[nm] = {"bytes": nbytes, "t_hbm_us": round(t_hbm, 2), "t_mfma_us": round(t_mfma, 2),
                     "max_frac_of_mfma_peak": round(t_mfma / max(t_hbm, t_mfma), 3),
                     "attained_frac": round(piece_tops[nm] / INT8_PEAK_TOPS, 4)}
    log("n=512 pieces (us): " + ", ".join(f"{k} {v}" for k, v in piece_us.items()))
    for L in layers:
        for w in L.values():
            gpu.release(w)
    for b in (xb, hb, qkv, act, gu, pbuf, pfbuf):
        b.free()
    return {"us": s["median_us"], "tops": s["value"], "trials_tops": s["trials"], "ops": total_ops,
            "us_unannounced": round(plain_us, 2),
            "frac": s["value"] / INT8_PEAK_TOPS, "ops_by_projection": ops, "copies": copies,
            "quantize_us": piece_us["quantize_x"], "projections_us": piece_us, "projections_tops": piece_tops,
            "projections_mall": piece_mall, "projections_traffic_bound": bound}


# ---------------------------------------------------------------------------
# configs[1], configs[2]
# ---------------------------------------------------------------------------

def bench_gemm_configs1(gpu, m, k, n, steps, warmup, rng, label):
    import oracle
    from llm_amd import q8
    base = make_weight(rng, m, k)
    per = m * k // 32 * 34 + n * k * 4 + 4 * n * m
    copies = copies_for(m * k // 32 * 34)
    weights = [base] + [q8.Weight(base.data.copy(), k, m) for _ in range(copies - 1)]
    for w in weights:
        gpu.resident(w)
    xb, yb = gpu.alloc(4 * n * k), gpu.alloc(4 * n * m)
    xb.upload(oracle.make_activations(rng, n, k, outlier_rate=0.01))
    ms = rotating_trials(gpu, lambda i: gpu.matmul(weights[i], xb, 0, n, yb, 0), copies, max(steps // 2, copies),
                         warmup)
    s = summary(ms, per, 1e-9)
    tops = 2 * m * n * k / (s["median_us"] * 1e-6) / 1e12
    log(f"{label}: {s['median_us']:.2f} us/matmul, {s['value']:.0f} GB/s, {tops:.1f} TOPS")
    for w in weights:
        gpu.release(w)
    xb.free()
    yb.free()
    return {"us": s["median_us"], "gbs": round(s["value"], 1), "tops": round(tops, 2), "bytes": per}


def bench_decode_layer(gpu, steps, warmup, rng):
    """the n = 1 layer set on rotating layer copies, and the
    lm_head GEMV + argmax (301 MB: larger than the Infinity Cache)."""
    from llm_amd import q8
    shapes = [(HID, HID)] * 4 + [(FFN, HID), (FFN, HID), (HID, FFN)]
    base = [make_weight(rng, *sh) for sh in shapes]
    wbytes = sum(w.data.size for w in base)
    copies = copies_for(wbytes)
    layers = [base] + [[q8.Weight(w.data.copy(), w.k, w.out) for w in base] for _ in range(copies - 1)]
    for L in layers:
        # q/k/v and gate/up as contiguous groups (q8_weight_group_resident),
        # as a decoder keeps them; O and down alone
        gpu.resident_group(L[0:3])
        gpu.resident_group(L[4:6], pair=True)
        for w in (L[3], L[6]):
            gpu.resident(w)
    x = rng.standard_normal(HID, dtype=np.float32)
    xb, qkv, hb, act = gpu.alloc(4 * HID), gpu.alloc(4 * 3 * HID), gpu.alloc(4 * HID), gpu.alloc(4 * FFN)
    xb.upload(x)
    hb.upload(x)

    def layer(i):
        wq, wk, wv, wo, wg, wu, wd = layers[i]
        gpu.matmul_decode_group([(wq, qkv, 0), (wk, qkv, HID), (wv, qkv, 2 * HID)], xb, 0, HID)
        gpu.matmul(wo, qkv, 0, 1, hb, 0, bias=hb)
        gpu.gate_up_silu(wg, wu, hb, 0, 1, act, 0)
        gpu.matmul(wd, act, 0, 1, hb, 0, bias=hb)

    s = summary(rotating_trials(gpu, layer, copies, max(steps // 2, copies), warmup), wbytes, 1e-9)
    log(f"decode layer set (MALL-cold, {copies} copies): {s['median_us']:.1f} us, {s['value']:.0f} GB/s of weights")
    for L in layers:
        for w in L:
            gpu.release(w)

    wl = make_weight(rng, VOCAB, HID)
    gpu.resident(wl)
    logits = gpu.alloc(4 * VOCAB)
    per = gemv_bytes(VOCAB, HID)
    h = summary(rotating_trials(gpu, lambda i: gpu.matmul(wl, xb, 0, 1, logits, 0), 1, 20, 2), per, 1e-9)
    t0 = time.perf_counter()
    best = gpu.lm_head_argmax(wl, xb, 0, logits, 0)
    call_us = round((time.perf_counter() - t0) * 1e6, 1)
    # the argmax check: the folded argmax against the first maximum of the
    # logits it wrote, and the top-2 logit gap (how far the winner stands clear)
    lv = logits.download(np.float32, VOCAB)
    order = np.argsort(lv, kind="stable")[::-1]
    first = int(np.flatnonzero(lv == lv[order[0]])[0])
    top2_gap = float(lv[order[0]] - lv[order[1]])
    log(f"lm_head 122880x2304: {h['median_us']:.1f} us, {h['value']:.0f} GB/s; argmax {best} "
        f"(first max of the logits {first}), top-2 gap {top2_gap:.3g}")
    gpu.release(wl)
    for b in (xb, qkv, hb, act, logits):
        b.free()
    return ({"us": s["median_us"], "weight_bytes": wbytes, "gbs": round(s["value"], 1), "copies": copies},
            {"us": h["median_us"], "gbs": round(h["value"], 1), "bytes": per, "argmax": best,
             "argmax_matches_logits": best == first, "top2_logit_gap": top2_gap,
             "top2_logits": [float(lv[order[0]]), float(lv[order[1]])], "argmax_call_us_host": call_us})


# ---------------------------------------------------------------------------
# the decoder, llama-bench style
# ---------------------------------------------------------------------------

def tactic_names(gpu):
    """The kernel each configs shape runs (the tactic table's choice)."""
    from llm_amd import q8
    shapes = {"configs0_gemv": (1, 5760, HID), "configs1_n8": (8, 5760, HID), "configs1_n64": (64, 5760, HID),
              "n512_qkv": (512, 3 * HID, HID), "n512_o": (512, HID, HID), "n512_gate_up": (512, 2 * FFN, HID),
              "n512_down": (512, HID, FFN), "decode_o": (1, HID, HID), "decode_down": (1, HID, FFN),
              "lm_head": (1, VOCAB, HID)}
    out = {}
    for name, (n, m, k) in shapes.items():
        t = gpu.plan(n, m, k)
        out[name] = t.get("name")
    return out


def bench_decoder(gpu, rng, prompt=512, steps=128, reps=5):
    """pp512 / tg128 as llama-bench reports them: each repeat
    resets the context, prefills `prompt` random ids (pp) and decodes `steps`
    greedy tokens (tg); tok/s mean and sample std over `reps` repeats, after
    one eager pass and one capture pass.  Host wall clock around calls that
    end in a wait.

    The model has an output head of its own (a GGUF with output.weight,
    model.rs:519-524: the same 122880 x 2304 Q8_0 bytes per token as the tied
    head) and embedding rows at scale std 4: with the head tied to a 0.02
    embedding the last hidden state barely depends on the current token and
    greedy decode repeats one token, so the fed-back token path would run on
    one value; here the tokens vary (distinct_tokens)."""
    from llm_amd import decoder as dm
    cfg = dm.config(n_layer=42, n_embd=HID, n_ff=FFN, n_head=36, n_head_kv=36, head_dim=64, n_vocab=VOCAB,
                    capacity=4096, max_batch=prompt, untied_output=1, embd_std=4.0)
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
    pp = [prompt / t for t in pre]
    tg = [steps / t for t in gen]
    layer_w = (HID * 3 * HID + HID * HID + 2 * FFN * HID + HID * FFN) // 32 * 34
    per_token = 42 * layer_w + VOCAB * HID // 32 * 34
    t_gen = statistics.mean(gen)
    out = {"r": reps,
           f"pp{prompt}_tok_s": round(statistics.mean(pp), 1), f"pp{prompt}_tok_s_std": round(statistics.stdev(pp), 1),
           f"tg{steps}_tok_s": round(statistics.mean(tg), 1), f"tg{steps}_tok_s_std": round(statistics.stdev(tg), 2),
           "prefill_ms": round(statistics.mean(pre) * 1e3, 3),
           "decode_ms_per_token": round(t_gen / steps * 1e3, 4),
           "decode_weight_bytes_per_token": per_token,
           "decode_weight_gbs": round(per_token * steps / t_gen / 1e9, 1),
           "decode_floor_ms_per_token_at_8tbs": round(per_token / 8e12 * 1e3, 3),
           "tokens_first_16": tokens[:16], "distinct_tokens": len(set(tokens))}
    log(f"decoder: pp{prompt} {out[f'pp{prompt}_tok_s']} +- {out[f'pp{prompt}_tok_s_std']} tok/s; tg{steps} "
        f"{out[f'tg{steps}_tok_s']} +- {out[f'tg{steps}_tok_s_std']} tok/s ({out['decode_ms_per_token']} ms/token, "
        f"{out['decode_weight_gbs']} GB/s of weights)")
    return out


def bench_decode_chain(gpu, steps=20, visible=600, splits=3):
    """configs[4]'s decode step as its op chain launched eagerly (no graph): the
    same calls q8_decoder_generate's captured step makes, for a kernel trace
    (a kernel trace of the captured step itself aborted on the host; the
    eager chain runs the same kernels, arguments and launch shapes).  The
    weights are a synthetic decoder's (generated on the device, q/k/v and
    gate/up as its contiguous groups); returns the host time per step."""
    from llm_amd import decoder as dm
    heads, hd, cap, n_layer = 36, 64, 4096, 42
    rng = np.random.default_rng(5)
    dec = dm.Decoder(gpu, dm.config(n_layer=n_layer, n_embd=HID, n_ff=FFN, n_head=heads, head_dim=hd, n_vocab=VOCAB,
                                    capacity=8, max_batch=1, untied_output=1), seed=5)
    layers = []
    for li in range(n_layer):
        w = {n: dec.weight(li, i) for i, n in enumerate("qkvogud")}
        w["an"] = (1.0 + 0.1 * rng.standard_normal(HID)).astype(np.float32)
        w["fn"] = (1.0 + 0.1 * rng.standard_normal(HID)).astype(np.float32)
        w["kc"], w["vc"] = gpu.alloc(2 * cap * HID), gpu.alloc(2 * cap * HID)
        layers.append(w)
    head = dec.weight(-1, dm.OUTPUT)
    onorm = (1.0 + 0.1 * rng.standard_normal(HID)).astype(np.float32)
    x, q, act = gpu.alloc(4 * HID), gpu.alloc(4 * HID), gpu.alloc(4 * FFN)
    logits, tok, pos = gpu.alloc(4 * VOCAB), gpu.alloc(4), gpu.alloc(4)
    x.upload(rng.standard_normal(HID).astype(np.float32))
    pos.upload(np.array([visible - 1], np.int32))
    scale = 1.0 / math.sqrt(hd)
    t0 = time.perf_counter()
    for _ in range(steps):
        for w in layers:
            gpu.norm_qkv_rope(w["an"], 1e-6, w["q"], w["k"], w["v"], x, 0, q, 0, w["kc"], w["vc"], heads, heads, hd,
                              hd, 10000.0, cap, pos)
            gpu.attention_matmul_add(q, w["kc"], w["vc"], heads, heads, hd, cap, scale, pos, splits, w["o"], x)
            gpu.norm_gate_up_silu(w["fn"], 1e-6, w["g"], w["u"], x, 0, act, 0)
            gpu.matmul(w["d"], act, 0, 1, x, 0, bias=x)
        gpu.norm_lm_head_argmax(onorm, 1e-6, head, x, 0, logits, 0, tok)
        gpu.sync()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    log(f"decode op chain, eager: {ms:.3f} ms a step (host clock; {steps} steps at {visible} positions)")
    for w in layers:
        w["kc"].free()
        w["vc"].free()
    dec.close()
    for b in (x, q, act, logits, tok, pos):
        b.free()
    return {"ms_per_step_host": round(ms, 3), "steps": steps, "visible": visible, "splits": splits}


# ---------------------------------------------------------------------------
# CPU baseline and counter calibration
# ---------------------------------------------------------------------------

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


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(seconds: float = 8.0):
    """The oracle (C restatement of tensor::matmul, rayon-style row split,
    AVX2 order) on this host: the configs[0] GEMV over rotating weight copies
    (GB/s) and the configs[3] n = 512 layer set (TOPS), each for about
    `seconds` of wall time.  Threads: every core this process may run on,
    capped at the box's CPU share for one GPU (OMP_NUM_THREADS, 16 on the
    GPU boxes), which rayon's default (available_parallelism) would not see."""
    import oracle
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = max(1, min(affinity, share) if share > 0 else affinity)
    rng = np.random.default_rng(0x5EED)
    m, k = 5760, HID
    base = oracle.make_q8_weight(rng, m, k)
    copies = copies_for(base.size)
    ws = [base] + [base.copy() for _ in range(copies - 1)]
    x = rng.standard_normal(k, dtype=np.float32)
    oracle.matmul(ws[0], k, m, x, 1, threads=threads)
    reps = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        oracle.matmul(ws[reps % copies], k, m, x, 1, threads=threads)
        reps += 1
    dt = time.perf_counter() - t0
    gbs = gemv_bytes(m, k) * reps / dt / 1e9
    del ws
    # the four projections at n = 512
    n = 512
    lw = {nm: oracle.make_q8_weight(rng, o, kk) for nm, (o, kk) in
          {"qkv": (3 * HID, HID), "o": (HID, HID), "gate_up": (2 * FFN, HID), "down": (HID, FFN)}.items()}
    xa = oracle.make_activations(rng, n, HID)
    xf = oracle.make_activations(rng, n, FFN)
    ops = 2 * n * (3 * HID * HID + HID * HID + 2 * FFN * HID + HID * FFN)
    layers = 0
    t0 = time.perf_counter()
    while True:
        oracle.matmul(lw["qkv"], HID, 3 * HID, xa, n, threads=threads)
        oracle.matmul(lw["o"], HID, HID, xa, n, threads=threads)
        oracle.matmul(lw["gate_up"], HID, 2 * FFN, xa, n, threads=threads)
        oracle.matmul(lw["down"], FFN, HID, xf, n, threads=threads)
        layers += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt2 = time.perf_counter() - t0
    tops = ops * layers / dt2 / 1e12
    model = cpu_model()
    log(f"cpu baseline ({model}, nproc {os.cpu_count()}, affinity {affinity}, {threads} threads, "
        f"{oracle.simd_path()}): GEMV {gbs:.1f} GB/s ({reps} GEMVs over {copies} copies); n=512 layer set "
        f"{tops:.3f} TOPS ({layers} layer sets in {dt2:.1f} s)")
    return {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{reps} configs[0] GEMVs (5760x2304, n=1, f32 x) over {copies} rotating weight copies in "
                      f"{dt:.1f} s; {layers} configs[3] n=512 layer sets in {dt2:.1f} s",
            "n512_layer_tops": round(tops, 4), "cpu_model": model, "nproc": os.cpu_count(),
            "affinity_cores": affinity, "threads": threads, "simd_path": oracle.simd_path(),
            "label": "C restatement of the reference rayon CPU path (oracle/q8_oracle.c)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=8.0)
    ap.add_argument("--sustained-seconds", type=float, default=6.0,
                    help="configs[0] GEMV replayed back to back for this long after its trials (0: skip)")
    ap.add_argument("--sections", default="all",
                    help="comma list of gemv,ceilings,reads,gemm,extras,decoder,cpu (default all) and chain (named "
                         "only); a profiler run names one so each kernel's average covers one workload")
    args = ap.parse_args()
    default = {"gemv", "ceilings", "reads", "gemm", "extras", "decoder", "cpu"}
    sections = set(default) if args.sections == "all" else set(args.sections.split(","))
    unknown = sections - default - {"chain"}
    if unknown:
        ap.error(f"unknown sections {sorted(unknown)}")
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus "
              f"{args.gpus}); it shards by output rows, which one GPU does not exercise", file=sys.stderr)
        sys.exit(2)
    steps = max(1, args.steps)
    warmup = max(0, args.warmup)

    from llm_amd import q8
    rng = np.random.default_rng(0x5EED)
    gpu = q8.Gpu(0)
    log(f"device {gpu.name}")
    calibration_copy(gpu)
    m, k = 5760, HID
    gemv = {"gbs": None, "us_per_step": None, "bytes_per_step": gemv_bytes(m, k), "copies": None}
    if "gemv" in sections:
        gemv = bench_gemv(gpu, m, k, steps, warmup, rng, args.sustained_seconds)
    ceil = bench_ceilings(gpu, steps, warmup, gemv_bytes(m, k)) if "ceilings" in sections else {}
    if "reads" in sections:
        ceil["decode_launch_reads"] = bench_launch_reads(gpu, steps, warmup)
    gemm = {"tops": None, "frac": None, "us": None, "ops": None}
    if "gemm" in sections:
        gemm = bench_layer_n512(gpu, steps, warmup, rng)
    extras = {}
    if "extras" in sections:
        extras["configs1_n8"] = bench_gemm_configs1(gpu, m, k, 8, steps, warmup, rng, "configs[1] n=8")
        extras["configs1_n64"] = bench_gemm_configs1(gpu, m, k, 64, steps, warmup, rng, "configs[1] n=64")
        layer, head = bench_decode_layer(gpu, steps, warmup, rng)
        extras["configs2_decode_layer"] = layer
        extras["configs2_lm_head"] = head
    decoder = bench_decoder(gpu, rng) if "decoder" in sections else None
    chain = bench_decode_chain(gpu) if "chain" in sections else None
    tactics = tactic_names(gpu)
    build = json.loads(q8.build_info())
    gpu.close()
    cpu = cpu_baseline(args.cpu_seconds) if "cpu" in sections and args.cpu_seconds > 0 else None

    value = gemv["gbs"]
    ceiling = ceil.get("ceiling_gbs")

    def r(v, nd=1):
        return round(v, nd) if v is not None else None

    line = {
        "metric": METRIC,
        "value": r(value),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": gemv["us_per_step"] / 1e3 if gemv["us_per_step"] is not None else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded random Q8_0 weights (q ~ U[-127,127], d = f16(|N(0,0.02)|/127)), x ~ N(0,1)",
        "config": {"workload": "configs[0] Q8_0 GEMV n=1, W 5760x2304 (q8_0 weights x f32 x, f32 FMA), MALL-cold "
                               "(rotating copies); median of 5 trials of --steps steps",
                   "M": m, "K": k, "n": 1, "rotating_copies": gemv["copies"], "trials": TRIALS},
        "roofline": {"bound": "hbm", "achieved": r(value), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4) if value is not None else None,
                     "traffic": traffic_from_profile(build),
                     "kernel": tactics.get("configs0_gemv"), "bytes_per_launch": gemv["bytes_per_step"],
                     "ceiling_gbs": ceiling, "ceiling_kernel": ceil.get("ceiling_kernel"),
                     "frac_of_ceiling": round(value / ceiling, 4) if value and ceiling else None,
                     "trials_gbs": gemv.get("trials_gbs"), "mall_hot_gbs": gemv.get("mall_hot_gbs")},
        "configs0_quantized_x": {"value": gemv.get("q8x_gbs"), "unit": "GB/s", "us_per_step": gemv.get("q8x_us"),
                                 "frac": round(gemv["q8x_gbs"] / HBM_PEAK_GBS, 4) if gemv.get("q8x_gbs") else None,
                                 "trials_gbs": gemv.get("q8x_trials_gbs"), "entry": "q8_matmul_q8",
                                 "workload": "configs[0] with x quantized to Q8_0 per 32-block in the same launch "
                                             "(the n >= 2 arithmetic at n = 1), int8 block dots"},
        "configs0_sustained": gemv.get("sustained"),
        "gemm_n512": {"value": r(gemm["tops"], 2), "unit": "TOPS", "peak": INT8_PEAK_TOPS,
                      "frac": round(gemm["frac"], 4) if gemm["frac"] is not None else None,
                      "us_per_layer": r(gemm["us"], 2), "ops_per_layer": gemm["ops"],
                      "us_per_layer_unannounced": gemm.get("us_unannounced"),
                      "mall": f"cold ({gemm.get('copies')} rotating layer copies)",
                      "trials_tops": gemm.get("trials_tops"),
                      "mfma_ceiling_tops": ceil.get("mfma_i8_tops"),
                      "tile_block_ceiling_tops": ceil.get("tile_block_mix_tops"),
                      "quantize_us": gemm.get("quantize_us"), "projections_us": gemm.get("projections_us"),
                      "projections_tops": gemm.get("projections_tops"),
                      "projections_mall": gemm.get("projections_mall"),
                      "projections_traffic_bound": gemm.get("projections_traffic_bound")},
        "ceilings": ceil,
        "extras": extras,
        "decoder_configs4": decoder,
        "decode_chain": chain,
        "build": {"code_object_sha256": build["code_object_sha256"], "hipcc": build.get("hipcc"),
                  "tactics": tactics},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "q8_gemv_configs0_traffic.md")


def traffic_from_profile(build):
    """HBM bytes per configs[0] GEMV launch from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary, if it was measured on the code object
    loaded now (its sha256 is recorded in the summary); otherwise None."""
    try:
        text = open(TRAFFIC_PROFILE).read()
    except OSError:
        return None
    fields = {}
    for line in text.splitlines():
        if line.startswith("- ") and ": " in line:
            key, val = line[2:].split(": ", 1)
            fields[key.strip("` ")] = val.strip("` ")
    if fields.get("code_object_sha256") != build["code_object_sha256"]:
        return None
    try:
        return int(fields["traffic_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


if __name__ == "__main__":
    main()
