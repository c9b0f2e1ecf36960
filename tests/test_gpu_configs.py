"""GPU parity at the benchmark configurations' full shapes, through the C-ABI.

the decoder layer's four projections at n = 512 tokens (hidden
2304, FFN 5760), each on the launch plan the tactic table picks for its shape
(no option overrides), against the oracle's tensor::matmul
(apps/engine/src/tensor.rs:104-148) under the n >= 2 bar of assert_parity:
  * the q/k/v group 3 x 2304 x 2304 on one prepared activation;
  * O 2304 x 2304 with the residual in its epilogue (Compute::matmul_add,
    compute.rs:537-581: matmul, then y += temp);
  * gate|up 2 x 5760 x 2304 with silu(gate) * up quantized to Q8_0 in the
    epilogue (q8_gate_up_silu_prepared), feeding down 2304 x 5760 with its
    residual;
  * down alone on f32 activations (K = 5760, +-20 outliers).
the synthetic decoder at the benchmark's geometry (hidden 2304,
FFN 5760, 36 x 64 MHA, vocab 122 880, f16 KV cache of 4096, a 512-token
prompt), two layers against the oracle's composition of the reference ops,
and all 42 layers for the properties a whole model has to keep.
"""
import numpy as np
import pytest

import oracle
from llm_amd import decoder as dm
from llm_amd import q8
from test_gpu_decoder import OracleDecoder, check_logits, model_bar
from test_gpu_q8 import assert_bits, assert_parity, exact_at, unpack_prepared

pytestmark = pytest.mark.gpu

SEED = 0x5EED
N, HID, FFN = 512, 2304, 5760


@pytest.fixture(scope="module")
def gpu():
    g = q8.Gpu(0)
    yield g
    g.close()


def weight(r, out, k):
    return q8.Weight(oracle.make_q8_weight(r, out, k), k, out)


def plan_name(gpu, n, out, k):
    t = gpu.plan(n, out, k)
    return ", ".join(f"{key}={t[key]}" for key in sorted(t) if key not in ("name", "evidence")) + f" ({t['name']})"


def test_configs3_qkv_group(gpu):
    r = np.random.default_rng(SEED + 301)
    ws = [weight(r, HID, HID) for _ in range(3)]
    x = oracle.make_activations(r, N, HID)
    xb, qkv = gpu.alloc(4 * N * HID), gpu.alloc(4 * 3 * N * HID)
    xb.upload(x)
    print(f"\nconfigs[3] q/k/v group 6912 x 2304, n=512: plan {plan_name(gpu, N, 3 * HID, HID)}", flush=True)
    p = gpu.prepare(xb, 0, N, HID)
    gpu.matmul_prompt_group([(ws[i], qkv, i * N * HID) for i in range(3)], p, N, HID)
    got = qkv.download(np.float32, 3 * N * HID).reshape(3, N, HID)
    for i, w in enumerate(ws):
        ref = oracle.matmul(w.data, HID, HID, x, N)
        assert_parity(got[i], ref, exact_at(w.data, HID, HID, x, N), f"configs[3] {'qkv'[i]} n=512")
    for w in ws:
        gpu.release(w)
    xb.free()
    qkv.free()


def test_configs3_o_projection_with_residual(gpu):
    r = np.random.default_rng(SEED + 302)
    w = weight(r, HID, HID)
    a = oracle.make_activations(r, N, HID)          # the attention output
    res = r.standard_normal((N, HID)).astype(np.float32)
    ab, yb = gpu.alloc(4 * N * HID), gpu.alloc(4 * N * HID)
    ab.upload(a)
    yb.upload(res)
    print(f"\nconfigs[3] O 2304 x 2304 + residual, n=512: plan {plan_name(gpu, N, HID, HID)}", flush=True)
    gpu.matmul(w, ab, 0, N, yb, 0, bias=yb)
    got = yb.download(np.float32, N * HID).reshape(N, HID)
    ref = (res + oracle.matmul(w.data, HID, HID, a, N)).astype(np.float32)
    ex = exact_at(w.data, HID, HID, a, N)
    assert_parity(got, ref, lambda idx: res.reshape(-1)[idx].astype(np.float64) + ex(idx), "configs[3] O+res n=512")
    gpu.release(w)
    ab.free()
    yb.free()


def test_configs3_gate_up_silu_then_down(gpu):
    """The fused FFN chain at its real shapes: the gate|up GEMM with the SiLU
    product quantized in its epilogue, then down on those prepared bytes with
    the residual.  The prepared bytes dequantize to the oracle's silu(g) * u
    within half a quantization step (plus the f32 bar of g and u); the down
    output is held to the n >= 2 bar against the oracle run on the same
    activation bytes (the oracle's quantize_q8_0 of the dequantized blocks
    gives back the same quants)."""
    r = np.random.default_rng(SEED + 303)
    wg, wu = weight(r, FFN, HID), weight(r, FFN, HID)
    wd = weight(r, HID, FFN)
    x = oracle.make_activations(r, N, HID)
    res = r.standard_normal((N, HID)).astype(np.float32)
    xb, yb, ab = gpu.alloc(4 * N * HID), gpu.alloc(4 * N * HID), gpu.alloc(4 * N * FFN)
    xb.upload(x)
    yb.upload(res)
    print(f"\nconfigs[3] gate|up 11520 x 2304 + SiLU -> Q8_0, n=512: plan {plan_name(gpu, N, 2 * FFN, HID)}; "
          f"down 2304 x 5760: plan {plan_name(gpu, N, HID, FFN)}", flush=True)
    px = gpu.prepare(xb, 0, N, HID)
    pa = gpu.gate_up_silu_prepared(wg, wu, px)
    assert pa.n == N and pa.k == FFN
    qa, sa = unpack_prepared(gpu, pa, N, FFN)
    qa, sa = qa[:N], sa[:N]
    # down reads the prepared bytes (ab is the f32 operand the call would
    # otherwise quantize; with `prepared` it is not read)
    gpu.matmul(wd, ab, 0, N, yb, 0, prepared=pa, bias=yb)
    got = yb.download(np.float32, N * HID).reshape(N, HID)

    g = oracle.matmul(wg.data, HID, FFN, x, N)
    u = oracle.matmul(wu.data, HID, FFN, x, N)
    act = oracle.silu_mul(g, u).reshape(N, FFN // 32, 32)
    deq = qa.astype(np.float32).reshape(N, FFN // 32, 32) * sa[:, :, None]
    bound = 0.5 * sa[:, :, None] * 1.001 + 1e-4 * np.abs(act) + 1e-5
    bad = ~(np.abs(deq - act) <= bound)
    assert not bad.any(), f"SiLU product bytes: {int(bad.sum())} values beyond half a step of the oracle's"
    # a block's peak maps to +-127 (quantize_q8_0: scale = peak / 127)
    peaks = np.abs(qa.reshape(N, FFN // 32, 32)).max(axis=2)
    assert np.all((peaks == 127) | (sa == 0))

    xd = deq.reshape(N, FFN).astype(np.float32)
    rq = np.stack([oracle.quantize_q8_0(xd[t])[0] for t in range(N)])
    assert np.array_equal(rq.reshape(N, FFN), qa.reshape(N, FFN)), "re-quantizing the bytes changed a quant"
    ref = (res + oracle.matmul(wd.data, FFN, HID, xd, N)).astype(np.float32)
    ex = exact_at(wd.data, FFN, HID, quants=qa.reshape(N, FFN), scales=sa)
    assert_parity(got, ref, lambda idx: res.reshape(-1)[idx].astype(np.float64) + ex(idx),
                  "configs[3] down(silu(gate)*up)+res n=512")
    for w in (wg, wu, wd):
        gpu.release(w)
    for b in (xb, yb, ab):
        b.free()


def test_configs3_down_on_f32_activations(gpu):
    r = np.random.default_rng(SEED + 304)
    w = weight(r, HID, FFN)
    x = oracle.make_activations(r, N, FFN, outlier_rate=0.01)
    xb, yb = gpu.alloc(4 * N * FFN), gpu.alloc(4 * N * HID)
    xb.upload(x)
    print(f"\nconfigs[3] down 2304 x 5760, n=512: plan {plan_name(gpu, N, HID, FFN)}", flush=True)
    gpu.matmul(w, xb, 0, N, yb, 0)
    got = yb.download(np.float32, N * HID).reshape(N, HID)
    ref = oracle.matmul(w.data, FFN, HID, x, N)
    assert_parity(got, ref, exact_at(w.data, FFN, HID, x, N), "configs[3] down K=5760 n=512")
    gpu.release(w)
    xb.free()
    yb.free()


# ---- the decoder at the benchmark geometry ----

def configs4(n_layer):
    return dm.config(n_layer=n_layer, n_embd=HID, n_ff=FFN, n_head=36, n_head_kv=36, head_dim=64, n_vocab=122880,
                     capacity=4096, max_batch=512)


def test_configs4_geometry_two_layers_match_the_oracle(gpu):
    """Two layers of the configs[4] decoder (the 512-token prompt, then four
    greedy decode steps through the captured graph) against the oracle's
    composition of rmsnorm, tensor::matmul, rope, the f16 cache, attention,
    silu_mul and the residuals.  The bar is the model's own sensitivity: the
    oracle run again with its input changed in the last bit moves the logits
    by ~1% of their scale at this width (int8 activation and f16 cache
    rounding flip on last-bit differences), so the device must stay within
    twice what the oracle moves by (model_bar)."""
    dec = dm.Decoder(gpu, configs4(2), seed=41)
    try:
        ref = OracleDecoder(gpu, dec)
        twin = ref.twin(2.0 ** -23)
        prompt = np.random.default_rng(SEED + 4).integers(0, 122880, N).astype(np.uint32)
        print("\nconfigs[4] geometry, 2 layers: prompt of 512", flush=True)
        nxt = dec.forward(prompt)
        ref_logits = ref.forward(prompt)
        tol, sens = model_bar(ref_logits, twin.forward(prompt))
        print(f"oracle moves by {sens:.3e} under a last-bit change of its input", flush=True)
        got = dec.logits()
        check_logits(got, ref_logits, "configs[4] prompt logits", tol)
        assert nxt == int(np.argmax(got))
        steps = dec.generate(4)
        assert dec.position == N + 4
        feed = [nxt] + [int(t) for t in steps[:-1]]
        for i, tok in enumerate(feed):
            logits = ref.forward([tok])
            tol, sens = model_bar(logits, twin.forward([tok]))
            top2 = np.sort(logits)[-2:]
            if top2[1] - top2[0] > 2 * tol:
                assert int(steps[i]) == oracle.argmax(logits), f"decode step {i}"
        check_logits(dec.logits(), logits, "configs[4] last decode step logits", tol)
    finally:
        dec.close()


def test_configs4_full_depth(gpu):
    """All 42 layers at the benchmark geometry.
    * A 48-token prompt and one decode step (the n = 1 GEMV path) against the
      oracle's 42-layer composition, to the model's own sensitivity
      (model_bar: the oracle rerun with its input changed in the last bit).
    * The eager pass and two replays of the captured prefill and decode graphs
      of the benchmark's 512-token prompt and 8 decode steps give
      bit-identical tokens and logits; all finite, all ids in the vocabulary."""
    dec = dm.Decoder(gpu, configs4(42), seed=0x5EED)
    try:
        prompt = np.random.default_rng(SEED + 42).integers(0, 122880, N).astype(np.uint32)
        ref = OracleDecoder(gpu, dec)
        twin = ref.twin(2.0 ** -23)
        print("\nconfigs[4] 42 layers: 48-token prompt vs the oracle", flush=True)
        nxt = dec.forward(prompt[:48])
        ref_logits = ref.forward(prompt[:48])
        tol, sens = model_bar(ref_logits, twin.forward(prompt[:48]))
        check_logits(dec.logits(), ref_logits, "42 layers, prompt of 48", tol)
        assert nxt == int(np.argmax(dec.logits()))
        dec.forward(prompt[48:49])  # one token: the decode path
        ref_logits = ref.forward(prompt[48:49])
        tol, sens = model_bar(ref_logits, twin.forward(prompt[48:49]))
        check_logits(dec.logits(), ref_logits, "42 layers, decode step 49", tol)
        del ref, twin

        runs = []
        for i in range(3):  # eager, capture + replay, replay
            print(f"configs[4] 42 layers: run {i}", flush=True)
            dec.reset()
            first = dec.forward(prompt)
            toks = dec.generate(8)
            runs.append((first, toks.copy(), dec.logits()))
        for first, toks, logits in runs[1:]:
            assert first == runs[0][0] and np.array_equal(toks, runs[0][1])
            assert_bits(logits, runs[0][2], "42-layer replayed logits")
        assert np.isfinite(runs[0][2]).all() and all(0 <= int(t) < 122880 for t in runs[0][1])
    finally:
        dec.close()
