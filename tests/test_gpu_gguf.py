"""GPU tests of the ingestion path: Q8_0 tensors memory-mapped from GGUF files
go to the device and through the kernels unchanged, and the embedding lookup
dequantizes rows of the resident copy bit-exactly.

  * GGUF -> resident weight -> GEMV / GEMM: the same bar as the in-memory
    weights (parity against the CPU oracle on the same bytes; bit-exact with
    gemv.exact = 1), including K = 5760 rows (6120-byte strides);
  * q8_gguf_weight (C path) and weight() + residency (Python path) resolve to
    the same resident copy, keyed by the map address (tensor.rs:40-42);
  * embeddings: out[t] == dequant_q8_0(row tokens[t]) bit for bit
    (quant.rs:184-203, gpu.cu:1754-1766), any offset, repeated ids, and the
    vocabulary check before any launch (model.rs:741-751).
"""
import numpy as np
import pytest

import gguf_writer as gw
import oracle
from llm_amd import q8
from llm_amd.gguf import GgufFile, weight
from test_gpu_q8 import assert_bits, assert_close, assert_parity, exact_matmul

pytestmark = pytest.mark.gpu

SEED = 0x5EED
HIDDEN, FFN, VOCAB = 2304, 5760, 4000


@pytest.fixture(scope="module")
def gpu():
    g = q8.Gpu(0)
    yield g
    g.close()


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    """A GGUF with the benchmark's projection shapes as Q8_0 tensors (dims
    [k, out]) and a tied token embedding / output matrix."""
    r = np.random.default_rng(SEED)
    tensors, raw = [], {}
    for name, k, out in [("token_embd.weight", HIDDEN, VOCAB), ("blk.0.ffn_up.weight", HIDDEN, FFN),
                         ("blk.0.ffn_down.weight", FFN, HIDDEN), ("blk.0.attn_output.weight", HIDDEN, HIDDEN)]:
        data = gw.q8_bytes(out, k, r)
        raw[name] = (data, k, out)
        tensors.append({"name": name, "dims": [k, out], "dtype": gw.T_Q8_0, "data": data.tobytes()})
    norm = {"name": "output_norm.weight", "dims": [HIDDEN], "dtype": gw.T_F32,
            "data": np.ones(HIDDEN, np.float32).tobytes()}
    meta = [("general.architecture", gw.STRING, "llama"), ("llama.embedding_length", gw.U32, HIDDEN),
            ("llama.vocab_size", gw.U32, VOCAB)]
    path = gw.write(tmp_path_factory.mktemp("gguf") / "model.gguf", meta, [tensors[0], norm] + tensors[1:])
    print(f"\nmodel gguf: {path}", flush=True)
    return GgufFile.open(path), raw


@pytest.mark.parametrize("name", ["blk.0.ffn_up.weight", "blk.0.ffn_down.weight", "blk.0.attn_output.weight"])
def test_gguf_weight_gemv_matches_the_oracle(gpu, model, name):
    g, raw = model
    data, k, out = raw[name]
    w = weight(g, name, k, out)
    np.testing.assert_array_equal(w.data, data)
    x = np.random.default_rng(SEED + 1).standard_normal(k).astype(np.float32)
    ref = oracle.matmul(data, k, out, x, 1).reshape(-1)
    c = q8.Compute(gpu)
    xb, yb = c.alloc(k), c.alloc(out)
    c.upload(xb, x)
    y = np.empty(out, np.float32)
    c.matmul(w, xb, 0, 1, yb, 0)
    c.download(yb, y)
    assert_close(y, ref, f"{name} n=1")
    gpu.set_option("gemv.exact", 1)
    try:
        c.matmul(w, xb, 0, 1, yb, 0)
        c.download(yb, y)
    finally:
        gpu.set_option("gemv.exact", -1)
    if oracle.simd_path() == "avx2+fma":
        assert_bits(y, ref, f"{name} n=1 exact")
    else:
        assert_close(y, ref, f"{name} n=1 exact")


def test_gguf_weight_gemm_matches_the_oracle(gpu, model):
    g, raw = model
    data, k, out = raw["blk.0.ffn_down.weight"]
    n = 64
    w = weight(g, "blk.0.ffn_down.weight", k, out)
    x = np.random.default_rng(SEED + 2).standard_normal((n, k)).astype(np.float32)
    ref = oracle.matmul(data, k, out, x.reshape(-1), n)
    c = q8.Compute(gpu)
    xb, yb = c.alloc(n * k), c.alloc(n * out)
    c.upload(xb, x)
    y = np.empty((n, out), np.float32)
    c.matmul(w, xb, 0, n, yb, 0)
    c.download(yb, y)
    assert_parity(y, ref, exact_matmul(data, k, out, x, n), "gguf down n=64")


def test_c_path_and_python_path_share_one_resident_copy(gpu, model):
    g, raw = model
    data, k, out = raw["blk.0.attn_output.weight"]
    h_c = gpu.gguf_weight(g, "blk.0.attn_output.weight", k, out)
    h_py = gpu.resident(weight(g, "blk.0.attn_output.weight", k, out))
    assert h_c == h_py
    np.testing.assert_array_equal(gpu.export(weight(g, "blk.0.attn_output.weight", k, out)), data)
    with pytest.raises(q8.Q8Error) as e:
        gpu.gguf_weight(g, "blk.0.attn_output.weight", out + 32, k)
    assert e.value.status == q8.Q8_ERR_FORMAT
    with pytest.raises(q8.Q8Error) as e:
        gpu.gguf_weight(g, "output_norm.weight", HIDDEN, 1)
    assert e.value.status in (q8.Q8_ERR_FORMAT, q8.Q8_ERR_UNSUPPORTED)


def dequant_rows(data, k, tokens):
    rows = np.asarray(data, np.uint8).reshape(-1, k // 32 * 34)
    return np.stack([oracle.dequant_q8_0(rows[t], k) for t in tokens]) if len(tokens) else np.zeros((0, k))


@pytest.mark.parametrize("tokens,offset", [([0], 0), ([VOCAB - 1, 0, 17, 17, 31, 32, 33], 0),
                                           (list(range(0, VOCAB, 97)), 5), ([3999] * 3, 2304 + 1)])
def test_embeddings_are_dequantized_rows_bit_for_bit(gpu, model, tokens, offset):
    g, raw = model
    data, k, vocab = raw["token_embd.weight"]
    w = weight(g, "token_embd.weight", k, vocab)
    c = q8.Compute(gpu)
    n = len(tokens)
    sentinel = np.full(offset + n * k + 7, -3.5, np.float32)
    out = c.alloc(sentinel.size)
    c.upload(out, sentinel)
    c.embeddings(w, tokens, out, offset)
    got = np.empty(sentinel.size, np.float32)
    c.download(out, got)
    assert_bits(got[offset:offset + n * k], dequant_rows(data, k, tokens).reshape(-1), f"embeddings {tokens[:4]}")
    assert (got[:offset] == -3.5).all() and (got[offset + n * k:] == -3.5).all()


def test_embedding_vocabulary_check_and_empty_prompt(gpu, model):
    g, raw = model
    data, k, vocab = raw["token_embd.weight"]
    w = weight(g, "token_embd.weight", k, vocab)
    c = q8.Compute(gpu)
    out = c.alloc(2 * k)
    c.upload(out, np.zeros(2 * k, np.float32))
    with pytest.raises(q8.Q8Error) as e:
        c.embeddings(w, [1, vocab], out, 0)
    assert e.value.status == q8.Q8_ERR_INVALID and "outside vocabulary" in e.value.message
    c.embeddings(w, [], out, 0)
    with pytest.raises(q8.Q8Error) as e:
        c.embeddings(w, [1, 2], out, 1)  # one float past the buffer
    assert e.value.status == q8.Q8_ERR_INVALID
    got = np.empty(2 * k, np.float32)
    c.download(out, got)
    assert not got.any()  # nothing was launched by the rejected calls


def test_tied_embedding_is_also_the_lm_head(gpu, model):
    """model.rs:519-524: without output.weight the embedding matrix is the
    lm_head; one resident copy serves both the lookup and the argmax GEMV."""
    g, raw = model
    data, k, vocab = raw["token_embd.weight"]
    w = weight(g, "token_embd.weight", k, vocab)
    c = q8.Compute(gpu)
    xb, logits = c.alloc(k), c.alloc(vocab)
    c.embeddings(w, [123], xb, 0)
    x = dequant_rows(data, k, [123]).reshape(-1).astype(np.float32)
    ref = oracle.matmul(data, k, vocab, x, 1).reshape(-1)
    exact = oracle.simd_path() == "avx2+fma"
    gpu.set_option("gemv.exact", 1 if exact else -1)
    try:
        top = gpu.lm_head_argmax(w, xb, 0, logits, 0)
    finally:
        gpu.set_option("gemv.exact", -1)
    y = np.empty(vocab, np.float32)
    c.download(logits, y)
    (assert_bits if exact else assert_close)(y, ref, "tied lm_head")
    assert top == oracle.argmax(ref)
