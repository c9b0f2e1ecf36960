"""CPU tests of the GGUF reader (include/q8gguf.h, llm_amd/gguf.py) -- the
ingestion side of the Q8_0 path (apps/engine/src/gguf.rs, model.rs:1670-1684).

Pinned against:
  * the reference's own fixtures (tests/golden/*.gguf, copied as data from
    tests/fixtures/): their metadata and tensor tables are the constants of
    the scripts that wrote them (scripts/make_tiny_moe.py:24-35,95-143;
    scripts/make_tiny_spm.py:16-30,80-92), and their tensor bytes are
    regenerated here from the same seeded generator (numpy default_rng(0x5EED),
    make_tiny_moe.py:95-120) -- an independent check of offsets, alignment
    and the [k, out] dims convention;
  * files written by tests/gguf_writer.py for every metadata type, the
    alignment rule and each error the reference raises.
"""
import os

import numpy as np
import pytest

import gguf_writer as gw
import oracle
from llm_amd import q8
from llm_amd.gguf import DType, GgufFile, weight

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DENSE = os.path.join(GOLDEN, "tiny_dense.gguf")
MOE = os.path.join(GOLDEN, "tiny_moe.gguf")
SPM = os.path.join(GOLDEN, "tiny_spm.gguf")

# make_tiny_moe.py:24-35
EMBD, HEADS, HEADS_KV, HEAD_DIM, FF, EXPERTS, USED, VOCAB, LAYERS = 32, 4, 2, 8, 32, 4, 2, 64, 2
EPS, ROPE_BASE, SEED = 1e-5, 10_000.0, 0x5EED


def regenerate():
    """The fixture's tensors, in the generator's draw order (make_tiny_moe.py:95-120)."""
    rng = np.random.default_rng(SEED)

    def matrix(k, out):
        return (rng.standard_normal((out, k)) * 0.2).astype(np.float32)

    def norm():
        return (1.0 + rng.standard_normal(EMBD) * 0.02).astype(np.float32)

    layers = []
    for _ in range(LAYERS):
        layer = {"attn_norm": norm(), "attn_q": matrix(EMBD, EMBD), "attn_k": matrix(EMBD, HEADS_KV * HEAD_DIM),
                 "attn_v": matrix(EMBD, HEADS_KV * HEAD_DIM), "attn_output": matrix(EMBD, EMBD)}
        layer["ffn_norm"] = norm()
        layer["ffn_gate"] = matrix(EMBD, FF)
        layer["ffn_up"] = matrix(EMBD, FF)
        layer["ffn_down"] = matrix(FF, EMBD)
        layers.append(layer)
    token_embd = matrix(EMBD, VOCAB)
    output = matrix(EMBD, VOCAB)
    return {"token_embd": token_embd, "output": output, "output_norm": norm(), "layers": layers}


def dense_table(model):
    """(name, dims, array) in file order (make_tiny_moe.py:122-143)."""
    t = [("token_embd.weight", (EMBD, VOCAB), model["token_embd"]),
         ("output_norm.weight", (EMBD,), model["output_norm"]),
         ("output.weight", (EMBD, VOCAB), model["output"])]
    for i, layer in enumerate(model["layers"]):
        p = f"blk.{i}"
        t += [(f"{p}.attn_norm.weight", (EMBD,), layer["attn_norm"]),
              (f"{p}.attn_q.weight", (EMBD, EMBD), layer["attn_q"]),
              (f"{p}.attn_k.weight", (EMBD, HEADS_KV * HEAD_DIM), layer["attn_k"]),
              (f"{p}.attn_v.weight", (EMBD, HEADS_KV * HEAD_DIM), layer["attn_v"]),
              (f"{p}.attn_output.weight", (EMBD, EMBD), layer["attn_output"]),
              (f"{p}.ffn_norm.weight", (EMBD,), layer["ffn_norm"]),
              (f"{p}.ffn_gate.weight", (EMBD, FF), layer["ffn_gate"]),
              (f"{p}.ffn_up.weight", (EMBD, FF), layer["ffn_up"]),
              (f"{p}.ffn_down.weight", (FF, EMBD), layer["ffn_down"])]
    return t


def status_of(fn, *args):
    with pytest.raises(q8.Q8Error) as e:
        fn(*args)
    return e.value.status, e.value.message


# ---- the reference's fixtures ----

def test_dense_fixture_metadata_is_the_generators():
    g = GgufFile.open(DENSE)
    assert g.layout() == {"version": 3, "alignment": 32, "data_start": 1728, "file_bytes": 67904}
    assert g.meta_str("general.architecture") == "llama"
    assert g.meta_str("general.name") == "tiny"
    for key, value in [("block_count", LAYERS), ("embedding_length", EMBD), ("feed_forward_length", FF),
                       ("attention.head_count", HEADS), ("attention.head_count_kv", HEADS_KV),
                       ("attention.key_length", HEAD_DIM), ("rope.dimension_count", HEAD_DIM),
                       ("vocab_size", VOCAB)]:
        assert g.meta_u64(f"llama.{key}") == value
    assert g.meta_f32("llama.rope.freq_base") == np.float32(ROPE_BASE)
    assert g.meta_f32("llama.attention.layer_norm_rms_epsilon") == np.float32(EPS)
    assert not g.has_key_prefix("llama.expert")
    assert g.has_key_prefix("llama.rope.")
    assert g.meta_u64_opt("llama.expert_count") is None
    assert g.meta_u64_opt("general.name") is None  # a string is not an integer
    assert g.meta_f32_opt("llama.block_count") is None


def test_dense_fixture_tensor_table_and_bytes_are_the_generators():
    g = GgufFile.open(DENSE)
    table = dense_table(regenerate())
    infos = g.tensors()
    assert [t.name for t in infos] == [name for name, _, _ in table]
    offset = 0
    for info, (name, dims, array) in zip(infos, table):
        assert info.dims == dims and info.dtype == DType.F32
        assert info.offset == offset  # 32-aligned running offset (make_tiny_moe.py:66-75)
        assert info.byte_len == array.nbytes == 4 * info.elements()
        data = g.data(name)
        assert not data.flags.writeable
        np.testing.assert_array_equal(data.view(np.float32), array.reshape(-1))
        offset = (offset + array.nbytes + 31) // 32 * 32
        # row-major out x k under GGUF dims [k, out]
        if len(dims) == 2:
            assert array.shape == (dims[1], dims[0])


def test_moe_fixture_reads_three_dimensional_expert_stacks():
    g = GgufFile.open(MOE)
    model = regenerate()
    assert g.meta_u64("llama.expert_count") == EXPERTS
    assert g.meta_u64("llama.expert_used_count") == USED
    assert g.meta_u64("llama.expert_feed_forward_length") == FF
    assert g.has_key_prefix("llama.expert")
    for i, layer in enumerate(model["layers"]):
        gate = g.tensor(f"blk.{i}.ffn_gate_exps.weight")
        assert gate.dims == (EMBD, FF, EXPERTS) and gate.byte_len == EMBD * FF * EXPERTS * 4
        stack = g.data(f"blk.{i}.ffn_gate_exps.weight").view(np.float32).reshape(EXPERTS, FF, EMBD)
        for e in range(EXPERTS):
            np.testing.assert_array_equal(stack[e], layer["ffn_gate"])
        down = g.data(f"blk.{i}.ffn_down_exps.weight").view(np.float32).reshape(EXPERTS, EMBD, FF)
        np.testing.assert_array_equal(down[1], layer["ffn_down"])
        router = g.data(f"blk.{i}.ffn_gate_inp.weight").view(np.float32)
        assert router.shape == (EMBD * EXPERTS,) and not router.any()
    np.testing.assert_array_equal(g.data("token_embd.weight").view(np.float32), model["token_embd"].reshape(-1))


def test_spm_fixture_arrays_decode_from_the_map():
    g = GgufFile.open(SPM)
    # make_tiny_spm.py:20-30: <unk>, <s>, </s>, then every prefix of each word
    pieces, scores = ["<unk>", "<s>", "</s>"], [0.0, 0.0, 0.0]
    for word in ("hello", "world"):
        for n in range(1, len(word) + 1):
            pieces.append("▁" + word[:n])
            scores.append(float(n))
    assert g.meta_str_array("tokenizer.ggml.tokens") == pieces
    np.testing.assert_array_equal(g.meta_f32_array("tokenizer.ggml.scores"), np.array(scores, np.float32))
    np.testing.assert_array_equal(g.meta_i32_array("tokenizer.ggml.token_type"),
                                  np.array([2, 3, 3] + [1] * (len(pieces) - 3), np.int32))
    assert g.meta_u64("tokenizer.ggml.bos_token_id") == 1
    assert g.meta_u64("tokenizer.ggml.eos_token_id") == 2
    assert g.meta_str("tokenizer.chat_template") == "[INST] {{ messages }} [/INST]"
    assert g.tensors() == []
    assert g.meta_type("tokenizer.ggml.tokens") == (gw.ARRAY, gw.STRING, len(pieces))
    # add_space_prefix is written as u32 (make_tiny_spm.py:88): not a bool
    status, msg = status_of(g.meta_bool, "tokenizer.ggml.add_space_prefix")
    assert status == q8.Q8_ERR_FORMAT and "is not a bool" in msg
    assert g.meta_u64("tokenizer.ggml.add_space_prefix") == 1
    # wrong array kinds
    assert status_of(g.meta_f32_array, "tokenizer.ggml.tokens")[0] == q8.Q8_ERR_FORMAT
    assert status_of(g.meta_str_array, "tokenizer.ggml.scores")[0] == q8.Q8_ERR_FORMAT
    assert status_of(g.meta_i32_array, "general.name")[1].endswith("is not an array")
    assert status_of(g.meta_str, "tokenizer.ggml.nope")[0] == q8.Q8_ERR_MISSING


def test_every_truncation_of_a_fixture_is_a_format_error():
    """No tensors: the data section (aligned to 32) must still exist
    (make_tiny_spm.py:77-79): 778 header bytes -> data start 800."""
    blob = open(SPM, "rb").read()
    assert GgufFile.open(SPM).layout()["data_start"] == 800
    import tempfile
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "cut.gguf")
        for n in list(range(0, 800, 7)) + [777, 778, 779, 799, 800, 801]:
            with open(p, "wb") as f:
                f.write(blob[:n])
            if n >= 800:
                assert GgufFile.open(p).layout()["data_start"] == 800
                continue
            status, msg = status_of(GgufFile.open, p)
            assert status == q8.Q8_ERR_FORMAT, (n, msg)
            assert ("unexpected end of file" in msg or "past end of file" in msg or "bad magic" in msg), (n, msg)


def _read_everything(g):
    """Every accessor over every key and tensor; errors are allowed, crashes are not."""
    for key in g.keys():
        kind = g.meta_type(key)
        for fn in (g.meta_u64, g.meta_f32, g.meta_bool, g.meta_str, g.meta_i32_array, g.meta_f32_array,
                   g.meta_str_array):
            try:
                fn(key)
            except (q8.Q8Error, ValueError, UnicodeDecodeError):
                pass
        assert kind is not None
    for t in g.tensors():
        try:
            d = g.data(t.name)
            assert d.size * d.itemsize == t.byte_len
        except q8.Q8Error:
            pass


@pytest.mark.parametrize("fixture", [SPM, DENSE])
def test_random_header_mutations_parse_or_fail_cleanly(tmp_path, fixture):
    """Seeded byte mutations of the header (metadata and tensor table): each
    file either parses -- and then every key, array and tensor view reads
    back inside the mapping -- or fails with a status, never a crash."""
    blob = open(fixture, "rb").read()
    header = GgufFile.open(fixture).layout()["data_start"]
    rng = np.random.default_rng(0x6775)
    path = os.path.join(tmp_path, "m.gguf")
    outcomes = {}
    for i in range(600):
        m = bytearray(blob)
        for _ in range(int(rng.integers(1, 5))):
            pos = int(rng.integers(4, header))  # past the magic: the interesting part
            m[pos] = int(rng.integers(0, 256)) if rng.random() < 0.5 else m[pos] ^ (1 << int(rng.integers(0, 8)))
        with open(path, "wb") as f:
            f.write(m)
        try:
            g = GgufFile.open(path)
        except q8.Q8Error as e:
            # EngineError::Format / Io / MissingTensor, or Unsupported for an unknown tensor type id
            assert e.status in (q8.Q8_ERR_FORMAT, q8.Q8_ERR_IO, q8.Q8_ERR_MISSING, q8.Q8_ERR_UNSUPPORTED), \
                (i, e.status, e.message)
            outcomes["error"] = outcomes.get("error", 0) + 1
            continue
        _read_everything(g)
        del g
        outcomes["parsed"] = outcomes.get("parsed", 0) + 1
    print(outcomes)
    assert outcomes.get("error", 0) > 0 and outcomes.get("parsed", 0) > 0


# ---- written files: value types, layout rules ----

ALL_TYPES = [("u8", gw.U8, 200), ("i8", gw.I8, -5), ("u16", gw.U16, 60000), ("i16", gw.I16, -300),
             ("u32", gw.U32, 4_000_000_000), ("i32", gw.I32, -7), ("f32", gw.F32, 0.1), ("b", gw.BOOL, 1),
             ("s", gw.STRING, "héllo ▁ \U0001f600"), ("u64", gw.U64, 2 ** 63 + 5), ("i64", gw.I64, -2 ** 40),
             ("f64", gw.F64, 0.1), ("ipos", gw.I64, 12), ("nested", gw.ARRAY, (gw.ARRAY, [(gw.U8, [1, 2]),
                                                                                         (gw.STRING, ["a", "bc"])])),
             ("u32s", gw.ARRAY, (gw.U32, [1, 2, 0xFFFFFFFF])), ("empty", gw.ARRAY, (gw.F32, [])),
             ("after", gw.U32, 99)]


def test_every_metadata_type_reads_as_the_reference_types_it(tmp_path):
    g = GgufFile.open(gw.write(tmp_path / "t.gguf", ALL_TYPES))
    assert g.keys() == [k for k, _, _ in ALL_TYPES]
    for key in ("u8", "u16", "u32", "u64"):
        assert g.meta_u64(key) == dict((k, v) for k, _, v in ALL_TYPES)[key]
    assert g.meta_u64("ipos") == 12  # a signed value >= 0 is accepted (gguf.rs:196)
    for key in ("i8", "i16", "i32", "i64"):
        status, msg = status_of(g.meta_u64, key)
        assert status == q8.Q8_ERR_FORMAT and "not an unsigned integer" in msg
    assert g.meta_f32("f32") == np.float32(0.1)
    assert g.meta_f32("f64") == np.float32(0.1)  # f64 rounded to f32
    assert status_of(g.meta_f32, "u8")[0] == q8.Q8_ERR_FORMAT
    assert g.meta_bool("b") is True
    assert status_of(g.meta_bool, "u8")[0] == q8.Q8_ERR_FORMAT
    assert g.meta_str("s") == "héllo ▁ \U0001f600"
    assert status_of(g.meta_str, "u8")[1].endswith("is not a string")
    np.testing.assert_array_equal(g.meta_i32_array("u32s"), np.array([1, 2, -1], np.int32))
    assert g.meta_f32_array("empty").size == 0
    assert g.meta_type("nested") == (gw.ARRAY, gw.ARRAY, 2)
    assert g.meta_u64("after") == 99  # the nested array was skipped exactly
    assert status_of(g.meta_u64, "missing") == (q8.Q8_ERR_MISSING, "missing metadata key: missing")


def test_repeated_key_keeps_the_last_value_and_repeated_tensor_the_first(tmp_path):
    t1 = {"name": "w", "dims": [4], "dtype": gw.T_F32, "data": np.arange(4, dtype=np.float32).tobytes()}
    t2 = {"name": "w", "dims": [8], "dtype": gw.T_F32, "data": np.ones(8, np.float32).tobytes()}
    g = GgufFile.open(gw.write(tmp_path / "t.gguf", [("k", gw.U32, 1), ("j", gw.U8, 2), ("k", gw.U32, 3)],
                               [t1, t2]))
    assert g.meta_u64("k") == 3 and g.keys() == ["k", "j"]
    assert g.tensor("w").dims == (4,)
    assert [t.dims for t in g.tensors()] == [(4,), (8,)]
    np.testing.assert_array_equal(g.data("w").view(np.float32), np.arange(4, dtype=np.float32))


@pytest.mark.parametrize("kind,expect", [(gw.U32, 64), (gw.U64, 64), (gw.U8, 64), (gw.I32, 32)])
def test_alignment_is_taken_only_from_an_unsigned_value(tmp_path, kind, expect):
    """gguf.rs:150-153: a signed general.alignment falls back to 32."""
    t = {"name": "w", "dims": [32], "dtype": gw.T_F32, "data": np.arange(32, dtype=np.float32).tobytes()}
    p = gw.write(tmp_path / "t.gguf", [("general.alignment", kind, 64)], [t], alignment=expect)
    g = GgufFile.open(p)
    lay = g.layout()
    assert lay["alignment"] == expect and lay["data_start"] % expect == 0
    np.testing.assert_array_equal(g.data("w").view(np.float32), np.arange(32, dtype=np.float32))


def test_q8_0_tensor_view_and_weight_identity(tmp_path):
    r = np.random.default_rng(3)
    k, out = 96, 40
    data = gw.q8_bytes(out, k, r)
    t = {"name": "blk.0.ffn_up.weight", "dims": [k, out], "dtype": gw.T_Q8_0, "data": data.tobytes()}
    f16 = {"name": "h", "dims": [6], "dtype": gw.T_F16, "data": np.arange(6, dtype=np.float16).tobytes()}
    g = GgufFile.open(gw.write(tmp_path / "q.gguf", [("general.architecture", gw.STRING, "llama")], [f16, t]))
    info = g.tensor("blk.0.ffn_up.weight")
    assert info.dtype == DType.Q8_0 and info.byte_len == out * k // 32 * 34 and info.elements() == out * k
    assert g.tensor("h").byte_len == 12
    w = weight(g, "blk.0.ffn_up.weight", k, out)
    np.testing.assert_array_equal(w.data, data)
    # the identity is the place in the map, stable across lookups (tensor.rs:40-42)
    assert w.identity() == weight(g, "blk.0.ffn_up.weight", k, out).identity()
    assert w.identity()[0] == g.data_address("blk.0.ffn_up.weight")
    # the oracle reads the mapped bytes as it reads a heap copy of them
    x = r.standard_normal(k).astype(np.float32)
    y = oracle.matmul(w.data, k, out, x, 1)
    assert y.shape == (1, out)
    np.testing.assert_array_equal(y.view(np.uint32), oracle.matmul(data.copy(), k, out, x, 1).view(np.uint32))
    status, msg = status_of(weight, g, "blk.0.ffn_up.weight", out, k)
    assert status == q8.Q8_ERR_FORMAT and msg.endswith(f"has shape [{k}, {out}], expected [{out}, {k}]")
    assert status_of(weight, g, "h", 6, 1)[0] == q8.Q8_ERR_FORMAT
    assert status_of(weight, g, "nope", 1, 1) == (q8.Q8_ERR_MISSING, "missing tensor: nope")


def test_a_view_keeps_the_file_mapped(tmp_path):
    t = {"name": "w", "dims": [32], "dtype": gw.T_F32, "data": np.arange(32, dtype=np.float32).tobytes()}
    g = GgufFile.open(gw.write(tmp_path / "t.gguf", [], [t]))
    view = g.data("w")
    del g
    import gc
    gc.collect()
    np.testing.assert_array_equal(view.view(np.float32), np.arange(32, dtype=np.float32))


# ---- errors (gguf.rs and the reference's EngineError kinds) ----

def _t(**kw):
    base = {"name": "w", "dims": [32], "dtype": gw.T_F32, "data": bytes(128)}
    base.update(kw)
    return base


@pytest.mark.parametrize("case,status,needle", [
    ("magic", q8.Q8_ERR_FORMAT, "bad magic 0x46554746"),
    ("version1", q8.Q8_ERR_FORMAT, "unsupported version 1"),
    ("version4", q8.Q8_ERR_FORMAT, "unsupported version 4"),
    ("meta_type", q8.Q8_ERR_FORMAT, "unknown metadata value type 13"),
    ("array_elem", q8.Q8_ERR_FORMAT, "unknown array element type 13"),
    ("dtype", q8.Q8_ERR_UNSUPPORTED, "tensor type id 2"),
    ("blocks", q8.Q8_ERR_FORMAT, "is not a multiple of the 32 block size"),
    ("past_end", q8.Q8_ERR_FORMAT, "tensor w runs past end of file"),
    ("offset_wrap", q8.Q8_ERR_FORMAT, "tensor w runs past end of file"),
    ("dims_overflow", q8.Q8_ERR_FORMAT, "element count overflows"),
    ("utf8_key", q8.Q8_ERR_FORMAT, "invalid utf-8 in string"),
    ("utf8_array", q8.Q8_ERR_FORMAT, "invalid utf-8 in string"),
    ("surrogate", q8.Q8_ERR_FORMAT, "invalid utf-8 in string"),
    ("zero_alignment", q8.Q8_ERR_FORMAT, "general.alignment is 0"),
    ("too_many_kv", q8.Q8_ERR_FORMAT, "unexpected end of file"),
    ("huge_array", q8.Q8_ERR_FORMAT, "unexpected end of file"),
    ("deep_nesting", q8.Q8_ERR_FORMAT, "nested too deeply"),
    ("empty", q8.Q8_ERR_FORMAT, "unexpected end of file"),
])
def test_malformed_files_fail_with_the_reference_error_kind(tmp_path, case, status, needle):
    import struct
    meta, tensors, kw = [("general.name", gw.STRING, "x")], [_t()], {}
    if case == "magic":
        kw["magic"] = 0x46554746
    elif case == "version1":
        kw["version"] = 1
    elif case == "version4":
        kw["version"] = 4
    elif case == "meta_type":
        meta.append(("bad", ("raw", 13), b""))
    elif case == "array_elem":
        meta.append(("bad", ("raw", gw.ARRAY), struct.pack("<IQ", 13, 1)))
    elif case == "dtype":
        tensors = [_t(dtype=2)]
    elif case == "blocks":
        tensors = [_t(dtype=gw.T_Q8_0, dims=[33], data=b"")]
    elif case == "past_end":
        tensors = [_t(offset=64, data=b"")]
    elif case == "offset_wrap":
        tensors = [_t(offset=2 ** 64 - 64, data=b"")]
    elif case == "dims_overflow":
        tensors = [_t(dims=[2 ** 33, 2 ** 33], data=b"")]
    elif case == "utf8_key":
        meta.append((b"\xff", gw.U8, 1))
    elif case == "utf8_array":
        meta.append(("arr", ("raw", gw.ARRAY), struct.pack("<IQ", gw.STRING, 2) + gw.enc_str("ok") + gw.enc_str(b"\xc0\x80")))
    elif case == "surrogate":
        meta.append(("s", ("raw", gw.STRING), gw.enc_str(b"\xed\xa0\x80")))
    elif case == "zero_alignment":
        meta.append(("general.alignment", gw.U32, 0))
    elif case == "too_many_kv":
        kw["kv_count"] = 5
        tensors = []
    elif case == "huge_array":
        meta.append(("big", ("raw", gw.ARRAY), struct.pack("<IQ", gw.U64, 2 ** 62)))
    elif case == "deep_nesting":
        payload = b""
        for _ in range(80):
            payload = struct.pack("<IQ", gw.ARRAY, 1) + payload
        meta.append(("deep", ("raw", gw.ARRAY), payload + struct.pack("<IQ", gw.U8, 0)))
    p = tmp_path / "bad.gguf"
    if case == "empty":
        p.write_bytes(b"")
    else:
        gw.write(p, meta, tensors, **kw)
    got, msg = status_of(GgufFile.open, str(p))
    assert got == status, msg
    assert needle in msg, msg


def test_missing_file_is_an_io_error(tmp_path):
    status, msg = status_of(GgufFile.open, str(tmp_path / "absent.gguf"))
    assert status == q8.Q8_ERR_IO and msg.startswith("io error:")
