"""The GGUF reader (llm_amd/csrc/q8_gguf.cpp) under AddressSanitizer and
UndefinedBehaviorSanitizer, on the CPU: built alone with g++ around
tests/gguf_sanitize_driver.cpp and run over the reference's fixtures, every
truncation of them (at a stride), seeded byte mutations of their headers and
written files of every metadata type.  Where test_gguf.py shows the reader
returns a status instead of crashing, this shows it also does no out-of-bounds
access to its own parsed tables (heap, instrumented) and no undefined
arithmetic on the way, and that every tensor view it hands out lies inside the
mapping (the driver reads every byte of every view: a view past the file's
end would fault).  A sanitizer report fails the run."""
import os
import shutil
import subprocess

import numpy as np
import pytest

import gguf_writer as gw

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
GOLDEN = os.path.join(HERE, "golden")
FIXTURES = [os.path.join(GOLDEN, f) for f in ("tiny_dense.gguf", "tiny_moe.gguf", "tiny_spm.gguf")]


def build_driver(out_dir: str) -> str:
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ is not installed")
    exe = os.path.join(out_dir, "gguf_sanitize")
    cmd = [gxx, "-std=c++17", "-g", "-O1", "-fsanitize=address,undefined", "-fno-omit-frame-pointer",
           "-fno-sanitize-recover=undefined", "-I", os.path.join(ROOT, "include"),
           "-I", os.path.join(ROOT, "llm_amd", "csrc"), os.path.join(ROOT, "llm_amd", "csrc", "q8_gguf.cpp"),
           os.path.join(HERE, "gguf_sanitize_driver.cpp"), "-o", exe]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert res.returncode == 0, res.stdout
    return exe


def data_start(blob: bytes) -> int:
    """The header's extent, from the reader itself (through the Python mirror)."""
    from llm_amd.gguf import GgufFile
    import tempfile
    with tempfile.NamedTemporaryFile(suffix=".gguf", delete=False) as f:
        f.write(blob)
        path = f.name
    try:
        return GgufFile.open(path).layout()["data_start"]
    finally:
        os.unlink(path)


def corpus(tmp_path) -> list[str]:
    paths = []

    def put(name: str, data: bytes):
        p = os.path.join(tmp_path, name)
        with open(p, "wb") as f:
            f.write(data)
        paths.append(p)

    rng = np.random.default_rng(0x5A17)
    for fx in FIXTURES:
        blob = open(fx, "rb").read()
        base = os.path.basename(fx)[:-5]
        put(f"{base}.gguf", blob)
        header = data_start(blob)
        # every truncation inside the header, then a stride through the data
        for n in list(range(0, header + 1)) + list(range(header, len(blob), 509)):
            put(f"{base}_cut{n}.gguf", blob[:n])
        for i in range(400):
            m = bytearray(blob)
            for _ in range(int(rng.integers(1, 6))):
                pos = int(rng.integers(4, header))
                m[pos] = int(rng.integers(0, 256)) if rng.random() < 0.5 else m[pos] ^ (1 << int(rng.integers(0, 8)))
            put(f"{base}_mut{i}.gguf", bytes(m))
    # written files: every value type, nested and empty arrays, an odd alignment
    meta = [("u8", gw.U8, 200), ("i8", gw.I8, -5), ("u16", gw.U16, 60000), ("i16", gw.I16, -300),
            ("u32", gw.U32, 4_000_000_000), ("i32", gw.I32, -7), ("f32", gw.F32, 0.1), ("b", gw.BOOL, 1),
            ("s", gw.STRING, "héllo ▁"), ("u64", gw.U64, 2 ** 63 + 5), ("i64", gw.I64, -2 ** 40),
            ("f64", gw.F64, 0.1), ("nested", gw.ARRAY, (gw.ARRAY, [(gw.U8, [1, 2]), (gw.STRING, ["a", "bc"])])),
            ("u32s", gw.ARRAY, (gw.U32, [1, 2, 0xFFFFFFFF])), ("empty", gw.ARRAY, (gw.F32, [])),
            ("general.alignment", gw.U32, 64)]
    rng_w = np.random.default_rng(7)
    blob = gw.build(meta, [{"name": "t.weight", "dims": (64, 3), "dtype": gw.T_Q8_0,
                            "data": gw.q8_bytes(3, 64, rng_w).tobytes()},
                           {"name": "n.weight", "dims": (64,), "dtype": gw.T_F32,
                            "data": np.ones(64, np.float32).tobytes()}], alignment=64)
    put("typed.gguf", blob)
    for n in range(0, len(blob), 7):
        put(f"typed_cut{n}.gguf", blob[:n])
    return paths


def test_reader_is_clean_under_address_and_ub_sanitizers(tmp_path):
    exe = build_driver(str(tmp_path))
    files = corpus(tmp_path)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    # one driver run per batch of files (the command line stays short)
    parsed = failed = 0
    for i in range(0, len(files), 400):
        res = subprocess.run([exe, *files[i:i + 400]], stdout=subprocess.PIPE, stderr=subprocess.STDOUT,
                             text=True, env=env)
        assert "Sanitizer" not in res.stdout and "runtime error" not in res.stdout, res.stdout[-4000:]
        assert res.returncode == 0, res.stdout[-4000:]
        parsed += res.stdout.count(" parsed\n")
        failed += res.stdout.count(" status ")
    print(f"{len(files)} files: {parsed} parsed, {failed} refused with a status")
    assert parsed >= len(FIXTURES) + 1 and failed > 0
