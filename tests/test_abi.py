"""CPU checks of the C-ABI library: it loads, exports exactly what
include/*.h declare, carries its build identity, and its host logic (the
tactic table, argument validation before any device work) behaves."""
import glob
import json
import os
import re
import subprocess

import pytest

import llm_amd
from llm_amd import q8

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(ROOT, "include", "*.h")))


def header_functions() -> set[str]:
    names = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(header).read(), flags=re.S)
        names |= set(re.findall(r"\b(q8_[a-z0-9_]+)\s*\(", text))
    return names


def library_exports() -> set[str]:
    out = subprocess.run(["nm", "-D", "--defined-only", q8.library_path()], stdout=subprocess.PIPE,
                         text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_library_loads():
    assert q8.lib() is not None


def test_a_missing_library_fails_loudly(tmp_path):
    """Without libq8mi.so the package raises on first use: there is no CPU
    fallback for the matmul path (run in a fresh interpreter, so this
    process keeps its loaded library)."""
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "from llm_amd import q8\n"
        "q8.LIB_PATH = %r\n"
        "q8._lib = None\n"
        "try:\n"
        "    q8.Gpu(0)\n"
        "except RuntimeError as e:\n"
        "    print('raised:', e)\n"
        "    sys.exit(0)\n"
        "sys.exit(3)\n"
    ) % (ROOT, str(tmp_path / "libq8mi.so"))
    res = subprocess.run(["python3", "-c", code], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert res.returncode == 0, res.stdout
    assert "is missing" in res.stdout and "no CPU fallback" in res.stdout


def test_every_declared_function_is_exported():
    declared = header_functions()
    exported = library_exports()
    assert declared, "no declarations parsed from the header"
    missing = declared - exported
    assert not missing, f"declared but not exported: {sorted(missing)}"
    extra = {s for s in exported if s.startswith("q8_")} - declared
    assert not extra, f"exported but not declared: {sorted(extra)}"
    assert declared == set(q8.EXPORTS)


def test_build_identity_names_its_artifact():
    info = json.loads(llm_amd.build_info())
    assert info["arch"] == "gfx950"
    assert len(info["code_object_sha256"]) == 64
    assert len(info["kernel_source_sha256"]) == 64
    for k in ("q8_repack", "q8_quantize", "q8_gemm_s1_t4", "q8_gemv_pb5_e1", "q8_argmax", "q8_silu_mul"):
        assert k in info["kernels"]
    assert "-ffp-contract=off" in info["hipcc_flags"]


def test_status_strings():
    L = q8.lib()
    for code in range(9):
        assert L.q8_status_string(code).decode() != "unknown status"
    assert L.q8_status_string(0).decode() == "ok"


def test_open_without_a_device_fails_cleanly():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU driver is present")
    with pytest.raises(q8.Q8Error) as err:
        q8.Gpu(0)
    assert err.value.status == q8.Q8_ERR_NO_DEVICE


# ---- tactic table invariants (the reference's, tactics.rs:453-501) ----

def test_tactic_table_invariants():
    rows = llm_amd.tactic_table()
    assert rows
    for row in rows:
        assert len(row["evidence"]) > 40, row["name"]
        if row["maturity"] != 0:
            assert row["rank"] > 0, row["name"]
    names = [r["name"] for r in rows]
    assert len(names) == len(set(names))


@pytest.mark.parametrize("out,k,rows,loads", [(2304, 2304, 16, 3), (2304, 5760, 16, 6), (5760, 2304, 8, 2),
                                              (4096, 4096, 8, 2), (6912, 2304, 16, 3), (4096, 8192, 32, 0),
                                              (122880, 2304, 32, 0), (64, 12288, 32, 0)])
def test_plan_row_slices_follow_the_measured_rule(out, k, rows, loads):
    """Single-matrix GEMVs with fewer 32-row tiles than CUs run in row
    slices: 8 rows at two loads per lane where 16-row slices would already
    fill the CUs and every 8-row workgroup is resident at once, else 16 rows
    (three loads per lane when K fits 16 waves, else six); the lm_head and K
    beyond 16 waves keep the tile kernel."""
    t = llm_amd.plan(1, out, k)
    assert (t["row_slice"], t["slice_loads"]) == (rows, loads)


@pytest.mark.parametrize("n,out,k", [(1, 5760, 2304), (1, 122880, 2304), (1, 2304, 5760), (1, 4, 32),
                                     (1, 33, 96), (1, 100, 11520), (1, 8000, 16384), (2, 64, 64),
                                     (8, 5760, 2304), (64, 5760, 2304), (512, 11520, 2304), (512, 2304, 5760),
                                     (1024, 2304, 5760)])
def test_plan_never_selects_a_rejected_tactic(n, out, k):
    rejected = {r["name"] for r in llm_amd.tactic_table() if r["maturity"] == 0}
    t = llm_amd.plan(n, out, k)
    assert t["name"] not in rejected
    if n == 1:
        assert t["kernel"] == q8.KERNEL_GEMV
        nb = k // 32
        npairs = (nb + 1) // 2
        assert 1 <= t["pairs_per_wave"] <= 12
        assert t["waves_per_tile"] * 64 <= (512 if t["pairs_per_batch"] == 9 else 1024)
        assert t["pairs_per_batch"] in (2, 3, 5, 9)
        s = t["kslices"]
        pps = -(-npairs // s)
        assert 1 <= s <= npairs and (s - 1) * pps < npairs  # no empty slice
        assert t["waves_per_tile"] * t["pairs_per_wave"] >= pps
        # row slices: a workgroup per 8 or 16 rows, at most 16 waves over K
        assert t["row_slice"] in (8, 16, 32)
        if t["row_slice"] != 32:
            assert t["slice_loads"] in ((2, 3, 6) if t["row_slice"] == 8 else (3, 6))
            blocks_per_wave = t["slice_loads"] * 64 // (2 * t["row_slice"])
            waves = -(-nb // blocks_per_wave)
            assert waves <= 16
            tiles = -(-out // 32)
            assert tiles < 256  # only where the tile kernel leaves CUs idle
            if t["slice_loads"] == 2:  # every workgroup resident at once (32 waves a CU, 256 CUs)
                assert 4 * tiles <= 256 * (32 // waves)
    elif t["kernel"] == q8.KERNEL_GEMM_F16:
        # f16-MFMA family: built variants t1_r4, t2_r2, t2_r4; <= 512 threads
        assert n >= 2
        assert (t["tpw"], t["rwaves"]) in ((1, 4), (2, 2), (2, 4))
        assert t["rwaves"] * t["kwaves"] <= 8
        npairs = (k // 32 + 1) // 2
        assert t["kwaves"] * t["pairs_per_wave"] >= npairs
        assert (t["kwaves"] - 1) * t["pairs_per_wave"] < npairs  # no K wave without pairs
    else:
        assert t["kernel"] == q8.KERNEL_GEMM
        assert t["tpw"] in (1, 2, 4)
        assert t["twaves"] * t["kwaves"] * 64 <= (1024 if t["tpw"] == 1 else 512)
        npairs = (k // 32 + 1) // 2
        pps = -(-npairs // t["kslices"])
        assert t["kwaves"] * t["pairs_per_wave"] >= pps


def test_plan_rejects_bad_shapes():
    with pytest.raises(q8.Q8Error) as e:
        llm_amd.plan(1, 10, 33)
    assert e.value.status == q8.Q8_ERR_INVALID
    with pytest.raises(q8.Q8Error) as e:
        llm_amd.plan(1025, 10, 32)
    assert e.value.status == q8.Q8_ERR_UNSUPPORTED
    with pytest.raises(q8.Q8Error) as e:
        llm_amd.plan(0, 10, 32)
    assert e.value.status == q8.Q8_ERR_INVALID


def test_weight_view_checks_its_byte_length():
    import numpy as np
    with pytest.raises(ValueError):
        q8.Weight(np.zeros(33, np.uint8), 32, 1)
    w = q8.Weight(np.zeros(68, np.uint8), 32, 2)
    assert w.identity()[1] == 68


# ---- kernel metadata and launch validation (cuda/mod.rs:229-283, 1835-1848) ----

ARG_STRUCTS = {  # kernel name prefix -> the argument struct every kernel of that family takes
    # the row-slice GEMVs: a preloadable scalar head (five pointers, three
    # ints, 56 bytes with padding), then the GEMV argument block
    "q8_gemv_r8_": "head + Q8GemvArgs", "q8_gemv_r16_": "head + Q8GemvArgs", "q8_gemv_rc": "head + Q8GemvArgs",
    "q8_gemv_q8x": "head + Q8GemvArgs",
    # the contiguous-group row-slice GEMVs: their own 56-byte head (five
    # pointers, four ints), then the same block
    "q8_gemv_hg": "head + Q8GemvArgs", "q8_gemv_hs": "head + Q8GemvArgs",
    "q8_gemv_hp": "head + Q8GemvArgs",
    # the decode attention: a preloadable head (five pointers, three ints, 56 bytes), then its block
    "q8_attn_decode": "head + Q8AttnDecodeArgs",
    "q8_gemm_": "Q8GemmArgs", "q8_gemv": "Q8GemvArgs", "q8_quantize": "Q8QuantArgs", "q8_rmsnorm": "Q8NormArgs",
    "q8_repack": "Q8RepackArgs", "q8_argmax": "Q8ArgmaxArgs", "q8_copy": "Q8CopyArgs", "q8_embed": "Q8EmbedArgs",
    "q8_silu_mul": "Q8EltArgs", "q8_rope_append": "Q8RopeArgs", "q8_attn_decode": "Q8AttnDecodeArgs",
    "q8_attn_prefill": "Q8AttnPrefillArgs", "q8_synth": "Q8SynthArgs", "q8_advance": "Q8AdvanceArgs",
    "q8_slice_copy": "Q8SliceArgs",
}


def test_every_kernel_carries_its_metadata():
    info = json.loads(llm_amd.build_info())
    sizes = {}
    for name in info["kernels"]:
        meta = q8.kernel_info(name)
        assert meta["args_bytes"] > 0, name
        assert meta["kernarg_bytes"] >= meta["args_bytes"], name
        assert meta["max_workgroup"] in (64, 128, 256, 512, 576, 1024), (name, meta["max_workgroup"])
        assert meta["private_bytes"] == 0, f"{name} spills {meta['private_bytes']} bytes per lane"
        assert 0 < meta["vgprs"] + meta["agprs"] <= 512, name
        family = next(s for p, s in ARG_STRUCTS.items() if name.startswith(p))
        sizes.setdefault(family, set()).add(meta["args_bytes"])
    # every kernel of a family takes the same struct, so the same argument bytes
    for family, seen in sizes.items():
        assert len(seen) == 1, f"{family}: kernels disagree on the argument size {sorted(seen)}"
    assert sizes["head + Q8GemvArgs"] == {56 + min(sizes["Q8GemvArgs"])}, "the row-slice head is 56 bytes"
    assert len([n for n in info["kernels"]
                if n.startswith(("q8_gemv_r8_", "q8_gemv_r16_", "q8_gemv_rc", "q8_gemv_q8x"))]) == 30
    assert len([n for n in info["kernels"] if n.startswith(("q8_gemv_hg", "q8_gemv_hs"))]) == 10
    assert len([n for n in info["kernels"] if n.startswith("q8_gemv_hp")]) == 4
    with pytest.raises(q8.Q8Error) as e:
        q8.kernel_info("q8_no_such_kernel")
    assert e.value.status == q8.Q8_ERR_INVALID


def test_launch_check_refuses_what_a_kernel_cannot_take():
    """The rules every launch of the library passes, host-only: the argument
    block is exactly the kernel's explicit arguments, the workgroup whole
    waves within the kernel's compiled bound, and static + dynamic LDS within
    the device's."""
    lds = 160 * 1024
    for name in ("q8_gemm_s1_t2", "q8_gemv_r8_l2", "q8_quantize", "q8_attn_prefill"):
        m = q8.kernel_info(name)
        ok = q8.launch_check(name, m["args_bytes"], 64, 0, lds)
        assert ok == q8.Q8_OK, (name, q8.lib().q8_last_error())
        assert q8.launch_check(name, m["args_bytes"], m["max_workgroup"], lds - m["static_lds"], lds) == q8.Q8_OK
        assert q8.launch_check(name, m["args_bytes"] + 8, 64, 0, lds) == q8.Q8_ERR_INVALID
        assert "argument block" in q8.lib().q8_last_error().decode()
        assert q8.launch_check(name, m["args_bytes"] - 4, 64, 0, lds) == q8.Q8_ERR_INVALID
        assert q8.launch_check(name, m["args_bytes"], m["max_workgroup"] + 64, 0, lds) == q8.Q8_ERR_INVALID
        assert q8.launch_check(name, m["args_bytes"], 96, 0, lds) == q8.Q8_ERR_INVALID   # not whole waves
        assert q8.launch_check(name, m["args_bytes"], 0, 0, lds) == q8.Q8_ERR_INVALID
        assert q8.launch_check(name, m["args_bytes"], 64, lds - m["static_lds"] + 1, lds) == q8.Q8_ERR_UNSUPPORTED
    assert q8.launch_check("q8_no_such_kernel", 8, 64, 0, lds) == q8.Q8_ERR_INVALID


# ---- the benchmark's probe library: outside the product boundary ----

def test_bench_library_exports_exactly_its_header():
    from llm_amd import probes
    text = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "q8bench.h")).read(), flags=re.S)
    declared = set(re.findall(r"\b(q8bench_[a-z0-9_]+)\s*\(", text))
    out = subprocess.run(["nm", "-D", "--defined-only", probes.LIB_PATH], stdout=subprocess.PIPE, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert declared == {s for s in exported if s.startswith("q8bench_")}
    assert declared == set(probes.EXPORTS)
    assert not {s for s in exported if s.startswith("q8_")}, "the bench library exports product symbols"
    product = json.loads(llm_amd.build_info())["kernels"]
    assert not [k for k in product if "probe" in k], "measurement kernels in the product code object"
    bench = json.loads(probes.lib().q8bench_build_info())
    assert "q8_probe_split_i8_valu" in bench["kernels"] and "q8_probe_read_l2_nt" in bench["kernels"]


# ---- the no-allocation scratch: one holding context per device ----

def test_noalloc_scratch_ownership_rule(tmp_path):
    """q8_noalloc_owner.h on its own (host code, g++): the first context to use
    a device's scratch holds it, a second is refused until the first releases,
    devices are independent, out-of-range devices are refused."""
    src = tmp_path / "owner_test.cpp"
    src.write_text(r'''
#include "q8_noalloc_owner.h"
#include <cstdio>
#define CHECK(c) do { if (!(c)) { std::printf("failed: %s (line %d)\n", #c, __LINE__); return 1; } } while (0)
int main() {
    q8i::NoallocOwners o;
    int a = 0, b = 0;
    CHECK(o.claim(0, &a));            // first user takes device 0
    CHECK(o.claim(0, &a));            // and keeps it
    CHECK(!o.claim(0, &b));           // a second context is refused
    CHECK(o.holder(0) == &a);
    CHECK(o.claim(1, &b));            // another device is independent
    CHECK(!o.claim(1, &a));
    o.release(&a);                    // q8_close of the holder
    CHECK(o.holder(0) == nullptr);
    CHECK(o.claim(0, &b));            // now the second context may take it
    CHECK(!o.claim(0, &a));
    CHECK(!o.claim(-1, &a) && !o.claim(q8i::NoallocOwners::kMaxDevices, &a));
    CHECK(!o.claim(2, nullptr));
    o.release(&b);
    CHECK(o.holder(0) == nullptr && o.holder(1) == nullptr);
    std::printf("ok\n");
    return 0;
}
''')
    exe = tmp_path / "owner_test"
    subprocess.run(["g++", "-std=c++17", "-O1", "-Wall", "-Werror", "-I", os.path.join(ROOT, "llm_amd", "csrc"),
                    str(src), "-o", str(exe)], check=True)
    res = subprocess.run([str(exe)], stdout=subprocess.PIPE, text=True)
    assert res.returncode == 0 and res.stdout.strip() == "ok", res.stdout


def test_noalloc_scratch_owner_table_under_threads(tmp_path):
    """The owner table under ThreadSanitizer (host code, g++): eight threads,
    each a context of its own, claim device 0 and release it in a loop; at
    most one holds it at any moment, every claim either succeeds for one
    thread or is refused, and TSan sees no data race."""
    src = tmp_path / "owner_threads.cpp"
    src.write_text(r'''
#include "q8_noalloc_owner.h"
#include <atomic>
#include <cstdio>
#include <thread>
#include <vector>
int main() {
    q8i::NoallocOwners o;
    std::atomic<int> inside{0}, bad{0}, taken{0};
    std::vector<std::thread> ts;
    for (int t = 0; t < 8; t++) {
        ts.emplace_back([&, t] {
            int me = t;
            for (int i = 0; i < 20000; i++) {
                if (o.claim(0, &me)) {
                    if (inside.fetch_add(1) != 0) bad++;
                    if (o.holder(0) != &me) bad++;
                    taken++;
                    inside.fetch_sub(1);
                    o.release(&me);
                } else if (o.holder(0) == &me) {
                    bad++;  // refused, yet recorded as the holder
                }
            }
        });
    }
    for (auto &th : ts) th.join();
    if (bad.load() != 0 || taken.load() == 0 || o.holder(0) != nullptr) {
        std::printf("failed: bad %d taken %d\n", bad.load(), taken.load());
        return 1;
    }
    std::printf("ok %d\n", taken.load());
    return 0;
}
''')
    exe = tmp_path / "owner_threads"
    subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=thread", "-Wall", "-Werror",
                    "-I", os.path.join(ROOT, "llm_amd", "csrc"), str(src), "-o", str(exe), "-pthread"], check=True)
    res = subprocess.run([str(exe)], stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True,
                         env=dict(os.environ, TSAN_OPTIONS="halt_on_error=1"))
    assert res.returncode == 0 and res.stdout.startswith("ok"), res.stdout[-3000:]
    assert "ThreadSanitizer" not in res.stdout, res.stdout[-3000:]
