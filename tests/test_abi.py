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
