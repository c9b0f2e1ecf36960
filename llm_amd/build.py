"""Build libq8mi.so: the gfx950 kernels as an embedded code object plus the
C-ABI runtime.

The counterpart of the reference's build script (apps/engine/build.rs:19-111),
which compiles gpu.cu to PTX with nvcc, embeds it, and records the build's
identity (source and PTX sha256, compiler, kernel names).  Here:

1. hipcc --genco --offload-arch=gfx950 compiles csrc/q8_kernels.hip to a code
   object (-ffp-contract=off: the reference's f32 arithmetic is uncontracted;
   packed FP32 off; MFMA results kept in VGPRs);
2. _build/q8_blob.S embeds that code object with .incbin, so the runtime loads
   it with hipModuleLoadData (a binary with NULs, hence bytes and not text);
3. _build/q8_manifest.h records arch, sha256 of the sources and the code
   object, the hipcc version and the kernel symbols (q8_build_info());
4. g++ compiles the host runtime (no device code) against the HIP runtime.

Run ``python -m llm_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import hashlib
import json
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(HERE, "libq8mi.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

KERNEL_SOURCES = ["q8_kernels.hip", "q8_attn.hip", "q8_layout.h"]
HOST_SOURCES = ["q8_runtime.cpp", "q8_tactics.cpp", "q8_gguf.cpp", "q8_decoder.cpp", "q8_tactics.h", "q8_layout.h",
                "q8_internal.h", "q8_noalloc.hip", "q8_noalloc_owner.h"]
# The measurement kernels live in a library of their own (libq8bench.so,
# include/q8bench.h): the benchmark's ceilings, not part of the product ABI.
BENCH_LIB = os.path.join(HERE, "libq8bench.so")
BENCH_SOURCES = ["q8_probe.hip", "q8_bench_args.h", "q8_bench.cpp"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    # the first 14 argument dwords of a kernel whose leading arguments are
    # scalars (the row-slice GEMVs, the read probes) arrive preloaded in SGPRs;
    # a kernel whose only argument is its argument block is unaffected
    "-mllvm", "-amdgpu-kernarg-preload-count=14",
]


def _sha256(path: str) -> str:
    h = hashlib.sha256()
    with open(path, "rb") as f:
        h.update(f.read())
    return h.hexdigest()


def _run(cmd: list[str]) -> str:
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in res.stdout.splitlines() if "packed-fp32-ops" not in line)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    return out


def _kernel_symbols(code_object: str) -> list[str]:
    """Kernel descriptors in our own code object (symbols ending in .kd)."""
    readelf = os.path.join(ROCM, "llvm", "bin", "llvm-readelf")
    out = _run([readelf, "-s", "--wide", code_object])
    names = sorted({tok[:-3] for line in out.splitlines() for tok in line.split() if tok.endswith(".kd")})
    return names


def _kernel_meta(code_object: str) -> list[dict]:
    """Each kernel's launch-relevant metadata from the code object's AMDGPU
    metadata note (our own build): bytes of explicit arguments (the extent of
    the non-hidden .args), the whole kernarg segment, VGPRs, AGPRs, SGPRs,
    static LDS, the largest workgroup the kernel was compiled for and its
    private (spill) bytes per lane.  The runtime checks every launch against
    it, as the reference inspects its kernels at load (cuda/mod.rs:229-283)."""
    import yaml
    readelf = os.path.join(ROCM, "llvm", "bin", "llvm-readelf")
    out = _run([readelf, "--notes", code_object])
    start = out.index("---")
    end = out.find("\n...", start)
    doc = yaml.safe_load(out[start:end if end >= 0 else len(out)])
    meta = []
    for k in doc["amdhsa.kernels"]:
        explicit = [a for a in k.get(".args", []) if not a[".value_kind"].startswith("hidden_")]
        meta.append({
            "name": k[".name"],
            "args": max((a[".offset"] + a[".size"] for a in explicit), default=0),
            "kernarg": k[".kernarg_segment_size"],
            "vgpr": k[".vgpr_count"],
            "agpr": k.get(".agpr_count", 0),
            "sgpr": k[".sgpr_count"],
            "lds": k[".group_segment_fixed_size"],
            "max_wg": k[".max_flat_workgroup_size"],
            "private": k[".private_segment_fixed_size"],
        })
    return sorted(meta, key=lambda m: m["name"])


def _meta_table(meta: list[dict], macro: str) -> str:
    """The metadata as a C initializer list (q8i::KernelMeta, q8_internal.h)."""
    rows = ",\\\n    ".join(
        f'{{"{m["name"]}", {m["args"]}u, {m["kernarg"]}u, {m["vgpr"]}u, {m["agpr"]}u, {m["sgpr"]}u, {m["lds"]}u, '
        f'{m["max_wg"]}u, {m["private"]}u}}' for m in meta)
    return f"#define {macro} \\\n    {rows}\n#define {macro}_COUNT {len(meta)}\n"


def _embed(asm_path: str, symbol: str, blob: str):
    """An assembly file that carries `blob` (a code object) as `symbol`."""
    with open(asm_path, "w") as f:
        f.write(
            "    .section .rodata\n"
            "    .p2align 12\n"
            f"    .globl {symbol}\n"
            f"{symbol}:\n"
            f"    .incbin \"{blob}\"\n"
            f"    .globl {symbol}_end\n"
            f"{symbol}_end:\n"
            "    .byte 0\n"
            "    .section .note.GNU-stack,\"\",@progbits\n")


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    hsaco = os.path.join(BUILD, "q8_kernels.hsaco")
    _run([hipcc, *HIPCC_FLAGS, "--genco", "--no-gpu-bundle-output", "-I", CSRC, "-o", hsaco, os.path.join(CSRC, "q8_kernels.hip")])

    version = _run([hipcc, "--version"]).splitlines()
    clang_line = next((v for v in version if "clang version" in v), version[0] if version else "")
    info = {
        "arch": ARCH,
        "kernel_source_sha256": hashlib.sha256(
            b"".join(open(os.path.join(CSRC, s), "rb").read() for s in KERNEL_SOURCES)).hexdigest(),
        "code_object_sha256": _sha256(hsaco),
        "host_source_sha256": hashlib.sha256(
            b"".join(open(os.path.join(CSRC, s), "rb").read() for s in HOST_SOURCES)).hexdigest(),
        "hipcc": clang_line.strip(),
        "hipcc_flags": " ".join(HIPCC_FLAGS),
        "kernels": _kernel_symbols(hsaco),
    }
    manifest = json.dumps(info, sort_keys=True)
    with open(os.path.join(BUILD, "q8_manifest.h"), "w") as f:
        f.write("/* generated by llm_amd/build.py */\n")
        f.write("#define Q8_BUILD_INFO " + json.dumps(manifest) + "\n")
        f.write(_meta_table(_kernel_meta(hsaco), "Q8_KERNEL_META"))
    _embed(os.path.join(BUILD, "q8_blob.S"), "q8_code_object", hsaco)

    # the static device scratch of q8_matmul_noalloc: host + device code in
    # the library's own fat binary (registered when the library loads)
    noalloc_obj = os.path.join(BUILD, "q8_noalloc.o")
    _run([hipcc, *HIPCC_FLAGS, "-fPIC", "-I", CSRC, "-I", INCLUDE, "-c", os.path.join(CSRC, "q8_noalloc.hip"),
          "-o", noalloc_obj])

    tmp = LIB + ".tmp"
    _run([
        "g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra", "-Wno-unused-parameter",
        "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"), "-I", CSRC, "-I", BUILD,
        "-I", INCLUDE,
        os.path.join(CSRC, "q8_runtime.cpp"), os.path.join(CSRC, "q8_tactics.cpp"), os.path.join(CSRC, "q8_gguf.cpp"),
        os.path.join(CSRC, "q8_decoder.cpp"),
        noalloc_obj,
        os.path.join(BUILD, "q8_blob.S"),
        "-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}",
        "-o", tmp,
    ])
    os.replace(tmp, LIB)
    build_bench(hipcc)
    if verbose:
        print(f"built {LIB} ({len(info['kernels'])} kernels, code object {info['code_object_sha256'][:12]}) "
              f"and {BENCH_LIB}")
    return LIB


def build_bench(hipcc: str) -> str:
    """libq8bench.so: the measurement kernels (q8_probe.hip) as a code object
    of their own, embedded like the product's, and their host launcher
    (q8_bench.cpp, include/q8bench.h)."""
    hsaco = os.path.join(BUILD, "q8_probe.hsaco")
    _run([hipcc, *HIPCC_FLAGS, "--genco", "--no-gpu-bundle-output", "-I", CSRC, "-o", hsaco,
          os.path.join(CSRC, "q8_probe.hip")])
    info = {"arch": ARCH, "code_object_sha256": _sha256(hsaco), "kernels": _kernel_symbols(hsaco),
            "source_sha256": hashlib.sha256(
                b"".join(open(os.path.join(CSRC, s), "rb").read() for s in BENCH_SOURCES)).hexdigest()}
    with open(os.path.join(BUILD, "q8_bench_manifest.h"), "w") as f:
        f.write("/* generated by llm_amd/build.py */\n")
        f.write("#define Q8_BENCH_BUILD_INFO " + json.dumps(json.dumps(info, sort_keys=True)) + "\n")
    _embed(os.path.join(BUILD, "q8_bench_blob.S"), "q8_bench_code_object", hsaco)
    tmp = BENCH_LIB + ".tmp"
    _run([
        "g++", "-std=c++17", "-O2", "-fPIC", "-shared", "-Wall", "-Wextra", "-Wno-unused-parameter",
        "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"), "-I", CSRC, "-I", BUILD, "-I", INCLUDE,
        os.path.join(CSRC, "q8_bench.cpp"), os.path.join(BUILD, "q8_bench_blob.S"),
        "-L", os.path.join(ROCM, "lib"), "-lamdhip64", f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}",
        "-o", tmp,
    ])
    os.replace(tmp, BENCH_LIB)
    return BENCH_LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
