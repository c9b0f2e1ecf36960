"""llm_amd: the MI355X-native (gfx950) Q8_0 matmul path of the reference engine.

The product is ``libq8mi.so`` (C-ABI in ``include/q8mi.h``): hand-written HIP
kernels for the n = 1 decode GEMV, the n >= 2 int8-MFMA prefill GEMM, the
activation quantizer, the fused gate/up + SiLU and the lm_head argmax, plus the
runtime that loads them (residency cache, workspaces, tactics table).
``llm_amd.q8`` is its Python binding, used by the tests and the benchmark.
"""
from .q8 import (Compute, DeviceBuffer, Gpu, GroupMember, Prepared, Q8Error, Weight, build_info,
                 lib, plan, tactic_table)

__all__ = ["Compute", "DeviceBuffer", "Gpu", "GroupMember", "Prepared", "Q8Error", "Weight",
           "build_info", "lib", "plan", "tactic_table"]
