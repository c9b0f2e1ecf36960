"""Python binding of libq8mi.so (include/q8mi.h) -- the test/bench host side.

``Gpu`` wraps the C-ABI one to one (it is what a Rust ``hip/sys.rs`` would
declare).  ``Compute`` mirrors the matmul entry points of
the reference engine's ``Compute`` (apps/engine/src/compute.rs:376-581,
931-1019) over device ``Activation``s, so the parity tests read like the
reference's own (apps/engine/tests/gpu_matmul.rs:57-65):

    compute.upload(source, x)
    compute.matmul(weight, source, 0, n, target, 0)
    compute.download(target, result)

There is no CPU fallback anywhere in this module: if the native library is
missing or no gfx950 device opens, every call raises.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libq8mi.so")

Q8_OK = 0
Q8_ERR_HIP = 1
Q8_ERR_INVALID = 2
Q8_ERR_UNSUPPORTED = 3
Q8_ERR_NO_DEVICE = 4
Q8_ERR_OUT_OF_MEMORY = 5
Q8_ERR_FORMAT = 6
Q8_ERR_MISSING = 7
Q8_ERR_IO = 8
MAX_TOKENS = 1024
GROUP_MAX = 4
KERNEL_GEMV, KERNEL_GEMM, KERNEL_GEMM_F16 = 1, 2, 3
PREPARED_I8, PREPARED_F16 = 0, 1

# Every function include/*.h declare (the ABI test checks the headers against
# this list and the library's exports).
EXPORTS = (
    "q8_status_string", "q8_last_error", "q8_build_info",
    "q8_open", "q8_close", "q8_device_name", "q8_device_info", "q8_stream", "q8_set_option",
    "q8_alloc", "q8_free", "q8_upload", "q8_download", "q8_sync",
    "q8_weight_resident", "q8_weight_group_resident", "q8_weight_release", "q8_weight_shape", "q8_weight_export",
    "q8_matmul", "q8_matmul_noalloc", "q8_matmul_q8", "q8_prepare", "q8_silu_mul_prepare", "q8_rmsnorm",
    "q8_norm_prepare", "q8_silu_mul",
    "q8_matmul_decode_group", "q8_matmul_prompt_group", "q8_gate_up_silu", "q8_gate_up_silu_prepared",
    "q8_gemm_prefetch", "q8_lm_head_argmax", "q8_argmax", "q8_copy_device", "q8_embeddings",
    "q8_kernel_info", "q8_launch_check",
    "q8_plan", "q8_tactic_count", "q8_tactic_row",
    "q8_event_create", "q8_event_record", "q8_event_elapsed_ms", "q8_event_destroy",
    "q8_graph_begin", "q8_graph_end", "q8_graph_launch", "q8_graph_destroy",
    "q8_gguf_open", "q8_gguf_close", "q8_gguf_layout", "q8_gguf_tensor_count", "q8_gguf_tensor_at",
    "q8_gguf_tensor", "q8_gguf_meta_count", "q8_gguf_meta_key_at", "q8_gguf_meta_type", "q8_gguf_meta_u64",
    "q8_gguf_meta_f32", "q8_gguf_meta_bool", "q8_gguf_meta_str", "q8_gguf_has_key_prefix",
    "q8_gguf_meta_i32_array", "q8_gguf_meta_f32_array", "q8_gguf_meta_str_array", "q8_gguf_weight",
    "q8_rope_append", "q8_attention", "q8_attention_prepare", "q8_attention_matmul_add", "q8_prompt_qkv_rope", "q8_embeddings_device", "q8_argmax_device", "q8_advance_position",
    "q8_norm_matmul_decode_group", "q8_norm_gate_up_silu",
    "q8_vector_release", "q8_norm_qkv_rope",
    "q8_weight_synthetic", "q8_decoder_create_synthetic", "q8_decoder_destroy", "q8_decoder_reset",
    "q8_decoder_position", "q8_decoder_forward", "q8_decoder_generate", "q8_decoder_logits", "q8_decoder_weight",
    "q8_decoder_norm", "q8_decoder_graph_stats", "q8_norm_lm_head_argmax",
    "q8_workspace_plan", "q8_workspace_query", "q8_workspace_region", "q8_vector_resident",
)



class Q8Error(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{message} [status {status}]")
        self.status = status
        self.message = message


class Prepared(ctypes.Structure):
    """q8_prepared: quantized activations (the reference's ``Prepared``)."""
    _fields_ = [("quants", ctypes.c_uint64), ("scales", ctypes.c_uint64),
                ("n", ctypes.c_int), ("k", ctypes.c_int), ("format", ctypes.c_int)]

    def quant_bytes(self) -> int:
        """Bytes of the quant plane: one unit per (32 tokens, block), 1 KB
        as int8 (PREPARED_I8) or 2 KB as f16 (PREPARED_F16)."""
        units = (self.n + 31) // 32 * (self.k // 32)
        return units * (2048 if self.format == PREPARED_F16 else 1024)

    def scale_bytes(self) -> int:
        return (self.n + 31) // 32 * (self.k // 32) * 32 * 4


class KernelInfo(ctypes.Structure):
    """q8_kernel_info_t: one kernel's metadata from the code object."""
    _fields_ = [("args_bytes", ctypes.c_uint32), ("kernarg_bytes", ctypes.c_uint32), ("vgprs", ctypes.c_uint32),
                ("agprs", ctypes.c_uint32), ("sgprs", ctypes.c_uint32), ("static_lds", ctypes.c_uint32),
                ("max_workgroup", ctypes.c_uint32), ("private_bytes", ctypes.c_uint32)]


def kernel_info(name: str) -> dict:
    """q8_kernel_info as a dict."""
    info = KernelInfo()
    _check(lib().q8_kernel_info(name.encode(), ctypes.byref(info)))
    return {f: getattr(info, f) for f, _ in info._fields_}


def launch_check(name: str, args_bytes: int, block: int, dynamic_lds: int, lds_limit: int) -> int:
    """q8_launch_check's status (no device needed)."""
    return lib().q8_launch_check(name.encode(), args_bytes, block, dynamic_lds, lds_limit)


class GgufTensorInfo(ctypes.Structure):
    """q8_gguf_tensor_info (include/q8gguf.h)."""
    _fields_ = [("name", ctypes.c_char_p), ("name_len", ctypes.c_uint64), ("n_dims", ctypes.c_uint32),
                ("dims", ctypes.POINTER(ctypes.c_uint64)), ("dtype", ctypes.c_uint32),
                ("offset", ctypes.c_uint64), ("byte_len", ctypes.c_uint64), ("elements", ctypes.c_uint64),
                ("data", ctypes.c_void_p)]


class DecoderConfig(ctypes.Structure):
    """q8_decoder_config (include/q8decoder.h)."""
    _fields_ = [(f, ctypes.c_int) for f in ("n_layer", "n_embd", "n_ff", "n_head", "n_head_kv", "head_dim",
                                            "n_rot", "n_vocab", "capacity", "max_batch")] + \
               [("eps", ctypes.c_float), ("rope_base", ctypes.c_float), ("untied_output", ctypes.c_int),
                ("embd_std", ctypes.c_float)]


class WorkspaceShape(ctypes.Structure):
    """q8_workspace_shape (include/q8mi.h)."""
    _fields_ = [(f, ctypes.c_int) for f in ("max_tokens", "max_k", "max_ff", "attn_heads", "attn_splits",
                                            "rope_n_rot")] + [("rope_base", ctypes.c_float)]


class WorkspaceInfo(ctypes.Structure):
    """q8_workspace_info (include/q8mi.h)."""
    _fields_ = [(f, ctypes.c_uint64) for f in ("bytes", "arena_bytes", "allocations", "generation")] + \
               [("regions", ctypes.c_int)]


class DecoderStats(ctypes.Structure):
    """q8_decoder_stats (include/q8decoder.h)."""
    _fields_ = [(f, ctypes.c_int) for f in ("graphs", "captured", "dropped", "eager")]


class _GroupEntry(ctypes.Structure):
    _fields_ = [("weight", ctypes.c_void_p), ("y", ctypes.c_uint64), ("y_offset", ctypes.c_size_t)]


class Tactic(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_int), ("waves_per_tile", ctypes.c_int),
                ("pairs_per_wave", ctypes.c_int), ("pairs_per_batch", ctypes.c_int),
                ("exact", ctypes.c_int), ("tpw", ctypes.c_int), ("twaves", ctypes.c_int),
                ("smode", ctypes.c_int),
                ("xcd_remap", ctypes.c_int), ("kslices", ctypes.c_int), ("kwaves", ctypes.c_int),
                ("rwaves", ctypes.c_int), ("pipe", ctypes.c_int),
                ("row_slice", ctypes.c_int), ("slice_loads", ctypes.c_int),
                ("name", ctypes.c_char_p), ("evidence", ctypes.c_char_p)]

    def as_dict(self) -> dict:
        d = {f: getattr(self, f) for f, _ in self._fields_}
        d["name"] = (self.name or b"").decode()
        d["evidence"] = (self.evidence or b"").decode()
        return d


_lib = None


def library_path() -> str:
    return LIB_PATH


def lib():
    """Load libq8mi.so; raises if it was not built (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m llm_amd.build` "
                           "(the Q8_0 path has no CPU fallback)")
    L = ctypes.CDLL(LIB_PATH)
    c_int, c_size, u64, vp = ctypes.c_int, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_void_p
    sig = {
        "q8_status_string": (ctypes.c_char_p, [c_int]),
        "q8_last_error": (ctypes.c_char_p, []),
        "q8_build_info": (ctypes.c_char_p, []),
        "q8_open": (c_int, [c_int, ctypes.POINTER(vp)]),
        "q8_close": (None, [vp]),
        "q8_device_name": (c_int, [vp, ctypes.c_char_p, c_size]),
        "q8_device_info": (c_int, [vp, ctypes.POINTER(c_int), ctypes.POINTER(c_size), ctypes.POINTER(c_size)]),
        "q8_stream": (vp, [vp]),
        "q8_set_option": (c_int, [vp, ctypes.c_char_p, c_int]),
        "q8_alloc": (c_int, [vp, c_size, ctypes.POINTER(u64)]),
        "q8_free": (c_int, [vp, u64]),
        "q8_upload": (c_int, [vp, u64, vp, c_size]),
        "q8_download": (c_int, [vp, vp, u64, c_size]),
        "q8_sync": (c_int, [vp]),
        "q8_weight_resident": (c_int, [vp, vp, c_size, c_int, c_int, ctypes.POINTER(vp)]),
        "q8_weight_group_resident": (c_int, [vp, c_int, ctypes.POINTER(vp), ctypes.POINTER(c_size), c_int,
                                             ctypes.POINTER(c_int), c_int, ctypes.POINTER(vp)]),
        "q8_weight_release": (c_int, [vp, vp]),
        "q8_weight_shape": (c_int, [vp, ctypes.POINTER(c_int), ctypes.POINTER(c_int), ctypes.POINTER(c_size)]),
        "q8_weight_export": (c_int, [vp, vp, vp, c_size]),
        "q8_matmul": (c_int, [vp, vp, u64, c_size, c_int, u64, c_size, ctypes.POINTER(Prepared), u64, c_size]),
        "q8_matmul_noalloc": (c_int, [vp, vp, u64, c_size, c_int, u64, c_size, u64, c_size]),
        "q8_matmul_q8": (c_int, [vp, vp, u64, c_size, c_int, u64, c_size, u64, c_size]),
        "q8_prepare": (c_int, [vp, u64, c_size, c_int, c_int, ctypes.POINTER(Prepared)]),
        "q8_silu_mul_prepare": (c_int, [vp, u64, u64, c_int, c_int, ctypes.POINTER(Prepared)]),
        "q8_silu_mul": (c_int, [vp, u64, u64, u64, c_size]),
        "q8_rmsnorm": (c_int, [vp, u64, c_size, vp, c_int, ctypes.c_float, c_int, u64, c_size]),
        "q8_norm_prepare": (c_int, [vp, u64, c_size, vp, c_int, ctypes.c_float, c_int, ctypes.POINTER(Prepared)]),
        "q8_matmul_decode_group": (c_int, [vp, ctypes.POINTER(_GroupEntry), c_int, u64, c_size, c_int, u64, c_size]),
        "q8_matmul_prompt_group": (c_int, [vp, ctypes.POINTER(_GroupEntry), c_int, ctypes.POINTER(Prepared),
                                           c_int, c_int, u64, c_size]),
        "q8_gate_up_silu": (c_int, [vp, vp, vp, u64, c_size, c_int, u64, c_size, ctypes.POINTER(Prepared)]),
        "q8_gemm_prefetch": (c_int, [vp, ctypes.POINTER(vp), c_int]),
        "q8_norm_matmul_decode_group": (c_int, [vp, vp, ctypes.c_float, ctypes.POINTER(_GroupEntry), c_int, u64,
                                                c_size, c_int]),
        "q8_norm_gate_up_silu": (c_int, [vp, vp, ctypes.c_float, vp, vp, u64, c_size, u64, c_size]),
        "q8_vector_release": (c_int, [vp, vp, c_size]),
        "q8_norm_qkv_rope": (c_int, [vp, vp, ctypes.c_float, vp, vp, vp, u64, c_size, u64, c_size, u64, u64, c_int,
                                     c_int, c_int, c_int, ctypes.c_float, c_int, u64]),
        "q8_gate_up_silu_prepared": (c_int, [vp, vp, vp, ctypes.POINTER(Prepared), ctypes.POINTER(Prepared)]),
        "q8_lm_head_argmax": (c_int, [vp, vp, u64, c_size, u64, c_size, ctypes.POINTER(ctypes.c_uint32)]),
        "q8_argmax": (c_int, [vp, u64, c_size, c_size, ctypes.POINTER(ctypes.c_uint32)]),
        "q8_copy_device": (c_int, [vp, u64, u64, c_size]),
        "q8_kernel_info": (c_int, [ctypes.c_char_p, ctypes.POINTER(KernelInfo)]),
        "q8_launch_check": (c_int, [ctypes.c_char_p, c_size, ctypes.c_uint, c_size, c_size]),
        "q8_embeddings": (c_int, [vp, vp, ctypes.POINTER(ctypes.c_uint32), c_size, u64, c_size]),
        "q8_plan": (c_int, [vp, c_int, c_int, c_int, ctypes.POINTER(Tactic)]),
        "q8_tactic_count": (c_int, []),
        "q8_tactic_row": (c_int, [c_int, ctypes.POINTER(Tactic), ctypes.POINTER(c_int), ctypes.POINTER(c_int)]),
        "q8_event_create": (c_int, [vp, ctypes.POINTER(vp)]),
        "q8_event_record": (c_int, [vp, vp]),
        "q8_event_elapsed_ms": (c_int, [vp, vp, ctypes.POINTER(ctypes.c_float)]),
        "q8_event_destroy": (c_int, [vp]),
        "q8_graph_begin": (c_int, [vp]),
        "q8_graph_end": (c_int, [vp, ctypes.POINTER(vp)]),
        "q8_graph_launch": (c_int, [vp, vp]),
        "q8_graph_destroy": (c_int, [vp]),
        "q8_gguf_open": (c_int, [ctypes.c_char_p, ctypes.POINTER(vp)]),
        "q8_gguf_close": (None, [vp]),
        "q8_gguf_layout": (c_int, [vp, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(u64), ctypes.POINTER(u64),
                                   ctypes.POINTER(u64)]),
        "q8_gguf_tensor_count": (c_int, [vp, ctypes.POINTER(u64)]),
        "q8_gguf_tensor_at": (c_int, [vp, u64, ctypes.POINTER(GgufTensorInfo)]),
        "q8_gguf_tensor": (c_int, [vp, ctypes.c_char_p, ctypes.POINTER(GgufTensorInfo)]),
        "q8_gguf_meta_count": (c_int, [vp, ctypes.POINTER(u64)]),
        "q8_gguf_meta_key_at": (c_int, [vp, u64, ctypes.POINTER(ctypes.c_char_p)]),
        "q8_gguf_meta_type": (c_int, [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32),
                                      ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(u64)]),
        "q8_gguf_meta_u64": (c_int, [vp, ctypes.c_char_p, ctypes.POINTER(u64)]),
        "q8_gguf_meta_f32": (c_int, [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float)]),
        "q8_gguf_meta_bool": (c_int, [vp, ctypes.c_char_p, ctypes.POINTER(c_int)]),
        "q8_gguf_meta_str": (c_int, [vp, ctypes.c_char_p, ctypes.POINTER(vp), ctypes.POINTER(u64)]),
        "q8_gguf_has_key_prefix": (c_int, [vp, ctypes.c_char_p]),
        "q8_gguf_meta_i32_array": (c_int, [vp, ctypes.c_char_p, vp, u64, ctypes.POINTER(u64)]),
        "q8_gguf_meta_f32_array": (c_int, [vp, ctypes.c_char_p, vp, u64, ctypes.POINTER(u64)]),
        "q8_gguf_meta_str_array": (c_int, [vp, ctypes.c_char_p, ctypes.POINTER(vp), ctypes.POINTER(u64), u64,
                                           ctypes.POINTER(u64)]),
        "q8_gguf_weight": (c_int, [vp, vp, ctypes.c_char_p, c_int, c_int, ctypes.POINTER(vp)]),
        "q8_rope_append": (c_int, [vp, u64, c_size, u64, c_size, u64, c_size, u64, u64, c_int, c_int, c_int, c_int,
                                   c_int, ctypes.c_float, c_int, u64]),
        "q8_attention": (c_int, [vp, u64, c_size, u64, u64, u64, c_size, c_int, c_int, c_int, c_int, c_int,
                                 ctypes.c_float, u64, c_int]),
        "q8_attention_matmul_add": (c_int, [vp, u64, c_size, u64, u64, c_int, c_int, c_int, c_int, ctypes.c_float,
                                            u64, c_int, vp, u64, c_size]),
        "q8_attention_prepare": (c_int, [vp, u64, c_size, u64, u64, c_int, c_int, c_int, c_int, c_int, ctypes.c_float,
                                         u64, ctypes.POINTER(Prepared)]),
        "q8_prompt_qkv_rope": (c_int, [vp, vp, vp, vp, vp, c_int, u64, c_size, u64, u64, c_int, c_int, c_int, c_int,
                                       ctypes.c_float, c_int, u64]),
        "q8_embeddings_device": (c_int, [vp, vp, u64, c_size, u64, c_size]),
        "q8_argmax_device": (c_int, [vp, u64, c_size, c_size, u64]),
        "q8_advance_position": (c_int, [vp, u64, c_int]),
        "q8_weight_synthetic": (c_int, [vp, c_int, c_int, u64, ctypes.c_float, ctypes.POINTER(vp)]),
        "q8_decoder_create_synthetic": (c_int, [vp, ctypes.POINTER(DecoderConfig), u64, ctypes.POINTER(vp)]),
        "q8_decoder_destroy": (None, [vp]),
        "q8_decoder_reset": (c_int, [vp]),
        "q8_decoder_position": (c_int, [vp, ctypes.POINTER(c_int)]),
        "q8_decoder_forward": (c_int, [vp, ctypes.POINTER(ctypes.c_uint32), c_int, ctypes.POINTER(ctypes.c_uint32)]),
        "q8_decoder_generate": (c_int, [vp, c_int, ctypes.POINTER(ctypes.c_uint32)]),
        "q8_decoder_logits": (c_int, [vp, ctypes.POINTER(ctypes.c_float), c_size]),
        "q8_decoder_weight": (c_int, [vp, c_int, c_int, ctypes.POINTER(vp)]),
        "q8_decoder_norm": (c_int, [vp, c_int, c_int, ctypes.POINTER(ctypes.POINTER(ctypes.c_float))]),
        "q8_decoder_graph_stats": (c_int, [vp, ctypes.POINTER(DecoderStats)]),
        "q8_norm_lm_head_argmax": (c_int, [vp, vp, ctypes.c_float, vp, u64, c_size, u64, c_size, u64]),
        "q8_workspace_plan": (c_int, [vp, ctypes.POINTER(WorkspaceShape)]),
        "q8_workspace_query": (c_int, [vp, ctypes.POINTER(WorkspaceInfo)]),
        "q8_workspace_region": (c_int, [vp, c_int, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(u64),
                                        ctypes.POINTER(u64)]),
        "q8_vector_resident": (c_int, [vp, vp, c_size]),
    }
    assert set(sig) == set(EXPORTS)
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def _check(status: int):
    if status != Q8_OK:
        msg = lib().q8_last_error().decode(errors="replace")
        raise Q8Error(status, msg or lib().q8_status_string(status).decode())


def build_info() -> str:
    return lib().q8_build_info().decode()


def tactic_table() -> list[dict]:
    out = []
    for i in range(lib().q8_tactic_count()):
        t, rank, maturity = Tactic(), ctypes.c_int(), ctypes.c_int()
        _check(lib().q8_tactic_row(i, ctypes.byref(t), ctypes.byref(rank), ctypes.byref(maturity)))
        d = t.as_dict()
        d["rank"] = rank.value
        d["maturity"] = maturity.value
        out.append(d)
    return out


def plan(n: int, out: int, k: int, gpu: "Gpu | None" = None) -> dict:
    t = Tactic()
    _check(lib().q8_plan(gpu.handle if gpu else None, n, out, k, ctypes.byref(t)))
    return t.as_dict()


class DeviceBuffer:
    """A q8_alloc'd device allocation (the reference's ``DeviceBuffer`` of f32,
    cuda/mod.rs:123-182); ``len`` counts f32 elements."""

    def __init__(self, gpu: "Gpu", nbytes: int):
        self.gpu = gpu
        self.nbytes = int(nbytes)
        p = ctypes.c_uint64()
        _check(lib().q8_alloc(gpu.handle, self.nbytes, ctypes.byref(p)))
        self.ptr = p.value

    def __len__(self):
        return self.nbytes // 4

    def free(self):
        if self.ptr and self.gpu.handle:
            _check(lib().q8_free(self.gpu.handle, self.ptr))
        self.ptr = 0

    def upload(self, values: np.ndarray, offset_bytes: int = 0):
        a = np.ascontiguousarray(values)
        assert offset_bytes + a.nbytes <= self.nbytes, "upload overruns the buffer"
        _check(lib().q8_upload(self.gpu.handle, self.ptr + offset_bytes, a.ctypes.data, a.nbytes))

    def download(self, dtype=np.float32, count: int | None = None, offset_bytes: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset_bytes) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        assert offset_bytes + out.nbytes <= self.nbytes, "download overruns the buffer"
        _check(lib().q8_download(self.gpu.handle, out.ctypes.data, self.ptr + offset_bytes, out.nbytes))
        return out


class Weight:
    """A host Q8_0 matrix ``out x k`` (the reference's ``Weight``,
    tensor.rs:15-51): GGUF bytes plus shape.  Its identity (address, length)
    keys the device residency cache, so the bytes are kept alive here."""

    def __init__(self, data: np.ndarray, k: int, out: int):
        data = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
        if k % 32 != 0 or data.size != out * (k // 32) * 34:
            raise ValueError("weight byte length mismatch")
        self.data, self.k, self.out = data, int(k), int(out)

    def identity(self):
        return (self.data.ctypes.data, self.data.nbytes)


class DeviceWeight:
    """A weight that lives only on the device (q8_weight_synthetic, or a
    decoder's): the C-ABI handle plus its shape.  Accepted wherever a
    ``Weight`` is; ``Gpu.export`` reads its GGUF bytes back."""

    def __init__(self, handle: int, k: int, out: int):
        self.handle, self.k, self.out = handle, int(k), int(out)

    def nbytes(self) -> int:
        return self.out * (self.k // 32) * 34


class Gpu:
    """The C-ABI context: Gpu::open / Drop (cuda/mod.rs:363-522, 1981-1993)."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        _check(lib().q8_open(device, ctypes.byref(h)))
        self.handle = h.value
        self._resident = {}
        self._pinned = {}  # norm weights made resident by host identity

    def close(self):
        if self.handle:
            lib().q8_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def name(self) -> str:
        buf = ctypes.create_string_buffer(256)
        _check(lib().q8_device_name(self.handle, buf, 256))
        return buf.value.decode()

    def info(self) -> dict:
        cu, tot, fr = ctypes.c_int(), ctypes.c_size_t(), ctypes.c_size_t()
        _check(lib().q8_device_info(self.handle, ctypes.byref(cu), ctypes.byref(tot), ctypes.byref(fr)))
        return {"cu_count": cu.value, "total_bytes": tot.value, "free_bytes": fr.value}

    def set_option(self, name: str, value: int):
        _check(lib().q8_set_option(self.handle, name.encode(), int(value)))

    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def sync(self):
        _check(lib().q8_sync(self.handle))

    def workspace_plan(self, max_tokens: int, max_k: int, max_ff: int = 0, attn_heads: int = 0,
                       attn_splits: int = 0, rope_n_rot: int = 0, rope_base: float = 10000.0):
        """q8_workspace_plan: size every workspace once for these shapes."""
        s = WorkspaceShape(max_tokens, max_k, max_ff, attn_heads, attn_splits, rope_n_rot, rope_base)
        _check(lib().q8_workspace_plan(self.handle, ctypes.byref(s)))

    def workspace(self) -> dict:
        """q8_workspace_query plus the plan's regions (name, offset, bytes)."""
        info = WorkspaceInfo()
        _check(lib().q8_workspace_query(self.handle, ctypes.byref(info)))
        d = {f: getattr(info, f) for f, _ in info._fields_}
        regions = []
        for i in range(info.regions):
            name, off, nb = ctypes.c_char_p(), ctypes.c_uint64(), ctypes.c_uint64()
            _check(lib().q8_workspace_region(self.handle, i, ctypes.byref(name), ctypes.byref(off), ctypes.byref(nb)))
            regions.append((name.value.decode(), off.value, nb.value))
        d["layout"] = regions
        return d

    def resident(self, weight: Weight):
        """Gpu::quantized: upload + repack once, cached by identity."""
        if isinstance(weight, DeviceWeight):
            return weight.handle
        h = ctypes.c_void_p()
        _check(lib().q8_weight_resident(self.handle, weight.data.ctypes.data, weight.data.nbytes,
                                        weight.k, weight.out, ctypes.byref(h)))
        self._resident[weight.identity()] = weight  # keep the host bytes alive
        return h.value

    def resident_group(self, weights, pair: bool = False):
        """q8_weight_group_resident: the weights (one k) as one contiguous
        group, each then resident on its own identity; pair = a gate/up pair."""
        n = len(weights)
        ptrs = (ctypes.c_void_p * n)(*[w.data.ctypes.data for w in weights])
        sizes = (ctypes.c_size_t * n)(*[w.data.nbytes for w in weights])
        outs = (ctypes.c_int * n)(*[w.out for w in weights])
        hs = (ctypes.c_void_p * n)()
        _check(lib().q8_weight_group_resident(self.handle, n, ptrs, sizes, weights[0].k, outs, int(pair), hs))
        for w in weights:
            self._resident[w.identity()] = w
        return list(hs)

    def release(self, weight: Weight):
        h = self.resident(weight)
        _check(lib().q8_weight_release(self.handle, h))
        self._resident.pop(weight.identity(), None)

    def export(self, weight: Weight) -> np.ndarray:
        h = self.resident(weight)
        out = np.empty(weight.nbytes() if isinstance(weight, DeviceWeight) else weight.data.nbytes, dtype=np.uint8)
        _check(lib().q8_weight_export(self.handle, h, out.ctypes.data, out.nbytes))
        return out

    def matmul(self, weight: Weight, x: DeviceBuffer, x_offset: int, n: int, y: DeviceBuffer,
               y_offset: int, prepared: Prepared | None = None, bias: DeviceBuffer | None = None,
               bias_offset: int = 0):
        h = self.resident(weight)
        _check(lib().q8_matmul(self.handle, h, x.ptr, x_offset, n, y.ptr, y_offset,
                               ctypes.byref(prepared) if prepared is not None else None,
                               bias.ptr if bias is not None else 0, bias_offset))

    def matmul_q8(self, weight: Weight, x: DeviceBuffer, x_offset: int, n: int, y: DeviceBuffer, y_offset: int,
                  bias: DeviceBuffer | None = None, bias_offset: int = 0):
        """q8_matmul_q8: x quantized to Q8_0 at every n, n = 1 included."""
        h = self.resident(weight)
        _check(lib().q8_matmul_q8(self.handle, h, x.ptr, x_offset, n, y.ptr, y_offset,
                                  bias.ptr if bias is not None else 0, bias_offset))

    def prepare(self, x: DeviceBuffer, x_offset: int, n: int, k: int) -> Prepared:
        p = Prepared()
        _check(lib().q8_prepare(self.handle, x.ptr, x_offset, n, k, ctypes.byref(p)))
        return p

    def silu_mul_prepare(self, gate: DeviceBuffer, up: DeviceBuffer, n: int, k: int) -> Prepared:
        p = Prepared()
        _check(lib().q8_silu_mul_prepare(self.handle, gate.ptr, up.ptr, n, k, ctypes.byref(p)))
        return p

    def _norm_weight(self, weight: np.ndarray) -> np.ndarray:
        """The library makes a norm weight resident by its host identity
        (pointer, length), as the reference's Gpu::plain does for its mmap'd
        slices.  The array is pinned here for the context's lifetime, so its
        address cannot be reused by another array while the copy is cached;
        its contents must not change."""
        if not (isinstance(weight, np.ndarray) and weight.dtype == np.float32 and weight.flags.c_contiguous):
            raise TypeError("norm weight must be a C-contiguous float32 numpy array")
        self._pinned.setdefault((weight.ctypes.data, weight.size), weight)
        return weight

    def rmsnorm(self, x: DeviceBuffer, x_offset: int, weight: np.ndarray, eps: float, rows: int,
                out: DeviceBuffer, out_offset: int = 0):
        """Gpu::rmsnorm_rows (compute.rs:584-614): f32 RMSNorm of `rows` rows."""
        w = self._norm_weight(weight)
        _check(lib().q8_rmsnorm(self.handle, x.ptr, x_offset, w.ctypes.data, w.size, float(eps), rows, out.ptr,
                                out_offset))

    def norm_prepare(self, x: DeviceBuffer, x_offset: int, weight: np.ndarray, eps: float, rows: int) -> Prepared:
        """Gpu::rmsnorm_prepare (cuda/mod.rs:1414-1445): quantize(rmsnorm(x))."""
        w = self._norm_weight(weight)
        p = Prepared()
        _check(lib().q8_norm_prepare(self.handle, x.ptr, x_offset, w.ctypes.data, w.size, float(eps), rows,
                                     ctypes.byref(p)))
        return p

    def silu_mul(self, act: DeviceBuffer, gate: DeviceBuffer, up: DeviceBuffer, length: int):
        _check(lib().q8_silu_mul(self.handle, act.ptr, gate.ptr, up.ptr, length))

    def _group(self, members):
        arr = (_GroupEntry * len(members))()
        for i, (w, y, y_off) in enumerate(members):
            arr[i].weight = self.resident(w)
            arr[i].y = y.ptr
            arr[i].y_offset = y_off
        return arr

    def matmul_decode_group(self, members, x: DeviceBuffer, x_offset: int, k: int,
                            bias: DeviceBuffer | None = None, bias_offset: int = 0):
        arr = self._group(members)
        _check(lib().q8_matmul_decode_group(self.handle, arr, len(members), x.ptr, x_offset, k,
                                            bias.ptr if bias is not None else 0, bias_offset))

    def norm_matmul_decode_group(self, weight: np.ndarray, eps: float, members, x: DeviceBuffer, x_offset: int,
                                 k: int):
        """rmsnorm(x) then matmul_decode_group, the norm folded into the GEMV."""
        w = self._norm_weight(weight)
        arr = self._group(members)
        _check(lib().q8_norm_matmul_decode_group(self.handle, w.ctypes.data, float(eps), arr, len(members), x.ptr,
                                                 x_offset, k))

    def norm_qkv_rope(self, weight: np.ndarray, eps: float, wq: Weight, wk: Weight, wv: Weight, x: DeviceBuffer,
                      x_offset: int, q: DeviceBuffer, q_offset: int, kcache: DeviceBuffer, vcache: DeviceBuffer,
                      n_head: int, n_kv: int, head_dim: int, n_rot: int, base: float, capacity: int,
                      position: DeviceBuffer):
        """rmsnorm + q/k/v decode GEMV + rope_append of one token, one launch."""
        w = self._norm_weight(weight)
        _check(lib().q8_norm_qkv_rope(self.handle, w.ctypes.data, float(eps), self.resident(wq), self.resident(wk),
                                      self.resident(wv), x.ptr, x_offset, q.ptr, q_offset, kcache.ptr, vcache.ptr,
                                      n_head, n_kv, head_dim, n_rot, float(base), capacity, position.ptr))

    def norm_gate_up_silu(self, weight: np.ndarray, eps: float, gate: Weight, up: Weight, x: DeviceBuffer,
                          x_offset: int, act: DeviceBuffer, act_offset: int):
        """rmsnorm(x) then gate_up_silu at n = 1, the norm folded into the GEMV."""
        w = self._norm_weight(weight)
        _check(lib().q8_norm_gate_up_silu(self.handle, w.ctypes.data, float(eps), self.resident(gate),
                                          self.resident(up), x.ptr, x_offset, act.ptr, act_offset))

    def gemm_prefetch(self, weights):
        """q8_gemm_prefetch: the next n >= 2 GEMM launch reads these weights
        (at most four) into the device caches beside its own work."""
        arr = (ctypes.c_void_p * max(1, len(weights)))(*[self.resident(w) for w in weights])
        _check(lib().q8_gemm_prefetch(self.handle, arr, len(weights)))

    def matmul_prompt_group(self, members, prepared: Prepared, n: int, k: int,
                            bias: DeviceBuffer | None = None, bias_offset: int = 0):
        arr = self._group(members)
        _check(lib().q8_matmul_prompt_group(self.handle, arr, len(members), ctypes.byref(prepared), n, k,
                                            bias.ptr if bias is not None else 0, bias_offset))

    def gate_up_silu(self, gate: Weight, up: Weight, x: DeviceBuffer, x_offset: int, n: int,
                     act: DeviceBuffer, act_offset: int, want_prepared: bool = False):
        p = Prepared()
        _check(lib().q8_gate_up_silu(self.handle, self.resident(gate), self.resident(up), x.ptr, x_offset,
                                     n, act.ptr, act_offset, ctypes.byref(p) if want_prepared else None))
        return p if want_prepared else None

    def gate_up_silu_prepared(self, gate: Weight, up: Weight, prepared: Prepared) -> Prepared:
        """matmul_prepared_group(gate, up) + silu_mul_prepare on prepared x (n >= 2)."""
        out = Prepared()
        _check(lib().q8_gate_up_silu_prepared(self.handle, self.resident(gate), self.resident(up),
                                              ctypes.byref(prepared), ctypes.byref(out)))
        return out

    def lm_head_argmax(self, weight: Weight, x: DeviceBuffer, x_offset: int, logits: DeviceBuffer,
                       logits_offset: int) -> int:
        out = ctypes.c_uint32()
        _check(lib().q8_lm_head_argmax(self.handle, self.resident(weight), x.ptr, x_offset, logits.ptr,
                                       logits_offset, ctypes.byref(out)))
        return int(out.value)

    def embeddings(self, weight: Weight, tokens, out: DeviceBuffer, out_offset: int = 0):
        """Gpu::embeddings (cuda/mod.rs:1690-1716): rows `tokens` of the
        resident weight, dequantized into out[out_offset:]."""
        ids = np.ascontiguousarray(np.asarray(tokens, dtype=np.int64))
        if ids.size and (ids.min() < 0 or ids.max() > 0xFFFFFFFF):
            raise Q8Error(Q8_ERR_INVALID, "token ids are u32")
        ids = ids.astype(np.uint32)
        _check(lib().q8_embeddings(self.handle, self.resident(weight),
                                   ids.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), ids.size, out.ptr,
                                   out_offset))

    def gguf_weight(self, gguf, name: str, k: int, out: int):
        """q8_gguf_weight: the shape-checked Q8_0 tensor of an open GgufFile
        made resident straight from the map.  The file is kept open while the
        context may use the weight."""
        h = ctypes.c_void_p()
        _check(lib().q8_gguf_weight(self.handle, gguf.handle, name.encode(), k, out, ctypes.byref(h)))
        info = gguf.tensor(name)
        self._resident[(gguf.data_address(name), info.byte_len)] = gguf
        return h.value

    def weight_synthetic(self, k: int, out: int, seed: int, scale_std: float = 0.02) -> DeviceWeight:
        h = ctypes.c_void_p()
        _check(lib().q8_weight_synthetic(self.handle, k, out, seed, scale_std, ctypes.byref(h)))
        return DeviceWeight(h.value, k, out)

    def release_device(self, weight: DeviceWeight):
        _check(lib().q8_weight_release(self.handle, weight.handle))

    def rope_append(self, q: DeviceBuffer, k: DeviceBuffer, v: DeviceBuffer, kcache: DeviceBuffer,
                    vcache: DeviceBuffer, n: int, n_head: int, n_kv: int, head_dim: int, n_rot: int, base: float,
                    capacity: int, position: DeviceBuffer, q_offset=0, k_offset=0, v_offset=0):
        _check(lib().q8_rope_append(self.handle, q.ptr, q_offset, k.ptr, k_offset, v.ptr, v_offset, kcache.ptr,
                                    vcache.ptr, n, n_head, n_kv, head_dim, n_rot, float(base), capacity,
                                    position.ptr))

    def attention(self, q: DeviceBuffer, kcache: DeviceBuffer, vcache: DeviceBuffer, out: DeviceBuffer, n: int,
                  n_head: int, n_kv: int, head_dim: int, capacity: int, scale: float, position: DeviceBuffer,
                  splits: int = 1, q_offset=0, out_offset=0):
        _check(lib().q8_attention(self.handle, q.ptr, q_offset, kcache.ptr, vcache.ptr, out.ptr, out_offset, n,
                                  n_head, n_kv, head_dim, capacity, float(scale), position.ptr, splits))

    def attention_matmul_add(self, q: DeviceBuffer, kcache: DeviceBuffer, vcache: DeviceBuffer, n_head: int,
                             n_kv: int, head_dim: int, capacity: int, scale: float, position: DeviceBuffer,
                             splits: int, wo: Weight, y: DeviceBuffer, q_offset: int = 0, y_offset: int = 0):
        """One token's attention then y += wo . attn (the split combine folded
        into the GEMV's prologue)."""
        _check(lib().q8_attention_matmul_add(self.handle, q.ptr, q_offset, kcache.ptr, vcache.ptr, n_head, n_kv,
                                             head_dim, capacity, float(scale), position.ptr, splits,
                                             self.resident(wo), y.ptr, y_offset))

    def attention_prepare(self, q: DeviceBuffer, kcache: DeviceBuffer, vcache: DeviceBuffer, n: int, n_head: int,
                          n_kv: int, head_dim: int, capacity: int, scale: float, position: DeviceBuffer,
                          q_offset: int = 0) -> Prepared:
        """Prompt attention with its output as prepared Q8_0 activations."""
        p = Prepared()
        _check(lib().q8_attention_prepare(self.handle, q.ptr, q_offset, kcache.ptr, vcache.ptr, n, n_head, n_kv,
                                          head_dim, capacity, float(scale), position.ptr, ctypes.byref(p)))
        return p

    def prompt_qkv_rope(self, wq: Weight, wk: Weight, wv: Weight, prepared: Prepared, n: int, q: DeviceBuffer,
                        kcache: DeviceBuffer, vcache: DeviceBuffer, n_head: int, n_kv: int, head_dim: int, n_rot: int,
                        base: float, capacity: int, position: DeviceBuffer, q_offset: int = 0):
        """The q, k, v prompt GEMM with RoPE + KV append in its epilogue."""
        _check(lib().q8_prompt_qkv_rope(self.handle, self.resident(wq), self.resident(wk), self.resident(wv),
                                        ctypes.byref(prepared), n, q.ptr, q_offset, kcache.ptr, vcache.ptr, n_head,
                                        n_kv, head_dim, n_rot, float(base), capacity, position.ptr))

    def embeddings_device(self, weight, tokens: DeviceBuffer, n: int, out: DeviceBuffer, out_offset: int = 0):
        _check(lib().q8_embeddings_device(self.handle, self.resident(weight), tokens.ptr, n, out.ptr, out_offset))

    def norm_lm_head_argmax(self, weight, eps: float, lm_head: Weight, x: DeviceBuffer, x_offset: int,
                            logits: DeviceBuffer, logits_offset: int, result: DeviceBuffer):
        """Output norm (weight None: none) + lm_head GEMV + greedy argmax into device memory."""
        w = self._norm_weight(weight).ctypes.data if weight is not None else None
        _check(lib().q8_norm_lm_head_argmax(self.handle, w, float(eps), self.resident(lm_head), x.ptr, x_offset,
                                            logits.ptr, logits_offset, result.ptr))

    def argmax_device(self, values: DeviceBuffer, offset: int, length: int, result: DeviceBuffer):
        _check(lib().q8_argmax_device(self.handle, values.ptr, offset, length, result.ptr))

    def advance_position(self, position: DeviceBuffer, by: int):
        _check(lib().q8_advance_position(self.handle, position.ptr, by))

    def argmax(self, values: DeviceBuffer, offset: int, length: int) -> int:
        out = ctypes.c_uint32()
        _check(lib().q8_argmax(self.handle, values.ptr, offset, length, ctypes.byref(out)))
        return int(out.value)

    def copy(self, dst: DeviceBuffer, src: DeviceBuffer, nbytes: int):
        _check(lib().q8_copy_device(self.handle, dst.ptr, src.ptr, nbytes))

    def plan(self, n: int, out: int, k: int) -> dict:
        return plan(n, out, k, self)

    def stream(self) -> int:
        """The context's HIP stream (q8_stream)."""
        return lib().q8_stream(self.handle)

    # ---- timing and graphs ----
    def event(self):
        e = ctypes.c_void_p()
        _check(lib().q8_event_create(self.handle, ctypes.byref(e)))
        return e.value

    def record(self, event):
        _check(lib().q8_event_record(self.handle, event))

    @staticmethod
    def elapsed_ms(start, end) -> float:
        ms = ctypes.c_float()
        _check(lib().q8_event_elapsed_ms(start, end, ctypes.byref(ms)))
        return float(ms.value)

    @staticmethod
    def destroy_event(event):
        _check(lib().q8_event_destroy(event))

    def graph_begin(self):
        _check(lib().q8_graph_begin(self.handle))

    def graph_end(self):
        g = ctypes.c_void_p()
        _check(lib().q8_graph_end(self.handle, ctypes.byref(g)))
        return g.value

    def graph_launch(self, graph):
        _check(lib().q8_graph_launch(self.handle, graph))

    @staticmethod
    def graph_destroy(graph):
        _check(lib().q8_graph_destroy(graph))


@dataclass
class GroupMember:
    """compute.rs:62-66: one matmul of a group sharing its activations."""
    weight: Weight
    out: DeviceBuffer
    out_offset: int = 0


class Compute:
    """The matmul surface of the reference's ``Compute`` on the device
    (compute.rs:376-581, 931-1019).  Activations are device buffers of f32;
    offsets and lengths are in f32 elements, as in the reference."""

    # Below this many tokens the reference's prepare is a no-op (tactics.rs:194);
    # here every n >= 2 runs the quantized GEMM, so preparing pays from n = 2.
    prepare_min_tokens = 2

    def __init__(self, gpu: Gpu):
        self.gpu = gpu

    def device_name(self) -> str:
        return self.gpu.name

    def alloc(self, length: int) -> DeviceBuffer:
        return self.gpu.alloc(4 * int(length))

    def upload(self, buf: DeviceBuffer, values: np.ndarray):
        buf.upload(np.ascontiguousarray(values, dtype=np.float32))

    def download(self, buf: DeviceBuffer, out: np.ndarray):
        out[...] = buf.download(np.float32, out.size).reshape(out.shape)

    def prepare(self, x, x_offset, n, k):
        if n < self.prepare_min_tokens:
            return None
        return self.gpu.prepare(x, x_offset, n, k)

    def matmul(self, weight, x, x_offset, n, y, y_offset):
        self.gpu.matmul(weight, x, x_offset, n, y, y_offset)

    def matmul_prepared(self, weight, x, x_offset, prepared, n, y, y_offset):
        self.gpu.matmul(weight, x, x_offset, n, y, y_offset, prepared=prepared)

    def matmul_prepared_group(self, members, x, x_offset, prepared, n):
        """compute.rs:437-472: one launch for up to four matrices."""
        k = members[0].weight.k
        entries = [(m.weight, m.out, m.out_offset) for m in members]
        if n == 1:
            self.gpu.matmul_decode_group(entries, x, x_offset, k)
        else:
            if prepared is None:
                prepared = self.gpu.prepare(x, x_offset, n, k)
            self.gpu.matmul_prompt_group(entries, prepared, n, k)

    def matmul_add(self, weight, x, x_offset, prepared, n, y, y_offset, temp=None):
        """compute.rs:537-581: y += W x with the residual in the epilogue."""
        self.gpu.matmul(weight, x, x_offset, n, y, y_offset, prepared=prepared, bias=y, bias_offset=y_offset)

    def silu_mul(self, act, gate, up, length):
        self.gpu.silu_mul(act, gate, up, length)

    def embeddings(self, weight, tokens, out, out_offset):
        """compute.rs:346-371 (device branch): the embedding rows of `tokens`."""
        self.gpu.embeddings(weight, tokens, out, out_offset)

    def rmsnorm(self, x, x_offset, weight, eps, rows, out, out_offset):
        """compute.rs:584-614."""
        self.gpu.rmsnorm(x, x_offset, weight, eps, rows, out, out_offset)

    def norm_prepare(self, x, x_offset, weight, eps, rows, out, out_offset):
        """compute.rs:959-984: quantized rmsnorm rows, or below the threshold
        the f32 norm written to `out` and no prepared buffer."""
        if rows < self.prepare_min_tokens:
            self.gpu.rmsnorm(x, x_offset, weight, eps, rows, out, out_offset)
            return None
        return self.gpu.norm_prepare(x, x_offset, weight, eps, rows)

    def silu_mul_prepare(self, act, gate, up, n, k):
        """compute.rs:993-1019."""
        if n < self.prepare_min_tokens:
            self.gpu.silu_mul(act, gate, up, n * k)
            return None
        return self.gpu.silu_mul_prepare(gate, up, n, k)
