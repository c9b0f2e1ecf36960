// q8_runtime.cpp -- host side of libq8mi.so: the C-ABI of include/q8mi.h over
// the HIP runtime.
//
// Structure follows the reference's device runtime `Gpu`
// (apps/engine/src/cuda/mod.rs): one context with one stream, a module loaded
// from an embedded code object (cuModuleLoadData of embedded PTX,
// cuda/mod.rs:406-411 -> hipModuleLoadData of an embedded gfx950 code object),
// a weight residency cache keyed by the host slice identity
// (cuda/mod.rs:1769-1790), a growing activation workspace for prepared
// activations (cuda/mod.rs:1629-1645), and launches through
// hipModuleLaunchKernel (cuda/mod.rs:1819-1902).  Before every launch the
// operand spans are checked on the host against the allocations this context
// made, so a wrong shape is an error here and never an out-of-bounds access on
// the device.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/q8decoder.h"
#include "../../include/q8mi.h"
#include "q8_internal.h"
#include "q8_layout.h"
#include "q8_manifest.h"
#include "q8_tactics.h"

extern "C" const unsigned char q8_code_object[];
extern "C" const unsigned char q8_code_object_end[];

namespace {

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int hip_fail(hipError_t e, const char *op) {
    return fail(e == hipErrorOutOfMemory ? Q8_ERR_OUT_OF_MEMORY : Q8_ERR_HIP, "hip: %s failed: %s", op,
                hipGetErrorString(e));
}

#define HIP_TRY(call, op)                             \
    do {                                              \
        hipError_t e_ = (call);                       \
        if (e_ != hipSuccess) return hip_fail(e_, op); \
    } while (0)

#define Q8_TRY(call)          \
    do {                      \
        int rc_ = (call);     \
        if (rc_ != Q8_OK) return rc_; \
    } while (0)

enum Fn {
    F_REPACK,
    F_GEMV_2_0, F_GEMV_2_1, F_GEMV_3_0, F_GEMV_3_1, F_GEMV_5_0, F_GEMV_5_1, F_GEMV_9_0, F_GEMV_9_1,
    F_GEMV1_2_0, F_GEMV1_2_1, F_GEMV1_3_0, F_GEMV1_3_1, F_GEMV1_5_0, F_GEMV1_5_1, F_GEMV1_9_0, F_GEMV1_9_1,
    F_GEMVC_2_0, F_GEMVC_2_1, F_GEMVC_3_0, F_GEMVC_3_1, F_GEMVC_5_0, F_GEMVC_5_1, F_GEMVC_9_0, F_GEMVC_9_1,
    F_GEMV_R8_3, F_GEMV_R8_6, F_GEMV_R16_3, F_GEMV_R16_6,
    F_GEMV_RC8_3, F_GEMV_RC8_6, F_GEMV_RC16_3, F_GEMV_RC16_6,
    F_GEMV_R8_3_E0, F_GEMV_R8_6_E0, F_GEMV_R16_3_E0, F_GEMV_R16_6_E0,
    F_GEMV_RC8_3_E0, F_GEMV_RC8_6_E0, F_GEMV_RC16_3_E0, F_GEMV_RC16_6_E0,
    F_GEMV_G8_3, F_GEMV_G16_3, F_GEMV_G16_6, F_GEMV_S8_3, F_GEMV_S16_6,
    F_GEMV_G8_3_E0, F_GEMV_G16_3_E0, F_GEMV_G16_6_E0, F_GEMV_S8_3_E0, F_GEMV_S16_6_E0,
    F_GEMV_Q8X1_8_3, F_GEMV_Q8X1_8_6, F_GEMV_Q8X1_16_3, F_GEMV_Q8X1_16_6,
    F_GEMV_Q8X2_8_3, F_GEMV_Q8X2_8_6, F_GEMV_Q8X2_16_3, F_GEMV_Q8X2_16_6,
    F_GEMV_R8_2, F_GEMV_RC8_2, F_GEMV_R8_2_E0, F_GEMV_RC8_2_E0, F_GEMV_Q8X1_8_2, F_GEMV_Q8X2_8_2,
    F_GEMM_S1_T1S,
    F_QUANTIZE,
    F_GEMM_S0_T1, F_GEMM_S1_T1, F_GEMM_S1_T2, F_GEMM_S1_T4,
    F_GEMM_H_T1_R4, F_GEMM_H_T2_R2, F_GEMM_H_T2_R4,
    F_GEMM_P_T1, F_GEMM_P_T2,
    F_GEMM_L_T1_R2, F_GEMM_L_T2_R2, F_GEMM_L_T2_R4,
    F_GEMM_SILU,
    F_RMSNORM, F_RMSNORM_ROW,
    F_ARGMAX,
    F_SILU_MUL,
    F_COPY,
    F_EMBED,
    F_ROPE, F_ATTN_DECODE, F_ATTN_DECODE_W4, F_ATTN_PREFILL, F_SYNTH, F_ADVANCE,
    F_SLICE_COPY,
    F_GEMV_HG8_3, F_GEMV_HG16_3, F_GEMV_HG16_6, F_GEMV_HS8_3, F_GEMV_HS16_6,
    F_GEMV_HG8_3_E0, F_GEMV_HG16_3_E0, F_GEMV_HG16_6_E0, F_GEMV_HS8_3_E0, F_GEMV_HS16_6_E0,
    F_GEMV_HP16_3, F_GEMV_HP16_6, F_GEMV_HP16_3_E0, F_GEMV_HP16_6_E0,
    F_ATTN_DECODE_W8,
    F_COUNT
};

const char *const kFnNames[F_COUNT] = {
    "q8_repack",
    "q8_gemv_pb2_e0", "q8_gemv_pb2_e1", "q8_gemv_pb3_e0", "q8_gemv_pb3_e1",
    "q8_gemv_pb5_e0", "q8_gemv_pb5_e1", "q8_gemv_pb9_e0", "q8_gemv_pb9_e1",
    "q8_gemv1_pb2_e0", "q8_gemv1_pb2_e1", "q8_gemv1_pb3_e0", "q8_gemv1_pb3_e1",
    "q8_gemv1_pb5_e0", "q8_gemv1_pb5_e1", "q8_gemv1_pb9_e0", "q8_gemv1_pb9_e1",
    "q8_gemvc_pb2_e0", "q8_gemvc_pb2_e1", "q8_gemvc_pb3_e0", "q8_gemvc_pb3_e1",
    "q8_gemvc_pb5_e0", "q8_gemvc_pb5_e1", "q8_gemvc_pb9_e0", "q8_gemvc_pb9_e1",
    "q8_gemv_r8_l3", "q8_gemv_r8_l6", "q8_gemv_r16_l3", "q8_gemv_r16_l6",
    "q8_gemv_rc8_l3", "q8_gemv_rc8_l6", "q8_gemv_rc16_l3", "q8_gemv_rc16_l6",
    "q8_gemv_r8_l3_e0", "q8_gemv_r8_l6_e0", "q8_gemv_r16_l3_e0", "q8_gemv_r16_l6_e0",
    "q8_gemv_rc8_l3_e0", "q8_gemv_rc8_l6_e0", "q8_gemv_rc16_l3_e0", "q8_gemv_rc16_l6_e0",
    "q8_gemv_g8_l3", "q8_gemv_g16_l3", "q8_gemv_g16_l6", "q8_gemv_s8_l3", "q8_gemv_s16_l6",
    "q8_gemv_g8_l3_e0", "q8_gemv_g16_l3_e0", "q8_gemv_g16_l6_e0", "q8_gemv_s8_l3_e0", "q8_gemv_s16_l6_e0",
    "q8_gemv_q8x1_r8_l3", "q8_gemv_q8x1_r8_l6", "q8_gemv_q8x1_r16_l3", "q8_gemv_q8x1_r16_l6",
    "q8_gemv_q8x2_r8_l3", "q8_gemv_q8x2_r8_l6", "q8_gemv_q8x2_r16_l3", "q8_gemv_q8x2_r16_l6",
    "q8_gemv_r8_l2", "q8_gemv_rc8_l2", "q8_gemv_r8_l2_e0", "q8_gemv_rc8_l2_e0", "q8_gemv_q8x1_r8_l2",
    "q8_gemv_q8x2_r8_l2",
    "q8_gemm_s1_t1s",
    "q8_quantize",
    "q8_gemm_s0_t1", "q8_gemm_s1_t1", "q8_gemm_s1_t2", "q8_gemm_s1_t4",
    "q8_gemm_h_t1_r4", "q8_gemm_h_t2_r2", "q8_gemm_h_t2_r4",
    "q8_gemm_p_t1", "q8_gemm_p_t2",
    "q8_gemm_l_t1_r2", "q8_gemm_l_t2_r2", "q8_gemm_l_t2_r4",
    "q8_gemm_silu",
    "q8_rmsnorm", "q8_rmsnorm_row",
    "q8_argmax",
    "q8_silu_mul",
    "q8_copy",
    "q8_embed",
    "q8_rope_append", "q8_attn_decode", "q8_attn_decode_w4", "q8_attn_prefill", "q8_synth", "q8_advance",
    "q8_slice_copy",
    "q8_gemv_hg8_l3", "q8_gemv_hg16_l3", "q8_gemv_hg16_l6", "q8_gemv_hs8_l3", "q8_gemv_hs16_l6",
    "q8_gemv_hg8_l3_e0", "q8_gemv_hg16_l3_e0", "q8_gemv_hg16_l6_e0", "q8_gemv_hs8_l3_e0", "q8_gemv_hs16_l6_e0",
    "q8_gemv_hp16_l3", "q8_gemv_hp16_l6", "q8_gemv_hp16_l3_e0", "q8_gemv_hp16_l6_e0",
    "q8_attn_decode_w8",
};

// Every kernel of the code object with its metadata (q8_manifest.h, from the
// code object's AMDGPU note at build time).
const q8i::KernelMeta kKernelMeta[] = {Q8_KERNEL_META};

const q8i::KernelMeta *find_meta(const char *name) {
    for (const q8i::KernelMeta &m : kKernelMeta)
        if (std::strcmp(m.name, name) == 0) return &m;
    return nullptr;
}

// A launch the kernel cannot take is refused before it reaches the device,
// as the reference refuses launch shapes its kernels' attributes do not
// allow (cuda/mod.rs:229-283) and checks a launch's argument count against
// the kernel (cuda/mod.rs:1835-1848): the host's argument block must be
// exactly the kernel's explicit arguments (every kernel here takes one
// struct by value), the workgroup a whole number of waves within the
// kernel's compiled bound, and static plus dynamic LDS within the device's.
int check_launch(const q8i::KernelMeta &m, size_t args_size, unsigned block, size_t dynamic_lds,
                 size_t lds_limit) {
    if (args_size != m.args)
        return fail(Q8_ERR_INVALID, "launch of %s: a %zu-byte argument block for %u bytes of kernel arguments",
                    m.name, args_size, m.args);
    if (block == 0 || block % 64 != 0 || block > m.max_wg)
        return fail(Q8_ERR_INVALID, "launch of %s: %u threads per workgroup (whole waves, at most %u)", m.name, block,
                    m.max_wg);
    if (m.lds + dynamic_lds > lds_limit)
        return fail(Q8_ERR_UNSUPPORTED, "launch of %s: %u + %zu bytes of LDS, the device allows %zu", m.name, m.lds,
                    dynamic_lds, lds_limit);
    return Q8_OK;
}

constexpr int kArgmaxParts = 1024;
// Partials the argmax workspace holds: the lm_head GEMV writes one per 32-row
// tile (122880 rows: 3840), the two-stage argmax kArgmaxParts.
constexpr int kArgmaxMaxParts = 65536;
// Split-K scratch, allocated once at open: 32 MiB of partial results and
// 65536 arrival counters (zeroed once; each launch's last workgroup re-zeroes
// the counters it used, so no memset is ever recorded into a graph).
constexpr size_t kSplitBytes = 32u << 20;
constexpr int kCounters = 65536;
// Decode attention's per-head arrival counters live at the top of the same
// array (the matmul split-K paths index from the bottom; launches on the one
// stream never overlap, and each resets what it used).
constexpr int kAttnCounterBase = 61440;
constexpr size_t kAlign = 256;

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
long long ceil_div(long long a, long long b) { return (a + b - 1) / b; }

}  // namespace

struct q8_weight {
    q8_ctx *ctx;
    void *base;
    uint8_t *quants;
    uint16_t *scales;
    int k, out, nb, tiles;
    size_t device_bytes;
    uintptr_t id_ptr;
    size_t id_len;
    uint8_t *slices = nullptr;  // slice-major copy of the quants (Q8SliceArgs), or none
    int slice_rows = 0;         // its rows per slice: 8 or 16
    int *group_refs = nullptr;  // a member of a contiguous group: the members still holding `base`
    uint8_t *pair_slices = nullptr;  // the gate of a contiguous gate/up pair: the pair's paired copy (Q8SliceArgs)
};

struct q8_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipModule_t module = nullptr;
    hipFunction_t fn[F_COUNT] = {};
    const q8i::KernelMeta *meta[F_COUNT] = {};
    std::recursive_mutex mu;
    std::map<std::pair<uintptr_t, size_t>, q8_weight *> weights;
    std::map<std::pair<uintptr_t, size_t>, float *> vectors;  // resident f32 norm weights, by host identity
    std::map<std::pair<int, uint32_t>, float *> rope_freq;    // rotation frequencies by (n_rot, bits of base)
    std::map<uintptr_t, size_t> allocs;  // buffers from q8_alloc, for span checks
    void *act_ws = nullptr;              // prepared activations
    size_t act_ws_bytes = 0;
    void *tmp_ws = nullptr;              // gate/up f32 products of the n >= 2 FFN pair
    size_t tmp_ws_bytes = 0;
    void *act2_ws = nullptr;             // prepared silu(gate) * up written by the fused gate/up GEMM
    size_t act2_ws_bytes = 0;
    void *norm_ws = nullptr;             // rmsnorm(x) when a norm cannot fold into the decode GEMV
    size_t norm_ws_bytes = 0;
    void *argmax_ws = nullptr;           // per-workgroup partials + result
    void *noalloc = nullptr;             // this device's static scratch of q8_matmul_noalloc (not owned)
    float *split_ws = nullptr;           // partial results of split-K workgroups
    unsigned *counters = nullptr;        // split-K arrival counters (kernels reset them to 0)
    void *token_ws = nullptr;            // token ids of the embedding lookup
    size_t token_ws_bytes = 0;
    void *attn_ws = nullptr;             // decode attention partials (acc, max, sum per head and split)
    size_t attn_ws_bytes = 0;
    void *attn_out_ws = nullptr;         // attention output when q8_attention_matmul_add runs two steps
    size_t attn_out_ws_bytes = 0;
    std::vector<q8_weight *> owned;      // weights generated on the device (no host identity)
    unsigned long long ws_generation = 0; // bumped whenever a workspace is reallocated
    unsigned long long allocations = 0;   // device allocations made through dev_malloc
    void *arena = nullptr;                // one allocation holding every planned workspace
    size_t arena_bytes = 0;
    struct Region {
        const char *name;
        size_t offset, bytes;
    };
    std::vector<Region> regions;          // the arena's layout, as planned
    int cu_count = 0;
    size_t total_mem = 0;
    size_t max_lds = 0;
    char name[256] = {};
    std::map<std::string, int> options;
    std::vector<const q8_weight *> next_weights;  // q8_gemm_prefetch: read by the next GEMM's riders
};

namespace {

// [p, p + bytes) must lie inside one buffer this context allocated, when p is
// one of ours; foreign pointers (a caller's own allocations) are not tracked.
int check_span(q8_ctx *c, q8_dptr p, size_t bytes, const char *what) {
    if (p == 0) return fail(Q8_ERR_INVALID, "%s: null device pointer", what);
    auto it = c->allocs.upper_bound((uintptr_t)p);
    if (it == c->allocs.begin()) return Q8_OK;
    --it;
    const uintptr_t base = it->first;
    const size_t size = it->second;
    if ((uintptr_t)p >= base + size) return Q8_OK;  // not inside a tracked buffer
    if ((uintptr_t)p + bytes > base + size)
        return fail(Q8_ERR_INVALID, "%s: %zu bytes at offset %zu overrun a %zu-byte buffer", what, bytes,
                    (size_t)((uintptr_t)p - base), size);
    return Q8_OK;
}

int option(q8_ctx *c, const char *name, int fallback) {
    auto it = c->options.find(name);
    return (it == c->options.end() || it->second < 0) ? fallback : it->second;
}

// The row-slice GEMVs' leading scalar arguments, in the kernels' parameter
// order (the RsHot the kernels rebuild from them), then the argument block at
// the next 8-byte boundary: the kernel's explicit arguments span
// sizeof(RsHead) + sizeof(Q8GemvArgs).
struct RsHead {
    const uint8_t *mq;
    const uint16_t *msc;
    float *my;
    const float *mbias;
    const float *xg;
    int mrows, nbw, tiles_xo, ms_off;
};
static_assert(sizeof(RsHead) == 56, "row-slice head: five pointers and four ints");

int launch_rs(q8_ctx *c, Fn f, unsigned grid, unsigned block, unsigned lds, RsHead &h, Q8GemvArgs &a) {
    if (grid == 0) return Q8_OK;
    Q8_TRY(check_launch(*c->meta[f], sizeof(RsHead) + sizeof(Q8GemvArgs), block, lds, c->max_lds));
    void *params[] = {&h.mq, &h.msc, &h.my, &h.mbias, &h.xg, &h.mrows, &h.nbw, &h.tiles_xo, &h.ms_off, &a};
    HIP_TRY(hipModuleLaunchKernel(c->fn[f], grid, 1, 1, block, 1, 1, lds, c->stream, params, nullptr),
            kFnNames[f]);
    return Q8_OK;
}

// The contiguous-group row-slice GEMVs' preloaded head (RsgHot in
// q8_kernels.hip): the group's load bases, x, the norm weight and the RoPE
// position, then nb | waves per slot << 16, total tiles | slice_major << 30 |
// xcd_order << 31 and the up member's first tile.
struct RsgHead {
    const uint8_t *mq;
    const uint16_t *msc;
    const float *xg;
    const float *norm_w;
    const int *rope_pos;
    int nbw, tiles_xo, up_off, hpad;
};
static_assert(sizeof(RsgHead) == 56, "group row-slice head: five pointers and four ints");

int launch_rsg(q8_ctx *c, Fn f, unsigned grid, unsigned block, unsigned lds, RsgHead &h, Q8GemvArgs &a) {
    if (grid == 0) return Q8_OK;
    Q8_TRY(check_launch(*c->meta[f], sizeof(RsgHead) + sizeof(Q8GemvArgs), block, lds, c->max_lds));
    void *params[] = {&h.mq, &h.msc, &h.xg, &h.norm_w, &h.rope_pos, &h.nbw, &h.tiles_xo, &h.up_off, &h.hpad, &a};
    HIP_TRY(hipModuleLaunchKernel(c->fn[f], grid, 1, 1, block, 1, 1, lds, c->stream, params, nullptr),
            kFnNames[f]);
    return Q8_OK;
}

int launch(q8_ctx *c, Fn f, unsigned grid, unsigned block, unsigned lds, void *args, size_t args_size) {
    if (grid == 0) return Q8_OK;
    Q8_TRY(check_launch(*c->meta[f], args_size, block, lds, c->max_lds));
    void *params[] = {args};  // every other kernel takes one argument block by value
    HIP_TRY(hipModuleLaunchKernel(c->fn[f], grid, 1, 1, block, 1, 1, lds, c->stream, params, nullptr),
            kFnNames[f]);
    return Q8_OK;
}

// Every device allocation of the context goes through here and is counted
// (q8_workspace_query): a caller that planned its workspaces can check that
// its token path allocates nothing.
hipError_t dev_malloc(q8_ctx *c, void **p, size_t bytes) {
    const hipError_t e = hipMalloc(p, bytes);
    if (e == hipSuccess) c->allocations++;
    return e;
}

bool in_arena(const q8_ctx *c, const void *p) {
    const uintptr_t a = (uintptr_t)c->arena, q = (uintptr_t)p;
    return c->arena && q >= a && q < a + c->arena_bytes;
}

// A workspace too small for `need` moves to an allocation of its own (the
// arena region it may have held stays reserved until the next plan).
int grow(q8_ctx *c, void **buf, size_t *have, size_t need, const char *what) {
    if (*have >= need) return Q8_OK;
    if (*buf) {
        HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        if (!in_arena(c, *buf)) HIP_TRY(hipFree(*buf), "hipFree");
        *buf = nullptr;
        *have = 0;
    }
    c->ws_generation++;  // graphs captured over the old buffer must not be replayed
    const size_t bytes = align_up(need, 1 << 20);
    HIP_TRY(dev_malloc(c, buf, bytes), what);
    *have = bytes;
    return Q8_OK;
}

// Prepared-activation format for n tokens: the tactic table's choice, or the
// "gemm.f16" option (0: always int8, 1: f16 whenever n >= 2).
int prepared_format(q8_ctx *c, int n) {
    const int f = option(c, "gemm.f16", -1);
    if (f == 0 || n < 2) return Q8_PREPARED_I8;
    if (f == 1) return Q8_PREPARED_F16;
    return q8_tactics_prepared_format(n);
}

// fmt >= 0: a GEMM plan for prepared activations of that format (the kernel
// family follows the operand's format).
q8_tactic plan(q8_ctx *c, int n, int out, int k, int slots = 1, int fmt = -1) {
    q8_tactic t{};
    q8_tactics_choose(n, out, k, c->cu_count, &t);
    if (fmt == Q8_PREPARED_F16 && t.kernel != Q8_KERNEL_GEMM_F16)
        q8_tactics_for_kernel(Q8_KERNEL_GEMM_F16, n, out, k, c->cu_count, &t);
    else if (fmt == Q8_PREPARED_I8 && t.kernel != Q8_KERNEL_GEMM)
        q8_tactics_for_kernel(Q8_KERNEL_GEMM, n, out, k, c->cu_count, &t);
    if (t.kernel == Q8_KERNEL_GEMM_F16) {
        const int npairs = (k / 32 + 1) / 2;
        const int ttiles = (int)ceil_div(n, 32);
        const int tpw = option(c, "gemm.tpw", -1);
        const int rw = option(c, "gemm.rwaves", -1);
        const int kw = option(c, "gemm.kwaves", -1);
        t.xcd_remap = option(c, "gemm.xcd_remap", t.xcd_remap) ? 1 : 0;
        if (tpw > 0) t.tpw = (tpw >= 2 && ttiles >= 2) ? 2 : 1;
        if (rw > 0) t.rwaves = rw >= 4 ? 4 : 2;
        if (t.tpw == 1) t.rwaves = 4;  // built variants: t1_r4, t2_r2, t2_r4
        if (tpw > 0 || rw > 0 || kw > 0) {
            int kws = kw > 0 ? kw : t.kwaves;
            const int lds_kw = (int)(c->max_lds / ((size_t)Q8_GEMM_H_STAGES * Q8_GEMM_H_BUF_BYTES(t.tpw, t.rwaves)));
            kws = std::max(1, std::min(std::min(std::min(kws, 8 / t.rwaves), npairs), lds_kw));
            t.pairs_per_wave = (int)ceil_div(npairs, kws);
            t.kwaves = (int)ceil_div(npairs, t.pairs_per_wave);
        }
        return t;
    }
    if (t.kernel == Q8_KERNEL_GEMV) {
        if (slots != 1) q8_gemv_shape(out, k, c->cu_count, slots, &t);
        const int nb = k / 32;
        const int npairs = (nb + 1) / 2;
        t.exact = option(c, "gemv.exact", t.exact) ? 1 : 0;
        const int sl = option(c, "gemv.slices", -1);
        if (sl > 0) t.kslices = std::min(sl, npairs);
        const int pps = (int)ceil_div(npairs, t.kslices);
        t.kslices = (int)ceil_div(npairs, pps);
        const int w = option(c, "gemv.waves", -1);
        if (w > 0 || sl > 0) {
            int ww = w > 0 ? std::min(w, pps) : std::min(t.waves_per_tile, pps);
            t.pairs_per_wave = (int)ceil_div(pps, ww);
            t.waves_per_tile = (int)ceil_div(pps, t.pairs_per_wave);
        }
        const int pb = option(c, "gemv.pairs", -1);
        if (pb > 0) t.pairs_per_batch = pb;
        // the tile kernel's own switches select the tile kernel
        if (w > 0 || sl > 0 || pb > 0 || t.kslices != 1) {
            t.row_slice = Q8_TILE_ROWS;
            t.slice_loads = 0;
        }
        const int rows = option(c, "gemv.rows", -1);
        if (rows > 0) t.row_slice = rows;
        if (t.row_slice != Q8_TILE_ROWS) {
            const int loads = option(c, "gemv.loads", -1);
            if (loads > 0) t.slice_loads = loads;
            if (t.slice_loads != 2 && t.slice_loads != 3 && t.slice_loads != 6) t.slice_loads = 6;
            if (t.slice_loads == 2 && t.row_slice != 8) t.slice_loads = 3;  // two loads: 8-row slices only
        }
    } else {
        t.smode = option(c, "gemm.smode", t.smode) ? 1 : 0;
        t.xcd_remap = option(c, "gemm.xcd_remap", t.xcd_remap) ? 1 : 0;
        t.pipe = option(c, "gemm.pipe", t.pipe) ? 1 : 0;
        if (option(c, "gemm.lds", t.rwaves > 0 ? 1 : 0)) {
            // the int8 units staged in LDS (q8_gemm_l): its own launch shape
            q8_tactic l = t;
            q8_gemm_staged_shape(n, out, k, c->cu_count, 1, &l);
            const int tpw = option(c, "gemm.tpw", -1);
            const int rw = option(c, "gemm.rwaves", -1);
            const int kw = option(c, "gemm.kwaves", -1);
            const int ttiles = (int)ceil_div(n, 32);
            const int npairs = (k / 32 + 1) / 2;
            if (tpw > 0) l.tpw = (tpw >= 2 && ttiles >= 2) ? 2 : 1;
            if (rw > 0) l.rwaves = rw >= 4 ? 4 : 2;
            if (l.tpw == 1) l.rwaves = 2;  // built variants: t1_r2, t2_r2, t2_r4
            if (tpw > 0 || rw > 0 || kw > 0) {
                int kws = kw > 0 ? kw : l.kwaves;
                const int lds_kw = (int)(c->max_lds / ((size_t)Q8_GEMM_H_STAGES * Q8_GEMM_L_BUF_BYTES(l.tpw, l.rwaves)));
                kws = std::max(1, std::min(std::min(std::min(kws, 8 / l.rwaves), npairs), lds_kw));
                l.pairs_per_wave = (int)ceil_div(npairs, kws);
                l.kwaves = (int)ceil_div(npairs, l.pairs_per_wave);
            }
            l.pipe = 0;
            l.kslices = 1;
            return l;
        }
        t.rwaves = 0;
        const int tpw = option(c, "gemm.tpw", -1);
        const int tw = option(c, "gemm.twaves", -1);
        const int kw = option(c, "gemm.kwaves", -1);
        int sl = option(c, "gemm.slices", -1);
        if (tpw > 0) t.tpw = (tpw >= 4) ? 4 : (tpw >= 2 ? 2 : 1);
        if (!t.smode) t.tpw = 1;  // the VALU-scale variant is built for one token tile per wave
        if (t.pipe && t.tpw == 4) t.tpw = 2;  // the pipelined kernel is built for one or two
        if (tpw > 0 || tw > 0 || kw > 0 || sl > 0 || !t.smode || t.pipe) {
            const int npairs = (k / 32 + 1) / 2;
            const int ttiles = (int)ceil_div(n, 32);
            const int groups = (int)ceil_div(ttiles, t.tpw);
            const int max_threads = (t.tpw == 1 && !t.pipe) ? 1024 : 512;
            if (t.pipe) sl = 1;
            int twv = tw > 0 ? tw : t.twaves;
            twv = std::max(1, std::min(twv, std::min(groups, max_threads / 64)));
            int kws = kw > 0 ? kw : t.kwaves;
            kws = std::max(1, std::min(kws, max_threads / 64 / twv));
            int s = sl > 0 ? sl : t.kslices;
            s = std::max(1, std::min(s, npairs));
            const int pps = (int)ceil_div(npairs, s);
            s = (int)ceil_div(npairs, pps);
            const int ppw = (int)ceil_div(pps, kws);
            t.twaves = twv;
            t.kslices = s;
            t.pairs_per_wave = ppw;
            t.kwaves = (int)ceil_div(pps, ppw);
        }
    }
    return t;
}

// one: a launch over a single matrix (q8_gemv1_*, no member selection);
// comb: a single matrix whose x is the folded attention combine (q8_gemvc_*).
Fn gemv_fn(int pb, int exact, bool one, bool comb = false) {
    const int base = comb ? F_GEMVC_2_0 : one ? F_GEMV1_2_0 : F_GEMV_2_0;
    const int i = pb == 2 ? 0 : pb == 3 ? 1 : pb == 5 ? 2 : 3;
    return (Fn)(base + 2 * i + (exact ? 1 : 0));
}

int valid_pb(int pb) { return pb == 2 || pb == 3 || pb == 5 || pb == 9; }

struct Member {
    const q8_weight *w;
    float *y;
};

// weight_synthetic_group's slice_rows for a gate/up pair's paired copy.
constexpr int kPairSlices = q8i::kGroupPairSlices;
// Loads a lane of the paired gate/up kernels (q8_gemv_hp16_l3 / _l6) at nb
// blocks a row, at most 16 waves; 0 where neither fits.
int pair_loads(int nb) { return nb <= 96 ? 3 : nb <= 192 ? 6 : 0; }
int build_group(q8_ctx *c, int k, int count, const int *outs, const void *const *bytes, const size_t *nbytes,
                const uint64_t *seeds, float scale_std, int slice_rows, const q8_weight **weights);

// Whether a launch's members lie back to back in one allocation (made by
// group residency, q8i::weight_synthetic_group): member i's quants and
// scales start where member i - 1's tiles end, and so does its slice-major
// copy where every member has one of the same height (*slice_rows, else 0).
// Such a group runs the contiguous-group row-slice kernels unless option
// "gemv.group_hot" is 0.
bool contiguous_group(q8_ctx *c, const Member *m, int count, int *slice_rows) {
    if (count < 2 || !option(c, "gemv.group_hot", 1)) return false;
    const q8_weight *w0 = m[0].w;
    const uintptr_t q0 = (uintptr_t)w0->quants, s0 = (uintptr_t)w0->scales, l0 = (uintptr_t)w0->slices;
    const size_t nb = (size_t)w0->nb;
    size_t t = 0;
    bool sl = w0->slices != nullptr;
    for (int i = 0; i < count; i++) {
        const q8_weight *w = m[i].w;
        if (w->nb != w0->nb || (uintptr_t)w->quants != q0 + t * nb * Q8_UNIT_BYTES ||
            (uintptr_t)w->scales != s0 + t * nb * Q8_TILE_ROWS * 2)
            return false;
        sl = sl && w->slices && w->slice_rows == w0->slice_rows && (uintptr_t)w->slices == l0 + t * nb * Q8_UNIT_BYTES;
        t += (size_t)w->tiles;
    }
    *slice_rows = sl ? w0->slice_rows : 0;
    return true;
}

// n = 1 over up to four weights sharing x; silu = 1 fuses silu(m0)*m1 into y of m0.
// The RoPE + KV append epilogue of a q, k, v decode group.
struct GemvRope {
    const int *position;
    const float *freq;
    uint16_t *kcache, *vcache;
    int head_dim, n_rot, capacity;
};

// Decode attention partials a GEMV prologue combines into its x.
struct GemvCombine {
    const float *acc, *ms;
    int splits;
};

// Row-slice GEMV over one matrix (q8_gemv_r{8,16}_l{3,6}; q8_gemv_rc* with
// x built by the folded attention combine): a workgroup per rs rows of a
// 32-row tile and the whole K range, nl loads per lane, exact block order.
// Returns Q8_ERR_UNSUPPORTED (without recording an error) when K needs more
// than 16 waves, or the combine more splits than it holds, so the caller
// keeps the tile kernel.
int run_gemv_rs(q8_ctx *c, const q8_weight *w, float *y, q8_dptr x, const float *bias, int rs, int nl,
                const GemvCombine *comb, int exact) {
    const int nb = w->nb;
    const int bpw = nl * (64 / (2 * rs));
    const int waves = (int)ceil_div(nb, bpw);
    if (waves > 16) return Q8_ERR_UNSUPPORTED;
    if (comb && (comb->splits < 1 || comb->splits > Q8_ATTN_COMBINE_MAX)) return Q8_ERR_UNSUPPORTED;
    Q8GemvArgs a{};
    a.members = 1;
    a.m[0].quants = w->quants;
    a.m[0].scales = w->scales;
    a.m[0].y = y;
    a.m[0].bias = bias;
    a.m[0].rows = w->out;
    a.total_tiles = w->tiles;
    a.x = reinterpret_cast<const float *>(x);
    a.nb = nb;
    a.waves_per_tile = waves;
    a.kslices = 1;
    if (comb) {
        a.attn_acc = comb->acc;
        a.attn_ms = comb->ms;
        a.attn_splits = comb->splits;
    }
    a.xcd_order = option(c, "gemv.xcd_order", 1) ? 1 : 0;
    const long long grid = (a.xcd_order ? ceil_div(w->tiles, 8) * 8 : (long long)w->tiles) * (Q8_TILE_ROWS / rs);
    if (grid > 0x7fffffffLL) return fail(Q8_ERR_UNSUPPORTED, "gemv: grid of %lld workgroups", grid);
    const unsigned lds = (unsigned)((nb * 32 + rs * Q8_GEMV_VROW(nb) + Q8_GEMV_PAD_FLOATS) * 4);
    Fn f;
    if (nl == 2) {  // built for 8-row slices only
        if (rs != 8) return Q8_ERR_UNSUPPORTED;
        f = exact ? (comb ? F_GEMV_RC8_2 : F_GEMV_R8_2) : (comb ? F_GEMV_RC8_2_E0 : F_GEMV_R8_2_E0);
    } else {
        const int fi = (rs == 8 ? 0 : 2) + (nl == 3 ? 0 : 1);
        f = (Fn)((exact ? (comb ? F_GEMV_RC8_3 : F_GEMV_R8_3) : (comb ? F_GEMV_RC8_3_E0 : F_GEMV_R8_3_E0)) + fi);
    }
    if (nb > 0xffff || w->tiles > 0x3fffffff) return fail(Q8_ERR_UNSUPPORTED, "gemv: %d blocks a row", nb);
    // the weight's slice-major copy where it has one for these slices
    // (option gemv.slice_copy = 0 reads the unit layout instead)
    const bool sm = w->slices && w->slice_rows == rs && option(c, "gemv.slice_copy", 1);
    if (w->out >= (1 << 24)) return fail(Q8_ERR_UNSUPPORTED, "gemv: %d rows in row slices", w->out);
    RsHead h{sm ? w->slices : a.m[0].quants, a.m[0].scales, a.m[0].y, a.m[0].bias, a.x, a.m[0].rows,
             nb | (waves << 16),
             (int)((unsigned)w->tiles | ((unsigned)sm << 30) | ((unsigned)a.xcd_order << 31)), 0};
    if (comb) {
        // the combine's partials in the head: sums in xg, (max, sum) at xg + ms_off, splits above the rows
        const long long off = comb->ms - comb->acc;
        if (off < INT32_MIN || off > INT32_MAX)
            return fail(Q8_ERR_UNSUPPORTED, "gemv: attention partials %lld floats apart", off);
        h.xg = comb->acc;
        h.ms_off = (int)off;
        h.mrows |= comb->splits << 24;
    }
    return launch_rs(c, f, (unsigned)grid, (unsigned)(waves * 64), lds, h, a);
}

// Row-slice shape of a multi-matrix decode launch (q8_gemv_g* for a group,
// q8_gemv_s* for the gate/up pair): rows per slice and loads per lane from
// the options "gemv.group_rows" (8 or 16; unset, 0 or 32: the tile kernel,
// which measured faster on the decode step's QKV and gate/up shapes) and
// "gemv.group_loads".  False when no built variant fits: more than 16 waves, or a folded
// norm without the 256 threads its reduction takes.
// hot: a contiguous group (q8_gemv_hg*, q8_gemv_hs*), whose default is
// 16-row slices: three loads a lane for a group, six for the SiLU pair
// (its two slots share a workgroup); "gemv.group_rows" = 32 keeps the tile
// kernel for it too.
bool rsg_shape(q8_ctx *c, int nb, int silu, bool norm, int *rs, int *nl, int *nw, bool hot = false) {
    int rows = option(c, "gemv.group_rows", -1);
    if (hot && rows < 0) rows = 16;
    if (rows <= 0 || rows == 32) return false;  // default: the tile kernel (faster at the decode shapes)
    int r = rows;
    int l = option(c, "gemv.group_loads", -1);
    if (l <= 0) l = 3;
    if (silu && r == 16) l = 6;  // built pair variants: s8_l3, s16_l6
    if (silu && r == 8) l = 3;
    if (!silu && r == 8) l = 3;  // built group variants: g8_l3, g16_l3, g16_l6
    const int bpw = l * (64 / (2 * r));
    const int waves_slot = (int)ceil_div(nb, bpw);
    const int waves = waves_slot * (silu ? 2 : 1);
    if (waves > 16) return false;
    if (norm && (waves * 64 < 256 || nb * 32 > 1024 * Q8_RSG_NORM_VEC)) return false;
    *rs = r;
    *nl = l;
    *nw = waves_slot;
    return true;
}

// norm_w (device f32[k]) folds rmsnorm(x) * norm_w into a multi-matrix
// launch (the caller checks gemv_folds_norm first); rope turns on the RoPE
// epilogue of a three-member q, k, v group.
// comb builds x from attention partials instead (the caller checks
// gemv_folds_combine first; x is then unused).
// amax: a one-matrix launch also writes each tile's greedy-argmax candidate
// (the tile kernel's epilogue; row slices are not taken).
struct GemvArgmax {
    float *value;
    unsigned *index;
};

int run_gemv(q8_ctx *c, const Member *m, int count, q8_dptr x, int k, const float *bias, int silu,
             const float *norm_w = nullptr, float norm_eps = 0.0f, const GemvRope *rope = nullptr,
             const GemvCombine *comb = nullptr, const GemvArgmax *amax = nullptr) {
    const int nb = k / 32;
    int rows_total = 0;
    Q8GemvArgs a{};
    a.members = count;
    int tile = 0;
    for (int i = 0; i < count; i++) {
        a.m[i].quants = m[i].w->quants;
        a.m[i].scales = m[i].w->scales;
        a.m[i].y = m[i].y;
        a.m[i].bias = (i == 0) ? bias : nullptr;
        a.m[i].rows = m[i].w->out;
        a.m[i].tile_begin = tile;
        tile += m[i].w->tiles;
        rows_total += m[i].w->out;
    }
    const int slots = silu ? 2 : 1;
    const q8_tactic t = plan(c, 1, silu ? m[0].w->out : rows_total, k, slots);
    if (amax && (count != 1 || silu || rope || comb))
        return fail(Q8_ERR_INVALID, "gemv: argmax partials come from one plain matrix");
    if (count == 1 && !silu && !norm_w && !rope && !amax && t.kslices == 1 &&
        (t.row_slice == 8 || t.row_slice == 16)) {
        const int rc = run_gemv_rs(c, m[0].w, m[0].y, x, bias, t.row_slice, t.slice_loads, comb, t.exact);
        if (rc != Q8_ERR_UNSUPPORTED) return rc;
    }
    int rs = 0, nl = 0, nw = 0, group_slices = 0;
    if (silu && !comb && !amax && contiguous_group(c, m, count, &group_slices) && option(c, "gemv.group_pair", 1) &&
        option(c, "gemv.group_rows", -1) < 0) {
        // a contiguous gate/up pair: 16-row slices of 8 gate rows and the same
        // 8 up rows (q8_gemv_hp16_*), from the pair's paired copy where it has one
        int pl = pair_loads(nb);
        const int po = option(c, "gemv.pair_loads", -1);
        if (pl && po > 0 && ceil_div(nb, 2 * po) <= 16) pl = po;
        const int pw = pl ? (int)ceil_div(nb, 2 * pl) : 0;
        const int total = m[0].w->tiles;
        if (pl && (!norm_w || (pw * 64 >= 256 && nb * 32 <= 1024 * Q8_RSG_NORM_VEC)) && nb <= 0xffff &&
            total <= 0x3fffffff) {
            a.total_tiles = total;
            a.x = reinterpret_cast<const float *>(x);
            a.nb = nb;
            a.waves_per_tile = pw;
            a.silu_pair = 1;
            a.kslices = 1;
            a.norm_w = norm_w;
            a.norm_eps = norm_eps;
            a.xcd_order = option(c, "gemv.xcd_order", 1) ? 1 : 0;
            const long long grid = (a.xcd_order ? ceil_div(total, 8) * 8 : (long long)total) * 4;
            if (grid > 0x7fffffffLL) return fail(Q8_ERR_UNSUPPORTED, "gemv: grid of %lld workgroups", grid);
            const unsigned lds =
                (unsigned)((nb * 32 + (t.exact ? 16 * Q8_GEMV_VROW(nb) : pw * 16) + Q8_GEMV_PAD_FLOATS) * 4);
            const Fn f = (Fn)((t.exact ? F_GEMV_HP16_3 : F_GEMV_HP16_3_E0) + (pl == 3 ? 0 : 1));
            const bool sm = m[0].w->pair_slices && option(c, "gemv.slice_copy", 1);
            RsgHead h{sm ? m[0].w->pair_slices : m[0].w->quants, m[0].w->scales, a.x, norm_w, nullptr, nb | (pw << 16),
                      (int)((unsigned)total | ((unsigned)sm << 30) | ((unsigned)a.xcd_order << 31)), total, 0};
            return launch_rsg(c, f, (unsigned)grid, (unsigned)(pw * 64), lds, h, a);
        }
    }
    if ((count > 1 || silu) && !comb && !amax && contiguous_group(c, m, count, &group_slices) &&
        rsg_shape(c, nb, silu, norm_w != nullptr, &rs, &nl, &nw, true)) {
        // a contiguous group: the preloaded-head kernels, reading the group's
        // slice-major copy where it has one of this height
        const int total = silu ? m[0].w->tiles : tile;
        if (nb > 0xffff || total > 0x3fffffff) return fail(Q8_ERR_UNSUPPORTED, "gemv: %d blocks a row", nb);
        a.total_tiles = total;
        a.x = reinterpret_cast<const float *>(x);
        a.nb = nb;
        a.waves_per_tile = nw;
        a.silu_pair = silu;
        a.kslices = 1;
        a.norm_w = norm_w;
        a.norm_eps = norm_eps;
        if (rope) {
            a.rope_pos = rope->position;
            a.rope_freq = rope->freq;
            a.kcache = rope->kcache;
            a.vcache = rope->vcache;
            a.head_dim = rope->head_dim;
            a.n_rot = rope->n_rot;
            a.capacity = rope->capacity;
        }
        a.xcd_order = option(c, "gemv.xcd_order", 1) ? 1 : 0;
        const long long grid = (a.xcd_order ? ceil_div(total, 8) * 8 : (long long)total) * (Q8_TILE_ROWS / rs);
        if (grid > 0x7fffffffLL) return fail(Q8_ERR_UNSUPPORTED, "gemv: grid of %lld workgroups", grid);
        const unsigned lds = (unsigned)((nb * 32 + (t.exact ? slots * rs * Q8_GEMV_VROW(nb) : slots * nw * rs) +
                                         Q8_GEMV_PAD_FLOATS) * 4);
        const int vi = silu ? (rs == 8 ? 3 : 4) : (rs == 8 ? 0 : nl == 3 ? 1 : 2);
        const Fn f = (Fn)((t.exact ? F_GEMV_HG8_3 : F_GEMV_HG8_3_E0) + vi);
        const bool sm = group_slices == rs && option(c, "gemv.slice_copy", 1);
        RsgHead h{sm ? m[0].w->slices : m[0].w->quants, m[0].w->scales, a.x, norm_w, a.rope_pos, nb | (nw << 16),
                  (int)((unsigned)total | ((unsigned)sm << 30) | ((unsigned)a.xcd_order << 31)),
                  silu ? m[0].w->tiles : 0, 0};
        return launch_rsg(c, f, (unsigned)grid, (unsigned)(nw * slots * 64), lds, h, a);
    }
    if ((count > 1 || silu) && !comb && rsg_shape(c, nb, silu, norm_w != nullptr, &rs, &nl, &nw)) {
        a.total_tiles = silu ? m[0].w->tiles : tile;
        a.x = reinterpret_cast<const float *>(x);
        a.nb = nb;
        a.waves_per_tile = nw;
        a.silu_pair = silu;
        a.kslices = 1;
        a.norm_w = norm_w;
        a.norm_eps = norm_eps;
        if (rope) {
            a.rope_pos = rope->position;
            a.rope_freq = rope->freq;
            a.kcache = rope->kcache;
            a.vcache = rope->vcache;
            a.head_dim = rope->head_dim;
            a.n_rot = rope->n_rot;
            a.capacity = rope->capacity;
        }
        a.xcd_order = option(c, "gemv.xcd_order", 1) ? 1 : 0;
        const long long grid =
            (a.xcd_order ? ceil_div(a.total_tiles, 8) * 8 : (long long)a.total_tiles) * (Q8_TILE_ROWS / rs);
        if (grid > 0x7fffffffLL) return fail(Q8_ERR_UNSUPPORTED, "gemv: grid of %lld workgroups", grid);
        const unsigned lds = (unsigned)((nb * 32 + (t.exact ? slots * rs * Q8_GEMV_VROW(nb) : slots * nw * rs) +
                                         Q8_GEMV_PAD_FLOATS) * 4);
        const int vi = silu ? (rs == 8 ? 3 : 4) : (rs == 8 ? 0 : nl == 3 ? 1 : 2);
        const Fn f = (Fn)((t.exact ? F_GEMV_G8_3 : F_GEMV_G8_3_E0) + vi);
        return launch(c, f, (unsigned)grid, (unsigned)(nw * slots * 64), lds, &a, sizeof a);
    }
    if (t.pairs_per_wave > 12)
        return fail(Q8_ERR_UNSUPPORTED, "gemv: %d block pairs per wave exceeds the staging bound of 12",
                    t.pairs_per_wave);
    const int pb = valid_pb(t.pairs_per_batch) ? t.pairs_per_batch : 5;
    a.total_tiles = silu ? m[0].w->tiles : tile;
    a.x = reinterpret_cast<const float *>(x);
    a.nb = nb;
    a.waves_per_tile = t.waves_per_tile;
    a.pairs_per_wave = t.pairs_per_wave;
    a.silu_pair = silu;
    a.kslices = t.kslices;
    a.slice_magic = ((1ULL << 32) + (unsigned long long)t.kslices - 1) / (unsigned long long)t.kslices;
    a.pairs_per_slice = (int)ceil_div((nb + 1) / 2, t.kslices);
    a.scratch = c->split_ws;
    a.counters = c->counters;
    a.norm_w = norm_w;
    a.norm_eps = norm_eps;
    if (rope) {
        a.rope_pos = rope->position;
        a.rope_freq = rope->freq;
        a.kcache = rope->kcache;
        a.vcache = rope->vcache;
        a.head_dim = rope->head_dim;
        a.n_rot = rope->n_rot;
        a.capacity = rope->capacity;
    }
    if (comb) {
        a.attn_acc = comb->acc;
        a.attn_ms = comb->ms;
        a.attn_splits = comb->splits;
    }
    if (amax) {
        if (tile > kArgmaxMaxParts) return fail(Q8_ERR_UNSUPPORTED, "argmax over %d tiles", tile);
        a.amax_value = amax->value;
        a.amax_index = amax->index;
    }
    const int waves = t.waves_per_tile * slots;
    const int max_threads = pb == 9 ? 512 : 1024;
    if (norm_w && (t.kslices != 1 || waves * 64 < 256 || k > 1024 * Q8_NORM_ROW_VEC))
        return fail(Q8_ERR_UNSUPPORTED, "gemv: the folded norm needs one K slice and >= 256 threads");
    if (comb && (t.kslices != 1 || nb * 8 > waves * 64 || comb->splits < 1 || comb->splits > Q8_ATTN_COMBINE_MAX))
        return fail(Q8_ERR_UNSUPPORTED, "gemv: the folded attention combine needs one K slice, a thread per float4 "
                                        "of x and at most %d splits", Q8_ATTN_COMBINE_MAX);
    if (waves * 64 > max_threads)
        return fail(Q8_ERR_UNSUPPORTED, "gemv: %d waves per workgroup exceed the %d-thread launch bound", waves,
                    max_threads);
    if (t.kslices > 1) {
        const size_t need = (size_t)slots * a.total_tiles * (t.exact ? nb : t.kslices) * 32 * sizeof(float);
        if (need > kSplitBytes || a.total_tiles > kAttnCounterBase)
            return fail(Q8_ERR_UNSUPPORTED, "gemv: split-K needs %zu bytes of scratch for %d tiles", need,
                        a.total_tiles);
    }
    const long long grid = (long long)a.total_tiles * t.kslices;
    if (grid > 0x7fffffffLL) return fail(Q8_ERR_UNSUPPORTED, "gemv: grid of %lld workgroups", grid);
    // the kernel divides workgroup indices by S with slice_magic: exact below 2^32
    if ((unsigned long long)grid * (unsigned long long)t.kslices >= (1ULL << 32))
        return fail(Q8_ERR_UNSUPPORTED, "gemv: %lld workgroups in %d K slices", grid, t.kslices);
    const unsigned lds =
        (unsigned)(nb * 32 * 4 + ((t.exact && t.kslices == 1) ? slots * 32 * Q8_GEMV_VROW(nb) * 4 : waves * 32 * 4) +
                   Q8_GEMV_PAD_FLOATS * 4);
    if (comb && (count != 1 || silu || norm_w || rope))
        return fail(Q8_ERR_UNSUPPORTED, "gemv: the folded attention combine serves one matrix");
    return launch(c, gemv_fn(pb, t.exact, count == 1 && !silu && !norm_w && !rope, comb != nullptr), (unsigned)grid,
                  (unsigned)(waves * 64), lds, &a, sizeof a);
}

// Whether run_gemv can build x from `splits` attention partials over one
// matrix of k = heads * 64: one K slice and a thread per float4 of x.
bool gemv_folds_combine(q8_ctx *c, const q8_weight *w, int splits) {
    const q8_tactic t = plan(c, 1, w->out, w->k, 1);
    const int pb = valid_pb(t.pairs_per_batch) ? t.pairs_per_batch : 5;
    const int threads = t.waves_per_tile * 64;
    return t.kslices == 1 && t.pairs_per_wave <= 12 && threads <= (pb == 9 ? 512 : 1024) &&
           (w->k / 32) * 8 <= threads && splits >= 1 && splits <= Q8_ATTN_COMBINE_MAX;
}

// Whether run_gemv can fold an RMSNorm into this launch: one K slice (each
// workgroup sees all of x), >= 256 threads (the row norm's reduction shape)
// and k within the row norm's reach.
bool gemv_folds_norm(q8_ctx *c, const Member *m, int count, int k, int silu) {
    int rs = 0, nl = 0, nw = 0, sl = 0;
    int rows_total = 0;
    for (int i = 0; i < count; i++) rows_total += m[i].w->out;
    const int slots = silu ? 2 : 1;
    const q8_tactic t = plan(c, 1, silu ? m[0].w->out : rows_total, k, slots);
    if ((count > 1 || silu) && rsg_shape(c, k / 32, silu, true, &rs, &nl, &nw, contiguous_group(c, m, count, &sl)))
        return true;
    const int pb = valid_pb(t.pairs_per_batch) ? t.pairs_per_batch : 5;
    const int waves = t.waves_per_tile * slots;
    return t.kslices == 1 && t.pairs_per_wave <= 12 && waves * 64 >= 256 && waves * 64 <= (pb == 9 ? 512 : 1024) &&
           k <= 1024 * Q8_NORM_ROW_VEC;
}

int run_rmsnorm(q8_ctx *c, const float *x, int rows, int k, const float *w, float eps, float *out, q8_prepared *p);

// rmsnorm(x) * norm_w then a decode GEMV: folded into one launch when it
// fits, else the row norm into the norm workspace first.
int run_norm_gemv(q8_ctx *c, const Member *m, int count, q8_dptr x, int k, int silu, const float *norm_w,
                  float eps, const GemvRope *rope = nullptr) {
    if (gemv_folds_norm(c, m, count, k, silu))
        return run_gemv(c, m, count, x, k, nullptr, silu, norm_w, eps, rope);
    Q8_TRY(grow(c, &c->norm_ws, &c->norm_ws_bytes, (size_t)k * sizeof(float), "hipMalloc(norm workspace)"));
    float *xn = static_cast<float *>(c->norm_ws);
    Q8_TRY(run_rmsnorm(c, reinterpret_cast<const float *>(x), 1, k, norm_w, eps, xn, nullptr));
    return run_gemv(c, m, count, (q8_dptr)(uintptr_t)xn, k, nullptr, silu, nullptr, 0.0f, rope);
}

int run_gemm_h(q8_ctx *c, const Member *m, int count, const q8_prepared *p, int n, const float *bias,
               const GemvRope *rope = nullptr);

// Cache riders of a GEMM launch (Q8GemmArgs::riders).  With weights
// announced by q8_gemm_prefetch, the riders read those (and the announcement
// is consumed); otherwise, with option gemm.riders > 0, the launch's own
// members.  Counts are rounded down to a multiple of 8 so every compute
// workgroup keeps its XCD.
void set_riders(q8_ctx *c, Q8GemmArgs &a, const q8_weight *const *own, int own_count, int threads) {
    a.riders = 0;
    a.rider_count = 0;
    const bool next = !c->next_weights.empty();
    const q8_weight *const *w = next ? c->next_weights.data() : own;
    const int count = next ? (int)c->next_weights.size() : own_count;
    size_t bytes = 0;
    for (int i = 0; i < count && i < Q8_RIDER_MAX; i++) {
        a.rider_q[i] = w[i]->quants;
        a.rider_s[i] = w[i]->scales;
        a.rider_units[i] = (unsigned)((size_t)w[i]->tiles * w[i]->nb);
        a.rider_count = i + 1;
        bytes += (size_t)a.rider_units[i] * (Q8_UNIT_BYTES + Q8_TILE_ROWS * 2);
    }
    c->next_weights.clear();
    if (next && !option(c, "gemm.prefetch", 1)) a.rider_count = 0;  // announcements switched off
    long long riders = next ? option(c, "gemm.next_riders", 0) : option(c, "gemm.riders", 0);
    if (next && riders == 0) {
        // a rider wave per gemm.rider_wave_kib KiB of the announced weights
        const long long per_wave = 1024LL * std::max(1, option(c, "gemm.rider_wave_kib", 32));
        const long long waves = ceil_div((long long)bytes, per_wave);
        riders = align_up(ceil_div(waves, std::max(1, threads / 64)), 8);
    }
    a.riders = a.rider_count ? (int)(std::min<long long>(std::max<long long>(riders, 0), 4096) & ~7LL) : 0;
    a.rider_first = option(c, next ? "gemm.next_rider_first" : "gemm.rider_first", next ? 0 : 1) ? 1 : 0;
    a.rider_nt = option(c, "gemm.rider_nt", 0) ? 1 : 0;
}

// Gate/up GEMM whose epilogue writes silu(gate) * up as prepared Q8_0
// (q8_gemm_silu) into the second activation workspace: the input stays
// readable in the first.  int8 prepared input only.
int run_gemm_silu(q8_ctx *c, const q8_weight *gate, const q8_weight *up, const q8_prepared *p, int n,
                  q8_prepared *out) {
    const int k = p->k, nb = k / 32, ffn = gate->out, nbo = ffn / 32;
    const long long ttiles = ceil_div(n, 32);
    const int fmt = prepared_format(c, n);
    const size_t qbytes = (size_t)ttiles * nbo * (fmt == Q8_PREPARED_F16 ? Q8_UNIT_F16_BYTES : Q8_UNIT_BYTES);
    const size_t sbytes = (size_t)ttiles * nbo * Q8_TILE_TOKENS * sizeof(float);
    Q8_TRY(grow(c, &c->act2_ws, &c->act2_ws_bytes, align_up(qbytes, kAlign) + sbytes, "hipMalloc(activation 2)"));
    Q8GemmArgs a{};
    a.members = 2;
    a.m[0] = {gate->quants, gate->scales, nullptr, nullptr, ffn, 0};
    a.m[1] = {up->quants, up->scales, nullptr, nullptr, ffn, gate->tiles};
    a.total_rtiles = gate->tiles;
    a.xq = reinterpret_cast<const uint8_t *>(p->quants);
    a.xs = reinterpret_cast<const float *>(p->scales);
    a.n = n;
    a.nb = nb;
    a.ttiles = (int)ttiles;
    a.twaves = 1;
    a.tgroups = (int)ttiles;
    a.kslices = 1;
    const int npairs = (nb + 1) / 2;
    a.pairs_per_slice = npairs;
    // >= 11 waves per CU (each wave carries a gate and an up tile, as the
    // paired-token-tile GEMM), >= 9 block pairs per wave; measured over
    // n = 32..1024 at 5760 x 2304
    const long long base = (long long)gate->tiles * ttiles;
    int kw = (int)std::max<long long>(1, ceil_div(11LL * std::max(c->cu_count, 1), base));
    kw = std::min(std::min(kw, 8), std::max(1, npairs / 9));
    const int kw_opt = option(c, "gemm.kwaves", -1);
    if (kw_opt > 0) kw = std::min(kw_opt, 8);
    kw = std::min(kw, npairs);
    const int ppw = (int)ceil_div(npairs, kw);
    kw = (int)ceil_div(npairs, ppw);
    a.pairs_per_wave = ppw;
    const long long nwg = base;
    if (nwg > 0x7fffffffLL - 4096) return fail(Q8_ERR_UNSUPPORTED, "gemm_silu: grid of %lld workgroups", nwg);
    a.nwg = (int)nwg;
    a.xcd_remap = nwg % 8 == 0 ? 1 : 0;
    a.oq = static_cast<uint8_t *>(c->act2_ws);
    a.os = reinterpret_cast<float *>(static_cast<uint8_t *>(c->act2_ws) + align_up(qbytes, kAlign));
    a.of16 = fmt == Q8_PREPARED_F16 ? 1 : 0;
    const unsigned lds = (unsigned)std::max<size_t>((size_t)(kw - 1) * 2 * 64 * 16 * sizeof(float), 32 * 33 * sizeof(float));
    const q8_weight *own[2] = {gate, up};
    set_riders(c, a, own, 2, 64 * kw);
    Q8_TRY(launch(c, F_GEMM_SILU, (unsigned)(nwg + a.riders), (unsigned)(64 * kw), lds, &a, sizeof a));
    out->quants = (q8_dptr)(uintptr_t)a.oq;
    out->scales = (q8_dptr)(uintptr_t)a.os;
    out->n = n;
    out->k = ffn;
    out->format = fmt;
    return Q8_OK;
}

// Sets the RoPE + KV append epilogue of a q, k, v group (rope non-null).
void set_gemm_rope(Q8GemmArgs &a, const GemvRope *rope) {
    if (!rope) return;
    a.rope_pos = rope->position;
    a.rope_freq = rope->freq;
    a.kcache = rope->kcache;
    a.vcache = rope->vcache;
    a.head_dim = rope->head_dim;
    a.n_rot = rope->n_rot;
    a.capacity = rope->capacity;
}

// no_split: keep every block of a row tile in one workgroup (no partial
// results or arrival counters in the context's split scratch).
int run_gemm(q8_ctx *c, const Member *m, int count, const q8_prepared *p, int n, const float *bias,
             const GemvRope *rope = nullptr, bool no_split = false) {
    if (p->format == Q8_PREPARED_F16) return run_gemm_h(c, m, count, p, n, bias, rope);
    if (p->format != Q8_PREPARED_I8) return fail(Q8_ERR_INVALID, "prepared activations: unknown format %d", p->format);
    {
        int rows_total = 0;
        for (int i = 0; i < count; i++) rows_total += m[i].w->out;
        const q8_tactic t = plan(c, n, rows_total, p->k, 1, Q8_PREPARED_I8);
        if (t.rwaves > 0) return run_gemm_h(c, m, count, p, n, bias, rope);
    }
    const int k = p->k;
    const int nb = k / 32;
    Q8GemmArgs a{};
    a.members = count;
    int rt = 0, rows_total = 0;
    for (int i = 0; i < count; i++) {
        a.m[i].quants = m[i].w->quants;
        a.m[i].scales = m[i].w->scales;
        a.m[i].y = m[i].y;
        a.m[i].bias = (i == 0) ? bias : nullptr;
        a.m[i].rows = m[i].w->out;
        a.m[i].tile_begin = rt;
        rt += m[i].w->tiles;
        rows_total += m[i].w->out;
    }
    q8_tactic t = plan(c, n, rows_total, k, 1, Q8_PREPARED_I8);
    if (no_split && t.kslices > 1) {
        t.kslices = 1;
        t.pairs_per_wave = (int)ceil_div((nb + 1) / 2, std::max(1, t.kwaves));
    }
    a.total_rtiles = rt;
    a.xq = reinterpret_cast<const uint8_t *>(p->quants);
    a.xs = reinterpret_cast<const float *>(p->scales);
    a.n = n;
    a.nb = nb;
    a.ttiles = (int)ceil_div(n, 32);
    const int tpw = t.tpw > 0 ? t.tpw : 1;
    a.twaves = std::max(1, t.twaves);
    a.tgroups = (int)ceil_div(a.ttiles, (long long)a.twaves * tpw);
    a.kslices = std::max(1, t.kslices);
    a.pairs_per_slice = (int)ceil_div((nb + 1) / 2, a.kslices);
    a.pairs_per_wave = std::max(1, t.pairs_per_wave);
    const int kwaves = std::max(1, t.kwaves);
    a.scratch = no_split ? nullptr : c->split_ws;
    a.counters = no_split ? nullptr : c->counters;
    set_gemm_rope(a, rope);
    const long long groups = (long long)rt * a.tgroups;
    if (a.kslices > 1) {
        const size_t need = (size_t)rt * a.ttiles * a.kslices * 64 * 16 * sizeof(float);
        if (need > kSplitBytes || groups > kAttnCounterBase)
            return fail(Q8_ERR_UNSUPPORTED, "gemm: split-K needs %zu bytes of scratch", need);
    }
    const long long nwg = groups * a.kslices;
    if (nwg > 0x7fffffffLL - 4096) return fail(Q8_ERR_UNSUPPORTED, "gemm: grid of %lld workgroups", nwg);
    a.nwg = (int)nwg;
    a.xcd_remap = (t.xcd_remap && nwg % 8 == 0) ? 1 : 0;
    const int threads = 64 * a.twaves * kwaves;
    const bool pipe = t.pipe && t.smode && a.kslices == 1 && tpw <= 2;
    const int max_threads = (tpw == 1 && !pipe) ? 1024 : 512;
    if (threads > max_threads) return fail(Q8_ERR_UNSUPPORTED, "gemm: %d threads per workgroup", threads);
    const unsigned lds = (unsigned)((kwaves - 1) * a.twaves * tpw * 64 * 16 * sizeof(float));
    Fn f = pipe ? (tpw == 2 ? F_GEMM_P_T2 : F_GEMM_P_T1)
                : !t.smode ? F_GEMM_S0_T1 : tpw == 4 ? F_GEMM_S1_T4 : tpw == 2 ? F_GEMM_S1_T2 : F_GEMM_S1_T1;
    // one token tile: every weight byte is read by one wave, once (option
    // gemm.stream = 0 keeps the default cache policy)
    if (f == F_GEMM_S1_T1 && a.ttiles == 1 && option(c, "gemm.stream", 1)) f = F_GEMM_S1_T1S;
    if (f != F_GEMM_P_T1 && f != F_GEMM_P_T2) {
        const q8_weight *own[Q8_GROUP_MAX];
        for (int i = 0; i < count; i++) own[i] = m[i].w;
        set_riders(c, a, own, count, threads);
    }
    return launch(c, f, (unsigned)(nwg + a.riders), (unsigned)threads, lds, &a, sizeof a);
}

// The staged GEMMs (gemm_h_body): RW row-tile waves x KW K groups per
// workgroup over TPW token tiles, activations staged in LDS per K group;
// f16 units on the f16 MFMA (q8_gemm_h) or int8 units on the int8 MFMA
// (q8_gemm_l), by the prepared format.
int run_gemm_h(q8_ctx *c, const Member *m, int count, const q8_prepared *p, int n, const float *bias,
               const GemvRope *rope) {
    const int k = p->k;
    const int nb = k / 32;
    Q8GemmArgs a{};
    a.members = count;
    int rt = 0, rows_total = 0;
    for (int i = 0; i < count; i++) {
        a.m[i].quants = m[i].w->quants;
        a.m[i].scales = m[i].w->scales;
        a.m[i].y = m[i].y;
        a.m[i].bias = (i == 0) ? bias : nullptr;
        a.m[i].rows = m[i].w->out;
        a.m[i].tile_begin = rt;
        rt += m[i].w->tiles;
        rows_total += m[i].w->out;
    }
    const bool i8 = p->format == Q8_PREPARED_I8;
    const q8_tactic t = plan(c, n, rows_total, k, 1, p->format);
    const int tpw = t.tpw == 2 ? 2 : 1;
    const int rw = tpw == 1 ? (i8 ? 2 : 4) : (t.rwaves >= 4 ? 4 : 2);
    const int kw = std::max(1, t.kwaves);
    if (rw * kw > 8) return fail(Q8_ERR_UNSUPPORTED, "gemm_h: %d x %d waves per workgroup", rw, kw);
    a.total_rtiles = rt;
    a.xq = reinterpret_cast<const uint8_t *>(p->quants);
    a.xs = reinterpret_cast<const float *>(p->scales);
    a.n = n;
    a.nb = nb;
    a.ttiles = (int)ceil_div(n, 32);
    a.twaves = 1;
    a.rwaves = rw;
    a.tgroups = (int)ceil_div(a.ttiles, tpw);
    a.kslices = 1;
    a.pairs_per_slice = (nb + 1) / 2;
    a.pairs_per_wave = std::max(1, t.pairs_per_wave);
    set_gemm_rope(a, rope);
    if ((long long)a.pairs_per_wave * kw < (nb + 1) / 2)
        return fail(Q8_ERR_UNSUPPORTED, "gemm_h: %d K waves x %d pairs miss blocks", kw, a.pairs_per_wave);
    const long long nwg = ceil_div(rt, rw) * (long long)a.tgroups;
    if (nwg > 0x7fffffffLL) return fail(Q8_ERR_UNSUPPORTED, "gemm_h: grid of %lld workgroups", nwg);
    a.nwg = (int)nwg;
    a.xcd_remap = (t.xcd_remap && nwg % 8 == 0) ? 1 : 0;
    const size_t stage =
        (size_t)kw * Q8_GEMM_H_STAGES * (i8 ? Q8_GEMM_L_BUF_BYTES(tpw, rw) : Q8_GEMM_H_BUF_BYTES(tpw, rw));
    const size_t reduce = (size_t)(kw - 1) * rw * tpw * 64 * 16 * sizeof(float);
    const unsigned lds = (unsigned)std::max(stage, reduce);
    const Fn f = i8 ? (tpw == 1 ? F_GEMM_L_T1_R2 : rw == 4 ? F_GEMM_L_T2_R4 : F_GEMM_L_T2_R2)
                    : (tpw == 1 ? F_GEMM_H_T1_R4 : rw == 4 ? F_GEMM_H_T2_R4 : F_GEMM_H_T2_R2);
    return launch(c, f, (unsigned)nwg, (unsigned)(64 * rw * kw), lds, &a, sizeof a);
}

// Bytes of prepared activations for n tokens of k in format fmt: the units
// (padded to kAlign) then the f32 scales.
size_t prepared_bytes(int n, int k, int fmt, size_t *qbytes_out) {
    const long long ttiles = ceil_div(n, 32);
    const size_t qbytes =
        (size_t)ttiles * (k / 32) * (fmt == Q8_PREPARED_F16 ? Q8_UNIT_F16_BYTES : Q8_UNIT_BYTES);
    if (qbytes_out) *qbytes_out = qbytes;
    return align_up(qbytes, kAlign) + (size_t)ttiles * (k / 32) * Q8_TILE_TOKENS * sizeof(float);
}

// q8_quantize of x (or of silu(gate) * up) into prepared activations at
// `base` (prepared_bytes(n, k, fmt) bytes).
int run_quantize(q8_ctx *c, q8_dptr x, q8_dptr gate, q8_dptr up, int n, int k, int fmt, void *base,
                 q8_prepared *out) {
    const int nb = k / 32;
    const long long ttiles = ceil_div(n, 32);
    size_t qbytes = 0;
    prepared_bytes(n, k, fmt, &qbytes);
    Q8QuantArgs a{};
    a.x = reinterpret_cast<const float *>(x);
    a.gate = reinterpret_cast<const float *>(gate);
    a.up = reinterpret_cast<const float *>(up);
    a.xq = static_cast<uint8_t *>(base);
    a.xs = reinterpret_cast<float *>(static_cast<uint8_t *>(base) + align_up(qbytes, kAlign));
    a.n = n;
    a.nb = nb;
    a.ttiles = (int)ttiles;
    a.mode = gate ? 1 : 0;
    a.f16 = fmt == Q8_PREPARED_F16 ? 1 : 0;
    const long long units = ttiles * nb;  // one wave per (token tile, block) unit, four per workgroup
    if (units > 0x7fffffffLL) return fail(Q8_ERR_UNSUPPORTED, "prepare: %lld units", units);
    Q8_TRY(launch(c, F_QUANTIZE, (unsigned)ceil_div(units, 4), 256, 0, &a, sizeof a));
    out->quants = (q8_dptr)(uintptr_t)a.xq;
    out->scales = (q8_dptr)(uintptr_t)a.xs;
    out->n = n;
    out->k = k;
    out->format = fmt;
    return Q8_OK;
}

int prepare_into(q8_ctx *c, q8_dptr x, q8_dptr gate, q8_dptr up, int n, int k, q8_prepared *out) {
    const int fmt = prepared_format(c, n);
    Q8_TRY(grow(c, &c->act_ws, &c->act_ws_bytes, prepared_bytes(n, k, fmt, nullptr), "hipMalloc(activation)"));
    return run_quantize(c, x, gate, up, n, k, fmt, c->act_ws, out);
}

// Gpu::plain (cuda/mod.rs, used by rmsnorm_prepare 1414-1445): an f32 vector
// copied to the device once, keyed by the host slice's identity (ptr, len).
int vector_resident(q8_ctx *c, const float *host, size_t len, float **out) {
    const auto key = std::make_pair((uintptr_t)host, len);
    auto it = c->vectors.find(key);
    if (it != c->vectors.end()) {
        *out = it->second;
        return Q8_OK;
    }
    float *dev = nullptr;
    HIP_TRY(dev_malloc(c, reinterpret_cast<void **>(&dev), len * sizeof(float)), "hipMalloc(norm weight)");
    hipError_t e = hipMemcpyAsync(dev, host, len * sizeof(float), hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        hipFree(dev);
        return hip_fail(e, "upload(norm weight)");
    }
    c->vectors[key] = dev;
    *out = dev;
    return Q8_OK;
}

// q8_rmsnorm kernel: f32 rows into `out` and/or prepared Q8_0 into `p`.
int run_rmsnorm(q8_ctx *c, const float *x, int rows, int k, const float *w, float eps, float *out, q8_prepared *p) {
    Q8NormArgs a{};
    a.x = x;
    a.w = w;
    a.out = out;
    a.n = rows;
    a.rows_launched = rows;
    a.k = k;
    a.eps = eps;
    if (p) {
        const int nb = k / 32;
        const long long ttiles = ceil_div(rows, 32);
        const int fmt = prepared_format(c, rows);
        const size_t qbytes = (size_t)ttiles * nb * (fmt == Q8_PREPARED_F16 ? Q8_UNIT_F16_BYTES : Q8_UNIT_BYTES);
        const size_t sbytes = (size_t)ttiles * nb * Q8_TILE_TOKENS * sizeof(float);
        Q8_TRY(grow(c, &c->act_ws, &c->act_ws_bytes, align_up(qbytes, kAlign) + sbytes, "hipMalloc(activation)"));
        a.xq = static_cast<uint8_t *>(c->act_ws);
        a.xs = reinterpret_cast<float *>(static_cast<uint8_t *>(c->act_ws) + align_up(qbytes, kAlign));
        a.f16 = fmt == Q8_PREPARED_F16 ? 1 : 0;
        a.rows_launched = (int)(ttiles * 32);
        p->quants = (q8_dptr)(uintptr_t)a.xq;
        p->scales = (q8_dptr)(uintptr_t)a.xs;
        p->n = rows;
        p->k = k;
        p->format = fmt;
    }
    // a workgroup per row, the row loaded once (k <= 8192, four floats per
    // thread per step); prepared output: rows to the token-tile boundary
    if (k <= 256 * 4 * Q8_NORM_ROW_VEC)
        return launch(c, F_RMSNORM_ROW, a.xq ? (unsigned)align_up((size_t)a.rows_launched, 64) : (unsigned)a.rows_launched, 256,
                      a.xq ? (unsigned)((k / 32) * Q8_NORM_LDS_PITCH * sizeof(float)) : 0u, &a, sizeof a);
    return launch(c, F_RMSNORM, (unsigned)ceil_div(a.rows_launched, 4), 256, 0, &a, sizeof a);
}

int check_k(int k) {
    if (k <= 0 || k % 32 != 0) return fail(Q8_ERR_INVALID, "Q8_0 rows are whole 32-element blocks (k = %d)", k);
    return Q8_OK;
}

int check_n(int n) {
    if (n < 1) return fail(Q8_ERR_INVALID, "n must be at least 1 (got %d)", n);
    if (n > Q8_MAX_TOKENS)
        return fail(Q8_ERR_UNSUPPORTED, "prompt matmul holds %d tokens, got %d", Q8_MAX_TOKENS, n);
    return Q8_OK;
}

int check_weight(q8_ctx *c, const q8_weight *w) {
    if (!w || w->ctx != c) return fail(Q8_ERR_INVALID, "weight handle does not belong to this context");
    return Q8_OK;
}

float *fptr(q8_dptr p, size_t off) { return p ? reinterpret_cast<float *>(p) + off : nullptr; }

int argmax_into(q8_ctx *c, q8_dptr values, size_t len, uint32_t *out) {
    if (len == 0) return fail(Q8_ERR_INVALID, "argmax of an empty vector");
    if (len > 0xfffffffeULL) return fail(Q8_ERR_INVALID, "argmax length %zu exceeds u32 indices", len);
    Q8_TRY(check_span(c, values, len * 4, "argmax values"));
    uint8_t *ws = static_cast<uint8_t *>(c->argmax_ws);
    Q8ArgmaxArgs a{};
    a.values = reinterpret_cast<const float *>(values);
    a.len = (long long)len;
    a.part_value = reinterpret_cast<float *>(ws);
    a.part_index = reinterpret_cast<unsigned *>(ws + kArgmaxMaxParts * 4);
    a.result = reinterpret_cast<unsigned *>(ws + kArgmaxMaxParts * 8);
    const int parts = (int)std::min<long long>(kArgmaxParts, std::max<long long>(1, ceil_div((long long)len, 4096)));
    a.parts = parts;
    a.stage = 0;
    Q8_TRY(launch(c, F_ARGMAX, (unsigned)parts, 256, 0, &a, sizeof a));
    a.stage = 1;
    Q8_TRY(launch(c, F_ARGMAX, 1, 256, 0, &a, sizeof a));
    uint32_t result = 0;
    HIP_TRY(hipMemcpyAsync(&result, a.result, 4, hipMemcpyDeviceToHost, c->stream), "hipMemcpyAsync(argmax)");
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    *out = result;
    return Q8_OK;
}

}  // namespace

namespace q8i {
unsigned long long workspace_generation(const q8_ctx *c) { return c->ws_generation; }

int set_error(int code, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}
}  // namespace q8i

// ===========================================================================
// C-ABI
// ===========================================================================
extern "C" {

const char *q8_status_string(int status) {
    switch (status) {
        case Q8_OK: return "ok";
        case Q8_ERR_HIP: return "HIP error";
        case Q8_ERR_INVALID: return "invalid argument";
        case Q8_ERR_UNSUPPORTED: return "unsupported";
        case Q8_ERR_NO_DEVICE: return "no device";
        case Q8_ERR_OUT_OF_MEMORY: return "out of device memory";
        case Q8_ERR_FORMAT: return "malformed gguf";
        case Q8_ERR_MISSING: return "missing tensor or metadata key";
        case Q8_ERR_IO: return "io error";
        default: return "unknown status";
    }
}

const char *q8_last_error(void) { return g_last_error.c_str(); }

const char *q8_build_info(void) { return Q8_BUILD_INFO; }

int q8_kernel_info(const char *name, q8_kernel_info_t *out) {
    if (!name || !out) return fail(Q8_ERR_INVALID, "q8_kernel_info: bad arguments");
    const q8i::KernelMeta *m = find_meta(name);
    if (!m) return fail(Q8_ERR_INVALID, "q8_kernel_info: no kernel %s in this build", name);
    *out = q8_kernel_info_t{m->args, m->kernarg, m->vgpr, m->agpr, m->sgpr, m->lds, m->max_wg, m->priv};
    return Q8_OK;
}

int q8_launch_check(const char *name, size_t args_size, unsigned block, size_t dynamic_lds, size_t lds_limit) {
    if (!name) return fail(Q8_ERR_INVALID, "q8_launch_check: null kernel name");
    const q8i::KernelMeta *m = find_meta(name);
    if (!m) return fail(Q8_ERR_INVALID, "q8_launch_check: no kernel %s in this build", name);
    return check_launch(*m, args_size, block, dynamic_lds, lds_limit);
}

int q8_open(int device, q8_ctx **out) {
    if (!out) return fail(Q8_ERR_INVALID, "q8_open: null output");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= device || device < 0)
        return fail(Q8_ERR_NO_DEVICE, "no HIP device %d (%d visible): %s", device, count,
                    e == hipSuccess ? "out of range" : hipGetErrorString(e));
    HIP_TRY(hipSetDevice(device), "hipSetDevice");
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(Q8_ERR_NO_DEVICE, "device %d is %s; this build carries gfx950 code only", device,
                    prop.gcnArchName);
    q8_ctx *c = new q8_ctx();
    c->device = device;
    c->cu_count = prop.multiProcessorCount;
    c->total_mem = prop.totalGlobalMem;
    c->max_lds = prop.sharedMemPerBlock;
    char market[256] = {0};
    if (hipDeviceGetName(market, sizeof market - 1, device) != hipSuccess || market[0] == 0)
        std::snprintf(market, sizeof market, "%s", prop.name[0] ? prop.name : "AMD Instinct");
    std::snprintf(c->name, sizeof c->name, "%s (%s, %d CUs, %zu KB LDS per workgroup)", market, prop.gcnArchName,
                  c->cu_count, c->max_lds / 1024);
    int rc = Q8_OK;
    do {
        hipError_t he = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
        if (he != hipSuccess) { rc = hip_fail(he, "hipStreamCreate"); break; }
        he = hipModuleLoadData(&c->module, q8_code_object);
        if (he != hipSuccess) { rc = fail(Q8_ERR_NO_DEVICE, "hip: hipModuleLoadData failed: %s", hipGetErrorString(he)); break; }
        for (int i = 0; i < F_COUNT && rc == Q8_OK; i++) {
            he = hipModuleGetFunction(&c->fn[i], c->module, kFnNames[i]);
            if (he != hipSuccess)
                rc = fail(Q8_ERR_NO_DEVICE, "hip: hipModuleGetFunction(%s) failed: %s", kFnNames[i],
                          hipGetErrorString(he));
            c->meta[i] = find_meta(kFnNames[i]);
            if (rc == Q8_OK && !c->meta[i])
                rc = fail(Q8_ERR_NO_DEVICE, "kernel %s has no metadata in this build", kFnNames[i]);
        }
        if (rc != Q8_OK) break;
        he = dev_malloc(c, &c->argmax_ws, kArgmaxMaxParts * 8 + 256);
        if (he != hipSuccess) { rc = hip_fail(he, "hipMalloc(argmax)"); break; }
        rc = q8i::noalloc_scratch(device, &c->noalloc);  // the device is current (hipSetDevice above)
        if (rc != Q8_OK) break;
        he = dev_malloc(c, (void **)&c->split_ws, kSplitBytes);
        if (he != hipSuccess) { rc = hip_fail(he, "hipMalloc(split scratch)"); break; }
        he = dev_malloc(c, (void **)&c->counters, kCounters * sizeof(unsigned));
        if (he != hipSuccess) { rc = hip_fail(he, "hipMalloc(counters)"); break; }
        he = hipMemset(c->counters, 0, kCounters * sizeof(unsigned));
        if (he == hipSuccess) he = hipDeviceSynchronize();
        if (he != hipSuccess) { rc = hip_fail(he, "hipMemset(counters)"); break; }
    } while (0);
    if (rc != Q8_OK) {
        q8_close(c);
        return rc;
    }
    *out = c;
    return Q8_OK;
}

void q8_close(q8_ctx *c) {
    if (!c) return;
    hipSetDevice(c->device);
    if (c->stream) hipStreamSynchronize(c->stream);
    q8i::noalloc_release(c);
    // a group's allocation goes with its last member
    auto drop = [](q8_weight *w) {
        if (!w->group_refs || --*w->group_refs == 0) {
            hipFree(w->base);
            delete w->group_refs;
        }
        delete w;
    };
    for (auto &kv : c->weights) drop(kv.second);
    for (auto &kv : c->vectors) hipFree(kv.second);
    for (auto &kv : c->rope_freq) hipFree(kv.second);
    for (auto &kv : c->allocs) hipFree(reinterpret_cast<void *>(kv.first));
    for (void *w : {c->act_ws, c->tmp_ws, c->act2_ws, c->norm_ws, c->token_ws, c->attn_ws, c->attn_out_ws})
        if (w && !in_arena(c, w)) hipFree(w);
    if (c->arena) hipFree(c->arena);
    if (c->argmax_ws) hipFree(c->argmax_ws);
    if (c->split_ws) hipFree(c->split_ws);
    if (c->counters) hipFree(c->counters);
    for (q8_weight *w : c->owned) drop(w);
    if (c->module) hipModuleUnload(c->module);
    if (c->stream) hipStreamDestroy(c->stream);
    delete c;
}

int q8_device_name(q8_ctx *c, char *buf, size_t len) {
    if (!c || !buf || len == 0) return fail(Q8_ERR_INVALID, "q8_device_name: bad arguments");
    std::snprintf(buf, len, "%s", c->name);
    return Q8_OK;
}

int q8_device_info(q8_ctx *c, int *cu_count, size_t *total_bytes, size_t *free_bytes) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_device_info: null context");
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    if (cu_count) *cu_count = c->cu_count;
    size_t fr = 0, tot = 0;
    HIP_TRY(hipMemGetInfo(&fr, &tot), "hipMemGetInfo");
    if (total_bytes) *total_bytes = tot;
    if (free_bytes) *free_bytes = fr;
    return Q8_OK;
}

void *q8_stream(q8_ctx *c) { return c ? (void *)c->stream : nullptr; }

int q8_set_option(q8_ctx *c, const char *name, int value) {
    if (!c || !name) return fail(Q8_ERR_INVALID, "q8_set_option: bad arguments");
    static const char *const known[] = {"gemv.exact", "gemv.waves",  "gemv.pairs",     "gemv.slices",
                                        "gemv.rows",  "gemv.loads", "gemv.xcd_order", "gemv.group_rows",
                                        "gemv.group_loads",
                                        "gemm.smode", "gemm.tpw",    "gemm.twaves",    "gemm.xcd_remap",
                                        "gemm.kwaves", "gemm.slices", "gemm.rwaves",    "gemm.f16",
                                        "gemm.pipe",  "gemm.lds",      "gemm.silu",      "gemm.small_gemv", "gemm.stream",
                                        "gemm.riders", "gemm.rider_nt", "gemm.rider_first", "gemm.next_riders",
                                        "gemm.next_rider_first", "gemm.rider_wave_kib", "gemm.prefetch",
                                        "gemv.slice_copy", "gemv.group_hot", "gemv.group_pair", "gemv.pair_loads",
                                        "attn.waves"};
    bool ok = false;
    for (const char *k : known) ok = ok || std::strcmp(k, name) == 0;
    if (!ok) return fail(Q8_ERR_INVALID, "unknown option %s", name);
    if (std::strcmp(name, "gemv.pairs") == 0 && value > 0 && !valid_pb(value))
        return fail(Q8_ERR_INVALID, "gemv.pairs must be one of 2, 3, 5, 9");
    if (std::strcmp(name, "gemv.rows") == 0 && value >= 0 && value != 0 && value != 8 && value != 16 && value != 32)
        return fail(Q8_ERR_INVALID, "gemv.rows must be 8, 16 or 32 (32: the tile kernel)");
    if (std::strcmp(name, "gemv.loads") == 0 && value > 0 && value != 2 && value != 3 && value != 6)
        return fail(Q8_ERR_INVALID, "gemv.loads must be 2 (8-row slices), 3 or 6");
    if (std::strcmp(name, "gemv.group_rows") == 0 && value > 0 && value != 8 && value != 16 && value != 32)
        return fail(Q8_ERR_INVALID, "gemv.group_rows must be 0 or 32 (the tile kernel), 8 or 16");
    if (std::strcmp(name, "attn.waves") == 0 && value >= 0 && value != 4 && value != 8)
        return fail(Q8_ERR_INVALID, "attn.waves must be 4 or 8 (the split attention's waves a workgroup)");
    if (std::strcmp(name, "gemv.pair_loads") == 0 && value > 0 && value != 3 && value != 6)
        return fail(Q8_ERR_INVALID, "gemv.pair_loads must be 3 or 6");
    if (std::strcmp(name, "gemv.group_loads") == 0 && value > 0 && value != 3 && value != 6)
        return fail(Q8_ERR_INVALID, "gemv.group_loads must be 3 or 6");
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    c->options[name] = value;
    return Q8_OK;
}

int q8_alloc(q8_ctx *c, size_t bytes, q8_dptr *out) {
    if (!c || !out || bytes == 0) return fail(Q8_ERR_INVALID, "q8_alloc: bad arguments");
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    void *p = nullptr;
    HIP_TRY(dev_malloc(c, &p, bytes), "hipMalloc");
    c->allocs[(uintptr_t)p] = bytes;
    *out = (q8_dptr)(uintptr_t)p;
    return Q8_OK;
}

int q8_free(q8_ctx *c, q8_dptr ptr) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_free: null context");
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    auto it = c->allocs.find((uintptr_t)ptr);
    if (it == c->allocs.end()) return fail(Q8_ERR_INVALID, "q8_free: pointer was not allocated by this context");
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    HIP_TRY(hipFree(reinterpret_cast<void *>(ptr)), "hipFree");
    c->allocs.erase(it);
    return Q8_OK;
}

int rope_table(q8_ctx *c, int n_rot, float base, const float **out);

// BufferPlan::plan / scratch_requests (apps/engine/src/workspace.rs:63-106,
// 171-342): every per-call workspace sized once for the largest shapes the
// caller will serve.  The reference packs requests whose phases do not
// overlap into shared offsets to fit consumer memory; here each workspace
// gets a region of its own in one allocation (a few tens of MB against
// 288 GB of HBM), so any order of calls is safe and no liveness analysis
// can be wrong.
int q8_workspace_plan(q8_ctx *c, const q8_workspace_shape *s) {
    if (!c || !s) return fail(Q8_ERR_INVALID, "q8_workspace_plan: bad arguments");
    if (s->max_tokens < 1 || s->max_tokens > Q8_MAX_TOKENS || s->max_k < 32 || s->max_k % 32 || s->max_ff < 0 ||
        s->max_ff % 32 || s->attn_heads < 0 || s->attn_heads > kCounters - kAttnCounterBase || s->attn_splits < 0 ||
        s->attn_splits > 1024 || s->rope_n_rot < 0 || s->rope_n_rot % 2 || s->rope_n_rot > Q8_ATTN_HEAD_DIM)
        return fail(Q8_ERR_INVALID,
                    "workspace shape: tokens %d (1..%d), k %d and ff %d (multiples of 32), heads %d, splits %d, "
                    "rot %d",
                    s->max_tokens, Q8_MAX_TOKENS, s->max_k, s->max_ff, s->attn_heads, s->attn_splits, s->rope_n_rot);
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    if (s->rope_n_rot > 0) {
        const float *freq = nullptr;
        Q8_TRY(rope_table(c, s->rope_n_rot, s->rope_base, &freq));
    }
    const int T = s->max_tokens, K = s->max_k, F = s->max_ff, H = s->attn_heads;
    auto prepared_max = [](int n, int k) {
        return std::max(prepared_bytes(n, k, Q8_PREPARED_I8, nullptr), prepared_bytes(n, k, Q8_PREPARED_F16, nullptr));
    };
    struct Slot {
        const char *name;
        void **buf;
        size_t *have;
        size_t need;
    };
    const Slot slots[] = {
        // prepared activations: prompts, prompt attention, the n = 1 quantize
        {"activation", &c->act_ws, &c->act_ws_bytes, prepared_max(T, K)},
        // silu(gate) * up prepared by the fused gate/up GEMM (n >= 2)
        {"activation 2", &c->act2_ws, &c->act2_ws_bytes, F && T >= 2 ? prepared_max(T, F) : 0},
        // gate and up f32 products of the unfused feed-forward pair
        {"ffn", &c->tmp_ws, &c->tmp_ws_bytes, F ? 2 * align_up((size_t)T * F * 4, kAlign) : 0},
        // one normalized row when a norm does not fold into its decode GEMV
        {"norm", &c->norm_ws, &c->norm_ws_bytes, (size_t)K * 4},
        // token ids of q8_embeddings
        {"token ids", &c->token_ws, &c->token_ws_bytes, (size_t)T * 4},
        // decode attention partials: accumulator, max and sum per head and split
        {"attention", &c->attn_ws, &c->attn_ws_bytes,
         H ? (size_t)H * std::max(1, s->attn_splits) * (Q8_ATTN_HEAD_DIM + 2) * 4 : 0},
        // attention output when it cannot fold into the output projection
        {"attention output", &c->attn_out_ws, &c->attn_out_ws_bytes, (size_t)H * Q8_ATTN_HEAD_DIM * 4},
    };
    bool covered = true;
    for (const Slot &sl : slots) covered = covered && *sl.have >= sl.need;
    if (covered) return Q8_OK;  // nothing moves: graphs over the current workspaces stay valid
    // each region is the larger of the plan and what the workspace holds, so
    // a plan never takes room from shapes earlier calls already used
    constexpr size_t kRegionAlign = 64 << 10;
    std::vector<q8_ctx::Region> layout;
    size_t total = 0;
    for (const Slot &sl : slots) {
        const size_t b = align_up(std::max(sl.need, *sl.have), kRegionAlign);
        layout.push_back({sl.name, total, b});
        total += b;
    }
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    void *arena = nullptr;
    HIP_TRY(dev_malloc(c, &arena, total), "hipMalloc(workspace arena)");
    for (const Slot &sl : slots)
        if (*sl.buf && !in_arena(c, *sl.buf)) hipFree(*sl.buf);
    if (c->arena) hipFree(c->arena);
    c->arena = arena;
    c->arena_bytes = total;
    c->regions = layout;
    for (size_t i = 0; i < layout.size(); i++) {
        *slots[i].buf = layout[i].bytes ? static_cast<uint8_t *>(arena) + layout[i].offset : nullptr;
        *slots[i].have = layout[i].bytes;
    }
    c->ws_generation++;  // every workspace moved
    return Q8_OK;
}

int q8_workspace_query(q8_ctx *c, q8_workspace_info *info) {
    if (!c || !info) return fail(Q8_ERR_INVALID, "q8_workspace_query: bad arguments");
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    uint64_t outside = 0;
    const std::pair<void *, size_t> ws[] = {{c->act_ws, c->act_ws_bytes},     {c->act2_ws, c->act2_ws_bytes},
                                            {c->tmp_ws, c->tmp_ws_bytes},     {c->norm_ws, c->norm_ws_bytes},
                                            {c->token_ws, c->token_ws_bytes}, {c->attn_ws, c->attn_ws_bytes},
                                            {c->attn_out_ws, c->attn_out_ws_bytes}};
    for (const auto &w : ws)
        if (w.first && !in_arena(c, w.first)) outside += w.second;
    info->bytes = c->arena_bytes + outside;
    info->arena_bytes = c->arena_bytes;
    info->allocations = c->allocations;
    info->generation = c->ws_generation;
    info->regions = (int)c->regions.size();
    return Q8_OK;
}

int q8_workspace_region(q8_ctx *c, int index, const char **name, uint64_t *offset, uint64_t *bytes) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_workspace_region: null context");
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    if (index < 0 || index >= (int)c->regions.size())
        return fail(Q8_ERR_INVALID, "workspace region %d of %zu", index, c->regions.size());
    const q8_ctx::Region &r = c->regions[index];
    if (name) *name = r.name;
    if (offset) *offset = r.offset;
    if (bytes) *bytes = r.bytes;
    return Q8_OK;
}

int q8_vector_resident(q8_ctx *c, const float *weight, size_t k) {
    if (!c || !weight || k == 0) return fail(Q8_ERR_INVALID, "q8_vector_resident: bad arguments");
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    float *w = nullptr;
    return vector_resident(c, weight, k, &w);
}

int q8_upload(q8_ctx *c, q8_dptr dst, const void *src, size_t bytes) {
    if (!c || (!src && bytes)) return fail(Q8_ERR_INVALID, "q8_upload: bad arguments");
    if (bytes == 0) return Q8_OK;
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    Q8_TRY(check_span(c, dst, bytes, "upload"));
    HIP_TRY(hipMemcpyAsync(reinterpret_cast<void *>(dst), src, bytes, hipMemcpyHostToDevice, c->stream),
            "hipMemcpyAsync(H2D)");
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return Q8_OK;
}

int q8_download(q8_ctx *c, void *dst, q8_dptr src, size_t bytes) {
    if (!c || (!dst && bytes)) return fail(Q8_ERR_INVALID, "q8_download: bad arguments");
    if (bytes == 0) return Q8_OK;
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    Q8_TRY(check_span(c, src, bytes, "download"));
    HIP_TRY(hipMemcpyAsync(dst, reinterpret_cast<const void *>(src), bytes, hipMemcpyDeviceToHost, c->stream),
            "hipMemcpyAsync(D2H)");
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return Q8_OK;
}

int q8_gemm_prefetch(q8_ctx *c, const q8_weight *const *weights, int count) {
    if (!c || count < 0 || count > Q8_RIDER_MAX || (count > 0 && !weights))
        return fail(Q8_ERR_INVALID, "q8_gemm_prefetch: bad arguments (count %d, at most %d)", count, Q8_RIDER_MAX);
    for (int i = 0; i < count; i++) Q8_TRY(check_weight(c, weights[i]));
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    c->next_weights.assign(weights, weights + count);
    return Q8_OK;
}

int q8_sync(q8_ctx *c) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_sync: null context");
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return Q8_OK;
}

// The device allocation of a weight: unit-layout quants, then the scales,
// then, where the weight's one-token GEMV runs in row slices under the
// default tactics, the slice-major copy of its quants (Q8SliceArgs): one more
// copy of the quants for one contiguous run per slice and wave load
// (configs[0] 4.50 -> 4.35 us a GEMV, down 2304 x 5760 5.25 -> 5.13 us).
struct WeightAlloc {
    size_t qbytes, sbytes, slices_off, total;
    int slice_rows;
};

WeightAlloc weight_alloc(q8_ctx *c, int out, int k, bool allow_slices = true) {
    WeightAlloc wa{};
    const int nb = k / 32;
    const int tiles = (int)ceil_div(out, Q8_TILE_ROWS);
    wa.qbytes = (size_t)tiles * nb * Q8_UNIT_BYTES;
    wa.sbytes = (size_t)tiles * nb * Q8_TILE_ROWS * 2;
    // the slice height this context's one-token GEMV of the shape runs in
    // (options gemv.rows / gemv.loads included, as they stand at residency)
    const q8_tactic t = plan(c, 1, out, k);
    // option gemv.slice_copy = 0: no copy (a context whose weights only ever
    // run in groups or GEMMs saves the memory)
    wa.slice_rows =
        ((t.row_slice == 8 || t.row_slice == 16) && allow_slices && option(c, "gemv.slice_copy", 1)) ? t.row_slice : 0;
    wa.slices_off = align_up(align_up(wa.qbytes, kAlign) + wa.sbytes, kAlign);
    wa.total = wa.slice_rows ? wa.slices_off + wa.qbytes : align_up(wa.qbytes, kAlign) + wa.sbytes;
    return wa;
}

// The slice-major copy of repacked quants (enqueued on the context's stream).
int slice_copy(q8_ctx *c, const uint8_t *quants, uint8_t *dst, int nb, int tiles, int rs, int pair_tiles = 0) {
    Q8SliceArgs a{quants, dst, nb, tiles, rs, pair_tiles};
    const long long threads = (long long)tiles * nb * 64;
    if (ceil_div(threads, 256) > 0x7fffffffLL) return fail(Q8_ERR_UNSUPPORTED, "weight of %d tiles is too large", tiles);
    return launch(c, F_SLICE_COPY, (unsigned)ceil_div(threads, 256), 256, 0, &a, sizeof a);
}

int q8_weight_resident(q8_ctx *c, const void *bytes, size_t nbytes, int k, int out, const q8_weight **weight) {
    if (!c || !bytes || !weight) return fail(Q8_ERR_INVALID, "q8_weight_resident: bad arguments");
    Q8_TRY(check_k(k));
    if (out <= 0) return fail(Q8_ERR_INVALID, "weight has %d rows", out);
    const int nb = k / 32;
    if (nbytes != (size_t)out * nb * Q8_BLOCK_BYTES)
        return fail(Q8_ERR_INVALID, "weight byte length mismatch: %zu bytes for %d x %d Q8_0", nbytes, out, k);
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    const auto key = std::make_pair((uintptr_t)bytes, nbytes);
    auto it = c->weights.find(key);
    if (it != c->weights.end()) {
        if (it->second->k != k || it->second->out != out)
            return fail(Q8_ERR_INVALID, "weight identity reused with another shape");
        *weight = it->second;
        return Q8_OK;
    }
    const int tiles = (int)ceil_div(out, Q8_TILE_ROWS);
    const WeightAlloc wa = weight_alloc(c, out, k);
    const size_t qbytes = wa.qbytes;
    const size_t total = wa.total;
    void *base = nullptr, *staging = nullptr;
    HIP_TRY(dev_malloc(c, &base, total), "hipMalloc(weight)");
    hipError_t e = dev_malloc(c, &staging, nbytes);
    if (e != hipSuccess) {
        hipFree(base);
        return hip_fail(e, "hipMalloc(weight staging)");
    }
    Q8RepackArgs a{};
    a.src = static_cast<const uint8_t *>(staging);
    a.quants = static_cast<uint8_t *>(base);
    a.scales = reinterpret_cast<uint16_t *>(static_cast<uint8_t *>(base) + align_up(qbytes, kAlign));
    a.rows = out;
    a.nb = nb;
    a.tiles = tiles;
    a.inverse = 0;
    int rc = Q8_OK;
    e = hipMemcpyAsync(staging, bytes, nbytes, hipMemcpyHostToDevice, c->stream);
    if (e != hipSuccess) rc = hip_fail(e, "hipMemcpyAsync(weight)");
    if (rc == Q8_OK) {
        const long long threads = (long long)tiles * Q8_TILE_ROWS * nb;
        if (threads > 0x7fffffffLL) rc = fail(Q8_ERR_UNSUPPORTED, "weight of %lld blocks is too large", threads);
        if (rc == Q8_OK) rc = launch(c, F_REPACK, (unsigned)ceil_div(threads, 256), 256, 0, &a, sizeof a);
    }
    uint8_t *slices = wa.slice_rows ? static_cast<uint8_t *>(base) + wa.slices_off : nullptr;
    if (rc == Q8_OK && slices) rc = slice_copy(c, a.quants, slices, nb, tiles, wa.slice_rows);
    if (rc == Q8_OK) {
        e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) rc = hip_fail(e, "hipStreamSynchronize");
    }
    hipFree(staging);
    if (rc != Q8_OK) {
        hipFree(base);
        return rc;
    }
    q8_weight *w = new q8_weight{c, base, a.quants, a.scales, k, out, nb, tiles, total, (uintptr_t)bytes, nbytes};
    w->slices = slices;
    w->slice_rows = wa.slice_rows;
    c->weights[key] = w;
    *weight = w;
    return Q8_OK;
}

int q8_weight_group_resident(q8_ctx *c, int count, const void *const *bytes, const size_t *nbytes, int k,
                             const int *outs, int pair, const q8_weight **weights) {
    if (!c || !bytes || !nbytes || !outs || !weights || (pair != 0 && pair != 1))
        return fail(Q8_ERR_INVALID, "q8_weight_group_resident: bad arguments");
    if (count < 1 || count > Q8_GROUP_MAX) return fail(Q8_ERR_INVALID, "a weight group holds one to four matrices");
    if (pair && (count != 2 || outs[0] != outs[1]))
        return fail(Q8_ERR_INVALID, "a gate/up pair holds two matrices of one shape");
    Q8_TRY(check_k(k));
    const int slice_rows = pair ? q8i::group_pair_slices(c, k) : q8i::group_slice_rows(c, k, 0);
    return build_group(c, k, count, outs, bytes, nbytes, nullptr, 0.0f, slice_rows, weights);
}

int q8_weight_release(q8_ctx *c, const q8_weight *w) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_weight_release: null context");
    Q8_TRY(check_weight(c, w));
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    // a pending announcement of this weight (q8_gemm_prefetch) goes with it:
    // no later launch may read its freed bytes
    c->next_weights.erase(std::remove(c->next_weights.begin(), c->next_weights.end(), w), c->next_weights.end());
    auto own = std::find(c->owned.begin(), c->owned.end(), w);
    if (own != c->owned.end()) {  // generated on the device
        HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
        // a group's allocation goes with its last member
        if (!w->group_refs || --*w->group_refs == 0) {
            hipFree(w->base);
            delete w->group_refs;
        }
        delete *own;
        c->owned.erase(own);
        return Q8_OK;
    }
    auto it = c->weights.find(std::make_pair(w->id_ptr, w->id_len));
    if (it == c->weights.end() || it->second != w) return fail(Q8_ERR_INVALID, "weight is not resident");
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (!w->group_refs || --*w->group_refs == 0) {
        hipFree(w->base);
        delete w->group_refs;
    }
    delete it->second;
    c->weights.erase(it);
    return Q8_OK;
}

int q8_vector_release(q8_ctx *c, const float *host, size_t len) {
    if (!c || !host) return fail(Q8_ERR_INVALID, "q8_vector_release: bad arguments");
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    auto it = c->vectors.find(std::make_pair((uintptr_t)host, len));
    if (it == c->vectors.end()) return Q8_OK;  // never made resident (or already released)
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");  // no kernel in flight reads it
    hipFree(it->second);
    c->vectors.erase(it);
    return Q8_OK;
}

int q8_weight_shape(const q8_weight *w, int *k, int *out, size_t *device_bytes) {
    if (!w) return fail(Q8_ERR_INVALID, "q8_weight_shape: null weight");
    if (k) *k = w->k;
    if (out) *out = w->out;
    if (device_bytes) *device_bytes = w->device_bytes;
    return Q8_OK;
}

int q8_weight_export(q8_ctx *c, const q8_weight *w, void *dst, size_t nbytes) {
    if (!c || !dst) return fail(Q8_ERR_INVALID, "q8_weight_export: bad arguments");
    Q8_TRY(check_weight(c, w));
    const size_t expect = (size_t)w->out * w->nb * Q8_BLOCK_BYTES;
    if (nbytes != expect) return fail(Q8_ERR_INVALID, "export buffer holds %zu bytes, weight is %zu", nbytes, expect);
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    void *staging = nullptr;
    HIP_TRY(dev_malloc(c, &staging, nbytes), "hipMalloc(export)");
    Q8RepackArgs a{};
    a.dst = static_cast<uint8_t *>(staging);
    a.quants = w->quants;
    a.scales = w->scales;
    a.rows = w->out;
    a.nb = w->nb;
    a.tiles = w->tiles;
    a.inverse = 1;
    const long long threads = (long long)w->tiles * Q8_TILE_ROWS * w->nb;
    int rc = launch(c, F_REPACK, (unsigned)ceil_div(threads, 256), 256, 0, &a, sizeof a);
    if (rc == Q8_OK) {
        hipError_t e = hipMemcpyAsync(dst, staging, nbytes, hipMemcpyDeviceToHost, c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) rc = hip_fail(e, "hipMemcpyAsync(export)");
    }
    hipFree(staging);
    return rc;
}

int q8_prepare(q8_ctx *c, q8_dptr x, size_t x_offset, int n, int k, q8_prepared *out) {
    if (!c || !out) return fail(Q8_ERR_INVALID, "q8_prepare: bad arguments");
    Q8_TRY(check_k(k));
    Q8_TRY(check_n(n));
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    const q8_dptr xp = (q8_dptr)(uintptr_t)fptr(x, x_offset);
    Q8_TRY(check_span(c, xp, (size_t)n * k * 4, "prepare x"));
    return prepare_into(c, xp, 0, 0, n, k, out);
}

int q8_silu_mul_prepare(q8_ctx *c, q8_dptr gate, q8_dptr up, int n, int k, q8_prepared *out) {
    if (!c || !out) return fail(Q8_ERR_INVALID, "q8_silu_mul_prepare: bad arguments");
    Q8_TRY(check_k(k));
    Q8_TRY(check_n(n));
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    Q8_TRY(check_span(c, gate, (size_t)n * k * 4, "silu gate"));
    Q8_TRY(check_span(c, up, (size_t)n * k * 4, "silu up"));
    return prepare_into(c, 0, gate, up, n, k, out);
}

int q8_silu_mul(q8_ctx *c, q8_dptr act, q8_dptr gate, q8_dptr up, size_t len) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_silu_mul: null context");
    if (len == 0) return Q8_OK;
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    Q8_TRY(check_span(c, act, len * 4, "silu act"));
    Q8_TRY(check_span(c, gate, len * 4, "silu gate"));
    Q8_TRY(check_span(c, up, len * 4, "silu up"));
    Q8EltArgs a{};
    a.act = reinterpret_cast<float *>(act);
    a.gate = reinterpret_cast<const float *>(gate);
    a.up = reinterpret_cast<const float *>(up);
    a.len = (long long)len;
    return launch(c, F_SILU_MUL, (unsigned)ceil_div((long long)len, 256), 256, 0, &a, sizeof a);
}

int q8_matmul_decode_group(q8_ctx *c, const q8_group_entry *group, int count, q8_dptr x, size_t x_offset, int k,
                           q8_dptr bias, size_t bias_offset) {
    if (!c || !group) return fail(Q8_ERR_INVALID, "q8_matmul_decode_group: bad arguments");
    if (count < 1 || count > Q8_GROUP_MAX)
        return fail(Q8_ERR_INVALID, "decode matmul group holds one to four matrices (got %d)", count);
    if (bias && count != 1) return fail(Q8_ERR_INVALID, "a residual add belongs to a single-matrix group");
    Q8_TRY(check_k(k));
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    Member m[Q8_GROUP_MAX];
    for (int i = 0; i < count; i++) {
        Q8_TRY(check_weight(c, group[i].weight));
        if (group[i].weight->k != k) return fail(Q8_ERR_INVALID, "group member %d has k = %d, not %d", i, group[i].weight->k, k);
        m[i].w = group[i].weight;
        m[i].y = fptr(group[i].y, group[i].y_offset);
        Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)m[i].y, (size_t)m[i].w->out * 4, "decode y"));
    }
    const q8_dptr xp = (q8_dptr)(uintptr_t)fptr(x, x_offset);
    Q8_TRY(check_span(c, xp, (size_t)k * 4, "decode x"));
    const float *b = fptr(bias, bias_offset);
    if (b) Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)b, (size_t)m[0].w->out * 4, "decode bias"));
    return run_gemv(c, m, count, xp, k, b, 0);
}

int q8_matmul_prompt_group(q8_ctx *c, const q8_group_entry *group, int count, const q8_prepared *prepared, int n,
                           int k, q8_dptr bias, size_t bias_offset) {
    if (!c || !group || !prepared) return fail(Q8_ERR_INVALID, "q8_matmul_prompt_group: bad arguments");
    if (count < 1 || count > Q8_GROUP_MAX)
        return fail(Q8_ERR_INVALID, "prompt matmul group holds one to four matrices (got %d)", count);
    if (bias && count != 1) return fail(Q8_ERR_INVALID, "a residual add belongs to a single-matrix group");
    Q8_TRY(check_k(k));
    Q8_TRY(check_n(n));
    if (prepared->n != n || prepared->k != k)
        return fail(Q8_ERR_INVALID, "prepared activations are %d x %d, the matmul wants %d x %d", prepared->n,
                    prepared->k, n, k);
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    Member m[Q8_GROUP_MAX];
    for (int i = 0; i < count; i++) {
        Q8_TRY(check_weight(c, group[i].weight));
        if (group[i].weight->k != k) return fail(Q8_ERR_INVALID, "group member %d has k = %d, not %d", i, group[i].weight->k, k);
        m[i].w = group[i].weight;
        m[i].y = fptr(group[i].y, group[i].y_offset);
        Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)m[i].y, (size_t)n * m[i].w->out * 4, "prompt y"));
    }
    const float *b = fptr(bias, bias_offset);
    if (b) Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)b, (size_t)n * m[0].w->out * 4, "prompt bias"));
    return run_gemm(c, m, count, prepared, n, b);
}

int run_gemv_q8x(q8_ctx *c, const q8_weight *w, q8_dptr x, size_t x_offset, int n, float *y, const float *bias);

int q8_matmul(q8_ctx *c, const q8_weight *w, q8_dptr x, size_t x_offset, int n, q8_dptr y, size_t y_offset,
              const q8_prepared *prepared, q8_dptr bias, size_t bias_offset) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_matmul: null context");
    Q8_TRY(check_weight(c, w));
    Q8_TRY(check_n(n));
    q8_group_entry e{w, y, y_offset};
    if (n == 1) return q8_matmul_decode_group(c, &e, 1, x, x_offset, w->k, bias, bias_offset);
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    if (!prepared && n == 2 && option(c, "gemm.small_gemv", 1)) {
        // two tokens of f32 x: the quantized-x GEMV reads the weights once for both
        const int rc = run_gemv_q8x(c, w, x, x_offset, n, fptr(y, y_offset), bias ? fptr(bias, bias_offset) : nullptr);
        if (rc != Q8_ERR_UNSUPPORTED) return rc;
    }
    q8_prepared own{};
    if (!prepared) {
        Q8_TRY(q8_prepare(c, x, x_offset, n, w->k, &own));
        prepared = &own;
    }
    return q8_matmul_prompt_group(c, &e, 1, prepared, n, w->k, bias, bias_offset);
}

// The quantized-x row-slice GEMV (q8_gemv_q8x{1,2}_*) over one or two
// tokens of f32 x: the f32 GEMV's row slices where its tactic takes them,
// else 16-row slices (8-row with six loads past 192 blocks), at most 16
// waves; Q8_ERR_UNSUPPORTED past that or past 64 KiB of LDS (the caller may
// keep the GEMM).
int run_gemv_q8x(q8_ctx *c, const q8_weight *w, q8_dptr x, size_t x_offset, int n, float *y, const float *bias) {
    const int k = w->k;
    const int nb = w->nb;
    if (n < 1 || n > 2) return fail(Q8_ERR_UNSUPPORTED, "quantized-x GEMV: %d tokens (1 or 2)", n);
    const int nt = n;
    const q8_dptr xp = (q8_dptr)(uintptr_t)fptr(x, x_offset);
    Q8_TRY(check_span(c, xp, (size_t)n * k * 4, "gemv x"));
    Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)y, (size_t)n * w->out * 4, "gemv y"));
    if (bias) Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)bias, (size_t)n * w->out * 4, "gemv bias"));
    const q8_tactic t = plan(c, 1, w->out, k, 1);
    int rs = 16, nl = nb <= 96 ? 3 : 6;
    if (t.row_slice == 8 || t.row_slice == 16) {
        rs = t.row_slice;
        nl = t.slice_loads == 2 || t.slice_loads == 3 ? t.slice_loads : 6;
    }
    if (nb > 16 * nl * (64 / (2 * rs))) {
        rs = 8;
        nl = 6;
    }
    const int bpw = nl * (64 / (2 * rs));
    const int waves = (int)ceil_div(nb, bpw);
    if (waves > 16)
        return fail(Q8_ERR_UNSUPPORTED, "quantized-x GEMV: k = %d needs %d waves a workgroup (16 at most)", k, waves);
    // quant bytes and block scales per token, the waves' row sums, the dead lanes' pad
    const size_t lds = ((size_t)nt * nb * 8 + (size_t)nt * nb + (size_t)nt * waves * rs + Q8_GEMV_PAD_FLOATS) * 4;
    if (lds > 65536)
        return fail(Q8_ERR_UNSUPPORTED, "quantized-x GEMV: %zu bytes of LDS for %d tokens of k = %d", lds, nt, k);
    Q8GemvArgs a{};
    a.members = 1;
    a.m[0].quants = w->quants;
    a.m[0].scales = w->scales;
    a.m[0].y = y;
    a.m[0].bias = bias;
    a.m[0].rows = w->out;
    a.total_tiles = w->tiles;
    a.x = reinterpret_cast<const float *>(xp);
    a.nb = nb;
    a.waves_per_tile = waves;
    a.kslices = 1;
    a.tokens = n;
    a.xcd_order = option(c, "gemv.xcd_order", 1) ? 1 : 0;
    const long long grid = (a.xcd_order ? ceil_div(w->tiles, 8) * 8 : (long long)w->tiles) * (Q8_TILE_ROWS / rs);
    if (grid > 0x7fffffffLL) return fail(Q8_ERR_UNSUPPORTED, "quantized-x GEMV: grid of %lld workgroups", grid);
    const Fn f = nl == 2 ? (nt == 1 ? F_GEMV_Q8X1_8_2 : F_GEMV_Q8X2_8_2)
                         : (Fn)(F_GEMV_Q8X1_8_3 + 4 * (nt - 1) + (rs == 8 ? 0 : 2) + (nl == 3 ? 0 : 1));
    if (nb > 0xffff || w->tiles > 0x3fffffff || w->out >= (1 << 24))
        return fail(Q8_ERR_UNSUPPORTED, "quantized-x GEMV: %d x %d", w->out, k);
    // the preloaded head of the row-slice GEMVs, the token count above the rows
    const bool sm = w->slices && w->slice_rows == rs && option(c, "gemv.slice_copy", 1);
    RsHead h{sm ? w->slices : w->quants, w->scales, y, bias, a.x, w->out | (nt << 24), nb | (waves << 16),
             (int)((unsigned)w->tiles | ((unsigned)sm << 30) | ((unsigned)a.xcd_order << 31)), 0};
    return launch_rs(c, f, (unsigned)grid, (unsigned)(waves * 64), (unsigned)lds, h, a);
}

int q8_matmul_q8(q8_ctx *c, const q8_weight *w, q8_dptr x, size_t x_offset, int n, q8_dptr y, size_t y_offset,
                 q8_dptr bias, size_t bias_offset) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_matmul_q8: null context");
    Q8_TRY(check_weight(c, w));
    Q8_TRY(check_n(n));
    if (n >= 2) return q8_matmul(c, w, x, x_offset, n, y, y_offset, nullptr, bias, bias_offset);
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    return run_gemv_q8x(c, w, x, x_offset, 1, fptr(y, y_offset), bias ? fptr(bias, bias_offset) : nullptr);
}

int q8_matmul_noalloc(q8_ctx *c, const q8_weight *w, q8_dptr x, size_t x_offset, int n, q8_dptr y,
                      size_t y_offset, q8_dptr bias, size_t bias_offset) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_matmul_noalloc: null context");
    Q8_TRY(check_weight(c, w));
    Q8_TRY(check_n(n));
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    const int k = w->k;
    if (n == 1) {
        // the GEMV reads x and writes y only, unless K is split over workgroups
        if (plan(c, 1, w->out, k, 1).kslices != 1)
            return fail(Q8_ERR_UNSUPPORTED, "q8_matmul_noalloc: the %d x %d GEMV splits K over workgroups, which "
                                            "needs scratch", w->out, k);
        q8_group_entry e{w, y, y_offset};
        return q8_matmul_decode_group(c, &e, 1, x, x_offset, k, bias, bias_offset);
    }
    if (n == 2 && option(c, "gemm.small_gemv", 1)) {
        // q8_matmul's two-token GEMV: x is quantized in LDS, no scratch
        const int rc = run_gemv_q8x(c, w, x, x_offset, n, fptr(y, y_offset), bias ? fptr(bias, bias_offset) : nullptr);
        if (rc != Q8_ERR_UNSUPPORTED) return rc;
    }
    if (!c->noalloc) return fail(Q8_ERR_NO_DEVICE, "q8_matmul_noalloc: no device scratch");
    const size_t need = prepared_bytes(n, k, Q8_PREPARED_I8, nullptr);
    if (need > Q8_NOALLOC_SCRATCH_BYTES)
        return fail(Q8_ERR_UNSUPPORTED, "q8_matmul_noalloc: %d tokens of k = %d need %zu bytes of quantized "
                                        "activations, more than the %u-byte scratch", n, k, need,
                    (unsigned)Q8_NOALLOC_SCRATCH_BYTES);
    const q8_dptr xp = (q8_dptr)(uintptr_t)fptr(x, x_offset);
    Q8_TRY(check_span(c, xp, (size_t)n * k * 4, "noalloc x"));
    Member m{w, fptr(y, y_offset)};
    Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)m.y, (size_t)n * w->out * 4, "noalloc y"));
    const float *b = fptr(bias, bias_offset);
    if (b) Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)b, (size_t)n * w->out * 4, "noalloc bias"));
    // claimed only by a call that passed every check and will use the array:
    // a refused call leaves the scratch to whoever takes it next
    if (!q8i::noalloc_claim(c->device, c))
        return fail(Q8_ERR_UNSUPPORTED, "q8_matmul_noalloc: device %d's scratch is held by another context (the "
                                        "first context to use it keeps it until q8_close)", c->device);
    q8_prepared p{};
    Q8_TRY(run_quantize(c, xp, 0, 0, n, k, Q8_PREPARED_I8, c->noalloc, &p));
    return run_gemm(c, &m, 1, &p, n, b, nullptr, true);
}

int q8_gate_up_silu(q8_ctx *c, const q8_weight *gate, const q8_weight *up, q8_dptr x, size_t x_offset, int n,
                    q8_dptr act, size_t act_offset, q8_prepared *prepared) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_gate_up_silu: null context");
    Q8_TRY(check_weight(c, gate));
    Q8_TRY(check_weight(c, up));
    Q8_TRY(check_n(n));
    if (gate->k != up->k || gate->out != up->out)
        return fail(Q8_ERR_INVALID, "gate is %d x %d but up is %d x %d", gate->out, gate->k, up->out, up->k);
    const int k = gate->k, ffn = gate->out;
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    float *actp = fptr(act, act_offset);
    Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)actp, (size_t)n * ffn * 4, "gate_up act"));
    const q8_dptr xp = (q8_dptr)(uintptr_t)fptr(x, x_offset);
    Q8_TRY(check_span(c, xp, (size_t)n * k * 4, "gate_up x"));
    if (n == 1) {
        const q8_tactic t = plan(c, 1, ffn, k, 2);
        if (t.pairs_per_wave <= 12 && t.waves_per_tile <= 8) {
            Member m[2] = {{gate, actp}, {up, nullptr}};
            Q8_TRY(run_gemv(c, m, 2, xp, k, nullptr, 1));
            if (prepared) Q8_TRY(prepare_into(c, (q8_dptr)(uintptr_t)actp, 0, 0, 1, ffn, prepared));
            return Q8_OK;
        }
    }
    if (n >= 2 && prepared && ffn % 32 == 0 && option(c, "gemm.silu", 1)) {
        q8_prepared px{};
        Q8_TRY(prepare_into(c, xp, 0, 0, n, k, &px));
        if (px.format == Q8_PREPARED_I8) return run_gemm_silu(c, gate, up, &px, n, prepared);
    }
    // gate and up products in f32 workspace, then the SiLU product.
    const size_t one = align_up((size_t)n * ffn * 4, kAlign);
    Q8_TRY(grow(c, &c->tmp_ws, &c->tmp_ws_bytes, 2 * one, "hipMalloc(ffn workspace)"));
    float *g = static_cast<float *>(c->tmp_ws);
    float *u = reinterpret_cast<float *>(static_cast<uint8_t *>(c->tmp_ws) + one);
    Member m[2] = {{gate, g}, {up, u}};
    if (n == 1) {
        Q8_TRY(run_gemv(c, m, 2, xp, k, nullptr, 0));
    } else {
        q8_prepared px{};
        Q8_TRY(prepare_into(c, xp, 0, 0, n, k, &px));
        Q8_TRY(run_gemm(c, m, 2, &px, n, nullptr));
    }
    if (prepared) {
        // compute.rs:993-1019: the product goes straight to Q8_0 for the down
        // matmul and is never written in f32
        return prepare_into(c, 0, (q8_dptr)(uintptr_t)g, (q8_dptr)(uintptr_t)u, n, ffn, prepared);
    }
    Q8EltArgs a{};
    a.act = actp;
    a.gate = g;
    a.up = u;
    a.len = (long long)n * ffn;
    return launch(c, F_SILU_MUL, (unsigned)ceil_div(a.len, 256), 256, 0, &a, sizeof a);
}

int q8_norm_matmul_decode_group(q8_ctx *c, const float *norm_weight, float eps, const q8_group_entry *group,
                                int count, q8_dptr x, size_t x_offset, int k) {
    if (!c || !group || !norm_weight) return fail(Q8_ERR_INVALID, "q8_norm_matmul_decode_group: bad arguments");
    if (count < 1 || count > Q8_GROUP_MAX)
        return fail(Q8_ERR_INVALID, "decode matmul group holds one to four matrices (got %d)", count);
    Q8_TRY(check_k(k));
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    Member m[Q8_GROUP_MAX];
    for (int i = 0; i < count; i++) {
        Q8_TRY(check_weight(c, group[i].weight));
        if (group[i].weight->k != k) return fail(Q8_ERR_INVALID, "group member %d has k = %d, not %d", i, group[i].weight->k, k);
        m[i].w = group[i].weight;
        m[i].y = fptr(group[i].y, group[i].y_offset);
        Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)m[i].y, (size_t)m[i].w->out * 4, "decode y"));
    }
    const q8_dptr xp = (q8_dptr)(uintptr_t)fptr(x, x_offset);
    Q8_TRY(check_span(c, xp, (size_t)k * 4, "decode x"));
    float *w = nullptr;
    Q8_TRY(vector_resident(c, norm_weight, (size_t)k, &w));
    return run_norm_gemv(c, m, count, xp, k, 0, w, eps);
}

int q8_norm_gate_up_silu(q8_ctx *c, const float *norm_weight, float eps, const q8_weight *gate, const q8_weight *up,
                         q8_dptr x, size_t x_offset, q8_dptr act, size_t act_offset) {
    if (!c || !norm_weight) return fail(Q8_ERR_INVALID, "q8_norm_gate_up_silu: bad arguments");
    Q8_TRY(check_weight(c, gate));
    Q8_TRY(check_weight(c, up));
    if (gate->k != up->k || gate->out != up->out)
        return fail(Q8_ERR_INVALID, "gate is %d x %d but up is %d x %d", gate->out, gate->k, up->out, up->k);
    const int k = gate->k, ffn = gate->out;
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    float *actp = fptr(act, act_offset);
    Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)actp, (size_t)ffn * 4, "gate_up act"));
    const q8_dptr xp = (q8_dptr)(uintptr_t)fptr(x, x_offset);
    Q8_TRY(check_span(c, xp, (size_t)k * 4, "gate_up x"));
    float *w = nullptr;
    Q8_TRY(vector_resident(c, norm_weight, (size_t)k, &w));
    const q8_tactic t = plan(c, 1, ffn, k, 2);
    Member m[2] = {{gate, actp}, {up, nullptr}};
    if (t.pairs_per_wave <= 12 && t.waves_per_tile <= 8) return run_norm_gemv(c, m, 2, xp, k, 1, w, eps);
    // the pair does not fit one launch: the norm, then the unfused gate/up path
    Q8_TRY(grow(c, &c->norm_ws, &c->norm_ws_bytes, (size_t)k * sizeof(float), "hipMalloc(norm workspace)"));
    float *xn = static_cast<float *>(c->norm_ws);
    Q8_TRY(run_rmsnorm(c, reinterpret_cast<const float *>(xp), 1, k, w, eps, xn, nullptr));
    return q8_gate_up_silu(c, gate, up, (q8_dptr)(uintptr_t)xn, 0, 1, act, act_offset, nullptr);
}

int q8_gate_up_silu_prepared(q8_ctx *c, const q8_weight *gate, const q8_weight *up, const q8_prepared *x,
                             q8_prepared *out) {
    if (!c || !x || !out) return fail(Q8_ERR_INVALID, "q8_gate_up_silu_prepared: bad arguments");
    Q8_TRY(check_weight(c, gate));
    Q8_TRY(check_weight(c, up));
    Q8_TRY(check_n(x->n));
    if (gate->k != up->k || gate->out != up->out)
        return fail(Q8_ERR_INVALID, "gate is %d x %d but up is %d x %d", gate->out, gate->k, up->out, up->k);
    if (x->k != gate->k) return fail(Q8_ERR_INVALID, "prepared activations have k = %d, weights %d", x->k, gate->k);
    if (x->n < 2) return fail(Q8_ERR_INVALID, "prepared activations are for n >= 2 (got %d)", x->n);
    Q8_TRY(check_k(gate->out));
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    const int n = x->n, ffn = gate->out;
    if (x->format == Q8_PREPARED_I8 && option(c, "gemm.silu", 1)) return run_gemm_silu(c, gate, up, x, n, out);
    const size_t one = align_up((size_t)n * ffn * 4, kAlign);
    Q8_TRY(grow(c, &c->tmp_ws, &c->tmp_ws_bytes, 2 * one, "hipMalloc(ffn workspace)"));
    float *g = static_cast<float *>(c->tmp_ws);
    float *u = reinterpret_cast<float *>(static_cast<uint8_t *>(c->tmp_ws) + one);
    Member m[2] = {{gate, g}, {up, u}};
    Q8_TRY(run_gemm(c, m, 2, x, n, nullptr));
    return prepare_into(c, 0, (q8_dptr)(uintptr_t)g, (q8_dptr)(uintptr_t)u, n, ffn, out);
}

int q8_rmsnorm(q8_ctx *c, q8_dptr x, size_t x_offset, const float *weight, int k, float eps, int rows, q8_dptr out,
               size_t out_offset) {
    if (!c || !weight) return fail(Q8_ERR_INVALID, "q8_rmsnorm: bad arguments");
    Q8_TRY(check_k(k));
    if (rows < 1) return fail(Q8_ERR_INVALID, "q8_rmsnorm: %d rows", rows);
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    const float *xp = fptr(x, x_offset);
    float *op = fptr(out, out_offset);
    Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)xp, (size_t)rows * k * 4, "rmsnorm x"));
    Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)op, (size_t)rows * k * 4, "rmsnorm out"));
    float *w = nullptr;
    Q8_TRY(vector_resident(c, weight, (size_t)k, &w));
    return run_rmsnorm(c, xp, rows, k, w, eps, op, nullptr);
}

int q8_norm_prepare(q8_ctx *c, q8_dptr x, size_t x_offset, const float *weight, int k, float eps, int rows,
                    q8_prepared *prepared) {
    if (!c || !weight || !prepared) return fail(Q8_ERR_INVALID, "q8_norm_prepare: bad arguments");
    Q8_TRY(check_k(k));
    Q8_TRY(check_n(rows));
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    const float *xp = fptr(x, x_offset);
    Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)xp, (size_t)rows * k * 4, "norm_prepare x"));
    float *w = nullptr;
    Q8_TRY(vector_resident(c, weight, (size_t)k, &w));
    return run_rmsnorm(c, xp, rows, k, w, eps, nullptr, prepared);
}

int q8_copy_device(q8_ctx *c, q8_dptr dst, q8_dptr src, size_t bytes) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_copy_device: null context");
    if (bytes == 0) return Q8_OK;
    if (bytes % 16 != 0 || dst % 16 != 0 || src % 16 != 0)
        return fail(Q8_ERR_INVALID, "q8_copy_device: pointers and size must be 16-byte multiples");
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    Q8_TRY(check_span(c, dst, bytes, "copy dst"));
    Q8_TRY(check_span(c, src, bytes, "copy src"));
    Q8CopyArgs a{};
    a.src = reinterpret_cast<const uint8_t *>(src);
    a.dst = reinterpret_cast<uint8_t *>(dst);
    a.bytes = (long long)bytes;
    a.blocks = (int)std::min<long long>(ceil_div((long long)(bytes / 16), 256), 8LL * c->cu_count);
    return launch(c, F_COPY, (unsigned)a.blocks, 256, 0, &a, sizeof a);
}

int q8_lm_head_argmax(q8_ctx *c, const q8_weight *w, q8_dptr x, size_t x_offset, q8_dptr logits,
                      size_t logits_offset, uint32_t *argmax) {
    if (!c || !argmax) return fail(Q8_ERR_INVALID, "q8_lm_head_argmax: bad arguments");
    Q8_TRY(check_weight(c, w));
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    uint8_t *ws = static_cast<uint8_t *>(c->argmax_ws);
    const q8_dptr slot = (q8_dptr)(uintptr_t)(ws + (size_t)kArgmaxMaxParts * 8);
    Q8_TRY(q8_norm_lm_head_argmax(c, nullptr, 0.0f, w, x, x_offset, logits, logits_offset, slot));
    uint32_t result = 0;
    HIP_TRY(hipMemcpyAsync(&result, reinterpret_cast<void *>(slot), 4, hipMemcpyDeviceToHost, c->stream),
            "hipMemcpyAsync(argmax)");
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    *argmax = result;
    return Q8_OK;
}

// Output norm, lm_head and greedy choice: the row norm into the norm
// workspace (not folded: every one of the lm_head's thousands of workgroups
// would sum the row's squares again, 63.8 against 49.4 + 3.7 us measured),
// the GEMV, which writes the logits and each 32-row tile's best candidate,
// and one workgroup of q8_argmax's second stage picking among the candidates
// -- the argmax's first pass over the logits is gone.  Shapes whose GEMV
// cannot carry the partials (a K split) run the two-stage argmax.
int q8_norm_lm_head_argmax(q8_ctx *c, const float *norm_weight, float eps, const q8_weight *w, q8_dptr x,
                           size_t x_offset, q8_dptr logits, size_t logits_offset, q8_dptr result) {
    if (!c || !w) return fail(Q8_ERR_INVALID, "q8_norm_lm_head_argmax: bad arguments");
    Q8_TRY(check_weight(c, w));
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    const int k = w->k;
    const q8_dptr xp = (q8_dptr)(uintptr_t)fptr(x, x_offset);
    Q8_TRY(check_span(c, xp, (size_t)k * 4, "lm_head x"));
    float *yp = fptr(logits, logits_offset);
    Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)yp, (size_t)w->out * 4, "lm_head logits"));
    Q8_TRY(check_span(c, result, 4, "argmax result"));
    q8_dptr xin = xp;
    if (norm_weight) {
        float *nw = nullptr;
        Q8_TRY(vector_resident(c, norm_weight, (size_t)k, &nw));
        Q8_TRY(grow(c, &c->norm_ws, &c->norm_ws_bytes, (size_t)k * sizeof(float), "hipMalloc(norm workspace)"));
        Q8_TRY(run_rmsnorm(c, reinterpret_cast<const float *>(xp), 1, k, nw, eps, static_cast<float *>(c->norm_ws),
                           nullptr));
        xin = (q8_dptr)(uintptr_t)c->norm_ws;
    }
    Member m{w, yp};
    const q8_tactic t = plan(c, 1, w->out, k, 1);
    if (t.kslices == 1 && w->tiles <= kArgmaxMaxParts) {
        uint8_t *ws = static_cast<uint8_t *>(c->argmax_ws);
        const GemvArgmax amax{reinterpret_cast<float *>(ws), reinterpret_cast<unsigned *>(ws + kArgmaxMaxParts * 4)};
        Q8_TRY(run_gemv(c, &m, 1, xin, k, nullptr, 0, nullptr, 0.0f, nullptr, nullptr, &amax));
        Q8ArgmaxArgs a{};
        a.values = yp;
        a.len = w->out;
        a.part_value = amax.value;
        a.part_index = amax.index;
        a.result = reinterpret_cast<unsigned *>(result);
        a.parts = w->tiles;
        a.stage = 1;
        return launch(c, F_ARGMAX, 1, 256, 0, &a, sizeof a);
    }
    Q8_TRY(run_gemv(c, &m, 1, xin, k, nullptr, 0));
    return q8_argmax_device(c, (q8_dptr)(uintptr_t)yp, 0, (size_t)w->out, result);
}

int q8_embeddings(q8_ctx *c, const q8_weight *w, const uint32_t *tokens, size_t n, q8_dptr out,
                  size_t out_offset) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_embeddings: null context");
    Q8_TRY(check_weight(c, w));
    if (n == 0) return Q8_OK;
    if (!tokens) return fail(Q8_ERR_INVALID, "q8_embeddings: null token ids");
    for (size_t i = 0; i < n; i++)
        if (tokens[i] >= (uint32_t)w->out) return fail(Q8_ERR_INVALID, "token %u outside vocabulary", tokens[i]);
    const long long threads = (long long)n * w->nb * 2;
    if (threads > 0x7fffffffLL) return fail(Q8_ERR_UNSUPPORTED, "embedding of %zu tokens is too large", n);
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    Q8_TRY(check_span(c, out, ((size_t)out_offset + n * (size_t)w->k) * sizeof(float), "embedding output"));
    Q8_TRY(grow(c, &c->token_ws, &c->token_ws_bytes, n * sizeof(uint32_t), "hipMalloc(token ids)"));
    HIP_TRY(hipMemcpyAsync(c->token_ws, tokens, n * sizeof(uint32_t), hipMemcpyHostToDevice, c->stream),
            "hipMemcpyAsync(token ids)");
    HIP_TRY(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return q8_embeddings_device(c, w, (q8_dptr)(uintptr_t)c->token_ws, n, out, out_offset);
}

int q8_embeddings_device(q8_ctx *c, const q8_weight *w, q8_dptr tokens, size_t n, q8_dptr out, size_t out_offset) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_embeddings_device: null context");
    Q8_TRY(check_weight(c, w));
    if (n == 0) return Q8_OK;
    const long long threads = (long long)n * w->nb * 2;
    if (threads > 0x7fffffffLL) return fail(Q8_ERR_UNSUPPORTED, "embedding of %zu tokens is too large", n);
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    Q8_TRY(check_span(c, tokens, n * sizeof(uint32_t), "embedding token ids"));
    Q8_TRY(check_span(c, out, ((size_t)out_offset + n * (size_t)w->k) * sizeof(float), "embedding output"));
    Q8EmbedArgs a{};
    a.quants = w->quants;
    a.scales = w->scales;
    a.tokens = reinterpret_cast<const uint32_t *>(tokens);
    a.out = fptr(out, out_offset);
    a.n = (int)n;
    a.nb = w->nb;
    a.rows = w->out;
    return launch(c, F_EMBED, (unsigned)ceil_div(threads, 256), 256, 0, &a, sizeof a);
}

int q8_argmax_device(q8_ctx *c, q8_dptr values, size_t offset, size_t len, q8_dptr result) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_argmax_device: null context");
    if (len == 0) return fail(Q8_ERR_INVALID, "argmax of an empty vector");
    if (len > 0xfffffffeULL) return fail(Q8_ERR_INVALID, "argmax length %zu exceeds u32 indices", len);
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    const q8_dptr v = (q8_dptr)(uintptr_t)fptr(values, offset);
    Q8_TRY(check_span(c, v, len * 4, "argmax values"));
    Q8_TRY(check_span(c, result, 4, "argmax result"));
    uint8_t *ws = static_cast<uint8_t *>(c->argmax_ws);
    Q8ArgmaxArgs a{};
    a.values = reinterpret_cast<const float *>(v);
    a.len = (long long)len;
    a.part_value = reinterpret_cast<float *>(ws);
    a.part_index = reinterpret_cast<unsigned *>(ws + kArgmaxMaxParts * 4);
    a.result = reinterpret_cast<unsigned *>(result);
    a.parts = (int)std::min<long long>(kArgmaxParts, std::max<long long>(1, ceil_div((long long)len, 4096)));
    a.stage = 0;
    Q8_TRY(launch(c, F_ARGMAX, (unsigned)a.parts, 256, 0, &a, sizeof a));
    a.stage = 1;
    return launch(c, F_ARGMAX, 1, 256, 0, &a, sizeof a);
}

// RopeTable::new (ops.rs:121-131): frequency = base.powf(-2.0 * pair / n_rot)
// in f32, from the C library's powf as the reference's table is; uploaded
// once per (n_rot, base) and kept (never inside a capture: the eager pass of a
// shape runs first).
int rope_table(q8_ctx *c, int n_rot, float base, const float **out) {
    uint32_t base_bits;
    std::memcpy(&base_bits, &base, 4);
    const auto fkey = std::make_pair(n_rot, base_bits);
    auto fit = c->rope_freq.find(fkey);
    if (fit == c->rope_freq.end()) {
        std::vector<float> table(std::max(1, n_rot / 2));
        for (int i = 0; i < n_rot / 2; i++) table[i] = powf(base, (-2.0f * (float)i) / (float)n_rot);
        float *dev = nullptr;
        HIP_TRY(dev_malloc(c, reinterpret_cast<void **>(&dev), table.size() * 4), "hipMalloc(rope table)");
        hipError_t e = hipMemcpyAsync(dev, table.data(), table.size() * 4, hipMemcpyHostToDevice, c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) {
            hipFree(dev);
            return hip_fail(e, "upload(rope table)");
        }
        fit = c->rope_freq.emplace(fkey, dev).first;
    }
    *out = fit->second;
    return Q8_OK;
}

int q8_norm_qkv_rope(q8_ctx *c, const float *norm_weight, float eps, const q8_weight *wq, const q8_weight *wk,
                     const q8_weight *wv, q8_dptr x, size_t x_offset, q8_dptr q, size_t q_offset, q8_dptr kcache,
                     q8_dptr vcache, int n_head, int n_kv, int head_dim, int n_rot, float base, int capacity,
                     q8_dptr position) {
    if (!c || !norm_weight) return fail(Q8_ERR_INVALID, "q8_norm_qkv_rope: bad arguments");
    if (n_head < 1 || n_kv < 1 || n_head % n_kv || head_dim < 2 || head_dim % 2 || n_rot < 0 || n_rot > head_dim ||
        n_rot % 2 || capacity < 1)
        return fail(Q8_ERR_INVALID, "norm_qkv_rope: bad geometry (heads %d/%d, head_dim %d, n_rot %d)", n_head, n_kv,
                    head_dim, n_rot);
    Q8_TRY(check_weight(c, wq));
    Q8_TRY(check_weight(c, wk));
    Q8_TRY(check_weight(c, wv));
    const int k = wq->k;
    const int kv_dim = n_kv * head_dim;
    if (wk->k != k || wv->k != k || wq->out != n_head * head_dim || wk->out != kv_dim || wv->out != kv_dim)
        return fail(Q8_ERR_INVALID, "norm_qkv_rope: q/k/v weights are %dx%d, %dx%d, %dx%d for %d/%d heads of %d",
                    wq->out, wq->k, wk->out, wk->k, wv->out, wv->k, n_head, n_kv, head_dim);
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    const q8_dptr xp = (q8_dptr)(uintptr_t)fptr(x, x_offset);
    float *qp = fptr(q, q_offset);
    Q8_TRY(check_span(c, xp, (size_t)k * 4, "qkv x"));
    Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)qp, (size_t)wq->out * 4, "rope q"));
    Q8_TRY(check_span(c, kcache, (size_t)capacity * kv_dim * 2, "key cache"));
    Q8_TRY(check_span(c, vcache, (size_t)capacity * kv_dim * 2, "value cache"));
    Q8_TRY(check_span(c, position, 4, "position"));
    float *w = nullptr;
    Q8_TRY(vector_resident(c, norm_weight, (size_t)k, &w));
    GemvRope rope{};
    Q8_TRY(rope_table(c, n_rot, base, &rope.freq));
    rope.position = reinterpret_cast<const int *>(position);
    rope.kcache = reinterpret_cast<uint16_t *>(kcache);
    rope.vcache = reinterpret_cast<uint16_t *>(vcache);
    rope.head_dim = head_dim;
    rope.n_rot = n_rot;
    rope.capacity = capacity;
    Member m[3] = {{wq, qp}, {wk, nullptr}, {wv, nullptr}};
    return run_norm_gemv(c, m, 3, xp, k, 0, w, eps, &rope);
}

int q8_prompt_qkv_rope(q8_ctx *c, const q8_weight *wq, const q8_weight *wk, const q8_weight *wv,
                       const q8_prepared *prepared, int n, q8_dptr q, size_t q_offset, q8_dptr kcache, q8_dptr vcache,
                       int n_head, int n_kv, int head_dim, int n_rot, float base, int capacity, q8_dptr position) {
    if (!c || !prepared) return fail(Q8_ERR_INVALID, "q8_prompt_qkv_rope: bad arguments");
    if (n_head < 1 || n_kv < 1 || n_head % n_kv || head_dim < 2 || head_dim % 2 || n_rot < 0 || n_rot > head_dim ||
        n_rot % 2 || capacity < 1)
        return fail(Q8_ERR_INVALID, "prompt_qkv_rope: bad geometry (heads %d/%d, head_dim %d, n_rot %d)", n_head, n_kv,
                    head_dim, n_rot);
    Q8_TRY(check_n(n));
    Q8_TRY(check_weight(c, wq));
    Q8_TRY(check_weight(c, wk));
    Q8_TRY(check_weight(c, wv));
    const int k = wq->k;
    const int kv_dim = n_kv * head_dim;
    if (wk->k != k || wv->k != k || wq->out != n_head * head_dim || wk->out != kv_dim || wv->out != kv_dim)
        return fail(Q8_ERR_INVALID, "prompt_qkv_rope: q/k/v weights are %dx%d, %dx%d, %dx%d for %d/%d heads of %d",
                    wq->out, wq->k, wk->out, wk->k, wv->out, wv->k, n_head, n_kv, head_dim);
    if (prepared->n != n || prepared->k != k)
        return fail(Q8_ERR_INVALID, "prepared activations are %d x %d, the matmul wants %d x %d", prepared->n,
                    prepared->k, n, k);
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    float *qp = fptr(q, q_offset);
    Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)qp, (size_t)n * wq->out * 4, "rope q"));
    Q8_TRY(check_span(c, kcache, (size_t)capacity * kv_dim * 2, "key cache"));
    Q8_TRY(check_span(c, vcache, (size_t)capacity * kv_dim * 2, "value cache"));
    Q8_TRY(check_span(c, position, 4, "position"));
    GemvRope rope{};
    Q8_TRY(rope_table(c, n_rot, base, &rope.freq));
    rope.position = reinterpret_cast<const int *>(position);
    rope.kcache = reinterpret_cast<uint16_t *>(kcache);
    rope.vcache = reinterpret_cast<uint16_t *>(vcache);
    rope.head_dim = head_dim;
    rope.n_rot = n_rot;
    rope.capacity = capacity;
    Member m[3] = {{wq, qp}, {wk, nullptr}, {wv, nullptr}};
    return run_gemm(c, m, 3, prepared, n, nullptr, &rope);
}

int q8_rope_append(q8_ctx *c, q8_dptr q, size_t q_offset, q8_dptr k, size_t k_offset, q8_dptr v, size_t v_offset,
                   q8_dptr kcache, q8_dptr vcache, int n, int n_head, int n_kv, int head_dim, int n_rot, float base,
                   int capacity, q8_dptr position) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_rope_append: null context");
    if (n < 1 || n_head < 1 || n_kv < 1 || n_head % n_kv || head_dim < 2 || head_dim % 2 || n_rot < 0 ||
        n_rot > head_dim || n_rot % 2 || capacity < 1)
        return fail(Q8_ERR_INVALID, "rope_append: bad geometry (n %d, heads %d/%d, head_dim %d, n_rot %d)", n, n_head,
                    n_kv, head_dim, n_rot);
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    const size_t kv_dim = (size_t)n_kv * head_dim;
    Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)fptr(q, q_offset), (size_t)n * n_head * head_dim * 4, "rope q"));
    Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)fptr(k, k_offset), (size_t)n * kv_dim * 4, "rope k"));
    Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)fptr(v, v_offset), (size_t)n * kv_dim * 4, "rope v"));
    Q8_TRY(check_span(c, kcache, (size_t)capacity * kv_dim * 2, "key cache"));
    Q8_TRY(check_span(c, vcache, (size_t)capacity * kv_dim * 2, "value cache"));
    Q8_TRY(check_span(c, position, 4, "position"));
    const float *freq = nullptr;
    Q8_TRY(rope_table(c, n_rot, base, &freq));
    Q8RopeArgs a{};
    a.freq = freq;
    a.q = fptr(q, q_offset);
    a.k = fptr(k, k_offset);
    a.v = fptr(v, v_offset);
    a.kcache = reinterpret_cast<uint16_t *>(kcache);
    a.vcache = reinterpret_cast<uint16_t *>(vcache);
    a.position = reinterpret_cast<const int *>(position);
    a.n = n;
    a.n_head = n_head;
    a.n_kv = n_kv;
    a.head_dim = head_dim;
    a.n_rot = n_rot;
    a.capacity = capacity;
    const long long items = (long long)n * (n_head + 2 * n_kv) * (head_dim / 2);
    const unsigned grid = (unsigned)std::min<long long>(ceil_div(items, 256), 4096);
    return launch(c, F_ROPE, grid, 256, 0, &a, sizeof a);
}

namespace {

// The decode attention kernel for `splits` workgroups per head: one split
// takes 16 waves over 1024-row chunks, more take 4 waves over 256-row chunks.
struct AttnShape {
    Fn fn;
    unsigned threads;
    int rows;  // positions per chunk
};
// With splits, the 256-row chunks run on eight waves (four rows a lane) while
// the launch's workgroups fit one per CU, else on four: configs[4] decode,
// attention + O at 600 positions 8.77 -> 8.53 us (3 splits), 2400 positions
// 13.62 -> 12.69 us (5), but 4000 positions 18.02 -> 19.13 us (8 splits:
// 288 workgroups, the heavier ones' second round); option "attn.waves"
// = 4 or 8 forces one.
AttnShape attn_shape(int splits, q8_ctx *c = nullptr, int n_head = 0) {
    if (splits == 1) return {F_ATTN_DECODE, 1024, 1024};
    const int w = c ? option(c, "attn.waves", -1) : 4;
    if (w == 8 || (w < 0 && (long long)n_head * splits <= c->cu_count)) return {F_ATTN_DECODE_W8, 512, 256};
    return {F_ATTN_DECODE_W4, 256, 256};
}

// Decode attention of one token (geometry and spans checked by the caller).
// defer leaves every split's partials in attn_ws for a GEMV prologue.
int run_attn_decode(q8_ctx *c, const float *q, q8_dptr kcache, q8_dptr vcache, float *out, int n_head, int n_kv,
                    int capacity, float scale, q8_dptr position, int splits, int defer) {
    if (splits < 1 || splits > 1024 || splits > capacity)
        return fail(Q8_ERR_INVALID, "attention: %d splits for capacity %d", splits, capacity);
    if (n_head > kCounters - kAttnCounterBase)
        return fail(Q8_ERR_UNSUPPORTED, "attention: %d heads exceed the %d arrival counters", n_head,
                    kCounters - kAttnCounterBase);
    const size_t parts = (size_t)n_head * splits;
    if (splits > 1 || defer)
        Q8_TRY(grow(c, &c->attn_ws, &c->attn_ws_bytes, parts * (Q8_ATTN_HEAD_DIM + 2) * 4, "hipMalloc(attention)"));
    Q8AttnDecodeArgs a{};
    a.q = q;
    a.kcache = reinterpret_cast<const uint16_t *>(kcache);
    a.vcache = reinterpret_cast<const uint16_t *>(vcache);
    a.part_acc = static_cast<float *>(c->attn_ws);
    a.part_ms = a.part_acc ? a.part_acc + parts * Q8_ATTN_HEAD_DIM : nullptr;
    a.out = out;
    a.counters = c->counters + kAttnCounterBase;
    a.position = reinterpret_cast<const int *>(position);
    a.n_head = n_head;
    a.n_kv = n_kv;
    a.splits = splits;
    a.capacity = capacity;
    a.scale = scale;
    a.defer = defer;
    const AttnShape sh = attn_shape(splits, c, n_head);
    if (n_head > 0xffff || n_kv > 0xffff)
        return fail(Q8_ERR_UNSUPPORTED, "attention: %d heads, %d key/value heads", n_head, n_kv);
    // the kernel's preloaded head, then the argument block (scale, out, counters)
    struct {
        const float *q;
        const uint16_t *kcache, *vcache;
        const int *position;
        float *part_acc;
        int dims, splits, cap;
    } h{a.q, a.kcache, a.vcache, a.position, a.part_acc, n_head | (n_kv << 16), splits,
        (int)((unsigned)capacity | ((unsigned)(defer ? 1 : 0) << 31))};
    static_assert(sizeof h == 56, "attention head: five pointers and three ints, padded to 8 bytes");
    Q8_TRY(check_launch(*c->meta[sh.fn], sizeof h + sizeof a, sh.threads, 0, c->max_lds));
    void *params[] = {&h.q, &h.kcache, &h.vcache, &h.position, &h.part_acc, &h.dims, &h.splits, &h.cap, &a};
    HIP_TRY(hipModuleLaunchKernel(c->fn[sh.fn], (unsigned)parts, 1, 1, sh.threads, 1, 1, 0, c->stream, params,
                                  nullptr),
            kFnNames[sh.fn]);
    return Q8_OK;
}

// Prompt attention (n >= 2): f32 rows into `out` and/or prepared Q8_0 into
// `p` (the context's activation workspace, as q8_prepare leaves it).
int run_attn_prefill(q8_ctx *c, const float *q, q8_dptr kcache, q8_dptr vcache, float *out, q8_prepared *p, int n,
                     int n_head, int n_kv, int capacity, float scale, q8_dptr position) {
    Q8AttnPrefillArgs a{};
    a.q = q;
    a.kcache = reinterpret_cast<const uint16_t *>(kcache);
    a.vcache = reinterpret_cast<const uint16_t *>(vcache);
    a.out = out;
    a.position = reinterpret_cast<const int *>(position);
    a.n = n;
    a.n_head = n_head;
    a.n_kv = n_kv;
    a.capacity = capacity;
    a.qtiles = (int)ceil_div(n, 32);
    a.scale = scale;
    if (p) {
        const int k = n_head * Q8_ATTN_HEAD_DIM;
        const int nb = k / 32;
        const int fmt = prepared_format(c, n);
        const size_t qbytes = (size_t)a.qtiles * nb * (fmt == Q8_PREPARED_F16 ? Q8_UNIT_F16_BYTES : Q8_UNIT_BYTES);
        const size_t sbytes = (size_t)a.qtiles * nb * Q8_TILE_TOKENS * sizeof(float);
        Q8_TRY(grow(c, &c->act_ws, &c->act_ws_bytes, align_up(qbytes, kAlign) + sbytes, "hipMalloc(activation)"));
        a.xq = static_cast<uint8_t *>(c->act_ws);
        a.xs = reinterpret_cast<float *>(static_cast<uint8_t *>(c->act_ws) + align_up(qbytes, kAlign));
        a.f16 = fmt == Q8_PREPARED_F16 ? 1 : 0;
        p->quants = (q8_dptr)(uintptr_t)a.xq;
        p->scales = (q8_dptr)(uintptr_t)a.xs;
        p->n = n;
        p->k = k;
        p->format = fmt;
    }
    return launch(c, F_ATTN_PREFILL, (unsigned)(n_head * a.qtiles), 128, 0, &a, sizeof a);
}

int check_attention(q8_ctx *c, q8_dptr qp, q8_dptr kcache, q8_dptr vcache, q8_dptr position, int n, int n_head,
                    int n_kv, int head_dim, int capacity) {
    if (head_dim != Q8_ATTN_HEAD_DIM)
        return fail(Q8_ERR_UNSUPPORTED, "attention kernels are built for head_dim %d, got %d", Q8_ATTN_HEAD_DIM,
                    head_dim);
    if (n < 1 || n_head < 1 || n_kv < 1 || n_head % n_kv || capacity < 1)
        return fail(Q8_ERR_INVALID, "attention: bad geometry (n %d, heads %d/%d, capacity %d)", n, n_head, n_kv,
                    capacity);
    const size_t kv_dim = (size_t)n_kv * head_dim;
    Q8_TRY(check_span(c, qp, (size_t)n * n_head * head_dim * 4, "attention q"));
    Q8_TRY(check_span(c, kcache, (size_t)capacity * kv_dim * 2, "key cache"));
    Q8_TRY(check_span(c, vcache, (size_t)capacity * kv_dim * 2, "value cache"));
    return check_span(c, position, 4, "position");
}

}  // namespace

int q8_attention(q8_ctx *c, q8_dptr q, size_t q_offset, q8_dptr kcache, q8_dptr vcache, q8_dptr out,
                 size_t out_offset, int n, int n_head, int n_kv, int head_dim, int capacity, float scale,
                 q8_dptr position, int splits) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_attention: null context");
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    const q8_dptr qp = (q8_dptr)(uintptr_t)fptr(q, q_offset);
    const q8_dptr op = (q8_dptr)(uintptr_t)fptr(out, out_offset);
    Q8_TRY(check_attention(c, qp, kcache, vcache, position, n, n_head, n_kv, head_dim, capacity));
    Q8_TRY(check_span(c, op, (size_t)n * n_head * head_dim * 4, "attention out"));
    if (n == 1)
        return run_attn_decode(c, reinterpret_cast<const float *>(qp), kcache, vcache, reinterpret_cast<float *>(op),
                               n_head, n_kv, capacity, scale, position, splits, 0);
    return run_attn_prefill(c, reinterpret_cast<const float *>(qp), kcache, vcache, reinterpret_cast<float *>(op),
                            nullptr, n, n_head, n_kv, capacity, scale, position);
}

int q8_attention_prepare(q8_ctx *c, q8_dptr q, size_t q_offset, q8_dptr kcache, q8_dptr vcache, int n, int n_head,
                         int n_kv, int head_dim, int capacity, float scale, q8_dptr position, q8_prepared *out) {
    if (!c || !out) return fail(Q8_ERR_INVALID, "q8_attention_prepare: bad arguments");
    if (n < 2) return fail(Q8_ERR_INVALID, "q8_attention_prepare: %d tokens (the prompt kernel takes n >= 2)", n);
    Q8_TRY(check_n(n));
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    const q8_dptr qp = (q8_dptr)(uintptr_t)fptr(q, q_offset);
    Q8_TRY(check_attention(c, qp, kcache, vcache, position, n, n_head, n_kv, head_dim, capacity));
    return run_attn_prefill(c, reinterpret_cast<const float *>(qp), kcache, vcache, nullptr, out, n, n_head, n_kv,
                            capacity, scale, position);
}

int q8_attention_matmul_add(q8_ctx *c, q8_dptr q, size_t q_offset, q8_dptr kcache, q8_dptr vcache, int n_head,
                            int n_kv, int head_dim, int capacity, float scale, q8_dptr position, int splits,
                            const q8_weight *wo, q8_dptr y, size_t y_offset) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_attention_matmul_add: null context");
    Q8_TRY(check_weight(c, wo));
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    const q8_dptr qp = (q8_dptr)(uintptr_t)fptr(q, q_offset);
    Q8_TRY(check_attention(c, qp, kcache, vcache, position, 1, n_head, n_kv, head_dim, capacity));
    if (wo->k != n_head * head_dim)
        return fail(Q8_ERR_INVALID, "output projection takes k = %d, the heads give %d", wo->k, n_head * head_dim);
    float *yp = fptr(y, y_offset);
    Q8_TRY(check_span(c, (q8_dptr)(uintptr_t)yp, (size_t)wo->out * 4, "attention output projection y"));
    const float *qf = reinterpret_cast<const float *>(qp);
    Member m{wo, yp};
    if (gemv_folds_combine(c, wo, splits)) {
        Q8_TRY(run_attn_decode(c, qf, kcache, vcache, nullptr, n_head, n_kv, capacity, scale, position, splits, 1));
        const size_t parts = (size_t)n_head * splits;
        const float *acc = static_cast<const float *>(c->attn_ws);
        const GemvCombine comb{acc, acc + parts * Q8_ATTN_HEAD_DIM, splits};
        return run_gemv(c, &m, 1, 0, wo->k, yp, 0, nullptr, 0.0f, nullptr, &comb);
    }
    // the two steps, through the attention output workspace
    Q8_TRY(grow(c, &c->attn_out_ws, &c->attn_out_ws_bytes, (size_t)wo->k * 4, "hipMalloc(attention output)"));
    float *att = static_cast<float *>(c->attn_out_ws);
    Q8_TRY(run_attn_decode(c, qf, kcache, vcache, att, n_head, n_kv, capacity, scale, position, splits, 0));
    return run_gemv(c, &m, 1, (q8_dptr)(uintptr_t)att, wo->k, yp, 0);
}

extern "C++" {
namespace q8i {
int attention_split_rows() { return attn_shape(2).rows; }
int group_rows(q8_ctx *c, int k, int silu) {
    int rs = 0, nl = 0, nw = 0;
    if (!c || k < 32 || k % 32 || !option(c, "gemv.group_hot", 1)) return 0;
    return rsg_shape(c, k / 32, silu, true, &rs, &nl, &nw, true) ? rs : 0;
}
int group_slice_rows(q8_ctx *c, int k, int silu) { return option(c, "gemv.slice_copy", 1) ? group_rows(c, k, silu) : 0; }
int group_pair_slices(q8_ctx *c, int k) {
    return (c && k >= 32 && k % 32 == 0 && option(c, "gemv.group_hot", 1) && option(c, "gemv.slice_copy", 1) &&
            pair_loads(k / 32))
               ? kGroupPairSlices
               : 0;
}
}  // namespace q8i
}

int q8_advance_position(q8_ctx *c, q8_dptr position, int by) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_advance_position: null context");
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    Q8_TRY(check_span(c, position, 4, "position"));
    Q8AdvanceArgs a{reinterpret_cast<int *>(position), by};
    return launch(c, F_ADVANCE, 1, 64, 0, &a, sizeof a);
}

int q8_weight_synthetic(q8_ctx *c, int k, int out, uint64_t seed, float scale_std, const q8_weight **weight) {
    return q8i::weight_synthetic(c, k, out, seed, scale_std, true, weight);
}

}  // extern "C"

int q8i::weight_synthetic(q8_ctx *c, int k, int out, uint64_t seed, float scale_std, bool with_slices,
                          const q8_weight **weight) {
    if (!c || !weight) return fail(Q8_ERR_INVALID, "q8_weight_synthetic: bad arguments");
    Q8_TRY(check_k(k));
    if (out <= 0) return fail(Q8_ERR_INVALID, "weight has %d rows", out);
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    const int nb = k / 32;
    const int tiles = (int)ceil_div(out, Q8_TILE_ROWS);
    const size_t nbytes = (size_t)out * nb * Q8_BLOCK_BYTES;
    const WeightAlloc wa = weight_alloc(c, out, k, with_slices);
    const size_t qbytes = wa.qbytes;
    const size_t total = wa.total;
    const long long threads = (long long)tiles * Q8_TILE_ROWS * nb;
    if (threads > 0x7fffffffLL) return fail(Q8_ERR_UNSUPPORTED, "weight of %lld blocks is too large", threads);
    void *base = nullptr, *staging = nullptr;
    HIP_TRY(dev_malloc(c, &base, total), "hipMalloc(weight)");
    hipError_t e = dev_malloc(c, &staging, nbytes);
    if (e != hipSuccess) {
        hipFree(base);
        return hip_fail(e, "hipMalloc(weight staging)");
    }
    Q8SynthArgs sa{static_cast<uint8_t *>(staging), (long long)out * nb, seed, scale_std};
    Q8RepackArgs a{};
    a.src = static_cast<const uint8_t *>(staging);
    a.quants = static_cast<uint8_t *>(base);
    a.scales = reinterpret_cast<uint16_t *>(static_cast<uint8_t *>(base) + align_up(qbytes, kAlign));
    a.rows = out;
    a.nb = nb;
    a.tiles = tiles;
    a.inverse = 0;
    int rc = launch(c, F_SYNTH, (unsigned)std::min<long long>(ceil_div(sa.blocks, 256), 65536), 256, 0, &sa, sizeof sa);
    if (rc == Q8_OK) rc = launch(c, F_REPACK, (unsigned)ceil_div(threads, 256), 256, 0, &a, sizeof a);
    uint8_t *slices = wa.slice_rows ? static_cast<uint8_t *>(base) + wa.slices_off : nullptr;
    if (rc == Q8_OK && slices) rc = slice_copy(c, a.quants, slices, nb, tiles, wa.slice_rows);
    if (rc == Q8_OK) {
        e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) rc = hip_fail(e, "hipStreamSynchronize");
    }
    hipFree(staging);
    if (rc != Q8_OK) {
        hipFree(base);
        return rc;
    }
    q8_weight *w = new q8_weight{c, base, a.quants, a.scales, k, out, nb, tiles, total, 0, 0};
    w->slices = slices;
    w->slice_rows = wa.slice_rows;
    c->owned.push_back(w);
    *weight = w;
    return Q8_OK;
}

// Synthetic matrices of one K as a contiguous group: one allocation holds
// every member's quants (their 32-row tiles back to back), then every
// member's scales, then, with slice_rows 8 or 16, the slice-major copy of all
// the tiles.  Each member is a weight of its own (the same bytes as
// q8_weight_synthetic with its seed) whose pointers lie inside the group's
// allocation; the allocation is freed with the last member released.  A
// decode group or gate/up pair of such members runs the contiguous-group
// row-slice GEMVs.
namespace {

// One contiguous group of `count` matrices of one k: one allocation holding
// every member's quants (tiles back to back), then every member's scales,
// then the slice-major copy of all the tiles (slice_rows 8 or 16) or a
// gate/up pair's paired copy (kPairSlices).  Member i's GGUF bytes come from
// the host (bytes[i]) or are synthesized on the device (seeds[i]).  Resident
// members are cached by host identity, synthetic ones owned by the context.
int build_group(q8_ctx *c, int k, int count, const int *outs, const void *const *bytes, const size_t *nbytes,
                const uint64_t *seeds, float scale_std, int slice_rows, const q8_weight **weights) {
    if (count < 1 || count > Q8_GROUP_MAX) return fail(Q8_ERR_INVALID, "a weight group holds one to four matrices");
    const bool pair = slice_rows == kPairSlices;
    if (pair && (count != 2 || outs[0] != outs[1]))
        return fail(Q8_ERR_INVALID, "weight group: a paired copy belongs to a gate/up pair of one shape");
    if (pair) slice_rows = 16;
    if (slice_rows != 0 && slice_rows != 8 && slice_rows != 16)
        return fail(Q8_ERR_INVALID, "weight group: slice rows %d (0, 8 or 16)", slice_rows);
    Q8_TRY(check_k(k));
    const int nb = k / 32;
    int total_tiles = 0, most_rows = 0;
    for (int i = 0; i < count; i++) {
        if (outs[i] <= 0) return fail(Q8_ERR_INVALID, "weight has %d rows", outs[i]);
        if (bytes) {
            if (!bytes[i]) return fail(Q8_ERR_INVALID, "weight group: member %d has no bytes", i);
            if (nbytes[i] != (size_t)outs[i] * nb * Q8_BLOCK_BYTES)
                return fail(Q8_ERR_INVALID, "weight byte length mismatch: %zu bytes for %d x %d Q8_0", nbytes[i],
                            outs[i], k);
            for (int j2 = 0; j2 < i; j2++)
                if (bytes[j2] == bytes[i] && nbytes[j2] == nbytes[i])
                    return fail(Q8_ERR_INVALID, "weight group: member %d repeats member %d", i, j2);
        }
        total_tiles += (int)ceil_div(outs[i], Q8_TILE_ROWS);
        most_rows = std::max(most_rows, outs[i]);
    }
    const long long threads = (long long)total_tiles * Q8_TILE_ROWS * nb;
    if (threads > 0x7fffffffLL) return fail(Q8_ERR_UNSUPPORTED, "weight group of %lld blocks is too large", threads);
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    if (bytes) {
        for (int i = 0; i < count; i++)
            if (c->weights.count(std::make_pair((uintptr_t)bytes[i], nbytes[i])))
                return fail(Q8_ERR_INVALID, "weight group: member %d is already resident", i);
    }
    HIP_TRY(hipSetDevice(c->device), "hipSetDevice");
    const size_t qbytes = (size_t)total_tiles * nb * Q8_UNIT_BYTES;
    const size_t sbytes = (size_t)total_tiles * nb * Q8_TILE_ROWS * 2;
    const size_t slices_off = align_up(align_up(qbytes, kAlign) + sbytes, kAlign);
    const size_t total = slice_rows ? slices_off + qbytes : align_up(qbytes, kAlign) + sbytes;
    void *base = nullptr, *staging = nullptr;
    HIP_TRY(dev_malloc(c, &base, total), "hipMalloc(weight group)");
    hipError_t e = dev_malloc(c, &staging, (size_t)most_rows * nb * Q8_BLOCK_BYTES);
    if (e != hipSuccess) {
        hipFree(base);
        return hip_fail(e, "hipMalloc(weight staging)");
    }
    uint8_t *quants = static_cast<uint8_t *>(base);
    uint16_t *scales = reinterpret_cast<uint16_t *>(quants + align_up(qbytes, kAlign));
    int rc = Q8_OK;
    int t0 = 0;
    for (int i = 0; i < count && rc == Q8_OK; i++) {
        const int tiles = (int)ceil_div(outs[i], Q8_TILE_ROWS);
        if (bytes) {
            e = hipMemcpyAsync(staging, bytes[i], nbytes[i], hipMemcpyHostToDevice, c->stream);
            if (e != hipSuccess) rc = hip_fail(e, "hipMemcpyAsync(weight)");
        } else {
            Q8SynthArgs sa{static_cast<uint8_t *>(staging), (long long)outs[i] * nb, seeds[i], scale_std};
            rc = launch(c, F_SYNTH, (unsigned)std::min<long long>(ceil_div(sa.blocks, 256), 65536), 256, 0, &sa,
                        sizeof sa);
        }
        Q8RepackArgs a{};
        a.src = static_cast<const uint8_t *>(staging);
        a.quants = quants + (size_t)t0 * nb * Q8_UNIT_BYTES;
        a.scales = scales + (size_t)t0 * nb * Q8_TILE_ROWS;
        a.rows = outs[i];
        a.nb = nb;
        a.tiles = tiles;
        a.inverse = 0;
        const long long th = (long long)tiles * Q8_TILE_ROWS * nb;
        if (rc == Q8_OK) rc = launch(c, F_REPACK, (unsigned)ceil_div(th, 256), 256, 0, &a, sizeof a);
        t0 += tiles;
    }
    uint8_t *slices = slice_rows ? quants + slices_off : nullptr;
    if (rc == Q8_OK && slices)
        rc = slice_copy(c, quants, slices, nb, total_tiles, slice_rows, pair ? total_tiles / 2 : 0);
    if (rc == Q8_OK) {  // the staging buffer is reused member by member and freed below
        e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) rc = hip_fail(e, "hipStreamSynchronize");
    }
    hipFree(staging);
    if (rc != Q8_OK) {
        hipFree(base);
        return rc;
    }
    int *refs = new int(count);
    t0 = 0;
    for (int i = 0; i < count; i++) {
        const int tiles = (int)ceil_div(outs[i], Q8_TILE_ROWS);
        const size_t off = (size_t)t0 * nb;
        q8_weight *w = new q8_weight{c, base, quants + off * Q8_UNIT_BYTES, scales + off * Q8_TILE_ROWS, k, outs[i],
                                     nb, tiles, total, bytes ? (uintptr_t)bytes[i] : 0, bytes ? nbytes[i] : 0};
        // a paired copy serves the pair's launch only (the gate holds it); a
        // member alone reads the unit layout
        w->slices = (slices && !pair) ? slices + off * Q8_UNIT_BYTES : nullptr;
        w->slice_rows = (slices && !pair) ? slice_rows : 0;
        w->pair_slices = (pair && i == 0) ? slices : nullptr;
        w->group_refs = refs;
        if (bytes)
            c->weights[std::make_pair(w->id_ptr, w->id_len)] = w;
        else
            c->owned.push_back(w);
        weights[i] = w;
        t0 += tiles;
    }
    return Q8_OK;
}

}  // namespace

int q8i::weight_synthetic_group(q8_ctx *c, int k, int count, const int *outs, const uint64_t *seeds, float scale_std,
                                int slice_rows, const q8_weight **weights) {
    if (!c || !outs || !seeds || !weights) return fail(Q8_ERR_INVALID, "weight group: bad arguments");
    return build_group(c, k, count, outs, nullptr, nullptr, seeds, scale_std, slice_rows, weights);
}

extern "C" {

int q8_argmax(q8_ctx *c, q8_dptr values, size_t offset, size_t len, uint32_t *argmax) {
    if (!c || !argmax) return fail(Q8_ERR_INVALID, "q8_argmax: bad arguments");
    std::lock_guard<std::recursive_mutex> lock(c->mu);
    return argmax_into(c, (q8_dptr)(uintptr_t)fptr(values, offset), len, argmax);
}

int q8_plan(q8_ctx *c, int n, int out, int k, q8_tactic *t) {
    if (!t) return fail(Q8_ERR_INVALID, "q8_plan: null output");
    Q8_TRY(check_k(k));
    Q8_TRY(check_n(n));
    if (out <= 0) return fail(Q8_ERR_INVALID, "q8_plan: %d rows", out);
    if (c) {
        // with a context: the plan q8_matmul runs, options and the prepared
        // format for n included
        std::lock_guard<std::recursive_mutex> lock(c->mu);
        *t = n == 1 ? plan(c, n, out, k) : plan(c, n, out, k, 1, prepared_format(c, n));
        return Q8_OK;
    }
    return q8_tactics_choose(n, out, k, 256, t);
}

int q8_tactic_count(void) { return q8_tactics_table_size(); }

int q8_tactic_row(int i, q8_tactic *t, int *rank, int *maturity) {
    if (i < 0 || i >= q8_tactics_table_size() || !t) return fail(Q8_ERR_INVALID, "q8_tactic_row: index %d", i);
    const Q8TacticRow &row = q8_tactics_row(i);
    *t = q8_tactic{};
    t->kernel = row.kernel;
    t->name = row.name;
    t->evidence = row.evidence;
    if (rank) *rank = row.rank;
    if (maturity) *maturity = row.maturity;
    return Q8_OK;
}

int q8_event_create(q8_ctx *c, void **ev) {
    if (!c || !ev) return fail(Q8_ERR_INVALID, "q8_event_create: bad arguments");
    hipEvent_t e;
    HIP_TRY(hipEventCreate(&e), "hipEventCreate");
    *ev = (void *)e;
    return Q8_OK;
}

int q8_event_record(q8_ctx *c, void *ev) {
    if (!c || !ev) return fail(Q8_ERR_INVALID, "q8_event_record: bad arguments");
    // during capture the record becomes an event node of the graph (timing
    // inside one graph, with no graph boundary in the timed region)
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    HIP_TRY(hipStreamIsCapturing(c->stream, &st), "hipStreamIsCapturing");
    if (st == hipStreamCaptureStatusActive)
        HIP_TRY(hipEventRecordWithFlags((hipEvent_t)ev, c->stream, hipEventRecordExternal), "hipEventRecordWithFlags");
    else
        HIP_TRY(hipEventRecord((hipEvent_t)ev, c->stream), "hipEventRecord");
    return Q8_OK;
}

int q8_event_elapsed_ms(void *start, void *end, float *ms) {
    if (!start || !end || !ms) return fail(Q8_ERR_INVALID, "q8_event_elapsed_ms: bad arguments");
    HIP_TRY(hipEventSynchronize((hipEvent_t)end), "hipEventSynchronize");
    HIP_TRY(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)end), "hipEventElapsedTime");
    return Q8_OK;
}

int q8_event_destroy(void *ev) {
    if (!ev) return Q8_OK;
    HIP_TRY(hipEventDestroy((hipEvent_t)ev), "hipEventDestroy");
    return Q8_OK;
}

int q8_graph_begin(q8_ctx *c) {
    if (!c) return fail(Q8_ERR_INVALID, "q8_graph_begin: null context");
    HIP_TRY(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    return Q8_OK;
}

int q8_graph_end(q8_ctx *c, void **graph) {
    if (!c || !graph) return fail(Q8_ERR_INVALID, "q8_graph_end: bad arguments");
    hipGraph_t g = nullptr;
    HIP_TRY(hipStreamEndCapture(c->stream, &g), "hipStreamEndCapture");
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) return hip_fail(e, "hipGraphInstantiate");
    *graph = (void *)ge;
    return Q8_OK;
}

int q8_graph_launch(q8_ctx *c, void *graph) {
    if (!c || !graph) return fail(Q8_ERR_INVALID, "q8_graph_launch: bad arguments");
    HIP_TRY(hipGraphLaunch((hipGraphExec_t)graph, c->stream), "hipGraphLaunch");
    return Q8_OK;
}

int q8_graph_destroy(void *graph) {
    if (!graph) return Q8_OK;
    HIP_TRY(hipGraphExecDestroy((hipGraphExec_t)graph), "hipGraphExecDestroy");
    return Q8_OK;
}

}  // extern "C"
