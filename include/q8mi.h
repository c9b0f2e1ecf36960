/*
 * q8mi.h -- C-ABI of the MI355X-native Q8_0 matmul path (libq8mi.so).
 *
 * This is the drop-in boundary for the reference engine's matmul hot path.
 * It replaces the libcuda driver FFI (apps/engine/src/cuda/sys.rs:54-137) and
 * the matmul methods of the CUDA device runtime `Gpu`
 * (apps/engine/src/cuda/mod.rs), which `Compute` (apps/engine/src/compute.rs)
 * calls.  Every entry point below names the reference interface it stands in
 * for; a Rust binding is a line-for-line `extern "C"` block over this header.
 *
 * Conventions (kept from the reference):
 *  - Status codes: 0 is success (sys.rs:49 `SUCCESS`); non-zero is one of
 *    Q8_ERR_*, and q8_last_error() holds the message the reference would have
 *    put in `EngineError::Unsupported("cuda: <op> failed: <msg>")`
 *    (cuda/mod.rs:2107-2115) -- here "hip: <op> failed: <msg>".
 *  - Shape violations the reference `assert!`s (cuda/mod.rs:817-822,
 *    1490-1500, 1562-1569) return Q8_ERR_INVALID instead of aborting, since a
 *    panic cannot cross a C-ABI.  Nothing is launched in that case.
 *  - Offsets (`x_offset`, `y_offset`, `bias_offset`) are in f32 elements, as
 *    `shifted()` takes them (cuda/mod.rs:2092-2094).
 *  - Device pointers are plain 64-bit integers (`DevicePtr`, sys.rs:44-47).
 *  - One context owns one HIP stream; every launch and copy is ordered on it
 *    (cuda/mod.rs:372-404).  Launches are asynchronous; q8_download and
 *    q8_sync wait.  A context may be shared between threads: calls are
 *    serialized by a mutex, as the reference's `Gpu` is `Send + Sync` over one
 *    stream (cuda/mod.rs:1975-1979).
 *  - The activations-and-weights data type is f32 in / f32 out, Q8_0 weights.
 *
 * Numerics (the reference CPU kernels are the oracle, apps/engine/src/quant.rs):
 *  - n == 1: f32 activations, no quantization (tensor.rs:96-101).  Each block
 *    value is the reference's AVX2 order of dot_q8_0 (quant.rs:54-78), bit
 *    for bit.  By default the block values of a row are then summed in a
 *    fixed tree (per lane, the two halves, then the waves): deterministic and
 *    within 2e-6 + 1e-5 |ref| of the reference, not bit-identical to it.
 *    With option "gemv.exact" = 1 the cross-block sum is the reference's
 *    left-to-right sum, so y is bit-identical to its AVX2 path (pinned by the
 *    exact-mode tests in tests/test_gpu_q8.py; about 0.4 us slower at
 *    configs[0]).
 *  - n >= 2: activations are quantized to Q8_0 exactly as quantize_q8_0 does
 *    (round half away from zero, saturating), then int8 x int8 per 32-block
 *    on v_mfma_i32_32x32x32_i8 (exact int32), f32 scale d_w*s_x per block.
 *    This follows the CPU semantics for every n >= 2 (tensor.rs:104-148), not
 *    the reference GPU's f32 path for 2 <= n <= 7 (cuda/mod.rs:883-891).
 */
#ifndef Q8MI_H
#define Q8MI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    Q8_OK = 0,
    Q8_ERR_HIP = 1,           /* a HIP call failed */
    Q8_ERR_INVALID = 2,       /* argument or shape error (the reference asserts) */
    Q8_ERR_UNSUPPORTED = 3,   /* EngineError::Unsupported (e.g. n above the prompt limit) */
    Q8_ERR_NO_DEVICE = 4,     /* no gfx950 device / code object does not load */
    Q8_ERR_OUT_OF_MEMORY = 5, /* device allocation failed */
    Q8_ERR_FORMAT = 6,        /* EngineError::Format: malformed GGUF (include/q8gguf.h) */
    Q8_ERR_MISSING = 7,       /* EngineError::MissingTensor / MissingMetadata */
    Q8_ERR_IO = 8,            /* EngineError::Io: the file cannot be opened or mapped */
};

/* Largest prompt one matmul takes: MMA_TOKENS (cuda/mod.rs:115). */
#define Q8_MAX_TOKENS 1024
/* Matrices one grouped launch carries: MMA_GROUP_MAX (cuda/mod.rs:63). */
#define Q8_GROUP_MAX_MEMBERS 4

typedef uint64_t q8_dptr;
typedef struct q8_ctx q8_ctx;
typedef struct q8_weight q8_weight;

/* Activations already quantized on the device: the reference's `Prepared`
 * (cuda/mod.rs:119), a non-owning view into the context's activation
 * workspace, valid until a later prepare needs a larger workspace.  `format`
 * says how the quants are stored: Q8_PREPARED_I8 as int8 units (1 KB per
 * 32 tokens x 32 elements), Q8_PREPARED_F16 as the same integers in f16 units
 * (2 KB), read by the f16-MFMA GEMM; q8_prepare picks it from n. */
enum { Q8_PREPARED_I8 = 0, Q8_PREPARED_F16 = 1 };
typedef struct {
    q8_dptr quants;
    q8_dptr scales;
    int n;
    int k;
    int format;
} q8_prepared;

/* One member of a grouped launch: `GroupEntry` (cuda/mod.rs:314-320). */
typedef struct {
    const q8_weight *weight;
    q8_dptr y;
    size_t y_offset;
} q8_group_entry;

/* Kernel variants a tactic can name. */
enum { Q8_KERNEL_GEMV = 1, Q8_KERNEL_GEMM = 2, Q8_KERNEL_GEMM_F16 = 3 };

/* The shape-keyed tactic chosen for one (n, out, k): the matmul counterpart
 * of `Tactic`/`Choice` (apps/engine/src/tactics.rs:229-347). */
typedef struct {
    int kernel;          /* Q8_KERNEL_* */
    int waves_per_tile;  /* GEMV: waves splitting one 32-row tile's blocks */
    int pairs_per_wave;  /* GEMV: block pairs per wave */
    int pairs_per_batch; /* GEMV: block pairs whose loads are issued together */
    int exact;           /* GEMV: 1 = left-to-right block sum (bit-exact) */
    int tpw;             /* GEMM: 32-token tiles per wave (1, 2 or 4) */
    int twaves;          /* GEMM: waves along the tokens per workgroup */
    int smode;           /* GEMM: 1 = scale products on the matrix cores */
    int xcd_remap;       /* GEMM: keep a row tile's workgroups on one XCD */
    int kslices;         /* workgroups splitting one output tile's blocks (1 = none) */
    int kwaves;          /* GEMM: waves splitting the blocks inside a workgroup */
    int rwaves;          /* f16 GEMM: row-tile waves per workgroup sharing staged activations */
    int pipe;            /* int8 GEMM: 1 = software-pipelined kernel (MFMAs one item ahead) */
    int row_slice;       /* GEMV over one matrix: rows per workgroup (8, 16; 32 = one 32-row tile) */
    int slice_loads;     /* GEMV row slices: 16-byte weight loads per lane (3 or 6) */
    const char *name;    /* tactic name, e.g. "matmul.gemv_f32" */
    const char *evidence;
} q8_tactic;

/* ---- status and build identity ---- */

/* Human-readable name of a status code (sys.rs:140-151 error_message). */
const char *q8_status_string(int status);
/* Message of the last failed call on this thread (EngineError's text). */
const char *q8_last_error(void);
/* Build identity: arch, source and code-object sha256, hipcc version, kernel
 * symbols (apps/engine/build.rs:53-61, apps/engine/src/manifest.rs:17-61). */
const char *q8_build_info(void);

/* ---- context: Gpu::open / Drop (cuda/mod.rs:363-522, 1981-1993) ---- */

int q8_open(int device, q8_ctx **out);
void q8_close(q8_ctx *ctx);
int q8_device_name(q8_ctx *ctx, char *buf, size_t len);
/* CU count, total and free bytes (cuDeviceGetAttribute / cuMemGetInfo,
 * sys.rs:59-62; Gpu::free_bytes). */
int q8_device_info(q8_ctx *ctx, int *cu_count, size_t *total_bytes, size_t *free_bytes);
/* The context's HIP stream (hipStream_t), for callers that order their own
 * work with this path's. */
void *q8_stream(q8_ctx *ctx);
/* Tuning/testing switches; value -1 restores the tactic table's choice.
 * Names: "gemv.exact", "gemv.waves", "gemv.pairs", "gemv.slices",
 * "gemv.rows" (8, 16 or 32), "gemv.loads" (2 with 8-row slices, 3 or 6), "gemv.xcd_order" (0 or 1),
 * "gemm.smode", "gemm.tpw", "gemm.twaves", "gemm.xcd_remap", "gemm.kwaves",
 * "gemm.slices", "gemm.rwaves", "gemm.pipe", "gemm.lds", "gemm.silu",
 * "gemm.f16" (0: int8 prepared activations and the int8-MFMA GEMM for every
 * n; 1: f16 and the f16-MFMA GEMM for every n >= 2), "gemm.small_gemv" (0:
 * n = 2 on f32 x takes the GEMM), "gemm.stream" (0: a one-token-tile GEMM
 * reads its weights with the default cache policy instead of non-temporally;
 * the results are the same bits either way), "gemv.group_hot" (0: the tile
 * kernels for contiguous groups too), "gemv.group_pair" (0: a contiguous
 * gate/up pair takes the two-slot row-slice kernel instead of its paired
 * slices), "gemv.pair_loads" (3 or 6: the paired slices' loads a lane, so
 * K / 32 / (2 * loads) waves a workgroup; by default 3 up to 96 blocks a row,
 * else 6; a value that would need more than 16 waves is ignored),
 * "gemv.slice_copy" (0, set before residency: no slice-major copies),
 * "attn.waves" (4 or 8: the split decode attention's waves a workgroup; by
 * default 8 while the heads x splits workgroups fit one per CU, else 4). */
int q8_set_option(q8_ctx *ctx, const char *name, int value);

/* ---- device memory: Gpu::alloc / upload / download (cuda/mod.rs:530-567) ---- */

int q8_alloc(q8_ctx *ctx, size_t bytes, q8_dptr *out);
int q8_free(q8_ctx *ctx, q8_dptr ptr);
int q8_upload(q8_ctx *ctx, q8_dptr dst, const void *src, size_t bytes);
int q8_download(q8_ctx *ctx, void *dst, q8_dptr src, size_t bytes);
int q8_sync(q8_ctx *ctx);

/* ---- workspace plan: BufferPlan / scratch_requests (apps/engine/src/workspace.rs:63-106, 171-342) ----
 * The context's per-call workspaces (prepared activations, the fused
 * feed-forward's second activation and f32 products, the norm row, token
 * ids, decode attention partials and output) grow on demand.  A caller that
 * knows the largest shapes it will serve plans them once: every workspace
 * gets a region of one device allocation, each as large as the shape needs
 * (or as it already is, if larger), and no call within the shape allocates
 * again.  A plan the current workspaces already cover changes nothing.  The
 * reference overlaps regions whose phases never meet; here they are
 * disjoint, so any order of calls is safe.  Planning moves workspaces when
 * it allocates, without copying them: graphs captured before must be dropped
 * (the generation in q8_workspace_info changes) and q8_prepared views taken
 * before no longer point at live activations -- plan first, then prepare. */
typedef struct {
    int max_tokens;  /* most tokens of any call, 1..Q8_MAX_TOKENS */
    int max_k;       /* longest activation row: the widest weight k, attention heads x 64, norm width */
    int max_ff;      /* width of the fused gate/up calls (0: none) */
    int attn_heads;  /* query heads of the decode attention calls (0: none) */
    int attn_splits; /* most splits those calls use (0 or 1: unsplit) */
    int rope_n_rot;  /* rotation table built now (RopeTable::new, ops.rs:121-131); 0: none */
    float rope_base;
} q8_workspace_shape;
typedef struct {
    uint64_t bytes;       /* device bytes the workspaces hold */
    uint64_t arena_bytes; /* of which in the planned allocation */
    uint64_t allocations; /* device allocations this context has made since q8_open */
    uint64_t generation;  /* changes whenever a workspace moves */
    int regions;          /* regions of the plan (q8_workspace_region) */
} q8_workspace_info;
int q8_workspace_plan(q8_ctx *ctx, const q8_workspace_shape *shape);
int q8_workspace_query(q8_ctx *ctx, q8_workspace_info *info);
int q8_workspace_region(q8_ctx *ctx, int index, const char **name, uint64_t *offset, uint64_t *bytes);

/* ---- weight residency: Gpu::quantized / reserve (cuda/mod.rs:1758-1790) ----
 * Uploads GGUF Q8_0 bytes (`out` rows of k/32 blocks of 34 bytes) once and
 * repacks them on the device into the tile layout; cached by the host
 * identity (bytes, nbytes) exactly as `Weight::identity()` keys the
 * reference's cache (tensor.rs:40-42).  The handle lives until q8_close or
 * q8_weight_release.  Where the weight's one-token GEMV runs in 8- or 16-row
 * slices, the allocation also holds a slice-major copy of the quants (each
 * slice's bytes in one run, read by that GEMV), so q8_weight_shape's
 * device_bytes is then about twice the GGUF bytes; option gemv.slice_copy = 0
 * (set before the upload) leaves the copy out. */
int q8_weight_resident(q8_ctx *ctx, const void *gguf_bytes, size_t nbytes, int k, int out,
                       const q8_weight **weight);
/* Weights of one k made resident together as a contiguous group (no
 * counterpart in the reference, which uploads each tensor alone and groups
 * them at call time: matmul_decode_group, compute.rs): the members' 32-row
 * tiles lie back to back in one allocation, quants then scales, so an n = 1
 * launch over the members in this order (q8_matmul_decode_group,
 * q8_norm_matmul_decode_group, q8_norm_qkv_rope) loads from one set of bases
 * its kernels take preloaded, in 16-row slices of a slice-major copy of the
 * group.  pair = 1 (two members of one shape: gate, then up) builds the
 * pair's paired copy instead -- slices of 8 gate rows and the same 8 up rows
 * -- read by q8_gate_up_silu / q8_norm_gate_up_silu at n = 1.  Each member is
 * a resident weight of its own, cached by its host identity (bytes[i],
 * nbytes[i]) as q8_weight_resident caches it, usable alone and released one
 * by one; the allocation goes with the last.  Q8_ERR_INVALID if a member is
 * already resident.  Outputs equal those of separately resident weights bit
 * for bit with "gemv.exact" = 1 and within 2e-6 + 1e-5 |ref| otherwise
 * (another fixed summation order); option "gemv.group_hot" = 0 keeps the
 * tile kernels for such groups. */
int q8_weight_group_resident(q8_ctx *ctx, int count, const void *const *bytes, const size_t *nbytes, int k,
                             const int *outs, int pair, const q8_weight **weights);
int q8_weight_release(q8_ctx *ctx, const q8_weight *weight);
/* k, rows, and the bytes of the device allocation holding the weight (for a
 * member of a contiguous group: the group's whole allocation). */
int q8_weight_shape(const q8_weight *weight, int *k, int *out, size_t *device_bytes);
/* Writes the resident weight back as GGUF bytes (inverse repack), so the
 * device layout can be checked byte-exactly against the upload. */
int q8_weight_export(q8_ctx *ctx, const q8_weight *weight, void *gguf_bytes, size_t nbytes);

/* ---- the matmul entry points ---- */

/* y[t*out + o] (+)= sum_i x[t*k + i] * W[o*k + i] for t < n.
 * Gpu::matmul (cuda/mod.rs:803-892) / Compute::matmul, matmul_prepared,
 * matmul_add (compute.rs:399-431, 537-581).  `prepared` may be NULL (the
 * activations are then quantized here for n >= 2); `bias` != 0 adds
 * bias[bias_offset + t*out + o] in the epilogue (the fused residual; it may
 * alias y).  n == 1 takes the GEMV; n == 2 without `prepared` the
 * quantized-x GEMV (x quantized to Q8_0 in the launch, the weights read once
 * for both tokens; option "gemm.small_gemv" = 0 turns it off), else the MFMA
 * GEMM -- both under the n >= 2 arithmetic; n > Q8_MAX_TOKENS
 * is Q8_ERR_UNSUPPORTED as in the reference. */
int q8_matmul(q8_ctx *ctx, const q8_weight *weight, q8_dptr x, size_t x_offset, int n, q8_dptr y,
              size_t y_offset, const q8_prepared *prepared, q8_dptr bias, size_t bias_offset);

/* q8_matmul with x quantized to Q8_0 at every n, n = 1 included: the n >= 2
 * arithmetic of tensor::matmul (tensor.rs:104-148 -- quantize_q8_0,
 * quant.rs:98-121, then Weight::dot_row_quantized / dot_q8_0_q8_0,
 * tensor.rs:56-73, quant.rs:127-154) for one token too, where the reference's
 * n = 1 path (q8_matmul) keeps x in f32.  n >= 2 is q8_matmul.  At n = 1 one
 * launch quantizes x (every workgroup the range it reads, bytes equal to
 * quantize_q8_0's), takes each block's int32 dot exactly and multiplies it by
 * d_w * d_x; the block values of a row are summed in a fixed tree, within the
 * n >= 2 parity bar of the reference.  `bias` as in q8_matmul. */
int q8_matmul_q8(q8_ctx *ctx, const q8_weight *weight, q8_dptr x, size_t x_offset, int n, q8_dptr y,
                 size_t y_offset, q8_dptr bias, size_t bias_offset);

/* The scratch of q8_matmul_noalloc: a static device array of this size on
 * each GPU the library runs on, held until the process ends. */
#define Q8_NOALLOC_SCRATCH_BYTES (8u << 20)

/* q8_matmul (above) without allocating: no counterpart in the reference.  For
 * callers that cannot allocate device memory -- code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc: this entry point calls
 * no hipMalloc, hipFree or allocating library routine.  The caller passes a
 * resident weight and its own x, y and bias; n == 2 takes q8_matmul's
 * quantized-x GEMV (x quantized in LDS, no scratch); larger n quantizes x into the
 * static array of Q8_NOALLOC_SCRATCH_BYTES (int8 units, at most
 * ceil(n/32) * (k/32) * 1152 bytes: n = 1024 at k = 5760 fits, larger shapes are
 * Q8_ERR_UNSUPPORTED), and the GEMM keeps every block of a row tile in one
 * workgroup (no split-K partials).  n == 1 runs the GEMV, which needs no
 * scratch (Q8_ERR_UNSUPPORTED if its K would be split).  Results equal
 * q8_matmul's within the n >= 2 parity bar (bit-identical where q8_matmul
 * does not split K).  Every call on one GPU shares that GPU's array, which
 * keeps the last call's bytes (each call rewrites all it reads).  Within one
 * process the first context that uses a GPU's array holds it until q8_close,
 * and a call that needs the array (n >= 3) from any other context on that GPU
 * is Q8_ERR_UNSUPPORTED before anything is launched (n = 1 and n = 2 need none
 * and run), so two contexts' streams never share it; calls of the holding
 * context are ordered on its stream.  Several processes on one GPU each have
 * their own copy. */
int q8_matmul_noalloc(q8_ctx *ctx, const q8_weight *weight, q8_dptr x, size_t x_offset, int n, q8_dptr y,
                      size_t y_offset, q8_dptr bias, size_t bias_offset);

/* Quantize n rows of k f32 activations once for several matmuls:
 * Gpu::prepare (cuda/mod.rs:1381-1410) / Compute::prepare (compute.rs:376-395). */
int q8_prepare(q8_ctx *ctx, q8_dptr x, size_t x_offset, int n, int k, q8_prepared *out);

/* quantize(silu(gate) * up) for the down projection without writing the f32
 * product: Gpu::silu_mul_quantize (cuda/mod.rs:1449-1476) /
 * Compute::silu_mul_prepare (compute.rs:993-1019).  gate and up are [n][k]. */
int q8_silu_mul_prepare(q8_ctx *ctx, q8_dptr gate, q8_dptr up, int n, int k, q8_prepared *out);

/* RMSNorm rows (ops.rs:5-30; Compute::rmsnorm -> Gpu::rmsnorm_rows,
 * compute.rs:584-614): out[t][i] = (x[t][i] * s_t) * weight[i], s_t =
 * 1 / sqrt(mean_t(x^2) + eps), the squares summed in f64.  `weight` is a host
 * f32[k] made resident on first use and cached by (pointer, length), as
 * Gpu::plain does; k % 32 == 0. */
int q8_rmsnorm(q8_ctx *ctx, q8_dptr x, size_t x_offset, const float *weight, int k, float eps, int rows, q8_dptr out,
               size_t out_offset);
/* Drops the device copy of a host vector that q8_rmsnorm / q8_norm_prepare
 * (or the norm-folded decode calls) made resident, so the host memory may be
 * freed and reused: the cache is keyed by (pointer, length), and a new vector
 * at a reused address would otherwise find the old copy.  The reference keeps
 * its copies for the life of the Gpu over mmap'd host weights that never
 * move; this is the counterpart of q8_weight_release for callers whose host
 * vectors do.  A vector that is not resident is a no-op. */
int q8_vector_release(q8_ctx *ctx, const float *weight, size_t k);
/* Makes a host vector resident now rather than on first use (Gpu::plain's
 * upload, cuda/mod.rs:1414-1445), so a planned token path allocates nothing. */
int q8_vector_resident(q8_ctx *ctx, const float *weight, size_t k);
/* prepare(rmsnorm(x)) in one pass, the f32 norm never written
 * (Gpu::rmsnorm_prepare, cuda/mod.rs:1414-1445; Compute::norm_prepare,
 * compute.rs:959-984, whose below-threshold f32 branch is q8_rmsnorm).
 * The result is a view into the activation workspace like q8_prepare's. */
int q8_norm_prepare(q8_ctx *ctx, q8_dptr x, size_t x_offset, const float *weight, int k, float eps, int rows,
                    q8_prepared *out);
/* act[i] = silu(gate[i]) * up[i] for i < len: Gpu::silu_mul / Compute::silu_mul
 * (compute.rs:931-953, ops.rs:33-35). */
int q8_silu_mul(q8_ctx *ctx, q8_dptr act, q8_dptr gate, q8_dptr up, size_t len);

/* Up to four n == 1 matmuls sharing x, one launch:
 * Gpu::matmul_decode_group (cuda/mod.rs:1482-1543).  `bias` only for a
 * single-member group, as in the reference. */
int q8_matmul_decode_group(q8_ctx *ctx, const q8_group_entry *group, int count, q8_dptr x,
                           size_t x_offset, int k, q8_dptr bias, size_t bias_offset);

/* Up to four n >= 2 matmuls sharing prepared activations, one launch:
 * Gpu::matmul_prompt_group (cuda/mod.rs:1549-1626) /
 * Compute::matmul_prepared_group (compute.rs:437-472). */
int q8_matmul_prompt_group(q8_ctx *ctx, const q8_group_entry *group, int count,
                           const q8_prepared *prepared, int n, int k, q8_dptr bias,
                           size_t bias_offset);

/* The feed-forward gate/up pair with SiLU: act[t*ffn + i] =
 * silu(gate(x)_i) * up(x)_i (model.rs:1170-1215 with compute.rs:937-953).
 * n == 1: one fused launch (both GEMVs and the SiLU product in the epilogue).
 * n >= 2: with `prepared`, the product goes to prepared Q8_0 for the down
 * matmul and is never written in f32 (as Compute::silu_mul_prepare does,
 * compute.rs:993-1019): x is quantized, then one gate/up GEMM whose epilogue
 * quantizes silu(gate) * up (see q8_gate_up_silu_prepared).  Without it, one
 * grouped GEMM into workspace, then the f32 product into `act`. */
int q8_gate_up_silu(q8_ctx *ctx, const q8_weight *gate, const q8_weight *up, q8_dptr x,
                    size_t x_offset, int n, q8_dptr act, size_t act_offset, q8_prepared *prepared);

/* The prompt form of the feed-forward pair on activations already prepared
 * (by q8_norm_prepare or q8_prepare): Compute::matmul_prepared_group over
 * gate and up (compute.rs:437-472) followed by silu_mul_prepare
 * (compute.rs:993-1019), returning silu(gate) * up as prepared Q8_0 for the
 * down matmul.  One launch for int8 prepared input (the GEMM's epilogue
 * quantizes the product; bytes equal quantize_q8_0 of the f32 product); the
 * output lives in a second workspace, so `x` stays valid.  n >= 2. */
int q8_gate_up_silu_prepared(q8_ctx *ctx, const q8_weight *gate, const q8_weight *up, const q8_prepared *x,
                             q8_prepared *out);

/* Announces up to four resident weights that a later GEMM will read: the
 * next launch of the int8 GEMM or the fused gate/up GEMM on this context
 * (any entry point at n >= 2) appends cache riders to its grid, workgroups
 * that only read these weights' device bytes once so that they sit in the
 * Infinity Cache when their own GEMM runs.  That launch consumes the
 * announcement; count = 0 withdraws it, and releasing an announced weight
 * removes it.  Results never change.  No counterpart in the reference: its
 * prefill GEMMs read MALL-cold weights as they come.  Meant for a caller that
 * knows its next projection, such as a layer's prefill (q8_decoder_forward's
 * prompt pass announces each next projection). */
int q8_gemm_prefetch(q8_ctx *ctx, const q8_weight *const *weights, int count);

/* lm_head GEMV on the last normed row plus the greedy argmax on the device:
 * model.rs:806-832 + sampler.rs:167-175.  Writes the logits and returns the
 * first index of the strictly greatest logit in *argmax (waits for it). */
int q8_lm_head_argmax(q8_ctx *ctx, const q8_weight *weight, q8_dptr x, size_t x_offset,
                      q8_dptr logits, size_t logits_offset, uint32_t *argmax);

/* Device-to-device copy (bytes, pointers 16-byte aligned): the reference's
 * copy_f32 kernel (gpu.cu:422-435, cuda/mod.rs:1008-1030); also the plain
 * streaming kernel the HBM counters are calibrated with. */
int q8_copy_device(q8_ctx *ctx, q8_dptr dst, q8_dptr src, size_t bytes);

/* Greedy argmax of len f32 values on the device (sampler.rs:167-175). */
int q8_argmax(q8_ctx *ctx, q8_dptr values, size_t offset, size_t len, uint32_t *argmax);

/* Embedding lookup: the rows of `weight` (k = embedding width, out = vocabulary)
 * named by the host token ids, dequantized (d * q, as dequant_q8_0,
 * quant.rs:184-203) into out[out_offset + t*k ...] for t < n, in one launch
 * over the resident device copy.  Replaces Gpu::embeddings (cuda/mod.rs:
 * 1690-1716, kernel embedding_rows gpu.cu:1754-1766) with the vocabulary check
 * of the caller (model.rs:741-751): an id >= out is Q8_ERR_INVALID and nothing
 * is launched.  The ids are copied to a device buffer of the context and the
 * call waits for that copy (cuda/mod.rs:540-552), so `tokens` may be reused on
 * return. */
int q8_embeddings(q8_ctx *ctx, const q8_weight *weight, const uint32_t *tokens, size_t n, q8_dptr out,
                  size_t out_offset);

/* ---- kernel inspection and launch validation ----
 * The reference inspects each kernel at load -- registers, shared memory,
 * occupancy -- and refuses launch shapes the kernel cannot take
 * (cuda/mod.rs:229-283); debug builds also check a launch's argument count
 * against the kernel (cuda/mod.rs:1835-1848).  Here every kernel's metadata
 * comes from the code object's AMDGPU note at build time, and every launch
 * the library makes passes q8_launch_check's rules before it is enqueued. */
typedef struct {
    uint32_t args_bytes;     /* explicit kernel arguments (one struct by value) */
    uint32_t kernarg_bytes;  /* the whole kernarg segment, hidden arguments included */
    uint32_t vgprs;          /* architected VGPRs per lane */
    uint32_t agprs;          /* accumulation VGPRs per lane */
    uint32_t sgprs;
    uint32_t static_lds;     /* bytes of LDS the kernel declares statically */
    uint32_t max_workgroup;  /* largest workgroup the kernel was compiled for (threads) */
    uint32_t private_bytes;  /* scratch (spills) per lane */
} q8_kernel_info_t;

/* The metadata of kernel `name` of this build; Q8_ERR_INVALID for a name the
 * code object does not hold. */
int q8_kernel_info(const char *name, q8_kernel_info_t *info);
/* Q8_OK when a launch of `name` with an argument block of args_bytes, `block`
 * threads per workgroup and dynamic_lds bytes of dynamic LDS fits the kernel
 * and a device of lds_limit bytes of LDS per workgroup: the block equals the
 * kernel's explicit arguments, the workgroup is a whole number of 64-lane
 * waves within the kernel's bound (else Q8_ERR_INVALID), static + dynamic
 * LDS <= lds_limit (else Q8_ERR_UNSUPPORTED).  Host-only: needs no device. */
int q8_launch_check(const char *name, size_t args_bytes, unsigned block, size_t dynamic_lds, size_t lds_limit);

/* ---- tactics: the shape-keyed plan (tactics.rs:229-347, for gfx950) ---- */

/* The tactic a matmul of n tokens over an out x k weight would run. */
int q8_plan(q8_ctx *ctx, int n, int out, int k, q8_tactic *tactic);
/* Number of rows in the tactic table and row i of it, for the invariant
 * checks the reference keeps (tactics.rs:453-501). */
int q8_tactic_count(void);
int q8_tactic_row(int i, q8_tactic *tactic, int *rank, int *maturity);

/* ---- timing and graphs (cuEvent* / cuGraph*, sys.rs:76-123) ---- */

int q8_event_create(q8_ctx *ctx, void **event);
/* Records on the context's stream; while the stream is being captured the
 * record becomes an event node of the graph (hipEventRecordExternal). */
int q8_event_record(q8_ctx *ctx, void *event);
/* Waits for `end`, then returns the milliseconds between the two. */
int q8_event_elapsed_ms(void *start, void *end, float *ms);
int q8_event_destroy(void *event);
/* Capture the context's stream into a graph (cuStreamBeginCapture /
 * cuStreamEndCapture / cuGraphInstantiate), then replay it. */
int q8_graph_begin(q8_ctx *ctx);
int q8_graph_end(q8_ctx *ctx, void **graph);
int q8_graph_launch(q8_ctx *ctx, void *graph);
int q8_graph_destroy(void *graph);

#ifdef __cplusplus
}
#endif

#endif /* Q8MI_H */
