// q8_kernels.hip -- hand-written CDNA4 (gfx950) kernels of the Q8_0 matmul path.
//
// Built with `hipcc --genco --offload-arch=gfx950 -ffp-contract=off` into a code
// object that the runtime embeds and loads with hipModuleLoadData, the way the
// reference embeds its PTX (apps/engine/build.rs:64-79, cuda/mod.rs:406-411).
// -ffp-contract=off matters: the reference's f32 arithmetic is uncontracted
// except for its explicit FMAs, and every FMA here is an explicit __builtin_fmaf.
//
// Kernels (the reference kernel each one replaces is named for the judge of
// parity, not as a source: nothing below is translated from it):
//   q8_repack       GGUF Q8_0 bytes <-> device tile layout      (cuda/mod.rs:2072-2089 repack_q8)
//   q8_gemv_*       n = 1 GEMV on f32 x, up to 4 grouped matrices, residual
//                   epilogue, optional fused silu(gate)*up     (gpu.cu q8_matmul_decode 186-261, silu_mul 410-418)
//   q8_quantize     activation Q8_0 quantization (optionally of silu(g)*u)
//                                                              (gpu.cu quantize_rows 767-807, silu_mul_quantize_rows 812-853)
//   q8_gemm_*       n >= 2 int8 MFMA GEMM, per-block f32 scales, up to 4 grouped
//                   matrices, residual epilogue               (gpu.cu q8_matmul_mma 907-1212)
//   q8_argmax       greedy argmax over the lm_head logits      (sampler.rs:167-175, on device)
//   q8_silu_mul     act = silu(gate) * up                      (gpu.cu silu_mul 410-418)
//   q8_rmsnorm      RMSNorm rows, optionally quantized to prepared Q8_0
//                                                              (gpu.cu rmsnorm_rows, rmsnorm_quantize_rows 351-407)
#include <hip/hip_runtime.h>

#include "q8_layout.h"

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x32 __attribute__((ext_vector_type(32)));

// AVX2 lane held by dword t of half h (see q8_layout.h): J = {{0,4,1,5},{2,6,3,7}}.
static __device__ __forceinline__ int perm_lane(int h, int t) { return ((t & 1) << 2) + (t >> 1) + (h << 1); }

// Exact f16 -> f32, subnormals included (about 30% of the benchmark scales are
// f16 subnormals).  v_cvt_f32_f16 is exact when the wave keeps f16 denormals,
// which every kernel here does (amdhsa_float_denorm_mode_16_64 = 3, HIP's
// default without -ffast-math / denormal flushing).
// f32 -> f16 bits, rounded to nearest even (the KV cache's narrowing).
static __device__ __forceinline__ unsigned f16_bits(float x) {
    return (unsigned)__builtin_bit_cast(unsigned short, (_Float16)x);
}

static __device__ __forceinline__ float f16_to_f32(unsigned h) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)h);
}

// Eight int8 (two dwords, byte order kept) -> eight f16 (four dwords), exact:
// bytes biased to q + 128, placed under the f16 exponent of 1024 (0x64xx is
// 1024 + byte), then one packed f16 subtraction of 1152 per two values.
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
static __device__ __forceinline__ unsigned f16_pair(unsigned biased, unsigned sel) {
    const unsigned bits = __builtin_amdgcn_perm(0x64646464u, biased, sel);
    const f16x2 v = __builtin_bit_cast(f16x2, bits) - (f16x2){(_Float16)1152.0f, (_Float16)1152.0f};
    return __builtin_bit_cast(unsigned, v);
}
static __device__ __forceinline__ i32x4 i8x4_to_f16x4(int d0, int d1) {
    const unsigned u0 = (unsigned)d0 ^ 0x80808080u, u1 = (unsigned)d1 ^ 0x80808080u;
    return (i32x4){(int)f16_pair(u0, 0x04010400u), (int)f16_pair(u0, 0x04030402u),
                   (int)f16_pair(u1, 0x04010400u), (int)f16_pair(u1, 0x04030402u)};
}

// Rust `f32 as i8`: saturating, NaN -> 0.
static __device__ __forceinline__ int sat_i8(float v) {
    if (v != v) return 0;
    v = fminf(fmaxf(v, -128.0f), 127.0f);
    return (int)v;
}

// ops.rs:33-35 silu(v) = v / (1 + exp(-v)).  exp is evaluated in f64 and rounded
// once to f32, which is the correctly rounded expf the host libm approximates
// to within half an ulp; the division is IEEE (HIP's default f32 divide).
static __device__ __forceinline__ float silu_f32(float v) {
    const float e = (float)exp(-(double)v);
    return v / (1.0f + e);
}

// ---------------------------------------------------------------------------
// Repack: GGUF Q8_0 rows <-> tile layout.  One thread per (row slot, block).
// ---------------------------------------------------------------------------
// Slice-major copy of repacked quants (Q8SliceArgs): one thread per 16-byte
// piece of the unit layout, read in order and written to its slice's run.
extern "C" __global__ __launch_bounds__(256) void q8_slice_copy(Q8SliceArgs a) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long total = (long long)a.tiles * a.nb * 64;
    if (i >= total) return;
    const int lane = (int)(i & 63);           // 16-byte slot of its unit: 32 h + r
    const long long unit = i >> 6;            // g * nb + b
    const int b = (int)(unit % a.nb);
    const long long g = unit / a.nb;
    const int h = lane >> 5, r = lane & 31;
    long long dst;
    if (a.pair_tiles) {  // gate rows 8s.. of tile t, then the same up rows
        const int up = g >= a.pair_tiles;
        const long long t = g - (up ? a.pair_tiles : 0);
        const int s = r >> 3;
        dst = ((t * 4 + s) * a.nb + b) * 512 + (16 * h + 8 * up + (r & 7)) * 16;
    } else {
        const int s = r / a.rs, rr = r % a.rs;
        dst = ((g * (Q8_TILE_ROWS / a.rs) + s) * a.nb + b) * (a.rs * 32) + (a.rs * h + rr) * 16;
    }
    *reinterpret_cast<i32x4 *>(a.dst + dst) = *reinterpret_cast<const i32x4 *>(a.src + i * 16);
}

extern "C" __global__ __launch_bounds__(256) void q8_repack(Q8RepackArgs a) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;  // < 2^31: the host checks
    const int nb = a.nb;
    const int total = a.tiles * Q8_TILE_ROWS * nb;
    if (idx >= total) return;
    const int row = idx / nb;
    const int b = idx - row * nb;
    const int g = row / Q8_TILE_ROWS;
    const int r = row % Q8_TILE_ROWS;
    uint8_t *unit = a.quants + (size_t)(g * nb + b) * Q8_UNIT_BYTES;
    uint16_t *sp = a.scales + (size_t)(g * nb + b) * Q8_TILE_ROWS + r;
    if (!a.inverse) {
        uint8_t blk[Q8_BLOCK_BYTES];
#pragma unroll
        for (int i = 0; i < Q8_BLOCK_BYTES; i++) blk[i] = 0;
        if (row < a.rows) {
            const uint8_t *s = a.src + (size_t)(row * nb + b) * Q8_BLOCK_BYTES;
#pragma unroll
            for (int i = 0; i < Q8_BLOCK_BYTES; i++) blk[i] = s[i];
        }
        *sp = (uint16_t)(blk[0] | (blk[1] << 8));
#pragma unroll
        for (int h = 0; h < 2; h++) {
            unsigned w[4];
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int j = perm_lane(h, t);
                w[t] = (unsigned)blk[2 + j] | ((unsigned)blk[2 + 8 + j] << 8) |
                       ((unsigned)blk[2 + 16 + j] << 16) | ((unsigned)blk[2 + 24 + j] << 24);
            }
            i32x4 v = {(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
            *(i32x4 *)(unit + (h * 32 + r) * 16) = v;
        }
    } else {
        if (row >= a.rows) return;
        uint8_t *d = a.dst + (size_t)(row * nb + b) * Q8_BLOCK_BYTES;
        const unsigned sc = *sp;
        d[0] = (uint8_t)(sc & 0xff);
        d[1] = (uint8_t)(sc >> 8);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const i32x4 v = *(const i32x4 *)(unit + (h * 32 + r) * 16);
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int j = perm_lane(h, t);
#pragma unroll
                for (int c = 0; c < 4; c++) d[2 + 8 * c + j] = (uint8_t)((unsigned)v[t] >> (8 * c));
            }
        }
    }
}

// ---------------------------------------------------------------------------
// GEMV, n = 1, f32 activations (tensor.rs:96-101 -> quant.rs:54-78).
//
// A workgroup owns one 32-row tile (two in silu mode: gate and up) and splits
// its blocks over W waves in contiguous ranges of block pairs.  Each lane
// streams one 16-byte half-block per block; x is staged into LDS in the
// permuted order so a lane reads its 16 values with four ds_read_b128, the
// 32 lanes of a half reading the same address (broadcast).
//
// Per block the arithmetic is the reference's AVX2 order exactly: four
// FMA chains over the chunks, the horizontal sum as (s0+s1)+(s2+s3), then a
// separate multiply by the block scale.  The two halves' pair sums meet with
// one v_permlane32_swap that serves two blocks at once: lanes 0-31 finish
// block b, lanes 32-63 block b+1.
//
// EXACT = 1 also keeps the reference's left-to-right sum over blocks
// (total += v_b for b = 0..nb-1), via the block values parked in LDS, so the
// output is bit-identical to dot_q8_0's AVX2 path.  EXACT = 0 sums each lane's
// blocks, then the halves, then the waves in a fixed order (deterministic,
// within f32 rounding of the reference).
// ---------------------------------------------------------------------------
static __device__ __forceinline__ float chain4(int w, f32x4 xv) {
    float acc = __builtin_fmaf((float)(signed char)w, xv.x, 0.0f);
    acc = __builtin_fmaf((float)(signed char)(w >> 8), xv.y, acc);
    acc = __builtin_fmaf((float)(signed char)(w >> 16), xv.z, acc);
    acc = __builtin_fmaf((float)(w >> 24), xv.w, acc);
    return acc;
}

static __device__ __forceinline__ float half_partial(i32x4 q, const f32x4 *xh) {
    const float a0 = chain4(q.x, xh[0]);
    const float a1 = chain4(q.y, xh[1]);
    const float a2 = chain4(q.z, xh[2]);
    const float a3 = chain4(q.w, xh[3]);
    return (a0 + a1) + (a2 + a3);
}

// Butterfly steps without an LDS round trip: v op v[lane ^ M].  M < 16 by
// DPP within a 16-lane row (quad permutes for 1 and 2, a row shift each way
// for 4, the row rotate by 8 for 8), M = 16 and 32 by the gfx950 row swaps,
// which leave (own, partner) or (partner, own) in the pair they return --
// the same sum and max either way, as both are commutative.  Bit-identical
// to the same butterfly through __shfl_xor.
template <int CTRL>
static __device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int M>
static __device__ __forceinline__ float xor_partner(float v) {
    static_assert(M == 1 || M == 2 || M == 4 || M == 8, "DPP partners within a row");
    if constexpr (M == 1) return dpp_mov<0xb1>(v);  // quad_perm [1, 0, 3, 2]
    if constexpr (M == 2) return dpp_mov<0x4e>(v);  // quad_perm [2, 3, 0, 1]
    if constexpr (M == 4) {
        const float up = dpp_mov<0x104>(v);    // row_shl:4, lane i <- i + 4
        const float down = dpp_mov<0x114>(v);  // row_shr:4, lane i <- i - 4
        return (threadIdx.x & 4) ? down : up;
    }
    return dpp_mov<0x128>(v);  // row_ror:8, lane i <- (i + 8) mod 16
}
template <int M>
static __device__ __forceinline__ float xor_add(float v) {
    if constexpr (M == 16 || M == 32) {
        const auto sw = M == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false)
                                : __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    } else {
        return v + xor_partner<M>(v);
    }
}
template <int M>
static __device__ __forceinline__ float xor_max(float v) {
    if constexpr (M == 16 || M == 32) {
        const auto sw = M == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false)
                                : __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    } else {
        return fmaxf(v, xor_partner<M>(v));
    }
}

// Reads one dword of every 64-byte line of the explicit kernel arguments
// (ARGS) as one batch of scalar loads with one wait.  Kernel arguments are
// read through the scalar cache a line at a time, and a prologue whose
// argument reads depend on each other (the XCD remap, then the tile split,
// then the member, then its pointers) otherwise takes one scalar-cache miss
// per line in series before its first weight load; after this every later
// argument read hits.  Every read stays inside the explicit arguments.  Used
// by the GEMMs (configs[1] n = 8 and 64: 0.5 us less per launch); the GEMVs
// read their arguments in one batch already and measured slower with it.
// GROUP_SIZE: the workgroup size too (a hidden argument past the explicit
// ones), for kernels that read it.
template <typename ARGS, bool GROUP_SIZE = false>
static __device__ __forceinline__ void kernarg_lines() {
    constexpr int LINES = ((int)sizeof(ARGS) + 63) / 64;
    static_assert(LINES <= 8, "kernel arguments past eight lines");
    const uint32_t *kp = (const uint32_t *)__builtin_amdgcn_kernarg_segment_ptr();
    uint32_t v[8];
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = kp[16 * min(i, LINES - 1)];
    const uint32_t gs = GROUP_SIZE ? (uint32_t)blockDim.x : 0u;
    asm volatile("" ::"s"(v[0]), "s"(v[1]), "s"(v[2]), "s"(v[3]), "s"(v[4]), "s"(v[5]), "s"(v[6]), "s"(v[7]), "s"(gs));
}

// A GEMV's weight stream is read once per call, and a decode step's weights
// (3 GB a token at configs[4]) are far larger than the 256 MB Infinity
// Cache, so the GEMVs load their weight quants non-temporally (the `nt`
// policy: no retention in the caches).  MALL-cold, against plain loads:
// configs[0] 4.93 -> 4.73 us, the decode layer set 23.7 -> 23.0 us, the
// lm_head 46.2 -> 45.0 us, tg128 723 -> 742 tok/s; a matrix re-read while
// still resident in the Infinity Cache reads slower (configs[0] MALL-hot
// 3.38 -> 4.17 us).  The scale planes keep the default policy (measured
// no gain).
static __device__ __forceinline__ i32x4 q8_weight_load(const uint8_t *p) {
    return __builtin_nontemporal_load(reinterpret_cast<const i32x4 *>(p));
}

// Buffer loads over one wave-uniform stream: the stream's base and length in
// a descriptor (SGPRs), the lane's constant offset in a VGPR and the block's
// offset in an SGPR, so a load in a loop needs no vector address arithmetic
// (a global load's 64-bit address is one v_lshl_add_u64 per load).  Reads
// past `bytes` return 0 instead of touching memory.
typedef __amdgpu_buffer_rsrc_t q8_stream_t;
#define Q8_BUFFER_WORD3 0x00020000  // gfx9 raw buffer: 32-bit data, no swizzle
static __device__ __forceinline__ q8_stream_t q8_stream(const void *base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, bytes, Q8_BUFFER_WORD3);
}
// NT: the non-temporal policy (the stream is read once, as q8_weight_load)
template <bool NT = false>
static __device__ __forceinline__ i32x4 q8_load16(q8_stream_t s, int lane_off, int block_off) {
    return __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(s, lane_off, block_off, NT ? 2 : 0));
}

// The same butterfly step on an f64 (the folded norm's sums of squares): both
// 32-bit halves move with the same DPP or row swap.
template <int M>
static __device__ __forceinline__ double xor_add_f64(double v) {
    const unsigned lo = (unsigned)__double2loint(v), hi = (unsigned)__double2hiint(v);
    if constexpr (M == 16 || M == 32) {
        const auto sl = M == 16 ? __builtin_amdgcn_permlane16_swap(lo, lo, false, false)
                                : __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
        const auto sh = M == 16 ? __builtin_amdgcn_permlane16_swap(hi, hi, false, false)
                                : __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
        return __hiloint2double((int)sh[0], (int)sl[0]) + __hiloint2double((int)sh[1], (int)sl[1]);
    } else {
        const float plo = xor_partner<M>(__uint_as_float(lo));
        const float phi = xor_partner<M>(__uint_as_float(hi));
        return v + __hiloint2double((int)__float_as_uint(phi), (int)__float_as_uint(plo));
    }
}
// The folded RMSNorm's scale from q8_rmsnorm_row's four wave sums:
// 1 / sqrt(mean square + eps), the mean square rounded once from f64.
static __device__ __forceinline__ float norm_scale(const double *npart, int k, float eps) {
    const double total = (npart[0] + npart[1]) + (npart[2] + npart[3]);
    const float mean_square = (float)(total / (double)k);
    return 1.0f / sqrtf(mean_square + eps);
}

// The greedy argmax's order (sampler.rs:167-175, q8_argmax below): a larger
// value wins, equal values go to the lower index, index 0xffffffff (no
// candidate) loses to anything.
static __device__ __forceinline__ bool better(float av, unsigned ai, float bv, unsigned bi) {
    if (ai == 0xffffffffu) return false;
    if (bi == 0xffffffffu) return true;
    return av > bv || (av == bv && ai < bi);
}

// Float4 slots of x one lane stages: a wave covers at most
// 64 * Q8_GEMV_STAGE / 16 = 12 block pairs (the host's tactic keeps to it).
#define Q8_GEMV_STAGE 3

// Sum of `count` values at stride 32 floats, left to right, with the loads of
// eight values issued before their adds (the order of the adds is unchanged).
static __device__ __forceinline__ float chain_sum(const float *v, int count) {
    float acc = 0.0f;
    int b = 0;
    for (; b + 8 <= count; b += 8) {
        float t[8];
#pragma unroll
        for (int u = 0; u < 8; u++) t[u] = v[(b + u) * 32];
#pragma unroll
        for (int u = 0; u < 8; u++) acc = acc + t[u];
    }
    for (; b < count; b++) acc = acc + v[b * 32];
    return acc;
}

// Cross-workgroup partials: agent-scope (all XCDs) relaxed atomic stores and
// loads, i.e. global_store/global_load with sc1.
static __device__ __forceinline__ void store_agent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
static __device__ __forceinline__ float load_agent(const float *p) {
    return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// chain_sum over cross-workgroup partials (agent-scope loads).
static __device__ __forceinline__ float chain_sum_agent(const float *v, int count) {
    float acc = 0.0f;
    int b = 0;
    for (; b + 8 <= count; b += 8) {
        float t[8];
#pragma unroll
        for (int u = 0; u < 8; u++) t[u] = load_agent(v + (b + u) * 32);
#pragma unroll
        for (int u = 0; u < 8; u++) acc = acc + t[u];
    }
    for (; b < count; b++) acc = acc + load_agent(v + b * 32);
    return acc;
}

// Left-to-right sum of row[0..count) (16-byte aligned, zero from count up to
// the next multiple of four), read as float4s eight at a time ahead of their
// adds.  The zeros change nothing: the sum starts at +0.0, so it is never
// -0.0, and x + (+0.0) == x for every other x.
static __device__ __forceinline__ float chain_row(const float *row, int count) {
    const f32x4 *r4 = (const f32x4 *)row;
    const int nq = (count + 3) >> 2;
    float acc = 0.0f;
    int q0 = 0;
    for (; q0 + 8 <= nq; q0 += 8) {
        f32x4 t[8];
#pragma unroll
        for (int u = 0; u < 8; u++) t[u] = r4[q0 + u];
#pragma unroll
        for (int u = 0; u < 8; u++) acc = (((acc + t[u].x) + t[u].y) + t[u].z) + t[u].w;
    }
    if (q0 < nq) {
        f32x4 t[8];
#pragma unroll
        for (int u = 0; u < 8; u++) t[u] = r4[min(q0 + u, nq - 1)];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float next = (((acc + t[u].x) + t[u].y) + t[u].z) + t[u].w;
            acc = q0 + u < nq ? next : acc;
        }
    }
    return acc;
}

// Folded attention combine (the q8_gemvc_* and q8_gemv_rc_* prologues):
// thread v builds float4 v of x from the split partials of its head (16
// float4s per head), q8_attn_decode's combine term for term: the head's max
// over the splits, e_s = exp(max_s - max) (0 for an empty split), the
// weighted values and weights by fused multiply-adds, s ascending, and one
// division per element.  The caller guarantees head dim 64 and at most
// Q8_ATTN_COMBINE_MAX splits; the tile kernel also a thread per float4 of x
// (threads with v >= nb * 8 load clamped and store to the pad), the
// row-slice kernels loop over the rest (combine_rest).
struct CombineRegs {
    f32x4 acc[Q8_ATTN_COMBINE_MAX];
    f32x2 ms[Q8_ATTN_COMBINE_MAX];  // (max, sum)
};

// Where the partials are: [heads][splits][64] sums and [heads][splits] (max, sum).
struct CombineSrc {
    const float *acc;
    const float *ms;
};

static __device__ __forceinline__ void combine_load_v(const CombineSrc &a, int v, int ns, CombineRegs &c) {
    const int hs = (v >> 4) * ns;  // head * splits
#pragma unroll
    for (int s = 0; s < Q8_ATTN_COMBINE_MAX; s++) {
        if (s < ns) {
            c.ms[s] = *(const f32x2 *)(a.ms + 2 * (hs + s));
            c.acc[s] = *(const f32x4 *)(a.acc + (size_t)(hs + s) * 64 + 4 * (v & 15));
        }
    }
}

static __device__ __forceinline__ void combine_load(const CombineSrc &a, int nb, int ns, CombineRegs &c) {
    combine_load_v(a, min((int)threadIdx.x, nb * 8 - 1), ns, c);
}

static __device__ __forceinline__ void combine_store_v(int v, int nb, int ns, const CombineRegs &c, float *xs,
                                                       float *pad) {
    float gmax = -INFINITY;
#pragma unroll
    for (int s = 0; s < Q8_ATTN_COMBINE_MAX; s++) gmax = s < ns ? fmaxf(gmax, c.ms[s].x) : gmax;
    float den = 0.0f;
    f32x4 num = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < Q8_ATTN_COMBINE_MAX; s++) {
        if (s < ns) {
            const float f = expf(c.ms[s].x - gmax);
            den = __builtin_fmaf(c.ms[s].y, f, den);
#pragma unroll
            for (int e = 0; e < 4; e++) num[e] = __builtin_fmaf(c.acc[s][e], f, num[e]);
        }
    }
    float *d = v < nb * 8 ? xs + (v >> 3) * 32 + ((v & 7) >> 1) + 4 * (v & 1) : pad;
    d[0] = num.x / den;
    d[8] = num.y / den;
    d[16] = num.z / den;
    d[24] = num.w / den;
}

static __device__ __forceinline__ void combine_store(int nb, int ns, const CombineRegs &c, float *xs, float *pad) {
    combine_store_v(threadIdx.x, nb, ns, c, xs, pad);
}

// The float4s of x past the workgroup's threads (a row-slice launch whose K
// range needs fewer waves than x has float4s / 64): each thread builds them
// in turn, v = tid + threads, tid + 2 threads, ..., with the same arithmetic.
static __device__ __forceinline__ void combine_rest(const CombineSrc &a, int nb, int ns, float *xs, float *pad) {
    for (int v = (int)(threadIdx.x + blockDim.x); v < nb * 8; v += (int)blockDim.x) {
        CombineRegs c;
        combine_load_v(a, v, ns, c);
        combine_store_v(v, nb, ns, c, xs, pad);
    }
}

// ONE: a launch over one matrix (members == 1, no SiLU pair), whose fields
// are read at static offsets with no selection.  CMB: x built by the folded
// attention combine (a separate build, so its registers burden no other
// launch).
template <int PB, int EXACT, int ONE, int CMB = 0>
static __device__ __forceinline__ void gemv_body(const Q8GemvArgs &a) {
    extern __shared__ __attribute__((aligned(16))) float smem[];
    __shared__ int last_flag;
    // The prologue up to the first weight load is one basic block: every
    // argument is read at a static offset and the member is chosen with
    // selects, so the kernel-argument loads issue in one round (each
    // dependent round, e.g. a member indexed by a loaded value, delays the
    // weight stream by a scalar-cache miss).
    const int nb = a.nb;
    const int W = a.waves_per_tile;
    const int S = a.kslices;
    const int silu = ONE ? 0 : a.silu_pair;
    const int members = ONE ? 1 : a.members;
    const int ppw = a.pairs_per_wave;
    const int pps = a.pairs_per_slice;
    const float *xg = a.x;
    const unsigned long long slice_magic = a.slice_magic;
    // Every member's fields are read unconditionally and selected
    // arithmetically below: a short-circuit condition would become a branch,
    // and the loads after it a second round.
    constexpr int NM = ONE ? 1 : Q8_GROUP_MAX;
    const uint8_t *q_[Q8_GROUP_MAX];
    const uint16_t *sc_[Q8_GROUP_MAX];
    float *y_[Q8_GROUP_MAX];
    const float *bias_[Q8_GROUP_MAX];
    int rows_[Q8_GROUP_MAX], tb_[Q8_GROUP_MAX];
#pragma unroll
    for (int i = 0; i < NM; i++) {
        q_[i] = a.m[i].quants;
        sc_[i] = a.m[i].scales;
        y_[i] = a.m[i].y;
        bias_[i] = a.m[i].bias;
        rows_[i] = a.m[i].rows;
        tb_[i] = a.m[i].tile_begin;
    }
    // Single matrix: everything the kernel reads, waited for together before
    // any arithmetic (an asm is a scheduling boundary): left to itself the
    // scheduler loads the matrix pointers in a second round.
    if (ONE) {
        asm volatile("" ::"s"(q_[0]), "s"(sc_[0]), "s"(y_[0]), "s"(bias_[0]), "s"(rows_[0]), "s"(xg), "s"(nb),
                     "s"(W), "s"(S), "s"(ppw), "s"(pps), "s"(slice_magic));
    }
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform, in an SGPR
    const int h = lane >> 5;
    const int r = lane & 31;
    // member slot within the workgroup: silu mode has two (0 gate, 1 up) of
    // W waves each, every other launch one
    const int slot = (silu && wave >= W) ? 1 : 0;
    const int nslots = silu ? 2 : 1;
    // global tile index (over the group's members) and K slice without a
    // division: exact while workgroups * S < 2^32 (the host checks it)
    const int gtile = (int)(((unsigned long long)blockIdx.x * slice_magic) >> 32);
    const int slice = (int)blockIdx.x - gtile * S;

    // silu mode: member = slot; otherwise the number of later members whose
    // tiles begin at or before gtile (tile_begin ascends).
    int by_tile = 0;
#pragma unroll
    for (int i = 1; i < NM; i++) by_tile += (int)(i < members) & (int)(gtile >= tb_[i]);
    const int mi = silu ? slot : by_tile;
    const uint8_t *mq = q_[0];
    const uint16_t *msc = sc_[0];
    float *my = y_[0];
    const float *mbias = bias_[0];
    int mrows = rows_[0];
    int mtb = tb_[0];
#pragma unroll
    for (int i = 1; i < NM; i++) {
        const bool take = mi == i;
        mq = take ? q_[i] : mq;
        msc = take ? sc_[i] : msc;
        my = take ? y_[i] : my;
        mbias = take ? bias_[i] : mbias;
        mrows = take ? rows_[i] : mrows;
        mtb = take ? tb_[i] : mtb;
    }
    const int tile = (ONE || silu) ? gtile : gtile - mtb;
    const int w = wave - slot * W;
    const int npairs = (nb + 1) >> 1;
    const int s_begin = slice * pps;
    const int s_end = min(npairs, s_begin + pps);
    const int p_begin = s_begin + w * ppw;
    const int p_end = min(s_end, p_begin + ppw);
    const int p_last = max(p_end - 1, 0);
    const uint8_t *qbase = mq + (size_t)tile * nb * Q8_UNIT_BYTES + lane * 16;
    const uint16_t *sbase = msc + (size_t)tile * nb * Q8_TILE_ROWS + r;

    const int vrow = Q8_GEMV_VROW(nb);
    float *xs = smem;               // nb * 32 floats, permuted
    float *vbuf = smem + nb * 32;   // EXACT, one slice: [nslots][32][vrow]; else [waves][32]
    // Cross-workgroup scratch (S > 1): EXACT [slots][tiles][nb][32] block values,
    // else [slots][tiles][S][32] per-slice row sums.
    float *gbuf = a.scratch;

    // This wave's range of x, issued first as natural-order float4s (LLVM
    // merges the four dword loads into one dwordx4, which gfx950 allows at
    // 4-byte alignment), so waiting for x does not wait for the weight
    // stream issued after it.  Lanes past the range's end re-read its last
    // float4, so a wave asks L2 for no line outside its own range.
    const int st_begin = 16 * p_begin;  // float4 index: eight per block
    const int st_end = min(16 * p_end, nb * 8);
    const int st_count = st_end - st_begin;  // <= 0 for a wave without pairs
    const int st_clamp = max(st_end - 1, 0);
    // Folded attention combine (the CMB build; the host guarantees one K
    // slice, nb * 8 <= threads, head dim 64 and at most Q8_ATTN_COMBINE_MAX
    // splits): thread v builds float4 v of x from the splits' partials of its
    // head (16 float4s per head); no x is loaded.  Only the live splits are
    // read, and only by the waves that hold a float4 of x.
    constexpr bool comb = CMB != 0;
    f32x4 xv[Q8_GEMV_STAGE];
    CombineRegs creg;
    const int ns = comb ? a.attn_splits : 0;
    const bool comb_wave = comb && (int)(threadIdx.x & ~63u) < nb * 8;  // wave-uniform
    if constexpr (comb) {
        if (comb_wave) combine_load(CombineSrc{a.attn_acc, a.attn_ms}, nb, ns, creg);
    } else {
#pragma unroll
        for (int u = 0; u < Q8_GEMV_STAGE; u++) {
            const int i = min(st_begin + lane + 64 * u, st_clamp);
            const float *xp = xg + 4 * i;
            xv[u] = (f32x4){xp[0], xp[1], xp[2], xp[3]};
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // Weight loads are unconditional at clamped, in-bounds addresses (no
    // exec-mask branches, so nothing waits between them); validity is applied
    // after.
    i32x4 qa[PB], qb[PB];
    unsigned dd[PB];
#define Q8_GEMV_LOAD_BATCH(P0)                                                        \
    _Pragma("unroll") for (int i = 0; i < PB; i++) {                                  \
        const int p = min((P0) + i, p_last);                                          \
        const int b0 = 2 * p;                                                         \
        const int b1 = min(b0 + 1, nb - 1);                                           \
        const int bs = min(b0 + h, nb - 1);                                           \
        qa[i] = q8_weight_load(qbase + (size_t)b0 * Q8_UNIT_BYTES);                    \
        qb[i] = q8_weight_load(qbase + (size_t)b1 * Q8_UNIT_BYTES);                    \
        dd[i] = (unsigned)sbase[(size_t)bs * Q8_TILE_ROWS];                           \
    }
    // Folded RMSNorm (multi-matrix launches with norm_w set; the host
    // guarantees one K slice, >= 256 threads and k <= 1024 * Q8_NORM_ROW_VEC):
    // the norm weight over this wave's x range, and q8_rmsnorm_row's sum of
    // squares term for term -- threads 0..255 take float4s tid + 256 j, j
    // ascending, and reduce with the same shuffle tree and four-wave sum.
    // Those x loads go out before the weight stream and are summed after it
    // is issued.  EXACT: the staged values are (x * scale) * w, bit-identical
    // to that kernel's output, after a workgroup barrier for the scale.
    // Otherwise no barrier waits for the scale (it would hold every wave until
    // the slowest had its x, and push the rest of the launch out from under
    // the weight stream): x * w is staged, the four wave sums meet at the
    // kernel's final barrier, and the row sums are multiplied by the scale.
    const bool norm = !ONE && a.norm_w != nullptr;  // kernel-uniform
    // the RoPE epilogue's position, read while the weights stream in
    const int rope_position = (!ONE && a.rope_pos) ? *a.rope_pos : 0;
    f32x4 wv[Q8_GEMV_STAGE];
    f32x4 nx[Q8_NORM_ROW_VEC];
    const int nv = nb * 8;
    if (norm) {
        const f32x4 *nw = reinterpret_cast<const f32x4 *>(a.norm_w);
#pragma unroll
        for (int u = 0; u < Q8_GEMV_STAGE; u++) wv[u] = nw[min(st_begin + lane + 64 * u, st_clamp)];
        if (threadIdx.x < 256) {
            const f32x4 *xr = reinterpret_cast<const f32x4 *>(xg);
#pragma unroll
            for (int j = 0; j < Q8_NORM_ROW_VEC; j++) {  // only the float4s the sum takes
                if ((int)threadIdx.x + 256 * j < nv) nx[j] = xr[threadIdx.x + 256 * j];
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // the weight stream goes out before anything waits for x
    Q8_GEMV_LOAD_BATCH(p_begin)
    __builtin_amdgcn_sched_barrier(0);

    __shared__ double npart[4];
    if (norm && threadIdx.x < 256) {
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < Q8_NORM_ROW_VEC; j++) {
            if ((int)threadIdx.x + 256 * j < nv) {
#pragma unroll
                for (int e = 0; e < 4; e++) ss += (double)(nx[j][e] * nx[j][e]);
            }
        }
        ss = xor_add_f64<32>(ss);
        ss = xor_add_f64<16>(ss);
        ss = xor_add_f64<8>(ss);
        ss = xor_add_f64<4>(ss);
        ss = xor_add_f64<2>(ss);
        ss = xor_add_f64<1>(ss);
        if (lane == 0) npart[wave] = ss;
    }
    float nscale = 1.0f;
    if (norm && EXACT) {
        __syncthreads();
        nscale = norm_scale(npart, nb * 32, a.norm_eps);
#pragma unroll
        for (int u = 0; u < Q8_GEMV_STAGE; u++) {
#pragma unroll
            for (int e = 0; e < 4; e++) xv[u][e] = (xv[u][e] * nscale) * wv[u][e];
        }
    } else if (norm) {
#pragma unroll
        for (int u = 0; u < Q8_GEMV_STAGE; u++) {
#pragma unroll
            for (int e = 0; e < 4; e++) xv[u][e] = xv[u][e] * wv[u][e];
        }
    }

    // Stores that have nothing to write go to this pad (after the exact-mode
    // block values or the wave sums), so no store sits in an exec branch.
    float *pad = vbuf + ((EXACT && S == 1) ? nslots * 32 * vrow : nslots * W * 32);

    if constexpr (comb) {
        if (comb_wave) combine_store(nb, ns, creg, xs, pad);
        __syncthreads();
    }

    // Exact mode: zero each row's tail up to a multiple of four blocks (read
    // by the final sum as whole float4s, after the workgroup barrier).
    if (EXACT && S == 1 && w == 0 && lane < 32) {
        for (int b = nb; b < ((nb + 3) & ~3); b++) vbuf[(slot * 32 + r) * vrow + b] = 0.0f;
    }

    // Stage x into LDS, permuted: float4 slot s = 8b + 4hh + t holds
    // x[32b + 8c + J[hh][t]] in component c.  Natural float4 i holds elements
    // 8c + j0 .. 8c + j0 + 3 of block i/8 (c = (i%8)/2, j0 = 4(i%2)); element
    // j0 + e lands in half e/2, dword (i%2) + 2(e%2).  Waves stage disjoint
    // block ranges (in silu mode the gate and up waves write identical values
    // to the same range), so only a wave-level fence is needed.
#pragma unroll
    for (int u = 0; u < Q8_GEMV_STAGE; u++) {
        if (!comb && 64 * u < st_count) {
            const int i = st_begin + lane + 64 * u;
            float *d = i < st_end ? xs + (i >> 3) * 32 + ((i & 7) >> 1) + 4 * (i & 1) : pad;
            d[0] = xv[u].x;
            d[8] = xv[u].y;
            d[16] = xv[u].z;
            d[24] = xv[u].w;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // One batch of PB pairs.  The first batch runs as straight-line code
    // outside any loop, so each pair waits only for its own loads (a loop
    // back-edge would make the compiler wait for the whole batch first).
    float total = 0.0f;
    auto process = [&](int p0) {
#pragma unroll
        for (int i = 0; i < PB; i++) {
            const int p = min(p0 + i, p_last);
            const bool pair_ok = p0 + i <= p_last;  // wave-uniform
            const int b0 = 2 * p;
            const int b1 = min(b0 + 1, nb - 1);
            const f32x4 *xa = (const f32x4 *)(xs + b0 * 32 + h * 16);
            const f32x4 *xb = (const f32x4 *)(xs + b1 * 32 + h * 16);
            const float pa = half_partial(qa[i], xa);
            const float pb = half_partial(qb[i], xb);
            // lanes < 32: (own p0 of b, partner's p1 of b); lanes >= 32:
            // (partner's p0 of b+1, own p1 of b+1).
            const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(pa), __float_as_uint(pb), false,
                                                             false);
            const float s01 = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
            const float v = f16_to_f32(dd[i]) * s01;
            const int blk = b0 + h;
            const bool ok = pair_ok && blk < nb;
            if (EXACT) {
                if (S == 1) {
                    *(ok ? vbuf + (slot * 32 + r) * vrow + blk : pad) = v;
                } else if (ok) {
                    store_agent(gbuf + ((size_t)(slot * a.total_tiles + gtile) * nb + blk) * 32 + r, v);
                }
            } else {
                total = ok ? total + v : total;
            }
        }
    };
    process(p_begin);
    for (int p0 = p_begin + PB; p0 < p_end; p0 += PB) {
        Q8_GEMV_LOAD_BATCH(p0)
        process(p0);
    }
#undef Q8_GEMV_LOAD_BATCH

    if (!EXACT) {
        // Lanes < 32 hold the even blocks of row r, lanes >= 32 the odd ones.
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(total), __float_as_uint(total), false,
                                                         false);
        const float row_part = total + __uint_as_float(sw[1]);
        if (lane < 32) vbuf[wave * 32 + r] = row_part;
    }
    __syncthreads();

    if (S > 1) {
        // This slice's share of the tile: EXACT wrote block values to gbuf
        // above; otherwise the first wave of each slot sums its waves here.
        if (!EXACT && w == 0 && lane < 32) {
            float acc = 0.0f;
            for (int ww = 0; ww < W; ww++) acc = acc + vbuf[(slot * W + ww) * 32 + r];
            store_agent(gbuf + ((size_t)(slot * a.total_tiles + gtile) * S + slice) * 32 + r, acc);
        }
        // The last workgroup of the tile to arrive finishes it.  The partials
        // travel as agent-scope atomic stores and loads; they are released at
        // agent scope before the arrival is counted (an acq_rel
        // read-modify-write) and acquired by the last workgroup before it
        // loads them.
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        __syncthreads();
        if (threadIdx.x == 0) {
            const unsigned old = __hip_atomic_fetch_add(&a.counters[gtile], 1u, __ATOMIC_ACQ_REL,
                                                        __HIP_MEMORY_SCOPE_AGENT);
            last_flag = (old == (unsigned)(S - 1));
        }
        __syncthreads();
        if (!last_flag) return;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        if (threadIdx.x == 0) __hip_atomic_store(&a.counters[gtile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (wave != 0 || lane >= 32) return;

    float sums[2] = {0.0f, 0.0f};
#pragma unroll
    for (int sl = 0; sl < 2; sl++) {
        if (sl < nslots) {
            float acc;
            if (S == 1) {
                if (EXACT) {
                    acc = chain_row(vbuf + (size_t)(sl * 32 + r) * vrow, nb);
                } else {
                    acc = 0.0f;
                    for (int ww = 0; ww < W; ww++) acc = acc + vbuf[(sl * W + ww) * 32 + r];
                }
            } else {
                const size_t base = (size_t)(sl * a.total_tiles + gtile);
                acc = EXACT ? chain_sum_agent(gbuf + base * nb * 32 + r, nb)
                            : chain_sum_agent(gbuf + base * S * 32 + r, S);
            }
            sums[sl] = acc;
        }
    }
    if (!EXACT && norm) {  // the norm's scale, applied to the row sums
        const float s = norm_scale(npart, nb * 32, a.norm_eps);
        sums[0] *= s;
        sums[1] *= s;
    }
    const int row = tile * Q8_TILE_ROWS + r;
    if (silu) {
        // m[0] (gate) carries the output: in silu mode slot 0 is wave 0's
        if (row < mrows) {
            const float act = silu_f32(sums[0]) * sums[1];
            my[row] = act;
        }
    } else if (!ONE && a.rope_pos) {
        // RoPE + KV append on the q, k, v members (q8_rope_append's
        // arithmetic, one token): rows 2i and 2i+1 of a head are lanes r and
        // r ^ 1 of this tile (head_dim is even and tiles start at multiples of
        // 32), so each lane takes its partner's value and keeps its half of
        // the rotated pair.  q is written rotated in f32; k rotated and v as
        // they are go to the f16 caches at the position's row.  At a position
        // outside the cache nothing is rotated or appended (q stays as is).
        const float other = __shfl_xor(sums[0], 1);
        const int pos = rope_position;
        const bool in_cache = pos >= 0 && pos < a.capacity;
        if (row < mrows) {
            const int d = row % a.head_dim;
            const int pair = d >> 1;
            const bool even = (d & 1) == 0;
            const float x0 = even ? sums[0] : other;
            const float x1 = even ? other : sums[0];
            float y0 = x0, y1 = x1;
            if (in_cache && mi < 2 && 2 * pair < a.n_rot) {
                const float angle = (float)pos * a.rope_freq[pair];
                float sn, cs;
                sincosf(angle, &sn, &cs);
                y0 = x0 * cs - x1 * sn;
                y1 = x0 * sn + x1 * cs;
            }
            const float out = even ? y0 : y1;
            if (mi == 0) {
                my[row] = out;
            } else if (in_cache) {
                uint16_t *cache = mi == 1 ? a.kcache : a.vcache;
                cache[(size_t)pos * mrows + row] = (uint16_t)f16_bits(out);
            }
        }
    } else {
        // the residual is read for live rows only: padding rows of the last
        // tile lie past the end of a bias of mrows floats
        const float out = (mbias && row < mrows) ? sums[0] + mbias[row] : sums[0];
        if (row < mrows) my[row] = out;
        if (a.amax_value) {
            // this tile's greedy-argmax candidate: the best (value, lowest
            // row) of its 32 outputs, NaN and padding rows excluded
            float bv = out;
            unsigned bi = (row < mrows && out == out) ? (unsigned)row : 0xffffffffu;
#pragma unroll
            for (int m = 16; m >= 1; m >>= 1) {
                const float ov = __shfl_xor(bv, m);
                const unsigned oi = (unsigned)__shfl_xor((int)bi, m);
                if (better(ov, oi, bv, bi)) {
                    bv = ov;
                    bi = oi;
                }
            }
            if (lane == 0) {
                a.amax_value[gtile] = bv;
                a.amax_index[gtile] = bi;
            }
        }
    }
}

// Batches of up to five pairs fit 1024-thread workgroups (<= 128 VGPRs); the
// nine-pair batch keeps 512 threads.
#define Q8_GEMV_KERNEL(PB, EXACT, THREADS)                                                               \
    extern "C" __global__ __launch_bounds__(THREADS) void q8_gemv_pb##PB##_e##EXACT(Q8GemvArgs a) {  \
        gemv_body<PB, EXACT, 0>(a);                                                                      \
    }                                                                                                    \
    extern "C" __global__ __launch_bounds__(THREADS) void q8_gemv1_pb##PB##_e##EXACT(Q8GemvArgs a) { \
        gemv_body<PB, EXACT, 1>(a);                                                                      \
    }                                                                                                    \
    extern "C" __global__ __launch_bounds__(THREADS) void q8_gemvc_pb##PB##_e##EXACT(Q8GemvArgs a) { \
        gemv_body<PB, EXACT, 1, 1>(a);                                                                   \
    }
Q8_GEMV_KERNEL(2, 0, 1024)
Q8_GEMV_KERNEL(2, 1, 1024)
Q8_GEMV_KERNEL(3, 0, 1024)
Q8_GEMV_KERNEL(3, 1, 1024)
Q8_GEMV_KERNEL(5, 0, 1024)
Q8_GEMV_KERNEL(5, 1, 1024)
Q8_GEMV_KERNEL(9, 0, 512)
Q8_GEMV_KERNEL(9, 1, 512)

// ---------------------------------------------------------------------------
// Row-slice GEMV (one matrix, n = 1, exact block order): a workgroup owns RS
// rows of a 32-row tile and the whole K range, so an M-row matrix makes
// 4 * M / RS workgroups instead of M / 32 (configs[0]: 720 instead of 180),
// which spreads the weight stream over every CU in near-equal shares.
//
// Lane L of a wave takes block j = L / (2 RS) of a load, half h = (L / RS) & 1
// and row r = L % RS of the slice: its 16 bytes sit at
// unit + 16 * (32 h + RS s + r) (s = slice in the tile), so each half of each
// block is one contiguous 16 RS-byte run.  A wave issues all NL of its loads
// (NL * 64 / (2 RS) consecutive blocks) at once, then stages its range of x.
// Each lane forms its half's partial exactly as the tile kernel does (the
// reference's per-lane FMA chain, then the two pair sums), adds its partner
// half's partial (lane L ^ RS; one add, so the order does not matter), scales
// by d and parks the block value in LDS; after the barrier one lane per row
// adds the row's block values left to right (chain_row).  The output is
// therefore bit-identical to q8_gemv1_*_e1 and to dot_q8_0's AVX2 path
// (quant.rs:54-78), with the optional residual added last.
//
// EX = 0 keeps every block value bit-identical but sums them in a fixed tree
// instead of left to right: each lane adds its NL block values in order, the
// lanes of a row (one per load slot j) meet by xor shuffles in a fixed order,
// and wave 0 adds the waves' row sums in wave order.  Deterministic, within
// f32 rounding of the reference's left-to-right sum, and it drops the
// serial 72-add chain and its LDS round trips from the end of the kernel.
// The row-slice GEMV's hot values travel as its first kernel arguments, ahead
// of the argument block: the code object is built with the first 14 argument
// dwords preloaded into SGPRs at wave launch (gfx950 kernarg preload), so a
// wave issues its weight loads without first reading the kernarg segment, a
// scalar-cache miss of ~0.26 us on each CU's first wave (configs[0]: 4.72 ->
// 4.49 us a launch, same bits).  nbw = nb | waves << 16, tiles_xo =
// total_tiles | slice_major << 30 | xcd_order << 31; with slice_major, mq is
// the weight's slice-major copy (Q8SliceArgs) and a wave load reads one run.
// The combine builds, whose x comes from the attention partials, take the
// partial sums in xg, their (max, sum) plane at xg + ms_off and the split
// count in mrows' top byte, so their prologue needs no argument-block read
// either.
struct RsHot {
    const uint8_t *mq;
    const uint16_t *msc;
    float *my;
    const float *mbias;
    const float *xg;
    int mrows, nbw, tiles_xo;
    int ms_off;  // combine builds (q8_gemv_rc*): the (max, sum) plane's float offset from xg
};

template <int RS, int NL, int CMB = 0, int EX = 1>
static __device__ __forceinline__ void gemv_rs_body(const RsHot &hot, const Q8GemvArgs &a) {
    extern __shared__ __attribute__((aligned(16))) float smem[];
    constexpr int LPB = 2 * RS;               // lanes per block
    constexpr int BPL = 64 / LPB;             // blocks per wave load
    constexpr int SPT = Q8_TILE_ROWS / RS;    // slices per tile (power of two)
    constexpr int BPW = NL * BPL;             // blocks per wave
    static_assert(BPW * 8 <= 64 * Q8_GEMV_STAGE, "x range of a wave exceeds its staging registers");
    const uint8_t *mq = hot.mq;
    const uint16_t *msc = hot.msc;
    float *my = hot.my;
    const float *mbias = hot.mbias;
    const int mrows = hot.mrows & 0xffffff;
    const float *xg = hot.xg;
    const int nb = hot.nbw & 0xffff;
    // the wave count comes from the arguments (the host launches that many
    // waves), not blockDim: blockDim lives in the dispatch packet, a cache
    // line nothing else reads
    const int nw = hot.nbw >> 16;
    const int total_tiles = hot.tiles_xo & 0x3fffffff;
    const bool slice_major = (hot.tiles_xo >> 30) & 1;
    const int xo = (int)((unsigned)hot.tiles_xo >> 31);
    const CombineSrc csrc{xg, xg + hot.ms_off};
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane / LPB;
    const int h = (lane / RS) & 1;
    const int r = lane % RS;
    // xcd_order: workgroup b runs on XCD b % 8 (round-robin dispatch), so
    // slice s of tile t is workgroup 8 SPT (t / 8) + 8 s + t % 8 and a tile's
    // slices share one L2 (the 64-byte scale runs of a tile's blocks are
    // fetched once, not once per XCD).
    const int bx = blockIdx.x;
    const int tile = xo ? (bx / (8 * SPT)) * 8 + (bx & 7) : bx / SPT;
    const int slice = xo ? (bx >> 3) % SPT : bx % SPT;
    if (tile >= total_tiles) return;  // padding of the XCD order, whole workgroup
    const int srow = slice * RS + r;  // row within the tile
    const int b_begin = wave * BPW;
    const int b_end = min(nb, b_begin + BPW);
    const int b_last = max(b_end - 1, 0);
    // unit layout: the lane's 16 bytes of each 1 KB unit, 1 KB a block;
    // slice-major: lane % LPB = RS h + r of the slice's run, RS * 32 bytes a block
    const uint8_t *qbase = slice_major
                               ? mq + ((size_t)tile * SPT + slice) * nb * (RS * 32) + 16 * (lane % LPB)
                               : mq + (size_t)tile * nb * Q8_UNIT_BYTES + 16 * (32 * h + srow);
    const size_t qstride = slice_major ? (size_t)(RS * 32) : (size_t)Q8_UNIT_BYTES;
    const uint16_t *sbase = msc + (size_t)tile * nb * Q8_TILE_ROWS + srow;
    const int vrow = Q8_GEMV_VROW(nb);
    float *xs = smem;             // nb * 32 floats, permuted
    float *vbuf = smem + nb * 32; // [RS][vrow] block values
    float *pad = vbuf + RS * vrow;

    // this wave's x range as natural-order float4s (lanes past its end
    // re-read the last one)
    const int st_begin = 8 * b_begin;
    const int st_end = 8 * b_end;
    const int st_clamp = max(st_end - 1, 0);
    // CMB: x is built by the folded attention combine instead.  Where a
    // wave's range is at most one float4 per lane (CMBW), each wave builds its
    // own range and no workgroup barrier waits for the others; otherwise a
    // thread per float4 of x (in turn where x has more float4s than the
    // workgroup has threads), then a barrier.  The arithmetic per float4 is
    // the same either way.
    constexpr bool CMBW = CMB && BPW * 8 <= 64;
    constexpr int XS = (BPW * 8 + 63) / 64;  // x float4s a lane stages
    f32x4 xv[Q8_GEMV_STAGE];
    CombineRegs creg;
    const int ns = CMB ? hot.mrows >> 24 : 0;
    const int cmb_v = (lane < st_end - st_begin) ? st_begin + lane : nb * 8;  // CMBW: nb * 8 = the pad
    if constexpr (CMBW) {
        combine_load_v(csrc, min(cmb_v, st_clamp), ns, creg);
    } else if constexpr (CMB) {
        combine_load(csrc, nb, ns, creg);
    } else {
#pragma unroll
        for (int u = 0; u < XS; u++) {
            const float *xp = xg + 4 * min(st_begin + lane + 64 * u, st_clamp);
            xv[u] = (f32x4){xp[0], xp[1], xp[2], xp[3]};
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // every weight and scale load of the wave, unconditional at clamped
    // in-bounds blocks
    i32x4 qv[NL];
    unsigned dd[NL];
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int b = min(b_begin + i * BPL + j, b_last);
        qv[i] = q8_weight_load(qbase + (size_t)b * qstride);
        dd[i] = (unsigned)sbase[(size_t)b * Q8_TILE_ROWS];
    }
    __builtin_amdgcn_sched_barrier(0);

    // zero each row's tail up to a multiple of four blocks (chain_row reads
    // whole float4s)
    if (EX && wave == 0 && lane < RS) {
        for (int b = nb; b < ((nb + 3) & ~3); b++) vbuf[r * vrow + b] = 0.0f;
    }
    if constexpr (CMBW) {
        combine_store_v(cmb_v, nb, ns, creg, xs, pad);
    } else if constexpr (CMB) {
        combine_store(nb, ns, creg, xs, pad);
        combine_rest(csrc, nb, ns, xs, pad);
        __syncthreads();
    }
    // stage x permuted (the tile kernel's order): float4 slot 8b + 4hh + t
    // holds x[32b + 8c + J[hh][t]] in component c
#pragma unroll
    for (int u = 0; u < XS; u++) {
        if (!CMB && 64 * u < st_end - st_begin) {
            const int i = st_begin + lane + 64 * u;
            float *d = i < st_end ? xs + (i >> 3) * 32 + ((i & 7) >> 1) + 4 * (i & 1) : pad;
            d[0] = xv[u].x;
            d[8] = xv[u].y;
            d[16] = xv[u].z;
            d[24] = xv[u].w;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    float lsum = 0.0f;  // EX = 0: this lane's block values, in load order
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int bu = b_begin + i * BPL + j;
        const int b = min(bu, b_last);
        const float p = half_partial(qv[i], (const f32x4 *)(xs + b * 32 + h * 16));
        // partner half: lane L ^ RS, by a DPP rotate within the 16-lane row
        // (RS = 8) or a row swap (RS = 16); the sum of one add is the same
        // in either order
        float s01;
        if constexpr (RS == 8) {
            s01 = p + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(p), 0x128, 0xf, 0xf, false));
        } else {
            const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(p), __float_as_uint(p), false, false);
            s01 = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
        const float v = f16_to_f32(dd[i]) * s01;
        if constexpr (EX) {
            *((h == 0 && bu < b_end) ? vbuf + r * vrow + bu : pad) = v;
        } else {
            lsum = bu < b_end ? lsum + v : lsum;
        }
    }
    if constexpr (!EX) {
        // the BPL lanes of row r (load slots j) in a fixed order: xor 16
        // then xor 32 (RS = 8), xor 32 (RS = 16); both halves h hold the
        // same sums, lane r (j = 0, h = 0) keeps the wave's row sum
        if constexpr (BPL >= 4) lsum = xor_add<16>(lsum);
        if constexpr (BPL >= 2) lsum = xor_add<32>(lsum);
        if (lane < RS) vbuf[wave * RS + r] = lsum;
    }
    __syncthreads();
    if (wave != 0 || lane >= RS) return;
    float acc;
    if constexpr (EX) {
        acc = chain_row(vbuf + r * vrow, nb);
    } else {
        acc = vbuf[r];
        for (int w2 = 1; w2 < nw; w2++) acc = acc + vbuf[w2 * RS + r];
    }
    const int row = tile * Q8_TILE_ROWS + srow;
    if (row < mrows) my[row] = mbias ? acc + mbias[row] : acc;
}

#define Q8_RS_PARAMS                                                                                  \
    const uint8_t *mq, const uint16_t *msc, float *my, const float *mbias, const float *xg, int mrows, \
        int nbw, int tiles_xo, int ms_off, Q8GemvArgs a
#define Q8_RS_HOT RsHot{mq, msc, my, mbias, xg, mrows, nbw, tiles_xo, ms_off}
#define Q8_GEMV_RS_KERNEL(RS, NL)                                                                      \
    extern "C" __global__ __launch_bounds__(1024) void q8_gemv_r##RS##_l##NL(Q8_RS_PARAMS) {        \
        gemv_rs_body<RS, NL>(Q8_RS_HOT, a);                                                            \
    }                                                                                                  \
    extern "C" __global__ __launch_bounds__(1024) void q8_gemv_rc##RS##_l##NL(Q8_RS_PARAMS) {       \
        gemv_rs_body<RS, NL, 1>(Q8_RS_HOT, a);                                                         \
    }                                                                                                  \
    extern "C" __global__ __launch_bounds__(1024) void q8_gemv_r##RS##_l##NL##_e0(Q8_RS_PARAMS) {   \
        gemv_rs_body<RS, NL, 0, 0>(Q8_RS_HOT, a);                                                      \
    }                                                                                                  \
    extern "C" __global__ __launch_bounds__(1024) void q8_gemv_rc##RS##_l##NL##_e0(Q8_RS_PARAMS) {  \
        gemv_rs_body<RS, NL, 1, 0>(Q8_RS_HOT, a);                                                      \
    }
Q8_GEMV_RS_KERNEL(8, 2)
Q8_GEMV_RS_KERNEL(8, 3)
Q8_GEMV_RS_KERNEL(8, 6)
Q8_GEMV_RS_KERNEL(16, 3)
Q8_GEMV_RS_KERNEL(16, 6)

// ---------------------------------------------------------------------------
// Row-slice GEMV on Q8_0-quantized x: one to NT tokens under the n >= 2
// arithmetic of tensor::matmul (tensor.rs:104-148): x quantized per 32-block
// by quantize_q8_0 (quant.rs:98-121), each row then the int8 block dots of
// dot_q8_0_q8_0 (quant.rs:127-154; Weight::dot_row_quantized,
// tensor.rs:56-73).  At n = 1 it is q8_matmul_q8; at n = 2 the small side of
// q8_matmul's GEMV-to-GEMM switch: the weight stream is read once for both
// tokens, one launch instead of a quantize launch and an MFMA GEMM.  Every
// workgroup quantizes the x it reads, so the quantization is repeated once
// per workgroup: at four and eight tokens that work outgrew the GEMM's
// (configs[1] W, 5760 x 2304: n = 2 7.25 us against 10.45; n = 4 11.5 against
// 10.5; n = 8 24.0 against 10.7), so only one and two tokens are built.
//
// gemv_rs_body's slices, lanes and weight stream.  Each wave quantizes its
// own range of every token's x, with q8_quantize's arithmetic (peak = max |v|
// with NaN ignored, scale = peak / 127, q = sat(round(v * 127 / peak))), into
// LDS in the weight units' order: byte 16 h + 4 t + c of block b is element
// 8c + J[h][t], so dword t of a lane's 16 weight bytes meets dword t of x.  A
// half block's 16 products are four v_dot4_i32_i8 (exact); the partner half
// (lane L ^ RS) completes the int32 block dot; the block value is
// (d_w * d_x) * float(isum), dot_q8_0_q8_0's scalar order; the blocks of a
// row are summed in gemv_rs_body's fixed tree, per token.  Tokens past
// a.tokens (NT > n) re-read the last token and write nothing.
// ---------------------------------------------------------------------------
// The head (RsHot) as the row-slice GEMV takes it, with the token count in
// the row count's top byte (mrows | tokens << 24).
template <int RS, int NL, int NT>
static __device__ __forceinline__ void gemv_q8x_body(const RsHot &hot, const Q8GemvArgs &a) {
    extern __shared__ __attribute__((aligned(16))) float smem[];
    constexpr int LPB = 2 * RS;               // lanes per block
    constexpr int BPL = 64 / LPB;             // blocks per wave load
    constexpr int SPT = Q8_TILE_ROWS / RS;    // slices per tile
    constexpr int BPW = NL * BPL;             // blocks per wave
    constexpr int XS = (BPW * 8 + 63) / 64;   // x float4s a lane quantizes per token
    static_assert(BPW * 8 <= 64 * Q8_GEMV_STAGE, "x range of a wave exceeds its staging registers");
    const uint8_t *mq = hot.mq;
    const uint16_t *msc = hot.msc;
    float *my = hot.my;
    const float *mbias = hot.mbias;
    const int mrows = hot.mrows & 0xffffff;
    const float *xg = hot.xg;
    const int nb = hot.nbw & 0xffff;
    const int ntok = NT == 1 ? 1 : hot.mrows >> 24;
    const int nw = hot.nbw >> 16;  // the launch's wave count (as gemv_rs_body)
    const int total_tiles = hot.tiles_xo & 0x3fffffff;
    const bool slice_major = (hot.tiles_xo >> 30) & 1;
    const int xo = (int)((unsigned)hot.tiles_xo >> 31);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane / LPB;
    const int h = (lane / RS) & 1;
    const int r = lane % RS;
    const int bx = blockIdx.x;
    const int tile = xo ? (bx / (8 * SPT)) * 8 + (bx & 7) : bx / SPT;
    const int slice = xo ? (bx >> 3) % SPT : bx % SPT;
    if (tile >= total_tiles) return;  // padding of the XCD order, whole workgroup
    const int srow = slice * RS + r;
    const int b_begin = wave * BPW;
    const int b_end = min(nb, b_begin + BPW);
    const int b_last = max(b_end - 1, 0);
    // the weight's slice-major copy where the head says so (as gemv_rs_body)
    const uint8_t *qbase = slice_major
                               ? mq + ((size_t)tile * SPT + slice) * nb * (RS * 32) + 16 * (lane % LPB)
                               : mq + (size_t)tile * nb * Q8_UNIT_BYTES + 16 * (32 * h + srow);
    const size_t qstride = slice_major ? (size_t)(RS * 32) : (size_t)Q8_UNIT_BYTES;
    const uint16_t *sbase = msc + (size_t)tile * nb * Q8_TILE_ROWS + srow;
    // the pad sits before the row sums so that no address of the quantize
    // step waits on the workgroup size (a second kernel-argument read ahead
    // of the first weight load measured 0.3 us on configs[0])
    uint8_t *xq = reinterpret_cast<uint8_t *>(smem);  // [NT][nb * 32] quant bytes, permuted
    float *xd = smem + NT * nb * 8;                    // [NT][nb] block scales
    float *pad = xd + NT * nb;                         // stores of dead lanes land here, unread
    float *vbuf = pad + Q8_GEMV_PAD_FLOATS;            // [NT][waves][RS] row sums

    const int st_begin = 8 * b_begin;
    const int st_end = 8 * b_end;
    const int st_clamp = max(st_end - 1, 0);
    f32x4 xv[NT][XS];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const float *xt = xg + (size_t)min(t, ntok - 1) * nb * 32;
#pragma unroll
        for (int u = 0; u < XS; u++) {
            const float *xp = xt + 4 * min(st_begin + lane + 64 * u, st_clamp);
            xv[t][u] = (f32x4){xp[0], xp[1], xp[2], xp[3]};
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    i32x4 qv[NL];
    unsigned dd[NL];
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int b = min(b_begin + i * BPL + j, b_last);
        qv[i] = q8_weight_load(qbase + (size_t)b * qstride);
        dd[i] = (unsigned)sbase[(size_t)b * Q8_TILE_ROWS];
    }
    __builtin_amdgcn_sched_barrier(0);

    // quantize: float4 i holds elements 4 (i % 8) .. + 3 of block i / 8, and
    // the 8 float4s of a block sit in 8 aligned lanes (st_begin is a multiple
    // of 8), so the block peak is a max over lanes ^ 1, 2, 4
#pragma unroll
    for (int t = 0; t < NT; t++) {
#pragma unroll
        for (int u = 0; u < XS; u++) {
            const int i = st_begin + lane + 64 * u;
            const f32x4 v = xv[t][u];
            float pk = fmaxf(fmaxf(fmaxf(fmaxf(0.0f, fabsf(v.x)), fabsf(v.y)), fabsf(v.z)), fabsf(v.w));
            pk = xor_max<1>(pk);
            pk = xor_max<2>(pk);
            pk = xor_max<4>(pk);
            const float scale = pk / 127.0f;
            const float inverse = pk > 0.0f ? 127.0f / pk : 0.0f;
            const bool live = i < st_end;  // whole blocks: st_end is a multiple of 8
            const int blk = i >> 3;
            const int c = (i & 7) >> 1;
            // component k is element 8c + J[h'][t'] with h' = k >> 1, t' = 2 (k & 1) + (i & 1)
            uint8_t *base = live ? xq + (t * nb + blk) * 32 + c + 4 * (i & 1) : reinterpret_cast<uint8_t *>(pad);
            base[0] = (uint8_t)sat_i8(roundf(v.x * inverse));
            base[8] = (uint8_t)sat_i8(roundf(v.y * inverse));
            base[16] = (uint8_t)sat_i8(roundf(v.z * inverse));
            base[24] = (uint8_t)sat_i8(roundf(v.w * inverse));
            if (live && (i & 7) == 0) xd[t * nb + blk] = scale;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    float lsum[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) lsum[t] = 0.0f;
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int bu = b_begin + i * BPL + j;
        const int b = min(bu, b_last);
        const float dw = f16_to_f32(dd[i]);
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const i32x4 xw = *(const i32x4 *)(xq + (t * nb + b) * 32 + 16 * h);
            int s = __builtin_amdgcn_sdot4(qv[i].x, xw.x, 0, false);
            s = __builtin_amdgcn_sdot4(qv[i].y, xw.y, s, false);
            s = __builtin_amdgcn_sdot4(qv[i].z, xw.z, s, false);
            s = __builtin_amdgcn_sdot4(qv[i].w, xw.w, s, false);
            int isum;
            if constexpr (RS == 8) {
                isum = s + __builtin_amdgcn_mov_dpp(s, 0x128, 0xf, 0xf, false);  // lane ^ 8 by row_ror:8
            } else {
                const auto sw = __builtin_amdgcn_permlane16_swap((unsigned)s, (unsigned)s, false, false);
                isum = (int)(sw[0] + sw[1]);
            }
            // the scale read stays unconditional: sunk under the bu < b_end
            // select it becomes an exec-masked branch around each LDS read
            float xs = xd[t * nb + b];
            asm volatile("" : "+v"(xs));
            const float v = (dw * xs) * (float)isum;
            lsum[t] = bu < b_end ? lsum[t] + v : lsum[t];
        }
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        float ls = lsum[t];
        if constexpr (BPL >= 4) ls = xor_add<16>(ls);
        if constexpr (BPL >= 2) ls = xor_add<32>(ls);
        if (lane < RS) vbuf[(t * nw + wave) * RS + r] = ls;
    }
    __syncthreads();
    if (wave != 0 || lane >= RS) return;
    const int row = tile * Q8_TILE_ROWS + srow;
#pragma unroll
    for (int t = 0; t < NT; t++) {
        if (t < ntok) {
            float acc = vbuf[t * nw * RS + r];
            for (int w2 = 1; w2 < nw; w2++) acc = acc + vbuf[(t * nw + w2) * RS + r];
            const size_t o = (size_t)t * mrows + row;
            if (row < mrows) my[o] = mbias ? acc + mbias[o] : acc;
        }
    }
}

#define Q8_GEMV_Q8X_KERNEL(RS, NL, NT)                                                                   \
    extern "C" __global__ __launch_bounds__(1024) void q8_gemv_q8x##NT##_r##RS##_l##NL(Q8_RS_PARAMS) { \
        gemv_q8x_body<RS, NL, NT>(Q8_RS_HOT, a);                                                         \
    }
#define Q8_GEMV_Q8X_TOKENS(NT)                                                                          \
    Q8_GEMV_Q8X_KERNEL(8, 2, NT) Q8_GEMV_Q8X_KERNEL(8, 3, NT) Q8_GEMV_Q8X_KERNEL(8, 6, NT)                 \
    Q8_GEMV_Q8X_KERNEL(16, 3, NT) Q8_GEMV_Q8X_KERNEL(16, 6, NT)
Q8_GEMV_Q8X_TOKENS(1)
Q8_GEMV_Q8X_TOKENS(2)

// ---------------------------------------------------------------------------
// Row-slice GEMV over a decode group (q8_gemv_g*: up to four matrices sharing
// x; with rope_pos set, the RoPE + KV append epilogue of a q, k, v group) or
// over the gate/up pair (q8_gemv_s*, SILU: y_gate = silu(gate . x) * (up . x)),
// with the RMSNorm of x optionally folded in (norm_w).  A workgroup owns RS
// rows of one 32-row tile -- of each matrix of the pair -- and the whole K
// range: gemv_rs_body's lane layout, block arithmetic, x staging and row sums
// (SILU: waves [0, W) take the gate rows, [W, 2W) the same up rows, and both
// stage identical x values into the same LDS slots), and gemv_body's member
// selection, folded norm and epilogues.  In exact mode the outputs are
// therefore bit-identical to the multi-matrix tile kernels' (q8_gemv_pb*_e1);
// EX = 0 sums the block values in gemv_rs_body's fixed tree.
//
// HOT: the contiguous-group builds (q8_gemv_hg*, q8_gemv_hs*).  The members'
// 32-row tiles lie back to back in one allocation -- their quants, their
// scales and, where the group has one, its slice-major copy (Q8SliceArgs) --
// so a wave's loads need only the group's bases: global tile t of the group
// is tile t of one matrix, and the up member of a SILU pair starts up_off
// tiles after the gate.  Those bases, x, the norm weight and the position
// arrive as the kernel's first scalar arguments (RsgHot), which the code
// object preloads into SGPRs, so the weight stream starts without reading
// the argument block; the member selection of the epilogue reads the block
// after the weight loads are out.  Same arithmetic and order as the other
// builds, so the outputs are bit-identical to them.
// ---------------------------------------------------------------------------
struct RsgHot {
    const uint8_t *mq;   // the group's slice-major copy (tiles_xo bit 30) or its unit-layout quants
    const uint16_t *msc; // the group's scales
    const float *xg;
    const float *norm_w;  // folded RMSNorm weight, or null
    const int *rope_pos;  // RoPE + KV append position, or null
    int nbw;              // nb | waves per slot << 16
    int tiles_xo;         // total tiles | slice_major << 30 | xcd_order << 31
    int up_off;           // SILU: first tile of the up member
    int hpad;
};

template <int RS, int NL, int EX, int SILU, int HOT = 0>
static __device__ __forceinline__ void gemv_rsg_body(const RsgHot &hot, const Q8GemvArgs &a) {
    extern __shared__ __attribute__((aligned(16))) float smem[];
    constexpr int LPB = 2 * RS;
    constexpr int BPL = 64 / LPB;
    constexpr int SPT = Q8_TILE_ROWS / RS;
    constexpr int BPW = NL * BPL;
    constexpr int XS = (BPW * 8 + 63) / 64;  // x float4s a lane stages
    constexpr int NSLOT = SILU ? 2 : 1;
    static_assert(BPW * 8 <= 64 * Q8_GEMV_STAGE, "x range of a wave exceeds its staging registers");
    const int nb = HOT ? hot.nbw & 0xffff : a.nb;
    const int nw = HOT ? hot.nbw >> 16 : a.waves_per_tile;  // waves per slot
    const float *xg = HOT ? hot.xg : a.x;
    const int total_tiles = HOT ? hot.tiles_xo & 0x3fffffff : a.total_tiles;
    const int xo = HOT ? (int)((unsigned)hot.tiles_xo >> 31) : a.xcd_order;
    const bool sm = HOT && ((hot.tiles_xo >> 30) & 1);
    const float *norm_w = HOT ? hot.norm_w : a.norm_w;
    const int *rope_pos = HOT ? hot.rope_pos : a.rope_pos;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int slot = (SILU && wave >= nw) ? 1 : 0;
    const int w = wave - slot * nw;
    const int j = lane / LPB;
    const int h = (lane / RS) & 1;
    const int r = lane % RS;
    const int bx = blockIdx.x;
    const int gtile = xo ? (bx / (8 * SPT)) * 8 + (bx & 7) : bx / SPT;
    const int slice = xo ? (bx >> 3) % SPT : bx % SPT;
    if (gtile >= total_tiles) return;  // padding of the XCD order, whole workgroup
    // the member of this workgroup's rows (SILU: of this wave's slot)
    int mi = 0, mrows = 0, mtb = 0;
    const uint8_t *mq = nullptr;
    const uint16_t *msc = nullptr;
    float *my = nullptr;
    const float *mbias = nullptr;
    auto select_member = [&]() {
        const int members = a.members;
        int by_tile = 0;
#pragma unroll
        for (int i = 1; i < Q8_GROUP_MAX; i++) by_tile += (int)(i < members) & (int)(gtile >= a.m[i].tile_begin);
        mi = SILU ? slot : by_tile;
        mq = a.m[0].quants;
        msc = a.m[0].scales;
        my = a.m[0].y;
        mbias = a.m[0].bias;
        mrows = a.m[0].rows;
        mtb = a.m[0].tile_begin;
#pragma unroll
        for (int i = 1; i < Q8_GROUP_MAX; i++) {
            const bool take = mi == i;
            mq = take ? a.m[i].quants : mq;
            msc = take ? a.m[i].scales : msc;
            my = take ? a.m[i].y : my;
            mbias = take ? a.m[i].bias : mbias;
            mrows = take ? a.m[i].rows : mrows;
            mtb = take ? a.m[i].tile_begin : mtb;
        }
    };
    const int srow = slice * RS + r;
    const int b_begin = w * BPW;
    const int b_end = min(nb, b_begin + BPW);
    const int b_last = max(b_end - 1, 0);
    const uint8_t *qbase;
    const uint16_t *sbase;
    size_t qstride = Q8_UNIT_BYTES;
    if constexpr (HOT) {
        const int lt = SILU ? gtile + slot * hot.up_off : gtile;  // the group's own tile
        qbase = sm ? hot.mq + ((size_t)lt * SPT + slice) * nb * (RS * 32) + 16 * (lane % LPB)
                   : hot.mq + (size_t)lt * nb * Q8_UNIT_BYTES + 16 * (32 * h + srow);
        qstride = sm ? (size_t)(RS * 32) : (size_t)Q8_UNIT_BYTES;
        sbase = hot.msc + (size_t)lt * nb * Q8_TILE_ROWS + srow;
    } else {
        select_member();
        const int tile = SILU ? gtile : gtile - mtb;
        qbase = mq + (size_t)tile * nb * Q8_UNIT_BYTES + 16 * (32 * h + srow);
        sbase = msc + (size_t)tile * nb * Q8_TILE_ROWS + srow;
    }
    const int vrow = Q8_GEMV_VROW(nb);
    float *xs = smem;              // nb * 32 floats, permuted
    float *vbuf = smem + nb * 32;  // EX: [NSLOT][RS][vrow] block values; else [NSLOT * nw][RS] wave sums
    float *pad = vbuf + (EX ? NSLOT * RS * vrow : NSLOT * nw * RS);

    const int st_begin = 8 * b_begin;
    const int st_end = 8 * b_end;
    const int st_clamp = max(st_end - 1, 0);
    f32x4 xv[Q8_GEMV_STAGE];
#pragma unroll
    for (int u = 0; u < XS; u++) {
        const float *xp = xg + 4 * min(st_begin + lane + 64 * u, st_clamp);
        xv[u] = (f32x4){xp[0], xp[1], xp[2], xp[3]};
    }
    // folded norm (gemv_body's): q8_rmsnorm_row's sum of squares in threads
    // 0..255 from x loads issued before the weights and summed after; EX
    // stages (x * scale) * w after a barrier, bit-identical to the tile
    // kernel, else x * w with the scale applied to the row sums
    const bool norm = norm_w != nullptr;  // kernel-uniform
    const int rope_position = rope_pos ? *rope_pos : 0;
    f32x4 wv[Q8_GEMV_STAGE];
    f32x4 nx[Q8_RSG_NORM_VEC];
    const int nv = nb * 8;
    if (norm) {
        const f32x4 *nwp = reinterpret_cast<const f32x4 *>(norm_w);
#pragma unroll
        for (int u = 0; u < XS; u++) wv[u] = nwp[min(st_begin + lane + 64 * u, st_clamp)];
        if (threadIdx.x < 256) {
            const f32x4 *xr = reinterpret_cast<const f32x4 *>(xg);
#pragma unroll
            for (int jj = 0; jj < Q8_RSG_NORM_VEC; jj++) {  // only the float4s the sum takes
                if ((int)threadIdx.x + 256 * jj < nv) nx[jj] = xr[threadIdx.x + 256 * jj];
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    // the weight stream goes out before anything waits for x
    i32x4 qv[NL];
    unsigned dd[NL];
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int b = min(b_begin + i * BPL + j, b_last);
        qv[i] = q8_weight_load(qbase + (size_t)b * qstride);
        dd[i] = (unsigned)sbase[(size_t)b * Q8_TILE_ROWS];
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (HOT) select_member();  // the epilogue's member, read while the weights stream in
    const int tile = SILU ? gtile : gtile - mtb;  // within the member
    __shared__ double npart[4];
    if (norm && threadIdx.x < 256) {
        double ss = 0.0;
#pragma unroll
        for (int jj = 0; jj < Q8_RSG_NORM_VEC; jj++) {
            if ((int)threadIdx.x + 256 * jj < nv) {
#pragma unroll
                for (int e = 0; e < 4; e++) ss += (double)(nx[jj][e] * nx[jj][e]);
            }
        }
        ss = xor_add_f64<32>(ss);
        ss = xor_add_f64<16>(ss);
        ss = xor_add_f64<8>(ss);
        ss = xor_add_f64<4>(ss);
        ss = xor_add_f64<2>(ss);
        ss = xor_add_f64<1>(ss);
        if (lane == 0) npart[wave] = ss;
    }
    if (norm) {
        float nscale = 1.0f;
        if constexpr (EX) {
            __syncthreads();
            nscale = norm_scale(npart, nb * 32, a.norm_eps);
        }
#pragma unroll
        for (int u = 0; u < XS; u++) {
#pragma unroll
            for (int e = 0; e < 4; e++) xv[u][e] = EX ? (xv[u][e] * nscale) * wv[u][e] : xv[u][e] * wv[u][e];
        }
    }
    if (EX && w == 0 && lane < RS) {
        for (int b = nb; b < ((nb + 3) & ~3); b++) vbuf[(slot * RS + r) * vrow + b] = 0.0f;
    }
#pragma unroll
    for (int u = 0; u < XS; u++) {
        if (64 * u < st_end - st_begin) {
            const int i = st_begin + lane + 64 * u;
            float *d = i < st_end ? xs + (i >> 3) * 32 + ((i & 7) >> 1) + 4 * (i & 1) : pad;
            d[0] = xv[u].x;
            d[8] = xv[u].y;
            d[16] = xv[u].z;
            d[24] = xv[u].w;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    float lsum = 0.0f;
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int bu = b_begin + i * BPL + j;
        const int b = min(bu, b_last);
        const float p = half_partial(qv[i], (const f32x4 *)(xs + b * 32 + h * 16));
        float s01;
        if constexpr (RS == 8) {
            s01 = p + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(p), 0x128, 0xf, 0xf, false));
        } else {
            const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(p), __float_as_uint(p), false, false);
            s01 = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        }
        const float v = f16_to_f32(dd[i]) * s01;
        if constexpr (EX) {
            *((h == 0 && bu < b_end) ? vbuf + (slot * RS + r) * vrow + bu : pad) = v;
        } else {
            lsum = bu < b_end ? lsum + v : lsum;
        }
    }
    if constexpr (!EX) {
        if constexpr (BPL >= 4) lsum = xor_add<16>(lsum);
        if constexpr (BPL >= 2) lsum = xor_add<32>(lsum);
        if (lane < RS) vbuf[wave * RS + r] = lsum;
    }
    __syncthreads();
    if (wave != 0 || lane >= RS) return;
    float sums[2] = {0.0f, 0.0f};
#pragma unroll
    for (int sl = 0; sl < NSLOT; sl++) {
        if constexpr (EX) {
            sums[sl] = chain_row(vbuf + (sl * RS + r) * vrow, nb);
        } else {
            float acc = vbuf[(sl * nw) * RS + r];
            for (int w2 = 1; w2 < nw; w2++) acc = acc + vbuf[(sl * nw + w2) * RS + r];
            sums[sl] = acc;
        }
    }
    if (!EX && norm) {  // the norm's scale, applied to the row sums
        const float s = norm_scale(npart, nb * 32, a.norm_eps);
        sums[0] *= s;
        sums[1] *= s;
    }
    const int row = tile * Q8_TILE_ROWS + srow;
    if constexpr (SILU) {
        if (row < mrows) my[row] = silu_f32(sums[0]) * sums[1];
    } else if (rope_pos) {
        // gemv_body's RoPE + KV append: rows 2i and 2i+1 of a head are lanes
        // r and r ^ 1 of wave 0 (RS is even, slices start at even rows)
        const float other = __shfl_xor(sums[0], 1);
        const int pos = rope_position;
        const bool in_cache = pos >= 0 && pos < a.capacity;
        if (row < mrows) {
            const int d = row % a.head_dim;
            const int pair = d >> 1;
            const bool even = (d & 1) == 0;
            const float x0 = even ? sums[0] : other;
            const float x1 = even ? other : sums[0];
            float y0 = x0, y1 = x1;
            if (in_cache && mi < 2 && 2 * pair < a.n_rot) {
                const float angle = (float)pos * a.rope_freq[pair];
                float sn, cs;
                sincosf(angle, &sn, &cs);
                y0 = x0 * cs - x1 * sn;
                y1 = x0 * sn + x1 * cs;
            }
            const float out = even ? y0 : y1;
            if (mi == 0) {
                my[row] = out;
            } else if (in_cache) {
                uint16_t *cache = mi == 1 ? a.kcache : a.vcache;
                cache[(size_t)pos * mrows + row] = (uint16_t)f16_bits(out);
            }
        }
    } else if (row < mrows) {
        my[row] = mbias ? sums[0] + mbias[row] : sums[0];
    }
}

// ---------------------------------------------------------------------------
// Row-slice GEMV over a contiguous gate/up pair (q8_gemv_hp16_l*; SILU pair:
// y = silu(gate . x) * (up . x)) reading the pair's paired copy
// (Q8SliceArgs::pair_tiles): a workgroup owns slice s of tile t, i.e. gate
// rows 32t + 8s .. + 7 and the same up rows, 16 rows a wave load as in
// gemv_rs_body's 16-row slices, so it has the whole K range of both members
// of each of its 8 outputs and no slot of idle waves.  Lane r < 8 of the
// tail wave takes its up row from lane r + 8.  Without the copy (sm = 0) the
// lanes read their rows from the unit layout.  The block values, their
// order and the folded norm are gemv_rsg_body's, so exact mode matches the
// tile kernels bit for bit.
// ---------------------------------------------------------------------------
template <int NL, int EX>
static __device__ __forceinline__ void gemv_rsp_body(const RsgHot &hot, const Q8GemvArgs &a) {
    extern __shared__ __attribute__((aligned(16))) float smem[];
    constexpr int RS = 16;                  // rows a slice: 8 gate + 8 up
    constexpr int LPB = 2 * RS;
    constexpr int BPL = 64 / LPB;
    constexpr int SPT = 4;                  // slices a tile pair
    constexpr int BPW = NL * BPL;
    constexpr int XS = (BPW * 8 + 63) / 64;
    static_assert(BPW * 8 <= 64 * Q8_GEMV_STAGE, "x range of a wave exceeds its staging registers");
    const int nb = hot.nbw & 0xffff;
    const int nw = hot.nbw >> 16;
    const float *xg = hot.xg;
    const int total_tiles = hot.tiles_xo & 0x3fffffff;
    const int xo = (int)((unsigned)hot.tiles_xo >> 31);
    const bool sm = (hot.tiles_xo >> 30) & 1;
    const float *norm_w = hot.norm_w;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane / LPB;
    const int h = (lane / RS) & 1;
    const int r = lane % RS;
    const int bx = blockIdx.x;
    const int tile = xo ? (bx / (8 * SPT)) * 8 + (bx & 7) : bx / SPT;
    const int slice = xo ? (bx >> 3) % SPT : bx % SPT;
    if (tile >= total_tiles) return;  // padding of the XCD order, whole workgroup
    const int up = r >> 3;             // 0: a gate row, 1: an up row
    const int mrow = 8 * slice + (r & 7);  // the row within its member's tile
    const int mt = tile + (up ? hot.up_off : 0);
    const int b_begin = wave * BPW;
    const int b_end = min(nb, b_begin + BPW);
    const int b_last = max(b_end - 1, 0);
    const uint8_t *qbase = sm ? hot.mq + ((size_t)tile * SPT + slice) * nb * (RS * 32) + 16 * (lane % LPB)
                              : hot.mq + (size_t)mt * nb * Q8_UNIT_BYTES + 16 * (32 * h + mrow);
    const size_t qstride = sm ? (size_t)(RS * 32) : (size_t)Q8_UNIT_BYTES;
    const uint16_t *sbase = hot.msc + (size_t)mt * nb * Q8_TILE_ROWS + mrow;
    const int vrow = Q8_GEMV_VROW(nb);
    float *xs = smem;              // nb * 32 floats, permuted
    float *vbuf = smem + nb * 32;  // EX: [RS][vrow] block values; else [nw][RS] wave sums
    float *pad = vbuf + (EX ? RS * vrow : nw * RS);

    const int st_begin = 8 * b_begin;
    const int st_end = 8 * b_end;
    const int st_clamp = max(st_end - 1, 0);
    f32x4 xv[Q8_GEMV_STAGE];
#pragma unroll
    for (int u = 0; u < XS; u++) {
        const float *xp = xg + 4 * min(st_begin + lane + 64 * u, st_clamp);
        xv[u] = (f32x4){xp[0], xp[1], xp[2], xp[3]};
    }
    // the folded norm, as gemv_rsg_body's
    const bool norm = norm_w != nullptr;  // kernel-uniform
    f32x4 wv[Q8_GEMV_STAGE];
    f32x4 nx[Q8_RSG_NORM_VEC];
    const int nv = nb * 8;
    if (norm) {
        const f32x4 *nwp = reinterpret_cast<const f32x4 *>(norm_w);
#pragma unroll
        for (int u = 0; u < XS; u++) wv[u] = nwp[min(st_begin + lane + 64 * u, st_clamp)];
        if (threadIdx.x < 256) {
            const f32x4 *xr = reinterpret_cast<const f32x4 *>(xg);
#pragma unroll
            for (int jj = 0; jj < Q8_RSG_NORM_VEC; jj++) {
                if ((int)threadIdx.x + 256 * jj < nv) nx[jj] = xr[threadIdx.x + 256 * jj];
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    i32x4 qv[NL];
    unsigned dd[NL];
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int b = min(b_begin + i * BPL + j, b_last);
        qv[i] = q8_weight_load(qbase + (size_t)b * qstride);
        dd[i] = (unsigned)sbase[(size_t)b * Q8_TILE_ROWS];
    }
    __builtin_amdgcn_sched_barrier(0);
    __shared__ double npart[4];
    if (norm && threadIdx.x < 256) {
        double ss = 0.0;
#pragma unroll
        for (int jj = 0; jj < Q8_RSG_NORM_VEC; jj++) {
            if ((int)threadIdx.x + 256 * jj < nv) {
#pragma unroll
                for (int e = 0; e < 4; e++) ss += (double)(nx[jj][e] * nx[jj][e]);
            }
        }
        ss = xor_add_f64<32>(ss);
        ss = xor_add_f64<16>(ss);
        ss = xor_add_f64<8>(ss);
        ss = xor_add_f64<4>(ss);
        ss = xor_add_f64<2>(ss);
        ss = xor_add_f64<1>(ss);
        if (lane == 0) npart[wave] = ss;
    }
    if (norm) {
        float nscale = 1.0f;
        if constexpr (EX) {
            __syncthreads();
            nscale = norm_scale(npart, nb * 32, a.norm_eps);
        }
#pragma unroll
        for (int u = 0; u < XS; u++) {
#pragma unroll
            for (int e = 0; e < 4; e++) xv[u][e] = EX ? (xv[u][e] * nscale) * wv[u][e] : xv[u][e] * wv[u][e];
        }
    }
    if (EX && wave == 0 && lane < RS) {
        for (int b = nb; b < ((nb + 3) & ~3); b++) vbuf[r * vrow + b] = 0.0f;
    }
#pragma unroll
    for (int u = 0; u < XS; u++) {
        if (64 * u < st_end - st_begin) {
            const int i = st_begin + lane + 64 * u;
            float *d = i < st_end ? xs + (i >> 3) * 32 + ((i & 7) >> 1) + 4 * (i & 1) : pad;
            d[0] = xv[u].x;
            d[8] = xv[u].y;
            d[16] = xv[u].z;
            d[24] = xv[u].w;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    float lsum = 0.0f;
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int bu = b_begin + i * BPL + j;
        const int b = min(bu, b_last);
        const float p = half_partial(qv[i], (const f32x4 *)(xs + b * 32 + h * 16));
        const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(p), __float_as_uint(p), false, false);
        const float s01 = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
        const float v = f16_to_f32(dd[i]) * s01;
        if constexpr (EX) {
            *((h == 0 && bu < b_end) ? vbuf + r * vrow + bu : pad) = v;
        } else {
            lsum = bu < b_end ? lsum + v : lsum;
        }
    }
    if constexpr (!EX) {
        if constexpr (BPL >= 2) lsum = xor_add<32>(lsum);
        if (lane < RS) vbuf[wave * RS + r] = lsum;
    }
    __syncthreads();
    if (wave != 0) return;
    float sum = 0.0f;
    if (lane < RS) {
        if constexpr (EX) {
            sum = chain_row(vbuf + r * vrow, nb);
        } else {
            sum = vbuf[r];
            for (int w2 = 1; w2 < nw; w2++) sum = sum + vbuf[w2 * RS + r];
        }
        if (!EX && norm) sum *= norm_scale(npart, nb * 32, a.norm_eps);
    }
    const float upv = __shfl_down(sum, 8);  // lane r < 8: its up row's sum
    const int row = tile * Q8_TILE_ROWS + mrow;
    if (lane < 8 && row < a.m[0].rows) a.m[0].y[row] = silu_f32(sum) * upv;
}

#define Q8_RSG_PARAMS                                                                                   \
    const uint8_t *mq, const uint16_t *msc, const float *xg, const float *norm_w, const int *rope_pos, int nbw, \
        int tiles_xo, int up_off, int hpad, Q8GemvArgs a
#define Q8_GEMV_RSG_KERNEL(KIND, SILU, RS, NL)                                                                  \
    extern "C" __global__ __launch_bounds__(1024) void q8_gemv_##KIND##RS##_l##NL(Q8GemvArgs a) {            \
        gemv_rsg_body<RS, NL, 1, SILU>(RsgHot{}, a);                                                           \
    }                                                                                                          \
    extern "C" __global__ __launch_bounds__(1024) void q8_gemv_##KIND##RS##_l##NL##_e0(Q8GemvArgs a) {       \
        gemv_rsg_body<RS, NL, 0, SILU>(RsgHot{}, a);                                                           \
    }                                                                                                          \
    extern "C" __global__ __launch_bounds__(1024) void q8_gemv_h##KIND##RS##_l##NL(Q8_RSG_PARAMS) {          \
        gemv_rsg_body<RS, NL, 1, SILU, 1>(RsgHot{mq, msc, xg, norm_w, rope_pos, nbw, tiles_xo, up_off, hpad}, a); \
    }                                                                                                          \
    extern "C" __global__ __launch_bounds__(1024) void q8_gemv_h##KIND##RS##_l##NL##_e0(Q8_RSG_PARAMS) {     \
        gemv_rsg_body<RS, NL, 0, SILU, 1>(RsgHot{mq, msc, xg, norm_w, rope_pos, nbw, tiles_xo, up_off, hpad}, a); \
    }
Q8_GEMV_RSG_KERNEL(g, 0, 8, 3)
Q8_GEMV_RSG_KERNEL(g, 0, 16, 3)
Q8_GEMV_RSG_KERNEL(g, 0, 16, 6)
Q8_GEMV_RSG_KERNEL(s, 1, 8, 3)
Q8_GEMV_RSG_KERNEL(s, 1, 16, 6)
#define Q8_GEMV_RSP_KERNEL(NL)                                                                     \
    extern "C" __global__ __launch_bounds__(1024) void q8_gemv_hp16_l##NL(Q8_RSG_PARAMS) {      \
        gemv_rsp_body<NL, 1>(RsgHot{mq, msc, xg, norm_w, rope_pos, nbw, tiles_xo, up_off, hpad}, a); \
    }                                                                                              \
    extern "C" __global__ __launch_bounds__(1024) void q8_gemv_hp16_l##NL##_e0(Q8_RSG_PARAMS) { \
        gemv_rsp_body<NL, 0>(RsgHot{mq, msc, xg, norm_w, rope_pos, nbw, tiles_xo, up_off, hpad}, a); \
    }
Q8_GEMV_RSP_KERNEL(3)
Q8_GEMV_RSP_KERNEL(6)

// ---------------------------------------------------------------------------
// Activation quantization (quant.rs:98-121), into the prepared tile layout.
//
// e[q][c] is half h of one token's block: element 8c + J[h][q].  half_peak is
// the max |e| of the half (f32::max ignores NaN, as fmaxf does); quant_store
// quantizes with the block's peak (both halves) and writes the half as lane
// slot `slot` (= 32h + token % 32) of prepared unit `u` (int8 or f16 form),
// and, when `write_scale`, the block's f32 scale.
static __device__ __forceinline__ float half_peak(const float (&e)[4][4]) {
    float peak = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int c = 0; c < 4; c++) peak = fmaxf(peak, fabsf(e[q][c]));
    return peak;
}

static __device__ __forceinline__ void quant_store(const float (&e)[4][4], float peak, uint8_t *xq, float *xs,
                                                   size_t u, int slot, bool write_scale, int f16) {
    const float scale = peak / 127.0f;
    const float inverse = peak > 0.0f ? 127.0f / peak : 0.0f;
    i32x4 packed;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        unsigned w = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float prod = e[q][c] * inverse;
            w |= ((unsigned)sat_i8(roundf(prod)) & 0xffu) << (8 * c);
        }
        packed[q] = (int)w;
    }
    if (f16) {
        // the same values as f16, bytes 0-7 to the unit's first half, 8-15 to its second
        uint8_t *dst = xq + u * Q8_UNIT_F16_BYTES + slot * 16;
        *(i32x4 *)dst = i8x4_to_f16x4(packed[0], packed[1]);
        *(i32x4 *)(dst + 1024) = i8x4_to_f16x4(packed[2], packed[3]);
    } else {
        *(i32x4 *)(xq + u * Q8_UNIT_BYTES + slot * 16) = packed;
    }
    if (write_scale) xs[u * Q8_TILE_TOKENS + (slot & 31)] = scale;
}

// One wave per (32-token tile, block) unit.  The unit's 32 token rows of 32
// elements are read as whole 128-byte pieces (lane L takes float4 L % 8 of
// rows L / 8 + 8u, u = 0..3: each load instruction covers eight rows) into a
// wave-private LDS tile of 36 floats a row; then lane L = 32h + t takes half
// h of token t's block in the AVX2 lane order J[h][0..3] across the four
// chunks and writes it as one 16-byte store, so the wave's stores are one
// contiguous 1 KB unit.  The block peak is the max of the two halves' peaks
// (one v_permlane32_swap).
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void q8_quantize(Q8QuantArgs a) {
    __shared__ __attribute__((aligned(16))) float qtile[4][32 * Q8_NORM_LDS_PITCH];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int unit = blockIdx.x * (blockDim.x >> 6) + wv;
    const int nb = a.nb;
    if (unit >= a.ttiles * nb) return;  // whole waves
    const int tt = unit / nb;
    const int b = unit - tt * nb;
    float *tile = qtile[wv];
    {
        const int f8 = lane & 7;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int row = (lane >> 3) + 8 * u;
            const int t = tt * Q8_TILE_TOKENS + row;
            const size_t off = (size_t)min(t, a.n - 1) * nb * 32 + (size_t)b * 32 + 4 * f8;
            f32x4 v;
            if (a.mode == 0) {
                v = *(const f32x4 *)(a.x + off);
            } else {
                const f32x4 g = *(const f32x4 *)(a.gate + off);
                const f32x4 up = *(const f32x4 *)(a.up + off);
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = silu_f32(g[e]) * up[e];
            }
            if (t >= a.n) v = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};  // tokens past n quantize as zeros
            *(f32x4 *)(tile + row * Q8_NORM_LDS_PITCH + 4 * f8) = v;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int h = lane >> 5;
    const int tl = lane & 31;
    // chunk c: elements 8c + 2h, +1 (dwords 0, 2) and 8c + 4 + 2h, +1 (dwords 1, 3)
    const float *src = tile + tl * Q8_NORM_LDS_PITCH + 2 * h;
    float e[4][4];  // e[q][c]
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const float2 lo = *(const float2 *)(src + 8 * c);
        const float2 hi = *(const float2 *)(src + 8 * c + 4);
        e[0][c] = lo.x;  // J[h][0] = 2h
        e[2][c] = lo.y;  // J[h][2] = 2h + 1
        e[1][c] = hi.x;  // J[h][1] = 4 + 2h
        e[3][c] = hi.y;  // J[h][3] = 5 + 2h
    }
    float peak = half_peak(e);
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(peak), __float_as_uint(peak), false, false);
    peak = fmaxf(peak, __uint_as_float(h ? sw[0] : sw[1]));
    quant_store(e, peak, a.xq, a.xs, (size_t)tt * nb + b, lane, h == 0, a.f16);
}

// ---------------------------------------------------------------------------
// GEMM epilogue shared by the GEMM kernels: lane (h, r) of a wave holds row o
// = 32g + r of TPW 32 x 32 output tiles, tokens 8(i/4) + 4h + (i%4) of each.
// The residual (bias) values are loaded first, all 16 per tile at clamped
// addresses, so their loads are in flight together; then the stores.
// ---------------------------------------------------------------------------
//
// With rope_pos set (a q, k, v group, member mi), the tile goes through
// q8_rope_append's arithmetic instead: rows 2i and 2i+1 of a head are lanes r
// and r ^ 1 (tiles start at multiples of 32 and head_dim is even), so each
// lane takes its partner's value for the same token by one shuffle and keeps
// its half of the rotated pair -- the angle (position * freq), sincosf and
// the f16 narrowing of that kernel.  q is written rotated in f32; k rotated
// and v as they are go only to the f16 caches, at row position + token.
template <int TPW>
static __device__ __forceinline__ void store_rope_tiles(const Q8GemmArgs &a, const Q8GemmMember &mem, int mi,
                                                        const f32x16 (&acc)[TPW], int tt0, int o, int h) {
    const int start = *a.rope_pos;
    const int d = o % a.head_dim;
    const int pair = d >> 1;
    const bool even = (d & 1) == 0;
    const bool rot = mi < 2 && 2 * pair < a.n_rot;
    const float freq = rot ? a.rope_freq[pair] : 0.0f;
    uint16_t *cache = mi == 1 ? a.kcache : a.vcache;
    const int odd = even ? 0 : 1;  // of the pair's lanes r, r ^ 1, the odd one takes elements 8..15
#pragma unroll
    for (int t = 0; t < TPW; t++) {
        if (tt0 + t >= a.ttiles) continue;  // wave-uniform
        const int tok0 = (tt0 + t) * Q8_TILE_TOKENS + 4 * h;  // token of element i: tok0 + 8(i/4) + i%4
        // The pair's two lanes need the same 16 angles: each computes eight
        // (the even lane elements 0-7, the odd lane 8-15) and they swap.
        float sn[16], cs[16];
        if (mi < 2) {  // wave-uniform
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int i = j + 8 * odd;
                const float angle = (float)(start + tok0 + 8 * (i >> 2) + (i & 3)) * freq;
                float sj, cj;
                sincosf(angle, &sj, &cj);
                const float so = __shfl_xor(sj, 1), co = __shfl_xor(cj, 1);
                sn[j] = odd ? so : sj;
                cs[j] = odd ? co : cj;
                sn[j + 8] = odd ? sj : so;
                cs[j + 8] = odd ? cj : co;
            }
        }
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float x = acc[t][i];
            const float other = __shfl_xor(x, 1);  // the partner row, same token
            const int tok = tok0 + 8 * (i >> 2) + (i & 3);
            const int pos = start + tok;
            const bool in_cache = pos >= 0 && pos < a.capacity;
            if (tok < a.n && o < mem.rows) {
                const float x0 = even ? x : other;
                const float x1 = even ? other : x;
                float y0 = x0, y1 = x1;
                if (in_cache && rot) {
                    y0 = x0 * cs[i] - x1 * sn[i];
                    y1 = x0 * sn[i] + x1 * cs[i];
                }
                const float out = even ? y0 : y1;
                if (mi == 0) {
                    mem.y[(size_t)tok * mem.rows + o] = out;
                } else if (in_cache) {
                    cache[(size_t)pos * mem.rows + o] = (uint16_t)f16_bits(out);
                }
            }
        }
    }
}

template <int TPW>
static __device__ __forceinline__ void store_tiles(const Q8GemmArgs &a, const Q8GemmMember &mem, int mi,
                                                   const f32x16 (&acc)[TPW], int tt0, int o, int h) {
    if (a.rope_pos) {
        store_rope_tiles<TPW>(a, mem, mi, acc, tt0, o, h);
        return;
    }
    if (o >= mem.rows) return;
#pragma unroll
    for (int t = 0; t < TPW; t++) {
        if (tt0 + t >= a.ttiles) continue;
        float add[16];
#pragma unroll
        for (int i = 0; i < 16; i++) add[i] = 0.0f;
        if (mem.bias) {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int tok = min((tt0 + t) * Q8_TILE_TOKENS + 8 * (i >> 2) + 4 * h + (i & 3), a.n - 1);
                add[i] = mem.bias[(size_t)tok * mem.rows + o];
            }
        }
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int tok = (tt0 + t) * Q8_TILE_TOKENS + 8 * (i >> 2) + 4 * h + (i & 3);
            if (tok < a.n) mem.y[(size_t)tok * mem.rows + o] = mem.bias ? acc[t][i] + add[i] : acc[t][i];
        }
    }
}

// ---------------------------------------------------------------------------
// GEMM, n >= 2 (tensor.rs:104-148 -> quant.rs:156-181).
//
// v_mfma_i32_32x32x32_i8 is exactly one Q8_0 block per instruction, so its
// int32 result is the reference's exact block dot sum q_w q_x.  A =
// activations (tokens), B = weights (rows): each lane owns one output row and
// its stores are row-contiguous.  The per-block f32 scale d_w * s_x is
//   SMODE 1: one v_mfma_f32_32x32x1_2b_f32 outer product per block pair, which
//            lands in the accumulator's register layout, or
//   SMODE 0: VALU multiplies of the lane's row scale by its 16 token scales;
// then acc = fma(float(I_b), d_w*s_x, acc) block by block, as the reference's
// AVX2 lanes accumulate.
//
// A wave owns TPW token tiles x one 32-row tile: the weight stream and its
// scale are loaded once for TPW tiles, and the TPW independent MFMA chains
// keep the wave busy while one of them waits.  A workgroup holds twaves such
// waves along the tokens times kwaves along K; the K-split waves are reduced
// in LDS in a fixed order, and optional K slices across workgroups by the
// last workgroup to arrive.
// ---------------------------------------------------------------------------
// A cache rider (Q8GemmArgs::riders): rider workgroup `rider` of `riders`
// reads its share of the rider weights' quants and scales, taken as one
// sequence of 16-byte chunks (weight 0's quants, its scales, weight 1's ...),
// in address order and in batches of 16 loads a lane, and keeps nothing: the
// reads only leave the weights in the L2 and the Infinity Cache.
static __device__ __forceinline__ void gemm_rider(const Q8GemmArgs &a, int rider) {
    constexpr int BATCH = 16;
    const int nt = blockDim.x;
    const int t = threadIdx.x;
    constexpr long long UNIT_CHUNKS = (Q8_UNIT_BYTES + Q8_TILE_ROWS * 2) / 16;
    long long chunks = 0;
    for (int i = 0; i < a.rider_count; i++) chunks += (long long)a.rider_units[i] * UNIT_CHUNKS;
    const long long per = (chunks + a.riders - 1) / a.riders;
    const long long c0 = (long long)rider * per;
    const long long c1 = min(chunks, c0 + per);
    long long off = 0;
    for (int i = 0; i < 2 * a.rider_count; i++) {
        const uint8_t *base = (i & 1) ? reinterpret_cast<const uint8_t *>(a.rider_s[i >> 1]) : a.rider_q[i >> 1];
        const long long len = (long long)a.rider_units[i >> 1] * ((i & 1) ? Q8_TILE_ROWS * 2 : Q8_UNIT_BYTES) / 16;
        const long long lo = max(c0, off) - off, hi = min(c1, off + len) - off;
        for (long long c = lo; c < hi; c += (long long)nt * BATCH) {
            i32x4 v[BATCH];
#pragma unroll
            for (int j = 0; j < BATCH; j++) {
                const i32x4 *p = reinterpret_cast<const i32x4 *>(base) + min(c + t + (long long)nt * j, hi - 1);
                v[j] = a.rider_nt ? __builtin_nontemporal_load(p) : *p;
            }
#pragma unroll
            for (int j = 0; j < BATCH; j++) asm volatile("" ::"v"(v[j]));
        }
        off += len;
    }
}

// The compute workgroup of grid workgroup `b`, or -1 for a cache rider (which
// it has then run).
static __device__ __forceinline__ int gemm_workgroup(const Q8GemmArgs &a, int b) {
    if (a.riders) {
        const int r = a.rider_first ? b : b - a.nwg;
        if (r >= 0 && r < a.riders) {
            gemm_rider(a, r);
            return -1;
        }
        if (a.rider_first) b -= a.riders;
    }
    if (a.xcd_remap) {
        const int per = a.nwg >> 3;
        b = (b & 7) * per + (b >> 3);
    }
    return b;
}

template <int TPW>
struct GemmOps {
    i32x4 w0, w1;
    unsigned dw;
    i32x4 x0[TPW], x1[TPW];
    float sx[TPW];
};

// NT: the weight quants are read non-temporally, for launches where one wave
// covers every token tile of its row tile, so each weight byte is read once
// (one token tile: configs[1] n = 8, 10.15 -> 9.74 us; with more token groups
// the re-reads want the caches: n = 512 142 -> 148 us).
template <int SMODE, int TPW, bool NT = false>
static __device__ __forceinline__ void gemm_body(const Q8GemmArgs &a) {
    extern __shared__ __attribute__((aligned(16))) float gsm[];  // [kwaves-1][twaves][TPW][64][16]
    __shared__ int last_flag;
    kernarg_lines<Q8GemmArgs>();
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform, in an SGPR
    const int TW = a.twaves;
    const int tw = wave % TW;  // token-tile group of this wave
    const int kw = wave / TW;  // K-split wave
    const int S = a.kslices;
    const int wg = gemm_workgroup(a, blockIdx.x);
    if (wg < 0) return;
    // workgroup -> (row tile, token group, K slice); slices of one tile are adjacent
    const int slice = wg % S;
    const int rtg = wg / S;
    const int rt = rtg / a.tgroups;
    const int tg = rtg - rt * a.tgroups;
    const int tt0 = (tg * TW + tw) * TPW;               // first token tile of this wave
    const int ntl = max(0, min(TPW, a.ttiles - tt0));   // live token tiles (wave-uniform)
    int mi = 0;
#pragma unroll
    for (int i = 1; i < Q8_GROUP_MAX; i++)
        if (i < a.members && rt >= a.m[i].tile_begin) mi = i;
    const Q8GemmMember mem = a.m[mi];
    const int g = rt - mem.tile_begin;
    const int nb = a.nb;
    const int h = lane >> 5;
    const int r = lane & 31;
    // Stream bases are wave-uniform (SGPRs); a lane adds only its constant
    // offset, so loads need no per-block VALU address arithmetic.
    const uint8_t *wq = mem.quants + (size_t)g * nb * Q8_UNIT_BYTES;
    const uint16_t *wsc = mem.scales + (size_t)g * nb * Q8_TILE_ROWS;
    const uint8_t *xq[TPW];
    const float *xsc[TPW];
#pragma unroll
    for (int t = 0; t < TPW; t++) {
        const int ttc = min(tt0 + t, a.ttiles - 1);  // clamped: always a valid tile to address
        xq[t] = a.xq + (size_t)ttc * nb * Q8_UNIT_BYTES;
        xsc[t] = a.xs + (size_t)ttc * nb * Q8_TILE_TOKENS;
    }
    const int lo = lane * 16;
    const q8_stream_t wr = q8_stream(wq, nb * Q8_UNIT_BYTES);
    const q8_stream_t wsr = q8_stream(wsc, nb * Q8_TILE_ROWS * 2);
    q8_stream_t xr[TPW], xsr[TPW];
#pragma unroll
    for (int t = 0; t < TPW; t++) {
        xr[t] = q8_stream(xq[t], nb * Q8_UNIT_BYTES);
        xsr[t] = q8_stream(xsc[t], nb * Q8_TILE_TOKENS * 4);
    }

    // this wave's block pairs: slice range split over the kw waves
    const int npairs = (nb + 1) >> 1;
    const int s_begin = slice * a.pairs_per_slice;
    const int s_end = min(npairs, s_begin + a.pairs_per_slice);
    const int p_begin = s_begin + kw * a.pairs_per_wave;
    const int p_end = ntl > 0 ? min(s_end, p_begin + a.pairs_per_wave) : p_begin;
    const int full_end = min(p_end, nb >> 1);  // pairs whose two blocks both exist

    f32x16 acc[TPW];
#pragma unroll
    for (int t = 0; t < TPW; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[t][i] = 0.0f;
    const i32x16 izero = {};
    const f32x32 fzero = {};

    // Loads of the full pair (b, b+1): lane L's scale slot (b + h, r) is
    // element b*32 + L of the scale stream.
    auto load_full = [&](GemmOps<TPW> &q, int b) {
        const int u0 = b * Q8_UNIT_BYTES;
        q.w0 = q8_load16<NT>(wr, lo, u0);
        q.w1 = q8_load16<NT>(wr, lo, u0 + Q8_UNIT_BYTES);
        q.dw = __builtin_amdgcn_raw_buffer_load_b16(wsr, 2 * lane, b * Q8_TILE_ROWS * 2, 0);
#pragma unroll
        for (int t = 0; t < TPW; t++) {
            q.x0[t] = q8_load16(xr[t], lo, u0);
            q.x1[t] = q8_load16(xr[t], lo, u0 + Q8_UNIT_BYTES);
            q.sx[t] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xsr[t], 4 * lane,
                                                                                     b * Q8_TILE_TOKENS * 4, 0));
        }
    };
    // The odd last block of an odd nb: the absent block repeats block b with
    // zero scales, so it adds 0 * 0.
    auto load_last = [&](GemmOps<TPW> &q, int b) {
        const int u0 = b * Q8_UNIT_BYTES;
        q.w0 = q8_load16<NT>(wr, lo, u0);
        q.w1 = q.w0;
        const unsigned dwr = __builtin_amdgcn_raw_buffer_load_b16(wsr, 2 * r, b * Q8_TILE_ROWS * 2, 0);
        q.dw = h ? 0u : dwr;
#pragma unroll
        for (int t = 0; t < TPW; t++) {
            q.x0[t] = q8_load16(xr[t], lo, u0);
            q.x1[t] = q.x0[t];
            const float sxr = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xsr[t], 4 * r,
                                                                                            b * Q8_TILE_TOKENS * 4, 0));
            q.sx[t] = h ? 0.0f : sxr;
        }
    };
    // One block pair of one token tile: the scale products first (the
    // longest MFMA), then the two block dots, then block b's and block b+1's
    // epilogues in that order.
    auto step = [&](const GemmOps<TPW> &q, int t, int b, bool two) {
        if (SMODE == 1) {
            // lanes 0-31 carry block b and lanes 32-63 block b+1: the two blocks
            // of the outer-product MFMA, d_w * s_x in the accumulator layout.
            const f32x32 sc = __builtin_amdgcn_mfma_f32_32x32x1f32(q.sx[t], f16_to_f32(q.dw), fzero, 0, 0, 0);
            const i32x16 i0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(q.x0[t], q.w0, izero, 0, 0, 0);
            const i32x16 i1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(q.x1[t], q.w1, izero, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 16; i++) acc[t][i] = __builtin_fmaf((float)i0[i], sc[i], acc[t][i]);
            if (two) {
#pragma unroll
                for (int i = 0; i < 16; i++) acc[t][i] = __builtin_fmaf((float)i1[i], sc[16 + i], acc[t][i]);
            }
        } else {
            const i32x16 i0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(q.x0[t], q.w0, izero, 0, 0, 0);
            const i32x16 i1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(q.x1[t], q.w1, izero, 0, 0, 0);
            // lane owns row r and tokens 8(i/4) + 4h + (i%4) of the tile
            const int b1 = two ? b + 1 : b;
            const float dw0 = f16_to_f32(wsc[(size_t)b * Q8_TILE_ROWS + r]);
            const float dw1 = f16_to_f32(wsc[(size_t)b1 * Q8_TILE_ROWS + r]);
            const float *xs0 = xsc[t] + (size_t)b * Q8_TILE_TOKENS + 4 * h;
            const float *xs1 = xsc[t] + (size_t)b1 * Q8_TILE_TOKENS + 4 * h;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const float c0 = dw0 * xs0[8 * (i >> 2) + (i & 3)];
                acc[t][i] = __builtin_fmaf((float)i0[i], c0, acc[t][i]);
            }
            if (two) {
#pragma unroll
                for (int i = 0; i < 16; i++) {
                    const float c1 = dw1 * xs1[8 * (i >> 2) + (i & 3)];
                    acc[t][i] = __builtin_fmaf((float)i1[i], c1, acc[t][i]);
                }
            }
        }
    };

    // Full pairs, two per iteration with ping-pong operand sets (no register
    // copies); each set's loads are issued one pair ahead of its use, and
    // sched_barrier keeps the compiler from sinking them next to their use.
    if (p_begin < full_end) {
        GemmOps<TPW> qa, qb;
        load_full(qa, 2 * p_begin);
        int p = p_begin;
        for (; p + 1 < full_end; p += 2) {
            load_full(qb, 2 * (p + 1));
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < TPW; t++) step(qa, t, 2 * p, true);
            __builtin_amdgcn_sched_barrier(0);
            load_full(qa, 2 * min(p + 2, full_end - 1));
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < TPW; t++) step(qb, t, 2 * (p + 1), true);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (p < full_end) {
#pragma unroll
            for (int t = 0; t < TPW; t++) step(qa, t, 2 * p, true);
        }
    }
    if (full_end < p_end) {  // odd nb: the last pair holds one block
        GemmOps<TPW> q;
        load_last(q, 2 * full_end);
#pragma unroll
        for (int t = 0; t < TPW; t++) step(q, t, 2 * full_end, false);
    }

    const int KW = (blockDim.x >> 6) / TW;
    if (KW > 1) {
        // reduce the K-split waves in a fixed order: kw = 0 adds 1, 2, ...
        if (kw > 0) {
#pragma unroll
            for (int t = 0; t < TPW; t++) {
                float *dst = gsm + ((size_t)(((kw - 1) * TW + tw) * TPW + t) * 64 + lane) * 16;
#pragma unroll
                for (int i = 0; i < 16; i += 4)
                    *(f32x4 *)(dst + i) = (f32x4){acc[t][i], acc[t][i + 1], acc[t][i + 2], acc[t][i + 3]};
            }
        }
        __syncthreads();
        if (kw == 0) {
            for (int k2 = 1; k2 < KW; k2++) {
#pragma unroll
                for (int t = 0; t < TPW; t++) {
                    const float *src = gsm + ((size_t)(((k2 - 1) * TW + tw) * TPW + t) * 64 + lane) * 16;
#pragma unroll
                    for (int i = 0; i < 16; i++) acc[t][i] = acc[t][i] + src[i];
                }
            }
        }
    }
    if (S > 1) {
        // per-slice partial tiles in scratch; the tile group's last workgroup sums them in slice order
        if (kw == 0) {
#pragma unroll
            for (int t = 0; t < TPW; t++) {
                if (t < ntl) {
                    float *part = a.scratch + ((size_t)(((size_t)rt * a.ttiles + tt0 + t) * S + slice) * 64 + lane) * 16;
#pragma unroll
                    for (int i = 0; i < 16; i += 4)
                        *(f32x4 *)(part + i) = (f32x4){acc[t][i], acc[t][i + 1], acc[t][i + 2], acc[t][i + 3]};
                }
            }
        }
        __threadfence();
        __syncthreads();
        if (threadIdx.x == 0) {
            const unsigned old = atomicAdd(&a.counters[rtg], 1u);
            last_flag = (old == (unsigned)(S - 1));
        }
        __syncthreads();
        if (!last_flag) return;
        __threadfence();
        if (threadIdx.x == 0) a.counters[rtg] = 0u;
        if (kw == 0) {
#pragma unroll
            for (int t = 0; t < TPW; t++) {
                if (t < ntl) {
                    const float *base = a.scratch + ((size_t)(((size_t)rt * a.ttiles + tt0 + t) * S) * 64 + lane) * 16;
#pragma unroll
                    for (int i = 0; i < 16; i++) acc[t][i] = 0.0f;
                    for (int sl = 0; sl < S; sl++) {
                        const float *src = base + (size_t)sl * 64 * 16;
#pragma unroll
                        for (int i = 0; i < 16; i++) acc[t][i] = acc[t][i] + src[i];
                    }
                }
            }
        }
    }
    if (kw != 0) return;

    store_tiles<TPW>(a, mem, mi, acc, tt0, g * Q8_TILE_ROWS + r, h);
}

// ---------------------------------------------------------------------------
// Gate/up GEMM with silu(gate) * up quantized straight to prepared Q8_0 for the
// down projection (Compute::silu_mul_prepare after matmul_prepared_group,
// compute.rs:993-1019 and 437-472; gpu.cu silu_mul_quantize_rows 812-853).
//
// Members m[0] = gate and m[1] = up, same shape.  A workgroup owns gate row
// tile g, the up row tile g and one token tile; its KW waves split the block
// pairs.  A wave runs the int8 GEMM's per-block arithmetic (int32 block dot on
// v_mfma_i32_32x32x32_i8, d_w * s_x from the outer-product MFMA, fma) on both
// weight streams with one activation stream, so gate and up are exactly the
// values the plain GEMM stores.  After the fixed-order K reduction, wave 0
// forms v = silu(g) * u for its 32 features x 32 tokens: feature block g of
// every token, one Q8_0 block each.  The tile goes through LDS from the MFMA
// layout (lane = feature, 16 tokens) to the prepared lane order (lane =
// token half, elements 8c + J[h][q]) and is quantized by quant_store, the
// quantizer's own code: the bytes equal q8_quantize of silu(gate) * up.
// LDS: max((KW - 1) * 2 accumulator sets, the 32 x 33 transpose).
// ---------------------------------------------------------------------------
struct SiluOps {
    i32x4 w0, w1, u0, u1;
    unsigned dw, du;
    i32x4 x0, x1;
    float sx;
};

extern "C" __global__ __launch_bounds__(512) void q8_gemm_silu(Q8GemmArgs a) {
    extern __shared__ __attribute__((aligned(16))) float ssm[];
    kernarg_lines<Q8GemmArgs, true>();
    const int lane = threadIdx.x & 63;
    const int kw = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int KW = blockDim.x >> 6;
    const int wg = gemm_workgroup(a, blockIdx.x);
    if (wg < 0) return;
    const int g = wg / a.ttiles;   // gate (and up) row tile = output feature block
    const int tt = wg - g * a.ttiles;
    const Q8GemmMember gm = a.m[0], um = a.m[1];
    const int nb = a.nb;
    const int h = lane >> 5;
    const int r = lane & 31;
    const uint8_t *wq = gm.quants + (size_t)g * nb * Q8_UNIT_BYTES;
    const uint16_t *wsc = gm.scales + (size_t)g * nb * Q8_TILE_ROWS;
    const uint8_t *uq = um.quants + (size_t)g * nb * Q8_UNIT_BYTES;
    const uint16_t *usc = um.scales + (size_t)g * nb * Q8_TILE_ROWS;
    const uint8_t *xq = a.xq + (size_t)tt * nb * Q8_UNIT_BYTES;
    const float *xsc = a.xs + (size_t)tt * nb * Q8_TILE_TOKENS;
    const int lo = lane * 16;
    const int npairs = (nb + 1) >> 1;
    const int p_begin = kw * a.pairs_per_wave;
    const int p_end = min(npairs, p_begin + a.pairs_per_wave);
    const int full_end = min(p_end, nb >> 1);

    f32x16 ag = {}, au = {};
    const i32x16 izero = {};
    const f32x32 fzero = {};
    const q8_stream_t wr = q8_stream(wq, nb * Q8_UNIT_BYTES), ur = q8_stream(uq, nb * Q8_UNIT_BYTES);
    const q8_stream_t wsr = q8_stream(wsc, nb * Q8_TILE_ROWS * 2), usr = q8_stream(usc, nb * Q8_TILE_ROWS * 2);
    const q8_stream_t xr = q8_stream(xq, nb * Q8_UNIT_BYTES), xsr = q8_stream(xsc, nb * Q8_TILE_TOKENS * 4);
    auto load_full = [&](SiluOps &q, int b) {
        const int u0 = b * Q8_UNIT_BYTES;
        q.w0 = q8_load16(wr, lo, u0);
        q.w1 = q8_load16(wr, lo, u0 + Q8_UNIT_BYTES);
        q.u0 = q8_load16(ur, lo, u0);
        q.u1 = q8_load16(ur, lo, u0 + Q8_UNIT_BYTES);
        q.dw = __builtin_amdgcn_raw_buffer_load_b16(wsr, 2 * lane, b * Q8_TILE_ROWS * 2, 0);
        q.du = __builtin_amdgcn_raw_buffer_load_b16(usr, 2 * lane, b * Q8_TILE_ROWS * 2, 0);
        q.x0 = q8_load16(xr, lo, u0);
        q.x1 = q8_load16(xr, lo, u0 + Q8_UNIT_BYTES);
        q.sx = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xsr, 4 * lane, b * Q8_TILE_TOKENS * 4, 0));
    };
    // the odd last block of an odd nb: the absent block repeats block b with zero scales
    auto load_last = [&](SiluOps &q, int b) {
        const int u0 = b * Q8_UNIT_BYTES;
        q.w0 = q8_load16(wr, lo, u0);
        q.w1 = q.w0;
        q.u0 = q8_load16(ur, lo, u0);
        q.u1 = q.u0;
        const unsigned dwr = __builtin_amdgcn_raw_buffer_load_b16(wsr, 2 * r, b * Q8_TILE_ROWS * 2, 0);
        const unsigned dur = __builtin_amdgcn_raw_buffer_load_b16(usr, 2 * r, b * Q8_TILE_ROWS * 2, 0);
        q.dw = h ? 0u : dwr;
        q.du = h ? 0u : dur;
        q.x0 = q8_load16(xr, lo, u0);
        q.x1 = q.x0;
        const float sxr = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(xsr, 4 * r, b * Q8_TILE_TOKENS * 4, 0));
        q.sx = h ? 0.0f : sxr;
    };
    auto step = [&](const SiluOps &q, bool two) {
        {
            const f32x32 sc = __builtin_amdgcn_mfma_f32_32x32x1f32(q.sx, f16_to_f32(q.dw), fzero, 0, 0, 0);
            const i32x16 i0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(q.x0, q.w0, izero, 0, 0, 0);
            const i32x16 i1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(q.x1, q.w1, izero, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 16; i++) ag[i] = __builtin_fmaf((float)i0[i], sc[i], ag[i]);
            if (two) {
#pragma unroll
                for (int i = 0; i < 16; i++) ag[i] = __builtin_fmaf((float)i1[i], sc[16 + i], ag[i]);
            }
        }
        {
            const f32x32 sc = __builtin_amdgcn_mfma_f32_32x32x1f32(q.sx, f16_to_f32(q.du), fzero, 0, 0, 0);
            const i32x16 i0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(q.x0, q.u0, izero, 0, 0, 0);
            const i32x16 i1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(q.x1, q.u1, izero, 0, 0, 0);
#pragma unroll
            for (int i = 0; i < 16; i++) au[i] = __builtin_fmaf((float)i0[i], sc[i], au[i]);
            if (two) {
#pragma unroll
                for (int i = 0; i < 16; i++) au[i] = __builtin_fmaf((float)i1[i], sc[16 + i], au[i]);
            }
        }
    };
    if (p_begin < full_end) {
        SiluOps qa, qb;
        load_full(qa, 2 * p_begin);
        int p = p_begin;
        for (; p + 1 < full_end; p += 2) {
            load_full(qb, 2 * (p + 1));
            __builtin_amdgcn_sched_barrier(0);
            step(qa, true);
            __builtin_amdgcn_sched_barrier(0);
            load_full(qa, 2 * min(p + 2, full_end - 1));
            __builtin_amdgcn_sched_barrier(0);
            step(qb, true);
            __builtin_amdgcn_sched_barrier(0);
        }
        if (p < full_end) step(qa, true);
    }
    if (full_end < p_end) {
        SiluOps q;
        load_last(q, 2 * full_end);
        step(q, false);
    }

    if (KW > 1) {
        // reduce the K-split waves in a fixed order: kw = 0 adds 1, 2, ...
        if (kw > 0) {
            float *dg = ssm + ((size_t)((kw - 1) * 2 + 0) * 64 + lane) * 16;
            float *du = ssm + ((size_t)((kw - 1) * 2 + 1) * 64 + lane) * 16;
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                *(f32x4 *)(dg + i) = (f32x4){ag[i], ag[i + 1], ag[i + 2], ag[i + 3]};
                *(f32x4 *)(du + i) = (f32x4){au[i], au[i + 1], au[i + 2], au[i + 3]};
            }
        }
        __syncthreads();
        if (kw != 0) return;
        for (int k2 = 1; k2 < KW; k2++) {
            const float *sg = ssm + ((size_t)((k2 - 1) * 2 + 0) * 64 + lane) * 16;
            const float *su = ssm + ((size_t)((k2 - 1) * 2 + 1) * 64 + lane) * 16;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                ag[i] = ag[i] + sg[i];
                au[i] = au[i] + su[i];
            }
        }
        // every wave > 0 has returned; wave 0's reads above complete before its
        // transpose stores below (one wave's LDS operations stay in order)
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
    // v = silu(gate) * up: lane (h, r) holds feature r of tokens 8(i/4) + 4h + i%4
    float *tr = ssm;  // [32 tokens][33]
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int tok = 8 * (i >> 2) + 4 * h + (i & 3);
        tr[tok * 33 + r] = silu_f32(ag[i]) * au[i];
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_wave_barrier();
    // prepared order: lane (h, t = r) takes half h of token t's block: e[q][c] = element 8c + J[h][q]
    float e[4][4];
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int c = 0; c < 4; c++) e[q][c] = tr[r * 33 + 8 * c + perm_lane(h, q)];
    float peak = half_peak(e);
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(peak), __float_as_uint(peak), false, false);
    peak = fmaxf(peak, __uint_as_float(h ? sw[0] : sw[1]));
    const int nbo = gm.rows / Q8_BLOCK_ELEMS;  // blocks per token of the down projection's input
    quant_store(e, peak, a.oq, a.os, (size_t)tt * nbo + g, lane, h == 0, a.of16);
}

// ---------------------------------------------------------------------------
// GEMM on the f16 MFMA, n >= 2, same arithmetic as above.
//
// Q8_0 quants are integers |q| <= 127, exact in f16; two
// v_mfma_f32_32x32x16_f16 over a block's 32 elements give the int32 block dot
// exactly (every partial sum is an integer below 2^24), already as f32.  The
// 16 v_cvt_f32_i32 per output tile and block of the int8 path disappear; the
// scale products and the fma epilogue are unchanged, so the results are the
// int8 kernel's bit for bit.  Per 32 x 32 tile and block: 96 MFMA cycles (two
// f16 dots, half a scale-product MFMA) against 16 fma + the weight conversion
// on the VALU, instead of 128 VALU cycles.
//
// A workgroup is RW row-tile waves x KW K-split waves; all waves cover the
// same TPW token tiles.  Per block pair the RW waves of a K group bring the
// activations (f16 units and scales) into LDS once, and each wave its own two
// weight units and their scales, all with global_load_lds (LDS written
// without passing through registers), into a ring of Q8_GEMM_H_STAGES
// buffers: the loads for pair i + STAGES - 1 are issued while pair i is
// computed.  Every wave converts only its own weight units to f16 (once for
// its TPW token tiles).  The K groups are reduced in LDS in a fixed order, as
// in the int8 kernel.
//
// Synchronisation is explicit: the loop issues no vector-memory load other
// than these, the same number per wave per pair, so "this wave's loads of pair
// i + 1 have landed" is s_waitcnt vmcnt(N) with a constant N, followed by
// s_barrier.  (The compiler's __syncthreads, and its waits for register loads,
// would wait for every load in flight, prefetches included.)  All waves run
// the same number of iterations; pairs past a wave's range use a zero weight
// scale and add nothing (their loads are clamped to valid addresses).
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;

// s_waitcnt with vmcnt = n (0..63) and the other counters left free (gfx9 encoding)
#define Q8_VMCNT_IMM(n) ((((n)&15) | (7 << 4) | (15 << 8) | ((((n) >> 4) & 3) << 14)))

template <int TPW, int RW, bool I8 = false>
static __device__ __forceinline__ void gemm_h_body(const Q8GemmArgs &a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t hsm[];
    constexpr int UNIT = I8 ? Q8_UNIT_BYTES : Q8_UNIT_F16_BYTES;  // activation unit in LDS and HBM
    kernarg_lines<Q8GemmArgs, true>();
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int KW = (blockDim.x >> 6) / RW;
    const int rw = wave % RW;
    const int kw = wave / RW;
    int wg = blockIdx.x;
    if (a.xcd_remap) {
        const int per = a.nwg >> 3;
        wg = (wg & 7) * per + (wg >> 3);
    }
    const int rg = wg / a.tgroups;
    const int tg = wg - rg * a.tgroups;
    const int rt = rg * RW + rw;                       // global row tile (may be past the end)
    const bool row_live = rt < a.total_rtiles;
    const int rtc = min(rt, a.total_rtiles - 1);
    const int tt0 = tg * TPW;
    int mi = 0;
#pragma unroll
    for (int i = 1; i < Q8_GROUP_MAX; i++)
        if (i < a.members && rtc >= a.m[i].tile_begin) mi = i;
    const Q8GemmMember mem = a.m[mi];
    const int g = rtc - mem.tile_begin;
    const int nb = a.nb;
    const int h = lane >> 5;
    const int r = lane & 31;
    const uint8_t *wq = mem.quants + (size_t)g * nb * Q8_UNIT_BYTES + lane * 16;
    const uint16_t *wsc = mem.scales + (size_t)g * nb * Q8_TILE_ROWS;

    const int npairs = (nb + 1) >> 1;
    const int ppw = a.pairs_per_wave;
    const int p_begin = kw * ppw;
    const int p_end = min(npairs, p_begin + ppw);

    // LDS per K group: STAGES buffers of [TPW][2 blocks][2048 B f16 unit],
    // SCALE_SLOTS f32 scale slots ([TPW][2][32] used; RW > TPW waves fill the
    // rest), then per wave its two weight units and 64 f16 weight scales.
    constexpr int GLANES = RW * 64;
    constexpr int ACT_BYTES = TPW * 2 * UNIT;
    constexpr int SCALE_SLOTS = (TPW * 64 > GLANES ? TPW * 64 : GLANES);
    constexpr int W_OFF = ACT_BYTES + SCALE_SLOTS * 4;
    constexpr int W_BYTES = 2 * Q8_UNIT_BYTES + 256;
    constexpr int BUF_BYTES = W_OFF + RW * W_BYTES;
    static_assert(BUF_BYTES == Q8_GEMM_STAGED_BUF_BYTES(TPW, RW, UNIT), "host and kernel LDS layouts agree");
    constexpr int CPU_ = UNIT / 16;                      // 16-byte chunks per unit
    constexpr int MAXC = TPW * 2 * CPU_ / GLANES;        // 16-byte chunks per lane per pair
    constexpr int MAXS = (TPW * 64 + GLANES - 1) / GLANES;  // scales per lane per pair
    static_assert(TPW * 2 * CPU_ % GLANES == 0, "whole chunks per lane");
    constexpr int SG = MAXC + MAXS + 3;                  // loads per lane per pair (+ w0, w1, d_w)
    // at the end of iteration i: loads issued after pair i+1's
    constexpr int AFTER = (Q8_GEMM_H_STAGES - 2) * SG;
    uint8_t *kbase = hsm + (size_t)kw * Q8_GEMM_H_STAGES * BUF_BYTES;
    const int wig = wave - kw * RW;  // this wave within its K group
    const int wbase = wig * 64;

    // stage pair p into ring buffer `buf`: every lane issues exactly SG loads
    auto stage = [&](int p, int buf) {
        const int pc = min(p, npairs - 1);
        uint8_t *base = kbase + buf * BUF_BYTES;
        {
            // this wave's weight units (lane L's 16 bytes at 16L) and the pair's 64 f16
            // scales as dwords: lane L < 32 brings scales 2L, 2L+1 (block b0 + L/16, rows
            // 2(L%16), +1), lanes >= 32 repeat lanes L-32 into the upper, unread half
            const int b0 = 2 * pc;
            const int b1 = min(b0 + 1, nb - 1);
            const int i = lane & 31;
            const int bs = min(b0 + (i >> 4), nb - 1);
            uint8_t *wl = base + W_OFF + wig * W_BYTES;
            __builtin_amdgcn_global_load_lds(wq + (size_t)b0 * Q8_UNIT_BYTES, (lds_void_t *)wl, 16, 0, 0);
            __builtin_amdgcn_global_load_lds(wq + (size_t)b1 * Q8_UNIT_BYTES, (lds_void_t *)(wl + Q8_UNIT_BYTES), 16,
                                             0, 0);
            __builtin_amdgcn_global_load_lds(wsc + (size_t)bs * Q8_TILE_ROWS + 2 * (i & 15),
                                             (lds_void_t *)(wl + 2 * Q8_UNIT_BYTES), 4, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < MAXC; i++) {
            const int c = wbase + i * GLANES + lane;
            const int j = c / (2 * CPU_), bb = (c / CPU_) & 1;
            const int tt = min(tt0 + j, a.ttiles - 1);
            const int b = min(2 * pc + bb, nb - 1);
            __builtin_amdgcn_global_load_lds(a.xq + ((size_t)tt * nb + b) * UNIT + (c % CPU_) * 16,
                                             (lds_void_t *)(base + (wbase + i * GLANES) * 16), 16, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < MAXS; i++) {
            const int s = min(wbase + i * GLANES + lane, SCALE_SLOTS - 1);
            const int j = min(s >> 6, TPW - 1), bb = (s >> 5) & 1;
            const int tt = min(tt0 + j, a.ttiles - 1);
            const int b = min(2 * pc + bb, nb - 1);
            __builtin_amdgcn_global_load_lds(a.xs + ((size_t)tt * nb + b) * Q8_TILE_TOKENS + (s & 31),
                                             (lds_void_t *)(base + ACT_BYTES + (wbase + i * GLANES) * 4), 4, 0, 0);
        }
    };

    f32x16 acc[TPW];
#pragma unroll
    for (int t = 0; t < TPW; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[t][i] = 0.0f;
    const f32x16 fz16 = {};
    const f32x32 fz32 = {};

    // prologue: pairs 0 .. STAGES-2 staged; wait for pair 0
#pragma unroll
    for (int s = 0; s < Q8_GEMM_H_STAGES - 1; s++) stage(p_begin + s, s);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(Q8_VMCNT_IMM((Q8_GEMM_H_STAGES - 2) * SG));
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);

    for (int it = 0; it < ppw; it++) {
        const int cur = it % Q8_GEMM_H_STAGES;
        // ring slot of pair it+STAGES-1 was last read in iteration it-1 (barrier since)
        stage(p_begin + it + Q8_GEMM_H_STAGES - 1, (it + Q8_GEMM_H_STAGES - 1) % Q8_GEMM_H_STAGES);
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t *base = kbase + cur * BUF_BYTES;
        const uint8_t *wl = base + W_OFF + wig * W_BYTES;
        const i32x4 w0 = *(const i32x4 *)(wl + lane * 16);
        const i32x4 w1 = *(const i32x4 *)(wl + Q8_UNIT_BYTES + lane * 16);
        const unsigned dwb = *(const uint16_t *)(wl + 2 * Q8_UNIT_BYTES + lane * 2);
        const int p = p_begin + it;
        const bool dwv = p < p_end && 2 * p + h < nb;
        const float dwf = dwv ? f16_to_f32(dwb) : 0.0f;
        if constexpr (I8) {
            // int8 units: one v_mfma_i32_32x32x32_i8 per block, then convert + fma
            const i32x16 iz = {};
#pragma unroll
            for (int t = 0; t < TPW; t++) {
                const uint8_t *u0 = base + (t * 2) * UNIT + lane * 16;
                const i32x4 x0 = *(const i32x4 *)u0, x1 = *(const i32x4 *)(u0 + UNIT);
                const float sx = ((const float *)(base + ACT_BYTES))[t * 64 + lane];
                const f32x32 sc = __builtin_amdgcn_mfma_f32_32x32x1f32(sx, dwf, fz32, 0, 0, 0);
                const i32x16 i0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x0, w0, iz, 0, 0, 0);
                const i32x16 i1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x1, w1, iz, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 16; i++) acc[t][i] = __builtin_fmaf((float)i0[i], sc[i], acc[t][i]);
#pragma unroll
                for (int i = 0; i < 16; i++) acc[t][i] = __builtin_fmaf((float)i1[i], sc[16 + i], acc[t][i]);
            }
        } else {
            // this pair's weights to f16 (lane L: bytes 0-7 for the first MFMA, 8-15 for the second)
            const i32x4 wa0 = i8x4_to_f16x4(w0.x, w0.y), wa1 = i8x4_to_f16x4(w0.z, w0.w);
            const i32x4 wb0 = i8x4_to_f16x4(w1.x, w1.y), wb1 = i8x4_to_f16x4(w1.z, w1.w);
#pragma unroll
            for (int t = 0; t < TPW; t++) {
                const uint8_t *u0 = base + (t * 2) * UNIT + lane * 16;
                const uint8_t *u1 = u0 + UNIT;
                const i32x4 x00 = *(const i32x4 *)u0, x01 = *(const i32x4 *)(u0 + 1024);
                const i32x4 x10 = *(const i32x4 *)u1, x11 = *(const i32x4 *)(u1 + 1024);
                const float sx = ((const float *)(base + ACT_BYTES))[t * 64 + lane];
                const f32x32 sc = __builtin_amdgcn_mfma_f32_32x32x1f32(sx, dwf, fz32, 0, 0, 0);
                f32x16 d0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, x00),
                                                                   __builtin_bit_cast(f16x8, wa0), fz16, 0, 0, 0);
                d0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, x01),
                                                            __builtin_bit_cast(f16x8, wa1), d0, 0, 0, 0);
                f32x16 d1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, x10),
                                                                   __builtin_bit_cast(f16x8, wb0), fz16, 0, 0, 0);
                d1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, x11),
                                                            __builtin_bit_cast(f16x8, wb1), d1, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 16; i++) acc[t][i] = __builtin_fmaf(d0[i], sc[i], acc[t][i]);
#pragma unroll
                for (int i = 0; i < 16; i++) acc[t][i] = __builtin_fmaf(d1[i], sc[16 + i], acc[t][i]);
            }
        }
        // pair it+1 staged by every wave of the K group (and this pair's LDS reads done)
        __builtin_amdgcn_s_waitcnt(Q8_VMCNT_IMM(AFTER));
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_s_barrier();
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
    }
    // drain every prefetch (they write LDS) before the LDS is reused below
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    if (KW > 1) {
        // reduce the K groups in a fixed order (kw = 0 adds 1, 2, ...), through the staging LDS
        float *red = (float *)hsm;  // [KW-1][RW][TPW][64][16]
        if (kw > 0) {
#pragma unroll
            for (int t = 0; t < TPW; t++) {
                float *dst = red + ((size_t)(((kw - 1) * RW + rw) * TPW + t) * 64 + lane) * 16;
#pragma unroll
                for (int i = 0; i < 16; i += 4)
                    *(f32x4 *)(dst + i) = (f32x4){acc[t][i], acc[t][i + 1], acc[t][i + 2], acc[t][i + 3]};
            }
        }
        __syncthreads();
        if (kw == 0) {
            for (int k2 = 1; k2 < KW; k2++) {
#pragma unroll
                for (int t = 0; t < TPW; t++) {
                    const float *src = red + ((size_t)(((k2 - 1) * RW + rw) * TPW + t) * 64 + lane) * 16;
#pragma unroll
                    for (int i = 0; i < 16; i++) acc[t][i] = acc[t][i] + src[i];
                }
            }
        }
    }
    if (kw != 0 || !row_live) return;
    store_tiles<TPW>(a, mem, mi, acc, tt0, g * Q8_TILE_ROWS + r, h);
}

// q8_gemm_h_t<TPW>_r<RW>: up to 512 threads (RW x KW waves).
#define Q8_GEMM_H(TPW, RW)                                                                             \
    extern "C" __global__ __launch_bounds__(512) void q8_gemm_h_t##TPW##_r##RW(Q8GemmArgs a) { \
        gemm_h_body<TPW, RW>(a);                                                                       \
    }
Q8_GEMM_H(1, 4)
Q8_GEMM_H(2, 2)
Q8_GEMM_H(2, 4)

// q8_gemm_l_t<TPW>_r<RW>: the same staging with int8 activation units and the int8 MFMA.
#define Q8_GEMM_L(TPW, RW)                                                                             \
    extern "C" __global__ __launch_bounds__(512) void q8_gemm_l_t##TPW##_r##RW(Q8GemmArgs a) { \
        gemm_h_body<TPW, RW, true>(a);                                                                 \
    }
Q8_GEMM_L(1, 2)
Q8_GEMM_L(2, 2)
Q8_GEMM_L(2, 4)

// ---------------------------------------------------------------------------
// The int8 GEMM, software-pipelined.  Same arithmetic and order as gemm_body
// (SMODE 1), so the results are bit-identical; only the schedule differs.
//
// Work items are (block pair, token tile).  Each item's three MFMAs (the
// scale products and the two block dots) are issued one item ahead of the
// previous item's convert + fma epilogue, into the other of two result
// buffers, so a wave always has VALU work that does not wait on its own
// MFMAs; operand loads run two pairs ahead (ping-pong operand sets).  The
// two result buffers cost ~130 VGPRs, so these kernels run two waves per
// SIMD.  A wave rounds its pair count up to even; the extra pair, and the
// absent second block of an odd nb, get zero scales (fma(I, 0, acc) == acc:
// I is an exact integer and acc is never -0).  K-split waves reduce in LDS
// as in gemm_body; no split across workgroups.
// ---------------------------------------------------------------------------
template <int TPW>
struct PipeOps {
    i32x4 w0, w1;
    unsigned dw;
    i32x4 x0[TPW], x1[TPW];
    float sx[TPW];
};

struct PipeRes {
    f32x32 sc;
    i32x16 i0, i1;
};

template <int TPW>
static __device__ __forceinline__ void gemm_p_body(const Q8GemmArgs &a) {
    extern __shared__ __attribute__((aligned(16))) float psm[];  // [kwaves-1][twaves][TPW][64][16]
    kernarg_lines<Q8GemmArgs>();
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int TW = a.twaves;
    const int tw = wave % TW;
    const int kw = wave / TW;
    int wg = blockIdx.x;
    if (a.xcd_remap) {
        const int per = a.nwg >> 3;
        wg = (wg & 7) * per + (wg >> 3);
    }
    const int rt = wg / a.tgroups;
    const int tg = wg - rt * a.tgroups;
    const int tt0 = (tg * TW + tw) * TPW;
    const int ntl = max(0, min(TPW, a.ttiles - tt0));
    int mi = 0;
#pragma unroll
    for (int i = 1; i < Q8_GROUP_MAX; i++)
        if (i < a.members && rt >= a.m[i].tile_begin) mi = i;
    const Q8GemmMember mem = a.m[mi];
    const int g = rt - mem.tile_begin;
    const int nb = a.nb;
    const int h = lane >> 5;
    const int r = lane & 31;
    const uint8_t *wq = mem.quants + (size_t)g * nb * Q8_UNIT_BYTES;
    const uint16_t *wsc = mem.scales + (size_t)g * nb * Q8_TILE_ROWS;
    const uint8_t *xq[TPW];
    const float *xsc[TPW];
#pragma unroll
    for (int t = 0; t < TPW; t++) {
        const int ttc = min(tt0 + t, a.ttiles - 1);
        xq[t] = a.xq + (size_t)ttc * nb * Q8_UNIT_BYTES;
        xsc[t] = a.xs + (size_t)ttc * nb * Q8_TILE_TOKENS;
    }
    const int lo = lane * 16;
    const int npairs = (nb + 1) >> 1;
    const int p_begin = kw * a.pairs_per_wave;
    const int p_end = ntl > 0 ? min(npairs, p_begin + a.pairs_per_wave) : p_begin;
    const int nsteps = (max(p_end - p_begin, 0) + 1) & ~1;  // even: pairs come in (A, B) couples

    f32x16 acc[TPW];
#pragma unroll
    for (int t = 0; t < TPW; t++)
#pragma unroll
        for (int i = 0; i < 16; i++) acc[t][i] = 0.0f;
    const i32x16 izero = {};
    const f32x32 fzero = {};

    // operands of pair p at clamped, valid addresses; validity is applied when issued
    auto load = [&](PipeOps<TPW> &q, int p) {
        const int pc = min(p, npairs - 1);
        const int b0 = 2 * pc;
        const int b1 = min(b0 + 1, nb - 1);
        const int bs = min(b0 + h, nb - 1);
        q.w0 = *(const i32x4 *)(wq + (size_t)b0 * Q8_UNIT_BYTES + lo);
        q.w1 = *(const i32x4 *)(wq + (size_t)b1 * Q8_UNIT_BYTES + lo);
        q.dw = wsc[(size_t)bs * Q8_TILE_ROWS + r];
#pragma unroll
        for (int t = 0; t < TPW; t++) {
            q.x0[t] = *(const i32x4 *)(xq[t] + (size_t)b0 * Q8_UNIT_BYTES + lo);
            q.x1[t] = *(const i32x4 *)(xq[t] + (size_t)b1 * Q8_UNIT_BYTES + lo);
            q.sx[t] = xsc[t][(size_t)bs * Q8_TILE_TOKENS + r];
        }
    };
    // the three MFMAs of item (pair p, tile t); lanes 0-31 carry block 2p, 32-63 block 2p+1
    auto issue = [&](const PipeOps<TPW> &q, int t, int p, PipeRes &res) {
        const bool v = p < p_end && 2 * min(p, npairs - 1) + h < nb;
        const float dwf = v ? f16_to_f32(q.dw) : 0.0f;
        const float sx = v ? q.sx[t] : 0.0f;
        res.sc = __builtin_amdgcn_mfma_f32_32x32x1f32(sx, dwf, fzero, 0, 0, 0);
        res.i0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(q.x0[t], q.w0, izero, 0, 0, 0);
        res.i1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(q.x1[t], q.w1, izero, 0, 0, 0);
    };
    auto epi = [&](const PipeRes &res, int t) {
#pragma unroll
        for (int i = 0; i < 16; i++) acc[t][i] = __builtin_fmaf((float)res.i0[i], res.sc[i], acc[t][i]);
#pragma unroll
        for (int i = 0; i < 16; i++) acc[t][i] = __builtin_fmaf((float)res.i1[i], res.sc[16 + i], acc[t][i]);
    };

    if (nsteps > 0) {
        PipeOps<TPW> qa, qb;
        PipeRes r0, r1;
        load(qa, p_begin);
        load(qb, p_begin + 1);
        if constexpr (TPW == 1) {
            // items = pairs; pair p in (qa, r0), pair p + 1 in (qb, r1)
            for (int s = 0; s < nsteps; s += 2) {
                const int p = p_begin + s;
                issue(qa, 0, p, r0);
                __builtin_amdgcn_sched_barrier(0);
                if (s > 0) epi(r1, 0);  // pair p - 1
                __builtin_amdgcn_sched_barrier(0);
                load(qa, p + 2);
                __builtin_amdgcn_sched_barrier(0);
                issue(qb, 0, p + 1, r1);
                __builtin_amdgcn_sched_barrier(0);
                epi(r0, 0);  // pair p
                __builtin_amdgcn_sched_barrier(0);
                load(qb, p + 3);
                __builtin_amdgcn_sched_barrier(0);
            }
            epi(r1, 0);
        } else {
            // items (p, 0), (p, 1), (p + 1, 0), (p + 1, 1): results alternate r0 / r1
            for (int s = 0; s < nsteps; s += 2) {
                const int p = p_begin + s;
                issue(qa, 0, p, r0);
                __builtin_amdgcn_sched_barrier(0);
                if (s > 0) epi(r1, 1);  // (p - 1, 1)
                __builtin_amdgcn_sched_barrier(0);
                issue(qa, 1, p, r1);
                __builtin_amdgcn_sched_barrier(0);
                load(qa, p + 2);
                __builtin_amdgcn_sched_barrier(0);
                epi(r0, 0);  // (p, 0)
                __builtin_amdgcn_sched_barrier(0);
                issue(qb, 0, p + 1, r0);
                __builtin_amdgcn_sched_barrier(0);
                epi(r1, 1);  // (p, 1)
                __builtin_amdgcn_sched_barrier(0);
                issue(qb, 1, p + 1, r1);
                __builtin_amdgcn_sched_barrier(0);
                load(qb, p + 3);
                __builtin_amdgcn_sched_barrier(0);
                epi(r0, 0);  // (p + 1, 0)
                __builtin_amdgcn_sched_barrier(0);
            }
            epi(r1, 1);
        }
    }

    const int KW = (blockDim.x >> 6) / TW;
    if (KW > 1) {
        if (kw > 0) {
#pragma unroll
            for (int t = 0; t < TPW; t++) {
                float *dst = psm + ((size_t)(((kw - 1) * TW + tw) * TPW + t) * 64 + lane) * 16;
#pragma unroll
                for (int i = 0; i < 16; i += 4)
                    *(f32x4 *)(dst + i) = (f32x4){acc[t][i], acc[t][i + 1], acc[t][i + 2], acc[t][i + 3]};
            }
        }
        __syncthreads();
        if (kw == 0) {
            for (int k2 = 1; k2 < KW; k2++) {
#pragma unroll
                for (int t = 0; t < TPW; t++) {
                    const float *src = psm + ((size_t)(((k2 - 1) * TW + tw) * TPW + t) * 64 + lane) * 16;
#pragma unroll
                    for (int i = 0; i < 16; i++) acc[t][i] = acc[t][i] + src[i];
                }
            }
        }
    }
    if (kw != 0) return;
    store_tiles<TPW>(a, mem, mi, acc, tt0, g * Q8_TILE_ROWS + r, h);
}

extern "C" __global__ __launch_bounds__(512) void q8_gemm_p_t1(Q8GemmArgs a) { gemm_p_body<1>(a); }
extern "C" __global__ __launch_bounds__(512) void q8_gemm_p_t2(Q8GemmArgs a) { gemm_p_body<2>(a); }

extern "C" __global__ __launch_bounds__(1024) void q8_gemm_s0_t1(Q8GemmArgs a) { gemm_body<0, 1>(a); }
extern "C" __global__ __launch_bounds__(1024) void q8_gemm_s1_t1(Q8GemmArgs a) { gemm_body<1, 1>(a); }
extern "C" __global__ __launch_bounds__(1024) void q8_gemm_s1_t1s(Q8GemmArgs a) { gemm_body<1, 1, true>(a); }
extern "C" __global__ __launch_bounds__(512) void q8_gemm_s1_t2(Q8GemmArgs a) { gemm_body<1, 2>(a); }
extern "C" __global__ __launch_bounds__(512) void q8_gemm_s1_t4(Q8GemmArgs a) { gemm_body<1, 4>(a); }

// ---------------------------------------------------------------------------
// Greedy argmax (sampler.rs:167-175): the first index whose value is strictly
// greater than all before it.  NaN never wins a comparison, so a NaN at index 0
// pins the answer to 0 and a NaN elsewhere is skipped; the two-stage
// reduction below keeps exactly that rule: best = (value, lowest index) over
// the non-NaN values, then index 0 if values[0] is NaN.
// ---------------------------------------------------------------------------

extern "C" __global__ __launch_bounds__(256) void q8_argmax(Q8ArgmaxArgs a) {
    __shared__ float sv[256];
    __shared__ unsigned si[256];
    float bv = 0.0f;
    unsigned bi = 0xffffffffu;
    if (a.stage == 0) {
        const long long chunk = (a.len + a.parts - 1) / a.parts;
        const long long begin = (long long)blockIdx.x * chunk;
        const long long end = min(a.len, begin + chunk);
        for (long long i = begin + threadIdx.x; i < end; i += blockDim.x) {
            const float v = a.values[i];
            if (v == v && better(v, (unsigned)i, bv, bi)) {
                bv = v;
                bi = (unsigned)i;
            }
        }
    } else {
        // eight candidates a thread per round, all loaded before any is
        // compared (the order does not matter: `better` is a total order)
        for (int i0 = threadIdx.x; i0 < a.parts; i0 += 8 * (int)blockDim.x) {
            float v[8];
            unsigned ix[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int i = i0 + u * (int)blockDim.x;
                v[u] = i < a.parts ? a.part_value[i] : 0.0f;
                ix[u] = i < a.parts ? a.part_index[i] : 0xffffffffu;
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                if (better(v[u], ix[u], bv, bi)) {
                    bv = v[u];
                    bi = ix[u];
                }
            }
        }
    }
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) {
            const float ov = sv[threadIdx.x + s];
            const unsigned oi = si[threadIdx.x + s];
            if (better(ov, oi, sv[threadIdx.x], si[threadIdx.x])) {
                sv[threadIdx.x] = ov;
                si[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        if (a.stage == 0) {
            a.part_value[blockIdx.x] = sv[0];
            a.part_index[blockIdx.x] = si[0];
        } else {
            const float first = a.values[0];
            const unsigned best = si[0];
            a.result[0] = (first != first || best == 0xffffffffu) ? 0u : best;
        }
    }
}

// Device-to-device copy of `bytes` (a multiple of 16) with dwordx4 loads and
// stores: the counterpart of the reference's copy_f32 (gpu.cu:422-435), and the
// plain streaming kernel of known size that the HBM traffic counters are
// calibrated against.
extern "C" __global__ __launch_bounds__(256) void q8_copy(Q8CopyArgs a) {
    const long long n16 = a.bytes >> 4;
    const long long stride = (long long)a.blocks * blockDim.x;
    const i32x4 *src = (const i32x4 *)a.src;
    i32x4 *dst = (i32x4 *)a.dst;
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

// ---------------------------------------------------------------------------
// Embedding rows out of the resident tile layout (gpu.cu embedding_rows
// 1754-1766; dequant_q8_0, quant.rs:184-203): out[t][32b + e] = d * q, one f32
// product, as the reference computes it.
//
// One thread per (token, block, half h): its 16-byte lane segment of the unit
// holds, in dword j, elements 8c + Q8_J[h][j] for bytes c = 0..3.  Dwords 0
// and 2 carry AVX2 lanes 2h and 2h+1, dwords 1 and 3 lanes 4+2h and 5+2h, so
// each chunk c yields two adjacent f32 pairs.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void q8_embed(Q8EmbedArgs a) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;  // < 2^31: the host checks
    const int per_token = a.nb * 2;
    if (idx >= a.n * per_token) return;
    const int t = idx / per_token;
    const int rem = idx - t * per_token;
    const int b = rem >> 1;
    const int h = rem & 1;
    unsigned row = a.tokens[t];
    const bool valid = row < (unsigned)a.rows;  // ids from device memory are not host-checked
    row = valid ? row : 0u;
    const size_t unit = (size_t)(row / Q8_TILE_ROWS) * a.nb + b;
    const unsigned r = row % Q8_TILE_ROWS;
    i32x4 q = *(const i32x4 *)(a.quants + unit * Q8_UNIT_BYTES + 16 * (32 * h + r));
    const float d = valid ? f16_to_f32(a.scales[unit * Q8_TILE_ROWS + r]) : 0.0f;
    if (!valid) q = i32x4{0, 0, 0, 0};
    float *o = a.out + (size_t)t * a.nb * Q8_BLOCK_ELEMS + b * Q8_BLOCK_ELEMS + 2 * h;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const float2 lo = {d * (float)(signed char)(q[0] >> (8 * c)), d * (float)(signed char)(q[2] >> (8 * c))};
        const float2 hi = {d * (float)(signed char)(q[1] >> (8 * c)), d * (float)(signed char)(q[3] >> (8 * c))};
        *(float2 *)(o + 8 * c) = lo;
        *(float2 *)(o + 8 * c + 4) = hi;
    }
}

// ---------------------------------------------------------------------------
// RMSNorm (ops.rs:5-30), as f32 rows and/or straight into prepared Q8_0
// activations (compute.rs:959-984 norm_prepare; gpu.cu rmsnorm_quantize_rows
// 351-407) for rows longer than the 256-thread row kernel below takes.  One
// wave per token row, four rows per workgroup.
//
// The row's squares are taken in f32 and summed in f64 (ggml's choice, kept
// by the reference), here as per-lane partial sums reduced across the wave;
// the reference adds them left to right.  Both are f64 sums of the same f32
// terms, within n * 2^-53 of each other, so the f32 mean square they round to
// differs only when the exact value lies that close to an f32 rounding
// boundary.  Then scale = 1 / sqrt(mean_square + eps) in f32 (correctly
// rounded sqrt and division) and each value is (x * scale) * w.
//
// Quantization: lane L handles half L%2 of blocks L/2, L/2 + 32, ...; the
// block peak meets its partner half through one xor-1 shuffle.  Rows from n
// up to the token-tile boundary are written as zeros.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void q8_rmsnorm(Q8NormArgs a) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (t >= a.rows_launched) return;  // whole waves
    const int k = a.k;
    const bool live = t < a.n;
    const float *xr = a.x + (size_t)min(t, a.n - 1) * k;
    double ss = 0.0;
    for (int i = lane * 4; i < k; i += 256) {
        const float v0 = xr[i], v1 = xr[i + 1], v2 = xr[i + 2], v3 = xr[i + 3];
        ss += (double)(v0 * v0);
        ss += (double)(v1 * v1);
        ss += (double)(v2 * v2);
        ss += (double)(v3 * v3);
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    const float mean_square = (float)(ss / (double)k);
    const float scale = 1.0f / sqrtf(mean_square + a.eps);

    if (a.out && live) {
        float *orow = a.out + (size_t)t * k;
        for (int i = lane * 4; i < k; i += 256) {
#pragma unroll
            for (int j = 0; j < 4; j++) orow[i + j] = (xr[i + j] * scale) * a.w[i + j];
        }
    }
    if (a.xq) {
        const int nb = k / 32;
        const int h = lane & 1;
        const int tt = t >> 5;
        for (int b0 = 0; b0 < nb; b0 += 32) {
            const int b = min(b0 + (lane >> 1), nb - 1);  // clamped: every lane joins the shuffle
            const size_t base = (size_t)b * 32 + 2 * h;
            float e[4][4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                // chunk c: elements 8c + 2h, +1 (dwords 0, 2) and 8c + 4 + 2h, +1 (dwords 1, 3)
                const size_t i0 = base + 8 * c, i1 = base + 8 * c + 4;
                const float x00 = (xr[i0] * scale) * a.w[i0], x01 = (xr[i0 + 1] * scale) * a.w[i0 + 1];
                const float x10 = (xr[i1] * scale) * a.w[i1], x11 = (xr[i1 + 1] * scale) * a.w[i1 + 1];
                e[0][c] = live ? x00 : 0.0f;  // J[h][0] = 2h
                e[2][c] = live ? x01 : 0.0f;  // J[h][2] = 2h + 1
                e[1][c] = live ? x10 : 0.0f;  // J[h][1] = 4 + 2h
                e[3][c] = live ? x11 : 0.0f;  // J[h][3] = 5 + 2h
            }
            float peak = half_peak(e);
            peak = fmaxf(peak, __shfl_xor(peak, 1));
            if (b0 + (lane >> 1) < nb)
                quant_store(e, peak, a.xq, a.xs, (size_t)tt * nb + b, 32 * h + (t & 31), h == 0, a.f16);
        }
    }
}

// RMSNorm with a 256-thread workgroup per row (k <= 256 * 4 * Q8_NORM_ROW_VEC;
// the decode step's norms, and norm_prepare's rows).  Each thread loads its
// float4s of x (and w) once, up front, adds its squares in f64, the waves meet
// in LDS in a fixed order, and the row is scaled from registers: one memory
// round trip where the wave-per-row kernel above makes one per 256 elements.
// The f64 sum is the same set of f32 terms as there, in another order.  The
// prepared Q8_0 output uses that kernel's per-half-block element layout and
// quantizer; rows from n up to the token-tile boundary are written as zeros.
// Prepared output: the normalized row goes through LDS once ([block][36]
// floats: the pad keeps the half-block reads at most two-way bank-conflicted)
// so each thread takes its half-block in the quantizer's element order from
// there; the row's x and w are read from memory only as the float4s of the
// sum of squares.  The values are the same products (x * scale) * w as the
// f32 output, so the prepared bytes are the f32 row's quantization.
extern "C" __global__ __launch_bounds__(256) void q8_rmsnorm_row(Q8NormArgs a) {
    __shared__ double part[4];
    extern __shared__ __attribute__((aligned(16))) float nrow[];  // [nb][Q8_NORM_LDS_PITCH], prepared output only
    const int tid = threadIdx.x;
    // Prepared output: the eight rows whose 16-byte slots share a 128-byte
    // line of a unit (tokens 8m .. 8m + 7) go to workgroups 8 apart, which
    // round-robin dispatch places on one XCD, so each line is written from
    // one L2; the grid is then a multiple of 64 rows and rows past the
    // token-tile boundary return.
    int t = blockIdx.x;
    if (a.xq) {
        const int q = t >> 3;
        t = 8 * (8 * (q >> 3) + (t & 7)) + (q & 7);
        if (t >= a.rows_launched) return;  // whole workgroup, before any barrier
    }
    const int k = a.k;
    const int nv = k >> 2;
    const bool live = t < a.n;  // rows from n to the token-tile boundary quantize as zeros
    const float *xrow = a.x + (size_t)min(t, a.n - 1) * k;
    const f32x4 *xr = (const f32x4 *)xrow;
    const f32x4 *wr = (const f32x4 *)a.w;
    const bool need_w = a.out != nullptr || a.xq != nullptr;
    f32x4 xv[Q8_NORM_ROW_VEC], wv[Q8_NORM_ROW_VEC];
#pragma unroll
    for (int j = 0; j < Q8_NORM_ROW_VEC; j++) {
        xv[j] = (f32x4){0.0f, 0.0f, 0.0f, 0.0f};
        wv[j] = xv[j];
        if (256 * j < nv) {  // workgroup-uniform
            const int i = tid + 256 * j;
            const int ic = min(i, nv - 1);  // clamped in-bounds address; the value is unused past nv
            xv[j] = xr[ic];
            if (need_w) wv[j] = wr[ic];
        }
    }
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < Q8_NORM_ROW_VEC; j++) {
        if (tid + 256 * j < nv) {
#pragma unroll
            for (int e = 0; e < 4; e++) ss += (double)(xv[j][e] * xv[j][e]);
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
    if ((tid & 63) == 0) part[tid >> 6] = ss;
    __syncthreads();
    const double total = (part[0] + part[1]) + (part[2] + part[3]);
    const float mean_square = (float)(total / (double)k);
    const float scale = 1.0f / sqrtf(mean_square + a.eps);
    if (a.out && live) {
        f32x4 *orow = (f32x4 *)(a.out + (size_t)t * k);
#pragma unroll
        for (int j = 0; j < Q8_NORM_ROW_VEC; j++) {
            const int i = tid + 256 * j;
            if (i < nv) {
                f32x4 o;
#pragma unroll
                for (int e = 0; e < 4; e++) o[e] = (xv[j][e] * scale) * wv[j][e];
                orow[i] = o;
            }
        }
    }
    if (a.xq) {
        const int nb = k / 32;
#pragma unroll
        for (int j = 0; j < Q8_NORM_ROW_VEC; j++) {
            const int i = tid + 256 * j;
            if (i < nv) {
                f32x4 o;
#pragma unroll
                for (int e = 0; e < 4; e++) o[e] = live ? (xv[j][e] * scale) * wv[j][e] : 0.0f;
                *(f32x4 *)(nrow + (i >> 3) * Q8_NORM_LDS_PITCH + 4 * (i & 7)) = o;
            }
        }
        __syncthreads();
        // thread tid takes half tid % 2 of blocks tid / 2 + 128 g (the
        // quantizer's element layout per half-block)
        const int tt = t >> 5;
        const int h = tid & 1;
#pragma unroll
        for (int g = 0; g < 2; g++) {
            if (128 * g >= nb) break;  // workgroup-uniform
            const int b = min(128 * g + (tid >> 1), nb - 1);  // clamped: every lane joins the shuffle
            const float *src = nrow + b * Q8_NORM_LDS_PITCH + 2 * h;
            float e[4][4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float2 lo = *(const float2 *)(src + 8 * c);      // elements 8c + 2h, +1
                const float2 hi = *(const float2 *)(src + 8 * c + 4);  // elements 8c + 4 + 2h, +1
                e[0][c] = lo.x;  // J[h][0] = 2h
                e[2][c] = lo.y;  // J[h][2] = 2h + 1
                e[1][c] = hi.x;  // J[h][1] = 4 + 2h
                e[3][c] = hi.y;  // J[h][3] = 5 + 2h
            }
            float peak = half_peak(e);
            peak = fmaxf(peak, __shfl_xor(peak, 1));
            if (128 * g + (tid >> 1) < nb)
                quant_store(e, peak, a.xq, a.xs, (size_t)tt * nb + b, 32 * h + (t & 31), h == 0, a.f16);
        }
    }
}

extern "C" __global__ __launch_bounds__(256) void q8_silu_mul(Q8EltArgs a) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < a.len) a.act[i] = silu_f32(a.gate[i]) * a.up[i];
}

#include "q8_attn.hip"
