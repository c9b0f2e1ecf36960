// q8_probe.hip -- the benchmark's measurement kernels (libq8bench.so,
// include/q8bench.h): the ceilings the benchmark quotes the hot-path kernels
// against.  No counterpart in the reference, and not part of the product
// code object: built by llm_amd/build.py into a code object of its own.
//
//   q8_probe_read_l{2,4,8,16}[_nt]  a plain streaming read of `bytes`: L
//                            16-byte loads per lane all issued before any is
//                            used, one pass; default or non-temporal policy
//                            (the GEMV's weight loads are non-temporal), any
//                            workgroup size (the launcher passes the GEMV's);
//   q8_probe_empty           a kernel that does nothing (per-launch cost);
//   q8_probe_mfma            int8 MFMA only: 4 independent accumulator chains
//                            of v_mfma_i32_32x32x32_i8 per wave;
//   q8_probe_valu            VALU only: the per-block scale arithmetic of the
//                            GEMM (16 v_cvt_f32_i32 + 16 v_fmac_f32 per lane);
//   q8_probe_mix             the GEMM's per-tile-block mix with operands in
//                            registers: one int8 MFMA, half an outer-product
//                            scale MFMA (v_mfma_f32_32x32x1_2b_f32 per block
//                            pair) and the 32 VALU of the block scale, with
//                            the next pair's MFMAs issued before this pair's
//                            VALU (what overlap one wave can get);
//   q8_probe_mix_f16         the same tile-blocks for the f16-MFMA family:
//                            two v_mfma_f32_32x32x16_f16 per block (the exact
//                            integer dot, already f32), half a scale-product
//                            MFMA and 16 fma (no converts);
//   q8_probe_split_*         two roles on the same SIMDs: in an 8-wave
//                            workgroup waves w and w + 4 share a SIMD (the
//                            dispatcher gives the waves of a workgroup to the
//                            four SIMDs in turn), so waves 0-3 run role A and
//                            waves 4-7 role B on every SIMD at once; `mask`
//                            switches each role on or off, so the time of A
//                            alone, B alone and both is measured at the same
//                            launch shape: both = the larger of the two when
//                            their pipes overlap, their sum when they share one.
// Results feed `sink` only when equal to `never` (the host passes a value no
// result takes), so no work is dead and nothing is written.
#include <hip/hip_runtime.h>

#include "q8_bench_args.h"

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x32 __attribute__((ext_vector_type(32)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// The read probes take their arguments as scalars, preloaded into SGPRs at
// wave launch (the code object is built with kernarg preload), and the
// workgroup size as an argument rather than from the dispatch packet: a wave
// issues its loads without a scalar-cache miss first, as the row-slice GEMVs
// they are the ceiling of do.
template <int L, bool NT>
static __device__ __forceinline__ void probe_read(const uint8_t *src, long long bytes, int threads, unsigned never,
                                                  unsigned *sink) {
    const long long base = (long long)blockIdx.x * threads * 16 * L + threadIdx.x * 16;
    i32x4 v[L];
#pragma unroll
    for (int i = 0; i < L; i++) {
        const long long off = min(base + (long long)i * threads * 16, bytes - 16);
        const i32x4 *p = (const i32x4 *)(src + off);
        v[i] = NT ? __builtin_nontemporal_load(p) : *p;
    }
    unsigned acc = 0;
#pragma unroll
    for (int i = 0; i < L; i++) acc ^= (unsigned)(v[i].x ^ v[i].y ^ v[i].z ^ v[i].w);
    if (acc == never) sink[0] = acc;
}

#define Q8_PROBE_READ_PARAMS const uint8_t *src, long long bytes, int threads, unsigned never, unsigned *sink
#define Q8_PROBE_READ(L)                                                                                    \
    extern "C" __global__ __launch_bounds__(1024) void q8_probe_read_l##L(Q8_PROBE_READ_PARAMS) {         \
        probe_read<L, false>(src, bytes, threads, never, sink);                                            \
    }                                                                                                      \
    extern "C" __global__ __launch_bounds__(1024) void q8_probe_read_l##L##_nt(Q8_PROBE_READ_PARAMS) {    \
        probe_read<L, true>(src, bytes, threads, never, sink);                                             \
    }
Q8_PROBE_READ(2)
Q8_PROBE_READ(4)
Q8_PROBE_READ(8)
Q8_PROBE_READ(16)

extern "C" __global__ __launch_bounds__(64) void q8_probe_empty(Q8ProbeArgs a) {
    if (threadIdx.x == 1024) a.sink[0] = a.never;
}

extern "C" __global__ __launch_bounds__(256) void q8_probe_mfma(Q8ProbeArgs a) {
    const int lane = threadIdx.x & 63;
    const i32x4 x = {lane, lane + 1, lane + 2, lane + 3};
    const i32x4 w = {3 * lane, lane ^ 5, lane * 7, 11};
    i32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int it = 0; it < a.iters; it++) {
        c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, w, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(w, x, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, x, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(w, w, c3, 0, 0, 0);
    }
    unsigned acc = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) acc ^= (unsigned)(c0[i] + c1[i] + c2[i] + c3[i]);
    if (acc == a.never) a.sink[0] = acc;
}

extern "C" __global__ __launch_bounds__(256) void q8_probe_valu(Q8ProbeArgs a) {
    const int lane = threadIdx.x & 63;
    i32x16 iv;
    f32x16 sc, acc = {};
#pragma unroll
    for (int i = 0; i < 16; i++) {
        iv[i] = lane * 37 + i;
        sc[i] = 1e-3f * (float)(i + 1);
    }
    for (int it = 0; it < a.iters; it++) {
        // an empty asm that "changes" the integers keeps the conversions in
        // the loop without adding instructions
        asm volatile("" : "+v"(iv));
#pragma unroll
        for (int i = 0; i < 16; i++) acc[i] = __builtin_fmaf((float)iv[i], sc[i], acc[i]);
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) s += acc[i];
    if (__float_as_uint(s) == a.never) a.sink[0] = 1u;
}

// One block pair's VALU (the 32 cvt + 32 fma of two tile-blocks) on (ia, ib,
// sc) while the next pair's three MFMAs run into (na, nb, nsc); the schedule
// groups interleave them MFMA, 21 VALU, MFMA, 21 VALU, MFMA, 22 VALU so the
// wave issues VALU while its own MFMAs execute.
#define Q8_PROBE_PAIR(ia, ib, sc, na, nb, nsc)                                                  \
    do {                                                                                       \
        asm volatile("" : "+v"(x0), "+v"(x1), "+v"(w0), "+v"(w1), "+v"(sx));                  \
        na = __builtin_amdgcn_mfma_i32_32x32x32_i8(x0, w0, izero, 0, 0, 0);                   \
        nb = __builtin_amdgcn_mfma_i32_32x32x32_i8(x1, w1, izero, 0, 0, 0);                   \
        nsc = __builtin_amdgcn_mfma_f32_32x32x1f32(sx, dw, fzero, 0, 0, 0);                   \
        _Pragma("unroll") for (int i = 0; i < 16; i++) acc[i] = __builtin_fmaf((float)ia[i], sc[i], acc[i]); \
        _Pragma("unroll") for (int i = 0; i < 16; i++) acc[i] = __builtin_fmaf((float)ib[i], sc[16 + i], acc[i]); \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                     \
        __builtin_amdgcn_sched_group_barrier(0x002, 21, 0);                                    \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                     \
        __builtin_amdgcn_sched_group_barrier(0x002, 21, 0);                                    \
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                     \
        __builtin_amdgcn_sched_group_barrier(0x002, 22, 0);                                    \
    } while (0)

extern "C" __global__ __launch_bounds__(256) void q8_probe_mix(Q8ProbeArgs a) {
    const int lane = threadIdx.x & 63;
    i32x4 x0 = {lane, lane + 1, lane + 2, lane + 3}, x1 = {lane ^ 9, 5, lane, 7};
    i32x4 w0 = {3 * lane, lane ^ 5, lane * 7, 11}, w1 = {lane, 2 * lane, 13, lane ^ 3};
    float sx = 1e-3f * (float)(lane + 1);
    const float dw = 2e-3f * (float)(64 - lane);
    const i32x16 izero = {};
    const f32x32 fzero = {};
    f32x16 acc = {};
    i32x16 i0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x0, w0, izero, 0, 0, 0);
    i32x16 i1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x1, w1, izero, 0, 0, 0);
    f32x32 sc = __builtin_amdgcn_mfma_f32_32x32x1f32(sx, dw, fzero, 0, 0, 0);
    i32x16 j0, j1;
    f32x32 tc;
    for (int it = 0; it < a.iters; it += 2) {
        Q8_PROBE_PAIR(i0, i1, sc, j0, j1, tc);
        Q8_PROBE_PAIR(j0, j1, tc, i0, i1, sc);
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) s += acc[i];
    if (__float_as_uint(s) == a.never) a.sink[0] = 1u;
}

// The f16-MFMA family's tile-block: the block dot as two K = 16 f16 MFMAs
// (quants are exact in f16) straight into f32, then acc += dot * (d_w s_x)
// from the outer-product MFMA; same software pipeline as q8_probe_mix.
#define Q8_PROBE_F16_DOT(xa, xb, wa, wb)                                                                   \
    __builtin_amdgcn_mfma_f32_32x32x16_f16(                                                              \
        __builtin_bit_cast(f16x8, xb), __builtin_bit_cast(f16x8, wb),                                    \
        __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, xa), __builtin_bit_cast(f16x8, wa), \
                                               f16zero, 0, 0, 0),                                        \
        0, 0, 0)
#define Q8_PROBE_F16_PAIR(ca, cb, sc, na, nb, nsc)                                                       \
    do {                                                                                                 \
        asm volatile("" : "+v"(hx0), "+v"(hx1), "+v"(hy0), "+v"(hy1), "+v"(hw0), "+v"(hw1), "+v"(hv0), "+v"(hv1)); \
        asm volatile("" : "+v"(sx));                                                                     \
        na = Q8_PROBE_F16_DOT(hx0, hx1, hw0, hw1);                                                       \
        nb = Q8_PROBE_F16_DOT(hy0, hy1, hv0, hv1);                                                       \
        nsc = __builtin_amdgcn_mfma_f32_32x32x1f32(sx, dw, fzero, 0, 0, 0);                              \
        _Pragma("unroll") for (int i = 0; i < 16; i++) acc[i] = __builtin_fmaf(ca[i], sc[i], acc[i]);    \
        _Pragma("unroll") for (int i = 0; i < 16; i++) acc[i] = __builtin_fmaf(cb[i], sc[16 + i], acc[i]); \
    } while (0)

extern "C" __global__ __launch_bounds__(256) void q8_probe_mix_f16(Q8ProbeArgs a) {
    const int lane = threadIdx.x & 63;
    // small integers as f16 bit patterns (exact), as the f16 prepared units hold
    i32x4 hx0, hx1, hy0, hy1, hw0, hw1, hv0, hv1;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const unsigned e = 0x3c00u + (unsigned)((lane + i) & 7) * 0x40u;  // 1.0 .. 1.4375
        hx0[i] = (int)(e | (e << 16)); hx1[i] = (int)((e + 0x10u) | (e << 16));
        hy0[i] = (int)(e ^ 0x8000u); hy1[i] = (int)(e | 0x80000000u);
        hw0[i] = (int)(e + 0x20u); hw1[i] = (int)(e << 16); hv0[i] = (int)e; hv1[i] = (int)(e | (e << 16));
    }
    float sx = 1e-3f * (float)(lane + 1);
    const float dw = 2e-3f * (float)(64 - lane);
    const f32x16 f16zero = {};
    const f32x32 fzero = {};
    f32x16 acc = {};
    f32x16 d0 = Q8_PROBE_F16_DOT(hx0, hx1, hw0, hw1), d1 = Q8_PROBE_F16_DOT(hy0, hy1, hv0, hv1);
    f32x32 sc = __builtin_amdgcn_mfma_f32_32x32x1f32(sx, dw, fzero, 0, 0, 0);
    f32x16 e0, e1;
    f32x32 tc;
    for (int it = 0; it < a.iters; it += 2) {
        Q8_PROBE_F16_PAIR(d0, d1, sc, e0, e1, tc);
        Q8_PROBE_F16_PAIR(e0, e1, tc, d0, d1, sc);
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) s += acc[i];
    if (__float_as_uint(s) == a.never) a.sink[0] = 1u;
}


// ---- co-resident roles (q8_probe_split_*) ----
// A: int8 MFMA, four independent chains (4 MFMAs a trip)
static __device__ __forceinline__ void role_i8(const Q8ProbeArgs &a) {
    const int lane = threadIdx.x & 63;
    const i32x4 x = {lane, lane + 1, lane + 2, lane + 3};
    const i32x4 w = {3 * lane, lane ^ 5, lane * 7, 11};
    i32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int it = 0; it < a.iters; it++) {
        c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, w, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(w, x, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(x, x, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(w, w, c3, 0, 0, 0);
    }
    unsigned acc = 0;
#pragma unroll
    for (int i = 0; i < 16; i++) acc ^= (unsigned)(c0[i] + c1[i] + c2[i] + c3[i]);
    if (acc == a.never) a.sink[0] = acc;
}
// A: f32 outer-product scale MFMA, two chains (2 MFMAs a trip: four tile-blocks' scale products)
static __device__ __forceinline__ void role_f32(const Q8ProbeArgs &a) {
    const int lane = threadIdx.x & 63;
    const float sx = 1e-3f * (float)(lane + 1), dw = 2e-3f * (float)(64 - lane);
    f32x32 c0 = {}, c1 = {};
    for (int it = 0; it < a.iters; it++) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x1f32(sx, dw, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x1f32(dw, sx, c1, 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; i++) s += c0[i] + c1[i];
    if (__float_as_uint(s) == a.never) a.sink[0] = 1u;
}
// B: the block-scale VALU (CVT = 1: 16 cvt + 16 fma a trip; CVT = 0: 32 fma a trip)
template <int CVT>
static __device__ __forceinline__ void role_valu(const Q8ProbeArgs &a) {
    const int lane = threadIdx.x & 63;
    i32x16 iv;
    f32x16 sc, acc = {}, acc2 = {};
#pragma unroll
    for (int i = 0; i < 16; i++) {
        iv[i] = lane * 37 + i;
        sc[i] = 1e-3f * (float)(i + 1);
    }
    for (int it = 0; it < a.iters; it++) {
        asm volatile("" : "+v"(iv), "+v"(sc));
        if (CVT) {
#pragma unroll
            for (int i = 0; i < 16; i++) acc[i] = __builtin_fmaf((float)iv[i], sc[i], acc[i]);
        } else {
#pragma unroll
            for (int i = 0; i < 16; i++) {
                acc[i] = __builtin_fmaf(sc[i], sc[i], acc[i]);
                acc2[i] = __builtin_fmaf(acc[i], sc[i], acc2[i]);
            }
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) s += acc[i] + acc2[i];
    if (__float_as_uint(s) == a.never) a.sink[0] = 1u;
}

#define Q8_PROBE_SPLIT(NAME, ROLE_A, ROLE_B)                                                    \
    extern "C" __global__ __launch_bounds__(512) void q8_probe_split_##NAME(Q8ProbeArgs a) {  \
        if ((threadIdx.x >> 6) < 4) {                                                          \
            if (a.mask & 1) ROLE_A(a);                                                         \
        } else {                                                                               \
            if (a.mask & 2) ROLE_B(a);                                                         \
        }                                                                                      \
    }
Q8_PROBE_SPLIT(i8_valu, role_i8, role_valu<1>)
Q8_PROBE_SPLIT(i8_fma, role_i8, role_valu<0>)
Q8_PROBE_SPLIT(f32_valu, role_f32, role_valu<1>)
