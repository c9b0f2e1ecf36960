// q8_probe.hip -- measurement kernels: the ceilings the benchmark quotes its
// hot-path kernels against (no counterpart in the reference; included at the
// end of q8_kernels.hip, so they share its code object and build flags).
//
//   q8_probe_read_l{4,8,16}  a plain streaming read of `bytes`: 256 threads a
//                            workgroup, L 16-byte loads per lane all issued
//                            before any is used, one pass (grid = bytes /
//                            (4096 L)); the best L at a given size is the
//                            "what can a single kernel read" ceiling of an
//                            HBM-bound launch of that size;
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
//                            MFMA and 16 fma (no converts).
// Results feed `sink` only when equal to `never` (the host passes a value no
// result takes), so no work is dead and nothing is written.

template <int L>
static __device__ __forceinline__ void probe_read(const Q8ProbeArgs &a) {
    const long long base = (long long)blockIdx.x * (256 * 16 * L) + threadIdx.x * 16;
    i32x4 v[L];
#pragma unroll
    for (int i = 0; i < L; i++) {
        const long long off = min(base + (long long)i * 256 * 16, a.bytes - 16);
        v[i] = *(const i32x4 *)(a.src + off);
    }
    unsigned acc = 0;
#pragma unroll
    for (int i = 0; i < L; i++) acc ^= (unsigned)(v[i].x ^ v[i].y ^ v[i].z ^ v[i].w);
    if (acc == a.never) a.sink[0] = acc;
}

extern "C" __global__ __launch_bounds__(256) void q8_probe_read_l4(Q8ProbeArgs a) { probe_read<4>(a); }
extern "C" __global__ __launch_bounds__(256) void q8_probe_read_l8(Q8ProbeArgs a) { probe_read<8>(a); }
extern "C" __global__ __launch_bounds__(256) void q8_probe_read_l16(Q8ProbeArgs a) { probe_read<16>(a); }

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
