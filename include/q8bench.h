/*
 * q8bench.h -- the benchmark's measurement kernels (libq8bench.so).
 *
 * Not part of the matmul path's boundary (include/q8mi.h) and with no
 * counterpart in the reference: these kernels measure what one MI355X can do
 * at the shapes the path runs, so the benchmark can quote each hot-path
 * kernel against a ceiling.  They live in a code object and a library of
 * their own; the product library neither contains nor calls them.
 *
 * A q8bench handle launches on a HIP stream the caller passes (for the
 * benchmark, the matmul context's stream from q8_stream(), so the probes
 * can be captured into the same graphs and timed with the same events).
 * Status codes are include/q8mi.h's (0 = success).
 */
#ifndef Q8BENCH_H
#define Q8BENCH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct q8bench q8bench;

/* Compute probes: `iters` loop trips per wave over `workgroups` workgroups.
 *   Q8BENCH_MFMA        4 independent chains of v_mfma_i32_32x32x32_i8 (4 per trip), 4 waves a workgroup;
 *   Q8BENCH_VALU        the per-block scale arithmetic: 16 v_cvt_f32_i32 + 16 v_fmac_f32 per trip;
 *   Q8BENCH_MIX         one GEMM tile-block per trip with operands in registers: an int8 MFMA,
 *                       half an f32 outer-product MFMA (v_mfma_f32_32x32x1_2b_f32), 16 cvt + 16 fma,
 *                       the next tile-blocks' MFMAs issued before this one's VALU;
 *   Q8BENCH_MIX_F16     the same for the f16-MFMA family (two v_mfma_f32_32x32x16_f16, no cvt);
 *   Q8BENCH_SPLIT_*     co-resident roles on one SIMD: 8-wave workgroups whose waves 0-3 (one
 *                       per SIMD) run role A and waves 4-7 (the same four SIMDs) role B, each
 *                       for `iters` trips; `mask` bit 0 runs A, bit 1 runs B, so A alone, B
 *                       alone and both together can be timed with the same launch shape:
 *     _I8_VALU          A: 4 int8 MFMAs per trip; B: 16 cvt + 16 fma per trip;
 *     _I8_FMA           A: 4 int8 MFMAs per trip; B: 32 fma per trip;
 *     _F32_VALU         A: 2 f32 outer-product MFMAs per trip; B: 16 cvt + 16 fma per trip. */
enum {
    Q8BENCH_EMPTY = 0,
    Q8BENCH_MFMA = 1,
    Q8BENCH_VALU = 2,
    Q8BENCH_MIX = 3,
    Q8BENCH_MIX_F16 = 4,
    Q8BENCH_SPLIT_I8_VALU = 5,
    Q8BENCH_SPLIT_I8_FMA = 6,
    Q8BENCH_SPLIT_F32_VALU = 7
};

/* Loads the probe code object for the device of `hip_stream` (a
 * hipStream_t) and allocates a 256-byte sink; launches go to that stream. */
int q8bench_open(void *hip_stream, q8bench **out);
void q8bench_close(q8bench *bench);
/* Message of the last failed call on this thread. */
const char *q8bench_last_error(void);
/* The probe code object's identity: sha256, kernel list. */
const char *q8bench_build_info(void);

/* A plain streaming read of `bytes` at `src` (16-byte aligned, a multiple of
 * 16): `loads` 16-byte loads per lane (2, 4, 8 or 16), all issued before any
 * is used, default or non-temporal cache policy (the GEMV's weight loads are
 * non-temporal), `threads` threads per workgroup (a multiple of 64, at most
 * 1024); one pass, ceil(bytes / (threads * 16 * loads)) workgroups. */
int q8bench_read(q8bench *bench, uint64_t src, size_t bytes, int loads, int nontemporal, int threads);
/* A compute probe (Q8BENCH_*); `mask` is read by the split probes only. */
int q8bench_probe(q8bench *bench, int which, int iters, int workgroups, int mask);

#ifdef __cplusplus
}
#endif

#endif /* Q8BENCH_H */
