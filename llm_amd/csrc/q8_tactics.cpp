// q8_tactics.cpp -- see q8_tactics.h.
#include "q8_tactics.h"
#include "q8_layout.h"

#include <algorithm>
#include <cmath>

namespace {

const Q8TacticRow kRows[] = {
    {"matmul.gemv_f32", Q8_KERNEL_GEMV, 1, 1, Q8_MATURITY_MEASURED, 10,
     "n = 1 keeps f32 activations (tensor.rs:96-101); one 64-lane dwordx4 load per 32-row x "
     "32-element unit, x staged in LDS, HBM-bound"},
    {"matmul.gemm_mfma_i8", Q8_KERNEL_GEMM, 2, Q8_MAX_TOKENS, Q8_MATURITY_MEASURED, 10,
     "n >= 2 quantizes activations (tensor.rs:104-125); v_mfma_i32_32x32x32_i8 is one Q8_0 block "
     "per instruction, exact int32, scale products on v_mfma_f32_32x32x1_2b_f32"},
    {"matmul.gemv_q8x_two_tokens", Q8_KERNEL_GEMV, 2, 2, Q8_MATURITY_MEASURED, 9,
     "f32 x at n = 2 (q8_matmul without prepared activations; ranked below the GEMM, which plans for "
     "prepared activations keep): x quantized to Q8_0 in the GEMV's own launch, four v_dot4_i32_i8 per "
     "half block, the weight stream read once for both tokens; configs[1]'s W: 7.25 us against 10.45 us "
     "for quantize + int8 MFMA GEMM.  At n = 4 and 8 the quantization every workgroup repeats outgrew "
     "the GEMM (11.5 and 24.0 us against 10.5)"},
    {"matmul.gemm_mfma_f16", Q8_KERNEL_GEMM_F16, 2, Q8_MAX_TOKENS, Q8_MATURITY_EXPERIMENTAL, 5,
     "quants are integers |q| <= 127, exact in f16: two v_mfma_f32_32x32x16_f16 give each block's int32 "
     "dot already in f32, removing the 16 v_cvt_f32_i32 per 32x32 tile and block that bound the int8 "
     "path on the VALU; bit-identical to the int8 kernel.  Measured slower so far (gate|up n=512 70 us "
     "vs 50 us): one wave per row tile reads 2 KB of f16 activations per block-tile from LDS, about "
     "150 B/clk per CU at the MFMA rate, above the LDS bandwidth; option gemm.f16 = 1 selects it"},
    {"matmul.gemm_mfma_i8_pipelined", Q8_KERNEL_GEMM, 2, Q8_MAX_TOKENS, Q8_MATURITY_REJECTED, 0,
     "each item's MFMAs issued one item ahead of the previous epilogue (option gemm.pipe): two result "
     "buffers cost ~130 VGPRs, two waves per SIMD instead of three; gate|up n=512 57 us vs 51 us"},
    {"matmul.gemm_mfma_i8_lds_staged", Q8_KERNEL_GEMM, 2, Q8_MAX_TOKENS, Q8_MATURITY_REJECTED, 0,
     "int8 activations staged once per workgroup in LDS with global_load_lds and shared by row-tile "
     "waves (option gemm.lds), cutting L2 reads (the plain kernel reads both operands from L2 at "
     "86-92% hit rates, its HBM fetch 1.4-3.4x the weight bytes: the activations once per XCD): one "
     "workgroup barrier per block pair costs more; gate|up n=512 56 us vs 51 us"},
    {"matmul.gemm_f32_small_n", Q8_KERNEL_GEMM, 2, 7, Q8_MATURITY_REJECTED, 0,
     "the reference GPU's f32-activation path for 2 <= n <= 7 (cuda/mod.rs:883-891) disagrees with "
     "the CPU kernels that define parity, which quantize for every n >= 2"},
    {"matmul.gemm_mfma_i8_16x16x64", Q8_KERNEL_GEMM, 2, Q8_MAX_TOKENS, Q8_MATURITY_REJECTED, 0,
     "K = 64 sums two Q8_0 blocks with different d_w*d_x in one int32 accumulator, so the per-block "
     "scale can no longer be applied exactly"},
};
constexpr int kCount = sizeof(kRows) / sizeof(kRows[0]);

int ceil_div(long long a, long long b) { return (int)((a + b - 1) / b); }

int pairs_per_batch(int ppw) { return ppw <= 2 ? 2 : ppw <= 3 ? 3 : ppw <= 5 ? 5 : 3; }

}  // namespace

// GEMV launch shape: one workgroup per 32-row tile (two for the fused
// gate/up pair), its block pairs split over W waves.  Large matrices (two or
// more tiles per CU) take four waves of up to nine pairs; smaller ones take
// waves of about three pairs, up to 16 waves, so the whole matrix is in
// flight at once.  Splitting a tile's blocks over several workgroups (kslices)
// needs an agent-scope release per workgroup, which on gfx950 writes back the
// XCD's L2; measured slower, so it is never chosen here (option "gemv.slices").
void q8_gemv_shape(int out, int k, int cu_count, int slots, q8_tactic *t) {
    const int nb = k / 32;
    const int tiles = ceil_div(out, 32);
    const int npairs = ceil_div(nb, 2);
    const int cus = std::max(cu_count, 1);
    const int max_w = 16 / slots;
    // about three block pairs per wave, at any tile count: the lm_head
    // (122880 x 2304, 3840 tiles) measured 46.3 us at four waves per tile and
    // 42.7 us at twelve (one 301 MB copy, gfx950)
    int w = std::min(max_w, std::max(1, ceil_div(npairs, 3)));
    int ppw = ceil_div(npairs, w);
    if (ppw > 12) ppw = 12;  // LDS staging bound of a wave
    w = ceil_div(npairs, ppw);
    int s = 1;
    if (w > max_w) {  // K too long for one workgroup: split it
        s = ceil_div(w, max_w);
        const int pps = ceil_div(npairs, s);
        s = ceil_div(npairs, pps);
        w = ceil_div(pps, ppw);
    }
    t->kslices = s;
    t->waves_per_tile = w;
    t->pairs_per_wave = ppw;
    t->pairs_per_batch = pairs_per_batch(ppw);
    if (w * slots > 8 && t->pairs_per_batch == 9) t->pairs_per_batch = 5;
    // Blocks are summed in a fixed tree (deterministic, within f32 rounding of
    // the reference's left-to-right sum; every block value is the reference's
    // own bits).  exact = 1 (option "gemv.exact") keeps the reference's
    // left-to-right order for bit-identical outputs; it costs a serial chain of
    // nb adds per row at the end of the kernel (configs[0]: 5.48 vs 5.26 us).
    t->exact = 0;
    // A single matrix with fewer tiles than CUs runs in row slices (whole K
    // per workgroup): 8-row slices (four per tile) when 16-row slices would
    // already fill every CU and the 8-row workgroups fit (below), else
    // 16-row slices with as many waves as fit 16 at three loads per lane,
    // else six.  Measured
    // MALL-cold on gfx950 (tile kernel -> slices): configs[0] 5760 x 2304
    // 5.50 -> 5.36 us (16-row slices 5.50), O 2304 x 2304 4.98 -> 3.95 us
    // (8-row 4.29), down 2304 x 5760 8.25 -> 6.2 us (8-row 6.84); the lm_head
    // (3840 tiles) keeps the tile kernel (51.5 us either way).
    t->row_slice = Q8_TILE_ROWS;
    t->slice_loads = 0;
    // 8-row slices take two loads per lane (eight blocks a wave, more and
    // shorter waves) and only where every workgroup is resident at once, 32
    // waves a CU (eight per SIMD): configs[0] 5.13 -> 4.94 us against three
    // loads, 4096 x 2304 4.43 -> 4.22 us.  Where they would need a second
    // round of workgroups the 16-row slices win (6912 x 2304 with
    // non-temporal weight loads: 16-row 5.22 us, 8-row 5.37 at two loads and
    // 5.54 at three).
    const int w2 = ceil_div(nb, 2 * 4);
    if (slots == 1 && tiles < cus && 2 * tiles >= cus && w2 <= 16 && 4 * tiles <= cus * (32 / w2)) {
        t->row_slice = 8;
        t->slice_loads = 2;
    } else if (slots == 1 && tiles < cus) {
        if (ceil_div(nb, 3 * 2) <= 16) {
            t->row_slice = 16;
            t->slice_loads = 3;
        } else if (ceil_div(nb, 6 * 2) <= 16) {
            t->row_slice = 16;
            t->slice_loads = 6;
        }
    }
}

// GEMM launch shape.  A wave owns TPW token tiles of one 32-row tile.  Two
// tiles per wave share the weight stream and measured best for wide matrices
// (n = 512: gate|up 11520 rows 51 us, QKV 6912 rows 37.5 us); one tile per
// wave with the block pairs split over eight waves of a workgroup (reduced in
// LDS in a fixed order) measured best for the 2304-row projections (O 18.6 us,
// down 33 us) and for small n.  Four tiles per wave needs ~240 VGPRs (two
// waves per SIMD) and measured slower everywhere; it stays an option.
void q8_gemm_shape(int n, int out, int k, int cu_count, q8_tactic *t) {
    // Measured on gfx950 (n = 8 ... 1024, M = 2304 ... 11 520, K = 2304 / 5760):
    // a wave costs a fixed prologue (first loads) and K reduction, so it wants
    // at least ~9 block pairs of work, and the launch wants ~18 waves per CU
    // (4.5 per SIMD) to hide the MFMA -> convert -> fma chain of each wave.
    // Very tall matrices (gate|up, 360 row tiles) already have enough waves
    // with two token tiles per wave and the full K; matrices of >= 128 row
    // tiles pair two token-tile waves in a workgroup, which then share the
    // weight units in L1.
    const int nb = k / 32;
    const int npairs = ceil_div(nb, 2);
    const int ttiles = ceil_div(n, 32);
    const int rtiles = ceil_div(out, 32);
    const int cus = std::max(cu_count, 1);
    const int tpw = (rtiles >= 300 && ttiles >= 2) ? 2 : 1;
    const int groups = ceil_div(ttiles, tpw);
    const long long base = (long long)rtiles * groups;  // waves without a K split
    const long long target = (tpw == 1 ? 18LL : 11LL) * cus;  // 4608 / 2816 waves on 256 CUs
    int kw = (int)std::max<long long>(1, (target + base - 1) / base);
    kw = std::min(kw, std::max(1, npairs / 9));
    kw = std::min(kw, 8);
    const int ppw = ceil_div(npairs, kw);
    kw = ceil_div(npairs, ppw);
    const int tw = (tpw == 1 && rtiles >= 128 && groups >= 2 && kw <= 8) ? 2 : 1;
    t->tpw = tpw;
    t->twaves = tw;
    t->kwaves = kw;
    t->kslices = 1;
    t->pairs_per_wave = ppw;
    t->smode = 1;
    t->xcd_remap = 1;
}

// f16 GEMM launch shape: TPW token tiles per wave (2 when there are two or
// more), RW row-tile waves sharing the LDS-staged activations, KW K-split
// waves, RW * KW <= 8.  The GEMM kernel runs two waves per SIMD (about 210
// VGPRs), so the chip holds 2 * 4 * cu_count waves at once; the search takes
// the (RW, KW) whose last round of waves is fullest, discounted for the fixed
// per-wave cost (about two block pairs of prologue, drain and K reduction).
void q8_gemm_h_shape(int n, int out, int k, int cu_count, q8_tactic *t) {
    q8_gemm_staged_shape(n, out, k, cu_count, 0, t);
}

void q8_gemm_staged_shape(int n, int out, int k, int cu_count, int i8, q8_tactic *t) {
    const int nb = k / 32;
    const int npairs = ceil_div(nb, 2);
    const int ttiles = ceil_div(n, 32);
    const int rtiles = ceil_div(out, 32);
    const double cap = 2.0 * 4.0 * std::max(cu_count, 1);
    const int tpw = ttiles >= 2 ? 2 : 1;
    double best = -1.0;
    int best_rw = (tpw == 1 && i8) ? 2 : 4, best_kw = 1;
    for (int rw : {2, 4}) {
        if (tpw == 1 && rw != (i8 ? 2 : 4)) continue;  // built: f16 t1_r4, t2_r2, t2_r4; int8 t1_r2, t2_r2, t2_r4
        for (int kw = 1; rw * kw <= 8 && kw <= npairs; kw++) {
            // LDS: KW K groups x the staging ring, within 64 KB
            const long long lds =
                (long long)kw * Q8_GEMM_H_STAGES * (i8 ? Q8_GEMM_L_BUF_BYTES(tpw, rw) : Q8_GEMM_H_BUF_BYTES(tpw, rw));
            if (lds > 65536) continue;
            const int ppw = ceil_div(npairs, kw);
            if (ceil_div(npairs, ppw) != kw) continue;  // no K wave without pairs
            const double waves = (double)ceil_div(rtiles, rw) * ceil_div(ttiles, tpw) * rw * kw;
            const double rounds = waves / cap;
            const double fill = rounds / std::ceil(rounds);
            const double live = (double)rtiles / (ceil_div(rtiles, rw) * rw);  // row waves past the end idle
            const double score = fill * live * ppw / (ppw + 2.0);
            if (score > best + 1e-9) {
                best = score;
                best_rw = rw;
                best_kw = kw;
            }
        }
    }
    t->tpw = tpw;
    t->rwaves = best_rw;
    t->kwaves = best_kw;
    t->pairs_per_wave = ceil_div(npairs, best_kw);
    t->twaves = 1;
    t->kslices = 1;
    t->smode = 1;
    t->xcd_remap = 1;
}

int q8_tactics_for_kernel(int kernel, int n, int out, int k, int cu_count, q8_tactic *t) {
    for (int i = 0; i < kCount; i++) {
        const Q8TacticRow &row = kRows[i];
        if (row.kernel != kernel || row.maturity == Q8_MATURITY_REJECTED) continue;
        *t = q8_tactic{};
        t->kernel = kernel;
        t->name = row.name;
        t->evidence = row.evidence;
        if (kernel == Q8_KERNEL_GEMV)
            q8_gemv_shape(out, k, cu_count, 1, t);
        else if (kernel == Q8_KERNEL_GEMM_F16)
            q8_gemm_h_shape(n, out, k, cu_count, t);
        else
            q8_gemm_shape(n, out, k, cu_count, t);
        return Q8_OK;
    }
    return Q8_ERR_UNSUPPORTED;
}

int q8_tactics_prepared_format(int n) {
    q8_tactic t{};
    if (q8_tactics_choose(n, 32, 32, 1, &t) != Q8_OK) return Q8_PREPARED_I8;
    return t.kernel == Q8_KERNEL_GEMM_F16 ? Q8_PREPARED_F16 : Q8_PREPARED_I8;
}

int q8_tactics_table_size() { return kCount; }

const Q8TacticRow &q8_tactics_row(int i) { return kRows[i]; }

int q8_tactics_choose(int n, int out, int k, int cu_count, q8_tactic *t) {
    const Q8TacticRow *best = nullptr;
    for (int i = 0; i < kCount; i++) {
        const Q8TacticRow &row = kRows[i];
        if (row.maturity == Q8_MATURITY_REJECTED) continue;
        if (n < row.n_min || n > row.n_max) continue;
        if (!best || row.rank > best->rank) best = &row;
    }
    if (!best) return Q8_ERR_UNSUPPORTED;
    *t = q8_tactic{};
    t->kernel = best->kernel;
    t->name = best->name;
    t->evidence = best->evidence;
    if (best->kernel == Q8_KERNEL_GEMV)
        q8_gemv_shape(out, k, cu_count, 1, t);
    else if (best->kernel == Q8_KERNEL_GEMM_F16)
        q8_gemm_h_shape(n, out, k, cu_count, t);
    else
        q8_gemm_shape(n, out, k, cu_count, t);
    return Q8_OK;
}
