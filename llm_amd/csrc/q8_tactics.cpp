// q8_tactics.cpp -- see q8_tactics.h.
#include "q8_tactics.h"

#include <algorithm>

namespace {

const Q8TacticRow kRows[] = {
    {"matmul.gemv_f32", Q8_KERNEL_GEMV, 1, 1, Q8_MATURITY_MEASURED, 10,
     "n = 1 keeps f32 activations (tensor.rs:96-101); one 64-lane dwordx4 load per 32-row x "
     "32-element unit, x staged in LDS, HBM-bound"},
    {"matmul.gemm_mfma_i8", Q8_KERNEL_GEMM, 2, Q8_MAX_TOKENS, Q8_MATURITY_MEASURED, 10,
     "n >= 2 quantizes activations (tensor.rs:104-125); v_mfma_i32_32x32x32_i8 is one Q8_0 block "
     "per instruction, exact int32, scale products on v_mfma_f32_32x32x1_2b_f32"},
    {"matmul.gemm_f32_small_n", Q8_KERNEL_GEMM, 2, 7, Q8_MATURITY_REJECTED, 0,
     "the reference GPU's f32-activation path for 2 <= n <= 7 (cuda/mod.rs:883-891) disagrees with "
     "the CPU kernels that define parity, which quantize for every n >= 2"},
    {"matmul.gemm_mfma_i8_16x16x64", Q8_KERNEL_GEMM, 2, Q8_MAX_TOKENS, Q8_MATURITY_REJECTED, 0,
     "K = 64 sums two Q8_0 blocks with different d_w*d_x in one int32 accumulator, so the per-block "
     "scale can no longer be applied exactly"},
};
constexpr int kCount = sizeof(kRows) / sizeof(kRows[0]);

int ceil_div(long long a, long long b) { return (int)((a + b - 1) / b); }

// GEMV launch shape: enough waves to cover every SIMD about twice, each wave
// taking a contiguous run of block pairs (at most 12, the LDS staging bound),
// with the first batch of loads covering the whole run when it is short.
void gemv_shape(int out, int k, int cu_count, q8_tactic *t) {
    const int nb = k / 32;
    const int tiles = ceil_div(out, 32);
    const int npairs = ceil_div(nb, 2);
    const long long target_waves = 2LL * 4 * std::max(cu_count, 1);
    int w = (int)std::min<long long>(8, std::max<long long>(1, (target_waves + tiles - 1) / tiles));
    w = std::max(w, ceil_div(npairs, 12));
    w = std::min(w, npairs);
    int ppw = ceil_div(npairs, w);
    w = ceil_div(npairs, ppw);
    int pb = ppw <= 2 ? 2 : ppw <= 3 ? 3 : ppw <= 5 ? 5 : ppw <= 9 ? 9 : 5;
    t->waves_per_tile = w;
    t->pairs_per_wave = ppw;
    t->pairs_per_batch = pb;
    t->exact = 1;
}

void gemm_shape(int n, int out, int /*k*/, int /*cu_count*/, q8_tactic *t) {
    const int ttiles = ceil_div(n, 32);
    (void)out;
    t->tt_per_wg = std::min(4, ttiles);
    t->smode = 1;
    t->xcd_remap = 1;
}

}  // namespace

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
        gemv_shape(out, k, cu_count, t);
    else
        gemm_shape(n, out, k, cu_count, t);
    return Q8_OK;
}
