/*
 * q8_oracle.c -- CPU restatement of the reference's Q8_0 matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP path is
 * compared against; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  Nothing in llm_amd/ links or calls it.
 *
 * It restates, function by function and in the same floating-point order:
 *   apps/engine/src/quant.rs:8-203   (block format, dot_q8_0 scalar + AVX2,
 *                                     horizontal_sum, quantize_q8_0,
 *                                     dot_q8_0_q8_0 scalar + AVX2, dequant)
 *   apps/engine/src/tensor.rs:92-149 (matmul: n == 1 f32 dot per row,
 *                                     n >= 2 quantize then int8 dot,
 *                                     transposed scratch)
 *   apps/engine/src/ops.rs:5-35      (rmsnorm with f64 sum of squares, silu)
 *   apps/engine/src/sampler.rs:167-175 (argmax: first strictly greatest)
 *
 * Rust semantics reproduced here:
 *   - f32::round rounds half away from zero            -> roundf
 *   - `as i8` saturates and maps NaN to 0               -> sat_i8()
 *   - f32::max ignores a NaN operand                    -> fmaxf
 *   - rustc never contracts a*b+c; the only FMAs are the explicit
 *     _mm256_fmadd_ps calls -> this file must be built with
 *     -ffp-contract=off (oracle/Makefile does).
 *   - half::f16::to_f32 is exact, subnormals included  -> f16_to_f32()
 *   - dispatch: AVX2 iff avx2 && fma at run time, else scalar
 *     (quant.rs:25-31, 136-140).
 * rayon only partitions output rows (every output element is computed by one
 * thread with no cross-thread reduction), so the thread count here has no
 * numeric effect; it exists for the CPU baseline timing.
 */
#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define Q8_BLOCK_ELEMS 32 /* quant.rs:8 */
#define Q8_BLOCK_BYTES 34 /* quant.rs:9 */

/* ---- f16 -> f32, exact (half 2.7.1 f16::to_f32; quant.rs:34-37) ---- */
float q8o_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0x1fu) {
        /* inf, or NaN with the payload kept and the quiet bit set */
        bits = man ? (sign | 0x7fc00000u | (man << 13)) : (sign | 0x7f800000u);
    } else if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            /* subnormal: value = man * 2^-24, exact in f32 */
            float v = (float)man * 5.9604644775390625e-8f; /* 2^-24, exact */
            uint32_t vb;
            memcpy(&vb, &v, 4);
            bits = sign | vb;
        }
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float out;
    memcpy(&out, &bits, 4);
    return out;
}

static float block_scale(const uint8_t *row, size_t block) {
    size_t base = block * Q8_BLOCK_BYTES;
    uint16_t bits = (uint16_t)(row[base] | ((uint16_t)row[base + 1] << 8));
    return q8o_f16_to_f32(bits);
}

/* ---- Rust `f32 as i8` (saturating, NaN -> 0) ---- */
static int8_t sat_i8(float v) {
    if (isnan(v)) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v; /* truncation toward zero, as `as` does */
}

/* ---- dot_q8_0: n == 1 path on f32 activations ---- */

/* quant.rs:39-52 */
float q8o_dot_q8_0_scalar(const uint8_t *row, const float *x, size_t blocks) {
    float total = 0.0f;
    for (size_t block = 0; block < blocks; block++) {
        size_t base = block * Q8_BLOCK_BYTES;
        const uint8_t *quants = row + base + 2;
        const float *values = x + block * Q8_BLOCK_ELEMS;
        float sum = 0.0f;
        for (int i = 0; i < Q8_BLOCK_ELEMS; i++) {
            float prod = (float)(int8_t)quants[i] * values[i];
            sum = sum + prod;
        }
        float scaled = block_scale(row, block) * sum;
        total = total + scaled;
    }
    return total;
}

/* quant.rs:80-91 */
__attribute__((target("avx2"))) static float horizontal_sum(__m256 vector) {
    __m128 low = _mm256_castps256_ps128(vector);
    __m128 high = _mm256_extractf128_ps(vector, 1);
    __m128 sum = _mm_add_ps(low, high);
    sum = _mm_hadd_ps(sum, sum);
    sum = _mm_hadd_ps(sum, sum);
    return _mm_cvtss_f32(sum);
}

/* quant.rs:54-78 */
__attribute__((target("avx2,fma"))) float q8o_dot_q8_0_avx2(const uint8_t *row, const float *x,
                                                            size_t blocks) {
    float total = 0.0f;
    for (size_t block = 0; block < blocks; block++) {
        size_t base = block * Q8_BLOCK_BYTES;
        __m256 acc = _mm256_setzero_ps();
        for (int chunk = 0; chunk < 4; chunk++) {
            __m128i packed = _mm_loadl_epi64((const __m128i *)(row + base + 2 + chunk * 8));
            __m256i widened = _mm256_cvtepi8_epi32(packed);
            __m256 as_float = _mm256_cvtepi32_ps(widened);
            __m256 vector = _mm256_loadu_ps(x + block * Q8_BLOCK_ELEMS + chunk * 8);
            acc = _mm256_fmadd_ps(as_float, vector, acc);
        }
        float scaled = block_scale(row, block) * horizontal_sum(acc);
        total = total + scaled;
    }
    return total;
}

static int have_avx2_fma(void) {
    static int cached = -1;
    if (cached < 0) {
        __builtin_cpu_init();
        cached = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
    }
    return cached;
}

int q8o_simd_path(void) { return have_avx2_fma(); }

/* quant.rs:12-32 (dispatch) */
float q8o_dot_q8_0(const uint8_t *row, const float *x, size_t blocks) {
    if (have_avx2_fma()) return q8o_dot_q8_0_avx2(row, x, blocks);
    return q8o_dot_q8_0_scalar(row, x, blocks);
}

/* ---- quantize_q8_0 (quant.rs:98-121) ---- */
void q8o_quantize_q8_0(const float *x, size_t len, int8_t *quants, float *scales) {
    size_t blocks = len / Q8_BLOCK_ELEMS;
    for (size_t block = 0; block < blocks; block++) {
        const float *values = x + block * Q8_BLOCK_ELEMS;
        float peak = 0.0f;
        for (int i = 0; i < Q8_BLOCK_ELEMS; i++) peak = fmaxf(peak, fabsf(values[i]));
        float scale = peak / 127.0f;
        float inverse = peak > 0.0f ? 127.0f / peak : 0.0f;
        scales[block] = scale;
        for (int i = 0; i < Q8_BLOCK_ELEMS; i++) {
            float product = values[i] * inverse;
            quants[block * Q8_BLOCK_ELEMS + i] = sat_i8(roundf(product));
        }
    }
}

/* ---- dot_q8_0_q8_0: n >= 2 path on pre-quantized activations ---- */

/* quant.rs:142-153 */
float q8o_dot_q8_0_q8_0_scalar(const uint8_t *row, const int8_t *quants, const float *scales,
                               size_t blocks) {
    float total = 0.0f;
    for (size_t block = 0; block < blocks; block++) {
        size_t base = block * Q8_BLOCK_BYTES;
        const uint8_t *weights = row + base + 2;
        const int8_t *values = quants + block * Q8_BLOCK_ELEMS;
        int32_t sum = 0;
        for (int i = 0; i < Q8_BLOCK_ELEMS; i++) sum += (int32_t)(int8_t)weights[i] * (int32_t)values[i];
        float combined = block_scale(row, block) * scales[block];
        float term = combined * (float)sum;
        total = total + term;
    }
    return total;
}

/* quant.rs:156-181 */
__attribute__((target("avx2,fma"))) float q8o_dot_q8_0_q8_0_avx2(const uint8_t *row,
                                                                 const int8_t *quants,
                                                                 const float *scales,
                                                                 size_t blocks) {
    __m256 acc = _mm256_setzero_ps();
    for (size_t block = 0; block < blocks; block++) {
        size_t base = block * Q8_BLOCK_BYTES;
        __m256i weight = _mm256_loadu_si256((const __m256i *)(row + base + 2));
        __m256i value = _mm256_loadu_si256((const __m256i *)(quants + block * Q8_BLOCK_ELEMS));
        __m256i magnitude = _mm256_sign_epi8(value, value);
        __m256i signed_weight = _mm256_sign_epi8(weight, value);
        __m256i pairs = _mm256_maddubs_epi16(magnitude, signed_weight);
        __m256i sums = _mm256_madd_epi16(pairs, _mm256_set1_epi16(1));
        __m256 combined = _mm256_set1_ps(block_scale(row, block) * scales[block]);
        acc = _mm256_fmadd_ps(combined, _mm256_cvtepi32_ps(sums), acc);
    }
    return horizontal_sum(acc);
}

/* quant.rs:127-140 (dispatch) */
float q8o_dot_q8_0_q8_0(const uint8_t *row, const int8_t *quants, const float *scales,
                        size_t blocks) {
    if (have_avx2_fma()) return q8o_dot_q8_0_q8_0_avx2(row, quants, scales, blocks);
    return q8o_dot_q8_0_q8_0_scalar(row, quants, scales, blocks);
}

/* The exact int32 block dot Σ q_w·q_x that both dot_q8_0_q8_0 orders build
 * on (quant.rs:147-150), by brute force in int64 and checked to fit i32. */
int64_t q8o_block_dot_i64(const uint8_t *row, const int8_t *quants, size_t block) {
    size_t base = block * Q8_BLOCK_BYTES;
    int64_t sum = 0;
    for (int i = 0; i < Q8_BLOCK_ELEMS; i++)
        sum += (int64_t)(int8_t)row[base + 2 + i] * (int64_t)quants[block * Q8_BLOCK_ELEMS + i];
    return sum;
}

/* quant.rs:184-203 */
void q8o_dequant_q8_0(const uint8_t *row, float *out, size_t len) {
    size_t blocks = len / Q8_BLOCK_ELEMS;
    for (size_t block = 0; block < blocks; block++) {
        size_t base = block * Q8_BLOCK_BYTES;
        float scale = block_scale(row, block);
        for (int i = 0; i < Q8_BLOCK_ELEMS; i++)
            out[block * Q8_BLOCK_ELEMS + i] = scale * (float)(int8_t)row[base + 2 + i];
    }
}

/* ---- tensor::matmul (tensor.rs:92-149), row-parallel like rayon ---- */

typedef struct {
    const uint8_t *data;
    size_t k, out, n;
    const float *x;
    float *y;
    const int8_t *quants;
    const float *scales;
    float *scratch;
    size_t row_begin, row_end;
    int phase; /* 0: n == 1 dots, 1: int8 dots into scratch, 2: transpose, 3: quantize */
    size_t tok_begin, tok_end;
} Job;

static void *run_job(void *arg) {
    Job *j = (Job *)arg;
    size_t blocks = j->k / Q8_BLOCK_ELEMS;
    size_t row_bytes = blocks * Q8_BLOCK_BYTES;
    if (j->phase == 0) {
        for (size_t o = j->row_begin; o < j->row_end; o++)
            j->y[o] = q8o_dot_q8_0(j->data + o * row_bytes, j->x, blocks);
    } else if (j->phase == 3) {
        for (size_t t = j->tok_begin; t < j->tok_end; t++)
            q8o_quantize_q8_0(j->x + t * j->k, j->k, (int8_t *)j->quants + t * j->k,
                              (float *)j->scales + t * blocks);
    } else if (j->phase == 1) {
        for (size_t o = j->row_begin; o < j->row_end; o++)
            for (size_t t = 0; t < j->n; t++)
                j->scratch[o * j->n + t] = q8o_dot_q8_0_q8_0(
                    j->data + o * row_bytes, j->quants + t * j->k, j->scales + t * blocks, blocks);
    } else {
        for (size_t t = j->tok_begin; t < j->tok_end; t++)
            for (size_t o = 0; o < j->out; o++) j->y[t * j->out + o] = j->scratch[o * j->n + t];
    }
    return NULL;
}

static void run_parallel(Job *proto, int threads, size_t rows, size_t toks) {
    if (threads < 1) threads = 1;
    pthread_t tid[256];
    Job jobs[256];
    if (threads > 256) threads = 256;
    for (int i = 0; i < threads; i++) {
        jobs[i] = *proto;
        jobs[i].row_begin = rows * (size_t)i / (size_t)threads;
        jobs[i].row_end = rows * (size_t)(i + 1) / (size_t)threads;
        jobs[i].tok_begin = toks * (size_t)i / (size_t)threads;
        jobs[i].tok_end = toks * (size_t)(i + 1) / (size_t)threads;
    }
    if (threads == 1) {
        run_job(&jobs[0]);
        return;
    }
    for (int i = 0; i < threads; i++) pthread_create(&tid[i], NULL, run_job, &jobs[i]);
    for (int i = 0; i < threads; i++) pthread_join(tid[i], NULL);
}

/* y[t*out + o] = Σ_i x[t*k + i] * W[o*k + i] over GGUF Q8_0 bytes `data`
 * (out rows of k/32 blocks of 34 bytes).  Returns 0, or -1 on a shape error
 * (the reference asserts; tensor.rs:93-94). */
int q8o_matmul(const uint8_t *data, size_t k, size_t out, const float *x, size_t n, float *y,
               int threads) {
    if (k % Q8_BLOCK_ELEMS != 0 || n == 0) return -1;
    Job proto;
    memset(&proto, 0, sizeof proto);
    proto.data = data;
    proto.k = k;
    proto.out = out;
    proto.n = n;
    proto.x = x;
    proto.y = y;
    if (n == 1) {
        proto.phase = 0;
        run_parallel(&proto, threads, out, 0);
        return 0;
    }
    size_t blocks = k / Q8_BLOCK_ELEMS;
    int8_t *quants = (int8_t *)malloc(n * k);
    float *scales = (float *)malloc(n * blocks * sizeof(float));
    float *scratch = (float *)malloc(out * n * sizeof(float));
    if (!quants || !scales || !scratch) {
        free(quants);
        free(scales);
        free(scratch);
        return -2;
    }
    proto.quants = quants;
    proto.scales = scales;
    proto.scratch = scratch;
    /* tensor.rs:110-125: quantize every token (parallel when n >= 8) */
    proto.phase = 3;
    run_parallel(&proto, n >= 8 ? threads : 1, 0, n);
    proto.phase = 1;
    run_parallel(&proto, threads, out, 0);
    proto.phase = 2;
    run_parallel(&proto, threads, 0, n);
    free(quants);
    free(scales);
    free(scratch);
    return 0;
}

/* ---- ops (ops.rs:5-35) and the greedy argmax (sampler.rs:167-175) ---- */

/* ops.rs:33-35 */
float q8o_silu(float value) { return value / (1.0f + expf(-value)); }

/* compute.rs:940-944: act[i] = silu(gate[i]) * up[i] */
void q8o_silu_mul(const float *gate, const float *up, float *act, size_t len) {
    for (size_t i = 0; i < len; i++) act[i] = q8o_silu(gate[i]) * up[i];
}

/* ops.rs:26-30 */
float q8o_rms_scale(const float *row, size_t len, float eps) {
    double sum = 0.0;
    for (size_t i = 0; i < len; i++) {
        float sq = row[i] * row[i];
        sum += (double)sq;
    }
    float mean_square = (float)(sum / (double)len);
    return 1.0f / sqrtf(mean_square + eps);
}

/* ops.rs:5-12 */
void q8o_rmsnorm(const float *x, const float *weight, size_t len, float eps, float *out) {
    float scale = q8o_rms_scale(x, len, eps);
    for (size_t i = 0; i < len; i++) {
        float a = x[i] * scale;
        out[i] = a * weight[i];
    }
}

/* sampler.rs:167-175 */
uint32_t q8o_argmax(const float *values, size_t len) {
    size_t best = 0;
    for (size_t i = 0; i < len; i++)
        if (values[i] > values[best]) best = i;
    return (uint32_t)best;
}
