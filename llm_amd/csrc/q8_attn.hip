// q8_attn.hip -- decoder support kernels around the Q8_0 matmuls, for the
// synthetic decoder and the decode graph (included by q8_kernels.hip, one code
// object):
//   q8_rope_append   rotary embedding of q and k, k and v narrowed to the f16
//                    KV cache                     (gpu.cu rope_append 525-581, ops.rs:152-166)
//   q8_attn_decode   one token against the cache, positions split over
//                    workgroups, combined by the last or by the next kernel
//                    (gpu.cu attention_split 649-733, combine 735-762)
//   q8_attn_prefill  causal attention of n tokens on f16 MFMA (split operands),
//                    online softmax               (compute.rs attend_host 1075-1126)
//   q8_synth         seeded synthetic Q8_0 blocks for the benchmark decoder
//   q8_advance       the position a captured step reads, moved on the device
//
// The position a step works at is read from device memory, so one captured
// graph replays at every position (model.rs:676-731, cuda/mod.rs position_ptr).
// Head width is Q8_ATTN_HEAD_DIM (64): the configuration these kernels serve.

// ---------------------------------------------------------------------------
// RoPE + KV append.  One thread per (token, head, dimension pair) over the q
// heads, then the k heads, then the v heads.  Pairs (2i, 2i+1) inside each head
// rotate by angle = position * freq[i] (pairs at or beyond n_rot/2 are
// copied), computed in f32 exactly as the reference writes it
// (x0*cos - x1*sin, x0*sin + x1*cos, no contraction).  freq[i] =
// base^(-2i/n_rot) comes from the host's powf, the function the reference's
// RopeTable calls (ops.rs:121-131): at position p an ulp of freq moves the
// angle by p ulps, so a device pow would drift from the reference's table by
// ~p * 6e-8 in cos and sin.  q is rotated in place;
// rotated k and plain v are rounded to f16 (nearest even) into the cache at
// rows position + t.  Rows at or past `capacity` are never written.
// ---------------------------------------------------------------------------

extern "C" __global__ __launch_bounds__(256) void q8_rope_append(Q8RopeArgs a) {
    const int start = *a.position;
    const int half = a.head_dim >> 1;
    const int kv_dim = a.n_kv * a.head_dim;
    const int heads = a.n_head + 2 * a.n_kv;
    const long long total = (long long)a.n * heads * half;
    for (long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (long long)gridDim.x * blockDim.x) {
        const int pair = (int)(idx % half);
        const long long th = idx / half;
        const int hh = (int)(th % heads);
        const int t = (int)(th / heads);
        const int pos = start + t;
        if (pos < 0 || pos >= a.capacity) continue;
        if (hh < a.n_head + a.n_kv) {
            const bool is_q = hh < a.n_head;
            const int head = is_q ? hh : hh - a.n_head;
            const float *src = is_q ? a.q + ((size_t)t * a.n_head + head) * a.head_dim + 2 * pair
                                    : a.k + ((size_t)t * a.n_kv + head) * a.head_dim + 2 * pair;
            const float x0 = src[0];
            const float x1 = src[1];
            float y0 = x0, y1 = x1;
            if (2 * pair < a.n_rot) {
                const float angle = (float)pos * a.freq[pair];
                float s, c;
                sincosf(angle, &s, &c);
                y0 = x0 * c - x1 * s;
                y1 = x0 * s + x1 * c;
            }
            if (is_q) {
                float *dq = a.q + ((size_t)t * a.n_head + head) * a.head_dim + 2 * pair;
                dq[0] = y0;
                dq[1] = y1;
            } else {
                unsigned *dk = (unsigned *)(a.kcache + (size_t)pos * kv_dim + head * a.head_dim + 2 * pair);
                *dk = f16_bits(y0) | (f16_bits(y1) << 16);
            }
        } else {
            const int head = hh - a.n_head - a.n_kv;
            const float *src = a.v + (size_t)t * kv_dim + head * a.head_dim + 2 * pair;
            unsigned *dv = (unsigned *)(a.vcache + (size_t)pos * kv_dim + head * a.head_dim + 2 * pair);
            *dv = f16_bits(src[0]) | (f16_bits(src[1]) << 16);
        }
    }
}

// ---------------------------------------------------------------------------
// Decode attention for one token: workgroup (head, split) of W waves takes
// positions [begin, end) of the position + 1 visible ones, in chunks of
// 8 W NP rows (NP passes of 8 W rows).  Eight lanes share a row (16 bytes =
// 8 dims of it each), and a chunk's key AND value rows are all loaded before
// any arithmetic, so the whole chunk costs one memory latency:
//   scores: each lane's 8-dim partial dot (q in registers), summed over the
//           row's 8 lanes by xor shuffles (every lane of the row ends with the
//           same bits), then * scale (the reference's dot * scale);
//   softmax: the chunk's workgroup max m', the running state rescaled by
//           exp(m - m'), p = exp(s - m') -- with one chunk per split m is
//           -inf first, so p = exp(s - max) exactly as the reference forms it;
//   values: each lane accumulates p * v over its rows for its 8 dims; the row
//           slots are summed by xor shuffles in a wave and in LDS across waves,
//           in a fixed order, and so are the weights.
// Two shapes: 16 waves x 8 passes (1024-row chunks) for one split per head,
// 4 waves x 8 passes (256-row chunks) when the positions are split over
// workgroups, so a split of about 256 positions is one chunk (measured
// against 16 x 2 and 8 x 2 passes: equal at 600 positions, faster at 4096).
// splits == 1 writes acc / sum.  defer writes every split's unnormalised
// (acc, max, sum) for the next kernel to combine (the O projection's GEMV
// prologue).  Otherwise each workgroup stores them with agent-scope atomic
// stores and the last workgroup of the head to arrive (an arrival counter,
// reset by it) combines them:
//     max = max_s max_s;  e_s = exp(max_s - max);
//     out = (sum_s acc_s * e_s) / (sum_s sum_s * e_s)   (s ascending, fused
//     multiply-adds)
// -- the same arithmetic as one softmax summed in another order (gpu.cu
// attention_combine 735-762), and the same as the GEMV prologue's.
// ---------------------------------------------------------------------------
static __device__ __forceinline__ float wave_max(float v) {
    v = xor_max<32>(v);
    v = xor_max<16>(v);
    v = xor_max<8>(v);
    v = xor_max<4>(v);
    v = xor_max<2>(v);
    return xor_max<1>(v);
}
static __device__ __forceinline__ float wave_sum(float v) {
    v = xor_add<32>(v);
    v = xor_add<16>(v);
    v = xor_add<8>(v);
    v = xor_add<4>(v);
    v = xor_add<2>(v);
    return xor_add<1>(v);
}

// What the decode attention reads before its first key, as its leading
// kernel arguments: preloaded into SGPRs at wave launch (the kernarg preload
// the row-slice GEMVs use), so the cache position's load, the first dependent
// read, issues at once.  dims = n_head | n_kv << 16; cap = capacity | defer <<
// 31; the (max, sum) plane follows the partial sums (part_acc + heads * splits
// * 64).  scale, out and counters stay in the argument block.
struct AttnHead {
    const float *q;
    const uint16_t *kcache, *vcache;
    const int *position;
    float *part_acc;
    int dims, splits, cap;
};

template <int W, int NP>
static __device__ __forceinline__ void attn_decode_body(const AttnHead &hd, const Q8AttnDecodeArgs &a) {
    constexpr int T = 64 * W;
    constexpr int HD = Q8_ATTN_HEAD_DIM;
    constexpr int RP = T / 8;  // rows per pass
    __shared__ float red[W];
    __shared__ float lsum[W];
    __shared__ __attribute__((aligned(16))) float part[W][HD];
    __shared__ int last_flag;
    const int n_head_ = hd.dims & 0xffff;
    const int n_kv_ = hd.dims >> 16;
    const int splits_ = hd.splits;
    const int capacity_ = hd.cap & 0x7fffffff;
    const int defer_ = (int)((unsigned)hd.cap >> 31);
    float *const part_acc_ = hd.part_acc;
    float *const part_ms_ = hd.part_acc + (size_t)n_head_ * splits_ * Q8_ATTN_HEAD_DIM;
    const int position = *hd.position;
    const int head = blockIdx.x / splits_;
    const int split = blockIdx.x - head * splits_;
    const int kvh = head / (n_head_ / n_kv_);
    const int kv_dim = n_kv_ * HD;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int kc = tid & 7;     // dims 8 kc .. 8 kc + 7
    const int slot = tid >> 3;  // row slot of the pass
    const uint16_t *kbase = hd.kcache + kvh * HD + 8 * kc;
    const uint16_t *vbase = hd.vcache + kvh * HD + 8 * kc;
    float m = -INFINITY;  // running max, workgroup-uniform
    float l = 0.0f;       // this lane's weights summed over its rows
    float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    // One chunk: rows c0 + slot + RP j (j < NP), live below `end`.
    auto chunk = [&](int c0, int end, const f32x4 &q0, const f32x4 &q1, const i32x4 *ku, const i32x4 *vu) {
        float sc[NP];
        float cmax = -INFINITY;
#pragma unroll
        for (int j = 0; j < NP; j++) {
            float dot = 0.0f;
            dot = __builtin_fmaf(q0[0], f16_to_f32((unsigned)ku[j][0] & 0xffffu), dot);
            dot = __builtin_fmaf(q0[1], f16_to_f32((unsigned)ku[j][0] >> 16), dot);
            dot = __builtin_fmaf(q0[2], f16_to_f32((unsigned)ku[j][1] & 0xffffu), dot);
            dot = __builtin_fmaf(q0[3], f16_to_f32((unsigned)ku[j][1] >> 16), dot);
            dot = __builtin_fmaf(q1[0], f16_to_f32((unsigned)ku[j][2] & 0xffffu), dot);
            dot = __builtin_fmaf(q1[1], f16_to_f32((unsigned)ku[j][2] >> 16), dot);
            dot = __builtin_fmaf(q1[2], f16_to_f32((unsigned)ku[j][3] & 0xffffu), dot);
            dot = __builtin_fmaf(q1[3], f16_to_f32((unsigned)ku[j][3] >> 16), dot);
            dot = xor_add<1>(dot);
            dot = xor_add<2>(dot);
            dot = xor_add<4>(dot);
            sc[j] = dot * a.scale;
            if (c0 + slot + RP * j < end) cmax = fmaxf(cmax, sc[j]);
        }
        cmax = wave_max(cmax);
        if (lane == 0) red[wave] = cmax;
        __syncthreads();
        float mx = m;
#pragma unroll
        for (int w = 0; w < W; w++) mx = fmaxf(mx, red[w]);
        __syncthreads();  // red is rewritten by the next chunk
        const float f = expf(m - mx);  // 0 on the first chunk (m = -inf), when l and acc are 0
        l *= f;
#pragma unroll
        for (int d = 0; d < 8; d++) acc[d] *= f;
#pragma unroll
        for (int j = 0; j < NP; j++) {
            if (c0 + slot + RP * j < end) {
                const float pj = expf(sc[j] - mx);
                l += pj;
#pragma unroll
                for (int d = 0; d < 8; d++) {
                    const unsigned bits = ((unsigned)vu[j][d >> 1] >> (16 * (d & 1))) & 0xffffu;
                    acc[d] = __builtin_fmaf(pj, f16_to_f32(bits), acc[d]);
                }
            }
        }
        m = mx;
    };
    const int visible = min(position + 1, capacity_);
    const int per = (visible + splits_ - 1) / splits_;
    const int begin = split * per;
    const int end = min(begin + per, visible);
    // A chunk's key and value rows, clamped to the last live row: rows past
    // `end` repeat its address (no extra traffic) and are masked.  The first
    // chunk is issued before q is read and every later one while the
    // previous is computed, so a split of one chunk waits for one memory
    // latency.
    i32x4 ku[NP], vu[NP];
    auto load_chunk = [&](int c0) {
#pragma unroll
        for (int j = 0; j < NP; j++) {
            const int p = min(c0 + slot + RP * j, end - 1);
            ku[j] = *(const i32x4 *)(kbase + (size_t)p * kv_dim);
            vu[j] = *(const i32x4 *)(vbase + (size_t)p * kv_dim);
        }
    };
    if (begin < end) load_chunk(begin);
    const f32x4 q0 = *(const f32x4 *)(hd.q + (size_t)head * HD + 8 * kc);
    const f32x4 q1 = *(const f32x4 *)(hd.q + (size_t)head * HD + 8 * kc + 4);
    __builtin_amdgcn_sched_barrier(0);
    for (int c0 = begin; c0 < end; c0 += RP * NP) {
        chunk(c0, end, q0, q1, ku, vu);
        if (c0 + RP * NP < end) load_chunk(c0 + RP * NP);
    }
    // row slots of a wave (lanes with the same kc), then the waves; the
    // weights once per row (the kc == 0 lanes)
#pragma unroll
    for (int d = 0; d < 8; d++) {
        acc[d] = xor_add<8>(acc[d]);
        acc[d] = xor_add<16>(acc[d]);
        acc[d] = xor_add<32>(acc[d]);
    }
    const float lw = wave_sum(kc == 0 ? l : 0.0f);
    if (lane < 8) {
        *(f32x4 *)(&part[wave][8 * lane]) = (f32x4){acc[0], acc[1], acc[2], acc[3]};
        *(f32x4 *)(&part[wave][8 * lane + 4]) = (f32x4){acc[4], acc[5], acc[6], acc[7]};
    }
    if (lane == 0) lsum[wave] = lw;
    __syncthreads();
    if (wave != 0) {
        if (splits_ == 1 || defer_) return;
    }
    float tot = 0.0f, sum = 0.0f;
    if (wave == 0) {
#pragma unroll
        for (int w = 0; w < W; w++) tot += part[w][lane];
#pragma unroll
        for (int w = 0; w < W; w++) sum += lsum[w];
    }
    const float mx = m;
    const size_t base = (size_t)head * splits_;
    if (defer_) {  // wave 0: the next kernel reads these after this one ends
        part_acc_[(base + split) * HD + lane] = tot;
        if (lane == 0) {
            *(f32x2 *)(part_ms_ + 2 * (base + split)) = (f32x2){mx, sum};
        }
        return;
    }
    if (splits_ == 1) {
        a.out[(size_t)head * HD + lane] = tot / sum;
        return;
    }
    if (wave == 0) {
        store_agent(part_acc_ + (base + split) * HD + lane, tot);
        if (lane == 0) {
            store_agent(part_ms_ + 2 * (base + split), mx);
            store_agent(part_ms_ + 2 * (base + split) + 1, sum);
        }
    }
    // Release the partials at agent scope, count the arrival with an acq_rel
    // read-modify-write, and acquire in the last workgroup before its loads:
    // the XCDs' L2s are not coherent with each other, so the ordering has to
    // be stated, not left to the stores having completed.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (tid == 0) {
        const unsigned old = __hip_atomic_fetch_add(&a.counters[head], 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        last_flag = (old == (unsigned)(splits_ - 1));
    }
    __syncthreads();
    if (!last_flag) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if (tid == 0) __hip_atomic_store(&a.counters[head], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (wave != 0) return;
    float gmax = -INFINITY;
    for (int s = 0; s < splits_; s++) gmax = fmaxf(gmax, load_agent(part_ms_ + 2 * (base + s)));
    float num = 0.0f, den = 0.0f;
    for (int s = 0; s < splits_; s++) {
        const float f = expf(load_agent(part_ms_ + 2 * (base + s)) - gmax);  // an empty split has max -inf: f = 0
        den = __builtin_fmaf(load_agent(part_ms_ + 2 * (base + s) + 1), f, den);
        num = __builtin_fmaf(load_agent(part_acc_ + (base + s) * HD + lane), f, num);
    }
    a.out[(size_t)head * HD + lane] = num / den;
}

#define Q8_ATTN_PARAMS                                                                                     \
    const float *q, const uint16_t *kcache, const uint16_t *vcache, const int *position, float *part_acc, int dims, \
        int splits, int cap, Q8AttnDecodeArgs a
extern "C" __global__ __launch_bounds__(1024) void q8_attn_decode(Q8_ATTN_PARAMS) {
    attn_decode_body<16, 8>(AttnHead{q, kcache, vcache, position, part_acc, dims, splits, cap}, a);
}
extern "C" __global__ __launch_bounds__(256) void q8_attn_decode_w4(Q8_ATTN_PARAMS) {
    attn_decode_body<4, 8>(AttnHead{q, kcache, vcache, position, part_acc, dims, splits, cap}, a);
}
// The split kernel's 256-row chunks over eight waves: four rows a lane instead of eight.
extern "C" __global__ __launch_bounds__(512) void q8_attn_decode_w8(Q8_ATTN_PARAMS) {
    attn_decode_body<8, 4>(AttnHead{q, kcache, vcache, position, part_acc, dims, splits, cap}, a);
}

// ---------------------------------------------------------------------------
// Prefill attention: n query tokens at cache positions start .. start+n-1, each
// seeing keys 0 .. its own position (causal), on v_mfma_f32_32x32x16_f16.
//
// Workgroup = (head, 32 queries), two waves splitting the 64-key tiles (wave w
// takes tiles w, w+2, ...), combined through LDS at the end.  Per tile a wave
// computes S^T = K Q^T (keys x queries) and O^T += V^T P^T (dims x queries),
// so a lane always holds one query (lane % 32): its scores, its running max
// and sum, and its output accumulators, and the softmax needs no transpose.
// f32 operands enter the MFMA exactly as two f16 parts (x = hi + lo, hi =
// f16(x), lo = f16(x - hi), ~22 significant bits; products of f16 are exact
// in f32): q for the scores, the probabilities for the values; keys and
// values are the f16 cache itself.  Accumulation is f32.  Element k of an
// MFMA operand sits in lane-half k / 8, slot k % 8, for A and B alike; D[m][n]
// has n = lane % 32, m = 8(v/4) + 4(lane/32) + v%4.  Keys past the last
// visible one read as zero values and -inf scores.  Heavier (later) query
// tiles are launched first.
// ---------------------------------------------------------------------------
#define Q8_ATTN_VT_STRIDE 72  /* f16 per V^T row in LDS: 64 keys + 8 of padding, 144 B (16-byte rows) */

// e^x for the softmax's x = s - max <= 0 (x = -inf or below the f32 range
// gives 0): x = n ln2 + r with n = rint(x log2e) and r from a two-part ln2
// (Cody-Waite reduction: ln2_hi has 15 significant bits, so n ln2_hi is exact
// for |n| < 2^9), then e^r = 2^(r log2e) on v_exp_f32 (|r log2e| <= 1/2) and
// 2^n by ldexp.  With a correctly rounded exp2 the result is within 0.85
// ulp of e^x on [-87, 0] (checked in f32 emulation); v_exp_f32 adds its own
// (at most 1 ulp).  Nine instructions where the library expf takes ~25.
static __device__ __forceinline__ float exp_nonpos(float x) {
    const float n = __builtin_rintf(x * 1.44269504f);
    float r = __builtin_fmaf(-n, 0.693145751953125f, x);
    r = __builtin_fmaf(-n, 1.42860682e-06f, r);
    const float e = __builtin_ldexpf(__builtin_amdgcn_exp2f(r * 1.44269504f), (int)n);
    return x >= -87.0f ? e : 0.0f;
}

static __device__ __forceinline__ void split_f16(const float *x, f16x8 &hi, f16x8 &lo) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const _Float16 h = (_Float16)x[i];
        hi[i] = h;
        lo[i] = (_Float16)(x[i] - (float)h);
    }
}

extern "C" __global__ __launch_bounds__(128) void q8_attn_prefill(Q8AttnPrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t vt_all[2][Q8_ATTN_HEAD_DIM * Q8_ATTN_VT_STRIDE];
    __shared__ float xm[64], xl[64];
    __shared__ __attribute__((aligned(16))) float xo[64][33];
    constexpr int HD = Q8_ATTN_HEAD_DIM;
    const int head = blockIdx.x / a.qtiles;
    const int qt = a.qtiles - 1 - (blockIdx.x - head * a.qtiles);
    const int kvh = head / (a.n_head / a.n_kv);
    const int kv_dim = a.n_kv * HD;
    const int start = *a.position;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int h = lane >> 5;
    const int r = lane & 31;
    uint16_t *vt = vt_all[wave];
    const int qrow = qt * 32 + r;  // this lane's query
    const int qa = start + qrow;   // its cache position
    const bool qlive = qrow < a.n;

    // Q^T operand, d-step s: q[qrow][16s + 8h .. +7] as f16 hi/lo
    f16x8 qhi[4], qlo[4];
    {
        const float *src = a.q + ((size_t)min(qrow, a.n - 1) * a.n_head + head) * HD + 8 * h;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            f32x4 u0 = *(const f32x4 *)(src + 16 * s), u1 = *(const f32x4 *)(src + 16 * s + 4);
            float x[8] = {u0[0], u0[1], u0[2], u0[3], u1[0], u1[1], u1[2], u1[3]};
            if (!qlive)
#pragma unroll
                for (int i = 0; i < 8; i++) x[i] = 0.0f;
            split_f16(x, qhi[s], qlo[s]);
        }
    }
    float m = -INFINITY, l = 0.0f;
    f32x16 o[2] = {};
    const f32x16 zero16 = {};
    const int last_q = min(qt * 32 + 31, a.n - 1);
    const int kend = min(start + last_q + 1, a.capacity);  // keys [0, kend)
    const int ntiles = (kend + 63) >> 6;
    // K operand rows (keys p0 + 32kt + r), d-slices 16s + 8h, of this wave's
    // tile t: the next tile's are loaded while the current one is computed
    i32x4 kn[2][4];
    auto load_k = [&](int t) {
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
            const int key = min(t * 64 + 32 * kt + r, a.capacity - 1);
            const uint16_t *krow = a.kcache + (size_t)key * kv_dim + kvh * HD + 8 * h;
#pragma unroll
            for (int s = 0; s < 4; s++) kn[kt][s] = *(const i32x4 *)(krow + 16 * s);
        }
    };
    if (wave < ntiles) load_k(wave);
    for (int t = wave; t < ntiles; t += 2) {
        const int p0 = t * 64;
        i32x4 kk[2][4];
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int s = 0; s < 4; s++) kk[kt][s] = kn[kt][s];
        // S^T: keys x queries
        f32x16 st[2];
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
            f32x16 acc = zero16;
#pragma unroll
            for (int s = 0; s < 4; s++) {
                const f16x8 kv = __builtin_bit_cast(f16x8, kk[kt][s]);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kv, qhi[s], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(kv, qlo[s], acc, 0, 0, 0);
            }
            st[kt] = acc;
        }
        // This tile's value rows (lane -> dims 2(lane%32), +1 at keys
        // 16(lane/32) .. +15 and +32), then the next tile's keys; both land
        // while the softmax runs.
        const int dp = lane & 31;
        unsigned w[2][16];
#pragma unroll
        for (int half_keys = 0; half_keys < 2; half_keys++) {
            const int kb = 32 * half_keys + 16 * h;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                // keys past the last visible one: a clamped (in-bounds) load, then zero
                const int key = p0 + kb + i;
                const unsigned u = *(const unsigned *)(a.vcache + (size_t)min(key, kend - 1) * kv_dim + kvh * HD + 2 * dp);
                w[half_keys][i] = key < kend ? u : 0u;
            }
        }
        if (t + 2 < ntiles) load_k(t + 2);
        // scale, causal mask, online softmax for query qrow; a tile whose last
        // key precedes the workgroup's first query needs no mask
        float tm = -INFINITY;
        if (p0 + 63 <= start + qt * 32) {
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    st[kt][v] = st[kt][v] * a.scale;
                    tm = fmaxf(tm, st[kt][v]);
                }
        } else {
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
                for (int v = 0; v < 16; v++) {
                    const int p = p0 + 32 * kt + 8 * (v >> 2) + 4 * h + (v & 3);
                    const float sc = (p <= qa) ? st[kt][v] * a.scale : -INFINITY;
                    st[kt][v] = sc;
                    tm = fmaxf(tm, sc);
                }
        }
        tm = fmaxf(tm, __shfl_xor(tm, 32));
        const float mn = fmaxf(m, tm);
        // a wave's first tile may be all masked for its queries only if it is
        // not tile 0; then m and mn stay -inf: no weight and no rescale
        const float corr = (mn == -INFINITY) ? 1.0f : exp_nonpos(m - mn);
        float rs = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int v = 0; v < 16; v++) {
                const float e = (mn == -INFINITY) ? 0.0f : exp_nonpos(st[kt][v] - mn);
                st[kt][v] = e;
                rs += e;
            }
        rs += __shfl_xor(rs, 32);
        l = l * corr + rs;
        m = mn;
#pragma unroll
        for (int dt = 0; dt < 2; dt++)
#pragma unroll
            for (int v = 0; v < 16; v++) o[dt][v] *= corr;
        // V^T tile (wave-private) from the value rows
#pragma unroll
        for (int half_keys = 0; half_keys < 2; half_keys++) {
            const int kb = 32 * half_keys + 16 * h;
            i32x4 r0[2], r1[2];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                r0[j >> 2][j & 3] =
                    (int)__builtin_amdgcn_perm(w[half_keys][2 * j + 1], w[half_keys][2 * j], 0x05040100u);
                r1[j >> 2][j & 3] =
                    (int)__builtin_amdgcn_perm(w[half_keys][2 * j + 1], w[half_keys][2 * j], 0x07060302u);
            }
            i32x4 *d0 = (i32x4 *)(vt + (2 * dp) * Q8_ATTN_VT_STRIDE + kb);
            i32x4 *d1 = (i32x4 *)(vt + (2 * dp + 1) * Q8_ATTN_VT_STRIDE + kb);
            d0[0] = r0[0];
            d0[1] = r0[1];
            d1[0] = r1[0];
            d1[1] = r1[1];
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's V^T stores are done
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_wave_barrier();
        // O^T += V^T P^T over four 16-key steps
#pragma unroll
        for (int j = 0; j < 4; j++) {
            float pv[8];
#pragma unroll
            for (int i = 0; i < 8; i++) pv[i] = st[j >> 1][8 * (j & 1) + i];
            f16x8 phi, plo;
            split_f16(pv, phi, plo);
#pragma unroll
            for (int dt = 0; dt < 2; dt++) {
                const uint16_t *row = vt + (32 * dt + r) * Q8_ATTN_VT_STRIDE + 16 * j + 4 * h;
                const uint2 lo4 = *(const uint2 *)row;
                const uint2 hi4 = *(const uint2 *)(row + 8);
                const i32x4 va = {(int)lo4.x, (int)lo4.y, (int)hi4.x, (int)hi4.y};
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, va), phi, o[dt], 0, 0, 0);
                o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, va), plo, o[dt], 0, 0, 0);
            }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // the tile's V^T reads are done before the next tile overwrites it
        __atomic_signal_fence(__ATOMIC_SEQ_CST);
        __builtin_amdgcn_wave_barrier();
    }
    // combine the two waves' partial softmax states (wave 1 -> LDS -> wave 0)
    if (wave == 1) {
        if (h == 0) {
            xm[r] = m;
            xl[r] = l;
        }
#pragma unroll
        for (int dt = 0; dt < 2; dt++)
#pragma unroll
            for (int v = 0; v < 16; v++) xo[32 * dt + 8 * (v >> 2) + 4 * h + (v & 3)][r] = o[dt][v];
    }
    __syncthreads();
    if (wave == 1) return;
    const float m1 = xm[r], l1 = xl[r];
    const float mt = fmaxf(m, m1);  // finite: key 0 is in tile 0 (wave 0) and visible to every query
    const float c0 = expf(m - mt);
    const float c1 = (m1 == -INFINITY) ? 0.0f : expf(m1 - mt);
    const float lt = l * c0 + l1 * c1;
    // res[dt][4g + e]: dim 32 dt + 8 g + 4 h + e of this lane's query (0 for
    // the padding queries of the last tile)
    float res[2][16];
#pragma unroll
    for (int dt = 0; dt < 2; dt++)
#pragma unroll
        for (int v = 0; v < 16; v++) {
            const int d = 32 * dt + 8 * (v >> 2) + 4 * h + (v & 3);
            res[dt][v] = qlive ? (o[dt][v] * c0 + xo[d][r] * c1) / lt : 0.0f;
        }
    if (a.out && qlive) {
        float *orow = a.out + ((size_t)qrow * a.n_head + head) * HD;
#pragma unroll
        for (int dt = 0; dt < 2; dt++)
#pragma unroll
            for (int g = 0; g < 4; g++)
                *(f32x4 *)(orow + 32 * dt + 8 * g + 4 * h) =
                    (f32x4){res[dt][4 * g], res[dt][4 * g + 1], res[dt][4 * g + 2], res[dt][4 * g + 3]};
    }
    if (a.xq) {
        // The head's 64 dims are Q8_0 blocks 2 head and 2 head + 1 of the
        // query's row, so this workgroup owns whole prepared units (32
        // queries x one block).  Unit half hh holds elements 8c + J[hh][q]
        // (J = {0,4,1,5}, {2,6,3,7}); this lane holds 8c + 4h + {0..3}, so
        // the pair (r, r + 32) trades two values per chunk, then quantizes
        // as q8_quantize does (quant_store, the block peak across the pair).
        const int nb = 2 * a.n_head;
#pragma unroll
        for (int dt = 0; dt < 2; dt++) {
            float e[4][4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float v0 = res[dt][4 * c], v1 = res[dt][4 * c + 1];
                const float v2 = res[dt][4 * c + 2], v3 = res[dt][4 * c + 3];
                const float p0 = __shfl_xor(v0, 32), p1 = __shfl_xor(v1, 32);
                const float p2 = __shfl_xor(v2, 32), p3 = __shfl_xor(v3, 32);
                e[0][c] = h == 0 ? v0 : p2;  // 8c + 0 | 8c + 2
                e[1][c] = h == 0 ? p0 : v2;  // 8c + 4 | 8c + 6
                e[2][c] = h == 0 ? v1 : p3;  // 8c + 1 | 8c + 3
                e[3][c] = h == 0 ? p1 : v3;  // 8c + 5 | 8c + 7
            }
            float peak = half_peak(e);
            peak = fmaxf(peak, __shfl_xor(peak, 32));
            quant_store(e, peak, a.xq, a.xs, (size_t)qt * nb + 2 * head + dt, 32 * h + r, h == 0, a.f16);
        }
    }
}

// ---------------------------------------------------------------------------
// Synthetic Q8_0 blocks (GGUF byte layout) from a counter-based generator:
// SplitMix64 of (seed, block).  q = byte % 255 - 127 (uniform over
// [-127, 127] up to a 1/255 bias), d = f16(|z| * scale_std / 127) with z a
// Box-Muller normal.  Deterministic for a seed; not the host generator's
// stream (the oracle checks against the bytes read back from the device).
// ---------------------------------------------------------------------------
static __device__ __forceinline__ unsigned long long splitmix64(unsigned long long z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

extern "C" __global__ __launch_bounds__(256) void q8_synth(Q8SynthArgs a) {
    for (long long b = (long long)blockIdx.x * blockDim.x + threadIdx.x; b < a.blocks;
         b += (long long)gridDim.x * blockDim.x) {
        uint8_t *dst = a.dst + b * Q8_BLOCK_BYTES;
        const unsigned long long h0 = splitmix64(a.seed ^ ((unsigned long long)b * 0xd1b54a32d192ed03ull));
        const float u1 = (float)((h0 >> 40) + 1) * (1.0f / 16777216.0f);  // (0, 1]
        const float u2 = (float)((h0 >> 16) & 0xffffffull) * (1.0f / 16777216.0f);
        const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.28318530718f * u2);
        const unsigned d = f16_bits(fabsf(z) * a.scale_std / 127.0f);
        dst[0] = (uint8_t)(d & 0xff);
        dst[1] = (uint8_t)(d >> 8);
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const unsigned long long h = splitmix64(h0 + (unsigned long long)(w + 1));
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const int q = (int)((h >> (8 * e)) & 0xffull) % 255 - 127;
                dst[2 + 8 * w + e] = (uint8_t)(signed char)q;
            }
        }
    }
}

extern "C" __global__ __launch_bounds__(64) void q8_advance(Q8AdvanceArgs a) {
    if (threadIdx.x == 0) a.position[0] += a.advance;
}
