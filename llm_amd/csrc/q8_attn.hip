// q8_attn.hip -- decoder support kernels around the Q8_0 matmuls, for the
// synthetic decoder and the decode graph (included by q8_kernels.hip, one code
// object):
//   q8_rope_append   rotary embedding of q and k, k and v narrowed to the f16
//                    KV cache                     (gpu.cu rope_append 525-581, ops.rs:152-166)
//   q8_attn_decode   one token against the cache, positions split over
//   q8_attn_combine  workgroups, then combined    (gpu.cu attention_split 649-733, combine 735-762)
//   q8_attn_prefill  causal attention of n tokens, 64 x 64 tiles, online softmax
//                                                 (compute.rs attend_host 1075-1126)
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
static __device__ __forceinline__ unsigned f16_bits(float x) {
    return (unsigned)__builtin_bit_cast(unsigned short, (_Float16)x);
}

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
// Decode attention for one token: workgroup (head, split) of 256 threads takes
// positions [begin, end) of the position + 1 visible ones.
//   scores: a thread per position, dot(q, k) over the 64 dims in order (q from
//           LDS, broadcast), then * scale (the reference's dot * scale);
//   softmax: workgroup max, exp(s - max) in LDS, workgroup sum;
//   values: lane = dimension, the four waves take every fourth position.
// splits == 1 writes acc / sum; otherwise the unnormalised (acc, max, sum) go
// to the partials and q8_attn_combine rescales them by exp(max_s - max), the
// same arithmetic as one softmax summed in another order (gpu.cu:735-762).
// Dynamic LDS: ceil(capacity / splits) floats of weights.
// ---------------------------------------------------------------------------
static __device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) v = fmaxf(v, __shfl_xor(v, m));
    return v;
}
static __device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

extern "C" __global__ __launch_bounds__(256) void q8_attn_decode(Q8AttnDecodeArgs a) {
    extern __shared__ __attribute__((aligned(16))) float wsm[];
    __shared__ __attribute__((aligned(16))) float qs[Q8_ATTN_HEAD_DIM];
    __shared__ float red[8];
    __shared__ float part[4][Q8_ATTN_HEAD_DIM];
    constexpr int HD = Q8_ATTN_HEAD_DIM;
    const int head = blockIdx.x / a.splits;
    const int split = blockIdx.x - head * a.splits;
    const int kvh = head / (a.n_head / a.n_kv);
    const int kv_dim = a.n_kv * HD;
    const int visible = min(*a.position + 1, a.capacity);
    const int per = (visible + a.splits - 1) / a.splits;
    const int begin = split * per;
    const int end = min(begin + per, visible);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    if (tid < HD) qs[tid] = a.q[(size_t)head * HD + tid];
    __syncthreads();

    float mx = -INFINITY;
    for (int p = begin + tid; p < end; p += 256) {
        const uint16_t *kr = a.kcache + (size_t)p * kv_dim + kvh * HD;
        float dot = 0.0f;
#pragma unroll
        for (int c = 0; c < HD / 8; c++) {
            const i32x4 u = *(const i32x4 *)(kr + 8 * c);
            const f32x4 q0 = *(const f32x4 *)(qs + 8 * c);
            const f32x4 q1 = *(const f32x4 *)(qs + 8 * c + 4);
            dot = __builtin_fmaf(q0[0], f16_to_f32((unsigned)u[0] & 0xffffu), dot);
            dot = __builtin_fmaf(q0[1], f16_to_f32((unsigned)u[0] >> 16), dot);
            dot = __builtin_fmaf(q0[2], f16_to_f32((unsigned)u[1] & 0xffffu), dot);
            dot = __builtin_fmaf(q0[3], f16_to_f32((unsigned)u[1] >> 16), dot);
            dot = __builtin_fmaf(q1[0], f16_to_f32((unsigned)u[2] & 0xffffu), dot);
            dot = __builtin_fmaf(q1[1], f16_to_f32((unsigned)u[2] >> 16), dot);
            dot = __builtin_fmaf(q1[2], f16_to_f32((unsigned)u[3] & 0xffffu), dot);
            dot = __builtin_fmaf(q1[3], f16_to_f32((unsigned)u[3] >> 16), dot);
        }
        const float s = dot * a.scale;
        wsm[p - begin] = s;
        mx = fmaxf(mx, s);
    }
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float sum = 0.0f;
    for (int p = begin + tid; p < end; p += 256) {
        const float e = expf(wsm[p - begin] - mx);
        wsm[p - begin] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    if (lane == 0) red[4 + wave] = sum;
    __syncthreads();  // weights and partial sums complete
    sum = (red[4] + red[5]) + (red[6] + red[7]);

    float acc = 0.0f;
    const uint16_t *vcol = a.vcache + kvh * HD + lane;
    for (int p = begin + wave; p < end; p += 4)
        acc = __builtin_fmaf(wsm[p - begin], f16_to_f32(vcol[(size_t)p * kv_dim]), acc);
    part[wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
        const float tot = (part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]);
        if (a.splits == 1) {
            a.out[(size_t)head * HD + lane] = tot / sum;
        } else {
            const size_t slot = (size_t)head * a.splits + split;
            a.part_acc[slot * HD + lane] = tot;
            if (lane == 0) {
                a.part_max[slot] = mx;
                a.part_sum[slot] = sum;
            }
        }
    }
}

extern "C" __global__ __launch_bounds__(64) void q8_attn_combine(Q8AttnDecodeArgs a) {
    constexpr int HD = Q8_ATTN_HEAD_DIM;
    const int head = blockIdx.x;
    const int d = threadIdx.x;
    const size_t base = (size_t)head * a.splits;
    float gmax = -INFINITY;
    for (int s = 0; s < a.splits; s++) gmax = fmaxf(gmax, a.part_max[base + s]);
    float num = 0.0f, den = 0.0f;
    for (int s = 0; s < a.splits; s++) {
        const float f = expf(a.part_max[base + s] - gmax);  // an empty split has max -inf: f = 0
        den += a.part_sum[base + s] * f;
        num += a.part_acc[(base + s) * HD + d] * f;
    }
    a.out[(size_t)head * HD + d] = num / den;
}

// ---------------------------------------------------------------------------
// Prefill attention: n query tokens at cache positions start .. start+n-1, each
// seeing keys 0 .. its own position (causal).  Workgroup = (head, 64-query
// tile), 256 threads; thread (qi, kj) = (tid / 16, tid % 16) owns queries
// 4qi..4qi+3 and, per 64-key tile, keys 4kj..4kj+3 of the scores and dims
// 4kj..4kj+3 of the output.  LDS: Q^T and K^T ([dim][row], so a thread's four
// rows are one 16-byte read), V and P^T, 64 KB.  Online softmax per query row
// (running max and sum across key tiles, the 16 lanes of a row meeting by
// xor shuffles), f32 throughout with f16 keys and values widened exactly.
// Heavier (later) query tiles are launched first.
// ---------------------------------------------------------------------------
extern "C" __global__ __launch_bounds__(256) void q8_attn_prefill(Q8AttnPrefillArgs a) {
    extern __shared__ __attribute__((aligned(16))) float psm_attn[];
    constexpr int HD = Q8_ATTN_HEAD_DIM;
    constexpr int T = Q8_ATTN_TILE;
    float *Qt = psm_attn;            // [HD][T]
    float *Kt = Qt + HD * T;         // [HD][T]
    float *Vs = Kt + HD * T;         // [T][HD]
    float *Pt = Vs + T * HD;         // [T][T]  (key, query)
    const int head = blockIdx.x / a.qtiles;
    const int qt = a.qtiles - 1 - (blockIdx.x - head * a.qtiles);
    const int kvh = head / (a.n_head / a.n_kv);
    const int kv_dim = a.n_kv * HD;
    const int start = *a.position;
    const int t0 = qt * T;
    const int tid = threadIdx.x;
    const int qi = tid >> 4;
    const int kj = tid & 15;
    {
        const int i = tid >> 2, qq = tid & 3;
        const int t = t0 + i;
        f32x4 v[4] = {};
        if (t < a.n) {
            const f32x4 *src = (const f32x4 *)(a.q + ((size_t)t * a.n_head + head) * HD + 16 * qq);
#pragma unroll
            for (int u = 0; u < 4; u++) v[u] = src[u];
        }
#pragma unroll
        for (int e = 0; e < 16; e++) Qt[(16 * qq + e) * T + i] = v[e >> 2][e & 3];
    }
    float m[4], l[4], o[4][4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        m[r] = -INFINITY;
        l[r] = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; c++) o[r][c] = 0.0f;
    }
    const int last_q = min(t0 + T - 1, a.n - 1);
    const int kend = min(start + last_q + 1, a.capacity);  // keys [0, kend)
    for (int p0 = 0; p0 < kend; p0 += T) {
        __syncthreads();  // the previous tile's readers are done (and Qt is complete)
        {
            const int j = tid >> 2, qq = tid & 3;
            const int p = p0 + j;
            i32x4 kw[2] = {}, vw[2] = {};
            if (p < kend) {
                const i32x4 *ks = (const i32x4 *)(a.kcache + (size_t)p * kv_dim + kvh * HD + 16 * qq);
                const i32x4 *vsrc = (const i32x4 *)(a.vcache + (size_t)p * kv_dim + kvh * HD + 16 * qq);
                kw[0] = ks[0];
                kw[1] = ks[1];
                vw[0] = vsrc[0];
                vw[1] = vsrc[1];
            }
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const unsigned bits = ((unsigned)kw[e >> 3][(e >> 1) & 3] >> (16 * (e & 1))) & 0xffffu;
                Kt[(16 * qq + e) * T + j] = f16_to_f32(bits);
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                f32x4 w;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int f = 4 * u + e;
                    w[e] = f16_to_f32(((unsigned)vw[f >> 3][(f >> 1) & 3] >> (16 * (f & 1))) & 0xffffu);
                }
                *(f32x4 *)(Vs + j * HD + 16 * qq + 4 * u) = w;
            }
        }
        __syncthreads();
        float s[4][4];
#pragma unroll
        for (int r = 0; r < 4; r++)
#pragma unroll
            for (int c = 0; c < 4; c++) s[r][c] = 0.0f;
#pragma unroll 8
        for (int d = 0; d < HD; d++) {
            const f32x4 qv = *(const f32x4 *)(Qt + d * T + 4 * qi);
            const f32x4 kv = *(const f32x4 *)(Kt + d * T + 4 * kj);
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int c = 0; c < 4; c++) s[r][c] = __builtin_fmaf(qv[r], kv[c], s[r][c]);
        }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int qa = start + t0 + 4 * qi + r;
            float tm = -INFINITY;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int p = p0 + 4 * kj + c;
                s[r][c] = (p <= qa) ? s[r][c] * a.scale : -INFINITY;
                tm = fmaxf(tm, s[r][c]);
            }
#pragma unroll
            for (int sh = 1; sh < 16; sh <<= 1) tm = fmaxf(tm, __shfl_xor(tm, sh));
            // key 0 is in the first tile and visible to every query, so m is
            // finite from the first tile on and mn never -inf
            const float mn = fmaxf(m[r], tm);
            const float corr = expf(m[r] - mn);
            float rs = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                s[r][c] = expf(s[r][c] - mn);
                rs += s[r][c];
            }
#pragma unroll
            for (int sh = 1; sh < 16; sh <<= 1) rs += __shfl_xor(rs, sh);
            l[r] = l[r] * corr + rs;
            m[r] = mn;
#pragma unroll
            for (int c = 0; c < 4; c++) o[r][c] *= corr;
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const f32x4 pc = {s[0][c], s[1][c], s[2][c], s[3][c]};
            *(f32x4 *)(Pt + (4 * kj + c) * T + 4 * qi) = pc;
        }
        __syncthreads();
#pragma unroll 8
        for (int k = 0; k < T; k++) {
            const f32x4 pv = *(const f32x4 *)(Pt + k * T + 4 * qi);
            const f32x4 vv = *(const f32x4 *)(Vs + k * HD + 4 * kj);
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int c = 0; c < 4; c++) o[r][c] = __builtin_fmaf(pv[r], vv[c], o[r][c]);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int t = t0 + 4 * qi + r;
        if (t < a.n) {
            const f32x4 res = {o[r][0] / l[r], o[r][1] / l[r], o[r][2] / l[r], o[r][3] / l[r]};
            *(f32x4 *)(a.out + ((size_t)t * a.n_head + head) * HD + 4 * kj) = res;
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
