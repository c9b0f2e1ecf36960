/*
 * q8_layout.h -- device data layout and kernel argument blocks, shared by the
 * gfx950 kernels (q8_kernels.hip) and the host runtime (q8_runtime.cpp).
 *
 * Q8_0 block (GGUF, apps/engine/src/quant.rs:8-9): [f16 LE scale d][32 x i8 q],
 * element value d*q.  A matrix is `rows x k`, row-major, k % 32 == 0.
 *
 * Device weight layout ("tile layout"), private to the residency cache exactly
 * as the reference's repacked planes are (apps/engine/src/cuda/mod.rs:2072-2089):
 *   rows are grouped in tiles of Q8_TILE_ROWS = 32 (the last tile zero-padded);
 *   for tile g and block b the 32x32 quants form one 1024-byte "unit" laid out
 *   in wave-lane order: lane L = 32*h + r (h = 0/1, r = row in tile) owns the
 *   16 bytes at unit + 16*L, holding half h of row r's block in the permuted
 *   element order Q8_PERM below;
 *   quants:  unit(g, b) = quants + (g*nb + b) * 1024
 *   scales:  f16 d of (row 32g+r, block b) at scales[(g*nb + b)*32 + r].
 * One 64-lane dwordx4 load therefore fetches a whole unit, which is both the
 * MFMA operand of v_mfma_i32_32x32x32_i8 and the GEMV's coalesced stream.
 *
 * Element permutation inside a block: byte p = 4*t + c of half h holds element
 * 8*c + Q8_J[h][t].  Dword t of half h is thus the AVX2 lane j = Q8_J[h][t]
 * across the four 8-wide chunks c (quant.rs:63-72), so one GPU lane can replay
 * the reference's per-lane FMA chain, and halves h=0/h=1 hold lanes {0,4,1,5}
 * and {2,6,3,7}: their pair sums are exactly the two halves of the reference's
 * horizontal_sum (quant.rs:80-91).  Both MFMA operands use the same
 * permutation, so the integer block dot is unchanged by it.
 *
 * Prepared activations (the quantized X of the prefill path, the reference's
 * opaque `Prepared`, apps/engine/src/cuda/mod.rs:1381-1410) use the same
 * lane-order units over tiles of Q8_TILE_TOKENS = 32 tokens:
 *   quants: unit(tt, b) = xq + (tt*nb + b) * 1024, lane L = 32*h + (t % 32)
 *   scales: f32 s of (token t, block b) at xs[((t/32)*nb + b)*32 + t%32]
 * Padding tokens (t >= n in the last tile) are written as zero.
 */
#ifndef Q8_LAYOUT_H
#define Q8_LAYOUT_H

#include <stdint.h>

#define Q8_BLOCK_ELEMS 32
#define Q8_BLOCK_BYTES 34
#define Q8_TILE_ROWS 32
#define Q8_TILE_TOKENS 32
#define Q8_UNIT_BYTES 1024
/* f16 form of a prepared activation unit: the same 16 values per lane as f16,
 * split in two 1 KB halves: half u holds, at 16*L, lane L's bytes 8u..8u+7
 * of the int8 unit as eight f16 (exact: |q| <= 127). */
#define Q8_UNIT_F16_BYTES 2048

/* f16-MFMA GEMM LDS: per K group, Q8_GEMM_H_STAGES ring buffers of
 * [TPW][2 blocks] f16 activation units, max(TPW, RW) * 64 f32 activation
 * scale slots, and per row wave two int8 weight units + 256 bytes of scales. */
#define Q8_GEMM_H_STAGES 3
#define Q8_GEMM_STAGED_BUF_BYTES(tpw, rw, unit) \
    ((tpw) * 2 * (unit) + ((tpw) > (rw) ? (tpw) : (rw)) * 64 * 4 + (rw) * (2 * Q8_UNIT_BYTES + 256))
#define Q8_GEMM_H_BUF_BYTES(tpw, rw) Q8_GEMM_STAGED_BUF_BYTES(tpw, rw, Q8_UNIT_F16_BYTES)
/* The int8-MFMA variant of the staged GEMM (q8_gemm_l): int8 activation units. */
#define Q8_GEMM_L_BUF_BYTES(tpw, rw) Q8_GEMM_STAGED_BUF_BYTES(tpw, rw, Q8_UNIT_BYTES)
#define Q8_GROUP_MAX 4 /* apps/engine/src/cuda/mod.rs:63 MMA_GROUP_MAX */
#define Q8_RIDER_MAX 4 /* weights one GEMM launch's cache riders read */

/* Q8_J[h][t]: the AVX2 lane held by dword t of half h. */
#define Q8_J_INIT {{0, 4, 1, 5}, {2, 6, 3, 7}}

static inline int q8_perm_element(int h, int p) {
    static const int J[2][4] = Q8_J_INIT;
    return 8 * (p & 3) + J[h][p >> 2];
}

/* GEMV exact mode parks each row's block values in LDS row-major, rows
 * Q8_GEMV_VROW(nb) floats apart: a multiple of four (16-byte reads) plus four,
 * so eight consecutive rows start in distinct bank groups. */
#define Q8_GEMV_VROW(nb) ((((nb) + 3) & ~3) + 4)
/* LDS floats after the GEMV's staging areas that absorb stores with nothing to write. */
#define Q8_GEMV_PAD_FLOATS 32

/* ---- kernel argument blocks (passed by value as the only kernel argument) ---- */

typedef struct {
    const uint8_t *src; /* GGUF Q8_0 bytes, rows * nb * 34 (inverse = 0) */
    uint8_t *dst;       /* GGUF Q8_0 bytes written back (inverse = 1) */
    uint8_t *quants;    /* tile layout quants */
    uint16_t *scales;   /* tile layout scales */
    int rows;
    int nb;
    int tiles;
    int inverse; /* 0: GGUF -> tile layout; 1: tile layout -> GGUF (test hook) */
} Q8RepackArgs;

/* Slice-major copy of a weight's quants, for the row-slice GEMVs: where a
 * weight's one-token GEMV runs in slices of RS = 8 or 16 rows, its quants are
 * also kept with each slice's bytes contiguous, so one 64-lane load reads
 * 1 KB in a single run:
 *   slice (g, s) of tile g, rows 32g + RS s .. + RS - 1, at
 *     slices + (g * (32 / RS) + s) * nb * RS * 32;
 *   block b of it at + b * RS * 32, row r' of half h at + (RS * h + r') * 16,
 * the 16 bytes the unit layout holds at unit(g, b) + 16 * (32 h + RS s + r').
 * Scales stay in the unit layout's plane.
 *
 * The paired copy of a gate/up pair (pair_tiles = T: gate tiles 0 .. T - 1
 * then up tiles T .. 2T - 1 in src, RS = 16): slice (t, s), s < 4, holds gate
 * rows 32t + 8s .. + 7 as its rows 0..7 and the same up rows as its rows
 * 8..15, at dst + (t * 4 + s) * nb * 512, block b at + b * 512, row r' of
 * half h at + (16 h + r') * 16, so one wave holds a gate row and its up row. */
typedef struct {
    const uint8_t *src; /* unit-layout quants, tiles * nb units */
    uint8_t *dst;       /* slice-major copy, the same byte count */
    int nb;
    int tiles;
    int rs;             /* rows per slice: 8 or 16 */
    int pair_tiles;     /* 0, or T: the paired copy of a gate/up pair (tiles = 2T, rs = 16) */
} Q8SliceArgs;

typedef struct {
    const uint8_t *quants;   /* resident weight, tile layout */
    const uint16_t *scales;
    const uint32_t *tokens;  /* n row ids; an id >= rows yields a zero row */
    float *out;              /* n rows of nb*32 f32 */
    int n;
    int nb;
    int rows;
} Q8EmbedArgs;

typedef struct {
    const uint8_t *quants;
    const uint16_t *scales;
    float *y;          /* rows f32 (n = 1) */
    const float *bias; /* residual added in the epilogue, or null */
    int rows;
    int tile_begin; /* first global tile index of this member */
} Q8GemvMember;

typedef struct {
    Q8GemvMember m[Q8_GROUP_MAX];
    int members;
    int total_tiles;
    const float *x; /* k f32 */
    int nb;
    int waves_per_tile;  /* W: waves splitting one tile's blocks */
    int pairs_per_wave;  /* ceil(ceil(nb/2) / W) */
    int silu_pair;       /* 1: m[0] = gate, m[1] = up; writes silu(g)*u to m[0].y */
    int kslices;         /* S: workgroups splitting one tile's block pairs */
    int pairs_per_slice; /* ceil(ceil(nb/2) / S) */
    float *scratch;      /* S > 1: partial results shared between a tile's workgroups */
    unsigned *counters;  /* S > 1: arrivals per tile, zero between launches */
    unsigned long long slice_magic; /* ceil(2^32 / S): workgroup / S = (workgroup * magic) >> 32 */
    const float *norm_w; /* non-null (multi-matrix kernels): x is rmsnorm(x) * norm_w, folded in */
    float norm_eps;
    /* RoPE + KV append epilogue (multi-matrix kernels; members q, k, v):
     * non-null rope_pos turns it on.  q rows rotated into m[0].y; k rotated
     * and v copied as f16 into kcache / vcache [capacity][rows] at *rope_pos. */
    const int *rope_pos;
    const float *rope_freq; /* n_rot / 2 frequencies base^(-2i/n_rot), from the host */
    uint16_t *kcache;
    uint16_t *vcache;
    int head_dim, n_rot, capacity;
    /* Attention split combine as the prologue (the q8_gemvc_* kernels, one
     * matrix; head dim Q8_ATTN_HEAD_DIM, at most Q8_ATTN_COMBINE_MAX splits,
     * one float4 of x per thread): x is
     * sum_s acc_s * e_s / sum_s sum_s * e_s with e_s = exp(max_s - max), per
     * head, from the partials q8_attn_decode leaves in defer mode. */
    const float *attn_acc; /* [heads][splits][head_dim] */
    const float *attn_ms;  /* [heads][splits][2]: max, sum */
    int attn_splits;
    /* Row-slice kernels: 1 = the slices of a tile are workgroups 8 apart
     * (one XCD under round-robin dispatch; the grid is padded to whole
     * groups of eight tiles), 0 = consecutive workgroups. */
    int xcd_order;
    /* Greedy-argmax partials of a one-matrix tile-kernel launch (the lm_head):
     * non-null, each 32-row tile writes its best (value, lowest index) over
     * its non-NaN outputs to [tile], or index 0xffffffff if it has none. */
    float *amax_value;
    unsigned *amax_index;
    /* The quantized-x kernels (q8_gemv_q8x_*): tokens 1..NT of x, k floats
     * apart; y and bias [tokens][rows]. */
    int tokens;
} Q8GemvArgs;

/* float4s per thread of the 256-thread row RMSNorm (k <= 1024 * this). */
#define Q8_NORM_ROW_VEC 8
/* The same for the norm folded into the group row-slice GEMVs, which hold
 * these x float4s in registers across their weight loads: k <= 1024 * this. */
#define Q8_RSG_NORM_VEC 3
// floats per block of the normalized row q8_rmsnorm_row stages in LDS for its
// prepared output (a block's 32 plus a pad against bank conflicts)
#define Q8_NORM_LDS_PITCH 36

typedef struct {
    const float *x;    /* [n][k] f32 (mode 0) */
    const float *gate; /* [n][k] f32 (mode 1) */
    const float *up;   /* [n][k] f32 (mode 1) */
    uint8_t *xq;       /* prepared quants */
    float *xs;         /* prepared scales */
    int n;
    int nb;
    int ttiles;
    int mode; /* 0: quantize x; 1: quantize silu(gate) * up */
    int f16;  /* 1: write the quants as f16 units (Q8_UNIT_F16_BYTES) for the f16-MFMA GEMM */
} Q8QuantArgs;

typedef struct {
    const uint8_t *quants;
    const uint16_t *scales;
    float *y;          /* [n][rows] f32 */
    const float *bias; /* [n][rows] residual, or null */
    int rows;
    int tile_begin; /* first global row tile of this member */
} Q8GemmMember;

typedef struct {
    Q8GemmMember m[Q8_GROUP_MAX];
    int members;
    int total_rtiles;
    const uint8_t *xq;
    const float *xs;
    int n;
    int nb;
    int ttiles;
    int twaves;     /* waves along the tokens per workgroup (each TPW token tiles) */
    int tgroups;    /* ceil(ttiles / (twaves * TPW)) */
    int nwg;        /* workgroups launched (total_rtiles * tgroups * kslices) */
    int xcd_remap;  /* 1: map workgroups so one row tile's token groups share an XCD */
    int kslices;          /* S: workgroups splitting the block pairs of one output tile group */
    int pairs_per_slice;  /* ceil(ceil(nb/2) / S) */
    int pairs_per_wave;   /* ceil(pairs_per_slice / kwaves) */
    float *scratch;       /* S > 1: [rtiles][ttiles][S][64][16] partial tiles */
    unsigned *counters;   /* S > 1: arrivals per (row tile, token group), zero between launches */
    int rwaves;           /* f16 GEMM: row-tile waves per workgroup sharing the LDS-staged activations */
    uint8_t *oq;          /* q8_gemm_silu: prepared Q8_0 output of silu(gate) * up (quants) */
    float *os;            /* q8_gemm_silu: its scales */
    int of16;             /* q8_gemm_silu: 1 = f16 prepared units */
    /* RoPE + KV append epilogue of a q, k, v prompt group (members 0, 1, 2;
     * non-null rope_pos turns it on): q rows rotated into m[0].y; k rotated
     * and v copied as f16 into kcache / vcache [capacity][rows] at rows
     * *rope_pos + token (nothing for tokens outside the cache, whose q stays
     * unrotated). */
    const int *rope_pos;
    const float *rope_freq; /* n_rot / 2 frequencies base^(-2i/n_rot), from the host */
    uint16_t *kcache;
    uint16_t *vcache;
    int head_dim, n_rot, capacity;
    /* Cache riders (q8_gemm_s* and q8_gemm_silu): `riders` extra workgroups
     * (a multiple of 8) that only read the weights in rider_q / rider_s once,
     * in address order, and exit, so the weights sit in the L2 and the
     * Infinity Cache when compute waves read them.  rider_first: the riders
     * are the grid's first workgroups (compute workgroup w is riders + w),
     * else its last (w is w).  rider_nt: non-temporal reads. */
    int riders;
    int rider_first;
    int rider_nt;
    int rider_count;                         /* weights in rider_q / rider_s */
    const uint8_t *rider_q[Q8_RIDER_MAX];    /* quants of a resident weight */
    const uint16_t *rider_s[Q8_RIDER_MAX];   /* its scales */
    unsigned rider_units[Q8_RIDER_MAX];      /* row tiles x blocks of it */
} Q8GemmArgs;

typedef struct {
    const float *x;
    float *act;
    const float *gate;
    const float *up;
    long long len;
} Q8EltArgs;

typedef struct {
    const float *x;    /* [n][k] f32 rows */
    const float *w;    /* [k] norm weight */
    float *out;        /* [n][k] f32 norm, or null */
    uint8_t *xq;       /* prepared quants (format by f16), or null */
    float *xs;         /* prepared scales */
    int n;
    int rows_launched; /* n, or the token-tile boundary when quantizing (padding rows zero) */
    int k;
    int f16;
    float eps;
} Q8NormArgs;

typedef struct {
    const uint8_t *src;
    uint8_t *dst;
    long long bytes;
    int blocks; /* workgroups launched */
} Q8CopyArgs;

typedef struct {
    const float *values;
    long long len;
    float *part_value;     /* per-workgroup best value */
    unsigned *part_index;  /* per-workgroup best index (UINT32_MAX = none) */
    unsigned *result;      /* final index */
    int parts;
    int stage; /* 0: per-workgroup; 1: combine parts */
} Q8ArgmaxArgs;

/* ---- decoder support: rotary embedding, f16 KV cache, attention ----
 * KV cache layout (one layer): f16 [capacity][n_kv * head_dim], position-major,
 * as the reference's device cache (gpu.cu kv_append 506-519). */
#define Q8_ATTN_HEAD_DIM 64 /* the head width the attention kernels are built for */
#define Q8_ATTN_COMBINE_MAX 8 /* most attention splits a GEMV prologue combines */
#define Q8_ATTN_TILE 64     /* prefill: queries and keys per tile */

typedef struct {
    float *q;            /* [n][n_head][head_dim] f32, rotated in place */
    const float *k;      /* [n][n_kv][head_dim] f32 */
    const float *v;      /* [n][n_kv * head_dim] f32 */
    uint16_t *kcache;    /* f16 cache */
    uint16_t *vcache;
    const int *position; /* device: cache position of the first of the n tokens */
    const float *freq;   /* n_rot / 2 rotation frequencies base^(-2i/n_rot), computed on the host */
    int n, n_head, n_kv, head_dim, n_rot, capacity;
} Q8RopeArgs;

typedef struct {
    const float *q;         /* [n_head][head_dim] (one token) */
    const uint16_t *kcache;
    const uint16_t *vcache;
    float *part_acc;        /* [n_head][splits][head_dim] unnormalised sums */
    float *part_ms;         /* [n_head][splits][2]: max, sum */
    float *out;             /* [n_head][head_dim] */
    unsigned *counters;     /* splits > 1: arrivals per head, zero between launches */
    const int *position;    /* device: the token's cache position; it sees position + 1 keys */
    int n_head, n_kv, splits, capacity;
    float scale;
    int defer;              /* 1: write every split's partials (also at splits = 1), no combine */
} Q8AttnDecodeArgs;

typedef struct {
    const float *q;         /* [n][n_head][head_dim] rotated queries */
    const uint16_t *kcache;
    const uint16_t *vcache;
    float *out;             /* [n][n_head][head_dim], or null */
    const int *position;    /* device: cache position of query 0 */
    int n, n_head, n_kv, capacity, qtiles;
    float scale;
    uint8_t *xq;            /* non-null: the output also as prepared Q8_0 (units, as q8_quantize writes them) */
    float *xs;              /* its block scales */
    int f16;                /* 1: f16 prepared units */
} Q8AttnPrefillArgs;

typedef struct {
    uint8_t *dst;           /* GGUF Q8_0 blocks */
    long long blocks;
    unsigned long long seed;
    float scale_std;        /* d = f16(|N(0, scale_std)| / 127) */
} Q8SynthArgs;

typedef struct {
    int *position;          /* device: advanced by `advance` */
    int advance;
} Q8AdvanceArgs;


#endif
