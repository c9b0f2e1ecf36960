/*
 * q8decoder.h -- the decoder around the Q8_0 matmul path of libq8mi.so: the
 * support operations a llama-style decoder step needs beside the matmuls
 * (rotary embedding into an f16 KV cache, attention, device-side token
 * feedback) and a synthetic decoder that runs them with the matmuls in situ.
 *
 * Positions are read from device memory (an int the caller allocates with
 * q8_alloc), so a captured step replays at any position, as the reference's
 * captured decode steps do (model.rs:676-731: "only the position changes, and
 * the kernels read that from device memory").
 */
#ifndef Q8DECODER_H
#define Q8DECODER_H

#include <stddef.h>
#include <stdint.h>

#include "q8mi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- support operations ---- */

/* Rotary embedding and KV append: Compute::rope_append (compute.rs:743-797),
 * kernel rope_append (gpu.cu:525-581) with the host path's semantics
 * (ops.rs:152-166 rotation of consecutive pairs, kv_append copying every
 * dimension).  q [n][n_head][head_dim] is rotated in place; k [n][n_kv][head_dim]
 * rotated and v [n][n_kv*head_dim] copied are rounded to f16 into the caches
 * (f16 [capacity][n_kv*head_dim]) at rows *position + t.  Pairs i < n_rot/2
 * rotate by position * base^(-2i/n_rot); the others are copied.  Rows at or
 * beyond `capacity` are not written (the caller checks the context first). */
int q8_rope_append(q8_ctx *ctx, q8_dptr q, size_t q_offset, q8_dptr k, size_t k_offset, q8_dptr v,
                   size_t v_offset, q8_dptr kcache, q8_dptr vcache, int n, int n_head, int n_kv, int head_dim,
                   int n_rot, float base, int capacity, q8_dptr position);

/* Causal attention of n query rows at cache positions *position + t, each
 * seeing cache rows 0 ..= its own position: Compute::attend (compute.rs,
 * attend_host 1075-1126 semantics: scores = dot(q, k) * scale, softmax, sum of
 * weighted values), with f16 keys and values as the reference's device cache.
 * n == 1 runs the split decode kernel (attention_split + attention_combine,
 * gpu.cu:649-762) over `splits` workgroups per head: one split reads its
 * positions in 1024-row chunks, more splits in 256-row chunks (so about
 * visible / 256 splits keep each to one chunk); n > 1 the tiled prefill
 * kernel (`splits` ignored).  head_dim must be 64; n_head a multiple of n_kv. */
int q8_attention(q8_ctx *ctx, q8_dptr q, size_t q_offset, q8_dptr kcache, q8_dptr vcache, q8_dptr out,
                 size_t out_offset, int n, int n_head, int n_kv, int head_dim, int capacity, float scale,
                 q8_dptr position, int splits);

/* q8_attention for a prompt (n >= 2) with its output written straight as
 * prepared Q8_0 activations (as q8_prepare of the f32 rows would leave them,
 * bit for bit, in the context's activation workspace: valid until the next
 * preparation), for the output projection's GEMM.  Each attention workgroup
 * owns whole Q8_0 blocks (a head's 64 dims are two), so it quantizes its own
 * rows; the f32 rows are not written.  The reference runs attend, then
 * prepare (model.rs dense_attention). */
int q8_attention_prepare(q8_ctx *ctx, q8_dptr q, size_t q_offset, q8_dptr kcache, q8_dptr vcache, int n, int n_head,
                         int n_kv, int head_dim, int capacity, float scale, q8_dptr position, q8_prepared *out);

/* q8_attention for one token (n = 1) followed by q8_matmul of its output
 * through `wo` with y as the residual (y[0 .. wo->out) += wo . attn):
 * the reference's attend then matmul_add of the output projection (model.rs
 * dense_attention).  The splits' partials go straight to the GEMV, whose
 * prologue combines them (the arithmetic of the in-launch combine), so the
 * attention output is never written and no workgroup waits for another; the
 * result is bit-identical to the two calls with the same `splits`.  Shapes
 * the GEMV cannot fold (more than 8 splits, a K split) run the two calls.
 * wo->k must be n_head * head_dim. */
int q8_attention_matmul_add(q8_ctx *ctx, q8_dptr q, size_t q_offset, q8_dptr kcache, q8_dptr vcache, int n_head,
                            int n_kv, int head_dim, int capacity, float scale, q8_dptr position, int splits,
                            const q8_weight *wo, q8_dptr y, size_t y_offset);

/* q8_embeddings with the token ids already in device memory (u32), so the
 * lookup can sit inside a captured step.  An id >= the vocabulary yields a
 * zero row (the host-side check of q8_embeddings cannot run here). */
int q8_embeddings_device(q8_ctx *ctx, const q8_weight *weight, q8_dptr tokens, size_t n, q8_dptr out,
                         size_t out_offset);

/* q8_argmax writing the index to device memory (u32 at `result`) instead of
 * returning it: the greedy token fed back to the next step on the device. */
int q8_argmax_device(q8_ctx *ctx, q8_dptr values, size_t offset, size_t len, q8_dptr result);

/* The output norm, lm_head and greedy choice of a decode step (model.rs
 * output_norm + lm_head, 806-832; sampler.rs:167-175 argmax): logits =
 * weight . (rmsnorm(x) * norm_weight) (norm_weight null: no norm) written to
 * `logits`, and the first index of their maximum (NaN never wins; a NaN at
 * index 0 gives 0) written as a u32 to device memory at `result`.  The norm
 * (q8_rmsnorm's kernel), then the GEMV, whose epilogue also leaves each
 * 32-row tile's best candidate, then one workgroup that picks among them
 * (q8_argmax's second stage): the argmax never reads the logits back (shapes
 * whose GEMV splits K take the two-stage argmax).  Bit-identical to
 * q8_rmsnorm + q8_matmul + q8_argmax_device with "gemv.exact" = 1, and in
 * the default block order wherever q8_matmul also runs the tile kernel (the
 * lm_head shapes: more row tiles than CUs); where q8_matmul takes row slices
 * instead, the two orders agree within 2e-6 + 1e-5 |ref|. */
int q8_norm_lm_head_argmax(q8_ctx *ctx, const float *norm_weight, float eps, const q8_weight *weight, q8_dptr x,
                           size_t x_offset, q8_dptr logits, size_t logits_offset, q8_dptr result);

/* *position += by, on the device (the end of a captured step). */
int q8_advance_position(q8_ctx *ctx, q8_dptr position, int by);

/* q8_rmsnorm (one row) followed by q8_matmul_decode_group on its output, with
 * the norm folded into the GEMV launch: every workgroup recomputes the row's
 * sum of squares exactly as the row norm kernel does, and the normalized row
 * is never written.  With option "gemv.exact" = 1 each workgroup waits for
 * the scale and multiplies x by it before the dot products, so the results
 * are bit-identical to the two calls; in the default block order it stages
 * x * weight and multiplies the row sums by the scale instead (no wait
 * inside the launch; within f32 rounding of the two calls).
 * The reference runs the two steps apart (model.rs decode step: rmsnorm then
 * matmul_decode_group); shapes whose GEMV needs a K split take the two-step
 * path on the device.  `norm_weight` is a host f32[k] made resident like
 * q8_rmsnorm's. */
int q8_norm_matmul_decode_group(q8_ctx *ctx, const float *norm_weight, float eps, const q8_group_entry *group,
                                int count, q8_dptr x, size_t x_offset, int k);

/* The attention input of one decode token in one launch: q8_rmsnorm, the
 * q, k, v decode GEMV group over its output, and q8_rope_append on the
 * results, with the norm folded into the GEMV (as q8_norm_matmul_decode_group)
 * and the rotation and KV append in its epilogue -- bit-identical to those
 * three calls with "gemv.exact" = 1, within f32 rounding of them otherwise
 * (the folded norm's two modes).  q [n_head*head_dim] f32 receives the rotated query; k and v
 * go only into the f16 caches, at row *position (nothing is appended, and q
 * is not rotated, at a position outside the cache).  The reference runs the
 * steps as separate kernels (model.rs dense_attention: rmsnorm,
 * matmul_decode_group, rope_append). */
int q8_norm_qkv_rope(q8_ctx *ctx, const float *norm_weight, float eps, const q8_weight *wq, const q8_weight *wk,
                     const q8_weight *wv, q8_dptr x, size_t x_offset, q8_dptr q, size_t q_offset, q8_dptr kcache,
                     q8_dptr vcache, int n_head, int n_kv, int head_dim, int n_rot, float base, int capacity,
                     q8_dptr position);

/* The prompt counterpart of q8_norm_qkv_rope: q8_matmul_prompt_group of the
 * q, k, v weights over prepared activations (n tokens) with q8_rope_append in
 * the GEMM's epilogue -- bit-identical to those two calls.  q [n][n_head *
 * head_dim] f32 receives the rotated queries; k and v go only into the f16
 * caches, at rows *position + t (tokens at or past capacity append nothing and
 * leave their q unrotated).  The reference runs the steps as separate kernels
 * (model.rs dense_attention: matmul_prompt_group, rope_append). */
int q8_prompt_qkv_rope(q8_ctx *ctx, const q8_weight *wq, const q8_weight *wk, const q8_weight *wv,
                       const q8_prepared *prepared, int n, q8_dptr q, size_t q_offset, q8_dptr kcache, q8_dptr vcache,
                       int n_head, int n_kv, int head_dim, int n_rot, float base, int capacity, q8_dptr position);

/* q8_rmsnorm (one row) followed by q8_gate_up_silu at n = 1, folded the same
 * way (bit-identical to the two calls with "gemv.exact" = 1):
 * act = silu(gate . xn) * (up . xn), xn = rmsnorm(x) * norm_weight. */
int q8_norm_gate_up_silu(q8_ctx *ctx, const float *norm_weight, float eps, const q8_weight *gate,
                         const q8_weight *up, q8_dptr x, size_t x_offset, q8_dptr act, size_t act_offset);

/* A random-init out x k Q8_0 weight generated on the device from `seed`
 * (quants uniform in [-127, 127], scales f16(|N(0, scale_std)| / 127)),
 * owned by the context until q8_weight_release or q8_close.  No counterpart in
 * the reference, whose weights always come from a GGUF; q8_weight_export reads
 * it back for the CPU checks. */
int q8_weight_synthetic(q8_ctx *ctx, int k, int out, uint64_t seed, float scale_std, const q8_weight **weight);

/* ---- the synthetic decoder ---- */

typedef struct q8_decoder q8_decoder;

/* Geometry of a dense llama-style decoder (Config, model.rs:20-180): separate
 * q, k, v projections, SiLU-gated feed-forward, RMSNorm before each block.
 * The output projection is the token embedding (a file without
 * `output.weight`) or a matrix of its own (a file with one): the two cases
 * model.rs:519-524 loads. */
typedef struct {
    int n_layer, n_embd, n_ff, n_head, n_head_kv, head_dim, n_rot, n_vocab;
    int capacity;   /* KV cache positions */
    int max_batch;  /* most tokens one forward takes (<= Q8_MAX_TOKENS) */
    float eps, rope_base;
    int untied_output; /* 0: the embedding is the output head; 1: a random output.weight of its own */
    float embd_std;    /* scale std of the random embedding rows (0: 0.02, as every other matrix) */
} q8_decoder_config;

enum { Q8_DEC_Q = 0, Q8_DEC_K, Q8_DEC_V, Q8_DEC_O, Q8_DEC_GATE, Q8_DEC_UP, Q8_DEC_DOWN, Q8_DEC_OUTPUT };

/* Random-init weights on the device (q8_weight_synthetic, one seed per
 * matrix), norm weights near 1, an f16 KV cache of `capacity` positions.
 * Creation also plans the context's workspaces for the decoder's largest
 * pass (q8_workspace_plan: max_batch tokens, the widest row, every attention
 * split count up to `capacity`), builds the rotation table, makes the norm
 * weights resident and reserves the pinned token buffer of q8_decoder_generate,
 * as the reference's Workspace is sized once per context (workspace.rs:171-342):
 * forwards and steps within the configuration allocate nothing. */
int q8_decoder_create_synthetic(q8_ctx *ctx, const q8_decoder_config *config, uint64_t seed, q8_decoder **out);
void q8_decoder_destroy(q8_decoder *dec);
/* Empty the cache: the next forward starts at position 0 (KvCache::reset). */
int q8_decoder_reset(q8_decoder *dec);
int q8_decoder_position(const q8_decoder *dec, int *position);

/* Model::forward (model.rs:652-673) for n prompt tokens at the current
 * position, then the greedy choice (sampler.rs:167-175) on the last row's
 * logits: *next is the argmax.  The pass is captured into a graph keyed by n
 * the second time that n runs and replayed after that.  Errors: an id outside
 * the vocabulary (Q8_ERR_INVALID), a full context (Q8_ERR_UNSUPPORTED). */
int q8_decoder_forward(q8_decoder *dec, const uint32_t *tokens, int n, uint32_t *next);

/* `steps` greedy decode steps (Model::forward_decode, model.rs:682-731): each
 * step feeds the previous argmax, which stays on the device, and the steps run
 * as replays of one captured graph (keyed by the attention split count) with
 * no host round trip between them.  out[i] receives the token step i chose. */
int q8_decoder_generate(q8_decoder *dec, int steps, uint32_t *out);

/* The logits of the last forward or step (n_vocab f32, waits). */
int q8_decoder_logits(q8_decoder *dec, float *host, size_t len);
/* Weights for the CPU checks: layer < 0 is the token embedding, or with
 * which = Q8_DEC_OUTPUT the output head (the embedding when tied); `which`
 * is Q8_DEC_*.  Norms: which 0 attention, 1 feed-forward;
 * layer < 0 the output norm (host pointer of n_embd floats). */
int q8_decoder_weight(const q8_decoder *dec, int layer, int which, const q8_weight **weight);
int q8_decoder_norm(const q8_decoder *dec, int layer, int which, const float **weight);

/* Graph bookkeeping of a decoder: graphs held now, captured and dropped
 * since creation, and passes run eagerly (the first of each shape).  A
 * dropped graph means a workspace moved under it. */
typedef struct {
    int graphs, captured, dropped, eager;
} q8_decoder_stats;
int q8_decoder_graph_stats(const q8_decoder *dec, q8_decoder_stats *stats);

#ifdef __cplusplus
}
#endif

#endif /* Q8DECODER_H */
