// q8_decoder.cpp -- the synthetic decoder of include/q8decoder.h, written
// against the library's own C-ABI the way the reference's Model is written
// against Compute (apps/engine/src/model.rs:652-1235): one pass per forward,
// every projection through the Q8_0 matmul entry points.
//
// A pass (Model::body, model.rs:755-826) per layer:
//   attention: norm (f32 rows for one token, straight to prepared Q8_0 for a
//              prompt), q/k/v as one grouped matmul, rope + f16 KV append,
//              attention, output projection with the residual in its epilogue;
//   feed-forward: norm, gate/up (one fused GEMV + SiLU for one token; for a
//              prompt one GEMM whose epilogue quantizes silu(gate)*up for the
//              down projection), down projection with the residual;
// then the output norm of the last row, the lm_head GEMV (the tied embedding)
// and the greedy argmax, written to the token slot the next step embeds.
//
// Graphs: a pass of shape (n, attention splits) runs eagerly the first time
// and is captured into a graph the next time; replays read the position from
// device memory.  Creation plans every workspace a pass uses, so passes
// allocate nothing; a captured graph is still dropped if the context's
// workspaces move (another caller of the context grew one), since its
// pointers would be stale.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <utility>
#include <vector>

#include "../../include/q8decoder.h"
#include "q8_internal.h"
#include "q8_layout.h"

namespace {

using q8i::set_error;

#define DEC_TRY(call)                 \
    do {                              \
        int rc_ = (call);             \
        if (rc_ != Q8_OK) return rc_; \
    } while (0)

unsigned long long mix(unsigned long long z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// Norm weights near one: 1 + 0.05 * (u - 0.5), u uniform from the seed.
std::vector<float> norm_weights(unsigned long long seed, int n) {
    std::vector<float> w(n);
    for (int i = 0; i < n; i++) {
        const double u = (double)(mix(seed + (unsigned long long)i) >> 11) * (1.0 / 9007199254740992.0);
        w[i] = (float)(1.0 + 0.05 * (u - 0.5));
    }
    return w;
}

struct Layer {
    const q8_weight *w[7] = {};
    std::vector<float> attn_norm, ffn_norm;
    q8_dptr kcache = 0, vcache = 0;
};

}  // namespace

struct q8_decoder {
    q8_ctx *c = nullptr;
    q8_decoder_config cfg{};
    std::vector<Layer> layers;
    const q8_weight *embd = nullptr;
    const q8_weight *output = nullptr;  // the output head: embd when tied
    std::vector<float> output_norm;
    q8_dptr x = 0, q = 0, act = 0, logits = 0;
    q8_dptr pos = 0, tokens = 0;
    int position = 0;  // host mirror of *pos
    std::map<std::pair<int, int>, void *> graphs;
    std::map<std::pair<int, int>, int> runs;  // eager runs per shape
    unsigned long long generation = 0;
    uint32_t *pinned = nullptr;  // generate(): tokens read back without a wait per step
    int pinned_len = 0;
    std::vector<q8_dptr> buffers;
    int captured = 0, dropped = 0, eager = 0;

    int alloc(size_t bytes, q8_dptr *p) {
        DEC_TRY(q8_alloc(c, bytes, p));
        buffers.push_back(*p);
        return Q8_OK;
    }
    void drop_graphs() {
        for (auto &g : graphs) q8_graph_destroy(g.second);
        dropped += (int)graphs.size();
        graphs.clear();
    }
    int plan();
    int splits_for(int visible) const {
        // Always the split kernel with its combine folded into the output
        // projection (two splits at least): one 16-wave workgroup per head
        // leaves most CUs idle (configs[4] geometry, whole decode step, 16 to
        // 256 positions: 1.38-1.42 ms with one split, 1.30-1.33 with two).
        // Each split walks its chunks in turn and every split adds to the
        // combine (at most eight), so: the fewest chunks per split that eight
        // splits allow, then the fewest splits at that many chunks (2400
        // positions: 5 splits 1.550 ms vs 8 splits 1.618; 3000: 6 splits
        // 1.593 vs 1.658; up to 2048 positions a split per chunk, measured
        // best or within 0.3%).
        const int rows = q8i::attention_split_rows();
        if (visible <= 1) return 1;
        if (visible <= 2 * rows) return 2;
        const int chunks = (visible + Q8_ATTN_COMBINE_MAX * rows - 1) / (Q8_ATTN_COMBINE_MAX * rows);
        return std::min(Q8_ATTN_COMBINE_MAX, (visible + chunks * rows - 1) / (chunks * rows));
    }
    int max_splits(int capacity) const {
        // the most splits any visible count up to `capacity` takes (counts
        // past eight chunks fall back to fewer splits)
        return splits_for(std::min(capacity, Q8_ATTN_COMBINE_MAX * q8i::attention_split_rows()));
    }
    int body(int n, int splits);
    int run(int n, int splits);
    void sync_generation() {
        const unsigned long long now = q8i::workspace_generation(c);
        if (now != generation) {
            drop_graphs();
            generation = now;
        }
    }
};

namespace {

int check_config(const q8_decoder_config &g) {
    if (g.n_layer < 1 || g.n_embd < 32 || g.n_embd % 32 || g.n_ff < 32 || g.n_ff % 32 || g.n_head < 1 ||
        g.n_head_kv < 1 || g.n_head % g.n_head_kv || g.head_dim != Q8_ATTN_HEAD_DIM ||
        g.n_head * g.head_dim != g.n_embd || g.n_rot < 0 || g.n_rot > g.head_dim || g.n_rot % 2 || g.n_vocab < 1 ||
        g.capacity < 1 || g.max_batch < 1 || g.max_batch > Q8_MAX_TOKENS || !(g.eps > 0.0f) ||
        (g.untied_output != 0 && g.untied_output != 1) || !(g.embd_std >= 0.0f) || g.embd_std > 1e3f)
        return set_error(Q8_ERR_INVALID,
                         "decoder config: layers %d, embd %d, ff %d, heads %d/%d x %d, rot %d, vocab %d, capacity %d, "
                         "batch %d, untied %d, embd_std %g (head_dim must be 64, heads x head_dim = embd, dims "
                         "multiples of 32, untied 0 or 1, 0 <= embd_std <= 1000)",
                         g.n_layer, g.n_embd, g.n_ff, g.n_head, g.n_head_kv, g.head_dim, g.n_rot, g.n_vocab, g.capacity,
                         g.max_batch, g.untied_output, (double)g.embd_std);
    return Q8_OK;
}

}  // namespace

// One pass of n tokens at the device position (Model::body, model.rs:755-826).
int q8_decoder::body(int n, int splits) {
    const q8_decoder_config &g = cfg;
    const int E = g.n_embd;
    const float scale = 1.0f / std::sqrt((float)g.head_dim);
    DEC_TRY(q8_embeddings_device(c, embd, tokens, (size_t)n, x, 0));
    // A prompt's GEMMs are compute-bound and leave HBM mostly idle, so each
    // announces the weights of the GEMM after it (q8_gemm_prefetch), whose
    // launch then finds them in the Infinity Cache instead of HBM.
    auto announce = [&](const q8_weight *a, const q8_weight *b = nullptr, const q8_weight *d = nullptr) {
        const q8_weight *w[3] = {a, b, d};
        return q8_gemm_prefetch(c, w, d ? 3 : b ? 2 : 1);
    };
    for (size_t li = 0; li < layers.size(); li++) {
        Layer &L = layers[li];
        // attention block (dense_attention, model.rs:869-1043)
        if (n == 1) {  // norm, q/k/v and rope + KV append in one launch
            DEC_TRY(q8_norm_qkv_rope(c, L.attn_norm.data(), g.eps, L.w[Q8_DEC_Q], L.w[Q8_DEC_K], L.w[Q8_DEC_V], x, 0,
                                     q, 0, L.kcache, L.vcache, g.n_head, g.n_head_kv, g.head_dim, g.n_rot,
                                     g.rope_base, g.capacity, pos));
        } else {
            q8_prepared p{};
            DEC_TRY(q8_norm_prepare(c, x, 0, L.attn_norm.data(), E, g.eps, n, &p));
            DEC_TRY(announce(L.w[Q8_DEC_O]));
            DEC_TRY(q8_prompt_qkv_rope(c, L.w[Q8_DEC_Q], L.w[Q8_DEC_K], L.w[Q8_DEC_V], &p, n, q, 0, L.kcache,
                                       L.vcache, g.n_head, g.n_head_kv, g.head_dim, g.n_rot, g.rope_base,
                                       g.capacity, pos));
        }
        if (n == 1) {  // attention, its split combine folded into the output projection
            DEC_TRY(q8_attention_matmul_add(c, q, 0, L.kcache, L.vcache, g.n_head, g.n_head_kv, g.head_dim,
                                            g.capacity, scale, pos, splits, L.w[Q8_DEC_O], x, 0));
        } else {  // attention written as the output projection's prepared activations
            q8_prepared pa{};
            DEC_TRY(q8_attention_prepare(c, q, 0, L.kcache, L.vcache, n, g.n_head, g.n_head_kv, g.head_dim,
                                         g.capacity, scale, pos, &pa));
            DEC_TRY(announce(L.w[Q8_DEC_GATE], L.w[Q8_DEC_UP]));
            DEC_TRY(q8_matmul(c, L.w[Q8_DEC_O], 0, 0, n, x, 0, &pa, x, 0));
        }
        // feed-forward block (feed_forward, model.rs:1162-1235)
        if (n == 1) {
            DEC_TRY(q8_norm_gate_up_silu(c, L.ffn_norm.data(), g.eps, L.w[Q8_DEC_GATE], L.w[Q8_DEC_UP], x, 0, act, 0));
            DEC_TRY(q8_matmul(c, L.w[Q8_DEC_DOWN], act, 0, 1, x, 0, nullptr, x, 0));
        } else {
            q8_prepared p{};
            DEC_TRY(q8_norm_prepare(c, x, 0, L.ffn_norm.data(), E, g.eps, n, &p));
            q8_prepared pd{};
            DEC_TRY(announce(L.w[Q8_DEC_DOWN]));
            DEC_TRY(q8_gate_up_silu_prepared(c, L.w[Q8_DEC_GATE], L.w[Q8_DEC_UP], &p, &pd));
            if (li + 1 < layers.size()) {
                const Layer &N = layers[li + 1];
                DEC_TRY(announce(N.w[Q8_DEC_Q], N.w[Q8_DEC_K], N.w[Q8_DEC_V]));
            }
            DEC_TRY(q8_matmul(c, L.w[Q8_DEC_DOWN], act, 0, n, x, 0, &pd, x, 0));
        }
    }
    // output norm of the last row, lm_head, greedy choice into the token slot
    DEC_TRY(q8_norm_lm_head_argmax(c, output_norm.data(), g.eps, output, x, (size_t)(n - 1) * E, logits, 0, tokens));
    return q8_advance_position(c, pos, n);
}

// A pass, through its graph once the shape has run eagerly.
int q8_decoder::run(int n, int splits) {
    const auto key = std::make_pair(n, splits);
    sync_generation();
    auto it = graphs.find(key);
    if (it != graphs.end()) return q8_graph_launch(c, it->second);
    if (runs[key]++ == 0) {
        eager++;
        const int rc = body(n, splits);
        sync_generation();  // the eager run may have grown workspaces under older graphs
        return rc;
    }
    DEC_TRY(q8_graph_begin(c));
    const int rc = body(n, splits);
    void *graph = nullptr;
    const int rc_end = q8_graph_end(c, &graph);
    if (rc != Q8_OK) {
        q8_graph_destroy(graph);
        return rc;
    }
    DEC_TRY(rc_end);
    if (q8i::workspace_generation(c) != generation) {  // cannot happen after an eager run; never replay stale
        q8_graph_destroy(graph);
        return set_error(Q8_ERR_HIP, "decoder: a workspace grew during capture");
    }
    graphs[key] = graph;
    captured++;
    return q8_graph_launch(c, graph);
}

// Everything a pass may allocate, allocated now (Workspace sizing per
// context, workspace.rs:171-342): the workspaces for max_batch tokens and
// the widest row, the attention partials for the most splits any position
// up to `capacity` uses, the rotation table, the resident norm weights, and
// the pinned buffer generate() reads tokens into.
int q8_decoder::plan() {
    const q8_decoder_config &g = cfg;
    q8_workspace_shape s{};
    s.max_tokens = g.max_batch;
    s.max_k = std::max(std::max(g.n_embd, g.n_ff), g.n_head * g.head_dim);
    s.max_ff = g.n_ff;
    s.attn_heads = g.n_head;
    s.attn_splits = max_splits(g.capacity);
    s.rope_n_rot = g.n_rot;
    s.rope_base = g.rope_base;
    DEC_TRY(q8_workspace_plan(c, &s));
    for (Layer &L : layers) {
        DEC_TRY(q8_vector_resident(c, L.attn_norm.data(), L.attn_norm.size()));
        DEC_TRY(q8_vector_resident(c, L.ffn_norm.data(), L.ffn_norm.size()));
    }
    DEC_TRY(q8_vector_resident(c, output_norm.data(), output_norm.size()));
    if (hipHostMalloc((void **)&pinned, (size_t)g.capacity * 4, 0) != hipSuccess) {
        pinned = nullptr;
        return set_error(Q8_ERR_OUT_OF_MEMORY, "hipHostMalloc(%d tokens)", g.capacity);
    }
    pinned_len = g.capacity;
    generation = q8i::workspace_generation(c);
    return Q8_OK;
}

extern "C" {

int q8_decoder_create_synthetic(q8_ctx *c, const q8_decoder_config *config, uint64_t seed, q8_decoder **out) {
    if (!c || !config || !out) return set_error(Q8_ERR_INVALID, "q8_decoder_create_synthetic: bad arguments");
    *out = nullptr;
    DEC_TRY(check_config(*config));
    q8_decoder *d = new q8_decoder;
    d->c = c;
    d->cfg = *config;
    const q8_decoder_config &g = d->cfg;
    const int E = g.n_embd, kv_dim = g.n_head_kv * g.head_dim, B = g.max_batch;
    const float std_w = 0.02f;
    auto fail = [&](int rc) {
        q8_decoder_destroy(d);
        return rc;
    };
    int rc = q8_weight_synthetic(c, E, g.n_vocab, mix(seed), g.embd_std > 0.0f ? g.embd_std : std_w, &d->embd);
    if (rc) return fail(rc);
    d->output = d->embd;
    if (g.untied_output) {
        rc = q8_weight_synthetic(c, E, g.n_vocab, mix(seed ^ 0x6f75747075742e77ull), std_w, &d->output);
        if (rc) return fail(rc);
    }
    d->output_norm = norm_weights(mix(seed ^ 0x6f75747075746e6full), E);
    d->layers.resize(g.n_layer);
    for (int l = 0; l < g.n_layer; l++) {
        Layer &L = d->layers[l];
        const int dims[7][2] = {{E, g.n_head * g.head_dim}, {E, kv_dim},  {E, kv_dim}, {g.n_head * g.head_dim, E},
                                {E, g.n_ff},                {E, g.n_ff}, {g.n_ff, E}};
        auto wseed = [&](int i) { return mix(seed + 1000003ull * (l + 1) + i); };
        // q/k/v and gate/up run as groups (one launch over several matrices):
        // each is made a contiguous group, whose launches read one run of
        // tiles from preloaded bases; O and down run alone, each with its
        // slice-major copy
        for (int i : {Q8_DEC_O, Q8_DEC_DOWN}) {
            rc = q8i::weight_synthetic(c, dims[i][0], dims[i][1], wseed(i), std_w, true, &L.w[i]);
            if (rc) return fail(rc);
        }
        const int qkv_rows[3] = {dims[Q8_DEC_Q][1], dims[Q8_DEC_K][1], dims[Q8_DEC_V][1]};
        const uint64_t qkv_seeds[3] = {wseed(Q8_DEC_Q), wseed(Q8_DEC_K), wseed(Q8_DEC_V)};
        const q8_weight *qkv[3] = {};
        rc = q8i::weight_synthetic_group(c, E, 3, qkv_rows, qkv_seeds, std_w, q8i::group_slice_rows(c, E, 0), qkv);
        if (rc) return fail(rc);
        L.w[Q8_DEC_Q] = qkv[0];
        L.w[Q8_DEC_K] = qkv[1];
        L.w[Q8_DEC_V] = qkv[2];
        const int ffn_rows[2] = {g.n_ff, g.n_ff};
        const uint64_t ffn_seeds[2] = {wseed(Q8_DEC_GATE), wseed(Q8_DEC_UP)};
        const q8_weight *ffn[2] = {};
        rc = q8i::weight_synthetic_group(c, E, 2, ffn_rows, ffn_seeds, std_w, q8i::group_pair_slices(c, E), ffn);
        if (rc) return fail(rc);
        L.w[Q8_DEC_GATE] = ffn[0];
        L.w[Q8_DEC_UP] = ffn[1];
        L.attn_norm = norm_weights(mix(seed + 7919ull * (l + 1)), E);
        L.ffn_norm = norm_weights(mix(seed + 104729ull * (l + 1)), E);
        const size_t cache = (size_t)g.capacity * kv_dim * 2;
        if ((rc = d->alloc(cache, &L.kcache)) || (rc = d->alloc(cache, &L.vcache))) return fail(rc);
    }
    const size_t f = sizeof(float);
    if ((rc = d->alloc((size_t)B * E * f, &d->x)) ||
        (rc = d->alloc((size_t)B * g.n_head * g.head_dim * f, &d->q)) ||
        (rc = d->alloc((size_t)B * g.n_ff * f, &d->act)) || (rc = d->alloc((size_t)g.n_vocab * f, &d->logits)) ||
        (rc = d->alloc(256, &d->pos)) || (rc = d->alloc((size_t)B * 4, &d->tokens)))
        return fail(rc);
    if ((rc = d->plan()) || (rc = q8_decoder_reset(d))) return fail(rc);
    *out = d;
    return Q8_OK;
}

void q8_decoder_destroy(q8_decoder *d) {
    if (!d) return;
    q8_sync(d->c);
    d->drop_graphs();
    for (Layer &L : d->layers)
        for (const q8_weight *w : L.w)
            if (w) q8_weight_release(d->c, w);
    if (d->output && d->output != d->embd) q8_weight_release(d->c, d->output);
    if (d->embd) q8_weight_release(d->c, d->embd);
    // the norm vectors' device copies are cached by host address: drop them
    // before the host vectors are freed and their addresses reused
    for (Layer &L : d->layers) {
        q8_vector_release(d->c, L.attn_norm.data(), L.attn_norm.size());
        q8_vector_release(d->c, L.ffn_norm.data(), L.ffn_norm.size());
    }
    q8_vector_release(d->c, d->output_norm.data(), d->output_norm.size());
    for (q8_dptr p : d->buffers) q8_free(d->c, p);
    if (d->pinned) (void)hipHostFree(d->pinned);
    delete d;
}

int q8_decoder_reset(q8_decoder *d) {
    if (!d) return set_error(Q8_ERR_INVALID, "q8_decoder_reset: null decoder");
    const int zero[2] = {0, 0};
    DEC_TRY(q8_upload(d->c, d->pos, zero, sizeof zero));
    d->position = 0;
    return Q8_OK;
}

int q8_decoder_position(const q8_decoder *d, int *position) {
    if (!d || !position) return set_error(Q8_ERR_INVALID, "q8_decoder_position: bad arguments");
    *position = d->position;
    return Q8_OK;
}

int q8_decoder_forward(q8_decoder *d, const uint32_t *tokens, int n, uint32_t *next) {
    if (!d || !tokens || !next) return set_error(Q8_ERR_INVALID, "q8_decoder_forward: bad arguments");
    if (n < 1) return set_error(Q8_ERR_INVALID, "empty prompt");
    if (n > d->cfg.max_batch)
        return set_error(Q8_ERR_UNSUPPORTED, "forward of %d tokens exceeds the decoder's batch of %d", n,
                         d->cfg.max_batch);
    if (d->position + n > d->cfg.capacity)
        return set_error(Q8_ERR_UNSUPPORTED, "context full: %d of %d tokens used", d->position + n, d->cfg.capacity);
    for (int i = 0; i < n; i++)
        if (tokens[i] >= (uint32_t)d->cfg.n_vocab) return set_error(Q8_ERR_INVALID, "token %u outside vocabulary", tokens[i]);
    DEC_TRY(q8_upload(d->c, d->tokens, tokens, (size_t)n * 4));
    DEC_TRY(d->run(n, d->splits_for(d->position + n)));
    DEC_TRY(q8_download(d->c, next, d->tokens, 4));
    d->position += n;
    return Q8_OK;
}

int q8_decoder_generate(q8_decoder *d, int steps, uint32_t *out) {
    if (!d || (!out && steps > 0)) return set_error(Q8_ERR_INVALID, "q8_decoder_generate: bad arguments");
    if (steps <= 0) return Q8_OK;
    if (d->position < 1) return set_error(Q8_ERR_INVALID, "generate needs a forward first (no token to feed)");
    if (d->position + steps > d->cfg.capacity)
        return set_error(Q8_ERR_UNSUPPORTED, "context full: %d of %d tokens used", d->position + steps,
                         d->cfg.capacity);
    if (d->pinned_len < steps)  // reserved for the whole context at creation
        return set_error(Q8_ERR_INVALID, "generate: %d steps exceed the %d-token pinned buffer", steps,
                         d->pinned_len);
    // one split count for the whole run, sized for its last step
    const int splits = d->splits_for(d->position + steps);
    hipStream_t stream = (hipStream_t)q8_stream(d->c);
    for (int i = 0; i < steps; i++) {
        DEC_TRY(d->run(1, splits));
        if (hipMemcpyAsync(d->pinned + i, (const void *)(uintptr_t)d->tokens, 4, hipMemcpyDeviceToHost, stream) !=
            hipSuccess)
            return set_error(Q8_ERR_HIP, "hip: hipMemcpyAsync(token) failed");
    }
    DEC_TRY(q8_sync(d->c));
    std::memcpy(out, d->pinned, (size_t)steps * 4);
    d->position += steps;
    return Q8_OK;
}

int q8_decoder_logits(q8_decoder *d, float *host, size_t len) {
    if (!d || !host) return set_error(Q8_ERR_INVALID, "q8_decoder_logits: bad arguments");
    if (len != (size_t)d->cfg.n_vocab)
        return set_error(Q8_ERR_INVALID, "logits hold %d values, %zu asked", d->cfg.n_vocab, len);
    return q8_download(d->c, host, d->logits, len * 4);
}

int q8_decoder_weight(const q8_decoder *d, int layer, int which, const q8_weight **weight) {
    if (!d || !weight) return set_error(Q8_ERR_INVALID, "q8_decoder_weight: bad arguments");
    if (layer < 0) {
        *weight = which == Q8_DEC_OUTPUT ? d->output : d->embd;
        return Q8_OK;
    }
    if (layer >= (int)d->layers.size() || which < 0 || which > Q8_DEC_DOWN)
        return set_error(Q8_ERR_INVALID, "decoder weight (%d, %d) out of range", layer, which);
    *weight = d->layers[layer].w[which];
    return Q8_OK;
}

int q8_decoder_graph_stats(const q8_decoder *d, q8_decoder_stats *stats) {
    if (!d || !stats) return set_error(Q8_ERR_INVALID, "q8_decoder_graph_stats: bad arguments");
    stats->graphs = (int)d->graphs.size();
    stats->captured = d->captured;
    stats->dropped = d->dropped;
    stats->eager = d->eager;
    return Q8_OK;
}

int q8_decoder_norm(const q8_decoder *d, int layer, int which, const float **weight) {
    if (!d || !weight) return set_error(Q8_ERR_INVALID, "q8_decoder_norm: bad arguments");
    if (layer < 0) {
        *weight = d->output_norm.data();
        return Q8_OK;
    }
    if (layer >= (int)d->layers.size() || which < 0 || which > 1)
        return set_error(Q8_ERR_INVALID, "decoder norm (%d, %d) out of range", layer, which);
    *weight = which == 0 ? d->layers[layer].attn_norm.data() : d->layers[layer].ffn_norm.data();
    return Q8_OK;
}

}  // extern "C"
