// Device-resident BitNet b1.58 model, KV cache and decode step.
//
// Reference: ModelGraph::from_gguf (src/model/graph.rs:79-237), KVCache
// (src/model/kv_cache.rs:49-259), forward_with_cache_into
// (src/model/cached_forward.rs:164-521), greedy_generate_with_cache
// (src/model/generate.rs:111-189).
//
// One decode step is a fixed sequence of kernels on the context's stream:
//   embed (Q6_K row) ->
//   per layer: [residual +] attn_norm+quant -> Q, K, V with RoPE and the K/V
//              absmax -> scores (new K row appended) -> softmax+V (new V row
//              appended) -> attn_sub_norm+quant -> O -> residual +
//              ffn_norm+quant -> gate/up with relu^2*up -> ffn_sub_norm+quant
//              -> down
//   -> residual + output_norm -> lm-head argmax (or logits).
// Every matvec keeps whole rows in one workgroup (its waves split K), so its
// f32 output is final; the residual add is folded into the next norm kernel.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <vector>

#include "wm_internal.h"

// launchers from k_layer.hip
bool wm_launch_rmsnorm_quant(float *x, const float *res_y, const float *w, uint32_t n, float eps,
                             uint8_t *act, wm_act_meta *meta_out, float *y_out,
                             uint32_t *err_flag, uint32_t layer_tag, void *q6k_prep,
                             uint32_t *clear2, hipStream_t s);
// decode attention's tag in the step's error flag (above any layer tag)
constexpr uint32_t kAttnWaitFlag = 0x80000000u;
bool wm_launch_attention(const float *q, const int8_t *k_cache, const float *k_scales,
                         const int8_t *v_cache, const float *v_scales, float *scores,
                         uint32_t score_stride, float *out, uint32_t n_heads, uint32_t n_kv_heads,
                         uint32_t head_dim, uint32_t n_past, float scale, const float *k_new,
                         const float *v_new, const uint32_t *kv_absmax, uint32_t kv_absmax_n,
                         uint32_t kv_absmax_stride, uint32_t tag, uint32_t *err_flag,
                         uint32_t err_tag, bool no_wait, hipStream_t s, const uint32_t *pos_dev = nullptr,
                         uint32_t n_max = 0);
bool wm_launch_attention_position_zero(const float *q, const float *k_new, const float *v_new,
                                       float *out, uint32_t n_heads, uint32_t n_kv_heads,
                                       uint32_t head_dim, float scale, hipStream_t s);
void wm_launch_kv_append(const float *k, const float *v, uint32_t kv_dim, uint32_t n_layers,
                         uint32_t pos0, uint32_t n_pos, uint32_t max_seq, int8_t *k_cache,
                         float *k_scales, int8_t *v_cache, float *v_scales, hipStream_t s);
void wm_launch_kv_dequant(const int8_t *k_cache, const float *k_scales, const int8_t *v_cache,
                          const float *v_scales, uint32_t n_pos, uint32_t kv_dim, float *k_out,
                          float *v_out, hipStream_t s);

namespace {

struct dev_lin {
    uint8_t *w = nullptr;  // library I2_S layout (owned copy)
    uint32_t n_groups = 0;
    float scale = 1.0f;
};

struct dev_layer {
    dev_lin q, k, v, o, gate, up, down;
    float *attn_norm = nullptr, *attn_sub_norm = nullptr, *ffn_norm = nullptr,
          *ffn_sub_norm = nullptr;
    bool set = false;
};

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

struct wm_model {
    wm_ctx *ctx = nullptr;
    int device = 0;
    wm_model_config cfg{};
    uint32_t kv_dim = 0;
    std::vector<dev_layer> layers;
    // tied embedding / lm-head (library Q6_K layout) and output norm
    uint8_t *embd = nullptr;
    uint32_t embd_blocks = 0, embd_rowgroups = 0;
    float *output_norm = nullptr;
    float *rope_cos = nullptr, *rope_sin = nullptr;
    // workspace
    uint8_t *ws = nullptr;
    float *hidden = nullptr, *hidden2 = nullptr;  // the residual stream, in two buffers
    float *q = nullptr, *attn_out = nullptr, *final_hidden = nullptr;
    float *h_ff = nullptr, *h_up = nullptr;  // the FFN's gate and up projections
    float *k_new = nullptr, *v_new = nullptr;  // this token's K (after RoPE) and V
    float *proj_out = nullptr;  // O's, then down's f32 output (the next norm adds it to hidden)
    float *logits = nullptr, *scores = nullptr;
    uint32_t *dscalars = nullptr;  // [0] token, [1] next token, [2] error flag, [3] greedy loop's
                                   // position
    // the tag of the last decode attention launch (k_attn.hip): every launch
    // takes the next one, 1 .. 2^32 - 1
    uint32_t attn_tag = 0;
    // this token's K/V absmax as the QKV launch leaves them (wm_fused_absmax):
    // kv_absmax_stride slots each, kv_absmax_n of them written by every launch
    uint32_t *kv_absmax = nullptr;
    uint32_t kv_absmax_stride = 0, kv_absmax_n = 0;
    void *lm_work = nullptr;
    // ragged-batch workspace, grown on demand to b_cap tokens
    uint8_t *bws = nullptr;
    uint32_t b_cap = 0;
    float *b_hidden = nullptr, *b_yqkv = nullptr, *b_q = nullptr, *b_attn = nullptr,
          *b_yo = nullptr, *b_ygu = nullptr, *b_ydown = nullptr, *b_final = nullptr;
    uint8_t *b_act = nullptr;
    wm_act_meta *b_meta = nullptr;
    wm_batch_tok *b_tok = nullptr;
    uint32_t *b_ids = nullptr, *b_next = nullptr;
    void *b_lmw = nullptr;  // the multi-vector lm-head's work area
    float *b_scores = nullptr;  // attention scores [t][head][context], grown on demand
    size_t b_scores_bytes = 0;
    // greedy decode's read-back ring: per step in flight, the next id and the
    // error flag (pinned host memory) and the event after that step's copy
    uint32_t *ring = nullptr, *ring_dev = nullptr;
    hipEvent_t ring_ev[16] = {};
};

struct wm_kv_cache {
    wm_model *m = nullptr;
    int device = 0;
    uint32_t max_seq = 0, pos = 0;
    int8_t *k = nullptr, *v = nullptr;   // [layer][max_seq][kv_dim]
    float *ks = nullptr, *vs = nullptr;  // [layer][max_seq]
};

namespace {

wm_status copy_lin(wm_model *m, const wm_tensor *t, uint64_t in_dim, uint64_t out_dim, dev_lin *out,
                   const char *name) {
    wm_ctx *ctx = m->ctx;
    if (!t) return wm_set_error(ctx, WM_E_ARG, "%s: missing tensor", name);
    if (t->type != WM_TYPE_I2S)
        return wm_set_error(ctx, WM_E_UNSUPPORTED_TYPE, "%s: tensor type %d is not I2_S", name, t->type);
    if (t->in_dim != in_dim || t->out_dim != out_dim)
        return wm_set_error(ctx, WM_E_SHAPE, "%s: shape [%llu, %llu] != [%llu, %llu]", name,
                            (unsigned long long)t->in_dim, (unsigned long long)t->out_dim,
                            (unsigned long long)in_dim, (unsigned long long)out_dim);
    if (out->w) WM_HIP(ctx, hipFree(out->w));
    out->w = nullptr;
    WM_HIP(ctx, hipMalloc(&out->w, t->bytes));
    WM_HIP(ctx, hipMemcpyAsync(out->w, t->d, t->bytes, hipMemcpyDeviceToDevice, ctx->stream));
    out->n_groups = t->n_groups;
    out->scale = t->scale;
    return WM_OK;
}

wm_status copy_norm(wm_model *m, const float *src, uint32_t n, float **dst, const char *name) {
    wm_ctx *ctx = m->ctx;
    if (!src) return wm_set_error(ctx, WM_E_ARG, "%s: missing norm weights", name);
    if (!*dst) WM_HIP(ctx, hipMalloc((void **)dst, (size_t)n * 4));
    WM_HIP(ctx, hipMemcpyAsync(*dst, src, (size_t)n * 4, hipMemcpyHostToDevice, ctx->stream));
    return WM_OK;
}

void free_lin(dev_lin &l) {
    if (l.w) hipFree(l.w);
    l.w = nullptr;
}

bool model_ready(const wm_model *m) {
    if (!m->embd || !m->output_norm) return false;
    for (auto &l : m->layers)
        if (!l.set) return false;
    return true;
}

// The kernels of one layer, in order (wm_debug_rerun_role's role numbers).
enum layer_role { ROLE_QKV = 0, ROLE_SCORES_SOFTMAX_V, ROLE_O, ROLE_GATE_UP, ROLE_DOWN, ROLE_ALL };

// Enqueue layer l at `pos`, the residual stream in H[cur] on entry (cur is
// updated as the layer's two residual adds move it).  With only < ROLE_ALL
// just that role's launches are enqueued (the buffers stay as they are).
// Returns false when a launcher had no kernel for the model's shape.
// The position of a step: a value, or (pos_dev) a device word read by the
// kernels, whose attention launches are then sized for n_max positions.
struct step_pos {
    uint32_t pos;
    const uint32_t *dev;
    uint32_t n_max;
};

// The tag for the next decode attention launch on m's scores buffer: the
// launches are counted, skipping 0 (the tag of the zeroed buffer).
uint32_t next_attn_tag(wm_model *m) {
    m->attn_tag = m->attn_tag == 0xFFFFFFFFu ? 1u : m->attn_tag + 1u;
    return m->attn_tag;
}

bool enqueue_layer(wm_model *m, wm_kv_cache *kv, uint32_t l, step_pos sp, float *const H[2],
                   int &cur, float *layer_trace_dev, int only = ROLE_ALL) {
    const uint32_t pos = sp.pos;
    const wm_model_config &c = m->cfg;
    hipStream_t s = m->ctx->stream;
    const uint32_t E = c.n_embd, KV = m->kv_dim;
    const uint32_t n_chunks_e = E / I2S_CHUNK_COLS, n_chunks_f = c.n_ff / I2S_CHUNK_COLS;
    const float scale = 1.0f / sqrtf((float)c.head_dim);  // primitives.rs:354
    // absmax of this token's K and V: slots written by the QKV launch, whose
    // maximum attention takes
    const wm_fused_absmax kv_absmax{m->kv_absmax, m->kv_absmax_stride, &m->kv_absmax_n};
    const auto want = [&](int r) { return only == ROLE_ALL || only == r; };
    const dev_layer &L = m->layers[l];
    // attn_norm, on hidden + the previous layer's ffn_down, then Q, K, V
    // (whole heads, or a head's rows split over a few workgroups; NEOX RoPE
    // on Q and K at `pos`)
    wm_fused_norm an{};
    an.debug = m->ctx->fused_debug;
    an.x = H[cur];
    an.w = L.attn_norm;
    an.eps = c.rms_eps;
    if (l > 0) {
        an.y = m->proj_out;
        an.x_out = H[cur ^ 1];
        an.err_flag = m->dscalars + 2;
        an.layer_tag = l;
        cur ^= 1;
    }
    wm_i2s_desc qkv[3] = {{L.q.w, L.q.n_groups}, {L.k.w, L.k.n_groups}, {L.v.w, L.v.n_groups}};
    const float qkv_scales[3] = {L.q.scale, L.k.scale, L.v.scale};
    float *qkv_out[3] = {m->q, m->k_new, m->v_new};
    if (want(ROLE_QKV) &&
        !wm_launch_i2s_fused(WM_FUSED_ROPE, qkv, qkv_scales, qkv_out, 3, n_chunks_e, c.head_dim / 64,
                             an, m->rope_cos, m->rope_sin, pos, c.n_rot, 0x3u, &kv_absmax, s, sp.dev))
        return false;
    if (layer_trace_dev && l > 0)
        hipMemcpyAsync(layer_trace_dev + (size_t)(l - 1) * E, H[cur], (size_t)E * 4,
                       hipMemcpyDeviceToDevice, s);
    // attention; this token's K/V row goes into the cache on the way (no
    // cache: the position-zero attention on this token's own K and V)
    if (want(ROLE_SCORES_SOFTMAX_V)) {
        if (!kv) {
            if (!wm_launch_attention_position_zero(m->q, m->k_new, m->v_new, m->attn_out, c.n_heads,
                                                   c.n_kv_heads, c.head_dim, scale, s))
                return false;
        } else {
            const size_t lay = (size_t)l * kv->max_seq;
            if (!wm_launch_attention(m->q, kv->k + lay * KV, kv->ks + lay, kv->v + lay * KV,
                                     kv->vs + lay, m->scores, c.context_length, m->attn_out,
                                     c.n_heads, c.n_kv_heads, c.head_dim, pos + 1, scale, m->k_new,
                                     m->v_new, m->kv_absmax, m->kv_absmax_n, m->kv_absmax_stride,
                                     next_attn_tag(m), m->dscalars + 2, kAttnWaitFlag | (l + 1),
                                     (m->ctx->fused_debug & WM_FUSED_DEBUG_ATTN_NO_WAIT) != 0, s,
                                     sp.dev, sp.n_max))
                return false;
        }
    }
    // attn_sub_norm, then O
    wm_fused_norm sn{};
    sn.debug = m->ctx->fused_debug;
    sn.x = m->attn_out;
    sn.w = L.attn_sub_norm;
    sn.eps = c.rms_eps;
    wm_i2s_desc od = {L.o.w, L.o.n_groups};
    float *o_out[1] = {m->proj_out};
    if (want(ROLE_O) && !wm_launch_i2s_fused(WM_FUSED_PLAIN, &od, &L.o.scale, o_out, 1, n_chunks_e,
                                             1, sn, nullptr, nullptr, 0, 0, 0, nullptr, s))
        return false;
    // ffn_norm on hidden + wo_out, then gate and up (relu^2 * up)
    wm_fused_norm fn{};
    fn.debug = m->ctx->fused_debug;
    fn.x = H[cur];
    fn.y = m->proj_out;
    fn.x_out = H[cur ^ 1];
    fn.w = L.ffn_norm;
    fn.eps = c.rms_eps;
    cur ^= 1;
    wm_i2s_desc gu[2] = {{L.gate.w, L.gate.n_groups}, {L.up.w, L.up.n_groups}};
    const float gu_scales[2] = {L.gate.scale, L.up.scale};
    // gate and up as two plain tensors, one 64-row group per workgroup
    // (twice the workgroups of a gate+up pairing, half the weight bytes
    // in flight per wave); relu(gate)^2 * up is formed where it is read,
    // in the down matvec's norm
    float *gu_out[2] = {m->h_ff, m->h_up};
    if (want(ROLE_GATE_UP) && !wm_launch_i2s_fused(WM_FUSED_PLAIN, gu, gu_scales, gu_out, 2,
                                                   n_chunks_e, 1, fn, nullptr, nullptr, 0, 0, 0,
                                                   nullptr, s))
        return false;
    // ffn_sub_norm of relu(gate)^2 * up, then down
    wm_fused_norm dn{};
    dn.debug = m->ctx->fused_debug;
    dn.x = m->h_ff;
    dn.y = m->h_up;
    dn.relu2_mul = 1;
    dn.w = L.ffn_sub_norm;
    dn.eps = c.rms_eps;
    wm_i2s_desc dd = {L.down.w, L.down.n_groups};
    float *d_out[1] = {m->proj_out};
    if (want(ROLE_DOWN) && !wm_launch_i2s_fused(WM_FUSED_PLAIN, &dd, &L.down.scale, d_out, 1,
                                                n_chunks_f, 1, dn, nullptr, nullptr, 0, 0, 0,
                                                nullptr, s))
        return false;
    return true;
}

// Enqueue the layers + output norm for one token at `pos`; the token id is
// read from m->dscalars[0] on the device.  Returns false when some launcher
// had no kernel for the model's shape (nothing after it was enqueued).
bool enqueue_forward(wm_model *m, wm_kv_cache *kv, step_pos sp, float *layer_trace_dev,
                     const uint32_t *token_dev = nullptr) {
    const wm_model_config &c = m->cfg;
    hipStream_t s = m->ctx->stream;
    const uint32_t E = c.n_embd;
    // The residual stream lives in two buffers: a norm that adds a matvec's
    // output reads one and writes the sum to the other (each workgroup its
    // share, while the launch's other workgroups still read the first).
    float *const H[2] = {m->hidden, m->hidden2};
    int cur = 0;
    wm_launch_q6k_dequant_row_dev(m->embd, m->embd_blocks, token_dev ? token_dev : m->dscalars,
                                  H[0], s);
    for (uint32_t l = 0; l < c.n_layers; l++)
        if (!enqueue_layer(m, kv, l, sp, H, cur, layer_trace_dev)) return false;
    // last residual + output_norm (f32 out, no quantisation)
    if (!wm_launch_rmsnorm_quant(H[cur], m->proj_out, m->output_norm, E, c.rms_eps, nullptr,
                                 nullptr, m->final_hidden, m->dscalars + 2, c.n_layers,
                                 wm_q6k_prep_area(m->lm_work, c.vocab_size, m->embd_blocks),
                                 nullptr, s))
        return false;
    if (layer_trace_dev)
        hipMemcpyAsync(layer_trace_dev + (size_t)(c.n_layers - 1) * E, H[cur], (size_t)E * 4,
                       hipMemcpyDeviceToDevice, s);
    return true;
}

wm_status check_step(wm_model *m, wm_kv_cache *kv, uint32_t token, uint32_t pos) {
    wm_ctx *ctx = m->ctx;
    if (!model_ready(m)) return wm_set_error(ctx, WM_E_STATE, "model: weights not fully set");
    if (kv->m != m) return wm_set_error(ctx, WM_E_ARG, "kv cache belongs to another model");
    if (pos != kv->pos)
        return wm_set_error(ctx, WM_E_STATE,
                            "forward_with_cache: cache.position()=%u != position=%u; tokens must be processed in order",
                            kv->pos, pos);
    if (pos >= kv->max_seq)
        return wm_set_error(ctx, WM_E_SHAPE, "KVCache::append: already at max_seq_len %u", kv->max_seq);
    if (token >= m->cfg.vocab_size)
        return wm_set_error(ctx, WM_E_SHAPE, "forward_with_cache: token_id %u out of vocab range %u",
                            token, m->cfg.vocab_size);
    return WM_OK;
}

// The step's error flag (dscalars[2]): layer + 1 of the first non-finite
// residual stream (the fused matvecs raise it), or kAttnWaitFlag | (layer +
// 1) when decode attention's workgroups gave up waiting for each other (a
// bounded wait that does not end in practice: every workgroup is resident).
wm_status step_flag_error(wm_ctx *ctx, const char *what, uint32_t flag) {
    if (flag & kAttnWaitFlag)
        return wm_set_error(ctx, WM_E_HIP, "%s: attention workgroups stopped waiting at layer %u", what,
                            (flag & ~kAttnWaitFlag) - 1);
    return wm_set_error(ctx, WM_E_NONFINITE, "%s: non-finite hidden after layer %u", what, flag - 1);
}

// After the step: read the error flag; on a non-finite hidden the cache is
// rolled back (cached_forward.rs:256-259) and the flag cleared.
wm_status finish_step(wm_model *m, wm_kv_cache *kv, uint32_t pos, bool *failed) {
    wm_ctx *ctx = m->ctx;
    uint32_t flag = 0;
    WM_HIP(ctx, hipMemcpyAsync(&flag, m->dscalars + 2, 4, hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    *failed = flag != 0;
    if (flag) {
        uint32_t zero = 0;
        WM_HIP(ctx, hipMemcpyAsync(m->dscalars + 2, &zero, 4, hipMemcpyHostToDevice, ctx->stream));
        WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        kv->pos = pos;
        return step_flag_error(ctx, "forward_with_cache", flag);
    }
    kv->pos = pos + 1;
    return WM_OK;
}

constexpr uint32_t kBatchMaxTokens = 16384;

wm_status rows_unsupported(wm_ctx *ctx) {
    return wm_set_error(ctx, WM_E_SHAPE, "batch_forward: no row-norm or GEMM kernel for this model shape");
}

// The ragged-batch kernels cover this model shape (else prompts are
// prefilled token by token).
bool batch_supported(const wm_model *m) {
    const wm_model_config &c = m->cfg;
    return wm_attn_rows_supported(c.head_dim, c.n_heads / c.n_kv_heads) && c.n_embd <= 8192 &&
           c.n_ff <= 8192;
}

constexpr uint32_t kPrefillChunk = 512;  // tokens per batched prefill call

wm_status prefill_tokens(wm_model *m, wm_kv_cache *kv, const uint32_t *tokens, uint32_t n,
                         float *last_hidden);

// Grow the ragged-batch workspace to hold `M` tokens.
wm_status ensure_batch_ws(wm_model *m, uint32_t M) {
    if (M <= m->b_cap) return WM_OK;
    wm_ctx *ctx = m->ctx;
    const uint32_t cap = (M + WM_GEMM_TILE_TOKENS - 1) / WM_GEMM_TILE_TOKENS * WM_GEMM_TILE_TOKENS;
    const size_t E = m->cfg.n_embd, F = m->cfg.n_ff, KV = m->kv_dim;
    const size_t sizes[] = {
        align256(cap * E * 4),             // hidden
        align256(cap * (E + 2 * KV) * 4),  // q|k|v BitLinear outputs
        align256(cap * E * 4),             // q after RoPE
        align256(cap * E * 4),             // attention output
        align256(cap * E * 4),             // wo output
        align256(cap * 2 * F * 4),         // gate|up outputs
        align256(cap * E * 4),             // down output
        align256(cap * E * 4),             // output_norm
        align256(cap * std::max(E, F)),    // int8 activations (GEMM layout)
        align256(cap * sizeof(wm_act_meta)),
        align256(cap * sizeof(wm_batch_tok)),
        align256(cap * 4),                 // token ids
        align256(cap * 4),                 // next tokens
        align256(wm_q6k_multi_work_bytes(m->cfg.vocab_size, m->embd_blocks)),  // lm-head, 4 vectors
    };
    size_t total = 0;
    for (size_t sz : sizes) total += sz;
    WM_HIP(ctx, hipSetDevice(m->device));
    if (m->bws) {
        WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        WM_HIP(ctx, hipFree(m->bws));
        m->bws = nullptr;
        m->b_cap = 0;
    }
    WM_HIP(ctx, hipMalloc((void **)&m->bws, total));
    uint8_t *p = m->bws;
    void **slots[] = {(void **)&m->b_hidden, (void **)&m->b_yqkv, (void **)&m->b_q,
                      (void **)&m->b_attn,   (void **)&m->b_yo,   (void **)&m->b_ygu,
                      (void **)&m->b_ydown,  (void **)&m->b_final, (void **)&m->b_act,
                      (void **)&m->b_meta,   (void **)&m->b_tok,  (void **)&m->b_ids,
                      (void **)&m->b_next,   (void **)&m->b_lmw};
    for (size_t i = 0; i < sizeof(sizes) / sizeof(sizes[0]); i++) {
        *slots[i] = p;
        p += sizes[i];
    }
    m->b_cap = cap;
    return WM_OK;
}

}  // namespace

// The ragged step with its results left on the device: row last_rows[i] of
// m->b_final is sequence i's last token after output_norm and, with
// want_next, m->b_next[i] its id-only argmax.  The caches advance on
// success; on a non-finite hidden none does.
wm_status batch_forward_dev(wm_model *m, wm_kv_cache *const *caches, uint32_t n_seqs,
                            const uint32_t *n_new, const uint32_t *tokens, bool want_next,
                            std::vector<uint32_t> &last_rows) {
    if (!m) return WM_E_ARG;
    wm_ctx *ctx = m->ctx;
    if (!caches || !n_new || !tokens || n_seqs == 0)
        return wm_set_error(ctx, WM_E_ARG, "batch_forward: empty batch");
    if (!model_ready(m)) return wm_set_error(ctx, WM_E_STATE, "model: weights not fully set");
    const wm_model_config &c = m->cfg;
    const uint32_t group = c.n_heads / c.n_kv_heads;
    if (!wm_attn_rows_supported(c.head_dim, group))
        return wm_set_error(ctx, WM_E_SHAPE, "batch_forward: head_dim %u with %u query heads per kv head is not supported",
                            c.head_dim, group);
    if (c.n_embd > 8192 || c.n_ff > 8192)  // one 1024-thread workgroup per row norm, <= 8 values per thread
        return wm_set_error(ctx, WM_E_SHAPE, "batch_forward: n_embd/n_ff above 8192 are not supported");
    uint64_t total = 0;
    for (uint32_t i = 0; i < n_seqs; i++) {
        const wm_kv_cache *kv = caches[i];
        if (!kv || kv->m != m) return wm_set_error(ctx, WM_E_ARG, "batch_forward: cache %u is not a cache of this model", i);
        for (uint32_t j = 0; j < i; j++)
            if (caches[j] == kv) return wm_set_error(ctx, WM_E_ARG, "batch_forward: cache %u appears twice", i);
        if (n_new[i] == 0)
            return wm_set_error(ctx, WM_E_ARG, "multi_token_forward: token_ids must not be empty (sequence %u)", i);
        if ((uint64_t)kv->pos + n_new[i] > kv->max_seq)
            return wm_set_error(ctx, WM_E_SHAPE, "KVCache::append: sequence %u would pass max_seq_len %u", i,
                                kv->max_seq);
        total += n_new[i];
    }
    if (total > kBatchMaxTokens)
        return wm_set_error(ctx, WM_E_SHAPE, "batch_forward: %llu tokens exceed the batch limit %u",
                            (unsigned long long)total, kBatchMaxTokens);
    const uint32_t M = (uint32_t)total;
    for (uint32_t t = 0; t < M; t++)
        if (tokens[t] >= c.vocab_size)
            return wm_set_error(ctx, WM_E_SHAPE, "forward_with_cache: token_id %u out of vocab range %u",
                                tokens[t], c.vocab_size);
    wm_status st = ensure_batch_ws(m, M);
    if (st) return st;
    std::vector<wm_batch_tok> tok(M);
    std::vector<uint32_t> last(n_seqs);
    uint32_t n_max = 1, t = 0;
    for (uint32_t i = 0; i < n_seqs; i++) {
        wm_kv_cache *kv = caches[i];
        for (uint32_t j = 0; j < n_new[i]; j++, t++) {
            tok[t] = wm_batch_tok{kv->k, kv->v, kv->ks, kv->vs, kv->max_seq, kv->pos + j};
            n_max = std::max(n_max, kv->pos + j + 1);
        }
        last[i] = t - 1;
    }
    hipStream_t s = ctx->stream;
    WM_HIP(ctx, hipSetDevice(m->device));
    std::vector<wm_attn_item> sc_items, sv_items;
    wm_attn_rows_plan(tok.data(), M, c.n_kv_heads, c.n_kv_heads * wm_attn_rows_sv_parts(group),
                      sc_items, sv_items);
    const uint32_t n_sc = (uint32_t)sc_items.size(), n_sv = (uint32_t)sv_items.size();
    sc_items.insert(sc_items.end(), sv_items.begin(), sv_items.end());
    const size_t sc_bytes = wm_attn_rows_scores_bytes(M, c.n_heads, n_max, n_sc + n_sv);
    if (sc_bytes > m->b_scores_bytes) {
        WM_HIP(ctx, hipStreamSynchronize(s));
        if (m->b_scores) WM_HIP(ctx, hipFree(m->b_scores));
        m->b_scores = nullptr;
        m->b_scores_bytes = 0;
        WM_HIP(ctx, hipMalloc((void **)&m->b_scores, sc_bytes));
        m->b_scores_bytes = sc_bytes;
    }
    WM_HIP(ctx, hipMemcpyAsync(m->b_tok, tok.data(), M * sizeof(wm_batch_tok), hipMemcpyHostToDevice, s));
    WM_HIP(ctx, hipMemcpyAsync(wm_attn_rows_items(m->b_scores, M, c.n_heads, n_max), sc_items.data(),
                               sc_items.size() * sizeof(wm_attn_item), hipMemcpyHostToDevice, s));
    WM_HIP(ctx, hipMemcpyAsync(m->b_ids, tokens, M * 4, hipMemcpyHostToDevice, s));

    const uint32_t E = c.n_embd, F = c.n_ff, KV = m->kv_dim, QKV = E + 2 * KV;
    const uint32_t m_pad = (M + WM_GEMM_TILE_TOKENS - 1) / WM_GEMM_TILE_TOKENS * WM_GEMM_TILE_TOKENS;
    const uint32_t nce = E / I2S_CHUNK_COLS, ncf = F / I2S_CHUNK_COLS;
    const float scale = 1.0f / sqrtf((float)c.head_dim);  // primitives.rs:354
    uint32_t *err = m->dscalars + 2;
    wm_launch_q6k_dequant_rows_dev(m->embd, m->embd_blocks, m->b_ids, M, m->b_hidden, E, s);
    for (uint32_t l = 0; l < c.n_layers; l++) {
        const dev_layer &L = m->layers[l];
        // [hidden += down of the previous layer], attn_norm, int8
        wm_norm_rows nr{m->b_hidden, E, l ? m->b_ydown : nullptr, E, nullptr, 0, L.attn_norm, E,
                        c.rms_eps, m->b_act, m_pad, m->b_meta, nullptr, 0, l ? err : nullptr, l};
        if (!wm_launch_rmsnorm_rows(nr, M, s)) return rows_unsupported(ctx);
        const wm_gemm_desc qkv[3] = {{L.q.w, L.q.n_groups, E, 0, L.q.scale},
                                     {L.k.w, L.k.n_groups, KV, E, L.k.scale},
                                     {L.v.w, L.v.n_groups, KV, E + KV, L.v.scale}};
        if (!wm_launch_i2s_gemm(qkv, 3, nce, m->b_act, M, m_pad, m->b_meta, m->b_yqkv, QKV, s))
            return rows_unsupported(ctx);
        wm_launch_qkv_rows(m->b_yqkv, QKV, m->rope_cos, m->rope_sin, m->b_tok, M, l, E, KV,
                           c.head_dim, c.n_rot, m->b_q, s);
        wm_launch_attn_rows(m->b_q, m->b_tok, M, n_max, l, c.n_kv_heads, c.head_dim, group, scale,
                            m->b_scores, m->b_attn, n_sc, n_sv, s);
        nr = wm_norm_rows{m->b_attn, E, nullptr, 0, nullptr, 0, L.attn_sub_norm, E, c.rms_eps,
                          m->b_act, m_pad, m->b_meta, nullptr, 0, nullptr, 0};
        if (!wm_launch_rmsnorm_rows(nr, M, s)) return rows_unsupported(ctx);
        const wm_gemm_desc od = {L.o.w, L.o.n_groups, E, 0, L.o.scale};
        if (!wm_launch_i2s_gemm(&od, 1, nce, m->b_act, M, m_pad, m->b_meta, m->b_yo, E, s))
            return rows_unsupported(ctx);
        // hidden += wo, ffn_norm, int8
        nr = wm_norm_rows{m->b_hidden, E, m->b_yo, E, nullptr, 0, L.ffn_norm, E, c.rms_eps,
                          m->b_act, m_pad, m->b_meta, nullptr, 0, nullptr, 0};
        if (!wm_launch_rmsnorm_rows(nr, M, s)) return rows_unsupported(ctx);
        const wm_gemm_desc gu[2] = {{L.gate.w, L.gate.n_groups, F, 0, L.gate.scale},
                                    {L.up.w, L.up.n_groups, F, F, L.up.scale}};
        if (!wm_launch_i2s_gemm(gu, 2, nce, m->b_act, M, m_pad, m->b_meta, m->b_ygu, 2 * F, s))
            return rows_unsupported(ctx);
        // relu^2(gate) * up, ffn_sub_norm, int8
        nr = wm_norm_rows{nullptr, 0, nullptr, 0, m->b_ygu, 2 * F, L.ffn_sub_norm, F, c.rms_eps,
                          m->b_act, m_pad, m->b_meta, nullptr, 0, nullptr, 0};
        if (!wm_launch_rmsnorm_rows(nr, M, s)) return rows_unsupported(ctx);
        const wm_gemm_desc dd = {L.down.w, L.down.n_groups, E, 0, L.down.scale};
        if (!wm_launch_i2s_gemm(&dd, 1, ncf, m->b_act, M, m_pad, m->b_meta, m->b_ydown, E, s))
            return rows_unsupported(ctx);
    }
    // hidden += down of the last layer, output_norm (f32)
    wm_norm_rows fin{m->b_hidden, E, m->b_ydown, E, nullptr, 0, m->output_norm, E, c.rms_eps,
                     nullptr, m_pad, nullptr, m->b_final, E, err, c.n_layers};
    if (!wm_launch_rmsnorm_rows(fin, M, s)) return rows_unsupported(ctx);
    if (want_next)  // every sequence's id-only lm-head, four per pass over the table
        wm_launch_q6k_argmax_multi(m->embd, m->embd_blocks, c.vocab_size, m->embd_rowgroups, m->b_final, E,
                                   last.data(), n_seqs, m->b_next, m->b_lmw, s);
    WM_HIP(ctx, hipGetLastError());
    uint32_t flag = 0;
    WM_HIP(ctx, hipMemcpyAsync(&flag, err, 4, hipMemcpyDeviceToHost, s));
    WM_HIP(ctx, hipStreamSynchronize(s));
    if (flag) {
        uint32_t zero = 0;
        WM_HIP(ctx, hipMemcpyAsync(err, &zero, 4, hipMemcpyHostToDevice, s));
        WM_HIP(ctx, hipStreamSynchronize(s));
        return wm_set_error(ctx, WM_E_NONFINITE,
                            "multi_token_forward: non-finite hidden after layer %u; no cache advanced",
                            flag - 1);
    }
    for (uint32_t i = 0; i < n_seqs; i++) caches[i]->pos += n_new[i];
    last_rows = last;
    return WM_OK;
}

extern "C" {

wm_status wm_batch_forward(wm_model *m, wm_kv_cache *const *caches, uint32_t n_seqs,
                           const uint32_t *n_new, const uint32_t *tokens, float *last_hidden,
                           uint32_t *next_tokens) {
    std::vector<uint32_t> last;
    wm_status st = batch_forward_dev(m, caches, n_seqs, n_new, tokens, next_tokens != nullptr, last);
    if (st) return st;
    wm_ctx *ctx = m->ctx;
    hipStream_t s = ctx->stream;
    const size_t E = m->cfg.n_embd;
    if (last_hidden)
        for (uint32_t i = 0; i < n_seqs; i++)
            WM_HIP(ctx, hipMemcpyAsync(last_hidden + i * E, m->b_final + (size_t)last[i] * E, E * 4,
                                       hipMemcpyDeviceToHost, s));
    if (next_tokens)
        WM_HIP(ctx, hipMemcpyAsync(next_tokens, m->b_next, n_seqs * 4, hipMemcpyDeviceToHost, s));
    WM_HIP(ctx, hipStreamSynchronize(s));
    return WM_OK;
}

wm_status wm_model_create(wm_ctx *ctx, const wm_model_config *cfg, wm_model **out) {
    if (!ctx || !cfg || !out) return WM_E_ARG;
    *out = nullptr;
    const wm_model_config &c = *cfg;
    if (!c.n_layers || !c.n_embd || !c.n_ff || !c.n_heads || !c.n_kv_heads || !c.head_dim ||
        !c.vocab_size || !c.context_length)
        return wm_set_error(ctx, WM_E_SHAPE, "model config: zero dimension");
    if (c.n_heads % c.n_kv_heads)
        return wm_set_error(ctx, WM_E_SHAPE, "gqa_group_size: n_heads (%u) not divisible by n_kv_heads (%u)",
                            c.n_heads, c.n_kv_heads);
    if (c.n_heads * c.head_dim != c.n_embd || (c.head_dim != 64 && c.head_dim != 128))
        return wm_set_error(ctx, WM_E_SHAPE, "model config: head_dim %u unsupported", c.head_dim);
    if (c.n_rot == 0 || c.n_rot % 2 || c.n_rot > c.head_dim)
        return wm_set_error(ctx, WM_E_SHAPE, "apply_rope_f32: n_rot=%u must be even and <= head_dim",
                            c.n_rot);
    if (c.n_embd % QK_I2S || c.n_ff % QK_I2S || c.n_embd % Q6K_VALUES)
        return wm_set_error(ctx, WM_E_SHAPE, "model config: n_embd/n_ff must be multiples of 256/128");
    // attention keeps a context's softmax weights in LDS (16 KB at 4096)
    // (the lm-head stages one hidden vector in LDS: n_embd <= 8192)
    if (c.n_ff > 16384 || c.n_embd > WM_Q6K_LOGITS_MAX_BLOCKS * Q6K_VALUES ||
        c.context_length > 4096 || c.vocab_size > WM_Q6K_LOGITS_MAX_ROWS)
        return wm_set_error(ctx, WM_E_SHAPE, "model config: dimensions beyond the supported range");
    WM_HIP(ctx, hipSetDevice(ctx->device));
    wm_model *m = new wm_model();
    m->ctx = ctx;
    m->device = ctx->device;
    m->cfg = c;
    m->kv_dim = c.n_kv_heads * c.head_dim;
    m->layers.resize(c.n_layers);
    // RoPE angle tables, computed with the host libm exactly as
    // apply_rope_f32 computes them (src/model/primitives.rs:313-318).
    const uint32_t half = c.n_rot / 2;
    std::vector<float> cs((size_t)c.context_length * half), sn(cs.size());
    for (uint32_t p = 0; p < c.context_length; p++) {
        const float pos = (float)p;
        for (uint32_t j = 0; j < half; j++) {
            float exponent = -2.0f * (float)j / (float)c.n_rot;
            float theta = pos * powf(c.rope_freq_base, exponent);
            sn[(size_t)p * half + j] = sinf(theta);
            cs[(size_t)p * half + j] = cosf(theta);
        }
    }
    const uint32_t E = c.n_embd, F = c.n_ff;
    const size_t sizes[] = {
        align256((size_t)E * 4), align256((size_t)E * 4),         // hidden, hidden2
        align256((size_t)E * 4),                                  // q
        align256((size_t)E * 4),                                  // attn_out
        align256((size_t)F * 4), align256((size_t)F * 4),         // h_ff, h_up
        align256((size_t)E * 4),                                  // final_hidden
        align256((size_t)m->kv_dim * 4), align256((size_t)m->kv_dim * 4),  // k_new, v_new
        align256((size_t)E * 4),                                  // proj_out
        align256((size_t)c.vocab_size * 4),                       // logits
        align256((size_t)c.n_heads * c.context_length * 8),       // decode attention's tagged scores
        256,                                                      // device scalars
        align256((size_t)2 * 16 * c.n_kv_heads * 4),              // K/V absmax slots
        align256(wm_q6k_logits_work_bytes(c.vocab_size, c.n_embd / Q6K_VALUES)),  // lm-head work
        align256(cs.size() * 4), align256(cs.size() * 4),         // rope tables
    };
    size_t total = 0;
    for (size_t sz : sizes) total += sz;
    hipError_t e = hipMalloc((void **)&m->ws, total);
    if (e != hipSuccess) {
        delete m;
        return wm_hip_error(ctx, e, "wm_model_create workspace");
    }
    uint8_t *p = m->ws;
    void **slots[] = {(void **)&m->hidden,   (void **)&m->hidden2,  (void **)&m->q,
                      (void **)&m->attn_out, (void **)&m->h_ff,     (void **)&m->h_up,
                      (void **)&m->final_hidden,
                      (void **)&m->k_new,    (void **)&m->v_new,    (void **)&m->proj_out,
                      (void **)&m->logits,   (void **)&m->scores,   (void **)&m->dscalars,
                      (void **)&m->kv_absmax,
                      (void **)&m->lm_work,  (void **)&m->rope_cos, (void **)&m->rope_sin};
    static_assert(sizeof(slots) / sizeof(slots[0]) == sizeof(sizes) / sizeof(sizes[0]),
                  "one slot per workspace size");
    for (size_t i = 0; i < sizeof(sizes) / sizeof(sizes[0]); i++) {
        *slots[i] = p;
        p += sizes[i];
    }
    m->kv_absmax_stride = 16 * c.n_kv_heads;  // two per workgroup, at most 8 workgroups per head
    e = hipMemsetAsync(m->ws, 0, total, ctx->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(m->rope_cos, cs.data(), cs.size() * 4, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess)
        e = hipMemcpyAsync(m->rope_sin, sn.data(), sn.size() * 4, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        hipFree(m->ws);
        delete m;
        return wm_hip_error(ctx, e, "wm_model_create");
    }
    *out = m;
    return WM_OK;
}

void wm_model_destroy(wm_model *m) {
    if (!m) return;
    hipSetDevice(m->device);
    for (auto &l : m->layers) {
        free_lin(l.q); free_lin(l.k); free_lin(l.v); free_lin(l.o);
        free_lin(l.gate); free_lin(l.up); free_lin(l.down);
        float *n[] = {l.attn_norm, l.attn_sub_norm, l.ffn_norm, l.ffn_sub_norm};
        for (float *x : n)
            if (x) hipFree(x);
    }
    if (m->embd) hipFree(m->embd);
    if (m->output_norm) hipFree(m->output_norm);
    if (m->ws) hipFree(m->ws);
    if (m->bws) hipFree(m->bws);
    if (m->b_scores) hipFree(m->b_scores);
    if (m->ring) hipHostFree(m->ring);
    for (hipEvent_t e : m->ring_ev)
        if (e) hipEventDestroy(e);
    delete m;
}

wm_status wm_model_set_layer(wm_model *m, uint32_t layer, const wm_tensor *attn_q,
                             const wm_tensor *attn_k, const wm_tensor *attn_v,
                             const wm_tensor *attn_output, const wm_tensor *ffn_gate,
                             const wm_tensor *ffn_up, const wm_tensor *ffn_down,
                             const float *attn_norm, const float *attn_sub_norm,
                             const float *ffn_norm, const float *ffn_sub_norm) {
    if (!m) return WM_E_ARG;
    wm_ctx *ctx = m->ctx;
    if (layer >= m->cfg.n_layers)
        return wm_set_error(ctx, WM_E_ARG, "layer %u >= n_layers %u", layer, m->cfg.n_layers);
    const uint64_t E = m->cfg.n_embd, F = m->cfg.n_ff, KV = m->kv_dim;
    // shapes of src/model/graph.rs role table (docs/BITLINEAR_I2S_MATVEC.md:26-34)
    const wm_tensor *ts[7] = {attn_q, attn_k, attn_v, attn_output, ffn_gate, ffn_up, ffn_down};
    const uint64_t ins[7] = {E, E, E, E, E, E, F}, outs[7] = {E, KV, KV, E, F, F, E};
    const char *names[7] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"};
    for (int i = 0; i < 7; i++) {
        if (!ts[i]) return wm_set_error(ctx, WM_E_ARG, "%s: missing tensor", names[i]);
        if (ts[i]->ctx != ctx) return wm_set_error(ctx, WM_E_ARG, "%s: tensor of another context", names[i]);
        if (ts[i]->type != WM_TYPE_I2S)
            return wm_set_error(ctx, WM_E_UNSUPPORTED_TYPE, "%s: tensor type %d is not I2_S", names[i],
                                ts[i]->type);
        if (ts[i]->in_dim != ins[i] || ts[i]->out_dim != outs[i])
            return wm_set_error(ctx, WM_E_SHAPE, "%s: shape [%llu, %llu] != [%llu, %llu]", names[i],
                                (unsigned long long)ts[i]->in_dim, (unsigned long long)ts[i]->out_dim,
                                (unsigned long long)ins[i], (unsigned long long)outs[i]);
    }
    if (!attn_norm || !attn_sub_norm || !ffn_norm || !ffn_sub_norm)
        return wm_set_error(ctx, WM_E_ARG, "layer %u: missing norm weights", layer);
    WM_HIP(ctx, hipSetDevice(ctx->device));
    dev_layer &L = m->layers[layer];
    dev_lin *dst[7] = {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down};
    wm_status st;
    for (int i = 0; i < 7; i++)
        if ((st = copy_lin(m, ts[i], ins[i], outs[i], dst[i], names[i]))) return st;
    if ((st = copy_norm(m, attn_norm, (uint32_t)E, &L.attn_norm, "attn_norm"))) return st;
    if ((st = copy_norm(m, attn_sub_norm, (uint32_t)E, &L.attn_sub_norm, "attn_sub_norm"))) return st;
    if ((st = copy_norm(m, ffn_norm, (uint32_t)E, &L.ffn_norm, "ffn_norm"))) return st;
    if ((st = copy_norm(m, ffn_sub_norm, (uint32_t)F, &L.ffn_sub_norm, "ffn_sub_norm"))) return st;
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    L.set = true;
    return WM_OK;
}

wm_status wm_model_set_output(wm_model *m, const wm_tensor *token_embd, const float *output_norm) {
    if (!m) return WM_E_ARG;
    wm_ctx *ctx = m->ctx;
    if (!token_embd || !output_norm) return wm_set_error(ctx, WM_E_ARG, "set_output: missing argument");
    if (token_embd->type != WM_TYPE_Q6K)
        return wm_set_error(ctx, WM_E_UNSUPPORTED_TYPE, "token_embd: tensor type %d is not Q6_K",
                            token_embd->type);
    if (token_embd->in_dim != m->cfg.n_embd || token_embd->out_dim != m->cfg.vocab_size)
        return wm_set_error(ctx, WM_E_SHAPE, "compute_logits: token_embd shape [%llu, %llu] != [%u, %u]",
                            (unsigned long long)token_embd->in_dim, (unsigned long long)token_embd->out_dim,
                            m->cfg.n_embd, m->cfg.vocab_size);
    WM_HIP(ctx, hipSetDevice(ctx->device));
    if (m->embd) WM_HIP(ctx, hipFree(m->embd));
    m->embd = nullptr;
    WM_HIP(ctx, hipMalloc((void **)&m->embd, token_embd->bytes));
    WM_HIP(ctx, hipMemcpyAsync(m->embd, token_embd->d, token_embd->bytes, hipMemcpyDeviceToDevice,
                               ctx->stream));
    m->embd_blocks = token_embd->n_blocks;
    m->embd_rowgroups = token_embd->n_rowgroups;
    wm_status st = copy_norm(m, output_norm, m->cfg.n_embd, &m->output_norm, "output_norm");
    if (st) return st;
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return WM_OK;
}

wm_status wm_kv_cache_create(wm_model *m, uint32_t max_seq_len, wm_kv_cache **out) {
    if (!m || !out) return WM_E_ARG;
    *out = nullptr;
    wm_ctx *ctx = m->ctx;
    if (max_seq_len == 0 || max_seq_len > m->cfg.context_length)
        return wm_set_error(ctx, WM_E_SHAPE, "KVCache::new: max_seq_len %u outside (0, context_length=%u]",
                            max_seq_len, m->cfg.context_length);
    WM_HIP(ctx, hipSetDevice(ctx->device));
    wm_kv_cache *kv = new wm_kv_cache();
    kv->m = m;
    kv->device = ctx->device;
    kv->max_seq = max_seq_len;
    const size_t nq = (size_t)m->cfg.n_layers * max_seq_len * m->kv_dim;
    const size_t ns = (size_t)m->cfg.n_layers * max_seq_len;
    hipError_t e = hipMalloc((void **)&kv->k, nq);
    if (e == hipSuccess) e = hipMalloc((void **)&kv->v, nq);
    if (e == hipSuccess) e = hipMalloc((void **)&kv->ks, ns * 4);
    if (e == hipSuccess) e = hipMalloc((void **)&kv->vs, ns * 4);
    if (e != hipSuccess) {
        wm_kv_cache_destroy(kv);
        return wm_hip_error(ctx, e, "KVCache::new");
    }
    *out = kv;
    return WM_OK;
}

void wm_kv_cache_destroy(wm_kv_cache *kv) {
    if (!kv) return;
    hipSetDevice(kv->device);
    if (kv->k) hipFree(kv->k);
    if (kv->v) hipFree(kv->v);
    if (kv->ks) hipFree(kv->ks);
    if (kv->vs) hipFree(kv->vs);
    delete kv;
}

uint32_t wm_kv_cache_position(const wm_kv_cache *kv) { return kv ? kv->pos : 0; }

wm_status wm_kv_cache_rollback(wm_kv_cache *kv, uint32_t position) {
    if (!kv) return WM_E_ARG;
    if (position < kv->pos) kv->pos = position;  // truncate (kv_cache.rs:141-149)
    return WM_OK;
}

wm_status wm_kv_cache_append_positions(wm_kv_cache *kv, const float *k, const float *v,
                                       uint32_t n_pos) {
    if (!kv || !k || !v) return WM_E_ARG;
    wm_model *m = kv->m;
    wm_ctx *ctx = m->ctx;
    if (n_pos == 0) return WM_OK;
    if ((uint64_t)kv->pos + n_pos > kv->max_seq)
        return wm_set_error(ctx, WM_E_SHAPE, "KVCache::append: already at max_seq_len %u", kv->max_seq);
    const size_t n = (size_t)n_pos * m->cfg.n_layers * m->kv_dim;
    void *scratch;
    wm_status st = wm_ctx_scratch(ctx, 2 * n * 4, &scratch);
    if (st) return st;
    float *dk = (float *)scratch, *dv = dk + n;
    WM_HIP(ctx, hipSetDevice(ctx->device));
    WM_HIP(ctx, hipMemcpyAsync(dk, k, n * 4, hipMemcpyHostToDevice, ctx->stream));
    WM_HIP(ctx, hipMemcpyAsync(dv, v, n * 4, hipMemcpyHostToDevice, ctx->stream));
    wm_launch_kv_append(dk, dv, m->kv_dim, m->cfg.n_layers, kv->pos, n_pos, kv->max_seq, kv->k, kv->ks,
                        kv->v, kv->vs, ctx->stream);
    WM_HIP(ctx, hipGetLastError());
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    kv->pos += n_pos;
    return WM_OK;
}

wm_status wm_kv_cache_append_position(wm_kv_cache *kv, const float *k, const float *v) {
    return wm_kv_cache_append_positions(kv, k, v, 1);
}

wm_status wm_kv_cache_read_raw(wm_kv_cache *kv, uint32_t layer, int8_t *k, float *k_scales,
                               int8_t *v, float *v_scales, uint32_t n_pos) {
    if (!kv) return WM_E_ARG;
    wm_ctx *ctx = kv->m->ctx;
    if (layer >= kv->m->cfg.n_layers || n_pos > kv->max_seq)
        return wm_set_error(ctx, WM_E_ARG, "read_raw: layer/position out of range");
    const size_t KV = kv->m->kv_dim, lay = (size_t)layer * kv->max_seq;
    WM_HIP(ctx, hipSetDevice(ctx->device));
    if (k) WM_HIP(ctx, hipMemcpyAsync(k, kv->k + lay * KV, n_pos * KV, hipMemcpyDeviceToHost, ctx->stream));
    if (v) WM_HIP(ctx, hipMemcpyAsync(v, kv->v + lay * KV, n_pos * KV, hipMemcpyDeviceToHost, ctx->stream));
    if (k_scales)
        WM_HIP(ctx, hipMemcpyAsync(k_scales, kv->ks + lay, n_pos * 4, hipMemcpyDeviceToHost, ctx->stream));
    if (v_scales)
        WM_HIP(ctx, hipMemcpyAsync(v_scales, kv->vs + lay, n_pos * 4, hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return WM_OK;
}

wm_status wm_kv_cache_read_into(wm_kv_cache *kv, uint32_t layer, float *out_k, float *out_v) {
    if (!kv || !out_k || !out_v) return WM_E_ARG;
    wm_ctx *ctx = kv->m->ctx;
    if (layer >= kv->m->cfg.n_layers)
        return wm_set_error(ctx, WM_E_SHAPE, "KVCache::read_into: layer_idx %u >= n_layers %u", layer,
                            kv->m->cfg.n_layers);
    const size_t KV = kv->m->kv_dim, lay = (size_t)layer * kv->max_seq, n = (size_t)kv->pos * KV;
    if (!n) return WM_OK;
    WM_HIP(ctx, hipSetDevice(ctx->device));
    void *buf = nullptr;
    wm_status st = wm_ctx_scratch(ctx, 2 * n * 4, &buf);
    if (st) return st;
    float *dk = static_cast<float *>(buf), *dv = dk + n;
    wm_launch_kv_dequant(kv->k + lay * KV, kv->ks + lay, kv->v + lay * KV, kv->vs + lay, kv->pos,
                         (uint32_t)KV, dk, dv, ctx->stream);
    WM_HIP(ctx, hipGetLastError());
    WM_HIP(ctx, hipMemcpyAsync(out_k, dk, n * 4, hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipMemcpyAsync(out_v, dv, n * 4, hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return WM_OK;
}

wm_status wm_forward_with_cache(wm_model *m, wm_kv_cache *kv, uint32_t token, uint32_t position,
                                float *hidden_out, float *layer_trace) {
    if (!m || !kv) return WM_E_ARG;
    wm_ctx *ctx = m->ctx;
    wm_status st = check_step(m, kv, token, position);
    if (st) return st;
    WM_HIP(ctx, hipSetDevice(ctx->device));
    float *trace_dev = nullptr;
    const size_t E = m->cfg.n_embd;
    if (layer_trace) {
        void *scratch;
        if ((st = wm_ctx_scratch(ctx, (size_t)m->cfg.n_layers * E * 4, &scratch))) return st;
        trace_dev = (float *)scratch;
    }
    WM_HIP(ctx, hipMemcpyAsync(m->dscalars, &token, 4, hipMemcpyHostToDevice, ctx->stream));
    if (!enqueue_forward(m, kv, step_pos{position, nullptr, 0}, trace_dev))
        return wm_set_error(ctx, WM_E_SHAPE, "forward_with_cache: no kernel for this model shape");
    WM_HIP(ctx, hipGetLastError());
    bool failed = false;
    if ((st = finish_step(m, kv, position, &failed))) return st;
    if (hidden_out)
        WM_HIP(ctx, hipMemcpyAsync(hidden_out, m->final_hidden, E * 4, hipMemcpyDeviceToHost, ctx->stream));
    if (layer_trace)
        WM_HIP(ctx, hipMemcpyAsync(layer_trace, trace_dev, (size_t)m->cfg.n_layers * E * 4,
                                   hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return WM_OK;
}

wm_status wm_forward_single_token_position_zero(wm_model *m, uint32_t token, float *hidden_out) {
    if (!m || !hidden_out) return WM_E_ARG;
    wm_ctx *ctx = m->ctx;
    if (!model_ready(m)) return wm_set_error(ctx, WM_E_STATE, "model: weights not fully set");
    if (token >= m->cfg.vocab_size)
        return wm_set_error(ctx, WM_E_SHAPE, "forward_single_token: token_id %u out of vocab range %u",
                            token, m->cfg.vocab_size);
    WM_HIP(ctx, hipSetDevice(ctx->device));
    WM_HIP(ctx, hipMemcpyAsync(m->dscalars, &token, 4, hipMemcpyHostToDevice, ctx->stream));
    if (!enqueue_forward(m, nullptr, step_pos{0, nullptr, 0}, nullptr))
        return wm_set_error(ctx, WM_E_SHAPE, "forward_single_token: no kernel for this model shape");
    WM_HIP(ctx, hipGetLastError());
    uint32_t flag = 0;
    WM_HIP(ctx, hipMemcpyAsync(&flag, m->dscalars + 2, 4, hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipMemcpyAsync(hidden_out, m->final_hidden, (size_t)m->cfg.n_embd * 4,
                               hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (flag) {
        uint32_t zero = 0;
        WM_HIP(ctx, hipMemcpyAsync(m->dscalars + 2, &zero, 4, hipMemcpyHostToDevice, ctx->stream));
        WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        return wm_set_error(ctx, WM_E_NONFINITE, "forward_single_token: non-finite hidden after layer %u",
                            flag - 1);
    }
    return WM_OK;
}

wm_status wm_decode_step(wm_model *m, wm_kv_cache *kv, uint32_t token, uint32_t position,
                         float *hidden_out, float *logits_out, uint32_t *next_token) {
    if (!m || !kv) return WM_E_ARG;
    wm_ctx *ctx = m->ctx;
    wm_status st = check_step(m, kv, token, position);
    if (st) return st;
    WM_HIP(ctx, hipSetDevice(ctx->device));
    WM_HIP(ctx, hipMemcpyAsync(m->dscalars, &token, 4, hipMemcpyHostToDevice, ctx->stream));
    if (!enqueue_forward(m, kv, step_pos{position, nullptr, 0}, nullptr))
        return wm_set_error(ctx, WM_E_SHAPE, "decode_step: no kernel for this model shape");
    // logits wanted: all of them in the reference's order; else the id-only path
    if (logits_out)
        wm_launch_q6k_logits_argmax(m->embd, m->embd_blocks, m->cfg.vocab_size, m->embd_rowgroups,
                                    m->final_hidden, m->logits, m->dscalars + 1, m->lm_work,
                                    ctx->stream);
    else
        wm_launch_q6k_argmax_fast(m->embd, m->embd_blocks, m->cfg.vocab_size, m->embd_rowgroups,
                                  m->final_hidden, m->logits, m->dscalars + 1, m->lm_work,
                                  true, ctx->stream);  // output_norm wrote the prep area
    WM_HIP(ctx, hipGetLastError());
    bool failed = false;
    if ((st = finish_step(m, kv, position, &failed))) return st;
    const size_t E = m->cfg.n_embd;
    if (hidden_out)
        WM_HIP(ctx, hipMemcpyAsync(hidden_out, m->final_hidden, E * 4, hipMemcpyDeviceToHost, ctx->stream));
    if (logits_out)
        WM_HIP(ctx, hipMemcpyAsync(logits_out, m->logits, (size_t)m->cfg.vocab_size * 4,
                                   hipMemcpyDeviceToHost, ctx->stream));
    uint32_t next = 0;
    WM_HIP(ctx, hipMemcpyAsync(&next, m->dscalars + 1, 4, hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (next_token) *next_token = next;
    return WM_OK;
}

wm_status wm_debug_rerun_role(wm_model *m, wm_kv_cache *kv, uint32_t layer, uint32_t role,
                              uint32_t reps) {
    if (!m || !kv) return WM_E_ARG;
    wm_ctx *ctx = m->ctx;
    if (!model_ready(m)) return wm_set_error(ctx, WM_E_STATE, "model: weights not fully set");
    if (kv->m != m) return wm_set_error(ctx, WM_E_ARG, "kv cache belongs to another model");
    if (kv->pos == 0) return wm_set_error(ctx, WM_E_STATE, "rerun_role: no decode step has run");
    if (layer >= m->cfg.n_layers || role >= ROLE_ALL)
        return wm_set_error(ctx, WM_E_ARG, "rerun_role: layer %u / role %u out of range", layer, role);
    WM_HIP(ctx, hipSetDevice(ctx->device));
    float *const H[2] = {m->hidden, m->hidden2};
    for (uint32_t i = 0; i < reps; i++) {
        int cur = layer == 0 ? 0 : 1;  // the residual buffer layer `layer` starts from
        if (!enqueue_layer(m, kv, layer, step_pos{kv->pos - 1, nullptr, 0}, H, cur, nullptr, (int)role))
            return wm_set_error(ctx, WM_E_SHAPE, "rerun_role: no kernel for this model shape");
    }
    WM_HIP(ctx, hipGetLastError());
    return WM_OK;
}

wm_status wm_greedy_generate(wm_model *m, wm_kv_cache *kv, const uint32_t *prompt,
                             uint32_t n_prompt, uint32_t max_new, int64_t eos, uint32_t *out_ids,
                             uint32_t *n_out) {
    if (!m || !kv || !n_out || (max_new && !out_ids)) return WM_E_ARG;
    wm_ctx *ctx = m->ctx;
    *n_out = 0;
    if (!prompt || n_prompt == 0)
        return wm_set_error(ctx, WM_E_ARG, "greedy_generate_with_cache: prompt_ids must not be empty");
    for (uint32_t i = 0; i < n_prompt; i++)
        if (prompt[i] >= m->cfg.vocab_size)
            return wm_set_error(ctx, WM_E_SHAPE,
                                "greedy_generate_with_cache: prompt token %u (idx %u) out of vocab range %u",
                                prompt[i], i, m->cfg.vocab_size);
    if ((uint64_t)kv->pos + n_prompt + (max_new ? max_new - 1 : 0) > kv->max_seq)
        return wm_set_error(ctx, WM_E_SHAPE, "greedy_generate_with_cache: budget exceeds max_seq_len %u",
                            kv->max_seq);
    const uint32_t start = kv->pos;
    wm_status st;
    if ((st = prefill_tokens(m, kv, prompt, n_prompt - 1, nullptr))) return st;
    if ((st = check_step(m, kv, prompt[n_prompt - 1], kv->pos))) {
        kv->pos = start;
        return st;
    }
    // The decode steps are enqueued ahead of the host, up to kAhead in
    // flight.  The step's token and position live on the device
    // (dscalars[1] and [3]): step k embeds the id in dscalars[1] (the
    // prompt's last token for k = 0), its lm-head writes the next id there,
    // copies it with the cumulative error flag to ring slot (position % 16)
    // in pinned host memory and advances the position, so no step waits for
    // the host.  The host reads slot k after step k's event and applies
    // generate_with_cache's rules (generate.rs:111-189) in order: a
    // non-finite step fails the call, EOS ends it.  Steps enqueued past the
    // end only wrote cache rows beyond the final position, which the cache
    // treats as free (kv_cache.rs:141-149).
    constexpr uint32_t kRing = 16, kAhead = 8;
    WM_HIP(ctx, hipSetDevice(ctx->device));
    if (!m->ring) {
        WM_HIP(ctx, hipHostMalloc((void **)&m->ring, kRing * 2 * sizeof(uint32_t), hipHostMallocMapped));
        WM_HIP(ctx, hipHostGetDevicePointer((void **)&m->ring_dev, m->ring, 0));
        for (hipEvent_t &e : m->ring_ev) WM_HIP(ctx, hipEventCreateWithFlags(&e, hipEventDisableTiming));
    }
    const uint32_t pos0 = kv->pos;
    // steps needed: step k yields id k; ids 0..max_new-1 are wanted, and at
    // least step 0 runs (it also appends the prompt's last token)
    const uint32_t n_steps = max_new ? max_new : 1;
    const wm_step_tail tail{m->dscalars + 3, m->ring_dev, m->dscalars + 2, kRing - 1};
    // step k at position pos0 + k: the kernels read the position from the
    // device, and the host sizes the attention launches for it (a test hook
    // sizes them for a few positions more)
    const bool loose = (ctx->fused_debug & WM_FUSED_DEBUG_ATTN_LOOSE_COUNT) != 0;
    const auto enqueue_step = [&](uint32_t k) -> bool {
        const uint32_t n_exp = pos0 + k + 1;
        const uint32_t n_max = loose ? std::min(n_exp + 9u, std::min(m->cfg.context_length, 4096u)) : n_exp;
        if (!enqueue_forward(m, kv, step_pos{0, m->dscalars + 3, n_max}, nullptr, m->dscalars + 1))
            return false;
        wm_launch_q6k_argmax_fast(m->embd, m->embd_blocks, m->cfg.vocab_size, m->embd_rowgroups,
                                  m->final_hidden, m->logits, m->dscalars + 1, m->lm_work, true,
                                  ctx->stream, &tail);
        return hipEventRecord(m->ring_ev[k % kRing], ctx->stream) == hipSuccess;
    };
    m->ring[0] = prompt[n_prompt - 1];
    m->ring[1] = 0;
    m->ring[2] = pos0;
    WM_HIP(ctx, hipMemcpyAsync(m->dscalars + 1, m->ring, 12, hipMemcpyHostToDevice, ctx->stream));
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));  // the ring is written by the steps below
    uint32_t enq = 0, n = 0, done = 0;
    bool stop = false;
    uint32_t failed_flag = 0;
    while (done < n_steps && !stop) {
        while (enq < n_steps && enq < done + kAhead) {
            if (!enqueue_step(enq)) {
                hipStreamSynchronize(ctx->stream);
                kv->pos = start;
                return wm_set_error(ctx, WM_E_SHAPE, "greedy_generate: could not enqueue a decode step");
            }
            enq++;
        }
        WM_HIP(ctx, hipEventSynchronize(m->ring_ev[done % kRing]));
        const uint32_t *slot = m->ring + 2 * ((pos0 + done) % kRing);
        const uint32_t id = slot[0], flag = slot[1];
        if (flag) {
            failed_flag = flag;
            break;
        }
        done++;  // step done-1 succeeded: the cache holds its position
        // the reference's loop: stop at EOS, else record the id and decode it
        if (eos >= 0 && (int64_t)id == eos) stop = true;
        else if (n < max_new) out_ids[n++] = id;
    }
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    WM_HIP(ctx, hipGetLastError());
    if (failed_flag) {
        m->ring[0] = 0;  // all reads of the ring are over
        WM_HIP(ctx, hipMemcpyAsync(m->dscalars + 2, m->ring, 4, hipMemcpyHostToDevice, ctx->stream));
        WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
        kv->pos = start;
        return step_flag_error(ctx, "forward_with_cache", failed_flag);
    }
    if (enq > done) {
        // Steps queued past an EOS stop ran as well, and the error flag is
        // cumulative: one of them (the EOS token's own step, say) may have
        // raised it.  The steps kept were all found finite above, so the
        // flag is cleared rather than left to fail the next call.
        m->ring[0] = 0;
        WM_HIP(ctx, hipMemcpyAsync(m->dscalars + 2, m->ring, 4, hipMemcpyHostToDevice, ctx->stream));
        WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    }
    kv->pos = pos0 + done;
    *n_out = n;
    return WM_OK;
}

}  // extern "C"

namespace {

// Prefill `n` tokens at the cache's position: ragged-batch calls of up to
// kPrefillChunk tokens (bit-identical to the token-by-token prefill of
// generate.rs:151-160), or forward_with_cache per token where the batch
// kernels do not cover the shape.  On an error the cache goes back to where
// it started.
wm_status prefill_tokens(wm_model *m, wm_kv_cache *kv, const uint32_t *tokens, uint32_t n,
                         float *last_hidden) {
    const uint32_t start = kv->pos;
    const bool batched = batch_supported(m);
    for (uint32_t off = 0; off < n;) {
        const uint32_t len = batched ? std::min(n - off, kPrefillChunk) : 1;
        float *lh = off + len == n ? last_hidden : nullptr;
        const wm_status st = batched ? wm_batch_forward(m, &kv, 1, &len, tokens + off, lh, nullptr)
                                     : wm_forward_with_cache(m, kv, tokens[off], kv->pos, lh, nullptr);
        if (st) {
            kv->pos = start;
            return st;
        }
        off += len;
    }
    return WM_OK;
}

// One decode step whose exact logits stay in m->logits on the device
// (forward_with_cache + compute_logits_from_graph).
wm_status step_with_logits(wm_model *m, wm_kv_cache *kv, uint32_t token) {
    wm_ctx *ctx = m->ctx;
    const uint32_t position = kv->pos;
    wm_status st = check_step(m, kv, token, position);
    if (st) return st;
    WM_HIP(ctx, hipSetDevice(ctx->device));
    WM_HIP(ctx, hipMemcpyAsync(m->dscalars, &token, 4, hipMemcpyHostToDevice, ctx->stream));
    if (!enqueue_forward(m, kv, step_pos{position, nullptr, 0}, nullptr))
        return wm_set_error(ctx, WM_E_SHAPE, "decode_step: no kernel for this model shape");
    wm_launch_q6k_logits_argmax(m->embd, m->embd_blocks, m->cfg.vocab_size, m->embd_rowgroups,
                                m->final_hidden, m->logits, m->dscalars + 1, m->lm_work, ctx->stream);
    WM_HIP(ctx, hipGetLastError());
    bool failed = false;
    return finish_step(m, kv, position, &failed);
}

}  // namespace

extern "C" {

wm_status wm_prefill(wm_model *m, wm_kv_cache *kv, const uint32_t *tokens, uint32_t n,
                     float *last_hidden) {
    if (!m || !kv) return WM_E_ARG;
    wm_ctx *ctx = m->ctx;
    if (!tokens || n == 0) return wm_set_error(ctx, WM_E_ARG, "prefill: token_ids must not be empty");
    if (!model_ready(m)) return wm_set_error(ctx, WM_E_STATE, "model: weights not fully set");
    if (kv->m != m) return wm_set_error(ctx, WM_E_ARG, "kv cache belongs to another model");
    for (uint32_t i = 0; i < n; i++)
        if (tokens[i] >= m->cfg.vocab_size)
            return wm_set_error(ctx, WM_E_SHAPE, "forward_with_cache: token_id %u out of vocab range %u",
                                tokens[i], m->cfg.vocab_size);
    if ((uint64_t)kv->pos + n > kv->max_seq)
        return wm_set_error(ctx, WM_E_SHAPE, "KVCache::append: %u tokens would pass max_seq_len %u", n,
                            kv->max_seq);
    return prefill_tokens(m, kv, tokens, n, last_hidden);
}

wm_status wm_generate_with_sampler(wm_model *m, wm_kv_cache *kv, const uint32_t *prompt,
                                   uint32_t n_prompt, uint32_t max_new, int64_t eos,
                                   const uint32_t *stop_ids, uint32_t n_stop, wm_sampler *s,
                                   uint32_t *out_ids, uint32_t *n_out) {
    if (!m || !kv || !s || !n_out || (max_new && !out_ids) || (n_stop && !stop_ids)) return WM_E_ARG;
    wm_ctx *ctx = m->ctx;
    *n_out = 0;
    if (wm_sampler_ctx(s) != ctx) return wm_set_error(ctx, WM_E_ARG, "sampler of another context");
    if (!prompt || n_prompt == 0)
        return wm_set_error(ctx, WM_E_ARG, "generate_with_cache_and_sampler: prompt_ids must not be empty");
    for (uint32_t i = 0; i < n_prompt; i++)
        if (prompt[i] >= m->cfg.vocab_size)
            return wm_set_error(ctx, WM_E_SHAPE,
                                "generate_with_cache_and_sampler: prompt token %u (idx %u) out of vocab range %u",
                                prompt[i], i, m->cfg.vocab_size);
    if ((uint64_t)kv->pos + n_prompt + (max_new ? max_new - 1 : 0) > kv->max_seq)
        return wm_set_error(ctx, WM_E_SHAPE,
                            "generate_with_cache_and_sampler: budget exceeds max_seq_len %u", kv->max_seq);
    if (!model_ready(m)) return wm_set_error(ctx, WM_E_STATE, "model: weights not fully set");
    if (kv->m != m) return wm_set_error(ctx, WM_E_ARG, "kv cache belongs to another model");
    // the prompt enters the repetition-penalty history (generate.rs:229-233)
    for (uint32_t i = 0; i < n_prompt; i++) wm_sampler_observe(s, prompt[i]);
    const uint32_t start = kv->pos;
    wm_status st = prefill_tokens(m, kv, prompt, n_prompt - 1, nullptr);
    if (!st) st = step_with_logits(m, kv, prompt[n_prompt - 1]);
    if (st) {
        kv->pos = start;
        return st;
    }
    uint32_t n = 0;
    for (uint32_t step = 0; step < max_new; step++) {
        uint32_t next = 0;
        if ((st = wm_sampler_run(s, m->logits, m->cfg.vocab_size, &next))) break;
        bool stop = eos >= 0 && (int64_t)next == eos;
        for (uint32_t j = 0; j < n_stop && !stop; j++) stop = stop_ids[j] == next;
        if (stop) break;
        out_ids[n++] = next;
        wm_sampler_observe(s, next);
        if (step + 1 < max_new && (st = step_with_logits(m, kv, next))) break;
    }
    if (st) {
        // The reference builds its cache inside the call and drops it with
        // the error (generate.rs:237); here the cache is the caller's,
        // so it goes back to where the call found it, as after a failed
        // greedy generation.  The sampler is the caller's in both: its
        // history and rng keep every id sampled before the error.
        kv->pos = start;
        n = 0;
    }
    *n_out = n;
    return st;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// internal interface for the continuous-batching driver (server.cpp)
// ---------------------------------------------------------------------------

wm_ctx *wm_model_ctx(const wm_model *m) { return m->ctx; }
const wm_model_config &wm_model_cfg(const wm_model *m) { return m->cfg; }
bool wm_model_batch_ready(const wm_model *m) { return model_ready(m) && batch_supported(m); }
uint32_t wm_kv_max_seq(const wm_kv_cache *kv) { return kv->max_seq; }

// Exact logits (compute_logits' order) of row `row` of the last batch step's
// final hidden rows, into the model's logits buffer on the device.
wm_status wm_batch_row_logits(wm_model *m, uint32_t row, const float **d_logits) {
    wm_ctx *ctx = m->ctx;
    WM_HIP(ctx, hipSetDevice(ctx->device));
    wm_launch_q6k_logits_argmax(m->embd, m->embd_blocks, m->cfg.vocab_size, m->embd_rowgroups,
                                m->b_final + (size_t)row * m->cfg.n_embd, m->logits, m->dscalars + 1,
                                m->lm_work, ctx->stream);
    WM_HIP(ctx, hipGetLastError());
    *d_logits = m->logits;
    return WM_OK;
}

// The id-only argmax of each sequence of the last batch step (want_next).
wm_status wm_batch_next_ids(wm_model *m, uint32_t n, uint32_t *out) {
    wm_ctx *ctx = m->ctx;
    WM_HIP(ctx, hipMemcpyAsync(out, m->b_next, (size_t)n * 4, hipMemcpyDeviceToHost, ctx->stream));
    WM_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return WM_OK;
}
