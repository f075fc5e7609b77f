/*
 * willamette_hip.h — C ABI of the MI355X (gfx950) BitNet b1.58 decode path.
 *
 * Drop-in boundary for project-willamette's CPU kernels: every entry point
 * below names the reference function it replaces (file:line in
 * project-willamette).  Plain pointers and sizes only; no HIP or torch types.
 *
 * Conventions
 *  - Host-pointer entry points (no suffix) take the same slices the Rust API
 *    takes (`&[f32]`, `&mut [f32]`), copy them to the device, run, and copy
 *    results back before returning.  `_dev` entry points take device pointers
 *    (from wm_dev_alloc) and are asynchronous on the context's stream.
 *  - Every call validates all arguments before touching the device; on a
 *    validation error nothing is written to any output (the reference's
 *    `Err(..)` before any work, src/model/bitlinear.rs:150-199).
 *  - A context is single-threaded: callers serialise calls on one context
 *    (the reference decode loop is single-threaded, src/model/stage_timing.rs:32-36).
 *  - Numerics: the device path reproduces the reference's x86_64 arithmetic
 *    bit for bit (int8 activations, i32 dots, Q6_K values, f32 reductions in
 *    the reference's sequential order, glibc-identical expf).
 */
#ifndef WILLAMETTE_HIP_H
#define WILLAMETTE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes; the Rust shim maps them onto WillametteError (src/error.rs:9-57). */
typedef enum wm_status {
    WM_OK = 0,
    WM_E_UNSUPPORTED_TYPE = 1, /* WillametteError::UnsupportedTensorType (src/error.rs:29) */
    WM_E_SHAPE = 2,            /* WillametteError::GgufParse shape/length errors (src/error.rs:14) */
    WM_E_NONFINITE = 3,        /* non-finite scale (src/gguf/tensor.rs:302-307) or hidden
                                  (src/model/cached_forward.rs:511-521) */
    WM_E_OOM = 4,              /* device allocation failed */
    WM_E_HIP = 5,              /* HIP runtime error; wm_last_error() has the text */
    WM_E_ARG = 6,              /* null pointer / out-of-range argument */
    WM_E_STATE = 7,            /* call out of protocol order (e.g. KV position mismatch,
                                  src/model/cached_forward.rs:271-305) */
    WM_E_PARSE = 8,            /* WillametteError::GgufParse from the GGUF reader and the
                                  model graph's dtype checks (src/error.rs:13-14) */
    WM_E_MAGIC = 9,            /* WillametteError::InvalidMagic (src/error.rs:16-17) */
    WM_E_VERSION = 10,         /* WillametteError::UnsupportedVersion (src/error.rs:19-20) */
    WM_E_ARCH = 11,            /* WillametteError::UnsupportedArchitecture (src/error.rs:22-23) */
    WM_E_METADATA = 12,        /* WillametteError::MissingMetadata: a metadata key or a
                                  required tensor (src/error.rs:25-26) */
    WM_E_BOUNDS = 13,          /* WillametteError::TensorOutOfBounds (src/error.rs:40-46) */
    WM_E_IO = 14,              /* WillametteError::Io / InvalidPath (src/error.rs:10-11, 37-38) */
    WM_E_NOT_IMPLEMENTED = 15  /* WillametteError::NotImplemented (src/error.rs:34-35) */
} wm_status;

typedef enum wm_tensor_type {
    WM_TYPE_I2S = 36, /* GgmlType::BitNetI2S raw id (src/gguf/types.rs:14-60) */
    WM_TYPE_Q6K = 14  /* GgmlType::Q6K raw id */
} wm_tensor_type;

typedef struct wm_ctx wm_ctx;
typedef struct wm_tensor wm_tensor;
typedef struct wm_model wm_model;
typedef struct wm_kv_cache wm_kv_cache;
typedef struct wm_gguf wm_gguf;

/* ---- context --------------------------------------------------------- */

/* One device, one stream.  Replaces the process-wide kernel selection
 * (src/model/dispatch.rs:111-114, :159-184) for a `Kernel::Hip` arm. */
wm_status wm_ctx_create(int device, wm_ctx **out);
void wm_ctx_destroy(wm_ctx *ctx);
/* Text of the last error on this context ("" if none).  Owned by ctx. */
const char *wm_last_error(const wm_ctx *ctx);
/* The context's hipStream_t, as an opaque pointer, for callers that time or
 * order their own work against the library's. */
void *wm_ctx_stream(wm_ctx *ctx);
wm_status wm_ctx_synchronize(wm_ctx *ctx);
const char *wm_version(void);

/* Device buffers for the `_dev` entry points. */
wm_status wm_dev_alloc(wm_ctx *ctx, size_t bytes, void **out);
wm_status wm_dev_free(wm_ctx *ctx, void *ptr);
wm_status wm_memcpy_h2d(wm_ctx *ctx, void *dst, const void *src, size_t bytes);
wm_status wm_memcpy_d2h(wm_ctx *ctx, void *dst, const void *src, size_t bytes);

/* ---- tensors (TensorView, src/gguf/tensor.rs:21-54) ------------------ */

/* Upload an I2_S BitLinear weight: `packed` is TensorView::data (out_dim rows
 * of in_dim/4 bytes, src/gguf/tensor.rs:45), `scale_block` is
 * TensorView::scale_data (the 32-byte trailing block whose first 4 bytes are
 * the LE f32 scale, src/gguf/tensor.rs:278-309).  Shape is GGUF order
 * [in_dim, out_dim].  Rejects in_dim not a positive multiple of 128 and
 * packed_len < in_dim/4*out_dim (src/model/bitlinear_sse2.rs:129-177), a
 * missing/short scale block, and a non-finite scale.  Host bytes are only
 * read during the call; the library owns the device copy. */
wm_status wm_tensor_upload_i2s(wm_ctx *ctx, const uint8_t *packed, size_t packed_len,
                               const uint8_t *scale_block, size_t scale_len, uint64_t in_dim,
                               uint64_t out_dim, wm_tensor **out);
/* Upload a Q6_K matrix of n_rows rows of row_len values (GGUF shape
 * [row_len, n_rows]); row_len must be a positive multiple of 256 and
 * len == n_rows * row_len/256 * 210 (src/gguf/tensor.rs:104-105, 206-231). */
wm_status wm_tensor_upload_q6k(wm_ctx *ctx, const uint8_t *blocks, size_t len, uint64_t row_len,
                               uint64_t n_rows, wm_tensor **out);
void wm_tensor_destroy(wm_tensor *t);
/* shape[0] = in_dim / row_len, shape[1] = out_dim / n_rows; type = wm_tensor_type */
wm_status wm_tensor_info(const wm_tensor *t, uint64_t shape[2], int *type, float *scale);

/* ---- BitLinear I2_S (src/model/bitlinear.rs, bitlinear_sse2.rs) ------ */

/* output = w_scale * in_scale * (ternary(W) . q(input)), q = per-vector
 * absmax int8 (src/model/bitlinear_sse2.rs:285-304), i32 accumulation.
 * Replaces bitlinear_i2s_matvec_f32 (src/model/bitlinear.rs:67) /
 * linear_matvec_f32 for I2_S (src/model/linear.rs:17). */
wm_status wm_bitlinear_i2s_matvec_f32(wm_ctx *ctx, const wm_tensor *w, const float *input,
                                      size_t input_len, float *output, size_t output_len);
/* Same, with taps: the quantised activation (in_dim i8), its scale, and the
 * per-row i32 dot before the f32 epilogue (any may be NULL). */
wm_status wm_bitlinear_i2s_matvec_f32_debug(wm_ctx *ctx, const wm_tensor *w, const float *input,
                                            size_t input_len, float *output, size_t output_len,
                                            int8_t *act, float *act_scale, int32_t *acc);
/* The scalar f32 path: no int8 activations; per row, f32 sums of the
 * inputs under +1 and under -1 codes in the packed byte order, then
 * out = scale * (pos - neg).  Replaces bitlinear_i2s_matvec_f32_scalar
 * (src/model/bitlinear.rs:146-233), the dispatcher's fallback arm
 * (src/model/bitlinear.rs:140); bit-identical to it, NaN/inf inputs
 * included (a NaN under a 0 code is skipped, as there). */
wm_status wm_bitlinear_i2s_matvec_f32_scalar(wm_ctx *ctx, const wm_tensor *w, const float *input,
                                             size_t input_len, float *output, size_t output_len);
/* Device-pointer form of the scalar path (one launch, no workspace). */
wm_status wm_bitlinear_i2s_matvec_f32_scalar_dev(wm_ctx *ctx, const wm_tensor *w,
                                                 const float *d_input, float *d_output);
/* Device-pointer form: d_input[in_dim] f32 -> d_output[out_dim] f32. */
wm_status wm_bitlinear_i2s_matvec_f32_dev(wm_ctx *ctx, const wm_tensor *w, const float *d_input,
                                          float *d_output);
/* Batched device form over `n_copies` weight tensors of one shape sharing one
 * input, one launch (used to measure HBM bandwidth on matrices far smaller
 * than the 256 MB Infinity Cache).  d_outputs is n_copies x out_dim. */
wm_status wm_bitlinear_i2s_matvec_f32_multi_dev(wm_ctx *ctx, const wm_tensor *const *ws,
                                                uint32_t n_copies, const float *d_input,
                                                float *d_outputs);

/* No counterpart in the reference: wm_bitlinear_i2s_matvec_f32_dev without
 * any device allocation, for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  Its
 * working memory is a fixed 4 MiB device array per GPU, held until the
 * process ends; shapes whose activation codes, scale record and partial dots
 * need more (far above BitNet-2B's, e.g. more than 65536 output rows) are
 * rejected with WM_E_SHAPE.  Calls that overlap on one GPU (other streams or
 * contexts) share that array and race.  Output identical to
 * wm_bitlinear_i2s_matvec_f32_dev. */
wm_status wm_bitlinear_i2s_matvec_f32_dev_noalloc(wm_ctx *ctx, const wm_tensor *w,
                                                  const float *d_input, float *d_output);

/* Batched BitLinear: m activation rows x [m][in_dim] (device), each row
 * quantised on its own (per-token absmax int8, src/model/bitlinear_sse2.rs:285-304),
 * y[m][out_dim] (device).  Row r of y is bit-identical to
 * wm_bitlinear_i2s_matvec_f32 on row r of x: the ternary x int8 products
 * are exact i32 sums, here from int8 MFMA.  Used by the ragged batch
 * (multi_token_forward's per-token linear_matvec_f32 calls,
 * src/model/multi_forward.rs:107-110, :176, :202-203, :226). */
wm_status wm_bitlinear_i2s_matmul_f32_dev(wm_ctx *ctx, const wm_tensor *w, const float *d_x,
                                          uint32_t m, float *d_y);
/* Host-slice form: x_len == m * in_dim, y_len == m * out_dim. */
wm_status wm_bitlinear_i2s_matmul_f32(wm_ctx *ctx, const wm_tensor *w, const float *x,
                                      size_t x_len, uint32_t m, float *y, size_t y_len);

/* ---- FFN block (src/model/ffn.rs) ------------------------------------ */

/* ffn_block_forward (src/model/ffn.rs:73-136) for one token: RMSNorm of x
 * (ffn_norm_weight, eps), the gate and up BitLinears, relu(gate)^2 * up,
 * RMSNorm of that (ffn_sub_norm_weight, width n_ff), and the down BitLinear
 * into output; no residual add.  n_embd = gate's in_dim, n_ff = gate's
 * out_dim; up must be [n_embd, n_ff] and down [n_ff, n_embd].  The
 * reference's length checks in its order: x_len, ffn_norm_len and output_len
 * against n_embd, ffn_sub_norm_len against n_ff (WM_E_SHAPE).  Bit-identical
 * to the reference: the norms' sums in its sequential order, the BitLinears
 * exact. */
wm_status wm_ffn_block_forward(wm_ctx *ctx, const float *x, size_t x_len, const float *ffn_norm_weight,
                               size_t ffn_norm_len, const wm_tensor *gate, const wm_tensor *up,
                               const wm_tensor *down, const float *ffn_sub_norm_weight,
                               size_t ffn_sub_norm_len, float eps, float *output, size_t output_len);
/* Device-pointer form (x, the two norm weights and output in device memory;
 * the gate and up outputs in the context's scratch): two launches. */
wm_status wm_ffn_block_forward_dev(wm_ctx *ctx, const float *d_x, const float *d_ffn_norm_weight,
                                   const wm_tensor *gate, const wm_tensor *up, const wm_tensor *down,
                                   const float *d_ffn_sub_norm_weight, float eps, float *d_output);

/* ---- Q6_K / lm-head (src/model/q6_k.rs, lm_head.rs) ------------------ */

/* Dequantise one row (src/model/q6_k.rs:59-69); embedding gather for a
 * Q6_K token_embd (src/model/primitives.rs:120-210). */
wm_status wm_q6k_dequantize_row(wm_ctx *ctx, const wm_tensor *t, uint64_t row, float *out,
                                size_t out_len);
/* logits[v] = q6_k::dot_row(row v, hidden) for every row, in the SSE2
 * accumulation order (src/model/lm_head.rs:29-108, q6_k_sse2.rs:46-116). */
wm_status wm_compute_logits(wm_ctx *ctx, const wm_tensor *token_embd, const float *hidden,
                            size_t hidden_len, float *logits, size_t vocab);
/* compute_logits + argmax (src/model/lm_head.rs:161-174: first index of the
 * maximum).  With `logits` non-NULL every logit is the reference's, bit for
 * bit.  With `logits` NULL only the id is computed: a bandwidth-bound
 * fixed-point pass bounds every row's distance from the reference's value,
 * and only rows whose bound reaches the best row are recomputed in the
 * reference's order, so the id is still exactly the reference's argmax.
 * Rows above 8192 values or beyond 4194304 rows: WM_E_SHAPE. */
wm_status wm_logits_argmax(wm_ctx *ctx, const wm_tensor *token_embd, const float *hidden,
                           size_t hidden_len, float *logits, uint32_t *argmax);
/* Device form: d_logits may be NULL (then the id-only path above runs);
 * d_argmax is one uint32 in device memory. */
wm_status wm_logits_argmax_dev(wm_ctx *ctx, const wm_tensor *token_embd, const float *d_hidden,
                               float *d_logits, uint32_t *d_argmax);
/* argmax over a host slice (src/model/lm_head.rs:161-174); WM_E_ARG when
 * n == 0 (the reference's None). */
wm_status wm_argmax(const float *logits, size_t n, uint32_t *out);

/* ---- model + KV cache (src/model/{graph,kv_cache,cached_forward,generate}.rs) */

/* ModelConfig fields the BitNet forward reads (src/model/config.rs:21-44). */
typedef struct wm_model_config {
    uint32_t n_layers;       /* block_count */
    uint32_t n_embd;         /* embedding_length */
    uint32_t n_ff;           /* feed_forward_length */
    uint32_t n_heads;        /* head_count */
    uint32_t n_kv_heads;     /* head_count_kv */
    uint32_t head_dim;       /* embedding_length / head_count */
    uint32_t n_rot;          /* rope_dimension_count */
    uint32_t vocab_size;
    uint32_t context_length; /* upper bound for KV caches */
    float rms_eps;           /* layer_norm_rms_epsilon */
    float rope_freq_base;    /* rope_freq_base (NEOX RoPE, src/model/primitives.rs:326-341) */
} wm_model_config;

/* ModelGraph::from_gguf (src/model/graph.rs:79-237): a device-resident
 * model.  Tensors passed to wm_model_set_* are copied into the model's own
 * fused device layout; the caller may destroy them afterwards. */
wm_status wm_model_create(wm_ctx *ctx, const wm_model_config *cfg, wm_model **out);
void wm_model_destroy(wm_model *m);
/* LayerWeights (src/model/graph.rs:23-53): seven I2_S BitLinears and four
 * f32 norm vectors (host pointers, n_embd or n_ff values). */
wm_status wm_model_set_layer(wm_model *m, uint32_t layer, const wm_tensor *attn_q,
                             const wm_tensor *attn_k, const wm_tensor *attn_v,
                             const wm_tensor *attn_output, const wm_tensor *ffn_gate,
                             const wm_tensor *ffn_up, const wm_tensor *ffn_down,
                             const float *attn_norm, const float *attn_sub_norm,
                             const float *ffn_norm, const float *ffn_sub_norm);
/* Tied Q6_K token_embd / lm_head (src/model/graph.rs:134-163) and output_norm. */
wm_status wm_model_set_output(wm_model *m, const wm_tensor *token_embd, const float *output_norm);

/* KVCache::try_new (src/model/kv_cache.rs:67-131): i8 codes + one f32 scale
 * per token per layer for K and V, on the device. */
wm_status wm_kv_cache_create(wm_model *m, uint32_t max_seq_len, wm_kv_cache **out);
void wm_kv_cache_destroy(wm_kv_cache *kv);
uint32_t wm_kv_cache_position(const wm_kv_cache *kv);            /* :121-128 */
wm_status wm_kv_cache_rollback(wm_kv_cache *kv, uint32_t position); /* :141-149 */
/* KVCache::append (src/model/kv_cache.rs:154-185) for every layer at the next
 * position: k and v are host f32, n_layers x kv_dim, layer-major. */
wm_status wm_kv_cache_append_position(wm_kv_cache *kv, const float *k, const float *v);
/* Same for n_pos positions at once: k and v are n_pos x n_layers x kv_dim. */
wm_status wm_kv_cache_append_positions(wm_kv_cache *kv, const float *k, const float *v,
                                       uint32_t n_pos);
/* Raw i8 codes and scales of one layer's first n_pos positions (any output
 * may be NULL). */
wm_status wm_kv_cache_read_raw(wm_kv_cache *kv, uint32_t layer, int8_t *k, float *k_scales,
                               int8_t *v, float *v_scales, uint32_t n_pos);
/* KVCache::read_into (src/model/kv_cache.rs:192-219): one layer's K and V
 * dequantised (code as f32 * the position's scale) for positions
 * [0, wm_kv_cache_position): out_k and out_v (host) each hold position x
 * kv_dim floats.  A layer out of range is WM_E_SHAPE (the reference's
 * GgufParse). */
wm_status wm_kv_cache_read_into(wm_kv_cache *kv, uint32_t layer, float *out_k, float *out_v);

/* forward_with_cache_into (src/model/cached_forward.rs:164-261): embed
 * `token`, run every layer at `position` (== wm_kv_cache_position), apply
 * output_norm.  hidden_out (n_embd, host, nullable) receives the final
 * hidden; layer_trace (n_layers x n_embd, host, nullable) the hidden after
 * each layer.  On a non-finite hidden the cache is rolled back and
 * WM_E_NONFINITE returned with outputs untouched. */
wm_status wm_forward_with_cache(wm_model *m, wm_kv_cache *kv, uint32_t token, uint32_t position,
                                float *hidden_out, float *layer_trace);
/* forward_single_token_position_zero (src/model/forward.rs:29-69): `token`
 * at position 0 with no cache (transformer_block_forward_position_zero,
 * src/model/block.rs:38-105: each head attends to this token's own K and V
 * as computed, f32, not through the int8 cache), then output_norm into
 * hidden_out (n_embd, host).  A non-finite hidden after a layer is
 * WM_E_NONFINITE (the reference's GgufParse). */
wm_status wm_forward_single_token_position_zero(wm_model *m, uint32_t token, float *hidden_out);
/* One greedy step: forward_with_cache + compute_logits + argmax
 * (src/model/generate.rs:165-187).  logits_out (vocab) and hidden_out may be
 * NULL. */
wm_status wm_decode_step(wm_model *m, wm_kv_cache *kv, uint32_t token, uint32_t position,
                         float *hidden_out, float *logits_out, uint32_t *next_token);
/* greedy_generate_with_cache (src/model/generate.rs:111-189) continuing an
 * existing cache: prefill `prompt` in order, then up to max_new greedy
 * tokens, stopping at `eos` (< 0: none).  Writes *n_out ids to out_ids.
 * Activations and the cache stay on the device; each step returns only its
 * 4-byte token id to the host, which feeds it to the next step. */
wm_status wm_greedy_generate(wm_model *m, wm_kv_cache *kv, const uint32_t *prompt,
                             uint32_t n_prompt, uint32_t max_new, int64_t eos, uint32_t *out_ids,
                             uint32_t *n_out);

/* Ragged multi-sequence step (continuous batching).  Sequence i appends
 * n_new[i] tokens (tokens[] holds them sequence after sequence) to its own
 * cache caches[i], starting at wm_kv_cache_position(caches[i]); each token
 * attends to its sequence's cache up to and including itself.  The result
 * is bit-identical to running wm_forward_with_cache on every token in order,
 * sequence by sequence: multi_token_forward (src/model/multi_forward.rs:49-243)
 * with a pre-filled cache, new K/V going through the int8 KV quantiser as in
 * the sequential prefill of src/model/generate.rs:151-160.
 *   last_hidden (n_seqs x n_embd, host, nullable): each sequence's last
 *     token after output_norm;
 *   next_tokens (n_seqs, host, nullable): argmax of that token's logits.
 * The caches must be distinct and belong to `m`; head_dim must be 64 or 128
 * and n_heads / n_kv_heads one of 1, 2, 4, 8.  A non-finite hidden in any
 * token leaves every cache at its starting position and returns
 * WM_E_NONFINITE. */
wm_status wm_batch_forward(wm_model *m, wm_kv_cache *const *caches, uint32_t n_seqs,
                           const uint32_t *n_new, const uint32_t *tokens, float *last_hidden,
                           uint32_t *next_tokens);

/* Batched prefill: `tokens` appended to `kv` at its current position through
 * the ragged-batch kernels (chunks of up to 512 tokens), bit-identical to
 * the token-by-token prefill of src/model/generate.rs:151-160.  On an
 * error the cache is left at its starting position.
 * last_hidden (n_embd, host, nullable): the last token after output_norm. */
wm_status wm_prefill(wm_model *m, wm_kv_cache *kv, const uint32_t *tokens, uint32_t n,
                     float *last_hidden);

/* ---- sampler (src/model/sampler.rs) ---------------------------------- */

/* SamplingParams (src/model/sampler.rs:40-79); the Option fields carry a
 * has_* flag. */
typedef struct wm_sampling_params {
    float temperature;                /* |t| < 1e-9 and no other knob: greedy */
    uint32_t has_top_k;
    uint64_t top_k;
    float top_p;
    uint32_t has_top_p;
    float repetition_penalty;
    uint32_t has_repetition_penalty;
} wm_sampling_params;
typedef struct wm_sampler wm_sampler;
/* Sampler::new (src/model/sampler.rs:94-101): xorshift64 seeded with `seed`
 * (0 -> 0xdeadbeefcafebabe, :18-25), empty history. */
wm_status wm_sampler_create(wm_ctx *ctx, const wm_sampling_params *params, uint64_t seed,
                            wm_sampler **out);
void wm_sampler_destroy(wm_sampler *s);
/* Sampler::observe (:105-107) */
wm_status wm_sampler_observe(wm_sampler *s, uint32_t id);
/* Sampler::checkpoint / rollback (:109-120) */
wm_status wm_sampler_checkpoint(const wm_sampler *s, uint64_t *rng_state, uint64_t *history_len);
wm_status wm_sampler_rollback(wm_sampler *s, uint64_t rng_state, uint64_t history_len);
/* Sampler::sample (:133-149): repetition penalty, temperature, top-k,
 * softmax, top-p and the multinomial draw (:178-196) on the device,
 * bit-identical to the reference (greedy: argmax, lm_head.rs:161-174).
 * Probabilities equal at the top-p cut are taken in index order (the
 * reference's unstable sort leaves it open), and NaN probabilities under
 * top-p with 0 < p < 1 are WM_E_NONFINITE (order unspecified there).  The
 * multinomial error (total not positive and finite) is WM_E_PARSE with the
 * reference's message; the xorshift state advances only when the draw runs.
 * _dev: logits on the device. */
wm_status wm_sampler_sample(wm_sampler *s, const float *logits, size_t n, uint32_t *out_id);
wm_status wm_sampler_sample_dev(wm_sampler *s, const float *d_logits, size_t n, uint32_t *out_id);
/* generate_with_cache_and_sampler (src/model/generate.rs:195-277) on an
 * existing cache: observe the prompt, prefill it (batched), then up to
 * max_new sampled tokens (logits and sampling on the device), stopping at
 * `eos` (< 0: none) or any of stop_ids; each accepted id is observed.  On
 * an error the cache goes back to its position at the call (the reference
 * drops its own cache with the error) and *n_out is 0; the sampler keeps
 * the ids it observed and its advanced rng, as the reference's caller-owned
 * sampler does. */
wm_status wm_generate_with_sampler(wm_model *m, wm_kv_cache *kv, const uint32_t *prompt,
                                   uint32_t n_prompt, uint32_t max_new, int64_t eos,
                                   const uint32_t *stop_ids, uint32_t n_stop, wm_sampler *s,
                                   uint32_t *out_ids, uint32_t *n_out);

/* ---- continuous batching --------------------------------------------- */

/* No single counterpart in the reference: a driver that runs many
 * generate_with_cache_and_sampler requests (src/model/generate.rs:195-277)
 * at once.  Each step packs every active request's next prompt chunk or
 * pending token into one ragged batch (wm_batch_forward); each request keeps
 * its own cache and sampler, so its ids equal wm_generate_with_sampler's on
 * its own (wm_greedy_generate's for greedy parameters).  At most max_seqs
 * requests are active (caches of max_seq_len positions, pooled); a step
 * feeds at most step_tokens tokens (max_seqs <= step_tokens <= 16384),
 * decoding requests first.  Single-threaded, like the context. */
typedef struct wm_server wm_server;
wm_status wm_server_create(wm_model *m, uint32_t max_seqs, uint32_t max_seq_len, uint32_t step_tokens,
                           wm_server **out);
void wm_server_destroy(wm_server *s);
/* Queue a request (prompt checks and budget as generate_with_cache_and_sampler,
 * generate.rs:209-226, against max_seq_len); *request_id identifies it. */
wm_status wm_server_submit(wm_server *s, const uint32_t *prompt, uint32_t n_prompt, uint32_t max_new,
                           int64_t eos, const uint32_t *stop_ids, uint32_t n_stop,
                           const wm_sampling_params *params, uint64_t seed, uint64_t *request_id);
/* One batch step; *n_active (nullable): requests still active or waiting. */
wm_status wm_server_step(wm_server *s, uint32_t *n_active);
/* The ids so far (up to cap copied, *n_out = all), whether the request has
 * finished, and its error status if it failed (a non-finite hidden, a
 * sampler error). */
wm_status wm_server_result(wm_server *s, uint64_t request_id, uint32_t *out_ids, uint32_t cap,
                           uint32_t *n_out, int *finished);
/* Forget a request (finished or not); its cache returns to the pool. */
wm_status wm_server_release(wm_server *s, uint64_t request_id);

/* ---- GGUF files (src/gguf/reader.rs, src/model/graph.rs) ------------- */

/* GgufFile::parse (src/gguf/reader.rs:120-415): the header, metadata and
 * tensor directory of a GGUF v2/v3 image with the reference's checks
 * (counts and array sizes against the bytes left, strings <= 1 MiB and
 * UTF-8, alignment a power of two, tensor byte lengths by type, every
 * tensor and I2_S trailing scale block inside the file and before the next
 * tensor).  Host-only: needs no device.  The result points into `data`,
 * which must outlive it.  On failure returns the error kind and writes the
 * reference's message into err (may be null). */
wm_status wm_gguf_parse(const uint8_t *data, size_t len, wm_gguf **out, char *err, size_t err_len);
/* ModelMmap::open (src/memory/mmap.rs:27-36) then GgufFile::parse: the
 * same over a read-only mapping of the file at path, owned by the result. */
wm_status wm_gguf_open(const char *path, wm_gguf **out, char *err, size_t err_len);
void wm_gguf_close(wm_gguf *g);
uint32_t wm_gguf_version(const wm_gguf *g);
uint64_t wm_gguf_alignment(const wm_gguf *g);
uint64_t wm_gguf_tensor_count(const wm_gguf *g);
/* Absolute offset of the tensor data section (reader.rs:244-256). */
uint64_t wm_gguf_data_offset(const wm_gguf *g);
/* Index of the tensor with this name, -1 if none. */
int64_t wm_gguf_find_tensor(const wm_gguf *g, const char *name);
/* TensorView (src/gguf/tensor.rs:21-54) of tensor `index`: name (owned by
 * g), raw GGML type id, dims, GGUF shape (unused dims 0), absolute offset,
 * byte length, data pointer, and for I2_S the 32-byte trailing scale block
 * (else null).  Any out pointer may be null. */
wm_status wm_gguf_tensor_info(const wm_gguf *g, uint64_t index, const char **name, uint32_t *type,
                              uint32_t *n_dims, uint64_t shape[4], uint64_t *offset, uint64_t *bytes,
                              const uint8_t **data, const uint8_t **scale_block);
/* GgufValue::as_u64 / as_f32 / as_str (src/gguf/reader.rs:48-76) of a
 * metadata key; WM_E_METADATA if absent or of another type. */
wm_status wm_gguf_meta_u64(const wm_gguf *g, const char *key, uint64_t *out);
wm_status wm_gguf_meta_f32(const wm_gguf *g, const char *key, float *out);
wm_status wm_gguf_meta_str(const wm_gguf *g, const char *key, const char **out);
/* ModelConfig::from_gguf_metadata (src/model/config.rs:61-160) for the
 * BitNet architectures "bitnet-b1.58", "bitnet-25", "bitnet"
 * (src/model/architecture/bitnet.rs:29-43); host-only. */
wm_status wm_gguf_bitnet_config(const wm_gguf *g, wm_model_config *cfg, char *err, size_t err_len);
/* ModelGraph::from_gguf's checks (src/model/graph.rs:79-237, :368-503)
 * without the upload, host-only: the config, unique names, no bias tensors,
 * every BitNet role present with its dtype and shape. */
wm_status wm_gguf_bitnet_check(const wm_gguf *g, char *err, size_t err_len);
/* ModelGraph::from_gguf (src/model/graph.rs:79-237) then the upload: every
 * tensor is found and checked (dtype, shape, no bias tensors, unique names)
 * before any device memory is taken; then the I2_S BitLinears with their
 * scale blocks, the f32 norms and the tied Q6_K token_embd go to the device
 * as by wm_model_create / wm_model_set_layer / wm_model_set_output.
 * max_context (0: the file's context_length) caps the KV caches the model
 * will serve.  token_embd in F16 (accepted by the reference) is
 * WM_E_UNSUPPORTED_TYPE here: the embedding and lm-head kernels read Q6_K. */
wm_status wm_model_from_gguf(wm_ctx *ctx, const wm_gguf *g, uint32_t max_context, wm_model **out);

/* ---- test hook ------------------------------------------------------- */

/* No counterpart in the reference: runs the device's exact evaluation of
 * the left-to-right f32 sum s = ((0 + a[0]) + a[1]) + ... of n non-negative
 * terms (host array), the routine behind every RMSNorm sum of squares and
 * softmax denominator, so tests can check it on adversarial inputs. */
wm_status wm_debug_seq_sum(wm_ctx *ctx, const float *values, size_t n, float *sum);

/* No counterpart in the reference: the id-only lm-head's bounded pass alone.
 * approx[v] is row v's fixed-point dot and bound[v] a bound on its distance
 * from the reference's f32 logit (the property the argmax proof rests on),
 * so tests can check |approx - logit| <= bound on every row. */
wm_status wm_debug_q6k_bounded_logits(wm_ctx *ctx, const wm_tensor *token_embd,
                                      const float *hidden, size_t hidden_len, float *approx,
                                      float *bound);
/* Device-pointer form, asynchronous, for timing the bounded pass (the kernel
 * the id-only lm-head spends its time in) alone: with reuse_prep != 0 the
 * fixed-point copy of the hidden vector made by the previous call on this
 * context (same tensor shape) is reused and only the pass itself runs. */
wm_status wm_debug_q6k_bounded_logits_dev(wm_ctx *ctx, const wm_tensor *token_embd,
                                          const float *d_hidden, float *d_approx, float *d_bound,
                                          int reuse_prep);

/* No counterpart in the reference: enqueue `reps` more launches of one
 * role of layer `layer` of the decode step just run (role 0 norm + Q/K/V,
 * 1 attention scores + softmax-V, 2 norm + O, 3 norm + gate/up, 4 norm +
 * down) at the cache's last position, on the context's stream, without
 * waiting, so that a caller can time that role's kernels back to back with
 * events.  The launches rewrite the same buffers and cache row the step
 * wrote; the results are not meant to be used. */
wm_status wm_debug_rerun_role(wm_model *m, wm_kv_cache *kv, uint32_t layer, uint32_t role,
                              uint32_t reps);

/* No counterpart in the reference: a test hook for the norm-fused matvecs
 * (every one launched on this context from now on).  They quantise
 * speculatively from an approximate rsqrt and max|y| while the exact sum of
 * squares runs, then correct the codes those could have changed; these bits
 * force the rarer paths, whose results must still be exact:
 *   WM_FUSED_DEBUG_SKEW_SMALL  the approximate max|y| off by 2^-12 (codes
 *                              near a rounding boundary corrected one by one),
 *   WM_FUSED_DEBUG_SKEW_LARGE  off by 2^-7 (too many: codes redone),
 *   WM_FUSED_DEBUG_NO_CANDIDATES  max|y| from every wave's own maximum
 *                              (the candidate lists treated as failed),
 *   WM_FUSED_DEBUG_ATTN_NO_WAIT, WM_FUSED_DEBUG_ATTN_LOOSE_COUNT   (below).
 * 0 restores the normal behaviour. */
#define WM_FUSED_DEBUG_SKEW_SMALL 1u
#define WM_FUSED_DEBUG_SKEW_LARGE 2u
#define WM_FUSED_DEBUG_NO_CANDIDATES 4u
/* Decode attention (one launch per layer) lets the workgroups that share a
 * kv head wait for each other's scores; with this bit every such wait gives
 * up at once, which must fail the step with WM_E_HIP and roll the cache
 * back (never hang). */
#define WM_FUSED_DEBUG_ATTN_NO_WAIT 8u
/* The greedy loop's steps read their position from the device, and each
 * attention launch is sized for the count the host expects, with which its
 * first loads go out before the device word arrives.  With this bit the
 * launches are sized for up to 9 more positions than the step has: the
 * kernel then starts its scores again with the device's count, and the ids
 * must be the same. */
#define WM_FUSED_DEBUG_ATTN_LOOSE_COUNT 16u
wm_status wm_debug_set_fused_flags(wm_ctx *ctx, uint32_t flags);

/* ---- synthetic BitNet-shaped inputs (src/synth.rs) ------------------- */

/* Counter-based SplitMix64 streams, identical on every host: value i of
 * stream (seed, tag) is the (i+1)-th SplitMix64 output from state
 * wm_synth_stream_seed(seed, tag). */
uint64_t wm_synth_stream_seed(uint64_t seed, uint64_t tag);
/* Ternary I2_S codes, each of {-1,0,+1} with probability 1/3, packed
 * c0<<6 | c1<<4 | c2<<2 | c3 (src/synth.rs:239-265). */
void wm_synth_i2s(uint64_t seed, uint64_t tag, uint8_t *packed, size_t n_bytes);
/* f32 ~ N(0, sigma) (Box-Muller in double) and ~ U(lo, hi). */
void wm_synth_normal(uint64_t seed, uint64_t tag, float *out, size_t n, double sigma);
void wm_synth_uniform(uint64_t seed, uint64_t tag, float *out, size_t n, double lo, double hi);
/* Q6_K rows: ql/qh uniform bytes, sub-scales uniform in [-32, 31],
 * d = f16(|N(0, d_sigma)|). */
void wm_synth_q6k(uint64_t seed, uint64_t tag, uint8_t *blocks, size_t n_blocks, double d_sigma);

#ifdef __cplusplus
}
#endif
#endif /* WILLAMETTE_HIP_H */
