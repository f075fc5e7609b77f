/*
 * TEST INFRASTRUCTURE ONLY — the parity oracle.
 *
 * A CPU restatement, in plain C, of project-willamette's BitNet b1.58 decode
 * path as its x86_64 build runs it (SSE2-i8 BitLinear, SSE2 Q6_K row-dot,
 * sequential f32 reductions, glibc libm).  Only tests/, the smoke() check in
 * __graft_entry__.py and bench.py's cpu_baseline leg may load this library,
 * and only as the checker / the timed CPU baseline.  The product library
 * (libwillamette_hip.so) never links, loads or calls it.
 *
 * Every function names the reference file:line whose behaviour it restates.
 */
#ifndef WM_ORACLE_H
#define WM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar helpers ---------------------------------------------------- */
float or_f16_to_f32(uint16_t bits);          /* src/model/primitives.rs:61-88 */
int8_t or_ternary_from_code(uint8_t code);   /* src/model/bitlinear.rs:43-50 */
float or_expf(float x);                      /* the libm expf the reference's f32::exp calls */

/* ---- BitLinear I2_S ---------------------------------------------------- */
/* src/model/bitlinear_sse2.rs:285-304 — returns the activation scale. */
float or_quantize_input_absmax_i8(const float *x, size_t n, int8_t *out);
/* src/model/bitlinear.rs:247-299 */
int or_i2s_unpack_row(const uint8_t *packed, size_t in_dim, size_t out_dim,
                      size_t row, int8_t *out);
/* src/model/bitlinear_sse2.rs:313-342 (+ validate_inputs :129-177).
 * dbg_* are nullable taps: quantised activation, its scale, and the i32
 * per-row dot before the f32 epilogue. Returns 0 or a negative error. */
int or_bitlinear_i2s_matvec_f32_sse2_i8(const uint8_t *packed, size_t packed_len,
                                        float w_scale, size_t in_dim, size_t out_dim,
                                        const float *x, float *y, int8_t *dbg_act,
                                        float *dbg_act_scale, int32_t *dbg_acc);
/* src/model/bitlinear.rs:146-233 (two-accumulator f32 form). */
int or_bitlinear_i2s_matvec_f32_scalar(const uint8_t *packed, size_t packed_len,
                                       float w_scale, size_t in_dim, size_t out_dim,
                                       const float *x, float *y);
/* src/gguf/tensor.rs:278-309 — reads the LE f32 in the 32-byte trailing block. */
int or_i2s_scale(const uint8_t *scale_block, size_t len, float *out);

/* ---- Q6_K -------------------------------------------------------------- */
/* src/model/q6_k.rs:25-69 */
int or_q6k_dequantize_row(const uint8_t *row, size_t row_len, float *out, size_t n);
/* src/model/q6_k_sse2.rs:46-116 (4 accumulators x 4 lanes, fixed hsum). */
float or_q6k_dot_row_sse2(const uint8_t *row, const float *x, size_t n);
/* src/model/q6_k.rs:84-96 */
float or_q6k_dot_row_scalar(const uint8_t *row, const float *x, size_t n);
/* src/model/lm_head.rs:29-108, rows split over `threads` workers like rayon. */
int or_compute_logits_q6k(const uint8_t *embd, size_t n_embd, size_t vocab,
                          const float *hidden, float *logits, int threads);
/* src/model/lm_head.rs:161-174; returns -1 for an empty slice. */
int64_t or_argmax(const float *logits, size_t n);

/* ---- f32 primitives ---------------------------------------------------- */
/* src/model/primitives.rs:227-255 */
void or_rms_norm(const float *x, const float *w, size_t n, float eps, float *out);
/* src/model/primitives.rs:285-345 (NEOX pairing, j with j + n_rot/2). */
void or_rope_neox(float *x, size_t head_dim, size_t n_rot, uint32_t pos, float freq_base);
/* src/model/attention.rs:45-73 */
void or_softmax_inplace(float *x, size_t n);
/* src/model/ffn.rs:37-65: out = relu(gate)^2 * up */
void or_relu_square_mul(const float *gate, const float *up, size_t n, float *out);
/* src/model/ffn.rs:73-136: ffn_norm, gate/up (I2_S packed, in_dim n_embd,
 * out_dim n_ff), relu^2 * up, ffn_sub_norm, down (in n_ff, out n_embd) */
int or_ffn_block_forward(const float *x, size_t n_embd, size_t n_ff, const float *ffn_norm_w,
                         const uint8_t *gate, float gate_scale, const uint8_t *up, float up_scale,
                         const uint8_t *down, float down_scale, const float *ffn_sub_norm_w,
                         float eps, float *out);
/* src/model/kv_cache.rs:245-259: q + scale for one token; returns the scale */
float or_kv_quantise(const float *x, size_t n, int8_t *q);
/* src/model/cached_forward.rs:417-449: q[n_heads*head_dim] attends to n_past
 * f32 K/V rows of n_kv_heads*head_dim values; out[n_heads*head_dim];
 * scores: n_past floats of scratch. */
void or_sdpa(const float *q, const float *kd, const float *vd, uint32_t n_past, uint32_t n_heads,
             uint32_t n_kv_heads, uint32_t head_dim, float *out, float *scores);

/* ---- model-level ------------------------------------------------------- */
typedef struct or_model or_model;
typedef struct or_kv or_kv;

or_model *or_model_create(uint32_t n_layers, uint32_t n_embd, uint32_t n_ff,
                          uint32_t n_heads, uint32_t n_kv_heads, uint32_t head_dim,
                          uint32_t vocab, float eps, float rope_base);
void or_model_destroy(or_model *m);
/* Borrowed pointers (the caller keeps the buffers alive), like TensorView. */
int or_model_set_layer(or_model *m, uint32_t layer,
                       const uint8_t *q, float q_scale, const uint8_t *k, float k_scale,
                       const uint8_t *v, float v_scale, const uint8_t *o, float o_scale,
                       const uint8_t *gate, float gate_scale, const uint8_t *up,
                       float up_scale, const uint8_t *down, float down_scale,
                       const float *attn_norm, const float *attn_sub_norm,
                       const float *ffn_norm, const float *ffn_sub_norm);
int or_model_set_output(or_model *m, const uint8_t *token_embd_q6k, const float *output_norm);
/* Number of worker threads for the lm-head row loop (default 1). */
void or_model_set_threads(or_model *m, int threads);

or_kv *or_kv_create(uint32_t n_layers, uint32_t kv_dim, uint32_t max_seq);
void or_kv_destroy(or_kv *kv);
uint32_t or_kv_position(const or_kv *kv);
void or_kv_rollback(or_kv *kv, uint32_t position);
/* src/model/kv_cache.rs:154-185 for every layer at the next position;
 * k and v are n_layers x kv_dim (layer-major). */
int or_kv_append_position(or_kv *kv, const float *k, const float *v);
/* Raw views for tests: i8 codes and scales of one layer. */
int or_kv_read_raw(const or_kv *kv, uint32_t layer, int8_t *k, float *ks, int8_t *v,
                   float *vs, uint32_t n_pos);

/* src/model/cached_forward.rs:164-261 (embedding, 30 x forward_one_layer,
 * output_norm).  layer_trace (nullable) receives the hidden state after each
 * layer, n_layers x n_embd.  Returns 0, or a negative error after rolling the
 * cache back (cached_forward.rs:256-259). */
int or_forward_with_cache(or_model *m, or_kv *kv, uint32_t token, uint32_t pos,
                          float *out_hidden, float *layer_trace);
/* src/model/lm_head.rs:112-122 + argmax. */
/* forward_single_token_position_zero (src/model/forward.rs:29-69): no
 * cache, attention over the one position with f32 K/V; -3 on a non-finite
 * hidden after a layer. */
int or_forward_single_token_position_zero(or_model *m, uint32_t token, float *out_hidden,
                                          float *layer_trace);
int or_logits_argmax(or_model *m, const float *hidden, float *logits, uint32_t *next);
/* src/model/generate.rs:111-189 on an existing cache (prefill of `prompt`,
 * then greedy steps).  logits_trace (nullable) gets max_new x vocab. */
int or_greedy_generate(or_model *m, or_kv *kv, const uint32_t *prompt, uint32_t n_prompt,
                       uint32_t max_new, int64_t eos, uint32_t *out_ids, uint32_t *n_out,
                       float *logits_trace);

/* ---- sampler (src/model/sampler.rs) ------------------------------------ */
/* XorShift64 (sampler.rs:13-38): the state a seed gives (0 -> 0xdeadbeefcafebabe),
 * the next value (state updated) and the unit draw from its high 24 bits. */
uint64_t or_xorshift64_seed(uint64_t seed);
uint64_t or_xorshift64_next(uint64_t *state);
float or_xorshift64_next_unit(uint64_t *state);
/* SamplingParams (sampler.rs:40-79); the Option fields as has_* flags. */
typedef struct or_sampling_params {
    float temperature;
    uint32_t has_top_k;
    uint64_t top_k;
    float top_p;
    uint32_t has_top_p;
    float repetition_penalty;
    uint32_t has_repetition_penalty;
} or_sampling_params;
int or_sampling_is_greedy(const or_sampling_params *p);                  /* :71-78 */
void or_apply_repetition_penalty(float *logits, size_t n, const uint32_t *history,
                                 size_t n_history, float r);             /* :151-164 */
void or_apply_temperature(float *logits, size_t n, float t);              /* :166-176 */
void or_apply_top_k(float *logits, size_t n, uint64_t k);                 /* :201-223 */
void or_softmax_to_probs(const float *logits, size_t n, float *out);      /* :225-252 */
/* :254-311; entries of equal probability are taken in index order (the
 * reference's unstable sort leaves their order open). */
void or_apply_top_p(float *probs, size_t n, float p);
/* Sampler::sample (:133-149) with multinomial (:178-196).  Returns 0 and
 * *out; -1 empty logits; -2 the multinomial error (probabilities not
 * summing to a positive finite value, *total_out set); -3 NaN
 * probabilities under top-p with 0 < p < 1 (where the reference's sort
 * order is unspecified).  *state advances only when the draw runs. */
int or_sample(const or_sampling_params *p, uint64_t *state, const uint32_t *history,
              size_t n_history, const float *logits, size_t n, uint32_t *out, float *total_out);

#ifdef __cplusplus
}
#endif
#endif
