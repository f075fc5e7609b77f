//! Raw declarations of include/willamette_hip.h (one `extern "C"` item per
//! entry point, same order).  tests/test_rust_binding.py checks that this
//! block declares exactly the header's functions with matching parameter
//! and return types.
#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_int, c_void};

pub type wm_status = c_int;

pub const WM_OK: wm_status = 0;
pub const WM_E_UNSUPPORTED_TYPE: wm_status = 1;
pub const WM_E_SHAPE: wm_status = 2;
pub const WM_E_NONFINITE: wm_status = 3;
pub const WM_E_OOM: wm_status = 4;
pub const WM_E_HIP: wm_status = 5;
pub const WM_E_ARG: wm_status = 6;
pub const WM_E_STATE: wm_status = 7;
pub const WM_E_PARSE: wm_status = 8;
pub const WM_E_MAGIC: wm_status = 9;
pub const WM_E_VERSION: wm_status = 10;
pub const WM_E_ARCH: wm_status = 11;
pub const WM_E_METADATA: wm_status = 12;
pub const WM_E_BOUNDS: wm_status = 13;
pub const WM_E_IO: wm_status = 14;
pub const WM_E_NOT_IMPLEMENTED: wm_status = 15;
pub const WM_FUSED_DEBUG_SKEW_SMALL: u32 = 1;
pub const WM_FUSED_DEBUG_SKEW_LARGE: u32 = 2;
pub const WM_FUSED_DEBUG_NO_CANDIDATES: u32 = 4;
pub const WM_FUSED_DEBUG_ATTN_NO_WAIT: u32 = 8;
pub const WM_FUSED_DEBUG_ATTN_LOOSE_COUNT: u32 = 16;

pub const WM_TYPE_I2S: c_int = 36;
pub const WM_TYPE_Q6K: c_int = 14;

#[repr(C)]
pub struct wm_ctx {
    _p: [u8; 0],
}
#[repr(C)]
pub struct wm_tensor {
    _p: [u8; 0],
}
#[repr(C)]
pub struct wm_model {
    _p: [u8; 0],
}
#[repr(C)]
pub struct wm_kv_cache {
    _p: [u8; 0],
}
#[repr(C)]
pub struct wm_gguf {
    _p: [u8; 0],
}
#[repr(C)]
pub struct wm_sampler {
    _p: [u8; 0],
}
#[repr(C)]
pub struct wm_server {
    _p: [u8; 0],
}

/// ModelConfig's fields (src/model/config.rs), as the C struct lays them out.
#[repr(C)]
#[derive(Debug, Clone, Copy, Default, PartialEq)]
pub struct wm_model_config {
    pub n_layers: u32,
    pub n_embd: u32,
    pub n_ff: u32,
    pub n_heads: u32,
    pub n_kv_heads: u32,
    pub head_dim: u32,
    pub n_rot: u32,
    pub vocab_size: u32,
    pub context_length: u32,
    pub rms_eps: f32,
    pub rope_freq_base: f32,
}

/// SamplingParams (src/model/sampler.rs:40-79) with each Option as a flag.
#[repr(C)]
#[derive(Debug, Clone, Copy, Default, PartialEq)]
pub struct wm_sampling_params {
    pub temperature: f32,
    pub has_top_k: u32,
    pub top_k: u64,
    pub top_p: f32,
    pub has_top_p: u32,
    pub repetition_penalty: f32,
    pub has_repetition_penalty: u32,
}

extern "C" {
    pub fn wm_ctx_create(device: c_int, out: *mut *mut wm_ctx) -> wm_status;
    pub fn wm_ctx_destroy(ctx: *mut wm_ctx);
    pub fn wm_last_error(ctx: *const wm_ctx) -> *const c_char;
    pub fn wm_ctx_stream(ctx: *mut wm_ctx) -> *mut c_void;
    pub fn wm_ctx_synchronize(ctx: *mut wm_ctx) -> wm_status;
    pub fn wm_version() -> *const c_char;
    pub fn wm_dev_alloc(ctx: *mut wm_ctx, bytes: usize, out: *mut *mut c_void) -> wm_status;
    pub fn wm_dev_free(ctx: *mut wm_ctx, ptr: *mut c_void) -> wm_status;
    pub fn wm_memcpy_h2d(ctx: *mut wm_ctx, dst: *mut c_void, src: *const c_void, bytes: usize) -> wm_status;
    pub fn wm_memcpy_d2h(ctx: *mut wm_ctx, dst: *mut c_void, src: *const c_void, bytes: usize) -> wm_status;
    pub fn wm_tensor_upload_i2s(ctx: *mut wm_ctx, packed: *const u8, packed_len: usize, scale_block: *const u8, scale_len: usize, in_dim: u64, out_dim: u64, out: *mut *mut wm_tensor) -> wm_status;
    pub fn wm_tensor_upload_q6k(ctx: *mut wm_ctx, blocks: *const u8, len: usize, row_len: u64, n_rows: u64, out: *mut *mut wm_tensor) -> wm_status;
    pub fn wm_tensor_destroy(t: *mut wm_tensor);
    pub fn wm_tensor_info(t: *const wm_tensor, shape: *mut u64, type_: *mut c_int, scale: *mut f32) -> wm_status;
    pub fn wm_bitlinear_i2s_matvec_f32(ctx: *mut wm_ctx, w: *const wm_tensor, input: *const f32, input_len: usize, output: *mut f32, output_len: usize) -> wm_status;
    pub fn wm_bitlinear_i2s_matvec_f32_debug(ctx: *mut wm_ctx, w: *const wm_tensor, input: *const f32, input_len: usize, output: *mut f32, output_len: usize, act: *mut i8, act_scale: *mut f32, acc: *mut i32) -> wm_status;
    pub fn wm_bitlinear_i2s_matvec_f32_scalar(ctx: *mut wm_ctx, w: *const wm_tensor, input: *const f32, input_len: usize, output: *mut f32, output_len: usize) -> wm_status;
    pub fn wm_bitlinear_i2s_matvec_f32_scalar_dev(ctx: *mut wm_ctx, w: *const wm_tensor, d_input: *const f32, d_output: *mut f32) -> wm_status;
    pub fn wm_bitlinear_i2s_matvec_f32_dev(ctx: *mut wm_ctx, w: *const wm_tensor, d_input: *const f32, d_output: *mut f32) -> wm_status;
    pub fn wm_bitlinear_i2s_matvec_f32_multi_dev(ctx: *mut wm_ctx, ws: *const *const wm_tensor, n_copies: u32, d_input: *const f32, d_outputs: *mut f32) -> wm_status;
    pub fn wm_bitlinear_i2s_matvec_f32_dev_noalloc(ctx: *mut wm_ctx, w: *const wm_tensor, d_input: *const f32, d_output: *mut f32) -> wm_status;
    pub fn wm_bitlinear_i2s_matmul_f32_dev(ctx: *mut wm_ctx, w: *const wm_tensor, d_x: *const f32, m: u32, d_y: *mut f32) -> wm_status;
    pub fn wm_bitlinear_i2s_matmul_f32(ctx: *mut wm_ctx, w: *const wm_tensor, x: *const f32, x_len: usize, m: u32, y: *mut f32, y_len: usize) -> wm_status;
    pub fn wm_ffn_block_forward(ctx: *mut wm_ctx, x: *const f32, x_len: usize, ffn_norm_weight: *const f32, ffn_norm_len: usize, gate: *const wm_tensor, up: *const wm_tensor, down: *const wm_tensor, ffn_sub_norm_weight: *const f32, ffn_sub_norm_len: usize, eps: f32, output: *mut f32, output_len: usize) -> wm_status;
    pub fn wm_ffn_block_forward_dev(ctx: *mut wm_ctx, d_x: *const f32, d_ffn_norm_weight: *const f32, gate: *const wm_tensor, up: *const wm_tensor, down: *const wm_tensor, d_ffn_sub_norm_weight: *const f32, eps: f32, d_output: *mut f32) -> wm_status;
    pub fn wm_q6k_dequantize_row(ctx: *mut wm_ctx, t: *const wm_tensor, row: u64, out: *mut f32, out_len: usize) -> wm_status;
    pub fn wm_compute_logits(ctx: *mut wm_ctx, token_embd: *const wm_tensor, hidden: *const f32, hidden_len: usize, logits: *mut f32, vocab: usize) -> wm_status;
    pub fn wm_logits_argmax(ctx: *mut wm_ctx, token_embd: *const wm_tensor, hidden: *const f32, hidden_len: usize, logits: *mut f32, argmax: *mut u32) -> wm_status;
    pub fn wm_logits_argmax_dev(ctx: *mut wm_ctx, token_embd: *const wm_tensor, d_hidden: *const f32, d_logits: *mut f32, d_argmax: *mut u32) -> wm_status;
    pub fn wm_argmax(logits: *const f32, n: usize, out: *mut u32) -> wm_status;
    pub fn wm_model_create(ctx: *mut wm_ctx, cfg: *const wm_model_config, out: *mut *mut wm_model) -> wm_status;
    pub fn wm_model_destroy(m: *mut wm_model);
    pub fn wm_model_set_layer(m: *mut wm_model, layer: u32, attn_q: *const wm_tensor, attn_k: *const wm_tensor, attn_v: *const wm_tensor, attn_output: *const wm_tensor, ffn_gate: *const wm_tensor, ffn_up: *const wm_tensor, ffn_down: *const wm_tensor, attn_norm: *const f32, attn_sub_norm: *const f32, ffn_norm: *const f32, ffn_sub_norm: *const f32) -> wm_status;
    pub fn wm_model_set_output(m: *mut wm_model, token_embd: *const wm_tensor, output_norm: *const f32) -> wm_status;
    pub fn wm_kv_cache_create(m: *mut wm_model, max_seq_len: u32, out: *mut *mut wm_kv_cache) -> wm_status;
    pub fn wm_kv_cache_destroy(kv: *mut wm_kv_cache);
    pub fn wm_kv_cache_position(kv: *const wm_kv_cache) -> u32;
    pub fn wm_kv_cache_rollback(kv: *mut wm_kv_cache, position: u32) -> wm_status;
    pub fn wm_kv_cache_append_position(kv: *mut wm_kv_cache, k: *const f32, v: *const f32) -> wm_status;
    pub fn wm_kv_cache_append_positions(kv: *mut wm_kv_cache, k: *const f32, v: *const f32, n_pos: u32) -> wm_status;
    pub fn wm_kv_cache_read_raw(kv: *mut wm_kv_cache, layer: u32, k: *mut i8, k_scales: *mut f32, v: *mut i8, v_scales: *mut f32, n_pos: u32) -> wm_status;
    pub fn wm_kv_cache_read_into(kv: *mut wm_kv_cache, layer: u32, out_k: *mut f32, out_v: *mut f32) -> wm_status;
    pub fn wm_forward_with_cache(m: *mut wm_model, kv: *mut wm_kv_cache, token: u32, position: u32, hidden_out: *mut f32, layer_trace: *mut f32) -> wm_status;
    pub fn wm_forward_single_token_position_zero(m: *mut wm_model, token: u32, hidden_out: *mut f32) -> wm_status;
    pub fn wm_decode_step(m: *mut wm_model, kv: *mut wm_kv_cache, token: u32, position: u32, hidden_out: *mut f32, logits_out: *mut f32, next_token: *mut u32) -> wm_status;
    pub fn wm_greedy_generate(m: *mut wm_model, kv: *mut wm_kv_cache, prompt: *const u32, n_prompt: u32, max_new: u32, eos: i64, out_ids: *mut u32, n_out: *mut u32) -> wm_status;
    pub fn wm_batch_forward(m: *mut wm_model, caches: *const *mut wm_kv_cache, n_seqs: u32, n_new: *const u32, tokens: *const u32, last_hidden: *mut f32, next_tokens: *mut u32) -> wm_status;
    pub fn wm_prefill(m: *mut wm_model, kv: *mut wm_kv_cache, tokens: *const u32, n: u32, last_hidden: *mut f32) -> wm_status;
    pub fn wm_sampler_create(ctx: *mut wm_ctx, params: *const wm_sampling_params, seed: u64, out: *mut *mut wm_sampler) -> wm_status;
    pub fn wm_sampler_destroy(s: *mut wm_sampler);
    pub fn wm_sampler_observe(s: *mut wm_sampler, id: u32) -> wm_status;
    pub fn wm_sampler_checkpoint(s: *const wm_sampler, rng_state: *mut u64, history_len: *mut u64) -> wm_status;
    pub fn wm_sampler_rollback(s: *mut wm_sampler, rng_state: u64, history_len: u64) -> wm_status;
    pub fn wm_sampler_sample(s: *mut wm_sampler, logits: *const f32, n: usize, out_id: *mut u32) -> wm_status;
    pub fn wm_sampler_sample_dev(s: *mut wm_sampler, d_logits: *const f32, n: usize, out_id: *mut u32) -> wm_status;
    pub fn wm_generate_with_sampler(m: *mut wm_model, kv: *mut wm_kv_cache, prompt: *const u32, n_prompt: u32, max_new: u32, eos: i64, stop_ids: *const u32, n_stop: u32, s: *mut wm_sampler, out_ids: *mut u32, n_out: *mut u32) -> wm_status;
    pub fn wm_server_create(m: *mut wm_model, max_seqs: u32, max_seq_len: u32, step_tokens: u32, out: *mut *mut wm_server) -> wm_status;
    pub fn wm_server_destroy(s: *mut wm_server);
    pub fn wm_server_submit(s: *mut wm_server, prompt: *const u32, n_prompt: u32, max_new: u32, eos: i64, stop_ids: *const u32, n_stop: u32, params: *const wm_sampling_params, seed: u64, request_id: *mut u64) -> wm_status;
    pub fn wm_server_step(s: *mut wm_server, n_active: *mut u32) -> wm_status;
    pub fn wm_server_result(s: *mut wm_server, request_id: u64, out_ids: *mut u32, cap: u32, n_out: *mut u32, finished: *mut c_int) -> wm_status;
    pub fn wm_server_release(s: *mut wm_server, request_id: u64) -> wm_status;
    pub fn wm_gguf_parse(data: *const u8, len: usize, out: *mut *mut wm_gguf, err: *mut c_char, err_len: usize) -> wm_status;
    pub fn wm_gguf_open(path: *const c_char, out: *mut *mut wm_gguf, err: *mut c_char, err_len: usize) -> wm_status;
    pub fn wm_gguf_close(g: *mut wm_gguf);
    pub fn wm_gguf_version(g: *const wm_gguf) -> u32;
    pub fn wm_gguf_alignment(g: *const wm_gguf) -> u64;
    pub fn wm_gguf_tensor_count(g: *const wm_gguf) -> u64;
    pub fn wm_gguf_data_offset(g: *const wm_gguf) -> u64;
    pub fn wm_gguf_find_tensor(g: *const wm_gguf, name: *const c_char) -> i64;
    pub fn wm_gguf_tensor_info(g: *const wm_gguf, index: u64, name: *mut *const c_char, type_: *mut u32, n_dims: *mut u32, shape: *mut u64, offset: *mut u64, bytes: *mut u64, data: *mut *const u8, scale_block: *mut *const u8) -> wm_status;
    pub fn wm_gguf_meta_u64(g: *const wm_gguf, key: *const c_char, out: *mut u64) -> wm_status;
    pub fn wm_gguf_meta_f32(g: *const wm_gguf, key: *const c_char, out: *mut f32) -> wm_status;
    pub fn wm_gguf_meta_str(g: *const wm_gguf, key: *const c_char, out: *mut *const c_char) -> wm_status;
    pub fn wm_gguf_bitnet_config(g: *const wm_gguf, cfg: *mut wm_model_config, err: *mut c_char, err_len: usize) -> wm_status;
    pub fn wm_gguf_bitnet_check(g: *const wm_gguf, err: *mut c_char, err_len: usize) -> wm_status;
    pub fn wm_model_from_gguf(ctx: *mut wm_ctx, g: *const wm_gguf, max_context: u32, out: *mut *mut wm_model) -> wm_status;
    pub fn wm_debug_seq_sum(ctx: *mut wm_ctx, values: *const f32, n: usize, sum: *mut f32) -> wm_status;
    pub fn wm_debug_q6k_bounded_logits(ctx: *mut wm_ctx, token_embd: *const wm_tensor, hidden: *const f32, hidden_len: usize, approx: *mut f32, bound: *mut f32) -> wm_status;
    pub fn wm_debug_q6k_bounded_logits_dev(ctx: *mut wm_ctx, token_embd: *const wm_tensor, d_hidden: *const f32, d_approx: *mut f32, d_bound: *mut f32, reuse_prep: c_int) -> wm_status;
    pub fn wm_debug_rerun_role(m: *mut wm_model, kv: *mut wm_kv_cache, layer: u32, role: u32, reps: u32) -> wm_status;
    pub fn wm_debug_set_fused_flags(ctx: *mut wm_ctx, flags: u32) -> wm_status;
    pub fn wm_synth_stream_seed(seed: u64, tag: u64) -> u64;
    pub fn wm_synth_i2s(seed: u64, tag: u64, packed: *mut u8, n_bytes: usize);
    pub fn wm_synth_normal(seed: u64, tag: u64, out: *mut f32, n: usize, sigma: f64);
    pub fn wm_synth_uniform(seed: u64, tag: u64, out: *mut f32, n: usize, lo: f64, hi: f64);
    pub fn wm_synth_q6k(seed: u64, tag: u64, blocks: *mut u8, n_blocks: usize, d_sigma: f64);
}
