//! Safe Rust wrappers over libwillamette_hip.so, the MI355X (gfx950) BitNet
//! b1.58 decode path.  The raw C ABI is in [`sys`]; the types here own their
//! handles (destroyed on drop) and turn status codes into [`Error`].
//!
//! Thread safety follows the C library: a [`Context`] and everything made on
//! it are used from one thread at a time (the reference's decode is
//! single-threaded per request, src/model/stage_timing.rs:32-36), so none of
//! the types is `Sync`; wrap a context in a `Mutex` to share it.

pub mod sys;

use std::ffi::{CStr, CString};
use std::marker::PhantomData;
use std::os::raw::c_char;
use std::path::Path;
use std::ptr;

/// The library's status codes, named after the WillametteError kinds they
/// map to (src/error.rs:9-57).
#[derive(Debug, Clone, Copy, PartialEq, Eq)]
pub enum Status {
    UnsupportedTensorType,
    Shape,
    NonFinite,
    OutOfMemory,
    Hip,
    Arg,
    State,
    GgufParse,
    InvalidMagic,
    UnsupportedVersion,
    UnsupportedArchitecture,
    MissingMetadata,
    TensorOutOfBounds,
    Io,
    NotImplemented,
    Other(i32),
}

impl Status {
    fn from_code(c: sys::wm_status) -> Status {
        match c {
            sys::WM_E_UNSUPPORTED_TYPE => Status::UnsupportedTensorType,
            sys::WM_E_SHAPE => Status::Shape,
            sys::WM_E_NONFINITE => Status::NonFinite,
            sys::WM_E_OOM => Status::OutOfMemory,
            sys::WM_E_HIP => Status::Hip,
            sys::WM_E_ARG => Status::Arg,
            sys::WM_E_STATE => Status::State,
            sys::WM_E_PARSE => Status::GgufParse,
            sys::WM_E_MAGIC => Status::InvalidMagic,
            sys::WM_E_VERSION => Status::UnsupportedVersion,
            sys::WM_E_ARCH => Status::UnsupportedArchitecture,
            sys::WM_E_METADATA => Status::MissingMetadata,
            sys::WM_E_BOUNDS => Status::TensorOutOfBounds,
            sys::WM_E_IO => Status::Io,
            sys::WM_E_NOT_IMPLEMENTED => Status::NotImplemented,
            other => Status::Other(other),
        }
    }
}

/// A failed call: its status and the library's message.
#[derive(Debug, Clone, PartialEq, Eq)]
pub struct Error {
    pub status: Status,
    pub message: String,
}

impl std::fmt::Display for Error {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        write!(f, "{:?}: {}", self.status, self.message)
    }
}

impl std::error::Error for Error {}

pub type Result<T> = std::result::Result<T, Error>;

fn err_text(buf: &[c_char]) -> String {
    unsafe { CStr::from_ptr(buf.as_ptr()) }.to_string_lossy().into_owned()
}

/// Library version string (names the target, gfx950).
pub fn version() -> String {
    unsafe { CStr::from_ptr(sys::wm_version()) }.to_string_lossy().into_owned()
}

/// argmax with the reference's rules (src/model/lm_head.rs:161-174): the
/// first of equal maxima; a NaN at index 0 wins.  None for an empty slice.
pub fn argmax(logits: &[f32]) -> Option<u32> {
    let mut out = 0u32;
    let st = unsafe { sys::wm_argmax(logits.as_ptr(), logits.len(), &mut out) };
    (st == sys::WM_OK).then_some(out)
}

// ---------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------

/// One device and one HIP stream (src/model/dispatch.rs:111-114's process-wide
/// choice, for a `Kernel::Hip` arm).
pub struct Context {
    h: *mut sys::wm_ctx,
}

impl Context {
    pub fn new(device: i32) -> Result<Context> {
        let mut h = ptr::null_mut();
        let st = unsafe { sys::wm_ctx_create(device, &mut h) };
        if st != sys::WM_OK {
            return Err(Error {
                status: Status::from_code(st),
                message: format!("wm_ctx_create(device={device}) failed"),
            });
        }
        Ok(Context { h })
    }

    pub fn raw(&self) -> *mut sys::wm_ctx {
        self.h
    }

    fn check(&self, st: sys::wm_status) -> Result<()> {
        if st == sys::WM_OK {
            return Ok(());
        }
        let message = unsafe { CStr::from_ptr(sys::wm_last_error(self.h)) }
            .to_string_lossy()
            .into_owned();
        Err(Error { status: Status::from_code(st), message })
    }

    pub fn synchronize(&self) -> Result<()> {
        self.check(unsafe { sys::wm_ctx_synchronize(self.h) })
    }

    /// Upload an I2_S weight: `packed` is TensorView::data and `scale_block`
    /// its 32-byte trailing block (src/gguf/tensor.rs:278-309); GGUF shape
    /// [in_dim, out_dim].
    pub fn upload_i2s(&self, packed: &[u8], scale_block: &[u8], in_dim: u64, out_dim: u64) -> Result<Tensor<'_>> {
        let mut t = ptr::null_mut();
        self.check(unsafe {
            sys::wm_tensor_upload_i2s(self.h, packed.as_ptr(), packed.len(), scale_block.as_ptr(),
                                      scale_block.len(), in_dim, out_dim, &mut t)
        })?;
        Ok(Tensor { h: t, ctx: self })
    }

    /// Upload a Q6_K matrix of n_rows rows of row_len values.
    pub fn upload_q6k(&self, blocks: &[u8], row_len: u64, n_rows: u64) -> Result<Tensor<'_>> {
        let mut t = ptr::null_mut();
        self.check(unsafe {
            sys::wm_tensor_upload_q6k(self.h, blocks.as_ptr(), blocks.len(), row_len, n_rows, &mut t)
        })?;
        Ok(Tensor { h: t, ctx: self })
    }

    /// bitlinear_i2s_matvec_f32 (src/model/bitlinear.rs:67): the x86 SSE2-i8
    /// result, bit for bit.
    pub fn bitlinear_i2s_matvec_f32(&self, w: &Tensor<'_>, input: &[f32], output: &mut [f32]) -> Result<()> {
        self.check(unsafe {
            sys::wm_bitlinear_i2s_matvec_f32(self.h, w.h, input.as_ptr(), input.len(),
                                             output.as_mut_ptr(), output.len())
        })
    }

    /// bitlinear_i2s_matvec_f32_scalar (src/model/bitlinear.rs:146-233).
    pub fn bitlinear_i2s_matvec_f32_scalar(&self, w: &Tensor<'_>, input: &[f32], output: &mut [f32]) -> Result<()> {
        self.check(unsafe {
            sys::wm_bitlinear_i2s_matvec_f32_scalar(self.h, w.h, input.as_ptr(), input.len(),
                                                    output.as_mut_ptr(), output.len())
        })
    }

    /// Rows of x ([m][in_dim]) through the batched BitLinear; row r equals
    /// bitlinear_i2s_matvec_f32 on x[r].
    pub fn bitlinear_i2s_matmul_f32(&self, w: &Tensor<'_>, x: &[f32], m: u32, y: &mut [f32]) -> Result<()> {
        self.check(unsafe {
            sys::wm_bitlinear_i2s_matmul_f32(self.h, w.h, x.as_ptr(), x.len(), m, y.as_mut_ptr(), y.len())
        })
    }

    /// q6_k::dequantize_row (src/model/q6_k.rs:59-69) of one row.
    pub fn q6k_dequantize_row(&self, t: &Tensor<'_>, row: u64, out: &mut [f32]) -> Result<()> {
        self.check(unsafe { sys::wm_q6k_dequantize_row(self.h, t.h, row, out.as_mut_ptr(), out.len()) })
    }

    /// compute_logits (src/model/lm_head.rs:29-108) for a Q6_K tied head.
    pub fn compute_logits(&self, token_embd: &Tensor<'_>, hidden: &[f32], logits: &mut [f32]) -> Result<()> {
        self.check(unsafe {
            sys::wm_compute_logits(self.h, token_embd.h, hidden.as_ptr(), hidden.len(),
                                   logits.as_mut_ptr(), logits.len())
        })
    }

    /// argmax(compute_logits(..)); with `logits` None only the id is
    /// computed (the id-only lm-head: same id, no logits written).
    pub fn logits_argmax(&self, token_embd: &Tensor<'_>, hidden: &[f32], logits: Option<&mut [f32]>) -> Result<u32> {
        let mut id = 0u32;
        let lp = logits.map_or(ptr::null_mut(), |l| l.as_mut_ptr());
        self.check(unsafe {
            sys::wm_logits_argmax(self.h, token_embd.h, hidden.as_ptr(), hidden.len(), lp, &mut id)
        })?;
        Ok(id)
    }

    pub fn sampler(&self, params: &SamplingParams, seed: u64) -> Result<Sampler<'_>> {
        let mut h = ptr::null_mut();
        let raw = params.raw();
        self.check(unsafe { sys::wm_sampler_create(self.h, &raw, seed, &mut h) })?;
        Ok(Sampler { h, ctx: self })
    }
}

impl Drop for Context {
    fn drop(&mut self) {
        unsafe { sys::wm_ctx_destroy(self.h) }
    }
}

/// A weight on the device, in the library's layout.
pub struct Tensor<'c> {
    h: *mut sys::wm_tensor,
    ctx: &'c Context,
}

impl Tensor<'_> {
    pub fn raw(&self) -> *const sys::wm_tensor {
        self.h
    }

    /// ([in_dim, out_dim] or [row_len, n_rows], type id, I2_S scale)
    pub fn info(&self) -> Result<([u64; 2], i32, f32)> {
        let mut shape = [0u64; 2];
        let (mut ty, mut scale) = (0, 0f32);
        self.ctx.check(unsafe { sys::wm_tensor_info(self.h, shape.as_mut_ptr(), &mut ty, &mut scale) })?;
        Ok((shape, ty, scale))
    }
}

impl Drop for Tensor<'_> {
    fn drop(&mut self) {
        unsafe { sys::wm_tensor_destroy(self.h) }
    }
}

// ---------------------------------------------------------------------------
// model, cache, generation
// ---------------------------------------------------------------------------

pub type ModelConfig = sys::wm_model_config;

/// The device model graph (src/model/graph.rs:56-237).
pub struct Model<'c> {
    h: *mut sys::wm_model,
    ctx: &'c Context,
}

/// Borrowed weights of one layer for Model::set_layer.
pub struct LayerWeights<'a, 'c> {
    pub attn_q: &'a Tensor<'c>,
    pub attn_k: &'a Tensor<'c>,
    pub attn_v: &'a Tensor<'c>,
    pub attn_output: &'a Tensor<'c>,
    pub ffn_gate: &'a Tensor<'c>,
    pub ffn_up: &'a Tensor<'c>,
    pub ffn_down: &'a Tensor<'c>,
    pub attn_norm: &'a [f32],
    pub attn_sub_norm: &'a [f32],
    pub ffn_norm: &'a [f32],
    pub ffn_sub_norm: &'a [f32],
}

impl<'c> Model<'c> {
    pub fn new(ctx: &'c Context, cfg: &ModelConfig) -> Result<Model<'c>> {
        let mut h = ptr::null_mut();
        ctx.check(unsafe { sys::wm_model_create(ctx.h, cfg, &mut h) })?;
        Ok(Model { h, ctx })
    }

    /// ModelGraph::from_gguf for BitNet b1.58 (src/model/graph.rs:79-237):
    /// every tensor uploaded from the file; max_context 0 keeps the
    /// file's context_length.
    pub fn from_gguf(ctx: &'c Context, g: &Gguf, max_context: u32) -> Result<Model<'c>> {
        let mut h = ptr::null_mut();
        ctx.check(unsafe { sys::wm_model_from_gguf(ctx.h, g.h, max_context, &mut h) })?;
        Ok(Model { h, ctx })
    }

    pub fn set_layer(&mut self, layer: u32, w: &LayerWeights<'_, 'c>) -> Result<()> {
        self.ctx.check(unsafe {
            sys::wm_model_set_layer(self.h, layer, w.attn_q.h, w.attn_k.h, w.attn_v.h, w.attn_output.h,
                                    w.ffn_gate.h, w.ffn_up.h, w.ffn_down.h, w.attn_norm.as_ptr(),
                                    w.attn_sub_norm.as_ptr(), w.ffn_norm.as_ptr(), w.ffn_sub_norm.as_ptr())
        })
    }

    pub fn set_output(&mut self, token_embd: &Tensor<'c>, output_norm: &[f32]) -> Result<()> {
        self.ctx.check(unsafe { sys::wm_model_set_output(self.h, token_embd.h, output_norm.as_ptr()) })
    }

    /// KVCache::try_new (src/model/kv_cache.rs:67) on the device: int8
    /// codes and one f32 scale per position.
    pub fn kv_cache(&self, max_seq_len: u32) -> Result<KvCache<'_, 'c>> {
        let mut h = ptr::null_mut();
        self.ctx.check(unsafe { sys::wm_kv_cache_create(self.h, max_seq_len, &mut h) })?;
        Ok(KvCache { h, model: self })
    }

    /// forward_single_token_position_zero (src/model/forward.rs:29).
    pub fn forward_position_zero(&self, token: u32, hidden_out: &mut [f32]) -> Result<()> {
        self.ctx.check(unsafe {
            sys::wm_forward_single_token_position_zero(self.h, token, hidden_out.as_mut_ptr())
        })
    }

    /// One ragged step over several caches (multi_token_forward with a
    /// pre-filled cache per sequence); returns each sequence's next id.
    pub fn batch_forward(&self, caches: &mut [&mut KvCache<'_, 'c>], seqs: &[&[u32]],
                         last_hidden: Option<&mut [f32]>) -> Result<Vec<u32>> {
        let hs: Vec<*mut sys::wm_kv_cache> = caches.iter().map(|c| c.h).collect();
        let n_new: Vec<u32> = seqs.iter().map(|s| s.len() as u32).collect();
        let toks: Vec<u32> = seqs.iter().flat_map(|s| s.iter().copied()).collect();
        let mut next = vec![0u32; hs.len()];
        let lh = last_hidden.map_or(ptr::null_mut(), |h| h.as_mut_ptr());
        self.ctx.check(unsafe {
            sys::wm_batch_forward(self.h, hs.as_ptr(), hs.len() as u32, n_new.as_ptr(), toks.as_ptr(),
                                  lh, next.as_mut_ptr())
        })?;
        Ok(next)
    }

    /// A continuous-batching driver over this model.
    pub fn server(&self, max_seqs: u32, max_seq_len: u32, step_tokens: u32) -> Result<Server<'_, 'c>> {
        let mut h = ptr::null_mut();
        self.ctx.check(unsafe { sys::wm_server_create(self.h, max_seqs, max_seq_len, step_tokens, &mut h) })?;
        Ok(Server { h, model: self })
    }
}

impl Drop for Model<'_> {
    fn drop(&mut self) {
        unsafe { sys::wm_model_destroy(self.h) }
    }
}

/// KVCache (src/model/kv_cache.rs:49-259) on the device.
pub struct KvCache<'m, 'c> {
    h: *mut sys::wm_kv_cache,
    model: &'m Model<'c>,
}

impl KvCache<'_, '_> {
    pub fn position(&self) -> u32 {
        unsafe { sys::wm_kv_cache_position(self.h) }
    }

    pub fn rollback(&mut self, position: u32) -> Result<()> {
        self.model.ctx.check(unsafe { sys::wm_kv_cache_rollback(self.h, position) })
    }

    /// KVCache::read_into (src/model/kv_cache.rs:192-219): the dequantised
    /// window of one layer, [position][kv_dim].
    pub fn read_into(&mut self, layer: u32, k: &mut [f32], v: &mut [f32]) -> Result<()> {
        self.model.ctx.check(unsafe { sys::wm_kv_cache_read_into(self.h, layer, k.as_mut_ptr(), v.as_mut_ptr()) })
    }

    /// forward_with_cache_into (src/model/cached_forward.rs:164).
    pub fn forward(&mut self, token: u32, position: u32, hidden_out: &mut [f32]) -> Result<()> {
        self.model.ctx.check(unsafe {
            sys::wm_forward_with_cache(self.model.h, self.h, token, position, hidden_out.as_mut_ptr(),
                                       ptr::null_mut())
        })
    }

    /// One greedy step: forward + logits (optional) + argmax.
    pub fn decode_step(&mut self, token: u32, position: u32, logits: Option<&mut [f32]>) -> Result<u32> {
        let mut next = 0u32;
        let lp = logits.map_or(ptr::null_mut(), |l| l.as_mut_ptr());
        self.model.ctx.check(unsafe {
            sys::wm_decode_step(self.model.h, self.h, token, position, ptr::null_mut(), lp, &mut next)
        })?;
        Ok(next)
    }

    /// Batched prefill (src/model/generate.rs:151-160 in one pass).
    pub fn prefill(&mut self, tokens: &[u32], last_hidden: Option<&mut [f32]>) -> Result<()> {
        let lh = last_hidden.map_or(ptr::null_mut(), |h| h.as_mut_ptr());
        self.model.ctx.check(unsafe {
            sys::wm_prefill(self.model.h, self.h, tokens.as_ptr(), tokens.len() as u32, lh)
        })
    }

    /// greedy_generate_with_cache (src/model/generate.rs:111-189).
    pub fn greedy(&mut self, prompt: &[u32], max_new: u32, eos: Option<u32>) -> Result<Vec<u32>> {
        let mut out = vec![0u32; max_new.max(1) as usize];
        let mut n = 0u32;
        self.model.ctx.check(unsafe {
            sys::wm_greedy_generate(self.model.h, self.h, prompt.as_ptr(), prompt.len() as u32, max_new,
                                    eos.map_or(-1, i64::from), out.as_mut_ptr(), &mut n)
        })?;
        out.truncate(n as usize);
        Ok(out)
    }

    /// generate_with_cache_and_sampler (src/model/generate.rs:195-277).
    pub fn generate(&mut self, prompt: &[u32], max_new: u32, eos: Option<u32>, stop_ids: &[u32],
                    sampler: &mut Sampler<'_>) -> Result<Vec<u32>> {
        let mut out = vec![0u32; max_new.max(1) as usize];
        let mut n = 0u32;
        self.model.ctx.check(unsafe {
            sys::wm_generate_with_sampler(self.model.h, self.h, prompt.as_ptr(), prompt.len() as u32,
                                          max_new, eos.map_or(-1, i64::from), stop_ids.as_ptr(),
                                          stop_ids.len() as u32, sampler.h, out.as_mut_ptr(), &mut n)
        })?;
        out.truncate(n as usize);
        Ok(out)
    }
}

impl Drop for KvCache<'_, '_> {
    fn drop(&mut self) {
        unsafe { sys::wm_kv_cache_destroy(self.h) }
    }
}

// ---------------------------------------------------------------------------
// sampler and continuous batching
// ---------------------------------------------------------------------------

/// SamplingParams (src/model/sampler.rs:40-79).
#[derive(Debug, Clone, Default, PartialEq)]
pub struct SamplingParams {
    pub temperature: f32,
    pub top_k: Option<usize>,
    pub top_p: Option<f32>,
    pub repetition_penalty: Option<f32>,
}

impl SamplingParams {
    fn raw(&self) -> sys::wm_sampling_params {
        sys::wm_sampling_params {
            temperature: self.temperature,
            has_top_k: self.top_k.is_some() as u32,
            top_k: self.top_k.unwrap_or(0) as u64,
            top_p: self.top_p.unwrap_or(0.0),
            has_top_p: self.top_p.is_some() as u32,
            repetition_penalty: self.repetition_penalty.unwrap_or(0.0),
            has_repetition_penalty: self.repetition_penalty.is_some() as u32,
        }
    }
}

/// Sampler (src/model/sampler.rs:81-149) whose draws run on the device.
pub struct Sampler<'c> {
    h: *mut sys::wm_sampler,
    ctx: &'c Context,
}

impl Sampler<'_> {
    pub fn observe(&mut self, id: u32) {
        unsafe { sys::wm_sampler_observe(self.h, id) };
    }

    /// (xorshift state, history length), as SamplerCheckpoint.
    pub fn checkpoint(&self) -> (u64, u64) {
        let (mut s, mut n) = (0u64, 0u64);
        unsafe { sys::wm_sampler_checkpoint(self.h, &mut s, &mut n) };
        (s, n)
    }

    pub fn rollback(&mut self, cp: (u64, u64)) -> Result<()> {
        self.ctx.check(unsafe { sys::wm_sampler_rollback(self.h, cp.0, cp.1) })
    }

    /// Sampler::sample on host logits.
    pub fn sample(&mut self, logits: &[f32]) -> Result<u32> {
        let mut id = 0u32;
        self.ctx.check(unsafe { sys::wm_sampler_sample(self.h, logits.as_ptr(), logits.len(), &mut id) })?;
        Ok(id)
    }
}

impl Drop for Sampler<'_> {
    fn drop(&mut self) {
        unsafe { sys::wm_sampler_destroy(self.h) }
    }
}

/// Continuous batching: many generate_with_cache_and_sampler requests
/// advanced together, one ragged batch per step.
pub struct Server<'m, 'c> {
    h: *mut sys::wm_server,
    model: &'m Model<'c>,
}

impl Server<'_, '_> {
    pub fn submit(&mut self, prompt: &[u32], max_new: u32, eos: Option<u32>, stop_ids: &[u32],
                  params: &SamplingParams, seed: u64) -> Result<u64> {
        let raw = params.raw();
        let mut id = 0u64;
        self.model.ctx.check(unsafe {
            sys::wm_server_submit(self.h, prompt.as_ptr(), prompt.len() as u32, max_new,
                                  eos.map_or(-1, i64::from), stop_ids.as_ptr(), stop_ids.len() as u32,
                                  &raw, seed, &mut id)
        })?;
        Ok(id)
    }

    /// One batch step; the number of requests still active or waiting.
    pub fn step(&mut self) -> Result<u32> {
        let mut n = 0u32;
        self.model.ctx.check(unsafe { sys::wm_server_step(self.h, &mut n) })?;
        Ok(n)
    }

    /// (ids so far, finished); the request's own error if it failed.
    pub fn result(&self, request: u64) -> Result<(Vec<u32>, bool)> {
        let (mut n, mut fin) = (0u32, 0);
        self.model.ctx.check(unsafe {
            sys::wm_server_result(self.h, request, ptr::null_mut(), 0, &mut n, &mut fin)
        })?;
        let mut out = vec![0u32; n as usize];
        self.model.ctx.check(unsafe {
            sys::wm_server_result(self.h, request, out.as_mut_ptr(), n, &mut n, &mut fin)
        })?;
        Ok((out, fin != 0))
    }

    pub fn release(&mut self, request: u64) -> Result<()> {
        self.model.ctx.check(unsafe { sys::wm_server_release(self.h, request) })
    }
}

impl Drop for Server<'_, '_> {
    fn drop(&mut self) {
        unsafe { sys::wm_server_destroy(self.h) }
    }
}

// ---------------------------------------------------------------------------
// GGUF
// ---------------------------------------------------------------------------

/// A parsed GGUF v2/v3 file (src/gguf/reader.rs:120-415), memory-mapped or
/// parsed from bytes the caller keeps alive.
pub struct Gguf<'b> {
    h: *mut sys::wm_gguf,
    _bytes: PhantomData<&'b [u8]>,
}

fn gguf_result<'b>(st: sys::wm_status, h: *mut sys::wm_gguf, err: &[c_char]) -> Result<Gguf<'b>> {
    if st != sys::WM_OK {
        return Err(Error { status: Status::from_code(st), message: err_text(err) });
    }
    Ok(Gguf { h, _bytes: PhantomData })
}

impl Gguf<'static> {
    pub fn open(path: &Path) -> Result<Gguf<'static>> {
        let c = CString::new(path.to_string_lossy().as_bytes()).map_err(|_| Error {
            status: Status::Io,
            message: "path contains NUL".into(),
        })?;
        let mut h = ptr::null_mut();
        let mut err = [0 as c_char; 512];
        let st = unsafe { sys::wm_gguf_open(c.as_ptr(), &mut h, err.as_mut_ptr(), err.len()) };
        gguf_result(st, h, &err)
    }
}

impl<'b> Gguf<'b> {
    pub fn parse(bytes: &'b [u8]) -> Result<Gguf<'b>> {
        let mut h = ptr::null_mut();
        let mut err = [0 as c_char; 512];
        let st = unsafe { sys::wm_gguf_parse(bytes.as_ptr(), bytes.len(), &mut h, err.as_mut_ptr(), err.len()) };
        gguf_result(st, h, &err)
    }

    pub fn version(&self) -> u32 {
        unsafe { sys::wm_gguf_version(self.h) }
    }

    pub fn tensor_count(&self) -> u64 {
        unsafe { sys::wm_gguf_tensor_count(self.h) }
    }

    /// ModelConfig::from_gguf_metadata for a BitNet file (src/model/config.rs:61-163).
    pub fn bitnet_config(&self) -> Result<ModelConfig> {
        let mut cfg = ModelConfig::default();
        let mut err = [0 as c_char; 512];
        let st = unsafe { sys::wm_gguf_bitnet_config(self.h, &mut cfg, err.as_mut_ptr(), err.len()) };
        if st != sys::WM_OK {
            return Err(Error { status: Status::from_code(st), message: err_text(&err) });
        }
        Ok(cfg)
    }
}

impl Drop for Gguf<'_> {
    fn drop(&mut self) {
        unsafe { sys::wm_gguf_close(self.h) }
    }
}
