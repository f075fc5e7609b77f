//! `src/model/hip.rs` for project-willamette: the `Kernel::Hip` backend.
//!
//! Not part of this crate's build: it names project-willamette's own types
//! (`TensorView`, `WillametteError`, `GgmlType`) and is meant to be added to
//! that crate next to `dispatch.rs`, with `willamette-hip-sys` as a
//! dependency.  See dispatch_hip.rs in this folder for the matching edits to
//! `src/model/dispatch.rs` and `src/model/bitlinear.rs`.
//!
//! One process-wide context on device 0, created on first use when
//! `WILLAMETTE_HIP=1`; weights are uploaded once, keyed by the address of
//! their bytes in the memory-mapped file (`TensorView::data`, stable for the
//! mapping's lifetime, src/gguf/tensor.rs:45).

use std::collections::HashMap;
use std::sync::{Mutex, OnceLock};

use willamette_hip_sys as hip;

use crate::error::WillametteError;
use crate::gguf::tensor::TensorView;
use crate::gguf::types::GgmlType;

pub(crate) struct HipBackend {
    ctx: &'static hip::Context,
    tensors: HashMap<usize, hip::Tensor<'static>>,
}

// The context and its tensors are only touched under the Mutex below.
unsafe impl Send for HipBackend {}

static BACKEND: OnceLock<Option<Mutex<HipBackend>>> = OnceLock::new();

/// The backend, if `WILLAMETTE_HIP=1` and a gfx950 device opens.
pub(crate) fn backend() -> Option<&'static Mutex<HipBackend>> {
    BACKEND
        .get_or_init(|| {
            if std::env::var("WILLAMETTE_HIP").ok().as_deref() != Some("1") {
                return None;
            }
            let ctx = hip::Context::new(0).ok()?;
            Some(Mutex::new(HipBackend { ctx: Box::leak(Box::new(ctx)), tensors: HashMap::new() }))
        })
        .as_ref()
}

/// The library's status as the reference's error (src/error.rs:9-57).
pub(crate) fn to_willamette(e: hip::Error, raw_type: u32) -> WillametteError {
    match e.status {
        hip::Status::UnsupportedTensorType => WillametteError::UnsupportedTensorType(raw_type),
        hip::Status::NotImplemented => WillametteError::NotImplemented(e.message),
        _ => WillametteError::GgufParse(e.message),
    }
}

impl HipBackend {
    fn tensor_for(&mut self, weight: &TensorView<'_>) -> Result<&hip::Tensor<'static>, WillametteError> {
        let key = weight.data.as_ptr() as usize;
        if !self.tensors.contains_key(&key) {
            if weight.ggml_type != GgmlType::BitNetI2S {
                return Err(WillametteError::UnsupportedTensorType(weight.ggml_type.to_raw()));
            }
            if weight.shape.len() != 2 {
                return Err(WillametteError::GgufParse(format!(
                    "bitlinear_i2s_matvec_f32: weight {:?} is not 2-D (shape={:?})",
                    weight.name, weight.shape
                )));
            }
            let scale = weight.scale_data.unwrap_or(&[]);
            let t = self
                .ctx
                .upload_i2s(weight.data, scale, weight.shape[0], weight.shape[1])
                .map_err(|e| to_willamette(e, weight.ggml_type.to_raw()))?;
            self.tensors.insert(key, t);
        }
        Ok(&self.tensors[&key])
    }

    /// bitlinear_i2s_matvec_f32 on the device: the SSE2-i8 result bit for bit.
    pub(crate) fn bitlinear_i2s_matvec_f32(
        &mut self,
        weight: &TensorView<'_>,
        input: &[f32],
        output: &mut [f32],
    ) -> Result<(), WillametteError> {
        let raw = weight.ggml_type.to_raw();
        let ctx = self.ctx;
        let t = self.tensor_for(weight)?;
        ctx.bitlinear_i2s_matvec_f32(t, input, output).map_err(|e| to_willamette(e, raw))
    }
}
