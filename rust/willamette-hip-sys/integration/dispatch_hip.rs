//! The edits to project-willamette that route BitLinear through the device
//! (not compiled here; shown as the code a maintainer would add).
//!
//! 1. src/model/mod.rs: `pub(crate) mod hip;` (integration/hip.rs).
//!
//! 2. src/model/dispatch.rs:47-71, one more variant:
//!
//!        pub enum Kernel { Scalar, AArch64Neon, X86Sse2, X86Sse2ScalarLut, Hip }
//!
//!    its label (`Kernel::label`, :73-104):
//!
//!        Kernel::Hip => "MI355X HIP (gfx950, i8)",
//!
//!    and the first test in `select_kernel` (:159-184), before the CPU
//!    feature checks:
//!
//!        if super::hip::backend().is_some() {
//!            return Kernel::Hip;
//!        }
//!
//! 3. src/model/bitlinear.rs:77-141, one more arm in
//!    `bitlinear_i2s_matvec_f32`'s match on `active_kernel()`:

use crate::error::WillametteError;
use crate::gguf::tensor::TensorView;

#[allow(dead_code)]
fn kernel_hip_arm(
    weight: &TensorView<'_>,
    input: &[f32],
    output: &mut [f32],
) -> Result<(), WillametteError> {
    // super::dispatch::Kernel::Hip => { ...this body... }
    let backend = super::hip::backend().expect("Kernel::Hip is selected only with a backend");
    let mut guard = backend.lock().expect("hip backend mutex");
    guard.bitlinear_i2s_matvec_f32(weight, input, output)
}
