//! The entry points det_hip.h adds to the C API shared with det_cuda.h (feature `hip`; include/det_hip.h).  The
//! shared declarations in det-sys's lib.rs apply unchanged: lib.rs's cfg gains `feature = "hip"` and declares
//! `#[cfg(feature = "hip")] pub mod hip;`.  UNVERIFIED: no Rust toolchain was available where this was written.

use crate::QLinear;
use std::ffi::{c_int, c_void};

pub type Stream = *mut c_void;

extern "C" {
    /// The stream det's work runs on (det_cuda_stream's counterpart): the null stream.
    pub fn det_hip_stream() -> *mut c_void;
    /// Byte sizes of the three planes det_linear_repack writes for an n x k linear of `bits`.
    pub fn det_linear_sizes(n: c_int, k: c_int, bits: c_int, wq_bytes: *mut usize, c_bytes: *mut usize, m_bytes: *mut usize);
    /// Load-time repack of n det rows (device memory) into this backend's private layout.
    pub fn det_linear_repack(rows: *const u8, n: c_int, k: c_int, bits: c_int, wq: *mut u8, c: *mut f32, m: *mut u16, st: Stream);
    /// det convert's quantizer (quantize.rs:33-100) on the device: n rows of k fp32 -> n det rows.
    pub fn det_quantize_rows(w: *const f32, n: c_int, k: c_int, bits: c_int, rows: *mut u8, st: Stream);
}

/// A QLinear whose planes come from det_linear_repack (the same struct as the CUDA runtime's).
pub fn qlinear(wq: *const u8, c: *const f32, m: *const u16, n: usize, k: usize, bits: u32) -> QLinear {
    QLinear { wq, c, m, n: n as c_int, k: k as c_int, bits: bits as c_int }
}
