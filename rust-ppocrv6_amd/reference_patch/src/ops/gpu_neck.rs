//! The SVTR mixing tail of the recognition model on the MI355X, for the segment of the
//! rec graph from Transpose.0 to Transpose.8 (src/engine/model.rs: the MatMul, LayerNorm
//! sub-graph, Softmax, Sigmoid, Mul and Add nodes that Model::forward runs between them).
//! Drop this file into the reference crate as `src/ops/gpu_neck.rs` (with
//! `pub mod gpu_neck;` in src/ops/mod.rs); its output is the input of `GpuHead`.
use std::ffi::CString;

use crate::error::{OcrError, Result};
use crate::ops::gpu_head::check;
use crate::tensor::Tensor;
use ppocr_hip_sys as sys;

/// The tail's weights resident in HBM (2 blocks of D = 120, 8 heads of 15, hidden 240 in
/// PP-OCRv6_small_rec).  Immutable after creation and shareable across the rec_pool
/// workers: every host-pointer call takes its own device arena and stream.
pub struct GpuNeck {
    h: *mut sys::ppocr_rn_t,
    dim: usize,
}
unsafe impl Send for GpuNeck {}
unsafe impl Sync for GpuNeck {}

impl GpuNeck {
    /// The tail found in the model's graph (the LayerNorm sub-graphs, attention and MLP
    /// nodes between the flatten's Transpose and the head's Transpose), weights read from
    /// the same file.
    pub fn from_model(path: &std::path::Path, device: i32) -> Result<Self> {
        use std::os::unix::ffi::OsStrExt;
        let p = CString::new(path.as_os_str().as_bytes())
            .map_err(|_| OcrError::ModelError("a path holds a NUL byte".into()))?;
        let mut h = std::ptr::null_mut();
        check("RecNeckHip", unsafe { sys::ppocr_rn_create_from_model(p.as_ptr(), device, &mut h) })?;
        let (mut dim, mut heads, mut hidden, mut blocks) = (0i64, 0i64, 0i64, 0i32);
        let rc = unsafe { sys::ppocr_rn_shape(h, &mut dim, &mut heads, &mut hidden, &mut blocks) };
        if rc != sys::PPOCR_OK {
            unsafe { sys::ppocr_rn_destroy(h) };
            check("RecNeckHip", rc)?;
        }
        Ok(Self { h, dim: dim as usize })
    }

    /// Transpose.0 -> ... -> Transpose.8 for a batch of equal-width lines: `x` the flatten
    /// output [B, D, T] and `shortcut` the tensor the final Add reads, [B, D, 1, T], both
    /// channels first as the graph holds them; returns [B, T, D], the head's input.
    pub fn forward_nct(&self, x: &Tensor, shortcut: &Tensor) -> Result<Tensor> {
        let s = x.shape();
        if s.len() != 3 || s[1] != self.dim {
            return Err(OcrError::OperatorError { op: "RecNeckHip".into(), msg: format!("expected [B, {}, T], got {:?}", self.dim, s) });
        }
        if shortcut.numel() != x.numel() {
            return Err(OcrError::OperatorError {
                op: "RecNeckHip".into(),
                msg: format!("shortcut {:?} does not match the input {:?}", shortcut.shape(), s),
            });
        }
        let (b, t) = (s[0], s[2]);
        let off: Vec<i64> = (0..=b).map(|i| (i * t) as i64).collect();
        let mut out = Tensor::empty(&[b, t, self.dim]);
        check("RecNeckHip", unsafe {
            sys::ppocr_rn_forward(self.h, x.as_slice().as_ptr(), shortcut.as_slice().as_ptr(), off.as_ptr(), b as i64,
                                  sys::PPOCR_NECK_CHANNELS_FIRST, out.as_mut_slice().as_mut_ptr())
        })?;
        Ok(out)
    }

    /// The same for ragged lines packed back to back as token rows (line i = rows
    /// line_off[i] .. line_off[i+1] of `x` and `shortcut`, [m, D] each): the page batch
    /// that `GpuHead::decode_lines` then decodes with the same offsets.
    pub fn forward_lines(&self, x: &Tensor, shortcut: &Tensor, line_off: &[i64]) -> Result<Tensor> {
        let m = line_off.last().copied().unwrap_or(0).max(0) as usize;
        if x.numel() < m * self.dim || shortcut.numel() < m * self.dim {
            return Err(OcrError::OperatorError { op: "RecNeckHip".into(), msg: "line offsets beyond the inputs".into() });
        }
        let lines = line_off.len().saturating_sub(1);
        let mut out = Tensor::empty(&[m, self.dim]);
        check("RecNeckHip", unsafe {
            sys::ppocr_rn_forward(self.h, x.as_slice().as_ptr(), shortcut.as_slice().as_ptr(), line_off.as_ptr(),
                                  lines as i64, sys::PPOCR_NECK_ROWS, out.as_mut_slice().as_mut_ptr())
        })?;
        Ok(out)
    }
}

impl Drop for GpuNeck {
    fn drop(&mut self) {
        unsafe { sys::ppocr_rn_destroy(self.h) }
    }
}
