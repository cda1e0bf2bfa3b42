//! The MI355X recognition head as an operator of rust_ppocrv6: drop this file into the
//! reference crate as `src/ops/gpu_head.rs` (with `pub mod gpu_head;` in src/ops/mod.rs and
//! `ppocr-hip-sys` as a dependency).  It binds the C ABI of libppocr_rechead
//! (include/ppocr_rechead.h) at the executor's MatMul dispatch (src/engine/model.rs:1261-1264)
//! and mirrors `matmul_quantized_b` (src/ops/matmul.rs:1204-1208).
use std::ffi::{CStr, CString};
use std::os::raw::c_char;
use std::path::Path;

use crate::error::{OcrError, Result};
use crate::ops::QuantizedWeight;
use crate::tensor::Tensor;
use ppocr_hip_sys as sys;

/// Where the recognition head runs: the new field `OcrEngineConfig::rec_head_backend`
/// (beside `quantize_rec_head`, src/pipeline.rs:38-40).
#[derive(Clone, Copy, Debug, Default, PartialEq, Eq)]
pub enum RecHeadBackend {
    /// The reference's own CPU operators (matmul_quantized_b / matmul_transposed_b,
    /// softmax_inplace, CtcDecoder::decode_batch).
    #[default]
    Cpu,
    /// The MI355X head on HIP device `device`: the INT8 head when `quantize_rec_head` is set
    /// (the packing of Model::quantize_matmul_weights, bit for bit), the FP32 head otherwise.
    Hip { device: i32 },
}

fn last_error() -> String {
    unsafe { CStr::from_ptr(sys::ppocr_last_error()) }.to_string_lossy().into_owned()
}

/// A library status as the reference's error (src/error.rs:4-27): model-file problems are
/// SafeTensorsError / ModelError, the rest OperatorError { op, msg } with the op name the
/// library puts before its message.
pub(crate) fn check(op: &str, rc: i32) -> Result<()> {
    if rc == sys::PPOCR_OK {
        return Ok(());
    }
    let text = last_error();
    if rc == sys::PPOCR_ERR_MODEL {
        return Err(OcrError::SafeTensorsError(text));
    }
    let (op, msg) = match text.split_once(": ") {
        Some((o, m)) => (o.to_string(), m.to_string()),
        None => (op.to_string(), text),
    };
    Err(OcrError::OperatorError { op, msg })
}

fn cstring(s: &[u8]) -> Result<CString> {
    CString::new(s).map_err(|_| OcrError::ModelError("a path or tensor name holds a NUL byte".into()))
}

/// The head weight resident in HBM.  Immutable after creation and shareable across the
/// rec_pool workers (src/pipeline.rs:417-433): the C handle is thread-safe, and every
/// host-pointer call takes its own device arena and stream.
pub struct GpuHead {
    h: *mut sys::ppocr_rh_t,
    n: usize,
    k: usize,
    quantized: bool,
    mode: i32,
}
unsafe impl Send for GpuHead {}
unsafe impl Sync for GpuHead {}

impl GpuHead {
    fn from_handle(h: *mut sys::ppocr_rh_t) -> Result<Self> {
        let (mut n, mut k, mut q) = (0i64, 0i64, 0i32);
        check("RecHeadHip", unsafe { sys::ppocr_rh_shape(h, &mut n, &mut k, &mut q) })?;
        // the split the library picks for these weights (bf16 or fp16 terms), with the
        // precision guard
        let mode = sys::PPOCR_MODE_AUTO;
        Ok(Self { h, n: n as usize, k: k as usize, quantized: q != 0, mode })
    }

    /// From the packed weight Model::quantize_matmul_weights built (src/engine/model.rs:628-638)
    /// and the folded bias.
    pub fn new(qw: &QuantizedWeight, bias: Option<&Tensor>, device: i32) -> Result<Self> {
        let mut h = std::ptr::null_mut();
        let b = bias.map_or(std::ptr::null(), |t| t.as_slice().as_ptr());
        check("MatMulQuantizedB", unsafe {
            sys::ppocr_rh_create(qw.data.as_ptr(), qw.scales.as_ptr(), b, qw.rows as i64, qw.cols as i64, device,
                                 &mut h)
        })?;
        Self::from_handle(h)
    }

    /// From an FP32 transposed weight W^T [n][k] (the prepack, src/engine/model.rs:565-605).
    pub fn new_f32(w_t: &Tensor, bias: Option<&Tensor>, device: i32) -> Result<Self> {
        let s = w_t.shape();
        if s.len() != 2 {
            return Err(OcrError::OperatorError { op: "MatMulTransposedB".into(), msg: format!("W^T must be 2-D, got {:?}", s) });
        }
        let mut h = std::ptr::null_mut();
        let b = bias.map_or(std::ptr::null(), |t| t.as_slice().as_ptr());
        check("MatMulTransposedB", unsafe {
            sys::ppocr_rh_create_f32(w_t.as_slice().as_ptr(), b, s[0] as i64, s[1] as i64, device, &mut h)
        })?;
        Self::from_handle(h)
    }

    /// Straight from the model file (load_safetensors_model, src/engine/loader.rs:34-92): the
    /// weight goes to HBM as stored; transpose, INT8 packing and tile records run on the GPU.
    pub fn from_safetensors(path: &Path, weight: &str, bias: Option<&str>, quantize: bool, device: i32)
                            -> Result<Self> {
        use std::os::unix::ffi::OsStrExt;
        let p = cstring(path.as_os_str().as_bytes())?;
        let w = cstring(weight.as_bytes())?;
        let b = bias.map(|b| cstring(b.as_bytes())).transpose()?;
        let mut h = std::ptr::null_mut();
        check("RecHeadHip", unsafe {
            sys::ppocr_rh_create_from_safetensors(p.as_ptr(), w.as_ptr(), b.as_ref().map_or(std::ptr::null(), |b| b.as_ptr()),
                                                  quantize as i32, device, &mut h)
        })?;
        Self::from_handle(h)
    }

    /// The head the fused hook replaces, found in the model's graph (MatMul -> [Add] ->
    /// Softmax over the last axis -> output, with the load-time Identity, bias-fold and axis
    /// rules of src/engine/model.rs:67-166, 1286-1302), built from the file.
    pub fn from_model(path: &Path, quantize: bool, device: i32) -> Result<Self> {
        use std::os::unix::ffi::OsStrExt;
        let p = cstring(path.as_os_str().as_bytes())?;
        let (mut wname, mut bname) = ([0 as c_char; 256], [0 as c_char; 256]);
        let (mut n, mut k) = (0i64, 0i64);
        check("RecHeadHip", unsafe {
            sys::ppocr_model_find_rec_head(p.as_ptr(), wname.as_mut_ptr(), wname.len(), bname.as_mut_ptr(), bname.len(),
                                           &mut n, &mut k)
        })?;
        let w = unsafe { CStr::from_ptr(wname.as_ptr()) }.to_string_lossy().into_owned();
        let b = unsafe { CStr::from_ptr(bname.as_ptr()) }.to_string_lossy().into_owned();
        Self::from_safetensors(path, &w, if b.is_empty() { None } else { Some(b.as_str()) }, quantize, device)
    }

    /// The head for an engine configuration (OcrEngine::with_config, src/pipeline.rs:195-199):
    /// None for the CPU backend; on HIP the INT8 head when `quantize_rec_head` is set and the
    /// FP32 head otherwise.  `enable_rec_quantization` (src/pipeline.rs:267-270) rebuilds it
    /// with `quantize_rec_head = true`.
    pub fn for_config(rec_path: &Path, backend: RecHeadBackend, quantize_rec_head: bool) -> Result<Option<Self>> {
        match backend {
            RecHeadBackend::Cpu => Ok(None),
            RecHeadBackend::Hip { device } => Self::from_model(rec_path, quantize_rec_head, device).map(Some),
        }
    }

    pub fn is_quantized(&self) -> bool {
        self.quantized
    }

    /// Classes (the vocabulary) and the width of an activation row.
    pub fn n(&self) -> usize {
        self.n
    }
    pub fn k(&self) -> usize {
        self.k
    }

    /// Model::weight_footprint_bytes' share of this weight (src/engine/model.rs:651-667).
    pub fn footprint_bytes(&self) -> usize {
        unsafe { sys::ppocr_rh_footprint_bytes(self.h) }
    }

    fn rows_of(&self, a: &Tensor, op: &str) -> Result<usize> {
        let shape = a.shape();
        if shape.is_empty() || shape[shape.len() - 1] != self.k {
            return Err(OcrError::OperatorError {
                op: op.into(),
                msg: format!("Inner dimensions must match: {} != {}", shape.last().copied().unwrap_or(0), self.k),
            });
        }
        Ok(a.numel() / self.k)
    }

    /// Drop-in for matmul_quantized_b(a, qw, bias) (src/ops/matmul.rs:1204-1208) or
    /// matmul_transposed_b (src/ops/matmul.rs:514): out shape a.shape[..-1] + [n].
    pub fn logits(&self, a: &Tensor) -> Result<Tensor> {
        let op = if self.quantized { "MatMulQuantizedB" } else { "MatMulTransposedB" };
        let m = self.rows_of(a, op)?;
        let mut out_shape = a.shape()[..a.shape().len() - 1].to_vec();
        out_shape.push(self.n);
        let mut out = Tensor::empty(&out_shape);
        check(op, unsafe {
            sys::ppocr_rh_logits(self.h, a.as_slice().as_ptr(), m as i64, self.mode, out.as_mut_slice().as_mut_ptr())
        })?;
        Ok(out)
    }

    /// MatMul.12 -> Softmax.2 (the graph output fetch_name_0): probabilities written straight
    /// from the projection.
    pub fn probs(&self, a: &Tensor) -> Result<Tensor> {
        let m = self.rows_of(a, "RecHeadHip")?;
        let mut out_shape = a.shape()[..a.shape().len() - 1].to_vec();
        out_shape.push(self.n);
        let mut out = Tensor::empty(&out_shape);
        check("RecHeadHip", unsafe {
            sys::ppocr_rh_probs(self.h, a.as_slice().as_ptr(), m as i64, self.mode, out.as_mut_slice().as_mut_ptr())
        })?;
        Ok(out)
    }

    /// MatMul.12 -> Softmax.2 -> find_argmax, compact: per row (argmax, max probability),
    /// all that CtcDecoder::decode_batch reads (src/postprocess/ctc.rs:151-163).
    pub fn argmax(&self, a: &Tensor) -> Result<(Vec<i32>, Vec<f32>)> {
        let m = self.rows_of(a, "RecHeadHip")?;
        let (mut idx, mut mp) = (vec![0i32; m], vec![0f32; m]);
        check("RecHeadHip", unsafe {
            sys::ppocr_rh_argmax(self.h, a.as_slice().as_ptr(), m as i64, self.mode, idx.as_mut_ptr(), mp.as_mut_ptr())
        })?;
        Ok((idx, mp))
    }

    /// The whole head for text lines packed back to back (line i = rows line_off[i] ..
    /// line_off[i+1]): per line the emitted class indices (seq[line_off[i] ..][.. seq_len[i]])
    /// and the score.
    pub(crate) fn decode_lines(&self, acts: &Tensor, line_off: &[i64]) -> Result<(Vec<i32>, Vec<i64>, Vec<f32>)> {
        self.rows_of(acts, "RecHeadHip")?;
        let lines = line_off.len().saturating_sub(1);
        let m = line_off.last().copied().unwrap_or(0).max(0) as usize;
        if m * self.k > acts.numel() {
            return Err(OcrError::OperatorError { op: "CtcDecode".into(), msg: "line offsets beyond the activations".into() });
        }
        let (mut seq, mut len, mut score) = (vec![0i32; m.max(1)], vec![0i64; lines.max(1)], vec![0f32; lines.max(1)]);
        check("RecHeadHip", unsafe {
            sys::ppocr_rh_decode(self.h, acts.as_slice().as_ptr(), line_off.as_ptr(), lines as i64, self.mode,
                                 std::ptr::null_mut(), std::ptr::null_mut(), seq.as_mut_ptr(), len.as_mut_ptr(),
                                 score.as_mut_ptr())
        })?;
        Ok((seq, len, score))
    }

    /// The same from the neck's output before Transpose.8 (src/engine/model.rs:1325-1342):
    /// x [lines][k][steps], channels first, read in place.
    pub(crate) fn decode_nct(&self, x: &Tensor) -> Result<(Vec<i32>, Vec<i64>, Vec<f32>, usize)> {
        let s = x.shape();
        if s.len() != 3 || s[1] != self.k {
            return Err(OcrError::OperatorError { op: "RecHeadHip".into(), msg: format!("expected [lines, {}, T], got {:?}", self.k, s) });
        }
        let (b, t) = (s[0], s[2]);
        let (mut seq, mut len, mut score) = (vec![0i32; (b * t).max(1)], vec![0i64; b.max(1)], vec![0f32; b.max(1)]);
        check("RecHeadHip", unsafe {
            sys::ppocr_rh_decode_nct(self.h, x.as_slice().as_ptr(), b as i64, t as i64, self.mode, std::ptr::null_mut(),
                                     std::ptr::null_mut(), seq.as_mut_ptr(), len.as_mut_ptr(), score.as_mut_ptr())
        })?;
        Ok((seq, len, score, t))
    }
}

impl Drop for GpuHead {
    fn drop(&mut self) {
        unsafe { sys::ppocr_rh_destroy(self.h) }
    }
}
