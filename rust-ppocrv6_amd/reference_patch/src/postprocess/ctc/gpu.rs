//! The compact CTC entries beside CtcDecoder::decode_batch (src/postprocess/ctc.rs:103-175):
//! drop this file into the reference crate as `src/postprocess/ctc/gpu.rs` with `mod gpu;`
//! in src/postprocess/ctc.rs (a child module sees the decoder's private vocabulary).  The
//! head call returns each line's emitted class indices and score under decode_batch's rules
//! (emit when idx != blank and idx != the previous step's, the previous index updated on
//! blanks too; score = f32 sum of the emitted maximum probabilities / count); these
//! functions only map indices to characters.
use super::CtcDecoder;
use crate::error::Result;
use crate::ops::gpu_head::{check, GpuHead};
use crate::tensor::Tensor;
use ppocr_hip_sys as sys;

impl CtcDecoder {
    fn text_of(&self, seq: &[i32]) -> String {
        seq.iter().map(|&c| self.vocab[c as usize].as_str()).collect()
    }

    /// Text lines packed back to back (line i = rows line_off[i] .. line_off[i+1] of the
    /// activations [sum T_i, k]): the whole head on the GPU, one call per page.
    pub fn decode_page(&self, head: &GpuHead, acts: &Tensor, line_off: &[i64]) -> Result<Vec<(String, f32)>> {
        let (seq, len, score) = head.decode_lines(acts, line_off)?;
        let lines = line_off.len().saturating_sub(1);
        Ok((0..lines)
            .map(|i| {
                let s0 = line_off[i] as usize;
                (self.text_of(&seq[s0..s0 + len[i] as usize]), score[i])
            })
            .collect())
    }

    /// The neck's output before Transpose.8, x [B, 120, T] (equal-width lines, channels
    /// first): line b is rows b*T .. b*T + T.
    pub fn decode_nct(&self, head: &GpuHead, x: &Tensor) -> Result<Vec<(String, f32)>> {
        let (seq, len, score, t) = head.decode_nct(x)?;
        Ok((0..len.len().min(x.shape()[0]))
            .map(|b| (self.text_of(&seq[b * t..b * t + len[b] as usize]), score[b]))
            .collect())
    }

    /// From per-step (argmax, maximum probability) rows of text lines (e.g. GpuHead::argmax):
    /// the collapse and score on the GPU (ppocr_ctc_greedy, blank 0).
    pub fn decode_compact(&self, idx: &[i32], maxprob: &[f32], line_off: &[i64]) -> Result<Vec<(String, f32)>> {
        let lines = line_off.len().saturating_sub(1);
        let steps = line_off.last().copied().unwrap_or(0).max(0) as usize;
        if idx.len() < steps || maxprob.len() < steps {
            return Err(crate::error::OcrError::OperatorError {
                op: "CtcDecode".into(),
                msg: format!("{} steps in the offsets, {} / {} given", steps, idx.len(), maxprob.len()),
            });
        }
        let (mut seq, mut len, mut score) = (vec![0i32; steps.max(1)], vec![0i64; lines.max(1)], vec![0f32; lines.max(1)]);
        check("CtcDecode", unsafe {
            sys::ppocr_ctc_greedy(idx.as_ptr(), maxprob.as_ptr(), line_off.as_ptr(), lines as i64, 0, seq.as_mut_ptr(),
                                  len.as_mut_ptr(), score.as_mut_ptr())
        })?;
        Ok((0..lines)
            .map(|i| {
                let s0 = line_off[i] as usize;
                (self.text_of(&seq[s0..s0 + len[i] as usize]), score[i])
            })
            .collect())
    }
}
