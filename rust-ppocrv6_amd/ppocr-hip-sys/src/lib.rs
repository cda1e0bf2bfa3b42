//! Raw FFI declarations of libppocr_rechead (include/ppocr_rechead.h): the MI355X (gfx950)
//! recognition head of rust_ppocrv6, i.e. the INT8 packer
//! (`QuantizedWeight::from_f32_transposed`, src/ops/matmul.rs:1173-1202), the vocabulary
//! projection MatMul.12 (`matmul_quantized_b`, src/ops/matmul.rs:1204-1208, and
//! `matmul_transposed_b`, src/ops/matmul.rs:514), Softmax.2 (`softmax_inplace`,
//! src/ops/softmax.rs:199) and the CTC greedy decode (`CtcDecoder::decode_batch`,
//! src/postprocess/ctc.rs:103-175), as bound at the executor's MatMul dispatch
//! (src/engine/model.rs:1261-1264).
//!
//! Every function returning `c_int` returns `PPOCR_OK` on success and otherwise a
//! `PPOCR_ERR_*` code, with `ppocr_last_error()` (thread-local) holding `"<op>: <msg>"`.
//! `_dev` functions take device pointers and a `hipStream_t` passed as `*mut c_void` (null:
//! the null stream) and only enqueue.  A head handle is immutable after creation and may be
//! shared by threads.
#![allow(non_camel_case_types)]
#![no_std]

use core::ffi::{c_char, c_int, c_void};

pub const PPOCR_OK: c_int = 0;
pub const PPOCR_ERR_INVALID_ARG: c_int = 1;
pub const PPOCR_ERR_DEVICE: c_int = 2;
pub const PPOCR_ERR_NO_MEMORY: c_int = 3;
pub const PPOCR_ERR_MODEL: c_int = 4;

pub const PPOCR_MODE_FP32_FMA: c_int = 0;
pub const PPOCR_MODE_BF16X1: c_int = 1;
pub const PPOCR_MODE_BF16X2: c_int = 2;
pub const PPOCR_MODE_BF16X3: c_int = 3;
pub const PPOCR_MODE_F16X2: c_int = 4;
pub const PPOCR_MODE_AUTO: c_int = 5;

pub const PPOCR_NECK_ROWS: c_int = 0;
pub const PPOCR_NECK_CHANNELS_FIRST: c_int = 1;

/// Opaque head handle (`ppocr_rh_t`).
#[repr(C)]
pub struct ppocr_rh_t {
    _private: [u8; 0],
}

/// Opaque neck handle (`ppocr_rn_t`).
#[repr(C)]
pub struct ppocr_rn_t {
    _private: [u8; 0],
}

/// One transformer block's weights (`ppocr_rn_block_t`), host pointers; MatMul weights
/// row-major [K][N] as the model stores them.
#[repr(C)]
#[derive(Clone, Copy)]
pub struct ppocr_rn_block_t {
    pub ln1_w: *const f32,
    pub ln1_b: *const f32,
    pub ln1_eps: f32,
    pub qkv_w: *const f32,
    pub qkv_b: *const f32,
    pub proj_w: *const f32,
    pub proj_b: *const f32,
    pub ln2_w: *const f32,
    pub ln2_b: *const f32,
    pub ln2_eps: f32,
    pub fc1_w: *const f32,
    pub fc1_b: *const f32,
    pub fc2_w: *const f32,
    pub fc2_b: *const f32,
}

extern "C" {
    pub fn ppocr_last_error() -> *const c_char;

    // ---- packer: QuantizedWeight::from_f32_transposed (src/ops/matmul.rs:1173-1202)
    pub fn ppocr_rh_pack_int8(w_t: *const f32, n: i64, k: i64, q_out: *mut i8, scales_out: *mut f32) -> c_int;
    pub fn ppocr_rh_pack_int8_dev(d_w_t: *const f32, n: i64, k: i64, d_q_out: *mut i8, d_scales_out: *mut f32,
                                  stream: *mut c_void) -> c_int;

    // ---- head handle: Model::quantize_matmul_weights (src/engine/model.rs:628-638) or the
    // FP32 prepack (src/engine/model.rs:565-605), bias folded (src/engine/model.rs:141-166)
    pub fn ppocr_rh_create(q: *const i8, scales: *const f32, bias: *const f32, n: i64, k: i64, device: c_int,
                           out: *mut *mut ppocr_rh_t) -> c_int;
    pub fn ppocr_rh_create_f32(w_t: *const f32, bias: *const f32, n: i64, k: i64, device: c_int,
                               out: *mut *mut ppocr_rh_t) -> c_int;
    pub fn ppocr_rh_create_from_safetensors(path: *const c_char, weight_name: *const c_char,
                                            bias_name: *const c_char, quantize: c_int, device: c_int,
                                            out: *mut *mut ppocr_rh_t) -> c_int;
    pub fn ppocr_model_find_rec_head(path: *const c_char, weight_name: *mut c_char, weight_cap: usize,
                                     bias_name: *mut c_char, bias_cap: usize, n: *mut i64, k: *mut i64) -> c_int;
    pub fn ppocr_rh_destroy(h: *mut ppocr_rh_t);
    /// Model::weight_footprint_bytes (src/engine/model.rs:651-667): n*k + 4*n for INT8.
    pub fn ppocr_rh_footprint_bytes(h: *const ppocr_rh_t) -> usize;
    pub fn ppocr_rh_device_bytes(h: *const ppocr_rh_t) -> usize;
    pub fn ppocr_rh_shape(h: *const ppocr_rh_t, n: *mut i64, k: *mut i64, quantized: *mut c_int) -> c_int;
    /// The mode PPOCR_MODE_AUTO runs for this head (no counterpart in the reference).
    pub fn ppocr_rh_auto_mode(h: *const ppocr_rh_t) -> c_int;
    /// Which rows take the rescue pass (no counterpart in the reference).
    pub fn ppocr_rh_guard_limits(h: *const ppocr_rh_t, mode: c_int, prec_limit: *mut f32,
                                 range_amax_limit: *mut f32, range_norm_limit: *mut f32) -> c_int;
    pub fn ppocr_rh_workspace_bytes(h: *const ppocr_rh_t, m: i64, mode: c_int) -> usize;

    // ---- MatMul.12: matmul_quantized_b (src/ops/matmul.rs:1204-1336) / matmul_transposed_b
    pub fn ppocr_rh_logits(h: *const ppocr_rh_t, a: *const f32, m: i64, mode: c_int, out: *mut f32) -> c_int;
    pub fn ppocr_rh_logits_dev(h: *const ppocr_rh_t, d_a: *const f32, m: i64, mode: c_int, d_out: *mut f32,
                               d_workspace: *mut c_void, workspace_bytes: usize, stream: *mut c_void) -> c_int;

    // ---- Softmax.2: softmax_inplace (src/ops/softmax.rs:199-285); find_argmax
    // (src/postprocess/ctc.rs:178-258)
    pub fn ppocr_softmax_rows(x: *mut f32, rows: i64, cols: i64) -> c_int;
    pub fn ppocr_softmax_rows_dev(d_x: *mut f32, rows: i64, cols: i64, d_idx: *mut i32, d_maxprob: *mut f32,
                                  stream: *mut c_void) -> c_int;
    pub fn ppocr_argmax_rows(x: *const f32, rows: i64, cols: i64, idx: *mut i32, val: *mut f32) -> c_int;
    pub fn ppocr_argmax_rows_dev(d_x: *const f32, rows: i64, cols: i64, d_idx: *mut i32, d_val: *mut f32,
                                 stream: *mut c_void) -> c_int;

    // ---- MatMul.12 -> Softmax.2 as one call (src/engine/model.rs:1245-1302)
    pub fn ppocr_rh_probs(h: *const ppocr_rh_t, a: *const f32, m: i64, mode: c_int, probs: *mut f32) -> c_int;
    pub fn ppocr_rh_probs_dev(h: *const ppocr_rh_t, d_a: *const f32, m: i64, mode: c_int, d_probs: *mut f32,
                              d_workspace: *mut c_void, workspace_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn ppocr_rh_argmax(h: *const ppocr_rh_t, a: *const f32, m: i64, mode: c_int, idx: *mut i32,
                           maxprob: *mut f32) -> c_int;
    pub fn ppocr_rh_argmax_dev(h: *const ppocr_rh_t, d_a: *const f32, m: i64, mode: c_int, d_idx: *mut i32,
                               d_maxprob: *mut f32, d_workspace: *mut c_void, workspace_bytes: usize,
                               stream: *mut c_void) -> c_int;

    // ---- CTC collapse and score: CtcDecoder::decode_batch (src/postprocess/ctc.rs:144-172)
    pub fn ppocr_ctc_greedy(idx: *const i32, maxprob: *const f32, line_off: *const i64, lines: i64, blank: i32,
                            seq: *mut i32, seq_len: *mut i64, score: *mut f32) -> c_int;
    pub fn ppocr_ctc_greedy_dev(d_idx: *const i32, d_maxprob: *const f32, d_line_off: *const i64, lines: i64,
                                blank: i32, d_seq: *mut i32, d_seq_len: *mut i64, d_score: *mut f32,
                                stream: *mut c_void) -> c_int;

    // ---- the whole head for a ragged batch of lines (recognize, src/pipeline.rs:395-436)
    pub fn ppocr_rh_decode(h: *const ppocr_rh_t, a: *const f32, line_off: *const i64, lines: i64, mode: c_int,
                           idx: *mut i32, maxprob: *mut f32, seq: *mut i32, seq_len: *mut i64,
                           score: *mut f32) -> c_int;
    pub fn ppocr_rh_decode_dev(h: *const ppocr_rh_t, d_a: *const f32, m: i64, d_line_off: *const i64, lines: i64,
                               mode: c_int, d_idx: *mut i32, d_maxprob: *mut f32, d_seq: *mut i32,
                               d_seq_len: *mut i64, d_score: *mut f32, d_workspace: *mut c_void,
                               workspace_bytes: usize, stream: *mut c_void) -> c_int;
    /// ppocr_rh_decode_dev without a workspace and without any allocation (no counterpart
    /// in the reference; for callers that cannot allocate).  32 MiB of scratch per GPU;
    /// calls that overlap on one GPU race.
    pub fn ppocr_rh_decode_dev_noalloc(h: *const ppocr_rh_t, d_a: *const f32, m: i64, d_line_off: *const i64,
                                       lines: i64, mode: c_int, d_idx: *mut i32, d_maxprob: *mut f32,
                                       d_seq: *mut i32, d_seq_len: *mut i64, d_score: *mut f32,
                                       stream: *mut c_void) -> c_int;

    // ---- the head entered at the neck's Transpose.8 (src/engine/model.rs:1325-1342):
    // x [lines][k][steps], channels first
    pub fn ppocr_rh_decode_nct(h: *const ppocr_rh_t, x: *const f32, lines: i64, steps: i64, mode: c_int,
                               idx: *mut i32, maxprob: *mut f32, seq: *mut i32, seq_len: *mut i64,
                               score: *mut f32) -> c_int;
    pub fn ppocr_rh_decode_nct_dev(h: *const ppocr_rh_t, d_x: *const f32, lines: i64, steps: i64, mode: c_int,
                                   d_idx: *mut i32, d_maxprob: *mut f32, d_seq: *mut i32, d_seq_len: *mut i64,
                                   d_score: *mut f32, d_workspace: *mut c_void, workspace_bytes: usize,
                                   stream: *mut c_void) -> c_int;

    // ---- the SVTR neck tail before the head (Model::forward's MatMul, LayerNorm, Softmax,
    // Sigmoid, Mul and Add nodes between Transpose.0 and Transpose.8, src/engine/model.rs)
    pub fn ppocr_rn_create(blocks: *const ppocr_rn_block_t, nblocks: c_int, lnf_w: *const f32, lnf_b: *const f32,
                           lnf_eps: f32, dim: i64, heads: i64, hidden: i64, scale: f32, device: c_int,
                           out: *mut *mut ppocr_rn_t) -> c_int;
    pub fn ppocr_rn_create_from_model(path: *const c_char, device: c_int, out: *mut *mut ppocr_rn_t) -> c_int;
    pub fn ppocr_rn_destroy(h: *mut ppocr_rn_t);
    pub fn ppocr_rn_shape(h: *const ppocr_rn_t, dim: *mut i64, heads: *mut i64, hidden: *mut i64,
                          blocks: *mut c_int) -> c_int;
    /// The tail's MatMul arithmetic: 1 fp16 halves, 0 fp32 (no counterpart in the reference).
    pub fn ppocr_rn_gemm_halves(h: *const ppocr_rn_t) -> c_int;
    pub fn ppocr_rn_workspace_bytes(h: *const ppocr_rn_t, m: i64) -> usize;
    pub fn ppocr_rn_forward_dev(h: *const ppocr_rn_t, d_x: *const f32, d_shortcut: *const f32, m: i64,
                                d_line_off: *const i64, lines: i64, layout: c_int, d_out: *mut f32,
                                d_workspace: *mut c_void, workspace_bytes: usize, stream: *mut c_void) -> c_int;
    pub fn ppocr_rn_forward(h: *const ppocr_rn_t, x: *const f32, shortcut: *const f32, line_off: *const i64,
                            lines: i64, layout: c_int, out: *mut f32) -> c_int;
    /// Measurement only (no counterpart in the reference): the forward with a HIP event
    /// recorded before the first kernel and after each one.
    pub fn ppocr_rn_forward_marked_dev(h: *const ppocr_rn_t, d_x: *const f32, d_shortcut: *const f32, m: i64,
                                       d_line_off: *const i64, lines: i64, layout: c_int, d_out: *mut f32,
                                       d_workspace: *mut c_void, workspace_bytes: usize, stream: *mut c_void,
                                       events: *const *mut c_void, nevents: c_int, names: *mut *const c_char,
                                       recorded: *mut c_int) -> c_int;
}
