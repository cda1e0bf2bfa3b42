/*
 * ppocr_rechead.h — C ABI of the MI355X (gfx950) recognition-head library.
 *
 * This is the drop-in boundary for the recognition head of rust_ppocrv6: the INT8
 * packer, the vocabulary projection MatMul.12 (x[.., T, 120] @ W^T[18710, 120] + b),
 * the 18710-way Softmax.2 and the CTC greedy decode.  Each entry point names the
 * reference function it replaces (file:line in the rust_ppocrv6 crate).
 *
 * Conventions
 *  - Every function returning int returns PPOCR_OK (0) on success.  On failure it
 *    returns a PPOCR_ERR_* code and ppocr_last_error() (thread-local) holds a message
 *    "<op>: <msg>" in the form of OcrError::OperatorError { op, msg } (src/error.rs:4-27).
 *    Nothing aborts or panics across this boundary.
 *  - Host-pointer entry points copy inputs to the device, run, copy results back and
 *    synchronise, on device memory and a stream of their own taken from a process-wide
 *    pool (one per concurrent call, kept for the next call).  `_dev` entry points take device pointers and a HIP stream
 *    (hipStream_t passed as void*, NULL = the null stream), enqueue only, and never
 *    synchronise.
 *  - Matrices are row-major and contiguous.  m is the number of activation rows (B*T),
 *    k the inner dimension (120 for PP-OCRv6_small_rec), n the number of classes (18710).
 *  - A head handle is immutable after creation and may be shared by threads; calls that
 *    overlap on one handle are safe as long as each passes its own workspace (or uses the
 *    host-pointer entry points).
 */
#ifndef PPOCR_RECHEAD_H
#define PPOCR_RECHEAD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PPOCR_OK 0
#define PPOCR_ERR_INVALID_ARG 1 /* shape / argument error (OperatorError) */
#define PPOCR_ERR_DEVICE 2      /* HIP runtime error */
#define PPOCR_ERR_NO_MEMORY 3   /* device allocation failed */
#define PPOCR_ERR_MODEL 4       /* model file unreadable or malformed (ModelError / SafeTensorsError) */

/* How the projection's inner products are computed.  All modes accumulate in fp32 and
 * apply the per-class scale and bias in fp32 in the epilogue. */
typedef enum {
    PPOCR_MODE_FP32_FMA = 0, /* fp32 vector FMA over dequantised weights */
    PPOCR_MODE_BF16X1 = 1,   /* bf16 MFMA, activation rounded to 1 bf16 term */
    PPOCR_MODE_BF16X2 = 2,   /* bf16 MFMA, activation split into 2 bf16 terms */
    PPOCR_MODE_BF16X3 = 3,   /* bf16 MFMA, activation split into 3 bf16 terms; for an
                                FP32 head, a_hi*w_hi + a_hi*w_lo + a_lo*w_hi */
    PPOCR_MODE_F16X2 = 4,    /* fp16 MFMA, activation split into 2 fp16 terms (22 bits of
                                it; int8 weights are exact in fp16); for an FP32 head,
                                a_hi*w_hi + a_hi*w_lo + a_lo*w_hi with fp16 halves (weights
                                below 32768 in magnitude) */
    PPOCR_MODE_AUTO = 5      /* chosen per head from its weights: F16X2, unless the bf16
                                split's precision guard leaves rows of max|a| up to 32 on the
                                split path (then BF16X2, or BF16X3 for an FP32 head; also when
                                an FP32 head's weights do not fit fp16).  The recognition
                                model's activations at the head reach |a| ~ 10-30, which the
                                bf16 guard of typical heads sends to the rescue pass.
                                ppocr_rh_auto_mode tells which. */
} ppocr_mode_t;

typedef struct ppocr_rh ppocr_rh_t;

/* Message of the last failed call on this thread ("" if none). */
const char* ppocr_last_error(void);

/* ---------------------------------------------------------------- packer
 * Replaces QuantizedWeight::from_f32_transposed (src/ops/matmul.rs:1173-1202): per row j
 * of W^T[n][k], scale = max|w|/127 if max|w| > 1e-8 else 1.0, q = round_half_away(w *
 * (1/scale)) clamped to [-127, 127] (NaN -> 0).  Bit-exact with the reference. */
int ppocr_rh_pack_int8(const float* w_t, int64_t n, int64_t k, int8_t* q_out, float* scales_out);
int ppocr_rh_pack_int8_dev(const float* d_w_t, int64_t n, int64_t k, int8_t* d_q_out,
                           float* d_scales_out, void* stream);

/* ---------------------------------------------------------------- head handle
 * Replaces the resident head weight of Model: the INT8 entry built by
 * Model::quantize_matmul_weights (src/engine/model.rs:628-638, QuantizedWeight
 * src/ops/matmul.rs:1165-1171) or the FP32 transposed copy of the prepack
 * (src/engine/model.rs:565-605), plus the bias folded into MatMul.12
 * (src/engine/model.rs:141-166).  Weights are uploaded once and stay resident in HBM.
 * bias may be NULL (no bias).  device is a HIP device ordinal. */
int ppocr_rh_create(const int8_t* q, const float* scales, const float* bias, int64_t n,
                    int64_t k, int device, ppocr_rh_t** out);
int ppocr_rh_create_f32(const float* w_t, const float* bias, int64_t n, int64_t k, int device,
                        ppocr_rh_t** out);
/* Head straight from a model file: replaces load_safetensors_model
 * (src/engine/loader.rs:34-92) for the head's tensors, the prepack transpose
 * (src/engine/model.rs:565-605) and, with quantize != 0, Model::quantize_matmul_weights
 * (src/engine/model.rs:628-638).  The F32 weight `weight_name` is read as the model stores
 * it, [k][n] (the B operand of MatMul.12, e.g. linear_8.w_0 [120, 18710]); `bias_name`
 * (may be NULL) is the F32 bias [n] folded from the following Add.  The file is
 * memory-mapped and the weight copied to the device as stored; the transpose, the INT8
 * packing (bit-exact with ppocr_rh_pack_int8), the guard limits and the MFMA tile records
 * are computed on the device.  The handle equals the one ppocr_rh_create (quantize != 0)
 * or ppocr_rh_create_f32 (quantize == 0) makes from the transposed weight.  A missing or
 * malformed file or tensor returns PPOCR_ERR_MODEL. */
int ppocr_rh_create_from_safetensors(const char* path, const char* weight_name, const char* bias_name,
                                     int quantize, int device, ppocr_rh_t** out);
/* Finds the recognition head in a model file's graph (the "graph" entry of the
 * safetensors metadata, src/engine/loader.rs:48-60): the segment MatMul(x, W) ->
 * Add(bias) (optional) -> Softmax over the last axis -> graph output that the engine-level
 * fused hook replaces, with the reference's load-time rules: Identity nodes are aliases
 * (src/engine/model.rs:67-95), the bias is folded when the MatMul's output is used only by
 * an Add whose other input is a weight (src/engine/model.rs:96-166), Softmax's axis
 * defaults to -1 and is normalised by the input's rank (src/engine/model.rs:1286-1302); a
 * non-negative axis is accepted when it is the last one, the rank being traced back to a
 * Transpose (the PP-OCRv6 models' Softmax has axis 2 on [1, T, classes]).  Writes the weight's name (an F32
 * [k][n] tensor) and the bias's ("" when there is none) as NUL-terminated strings, and n
 * and k (may be NULL).  PPOCR_ERR_MODEL when the file has no graph or no such segment;
 * PPOCR_ERR_INVALID_ARG when a name does not fit its buffer. */
int ppocr_model_find_rec_head(const char* path, char* weight_name, size_t weight_cap, char* bias_name,
                              size_t bias_cap, int64_t* n, int64_t* k);
void ppocr_rh_destroy(ppocr_rh_t* h);

/* Bytes this weight contributes to Model::weight_footprint_bytes
 * (src/engine/model.rs:651-667): n*k + 4*n for an INT8 head (2,320,040 for the
 * 18710x120 head), 4*n*k for an FP32 transposed head.  The bias is not counted, as in
 * the reference. */
size_t ppocr_rh_footprint_bytes(const ppocr_rh_t* h);
/* Bytes of device memory the handle holds (packed weights, scales, bias, MFMA tiles). */
size_t ppocr_rh_device_bytes(const ppocr_rh_t* h);
/* n, k and whether the head is INT8 (1) or FP32 (0). */
int ppocr_rh_shape(const ppocr_rh_t* h, int64_t* n, int64_t* k, int* quantized);
/* The mode PPOCR_MODE_AUTO runs for this head (PPOCR_MODE_BF16X2, PPOCR_MODE_BF16X3 or
 * PPOCR_MODE_F16X2), -1 for a null handle.  No counterpart in the reference, whose CPU
 * kernels have one precision. */
int ppocr_rh_auto_mode(const ppocr_rh_t* h);
/* The precision guard of `mode` on this head: a row a goes to the rescue pass of argmax,
 * decode and probabilities when max|a| > *prec_limit, or when max|a| > *range_amax_limit
 * and ||a||_2 > *range_norm_limit (its logits not proven to lie within the range the
 * statistics pass's unshifted softmax sums allow); of logits when max|a| > *prec_limit.
 * INFINITY: no such limit in this mode.  No counterpart in the reference; for callers that
 * want to know how many rows of a batch take the slower path. */
int ppocr_rh_guard_limits(const ppocr_rh_t* h, int mode, float* prec_limit, float* range_amax_limit,
                          float* range_norm_limit);

/* Device workspace needed by the `_dev` entry points below for m rows (0 if none).  A
 * NULL workspace makes the call allocate one on its stream (stream-ordered) and free it
 * after use.  Calls that share one workspace must not overlap.  One workspace may serve
 * calls of any size in turn: its first 8 bytes hold the precision guard's list header,
 * which every guarded call leaves empty when it ends; what a new workspace holds there is
 * told apart by the call's epoch (zeroing a new workspace once makes that certain). */
size_t ppocr_rh_workspace_bytes(const ppocr_rh_t* h, int64_t m, int mode);

/* ---------------------------------------------------------------- MatMul.12
 * Replaces matmul_quantized_b (src/ops/matmul.rs:1204-1336) for an INT8 head and
 * matmul_transposed_b (src/ops/matmul.rs:514-897) for an FP32 head:
 * out[r][j] = (sum_k a[r][k] * w[j][k]) * scale[j] + bias[j], a [m][k] -> out [m][n].
 * The split modes carry a precision guard (the same in the probs/argmax/decode entry
 * points): in PPOCR_MODE_BF16X2 and PPOCR_MODE_F16X2, rows whose largest |a| exceeds a
 * limit set by the head's weights (the largest L2 norm of a dequantised class row; for
 * F16X2 also the fp16 range) are recomputed with three bf16 activation terms (INT8 head) or
 * in fp32 FMA (FP32 head, and PPOCR_MODE_BF16X3 on an FP32 head), so logits stay within
 * 1e-4 of the reference. */
int ppocr_rh_logits(const ppocr_rh_t* h, const float* a, int64_t m, int mode, float* out);
int ppocr_rh_logits_dev(const ppocr_rh_t* h, const float* d_a, int64_t m, int mode, float* d_out,
                        void* d_workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- Softmax.2
 * Replaces softmax_inplace(x, -1) (src/ops/softmax.rs:199-285) on rows [rows][cols]:
 * max, exp(x - max), sum, multiply by 1/sum (1 if the sum is 0).  The `_dev` variant can
 * also emit the first-index argmax of each probability row and its value (the per-step
 * find_argmax of CtcDecoder::decode_batch, src/postprocess/ctc.rs:151-154); d_idx and
 * d_maxprob may be NULL. */
int ppocr_softmax_rows(float* x, int64_t rows, int64_t cols);
int ppocr_softmax_rows_dev(float* d_x, int64_t rows, int64_t cols, int32_t* d_idx,
                           float* d_maxprob, void* stream);

/* find_argmax (src/postprocess/ctc.rs:178-258) of every row of x [rows][cols]: the first
 * index of the maximum (strict >, NaN never wins; (0, -inf) for an all-NaN row). */
int ppocr_argmax_rows(const float* x, int64_t rows, int64_t cols, int32_t* idx, float* val);
int ppocr_argmax_rows_dev(const float* d_x, int64_t rows, int64_t cols, int32_t* d_idx,
                          float* d_val, void* stream);

/* ---------------------------------------------------------------- MatMul.12 + Softmax.2
 * The graph segment MatMul.12 -> Softmax.2 -> output (src/engine/model.rs:1245-1302)
 * as one call.  _probs writes the softmax probabilities [m][n] (the graph output
 * fetch_name_0); the logits never round-trip through HBM.  _argmax writes only, per
 * row, the first-index argmax of the probabilities and the maximum probability
 * (= 1 / sum exp(l - max)), which is all CtcDecoder::decode_batch reads
 * (src/postprocess/ctc.rs:151-163). */
int ppocr_rh_probs(const ppocr_rh_t* h, const float* a, int64_t m, int mode, float* probs);
int ppocr_rh_probs_dev(const ppocr_rh_t* h, const float* d_a, int64_t m, int mode, float* d_probs,
                       void* d_workspace, size_t workspace_bytes, void* stream);
int ppocr_rh_argmax(const ppocr_rh_t* h, const float* a, int64_t m, int mode, int32_t* idx,
                    float* maxprob);
int ppocr_rh_argmax_dev(const ppocr_rh_t* h, const float* d_a, int64_t m, int mode, int32_t* d_idx,
                        float* d_maxprob, void* d_workspace, size_t workspace_bytes,
                        void* stream);

/* ---------------------------------------------------------------- CTC greedy
 * Replaces the collapse and score of CtcDecoder::decode_batch
 * (src/postprocess/ctc.rs:144-172) for `lines` text lines whose per-step argmax and max
 * probability are idx/maxprob [line_off[lines]] (line i = steps line_off[i] ..
 * line_off[i+1]).  A step is emitted when idx != blank and idx != the previous step's
 * idx (the previous index starts as blank, and is updated on blanks too).  Emitted
 * indices of line i are written to seq[line_off[i] ...], their count to seq_len[i] and
 * score[i] = (f32 sum of the emitted maxprob, in order) / count, 0 when none.  The
 * reference's blank is 0.  The host form rejects offsets that do not start at 0 or go
 * backwards; the `_dev` form reads them on the device and clamps them instead: every line
 * is cut to [0, line_off[lines]] (idx, maxprob and seq must hold line_off[lines] steps), and
 * a line whose end precedes its start is empty. */
int ppocr_ctc_greedy(const int32_t* idx, const float* maxprob, const int64_t* line_off,
                     int64_t lines, int32_t blank, int32_t* seq, int64_t* seq_len, float* score);
int ppocr_ctc_greedy_dev(const int32_t* d_idx, const float* d_maxprob, const int64_t* d_line_off,
                         int64_t lines, int32_t blank, int32_t* d_seq, int64_t* d_seq_len,
                         float* d_score, void* stream);

/* ---------------------------------------------------------------- whole head
 * recognize() for a ragged batch of text lines (src/pipeline.rs:395-436, one
 * Model::forward + CtcDecoder::decode per line): a [line_off[lines]][k] holds the lines'
 * activations back to back.  Runs the fused projection/softmax/argmax and the CTC
 * collapse; outputs as ppocr_rh_argmax and ppocr_ctc_greedy.  idx and maxprob may be
 * NULL. */
int ppocr_rh_decode(const ppocr_rh_t* h, const float* a, const int64_t* line_off, int64_t lines,
                    int mode, int32_t* idx, float* maxprob, int32_t* seq, int64_t* seq_len,
                    float* score);
/* The same on device pointers, enqueued on `stream` (the engine-level fused hook of the
 * recognition head, with the compact CTC entry: CtcDecoder::decode_batch,
 * src/postprocess/ctc.rs:144-172, on (argmax, max probability) rows).  m is the number of
 * activation rows, d_a [m][k]; d_line_off [lines + 1] is a device array with
 * d_line_off[lines] = m, read on the device (offsets are clamped into [0, m]; a line whose
 * end precedes its start is empty).  d_idx and d_maxprob may be NULL.  The workspace is the
 * one of ppocr_rh_argmax_dev (ppocr_rh_workspace_bytes(h, m, mode)).  The merge of the
 * vocabulary chunks and the CTC collapse run as one kernel. */
int ppocr_rh_decode_dev(const ppocr_rh_t* h, const float* d_a, int64_t m, const int64_t* d_line_off,
                        int64_t lines, int mode, int32_t* d_idx, float* d_maxprob, int32_t* d_seq,
                        int64_t* d_seq_len, float* d_score, void* d_workspace,
                        size_t workspace_bytes, void* stream);

/* ppocr_rh_decode_dev without a workspace and without any device allocation.  It has no
 * counterpart in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Scratch comes from a fixed 32 MiB device array per GPU, held until the process ends,
 * which covers m up to 245760 rows of the 18710-class head (PPOCR_ERR_INVALID_ARG beyond
 * what it holds).  The array is part of the library's code object: every GPU the library's
 * kernels are loaded on holds it, whether or not this entry is ever called, and
 * ppocr_rh_device_bytes does not count it.  All calls on one GPU share that array: calls that overlap on one GPU
 * (other streams, other threads) race and must be serialised by the caller.  The first
 * call on a device takes the array's address and clears its list header on `stream`. */
int ppocr_rh_decode_dev_noalloc(const ppocr_rh_t* h, const float* d_a, int64_t m, const int64_t* d_line_off,
                                int64_t lines, int mode, int32_t* d_idx, float* d_maxprob, int32_t* d_seq,
                                int64_t* d_seq_len, float* d_score, void* stream);

/* The whole head entered one node earlier, at the neck's Transpose.8 (perm [0,2,1]:
 * Model::forward's Transpose, src/engine/model.rs:1325-1342, x.into_permute then a
 * contiguous copy, src/tensor.rs:621-633): x [lines][k][steps] is the neck's output,
 * channels first, for `lines` text lines of `steps` time steps each.  The transpose is
 * folded into the head's activation loads (no transposed copy is made): the results are
 * those of ppocr_rh_decode for the lines x[b] transposed, line b being rows
 * b*steps .. b*steps + steps - 1 (idx, maxprob and seq in that row order).  The workspace
 * is ppocr_rh_workspace_bytes(h, lines * steps, mode). */
int ppocr_rh_decode_nct(const ppocr_rh_t* h, const float* x, int64_t lines, int64_t steps, int mode,
                        int32_t* idx, float* maxprob, int32_t* seq, int64_t* seq_len, float* score);
int ppocr_rh_decode_nct_dev(const ppocr_rh_t* h, const float* d_x, int64_t lines, int64_t steps,
                            int mode, int32_t* d_idx, float* d_maxprob, int32_t* d_seq,
                            int64_t* d_seq_len, float* d_score, void* d_workspace,
                            size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- the SVTR neck tail
 * The recognition model's mixing tail before the head, PP-OCRv6_small_rec's graph from
 * Transpose.0 (perm [0,2,1]) to Transpose.8: `blocks` transformer blocks over the T tokens
 * of each text line,
 *     x = x + proj(attention(LayerNorm1(x)))      LayerNorm, MatMul.0 + Add (qkv), Reshape
 *                                                 [0,-1,3,heads,dim/heads], Mul(scale),
 *                                                 MatMul(q, k^T), Softmax over the keys,
 *                                                 MatMul(p, v), MatMul.3 + Add
 *     x = x + fc2(swish(fc1(LayerNorm2(x))))      MatMul.4 + Add, Sigmoid and Mul, MatMul.5 + Add
 * then the final LayerNorm plus the convolution shortcut (Add.202), whose sum, as token
 * rows, is the input of the head's MatMul.12.  The reference runs these nodes one by one in
 * its executor (Model::forward, src/engine/model.rs: MatMul 1245-1272, LayerNorm 1274-1284
 * after the fusion of src/engine/model.rs:2143-2245, Softmax 1286-1302, Sigmoid 953-963;
 * src/ops/layernorm.rs:5-244, src/ops/matmul.rs:9-96, src/ops/softmax.rs:199-285,
 * src/ops/activation.rs:25-94).  All arithmetic is fp32.  The kernels are built for
 * dim = 120, 8 heads of 15 and hidden = 240 (PPOCR_ERR_INVALID_ARG otherwise). */
typedef struct ppocr_rn ppocr_rn_t;

/* Input and output layouts of the neck (per text line b with T_b steps, the lines packed
 * back to back, line b starting at token row t0_b). */
#define PPOCR_NECK_ROWS 0           /* token rows [m][dim] (the tensor after Transpose.0) */
#define PPOCR_NECK_CHANNELS_FIRST 1 /* line b as [dim][T_b] at dim * t0_b (the graph's
                                       [1, dim, T] flatten output and shortcut) */

/* One block's weights, host pointers, MatMul weights row-major [K][N] as the model stores
 * them: ln1 (w, b [dim], eps), qkv [dim][3 dim] + [3 dim], proj [dim][dim] + [dim],
 * ln2, fc1 [dim][hidden] + [hidden], fc2 [hidden][dim] + [dim]. */
typedef struct {
    const float* ln1_w;
    const float* ln1_b;
    float ln1_eps;
    const float* qkv_w;
    const float* qkv_b;
    const float* proj_w;
    const float* proj_b;
    const float* ln2_w;
    const float* ln2_b;
    float ln2_eps;
    const float* fc1_w;
    const float* fc1_b;
    const float* fc2_w;
    const float* fc2_b;
} ppocr_rn_block_t;

/* The neck's weights resident in HBM (Model keeps them in its weight map,
 * src/engine/loader.rs:34-92).  scale: the attention's Mul constant (finite; otherwise
 * PPOCR_ERR_INVALID_ARG). */
int ppocr_rn_create(const ppocr_rn_block_t* blocks, int nblocks, const float* lnf_w, const float* lnf_b,
                    float lnf_eps, int64_t dim, int64_t heads, int64_t hidden, float scale, int device,
                    ppocr_rn_t** out);
/* The neck of a model file: the transformer blocks, the final LayerNorm and the shortcut
 * Add found in its graph between Transpose.0 and the head (PPOCR_ERR_MODEL when the graph
 * has no such tail, e.g. PP-OCRv6_tiny_rec), weights uploaded from the file. */
int ppocr_rn_create_from_model(const char* path, int device, ppocr_rn_t** out);
void ppocr_rn_destroy(ppocr_rn_t* h);
/* dim, heads, hidden and the number of blocks. */
int ppocr_rn_shape(const ppocr_rn_t* h, int64_t* dim, int64_t* heads, int64_t* hidden, int* blocks);
/* No counterpart in the reference: the arithmetic of the tail's MatMuls, 1 when they run on
 * fp16 halves of both operands (three exact products summed in fp32, 22 bits of each
 * operand; chosen at creation when the weights bound every MatMul operand inside fp16's
 * range), 0 when on fp32 products; a negative status for a null handle. */
int ppocr_rn_gemm_halves(const ppocr_rn_t* h);
/* Device workspace of ppocr_rn_forward_dev for m token rows. */
size_t ppocr_rn_workspace_bytes(const ppocr_rn_t* h, int64_t m);
/* out [m][dim] token rows = the tail applied to x and shortcut (both in `layout`), lines
 * by d_line_off[0..lines] (read on the device, clamped into [0, m]; attention never mixes
 * tokens of different lines).  Rows of [0, m) that no line covers (offsets that leave gaps
 * or end before m) have no attention output, and their rows of out are undefined.
 * d_workspace: ppocr_rn_workspace_bytes(h, m) bytes, 16-byte aligned, or NULL
 * (stream-ordered scratch). */
int ppocr_rn_forward_dev(const ppocr_rn_t* h, const float* d_x, const float* d_shortcut, int64_t m,
                         const int64_t* d_line_off, int64_t lines, int layout, float* d_out, void* d_workspace,
                         size_t workspace_bytes, void* stream);
int ppocr_rn_forward(const ppocr_rn_t* h, const float* x, const float* shortcut, const int64_t* line_off,
                     int64_t lines, int layout, float* out);
/* No counterpart in the reference (measurement of the tail's kernels one by one):
 * ppocr_rn_forward_dev, with events[0] (hipEvent_t handles, created by the caller) recorded
 * on the stream before the first kernel and events[i] after the i-th; names[i] receives the
 * name of the kernel that ends at events[i] (static strings; "start" for events[0]) and
 * *recorded the number of events used.  PPOCR_ERR_INVALID_ARG when nevents is too small
 * (2 blocks in the row layout take 9). */
int ppocr_rn_forward_marked_dev(const ppocr_rn_t* h, const float* d_x, const float* d_shortcut, int64_t m,
                                const int64_t* d_line_off, int64_t lines, int layout, float* d_out,
                                void* d_workspace, size_t workspace_bytes, void* stream, void* const* events,
                                int nevents, const char** names, int* recorded);

#ifdef __cplusplus
}
#endif
#endif /* PPOCR_RECHEAD_H */
