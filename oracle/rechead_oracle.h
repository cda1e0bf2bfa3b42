/*
 * CPU oracle for the recognition-head hot path (INT8 packer, W8A32 projection,
 * FP32 transposed projection, 18710-way softmax, CTC greedy decode).
 *
 * TEST INFRASTRUCTURE, NOT PRODUCT CODE.  This library is a C restatement of the
 * reference's CPU kernels, written with the same AVX2/FMA intrinsic sequence and the
 * same scalar fallbacks, so that the HIP path can be checked against it.  Only the test
 * suite, the smoke check and the CPU-baseline leg of the benchmark load it.  The product
 * library never links, loads or calls it.
 *
 * Every function names the reference file:line it restates (paths relative to the
 * rust_ppocrv6 crate root).  How each function is pinned (closed forms, f64 brute
 * force, the reference's own known-answer tests) is listed in the test files that
 * exercise it; see tests/test_oracle_*.py.
 *
 * Numerics: compiled with -mavx2 -mfma -ffp-contract=off so that scalar code gains
 * no fused multiply-adds the Rust code does not have.  libm expf is called where the
 * reference calls f32::exp.
 */
#ifndef PPOCR_RECHEAD_ORACLE_H
#define PPOCR_RECHEAD_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* QuantizedWeight::from_f32_transposed, src/ops/matmul.rs:1173-1202 */
void orc_pack_int8(const float* w_t, int64_t n, int64_t k, int8_t* q, float* scales);

/* matmul_quantized_b, src/ops/matmul.rs:1204-1336 (AVX2 kernel 1338-1443, tail
 * columns 1473-1514, scalar 1445-1471).  `partition_threads` reproduces the rayon
 * column-chunk partition (<=1: serial row path).  `exec_threads` only sets how many
 * OpenMP threads execute it; results do not depend on it. */
void orc_matmul_quantized_b(const float* a, int64_t rows, const int8_t* q,
                            const float* scales, const float* bias, int64_t n, int64_t k,
                            int partition_threads, int use_avx2, int exec_threads,
                            float* out);

/* matmul_transposed_b, src/ops/matmul.rs:514-897 (tile 1000-1087, column kernel
 * 912-998, dot product 1118-1163, scalar 1096-1116). */
void orc_matmul_transposed_b(const float* a, int64_t rows, const float* w_t,
                             const float* bias, int64_t n, int64_t k,
                             int partition_threads, int use_avx2, int exec_threads,
                             float* out);

/* avx2_exp_ps, src/ops/softmax.rs:5-47, applied to `count` floats (count % 8 == 0). */
void orc_exp_ps(const float* x, int64_t count, float* out);

/* softmax_inplace over the last axis, src/ops/softmax.rs:199-285, rows computed by
 * compute_row_avx2 (313-416) or compute_row_scalar (418-436). */
void orc_softmax_rows(float* x, int64_t rows, int64_t n, int use_avx2, int exec_threads);

/* layer_norm over the last axis of x [rows][n] with weight and bias (both required),
 * src/ops/layernorm.rs:5-244: rows by compute_layer_norm_row_fma (146-244) with use_avx2,
 * compute_layer_norm_row (120-144) without. */
void orc_layer_norm_rows(const float* x, int64_t rows, int64_t n, const float* w, const float* b, float eps,
                         int use_avx2, float* out);

/* sigmoid_inplace, src/ops/activation.rs:31-94 (sigmoid_avx2_chunk: 16- then 8-wide
 * 1 / (1 + avx2_exp_ps(0 - x)), scalar tail 1 / (1 + expf(-x))), on `count` floats as one
 * chunk (the reference's 16384-float rayon chunks are multiples of 8, so only the tensor's
 * last count % 8 floats take the scalar tail either way). */
void orc_sigmoid(const float* x, int64_t count, float* out);

/* find_argmax, src/postprocess/ctc.rs:178-258.  Returns the index; *val gets the value. */
int64_t orc_find_argmax(const float* x, int64_t n, int use_avx2, float* val);

/* Argmax of every row of probs [rows][n] (CtcDecoder::decode_batch's per-step call,
 * src/postprocess/ctc.rs:151-154). */
void orc_argmax_rows(const float* probs, int64_t rows, int64_t n, int use_avx2,
                     int exec_threads, int32_t* idx, float* val);

/* Collapse and score of CtcDecoder::decode_batch, src/postprocess/ctc.rs:144-172,
 * applied to per-step (idx, val) with lines given by offsets line_off[lines+1].
 * Emitted indices of line i go to seq[line_off[i] ...]; seq_len[i] = count. */
void orc_ctc_collapse(const int32_t* idx, const float* val, const int64_t* line_off,
                      int64_t lines, int32_t blank, int32_t* seq, int64_t* seq_len,
                      float* score);

/* The whole head for a ragged batch of text lines the way the pipeline runs it for more
 * than one box (src/pipeline.rs:417-433): one line per worker, inner parallelism off,
 * so each line takes the serial row path of matmul_quantized_b, then softmax_inplace,
 * then the CTC decode.  probs_out may be NULL. */
void orc_rechead_lines(const float* a, const int64_t* line_off, int64_t lines,
                       const int8_t* q, const float* scales, const float* bias,
                       int64_t n, int64_t k, int use_avx2, int exec_threads,
                       int32_t* idx, float* maxprob, int32_t* seq, int64_t* seq_len,
                       float* score, float* probs_out);

#ifdef __cplusplus
}
#endif
#endif
