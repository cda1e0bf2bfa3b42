/*
 * CPU oracle for the recognition-head hot path.  TEST INFRASTRUCTURE ONLY: only the
 * test suite, the smoke check and the CPU-baseline leg of the benchmark load this
 * library; the product library never does.  See rechead_oracle.h for the contract.
 *
 * Each function restates one reference function with the same intrinsic sequence, in
 * the same order, so that its floating-point results are those of the reference's
 * AVX2 (or scalar) path.  Citations are file:line in the rust_ppocrv6 crate.
 */
#include "rechead_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

/* Rust's `impl Sum for f32` folds from -0.0. */
#define RUST_SUM_START (-0.0f)

/* ------------------------------------------------------------------ helpers */

/* hsum256, src/ops/matmul.rs:899-910 (identical copy at src/ops/softmax.rs:300-311). */
static inline float hsum256(__m256 v) {
    __m128 hi128 = _mm256_extractf128_ps(v, 1);
    __m128 lo128 = _mm256_castps256_ps128(v);
    __m128 sum128 = _mm_add_ps(lo128, hi128);
    __m128 hi64 = _mm_movehl_ps(sum128, sum128);
    __m128 sum64 = _mm_add_ps(sum128, hi64);
    __m128 hi32 = _mm_shuffle_ps(sum64, sum64, 1);
    return _mm_cvtss_f32(_mm_add_ss(sum64, hi32));
}

/* hmax256, src/ops/softmax.rs:287-298. */
static inline float hmax256(__m256 v) {
    __m128 hi128 = _mm256_extractf128_ps(v, 1);
    __m128 lo128 = _mm256_castps256_ps128(v);
    __m128 max128 = _mm_max_ps(lo128, hi128);
    __m128 hi64 = _mm_movehl_ps(max128, max128);
    __m128 max64 = _mm_max_ps(max128, hi64);
    __m128 hi32 = _mm_shuffle_ps(max64, max64, 1);
    return _mm_cvtss_f32(_mm_max_ss(max64, hi32));
}

/* Rust `f32::clamp(x, lo, hi)`: NaN passes through. */
static inline float rust_clamp(float x, float lo, float hi) {
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return x;
}

/* Rust `x as i8` for a float already in [-127, 127] or NaN: saturating, NaN -> 0. */
static inline int8_t rust_as_i8(float x) {
    if (x != x) return 0;
    if (x <= -128.0f) return -128;
    if (x >= 127.0f) return 127;
    return (int8_t)x; /* truncation toward zero; x is integral here */
}

/* ------------------------------------------------------------------ packer (a2) */

/* QuantizedWeight::from_f32_transposed, src/ops/matmul.rs:1173-1202.
 *   max_abs = fold(0.0, f32::max) over |w|   (f32::max ignores NaN, as fmaxf does)
 *   scale   = max_abs > 1e-8 ? max_abs / 127 : 1.0
 *   q       = (w * (1/scale)).round().clamp(-127, 127) as i8   (round: half away from 0) */
void orc_pack_int8(const float* w_t, int64_t n, int64_t k, int8_t* q, float* scales) {
    for (int64_t j = 0; j < n; ++j) {
        const float* row = w_t + j * k;
        float max_abs = 0.0f;
        for (int64_t i = 0; i < k; ++i) max_abs = fmaxf(max_abs, fabsf(row[i]));
        float scale = (max_abs > 1e-8f) ? max_abs / 127.0f : 1.0f;
        float inv_scale = 1.0f / scale;
        scales[j] = scale;
        for (int64_t i = 0; i < k; ++i) {
            float v = row[i] * inv_scale;
            q[j * k + i] = rust_as_i8(rust_clamp(roundf(v), -127.0f, 127.0f));
        }
    }
}

/* ------------------------------------------------------------------ INT8 matmul (a5-a9) */

/* avx2_dot_product_w8, src/ops/matmul.rs:1473-1514: the leftover-column dot product. */
static float dot_w8_avx2(const float* a, const int8_t* w8, int64_t n) {
    int64_t i = 0;
    __m256 v0 = _mm256_setzero_ps();
    __m256 v1 = _mm256_setzero_ps();
    while (i + 16 <= n) {
        __m256 va0 = _mm256_loadu_ps(a + i);
        __m256 va1 = _mm256_loadu_ps(a + i + 8);
        __m128i b0 = _mm_loadl_epi64((const __m128i*)(w8 + i));
        __m256 bf0 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(b0));
        v0 = _mm256_fmadd_ps(va0, bf0, v0);
        __m128i b1 = _mm_loadl_epi64((const __m128i*)(w8 + i + 8));
        __m256 bf1 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(b1));
        v1 = _mm256_fmadd_ps(va1, bf1, v1);
        i += 16;
    }
    v0 = _mm256_add_ps(v0, v1);
    while (i + 8 <= n) {
        __m256 va = _mm256_loadu_ps(a + i);
        __m128i b = _mm_loadl_epi64((const __m128i*)(w8 + i));
        __m256 bf = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(b));
        v0 = _mm256_fmadd_ps(va, bf, v0);
        i += 8;
    }
    float sum = hsum256(v0);
    while (i < n) {
        sum += a[i] * (float)w8[i];
        ++i;
    }
    return sum;
}

/* compute_quantized_b_cols_avx2, src/ops/matmul.rs:1338-1443.  4-column groups from
 * col_start: per column an 8-lane FMA accumulator over k, hsum256, scalar k tail,
 * then `dot = sum * scale` and `out = dot + bias` (two roundings). */
static void q_cols_avx2(const float* a_row, const int8_t* w, const float* s,
                        const float* bias, float* out_chunk, int64_t col_start,
                        int64_t col_count, int64_t k) {
    int64_t c = 0;
    while (c + 4 <= col_count) {
        int64_t j0 = col_start + c;
        const int8_t* w0 = w + j0 * k;
        const int8_t* w1 = w0 + k;
        const int8_t* w2 = w1 + k;
        const int8_t* w3 = w2 + k;
        __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
        __m256 acc2 = _mm256_setzero_ps(), acc3 = _mm256_setzero_ps();
        int64_t i = 0;
        while (i + 8 <= k) {
            __m256 va = _mm256_loadu_ps(a_row + i);
            __m256 bf0 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i*)(w0 + i))));
            acc0 = _mm256_fmadd_ps(va, bf0, acc0);
            __m256 bf1 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i*)(w1 + i))));
            acc1 = _mm256_fmadd_ps(va, bf1, acc1);
            __m256 bf2 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i*)(w2 + i))));
            acc2 = _mm256_fmadd_ps(va, bf2, acc2);
            __m256 bf3 = _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i*)(w3 + i))));
            acc3 = _mm256_fmadd_ps(va, bf3, acc3);
            i += 8;
        }
        float sum0 = hsum256(acc0), sum1 = hsum256(acc1);
        float sum2 = hsum256(acc2), sum3 = hsum256(acc3);
        while (i < k) {
            float av = a_row[i];
            sum0 += av * (float)w0[i];
            sum1 += av * (float)w1[i];
            sum2 += av * (float)w2[i];
            sum3 += av * (float)w3[i];
            ++i;
        }
        float d0 = sum0 * s[j0], d1 = sum1 * s[j0 + 1];
        float d2 = sum2 * s[j0 + 2], d3 = sum3 * s[j0 + 3];
        if (bias) {
            out_chunk[c] = d0 + bias[j0];
            out_chunk[c + 1] = d1 + bias[j0 + 1];
            out_chunk[c + 2] = d2 + bias[j0 + 2];
            out_chunk[c + 3] = d3 + bias[j0 + 3];
        } else {
            out_chunk[c] = d0;
            out_chunk[c + 1] = d1;
            out_chunk[c + 2] = d2;
            out_chunk[c + 3] = d3;
        }
        c += 4;
    }
    while (c < col_count) {
        int64_t j = col_start + c;
        float dot = dot_w8_avx2(a_row, w + j * k, k) * s[j];
        out_chunk[c] = bias ? dot + bias[j] : dot;
        ++c;
    }
}

/* compute_quantized_b_cols_scalar, src/ops/matmul.rs:1445-1471. */
static void q_cols_scalar(const float* a_row, const int8_t* w, const float* s,
                          const float* bias, float* out_chunk, int64_t col_start,
                          int64_t col_count, int64_t k) {
    for (int64_t c = 0; c < col_count; ++c) {
        int64_t j = col_start + c;
        const int8_t* wc = w + j * k;
        float sum = RUST_SUM_START;
        for (int64_t i = 0; i < k; ++i) sum = sum + a_row[i] * (float)wc[i];
        float dot = sum * s[j];
        out_chunk[c] = bias ? dot + bias[j] : dot;
    }
}

static void q_cols(int use_avx2, const float* a_row, const int8_t* w, const float* s,
                   const float* bias, float* out_chunk, int64_t col_start,
                   int64_t col_count, int64_t k) {
    if (use_avx2)
        q_cols_avx2(a_row, w, s, bias, out_chunk, col_start, col_count, k);
    else
        q_cols_scalar(a_row, w, s, bias, out_chunk, col_start, col_count, k);
}

/* matmul_quantized_b partition, src/ops/matmul.rs:1297-1333:
 *   parallel allowed and n >= 512: column chunks of max(ceil(n/threads), 64) (<= n),
 *   each chunk over all rows; otherwise each row over all n columns. */
void orc_matmul_quantized_b(const float* a, int64_t rows, const int8_t* q,
                            const float* scales, const float* bias, int64_t n, int64_t k,
                            int partition_threads, int use_avx2, int exec_threads,
                            float* out) {
    if (exec_threads < 1) exec_threads = 1;
    int parallel = partition_threads > 1 && rows * n >= 512;
    if (parallel && n >= 512) {
        int64_t chunk = (n + partition_threads - 1) / partition_threads;
        if (chunk < 64) chunk = 64;
        if (chunk > n) chunk = n;
        int64_t num_chunks = (n + chunk - 1) / chunk;
#pragma omp parallel for num_threads(exec_threads) schedule(dynamic, 1)
        for (int64_t ci = 0; ci < num_chunks; ++ci) {
            int64_t c0 = ci * chunk;
            int64_t cnt = (n - c0) < chunk ? (n - c0) : chunk;
            for (int64_t r = 0; r < rows; ++r)
                q_cols(use_avx2, a + r * k, q, scales, bias, out + r * n + c0, c0, cnt, k);
        }
    } else {
#pragma omp parallel for num_threads(exec_threads) schedule(dynamic, 16)
        for (int64_t r = 0; r < rows; ++r)
            q_cols(use_avx2, a + r * k, q, scales, bias, out + r * n, 0, n, k);
    }
}

/* ------------------------------------------------------------------ FP32 matmul (a10) */

/* avx2_dot_product, src/ops/matmul.rs:1118-1163. */
static float dot_f32_avx2(const float* a, const float* b, int64_t n) {
    int64_t i = 0;
    __m256 v0 = _mm256_setzero_ps(), v1 = _mm256_setzero_ps();
    __m256 v2 = _mm256_setzero_ps(), v3 = _mm256_setzero_ps();
    while (i + 32 <= n) {
        v0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), v0);
        v1 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 8), _mm256_loadu_ps(b + i + 8), v1);
        v2 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 16), _mm256_loadu_ps(b + i + 16), v2);
        v3 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i + 24), _mm256_loadu_ps(b + i + 24), v3);
        i += 32;
    }
    v0 = _mm256_add_ps(_mm256_add_ps(v0, v1), _mm256_add_ps(v2, v3));
    while (i + 8 <= n) {
        v0 = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), v0);
        i += 8;
    }
    float sum = hsum256(v0);
    while (i < n) {
        sum += a[i] * b[i];
        ++i;
    }
    return sum;
}

/* compute_transposed_b_cols_avx2, src/ops/matmul.rs:912-998. */
static void t_cols_avx2(const float* a_row, const float* b, const float* bias,
                        float* out_chunk, int64_t col_start, int64_t col_count, int64_t k) {
    int64_t c = 0;
    while (c + 4 <= col_count) {
        int64_t j0 = col_start + c;
        const float* b0 = b + j0 * k;
        const float* b1 = b0 + k;
        const float* b2 = b1 + k;
        const float* b3 = b2 + k;
        __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
        __m256 acc2 = _mm256_setzero_ps(), acc3 = _mm256_setzero_ps();
        int64_t i = 0;
        while (i + 8 <= k) {
            __m256 va = _mm256_loadu_ps(a_row + i);
            acc0 = _mm256_fmadd_ps(va, _mm256_loadu_ps(b0 + i), acc0);
            acc1 = _mm256_fmadd_ps(va, _mm256_loadu_ps(b1 + i), acc1);
            acc2 = _mm256_fmadd_ps(va, _mm256_loadu_ps(b2 + i), acc2);
            acc3 = _mm256_fmadd_ps(va, _mm256_loadu_ps(b3 + i), acc3);
            i += 8;
        }
        float s0 = hsum256(acc0), s1 = hsum256(acc1), s2 = hsum256(acc2), s3 = hsum256(acc3);
        while (i < k) {
            float av = a_row[i];
            s0 += av * b0[i];
            s1 += av * b1[i];
            s2 += av * b2[i];
            s3 += av * b3[i];
            ++i;
        }
        if (bias) {
            out_chunk[c] = s0 + bias[j0];
            out_chunk[c + 1] = s1 + bias[j0 + 1];
            out_chunk[c + 2] = s2 + bias[j0 + 2];
            out_chunk[c + 3] = s3 + bias[j0 + 3];
        } else {
            out_chunk[c] = s0;
            out_chunk[c + 1] = s1;
            out_chunk[c + 2] = s2;
            out_chunk[c + 3] = s3;
        }
        c += 4;
    }
    while (c < col_count) {
        int64_t j = col_start + c;
        float dot = dot_f32_avx2(a_row, b + j * k, k);
        out_chunk[c] = bias ? dot + bias[j] : dot;
        ++c;
    }
}

/* compute_transposed_b_cols_scalar, src/ops/matmul.rs:1096-1116. */
static void t_cols_scalar(const float* a_row, const float* b, const float* bias,
                          float* out_chunk, int64_t col_start, int64_t col_count, int64_t k) {
    for (int64_t c = 0; c < col_count; ++c) {
        int64_t j = col_start + c;
        const float* bc = b + j * k;
        float sum = RUST_SUM_START;
        for (int64_t i = 0; i < k; ++i) sum = sum + a_row[i] * bc[i];
        out_chunk[c] = bias ? sum + bias[j] : sum;
    }
}

/* transposed_b_tile_fma::<1> for one row and 4 columns, src/ops/matmul.rs:1025-1087.
 * Rows of a tile are independent, so MR only changes which rows share a pass, never a
 * result: one row at a time gives the same bits as MR = 1, 2 or 3. */
static void t_tile_row(const float* a_row, const float* b, float* out, int64_t c,
                       const float* bias, int64_t k) {
    const float* b0 = b;
    const float* b1 = b + k;
    const float* b2 = b + 2 * k;
    const float* b3 = b + 3 * k;
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    __m256 acc2 = _mm256_setzero_ps(), acc3 = _mm256_setzero_ps();
    for (int64_t i = 0; i < k; i += 8) {
        __m256 bv0 = _mm256_loadu_ps(b0 + i), bv1 = _mm256_loadu_ps(b1 + i);
        __m256 bv2 = _mm256_loadu_ps(b2 + i), bv3 = _mm256_loadu_ps(b3 + i);
        __m256 av = _mm256_loadu_ps(a_row + i);
        acc0 = _mm256_fmadd_ps(av, bv0, acc0);
        acc1 = _mm256_fmadd_ps(av, bv1, acc1);
        acc2 = _mm256_fmadd_ps(av, bv2, acc2);
        acc3 = _mm256_fmadd_ps(av, bv3, acc3);
    }
    __m256 h01 = _mm256_hadd_ps(acc0, acc1);
    __m256 h23 = _mm256_hadd_ps(acc2, acc3);
    __m256 h0123 = _mm256_hadd_ps(h01, h23);
    __m128 lo = _mm256_castps256_ps128(h0123);
    __m128 hi = _mm256_extractf128_ps(h0123, 1);
    __m128 sums = _mm_add_ps(lo, hi);
    if (bias) sums = _mm_add_ps(sums, _mm_loadu_ps(bias + c));
    _mm_storeu_ps(out, sums);
}

/* matmul_transposed_b, src/ops/matmul.rs:514-897.  Three numerically distinct paths:
 *  - one output row and parallelism on: column chunks of clamp(n/threads, 1, 2048), each
 *    through compute_transposed_b_cols_avx2 (4-col hsum groups from the chunk start);
 *  - AVX2 and k % 8 == 0: the register-blocked tile for every 4-column group of
 *    0..n - n%4 (all partitions give the same groups) and avx2_dot_product for n % 4;
 *  - otherwise compute_transposed_b_cols_{avx2,scalar} over the whole row. */
void orc_matmul_transposed_b(const float* a, int64_t rows, const float* w_t,
                             const float* bias, int64_t n, int64_t k,
                             int partition_threads, int use_avx2, int exec_threads,
                             float* out) {
    if (exec_threads < 1) exec_threads = 1;
    if (rows == 1 && partition_threads > 1 && n >= 512) {
        int64_t chunk = n / partition_threads;
        if (chunk < 1) chunk = 1;
        if (chunk > 2048) chunk = 2048;
        int64_t num_chunks = (n + chunk - 1) / chunk;
#pragma omp parallel for num_threads(exec_threads) schedule(dynamic, 1)
        for (int64_t ci = 0; ci < num_chunks; ++ci) {
            int64_t c0 = ci * chunk;
            int64_t cnt = (n - c0) < chunk ? (n - c0) : chunk;
            if (use_avx2)
                t_cols_avx2(a, w_t, bias, out + c0, c0, cnt, k);
            else
                t_cols_scalar(a, w_t, bias, out + c0, c0, cnt, k);
        }
        return;
    }
    if (use_avx2 && k % 8 == 0 && rows > 0) {
        int64_t cols_full = n - n % 4;
#pragma omp parallel for num_threads(exec_threads) schedule(dynamic, 4)
        for (int64_t r = 0; r < rows; ++r) {
            const float* a_row = a + r * k;
            float* o = out + r * n;
            for (int64_t c = 0; c < cols_full; c += 4) t_tile_row(a_row, w_t + c * k, o + c, c, bias, k);
            if (cols_full < n) t_cols_avx2(a_row, w_t, bias, o + cols_full, cols_full, n - cols_full, k);
        }
        return;
    }
#pragma omp parallel for num_threads(exec_threads) schedule(dynamic, 4)
    for (int64_t r = 0; r < rows; ++r) {
        if (use_avx2)
            t_cols_avx2(a + r * k, w_t, bias, out + r * n, 0, n, k);
        else
            t_cols_scalar(a + r * k, w_t, bias, out + r * n, 0, n, k);
    }
}

/* ------------------------------------------------------------------ softmax (a12-a14) */

/* avx2_exp_ps, src/ops/softmax.rs:5-47: clamp, round(x*log2e) to nearest even,
 * Cody-Waite reduction with c1/c2, degree-6 Horner polynomial, times 2^fx built from
 * the exponent bits. */
static inline __m256 exp_ps_avx2(__m256 x) {
    x = _mm256_max_ps(x, _mm256_set1_ps(-87.336544f));
    x = _mm256_min_ps(x, _mm256_set1_ps(88.722839f));
    __m256 log2e = _mm256_set1_ps(1.4426950408889634f);
    __m256 fx = _mm256_round_ps(_mm256_mul_ps(x, log2e), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
    __m256 c1 = _mm256_set1_ps(0.693145751953125f);
    __m256 c2 = _mm256_set1_ps(1.42860682030941723212e-6f);
    __m256 g = _mm256_sub_ps(_mm256_sub_ps(x, _mm256_mul_ps(fx, c1)), _mm256_mul_ps(fx, c2));
    __m256 p6 = _mm256_set1_ps(1.3888889e-3f);
    __m256 p5 = _mm256_set1_ps(8.3333333e-3f);
    __m256 p4 = _mm256_set1_ps(4.1666668e-2f);
    __m256 p3 = _mm256_set1_ps(1.6666667e-1f);
    __m256 p2 = _mm256_set1_ps(0.5f);
    __m256 p1 = _mm256_set1_ps(1.0f);
    __m256 y = _mm256_fmadd_ps(p6, g, p5);
    y = _mm256_fmadd_ps(y, g, p4);
    y = _mm256_fmadd_ps(y, g, p3);
    y = _mm256_fmadd_ps(y, g, p2);
    y = _mm256_fmadd_ps(y, g, p1);
    y = _mm256_fmadd_ps(y, g, p1);
    __m256i emm0 = _mm256_cvtps_epi32(fx);
    emm0 = _mm256_add_epi32(emm0, _mm256_set1_epi32(127));
    emm0 = _mm256_slli_epi32(emm0, 23);
    __m256 pow2n = _mm256_castsi256_ps(emm0);
    return _mm256_mul_ps(y, pow2n);
}

void orc_exp_ps(const float* x, int64_t count, float* out) {
    for (int64_t i = 0; i + 8 <= count; i += 8) _mm256_storeu_ps(out + i, exp_ps_avx2(_mm256_loadu_ps(x + i)));
}

/* compute_row_avx2 with in == out (softmax_inplace), src/ops/softmax.rs:313-416. */
static void softmax_row_avx2(float* row, int64_t n) {
    float* in_ptr = row;
    float* out_ptr = row;
    __m256 vm0 = _mm256_set1_ps(-INFINITY), vm1 = _mm256_set1_ps(-INFINITY);
    __m256 vm2 = _mm256_set1_ps(-INFINITY), vm3 = _mm256_set1_ps(-INFINITY);
    int64_t i = 0;
    while (i + 32 <= n) {
        vm0 = _mm256_max_ps(vm0, _mm256_loadu_ps(in_ptr + i));
        vm1 = _mm256_max_ps(vm1, _mm256_loadu_ps(in_ptr + i + 8));
        vm2 = _mm256_max_ps(vm2, _mm256_loadu_ps(in_ptr + i + 16));
        vm3 = _mm256_max_ps(vm3, _mm256_loadu_ps(in_ptr + i + 24));
        i += 32;
    }
    __m256 v_max = _mm256_max_ps(_mm256_max_ps(vm0, vm1), _mm256_max_ps(vm2, vm3));
    while (i + 8 <= n) {
        v_max = _mm256_max_ps(v_max, _mm256_loadu_ps(in_ptr + i));
        i += 8;
    }
    float max_val = (i > 0) ? hmax256(v_max) : -INFINITY;
    while (i < n) {
        if (in_ptr[i] > max_val) max_val = in_ptr[i];
        ++i;
    }

    __m256 vmax = _mm256_set1_ps(max_val);
    __m256 s0 = _mm256_setzero_ps(), s1 = _mm256_setzero_ps();
    __m256 s2 = _mm256_setzero_ps(), s3 = _mm256_setzero_ps();
    i = 0;
    while (i + 32 <= n) {
        __m256 e0 = exp_ps_avx2(_mm256_sub_ps(_mm256_loadu_ps(in_ptr + i), vmax));
        __m256 e1 = exp_ps_avx2(_mm256_sub_ps(_mm256_loadu_ps(in_ptr + i + 8), vmax));
        __m256 e2 = exp_ps_avx2(_mm256_sub_ps(_mm256_loadu_ps(in_ptr + i + 16), vmax));
        __m256 e3 = exp_ps_avx2(_mm256_sub_ps(_mm256_loadu_ps(in_ptr + i + 24), vmax));
        _mm256_storeu_ps(out_ptr + i, e0);
        _mm256_storeu_ps(out_ptr + i + 8, e1);
        _mm256_storeu_ps(out_ptr + i + 16, e2);
        _mm256_storeu_ps(out_ptr + i + 24, e3);
        s0 = _mm256_add_ps(s0, e0);
        s1 = _mm256_add_ps(s1, e1);
        s2 = _mm256_add_ps(s2, e2);
        s3 = _mm256_add_ps(s3, e3);
        i += 32;
    }
    __m256 v_sum = _mm256_add_ps(_mm256_add_ps(s0, s1), _mm256_add_ps(s2, s3));
    while (i + 8 <= n) {
        __m256 e = exp_ps_avx2(_mm256_sub_ps(_mm256_loadu_ps(in_ptr + i), vmax));
        _mm256_storeu_ps(out_ptr + i, e);
        v_sum = _mm256_add_ps(v_sum, e);
        i += 8;
    }
    float sum_exp = (i > 0) ? hsum256(v_sum) : 0.0f;
    while (i < n) {
        float e = expf(in_ptr[i] - max_val);
        out_ptr[i] = e;
        sum_exp += e;
        ++i;
    }

    float inv_sum = (sum_exp > 0.0f) ? 1.0f / sum_exp : 1.0f;
    __m256 v_inv = _mm256_set1_ps(inv_sum);
    i = 0;
    while (i + 32 <= n) {
        __m256 a0 = _mm256_loadu_ps(out_ptr + i), a1 = _mm256_loadu_ps(out_ptr + i + 8);
        __m256 a2 = _mm256_loadu_ps(out_ptr + i + 16), a3 = _mm256_loadu_ps(out_ptr + i + 24);
        _mm256_storeu_ps(out_ptr + i, _mm256_mul_ps(a0, v_inv));
        _mm256_storeu_ps(out_ptr + i + 8, _mm256_mul_ps(a1, v_inv));
        _mm256_storeu_ps(out_ptr + i + 16, _mm256_mul_ps(a2, v_inv));
        _mm256_storeu_ps(out_ptr + i + 24, _mm256_mul_ps(a3, v_inv));
        i += 32;
    }
    while (i + 8 <= n) {
        _mm256_storeu_ps(out_ptr + i, _mm256_mul_ps(_mm256_loadu_ps(out_ptr + i), v_inv));
        i += 8;
    }
    while (i < n) {
        out_ptr[i] *= inv_sum;
        ++i;
    }
}

/* compute_row_scalar, src/ops/softmax.rs:418-436. */
static void softmax_row_scalar(float* row, int64_t n) {
    float max_val = -INFINITY;
    for (int64_t i = 0; i < n; ++i)
        if (row[i] > max_val) max_val = row[i];
    float sum_exp = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
        float e = expf(row[i] - max_val);
        row[i] = e;
        sum_exp += e;
    }
    float inv_sum = (sum_exp > 0.0f) ? 1.0f / sum_exp : 1.0f;
    for (int64_t i = 0; i < n; ++i) row[i] *= inv_sum;
}

/* softmax_inplace over contiguous rows, src/ops/softmax.rs:199-285 (an empty tensor is a
 * no-op, 226-229). */
/* compute_layer_norm_row_fma, src/ops/layernorm.rs:146-244: 8-lane sums of x, the lanes
 * added in order, the scalar tail; the same for fma(d, d, .) of the differences; inv_std =
 * 1 / sqrt(var + eps); out = fma((x - mean) * inv_std, w, b) in 8-wide steps, scalar tail
 * ((x - mean) * inv_std) * w + b. */
static void layer_norm_row_avx2(const float* x, int64_t n, const float* w, const float* b, float eps, float* out) {
    __m256 vs = _mm256_setzero_ps();
    int64_t i = 0;
    for (; i + 8 <= n; i += 8) vs = _mm256_add_ps(vs, _mm256_loadu_ps(x + i));
    float buf[8];
    _mm256_storeu_ps(buf, vs);
    float sum = 0.0f;
    for (int l = 0; l < 8; ++l) sum += buf[l];
    for (; i < n; ++i) sum += x[i];
    const float mean = sum / (float)n;
    const __m256 vm = _mm256_set1_ps(mean);
    __m256 vv = _mm256_setzero_ps();
    for (i = 0; i + 8 <= n; i += 8) {
        const __m256 d = _mm256_sub_ps(_mm256_loadu_ps(x + i), vm);
        vv = _mm256_fmadd_ps(d, d, vv);
    }
    _mm256_storeu_ps(buf, vv);
    float vsum = 0.0f;
    for (int l = 0; l < 8; ++l) vsum += buf[l];
    for (; i < n; ++i) {
        const float d = x[i] - mean;
        vsum += d * d;
    }
    const float var = vsum / (float)n;
    const float inv_std = 1.0f / sqrtf(var + eps);
    const __m256 vi = _mm256_set1_ps(inv_std);
    for (i = 0; i + 8 <= n; i += 8) {
        const __m256 v = _mm256_mul_ps(_mm256_sub_ps(_mm256_loadu_ps(x + i), vm), vi);
        _mm256_storeu_ps(out + i, _mm256_fmadd_ps(v, _mm256_loadu_ps(w + i), _mm256_loadu_ps(b + i)));
    }
    for (; i < n; ++i) {
        float v = (x[i] - mean) * inv_std;
        v *= w[i];
        v += b[i];
        out[i] = v;
    }
}

/* compute_layer_norm_row, src/ops/layernorm.rs:120-144: iterator sums (sequential). */
static void layer_norm_row_scalar(const float* x, int64_t n, const float* w, const float* b, float eps, float* out) {
    float sum = 0.0f;
    for (int64_t i = 0; i < n; ++i) sum += x[i];
    const float mean = sum / (float)n;
    float vs = 0.0f;
    for (int64_t i = 0; i < n; ++i) vs += (x[i] - mean) * (x[i] - mean);
    const float var = vs / (float)n;
    const float inv_std = 1.0f / sqrtf(var + eps);
    for (int64_t i = 0; i < n; ++i) {
        float v = (x[i] - mean) * inv_std;
        v *= w[i];
        v += b[i];
        out[i] = v;
    }
}

void orc_layer_norm_rows(const float* x, int64_t rows, int64_t n, const float* w, const float* b, float eps,
                         int use_avx2, float* out) {
    for (int64_t r = 0; r < rows; ++r) {
        if (use_avx2) layer_norm_row_avx2(x + r * n, n, w, b, eps, out + r * n);
        else layer_norm_row_scalar(x + r * n, n, w, b, eps, out + r * n);
    }
}

void orc_sigmoid(const float* x, int64_t count, float* out) {
    const __m256 zero = _mm256_setzero_ps(), one = _mm256_set1_ps(1.0f);
    int64_t i = 0;
    for (; i + 8 <= count; i += 8) {
        const __m256 e = exp_ps_avx2(_mm256_sub_ps(zero, _mm256_loadu_ps(x + i)));
        _mm256_storeu_ps(out + i, _mm256_div_ps(one, _mm256_add_ps(one, e)));
    }
    for (; i < count; ++i) out[i] = 1.0f / (1.0f + expf(-x[i]));
}

void orc_softmax_rows(float* x, int64_t rows, int64_t n, int use_avx2, int exec_threads) {
    if (rows <= 0 || n <= 0) return;
    if (exec_threads < 1) exec_threads = 1;
#pragma omp parallel for num_threads(exec_threads) schedule(dynamic, 4)
    for (int64_t r = 0; r < rows; ++r) {
        if (use_avx2)
            softmax_row_avx2(x + r * n, n);
        else
            softmax_row_scalar(x + r * n, n);
    }
}

/* ------------------------------------------------------------------ CTC (a15-a17) */

/* find_argmax_scalar, src/postprocess/ctc.rs:187-197: strict `>`, first occurrence. */
static int64_t argmax_scalar(const float* x, int64_t n, float* val) {
    int64_t best_i = 0;
    float best = -INFINITY;
    for (int64_t i = 0; i < n; ++i)
        if (x[i] > best) {
            best = x[i];
            best_i = i;
        }
    *val = best;
    return best_i;
}

/* find_argmax_avx2, src/postprocess/ctc.rs:199-258: per-lane strict GT_OQ blend, lowest
 * index among equal lane maxima, then a strict scalar tail. */
static int64_t argmax_avx2(const float* x, int64_t n, float* val) {
    __m256 v_max = _mm256_set1_ps(-INFINITY);
    __m256i v_idx = _mm256_setzero_si256();
    __m256i cur = _mm256_set_epi32(7, 6, 5, 4, 3, 2, 1, 0);
    __m256i step = _mm256_set1_epi32(8);
    int64_t i = 0;
    while (i + 8 <= n) {
        __m256 v = _mm256_loadu_ps(x + i);
        __m256 cmp = _mm256_cmp_ps(v, v_max, _CMP_GT_OQ);
        v_max = _mm256_blendv_ps(v_max, v, cmp);
        v_idx = _mm256_castps_si256(
            _mm256_blendv_ps(_mm256_castsi256_ps(v_idx), _mm256_castsi256_ps(cur), cmp));
        cur = _mm256_add_epi32(cur, step);
        i += 8;
    }
    float mb[8];
    int32_t ib[8];
    _mm256_storeu_ps(mb, v_max);
    _mm256_storeu_si256((__m256i*)ib, v_idx);
    float best = mb[0];
    int64_t best_i = ib[0];
    for (int lane = 1; lane < 8; ++lane) {
        float v = mb[lane];
        int64_t id = ib[lane];
        if (v > best) {
            best = v;
            best_i = id;
        } else if (v == best && id < best_i) {
            best_i = id;
        }
    }
    while (i < n) {
        if (x[i] > best) {
            best = x[i];
            best_i = i;
        }
        ++i;
    }
    *val = best;
    return best_i;
}

/* find_argmax dispatch, src/postprocess/ctc.rs:178-185. */
int64_t orc_find_argmax(const float* x, int64_t n, int use_avx2, float* val) {
    if (n <= 0) {
        *val = -INFINITY;
        return 0;
    }
    if (use_avx2 && n >= 16) return argmax_avx2(x, n, val);
    return argmax_scalar(x, n, val);
}

void orc_argmax_rows(const float* probs, int64_t rows, int64_t n, int use_avx2,
                     int exec_threads, int32_t* idx, float* val) {
    if (exec_threads < 1) exec_threads = 1;
#pragma omp parallel for num_threads(exec_threads) schedule(static)
    for (int64_t r = 0; r < rows; ++r) idx[r] = (int32_t)orc_find_argmax(probs + r * n, n, use_avx2, &val[r]);
}

/* decode_batch collapse and score, src/postprocess/ctc.rs:144-172: emit idx when
 * idx != blank and idx != last, last = idx every step (starting from blank); score is the
 * f32 sum of emitted values divided by their count (0 when none). */
void orc_ctc_collapse(const int32_t* idx, const float* val, const int64_t* line_off,
                      int64_t lines, int32_t blank, int32_t* seq, int64_t* seq_len,
                      float* score) {
    for (int64_t b = 0; b < lines; ++b) {
        int64_t t0 = line_off[b], t1 = line_off[b + 1];
        int32_t last = blank;
        int64_t cnt = 0;
        float sum = RUST_SUM_START;
        for (int64_t t = t0; t < t1; ++t) {
            int32_t id = idx[t];
            if (id != blank && id != last) {
                seq[t0 + cnt] = id;
                ++cnt;
                sum = sum + val[t];
            }
            last = id;
        }
        seq_len[b] = cnt;
        score[b] = cnt ? sum / (float)cnt : 0.0f;
    }
}

/* ------------------------------------------------------------------ whole head, per line */

void orc_rechead_lines(const float* a, const int64_t* line_off, int64_t lines,
                       const int8_t* q, const float* scales, const float* bias,
                       int64_t n, int64_t k, int use_avx2, int exec_threads,
                       int32_t* idx, float* maxprob, int32_t* seq, int64_t* seq_len,
                       float* score, float* probs_out) {
    if (exec_threads < 1) exec_threads = 1;
    int64_t tmax = 0;
    for (int64_t b = 0; b < lines; ++b)
        if (line_off[b + 1] - line_off[b] > tmax) tmax = line_off[b + 1] - line_off[b];
#pragma omp parallel num_threads(exec_threads)
    {
        float* buf = (float*)malloc(sizeof(float) * (size_t)(tmax > 0 ? tmax : 1) * (size_t)n);
#pragma omp for schedule(dynamic, 1)
        for (int64_t b = 0; b < lines; ++b) {
            int64_t t0 = line_off[b], T = line_off[b + 1] - line_off[b];
            /* inner parallelism is off on a line worker: serial row path */
            for (int64_t r = 0; r < T; ++r)
                q_cols(use_avx2, a + (t0 + r) * k, q, scales, bias, buf + r * n, 0, n, k);
            for (int64_t r = 0; r < T; ++r) {
                if (use_avx2)
                    softmax_row_avx2(buf + r * n, n);
                else
                    softmax_row_scalar(buf + r * n, n);
                idx[t0 + r] = (int32_t)orc_find_argmax(buf + r * n, n, use_avx2, &maxprob[t0 + r]);
            }
            if (probs_out) memcpy(probs_out + t0 * n, buf, sizeof(float) * (size_t)(T * n));
        }
        free(buf);
    }
    orc_ctc_collapse(idx, maxprob, line_off, lines, 0, seq, seq_len, score);
}
