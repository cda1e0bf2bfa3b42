// fp32 vector-FMA kernels of MatMul.12: the accuracy anchor for the MFMA kernels.
// Same contraction as compute_quantized_b_cols_avx2 (src/ops/matmul.rs:1338-1443) and
// transposed_b_tile_fma (src/ops/matmul.rs:1025-1087): fp32 products of the activation
// and the (exactly dequantised) weight, fp32 accumulation, then (sum * scale) + bias.
// Register tile: every thread owns 8 rows x 8 classes of a 128 x 128 block (classes
// 4 tn .. + 3 and 64 + 4 tn .. + 3, so each k step is four 16-byte LDS reads for 64 FMAs); k
// is staged through LDS in chunks of 32.
#include <algorithm>

#include "kernels.hpp"

namespace ppocr {

namespace {
constexpr int BM = kFmaRowsPerBlock, BN = kFmaCols, KC = 32;
constexpr int64_t kFmaRescueSlots = 128;  // row-block slots of a gather-mode (rescue) launch
constexpr int AST = BM + 4;  // LDS row strides (floats); +4 keeps 16-byte alignment
constexpr int WST = BN + 4;
static_assert(BM == 128 && BN == 128 && KC == 32, "the thread mappings below");


// Rows of a block: contiguous rows m0 .. m0 + BM - 1, or (GATHER) entries of the precision
// guard's row list of another kernel's pass (checked, not trusted: an entry outside [0, m)
// is skipped).  cpc: classes per vocabulary chunk; chunk c covers [c * cpc, (c + 1) * cpc).
struct FmaRows {
    const int* list;  // null: contiguous rows
    int count;
    __device__ __forceinline__ int64_t row(int64_t j, int64_t m, bool& valid) const {
        if (list) {
            const int64_t r = j < count ? (int64_t)list[j] : -1;
            valid = r >= 0 && r < m;
            return valid ? r : 0;
        }
        valid = j < m;
        return j;
    }
};

template <int EPI, bool GATHER>
__global__ __launch_bounds__(256) void head_fma_kernel(
    const int8_t* __restrict__ q, const float* __restrict__ w, const float* __restrict__ scale,
    const float* __restrict__ bias, const float* __restrict__ a, int64_t m, int n, int k, int cpc,
    float* __restrict__ out, const float* __restrict__ row_max, const float* __restrict__ row_inv,
    Partial* __restrict__ part, int64_t line_len,
    const unsigned long long* __restrict__ guard_header, const int* __restrict__ guard_rows, unsigned guard_epoch,
    int guard_cap) {
    __shared__ __align__(16) float As[KC * AST];  // [k][row]
    __shared__ __align__(16) float Ws[KC * WST];  // [k][class]
    __shared__ int64_t s_row[BM];                 // the block's rows (-1: none), read by the staging

    const int tid = threadIdx.x, tm = tid >> 4, tn = tid & 15;
    const int chunk = blockIdx.x;
    const int c0 = chunk * cpc;
    const int c1 = min(c0 + cpc, n);
    FmaRows src{nullptr, 0};
    if constexpr (GATHER) {
        const unsigned long long hv = *guard_header;
        const unsigned c = (unsigned)(hv >> 32) == guard_epoch ? (unsigned)hv : 0u;
        src = FmaRows{guard_rows, c < (unsigned)guard_cap ? (int)c : guard_cap};
    }
    const int64_t nrows = GATHER ? (int64_t)src.count : m;
    // class j of this thread within a tile: 4 tn + j (j < 4), 64 + 4 tn + j - 4 (j >= 4), in
    // increasing class order
    auto cls = [&](int j) { return (j < 4 ? 0 : 64 - 4) + 4 * tn + j; };

    for (int64_t m0 = (int64_t)blockIdx.y * BM; m0 < nrows; m0 += (int64_t)gridDim.y * BM) {
        // this thread's 8 rows (local slots 8 * tm .. 8 * tm + 7 of the block)
        int64_t rows[8];
        bool rvalid[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) rows[r] = src.row(m0 + 8 * tm + r, m, rvalid[r]);
        __syncthreads();  // the previous block's staging is done with the table
        if (tid < BM) {
            bool v;
            const int64_t r = src.row(m0 + tid, m, v);
            s_row[tid] = v ? r : -1;
        }

        RowStat st[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) st[r] = RowStat{-INFINITY, 0.0f, 0.0f, 0};
        bool refzero = true;
        float rmax[8], rinv[8];
        if (EPI == EPI_PROBS) {
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                rmax[r] = rvalid[r] ? row_max[rows[r]] : 0.0f;
                rinv[r] = rvalid[r] ? row_inv[rows[r]] : 0.0f;
            }
        }

        for (int n0 = c0; n0 < c1; n0 += BN) {
            float acc[8][8];
#pragma unroll
            for (int r = 0; r < 8; ++r)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[r][j] = 0.0f;
            // this thread's eight columns' constants, loaded once per tile of classes
            float csc[8], cbi[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int col = n0 + cls(j);
                csc[j] = col < c1 ? scale[col] : 0.0f;
                cbi[j] = col < c1 ? bias[col] : 0.0f;
            }

            for (int k0 = 0; k0 < k; k0 += KC) {
                // stage the chunk.  Rows layout: thread tid takes k0 + tid % 32 of rows
                // tid / 32 + 8 it (classes likewise); channels-first [lines][k][line_len]:
                // neighbouring threads take neighbouring steps (row tid % 128 at k0 + tid / 128
                // + 2 it).  Past the rows, classes or k: zeros.
                constexpr int IT = BM * KC / 256;
                __syncthreads();  // the previous chunk's readers are done
#pragma unroll 4
                for (int it = 0; it < IT; ++it) {
                    const int mm = line_len > 0 ? (tid & (BM - 1)) : (tid >> 5) + 8 * it;
                    const int kk = line_len > 0 ? (tid >> 7) + 2 * it : (tid & 31);
                    const int64_t row = s_row[mm];
                    float v = 0.0f;
                    if (row >= 0 && k0 + kk < k) {
                        if (line_len > 0) {
                            const int64_t line = row / line_len;
                            v = a[(line * k + k0 + kk) * line_len + (row - line * line_len)];
                        } else {
                            v = a[row * k + k0 + kk];
                        }
                    }
                    As[kk * AST + mm] = v;
                }
#pragma unroll 4
                for (int it = 0; it < IT; ++it) {
                    const int nn = (tid >> 5) + 8 * it, kk = tid & 31;
                    float v = 0.0f;
                    if (n0 + nn < c1 && k0 + kk < k) {
                        const int64_t e = (int64_t)(n0 + nn) * k + k0 + kk;
                        v = q ? (float)q[e] : w[e];
                    }
                    Ws[kk * WST + nn] = v;
                }
                __syncthreads();
                const int kend = min(KC, k - k0);
                for (int kk = 0; kk < kend; ++kk) {
                    const f32x4 a0 = *reinterpret_cast<const f32x4*>(&As[kk * AST + 8 * tm]);
                    const f32x4 a1 = *reinterpret_cast<const f32x4*>(&As[kk * AST + 8 * tm + 4]);
                    const f32x4 w0 = *reinterpret_cast<const f32x4*>(&Ws[kk * WST + 4 * tn]);
                    const f32x4 w1 = *reinterpret_cast<const f32x4*>(&Ws[kk * WST + 64 + 4 * tn]);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            acc[r][j] = fmaf(a0[r], w0[j], acc[r][j]);
                            acc[r + 4][j] = fmaf(a1[r], w0[j], acc[r + 4][j]);
                            acc[r][j + 4] = fmaf(a0[r], w1[j], acc[r][j + 4]);
                            acc[r + 4][j + 4] = fmaf(a1[r], w1[j], acc[r + 4][j + 4]);
                        }
                    }
                }
            }

            if (EPI == EPI_STATS) {
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    float tv[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        tv[j] = n0 + cls(j) < c1 ? fmaf(acc[r][j], csc[j] * kLog2e, cbi[j] * kLog2e) : -INFINITY;
                    const float tmax = fmaxf(fmaxf(fmaxf(tv[0], tv[1]), fmaxf(tv[2], tv[3])),
                                             fmaxf(fmaxf(tv[4], tv[5]), fmaxf(tv[6], tv[7])));
                    const bool better = tmax > st[r].best;
                    if (better) {
                        // the first of this thread's columns (in class order) holding the maximum
                        int jj = 7;
#pragma unroll
                        for (int j = 6; j >= 0; --j) jj = (tv[j] == tmax) ? j : jj;
                        st[r].best = tmax;
                        st[r].idx = n0 + cls(jj);
                    }
                    const bool shift = st[r].best != -INFINITY &&
                                       (st[r].best > st[r].ref + 64.0f || st[r].best < st[r].ref - 64.0f);
                    if (__any(shift)) {
                        if (shift) {
                            const float nr = st[r].best;
                            st[r].sum *= __builtin_amdgcn_exp2f(st[r].ref - nr);
                            st[r].ref = nr;
                        }
                        refzero = false;
                    }
                    float e = 0.0f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) e += __builtin_amdgcn_exp2f(refzero ? tv[j] : tv[j] - st[r].ref);
                    st[r].sum += e;
                }
            } else {
                auto value = [&](int r, int j) {
                    if (EPI == EPI_LOGITS) return __fadd_rn(__fmul_rn(acc[r][j], csc[j]), cbi[j]);
                    return __builtin_amdgcn_exp2f(fmaf(acc[r][j], csc[j] * kLog2e, cbi[j] * kLog2e) - rmax[r]) *
                           rinv[r];
                };
                bool all = n0 + BN <= c1;
#pragma unroll
                for (int r = 0; r < 8; ++r) all = all && rvalid[r];
                if (all) {
                    // no branch per value: at a branch the compiler waits for every store in
                    // flight
#pragma unroll
                    for (int r = 0; r < 8; ++r)
#pragma unroll
                        for (int j = 0; j < 8; ++j) out[rows[r] * n + n0 + cls(j)] = value(r, j);
                } else {
#pragma unroll
                    for (int r = 0; r < 8; ++r) {
                        if (!rvalid[r]) continue;
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            if (n0 + cls(j) < c1) out[rows[r] * n + n0 + cls(j)] = value(r, j);
                    }
                }
            }
        }

        if (EPI == EPI_STATS) {
            // the 16 threads of one tm are 16 consecutive lanes: butterfly over them (ties keep
            // the lower class).
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                RowStat s = st[r];
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) {
                    RowStat other;
                    other.best = __shfl_xor(s.best, o, 64);
                    other.sum = __shfl_xor(s.sum, o, 64);
                    other.ref = __shfl_xor(s.ref, o, 64);
                    other.idx = __shfl_xor(s.idx, o, 64);
                    s = stat_merge(s, other);
                }
                if (tn == 0 && rvalid[r]) {
                    part[(int64_t)chunk * m + rows[r]] = Partial{s.best, s.sum, s.idx};
                }
            }
        }
    }
}

int check_fma_args(int64_t m, int64_t n, int64_t k) {
    if (n > 0x7fffffff - BN || k > 0x7fffffff) return fail(PPOCR_ERR_INVALID_ARG, "MatMulQuantizedB: shape too large");
    if ((m + BM - 1) / BM > 65535) return fail(PPOCR_ERR_INVALID_ARG, "MatMulQuantizedB: m too large for the fp32 path");
    return PPOCR_OK;
}
}  // namespace

int launch_logits_fma(const int8_t* q, const float* w, const float* scale, const float* bias,
                      const float* a, int64_t m, int64_t n, int64_t k, float* out, hipStream_t st) {
    if (int e = check_fma_args(m, n, k)) return e;
    if (m <= 0 || n <= 0) return PPOCR_OK;
    const int ntiles = (int)((n + BN - 1) / BN);
    dim3 grid(ntiles, (unsigned)((m + BM - 1) / BM));
    head_fma_kernel<EPI_LOGITS, false><<<grid, 256, 0, st>>>(q, w, scale, bias, a, m, (int)n, (int)k, BN, out,
                                                             nullptr, nullptr, nullptr, 0, nullptr, nullptr, 0u, 0);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

int launch_probs_fma(const int8_t* q, const float* w, const float* scale, const float* bias,
                     const float* a, int64_t m, int64_t n, int64_t k, const float* row_max,
                     const float* row_inv, float* probs, hipStream_t st) {
    if (int e = check_fma_args(m, n, k)) return e;
    if (m <= 0 || n <= 0) return PPOCR_OK;
    const int ntiles = (int)((n + BN - 1) / BN);
    dim3 grid(ntiles, (unsigned)((m + BM - 1) / BM));
    head_fma_kernel<EPI_PROBS, false><<<grid, 256, 0, st>>>(q, w, scale, bias, a, m, (int)n, (int)k, BN, probs,
                                                            row_max, row_inv, nullptr, 0, nullptr, nullptr, 0u, 0);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

int launch_stats_fma(const int8_t* q, const float* w, const float* scale, const float* bias,
                     const float* a, int64_t m, int64_t n, int64_t k, int nsplit, Partial* part,
                     hipStream_t st, int64_t line_len) {
    if (int e = check_fma_args(m, n, k)) return e;
    if (line_len < 0) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: bad line length");
    if (nsplit < 1 || nsplit > 1024) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: bad nsplit");
    if (m <= 0) return PPOCR_OK;
    const int ntiles = (int)((n + BN - 1) / BN);
    const int tpc = (ntiles + nsplit - 1) / nsplit;
    dim3 grid(nsplit, (unsigned)((m + BM - 1) / BM));
    head_fma_kernel<EPI_STATS, false><<<grid, 256, 0, st>>>(q, w, scale, bias, a, m, (int)n, (int)k, tpc * BN,
                                                            nullptr, nullptr, nullptr, part, line_len,
                                                            nullptr, nullptr, 0u, 0);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

int launch_rescue_fma(int epi, const FmaWeights& fw, const float* a, int64_t m, int64_t n, int64_t k, int nsplit,
                      int classes_per_chunk, float* out, const float* row_max, const float* row_inv, Partial* part,
                      int64_t line_len, const Guard& guard, hipStream_t st) {
    if (int e = check_fma_args(m, n, k)) return e;
    if (line_len < 0) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: bad line length");
    if (m <= 0 || n <= 0) return PPOCR_OK;
    if (!guard.header || !guard.rows) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: rescue without a guard list");
    // the row count is on the device: a fixed number of row-block slots walk the list
    const unsigned slots = (unsigned)std::min<int64_t>((m + BM - 1) / BM, kFmaRescueSlots);
    int cpc = BN, chunks = (int)((n + BN - 1) / BN);
    if (epi == EPI_STATS) {
        if (nsplit < 1 || nsplit > 1024 || classes_per_chunk <= 0 || (int64_t)classes_per_chunk * nsplit < n)
            return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: bad vocabulary chunks");
        cpc = classes_per_chunk;
        chunks = nsplit;
    }
    dim3 grid((unsigned)chunks, slots);
    auto args = [&](auto kern) {
        kern<<<grid, 256, 0, st>>>(fw.q, fw.w, fw.scale, fw.bias, a, m, (int)n, (int)k, cpc, out, row_max, row_inv,
                                   part, line_len, guard.header, guard.rows, guard.epoch,
                                   guard.capacity);
    };
    if (epi == EPI_LOGITS) args(head_fma_kernel<EPI_LOGITS, true>);
    else if (epi == EPI_PROBS) args(head_fma_kernel<EPI_PROBS, true>);
    else args(head_fma_kernel<EPI_STATS, true>);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

}  // namespace ppocr
