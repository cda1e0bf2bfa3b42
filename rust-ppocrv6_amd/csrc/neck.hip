// The SVTR mixing tail of the recognition model, before the head (the graph between
// Transpose.0 and Transpose.8 of PP-OCRv6_small_rec: two transformer blocks over the T
// tokens of each text line, a final LayerNorm and the convolution shortcut), as the
// reference's executor runs it node by node: LayerNorm (src/ops/layernorm.rs:5-244, the
// fused ReduceMean..Add pattern of src/engine/model.rs:2143-2245), MatMul + Add bias
// (src/ops/matmul.rs:9-96), the attention's Mul(scale), MatMul(q, k^T), Softmax over the
// keys (src/ops/softmax.rs:199-285) and MatMul(p, v), Sigmoid (src/ops/activation.rs:25-94)
// and Mul for the swish, and the residual Adds.
//
// gfx950 layout: the token rows of all lines packed back to back, channels contiguous
// ([m][D], D = 120).  Four kinds of kernels:
//   neck_gemm_kernel   rows x W[K][N] on fp32 MFMA (v_mfma_f32_32x32x2_f32: fp32 products,
//                      fp32 sums), with the LayerNorm of the rows folded into the operand
//                      load and bias, swish and the residual Add folded into the epilogue;
//   neck_attn_kernel   one workgroup per (line, head), the line's keys and values in LDS,
//                      a 16-lane group per query (two passes: maximum, then sums);
//   neck_cf_rows_kernel  a line's channels-first [D][T] block to token rows;
//   neck_final_kernel  the last LayerNorm plus the shortcut.
#include <algorithm>

#include "kernels.hpp"
#include "neck.hpp"

namespace ppocr {

namespace {

// 1 / sqrt(var + eps) with correctly rounded square root and division, as the reference's
// `1.0 / (var + eps).sqrt()`.
__device__ __forceinline__ float inv_std_of(float var, float eps) { return __fdiv_rn(1.0f, __fsqrt_rn(var + eps)); }

// sigmoid(x) = 1 / (1 + exp(-x)) and the swish x * sigmoid(x), each step rounded as the
// reference's Sigmoid and Mul nodes round it.
__device__ __forceinline__ float swish_of(float x) { return x * __fdiv_rn(1.0f, 1.0f + expf(-x)); }

// Line of token row r: the last line whose (clamped) start is at most r, by binary search
// over the device offsets; -1 when r lies in no line.  t0, t1: that line's rows.
__device__ __forceinline__ int64_t line_of_row(const int64_t* line_off, int64_t lines, int64_t line_len, int64_t m,
                                               int64_t r, int64_t* t0, int64_t* t1) {
    int64_t line;
    if (!line_off) {
        line = r / line_len;
    } else {
        int64_t lo = 0, hi = lines - 1;
        while (lo < hi) {
            const int64_t mid = (lo + hi + 1) >> 1;
            if (min(max(line_off[mid], (int64_t)0), m) <= r) lo = mid;
            else hi = mid - 1;
        }
        line = lo;
    }
    *t0 = line_off ? min(max(line_off[line], (int64_t)0), m) : min(line * line_len, m);
    *t1 = line_off ? min(max(line_off[line + 1], *t0), m) : min(*t0 + line_len, m);
    return (r >= *t0 && r < *t1) ? line : -1;
}

// ---------------------------------------------------------------- GEMM
// out[r][n] = EPI(LN?(a[r])[.] . W[.][n] + bias[n]) (+ res[r][n]), W row-major [K][N] as the
// model stores a MatMul weight.  A workgroup owns 128 rows x 128 columns; each wave 32 rows x
// 4 tiles of 32 columns.  The contraction index is split in halves: lanes 0-31 take
// k = s, lanes 32-63 take k = K/2 + s at MFMA step s, so each lane holds one contiguous half
// of its row in registers (and can normalise it: the row's two halves meet in one xor-32
// shuffle).  The workgroup's W columns are staged once in LDS.
constexpr int kGemmRows = 128, kGemmCols = 128;

template <int K, bool LN, bool SWISH, bool RES>
__global__ __launch_bounds__(256) void neck_gemm_kernel(const float* __restrict__ a, int64_t m,
                                                        const float* __restrict__ w, int n,
                                                        const float* __restrict__ bias,
                                                        const float* __restrict__ ln_w,
                                                        const float* __restrict__ ln_b, float eps,
                                                        const float* res, float* out) {
    constexpr int KH = K / 2;
    static_assert(K % 8 == 0, "rows are loaded 4 floats at a time per half");
    extern __shared__ __align__(16) float wl[];  // [K][kGemmCols]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, i = lane & 31, half = lane >> 5;
    const int n0 = blockIdx.y * kGemmCols;
    // stage W[:, n0 .. n0 + 128) (columns past n as zeros)
    for (int e = tid; e < K * (kGemmCols / 4); e += 256) {
        const int kk = e / (kGemmCols / 4), c4 = (e % (kGemmCols / 4)) * 4;
        f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
        const float* src = w + (size_t)kk * n + n0 + c4;
        if (n0 + c4 + 3 < n) {
            v = f32x4{src[0], src[1], src[2], src[3]};
        } else {
#pragma unroll
            for (int x = 0; x < 4; ++x)
                if (n0 + c4 + x < n) v[x] = src[x];
        }
        *reinterpret_cast<f32x4*>(wl + kk * kGemmCols + c4) = v;
    }
    // this lane's half row
    const int64_t row = (int64_t)blockIdx.x * kGemmRows + wave * 32 + i;
    float av[KH];
    if (row < m) {
        const f32x4* src = reinterpret_cast<const f32x4*>(a + row * K + half * KH);
#pragma unroll
        for (int x = 0; x < KH / 4; ++x) {
            const f32x4 v = src[x];
            av[4 * x] = v[0];
            av[4 * x + 1] = v[1];
            av[4 * x + 2] = v[2];
            av[4 * x + 3] = v[3];
        }
    } else {
#pragma unroll
        for (int x = 0; x < KH; ++x) av[x] = 0.0f;
    }
    if constexpr (LN) {
        float s = 0.0f;
#pragma unroll
        for (int x = 0; x < KH; ++x) s += av[x];
        s += __shfl_xor(s, 32, 64);
        const float mean = __fdiv_rn(s, (float)K);
        float v = 0.0f;
#pragma unroll
        for (int x = 0; x < KH; ++x) {
            const float d = av[x] - mean;
            v = fmaf(d, d, v);
        }
        v += __shfl_xor(v, 32, 64);
        const float inv = inv_std_of(__fdiv_rn(v, (float)K), eps);
#pragma unroll
        for (int x = 0; x < KH; ++x) av[x] = fmaf((av[x] - mean) * inv, ln_w[half * KH + x], ln_b[half * KH + x]);
    }
    __syncthreads();

    f32x16 acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = f32x16{};
#pragma unroll
    for (int s = 0; s < KH; ++s) {
        const float* wr = wl + (half * KH + s) * kGemmCols + i;
#pragma unroll
        for (int t = 0; t < 4; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[s], wr[32 * t], acc[t], 0, 0, 0);
    }

    // epilogue: lane (i, half) holds column n0 + 32t + i of rows 8(r/4) + 4 half + r%4
    const int64_t rbase = (int64_t)blockIdx.x * kGemmRows + wave * 32;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const int col = n0 + 32 * t + i;
        if (col >= n) continue;
        const float bc = bias[col];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t rr = rbase + 8 * (r >> 2) + 4 * half + (r & 3);
            if (rr >= m) continue;
            float v = acc[t][r] + bc;
            if constexpr (SWISH) v = swish_of(v);
            if constexpr (RES) v = res[rr * n + col] + v;
            out[rr * n + col] = v;
        }
    }
}

// ---------------------------------------------------------------- attention
// qkv rows [m][3D] hold (q | k | v), each head h at columns h*HD .. h*HD + HD - 1 of its
// third (the Reshape [0, -1, 3, H, HD] of the graph).  One workgroup per (line, head): the
// line's keys and values of that head are staged once in LDS (rows of kKvStride floats:
// 16-byte aligned, and the 16 keys a lane group reads at once fall in distinct banks), then
// each wave takes 4 queries at a time, lane group g = lane / 16 one query, lane j of the
// group the keys j, j + 16, ...: pass 1 the scores s = (q * scale) . k and their maximum
// (xor-shuffled over the group), pass 2 the same scores, p = exp(s - max), the sums of p and
// of p * v, summed over the group; o = (sum p v) / (sum p).  Lines longer than
// kAttnLdsSteps stream their keys from global memory with a running maximum instead.
constexpr int kAttnLdsSteps = 256;
constexpr int kKvStride = 20;

template <int HD>
__device__ __forceinline__ float score(const float (&q)[16], const float* kr) {
    const f32x4* k4 = reinterpret_cast<const f32x4*>(kr);
    float s = 0.0f;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
        const f32x4 kv = k4[x];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (4 * x + e < HD) s = fmaf(q[4 * x + e], kv[e], s);
    }
    return s;
}

template <int HD>
__global__ __launch_bounds__(256) void neck_attn_kernel(const float* __restrict__ qkv, int64_t m,
                                                        const int64_t* __restrict__ line_off, int64_t lines,
                                                        int64_t line_len, int dim, float scale,
                                                        float* __restrict__ o) {
    static_assert(HD <= 16, "a lane group holds one head's query");
    __shared__ __align__(16) float ks[kAttnLdsSteps * kKvStride];
    __shared__ __align__(16) float vs[kAttnLdsSteps * kKvStride];
    const int64_t line = blockIdx.x;
    const int h = blockIdx.y;
    const int64_t t0 = line_off ? min(max(line_off[line], (int64_t)0), m) : min(line * line_len, m);
    const int64_t t1 = line_off ? min(max(line_off[line + 1], t0), m) : min(t0 + line_len, m);
    const int64_t T = t1 - t0;
    if (T <= 0) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, j = lane & 15;
    const int64_t stride = 3 * (int64_t)dim;
    const bool in_lds = T <= kAttnLdsSteps;
    if (in_lds) {
        for (int e = tid; e < (int)T * 16; e += 256) {
            const int t = e >> 4, d = e & 15;
            const float* row = qkv + (t0 + t) * stride + h * HD;
            ks[t * kKvStride + d] = d < HD ? row[dim + d] : 0.0f;
            vs[t * kKvStride + d] = d < HD ? row[2 * dim + d] : 0.0f;
        }
        __syncthreads();
    }
    for (int64_t qi = (int64_t)wave * 4 + g; qi - g < T; qi += 16) {
        const bool valid = qi < T;  // uniform over the lane group
        const int64_t r = t0 + qi;
        float q[16];
#pragma unroll
        for (int d = 0; d < 16; ++d) q[d] = (valid && d < HD) ? qkv[r * stride + h * HD + d] * scale : 0.0f;
        float l = 0.0f, acc[HD];
#pragma unroll
        for (int d = 0; d < HD; ++d) acc[d] = 0.0f;
        if (in_lds) {
            float mx = -INFINITY;
            for (int t = j; t < (int)T; t += 16) mx = fmaxf(mx, score<HD>(q, ks + t * kKvStride));
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
            for (int t = j; t < (int)T; t += 16) {
                const float p = __expf(score<HD>(q, ks + t * kKvStride) - mx);
                l += p;
                const f32x4* v4 = reinterpret_cast<const f32x4*>(vs + t * kKvStride);
#pragma unroll
                for (int x = 0; x < 4; ++x) {
                    const f32x4 vv = v4[x];
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (4 * x + e < HD) acc[4 * x + e] = fmaf(p, vv[e], acc[4 * x + e]);
                }
            }
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) {
                l += __shfl_xor(l, off, 64);
#pragma unroll
                for (int d = 0; d < HD; ++d) acc[d] += __shfl_xor(acc[d], off, 64);
            }
        } else {
            float mx = -INFINITY;
            for (int64_t t = t0 + j; t < t1; t += 16) {
                const float* kr = qkv + t * stride + dim + h * HD;
                const float* vr = qkv + t * stride + 2 * dim + h * HD;
                float s = 0.0f;
#pragma unroll
                for (int d = 0; d < HD; ++d) s = fmaf(q[d], kr[d], s);
                const float nm = fmaxf(mx, s);
                const float corr = (mx == -INFINITY) ? 0.0f : __expf(mx - nm);
                const float p = __expf(s - nm);
                l = fmaf(l, corr, p);
#pragma unroll
                for (int d = 0; d < HD; ++d) acc[d] = fmaf(acc[d], corr, p * vr[d]);
                mx = nm;
            }
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) {
                const float om = __shfl_xor(mx, off, 64);
                const float ol = __shfl_xor(l, off, 64);
                const float nm = fmaxf(mx, om);
                const float ca = (mx == -INFINITY) ? 0.0f : __expf(mx - nm);
                const float cb = (om == -INFINITY) ? 0.0f : __expf(om - nm);
                l = l * ca + ol * cb;
#pragma unroll
                for (int d = 0; d < HD; ++d) {
                    const float oa = __shfl_xor(acc[d], off, 64);
                    acc[d] = acc[d] * ca + oa * cb;
                }
                mx = nm;
            }
        }
        // lane j of the group writes dimension j
        float mine = 0.0f;
#pragma unroll
        for (int d = 0; d < HD; ++d) mine = (j == d) ? acc[d] : mine;
        if (valid && j < HD) o[r * dim + h * HD + j] = l > 0.0f ? __fdiv_rn(mine, l) : 0.0f;
    }
}

// ---------------------------------------------------------------- layouts and the end
// Channels-first lines (line b: [D][T_b] at D * t0_b, the graph's [1, D, T] per line) to
// token rows [m][D]: a 32-row x 32-channel tile per workgroup through LDS (reads along the
// steps of a channel, writes along the channels of a row).
__global__ __launch_bounds__(256) void neck_cf_rows_kernel(const float* __restrict__ src, int64_t m, int dim,
                                                           const int64_t* __restrict__ line_off, int64_t lines,
                                                           int64_t line_len, float* __restrict__ dst) {
    __shared__ float tile[32][33];
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    const int64_t r0 = (int64_t)blockIdx.x * 32;
    const int c0 = blockIdx.y * 32;
    for (int y = ty; y < 32; y += 8) {
        // read: row r0 + tx, channel c0 + y
        const int64_t r = r0 + tx;
        const int c = c0 + y;
        float v = 0.0f;
        if (r < m && c < dim) {
            int64_t t0, t1;
            if (line_of_row(line_off, lines, line_len, m, r, &t0, &t1) >= 0)
                v = src[dim * t0 + (int64_t)c * (t1 - t0) + (r - t0)];
        }
        tile[y][tx] = v;
    }
    __syncthreads();
    for (int y = ty; y < 32; y += 8) {
        const int64_t r = r0 + y;
        const int c = c0 + tx;
        if (r < m && c < dim) dst[r * dim + c] = tile[tx][y];
    }
}

// out[r] = LayerNorm(x[r]) + shortcut[r]: one wave per row, D <= 128 (two channels a lane).
__global__ __launch_bounds__(256) void neck_final_kernel(const float* __restrict__ x, int64_t m, int dim,
                                                         const float* __restrict__ ln_w,
                                                         const float* __restrict__ ln_b, float eps,
                                                         const float* __restrict__ shortcut,
                                                         float* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= m) return;
    const int c0 = 2 * lane, c1 = 2 * lane + 1;
    const float v0 = c0 < dim ? x[r * dim + c0] : 0.0f;
    const float v1 = c1 < dim ? x[r * dim + c1] : 0.0f;
    const float mean = __fdiv_rn(wave_sum(v0 + v1), (float)dim);
    const float d0 = c0 < dim ? v0 - mean : 0.0f, d1 = c1 < dim ? v1 - mean : 0.0f;
    const float var = __fdiv_rn(wave_sum(fmaf(d0, d0, d1 * d1)), (float)dim);
    const float inv = inv_std_of(var, eps);
    if (c0 < dim) out[r * dim + c0] = fmaf(d0 * inv, ln_w[c0], ln_b[c0]) + shortcut[r * dim + c0];
    if (c1 < dim) out[r * dim + c1] = fmaf(d1 * inv, ln_w[c1], ln_b[c1]) + shortcut[r * dim + c1];
}

template <int K, bool LN, bool SWISH, bool RES>
int gemm_go(const float* a, int64_t m, const float* w, int n, const float* bias, const float* ln_w,
            const float* ln_b, float eps, const float* res, float* out, hipStream_t st) {
    const int64_t gx = (m + kGemmRows - 1) / kGemmRows;
    const int gy = (n + kGemmCols - 1) / kGemmCols;
    if (gx > 0x7fffffffLL) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: too many rows");
    neck_gemm_kernel<K, LN, SWISH, RES><<<dim3((unsigned)gx, (unsigned)gy), 256, K * kGemmCols * 4, st>>>(
        a, m, w, n, bias, ln_w, ln_b, eps, res, out);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

}  // namespace

int launch_neck(const NeckDev& nk, const float* x_in, const float* shortcut_in, int64_t m, const int64_t* line_off,
                int64_t lines, int64_t line_len, int layout, float* out, float* ws, hipStream_t st) {
    const int D = nk.dim, H = nk.hidden;
    if (D != kNeckDim || H != kNeckHidden || nk.heads * kNeckHeadDim != D)
        return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: unsupported neck geometry");
    if (layout != PPOCR_NECK_ROWS && layout != PPOCR_NECK_CHANNELS_FIRST)
        return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: unknown layout");
    if (m <= 0) return PPOCR_OK;
    if (lines <= 0 || (!line_off && line_len <= 0)) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: no lines");
    if (lines > 0x7fffffffLL) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: too many lines");
    float* x = ws;                       // residual stream [m][D]
    float* sc = x + m * D;               // shortcut rows [m][D]
    float* qkv = sc + m * D;             // [m][3D]
    float* att = qkv + m * 3 * D;        // [m][D]
    float* hid = att + m * D;            // [m][H]
    const float* scr = shortcut_in;
    if (layout == PPOCR_NECK_CHANNELS_FIRST) {
        const dim3 grid((unsigned)((m + 31) / 32), (unsigned)((D + 31) / 32));
        neck_cf_rows_kernel<<<grid, 256, 0, st>>>(x_in, m, D, line_off, lines, line_len, x);
        neck_cf_rows_kernel<<<grid, 256, 0, st>>>(shortcut_in, m, D, line_off, lines, line_len, sc);
        PPOCR_HIP(hipGetLastError());
        scr = sc;
    } else {
        PPOCR_HIP(hipMemcpyAsync(x, x_in, (size_t)m * D * 4, hipMemcpyDeviceToDevice, st));
    }
    for (int b = 0; b < nk.blocks; ++b) {
        const NeckBlockDev& k = nk.block[b];
        // LN1 -> qkv
        if (int e = gemm_go<kNeckDim, true, false, false>(x, m, k.qkv_w, 3 * D, k.qkv_b, k.ln1_w, k.ln1_b, k.ln1_eps,
                                                          nullptr, qkv, st))
            return e;
        const dim3 ag((unsigned)lines, (unsigned)nk.heads);
        neck_attn_kernel<kNeckHeadDim><<<ag, 256, 0, st>>>(qkv, m, line_off, lines, line_len, D, nk.scale, att);
        PPOCR_HIP(hipGetLastError());
        // x = x + proj(att)
        if (int e = gemm_go<kNeckDim, false, false, true>(att, m, k.proj_w, D, k.proj_b, nullptr, nullptr, 0.0f, x, x,
                                                          st))
            return e;
        // LN2 -> fc1 -> swish
        if (int e = gemm_go<kNeckDim, true, true, false>(x, m, k.fc1_w, H, k.fc1_b, k.ln2_w, k.ln2_b, k.ln2_eps,
                                                         nullptr, hid, st))
            return e;
        // x = x + fc2(hid)
        if (int e = gemm_go<kNeckHidden, false, false, true>(hid, m, k.fc2_w, D, k.fc2_b, nullptr, nullptr, 0.0f, x,
                                                             x, st))
            return e;
    }
    neck_final_kernel<<<(unsigned)((m + 3) / 4), 256, 0, st>>>(x, m, D, nk.lnf_w, nk.lnf_b, nk.lnf_eps, scr, out);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

}  // namespace ppocr
