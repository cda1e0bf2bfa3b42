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
//   neck_gemm16_kernel rows x W[K][N] on fp16 halves of both operands (three exact products
//                      per f16 MFMA step, fp32 sums), with the LayerNorm of the rows folded
//                      into the operand load and bias, swish and the residual Add folded into
//                      the epilogue; neck_gemm_kernel the same on fp32 MFMA, for weights that
//                      do not bound the operands inside fp16's range;
//   neck_attn16_kernel one workgroup per (line, head): the line's K and V of the head in LDS,
//                      scores and weighted sums on MFMA (fp16 halves; neck_attn_kernel on
//                      fp32), an online softmax between;
//   neck_cf_rows_kernel  a line's channels-first [D][T] block to token rows;
//   neck_final_kernel  the last LayerNorm plus the shortcut.
#include <algorithm>
#include <cmath>

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

// The final LayerNorm of one row by a quad of lanes (lane % 4 = q holds the row's values
// 30 q .. 30 q + 29 in v): sums in a fixed order, each lane's values in turn and then the
// quad's partial sums in two xor shuffles, so the fused and the separate kernel give the
// same bits.  v becomes the normalised values.
constexpr int kLnQuad = kNeckDim / 4;
__device__ __forceinline__ void final_ln_quad(float (&v)[kLnQuad], const float* lnw_q, const float* lnb_q,
                                              float eps) {
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < kLnQuad; ++e) s += v[e];
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    const float mean = __fdiv_rn(s, (float)kNeckDim);
    float t = 0.0f;
#pragma unroll
    for (int e = 0; e < kLnQuad; ++e) {
        v[e] -= mean;
        t = fmaf(v[e], v[e], t);
    }
    t += __shfl_xor(t, 1, 64);
    t += __shfl_xor(t, 2, 64);
    const float inv = inv_std_of(__fdiv_rn(t, (float)kNeckDim), eps);
#pragma unroll
    for (int e = 0; e < kLnQuad; ++e) v[e] = fmaf(v[e] * inv, lnw_q[e], lnb_q[e]);
}

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
// model stores a MatMul weight.  A workgroup owns 128 rows x 128 columns, staged once in
// LDS; it has 4 row groups of 32 rows times 4 / TPW column groups, a wave each, and a wave
// owns TPW tiles of 32 columns, interleaved (tile t holds the group's columns TPW i + t, so
// a lane's TPW B operands of an MFMA step are one LDS read).  With TPW = 2 a workgroup has 8
// waves: two per SIMD, so one wave's loads and stores overlap another's MFMAs.  The
// contraction index is split in halves: lanes 0-31 take k = s, lanes 32-63 take
// k = K/2 + s at MFMA step s, so each lane holds one contiguous half of its row in
// registers (and can normalise it: the row's two halves meet in one xor-32 shuffle).
constexpr int kGemmRows = 128, kGemmCols = 128;

template <int N>
struct FVec;
template <>
struct FVec<2> {
    typedef float type __attribute__((ext_vector_type(2)));
};
template <>
struct FVec<4> {
    typedef float type __attribute__((ext_vector_type(4)));
};

// Epilogue of the tail's GEMMs: lane (i, half) holds columns col .. col + TPW - 1 (tile t:
// col + t) of rows rbase + 8(r/4) + 4 half + r%4; the columns are one chunk wholly inside or
// outside [0, n).  Bias, then the swish (fc1) or the residual Add (proj, fc2).  The residual
// Add reads the rows it overwrites (res == out in place), so every residual is loaded
// before the first store: with the stores in between, each load would wait for the one
// before it.
template <bool SWISH, bool RES, int TPW>
__device__ __forceinline__ void gemm_epilogue_with_bias(const f32x16 (&acc)[TPW],
                                                        const typename FVec<TPW>::type& bc, int64_t rbase, int half,
                                                        int col, int64_t m, int n, const float* res, float* out) {
    using VT = typename FVec<TPW>::type;
    if (col >= n) return;
    VT rv[16];
    if constexpr (RES) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t rr = rbase + 8 * (r >> 2) + 4 * half + (r & 3);
            rv[r] = rr < m ? *reinterpret_cast<const VT*>(res + rr * n + col) : VT{};
        }
    }
    auto value = [&](int r) {
        VT v;
#pragma unroll
        for (int t = 0; t < TPW; ++t) {
            float x = acc[t][r] + bc[t];
            if constexpr (SWISH) x = swish_of(x);
            if constexpr (RES) x = rv[r][t] + x;
            v[t] = x;
        }
        return v;
    };
    // a block wholly inside the batch stores without a branch per row: at a branch the
    // compiler waits for every access in flight (stores included), once per row
    if (rbase + 32 <= m) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t rr = rbase + 8 * (r >> 2) + 4 * half + (r & 3);
            *reinterpret_cast<VT*>(out + rr * n + col) = value(r);
        }
    } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t rr = rbase + 8 * (r >> 2) + 4 * half + (r & 3);
            if (rr < m) *reinterpret_cast<VT*>(out + rr * n + col) = value(r);
        }
    }
}

template <bool SWISH, bool RES, int TPW>
__device__ __forceinline__ void gemm_epilogue(const f32x16 (&acc)[TPW], int64_t rbase, int half, int col, int64_t m,
                                              int n, const float* __restrict__ bias, const float* res, float* out) {
    using VT = typename FVec<TPW>::type;
    if (col >= n) return;
    gemm_epilogue_with_bias<SWISH, RES, TPW>(acc, *reinterpret_cast<const VT*>(bias + col), rbase, half, col, m, n, res,
                                             out);
}

template <int TPW>
constexpr int gemm_threads() {
    return 64 * 4 * (4 / TPW);
}

template <int K, bool LN, bool SWISH, bool RES, int TPW>
__global__ __launch_bounds__(gemm_threads<TPW>()) void neck_gemm_kernel(
    const float* __restrict__ a, int64_t m, const float* __restrict__ w, int n, const float* __restrict__ bias,
    const float* __restrict__ ln_w, const float* __restrict__ ln_b, float eps, const float* res, float* out) {
    static_assert(TPW == 2 || TPW == 4, "tiles per wave");
    using VT = typename FVec<TPW>::type;
    constexpr int KH = K / 2, NW = gemm_threads<TPW>() / 64, GC = 32 * TPW;  // waves, a group's columns
    static_assert(K % 8 == 0, "rows are loaded 4 floats at a time per half");
    extern __shared__ __align__(16) float wl[];  // [K][kGemmCols], then (LN) [2][K]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, i = lane & 31, half = lane >> 5;
    const int rg = wave & 3, cg = wave >> 2;  // row group, column group
    const int n0 = blockIdx.y * kGemmCols;
    // stage W[:, n0 .. n0 + 128) straight from global memory into LDS, all loads in flight
    // at once: one instruction of a wave fills two rows of the stage (64 lanes x 16 bytes),
    // lane L row 2x + L / 32, columns 4 (L % 32) .. + 3.  n is a multiple of 4 and W 16-byte
    // aligned, so a 16-byte chunk lies wholly inside or outside the columns; a chunk past n
    // reloads the row's first chunk instead (it lands in columns whose results are never
    // stored, and each output column depends only on its own W column).
    static_assert(K % 2 == 0, "two stage rows per instruction");
    for (int x = wave; x < K / 2; x += NW) {
        const int kk = 2 * x + (lane >> 5), c4 = n0 + 4 * (lane & 31);
        const float* src = w + (size_t)kk * n + (c4 < n ? c4 : 0);
        __builtin_amdgcn_global_load_lds(
            static_cast<const void*>(src),
            reinterpret_cast<__attribute__((address_space(3))) void*>(
                reinterpret_cast<uintptr_t>(wl + (size_t)x * 2 * kGemmCols)),
            16, 0, 0);
    }
    // the LayerNorm weights and biases after the stage ([K] then [K]), by wave 0: lane L the
    // 16-byte chunk L of the two
    float* lnl = wl + K * kGemmCols;
    if constexpr (LN) {
        static_assert(K % 4 == 0 && K / 2 <= 64, "LayerNorm parameters in one instruction");
        if (wave == 0 && lane < K / 2) {
            const float* src = lane < K / 4 ? ln_w + 4 * lane : ln_b + 4 * (lane - K / 4);
            __builtin_amdgcn_global_load_lds(
                static_cast<const void*>(src),
                reinterpret_cast<__attribute__((address_space(3))) void*>(reinterpret_cast<uintptr_t>(lnl)), 16, 0,
                0);
        }
    }
    // this lane's half row
    const int64_t row = (int64_t)blockIdx.x * kGemmRows + rg * 32 + i;
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
    float mean = 0.0f, inv = 0.0f;
    if constexpr (LN) {
        float s = 0.0f;
#pragma unroll
        for (int x = 0; x < KH; ++x) s += av[x];
        s += __shfl_xor(s, 32, 64);
        mean = __fdiv_rn(s, (float)K);
        float v = 0.0f;
#pragma unroll
        for (int x = 0; x < KH; ++x) {
            const float d = av[x] - mean;
            v = fmaf(d, d, v);
        }
        v += __shfl_xor(v, 32, 64);
        inv = inv_std_of(__fdiv_rn(v, (float)K), eps);
    }
    // the direct loads count in this wave's vmcnt: wait for them, then for the other waves'
    __builtin_amdgcn_s_waitcnt(0x0 | (0x7 << 4) | (0xF << 8));  // vmcnt(0)
    __syncthreads();
    if constexpr (LN) {
#pragma unroll
        for (int x = 0; x < KH; ++x) av[x] = fmaf((av[x] - mean) * inv, lnl[half * KH + x], lnl[K + half * KH + x]);
    }

    // MFMA column i of tile t is W column n0 + GC cg + TPW i + t: a lane's B operands of a
    // step are one LDS read, issued kWPrefetch steps ahead of its MFMAs
    constexpr int kWPrefetch = 4;
    f32x16 acc[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) acc[t] = f32x16{};
    const float* wbase = wl + half * KH * kGemmCols + GC * cg + TPW * i;
    VT wq[kWPrefetch];
#pragma unroll
    for (int p = 0; p < kWPrefetch; ++p) wq[p] = *reinterpret_cast<const VT*>(wbase + p * kGemmCols);
#pragma unroll
    for (int st = 0; st < KH; ++st) {
        const VT cur = wq[st % kWPrefetch];
        if (st + kWPrefetch < KH) wq[st % kWPrefetch] = *reinterpret_cast<const VT*>(wbase + (st + kWPrefetch) * kGemmCols);
#pragma unroll
        for (int t = 0; t < TPW; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[st], cur[t], acc[t], 0, 0, 0);
    }

    gemm_epilogue<SWISH, RES, TPW>(acc, (int64_t)blockIdx.x * kGemmRows + rg * 32, half, n0 + GC * cg + TPW * i, m,
                                   n, bias, res, out);
}

// ---------------------------------------------------------------- GEMM, fp16 halves
// The same products with both operands split into fp16 halves, x = x_hi + x_lo (x_hi the
// nearest half, x_lo the nearest half of what it leaves: 22 bits of x), as three products
// a_hi w_hi + a_hi w_lo + a_lo w_hi on v_mfma_f32_32x32x16_f16 (exact products, fp32 sums);
// the dropped a_lo w_lo is below 2^-22 of each product.  Used when the weights bound every
// operand inside fp16's range (neck creation checks it).  The weights come as fp16 planes of
// W^T, [2][N][KP] (hi, then lo; k padded with zeros to KP); a workgroup stages its 128
// columns of both planes in LDS, the 16-byte chunk q of column c at slot q ^ ((c / 4) % 8),
// so that the lanes reading chunk q of columns 4 i + t (i = 0..7) hit 8 different bank
// groups.  Lane (i, h) holds k = 16 s + 8 h + e (e < 8) of its row at MFMA step s, for the
// activation (A, row i) and the weights (B, column i) alike; the row's LayerNorm meets its
// two halves in xor-32 shuffles as in the fp32 kernel, and the epilogue is the same.
template <int K>
constexpr int gemm16_kp() {
    return K <= 128 ? 128 : 256;
}
// NCB > 1: a workgroup computes NCB column blocks of 32 TPW columns in turn, its rows'
// LayerNorm and halves computed once; the weights of block c + 1 are staged (a second LDS
// buffer) while block c computes and stores.
template <int K, bool LN, int TPW, int NCB = 1>
constexpr size_t gemm16_lds_bytes() {
    return (size_t)(NCB > 1 ? 2 : 1) * 2 * (32 * TPW) * gemm16_kp<K>() * 2 + (LN ? 2 * K * 4 : 0);
}

// TPW: tiles of 32 columns per wave, so 32 TPW columns per column block; NCB column blocks
// per workgroup (NCB > 1 needs n to be a multiple of 32 TPW, and no residual).
template <int K, bool LN, bool SWISH, bool RES, int TPW, int NCB = 1>
__global__ __launch_bounds__(256, 2) void neck_gemm16_kernel(const float* __restrict__ a, int64_t m,
                                                          const uint16_t* __restrict__ wt, int n,
                                                          const float* __restrict__ bias,
                                                          const float* __restrict__ ln_w,
                                                          const float* __restrict__ ln_b, float eps,
                                                          const float* res, float* out) {
    constexpr int KP = gemm16_kp<K>(), S = KP / 16, NCH = KP / 8, NC = 32 * TPW;
    static_assert(K % 8 == 0 && K <= KP, "8-element chunks of k");
    static_assert(TPW == 2 || TPW == 4, "tiles per wave");
    static_assert(NCB == 1 || !RES, "several column blocks per workgroup: no residual loads in the epilogue");
    // [NCB > 1 ? 2 : 1][2][NC][NCH] chunks of 16 bytes, then (LN) [2][K] floats
    extern __shared__ __align__(16) uint8_t ls16[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, i = lane & 31, h = lane >> 5;
    // stage both planes of column block cb into buffer buf: chunk e of the stage = plane
    // e / (NC NCH), column (e / NCH) % NC, slot e % NCH, holding the column's chunk
    // slot ^ ((column / TPW) % 8); a column past n reloads column 0 (its results are never
    // stored, and each output column depends only on its own weights)
    constexpr int CH = 2 * NC * NCH;
    constexpr size_t STAGE = (size_t)CH * 16;
    static_assert(CH % 64 == 0 && NCH % 8 == 0, "whole instructions; slots permuted within groups of 8");
    auto stage = [&](int cb, int buf) {
        const int n0 = ((int)blockIdx.y * NCB + cb) * NC;
        for (int x = wave; x < CH / 64; x += 4) {
            const int e = 64 * x + lane;
            const int p = e / (NC * NCH), c = (e / NCH) % NC, sl = e % NCH;
            const int col = n0 + c < n ? n0 + c : 0;
            const uint16_t* src = wt + ((size_t)p * n + col) * KP + 8 * (sl ^ ((c / TPW) & 7));
            __builtin_amdgcn_global_load_lds(static_cast<const void*>(src),
                                             reinterpret_cast<__attribute__((address_space(3))) void*>(
                                                 reinterpret_cast<uintptr_t>(ls16 + buf * STAGE + 1024 * x)),
                                             16, 0, 0);
        }
    };
    stage(0, 0);
    const float* lnl = reinterpret_cast<const float*>(ls16 + (NCB > 1 ? 2 : 1) * STAGE);
    if constexpr (LN) {
        static_assert(K % 4 == 0 && K / 2 <= 64, "LayerNorm parameters in one instruction");
        if (wave == 0 && lane < K / 2) {
            const float* src = lane < K / 4 ? ln_w + 4 * lane : ln_b + 4 * (lane - K / 4);
            __builtin_amdgcn_global_load_lds(
                static_cast<const void*>(src),
                reinterpret_cast<__attribute__((address_space(3))) void*>(reinterpret_cast<uintptr_t>(lnl)), 16, 0,
                0);
        }
    }
    // this lane's chunks of its row: k = 16 s + 8 h .. + 7 (zeros past K and past m), every
    // load from an address inside the batch and issued before any is used (a branch per
    // chunk made the compiler wait for each)
    const int64_t row = (int64_t)blockIdx.x * kGemmRows + wave * 32 + i;
    const bool row_ok = row < m;
    const float* arow = a + (row_ok ? row : 0) * K;
    float av[S][8];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int k0 = 16 * s + 8 * h;
        const bool ok = row_ok && k0 < K;
        const f32x4* src = reinterpret_cast<const f32x4*>(arow + (k0 < K ? k0 : 0));
        const f32x4 v0 = src[0], v1 = src[1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            av[s][e] = ok ? v0[e] : 0.0f;
            av[s][4 + e] = ok ? v1[e] : 0.0f;
        }
    }
    float mean = 0.0f, inv = 0.0f;
    if constexpr (LN) {
        float sm = 0.0f;
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int e = 0; e < 8; ++e) sm += av[s][e];
        sm += __shfl_xor(sm, 32, 64);
        mean = __fdiv_rn(sm, (float)K);
        float v = 0.0f;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            if (16 * s + 8 * h < K) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float d = av[s][e] - mean;
                    v = fmaf(d, d, v);
                }
            }
        }
        v += __shfl_xor(v, 32, 64);
        inv = inv_std_of(__fdiv_rn(v, (float)K), eps);
    }
    __builtin_amdgcn_s_waitcnt(0x0 | (0x7 << 4) | (0xF << 8));  // vmcnt(0): this wave's direct loads
    __syncthreads();
    // the operand halves
    u16x8 ahi[S], alo[S];
#pragma unroll
    for (int s = 0; s < S; ++s) {
        const int k0 = 16 * s + 8 * h;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float x = av[s][e];
            if constexpr (LN) {
                // computed for every k (the parameters' index clamped to the last k, inside
                // the LDS block) and then masked
                const int kc = min(k0 + e, K - 1);
                const float y = fmaf((x - mean) * inv, lnl[kc], lnl[K + kc]);
                x = k0 < K ? y : 0.0f;
            }
            const _Float16 xh = (_Float16)x;
            const _Float16 xl = (_Float16)(x - (float)xh);
            ahi[s][e] = __builtin_bit_cast(unsigned short, xh);
            alo[s][e] = __builtin_bit_cast(unsigned short, xl);
        }
    }
    const int64_t rbase = (int64_t)blockIdx.x * kGemmRows + wave * 32;
    using VT = typename FVec<TPW>::type;
#pragma unroll 1
    for (int cb = 0; cb < NCB; ++cb) {
        const int n0 = ((int)blockIdx.y * NCB + cb) * NC;
        if (n0 >= n) break;  // uniform over the workgroup
        // this block's bias, loaded before the next block's weights (kept in that order), so
        // that the stores wait for it alone
        const int bcol = n0 + TPW * i;
        const VT bc = *reinterpret_cast<const VT*>(bias + (bcol < n ? bcol : 0));
        __builtin_amdgcn_sched_barrier(0);
        // NCB > 1: the next block's weights, loaded into registers while this block computes
        // and stores, then written to the other LDS buffer (the compiler waits for these
        // loads alone, not for the stores issued after them)
        constexpr int PER = NCB > 1 ? CH / 64 / 4 : 1;
        u32x4 nx[PER];
        const bool next = NCB > 1 && cb + 1 < NCB && n0 + NC < n;
        if (next) {
            const int n1 = n0 + NC;
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const int e = 64 * (wave + 4 * j) + lane;
                const int p = e / (NC * NCH), c = (e / NCH) % NC, sl = e % NCH;
                const int col = n1 + c < n ? n1 + c : 0;
                nx[j] = *reinterpret_cast<const u32x4*>(wt + ((size_t)p * n + col) * KP + 8 * (sl ^ ((c / TPW) & 7)));
            }
        }
        f32x16 acc[TPW];
#pragma unroll
        for (int t = 0; t < TPW; ++t) acc[t] = f32x16{};
        // column TPW i + t, chunk 2 s + h: slot (2 s + h) ^ (i % 8)
        const uint8_t* whi = ls16 + (size_t)(cb & 1) * STAGE + (size_t)(TPW * i) * NCH * 16;
        const uint8_t* wlo = whi + (size_t)NC * NCH * 16;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int sl = (2 * s + h) ^ (i & 7);
#pragma unroll
            for (int t = 0; t < TPW; ++t) {
                const u16x8 bh = *reinterpret_cast<const u16x8*>(whi + ((size_t)t * NCH + sl) * 16);
                const u16x8 bl = *reinterpret_cast<const u16x8*>(wlo + ((size_t)t * NCH + sl) * 16);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, ahi[s]),
                                                                __builtin_bit_cast(f16x8, bh), acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, ahi[s]),
                                                                __builtin_bit_cast(f16x8, bl), acc[t], 0, 0, 0);
                acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, alo[s]),
                                                                __builtin_bit_cast(f16x8, bh), acc[t], 0, 0, 0);
            }
        }
        gemm_epilogue_with_bias<SWISH, RES, TPW>(acc, bc, rbase, h, bcol, m, n, res, out);
        if constexpr (NCB > 1) {
            if (next) {
                uint8_t* dst = ls16 + (size_t)((cb + 1) & 1) * STAGE;
#pragma unroll
                for (int j = 0; j < PER; ++j)
                    *reinterpret_cast<u32x4*>(dst + (size_t)1024 * (wave + 4 * j) + 16 * lane) = nx[j];
            }
            // the next block's weights are in LDS, and no wave still reads this block's
            __syncthreads();
        }
    }
}

// ---------------------------------------------------------------- MLP
// x = x + fc2(swish(fc1(LN2(x)))) for 128 token rows per workgroup, the hidden layer never
// leaving the chip (fp16 halves, as neck_gemm16_kernel).  fc1 runs transposed, hidden
// units as MFMA rows and token rows as columns: lane (i, h) then holds, for its token row i,
// the units 8 (r / 4) + 4 h + r % 4 (r < 16) of each tile of 32 units, which are exactly the
// eight contraction values a lane of fc2's B operand supplies per MFMA step once fc2's
// contraction index runs in the order K' = 32 T + 16 q + 8 h + e <-> unit 32 T + 16 q +
// 8 (e / 4) + 4 h + e % 4 (fc2's weight planes are stored in that order).
// Eight waves, a producer and a consumer per row group of 32 rows, one of each per SIMD: in
// step j the producer (waves 0-3) runs the bias, swish and split of unit tile j, interleaved
// with the MFMAs of tile j + 1's fc1 (the swish's vector work runs while the matrix core
// works), and writes the halves to LDS, lane by lane in the order the consumer's lanes read
// them; the consumer (waves 4-7) runs fc2 of tile j - 1 on the halves written in the step
// before.  (With both roles in one wave each did them in turn, and the barriers kept the two
// waves of a SIMD in the same phase.)  One barrier per step.  The weights stream through
// two LDS rings, fc1's part of
// each tile for the producer and fc2's for the consumer (NeckBlockDev::mlp_h: per tile,
// fc1's rows as [plane][k chunk][unit], 16 KB, then fc2's matching contraction block as
// [plane][chunk][output column], 16 KB, laid out in memory as in LDS, so each load
// instruction reads 1 KB in one piece); the 32 lanes of a half-wave read 32 consecutive
// chunks.  After the last step the consumer holds its rows' complete fc2 sums.
// Operands are scaled by powers of two before their splits (sy, sh; the weight planes hold
// scaled weights) so that the low halves stay above fp16's subnormals, which these MFMAs
// do not all keep; s1, s2 undo the scaling of the products exactly.
// The swish here uses the hardware exp2 and reciprocal (a few ulp from the correctly
// rounded sigmoid, far below the tail's parity bar).
constexpr int kMlpRows = 128;
constexpr int kMlpTiles = 8;     // tiles of 32 hidden units (240 padded to 256)
constexpr int kMlpPart = 16384;  // bytes of a tile's fc1 part, of its fc2 part, of a hidden buffer
constexpr int kMlpCols = 128;    // fc2's output columns, padded
static_assert(kNeckHidden <= 32 * kMlpTiles && kNeckDim <= kMlpCols && kNeckDim <= 128, "MLP geometry");
// LDS: the fc1 ring (4 parts: each is loaded three steps before the step that reads it),
// hidden buffer 0, the fc2 ring (3 parts, loaded two steps ahead), hidden buffer 1, then the
// constants: LN2's weight and bias, fc1's bias, fc2's bias (each padded to whole 16-byte
// chunks; padding never reaches an output), the final LayerNorm's weight and bias.  From
// step 7 on the fc1 ring is not read, and its 64 KB take the workgroup's rows of x, the
// residual.
constexpr int kMlpRing1 = 4, kMlpRing2 = 3;
constexpr int kMlpW1 = 0, kMlpH0 = kMlpRing1 * kMlpPart, kMlpW2 = kMlpH0 + kMlpPart;
constexpr int kMlpH1 = kMlpW2 + kMlpRing2 * kMlpPart, kMlpConst = kMlpH1 + kMlpPart;
constexpr int kMlpConstChunks = 256;
static_assert(kMlpW1 == 0 && kMlpRows * kNeckDim * 4 <= kMlpRing1 * kMlpPart, "the rows of x fit the fc1 ring");
constexpr size_t mlp16_lds_bytes() { return (size_t)kMlpConst + kMlpConstChunks * 16; }

__device__ __forceinline__ float swish_fast(float z) { return z * __builtin_amdgcn_rcpf(1.0f + __expf(-z)); }

// FINAL (the last block): the rows are then taken through the final LayerNorm and the
// shortcut Add (neck_final_kernel's arithmetic) before the store, into fin_out.
template <bool FINAL>
__global__ __launch_bounds__(512, 1) void neck_mlp16_kernel(const float* x, int64_t m,
                                                          const uint16_t* __restrict__ wt,
                                                          const float* __restrict__ b1,
                                                          const float* __restrict__ ln_w,
                                                          const float* __restrict__ ln_b, float eps,
                                                          const float* __restrict__ b2, float sy, float s1, float sh,
                                                          float s2, float* out, const float* __restrict__ lnf_w,
                                                          const float* __restrict__ lnf_b, float lnf_eps,
                                                          const float* __restrict__ shortcut,
                                                          float* __restrict__ fin_out) {
    constexpr int D = kNeckDim, H = kNeckHidden, S = 8;  // fc1: k = 120 in 8 steps of 16
    extern __shared__ __align__(16) uint8_t lm[];
    // constants: chunks 0-29 LN2 weight, 30-59 LN2 bias, 60-123 fc1 bias, 124-155 fc2 bias,
    // 156-185 the final LayerNorm's weight, 186-215 its bias
    const float* lnw = reinterpret_cast<const float*>(lm + kMlpConst);
    const float* lnb = lnw + D;
    const float* b1s = lnw + 2 * D;
    const float* b2s = b1s + 32 * kMlpTiles;
    const float* lfw = b2s + kMlpCols;
    const float* lfb = lfw + D;
    static_assert(D % 4 == 0 && H % 4 == 0 && 4 * D + 32 * kMlpTiles + kMlpCols <= 4 * kMlpConstChunks, "chunks");
    const int tid = threadIdx.x, lane = tid & 63, i = lane & 31, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave & 3;
    const bool producer = wave < 4;
    const int64_t r0 = (int64_t)blockIdx.x * kMlpRows;
    const int64_t row = r0 + grp * 32 + i;
    const int nb = (int)(min((int64_t)kMlpRows, m - r0) * D * 4);  // bytes of the block's rows

    if (wave < (FINAL ? 4 : 3)) {
        const int c = 64 * wave + lane;
        const float* src = c < 30 ? ln_w + 4 * c
                           : c < 60 ? ln_b + 4 * (c - 30)
                           : c < 60 + H / 4 ? b1 + 4 * (c - 60)
                           : c >= 124 && c < 124 + D / 4 ? b2 + 4 * (c - 124)
                           : c >= 156 && c < 186 ? lnf_w + 4 * (c - 156)
                           : c >= 186 && c < 216 ? lnf_b + 4 * (c - 186)
                                                  : b2;  // padding: any finite values
        if (c < (FINAL ? 216 : 156))
            __builtin_amdgcn_global_load_lds(
                static_cast<const void*>(src),
                reinterpret_cast<__attribute__((address_space(3))) void*>(
                    reinterpret_cast<uintptr_t>(lm + kMlpConst + 1024 * wave)),
                16, 0, 0);
    }
    // one 16 KB part (0: fc1's, 1: fc2's) of unit tile T into LDS at dst: 16 instructions of
    // 1 KB, two per wave
    auto stage_part = [&](int T, int part, int dst) {
#pragma unroll
        for (int x2 = 0; x2 < 2; ++x2) {
            const int xi = wave + 8 * x2;
            const uint8_t* src =
                reinterpret_cast<const uint8_t*>(wt) + (size_t)T * (2 * kMlpPart) + part * kMlpPart + 1024 * xi + 16 * lane;
            __builtin_amdgcn_global_load_lds(
                static_cast<const void*>(src),
                reinterpret_cast<__attribute__((address_space(3))) void*>(reinterpret_cast<uintptr_t>(lm + dst + 1024 * xi)),
                16, 0, 0);
        }
    };
    // the workgroup's rows of x (128 x 480 bytes, contiguous) into LDS at 0, whole 16-byte
    // chunks of the rows inside the batch: up to 60 instructions of 1 KB, at most 8 per wave
    auto stage_rows = [&] {
        const uint8_t* src = reinterpret_cast<const uint8_t*>(x + r0 * D);
#pragma unroll
        for (int x8 = 0; x8 < 8; ++x8) {
            const int xi = wave + 8 * x8;
            if (xi < kMlpRows * D * 4 / 1024 && 1024 * xi + 16 * lane < nb)
                __builtin_amdgcn_global_load_lds(
                    static_cast<const void*>(src + 1024 * xi + 16 * lane),
                    reinterpret_cast<__attribute__((address_space(3))) void*>(reinterpret_cast<uintptr_t>(lm + 1024 * xi)),
                    16, 0, 0);
        }
    };
    stage_part(0, 0, kMlpW1);
    stage_part(1, 0, kMlpW1 + kMlpPart);
    stage_part(2, 0, kMlpW1 + 2 * kMlpPart);
    stage_part(0, 1, kMlpW2);

    // producer: its row's chunks k = 16 s + 8 h .. + 7 (zeros past D), every load issued
    // before any is used, then LN2 (the row's two halves meet in xor-32 shuffles)
    float av[S][8];
    float mean = 0.0f, inv = 0.0f;
    if (producer) {
        const int64_t rr = row < m ? row : 0;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int k0 = 16 * s + 8 * h;
            const f32x4* src = reinterpret_cast<const f32x4*>(x + rr * D + (k0 < D ? k0 : 0));
            const f32x4 v0 = src[0], v1 = src[1];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                av[s][e] = k0 < D ? v0[e] : 0.0f;
                av[s][4 + e] = k0 < D ? v1[e] : 0.0f;
            }
        }
        float sm = 0.0f;
#pragma unroll
        for (int s = 0; s < S; ++s)
#pragma unroll
            for (int e = 0; e < 8; ++e) sm += av[s][e];
        sm += __shfl_xor(sm, 32, 64);
        mean = __fdiv_rn(sm, (float)D);
        float var = 0.0f;
#pragma unroll
        for (int s = 0; s < S; ++s) {
            if (16 * s + 8 * h < D) {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float d = av[s][e] - mean;
                    var = fmaf(d, d, var);
                }
            }
        }
        var += __shfl_xor(var, 32, 64);
        inv = inv_std_of(__fdiv_rn(var, (float)D), eps);
    }
    __builtin_amdgcn_s_waitcnt(0x0 | (0x7 << 4) | (0xF << 8));  // vmcnt(0): the first parts, the constants
    __syncthreads();
    // producer: fc1's B operand, the normalised row times sy, fp16 halves
    u16x8 xh[S], xl[S];
    if (producer) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const int k0 = 16 * s + 8 * h;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                // computed for every k (past D it reads other constants of LDS) and then
                // masked, so no branch per value
                const float yv = fmaf((av[s][e] - mean) * inv, lnw[k0 + e], lnb[k0 + e]) * sy;
                const float y = k0 < D ? yv : 0.0f;
                const _Float16 yh = (_Float16)y;
                xh[s][e] = __builtin_bit_cast(unsigned short, yh);
                xl[s][e] = __builtin_bit_cast(unsigned short, (_Float16)(y - (float)yh));
            }
        }
    }
    // hidden buffer of tile T for this row group: [q][plane][lane] 16-byte chunks
    auto hbuf = [&](int T) { return lm + ((T & 1) ? kMlpH1 : kMlpH0) + grp * 4096; };
    // producer: MFMA step s of fc1, transposed (units 32 T + i, A from LDS, x the row, B)
    auto fc1_step = [&](int T, int s, f32x16& a) {
        const uint8_t* w1 = lm + kMlpW1 + (T % kMlpRing1) * kMlpPart;
        const int c = 2 * s + h;
        const u16x8 wh = *reinterpret_cast<const u16x8*>(w1 + ((size_t)c * 32 + i) * 16);
        const u16x8 wl = *reinterpret_cast<const u16x8*>(w1 + ((size_t)(16 + c) * 32 + i) * 16);
        a = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, wh), __builtin_bit_cast(f16x8, xh[s]), a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, wh), __builtin_bit_cast(f16x8, xl[s]), a, 0, 0, 0);
        a = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, wl), __builtin_bit_cast(f16x8, xh[s]), a, 0, 0, 0);
    };
    // producer: hidden value r = 8 q + e of tile T (fc2's contraction value e of step 2 T + q):
    // bias, swish, the mask past H and the split; computed for every unit (b1s holds
    // 32 * kMlpTiles values, padded) and then masked, as a condition around the swish each
    // value became a branch
    auto hidden = [&](const f32x16& a, int T, int r, u16x8 (&hh)[2], u16x8 (&hl)[2]) {
        const int u = 32 * T + 8 * (r >> 2) + 4 * h + (r & 3);
        const float sw = swish_fast(a[r] * s1 + b1s[u]) * sh;
        const float v = u < H ? sw : 0.0f;
        const _Float16 vh = (_Float16)v;
        hh[r >> 3][r & 7] = __builtin_bit_cast(unsigned short, vh);
        hl[r >> 3][r & 7] = __builtin_bit_cast(unsigned short, (_Float16)(v - (float)vh));
    };
    f32x16 a1 = f32x16{};  // producer: fc1 of the tile whose swish the step computes
    if (producer) {
#pragma unroll
        for (int s = 0; s < S; ++s) fc1_step(0, s, a1);
    }
    f32x16 acc2[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc2[t] = f32x16{};
    for (int j = 0; j <= kMlpTiles; ++j) {
        // loads: fc1 of tile j + 3 and fc2 of tile j + 1 (their ring slots were last read two
        // steps and a step before); in step 7, the rows of x into the fc1 ring
        const bool ld1 = j + 3 < kMlpTiles, ld2 = j + 1 < kMlpTiles;
        if (ld1) stage_part(j + 3, 0, kMlpW1 + ((j + 3) % kMlpRing1) * kMlpPart);
        if (ld2) stage_part(j + 1, 1, kMlpW2 + ((j + 1) % kMlpRing2) * kMlpPart);
        if (j == kMlpTiles - 1) stage_rows();
        if (producer) {
            if (j < kMlpTiles) {
                // the swish of tile j (a1) interleaved with the MFMAs of tile j + 1's fc1 (an):
                // the vector work runs while the matrix core works
                u16x8 hh[2], hl[2];
                f32x16 an = f32x16{};
                if (j + 1 < kMlpTiles) {
#pragma unroll
                    for (int s = 0; s < S; ++s) {
                        fc1_step(j + 1, s, an);
#pragma unroll
                        for (int r = 2 * s; r < 2 * s + 2; ++r) hidden(a1, j, r, hh, hl);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 16; ++r) hidden(a1, j, r, hh, hl);
                }
                uint8_t* hb = hbuf(j);
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    *reinterpret_cast<u16x8*>(hb + ((size_t)(2 * q) * 64 + lane) * 16) = hh[q];
                    *reinterpret_cast<u16x8*>(hb + ((size_t)(2 * q + 1) * 64 + lane) * 16) = hl[q];
                }
                a1 = an;
            }
        } else if (j >= 1) {
            const int T = j - 1;
            const uint8_t* w2 = lm + kMlpW2 + (T % kMlpRing2) * kMlpPart;
            const uint8_t* hb = hbuf(T);
            // fc2, transposed: output columns 32 t + i (A, from LDS) x the row's hidden values (B)
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const u16x8 hh = *reinterpret_cast<const u16x8*>(hb + ((size_t)(2 * q) * 64 + lane) * 16);
                const u16x8 hl = *reinterpret_cast<const u16x8*>(hb + ((size_t)(2 * q + 1) * 64 + lane) * 16);
                const int c = 2 * q + h;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const u16x8 bh = *reinterpret_cast<const u16x8*>(w2 + ((size_t)c * kMlpCols + 32 * t + i) * 16);
                    const u16x8 bl = *reinterpret_cast<const u16x8*>(w2 + ((size_t)(4 + c) * kMlpCols + 32 * t + i) * 16);
                    acc2[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, bh),
                                                                     __builtin_bit_cast(f16x8, hh), acc2[t], 0, 0, 0);
                    acc2[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, bl),
                                                                     __builtin_bit_cast(f16x8, hh), acc2[t], 0, 0, 0);
                    acc2[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, bh),
                                                                     __builtin_bit_cast(f16x8, hl), acc2[t], 0, 0, 0);
                }
            }
        }
        // what the next step reads has landed (fc1 of tile j + 2 and fc2 of tile j, issued a
        // step ago); this step's own loads (two instructions per part, per wave) may stay in
        // flight, except the rows of x, waited for here in steps 7 and 8
        if (j >= kMlpTiles - 1) __builtin_amdgcn_s_waitcnt(0x0 | (0x7 << 4) | (0xF << 8));  // vmcnt(0)
        else if (ld1 && ld2) __builtin_amdgcn_s_waitcnt(0x4 | (0x7 << 4) | (0xF << 8));    // vmcnt(4)
        else if (ld1 || ld2) __builtin_amdgcn_s_waitcnt(0x2 | (0x7 << 4) | (0xF << 8));    // vmcnt(2)
        else __builtin_amdgcn_s_waitcnt(0x0 | (0x7 << 4) | (0xF << 8));                   // vmcnt(0)
        __syncthreads();  // every wave is done with this step's parts
    }
    // lane (i, h) of a consumer holds fc2 of row grp * 32 + i at columns 32 t + 8 v + 4 h +
    // 0..3 (acc2[t][4 v ..]): bias and the residual into the rows of x in LDS; then the
    // workgroup stores those rows in one contiguous piece.
    f32x4 scv[8];  // FINAL: the shortcut rows, loaded while the sums are added
    if constexpr (FINAL) {
        const uint8_t* sc = reinterpret_cast<const uint8_t*>(shortcut + r0 * D);
#pragma unroll
        for (int k8 = 0; k8 < 8; ++k8) {
            const int b0 = 16 * tid + 8192 * k8;
            scv[k8] = b0 < nb ? *reinterpret_cast<const f32x4*>(sc + b0) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    if (!producer) {
        float* xr = reinterpret_cast<float*>(lm) + (grp * 32 + i) * D;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int col = 32 * t + 8 * v + 4 * h;
                if (col < D) {
                    f32x4 xv = *reinterpret_cast<const f32x4*>(xr + col);
#pragma unroll
                    for (int e = 0; e < 4; ++e) xv[e] = xv[e] + (acc2[t][4 * v + e] * s2 + b2s[col + e]);
                    *reinterpret_cast<f32x4*>(xr + col) = xv;
                }
            }
    }
    __syncthreads();
    if constexpr (FINAL) {
        // the final LayerNorm of each row in place, a quad of lanes per row
        {
            float* xr = reinterpret_cast<float*>(lm) + (tid >> 2) * D + kLnQuad * (tid & 3);
            float v[kLnQuad];
#pragma unroll
            for (int e = 0; e < kLnQuad; e += 2) {
                const f32x2 p = *reinterpret_cast<const f32x2*>(xr + e);
                v[e] = p[0];
                v[e + 1] = p[1];
            }
            final_ln_quad(v, lfw + kLnQuad * (tid & 3), lfb + kLnQuad * (tid & 3), lnf_eps);
#pragma unroll
            for (int e = 0; e < kLnQuad; e += 2) *reinterpret_cast<f32x2*>(xr + e) = f32x2{v[e], v[e + 1]};
        }
        __syncthreads();
        // out = the normalised rows + the shortcut rows (loaded before the reduction), both
        // contiguous
        uint8_t* dst = reinterpret_cast<uint8_t*>(fin_out + r0 * D);
#pragma unroll
        for (int k8 = 0; k8 < 8; ++k8) {
            const int b0 = 16 * tid + 8192 * k8;
            if (b0 < nb) *reinterpret_cast<f32x4*>(dst + b0) = *reinterpret_cast<const f32x4*>(lm + b0) + scv[k8];
        }
    } else {
        uint8_t* dst = reinterpret_cast<uint8_t*>(out + r0 * D);
        for (int b0 = 16 * tid; b0 < nb; b0 += 16 * 512)
            *reinterpret_cast<f32x4*>(dst + b0) = *reinterpret_cast<const f32x4*>(lm + b0);
    }
}

// ---------------------------------------------------------------- attention
// One workgroup per (line, head), on fp32 MFMA (v_mfma_f32_16x16x4_f32: fp32 products and
// sums, the reference's arithmetic class).  Each wave takes blocks of 16 queries (up to
// kAttnQBlocks of them per pass over the keys, 4 * 16 * kAttnQBlocks queries per pass) and,
// for every block of kAttnKeys keys staged in LDS (K with its dims permuted, V transposed):
//   S^T = K Q^T      key tiles of 16 x 16, contraction over the head's dims (15 padded to 16);
//   the block's maximum per query (column of S^T), meeting across the lane groups in two
//   xor shuffles; the running maximum, and the rescaling of the running sums by
//   exp(old - new) (an online softmax: the first block of a line needs no rescaling);
//   O^T += V^T P^T   contraction over the block's keys.
// In the 16x16 output layout lane l holds column l % 16 and rows 4 * (l / 16) + j, j < 4;
// A and B operands: lane l holds row (A) or column (B) l % 16 at contraction index l / 16.
// So lane l's scores are query l % 16 at keys 16 t + 4 g + j (g = l / 16), and the second
// product takes, at MFMA step s of key tile t, key 16 t + 4 g + s for lane group g on both
// operands: P^T's operand is then the lane's own score j = s, with no data movement.  Dims
// are stored permuted (dim 4 s + g at position 4 g + s) so that one 16-byte LDS read gives a
// lane its four contraction steps.  o = (sum p v) / (sum p) per query.
constexpr int kAttnKeys = 128;                 // keys per LDS block
constexpr int kAttnKeyTiles = kAttnKeys / 16;  // 16-key tiles per block
constexpr int kAttnQBlocks = 2;                // 16-query blocks per wave and pass
constexpr int kAttnSubTiles = 4;               // key tiles per online-softmax step (fp16 kernel)
constexpr int kVtStride = kAttnKeys + 4;

__device__ __forceinline__ int perm_dim(int d) { return 4 * (d & 3) + (d >> 2); }

// max(a, b) as one v_max_f32 (fmaxf on values the compiler cannot prove canonical, MFMA
// results and shuffles, costs a v_max_f32 x, x, x per operand first).  Operands here are
// scores, never NaN unless the inputs are.
__device__ __forceinline__ float max_f32(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ float max3_f32(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

template <int HD>
__global__ __launch_bounds__(256) void neck_attn_kernel(const float* __restrict__ qkv, int64_t m,
                                                        const int64_t* __restrict__ line_off, int64_t lines,
                                                        int64_t line_len, int dim, float scale,
                                                        float* __restrict__ o) {
    static_assert(HD <= 16, "one 16-wide MFMA tile holds a head's dims");
    constexpr int KT = kAttnKeyTiles, QB = kAttnQBlocks;
    __shared__ __align__(16) float ks[kAttnKeys * 16];  // K block [t][dim permuted]
    __shared__ __align__(16) float vt[16 * kVtStride];  // V block transposed [dim][t]
    const int64_t line = blockIdx.x;
    const int h = blockIdx.y;
    const int64_t t0 = line_off ? min(max(line_off[line], (int64_t)0), m) : min(line * line_len, m);
    const int64_t t1 = line_off ? min(max(line_off[line + 1], t0), m) : min(t0 + line_len, m);
    if (t1 - t0 <= 0) return;
    const int T = (int)(t1 - t0);  // the launcher bounds m by INT32_MAX
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = lane & 15, g = lane >> 4;
    const int64_t stride = 3 * (int64_t)dim;
    const float* base = qkv + t0 * stride + h * HD;  // the line's first row, this head
    const int sd = tid & 15, st0 = tid >> 4;  // staging: dim tid % 16 of rows tid / 16 + 16 x
    for (int qpass = 0; qpass < T; qpass += 4 * 16 * QB) {
        // this wave's query blocks: queries qpass + 16 (wave + 4 x) + c
        f32x4 qf[QB], oa[QB], ob[QB];
        float mx[QB], ls[QB];
#pragma unroll
        for (int x = 0; x < QB; ++x) {
            const int q = qpass + 16 * (wave + 4 * x) + c;
            const float* row = base + (int64_t)q * stride;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int d = 4 * s + g;
                qf[x][s] = (q < T && d < HD) ? row[d] : 0.0f;
            }
            oa[x] = ob[x] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            mx[x] = -INFINITY;
            ls[x] = 0.0f;
        }
#pragma unroll
        for (int x = 0; x < QB; ++x) qf[x] = qf[x] * scale;  // the Mul(scale) node, rounded as it
        for (int kb = 0; kb < T; kb += kAttnKeys) {
            const int rem = T - kb;  // keys of the line from this block on
            // stage keys kb .. kb + 127 (zeros past the line's end and past the head's dims),
            // every load issued before the first LDS store
            float kv[KT], vv[KT];
#pragma unroll
            for (int x = 0; x < KT; ++x) {
                const int t = st0 + 16 * x;
                kv[x] = vv[x] = 0.0f;
                if (t < rem && sd < HD) {
                    const float* row = base + (int64_t)(kb + t) * stride + sd;
                    kv[x] = row[dim];
                    vv[x] = row[2 * dim];
                }
            }
            __syncthreads();  // the previous block's readers are done
#pragma unroll
            for (int x = 0; x < KT; ++x) {
                const int tl = st0 + 16 * x;
                ks[tl * 16 + perm_dim(sd)] = kv[x];
                vt[sd * kVtStride + tl] = vv[x];
            }
            __syncthreads();
#pragma unroll
            for (int x = 0; x < QB; ++x) {
                const int q0 = qpass + 16 * (wave + 4 * x);
                if (q0 >= T) continue;  // uniform over the wave
                // one query block at a time: interleaved, their scores would all be live
                __builtin_amdgcn_sched_barrier(0);
                f32x4 sc[KT];
#pragma unroll
                for (int t = 0; t < KT; ++t) {
                    const f32x4 kf = *reinterpret_cast<const f32x4*>(ks + (16 * t + c) * 16 + 4 * g);
                    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[s], qf[x][s], acc, 0, 0, 0);
                    sc[t] = acc;
                }
                // keys past the line's end score -inf (their p is then exactly 0); the block's
                // maximum for query q0 + c: this lane's keys, then the lane groups
                float bm = -INFINITY;
#pragma unroll
                for (int t = 0; t < KT; ++t) {
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        sc[t][jj] = (16 * t + 4 * g + jj < rem) ? sc[t][jj] : -INFINITY;
                        bm = max_f32(bm, sc[t][jj]);
                    }
                }
                bm = max_f32(bm, __shfl_xor(bm, 16, 64));
                bm = max_f32(bm, __shfl_xor(bm, 32, 64));
                const float nm = max_f32(mx[x], bm);
                if (kb > 0) {
                    // rescale the sums so far (every block of a pass after the first follows one
                    // that set a finite maximum)
                    const float corr = __expf(mx[x] - nm);
                    ls[x] *= corr;
                    oa[x] = oa[x] * corr;
                    ob[x] = ob[x] * corr;
                }
                mx[x] = nm;
                float l = 0.0f;
#pragma unroll
                for (int t = 0; t < KT; ++t) {
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        const float p = __expf(sc[t][jj] - nm);
                        sc[t][jj] = p;
                        l += p;
                    }
                }
                ls[x] += l;
                // O^T += V^T P^T, even and odd key tiles on two accumulators
#pragma unroll
                for (int t = 0; t < KT; ++t) {
                    const f32x4 vf = *reinterpret_cast<const f32x4*>(vt + c * kVtStride + 16 * t + 4 * g);
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        if (t & 1) ob[x] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[s], sc[t][s], ob[x], 0, 0, 0);
                        else oa[x] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[s], sc[t][s], oa[x], 0, 0, 0);
                    }
                }
            }
        }
        // per query: the sums of the four lane groups; lane l writes query q0 + c, dims 4 g + j
#pragma unroll
        for (int x = 0; x < QB; ++x) {
            const int q = qpass + 16 * (wave + 4 * x) + c;
            float l = ls[x];
            l += __shfl_xor(l, 16, 64);
            l += __shfl_xor(l, 32, 64);
            if (q < T) {
                float* orow = o + (t0 + q) * (int64_t)dim + h * HD;
#pragma unroll
                for (int jj = 0; jj < 4; ++jj)
                    if (4 * g + jj < HD) orow[4 * g + jj] = __fdiv_rn(oa[x][jj] + ob[x][jj], l);
            }
        }
    }
}

// The same attention on fp16 halves (when the weights bound q, k and v inside fp16's range,
// as for the MatMuls): x = x_hi + x_lo for q * scale, k, v and the probabilities p, three
// products per MFMA step (hi hi, hi lo, lo hi; exact, summed in fp32) on
// v_mfma_f32_16x16x16_f16, which takes a head's 16 dims (or 16 keys) in one step.  The
// operand layouts of the 16x16x16 form: lane l holds row (A) or column (B) l % 16 at
// contraction indices 4 (l / 16) .. + 3; so K rows and V^T rows are read 4 halves at a
// time in their natural order, and P^T's operand of key tile t is again the lane's own
// scores (keys 16 t + 4 g + j), split in place.  Every operand is split after an exact
// scaling by a power of two, undone on the scores and the output: the MFMA takes fp16
// subnormal inputs as zeros (measured: the halves of values below 0.25 would vanish), so
// the scalings lift the low halves above fp16's smallest normal (6.1e-5).  q, k and v use
// exponents from their bounds (neck creation); the probabilities, in (0, 1], 2^15.  The
// head's 16th dim (padding) of V holds 1, so row 15 of O^T accumulates sum(p) beside the
// weighted values (rescaled with them by the online softmax), and the softmax's exponent
// folds the scalings: p = 2^{s ec + eb} with one fma.
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
constexpr int kKhStride = 20;  // halves per K row in LDS: 16 dims + 4, so the 16 rows a
                               // lane group reads at once fall in distinct banks

__device__ __forceinline__ void split_half(float x, _Float16& hi, _Float16& lo) {
    hi = (_Float16)x;
    lo = (_Float16)(x - (float)hi);
}

// qkv rows [m][kNeckQkvPad] (q, k, v of head h at 128 part + 16 h), output rows
// [m][kNeckAttPad] (head h at 16 h; the padding value 15 of each head is written as 0).
template <int HD>
__global__ __launch_bounds__(256) void neck_attn16_kernel(const float* __restrict__ qkv, int64_t m,
                                                          const int64_t* __restrict__ line_off, int64_t lines,
                                                          int64_t line_len, float scale, int eq, int ek, int ev,
                                                          float* __restrict__ o) {
    // powers of two: exact scalings of the operands before the split, undone on the scores
    // and the output
    const float qmul = ldexpf(1.0f, eq), kmul = ldexpf(1.0f, ek), vmul = ldexpf(1.0f, ev);
    const float vdiv = ldexpf(1.0f, -ev);
    // the exponent of the softmax per unit of raw score: 2^-(eq + ek) log2(e)
    const float ec = ldexpf(1.4426950408889634f, -(eq + ek));
    static_assert(HD <= 16, "one 16-wide MFMA tile holds a head's dims");
    constexpr int KT = kAttnKeyTiles, QB = kAttnQBlocks, KS = kAttnSubTiles;
    static_assert(KT % KS == 0, "whole sub-blocks");
    __shared__ __align__(16) _Float16 ks[2][kAttnKeys * kKhStride];  // K block [hi, lo][t][dim]
    __shared__ __align__(16) _Float16 vt[2][16 * kVtStride];         // V block transposed [hi, lo][dim][t]
    const int64_t line = blockIdx.x;
    const int h = blockIdx.y;
    const int64_t t0 = line_off ? min(max(line_off[line], (int64_t)0), m) : min(line * line_len, m);
    const int64_t t1 = line_off ? min(max(line_off[line + 1], t0), m) : min(t0 + line_len, m);
    if (t1 - t0 <= 0) return;
    const int T = (int)(t1 - t0);  // the launcher bounds m by INT32_MAX
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = lane & 15, g = lane >> 4;
    static_assert(HD < 16 && kNeckQkvPad == 3 * 128, "padded heads");
    constexpr int64_t stride = kNeckQkvPad;
    const float* base = qkv + t0 * stride + 16 * h;  // the line's first row, this head
    const int sd = 4 * (tid & 3), st0 = tid >> 2;  // staging: values sd .. sd + 3 of rows tid / 4 + 64 x
    for (int qpass = 0; qpass < T; qpass += 4 * 16 * QB) {
        // this wave's query blocks: queries qpass + 16 (wave + 4 x) + c, dims 4 g .. + 3
        f16x4 qh[QB], ql[QB];
        f32x4 oa[QB];
        float mx[QB];
#pragma unroll
        for (int x = 0; x < QB; ++x) {
            const int q = qpass + 16 * (wave + 4 * x) + c;
            // values 4 g .. 4 g + 3 of the query (the padding value is 0)
            const f32x4 qv = q < T ? *reinterpret_cast<const f32x4*>(base + (int64_t)q * stride + 4 * g)
                                   : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                _Float16 hi, lo;
                split_half((qv[e] * scale) * qmul, hi, lo);  // the Mul(scale) node, rounded as it
                qh[x][e] = hi;
                ql[x][e] = lo;
            }
            oa[x] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            mx[x] = -INFINITY;
        }
        for (int kb = 0; kb < T; kb += kAttnKeys) {
            const int rem = T - kb;  // keys of the line from this block on
            // stage keys kb .. kb + 127 (zeros past the line's end; the padding value is 0),
            // every load issued before the first LDS store
            static_assert(kAttnKeys == 128, "two rows of 64 per thread");
            f32x4 kv[2], vv[2];
#pragma unroll
            for (int x = 0; x < 2; ++x) {
                const int t = st0 + 64 * x;
                const float* row = base + (int64_t)(kb + (t < rem ? t : 0)) * stride + sd;
                const f32x4 k4 = *reinterpret_cast<const f32x4*>(row + 128);
                const f32x4 v4 = *reinterpret_cast<const f32x4*>(row + 256);
                kv[x] = t < rem ? k4 : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                vv[x] = t < rem ? v4 : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
            __syncthreads();  // the previous block's readers are done
#pragma unroll
            for (int x = 0; x < 2; ++x) {
                const int tl = st0 + 64 * x;
                f16x4 kh, kl;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    _Float16 hi, lo;
                    split_half(kv[x][e] * kmul, hi, lo);
                    kh[e] = hi;
                    kl[e] = lo;
                    if (sd + e == 15) {
                        // the padding dim of V holds 1: row 15 of O^T is then sum(p)
                        vt[0][15 * kVtStride + tl] = (_Float16)1.0f;
                        vt[1][15 * kVtStride + tl] = (_Float16)0.0f;
                    } else {
                        split_half(vv[x][e] * vmul, vt[0][(sd + e) * kVtStride + tl], vt[1][(sd + e) * kVtStride + tl]);
                    }
                }
                *reinterpret_cast<f16x4*>(&ks[0][tl * kKhStride + sd]) = kh;
                *reinterpret_cast<f16x4*>(&ks[1][tl * kKhStride + sd]) = kl;
            }
            __syncthreads();
#pragma unroll
            for (int x = 0; x < QB; ++x) {
                const int q0 = qpass + 16 * (wave + 4 * x);
                if (q0 >= T) continue;  // uniform over the wave
                // one query block at a time: interleaved, their scores would all be live
                __builtin_amdgcn_sched_barrier(0);
                // the block's keys in sub-blocks of KS tiles (an online softmax over them: fewer
                // scores live at once); a sub-block wholly past the line's end is skipped
#pragma unroll
                for (int sb = 0; sb < KT / KS; ++sb) {
                    if (16 * KS * sb >= rem) break;  // uniform
                    // scores in the MFMA's units (q and k scaled by 2^eq and 2^ek; the softmax's
                    // exponent takes the scaling back, below)
                    f32x4 sc[KS];
#pragma unroll
                    for (int u = 0; u < KS; ++u) {
                        const int t = KS * sb + u;
                        const f16x4 kh = *reinterpret_cast<const f16x4*>(&ks[0][(16 * t + c) * kKhStride + 4 * g]);
                        const f16x4 kl = *reinterpret_cast<const f16x4*>(&ks[1][(16 * t + c) * kKhStride + 4 * g]);
                        f32x4 acc =
                            __builtin_amdgcn_mfma_f32_16x16x16f16(kh, qh[x], f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(kh, ql[x], acc, 0, 0, 0);
                        sc[u] = __builtin_amdgcn_mfma_f32_16x16x16f16(kl, qh[x], acc, 0, 0, 0);
                    }
                    // keys past the line's end score -inf (their p is then exactly 0), tested only
                    // in the tiles that reach past it; the sub-block's maximum for query q0 + c:
                    // this lane's keys, then the lane groups
                    float bm = -INFINITY;
#pragma unroll
                    for (int u = 0; u < KS; ++u) {
                        const int t = KS * sb + u;
                        if (16 * t + 16 > rem) {  // uniform; the asm keeps it a branch, not selects
                            asm volatile("");
#pragma unroll
                            for (int jj = 0; jj < 4; ++jj)
                                sc[u][jj] = (16 * t + 4 * g + jj < rem) ? sc[u][jj] : -INFINITY;
                        }
                        bm = max3_f32(max3_f32(bm, sc[u][0], sc[u][1]), sc[u][2], sc[u][3]);
                    }
                    bm = max_f32(bm, __shfl_xor(bm, 16, 64));
                    bm = max_f32(bm, __shfl_xor(bm, 32, 64));
                    const float nm = max_f32(mx[x], bm);
                    if (kb > 0 || sb > 0) {
                        // rescale the sums so far (every sub-block after the pass's first follows
                        // one that set a finite maximum: its first key is inside the line)
                        const float corr = __builtin_amdgcn_exp2f((mx[x] - nm) * ec);
                        oa[x] = oa[x] * corr;  // the sum of p (row 15) with the rest
                    }
                    mx[x] = nm;
                    // p = 2^15 e^{(s - max) 2^-(eq+ek)} = 2^{s ec + eb}: one fma and one exp2 per key.
                    // The 2^15 (exact; it cancels in sum(p v) / sum(p)) keeps the halves of small
                    // probabilities above fp16's subnormals.
                    const float eb = fmaf(-nm, ec, 15.0f);
                    f32x4 ob = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                    for (int u = 0; u < KS; ++u) {
                        const int t = KS * sb + u;
                        f16x4 ph, pl;
#pragma unroll
                        for (int jj = 0; jj < 4; ++jj) {
                            const float p = __builtin_amdgcn_exp2f(fmaf(sc[u][jj], ec, eb));
                            // the halves: p with its low 13 mantissa bits cleared (exact in fp16
                            // for p >= 2^-14; below, the conversion rounds it, an error under
                            // 2^-25 on p's scale of 2^15) and the exact remainder, rounded to fp16
                            const float hi = __uint_as_float(__float_as_uint(p) & 0xffffe000u);
                            ph[jj] = (_Float16)hi;
                            pl[jj] = (_Float16)(p - hi);
                        }
                        // O^T += V^T P^T: even and odd key tiles on two accumulators
                        const f16x4 vh = *reinterpret_cast<const f16x4*>(&vt[0][c * kVtStride + 16 * t + 4 * g]);
                        const f16x4 vl = *reinterpret_cast<const f16x4*>(&vt[1][c * kVtStride + 16 * t + 4 * g]);
                        f32x4& acc = (u & 1) ? ob : oa[x];
                        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(vh, ph, acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(vh, pl, acc, 0, 0, 0);
                        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(vl, ph, acc, 0, 0, 0);
                    }
                    oa[x] += ob;
                }
            }
        }
        // per query: the sums of the four lane groups; lane l writes query q0 + c, dims 4 g + j
#pragma unroll
        for (int x = 0; x < QB; ++x) {
            const int q = qpass + 16 * (wave + 4 * x) + c;
            // sum(p) of query c: row 15 of O^T, held by lane group 3
            const float l = __shfl(oa[x][3], 48 + c, 64);
            if (q < T) {
                f32x4 ov;
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) ov[jj] = __fdiv_rn(oa[x][jj] * vdiv, l);
                if (g == 3) ov[3] = 0.0f;  // the padding value
                *reinterpret_cast<f32x4*>(o + (t0 + q) * (int64_t)kNeckAttPad + 16 * h + 4 * g) = ov;
            }
        }
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
__global__ __launch_bounds__(256) void neck_final_kernel(const float* __restrict__ x, int64_t m,
                                                         const float* __restrict__ ln_w,
                                                         const float* __restrict__ ln_b, float eps,
                                                         const float* __restrict__ shortcut,
                                                         float* __restrict__ out) {
    // a quad of lanes per row (whole quads leave together, so the shuffles stay within rows);
    // x is the 16-byte aligned workspace
    const int64_t r = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 2;
    const int q = threadIdx.x & 3;
    if (r >= m) return;
    static_assert(kLnQuad % 2 == 0, "float2 accesses (rows of 480 bytes, quarters of 120)");
    const float* xr = x + r * kNeckDim + kLnQuad * q;
    float v[kLnQuad];
#pragma unroll
    for (int e = 0; e < kLnQuad; e += 2) {
        const f32x2 p = *reinterpret_cast<const f32x2*>(xr + e);
        v[e] = p[0];
        v[e + 1] = p[1];
    }
    final_ln_quad(v, ln_w + kLnQuad * q, ln_b + kLnQuad * q, eps);
    // the shortcut rows and out may be only 4-byte aligned here (the fused path takes the
    // 16-byte aligned ones)
    const float* sr = shortcut + r * kNeckDim + kLnQuad * q;
    float* orow = out + r * kNeckDim + kLnQuad * q;
#pragma unroll
    for (int e = 0; e < kLnQuad; ++e) orow[e] = v[e] + sr[e];
}

// Tiles of 32 columns per wave of the fp16-halves GEMMs: 2, so 64-column blocks with 32 KB
// of weights each.  proj (120 columns) runs a workgroup per column block; qkv (384 columns)
// runs 3 column blocks per workgroup, the rows' LayerNorm and halves computed once per
// workgroup (480 workgroups for the dense batch instead of 1440).
constexpr int kGemm16TilesPerWave = 2;

template <int K, bool LN, bool SWISH, bool RES, int NCB = 1>
int gemm16_go(const float* a, int64_t m, const uint16_t* wt, int n, const float* bias, const float* ln_w,
              const float* ln_b, float eps, const float* res, float* out, hipStream_t st) {
    static_assert(gemm16_kp<K>() == neck_f16_kp(K), "the planes' padding");
    constexpr int TPW = kGemm16TilesPerWave, NC = 32 * TPW;
    if (NCB > 1 && n % NC != 0) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: column blocks do not tile the columns");
    const int64_t gx = (m + kGemmRows - 1) / kGemmRows;
    const int gy = (n + NC * NCB - 1) / (NC * NCB);
    if (gx > 0x7fffffffLL) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: too many rows");
    neck_gemm16_kernel<K, LN, SWISH, RES, TPW, NCB>
        <<<dim3((unsigned)gx, (unsigned)gy), 256, gemm16_lds_bytes<K, LN, TPW, NCB>(), st>>>(
            a, m, wt, n, bias, ln_w, ln_b, eps, res, out);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

// Tiles of 32 columns per wave of the tail's GEMMs (4: 4-wave workgroups; 2, 8-wave
// workgroups with two waves per SIMD, measured 2% slower).
constexpr int kGemmTilesPerWave = 4;

template <int K, bool LN, bool SWISH, bool RES>
int gemm_go(const float* a, int64_t m, const float* w, int n, const float* bias, const float* ln_w,
            const float* ln_b, float eps, const float* res, float* out, hipStream_t st) {
    const int64_t gx = (m + kGemmRows - 1) / kGemmRows;
    const int gy = (n + kGemmCols - 1) / kGemmCols;
    if (gx > 0x7fffffffLL) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: too many rows");
    const size_t lds = (size_t)K * kGemmCols * 4 + (LN ? 2 * K * 4 : 0);
    constexpr int TPW = kGemmTilesPerWave;
    neck_gemm_kernel<K, LN, SWISH, RES, TPW><<<dim3((unsigned)gx, (unsigned)gy), gemm_threads<TPW>(), lds, st>>>(
        a, m, w, n, bias, ln_w, ln_b, eps, res, out);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

}  // namespace

int launch_neck(const NeckDev& nk, const float* x_in, const float* shortcut_in, int64_t m, const int64_t* line_off,
                int64_t lines, int64_t line_len, int layout, float* out, float* ws, hipStream_t st, NeckMarks* marks) {
    // an event after the kernel just launched (and its name), when marks are asked for
    auto mark = [&](const char* name) -> int {
        if (!marks) return PPOCR_OK;
        if (marks->count >= marks->capacity) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: too few events");
        PPOCR_HIP(hipEventRecord(marks->events[marks->count], st));
        marks->names[marks->count++] = name;
        return PPOCR_OK;
    };
    const int D = nk.dim, H = nk.hidden;
    if (D != kNeckDim || H != kNeckHidden || nk.heads * kNeckHeadDim != D)
        return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: unsupported neck geometry");
    if (layout != PPOCR_NECK_ROWS && layout != PPOCR_NECK_CHANNELS_FIRST)
        return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: unknown layout");
    if (m <= 0) return PPOCR_OK;
    if (lines <= 0 || (!line_off && line_len <= 0)) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: no lines");
    if (lines > 0x7fffffffLL) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: too many lines");
    if (int e = mark("start")) return e;
    float* x = ws;                       // residual stream [m][D]
    float* sc = x + m * D;               // shortcut rows [m][D]
    float* qkv = sc + m * D;             // [m][3D], or [m][kNeckQkvPad] on fp16 halves
    float* att = qkv + m * kNeckQkvPad;  // [m][D], or [m][kNeckAttPad]
    float* hid = att + m * kNeckAttPad;  // [m][H]
    const float* scr = shortcut_in;
    if (layout == PPOCR_NECK_CHANNELS_FIRST) {
        const dim3 grid((unsigned)((m + 31) / 32), (unsigned)((D + 31) / 32));
        neck_cf_rows_kernel<<<grid, 256, 0, st>>>(x_in, m, D, line_off, lines, line_len, x);
        neck_cf_rows_kernel<<<grid, 256, 0, st>>>(shortcut_in, m, D, line_off, lines, line_len, sc);
        PPOCR_HIP(hipGetLastError());
        if (int e = mark("channels_first_to_rows")) return e;
        scr = sc;
    }
    // the residual stream: the first block reads it from the input rows (row layout; the
    // GEMMs load rows 16 bytes at a time, so an input that is not 16-byte aligned is copied
    // into the workspace first) and writes it to the workspace with its first residual Add;
    // later blocks work in place
    const float* xin = x;
    if (layout == PPOCR_NECK_ROWS) {
        if (reinterpret_cast<uintptr_t>(x_in) & 15) {
            PPOCR_HIP(hipMemcpyAsync(x, x_in, (size_t)m * D * 4, hipMemcpyDeviceToDevice, st));
            if (int e = mark("copy")) return e;
        } else
            xin = x_in;
    }
    // the fused MLP kernel of the last block finishes the tail itself when the shortcut rows
    // and out are 16-byte aligned
    const bool fused_final =
        ((reinterpret_cast<uintptr_t>(scr) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    for (int b = 0; b < nk.blocks; ++b) {
        const NeckBlockDev& k = nk.block[b];
        const float* xr = b == 0 ? xin : x;
        // LN1 -> qkv
        // qkv's 6 column blocks in two workgroups per row block (480 workgroups for the dense
        // batch; measured 0.1427 ms per forward, against 0.146 with all 6 in one workgroup, 0.150
        // with 2 and 0.151 with a workgroup per block)
        constexpr int kQkvBlocks = kNeckQkvPad / (32 * kGemm16TilesPerWave) / 2;
        if (int e = nk.f16 ? gemm16_go<kNeckDim, true, false, false, kQkvBlocks>(xr, m, k.qkv_h, kNeckQkvPad, k.qkv_bp,
                                                                                k.ln1_w, k.ln1_b, k.ln1_eps, nullptr,
                                                                                qkv, st)
                           : gemm_go<kNeckDim, true, false, false>(xr, m, k.qkv_w, 3 * D, k.qkv_b, k.ln1_w, k.ln1_b,
                                                                   k.ln1_eps, nullptr, qkv, st))
            return e;
        if (int e = mark("ln1_qkv")) return e;
        const dim3 ag((unsigned)lines, (unsigned)nk.heads);
        if (nk.f16)
            neck_attn16_kernel<kNeckHeadDim><<<ag, 256, 0, st>>>(qkv, m, line_off, lines, line_len, nk.scale,
                                                                k.attn_eq, k.attn_ek, k.attn_ev, att);
        else
            neck_attn_kernel<kNeckHeadDim><<<ag, 256, 0, st>>>(qkv, m, line_off, lines, line_len, D, nk.scale, att);
        PPOCR_HIP(hipGetLastError());
        if (int e = mark("attention")) return e;
        // x = x + proj(att)
        if (int e = nk.f16 ? gemm16_go<kNeckAttPad, false, false, true>(att, m, k.proj_h, D, k.proj_b, nullptr, nullptr,
                                                                       0.0f, xr, x, st)
                           : gemm_go<kNeckDim, false, false, true>(att, m, k.proj_w, D, k.proj_b, nullptr, nullptr,
                                                                   0.0f, xr, x, st))
            return e;
        if (int e = mark("proj_residual")) return e;
        if (nk.f16) {
            // x = x + fc2(swish(fc1(LN2(x)))) in one pass
            const int64_t gx = (m + kMlpRows - 1) / kMlpRows;
            if (gx > 0x7fffffffLL) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: too many rows");
            // the last block also applies the final LayerNorm and the shortcut (the rows are 16-byte
            // aligned: the workspace, the shortcut rows and out, checked below)
            const bool fin = b + 1 == nk.blocks && fused_final;
            auto* kern = fin ? neck_mlp16_kernel<true> : neck_mlp16_kernel<false>;
            kern<<<(unsigned)gx, 512, mlp16_lds_bytes(), st>>>(
                x, m, k.mlp_h, k.fc1_b, k.ln2_w, k.ln2_b, k.ln2_eps, k.fc2_b, std::ldexp(1.0f, k.mlp_ey),
                std::ldexp(1.0f, -(k.mlp_e1 + k.mlp_ey)), std::ldexp(1.0f, k.mlp_eh), std::ldexp(1.0f, -(k.mlp_eh + k.mlp_e2)),
                x, nk.lnf_w, nk.lnf_b, nk.lnf_eps, scr, out);
            PPOCR_HIP(hipGetLastError());
            if (int e = mark(fin ? "mlp_final_ln_shortcut" : "mlp")) return e;
            if (fin) return PPOCR_OK;
            continue;
        }
        // LN2 -> fc1 -> swish
        if (int e = gemm_go<kNeckDim, true, true, false>(x, m, k.fc1_w, H, k.fc1_b, k.ln2_w, k.ln2_b, k.ln2_eps,
                                                         nullptr, hid, st))
            return e;
        if (int e = mark("ln2_fc1_swish")) return e;
        // x = x + fc2(hid)
        if (int e = gemm_go<kNeckHidden, false, false, true>(hid, m, k.fc2_w, D, k.fc2_b, nullptr, nullptr, 0.0f, x,
                                                             x, st))
            return e;
        if (int e = mark("fc2_residual")) return e;
    }
    neck_final_kernel<<<(unsigned)((m + 63) / 64), 256, 0, st>>>(x, m, nk.lnf_w, nk.lnf_b, nk.lnf_eps, scr, out);
    PPOCR_HIP(hipGetLastError());
    return mark("final_ln_shortcut");
}

}  // namespace ppocr
