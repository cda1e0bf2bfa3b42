// Head preparation on the device, for a head created from a model file: the prepack
// transpose (src/engine/model.rs:565-605), the precision and range limits of the split
// activation modes, and the MFMA tile records.  Each produces exactly what the host path
// of ppocr_rh_create / ppocr_rh_create_f32 computes from host arrays.
#include <algorithm>

#include "kernels.hpp"

namespace ppocr {

// dst[c][r] = src[r][c] for src [rows][cols], through a 32x33 LDS tile (coalesced reads
// and writes).  Block 32x8 threads, one 32x32 tile per block.
__global__ __launch_bounds__(256) void transpose_kernel(const float* __restrict__ src, int64_t rows, int64_t cols,
                                                        float* __restrict__ dst) {
    __shared__ float tile[32][33];
    const int64_t c0 = (int64_t)blockIdx.x * 32, r0 = (int64_t)blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
#pragma unroll
    for (int y = ty; y < 32; y += 8) {
        const int64_t r = r0 + y, c = c0 + tx;
        if (r < rows && c < cols) tile[y][tx] = src[r * cols + c];
    }
    __syncthreads();
#pragma unroll
    for (int y = ty; y < 32; y += 8) {
        const int64_t c = c0 + y, r = r0 + tx;
        if (c < cols && r < rows) dst[c * rows + r] = tile[tx][y];
    }
}

int launch_transpose(const float* src, int64_t rows, int64_t cols, float* dst, hipStream_t st) {
    if (rows <= 0 || cols <= 0) return PPOCR_OK;
    const int64_t gx = (cols + 31) / 32, gy = (rows + 31) / 32;
    if (gx > 0x7fffffffLL || gy > 65535) return fail(PPOCR_ERR_INVALID_ARG, "Transpose: matrix too large");
    transpose_kernel<<<dim3((unsigned)gx, (unsigned)gy), 256, 0, st>>>(src, rows, cols, dst);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

// Per class row j (one wave per row, rows strided over the grid), for the guard limits of
// the split-activation modes: the largest |dequantised weight| (float; (float)max|q| *
// scale for an INT8 head), the L1 and L2 norms of the dequantised row and |bias|, in
// double (NaN ignored).  An INT8 row's sums are exact integers scaled once; an FP32 row's
// are summed in a fixed order (lane strides, then xor shuffles), so every call gives the
// same bits.  Each wave keeps its maxima, the workgroup combines its four in LDS and one
// thread publishes them with atomic maxima (one set per workgroup: the four result words
// would serialise an atomic per row).  Maxima of non-negative values are taken on their
// bit patterns, which order the same way.
constexpr int kLimitBlocks = 512;
__global__ __launch_bounds__(256) void head_limits_kernel(const int8_t* __restrict__ q, const float* __restrict__ w,
                                                          const float* __restrict__ scales,
                                                          const float* __restrict__ bias, int64_t n, int64_t k,
                                                          HeadLimitBits* __restrict__ out) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    unsigned wm_bits = 0;
    unsigned long long w1_bits = 0, l2_bits = 0, b_bits = 0;
    for (int64_t row = (int64_t)blockIdx.x * 4 + wave; row < n; row += (int64_t)gridDim.x * 4) {
        float wm;
        double w1, l2;
        if (q) {
            int qm = 0, s1 = 0, s2 = 0;
            for (int64_t i = lane; i < k; i += 64) {
                const int v = abs((int)q[row * k + i]);
                qm = max(qm, v);
                s1 += v;
                s2 += v * v;
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                qm = max(qm, __shfl_xor(qm, o, 64));
                s1 += __shfl_xor(s1, o, 64);
                s2 += __shfl_xor(s2, o, 64);
            }
            wm = __fmul_rn((float)qm, scales[row]);
            w1 = (double)s1 * (double)scales[row];
            l2 = __dsqrt_rn((double)s2) * (double)scales[row];
        } else {
            float m = 0.0f;
            double s1 = 0.0, s2 = 0.0;
            for (int64_t i = lane; i < k; i += 64) {
                const float v = fabsf(w[row * k + i]);
                m = fmaxf(m, v);
                s1 += (double)v;
                s2 = fma((double)v, (double)v, s2);
            }
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) {
                m = fmaxf(m, __shfl_xor(m, o, 64));
                s1 += __shfl_xor(s1, o, 64);
                s2 += __shfl_xor(s2, o, 64);
            }
            wm = m;
            w1 = s1;
            l2 = __dsqrt_rn(s2);
        }
        if (wm == wm) wm_bits = max(wm_bits, __float_as_uint(wm));
        if (w1 == w1) w1_bits = max(w1_bits, (unsigned long long)__double_as_longlong(w1));
        if (l2 == l2) l2_bits = max(l2_bits, (unsigned long long)__double_as_longlong(l2));
        if (bias) {
            const double b = fabs((double)bias[row]);
            if (b == b) b_bits = max(b_bits, (unsigned long long)__double_as_longlong(b));
        }
    }
    __shared__ unsigned s_wm[4];
    __shared__ unsigned long long s_w1[4], s_l2[4], s_b[4];
    if (lane == 0) {
        s_wm[wave] = wm_bits;
        s_w1[wave] = w1_bits;
        s_l2[wave] = l2_bits;
        s_b[wave] = b_bits;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int x = 1; x < 4; ++x) {
            wm_bits = max(wm_bits, s_wm[x]);
            w1_bits = max(w1_bits, s_w1[x]);
            l2_bits = max(l2_bits, s_l2[x]);
            b_bits = max(b_bits, s_b[x]);
        }
        atomicMax(&out->wmax, wm_bits);
        atomicMax(&out->w1, w1_bits);
        atomicMax(&out->l2, l2_bits);
        if (bias) atomicMax(&out->bmax, b_bits);
    }
}

int launch_head_limits(const int8_t* q, const float* w, const float* scales, const float* bias, int64_t n, int64_t k,
                       HeadLimitBits* out, hipStream_t st) {
    if (n <= 0) return PPOCR_OK;
    if ((n + 3) / 4 > 0x7fffffffLL) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: too many classes");
    if (!q && !w) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: no weights");
    head_limits_kernel<<<(unsigned)std::min<int64_t>((n + 3) / 4, kLimitBlocks), 256, 0, st>>>(q, w, scales, bias,
                                                                                             n, k, out);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

// bf16 bits of x, rounded to nearest even; NaN stays NaN (quiet).  The same integer steps
// as the host's record builder.
__device__ __forceinline__ unsigned short bf16_bits_rne_dev(float x) {
    unsigned u = __float_as_uint(x);
    if ((u & 0x7f800000u) == 0x7f800000u) return (unsigned short)((u >> 16) | ((u & 0xffffu) ? 0x40u : 0u));
    u += 0x7fffu + ((u >> 16) & 1u);
    return (unsigned short)(u >> 16);
}

// One thread per (tile, class i, group g): the 8 weights of that group as bf16, or fp16 with
// f16 (and the low plane of an FP32 head); the threads of group 0 also write the class's epilogue
// constants.  Entries past k stay zero, classes past n get zero weights, scale 0 and
// bias*log2e = -inf.
__global__ __launch_bounds__(256) void build_records_kernel(int tiles, int G, int wplanes, int64_t n, int64_t k,
                                                            const int8_t* __restrict__ q, const float* __restrict__ w,
                                                            const float* __restrict__ scale,
                                                            const float* __restrict__ bias, bool f16,
                                                            uint8_t* __restrict__ rec) {
    const int64_t x = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t per_tile = 32LL * G;
    if (x >= (int64_t)tiles * per_tile) return;
    const int t = (int)(x / per_tile);
    const int rem = (int)(x % per_tile);
    const int g = rem / 32, i = rem % 32;
    const size_t frag_bytes = (size_t)wplanes * G * 512;
    uint8_t* r = rec + (size_t)t * (frag_bytes + 512);
    unsigned short* frag = reinterpret_cast<unsigned short*>(r);
    const int64_t row = (int64_t)t * 32 + i;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int64_t kk = (int64_t)g * 8 + e;
        unsigned short hi = 0, lo = 0;
        if (row < n && kk < k) {
            if (f16) {
                // fp16 halves, rounded to nearest even; int8 values are exact
                const float v = q ? (float)q[row * k + kk] : w[row * k + kk];
                const _Float16 h = (_Float16)v;
                hi = __builtin_bit_cast(unsigned short, h);
                if (!q) lo = __builtin_bit_cast(unsigned short, (_Float16)__fsub_rn(v, (float)h));
            } else if (q) {
                hi = bf16_bits_rne_dev((float)q[row * k + kk]);  // exact
            } else {
                const float v = w[row * k + kk];
                hi = bf16_bits_rne_dev(v);
                lo = bf16_bits_rne_dev(__fsub_rn(v, __uint_as_float((unsigned)hi << 16)));
            }
        }
        frag[((size_t)(0 * G + g) * 32 + i) * 8 + e] = hi;
        if (wplanes == 2) frag[((size_t)(1 * G + g) * 32 + i) * 8 + e] = lo;
    }
    if (g == 0) {
        float* ep = reinterpret_cast<float*>(r + frag_bytes);
        if (row < n) {
            const float sc = scale[row], bi = bias ? bias[row] : 0.0f;
            ep[i] = __fmul_rn(sc, kLog2e);
            ep[32 + i] = __fmul_rn(bi, kLog2e);
            ep[64 + i] = sc;
            ep[96 + i] = bi;
        } else {
            ep[i] = 0.0f;
            ep[32 + i] = -INFINITY;
            ep[64 + i] = 0.0f;
            ep[96 + i] = 0.0f;
        }
    }
}

int launch_build_records(const TileGeom& g, int64_t n, int64_t k, const int8_t* q, const float* w,
                         const float* scale, const float* bias, bool f16, uint8_t* rec, hipStream_t st) {
    if (k > 8LL * g.G || g.tiles != (int)((n + 31) / 32) || (q == nullptr) != (g.wplanes == 2))
        return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: tile geometry mismatch");
    const int64_t threads = (int64_t)g.tiles * 32 * g.G;
    if (threads <= 0) return PPOCR_OK;
    if ((threads + 255) / 256 > 0x7fffffffLL) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: too many classes");
    build_records_kernel<<<(unsigned)((threads + 255) / 256), 256, 0, st>>>(g.tiles, g.G, g.wplanes, n, k, q, w, scale,
                                                                             bias, f16, rec);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

}  // namespace ppocr
