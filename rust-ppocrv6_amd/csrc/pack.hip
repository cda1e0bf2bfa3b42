// Per-class symmetric INT8 packer: QuantizedWeight::from_f32_transposed,
// src/ops/matmul.rs:1173-1202, one wavefront per class row.
#include "kernels.hpp"

namespace ppocr {

// One 64-lane wave per row of W^T [n][k].  The max-abs reduction is order-free (max is
// associative and fmaxf drops NaN, like the reference's fold(0.0, f32::max)), so the
// wave-shuffle tree gives the reference's value exactly.  Scale and its reciprocal use
// correctly rounded division; q = w * inv is a single rounded product; rounding is half
// away from zero; NaN maps to 0 as Rust's saturating `as i8` does.
__global__ __launch_bounds__(256) void pack_int8_kernel(const float* __restrict__ w_t, int64_t n,
                                                        int64_t k, int8_t* __restrict__ q,
                                                        float* __restrict__ scales) {
    // No contraction: q must be rounded from the rounded product w * inv, never from an
    // fma of the unrounded one.
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n) return;
    const float* src = w_t + row * k;
    float mx = 0.0f;
    for (int64_t i = lane; i < k; i += 64) mx = fmaxf(mx, fabsf(src[i]));
    mx = wave_max(mx);
    const float scale = (mx > 1e-8f) ? __fdiv_rn(mx, 127.0f) : 1.0f;
    const float inv = __fdiv_rn(1.0f, scale);
    for (int64_t i = lane; i < k; i += 64) {
        float v = __fmul_rn(src[i], inv);
        float r = round_half_away(v);
        int8_t out;
        if (r != r) {
            out = 0;
        } else {
            r = fminf(fmaxf(r, -127.0f), 127.0f);
            out = (int8_t)(int)r;
        }
        q[row * k + i] = out;
    }
    if (lane == 0) scales[row] = scale;
}

int launch_pack_int8(const float* w_t, int64_t n, int64_t k, int8_t* q, float* scales,
                     hipStream_t st) {
    if (n < 0 || k < 0) return fail(PPOCR_ERR_INVALID_ARG, "QuantizedWeight: negative shape");
    if (n == 0) return PPOCR_OK;
    if ((n + 3) / 4 > 0x7fffffffLL) return fail(PPOCR_ERR_INVALID_ARG, "QuantizedWeight: too many rows");
    dim3 grid((unsigned)((n + 3) / 4));
    pack_int8_kernel<<<grid, 256, 0, st>>>(w_t, n, k, q, scales);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

}  // namespace ppocr
