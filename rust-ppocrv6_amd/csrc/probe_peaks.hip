// Peak probes of the benchmark (not part of the head library's interface): dense bf16
// MFMA throughput with every operand in registers, i.e. the matrix cores' ceiling at the
// clock the GPU holds under this load, to set beside the datasheet peak; once with
// few-bit constant operands and once with operands like the statistics pass's; dense fp16
// MFMA with operands like the SVTR tail's.  And the HBM write ceiling: streaming 16-byte stores over a buffer of a given size (the unfused
// logits writer's bound).
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Four independent accumulation chains per wave, so the matrix core never waits on a
// chain's previous result; the sums are stored so nothing is optimised away.
__global__ __launch_bounds__(256) void mfma_peak_kernel(float* __restrict__ out, int iters) {
    const int lane = threadIdx.x & 63;
    bf16x8 a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[e] = (__bf16)(0.001f * (float)((lane + e) % 7));
        b[e] = (__bf16)(0.002f * (float)((3 * lane + e) % 5));
    }
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int it = 0; it < iters; ++it) {
        c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, a, c1, 0, 0, 0);
        c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, a, c2, 0, 0, 0);
        c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b, b, c3, 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) s += (c0[r] + c1[r]) + (c2[r] + c3[r]);
    out[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

// Operands with the statistics pass's bit patterns, made per lane from a hash: A = weights,
// bf16 of integers uniform in -127..127; B = activation terms, the bf16 nearest a value of
// about N(0, 1) (a sum of four uniforms) and the bf16 nearest its remainder, in turn.  The
// matrix cores draw more power on such operands than on the peak probe's few-bit constants,
// and the GPU lowers their clock to hold its power limit, so this rate is the one the
// statistics pass can reach.
__device__ __forceinline__ unsigned mix32(unsigned x) {
    x ^= x >> 16;
    x *= 0x7feb352dU;
    x ^= x >> 15;
    x *= 0x846ca68bU;
    x ^= x >> 16;
    return x;
}
__global__ __launch_bounds__(256) void mfma_data_kernel(float* __restrict__ out, int iters) {
    const unsigned seed = (unsigned)(blockIdx.x * 256 + threadIdx.x) * 64u;
    bf16x8 w[8], x[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const unsigned h = mix32(seed + (unsigned)(s * 8 + e));
            w[s][e] = (__bf16)(float)((int)(h % 255u) - 127);
            float g = 0.0f;
#pragma unroll
            for (int u = 0; u < 4; ++u) g += (float)((mix32(h + 0x9e3779b9U * (unsigned)(u + 1)) >> 8) & 0xffff);
            g = (g * (1.0f / 65536.0f) - 2.0f) * 1.7320508f;
            const __bf16 hi = (__bf16)g;
            x[s][e] = (s & 1) ? (__bf16)(g - (float)hi) : hi;
        }
    }
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int s = 0; s < 8; s += 4) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w[s], x[s], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w[s + 1], x[s + 1], c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w[s + 2], x[s + 2], c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w[s + 3], x[s + 3], c3, 0, 0, 0);
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) s += (c0[r] + c1[r]) + (c2[r] + c3[r]);
    out[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

// The same for fp16 (v_mfma_f32_32x32x16_f16) with operands like the SVTR tail's GEMMs,
// which multiply fp16 halves of both operands: A and B alternate between the fp16 nearest a
// value of about N(0, 1) and the fp16 nearest its remainder.
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
__global__ __launch_bounds__(256) void mfma_f16_data_kernel(float* __restrict__ out, int iters) {
    const unsigned seed = (unsigned)(blockIdx.x * 256 + threadIdx.x) * 64u + 0x5bd1e995U;
    f16x8 w[8], x[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float g[2];
#pragma unroll
            for (int o = 0; o < 2; ++o) {
                const unsigned h = mix32(seed + (unsigned)(2 * (s * 8 + e) + o));
                float v = 0.0f;
#pragma unroll
                for (int u = 0; u < 4; ++u) v += (float)((mix32(h + 0x9e3779b9U * (unsigned)(u + 1)) >> 8) & 0xffff);
                g[o] = (v * (1.0f / 65536.0f) - 2.0f) * 1.7320508f;
            }
            const _Float16 wh = (_Float16)g[0], xh = (_Float16)g[1];
            w[s][e] = (s & 1) ? (_Float16)(g[0] - (float)wh) : wh;
            x[s][e] = (s & 2) ? (_Float16)(g[1] - (float)xh) : xh;
        }
    }
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int s = 0; s < 8; s += 4) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(w[s], x[s], c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(w[s + 1], x[s + 1], c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(w[s + 2], x[s + 2], c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(w[s + 3], x[s + 3], c3, 0, 0, 0);
        }
    }
    float s = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) s += (c0[r] + c1[r]) + (c2[r] + c3[r]);
    out[(int64_t)blockIdx.x * 256 + threadIdx.x] = s;
}

// Streaming writes: each thread stores 16-byte vectors at a grid stride, so every wave
// writes 1 KiB of consecutive bytes per instruction and the whole buffer is written once.
__global__ __launch_bounds__(256) void write_probe_kernel(float4* __restrict__ dst, int64_t n4, float v) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += stride) dst[i] = make_float4(v, v, v, v);
}

// One probe kernel: 4 workgroups of 4 waves per CU (4 waves per SIMD), `iters` steps of
// 4 (PER_STEP) MFMAs per wave, timed after a shorter warm-up launch.
template <int PER_STEP>
int run_probe(void (*kernel)(float*, int), int iters, double* tflops, double* ms) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 1;
    const int blocks = 4 * cus;
    float* out = nullptr;
    if (hipMalloc(&out, (size_t)blocks * 256 * sizeof(float)) != hipSuccess) return 2;
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    kernel<<<blocks, 256>>>(out, iters / 4 + 1);  // warm-up, clocks up
    (void)hipEventRecord(e0, nullptr);
    kernel<<<blocks, 256>>>(out, iters);
    (void)hipEventRecord(e1, nullptr);
    hipError_t rc = hipEventSynchronize(e1);
    float t = 0.0f;
    if (rc == hipSuccess) rc = hipEventElapsedTime(&t, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    (void)hipFree(out);
    if (rc != hipSuccess) return (int)rc;
    const double flops = (double)blocks * 4.0 * (double)iters * PER_STEP * (32.0 * 32.0 * 16.0 * 2.0);
    *ms = t;
    *tflops = flops / ((double)t * 1e-3) / 1e12;
    return 0;
}

}  // namespace

// Runs the probe on the current device with 4 workgroups of 4 waves per CU (4 waves per
// SIMD) and `iters` steps of 4 MFMAs per wave; returns 0 and the rate in TFLOP/s (2 flops
// per multiply-add) and the kernel time, or the HIP error code.
extern "C" int ppocr_probe_mfma_bf16(int iters, double* tflops, double* ms) {
    return run_probe<4>(mfma_peak_kernel, iters, tflops, ms);
}

// The same with the statistics pass's operand bit patterns (mfma_data_kernel, 8 MFMAs per
// step): the rate its matrix cores can reach under the GPU's power limit.
extern "C" int ppocr_probe_mfma_bf16_data(int iters, double* tflops, double* ms) {
    return run_probe<8>(mfma_data_kernel, iters, tflops, ms);
}

// Dense fp16 MFMA with operands like the SVTR tail's (fp16 halves, mfma_f16_data_kernel, 8
// MFMAs per step): the tail's GEMMs issue three such products per multiply-add.
extern "C" int ppocr_probe_mfma_f16_data(int iters, double* tflops, double* ms) {
    return run_probe<8>(mfma_f16_data_kernel, iters, tflops, ms);
}

// Writes `bytes` (a multiple of 16) to the device buffer `dst` with streaming 16-byte stores
// (8 workgroups of 4 waves per CU, grid-stride), once to warm up and once timed; returns 0,
// the write rate in GB/s and the kernel time, or the HIP error code.
extern "C" int ppocr_probe_write(void* dst, int64_t bytes, double* gbps, double* ms) {
    if (!dst || bytes <= 0 || (bytes & 15) || (reinterpret_cast<uintptr_t>(dst) & 15)) return 1;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 1;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 1;
    const int blocks = 8 * cus;
    float4* d = static_cast<float4*>(dst);
    hipEvent_t e0, e1;
    (void)hipEventCreate(&e0);
    (void)hipEventCreate(&e1);
    write_probe_kernel<<<blocks, 256>>>(d, bytes / 16, 1.0f);  // warm-up, clocks up
    (void)hipEventRecord(e0, nullptr);
    write_probe_kernel<<<blocks, 256>>>(d, bytes / 16, 2.0f);
    (void)hipEventRecord(e1, nullptr);
    hipError_t rc = hipEventSynchronize(e1);
    float t = 0.0f;
    if (rc == hipSuccess) rc = hipEventElapsedTime(&t, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (rc != hipSuccess) return (int)rc;
    *ms = t;
    *gbps = (double)bytes / ((double)t * 1e-3) / 1e9;
    return 0;
}
