// Shared device/host helpers for the recognition-head library (gfx950 only).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/ppocr_rechead.h"

namespace ppocr {

// ---------------------------------------------------------------- error reporting
// Status codes mirror OcrError (src/error.rs:4-27): argument/shape problems are
// OperatorError, runtime failures are device errors.  The message is thread-local.
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);

#define PPOCR_HIP(call)                                                                     \
    do {                                                                                    \
        hipError_t e_ = (call);                                                             \
        if (e_ != hipSuccess)                                                               \
            return ::ppocr::fail(PPOCR_ERR_DEVICE, std::string(#call) + ": " +              \
                                                       hipGetErrorString(e_));              \
    } while (0)

// ---------------------------------------------------------------- device helpers
constexpr float kLog2e = 1.4426950408889634f;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Round half away from zero, exactly (the semantics of C roundf / Rust f32::round):
// trunc, then step away from zero when the dropped fraction is at least one half.
__device__ __forceinline__ float round_half_away(float x) {
#pragma clang fp contract(off)  // d must come from the rounded x, not an fma with its producer
    float t = __builtin_truncf(x);
    float d = x - t;  // exact
    return (__builtin_fabsf(d) >= 0.5f) ? t + __builtin_copysignf(1.0f, x) : t;
}

// One row's online softmax statistics in log2 units: running maximum `best` of
// t = logit*log2(e) with the first index reaching it, and `sum` = sum of
// exp2(t - ref) over the values seen.  `ref` is a shift that stays within 64 of `best`
// so the sum neither overflows nor underflows; it is 0 for ordinary rows.
struct RowStat {
    float best;
    float sum;
    float ref;
    int idx;
};

// Sum of exp2(t - best) of a statistic, i.e. the softmax denominator relative to its
// own maximum.  An empty statistic (best = -inf) contributes nothing.
__device__ __forceinline__ float stat_rel_sum(float best, float sum, float ref) {
    return (best == -INFINITY) ? 0.0f : sum * exp2f(ref - best);
}

// Combine two statistics of the same row (by value, field by field, so nothing is
// forced into memory).  Ties on the maximum keep the lower index, which is the
// first-occurrence rule of find_argmax (src/postprocess/ctc.rs:236-254).  The result
// has ref = best.
__device__ __forceinline__ RowStat stat_merge(RowStat a, RowStat b) {
    const float sa = stat_rel_sum(a.best, a.sum, a.ref);
    const float sb = stat_rel_sum(b.best, b.sum, b.ref);
    const bool take_a = (a.best > b.best) || (a.best == b.best && a.idx <= b.idx);
    RowStat r;
    r.best = take_a ? a.best : b.best;
    r.idx = take_a ? a.idx : b.idx;
    const float m = r.best;
    float s = 0.0f;
    if (a.best != -INFINITY) s += sa * exp2f(a.best - m);
    if (b.best != -INFINITY) s += sb * exp2f(b.best - m);
    r.sum = s;
    r.ref = (m == -INFINITY) ? 0.0f : m;
    return r;
}

// stat_merge of two normalised statistics (ref = best, or best = -inf with sum = 0), as the
// merge of chunk partials sees them: the winner's own term is sum * exp2(0) = sum, so only
// the loser's rescaling needs an exp2 (stat_merge takes four).  The same value as
// stat_merge up to the rounding of the last addition (the loser's term is added to the
// winner's sum, with contraction); non-finite maxima give a NaN sum as there (best - best
// is NaN).  Sums are never -0, so w.sum + 0 = w.sum.
__device__ __forceinline__ RowStat stat_merge_norm(RowStat a, RowStat b) {
    const bool take_a = (a.best > b.best) || (a.best == b.best && a.idx <= b.idx);
    const RowStat w = take_a ? a : b;
    const RowStat l = take_a ? b : a;
    const float m = w.best;
    float s = 0.0f;
    if (w.best != -INFINITY) s = w.sum + (w.best - w.best);
    if (l.best != -INFINITY) s += (l.sum + (l.best - l.best)) * exp2f(l.best - m);
    RowStat r;
    r.best = m;
    r.idx = w.idx;
    r.sum = s;
    r.ref = (m == -INFINITY) ? 0.0f : m;
    return r;
}

}  // namespace ppocr
