// Softmax.2 (softmax_inplace, src/ops/softmax.rs:199-285), the per-step argmax of the CTC
// decoder (find_argmax, src/postprocess/ctc.rs:178-258), the merge of the fused head's
// per-chunk statistics, and the CTC collapse (CtcDecoder::decode_batch,
// src/postprocess/ctc.rs:144-172).
#include "kernels.hpp"

namespace ppocr {

namespace {

// (value, index) pair reduction: larger value wins, equal values keep the lower index
// (first occurrence).  NaN never wins because every comparison with it is false.
__device__ __forceinline__ void argmax_pair(float& v, int& i, float ov, int oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(v, o, 64);
        const int oi = __shfl_xor(i, o, 64);
        argmax_pair(v, i, ov, oi);
    }
}

// Block (256 threads) reductions through LDS; every thread gets the result.
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}
__device__ __forceinline__ void block_argmax(float& v, int& i, float* redv, int* redi) {
    wave_argmax(v, i);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
        redv[w] = v;
        redi[w] = i;
    }
    __syncthreads();
    v = redv[0];
    i = redi[0];
#pragma unroll
    for (int j = 1; j < 4; ++j) argmax_pair(v, i, redv[j], redi[j]);
}

// One 256-thread workgroup per row.  Rows up to 256*VPT classes stay in registers, so
// the row is read once and written once.  exp(x - max) is computed as
// exp2((x - max) * log2(e)) on the hardware exp2.
template <int VPT>
__global__ __launch_bounds__(256) void softmax_rows_kernel(float* __restrict__ x, int64_t rows, int cols,
                                                           int32_t* __restrict__ idx,
                                                           float* __restrict__ maxprob) {
    __shared__ float redf[4];
    __shared__ int redi[4];
    const int64_t row = blockIdx.x;
    float* p = x + row * (int64_t)cols;
    const int tid = threadIdx.x;
    float v[VPT];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int c = tid + 256 * j;
        v[j] = c < cols ? p[c] : -INFINITY;
        mx = fmaxf(mx, v[j]);
    }
    mx = block_max(mx, redf);
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int c = tid + 256 * j;
        v[j] = c < cols ? __builtin_amdgcn_exp2f((v[j] - mx) * kLog2e) : 0.0f;
        s += v[j];
    }
    s = block_sum(s, redf);
    const float inv = s > 0.0f ? __fdiv_rn(1.0f, s) : 1.0f;
    float bv = -INFINITY;
    int bi = 0;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const int c = tid + 256 * j;
        if (c < cols) {
            const float pv = v[j] * inv;
            p[c] = pv;
            if (pv > bv) {
                bv = pv;
                bi = c;
            }
        }
    }
    if (idx || maxprob) {
        block_argmax(bv, bi, redf, redi);
        if (tid == 0) {
            if (idx) idx[row] = bi;
            if (maxprob) maxprob[row] = bv;
        }
    }
}

// Rows too long for registers: three passes over global memory.
__global__ __launch_bounds__(256) void softmax_rows_stream_kernel(float* __restrict__ x, int64_t rows,
                                                                  int64_t cols, int32_t* __restrict__ idx,
                                                                  float* __restrict__ maxprob) {
    __shared__ float redf[4];
    __shared__ int redi[4];
    float* p = x + (int64_t)blockIdx.x * cols;
    float mx = -INFINITY;
    for (int64_t c = threadIdx.x; c < cols; c += 256) mx = fmaxf(mx, p[c]);
    mx = block_max(mx, redf);
    float s = 0.0f;
    for (int64_t c = threadIdx.x; c < cols; c += 256) {
        const float e = __builtin_amdgcn_exp2f((p[c] - mx) * kLog2e);
        p[c] = e;
        s += e;
    }
    s = block_sum(s, redf);
    const float inv = s > 0.0f ? __fdiv_rn(1.0f, s) : 1.0f;
    float bv = -INFINITY;
    int bi = 0;
    for (int64_t c = threadIdx.x; c < cols; c += 256) {
        const float pv = p[c] * inv;
        p[c] = pv;
        if (pv > bv) {
            bv = pv;
            bi = (int)c;
        }
    }
    if (idx || maxprob) {
        block_argmax(bv, bi, redf, redi);
        if (threadIdx.x == 0) {
            if (idx) idx[blockIdx.x] = bi;
            if (maxprob) maxprob[blockIdx.x] = bv;
        }
    }
}

__global__ __launch_bounds__(256) void argmax_rows_kernel(const float* __restrict__ x, int64_t cols,
                                                          int32_t* __restrict__ idx, float* __restrict__ val) {
    __shared__ float redf[4];
    __shared__ int redi[4];
    const float* p = x + (int64_t)blockIdx.x * cols;
    float bv = -INFINITY;
    int bi = 0;
    for (int64_t c = threadIdx.x; c < cols; c += 256) {
        const float v = p[c];
        if (v > bv) {
            bv = v;
            bi = (int)c;
        }
    }
    block_argmax(bv, bi, redf, redi);
    if (threadIdx.x == 0) {
        idx[blockIdx.x] = bi;
        val[blockIdx.x] = bv;
    }
}

// A row's statistics merged over its vocabulary chunks: kMergeLanes threads per row,
// thread g taking chunks g, g + kMergeLanes, ... in order (merge_batch), then the eight
// results merged pairwise in a fixed tree (merge_tree8), so every lane of every merge kernel
// that reads the partials produces the same merged statistic (first-index argmax) and
// 1 / sum exp2(t - max) (the maximum probability), bit for bit.  The threads of one load
// instruction take consecutive rows of one chunk (whole runs of records, not 8-row
// pieces of 8 chunks); their statistics meet in LDS.
constexpr int kMergeLanes = 8;
constexpr int kMergeBatch = 8;  // partials per lane loaded together (all of them for nsplit <= 64)
// The partials of one row a lane merges, chunks c0, c0 + 8, ..., loaded before any is used
struct MergeLoad {
    float bv[kMergeBatch], sv[kMergeBatch];
    int iv[kMergeBatch];
};
__device__ __forceinline__ void merge_issue(const Partial* __restrict__ part, int64_t m, int nsplit, int64_t row,
                                            bool valid, int c0, MergeLoad& ld) {
    if (valid) {
#pragma unroll
        for (int x = 0; x < kMergeBatch; ++x) {
            const int c = c0 + x * kMergeLanes;
            if (c < nsplit) {
                const Partial p = part[(int64_t)c * m + row];
                ld.bv[x] = p.best;
                ld.sv[x] = p.sum;
                ld.iv[x] = p.idx;
            }
        }
    }
}
__device__ __forceinline__ void merge_batch(RowStat& s, const MergeLoad& ld, int nsplit, int c0) {
#pragma unroll
    for (int x = 0; x < kMergeBatch; ++x) {
        if (c0 + x * kMergeLanes < nsplit) {
            // partial sums are relative to their own maximum: both operands are normalised
            const RowStat o{ld.bv[x], ld.sv[x], (ld.bv[x] == -INFINITY) ? 0.0f : ld.bv[x], ld.iv[x]};
            s = stat_merge_norm(s, o);
        }
    }
}
// 1 / the row's sum: s.sum is relative to s.best, so the maximum itself contributes
// exp2(0) = 1 and the sum is at least 1 (rounding of the rescaling could leave it an ulp
// below).
__device__ __forceinline__ float merged_inv(const RowStat& s) {
    const float S = (s.best == -INFINITY) ? 0.0f : fmaxf(s.sum, 1.0f);
    return S > 0.0f ? __fdiv_rn(1.0f, S) : 0.0f;
}
// The eight threads' statistics of a row (s[g * stride], g = 0..7) merged as
// ((0,1),(2,3)),((4,5),(6,7)), the lower group first in each pair.
__device__ __forceinline__ RowStat merge_tree8(const RowStat* s, int stride) {
    static_assert(kMergeLanes == 8, "a tree of eight");
    const RowStat m01 = stat_merge_norm(s[0], s[stride]);
    const RowStat m23 = stat_merge_norm(s[2 * stride], s[3 * stride]);
    const RowStat m45 = stat_merge_norm(s[4 * stride], s[5 * stride]);
    const RowStat m67 = stat_merge_norm(s[6 * stride], s[7 * stride]);
    return stat_merge_norm(stat_merge_norm(m01, m23), stat_merge_norm(m45, m67));
}
// Rows per merge_ctc_kernel round (1024 threads) and per merge_stats_kernel workgroup (256
// threads: four workgroups per 128 rows, so a single line's rows load through four CUs;
// each load instruction reads two chunks of 32 consecutive rows).
constexpr int kCtcRound = 1024 / kMergeLanes;
constexpr int kStatRows = 256 / kMergeLanes;
__global__ __launch_bounds__(256) void merge_stats_kernel(const Partial* __restrict__ part, int64_t m, int nsplit,
                                                          int32_t* __restrict__ idx, float* __restrict__ maxprob,
                                                          float* __restrict__ row_max, float* __restrict__ row_inv,
                                                          unsigned long long* __restrict__ guard_header,
                                                          unsigned guard_epoch) {
    __shared__ RowStat s_st[kMergeLanes * kStatRows];  // [g][row of the workgroup]
    const int tid = threadIdx.x, g = tid / kStatRows, step = tid % kStatRows;
    const int64_t row = (int64_t)blockIdx.x * kStatRows + step;
    RowStat s0{-INFINITY, 0.0f, 0.0f, 0};
    if (row < m) {
        for (int c0 = g; c0 < nsplit; c0 += kMergeLanes * kMergeBatch) {
            MergeLoad ld;
            merge_issue(part, m, nsplit, row, true, c0, ld);
            merge_batch(s0, ld, nsplit, c0);
        }
    }
    s_st[g * kStatRows + step] = s0;
    // the guard list of this call is emptied for the next (row 0 exists: m >= 1)
    if (guard_header && row == 0 && g == 0) *guard_header = (unsigned long long)guard_epoch << 32;
    __syncthreads();
    if (row >= m || g != 0) return;
    const RowStat s = merge_tree8(s_st + step, kStatRows);
    const float inv = merged_inv(s);
    if (idx) idx[row] = s.idx;
    if (maxprob) maxprob[row] = inv;
    if (row_max) row_max[row] = s.best;
    if (row_inv) row_inv[row] = inv;
}

// sum + x(lane 0) + x(lane 1) + ... + x(lane 63), added in lane order in f32 (the same
// value in every lane).  A lane that contributes nothing passes -0.0, which is the exact
// identity of IEEE addition (x + -0.0 = x for every x, -0.0 included), so the result is
// bit for bit the sequential sum over the contributing lanes alone.
__device__ __forceinline__ float ordered_lane_sum(float sum, float x) {
    const int xi = __float_as_int(x);
#pragma unroll
    for (int l = 0; l < 64; ++l) sum += __int_as_float(__builtin_amdgcn_readlane(xi, l));
    return sum;
}

// One wavefront per text line.  Steps are taken 64 at a time; the emit mask is a ballot,
// emitted indices are compacted by prefix popcount, and the score is summed in step order
// (every lane runs the same sequential sum over the emitting lanes' values, read lane by
// lane, ordered_lane_sum).  The offsets live on the device and are not trusted: each line
// is clamped into [0, line_off[lines]] (the step count the arrays hold) and a line whose end
// precedes its start is empty, as merge_ctc_kernel does.
__global__ __launch_bounds__(256) void ctc_greedy_kernel(const int32_t* __restrict__ idx,
                                                         const float* __restrict__ val,
                                                         const int64_t* __restrict__ line_off, int64_t lines,
                                                         int32_t blank, int32_t* __restrict__ seq,
                                                         int64_t* __restrict__ seq_len, float* __restrict__ score) {
    const int lane = threadIdx.x & 63;
    const int64_t line = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (line >= lines) return;
    const int64_t total = max(line_off[lines], (int64_t)0);
    const int64_t t0 = min(max(line_off[line], (int64_t)0), total);
    const int64_t t1 = min(max(line_off[line + 1], t0), total);
    int64_t cnt = 0;
    float sum = -0.0f;
    for (int64_t base = t0; base < t1; base += 64) {
        const int64_t t = base + lane;
        const bool valid = t < t1;
        const int32_t id = valid ? idx[t] : blank;
        const int32_t prev = (valid && t > t0) ? idx[t - 1] : blank;
        const bool emit = valid && id != blank && id != prev;
        const float v = valid ? val[t] : 0.0f;
        const uint64_t mask = __ballot(emit);
        const int pos = __popcll(mask & ((1ull << lane) - 1ull));
        if (emit) seq[t0 + cnt + pos] = id;
        sum = ordered_lane_sum(sum, emit ? v : -0.0f);
        cnt += __popcll(mask);
    }
    if (lane == 0) {
        seq_len[line] = cnt;
        score[line] = cnt ? sum / (float)cnt : 0.0f;
    }
}

// The merge of the vocabulary chunks and the CTC collapse in one pass: one workgroup of
// 1024 threads per text line.  The line is taken kCtcRound steps at a time.  Thread
// (g, step) merges chunks g, g + 8, ... of the round's row `step`, so each load instruction
// of a wave reads 64 consecutive rows of one chunk (768 contiguous bytes; 8 chunks of 8 rows
// per instruction read eight 96-byte pieces, about twice the cache lines, and took an A4
// page's step from 32.8 to 34.2 us); the eight statistics of a row meet in LDS and are
// merged by merge_tree8.  Then wave 0 collapses the round as ctc_greedy_kernel does (ballot,
// prefix popcount, score summed in step order), carrying the previous index between
// rounds.  Offsets are clamped into [0, m] (a line with t1 < t0
// is empty); with no offsets, line i is steps i * line_len .. (i + 1) * line_len - 1.
__global__ __launch_bounds__(1024) void merge_ctc_kernel(const Partial* __restrict__ part, int64_t m, int nsplit,
                                                         const int64_t* __restrict__ line_off, int64_t lines,
                                                         int32_t blank, int32_t* __restrict__ idx_out,
                                                         float* __restrict__ val_out, int32_t* __restrict__ seq,
                                                         int64_t* __restrict__ seq_len, float* __restrict__ score,
                                                         unsigned long long* __restrict__ guard_header,
                                                         unsigned guard_epoch, int64_t line_len) {
    __shared__ int32_t s_id[kCtcRound];
    __shared__ float s_v[kCtcRound];
    __shared__ RowStat s_st[kMergeLanes * kCtcRound];  // [g][step]
    const int tid = threadIdx.x, lane = tid & 63, g = tid / kCtcRound, step = tid % kCtcRound;
    const int64_t line = blockIdx.x;
    // The partials are loaded once the line's offsets are known.  Loading the first round's
    // rows at a guessed start meanwhile (the start with equal lines) measured slower even
    // where the guess held: its loads queue beside the real ones (an A4 page of ragged lines
    // 34.5 -> 33.9 us per step without it, four lines of 120 steps 17.4 -> 17.2).
    // both offsets of the line in one wait
    int64_t o0 = line * line_len, o1 = o0 + line_len;
    if (line_off) {
        o0 = line_off[line];
        o1 = line_off[line + 1];
    }
    const int64_t t0 = min(max(o0, (int64_t)0), m);
    const int64_t t1 = line_off ? min(max(o1, t0), m) : min(t0 + line_len, m);
    int64_t cnt = 0;
    float sum = -0.0f;
    int32_t carry = blank;  // index of the step before the current one
    for (int64_t base = t0; base < t1; base += kCtcRound) {
        const int64_t t = base + step;
        RowStat s0{-INFINITY, 0.0f, 0.0f, 0};
        if (t < t1) {
            for (int c0 = g; c0 < nsplit; c0 += kMergeLanes * kMergeBatch) {
                MergeLoad ld;
                merge_issue(part, m, nsplit, t, true, c0, ld);
                merge_batch(s0, ld, nsplit, c0);
            }
        }
        s_st[g * kCtcRound + step] = s0;
        __syncthreads();
        if (g == 0) {
            const RowStat st = merge_tree8(s_st + step, kCtcRound);
            const float v = merged_inv(st);
            const int32_t id = t < t1 ? st.idx : blank;
            if (t < t1) {
                if (idx_out) idx_out[t] = id;
                if (val_out) val_out[t] = v;
            }
            s_id[step] = id;
            s_v[step] = t < t1 ? v : 0.0f;
        }
        __syncthreads();
        if (tid < 64) {
            const int64_t rem = min(t1 - base, (int64_t)kCtcRound);
            for (int c0 = 0; c0 < rem; c0 += 64) {
                const bool valid = c0 + lane < rem;
                const int32_t cid = valid ? s_id[c0 + lane] : blank;
                const float cv = valid ? s_v[c0 + lane] : 0.0f;
                const int32_t prev = (c0 + lane == 0) ? carry : s_id[c0 + lane - 1];
                const bool emit = valid && cid != blank && cid != prev;
                const uint64_t mask = __ballot(emit);
                const int pos = __popcll(mask & ((1ull << lane) - 1ull));
                if (emit) seq[t0 + cnt + pos] = cid;
                sum = ordered_lane_sum(sum, emit ? cv : -0.0f);
                cnt += __popcll(mask);
            }
            carry = s_id[rem - 1];
        }
        __syncthreads();
    }
    if (tid == 0) {
        seq_len[line] = cnt;
        score[line] = cnt ? sum / (float)cnt : 0.0f;
        // the guard list of this call is emptied for the next (written last, so the
        // kernel's first loads do not wait behind it)
        if (guard_header && line == 0) *guard_header = (unsigned long long)guard_epoch << 32;
    }
}

}  // namespace

int launch_softmax_rows(float* x, int64_t rows, int64_t cols, int32_t* idx, float* maxprob, hipStream_t st) {
    if (rows < 0 || cols < 0) return fail(PPOCR_ERR_INVALID_ARG, "Softmax: negative shape");
    if (rows == 0 || cols == 0) return PPOCR_OK;
    if (rows > 0x7fffffffLL || cols > 0x7fffffffLL) return fail(PPOCR_ERR_INVALID_ARG, "Softmax: shape too large");
    if (cols <= 256 * 8)
        softmax_rows_kernel<8><<<(unsigned)rows, 256, 0, st>>>(x, rows, (int)cols, idx, maxprob);
    else if (cols <= 256 * 80)
        softmax_rows_kernel<80><<<(unsigned)rows, 256, 0, st>>>(x, rows, (int)cols, idx, maxprob);
    else
        softmax_rows_stream_kernel<<<(unsigned)rows, 256, 0, st>>>(x, rows, cols, idx, maxprob);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

int launch_argmax_rows(const float* x, int64_t rows, int64_t cols, int32_t* idx, float* val, hipStream_t st) {
    if (rows < 0 || cols < 0) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: negative shape");
    if (rows == 0) return PPOCR_OK;
    if (rows > 0x7fffffffLL || cols > 0x7fffffffLL) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: shape too large");
    argmax_rows_kernel<<<(unsigned)rows, 256, 0, st>>>(x, cols, idx, val);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

int launch_merge_stats(const Partial* part, int64_t m, int nsplit,
                       int32_t* idx, float* maxprob, float* row_max, float* row_inv, const Guard* guard,
                       hipStream_t st) {
    if (m <= 0) return PPOCR_OK;
    const int64_t blocks = (m + kStatRows - 1) / kStatRows;
    if (blocks > 0x7fffffffLL) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: m too large");
    merge_stats_kernel<<<(unsigned)blocks, 256, 0, st>>>(part, m, nsplit, idx, maxprob, row_max,
                                                         row_inv, guard ? guard->header : nullptr,
                                                         guard ? guard->epoch : 0u);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

int launch_ctc_greedy(const int32_t* idx, const float* maxprob, const int64_t* line_off, int64_t lines,
                      int32_t blank, int32_t* seq, int64_t* seq_len, float* score, hipStream_t st) {
    if (lines < 0) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: negative line count");
    if (lines == 0) return PPOCR_OK;
    const int64_t blocks = (lines + 3) / 4;
    if (blocks > 0x7fffffffLL) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: too many lines");
    ctc_greedy_kernel<<<(unsigned)blocks, 256, 0, st>>>(idx, maxprob, line_off, lines, blank, seq, seq_len, score);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

int launch_merge_ctc(const Partial* part, int64_t m, int nsplit,
                     const CtcOut& ctc, int32_t* idx, float* maxprob, const Guard* guard, hipStream_t st) {
    if (ctc.lines < 0) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: negative line count");
    if (ctc.lines == 0) return PPOCR_OK;
    if (ctc.lines > 0x7fffffffLL) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: too many lines");
    merge_ctc_kernel<<<(unsigned)ctc.lines, 1024, 0, st>>>(part, m, nsplit, ctc.line_off, ctc.lines,
                                                       ctc.blank, idx, maxprob, ctc.seq, ctc.seq_len, ctc.score,
                                                       guard ? guard->header : nullptr, guard ? guard->epoch : 0u,
                                                       ctc.line_len);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

}  // namespace ppocr
