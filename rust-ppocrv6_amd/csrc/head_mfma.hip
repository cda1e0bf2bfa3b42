// Host side of the MFMA projection kernels (head_mfma.hpp, instantiated in head_cfg_*.hip):
// grid shapes, the vocabulary-chunk model, the precision guard's rescue passes and the
// dispatch of each call to the kernels of its arithmetic configuration.
#include <algorithm>
#include <utility>

#include "kernels.hpp"

namespace ppocr {

bool mfma_supports_groups(int G) { return G == 15 || G == 10; }

// Grid of row blocks x vocabulary chunks, laid out as map_block<rows_on_one_xcd> reads it
// (workgroup id mod 8 is the XCD a workgroup lands on).
static int grid_blocks(int mblocks, int nsplit, bool rows_on_one_xcd) {
    if (nsplit >= 8) return mblocks * 8 * ((nsplit + 7) / 8);
    if (rows_on_one_xcd) return ((mblocks + 7) / 8) * nsplit * 8;
    const int r8 = 8 / nsplit;
    return ((mblocks + r8 - 1) / r8) * 8;
}

// Row blocks of the statistics pass whose rows the guard surely sends to the rescue: each
// row's max|a| (exact, as the pass computes it) and sum of squares in fp64 (exact products),
// and the row is sure when max|a| > prec, or max|a| > range_amax and the sum exceeds
// range_ss by 1e-4 (the pass sums the squares in fp32 in its own order, within 1e-5 of the
// exact sum for k <= 120): a sure row is one the pass's own test flags.  A block of sure rows
// is marked in skip and its rows listed here (one atomic per workgroup); the pass then skips
// the block, and lists the flagged rows of the other blocks itself.  A NaN never makes a row
// sure.  Rows [rows][k]: eight lanes per row, eight consecutive rows per wave and load, so a
// wave reads whole lines of 8 x 4k bytes; channels-first rows ([lines][k][T], vec = -T): one
// thread per row, consecutive rows being consecutive floats of each channel.
__device__ __forceinline__ bool guard_sure(float amax, double ss, const GuardLimits& lim) {
    return amax > lim.prec || (amax > lim.range_amax && ss > (double)lim.range_ss * (1.0 + 1e-4));
}

// Rows [rows][k], k <= 128, of one workgroup of guard_scan_kernel: a lane reads columns
// 4 sub + 32 j (V4: float4) or sub + 8 j (scalars) of two rows, every load issued (at a clamped
// address) before the first use and the values outside the rows zeroed after it.
template <bool V4>
__device__ __forceinline__ bool guard_scan_rows(const float* __restrict__ a, int64_t m, int k,
                                                const GuardLimits& lim, int rpb, int64_t row0, int tid) {
    const int sub = tid & 7;                             // lane within the row's eight
    const int r_in = (tid >> 6) * 8 + ((tid >> 3) & 7);  // wave w reads rows 8w..8w+7 of each 32
    bool sure = true;
    for (int i = 0; i < rpb; i += 64) {
        float v[2][16];
        bool live[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int64_t row = row0 + i + 32 * h + r_in;
            live[h] = i + 32 * h + r_in < rpb && row < m;
            const float* rp = a + (live[h] ? row : row0) * (int64_t)k;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if constexpr (V4) {
                    const int c = min(4 * sub + 32 * j, k - 4);
                    const float4 x = *reinterpret_cast<const float4*>(rp + c);
                    v[h][4 * j] = x.x;
                    v[h][4 * j + 1] = x.y;
                    v[h][4 * j + 2] = x.z;
                    v[h][4 * j + 3] = x.w;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[h][4 * j + e] = rp[min(sub + 32 * j + 8 * e, k - 1)];
                }
            }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float amax = 0.0f;
            double ss = 0.0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int c = V4 ? 4 * sub + 32 * j + e : sub + 32 * j + 8 * e;
                    const float x = c < k ? v[h][4 * j + e] : 0.0f;
                    amax = fmaxf(amax, __builtin_fabsf(x));
                    ss = fma((double)x, (double)x, ss);
                }
            }
            // the eight lanes of a row are consecutive, and every lane takes part in the shuffles
#pragma unroll
            for (int o = 1; o < 8; o <<= 1) {
                amax = fmaxf(amax, __shfl_xor(amax, o, 64));
                ss += __shfl_xor(ss, o, 64);
            }
            if (live[h]) sure = sure && guard_sure(amax, ss, lim);
        }
    }
    return sure;
}

__global__ __launch_bounds__(256) void guard_scan_kernel(const float* __restrict__ a, int64_t m, int k, int vec,
                                                         GuardLimits lim, int rpb, uint8_t* __restrict__ skip,
                                                         unsigned long long* __restrict__ guard_header,
                                                         int* __restrict__ guard_rows, unsigned epoch, int capacity) {
    __shared__ unsigned s_base;
    const int64_t blk = blockIdx.x;
    const int tid = threadIdx.x;
    const int64_t row0 = blk * rpb;
    bool sure = true;  // rows past the batch do not hold a block back
    if (vec < 0) {
        const int64_t row = row0 + tid;
        if (tid < rpb && row < m) {
            const int64_t T = -(int64_t)vec;
            const int64_t line = row / T;
            const float* rp = a + line * T * k + (row - line * T);
            float amax = 0.0f;
            double ss = 0.0;
            for (int kk = 0; kk < k; ++kk) {
                const float x = rp[kk * T];
                amax = fmaxf(amax, __builtin_fabsf(x));
                ss = fma((double)x, (double)x, ss);
            }
            sure = guard_sure(amax, ss, lim);
        }
    } else if (vec > 0) {
        sure = guard_scan_rows<true>(a, m, k, lim, rpb, row0, tid);
    } else {
        sure = guard_scan_rows<false>(a, m, k, lim, rpb, row0, tid);
    }
    if (!__syncthreads_and(sure ? 1 : 0)) {
        if (tid == 0) skip[blk] = 0;
        return;
    }
    if (tid == 0) {
        const int64_t nrows = min((int64_t)rpb, m - row0);
        unsigned long long cur = __hip_atomic_load(guard_header, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        while ((unsigned)(cur >> 32) != epoch) {
            const unsigned long long prev = atomicCAS(guard_header, cur, (unsigned long long)epoch << 32);
            if (prev == cur) break;
            cur = prev;  // another workgroup changed it first; look again
        }
        s_base = (unsigned)atomicAdd(guard_header, (unsigned long long)nrows);
        skip[blk] = 1;
    }
    __syncthreads();
    const int64_t row = row0 + tid;
    if (tid < rpb && row < m) {
        const int pos = (int)(s_base + (unsigned)tid);
        if (pos >= 0 && pos < capacity) guard_rows[pos] = (int)row;
    }
}

// Sets the guard list's header to (epoch, 0) before a pass that is not followed by a merge.
__global__ void guard_reset_kernel(unsigned long long* guard_header, unsigned epoch) {
    *guard_header = (unsigned long long)epoch << 32;
}

// ============================================================ launchers
// Small batches of the two-term mode run one block per wave instead: the workgroup's rows
// (128) are then mostly real rows, and its per-tile work halves (measured on the MI355X:
// one 120-row line 0.033 -> 0.027 ms, a 2245-row page 0.051 -> 0.050 ms; 30720 rows
// 0.259 -> 0.295 ms, so large batches keep two blocks).
constexpr int64_t kSmallBatchRows = 8192;
// 32-row blocks per wave of the main statistics pass: two for the one- and two-term modes
// (each weight fragment read from LDS serves both), one for three products (registers).
static int main_blocks(int cfg, int64_t m) {
    if (cfg == CFG_Q2 || cfg == CFG_H2) return m <= kSmallBatchRows ? 1 : 2;
    return (cfg == CFG_Q1 || cfg == CFG_F1) ? 2 : 1;
}

// Rows per workgroup of the main statistics pass for a batch of m rows, and of the rescue
// pass (4 waves).
int stats_rows_per_block_mfma(int cfg, int64_t m) { return 32 * kStatsWaves * main_blocks(cfg, m); }

// Vocabulary chunks per row block.  The grid runs in rounds of `slots` workgroups (those
// that fit on the 256 CUs of an MI355X at once), and a workgroup costs a fixed start and
// finish (its rows' activations, the pipeline fill, the partials) worth about `fixed`
// tiles of the main loop.  The chunk count minimising rounds x (fixed + tiles per chunk)
// is taken, from 4, 8, 16, 32, 64, 128 and, when the grid fits in one round, the multiples
// of 8 between them (2245 rows: 39 chunks of 15 tiles instead of 32 of 19, 37.2 -> 35.9 us
// per step), without empty chunks; above 64 only for grids of at most a workgroup per CU.  From 8 chunks up each XCD keeps its slice of the weight
// records (the chunks of workgroup id mod 8) in its L2; with 4, an XCD takes all chunks of
// its row blocks, and its workgroups walk the chunks' tiles in step.  Most kernels run 2
// workgroups per CU with a fixed cost of 8 tiles (measured: 30720 rows run 5% faster in 4
// chunks of 147 tiles, one round, than in 8 chunks of 74, two rounds).  The two-term modes'
// one-block-per-wave kernel (small batches: 128-row workgroups, 51 KB of LDS, 154 VGPRs) runs 3 per CU, fixed
// 10 tiles (measured against 2 per CU and 8 tiles: 2280 rows 43.8 -> 40.5 us per step in 32
// chunks instead of 16, 4800 rows 63.5 -> 61.6 in 16 instead of 8; 8160 rows keep 8
// chunks, which the 8-tile estimate would have traded for 32 in three rounds, 84 -> 95 us).
// Most vocabulary chunks of the statistics pass.
constexpr int kMaxChunks = 128;
int stats_per_cu_mfma(int cfg, int64_t m) { return main_blocks(cfg, m) == 1 && (cfg == CFG_Q2 || cfg == CFG_H2) ? 3 : 2; }
int stats_nsplit(int64_t m, int rows_per_block, int tiles, int per_cu) {
    const int64_t mblocks = (m + rows_per_block - 1) / rows_per_block;
    const int64_t xcd_slots = 32 * (int64_t)per_cu;
    const int64_t fixed = per_cu == 3 ? 10 : 8;
    int best = 4;
    int64_t best_cost = -1;
    for (int cand = 4; cand <= kMaxChunks; cand += cand < 8 ? 4 : 8) {
        // the chunks that hold tiles (no empty one; below 8 a count that divides 8, empty
        // chunks included), and their tiles as the kernels split them
        int ns = (tiles + (tiles + cand - 1) / cand - 1) / ((tiles + cand - 1) / cand);
        if (ns < 8) ns = ns <= 1 ? 1 : ns <= 2 ? 2 : ns <= 4 ? 4 : 8;
        const int tpc = (tiles + ns - 1) / ns;
        // workgroups per XCD: a row block's ceil(ns / 8) chunk slots there, or (fewer than 8
        // chunks) all chunks of every 8th row block
        const int64_t per_xcd = ns >= 8 ? mblocks * ((ns + 7) / 8) : (mblocks + 7) / 8 * ns;
        const int64_t rounds = (per_xcd + xcd_slots - 1) / xcd_slots;
        const int64_t cost = rounds * (fixed + tpc);
        // counts between the powers of two only in one round, where every CU's share is set
        // by the grid (over several rounds the estimate favoured them wrongly: 8160 rows 78.4
        // -> 84.5 us in 24 chunks, two rounds, against 8 in one)
        if ((cand & (cand - 1)) != 0 && rounds > 1) continue;
        // more than 64 chunks only for grids of at most one workgroup per CU (a line or two):
        // the merge then reads its rows' partials in two batches, which the estimate leaves
        // out (one line: 59 chunks 16.4 us per step, 117 chunks 15.2, 147 chunks 15.7)
        if (ns > 64 && per_xcd > 32) continue;
        if (best_cost < 0 || cost < best_cost) {
            best = ns;
            best_cost = cost;
        }
    }
    return best;
}

// The kernels of configuration cfg for group count G (k = 8G - 7 .. 8G).
static int call_stats_main(int cfg, int G, const StatsLaunch& x, int mb, bool noref, unsigned grid, hipStream_t st) {
#define PPOCR_CASE(CC, GG) \
    if (cfg == CC && G == GG) return stats_main_cfg<CC, GG>(x, mb, noref, grid, st);
    PPOCR_CASE(CFG_Q1, 15) PPOCR_CASE(CFG_Q2, 15) PPOCR_CASE(CFG_Q3, 15) PPOCR_CASE(CFG_F1, 15)
    PPOCR_CASE(CFG_F3, 15) PPOCR_CASE(CFG_H2, 15) PPOCR_CASE(CFG_HF3, 15)
    PPOCR_CASE(CFG_Q1, 10) PPOCR_CASE(CFG_Q2, 10) PPOCR_CASE(CFG_Q3, 10) PPOCR_CASE(CFG_F1, 10)
    PPOCR_CASE(CFG_F3, 10) PPOCR_CASE(CFG_H2, 10) PPOCR_CASE(CFG_HF3, 10)
#undef PPOCR_CASE
    return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: no MFMA kernel for this k / mode");
}
static int call_rows(int cfg, int G, bool gather, const RowsLaunch& x, int epi, unsigned grid, hipStream_t st) {
    if (gather) {
        if (cfg == CFG_Q3 && G == 15) return rows_cfg<CFG_Q3, 15, true>(x, epi, grid, st);
        if (cfg == CFG_Q3 && G == 10) return rows_cfg<CFG_Q3, 10, true>(x, epi, grid, st);
        return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: no rescue kernel for this k / mode");
    }
#define PPOCR_CASE(CC, GG) \
    if (cfg == CC && G == GG) return rows_cfg<CC, GG, false>(x, epi, grid, st);
    PPOCR_CASE(CFG_Q1, 15) PPOCR_CASE(CFG_Q2, 15) PPOCR_CASE(CFG_Q3, 15) PPOCR_CASE(CFG_F1, 15)
    PPOCR_CASE(CFG_F3, 15) PPOCR_CASE(CFG_H2, 15) PPOCR_CASE(CFG_HF3, 15)
    PPOCR_CASE(CFG_Q1, 10) PPOCR_CASE(CFG_Q2, 10) PPOCR_CASE(CFG_Q3, 10) PPOCR_CASE(CFG_F1, 10)
    PPOCR_CASE(CFG_F3, 10) PPOCR_CASE(CFG_H2, 10) PPOCR_CASE(CFG_HF3, 10)
#undef PPOCR_CASE
    return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: no MFMA kernel for this k / mode");
}
static int call_stats_gather(int cfg, int G, const StatsLaunch& x, unsigned grid, hipStream_t st) {
    if (cfg == CFG_Q3 && G == 15) return stats_gather_cfg<CFG_Q3, 15>(x, grid, st);
    if (cfg == CFG_Q3 && G == 10) return stats_gather_cfg<CFG_Q3, 10>(x, grid, st);
    return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: no rescue kernel for this k / mode");
}

static bool check_geom(int cfg, const TileGeom& tg, int64_t n, int64_t k) {
    const int wpl = cfg_is_fp32_head(cfg) ? 2 : 1;
    return tg.wplanes == wpl && k >= 1 && k <= 8LL * tg.G && tg.tiles == (int)((n + 31) / 32) &&
           mfma_supports_groups(tg.G);
}

// Rows of a are 16-byte aligned and hold whole float4s: fragments load as float4 pairs.
static int vec_ok(const float* a, int64_t k) {
    return ((reinterpret_cast<uintptr_t>(a) & 15) == 0 && (k & 3) == 0) ? 1 : 0;
}

// Vocabulary chunks of the writer (128-row workgroups, one per CU).  HBM write bandwidth
// falls with the number of row segments written at once (measured on the logits layout,
// 30720 x 18710 fp32: 4.3 TB/s with one chunk per row, 3.0 with two, 2.6 with eight), so a
// batch with enough rows to fill the GPU walks each row's vocabulary in one pass; small
// batches split the vocabulary to fill it.
static int rows_nsplit(int64_t mblocks) {
    int ns = 1;
    while (mblocks * ns < 192 && ns < 64) ns *= 2;
    return ns;
}

// Row-block slots of a rescue pass: its grid is sized before the number of guarded rows
// is known (it is on the device); each slot walks the row list in strides.  An empty
// rescue costs the launch whatever the grid, and a heavy one (a head with large weight
// outliers guards many rows) needs the whole GPU.
constexpr int kRescueSlots = 128;
// Workgroups of a statistics rescue: one round of the GPU at the three-term pass's two
// workgroups per CU.  A larger grid walks no more blocks at once (a full list of 18 blocks
// in 64 chunks takes three rounds either way) and an empty list still dispatches all of it.
constexpr int kRescueGrid = 2 * 256;
// Precision limits below it make the two-term bf16 main pass skip the row blocks whose rows
// all go to the rescue (guard_scan_kernel marks them).
constexpr float kScanLimit = 4.0f;

// How the rows flagged by the precision guard of `cfg` are recomputed: an INT8 head's two
// activation terms become three bf16 terms (exact products with int8 weights); an FP32
// head's three products, whose error floor is the two-plane split of the weight itself, are
// redone in fp32 FMA.  Other configurations have no guard.
constexpr int kRescueNone = -1, kRescueFma = -2;
static int rescue_cfg(int cfg) {
    if (cfg == CFG_Q2 || cfg == CFG_H2) return CFG_Q3;
    if (cfg == CFG_F3 || cfg == CFG_HF3) return kRescueFma;
    return kRescueNone;
}

// The statistics pass of the two-term INT8 mode skips the reference shift of the softmax
// sum (NOREF) when the head allows it, flagging also the rows whose logits are not proven
// to lie in [-kLogitBound, kLogitBound] (the range limits of GuardLimits).
static bool stats_noref_of(int cfg, const Guard& g) { return g.stats_noref && (cfg == CFG_Q2 || cfg == CFG_H2); }
static GuardLimits stats_limit_of(int cfg, const Guard& g) {
    if (stats_noref_of(cfg, g)) return GuardLimits{g.amax_limit, g.range_amax_limit, g.range_ss_limit};
    return GuardLimits{g.amax_limit, INFINITY, INFINITY};
}

static int launch_rows(int cfg, int epi, const TileGeom& tg, const uint8_t* rec, const uint8_t* rec_rescue,
                       const float* a, int64_t m, int64_t n, int64_t k, const float* row_max, const float* row_inv,
                       float* out, const Guard* guard, hipStream_t st) {
    if (!check_geom(cfg, tg, n, k)) return fail(PPOCR_ERR_INVALID_ARG, "MatMulQuantizedB: tile geometry mismatch");
    if (m <= 0 || n <= 0) return PPOCR_OK;
    constexpr int ROWS = 32 * kWriterWaves;
    const int64_t mblocks = (m + ROWS - 1) / ROWS;
    if (mblocks > (1 << 24)) return fail(PPOCR_ERR_INVALID_ARG, "MatMulQuantizedB: m too large");
    const int nsplit = rows_nsplit(mblocks);
    const int tpc = (tg.tiles + nsplit - 1) / nsplit;
    const int64_t grid = grid_blocks((int)mblocks, nsplit, false);
    if (grid > 0x7fffffff) return fail(PPOCR_ERR_INVALID_ARG, "MatMulQuantizedB: m too large");
    const int vec = vec_ok(a, k);
    const int rcfg = rescue_cfg(cfg);
    const bool guarded = guard && guard->header && rcfg != kRescueNone;
    // Probabilities are exp2(t - row_max) * row_inv with row_max and row_inv from the
    // statistics pass, so this pass must compute every t exactly as that pass did: the
    // same rows take the rescue (that pass's limit, the lower one when it skips the
    // reference shift).  Logits need only the precision limit.
    const GuardLimits none{0.0f, 0.0f, 0.0f};
    const GuardLimits limit = !guarded ? none
                              : epi == 1 ? stats_limit_of(cfg, *guard)
                                         : GuardLimits{guard->amax_limit, INFINITY, INFINITY};
    if (guarded) {
        // a replay of this call (same epoch) must start from an empty list too
        guard_reset_kernel<<<1, 1, 0, st>>>(guard->header, guard->epoch);
        PPOCR_HIP(hipGetLastError());
    }
    RowsLaunch x{a,
                 m,
                 (int)k,
                 vec,
                 rec,
                 tg.tiles,
                 (int)n,
                 nsplit,
                 tpc,
                 (int)mblocks,
                 row_max,
                 row_inv,
                 out,
                 limit,
                 guarded ? guard->header : nullptr,
                 guarded ? guard->rows : nullptr,
                 guarded ? guard->epoch : 0u,
                 guarded ? guard->capacity : 0};
    if (int e = call_rows(cfg, tg.G, false, x, epi, (unsigned)grid, st)) return e;
    if (!guarded) return PPOCR_OK;
    if (rcfg == kRescueFma)
        return launch_rescue_fma(epi == 0 ? EPI_LOGITS : EPI_PROBS, guard->fma, a, m, n, k, 0, 0, out, row_max, row_inv,
                                 nullptr, 0, *guard, st);
    // rescue: the flagged rows again, three bf16 activation terms, every column
    const int slots = (int)std::min<int64_t>(mblocks, kRescueSlots);
    const int rgrid = grid_blocks(slots, nsplit, false);
    x.rec = rec_rescue;
    x.mblocks = slots;
    x.lim = none;
    x.guard_header = guard->header;
    x.guard_rows = guard->rows;
    x.guard_epoch = guard->epoch;
    x.guard_cap = guard->capacity;
    return call_rows(rcfg, tg.G, true, x, epi, (unsigned)rgrid, st);
}

int launch_guard_clear(unsigned long long* guard_header, hipStream_t st) {
    guard_reset_kernel<<<1, 1, 0, st>>>(guard_header, 0u);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

int launch_logits_mfma(int cfg, const TileGeom& tg, const uint8_t* rec, const uint8_t* rec_rescue, const float* a,
                       int64_t m, int64_t n, int64_t k, float* out, const Guard* guard, hipStream_t st) {
    return launch_rows(cfg, 0, tg, rec, rec_rescue, a, m, n, k, nullptr, nullptr, out, guard, st);
}

int launch_probs_mfma(int cfg, const TileGeom& tg, const uint8_t* rec, const uint8_t* rec_rescue, const float* a,
                      int64_t m, int64_t n, int64_t k, const float* row_max, const float* row_inv, float* probs,
                      const Guard* guard, hipStream_t st) {
    return launch_rows(cfg, 1, tg, rec, rec_rescue, a, m, n, k, row_max, row_inv, probs, guard, st);
}

int launch_stats_mfma(int cfg, const TileGeom& tg, const uint8_t* rec, const uint8_t* rec_rescue, const float* a,
                      int64_t m, int64_t n, int64_t k, int nsplit, Partial* part,
                      const Guard* guard, int32_t* idx, float* maxprob, float* row_max, float* row_inv,
                      const CtcOut* ctc, hipStream_t st, int64_t line_len) {
    if (line_len < 0 || line_len > INT32_MAX) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: bad line length");
    if (!check_geom(cfg, tg, n, k)) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: tile geometry mismatch");
    if (nsplit != 1 && nsplit != 2 && nsplit != 4 && (nsplit < 8 || nsplit > kMaxChunks))
        return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: nsplit must be 1, 2, 4 or 8..128");
    if (m <= 0) return PPOCR_OK;
    const int rpb = stats_rows_per_block_mfma(cfg, m);
    const int64_t mblocks = (m + rpb - 1) / rpb;
    if (mblocks > (1 << 24)) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: m too large");
    const int tpc = (tg.tiles + nsplit - 1) / nsplit;
    const int grid = grid_blocks((int)mblocks, nsplit, true);
    const int vec = line_len > 0 ? -(int)line_len : vec_ok(a, k);
    const int rcfg = rescue_cfg(cfg);
    // No reset launch: the list is emptied by its epoch (first use) and by the merge below.
    const bool guarded = guard && guard->header && rcfg != kRescueNone;
    // With the guard, rows whose logits could leave [-kLogitBound, kLogitBound] go to the
    // rescue pass, so the main pass may skip the reference shift (NOREF; built for the
    // two-term INT8 modes).
    const bool noref = guarded && stats_noref_of(cfg, *guard);
    StatsLaunch x{a,
                  m,
                  (int)k,
                  vec,
                  rec,
                  tg.tiles,
                  nsplit,
                  tpc,
                  (int)mblocks,
                  part,
                  guarded ? stats_limit_of(cfg, *guard) : GuardLimits{0.0f, 0.0f, 0.0f},
                  guarded ? guard->header : nullptr,
                  guarded ? guard->rows : nullptr,
                  guarded ? guard->epoch : 0u,
                  guarded ? guard->capacity : 0};
    // A precision limit below typical |a| (rows of unit variance reach max|a| ~ 2.5-3.5 over
    // 120 values) sends nearly every row to the rescue: a scan then marks the row blocks whose
    // rows are all surely rescued, and the main pass skips them instead of computing them for
    // nothing.  Above the limit whole blocks are not flagged, and the scan would only cost
    // time: the plain main pass runs.
    if (guarded && cfg == CFG_Q2 && rcfg == CFG_Q3 && guard->amax_limit < kScanLimit && guard->skip && rpb <= 256 &&
        rpb % 32 == 0 && k <= 128) {
        guard_scan_kernel<<<(unsigned)mblocks, 256, 0, st>>>(a, m, (int)k, vec, x.lim, rpb, guard->skip, guard->header,
                                                            guard->rows, guard->epoch, guard->capacity);
        PPOCR_HIP(hipGetLastError());
        x.skip = guard->skip;
    }
    const int mb = rpb / (32 * kStatsWaves);
    // one block per wave (small batches) of the two-term modes: the main pass recomputes its
    // flagged rows itself, in three bf16 terms, and no rescue is launched
    // (its three-term pass holds about 220 registers, two workgroups per CU: used when the
    // grid fits on the GPU at that occupancy, a single line and a few lines)
    const bool fused = guarded && rcfg == CFG_Q3 && (cfg == CFG_Q2 || cfg == CFG_H2) && mb == 1 && !x.skip &&
                       grid <= 2 * 256;
    if (fused) x.rec3 = rec_rescue;
    if (int e = call_stats_main(cfg, tg.G, x, mb, noref, (unsigned)grid, st)) return e;
    if (fused) {
        // the list stays empty; the merge below resets its header as after a rescue
    } else if (guarded && rcfg == kRescueFma) {
        if (int e = launch_rescue_fma(EPI_STATS, guard->fma, a, m, n, k, nsplit, tpc * 32, nullptr, nullptr, nullptr,
                                      part, line_len, *guard, st))
            return e;
    } else if (guarded) {
        // rescue: same vocabulary chunks, so each flagged row's partials are overwritten
        // (with exact class indices)
        const int rrpb = stats_rows_per_block_mfma(rcfg, m);
        const int slots = (int)std::min<int64_t>({(m + rrpb - 1) / rrpb, (int64_t)kRescueSlots,
                                                  (int64_t)std::max(1, kRescueGrid / nsplit)});
        const int rgrid = grid_blocks(slots, nsplit, true);
        x.rec = rec_rescue;
        x.mblocks = slots;
        x.lim = GuardLimits{0.0f, 0.0f, 0.0f};
        if (int e = call_stats_gather(rcfg, tg.G, x, (unsigned)rgrid, st)) return e;
    }
    const Guard* reset = guarded ? guard : nullptr;
    if (ctc) return launch_merge_ctc(part, m, nsplit, *ctc, idx, maxprob, reset, st);
    return launch_merge_stats(part, m, nsplit, idx, maxprob, row_max, row_inv, reset, st);
}

}  // namespace ppocr
