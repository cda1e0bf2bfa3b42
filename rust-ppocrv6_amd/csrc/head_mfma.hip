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
    if (nsplit >= 8) return mblocks * nsplit;
    if (rows_on_one_xcd) return ((mblocks + 7) / 8) * nsplit * 8;
    const int r8 = 8 / nsplit;
    return ((mblocks + r8 - 1) / r8) * 8;
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
// tiles of the main loop.  The chunk count from 4 to 64 minimising rounds x (fixed + tiles
// per chunk) is taken.  From 8 chunks up each XCD keeps its slice of the weight records (the
// chunks of workgroup id mod 8) in its L2; with 4, an XCD takes all chunks of its row blocks,
// and its workgroups walk the chunks' tiles in step.  Most kernels run 2 workgroups per CU with
// a fixed cost of 8 tiles (measured: 30720 rows run 5% faster in 4 chunks of 147 tiles,
// one round, than in 8 chunks of 74, two rounds).  The two-term modes' one-block-per-wave
// kernel (small batches: 128-row workgroups, 51 KB of LDS, 148 VGPRs) runs 3 per CU, fixed
// 10 tiles (measured against 2 per CU and 8 tiles: 2280 rows 43.8 -> 40.5 us per step in 32
// chunks instead of 16, 4800 rows 63.5 -> 61.6 in 16 instead of 8; 8160 rows keep 8
// chunks, which the 8-tile estimate would have traded for 32 in three rounds, 84 -> 95 us).
int stats_per_cu_mfma(int cfg, int64_t m) { return main_blocks(cfg, m) == 1 && (cfg == CFG_Q2 || cfg == CFG_H2) ? 3 : 2; }
int stats_nsplit(int64_t m, int rows_per_block, int tiles, int per_cu) {
    const int64_t mblocks = (m + rows_per_block - 1) / rows_per_block;
    const int64_t slots = 256 * (int64_t)per_cu;
    const int64_t fixed = per_cu == 3 ? 10 : 8;
    int best = 4;
    int64_t best_cost = -1;
    for (int ns = 4; ns <= 64; ns *= 2) {
        const int64_t rounds = (mblocks * ns + slots - 1) / slots;
        const int64_t cost = rounds * (fixed + (tiles + ns - 1) / ns);
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
// Precision limits below it make the two-term bf16 main pass skip row blocks whose rows all
// go to the rescue.
constexpr float kVoteLimit = 4.0f;

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
                                 nullptr, nullptr, nullptr, 0, *guard, st);
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
                      int64_t m, int64_t n, int64_t k, int nsplit, float* p_best, float* p_sum, int* p_idx,
                      const Guard* guard, int32_t* idx, float* maxprob, float* row_max, float* row_inv,
                      const CtcOut* ctc, hipStream_t st, int64_t line_len) {
    if (line_len < 0 || line_len > INT32_MAX) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: bad line length");
    if (!check_geom(cfg, tg, n, k)) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: tile geometry mismatch");
    if (nsplit != 1 && nsplit != 2 && nsplit != 4 && nsplit != 8 && nsplit != 16 && nsplit != 32 && nsplit != 64)
        return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: nsplit must be a power of two <= 64");
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
                  p_best,
                  p_sum,
                  p_idx,
                  guarded ? stats_limit_of(cfg, *guard) : GuardLimits{0.0f, 0.0f, 0.0f},
                  guarded ? guard->header : nullptr,
                  guarded ? guard->rows : nullptr,
                  guarded ? guard->epoch : 0u,
                  guarded ? guard->capacity : 0};
    // A precision limit below typical |a| (rows of unit variance reach max|a| ~ 2.5-3.5 over
    // 120 values) sends nearly every row to the rescue: the main pass then votes per row
    // block and skips the blocks it would compute for nothing.  Above the limit the vote
    // would only cost time (0.3% on the dense batch, 2% on one line): the other variant runs.
    x.vote = guarded && cfg == CFG_Q2 && rcfg == CFG_Q3 && guard->amax_limit < kVoteLimit;
    const int mb = rpb / (32 * kStatsWaves);
    if (int e = call_stats_main(cfg, tg.G, x, mb, noref, (unsigned)grid, st)) return e;
    if (guarded && rcfg == kRescueFma) {
        if (int e = launch_rescue_fma(EPI_STATS, guard->fma, a, m, n, k, nsplit, tpc * 32, nullptr, nullptr, nullptr,
                                      p_best, p_sum, p_idx, line_len, *guard, st))
            return e;
    } else if (guarded) {
        // rescue: same vocabulary chunks, so each flagged row's partials are overwritten
        // (with exact class indices)
        const int rrpb = stats_rows_per_block_mfma(rcfg, m);
        const int slots = (int)std::min<int64_t>((m + rrpb - 1) / rrpb, kRescueSlots);
        const int rgrid = grid_blocks(slots, nsplit, true);
        x.rec = rec_rescue;
        x.mblocks = slots;
        x.lim = GuardLimits{0.0f, 0.0f, 0.0f};
        if (int e = call_stats_gather(rcfg, tg.G, x, (unsigned)rgrid, st)) return e;
    }
    const Guard* reset = guarded ? guard : nullptr;
    if (ctc) return launch_merge_ctc(p_best, p_sum, p_idx, m, nsplit, *ctc, idx, maxprob, reset, st);
    return launch_merge_stats(p_best, p_sum, p_idx, m, nsplit, idx, maxprob, row_max, row_inv, reset, st);
}

}  // namespace ppocr
