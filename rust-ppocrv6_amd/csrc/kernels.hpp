// Launch wrappers of the recognition-head kernels (host side).  Every wrapper checks
// the shapes its grid assumes before it launches and returns a PPOCR_* status.
#pragma once
#include "common.hpp"

namespace ppocr {

// ---------------------------------------------------------------- tile records
// The projection weights live in HBM as one record per 32-class tile:
//   [plane][group g][row i][8 x 16 bit]  weight fragments, g = k / 8 (bf16 or fp16)
//   [4][32] f32                          scale*log2e, bias*log2e, scale, bias
// A head holds two record sets with the same layout: bf16 fragments (the BF16Xn modes) and
// fp16 fragments (F16X2).
// Rows past n hold zero weights, scale 0, bias 0 and bias*log2e = -inf, so they never
// win a maximum and add exp2(-inf) = 0 to a softmax sum.
struct TileGeom {
    int G;        // groups of 8 along k (k <= 8*G)
    int wplanes;  // 1 for an INT8 head (q as bf16), 2 for an FP32 head (hi, lo)
    int tiles;    // ceil(n / 32)
    size_t frag_bytes() const { return (size_t)wplanes * G * 512; }
    size_t rec_bytes() const { return frag_bytes() + 512; }
};

// Arithmetic configurations of the MFMA kernels: which activation term multiplies which
// weight plane in each of the K-concatenated products, in bf16 (Q*, F*) or fp16 (H*).
//   Q1, Q2, Q3   INT8 head, 1 / 2 / 3 bf16 activation terms
//   F1, F3       FP32 head (two bf16 weight planes): a0*w0; a0*w0 + a0*w1 + a1*w0
//   H2           INT8 head, 2 fp16 activation terms
//   HF3          FP32 head, a0*w0 + a0*w1 + a1*w0 with fp16 halves
enum Cfg : int { CFG_Q1 = 0, CFG_Q2 = 1, CFG_Q3 = 2, CFG_F1 = 3, CFG_F3 = 4, CFG_H2 = 5, CFG_HF3 = 6 };
inline bool cfg_is_f16(int cfg) { return cfg == CFG_H2 || cfg == CFG_HF3; }
inline bool cfg_is_fp32_head(int cfg) { return cfg == CFG_F1 || cfg == CFG_F3 || cfg == CFG_HF3; }

// Which rows a pass of a split mode sends to the rescue: max|a| > prec (the precision
// limit), or, when the pass skips the softmax's reference shift, rows whose logits are not
// proven to lie in [-kLogitBound, kLogitBound]: max|a| > range_amax (the bound
// max|a| * max_c ||w_c||_1) and ||a||_2^2 > range_ss (the bound ||a||_2 * max_c ||w_c||_2,
// Cauchy-Schwarz).  Infinite limits send nothing.
struct GuardLimits {
    float prec, range_amax, range_ss;
};

// One row's softmax statistics over one vocabulary chunk, as the statistics passes write
// them and the merges read them: partials [nsplit][m], one 12-byte record per (chunk, row),
// so a merge loads a chunk's three values in one instruction.
struct Partial {
    float best;  // log2-domain maximum of the chunk's logits
    float sum;   // sum of exp2 over the chunk (relative to the reference, see the kernels)
    int idx;     // first class reaching the maximum
};
static_assert(sizeof(Partial) == 12, "partial record");

// Arguments of one launch of the statistics kernels and of the writer (head_mfma.hpp).
struct StatsLaunch {
    const float* a;
    int64_t m;
    int k, vec;
    const uint8_t* rec;
    int tiles, nsplit, tpc, mblocks;
    Partial* part;
    GuardLimits lim;
    unsigned long long* guard_header;
    int* guard_rows;
    unsigned guard_epoch;
    int guard_cap;
    // per row block of the main pass: 1 when the guard surely sends all of its rows to the
    // rescue (guard_scan_kernel); null: no block is skipped
    const uint8_t* skip = nullptr;
    // small batches of the two-term modes: the three-term records the main pass's own
    // workgroups recompute their flagged rows with (no rescue launch, no row list); null: the
    // rescue is a pass of its own
    const uint8_t* rec3 = nullptr;
};
struct RowsLaunch {
    const float* a;
    int64_t m;
    int k, vec;
    const uint8_t* rec;
    int tiles, n, nsplit, tpc, mblocks;
    const float* row_max;
    const float* row_inv;
    float* out;
    GuardLimits lim;
    unsigned long long* guard_header;
    int* guard_rows;
    unsigned guard_epoch;
    int guard_cap;
};
constexpr int kStatsWaves = 4;   // waves per workgroup of the statistics pass: two workgroups per CU
constexpr int kWriterWaves = 4;  // consumer waves of the writer, 32 rows each (plus one loader)

// Per-configuration launchers, explicitly instantiated in head_cfg_*.hip.
template <int C, int G>
int stats_main_cfg(const StatsLaunch& x, int mb, bool noref, unsigned grid, hipStream_t st);
template <int C, int G>
int stats_gather_cfg(const StatsLaunch& x, unsigned grid, hipStream_t st);
template <int C, int G, bool GATHER>
int rows_cfg(const RowsLaunch& x, int epi, unsigned grid, hipStream_t st);

// Precision guard of the split-activation modes: rows whose max |a| exceeds amax_limit
// are collected in rows[0 .. count) and recomputed with one more activation term.  The
// 64-bit header holds (epoch << 32) | count.  Every call draws a new epoch; the first
// append of a call installs it (count 0), and a header with another epoch counts as empty,
// so a fresh or stale workspace needs no reset.  Paths that end with a merge kernel reset
// the header to (epoch, 0) there, so a replay of the same call (same epoch) starts empty.
// The statistics pass may skip the reference shift of the softmax sum (stats_noref) when
// the head bounds its logits: its rescue pass, which keeps the shift, then also takes the
// rows whose logits are not proven to lie in [-kLogitBound, kLogitBound] (GuardLimits).
constexpr float kLogitBound = 60.0f;
struct FmaWeights;
struct Guard {
    float amax_limit;
    unsigned long long* header;
    int* rows;
    int capacity;  // entries of rows (the batch's row count)
    unsigned epoch;
    float range_amax_limit;  // rows up to it have every logit within kLogitBound (L1 bound)
    float range_ss_limit;    // or rows with ||a||_2^2 up to it (L2 bound)
    bool stats_noref;
    const FmaWeights& fma;  // the head's fp32 weights, for a rescue in fp32 FMA
    uint8_t* skip;          // a byte per 128 rows: the statistics pass's skipped row blocks
};

// Supported group counts (k = 113..120 and k = 73..80, the PP-OCRv6 small and tiny heads).
bool mfma_supports_groups(int G);

int launch_pack_int8(const float* w_t, int64_t n, int64_t k, int8_t* q, float* scales,
                     hipStream_t st);

// Head preparation on the device: dst [cols][rows] = src [rows][cols]; the quantities
// behind the guard limits (largest |w|, largest L1 and L2 norm of a dequantised class row,
// largest |bias|) as bit patterns of non-negative values (maxima taken with atomicMax, so
// *out must start zeroed), from q and scales (INT8 head) or w (FP32 head); the MFMA tile
// records (rec zeroed beforehand; q for an INT8 head, w for an FP32 head).
struct HeadLimitBits {
    unsigned long long w1;    // double
    unsigned long long bmax;  // double
    unsigned long long l2;    // double
    unsigned wmax;            // float
    unsigned pad;
};
int launch_transpose(const float* src, int64_t rows, int64_t cols, float* dst, hipStream_t st);
int launch_head_limits(const int8_t* q, const float* w, const float* scales, const float* bias, int64_t n, int64_t k,
                       HeadLimitBits* out, hipStream_t st);
int launch_build_records(const TileGeom& g, int64_t n, int64_t k, const int8_t* q, const float* w,
                         const float* scale, const float* bias, bool f16, uint8_t* rec, hipStream_t st);

// Writes an empty guard header (epoch 0, which no call uses): run once on every workspace
// the library allocates, before its first use.
int launch_guard_clear(unsigned long long* guard_header, hipStream_t st);

// rec: the records the configuration reads (fp16 for H*, bf16 otherwise); rec_rescue: the
// bf16 records of the three-term rescue of guarded rows (INT8 heads).
int launch_logits_mfma(int cfg, const TileGeom& tg, const uint8_t* rec, const uint8_t* rec_rescue, const float* a,
                       int64_t m, int64_t n, int64_t k, float* out, const Guard* guard, hipStream_t st);
// Fused projection + online softmax statistics: per (row, vocabulary chunk) partials.
int stats_per_cu_mfma(int cfg, int64_t m);  // workgroups of the main statistics pass per CU
int stats_nsplit(int64_t m, int rows_per_block, int tiles, int per_cu);
int stats_rows_per_block_mfma(int cfg, int64_t m);
// Main pass, rescue of the guarded rows, then one wave per row merges the partials and
// resolves the argmax: idx, maxprob (1/sum) and, when non-null, row_max (log2-domain
// maximum) and row_inv (1/sum) for a probs pass.
// CTC collapse of text lines fused into the statistics merge (device pointers): line i is
// rows line_off[i] .. line_off[i+1]; outputs as ppocr_ctc_greedy.
struct CtcOut {
    const int64_t* line_off;  // null: every line has line_len steps
    int64_t lines;
    int32_t blank;
    int32_t* seq;
    int64_t* seq_len;
    float* score;
    int64_t line_len = 0;
};

// With `ctc`, the final merge also runs the CTC collapse (row_max and row_inv unused).
// line_len > 0: `a` is channels-first, [m / line_len][k][line_len] (the tensor before the
// neck's transpose); row r is step r % line_len of line r / line_len.
int launch_stats_mfma(int cfg, const TileGeom& tg, const uint8_t* rec, const uint8_t* rec_rescue, const float* a, int64_t m,
                      int64_t n, int64_t k, int nsplit, Partial* part,
                      const Guard* guard, int32_t* idx, float* maxprob, float* row_max, float* row_inv,
                      const CtcOut* ctc, hipStream_t st, int64_t line_len = 0);
int launch_probs_mfma(int cfg, const TileGeom& tg, const uint8_t* rec, const uint8_t* rec_rescue, const float* a, int64_t m,
                      int64_t n, int64_t k, const float* row_max, const float* row_inv, float* probs,
                      const Guard* guard, hipStream_t st);

// Epilogues of the projection kernels: logits, probabilities, per-chunk softmax statistics.
enum Epi : int { EPI_LOGITS = 0, EPI_PROBS = 1, EPI_STATS = 2 };

// fp32 vector FMA path over the packed int8 weights (q != null) or fp32 weights (w != null).
int launch_logits_fma(const int8_t* q, const float* w, const float* scale, const float* bias,
                      const float* a, int64_t m, int64_t n, int64_t k, float* out, hipStream_t st);
constexpr int kFmaRowsPerBlock = 128, kFmaCols = 128;  // rows and classes of a workgroup's tile
int launch_stats_fma(const int8_t* q, const float* w, const float* scale, const float* bias,
                     const float* a, int64_t m, int64_t n, int64_t k, int nsplit, Partial* part,
                     hipStream_t st, int64_t line_len = 0);
int launch_probs_fma(const int8_t* q, const float* w, const float* scale, const float* bias,
                     const float* a, int64_t m, int64_t n, int64_t k, const float* row_max,
                     const float* row_inv, float* probs, hipStream_t st);
// The fp32 weights of the FMA path: q (INT8 head) or w (FP32 head), scale, bias.
struct FmaWeights {
    const int8_t* q;
    const float* w;
    const float* scale;
    const float* bias;
};
// Rescue in fp32 FMA of the rows on a guard list (Guard) of an MFMA pass, with the same
// epilogue: logits or probabilities of every class (epi EPI_LOGITS / EPI_PROBS), or the
// statistics partials of the MFMA pass's vocabulary chunks (EPI_STATS: nsplit chunks of
// classes_per_chunk classes), overwriting what that pass wrote for those rows.
int launch_rescue_fma(int epi, const FmaWeights& fw, const float* a, int64_t m, int64_t n, int64_t k, int nsplit,
                      int classes_per_chunk, float* out, const float* row_max, const float* row_inv, Partial* part,
                      int64_t line_len, const Guard& guard, hipStream_t st);

// Merge the per-chunk partials of each row: argmax index, max probability, and (when
// row_max/row_inv are non-null) the row's log2-domain maximum and 1/sum for a probs pass.
// With `guard`, the merge also resets the guard header to (epoch, 0) (see Guard).
int launch_merge_stats(const Partial* part, int64_t m, int nsplit, int32_t* idx, float* maxprob, float* row_max, float* row_inv,
                       const Guard* guard, hipStream_t st);

int launch_softmax_rows(float* x, int64_t rows, int64_t cols, int32_t* idx, float* maxprob,
                        hipStream_t st);
int launch_argmax_rows(const float* x, int64_t rows, int64_t cols, int32_t* idx, float* val,
                       hipStream_t st);
int launch_ctc_greedy(const int32_t* idx, const float* maxprob, const int64_t* line_off,
                      int64_t lines, int32_t blank, int32_t* seq, int64_t* seq_len, float* score,
                      hipStream_t st);
// Merge of the vocabulary-chunk partials and the CTC collapse in one kernel; idx and
// maxprob (per row) may be null.
int launch_merge_ctc(const Partial* part, int64_t m, int nsplit,
                     const CtcOut& ctc, int32_t* idx, float* maxprob, const Guard* guard, hipStream_t st);

}  // namespace ppocr
