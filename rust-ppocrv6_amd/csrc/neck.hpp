// The SVTR mixing tail before the recognition head (neck.hip): device weights and launcher.
#pragma once
#include "common.hpp"

namespace ppocr {

// The geometry the kernels are built for: PP-OCRv6_small_rec's tail, D = 120 channels,
// 8 heads of 15, MLP hidden width 240.
constexpr int kNeckDim = 120;
constexpr int kNeckHeadDim = 15;
constexpr int kNeckHidden = 240;
constexpr int kNeckMaxBlocks = 8;

// One transformer block, device pointers: LayerNorm (w, b, eps), qkv [D][3D] + [3D],
// proj [D][D] + [D], LayerNorm, fc1 [D][H] + [H], fc2 [H][D] + [D] (MatMul weights as the
// model stores them, row-major [K][N]).
struct NeckBlockDev {
    const float *ln1_w, *ln1_b;
    float ln1_eps;
    const float *qkv_w, *qkv_b, *proj_w, *proj_b;
    const float *ln2_w, *ln2_b;
    float ln2_eps;
    const float *fc1_w, *fc1_b, *fc2_w, *fc2_b;
    // fp16 planes of qkv's and proj's W^T, [2][N][kp] (the nearest half of each weight, then
    // the nearest half of what it leaves; k padded with zeros to kp = 128), used when
    // NeckDev::f16 is set
    // qkv's columns padded per head to 16 (q, k, v of head h at 128 part + 16 h + d, zero
    // weights and bias at d = 15) and proj's rows alike (kNeckQkvPad, kNeckAttPad): with
    // fp16 halves the attention reads and writes whole 16-byte vectors
    const uint16_t *qkv_h, *proj_h;
    const float* qkv_bp;  // qkv's bias in the padded column order
    // fc1's and fc2's fp16 planes as the fused MLP kernel stages them: 8 tiles of 32 hidden
    // units, 32 KB each, tile T = fc1's planes of units 32 T .. 32 T + 31 as [plane][k chunk
    // of 8][unit] then fc2's planes of the matching contraction block as [plane][chunk]
    // [output column (128)], 8 halves per entry, zeros past the hidden units and columns
    const uint16_t* mlp_h;
    // the attention's operands scaled by powers of two before the fp16 split (q * scale by
    // 2^attn_eq, k by 2^attn_ek, v by 2^attn_ev), chosen from their bounds so that the halves
    // of all but negligible values stay above fp16's subnormals
    int attn_eq, attn_ek, attn_ev;
    // the fused MLP's operands scaled the same way: fc1's and fc2's weight planes hold the
    // weights times 2^mlp_e1 and 2^mlp_e2, the kernel scales LN2's output by 2^mlp_ey and
    // the hidden layer by 2^mlp_eh before their splits, and each product by the inverse
    int mlp_e1, mlp_e2, mlp_ey, mlp_eh;
};

struct NeckDev {
    int dim = 0, heads = 0, hidden = 0, blocks = 0;
    float scale = 0.0f;  // the attention's Mul constant (head_dim^-1/2 in the model)
    NeckBlockDev block[kNeckMaxBlocks];
    const float *lnf_w = nullptr, *lnf_b = nullptr;
    float lnf_eps = 0.0f;
    // the GEMMs run on fp16 halves (three products): set when the weights bound every GEMM
    // operand inside fp16's range (neck_f16_bounds_ok)
    bool f16 = false;
};

// k of a weight's fp16 planes, padded: 128 for K <= 128, else 256.
constexpr int neck_f16_kp(int k) { return k <= 128 ? 128 : 256; }

// Row widths of qkv and of the attention output when each head's 15 values are padded to
// 16 (the fp16-halves path).
constexpr int kNeckQkvPad = 3 * 128, kNeckAttPad = 128;
static_assert(kNeckDim == 8 * kNeckHeadDim && kNeckHeadDim < 16, "eight heads of at most 16 values");

// Floats of workspace per token row: the residual stream and the shortcut rows (D each),
// qkv (3D, or kNeckQkvPad), the attention output (D, or kNeckAttPad) and the MLP hidden
// layer (H).
constexpr int64_t kNeckWsFloatsPerRow = 2 * kNeckDim + kNeckQkvPad + kNeckAttPad + kNeckHidden;

// The whole tail on token rows: x_in and shortcut_in in `layout` (PPOCR_NECK_ROWS: [m][D];
// PPOCR_NECK_CHANNELS_FIRST: line b as [D][T_b] at D * (first row of b)), lines given by
// device offsets line_off[0..lines] or, with line_off null, line_len rows each; out [m][D]
// token rows (the input of the head's MatMul).  ws: kNeckWsFloatsPerRow * m floats.
// With `marks`, an event is recorded on st before the first kernel and after each kernel,
// and the kernel's name kept beside it (measurement of the kernels one by one).
struct NeckMarks {
    hipEvent_t* events;
    const char** names;  // names[i]: the kernel that ends at events[i] ("start" for events[0])
    int capacity;
    int count;
};
int launch_neck(const NeckDev& nk, const float* x_in, const float* shortcut_in, int64_t m, const int64_t* line_off,
                int64_t lines, int64_t line_len, int layout, float* out, float* ws, hipStream_t st,
                NeckMarks* marks = nullptr);

}  // namespace ppocr
