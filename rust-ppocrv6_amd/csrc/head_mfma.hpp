// MFMA kernels (device templates) of the vocabulary projection MatMul.12
// (matmul_quantized_b, src/ops/matmul.rs:1204-1336; matmul_transposed_b,
// src/ops/matmul.rs:514-897) and of its fusion with Softmax.2 (src/ops/softmax.rs:199-285)
// and the CTC argmax (src/postprocess/ctc.rs:151-163), with the per-configuration launchers
// that the head_cfg_*.hip translation units instantiate.
//
// Exactness: int8 weights are exact in bf16 and in fp16 (|q| <= 127 < 2^8).  The fp32
// activation is split into 16-bit terms a = a0 + a1 + a2 + ... (each term the rounding of
// what the previous ones left), and the products of all terms are summed by the MFMA in
// fp32: the terms are concatenated along k, so one accumulation chain covers every term.
// Two bf16 terms carry 16 bits of the activation, two fp16 terms 22 (fp16 keeps 11
// significant bits to bf16's 8, at the same MFMA rate; its range, |a| < 65504, is held by
// the precision guard).
//
// Operand layout of v_mfma_f32_32x32x16_bf16 (checked on gfx950): lane l holds row
// (l % 32) of A and column (l % 32) of B for k in [8*(l/32), 8*(l/32) + 8); the result
// D[i][j] sits in lane j + 32*((i/4) % 2), register (i % 4) + 4*(i/8).
//
// K-concatenation: the product list ("pairs") of a configuration, times the G groups of
// 8 along k, gives P = pairs*G (product, group) slots; each MFMA step feeds one slot to
// lanes 0-31 and one to lanes 32-63 (a slot past the end is a zero block).  The steps walk
// the groups two at a time and, for each pair of groups, every product in turn, products
// on the same weight plane adjacent: consecutive steps of the same plane then read the same
// weight fragment (an INT8 head's activation terms all multiply q), so the two-term mode
// reads 8 weight fragments per tile for its 15 steps.
#pragma once
#include <type_traits>
#include <utility>

#include "kernels.hpp"

namespace ppocr {

template <int C>
struct CfgT;
template <>
struct CfgT<CFG_Q1> {  // a0 * q
    static constexpr bool f16 = false;
    static constexpr int pairs = 1, wplanes = 1, terms = 1;
    __host__ __device__ static constexpr int act(int) { return 0; }
    __host__ __device__ static constexpr int wpl(int) { return 0; }
};
template <>
struct CfgT<CFG_Q2> {  // a0 * q + a1 * q
    static constexpr bool f16 = false;
    static constexpr int pairs = 2, wplanes = 1, terms = 2;
    __host__ __device__ static constexpr int act(int p) { return p; }
    __host__ __device__ static constexpr int wpl(int) { return 0; }
};
template <>
struct CfgT<CFG_Q3> {  // a0 * q + a1 * q + a2 * q
    static constexpr bool f16 = false;
    static constexpr int pairs = 3, wplanes = 1, terms = 3;
    __host__ __device__ static constexpr int act(int p) { return p; }
    __host__ __device__ static constexpr int wpl(int) { return 0; }
};
template <>
struct CfgT<CFG_F1> {  // a0 * w0
    static constexpr bool f16 = false;
    static constexpr int pairs = 1, wplanes = 2, terms = 1;
    __host__ __device__ static constexpr int act(int) { return 0; }
    __host__ __device__ static constexpr int wpl(int) { return 0; }
};
template <>
struct CfgT<CFG_F3> {  // a0 * w0 + a0 * w1 + a1 * w0
    static constexpr bool f16 = false;
    static constexpr int pairs = 3, wplanes = 2, terms = 2;
    __host__ __device__ static constexpr int act(int p) { return p == 2 ? 1 : 0; }
    __host__ __device__ static constexpr int wpl(int p) { return p == 1 ? 1 : 0; }
};
template <>
struct CfgT<CFG_H2> {  // a0 * q + a1 * q, fp16 terms
    static constexpr bool f16 = true;
    static constexpr int pairs = 2, wplanes = 1, terms = 2;
    __host__ __device__ static constexpr int act(int p) { return p; }
    __host__ __device__ static constexpr int wpl(int) { return 0; }
};
template <>
struct CfgT<CFG_HF3> {  // a0 * w0 + a0 * w1 + a1 * w0, fp16 halves of both operands
    static constexpr bool f16 = true;
    static constexpr int pairs = 3, wplanes = 2, terms = 2;
    __host__ __device__ static constexpr int act(int p) { return p == 2 ? 1 : 0; }
    __host__ __device__ static constexpr int wpl(int p) { return p == 1 ? 1 : 0; }
};

// One 32x32x16 MFMA step on 16-bit operands held as raw bits: fp16 or bf16 products,
// fp32 accumulation.
template <bool F16>
__device__ __forceinline__ f32x16 mfma16(u16x8 a, u16x8 b, f32x16 c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                      0, 0);
    else
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(u16x8, a), __builtin_bit_cast(u16x8, b), c,
                                                       0, 0, 0);
}

// Tile geometry of a configuration: P (product, group) slots, S MFMA steps, FRAG bytes of
// weight fragments per staged tile, REC bytes per tile record (fragments + epilogue
// constants), BUF bytes per LDS buffer (record + a 512-byte zero block for empty slots).
struct Slot {
    int p;  // product (index into CfgT::act / wpl); < 0: the zero block
    int g;  // group of 8 along k
};
template <int C, int G>
struct Geo {
    static constexpr int NPROD = CfgT<C>::pairs;
    static constexpr int P = NPROD * G;
    static constexpr int S = (P + 1) / 2;
    static constexpr int FRAG = CfgT<C>::wplanes * G * 512;
    static constexpr int REC = FRAG + 512;
    static constexpr int BUF = REC + 512;
    // the x-th product when they are ordered by weight plane (stable), so products that
    // share a plane are adjacent
    __host__ __device__ static constexpr int prod(int x) {
        int n = 0;
        for (int pl = 0; pl < 2; ++pl)
            for (int p = 0; p < NPROD; ++p)
                if (CfgT<C>::wpl(p) == pl && n++ == x) return p;
        return -1;
    }
    // Slot fed to lane half h by MFMA step s: over the G/2 full pairs of groups, one step
    // per product with groups 2j and 2j+1 on the two halves; an odd last group then takes
    // the products two per step.
    __host__ __device__ static constexpr Slot slot(int s, int h) {
        const int body = (G / 2) * NPROD;
        if (s < body) return Slot{prod(s % NPROD), 2 * (s / NPROD) + h};
        const int x = 2 * (s - body) + h;
        if ((G & 1) && x < NPROD) return Slot{prod(x), G - 1};
        return Slot{-1, 0};
    }
    // LDS byte offset of the weight fragment of step s, half h, within a staged tile
    __host__ __device__ static constexpr int off(int s, int h) {
        const Slot sl = slot(s, h);
        return sl.p < 0 ? REC : (CfgT<C>::wpl(sl.p) * G + sl.g) * 512;
    }
    // step s reads a weight fragment other than step s-1's
    __host__ __device__ static constexpr bool fresh(int s) {
        return s == 0 || off(s, 0) != off(s - 1, 0) || off(s, 1) != off(s - 1, 1);
    }
    // index of the fragment step s uses, counted in step order
    __host__ __device__ static constexpr int fid(int s) {
        int f = 0;
        for (int x = 1; x <= s; ++x) f += fresh(x) ? 1 : 0;
        return f;
    }
};

// Weight fragment of MFMA step s for lane (i, h).  In the common case the two lane halves
// read consecutive fragments, so the address is one per-lane register plus an immediate.
template <int C, int G>
__device__ __forceinline__ u16x8 weight_frag(const uint8_t* buf, int s, int lane_base, int i16, int h) {
    const int o0 = Geo<C, G>::off(s, 0);
    const int o1 = Geo<C, G>::off(s, 1);
    const int addr = (o1 - o0 == 512) ? lane_base + o0 : i16 + (h ? o1 : o0);
    return *reinterpret_cast<const u16x8*>(buf + addr);
}

// Weight fragments in flight, NB register buffers: the fragment of step s sits in buffer
// fid(s) % NB, and the fragment of step s + NB is read (when it is a new one) right after
// the MFMAs of step s.  That read overwrites fragment fid(s + NB) - NB, which is at most
// fid(s) and, when equal, is last used by step s (every step after s up to s + NB starts
// a new fragment), so no fragment is overwritten while a later step still needs it.
template <int C, int G, int NB>
__device__ __forceinline__ void frag_prefetch_first(u16x8 (&wq)[NB], const uint8_t* buf, int lane_base, int i16,
                                                    int h) {
    [&]<int... x>(std::integer_sequence<int, x...>) {
        ([&] {
            if constexpr (x < Geo<C, G>::S && Geo<C, G>::fresh(x))
                wq[Geo<C, G>::fid(x) % NB] = weight_frag<C, G>(buf, x, lane_base, i16, h);
        }(), ...);
    }(std::make_integer_sequence<int, NB>{});
}
template <int C, int G, int NB, int s>
__device__ __forceinline__ void frag_prefetch_after(u16x8 (&wq)[NB], const uint8_t* buf, int lane_base, int i16,
                                                    int h) {
    if constexpr (s + NB < Geo<C, G>::S) {
        if constexpr (Geo<C, G>::fresh(s + NB))
            wq[Geo<C, G>::fid(s + NB) % NB] = weight_frag<C, G>(buf, s + NB, lane_base, i16, h);
    }
}
template <int C, int G, int NB, int s>
__device__ __forceinline__ const u16x8& frag_of(const u16x8 (&wq)[NB]) {
    return wq[Geo<C, G>::fid(s) % NB];
}

// Grid position -> (block of rows, vocabulary chunk).  Workgroups go to the 8 XCDs of
// the MI355X round-robin by id.  With 8 or more chunks, ids are arranged so that every XCD
// works on its own 1/8 of the vocabulary (or of a multiple of it) and keeps that slice of
// the weight tiles resident in its L2.  With fewer chunks, ROWS_ON_ONE_XCD puts all chunks
// of a row block on one XCD, so its activation rows are read through one L2 instead of
// one per chunk (the statistics pass: the XCD's workgroups walk the chunks' tiles in step,
// so each tile is fetched once per XCD and read from L2 by the others; measured on the
// 30720-row batch in 4 chunks, 0.2250 -> 0.2220 ms per launch); otherwise each XCD takes
// one chunk (the writer).  From 8 chunks up the count need not be a multiple of 8: every
// XCD gets ceil(nsplit / 8) chunk slots, and the workgroups whose chunk is nsplit or more
// (on the last XCDs) have nothing to do.  Below 8 it divides 8.
template <bool ROWS_ON_ONE_XCD>
__device__ __forceinline__ void map_block(int bid, int nsplit, int* mbi, int* chunk) {
    const int x = bid & 7, slot = bid >> 3;
    if (nsplit >= 8) {
        const int per = (nsplit + 7) >> 3;
        *chunk = x * per + slot % per;
        *mbi = slot / per;
    } else if (ROWS_ON_ONE_XCD) {
        *chunk = slot % nsplit;
        *mbi = (slot / nsplit) * 8 + x;
    } else {
        const int r8 = 8 / nsplit;
        *chunk = x % nsplit;
        *mbi = slot * r8 + x / nsplit;
    }
}

// Split x into 16-bit terms (bf16, or fp16 with F16) and return the bits of term t (0 =
// nearest, 1 = nearest of the remainder, 2 = of the remainder after that).  Every
// subtraction is exact (below fp16's overflow).
template <bool F16>
__device__ __forceinline__ unsigned short split_term(float x, int t) {
    using T = typename std::conditional<F16, _Float16, __bf16>::type;
    const T b0 = (T)x;
    if (t == 0) return __builtin_bit_cast(unsigned short, b0);
    const float r1 = x - (float)b0;
    const T b1 = (T)r1;
    if (t == 1) return __builtin_bit_cast(unsigned short, b1);
    const float r2 = r1 - (float)b1;
    return __builtin_bit_cast(unsigned short, (T)r2);
}

// Activation fragments of one lane for every MFMA step of a 32-row block.  A step takes
// the 8 k values of its slot (group g of 8 along k) as the 16-bit term its product uses;
// consecutive steps that feed both lane halves the same groups (the products of one group
// pair) share one load.  Every load of the block is issued before any value is used, so a
// wave waits for memory once per block, not once per step.  `row` must be a row of a
// (callers pass row 0 for lanes past the batch: their results are never written).
// `amax` is raised to the largest |value| loaded, `ss` accumulates the squares of the
// values of product 0 (each k once over the two halves).  `vec` > 0: rows and groups are
// 16-byte aligned, so a group is two float4 loads; vec < 0 selects the channels-first
// layout [lines][k][T] of the tensor before the neck's transpose, T = -vec: row r is step
// r % T of line r / T, and its k values are T floats apart.  Only the last group can
// reach past k (k > 8G - 8); its missing values are zeros, read from a clamped address.
template <int C, int G>
struct ActPlan {
    using GE = Geo<C, G>;
    static constexpr int S = GE::S;
    // group of step s on half h, -1 for a padding slot
    __host__ __device__ static constexpr int grp(int s, int h) {
        const Slot sl = GE::slot(s, h);
        return sl.p < 0 ? -1 : sl.g;
    }
    // step s needs values other than step s-1's on some half
    __host__ __device__ static constexpr bool fresh(int s) {
        if (s == 0) return true;
        for (int h = 0; h < 2; ++h)
            if (grp(s, h) >= 0 && grp(s, h) != grp(s - 1, h)) return true;
        return false;
    }
    // load used by step s, counted in step order
    __host__ __device__ static constexpr int lid(int s) {
        int l = 0;
        for (int x = 1; x <= s; ++x) l += fresh(x) ? 1 : 0;
        return l;
    }
    static constexpr int NL = lid(S - 1) + 1;
    // group loaded for half h at fresh step s: its own, else (padding) the other half's
    __host__ __device__ static constexpr int load_grp(int s, int h) {
        return grp(s, h) >= 0 ? grp(s, h) : (grp(s, 1 - h) >= 0 ? grp(s, 1 - h) : 0);
    }
};

template <int C, int G, int s>
__device__ __forceinline__ void act_load(const float* __restrict__ rp, int64_t kst, int k, bool vec4, int h,
                                         float (&x)[ActPlan<C, G>::NL][8]) {
    using AP = ActPlan<C, G>;
    if constexpr (AP::fresh(s)) {
        constexpr int l = AP::lid(s), g0 = AP::load_grp(s, 0), g1 = AP::load_grp(s, 1);
        constexpr bool last = g0 == G - 1 || g1 == G - 1;
        const int g = h ? g1 : g0;
        if (vec4) {
            // 16-byte aligned rows, k % 4 == 0: a partial last group holds 4 values
            const float* p = rp + 8 * g;
            const bool hi = !last || 8 * g + 8 <= k;
            const f32x4 v0 = reinterpret_cast<const f32x4*>(p)[0];
            const f32x4 v1 = reinterpret_cast<const f32x4*>(p + (hi ? 4 : 0))[0];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[l][e] = v0[e];
                x[l][4 + e] = hi ? v1[e] : 0.0f;
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int kk = 8 * g + e;
                const float v = rp[(int64_t)(last ? min(kk, k - 1) : kk) * kst];
                x[l][e] = (!last || kk < k) ? v : 0.0f;
            }
        }
    }
}

template <int C, int G, int s>
__device__ __forceinline__ u16x8 act_split(const float (&x)[ActPlan<C, G>::NL][8], int h, float& amax, float& ss) {
    using AP = ActPlan<C, G>;
    constexpr Slot s0 = Geo<C, G>::slot(s, 0), s1 = Geo<C, G>::slot(s, 1);
    constexpr int l = AP::lid(s);
    if constexpr (AP::fresh(s)) {
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, __builtin_fabsf(x[l][e]));
    }
    // every group is fed to product 0 once, on one half, so its squares are counted once
    if constexpr (s0.p == 0 || s1.p == 0) {
        const bool p0 = h ? s1.p == 0 : s0.p == 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = p0 ? fmaf(x[l][e], x[l][e], ss) : ss;
    }
    constexpr int t0 = s0.p < 0 ? 0 : CfgT<C>::act(s0.p), t1 = s1.p < 0 ? 0 : CfgT<C>::act(s1.p);
    const int term = h ? t1 : t0;
    u16x8 f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = split_term<CfgT<C>::f16>(x[l][e], term);
    if constexpr (s0.p < 0 || s1.p < 0) {
        const bool pad = h ? s1.p < 0 : s0.p < 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = pad ? (unsigned short)0 : f[e];
    }
    return f;
}

// `x` in a vector register, opaque to the optimiser: values computed from it are computed
// where they are used.  The gather kernels pass k through it, so the last group's bounds
// (eight offsets and masks) are not hoisted out of the row-block loop and kept live in
// scalar registers across the tile loop, which spills them.
__device__ __forceinline__ int opaque_vgpr(int x) {
    asm volatile("" : "+v"(x));
    return x;
}

// First value of row `row` of a, and (kst) the floats between its consecutive k values.
// vec >= 0: rows of k floats.  vec < 0: the channels-first layout [lines][k][T] of the
// tensor before the neck's transpose, T = -vec: row r is step r % T of line r / T, and its
// k values are T floats apart.
__device__ __forceinline__ const float* row_ptr(const float* a, int64_t row, int k, int vec, int64_t& kst) {
    if (vec >= 0) {
        kst = 1;
        return a + row * (int64_t)k;
    }
    kst = -(int64_t)vec;
    const int64_t line = row / kst;
    return a + line * kst * k + (row - line * kst);
}

// Issue the loads of a block (act_issue), then split what they return (act_split_all).
template <int C, int G>
__device__ __forceinline__ void act_issue(const float* __restrict__ a, int64_t row, int k, int vec, int h,
                                          float (&x)[ActPlan<C, G>::NL][8]) {
    int64_t kst = 1;
    const float* rp = a + row * (int64_t)k;
    if (vec < 0) {
        kst = -(int64_t)vec;
        const int64_t line = row / kst;
        rp = a + line * kst * k + (row - line * kst);
    }
    const bool vec4 = vec > 0;
    [&]<int... s>(std::integer_sequence<int, s...>) {
        (act_load<C, G, s>(rp, kst, k, vec4, h, x), ...);
    }(std::make_integer_sequence<int, ActPlan<C, G>::S>{});
}
template <int C, int G>
__device__ __forceinline__ void act_split_all(const float (&x)[ActPlan<C, G>::NL][8], int h,
                                              u16x8 (&bf)[Geo<C, G>::S], float& amax, float& ss) {
    [&]<int... s>(std::integer_sequence<int, s...>) {
        ((bf[s] = act_split<C, G, s>(x, h, amax, ss)), ...);
    }(std::make_integer_sequence<int, ActPlan<C, G>::S>{});
}

// Activation fragment of one lane for MFMA step s, loaded and split on its own (the
// rescue passes' gather kernels, which hold more state, use this form: it keeps fewer
// values live): row `row` of a (zero when the row is not valid), the 8 k values of the
// lane's slot, as the bf16 term its product uses; `rp` points at the row's first value
// and `kst` floats separate consecutive k (row_ptr).  `amax` is raised to the largest
// |value| loaded, `ss` accumulates the squares of the values loaded for product 0 (each k
// once).  G = ceil(k / 8), so only group G - 1 can be partial, and only the steps that
// feed it compare k values against k (per-element compares on every step are loop
// invariants the compiler keeps in scalar registers, which spill).  `vec4`: rows are
// 16-byte aligned and k % 4 == 0, so a fragment is two float4 loads and a partial last
// group holds 4 values.
template <int C, int G, int s>
__device__ __forceinline__ u16x8 act_frag(const float* __restrict__ rp, int64_t kst, bool valid, int k, bool vec4,
                                          int h, float& amax, float& ss) {
    u16x8 f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = 0;
    constexpr Slot s0 = Geo<C, G>::slot(s, 0), s1 = Geo<C, G>::slot(s, 1);
    constexpr bool last = (s0.p >= 0 && s0.g == G - 1) || (s1.p >= 0 && s1.g == G - 1);
    const int p = h ? s1.p : s0.p, g = h ? s1.g : s0.g;
    if (p < 0 || !valid) return f;
    constexpr int t0 = s0.p < 0 ? 0 : CfgT<C>::act(s0.p), t1 = s1.p < 0 ? 0 : CfgT<C>::act(s1.p);
    const int term = h ? t1 : t0;
    const float* src = rp + 8 * g * kst;
    float x[8];
    if (vec4) {
        const bool hi = !last || 8 * g + 8 <= k;
        const f32x4 v0 = reinterpret_cast<const f32x4*>(src)[0];
        const f32x4 v1 = reinterpret_cast<const f32x4*>(src + (hi ? 4 : 0))[0];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            x[e] = v0[e];
            x[4 + e] = hi ? v1[e] : 0.0f;
        }
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int kk = 8 * g + e;
            const float v = src[(int64_t)(last ? min(kk, k - 1) - 8 * g : e) * kst];
            x[e] = (!last || kk < k) ? v : 0.0f;
        }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        amax = fmaxf(amax, __builtin_fabsf(x[e]));
        f[e] = split_term<CfgT<C>::f16>(x[e], term);
    }
    // every group g is loaded once for product 0, so the squares are counted once
    if (p == 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(x[e], x[e], ss);
    }
    return f;
}

// Rows of the batch a workgroup works on: a contiguous block of rows, or (rescue pass)
// entries of a device-side row list.
struct RowSource {
    const int* list;  // null: contiguous rows
    int count;        // list length
    __device__ __forceinline__ int64_t row(int64_t j, int64_t m, bool& valid) const {
        if (list) {
            const int64_t r = j < count ? (int64_t)list[j] : -1;
            valid = r >= 0 && r < m;  // list entries are checked, not trusted
            return valid ? r : 0;
        }
        valid = j < m;
        return j;
    }
};

// Precision guard of the split-activation modes: a row whose largest |a| times the
// head's largest |w| exceeds the limit is appended to a device list, to be recomputed
// with one more activation term.  lanes i and i+32 see complementary k groups.
// The list's header is (epoch << 32) | count: the first append of a call installs the
// call's epoch with count 0 (a header with another epoch counts as empty; epochs have the
// top bit set, so no index, count or non-negative float left in the workspace matches
// one), then each append takes the next slot.  Slots past the capacity are dropped (the
// capacity is the batch's row count, and each row is appended once per call).  The test
// takes the |a| maximum and the sum of squares of both lanes' k groups.
// Appends the rows of the lanes whose `hit` is set, one atomic per wave: the wave's first
// such lane reserves popcount(hits) slots, and each lane writes at the base plus the hits
// of the lanes below it (one atomic per row serialises on the header when a head guards
// most rows).  Called by every lane of the wave.
__device__ __forceinline__ void guard_push(bool hit, int64_t row, unsigned long long* guard_header, int* guard_rows,
                                           unsigned epoch, int capacity) {
    const unsigned long long mask = __ballot(hit);
    if (mask == 0ull) return;
    const int lane = (int)__lane_id();
    const int leader = __ffsll((long long)mask) - 1;
    unsigned base = 0;
    if (lane == leader) {
        unsigned long long cur = __hip_atomic_load(guard_header, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        while ((unsigned)(cur >> 32) != epoch) {
            const unsigned long long prev = atomicCAS(guard_header, cur, (unsigned long long)epoch << 32);
            if (prev == cur) break;
            cur = prev;  // another lane or workgroup changed it first; look again
        }
        base = (unsigned)atomicAdd(guard_header, (unsigned long long)__popcll(mask));
    }
    base = (unsigned)__shfl((int)base, leader, 64);
    if (hit) {
        const int pos = (int)(base + (unsigned)__popcll(mask & ((1ull << lane) - 1ull)));
        if (pos >= 0 && pos < capacity) guard_rows[pos] = (int)row;
    }
}
__device__ __forceinline__ void guard_append(float amax, float ss, const GuardLimits& lim, bool valid, int64_t row,
                                             int h, unsigned long long* guard_header, int* guard_rows, unsigned epoch,
                                             int capacity) {
    amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
    ss += __shfl_xor(ss, 32, 64);
    const bool hit = h == 0 && valid && (amax > lim.prec || (amax > lim.range_amax && ss > lim.range_ss));
    guard_push(hit, row, guard_header, guard_rows, epoch, capacity);
}

// Entries of the guard list for this call's epoch (0 for a header of another epoch).
__device__ __forceinline__ int guard_count_of(const unsigned long long* guard_header, unsigned epoch, int capacity) {
    const unsigned long long v = *guard_header;
    if ((unsigned)(v >> 32) != epoch) return 0;
    const unsigned c = (unsigned)v;
    return c < (unsigned)capacity ? (int)c : capacity;
}

// Global -> LDS staging of one tile record by all NT threads of a workgroup, without
// registers: each wave issues direct 16-byte-per-lane loads into LDS (wave w, instruction
// x covers 16-byte chunks x*NT + 64*w .. +63).  The loads count in each wave's vmcnt;
// ring_barrier below waits for them before any wave reads the slot.
template <int REC, int NT = 256>
__device__ __forceinline__ void stage_direct(const uint8_t* __restrict__ src, uint8_t* dst, int tid) {
    constexpr int CH = REC / 16;
    constexpr int PER = (CH + NT - 1) / NT;
    static_assert(REC % 16 == 0 && PER >= 1 && PER <= 4, "tile record size");
    const int wave_chunk = tid & ~63;  // 64 * wave
#pragma unroll
    for (int x = 0; x < PER; ++x) {
        const int c0 = x * NT + wave_chunk;  // first chunk of this wave's instruction (uniform)
        if (CH % NT == 0 || c0 + (tid & 63) < CH)
            __builtin_amdgcn_global_load_lds(
                static_cast<const void*>(src + (size_t)(c0 + (tid & 63)) * 16),
                reinterpret_cast<__attribute__((address_space(3))) void*>(
                    reinterpret_cast<uintptr_t>(dst + (size_t)c0 * 16)),
                16, 0, 0);
    }
}

// Number of direct-load instructions every wave issues per staged tile record (waves past
// the end of a partial last round issue one fewer).
template <int REC, int NT = 256>
constexpr int stage_direct_min_ops() {
    return (REC / 16) / NT;
}

// Wait until at most N of this wave's global memory operations are outstanding.  They
// complete in issue order, so every older one has completed.
template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt field");
    __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));  // vmcnt(N) only
}
// Workgroup barrier for a ring whose newest N direct loads per wave may still be in
// flight: wait until at most N of this wave's loads are outstanding (so every older tile
// is in LDS) and all of its LDS accesses are done, then synchronise.  The barrier is
// written as an asm statement with a memory clobber: the compiler keeps every memory
// access on its side, and adds no wait for the newest loads (a fence would wait for all).
template <int N>
__device__ __forceinline__ void ring_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt field");
    __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0x0 << 8) | ((N >> 4) << 14));  // vmcnt(N) lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
}

// ============================================================ fused statistics, main pass
// One piece of the epilogue of a tile (compile-time piece number P; MB blocks of 32
// activation rows).  The pieces of a tile, in order:
//   0..3            t = acc*scale*log2e + bias*log2e for accumulator quad q (classes
//                   8q + 4h + 0..3), then the LDS load of quad q+2's constants
//   4..4+MB-1       the tile maximum of block b, and whether it beats the running maximum
//   4+MB..4+5MB-1   exp2(t - ref) and the tile sum, for quad (g % 4) of block (g / 4)
//   4+5MB           a lane whose maximum was beaten saves the tile's 16 values of its rows
//                   and the tile number (masked LDS stores)
//   5+5MB           running maximum, and whether ref must move
// Pieces are spread over the MFMA steps of the next tile, so each wave keeps the vector
// ALU and the LDS busy while its own MFMAs run.
template <int MB>
struct EpiState {
    float tmax[MB], tsum[MB];
    bool better[MB];
    bool need;
};

// Epilogue of one tile on the accumulators t of MB row blocks, cut into NP = 13 * MB + 2
// pieces of at most two exps each, in dependency order:
//   for each quad q of the lane's 16 values: the fma of quad q of every block (after the
//   last one, the constants of quad q + 2 are loaded into that quad's slot), then the exps
//   and sums of quad q, two values per piece;
//   then the tile maximum of each block, the saves of a raised maximum, the running maximum.
template <int MB>
constexpr int epi_pieces() {
    return 13 * MB + 2;
}

// Largest of three values, as one v_max3_f32.  A quiet NaN operand is ignored (IEEE
// maxNum, the behaviour of fmaxf); written out because fmaxf on values the compiler cannot
// prove canonical (loop-carried, MFMA results) costs a v_max_f32 x, x, x per operand first.
__device__ __forceinline__ float max3_f32(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

template <int P, int MB, bool NOREF>
__device__ __forceinline__ void epi_piece(f32x16 (&t)[MB], const float* __restrict__ ep, int h, int j,
                                          f32x4 (&cs)[2], f32x4 (&cb)[2], const float (&ref)[MB],
                                          float (&best)[MB], int (&bt)[MB], f32x4* save, EpiState<MB>& st) {
    constexpr int per_q = 3 * MB;
    if constexpr (P < 4 * per_q) {
        constexpr int q = P / per_q, x = P % per_q;
        if constexpr (x < MB) {
            constexpr int b = x;
#pragma unroll
            for (int e = 0; e < 4; ++e) t[b][4 * q + e] = fmaf(t[b][4 * q + e], cs[q & 1][e], cb[q & 1][e]);
            if constexpr (b == MB - 1 && q < 2) {
                cs[q & 1] = *reinterpret_cast<const f32x4*>(ep + 8 * (q + 2) + 4 * h);
                cb[q & 1] = *reinterpret_cast<const f32x4*>(ep + 32 + 8 * (q + 2) + 4 * h);
            }
        } else {
            constexpr int y = x - MB, b = y / 2, r = 4 * q + 2 * (y % 2);
            const float e0 = __builtin_amdgcn_exp2f(NOREF ? t[b][r] : t[b][r] - ref[b]);
            const float e1 = __builtin_amdgcn_exp2f(NOREF ? t[b][r + 1] : t[b][r + 1] - ref[b]);
            st.tsum[b] = (r == 0) ? e0 + e1 : st.tsum[b] + (e0 + e1);
            // keep the sum here: without a use in this piece the exps would be sunk past the
            // pieces that follow, out of the MFMA steps they are meant to overlap
            asm volatile("" : "+v"(st.tsum[b]));
        }
    } else if constexpr (P < 4 * per_q + MB) {
        constexpr int b = P - 4 * per_q;
        const float m01 = max3_f32(t[b][0], t[b][1], t[b][2]);
        const float m02 = max3_f32(t[b][3], t[b][4], t[b][5]);
        const float m03 = max3_f32(t[b][6], t[b][7], t[b][8]);
        const float m04 = max3_f32(t[b][9], t[b][10], t[b][11]);
        const float m05 = max3_f32(t[b][12], t[b][13], t[b][14]);
        st.tmax[b] = max3_f32(max3_f32(m01, m02, m03), max3_f32(m04, m05, t[b][15]), -INFINITY);
        st.better[b] = st.tmax[b] > best[b];
    } else if constexpr (P == 4 * per_q + MB) {
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            if (st.better[b]) {
                bt[b] = j;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    save[(b * 4 + q) * 64] = f32x4{t[b][4 * q], t[b][4 * q + 1], t[b][4 * q + 2], t[b][4 * q + 3]};
            }
        }
    } else {
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            best[b] = max3_f32(best[b], st.tmax[b], -INFINITY);
            if constexpr (!NOREF)
                st.need = st.need | ((best[b] != -INFINITY) & (__builtin_fabsf(best[b] - ref[b]) > 64.0f));
        }
    }
}

// The pieces of half-step x of H: each MFMA step of a tile is two half-steps, one after
// the MFMA of block 0 and one after the MFMAs of the other blocks.
template <int H, int x, int MB, bool NOREF>
__device__ __forceinline__ void epi_pieces_of_half(f32x16 (&t)[MB], const float* __restrict__ ep, int h, int j,
                                                   f32x4 (&cs)[2], f32x4 (&cb)[2], const float (&ref)[MB],
                                                   float (&best)[MB], int (&bt)[MB], f32x4* save,
                                                   EpiState<MB>& st) {
    constexpr int NP = epi_pieces<MB>();
    constexpr int p0 = x * NP / H, p1 = (x + 1) * NP / H;
    [&]<int... I>(std::integer_sequence<int, I...>) {
        (epi_piece<p0 + I, MB, NOREF>(t, ep, h, j, cs, cb, ref, best, bt, save, st), ...);
    }(std::make_integer_sequence<int, p1 - p0>{});
}

// Fused projection + softmax statistics, main pass.  Rows of the MFMA = classes, columns
// = activation rows: lane (i, h) owns activation row i of each block and 16 classes of
// each tile (n0 + 8*(r/4) + 4*h + (r%4)), so a row's statistics need no cross-lane
// traffic until the end of the chunk.  Per row the kernel keeps the running maximum of
// t = logit*log2(e), sum exp2(t - ref), the first tile that reached the maximum and, in
// LDS, that tile's 16 values of the lane: the first class reaching the maximum is found
// once, at the end of the chunk.  `ref` stays put unless the maximum moves more than 64
// away from it (a rare, wave-uniform branch).  Software pipeline: the MFMAs of tile j+1
// (second accumulator set) and the epilogue of tile j are issued interleaved in one
// instruction stream; weight tiles pass through a 4-slot LDS ring (tile j: epilogue
// constants, j+1: MFMA fragments, j+2 and j+3: being loaded straight from global memory
// into LDS), one barrier per tile.
constexpr int kPrefetch = 2;
constexpr int kRing = 4;  // LDS tile slots of the main statistics pass (a power of two)

// Kernel arguments read all at once: left to itself the compiler loads each one where it is
// first used, and a kernel whose first steps depend on each other (grid position, then the
// row list) waits for several scalar-cache misses in a row.
template <typename T>
__device__ __forceinline__ void arg_now(const T& x) {
    asm volatile("" ::"s"(x));
}
template <typename... T>
__device__ __forceinline__ void args_now(const T&... x) {
    (arg_now(x), ...);
}

// LDS of the main statistics pass: the tile ring and each wave's saved best tile.
template <int C, int G, int MB>
constexpr int main_lds_bytes() {
    return kRing * Geo<C, G>::BUF + kStatsWaves * MB * 16 * 64 * 4;
}

template <int C, int G, int MB, bool GATHER, bool NOREF, bool SKIP = false, bool FUSE = false,
          int OCC = 8 / kStatsWaves>
__global__ __launch_bounds__(64 * kStatsWaves, OCC) void stats_main_kernel(
    const float* __restrict__ a, int64_t m, int k, int vec, const uint8_t* __restrict__ rec, int tiles,
    int nsplit, int tiles_per_chunk, int mblocks, Partial* __restrict__ part, GuardLimits lim, unsigned long long* __restrict__ guard_header,
    int* __restrict__ guard_rows, unsigned guard_epoch, int guard_cap, const uint8_t* __restrict__ skip,
    const uint8_t* __restrict__ rec3) {
    using GE = Geo<C, G>;
    constexpr int RPB = 32 * kStatsWaves * MB;
    constexpr int NT = 64 * kStatsWaves;
    extern __shared__ __align__(16) uint8_t lds[];
    args_now(a, m, k, vec, rec, tiles, nsplit, tiles_per_chunk, mblocks, part, lim.prec,
             lim.range_amax, lim.range_ss, guard_header, guard_rows, guard_epoch, guard_cap);

    int mbi, chunk;
    map_block<true>(blockIdx.x, nsplit, &mbi, &chunk);
    if (mbi >= mblocks || chunk >= nsplit) return;
    // SKIP: a row block whose rows the guard surely sends to the rescue (guard_scan_kernel,
    // which also listed them) is skipped: the rescue pass overwrites all of their partials,
    // in every chunk
    if constexpr (SKIP && !GATHER) {
        if (skip[mbi]) return;
    }
    const int t0 = chunk * tiles_per_chunk;
    const int t1 = min(t0 + tiles_per_chunk, tiles);
    // one row block, or (GATHER) the row blocks of a device-side row list, mblocks apart
    const RowSource src{GATHER ? guard_rows : nullptr, GATHER ? guard_count_of(guard_header, guard_epoch, guard_cap) : 0};
    const int64_t blk_end = GATHER ? ((int64_t)src.count + RPB - 1) / RPB : (int64_t)mbi + 1;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, i = lane & 31, h = lane >> 5;
    if (tid < 32 * kRing)
        reinterpret_cast<u32x4*>(lds + (tid >> 5) * GE::BUF + GE::REC)[tid & 31] = u32x4{0, 0, 0, 0};
    const int lb = i * 16 + h * 512;
    // this lane's saved values of its best tile: [block][quad][lane] x 4 floats
    f32x4* save = reinterpret_cast<f32x4*>(lds + kRing * GE::BUF) + wave * (MB * 4 * 64) + lane;

    // one row block over this chunk's tiles, in arithmetic configuration CC (NR: without the
    // reference shift); RESCUE: the fused rescue, writing the partials of the rows set in
    // `keep` only.  Returns (FUSE, first pass) the rows of its blocks the guard flags.
    auto row_block = [&]<int CC, bool NR, bool RESCUE>(int64_t blk, const uint8_t* recc, unsigned keep) -> unsigned {
        using GE = Geo<CC, G>;
        constexpr int S = GE::S;
        unsigned flagged = 0;
        (void)keep;
        const int64_t mrow0 = blk * RPB + wave * (32 * MB);
        int64_t arow[MB];
        bool valid[MB];
        u16x8 bf[MB][S];
        constexpr int kOps = stage_direct_min_ops<GE::REC, NT>();
        // the first tiles start loading before the activations, so the two waits overlap
        if (t0 < t1) {
            if constexpr (GATHER) ring_barrier<0>();  // a previous row block's tiles are no longer read
#pragma unroll
            for (int x = 0; x < kRing - 1; ++x)
                stage_direct<GE::REC, NT>(recc + (size_t)min(t0 + x, t1 - 1) * GE::REC, lds + x * GE::BUF, tid);
        }
        if constexpr (GATHER) {
#pragma unroll
            for (int b = 0; b < MB; ++b) {
                arow[b] = src.row(mrow0 + 32 * b + i, m, valid[b]);
                float amax = 0.0f, ss = 0.0f;
                int64_t kst;
                const float* rp = row_ptr(a, arow[b], k, vec, kst);
                const int kv = opaque_vgpr(k);
                [&]<int... s>(std::integer_sequence<int, s...>) {
                    ((bf[b][s] = act_frag<CC, G, s>(rp, kst, valid[b], kv, vec > 0, h, amax, ss)), ...);
                }(std::make_integer_sequence<int, S>{});
            }
        } else {
            float araw[MB][ActPlan<CC, G>::NL][8];
#pragma unroll
            for (int b = 0; b < MB; ++b) {
                arow[b] = src.row(mrow0 + 32 * b + i, m, valid[b]);
                act_issue<CC, G>(a, valid[b] ? arow[b] : 0, k, vec, h, araw[b]);
            }
#pragma unroll
            for (int b = 0; b < MB; ++b) {
                float amax = 0.0f, ss = 0.0f;
                act_split_all<CC, G>(araw[b], h, bf[b], amax, ss);
                if constexpr (FUSE) {
                    // the guard's test, for this workgroup's own rescue below (no row list)
                    if constexpr (!RESCUE) {
                        const float am = fmaxf(amax, __shfl_xor(amax, 32, 64));
                        const float s2 = ss + __shfl_xor(ss, 32, 64);
                        if (valid[b] && (am > lim.prec || (am > lim.range_amax && s2 > lim.range_ss)))
                            flagged |= 1u << b;
                    }
                } else if (guard_header && chunk == 0) {
                    guard_append(amax, ss, lim, valid[b], arow[b], h, guard_header, guard_rows, guard_epoch,
                                 guard_cap);
                }
            }
        }

        float best[MB], sum[MB], ref[MB];
        int bt[MB];
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            best[b] = -INFINITY;
            sum[b] = 0.0f;
            ref[b] = 0.0f;
            bt[b] = -1;
        }

        // the loads of the kRing - 3 newest staged tiles may still be in flight at a barrier
        constexpr int kLead = (kRing - 3) * kOps;
        if (t0 < t1) {
            ring_barrier<kLead>();  // tiles t0 and t0+1 are in LDS
            f32x16 acc_a[MB], acc_b[MB];
#pragma unroll
            for (int b = 0; b < MB; ++b) acc_a[b] = f32x16{};
#pragma unroll
            for (int s = 0; s < S; ++s) {
                const u16x8 wf = weight_frag<CC, G>(lds, s, lb, i * 16, h);
#pragma unroll
                for (int b = 0; b < MB; ++b) acc_a[b] = mfma16<CfgT<CC>::f16>(wf, bf[b][s], acc_a[b]);
            }
            // One tile: start loading tile j+3, the MFMAs of tile j+1 into accM interleaved
            // with the epilogue of tile j on accE, the saves of a raised maximum, the rare
            // re-reference, the barrier (after which tile j+2 is in LDS).  Past the end the
            // MFMAs read a stale ring slot and the load repeats the last tile: harmless, and it
            // keeps the body branch-free.
            auto step = [&]<int R>(int j, f32x16 (&accE)[MB], f32x16 (&accM)[MB]) {
                constexpr unsigned rel = (unsigned)R;  // (j - t0) % kRing
                stage_direct<GE::REC, NT>(recc + (size_t)min(j + kRing - 1, t1 - 1) * GE::REC,
                                      lds + ((rel + kRing - 1) & (kRing - 1)) * GE::BUF, tid);
                const uint8_t* bufn = lds + ((rel + 1) & (kRing - 1)) * GE::BUF;
                const float* ep = reinterpret_cast<const float*>(lds + (rel & (kRing - 1)) * GE::BUF + GE::FRAG);
                f32x4 cs[2], cb[2];
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    cs[q] = *reinterpret_cast<const f32x4*>(ep + 8 * q + 4 * h);
                    cb[q] = *reinterpret_cast<const f32x4*>(ep + 32 + 8 * q + 4 * h);
                }
                EpiState<MB> st;
                st.need = false;
#pragma unroll
                for (int b = 0; b < MB; ++b) accM[b] = f32x16{};
                // weight fragments are read kPrefetch MFMA steps ahead of their use, so a wave
                // never waits on LDS with epilogue work queued behind the wait
                u16x8 wq[kPrefetch];
                frag_prefetch_first<CC, G, kPrefetch>(wq, bufn, lb, i * 16, h);
                // each MFMA step: the MFMA of block 0, half of the step's epilogue work, the
                // MFMAs of the other blocks and the fragment prefetch, the other half; so a
                // wave always has vector work to issue while its MFMAs run
                [&]<int... s>(std::integer_sequence<int, s...>) {
                    ([&] {
                        const u16x8& wf = frag_of<CC, G, kPrefetch, s>(wq);
                        accM[0] = mfma16<CfgT<CC>::f16>(wf, bf[0][s], accM[0]);
                        __builtin_amdgcn_sched_barrier(0);
                        epi_pieces_of_half<2 * S, 2 * s, MB, NR>(accE, ep, h, j, cs, cb, ref, best, bt, save, st);
                        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                        for (int b = 1; b < MB; ++b)
                            accM[b] = mfma16<CfgT<CC>::f16>(wf, bf[b][s], accM[b]);
                        frag_prefetch_after<CC, G, kPrefetch, s>(wq, bufn, lb, i * 16, h);
                        __builtin_amdgcn_sched_barrier(0);
                        epi_pieces_of_half<2 * S, 2 * s + 1, MB, NR>(accE, ep, h, j, cs, cb, ref, best, bt, save, st);
                        __builtin_amdgcn_sched_barrier(0);
                    }(), ...);
                }(std::make_integer_sequence<int, S>{});
                if (!NR && __any(st.need)) {
#pragma unroll
                    for (int b = 0; b < MB; ++b) {
                        if (best[b] != -INFINITY && __builtin_fabsf(best[b] - ref[b]) > 64.0f) {
                            const float nr = best[b];
                            sum[b] = (sum[b] == 0.0f) ? 0.0f : sum[b] * __builtin_amdgcn_exp2f(ref[b] - nr);
                            float s = 0.0f;
#pragma unroll
                            for (int r = 0; r < 16; ++r) s += __builtin_amdgcn_exp2f(accE[b][r] - nr);
                            st.tsum[b] = s;
                            ref[b] = nr;
                        }
                    }
                }
#pragma unroll
                for (int b = 0; b < MB; ++b) sum[b] += st.tsum[b];
                ring_barrier<kLead>();
            };
            // step R of the ring: the accumulator sets alternate (kRing is even)
            auto step_of = [&]<int R>(int jj) {
                if constexpr (R % 2 == 0) step.template operator()<R>(jj, acc_a, acc_b);
                else step.template operator()<R>(jj, acc_b, acc_a);
            };
            int j = t0;
            // unrolled by the ring's size, so every ring slot offset is a constant (immediate
            // LDS offsets, no address arithmetic per tile)
            static_assert(kRing >= 4 && (kRing & (kRing - 1)) == 0, "the ring is a power of two, at least 4");
            for (; j + kRing - 1 < t1; j += kRing)
                [&]<int... R>(std::integer_sequence<int, R...>) {
                    (step_of.template operator()<R>(j + R), ...);
                }(std::make_integer_sequence<int, kRing>{});
            [&]<int... R>(std::integer_sequence<int, R...>) {
                ((j + R < t1 ? step_of.template operator()<R>(j + R) : void()), ...);
            }(std::make_integer_sequence<int, kRing - 1>{});
            // the ring's last loads (repeats of the last tile) land before the workgroup ends
            __builtin_amdgcn_s_waitcnt(0x0 | (0x7 << 4) | (0xF << 8));  // vmcnt(0)
        }

        // first class of the best tile reaching the maximum; then lanes i and i+32 (same
        // activation row) merge and lanes 0-31 write.
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            int cls = 0;
            if (bt[b] >= 0) {
                int r0 = 16;
#pragma unroll
                for (int q = 3; q >= 0; --q) {
                    const f32x4 v = save[(b * 4 + q) * 64];
#pragma unroll
                    for (int e = 3; e >= 0; --e) r0 = (v[e] == best[b]) ? 4 * q + e : r0;
                }
                cls = bt[b] * 32 + (r0 < 16 ? 8 * (r0 >> 2) + 4 * h + (r0 & 3) : 0);
            }
            RowStat mine{best[b], sum[b], ref[b], cls};
            RowStat other{__shfl_xor(best[b], 32, 64), __shfl_xor(sum[b], 32, 64), __shfl_xor(ref[b], 32, 64),
                          __shfl_xor(cls, 32, 64)};
            const RowStat r = stat_merge(mine, other);
            if (h == 0 && valid[b] && (!RESCUE || ((keep >> b) & 1u))) {
                part[(int64_t)chunk * m + arow[b]] = Partial{r.best, r.sum, r.idx};
            }
        }
        return flagged;
    };
    if constexpr (GATHER) {
        for (int64_t blk = mbi; blk < blk_end; blk += mblocks)
            row_block.template operator()<C, NOREF, false>(blk, rec, 0u);
    } else if constexpr (FUSE) {
        // small batches: the rows the guard flags are recomputed here, by the workgroups that
        // hold them, with three bf16 terms (the rescue configuration's records, rec3), instead
        // of by a rescue launch; every wave has left the first pass's ring at the barrier
        static_assert(MB == 1 && Geo<CFG_Q3, G>::BUF == GE::BUF, "the fused rescue shares the ring");
        (void)blk_end;
        const unsigned fl = row_block.template operator()<C, NOREF, false>(mbi, rec, 0u);
        if (__syncthreads_or(fl != 0u)) {
            // the first pass's last (clamped) tile loads may still be landing in the ring:
            // every wave drains its own before any restages a slot
            ring_barrier<0>();
            row_block.template operator()<CFG_Q3, false, true>(mbi, rec3, fl);
        }
    } else {
        (void)blk_end;
        (void)rec3;
        row_block.template operator()<C, NOREF, false>(mbi, rec, 0u);
    }
}


// ============================================================ logits / probabilities writer
// One producer wave loads weight tiles from global memory straight into LDS; the consumer
// waves compute and store.  Every access by one wave to global memory counts in its one
// in-order vmcnt, so a wave that both stored results and loaded tiles would wait for its
// own stores each time it waited for a tile.  Here the producer never stores, and the
// consumers never wait for memory: their stores stay in flight while they compute the
// next tiles.  Direct loads of one wave (64 lanes x 16 bytes per instruction):
template <int REC>
__device__ __forceinline__ void stage_wave(const uint8_t* __restrict__ src, uint8_t* dst, int lane) {
    constexpr int CH = REC / 16;
    constexpr int PER = (CH + 63) / 64;
    static_assert(REC % 16 == 0, "tile record size");
#pragma unroll
    for (int x = 0; x < PER; ++x) {
        // the last instruction of a record that is not a multiple of 1 KiB has some lanes off,
        // never all of them, so each instruction counts once in vmcnt
        if (CH % 64 == 0 || x * 64 + lane < CH)
            __builtin_amdgcn_global_load_lds(
                static_cast<const void*>(src + (size_t)(x * 64 + lane) * 16),
                reinterpret_cast<__attribute__((address_space(3))) void*>(
                    reinterpret_cast<uintptr_t>(dst + (size_t)x * 1024)),
                16, 0, 0);
    }
}
template <int REC>
constexpr int stage_wave_ops() {
    return (REC / 16 + 63) / 64;
}
__device__ __forceinline__ void barrier_lds() {
    __builtin_amdgcn_s_waitcnt(0xF | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));  // lgkmcnt(0) only
    asm volatile("s_barrier" ::: "memory");
}

// Ring depth of the writer: tiles held in LDS, limited by the vmcnt range of the
// producer's wait (R - 2 tiles of loads in flight).
template <int REC>
constexpr int writer_ring() {
    return 2 + 63 / stage_wave_ops<REC>() < 8 ? 2 + 63 / stage_wave_ops<REC>() : 8;
}

// Projection writing logits (EPI 0) or softmax probabilities (EPI 1).  A workgroup owns
// 32 * NC activation rows.  Waves 0..NC-1 are consumers, one 32-row block each; wave NC is
// the producer: it keeps a ring of R weight tiles in LDS, R - 1 tiles ahead of the
// consumers, so every tile read from L2 serves 32 * NC rows.  Each step all consumers
// take the same tile and write its 32 classes of their rows, rows front to back.
// Orientation: rows of the MFMA = activation rows, columns = classes; a lane holds one
// class of 16 rows, so each store instruction writes 32 consecutive classes of two rows.
// GATHER: the rows are the entries of the guard list (the rescue of guarded rows); a
// workgroup then takes several row blocks and the producer streams the tiles once per block.
template <int C, int G, int EPI, bool GATHER>
__global__ __launch_bounds__(64 * (kWriterWaves + 1), 1) void rows_w_kernel(
    const float* __restrict__ a, int64_t m, int k, int vec, const uint8_t* __restrict__ rec, int tiles, int n,
    int nsplit, int tiles_per_chunk, int mblocks, const float* __restrict__ row_max,
    const float* __restrict__ row_inv, float* __restrict__ out, GuardLimits lim,
    unsigned long long* __restrict__ guard_header, int* __restrict__ guard_rows, unsigned guard_epoch, int guard_cap) {
    using GE = Geo<C, G>;
    constexpr int S = GE::S;
    constexpr int NC = kWriterWaves;
    constexpr int R = writer_ring<GE::REC>();
    constexpr int ROWS = 32 * NC;
    extern __shared__ __align__(16) uint8_t lds[];  // [R tiles] x BUF

    int mbi, chunk;
    map_block<false>(blockIdx.x, nsplit, &mbi, &chunk);
    if (mbi >= mblocks) return;
    const int t0 = chunk * tiles_per_chunk;
    const int t1 = min(t0 + tiles_per_chunk, tiles);
    if (t0 >= t1) return;
    const RowSource src{GATHER ? guard_rows : nullptr, GATHER ? guard_count_of(guard_header, guard_epoch, guard_cap) : 0};
    const int64_t blk_end = GATHER ? ((int64_t)src.count + ROWS - 1) / ROWS : (int64_t)mbi + 1;
    const int64_t nblk = (blk_end - mbi + mblocks - 1) / mblocks;  // row blocks of this workgroup
    if (nblk <= 0) return;
    const int ntiles = t1 - t0;
    // Each workgroup walks its chunk's tiles from its own starting tile.  Walking them in
    // step, the CUs of an XCD read the same tile record at once and its L2 channels queue:
    // with the write stream running, L2 read latency rose from about 300 cycles (one tile
    // re-read) to 1450 and write latency from 320 to 1000 (TCP_TCC_*_REQ_LATENCY), and the
    // logits kernel took 843 us instead of 648 (dense batch, same box).
    const int rot = (int)(((int64_t)mbi * 149) % ntiles);
    const int64_t total = nblk * ntiles;

    const int tid = threadIdx.x, lane = tid & 63, i = lane & 31, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    if (wave == NC) {
        // ---- producer: the g-th tile of the sequence goes to ring slot g % R
        constexpr int kOps = stage_wave_ops<GE::REC>();
        int pt = t0 + rot, pslot = 0;  // next tile to stage and its ring slot
        auto stage_next = [&] {
            stage_wave<GE::REC>(rec + (size_t)pt * GE::REC, lds + pslot * GE::BUF, lane);
            pt = pt + 1 == t1 ? t0 : pt + 1;
            pslot = pslot + 1 == R ? 0 : pslot + 1;
        };
#pragma unroll
        for (int g = 0; g < R - 1; ++g) stage_next();
        vm_wait<kOps * (R - 2)>();  // tile 0 is in LDS
        barrier_lds();
        for (int64_t g = 0; g < total; ++g) {
            // tile g + R - 1 goes to the slot read at step g - 1, which every consumer has
            // finished; past the end the loads repeat tiles into slots nobody reads
            stage_next();
            vm_wait<kOps * (R - 2)>();  // tile g + 1 is in LDS
            barrier_lds();
        }
        vm_wait<0>();  // the ring's last loads land before the workgroup ends
        return;
    }

    // ---- consumers
    // the zero block after each of the R slots
    for (int x = tid >> 5; x < R; x += 2 * NC)
        reinterpret_cast<u32x4*>(lds + x * GE::BUF + GE::REC)[tid & 31] = u32x4{0, 0, 0, 0};
    barrier_lds();  // zero blocks written; tile 0 is in LDS
    int cslot = 0;  // ring slot of the current tile
    auto row_block = [&](int64_t blk) {
        const int64_t j0 = blk * ROWS + wave * 32;
        bool valid;
        const int64_t arow = src.row(j0 + i, m, valid);
        float amax = 0.0f, ss = 0.0f;
        u16x8 bf[S];
        if constexpr (GATHER) {
            int64_t kst;
            const float* rp = row_ptr(a, arow, k, vec, kst);
            const int kv = opaque_vgpr(k);
            [&]<int... s>(std::integer_sequence<int, s...>) {
                ((bf[s] = act_frag<C, G, s>(rp, kst, valid, kv, vec > 0, h, amax, ss)), ...);
            }(std::make_integer_sequence<int, S>{});
        } else {
            float araw[ActPlan<C, G>::NL][8];
            act_issue<C, G>(a, valid ? arow : 0, k, vec, h, araw);
            act_split_all<C, G>(araw, h, bf, amax, ss);
        }
        if (!GATHER && guard_header && chunk == 0)
            guard_append(amax, ss, lim, valid, arow, h, guard_header, guard_rows, guard_epoch, guard_cap);
        // rows of this lane's 16 accumulators (r -> row slot 8*(r/4) + 4*h + (r%4))
        int orow[16];  // rows are below 2^31 (the entry points check m)
        bool ovalid[16];
        bool all_valid = true;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            bool v;
            orow[r] = (int)src.row(j0 + 8 * (r >> 2) + 4 * h + (r & 3), m, v);
            ovalid[r] = v;
            all_valid = all_valid && v;
        }
        all_valid = __all(all_valid);
        float rmax[16], rinv[16];
        if constexpr (EPI == 1) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                rmax[r] = ovalid[r] ? row_max[orow[r]] : 0.0f;
                rinv[r] = ovalid[r] ? row_inv[orow[r]] : 0.0f;
            }
        }

        for (int t = t0; t < t1; ++t) {
            const uint8_t* buf = lds + cslot * GE::BUF;
            cslot = cslot + 1 == R ? 0 : cslot + 1;
            // weight fragments are read kAhead MFMA steps ahead of their use, so the LDS reads
            // overlap instead of each MFMA waiting on its own
            // (the gathered probabilities variant also holds each row's statistics: a lead
            // of two keeps it within its registers, without scratch)
            constexpr int kLead = (GATHER && EPI == 1) ? 2 : 8;
            constexpr int kAhead = S < kLead ? S : kLead;
            u16x8 wq[kAhead];
            frag_prefetch_first<C, G, kAhead>(wq, buf, i * 16 + h * 512, i * 16, h);
            f32x16 acc = {};
            [&]<int... st>(std::integer_sequence<int, st...>) {
                ([&] {
                    acc = mfma16<CfgT<C>::f16>(bf[st], frag_of<C, G, kAhead, st>(wq), acc);
                    frag_prefetch_after<C, G, kAhead, st>(wq, buf, i * 16 + h * 512, i * 16, h);
                    __builtin_amdgcn_sched_barrier(0);
                }(), ...);
            }(std::make_integer_sequence<int, S>{});
            const float* ep = reinterpret_cast<const float*>(buf + GE::FRAG);
            float c0, c1;
            if constexpr (EPI == 0) {
                c0 = ep[64 + i];  // scale
                c1 = ep[96 + i];  // bias
            } else {
                c0 = ep[i];       // scale * log2(e)
                c1 = ep[32 + i];  // bias * log2(e)
            }
            const int tt = t0 + (t - t0 + rot) % ntiles;  // the producer's sequence starts at t0 + rot
            const int col = tt * 32 + i;
            float v[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                if constexpr (EPI == 0) {
#pragma clang fp contract(off)
                    v[r] = acc[r] * c0 + c1;  // (sum * scale) + bias, two roundings (src/ops/matmul.rs:1396-1409)
                } else {
                    v[r] = __builtin_amdgcn_exp2f(fmaf(acc[r], c0, c1) - rmax[r]) * rinv[r];
                }
            }
            if (all_valid && tt * 32 + 32 <= n) {
#pragma unroll
                for (int r = 0; r < 16; ++r) out[(int64_t)orow[r] * n + col] = v[r];
            } else if (col < n) {
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (ovalid[r]) out[(int64_t)orow[r] * n + col] = v[r];
            }
            barrier_lds();  // this slot is read; tile g + 1 is in LDS
        }
    };
    if constexpr (GATHER) {
        for (int64_t blk = mbi; blk < blk_end; blk += mblocks) row_block(blk);
    } else {
        row_block(mbi);
    }
}

// ============================================================ per-configuration launchers
// Each is instantiated explicitly in one of the head_cfg_*.hip translation units (one per
// family of configurations, so the kernels compile in parallel) and called by the host
// dispatch in head_mfma.hip.

// 32-row blocks per wave of the main statistics pass: two for the one- and two-term modes
// (each weight fragment read from LDS serves both), one for three products (registers).
template <int C>
constexpr int mb_of() {
    return (C == CFG_Q1 || C == CFG_Q2 || C == CFG_F1 || C == CFG_H2) ? 2 : 1;
}
template <int C, int G, int MB, bool GATHER, bool NOREF, bool SKIP = false, bool FUSE = false>
static void stats_go(const StatsLaunch& x, unsigned grid, hipStream_t st) {
    stats_main_kernel<C, G, MB, GATHER, NOREF, SKIP, FUSE><<<grid, 64 * kStatsWaves, main_lds_bytes<C, G, MB>(), st>>>(
        x.a, x.m, x.k, x.vec, x.rec, x.tiles, x.nsplit, x.tpc, x.mblocks, x.part, x.lim,
        x.guard_header, x.guard_rows, x.guard_epoch, x.guard_cap, x.skip, x.rec3);
}

// Main statistics pass.  The two-term modes run mb = 1 (small batches) or 2 blocks per
// wave, with or without the reference shift (noref); the others their one variant.
template <int C, int G>
int stats_main_cfg(const StatsLaunch& x, int mb, bool noref, unsigned grid, hipStream_t st) {
    if constexpr (C == CFG_Q2) {
        // the variants that skip listed row blocks only where the host asks for them
        if (mb == 1) {
            if (x.skip) {
                if (noref) stats_go<C, G, 1, false, true, true>(x, grid, st);
                else stats_go<C, G, 1, false, false, true>(x, grid, st);
            } else if (x.rec3) {
                if (noref) stats_go<C, G, 1, false, true, false, true>(x, grid, st);
                else stats_go<C, G, 1, false, false, false, true>(x, grid, st);
            } else {
                if (noref) stats_go<C, G, 1, false, true>(x, grid, st);
                else stats_go<C, G, 1, false, false>(x, grid, st);
            }
        } else {
            if (x.skip) {
                if (noref) stats_go<C, G, 2, false, true, true>(x, grid, st);
                else stats_go<C, G, 2, false, false, true>(x, grid, st);
            } else {
                if (noref) stats_go<C, G, 2, false, true>(x, grid, st);
                else stats_go<C, G, 2, false, false>(x, grid, st);
            }
        }
    } else if constexpr (C == CFG_H2) {
        if (mb == 1) {
            if (x.rec3) {
                if (noref) stats_go<C, G, 1, false, true, false, true>(x, grid, st);
                else stats_go<C, G, 1, false, false, false, true>(x, grid, st);
            } else {
                if (noref) stats_go<C, G, 1, false, true>(x, grid, st);
                else stats_go<C, G, 1, false, false>(x, grid, st);
            }
        } else {
            if (noref) stats_go<C, G, 2, false, true>(x, grid, st);
            else stats_go<C, G, 2, false, false>(x, grid, st);
        }
    } else {
        (void)mb;
        (void)noref;
        stats_go<C, G, mb_of<C>(), false, false>(x, grid, st);
    }
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

// Rescue pass of the statistics: the rows of the guard list (gather mode).
template <int C, int G>
int stats_gather_cfg(const StatsLaunch& x, unsigned grid, hipStream_t st) {
    stats_go<C, G, mb_of<C>(), true, false>(x, grid, st);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

// Logits (epi 0) or probabilities (epi 1) writer; GATHER: the rows of the guard list.
template <int C, int G, bool GATHER>
int rows_cfg(const RowsLaunch& x, int epi, unsigned grid, hipStream_t st) {
    constexpr int LDS = writer_ring<Geo<C, G>::REC>() * Geo<C, G>::BUF;
    auto kern = epi == 0 ? rows_w_kernel<C, G, 0, GATHER> : rows_w_kernel<C, G, 1, GATHER>;
    kern<<<grid, 64 * (kWriterWaves + 1), LDS, st>>>(x.a, x.m, x.k, x.vec, x.rec, x.tiles, x.n, x.nsplit, x.tpc,
                                                      x.mblocks, x.row_max, x.row_inv, x.out, x.lim,
                                                      x.guard_header, x.guard_rows, x.guard_epoch, x.guard_cap);
    PPOCR_HIP(hipGetLastError());
    return PPOCR_OK;
}

}  // namespace ppocr
