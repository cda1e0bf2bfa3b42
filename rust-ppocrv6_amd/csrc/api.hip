// The extern "C" boundary (include/ppocr_rechead.h): head handles, argument checks with
// the reference's error messages, and the host/device entry points.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "model_graph.hpp"
#include "neck.hpp"
#include "safetensors.hpp"

namespace ppocr {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
int fail(int code, const std::string& msg) {
    set_error(msg);
    return code;
}

}  // namespace ppocr

using namespace ppocr;

struct ppocr_rh {
    int device = 0;
    int64_t n = 0, k = 0;
    bool quantized = true;
    TileGeom geom{};
    bool mfma_ok = false;
    // device memory
    int8_t* d_q = nullptr;     // [n][k] packed INT8 weight (INT8 head)
    float* d_w = nullptr;      // [n][k] fp32 W^T (FP32 head)
    float* d_scale = nullptr;  // [n] per-class scale (1.0 for an FP32 head)
    float* d_bias = nullptr;   // [n] bias (0 when absent)
    uint8_t* d_rec = nullptr;    // tiles x rec_bytes MFMA tile records, bf16 fragments
    uint8_t* d_rec_h = nullptr;  // the same with fp16 fragments (F16X2)
    size_t device_bytes = 0;
    FmaWeights fma{};            // the device weights above, for the fp32 FMA kernels
    // Precision guards of the split modes: rows with max|a| above the limit are recomputed
    // (three bf16 terms for an INT8 head, fp32 FMA for an FP32 head).  amax_limit: bf16
    // terms (BF16X2, an FP32 head's BF16X3); amax_limit_h: fp16 terms (F16X2).
    float amax_limit = INFINITY;
    float amax_limit_h = INFINITY;
    bool f16_ok = true;  // the weights fit fp16 (always for INT8; |w| < 32768 for FP32)
    // Rows with max|a| at most range_limit have every logit in [-kLogitBound, kLogitBound]:
    // |logit| <= max|a| * max_c sum_k |w_ck| + max_c |b_c| (range_ok: such a bound exists).
    float range_limit = 0.0f;
    // ... or rows with ||a||_2^2 at most range_ss: |logit| <= ||a||_2 * max_c ||w_c||_2 + max_c |b_c|
    float range_ss = 0.0f;
    bool range_ok = false;
};

namespace {

// Every device allocation of the library goes through these two, so that tests can make
// them fail: with PPOCR_RECHEAD_FAULT=alloc in the environment (read at each allocation),
// they return hipErrorOutOfMemory without allocating, as an exhausted HBM would, and the
// calls report PPOCR_ERR_NO_MEMORY.
bool alloc_fault() {
    const char* v = std::getenv("PPOCR_RECHEAD_FAULT");
    return v && std::strcmp(v, "alloc") == 0;
}
hipError_t dev_malloc(void** p, size_t bytes) {
    if (alloc_fault()) {
        *p = nullptr;
        return hipErrorOutOfMemory;
    }
    return hipMalloc(p, bytes);
}
hipError_t dev_malloc_async(void** p, size_t bytes, hipStream_t st) {
    if (alloc_fault()) {
        *p = nullptr;
        return hipErrorOutOfMemory;
    }
    return hipMallocAsync(p, bytes, st);
}

struct DeviceGuard {
    int prev = -1;
    int err = 0;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev && hipSetDevice(dev) != hipSuccess) err = 1;
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

// Device memory of the host-pointer entry points.  Each call takes an arena (one device
// allocation, a pinned host staging buffer and a stream of its own) from a pool, lays its
// inputs, outputs and workspace out in it, and gives it back, so a call costs its copies
// and kernels rather than allocations.  Inputs and outputs of up to kStageBytes move as
// one copy each way through the pinned buffer; larger ones are copied directly.  Calls
// running at the same time take different arenas.  Arenas above kArenaKeepBytes are freed
// after the call instead of kept (the logits of a large batch need gigabytes once).  The
// pool lives until the process ends.
constexpr size_t kArenaKeepBytes = 256u << 20;
constexpr size_t kStageBytes = 4u << 20;

struct HostArena {
    int device = -1;
    hipStream_t stream = nullptr;
    uint8_t* base = nullptr;
    size_t cap = 0;
    uint8_t* pinned = nullptr;  // kStageBytes, allocated on first use
};

class ArenaPool {
public:
    HostArena* take(int device) {
        std::lock_guard<std::mutex> lk(mu_);
        for (size_t i = 0; i < idle_.size(); ++i) {
            if (idle_[i]->device == device) {
                HostArena* a = idle_[i];
                idle_.erase(idle_.begin() + (std::ptrdiff_t)i);
                return a;
            }
        }
        HostArena* a = new (std::nothrow) HostArena;
        if (a) a->device = device;
        return a;
    }
    void give(HostArena* a) {
        std::lock_guard<std::mutex> lk(mu_);
        idle_.push_back(a);
    }

private:
    std::mutex mu_;
    std::vector<HostArena*> idle_;
};

ArenaPool& arena_pool() {
    static ArenaPool* pool = new ArenaPool;  // never destroyed: arenas may be in use until exit
    return *pool;
}

size_t align256(size_t x) { return (std::max<size_t>(x, 1) + 255) / 256 * 256; }

// One host-pointer call on the current device: the workspace, then the inputs, then the
// outputs, each 256-byte aligned in the arena.  The workspace starts the arena, so its
// guard header (offset 0) is the same word in every call; it is cleared whenever the arena
// is allocated.  The destructor waits for the call's stream before the arena goes back.
class HostCall {
public:
    ~HostCall() {
        if (!a_) return;
        (void)hipStreamSynchronize(a_->stream);
        if (a_->cap > kArenaKeepBytes) {
            (void)hipFree(a_->base);
            a_->base = nullptr;
            a_->cap = 0;
        }
        arena_pool().give(a_);
    }
    int begin(std::initializer_list<size_t> in, std::initializer_list<size_t> out, size_t ws) {
        int dev = 0;
        PPOCR_HIP(hipGetDevice(&dev));
        a_ = arena_pool().take(dev);
        if (!a_) return fail(PPOCR_ERR_NO_MEMORY, "RecHeadHip: host allocation failed");
        if (!a_->stream) PPOCR_HIP(hipStreamCreateWithFlags(&a_->stream, hipStreamNonBlocking));
        ws_off_ = 0;
        ws_bytes_ = align256(ws);
        size_t total = ws_bytes_;
        in_begin_ = total;
        for (size_t r : in) place(r, &total, &in_);
        in_end_ = total;
        for (size_t r : out) place(r, &total, &out_);
        out_end_ = total;
        if (a_->cap < total) {
            if (a_->base) (void)hipFree(a_->base);
            a_->base = nullptr;
            a_->cap = 0;
            void* p = nullptr;
            if (dev_malloc(&p, total) != hipSuccess) {
                (void)hipGetLastError();
                return fail(PPOCR_ERR_NO_MEMORY, "RecHeadHip: device allocation of " + std::to_string(total) +
                                                     " bytes failed");
            }
            a_->base = static_cast<uint8_t*>(p);
            a_->cap = total;
            if (int e = launch_guard_clear(reinterpret_cast<unsigned long long*>(a_->base), a_->stream)) return e;
        }
        if (!a_->pinned && (in_end_ - in_begin_ <= kStageBytes || out_end_ - in_end_ <= kStageBytes)) {
            void* p = nullptr;
            if (hipHostMalloc(&p, kStageBytes, hipHostMallocDefault) == hipSuccess) a_->pinned = static_cast<uint8_t*>(p);
            else (void)hipGetLastError();  // no staging: copies go directly
        }
        return PPOCR_OK;
    }
    template <typename T>
    T* in(size_t i) const {
        return reinterpret_cast<T*>(a_->base + in_[i].first);
    }
    template <typename T>
    T* out(size_t i) const {
        return reinterpret_cast<T*>(a_->base + out_[i].first);
    }
    uint8_t* ws() const { return a_->base + ws_off_; }
    size_t ws_bytes() const { return ws_bytes_; }
    hipStream_t stream() const { return a_->stream; }
    // Copies the inputs (srcs in the order given to begin) to the device.
    int copy_in(std::initializer_list<const void*> srcs) const {
        size_t i = 0;
        const size_t span = in_end_ - in_begin_;
        const bool staged = a_->pinned && span <= kStageBytes;
        for (const void* src : srcs) {
            const auto [off, n] = in_[i++];
            if (!n || !src) continue;
            if (staged) std::memcpy(a_->pinned + (off - in_begin_), src, n);
            else PPOCR_HIP(hipMemcpyAsync(a_->base + off, src, n, hipMemcpyHostToDevice, a_->stream));
        }
        if (staged && span)
            PPOCR_HIP(hipMemcpyAsync(a_->base + in_begin_, a_->pinned, span, hipMemcpyHostToDevice, a_->stream));
        return PPOCR_OK;
    }
    // Copies the outputs back (dsts in the order given to begin; null ones are skipped) and
    // waits for the call to finish.
    int copy_out(std::initializer_list<void*> dsts) const {
        const size_t span = out_end_ - in_end_;
        const bool staged = a_->pinned && span <= kStageBytes;
        if (staged) {
            if (span) PPOCR_HIP(hipMemcpyAsync(a_->pinned, a_->base + in_end_, span, hipMemcpyDeviceToHost, a_->stream));
        } else {
            size_t i = 0;
            for (void* dst : dsts) {
                const auto [off, n] = out_[i++];
                if (n && dst) PPOCR_HIP(hipMemcpyAsync(dst, a_->base + off, n, hipMemcpyDeviceToHost, a_->stream));
            }
        }
        PPOCR_HIP(hipStreamSynchronize(a_->stream));
        if (staged) {
            size_t i = 0;
            for (void* dst : dsts) {
                const auto [off, n] = out_[i++];
                if (n && dst) std::memcpy(dst, a_->pinned + (off - in_end_), n);
            }
        }
        return PPOCR_OK;
    }

private:
    static void place(size_t bytes, size_t* total, std::vector<std::pair<size_t, size_t>>* v) {
        v->push_back({*total, bytes});
        *total += align256(bytes);
    }
    HostArena* a_ = nullptr;
    std::vector<std::pair<size_t, size_t>> in_, out_;  // (offset, bytes)
    size_t in_begin_ = 0, in_end_ = 0, out_end_ = 0, ws_off_ = 0, ws_bytes_ = 0;
};

// Device buffer owned for the duration of a host-pointer call.
struct DevBuf {
    void* p = nullptr;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
    int alloc(size_t bytes) {
        if (bytes == 0) bytes = 1;
        if (dev_malloc(&p, bytes) != hipSuccess) {
            p = nullptr;
            (void)hipGetLastError();
            return fail(PPOCR_ERR_NO_MEMORY, "RecHeadHip: device allocation of " + std::to_string(bytes) + " bytes failed");
        }
        return PPOCR_OK;
    }
    template <typename T>
    T* as() const {
        return static_cast<T*>(p);
    }
};

uint16_t bf16_bits_rne(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffff) ? 0x40 : 0));
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
float bf16_to_float(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// Build the MFMA tile records on the host (see TileGeom in kernels.hpp).
uint16_t f16_bits_rne(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }
float f16_to_float(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }

std::vector<uint8_t> build_records(const TileGeom& g, int64_t n, int64_t k, const int8_t* q, const float* w,
                                   const float* scale, const float* bias, bool f16) {
    std::vector<uint8_t> rec((size_t)g.tiles * g.rec_bytes(), 0);
    for (int t = 0; t < g.tiles; ++t) {
        uint8_t* r = rec.data() + (size_t)t * g.rec_bytes();
        uint16_t* frag = reinterpret_cast<uint16_t*>(r);
        for (int i = 0; i < 32; ++i) {
            const int64_t row = (int64_t)t * 32 + i;
            if (row >= n) continue;
            for (int64_t kk = 0; kk < k; ++kk) {
                const int gg = (int)(kk / 8), e = (int)(kk % 8);
                uint16_t hi, lo = 0;
                if (f16) {
                    const float v = q ? (float)q[row * k + kk] : w[row * k + kk];
                    hi = f16_bits_rne(v);  // exact for int8 values
                    if (!q) lo = f16_bits_rne(v - f16_to_float(hi));
                } else if (q) {
                    hi = bf16_bits_rne((float)q[row * k + kk]);  // exact
                } else {
                    const float v = w[row * k + kk];
                    hi = bf16_bits_rne(v);
                    lo = bf16_bits_rne(v - bf16_to_float(hi));
                }
                frag[((size_t)(0 * g.G + gg) * 32 + i) * 8 + e] = hi;
                if (g.wplanes == 2) frag[((size_t)(1 * g.G + gg) * 32 + i) * 8 + e] = lo;
            }
        }
        float* ep = reinterpret_cast<float*>(r + g.frag_bytes());
        for (int i = 0; i < 32; ++i) {
            const int64_t row = (int64_t)t * 32 + i;
            if (row < n) {
                const float sc = scale[row], bi = bias ? bias[row] : 0.0f;
                ep[i] = sc * kLog2e;
                ep[32 + i] = bi * kLog2e;
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
    return rec;
}

void free_handle(ppocr_rh* h) {
    if (!h) return;
    DeviceGuard dg(h->device);
    if (h->d_q) (void)hipFree(h->d_q);
    if (h->d_w) (void)hipFree(h->d_w);
    if (h->d_scale) (void)hipFree(h->d_scale);
    if (h->d_bias) (void)hipFree(h->d_bias);
    if (h->d_rec) (void)hipFree(h->d_rec);
    if (h->d_rec_h) (void)hipFree(h->d_rec_h);
    delete h;
}

template <typename T>
int upload(T** dst, const T* src, size_t count, size_t* total) {
    const size_t bytes = std::max<size_t>(count * sizeof(T), 1);
    if (dev_malloc((void**)dst, bytes) != hipSuccess) {
        *dst = nullptr;
        (void)hipGetLastError();
        return fail(PPOCR_ERR_NO_MEMORY, "RecHeadHip: device allocation failed");
    }
    *total += bytes;
    if (count) PPOCR_HIP(hipMemcpy(*dst, src, count * sizeof(T), hipMemcpyHostToDevice));
    return PPOCR_OK;
}

// Checks shared by every way of creating a head; makes `device` current.
int check_create(const char* op, int64_t n, int64_t k, int device, ppocr_rh_t** out) {
    if (!out) return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": out handle pointer is null");
    *out = nullptr;
    if (n <= 0 || k <= 0) return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": weight must have positive shape");
    if (n > (1LL << 30) || k > (1LL << 20)) return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": weight too large");
    int ndev = 0;
    PPOCR_HIP(hipGetDeviceCount(&ndev));
    if (device < 0 || device >= ndev)
        return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: device " + std::to_string(device) + " out of range");
    return PPOCR_OK;
}

ppocr_rh* new_handle(int64_t n, int64_t k, bool quantized, int device) {
    ppocr_rh* h = new (std::nothrow) ppocr_rh;
    if (!h) return nullptr;
    h->device = device;
    h->n = n;
    h->k = k;
    h->quantized = quantized;
    h->geom.G = (int)((k + 7) / 8);
    h->geom.wplanes = quantized ? 1 : 2;
    h->geom.tiles = (int)((n + 31) / 32);
    h->mfma_ok = mfma_supports_groups(h->geom.G);
    return h;
}

// The split modes' logit error grows with max|a| * ||w_c||_2.  Measured on N(0, 0.05^2)
// heads (k = 120, 18710 classes, rows scaled to a given max|a|), the largest error over
// 4.8M logits is about 4.7e-6 * max|a| * L2 for the INT8 head's two activation terms and
// 9.5e-6 * max|a| * L2 for an FP32 head's three bf16 products (whose floor is the
// two-plane split of the weight).  These bounds on max|a| * L2 keep it near 5e-5, half the
// 1e-4 bar; rows above are recomputed.
constexpr double kSplitBoundInt8 = 8.0;
constexpr double kSplitBoundF32 = 4.0;
// Two fp16 terms keep 22 bits of the activation: measured the same way, the largest error
// is about 8.7e-8 * max|a| * L2 (INT8 head) and 6.6e-7 * max|a| * L2 (an FP32 head with fp16
// halves of both operands, as accurate as the fp32 product itself).  An fp16 term also
// caps the magnitude: rows with max|a| above kF16Range are recomputed whatever the weights.
constexpr double kSplitBoundF16Int8 = 512.0;
constexpr double kSplitBoundF16F32 = 64.0;
constexpr double kF16Range = 32768.0;

// Guard limits from wmax = max_c max_k |w_ck| (float), w1 = max_c sum_k |w_ck|,
// l2 = max_c ||w_c||_2 and bmax = max_c |b_c| (double), w the dequantised weight.
void set_limits(ppocr_rh* h, float wmax, double w1, double l2, double bmax) {
    double lim = wmax > 0.0f ? 16.0 / (double)wmax : INFINITY;
    double lim_h = kF16Range;
    if (l2 > 0.0 && std::isfinite(l2)) {
        lim = std::min(lim, (h->quantized ? kSplitBoundInt8 : kSplitBoundF32) / l2);
        lim_h = std::min(lim_h, (h->quantized ? kSplitBoundF16Int8 : kSplitBoundF16F32) / l2);
    }
    if (!std::isfinite(l2)) lim = lim_h = 0.0;  // inf or NaN weights: every row goes to the rescue
    h->amax_limit = (float)lim;
    h->amax_limit_h = (float)lim_h;
    h->f16_ok = h->quantized || (double)wmax < kF16Range;
    // logit range bound: the largest L1 norm of a dequantised weight row and the largest
    // |bias|, rounded up by a small margin
    const double room = (double)kLogitBound - bmax * 1.001;
    if (room > 0.0 && std::isfinite(w1) && std::isfinite(bmax) && std::isfinite(l2)) {
        h->range_limit = (float)(w1 > 0.0 ? room / (w1 * 1.001) : INFINITY);
        // the kernels sum the squares in fp32 (120 terms: relative error below 1e-5), so
        // the limit on ||a||_2^2 keeps a further 0.1% margin
        const double nl = l2 > 0.0 ? room / (l2 * 1.001) : INFINITY;
        h->range_ss = (float)(nl * nl * 0.999);
        h->range_ok = true;
    }
}

// Guard limits of a head whose weights, scales and bias are on the device, reduced there
// (the same kernel for every way of creating a head, so equal weights give equal limits).
int device_limits(ppocr_rh* h, bool has_bias) {
    DevBuf lim;
    if (int e = lim.alloc(sizeof(HeadLimitBits))) return e;
    PPOCR_HIP(hipMemset(lim.p, 0, sizeof(HeadLimitBits)));
    if (int e = launch_head_limits(h->d_q, h->d_w, h->d_scale, has_bias ? h->d_bias : nullptr, h->n, h->k,
                                   lim.as<HeadLimitBits>(), nullptr))
        return e;
    HeadLimitBits hl;
    PPOCR_HIP(hipMemcpy(&hl, lim.p, sizeof(hl), hipMemcpyDeviceToHost));
    float wmax;
    double w1, l2, bmax;
    const unsigned wbits = hl.wmax;
    std::memcpy(&wmax, &wbits, 4);
    std::memcpy(&w1, &hl.w1, 8);
    std::memcpy(&l2, &hl.l2, 8);
    std::memcpy(&bmax, &hl.bmax, 8);
    set_limits(h, wmax, w1, l2, bmax);
    return PPOCR_OK;
}

int create_common(const int8_t* q, const float* w_t, const float* scales, const float* bias, int64_t n, int64_t k,
                  int device, ppocr_rh_t** out) {
    const char* op = q ? "MatMulQuantizedB" : "MatMulTransposedB";
    if (int e = check_create(op, n, k, device, out)) return e;
    if ((q && !scales) || (!q && !w_t)) return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": null weight pointer");
    DeviceGuard dg(device);
    if (dg.err) return fail(PPOCR_ERR_DEVICE, "RecHeadHip: hipSetDevice failed");

    std::unique_ptr<ppocr_rh, void (*)(ppocr_rh*)> h(new_handle(n, k, q != nullptr, device), free_handle);
    if (!h) return fail(PPOCR_ERR_NO_MEMORY, "RecHeadHip: host allocation failed");

    std::vector<float> sc_host;
    const float* sc = scales;
    if (!q) {
        sc_host.assign((size_t)n, 1.0f);
        sc = sc_host.data();
    }
    std::vector<float> bias_host;
    const float* bi = bias;
    if (!bias) {
        bias_host.assign((size_t)n, 0.0f);
        bi = bias_host.data();
    }
    size_t total = 0;
    if (q) {
        if (int e = upload(&h->d_q, q, (size_t)(n * k), &total)) return e;
    } else {
        if (int e = upload(&h->d_w, w_t, (size_t)(n * k), &total)) return e;
    }
    if (int e = upload(&h->d_scale, sc, (size_t)n, &total)) return e;
    if (int e = upload(&h->d_bias, bi, (size_t)n, &total)) return e;
    h->fma = FmaWeights{h->d_q, h->d_w, h->d_scale, h->d_bias};
    if (int e = device_limits(h.get(), bias != nullptr)) return e;
    if (h->mfma_ok) {
        for (int half = 0; half < 2; ++half) {
            std::vector<uint8_t> rec = build_records(h->geom, n, k, q, w_t, sc, bias, half != 0);
            if (int e = upload(half ? &h->d_rec_h : &h->d_rec, rec.data(), rec.size(), &total)) return e;
        }
    }
    h->device_bytes = total;
    *out = h.release();
    return PPOCR_OK;
}

int check_head(const ppocr_rh* h, const char* op) {
    if (!h) return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": null head handle");
    return PPOCR_OK;
}

// PPOCR_MODE_AUTO: the fp16 split, unless the bf16 split's precision guard leaves rows of
// max|a| up to kAutoSplitRows on the split path (then the bf16 split, ~3% faster).  The
// activations the head sees in the recognition model (after the SVTR tail's final
// LayerNorm, whose weights are ~3, plus the shortcut) reach |a| ~ 10-30: with the bf16
// split most of those rows would go to the rescue pass (the synthetic 18710-class head's
// bf16 limit is 11.7), with the fp16 split (limit 747) none.  Measured after the tail on
// the 30720-row batch: head 0.225 ms in F16X2, 0.535 ms in BF16X2.
constexpr float kAutoSplitRows = 32.0f;
int auto_mode(const ppocr_rh* h) {
    if (h->amax_limit >= kAutoSplitRows || !h->f16_ok) return h->quantized ? PPOCR_MODE_BF16X2 : PPOCR_MODE_BF16X3;
    return PPOCR_MODE_F16X2;
}

// Which MFMA configuration a mode maps to for this head (-1: fp32 FMA path).
int mode_cfg(const ppocr_rh* h, int mode, int* cfg) {
    if (mode == PPOCR_MODE_AUTO) mode = auto_mode(h);
    switch (mode) {
        case PPOCR_MODE_FP32_FMA: *cfg = -1; return PPOCR_OK;
        case PPOCR_MODE_BF16X1: *cfg = h->quantized ? CFG_Q1 : CFG_F1; break;
        case PPOCR_MODE_BF16X2:
            if (!h->quantized)
                return fail(PPOCR_ERR_INVALID_ARG,
                            "MatMulTransposedB: an FP32 head supports modes FP32_FMA, BF16X1, BF16X3 and F16X2");
            *cfg = CFG_Q2;
            break;
        case PPOCR_MODE_BF16X3: *cfg = h->quantized ? CFG_Q3 : CFG_F3; break;
        case PPOCR_MODE_F16X2:
            if (!h->f16_ok)
                return fail(PPOCR_ERR_INVALID_ARG,
                            "MatMulTransposedB: weights beyond the fp16 range (|w| >= 32768); use BF16X3 or FP32_FMA");
            *cfg = h->quantized ? CFG_H2 : CFG_HF3;
            break;
        default: return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: unknown mode " + std::to_string(mode));
    }
    if (!h->mfma_ok)
        return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: no MFMA kernel for k = " + std::to_string(h->k) +
                                               " (supported: 73..80, 113..120); use PPOCR_MODE_FP32_FMA");
    return PPOCR_OK;
}

int fma_nsplit(int64_t m, int64_t n) {
    const int64_t mblocks = (m + kFmaRowsPerBlock - 1) / kFmaRowsPerBlock;
    const int64_t ntiles = (n + kFmaCols - 1) / kFmaCols;
    int64_t ns = (1024 + mblocks - 1) / std::max<int64_t>(mblocks, 1);
    ns = std::min<int64_t>(std::max<int64_t>(ns, 1), std::min<int64_t>(ntiles, 1024));
    return (int)ns;
}

int nsplit_for(const ppocr_rh* h, int64_t m, int cfg) {
    if (cfg < 0) return fma_nsplit(m, h->n);
    return stats_nsplit(m, stats_rows_per_block_mfma(cfg, m), h->geom.tiles, stats_per_cu_mfma(cfg, m));
}

constexpr size_t kAlign = 256;
size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

struct WsLayout {
    size_t part, row_max, row_inv, guard_header, guard_rows, skip, total;
};
// The guard header sits at offset 0 whatever m and nsplit are, so a workspace reused for
// batches of other sizes finds there the header its previous call left (emptied by that
// call's merge), never a partial or a list entry of another layout.
WsLayout ws_layout(int64_t m, int nsplit) {
    WsLayout L;
    const size_t pm = align_up((size_t)nsplit * (size_t)m * sizeof(Partial));
    const size_t rm = align_up((size_t)m * 4);
    L.guard_header = 0;
    L.part = kAlign;
    L.row_max = L.part + pm;
    L.row_inv = L.row_max + rm;
    L.guard_rows = L.row_inv + rm;
    L.skip = L.guard_rows + rm;  // a byte per row block of 128 rows or more
    L.total = L.skip + align_up((size_t)((m + 127) / 128));
    return L;
}

// A new epoch for every guarded pass: a mixed counter with the top bit set.  A header whose
// epoch differs from the call's counts as an empty list, so the epoch must not match what a
// workspace may hold before its first use: with the top bit set it never equals a row or
// class index, a count or a non-negative float, and it is never 0 (the cleared header).
unsigned next_epoch() {
    static std::atomic<unsigned> counter{0};
    unsigned x = counter.fetch_add(1, std::memory_order_relaxed) * 0x9E3779B9u + 0x7F4A7C15u;
    x ^= x >> 16;
    x *= 0x85EBCA6Bu;
    x ^= x >> 13;
    return x | 0x80000000u;
}

// The guard of configuration cfg: the precision limit of its term type, and the lower
// statistics limit (the logit range bound as well) when the head has one.
Guard make_guard(const ppocr_rh* h, int cfg, const WsLayout& L, uint8_t* ws, int64_t m) {
    const float prec = cfg_is_f16(cfg) ? h->amax_limit_h : h->amax_limit;
    return Guard{prec,
                 reinterpret_cast<unsigned long long*>(ws + L.guard_header),
                 reinterpret_cast<int*>(ws + L.guard_rows),
                 (int)std::min<int64_t>(m, INT32_MAX),
                 next_epoch(),
                 h->range_ok ? h->range_limit : 0.0f,
                 h->range_ok ? h->range_ss : 0.0f,
                 h->range_ok,
                 h->fma,
                 ws + L.skip};
}

// The tile records configuration cfg reads.
const uint8_t* rec_of(const ppocr_rh* h, int cfg) { return cfg_is_f16(cfg) ? h->d_rec_h : h->d_rec; }

// Projection + softmax statistics + merge (+ the CTC collapse with `ctc`), on device pointers.
// line_len > 0: d_a is channels-first, [m / line_len][k][line_len].
int run_stats(const ppocr_rh* h, int cfg, const float* d_a, int64_t m, int32_t* d_idx, float* d_maxprob,
              float* d_row_max, float* d_row_inv, uint8_t* ws, hipStream_t st, const CtcOut* ctc = nullptr,
              int64_t line_len = 0) {
    const int nsplit = nsplit_for(h, m, cfg);
    const WsLayout L = ws_layout(m, nsplit);
    Partial* part = reinterpret_cast<Partial*>(ws + L.part);
    if (cfg >= 0) {
        const Guard g = make_guard(h, cfg, L, ws, m);
        return launch_stats_mfma(cfg, h->geom, rec_of(h, cfg), h->d_rec, d_a, m, h->n, h->k, nsplit, part, &g, d_idx, d_maxprob, d_row_max, d_row_inv, ctc, st, line_len);
    }
    if (int e = launch_stats_fma(h->d_q, h->d_w, h->d_scale, h->d_bias, d_a, m, h->n, h->k, nsplit, part, st, line_len))
        return e;
    if (ctc) return launch_merge_ctc(part, m, nsplit, *ctc, d_idx, d_maxprob, nullptr, st);
    return launch_merge_stats(part, m, nsplit, d_idx, d_maxprob, d_row_max, d_row_inv, nullptr, st);
}

// Workspace: caller's, or stream-ordered scratch freed on the same stream.
struct Workspace {
    uint8_t* p = nullptr;
    bool owned = false;
    hipStream_t st = nullptr;
    ~Workspace() {
        if (owned && p) (void)hipFreeAsync(p, st);
    }
    int get(void* user, size_t user_bytes, size_t need, hipStream_t s, const char* op) {
        st = s;
        if (user) {
            if (user_bytes < need)
                return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": workspace of " + std::to_string(user_bytes) +
                                                       " bytes, need " + std::to_string(need));
            p = static_cast<uint8_t*>(user);
            return PPOCR_OK;
        }
        void* q = nullptr;
        if (dev_malloc_async(&q, std::max<size_t>(need, kAlign), s) != hipSuccess) {
            (void)hipGetLastError();
            return fail(PPOCR_ERR_NO_MEMORY, std::string(op) + ": workspace allocation failed");
        }
        p = static_cast<uint8_t*>(q);
        owned = true;
        return launch_guard_clear(reinterpret_cast<unsigned long long*>(p), s);  // the header, at offset 0
    }
};

// ---------------------------------------------------------------- allocation-free scratch
// The scratch of ppocr_rh_decode_dev_noalloc: a file-scope device array standing in for
// the workspace, one per GPU the library runs on, held until the process ends.  In host
// code `scratch` names a host-side stand-in, not device memory: its device address is
// taken once per device with hipGetSymbolAddress (with that device current) and only that
// address is ever passed to kernels.  Every call on a GPU shares its array, so calls that
// overlap on one GPU race; what a call needs cleared (the guard list's header) is told
// apart from what a previous call left by the call's epoch.
constexpr size_t kNoAllocScratchBytes = 32u << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch[kMaxDevices] = {};

// Device address of this device's scratch (`device` current); the first call on a device
// takes the address and clears the guard header at its start (a fill kernel on `st`, no
// memset node, so a captured first call replays correctly).
int scratch_of(int device, hipStream_t st, uint8_t** out) {
    if (device < 0 || device >= kMaxDevices)
        return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: device " + std::to_string(device) +
                                               " beyond the allocation-free scratch table");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[device]) {
        void* p = nullptr;
        PPOCR_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) return fail(PPOCR_ERR_DEVICE, "RecHeadHip: no device address for the scratch array");
        if (int e = launch_guard_clear(static_cast<unsigned long long*>(p), st)) return e;
        g_scratch[device] = static_cast<uint8_t*>(p);
    }
    *out = g_scratch[device];
    return PPOCR_OK;
}

int check_m(int64_t m, const char* op) {
    if (m < 0) return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": negative row count");
    if (m > (1LL << 31)) return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": too many rows");
    return PPOCR_OK;
}

}  // namespace

extern "C" {

const char* ppocr_last_error(void) { return g_last_error.c_str(); }

int ppocr_rh_pack_int8_dev(const float* d_w_t, int64_t n, int64_t k, int8_t* d_q_out, float* d_scales_out,
                           void* stream) {
    if (n < 0 || k < 0) return fail(PPOCR_ERR_INVALID_ARG, "QuantizedWeight: negative shape");
    if (n > 0 && (!d_w_t || !d_q_out || !d_scales_out)) return fail(PPOCR_ERR_INVALID_ARG, "QuantizedWeight: null pointer");
    return launch_pack_int8(d_w_t, n, k, d_q_out, d_scales_out, (hipStream_t)stream);
}

int ppocr_rh_pack_int8(const float* w_t, int64_t n, int64_t k, int8_t* q_out, float* scales_out) {
    if (n < 0 || k < 0) return fail(PPOCR_ERR_INVALID_ARG, "QuantizedWeight: negative shape");
    if (n == 0) return PPOCR_OK;
    if (!w_t || !q_out || !scales_out) return fail(PPOCR_ERR_INVALID_ARG, "QuantizedWeight: null pointer");
    DevBuf dw, dq, ds;
    if (int e = dw.alloc((size_t)(n * k) * 4)) return e;
    if (int e = dq.alloc((size_t)(n * k))) return e;
    if (int e = ds.alloc((size_t)n * 4)) return e;
    if (n * k) PPOCR_HIP(hipMemcpy(dw.p, w_t, (size_t)(n * k) * 4, hipMemcpyHostToDevice));
    if (int e = launch_pack_int8(dw.as<float>(), n, k, dq.as<int8_t>(), ds.as<float>(), nullptr)) return e;
    if (n * k) PPOCR_HIP(hipMemcpy(q_out, dq.p, (size_t)(n * k), hipMemcpyDeviceToHost));
    PPOCR_HIP(hipMemcpy(scales_out, ds.p, (size_t)n * 4, hipMemcpyDeviceToHost));
    return PPOCR_OK;
}

int ppocr_rh_create(const int8_t* q, const float* scales, const float* bias, int64_t n, int64_t k, int device,
                    ppocr_rh_t** out) {
    if (!q) {
        if (out) *out = nullptr;
        return fail(PPOCR_ERR_INVALID_ARG, "MatMulQuantizedB: null weight pointer");
    }
    return create_common(q, nullptr, scales, bias, n, k, device, out);
}

int ppocr_rh_create_f32(const float* w_t, const float* bias, int64_t n, int64_t k, int device, ppocr_rh_t** out) {
    if (!w_t) {
        if (out) *out = nullptr;
        return fail(PPOCR_ERR_INVALID_ARG, "MatMulTransposedB: null weight pointer");
    }
    return create_common(nullptr, w_t, nullptr, bias, n, k, device, out);
}

int ppocr_rh_create_from_safetensors(const char* path, const char* weight_name, const char* bias_name, int quantize,
                                     int device, ppocr_rh_t** out) {
    const char* op = quantize ? "MatMulQuantizedB" : "MatMulTransposedB";
    if (out) *out = nullptr;
    if (!weight_name) return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": null weight name");
    StFile f;
    if (int e = f.open(path)) return e;
    const StTensor* w = f.find(weight_name);
    if (!w) return fail(PPOCR_ERR_MODEL, std::string("Model: tensor '") + weight_name + "' not found in the model file");
    if (w->dtype != "F32" || w->shape.size() != 2)
        return fail(PPOCR_ERR_MODEL, std::string("Model: tensor '") + weight_name + "' must be a 2-D F32 matrix [k][n]");
    const int64_t k = w->shape[0], n = w->shape[1];
    const StTensor* b = nullptr;
    if (bias_name) {
        b = f.find(bias_name);
        if (!b) return fail(PPOCR_ERR_MODEL, std::string("Model: tensor '") + bias_name + "' not found in the model file");
        if (b->dtype != "F32" || (int64_t)(b->bytes / 4) != n)
            return fail(PPOCR_ERR_MODEL, std::string("Model: tensor '") + bias_name + "' must be F32 with " +
                                             std::to_string(n) + " values");
    }
    if (int e = check_create(op, n, k, device, out)) return e;
    DeviceGuard dg(device);
    if (dg.err) return fail(PPOCR_ERR_DEVICE, "RecHeadHip: hipSetDevice failed");
    std::unique_ptr<ppocr_rh, void (*)(ppocr_rh*)> h(new_handle(n, k, quantize != 0, device), free_handle);
    if (!h) return fail(PPOCR_ERR_NO_MEMORY, "RecHeadHip: host allocation failed");

    // the weight as stored ([k][n], straight from the mapped file), then W^T [n][k] on the
    // device (the prepack), then the packed INT8 weight and its scales
    const size_t nk = (size_t)(n * k);
    DevBuf raw, wt;
    if (int e = raw.alloc(nk * 4)) return e;
    if (int e = wt.alloc(nk * 4)) return e;
    PPOCR_HIP(hipMemcpy(raw.p, w->data, nk * 4, hipMemcpyHostToDevice));
    if (int e = launch_transpose(raw.as<float>(), k, n, wt.as<float>(), nullptr)) return e;
    size_t total = 0;
    auto dev_alloc = [&](void** p, size_t bytes) -> int {
        bytes = std::max<size_t>(bytes, 1);
        if (dev_malloc(p, bytes) != hipSuccess) {
            *p = nullptr;
            (void)hipGetLastError();
            return fail(PPOCR_ERR_NO_MEMORY, "RecHeadHip: device allocation failed");
        }
        total += bytes;
        return PPOCR_OK;
    };
    if (quantize) {
        if (int e = dev_alloc((void**)&h->d_q, nk)) return e;
    } else {
        h->d_w = wt.as<float>();  // the handle keeps W^T
        wt.p = nullptr;
        total += std::max<size_t>(nk * 4, 1);
    }
    if (int e = dev_alloc((void**)&h->d_scale, (size_t)n * 4)) return e;
    if (int e = dev_alloc((void**)&h->d_bias, (size_t)n * 4)) return e;
    if (quantize) {
        if (int e = launch_pack_int8(wt.as<float>(), n, k, h->d_q, h->d_scale, nullptr)) return e;
    } else {
        std::vector<float> ones((size_t)n, 1.0f);
        PPOCR_HIP(hipMemcpy(h->d_scale, ones.data(), (size_t)n * 4, hipMemcpyHostToDevice));
    }
    if (b) PPOCR_HIP(hipMemcpy(h->d_bias, b->data, (size_t)n * 4, hipMemcpyHostToDevice));
    else PPOCR_HIP(hipMemset(h->d_bias, 0, (size_t)n * 4));
    h->fma = FmaWeights{h->d_q, h->d_w, h->d_scale, h->d_bias};
    if (int e = device_limits(h.get(), b != nullptr)) return e;
    if (h->mfma_ok) {
        const size_t rec_bytes = (size_t)h->geom.tiles * h->geom.rec_bytes();
        for (int half = 0; half < 2; ++half) {
            uint8_t** dst = half ? &h->d_rec_h : &h->d_rec;
            if (int e = dev_alloc((void**)dst, rec_bytes)) return e;
            PPOCR_HIP(hipMemset(*dst, 0, rec_bytes));
            if (int e = launch_build_records(h->geom, n, k, h->d_q, h->d_w, h->d_scale, b ? h->d_bias : nullptr,
                                             half != 0, *dst, nullptr))
                return e;
        }
    }
    PPOCR_HIP(hipDeviceSynchronize());
    h->device_bytes = total;
    *out = h.release();
    return PPOCR_OK;
}

int ppocr_model_find_rec_head(const char* path, char* weight_name, size_t weight_cap, char* bias_name,
                              size_t bias_cap, int64_t* n, int64_t* k) {
    StFile f;
    if (int e = f.open(path)) return e;
    RecHeadNames r;
    if (int e = find_rec_head(f, &r)) return e;
    if (!weight_name || r.weight.size() + 1 > weight_cap || !bias_name || r.bias.size() + 1 > bias_cap)
        return fail(PPOCR_ERR_INVALID_ARG, "Model: a tensor name does not fit its buffer");
    std::memcpy(weight_name, r.weight.c_str(), r.weight.size() + 1);
    std::memcpy(bias_name, r.bias.c_str(), r.bias.size() + 1);
    if (n) *n = r.n;
    if (k) *k = r.k;
    return PPOCR_OK;
}

void ppocr_rh_destroy(ppocr_rh_t* h) { free_handle(h); }

size_t ppocr_rh_footprint_bytes(const ppocr_rh_t* h) {
    if (!h) return 0;
    // src/engine/model.rs:657-666: INT8 data.len() + 4*scales.len(); FP32 numel*4.
    return h->quantized ? (size_t)(h->n * h->k) + 4 * (size_t)h->n : 4 * (size_t)(h->n * h->k);
}

size_t ppocr_rh_device_bytes(const ppocr_rh_t* h) { return h ? h->device_bytes : 0; }

int ppocr_rh_shape(const ppocr_rh_t* h, int64_t* n, int64_t* k, int* quantized) {
    if (int e = check_head(h, "RecHeadHip")) return e;
    if (n) *n = h->n;
    if (k) *k = h->k;
    if (quantized) *quantized = h->quantized ? 1 : 0;
    return PPOCR_OK;
}

int ppocr_rh_auto_mode(const ppocr_rh_t* h) { return h ? auto_mode(h) : -1; }

int ppocr_rh_guard_limits(const ppocr_rh_t* h, int mode, float* prec_limit, float* range_amax_limit,
                          float* range_norm_limit) {
    if (!h || !prec_limit || !range_amax_limit || !range_norm_limit)
        return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: null pointer");
    int cfg;
    if (int e = mode_cfg(h, mode, &cfg)) return e;
    *prec_limit = *range_amax_limit = *range_norm_limit = INFINITY;
    if (cfg == CFG_Q2 || cfg == CFG_H2 || cfg == CFG_F3 || cfg == CFG_HF3) {
        *prec_limit = cfg_is_f16(cfg) ? h->amax_limit_h : h->amax_limit;
        // the two-term INT8 statistics pass skips the reference shift when the head has a
        // logit range bound, and then also rescues the rows not proven to stay in range
        if (h->range_ok && (cfg == CFG_Q2 || cfg == CFG_H2)) {
            *range_amax_limit = h->range_limit;
            *range_norm_limit = std::sqrt(h->range_ss);
        }
    }
    return PPOCR_OK;
}

size_t ppocr_rh_workspace_bytes(const ppocr_rh_t* h, int64_t m, int mode) {
    if (!h || m <= 0) return 0;
    int cfg;
    if (mode_cfg(h, mode, &cfg)) return 0;
    return ws_layout(m, nsplit_for(h, m, cfg)).total;
}

int ppocr_rh_logits_dev(const ppocr_rh_t* h, const float* d_a, int64_t m, int mode, float* d_out, void* d_workspace,
                        size_t workspace_bytes, void* stream) {
    const char* op = (h && !h->quantized) ? "MatMulTransposedB" : "MatMulQuantizedB";
    if (int e = check_head(h, op)) return e;
    if (int e = check_m(m, op)) return e;
    int cfg;
    if (int e = mode_cfg(h, mode, &cfg)) return e;
    if (m == 0) return PPOCR_OK;
    if (!d_a || !d_out) return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": null pointer");
    DeviceGuard dg(h->device);
    hipStream_t st = (hipStream_t)stream;
    if (cfg < 0) return launch_logits_fma(h->d_q, h->d_w, h->d_scale, h->d_bias, d_a, m, h->n, h->k, d_out, st);
    const WsLayout L = ws_layout(m, nsplit_for(h, m, cfg));
    Workspace ws;
    if (int e = ws.get(d_workspace, workspace_bytes, L.total, st, op)) return e;
    const Guard g = make_guard(h, cfg, L, ws.p, m);
    return launch_logits_mfma(cfg, h->geom, rec_of(h, cfg), h->d_rec, d_a, m, h->n, h->k, d_out, &g, st);
}

int ppocr_rh_logits(const ppocr_rh_t* h, const float* a, int64_t m, int mode, float* out) {
    const char* op = (h && !h->quantized) ? "MatMulTransposedB" : "MatMulQuantizedB";
    if (int e = check_head(h, op)) return e;
    if (int e = check_m(m, op)) return e;
    int cfg;
    if (int e = mode_cfg(h, mode, &cfg)) return e;
    if (m == 0) return PPOCR_OK;
    if (!a || !out) return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": null pointer");
    DeviceGuard dg(h->device);
    const size_t ab = (size_t)(m * h->k) * 4, ob = (size_t)(m * h->n) * 4;
    const size_t wsb = cfg >= 0 ? ws_layout(m, nsplit_for(h, m, cfg)).total : 0;
    HostCall hc;
    if (int e = hc.begin({ab}, {ob}, wsb)) return e;
    if (int e = hc.copy_in({a})) return e;
    if (int e = ppocr_rh_logits_dev(h, hc.in<float>(0), m, mode, hc.out<float>(0), hc.ws(), hc.ws_bytes(), hc.stream()))
        return e;
    return hc.copy_out({out});
}

int ppocr_softmax_rows_dev(float* d_x, int64_t rows, int64_t cols, int32_t* d_idx, float* d_maxprob, void* stream) {
    if (rows < 0 || cols < 0) return fail(PPOCR_ERR_INVALID_ARG, "Softmax: negative shape");
    if (rows == 0 || cols == 0) return PPOCR_OK;
    if (!d_x) return fail(PPOCR_ERR_INVALID_ARG, "Softmax: null pointer");
    return launch_softmax_rows(d_x, rows, cols, d_idx, d_maxprob, (hipStream_t)stream);
}

int ppocr_softmax_rows(float* x, int64_t rows, int64_t cols) {
    if (rows < 0 || cols < 0) return fail(PPOCR_ERR_INVALID_ARG, "Softmax: negative shape");
    if (rows == 0 || cols == 0) return PPOCR_OK;  // empty input: nothing to do (src/ops/softmax.rs:226-229)
    if (!x) return fail(PPOCR_ERR_INVALID_ARG, "Softmax: null pointer");
    const size_t xb = (size_t)(rows * cols) * 4;
    HostCall hc;
    if (int e = hc.begin({xb}, {}, 0)) return e;
    if (int e = hc.copy_in({x})) return e;
    if (int e = launch_softmax_rows(hc.in<float>(0), rows, cols, nullptr, nullptr, hc.stream())) return e;
    // in place: the result goes back over the input
    PPOCR_HIP(hipMemcpyAsync(x, hc.in<float>(0), xb, hipMemcpyDeviceToHost, hc.stream()));
    return hc.copy_out({});
}

int ppocr_argmax_rows_dev(const float* d_x, int64_t rows, int64_t cols, int32_t* d_idx, float* d_val, void* stream) {
    if (rows < 0 || cols < 0) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: negative shape");
    if (rows == 0) return PPOCR_OK;
    if ((!d_x && cols) || !d_idx || !d_val) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: null pointer");
    return launch_argmax_rows(d_x, rows, cols, d_idx, d_val, (hipStream_t)stream);
}

int ppocr_argmax_rows(const float* x, int64_t rows, int64_t cols, int32_t* idx, float* val) {
    if (rows < 0 || cols < 0) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: negative shape");
    if (rows == 0) return PPOCR_OK;
    if ((!x && cols) || !idx || !val) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: null pointer");
    const size_t xb = (size_t)(rows * cols) * 4, rb = (size_t)rows * 4;
    HostCall hc;
    if (int e = hc.begin({xb}, {rb, rb}, 0)) return e;
    if (int e = hc.copy_in({x})) return e;
    if (int e = launch_argmax_rows(hc.in<float>(0), rows, cols, hc.out<int32_t>(0), hc.out<float>(1), hc.stream()))
        return e;
    return hc.copy_out({idx, val});
}

int ppocr_rh_argmax_dev(const ppocr_rh_t* h, const float* d_a, int64_t m, int mode, int32_t* d_idx, float* d_maxprob,
                        void* d_workspace, size_t workspace_bytes, void* stream) {
    if (int e = check_head(h, "RecHeadHip")) return e;
    if (int e = check_m(m, "RecHeadHip")) return e;
    int cfg;
    if (int e = mode_cfg(h, mode, &cfg)) return e;
    if (m == 0) return PPOCR_OK;
    if (!d_a || !d_idx || !d_maxprob) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: null pointer");
    DeviceGuard dg(h->device);
    hipStream_t st = (hipStream_t)stream;
    const WsLayout L = ws_layout(m, nsplit_for(h, m, cfg));
    Workspace ws;
    if (int e = ws.get(d_workspace, workspace_bytes, L.total, st, "RecHeadHip")) return e;
    return run_stats(h, cfg, d_a, m, d_idx, d_maxprob, nullptr, nullptr, ws.p, st);
}

int ppocr_rh_argmax(const ppocr_rh_t* h, const float* a, int64_t m, int mode, int32_t* idx, float* maxprob) {
    if (int e = check_head(h, "RecHeadHip")) return e;
    if (int e = check_m(m, "RecHeadHip")) return e;
    int cfg;
    if (int e = mode_cfg(h, mode, &cfg)) return e;
    if (m == 0) return PPOCR_OK;
    if (!a || !idx || !maxprob) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: null pointer");
    DeviceGuard dg(h->device);
    const size_t ab = (size_t)(m * h->k) * 4, rb = (size_t)m * 4;
    HostCall hc;
    if (int e = hc.begin({ab}, {rb, rb}, ws_layout(m, nsplit_for(h, m, cfg)).total)) return e;
    if (int e = hc.copy_in({a})) return e;
    if (int e = ppocr_rh_argmax_dev(h, hc.in<float>(0), m, mode, hc.out<int32_t>(0), hc.out<float>(1), hc.ws(),
                                    hc.ws_bytes(), hc.stream()))
        return e;
    return hc.copy_out({idx, maxprob});
}

int ppocr_rh_probs_dev(const ppocr_rh_t* h, const float* d_a, int64_t m, int mode, float* d_probs, void* d_workspace,
                       size_t workspace_bytes, void* stream) {
    if (int e = check_head(h, "RecHeadHip")) return e;
    if (int e = check_m(m, "RecHeadHip")) return e;
    int cfg;
    if (int e = mode_cfg(h, mode, &cfg)) return e;
    if (m == 0) return PPOCR_OK;
    if (!d_a || !d_probs) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: null pointer");
    DeviceGuard dg(h->device);
    hipStream_t st = (hipStream_t)stream;
    const WsLayout L = ws_layout(m, nsplit_for(h, m, cfg));
    Workspace ws;
    if (int e = ws.get(d_workspace, workspace_bytes, L.total, st, "RecHeadHip")) return e;
    float* rmax = reinterpret_cast<float*>(ws.p + L.row_max);
    float* rinv = reinterpret_cast<float*>(ws.p + L.row_inv);
    if (int e = run_stats(h, cfg, d_a, m, nullptr, nullptr, rmax, rinv, ws.p, st)) return e;
    if (cfg < 0)
        return launch_probs_fma(h->d_q, h->d_w, h->d_scale, h->d_bias, d_a, m, h->n, h->k, rmax, rinv, d_probs, st);
    const Guard g = make_guard(h, cfg, L, ws.p, m);
    return launch_probs_mfma(cfg, h->geom, rec_of(h, cfg), h->d_rec, d_a, m, h->n, h->k, rmax, rinv, d_probs, &g, st);
}

int ppocr_rh_probs(const ppocr_rh_t* h, const float* a, int64_t m, int mode, float* probs) {
    if (int e = check_head(h, "RecHeadHip")) return e;
    if (int e = check_m(m, "RecHeadHip")) return e;
    int cfg;
    if (int e = mode_cfg(h, mode, &cfg)) return e;
    if (m == 0) return PPOCR_OK;
    if (!a || !probs) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: null pointer");
    DeviceGuard dg(h->device);
    const size_t ab = (size_t)(m * h->k) * 4, pb = (size_t)(m * h->n) * 4;
    HostCall hc;
    if (int e = hc.begin({ab}, {pb}, ws_layout(m, nsplit_for(h, m, cfg)).total)) return e;
    if (int e = hc.copy_in({a})) return e;
    if (int e = ppocr_rh_probs_dev(h, hc.in<float>(0), m, mode, hc.out<float>(0), hc.ws(), hc.ws_bytes(), hc.stream()))
        return e;
    return hc.copy_out({probs});
}

int ppocr_ctc_greedy_dev(const int32_t* d_idx, const float* d_maxprob, const int64_t* d_line_off, int64_t lines,
                         int32_t blank, int32_t* d_seq, int64_t* d_seq_len, float* d_score, void* stream) {
    if (lines < 0) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: negative line count");
    if (lines == 0) return PPOCR_OK;
    if (!d_line_off || !d_seq_len || !d_score) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: null pointer");
    return launch_ctc_greedy(d_idx, d_maxprob, d_line_off, lines, blank, d_seq, d_seq_len, d_score,
                             (hipStream_t)stream);
}

static int check_offsets(const int64_t* line_off, int64_t lines) {
    if (line_off[0] != 0) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: line offsets must start at 0");
    for (int64_t i = 0; i < lines; ++i)
        if (line_off[i + 1] < line_off[i])
            return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: line offsets must be non-decreasing");
    return PPOCR_OK;
}

int ppocr_ctc_greedy(const int32_t* idx, const float* maxprob, const int64_t* line_off, int64_t lines, int32_t blank,
                     int32_t* seq, int64_t* seq_len, float* score) {
    if (lines < 0) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: negative line count");
    if (lines == 0) return PPOCR_OK;
    if (!line_off || !seq_len || !score) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: null pointer");
    if (int e = check_offsets(line_off, lines)) return e;
    const int64_t steps = line_off[lines];
    if (steps > 0 && (!idx || !maxprob || !seq)) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: null pointer");
    const size_t sb = (size_t)steps * 4, ob = (size_t)(lines + 1) * 8;
    HostCall hc;
    if (int e = hc.begin({sb, sb, ob}, {sb, (size_t)lines * 8, (size_t)lines * 4}, 0)) return e;
    if (int e = hc.copy_in({idx, maxprob, line_off})) return e;
    if (int e = launch_ctc_greedy(hc.in<int32_t>(0), hc.in<float>(1), hc.in<int64_t>(2), lines, blank,
                                  hc.out<int32_t>(0), hc.out<int64_t>(1), hc.out<float>(2), hc.stream()))
        return e;
    return hc.copy_out({seq, seq_len, score});
}

// ppocr_rh_decode_dev and its allocation-free variant (noalloc: the device's scratch array
// instead of a caller workspace or a stream-ordered allocation).
static int decode_dev_common(const ppocr_rh_t* h, const float* d_a, int64_t m, const int64_t* d_line_off,
                             int64_t lines, int mode, int32_t* d_idx, float* d_maxprob, int32_t* d_seq,
                             int64_t* d_seq_len, float* d_score, void* d_workspace, size_t workspace_bytes,
                             void* stream, bool noalloc) {
    if (int e = check_head(h, "RecHeadHip")) return e;
    if (lines < 0) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: negative line count");
    if (int e = check_m(m, "RecHeadHip")) return e;
    int cfg;
    if (int e = mode_cfg(h, mode, &cfg)) return e;
    if (lines == 0) return PPOCR_OK;
    if (!d_line_off || !d_seq_len || !d_score) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: null pointer");
    if (m > 0 && (!d_a || !d_seq)) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: null pointer");
    const size_t need = m > 0 ? ws_layout(m, nsplit_for(h, m, cfg)).total : 0;
    if (noalloc && need > kNoAllocScratchBytes)
        return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: " + std::to_string(m) + " rows need " + std::to_string(need) +
                                               " bytes of scratch, more than the " +
                                               std::to_string(kNoAllocScratchBytes) +
                                               " of the allocation-free entry point; use ppocr_rh_decode_dev");
    DeviceGuard dg(h->device);
    if (dg.err) return fail(PPOCR_ERR_DEVICE, "RecHeadHip: hipSetDevice failed");
    hipStream_t st = (hipStream_t)stream;
    const CtcOut ctc{d_line_off, lines, 0, d_seq, d_seq_len, d_score};
    if (m == 0) return launch_merge_ctc(nullptr, 0, 1, ctc, nullptr, nullptr, nullptr, st);
    if (noalloc) {
        uint8_t* ws = nullptr;
        if (int e = scratch_of(h->device, st, &ws)) return e;
        return run_stats(h, cfg, d_a, m, d_idx, d_maxprob, nullptr, nullptr, ws, st, &ctc);
    }
    Workspace ws;
    if (int e = ws.get(d_workspace, workspace_bytes, need, st, "RecHeadHip")) return e;
    return run_stats(h, cfg, d_a, m, d_idx, d_maxprob, nullptr, nullptr, ws.p, st, &ctc);
}

int ppocr_rh_decode_dev(const ppocr_rh_t* h, const float* d_a, int64_t m, const int64_t* d_line_off, int64_t lines,
                        int mode, int32_t* d_idx, float* d_maxprob, int32_t* d_seq, int64_t* d_seq_len,
                        float* d_score, void* d_workspace, size_t workspace_bytes, void* stream) {
    return decode_dev_common(h, d_a, m, d_line_off, lines, mode, d_idx, d_maxprob, d_seq, d_seq_len, d_score,
                             d_workspace, workspace_bytes, stream, false);
}

int ppocr_rh_decode_dev_noalloc(const ppocr_rh_t* h, const float* d_a, int64_t m, const int64_t* d_line_off,
                                int64_t lines, int mode, int32_t* d_idx, float* d_maxprob, int32_t* d_seq,
                                int64_t* d_seq_len, float* d_score, void* stream) {
    return decode_dev_common(h, d_a, m, d_line_off, lines, mode, d_idx, d_maxprob, d_seq, d_seq_len, d_score,
                             nullptr, 0, stream, true);
}

int ppocr_rh_decode(const ppocr_rh_t* h, const float* a, const int64_t* line_off, int64_t lines, int mode,
                    int32_t* idx, float* maxprob, int32_t* seq, int64_t* seq_len, float* score) {
    if (int e = check_head(h, "RecHeadHip")) return e;
    if (lines < 0) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: negative line count");
    if (lines == 0) return PPOCR_OK;
    if (!line_off || !seq_len || !score) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: null pointer");
    if (int e = check_offsets(line_off, lines)) return e;
    const int64_t m = line_off[lines];
    if (int e = check_m(m, "RecHeadHip")) return e;
    int cfg;
    if (int e = mode_cfg(h, mode, &cfg)) return e;
    if (m > 0 && (!a || !seq)) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: null pointer");
    DeviceGuard dg(h->device);
    const size_t wsb = m > 0 ? ws_layout(m, nsplit_for(h, m, cfg)).total : 0;
    const size_t ab = (size_t)(m * h->k) * 4, rb = (size_t)m * 4, ob = (size_t)(lines + 1) * 8;
    HostCall hc;
    if (int e = hc.begin({ab, ob}, {rb, (size_t)lines * 8, (size_t)lines * 4, idx ? rb : 0, maxprob ? rb : 0}, wsb))
        return e;
    if (int e = hc.copy_in({a, line_off})) return e;
    if (int e = ppocr_rh_decode_dev(h, hc.in<float>(0), m, hc.in<int64_t>(1), lines, mode,
                                    idx ? hc.out<int32_t>(3) : nullptr, maxprob ? hc.out<float>(4) : nullptr,
                                    hc.out<int32_t>(0), hc.out<int64_t>(1), hc.out<float>(2), hc.ws(), hc.ws_bytes(),
                                    hc.stream()))
        return e;
    return hc.copy_out({seq, seq_len, score, idx, maxprob});
}

int ppocr_rh_decode_nct_dev(const ppocr_rh_t* h, const float* d_x, int64_t lines, int64_t steps, int mode,
                            int32_t* d_idx, float* d_maxprob, int32_t* d_seq, int64_t* d_seq_len, float* d_score,
                            void* d_workspace, size_t workspace_bytes, void* stream) {
    if (int e = check_head(h, "RecHeadHip")) return e;
    if (lines < 0 || steps < 0) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: negative line count or length");
    if (steps > INT32_MAX || (steps > 0 && lines > INT64_MAX / steps))
        return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: line length too large");
    const int64_t m = lines * steps;
    if (int e = check_m(m, "RecHeadHip")) return e;
    int cfg;
    if (int e = mode_cfg(h, mode, &cfg)) return e;
    if (lines == 0) return PPOCR_OK;
    if (!d_seq_len || !d_score) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: null pointer");
    if (m > 0 && (!d_x || !d_seq)) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: null pointer");
    DeviceGuard dg(h->device);
    hipStream_t st = (hipStream_t)stream;
    const CtcOut ctc{nullptr, lines, 0, d_seq, d_seq_len, d_score, steps};
    if (m == 0) return launch_merge_ctc(nullptr, 0, 1, ctc, nullptr, nullptr, nullptr, st);
    const WsLayout L = ws_layout(m, nsplit_for(h, m, cfg));
    Workspace ws;
    if (int e = ws.get(d_workspace, workspace_bytes, L.total, st, "RecHeadHip")) return e;
    return run_stats(h, cfg, d_x, m, d_idx, d_maxprob, nullptr, nullptr, ws.p, st, &ctc, steps);
}

int ppocr_rh_decode_nct(const ppocr_rh_t* h, const float* x, int64_t lines, int64_t steps, int mode, int32_t* idx,
                        float* maxprob, int32_t* seq, int64_t* seq_len, float* score) {
    if (int e = check_head(h, "RecHeadHip")) return e;
    if (lines < 0 || steps < 0) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: negative line count or length");
    if (steps > INT32_MAX || (steps > 0 && lines > INT64_MAX / steps))
        return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: line length too large");
    const int64_t m = lines * steps;
    if (int e = check_m(m, "RecHeadHip")) return e;
    int cfg;
    if (int e = mode_cfg(h, mode, &cfg)) return e;
    if (lines == 0) return PPOCR_OK;
    if (!seq_len || !score) return fail(PPOCR_ERR_INVALID_ARG, "CtcDecode: null pointer");
    if (m > 0 && (!x || !seq)) return fail(PPOCR_ERR_INVALID_ARG, "RecHeadHip: null pointer");
    DeviceGuard dg(h->device);
    const size_t wsb = m > 0 ? ws_layout(m, nsplit_for(h, m, cfg)).total : 0;
    const size_t xb = (size_t)(m * h->k) * 4, rb = (size_t)m * 4;
    HostCall hc;
    if (int e = hc.begin({xb}, {rb, (size_t)lines * 8, (size_t)lines * 4, idx ? rb : 0, maxprob ? rb : 0}, wsb))
        return e;
    if (int e = hc.copy_in({x})) return e;
    if (int e = ppocr_rh_decode_nct_dev(h, hc.in<float>(0), lines, steps, mode, idx ? hc.out<int32_t>(3) : nullptr,
                                        maxprob ? hc.out<float>(4) : nullptr, hc.out<int32_t>(0), hc.out<int64_t>(1),
                                        hc.out<float>(2), hc.ws(), hc.ws_bytes(), hc.stream()))
        return e;
    return hc.copy_out({seq, seq_len, score, idx, maxprob});
}


// ---------------------------------------------------------------- the SVTR neck tail
struct ppocr_rn {
    int device = 0;
    ppocr::NeckDev dev;
    float* d_weights = nullptr;  // every weight of the neck in one allocation
    size_t device_bytes = 0;
};

// the neck's host helpers have C++ linkage (some return C++ types)
extern "C++" {
namespace {

void free_neck(ppocr_rn* h) {
    if (!h) return;
    if (h->d_weights) {
        DeviceGuard dg(h->device);
        (void)hipFree(h->d_weights);
    }
    delete h;
}

// Host pointers of the neck's weights, in upload order, with their float counts.
struct NeckHost {
    int64_t dim = 0, heads = 0, hidden = 0;
    float scale = 0.0f, lnf_eps = 0.0f;
    std::vector<ppocr_rn_block_t> blocks;
    const float *lnf_w = nullptr, *lnf_b = nullptr;
};

// fp16 planes of W^T for the tail's fp16-halves GEMMs: [2][N][kp], the nearest half of each
// weight, then the nearest half of what it leaves, k padded with zeros.
std::vector<uint16_t> neck_half_planes(const float* w, int64_t K, int64_t N) {
    const int64_t kp = neck_f16_kp((int)K);
    std::vector<uint16_t> out((size_t)(2 * N * kp), 0);
    for (int64_t k = 0; k < K; ++k)
        for (int64_t c = 0; c < N; ++c) {
            const float x = w[k * N + c];
            const _Float16 hi = (_Float16)x;
            const _Float16 lo = (_Float16)(x - (float)hi);
            out[(size_t)(c * kp + k)] = __builtin_bit_cast(uint16_t, hi);
            out[(size_t)((N + c) * kp + k)] = __builtin_bit_cast(uint16_t, lo);
        }
    return out;
}

// Column of the padded qkv row (or attention row) that holds column c of the model's:
// part c / D (q, k, v), head (c % D) / 15, value c % 15 -> 128 part + 16 head + value.
int64_t neck_pad_col(int64_t c) {
    const int64_t part = c / kNeckDim, r = c % kNeckDim;
    return 128 * part + 16 * (r / kNeckHeadDim) + r % kNeckHeadDim;
}

// fc1's and fc2's weights in the fused MLP kernel's staging order (NeckBlockDev::mlp_h),
// each weight times 2^e1 (fc1) or 2^e2 (fc2), exact, before the split, so that the low
// halves stay above fp16's subnormals.  fc2's contraction index runs in the order
// K' = 32 T + 16 q + 8 h + e <-> hidden unit 32 T + 16 q + 8 (e / 4) + 4 h + e % 4, the
// order in which fc1's transposed MFMA output leaves the hidden values in registers.
std::vector<uint16_t> neck_mlp_tiles(const ppocr_rn_block_t& b, int64_t D, int64_t H, int e1, int e2) {
    constexpr int kTiles = 8, kTileHalves = 16384;  // 32 KB per tile
    std::vector<uint16_t> out((size_t)kTiles * kTileHalves, 0);
    auto split = [](float v, uint16_t* hi, uint16_t* lo) {
        const _Float16 h = (_Float16)v;
        *hi = __builtin_bit_cast(uint16_t, h);
        *lo = __builtin_bit_cast(uint16_t, (_Float16)(v - (float)h));
    };
    for (int T = 0; T < kTiles; ++T) {
        uint16_t* t = out.data() + (size_t)T * kTileHalves;
        // fc1: [plane][chunk c (16)][unit u (32)][8]: unit 32 T + u, k = 8 c + e
        for (int c = 0; c < 16; ++c)
            for (int u = 0; u < 32; ++u)
                for (int e = 0; e < 8; ++e) {
                    const int64_t unit = 32 * T + u, k = 8 * c + e;
                    if (unit >= H || k >= D) continue;
                    split(std::ldexp(b.fc1_w[k * H + unit], e1), &t[((size_t)c * 32 + u) * 8 + e],
                          &t[((size_t)(16 + c) * 32 + u) * 8 + e]);
                }
        // fc2: [plane][chunk c (4)][column (128)][8]: contraction position K' = 32 T + 8 c + e
        uint16_t* t2 = t + 8192;
        for (int c = 0; c < 4; ++c)
            for (int col = 0; col < 128; ++col)
                for (int e = 0; e < 8; ++e) {
                    const int kp = 32 * T + 8 * c + e;
                    const int ee = kp & 7, hh = (kp >> 3) & 1, q = (kp >> 4) & 1;
                    const int64_t unit = 32 * T + 16 * q + 8 * (ee >> 2) + 4 * hh + (ee & 3);
                    if (unit >= H || col >= D) continue;
                    split(std::ldexp(b.fc2_w[unit * D + col], e2), &t2[((size_t)c * 128 + col) * 8 + e],
                          &t2[((size_t)(4 + c) * 128 + col) * 8 + e]);
                }
    }
    return out;
}

// Whether the weights keep every operand of the tail's GEMMs and attention inside fp16's range,
// with room: each operand is a LayerNorm output (|z_k| <= sqrt(D - 1) for the normalised row, so
// |y_k| <= sqrt(D - 1) |w_k| + |b_k|), the attention's output (a convex combination of the
// value rows, so no larger than them), q, k or v (products of LN1's output), or the swish of
// fc1's output (|x sigmoid(x)| <= |x|); the attention's probabilities lie in [0, 1];
// a product's bound is max_c sum_k |W[k][c]| times its input's bound plus max |bias|.
// The largest e <= 15 with bound * 2^e <= 32768 (half of fp16's largest finite value).
int neck_f16_exponent(double bound) {
    int e = 0;
    while (e < 15 && bound * std::ldexp(1.0, e + 1) <= 32768.0) ++e;
    return e;
}

bool neck_f16_bounds_ok(const NeckHost& nh, int (*exps)[7]) {
    const int64_t D = nh.dim, H = nh.hidden;
    constexpr double kLimit = 16384.0;  // a quarter of fp16's largest finite value
    auto amax = [](const float* v, int64_t n) {
        double r = 0.0;
        for (int64_t i = 0; i < n; ++i) r = std::max(r, (double)std::fabs(v[i]));
        return r;
    };
    // max over columns c0 .. c0 + nc - 1 of sum_k |W[k][c]| (W [K][N])
    auto col_l1 = [](const float* w, int64_t K, int64_t N, int64_t c0, int64_t nc) {
        double r = 0.0;
        for (int64_t c = c0; c < c0 + nc; ++c) {
            double s = 0.0;
            for (int64_t k = 0; k < K; ++k) s += std::fabs(w[k * N + c]);
            r = std::max(r, s);
        }
        return r;
    };
    const double zmax = std::sqrt((double)(D - 1)) * 1.001;
    for (const ppocr_rn_block_t& b : nh.blocks) {
        const double y1 = zmax * amax(b.ln1_w, D) + amax(b.ln1_b, D);  // qkv's input
        const double y2 = zmax * amax(b.ln2_w, D) + amax(b.ln2_b, D);  // fc1's input
        const double qk = y1 * col_l1(b.qkv_w, D, 3 * D, 0, 2 * D) + amax(b.qkv_b, 2 * D);     // the attention's q, k
        const double v = y1 * col_l1(b.qkv_w, D, 3 * D, 2 * D, D) + amax(b.qkv_b + 2 * D, D);  // its v, proj's input
        const double hs = y2 * col_l1(b.fc1_w, D, H, 0, H) + amax(b.fc1_b, H);               // fc2's input
        const double wmax = std::max(std::max(amax(b.qkv_w, D * 3 * D), amax(b.proj_w, D * D)),
                                     std::max(amax(b.fc1_w, D * H), amax(b.fc2_w, H * D)));
        // q is split into fp16 halves after its scaling, so q * |scale| is held to the limit too
        const double qs = qk * (double)std::fabs(nh.scale);
        if (!(y1 <= kLimit && y2 <= kLimit && qk <= kLimit && qs <= kLimit && v <= kLimit && hs <= kLimit &&
              wmax <= kLimit))
            return false;
        const size_t i = (size_t)(&b - nh.blocks.data());
        exps[i][0] = neck_f16_exponent(qs);                                // q * scale
        exps[i][1] = neck_f16_exponent(qk);                                // k
        exps[i][2] = neck_f16_exponent(v);                                 // v
        exps[i][3] = neck_f16_exponent(amax(b.fc1_w, D * H));              // fc1's weights
        exps[i][4] = neck_f16_exponent(amax(b.fc2_w, H * D));              // fc2's weights
        exps[i][5] = neck_f16_exponent(y2);                                // LN2's output
        exps[i][6] = neck_f16_exponent(hs);                                // the hidden layer
    }
    return true;
}

int neck_create(const NeckHost& nh, int device, ppocr_rn_t** out) {
    const char* op = "RecNeckHip";
    if (!out) return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": null output handle");
    *out = nullptr;
    if (nh.dim != kNeckDim || nh.hidden != kNeckHidden || nh.heads <= 0 || nh.heads * kNeckHeadDim != nh.dim)
        return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": unsupported geometry dim " + std::to_string(nh.dim) +
                                               ", heads " + std::to_string(nh.heads) + ", hidden " +
                                               std::to_string(nh.hidden) + " (built for 120, 8 x 15, 240)");
    if (nh.blocks.empty() || nh.blocks.size() > (size_t)kNeckMaxBlocks)
        return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": 1 to " + std::to_string(kNeckMaxBlocks) + " blocks");
    if (!nh.lnf_w || !nh.lnf_b || !std::isfinite(nh.scale) || !(nh.lnf_eps >= 0.0f))
        return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": null final LayerNorm or bad constants");
    const int64_t D = nh.dim, H = nh.hidden;
    // per block: ln1 w,b (D each), qkv (D*3D + 3D), proj (D*D + D), ln2 (2D), fc1 (D*H + H), fc2 (H*D + D)
    std::vector<std::pair<const float*, int64_t>> parts;
    for (const ppocr_rn_block_t& b : nh.blocks) {
        const float* ptrs[12] = {b.ln1_w, b.ln1_b, b.qkv_w, b.qkv_b, b.proj_w, b.proj_b,
                                 b.ln2_w, b.ln2_b, b.fc1_w, b.fc1_b, b.fc2_w, b.fc2_b};
        const int64_t counts[12] = {D, D, D * 3 * D, 3 * D, D * D, D, D, D, D * H, H, H * D, D};
        for (int i = 0; i < 12; ++i) {
            if (!ptrs[i]) return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": null weight pointer");
            parts.push_back({ptrs[i], counts[i]});
        }
        if (!(b.ln1_eps >= 0.0f) || !(b.ln2_eps >= 0.0f))
            return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": bad LayerNorm epsilon");
    }
    parts.push_back({nh.lnf_w, D});
    parts.push_back({nh.lnf_b, D});
    // the fp16 planes of each block's four weights, as float-sized parts after the rest
    int exps[kNeckMaxBlocks][7] = {};
    const bool f16 = neck_f16_bounds_ok(nh, exps);
    std::vector<std::vector<uint16_t>> planes;
    std::vector<std::vector<float>> padded_bias;
    if (f16) {
        for (const ppocr_rn_block_t& b : nh.blocks) {
            const size_t bi = (size_t)(&b - nh.blocks.data());
            // qkv's columns and proj's rows padded per head to 16 (zeros at d = 15)
            std::vector<float> qp((size_t)D * kNeckQkvPad, 0.0f), pp((size_t)kNeckAttPad * D, 0.0f);
            for (int64_t k = 0; k < D; ++k)
                for (int64_t c = 0; c < 3 * D; ++c)
                    qp[(size_t)(k * kNeckQkvPad + neck_pad_col(c))] = b.qkv_w[k * 3 * D + c];
            for (int64_t k = 0; k < D; ++k) std::memcpy(&pp[(size_t)(neck_pad_col(k) * D)], b.proj_w + k * D, (size_t)D * 4);
            planes.push_back(neck_half_planes(qp.data(), D, kNeckQkvPad));
            planes.push_back(neck_half_planes(pp.data(), kNeckAttPad, D));
            planes.push_back(neck_mlp_tiles(b, D, H, exps[bi][3], exps[bi][4]));
        }
        for (const auto& pl : planes)
            parts.push_back({reinterpret_cast<const float*>(pl.data()), (int64_t)(pl.size() / 2)});
        for (const ppocr_rn_block_t& b : nh.blocks) {
            std::vector<float> bp(kNeckQkvPad, 0.0f);
            for (int64_t c = 0; c < 3 * D; ++c) bp[(size_t)neck_pad_col(c)] = b.qkv_b[c];
            padded_bias.push_back(std::move(bp));
        }
        for (const auto& bp : padded_bias) parts.push_back({bp.data(), (int64_t)bp.size()});
    }
    int64_t total = 0;
    for (const auto& pt : parts) total += (pt.second + 3) / 4 * 4;  // each part 16-byte aligned
    if (device < 0) return fail(PPOCR_ERR_INVALID_ARG, std::string(op) + ": negative device");
    DeviceGuard dg(device);
    if (dg.err) return fail(PPOCR_ERR_DEVICE, std::string(op) + ": hipSetDevice failed");
    std::unique_ptr<ppocr_rn, void (*)(ppocr_rn*)> h(new (std::nothrow) ppocr_rn, free_neck);
    if (!h) return fail(PPOCR_ERR_NO_MEMORY, std::string(op) + ": host allocation failed");
    h->device = device;
    void* p = nullptr;
    if (dev_malloc(&p, (size_t)total * 4) != hipSuccess) {
        (void)hipGetLastError();
        return fail(PPOCR_ERR_NO_MEMORY, std::string(op) + ": device allocation failed");
    }
    h->d_weights = static_cast<float*>(p);
    h->device_bytes = (size_t)total * 4;
    std::vector<float> host((size_t)total, 0.0f);
    std::vector<const float*> dev_ptr;
    int64_t off = 0;
    for (const auto& pt : parts) {
        std::memcpy(host.data() + off, pt.first, (size_t)pt.second * 4);
        dev_ptr.push_back(h->d_weights + off);
        off += (pt.second + 3) / 4 * 4;
    }
    PPOCR_HIP(hipMemcpy(h->d_weights, host.data(), (size_t)total * 4, hipMemcpyHostToDevice));
    NeckDev& nd = h->dev;
    nd.dim = (int)D;
    nd.heads = (int)nh.heads;
    nd.hidden = (int)H;
    nd.scale = nh.scale;
    nd.blocks = (int)nh.blocks.size();
    size_t q = 0;
    for (size_t i = 0; i < nh.blocks.size(); ++i) {
        NeckBlockDev& b = nd.block[i];
        b.ln1_w = dev_ptr[q++];
        b.ln1_b = dev_ptr[q++];
        b.qkv_w = dev_ptr[q++];
        b.qkv_b = dev_ptr[q++];
        b.proj_w = dev_ptr[q++];
        b.proj_b = dev_ptr[q++];
        b.ln2_w = dev_ptr[q++];
        b.ln2_b = dev_ptr[q++];
        b.fc1_w = dev_ptr[q++];
        b.fc1_b = dev_ptr[q++];
        b.fc2_w = dev_ptr[q++];
        b.fc2_b = dev_ptr[q++];
        b.ln1_eps = nh.blocks[i].ln1_eps;
        b.ln2_eps = nh.blocks[i].ln2_eps;
    }
    nd.lnf_w = dev_ptr[q++];
    nd.lnf_b = dev_ptr[q++];
    nd.lnf_eps = nh.lnf_eps;
    nd.f16 = f16;
    for (size_t i = 0; f16 && i < nh.blocks.size(); ++i) {
        NeckBlockDev& b = nd.block[i];
        b.qkv_h = reinterpret_cast<const uint16_t*>(dev_ptr[q++]);
        b.proj_h = reinterpret_cast<const uint16_t*>(dev_ptr[q++]);
        b.mlp_h = reinterpret_cast<const uint16_t*>(dev_ptr[q++]);
        b.attn_eq = exps[i][0];
        b.attn_ek = exps[i][1];
        b.attn_ev = exps[i][2];
        b.mlp_e1 = exps[i][3];
        b.mlp_e2 = exps[i][4];
        b.mlp_ey = exps[i][5];
        b.mlp_eh = exps[i][6];
    }
    for (size_t i = 0; f16 && i < nh.blocks.size(); ++i) nd.block[i].qkv_bp = dev_ptr[q++];
    *out = h.release();
    return PPOCR_OK;
}

int check_neck(const ppocr_rn_t* h) {
    if (!h) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: null neck handle");
    return PPOCR_OK;
}

}  // namespace
}  // extern "C++"

int ppocr_rn_create(const ppocr_rn_block_t* blocks, int nblocks, const float* lnf_w, const float* lnf_b,
                    float lnf_eps, int64_t dim, int64_t heads, int64_t hidden, float scale, int device,
                    ppocr_rn_t** out) {
    if (out) *out = nullptr;
    if (!blocks || nblocks <= 0) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: no blocks");
    NeckHost nh;
    nh.dim = dim;
    nh.heads = heads;
    nh.hidden = hidden;
    nh.scale = scale;
    nh.lnf_w = lnf_w;
    nh.lnf_b = lnf_b;
    nh.lnf_eps = lnf_eps;
    nh.blocks.assign(blocks, blocks + nblocks);
    return neck_create(nh, device, out);
}

int ppocr_rn_create_from_model(const char* path, int device, ppocr_rn_t** out) {
    if (out) *out = nullptr;
    StFile f;
    if (int e = f.open(path)) return e;
    RecNeckNames nn;
    if (int e = find_rec_neck(f, &nn)) return e;
    auto vec = [&](const std::string& name, int64_t count, const float** dst) -> int {
        const StTensor* t = f.find(name.c_str());
        if (!t || t->dtype != "F32" || (int64_t)(t->bytes / 4) != count)
            return fail(PPOCR_ERR_MODEL, "Model: tensor '" + name + "' must be F32 with " + std::to_string(count) +
                                             " values");
        *dst = reinterpret_cast<const float*>(t->data);  // the map is 4-byte aligned for F32 data
        return PPOCR_OK;
    };
    NeckHost nh;
    nh.dim = nn.dim;
    nh.heads = nn.heads;
    nh.hidden = nn.hidden;
    nh.scale = nn.scale;
    nh.lnf_eps = nn.lnf_eps;
    const int64_t D = nn.dim, H = nn.hidden;
    // tensor data in the file need not be 4-byte aligned: copy each into owned storage
    std::vector<std::vector<float>> keep;
    auto owned = [&](const std::string& name, int64_t count, const float** dst) -> int {
        const float* src;
        if (int e = vec(name, count, &src)) return e;
        keep.emplace_back((size_t)count);
        std::memcpy(keep.back().data(), src, (size_t)count * 4);
        *dst = keep.back().data();
        return PPOCR_OK;
    };
    keep.reserve(nn.blocks.size() * 12 + 2);
    for (const RecNeckBlockNames& b : nn.blocks) {
        ppocr_rn_block_t hb{};
        if (int e = owned(b.ln1_w, D, &hb.ln1_w)) return e;
        if (int e = owned(b.ln1_b, D, &hb.ln1_b)) return e;
        if (int e = owned(b.qkv_w, D * 3 * D, &hb.qkv_w)) return e;
        if (int e = owned(b.qkv_b, 3 * D, &hb.qkv_b)) return e;
        if (int e = owned(b.proj_w, D * D, &hb.proj_w)) return e;
        if (int e = owned(b.proj_b, D, &hb.proj_b)) return e;
        if (int e = owned(b.ln2_w, D, &hb.ln2_w)) return e;
        if (int e = owned(b.ln2_b, D, &hb.ln2_b)) return e;
        if (int e = owned(b.fc1_w, D * H, &hb.fc1_w)) return e;
        if (int e = owned(b.fc1_b, H, &hb.fc1_b)) return e;
        if (int e = owned(b.fc2_w, H * D, &hb.fc2_w)) return e;
        if (int e = owned(b.fc2_b, D, &hb.fc2_b)) return e;
        hb.ln1_eps = b.ln1_eps;
        hb.ln2_eps = b.ln2_eps;
        nh.blocks.push_back(hb);
    }
    if (int e = owned(nn.lnf_w, D, &nh.lnf_w)) return e;
    if (int e = owned(nn.lnf_b, D, &nh.lnf_b)) return e;
    return neck_create(nh, device, out);
}

void ppocr_rn_destroy(ppocr_rn_t* h) { free_neck(h); }

int ppocr_rn_shape(const ppocr_rn_t* h, int64_t* dim, int64_t* heads, int64_t* hidden, int* blocks) {
    if (int e = check_neck(h)) return e;
    if (dim) *dim = h->dev.dim;
    if (heads) *heads = h->dev.heads;
    if (hidden) *hidden = h->dev.hidden;
    if (blocks) *blocks = h->dev.blocks;
    return PPOCR_OK;
}

int ppocr_rn_gemm_halves(const ppocr_rn_t* h) {
    if (int e = check_neck(h)) return e;
    return h->dev.f16 ? 1 : 0;
}

size_t ppocr_rn_workspace_bytes(const ppocr_rn_t* h, int64_t m) {
    if (!h || m <= 0 || m > INT64_MAX / (kNeckWsFloatsPerRow * 4)) return 0;
    return (size_t)(m * kNeckWsFloatsPerRow * 4);
}

int ppocr_rn_forward_dev(const ppocr_rn_t* h, const float* d_x, const float* d_shortcut, int64_t m,
                         const int64_t* d_line_off, int64_t lines, int layout, float* d_out, void* d_workspace,
                         size_t workspace_bytes, void* stream) {
    if (int e = check_neck(h)) return e;
    if (m < 0 || lines < 0) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: negative row or line count");
    if (layout != PPOCR_NECK_ROWS && layout != PPOCR_NECK_CHANNELS_FIRST)
        return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: unknown layout " + std::to_string(layout));
    if (m == 0) return PPOCR_OK;
    if (m > INT32_MAX) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: too many rows");
    if (!d_x || !d_shortcut || !d_out || !d_line_off || lines == 0)
        return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: null pointer or no lines");
    const size_t need = ppocr_rn_workspace_bytes(h, m);
    if (reinterpret_cast<uintptr_t>(d_workspace) & 15)
        return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: the workspace must be 16-byte aligned");
    DeviceGuard dg(h->device);
    if (dg.err) return fail(PPOCR_ERR_DEVICE, "RecNeckHip: hipSetDevice failed");
    hipStream_t st = static_cast<hipStream_t>(stream);
    Workspace ws;
    if (int e = ws.get(d_workspace, workspace_bytes, need, st, "RecNeckHip")) return e;
    return launch_neck(h->dev, d_x, d_shortcut, m, d_line_off, lines, 0, layout, d_out,
                       reinterpret_cast<float*>(ws.p), st);
}

int ppocr_rn_forward_marked_dev(const ppocr_rn_t* h, const float* d_x, const float* d_shortcut, int64_t m,
                                const int64_t* d_line_off, int64_t lines, int layout, float* d_out,
                                void* d_workspace, size_t workspace_bytes, void* stream, void* const* events,
                                int nevents, const char** names, int* recorded) {
    if (int e = check_neck(h)) return e;
    if (!events || !names || !recorded || nevents < 1)
        return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: null event list");
    *recorded = 0;
    if (m < 0 || lines < 0) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: negative row or line count");
    if (layout != PPOCR_NECK_ROWS && layout != PPOCR_NECK_CHANNELS_FIRST)
        return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: unknown layout " + std::to_string(layout));
    if (m == 0) return PPOCR_OK;
    if (m > INT32_MAX) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: too many rows");
    if (!d_x || !d_shortcut || !d_out || !d_line_off || lines == 0)
        return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: null pointer or no lines");
    const size_t need = ppocr_rn_workspace_bytes(h, m);
    if (reinterpret_cast<uintptr_t>(d_workspace) & 15)
        return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: the workspace must be 16-byte aligned");
    DeviceGuard dg(h->device);
    if (dg.err) return fail(PPOCR_ERR_DEVICE, "RecNeckHip: hipSetDevice failed");
    hipStream_t st = static_cast<hipStream_t>(stream);
    Workspace ws;
    if (int e = ws.get(d_workspace, workspace_bytes, need, st, "RecNeckHip")) return e;
    NeckMarks marks{reinterpret_cast<hipEvent_t*>(const_cast<void**>(events)), names, nevents, 0};
    const int e = launch_neck(h->dev, d_x, d_shortcut, m, d_line_off, lines, 0, layout, d_out,
                              reinterpret_cast<float*>(ws.p), st, &marks);
    *recorded = marks.count;
    return e;
}

int ppocr_rn_forward(const ppocr_rn_t* h, const float* x, const float* shortcut, const int64_t* line_off,
                     int64_t lines, int layout, float* out) {
    if (int e = check_neck(h)) return e;
    if (lines < 0) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: negative line count");
    if (layout != PPOCR_NECK_ROWS && layout != PPOCR_NECK_CHANNELS_FIRST)
        return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: unknown layout " + std::to_string(layout));
    if (lines == 0) return PPOCR_OK;
    if (!line_off) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: null line offsets");
    if (int e = check_offsets(line_off, lines)) return e;
    const int64_t m = line_off[lines];
    if (m == 0) return PPOCR_OK;
    if (!x || !shortcut || !out) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: null pointer");
    if (m > INT32_MAX) return fail(PPOCR_ERR_INVALID_ARG, "RecNeckHip: too many rows");
    DeviceGuard dg(h->device);
    if (dg.err) return fail(PPOCR_ERR_DEVICE, "RecNeckHip: hipSetDevice failed");
    const size_t xb = (size_t)m * h->dev.dim * 4;
    HostCall hc;
    if (int e = hc.begin({xb, xb, (size_t)(lines + 1) * 8}, {xb}, ppocr_rn_workspace_bytes(h, m))) return e;
    if (int e = hc.copy_in({x, shortcut, line_off})) return e;
    if (int e = launch_neck(h->dev, hc.in<float>(0), hc.in<float>(1), m, hc.in<int64_t>(2), lines, 0, layout,
                           hc.out<float>(0), reinterpret_cast<float*>(hc.ws()), hc.stream()))
        return e;
    return hc.copy_out({out});
}

}  // extern "C"
