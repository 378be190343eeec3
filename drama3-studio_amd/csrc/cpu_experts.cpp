// CPU expert executor of the cooperative decode mode: the host cores take
// some route slots of a one-token FP8 layer call while the GPU runs the rest.
//
// Reference: the C++ Executor of native/src/runtime.cpp:68-276 with its
// route planner drama_partition_routes (runtime.cpp:291-335) and the FP8
// boundary guard (fp8_reference.cpp:52-93), driven by HybridDecodeRuntime
// (src/drama_low_vram/hybrid_decode.py:33-416).
//
// The arithmetic is the GPU decode's own, step for step, except inside a
// 128-column block product:
//   - a block product sums its 128 FP8 x FP8 products (each exact in fp32)
//     in fp32, in a fixed order on every ISA (16 lane sums, then a halving
//     fold).  The gfx950 FP8 MFMA instead truncates each product to 13
//     fractional bits below the largest exponent sum of its group of 8
//     (toward zero) and rounds its groups into the fp32 accumulator two at a
//     time, so host and device slots agree within the path's tolerance, not
//     bit for bit;
//   - gate / up: per K block dot * activation scale, then fma with the weight
//     scale, chained over the blocks kb = w, w + 8, ... of each of the 8
//     waves that split K on the GPU, and the 8 chains summed in wave order;
//     rounded through bf16; SiLU from a table the GPU filled with its own
//     expression for every bf16 gate value; h = silu * up;
//   - the FP8 128-group quantization of h (scale = max(amax, 1e-10) *
//     fl(1/448), true division, E4M3 round-to-nearest-even with saturation);
//   - down: one fma chain over the K blocks in order, then * route weight.
// The guard (on by default in the Python runtime) reports a call whose
// hidden quantization lands within 4 fp32 ulps of an E4M3 rounding midpoint,
// so the caller recomputes those slots on the GPU, as the reference's guard
// does.
//
// Threads: one persistent pool; a call splits the gate/up rows and the down
// rows of all its slots into chunks that every thread (the caller included)
// takes from a shared counter -- not one slot per thread as the reference's
// executor, so all host cores work even on one slot.
#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <exception>
#include <functional>
#include <limits>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "drama_moe.h"

namespace dmoe {
void set_last_error(const char* message);  // abi.cpp
}

namespace {

constexpr int kWaveSplit = 8;  // K blocks of gate/up are split over 8 waves on the GPU
constexpr float kInv448 = 1.0f / 448.0f;

// ---------------------------------------------------------------- E4M3 codec

float e4m3_value(uint8_t b) {
    const int mag = b & 127, e = mag >> 3, m = mag & 7;
    float v = e == 0 ? std::ldexp((float)m, -9) : std::ldexp(1.0f + m * 0.125f, e - 7);
    if (mag == 127) v = std::numeric_limits<float>::quiet_NaN();
    return (b & 128) ? -v : v;
}

struct DecodeTable {
    float v[256];
    DecodeTable() {
        for (int i = 0; i < 256; ++i) v[i] = e4m3_value((uint8_t)i);
    }
};
const DecodeTable& table() {
    static const DecodeTable t;
    return t;
}

// Round-to-nearest-even E4M3 of a finite float, saturating at 448.
uint8_t e4m3_encode(float v) {
    const uint8_t sign = std::signbit(v) ? 128 : 0;
    const float a = std::min(std::fabs(v), 448.0f);
    uint32_t mag;
    if (a < 0.015625f) {
        mag = (uint32_t)std::nearbyint(a * 512.0f);  // subnormal steps of 2^-9 (default rounding: to even)
    } else {
        uint32_t u;
        std::memcpy(&u, &a, 4);
        u += 0x7FFFFu + ((u >> 20) & 1u);
        mag = (u >> 20) - (120u << 3);
    }
    return sign | (uint8_t)mag;
}

// Whether |q| lies within 4 fp32 ulps of an E4M3 rounding midpoint (normal
// range: the 20 dropped mantissa bits near 0x80000; subnormal range: the
// fraction of |q| * 512 near one half).
bool near_e4m3_midpoint(float q) {
    const float a = std::fabs(q);
    if (a >= 0.015625f && a < 448.0f) {
        uint32_t u;
        std::memcpy(&u, &a, 4);
        return std::abs((int)(u & 0xFFFFFu) - 0x80000) <= 4;
    }
    if (a > 0.0f && a < 0.015625f) {
        const float s = a * 512.0f;
        return std::fabs(s - std::floor(s) - 0.5f) <= std::max(1e-12f, s * (4.0f / 8388608.0f));
    }
    return false;
}

float bf16_round(float v) {
    uint32_t u;
    std::memcpy(&u, &v, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return v;
    u += 0x7FFFu + ((u >> 16) & 1u);
    u &= 0xFFFF0000u;
    float r;
    std::memcpy(&r, &u, 4);
    return r;
}

uint16_t bf16_bits(float v) {  // of a value already rounded to bf16
    uint32_t u;
    std::memcpy(&u, &v, 4);
    return (uint16_t)(u >> 16);
}

// --------------------------------------------------- 128-value block products
// dot of 128 E4M3 weight bytes with 128 activation values that are exact E4M3
// values (decoded FP8, times 256 in the vector paths so that the weights can
// be widened through fp16 as value / 256).  Every product is exact in fp32
// (two 4-bit significands), so a multiply-add rounds only the sum.  Fixed
// order on every ISA: lane l (0..15) sums the products k = l, l + 16, ...
// in k order, then the lanes fold in halves (l += l + 8, l += l + 4,
// l += l + 2, l += l + 1): the scalar, AVX2 and AVX-512 paths give the same
// bits.

inline float fold16(float (&l)[16]) {
    for (int width = 8; width >= 1; width /= 2)
        for (int i = 0; i < width; ++i) l[i] = l[i] + l[i + width];
    return l[0];
}

inline float dot128_scalar(const uint8_t* w, const float* x) {
    const float* t = table().v;
    float l[16] = {};
    for (int k = 0; k < 128; ++k) l[k % 16] = l[k % 16] + t[w[k]] * x[k];
    return fold16(l);
}

// fp16 bits of byte b: b placed in the high byte of a 16-bit word, shifted
// right arithmetically by one (the sign lands on bits 15 and 14), bit 14 and
// the low 7 bits cleared: sign to bit 15, exponent and mantissa to bits
// 7..13, i.e. the E4M3 value / 256 as an fp16 value (normals and subnormals
// alike).
#define DMOE_AVX2 __attribute__((target("avx2,f16c,fma")))
#define DMOE_AVX512 __attribute__((target("avx512f,avx512bw,avx512vl,avx2,f16c,fma")))

DMOE_AVX2 inline float dot128_avx2(const uint8_t* w, const float* x256) {
    __m256 lo = _mm256_setzero_ps(), hi = _mm256_setzero_ps();  // lanes 0..7, 8..15
    const __m256i keep = _mm256_set1_epi16((short)0xBF80);
    for (int k = 0; k < 128; k += 16) {
        const __m256i b = _mm256_cvtepu8_epi16(_mm_loadu_si128((const __m128i*)(w + k)));
        const __m256i h = _mm256_and_si256(_mm256_srai_epi16(_mm256_slli_epi16(b, 8), 1), keep);
        lo = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm256_castsi256_si128(h)), _mm256_loadu_ps(x256 + k), lo);
        hi = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm256_extracti128_si256(h, 1)), _mm256_loadu_ps(x256 + k + 8), hi);
    }
    const __m256 a8 = _mm256_add_ps(lo, hi);
    const __m128 a4 = _mm_add_ps(_mm256_castps256_ps128(a8), _mm256_extractf128_ps(a8, 1));
    const __m128 a2 = _mm_add_ps(a4, _mm_movehl_ps(a4, a4));
    return _mm_cvtss_f32(_mm_add_ss(a2, _mm_movehdup_ps(a2)));
}

DMOE_AVX512 inline float dot128_avx512(const uint8_t* w, const float* x256) {
    __m512 acc = _mm512_setzero_ps();
    const __m512i keep = _mm512_set1_epi16((short)0xBF80);
    for (int k = 0; k < 128; k += 32) {
        const __m512i b = _mm512_cvtepu8_epi16(_mm256_loadu_si256((const __m256i*)(w + k)));
        const __m512i h = _mm512_and_si512(_mm512_srai_epi16(_mm512_slli_epi16(b, 8), 1), keep);
        acc = _mm512_fmadd_ps(_mm512_cvtph_ps(_mm512_castsi512_si256(h)), _mm512_loadu_ps(x256 + k), acc);
        acc = _mm512_fmadd_ps(_mm512_cvtph_ps(_mm512_extracti64x4_epi64(h, 1)), _mm512_loadu_ps(x256 + k + 16), acc);
    }
    const __m256 a8 = _mm256_add_ps(_mm512_castps512_ps256(acc),
                                    _mm256_castpd_ps(_mm512_extractf64x4_pd(_mm512_castps_pd(acc), 1)));
    const __m128 a4 = _mm_add_ps(_mm256_castps256_ps128(a8), _mm256_extractf128_ps(a8, 1));
    const __m128 a2 = _mm_add_ps(a4, _mm_movehl_ps(a4, a4));
    return _mm_cvtss_f32(_mm_add_ss(a2, _mm_movehdup_ps(a2)));
}

// One gate or up row: per wave w the fma chain over K blocks w, w + 8, ...,
// then the 8 waves' chains summed in wave order (the decode kernels' order; a
// wave without blocks adds its +0).  One down row: one fma chain over the K
// blocks in order.  `srow` is the row's scales, `kstep` their K-block stride
// (0 for one scale per channel).  One copy per ISA so that the block products
// inline.
#define DMOE_ROW_KERNELS(NAME, ATTR, DOT)                                                                  \
    ATTR float NAME##_gate_up_row(const uint8_t* wr, const float* srow, int64_t kstep, const float* x,      \
                                  const float* xs, int KB) {                                                \
        float sum = 0.0f;                                                                                   \
        for (int w = 0; w < kWaveSplit; ++w) {                                                              \
            float acc = 0.0f;                                                                               \
            for (int kb = w; kb < KB; kb += kWaveSplit)                                                     \
                acc = std::fma(DOT(wr + kb * 128, x + kb * 128) * xs[kb], srow[kb * kstep], acc);          \
            sum = w == 0 ? acc : sum + acc;                                                                 \
        }                                                                                                   \
        return sum;                                                                                         \
    }                                                                                                       \
    ATTR float NAME##_down_row(const uint8_t* wr, const float* srow, int64_t kstep, const float* hq,       \
                               const float* hs, int KB) {                                                   \
        float acc = 0.0f;                                                                                   \
        for (int kb = 0; kb < KB; ++kb)                                                                     \
            acc = std::fma(DOT(wr + kb * 128, hq + kb * 128) * hs[kb], srow[kb * kstep], acc);             \
        return acc;                                                                                         \
    }

DMOE_ROW_KERNELS(scalar, , dot128_scalar)
DMOE_ROW_KERNELS(avx2, DMOE_AVX2, dot128_avx2)
DMOE_ROW_KERNELS(avx512, DMOE_AVX512, dot128_avx512)

using RowFn = float (*)(const uint8_t* w, const float* srow, int64_t kstep, const float* x, const float* xs, int KB);

// The best vector ISA of this host: 3 AVX-512 (F, BW, VL), 2 AVX2 + F16C, 1 scalar.
int detect_isa() {
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512f") && __builtin_cpu_supports("avx512bw") && __builtin_cpu_supports("avx512vl"))
        return 3;
    if (__builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma")) return 2;
    return 1;
}

// ------------------------------------------------------------------ banks

struct Proj {
    const uint8_t* w;
    const float* s;
    int64_t w_se, w_sn, s_se, s_sn, s_sk;
    int n_div, kb_div, N, K;
    const uint8_t* row(int64_t e, int n) const { return w + e * w_se + (int64_t)n * w_sn; }
    // scales of row n of expert e, K block kb at srow(e, n)[kb * kstep()]
    const float* srow(int64_t e, int n) const { return s + e * s_se + (int64_t)(n / n_div) * s_sn; }
    int64_t kstep() const { return kb_div == 1 ? s_sk : 0; }  // kb_div is 1 or K / 128 (one scale per row)
};

Proj host_proj(const DmoeFp8Proj& p) {
    if (!p.weight || !p.scale) throw std::invalid_argument("FP8 projection weight and scale pointers are required");
    if (p.k < 128 || p.k % 128 || p.n < 16) throw std::invalid_argument("FP8 projection geometry");
    if (p.weight_stride_n < p.k || p.weight_stride_e < 0) throw std::invalid_argument("FP8 weight strides");
    const bool chan = p.scale_rows == p.n, block = p.n % 128 == 0 && p.scale_rows == p.n / 128;
    if (!(chan || block) || !(p.scale_cols == 1 || p.scale_cols == p.k / 128))
        throw std::invalid_argument("FP8 scales must be per channel or 128x128 blocks");
    return Proj{p.weight, p.scale, p.weight_stride_e, p.weight_stride_n, p.scale_stride_e, p.scale_stride_n,
                p.scale_stride_k, p.n / p.scale_rows, (p.k / 128) / p.scale_cols, p.n, p.k};
}

// ------------------------------------------------------------- thread pool

class Pool {
   public:
    explicit Pool(int threads) {
        for (int i = 1; i < threads; ++i) workers_.emplace_back([this] { loop(); });
    }
    ~Pool() {
        {
            std::lock_guard<std::mutex> lock(mu_);
            stop_ = true;
            epoch_.fetch_add(1, std::memory_order_release);
        }
        start_.notify_all();
        for (auto& t : workers_) t.join();
    }
    int threads() const { return (int)workers_.size() + 1; }

    // Runs fn(0 .. tasks-1) on every thread (the caller included); rethrows
    // the first exception once all threads are done.  Idle threads spin for
    // up to kSpinMicros before they block, so the phases of one call and
    // back-to-back calls do not wait for thread wake-ups.
    void run(int tasks, const std::function<void(int)>& fn) {
        {
            std::lock_guard<std::mutex> lock(mu_);
            fn_ = &fn;
            tasks_ = tasks;
            next_.store(0);
            failure_ = nullptr;
            busy_.store((int)workers_.size(), std::memory_order_relaxed);
            epoch_.fetch_add(1, std::memory_order_release);
        }
        start_.notify_all();
        consume();
        spin_until([&] { return busy_.load(std::memory_order_acquire) == 0; });
        if (busy_.load(std::memory_order_acquire) != 0) {
            std::unique_lock<std::mutex> lock(mu_);
            done_.wait(lock, [this] { return busy_.load(std::memory_order_acquire) == 0; });
        }
        fn_ = nullptr;
        if (failure_) std::rethrow_exception(failure_);
    }

   private:
    static constexpr int kSpinMicros = 200;
    template <class Ready>
    static void spin_until(Ready&& ready) {
        const auto limit = std::chrono::steady_clock::now() + std::chrono::microseconds(kSpinMicros);
        for (;;) {
            for (int i = 0; i < 64; ++i) {
                if (ready()) return;
                _mm_pause();
            }
            if (std::chrono::steady_clock::now() >= limit) return;
        }
    }
    void consume() {
        try {
            for (int t; (t = next_.fetch_add(1)) < tasks_;) (*fn_)(t);
        } catch (...) {
            std::lock_guard<std::mutex> lock(mu_);
            if (!failure_) failure_ = std::current_exception();
            next_.store(tasks_);
        }
    }
    void loop() {
        uint64_t seen = 0;
        for (;;) {
            spin_until([&] { return epoch_.load(std::memory_order_acquire) != seen; });
            {
                std::unique_lock<std::mutex> lock(mu_);
                start_.wait(lock, [&] { return epoch_.load(std::memory_order_acquire) != seen; });
                if (stop_) return;
                seen = epoch_.load(std::memory_order_relaxed);
            }
            consume();
            if (busy_.fetch_sub(1, std::memory_order_acq_rel) == 1) {
                std::lock_guard<std::mutex> lock(mu_);
                done_.notify_one();
            }
        }
    }
    std::vector<std::thread> workers_;
    std::mutex mu_;
    std::condition_variable start_, done_;
    const std::function<void(int)>* fn_ = nullptr;
    int tasks_ = 0;
    std::atomic<int> next_{0}, busy_{0};
    std::atomic<uint64_t> epoch_{0};
    bool stop_ = false;
    std::exception_ptr failure_;
};

// ---------------------------------------------------------------- executor

struct GuardHit : std::exception {};

class Executor {
   public:
    Executor(int hidden, int inter, int capacity, int threads, int isa)
        : H_(hidden), I_(inter), cap_(capacity), isa_(isa), pool_(threads),
          x256_(hidden), xs_(hidden / 128), h_((size_t)capacity * inter), hq256_((size_t)capacity * inter),
          hs_((size_t)capacity * (inter / 128)), parts_done_((size_t)capacity * (inter / 128)) {
        gate_up_row_ = isa_ == 3 ? avx512_gate_up_row : isa_ == 2 ? avx2_gate_up_row : scalar_gate_up_row;
        down_row_ = isa_ == 3 ? avx512_down_row : isa_ == 2 ? avx2_down_row : scalar_down_row;
    }
    int isa() const { return isa_; }
    int threads() const { return pool_.threads(); }
    void set_guard(bool on) { guard_ = on; }
    void set_silu_table(const float* t) { silu_ = t; }

    // Returns false when the guard found an E4M3 rounding midpoint.
    bool pairs(const DmoeFp8Bank& bank, const uint8_t* xq, const float* xs, int x_group, const int64_t* ids,
               const float* weights, int jobs, float* out) {
        std::lock_guard<std::mutex> one_call(call_mu_);
        const Proj w13 = host_proj(bank.w13), w2 = host_proj(bank.w2);
        if (w13.K != H_ || w13.N != 2 * I_ || w2.N != H_ || w2.K != I_)
            throw std::invalid_argument("bank geometry differs from the executor's");
        if (jobs < 1 || jobs > cap_) throw std::invalid_argument("route slot count outside the executor's capacity");
        if (!silu_) throw std::invalid_argument("the executor needs the device SiLU table (dmoe_silu_table)");
        if (x_group != 128 && x_group != H_) throw std::invalid_argument("activation group must be 128 or the hidden size");
        for (int j = 0; j < jobs; ++j) {
            if (ids[j] < 0 || ids[j] >= bank.experts) throw std::invalid_argument("route expert id outside the bank");
            if (!std::isfinite(weights[j])) throw std::invalid_argument("non-finite route weight");
        }
        const bool vec = isa_ > 1;
        for (int k = 0; k < H_; ++k) {
            const float v = table().v[xq[k]];
            if (!std::isfinite(v)) throw std::invalid_argument("non-finite FP8 activation");
            x256_[k] = vec ? v * 256.0f : v;
        }
        for (int g = 0; g < H_ / 128; ++g) {
            const float s = xs[x_group == 128 ? g : 0];
            if (!(s > 0.0f) || !std::isfinite(s)) throw std::invalid_argument("invalid FP8 activation scale");
            xs_[g] = s;
        }
        // Phase 1: gate/up rows in tasks of kUpRows (every slot at once); the
        // task that completes a 128-row group of h quantizes that group.
        constexpr int kUpRows = 32, kParts = 128 / kUpRows;
        const int groups = I_ / 128, up_tasks = I_ / kUpRows;
        for (int i = 0; i < jobs * groups; ++i) parts_done_[i].store(0, std::memory_order_relaxed);
        std::atomic<bool> boundary{false};
        const int KB = H_ / 128, KBd = I_ / 128;
        const int64_t ks13 = w13.kstep(), ks2 = w2.kstep();
        pool_.run(jobs * up_tasks, [&](int task) {
            const int j = task / up_tasks, n0 = (task % up_tasks) * kUpRows, g = n0 / 128;
            const int64_t e = ids[j];
            for (int n = n0; n < n0 + kUpRows; ++n) {
                const float gv = bf16_round(gate_up_row_(w13.row(e, n), w13.srow(e, n), ks13, x256_.data(), xs_.data(), KB));
                const float uv = bf16_round(
                    gate_up_row_(w13.row(e, I_ + n), w13.srow(e, I_ + n), ks13, x256_.data(), xs_.data(), KB));
                h_[(size_t)j * I_ + n] = silu_[bf16_bits(gv)] * uv;
            }
            if (parts_done_[(size_t)j * groups + g].fetch_add(1, std::memory_order_acq_rel) == kParts - 1 &&
                quantize_group(j, g, vec))
                boundary.store(true, std::memory_order_relaxed);
        });
        if (boundary.load()) return false;
        // Phase 2: down rows.
        constexpr int kDownRows = 64;
        const int dn_tasks = (H_ + kDownRows - 1) / kDownRows;
        pool_.run(jobs * dn_tasks, [&](int task) {
            const int j = task / dn_tasks, n0 = (task % dn_tasks) * kDownRows, n1 = std::min(H_, n0 + kDownRows);
            const int64_t e = ids[j];
            const float* hq = &hq256_[(size_t)j * I_];
            const float* hs = &hs_[(size_t)j * KBd];
            for (int n = n0; n < n1; ++n) {
                const float y = down_row_(w2.row(e, n), w2.srow(e, n), ks2, hq, hs, KBd) * weights[j];
                if (!std::isfinite(y)) throw std::invalid_argument("non-finite expert output");
                out[(size_t)j * H_ + n] = y;
            }
        });
        return true;
    }

   private:
    // FP8 128-group g of slot j's h (scale = max(amax, 1e-10) * fl(1/448),
    // true division, E4M3 round-to-nearest-even); true when the guard finds a
    // quotient near an E4M3 rounding midpoint.
    bool quantize_group(int j, int g, bool vec) {
        const float* h = &h_[(size_t)j * I_ + g * 128];
        float amax = 0.0f;
        for (int k = 0; k < 128; ++k) {
            if (!std::isfinite(h[k])) throw std::invalid_argument("non-finite hidden activation");
            amax = std::max(amax, std::fabs(h[k]));
        }
        const float scale = std::max(amax, 1e-10f) * kInv448;
        hs_[(size_t)j * (I_ / 128) + g] = scale;
        float* q = &hq256_[(size_t)j * I_ + g * 128];
        bool near = false;
        for (int k = 0; k < 128; ++k) {
            const float r = h[k] / scale;
            if (guard_ && near_e4m3_midpoint(r)) near = true;
            const float v = table().v[e4m3_encode(r)];
            q[k] = vec ? v * 256.0f : v;
        }
        return near;
    }

    int H_, I_, cap_, isa_;
    RowFn gate_up_row_, down_row_;
    Pool pool_;
    bool guard_ = false;
    const float* silu_ = nullptr;
    std::vector<float> x256_, xs_, h_, hq256_, hs_;
    std::vector<std::atomic<int>> parts_done_;
    std::mutex call_mu_;
};

template <class F>
int guarded(F&& body) {
    try {
        body();
        return 0;
    } catch (const std::exception& e) {
        dmoe::set_last_error(e.what());
    } catch (...) {
        dmoe::set_last_error("unknown native exception");
    }
    return -1;
}

}  // namespace

extern "C" {

void* dmoe_cpu_executor_create(int hidden, int inter, int capacity, int threads, int isa) {
    Executor* ex = nullptr;
    guarded([&] {
        if (hidden < 128 || hidden > 32768 || hidden % 128 || inter < 128 || inter > 16384 || inter % 128 ||
            capacity < 1 || capacity > 256 || threads < 1 || threads > 256)
            throw std::invalid_argument("unsupported CPU executor geometry, capacity or thread count");
        const int best = detect_isa();
        if (isa < 0 || isa > 3 || isa > best) throw std::invalid_argument("requested CPU vector ISA is unavailable");
        ex = new Executor(hidden, inter, capacity, threads, isa == 0 ? best : isa);
        dmoe::set_last_error("");
    });
    return ex;
}

void dmoe_cpu_executor_destroy(void* executor) { delete static_cast<Executor*>(executor); }

int dmoe_cpu_executor_isa(void* executor) { return executor ? static_cast<Executor*>(executor)->isa() : 0; }

int dmoe_cpu_executor_threads(void* executor) { return executor ? static_cast<Executor*>(executor)->threads() : 0; }

int dmoe_cpu_executor_set_guard(void* executor, int enabled) {
    return guarded([&] {
        if (!executor) throw std::invalid_argument("missing CPU executor");
        static_cast<Executor*>(executor)->set_guard(enabled != 0);
    });
}

int dmoe_cpu_executor_set_silu_table(void* executor, const float* table) {
    return guarded([&] {
        if (!executor || !table) throw std::invalid_argument("missing CPU executor or SiLU table");
        static_cast<Executor*>(executor)->set_silu_table(table);
    });
}

int dmoe_cpu_expert_pairs(void* executor, const DmoeFp8Bank* bank, const uint8_t* xq, const float* xs, int x_group,
                          const int64_t* ids, const float* weights, int jobs, float* out) {
    int result = -1;
    const int rc = guarded([&] {
        if (!executor || !bank || !xq || !xs || !ids || !weights || !out)
            throw std::invalid_argument("CPU expert call: missing executor or buffer");
        result = static_cast<Executor*>(executor)->pairs(*bank, xq, xs, x_group, ids, weights, jobs, out)
                     ? 0
                     : DMOE_CPU_GPU_RECOMPUTE;
        if (result != 0) dmoe::set_last_error("an FP8 rounding midpoint of the hidden activation: recompute on the GPU");
    });
    return rc == 0 ? result : -1;
}

int dmoe_cpu_partition_routes(const int64_t* ids, int count, const int64_t* resident, int resident_count, int experts,
                              int cpu_jobs, int64_t* cpu_slots, int64_t* gpu_slots) {
    return guarded([&] {
        if (!ids || !cpu_slots || !gpu_slots || count < 1 || count > 64 || experts < 1 || resident_count < 0 ||
            (resident_count > 0 && !resident) || cpu_jobs < 0 || cpu_jobs > count)
            throw std::invalid_argument("route partition: bad counts or buffers");
        for (int i = 0; i < count; ++i)
            if (ids[i] < 0 || ids[i] >= experts) throw std::invalid_argument("route expert id outside the bank");
        // the cold slots (expert not resident on the GPU) from the lowest
        // rank up, then the resident ones; both lists keep slot order
        std::vector<char> cpu(count, 0);
        int left = cpu_jobs;
        for (int pass = 0; pass < 2 && left > 0; ++pass)
            for (int slot = count - 1; slot >= 0 && left > 0; --slot) {
                const bool hot = std::find(resident, resident + resident_count, ids[slot]) != resident + resident_count;
                if (hot == (pass == 1)) {
                    cpu[slot] = 1;
                    --left;
                }
            }
        int c = 0, g = 0;
        for (int slot = 0; slot < count; ++slot) (cpu[slot] ? cpu_slots[c++] : gpu_slots[g++]) = slot;
    });
}

}  // extern "C"
