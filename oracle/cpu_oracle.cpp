// CPU oracle for the FP16 conv-graph path — TEST INFRASTRUCTURE ONLY.
//
// Restates the reference CPU backend (backends/cpu) for the operators on the
// conv-graph path, to serve as the parity checker of the HIP backend and as
// the CPU baseline timed beside it. Only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg load this library; the product never does.
//
// What is restated, with the reference lines it follows:
//   * FP16 <-> FP32 RNE conversion: core/include/mlvc/core/half.hpp:10-87
//     (the AVX2 path converts with F16C, kernels_x86_avx2.cpp:17-28; both
//     round to nearest even).
//   * Weight packing f16p16x1bias: kernels_scalar.cpp:14-56 (per 16 output
//     channels: 16 biases, then K rows of 16 weights, K = (ky, kx, ic));
//     depthwise packing kernels_scalar.cpp:58-77.
//   * GEMM micro-kernel: kernels_x86_avx2.cpp:69-235 (accumulator seeded with
//     the bias, one fused multiply-add per K step in K order, FP16 rounding
//     before the epilogue) used when N % 16 == 0; otherwise the scalar
//     kernel kernels_scalar.cpp:160-195, whose multiply and add round
//     separately (that file is built without FMA).
//   * 1x1 conv: execute_gemm_nhwc kernels_scalar.cpp:627-692; KxK conv:
//     execute_spatial_conv_nhwc :694-781 (im2col with zero-filled halos).
//   * Depthwise: avx2_depthwise3x3_s1p1 kernels_x86_avx2.cpp:237-302 (C % 8
//     == 0, fused taps in (ky,kx) order skipping out-of-range taps), else
//     scalar_depthwise3x3_s1p1 kernels_scalar.cpp:198-242; other shapes
//     execute_depthwise_generic_nhwc :783-828.
//   * LeakyReLU / ADD: kernels_x86_avx2.cpp:304-322,382-398 and scalar
//     :244-268. Pixel shuffle/unshuffle (CRD): kernels_scalar.cpp:954-1026.
//     Channel CONCAT: kernels_scalar.cpp:893-928 (axis 1 case).
//   * Codec I/O around the encoder/decoder graphs: frame -> model input and
//     model output -> frame conversions, execution_plan.cpp:1044-1322, and
//     frame_padding, core/src/yuv.cpp:325-337.
//   * Plan: NHWC re-layout of 4-D FP16 tensors with C > 1 and H*W > 1
//     (execution_plan.cpp:78-82, 639-665, 1324-1358), conv classification
//     (:410-462), state bindings (:349-369, 806-816, 1033-1042), run()
//     checks (:1623-1675), the conv epilogue matcher
//     (fusion_matcher.cpp:352-411) and the thread-count rule
//     (thread_pool.cpp:35-69).
//
//   * Operators of the real-model graphs: CLIP / SIGMOID / RECIPROCAL /
//     ROUND (scalar_unary kernels_scalar.cpp:80-97, 244-255; avx2_unary
//     kernels_x86_avx2.cpp:30-62, 304-352 with its polynomial exp), ADD /
//     SUB / MUL with every broadcast form (execution_plan.cpp:170-236,
//     527-563, 958-985), SLICE (:565-604; kernels_scalar.cpp:830-890),
//     CONCAT on any axis (:606-620; kernels_scalar.cpp:892-952), GATHER
//     (:101-168, 1004-1012).
//   * The real-model fusions and their matcher (fusion_matcher.cpp:258-850):
//     ReGLU (standalone and as a 1x1 conv epilogue), the recurrent feature
//     update (one- and three-output forms), the y0 / y1 quantisation tails
//     (kernels_scalar.cpp:304-537, kernels_x86_avx2.cpp:443-712).
// Parity pins: see the test files under tests/ (bit-exact against the
// reference kernels built from source, known-answer graphs, brute force,
// numpy semantics where the reference code sits in its plan).

#include "oracle.h"

#include <immintrin.h>

#include <algorithm>
#include <array>
#include <cmath>
#include <atomic>
#include <bit>
#include <condition_variable>
#include <cstring>
#include <fstream>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

namespace {

using u16 = std::uint16_t;
thread_local std::string g_error;

// ---------------------------------------------------------------- FP16
float h2f(u16 h)
{
    const std::uint32_t sign = (static_cast<std::uint32_t>(h) & 0x8000U) << 16;
    const std::uint32_t e = (h >> 10) & 0x1FU;
    std::uint32_t m = h & 0x3FFU;
    std::uint32_t bits;
    if (e == 0x1F) {
        bits = sign | 0x7F800000U | (m << 13) | (m ? 0x400000U : 0U);
    } else if (e) {
        bits = sign | ((e + 112U) << 23) | (m << 13);
    } else if (!m) {
        bits = sign;
    } else {
        int ex = 113;
        while (!(m & 0x400U)) { m <<= 1; --ex; }
        bits = sign | (static_cast<std::uint32_t>(ex) << 23) | ((m & 0x3FFU) << 13);
    }
    return std::bit_cast<float>(bits);
}

u16 f2h(float f)
{
    const std::uint32_t x = std::bit_cast<std::uint32_t>(f);
    const auto sign = static_cast<u16>((x >> 16) & 0x8000U);
    const std::uint32_t e = (x >> 23) & 0xFF, m = x & 0x7FFFFF;
    if (e == 0xFF) return static_cast<u16>(sign | 0x7C00U | (m ? (0x200U | (m >> 13)) : 0U));
    int he = static_cast<int>(e) - 112;
    if (he >= 31) return static_cast<u16>(sign | 0x7C00U);
    if (he <= 0) {
        if (he < -10) return sign;
        const std::uint32_t mm = m | 0x800000U;
        const unsigned sh = static_cast<unsigned>(14 - he);
        std::uint32_t q = mm >> sh;
        const std::uint32_t r = mm & ((1U << sh) - 1U), hw = 1U << (sh - 1U);
        if (r > hw || (r == hw && (q & 1U))) ++q;
        return static_cast<u16>(sign | q);
    }
    std::uint32_t q = m >> 13;
    const std::uint32_t r = m & 0x1FFFU;
    if (r > 0x1000U || (r == 0x1000U && (q & 1U))) {
        if (++q == 0x400U) {
            q = 0;
            if (++he >= 31) return static_cast<u16>(sign | 0x7C00U);
        }
    }
    return static_cast<u16>(sign | (static_cast<u16>(he) << 10) | q);
}

inline __m256 ld8(const u16* p) { return _mm256_cvtph_ps(_mm_loadu_si128(reinterpret_cast<const __m128i*>(p))); }
inline void st8(u16* p, __m256 v)
{
    _mm_storeu_si128(reinterpret_cast<__m128i*>(p), _mm256_cvtps_ph(v, _MM_FROUND_TO_NEAREST_INT));
}
inline __m256 round_h(__m256 v) { return _mm256_cvtph_ps(_mm256_cvtps_ph(v, _MM_FROUND_TO_NEAREST_INT)); }

// --------------------------------------------------------------- threads
int default_threads()
{
    const unsigned hw = std::max(1U, std::thread::hardware_concurrency());
    std::vector<unsigned long> freqs;
    for (unsigned cpu = 0; cpu < hw; ++cpu) {
        std::ifstream f("/sys/devices/system/cpu/cpu" + std::to_string(cpu) + "/cpufreq/cpuinfo_max_freq");
        unsigned long v = 0;
        if (f >> v && v > 0) freqs.push_back(v);
    }
    if (!freqs.empty()) {
        const unsigned long peak = *std::max_element(freqs.begin(), freqs.end());
        int fast = 0;
        for (unsigned long v : freqs) fast += (v * 100 >= peak * 60) ? 1 : 0;
        if (fast > 0) return std::min(fast, 16);
    }
    return static_cast<int>(std::min(hw, 16U));
}

class Pool {
public:
    explicit Pool(int n) : n_(std::max(1, n))
    {
        for (int i = 1; i < n_; ++i) workers_.emplace_back([this] { loop(); });
    }
    ~Pool()
    {
        {
            std::lock_guard<std::mutex> l(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto& t : workers_) t.join();
    }
    int size() const { return n_; }
    // Runs fn(begin, end) over [0, total) in chunks of `grain`.
    void parallel_for(std::size_t total, std::size_t grain, const std::function<void(std::size_t, std::size_t)>& fn)
    {
        if (total == 0) return;
        grain = std::max<std::size_t>(1, grain);
        if (n_ == 1 || total <= grain) { fn(0, total); return; }
        {
            std::unique_lock<std::mutex> l(mu_);
            job_ = &fn;
            total_ = total;
            grain_ = grain;
            next_.store(0);
            active_ = static_cast<int>(workers_.size());
            ++gen_;
        }
        cv_.notify_all();
        work();
        std::unique_lock<std::mutex> l(mu_);
        done_cv_.wait(l, [this] { return active_ == 0; });
        job_ = nullptr;
        if (err_) { auto e = err_; err_ = nullptr; std::rethrow_exception(e); }
    }

private:
    void work()
    {
        for (;;) {
            const std::size_t b = next_.fetch_add(grain_);
            if (b >= total_) return;
            try {
                (*job_)(b, std::min(total_, b + grain_));
            } catch (...) {
                std::lock_guard<std::mutex> l(mu_);
                if (!err_) err_ = std::current_exception();
            }
        }
    }
    void loop()
    {
        std::uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> l(mu_);
                cv_.wait(l, [&] { return stop_ || gen_ != seen; });
                if (stop_) return;
                seen = gen_;
            }
            work();
            std::lock_guard<std::mutex> l(mu_);
            if (--active_ == 0) done_cv_.notify_all();
        }
    }
    int n_;
    std::vector<std::thread> workers_;
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    const std::function<void(std::size_t, std::size_t)>* job_ = nullptr;
    std::size_t total_ = 0, grain_ = 1;
    std::atomic<std::size_t> next_{0};
    int active_ = 0;
    std::uint64_t gen_ = 0;
    bool stop_ = false;
    std::exception_ptr err_;
};

// --------------------------------------------------------------- packing
std::size_t packed_conv_elems(std::size_t oc, std::size_t ic, std::size_t kh, std::size_t kw)
{
    return (oc + 15) / 16 * (16 + kh * kw * ic * 16);
}

void pack_conv(const u16* w, const u16* bias, std::size_t oc, std::size_t ic, std::size_t kh,
               std::size_t kw, u16* out)
{
    const std::size_t kdim = kh * kw * ic, blk = 16 + kdim * 16;
    std::fill(out, out + packed_conv_elems(oc, ic, kh, kw), u16{0});
    for (std::size_t n0 = 0; n0 < oc; n0 += 16) {
        u16* b = out + n0 / 16 * blk;
        const std::size_t vn = std::min<std::size_t>(16, oc - n0);
        for (std::size_t j = 0; j < vn; ++j) b[j] = bias ? bias[n0 + j] : 0;
        for (std::size_t ky = 0; ky < kh; ++ky)
            for (std::size_t kx = 0; kx < kw; ++kx)
                for (std::size_t c = 0; c < ic; ++c) {
                    u16* row = b + 16 + ((ky * kw + kx) * ic + c) * 16;
                    for (std::size_t j = 0; j < vn; ++j) row[j] = w[(((n0 + j) * ic + c) * kh + ky) * kw + kx];
                }
    }
}

std::size_t packed_dw_elems(std::size_t c, std::size_t kh, std::size_t kw)
{
    return (kh * kw + 1) * ((c + 15) / 16 * 16);
}

void pack_dw(const u16* w, const u16* bias, std::size_t c, std::size_t kh, std::size_t kw, u16* out)
{
    const std::size_t pc = (c + 15) / 16 * 16, taps = kh * kw;
    std::fill(out, out + packed_dw_elems(c, kh, kw), u16{0});
    for (std::size_t i = 0; i < c; ++i) out[i] = bias ? bias[i] : 0;
    for (std::size_t t = 0; t < taps; ++t)
        for (std::size_t i = 0; i < c; ++i) out[pc + t * pc + i] = w[i * taps + t];
}

// ------------------------------------------------------------------ GEMM
enum Epi { kNone = 0, kClamp = 1, kLeaky = 2, kResidual = 3 };
struct Epilogue {
    int kind = kNone;
    float alpha = 0.0F, cmin = 0.0F, cmax = 0.0F;
    const u16* residual = nullptr;  // row-major [rows, dst_stride]
};

// Rows [row0, row0+m) of dst (stride n) from lhs rows (stride lhs_stride).
void block_avx2(std::size_t m, std::size_t n, std::size_t k, const u16* lhs, std::size_t lhs_stride,
                const u16* packed, u16* dst, const Epilogue& e, std::size_t row0)
{
    const std::size_t blk = 16 + k * 16;
    const __m256 valpha = _mm256_set1_ps(e.alpha), vmin = _mm256_set1_ps(e.cmin),
                 vmax = _mm256_set1_ps(e.cmax), vzero = _mm256_setzero_ps();
    for (std::size_t mi = 0; mi < m; mi += 6) {
        const std::size_t mr = std::min<std::size_t>(6, m - mi);
        const u16* a[6];
        for (std::size_t r = 0; r < 6; ++r) a[r] = lhs + (mi + std::min(r, mr - 1)) * lhs_stride;
        for (std::size_t nb = 0; nb < n; nb += 16) {
            const u16* wb = packed + nb / 16 * blk;
            __m256 c0[6], c1[6];
            const __m256 b0 = ld8(wb), b1 = ld8(wb + 8);
            for (int r = 0; r < 6; ++r) { c0[r] = b0; c1[r] = b1; }
            const u16* wp = wb + 16;
            for (std::size_t kk = 0; kk < k; ++kk, wp += 16) {
                const __m256 w0 = ld8(wp), w1 = ld8(wp + 8);
                for (std::size_t r = 0; r < mr; ++r) {
                    const __m256 s = _mm256_set1_ps(_cvtsh_ss(a[r][kk]));
                    c0[r] = _mm256_fmadd_ps(w0, s, c0[r]);
                    c1[r] = _mm256_fmadd_ps(w1, s, c1[r]);
                }
            }
            for (std::size_t r = 0; r < mr; ++r) {
                __m256 h0 = round_h(c0[r]), h1 = round_h(c1[r]);
                if (e.kind == kClamp) {
                    h0 = _mm256_max_ps(_mm256_min_ps(h0, vmax), vmin);
                    h1 = _mm256_max_ps(_mm256_min_ps(h1, vmax), vmin);
                } else if (e.kind == kLeaky) {
                    h0 = _mm256_blendv_ps(h0, _mm256_mul_ps(h0, valpha), _mm256_cmp_ps(h0, vzero, _CMP_LT_OQ));
                    h1 = _mm256_blendv_ps(h1, _mm256_mul_ps(h1, valpha), _mm256_cmp_ps(h1, vzero, _CMP_LT_OQ));
                } else if (e.kind == kResidual && e.residual) {
                    const u16* rr = e.residual + (row0 + mi + r) * n + nb;
                    h0 = _mm256_add_ps(h0, ld8(rr));
                    h1 = _mm256_add_ps(h1, ld8(rr + 8));
                }
                u16* o = dst + (mi + r) * n + nb;
                st8(o, h0);
                st8(o + 8, h1);
            }
        }
    }
}

void block_scalar(std::size_t m, std::size_t n, std::size_t k, const u16* lhs, std::size_t lhs_stride,
                  const u16* packed, u16* dst, const Epilogue& e, std::size_t row0)
{
    const std::size_t blk = 16 + k * 16;
    for (std::size_t mi = 0; mi < m; ++mi) {
        const u16* a = lhs + mi * lhs_stride;
        for (std::size_t nb = 0; nb < n; nb += 16) {
            const u16* wb = packed + nb / 16 * blk;
            const std::size_t vn = std::min<std::size_t>(16, n - nb);
            float acc[16];
            for (std::size_t j = 0; j < vn; ++j) acc[j] = h2f(wb[j]);
            for (std::size_t kk = 0; kk < k; ++kk) {
                const float av = h2f(a[kk]);
                const u16* wr = wb + 16 + kk * 16;
                for (std::size_t j = 0; j < vn; ++j) {
                    const float p = av * h2f(wr[j]);  // rounded product, then rounded sum
                    acc[j] = acc[j] + p;
                }
            }
            for (std::size_t j = 0; j < vn; ++j) {
                u16 hv = f2h(acc[j]);
                if (e.kind == kClamp) {
                    hv = f2h(std::min(std::max(h2f(hv), e.cmin), e.cmax));
                } else if (e.kind == kLeaky) {
                    const float fv = h2f(hv);
                    if (fv < 0.0F) hv = f2h(fv * e.alpha);
                } else if (e.kind == kResidual && e.residual) {
                    hv = f2h(h2f(hv) + h2f(e.residual[(row0 + mi) * n + nb + j]));
                }
                dst[mi * n + nb + j] = hv;
            }
        }
    }
}

// isa 2 (test-only, not a reference path): the GPU kernels' accumulation.
// The GPU convs take K as (16-channel step, tap): for each step of up to 16
// input channels, each tap's 16 products are one v_mfma_f32_32x32x16_f16
// step (channels c0..c0+7 in one half of the wave, c0+8..c0+15 in the
// other). mfma_step() is that instruction's arithmetic as measured on
// MI355X with a probe of single instructions (every output of 163,568 test
// cases reproduced bit for bit, ordinary, cancelling, wide-exponent,
// tiny-addend and structured cases): the two halves of K are added in turn,
// each half as
//   E = max over its non-zero products of exp(a) + exp(b) (FP16 exponents,
//       subnormals at -14);
//   products truncated toward zero, and the FP32 accumulator floored, to
//   multiples of 2^(E-24); their sum floored to 8 bits below the ulp of its
//   leading bit; then rounded to FP32, nearest even.
// The accumulator is seeded with the bias; FP16 rounding and the epilogue
// are the scalar kernel's.
// An FP16 value as (signed integer mantissa m, exponent e) with value
// m * 2^(e - 10); subnormals have e = -14. Packed as (m << 8) | (e + 64).
inline std::int32_t fp16_q(u16 h)
{
    const int ef = (h >> 10) & 31, f = h & 1023;
    const int m = ef ? (f | 1024) : f;
    return static_cast<std::int32_t>(((h & 0x8000) ? -m : m) * 256) | ((ef ? ef - 15 : -14) + 64);
}


inline double pow2i(int e)  // 2^e for -1022 <= e <= 1023
{
    return std::bit_cast<double>(static_cast<std::uint64_t>(static_cast<std::uint32_t>(e + 1023)) << 52);
}

// One half of an MFMA K step: acc + sum of n products, product i being
// P[i] * 2^(E[i] - 20) (P the product of the two integer mantissas, E the
// sum of the two exponents); zero products are skipped.
float mfma_half(float acc, const std::int32_t* P, const int* E, int n)
{
    int emax = INT32_MIN;
    for (int i = 0; i < n; ++i)
        if (P[i] != 0) emax = std::max(emax, E[i]);
    if (emax == INT32_MIN) return acc;
    int frame = emax - 24;  // units of 2^frame
    std::int64_t prod = 0;
    for (int i = 0; i < n; ++i) {
        if (P[i] == 0) continue;
        const int d = emax - E[i] - 4;  // product in frame units: P * 2^-d
        const std::int64_t v = P[i];
        if (d <= 0)
            prod += v << -d;
        else if (d < 23)
            prod += v >= 0 ? (v >> d) : -((-v) >> d);  // toward zero
    }
    __int128 s = prod;
    const auto bits = std::bit_cast<std::uint32_t>(acc);
    const int ef = static_cast<int>((bits >> 23) & 255);
    const std::int64_t frac = bits & 0x7FFFFF;
    if (ef != 0 || frac != 0) {
        const std::int64_t m = (ef ? (frac | 0x800000) : frac) * ((bits >> 31) ? -1 : 1);
        const int shift = (ef ? ef - 127 : -126) - 23 - frame;  // acc = m * 2^(shift + frame)
        if (shift >= 100) {
            // The products sit far below the accumulator's last bit: only
            // their sign can move the floors below.
            s = (static_cast<__int128>(m) << 64) + (prod > 0 ? 1 : prod < 0 ? -1 : 0);
            frame += shift - 64;
        } else if (shift >= 0) {
            s += static_cast<__int128>(m) << shift;
        } else {
            s += shift <= -63 ? (m < 0 ? -1 : 0) : (m >> -shift);  // arithmetic shift: floor
        }
    }
    if (s == 0) return 0.0F;
    const unsigned __int128 mag = s < 0 ? static_cast<unsigned __int128>(-s) : static_cast<unsigned __int128>(s);
    const auto hi = static_cast<std::uint64_t>(mag >> 64), lo = static_cast<std::uint64_t>(mag);
    const int msb = hi ? 127 - std::countl_zero(hi) : 63 - std::countl_zero(lo);
    const int lead = std::max(msb + frame, -126);  // exponent of the leading bit (FP32 normal range)
    const int keep = lead - 23 - 8;                // 8 bits below the ulp
    if (keep > frame) {
        s >>= (keep - frame);  // floor
        frame = keep;
    }
    // |s| < 2^33: exact in double; the float conversion rounds to nearest
    // even.
    return static_cast<float>(static_cast<double>(static_cast<std::int64_t>(s)) * pow2i(frame));
}

// mfma_half for the 16 outputs of one column block at once, in double:
// p[i*16+j] are the exact products, E[i*16+j] their exponent sums. Every
// term is an integer number of frame units, so the sums are exact while the
// accumulator spans fewer than 2^52 units; the loops are branch-free over the
// columns, and a column outside that range goes through mfma_half. Same
// result as mfma_half, bit for bit.
void mfma_half16(float* acc, const double* p, const int* E, int cn, std::size_t vn)
{
    constexpr int kNone = -4000;
    alignas(64) int emax[16], scale_e[16];
    alignas(64) double s[16], a[16], scale[16];
    for (std::size_t j = 0; j < 16; ++j) emax[j] = kNone;
    for (int i = 0; i < cn; ++i)
        for (std::size_t j = 0; j < 16; ++j)
            emax[j] = p[i * 16 + j] != 0.0 ? std::max(emax[j], E[i * 16 + j]) : emax[j];
    for (std::size_t j = 0; j < 16; ++j) {
        scale_e[j] = std::min(std::max(24 - emax[j], -1000), 1000);
        scale[j] = pow2i(scale_e[j]);
        s[j] = 0.0;
    }
    for (int i = 0; i < cn; ++i)
        for (std::size_t j = 0; j < 16; ++j)  // product in frame units, toward zero
            s[j] += std::trunc(p[i * 16 + j] * scale[j]);
    for (std::size_t j = 0; j < 16; ++j) {
        a[j] = static_cast<double>(acc[j]) * scale[j];
        s[j] += std::floor(a[j]);
    }
    for (std::size_t j = 0; j < vn; ++j) {
        if (emax[j] == kNone) continue;
        if (!(std::fabs(a[j]) < 0x1p52)) {
            std::int32_t p8[8];
            int e8[8];
            for (int i = 0; i < cn; ++i) {
                // back to integer mantissa products: p = P * 2^(E - 20)
                p8[i] = static_cast<std::int32_t>(p[i * 16 + j] * pow2i(20 - E[i * 16 + j]));
                e8[i] = E[i * 16 + j];
            }
            acc[j] = mfma_half(acc[j], p8, e8, cn);
            continue;
        }
        const int lsb = emax[j] - 24;
        const int msb = static_cast<int>((std::bit_cast<std::uint64_t>(s[j]) >> 52) & 2047) - 1023;
        const int lead = std::max(msb + lsb, -126);
        const int drop = std::max(lead - 31 - lsb, 0);  // floor to 8 bits below the ulp
        acc[j] = static_cast<float>(std::floor(s[j] * pow2i(-drop)) * pow2i(lsb + drop));
    }
}

// wq: the packed weights (without the bias rows) as fp16_q, [16-column
// block][k][16]; computed here when the caller has none.
// split_c > 0: the GPU's split K (a multiple of 16 channels): each range of
// split_c input channels is summed from zero (the first from the bias) and
// the partial sums are added in order in FP32.
void block_mfma_order(std::size_t m, std::size_t n, std::size_t k, std::size_t ic, const u16* lhs,
                      std::size_t lhs_stride, const u16* packed, u16* dst, const Epilogue& e, std::size_t row0,
                      const std::int32_t* wq, std::size_t split_c)
{
    const std::size_t blk = 16 + k * 16, taps = k / ic, nblk = (n + 15) / 16;
    thread_local std::vector<std::int32_t> wd;
    thread_local std::vector<double> ad, wv;
    thread_local std::vector<int> ae, we;
    if (!wq) {
        wd.resize(nblk * k * 16);
        for (std::size_t b = 0; b < nblk; ++b)
            for (std::size_t i = 0; i < k * 16; ++i) wd[b * k * 16 + i] = fp16_q(packed[b * blk + 16 + i]);
        wq = wd.data();
    }
    wv.resize(nblk * k * 16);
    we.resize(nblk * k * 16);
    for (std::size_t i = 0; i < nblk * k * 16; ++i) {
        wv[i] = static_cast<double>(wq[i] >> 8) * pow2i(((wq[i] & 255) - 64) - 10);
        we[i] = (wq[i] & 255) - 64;
    }
    ad.resize(k);
    ae.resize(k);
    for (std::size_t mi = 0; mi < m; ++mi) {
        const u16* a = lhs + mi * lhs_stride;
        for (std::size_t kk = 0; kk < k; ++kk) {
            const std::int32_t q = fp16_q(a[kk]);
            ad[kk] = static_cast<double>(q >> 8) * pow2i(((q & 255) - 64) - 10);
            ae[kk] = (q & 255) - 64;
        }
        for (std::size_t b = 0; b < nblk; ++b) {
            const std::size_t vn = std::min<std::size_t>(16, n - b * 16);
            float acc[16], total[16] = {};
            bool split_seen = false;
            for (std::size_t j = 0; j < 16; ++j) acc[j] = j < vn ? h2f(packed[b * blk + j]) : 0.0F;
            for (std::size_t c0 = 0; c0 < ic; c0 += 16) {
                if (split_c && c0 > 0 && c0 % split_c == 0) {
                    for (std::size_t j = 0; j < 16; ++j) {
                        total[j] = split_seen ? total[j] + acc[j] : acc[j];
                        acc[j] = 0.0F;
                    }
                    split_seen = true;
                }
                for (std::size_t t = 0; t < taps; ++t)
                    for (std::size_t h0 = c0; h0 < std::min(c0 + 16, ic); h0 += 8) {
                        const int cn = static_cast<int>(std::min<std::size_t>(8, std::min(c0 + 16, ic) - h0));
                        const std::size_t k0 = t * ic + h0, w0 = (b * k + k0) * 16;
                        alignas(64) double P[8 * 16];
                        alignas(64) int E[8 * 16];
                        for (int i = 0; i < cn; ++i)
                            for (std::size_t j = 0; j < 16; ++j) {
                                P[i * 16 + j] = ad[k0 + i] * wv[w0 + i * 16 + j];
                                E[i * 16 + j] = ae[k0 + i] + we[w0 + i * 16 + j];
                            }
                        mfma_half16(acc, P, E, cn, vn);
                    }
            }
            if (split_seen)
                for (std::size_t j = 0; j < 16; ++j) acc[j] = total[j] + acc[j];
            for (std::size_t j = 0; j < vn; ++j) {
                u16 hv = f2h(acc[j]);
                if (e.kind == kClamp) {
                    hv = f2h(std::min(std::max(h2f(hv), e.cmin), e.cmax));
                } else if (e.kind == kLeaky) {
                    const float fv = h2f(hv);
                    if (fv < 0.0F) hv = f2h(fv * e.alpha);
                } else if (e.kind == kResidual && e.residual) {
                    hv = f2h(h2f(hv) + h2f(e.residual[(row0 + mi) * n + b * 16 + j]));
                }
                dst[mi * n + b * 16 + j] = hv;
            }
        }
    }
}

// ic: input channels per tap (k / ic taps) and wconv: the weights as
// fp16_q (or null); only the isa 2 model uses them.
void run_block(int isa, std::size_t m, std::size_t n, std::size_t k, const u16* lhs, std::size_t lhs_stride,
               const u16* packed, u16* dst, const Epilogue& e, std::size_t row0, std::size_t ic = 0,
               const std::int32_t* wconv = nullptr, std::size_t split_c = 0)
{
    if (isa == 2)
        block_mfma_order(m, n, k, ic ? ic : k, lhs, lhs_stride, packed, dst, e, row0, wconv, split_c);
    else if (isa == 0 && n % 16 == 0)
        block_avx2(m, n, k, lhs, lhs_stride, packed, dst, e, row0);
    else
        block_scalar(m, n, k, lhs, lhs_stride, packed, dst, e, row0);
}

constexpr std::size_t kRows = 24;

void gemm_nhwc(Pool& pool, int isa, std::size_t m, std::size_t n, std::size_t k, const u16* lhs,
               const u16* packed, u16* dst, const Epilogue& e, const std::int32_t* wconv = nullptr,
               std::size_t split_c = 0)
{
    const std::size_t tiles = (m + kRows - 1) / kRows;
    pool.parallel_for(tiles, 1, [&](std::size_t t0, std::size_t t1) {
        for (std::size_t t = t0; t < t1; ++t) {
            const std::size_t m0 = t * kRows, mc = std::min(kRows, m - m0);
            run_block(isa, mc, n, k, lhs + m0 * k, k, packed, dst + m0 * n, e, m0, k, wconv, split_c);
        }
    });
}

void spatial_conv_nhwc(Pool& pool, int isa, const u16* in, const u16* packed, u16* out, int bn, int ic,
                       int ih, int iw, int oc, int oh, int ow, int kh, int kw, int sh, int sw, int ph,
                       int pw, const Epilogue& e, const std::int32_t* wconv = nullptr, std::size_t split_c = 0)
{
    const std::size_t total = static_cast<std::size_t>(bn) * oh * ow;
    const std::size_t kdim = static_cast<std::size_t>(kh) * kw * ic;
    const std::size_t strips = (total + kRows - 1) / kRows;
    pool.parallel_for(strips, 1, [&](std::size_t s0, std::size_t s1) {
        std::vector<u16> col(kRows * kdim);
        for (std::size_t s = s0; s < s1; ++s) {
            const std::size_t m0 = s * kRows, mc = std::min(kRows, total - m0);
            for (std::size_t r = 0; r < mc; ++r) {
                const std::size_t lin = m0 + r;
                const int b = static_cast<int>(lin / (static_cast<std::size_t>(oh) * ow));
                const int pl = static_cast<int>(lin % (static_cast<std::size_t>(oh) * ow));
                const int oy = pl / ow, ox = pl % ow;
                u16* dstc = col.data() + r * kdim;
                const u16* ib = in + static_cast<std::size_t>(b) * ih * iw * ic;
                for (int ky = 0; ky < kh; ++ky)
                    for (int kx = 0; kx < kw; ++kx) {
                        const int iy = oy * sh - ph + ky, ix = ox * sw - pw + kx;
                        u16* d = dstc + (static_cast<std::size_t>(ky) * kw + kx) * ic;
                        if (iy < 0 || iy >= ih || ix < 0 || ix >= iw)
                            std::fill(d, d + ic, u16{0});
                        else
                            std::memcpy(d, ib + (static_cast<std::size_t>(iy) * iw + ix) * ic, ic * sizeof(u16));
                    }
            }
            run_block(isa, mc, static_cast<std::size_t>(oc), kdim, col.data(), kdim, packed,
                      out + m0 * static_cast<std::size_t>(oc), e, m0, static_cast<std::size_t>(ic), wconv, split_c);
        }
    });
}

void depthwise_nhwc(Pool& pool, int isa, const u16* in, const u16* packed, u16* out, int bn, int c,
                    int ih, int iw, int oh, int ow, int kh, int kw, int sh, int sw, int ph, int pw)
{
    const std::size_t pc = (static_cast<std::size_t>(c) + 15) / 16 * 16;
    const u16* bias = packed;
    const u16* wts = packed + pc;
    const bool s1p1 = kh == 3 && kw == 3 && sh == 1 && sw == 1 && ph == 1 && pw == 1 && oh == ih && ow == iw;
    const bool vec = s1p1 && isa == 0 && c % 8 == 0;
    pool.parallel_for(static_cast<std::size_t>(bn) * oh, 2, [&](std::size_t r0, std::size_t r1) {
        for (std::size_t row = r0; row < r1; ++row) {
            const int b = static_cast<int>(row / static_cast<std::size_t>(oh));
            const int oy = static_cast<int>(row % static_cast<std::size_t>(oh));
            const u16* ib = in + static_cast<std::size_t>(b) * ih * iw * c;
            u16* orow = out + (static_cast<std::size_t>(b) * oh + oy) * ow * c;
            for (int ox = 0; ox < ow; ++ox) {
                u16* op = orow + static_cast<std::size_t>(ox) * c;
                if (vec) {
                    for (int ch = 0; ch < c; ch += 8) {
                        __m256 acc = ld8(bias + ch);
                        for (int ky = 0; ky < 3; ++ky) {
                            const int iy = oy + ky - 1;
                            if (iy < 0 || iy >= ih) continue;
                            for (int kx = 0; kx < 3; ++kx) {
                                const int ix = ox + kx - 1;
                                if (ix < 0 || ix >= iw) continue;
                                acc = _mm256_fmadd_ps(ld8(ib + (static_cast<std::size_t>(iy) * iw + ix) * c + ch),
                                                      ld8(wts + static_cast<std::size_t>(ky * 3 + kx) * pc + ch), acc);
                            }
                        }
                        st8(op + ch, acc);
                    }
                    continue;
                }
                for (int ch = 0; ch < c; ++ch) {
                    float acc = h2f(bias[ch]);
                    for (int ky = 0; ky < kh; ++ky) {
                        const int iy = oy * sh - ph + ky;
                        if (iy < 0 || iy >= ih) continue;
                        for (int kx = 0; kx < kw; ++kx) {
                            const int ix = ox * sw - pw + kx;
                            if (ix < 0 || ix >= iw) continue;
                            const float p = h2f(ib[(static_cast<std::size_t>(iy) * iw + ix) * c + ch]) *
                                            h2f(wts[static_cast<std::size_t>(ky * kw + kx) * pc + ch]);
                            acc = acc + p;
                        }
                    }
                    op[ch] = f2h(acc);
                }
            }
        }
    });
}

void leaky(const u16* in, u16* out, std::size_t count, float alpha, int isa)
{
    std::size_t i = 0;
    if (isa == 0) {
        const __m256 va = _mm256_set1_ps(alpha), z = _mm256_setzero_ps();
        for (; i + 8 <= count; i += 8) {
            const __m256 v = ld8(in + i);
            st8(out + i, _mm256_blendv_ps(v, _mm256_mul_ps(v, va), _mm256_cmp_ps(v, z, _CMP_LT_OQ)));
        }
    }
    for (; i < count; ++i) {
        const float x = h2f(in[i]);
        out[i] = f2h(x < 0.0F ? x * alpha : x);
    }
}

void add(const u16* a, const u16* b, u16* out, std::size_t count, int isa)
{
    std::size_t i = 0;
    if (isa == 0)
        for (; i + 8 <= count; i += 8) st8(out + i, _mm256_add_ps(ld8(a + i), ld8(b + i)));
    for (; i < count; ++i) out[i] = f2h(h2f(a[i]) + h2f(b[i]));
}

void d2s_nhwc(const u16* in, u16* out, int n, int ic, int h, int w, int bs)
{
    const int b2 = bs * bs, oc = ic / b2, ow = w * bs;
    for (int b = 0; b < n; ++b)
        for (int y = 0; y < h; ++y)
            for (int x = 0; x < w; ++x) {
                const u16* ip = in + ((static_cast<std::size_t>(b) * h + y) * w + x) * ic;
                for (int dy = 0; dy < bs; ++dy)
                    for (int dx = 0; dx < bs; ++dx) {
                        u16* op = out + ((static_cast<std::size_t>(b) * h * bs + y * bs + dy) * ow + x * bs + dx) * oc;
                        for (int c = 0; c < oc; ++c) op[c] = ip[c * b2 + dy * bs + dx];
                    }
            }
}

void s2d_nhwc(const u16* in, u16* out, int n, int ic, int h, int w, int bs)
{
    const int b2 = bs * bs, oh = h / bs, ow = w / bs, oc = ic * b2;
    for (int b = 0; b < n; ++b)
        for (int y = 0; y < oh; ++y)
            for (int x = 0; x < ow; ++x) {
                u16* op = out + ((static_cast<std::size_t>(b) * oh + y) * ow + x) * oc;
                for (int dy = 0; dy < bs; ++dy)
                    for (int dx = 0; dx < bs; ++dx) {
                        const u16* ip = in + ((static_cast<std::size_t>(b) * h + y * bs + dy) * w + x * bs + dx) * ic;
                        for (int c = 0; c < ic; ++c) op[c * b2 + dy * bs + dx] = ip[c];
                    }
            }
}

void nchw_to_nhwc(const u16* in, u16* out, std::size_t n, std::size_t c, std::size_t hw)
{
    for (std::size_t b = 0; b < n; ++b)
        for (std::size_t ch = 0; ch < c; ++ch)
            for (std::size_t p = 0; p < hw; ++p) out[(b * hw + p) * c + ch] = in[(b * c + ch) * hw + p];
}

void nhwc_to_nchw(const u16* in, u16* out, std::size_t n, std::size_t hw, std::size_t c)
{
    for (std::size_t b = 0; b < n; ++b)
        for (std::size_t p = 0; p < hw; ++p)
            for (std::size_t ch = 0; ch < c; ++ch) out[(b * c + ch) * hw + p] = in[(b * hw + p) * c + ch];
}

// ------------------------------------- elementwise and layout operators
// UnaryKind / BinaryKind of kernels_common.hpp:34-46.
enum Unary { kUClip = 0, kUSigmoid = 1, kUReciprocal = 2, kURound = 3 };
enum Binary { kBAdd = 0, kBSub = 1, kBMul = 2 };

// MAXPS / MINPS lane semantics (the second operand wins when either is NaN).
inline float maxps(float a, float b) { return a > b ? a : b; }
inline float minps(float a, float b) { return a < b ? a : b; }

// exp of one AVX2 lane, kernels_x86_avx2.cpp:30-55: clamp to
// [-87.33654475, 88.72283905], n = rne(x * log2(e)), r = x - n*ln2 with ln2
// split in two parts (fused steps), a degree-6 Taylor polynomial by Horner
// with fused steps, then times 2^n assembled from exponent bits.
float exp_lane(float x)
{
    x = minps(maxps(x, -87.33654475F), 88.72283905F);
    const float fx = std::nearbyint(x * 1.4426950408889634F);
    const float r = std::fma(-fx, 1.428606765330187E-6F, std::fma(-fx, 0.693145751953125F, x));
    float p = 0.0013888889F;
    p = std::fma(p, r, 0.0083333338F);
    p = std::fma(p, r, 0.0416666679F);
    p = std::fma(p, r, 0.1666666716F);
    p = std::fma(p, r, 0.5F);
    p = std::fma(p, r, 1.0F);
    p = std::fma(p, r, 1.0F);
    const auto bits = static_cast<std::uint32_t>(static_cast<std::int32_t>(fx) + 127) << 23;
    return p * std::bit_cast<float>(bits);
}

// fast_sigmoid_ps_avx2 (kernels_x86_avx2.cpp:57-62) lane-wise, and the
// scalar form used by the scalar kernels and the AVX2 tails.
float sigmoid_lane(float x) { return 1.0F / (1.0F + exp_lane(0.0F - x)); }
float sigmoid_exact(float x) { return 1.0F / (1.0F + std::exp(-x)); }

// scalar_unary (kernels_scalar.cpp:80-97, 244-255) and avx2_unary
// (kernels_x86_avx2.cpp:304-352). The AVX2 path works in lanes of 8 inside
// chunks of 4096 that start at multiples of 4096 (thread_pool.cpp:185-192),
// so only the last count % 8 values take its scalar tail.
void unary(const u16* in, u16* out, std::size_t count, int op, float lo, float hi, int isa)
{
    const std::size_t vec = isa == 0 ? count - count % 8 : 0;
    for (std::size_t i = 0; i < count; ++i) {
        const float x = h2f(in[i]);
        const bool lane = i < vec;
        float r;
        switch (op) {
        case kUClip: r = lane ? maxps(minps(x, hi), lo) : std::min(std::max(x, lo), hi); break;
        case kUSigmoid: r = lane ? sigmoid_lane(x) : sigmoid_exact(x); break;
        case kUReciprocal: r = 1.0F / x; break;
        default: r = std::nearbyint(x); break;
        }
        out[i] = f2h(r);
    }
}

inline float binary_op(float a, float b, int op) { return op == kBSub ? a - b : op == kBMul ? a * b : a + b; }

// binary_contiguous (kernels_scalar.cpp:257-268; the AVX2 lanes compute the
// same single rounding).
void binary_same(const u16* a, const u16* b, u16* out, std::size_t count, int op)
{
    for (std::size_t i = 0; i < count; ++i) out[i] = f2h(binary_op(h2f(a[i]), h2f(b[i]), op));
}

// binary_scalar_bcast (kernels_scalar.cpp:289-302).
void binary_scalar(const u16* vec, u16 scalar, u16* out, std::size_t count, int op, bool scalar_lhs)
{
    const float s = h2f(scalar);
    for (std::size_t i = 0; i < count; ++i) {
        const float v = h2f(vec[i]);
        out[i] = f2h(scalar_lhs ? binary_op(s, v, op) : binary_op(v, s, op));
    }
}

// binary_channel_bcast over an NHWC [spatial, C] operand (kernels_scalar.cpp:270-287).
void binary_channel(const u16* vec, const u16* chan, u16* out, std::size_t spatial, std::size_t c, int op, bool chan_lhs)
{
    for (std::size_t p = 0; p < spatial; ++p)
        for (std::size_t ch = 0; ch < c; ++ch) {
            const float v = h2f(vec[p * c + ch]), k = h2f(chan[ch]);
            out[p * c + ch] = f2h(chan_lhs ? binary_op(k, v, op) : binary_op(v, k, op));
        }
}

// execute_binary_broadcast_fallback_nhwc (execution_plan.cpp:170-236): flat
// modulo indexing when the output is not 4-D; otherwise shapes right-aligned
// to 4-D and every operand indexed as NHWC, size-1 dimensions broadcast.
void binary_broadcast(const u16* a, const std::vector<std::int64_t>& as, const u16* b, const std::vector<std::int64_t>& bs,
                      u16* out, const std::vector<std::int64_t>& os, int op)
{
    auto count = [](const std::vector<std::int64_t>& s) {
        std::size_t n = 1;
        for (auto d : s) n *= static_cast<std::size_t>(d);
        return n;
    };
    if (os.size() != 4) {
        const std::size_t total = count(os), na = count(as), nb = count(bs);
        for (std::size_t i = 0; i < total; ++i)
            out[i] = f2h(binary_op(h2f(a[na == 1 ? 0 : i % na]), h2f(b[nb == 1 ? 0 : i % nb]), op));
        return;
    }
    auto dim4 = [](const std::vector<std::int64_t>& s) {
        std::array<std::size_t, 4> r{1, 1, 1, 1};
        const std::size_t off = 4 - s.size();
        for (std::size_t i = 0; i < s.size(); ++i) r[off + i] = static_cast<std::size_t>(s[i]);
        return r;
    };
    const auto ad = dim4(as), bd = dim4(bs), od = dim4(os);
    for (std::size_t bi = 0; bi < od[0]; ++bi)
        for (std::size_t y = 0; y < od[2]; ++y)
            for (std::size_t x = 0; x < od[3]; ++x) {
                const u16* ap = a + (((ad[0] == 1 ? 0 : bi) * ad[2] + (ad[2] == 1 ? 0 : y)) * ad[3] + (ad[3] == 1 ? 0 : x)) * ad[1];
                const u16* bp = b + (((bd[0] == 1 ? 0 : bi) * bd[2] + (bd[2] == 1 ? 0 : y)) * bd[3] + (bd[3] == 1 ? 0 : x)) * bd[1];
                u16* dst = out + ((bi * od[2] + y) * od[3] + x) * od[1];
                for (std::size_t c = 0; c < od[1]; ++c)
                    dst[c] = f2h(binary_op(h2f(ap[ad[1] == 1 ? 0 : c]), h2f(bp[bd[1] == 1 ? 0 : c]), op));
            }
}

// ADD / SUB / MUL dispatch of the reference plan, execution_plan.cpp:527-563
// (classification) and 958-985 (execution), over NHWC buffers.
void binary_dispatch(const u16* a, const std::vector<std::int64_t>& as, const u16* b, const std::vector<std::int64_t>& bs, u16* o,
                     const std::vector<std::int64_t>& os, int op)
{
    auto count_of = [](const std::vector<std::int64_t>& s) {
        std::size_t n = 1;
        for (auto d : s) n *= static_cast<std::size_t>(d);
        return n;
    };
    // The output must be the broadcast of the operand shapes (the
    // reference reads out of bounds otherwise).
    const std::size_t r = std::max(as.size(), bs.size());
    std::vector<std::int64_t> want(r, 1);
    for (std::size_t i = 0; i < r; ++i) {
        const std::int64_t x = i + as.size() >= r ? as[i + as.size() - r] : 1;
        const std::int64_t y = i + bs.size() >= r ? bs[i + bs.size() - r] : 1;
        if (x != y && x != 1 && y != 1) throw std::runtime_error("oracle: binary operand shapes do not broadcast");
        want[i] = std::max(x, y);
    }
    if (want != os) throw std::runtime_error("oracle: binary output shape is not the broadcast shape");
    const std::size_t count = count_of(os);
    if (as == os && bs == os) {
        binary_same(a, b, o, count, op);
    } else if (count_of(bs) == 1) {
        binary_scalar(a, b[0], o, count, op, false);
    } else if (count_of(as) == 1) {
        binary_scalar(b, a[0], o, count, op, true);
    } else if (os.size() == 4 && as == os && bs == std::vector<std::int64_t>{1, os[1], 1, 1}) {
        binary_channel(a, b, o, static_cast<std::size_t>(os[0] * os[2] * os[3]), static_cast<std::size_t>(os[1]), op, false);
    } else if (os.size() == 4 && bs == os && as == std::vector<std::int64_t>{1, os[1], 1, 1}) {
        binary_channel(b, a, o, static_cast<std::size_t>(os[0] * os[2] * os[3]), static_cast<std::size_t>(os[1]), op, true);
    } else {
        binary_broadcast(a, as, b, bs, o, os, op);
    }
}

// execute_slice_nhwc (kernels_scalar.cpp:830-890): dims, starts and steps
// are logical NCHW, buffers NHWC; its block-copy fast paths give the same
// values as this element loop.
void slice_nhwc(const u16* in, u16* out, const int* id, const int* od, const int* starts, const int* steps)
{
    std::size_t o = 0;
    for (int b = 0; b < od[0]; ++b)
        for (int y = 0; y < od[2]; ++y)
            for (int x = 0; x < od[3]; ++x)
                for (int c = 0; c < od[1]; ++c, ++o) {
                    const std::size_t ib = static_cast<std::size_t>(starts[0] + b * steps[0]);
                    const std::size_t iy = static_cast<std::size_t>(starts[2] + y * steps[2]);
                    const std::size_t ix = static_cast<std::size_t>(starts[3] + x * steps[3]);
                    const std::size_t ic = static_cast<std::size_t>(starts[1] + c * steps[1]);
                    out[o] = in[((ib * id[2] + iy) * id[3] + ix) * id[1] + ic];
                }
}

// execute_concat_nhwc (kernels_scalar.cpp:892-952): inputs placed one after
// another along the logical axis.
void concat_nhwc(const std::vector<const u16*>& ins, const std::vector<std::array<int, 4>>& dims, u16* out,
                 const std::array<int, 4>& od, int axis)
{
    std::array<int, 4> off{0, 0, 0, 0};
    for (std::size_t k = 0; k < ins.size(); ++k) {
        const auto& d = dims[k];
        const u16* in = ins[k];
        for (int b = 0; b < d[0]; ++b)
            for (int y = 0; y < d[2]; ++y)
                for (int x = 0; x < d[3]; ++x) {
                    const u16* src = in + ((static_cast<std::size_t>(b) * d[2] + y) * d[3] + x) * d[1];
                    u16* dst = out + ((static_cast<std::size_t>(b + off[0]) * od[2] + y + off[2]) * od[3] + x + off[3]) * od[1] + off[1];
                    std::memcpy(dst, src, static_cast<std::size_t>(d[1]) * 2);
                }
        off[static_cast<std::size_t>(axis)] += d[static_cast<std::size_t>(axis)];
    }
}

// execute_gather_general (execution_plan.cpp:101-168): 4-D data is indexed
// in its NHWC order (logical axis a -> physical {0, 3, 1, 2}[a]); negative
// indices count from the end; an index outside the axis is an error.
void gather(const u16* data, const std::vector<std::int64_t>& shape, const std::int32_t* idx32, const std::int64_t* idx64,
            std::size_t count, int axis, u16* out)
{
    const int rank = static_cast<int>(shape.size());
    const int ax = axis < 0 ? axis + rank : axis;
    if (ax < 0 || ax >= rank) throw std::runtime_error("oracle: GATHER axis out of range");
    std::vector<std::int64_t> phys = shape;
    int pax = ax;
    if (rank == 4) {
        phys = {shape[0], shape[2], shape[3], shape[1]};
        static constexpr int kMap[4] = {0, 3, 1, 2};
        pax = kMap[ax];
    }
    std::size_t outer = 1, inner = 1;
    for (int d = 0; d < pax; ++d) outer *= static_cast<std::size_t>(phys[static_cast<std::size_t>(d)]);
    for (int d = pax + 1; d < rank; ++d) inner *= static_cast<std::size_t>(phys[static_cast<std::size_t>(d)]);
    const auto dim = static_cast<std::size_t>(phys[static_cast<std::size_t>(pax)]);
    for (std::size_t o = 0; o < outer; ++o)
        for (std::size_t i = 0; i < count; ++i) {
            std::int64_t raw = idx32 ? idx32[i] : idx64[i];
            if (raw < 0) raw += static_cast<std::int64_t>(dim);
            if (raw < 0 || static_cast<std::size_t>(raw) >= dim) throw std::runtime_error("oracle: GATHER index out of range");
            std::memcpy(out + (o * count + i) * inner, data + (o * dim + static_cast<std::size_t>(raw)) * inner, inner * 2);
        }
}

// ------------------------------------------- real-model fused operators
// reglu_nhwc (kernels_scalar.cpp:304-322, kernels_x86_avx2.cpp:443-470):
// out = fp16(fp16(clamp(gate)) * linear), gate = channels [0, G), linear
// [G, 2G) of each pixel. AVX2 lanes clamp as max(min(g, hi), lo).
void reglu(const u16* in, u16* out, std::size_t spatial, std::size_t g, float lo, float hi, int isa)
{
    const std::size_t vec = isa == 0 ? g - g % 8 : 0;
    for (std::size_t p = 0; p < spatial; ++p) {
        const u16* ip = in + p * 2 * g;
        for (std::size_t c = 0; c < g; ++c) {
            const float x = h2f(ip[c]);
            const float cg = h2f(f2h(c < vec ? maxps(minps(x, hi), lo) : std::min(std::max(x, lo), hi)));
            out[p * g + c] = f2h(cg * h2f(ip[c + g]));
        }
    }
}

// feature_update_nhwc / feature_update_outputs_nhwc (kernels_scalar.cpp:
// 324-405, kernels_x86_avx2.cpp:472-583). Per pixel, with input channels
// a | b | c (C each) and the previous feature h:
//   sb = fp16(sigmoid(b)), sc = fp16(sigmoid(c)),
//   blended = fp16(fp16(sb*h) + fp16(fp16(1 - sb)*a)),
//   scaled = fp16(fp16(sc*blended) * scale[ch]).
// `feature` (stride 2C) gets scaled | blended; `scaled_out` / `blended_out`
// (stride C) are optional. AVX2 lanes use the polynomial sigmoid for
// channels below C - C % 8.
void feature_update(const u16* in, const u16* hist, const u16* scale, u16* scaled_out, u16* blended_out, u16* feature,
                    std::size_t spatial, std::size_t ch, int isa)
{
    const std::size_t vec = isa == 0 ? ch - ch % 8 : 0;
    for (std::size_t p = 0; p < spatial; ++p) {
        const u16* ip = in + p * 3 * ch;
        for (std::size_t c = 0; c < ch; ++c) {
            const bool lane = c < vec;
            const float a = h2f(ip[c]), b = h2f(ip[c + ch]), cg = h2f(ip[c + 2 * ch]), prev = h2f(hist[p * ch + c]);
            const float sb = h2f(f2h(lane ? sigmoid_lane(b) : sigmoid_exact(b)));
            const float sc = h2f(f2h(lane ? sigmoid_lane(cg) : sigmoid_exact(cg)));
            const float wb = h2f(f2h(sb * prev));
            const float inv = h2f(f2h(1.0F - sb));
            const float wa = h2f(f2h(inv * a));
            const u16 blended = f2h(wb + wa);
            const float gated = h2f(f2h(sc * h2f(blended)));
            const u16 scaled = f2h(gated * h2f(scale[c]));
            feature[p * 2 * ch + c] = scaled;
            feature[p * 2 * ch + ch + c] = blended;
            if (scaled_out) scaled_out[p * ch + c] = scaled;
            if (blended_out) blended_out[p * ch + c] = blended;
        }
    }
}

// y0_tail_nhwc (kernels_scalar.cpp:407-481, kernels_x86_avx2.cpp:585-656;
// the AVX2 form needs Q % 8 == 0). Channels of one pixel, q = 0..Q-1 and
// its pair q + Q: prior = head (2Q) | tail (2Q).
//   clipped = fp16(max(head, clip_min)), normalized = fp16(latent * fp16(1/clipped)),
//   s = fp16(fp16(normalized - tail) * quant_scale),
//   y_raw[q] = fp16(rne(fp16(s[q] + s[q+Q]))),
//   upd = fp16(fp16(y_raw + tail) * update_scale{0,1}),
//   concat2 = upd (2Q), concat3 = upd | prior (6Q).
void y0_tail(const u16* latent, const u16* prior, const u16* qs, const u16* us0, const u16* us1, u16* normalized,
             u16* clipped, u16* y_raw, u16* concat2, u16* concat3, float clip_min, std::size_t spatial, std::size_t q,
             int isa)
{
    const bool lanes = isa == 0 && q % 8 == 0;
    const std::size_t nc = 2 * q;
    for (std::size_t p = 0; p < spatial; ++p) {
        const u16* pri = prior + p * 4 * q;
        for (std::size_t c = 0; c < q; ++c) {
            float upd[2];
            float s[2];
            float tail[2];
            for (int h = 0; h < 2; ++h) {
                const std::size_t cc = c + static_cast<std::size_t>(h) * q;
                const float head = h2f(pri[cc]);
                const u16 clip = f2h(lanes ? maxps(head, clip_min) : std::max(head, clip_min));
                const float inv = h2f(f2h(1.0F / h2f(clip)));
                const u16 nrm = f2h(h2f(latent[p * nc + cc]) * inv);
                normalized[p * nc + cc] = nrm;
                clipped[p * nc + cc] = clip;
                tail[h] = h2f(pri[cc + nc]);
                const float d = h2f(f2h(h2f(nrm) - tail[h]));
                s[h] = h2f(f2h(d * h2f(qs[p * nc + cc])));
            }
            const float sum = h2f(f2h(s[0] + s[1]));
            const u16 rounded = f2h(std::nearbyint(sum));
            y_raw[p * q + c] = rounded;
            for (int h = 0; h < 2; ++h) {
                const u16* us = h ? us1 : us0;
                const float uin = h2f(f2h(h2f(rounded) + tail[h]));
                upd[h] = h2f(f2h(uin * h2f(us[p * q + c])));
                const std::size_t cc = c + static_cast<std::size_t>(h) * q;
                concat2[p * nc + cc] = f2h(upd[h]);
                concat3[p * 6 * q + cc] = f2h(upd[h]);
            }
        }
        std::memcpy(concat3 + p * 6 * q + nc, pri, 4 * q * 2);
    }
}

// y1_tail_nhwc (kernels_scalar.cpp:483-537, kernels_x86_avx2.cpp:658-712):
//   s = fp16(fp16(normalized - prior) * quant_scale), y_raw as in y0_tail,
//   upd = fp16(fp16(y_raw + prior) * update_scale{0,1}),
//   out = fp16(fp16(concat2 + upd) * clipped).
void y1_tail(const u16* normalized, const u16* prior, const u16* qs, const u16* us0, const u16* us1, const u16* concat2,
             const u16* clipped, u16* y_raw, u16* out, std::size_t spatial, std::size_t q)
{
    const std::size_t nc = 2 * q;
    for (std::size_t p = 0; p < spatial; ++p)
        for (std::size_t c = 0; c < q; ++c) {
            float s[2];
            for (int h = 0; h < 2; ++h) {
                const std::size_t cc = p * nc + c + static_cast<std::size_t>(h) * q;
                const float d = h2f(f2h(h2f(normalized[cc]) - h2f(prior[cc])));
                s[h] = h2f(f2h(d * h2f(qs[cc])));
            }
            const u16 rounded = f2h(std::nearbyint(h2f(f2h(s[0] + s[1]))));
            y_raw[p * q + c] = rounded;
            for (int h = 0; h < 2; ++h) {
                const std::size_t cc = p * nc + c + static_cast<std::size_t>(h) * q;
                const u16* us = h ? us1 : us0;
                const float uin = h2f(f2h(h2f(rounded) + h2f(prior[cc])));
                const float upd = h2f(f2h(uin * h2f(us[p * q + c])));
                const float add = h2f(f2h(h2f(concat2[cc]) + upd));
                out[cc] = f2h(add * h2f(clipped[cc]));
            }
        }
}

// ------------------------------------------------------ graph file parse
// Minimal protobuf reader for mlvc.wire.Graph (proto/mlvc_model.proto:30-83).
struct PbReader {
    const std::uint8_t* p;
    const std::uint8_t* e;
    bool done() const { return p >= e; }
    std::uint64_t varint()
    {
        std::uint64_t v = 0;
        for (int s = 0; s < 70; s += 7) {
            if (p >= e) throw std::runtime_error("oracle: truncated varint");
            const std::uint8_t b = *p++;
            v |= static_cast<std::uint64_t>(b & 0x7F) << s;
            if (!(b & 0x80)) return v;
        }
        throw std::runtime_error("oracle: bad varint");
    }
    PbReader sub()
    {
        const std::uint64_t n = varint();
        if (n > static_cast<std::uint64_t>(e - p)) throw std::runtime_error("oracle: truncated field");
        PbReader r{p, p + n};
        p += n;
        return r;
    }
    void skip(int wt)
    {
        if (wt == 0) varint();
        else if (wt == 1) p += 8;
        else if (wt == 2) sub();
        else if (wt == 5) p += 4;
        else throw std::runtime_error("oracle: bad wire type");
    }
    template <typename T>
    void repeated(int wt, std::vector<T>& out)
    {
        if (wt == 2) {
            PbReader s = sub();
            while (!s.done()) out.push_back(static_cast<T>(s.varint()));
        } else {
            out.push_back(static_cast<T>(varint()));
        }
    }
};

// OpKind, proto/mlvc_model.proto:12-28.
enum Op {
    ADD = 1, SUB = 2, MUL = 3, CLIP = 4, CONCAT = 5, CONV = 6, D2S = 7, GATHER = 8, LEAKY = 9, RECIPROCAL = 10,
    ROUND = 11, SIGMOID = 12, SLICE = 13, S2D = 14
};

struct GTensor {
    std::string name;
    int dtype = 0;
    std::vector<std::int64_t> shape;
    bool weight = false, arena = false;
    std::uint64_t woff = 0, wbytes = 0;
};
struct GNode {
    int op = 0;
    std::vector<std::uint32_t> in, out;
    int attr = 0;
    std::vector<std::uint32_t> strides, pads, dil;
    std::uint32_t groups = 0, block = 0;
    int axis = 0;
    float alpha = 0.01F;
};
struct Graph {
    std::vector<GTensor> t;  // by id
    std::vector<std::uint32_t> inputs, outputs;
    std::vector<GNode> nodes;
};

std::vector<std::uint8_t> read_file(const std::string& path)
{
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("oracle: cannot open " + path);
    return std::vector<std::uint8_t>(std::istreambuf_iterator<char>(f), {});
}

Graph parse_graph(const std::vector<std::uint8_t>& bytes)
{
    Graph g;
    std::vector<std::pair<std::uint32_t, GTensor>> ts;
    PbReader r{bytes.data(), bytes.data() + bytes.size()};
    while (!r.done()) {
        const std::uint64_t tag = r.varint();
        const int f = static_cast<int>(tag >> 3), wt = static_cast<int>(tag & 7);
        if (f == 3 && wt == 2) {
            PbReader s = r.sub();
            std::uint32_t id = 0;
            GTensor t;
            while (!s.done()) {
                const std::uint64_t tg = s.varint();
                const int ff = static_cast<int>(tg >> 3), w = static_cast<int>(tg & 7);
                if (ff == 1 && w == 0) id = static_cast<std::uint32_t>(s.varint());
                else if (ff == 2 && w == 2) { PbReader n = s.sub(); t.name.assign(reinterpret_cast<const char*>(n.p), static_cast<std::size_t>(n.e - n.p)); }
                else if (ff == 3 && w == 0) t.dtype = static_cast<int>(s.varint());
                else if (ff == 4) s.repeated(w, t.shape);
                else if ((ff == 5 || ff == 6) && w == 2) {
                    PbReader a = s.sub();
                    t.arena = ff == 5;
                    t.weight = ff == 6;
                    while (!a.done()) {
                        const std::uint64_t at = a.varint();
                        const std::uint64_t v = a.varint();
                        if (ff == 6 && (at >> 3) == 1) t.woff = v;
                        if (ff == 6 && (at >> 3) == 2) t.wbytes = v;
                    }
                } else s.skip(w);
            }
            ts.emplace_back(id, std::move(t));
        } else if (f == 4) r.repeated(wt, g.inputs);
        else if (f == 5) r.repeated(wt, g.outputs);
        else if (f == 6 && wt == 2) {
            PbReader s = r.sub();
            GNode n;
            while (!s.done()) {
                const std::uint64_t tg = s.varint();
                const int ff = static_cast<int>(tg >> 3), w = static_cast<int>(tg & 7);
                if (ff == 1 && w == 0) n.op = static_cast<int>(s.varint());
                else if (ff == 2) s.repeated(w, n.in);
                else if (ff == 3) s.repeated(w, n.out);
                else if (ff >= 4 && ff <= 7 && w == 2) {
                    n.attr = ff;
                    PbReader a = s.sub();
                    while (!a.done()) {
                        const std::uint64_t at = a.varint();
                        const int af = static_cast<int>(at >> 3), aw = static_cast<int>(at & 7);
                        if (ff == 4 && af == 1) a.repeated(aw, n.strides);
                        else if (ff == 4 && af == 2) a.repeated(aw, n.pads);
                        else if (ff == 4 && af == 3) a.repeated(aw, n.dil);
                        else if (ff == 4 && af == 4) n.groups = static_cast<std::uint32_t>(a.varint());
                        else if (ff == 5 && af == 1) { const auto z = static_cast<std::uint32_t>(a.varint()); n.axis = static_cast<int>((z >> 1) ^ (~(z & 1U) + 1U)); }
                        else if (ff == 6 && af == 1 && aw == 5) { std::uint32_t b; std::memcpy(&b, a.p, 4); a.p += 4; n.alpha = std::bit_cast<float>(b); }
                        else if (ff == 7 && af == 1) n.block = static_cast<std::uint32_t>(a.varint());
                        else a.skip(aw);
                    }
                } else s.skip(w);
            }
            g.nodes.push_back(std::move(n));
        } else r.skip(wt);
    }
    g.t.resize(ts.size() + 1);
    for (auto& [id, t] : ts) {
        if (id == 0 || id >= g.t.size()) throw std::runtime_error("oracle: tensor id out of range");
        g.t[id] = std::move(t);
    }
    return g;
}

std::size_t elems(const std::vector<std::int64_t>& s)
{
    std::size_t n = 1;
    for (auto d : s) n *= static_cast<std::size_t>(d);
    return n;
}

bool needs_nhwc(const GTensor& t)
{
    return t.dtype == 1 && t.shape.size() == 4 && t.shape[1] > 1 && t.shape[2] * t.shape[3] > 1;
}

// ------------------------------------------------------------------ plan
struct ConvInfo {
    bool depthwise = false, is1x1 = false;
    int n = 0, ic = 0, ih = 0, iw = 0, oc = 0, oh = 0, ow = 0, kh = 0, kw = 0, sh = 1, sw = 1, ph = 0, pw = 0;
    std::vector<u16> packed;
    std::vector<std::int32_t> wconv;  // isa 2 only: the packed weights as fp16_q, [16-column block][k][16]
    std::size_t split_c = 0;          // isa 2 only: the GPU's split K (channels per split), 0 when not split
};

// isa 2: the GPU backend's split-K rule (mlvc_hip_conv_plan in
// include/mlvc_hip_device.h), a function of the conv geometry alone: a 1x1
// conv (stride 1, no padding) with K = ic >= 576 and items = n *
// ceil(oc/128) * ceil(oh*ow/128): s = min(8, 512 / items, ic / 64); for
// s > 1 the channels split into ranges of 64 * ceil(ic / (64 s)).
std::size_t gpu_split_channels(const ConvInfo& c)
{
    const bool k1 = c.kh == 1 && c.kw == 1 && c.sh == 1 && c.sw == 1 && c.ph == 0 && c.pw == 0;
    if (!k1 || c.ic < 576) return 0;
    const long long items =
        static_cast<long long>(c.n) * ((c.oc + 127) / 128) * ((static_cast<long long>(c.oh) * c.ow + 127) / 128);
    const long long s = std::min<long long>({8, 512 / items, c.ic / 64});
    if (s <= 1) return 0;
    const long long cs = 64 * ((c.ic + 64 * s - 1) / (64 * s));
    return (c.ic + cs - 1) / cs > 1 ? static_cast<std::size_t>(cs) : 0;
}
// FusedStepKind of fusion_matcher.hpp:12-20.
enum StepKind { kSingle = 0, kConvEpi = 1, kRegluStep = 2, kFeature = 3, kFeatureOutputs = 4, kY0 = 5, kY1 = 6 };
struct Step {
    int kind = kSingle;
    std::size_t node = 0, end = 0;  // nodes [node, end) of the schedule
    Epilogue epi;
    bool reglu_epi = false;  // kConvEpi with the ReGLU epilogue
    std::uint32_t conv_in = 0, residual = 0, out = 0;
    ConvInfo conv;
    float lo = 0.0F, hi = 0.0F;
    std::size_t ch = 0;                // gate / feature / quantised channels
    std::vector<std::uint32_t> ids;    // operands and results of fused kinds
    std::array<int, 4> id4{}, od4{}, starts{}, steps{};  // SLICE
};

class Plan {
public:
    Plan(const std::string& dir, const std::string& model, const std::vector<std::pair<std::size_t, std::size_t>>& bind,
         int threads, int isa, bool fuse)
        : pool_(threads > 0 ? threads : default_threads()), isa_(isa == 2 ? 0 : isa), conv_isa_(isa)
    {
        if (isa < 0 || isa > 2) throw std::runtime_error("oracle: isa must be 0, 1 or 2");
        g_ = parse_graph(read_file(dir + "/aot/" + model + "/graph.pb"));
        weights_ = read_file(dir + "/aot/" + model + "/weights.bin");
        bufs_.resize(g_.t.size());
        state_in_.assign(g_.t.size(), -1);
        state_out_.assign(g_.t.size(), -1);
        for (std::size_t i = 0; i < g_.inputs.size(); ++i) in_pos_[g_.inputs[i]] = i;
        for (auto [ii, oi] : bind) {
            if (ii >= g_.inputs.size() || oi >= g_.outputs.size()) throw std::runtime_error("oracle: state binding index out of range");
            const auto in_id = g_.inputs[ii], out_id = g_.outputs[oi];
            if (state_in_[in_id] >= 0 || state_out_[out_id] >= 0) throw std::runtime_error("oracle: duplicate state tensor binding");
            if (g_.t[in_id].shape != g_.t[out_id].shape || g_.t[in_id].dtype != g_.t[out_id].dtype)
                throw std::runtime_error("oracle: state binding shape or dtype mismatch");
            state_in_[in_id] = state_out_[out_id] = static_cast<int>(bindings_.size());
            bindings_.push_back({in_id, out_id});
        }
        for (std::size_t i = 0; i < g_.inputs.size(); ++i)
            if (state_in_[g_.inputs[i]] < 0) external_.push_back(g_.inputs[i]);
        for (auto o : g_.outputs)
            if (state_out_[o] < 0) ext_out_.push_back(o);
        for (std::size_t id = 1; id < g_.t.size(); ++id) {
            const GTensor& t = g_.t[id];
            if (t.name.empty()) continue;
            // FP16 activations; INT32 graph inputs (q_index_shifted, read by
            // GATHER as indices) are carried as raw bytes.
            const bool int32_input = t.dtype == 2 && in_pos_.count(static_cast<std::uint32_t>(id));
            if (t.dtype != 1 && !t.weight && !int32_input)
                throw std::runtime_error("oracle: only FP16 activations are on this path");
            if (t.dtype == 1) bufs_[id].assign(elems(t.shape), 0);
            if (int32_input) bufs_[id].assign(2 * elems(t.shape), 0);
        }
        for (std::size_t id = 1; id < g_.t.size(); ++id) {
            const GTensor& t = g_.t[id];
            if (!t.weight || t.dtype != 1) continue;
            std::vector<u16> raw(elems(t.shape));
            std::memcpy(raw.data(), weights_.data() + t.woff, raw.size() * 2);
            if (needs_nhwc(t)) nchw_to_nhwc(raw.data(), bufs_[id].data(), static_cast<std::size_t>(t.shape[0]), static_cast<std::size_t>(t.shape[1]), static_cast<std::size_t>(t.shape[2] * t.shape[3]));
            else bufs_[id] = raw;
        }
        for (const GNode& n : g_.nodes) {
            if (n.out.size() != 1) throw std::runtime_error("oracle: every node has one output");
            for (auto id : n.in)
                if (id >= g_.t.size() || (id && g_.t[id].name.empty())) throw std::runtime_error("oracle: node input is not a tensor");
            if (!n.out[0] || n.out[0] >= g_.t.size() || g_.t[n.out[0]].name.empty()) throw std::runtime_error("oracle: node output is not a tensor");
        }
        compile(fuse);
        initialized_ = bindings_.empty();
    }

    int threads() const { return pool_.size(); }
    std::size_t steps() const { return steps_.size(); }
    const std::vector<std::uint32_t>& ext_in() const { return external_; }
    const std::vector<std::uint32_t>& ext_out() const { return ext_out_; }
    const GTensor& tensor(std::uint32_t id) const { return g_.t[id]; }

    void reset()
    {
        for (auto [i, o] : bindings_) {
            std::fill(bufs_[i].begin(), bufs_[i].end(), u16{0});
            std::fill(bufs_[o].begin(), bufs_[o].end(), u16{0});
        }
        initialized_ = true;
    }

    void run(const u16* const* inputs, u16* const* outputs)
    {
        if (!initialized_) throw std::runtime_error("oracle: reset_state() must be called before run()");
        for (std::size_t i = 0; i < external_.size(); ++i) store_io(external_[i], inputs[i]);
        for (const Step& s : steps_) exec(s);
        for (auto [i, o] : bindings_) bufs_[i].swap(bufs_[o]);
        for (std::size_t i = 0; i < ext_out_.size(); ++i) load_io(ext_out_[i], outputs[i]);
    }

private:
    void store_io(std::uint32_t id, const u16* src)
    {
        const GTensor& t = g_.t[id];
        if (needs_nhwc(t)) nchw_to_nhwc(src, bufs_[id].data(), static_cast<std::size_t>(t.shape[0]), static_cast<std::size_t>(t.shape[1]), static_cast<std::size_t>(t.shape[2] * t.shape[3]));
        else std::memcpy(bufs_[id].data(), src, bufs_[id].size() * 2);
    }
    void load_io(std::uint32_t id, u16* dst) const
    {
        const GTensor& t = g_.t[id];
        if (needs_nhwc(t)) nhwc_to_nchw(bufs_[id].data(), dst, static_cast<std::size_t>(t.shape[0]), static_cast<std::size_t>(t.shape[2] * t.shape[3]), static_cast<std::size_t>(t.shape[1]));
        else std::memcpy(dst, bufs_[id].data(), bufs_[id].size() * 2);
    }

    bool is_init(std::uint32_t id) const { return id && id < g_.t.size() && g_.t[id].weight; }

    ConvInfo conv_info(const GNode& n) const
    {
        ConvInfo c;
        const auto& is = g_.t[n.in[0]].shape;
        const auto& ws = g_.t[n.in[1]].shape;
        const auto& os = g_.t[n.out[0]].shape;
        if (is.size() != 4 || ws.size() != 4 || os.size() != 4) throw std::runtime_error("oracle: expected 4D NCHW tensor");
        c.n = static_cast<int>(is[0]); c.ic = static_cast<int>(is[1]); c.ih = static_cast<int>(is[2]); c.iw = static_cast<int>(is[3]);
        c.oc = static_cast<int>(os[1]); c.oh = static_cast<int>(os[2]); c.ow = static_cast<int>(os[3]);
        c.kh = static_cast<int>(ws[2]); c.kw = static_cast<int>(ws[3]);
        c.sh = static_cast<int>(n.strides.at(0)); c.sw = static_cast<int>(n.strides.at(1));
        c.ph = static_cast<int>(n.pads.at(0)); c.pw = static_cast<int>(n.pads.at(1));
        const GTensor& wt = g_.t[n.in[1]];
        std::vector<u16> w(elems(wt.shape));
        std::memcpy(w.data(), weights_.data() + wt.woff, w.size() * 2);
        std::vector<u16> b;
        if (n.in.size() >= 3 && n.in[2]) {
            const GTensor& bt = g_.t[n.in[2]];
            b.resize(elems(bt.shape));
            std::memcpy(b.data(), weights_.data() + bt.woff, b.size() * 2);
            if (static_cast<int>(b.size()) != c.oc) throw std::runtime_error("oracle: conv bias length mismatch");
        }
        const int groups = static_cast<int>(n.groups);
        if (groups == 1) {
            c.is1x1 = c.kh == 1 && c.kw == 1 && c.sh == 1 && c.sw == 1 && c.ph == 0 && c.pw == 0;
            c.packed.resize(packed_conv_elems(static_cast<std::size_t>(c.oc), static_cast<std::size_t>(c.ic), static_cast<std::size_t>(c.kh), static_cast<std::size_t>(c.kw)));
            pack_conv(w.data(), b.empty() ? nullptr : b.data(), static_cast<std::size_t>(c.oc), static_cast<std::size_t>(c.ic), static_cast<std::size_t>(c.kh), static_cast<std::size_t>(c.kw), c.packed.data());
            if (conv_isa_ == 2) {
                c.split_c = gpu_split_channels(c);
                const std::size_t k = static_cast<std::size_t>(c.kh) * c.kw * c.ic, nblk = (static_cast<std::size_t>(c.oc) + 15) / 16;
                c.wconv.resize(nblk * k * 16);
                for (std::size_t bb = 0; bb < nblk; ++bb)
                    for (std::size_t i = 0; i < k * 16; ++i) c.wconv[bb * k * 16 + i] = fp16_q(c.packed[bb * (16 + k * 16) + 16 + i]);
            }
        } else if (groups == c.ic && c.oc == c.ic && ws[1] == 1) {
            c.depthwise = true;
            c.packed.resize(packed_dw_elems(static_cast<std::size_t>(c.ic), static_cast<std::size_t>(c.kh), static_cast<std::size_t>(c.kw)));
            pack_dw(w.data(), b.empty() ? nullptr : b.data(), static_cast<std::size_t>(c.ic), static_cast<std::size_t>(c.kh), static_cast<std::size_t>(c.kw), c.packed.data());
        } else {
            throw std::runtime_error("oracle: general grouped convolution (1 < groups < IC) unsupported");
        }
        return c;
    }

    // fusion_matcher.cpp:230-256 (is_standard_conv) and :352-411.
    bool try_epilogue(std::size_t i, const std::map<std::uint32_t, int>& consumers, Step& s) const
    {
        if (i + 2 > g_.nodes.size()) return false;
        const GNode& c = g_.nodes[i];
        if (c.op != CONV || c.in.size() < 2 || c.out.size() != 1 || c.groups != 1 || c.strides.size() != 2 ||
            c.pads.size() != 4 || c.dil.size() != 2 || c.dil[0] != 1 || c.dil[1] != 1)
            return false;
        const GTensor& w = g_.t[c.in[1]];
        if (!w.weight || w.dtype != 1 || w.shape.size() != 4) return false;
        if (g_.t[c.in[0]].shape.size() != 4 || g_.t[c.out[0]].shape.size() != 4) return false;
        const std::uint32_t co = c.out[0];
        const bool is_output = std::find(g_.outputs.begin(), g_.outputs.end(), co) != g_.outputs.end();
        const auto it = consumers.find(co);
        if (is_output || it == consumers.end() || it->second != 1) return false;
        const GNode& nx = g_.nodes[i + 1];
        s = Step{};
        s.kind = 1;
        s.node = i;
        s.conv_in = c.in[0];
        if (nx.op == LEAKY && nx.in.size() == 1 && nx.in[0] == co && nx.out.size() == 1) {
            s.epi.kind = kLeaky;
            s.epi.alpha = nx.attr == 6 ? nx.alpha : 0.01F;
            s.out = nx.out[0];
            return true;
        }
        if (nx.op == CLIP && nx.in.size() >= 2 && nx.out.size() == 1 && nx.in[0] == co) {
            float lo = -HUGE_VALF, hi = HUGE_VALF;
            auto scalar = [&](std::uint32_t id, float& v) {
                if (!id) return true;
                const GTensor& t = g_.t[id];
                if (!t.weight || t.dtype != 1 || t.wbytes != 2) return false;
                u16 h;
                std::memcpy(&h, weights_.data() + t.woff, 2);
                v = h2f(h);
                return true;
            };
            if (scalar(nx.in[1], lo) && (nx.in.size() < 3 || scalar(nx.in[2], hi))) {
                s.epi.kind = kClamp;
                s.epi.cmin = lo;
                s.epi.cmax = hi;
                s.out = nx.out[0];
                return true;
            }
            return false;
        }
        if (nx.op == ADD && nx.in.size() == 2 && nx.out.size() == 1 && (nx.in[0] == co || nx.in[1] == co)) {
            const std::uint32_t r = nx.in[0] == co ? nx.in[1] : nx.in[0];
            if (r != co && r && !is_init(r) && g_.t[r].dtype == 1 && g_.t[r].shape == g_.t[co].shape) {
                s.epi.kind = kResidual;
                s.residual = r;
                s.out = nx.out[0];
                return true;
            }
        }
        return false;
    }

    // ---- helpers of the fusion matcher (fusion_matcher.cpp:78-256)
    bool is_output(std::uint32_t id) const { return std::find(g_.outputs.begin(), g_.outputs.end(), id) != g_.outputs.end(); }
    bool internal_only(std::uint32_t id, int n) const
    {
        const auto it = consumers_.find(id);
        return id && !is_output(id) && (it == consumers_.end() ? 0 : it->second) == n;
    }
    bool int64_init(std::uint32_t id, std::vector<std::int64_t>& v) const
    {
        if (!is_init(id) || g_.t[id].dtype != 3 || g_.t[id].wbytes % 8) return false;
        v.resize(g_.t[id].wbytes / 8);
        if (!v.empty()) std::memcpy(v.data(), weights_.data() + g_.t[id].woff, g_.t[id].wbytes);
        return true;
    }
    bool fp16_scalar_init(std::uint32_t id, float& v) const
    {
        if (!is_init(id) || g_.t[id].dtype != 1 || g_.t[id].wbytes != 2) return false;
        u16 h;
        std::memcpy(&h, weights_.data() + g_.t[id].woff, 2);
        v = h2f(h);
        return true;
    }
    bool clip_constants(const GNode& n, float& lo, float& hi) const
    {
        if (n.op != CLIP || n.in.size() < 2 || n.out.size() != 1) return false;
        lo = -HUGE_VALF;
        hi = HUGE_VALF;
        if (n.in[1] && !fp16_scalar_init(n.in[1], lo)) return false;
        if (n.in.size() >= 3 && n.in[2] && !fp16_scalar_init(n.in[2], hi)) return false;
        return true;
    }
    bool channel_slice(const GNode& n, std::uint32_t x, std::int64_t b, std::int64_t e) const
    {
        if (n.op != SLICE || n.in.size() < 3 || n.out.size() != 1 || n.in[0] != x) return false;
        std::vector<std::int64_t> st, en, ax, sp;
        if (!int64_init(n.in[1], st) || !int64_init(n.in[2], en) || st.size() != 1 || en.size() != 1 || st[0] != b || en[0] != e)
            return false;
        if (n.in.size() < 4 || !n.in[3] || !int64_init(n.in[3], ax) || ax.size() != 1 || ax[0] != 1) return false;
        if (n.in.size() >= 5 && n.in[4] && (!int64_init(n.in[4], sp) || sp.size() != 1 || sp[0] != 1)) return false;
        const GTensor& o = g_.t[n.out[0]];
        return o.dtype == 1 && o.shape.size() == 4 && o.shape[1] == e - b;
    }
    static bool pair(const GNode& n, int op, std::uint32_t x, std::uint32_t y)
    {
        return n.op == op && n.in.size() == 2 && n.out.size() == 1 &&
               ((n.in[0] == x && n.in[1] == y) || (n.in[0] == y && n.in[1] == x));
    }
    static bool other_in_pair(const GNode& n, int op, std::uint32_t x, std::uint32_t& other)
    {
        if (n.op != op || n.in.size() != 2 || n.out.size() != 1) return false;
        if (n.in[0] == x) { other = n.in[1]; return true; }
        if (n.in[1] == x) { other = n.in[0]; return true; }
        return false;
    }
    bool fp16_of(std::uint32_t id, const std::vector<std::int64_t>& shape) const
    {
        return id && id < g_.t.size() && !g_.t[id].name.empty() && g_.t[id].dtype == 1 && g_.t[id].shape == shape;
    }
    // is_standard_conv (fusion_matcher.cpp:230-256) with require_1x1.
    bool std_1x1_conv(const GNode& c) const
    {
        if (c.op != CONV || c.in.size() < 2 || c.out.size() != 1 || c.groups != 1 || c.strides.size() != 2 ||
            c.pads.size() != 4 || c.dil.size() != 2 || c.dil[0] != 1 || c.dil[1] != 1)
            return false;
        const GTensor& w = g_.t[c.in[1]];
        if (!w.weight || w.dtype != 1 || w.shape.size() != 4) return false;
        if (g_.t[c.in[0]].dtype != 1 || g_.t[c.in[0]].shape.size() != 4 || g_.t[c.out[0]].dtype != 1 || g_.t[c.out[0]].shape.size() != 4)
            return false;
        return w.shape[2] == 1 && w.shape[3] == 1 && c.strides[0] == 1 && c.strides[1] == 1 && c.pads[0] == 0 && c.pads[1] == 0 &&
               c.pads[2] == 0 && c.pads[3] == 0;
    }

    // try_pointwise_reglu (fusion_matcher.cpp:258-302): 1x1 conv (2G
    // outputs) -> SLICE [0,G) / [G,2G) -> CLIP(gate) -> MUL(clipped, linear).
    bool try_conv_reglu(std::size_t i, Step& s) const
    {
        const auto& ns = g_.nodes;
        if (i + 5 > ns.size() || !std_1x1_conv(ns[i])) return false;
        const std::uint32_t co = ns[i].out[0];
        if (!internal_only(co, 2)) return false;
        const auto& cs = g_.t[co].shape;
        if (cs[1] <= 0 || cs[1] % 2) return false;
        const std::int64_t g = cs[1] / 2;
        if (!channel_slice(ns[i + 1], co, 0, g) || !channel_slice(ns[i + 2], co, g, 2 * g)) return false;
        const std::uint32_t gate = ns[i + 1].out[0], lin = ns[i + 2].out[0];
        if (!internal_only(gate, 1) || !internal_only(lin, 1)) return false;
        float lo, hi;
        if (!clip_constants(ns[i + 3], lo, hi) || ns[i + 3].in[0] != gate) return false;
        const std::uint32_t clipped = ns[i + 3].out[0];
        if (!internal_only(clipped, 1) || !pair(ns[i + 4], MUL, clipped, lin)) return false;
        s = Step{};
        s.kind = kConvEpi;
        s.reglu_epi = true;
        s.node = i;
        s.end = i + 5;
        s.lo = lo;
        s.hi = hi;
        s.conv_in = ns[i].in[0];
        s.out = ns[i + 4].out[0];
        s.ch = static_cast<std::size_t>(g);
        return true;
    }

    // try_reglu (fusion_matcher.cpp:304-346).
    bool try_reglu(std::size_t i, Step& s) const
    {
        const auto& ns = g_.nodes;
        if (i + 4 > ns.size() || ns[i].op != SLICE || ns[i].in.empty()) return false;
        const std::uint32_t x = ns[i].in[0];
        const GTensor& t = g_.t[x];
        if (t.name.empty() || t.dtype != 1 || t.shape.size() != 4 || t.shape[1] <= 0 || t.shape[1] % 2) return false;
        const std::int64_t g = t.shape[1] / 2;
        if (!channel_slice(ns[i], x, 0, g) || !channel_slice(ns[i + 1], x, g, 2 * g)) return false;
        const std::uint32_t gate = ns[i].out[0], lin = ns[i + 1].out[0];
        if (!internal_only(gate, 1) || !internal_only(lin, 1)) return false;
        float lo, hi;
        if (!clip_constants(ns[i + 2], lo, hi) || ns[i + 2].in[0] != gate) return false;
        const std::uint32_t clipped = ns[i + 2].out[0];
        if (!internal_only(clipped, 1) || !pair(ns[i + 3], MUL, clipped, lin)) return false;
        s = Step{};
        s.kind = kRegluStep;
        s.node = i;
        s.end = i + 4;
        s.lo = lo;
        s.hi = hi;
        s.ids = {x};
        s.out = ns[i + 3].out[0];
        s.ch = static_cast<std::size_t>(g);
        return true;
    }

    // try_feature_update (fusion_matcher.cpp:413-541): three channel slices
    // a | b | c, two SIGMOIDs, w_b = sb*h, inv = 1 - sb, w_a = inv*a,
    // blended = w_b + w_a, gated = sc*blended, scaled = gated*scale[1,C,1,1],
    // then CONCAT(scaled, blended) right after (one output) or further down
    // (three outputs; the CONCAT node is then skipped).
    bool try_feature(std::size_t i, std::vector<bool>& elided, Step& s) const
    {
        const auto& ns = g_.nodes;
        if (i + 11 > ns.size() || ns[i].op != SLICE || ns[i].in.empty()) return false;
        const std::uint32_t x = ns[i].in[0];
        const GTensor& t = g_.t[x];
        if (t.name.empty() || t.dtype != 1 || t.shape.size() != 4 || t.shape[1] <= 0 || t.shape[1] % 3) return false;
        const std::int64_t ch = t.shape[1] / 3;
        if (!channel_slice(ns[i], x, 0, ch) || !channel_slice(ns[i + 1], x, ch, 2 * ch) || !channel_slice(ns[i + 2], x, 2 * ch, 3 * ch))
            return false;
        const std::uint32_t a = ns[i].out[0], b = ns[i + 1].out[0], cg = ns[i + 2].out[0];
        if (!internal_only(a, 1) || !internal_only(b, 1) || !internal_only(cg, 1)) return false;
        const GNode& s0 = ns[i + 3];
        const GNode& s1 = ns[i + 4];
        if (s0.op != SIGMOID || s0.in.size() != 1 || s0.in[0] != b || s0.out.size() != 1 || s1.op != SIGMOID ||
            s1.in.size() != 1 || s1.in[0] != cg || s1.out.size() != 1)
            return false;
        const std::uint32_t sb = s0.out[0], sc = s1.out[0];
        if (!internal_only(sb, 2) || !internal_only(sc, 1)) return false;
        std::uint32_t hist = 0;
        if (!other_in_pair(ns[i + 5], MUL, sb, hist)) return false;
        if (is_init(hist) || !fp16_of(hist, g_.t[a].shape)) return false;
        const std::uint32_t wb = ns[i + 5].out[0];
        if (!internal_only(wb, 1)) return false;
        const GNode& sub = ns[i + 6];
        if (sub.op != SUB || sub.in.size() != 2 || sub.out.size() != 1 || sub.in[1] != sb) return false;
        float one = 0.0F;
        if (!fp16_scalar_init(sub.in[0], one) || std::fabs(one - 1.0F) > 1e-4F) return false;
        const std::uint32_t inv = sub.out[0];
        if (!internal_only(inv, 1) || !pair(ns[i + 7], MUL, inv, a)) return false;
        const std::uint32_t wa = ns[i + 7].out[0];
        if (!internal_only(wa, 1) || !pair(ns[i + 8], ADD, wb, wa)) return false;
        const std::uint32_t blended = ns[i + 8].out[0];
        if (!pair(ns[i + 9], MUL, sc, blended)) return false;
        const std::uint32_t gated = ns[i + 9].out[0];
        if (!internal_only(gated, 1)) return false;
        std::uint32_t scale = 0;
        if (!other_in_pair(ns[i + 10], MUL, gated, scale)) return false;
        if (!fp16_of(scale, {1, ch, 1, 1})) return false;
        const std::uint32_t scaled = ns[i + 10].out[0];
        auto concat_of = [&](const GNode& c) {
            const int ax = c.attr == 5 ? c.axis : 0;
            return c.op == CONCAT && ax == 1 && c.in.size() == 2 && c.in[0] == scaled && c.in[1] == blended && c.out.size() == 1;
        };
        if (i + 12 <= ns.size() && internal_only(scaled, 1) && internal_only(blended, 2) && concat_of(ns[i + 11])) {
            s = Step{};
            s.kind = kFeature;
            s.node = i;
            s.end = i + 12;
            s.ids = {x, hist, scale};
            s.out = ns[i + 11].out[0];
            s.ch = static_cast<std::size_t>(ch);
            return true;
        }
        if (!is_output(scaled) && internal_only(blended, 2)) {
            for (std::size_t j = i + 11; j < ns.size(); ++j) {
                if (!concat_of(ns[j])) continue;
                elided[j] = true;
                s = Step{};
                s.kind = kFeatureOutputs;
                s.node = i;
                s.end = i + 11;
                s.ids = {x, hist, scale, scaled, blended};
                s.out = ns[j].out[0];
                s.ch = static_cast<std::size_t>(ch);
                return true;
            }
        }
        return false;
    }

    // The update part shared by both quantisation tails
    // (fusion_matcher.cpp:620-697 and 760-836), starting at node k with
    // `scaled` = fp16((normalized - tail) * quant_scale) already matched:
    // two half slices, ADD, ROUND, two tail slices, (y_raw + tail_h) *
    // update_scale_h. Returns the first node after it, or 0.
    std::size_t match_update(std::size_t k, std::uint32_t scaled, std::uint32_t tail, std::int64_t q,
                             const std::vector<std::int64_t>& qshape, std::uint32_t& y_raw, std::uint32_t& u0,
                             std::uint32_t& u1, std::uint32_t& us0, std::uint32_t& us1) const
    {
        const auto& ns = g_.nodes;
        if (!channel_slice(ns[k], scaled, 0, q) || !channel_slice(ns[k + 1], scaled, q, 2 * q)) return 0;
        const std::uint32_t h0 = ns[k].out[0], h1 = ns[k + 1].out[0];
        if (!internal_only(h0, 1) || !internal_only(h1, 1) || !pair(ns[k + 2], ADD, h0, h1)) return 0;
        const std::uint32_t sum = ns[k + 2].out[0];
        if (!internal_only(sum, 1)) return 0;
        const GNode& rnd = ns[k + 3];
        if (rnd.op != ROUND || rnd.in.size() != 1 || rnd.in[0] != sum || rnd.out.size() != 1) return 0;
        y_raw = rnd.out[0];
        if (!channel_slice(ns[k + 4], tail, 0, q) || !channel_slice(ns[k + 5], tail, q, 2 * q)) return 0;
        const std::uint32_t t0 = ns[k + 4].out[0], t1 = ns[k + 5].out[0];
        if (!internal_only(t0, 1) || !internal_only(t1, 1)) return 0;
        if (!pair(ns[k + 6], ADD, y_raw, t0)) return 0;
        const std::uint32_t a0 = ns[k + 6].out[0];
        if (!internal_only(a0, 1) || !other_in_pair(ns[k + 7], MUL, a0, us0) || !fp16_of(us0, qshape)) return 0;
        u0 = ns[k + 7].out[0];
        if (!internal_only(u0, 1) || !pair(ns[k + 8], ADD, y_raw, t1)) return 0;
        const std::uint32_t a1 = ns[k + 8].out[0];
        if (!internal_only(a1, 1) || !other_in_pair(ns[k + 9], MUL, a1, us1) || !fp16_of(us1, qshape)) return 0;
        u1 = ns[k + 9].out[0];
        if (!internal_only(u1, 1)) return 0;
        return k + 10;
    }

    // try_y0_tail (fusion_matcher.cpp:543-696).
    bool try_y0(std::size_t i, Step& s) const
    {
        const auto& ns = g_.nodes;
        if (i + 19 > ns.size() || ns[i].op != SLICE || ns[i].in.empty()) return false;
        const std::uint32_t prior = ns[i].in[0];
        const GTensor& pt = g_.t[prior];
        if (pt.name.empty() || pt.dtype != 1 || pt.shape.size() != 4 || pt.shape[1] <= 0 || pt.shape[1] % 4) return false;
        const std::int64_t q = pt.shape[1] / 4;
        if (!channel_slice(ns[i], prior, 0, 2 * q) || !channel_slice(ns[i + 1], prior, 2 * q, 4 * q)) return false;
        const std::uint32_t head = ns[i].out[0], tail = ns[i + 1].out[0];
        if (!internal_only(head, 1) || !internal_only(tail, 3)) return false;
        float lo, hi;
        if (!clip_constants(ns[i + 2], lo, hi) || ns[i + 2].in[0] != head || hi < 65504.0F) return false;
        const std::uint32_t clipped = ns[i + 2].out[0];
        if (is_output(clipped)) return false;
        const GNode& rec = ns[i + 3];
        if (rec.op != RECIPROCAL || rec.in.size() != 1 || rec.in[0] != clipped || rec.out.size() != 1) return false;
        std::uint32_t inv = rec.out[0];
        if (!internal_only(inv, 1)) return false;
        std::size_t k = i + 4;
        if (k + 15 <= ns.size() && ns[k].op == MUL && ns[k].in.size() == 2 && ns[k].out.size() == 1) {
            std::uint32_t other = 0;
            float one = 0.0F;
            if (other_in_pair(ns[k], MUL, inv, other) && fp16_scalar_init(other, one) && std::fabs(one - 1.0F) <= 1e-4F) {
                inv = ns[k].out[0];
                if (!internal_only(inv, 1)) return false;
                ++k;
            }
        }
        if (k + 15 > ns.size()) return false;
        const std::vector<std::int64_t> nshape{pt.shape[0], 2 * q, pt.shape[2], pt.shape[3]};
        const std::vector<std::int64_t> qshape{pt.shape[0], q, pt.shape[2], pt.shape[3]};
        std::uint32_t latent = 0;
        if (!other_in_pair(ns[k], MUL, inv, latent) || is_init(latent) || !fp16_of(latent, nshape)) return false;
        const std::uint32_t normalized = ns[k].out[0];
        const GNode& sub = ns[k + 1];
        if (sub.op != SUB || sub.in.size() != 2 || sub.out.size() != 1 || sub.in[0] != normalized || sub.in[1] != tail) return false;
        const std::uint32_t diff = sub.out[0];
        std::uint32_t qs = 0;
        if (!internal_only(diff, 1) || !other_in_pair(ns[k + 2], MUL, diff, qs) || !fp16_of(qs, nshape)) return false;
        const std::uint32_t scaled = ns[k + 2].out[0];
        if (!internal_only(scaled, 2)) return false;
        std::uint32_t y_raw, u0, u1, us0, us1;
        const std::size_t e = match_update(k + 3, scaled, tail, q, qshape, y_raw, u0, u1, us0, us1);
        if (!e) return false;
        const GNode& c2 = ns[e];
        const GNode& c3 = ns[e + 1];
        auto axis1 = [](const GNode& c) { return (c.attr == 5 ? c.axis : 0) == 1; };
        if (c2.op != CONCAT || !axis1(c2) || c2.in.size() != 2 || c2.in[0] != u0 || c2.in[1] != u1 || c2.out.size() != 1) return false;
        const std::uint32_t concat2 = c2.out[0];
        if (c3.op != CONCAT || !axis1(c3) || c3.in.size() != 2 || c3.in[0] != concat2 || c3.in[1] != prior || c3.out.size() != 1)
            return false;
        s = Step{};
        s.kind = kY0;
        s.node = i;
        s.end = e + 2;
        s.ids = {latent, prior, qs, us0, us1, normalized, clipped, y_raw, concat2, c3.out[0]};
        s.out = c3.out[0];
        s.lo = lo;
        s.ch = static_cast<std::size_t>(q);
        return true;
    }

    // try_y1_tail (fusion_matcher.cpp:698-850).
    bool try_y1(std::size_t i, Step& s) const
    {
        const auto& ns = g_.nodes;
        if (i + 15 > ns.size()) return false;
        const GNode& sub = ns[i];
        if (sub.op != SUB || sub.in.size() != 2 || sub.out.size() != 1) return false;
        const std::uint32_t normalized = sub.in[0], prior = sub.in[1];
        const GTensor& nt = g_.t[normalized];
        const GTensor& pt = g_.t[prior];
        if (!normalized || !prior || nt.name.empty() || pt.name.empty() || nt.dtype != 1 || pt.dtype != 1 || nt.shape.size() != 4 ||
            nt.shape != pt.shape || nt.shape[1] <= 0 || nt.shape[1] % 2)
            return false;
        const std::int64_t q = nt.shape[1] / 2;
        const std::vector<std::int64_t> qshape{nt.shape[0], q, nt.shape[2], nt.shape[3]};
        const std::uint32_t diff = sub.out[0];
        std::uint32_t qs = 0;
        if (!internal_only(diff, 1) || !other_in_pair(ns[i + 1], MUL, diff, qs) || !fp16_of(qs, nt.shape)) return false;
        const std::uint32_t scaled = ns[i + 1].out[0];
        if (!internal_only(scaled, 2)) return false;
        std::uint32_t y_raw, u0, u1, us0, us1;
        const std::size_t e = match_update(i + 2, scaled, prior, q, qshape, y_raw, u0, u1, us0, us1);
        if (!e) return false;
        const GNode& c2 = ns[e];
        if (c2.op != CONCAT || (c2.attr == 5 ? c2.axis : 0) != 1 || c2.in.size() != 2 || c2.in[0] != u0 || c2.in[1] != u1 ||
            c2.out.size() != 1)
            return false;
        const std::uint32_t cat = c2.out[0];
        std::uint32_t concat2 = 0, clipped = 0;
        if (!internal_only(cat, 1) || !other_in_pair(ns[e + 1], ADD, cat, concat2) || is_init(concat2) || !fp16_of(concat2, nt.shape))
            return false;
        const std::uint32_t added = ns[e + 1].out[0];
        if (!internal_only(added, 1) || !other_in_pair(ns[e + 2], MUL, added, clipped) || is_init(clipped) ||
            !fp16_of(clipped, nt.shape))
            return false;
        s = Step{};
        s.kind = kY1;
        s.node = i;
        s.end = e + 3;
        s.ids = {normalized, prior, qs, us0, us1, concat2, clipped, y_raw, ns[e + 2].out[0]};
        s.out = ns[e + 2].out[0];
        s.ch = static_cast<std::size_t>(q);
        return true;
    }

    static std::array<int, 4> dims4(const std::vector<std::int64_t>& s)
    {
        if (s.size() != 4) throw std::runtime_error("oracle: expected 4D NCHW tensor");
        std::array<int, 4> d{};
        for (std::size_t i = 0; i < 4; ++i) {
            if (s[i] <= 0 || s[i] > 0x7FFFFFFF) throw std::runtime_error("oracle: tensor dimension out of int range");
            d[i] = static_cast<int>(s[i]);
        }
        return d;
    }

    // SLICE parameters (execution_plan.cpp:565-604): starts (negative ones
    // count from the end, clamped to [0, dim]) and steps per axis; the
    // output shape gives the extent, `ends` is not read.
    void compile_slice(const GNode& n, Step& s) const
    {
        const GTensor& in = g_.t[n.in.at(0)];
        s.id4 = dims4(in.shape);
        s.od4 = dims4(g_.t[n.out.at(0)].shape);
        s.starts = {0, 0, 0, 0};
        s.steps = {1, 1, 1, 1};
        std::vector<std::int64_t> st, en, ax, sp;
        if (n.in.size() < 3 || !int64_init(n.in[1], st) || !int64_init(n.in[2], en))
            throw std::runtime_error("oracle: SLICE starts/ends must be INT64 initializers");
        if (n.in.size() > 3 && n.in[3]) {
            if (!int64_init(n.in[3], ax)) throw std::runtime_error("oracle: SLICE axes must be an INT64 initializer");
        } else {
            for (std::size_t a = 0; a < st.size(); ++a) ax.push_back(static_cast<std::int64_t>(a));
        }
        sp.assign(st.size(), 1);
        if (n.in.size() > 4 && n.in[4] && !int64_init(n.in[4], sp)) throw std::runtime_error("oracle: SLICE steps must be an INT64 initializer");
        if (ax.size() < st.size() || sp.size() < st.size()) throw std::runtime_error("oracle: SLICE parameter lengths differ");
        for (std::size_t a = 0; a < st.size(); ++a) {
            int x = static_cast<int>(ax[a]);
            if (x < 0) x += 4;
            if (x < 0 || x >= 4) throw std::runtime_error("oracle: SLICE axis out of range");
            const std::int64_t dim = in.shape[static_cast<std::size_t>(x)];
            std::int64_t v = st[a];
            if (v < 0) v += dim;
            v = std::clamp<std::int64_t>(v, 0, dim);
            s.starts[static_cast<std::size_t>(x)] = static_cast<int>(v);
            s.steps[static_cast<std::size_t>(x)] = static_cast<int>(sp[a]);
        }
        // Every element read must lie inside the input (the reference does
        // not check; an out-of-range read is undefined there).
        for (std::size_t d = 0; d < 4; ++d) {
            const std::int64_t last = s.starts[d] + static_cast<std::int64_t>(s.od4[d] - 1) * s.steps[d];
            if (s.starts[d] >= s.id4[d] || last < 0 || last >= s.id4[d]) throw std::runtime_error("oracle: SLICE reads outside its input");
        }
    }

    void compile(bool fuse)
    {
        consumers_.clear();
        for (const GNode& n : g_.nodes)
            for (auto id : n.in)
                if (id) ++consumers_[id];
        std::vector<bool> elided(g_.nodes.size(), false);
        for (std::size_t i = 0; i < g_.nodes.size();) {
            if (elided[i]) {
                ++i;
                continue;
            }
            Step s;
            // build_fused_schedule's order (fusion_matcher.cpp:50-72).
            if (fuse && (try_y0(i, s) || try_y1(i, s) || try_feature(i, elided, s) || try_conv_reglu(i, s) || try_reglu(i, s) ||
                         try_epilogue(i, consumers_, s))) {
                if (s.kind == kConvEpi) s.conv = conv_info(g_.nodes[i]);
                if (s.end == 0) s.end = i + 2;
                i = s.end;
                steps_.push_back(std::move(s));
                continue;
            }
            s = Step{};
            s.node = i;
            s.end = i + 1;
            const GNode& n = g_.nodes[i];
            switch (n.op) {
            case CONV: s.conv = conv_info(n); break;
            case SLICE: compile_slice(n, s); break;
            case CLIP:
                s.lo = -HUGE_VALF;
                s.hi = HUGE_VALF;
                if (n.in.size() > 1 && n.in[1] && !fp16_scalar_init(n.in[1], s.lo)) throw std::runtime_error("oracle: expected scalar FP16 initializer");
                if (n.in.size() > 2 && n.in[2] && !fp16_scalar_init(n.in[2], s.hi)) throw std::runtime_error("oracle: expected scalar FP16 initializer");
                break;
            case LEAKY: case ADD: case SUB: case MUL: case D2S: case S2D: case CONCAT: case GATHER: case SIGMOID: case RECIPROCAL:
            case ROUND:
                break;
            default: throw std::runtime_error("oracle: unsupported AOT operator: " + std::to_string(n.op));
            }
            s.out = n.out.at(0);
            steps_.push_back(std::move(s));
            ++i;
        }
    }

    void run_conv(const ConvInfo& c, std::uint32_t in, std::uint32_t out, Epilogue e)
    {
        run_conv_ptr(c, bufs_[in].data(), bufs_[out].data(), e);
    }

    void run_conv_ptr(const ConvInfo& c, const u16* ip, u16* op, Epilogue e)
    {
        const std::size_t split = c.split_c;
        if (c.depthwise) {
            depthwise_nhwc(pool_, isa_, ip, c.packed.data(), op, c.n, c.ic, c.ih, c.iw, c.oh, c.ow, c.kh, c.kw, c.sh, c.sw, c.ph, c.pw);
        } else if (c.is1x1) {
            gemm_nhwc(pool_, conv_isa_, static_cast<std::size_t>(c.n) * c.oh * c.ow, static_cast<std::size_t>(c.oc), static_cast<std::size_t>(c.ic), ip, c.packed.data(), op, e,
                      c.wconv.empty() ? nullptr : c.wconv.data(), split);
        } else {
            spatial_conv_nhwc(pool_, conv_isa_, ip, c.packed.data(), op, c.n, c.ic, c.ih, c.iw, c.oc, c.oh, c.ow, c.kh, c.kw, c.sh, c.sw, c.ph, c.pw, e,
                              c.wconv.empty() ? nullptr : c.wconv.data(), split);
        }
    }

    static std::size_t spatial_of(const std::vector<std::int64_t>& shape)
    {
        const auto d = dims4(shape);
        return static_cast<std::size_t>(d[0]) * d[2] * d[3];
    }

    void exec_binary(const GNode& n, u16* o)
    {
        const int op = n.op == SUB ? kBSub : n.op == MUL ? kBMul : kBAdd;
        binary_dispatch(bufs_[n.in.at(0)].data(), g_.t[n.in[0]].shape, bufs_[n.in.at(1)].data(), g_.t[n.in[1]].shape, o,
                        g_.t[n.out[0]].shape, op);
    }

    // execute_gather_general call site, execution_plan.cpp:1004-1012: INT32
    // indices (a graph input such as q_index_shifted) or INT64 initializers.
    void exec_gather(const GNode& n, u16* o)
    {
        const std::uint32_t d = n.in.at(0), ix = n.in.at(1);
        const GTensor& it = g_.t[ix];
        const std::size_t count = elems(it.shape);
        std::vector<std::int64_t> i64;
        const std::int32_t* i32 = nullptr;
        if (it.dtype == 2 && !it.weight) {
            i32 = reinterpret_cast<const std::int32_t*>(bufs_[ix].data());
        } else if (!int64_init(ix, i64)) {
            throw std::runtime_error("oracle: GATHER indices must be INT32 graph inputs or INT64 initializers");
        }
        const auto& ds = g_.t[d].shape;
        const int rank = static_cast<int>(ds.size());
        const int ax = n.axis < 0 ? n.axis + rank : n.axis;
        if (ax < 0 || ax >= rank) throw std::runtime_error("oracle: GATHER axis out of range");
        if (elems(ds) / static_cast<std::size_t>(ds[static_cast<std::size_t>(ax)]) * count != bufs_[n.out[0]].size())
            throw std::runtime_error("oracle: GATHER output size mismatch");
        gather(bufs_[d].data(), ds, i32, i32 ? nullptr : i64.data(), count, n.axis, o);
    }

    void exec(const Step& s)
    {
        switch (s.kind) {
        case kConvEpi:
            if (s.reglu_epi) {
                // The GEMM writes the rounded 2G-channel conv output, then the
                // ReGLU post-pass (kernels_x86_avx2.cpp:216-233, kernels_scalar.cpp:121-152).
                const auto& cs = g_.t[g_.nodes[s.node].out[0]].shape;
                std::vector<u16> tmp(elems(cs));
                run_conv_ptr(s.conv, bufs_[s.conv_in].data(), tmp.data(), Epilogue{});
                reglu(tmp.data(), bufs_[s.out].data(), spatial_of(cs), s.ch, s.lo, s.hi, isa_);
            } else {
                Epilogue e = s.epi;
                if (s.residual) e.residual = bufs_[s.residual].data();
                run_conv(s.conv, s.conv_in, s.out, e);
            }
            return;
        case kRegluStep:
            reglu(bufs_[s.ids[0]].data(), bufs_[s.out].data(), spatial_of(g_.t[s.out].shape), s.ch, s.lo, s.hi, isa_);
            return;
        case kFeature:
        case kFeatureOutputs: {
            const bool three = s.kind == kFeatureOutputs;
            feature_update(bufs_[s.ids[0]].data(), bufs_[s.ids[1]].data(), bufs_[s.ids[2]].data(),
                           three ? bufs_[s.ids[3]].data() : nullptr, three ? bufs_[s.ids[4]].data() : nullptr, bufs_[s.out].data(),
                           spatial_of(g_.t[s.ids[1]].shape), s.ch, isa_);
            return;
        }
        case kY0: {
            auto p = [&](int k) { return bufs_[s.ids[static_cast<std::size_t>(k)]].data(); };
            y0_tail(p(0), p(1), p(2), p(3), p(4), p(5), p(6), p(7), p(8), p(9), s.lo, spatial_of(g_.t[s.ids[7]].shape), s.ch, isa_);
            return;
        }
        case kY1: {
            auto p = [&](int k) { return bufs_[s.ids[static_cast<std::size_t>(k)]].data(); };
            y1_tail(p(0), p(1), p(2), p(3), p(4), p(5), p(6), p(7), p(8), spatial_of(g_.t[s.ids[7]].shape), s.ch);
            return;
        }
        default: break;
        }
        const GNode& n = g_.nodes[s.node];
        const GTensor& ot = g_.t[s.out];
        u16* o = bufs_[s.out].data();
        switch (n.op) {
        case CONV: run_conv(s.conv, n.in[0], s.out, Epilogue{}); break;
        case LEAKY: leaky(bufs_[n.in[0]].data(), o, bufs_[s.out].size(), n.attr == 6 ? n.alpha : 0.01F, isa_); break;
        case ADD: case SUB: case MUL: exec_binary(n, o); break;
        case CLIP: unary(bufs_[n.in[0]].data(), o, bufs_[s.out].size(), kUClip, s.lo, s.hi, isa_); break;
        case SIGMOID: unary(bufs_[n.in[0]].data(), o, bufs_[s.out].size(), kUSigmoid, 0.0F, 0.0F, isa_); break;
        case RECIPROCAL: unary(bufs_[n.in[0]].data(), o, bufs_[s.out].size(), kUReciprocal, 0.0F, 0.0F, isa_); break;
        case ROUND: unary(bufs_[n.in[0]].data(), o, bufs_[s.out].size(), kURound, 0.0F, 0.0F, isa_); break;
        case SLICE: slice_nhwc(bufs_[n.in[0]].data(), o, s.id4.data(), s.od4.data(), s.starts.data(), s.steps.data()); break;
        case GATHER: exec_gather(n, o); break;
        case D2S: {
            const auto& is = g_.t[n.in[0]].shape;
            d2s_nhwc(bufs_[n.in[0]].data(), o, static_cast<int>(is[0]), static_cast<int>(is[1]), static_cast<int>(is[2]), static_cast<int>(is[3]), static_cast<int>(n.block));
            break;
        }
        case S2D: {
            const auto& is = g_.t[n.in[0]].shape;
            s2d_nhwc(bufs_[n.in[0]].data(), o, static_cast<int>(is[0]), static_cast<int>(is[1]), static_cast<int>(is[2]), static_cast<int>(is[3]), static_cast<int>(n.block));
            break;
        }
        case CONCAT: {
            // execution_plan.cpp:606-620, 993-1002: 4-D inputs along any axis.
            const int axis = n.axis < 0 ? n.axis + 4 : n.axis;
            if (axis < 0 || axis >= 4) throw std::runtime_error("oracle: CONCAT axis out of range");
            const auto od = dims4(ot.shape);
            std::vector<const u16*> ins;
            std::vector<std::array<int, 4>> dims;
            int along = 0;
            for (auto id : n.in) {
                dims.push_back(dims4(g_.t[id].shape));
                for (int d = 0; d < 4; ++d)
                    if (d != axis && dims.back()[static_cast<std::size_t>(d)] != od[static_cast<std::size_t>(d)])
                        throw std::runtime_error("oracle: CONCAT input shape mismatch");
                along += dims.back()[static_cast<std::size_t>(axis)];
                ins.push_back(bufs_[id].data());
            }
            if (along != od[static_cast<std::size_t>(axis)]) throw std::runtime_error("oracle: CONCAT output shape mismatch");
            concat_nhwc(ins, dims, o, od, axis);
            break;
        }
        default: throw std::runtime_error("oracle: unsupported operator during execution");
        }
    }

    Pool pool_;
    int isa_;
    int conv_isa_;  // isa_, or 2 for the GPU summation-order model (groups == 1 convs only)
    Graph g_;
    std::vector<std::uint8_t> weights_;
    std::vector<std::vector<u16>> bufs_;
    std::vector<int> state_in_, state_out_;
    std::map<std::uint32_t, std::size_t> in_pos_;
    std::map<std::uint32_t, int> consumers_;
    std::vector<std::pair<std::uint32_t, std::uint32_t>> bindings_;
    std::vector<std::uint32_t> external_, ext_out_;
    std::vector<Step> steps_;
    bool initialized_ = false;
};

template <typename F>
int guard(F&& f)
{
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return -1;
    }
}

Pool& kernel_pool(int threads)
{
    static std::map<int, std::unique_ptr<Pool>> pools;
    static std::mutex mu;
    std::lock_guard<std::mutex> l(mu);
    const int n = threads > 0 ? threads : default_threads();
    auto& p = pools[n];
    if (!p) p = std::make_unique<Pool>(n);
    return *p;
}

}  // namespace

// ---- codec I/O conversions around the encoder / decoder graphs ----------
// Frames are I420: Y plane w*h bytes, then U and V planes of (w/2)*(h/2).

// Byte -> FP16 input value: float_to_half((v / 255) * pixel_range),
// execution_plan.cpp:1452-1458 (the same table as yuv.cpp:350-354).
void byte_lut(float range, u16* lut)
{
    for (int v = 0; v < 256; ++v) lut[v] = f2h((static_cast<float>(v) / 255.0F) * range);
}

// Frame -> model input [3, mh, mw]: write_yuv420_to_nhwc_fp16,
// execution_plan.cpp:1052-1150, in NCHW order. The frame sits at model
// (0, 0); columns past it repeat its last column (:1101-1114) and rows past
// it its last row (:1116-1124). A rotated frame is transposed into the model
// (:1128-1149). Chroma samples cover 2x2 luma pixels.
void yuv_to_model(const std::uint8_t* yuv, int w, int h, int mw, int mh, int rotated, float range, u16* out)
{
    u16 lut[256];
    byte_lut(range, lut);
    const std::size_t ysz = static_cast<std::size_t>(w) * h, uvsz = ysz / 4;
    const std::uint8_t* pu = yuv + ysz;
    const std::uint8_t* pv = pu + uvsz;
    const std::size_t plane = static_cast<std::size_t>(mw) * mh;
    for (int y = 0; y < mh; ++y)
        for (int x = 0; x < mw; ++x) {
            int sy, sx;
            if (rotated) {
                sx = std::min(y, w - 1);
                sy = std::min(x, h - 1);
            } else {
                sy = std::min(y, h - 1);
                sx = std::min(x, w - 1);
            }
            const std::size_t o = static_cast<std::size_t>(y) * mw + x;
            const std::size_t uv = static_cast<std::size_t>(sy / 2) * (w / 2) + sx / 2;
            out[o] = lut[yuv[static_cast<std::size_t>(sy) * w + sx]];
            out[plane + o] = lut[pu[uv]];
            out[2 * plane + o] = lut[pv[uv]];
        }
}

// clamp to [0, 1], then nearbyint(v * 255) (round half to even):
// execution_plan.cpp:1046-1050.
std::uint8_t quantize_byte(float v)
{
    const float c = std::clamp(v, 0.0F, 1.0F);
    return static_cast<std::uint8_t>(std::nearbyint(c * 255.0F));
}

// Model output [3, mh, mw] -> frame: read_nhwc_fp16_to_yuv420,
// execution_plan.cpp:1211-1322. The active region starts at (pad_top,
// pad_left); each value is divided by pixel_range; chroma is the mean of
// its 2x2 block summed as ((s00 + s01) + s10) + s11 then scaled by 0.25
// (:1280-1291); a rotated frame reads the model transposed (:1296-1321).
void model_to_yuv(const u16* x, int w, int h, int mw, int mh, int pad_left, int pad_top, int rotated, float range,
                  std::uint8_t* yuv)
{
    const std::size_t ysz = static_cast<std::size_t>(w) * h, uvsz = ysz / 4;
    const std::size_t plane = static_cast<std::size_t>(mw) * mh;
    std::uint8_t* yo = yuv;
    std::uint8_t* uo = yuv + ysz;
    std::uint8_t* vo = uo + uvsz;
    auto sample = [&](int c, int y, int xx) {
        const int my = rotated ? xx + pad_top : y + pad_top;
        const int mx = rotated ? y + pad_left : xx + pad_left;
        return h2f(x[c * plane + static_cast<std::size_t>(my) * mw + mx]) / range;
    };
    for (int y = 0; y < h; ++y)
        for (int xx = 0; xx < w; ++xx) yo[static_cast<std::size_t>(y) * w + xx] = quantize_byte(sample(0, y, xx));
    for (int uy = 0; uy < h / 2; ++uy)
        for (int ux = 0; ux < w / 2; ++ux) {
            const std::size_t o = static_cast<std::size_t>(uy) * (w / 2) + ux;
            float su, sv;
            if (rotated) {
                su = 0.0F;
                sv = 0.0F;
                for (int dy = 0; dy < 2; ++dy)
                    for (int dx = 0; dx < 2; ++dx) {
                        su += sample(1, 2 * uy + dy, 2 * ux + dx);
                        sv += sample(2, 2 * uy + dy, 2 * ux + dx);
                    }
            } else {
                su = sample(1, 2 * uy, 2 * ux) + sample(1, 2 * uy, 2 * ux + 1) + sample(1, 2 * uy + 1, 2 * ux) +
                     sample(1, 2 * uy + 1, 2 * ux + 1);
                sv = sample(2, 2 * uy, 2 * ux) + sample(2, 2 * uy, 2 * ux + 1) + sample(2, 2 * uy + 1, 2 * ux) +
                     sample(2, 2 * uy + 1, 2 * ux + 1);
            }
            uo[o] = quantize_byte(su * 0.25F);
            vo[o] = quantize_byte(sv * 0.25F);
        }
}

// frame_padding, yuv.cpp:325-337: the frame fits as is, or transposed.
void frame_padding(int w, int h, int mw, int mh, int* pad)
{
    auto bad = [](int a, int b) { return a <= 0 || b <= 0 || a % 2 || b % 2; };
    if (bad(w, h) || bad(mw, mh)) throw std::runtime_error("YUV420 dimensions must be positive and even");
    const bool native = w <= mw && h <= mh;
    const bool rotated = h <= mw && w <= mh;
    if (!native && !rotated) throw std::runtime_error("input frame is larger than the model dimensions");
    const int aw = native ? w : h, ah = native ? h : w;
    pad[0] = 0;
    pad[1] = mw - aw;
    pad[2] = 0;
    pad[3] = mh - ah;
    pad[4] = native ? 0 : 1;
}

extern "C" {

const char* oracle_last_error(void) { return g_error.c_str(); }

int oracle_mfma_step(const uint16_t* a, const uint16_t* b, const float* c, float* out, size_t count)
{
    for (size_t i = 0; i < count; ++i) {
        float acc = c[i];
        for (int h = 0; h < 16; h += 8) {
            std::int32_t P[8];
            int E[8];
            for (int j = 0; j < 8; ++j) {
                const std::int32_t x = fp16_q(a[16 * i + h + j]), y = fp16_q(b[16 * i + h + j]);
                P[j] = (x >> 8) * (y >> 8);
                E[j] = (x & 255) + (y & 255) - 128;
            }
            acc = mfma_half(acc, P, E, 8);
        }
        out[i] = acc;
    }
    return 0;
}

void* oracle_load(const char* model_dir, const char* model_name, const int64_t* bindings, int n_bindings,
                  int num_threads, int isa, int enable_fusion)
{
    try {
        std::vector<std::pair<std::size_t, std::size_t>> b;
        for (int i = 0; i < n_bindings; ++i)
            b.emplace_back(static_cast<std::size_t>(bindings[2 * i]), static_cast<std::size_t>(bindings[2 * i + 1]));
        return new Plan(model_dir, model_name, b, num_threads, isa, enable_fusion != 0);
    } catch (const std::exception& e) {
        g_error = e.what();
        return nullptr;
    }
}

void oracle_free(void* plan) { delete static_cast<Plan*>(plan); }
int oracle_reset_state(void* plan) { return guard([&] { static_cast<Plan*>(plan)->reset(); }); }
int oracle_thread_count(void* plan) { return static_cast<Plan*>(plan)->threads(); }
int oracle_step_count(void* plan) { return static_cast<int>(static_cast<Plan*>(plan)->steps()); }

int oracle_io_count(void* plan, int is_output)
{
    auto* p = static_cast<Plan*>(plan);
    return static_cast<int>(is_output ? p->ext_out().size() : p->ext_in().size());
}

int oracle_io_shape(void* plan, int is_output, int index, int64_t* shape4, int* rank)
{
    return guard([&] {
        auto* p = static_cast<Plan*>(plan);
        const auto& ids = is_output ? p->ext_out() : p->ext_in();
        const auto& s = p->tensor(ids.at(static_cast<std::size_t>(index))).shape;
        *rank = static_cast<int>(s.size());
        for (std::size_t i = 0; i < s.size() && i < 4; ++i) shape4[i] = s[i];
    });
}

int oracle_run(void* plan, const uint16_t* const* inputs, uint16_t* const* outputs)
{
    return guard([&] { static_cast<Plan*>(plan)->run(inputs, outputs); });
}

size_t oracle_packed_conv_elems(int oc, int ic, int kh, int kw)
{
    return packed_conv_elems(static_cast<std::size_t>(oc), static_cast<std::size_t>(ic), static_cast<std::size_t>(kh), static_cast<std::size_t>(kw));
}

int oracle_pack_conv(const uint16_t* w, const uint16_t* bias, int oc, int ic, int kh, int kw, uint16_t* packed,
                     size_t packed_elems)
{
    return guard([&] {
        if (packed_elems < oracle_packed_conv_elems(oc, ic, kh, kw)) throw std::runtime_error("packed buffer too small");
        pack_conv(w, bias, static_cast<std::size_t>(oc), static_cast<std::size_t>(ic), static_cast<std::size_t>(kh), static_cast<std::size_t>(kw), packed);
    });
}

size_t oracle_packed_depthwise_elems(int c, int kh, int kw)
{
    return packed_dw_elems(static_cast<std::size_t>(c), static_cast<std::size_t>(kh), static_cast<std::size_t>(kw));
}

int oracle_pack_depthwise(const uint16_t* w, const uint16_t* bias, int c, int kh, int kw, uint16_t* packed,
                          size_t packed_elems)
{
    return guard([&] {
        if (packed_elems < oracle_packed_depthwise_elems(c, kh, kw)) throw std::runtime_error("packed buffer too small");
        pack_dw(w, bias, static_cast<std::size_t>(c), static_cast<std::size_t>(kh), static_cast<std::size_t>(kw), packed);
    });
}

int oracle_gemm_nhwc(size_t m, size_t n, size_t k, const uint16_t* lhs, const uint16_t* packed, uint16_t* dst,
                     int epi, float alpha, float cmin, float cmax, const uint16_t* residual, int isa, int threads)
{
    return guard([&] {
        Epilogue e{epi, alpha, cmin, cmax, residual};
        gemm_nhwc(kernel_pool(threads), isa, m, n, k, lhs, packed, dst, e);
    });
}

int oracle_spatial_conv_nhwc(const uint16_t* input, const uint16_t* packed, uint16_t* output, int n, int ic,
                             int ih, int iw, int oc, int oh, int ow, int kh, int kw, int sh, int sw, int ph,
                             int pw, int epi, float alpha, const uint16_t* residual, int isa, int threads)
{
    return guard([&] {
        Epilogue e{epi, alpha, 0.0F, 0.0F, residual};
        spatial_conv_nhwc(kernel_pool(threads), isa, input, packed, output, n, ic, ih, iw, oc, oh, ow, kh, kw, sh, sw, ph, pw, e);
    });
}

int oracle_depthwise_nhwc(const uint16_t* input, const uint16_t* packed, uint16_t* output, int n, int c, int ih,
                          int iw, int oh, int ow, int kh, int kw, int sh, int sw, int ph, int pw, int isa, int threads)
{
    return guard([&] { depthwise_nhwc(kernel_pool(threads), isa, input, packed, output, n, c, ih, iw, oh, ow, kh, kw, sh, sw, ph, pw); });
}

int oracle_leaky_relu(const uint16_t* in, uint16_t* out, size_t count, float alpha, int isa)
{
    return guard([&] { leaky(in, out, count, alpha, isa); });
}

int oracle_add(const uint16_t* a, const uint16_t* b, uint16_t* out, size_t count, int isa)
{
    return guard([&] { add(a, b, out, count, isa); });
}

int oracle_depth_to_space_nhwc(const uint16_t* in, uint16_t* out, int n, int c, int h, int w, int block)
{
    return guard([&] { d2s_nhwc(in, out, n, c, h, w, block); });
}

int oracle_space_to_depth_nhwc(const uint16_t* in, uint16_t* out, int n, int c, int h, int w, int block)
{
    return guard([&] { s2d_nhwc(in, out, n, c, h, w, block); });
}

int oracle_nchw_to_nhwc(const uint16_t* in, uint16_t* out, size_t n, size_t c, size_t hw)
{
    return guard([&] { nchw_to_nhwc(in, out, n, c, hw); });
}

int oracle_nhwc_to_nchw(const uint16_t* in, uint16_t* out, size_t n, size_t hw, size_t c)
{
    return guard([&] { nhwc_to_nchw(in, out, n, hw, c); });
}

int oracle_yuv420_to_model(const uint8_t* yuv, int w, int h, int mw, int mh, int rotated, float pixel_range,
                           uint16_t* out)
{
    return guard([&] { yuv_to_model(yuv, w, h, mw, mh, rotated, pixel_range, out); });
}

int oracle_model_to_yuv420(const uint16_t* x, int w, int h, int mw, int mh, int pad_left, int pad_top, int rotated,
                           float pixel_range, uint8_t* yuv)
{
    return guard([&] { model_to_yuv(x, w, h, mw, mh, pad_left, pad_top, rotated, pixel_range, yuv); });
}

int oracle_frame_padding(int w, int h, int mw, int mh, int* pad5)
{
    return guard([&] { frame_padding(w, h, mw, mh, pad5); });
}

int oracle_unary(const uint16_t* in, uint16_t* out, size_t count, int op, float lo, float hi, int isa)
{
    return guard([&] { unary(in, out, count, op, lo, hi, isa); });
}

int oracle_binary(const uint16_t* a, const int64_t* a_shape, int a_rank, const uint16_t* b, const int64_t* b_shape, int b_rank,
                  uint16_t* out, const int64_t* out_shape, int out_rank, int op)
{
    return guard([&] {
        binary_dispatch(a, std::vector<std::int64_t>(a_shape, a_shape + a_rank), b, std::vector<std::int64_t>(b_shape, b_shape + b_rank),
                        out, std::vector<std::int64_t>(out_shape, out_shape + out_rank), op);
    });
}

int oracle_slice_nhwc(const uint16_t* in, uint16_t* out, const int* id4, const int* od4, const int* starts, const int* steps)
{
    return guard([&] { slice_nhwc(in, out, id4, od4, starts, steps); });
}

int oracle_concat_nhwc(const uint16_t* const* ins, const int* dims4, int n, uint16_t* out, const int* od4, int axis)
{
    return guard([&] {
        std::vector<const u16*> v(ins, ins + n);
        std::vector<std::array<int, 4>> d(static_cast<std::size_t>(n));
        for (int i = 0; i < n; ++i)
            for (int k = 0; k < 4; ++k) d[static_cast<std::size_t>(i)][static_cast<std::size_t>(k)] = dims4[4 * i + k];
        concat_nhwc(v, d, out, {od4[0], od4[1], od4[2], od4[3]}, axis);
    });
}

int oracle_gather(const uint16_t* data, const int64_t* shape, int rank, const int32_t* idx32, const int64_t* idx64, size_t count,
                  int axis, uint16_t* out)
{
    return guard([&] { gather(data, std::vector<std::int64_t>(shape, shape + rank), idx32, idx64, count, axis, out); });
}

int oracle_reglu_nhwc(const uint16_t* in, uint16_t* out, size_t spatial, size_t gate_channels, float lo, float hi, int isa)
{
    return guard([&] { reglu(in, out, spatial, gate_channels, lo, hi, isa); });
}

int oracle_feature_update_nhwc(const uint16_t* in, const uint16_t* history, const uint16_t* scale, uint16_t* scaled_out,
                               uint16_t* blended_out, uint16_t* feature_out, size_t spatial, size_t channels, int isa)
{
    return guard([&] { feature_update(in, history, scale, scaled_out, blended_out, feature_out, spatial, channels, isa); });
}

int oracle_y0_tail_nhwc(const uint16_t* latent, const uint16_t* prior, const uint16_t* quant_scale, const uint16_t* us0,
                        const uint16_t* us1, uint16_t* normalized, uint16_t* clipped, uint16_t* y_raw, uint16_t* concat2,
                        uint16_t* concat3, float clip_min, size_t spatial, size_t q, int isa)
{
    return guard([&] { y0_tail(latent, prior, quant_scale, us0, us1, normalized, clipped, y_raw, concat2, concat3, clip_min, spatial, q, isa); });
}

int oracle_y1_tail_nhwc(const uint16_t* normalized, const uint16_t* prior, const uint16_t* quant_scale, const uint16_t* us0,
                        const uint16_t* us1, const uint16_t* concat2, const uint16_t* clipped, uint16_t* y_raw, uint16_t* out,
                        size_t spatial, size_t q)
{
    return guard([&] { y1_tail(normalized, prior, quant_scale, us0, us1, concat2, clipped, y_raw, out, spatial, q); });
}

uint16_t oracle_float_to_half(float f) { return f2h(f); }
float oracle_half_to_float(uint16_t h) { return h2f(h); }

}  // extern "C"
