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
// The reference's real-model fusions (ReGLU, recurrent feature update,
// quantisation tails) and the SLICE/GATHER/CLIP/SIGMOID/... operators are not
// on the conv-graph path and are not restated; graphs that need them are
// rejected. Parity pins: see the test files under tests/ (bit-exact against
// the reference kernels built from source, known-answer graphs, brute force).

#include "oracle.h"

#include <immintrin.h>

#include <algorithm>
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

void run_block(int isa, std::size_t m, std::size_t n, std::size_t k, const u16* lhs, std::size_t lhs_stride,
               const u16* packed, u16* dst, const Epilogue& e, std::size_t row0)
{
    if (isa == 0 && n % 16 == 0)
        block_avx2(m, n, k, lhs, lhs_stride, packed, dst, e, row0);
    else
        block_scalar(m, n, k, lhs, lhs_stride, packed, dst, e, row0);
}

constexpr std::size_t kRows = 24;

void gemm_nhwc(Pool& pool, int isa, std::size_t m, std::size_t n, std::size_t k, const u16* lhs,
               const u16* packed, u16* dst, const Epilogue& e)
{
    const std::size_t tiles = (m + kRows - 1) / kRows;
    pool.parallel_for(tiles, 1, [&](std::size_t t0, std::size_t t1) {
        for (std::size_t t = t0; t < t1; ++t) {
            const std::size_t m0 = t * kRows, mc = std::min(kRows, m - m0);
            run_block(isa, mc, n, k, lhs + m0 * k, k, packed, dst + m0 * n, e, m0);
        }
    });
}

void spatial_conv_nhwc(Pool& pool, int isa, const u16* in, const u16* packed, u16* out, int bn, int ic,
                       int ih, int iw, int oc, int oh, int ow, int kh, int kw, int sh, int sw, int ph,
                       int pw, const Epilogue& e)
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
                      out + m0 * static_cast<std::size_t>(oc), e, m0);
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

enum Op { ADD = 1, CLIP = 4, CONCAT = 5, CONV = 6, D2S = 7, LEAKY = 9, S2D = 14 };

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
};
struct Step {
    int kind = 0;  // 0 single node, 1 conv with epilogue
    std::size_t node = 0;
    Epilogue epi;
    std::uint32_t conv_in = 0, residual = 0, out = 0;
    ConvInfo conv;
};

class Plan {
public:
    Plan(const std::string& dir, const std::string& model, const std::vector<std::pair<std::size_t, std::size_t>>& bind,
         int threads, int isa, bool fuse)
        : pool_(threads > 0 ? threads : default_threads()), isa_(isa)
    {
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
            // FP16 activations; INT32 graph inputs (q_index_shifted, which no
            // operator of this path reads) are carried as raw bytes.
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

    void compile(bool fuse)
    {
        std::map<std::uint32_t, int> consumers;
        for (const GNode& n : g_.nodes)
            for (auto id : n.in)
                if (id) ++consumers[id];
        for (std::size_t i = 0; i < g_.nodes.size();) {
            Step s;
            if (fuse && try_epilogue(i, consumers, s)) {
                s.conv = conv_info(g_.nodes[i]);
                steps_.push_back(std::move(s));
                i += 2;
                continue;
            }
            s = Step{};
            s.node = i;
            const GNode& n = g_.nodes[i];
            switch (n.op) {
            case CONV: s.conv = conv_info(n); break;
            case LEAKY: case ADD: case D2S: case S2D: case CONCAT: break;
            default: throw std::runtime_error("oracle: operator outside the conv-graph path: " + std::to_string(n.op));
            }
            s.out = n.out.at(0);
            steps_.push_back(std::move(s));
            ++i;
        }
    }

    void run_conv(const ConvInfo& c, std::uint32_t in, std::uint32_t out, Epilogue e)
    {
        const u16* ip = bufs_[in].data();
        u16* op = bufs_[out].data();
        if (c.depthwise) {
            depthwise_nhwc(pool_, isa_, ip, c.packed.data(), op, c.n, c.ic, c.ih, c.iw, c.oh, c.ow, c.kh, c.kw, c.sh, c.sw, c.ph, c.pw);
        } else if (c.is1x1) {
            gemm_nhwc(pool_, isa_, static_cast<std::size_t>(c.n) * c.oh * c.ow, static_cast<std::size_t>(c.oc), static_cast<std::size_t>(c.ic), ip, c.packed.data(), op, e);
        } else {
            spatial_conv_nhwc(pool_, isa_, ip, c.packed.data(), op, c.n, c.ic, c.ih, c.iw, c.oc, c.oh, c.ow, c.kh, c.kw, c.sh, c.sw, c.ph, c.pw, e);
        }
    }

    void exec(const Step& s)
    {
        if (s.kind == 1) {
            Epilogue e = s.epi;
            if (s.residual) e.residual = bufs_[s.residual].data();
            run_conv(s.conv, s.conv_in, s.out, e);
            return;
        }
        const GNode& n = g_.nodes[s.node];
        const GTensor& ot = g_.t[s.out];
        u16* o = bufs_[s.out].data();
        switch (n.op) {
        case CONV: run_conv(s.conv, n.in[0], s.out, Epilogue{}); break;
        case LEAKY: leaky(bufs_[n.in[0]].data(), o, bufs_[s.out].size(), n.attr == 6 ? n.alpha : 0.01F, isa_); break;
        case ADD:
            if (g_.t[n.in[0]].shape != ot.shape || g_.t[n.in[1]].shape != ot.shape)
                throw std::runtime_error("oracle: broadcast ADD is outside the conv-graph path");
            add(bufs_[n.in[0]].data(), bufs_[n.in[1]].data(), o, bufs_[s.out].size(), isa_);
            break;
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
            int axis = n.axis < 0 ? n.axis + 4 : n.axis;
            if (axis != 1 || ot.shape.size() != 4) throw std::runtime_error("oracle: only channel CONCAT is on this path");
            const std::size_t px = static_cast<std::size_t>(ot.shape[0] * ot.shape[2] * ot.shape[3]);
            const std::size_t oc = static_cast<std::size_t>(ot.shape[1]);
            std::size_t off = 0;
            for (auto id : n.in) {
                const std::size_t ic = static_cast<std::size_t>(g_.t[id].shape[1]);
                const u16* src = bufs_[id].data();
                for (std::size_t p = 0; p < px; ++p) std::memcpy(o + p * oc + off, src + p * ic, ic * 2);
                off += ic;
            }
            break;
        }
        default: throw std::runtime_error("oracle: unsupported operator during execution");
        }
    }

    Pool pool_;
    int isa_;
    Graph g_;
    std::vector<std::uint8_t> weights_;
    std::vector<std::vector<u16>> bufs_;
    std::vector<int> state_in_, state_out_;
    std::map<std::uint32_t, std::size_t> in_pos_;
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

uint16_t oracle_float_to_half(float f) { return f2h(f); }
float oracle_half_to_float(uint16_t h) { return h2f(h); }

}  // extern "C"
