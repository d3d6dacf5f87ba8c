// Shared helpers of the gfx950 device library.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace mlvc_hip {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

void set_error(const std::string& message);

inline void check(hipError_t err, const char* what)
{
    if (err != hipSuccess)
        throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(err));
}

// Runs `fn`, converting exceptions into the C ABI's -1 + message.
template <typename F>
int guard(F&& fn)
{
    try {
        fn();
        return 0;
    } catch (const std::exception& e) {
        set_error(e.what());
        return -1;
    }
}

// gfx950 deals the workgroups of a dispatch round-robin over its 8 XCDs
// (workgroup i runs on XCD i % 8), and each XCD has its own L2. xcd_order
// renumbers a 1-D grid of n workgroups so that XCD k runs the contiguous
// range of logical work items [k*(n/8) + min(k, n%8), ...) in order: work
// items that share input (neighbouring tiles, the output-channel blocks of
// one tile) then share an L2 instead of being fetched once per XCD. It is a
// bijection on [0, n) whatever n is.
constexpr int kXcds = 8;
__device__ __forceinline__ int xcd_order(int id, int n)
{
    const int per = n / kXcds, rem = n % kXcds, xcd = id % kXcds;
    return xcd * per + min(xcd, rem) + id / kXcds;
}

inline hipStream_t to_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

namespace conv {
// Compute units of the current device (queried once).
int cu_count();
}  // namespace conv

__device__ __forceinline__ float h2f(std::uint16_t h)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// Round-to-nearest-even narrowing (v_cvt_f16_f32 in the default mode).
__device__ __forceinline__ std::uint16_t f2h(float f)
{
    return __builtin_bit_cast(std::uint16_t, static_cast<_Float16>(f));
}

// LeakyReLU of an FP16 value f: fp16(f * alpha) with the product rounded to
// FP32 first, as the reference computes it. The multiply is issued as a plain
// v_mul_f32 so it stays a separate rounding step: left alone the compiler
// folds multiply and narrowing into v_fma_mixlo_f16, which rounds once and
// gives a different FP16 result when the FP32 product is an FP16 tie
// (e.g. 0x815E * 0.01f: -3.5 ulp after the FP32 rounding -> -4, not -3).
__device__ __forceinline__ float mul_f32(float a, float b)
{
    float p;
    asm("v_mul_f32 %0, %1, %2" : "=v"(p) : "v"(a), "v"(b));
    return p;
}

__device__ __forceinline__ std::uint16_t leaky_f16(float f, float alpha) { return f2h(mul_f32(f, alpha)); }

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float lo_f16(std::uint32_t v) { return h2f(static_cast<std::uint16_t>(v & 0xFFFFu)); }
__device__ __forceinline__ float hi_f16(std::uint32_t v) { return h2f(static_cast<std::uint16_t>(v >> 16)); }

// Two FP32 values -> packed FP16 pair (RNE), low half first.
__device__ __forceinline__ std::uint32_t pack_f16(float a0, float a1)
{
    const half2_t h = {static_cast<_Float16>(a0), static_cast<_Float16>(a1)};
    return __builtin_bit_cast(std::uint32_t, h);
}

// LeakyReLU of a packed pair of FP16 values h (already rounded): the
// reference's select, h < 0 ? fp16(fp32(h * alpha)) : h. The product is
// computed for both lanes unconditionally and the choice is a per-lane
// select, so the code is straight-line (no divergent branches around the
// multiply). For 0 <= alpha <= 1 the select equals max(h, fp16(h * alpha))
// (rounding is monotonic; NaN and -0 keep h), one packed max.
__device__ __forceinline__ std::uint32_t leaky_h2(std::uint32_t hv, float alpha, bool max_form)
{
    const half2_t h = __builtin_bit_cast(half2_t, hv);
    const float f0 = static_cast<float>(h[0]), f1 = static_cast<float>(h[1]);
    const half2_t p = {static_cast<_Float16>(mul_f32(f0, alpha)), static_cast<_Float16>(mul_f32(f1, alpha))};
    if (max_form) return __builtin_bit_cast(std::uint32_t, __builtin_elementwise_max(h, p));
    const half2_t r = {f0 < 0.0f ? p[0] : h[0], f1 < 0.0f ? p[1] : h[1]};
    return __builtin_bit_cast(std::uint32_t, r);
}

// Two FP32 accumulators -> packed FP16 pair (RNE) after LeakyReLU on the
// rounded values, as leaky_h2.
__device__ __forceinline__ std::uint32_t leaky_pair(float a0, float a1, float alpha, bool max_form)
{
    return leaky_h2(pack_f16(a0, a1), alpha, max_form);
}

// Epilogue modes fixed at compile time: 0 none, 1 LeakyReLU with
// 0 <= alpha <= 1 (max form), 2 LeakyReLU with any other alpha (select form).
inline int epi_mode(int epi_is_leaky, float alpha)
{
    return epi_is_leaky ? (alpha >= 0.0f && alpha <= 1.0f ? 1 : 2) : 0;
}

template <int MODE>
__device__ __forceinline__ std::uint32_t epi_pair(float a0, float a1, float alpha)
{
    if constexpr (MODE == 0) return pack_f16(a0, a1);
    else return leaky_h2(pack_f16(a0, a1), alpha, MODE == 1);
}

}  // namespace mlvc_hip
