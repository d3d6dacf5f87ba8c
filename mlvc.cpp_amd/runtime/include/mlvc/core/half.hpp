#pragma once
// IEEE-754 binary16 <-> binary32 conversion with round-to-nearest-even.
//
// Matches the semantics of the reference's software converters
// (core/include/mlvc/core/half.hpp:10-87): exact widening, RNE narrowing,
// overflow to signed infinity, gradual underflow to subnormals, NaNs kept
// quiet with the top mantissa bits carried over. Written from the IEEE-754
// encoding rules; the FP16 GPU path uses the hardware conversion, which
// rounds the same way.

#include "mlvc/core/tensor.hpp"

#include <bit>
#include <cstdint>

namespace mlvc {

inline float half_to_float(Float16Storage h) noexcept
{
    const std::uint32_t sign = (static_cast<std::uint32_t>(h) & 0x8000U) << 16;
    const std::uint32_t exp = (h >> 10) & 0x1FU;
    std::uint32_t frac = h & 0x3FFU;
    std::uint32_t out;
    if (exp == 0x1FU) {
        // Inf / NaN; a NaN is forced quiet.
        out = sign | 0x7F800000U | (frac << 13) | (frac ? 0x00400000U : 0U);
    } else if (exp != 0) {
        out = sign | ((exp + 112U) << 23) | (frac << 13);
    } else if (frac == 0) {
        out = sign;
    } else {
        // Subnormal: value = frac * 2^-24. Move the leading one to bit 10
        // (the implicit position); its bit index 31-lz sets the exponent.
        const int lz = std::countl_zero(frac);
        frac = (frac << (lz - 21)) & 0x3FFU;
        out = sign | (static_cast<std::uint32_t>(134 - lz) << 23) | (frac << 13);
    }
    return std::bit_cast<float>(out);
}

inline Float16Storage float_to_half(float f) noexcept
{
    const std::uint32_t x = std::bit_cast<std::uint32_t>(f);
    const auto sign = static_cast<std::uint16_t>((x >> 16) & 0x8000U);
    const std::uint32_t exp = (x >> 23) & 0xFFU;
    const std::uint32_t frac = x & 0x7FFFFFU;
    if (exp == 0xFFU) {
        if (frac == 0)
            return static_cast<Float16Storage>(sign | 0x7C00U);
        return static_cast<Float16Storage>(sign | 0x7E00U | (frac >> 13));
    }
    const int e = static_cast<int>(exp) - 112;  // biased binary16 exponent
    if (e >= 31)
        return static_cast<Float16Storage>(sign | 0x7C00U);
    std::uint32_t mant;
    int shift;
    if (e <= 0) {
        if (e < -10)
            return sign;  // below half the smallest subnormal
        mant = frac | 0x800000U;
        shift = 14 - e;
    } else {
        mant = frac;
        shift = 13;
    }
    std::uint32_t q = mant >> shift;
    const std::uint32_t rem = mant & ((1U << shift) - 1U);
    const std::uint32_t half = 1U << (shift - 1);
    if (rem > half || (rem == half && (q & 1U)))
        ++q;  // a carry out of the fraction bumps the exponent, possibly to inf
    const std::uint32_t base = e <= 0 ? 0U : (static_cast<std::uint32_t>(e) << 10);
    return static_cast<Float16Storage>(sign | (base + q));
}

}  // namespace mlvc
