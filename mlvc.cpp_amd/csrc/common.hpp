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

inline hipStream_t to_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

__device__ __forceinline__ float h2f(std::uint16_t h)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// Round-to-nearest-even narrowing (v_cvt_f16_f32 in the default mode).
__device__ __forceinline__ std::uint16_t f2h(float f)
{
    return __builtin_bit_cast(std::uint16_t, static_cast<_Float16>(f));
}

}  // namespace mlvc_hip
