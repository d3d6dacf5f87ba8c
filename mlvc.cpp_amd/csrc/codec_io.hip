// Codec I/O conversions on either side of the encoder / decoder graphs.
//
// Frames are I420 bytes: the Y plane (w x h), then U and V planes of
// (w/2) x (h/2). The model image is FP16 [3, mh, mw] (NCHW, batch 1).
//
//   frame -> model (encoder input): byte v of each plane becomes the FP16
//   value lut[v] = float_to_half(v / 255 * pixel_range), chroma samples
//   cover 2x2 luma pixels, columns past the frame repeat its last column and
//   rows past it its last row; a rotated frame is transposed into the model.
//   Same values as the reference CPU backend's write_yuv420_to_nhwc_fp16
//   (backends/cpu/src/execution_plan.cpp:1052-1150) and the driver backend's
//   mlvc_yuv420_to_nchw_fp16 (backends/driver_cubin/kernels/codec_io.cu:31-64).
//
//   model -> frame (decoder output): the active area starts at (pad_top,
//   pad_left); value / pixel_range (IEEE division, as the CPU backend), chroma
//   is ((s00 + s01) + s10) + s11 times 0.25, then clamp to [0, 1] and
//   round-half-even of v * 255 (execution_plan.cpp:1046-1050, 1211-1322).
//   The driver backend multiplies by the reciprocal instead
//   (codec_io.cu:66-107); dividing keeps the bytes equal to the CPU backend's
//   for every pixel range.
//
// Both directions are HBM-bound byte/half streams: one thread converts 8
// model columns (frame -> model) or a 2x16 luma block with its 8 U and 8 V
// samples (model -> frame), with 8- and 16-byte accesses where the shapes
// keep them aligned and a per-element path otherwise.

#include "common.hpp"
#include "mlvc_hip_device.h"

#include <algorithm>

namespace mlvc_hip {
namespace {

__device__ __forceinline__ std::uint8_t quantize_byte(float v)
{
    // fmaxf/fminf map NaN to 0; the reference leaves NaN to an undefined cast.
    const float c = fminf(fmaxf(v, 0.0F), 1.0F);
    return static_cast<std::uint8_t>(static_cast<int>(__builtin_rintf(c * 255.0F)));
}

constexpr int kYuvThreads = 256;

// One thread: model columns [8t, 8t + 8) of row y of channel c (grid
// x: column groups, y: rows, z: channel).
__global__ __launch_bounds__(kYuvThreads) void yuv_to_model_kernel(const std::uint8_t* __restrict__ yuv,
                                                                   const std::uint16_t* __restrict__ lut_g,
                                                                   std::uint16_t* __restrict__ out, int w, int h,
                                                                   int mw, int mh)
{
    __shared__ std::uint16_t lut[256];
    lut[threadIdx.x] = lut_g[threadIdx.x];
    __syncthreads();
    const int t = blockIdx.x * kYuvThreads + threadIdx.x;
    const int y = blockIdx.y, c = blockIdx.z;
    const int x0 = t * 8;
    if (x0 >= mw) return;
    const int sy = min(y, h - 1);
    const size_t ysz = static_cast<size_t>(w) * h;
    const std::uint8_t* row;
    if (c == 0)
        row = yuv + static_cast<size_t>(sy) * w;
    else
        row = yuv + ysz + static_cast<size_t>(c - 1) * (ysz / 4) + static_cast<size_t>(sy / 2) * (w / 2);
    std::uint16_t v[8];
    if (x0 + 8 <= w && (w & 7) == 0) {
        // Inside the frame, 8-aligned rows: one 8-byte (luma) or 4-byte
        // (chroma) load.
        if (c == 0) {
            const uint2 b = *reinterpret_cast<const uint2*>(row + x0);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                v[k] = lut[(b.x >> (8 * k)) & 0xFF];
                v[4 + k] = lut[(b.y >> (8 * k)) & 0xFF];
            }
        } else {
            const std::uint32_t b = *reinterpret_cast<const std::uint32_t*>(row + x0 / 2);
#pragma unroll
            for (int k = 0; k < 4; ++k) v[2 * k] = v[2 * k + 1] = lut[(b >> (8 * k)) & 0xFF];
        }
    } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int sx = min(x0 + k, w - 1);
            v[k] = lut[row[c == 0 ? sx : sx / 2]];
        }
    }
    std::uint16_t* dst = out + (static_cast<size_t>(c) * mh + y) * mw + x0;
    if (x0 + 8 <= mw && (mw & 7) == 0) {
        u32x4 q;
#pragma unroll
        for (int k = 0; k < 4; ++k) q[k] = static_cast<std::uint32_t>(v[2 * k]) | (static_cast<std::uint32_t>(v[2 * k + 1]) << 16);
        *reinterpret_cast<u32x4*>(dst) = q;
    } else {
        for (int k = 0; k < 8 && x0 + k < mw; ++k) dst[k] = v[k];
    }
}

// Rotated frames: model (y, x) reads frame (min(x, h-1), min(y, w-1)).
__global__ __launch_bounds__(kYuvThreads) void yuv_to_model_rotated_kernel(const std::uint8_t* __restrict__ yuv,
                                                                           const std::uint16_t* __restrict__ lut_g,
                                                                           std::uint16_t* __restrict__ out, int w,
                                                                           int h, int mw, int mh)
{
    __shared__ std::uint16_t lut[256];
    lut[threadIdx.x] = lut_g[threadIdx.x];
    __syncthreads();
    const size_t plane = static_cast<size_t>(mw) * mh;
    const size_t ysz = static_cast<size_t>(w) * h;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kYuvThreads + threadIdx.x; i < 3 * plane;
         i += static_cast<size_t>(gridDim.x) * kYuvThreads) {
        const int c = static_cast<int>(i / plane);
        const size_t sp = i - static_cast<size_t>(c) * plane;
        const int y = static_cast<int>(sp / mw), x = static_cast<int>(sp % mw);
        const int sx = min(y, w - 1), sy = min(x, h - 1);
        const std::uint8_t b = c == 0 ? yuv[static_cast<size_t>(sy) * w + sx]
                                      : yuv[ysz + static_cast<size_t>(c - 1) * (ysz / 4) +
                                            static_cast<size_t>(sy / 2) * (w / 2) + sx / 2];
        out[i] = lut[b];
    }
}

constexpr int kToYuvThreads = 128;
constexpr int kChromaPerThread = 8;  // 2x16 luma pixels, 8 U and 8 V samples per thread

// value / pixel_range as the CPU backend computes it; x / 1 is exact, so the
// unit-range instantiation has no IEEE division.
template <bool UNIT>
__device__ __forceinline__ float scaled(std::uint16_t h, float range)
{
    if constexpr (UNIT)
        return h2f(h);
    else
        return h2f(h) / range;
}

// One thread: chroma samples [8t, 8t + 8) of chroma row uy, i.e. luma rows
// 2uy, 2uy + 1 and columns [16t, 16t + 16) (grid x: column groups, y:
// chroma rows). VEC (the launch checks the alignment): every row segment is
// two 16-byte loads, the luma rows leave as 16-byte stores and U / V as
// 8-byte stores; otherwise element by element.
template <bool UNIT, bool VEC>
__global__ __launch_bounds__(kToYuvThreads) void model_to_yuv_kernel(const std::uint16_t* __restrict__ x,
                                                                     std::uint8_t* __restrict__ yuv, int w, int h,
                                                                     int mw, int mh, int pad_left, int pad_top,
                                                                     float range)
{
    constexpr int CPT = kChromaPerThread, LPT = 2 * CPT;  // chroma / luma columns per thread
    const int t = blockIdx.x * kToYuvThreads + threadIdx.x;
    const int uy = blockIdx.y;
    const int uw = w / 2;
    const int ux0 = t * CPT;
    if (ux0 >= uw) return;
    const size_t plane = static_cast<size_t>(mw) * mh;
    const size_t ysz = static_cast<size_t>(w) * h, uvsz = ysz / 4;
    const int n = min(CPT, uw - ux0);  // chroma samples of this thread
    const int col0 = pad_left + 2 * ux0;
    const size_t r0 = static_cast<size_t>(pad_top + 2 * uy) * mw + col0;
    const size_t r1 = r0 + mw;
    float s[3][2][LPT];
    if (VEC && n == CPT) {
        // All twelve loads are issued before the first use.
        u32x4 q[3][2][2];
#pragma unroll
        for (int c = 0; c < 3; ++c)
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int k = 0; k < 2; ++k)
                    q[c][r][k] = *reinterpret_cast<const u32x4*>(x + static_cast<size_t>(c) * plane + (r ? r1 : r0) + 8 * k);
#pragma unroll
        for (int c = 0; c < 3; ++c)
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int k = 0; k < 2; ++k)
#pragma unroll
                    for (int d = 0; d < 4; ++d) {
                        s[c][r][8 * k + 2 * d] = scaled<UNIT>(static_cast<std::uint16_t>(q[c][r][k][d] & 0xFFFFu), range);
                        s[c][r][8 * k + 2 * d + 1] = scaled<UNIT>(static_cast<std::uint16_t>(q[c][r][k][d] >> 16), range);
                    }
    } else {
#pragma unroll
        for (int c = 0; c < 3; ++c)
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const std::uint16_t* src = x + static_cast<size_t>(c) * plane + (r ? r1 : r0);
#pragma unroll
                for (int k = 0; k < LPT; ++k) s[c][r][k] = k < 2 * n ? scaled<UNIT>(src[k], range) : 0.0F;
            }
    }
    std::uint8_t yb[2][LPT], ub[CPT], vb[CPT];
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int k = 0; k < LPT; ++k) yb[r][k] = quantize_byte(s[0][r][k]);
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
        const float su = s[1][0][2 * k] + s[1][0][2 * k + 1] + s[1][1][2 * k] + s[1][1][2 * k + 1];
        const float sv = s[2][0][2 * k] + s[2][0][2 * k + 1] + s[2][1][2 * k] + s[2][1][2 * k + 1];
        ub[k] = quantize_byte(su * 0.25F);
        vb[k] = quantize_byte(sv * 0.25F);
    }
    std::uint8_t* yo = yuv + static_cast<size_t>(2 * uy) * w + 2 * ux0;
    std::uint8_t* uo = yuv + ysz + static_cast<size_t>(uy) * uw + ux0;
    std::uint8_t* vo = uo + uvsz;
    auto pack4 = [](const std::uint8_t* b) {
        return static_cast<std::uint32_t>(b[0]) | (static_cast<std::uint32_t>(b[1]) << 8) |
               (static_cast<std::uint32_t>(b[2]) << 16) | (static_cast<std::uint32_t>(b[3]) << 24);
    };
    if (VEC && n == CPT) {
#pragma unroll
        for (int r = 0; r < 2; ++r)
            *reinterpret_cast<u32x4*>(yo + static_cast<size_t>(r) * w) =
                u32x4{pack4(&yb[r][0]), pack4(&yb[r][4]), pack4(&yb[r][8]), pack4(&yb[r][12])};
        typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
        *reinterpret_cast<u32x2*>(uo) = u32x2{pack4(&ub[0]), pack4(&ub[4])};
        *reinterpret_cast<u32x2*>(vo) = u32x2{pack4(&vb[0]), pack4(&vb[4])};
    } else {
        for (int k = 0; k < n; ++k) {
            yo[2 * k] = yb[0][2 * k];
            yo[2 * k + 1] = yb[0][2 * k + 1];
            yo[w + 2 * k] = yb[1][2 * k];
            yo[w + 2 * k + 1] = yb[1][2 * k + 1];
            uo[k] = ub[k];
            vo[k] = vb[k];
        }
    }
}

// Rotated frames: frame (y, x) reads model (x + pad_top, y + pad_left).
// One thread per luma pixel; threads of the first (w/2)*(h/2) also produce
// one U and one V sample.
__global__ __launch_bounds__(kYuvThreads) void model_to_yuv_rotated_kernel(const std::uint16_t* __restrict__ x,
                                                                           std::uint8_t* __restrict__ yuv, int w,
                                                                           int h, int mw, int mh, int pad_left,
                                                                           int pad_top, float range)
{
    const size_t plane = static_cast<size_t>(mw) * mh;
    const size_t ysz = static_cast<size_t>(w) * h, uvsz = ysz / 4;
    const int uw = w / 2;
    auto sample = [&](int c, int fy, int fx) {
        return scaled<false>(x[static_cast<size_t>(c) * plane + static_cast<size_t>(fx + pad_top) * mw + fy + pad_left],
                             range);
    };
    for (size_t i = static_cast<size_t>(blockIdx.x) * kYuvThreads + threadIdx.x; i < ysz;
         i += static_cast<size_t>(gridDim.x) * kYuvThreads) {
        const int fy = static_cast<int>(i / w), fx = static_cast<int>(i % w);
        yuv[i] = quantize_byte(sample(0, fy, fx));
        if (i < uvsz) {
            const int uy = static_cast<int>(i / uw), ux = static_cast<int>(i % uw);
            float su = 0.0F, sv = 0.0F;
#pragma unroll
            for (int dy = 0; dy < 2; ++dy)
#pragma unroll
                for (int dx = 0; dx < 2; ++dx) {
                    su += sample(1, 2 * uy + dy, 2 * ux + dx);
                    sv += sample(2, 2 * uy + dy, 2 * ux + dx);
                }
            yuv[ysz + i] = quantize_byte(su * 0.25F);
            yuv[ysz + uvsz + i] = quantize_byte(sv * 0.25F);
        }
    }
}

void validate_frame(int w, int h, int mw, int mh, int rotated)
{
    if (w <= 0 || h <= 0 || (w & 1) || (h & 1) || mw <= 0 || mh <= 0)
        throw std::runtime_error("codec I/O: frame dimensions must be positive and even");
    const int aw = rotated ? h : w, ah = rotated ? w : h;
    if (aw > mw || ah > mh) throw std::runtime_error("codec I/O: frame is larger than the model image");
    if (mh > 65535 || static_cast<unsigned long long>(mw) * mh * 3 >= (1ull << 40))
        throw std::runtime_error("codec I/O: model image too large");
}

unsigned grid_1d(size_t count)
{
    return static_cast<unsigned>(std::min<size_t>((count + kYuvThreads - 1) / kYuvThreads, 65536));
}

}  // namespace
}  // namespace mlvc_hip

using namespace mlvc_hip;

extern "C" {

int mlvc_hip_yuv420_to_model(const uint8_t* yuv, const uint16_t* lut, void* out, int w, int h, int mw, int mh,
                             int rotated, mlvc_hip_stream s)
{
    return guard([&] {
        validate_frame(w, h, mw, mh, rotated);
        auto* o = static_cast<std::uint16_t*>(out);
        if (rotated) {
            hipLaunchKernelGGL(yuv_to_model_rotated_kernel, dim3(grid_1d(static_cast<size_t>(3) * mw * mh)),
                               dim3(kYuvThreads), 0, to_stream(s), yuv, lut, o, w, h, mw, mh);
        } else {
            const int groups = (mw + 7) / 8;
            const dim3 grid((groups + kYuvThreads - 1) / kYuvThreads, mh, 3);
            hipLaunchKernelGGL(yuv_to_model_kernel, grid, dim3(kYuvThreads), 0, to_stream(s), yuv, lut, o, w, h, mw, mh);
        }
        check(hipGetLastError(), "codec I/O kernel launch");
    });
}

int mlvc_hip_model_to_yuv420(const void* x, uint8_t* yuv, int w, int h, int mw, int mh, int pad_left, int pad_top,
                             int rotated, float pixel_range, mlvc_hip_stream s)
{
    return guard([&] {
        validate_frame(w, h, mw, mh, rotated);
        const int aw = rotated ? h : w, ah = rotated ? w : h;
        if (pad_left < 0 || pad_top < 0 || pad_left + aw > mw || pad_top + ah > mh)
            throw std::runtime_error("codec I/O: active area outside the model image");
        if (!(pixel_range > 0.0F) || pixel_range > 3.0e38F)
            throw std::runtime_error("codec I/O: pixel range must be finite and positive");
        const auto* xi = static_cast<const std::uint16_t*>(x);
        if (rotated) {
            hipLaunchKernelGGL(model_to_yuv_rotated_kernel, dim3(grid_1d(static_cast<size_t>(w) * h)),
                               dim3(kYuvThreads), 0, to_stream(s), xi, yuv, w, h, mw, mh, pad_left, pad_top,
                               pixel_range);
        } else {
            const int groups = (w / 2 + kChromaPerThread - 1) / kChromaPerThread;
            const dim3 grid((groups + kToYuvThreads - 1) / kToYuvThreads, h / 2);
            // 16-byte model row segments (base, plane, row and active-area
            // origin on 8 halves) and 16-byte luma / 8-byte chroma stores
            // (base on 16 bytes, w on 16 columns, so Y, U and V rows and
            // plane starts keep that alignment).
            const bool vec = (reinterpret_cast<std::uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<std::uintptr_t>(yuv) & 15u) == 0 &&
                             mw % 8 == 0 && pad_left % 8 == 0 && w % 16 == 0;
            auto go = [&](auto kernel) {
                hipLaunchKernelGGL(kernel, grid, dim3(kToYuvThreads), 0, to_stream(s), xi, yuv, w, h, mw, mh, pad_left,
                                   pad_top, pixel_range);
            };
            if (pixel_range == 1.0F)
                vec ? go(model_to_yuv_kernel<true, true>) : go(model_to_yuv_kernel<true, false>);
            else
                vec ? go(model_to_yuv_kernel<false, true>) : go(model_to_yuv_kernel<false, false>);
        }
        check(hipGetLastError(), "codec I/O kernel launch");
    });
}

}  // extern "C"
