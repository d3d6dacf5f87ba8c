// Bandwidth-bound kernels of the conv-graph path: depthwise KxK, CRD pixel
// shuffle/unshuffle, LeakyReLU, ADD, channel concat and zero fill. All
// tensors are NCHW FP16; arithmetic is FP32 with one RNE rounding to FP16
// per materialised value, as in the reference CPU kernels
// (backends/cpu/src/kernels_x86_avx2.cpp:237-398).

#include "common.hpp"
#include "mlvc_hip_device.h"

#include <algorithm>

namespace mlvc_hip {
namespace {

constexpr int kBlock = 256;

unsigned grid_for(size_t work)
{
    return static_cast<unsigned>(std::max<size_t>(1, std::min<size_t>((work + kBlock - 1) / kBlock, 1u << 20)));
}

// Four consecutive outputs of one row per thread. Accumulator seeded with
// the bias, taps in (ky, kx) order, out-of-range taps skipped, one fused
// multiply-add per tap (reference: avx2_depthwise3x3_s1p1).
__global__ __launch_bounds__(kBlock) void depthwise_kernel(const std::uint16_t* __restrict__ x,
                                                           const std::uint16_t* __restrict__ w,
                                                           const float* __restrict__ bias,
                                                           std::uint16_t* __restrict__ y, int planes, int c,
                                                           int ih, int iw, int oh, int ow, int kh, int kw,
                                                           int sh, int sw, int ph, int pw)
{
    const int quads = (ow + 3) / 4;
    const size_t total = static_cast<size_t>(planes) * oh * quads;
    for (size_t i = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * kBlock) {
        const int q = static_cast<int>(i % quads);
        const int oy = static_cast<int>((i / quads) % oh);
        const int plane = static_cast<int>(i / (static_cast<size_t>(quads) * oh));
        const int ch = plane % c;
        const std::uint16_t* xp = x + static_cast<size_t>(plane) * ih * iw;
        const std::uint16_t* wp = w + static_cast<size_t>(ch) * kh * kw;
        const int ox0 = q * 4;
        float acc[4];
        const float b = bias[ch];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = b;
        for (int ky = 0; ky < kh; ++ky) {
            const int iy = oy * sh - ph + ky;
            if (iy < 0 || iy >= ih) continue;
            const std::uint16_t* row = xp + static_cast<size_t>(iy) * iw;
            for (int kx = 0; kx < kw; ++kx) {
                const float wv = h2f(wp[ky * kw + kx]);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int ix = (ox0 + j) * sw - pw + kx;
                    if (ox0 + j < ow && ix >= 0 && ix < iw) acc[j] = fmaf(h2f(row[ix]), wv, acc[j]);
                }
            }
        }
        std::uint16_t* yp = y + (static_cast<size_t>(plane) * oh + oy) * ow + ox0;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (ox0 + j < ow) yp[j] = f2h(acc[j]);
    }
}

// DEPTH_TO_SPACE (CRD): out[b][c][y*s+dy][x*s+dx] = in[b][c*s*s + dy*s + dx][y][x].
__global__ __launch_bounds__(kBlock) void d2s_kernel(const std::uint16_t* __restrict__ x, std::uint16_t* __restrict__ y,
                                                     int n, int oc, int h, int w, int s)
{
    const int H = h * s, W = w * s;
    const size_t total = static_cast<size_t>(n) * oc * H * W;
    for (size_t i = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * kBlock) {
        const int X = static_cast<int>(i % W);
        const int Y = static_cast<int>((i / W) % H);
        const size_t plane = i / (static_cast<size_t>(W) * H);  // b*oc + c
        const int dy = Y % s, dx = X % s;
        const size_t in_plane = plane * s * s + static_cast<size_t>(dy * s + dx);
        y[i] = x[(in_plane * h + Y / s) * w + X / s];
    }
}

// SPACE_TO_DEPTH (CRD): out[b][c*s*s + dy*s + dx][y][x] = in[b][c][y*s+dy][x*s+dx].
__global__ __launch_bounds__(kBlock) void s2d_kernel(const std::uint16_t* __restrict__ x, std::uint16_t* __restrict__ y,
                                                     int n, int ic, int h, int w, int s)
{
    const int oh = h / s, ow = w / s, oc = ic * s * s;
    const size_t total = static_cast<size_t>(n) * oc * oh * ow;
    for (size_t i = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * kBlock) {
        const int ox = static_cast<int>(i % ow);
        const int oy = static_cast<int>((i / ow) % oh);
        const int ocx = static_cast<int>((i / (static_cast<size_t>(ow) * oh)) % oc);
        const int b = static_cast<int>(i / (static_cast<size_t>(ow) * oh * oc));
        const int c = ocx / (s * s), r = ocx % (s * s), dy = r / s, dx = r % s;
        y[i] = x[((static_cast<size_t>(b) * ic + c) * h + oy * s + dy) * w + ox * s + dx];
    }
}

template <int OP>  // 0: leaky relu, 1: add
__global__ __launch_bounds__(kBlock) void eltwise_kernel(const std::uint16_t* __restrict__ a,
                                                         const std::uint16_t* __restrict__ b,
                                                         std::uint16_t* __restrict__ y, size_t count, float alpha)
{
    const size_t vecs = count / 8;
    for (size_t i = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; i < vecs;
         i += static_cast<size_t>(gridDim.x) * kBlock) {
        const uint4 va = reinterpret_cast<const uint4*>(a)[i];
        uint4 vb = {};
        if (OP == 1) vb = reinterpret_cast<const uint4*>(b)[i];
        const std::uint16_t* pa = reinterpret_cast<const std::uint16_t*>(&va);
        const std::uint16_t* pb = reinterpret_cast<const std::uint16_t*>(&vb);
        uint4 out;
        std::uint16_t* po = reinterpret_cast<std::uint16_t*>(&out);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float f = h2f(pa[j]);
            po[j] = OP == 0 ? (f < 0.0f ? leaky_f16(f, alpha) : pa[j]) : f2h(f + h2f(pb[j]));
        }
        reinterpret_cast<uint4*>(y)[i] = out;
    }
    for (size_t i = vecs * 8 + blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; i < count;
         i += static_cast<size_t>(gridDim.x) * kBlock) {
        const float f = h2f(a[i]);
        y[i] = OP == 0 ? (f < 0.0f ? leaky_f16(f, alpha) : a[i]) : f2h(f + h2f(b[i]));
    }
}

__global__ __launch_bounds__(kBlock) void concat_kernel(const std::uint16_t* __restrict__ a, size_t sa,
                                                        const std::uint16_t* __restrict__ b, size_t sb,
                                                        std::uint16_t* __restrict__ y, int n)
{
    const size_t per = sa + sb, total = per * n;
    for (size_t i = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * kBlock) {
        const size_t bi = i / per, r = i % per;
        y[i] = r < sa ? a[bi * sa + r] : b[bi * sb + (r - sa)];
    }
}

__global__ __launch_bounds__(kBlock) void zero_kernel(std::uint8_t* __restrict__ y, size_t bytes)
{
    const size_t vecs = bytes / 16;
    for (size_t i = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; i < vecs;
         i += static_cast<size_t>(gridDim.x) * kBlock)
        reinterpret_cast<uint4*>(y)[i] = uint4{0, 0, 0, 0};
    for (size_t i = vecs * 16 + blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; i < bytes;
         i += static_cast<size_t>(gridDim.x) * kBlock)
        y[i] = 0;
}

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace mlvc_hip

using namespace mlvc_hip;

extern "C" {

int mlvc_hip_depthwise(const void* x, const uint16_t* w, const float* bias, void* y, int n, int c, int ih, int iw,
                       int oh, int ow, int kh, int kw, int stride_h, int stride_w, int pad_h, int pad_w,
                       mlvc_hip_stream s)
{
    return guard([&] {
        if (n <= 0 || c <= 0 || ih <= 0 || iw <= 0 || oh <= 0 || ow <= 0 || kh <= 0 || kw <= 0 || stride_h <= 0 ||
            stride_w <= 0 || pad_h < 0 || pad_w < 0)
            throw std::runtime_error("depthwise: invalid geometry");
        if (oh != (ih + 2 * pad_h - kh) / stride_h + 1 || ow != (iw + 2 * pad_w - kw) / stride_w + 1)
            throw std::runtime_error("depthwise: output shape does not match the geometry");
        const size_t work = static_cast<size_t>(n) * c * oh * ((ow + 3) / 4);
        hipLaunchKernelGGL(depthwise_kernel, dim3(grid_for(work)), dim3(kBlock), 0, to_stream(s),
                           static_cast<const std::uint16_t*>(x), w, bias, static_cast<std::uint16_t*>(y), n * c, c,
                           ih, iw, oh, ow, kh, kw, stride_h, stride_w, pad_h, pad_w);
        check(hipGetLastError(), "depthwise launch");
    });
}

int mlvc_hip_depth_to_space(const void* x, void* y, int n, int in_c, int h, int w, int block, mlvc_hip_stream s)
{
    return guard([&] {
        if (n <= 0 || h <= 0 || w <= 0 || block <= 0 || in_c <= 0 || in_c % (block * block) != 0)
            throw std::runtime_error("depth_to_space: invalid geometry");
        const int oc = in_c / (block * block);
        const size_t total = static_cast<size_t>(n) * in_c * h * w;
        hipLaunchKernelGGL(d2s_kernel, dim3(grid_for(total)), dim3(kBlock), 0, to_stream(s),
                           static_cast<const std::uint16_t*>(x), static_cast<std::uint16_t*>(y), n, oc, h, w, block);
        check(hipGetLastError(), "depth_to_space launch");
    });
}

int mlvc_hip_space_to_depth(const void* x, void* y, int n, int in_c, int h, int w, int block, mlvc_hip_stream s)
{
    return guard([&] {
        if (n <= 0 || in_c <= 0 || block <= 0 || h <= 0 || w <= 0 || h % block != 0 || w % block != 0)
            throw std::runtime_error("space_to_depth: invalid geometry");
        const size_t total = static_cast<size_t>(n) * in_c * h * w;
        hipLaunchKernelGGL(s2d_kernel, dim3(grid_for(total)), dim3(kBlock), 0, to_stream(s),
                           static_cast<const std::uint16_t*>(x), static_cast<std::uint16_t*>(y), n, in_c, h, w, block);
        check(hipGetLastError(), "space_to_depth launch");
    });
}

int mlvc_hip_leaky_relu(const void* x, void* y, size_t count, float alpha, mlvc_hip_stream s)
{
    return guard([&] {
        if (!aligned16(x) || !aligned16(y)) throw std::runtime_error("leaky_relu: buffers must be 16-byte aligned");
        hipLaunchKernelGGL(eltwise_kernel<0>, dim3(grid_for(count / 8 + 1)), dim3(kBlock), 0, to_stream(s),
                           static_cast<const std::uint16_t*>(x), nullptr, static_cast<std::uint16_t*>(y), count, alpha);
        check(hipGetLastError(), "leaky_relu launch");
    });
}

int mlvc_hip_add(const void* a, const void* b, void* y, size_t count, mlvc_hip_stream s)
{
    return guard([&] {
        if (!aligned16(a) || !aligned16(b) || !aligned16(y)) throw std::runtime_error("add: buffers must be 16-byte aligned");
        hipLaunchKernelGGL(eltwise_kernel<1>, dim3(grid_for(count / 8 + 1)), dim3(kBlock), 0, to_stream(s),
                           static_cast<const std::uint16_t*>(a), static_cast<const std::uint16_t*>(b),
                           static_cast<std::uint16_t*>(y), count, 0.0f);
        check(hipGetLastError(), "add launch");
    });
}

int mlvc_hip_concat_channels(const void* a, int ca, const void* b, int cb, void* y, int n, size_t hw, mlvc_hip_stream s)
{
    return guard([&] {
        if (ca <= 0 || cb <= 0 || n <= 0) throw std::runtime_error("concat: invalid geometry");
        const size_t sa = static_cast<size_t>(ca) * hw, sb = static_cast<size_t>(cb) * hw;
        hipLaunchKernelGGL(concat_kernel, dim3(grid_for((sa + sb) * n)), dim3(kBlock), 0, to_stream(s),
                           static_cast<const std::uint16_t*>(a), sa, static_cast<const std::uint16_t*>(b), sb,
                           static_cast<std::uint16_t*>(y), n);
        check(hipGetLastError(), "concat launch");
    });
}

int mlvc_hip_zero(void* y, size_t bytes, mlvc_hip_stream s)
{
    return guard([&] {
        if (!aligned16(y)) throw std::runtime_error("zero: buffer must be 16-byte aligned");
        hipLaunchKernelGGL(zero_kernel, dim3(grid_for(bytes / 16 + 1)), dim3(kBlock), 0, to_stream(s),
                           static_cast<std::uint8_t*>(y), bytes);
        check(hipGetLastError(), "zero launch");
    });
}

}  // extern "C"
