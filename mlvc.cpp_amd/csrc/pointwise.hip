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

// Opaque to the optimiser: keeps f2h(fmaf(a, b, c)) from becoming one
// v_fma_mixlo_f16, which rounds once to FP16 where the reference rounds the
// FP32 result of the multiply-add to FP16 (two roundings).
__device__ __forceinline__ float keep(float x)
{
    asm("" : "+v"(x));
    return x;
}

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
            if (ox0 + j < ow) yp[j] = f2h(keep(acc[j]));
    }
}

// 3x3, stride 1, pad 1 on rows of a multiple of 8 pixels (16-byte aligned):
// one thread computes eight consecutive outputs in each of kDwRows rows, so
// each input row segment it loads serves up to three of its output rows.
// Every load is issued up front from clamped addresses (kDwRows + 2
// 16-byte row segments, the pixels beside them, the nine taps) and a thread
// waits for memory once; taps whose input lies outside the image are then
// skipped by selects. The arithmetic is the kernel above's: bias-seeded,
// taps in (ky, kx) order, one fused multiply-add each. grid.x: 8-pixel
// segments x row groups of one plane; grid.y: planes.
constexpr int kDwRows = 4;

__global__ __launch_bounds__(kBlock) void depthwise3x3_row8_kernel(const std::uint16_t* __restrict__ x,
                                                                   const std::uint16_t* __restrict__ w,
                                                                   const float* __restrict__ bias,
                                                                   std::uint16_t* __restrict__ y, int c, int h, int wd)
{
    constexpr int R = kDwRows, NR = R + 2;
    const int segs = wd / 8, groups = (h + R - 1) / R;
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= segs * groups) return;
    const int plane = blockIdx.y, ch = plane % c;
    const int g = i / segs, x0 = (i - g * segs) * 8, oy0 = g * R;
    const std::uint16_t* xp = x + static_cast<size_t>(plane) * h * wd;
    const std::uint16_t* wp = w + ch * 9;
    const int xl = x0 > 0 ? x0 - 1 : 0, xr = x0 + 8 < wd ? x0 + 8 : wd - 1;
    u32x4 v[NR];
    std::uint32_t lft[NR], rgt[NR], tap[9];
#pragma unroll
    for (int r = 0; r < NR; ++r) {  // input rows oy0 - 1 .. oy0 + R
        const int iy = min(max(oy0 - 1 + r, 0), h - 1);
        const std::uint16_t* row = xp + static_cast<size_t>(iy) * wd;
        v[r] = *reinterpret_cast<const u32x4*>(row + x0);
        lft[r] = row[xl];
        rgt[r] = row[xr];
    }
#pragma unroll
    for (int k = 0; k < 9; ++k) tap[k] = wp[k];
    // Keeps the compiler from sinking the pixel loads into the selects below
    // (a load per skipped-tap branch, each with its own wait).
#pragma unroll
    for (int r = 0; r < NR; ++r) asm volatile("" : "+v"(lft[r]), "+v"(rgt[r]));
    const float b = bias[ch];
    const bool left_in = x0 > 0, right_in = x0 + 8 < wd;
    // Each staged row converted to FP32 once and kept opaque, so the taps are
    // plain FP32 multiply-adds rather than mixed-precision ones that convert
    // the same pixel again for each of its taps.
    float pxr[NR][10];  // input columns x0 - 1 .. x0 + 8 of each staged row
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        pxr[r][0] = keep(h2f(static_cast<std::uint16_t>(lft[r])));
        pxr[r][9] = keep(h2f(static_cast<std::uint16_t>(rgt[r])));
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            pxr[r][1 + 2 * k] = keep(h2f(static_cast<std::uint16_t>(v[r][k] & 0xFFFFu)));
            pxr[r][2 + 2 * k] = keep(h2f(static_cast<std::uint16_t>(v[r][k] >> 16)));
        }
    }
    // All rows are computed before the first store: loads and stores share
    // one in-order counter, so a store issued between two waits for loads
    // would make the second wait also wait for the store's write.
    u32x4 o[R];
#pragma unroll
    for (int orow = 0; orow < R; ++orow) {
        const int oy = oy0 + orow;
        float acc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = b;
#pragma unroll
        for (int ky = 0; ky < 3; ++ky) {
            const int r = orow + ky;
            // Rows outside the image are skipped as a whole; within a row only
            // the two edge taps (column x0 - 1 at the left border, x0 + 8 at
            // the right one, x0 being a multiple of 8) can fall outside, so
            // every other tap is an unconditional multiply-add.
            if (oy - 1 + ky < 0 || oy - 1 + ky >= h) continue;
            const float* px = pxr[r];
#pragma unroll
            for (int kx = 0; kx < 3; ++kx) {
                const float wv = keep(h2f(static_cast<std::uint16_t>(tap[ky * 3 + kx])));
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if (j == 0 && kx == 0)
                        acc[j] = left_in ? fmaf(px[j + kx], wv, acc[j]) : acc[j];
                    else if (j == 7 && kx == 2)
                        acc[j] = right_in ? fmaf(px[j + kx], wv, acc[j]) : acc[j];
                    else
                        acc[j] = fmaf(px[j + kx], wv, acc[j]);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
            o[orow][k] = static_cast<std::uint32_t>(f2h(keep(acc[2 * k]))) |
                         (static_cast<std::uint32_t>(f2h(keep(acc[2 * k + 1]))) << 16);
    }
#pragma unroll
    for (int orow = 0; orow < R; ++orow) asm volatile("" : "+v"(o[orow]));  // every row done before any store
#pragma unroll
    for (int orow = 0; orow < R; ++orow)
        if (oy0 + orow < h) *reinterpret_cast<u32x4*>(y + (static_cast<size_t>(plane) * h + oy0 + orow) * wd + x0) = o[orow];
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

// Block 2 on input rows of a multiple of 4 pixels (8-byte aligned): one
// thread takes four input pixels of each of the two planes c*4 + dy*2 +
// {0, 1} at input row y (8-byte loads) and writes the eight output pixels
// they interleave into as one 16-byte store, so consecutive lanes load and
// store consecutive bytes. grid.x: 16-byte output chunks x output rows of
// one output plane; grid.y: output planes (b*oc + c).
__global__ __launch_bounds__(kBlock) void d2s2_row4_kernel(const std::uint16_t* __restrict__ x, std::uint16_t* __restrict__ y,
                                                          int h, int w)
{
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    const int cw = w / 4;  // 16-byte chunks per output row
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= cw * 2 * h) return;
    const int Y = i / cw, k = i - Y * cw, iy = Y >> 1, dy = Y & 1;
    const size_t plane = blockIdx.y, hw = static_cast<size_t>(h) * w;
    const std::uint16_t* in = x + (plane * 4 + static_cast<size_t>(dy) * 2) * hw + static_cast<size_t>(iy) * w + 4 * k;
    const u32x2 a = *reinterpret_cast<const u32x2*>(in);       // dx = 0
    const u32x2 b = *reinterpret_cast<const u32x2*>(in + hw);  // dx = 1
    u32x4 o;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        o[2 * q] = (a[q] & 0xFFFFu) | (b[q] << 16);
        o[2 * q + 1] = (a[q] >> 16) | (b[q] & 0xFFFF0000u);
    }
    *reinterpret_cast<u32x4*>(y + (plane * 2 * h + Y) * (2 * static_cast<size_t>(w)) + 8 * k) = o;
}

// Block 2 on input rows of a multiple of 16 pixels (16-byte aligned): one
// thread reads sixteen pixels of input row 2*oy + dy and writes their even
// (dx = 0) and odd (dx = 1) halves to planes c*4 + dy*2 + {0, 1} at row oy,
// one 16-byte store each. grid.x: segments x output rows x dy of one input
// plane; grid.y: input planes (b*ic + c).
__global__ __launch_bounds__(kBlock) void s2d2_row8_kernel(const std::uint16_t* __restrict__ x, std::uint16_t* __restrict__ y,
                                                          int h, int w)
{
    const int ow = w / 2, oh = h / 2, segs = ow / 8;
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= segs * h) return;
    const int Y = i / segs, ox0 = (i - Y * segs) * 8, oy = Y >> 1, dy = Y & 1;
    const size_t plane = blockIdx.y, ohw = static_cast<size_t>(oh) * ow;
    const std::uint16_t* in = x + (plane * h + Y) * static_cast<size_t>(w) + 2 * ox0;
    const u32x4 a = *reinterpret_cast<const u32x4*>(in);
    const u32x4 b = *reinterpret_cast<const u32x4*>(in + 8);
    u32x4 ev, od;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        ev[k] = (a[2 * k] & 0xFFFFu) | (a[2 * k + 1] << 16);
        od[k] = (a[2 * k] >> 16) | (a[2 * k + 1] & 0xFFFF0000u);
        ev[k + 2] = (b[2 * k] & 0xFFFFu) | (b[2 * k + 1] << 16);
        od[k + 2] = (b[2 * k] >> 16) | (b[2 * k + 1] & 0xFFFF0000u);
    }
    std::uint16_t* out = y + (plane * 4 + static_cast<size_t>(dy) * 2) * ohw + static_cast<size_t>(oy) * ow + ox0;
    *reinterpret_cast<u32x4*>(out) = ev;
    *reinterpret_cast<u32x4*>(out + ohw) = od;
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

// FP16 values in [-1, 1) from a hash of (element index, seed): a stand-in
// for real activations where only the timing of the kernels reading them
// matters (load-time tuning), since matrix cores fed zeros draw less power
// and run faster than on real data.
__global__ __launch_bounds__(kBlock) void pattern_kernel(std::uint16_t* __restrict__ y, size_t count, std::uint32_t seed)
{
    for (size_t i = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; i < count;
         i += static_cast<size_t>(gridDim.x) * kBlock) {
        std::uint32_t h = static_cast<std::uint32_t>(i) * 0x9E3779B1u ^ (static_cast<std::uint32_t>(i >> 32) + seed) * 0x85EBCA77u;
        h ^= h >> 15;
        h *= 0x2C1B3C6Du;
        h ^= h >> 13;
        // sign | exponent 14 (0x3800 = 0.5) | 10 random mantissa bits: |v| in [0.5, 1)
        y[i] = static_cast<std::uint16_t>((h & 0x8000u) | 0x3800u | ((h >> 4) & 0x03FFu));
    }
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
        const size_t planes = static_cast<size_t>(n) * c;
        if (kh == 3 && kw == 3 && stride_h == 1 && stride_w == 1 && pad_h == 1 && pad_w == 1 && iw % 8 == 0 &&
            planes <= 65535 && static_cast<size_t>(ih) * (iw / 8) < (1u << 30) && aligned16(x) && aligned16(y)) {
            const size_t threads = static_cast<size_t>((ih + kDwRows - 1) / kDwRows) * (iw / 8);
            const unsigned gx = static_cast<unsigned>((threads + kBlock - 1) / kBlock);
            hipLaunchKernelGGL(depthwise3x3_row8_kernel, dim3(gx, static_cast<unsigned>(planes)), dim3(kBlock), 0, to_stream(s),
                               static_cast<const std::uint16_t*>(x), w, bias, static_cast<std::uint16_t*>(y), c, ih, iw);
            check(hipGetLastError(), "depthwise launch");
            return;
        }
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
        const size_t planes = static_cast<size_t>(n) * oc;
        if (block == 2 && w % 4 == 0 && planes <= 65535 && static_cast<size_t>(h) * (w / 2) < (1u << 30) && aligned16(x) &&
            aligned16(y)) {
            const unsigned gx = static_cast<unsigned>((static_cast<size_t>(h) * (w / 2) + kBlock - 1) / kBlock);
            hipLaunchKernelGGL(d2s2_row4_kernel, dim3(gx, static_cast<unsigned>(planes)), dim3(kBlock), 0, to_stream(s),
                               static_cast<const std::uint16_t*>(x), static_cast<std::uint16_t*>(y), h, w);
            check(hipGetLastError(), "depth_to_space launch");
            return;
        }
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
        const size_t planes = static_cast<size_t>(n) * in_c;
        if (block == 2 && w % 16 == 0 && planes <= 65535 && static_cast<size_t>(h) * (w / 16) < (1u << 30) && aligned16(x) &&
            aligned16(y)) {
            const unsigned gx = static_cast<unsigned>((static_cast<size_t>(h) * (w / 16) + kBlock - 1) / kBlock);
            hipLaunchKernelGGL(s2d2_row8_kernel, dim3(gx, static_cast<unsigned>(planes)), dim3(kBlock), 0, to_stream(s),
                               static_cast<const std::uint16_t*>(x), static_cast<std::uint16_t*>(y), h, w);
            check(hipGetLastError(), "space_to_depth launch");
            return;
        }
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

int mlvc_hip_fill_pattern(void* y, size_t bytes, unsigned seed, mlvc_hip_stream s)
{
    return guard([&] {
        if (!y || bytes % 2 != 0) throw std::runtime_error("fill_pattern: null buffer or odd byte count");
        const size_t count = bytes / 2;
        hipLaunchKernelGGL(pattern_kernel, dim3(grid_for(count)), dim3(kBlock), 0, to_stream(s), static_cast<std::uint16_t*>(y),
                           count, static_cast<std::uint32_t>(seed));
        check(hipGetLastError(), "fill_pattern launch");
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
