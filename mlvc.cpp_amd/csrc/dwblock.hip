// Fused depthwise-separable residual block on gfx950:
//
//   d = fp16(DW3x3(x) + b0)                     (bias-seeded FMA taps, (ky,kx) order)
//   e = fp16(LeakyReLU(fp16(W1 d + b1)))        (1x1 C -> E, MFMA)
//   y = fp16(fp16(W2 e + b2) + x)               (1x1 E -> C, MFMA, residual)
//
// Same rounding points as the unfused schedule (the reference runs DW, a
// conv with a LeakyReLU epilogue and a conv with a residual epilogue:
// backends/cpu/src/kernels_x86_avx2.cpp:237-302, kernels_scalar.cpp:178-192),
// but d and e never leave the chip. One workgroup (4 waves) owns a 4x8 pixel
// tile and all channels:
//   1. x is staged in channel chunks of 64 as 16-byte vectors (rows padded to
//      24 halves so the 3x3 halo of an 8-wide, 8-aligned tile is covered);
//      the depthwise result goes to LDS channel-last, d[pixel][C + 8];
//   2. expand: each wave owns E/128 m-tiles of 32 channels; A fragments (W1,
//      pre-packed in fragment order) stream from L2 one k-step ahead, B
//      fragments are 16-byte LDS reads of d; e goes to LDS as e[pixel][E + 8];
//   3. project: each wave owns C/128 m-tiles; the residual is read from x in
//      global memory (L2-hot) and the result stored NCHW.
// Requires W % 8 == 0 (16-byte aligned rows); other shapes run unfused.

#include "common.hpp"
#include "mlvc_hip_device.h"

#include <cstring>

namespace mlvc_hip {
namespace {

constexpr int kTH = 4, kTW = 8, kP = kTH * kTW;  // 32 pixels per workgroup
constexpr int kCC = 64;                           // depthwise channel chunk
constexpr int kRow = 24;                          // staged halves per input row

struct DwBlockArgs {
    const std::uint16_t* x;
    std::uint16_t* y;
    const std::uint16_t* dw_w;
    const float* dw_b;
    const std::uint16_t* w1;
    const float* b1;
    const std::uint16_t* w2;
    const float* b2;
    int h, w, tiles_x;
    float alpha;
};

template <int C, int E>
__global__ __launch_bounds__(256) void dwblock_kernel(DwBlockArgs a)
{
    constexpr int DST = C + 8, EST = E + 8;
    constexpr int XS = kCC * (kTH + 2) * kRow;
    constexpr int MT1 = E / 32 / 4, MT2 = C / 32 / 4;  // m-tiles per wave
    constexpr int KS1 = C / 16, KS2 = E / 16;
    static_assert(C % 128 == 0 && E % 128 == 0, "channel counts");
    __shared__ __attribute__((aligned(16))) std::uint16_t xs[XS];
    __shared__ __attribute__((aligned(16))) std::uint16_t ds[kP * DST];
    __shared__ __attribute__((aligned(16))) std::uint16_t es[kP * EST];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int x0 = (blockIdx.x % a.tiles_x) * kTW, y0 = (blockIdx.x / a.tiles_x) * kTH;
    const int b = blockIdx.y;
    const size_t plane = static_cast<size_t>(a.h) * a.w;
    const std::uint16_t* xb = a.x + static_cast<size_t>(b) * C * plane;

    // ---- 1. depthwise 3x3, channel chunks of 64 -------------------------
    for (int c0 = 0; c0 < C; c0 += kCC) {
        // 64 channels x 6 rows x 3 vectors of 8 halves.
        for (int v = tid; v < kCC * (kTH + 2) * 3; v += 256) {
            const int seg = v % 3, row = (v / 3) % (kTH + 2), c = v / (3 * (kTH + 2));
            const int iy = y0 - 1 + row, ix = x0 - 8 + seg * 8;
            u32x4 val = {0u, 0u, 0u, 0u};
            if (iy >= 0 && iy < a.h && ix >= 0 && ix < a.w)
                val = *reinterpret_cast<const u32x4*>(xb + (c0 + c) * plane + static_cast<size_t>(iy) * a.w + ix);
            *reinterpret_cast<u32x4*>(&xs[(c * (kTH + 2) + row) * kRow + seg * 8]) = val;
        }
        __syncthreads();
        for (int o = tid; o < kCC * kP; o += 256) {
            const int p = o % kP, c = o / kP;
            const int py = p / kTW, px = p % kTW;
            const int gy = y0 + py, gx = x0 + px;
            const int ch = c0 + c;
            float acc = a.dw_b[ch];
            const std::uint16_t* wc = a.dw_w + ch * 9;
#pragma unroll
            for (int ky = 0; ky < 3; ++ky) {
                const int iy = gy + ky - 1;
                if (iy < 0 || iy >= a.h) continue;
#pragma unroll
                for (int kx = 0; kx < 3; ++kx) {
                    const int ix = gx + kx - 1;
                    if (ix < 0 || ix >= a.w) continue;
                    acc = fmaf(h2f(xs[(c * (kTH + 2) + py + ky) * kRow + 7 + px + kx]), h2f(wc[ky * 3 + kx]), acc);
                }
            }
            ds[p * DST + ch] = f2h(acc);
        }
        __syncthreads();
    }

    const int koff = (lane >> 5) * 8, pl = lane & 31;
    // ---- 2. expand 1x1 C -> E, bias, round, LeakyReLU, round -------------
    {
        floatx16 acc[MT1];
#pragma unroll
        for (int m = 0; m < MT1; ++m) {
            const int mt = wave * MT1 + m;
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[m][r] = a.b1[mt * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)];
        }
        const u32x4* w1 = reinterpret_cast<const u32x4*>(a.w1);
        u32x4 cur[MT1], nxt[MT1];
#pragma unroll
        for (int m = 0; m < MT1; ++m) cur[m] = w1[((wave * MT1 + m) * KS1 + 0) * 64 + lane];
        for (int ks = 0; ks < KS1; ++ks) {
            if (ks + 1 < KS1) {
#pragma unroll
                for (int m = 0; m < MT1; ++m) nxt[m] = w1[((wave * MT1 + m) * KS1 + ks + 1) * 64 + lane];
            }
            const half8 bv = *reinterpret_cast<const half8*>(&ds[pl * DST + ks * 16 + koff]);
#pragma unroll
            for (int m = 0; m < MT1; ++m)
                acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, cur[m]), bv, acc[m], 0, 0, 0);
            if (ks + 1 < KS1) {
#pragma unroll
                for (int m = 0; m < MT1; ++m) cur[m] = nxt[m];
            }
        }
#pragma unroll
        for (int m = 0; m < MT1; ++m) {
            const int mt = wave * MT1 + m;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                std::uint16_t hv = f2h(acc[m][r]);
                const float f = h2f(hv);
                if (f < 0.0f) hv = f2h(f * a.alpha);
                es[pl * EST + mt * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)] = hv;
            }
        }
    }
    __syncthreads();
    // ---- 3. project 1x1 E -> C, bias, round, + residual, round -----------
    {
        floatx16 acc[MT2];
#pragma unroll
        for (int m = 0; m < MT2; ++m) {
            const int mt = wave * MT2 + m;
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[m][r] = a.b2[mt * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)];
        }
        const u32x4* w2 = reinterpret_cast<const u32x4*>(a.w2);
        u32x4 cur[MT2], nxt[MT2];
#pragma unroll
        for (int m = 0; m < MT2; ++m) cur[m] = w2[((wave * MT2 + m) * KS2 + 0) * 64 + lane];
        for (int ks = 0; ks < KS2; ++ks) {
            if (ks + 1 < KS2) {
#pragma unroll
                for (int m = 0; m < MT2; ++m) nxt[m] = w2[((wave * MT2 + m) * KS2 + ks + 1) * 64 + lane];
            }
            const half8 bv = *reinterpret_cast<const half8*>(&es[pl * EST + ks * 16 + koff]);
#pragma unroll
            for (int m = 0; m < MT2; ++m)
                acc[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, cur[m]), bv, acc[m], 0, 0, 0);
            if (ks + 1 < KS2) {
#pragma unroll
                for (int m = 0; m < MT2; ++m) cur[m] = nxt[m];
            }
        }
        const int gy = y0 + pl / kTW, gx = x0 + pl % kTW;
        if (gy < a.h && gx < a.w) {
            const size_t po = static_cast<size_t>(gy) * a.w + gx;
            std::uint16_t* yb = a.y + static_cast<size_t>(b) * C * plane;
#pragma unroll
            for (int m = 0; m < MT2; ++m) {
                const int mt = wave * MT2 + m;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int ch = mt * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    const std::uint16_t hv = f2h(acc[m][r]);
                    yb[ch * plane + po] = f2h(h2f(hv) + h2f(xb[ch * plane + po]));
                }
            }
        }
    }
}

template <int C, int E>
void launch(const DwBlockArgs& a, dim3 grid, hipStream_t s)
{
    hipLaunchKernelGGL((dwblock_kernel<C, E>), grid, dim3(256), 0, s, a);
}

}  // namespace
}  // namespace mlvc_hip

using namespace mlvc_hip;

extern "C" {

int mlvc_hip_dwblock_supported(int c, int e, int h, int w)
{
    return ((c == 256 && e == 512) || (c == 128 && e == 256) || (c == 128 && e == 512)) && h > 0 && w > 0 && w % 8 == 0;
}

size_t mlvc_hip_dwblock_packed_bytes(int m, int k) { return static_cast<size_t>(m) * k * 2; }

int mlvc_hip_dwblock_pack(const uint16_t* w_mk, int m, int k, void* dst_host)
{
    return guard([&] {
        if (m % 32 != 0 || k % 16 != 0) throw std::runtime_error("dwblock: weight shape not tileable");
        auto* out = static_cast<std::uint16_t*>(dst_host);
        size_t o = 0;
        // [m-tile][k-step][lane][8]: lane l holds W[mt*32 + l%32][ks*16 + 8*(l/32) + j].
        for (int mt = 0; mt < m / 32; ++mt)
            for (int ks = 0; ks < k / 16; ++ks)
                for (int lane = 0; lane < 64; ++lane)
                    for (int j = 0; j < 8; ++j)
                        out[o++] = w_mk[static_cast<size_t>(mt * 32 + (lane & 31)) * k + ks * 16 + 8 * (lane >> 5) + j];
    });
}

int mlvc_hip_dwblock_launch(const mlvc_hip_dwblock_desc* d, mlvc_hip_stream s)
{
    return guard([&] {
        if (!mlvc_hip_dwblock_supported(d->c, d->e, d->h, d->w) || d->n <= 0)
            throw std::runtime_error("dwblock: unsupported geometry");
        if (!d->x || !d->y || !d->dw_w || !d->dw_b || !d->w1 || !d->b1 || !d->w2 || !d->b2)
            throw std::runtime_error("dwblock: null tensor");
        DwBlockArgs a{static_cast<const std::uint16_t*>(d->x), static_cast<std::uint16_t*>(d->y),
                      static_cast<const std::uint16_t*>(d->dw_w), d->dw_b,
                      static_cast<const std::uint16_t*>(d->w1), d->b1,
                      static_cast<const std::uint16_t*>(d->w2), d->b2,
                      d->h, d->w, (d->w + kTW - 1) / kTW, d->alpha};
        const dim3 grid(static_cast<unsigned>(a.tiles_x * ((d->h + kTH - 1) / kTH)), static_cast<unsigned>(d->n));
        if (d->c == 256 && d->e == 512) launch<256, 512>(a, grid, to_stream(s));
        else if (d->c == 128 && d->e == 256) launch<128, 256>(a, grid, to_stream(s));
        else launch<128, 512>(a, grid, to_stream(s));
        check(hipGetLastError(), "dwblock launch");
    });
}

}  // extern "C"
