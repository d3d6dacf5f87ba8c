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
// tile and all channels. At 1920x1088 / 16 the grid is one workgroup per CU,
// so the kernel is bound by how fast each CU streams the 2*C*E weight halves
// it needs, not by MFMA issue. It is organised around that stream:
//   * every wave runs ONE register ring of RING weight fragments (16 bytes per
//     lane, pre-packed in A-fragment order) through both GEMMs, so W1 and then
//     W2 are in flight from the first instruction to the last MFMA, across
//     the depthwise stage and the barriers between stages;
//   * the 6x24 halo tile of all C channels is staged with one batch of
//     16-byte loads; each thread then runs the depthwise taps for two
//     adjacent channels from registers and writes d[pixel][C + 8] as packed
//     pairs;
//   * accumulators are seeded with the bias (float4 loads issued at start);
//   * the project result is rounded into LDS as [channel][pixel] and leaves
//     as 16-byte rows with the residual added from 16-byte loads of x.
// LDS: xs (halo tile) aliases es (expand result); ds (depthwise result)
// aliases ys (project result). Requires W % 8 == 0 (16-byte rows).

#include "common.hpp"
#include "mlvc_hip_device.h"

#include <cstring>

namespace mlvc_hip {
namespace {

constexpr int kTH = 4, kTW = 8, kP = kTH * kTW;  // 32 pixels per workgroup
constexpr int kRow = 24;                          // staged halves per input row
constexpr int kXC = (kTH + 2) * kRow + 8;         // staged halves per channel (+8: bank spread)
constexpr int kYS = kP + 8;                       // ys row stride (halves)
constexpr int kRing = 16;                         // weight fragments in flight per wave

struct DwBlockArgs {
    const std::uint16_t* x;
    std::uint16_t* y;
    const std::uint16_t* dw_w;
    const float* dw_b;
    const std::uint16_t* w1;
    const float* b1;
    const std::uint16_t* w2;
    const float* b2;
    int h, w, tiles_x, tiles, nwg;  // nwg = tiles * n
    float alpha;
};

// LDS-only barrier: waits for this wave's LDS traffic, not for its global
// loads, so the weight ring stays in flight across stages.
__device__ __forceinline__ void lds_barrier()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float lo_h(std::uint32_t v) { return h2f(static_cast<std::uint16_t>(v & 0xFFFFu)); }
__device__ __forceinline__ float hi_h(std::uint32_t v) { return h2f(static_cast<std::uint16_t>(v >> 16)); }

template <int C, int E>
__global__ __launch_bounds__(256) void dwblock_kernel(DwBlockArgs a)
{
    constexpr int DST = C + 8, EST = E + 8;
    constexpr int MT1 = E / 32 / 4, MT2 = C / 32 / 4;  // m-tiles per wave
    constexpr int KS1 = C / 16, KS2 = E / 16;
    constexpr int NF1 = MT1 * KS1, NF = NF1 + MT2 * KS2;  // fragments per wave
    constexpr int XV = C * (kTH + 2) * 3 / 256;           // staged 16-byte vectors per thread
    constexpr int RV = C * kTH / 256;                     // residual rows per thread
    constexpr int CP = C / 2, RPT = kTH * CP / 256;       // channel pairs, output rows per thread
    static_assert(C % 128 == 0 && E % 128 == 0, "channel counts");
    static_assert(C * (kTH + 2) * 3 % 256 == 0 && C * kTH % 256 == 0 && kTH * CP % 256 == 0, "thread mapping");
    constexpr int XS_BYTES = C * kXC * 2, ES_BYTES = kP * EST * 2;
    constexpr int DS_BYTES = kP * DST * 2, YS_BYTES = C * kYS * 2;
    __shared__ __attribute__((aligned(16))) std::uint8_t lds_a[XS_BYTES > ES_BYTES ? XS_BYTES : ES_BYTES];
    __shared__ __attribute__((aligned(16))) std::uint8_t lds_b[DS_BYTES > YS_BYTES ? DS_BYTES : YS_BYTES];
    std::uint16_t* xs = reinterpret_cast<std::uint16_t*>(lds_a);
    std::uint16_t* es = reinterpret_cast<std::uint16_t*>(lds_a);
    std::uint16_t* ds = reinterpret_cast<std::uint16_t*>(lds_b);
    std::uint16_t* ys = reinterpret_cast<std::uint16_t*>(lds_b);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Each XCD runs a contiguous band of tiles, so the halo rows it stages
    // and the residual it re-reads stay in its own L2.
    const int item = xcd_order(blockIdx.x, a.nwg), tile = item % a.tiles, b = item / a.tiles;
    const int x0 = (tile % a.tiles_x) * kTW, y0 = (tile / a.tiles_x) * kTH;
    const size_t plane = static_cast<size_t>(a.h) * a.w;
    const std::uint16_t* xb = a.x + static_cast<size_t>(b) * C * plane;
    const u32x4* w1 = reinterpret_cast<const u32x4*>(a.w1);
    const u32x4* w2 = reinterpret_cast<const u32x4*>(a.w2);
    const int koff = (lane >> 5) * 8, pl = lane & 31, hsel = 4 * (lane >> 5);

    // Fragment f of this wave's stream: W1 in (k-step, m-tile) order, then W2.
    auto frag = [&](int f) -> u32x4 {
        if (f < NF1) return w1[((wave * MT1 + f % MT1) * KS1 + f / MT1) * 64 + lane];
        f -= NF1;
        return w2[((wave * MT2 + f % MT2) * KS2 + f / MT2) * 64 + lane];
    };
    u32x4 ring[kRing];
#pragma unroll
    for (int f = 0; f < kRing; ++f) ring[f] = frag(f);

    // Expand accumulators seeded with b1: lane holds rows 8j + hsel + (0..3).
    floatx16 acc1[MT1];
#pragma unroll
    for (int m = 0; m < MT1; ++m)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const floatx4 bv = *reinterpret_cast<const floatx4*>(a.b1 + (wave * MT1 + m) * 32 + 8 * j + hsel);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc1[m][4 * j + i] = bv[i];
        }
    // The scheduler would otherwise sink every ring load down to its MFMA
    // (minimising live registers) and serialise the stream on L2 latency;
    // scheduling barriers keep each load in the stage that issues it.
    __builtin_amdgcn_sched_barrier(0);

    // ---- 1. stage the 6-row halo of all C channels (one batch of loads) ----
    // Loads are unconditional (addresses clamped into the image, out-of-image
    // vectors zeroed afterwards): a branch around a load makes the compiler
    // wait for every load in flight, the weight ring included.
    {
        u32x4 v[XV];
#pragma unroll
        for (int i = 0; i < XV; ++i) {
            const int q = tid + 256 * i;
            const int seg = q % 3, row = (q / 3) % (kTH + 2), c = q / (3 * (kTH + 2));
            const int iy = min(max(y0 - 1 + row, 0), a.h - 1), ix = min(max(x0 - 8 + seg * 8, 0), a.w - 8);
            v[i] = *reinterpret_cast<const u32x4*>(xb + c * plane + static_cast<size_t>(iy) * a.w + ix);
        }
#pragma unroll
        for (int i = 0; i < XV; ++i) {
            const int q = tid + 256 * i;
            const int seg = q % 3, row = (q / 3) % (kTH + 2), c = q / (3 * (kTH + 2));
            const int iy = y0 - 1 + row, ix = x0 - 8 + seg * 8;
            const bool in = iy >= 0 && iy < a.h && ix >= 0 && ix < a.w;
            *reinterpret_cast<u32x4*>(&xs[c * kXC + row * kRow + seg * 8]) = in ? v[i] : u32x4{0u, 0u, 0u, 0u};
        }
    }
    // Depthwise weights and bias of this thread's channel pair.
    const int cp = tid % CP, rg = tid / CP;
    std::uint32_t wdw[9];
#pragma unroll
    for (int i = 0; i < 9; ++i) wdw[i] = reinterpret_cast<const std::uint32_t*>(a.dw_w)[cp * 9 + i];
    const float bd0 = a.dw_b[2 * cp], bd1 = a.dw_b[2 * cp + 1];
    lds_barrier();

    // ---- 2. depthwise 3x3 for channels 2cp, 2cp+1, output rows rg*RPT.. ----
    {
        const bool left = x0 > 0, right = x0 + kTW < a.w;
        float d0[RPT][kTW], d1[RPT][kTW];
#pragma unroll
        for (int r = 0; r < RPT; ++r)
#pragma unroll
            for (int px = 0; px < kTW; ++px) {
                d0[r][px] = bd0;
                d1[r][px] = bd1;
            }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const std::uint16_t* xc = xs + (2 * cp + j) * kXC;
            float wt[9];
#pragma unroll
            for (int t = 0; t < 9; ++t) {
                const int e = j * 9 + t;  // halves 18cp + e of the pair's weights
                wt[t] = (e & 1) ? hi_h(wdw[e >> 1]) : lo_h(wdw[e >> 1]);
            }
#pragma unroll
            for (int r = 0; r < RPT; ++r) {
                const int orow = rg * RPT + r, gy = y0 + orow;
#pragma unroll
                for (int ky = 0; ky < 3; ++ky) {
                    const int iy = gy + ky - 1;
                    if (iy < 0 || iy >= a.h) continue;
                    const std::uint16_t* row = xc + (orow + ky) * kRow;
                    const std::uint32_t l = *reinterpret_cast<const std::uint32_t*>(row + 6);
                    const u32x4 m = *reinterpret_cast<const u32x4*>(row + 8);
                    const std::uint32_t rr = *reinterpret_cast<const std::uint32_t*>(row + 16);
                    float xv[kTW + 2];
                    xv[0] = hi_h(l);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        xv[1 + 2 * i] = lo_h(m[i]);
                        xv[2 + 2 * i] = hi_h(m[i]);
                    }
                    xv[kTW + 1] = lo_h(rr);
#pragma unroll
                    for (int px = 0; px < kTW; ++px)
#pragma unroll
                        for (int kx = 0; kx < 3; ++kx) {
                            if (px + kx == 0 && !left) continue;
                            if (px + kx == kTW + 1 && !right) continue;
                            float& acc = j ? d1[r][px] : d0[r][px];
                            acc = fmaf(xv[px + kx], wt[ky * 3 + kx], acc);
                        }
                }
            }
        }
#pragma unroll
        for (int r = 0; r < RPT; ++r)
#pragma unroll
            for (int px = 0; px < kTW; ++px) {
                const int p = (rg * RPT + r) * kTW + px;
                const std::uint32_t v = static_cast<std::uint32_t>(f2h(d0[r][px])) |
                                        (static_cast<std::uint32_t>(f2h(d1[r][px])) << 16);
                *reinterpret_cast<std::uint32_t*>(&ds[p * DST + 2 * cp]) = v;
            }
    }
    lds_barrier();

    // ---- 3. expand 1x1 C -> E, round, LeakyReLU, round -> es --------------
#pragma unroll
    for (int ks = 0; ks < KS1; ++ks) {
        const half8 bv = *reinterpret_cast<const half8*>(&ds[pl * DST + ks * 16 + koff]);
#pragma unroll
        for (int m = 0; m < MT1; ++m) {
            const int f = ks * MT1 + m;
            const u32x4 av = ring[f % kRing];
            if (f + kRing < NF) ring[f % kRing] = frag(f + kRing);
            acc1[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, av), bv, acc1[m], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    // Project accumulators (b2) and the residual rows, loaded ahead of use.
    floatx16 acc2[MT2];
#pragma unroll
    for (int m = 0; m < MT2; ++m)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const floatx4 bv = *reinterpret_cast<const floatx4*>(a.b2 + (wave * MT2 + m) * 32 + 8 * j + hsel);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc2[m][4 * j + i] = bv[i];
        }
    u32x4 res[RV];
#pragma unroll
    for (int i = 0; i < RV; ++i) {
        const int q = tid + 256 * i, ch = q / kTH, gy = min(y0 + q % kTH, a.h - 1);  // rows past h are not stored
        res[i] = *reinterpret_cast<const u32x4*>(xb + ch * plane + static_cast<size_t>(gy) * a.w + x0);
    }
    // es aliases xs: every wave finished its depthwise reads before the
    // barrier above, so the expand results may overwrite the halo tile.
#pragma unroll
    for (int m = 0; m < MT1; ++m) {
        const int mt = wave * MT1 + m;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            std::uint16_t hv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                hv[i] = f2h(acc1[m][4 * j + i]);
                const float f = h2f(hv[i]);
                if (f < 0.0f) hv[i] = leaky_f16(f, a.alpha);
            }
            const std::uint32_t lo = hv[0] | (static_cast<std::uint32_t>(hv[1]) << 16);
            const std::uint32_t hi = hv[2] | (static_cast<std::uint32_t>(hv[3]) << 16);
            typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
            *reinterpret_cast<u32x2*>(&es[pl * EST + mt * 32 + 8 * j + hsel]) = u32x2{lo, hi};
        }
    }
    lds_barrier();

    // ---- 4. project 1x1 E -> C, round -> ys[channel][pixel] ---------------
#pragma unroll
    for (int ks = 0; ks < KS2; ++ks) {
        const half8 bv = *reinterpret_cast<const half8*>(&es[pl * EST + ks * 16 + koff]);
#pragma unroll
        for (int m = 0; m < MT2; ++m) {
            const int f = NF1 + ks * MT2 + m;
            const u32x4 av = ring[f % kRing];
            if (f + kRing < NF) ring[f % kRing] = frag(f + kRing);
            acc2[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, av), bv, acc2[m], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    // ys aliases ds, which no wave reads after the expand stage.
#pragma unroll
    for (int m = 0; m < MT2; ++m) {
        const int mt = wave * MT2 + m;
#pragma unroll
        for (int r = 0; r < 16; ++r)
            ys[(mt * 32 + 8 * (r >> 2) + hsel + (r & 3)) * kYS + pl] = f2h(acc2[m][r]);
    }
    lds_barrier();

    // ---- 5. residual add, 16-byte rows out ------------------------------
    std::uint16_t* yb = a.y + static_cast<size_t>(b) * C * plane;
#pragma unroll
    for (int i = 0; i < RV; ++i) {
        const int q = tid + 256 * i, ch = q / kTH, row = q % kTH, gy = y0 + row;
        if (gy >= a.h) continue;
        const u32x4 pv = *reinterpret_cast<const u32x4*>(&ys[ch * kYS + row * kTW]);
        u32x4 o;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const std::uint32_t lo = f2h(lo_h(pv[k]) + lo_h(res[i][k]));
            const std::uint32_t hi = f2h(hi_h(pv[k]) + hi_h(res[i][k]));
            o[k] = lo | (hi << 16);
        }
        *reinterpret_cast<u32x4*>(yb + ch * plane + static_cast<size_t>(gy) * a.w + x0) = o;
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
                      d->h, d->w, (d->w + kTW - 1) / kTW, 0, 0, d->alpha};
        a.tiles = a.tiles_x * ((d->h + kTH - 1) / kTH);
        const long long nwg = static_cast<long long>(a.tiles) * d->n;
        if (nwg > 0x7FFFFFFF) throw std::runtime_error("dwblock: grid too large");
        a.nwg = static_cast<int>(nwg);
        const dim3 grid(static_cast<unsigned>(a.nwg));
        if (d->c == 256 && d->e == 512) launch<256, 512>(a, grid, to_stream(s));
        else if (d->c == 128 && d->e == 256) launch<128, 256>(a, grid, to_stream(s));
        else launch<128, 512>(a, grid, to_stream(s));
        check(hipGetLastError(), "dwblock launch");
    });
}

}  // extern "C"
