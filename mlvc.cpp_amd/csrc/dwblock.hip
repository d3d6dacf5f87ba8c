// Fused depthwise-separable residual block on gfx950:
//
//   d = fp16(DW3x3(x) + b0)                     (bias-seeded FMA taps, (ky,kx) order)
//   e = fp16(LeakyReLU(fp16(W1 d + b1)))        (1x1 C -> E, MFMA)
//   y = fp16(fp16(W2 e + b2) + x)               (1x1 E -> C, MFMA, residual)
//
// Same rounding points as the unfused schedule (the reference runs DW, a
// conv with a LeakyReLU epilogue and a conv with a residual epilogue:
// backends/cpu/src/kernels_x86_avx2.cpp:237-302, kernels_scalar.cpp:178-192),
// but d and e never leave the chip. One workgroup owns a 4x8 pixel tile and
// all channels; at 1920x1088 / 16 that is one workgroup per CU, so the
// kernel is bound by how fast each CU streams the 2*C*E weight halves and by
// the per-pixel VALU work, not by MFMA issue. It is organised around that:
//   * 8 waves (2 per SIMD) for C = 256, so one wave's VALU work and waits
//     overlap the other's MFMAs;
//   * every wave runs ONE register ring of kRing weight fragments (16 bytes
//     per lane, pre-packed in A-fragment order) through both GEMMs, filled
//     between the depthwise rows, so W1 and then W2 are in flight from the
//     depthwise stage to the last MFMA, across the barriers (LDS-only fences);
//   * the input tile (6 rows x 24 columns of every channel: the 4x8 tile,
//     its halo and 8-column alignment) is staged into LDS by coalesced
//     16-byte loads, consecutive lanes reading consecutive 16-byte pieces of
//     one channel row. Loading it per channel instead (lane = channel) made
//     every load instruction touch 64 cache lines, and issuing them took a
//     quarter of the kernel. Two threads per channel then run the depthwise
//     taps from the staged rows; taps outside the image are skipped, so what
//     the range-checked loads return there is unused. The residual is read
//     from the same staged tile;
//   * accumulators are seeded with the bias (float4 loads issued at start);
//   * LeakyReLU for 0 <= alpha <= 1 is max(fp16(v), fp16(v * alpha)) on
//     packed halves (rounding is monotonic, so this equals the reference's
//     select), with the product rounded to FP32 first;
//   * the project result is rounded into LDS as [channel][pixel] and leaves
//     as 16-byte rows with the residual added from the staged tile.
// Chained blocks hand their activations over channel-last: a block whose
// output feeds only the next block writes it [n][h][w][C] (OUT_NHWC), and
// that block stages it (IN_NHWC) as 16-byte pieces of 8 channels of one
// pixel. Its halo is then the 6 x 10 pixels it needs (60 x C x 2 bytes,
// 240 cache lines at C = 256) instead of 6 rows x 24 columns of every
// channel (74 KB, about 2.2k cache lines). Arithmetic and rounding are the
// same in every layout.
// LDS: x[channel][6 rows][24 columns] (+8 halves per channel) or, channel-
// last, x[6 rows][10 pixels][C + 8]; d[pixel][C + 8] (later reused as
// y[channel][pixel], or y[pixel][C + 8] for a channel-last output) and
// e[pixel][E + 8]. Requires W % 8 == 0 (16-byte rows).

#include "common.hpp"
#include "mlvc_hip_device.h"

#include <cstring>

namespace mlvc_hip {
namespace {

constexpr int kTH = 4, kTW = 8, kP = kTH * kTW;  // 32 pixels per workgroup
constexpr int kYS = kP + 8;                       // y staging row stride (halves)
#ifndef MLVC_DW_RING
#define MLVC_DW_RING 24
#endif
constexpr int kRing = MLVC_DW_RING;               // weight fragments in flight per wave
#ifndef MLVC_DW_EARLY
#define MLVC_DW_EARLY 8
#endif
// Ring slots filled before the depthwise stage; the rest are requested
// between its rows. A wave stalls at a load while the memory request queue
// is full, so fragments requested up front delay the start of its
// depthwise work; requested between the depthwise rows, they keep the weight
// stream going while the VALU works (24 slots, none up front: 12.3-14.1 to
// 11.8-13.0 us per block with the 74 KB NCHW input tile). With the 30 KB
// channel-last tile, 8 of them up front: 10.44 -> 10.27 us.
constexpr int kEarly = MLVC_DW_EARLY;
constexpr int kXR = kTH + 2, kXW = kTW + 16;      // staged input rows and columns (x0 - 8 .. x0 + kTW + 7)
constexpr int kXP = kTW + 2;                      // channel-last staging: pixels x0 - 1 .. x0 + kTW per row
// Halves per staged channel: 304 bytes, 76 dwords, so 16 lanes reading 16
// bytes at the same offset of 16 consecutive channels hit distinct banks.
constexpr int kXCS = kXR * kXW + 8;
constexpr int kRawBufferFlags = 0x00020000;       // raw buffer resource word 3 (gfx950)
constexpr int kOutOfRange = 0x40000000;           // byte offset past every staged tensor (< 2^30 bytes)

template <int C, int E>
struct BlockCfg {
    static constexpr int WAVES = C >= 256 ? 8 : 4;
    static constexpr int T = 64 * WAVES;
    static constexpr int MT1 = E / 32 / WAVES, MT2 = C / 32 / WAVES;  // m-tiles per wave
    static constexpr int KS1 = C / 16, KS2 = E / 16;
    static constexpr int NF1 = MT1 * KS1, NF = NF1 + MT2 * KS2;       // fragments per wave
    static constexpr int TPC = T / C;                                 // depthwise threads per channel
    static constexpr int ORT = kTH / TPC;                             // depthwise output rows per thread
    static constexpr int RV = C * kTH / T;                            // output rows (16 B) per thread
    static constexpr int DST = C + 8, EST = E + 8;
    static constexpr int XPS = C + 8;                                 // channel-last staging: halves per pixel
    static constexpr int XN_PIECES = kXR * kXP * 4;                   // its 16-byte pieces per wave (32 channels)
    static constexpr int XNU = (XN_PIECES + 63) / 64;                 // per lane
    static constexpr int DS_HALVES = kP * DST > C * kYS ? kP * DST : C * kYS;
    static constexpr int XUNITS = C * kXR * (kXW / 8);                // 16-byte pieces of the staged tile
    static constexpr int XU = (XUNITS + T - 1) / T;                   // per thread
    static constexpr int TAP_PIECES = C * 9 * 2 / 16;                 // 16-byte pieces of the depthwise taps
    static constexpr int WTAP = TAP_PIECES / WAVES;                   // per wave (32 channels)
    static_assert(C * 9 * 2 % 16 == 0 && TAP_PIECES <= T && WTAP <= 64, "tap staging");
    // Wave w stages and runs the depthwise taps of channels 32w .. 32w + 31.
    static_assert(C == 32 * WAVES && TPC == 2 && XUNITS == XU * T, "per-wave channel slices");
    static_assert(C % 128 == 0 && E % 128 == 0 && MT1 >= 1 && MT2 >= 1, "channel counts");
    static_assert(TPC * ORT == kTH && C * kTH % T == 0, "thread mapping");
};

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

template <int C, int E, int MODE, bool IN_NHWC, bool OUT_NHWC>
__global__ __launch_bounds__((BlockCfg<C, E>::T)) void dwblock_kernel(DwBlockArgs a)
{
    using B = BlockCfg<C, E>;
    constexpr int DST = B::DST, EST = B::EST, MT1 = B::MT1, MT2 = B::MT2, KS1 = B::KS1, KS2 = B::KS2;
    constexpr int NF1 = B::NF1, NF = B::NF, ORT = B::ORT, RV = B::RV, T = B::T, XPS = B::XPS;
    constexpr int XS_HALVES = IN_NHWC ? kXR * kXP * XPS : C * kXCS;
    __shared__ __attribute__((aligned(16))) std::uint16_t es[kP * EST];
    __shared__ __attribute__((aligned(16))) std::uint16_t dys[B::DS_HALVES];
    // x[channel][row][column], or channel-last x[row][pixel][channel]
    __shared__ __attribute__((aligned(16))) std::uint16_t xs[XS_HALVES];
    __shared__ __attribute__((aligned(16))) std::uint16_t taps[C * 9];  // depthwise taps [channel][ky][kx]
    std::uint16_t* const ds = dys;  // d[pixel][C + 8]
    std::uint16_t* const ys = dys;  // y[channel][kYS], after the expand stage

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Each XCD runs a contiguous band of tiles, so the halo rows it loads
    // and the residual it re-reads stay in its own L2.
    const int item = xcd_order(blockIdx.x, a.nwg), tile = item % a.tiles, b = item / a.tiles;
    const int x0 = (tile % a.tiles_x) * kTW, y0 = (tile / a.tiles_x) * kTH;
    const size_t plane = static_cast<size_t>(a.h) * a.w;
    const std::uint16_t* xb = a.x + static_cast<size_t>(b) * C * plane;
    const u32x4* w1 = reinterpret_cast<const u32x4*>(a.w1);
    const u32x4* w2 = reinterpret_cast<const u32x4*>(a.w2);
    const int koff = (lane >> 5) * 8, pl = lane & 31, hsel = 4 * (lane >> 5);

    // Fragment f of this wave's stream: W1 in (k-step, m-tile) order, then
    // W2. The packing puts one k-step's fragments of all m-tiles next to each
    // other, so the loads in flight across the waves of every CU cover
    // contiguous bytes rather than one piece every 16 KB.
    auto frag = [&](int f) -> u32x4 {
        if (f < NF1) return w1[((f / MT1) * (E / 32) + wave * MT1 + f % MT1) * 64 + lane];
        f -= NF1;
        return w2[((f / MT2) * (C / 32) + wave * MT2 + f % MT2) * 64 + lane];
    };
    // ---- 1. input tile into LDS, coalesced --------------------------------
    // Piece u: 8 columns (x0 - 8 + 8k .. + 7) of staged row r (image row
    // y0 - 1 + r) of channel c; k fastest, then r, then c. The whole byte
    // offset goes in the VGPR operand: the range check applies to that
    // operand alone, not to the SGPR offset. Pieces outside the image get an
    // offset past the end (zeros); the taps that would read them are skipped.
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<std::uint16_t*>(xb), 0, static_cast<int>(C * plane * 2), kRawBufferFlags);
    // Wave w loads the pieces of channels 32w .. 32w + 31 (64 consecutive
    // pieces per instruction, as above) and its depthwise threads use only
    // those channels: thread (c, g), c = 32w + lane % 32, row group
    // g = lane / 32. So the staged tile needs no workgroup barrier before the
    // depthwise stage.
    // Channel-last: piece u of wave w is channels 32w + 8 (u % 4) .. + 7 of
    // staged pixel u / 4 (row-major over 6 rows x 10 pixels, image pixel
    // (y0 - 1 + row, x0 - 1 + column)), so four lanes read 64 contiguous
    // bytes of one pixel.
    constexpr int XU = IN_NHWC ? B::XNU : B::XU;
    u32x4 xp[XU];
#pragma unroll
    for (int i = 0; i < XU; ++i) {
        if constexpr (IN_NHWC) {
            const int u = lane + 64 * i, pix = u >> 2, sub = u & 3, r = pix / kXP, px = pix % kXP;
            const int iy = y0 - 1 + r, ix = x0 - 1 + px;
            const bool ok = u < B::XN_PIECES && iy >= 0 && iy < a.h && ix >= 0 && ix < a.w;
            xp[i] = __builtin_amdgcn_raw_buffer_load_b128(
                rx, ok ? ((iy * a.w + ix) * C + 32 * wave + 8 * sub) * 2 : kOutOfRange, 0, 0);
        } else {
            const int u = wave * 64 * B::XU + lane + 64 * i, k = u % (kXW / 8), r = (u / (kXW / 8)) % kXR,
                      ch = u / ((kXW / 8) * kXR);
            const int iy = y0 - 1 + r, ix = x0 - 8 + 8 * k;
            const bool ok = iy >= 0 && iy < a.h && ix >= 0 && ix < a.w;
            xp[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? ((ch * a.h + iy) * a.w + ix) * 2 : kOutOfRange, 0, 0);
        }
    }
    const int c = 32 * wave + (lane & 31), g = lane >> 5;
    // The taps of this wave's channels as 16-byte pieces, staged with the
    // tile (a thread's own nine taps per channel would be nine loads, each
    // touching as many cache lines as the wave has channels).
    u32x4 tp = {0u, 0u, 0u, 0u};
    if (lane < B::WTAP) tp = reinterpret_cast<const u32x4*>(a.dw_w)[wave * B::WTAP + lane];
    const float bdw = a.dw_b[c];
    // The depthwise operands are requested first: loads complete in issue
    // order for the wait counter, so the staging below waits for them only,
    // and the depthwise stage runs while the weight ring is still in flight.
    __builtin_amdgcn_sched_barrier(0);

    // The weight ring, then the expand bias.
    u32x4 ring[kRing];
#pragma unroll
    for (int f = 0; f < kEarly; ++f) ring[f] = f < NF ? frag(f) : u32x4{0u, 0u, 0u, 0u};

    // Expand bias (lane rows 8j + hsel + (0..3)), requested with the first
    // depthwise row's ring fragments rather than up front.
    floatx4 b1v[MT1][4];

    // The scheduler would otherwise sink the ring loads down to their MFMAs
    // (minimising live registers) and serialise the stream on L2 latency.
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int i = 0; i < XU; ++i) {
        if constexpr (IN_NHWC) {
            const int u = lane + 64 * i, pix = u >> 2, sub = u & 3;
            if (u < B::XN_PIECES) *reinterpret_cast<u32x4*>(&xs[pix * XPS + 32 * wave + 8 * sub]) = xp[i];
        } else {
            const int u = wave * 64 * B::XU + lane + 64 * i, k = u % (kXW / 8), r = (u / (kXW / 8)) % kXR,
                      ch = u / ((kXW / 8) * kXR);
            *reinterpret_cast<u32x4*>(&xs[ch * kXCS + r * kXW + 8 * k]) = xp[i];
        }
    }
    if (lane < B::WTAP) *reinterpret_cast<u32x4*>(&taps[(wave * B::WTAP + lane) * 8]) = tp;
    // Lanes read what other lanes of this wave wrote (LDS runs a wave's
    // instructions in order).
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
    std::uint16_t wdw[9];
#pragma unroll
    for (int t = 0; t < 9; ++t) wdw[t] = taps[c * 9 + t];
    // This thread's halo rows from the staged tile: per row the dword of
    // columns x0-2, x0-1, the 16 bytes x0 .. x0+7 and the dword x0+8, x0+9.
    // Channel-last: the 10 pixels of each row, one half each.
    const int row0 = g * ORT;  // staged row of image row y0 + g*ORT - 1
    std::uint32_t xl[ORT + 2], xr[ORT + 2];
    u32x4 xm[ORT + 2];
    std::uint16_t xn[IN_NHWC ? ORT + 2 : 1][kXP];
#pragma unroll
    for (int r = 0; r < ORT + 2; ++r) {
        if constexpr (IN_NHWC) {
#pragma unroll
            for (int px = 0; px < kXP; ++px) xn[r][px] = xs[((row0 + r) * kXP + px) * XPS + c];
        } else {
            const std::uint16_t* rowp = &xs[c * kXCS + (row0 + r) * kXW];
            xl[r] = *reinterpret_cast<const std::uint32_t*>(rowp + 6);
            xm[r] = *reinterpret_cast<const u32x4*>(rowp + 8);
            xr[r] = *reinterpret_cast<const std::uint32_t*>(rowp + 16);
        }
    }

    {
        const bool left = x0 > 0, right = x0 + kTW < a.w;
        float d[ORT][kTW];
#pragma unroll
        for (int r = 0; r < ORT; ++r)
#pragma unroll
            for (int px = 0; px < kTW; ++px) d[r][px] = bdw;
#pragma unroll
        for (int r = 0; r < ORT; ++r) {
            const int gy = y0 + g * ORT + r;
#pragma unroll
            for (int ky = 0; ky < 3; ++ky) {
                if constexpr (kRing > kEarly) {
                    constexpr int kLate = kRing - kEarly, kPer = (kLate + 3 * ORT - 1) / (3 * ORT);
                    const int it = r * 3 + ky;
#pragma unroll
                    for (int q = 0; q < kPer; ++q) {
                        const int f = kEarly + it * kPer + q;
                        if (f < kRing) ring[f] = f < NF ? frag(f) : u32x4{0u, 0u, 0u, 0u};
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (r == 0 && ky == 0) {
#pragma unroll
                    for (int m = 0; m < MT1; ++m)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            b1v[m][j] = *reinterpret_cast<const floatx4*>(a.b1 + (wave * MT1 + m) * 32 + 8 * j + hsel);
                    __builtin_amdgcn_sched_barrier(0);
                }
                const int iy = gy + ky - 1;
                if (iy < 0 || iy >= a.h) continue;
                const int rr = r + ky;
                float xv[kTW + 2];
                if constexpr (IN_NHWC) {
#pragma unroll
                    for (int px = 0; px < kXP; ++px) xv[px] = h2f(xn[rr][px]);
                } else {
                    xv[0] = hi_h(xl[rr]);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        xv[1 + 2 * i] = lo_h(xm[rr][i]);
                        xv[2 + 2 * i] = hi_h(xm[rr][i]);
                    }
                    xv[kTW + 1] = lo_h(xr[rr]);
                }
#pragma unroll
                for (int px = 0; px < kTW; ++px)
#pragma unroll
                    for (int kx = 0; kx < 3; ++kx) {
                        if (px + kx == 0 && !left) continue;
                        if (px + kx == kTW + 1 && !right) continue;
                        d[r][px] = fmaf(xv[px + kx], h2f(wdw[ky * 3 + kx]), d[r][px]);
                    }
            }
        }
#pragma unroll
        for (int r = 0; r < ORT; ++r)
#pragma unroll
            for (int px = 0; px < kTW; ++px) ds[((g * ORT + r) * kTW + px) * DST + c] = f2h(d[r][px]);
    }
    lds_barrier();

    // ---- 2. expand 1x1 C -> E, round, LeakyReLU, round -> es --------------
    floatx16 acc1[MT1];
#pragma unroll
    for (int m = 0; m < MT1; ++m)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc1[m][4 * j + i] = b1v[m][j][i];
    // The B fragment of step ks + 1 is read from LDS during step ks (the
    // scheduling barrier that keeps the ring refills in place would otherwise
    // leave each read's latency in front of its MFMAs).
    half8 bnext = *reinterpret_cast<const half8*>(&ds[pl * DST + koff]);
#pragma unroll
    for (int ks = 0; ks < KS1; ++ks) {
        const half8 bv = bnext;
        if (ks + 1 < KS1) bnext = *reinterpret_cast<const half8*>(&ds[pl * DST + (ks + 1) * 16 + koff]);
#pragma unroll
        for (int m = 0; m < MT1; ++m) {
            const int f = ks * MT1 + m;
            const u32x4 av = ring[f % kRing];
            if (f + kRing < NF) ring[f % kRing] = frag(f + kRing);
            acc1[m] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, av), bv, acc1[m], 0, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    // Project accumulators seeded with b2.
    floatx16 acc2[MT2];
#pragma unroll
    for (int m = 0; m < MT2; ++m)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const floatx4 bv = *reinterpret_cast<const floatx4*>(a.b2 + (wave * MT2 + m) * 32 + 8 * j + hsel);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc2[m][4 * j + i] = bv[i];
        }
    {
        typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
        for (int m = 0; m < MT1; ++m) {
            const int mt = wave * MT1 + m;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const std::uint32_t lo = epi_pair<MODE>(acc1[m][4 * j], acc1[m][4 * j + 1], a.alpha);
                const std::uint32_t hi = epi_pair<MODE>(acc1[m][4 * j + 2], acc1[m][4 * j + 3], a.alpha);
                *reinterpret_cast<u32x2*>(&es[pl * EST + mt * 32 + 8 * j + hsel]) = u32x2{lo, hi};
            }
        }
    }
    lds_barrier();

    // ---- 3. project 1x1 E -> C, round -> ys[channel][pixel] ---------------
    bnext = *reinterpret_cast<const half8*>(&es[pl * EST + koff]);
#pragma unroll
    for (int ks = 0; ks < KS2; ++ks) {
        const half8 bv = bnext;
        if (ks + 1 < KS2) bnext = *reinterpret_cast<const half8*>(&es[pl * EST + (ks + 1) * 16 + koff]);
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
        if constexpr (OUT_NHWC) {
            // y[pixel][channel]: the lane's four consecutive channels per j.
            typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const std::uint32_t lo = f2h(acc2[m][4 * j]) | (static_cast<std::uint32_t>(f2h(acc2[m][4 * j + 1])) << 16);
                const std::uint32_t hi = f2h(acc2[m][4 * j + 2]) | (static_cast<std::uint32_t>(f2h(acc2[m][4 * j + 3])) << 16);
                *reinterpret_cast<u32x2*>(&ys[pl * DST + mt * 32 + 8 * j + hsel]) = u32x2{lo, hi};
            }
        } else {
#pragma unroll
            for (int r = 0; r < 16; ++r)
                ys[(mt * 32 + 8 * (r >> 2) + hsel + (r & 3)) * kYS + pl] = f2h(acc2[m][r]);
        }
    }
    // Each wave writes out the channels it computed, so it waits for its own
    // LDS writes only, not for the other waves (LDS runs a wave's
    // instructions in order).
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");

    // ---- 4. residual add, 16-byte rows out ------------------------------
    static_assert(MT2 * 32 * kTH == 64 * RV, "output rows per lane");
    std::uint16_t* yb = a.y + static_cast<size_t>(b) * C * plane;
    // The residual x of 8 consecutive halves of the output piece: 8 channels
    // of one pixel (channel-last output) or 8 pixels of one channel.
    auto residual = [&](int ch, int row, int px) -> u32x4 {
        std::uint16_t v[8];
        if constexpr (IN_NHWC && OUT_NHWC) {
            return *reinterpret_cast<const u32x4*>(&xs[((row + 1) * kXP + px + 1) * XPS + ch]);
        } else if constexpr (IN_NHWC) {
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = xs[((row + 1) * kXP + px + 1 + k) * XPS + ch];
        } else if constexpr (OUT_NHWC) {
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] = xs[(ch + k) * kXCS + (row + 1) * kXW + 8 + px];
        } else {
            return *reinterpret_cast<const u32x4*>(&xs[ch * kXCS + (row + 1) * kXW + 8 + px]);
        }
        u32x4 r;
#pragma unroll
        for (int k = 0; k < 4; ++k) r[k] = v[2 * k] | (static_cast<std::uint32_t>(v[2 * k + 1]) << 16);
        return r;
    };
    if constexpr (OUT_NHWC) {
        constexpr int PER = MT2 * 4;         // 16-byte pieces per pixel of this wave's channels
        constexpr int PV = PER * kP / 64;    // per lane
        static_assert(PER * kP % 64 == 0, "output pieces per lane");
#pragma unroll
        for (int i = 0; i < PV; ++i) {
            const int v = lane + 64 * i, p = v / PER, ch = wave * MT2 * 32 + 8 * (v % PER);
            const int row = p / kTW, px = p % kTW, gy = y0 + row;
            if (gy >= a.h) continue;
            const u32x4 pv = *reinterpret_cast<const u32x4*>(&ys[p * DST + ch]);
            const u32x4 rv = residual(ch, row, px);
            u32x4 o;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const std::uint32_t lo = f2h(lo_h(pv[k]) + lo_h(rv[k]));
                const std::uint32_t hi = f2h(hi_h(pv[k]) + hi_h(rv[k]));
                o[k] = lo | (hi << 16);
            }
            *reinterpret_cast<u32x4*>(yb + (static_cast<size_t>(gy) * a.w + x0 + px) * C + ch) = o;
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < RV; ++i) {
        const int q = lane + 64 * i, ch = wave * MT2 * 32 + q / kTH, row = q % kTH, gy = y0 + row;
        if (gy >= a.h) continue;
        const u32x4 pv = *reinterpret_cast<const u32x4*>(&ys[ch * kYS + row * kTW]);
        const u32x4 rv = residual(ch, row, 0);
        u32x4 o;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const std::uint32_t lo = f2h(lo_h(pv[k]) + lo_h(rv[k]));
            const std::uint32_t hi = f2h(hi_h(pv[k]) + hi_h(rv[k]));
            o[k] = lo | (hi << 16);
        }
        *reinterpret_cast<u32x4*>(yb + ch * plane + static_cast<size_t>(gy) * a.w + x0) = o;
    }
}

template <int C, int E, bool IN_NHWC, bool OUT_NHWC>
void launch_layout(const DwBlockArgs& a, dim3 grid, hipStream_t s)
{
    // LeakyReLU form fixed at compile time (max form for 0 <= alpha <= 1).
    if (epi_mode(1, a.alpha) == 1)
        hipLaunchKernelGGL((dwblock_kernel<C, E, 1, IN_NHWC, OUT_NHWC>), grid, dim3(BlockCfg<C, E>::T), 0, s, a);
    else
        hipLaunchKernelGGL((dwblock_kernel<C, E, 2, IN_NHWC, OUT_NHWC>), grid, dim3(BlockCfg<C, E>::T), 0, s, a);
}

template <int C, int E>
void launch(const DwBlockArgs& a, bool in_nhwc, bool out_nhwc, dim3 grid, hipStream_t s)
{
    if (in_nhwc && out_nhwc) launch_layout<C, E, true, true>(a, grid, s);
    else if (in_nhwc) launch_layout<C, E, true, false>(a, grid, s);
    else if (out_nhwc) launch_layout<C, E, false, true>(a, grid, s);
    else launch_layout<C, E, false, false>(a, grid, s);
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
        // [k-step][m-tile][lane][8]: lane l holds W[mt*32 + l%32][ks*16 + 8*(l/32) + j].
        for (int ks = 0; ks < k / 16; ++ks)
            for (int mt = 0; mt < m / 32; ++mt)
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
        if ((reinterpret_cast<std::uintptr_t>(d->dw_w) | reinterpret_cast<std::uintptr_t>(d->x) |
             reinterpret_cast<std::uintptr_t>(d->y)) & 15u)
            throw std::runtime_error("dwblock: x, y and the depthwise taps must be 16-byte aligned");
        if (static_cast<std::uint64_t>(d->c) * d->h * d->w * 2 + 64 >= static_cast<std::uint64_t>(kOutOfRange))
            throw std::runtime_error("dwblock: image too large for 32-bit buffer offsets");
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
        if ((d->in_nhwc != 0 && d->in_nhwc != 1) || (d->out_nhwc != 0 && d->out_nhwc != 1))
            throw std::runtime_error("dwblock: in_nhwc / out_nhwc must be 0 or 1");
        if (d->x == d->y) throw std::runtime_error("dwblock: x and y must not alias (workgroups read their neighbours' x)");
        const bool in = d->in_nhwc != 0, out = d->out_nhwc != 0;
        if (d->c == 256 && d->e == 512) launch<256, 512>(a, in, out, grid, to_stream(s));
        else if (d->c == 128 && d->e == 256) launch<128, 256>(a, in, out, grid, to_stream(s));
        else launch<128, 512>(a, in, out, grid, to_stream(s));
        check(hipGetLastError(), "dwblock launch");
    });
}

}  // extern "C"
