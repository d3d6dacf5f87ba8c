// Fused conv pair on gfx950 MFMA:
//
//   t = epi_a(fp16(Wa * x + ba))          3x3, stride 1, pad 1, oca = 64
//   y = epi_b(fp16(Wb [t ; r] + bb))      1x1 over the channel CONCAT of t and r
//
// This is the frame stem of the MLVC-shaped graphs (unshuffled frame -> 3x3 ->
// concat with the recurrent reference -> 1x1), which otherwise writes t to HBM
// and reads it straight back. One workgroup (4 waves) owns a TH x TW pixel
// tile and every channel:
//   phase A  the 3x3 conv exactly as conv_mfma_kernel does it for BM = 64
//            (same LDS staging, same K order: 16-channel chunk, then tap);
//   P tile   r is staged into P[pixel][64, 128) with 16-byte loads issued
//            with the first input chunk and an 8x8 register transpose; after
//            phase A the rounded, activated t is written channel-last into
//            P[pixel][0, 64) (a lane's 4 consecutive accumulator rows are 4
//            consecutive channels of one pixel: one 8-byte write);
//   phase B  the 1x1 GEMM reads its B fragments from P and its weight
//            fragments from registers (the same 16 KB for every wave, loaded
//            while phase A's results are written),
//            K in 16-channel steps over [t ; r] as the unfused 1x1 kernel;
//   out      rounded, activated, through an LDS [channel][pixel] tile to
//            16-byte NCHW rows.
// Rounding points and K orders are those of the unfused kernels, so the
// results are bit-identical to running them separately.

#include "conv_kernel.hpp"

namespace mlvc_hip {
namespace conv {
namespace {

struct PairArgs {
    const std::uint16_t* x;
    const std::uint16_t* r;
    const std::uint16_t* wa;
    const float* ba;
    const std::uint16_t* wb;
    const float* bb;
    std::uint16_t* y;
    int ica, h, w, nchunks;
    int epi_a, epi_b;
    float alpha_a, alpha_b;
    int tiles_x, tiles, nwg;
};

template <int TH_, int TW_, int STG_>
struct PairCfg {
    static constexpr int TH = TH_, TW = TW_, STG = STG_;  // STG 1: plain input, 2: SPACE_TO_DEPTH(2) source
    static constexpr int OCA = 64, CR = 64, OCB = 64, KB = OCA + CR;
    static constexpr int kThreads = 256;
    static constexpr int BN = TH * TW, WN = BN / 4, NT = WN / 32;
    static constexpr int MTA = OCA / 32, MTB = OCB / 32, KSB = KB / 16;
    static constexpr int KC = 16;
    static constexpr int IH_T = TH + 2, IW_T = TW + 2;
    static constexpr int NSEG = (IW_T + 14) / 8, IW_S = NSEG * 8;
    static constexpr int PST = KC + 8;
    static constexpr int ROW = IW_S * PST + 8;
    static constexpr int IN_LDS = IH_T * ROW;
    static constexpr int WA_LDS = 9 * MTA * 64 * 8;  // halves per chunk
    static constexpr int WA_VEC = WA_LDS / 8, WA_PER_T = (WA_VEC + kThreads - 1) / kThreads;
    static constexpr int A_LDS = IN_LDS + WA_LDS;
    static constexpr int EPI_ROW = BN + 8;
    static constexpr int EPI_LDS = OCB * EPI_ROW;
    static constexpr int P0 = A_LDS > EPI_LDS ? A_LDS : EPI_LDS;  // P follows the phase A / output region
    static constexpr int PS = KB + 8;                              // P row (one pixel), halves
    static constexpr int LDS = P0 + BN * PS;
    static constexpr int UNITS = STG == 1 ? (KC / 8) * IH_T * NSEG : IH_T * NSEG;
    static constexpr int UNITS_PER_T = (UNITS + kThreads - 1) / kThreads;
    static constexpr int RUNITS = (CR / 8) * (BN / 8);  // r staging: 8 channels x 8 pixels
    static constexpr int RUNITS_PER_T = (RUNITS + kThreads - 1) / kThreads;
    static_assert(WN % 32 == 0 && TW % 8 == 0 && LDS * 2 <= 160 * 1024 && P0 % 8 == 0, "pair tile");
    __device__ static constexpr int at(int row, int x) { return row * ROW + x * PST; }
};

template <class C>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void conv_pair_kernel(PairArgs a)
{
    __shared__ __attribute__((aligned(16))) std::uint16_t lds[C::LDS];
    std::uint16_t* const in_s = lds;
    std::uint16_t* const wa_s = lds + C::IN_LDS;
    std::uint16_t* const ps = lds + C::P0;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int item = xcd_order(blockIdx.x, a.nwg), tile = item % a.tiles, b = item / a.tiles;
    const int tx0 = (tile % a.tiles_x) * C::TW, ty0 = (tile / a.tiles_x) * C::TH;
    const int iy0 = ty0 - 1, ix0 = tx0 - 1;
    const int xa = ix0 - (((ix0 % 8) + 8) % 8), col_off = ix0 - xa;
    const int koff = (lane >> 5) * 8, hsel = 4 * (lane >> 5);
    const std::uint32_t hw = static_cast<std::uint32_t>(a.h) * a.w, hw2 = hw * 2u;
    const bool max_a = a.alpha_a >= 0.0f && a.alpha_a <= 1.0f, max_b = a.alpha_b >= 0.0f && a.alpha_b <= 1.0f;

    // ---- phase A: 3x3 conv, BM = 64 --------------------------------------
    floatx16 acc[C::MTA][C::NT];
#pragma unroll
    for (int mt = 0; mt < C::MTA; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float bv = a.ba[mt * 32 + 8 * (r >> 2) + hsel + (r & 3)];
#pragma unroll
            for (int nt = 0; nt < C::NT; ++nt) acc[mt][nt][r] = bv;
        }
    // Raw buffer resource over this image's input (range-checked: padding
    // and channels past ica read zeros; whole offsets in the VGPR operand).
    const int csrc = C::STG == 2 ? a.ica / 4 : a.ica;
    const std::uint32_t plane_src = C::STG == 2 ? 4u * hw2 : hw2;  // bytes per source channel
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<std::uint16_t*>(a.x + static_cast<size_t>(b) * csrc * (plane_src / 2)), 0,
        static_cast<int>(csrc * plane_src), kRawBufferFlags);
    const int sw = C::STG == 2 ? a.w * 2 : a.w;
    std::uint32_t uoff[C::UNITS_PER_T];
    int uc8[C::UNITS_PER_T];
#pragma unroll
    for (int i = 0; i < C::UNITS_PER_T; ++i) {
        const int u = tid + i * C::kThreads;
        const int yi = u % C::IH_T, sg = (u / C::IH_T) % C::NSEG;
        const int iy = iy0 + yi, ix = xa + sg * 8;
        const bool ok = u < C::UNITS && iy >= 0 && iy < a.h && ix >= 0 && ix < a.w;
        uoff[i] = ok ? (C::STG == 2 ? static_cast<std::uint32_t>(2 * iy * sw + 2 * ix) * 2u
                                    : static_cast<std::uint32_t>(iy * a.w + ix) * 2u)
                     : kOutOfRange;
        uc8[i] = u / (C::IH_T * C::NSEG);
    }
    u32x4 vin[C::UNITS_PER_T][C::STG == 2 ? 16 : 8];
    u32x4 wreg[C::WA_PER_T];
    auto fetch = [&](int chunk) {
        const int c0 = chunk * C::KC;
#pragma unroll
        for (int i = 0; i < C::UNITS_PER_T; ++i) {
            if constexpr (C::STG == 2) {
                // Source channels c0/4 .. c0/4 + 3, rows 2iy and 2iy+1, 32 bytes each.
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int dy = 0; dy < 2; ++dy)
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh) {
                            const std::uint32_t off =
                                uoff[i] == kOutOfRange
                                    ? kOutOfRange
                                    : uoff[i] + static_cast<std::uint32_t>(c0 / 4 + q) * plane_src +
                                          static_cast<std::uint32_t>(dy * sw * 2 + hh * 16);
                            vin[i][(q * 2 + dy) * 2 + hh] = __builtin_amdgcn_raw_buffer_load_b128(rx, static_cast<int>(off), 0, 0);
                        }
            } else {
                const std::uint32_t base =
                    uoff[i] == kOutOfRange ? kOutOfRange : uoff[i] + static_cast<std::uint32_t>(c0 + uc8[i] * 8) * hw2;
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    vin[i][k] = __builtin_amdgcn_raw_buffer_load_b128(rx, static_cast<int>(base + k * hw2), 0, 0);
            }
        }
        const u32x4* ws = reinterpret_cast<const u32x4*>(a.wa + static_cast<size_t>(chunk) * C::WA_LDS);
#pragma unroll
        for (int i = 0; i < C::WA_PER_T; ++i) {
            const int e = tid + i * C::kThreads;
            if (e < C::WA_VEC) wreg[i] = ws[e];
        }
    };
    auto commit = [&]() {
#pragma unroll
        for (int i = 0; i < C::UNITS_PER_T; ++i) {
            const int u = tid + i * C::kThreads;
            if (u >= C::UNITS) continue;
            const int yi = u % C::IH_T, sg = (u / C::IH_T) % C::NSEG;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if constexpr (C::STG == 2) {
                    // Dword j%4 of source half j/4 is the (dx = 0, 1) pair of staged pixel j.
                    const int hh = j >> 2, wd = j & 3;
#pragma unroll
                    for (int g = 0; g < 2; ++g) {
                        const u32x4 t = {vin[i][((2 * g) * 2 + 0) * 2 + hh][wd], vin[i][((2 * g) * 2 + 1) * 2 + hh][wd],
                                         vin[i][((2 * g + 1) * 2 + 0) * 2 + hh][wd], vin[i][((2 * g + 1) * 2 + 1) * 2 + hh][wd]};
                        *reinterpret_cast<u32x4*>(&in_s[C::at(yi, sg * 8 + j) + g * 8]) = t;
                    }
                } else {
                    const bool up = j & 1;
                    const int wd = j >> 1;
                    const u32x4 t = {pack_half(vin[i][0][wd], vin[i][1][wd], up), pack_half(vin[i][2][wd], vin[i][3][wd], up),
                                     pack_half(vin[i][4][wd], vin[i][5][wd], up), pack_half(vin[i][6][wd], vin[i][7][wd], up)};
                    *reinterpret_cast<u32x4*>(&in_s[C::at(yi, sg * 8 + j) + uc8[i] * 8]) = t;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < C::WA_PER_T; ++i) {
            const int e = tid + i * C::kThreads;
            if (e < C::WA_VEC) reinterpret_cast<u32x4*>(wa_s)[e] = wreg[i];
        }
    };
    int pyi[C::NT], pxi[C::NT];
#pragma unroll
    for (int nt = 0; nt < C::NT; ++nt) {
        const int p = wave * C::WN + nt * 32 + (lane & 31);
        pyi[nt] = p / C::TW;
        pxi[nt] = p % C::TW + col_off;
    }
    // r (the second half of P) is loaded with the first input chunk and
    // committed with it, so its latency overlaps phase A's.
    const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<std::uint16_t*>(a.r + static_cast<size_t>(b) * C::CR * hw), 0, static_cast<int>(C::CR * hw2), kRawBufferFlags);
    u32x4 rv[C::RUNITS_PER_T][8];
#pragma unroll
    for (int i = 0; i < C::RUNITS_PER_T; ++i) {
        // Channel group fastest: 8 lanes write 8 different 16-byte slots of
        // one P row, free of bank conflicts.
        const int u = tid + i * C::kThreads;
        const int c8 = u % (C::CR / 8), pg = u / (C::CR / 8);
        const int oy = ty0 + (pg * 8) / C::TW, ox = tx0 + (pg * 8) % C::TW;
        const std::uint32_t base = u < C::RUNITS && oy < a.h && ox < a.w
                                       ? (static_cast<std::uint32_t>(c8 * 8) * hw + static_cast<std::uint32_t>(oy * a.w + ox)) * 2u
                                       : kOutOfRange;
#pragma unroll
        for (int k = 0; k < 8; ++k) rv[i][k] = __builtin_amdgcn_raw_buffer_load_b128(rr, static_cast<int>(base + k * hw2), 0, 0);
    }
    fetch(0);
    commit();
#pragma unroll
    for (int i = 0; i < C::RUNITS_PER_T; ++i) {
        const int u = tid + i * C::kThreads;
        if (u >= C::RUNITS) continue;
        const int c8 = u % (C::CR / 8), pg = u / (C::CR / 8);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const bool up = j & 1;
            const int wd = j >> 1;
            const u32x4 t = {pack_half(rv[i][0][wd], rv[i][1][wd], up), pack_half(rv[i][2][wd], rv[i][3][wd], up),
                             pack_half(rv[i][4][wd], rv[i][5][wd], up), pack_half(rv[i][6][wd], rv[i][7][wd], up)};
            *reinterpret_cast<u32x4*>(&ps[(pg * 8 + j) * C::PS + C::OCA + c8 * 8]) = t;
        }
    }
    __syncthreads();
    for (int chunk = 0; chunk < a.nchunks; ++chunk) {
        const bool more = chunk + 1 < a.nchunks;
        if (more) fetch(chunk + 1);
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
            const int ky = tap / 3, kx = tap % 3;
            half8 av[C::MTA], bv[C::NT];
#pragma unroll
            for (int mt = 0; mt < C::MTA; ++mt)
                av[mt] = *reinterpret_cast<const half8*>(&wa_s[((tap * C::MTA + mt) * 64 + lane) * 8]);
#pragma unroll
            for (int nt = 0; nt < C::NT; ++nt)
                bv[nt] = *reinterpret_cast<const half8*>(&in_s[C::at(pyi[nt] + ky, pxi[nt] + kx) + koff]);
#pragma unroll
            for (int mt = 0; mt < C::MTA; ++mt)
#pragma unroll
                for (int nt = 0; nt < C::NT; ++nt)
                    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[mt], bv[nt], acc[mt][nt], 0, 0, 0);
        }
        __syncthreads();
        if (more) {
            commit();
            __syncthreads();
        }
    }

    // 1x1 weight fragments (16 KB, the same for every wave: L1 hits), loaded
    // before t is written so their latency overlaps the epilogue and barrier.
    const u32x4* wb = reinterpret_cast<const u32x4*>(a.wb);
    u32x4 wbr[C::KSB][C::MTB];
#pragma unroll
    for (int ks = 0; ks < C::KSB; ++ks)
#pragma unroll
        for (int mt = 0; mt < C::MTB; ++mt) wbr[ks][mt] = wb[(ks * C::MTB + mt) * 64 + lane];

    // ---- t into P[pixel][0, 64): rounded, activated, 4 channels per write ----
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int mt = 0; mt < C::MTA; ++mt)
#pragma unroll
        for (int nt = 0; nt < C::NT; ++nt) {
            const int p = wave * C::WN + nt * 32 + (lane & 31);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float v0 = acc[mt][nt][4 * j], v1 = acc[mt][nt][4 * j + 1];
                const float v2 = acc[mt][nt][4 * j + 2], v3 = acc[mt][nt][4 * j + 3];
                const bool act = a.epi_a == MLVC_EPI_LEAKY_RELU;
                const std::uint32_t lo = act ? leaky_pair(v0, v1, a.alpha_a, max_a) : pack_f16(v0, v1);
                const std::uint32_t hi = act ? leaky_pair(v2, v3, a.alpha_a, max_a) : pack_f16(v2, v3);
                *reinterpret_cast<u32x2*>(&ps[p * C::PS + mt * 32 + 8 * j + hsel]) = u32x2{lo, hi};
            }
        }
    __syncthreads();

    // ---- phase B: 1x1 over [t ; r] ----------------------------------------
    floatx16 acc2[C::MTB][C::NT];
#pragma unroll
    for (int mt = 0; mt < C::MTB; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float bv = a.bb[mt * 32 + 8 * (r >> 2) + hsel + (r & 3)];
#pragma unroll
            for (int nt = 0; nt < C::NT; ++nt) acc2[mt][nt][r] = bv;
        }
#pragma unroll
    for (int ks = 0; ks < C::KSB; ++ks) {
        half8 av[C::MTB], bv[C::NT];
#pragma unroll
        for (int mt = 0; mt < C::MTB; ++mt) av[mt] = __builtin_bit_cast(half8, wbr[ks][mt]);
#pragma unroll
        for (int nt = 0; nt < C::NT; ++nt) {
            const int p = wave * C::WN + nt * 32 + (lane & 31);
            bv[nt] = *reinterpret_cast<const half8*>(&ps[p * C::PS + ks * 16 + koff]);
        }
#pragma unroll
        for (int mt = 0; mt < C::MTB; ++mt)
#pragma unroll
            for (int nt = 0; nt < C::NT; ++nt)
                acc2[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[mt], bv[nt], acc2[mt][nt], 0, 0, 0);
    }

    // ---- output: rounded into LDS [channel][pixel] (phase A region, free
    // since the barrier above), activated, 16-byte NCHW rows ---------------
#pragma unroll
    for (int mt = 0; mt < C::MTB; ++mt)
#pragma unroll
        for (int nt = 0; nt < C::NT; ++nt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int ocl = mt * 32 + 8 * (r >> 2) + hsel + (r & 3);
                const int pl = wave * C::WN + nt * 32 + (lane & 31);
                lds[ocl * C::EPI_ROW + pl] = f2h(acc2[mt][nt][r]);
            }
    __syncthreads();
    constexpr int GROUPS = C::BN / 8;
    for (int u = tid; u < C::OCB * GROUPS; u += C::kThreads) {
        const int g = u % GROUPS, oc = u / GROUPS;
        const int pl = g * 8, oy = ty0 + pl / C::TW, ox = tx0 + pl % C::TW;
        if (oy >= a.h || ox >= a.w) continue;
        u32x4 hv = *reinterpret_cast<const u32x4*>(&lds[oc * C::EPI_ROW + pl]);
        if (a.epi_b == MLVC_EPI_LEAKY_RELU) {
#pragma unroll
            for (int k = 0; k < 4; ++k) hv[k] = leaky_h2(hv[k], a.alpha_b, max_b);
        }
        *reinterpret_cast<u32x4*>(a.y + (static_cast<size_t>(b) * C::OCB + oc) * hw + static_cast<size_t>(oy) * a.w + ox) = hv;
    }
}

// Streaming form for a single input chunk (ica <= 16, as in the frame stem:
// 12 channels after SPACE_TO_DEPTH(2)). Same tile, K orders and rounding
// points as conv_pair_kernel (bit-identical results), organised so that HBM
// reads overlap compute instead of alternating with it:
//   * a persistent grid (two workgroups per CU) walks the tiles; the 3x3
//     weights stay in LDS and the 1x1 weight fragments in registers for the
//     whole walk;
//   * the input units and r of tile i + 1 are loaded into registers while
//     tile i is computed;
//   * each wave owns one row of 32 pixels: it stages that row's r into P
//     and writes its own t there, and phase B reads only those rows, so P
//     needs no barrier; the two barriers per tile guard the shared input
//     halo tile;
//   * phase B runs with the MFMA operands swapped (pixels as M, output
//     channels as N; the same products and K order, so the same bits), which
//     leaves 4 consecutive pixels of one channel in each lane: the rounded,
//     activated results go into the wave's (now dead) P rows as a
//     [channel][pixel] tile with 8-byte writes and leave as 16-byte rows.
template <class C, int EA, int EB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void conv_pair_stream_kernel(PairArgs a)
{
    static_assert(C::TW == 32 && C::TH == 4 && C::NT == 1 && C::WN == 32, "one 32-pixel row per wave");
    constexpr int IN0 = C::WA_LDS, PS0 = C::WA_LDS + C::IN_LDS, LDS_S = PS0 + C::BN * C::PS;
    constexpr int XUNITS = 2 * C::IH_T * C::NSEG;  // 8 loads each
    constexpr int kStgRow = 40;                    // output staging row (one channel, 32 pixels), halves
    static_assert(C::OCB * kStgRow <= 32 * C::PS, "staging fits a wave's P rows");
    static_assert(XUNITS <= C::kThreads && IN0 % 8 == 0 && PS0 % 8 == 0 && LDS_S * 2 <= 80 * 1024, "stream tile");
    __shared__ __attribute__((aligned(16))) std::uint16_t lds[LDS_S];
    std::uint16_t* const wa_s = lds;
    std::uint16_t* const in_s = lds + IN0;
    std::uint16_t* const ps = lds + PS0;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int koff = (lane >> 5) * 8, hsel = 4 * (lane >> 5);
    const std::uint32_t hw = static_cast<std::uint32_t>(a.h) * a.w, hw2 = hw * 2u;
    const int csrc = C::STG == 2 ? a.ica / 4 : a.ica;
    const std::uint32_t plane_src = C::STG == 2 ? 4u * hw2 : hw2;  // bytes per source channel
    const int sw = C::STG == 2 ? a.w * 2 : a.w;
    const int G = static_cast<int>(gridDim.x);
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

    // Resident weights: the 3x3 chunk in LDS, the 1x1 fragments in registers.
    {
        const u32x4* ws = reinterpret_cast<const u32x4*>(a.wa);
        for (int e = tid; e < C::WA_VEC; e += C::kThreads) reinterpret_cast<u32x4*>(wa_s)[e] = ws[e];
    }
    const u32x4* wb = reinterpret_cast<const u32x4*>(a.wb);
    u32x4 wbr[C::KSB][C::MTB];
#pragma unroll
    for (int ks = 0; ks < C::KSB; ++ks)
#pragma unroll
        for (int mt = 0; mt < C::MTB; ++mt) wbr[ks][mt] = wb[(ks * C::MTB + mt) * 64 + lane];

    struct Tile {
        int b, ty0, tx0;
    };
    auto tile_of = [&](int v) {
        const int item = xcd_order(v, a.nwg), tile = item % a.tiles;
        return Tile{item / a.tiles, (tile / a.tiles_x) * C::TH, (tile % a.tiles_x) * C::TW};
    };

    // Input unit of this thread (tid < XUNITS): STG 2 (yi, sg, g) = source
    // channels 2g, 2g + 1, rows 2iy, 2iy + 1, 32 bytes each; STG 1 (yi, sg,
    // c8) = 8 channels x 16 bytes. Either way 8 loads.
    const int uyi = tid % C::IH_T, usg = (tid / C::IH_T) % C::NSEG, ug = tid / (C::IH_T * C::NSEG);
    // r unit of this lane (lane < 32): 8 channels x 8 pixels of this wave's row.
    const int rc8 = lane % 8, rpx = (lane / 8) * 8;
    u32x4 vin[8], rv[8];
    // Load k (0..7) of this thread's input unit and r unit of tile t; with
    // valid false every offset is out of range (nothing is read).
    auto fetch_k = [&](const Tile& t, bool valid, int k) {
        if (tid < XUNITS) {
            const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<std::uint16_t*>(a.x + static_cast<size_t>(t.b) * csrc * (plane_src / 2)), 0,
                static_cast<int>(csrc * plane_src), kRawBufferFlags);
            const int ix0 = t.tx0 - 1, xa = ix0 - (((ix0 % 8) + 8) % 8);
            const int iy = t.ty0 - 1 + uyi, ix = xa + usg * 8;
            const bool ok = valid && iy >= 0 && iy < a.h && ix >= 0 && ix < a.w;
            if constexpr (C::STG == 2) {
                const std::uint32_t base = static_cast<std::uint32_t>(2 * iy * sw + 2 * ix) * 2u;
                const int ql = k >> 2, dy = (k >> 1) & 1, hh = k & 1;
                // Source channels past the input (the zero padding of the
                // last chunk) are not fetched at all.
                const bool real = 2 * ug + ql < csrc;
                const std::uint32_t off = ok ? base + static_cast<std::uint32_t>(2 * ug + ql) * plane_src +
                                                   static_cast<std::uint32_t>(dy * sw * 2 + hh * 16)
                                             : kOutOfRange;
                vin[k] = real ? __builtin_amdgcn_raw_buffer_load_b128(rx, static_cast<int>(off), 0, 0) : u32x4{0u, 0u, 0u, 0u};
            } else {
                const std::uint32_t base =
                    ok ? static_cast<std::uint32_t>(iy * a.w + ix) * 2u + static_cast<std::uint32_t>(ug * 8) * hw2 : kOutOfRange;
                vin[k] = __builtin_amdgcn_raw_buffer_load_b128(rx, static_cast<int>(ok ? base + k * hw2 : kOutOfRange), 0, 0);
            }
        }
        if (lane < 32) {
            const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<std::uint16_t*>(a.r + static_cast<size_t>(t.b) * C::CR * hw), 0, static_cast<int>(C::CR * hw2),
                kRawBufferFlags);
            const int oy = t.ty0 + wave, ox = t.tx0 + rpx;
            const bool ok = valid && oy < a.h && ox < a.w;
            const std::uint32_t base = (static_cast<std::uint32_t>(rc8 * 8) * hw + static_cast<std::uint32_t>(oy * a.w + ox)) * 2u;
            rv[k] = __builtin_amdgcn_raw_buffer_load_b128(rr, static_cast<int>(ok ? base + k * hw2 : kOutOfRange), 0, 0);
        }
    };

    int v = static_cast<int>(blockIdx.x);
    if (v < a.nwg) {
#pragma unroll
        for (int k = 0; k < 8; ++k) fetch_k(tile_of(v), true, k);
    }
    for (; v < a.nwg; v += G) {
        const Tile t = tile_of(v);
        // The previous tile's phase A has finished reading the halo tile
        // (and, the first time, the resident 3x3 weights are in place).
        __syncthreads();
        if (tid < XUNITS) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                u32x4 q;
                if constexpr (C::STG == 2) {
                    // Dword j%4 of source half j/4 is the (dx = 0, 1) pair of staged pixel j.
                    const int hh = j >> 2, wd = j & 3;
                    q = u32x4{vin[(0 * 2 + 0) * 2 + hh][wd], vin[(0 * 2 + 1) * 2 + hh][wd], vin[(1 * 2 + 0) * 2 + hh][wd],
                              vin[(1 * 2 + 1) * 2 + hh][wd]};
                } else {
                    const bool up = j & 1;
                    const int wd = j >> 1;
                    q = u32x4{pack_half(vin[0][wd], vin[1][wd], up), pack_half(vin[2][wd], vin[3][wd], up),
                              pack_half(vin[4][wd], vin[5][wd], up), pack_half(vin[6][wd], vin[7][wd], up)};
                }
                *reinterpret_cast<u32x4*>(&in_s[C::at(uyi, usg * 8 + j) + ug * 8]) = q;
            }
        }
        if (lane < 32) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const bool up = j & 1;
                const int wd = j >> 1;
                const u32x4 q = {pack_half(rv[0][wd], rv[1][wd], up), pack_half(rv[2][wd], rv[3][wd], up),
                                 pack_half(rv[4][wd], rv[5][wd], up), pack_half(rv[6][wd], rv[7][wd], up)};
                *reinterpret_cast<u32x4*>(&ps[(wave * 32 + rpx + j) * C::PS + C::OCA + rc8 * 8]) = q;
            }
        }
        __syncthreads();
        // The next tile's loads go out one pair per tap of phase A rather than
        // in one burst here: a wave stalls at a load while the memory request
        // queue is full, which would hold back the MFMAs behind the burst.
        // After the last tile they are issued out of range (nothing is read),
        // so no branch decides whether they happen.
        const bool more = v + G < a.nwg;
        const Tile tn = tile_of(more ? v + G : v);

        // ---- phase A: 3x3 conv, BM = 64 ----
        floatx16 acc[C::MTA];
#pragma unroll
        for (int mt = 0; mt < C::MTA; ++mt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const floatx4 bv = *reinterpret_cast<const floatx4*>(a.ba + mt * 32 + 8 * j + hsel);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mt][4 * j + i] = bv[i];
            }
        const int ix0 = t.tx0 - 1, col_off = ix0 - (ix0 - (((ix0 % 8) + 8) % 8));
        const int pxi = (lane & 31) + col_off;
        // The operands of tap t + 1 are read from LDS during tap t (after its
        // loads, before its MFMAs), so each tap's MFMAs find theirs in
        // registers: with the scheduling barriers that keep the loads one per
        // tap, reads issued at their own tap left the LDS latency in front of
        // every pair of MFMAs (phase A 3.45k -> 2.9k cycles per tile).
        auto bfrag = [&](int tap) { return *reinterpret_cast<const half8*>(&in_s[C::at(wave + tap / 3, pxi + tap % 3) + koff]); };
        auto afrag = [&](int tap, int mt) { return *reinterpret_cast<const half8*>(&wa_s[((tap * C::MTA + mt) * 64 + lane) * 8]); };
        half8 bcur = bfrag(0), acur[C::MTA];
#pragma unroll
        for (int mt = 0; mt < C::MTA; ++mt) acur[mt] = afrag(0, mt);
#pragma unroll
        for (int tap = 0; tap < 9; ++tap) {
            if (tap < 8) {
                fetch_k(tn, more, tap);
                __builtin_amdgcn_sched_barrier(0);
            }
            half8 bnext = bcur, anext[C::MTA];
#pragma unroll
            for (int mt = 0; mt < C::MTA; ++mt) anext[mt] = acur[mt];
            if (tap < 8) {
                bnext = bfrag(tap + 1);
#pragma unroll
                for (int mt = 0; mt < C::MTA; ++mt) anext[mt] = afrag(tap + 1, mt);
            }
#pragma unroll
            for (int mt = 0; mt < C::MTA; ++mt) acc[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(acur[mt], bcur, acc[mt], 0, 0, 0);
            bcur = bnext;
#pragma unroll
            for (int mt = 0; mt < C::MTA; ++mt) acur[mt] = anext[mt];
        }

        // ---- t into this wave's P rows: rounded, activated, 4 channels per write ----
        const int p = wave * 32 + (lane & 31);
#pragma unroll
        for (int mt = 0; mt < C::MTA; ++mt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const std::uint32_t lo = epi_pair<EA>(acc[mt][4 * j], acc[mt][4 * j + 1], a.alpha_a);
                const std::uint32_t hi = epi_pair<EA>(acc[mt][4 * j + 2], acc[mt][4 * j + 3], a.alpha_a);
                *reinterpret_cast<u32x2*>(&ps[p * C::PS + mt * 32 + 8 * j + hsel]) = u32x2{lo, hi};
            }

        // ---- phase B: 1x1 over [t ; r] of this wave's rows, transposed:
        // lane l accumulates output channel mt*32 + l%32 for pixels
        // 8j + 4*(l/32) + i of the row ----
        floatx16 acc2[C::MTB];
#pragma unroll
        for (int mt = 0; mt < C::MTB; ++mt) {
            const float bv = a.bb[mt * 32 + (lane & 31)];
#pragma unroll
            for (int r = 0; r < 16; ++r) acc2[mt][r] = bv;
        }
#pragma unroll
        for (int ks = 0; ks < C::KSB; ++ks) {
            const half8 pv = *reinterpret_cast<const half8*>(&ps[p * C::PS + ks * 16 + koff]);
#pragma unroll
            for (int mt = 0; mt < C::MTB; ++mt)
                acc2[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(pv, __builtin_bit_cast(half8, wbr[ks][mt]), acc2[mt], 0, 0, 0);
        }

        // ---- out: [channel][pixel] tile in this wave's P rows (the last
        // reads of them are above, in this wave), 16-byte NCHW rows ----
        std::uint16_t* const stg = ps + wave * 32 * C::PS;
#pragma unroll
        for (int mt = 0; mt < C::MTB; ++mt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const std::uint32_t lo = epi_pair<EB>(acc2[mt][4 * j], acc2[mt][4 * j + 1], a.alpha_b);
                const std::uint32_t hi = epi_pair<EB>(acc2[mt][4 * j + 2], acc2[mt][4 * j + 3], a.alpha_b);
                *reinterpret_cast<u32x2*>(&stg[(mt * 32 + (lane & 31)) * kStgRow + 8 * j + hsel]) = u32x2{lo, hi};
            }
        const int oy = t.ty0 + wave;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int e = lane + 64 * k, oc = e >> 2, px = (e & 3) * 8;
            const u32x4 hv = *reinterpret_cast<const u32x4*>(&stg[oc * kStgRow + px]);
            if (oy < a.h && t.tx0 + px < a.w)
                *reinterpret_cast<u32x4*>(a.y + (static_cast<size_t>(t.b) * C::OCB + oc) * hw + static_cast<size_t>(oy) * a.w +
                                          t.tx0 + px) = hv;
        }
    }
}

template <class C, int EA, int EB>
void launch_pair_stream_epi(const PairArgs& a, hipStream_t s)
{
    // Two workgroups per CU (the LDS budget), a multiple of the 8 XCDs.
    int g = 2 * cu_count();
    if (g > a.nwg) g = a.nwg;
    if (g >= 8) g -= g % 8;
    hipLaunchKernelGGL((conv_pair_stream_kernel<C, EA, EB>), dim3(static_cast<unsigned>(g)), dim3(C::kThreads), 0, s, a);
}

template <class C, int EA>
void launch_pair_stream_b(const PairArgs& a, hipStream_t s)
{
    switch (epi_mode(a.epi_b == MLVC_EPI_LEAKY_RELU, a.alpha_b)) {
    case 0: launch_pair_stream_epi<C, EA, 0>(a, s); break;
    case 1: launch_pair_stream_epi<C, EA, 1>(a, s); break;
    default: launch_pair_stream_epi<C, EA, 2>(a, s); break;
    }
}

template <class C>
void launch_pair_stream(const PairArgs& a, hipStream_t s)
{
    switch (epi_mode(a.epi_a == MLVC_EPI_LEAKY_RELU, a.alpha_a)) {
    case 0: launch_pair_stream_b<C, 0>(a, s); break;
    case 1: launch_pair_stream_b<C, 1>(a, s); break;
    default: launch_pair_stream_b<C, 2>(a, s); break;
    }
}

template <class C>
void launch_pair(const PairArgs& a, hipStream_t s)
{
    hipLaunchKernelGGL(conv_pair_kernel<C>, dim3(static_cast<unsigned>(a.nwg)), dim3(C::kThreads), 0, s, a);
}

constexpr int kPairTH = 4, kPairTW = 32;

}  // namespace
}  // namespace conv
}  // namespace mlvc_hip

using namespace mlvc_hip;
using namespace mlvc_hip::conv;

extern "C" {

int mlvc_hip_convpair_supported(const mlvc_hip_convpair_desc* d)
{
    if (!d) return 0;
    const bool epi_ok = (d->epi_a == MLVC_EPI_NONE || d->epi_a == MLVC_EPI_LEAKY_RELU) &&
                        (d->epi_b == MLVC_EPI_NONE || d->epi_b == MLVC_EPI_LEAKY_RELU);
    const bool s2d_ok = d->in_s2d_block <= 1 || (d->in_s2d_block == 2 && d->ica % 4 == 0);
    const std::uint64_t plane = static_cast<std::uint64_t>(d->h) * d->w * 2;
    return d->n > 0 && d->ica > 0 && d->h > 0 && d->w > 0 && d->w % 8 == 0 && d->oca == 64 && d->cr == 64 &&
           d->ocb == 64 && epi_ok && s2d_ok && (static_cast<std::uint64_t>(d->ica) + 32) * plane < (1ull << 30) &&
           64 * plane < (1ull << 30);
}

size_t mlvc_hip_convpair_packed_a_bytes(const mlvc_hip_convpair_desc* d)
{
    return static_cast<size_t>((d->ica + 15) / 16) * 9 * 16 * 64 * 2;
}

size_t mlvc_hip_convpair_packed_b_bytes(const mlvc_hip_convpair_desc*) { return static_cast<size_t>(64) * 128 * 2; }

int mlvc_hip_convpair_pack(const mlvc_hip_convpair_desc* d, const uint16_t* wa, const uint16_t* wb, void* dst_a,
                           void* dst_b)
{
    return guard([&] {
        if (!mlvc_hip_convpair_supported(d)) throw std::runtime_error("convpair: unsupported geometry");
        auto* oa = static_cast<std::uint16_t*>(dst_a);
        size_t o = 0;
        // A: [chunk][tap][mt][lane][8], lane l of m-tile mt holds
        // Wa[oc = mt*32 + l%32][ic = chunk*16 + 8*(l/32) + j][tap].
        const int chunks = (d->ica + 15) / 16;
        for (int ch = 0; ch < chunks; ++ch)
            for (int tap = 0; tap < 9; ++tap)
                for (int mt = 0; mt < 2; ++mt)
                    for (int lane = 0; lane < 64; ++lane)
                        for (int j = 0; j < 8; ++j) {
                            const int oc = mt * 32 + (lane & 31), ic = ch * 16 + 8 * (lane >> 5) + j;
                            oa[o++] = ic < d->ica ? wa[(static_cast<size_t>(oc) * d->ica + ic) * 9 + tap] : std::uint16_t{0};
                        }
        // B: [ks][mt][lane][8], lane l holds Wb[mt*32 + l%32][ks*16 + 8*(l/32) + j].
        auto* ob = static_cast<std::uint16_t*>(dst_b);
        o = 0;
        for (int ks = 0; ks < 8; ++ks)
            for (int mt = 0; mt < 2; ++mt)
                for (int lane = 0; lane < 64; ++lane)
                    for (int j = 0; j < 8; ++j)
                        ob[o++] = wb[static_cast<size_t>(mt * 32 + (lane & 31)) * 128 + ks * 16 + 8 * (lane >> 5) + j];
    });
}

int mlvc_hip_convpair_launch(const mlvc_hip_convpair_desc* d, mlvc_hip_stream s)
{
    return guard([&] {
        if (!mlvc_hip_convpair_supported(d)) throw std::runtime_error("convpair: unsupported geometry");
        if (!d->x || !d->r || !d->wa || !d->ba || !d->wb || !d->bb || !d->y) throw std::runtime_error("convpair: null tensor");
        for (const void* p : {d->x, d->r, d->wa, d->wb, static_cast<const void*>(d->y)})
            if (reinterpret_cast<std::uintptr_t>(p) & 15u) throw std::runtime_error("convpair: tensors must be 16-byte aligned");
        PairArgs a{};
        a.x = static_cast<const std::uint16_t*>(d->x);
        a.r = static_cast<const std::uint16_t*>(d->r);
        a.wa = static_cast<const std::uint16_t*>(d->wa);
        a.ba = d->ba;
        a.wb = static_cast<const std::uint16_t*>(d->wb);
        a.bb = d->bb;
        a.y = static_cast<std::uint16_t*>(d->y);
        a.ica = d->ica;
        a.h = d->h;
        a.w = d->w;
        a.nchunks = (d->ica + 15) / 16;
        a.epi_a = d->epi_a;
        a.epi_b = d->epi_b;
        a.alpha_a = d->alpha_a;
        a.alpha_b = d->alpha_b;
        a.tiles_x = (d->w + kPairTW - 1) / kPairTW;
        a.tiles = a.tiles_x * ((d->h + kPairTH - 1) / kPairTH);
        const long long nwg = static_cast<long long>(a.tiles) * d->n;
        if (nwg > 0x7FFFFFFF) throw std::runtime_error("convpair: grid too large");
        a.nwg = static_cast<int>(nwg);
        if (a.nchunks == 1) {
            if (d->in_s2d_block == 2)
                launch_pair_stream<PairCfg<kPairTH, kPairTW, 2>>(a, to_stream(s));
            else
                launch_pair_stream<PairCfg<kPairTH, kPairTW, 1>>(a, to_stream(s));
        } else if (d->in_s2d_block == 2) {
            launch_pair<PairCfg<kPairTH, kPairTW, 2>>(a, to_stream(s));
        } else {
            launch_pair<PairCfg<kPairTH, kPairTW, 1>>(a, to_stream(s));
        }
        check(hipGetLastError(), "convpair launch");
    });
}

}  // extern "C"
