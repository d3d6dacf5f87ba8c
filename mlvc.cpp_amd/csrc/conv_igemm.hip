// FP16 convolution (groups == 1) on gfx950 MFMA as an implicit GEMM.
//
//   D[oc, p] = bias[oc] + sum_k W[oc, k] * X[k, p],  k = (chunk, tap, c16)
//
// One workgroup (4 waves) owns BM output channels x a TH x TW output-pixel
// tile. Per input-channel chunk of KC channels it stages
//   * the NCHW input halo tile into LDS channel-last ([pixel][KC + 8 pad]),
//     so the MFMA B fragment of a lane (8 consecutive channels of one pixel)
//     is a single 16-byte LDS read for every tap; for stride 2 the even and
//     odd input columns are stored in separate halves of an LDS row so that
//     consecutive output pixels read consecutive LDS pixels;
//   * the chunk's weights, pre-packed at load time in exact A-fragment order
//     ([tap][k16][m32][lane][8]), as a contiguous 16-byte-vector copy.
// The next chunk is fetched into registers while the current one is
// consumed (v_mfma_f32_32x32x16_f16, FP32 accumulators seeded with the
// bias). The epilogue rounds to FP16 (RNE), applies LeakyReLU or the
// residual add on the rounded value exactly like the reference CPU GEMM
// epilogue (backends/cpu/src/kernels_scalar.cpp:178-192), and stores either
// plainly or through the DEPTH_TO_SPACE (CRD) index map.
//
// Reference kernels this replaces: pointwise_conv.cu:116-338 (1x1 mma.sync),
// cutlass.cu:116-161 (1x1 EVT epilogues, spatial fprop), spatial_conv.cu:
// 1-293 (implicit-GEMM KxK), generic_conv.cu:1-82 (fallback).

#include "common.hpp"
#include "mlvc_hip_device.h"

#include <algorithm>
#include <cstring>
#include <vector>

namespace mlvc_hip {
namespace {

// Raw buffer resource word 3 for gfx950 (32-bit data format, no swizzle).
constexpr int kRawBufferFlags = 0x00020000;
// Byte offset past the end of every staged tensor (each < 2 GiB), also after
// adding up to 7 channel planes; raw buffer loads there return zeros.
constexpr std::uint32_t kOutOfRange = 0x80000000u;

struct ConvArgs {
    const std::uint16_t* x;
    const std::uint16_t* x2;
    const std::uint16_t* w;
    const float* bias;
    const std::uint16_t* res;
    std::uint16_t* y;
    int ic_split, s2d, d2s;
    int ic, ih, iw, oc, oh, ow, kh, kw, sh, sw, ph, pw;
    int epi;
    float alpha;
    int tiles_x, nchunks;
    int tiles, ocbs, nwg;  // pixel tiles per image, output-channel blocks, workgroups (tiles*ocbs*n)
};

// KC consecutive channels [c0, c0 + KC) of input pixel (iy, ix) of batch b,
// packed in pairs, through the optional SPACE_TO_DEPTH / CONCAT maps. Zero
// outside the image (padding) and for channels past IC (chunk padding).
template <int KC>
__device__ __forceinline__ void load_pixel(const ConvArgs& a, int b, int c0, int iy, int ix, std::uint32_t (&out)[KC / 2])
{
    std::uint16_t v[KC];
#pragma unroll
    for (int j = 0; j < KC; ++j) v[j] = 0;
    if (iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw) {
        if (a.s2d > 1) {
            const int bs = a.s2d, b2 = bs * bs;
            const int sW = a.iw * bs;
            const size_t splane = static_cast<size_t>(a.ih) * bs * sW;
            const std::uint16_t* p = a.x + static_cast<size_t>(b) * (a.ic / b2) * splane +
                                     static_cast<size_t>(iy * bs) * sW + ix * bs;
#pragma unroll
            for (int j = 0; j < KC; ++j) {
                const int c = c0 + j;
                if (c < a.ic) {
                    const int cs = c / b2, r = c - cs * b2, dy = r / bs, dx = r - dy * bs;
                    v[j] = p[cs * splane + static_cast<size_t>(dy) * sW + dx];
                }
            }
        } else {
            const size_t hw = static_cast<size_t>(a.ih) * a.iw;
            const size_t po = static_cast<size_t>(iy) * a.iw + ix;
            const int c1 = a.x2 ? a.ic_split : a.ic;
            const std::uint16_t* p = a.x + static_cast<size_t>(b) * c1 * hw + po;
            const std::uint16_t* p2 = a.x2 ? a.x2 + static_cast<size_t>(b) * (a.ic - c1) * hw + po : nullptr;
#pragma unroll
            for (int j = 0; j < KC; ++j) {
                const int c = c0 + j;
                if (c < c1)
                    v[j] = p[c * hw];
                else if (c < a.ic)
                    v[j] = p2[(c - c1) * hw];
            }
        }
    }
#pragma unroll
    for (int j = 0; j < KC / 2; ++j) out[j] = static_cast<std::uint32_t>(v[2 * j]) | (static_cast<std::uint32_t>(v[2 * j + 1]) << 16);
}

// Single element of the conv input (used by the direct fallback).
__device__ __forceinline__ std::uint16_t load_input(const ConvArgs& a, int b, int c, int iy, int ix)
{
    if (c >= a.ic || iy < 0 || iy >= a.ih || ix < 0 || ix >= a.iw) return 0;
    if (a.s2d > 1) {
        const int bs = a.s2d, b2 = bs * bs;
        const int cs = c / b2, r = c - cs * b2, dy = r / bs, dx = r - dy * bs;
        const int sc = a.ic / b2, sh = a.ih * bs, sw = a.iw * bs;
        return a.x[(static_cast<size_t>(b * sc + cs) * sh + iy * bs + dy) * sw + ix * bs + dx];
    }
    if (a.x2) {
        if (c >= a.ic_split)
            return a.x2[(static_cast<size_t>(b * (a.ic - a.ic_split) + c - a.ic_split) * a.ih + iy) * a.iw + ix];
        return a.x[(static_cast<size_t>(b * a.ic_split + c) * a.ih + iy) * a.iw + ix];
    }
    return a.x[(static_cast<size_t>(b * a.ic + c) * a.ih + iy) * a.iw + ix];
}

__device__ __forceinline__ std::uint16_t finish(const ConvArgs& a, float acc, int b, int oc, int oy, int ox)
{
    std::uint16_t h = f2h(acc);
    if (a.epi == MLVC_EPI_LEAKY_RELU) {
        const float f = h2f(h);
        if (f < 0.0f) h = leaky_f16(f, a.alpha);
    } else if (a.epi == MLVC_EPI_RESIDUAL_ADD) {
        h = f2h(h2f(h) + h2f(a.res[(static_cast<size_t>(b * a.oc + oc) * a.oh + oy) * a.ow + ox]));
    }
    return h;
}

__device__ __forceinline__ void store_output(const ConvArgs& a, std::uint16_t h, int b, int oc, int oy, int ox)
{
    if (a.d2s > 1) {
        const int bs = a.d2s, b2 = bs * bs;
        const int c = oc / b2, r = oc - c * b2, dy = r / bs, dx = r - dy * bs;
        const int occ = a.oc / b2, H = a.oh * bs, W = a.ow * bs;
        a.y[(static_cast<size_t>(b * occ + c) * H + oy * bs + dy) * W + ox * bs + dx] = h;
    } else {
        a.y[(static_cast<size_t>(b * a.oc + oc) * a.oh + oy) * a.ow + ox] = h;
    }
}

template <int BM_, int TH_, int TW_, int KH_, int KW_, int S_, int KC_, bool VEC_, bool DB_>
struct Cfg {
    static constexpr int BM = BM_, TH = TH_, TW = TW_, KH = KH_, KW = KW_, S = S_, KC = KC_;
    static constexpr bool VEC = VEC_;  // 16-byte row-segment staging (needs W % 8 == 0)
    // Two LDS stages: chunk k+1 is staged (weights by LDS DMA) while chunk k
    // is multiplied, one barrier per chunk. Otherwise one stage, weights
    // staged through registers, two barriers per chunk, half the LDS.
    static constexpr bool DB = DB_;
    static constexpr int kThreads = 256;
    static constexpr int BN = TH * TW;
    static constexpr int TAPS = KH * KW;
    static constexpr int KS = KC / 16;  // 16-deep MFMA K steps per tap
    static constexpr int MT = BM / 32;
    static constexpr int WN = BN / 4;
    static constexpr int NT = WN / 32;
    static constexpr int IH_T = (TH - 1) * S + KH;
    static constexpr int IW_T = (TW - 1) * S + KW;
    // Vector staging covers input columns [floor8(ix0), floor8(ix0) + IW_S).
    static constexpr int NSEG = (IW_T + 14) / 8;
    static constexpr int IW_S = VEC ? NSEG * 8 : IW_T;
    static constexpr int IW_E = (IW_S + 1) / 2;  // even columns (stride-2 layout)
    static constexpr int PST = KC + 8;           // LDS halves per staged pixel
    // Staged rows are padded by 16 bytes, so consecutive rows start 4 banks
    // apart: the transposed commit writes (8 lanes = 8 consecutive rows of
    // one pixel column) and the B reads (8 lanes = 8 consecutive pixels of a
    // row, PST = 12 dwords apart, any alignment) are both free of conflicts.
    static constexpr int ROW = IW_S * PST + 8;
    static constexpr int IN_LDS = IH_T * ROW;
    static constexpr int UNITS = (KC / 8) * IH_T * NSEG;  // 8 channels x 8 columns
    static constexpr int UNITS_PER_T = (UNITS + kThreads - 1) / kThreads;
    static constexpr int IN_PIX = IH_T * IW_T;
    static constexpr int PIX_PER_T = (IN_PIX + kThreads - 1) / kThreads;
    static constexpr int W_LDS = TAPS * KS * MT * 64 * 8;  // halves per chunk
    static constexpr int W_VEC = W_LDS / 8;
    static constexpr int W_PER_T = (W_VEC + kThreads - 1) / kThreads;
    static constexpr int EPI_ROW = BN + 8;  // output staging row (one channel), halves
    static constexpr int EPI_LDS = BM * EPI_ROW;
    static constexpr int STAGE = IN_LDS + W_LDS;
    static constexpr int W_INST = W_VEC / 64;  // 1 KB LDS DMA instructions per chunk
    static constexpr int LDS = (DB ? 2 * STAGE : STAGE) > EPI_LDS ? (DB ? 2 * STAGE : STAGE) : EPI_LDS;
    static_assert(BM % 32 == 0 && WN % 32 == 0 && KC % 16 == 0 && TW % 8 == 0 && W_VEC % 64 == 0, "tile shape");
    static_assert(STAGE % 8 == 0, "stage alignment");
    static_assert(LDS * 2 <= 160 * 1024, "LDS budget");

    __device__ static constexpr int col(int x) { return S == 2 ? ((x & 1) ? IW_E + (x >> 1) : (x >> 1)) : x; }
    // LDS offset (halves) of staged pixel (row, column).
    __device__ static constexpr int at(int row, int x) { return row * ROW + col(x) * PST; }
};

__device__ __forceinline__ std::uint32_t pack_half(std::uint32_t lo_word, std::uint32_t hi_word, bool upper)
{
    return upper ? ((lo_word >> 16) | (hi_word & 0xFFFF0000u)) : ((lo_word & 0xFFFFu) | (hi_word << 16));
}

template <class C>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void conv_mfma_kernel(ConvArgs a)
{
    __shared__ __attribute__((aligned(16))) std::uint16_t lds[C::LDS];
    auto lds_in = [&](int stage) { return lds + stage * C::STAGE; };
    auto lds_w = [&](int stage) { return lds + stage * C::STAGE + C::IN_LDS; };

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // Logical work item: output-channel block fastest, then pixel tiles in
    // row-major order, then images; each XCD runs a contiguous range of them.
    const int item = xcd_order(blockIdx.x, a.nwg);
    const int ocb = item % a.ocbs, tile = (item / a.ocbs) % a.tiles, b = item / (a.ocbs * a.tiles);
    const int tx0 = (tile % a.tiles_x) * C::TW, ty0 = (tile / a.tiles_x) * C::TH;
    const int iy0 = ty0 * C::S - a.ph, ix0 = tx0 * C::S - a.pw;
    // First staged input column (8-aligned for the vector path).
    const int xa = C::VEC ? ix0 - (((ix0 % 8) + 8) % 8) : ix0;
    const int col_off = ix0 - xa;

    floatx16 acc[C::MT][C::NT];
#pragma unroll
    for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float bv = a.bias[ocb * C::BM + mt * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)];
#pragma unroll
            for (int nt = 0; nt < C::NT; ++nt) acc[mt][nt][r] = bv;
        }

    const size_t hw = static_cast<size_t>(a.ih) * a.iw;
    const int c1 = a.x2 ? a.ic_split : a.ic;
    u32x4 vin[C::VEC ? C::UNITS_PER_T : 1][8];
    std::uint32_t in_reg[C::VEC ? 1 : C::PIX_PER_T][C::KC / 2];
    u32x4 w_reg[C::DB ? 1 : C::W_PER_T];
    // Vector staging reads through raw buffer resources sized to this
    // image's part of x (channels [0, c1)) and of x2 (the concat rest): a
    // load past the end returns zeros, so padding rows/columns (offset set
    // past the end) and channels past IC need no branch. The concat split
    // falls on a chunk boundary, so each chunk reads one resource.
    const std::uint32_t hw2 = static_cast<std::uint32_t>(hw) * 2u;
    const std::uint16_t* x_img = a.x + static_cast<size_t>(b) * c1 * hw;
    const std::uint16_t* x2_img = a.x2 ? a.x2 + static_cast<size_t>(b) * (a.ic - c1) * hw : x_img;
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<std::uint16_t*>(x_img), 0, static_cast<int>(c1 * hw2), kRawBufferFlags);
    const __amdgpu_buffer_rsrc_t rx2 = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<std::uint16_t*>(x2_img), 0, static_cast<int>(a.x2 ? (a.ic - c1) * hw2 : 0u), kRawBufferFlags);
    std::uint32_t pix_off[C::VEC ? C::UNITS_PER_T : 1];
    int unit_c8[C::VEC ? C::UNITS_PER_T : 1];
    if constexpr (C::VEC) {
#pragma unroll
        for (int i = 0; i < C::UNITS_PER_T; ++i) {
            const int u = tid + i * C::kThreads;
            const int yi = u % C::IH_T, sg = (u / C::IH_T) % C::NSEG;
            const int iy = iy0 + yi, ix = xa + sg * 8;
            const bool ok = u < C::UNITS && iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw;
            pix_off[i] = ok ? static_cast<std::uint32_t>(iy * a.iw + ix) * 2u : kOutOfRange;
            unit_c8[i] = u / (C::NSEG * C::IH_T);  // units: rows fastest, then segments, then channel groups
        }
    }
    auto fetch = [&](int chunk, int stage) {
        const int c0 = chunk * C::KC;
        if constexpr (C::VEC) {
            const bool second = a.x2 && c0 >= c1;
            const __amdgpu_buffer_rsrc_t r = second ? rx2 : rx;
            const std::uint32_t cbase = static_cast<std::uint32_t>(second ? c0 - c1 : c0);
#pragma unroll
            for (int i = 0; i < C::UNITS_PER_T; ++i) {
                const std::uint32_t off = pix_off[i] == kOutOfRange
                                              ? kOutOfRange
                                              : pix_off[i] + (cbase + static_cast<std::uint32_t>(unit_c8[i]) * 8u) * hw2;
                // The channel offset goes in the VGPR operand: the range check
                // covers that operand only, so channels past the end read zeros.
#pragma unroll
                for (int k = 0; k < 8; ++k)
                    vin[i][k] = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(off + k * hw2), 0, 0);
            }
        } else {
#pragma unroll
            for (int i = 0; i < C::PIX_PER_T; ++i) {
                const int pix = tid + i * C::kThreads;
                if (pix < C::IN_PIX) {
                    const int yi = pix / C::IW_T, xi = pix - yi * C::IW_T;
                    load_pixel<C::KC>(a, b, c0, iy0 + yi, ix0 + xi, in_reg[i]);
                }
            }
        }
        const u32x4* ws = reinterpret_cast<const u32x4*>(a.w + (static_cast<size_t>(ocb) * a.nchunks + chunk) * C::W_LDS);
        if constexpr (C::DB) {
            // The packed chunk is copied verbatim: LDS DMA, 1 KB per wave
            // instruction, lane l of instruction j moving vector 64*j + l.
            u32x4* dst = reinterpret_cast<u32x4*>(lds_w(stage));
#pragma unroll
            for (int i = 0; i < (C::W_INST + 3) / 4; ++i) {
                const int j = wave + 4 * i;
                if (j < C::W_INST)
                    __builtin_amdgcn_global_load_lds(ws + j * 64 + lane,
                                                     (__attribute__((address_space(3))) void*)(dst + j * 64), 16, 0, 0);
            }
        } else {
#pragma unroll
            for (int i = 0; i < C::W_PER_T; ++i) {
                const int e = tid + i * C::kThreads;
                if (e < C::W_VEC) w_reg[i] = ws[e];
            }
        }
    };
    auto commit = [&](int stage) {
        std::uint16_t* const in_s = lds_in(stage);
        if constexpr (C::VEC) {
            // 8x8 transpose in registers: staged pixel j of the segment gets
            // the 8 channels of the unit as one 16-byte LDS write.
#pragma unroll
            for (int i = 0; i < C::UNITS_PER_T; ++i) {
                const int u = tid + i * C::kThreads;
                if (u < C::UNITS) {
                    const int yi = u % C::IH_T, sg = (u / C::IH_T) % C::NSEG, c8 = u / (C::NSEG * C::IH_T);
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const bool up = j & 1;
                        const int wd = j >> 1;
                        const u32x4 t = {pack_half(vin[i][0][wd], vin[i][1][wd], up), pack_half(vin[i][2][wd], vin[i][3][wd], up),
                                         pack_half(vin[i][4][wd], vin[i][5][wd], up), pack_half(vin[i][6][wd], vin[i][7][wd], up)};
                        *reinterpret_cast<u32x4*>(&in_s[C::at(yi, sg * 8 + j) + c8 * 8]) = t;
                    }
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < C::PIX_PER_T; ++i) {
                const int pix = tid + i * C::kThreads;
                if (pix < C::IN_PIX) {
                    const int yi = pix / C::IW_T, xi = pix - yi * C::IW_T;
                    u32x4* dst = reinterpret_cast<u32x4*>(&in_s[C::at(yi, xi)]);
#pragma unroll
                    for (int q = 0; q < C::KC / 8; ++q)
                        dst[q] = u32x4{in_reg[i][4 * q], in_reg[i][4 * q + 1], in_reg[i][4 * q + 2], in_reg[i][4 * q + 3]};
                }
            }
        }
        if constexpr (!C::DB) {
#pragma unroll
            for (int i = 0; i < C::W_PER_T; ++i) {
                const int e = tid + i * C::kThreads;
                if (e < C::W_VEC) reinterpret_cast<u32x4*>(lds_w(0))[e] = w_reg[i];
            }
        }
    };

    // Per-lane output pixel of each 32-wide N block, in tile coordinates.
    int pyi[C::NT], pxi[C::NT];
#pragma unroll
    for (int nt = 0; nt < C::NT; ++nt) {
        const int p = wave * C::WN + nt * 32 + (lane & 31);
        pyi[nt] = (p / C::TW) * C::S;
        pxi[nt] = (p % C::TW) * C::S + col_off;
    }
    const int koff = (lane >> 5) * 8;

    auto compute = [&](int stage) {
        const std::uint16_t* const in_s = lds_in(stage);
        const std::uint16_t* const w_s = lds_w(stage);
#pragma unroll
        for (int tap = 0; tap < C::TAPS; ++tap) {
            const int ky = tap / C::KW, kx = tap % C::KW;
            int boff[C::NT];
#pragma unroll
            for (int nt = 0; nt < C::NT; ++nt) boff[nt] = C::at(pyi[nt] + ky, pxi[nt] + kx) + koff;
#pragma unroll
            for (int ks = 0; ks < C::KS; ++ks) {
                half8 av[C::MT], bv[C::NT];
#pragma unroll
                for (int mt = 0; mt < C::MT; ++mt)
                    av[mt] = *reinterpret_cast<const half8*>(&w_s[(((tap * C::KS + ks) * C::MT + mt) * 64 + lane) * 8]);
#pragma unroll
                for (int nt = 0; nt < C::NT; ++nt) bv[nt] = *reinterpret_cast<const half8*>(&in_s[boff[nt] + ks * 16]);
#pragma unroll
                for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
                    for (int nt = 0; nt < C::NT; ++nt)
                        acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[mt], bv[nt], acc[mt][nt], 0, 0, 0);
            }
        }
    };

    if constexpr (C::DB) {
        fetch(0, 0);
        commit(0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's LDS DMA has landed
        __syncthreads();
        for (int chunk = 0; chunk < a.nchunks; ++chunk) {
            const int cur = chunk & 1;
            const bool more = chunk + 1 < a.nchunks;
            // Stage cur^1 was last read before the previous barrier.
            if (more) fetch(chunk + 1, cur ^ 1);
            compute(cur);
            if (more) {
                commit(cur ^ 1);
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
            __syncthreads();
        }
    } else {
        fetch(0, 0);
        commit(0);
        __syncthreads();
        for (int chunk = 0; chunk < a.nchunks; ++chunk) {
            const bool more = chunk + 1 < a.nchunks;
            if (more) fetch(chunk + 1, 0);
            compute(0);
            __syncthreads();
            if (more) {
                commit(0);
                __syncthreads();
            }
        }
    }

    // Epilogue, stage 1: each lane writes its FP16-rounded accumulators into
    // an LDS tile [oc][pixel] (all indices static, so nothing spills).
    // The main loop ended with a barrier, so the staging buffers are free.
#pragma unroll
    for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < C::NT; ++nt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int ocl = mt * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int pl = wave * C::WN + nt * 32 + (lane & 31);
                lds[ocl * C::EPI_ROW + pl] = f2h(acc[mt][nt][r]);
            }
    __syncthreads();

    // Stage 2: the epilogue acts on the rounded value. Vector path: 8
    // consecutive pixels of a channel per thread, 16-byte stores; with a
    // fused DEPTH_TO_SPACE(2) the two dx channels of one (c, dy) are
    // interleaved into 16 contiguous output pixels.
    constexpr int GROUPS = C::BN / 8;
    auto epi8 = [&](std::uint16_t (&h)[8], int oc, int oy, int ox) {
        if (a.epi == MLVC_EPI_LEAKY_RELU) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float f = h2f(h[j]);
                if (f < 0.0f) h[j] = leaky_f16(f, a.alpha);
            }
        } else if (a.epi == MLVC_EPI_RESIDUAL_ADD) {
            const u32x4 rv = *reinterpret_cast<const u32x4*>(a.res + (static_cast<size_t>(b * a.oc + oc) * a.oh + oy) * a.ow + ox);
            const std::uint16_t* r = reinterpret_cast<const std::uint16_t*>(&rv);
#pragma unroll
            for (int j = 0; j < 8; ++j) h[j] = f2h(h2f(h[j]) + h2f(r[j]));
        }
    };
    if (a.ow % 8 == 0 && (a.d2s <= 1 || a.d2s == 2)) {
        const bool d2s2 = a.d2s == 2;
        const int units = d2s2 ? (C::BM / 4) * 2 * GROUPS : C::BM * GROUPS;
        for (int u = tid; u < units; u += C::kThreads) {
            const int g = u % GROUPS;
            const int pl = g * 8;
            const int oy = ty0 + pl / C::TW, ox = tx0 + pl % C::TW;
            if (oy >= a.oh || ox >= a.ow) continue;
            if (d2s2) {
                const int dy = (u / GROUPS) & 1, cq = u / (2 * GROUPS);
                const int ocl = cq * 4 + dy * 2, oc = ocb * C::BM + ocl;
                if (oc >= a.oc) continue;
                std::uint16_t h0[8], h1[8];
                *reinterpret_cast<u32x4*>(h0) = *reinterpret_cast<const u32x4*>(&lds[ocl * C::EPI_ROW + pl]);
                *reinterpret_cast<u32x4*>(h1) = *reinterpret_cast<const u32x4*>(&lds[(ocl + 1) * C::EPI_ROW + pl]);
                epi8(h0, oc, oy, ox);
                epi8(h1, oc + 1, oy, ox);
                std::uint16_t o[16];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    o[2 * j] = h0[j];
                    o[2 * j + 1] = h1[j];
                }
                const int W2 = a.ow * 2;
                std::uint16_t* dst = a.y + (static_cast<size_t>(b * (a.oc / 4) + oc / 4) * (a.oh * 2) + oy * 2 + dy) * W2 + ox * 2;
                reinterpret_cast<u32x4*>(dst)[0] = *reinterpret_cast<const u32x4*>(o);
                reinterpret_cast<u32x4*>(dst)[1] = *reinterpret_cast<const u32x4*>(o + 8);
            } else {
                const int ocl = u / GROUPS, oc = ocb * C::BM + ocl;
                if (oc >= a.oc) continue;
                std::uint16_t h[8];
                *reinterpret_cast<u32x4*>(h) = *reinterpret_cast<const u32x4*>(&lds[ocl * C::EPI_ROW + pl]);
                epi8(h, oc, oy, ox);
                *reinterpret_cast<u32x4*>(a.y + (static_cast<size_t>(b * a.oc + oc) * a.oh + oy) * a.ow + ox) =
                    *reinterpret_cast<const u32x4*>(h);
            }
        }
    } else {
        for (int e = tid; e < C::BM * C::BN; e += C::kThreads) {
            const int ocl = e / C::BN, pl = e - ocl * C::BN;
            const int oc = ocb * C::BM + ocl;
            const int oy = ty0 + pl / C::TW, ox = tx0 + pl % C::TW;
            if (oc < a.oc && oy < a.oh && ox < a.ow) {
                std::uint16_t h = lds[ocl * C::EPI_ROW + pl];
                if (a.epi == MLVC_EPI_LEAKY_RELU) {
                    const float f = h2f(h);
                    if (f < 0.0f) h = leaky_f16(f, a.alpha);
                } else if (a.epi == MLVC_EPI_RESIDUAL_ADD) {
                    h = f2h(h2f(h) + h2f(a.res[(static_cast<size_t>(b * a.oc + oc) * a.oh + oy) * a.ow + ox]));
                }
                store_output(a, h, b, oc, oy, ox);
            }
        }
    }
}

// Generic fallback: one thread per output, FP32 fused multiply-add in
// (ic, ky, kx) order. Used only for shapes without an MFMA variant.
__global__ __launch_bounds__(256) void conv_direct_kernel(ConvArgs a, int n)
{
    const size_t total = static_cast<size_t>(n) * a.oc * a.oh * a.ow;
    for (size_t i = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const int ox = static_cast<int>(i % a.ow);
        const int oy = static_cast<int>((i / a.ow) % a.oh);
        const int oc = static_cast<int>((i / (static_cast<size_t>(a.ow) * a.oh)) % a.oc);
        const int b = static_cast<int>(i / (static_cast<size_t>(a.ow) * a.oh * a.oc));
        float acc = a.bias[oc];
        const std::uint16_t* wr = a.w + static_cast<size_t>(oc) * a.ic * a.kh * a.kw;
        for (int c = 0; c < a.ic; ++c)
            for (int ky = 0; ky < a.kh; ++ky)
                for (int kx = 0; kx < a.kw; ++kx) {
                    const int iy = oy * a.sh - a.ph + ky, ix = ox * a.sw - a.pw + kx;
                    if (iy < 0 || iy >= a.ih || ix < 0 || ix >= a.iw) continue;
                    acc = fmaf(h2f(load_input(a, b, c, iy, ix)), h2f(wr[(c * a.kh + ky) * a.kw + kx]), acc);
                }
        store_output(a, finish(a, acc, b, oc, oy, ox), b, oc, oy, ox);
    }
}

// ---------------------------------------------------------------- variants
struct Variant {
    const char* name;
    int bm, th, tw, kh, kw, s, kc;  // bm == 0: direct fallback
    void (*launch_scalar)(const ConvArgs&, dim3, hipStream_t);
    void (*launch_vec)(const ConvArgs&, dim3, hipStream_t);
};

template <class C>
void launch_mfma(const ConvArgs& a, dim3 grid, hipStream_t s)
{
    hipLaunchKernelGGL(conv_mfma_kernel<C>, grid, dim3(C::kThreads), 0, s, a);
}

#define MLVC_VARIANT(BM, TH, TW, KH, KW, S, KC)                                                              \
    Variant{"mfma_bm" #BM "_" #TH "x" #TW "_k" #KH "x" #KW "_s" #S "_kc" #KC, BM, TH, TW, KH, KW, S, KC,        \
            &launch_mfma<Cfg<BM, TH, TW, KH, KW, S, KC, false, false>>, &launch_mfma<Cfg<BM, TH, TW, KH, KW, S, KC, true, false>>}
// Two-stage pipeline (vector staging only; the scalar staging path keeps the one-stage kernel).
#define MLVC_VARIANT_DB(BM, TH, TW, KH, KW, S, KC)                                                           \
    Variant{"mfma_bm" #BM "_" #TH "x" #TW "_k" #KH "x" #KW "_s" #S "_kc" #KC "_db", BM, TH, TW, KH, KW, S, KC,  \
            &launch_mfma<Cfg<BM, TH, TW, KH, KW, S, KC, false, false>>, &launch_mfma<Cfg<BM, TH, TW, KH, KW, S, KC, true, true>>}

const Variant kVariants[] = {
    Variant{"direct_fp32", 0, 0, 0, 0, 0, 0, 0, nullptr, nullptr},
    // 3x3 stride 1
    MLVC_VARIANT(32, 4, 64, 3, 3, 1, 16),
    MLVC_VARIANT(32, 8, 32, 3, 3, 1, 16),
    MLVC_VARIANT(64, 4, 64, 3, 3, 1, 16),
    MLVC_VARIANT(64, 8, 32, 3, 3, 1, 16),
    MLVC_VARIANT(64, 16, 16, 3, 3, 1, 16),
    MLVC_VARIANT(64, 2, 64, 3, 3, 1, 16),
    MLVC_VARIANT(64, 4, 32, 3, 3, 1, 16),
    MLVC_VARIANT(64, 8, 16, 3, 3, 1, 16),
    MLVC_VARIANT(128, 4, 64, 3, 3, 1, 16),
    MLVC_VARIANT(128, 8, 32, 3, 3, 1, 16),
    MLVC_VARIANT(128, 16, 16, 3, 3, 1, 16),
    MLVC_VARIANT_DB(64, 8, 32, 3, 3, 1, 16),
    MLVC_VARIANT_DB(32, 8, 32, 3, 3, 1, 16),
    MLVC_VARIANT_DB(128, 8, 32, 3, 3, 1, 16),
    MLVC_VARIANT_DB(128, 4, 64, 3, 3, 1, 16),
    MLVC_VARIANT_DB(64, 4, 64, 3, 3, 1, 16),
    // 3x3 stride 2
    MLVC_VARIANT(32, 4, 64, 3, 3, 2, 16),
    MLVC_VARIANT(64, 2, 64, 3, 3, 2, 16),
    MLVC_VARIANT(64, 4, 32, 3, 3, 2, 16),
    MLVC_VARIANT(64, 8, 16, 3, 3, 2, 16),
    MLVC_VARIANT(128, 2, 64, 3, 3, 2, 16),
    // 1x1 (flattened pixels unless an unshuffle is fused)
    MLVC_VARIANT(32, 1, 256, 1, 1, 1, 32),
    MLVC_VARIANT(64, 1, 256, 1, 1, 1, 32),
    MLVC_VARIANT(64, 1, 128, 1, 1, 1, 32),
    MLVC_VARIANT(128, 1, 128, 1, 1, 1, 32),
    MLVC_VARIANT(64, 2, 64, 1, 1, 1, 32),
    MLVC_VARIANT(64, 4, 32, 1, 1, 1, 32),
};
constexpr int kVariantCount = static_cast<int>(sizeof(kVariants) / sizeof(kVariants[0]));

int cu_count()
{
    static int cus = [] {
        int dev = 0, n = 256;
        if (hipGetDevice(&dev) == hipSuccess) {
            hipDeviceProp_t p;
            if (hipGetDeviceProperties(&p, dev) == hipSuccess) n = p.multiProcessorCount;
        }
        return n;
    }();
    return cus;
}

bool flat_1x1(const mlvc_hip_conv_desc& d)
{
    return d.kh == 1 && d.kw == 1 && d.in_s2d_block <= 1 && d.out_d2s_block <= 1;
}

const Variant& variant_of(const mlvc_hip_conv_desc& d)
{
    if (d.variant < 0 || d.variant >= kVariantCount) throw std::runtime_error("conv: invalid variant");
    return kVariants[d.variant];
}

// Geometry and fusion checks (planning and launch); pointers at launch only.
void validate(const mlvc_hip_conv_desc& d, bool pointers)
{
    if (d.n <= 0 || d.ic <= 0 || d.ih <= 0 || d.iw <= 0 || d.oc <= 0 || d.oh <= 0 || d.ow <= 0 || d.kh <= 0 ||
        d.kw <= 0 || d.stride_h <= 0 || d.stride_w <= 0 || d.pad_h < 0 || d.pad_w < 0)
        throw std::runtime_error("conv: invalid geometry");
    if (d.oh != (d.ih + 2 * d.pad_h - d.kh) / d.stride_h + 1 || d.ow != (d.iw + 2 * d.pad_w - d.kw) / d.stride_w + 1)
        throw std::runtime_error("conv: output shape does not match the geometry");
    if (d.in_s2d_block > 1 && (d.ic % (d.in_s2d_block * d.in_s2d_block) != 0 || d.x2))
        throw std::runtime_error("conv: invalid space_to_depth fusion");
    if (d.x2 && (d.ic_split <= 0 || d.ic_split >= d.ic)) throw std::runtime_error("conv: invalid concat split");
    if (d.out_d2s_block > 1 && d.oc % (d.out_d2s_block * d.out_d2s_block) != 0)
        throw std::runtime_error("conv: invalid depth_to_space fusion");
    if (!pointers) return;
    if (d.epilogue == MLVC_EPI_RESIDUAL_ADD && !d.residual) throw std::runtime_error("conv: residual missing");
    if (!d.x || !d.y || !d.packed_w || !d.bias) throw std::runtime_error("conv: null tensor");
}

// A tile variant can run the geometry: kernel size and stride match, 1x1
// variants without padding, flattened 1x1 geometry on one-row tiles only.
bool eligible(const mlvc_hip_conv_desc& d, const Variant& k);

// Geometry as the kernel sees it (1x1 convs run over flattened pixels).
void kernel_geometry(const mlvc_hip_conv_desc& d, int& ih, int& iw, int& oh, int& ow)
{
    if (flat_1x1(d) && d.stride_h == 1 && d.stride_w == 1 && d.pad_h == 0 && d.pad_w == 0) {
        ih = oh = 1;
        iw = ow = d.oh * d.ow;
    } else {
        ih = d.ih;
        iw = d.iw;
        oh = d.oh;
        ow = d.ow;
    }
}

bool eligible(const mlvc_hip_conv_desc& d, const Variant& k)
{
    if (k.bm == 0 || k.kh != d.kh || k.kw != d.kw || k.s != d.stride_h || k.s != d.stride_w) return false;
    if (d.kh == 1 && (d.pad_h || d.pad_w)) return false;
    int ih, iw, oh, ow;
    kernel_geometry(d, ih, iw, oh, ow);
    const bool flat = ih == 1 && oh == 1 && d.kh == 1 && d.kw == 1;
    return !(d.kh == 1 && flat != (k.th == 1));
}

}  // namespace
}  // namespace mlvc_hip

using namespace mlvc_hip;

extern "C" {

int mlvc_hip_conv_plan(mlvc_hip_conv_desc* desc)
{
    return guard([&] {
        validate(*desc, false);
        const mlvc_hip_conv_desc& d = *desc;
        int ih, iw, oh, ow;
        kernel_geometry(d, ih, iw, oh, ow);
        const int slots = 2 * cu_count();
        int best = 0;
        double best_cost = 0.0;
        for (int v = 1; v < kVariantCount; ++v) {
            if (!eligible(d, kVariants[v])) continue;
            const Variant& k = kVariants[v];
            const long tiles = static_cast<long>((oh + k.th - 1) / k.th) * ((ow + k.tw - 1) / k.tw) *
                               ((d.oc + k.bm - 1) / k.bm) * d.n;
            const long rounds = (tiles + slots - 1) / slots;
            // Work per round in MACs plus a fixed per-tile overhead.
            const double cost = static_cast<double>(rounds) * (static_cast<double>(k.bm) * k.th * k.tw + 4096.0);
            if (best == 0 || cost < best_cost) {
                best = v;
                best_cost = cost;
            }
        }
        desc->variant = best;
        // 16-byte row-segment staging: plain or channel-concat input whose
        // split falls on 8 channels, rows of 8-aligned width.
        desc->vector_io = best != 0 && d.in_s2d_block <= 1 && (!d.x2 || d.ic_split % 8 == 0) && iw % 8 == 0;
    });
}

int mlvc_hip_conv_candidates(const mlvc_hip_conv_desc* desc, int* variants, int capacity, int* count)
{
    return guard([&] {
        validate(*desc, false);
        if (!count || (capacity > 0 && !variants)) throw std::runtime_error("conv: null candidate buffer");
        int n = 0;
        for (int v = 1; v < kVariantCount; ++v)
            if (eligible(*desc, kVariants[v])) {
                if (n < capacity) variants[n] = v;
                ++n;
            }
        *count = n;
    });
}

const char* mlvc_hip_conv_variant_name(int variant)
{
    return variant >= 0 && variant < kVariantCount ? kVariants[variant].name : "invalid";
}

size_t mlvc_hip_conv_bias_len(const mlvc_hip_conv_desc* desc)
{
    const Variant& k = variant_of(*desc);
    if (k.bm == 0) return static_cast<size_t>(desc->oc);
    return static_cast<size_t>((desc->oc + k.bm - 1) / k.bm * k.bm);
}

size_t mlvc_hip_conv_packed_bytes(const mlvc_hip_conv_desc* desc)
{
    const mlvc_hip_conv_desc& d = *desc;
    const Variant& k = variant_of(d);
    if (k.bm == 0) return static_cast<size_t>(d.oc) * d.ic * d.kh * d.kw * 2;
    const size_t ocb = static_cast<size_t>((d.oc + k.bm - 1) / k.bm);
    const size_t chunks = static_cast<size_t>((d.ic + k.kc - 1) / k.kc);
    return ocb * chunks * static_cast<size_t>(k.kh * k.kw) * k.kc * k.bm * 2;
}

int mlvc_hip_conv_pack(const mlvc_hip_conv_desc* desc, const uint16_t* w, void* dst_host)
{
    return guard([&] {
        const mlvc_hip_conv_desc& d = *desc;
        const Variant& k = variant_of(d);
        auto* out = static_cast<std::uint16_t*>(dst_host);
        if (k.bm == 0) {
            std::memcpy(out, w, static_cast<size_t>(d.oc) * d.ic * d.kh * d.kw * 2);
            return;
        }
        const int taps = k.kh * k.kw, ks_n = k.kc / 16, mt_n = k.bm / 32;
        const int ocb_n = (d.oc + k.bm - 1) / k.bm, chunks = (d.ic + k.kc - 1) / k.kc;
        size_t o = 0;
        // Layout [ocb][chunk][tap][ks][mt][lane][8]: lane l of m-tile mt
        // holds W[oc = ocb*BM + mt*32 + l%32][ic = chunk*KC + ks*16 + 8*(l/32) + j][tap].
        for (int ocb = 0; ocb < ocb_n; ++ocb)
            for (int ch = 0; ch < chunks; ++ch)
                for (int tap = 0; tap < taps; ++tap)
                    for (int ks = 0; ks < ks_n; ++ks)
                        for (int mt = 0; mt < mt_n; ++mt)
                            for (int lane = 0; lane < 64; ++lane)
                                for (int j = 0; j < 8; ++j) {
                                    const int oc = ocb * k.bm + mt * 32 + (lane & 31);
                                    const int ic = ch * k.kc + ks * 16 + 8 * (lane >> 5) + j;
                                    out[o++] = (oc < d.oc && ic < d.ic)
                                                   ? w[(static_cast<size_t>(oc) * d.ic + ic) * taps + tap]
                                                   : std::uint16_t{0};
                                }
    });
}

int mlvc_hip_conv_launch(const mlvc_hip_conv_desc* desc, mlvc_hip_stream s)
{
    return guard([&] {
        const mlvc_hip_conv_desc& d = *desc;
        validate(d, true);
        const Variant& k = variant_of(d);
        ConvArgs a{};
        a.x = static_cast<const std::uint16_t*>(d.x);
        a.x2 = static_cast<const std::uint16_t*>(d.x2);
        a.w = static_cast<const std::uint16_t*>(d.packed_w);
        a.bias = d.bias;
        a.res = static_cast<const std::uint16_t*>(d.residual);
        a.y = static_cast<std::uint16_t*>(d.y);
        a.ic_split = d.x2 ? d.ic_split : 0;
        a.s2d = d.in_s2d_block;
        a.d2s = d.out_d2s_block;
        a.ic = d.ic;
        a.oc = d.oc;
        a.kh = d.kh;
        a.kw = d.kw;
        a.sh = d.stride_h;
        a.sw = d.stride_w;
        a.ph = d.pad_h;
        a.pw = d.pad_w;
        a.epi = d.epilogue;
        a.alpha = d.alpha;
        if (k.bm == 0) {
            a.ih = d.ih; a.iw = d.iw; a.oh = d.oh; a.ow = d.ow;
            const size_t total = static_cast<size_t>(d.n) * d.oc * d.oh * d.ow;
            const unsigned blocks = static_cast<unsigned>(std::min<size_t>((total + 255) / 256, 65535));
            hipLaunchKernelGGL(conv_direct_kernel, dim3(blocks), dim3(256), 0, to_stream(s), a, d.n);
        } else {
            if (k.kh != d.kh || k.kw != d.kw || k.s != d.stride_h || k.s != d.stride_w)
                throw std::runtime_error("conv: variant does not match the geometry");
            kernel_geometry(d, a.ih, a.iw, a.oh, a.ow);
            if (a.s2d > 1 && a.ih == 1 && d.ih != 1) throw std::runtime_error("conv: flattened geometry with fusion");
            const bool aligned = (reinterpret_cast<std::uintptr_t>(d.x) & 15u) == 0 &&
                                 (!d.x2 || (reinterpret_cast<std::uintptr_t>(d.x2) & 15u) == 0);
            // Buffer offsets of the vector path stay below 2^31 (range check
            // and the out-of-range marker); the concat split falls on a chunk.
            const std::uint64_t plane_bytes = static_cast<std::uint64_t>(a.ih) * a.iw * 2;
            const bool vec = d.vector_io && aligned && a.s2d <= 1 && (!a.x2 || a.ic_split % k.kc == 0) &&
                             a.iw % 8 == 0 && (static_cast<std::uint64_t>(d.ic) + k.kc) * plane_bytes < (1ull << 31);
            a.tiles_x = (a.ow + k.tw - 1) / k.tw;
            a.nchunks = (d.ic + k.kc - 1) / k.kc;
            a.tiles = a.tiles_x * ((a.oh + k.th - 1) / k.th);
            a.ocbs = (d.oc + k.bm - 1) / k.bm;
            const long long nwg = static_cast<long long>(a.tiles) * a.ocbs * d.n;
            if (nwg > 0x7FFFFFFF) throw std::runtime_error("conv: grid too large");
            a.nwg = static_cast<int>(nwg);
            const dim3 grid(static_cast<unsigned>(a.nwg));
            (vec ? k.launch_vec : k.launch_scalar)(a, grid, to_stream(s));
        }
        check(hipGetLastError(), "conv kernel launch");
    });
}

}  // extern "C"
