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
//
// This header holds the kernel template and its configuration; each
// conv_k*.hip file instantiates the tile variants of one kernel size (so the
// families compile in parallel), and conv_igemm.hip assembles the variant
// table, plans and launches.

#pragma once

#include "common.hpp"
#include "mlvc_hip_device.h"

#include <cstring>

namespace mlvc_hip {
namespace conv {


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
    float lo, hi;  // MLVC_EPI_CLAMP / MLVC_EPI_REGLU clip bounds
    int tiles_x, nchunks;
    int tiles, ocbs, nwg;  // pixel tiles per image, output-channel blocks, workgroups (tiles*ocbs*n)
    // Split K: ksplit > 1 workgroups per (tile, output-channel block), split
    // s summing input channels [s * split_c, (s + 1) * split_c) (split_c a
    // multiple of KC) into an FP32 partial part[s][n][oc][oh][ow]; split 0
    // seeds its accumulators with the bias, the others with zero.
    int ksplit, split_c;
    float* part;
    // Channel-last x ([n][ih][iw][ic]) / y ([n][oh][ow][oc]); weight-
    // streaming kernel only.
    int in_nhwc, out_nhwc;
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

// Clamp epilogue on a rounded value: max(min(h, hi), lo) as the reference's
// vector GEMM epilogue computes it (MINPS / MAXPS operand order: a NaN gives
// hi). The bounds are FP16 values, so the result needs no further rounding.
__device__ __forceinline__ std::uint16_t clamp_h(std::uint16_t h, float lo, float hi)
{
    float c = h2f(h);
    c = c < hi ? c : hi;
    c = c > lo ? c : lo;
    return f2h(c);
}
__device__ __forceinline__ std::uint32_t clamp_h2(std::uint32_t h, float lo, float hi)
{
    return clamp_h(static_cast<std::uint16_t>(h), lo, hi) |
           (static_cast<std::uint32_t>(clamp_h(static_cast<std::uint16_t>(h >> 16), lo, hi)) << 16);
}

__device__ __forceinline__ std::uint16_t finish(const ConvArgs& a, float acc, int b, int oc, int oy, int ox)
{
    std::uint16_t h = f2h(acc);
    if (a.epi == MLVC_EPI_CLAMP) {
        h = clamp_h(h, a.lo, a.hi);
    } else if (a.epi == MLVC_EPI_LEAKY_RELU) {
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

// ReGLU of a rounded (gate, linear) pair: fp16(fp16(clip(gate)) * linear),
// the clip as MINPS / MAXPS selects (a NaN gate gives hi, then stays), the
// product a plain FP32 multiply rounded once.
__device__ __forceinline__ std::uint16_t reglu_h(std::uint16_t g, std::uint16_t l, float lo, float hi)
{
    float c = h2f(g);
    c = c < hi ? c : hi;
    c = c > lo ? c : lo;
    return f2h(mul_f32(h2f(f2h(c)), h2f(l)));
}

template <int BM_, int TH_, int TW_, int KH_, int KW_, int S_, int KC_, int STG_, bool DB_, int WM_ = 1, int WNW_ = 4,
          int OCC_ = 2>
struct Cfg {
    static constexpr int BM = BM_, TH = TH_, TW = TW_, KH = KH_, KW = KW_, S = S_, KC = KC_;
    // Input staging: 0 = per-pixel loads through the SPACE_TO_DEPTH / CONCAT
    // maps; 1 = 16-byte row segments of 8 channels, transposed in registers;
    // 2 = 16-byte source-row segments through SPACE_TO_DEPTH(2) (each dword
    // already holds the dx = 0, 1 channel pair of one staged pixel).
    // 1 and 2 need W % 8 == 0.
    static constexpr int STG = STG_;
    static constexpr bool VEC = STG_ != 0;
    // Two LDS stages: chunk k+1 is staged (weights by LDS DMA) while chunk k
    // is multiplied, one barrier per chunk. Otherwise one stage, weights
    // staged through registers, two barriers per chunk, half the LDS.
    static constexpr bool DB = DB_;
    // Waves: WM along the output channels x WNW along the pixels; each wave
    // computes (BM / WM) channels x (BN / WNW) pixels.
    static constexpr int WM = WM_, WNW = WNW_, WAVES = WM_ * WNW_;
    // Register budget: at least OCC waves per SIMD (2 leaves up to 256
    // registers for the large tiles; short-K layers want more waves to hide
    // their per-tile load latency).
    static constexpr int OCC = OCC_;
    static constexpr int kThreads = 64 * WAVES;
    static constexpr int BN = TH * TW;
    static constexpr int TAPS = KH * KW;
    static constexpr int KS = KC / 16;  // 16-deep MFMA K steps per tap
    static constexpr int MTT = BM / 32;  // m-tiles of the workgroup (weight layout)
    static constexpr int MT = MTT / WM;  // m-tiles per wave
    static constexpr int WN = BN / WNW;  // pixels per wave
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
    static constexpr int UNITS2 = IH_T * NSEG;  // STG 2: 8 staged pixels x all KC channels
    static constexpr int UNITS2_PER_T = (UNITS2 + kThreads - 1) / kThreads;
    static constexpr int IN_PIX = IH_T * IW_T;
    static constexpr int PIX_PER_T = (IN_PIX + kThreads - 1) / kThreads;
    static constexpr int W_LDS = TAPS * KS * MTT * 64 * 8;  // halves per chunk
    static constexpr int W_VEC = W_LDS / 8;
    static constexpr int W_PER_T = (W_VEC + kThreads - 1) / kThreads;
    static constexpr int EPI_ROW = BN + 8;  // output staging row (one channel), halves
    static constexpr int EPI_LDS = BM * EPI_ROW;
    static constexpr int STAGE = IN_LDS + W_LDS;
    static constexpr int W_INST = W_VEC / 64;  // 1 KB LDS DMA instructions per chunk
    static constexpr int LDS = (DB ? 2 * STAGE : STAGE) > EPI_LDS ? (DB ? 2 * STAGE : STAGE) : EPI_LDS;
    static_assert(BM % 32 == 0 && MTT % WM == 0 && WN % 32 == 0 && BN % WNW == 0 && KC % 16 == 0 && TW % 8 == 0 &&
                      W_VEC % 64 == 0,
                  "tile shape");
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
__global__ __launch_bounds__(C::kThreads) __attribute__((amdgpu_waves_per_eu(C::OCC))) void conv_mfma_kernel(ConvArgs a)
{
    __shared__ __attribute__((aligned(16))) std::uint16_t lds[C::LDS];
    auto lds_in = [&](int stage) { return lds + stage * C::STAGE; };
    auto lds_w = [&](int stage) { return lds + stage * C::STAGE + C::IN_LDS; };

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / C::WNW, wn = wave % C::WNW;  // this wave's channel and pixel slices
    const int mt0 = wm * C::MT;                        // first m-tile of this wave
    // Logical work item: output-channel block fastest, then pixel tiles in
    // row-major order, then images; each XCD runs a contiguous range of them.
    // With split K the splits are outermost, so an XCD's range shares one
    // split's weights.
    const int item_all = xcd_order(blockIdx.x, a.nwg * a.ksplit);
    const int split = item_all / a.nwg, item = item_all - split * a.nwg;
    const int ocb = item % a.ocbs, tile = (item / a.ocbs) % a.tiles, b = item / (a.ocbs * a.tiles);
    const int chunk0 = split * (a.split_c / C::KC);
    const int chunk1 = a.ksplit > 1 ? min(a.nchunks, chunk0 + a.split_c / C::KC) : a.nchunks;
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
            const float bv = split == 0 ? a.bias[ocb * C::BM + (mt0 + mt) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3)] : 0.0f;
#pragma unroll
            for (int nt = 0; nt < C::NT; ++nt) acc[mt][nt][r] = bv;
        }

    const size_t hw = static_cast<size_t>(a.ih) * a.iw;
    const int c1 = a.x2 ? a.ic_split : a.ic;
    u32x4 vin[C::STG == 1 ? C::UNITS_PER_T : 1][8];
    u32x4 vs2[C::STG == 2 ? C::UNITS2_PER_T : 1][C::STG == 2 ? C::KC / 4 : 1][2][2];
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
    std::uint32_t pix_off[C::STG == 1 ? C::UNITS_PER_T : 1];
    int unit_c8[C::STG == 1 ? C::UNITS_PER_T : 1];
    // STG 2: the source image is [IC/4][2*IH][2*IW]; staged pixel (iy, ix)
    // channel 4*cs + 2*dy + dx is source (cs, 2*iy + dy, 2*ix + dx).
    const int sw2 = a.iw * 2, sh2 = a.ih * 2;
    const std::uint32_t splane2 = static_cast<std::uint32_t>(sw2) * sh2 * 2u;  // bytes per source channel
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<std::uint16_t*>(a.x + static_cast<size_t>(b) * (a.ic / 4) * sw2 * sh2), 0,
        static_cast<int>(C::STG == 2 ? (a.ic / 4) * splane2 : 0u), kRawBufferFlags);
    std::uint32_t src_off[C::STG == 2 ? C::UNITS2_PER_T : 1];
    if constexpr (C::STG == 2) {
#pragma unroll
        for (int i = 0; i < C::UNITS2_PER_T; ++i) {
            const int u = tid + i * C::kThreads;
            const int yi = u % C::IH_T, sg = (u / C::IH_T) % C::NSEG;
            const int iy = iy0 + yi, ix = xa + sg * 8;
            const bool ok = u < C::UNITS2 && iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw;
            src_off[i] = ok ? static_cast<std::uint32_t>(2 * iy * sw2 + 2 * ix) * 2u : kOutOfRange;
        }
    }
    if constexpr (C::STG == 1) {
#pragma unroll
        for (int i = 0; i < C::UNITS_PER_T; ++i) {
            const int u = tid + i * C::kThreads;
            const int sg = u % C::NSEG, yi = (u / C::NSEG) % C::IH_T;
            const int iy = iy0 + yi, ix = xa + sg * 8;
            const bool ok = u < C::UNITS && iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw;
            pix_off[i] = ok ? static_cast<std::uint32_t>(iy * a.iw + ix) * 2u : kOutOfRange;
            unit_c8[i] = u / (C::NSEG * C::IH_T);  // units: segments fastest, then rows, then channel groups
        }
    }
    auto fetch = [&](int chunk, int stage) {
        const int c0 = chunk * C::KC;
        if constexpr (C::STG == 2) {
            // Per unit and source channel: rows 2*iy and 2*iy + 1, 32 bytes
            // (16 source columns = 8 staged pixels x dx) each. Channels past
            // IC/4 fall past the end of the resource and read zeros.
            const std::uint32_t cs0 = static_cast<std::uint32_t>(c0 / 4);
#pragma unroll
            for (int i = 0; i < C::UNITS2_PER_T; ++i)
#pragma unroll
                for (int q = 0; q < C::KC / 4; ++q)
#pragma unroll
                    for (int dy = 0; dy < 2; ++dy)
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh) {
                            const std::uint32_t off =
                                src_off[i] == kOutOfRange
                                    ? kOutOfRange
                                    : src_off[i] + (cs0 + q) * splane2 + static_cast<std::uint32_t>(dy * sw2 * 2 + hh * 16);
                            vs2[i][q][dy][hh] = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(off), 0, 0);
                        }
        } else if constexpr (C::STG == 1) {
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
            for (int i = 0; i < (C::W_INST + C::WAVES - 1) / C::WAVES; ++i) {
                const int j = wave + C::WAVES * i;
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
        if constexpr (C::STG == 2) {
            // Staged pixel j of the unit: dword j%4 of source half j/4 holds
            // its (dx = 0, 1) pair for each (cs, dy); 8 channels per write.
#pragma unroll
            for (int i = 0; i < C::UNITS2_PER_T; ++i) {
                const int u = tid + i * C::kThreads;
                if (u < C::UNITS2) {
                    const int yi = u % C::IH_T, sg = (u / C::IH_T) % C::NSEG;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const int hh = j >> 2, w = j & 3;
#pragma unroll
                        for (int g = 0; g < C::KC / 8; ++g) {
                            const u32x4 t = {vs2[i][2 * g][0][hh][w], vs2[i][2 * g][1][hh][w], vs2[i][2 * g + 1][0][hh][w],
                                             vs2[i][2 * g + 1][1][hh][w]};
                            *reinterpret_cast<u32x4*>(&in_s[C::at(yi, sg * 8 + j) + g * 8]) = t;
                        }
                    }
                }
            }
        } else if constexpr (C::STG == 1) {
            // 8x8 transpose in registers: staged pixel j of the segment gets
            // the 8 channels of the unit as one 16-byte LDS write.
#pragma unroll
            for (int i = 0; i < C::UNITS_PER_T; ++i) {
                const int u = tid + i * C::kThreads;
                if (u < C::UNITS) {
                    const int sg = u % C::NSEG, yi = (u / C::NSEG) % C::IH_T, c8 = u / (C::NSEG * C::IH_T);
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
        const int p = wn * C::WN + nt * 32 + (lane & 31);
        pyi[nt] = (p / C::TW) * C::S;
        pxi[nt] = (p % C::TW) * C::S + col_off;
    }
    const int koff = (lane >> 5) * 8;

    // K order within a chunk: 16-channel step outer, tap inner, so a chunk
    // of 32 channels accumulates exactly like two chunks of 16 and every
    // variant of one kernel size gives the same bits.
    auto compute = [&](int stage) {
        const std::uint16_t* const in_s = lds_in(stage);
        const std::uint16_t* const w_s = lds_w(stage);
#pragma unroll
        for (int ks = 0; ks < C::KS; ++ks)
#pragma unroll
            for (int tap = 0; tap < C::TAPS; ++tap) {
                const int ky = tap / C::KW, kx = tap % C::KW;
                half8 av[C::MT], bv[C::NT];
#pragma unroll
                for (int mt = 0; mt < C::MT; ++mt)
                    av[mt] = *reinterpret_cast<const half8*>(&w_s[(((tap * C::KS + ks) * C::MTT + mt0 + mt) * 64 + lane) * 8]);
#pragma unroll
                for (int nt = 0; nt < C::NT; ++nt)
                    bv[nt] = *reinterpret_cast<const half8*>(&in_s[C::at(pyi[nt] + ky, pxi[nt] + kx) + koff + ks * 16]);
#pragma unroll
                for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
                    for (int nt = 0; nt < C::NT; ++nt)
                        acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[mt], bv[nt], acc[mt][nt], 0, 0, 0);
            }
    };

    if constexpr (C::DB) {
        fetch(chunk0, 0);
        commit(0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's LDS DMA has landed
        __syncthreads();
        for (int chunk = chunk0; chunk < chunk1; ++chunk) {
            const int cur = (chunk - chunk0) & 1;
            const bool more = chunk + 1 < chunk1;
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
        fetch(chunk0, 0);
        commit(0);
        __syncthreads();
        for (int chunk = chunk0; chunk < chunk1; ++chunk) {
            const bool more = chunk + 1 < chunk1;
            if (more) fetch(chunk + 1, 0);
            compute(0);
            __syncthreads();
            if (more) {
                commit(0);
                __syncthreads();
            }
        }
    }

    // Epilogue. Lane l of accumulator (mt, nt) holds output channels oc0 + i,
    // oc0 = ocb*BM + (mt0 + mt)*32 + 8j + 4*(l/32) (j, i = 0..3), of tile pixel
    // wn*WN + nt*32 + l%32: 32 lanes hold 32 consecutive pixels of each
    // channel. Values are rounded to FP16 first and the epilogue acts on the
    // rounded value. With a fused DEPTH_TO_SPACE(2) the 4 channels of a lane
    // are the (dy, dx) block of output channel oc0/4, so the stores go
    // straight from registers: two 4-byte pairs per lane, 32 lanes covering
    // 128 contiguous bytes of a row. Plain outputs go through an LDS
    // [channel][pixel] tile and leave as 16-byte rows.
    if (a.ksplit > 1) {
        // Split K: the FP32 partial of this split, in the conv's output
        // geometry (the reduce kernel rounds, applies the epilogue and the
        // DEPTH_TO_SPACE store). 32 lanes write 32 consecutive pixels.
        const size_t ohw = static_cast<size_t>(a.oh) * a.ow;
        float* const pd = a.part + (static_cast<size_t>(split) * (a.nwg / (a.tiles * a.ocbs)) + b) * a.oc * ohw;
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < C::NT; ++nt) {
                const int p = wn * C::WN + nt * 32 + (lane & 31);
                const int oy = ty0 + (p / C::TW), ox = tx0 + (p % C::TW);
                if (oy >= a.oh || ox >= a.ow) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int oc = ocb * C::BM + (mt0 + mt) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (oc < a.oc) pd[oc * ohw + static_cast<size_t>(oy) * a.ow + ox] = acc[mt][nt][r];
                }
            }
        return;
    }
    const bool max_form = a.alpha >= 0.0f && a.alpha <= 1.0f;
    if (a.d2s == 2) {
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < C::NT; ++nt) {
                const int p = wn * C::WN + nt * 32 + (lane & 31);
                const int oy = ty0 + (p / C::TW), ox = tx0 + (p % C::TW);
                const bool inside = oy < a.oh && ox < a.ow;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int oc0 = ocb * C::BM + (mt0 + mt) * 32 + 8 * j + 4 * (lane >> 5);
                    const float v[4] = {acc[mt][nt][4 * j], acc[mt][nt][4 * j + 1], acc[mt][nt][4 * j + 2],
                                        acc[mt][nt][4 * j + 3]};
                    std::uint32_t h01, h23;
                    if (a.epi == MLVC_EPI_LEAKY_RELU) {
                        h01 = leaky_pair(v[0], v[1], a.alpha, max_form);
                        h23 = leaky_pair(v[2], v[3], a.alpha, max_form);
                    } else {
                        h01 = pack_f16(v[0], v[1]);
                        h23 = pack_f16(v[2], v[3]);
                        if (a.epi == MLVC_EPI_CLAMP) {
                            h01 = clamp_h2(h01, a.lo, a.hi);
                            h23 = clamp_h2(h23, a.lo, a.hi);
                        }
                        if (a.epi == MLVC_EPI_RESIDUAL_ADD && inside) {
                            std::uint16_t r[4];
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                r[i] = oc0 + i < a.oc ? a.res[(static_cast<size_t>(b * a.oc + oc0 + i) * a.oh + oy) * a.ow + ox] : 0;
                            h01 = f2h(lo_f16(h01) + h2f(r[0])) | (static_cast<std::uint32_t>(f2h(hi_f16(h01) + h2f(r[1]))) << 16);
                            h23 = f2h(lo_f16(h23) + h2f(r[2])) | (static_cast<std::uint32_t>(f2h(hi_f16(h23) + h2f(r[3]))) << 16);
                        }
                    }
                    if (!inside) continue;
                    if (oc0 >= a.oc) continue;
                    const int W2 = a.ow * 2;
                    std::uint16_t* dst = a.y + (static_cast<size_t>(b * (a.oc / 4) + oc0 / 4) * (a.oh * 2) + oy * 2) * W2 + ox * 2;
                    *reinterpret_cast<std::uint32_t*>(dst) = h01;
                    *reinterpret_cast<std::uint32_t*>(dst + W2) = h23;
                }
            }
        return;
    }

    // LDS path, stage 1: each lane writes its FP16-rounded accumulators into
    // an LDS tile [oc][pixel] (all indices static, so nothing spills).
    // The main loop ended with a barrier, so the staging buffers are free.
#pragma unroll
    for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < C::NT; ++nt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int ocl = (mt0 + mt) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int pl = wn * C::WN + nt * 32 + (lane & 31);
                lds[ocl * C::EPI_ROW + pl] = f2h(acc[mt][nt][r]);
            }
    __syncthreads();

    // ReGLU: the tile's rows 64k + i (gate) and 64k + 32 + i (linear) give
    // output channel ocb * BM/2 + 32k + i of the G-channel output.
    if (a.epi == MLVC_EPI_REGLU) {
        const int half = a.oc / 2;
        const size_t hw_out = static_cast<size_t>(a.oh) * a.ow;
        if (a.ow % 8 == 0) {
            constexpr int GROUPS = C::BN / 8;
            for (int u = tid; u < (C::BM / 2) * GROUPS; u += C::kThreads) {
                const int g = u % GROUPS, ol = u / GROUPS, rg = (ol / 32) * 64 + ol % 32;
                const int oc = ocb * (C::BM / 2) + ol;
                const int pl = g * 8, oy = ty0 + pl / C::TW, ox = tx0 + pl % C::TW;
                if (oc >= half || oy >= a.oh || ox >= a.ow) continue;
                const u32x4 hg = *reinterpret_cast<const u32x4*>(&lds[rg * C::EPI_ROW + pl]);
                const u32x4 hl = *reinterpret_cast<const u32x4*>(&lds[(rg + 32) * C::EPI_ROW + pl]);
                u32x4 o;
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    o[k] = reglu_h(static_cast<std::uint16_t>(hg[k]), static_cast<std::uint16_t>(hl[k]), a.lo, a.hi) |
                           (static_cast<std::uint32_t>(reglu_h(static_cast<std::uint16_t>(hg[k] >> 16),
                                                               static_cast<std::uint16_t>(hl[k] >> 16), a.lo, a.hi))
                            << 16);
                *reinterpret_cast<u32x4*>(a.y + (static_cast<size_t>(b) * half + oc) * hw_out + static_cast<size_t>(oy) * a.ow + ox) = o;
            }
        } else {
            for (int e = tid; e < (C::BM / 2) * C::BN; e += C::kThreads) {
                const int ol = e / C::BN, pl = e - ol * C::BN, rg = (ol / 32) * 64 + ol % 32;
                const int oc = ocb * (C::BM / 2) + ol;
                const int oy = ty0 + pl / C::TW, ox = tx0 + pl % C::TW;
                if (oc < half && oy < a.oh && ox < a.ow)
                    a.y[(static_cast<size_t>(b) * half + oc) * hw_out + static_cast<size_t>(oy) * a.ow + ox] =
                        reglu_h(lds[rg * C::EPI_ROW + pl], lds[(rg + 32) * C::EPI_ROW + pl], a.lo, a.hi);
            }
        }
        return;
    }

    // Stage 2: the epilogue acts on the rounded value. Vector path: 8
    // consecutive pixels of a channel per thread, 16-byte loads and stores.
    if (a.ow % 8 == 0 && a.d2s <= 1) {
        constexpr int GROUPS = C::BN / 8;
        for (int u = tid; u < C::BM * GROUPS; u += C::kThreads) {
            const int g = u % GROUPS, ocl = u / GROUPS, oc = ocb * C::BM + ocl;
            const int pl = g * 8, oy = ty0 + pl / C::TW, ox = tx0 + pl % C::TW;
            if (oc >= a.oc || oy >= a.oh || ox >= a.ow) continue;
            u32x4 h = *reinterpret_cast<const u32x4*>(&lds[ocl * C::EPI_ROW + pl]);
            const size_t o = (static_cast<size_t>(b * a.oc + oc) * a.oh + oy) * a.ow + ox;
            if (a.epi == MLVC_EPI_LEAKY_RELU) {
#pragma unroll
                for (int k = 0; k < 4; ++k) h[k] = leaky_h2(h[k], a.alpha, max_form);
            } else if (a.epi == MLVC_EPI_CLAMP) {
#pragma unroll
                for (int k = 0; k < 4; ++k) h[k] = clamp_h2(h[k], a.lo, a.hi);
            } else if (a.epi == MLVC_EPI_RESIDUAL_ADD) {
                const u32x4 r = *reinterpret_cast<const u32x4*>(a.res + o);
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    h[k] = f2h(lo_f16(h[k]) + lo_f16(r[k])) | (static_cast<std::uint32_t>(f2h(hi_f16(h[k]) + hi_f16(r[k]))) << 16);
            }
            *reinterpret_cast<u32x4*>(a.y + o) = h;
        }
        return;
    }
    // Element by element (ragged widths, other DEPTH_TO_SPACE blocks).
    for (int e = tid; e < C::BM * C::BN; e += C::kThreads) {
        const int ocl = e / C::BN, pl = e - ocl * C::BN;
        const int oc = ocb * C::BM + ocl;
        const int oy = ty0 + pl / C::TW, ox = tx0 + pl % C::TW;
        if (oc < a.oc && oy < a.oh && ox < a.ow) {
            std::uint16_t h = lds[ocl * C::EPI_ROW + pl];
            if (a.epi == MLVC_EPI_LEAKY_RELU) {
                const float f = h2f(h);
                if (f < 0.0f) h = leaky_f16(f, a.alpha);
            } else if (a.epi == MLVC_EPI_CLAMP) {
                h = clamp_h(h, a.lo, a.hi);
            } else if (a.epi == MLVC_EPI_RESIDUAL_ADD) {
                h = f2h(h2f(h) + h2f(a.res[(static_cast<size_t>(b * a.oc + oc) * a.oh + oy) * a.ow + ox]));
            }
            store_output(a, h, b, oc, oy, ox);
        }
    }
}

struct Variant {
    const char* name;
    int bm, th, tw, kh, kw, s, kc;  // bm == 0: direct fallback
    void (*launch_scalar)(const ConvArgs&, dim3, hipStream_t);
    void (*launch_vec)(const ConvArgs&, dim3, hipStream_t);
    void (*launch_s2d)(const ConvArgs&, dim3, hipStream_t);  // SPACE_TO_DEPTH(2) staging, or null
    // Weight-streaming kernel (conv_ws.hpp) staging ws_ic input channels
    // per pass; 0 for conv_mfma_kernel variants.
    int ws_ic = 0;
    // Its channel-last output tile fits the LDS: bit 0 plain, bit 1 with
    // DEPTH_TO_SPACE(2).
    int nhwc_out = 0;
};

template <class C>
void launch_mfma(const ConvArgs& a, dim3 grid, hipStream_t s)
{
    hipLaunchKernelGGL(conv_mfma_kernel<C>, grid, dim3(C::kThreads), 0, s, a);
}

#define MLVC_VARIANT(BM, TH, TW, KH, KW, S, KC)                                                              \
    Variant{"mfma_bm" #BM "_" #TH "x" #TW "_k" #KH "x" #KW "_s" #S "_kc" #KC, BM, TH, TW, KH, KW, S, KC,        \
            &launch_mfma<Cfg<BM, TH, TW, KH, KW, S, KC, 0, false>>, &launch_mfma<Cfg<BM, TH, TW, KH, KW, S, KC, 1, false>>, nullptr}
// 8-wave (or other) workgroups: WM waves along the channels x WNW along the pixels.
#define MLVC_VARIANT_W(BM, TH, TW, KH, KW, S, KC, WM, WNW)                                                      \
    Variant{"mfma_bm" #BM "_" #TH "x" #TW "_k" #KH "x" #KW "_s" #S "_kc" #KC "_w" #WM "x" #WNW, BM, TH, TW, KH, KW, S, \
            KC, &launch_mfma<Cfg<BM, TH, TW, KH, KW, S, KC, 0, false, WM, WNW>>,                                      \
            &launch_mfma<Cfg<BM, TH, TW, KH, KW, S, KC, 1, false, WM, WNW>>, nullptr}
// Higher-occupancy build (register budget for OCC waves per SIMD).
#define MLVC_VARIANT_OCC(BM, TH, TW, KH, KW, S, KC, OCC)                                                          \
    Variant{"mfma_bm" #BM "_" #TH "x" #TW "_k" #KH "x" #KW "_s" #S "_kc" #KC "_occ" #OCC, BM, TH, TW, KH, KW, S, KC,  \
            &launch_mfma<Cfg<BM, TH, TW, KH, KW, S, KC, 0, false, 1, 4, OCC>>,                                      \
            &launch_mfma<Cfg<BM, TH, TW, KH, KW, S, KC, 1, false, 1, 4, OCC>>, nullptr}
// Waves and occupancy both set (small tiles: more workgroups per CU).
#define MLVC_VARIANT_WO(BM, TH, TW, KH, KW, S, KC, WM, WNW, OCC)                                                    \
    Variant{"mfma_bm" #BM "_" #TH "x" #TW "_k" #KH "x" #KW "_s" #S "_kc" #KC "_w" #WM "x" #WNW "_occ" #OCC, BM, TH, \
            TW, KH, KW, S, KC, &launch_mfma<Cfg<BM, TH, TW, KH, KW, S, KC, 0, false, WM, WNW, OCC>>,                      \
            &launch_mfma<Cfg<BM, TH, TW, KH, KW, S, KC, 1, false, WM, WNW, OCC>>, nullptr}
// With SPACE_TO_DEPTH(2) vector staging.
#define MLVC_VARIANT_S2D(BM, TH, TW, KH, KW, S, KC)                                                          \
    Variant{"mfma_bm" #BM "_" #TH "x" #TW "_k" #KH "x" #KW "_s" #S "_kc" #KC, BM, TH, TW, KH, KW, S, KC,        \
            &launch_mfma<Cfg<BM, TH, TW, KH, KW, S, KC, 0, false>>, &launch_mfma<Cfg<BM, TH, TW, KH, KW, S, KC, 1, false>>, \
            &launch_mfma<Cfg<BM, TH, TW, KH, KW, S, KC, 2, false>>}
// Two-stage pipeline (vector staging only; the scalar staging path keeps the one-stage kernel).
#define MLVC_VARIANT_DB(BM, TH, TW, KH, KW, S, KC)                                                           \
    Variant{"mfma_bm" #BM "_" #TH "x" #TW "_k" #KH "x" #KW "_s" #S "_kc" #KC "_db", BM, TH, TW, KH, KW, S, KC,  \
            &launch_mfma<Cfg<BM, TH, TW, KH, KW, S, KC, 0, false>>, &launch_mfma<Cfg<BM, TH, TW, KH, KW, S, KC, 1, true>>, nullptr}

}  // namespace conv
}  // namespace mlvc_hip
