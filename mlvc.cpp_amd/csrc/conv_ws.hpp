// Weight-streaming MFMA implicit GEMM for the MFMA-bound KxK convs.
//
//   D[oc, p] = bias[oc] + sum_k W[oc, k] X[k, p],  k = (16-channel step, tap)
//
// Same product order and rounding as conv_mfma_kernel (conv_kernel.hpp), so
// every variant of a kernel size gives the same bits; different data flow:
//   * the input halo of the tile is staged into LDS channel-last,
//     [row][pixel][SC + 8], SC channels per pass (all of them in one pass
//     when IC <= SC), from 16-byte NCHW row segments transposed in
//     registers; the K loop then runs all (16-channel step, tap) steps of
//     the pass with no barrier;
//   * the waves split the output channels (wave w owns m-tiles
//     w*MT .. w*MT + MT - 1) and each streams its own A fragments (weights
//     pre-packed in fragment order, [ocb][c16][tap][m-tile][lane][8]) from
//     L2 straight into a register ring three steps deep, so weights never
//     pass through LDS and no two waves of a workgroup fetch the same ones;
//   * every wave covers all BN pixels, reading its B fragments from the
//     staged halo;
//   * two workgroups per CU (halo <= 80 KB, 128 accumulator registers), so
//     one workgroup's staging and epilogue overlap the other's MFMAs;
//   * a channel-last input ([n][h][w][c], from a producer that hands its
//     output over that way) is staged into the same halo layout as 16-byte
//     pieces of 8 channels of one pixel, channel groups fastest across the
//     lanes, with no transposes; a channel-last output leaves through a
//     [pixel][channel] LDS tile as 16-byte pieces of 8 channels.
// The conv kernel it competes with stages 16 input channels of weights and
// input per chunk through registers and LDS with two barriers each; per
// 128x256 tile that re-reads every weight once per 16 channels for each
// workgroup, which phase timing showed to be 70% of its staging traffic.

#pragma once

#include "conv_kernel.hpp"

namespace mlvc_hip {
namespace conv {

template <int BM_, int TH_, int TW_, int SC_, int OCC_ = 2, int S_ = 1, int WAVES_ = 4, int RING_ = 3, bool PIPE_ = false,
          bool CL_D2S_ = false>
struct WsCfg {
    static constexpr int BM = BM_, TH = TH_, TW = TW_, SC = SC_, OCC = OCC_, S = S_;
    static constexpr int KH = 3, KW = 3, TAPS = 9;
    static constexpr int WAVES = WAVES_, kThreads = 64 * WAVES;
    static constexpr int BN = TH * TW, MTT = BM / 32, MT = MTT / WAVES, NT = BN / 32;
    static constexpr int IH_T = (TH - 1) * S + 3, IW_T = (TW - 1) * S + 3;
    // Staged columns: the halo plus up to 7 columns of 8-alignment on the left.
    // With stride 2, even input columns fill the first HALF of a row and odd
    // ones the second, so the 32 pixels of a B fragment read consecutive
    // entries for every tap.
    static constexpr int NSEG = (IW_T + 14) / 8, IW_S = NSEG * 8, HALF = IW_S / 2;
    static constexpr int PST = SC + 8;               // halves per staged pixel
    static constexpr int ROW = IW_S * PST + 8;       // rows start 4 banks apart
    static constexpr int IN_LDS = IH_T * ROW;
    static constexpr int UNITS = (SC / 8) * IH_T * NSEG;  // 8 channels x 8 columns each
    static constexpr int UNITS_PER_T = (UNITS + kThreads - 1) / kThreads;
    static constexpr int EPI_ROW = BN + 8, EPI_LDS = BM * EPI_ROW;
    // Channel-last input: 16-byte pieces, 8 channels of one staged pixel
    // each (as many as the NCHW units' row loads, so the same registers).
    static constexpr int NPIECE = (SC / 8) * IH_T * IW_S;
    static constexpr int NP_PER_T = (NPIECE + kThreads - 1) / kThreads;
    // Pipelined passes: two halo buffers; pass p+1 is loaded into registers
    // at the start of pass p and written to the other buffer after its first
    // 16-channel step, so one barrier per pass and no exposed staging after
    // the first pass.
    static constexpr bool PIPE = PIPE_;
    static constexpr int NBUF = PIPE ? 2 : 1;
    // Channel-last output: [pixel][BM + 8] tile, or with DEPTH_TO_SPACE(2)
    // [subpixel][pixel][BM/4 + 8], where it fits the LDS (bit 0: plain,
    // bit 1: DEPTH_TO_SPACE). CL_D2S sizes the LDS for the second one.
    static constexpr int EPI_ROW_N = BM + 8, EPI_ROW_D = BM / 4 + 8;
    static constexpr int LDS_HALO = NBUF * IN_LDS > EPI_LDS ? NBUF * IN_LDS : EPI_LDS;  // the plain epilogue's tile aliases the halo
    static constexpr int LDS = CL_D2S_ && 4 * BN * EPI_ROW_D > LDS_HALO ? 4 * BN * EPI_ROW_D : LDS_HALO;
    static constexpr int RING = RING_;               // A-fragment prefetch distance in k-steps
    // Staging units in flight per thread: 2, or 1 where the accumulators and
    // the ring leave no room for a second unit's 32 registers.
    static constexpr int STAGE_BATCH = MT * NT * 16 + RING * MT * 4 > 160 ? 1 : 2;
    static_assert(MTT % WAVES == 0 && MT >= 1 && BN % 32 == 0 && TW % 8 == 0 && SC % 16 == 0, "tile shape");
    static_assert(S == 1 || S == 2, "stride");
    static_assert(TAPS % RING == 0, "ring slots are static per tap");
    static_assert(LDS * 2 * OCC <= 160 * 1024, "LDS budget");
    static_assert(NP_PER_T <= UNITS_PER_T * 8, "channel-last staging registers");
    static constexpr bool NHWC_EPI = BN * EPI_ROW_N <= LDS, NHWC_D2S_EPI = 4 * BN * EPI_ROW_D <= LDS;
    static constexpr int NHWC_OUT = (NHWC_EPI ? 1 : 0) | (NHWC_D2S_EPI ? 2 : 0);
    __device__ static constexpr int at(int row, int x) { return row * ROW + x * PST; }
};

template <class C>
__global__ __launch_bounds__(C::kThreads) __attribute__((amdgpu_waves_per_eu(C::OCC))) void conv_ws_kernel(ConvArgs a)
{
    __shared__ __attribute__((aligned(16))) std::uint16_t lds[C::LDS];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int item = xcd_order(blockIdx.x, a.nwg);
    const int ocb = item % a.ocbs, tile = (item / a.ocbs) % a.tiles, b = item / (a.ocbs * a.tiles);
    const int tx0 = (tile % a.tiles_x) * C::TW, ty0 = (tile / a.tiles_x) * C::TH;
    const int iy0 = ty0 * C::S - a.ph, ix0 = tx0 * C::S - a.pw;
    const int xa = ix0 - (((ix0 % 8) + 8) % 8);  // first staged column, 8-aligned
    const int col_off = ix0 - xa;
    const int mt0 = wave * C::MT, hsel = 4 * (lane >> 5);
    const int nsteps16 = a.nchunks;  // 16-channel steps over all input channels

    // Halo of channels [cb, cb + SC) into LDS, 16-byte NCHW row segments
    // transposed in registers. Unit u: 8 consecutive channels x 8 columns of
    // one halo row (segments fastest, then rows, then channel groups). Raw
    // buffer loads: rows and columns outside the image and channels past IC
    // read zeros.
    const size_t hw = static_cast<size_t>(a.ih) * a.iw;
    const std::uint32_t hw2 = static_cast<std::uint32_t>(hw) * 2u;
    const std::uint16_t* x_img = a.x + static_cast<size_t>(b) * a.ic * hw;
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<std::uint16_t*>(x_img), 0, static_cast<int>(a.ic * hw2), kRawBufferFlags);
    // Unit i of this thread (units i0 .. i0 + N - 1 in v[0 .. N-1]): issue
    // its eight row loads, then write it transposed into the halo buffer at
    // LDS offset boff.
    auto unit_off = [&](int cb, int i) -> std::uint32_t {
        const int u = tid + i * C::kThreads;
        const int sg = u % C::NSEG, yi = (u / C::NSEG) % C::IH_T, c8 = u / (C::NSEG * C::IH_T);
        const int iy = iy0 + yi, ix = xa + sg * 8;
        const bool ok = i < C::UNITS_PER_T && u < C::UNITS && iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw;
        return ok ? static_cast<std::uint32_t>(iy * a.iw + ix) * 2u + static_cast<std::uint32_t>(cb + c8 * 8) * hw2 : kOutOfRange;
    };
    auto load_row = [&](std::uint32_t off, int k) {  // channel k of a unit
        return __builtin_amdgcn_raw_buffer_load_b128(rx, static_cast<int>(off == kOutOfRange ? off : off + k * hw2), 0, 0);
    };
    auto issue = [&](int cb, int i, u32x4 (&v)[8]) {
        const std::uint32_t off = unit_off(cb, i);
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = load_row(off, k);
    };
    auto put = [&](int i, const u32x4 (&v)[8], int boff) {
        const int u = tid + i * C::kThreads;
        if (i >= C::UNITS_PER_T || u >= C::UNITS) return;
        const int sg = u % C::NSEG, yi = (u / C::NSEG) % C::IH_T, c8 = u / (C::NSEG * C::IH_T);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const bool up = j & 1;
            const int wd = j >> 1;
            const u32x4 t = {pack_half(v[0][wd], v[1][wd], up), pack_half(v[2][wd], v[3][wd], up),
                             pack_half(v[4][wd], v[5][wd], up), pack_half(v[6][wd], v[7][wd], up)};
            const int col = C::S == 1 ? sg * 8 + j : (j & 1) * C::HALF + sg * 4 + (j >> 1);
            *reinterpret_cast<u32x4*>(&lds[boff + C::at(yi, col) + c8 * 8]) = t;
        }
    };
    // Channel-last piece q (thread t stages q = t + i * kThreads): channel
    // group q % (SC/8) of staged pixel q / (SC/8), columns fastest, then
    // rows; past the image, the pass or IC (a partial last pass) it reads
    // zeros.
    auto piece_off = [&](int cb, int q) -> std::uint32_t {
        const int c8 = q % (C::SC / 8), pix = q / (C::SC / 8), col = pix % C::IW_S, yi = pix / C::IW_S;
        const int iy = iy0 + yi, ix = xa + col, c = cb + 8 * c8;
        const bool ok = q < C::NPIECE && iy >= 0 && iy < a.ih && ix >= 0 && ix < a.iw && c < a.ic;
        return ok ? (static_cast<std::uint32_t>(iy * a.iw + ix) * static_cast<std::uint32_t>(a.ic) + c) * 2u : kOutOfRange;
    };
    auto load_piece = [&](std::uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(rx, static_cast<int>(off), 0, 0); };
    auto piece_put = [&](int q, const u32x4& v, int boff) {
        if (q >= C::NPIECE) return;
        const int c8 = q % (C::SC / 8), pix = q / (C::SC / 8), col = pix % C::IW_S, yi = pix / C::IW_S;
        const int lc = C::S == 1 ? col : (col & 1) * C::HALF + (col >> 1);
        *reinterpret_cast<u32x4*>(&lds[boff + C::at(yi, lc) + c8 * 8]) = v;
    };
    auto stage = [&](int cb) {
        if (a.in_nhwc) {
            constexpr int PB = 8;  // pieces in flight per thread
#pragma unroll
            for (int i0 = 0; i0 < C::NP_PER_T; i0 += PB) {
                u32x4 v[PB];
#pragma unroll
                for (int ii = 0; ii < PB; ++ii)
                    if (i0 + ii < C::NP_PER_T) v[ii] = load_piece(piece_off(cb, tid + (i0 + ii) * C::kThreads));
#pragma unroll
                for (int ii = 0; ii < PB; ++ii)
                    if (i0 + ii < C::NP_PER_T) piece_put(tid + (i0 + ii) * C::kThreads, v[ii], 0);
            }
            return;
        }
        constexpr int BATCH = C::STAGE_BATCH;  // units in flight per thread (bounds the staging registers)
#pragma unroll
        for (int i0 = 0; i0 < C::UNITS_PER_T; i0 += BATCH) {
            u32x4 v[BATCH][8];
#pragma unroll
            for (int ii = 0; ii < BATCH; ++ii) issue(cb, i0 + ii, v[ii]);
#pragma unroll
            for (int ii = 0; ii < BATCH; ++ii) put(i0 + ii, v[ii], 0);
        }
    };

    // A fragment (step, m-tile) of this wave, steps s = c16 * 9 + tap; a
    // ring RING steps deep that runs on across staging passes.
    const u32x4* wbase = reinterpret_cast<const u32x4*>(a.w) +
                         (static_cast<size_t>(ocb) * nsteps16 * C::TAPS * C::MTT + mt0) * 64 + lane;
    auto frag = [&](int s, int mt) { return wbase[(static_cast<size_t>(s) * C::MTT + mt) * 64]; };
    const int total = nsteps16 * C::TAPS;

    stage(0);
    u32x4 ring[C::RING][C::MT];
#pragma unroll
    for (int s = 0; s < C::RING; ++s)
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt) ring[s][mt] = frag(s, mt);
    floatx16 acc[C::MT][C::NT];
#pragma unroll
    for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const floatx4 bv = *reinterpret_cast<const floatx4*>(a.bias + ocb * C::BM + (mt0 + mt) * 32 + 8 * j + hsel);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int nt = 0; nt < C::NT; ++nt) acc[mt][nt][4 * j + i] = bv[i];
        }
    // B fragment of pixel p at tap (ky, kx): staged row S*py + ky, staged
    // column px + kx + col_off (stride 1) or, for input column
    // c = 2*px + kx + col_off, entry c/2 of the half of c's parity (stride 2).
    int pbase[C::NT];
#pragma unroll
    for (int nt = 0; nt < C::NT; ++nt) {
        const int p = nt * 32 + (lane & 31);
        pbase[nt] = C::at(C::S * (p / C::TW), p % C::TW) + (lane >> 5) * 8;
    }
    int toff[C::KW];  // column part of the tap offset, per kx
#pragma unroll
    for (int kx = 0; kx < C::KW; ++kx) {
        const int c = kx + col_off;
        toff[kx] = (C::S == 1 ? c : (c & 1) * C::HALF + (c >> 1)) * C::PST;
    }
    __syncthreads();

    // One (16-channel step, tap) step of the K loop on the halo buffer at
    // LDS offset boff.
    // Pipelined passes: row loads of the next pass, NL per thread, issued
    // inside the K loop (see below).
    constexpr int NL = C::UNITS_PER_T * 8, NLN = C::NP_PER_T;
    u32x4 pv[C::UNITS_PER_T][8];
    std::uint32_t poff[C::UNITS_PER_T];
    int cb_next = 0;  // channel-last: first channel of the pass being loaded
    auto kstep = [&](int c16, int tap, int coff, int boff, bool pipe_issue) {
        const int s = c16 * C::TAPS + tap;
        const int ky = tap / C::KW, kx = tap % C::KW;
        half8 bv[C::NT];
#pragma unroll
        for (int nt = 0; nt < C::NT; ++nt)
            bv[nt] = *reinterpret_cast<const half8*>(&lds[boff + pbase[nt] + ky * C::ROW + toff[kx] + coff]);
        half8 av[C::MT];
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt) {
            av[mt] = __builtin_bit_cast(half8, ring[tap % C::RING][mt]);
            ring[tap % C::RING][mt] = frag(min(s + C::RING, total - 1), mt);
        }
        if (C::PIPE && pipe_issue) {
            if (a.in_nhwc) {
#pragma unroll
                for (int q = 0; q < NLN; ++q)
                    if (q * C::TAPS / NLN == tap) pv[q / 8][q % 8] = load_piece(piece_off(cb_next, tid + q * C::kThreads));
            } else {
#pragma unroll
                for (int q = 0; q < NL; ++q)
                    if (q * C::TAPS / NL == tap) pv[q / 8][q % 8] = load_row(poff[q / 8], q % 8);
            }
        }
        // The refill is issued here, before this tap's MFMAs, and
        // unconditionally (past the last step it re-reads that step):
        // the wait counter then stays at the ring depth. A conditional
        // refill made the compiler wait for every load where its
        // branch joined, and left alone it sinks the loads to their
        // use, either way exposing the L2 latency every few taps.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < C::NT; ++nt)
                acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[mt], bv[nt], acc[mt][nt], 0, 0, 0);
    };

    // ---- K loop: 16-channel step outer, tap inner, in passes of SC channels;
    // no barrier inside a pass.
    if constexpr (C::PIPE) {
        // The next pass's row loads are spread over the taps of this pass's
        // first 16-channel step, after each tap's ring refill: a wave stalls
        // at a load while the memory request queue is full, and issued in one
        // burst they would hold back the MFMAs behind them. They are written
        // to the other buffer after the pass's last step (no wave has read
        // that buffer since the previous pass's closing barrier).
        int buf = 0;
        for (int cb = 0; cb < nsteps16 * 16; cb += C::SC) {
            const bool next = cb + C::SC < nsteps16 * 16;  // only the last pass can be partial
            cb_next = cb + C::SC;
            if (next && !a.in_nhwc) {
#pragma unroll
                for (int i = 0; i < C::UNITS_PER_T; ++i) poff[i] = unit_off(cb + C::SC, i);
            }
#pragma unroll
            for (int j = 0; j < C::SC / 16; ++j) {
                const int c16 = cb / 16 + j;
                if (c16 < nsteps16) {
#pragma unroll
                    for (int tap = 0; tap < C::TAPS; ++tap) kstep(c16, tap, j * 16, buf * C::IN_LDS, j == 0 && next);
                }
                if (j == C::SC / 16 - 1 && next) {
                    if (a.in_nhwc) {
#pragma unroll
                        for (int q = 0; q < NLN; ++q) piece_put(tid + q * C::kThreads, pv[q / 8][q % 8], (buf ^ 1) * C::IN_LDS);
                    } else {
#pragma unroll
                        for (int i = 0; i < C::UNITS_PER_T; ++i) put(i, pv[i], (buf ^ 1) * C::IN_LDS);
                    }
                }
            }
            __syncthreads();
            buf ^= 1;
        }
    } else {
        for (int cb = 0; cb < nsteps16 * 16; cb += C::SC) {
            if (cb > 0) {
                __syncthreads();  // every wave is done with the previous pass's halo
                stage(cb);
                __syncthreads();
            }
            const int c16_end = min(nsteps16, (cb + C::SC) / 16);
            for (int c16 = cb / 16; c16 < c16_end; ++c16) {
#pragma unroll
                for (int tap = 0; tap < C::TAPS; ++tap) kstep(c16, tap, c16 * 16 - cb, 0, false);
            }
        }
    }

    // ---- epilogue (as conv_mfma_kernel): round, then the epilogue on the
    // rounded value. Lane l of accumulator (mt, nt) holds channels oc0 + i,
    // oc0 = ocb*BM + (mt0+mt)*32 + 8j + 4*(l/32), of tile pixel nt*32 + l%32.
    // Plain outputs go through an LDS [channel][pixel] tile and leave as
    // 16-byte rows; with DEPTH_TO_SPACE(2) the 4 channels of a lane are the
    // (dy, dx) block of output channel oc0/4, stored as two 4-byte pairs.
    const bool max_form = a.alpha >= 0.0f && a.alpha <= 1.0f;
    if constexpr (C::NHWC_D2S_EPI) {
        if (a.d2s == 2 && a.out_nhwc) {
            // Channel-last DEPTH_TO_SPACE(2): conv channel ocl is output
            // channel ocl / 4 of subpixel ocl % 4 = (dy, dx). The rounded,
            // epilogued halves go to a [subpixel][pixel][channel] tile, which
            // leaves as 16-byte pieces of 8 output channels of one output
            // pixel (the host allows no residual here).
            __syncthreads();  // every wave is done reading the halo
#pragma unroll
            for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < C::NT; ++nt)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int cl = ((mt0 + mt) * 32 + 8 * j + hsel) / 4, p = nt * 32 + (lane & 31);
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
                        }
                        const std::uint16_t h[4] = {static_cast<std::uint16_t>(h01), static_cast<std::uint16_t>(h01 >> 16),
                                                    static_cast<std::uint16_t>(h23), static_cast<std::uint16_t>(h23 >> 16)};
#pragma unroll
                        for (int r = 0; r < 4; ++r) lds[(r * C::BN + p) * C::EPI_ROW_D + cl] = h[r];
                    }
            __syncthreads();
            constexpr int G8 = C::BM / 32;  // 8-channel pieces per output pixel of this block
            const int occ = a.oc / 4, OW2 = a.ow * 2, OH2 = a.oh * 2;
            for (int u = tid; u < 4 * C::BN * G8; u += C::kThreads) {
                const int g = u % G8, rp = u / G8, r = rp / C::BN, p = rp % C::BN;
                const int oy = ty0 + p / C::TW, ox = tx0 + p % C::TW, c = ocb * (C::BM / 4) + 8 * g;
                if (c >= occ || oy >= a.oh || ox >= a.ow) continue;
                const u32x4 h = *reinterpret_cast<const u32x4*>(&lds[rp * C::EPI_ROW_D + 8 * g]);
                const int Y = 2 * oy + (r >> 1), X = 2 * ox + (r & 1);
                *reinterpret_cast<u32x4*>(a.y + ((static_cast<size_t>(b) * OH2 + Y) * OW2 + X) * occ + c) = h;
            }
            return;
        }
    }
    if (a.d2s == 2) {
        // Straight from the accumulators, no LDS and no barrier: each wave
        // writes as soon as its own K loop ends. Lanes 0-31 and 32-63 each
        // write 32 consecutive pixel pairs, 128 contiguous bytes per row.
        const int OW2 = a.ow * 2, OH2 = a.oh * 2, occ = a.oc / 4;
#pragma unroll
        for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
            for (int nt = 0; nt < C::NT; ++nt) {
                const int p = nt * 32 + (lane & 31), py = p / C::TW, px = p % C::TW;
                const int oy = ty0 + py, ox = tx0 + px;
                const bool inside = oy < a.oh && ox < a.ow;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int ocl = (mt0 + mt) * 32 + 8 * j + hsel, oc0 = ocb * C::BM + ocl;
                    const float v[4] = {acc[mt][nt][4 * j], acc[mt][nt][4 * j + 1], acc[mt][nt][4 * j + 2], acc[mt][nt][4 * j + 3]};
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
                    // Rows oc0 .. oc0+3 are the (dy, dx) block of output channel oc0 / 4.
                    const int c = oc0 / 4;
                    if (inside && c < occ) {
                        std::uint16_t* dst = a.y + (static_cast<size_t>(b * occ + c) * OH2 + 2 * oy) * OW2 + 2 * ox;
                        *reinterpret_cast<std::uint32_t*>(dst) = h01;
                        *reinterpret_cast<std::uint32_t*>(dst + OW2) = h23;
                    }
                }
            }
        return;
    }
    if constexpr (C::NHWC_EPI) {
        if (a.out_nhwc) {
            // [pixel][channel] tile: the lane's four consecutive channels of
            // one pixel per (m-tile, n-tile, j), then 16-byte pieces of 8
            // channels of one pixel out (the host allows no residual here).
            typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
            __syncthreads();  // every wave is done reading the halo
#pragma unroll
            for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
                for (int nt = 0; nt < C::NT; ++nt)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int ocl = (mt0 + mt) * 32 + 8 * j + hsel, p = nt * 32 + (lane & 31);
                        *reinterpret_cast<u32x2*>(&lds[p * C::EPI_ROW_N + ocl]) =
                            u32x2{pack_f16(acc[mt][nt][4 * j], acc[mt][nt][4 * j + 1]),
                                  pack_f16(acc[mt][nt][4 * j + 2], acc[mt][nt][4 * j + 3])};
                    }
            __syncthreads();
            constexpr int G8 = C::BM / 8;
            for (int u = tid; u < C::BN * G8; u += C::kThreads) {
                const int p = u / G8, oc = ocb * C::BM + 8 * (u % G8);
                const int oy = ty0 + p / C::TW, ox = tx0 + p % C::TW;
                if (oc >= a.oc || oy >= a.oh || ox >= a.ow) continue;
                u32x4 h = *reinterpret_cast<const u32x4*>(&lds[p * C::EPI_ROW_N + 8 * (u % G8)]);
                if (a.epi == MLVC_EPI_LEAKY_RELU) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) h[k] = leaky_h2(h[k], a.alpha, max_form);
                } else if (a.epi == MLVC_EPI_CLAMP) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) h[k] = clamp_h2(h[k], a.lo, a.hi);
                }
                *reinterpret_cast<u32x4*>(a.y + ((static_cast<size_t>(b) * a.oh + oy) * a.ow + ox) * a.oc + oc) = h;
            }
            return;
        }
    }
    __syncthreads();  // every wave is done reading the halo
#pragma unroll
    for (int mt = 0; mt < C::MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < C::NT; ++nt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int ocl = (mt0 + mt) * 32 + 8 * (r >> 2) + hsel + (r & 3);
                lds[ocl * C::EPI_ROW + nt * 32 + (lane & 31)] = f2h(acc[mt][nt][r]);
            }
    __syncthreads();
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
}

template <class C>
void launch_ws(const ConvArgs& a, dim3 grid, hipStream_t s)
{
    hipLaunchKernelGGL(conv_ws_kernel<C>, grid, dim3(C::kThreads), 0, s, a);
}

// Variant entry: weights packed with kc = 16 ([ocb][c16][tap][m-tile][lane][8]);
// eligible for plain NCHW inputs with 16-byte rows (the vector launch slot),
// staged SC channels per pass; no scalar or SPACE_TO_DEPTH staging.
#define MLVC_VARIANT_WS(BM, TH, TW, SC, OCC)                                                                   \
    Variant{"ws_bm" #BM "_" #TH "x" #TW "_k3x3_s1_sc" #SC "_occ" #OCC, BM, TH, TW, 3, 3, 1, 16, nullptr,          \
            &launch_ws<WsCfg<BM, TH, TW, SC, OCC>>, nullptr, SC, WsCfg<BM, TH, TW, SC, OCC>::NHWC_OUT}
// A ring RING k-steps deep (3 or 9): with one m-tile per wave, 9 steps of
// fragments cover the L2 latency that 3 do not.
#define MLVC_VARIANT_WSR(BM, TH, TW, SC, OCC, RING)                                                            \
    Variant{"ws_bm" #BM "_" #TH "x" #TW "_k3x3_s1_sc" #SC "_occ" #OCC "_r" #RING, BM, TH, TW, 3, 3, 1, 16, nullptr, \
            &launch_ws<WsCfg<BM, TH, TW, SC, OCC, 1, 4, RING>>, nullptr, SC, WsCfg<BM, TH, TW, SC, OCC, 1, 4, RING>::NHWC_OUT}
// Stride 2, WAVES waves splitting the BM output channels.
#define MLVC_VARIANT_WS2(BM, TH, TW, SC, OCC, WAVES)                                                           \
    Variant{"ws_bm" #BM "_" #TH "x" #TW "_k3x3_s2_sc" #SC "_occ" #OCC "_w" #WAVES, BM, TH, TW, 3, 3, 2, 16, nullptr, \
            &launch_ws<WsCfg<BM, TH, TW, SC, OCC, 2, WAVES>>, nullptr, SC, WsCfg<BM, TH, TW, SC, OCC, 2, WAVES>::NHWC_OUT}
// Pipelined passes (two halo buffers, next pass staged under the current one).
#define MLVC_VARIANT_WSP(BM, TH, TW, SC, OCC, RING)                                                            \
    Variant{"ws_bm" #BM "_" #TH "x" #TW "_k3x3_s1_sc" #SC "_occ" #OCC "_r" #RING "_pipe", BM, TH, TW, 3, 3, 1, 16,     \
            nullptr, &launch_ws<WsCfg<BM, TH, TW, SC, OCC, 1, 4, RING, true>>, nullptr, SC, WsCfg<BM, TH, TW, SC, OCC, 1, 4, RING, true>::NHWC_OUT}
// Stride 1 with WAVES waves (BM = 64 over two waves: 64-channel convs
// without padded output rows).
#define MLVC_VARIANT_WSW(BM, TH, TW, SC, OCC, WAVES, RING)                                                     \
    Variant{"ws_bm" #BM "_" #TH "x" #TW "_k3x3_s1_sc" #SC "_occ" #OCC "_w" #WAVES "_r" #RING, BM, TH, TW, 3, 3, 1, 16, \
            nullptr, &launch_ws<WsCfg<BM, TH, TW, SC, OCC, 1, WAVES, RING>>, nullptr, SC, WsCfg<BM, TH, TW, SC, OCC, 1, WAVES, RING>::NHWC_OUT}
// Stride 2 with a ring RING k-steps deep.
#define MLVC_VARIANT_WS2R(BM, TH, TW, SC, OCC, WAVES, RING)                                                    \
    Variant{"ws_bm" #BM "_" #TH "x" #TW "_k3x3_s2_sc" #SC "_occ" #OCC "_w" #WAVES "_r" #RING, BM, TH, TW, 3, 3, 2, 16, \
            nullptr, &launch_ws<WsCfg<BM, TH, TW, SC, OCC, 2, WAVES, RING>>, nullptr, SC, WsCfg<BM, TH, TW, SC, OCC, 2, WAVES, RING>::NHWC_OUT}
// Pipelined passes, with the LDS sized for the channel-last
// DEPTH_TO_SPACE(2) output tile.
#define MLVC_VARIANT_WSPD(BM, TH, TW, SC, OCC, RING)                                                           \
    Variant{"ws_bm" #BM "_" #TH "x" #TW "_k3x3_s1_sc" #SC "_occ" #OCC "_r" #RING "_pipe", BM, TH, TW, 3, 3, 1, 16,     \
            nullptr, &launch_ws<WsCfg<BM, TH, TW, SC, OCC, 1, 4, RING, true, true>>, nullptr, SC,                     \
            WsCfg<BM, TH, TW, SC, OCC, 1, 4, RING, true, true>::NHWC_OUT}
// Stride 2 with a ring RING k-steps deep and pipelined passes.
#define MLVC_VARIANT_WS2P(BM, TH, TW, SC, OCC, WAVES, RING)                                                    \
    Variant{"ws_bm" #BM "_" #TH "x" #TW "_k3x3_s2_sc" #SC "_occ" #OCC "_w" #WAVES "_r" #RING "_pipe", BM, TH, TW, 3, 3, 2, \
            16, nullptr, &launch_ws<WsCfg<BM, TH, TW, SC, OCC, 2, WAVES, RING, true>>, nullptr, SC,                     \
            WsCfg<BM, TH, TW, SC, OCC, 2, WAVES, RING, true>::NHWC_OUT}

}  // namespace conv
}  // namespace mlvc_hip
