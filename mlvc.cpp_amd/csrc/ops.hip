// Elementwise, layout and fused operators of the real MLVC graphs outside
// the conv path: CLIP / SIGMOID / RECIPROCAL / ROUND, ADD / SUB / MUL with
// broadcasting, SLICE, CONCAT pieces, GATHER, and the fused ReGLU,
// recurrent feature update and y0 / y1 quantisation tails.
//
// All tensors are NCHW FP16. Every materialised value is one FP32 operation
// on FP16-widened operands rounded once to FP16 (RNE), in the order of the
// reference CPU kernels (backends/cpu/src/kernels_scalar.cpp:80-110,
// 244-537 and kernels_x86_avx2.cpp:30-62, 304-712), so results are
// bit-identical to them. Three details keep it so:
//   * contraction is off in this file and `keep` pins each FP32 result in a
//     register before it is narrowed, so the compiler neither fuses a
//     multiply and an add nor folds an operation and its narrowing into one
//     v_fma_mix rounding;
//   * min / max are selects with the MINPS / MAXPS operand order (the
//     second operand wins on NaN), as the reference's vector lanes;
//   * SIGMOID uses the reference's vector-lane exponential (range reduction
//     by ln 2 in two parts, degree-6 Taylor polynomial by fused Horner
//     steps, exponent-bit scaling), kernels_x86_avx2.cpp:30-62.
//
// These kernels are HBM-bound: each thread moves 8 consecutive FP16 values
// of a plane (16-byte accesses when planes are multiples of 8 and buffers
// 16-byte aligned), and a grid-stride loop covers the planes.

#include "common.hpp"
#include "mlvc_hip_device.h"

#include <algorithm>
#include <mutex>

#pragma clang fp contract(off)

namespace mlvc_hip {
namespace {

using u16 = std::uint16_t;
constexpr int kBlock = 256;

unsigned grid_for(size_t work)
{
    return static_cast<unsigned>(std::max<size_t>(1, std::min<size_t>((work + kBlock - 1) / kBlock, 1u << 20)));
}

__device__ __forceinline__ float keep(float x)
{
    asm("" : "+v"(x));
    return x;
}
__device__ __forceinline__ u16 rnd(float x) { return f2h(keep(x)); }
__device__ __forceinline__ float r16(float x) { return h2f(f2h(keep(x))); }
__device__ __forceinline__ float minps(float a, float b) { return a < b ? a : b; }
__device__ __forceinline__ float maxps(float a, float b) { return a > b ? a : b; }

__device__ __forceinline__ float exp_lane(float x)
{
    x = minps(maxps(x, -87.33654475f), 88.72283905f);
    const float fx = __builtin_rintf(keep(x * 1.4426950408889634f));
    const float r = __builtin_fmaf(-fx, 1.428606765330187e-6f, __builtin_fmaf(-fx, 0.693145751953125f, x));
    float p = 0.0013888889f;
    p = __builtin_fmaf(p, r, 0.0083333338f);
    p = __builtin_fmaf(p, r, 0.0416666679f);
    p = __builtin_fmaf(p, r, 0.1666666716f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const unsigned bits = static_cast<unsigned>(static_cast<int>(fx) + 127) << 23;
    return keep(p * __builtin_bit_cast(float, bits));
}

__device__ __forceinline__ float sigmoid(float x) { return 1.0f / keep(1.0f + exp_lane(keep(0.0f - x))); }

// Eight consecutive FP16 values of a plane; n < 8 only at a plane's end.
template <bool VEC>
__device__ __forceinline__ void ld8(const u16* p, int n, u16 (&v)[8])
{
    if (VEC && n == 8) {
        const uint4 q = *reinterpret_cast<const uint4*>(p);
        __builtin_memcpy(v, &q, 16);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = j < n ? p[j] : u16{0};
    }
}
template <bool VEC>
__device__ __forceinline__ void st8(u16* p, int n, const u16 (&v)[8])
{
    if (VEC && n == 8) {
        uint4 q;
        __builtin_memcpy(&q, v, 16);
        *reinterpret_cast<uint4*>(p) = q;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (j < n) p[j] = v[j];
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0; }

// ------------------------------------------------------------------ unary
template <int OP>
__device__ __forceinline__ u16 unary_op(u16 h, float lo, float hi)
{
    const float x = h2f(h);
    if (OP == MLVC_UNARY_CLIP) return rnd(maxps(minps(x, hi), lo));
    if (OP == MLVC_UNARY_SIGMOID) return rnd(sigmoid(x));
    if (OP == MLVC_UNARY_RECIPROCAL) return rnd(1.0f / x);
    return rnd(__builtin_rintf(x));
}

template <int OP>
__global__ __launch_bounds__(kBlock) void unary_kernel(const u16* __restrict__ x, u16* __restrict__ y, size_t count, float lo,
                                                       float hi)
{
    const size_t groups = (count + 7) / 8;
    for (size_t i = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; i < groups; i += static_cast<size_t>(gridDim.x) * kBlock) {
        const int n = static_cast<int>(std::min<size_t>(8, count - i * 8));
        u16 v[8];
        ld8<true>(x + i * 8, n, v);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = unary_op<OP>(v[j], lo, hi);
        st8<true>(y + i * 8, n, v);
    }
}

// ----------------------------------------------------------------- binary
template <int OP>
__device__ __forceinline__ u16 binary_op(u16 a, u16 b)
{
    const float x = h2f(a), z = h2f(b);
    return rnd(OP == MLVC_BINARY_SUB ? x - z : OP == MLVC_BINARY_MUL ? x * z : x + z);
}

template <int OP>
__global__ __launch_bounds__(kBlock) void binary_same_kernel(const u16* __restrict__ a, const u16* __restrict__ b, u16* __restrict__ y,
                                                             size_t count)
{
    const size_t groups = (count + 7) / 8;
    for (size_t i = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; i < groups; i += static_cast<size_t>(gridDim.x) * kBlock) {
        const int n = static_cast<int>(std::min<size_t>(8, count - i * 8));
        u16 va[8], vb[8];
        ld8<true>(a + i * 8, n, va);
        ld8<true>(b + i * 8, n, vb);
#pragma unroll
        for (int j = 0; j < 8; ++j) va[j] = binary_op<OP>(va[j], vb[j]);
        st8<true>(y + i * 8, n, va);
    }
}

struct Dims4 {
    long long d[4];   // output dims
    long long sa[4];  // element strides of a (0 along broadcast dims)
    long long sb[4];
};

// One thread: 8 consecutive outputs of one output row (fixed n, c, h).
template <int OP>
__global__ __launch_bounds__(kBlock) void binary_bcast_kernel(const u16* __restrict__ a, const u16* __restrict__ b,
                                                              u16* __restrict__ y, Dims4 g)
{
    const long long w8 = (g.d[3] + 7) / 8, rows = g.d[0] * g.d[1] * g.d[2];
    for (long long i = blockIdx.x * static_cast<long long>(kBlock) + threadIdx.x; i < rows * w8;
         i += static_cast<long long>(gridDim.x) * kBlock) {
        const long long row = i / w8, w0 = (i % w8) * 8;
        const long long h = row % g.d[2], c = (row / g.d[2]) % g.d[1], n = row / (g.d[2] * g.d[1]);
        const u16* pa = a + n * g.sa[0] + c * g.sa[1] + h * g.sa[2];
        const u16* pb = b + n * g.sb[0] + c * g.sb[1] + h * g.sb[2];
        u16* py = y + row * g.d[3];
        const int cnt = static_cast<int>(std::min<long long>(8, g.d[3] - w0));
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (j < cnt) py[w0 + j] = binary_op<OP>(pa[(w0 + j) * g.sa[3]], pb[(w0 + j) * g.sb[3]]);
    }
}

// Vector form for rows whose W stride is 1 or 0 for both operands (full rows
// or a value broadcast along W) with W a multiple of 8: 16-byte loads of the
// full operands, one load of a broadcast value, 16-byte stores.
template <int OP, bool AV, bool BV>
__global__ __launch_bounds__(kBlock) void binary_rows_kernel(const u16* __restrict__ a, const u16* __restrict__ b,
                                                             u16* __restrict__ y, Dims4 g)
{
    const long long w8 = g.d[3] / 8, rows = g.d[0] * g.d[1] * g.d[2];
    for (long long i = blockIdx.x * static_cast<long long>(kBlock) + threadIdx.x; i < rows * w8;
         i += static_cast<long long>(gridDim.x) * kBlock) {
        const long long row = i / w8, w0 = (i % w8) * 8;
        const long long h = row % g.d[2], c = (row / g.d[2]) % g.d[1], n = row / (g.d[2] * g.d[1]);
        const u16* pa = a + n * g.sa[0] + c * g.sa[1] + h * g.sa[2];
        const u16* pb = b + n * g.sb[0] + c * g.sb[1] + h * g.sb[2];
        u16 va[8], vb[8];
        if (AV) {
            ld8<true>(pa + w0, 8, va);
        } else {
            const u16 s = *pa;
#pragma unroll
            for (int j = 0; j < 8; ++j) va[j] = s;
        }
        if (BV) {
            ld8<true>(pb + w0, 8, vb);
        } else {
            const u16 s = *pb;
#pragma unroll
            for (int j = 0; j < 8; ++j) vb[j] = s;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) va[j] = binary_op<OP>(va[j], vb[j]);
        st8<true>(y + row * g.d[3] + w0, 8, va);
    }
}

// ------------------------------------------------------------------ slice
struct SliceArgs {
    long long id[4], od[4], st[4], sp[4];
};

// Unit W step, W start / extents multiples of 8: whole 16-byte groups.
__global__ __launch_bounds__(kBlock) void slice_rows_kernel(const u16* __restrict__ x, u16* __restrict__ y, SliceArgs s)
{
    const long long w8 = s.od[3] / 8, rows = s.od[0] * s.od[1] * s.od[2];
    for (long long i = blockIdx.x * static_cast<long long>(kBlock) + threadIdx.x; i < rows * w8;
         i += static_cast<long long>(gridDim.x) * kBlock) {
        const long long row = i / w8, w0 = (i % w8) * 8;
        const long long h = row % s.od[2], c = (row / s.od[2]) % s.od[1], n = row / (s.od[2] * s.od[1]);
        const long long in_row = ((s.st[0] + n * s.sp[0]) * s.id[1] + s.st[1] + c * s.sp[1]) * s.id[2] + s.st[2] + h * s.sp[2];
        u16 v[8];
        ld8<true>(x + in_row * s.id[3] + s.st[3] + w0, 8, v);
        st8<true>(y + row * s.od[3] + w0, 8, v);
    }
}

__global__ __launch_bounds__(kBlock) void slice_kernel(const u16* __restrict__ x, u16* __restrict__ y, SliceArgs s)
{
    const long long w8 = (s.od[3] + 7) / 8, rows = s.od[0] * s.od[1] * s.od[2];
    for (long long i = blockIdx.x * static_cast<long long>(kBlock) + threadIdx.x; i < rows * w8;
         i += static_cast<long long>(gridDim.x) * kBlock) {
        const long long row = i / w8, w0 = (i % w8) * 8;
        const long long h = row % s.od[2], c = (row / s.od[2]) % s.od[1], n = row / (s.od[2] * s.od[1]);
        const long long in_row = ((s.st[0] + n * s.sp[0]) * s.id[1] + s.st[1] + c * s.sp[1]) * s.id[2] + s.st[2] + h * s.sp[2];
        const u16* px = x + in_row * s.id[3] + s.st[3];
        u16* py = y + row * s.od[3];
        const int cnt = static_cast<int>(std::min<long long>(8, s.od[3] - w0));
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (j < cnt) py[w0 + j] = px[(w0 + j) * s.sp[3]];
    }
}

// ------------------------------------------------------------- copy rows
// rows x row_elems block from x (row stride xs) into y (row stride ys).
template <bool VEC>
__global__ __launch_bounds__(kBlock) void copy_rows_kernel(const u16* __restrict__ x, u16* __restrict__ y, size_t rows,
                                                           size_t row_elems, size_t xs, size_t ys)
{
    const size_t e8 = (row_elems + 7) / 8;
    for (size_t i = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; i < rows * e8; i += static_cast<size_t>(gridDim.x) * kBlock) {
        const size_t r = i / e8, e0 = (i % e8) * 8;
        const int n = static_cast<int>(std::min<size_t>(8, row_elems - e0));
        u16 v[8];
        ld8<VEC>(x + r * xs + e0, n, v);
        st8<VEC>(y + r * ys + e0, n, v);
    }
}

// ----------------------------------------------------------------- gather
// y[o][i][r] = data[o][idx[i]][r]; negative indices count from the end and
// indices are clamped into the axis, so no access leaves the tensor (the
// host rejects out-of-range indices before launching).
template <typename I, bool VEC>
__global__ __launch_bounds__(kBlock) void gather_kernel(const u16* __restrict__ data, const I* __restrict__ idx, u16* __restrict__ y,
                                                        size_t outer, size_t dim, size_t count, size_t inner)
{
    const size_t r8 = (inner + 7) / 8;
    for (size_t t = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; t < outer * count * r8;
         t += static_cast<size_t>(gridDim.x) * kBlock) {
        const size_t r0 = (t % r8) * 8, oi = t / r8, i = oi % count, o = oi / count;
        long long v = static_cast<long long>(idx[i]);
        if (v < 0) v += static_cast<long long>(dim);
        v = std::min<long long>(std::max<long long>(v, 0), static_cast<long long>(dim) - 1);
        const int n = static_cast<int>(std::min<size_t>(8, inner - r0));
        u16 e[8];
        ld8<VEC>(data + (o * dim + static_cast<size_t>(v)) * inner + r0, n, e);
        st8<VEC>(y + oi * inner + r0, n, e);
    }
}

// ------------------------------------------------------------------ ReGLU
// x [N, 2G, HW] -> y [N, G, HW]: fp16(fp16(clamp(gate)) * linear).
template <bool VEC>
__global__ __launch_bounds__(kBlock) void reglu_kernel(const u16* __restrict__ x, u16* __restrict__ y, int n, int g, size_t hw,
                                                       float lo, float hi)
{
    const size_t p8 = (hw + 7) / 8, total = static_cast<size_t>(n) * g * p8;
    for (size_t t = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; t < total; t += static_cast<size_t>(gridDim.x) * kBlock) {
        const size_t p0 = (t % p8) * 8, plane = t / p8, c = plane % g, b = plane / g;
        const int cnt = static_cast<int>(std::min<size_t>(8, hw - p0));
        u16 gv[8], lv[8];
        ld8<VEC>(x + (b * 2 * g + c) * hw + p0, cnt, gv);
        ld8<VEC>(x + (b * 2 * g + g + c) * hw + p0, cnt, lv);
#pragma unroll
        for (int j = 0; j < 8; ++j) gv[j] = rnd(r16(maxps(minps(h2f(gv[j]), hi), lo)) * h2f(lv[j]));
        st8<VEC>(y + plane * hw + p0, cnt, gv);
    }
}

// ------------------------------------------------------- feature update
// x [N, 3C, HW] = a | b | c, history h [N, C, HW], scale [C]:
//   sb = fp16(sigmoid(b)), sc = fp16(sigmoid(c)),
//   blended = fp16(fp16(sb*h) + fp16(fp16(1 - sb) * a)),
//   scaled = fp16(fp16(sc * blended) * scale).
// feature [N, 2C, HW] = scaled | blended; scaled_out / blended_out [N, C, HW]
// are written when non-null.
//
// fp16(sigmoid(v)) of an FP16 gate v is a function of 16 bits: it is read
// from a table computed once per device by the same device code
// (sigmoid_lut_kernel), held in LDS, so the two gates per element cost a
// table read instead of a polynomial exponential and a division. The table
// covers v in [0, 16) (bits 0x0000-0x4BFF) and (-18, -0] (0x8000-0xCC7F);
// other gates (rare: |v| large, NaN) take the arithmetic path.
constexpr int kSigPos = 0x4C00, kSigNeg = 0x4C80, kSigLutN = kSigPos + kSigNeg;
__device__ __attribute__((aligned(16))) u16 g_sigmoid_lut[kSigLutN];

__global__ __launch_bounds__(kBlock) void sigmoid_lut_kernel()
{
    const int i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= kSigLutN) return;
    const u16 h = static_cast<u16>(i < kSigPos ? i : 0x8000 + (i - kSigPos));
    g_sigmoid_lut[i] = rnd(sigmoid(h2f(h)));
}

__device__ __forceinline__ float gate(const u16* lut, u16 h)
{
    const int idx = h < kSigPos ? h : (h >= 0x8000 && h < 0x8000 + kSigNeg ? kSigPos + (h - 0x8000) : -1);
    return idx >= 0 ? h2f(lut[idx]) : r16(sigmoid(h2f(h)));
}

constexpr int kFeatureBlock = 1024;

template <bool VEC>
__global__ __launch_bounds__(kFeatureBlock) void feature_kernel(const u16* __restrict__ x, const u16* __restrict__ hist,
                                                                const u16* __restrict__ scale, u16* __restrict__ feature,
                                                                u16* __restrict__ scaled_out, u16* __restrict__ blended_out, int n,
                                                                int ch, size_t hw)
{
    __shared__ __attribute__((aligned(16))) u16 lut[kSigLutN];
    for (int i = threadIdx.x; i < kSigLutN / 8; i += kFeatureBlock)
        reinterpret_cast<uint4*>(lut)[i] = reinterpret_cast<const uint4*>(g_sigmoid_lut)[i];
    __syncthreads();
    const size_t p8 = (hw + 7) / 8, total = static_cast<size_t>(n) * ch * p8;
    for (size_t t = blockIdx.x * static_cast<size_t>(kFeatureBlock) + threadIdx.x; t < total;
         t += static_cast<size_t>(gridDim.x) * kFeatureBlock) {
        const size_t p0 = (t % p8) * 8, plane = t / p8, c = plane % ch, b = plane / ch;
        const int cnt = static_cast<int>(std::min<size_t>(8, hw - p0));
        u16 va[8], vb[8], vc[8], vh[8], so[8], bo[8];
        ld8<VEC>(x + (b * 3 * ch + c) * hw + p0, cnt, va);
        ld8<VEC>(x + (b * 3 * ch + ch + c) * hw + p0, cnt, vb);
        ld8<VEC>(x + (b * 3 * ch + 2 * ch + c) * hw + p0, cnt, vc);
        ld8<VEC>(hist + plane * hw + p0, cnt, vh);
        const float s = h2f(scale[c]);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float sb = gate(lut, vb[j]);
            const float sc = gate(lut, vc[j]);
            const float wb = r16(sb * h2f(vh[j]));
            const float inv = r16(1.0f - sb);
            const float wa = r16(inv * h2f(va[j]));
            bo[j] = rnd(wb + wa);
            const float gated = r16(sc * h2f(bo[j]));
            so[j] = rnd(gated * s);
        }
        st8<VEC>(feature + (b * 2 * ch + c) * hw + p0, cnt, so);
        st8<VEC>(feature + (b * 2 * ch + ch + c) * hw + p0, cnt, bo);
        if (scaled_out) st8<VEC>(scaled_out + plane * hw + p0, cnt, so);
        if (blended_out) st8<VEC>(blended_out + plane * hw + p0, cnt, bo);
    }
}

// ------------------------------------------------------ quantisation tails
// Per pixel and q in [0, Q) with its pair q + Q (planes of [N, 2Q, HW]);
// prior [N, 4Q, HW] = head | tail:
//   clipped = fp16(max(head, clip_min)), normalized = fp16(latent * fp16(1/clipped)),
//   s = fp16(fp16(normalized - tail) * quant_scale),
//   y_raw[q] = fp16(rne(fp16(s[q] + s[q+Q]))),
//   upd = fp16(fp16(y_raw + tail) * update_scale{0,1}),
//   concat2 = upd, concat3 [N, 6Q, HW] = upd | prior.
template <bool VEC>
__global__ __launch_bounds__(kBlock) void y0_tail_kernel(mlvc_hip_y0_tail_desc d)
{
    const size_t hw = d.hw, q = static_cast<size_t>(d.q), p8 = (hw + 7) / 8, total = static_cast<size_t>(d.n) * q * p8;
    const auto* latent = static_cast<const u16*>(d.latent);
    const auto* prior = static_cast<const u16*>(d.prior);
    const auto* qs = static_cast<const u16*>(d.quant_scale);
    const u16* us[2] = {static_cast<const u16*>(d.update_scale0), static_cast<const u16*>(d.update_scale1)};
    auto* normalized = static_cast<u16*>(d.normalized);
    auto* clipped = static_cast<u16*>(d.clipped);
    auto* y_raw = static_cast<u16*>(d.y_raw);
    auto* concat2 = static_cast<u16*>(d.concat2);
    auto* concat3 = static_cast<u16*>(d.concat3);
    for (size_t t = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; t < total; t += static_cast<size_t>(gridDim.x) * kBlock) {
        const size_t p0 = (t % p8) * 8, qc = (t / p8) % q, b = t / p8 / q;
        const int cnt = static_cast<int>(std::min<size_t>(8, hw - p0));
        float sv[2][8], tl[2][8];
        u16 pv[4][8];  // prior planes qc, qc+Q (head) and 2Q+qc, 3Q+qc (tail)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const size_t cc = qc + h * q;
            u16 (&vh)[8] = pv[h];
            u16 (&vt)[8] = pv[2 + h];
            u16 vl[8], vq[8], cl[8], nr[8];
            ld8<VEC>(prior + (b * 4 * q + cc) * hw + p0, cnt, vh);
            ld8<VEC>(prior + (b * 4 * q + 2 * q + cc) * hw + p0, cnt, vt);
            ld8<VEC>(latent + (b * 2 * q + cc) * hw + p0, cnt, vl);
            ld8<VEC>(qs + (b * 2 * q + cc) * hw + p0, cnt, vq);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                cl[j] = rnd(maxps(h2f(vh[j]), d.clip_min));
                const float inv = r16(1.0f / h2f(cl[j]));
                nr[j] = rnd(h2f(vl[j]) * inv);
                tl[h][j] = h2f(vt[j]);
                const float diff = r16(h2f(nr[j]) - tl[h][j]);
                sv[h][j] = r16(diff * h2f(vq[j]));
            }
            st8<VEC>(normalized + (b * 2 * q + cc) * hw + p0, cnt, nr);
            st8<VEC>(clipped + (b * 2 * q + cc) * hw + p0, cnt, cl);
        }
        u16 raw[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) raw[j] = rnd(__builtin_rintf(r16(sv[0][j] + sv[1][j])));
        st8<VEC>(y_raw + (b * q + qc) * hw + p0, cnt, raw);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const size_t cc = qc + h * q;
            u16 vu[8], up[8];
            ld8<VEC>(us[h] + (b * q + qc) * hw + p0, cnt, vu);
#pragma unroll
            for (int j = 0; j < 8; ++j) up[j] = rnd(r16(h2f(raw[j]) + tl[h][j]) * h2f(vu[j]));
            st8<VEC>(concat2 + (b * 2 * q + cc) * hw + p0, cnt, up);
            st8<VEC>(concat3 + (b * 6 * q + cc) * hw + p0, cnt, up);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) st8<VEC>(concat3 + (b * 6 * q + 2 * q + qc + k * q) * hw + p0, cnt, pv[k]);
    }
}

//   s = fp16(fp16(normalized - prior) * quant_scale), y_raw as above,
//   upd = fp16(fp16(y_raw + prior) * update_scale{0,1}),
//   out = fp16(fp16(concat2 + upd) * clipped).
template <bool VEC>
__global__ __launch_bounds__(kBlock) void y1_tail_kernel(mlvc_hip_y1_tail_desc d)
{
    const size_t hw = d.hw, q = static_cast<size_t>(d.q), p8 = (hw + 7) / 8, total = static_cast<size_t>(d.n) * q * p8;
    const auto* normalized = static_cast<const u16*>(d.normalized);
    const auto* prior = static_cast<const u16*>(d.prior);
    const auto* qs = static_cast<const u16*>(d.quant_scale);
    const u16* us[2] = {static_cast<const u16*>(d.update_scale0), static_cast<const u16*>(d.update_scale1)};
    const auto* concat2 = static_cast<const u16*>(d.concat2);
    const auto* clipped = static_cast<const u16*>(d.clipped);
    auto* y_raw = static_cast<u16*>(d.y_raw);
    auto* out = static_cast<u16*>(d.out);
    for (size_t t = blockIdx.x * static_cast<size_t>(kBlock) + threadIdx.x; t < total; t += static_cast<size_t>(gridDim.x) * kBlock) {
        const size_t p0 = (t % p8) * 8, qc = (t / p8) % q, b = t / p8 / q;
        const int cnt = static_cast<int>(std::min<size_t>(8, hw - p0));
        float sv[2][8], pr[2][8];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const size_t off = (b * 2 * q + qc + h * q) * hw + p0;
            u16 vn[8], vp[8], vq[8];
            ld8<VEC>(normalized + off, cnt, vn);
            ld8<VEC>(prior + off, cnt, vp);
            ld8<VEC>(qs + off, cnt, vq);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                pr[h][j] = h2f(vp[j]);
                sv[h][j] = r16(r16(h2f(vn[j]) - pr[h][j]) * h2f(vq[j]));
            }
        }
        u16 raw[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) raw[j] = rnd(__builtin_rintf(r16(sv[0][j] + sv[1][j])));
        st8<VEC>(y_raw + (b * q + qc) * hw + p0, cnt, raw);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const size_t off = (b * 2 * q + qc + h * q) * hw + p0;
            u16 vu[8], v2[8], vc[8], o[8];
            ld8<VEC>(us[h] + (b * q + qc) * hw + p0, cnt, vu);
            ld8<VEC>(concat2 + off, cnt, v2);
            ld8<VEC>(clipped + off, cnt, vc);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float upd = r16(r16(h2f(raw[j]) + pr[h][j]) * h2f(vu[j]));
                const float add = r16(h2f(v2[j]) + upd);
                o[j] = rnd(add * h2f(vc[j]));
            }
            st8<VEC>(out + off, cnt, o);
        }
    }
}

void need(bool ok, const char* what)
{
    if (!ok) throw std::runtime_error(what);
}

template <typename K, typename... A>
void launch(K kernel, size_t work, hipStream_t s, A... args)
{
    hipLaunchKernelGGL(kernel, dim3(grid_for(work)), dim3(kBlock), 0, s, args...);
    check(hipGetLastError(), "kernel launch");
}

// Device tables (the gate table of the feature update), computed once per
// device on stream s and waited for. Not under graph capture: a caller that
// captures prepares them first (mlvc_hip_prepare_tables).
void prepare_tables(hipStream_t s)
{
    static std::mutex mu;
    static bool ready[64] = {};
    int dev = 0;
    check(hipGetDevice(&dev), "hipGetDevice");
    if (dev < 0 || dev >= 64) throw std::runtime_error("device tables: device index out of range");
    std::lock_guard<std::mutex> lock(mu);
    if (ready[dev]) return;
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    check(hipStreamIsCapturing(s, &status), "hipStreamIsCapturing");
    if (status != hipStreamCaptureStatusNone)
        throw std::runtime_error("device tables are not prepared: call mlvc_hip_prepare_tables before graph capture");
    hipLaunchKernelGGL(sigmoid_lut_kernel, dim3((kSigLutN + kBlock - 1) / kBlock), dim3(kBlock), 0, s);
    check(hipGetLastError(), "table kernel launch");
    check(hipStreamSynchronize(s), "table kernel");
    ready[dev] = true;
}

}  // namespace
}  // namespace mlvc_hip

using namespace mlvc_hip;

extern "C" {

int mlvc_hip_prepare_tables(mlvc_hip_stream s)
{
    return guard([&] { prepare_tables(to_stream(s)); });
}

int mlvc_hip_unary(const void* x, void* y, size_t count, int op, float lo, float hi, mlvc_hip_stream s)
{
    return guard([&] {
        need(x && y && aligned16(x) && aligned16(y), "unary: buffers must be non-null and 16-byte aligned");
        const auto* in = static_cast<const u16*>(x);
        auto* out = static_cast<u16*>(y);
        const size_t work = (count + 7) / 8;
        switch (op) {
        case MLVC_UNARY_CLIP: launch(unary_kernel<MLVC_UNARY_CLIP>, work, to_stream(s), in, out, count, lo, hi); break;
        case MLVC_UNARY_SIGMOID: launch(unary_kernel<MLVC_UNARY_SIGMOID>, work, to_stream(s), in, out, count, lo, hi); break;
        case MLVC_UNARY_RECIPROCAL: launch(unary_kernel<MLVC_UNARY_RECIPROCAL>, work, to_stream(s), in, out, count, lo, hi); break;
        case MLVC_UNARY_ROUND: launch(unary_kernel<MLVC_UNARY_ROUND>, work, to_stream(s), in, out, count, lo, hi); break;
        default: throw std::runtime_error("unary: unknown operator");
        }
    });
}

int mlvc_hip_binary(const void* a, const int64_t* a_dims, const void* b, const int64_t* b_dims, void* y, const int64_t* y_dims,
                    int op, mlvc_hip_stream s)
{
    return guard([&] {
        need(a && b && y && a_dims && b_dims && y_dims, "binary: null argument");
        need(op >= MLVC_BINARY_ADD && op <= MLVC_BINARY_MUL, "binary: unknown operator");
        Dims4 g{};
        bool same = true;
        long long sa = 1, sb = 1;
        for (int k = 3; k >= 0; --k) {
            need(y_dims[k] > 0 && (a_dims[k] == y_dims[k] || a_dims[k] == 1) && (b_dims[k] == y_dims[k] || b_dims[k] == 1),
                 "binary: operand dims do not broadcast to the output");
            g.d[k] = y_dims[k];
            g.sa[k] = a_dims[k] == 1 && y_dims[k] != 1 ? 0 : sa;
            g.sb[k] = b_dims[k] == 1 && y_dims[k] != 1 ? 0 : sb;
            sa *= a_dims[k];
            sb *= b_dims[k];
            same = same && a_dims[k] == y_dims[k] && b_dims[k] == y_dims[k];
        }
        const auto* pa = static_cast<const u16*>(a);
        const auto* pb = static_cast<const u16*>(b);
        auto* py = static_cast<u16*>(y);
        const hipStream_t st = to_stream(s);
        if (same && aligned16(a) && aligned16(b) && aligned16(y)) {
            const size_t count = static_cast<size_t>(g.d[0] * g.d[1] * g.d[2] * g.d[3]);
            if (op == MLVC_BINARY_ADD) launch(binary_same_kernel<MLVC_BINARY_ADD>, (count + 7) / 8, st, pa, pb, py, count);
            if (op == MLVC_BINARY_SUB) launch(binary_same_kernel<MLVC_BINARY_SUB>, (count + 7) / 8, st, pa, pb, py, count);
            if (op == MLVC_BINARY_MUL) launch(binary_same_kernel<MLVC_BINARY_MUL>, (count + 7) / 8, st, pa, pb, py, count);
            return;
        }
        const size_t work = static_cast<size_t>(g.d[0] * g.d[1] * g.d[2] * ((g.d[3] + 7) / 8));
        if (g.d[3] % 8 == 0 && g.sa[3] <= 1 && g.sb[3] <= 1 && aligned16(a) && aligned16(b) && aligned16(y)) {
            // Full operands have W stride 1 and row offsets that are multiples
            // of W, so every 8-group is 16-byte aligned.
            const int av = g.sa[3] == 1, bv = g.sb[3] == 1;
            const int key = op * 4 + av * 2 + bv;
#define MLVC_ROWS(O, A, B) \
    case O * 4 + A * 2 + B: launch(binary_rows_kernel<O, A, B>, work, st, pa, pb, py, g); return;
            switch (key) {
                MLVC_ROWS(0, 0, 0) MLVC_ROWS(0, 0, 1) MLVC_ROWS(0, 1, 0) MLVC_ROWS(0, 1, 1)
                MLVC_ROWS(1, 0, 0) MLVC_ROWS(1, 0, 1) MLVC_ROWS(1, 1, 0) MLVC_ROWS(1, 1, 1)
                MLVC_ROWS(2, 0, 0) MLVC_ROWS(2, 0, 1) MLVC_ROWS(2, 1, 0) MLVC_ROWS(2, 1, 1)
            default: break;
            }
#undef MLVC_ROWS
        }
        if (op == MLVC_BINARY_ADD) launch(binary_bcast_kernel<MLVC_BINARY_ADD>, work, st, pa, pb, py, g);
        if (op == MLVC_BINARY_SUB) launch(binary_bcast_kernel<MLVC_BINARY_SUB>, work, st, pa, pb, py, g);
        if (op == MLVC_BINARY_MUL) launch(binary_bcast_kernel<MLVC_BINARY_MUL>, work, st, pa, pb, py, g);
    });
}

int mlvc_hip_slice(const void* x, const int64_t* x_dims, void* y, const int64_t* y_dims, const int64_t* starts,
                   const int64_t* steps, mlvc_hip_stream s)
{
    return guard([&] {
        need(x && y && x_dims && y_dims && starts && steps, "slice: null argument");
        SliceArgs a{};
        for (int k = 0; k < 4; ++k) {
            need(x_dims[k] > 0 && y_dims[k] > 0 && steps[k] != 0, "slice: invalid geometry");
            const long long last = starts[k] + (y_dims[k] - 1) * steps[k];
            need(starts[k] >= 0 && starts[k] < x_dims[k] && last >= 0 && last < x_dims[k], "slice: reads outside its input");
            a.id[k] = x_dims[k];
            a.od[k] = y_dims[k];
            a.st[k] = starts[k];
            a.sp[k] = steps[k];
        }
        const size_t work = static_cast<size_t>(a.od[0] * a.od[1] * a.od[2] * ((a.od[3] + 7) / 8));
        const bool rows = a.sp[3] == 1 && a.st[3] % 8 == 0 && a.id[3] % 8 == 0 && a.od[3] % 8 == 0 && aligned16(x) && aligned16(y);
        if (rows) launch(slice_rows_kernel, work, to_stream(s), static_cast<const u16*>(x), static_cast<u16*>(y), a);
        else launch(slice_kernel, work, to_stream(s), static_cast<const u16*>(x), static_cast<u16*>(y), a);
    });
}

int mlvc_hip_copy_rows(const void* x, void* y, size_t rows, size_t row_elems, size_t x_stride, size_t y_stride, mlvc_hip_stream s)
{
    return guard([&] {
        need(x && y && row_elems <= x_stride && row_elems <= y_stride, "copy_rows: invalid geometry");
        const bool vec = aligned16(x) && aligned16(y) && row_elems % 8 == 0 && x_stride % 8 == 0 && y_stride % 8 == 0;
        const size_t work = rows * ((row_elems + 7) / 8);
        const auto* px = static_cast<const u16*>(x);
        auto* py = static_cast<u16*>(y);
        if (vec) launch(copy_rows_kernel<true>, work, to_stream(s), px, py, rows, row_elems, x_stride, y_stride);
        else launch(copy_rows_kernel<false>, work, to_stream(s), px, py, rows, row_elems, x_stride, y_stride);
    });
}

int mlvc_hip_gather(const void* data, const void* indices, int indices_int64, size_t count, size_t outer, size_t axis_dim,
                    size_t inner, void* y, mlvc_hip_stream s)
{
    return guard([&] {
        need(data && indices && y && axis_dim > 0 && count > 0, "gather: invalid arguments");
        const bool vec = aligned16(data) && aligned16(y) && inner % 8 == 0;
        const size_t work = outer * count * ((inner + 7) / 8);
        const auto* pd = static_cast<const u16*>(data);
        auto* py = static_cast<u16*>(y);
        const hipStream_t st = to_stream(s);
        if (indices_int64) {
            const auto* pi = static_cast<const long long*>(indices);
            if (vec) launch(gather_kernel<long long, true>, work, st, pd, pi, py, outer, axis_dim, count, inner);
            else launch(gather_kernel<long long, false>, work, st, pd, pi, py, outer, axis_dim, count, inner);
        } else {
            const auto* pi = static_cast<const int*>(indices);
            if (vec) launch(gather_kernel<int, true>, work, st, pd, pi, py, outer, axis_dim, count, inner);
            else launch(gather_kernel<int, false>, work, st, pd, pi, py, outer, axis_dim, count, inner);
        }
    });
}

int mlvc_hip_reglu(const void* x, void* y, int n, int gate_channels, size_t hw, float lo, float hi, mlvc_hip_stream s)
{
    return guard([&] {
        need(x && y && n > 0 && gate_channels > 0 && hw > 0, "reglu: invalid arguments");
        const bool vec = aligned16(x) && aligned16(y) && hw % 8 == 0;
        const size_t work = static_cast<size_t>(n) * gate_channels * ((hw + 7) / 8);
        const auto* px = static_cast<const u16*>(x);
        auto* py = static_cast<u16*>(y);
        if (vec) launch(reglu_kernel<true>, work, to_stream(s), px, py, n, gate_channels, hw, lo, hi);
        else launch(reglu_kernel<false>, work, to_stream(s), px, py, n, gate_channels, hw, lo, hi);
    });
}

int mlvc_hip_feature_update(const void* x, const void* history, const void* scale, void* feature, void* scaled, void* blended, int n,
                            int channels, size_t hw, mlvc_hip_stream s)
{
    return guard([&] {
        need(x && history && scale && feature && n > 0 && channels > 0 && hw > 0, "feature_update: invalid arguments");
        need((scaled == nullptr) == (blended == nullptr), "feature_update: scaled and blended outputs go together");
        bool vec = aligned16(x) && aligned16(history) && aligned16(feature) && hw % 8 == 0;
        if (scaled) vec = vec && aligned16(scaled) && aligned16(blended);
        const size_t work = static_cast<size_t>(n) * channels * ((hw + 7) / 8);
        const auto* px = static_cast<const u16*>(x);
        const auto* ph = static_cast<const u16*>(history);
        const auto* pc = static_cast<const u16*>(scale);
        auto* pf = static_cast<u16*>(feature);
        auto* ps = static_cast<u16*>(scaled);
        auto* pb = static_cast<u16*>(blended);
        prepare_tables(to_stream(s));
        // Every block copies the gate table into LDS first: a grid of the
        // blocks the device holds at once (two per CU) walks the work.
        const unsigned grid = static_cast<unsigned>(
            std::max<size_t>(1, std::min<size_t>((work + kFeatureBlock - 1) / kFeatureBlock, 2 * static_cast<size_t>(conv::cu_count()))));
        if (vec)
            hipLaunchKernelGGL(feature_kernel<true>, dim3(grid), dim3(kFeatureBlock), 0, to_stream(s), px, ph, pc, pf, ps, pb, n,
                               channels, hw);
        else
            hipLaunchKernelGGL(feature_kernel<false>, dim3(grid), dim3(kFeatureBlock), 0, to_stream(s), px, ph, pc, pf, ps, pb, n,
                               channels, hw);
        check(hipGetLastError(), "feature_update launch");
    });
}

int mlvc_hip_y0_tail(const mlvc_hip_y0_tail_desc* d, mlvc_hip_stream s)
{
    return guard([&] {
        need(d && d->latent && d->prior && d->quant_scale && d->update_scale0 && d->update_scale1 && d->normalized && d->clipped &&
                 d->y_raw && d->concat2 && d->concat3 && d->n > 0 && d->q > 0 && d->hw > 0,
             "y0_tail: invalid descriptor");
        const void* ptrs[] = {d->latent, d->prior, d->quant_scale, d->update_scale0, d->update_scale1, d->normalized, d->clipped,
                              d->y_raw, d->concat2, d->concat3};
        bool vec = d->hw % 8 == 0;
        for (const void* p : ptrs) vec = vec && aligned16(p);
        const size_t work = static_cast<size_t>(d->n) * d->q * ((d->hw + 7) / 8);
        if (vec) launch(y0_tail_kernel<true>, work, to_stream(s), *d);
        else launch(y0_tail_kernel<false>, work, to_stream(s), *d);
    });
}

int mlvc_hip_y1_tail(const mlvc_hip_y1_tail_desc* d, mlvc_hip_stream s)
{
    return guard([&] {
        need(d && d->normalized && d->prior && d->quant_scale && d->update_scale0 && d->update_scale1 && d->concat2 && d->clipped &&
                 d->y_raw && d->out && d->n > 0 && d->q > 0 && d->hw > 0,
             "y1_tail: invalid descriptor");
        const void* ptrs[] = {d->normalized, d->prior, d->quant_scale, d->update_scale0, d->update_scale1, d->concat2, d->clipped,
                              d->y_raw, d->out};
        bool vec = d->hw % 8 == 0;
        for (const void* p : ptrs) vec = vec && aligned16(p);
        const size_t work = static_cast<size_t>(d->n) * d->q * ((d->hw + 7) / 8);
        if (vec) launch(y1_tail_kernel<true>, work, to_stream(s), *d);
        else launch(y1_tail_kernel<false>, work, to_stream(s), *d);
    });
}

}  // extern "C"
