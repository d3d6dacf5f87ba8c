// FP16 convolution (groups == 1): variant table, planning, weight packing
// and launch behind the device C ABI. The MFMA kernel template is in
// conv_kernel.hpp and its tile variants are instantiated per kernel size in
// conv_k3s1.hip, conv_k3s2.hip and conv_k1.hip.

#include "conv_kernel.hpp"

#include <algorithm>
#include <map>
#include <mutex>
#include <vector>

namespace mlvc_hip {
namespace conv {

// Host-side tables of the per-size files (count returned through n).
const Variant* variants_k3s1(int* n);
const Variant* variants_k3s2(int* n);
const Variant* variants_k1(int* n);

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

// Split K, second kernel: out = epilogue(fp16(part[0] + part[1] + ...)) for
// every output of the conv geometry, the partials added in split order
// (FP32, nearest even), stored plainly or through DEPTH_TO_SPACE. Four
// consecutive outputs per thread when the plane is a multiple of 4.
__device__ __forceinline__ float splitk_sum(const ConvArgs& a, size_t stride, size_t e)
{
    float v = a.part[e];
    for (int sp = 1; sp < a.ksplit; ++sp) v = v + a.part[sp * stride + e];
    return v;
}

__global__ __launch_bounds__(256) void conv_splitk_reduce_kernel(ConvArgs a, int n)
{
    if (a.epi == MLVC_EPI_REGLU) {
        // Output channel g of the G-channel ReGLU output pairs the rounded
        // sums of rows 64 (g / 32) + g % 32 (gate) and that + 32 (linear).
        const size_t ohw = static_cast<size_t>(a.oh) * a.ow, stride = static_cast<size_t>(n) * a.oc * ohw;
        const int half = a.oc / 2;
        const size_t total = static_cast<size_t>(n) * half * ohw;
        for (size_t e = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; e < total;
             e += static_cast<size_t>(gridDim.x) * blockDim.x) {
            const size_t p = e % ohw;
            const int g = static_cast<int>((e / ohw) % half), b = static_cast<int>(e / (ohw * half));
            const int rg = (g / 32) * 64 + g % 32;
            const size_t base = static_cast<size_t>(b) * a.oc * ohw + p;
            const float vg = splitk_sum(a, stride, base + static_cast<size_t>(rg) * ohw);
            const float vl = splitk_sum(a, stride, base + static_cast<size_t>(rg + 32) * ohw);
            a.y[e] = reglu_h(f2h(vg), f2h(vl), a.lo, a.hi);
        }
        return;
    }
    const size_t ohw = static_cast<size_t>(a.oh) * a.ow;
    const size_t total = static_cast<size_t>(n) * a.oc * ohw, stride = total;
    const bool quad = ohw % 4 == 0;
    const size_t units = quad ? total / 4 : total;
    for (size_t u = blockIdx.x * static_cast<size_t>(blockDim.x) + threadIdx.x; u < units;
         u += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const size_t e0 = quad ? 4 * u : u;
        float v[4];
        if (quad) {
            const floatx4 p0 = *reinterpret_cast<const floatx4*>(a.part + e0);
            v[0] = p0[0]; v[1] = p0[1]; v[2] = p0[2]; v[3] = p0[3];
            for (int sp = 1; sp < a.ksplit; ++sp) {
                const floatx4 p = *reinterpret_cast<const floatx4*>(a.part + sp * stride + e0);
                v[0] = v[0] + p[0];
                v[1] = v[1] + p[1];
                v[2] = v[2] + p[2];
                v[3] = v[3] + p[3];
            }
        } else {
            v[0] = a.part[e0];
            for (int sp = 1; sp < a.ksplit; ++sp) v[0] = v[0] + a.part[sp * stride + e0];
        }
        for (int i = 0; i < (quad ? 4 : 1); ++i) {
            const size_t e = e0 + i;
            const int ox = static_cast<int>(e % a.ow), oy = static_cast<int>((e / a.ow) % a.oh);
            const int oc = static_cast<int>((e / ohw) % a.oc), b = static_cast<int>(e / (ohw * a.oc));
            store_output(a, finish(a, v[i], b, oc, oy, ox), b, oc, oy, ox);
        }
    }
}

// ---------------------------------------------------------------- variants

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

}  // namespace conv

namespace {

using namespace conv;

// Variant 0 is the direct fallback, then the MFMA tile variants.
const std::vector<Variant>& variants()
{
    static const std::vector<Variant> table = [] {
        std::vector<Variant> t{Variant{"direct_fp32", 0, 0, 0, 0, 0, 0, 0, nullptr, nullptr, nullptr}};
        for (auto family : {variants_k3s1, variants_k3s2, variants_k1}) {
            int n = 0;
            const Variant* v = family(&n);
            t.insert(t.end(), v, v + n);
        }
        return t;
    }();
    return table;
}

int variant_count() { return static_cast<int>(variants().size()); }

bool flat_1x1(const mlvc_hip_conv_desc& d)
{
    return d.kh == 1 && d.kw == 1 && d.in_s2d_block <= 1 && d.out_d2s_block <= 1;
}

const Variant& variant_of(const mlvc_hip_conv_desc& d)
{
    if (d.variant < 0 || d.variant >= variant_count()) throw std::runtime_error("conv: invalid variant");
    return variants()[d.variant];
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
    if (d.epilogue == MLVC_EPI_REGLU && (d.oc % 64 != 0 || d.out_d2s_block > 1))
        throw std::runtime_error("conv: ReGLU epilogue needs 64-channel gate/linear blocks and no depth_to_space");
    if ((d.in_nhwc != 0 && d.in_nhwc != 1) || (d.out_nhwc != 0 && d.out_nhwc != 1))
        throw std::runtime_error("conv: in_nhwc / out_nhwc must be 0 or 1");
    if (d.in_nhwc && (d.x2 || d.in_s2d_block > 1 || d.ic % 8 != 0))
        throw std::runtime_error("conv: a channel-last input needs 8-channel groups and no concat or space_to_depth fusion");
    if (d.out_nhwc && (d.out_d2s_block > 2 || d.oc % (d.out_d2s_block == 2 ? 32 : 8) != 0 ||
                       !(d.epilogue == MLVC_EPI_NONE || d.epilogue == MLVC_EPI_LEAKY_RELU || d.epilogue == MLVC_EPI_CLAMP)))
        throw std::runtime_error("conv: a channel-last output needs 8-channel groups (after depth_to_space(2), if "
                                 "fused) and a LeakyReLU, clamp or no epilogue");
    if (!pointers) return;
    if (d.out_nhwc && (reinterpret_cast<std::uintptr_t>(d.y) & 15u)) throw std::runtime_error("conv: channel-last y must be 16-byte aligned");
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

// Split K of a geometry (see mlvc_hip_conv_plan in the header): a fixed
// function of the geometry, so the summation order never depends on the
// tile variant or on tuning.
void split_rule(const mlvc_hip_conv_desc& d, int& ksplit, int& split_c)
{
    ksplit = 1;
    split_c = d.ic;
    if (d.kh != 1 || d.kw != 1 || d.ic < 576) return;
    const long long items =
        static_cast<long long>(d.n) * ((d.oc + 127) / 128) * ((static_cast<long long>(d.oh) * d.ow + 127) / 128);
    const long long s = std::min<long long>({8, 512 / items, d.ic / 64});
    if (s <= 1) return;
    const int c = static_cast<int>(64 * ((d.ic + 64 * s - 1) / (64 * s)));
    const int k = (d.ic + c - 1) / c;
    if (k > 1) {
        ksplit = k;
        split_c = c;
    }
}

bool eligible(const mlvc_hip_conv_desc& d, const Variant& k)
{
    if (k.bm == 0 || k.kh != d.kh || k.kw != d.kw || k.s != d.stride_h || k.s != d.stride_w) return false;
    // Channel-last operands: the weight-streaming kernel (an output only
    // where its [pixel][channel] tile fits the LDS).
    if ((d.in_nhwc || d.out_nhwc) && !k.ws_ic) return false;
    if (d.out_nhwc && !(k.nhwc_out & (d.out_d2s_block == 2 ? 2 : 1))) return false;
    // Split K: conv_mfma variants whose chunk divides the split.
    if (d.ksplit > 1 && (k.ws_ic || d.split_c % k.kc != 0)) return false;
    // ReGLU pairs gate and linear rows inside 64-row blocks of one tile.
    if (d.epilogue == MLVC_EPI_REGLU && k.bm % 64 != 0) return false;
    if (d.kh == 1 && (d.pad_h || d.pad_w)) return false;
    // The weight-streaming kernel: plain NCHW input staged as 16-byte rows,
    // no ReGLU, DEPTH_TO_SPACE(2) or none, 8-aligned output rows.
    if (k.ws_ic && (d.x2 || d.in_s2d_block > 1 || d.epilogue == MLVC_EPI_REGLU || d.out_d2s_block > 2 ||
                    d.iw % 8 != 0 || d.ow % 8 != 0))
        return false;
    int ih, iw, oh, ow;
    kernel_geometry(d, ih, iw, oh, ow);
    // ...and its 16-byte row staging keeps buffer offsets (up to KC channel
    // planes past the last one) below 2^31, as the launch requires.
    if (k.ws_ic && (static_cast<std::uint64_t>(d.ic) + k.kc) * static_cast<std::uint64_t>(ih) * iw * 2 >= (1ull << 31))
        return false;
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
        split_rule(*desc, desc->ksplit, desc->split_c);
        const mlvc_hip_conv_desc& d = *desc;
        int ih, iw, oh, ow;
        kernel_geometry(d, ih, iw, oh, ow);
        const int slots = 2 * cu_count();
        int best = 0;
        double best_cost = 0.0;
        for (int v = 1; v < variant_count(); ++v) {
            if (!eligible(d, variants()[v])) continue;
            const Variant& k = variants()[v];
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
        if (best == 0) {  // the direct fallback sums every channel itself
            desc->ksplit = 1;
            desc->split_c = d.ic;
        }
        // 16-byte row-segment staging: plain or channel-concat input whose
        // split falls on 8 channels, rows of 8-aligned width.
        desc->vector_io = best != 0 && d.in_s2d_block <= 1 && (!d.x2 || d.ic_split % 8 == 0) && iw % 8 == 0;
    });
}

size_t mlvc_hip_conv_workspace_bytes(const mlvc_hip_conv_desc* desc)
{
    if (!desc || desc->ksplit <= 1) return 0;
    return static_cast<size_t>(desc->ksplit) * desc->n * desc->oc * desc->oh * desc->ow * sizeof(float);
}

int mlvc_hip_conv_candidates(const mlvc_hip_conv_desc* desc, int* out, int capacity, int* count)
{
    return guard([&] {
        validate(*desc, false);
        if (!count || (capacity > 0 && !out)) throw std::runtime_error("conv: null candidate buffer");
        int n = 0;
        for (int v = 1; v < variant_count(); ++v)
            if (eligible(*desc, variants()[v])) {
                if (n < capacity) out[n] = v;
                ++n;
            }
        *count = n;
    });
}

const char* mlvc_hip_conv_variant_name(int variant)
{
    return variant >= 0 && variant < variant_count() ? variants()[variant].name : "invalid";
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

}  // extern "C"

namespace mlvc_hip {
namespace {

// The launch behind mlvc_hip_conv_launch and mlvc_hip_conv_launch_noalloc.
void launch_conv(const mlvc_hip_conv_desc& d, void* s)
{
    {
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
        a.lo = d.clip_lo;
        a.hi = d.clip_hi;
        a.ksplit = 1;
        a.split_c = d.ic;
        a.in_nhwc = d.in_nhwc;
        a.out_nhwc = d.out_nhwc;
        if ((d.in_nhwc || d.out_nhwc) && (!k.ws_ic || (d.out_nhwc && !(k.nhwc_out & (d.out_d2s_block == 2 ? 2 : 1))) ||
                                          d.ksplit > 1))
            throw std::runtime_error("conv: channel-last operands need a weight-streaming variant");
        if (d.ksplit > 1) {
            if (k.bm == 0 || k.ws_ic || d.split_c <= 0 || d.split_c % k.kc != 0 ||
                static_cast<long long>(d.split_c) * (d.ksplit - 1) >= d.ic || static_cast<long long>(d.split_c) * d.ksplit < d.ic)
                throw std::runtime_error("conv: split K needs a conv_mfma variant whose chunk divides the split");
            if (!d.workspace || d.workspace_bytes < mlvc_hip_conv_workspace_bytes(&d) ||
                (reinterpret_cast<std::uintptr_t>(d.workspace) & 15u))
                throw std::runtime_error("conv: split K needs a 16-byte aligned workspace of mlvc_hip_conv_workspace_bytes");
            a.ksplit = d.ksplit;
            a.split_c = d.split_c;
            a.part = static_cast<float*>(d.workspace);
        }
        if (k.bm == 0) {
            if (d.epilogue == MLVC_EPI_REGLU) throw std::runtime_error("conv: no tile variant runs this ReGLU conv");
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
            if (nwg * a.ksplit > 0x7FFFFFFF) throw std::runtime_error("conv: grid too large");
            a.nwg = static_cast<int>(nwg);
            const dim3 grid(static_cast<unsigned>(a.nwg * a.ksplit));
            // SPACE_TO_DEPTH(2) vector staging: 32-byte aligned source rows
            // and offsets (up to KC/4 channel planes past the end) < 2^31.
            const std::uint64_t src_plane = static_cast<std::uint64_t>(a.ih) * a.iw * 4 * 2;
            const bool s2d_vec = k.launch_s2d && a.s2d == 2 && (reinterpret_cast<std::uintptr_t>(d.x) & 15u) == 0 &&
                                 a.iw % 8 == 0 && (static_cast<std::uint64_t>(d.ic / 4) + k.kc / 4 + 1) * src_plane < (1ull << 31);
            if (k.ws_ic && !vec) throw std::runtime_error("conv: variant needs 16-byte row staging");
            (s2d_vec ? k.launch_s2d : vec ? k.launch_vec : k.launch_scalar)(a, grid, to_stream(s));
            if (a.ksplit > 1) {
                ConvArgs r = a;  // the reduce works in the real output geometry
                r.ih = d.ih;
                r.iw = d.iw;
                r.oh = d.oh;
                r.ow = d.ow;
                const size_t ohw = static_cast<size_t>(d.oh) * d.ow;
                const size_t units = d.epilogue == MLVC_EPI_REGLU ? static_cast<size_t>(d.n) * (d.oc / 2) * ohw
                                                                  : static_cast<size_t>(d.n) * d.oc * (ohw % 4 == 0 ? ohw / 4 : ohw);
                const unsigned blocks = static_cast<unsigned>(std::min<size_t>((units + 255) / 256, 8192));
                hipLaunchKernelGGL(conv_splitk_reduce_kernel, dim3(blocks), dim3(256), 0, to_stream(s), r, d.n);
            }
        }
        check(hipGetLastError(), "conv kernel launch");
    }
}

// Scratch of the no-allocation launch: the FP32 partials of a split-K conv.
// Every split the planner chooses fits: ksplit * items <= 512 and an item
// covers at most 128 x 128 outputs, so the partials take at most
// 512 * 128 * 128 * 4 bytes.
constexpr size_t kScratchBytes = size_t{512} * 128 * 128 * sizeof(float);

}  // namespace
}  // namespace mlvc_hip

// One copy per device, held until the process ends.
static __device__ __align__(256) float scratch[mlvc_hip::kScratchBytes / sizeof(float)];

namespace mlvc_hip {
namespace {

// Device address of `scratch` on the current device, looked up on the first
// call per device (the array's name is a host-side stand-in that must not
// reach a kernel).
void* scratch_ptr()
{
    int dev = 0;
    check(hipGetDevice(&dev), "current device");
    static std::mutex mutex;
    static std::map<int, void*> ptrs;
    std::lock_guard<std::mutex> lock(mutex);
    if (const auto it = ptrs.find(dev); it != ptrs.end()) return it->second;
    void* p = nullptr;
    check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "no-allocation scratch address");
    if (!p) throw std::runtime_error("conv: no-allocation scratch has no device address");
    ptrs.emplace(dev, p);
    return p;
}

}  // namespace
}  // namespace mlvc_hip

extern "C" {

int mlvc_hip_conv_launch(const mlvc_hip_conv_desc* desc, mlvc_hip_stream s)
{
    return guard([&] {
        if (!desc) throw std::runtime_error("conv: null descriptor");
        launch_conv(*desc, s);
    });
}

int mlvc_hip_conv_launch_noalloc(const mlvc_hip_conv_desc* desc, mlvc_hip_stream s)
{
    return guard([&] {
        if (!desc) throw std::runtime_error("conv: null descriptor");
        mlvc_hip_conv_desc d = *desc;
        d.workspace = nullptr;
        d.workspace_bytes = 0;
        if (d.ksplit > 1) {
            const size_t need = mlvc_hip_conv_workspace_bytes(&d);
            if (need > kScratchBytes)
                throw std::runtime_error("conv: split K needs " + std::to_string(need) +
                                         " bytes of partials; the no-allocation launch holds " +
                                         std::to_string(kScratchBytes));
            d.workspace = scratch_ptr();
            d.workspace_bytes = kScratchBytes;
        }
        launch_conv(d, s);
    });
}

}  // extern "C"
