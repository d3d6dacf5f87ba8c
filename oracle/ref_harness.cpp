// Calls the reference CPU kernels — TEST INFRASTRUCTURE ONLY.
//
// Built by oracle/build_ref.sh together with the reference's own sources
// backends/cpu/src/{kernels_scalar,kernels_x86_avx2,thread_pool,cpu_features}.cpp
// and core/src/yuv.cpp (compiled where they lie under the reference checkout)
// into
// oracle/_ref/libmlvc_ref_kernels.so. It exposes the kernel-level entry
// points of oracle.h under a ref_ prefix so tests can compare the oracle's
// restatement with the reference kernels on identical inputs. The graph-level
// reference plan (execution_plan.cpp) is not built: it needs
// runtime/src/aot_graph.cpp, which includes protoc-generated headers that do
// not exist in this environment.

#include "kernels_common.hpp"
#include "mlvc/core/half.hpp"
#include "mlvc/core/yuv.hpp"

#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

using namespace mlvc;
using namespace mlvc::cpu_backend;

namespace {

thread_local std::string g_error;

const KernelSet& kernels(int isa)
{
    return isa == 0 ? get_x86_avx2_kernels() : get_scalar_kernels();
}

CpuThreadPool& pool(int threads)
{
    static std::map<int, std::unique_ptr<CpuThreadPool>> pools;
    static std::mutex mu;
    std::lock_guard<std::mutex> l(mu);
    auto& p = pools[threads];
    if (!p) p = std::make_unique<CpuThreadPool>(threads);
    return *p;
}

GemmEpilogue epilogue(int epi, float alpha, float cmin, float cmax, const std::uint16_t* residual)
{
    GemmEpilogue e;
    e.kind = epi == 1 ? GemmEpilogueKind::kClamp
           : epi == 2 ? GemmEpilogueKind::kLeakyRelu
           : epi == 3 ? GemmEpilogueKind::kResidualAdd
                      : GemmEpilogueKind::kNone;
    e.alpha = alpha;
    e.clamp_min = cmin;
    e.clamp_max = cmax;
    e.residual = residual;
    return e;
}

template <typename F>
int guard(F&& f)
{
    try {
        f();
        return 0;
    } catch (const std::exception& e) {
        g_error = e.what();
        return -1;
    }
}

}  // namespace

extern "C" {

const char* ref_last_error(void) { return g_error.c_str(); }

int ref_pack_conv(const std::uint16_t* w, const std::uint16_t* bias, int oc, int ic, int kh, int kw,
                  std::uint16_t* packed, std::size_t packed_elems)
{
    return guard([&] {
        const auto v = pack_conv_weights_f16p16x1bias(w, bias, static_cast<std::size_t>(oc), static_cast<std::size_t>(ic),
                                                      static_cast<std::size_t>(kh), static_cast<std::size_t>(kw));
        if (v.size() > packed_elems) throw std::runtime_error("packed buffer too small");
        std::memcpy(packed, v.data(), v.size() * 2);
    });
}

int ref_pack_depthwise(const std::uint16_t* w, const std::uint16_t* bias, int c, int kh, int kw,
                       std::uint16_t* packed, std::size_t packed_elems)
{
    return guard([&] {
        const auto v = pack_depthwise_weights(w, bias, static_cast<std::size_t>(c), static_cast<std::size_t>(kh),
                                              static_cast<std::size_t>(kw));
        if (v.size() > packed_elems) throw std::runtime_error("packed buffer too small");
        std::memcpy(packed, v.data(), v.size() * 2);
    });
}

int ref_gemm_nhwc(std::size_t m, std::size_t n, std::size_t k, const std::uint16_t* lhs, const std::uint16_t* packed,
                  std::uint16_t* dst, int epi, float alpha, float cmin, float cmax, const std::uint16_t* residual,
                  int isa, int threads)
{
    return guard([&] {
        execute_gemm_nhwc(kernels(isa), m, n, k, lhs, packed, dst, epilogue(epi, alpha, cmin, cmax, residual),
                          pool(threads));
    });
}

int ref_spatial_conv_nhwc(const std::uint16_t* input, const std::uint16_t* packed, std::uint16_t* output, int n,
                          int ic, int ih, int iw, int oc, int oh, int ow, int kh, int kw, int sh, int sw, int ph,
                          int pw, int epi, float alpha, const std::uint16_t* residual, int isa, int threads)
{
    return guard([&] {
        execute_spatial_conv_nhwc(kernels(isa), input, packed, output, n, ic, ih, iw, oc, oh, ow, kh, kw, sh, sw, ph,
                                  pw, epilogue(epi, alpha, 0.0F, 0.0F, residual), pool(threads));
    });
}

int ref_depthwise_nhwc(const std::uint16_t* input, const std::uint16_t* packed, std::uint16_t* output, int n, int c,
                       int ih, int iw, int oh, int ow, int kh, int kw, int sh, int sw, int ph, int pw, int isa,
                       int threads)
{
    return guard([&] {
        // Same dispatch as CpuExecutionPlan::execute_step's run_conv.
        const bool s1p1 = kh == 3 && kw == 3 && sh == 1 && sw == 1 && ph == 1 && pw == 1 && oh == ih && ow == iw;
        if (s1p1)
            kernels(isa).depthwise3x3_s1p1(input, packed, output, n, ih, iw, c, pool(threads));
        else
            execute_depthwise_generic_nhwc(input, packed, output, n, c, ih, iw, oh, ow, kh, kw, sh, sw, ph, pw,
                                           pool(threads));
    });
}

int ref_leaky_relu(const std::uint16_t* in, std::uint16_t* out, std::size_t count, float alpha, int isa)
{
    return guard([&] { kernels(isa).unary(in, out, count, UnaryKind::kLeakyRelu, alpha, 0.0F, 0.0F, pool(1)); });
}

int ref_add(const std::uint16_t* a, const std::uint16_t* b, std::uint16_t* out, std::size_t count, int isa)
{
    return guard([&] { kernels(isa).binary_contiguous(a, b, out, count, BinaryKind::kAdd, pool(1)); });
}

int ref_depth_to_space_nhwc(const std::uint16_t* in, std::uint16_t* out, int n, int c, int h, int w, int block)
{
    return guard([&] { execute_depth_to_space_nhwc(in, out, n, c, h, w, block, pool(1)); });
}

int ref_space_to_depth_nhwc(const std::uint16_t* in, std::uint16_t* out, int n, int c, int h, int w, int block)
{
    return guard([&] { execute_space_to_depth_nhwc(in, out, n, c, h, w, block, pool(1)); });
}

int ref_nchw_to_nhwc(const std::uint16_t* in, std::uint16_t* out, std::size_t n, std::size_t c, std::size_t hw)
{
    return guard([&] { get_x86_avx2_kernels().nchw_to_nhwc(in, out, n, c, hw, pool(1)); });
}

int ref_nhwc_to_nchw(const std::uint16_t* in, std::uint16_t* out, std::size_t n, std::size_t hw, std::size_t c)
{
    return guard([&] { get_x86_avx2_kernels().nhwc_to_nchw(in, out, n, hw, c, pool(1)); });
}

// core/src/yuv.cpp: prepare_model_input (frame -> [1, 3, mh, mw], padding
// chosen by frame_padding) and prepare_model_output_into (model image ->
// frame). pad5 = {left, right, top, bottom, rotated}.
int ref_prepare_model_input(const std::uint8_t* yuv, int w, int h, int mw, int mh, float pixel_range,
                            std::uint16_t* out, int* pad5)
{
    return guard([&] {
        const std::size_t ysz = static_cast<std::size_t>(w) * h, uvsz = ysz / 4;
        const Yuv420FrameView view(w, h, std::span<const std::uint8_t>(yuv, ysz),
                                   std::span<const std::uint8_t>(yuv + ysz, uvsz),
                                   std::span<const std::uint8_t>(yuv + ysz + uvsz, uvsz));
        FramePadding pad;
        const Tensor t = prepare_model_input(view, mw, mh, pixel_range, pad);
        const auto& v = std::get<std::vector<Float16Storage>>(t.data);
        std::memcpy(out, v.data(), v.size() * sizeof(Float16Storage));
        pad5[0] = pad.left;
        pad5[1] = pad.right;
        pad5[2] = pad.top;
        pad5[3] = pad.bottom;
        pad5[4] = pad.rotated ? 1 : 0;
    });
}

int ref_prepare_model_output(const std::uint16_t* x, int w, int h, int mw, int mh, float pixel_range, const int* pad5,
                             std::uint8_t* yuv)
{
    return guard([&] {
        Tensor t{"x_hat", {1, 3, mh, mw}, std::vector<Float16Storage>(x, x + static_cast<std::size_t>(3) * mw * mh)};
        const std::size_t ysz = static_cast<std::size_t>(w) * h, uvsz = ysz / 4;
        const MutableYuv420FrameView view(w, h, std::span<std::uint8_t>(yuv, ysz),
                                          std::span<std::uint8_t>(yuv + ysz, uvsz),
                                          std::span<std::uint8_t>(yuv + ysz + uvsz, uvsz));
        FramePadding pad{pad5[0], pad5[1], pad5[2], pad5[3], pad5[4] != 0};
        prepare_model_output_into(t, view, pixel_range, pad);
    });
}

// Operators of the real-model graphs: the KernelSet entries and the slice /
// concat helpers of kernels_scalar.cpp, on NHWC buffers. unary op: 0 clip,
// 1 sigmoid, 2 reciprocal, 3 round; binary op: 0 add, 1 sub, 2 mul.
int ref_unary(const std::uint16_t* in, std::uint16_t* out, std::size_t count, int op, float lo, float hi, int isa, int threads)
{
    static constexpr UnaryKind kinds[4] = {UnaryKind::kClip, UnaryKind::kSigmoid, UnaryKind::kReciprocal, UnaryKind::kRound};
    return guard([&] { kernels(isa).unary(in, out, count, kinds[op & 3], 0.0F, lo, hi, pool(threads)); });
}

BinaryKind binary_kind(int op) { return op == 1 ? BinaryKind::kSub : op == 2 ? BinaryKind::kMul : BinaryKind::kAdd; }

int ref_binary_contiguous(const std::uint16_t* a, const std::uint16_t* b, std::uint16_t* out, std::size_t count, int op, int isa)
{
    return guard([&] { kernels(isa).binary_contiguous(a, b, out, count, binary_kind(op), pool(1)); });
}

int ref_binary_scalar(const std::uint16_t* vec, std::uint16_t scalar, std::uint16_t* out, std::size_t count, int op, int scalar_lhs,
                      int isa)
{
    return guard([&] { kernels(isa).binary_scalar_bcast(vec, scalar, out, count, binary_kind(op), scalar_lhs != 0, pool(1)); });
}

int ref_binary_channel(const std::uint16_t* vec, const std::uint16_t* chan, std::uint16_t* out, std::size_t spatial,
                       std::size_t channels, int op, int chan_lhs, int isa)
{
    return guard([&] {
        kernels(isa).binary_channel_bcast(vec, chan, out, spatial, channels, binary_kind(op), chan_lhs != 0, pool(1));
    });
}

int ref_slice_nhwc(const std::uint16_t* in, std::uint16_t* out, const int* id4, const int* od4, const int* starts,
                   const int* steps)
{
    return guard([&] { execute_slice_nhwc(in, out, id4, od4, starts, steps, pool(1)); });
}

int ref_concat_nhwc(const std::uint16_t* const* ins, const int* dims4, int n, std::uint16_t* out, const int* od4, int axis)
{
    return guard([&] {
        std::vector<const int*> dims(static_cast<std::size_t>(n));
        for (int i = 0; i < n; ++i) dims[static_cast<std::size_t>(i)] = dims4 + 4 * i;
        execute_concat_nhwc(ins, dims.data(), static_cast<std::size_t>(n), out, od4, axis, pool(1));
    });
}

int ref_reglu_nhwc(const std::uint16_t* in, std::uint16_t* out, std::size_t spatial, std::size_t g, float lo, float hi, int isa)
{
    return guard([&] { kernels(isa).reglu_nhwc(in, out, spatial, g, lo, hi, pool(1)); });
}

// 1x1 conv with the ReGLU epilogue (GemmEpilogueKind::kReglu), as the plan
// runs a matched CONV -> SLICE -> SLICE -> CLIP -> MUL chain.
int ref_gemm_reglu_nhwc(std::size_t m, std::size_t n, std::size_t k, const std::uint16_t* lhs, const std::uint16_t* packed,
                        std::uint16_t* dst, float lo, float hi, int isa, int threads)
{
    return guard([&] {
        GemmEpilogue e;
        e.kind = GemmEpilogueKind::kReglu;
        e.clamp_min = lo;
        e.clamp_max = hi;
        execute_gemm_nhwc(kernels(isa), m, n, k, lhs, packed, dst, e, pool(threads));
    });
}

int ref_feature_update_nhwc(const std::uint16_t* in, const std::uint16_t* history, const std::uint16_t* scale,
                            std::uint16_t* scaled_out, std::uint16_t* blended_out, std::uint16_t* feature_out,
                            std::size_t spatial, std::size_t channels, int isa)
{
    return guard([&] {
        if (scaled_out)
            kernels(isa).feature_update_outputs_nhwc(in, history, scale, scaled_out, blended_out, feature_out, spatial, channels,
                                                     pool(1));
        else
            kernels(isa).feature_update_nhwc(in, history, scale, feature_out, spatial, channels, pool(1));
    });
}

int ref_y0_tail_nhwc(const std::uint16_t* latent, const std::uint16_t* prior, const std::uint16_t* qs, const std::uint16_t* us0,
                     const std::uint16_t* us1, std::uint16_t* normalized, std::uint16_t* clipped, std::uint16_t* y_raw,
                     std::uint16_t* concat2, std::uint16_t* concat3, float clip_min, std::size_t spatial, std::size_t q, int isa)
{
    return guard([&] {
        kernels(isa).y0_tail_nhwc(latent, prior, qs, us0, us1, normalized, clipped, y_raw, concat2, concat3, clip_min, spatial, q,
                                  pool(1));
    });
}

int ref_y1_tail_nhwc(const std::uint16_t* normalized, const std::uint16_t* prior, const std::uint16_t* qs, const std::uint16_t* us0,
                     const std::uint16_t* us1, const std::uint16_t* concat2, const std::uint16_t* clipped, std::uint16_t* y_raw,
                     std::uint16_t* out, std::size_t spatial, std::size_t q, int isa)
{
    return guard([&] {
        kernels(isa).y1_tail_nhwc(normalized, prior, qs, us0, us1, concat2, clipped, y_raw, out, spatial, q, pool(1));
    });
}

std::uint16_t ref_float_to_half(float f) { return float_to_half(f); }
float ref_half_to_float(std::uint16_t h) { return half_to_float(h); }

}  // extern "C"
