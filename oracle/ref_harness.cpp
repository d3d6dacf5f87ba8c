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

std::uint16_t ref_float_to_half(float f) { return float_to_half(f); }
float ref_half_to_float(std::uint16_t h) { return half_to_float(h); }

}  // extern "C"
