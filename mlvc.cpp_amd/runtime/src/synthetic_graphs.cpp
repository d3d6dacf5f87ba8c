// Seeded synthetic conv graphs for the fixed-shape FP16 schedule.
//
// Every weight and input value is drawn from Rng (SplitMix64, Box-Muller in
// double) and rounded to FP16 with RNE before use. Topologies:
//
//   conv3x3_184x320      x[1,64,184,320] U[-1,1] -> CONV 3x3 s1 p1 64->64
//                        (W~N(0,0.05), b~N(0,0.01)) -> LEAKY_RELU(0.01)
//   conv_sweep_640x368   x[1,64,184,320] U[-1,1]; per level 3x3 + 1x1 at
//                        184x320/C64, 92x160/C128, 46x80/C256 with 3x3 s2
//                        convs between levels; LeakyReLU after the first six
//                        convs; W~N(0,1/sqrt(Cin*k*k)), b~N(0,0.01)
//   dwblock_<HxW>_c<C>   x[1,C,H,W] U[-1,1]; DW3x3 -> 1x1 C->2C + LeakyReLU
//                        -> 1x1 2C->C -> ADD x  (= y1); outputs
//                        1x1 4C->C of unshuffle2(y1) and shuffle2(3x3 C->4C
//                        of y1); W,b ~ N(0,0.02)
//   mlvc_s_640x368       MLVC-S-shaped per-frame graph, 8 frames (below)
//   mlvc_1920x1088       the same topology widened to 1/16, 32 frames
//   codec_{enc,dec}_*    the MLVCEncoder / MLVCDecoder pair of the buffered
//                        codec path (build_codec below)
//
// MLVC-shaped topology (frame x[1,3,H,W] U[0,1], state ref[1,64,H/2,W/2]):
//   SPACE_TO_DEPTH 2 -> 3x3 12->64 + LReLU -> CONCAT(ref) -> 1x1 128->64 +
//   LReLU -> 3x3 s2 convs 64->128->192(->256 at 1/16) + LReLU [-> 3x3 192->256
//   + LReLU at 1/8] -> B depthwise-separable residual blocks (C=256:
//   DW3x3, 1x1 256->512 + LReLU, 1x1 512->256, ADD) -> synthesis 3x3 convs +
//   LReLU each followed by DEPTH_TO_SPACE 2 back to 64 ch at 1/2 (= next
//   ref, state output) -> 3x3 64->12 -> DEPTH_TO_SPACE 2 -> recon [1,3,H,W].
// Convs followed by LeakyReLU use He scaling N(0, sqrt(2/fan_in)); linear
// convs N(0, 1/sqrt(fan_in)); residual-project convs are scaled by 0.1; all
// biases N(0, 0.01). This keeps activation RMS O(1) through depth and across
// frames of the recurrence.

#include "mlvc/runtime/graph_builder.hpp"
#include "mlvc/core/half.hpp"

#include <cmath>
#include <functional>
#include <map>
#include <mutex>
#include <stdexcept>

namespace mlvc::synth {
namespace {

using Id = GraphBuilder::Id;
using aot::Op;

std::vector<Float16Storage> normal_fp16(Rng& rng, std::size_t n, double std)
{
    std::vector<Float16Storage> v(n);
    for (auto& x : v) x = float_to_half(static_cast<float>(rng.normal() * std));
    return v;
}

struct Ctx {
    GraphBuilder& g;
    Rng& rng;
    int counter = 0;
    std::string next(const std::string& what) { return "n" + std::to_string(counter++) + "_" + what; }

    Id conv(Id x, int oc, int k, int stride, double wstd, double bstd = 0.01, int groups = 1)
    {
        const auto& xs = g.shape(x);
        const int ic = static_cast<int>(xs[1]);
        const int icg = ic / groups;
        const std::string base = next(k == 1 ? "conv1x1" : (groups > 1 ? "dwconv" : "conv3x3"));
        const Id w = g.weight_fp16(base + ".w", {oc, icg, k, k},
                                   normal_fp16(rng, static_cast<std::size_t>(oc) * icg * k * k, wstd));
        const Id b = g.weight_fp16(base + ".b", {oc}, normal_fp16(rng, static_cast<std::size_t>(oc), bstd));
        return g.conv(base, x, w, b, {stride, stride}, {k / 2, k / 2}, groups);
    }
    Id lrelu(Id x) { return g.leaky_relu(next("lrelu"), x, 0.01F); }
    Id conv_act(Id x, int oc, int k, int stride)
    {
        const auto& xs = g.shape(x);
        const double fan_in = static_cast<double>(xs[1]) * k * k;
        return lrelu(conv(x, oc, k, stride, std::sqrt(2.0 / fan_in)));
    }
    Id conv_lin(Id x, int oc, int k, int stride, double scale = 1.0)
    {
        const auto& xs = g.shape(x);
        const double fan_in = static_cast<double>(xs[1]) * k * k;
        return conv(x, oc, k, stride, scale / std::sqrt(fan_in));
    }
};

void build_conv3x3(GraphBuilder& g, Rng& rng, SyntheticModel& info)
{
    Ctx c{g, rng};
    const Id x = g.input("x", {1, 64, 184, 320});
    const Id y = c.lrelu(c.conv(x, 64, 3, 1, 0.05, 0.01));
    g.output(y);
    info.external_inputs = {{1, 64, 184, 320}};
    info.external_input_names = {"x"};
    info.input_lo = {-1.0};
    info.input_hi = {1.0};
}

void build_conv_sweep(GraphBuilder& g, Rng& rng, SyntheticModel& info)
{
    Ctx c{g, rng};
    auto sigma = [&](Id x, int k) { return 1.0 / std::sqrt(static_cast<double>(g.shape(x)[1]) * k * k); };
    const Id x = g.input("x", {1, 64, 184, 320});
    Id t = c.lrelu(c.conv(x, 64, 3, 1, sigma(x, 3)));
    t = c.lrelu(c.conv(t, 64, 1, 1, sigma(t, 1)));
    t = c.lrelu(c.conv(t, 128, 3, 2, sigma(t, 3)));
    t = c.lrelu(c.conv(t, 128, 3, 1, sigma(t, 3)));
    t = c.lrelu(c.conv(t, 128, 1, 1, sigma(t, 1)));
    t = c.lrelu(c.conv(t, 256, 3, 2, sigma(t, 3)));
    t = c.conv(t, 256, 3, 1, sigma(t, 3));
    t = c.conv(t, 256, 1, 1, sigma(t, 1));
    g.output(t);
    info.external_inputs = {{1, 64, 184, 320}};
    info.external_input_names = {"x"};
    info.input_lo = {-1.0};
    info.input_hi = {1.0};
}

void build_dwblock(GraphBuilder& g, Rng& rng, SyntheticModel& info, int h, int w, int ch)
{
    Ctx c{g, rng};
    const Id x = g.input("x", {1, ch, h, w});
    const Id d = c.conv(x, ch, 3, 1, 0.02, 0.02, ch);
    const Id e = c.lrelu(c.conv(d, 2 * ch, 1, 1, 0.02, 0.02));
    const Id f = c.conv(e, ch, 1, 1, 0.02, 0.02);
    const Id y1 = g.binary(Op::ADD, c.next("residual"), f, x);
    const Id u = g.pixel(Op::SPACE_TO_DEPTH, c.next("unshuffle"), y1, 2);
    const Id y2 = c.conv(u, ch, 1, 1, 0.02, 0.02);
    const Id s = c.conv(y1, 4 * ch, 3, 1, 0.02, 0.02);
    const Id y3 = g.pixel(Op::DEPTH_TO_SPACE, c.next("shuffle"), s, 2);
    g.output(y2);
    g.output(y3);
    info.external_inputs = {{1, ch, h, w}};
    info.external_input_names = {"x"};
    info.input_lo = {-1.0};
    info.input_hi = {1.0};
}

// levels == 3: analysis to 1/8 (C3 shape); levels == 4: to 1/16 (C4 shape).
void build_mlvc(GraphBuilder& g, Rng& rng, SyntheticModel& info, int h, int w, int levels,
                int blocks, int frames)
{
    Ctx c{g, rng};
    const Id x = g.input("x", {1, 3, h, w});
    const Id ref = g.input("ref_in", {1, 64, h / 2, w / 2});
    Id t = g.pixel(Op::SPACE_TO_DEPTH, c.next("unshuffle"), x, 2);
    t = c.conv_act(t, 64, 3, 1);
    t = g.concat(c.next("concat_ref"), {t, ref}, 1);
    t = c.conv_act(t, 64, 1, 1);
    t = c.conv_act(t, 128, 3, 2);
    t = c.conv_act(t, 192, 3, 2);
    if (levels == 3)
        t = c.conv_act(t, 256, 3, 1);
    else
        t = c.conv_act(t, 256, 3, 2);
    // Residual blocks (depthwise 3x3 has fan_in 9).
    for (int b = 0; b < blocks; ++b) {
        const std::string base = c.next("dw");
        const Id wd = g.weight_fp16(base + ".w", {256, 1, 3, 3}, normal_fp16(rng, 256 * 9, 1.0 / 3.0));
        const Id bd = g.weight_fp16(base + ".b", {256}, normal_fp16(rng, 256, 0.01));
        const Id d = g.conv(base, t, wd, bd, {1, 1}, {1, 1}, 256);
        const Id e = c.conv_act(d, 512, 1, 1);
        const Id f = c.conv_lin(e, 256, 1, 1, 0.1);
        t = g.binary(Op::ADD, c.next("residual"), f, t);
    }
    // Each conv is created before the shuffle that consumes it, so tensor
    // names and the order of random draws do not depend on argument
    // evaluation order.
    auto conv_shuffle = [&](Id in, int oc, bool act, const std::string& what) {
        const Id y = act ? c.conv_act(in, oc, 3, 1) : c.conv_lin(in, oc, 3, 1);
        return g.pixel(Op::DEPTH_TO_SPACE, c.next(what), y, 2);
    };
    if (levels == 3) {
        t = c.conv_act(t, 192, 3, 1);
        t = conv_shuffle(t, 512, true, "shuffle");  // 128 @1/4
    } else {
        t = conv_shuffle(t, 768, true, "shuffle");  // 192 @1/8
        t = conv_shuffle(t, 512, true, "shuffle");  // 128 @1/4
    }
    const Id state = conv_shuffle(t, 256, true, "shuffle_ref");     // 64 @1/2, next reference
    const Id recon = conv_shuffle(state, 12, false, "shuffle_recon");  // 3 @1/1
    g.output(recon);
    g.output(state);
    info.external_inputs = {{1, 3, h, w}};
    info.external_input_names = {"x"};
    info.input_lo = {0.0};
    info.input_hi = {1.0};
    info.state_bindings = {StateTensorBinding{1, 1, TensorDataType::kFloat16, {1, 64, h / 2, w / 2}}};
    info.frames = frames;
}

// Encoder / decoder pair of the buffered codec path (graph names
// MLVCEncoder / MLVCDecoder, as the reference's codec bundles use), built
// from the MLVC-shaped topology above at 1/16:
//   MLVCEncoder(x[1,3,h,w], q_index_shifted INT32[1], ref_in) ->
//     (y = analysis latent [1,256,h/16,w/16], ref_out)
//   MLVCDecoder(y, q_index_shifted, ref_in) -> (x_hat[1,3,h,w], ref_out)
// Analysis: SPACE_TO_DEPTH 2 -> 3x3 12->64 + LReLU -> CONCAT(ref_in) -> 1x1
// 128->64 + LReLU -> 3x3 s2 64->128->192->256 + LReLU -> B depthwise-separable
// residual blocks = y. Synthesis (both graphs, the same weights from their
// own Rng stream): 3x3 256->768, 192->512, 128->256 (+ LReLU, each followed by
// DEPTH_TO_SPACE 2) -> CONCAT(ref_in) -> 1x1 128->64 + LReLU = ref_out (the
// state, carried frame to frame); the decoder adds 3x3 64->12 -> DEPTH_TO_SPACE
// 2 = x_hat. The encoder runs the synthesis state path too, so its ref_out
// equals the decoder's for the same y and ref_in. q_index_shifted is the
// graphs' INT32 control input: no operator of this path reads it (the real
// models look up quantisation scales with it).
void build_codec(GraphBuilder& g, Rng& rng, SyntheticModel& info, int h, int w, int blocks, int frames, bool encoder)
{
    Ctx c{g, rng};
    const Id lead = encoder ? g.input("x", {1, 3, h, w}) : g.input("y", {1, 256, h / 16, w / 16});
    g.input("q_index_shifted", {1}, aot::DataType::INT32);
    const Id ref = g.input("ref_in", {1, 64, h / 2, w / 2});
    Id y = lead;
    if (encoder) {
        Id t = g.pixel(Op::SPACE_TO_DEPTH, c.next("unshuffle"), lead, 2);
        t = c.conv_act(t, 64, 3, 1);
        t = g.concat(c.next("concat_ref"), {t, ref}, 1);
        t = c.conv_act(t, 64, 1, 1);
        t = c.conv_act(t, 128, 3, 2);
        t = c.conv_act(t, 192, 3, 2);
        t = c.conv_act(t, 256, 3, 2);
        for (int b = 0; b < blocks; ++b) {
            const std::string base = c.next("dw");
            const Id wd = g.weight_fp16(base + ".w", {256, 1, 3, 3}, normal_fp16(rng, 256 * 9, 1.0 / 3.0));
            const Id bd = g.weight_fp16(base + ".b", {256}, normal_fp16(rng, 256, 0.01));
            const Id d = g.conv(base, t, wd, bd, {1, 1}, {1, 1}, 256);
            const Id e = c.conv_act(d, 512, 1, 1);
            const Id f = c.conv_lin(e, 256, 1, 1, 0.1);
            t = g.binary(Op::ADD, b + 1 == blocks ? std::string("y") : c.next("residual"), f, t);
        }
        y = t;
    }
    Rng syn_rng(0x5EEDC0DEC0DEULL);
    Ctx s{g, syn_rng, 1000};
    auto conv_shuffle = [&](Id in, int oc, bool act, const std::string& what) {
        const Id t = act ? s.conv_act(in, oc, 3, 1) : s.conv_lin(in, oc, 3, 1);
        return g.pixel(Op::DEPTH_TO_SPACE, s.next(what), t, 2);
    };
    Id t = conv_shuffle(y, 768, true, "shuffle");   // 192 @1/8
    t = conv_shuffle(t, 512, true, "shuffle");       // 128 @1/4
    t = conv_shuffle(t, 256, true, "shuffle");       // 64 @1/2
    t = g.concat(s.next("concat_ref"), {t, ref}, 1);
    const Id state = s.conv_act(t, 64, 1, 1);        // next reference
    if (encoder) {
        g.output(y);
        g.output(state);
        info.external_inputs = {{1, 3, h, w}, {1}};
        info.external_input_names = {"x", "q_index_shifted"};
        info.input_lo = {0.0, 0.0};
        info.input_hi = {1.0, 0.0};
    } else {
        const Id rec = s.conv_lin(state, 12, 3, 1);
        const Id xh = g.pixel(Op::DEPTH_TO_SPACE, "x_hat", rec, 2);
        g.output(xh);
        g.output(state);
        info.external_inputs = {{1, 256, h / 16, w / 16}, {1}};
        info.external_input_names = {"y", "q_index_shifted"};
        info.input_lo = {-1.0, 0.0};
        info.input_hi = {1.0, 0.0};
    }
    info.model_name = encoder ? "MLVCEncoder" : "MLVCDecoder";
    info.profile = "synthetic/codec_" + std::to_string(w) + "x" + std::to_string(h);
    info.state_bindings = {StateTensorBinding{2, 1, TensorDataType::kFloat16, {1, 64, h / 2, w / 2}}};
    info.frames = frames;
}

struct ConfigEntry {
    const char* name;
    std::function<void(GraphBuilder&, Rng&, SyntheticModel&)> make;
};

const std::vector<ConfigEntry>& registry()
{
    static const std::vector<ConfigEntry> entries = {
        {"conv3x3_184x320", build_conv3x3},
        {"conv_sweep_640x368", build_conv_sweep},
        {"dwblock_92x160_c128", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_dwblock(g, r, i, 92, 160, 128); }},
        {"dwblock_46x80_c256", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_dwblock(g, r, i, 46, 80, 256); }},
        {"dwblock_tiny", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_dwblock(g, r, i, 6, 10, 16); }},
        {"mlvc_s_640x368", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_mlvc(g, r, i, 368, 640, 3, 6, 8); }},
        {"mlvc_1920x1088", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_mlvc(g, r, i, 1088, 1920, 4, 12, 32); }},
        {"mlvc_s_tiny", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_mlvc(g, r, i, 32, 64, 3, 2, 4); }},
        {"mlvc_tiny", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_mlvc(g, r, i, 64, 128, 4, 2, 4); }},
        {"codec_enc_1920x1088", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_codec(g, r, i, 1088, 1920, 12, 32, true); }},
        {"codec_dec_1920x1088", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_codec(g, r, i, 1088, 1920, 12, 32, false); }},
        {"codec_enc_tiny", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_codec(g, r, i, 64, 128, 2, 4, true); }},
        {"codec_dec_tiny", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_codec(g, r, i, 64, 128, 2, 4, false); }},
    };
    return entries;
}

const ConfigEntry& find(const std::string& config)
{
    for (const auto& e : registry())
        if (config == e.name) return e;
    throw std::runtime_error("unknown synthetic config: " + config);
}

}  // namespace

std::vector<std::string> synthetic_configs()
{
    std::vector<std::string> names;
    for (const auto& e : registry()) names.emplace_back(e.name);
    return names;
}

GraphBuilder build_synthetic(const std::string& config, std::uint64_t seed, SyntheticModel* info)
{
    GraphBuilder g;
    Rng rng(seed);
    SyntheticModel local;
    find(config).make(g, rng, local);
    if (local.model_name.empty()) local.model_name = config;
    if (local.profile.empty()) local.profile = "synthetic/" + config;
    if (info) *info = local;
    return g;
}

SyntheticModel synthetic_info(const std::string& config)
{
    static std::mutex mu;
    static std::map<std::string, SyntheticModel> cache;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(config);
    if (it == cache.end()) {
        SyntheticModel info;
        build_synthetic(config, 0, &info);
        it = cache.emplace(config, info).first;
    }
    return it->second;
}

std::vector<Float16Storage> synthetic_input(const std::string& config, std::size_t input_index,
                                            int frame, std::uint64_t seed)
{
    const SyntheticModel info = synthetic_info(config);
    if (input_index >= info.external_inputs.size()) throw std::runtime_error("input index out of range");
    std::size_t n = 1;
    for (auto d : info.external_inputs[input_index]) n *= static_cast<std::size_t>(d);
    Rng rng(seed ^ (0xA5A5A5A5ULL + 0x1000193ULL * (input_index + 1)) ^
            (static_cast<std::uint64_t>(frame + 1) * 0x9E3779B97F4A7C15ULL));
    const double lo = info.input_lo[input_index], hi = info.input_hi[input_index];
    if (info.external_input_names[input_index] == "q_index_shifted")
        throw std::runtime_error("q_index_shifted is an INT32 control input; pass it directly");
    std::vector<Float16Storage> v(n);
    for (auto& x : v) x = float_to_half(static_cast<float>(lo + (hi - lo) * rng.uniform()));
    return v;
}

}  // namespace mlvc::synth
