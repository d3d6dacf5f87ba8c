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
//   mlvc_s_320x192       the same graph at 320x192, 12 frames
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
    info.profile = "synthetic-codec_" + std::to_string(w) + "x" + std::to_string(h);
    // The bundle's model description (metadata.pb), shared by both graphs:
    // 64-channel feature at 1/2, 256-channel latent at 1/16, hyperprior at
    // 1/64, QP table of 64 of 72 with a 4-frame shift cycle, no feature reset.
    wire::ModelMetadata meta;
    meta.model_version = "synthetic-v1";
    meta.width = static_cast<std::uint32_t>(w);
    meta.height = static_cast<std::uint32_t>(h);
    meta.pixel_range = 1.0F;
    meta.qp_num = 64;
    meta.total_qp_num = 72;
    meta.frame_index_map = {0, 1, 2, 3};
    meta.qp_shift = {0, 8, 4, 8};
    meta.feature_channels = 64;
    meta.latent_channels = 256;
    meta.hyperprior_channels = 128;
    meta.downsample_feature = 2;
    meta.downsample_latent = 16;
    meta.downsample_hyperprior = 4;
    meta.y_scale_repeat = 2;
    meta.disable_feature_reset = true;
    g.set_metadata(meta);
    info.state_bindings = {StateTensorBinding{2, 1, TensorDataType::kFloat16, {1, 64, h / 2, w / 2}}};
    info.frames = frames;
}

std::vector<Float16Storage> uniform_fp16(Rng& rng, std::size_t n, double lo, double hi)
{
    std::vector<Float16Storage> v(n);
    for (auto& x : v) x = float_to_half(static_cast<float>(lo + (hi - lo) * rng.uniform()));
    return v;
}

Id scalar_fp16(GraphBuilder& g, const std::string& name, float v)
{
    return g.weight_fp16(name, {1}, {float_to_half(v)});
}

// Every single operator of the schema outside the conv path, one node each,
// with every broadcast form, slice form, concat axis and gather source:
//   x[1,24,12,20] U[-2,2], q_index_shifted INT32[1] (0..71), z[2,8,6,10] U[-2,2].
void build_ops_zoo(GraphBuilder& g, Rng& rng, SyntheticModel& info)
{
    Ctx c{g, rng};
    const Id x = g.input("x", {1, 24, 12, 20});
    const Id q = g.input("q_index_shifted", {1}, aot::DataType::INT32);
    const Id z = g.input("z", {2, 8, 6, 10});
    auto w16 = [&](const std::string& name, const GraphBuilder::Shape& s, double lo, double hi) {
        std::size_t n = 1;
        for (auto d : s) n *= static_cast<std::size_t>(d);
        return g.weight_fp16(name, s, uniform_fp16(rng, n, lo, hi));
    };
    // Unary.
    const Id c1 = g.clip("clip_both", x, scalar_fp16(g, "clip_both/min", -1.0F), scalar_fp16(g, "clip_both/max", 1.0F));
    const Id c2 = g.clip("clip_min", x, scalar_fp16(g, "clip_min/min", 0.25F), 0);
    const Id c3 = g.clip("clip_max", x, 0, scalar_fp16(g, "clip_max/max", 0.5F));
    const Id sg = g.unary(Op::SIGMOID, "sigmoid", x);
    const Id rc = g.unary(Op::RECIPROCAL, "reciprocal", c2);
    const Id x3 = g.binary(Op::MUL, "times3", x, scalar_fp16(g, "three", 3.0F));
    const Id rd = g.unary(Op::ROUND, "round", x3);
    // Binary broadcast forms.
    const Id b1 = g.binary(Op::SUB, "scalar_lhs", scalar_fp16(g, "half", 0.5F), sg);
    const Id b2 = g.binary(Op::MUL, "chan_rhs", rc, w16("chan24", {1, 24, 1, 1}, -2, 2));
    const Id b3 = g.binary(Op::SUB, "chan_lhs", w16("chanb24", {1, 24, 1, 1}, -2, 2), c1);
    const Id b4 = g.binary(Op::ADD, "spatial", rd, w16("plane", {1, 1, 12, 20}, -1, 1));
    const Id rowv = g.slice("row", c3, {0}, {1}, {2});              // [1,24,1,20]
    const Id colv = g.slice("col", x, {0, 5}, {1, 6}, {1, 3});      // [1,1,12,1]
    const Id b5 = g.binary(Op::MUL, "outer", rowv, colv);           // [1,24,12,20]
    const Id b6 = g.binary(Op::ADD, "same", b4, b5);
    // Slices.
    const Id s1 = g.slice("chan_slice", b2, {4}, {12}, {1});                          // [1,8,12,20]
    const Id s2 = g.slice("strided", b3, {1, 2, 19}, {24, 12, 0}, {1, 2, 3}, {3, 2, -2});  // [1,8,5,10]
    const Id s3 = g.slice("neg_start", b6, {-6}, {100}, {2});                           // [1,24,6,20]
    // Concats along every axis.
    const Id k1 = g.concat("cat_c", {s1, b1, s1}, 1);                                    // [1,40,12,20]
    const Id k2 = g.concat("cat_h", {s3, b6}, 2);                                        // [1,24,18,20]
    const Id zz = g.unary(Op::SIGMOID, "z_sig", z);
    const Id k3 = g.concat("cat_w", {z, zz}, 3);                                         // [2,8,6,20]
    const Id k4 = g.concat("cat_n", {z, zz}, 0);                                         // [4,8,6,10]
    // Gathers: a quantisation-style table row picked by the INT32 control
    // input, INT64 channel and column indices.
    const Id row = g.gather("q_row", w16("table", {72, 24, 1, 1}, 0.5, 1.5), q, 0);       // [1,24,1,1]
    const Id gq = g.binary(Op::MUL, "q_scaled", x, row);
    const Id pick = g.weight_int64("chan_pick/idx", {3}, {5, -1, 0});
    const Id gi = g.gather("chan_pick", gq, pick, 1);                                     // [1,3,12,20]
    const Id gw = g.gather("col_pick", k2, g.weight_int64("col_pick/idx", {2}, {19, 3}), 3);        // [1,24,18,2]
    // A second GATHER sharing the first one's index initializer.
    const Id gs = g.gather("chan_pick_shared", b2, pick, 1);                              // [1,3,12,20]
    const Id bz = g.binary(Op::MUL, "z_batch", k4, w16("zb", {4, 1, 1, 1}, -1, 1));
    for (Id o : {k1, s2, k3, gi, gw, bz, gs}) g.output(o);
    info.external_inputs = {{1, 24, 12, 20}, {1}, {2, 8, 6, 10}};
    info.external_input_names = {"x", "q_index_shifted", "z"};
    info.input_lo = {-2.0, 0.0, -2.0};
    info.input_hi = {2.0, 71.0, 2.0};
}

// Node chains of the real-model patterns the reference CPU matcher fuses
// (backends/cpu/src/fusion_matcher.cpp:258-850), emitted node by node in
// the order the matcher expects.
struct Patterns {
    GraphBuilder& g;
    Rng& rng;
    Id one;

    Id w16(const std::string& name, const GraphBuilder::Shape& s, double lo, double hi)
    {
        std::size_t n = 1;
        for (auto d : s) n *= static_cast<std::size_t>(d);
        return g.weight_fp16(name, s, uniform_fp16(rng, n, lo, hi));
    }
    Id slice_c(const std::string& name, Id t, std::int64_t b, std::int64_t e) { return g.slice(name, t, {b}, {e}, {1}); }
    // SLICE gate / linear -> CLIP(gate, -1, 6) -> MUL.
    Id reglu(const std::string& p, Id u)
    {
        const std::int64_t gc = g.shape(u)[1] / 2;
        const Id gate = slice_c(p + "_gate", u, 0, gc);
        const Id lin = slice_c(p + "_lin", u, gc, 2 * gc);
        const Id lo = scalar_fp16(g, p + "_lo", -1.0F);
        const Id hi = scalar_fp16(g, p + "_hi", 6.0F);
        const Id cg = g.clip(p + "_clip", gate, lo, hi);
        return g.binary(Op::MUL, p + "_out", cg, lin);
    }
    // a | b | c slices, sb = SIGMOID(b), sc = SIGMOID(c), blended =
    // sb*h + (1 - sb)*a, scaled = sc*blended*scale[1,C,1,1].
    std::pair<Id, Id> feature(const std::string& p, Id in, Id h0)
    {
        const std::int64_t cc = g.shape(in)[1] / 3;
        const Id a = slice_c(p + "_a", in, 0, cc);
        const Id b = slice_c(p + "_b", in, cc, 2 * cc);
        const Id c = slice_c(p + "_c", in, 2 * cc, 3 * cc);
        const Id sb = g.unary(Op::SIGMOID, p + "_sb", b);
        const Id sc = g.unary(Op::SIGMOID, p + "_sc", c);
        const Id wb = g.binary(Op::MUL, p + "_wb", sb, h0);
        const Id inv = g.binary(Op::SUB, p + "_inv", one, sb);
        const Id wa = g.binary(Op::MUL, p + "_wa", inv, a);
        const Id bl = g.binary(Op::ADD, p + "_blend", wb, wa);
        const Id gt = g.binary(Op::MUL, p + "_gated", sc, bl);
        const Id scale = w16(p + "_scale", {1, cc, 1, 1}, 0.5, 1.5);
        return {g.binary(Op::MUL, p + "_scaled", gt, scale), bl};
    }
    // (normalized - prior) * quant_scale -> halves -> ADD -> ROUND = y_raw;
    // (y_raw + prior half) * update_scale per half -> CONCAT. Returns
    // (y_raw, concat).
    std::pair<Id, Id> update(const std::string& p, Id normalized, Id pri, Id qscale, Id u0s, Id u1s)
    {
        const std::int64_t q = g.shape(normalized)[1] / 2;
        const Id d = g.binary(Op::SUB, p + "_diff", normalized, pri);
        const Id sc = g.binary(Op::MUL, p + "_scaled", d, qscale);
        const Id h0 = slice_c(p + "_s0", sc, 0, q);
        const Id h1 = slice_c(p + "_s1", sc, q, 2 * q);
        const Id sum = g.binary(Op::ADD, p + "_sum", h0, h1);
        const Id raw = g.unary(Op::ROUND, p + "_raw", sum);
        const Id t0 = slice_c(p + "_t0", pri, 0, q);
        const Id t1 = slice_c(p + "_t1", pri, q, 2 * q);
        const Id a0 = g.binary(Op::ADD, p + "_a0", raw, t0);
        const Id u0 = g.binary(Op::MUL, p + "_u0", a0, u0s);
        const Id a1 = g.binary(Op::ADD, p + "_a1", raw, t1);
        const Id u1 = g.binary(Op::MUL, p + "_u1", a1, u1s);
        return {raw, g.concat(p + "_cat", {u0, u1}, 1)};
    }
    struct Y0 {
        Id normalized, clipped, raw, concat2, concat3;
    };
    // prior head / tail slices, CLIP(head, 0.11) -> RECIPROCAL -> MUL(1) ->
    // MUL(latent) = normalized, update, CONCAT(concat2, prior).
    Y0 y0(Id latent, Id prior, Id qs, Id us0, Id us1)
    {
        const std::int64_t q = g.shape(prior)[1] / 4;
        const Id head = slice_c("y0_head", prior, 0, 2 * q);
        const Id tail = slice_c("y0_tail", prior, 2 * q, 4 * q);
        const Id clipped = g.clip("y0_clip", head, scalar_fp16(g, "y0_clip/min", 0.11F), 0);
        const Id inv0 = g.unary(Op::RECIPROCAL, "y0_inv", clipped);
        const Id inv = g.binary(Op::MUL, "y0_inv1", inv0, one);
        const Id nrm = g.binary(Op::MUL, "y0_norm", inv, latent);
        const auto [raw, cat2] = update("y0", nrm, tail, qs, us0, us1);
        return {nrm, clipped, raw, cat2, g.concat("y0_cat3", {cat2, prior}, 1)};
    }
    // update on (normalized, prior), + concat2 (of y0), * clipped (of y0).
    std::pair<Id, Id> y1(Id normalized, Id prior, Id qs, Id us0, Id us1, Id concat2, Id clipped)
    {
        const auto [raw, cat] = update("y1", normalized, prior, qs, us0, us1);
        const Id added = g.binary(Op::ADD, "y1_add", cat, concat2);
        return {raw, g.binary(Op::MUL, "y1_out", added, clipped)};
    }
};

// The real-model patterns with the recurrent feature as bound state
// (x[1,16,h,w] U[-1,1], q_index_shifted INT32[1], state feat[1,C,h,w]):
//   t = 3x3 16->32 + LReLU; ReGLU FFN: 1x1 32->64 -> SLICE gate/linear ->
//   CLIP(gate, -1, 6) -> MUL, + t; scale by a [72,32,1,1] table row
//   GATHERed at q; feature update (case A) on 1x1 ->3C with the state as
//   history: CONCAT(scaled, blended) -> 1x1 2C->C + LReLU = next state;
//   a standalone ReGLU on a graph-output tensor; a second feature update
//   whose CONCAT is deferred past another node (case B); the y0 and y1
//   quantisation tails at half resolution (Q channels) on 1x1 convs of a
//   3x3 s2 conv of the state, y1 reusing y0's concat2 and clipped outputs.
void build_realops(GraphBuilder& g, Rng& rng, SyntheticModel& info, int h, int w, int ch, int q, int frames)
{
    Ctx c{g, rng};
    const Id x = g.input("x", {1, 16, h, w});
    const Id qi = g.input("q_index_shifted", {1}, aot::DataType::INT32);
    const Id hist = g.input("feat_in", {1, ch, h, w});
    Patterns pt{g, rng, scalar_fp16(g, "one", 1.0F)};

    Id t = c.conv_act(x, 32, 3, 1);
    const Id ffn = pt.reglu("ffn", c.conv_lin(t, 64, 1, 1));
    t = g.binary(Op::ADD, "ffn_res", ffn, t);
    const Id row = g.gather("qrow", pt.w16("qtable", {72, 32, 1, 1}, 0.5, 1.5), qi, 0);
    t = g.binary(Op::MUL, "qscale", t, row);
    // Feature update, CONCAT right after (case A) -> next state.
    const auto [fa_scaled, fa_blended] = pt.feature("fu", c.conv_lin(t, 3 * ch, 1, 1), hist);
    const Id feat = g.concat("fu_feature", {fa_scaled, fa_blended}, 1);
    const Id state = c.conv_act(feat, ch, 1, 1);
    // Standalone ReGLU on a tensor that is also a graph output.
    const Id rin = c.conv_lin(feat, 2 * ch, 1, 1);
    const Id rout = pt.reglu("glu", rin);
    // Feature update with its CONCAT deferred (case B).
    const int c2 = ch / 2;
    const Id fv_in = c.conv_lin(rout, 3 * c2, 1, 1);
    const Id fv_hist = pt.slice_c("fv_hist", state, 0, c2);
    const auto [fb_scaled, fb_blended] = pt.feature("fv", fv_in, fv_hist);
    const Id between = c.lrelu(rout);
    const Id featb = g.concat("fv_feature", {fb_scaled, fb_blended}, 1);
    // Quantisation tails at half resolution.
    const Id lat_src = c.conv_act(state, 32, 3, 2);
    const Id latent = c.conv_lin(lat_src, 2 * q, 1, 1);
    const Id prior = c.conv_lin(lat_src, 4 * q, 1, 1);
    const Id qs = c.conv_lin(lat_src, 2 * q, 1, 1);
    const Id us0 = c.conv_lin(lat_src, q, 1, 1);
    const Id us1 = c.conv_lin(lat_src, q, 1, 1);
    const auto y0 = pt.y0(latent, prior, qs, us0, us1);
    const Id src1 = c.conv_act(lat_src, 32, 1, 1);
    const Id nrm1 = c.conv_lin(src1, 2 * q, 1, 1);
    const Id pri1 = c.conv_lin(src1, 2 * q, 1, 1);
    const Id qs1 = c.conv_lin(src1, 2 * q, 1, 1);
    const Id us10 = c.conv_lin(src1, q, 1, 1);
    const Id us11 = c.conv_lin(src1, q, 1, 1);
    const auto [raw1, y1out] = pt.y1(nrm1, pri1, qs1, us10, us11, y0.concat2, y0.clipped);
    g.output(state);
    for (Id o : {rin, rout, between, featb, y0.normalized, y0.raw, y0.concat3, raw1, y1out}) g.output(o);
    info.external_inputs = {{1, 16, h, w}, {1}};
    info.external_input_names = {"x", "q_index_shifted"};
    info.input_lo = {-1.0, 0.0};
    info.input_hi = {1.0, 71.0};
    info.state_bindings = {StateTensorBinding{2, 0, TensorDataType::kFloat16, {1, ch, h, w}}};
    info.frames = frames;
}

// Every fused pattern on graph inputs directly (no convs), so the GPU and
// the oracle see identical operands: ReGLU of u[1,2G,h,w]; feature update
// case A on (fa[1,3C,h,w], ha[1,C,h,w]) and case B on (fb, hb); y0 on
// (latent[1,2Q], prior[1,4Q], qs[1,2Q], us0, us1[1,Q]) and y1 on
// (n1, p1, qs1[1,2Q], v0, v1[1,Q]) with y0's concat2 and clipped.
void build_fused(GraphBuilder& g, Rng& rng, SyntheticModel& info, int h, int w, int gc, int ch, int q)
{
    Patterns pt{g, rng, scalar_fp16(g, "one", 1.0F)};
    std::vector<std::vector<std::int64_t>> shapes;
    std::vector<std::string> names;
    auto in = [&](const std::string& name, std::int64_t c) {
        shapes.push_back({1, c, h, w});
        names.push_back(name);
        return g.input(name, {1, c, h, w});
    };
    const Id u = in("u", 2 * gc);
    const Id fa = in("fa", 3 * ch), ha = in("ha", ch), fb = in("fb", 3 * ch), hb = in("hb", ch);
    const Id latent = in("latent", 2 * q), prior = in("prior", 4 * q), qs = in("qs", 2 * q), us0 = in("us0", q), us1 = in("us1", q);
    const Id n1 = in("n1", 2 * q), p1 = in("p1", 2 * q), qs1 = in("qs1", 2 * q), v0 = in("v0", q), v1 = in("v1", q);
    const Id r = pt.reglu("glu", u);
    const auto [sa, ba] = pt.feature("fu", fa, ha);
    const Id feat_a = g.concat("fu_feature", {sa, ba}, 1);
    const auto [sb, bb] = pt.feature("fv", fb, hb);
    const Id between = g.leaky_relu("between", r, 0.01F);
    const Id feat_b = g.concat("fv_feature", {sb, bb}, 1);
    const auto y0 = pt.y0(latent, prior, qs, us0, us1);
    const auto [raw1, y1out] = pt.y1(n1, p1, qs1, v0, v1, y0.concat2, y0.clipped);
    for (Id o : {r, feat_a, between, feat_b, y0.normalized, y0.raw, y0.concat3, raw1, y1out}) g.output(o);
    info.external_inputs = shapes;
    info.external_input_names = names;
    info.input_lo.assign(shapes.size(), -2.0);
    info.input_hi.assign(shapes.size(), 2.0);
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
        {"mlvc_s_320x192", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_mlvc(g, r, i, 192, 320, 3, 6, 12); }},
        {"mlvc_s_tiny", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_mlvc(g, r, i, 32, 64, 3, 2, 4); }},
        {"mlvc_tiny", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_mlvc(g, r, i, 64, 128, 4, 2, 4); }},
        {"codec_enc_1920x1088", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_codec(g, r, i, 1088, 1920, 12, 32, true); }},
        {"codec_dec_1920x1088", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_codec(g, r, i, 1088, 1920, 12, 32, false); }},
        {"codec_enc_tiny", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_codec(g, r, i, 64, 128, 2, 4, true); }},
        {"codec_dec_tiny", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_codec(g, r, i, 64, 128, 2, 4, false); }},
        {"ops_zoo_tiny", build_ops_zoo},
        {"realops_tiny", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_realops(g, r, i, 16, 24, 32, 16, 3); }},
        {"realops_odd_tiny", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_realops(g, r, i, 10, 14, 12, 6, 2); }},
        {"realops_544x960", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_realops(g, r, i, 544, 960, 64, 96, 8); }},
        {"fused_tiny", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_fused(g, r, i, 12, 20, 16, 16, 8); }},
        {"fused_odd_tiny", [](GraphBuilder& g, Rng& r, SyntheticModel& i) { build_fused(g, r, i, 5, 7, 12, 13, 6); }},
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
    if (local.profile.empty()) local.profile = "synthetic-" + config;  // one path component, as embedded profiles are
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
