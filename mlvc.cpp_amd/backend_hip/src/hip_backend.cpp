// "hip" backend: graph lowering, fusion, memory planning and hipGraph replay.
//
// Behavioural references (nothing of the CUDA code is reused):
//   * lifecycle and run() checks: backends/cpu/src/execution_plan.cpp:1623-
//     1675 and backends/driver_cubin/src/cuda_graph_executor.cpp:90-154;
//   * conv classification (groups == 1 vs depthwise, error on other
//     grouped convs): execution_plan.cpp:410-462;
//   * conv epilogue fusion rule (LeakyReLU / same-shape non-initializer ADD
//     after a conv whose output has one consumer and is not a graph output):
//     fusion_matcher.cpp:352-411;
//   * state bindings (feature_out(t) -> ref_in(t+1), zeroed by reset_state):
//     backend.hpp:34-46, execution_plan.cpp:349-369/806-816/1033-1042. The
//     driver backend aliases the state output onto its input and therefore
//     requires the final node to produce it (graph_validator.cpp:11-46);
//     this backend instead keeps two state buffers and captures one
//     hipGraph per parity, so the state output may be produced anywhere;
//   * one graph replay per frame: cuda_graph_executor.cpp:38-52.
// MI355X-specific lowering on top of the reference rules: SPACE_TO_DEPTH and
// channel CONCAT feeding a conv are folded into the conv's input staging,
// DEPTH_TO_SPACE consuming a conv is folded into its store, and device
// memory is re-planned over the fused launch schedule.

#include "hip_backend.hpp"

#include "mlvc/core/half.hpp"
#include "mlvc_hip_device.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <set>
#include <stdexcept>

#include <unistd.h>

namespace mlvc::hip_backend {
namespace {

using aot::Op;
using aot::TensorId;

[[noreturn]] void fail(const std::string& what) { throw std::runtime_error("hip: " + what); }

// MLVC_HIP_DISABLE_FUSION=1 lowers every node to its own kernel (the
// counterpart of the reference's MLVC_CPU_DISABLE_FUSION,
// backends/cpu/src/execution_plan.cpp:89-93); used to check that fused and
// unfused schedules agree.
bool fusion_enabled()
{
    const char* env = std::getenv("MLVC_HIP_DISABLE_FUSION");
    return !(env && env[0] == '1' && env[1] == '\0');
}

// MLVC_HIP_BLOCK_HANDOVER=nchw keeps every activation NCHW (default: fused
// blocks and the 3x3 convs around them hand over channel-last where they
// can); for comparing the two layouts, which give identical results.
bool block_handover_nhwc()
{
    const char* env = std::getenv("MLVC_HIP_BLOCK_HANDOVER");
    return !(env && std::string(env) == "nchw");
}

// MLVC_HIP_CONV_VARIANT=<variant name> runs every conv that variant can
// run with it, untuned (tests sweep the variants this way).
std::string forced_conv_variant()
{
    const char* env = std::getenv("MLVC_HIP_CONV_VARIANT");
    return env ? std::string(env) : std::string();
}

void hip_check(int rc, const char* what)
{
    if (rc != 0) fail(std::string(what) + ": " + mlvc_hip_last_error());
}

std::size_t elem_count(const std::vector<std::int64_t>& s)
{
    std::size_t n = 1;
    for (auto d : s) n *= static_cast<std::size_t>(d);
    return n;
}

// Bytes of a tensor from its descriptor. Computed here from the schema-3
// types only (aot_graph.hpp:36-41, 98-103), so the backend builds against
// the reference's runtime headers, which declare no such helper.
std::size_t desc_bytes(const aot::TensorDescriptor& t)
{
    std::size_t elem = 0;
    switch (t.dtype) {
    case aot::DataType::FP16: elem = 2; break;
    case aot::DataType::INT32: elem = 4; break;
    case aot::DataType::INT64: elem = 8; break;
    default: fail("unsupported tensor data type");
    }
    return elem * elem_count(t.shape);
}

struct DeviceMem {
    void* ptr = nullptr;
    DeviceMem() = default;
    explicit DeviceMem(std::size_t bytes) { hip_check(mlvc_hip_malloc(&ptr, bytes), "device allocation"); }
    DeviceMem(const DeviceMem&) = delete;
    DeviceMem& operator=(const DeviceMem&) = delete;
    DeviceMem(DeviceMem&& o) noexcept : ptr(o.ptr) { o.ptr = nullptr; }
    DeviceMem& operator=(DeviceMem&& o) noexcept
    {
        std::swap(ptr, o.ptr);
        return *this;
    }
    ~DeviceMem()
    {
        if (ptr) mlvc_hip_free(ptr);
    }
};

struct HostMem {
    void* ptr = nullptr;
    HostMem() = default;
    explicit HostMem(std::size_t bytes) { hip_check(mlvc_hip_host_alloc(&ptr, bytes), "pinned allocation"); }
    HostMem(const HostMem&) = delete;
    HostMem& operator=(const HostMem&) = delete;
    HostMem(HostMem&& o) noexcept : ptr(o.ptr) { o.ptr = nullptr; }
    HostMem& operator=(HostMem&& o) noexcept
    {
        std::swap(ptr, o.ptr);
        return *this;
    }
    ~HostMem()
    {
        if (ptr) mlvc_hip_host_free(ptr);
    }
};

struct Launch {
    enum Kind {
        kConv, kDepthwise, kDwBlock, kPair, kLeaky, kAdd, kD2S, kS2D, kConcat,
        kUnary, kBinary, kSlice, kConcatAny, kGather, kReglu, kFeature, kY0, kY1
    } kind = kConv;
    std::string name, kind_name;
    TensorId x = 0, x2 = 0, res = 0, y = 0;  // tensors read (x, x2, res) and written (y)
    std::vector<TensorId> ins, outs;         // further tensors read / written
    int op = 0;
    float lo = 0.0F, hi = 0.0F;
    std::int64_t da[4] = {}, db[4] = {}, dy[4] = {}, starts[4] = {}, steps[4] = {};
    struct Piece {
        std::size_t rows, row_elems, y_offset, y_stride;
    };
    std::vector<Piece> pieces;  // CONCAT: one block copy per input (ins)
    std::size_t outer = 0, dim = 0, inner = 0;
    bool idx64 = false;
    mlvc_hip_conv_desc conv{};
    mlvc_hip_dwblock_desc blk{};
    mlvc_hip_convpair_desc pair{};
    DeviceMem packed, bias, packed2, bias2, packed3, bias3;
    std::vector<std::uint16_t> w_oihw;  // conv weights kept for re-packing after tuning
    std::vector<float> bias_oc;         // conv bias, unpadded
    bool forced = false;                // variant set by MLVC_HIP_CONV_VARIANT, not tuned
    int n = 0, c = 0, ih = 0, iw = 0, oh = 0, ow = 0, kh = 0, kw = 0, sh = 1, sw = 1, ph = 0, pw = 0;
    int block = 0, ca = 0, cb = 0;
    std::size_t count = 0, hw = 0;
    float alpha = 0.0F;
    double flops = 0.0, bytes = 0.0;
};

}  // namespace

class Plan {
public:
    Plan(const BackendOptions& options, const std::string& model, const ModelExecutionConfig& config)
        : device_(options.device_id), model_(model)
    {
        int count = 0;
        hip_check(mlvc_hip_device_count(&count), "device query");
        if (count <= device_) fail("HIP device " + std::to_string(device_) + " is not available");
        hip_check(mlvc_hip_set_device(device_), "set device");
        const auto assets = resolve_model_asset_reader(options.model_dir, options.asset_reader);
        graph_ = aot::load_aot_graph(*assets, model);
        hip_check(mlvc_hip_stream_create(&stream_), "stream creation");
        hip_check(mlvc_hip_event_create(&ev0_), "event creation");
        hip_check(mlvc_hip_event_create(&ev1_), "event creation");
        bind_state(config);
        lower();
        plan_memory();
        allocate_io();
        upload_parameters();
        if (tuning_enabled()) tune();
        // Kernel tables are computed before capture (nothing synchronous
        // may run while the stream is capturing).
        hip_check(mlvc_hip_prepare_tables(stream_), "device tables");
        capture();
        initialized_ = bindings_.empty();
    }

    ~Plan()
    {
        // Pending codec slots and any queued work finish before buffers go.
        mlvc_hip_set_device(device_);
        mlvc_hip_stream_synchronize(stream_);
        for (auto& sl : slots_)
            if (sl.done) mlvc_hip_event_destroy(sl.done);
        for (auto g : graphs_) mlvc_hip_graph_destroy(g);
        mlvc_hip_event_destroy(ev0_);
        mlvc_hip_event_destroy(ev1_);
        for (auto e : frame_evs_) mlvc_hip_event_destroy(e);
        if (flush_buf_) mlvc_hip_free(flush_buf_);
        mlvc_hip_stream_destroy(stream_);
    }

    std::vector<std::vector<std::int64_t>> io_shapes(bool outputs) const
    {
        std::vector<std::vector<std::int64_t>> s;
        for (TensorId id : outputs ? ext_out_ : ext_in_) s.push_back(desc(id).shape);
        return s;
    }

    std::vector<TensorDataType> io_dtypes(bool outputs) const
    {
        std::vector<TensorDataType> t;
        for (TensorId id : outputs ? ext_out_ : ext_in_)
            t.push_back(desc(id).dtype == aot::DataType::INT32 ? TensorDataType::kInt32 : TensorDataType::kFloat16);
        return t;
    }

    // ------------------------------------------------------- codec I/O
    // The buffered path of the reference's GPU backend
    // (backends/driver_cubin/src/cuda_graph_executor.cpp:156-400) with the
    // checks of the CPU backend's configure_codec_io
    // (backends/cpu/src/execution_plan.cpp:1386-1486): per slot a pinned
    // frame, pinned copies of the graph's external outputs (encoder) or
    // inputs (decoder) and an event; submits run upload -> conversion kernel
    // -> frame graph -> download on the backend's stream.
    void configure_codec_io(const CodecIoConfig& cfg)
    {
        if (codec_on_) fail("codec I/O is already configured");
        if (model_ != "MLVCEncoder" && model_ != "MLVCDecoder") fail("unsupported codec graph");
        if (cfg.slots == 0U) fail("codec slot count must be positive");
        if (!std::isfinite(cfg.pixel_range) || cfg.pixel_range <= 0.0F) fail("pixel range must be finite and positive");
        const FramePadding& pad = cfg.padding;
        if (pad.left < 0 || pad.right < 0 || pad.top < 0 || pad.bottom < 0) fail("codec frame padding must be non-negative");
        std::size_t frame_bytes = 0;
        try {
            frame_bytes = yuv420_frame_bytes(cfg.width, cfg.height);
        } catch (const std::exception& e) {
            fail(std::string("codec I/O: ") + e.what());
        }
        const int active_w = pad.rotated ? cfg.height : cfg.width;
        const int active_h = pad.rotated ? cfg.width : cfg.height;
        if (static_cast<long long>(active_w) + pad.left + pad.right != cfg.model_width ||
            static_cast<long long>(active_h) + pad.top + pad.bottom != cfg.model_height)
            fail("codec I/O padded dimensions do not match model dimensions");
        const bool encoder = model_ == "MLVCEncoder";
        const std::vector<std::int64_t> image{1, 3, cfg.model_height, cfg.model_width};
        int q = -1, img = -1;
        for (std::size_t i = 0; i < ext_in_.size(); ++i) {
            const auto& d = desc(ext_in_[i]);
            if (d.name == "q_index_shifted") {
                if (d.dtype != aot::DataType::INT32 || d.shape != std::vector<std::int64_t>{1})
                    fail("invalid q_index_shifted input");
                q = static_cast<int>(i);
            } else if (encoder && d.name == "x") {
                if (d.dtype != aot::DataType::FP16 || d.shape != image) fail("codec I/O model dimensions do not match graph");
                img = static_cast<int>(i);
            }
        }
        if (!encoder)
            for (std::size_t i = 0; i < ext_out_.size(); ++i) {
                const auto& d = desc(ext_out_[i]);
                if (d.name != "x_hat") continue;
                if (d.dtype != aot::DataType::FP16 || d.shape != image) fail("codec I/O model dimensions do not match graph");
                img = static_cast<int>(i);
                break;
            }
        if (q < 0 || img < 0) fail("missing required codec I/O tensors");

        select();
        codec_frame_ = DeviceMem(frame_bytes);
        if (encoder) {
            std::uint16_t lut[256];
            for (int v = 0; v < 256; ++v) lut[v] = float_to_half((static_cast<float>(v) / 255.0F) * cfg.pixel_range);
            codec_lut_ = DeviceMem(sizeof(lut));
            hip_check(mlvc_hip_memcpy_h2d(codec_lut_.ptr, lut, sizeof(lut), stream_), "codec LUT upload");
            hip_check(mlvc_hip_stream_synchronize(stream_), "stream sync");
        }
        std::vector<CodecSlot> slots(cfg.slots);
        for (CodecSlot& sl : slots) {
            sl.frame = HostMem(frame_bytes);
            std::memset(sl.frame.ptr, 0, frame_bytes);
            sl.q = HostMem(sizeof(std::int32_t));
            const auto& ids = encoder ? ext_out_ : ext_in_;
            sl.io.resize(ids.size());
            for (std::size_t i = 0; i < ids.size(); ++i)
                if (encoder || static_cast<int>(i) != q) {
                    sl.io[i] = HostMem(desc_bytes(desc(ids[i])));
                    std::memset(sl.io[i].ptr, 0, desc_bytes(desc(ids[i])));
                }
            hip_check(mlvc_hip_event_create(&sl.done), "event creation");
        }
        slots_ = std::move(slots);
        codec_ = cfg;
        codec_frame_bytes_ = frame_bytes;
        codec_q_ = q;
        codec_img_ = img;
        codec_encoder_ = encoder;
        codec_on_ = true;
    }

    std::size_t codec_slot_count() const noexcept { return codec_on_ ? slots_.size() : 0U; }

    MutableYuv420FrameView encoder_input_yuv(std::size_t index)
    {
        CodecSlot& sl = idle_slot(index, true, "encoder");
        return frame_view(sl);
    }

    void submit_encoder(std::size_t index, int shifted_q)
    {
        CodecSlot& sl = idle_slot(index, true, "encoder");
        if (!initialized_) fail("reset_state() must be called before submit_encoder()");
        const std::int32_t q32 = static_cast<std::int32_t>(shifted_q);
        check_gather_indices(static_cast<std::size_t>(codec_q_), &q32);
        select();
        hip_check(mlvc_hip_memcpy_h2d(codec_frame_.ptr, sl.frame.ptr, codec_frame_bytes_, stream_), "frame upload");
        const FramePadding& pad = codec_.padding;
        hip_check(mlvc_hip_yuv420_to_model(static_cast<const std::uint8_t*>(codec_frame_.ptr),
                                           static_cast<const std::uint16_t*>(codec_lut_.ptr),
                                           input_buf_.at(ext_in_[static_cast<std::size_t>(codec_img_)]).ptr, codec_.width,
                                           codec_.height, codec_.model_width, codec_.model_height, pad.rotated ? 1 : 0,
                                           stream_),
                  "frame conversion");
        enqueue_q(sl, shifted_q);
        hip_check(mlvc_hip_graph_launch(graphs_[static_cast<std::size_t>(parity_)], stream_), "graph launch");
        for (std::size_t i = 0; i < ext_out_.size(); ++i)
            hip_check(mlvc_hip_memcpy_d2h(sl.io[i].ptr, ptr(ext_out_[i], parity_), desc_bytes(desc(ext_out_[i])), stream_),
                      "output download");
        finish_submit(sl);
    }

    std::vector<TensorView> encoder_outputs(std::size_t index) const
    {
        const CodecSlot& sl = idle_slot(index, true, "encoder");
        std::vector<TensorView> v;
        for (std::size_t i = 0; i < ext_out_.size(); ++i) {
            const auto& d = desc(ext_out_[i]);
            v.push_back(TensorView::from_raw(d.name, d.shape, public_dtype(d.dtype), sl.io[i].ptr, desc_bytes(d)));
        }
        return v;
    }

    std::vector<MutableTensorView> decoder_inputs(std::size_t index)
    {
        CodecSlot& sl = idle_slot(index, false, "decoder");
        std::vector<MutableTensorView> v;
        for (std::size_t i = 0; i < ext_in_.size(); ++i) {
            if (static_cast<int>(i) == codec_q_) continue;
            const auto& d = desc(ext_in_[i]);
            v.push_back(MutableTensorView::from_raw(d.name, d.shape, public_dtype(d.dtype), sl.io[i].ptr, desc_bytes(d)));
        }
        return v;
    }

    void submit_decoder(std::size_t index, int shifted_q)
    {
        CodecSlot& sl = idle_slot(index, false, "decoder");
        if (!initialized_) fail("reset_state() must be called before submit_decoder()");
        const std::int32_t q32 = static_cast<std::int32_t>(shifted_q);
        check_gather_indices(static_cast<std::size_t>(codec_q_), &q32);
        select();
        for (std::size_t i = 0; i < ext_in_.size(); ++i) {
            if (static_cast<int>(i) == codec_q_) continue;
            hip_check(mlvc_hip_memcpy_h2d(input_buf_.at(ext_in_[i]).ptr, sl.io[i].ptr, desc_bytes(desc(ext_in_[i])), stream_),
                      "input upload");
        }
        enqueue_q(sl, shifted_q);
        hip_check(mlvc_hip_graph_launch(graphs_[static_cast<std::size_t>(parity_)], stream_), "graph launch");
        const FramePadding& pad = codec_.padding;
        hip_check(mlvc_hip_model_to_yuv420(ptr(ext_out_[static_cast<std::size_t>(codec_img_)], parity_),
                                           static_cast<std::uint8_t*>(codec_frame_.ptr), codec_.width, codec_.height,
                                           codec_.model_width, codec_.model_height, pad.left, pad.top,
                                           pad.rotated ? 1 : 0, codec_.pixel_range, stream_),
                  "frame conversion");
        hip_check(mlvc_hip_memcpy_d2h(sl.frame.ptr, codec_frame_.ptr, codec_frame_bytes_, stream_), "frame download");
        finish_submit(sl);
    }

    Yuv420FrameView decoder_output_yuv(std::size_t index) const
    {
        const CodecSlot& sl = idle_slot(index, false, "decoder");
        return frame_view(sl);
    }

    void wait_codec_slot(std::size_t index)
    {
        if (!codec_on_) fail("codec I/O is unavailable");
        if (index >= slots_.size()) fail("codec slot is out of range");
        CodecSlot& sl = slots_[index];
        if (!sl.pending) return;
        select();
        hip_check(mlvc_hip_event_synchronize(sl.done), "codec slot wait");
        sl.pending = false;
    }

    void reset_state()
    {
        select();
        for (auto& b : bindings_)
            for (auto& buf : b.buf) hip_check(mlvc_hip_zero(buf.ptr, b.bytes, stream_), "state reset");
        hip_check(mlvc_hip_stream_synchronize(stream_), "stream sync");
        parity_ = 0;
        initialized_ = true;
    }

    std::vector<Tensor> run(const std::vector<Tensor>& inputs)
    {
        if (!initialized_) fail("reset_state() must be called before run()");
        if (inputs.size() != ext_in_.size()) fail("graph input count mismatch");
        select();
        for (std::size_t i = 0; i < inputs.size(); ++i) {
            const Tensor& t = inputs[i];
            t.validate();
            const auto& d = desc(ext_in_[i]);
            if (t.shape != d.shape || t.data_type() != public_dtype(d.dtype) || t.byte_size() != desc_bytes(d))
                fail("graph input shape, dtype, or byte size mismatch");
            check_gather_indices(i, t.raw_data());
            std::memcpy(in_stage_[i].ptr, t.raw_data(), t.byte_size());
            hip_check(mlvc_hip_memcpy_h2d(input_buf_.at(ext_in_[i]).ptr, in_stage_[i].ptr, t.byte_size(), stream_), "input upload");
        }
        hip_check(mlvc_hip_graph_launch(graphs_[static_cast<std::size_t>(parity_)], stream_), "graph launch");
        enqueue_downloads();
        hip_check(mlvc_hip_stream_synchronize(stream_), "stream sync");
        std::vector<Tensor> out;
        for (std::size_t i = 0; i < ext_out_.size(); ++i) {
            const auto& d = desc(ext_out_[i]);
            Tensor t;
            t.name = d.name;
            t.shape = d.shape;
            std::vector<Float16Storage> v(elem_count(d.shape));
            std::memcpy(v.data(), out_stage_[i].ptr, v.size() * 2);
            t.data = std::move(v);
            out.push_back(std::move(t));
        }
        advance();
        return out;
    }

    void upload_inputs(const std::vector<const void*>& inputs)
    {
        if (inputs.size() != ext_in_.size()) fail("graph input count mismatch");
        for (std::size_t i = 0; i < inputs.size(); ++i) check_gather_indices(i, inputs[i]);
        select();
        for (std::size_t i = 0; i < inputs.size(); ++i)
            hip_check(mlvc_hip_memcpy_h2d(input_buf_.at(ext_in_[i]).ptr, inputs[i], desc_bytes(desc(ext_in_[i])), stream_),
                      "input upload");
        hip_check(mlvc_hip_stream_synchronize(stream_), "stream sync");
    }

    float time_frames(int frames)
    {
        if (!initialized_) fail("reset_state() must be called before running frames");
        select();
        hip_check(mlvc_hip_event_record(ev0_, stream_), "event record");
        for (int f = 0; f < frames; ++f) {
            hip_check(mlvc_hip_graph_launch(graphs_[static_cast<std::size_t>(parity_)], stream_), "graph launch");
            advance();
        }
        hip_check(mlvc_hip_event_record(ev1_, stream_), "event record");
        hip_check(mlvc_hip_event_synchronize(ev1_), "event sync");
        float ms = 0.0F;
        hip_check(mlvc_hip_event_elapsed_ms(ev0_, ev1_, &ms), "event timing");
        return ms;
    }

    // Per-frame GPU times of `frames` replays submitted back to back: events
    // are recorded just before and just after every frame. With
    // flush_bytes > 0, a device-to-device copy of flush_bytes / 2 bytes runs
    // before each frame, outside its events, so every frame starts with its
    // weights and activations evicted from L2 and the MALL (a cold frame).
    void time_frames_each(int frames, std::size_t flush_bytes, float* ms_each)
    {
        if (!initialized_) fail("reset_state() must be called before running frames");
        if (frames <= 0 || frames > 4096) fail("time_frames_each: frames must be in 1..4096");
        select();
        while (frame_evs_.size() < 2 * static_cast<std::size_t>(frames)) {
            mlvc_hip_event e = nullptr;
            hip_check(mlvc_hip_event_create(&e), "event creation");
            frame_evs_.push_back(e);
        }
        ensure_flush_buffer(flush_bytes);
        const std::size_t half = flush_bytes / 2;
        auto* fb = static_cast<std::uint8_t*>(flush_buf_);
        for (int f = 0; f < frames; ++f) {
            if (half) hip_check(mlvc_hip_memcpy_d2d(fb + half, fb, half, stream_), "cache flush copy");
            hip_check(mlvc_hip_event_record(frame_evs_[2 * f], stream_), "event record");
            hip_check(mlvc_hip_graph_launch(graphs_[static_cast<std::size_t>(parity_)], stream_), "graph launch");
            advance();
            hip_check(mlvc_hip_event_record(frame_evs_[2 * f + 1], stream_), "event record");
        }
        hip_check(mlvc_hip_event_synchronize(frame_evs_[2 * frames - 1]), "event sync");
        for (int f = 0; f < frames; ++f)
            hip_check(mlvc_hip_event_elapsed_ms(frame_evs_[2 * f], frame_evs_[2 * f + 1], &ms_each[f]), "event timing");
    }

    void download_outputs(const std::vector<std::uint16_t*>& outputs)
    {
        if (outputs.size() != ext_out_.size()) fail("graph output count mismatch");
        select();
        // Outputs of the last frame were produced with the previous parity.
        const int produced = bindings_.empty() ? 0 : parity_ ^ 1;
        for (std::size_t i = 0; i < outputs.size(); ++i)
            hip_check(mlvc_hip_memcpy_d2h(outputs[i], ptr(ext_out_[i], produced), desc_bytes(desc(ext_out_[i])), stream_),
                      "output download");
        hip_check(mlvc_hip_stream_synchronize(stream_), "stream sync");
    }

    std::size_t launch_count() const { return launches_.size(); }

    LaunchInfo launch_info(std::size_t i) const
    {
        const Launch& l = *launches_.at(i);
        return {l.name, l.kind_name, l.flops, l.bytes};
    }

    // Per-launch GPU times of `reps` single launches of kernel i, each after a
    // device-to-device copy of flush_bytes / 2 bytes (outside its events)
    // that evicts L2 and the MALL: the launch reads its inputs and weights
    // from HBM, as a launch whose producer ran long before would.
    void time_launch_cold(std::size_t i, int reps, std::size_t flush_bytes, float* ms_each)
    {
        if (reps <= 0 || reps > 4096) fail("time_launch_cold: reps must be in 1..4096");
        if (flush_bytes < 2) fail("time_launch_cold: flush_bytes must be at least 2");
        select();
        Launch& l = *launches_.at(i);
        ensure_flush_buffer(flush_bytes);
        const std::size_t half = flush_bytes / 2;
        auto* fb = static_cast<std::uint8_t*>(flush_buf_);
        enqueue_one(l, 0);
        for (int r = 0; r < reps; ++r) {
            hip_check(mlvc_hip_memcpy_d2d(fb + half, fb, half, stream_), "cache flush copy");
            hip_check(mlvc_hip_event_record(ev0_, stream_), "event record");
            enqueue_one(l, 0);
            hip_check(mlvc_hip_event_record(ev1_, stream_), "event record");
            hip_check(mlvc_hip_event_synchronize(ev1_), "event sync");
            hip_check(mlvc_hip_event_elapsed_ms(ev0_, ev1_, &ms_each[r]), "event timing");
        }
    }

    float time_launch(std::size_t i, int reps)
    {
        select();
        Launch& l = *launches_.at(i);
        enqueue_one(l, 0);
        hip_check(mlvc_hip_event_record(ev0_, stream_), "event record");
        for (int r = 0; r < reps; ++r) enqueue_one(l, 0);
        hip_check(mlvc_hip_event_record(ev1_, stream_), "event record");
        hip_check(mlvc_hip_event_synchronize(ev1_), "event sync");
        float ms = 0.0F;
        hip_check(mlvc_hip_event_elapsed_ms(ev0_, ev1_, &ms), "event timing");
        return ms / static_cast<float>(std::max(1, reps));
    }

private:
    struct Binding {
        TensorId in = 0, out = 0;
        std::size_t bytes = 0;
        DeviceMem buf[2];
    };

    const aot::TensorDescriptor& desc(TensorId id) const { return graph_.descriptor.tensors.at(id); }
    const std::vector<aot::Node>& nodes() const { return graph_.descriptor.nodes; }
    bool is_weight(TensorId id) const { return std::holds_alternative<aot::WeightLocation>(desc(id).storage); }

    void select() { hip_check(mlvc_hip_set_device(device_), "set device"); }

    void advance()
    {
        if (!bindings_.empty()) parity_ ^= 1;
    }

    void bind_state(const ModelExecutionConfig& config)
    {
        const auto& g = graph_.descriptor;
        std::set<TensorId> seen_in, seen_out;
        for (const StateTensorBinding& b : config.state_bindings) {
            if (b.input_index >= g.inputs.size() || b.output_index >= g.outputs.size())
                fail("state binding index out of range");
            const TensorId in = g.inputs[b.input_index], out = g.outputs[b.output_index];
            if (!seen_in.insert(in).second || !seen_out.insert(out).second) fail("duplicate state tensor binding");
            if (desc(in).dtype != desc(out).dtype || desc(in).shape != desc(out).shape ||
                desc(in).dtype != aot::DataType::FP16 || b.data_type != TensorDataType::kFloat16 || b.shape != desc(in).shape)
                fail("state binding shape or dtype mismatch");
            Binding nb;
            nb.in = in;
            nb.out = out;
            nb.bytes = desc_bytes(desc(in));
            bindings_.push_back(std::move(nb));
            state_in_[in] = bindings_.size() - 1;
            state_out_[out] = bindings_.size() - 1;
        }
        // FP16 activations, plus INT32 control inputs such as q_index_shifted
        // (read only as GATHER indices; any other operator reading one is
        // rejected when the graph is lowered).
        for (TensorId id : g.inputs) {
            const auto dt = desc(id).dtype;
            if (dt != aot::DataType::FP16 && !(dt == aot::DataType::INT32 && !state_in_.count(id)))
                fail("only FP16 activations and INT32 control inputs are on this path");
            if (!state_in_.count(id)) ext_in_.push_back(id);
        }
        for (TensorId id : g.outputs) {
            if (desc(id).dtype != aot::DataType::FP16) fail("only FP16 graph outputs are on this path");
            if (!state_out_.count(id)) ext_out_.push_back(id);
        }
    }

    // ------------------------------------- real-model pattern matching
    // The reference CPU matcher's patterns (fusion_matcher.cpp:78-850): a
    // matched chain becomes one kernel that writes every tensor of the chain
    // that is read outside it. The matcher's consumer-count and shape rules
    // are kept, so exactly the chains it fuses are fused here.
    bool graph_output(TensorId id) const
    {
        const auto& o = graph_.descriptor.outputs;
        return std::find(o.begin(), o.end(), id) != o.end();
    }
    bool internal_only(TensorId id, int n) const
    {
        const auto it = consumers_.find(id);
        return id && !graph_output(id) && (it == consumers_.end() ? 0 : it->second) == n;
    }
    bool named(TensorId id) const
    {
        return id && id < graph_.descriptor.tensors.size() && !desc(id).name.empty();
    }
    std::vector<std::uint8_t> weight_bytes(TensorId id) const
    {
        const auto& w = std::get<aot::WeightLocation>(desc(id).storage);
        const auto* p = reinterpret_cast<const std::uint8_t*>(graph_.weights.data()) + w.offset;
        return std::vector<std::uint8_t>(p, p + w.bytes);
    }
    bool int64_init(TensorId id, std::vector<std::int64_t>& v) const
    {
        if (!named(id) || !is_weight(id) || desc(id).dtype != aot::DataType::INT64) return false;
        const auto raw = weight_bytes(id);
        if (raw.size() % 8) return false;
        v.resize(raw.size() / 8);
        if (!raw.empty()) std::memcpy(v.data(), raw.data(), raw.size());
        return true;
    }
    bool fp16_scalar_init(TensorId id, float& v) const
    {
        if (!named(id) || !is_weight(id) || desc(id).dtype != aot::DataType::FP16) return false;
        const auto raw = weight_bytes(id);
        if (raw.size() != 2) return false;
        std::uint16_t h;
        std::memcpy(&h, raw.data(), 2);
        v = half_to_float(h);
        return true;
    }
    static int axis_of(const aot::Node& n)
    {
        const auto* a = std::get_if<aot::AxisAttributes>(&n.attributes);
        return a ? a->axis : 0;
    }
    bool clip_constants(const aot::Node& n, float& lo, float& hi) const
    {
        if (n.op != Op::CLIP || n.inputs.size() < 2 || n.outputs.size() != 1) return false;
        lo = -HUGE_VALF;
        hi = HUGE_VALF;
        if (n.inputs[1] && !fp16_scalar_init(n.inputs[1], lo)) return false;
        if (n.inputs.size() >= 3 && n.inputs[2] && !fp16_scalar_init(n.inputs[2], hi)) return false;
        return true;
    }
    bool channel_slice(const aot::Node& n, TensorId x, std::int64_t b, std::int64_t e) const
    {
        if (n.op != Op::SLICE || n.inputs.size() < 3 || n.outputs.size() != 1 || n.inputs[0] != x) return false;
        std::vector<std::int64_t> st, en, ax, sp;
        if (!int64_init(n.inputs[1], st) || !int64_init(n.inputs[2], en) || st.size() != 1 || en.size() != 1 || st[0] != b ||
            en[0] != e)
            return false;
        if (n.inputs.size() < 4 || !n.inputs[3] || !int64_init(n.inputs[3], ax) || ax.size() != 1 || ax[0] != 1) return false;
        if (n.inputs.size() >= 5 && n.inputs[4] && (!int64_init(n.inputs[4], sp) || sp.size() != 1 || sp[0] != 1)) return false;
        const auto& o = desc(n.outputs[0]);
        return o.dtype == aot::DataType::FP16 && o.shape.size() == 4 && o.shape[1] == e - b;
    }
    static bool pair(const aot::Node& n, Op op, TensorId x, TensorId y)
    {
        return n.op == op && n.inputs.size() == 2 && n.outputs.size() == 1 &&
               ((n.inputs[0] == x && n.inputs[1] == y) || (n.inputs[0] == y && n.inputs[1] == x));
    }
    static bool other_in_pair(const aot::Node& n, Op op, TensorId x, TensorId& other)
    {
        if (n.op != op || n.inputs.size() != 2 || n.outputs.size() != 1) return false;
        if (n.inputs[0] == x) { other = n.inputs[1]; return true; }
        if (n.inputs[1] == x) { other = n.inputs[0]; return true; }
        return false;
    }
    bool fp16_of(TensorId id, const std::vector<std::int64_t>& shape) const
    {
        return named(id) && desc(id).dtype == aot::DataType::FP16 && desc(id).shape == shape;
    }
    bool fp16_4d(TensorId id) const { return named(id) && desc(id).dtype == aot::DataType::FP16 && desc(id).shape.size() == 4; }

    // try_reglu (fusion_matcher.cpp:304-346): SLICE [0,G) / [G,2G) of x ->
    // CLIP(gate) -> MUL(clipped, linear). A 1x1 conv producing x is lowered on
    // its own, so this also covers try_pointwise_reglu (:258-302).
    bool match_reglu(std::size_t i, Launch& L, std::vector<bool>& done)
    {
        const auto& ns = nodes();
        if (i + 4 > ns.size() || ns[i].op != Op::SLICE || ns[i].inputs.empty()) return false;
        const TensorId x = ns[i].inputs[0];
        if (!fp16_4d(x) || desc(x).shape[1] <= 0 || desc(x).shape[1] % 2) return false;
        const std::int64_t g = desc(x).shape[1] / 2;
        if (!channel_slice(ns[i], x, 0, g) || !channel_slice(ns[i + 1], x, g, 2 * g)) return false;
        const TensorId gate = ns[i].outputs[0], lin = ns[i + 1].outputs[0];
        if (!internal_only(gate, 1) || !internal_only(lin, 1)) return false;
        float lo, hi;
        if (!clip_constants(ns[i + 2], lo, hi) || ns[i + 2].inputs[0] != gate) return false;
        const TensorId clipped = ns[i + 2].outputs[0];
        if (!internal_only(clipped, 1) || !pair(ns[i + 3], Op::MUL, clipped, lin)) return false;
        const auto& s = desc(x).shape;
        if (desc(ns[i + 3].outputs[0]).shape != std::vector<std::int64_t>{s[0], g, s[2], s[3]}) return false;
        L.kind = Launch::kReglu;
        L.kind_name = "reglu";
        L.x = x;
        L.y = ns[i + 3].outputs[0];
        L.n = static_cast<int>(s[0]);
        L.c = static_cast<int>(g);
        L.hw = static_cast<std::size_t>(s[2] * s[3]);
        L.lo = lo;
        L.hi = hi;
        L.bytes = 2.0 * static_cast<double>(elem_count(s)) * 1.5;
        for (std::size_t k = i; k < i + 4; ++k) done[k] = true;
        return true;
    }

    // try_feature_update (fusion_matcher.cpp:413-541).
    bool match_feature(std::size_t i, Launch& L, std::vector<bool>& done)
    {
        const auto& ns = nodes();
        if (i + 11 > ns.size() || ns[i].op != Op::SLICE || ns[i].inputs.empty()) return false;
        const TensorId x = ns[i].inputs[0];
        if (!fp16_4d(x) || desc(x).shape[1] <= 0 || desc(x).shape[1] % 3) return false;
        const std::int64_t ch = desc(x).shape[1] / 3;
        if (!channel_slice(ns[i], x, 0, ch) || !channel_slice(ns[i + 1], x, ch, 2 * ch) || !channel_slice(ns[i + 2], x, 2 * ch, 3 * ch))
            return false;
        const TensorId a = ns[i].outputs[0], b = ns[i + 1].outputs[0], cg = ns[i + 2].outputs[0];
        if (!internal_only(a, 1) || !internal_only(b, 1) || !internal_only(cg, 1)) return false;
        const aot::Node& s0 = ns[i + 3];
        const aot::Node& s1 = ns[i + 4];
        if (s0.op != Op::SIGMOID || s0.inputs.size() != 1 || s0.inputs[0] != b || s0.outputs.size() != 1 || s1.op != Op::SIGMOID ||
            s1.inputs.size() != 1 || s1.inputs[0] != cg || s1.outputs.size() != 1)
            return false;
        const TensorId sb = s0.outputs[0], sc = s1.outputs[0];
        if (!internal_only(sb, 2) || !internal_only(sc, 1)) return false;
        TensorId hist = 0;
        if (!other_in_pair(ns[i + 5], Op::MUL, sb, hist) || !named(hist) || is_weight(hist) || !fp16_of(hist, desc(a).shape)) return false;
        const TensorId wb = ns[i + 5].outputs[0];
        if (!internal_only(wb, 1)) return false;
        const aot::Node& sub = ns[i + 6];
        if (sub.op != Op::SUB || sub.inputs.size() != 2 || sub.outputs.size() != 1 || sub.inputs[1] != sb) return false;
        float one = 0.0F;
        if (!fp16_scalar_init(sub.inputs[0], one) || std::fabs(one - 1.0F) > 1e-4F) return false;
        const TensorId inv = sub.outputs[0];
        if (!internal_only(inv, 1) || !pair(ns[i + 7], Op::MUL, inv, a)) return false;
        const TensorId wa = ns[i + 7].outputs[0];
        if (!internal_only(wa, 1) || !pair(ns[i + 8], Op::ADD, wb, wa)) return false;
        const TensorId blended = ns[i + 8].outputs[0];
        if (!pair(ns[i + 9], Op::MUL, sc, blended)) return false;
        const TensorId gated = ns[i + 9].outputs[0];
        if (!internal_only(gated, 1)) return false;
        TensorId scale = 0;
        if (!other_in_pair(ns[i + 10], Op::MUL, gated, scale) || !fp16_of(scale, {1, ch, 1, 1})) return false;
        const TensorId scaled = ns[i + 10].outputs[0];
        auto concat_of = [&](const aot::Node& c) {
            return c.op == Op::CONCAT && axis_of(c) == 1 && c.inputs.size() == 2 && c.inputs[0] == scaled && c.inputs[1] == blended &&
                   c.outputs.size() == 1;
        };
        std::size_t cat = 0, end = 0;
        if (i + 12 <= ns.size() && internal_only(scaled, 1) && internal_only(blended, 2) && concat_of(ns[i + 11])) {
            cat = i + 11;
            end = i + 12;
        } else if (!graph_output(scaled) && internal_only(blended, 2)) {
            for (std::size_t j = i + 11; j < ns.size() && !cat; ++j)
                if (concat_of(ns[j])) cat = j;
            end = i + 11;
            if (cat) {
                L.outs = {scaled, blended};
            }
        }
        if (!cat) return false;
        const auto& s = desc(x).shape;
        const std::vector<std::int64_t> cs{s[0], ch, s[2], s[3]}, fs{s[0], 2 * ch, s[2], s[3]};
        if (desc(ns[cat].outputs[0]).shape != fs || desc(scaled).shape != cs || desc(blended).shape != cs) return false;
        L.kind = Launch::kFeature;
        L.kind_name = L.outs.empty() ? "feature_update" : "feature_update_outputs";
        L.x = x;
        L.ins = {hist, scale};
        L.y = ns[cat].outputs[0];
        L.n = static_cast<int>(s[0]);
        L.c = static_cast<int>(ch);
        L.hw = static_cast<std::size_t>(s[2] * s[3]);
        const double plane = 2.0 * static_cast<double>(s[0] * s[2] * s[3]);
        L.bytes = plane * static_cast<double>(ch) * (3 + 1 + 2 + (L.outs.empty() ? 0 : 2));
        for (std::size_t k = i; k < end; ++k) done[k] = true;
        done[cat] = true;
        return true;
    }

    // The update shared by both quantisation tails (fusion_matcher.cpp:
    // 620-697, 760-836), from node k with `scaled` matched.
    std::size_t match_update(std::size_t k, TensorId scaled, TensorId tail, std::int64_t q, const std::vector<std::int64_t>& qshape,
                             TensorId& y_raw, TensorId& u0, TensorId& u1, TensorId& us0, TensorId& us1) const
    {
        const auto& ns = nodes();
        if (!channel_slice(ns[k], scaled, 0, q) || !channel_slice(ns[k + 1], scaled, q, 2 * q)) return 0;
        const TensorId h0 = ns[k].outputs[0], h1 = ns[k + 1].outputs[0];
        if (!internal_only(h0, 1) || !internal_only(h1, 1) || !pair(ns[k + 2], Op::ADD, h0, h1)) return 0;
        const TensorId sum = ns[k + 2].outputs[0];
        if (!internal_only(sum, 1)) return 0;
        const aot::Node& rnd = ns[k + 3];
        if (rnd.op != Op::ROUND || rnd.inputs.size() != 1 || rnd.inputs[0] != sum || rnd.outputs.size() != 1) return 0;
        y_raw = rnd.outputs[0];
        if (!channel_slice(ns[k + 4], tail, 0, q) || !channel_slice(ns[k + 5], tail, q, 2 * q)) return 0;
        const TensorId t0 = ns[k + 4].outputs[0], t1 = ns[k + 5].outputs[0];
        if (!internal_only(t0, 1) || !internal_only(t1, 1) || !pair(ns[k + 6], Op::ADD, y_raw, t0)) return 0;
        const TensorId a0 = ns[k + 6].outputs[0];
        if (!internal_only(a0, 1) || !other_in_pair(ns[k + 7], Op::MUL, a0, us0) || !fp16_of(us0, qshape)) return 0;
        u0 = ns[k + 7].outputs[0];
        if (!internal_only(u0, 1) || !pair(ns[k + 8], Op::ADD, y_raw, t1)) return 0;
        const TensorId a1 = ns[k + 8].outputs[0];
        if (!internal_only(a1, 1) || !other_in_pair(ns[k + 9], Op::MUL, a1, us1) || !fp16_of(us1, qshape)) return 0;
        u1 = ns[k + 9].outputs[0];
        if (!internal_only(u1, 1)) return 0;
        return k + 10;
    }

    // try_y0_tail (fusion_matcher.cpp:543-696).
    bool match_y0(std::size_t i, Launch& L, std::vector<bool>& done)
    {
        const auto& ns = nodes();
        if (i + 19 > ns.size() || ns[i].op != Op::SLICE || ns[i].inputs.empty()) return false;
        const TensorId prior = ns[i].inputs[0];
        if (!fp16_4d(prior) || desc(prior).shape[1] <= 0 || desc(prior).shape[1] % 4) return false;
        const auto& ps = desc(prior).shape;
        const std::int64_t q = ps[1] / 4;
        if (!channel_slice(ns[i], prior, 0, 2 * q) || !channel_slice(ns[i + 1], prior, 2 * q, 4 * q)) return false;
        const TensorId head = ns[i].outputs[0], tail = ns[i + 1].outputs[0];
        if (!internal_only(head, 1) || !internal_only(tail, 3)) return false;
        float lo, hi;
        if (!clip_constants(ns[i + 2], lo, hi) || ns[i + 2].inputs[0] != head || hi < 65504.0F) return false;
        const TensorId clipped = ns[i + 2].outputs[0];
        if (graph_output(clipped)) return false;
        const aot::Node& rec = ns[i + 3];
        if (rec.op != Op::RECIPROCAL || rec.inputs.size() != 1 || rec.inputs[0] != clipped || rec.outputs.size() != 1) return false;
        TensorId inv = rec.outputs[0];
        if (!internal_only(inv, 1)) return false;
        std::size_t k = i + 4;
        if (k + 15 <= ns.size() && ns[k].op == Op::MUL && ns[k].inputs.size() == 2 && ns[k].outputs.size() == 1) {
            TensorId other = 0;
            float one = 0.0F;
            if (other_in_pair(ns[k], Op::MUL, inv, other) && fp16_scalar_init(other, one) && std::fabs(one - 1.0F) <= 1e-4F) {
                inv = ns[k].outputs[0];
                if (!internal_only(inv, 1)) return false;
                ++k;
            }
        }
        if (k + 15 > ns.size()) return false;
        const std::vector<std::int64_t> nshape{ps[0], 2 * q, ps[2], ps[3]}, qshape{ps[0], q, ps[2], ps[3]};
        TensorId latent = 0;
        if (!other_in_pair(ns[k], Op::MUL, inv, latent) || !named(latent) || is_weight(latent) || !fp16_of(latent, nshape)) return false;
        const TensorId normalized = ns[k].outputs[0];
        const aot::Node& sub = ns[k + 1];
        if (sub.op != Op::SUB || sub.inputs.size() != 2 || sub.outputs.size() != 1 || sub.inputs[0] != normalized || sub.inputs[1] != tail)
            return false;
        const TensorId diff = sub.outputs[0];
        TensorId qs = 0;
        if (!internal_only(diff, 1) || !other_in_pair(ns[k + 2], Op::MUL, diff, qs) || !fp16_of(qs, nshape)) return false;
        const TensorId scaled = ns[k + 2].outputs[0];
        if (!internal_only(scaled, 2)) return false;
        TensorId y_raw, u0, u1, us0, us1;
        const std::size_t e = match_update(k + 3, scaled, tail, q, qshape, y_raw, u0, u1, us0, us1);
        if (!e) return false;
        const aot::Node& c2 = ns[e];
        const aot::Node& c3 = ns[e + 1];
        if (c2.op != Op::CONCAT || axis_of(c2) != 1 || c2.inputs.size() != 2 || c2.inputs[0] != u0 || c2.inputs[1] != u1 ||
            c2.outputs.size() != 1)
            return false;
        const TensorId concat2 = c2.outputs[0];
        if (c3.op != Op::CONCAT || axis_of(c3) != 1 || c3.inputs.size() != 2 || c3.inputs[0] != concat2 || c3.inputs[1] != prior ||
            c3.outputs.size() != 1)
            return false;
        const std::vector<std::int64_t> c6{ps[0], 6 * q, ps[2], ps[3]};
        if (desc(normalized).shape != nshape || desc(clipped).shape != nshape || desc(y_raw).shape != qshape ||
            desc(concat2).shape != nshape || desc(c3.outputs[0]).shape != c6)
            return false;
        L.kind = Launch::kY0;
        L.kind_name = "y0_tail";
        L.ins = {latent, prior, qs, us0, us1};
        L.outs = {normalized, clipped, y_raw, concat2};
        L.y = c3.outputs[0];
        L.n = static_cast<int>(ps[0]);
        L.c = static_cast<int>(q);
        L.hw = static_cast<std::size_t>(ps[2] * ps[3]);
        L.lo = lo;
        L.bytes = 2.0 * static_cast<double>(ps[0] * ps[2] * ps[3]) * static_cast<double>(q) * (10 + 13);
        for (std::size_t n = i; n < e + 2; ++n) done[n] = true;
        return true;
    }

    // try_y1_tail (fusion_matcher.cpp:698-850).
    bool match_y1(std::size_t i, Launch& L, std::vector<bool>& done)
    {
        const auto& ns = nodes();
        if (i + 15 > ns.size()) return false;
        const aot::Node& sub = ns[i];
        if (sub.op != Op::SUB || sub.inputs.size() != 2 || sub.outputs.size() != 1) return false;
        const TensorId normalized = sub.inputs[0], prior = sub.inputs[1];
        if (!fp16_4d(normalized) || !fp16_4d(prior) || desc(normalized).shape != desc(prior).shape) return false;
        const auto& ns_shape = desc(normalized).shape;
        if (ns_shape[1] <= 0 || ns_shape[1] % 2) return false;
        const std::int64_t q = ns_shape[1] / 2;
        const std::vector<std::int64_t> qshape{ns_shape[0], q, ns_shape[2], ns_shape[3]};
        const TensorId diff = sub.outputs[0];
        TensorId qs = 0;
        if (!internal_only(diff, 1) || !other_in_pair(ns[i + 1], Op::MUL, diff, qs) || !fp16_of(qs, ns_shape)) return false;
        const TensorId scaled = ns[i + 1].outputs[0];
        if (!internal_only(scaled, 2)) return false;
        TensorId y_raw, u0, u1, us0, us1;
        const std::size_t e = match_update(i + 2, scaled, prior, q, qshape, y_raw, u0, u1, us0, us1);
        if (!e) return false;
        const aot::Node& c2 = ns[e];
        if (c2.op != Op::CONCAT || axis_of(c2) != 1 || c2.inputs.size() != 2 || c2.inputs[0] != u0 || c2.inputs[1] != u1 ||
            c2.outputs.size() != 1)
            return false;
        const TensorId cat = c2.outputs[0];
        TensorId concat2 = 0, clipped = 0;
        if (!internal_only(cat, 1) || !other_in_pair(ns[e + 1], Op::ADD, cat, concat2) || !named(concat2) || is_weight(concat2) ||
            !fp16_of(concat2, ns_shape))
            return false;
        const TensorId added = ns[e + 1].outputs[0];
        if (!internal_only(added, 1) || !other_in_pair(ns[e + 2], Op::MUL, added, clipped) || !named(clipped) || is_weight(clipped) ||
            !fp16_of(clipped, ns_shape))
            return false;
        if (desc(y_raw).shape != qshape || desc(ns[e + 2].outputs[0]).shape != ns_shape) return false;
        L.kind = Launch::kY1;
        L.kind_name = "y1_tail";
        L.ins = {normalized, prior, qs, us0, us1, concat2, clipped};
        L.outs = {y_raw};
        L.y = ns[e + 2].outputs[0];
        L.n = static_cast<int>(ns_shape[0]);
        L.c = static_cast<int>(q);
        L.hw = static_cast<std::size_t>(ns_shape[2] * ns_shape[3]);
        L.bytes = 2.0 * static_cast<double>(ns_shape[0] * ns_shape[2] * ns_shape[3]) * static_cast<double>(q) * (12 + 3);
        for (std::size_t n = i; n < e + 3; ++n) done[n] = true;
        return true;
    }

    // ------------------------------------------------- single operators
    // FP16 operand of an elementwise / layout operator: an activation or an
    // FP16 initializer (uploaded once as a constant buffer).
    void fp16_operand(TensorId id)
    {
        if (!named(id) || desc(id).dtype != aot::DataType::FP16) fail("operand must be an FP16 tensor");
        if (is_weight(id) && !const_buf_.count(id)) {
            auto raw = weight_bytes(id);
            DeviceMem m(std::max<std::size_t>(raw.size(), 16));
            pending_uploads_.push_back({m.ptr, std::move(raw)});
            const_buf_.emplace(id, std::move(m));
        }
    }

    static void dims4(const std::vector<std::int64_t>& s, std::int64_t (&d)[4])
    {
        if (s.size() > 4) fail("tensors of rank above 4 are not supported");
        for (int k = 0; k < 4; ++k) d[k] = 1;
        for (std::size_t k = 0; k < s.size(); ++k) d[4 - s.size() + k] = s[k];
    }

    void lower_unary(Launch& L, const aot::Node& n)
    {
        fp16_operand(n.inputs.at(0));
        if (desc(n.inputs[0]).shape != desc(n.outputs[0]).shape) fail("unary operator output shape differs from its input");
        L.kind = Launch::kUnary;
        L.x = n.inputs[0];
        L.y = n.outputs[0];
        L.count = elem_count(desc(L.y).shape);
        L.lo = 0.0F;
        L.hi = 0.0F;
        switch (n.op) {
        case Op::CLIP:
            // execution_plan.cpp:512-520: absent bounds are -inf / +inf.
            L.op = MLVC_UNARY_CLIP;
            L.kind_name = "clip";
            L.lo = -HUGE_VALF;
            L.hi = HUGE_VALF;
            if (n.inputs.size() > 1 && n.inputs[1] && !fp16_scalar_init(n.inputs[1], L.lo)) fail("expected scalar FP16 initializer");
            if (n.inputs.size() > 2 && n.inputs[2] && !fp16_scalar_init(n.inputs[2], L.hi)) fail("expected scalar FP16 initializer");
            break;
        case Op::SIGMOID: L.op = MLVC_UNARY_SIGMOID; L.kind_name = "sigmoid"; break;
        case Op::RECIPROCAL: L.op = MLVC_UNARY_RECIPROCAL; L.kind_name = "reciprocal"; break;
        default: L.op = MLVC_UNARY_ROUND; L.kind_name = "round"; break;
        }
        L.bytes = 4.0 * static_cast<double>(L.count);
    }

    // ADD / SUB / MUL with numpy broadcasting (execution_plan.cpp:527-563,
    // 958-985). Outputs of rank other than 4 are indexed flat modulo the
    // operand size there, which is numpy broadcasting only when each operand
    // shape is a suffix of the output's; other such graphs are rejected.
    void lower_binary(Launch& L, const aot::Node& n)
    {
        const TensorId a = n.inputs.at(0), b = n.inputs.at(1), y = n.outputs[0];
        fp16_operand(a);
        fp16_operand(b);
        const auto& as = desc(a).shape;
        const auto& bs = desc(b).shape;
        const auto& ys = desc(y).shape;
        const std::size_t r = std::max(as.size(), bs.size());
        std::vector<std::int64_t> want(r, 1);
        for (std::size_t i = 0; i < r; ++i) {
            const std::int64_t u = i + as.size() >= r ? as[i + as.size() - r] : 1;
            const std::int64_t v = i + bs.size() >= r ? bs[i + bs.size() - r] : 1;
            if (u != v && u != 1 && v != 1) fail("binary operand shapes do not broadcast");
            want[i] = std::max(u, v);
        }
        if (want != ys) fail("binary output shape is not the broadcast of its operands");
        auto suffix_or_scalar = [&](const std::vector<std::int64_t>& s) {
            if (elem_count(s) == 1) return true;
            std::vector<std::int64_t> t = s;
            while (!t.empty() && t.front() == 1) t.erase(t.begin());
            return t.size() <= ys.size() && std::equal(t.rbegin(), t.rend(), ys.rbegin());
        };
        if (ys.size() != 4 && !(suffix_or_scalar(as) && suffix_or_scalar(bs)))
            fail("broadcast of a non-4-D output with a non-trailing operand is not supported");
        // A rank < 4 operand of a 4-D output is indexed as NHWC there; that
        // equals NCHW broadcasting only when its padded shape has a single
        // channel or a single pixel.
        for (const auto* s : {&as, &bs})
            if (ys.size() == 4 && s->size() < 4 && elem_count(*s) > 1) {
                std::int64_t d[4];
                dims4(*s, d);
                if (d[1] > 1 && d[2] * d[3] > 1) fail("broadcast operand of rank < 4 with channels and pixels is not supported");
            }
        L.kind = n.op == Op::ADD && as == ys && bs == ys ? Launch::kAdd : Launch::kBinary;
        L.op = n.op == Op::SUB ? MLVC_BINARY_SUB : n.op == Op::MUL ? MLVC_BINARY_MUL : MLVC_BINARY_ADD;
        L.kind_name = n.op == Op::SUB ? "sub" : n.op == Op::MUL ? "mul" : "add";
        L.x = a;
        L.x2 = b;
        L.y = y;
        L.count = elem_count(ys);
        dims4(as, L.da);
        dims4(bs, L.db);
        dims4(ys, L.dy);
        L.bytes = 2.0 * static_cast<double>(elem_count(as) + elem_count(bs) + elem_count(ys));
    }

    // SLICE (execution_plan.cpp:565-604): INT64 starts / ends / axes / steps
    // initializers; negative starts count from the end and are clamped to
    // [0, dim]; the output shape gives the extent.
    void lower_slice(Launch& L, const aot::Node& n)
    {
        const TensorId x = n.inputs.at(0), y = n.outputs[0];
        fp16_operand(x);
        const auto& xs = desc(x).shape;
        const auto& ys = desc(y).shape;
        if (xs.size() != 4 || ys.size() != 4) fail("expected 4D NCHW tensor");
        std::vector<std::int64_t> st, en, ax, sp;
        if (n.inputs.size() < 3 || !int64_init(n.inputs[1], st) || !int64_init(n.inputs[2], en))
            fail("SLICE starts and ends must be INT64 initializers");
        if (n.inputs.size() > 3 && n.inputs[3]) {
            if (!int64_init(n.inputs[3], ax)) fail("SLICE axes must be an INT64 initializer");
        } else {
            for (std::size_t a = 0; a < st.size(); ++a) ax.push_back(static_cast<std::int64_t>(a));
        }
        sp.assign(st.size(), 1);
        if (n.inputs.size() > 4 && n.inputs[4] && !int64_init(n.inputs[4], sp)) fail("SLICE steps must be an INT64 initializer");
        if (ax.size() < st.size() || sp.size() < st.size()) fail("SLICE parameter lengths differ");
        for (int k = 0; k < 4; ++k) {
            L.starts[k] = 0;
            L.steps[k] = 1;
            L.da[k] = xs[static_cast<std::size_t>(k)];
            L.dy[k] = ys[static_cast<std::size_t>(k)];
        }
        for (std::size_t a = 0; a < st.size(); ++a) {
            std::int64_t k = ax[a];
            if (k < 0) k += 4;
            if (k < 0 || k >= 4) fail("SLICE axis out of range");
            const std::int64_t dim = xs[static_cast<std::size_t>(k)];
            std::int64_t v = st[a];
            if (v < 0) v += dim;
            L.starts[k] = std::clamp<std::int64_t>(v, 0, dim);
            L.steps[k] = sp[a];
        }
        for (int k = 0; k < 4; ++k) {
            const std::int64_t last = L.starts[k] + (L.dy[k] - 1) * L.steps[k];
            if (L.steps[k] == 0 || L.starts[k] >= L.da[k] || last < 0 || last >= L.da[k]) fail("SLICE reads outside its input");
        }
        L.kind = Launch::kSlice;
        L.kind_name = "slice";
        L.x = x;
        L.y = y;
        L.bytes = 4.0 * static_cast<double>(elem_count(ys));
    }

    // CONCAT of 4-D tensors along any axis (execution_plan.cpp:606-620):
    // every input is one block copy into its place in the output.
    void lower_concat(Launch& L, const aot::Node& n)
    {
        const TensorId y = n.outputs[0];
        const auto& ys = desc(y).shape;
        if (ys.size() != 4) fail("expected 4D NCHW tensor");
        int axis = axis_of(n);
        if (axis < 0) axis += 4;
        if (axis < 0 || axis >= 4) fail("CONCAT axis out of range");
        std::size_t after = 1;
        for (int k = axis + 1; k < 4; ++k) after *= static_cast<std::size_t>(ys[static_cast<std::size_t>(k)]);
        std::size_t rows = 1;
        for (int k = 0; k < axis; ++k) rows *= static_cast<std::size_t>(ys[static_cast<std::size_t>(k)]);
        std::int64_t off = 0;
        for (TensorId id : n.inputs) {
            fp16_operand(id);
            const auto& s = desc(id).shape;
            if (s.size() != 4) fail("expected 4D NCHW tensor");
            for (int k = 0; k < 4; ++k)
                if (k != axis && s[static_cast<std::size_t>(k)] != ys[static_cast<std::size_t>(k)]) fail("CONCAT input shape mismatch");
            const std::size_t along = static_cast<std::size_t>(s[static_cast<std::size_t>(axis)]);
            L.ins.push_back(id);
            L.pieces.push_back({rows, along * after, static_cast<std::size_t>(off) * after,
                                static_cast<std::size_t>(ys[static_cast<std::size_t>(axis)]) * after});
            off += s[static_cast<std::size_t>(axis)];
        }
        if (off != ys[static_cast<std::size_t>(axis)]) fail("CONCAT output shape mismatch");
        L.kind = Launch::kConcatAny;
        L.kind_name = "concat";
        L.y = y;
        L.bytes = 4.0 * static_cast<double>(elem_count(ys));
    }

    // GATHER (execution_plan.cpp:1004-1012, 101-168): FP16 data, INT64
    // initializer indices or INT32 graph-input indices (q_index_shifted);
    // out = take(data, indices, axis). Initializer indices are range-checked
    // here, graph-input indices on every upload.
    void lower_gather(Launch& L, const aot::Node& n)
    {
        const TensorId d = n.inputs.at(0), ix = n.inputs.at(1), y = n.outputs[0];
        fp16_operand(d);
        const auto& ds = desc(d).shape;
        const int rank = static_cast<int>(ds.size());
        int axis = axis_of(n);
        if (axis < 0) axis += rank;
        if (axis < 0 || axis >= rank) fail("GATHER axis out of range");
        // The reference indexes 4-D data in its NHWC order; the result is
        // take() on the logical array when the output keeps rank 4 or the data
        // is one pixel per row (its [72, C, 1, 1] table case).
        const auto& is = desc(ix).shape;
        const bool pixel_rows = axis == 0 && (rank != 4 || (ds[2] == 1 && ds[3] == 1));
        if (rank == 4 && !pixel_rows && is.size() != 1) fail("GATHER of 4-D data with indices of rank other than 1 is not supported");
        L.outer = 1;
        L.inner = 1;
        for (int k = 0; k < axis; ++k) L.outer *= static_cast<std::size_t>(ds[static_cast<std::size_t>(k)]);
        for (int k = axis + 1; k < rank; ++k) L.inner *= static_cast<std::size_t>(ds[static_cast<std::size_t>(k)]);
        L.dim = static_cast<std::size_t>(ds[static_cast<std::size_t>(axis)]);
        L.count = elem_count(is);
        if (L.count == 0 || elem_count(desc(y).shape) != L.outer * L.count * L.inner) fail("GATHER output size mismatch");
        if (is_weight(ix)) {
            std::vector<std::int64_t> v;
            if (!int64_init(ix, v)) fail("GATHER indices must be INT64 initializers or INT32 graph inputs");
            for (std::int64_t i : v)
                if ((i < 0 ? i + static_cast<std::int64_t>(L.dim) : i) < 0 || (i < 0 ? i + static_cast<std::int64_t>(L.dim) : i) >=
                                                                                   static_cast<std::int64_t>(L.dim))
                    fail("GATHER index out of range");
            // Several GATHERs may share one index initializer: upload it once.
            if (!const_buf_.count(ix)) {
                auto raw = weight_bytes(ix);
                DeviceMem m(raw.size());
                pending_uploads_.push_back({m.ptr, std::move(raw)});
                const_buf_.emplace(ix, std::move(m));
            }
            L.idx64 = true;
        } else {
            const auto& g = graph_.descriptor.inputs;
            const auto it = std::find(ext_in_.begin(), ext_in_.end(), ix);
            if (desc(ix).dtype != aot::DataType::INT32 || it == ext_in_.end() || std::find(g.begin(), g.end(), ix) == g.end())
                fail("GATHER indices must be INT64 initializers or INT32 graph inputs");
            gather_checks_.push_back({static_cast<std::size_t>(it - ext_in_.begin()), L.dim});
            L.idx64 = false;
        }
        L.kind = Launch::kGather;
        L.kind_name = "gather";
        L.x = d;
        L.x2 = ix;
        L.y = y;
        L.bytes = 4.0 * static_cast<double>(elem_count(desc(y).shape));
    }

    // Host check of graph-input GATHER indices (the reference throws
    // "GATHER index out of range" while executing).
    void check_gather_indices(std::size_t ext_pos, const void* data) const
    {
        for (const auto& [pos, dim] : gather_checks_) {
            if (pos != ext_pos) continue;
            const std::size_t n = elem_count(desc(ext_in_[pos]).shape);
            const auto* v = static_cast<const std::int32_t*>(data);
            for (std::size_t i = 0; i < n; ++i) {
                const std::int64_t k = v[i] < 0 ? static_cast<std::int64_t>(v[i]) + static_cast<std::int64_t>(dim) : v[i];
                if (k < 0 || k >= static_cast<std::int64_t>(dim)) fail("GATHER index out of range");
            }
        }
    }

    // ---------------------------------------------------------- lowering
    void lower()
    {
        const auto& g = graph_.descriptor;
        const auto& ns = nodes();
        std::map<TensorId, int>& consumers = consumers_;
        std::map<TensorId, std::size_t> producer, first_consumer;
        for (const aot::Node& n : ns) {
            for (TensorId id : n.inputs)
                if (id) {
                    if (!consumers[id]++) first_consumer[id] = n.index;
                }
            producer[n.outputs[0]] = n.index;
        }
        std::set<TensorId> outputs(g.outputs.begin(), g.outputs.end());
        auto internal_single = [&](TensorId id) { return !outputs.count(id) && consumers[id] == 1; };
        auto fp16_4d = [&](TensorId id) { return desc(id).dtype == aot::DataType::FP16 && desc(id).shape.size() == 4; };
        auto is_std_conv = [&](const aot::Node& n) {
            return n.op == Op::CONV && n.conv().groups == 1 && fp16_4d(n.inputs[0]) && fp16_4d(n.outputs[0]) &&
                   is_weight(n.inputs[1]) && desc(n.inputs[1]).dtype == aot::DataType::FP16;
        };
        // Producers folded into the input staging of their only consumer conv.
        std::vector<bool> folded(ns.size(), false);
        const bool fuse = fusion_enabled();
        for (const aot::Node& n : ns) {
            if (!fuse) break;
            const TensorId out = n.outputs[0];
            if ((n.op != Op::SPACE_TO_DEPTH && n.op != Op::CONCAT) || !internal_single(out)) continue;
            const aot::Node& c = ns[first_consumer[out]];
            if (!is_std_conv(c) || c.inputs[0] != out || !fp16_4d(n.inputs[0])) continue;
            if (n.op == Op::CONCAT) {
                const int axis = n.axis() < 0 ? n.axis() + 4 : n.axis();
                if (axis != 1 || n.inputs.size() != 2 || !fp16_4d(n.inputs[1]) || is_weight(n.inputs[0]) || is_weight(n.inputs[1]))
                    continue;
            } else if (is_weight(n.inputs[0])) {
                continue;
            }
            folded[n.index] = true;
        }

        std::vector<bool> done(ns.size(), false);
        for (const aot::Node& n : ns) {
            if (done[n.index] || folded[n.index]) continue;
            auto L = std::make_unique<Launch>();
            // Real-model chains, in the reference matcher's order
            // (fusion_matcher.cpp:50-72); a chain is taken only when none of
            // its nodes was already lowered into another launch.
            if (fuse && (n.op == Op::SLICE || n.op == Op::SUB)) {
                std::vector<bool> take(ns.size(), false);
                const bool hit = match_y0(n.index, *L, take) || match_y1(n.index, *L, take) || match_feature(n.index, *L, take) ||
                                 match_reglu(n.index, *L, take);
                bool free = hit;
                for (std::size_t k = 0; hit && k < ns.size(); ++k)
                    if (take[k] && (done[k] || folded[k])) free = false;
                if (free) {
                    for (std::size_t k = 0; k < ns.size(); ++k)
                        if (take[k]) done[k] = true;
                    if (L->x) fp16_operand(L->x);
                    for (TensorId id : L->ins) fp16_operand(id);
                    L->name = desc(L->y).name;
                    launches_.push_back(std::move(L));
                    continue;
                }
                L = std::make_unique<Launch>();
            }
            done[n.index] = true;
            switch (n.op) {
            case Op::CONV:
                if (n.conv().groups == 1) {
                    if (!(fuse && lower_pair(*L, n, producer, folded, done, internal_single, first_consumer)))
                        lower_conv(*L, n, producer, folded, done, internal_single, first_consumer, fuse);
                } else if (!(fuse && lower_dwblock(*L, n, done, internal_single, first_consumer))) {
                    lower_depthwise(*L, n);
                }
                break;
            case Op::LEAKY_RELU:
                require_fp16_activation(n.inputs[0]);
                L->kind = Launch::kLeaky;
                L->kind_name = "leaky_relu";
                L->x = n.inputs[0];
                L->y = n.outputs[0];
                L->count = elem_count(desc(L->y).shape);
                L->alpha = n.alpha();
                L->bytes = 4.0 * static_cast<double>(L->count);
                break;
            case Op::ADD:
            case Op::SUB:
            case Op::MUL:
                lower_binary(*L, n);
                break;
            case Op::CLIP:
            case Op::SIGMOID:
            case Op::RECIPROCAL:
            case Op::ROUND:
                lower_unary(*L, n);
                break;
            case Op::SLICE:
                lower_slice(*L, n);
                break;
            case Op::GATHER:
                lower_gather(*L, n);
                break;
            case Op::DEPTH_TO_SPACE:
            case Op::SPACE_TO_DEPTH: {
                require_fp16_activation(n.inputs[0]);
                const auto& s = desc(n.inputs[0]).shape;
                if (s.size() != 4) fail("pixel shuffle needs a 4-D tensor");
                L->kind = n.op == Op::DEPTH_TO_SPACE ? Launch::kD2S : Launch::kS2D;
                L->kind_name = n.op == Op::DEPTH_TO_SPACE ? "depth_to_space" : "space_to_depth";
                L->x = n.inputs[0];
                L->y = n.outputs[0];
                L->n = static_cast<int>(s[0]);
                L->c = static_cast<int>(s[1]);
                L->ih = static_cast<int>(s[2]);
                L->iw = static_cast<int>(s[3]);
                L->block = n.block_size();
                L->bytes = 4.0 * static_cast<double>(elem_count(s));
                break;
            }
            case Op::CONCAT: {
                const int axis = n.axis() < 0 ? n.axis() + 4 : n.axis();
                const bool two_channel = axis == 1 && n.inputs.size() == 2 && fp16_4d(n.inputs[0]) && fp16_4d(n.inputs[1]) &&
                                         !is_weight(n.inputs[0]) && !is_weight(n.inputs[1]) &&
                                         desc(n.outputs[0]).shape.size() == 4;
                if (!two_channel) {
                    lower_concat(*L, n);
                    break;
                }
                const auto& a = desc(n.inputs[0]).shape;
                const auto& b = desc(n.inputs[1]).shape;
                if (a[0] != b[0] || a[2] != b[2] || a[3] != b[3] || desc(n.outputs[0]).shape != std::vector<std::int64_t>{a[0], a[1] + b[1], a[2], a[3]})
                    fail("CONCAT input shape mismatch");
                L->kind = Launch::kConcat;
                L->kind_name = "concat";
                L->x = n.inputs[0];
                L->x2 = n.inputs[1];
                L->y = n.outputs[0];
                L->n = static_cast<int>(a[0]);
                L->ca = static_cast<int>(a[1]);
                L->cb = static_cast<int>(b[1]);
                L->hw = static_cast<std::size_t>(a[2] * a[3]);
                L->bytes = 4.0 * static_cast<double>(elem_count(desc(L->y).shape));
                break;
            }
            default:
                fail("operator " + std::to_string(static_cast<int>(n.op)) + " is outside the conv-graph path");
            }
            if (L->name.empty()) L->name = desc(L->y).name;
            launches_.push_back(std::move(L));
        }
        if (block_handover_nhwc()) lower_channel_last(outputs);
    }

    // Channel-last handover: a tensor whose producer and every reader can
    // take it as [n][h][w][c] is handed over that way. A fused block then
    // stages a 30 KB halo of whole pixels instead of 74 KB of channel rows,
    // and a weight-streaming conv stages 16-byte pixel pieces with no
    // transposes. Readers are fused blocks (their depthwise conv and
    // residual ADD: two nodes reading the tensor) and 3x3 convs reading it
    // as their plain input (one node); every node that reads the tensor
    // must belong to one of them, and no graph output or state is changed.
    void lower_channel_last(const std::set<TensorId>& outputs)
    {
        auto conv_ok = [&](const Launch& L, int in, int out) {
            if (L.kind != Launch::kConv || L.forced) return false;
            mlvc_hip_conv_desc d = L.conv;
            d.in_nhwc = in;
            d.out_nhwc = out;
            int count = 0;
            return mlvc_hip_conv_candidates(&d, nullptr, 0, &count) == 0 && count > 0;
        };
        std::set<TensorId> cl;
        for (const auto& P : launches_) {
            const TensorId t = P->y;
            if (!t || outputs.count(t) || state_out_.count(t) || !(P->kind == Launch::kDwBlock || P->kind == Launch::kConv))
                continue;
            int node_reads = 0, readers = 0;
            bool ok = true;
            for (const auto& Q : launches_) {
                if (Q->x2 == t || Q->res == t || std::find(Q->ins.begin(), Q->ins.end(), t) != Q->ins.end()) ok = false;
                if (!ok) break;
                if (Q->x != t) continue;
                ++readers;
                if (Q->kind == Launch::kDwBlock) node_reads += 2;
                else if (Q->kind == Launch::kConv) node_reads += 1;
                else ok = false;
            }
            if (ok && readers > 0 && node_reads == consumers_[t]) cl.insert(t);
        }
        // A conv needs a variant for the layouts of both its operands; drop
        // handovers until every conv has one.
        for (bool changed = true; changed;) {
            changed = false;
            for (const auto& Lp : launches_) {
                if (Lp->kind != Launch::kConv) continue;
                const int in = cl.count(Lp->x) ? 1 : 0, out = cl.count(Lp->y) ? 1 : 0;
                if ((in || out) && !conv_ok(*Lp, in, out)) {
                    cl.erase(out ? Lp->y : Lp->x);
                    changed = true;
                }
            }
        }
        for (const auto& Lp : launches_) {
            Launch& L = *Lp;
            const int in = cl.count(L.x) ? 1 : 0, out = cl.count(L.y) ? 1 : 0;
            if (!in && !out) continue;
            const std::string tag = std::string(in ? "+nhwc_in" : "") + (out ? "+nhwc_out" : "");
            if (L.kind == Launch::kDwBlock) {
                L.blk.in_nhwc = in;
                L.blk.out_nhwc = out;
                L.kind_name += tag;
                continue;
            }
            // Re-plan among the variants that take the layouts and re-pack
            // for the one chosen (its weight order can differ).
            const std::string tags = L.kind_name.substr(std::string(mlvc_hip_conv_variant_name(L.conv.variant)).size());
            L.conv.in_nhwc = in;
            L.conv.out_nhwc = out;
            hip_check(mlvc_hip_conv_plan(&L.conv), "conv planning");
            L.kind_name = std::string(mlvc_hip_conv_variant_name(L.conv.variant)) + tags + tag;
            for (void* old : {L.packed.ptr, L.bias.ptr})
                pending_uploads_.erase(std::remove_if(pending_uploads_.begin(), pending_uploads_.end(),
                                                      [&](const auto& u) { return u.first == old; }),
                                       pending_uploads_.end());
            pack_conv(L, L.packed, L.bias, L.conv);
        }
    }

    void require_fp16_activation(TensorId id) const
    {
        if (is_weight(id) || desc(id).dtype != aot::DataType::FP16) fail("operand must be an FP16 activation");
    }

    std::vector<std::uint16_t> weight_fp16(TensorId id) const
    {
        const auto& w = std::get<aot::WeightLocation>(desc(id).storage);
        std::vector<std::uint16_t> v(w.bytes / 2);
        std::memcpy(v.data(), graph_.weights.data() + w.offset, w.bytes);
        return v;
    }

    std::vector<float> bias_f32(const aot::Node& n, int oc, std::size_t padded) const
    {
        std::vector<float> b(padded, 0.0F);
        if (n.inputs.size() >= 3 && n.inputs[2]) {
            if (!is_weight(n.inputs[2]) || desc(n.inputs[2]).dtype != aot::DataType::FP16) fail("conv bias must be an FP16 initializer");
            const auto raw = weight_fp16(n.inputs[2]);
            if (static_cast<int>(raw.size()) != oc) fail("conv bias length mismatch");
            for (int i = 0; i < oc; ++i) b[static_cast<std::size_t>(i)] = half_to_float(raw[static_cast<std::size_t>(i)]);
        }
        return b;
    }

    // Packs L's weights into the fragment order of d.variant and queues the
    // upload of weights and padded FP32 bias into (w, b).
    void pack_conv(const Launch& L, DeviceMem& w, DeviceMem& b, const mlvc_hip_conv_desc& d)
    {
        std::vector<std::uint8_t> packed(mlvc_hip_conv_packed_bytes(&d));
        hip_check(mlvc_hip_conv_pack(&d, L.w_oihw.data(), packed.data()), "weight packing");
        w = DeviceMem(packed.size());
        pending_uploads_.push_back({w.ptr, std::move(packed)});
        std::vector<float> bias(mlvc_hip_conv_bias_len(&d), 0.0F);
        std::copy(L.bias_oc.begin(), L.bias_oc.end(), bias.begin());
        b = DeviceMem(bias.size() * 4);
        std::vector<std::uint8_t> braw(bias.size() * 4);
        std::memcpy(braw.data(), bias.data(), braw.size());
        pending_uploads_.push_back({b.ptr, std::move(braw)});
    }

    // try_pointwise_reglu (fusion_matcher.cpp:258-302): a 1x1 stride-1
    // unpadded conv whose output only feeds SLICE [0,G) and SLICE [G,2G)
    // (nodes i+1, i+2) -> CLIP(gate) (i+3) -> MUL(clipped, linear) (i+4).
    // Returns the MUL output, or 0. G is a multiple of 32 here (the kernel
    // pairs 32 gate rows with 32 linear rows per 64-row block).
    TensorId pointwise_reglu(const aot::Node& n, float& lo, float& hi) const
    {
        const auto& ns = nodes();
        const std::size_t i = n.index;
        if (i + 5 > ns.size() || n.conv().groups != 1) return 0;
        const auto& a = n.conv();
        const auto& ws = desc(n.inputs[1]).shape;
        if (ws[2] != 1 || ws[3] != 1 || a.strides[0] != 1 || a.strides[1] != 1 || a.pads[0] || a.pads[1]) return 0;
        const TensorId x = n.outputs[0];
        if (!internal_only(x, 2) || !fp16_4d(x)) return 0;
        const std::int64_t g = desc(x).shape[1] / 2;
        if (desc(x).shape[1] % 2 || g % 32) return 0;
        if (!channel_slice(ns[i + 1], x, 0, g) || !channel_slice(ns[i + 2], x, g, 2 * g)) return 0;
        const TensorId gate = ns[i + 1].outputs[0], lin = ns[i + 2].outputs[0];
        if (!internal_only(gate, 1) || !internal_only(lin, 1)) return 0;
        if (!clip_constants(ns[i + 3], lo, hi) || ns[i + 3].inputs[0] != gate) return 0;
        const TensorId clipped = ns[i + 3].outputs[0];
        if (!internal_only(clipped, 1) || !pair(ns[i + 4], Op::MUL, clipped, lin)) return 0;
        const auto& s = desc(x).shape;
        const TensorId y = ns[i + 4].outputs[0];
        if (!fp16_of(y, {s[0], g, s[2], s[3]})) return 0;
        return y;
    }

    // Weight and bias rows of a ReGLU conv in the kernel's pairing order:
    // 64-row blocks of 32 gate rows (g..g+31) then the matching linear rows.
    static void reglu_row_order(Launch& L, int oc, std::size_t row_len)
    {
        const int g = oc / 2;
        std::vector<std::uint16_t> w(L.w_oihw.size());
        std::vector<float> b(L.bias_oc.size());
        for (int r = 0; r < oc; ++r) {
            const int blk = r / 64, k = r % 64;
            const int src = k < 32 ? blk * 32 + k : g + blk * 32 + (k - 32);
            std::copy_n(L.w_oihw.begin() + static_cast<std::ptrdiff_t>(src * row_len), row_len,
                        w.begin() + static_cast<std::ptrdiff_t>(r * row_len));
            b[static_cast<std::size_t>(r)] = L.bias_oc[static_cast<std::size_t>(src)];
        }
        L.w_oihw = std::move(w);
        L.bias_oc = std::move(b);
    }

    template <typename SingleFn>
    void lower_conv(Launch& L, const aot::Node& n, std::map<TensorId, std::size_t>& producer, const std::vector<bool>& folded,
                    std::vector<bool>& done, SingleFn internal_single, std::map<TensorId, std::size_t>& first_consumer,
                    bool fuse)
    {
        const auto& ns = nodes();
        const auto& xs = desc(n.inputs[0]).shape;
        const auto& ws = desc(n.inputs[1]).shape;
        const auto& ys = desc(n.outputs[0]).shape;
        if (xs.size() != 4 || ws.size() != 4 || ys.size() != 4) fail("conv expects 4-D NCHW tensors");
        if (!is_weight(n.inputs[1])) fail("conv weights must be an initializer");
        const auto& a = n.conv();
        mlvc_hip_conv_desc& d = L.conv;
        d = mlvc_hip_conv_desc{};
        d.n = static_cast<int>(xs[0]);
        d.ic = static_cast<int>(xs[1]);
        d.ih = static_cast<int>(xs[2]);
        d.iw = static_cast<int>(xs[3]);
        d.oc = static_cast<int>(ys[1]);
        d.oh = static_cast<int>(ys[2]);
        d.ow = static_cast<int>(ys[3]);
        d.kh = static_cast<int>(ws[2]);
        d.kw = static_cast<int>(ws[3]);
        d.stride_h = a.strides[0];
        d.stride_w = a.strides[1];
        d.pad_h = a.pads[0];
        d.pad_w = a.pads[1];
        if (ws[0] != ys[1] || ws[1] != xs[1]) fail("conv weight shape mismatch");
        L.kind = Launch::kConv;
        L.name = desc(n.outputs[0]).name;
        std::string tags;

        // Input side: a folded SPACE_TO_DEPTH or CONCAT producer.
        TensorId in = n.inputs[0];
        L.x = in;
        if (producer.count(in) && folded[producer[in]]) {
            const aot::Node& p = ns[producer[in]];
            if (p.op == Op::SPACE_TO_DEPTH) {
                L.x = p.inputs[0];
                d.in_s2d_block = p.block_size();
                tags += "+s2d";
            } else {
                L.x = p.inputs[0];
                L.x2 = p.inputs[1];
                d.ic_split = static_cast<int>(desc(p.inputs[0]).shape[1]);
                tags += "+concat";
            }
        }
        // Epilogue (fusion_matcher.cpp:352-411).
        TensorId out = n.outputs[0];
        bool reglu = false;
        if (fuse && !L.x2 && d.in_s2d_block <= 1) {
            float lo = 0.0F, hi = 0.0F;
            if (TensorId y = pointwise_reglu(n, lo, hi)) {
                d.epilogue = MLVC_EPI_REGLU;
                d.clip_lo = lo;
                d.clip_hi = hi;
                for (std::size_t k = n.index + 1; k < n.index + 5; ++k) done[k] = true;
                out = y;
                reglu = true;
                tags += "+reglu";
            }
        }
        if (!reglu && fuse && n.index + 1 < ns.size() && internal_single(out)) {
            const aot::Node& nx = ns[n.index + 1];
            if (nx.op == Op::LEAKY_RELU && nx.inputs[0] == out) {
                d.epilogue = MLVC_EPI_LEAKY_RELU;
                d.alpha = nx.alpha();
                done[nx.index] = true;
                out = nx.outputs[0];
                tags += "+lrelu";
            } else if (float lo = 0.0F, hi = 0.0F; clip_constants(nx, lo, hi) && nx.inputs[0] == out &&
                                                   desc(nx.outputs[0]).shape == desc(out).shape) {
                d.epilogue = MLVC_EPI_CLAMP;
                d.clip_lo = lo;
                d.clip_hi = hi;
                done[nx.index] = true;
                out = nx.outputs[0];
                tags += "+clip";
            } else if (nx.op == Op::ADD && (nx.inputs[0] == out || nx.inputs[1] == out)) {
                const TensorId r = nx.inputs[0] == out ? nx.inputs[1] : nx.inputs[0];
                if (r != out && !is_weight(r) && desc(r).dtype == aot::DataType::FP16 && desc(r).shape == desc(out).shape) {
                    d.epilogue = MLVC_EPI_RESIDUAL_ADD;
                    L.res = r;
                    done[nx.index] = true;
                    out = nx.outputs[0];
                    tags += "+residual";
                }
            }
        }
        // Output side: a DEPTH_TO_SPACE that is the only consumer.
        if (!reglu && fuse && internal_single(out)) {
            const aot::Node& c = ns[first_consumer[out]];
            if (c.op == Op::DEPTH_TO_SPACE && c.inputs[0] == out && !done[c.index]) {
                d.out_d2s_block = c.block_size();
                done[c.index] = true;
                out = c.outputs[0];
                tags += "+d2s";
            }
        }
        L.y = out;
        hip_check(mlvc_hip_conv_plan(&d), "conv planning");
        if (d.ksplit > 1) tags = "+split" + std::to_string(d.ksplit) + tags;
        if (const std::string want = forced_conv_variant(); !want.empty()) {
            int count = 0;
            hip_check(mlvc_hip_conv_candidates(&d, nullptr, 0, &count), "conv candidates");
            std::vector<int> cand(static_cast<std::size_t>(count));
            hip_check(mlvc_hip_conv_candidates(&d, cand.data(), count, &count), "conv candidates");
            for (int v : cand)
                if (want == mlvc_hip_conv_variant_name(v)) {
                    d.variant = v;
                    L.forced = true;
                }
        }
        L.kind_name = std::string(mlvc_hip_conv_variant_name(d.variant)) + tags;
        // Pack weights into the variant's fragment order, widen the bias.
        L.w_oihw = weight_fp16(n.inputs[1]);
        L.bias_oc = bias_f32(n, d.oc, static_cast<std::size_t>(d.oc));
        if (reglu) reglu_row_order(L, d.oc, static_cast<std::size_t>(d.ic) * d.kh * d.kw);
        pack_conv(L, L.packed, L.bias, d);
        // Algorithmic work: 2*N*OC*OH*OW*IC*KH*KW FLOPs; bytes = each tensor once
        // (a ReGLU epilogue writes OC/2 channels).
        L.flops = 2.0 * d.n * d.oc * d.oh * d.ow * static_cast<double>(d.ic) * d.kh * d.kw;
        L.bytes = 2.0 * (static_cast<double>(d.n) * d.ic * d.ih * d.iw + static_cast<double>(d.oc) * d.ic * d.kh * d.kw + d.oc +
                         static_cast<double>(d.n) * d.oc * d.oh * d.ow * (L.res ? 2.0 : reglu ? 0.5 : 1.0));
    }

    // 3x3 s1 p1 conv (input plain or a folded SPACE_TO_DEPTH(2)) [-> LEAKY_RELU]
    // -> CONCAT(t, r) -> 1x1 conv [-> LEAKY_RELU], every intermediate with
    // one consumer and not a graph output: one fused launch, t stays on chip.
    template <typename SingleFn>
    bool lower_pair(Launch& L, const aot::Node& n, std::map<TensorId, std::size_t>& producer, const std::vector<bool>& folded,
                    std::vector<bool>& done, SingleFn internal_single, std::map<TensorId, std::size_t>& first_consumer)
    {
        const auto& ns = nodes();
        const auto& ws = desc(n.inputs[1]).shape;
        if (ws.size() != 4 || ws[2] != 3 || ws[3] != 3 || n.conv().strides != std::array<int, 2>{1, 1} ||
            n.conv().pads != std::array<int, 4>{1, 1, 1, 1} || !is_weight(n.inputs[1]))
            return false;
        TensorId x = n.inputs[0];
        int s2d = 0;
        if (producer.count(x) && folded[producer[x]]) {
            const aot::Node& pn = ns[producer[x]];
            if (pn.op != Op::SPACE_TO_DEPTH || pn.block_size() != 2) return false;
            x = pn.inputs[0];
            s2d = 2;
        }
        auto next = [&](TensorId id) -> const aot::Node* {
            if (!internal_single(id)) return nullptr;
            return &ns[first_consumer[id]];
        };
        TensorId t = n.outputs[0];
        const aot::Node* act_a = nullptr;
        const aot::Node* c = next(t);
        if (c && c->op == Op::LEAKY_RELU && c->inputs[0] == t) {
            act_a = c;
            t = c->outputs[0];
            c = next(t);
        }
        if (!c || c->op != Op::CONCAT || c->inputs.size() != 2 || c->inputs[0] != t) return false;
        const int axis = c->axis() < 0 ? c->axis() + 4 : c->axis();
        const TensorId r = c->inputs[1];
        if (axis != 1 || is_weight(r) || desc(r).dtype != aot::DataType::FP16 || desc(r).shape.size() != 4) return false;
        const aot::Node* m = next(c->outputs[0]);
        if (!m || m->op != Op::CONV || m->inputs[0] != c->outputs[0] || m->conv().groups != 1 || !is_weight(m->inputs[1]))
            return false;
        const auto& wm = desc(m->inputs[1]).shape;
        if (wm.size() != 4 || wm[2] != 1 || wm[3] != 1 || m->conv().strides != std::array<int, 2>{1, 1} ||
            m->conv().pads != std::array<int, 4>{0, 0, 0, 0})
            return false;
        TensorId y = m->outputs[0];
        const aot::Node* act_b = nullptr;
        if (const aot::Node* nb = next(y); nb && nb->op == Op::LEAKY_RELU && nb->inputs[0] == y) {
            act_b = nb;
            y = nb->outputs[0];
        }
        const auto& ts = desc(n.outputs[0]).shape;
        const auto& rs = desc(r).shape;
        const auto& ys = desc(y).shape;
        mlvc_hip_convpair_desc& d = L.pair;
        d = mlvc_hip_convpair_desc{};
        d.n = static_cast<int>(ts[0]);
        d.ica = static_cast<int>(ws[1]);
        d.h = static_cast<int>(ts[2]);
        d.w = static_cast<int>(ts[3]);
        d.in_s2d_block = s2d;
        d.oca = static_cast<int>(ts[1]);
        d.cr = static_cast<int>(rs[1]);
        d.ocb = static_cast<int>(wm[0]);
        d.epi_a = act_a ? MLVC_EPI_LEAKY_RELU : MLVC_EPI_NONE;
        d.alpha_a = act_a ? act_a->alpha() : 0.0F;
        d.epi_b = act_b ? MLVC_EPI_LEAKY_RELU : MLVC_EPI_NONE;
        d.alpha_b = act_b ? act_b->alpha() : 0.0F;
        if (rs[0] != ts[0] || rs[2] != ts[2] || rs[3] != ts[3] || wm[1] != d.oca + d.cr || ys[1] != d.ocb ||
            ys[2] != ts[2] || ys[3] != ts[3] || !mlvc_hip_convpair_supported(&d))
            return false;
        L.kind = Launch::kPair;
        L.kind_name = std::string("convpair_3x3_1x1") + (s2d ? "+s2d" : "") + "+concat";
        L.name = desc(y).name;
        L.x = x;
        L.x2 = r;
        L.y = y;
        const auto wa = weight_fp16(n.inputs[1]);
        const auto wb = weight_fp16(m->inputs[1]);
        std::vector<std::uint8_t> pa(mlvc_hip_convpair_packed_a_bytes(&d)), pb(mlvc_hip_convpair_packed_b_bytes(&d));
        hip_check(mlvc_hip_convpair_pack(&d, wa.data(), wb.data(), pa.data(), pb.data()), "pair weight packing");
        auto upload = [&](DeviceMem& dst, std::vector<std::uint8_t> bytes) {
            dst = DeviceMem(bytes.size());
            pending_uploads_.push_back({dst.ptr, std::move(bytes)});
        };
        auto f32_bytes = [](const std::vector<float>& v) {
            std::vector<std::uint8_t> b(v.size() * 4);
            std::memcpy(b.data(), v.data(), b.size());
            return b;
        };
        upload(L.packed, std::move(pa));
        upload(L.bias, f32_bytes(bias_f32(n, d.oca, static_cast<std::size_t>(d.oca))));
        upload(L.packed2, std::move(pb));
        upload(L.bias2, f32_bytes(bias_f32(*m, d.ocb, static_cast<std::size_t>(d.ocb))));
        for (const aot::Node* q : {act_a, c, m, act_b})
            if (q) done[q->index] = true;
        const double px = static_cast<double>(d.n) * d.h * d.w;
        L.flops = 2.0 * px * d.oca * d.ica * 9 + 2.0 * px * d.ocb * (d.oca + d.cr);
        L.bytes = 2.0 * (px * d.ica + px * d.cr + px * d.ocb + 9.0 * d.oca * d.ica + static_cast<double>(d.ocb) * (d.oca + d.cr)) +
                  4.0 * (d.oca + d.ocb);
        return true;
    }

    // DW3x3 s1 p1 -> 1x1 C->E -> LEAKY_RELU -> 1x1 E->C -> ADD(block input),
    // every intermediate with exactly one consumer and not a graph output.
    template <typename SingleFn>
    bool lower_dwblock(Launch& L, const aot::Node& n0, std::vector<bool>& done, SingleFn internal_single,
                       std::map<TensorId, std::size_t>& first_consumer)
    {
        const auto& ns = nodes();
        const TensorId t = n0.inputs[0];
        const auto& xs = desc(t).shape;
        const auto& ws = desc(n0.inputs[1]).shape;
        if (xs.size() != 4 || ws.size() != 4 || is_weight(t) || desc(t).dtype != aot::DataType::FP16) return false;
        const auto& a0 = n0.conv();
        const int c = static_cast<int>(xs[1]);
        if (a0.groups != c || ws[0] != c || ws[1] != 1 || ws[2] != 3 || ws[3] != 3 || a0.strides != std::array<int, 2>{1, 1} ||
            a0.pads != std::array<int, 4>{1, 1, 1, 1} || desc(n0.outputs[0]).shape != xs)
            return false;
        auto next = [&](TensorId id) -> const aot::Node* {
            if (!internal_single(id)) return nullptr;
            return &ns[first_consumer[id]];
        };
        auto is_pointwise = [&](const aot::Node* m, TensorId in) {
            if (!m || m->op != Op::CONV || m->inputs[0] != in || m->conv().groups != 1 || !is_weight(m->inputs[1])) return false;
            const auto& w = desc(m->inputs[1]).shape;
            return w.size() == 4 && w[2] == 1 && w[3] == 1 && m->conv().strides == std::array<int, 2>{1, 1} &&
                   m->conv().pads == std::array<int, 4>{0, 0, 0, 0};
        };
        const aot::Node* n1 = next(n0.outputs[0]);
        if (!is_pointwise(n1, n0.outputs[0])) return false;
        const aot::Node* n2 = next(n1->outputs[0]);
        if (!n2 || n2->op != Op::LEAKY_RELU || n2->inputs[0] != n1->outputs[0]) return false;
        const aot::Node* n3 = next(n2->outputs[0]);
        if (!is_pointwise(n3, n2->outputs[0])) return false;
        const aot::Node* n4 = next(n3->outputs[0]);
        if (!n4 || n4->op != Op::ADD) return false;
        const TensorId f = n3->outputs[0];
        if (!((n4->inputs[0] == f && n4->inputs[1] == t) || (n4->inputs[1] == f && n4->inputs[0] == t))) return false;
        const int e = static_cast<int>(desc(n1->inputs[1]).shape[0]);
        if (desc(n3->inputs[1]).shape[0] != c || desc(n3->inputs[1]).shape[1] != e || desc(n1->inputs[1]).shape[1] != c ||
            desc(n4->outputs[0]).shape != xs)
            return false;
        const int h = static_cast<int>(xs[2]), w = static_cast<int>(xs[3]);
        if (!mlvc_hip_dwblock_supported(c, e, h, w)) return false;

        L.kind = Launch::kDwBlock;
        L.kind_name = "dwblock_c" + std::to_string(c) + "_e" + std::to_string(e);
        L.name = desc(n0.outputs[0]).name + "+block";
        L.x = t;
        L.y = n4->outputs[0];
        auto upload = [&](DeviceMem& dst, std::vector<std::uint8_t> bytes) {
            dst = DeviceMem(bytes.size());
            pending_uploads_.push_back({dst.ptr, std::move(bytes)});
        };
        auto as_bytes = [](const void* p, std::size_t n) {
            std::vector<std::uint8_t> v(n);
            std::memcpy(v.data(), p, n);
            return v;
        };
        const auto wdw = weight_fp16(n0.inputs[1]);
        upload(L.packed, as_bytes(wdw.data(), wdw.size() * 2));
        const auto bdw = bias_f32(n0, c, static_cast<std::size_t>(c));
        upload(L.bias, as_bytes(bdw.data(), bdw.size() * 4));
        const auto w1 = weight_fp16(n1->inputs[1]);
        std::vector<std::uint8_t> p1(mlvc_hip_dwblock_packed_bytes(e, c));
        hip_check(mlvc_hip_dwblock_pack(w1.data(), e, c, p1.data()), "block weight packing");
        upload(L.packed2, std::move(p1));
        const auto b1 = bias_f32(*n1, e, static_cast<std::size_t>(e));
        upload(L.bias2, as_bytes(b1.data(), b1.size() * 4));
        const auto w2 = weight_fp16(n3->inputs[1]);
        std::vector<std::uint8_t> p2(mlvc_hip_dwblock_packed_bytes(c, e));
        hip_check(mlvc_hip_dwblock_pack(w2.data(), c, e, p2.data()), "block weight packing");
        upload(L.packed3, std::move(p2));
        const auto b2 = bias_f32(*n3, c, static_cast<std::size_t>(c));
        upload(L.bias3, as_bytes(b2.data(), b2.size() * 4));
        mlvc_hip_dwblock_desc& d = L.blk;
        d = mlvc_hip_dwblock_desc{};
        d.n = static_cast<int>(xs[0]);
        d.c = c;
        d.e = e;
        d.h = h;
        d.w = w;
        d.alpha = n2->alpha();
        for (const aot::Node* m : {n1, n2, n3, n4}) done[m->index] = true;
        const double px = static_cast<double>(d.n) * h * w;
        L.flops = 2.0 * px * c * 9 + 4.0 * px * c * e;
        L.bytes = 2.0 * (2.0 * px * c + 9.0 * c + 2.0 * c * e) + 4.0 * (2.0 * c + e);
        return true;
    }

    void lower_depthwise(Launch& L, const aot::Node& n)
    {
        const auto& xs = desc(n.inputs[0]).shape;
        const auto& ws = desc(n.inputs[1]).shape;
        const auto& ys = desc(n.outputs[0]).shape;
        if (xs.size() != 4 || ws.size() != 4 || ys.size() != 4) fail("conv expects 4-D NCHW tensors");
        const int groups = n.conv().groups;
        if (!(groups == xs[1] && ys[1] == xs[1] && ws[1] == 1)) fail("general grouped convolution (1 < groups < IC) unsupported");
        require_fp16_activation(n.inputs[0]);
        const auto& a = n.conv();
        L.kind = Launch::kDepthwise;
        L.kind_name = "depthwise";
        L.x = n.inputs[0];
        L.y = n.outputs[0];
        L.n = static_cast<int>(xs[0]);
        L.c = static_cast<int>(xs[1]);
        L.ih = static_cast<int>(xs[2]);
        L.iw = static_cast<int>(xs[3]);
        L.oh = static_cast<int>(ys[2]);
        L.ow = static_cast<int>(ys[3]);
        L.kh = static_cast<int>(ws[2]);
        L.kw = static_cast<int>(ws[3]);
        L.sh = a.strides[0];
        L.sw = a.strides[1];
        L.ph = a.pads[0];
        L.pw = a.pads[1];
        const auto w = weight_fp16(n.inputs[1]);
        std::vector<std::uint8_t> wr(w.size() * 2);
        std::memcpy(wr.data(), w.data(), wr.size());
        L.packed = DeviceMem(wr.size());
        pending_uploads_.push_back({L.packed.ptr, std::move(wr)});
        const auto b = bias_f32(n, L.c, static_cast<std::size_t>(L.c));
        std::vector<std::uint8_t> braw(b.size() * 4);
        std::memcpy(braw.data(), b.data(), braw.size());
        L.bias = DeviceMem(braw.size());
        pending_uploads_.push_back({L.bias.ptr, std::move(braw)});
        L.flops = 2.0 * L.n * L.c * L.oh * L.ow * static_cast<double>(L.kh) * L.kw;
        L.bytes = 2.0 * (static_cast<double>(L.n) * L.c * L.ih * L.iw + static_cast<double>(L.n) * L.c * L.oh * L.ow +
                         static_cast<double>(L.c) * (L.kh * L.kw + 1));
    }

    // ---------------------------------------------------------- memory
    // Tensors live in one device arena, re-planned over the fused launch
    // schedule: a tensor is live from the launch that writes it to the last
    // launch that reads it (graph outputs to the end); first-fit placement
    // by start then size, 256-byte aligned (the reference CPU plan does the
    // same over its fused steps, execution_plan.cpp:668-804).
    void plan_memory()
    {
        const std::size_t n = launches_.size();
        std::map<TensorId, std::pair<std::size_t, std::size_t>> live;
        auto arena_resident = [&](TensorId id) {
            return id && !is_weight(id) && !state_in_.count(id) && !state_out_.count(id) &&
                   std::find(graph_.descriptor.inputs.begin(), graph_.descriptor.inputs.end(), id) == graph_.descriptor.inputs.end();
        };
        for (std::size_t i = 0; i < n; ++i) {
            const Launch& l = *launches_[i];
            std::vector<TensorId> writes{l.y}, reads{l.x, l.x2, l.res};
            writes.insert(writes.end(), l.outs.begin(), l.outs.end());
            reads.insert(reads.end(), l.ins.begin(), l.ins.end());
            for (TensorId w : writes) {
                if (!arena_resident(w)) continue;
                auto it = live.find(w);
                if (it == live.end()) live[w] = {i, i};
                else it->second.second = std::max(it->second.second, i);
            }
            for (TensorId r : reads) {
                if (!arena_resident(r)) continue;
                auto it = live.find(r);
                if (it == live.end()) fail("tensor read before it is written: " + desc(r).name);
                it->second.second = std::max(it->second.second, i);
            }
        }
        for (TensorId o : graph_.descriptor.outputs)
            if (live.count(o)) live[o].second = n;
        std::vector<TensorId> order;
        for (auto& kv : live) order.push_back(kv.first);
        std::sort(order.begin(), order.end(), [&](TensorId a, TensorId b) {
            if (live[a].first != live[b].first) return live[a].first < live[b].first;
            return desc_bytes(desc(a)) > desc_bytes(desc(b));
        });
        struct Placed { std::size_t off, size, first, last; };
        std::vector<Placed> placed;
        std::size_t peak = 256;
        for (TensorId id : order) {
            const std::size_t sz = (desc_bytes(desc(id)) + 255) / 256 * 256;
            const auto [f, l] = live[id];
            std::vector<std::pair<std::size_t, std::size_t>> busy;
            for (const Placed& p : placed)
                if (p.first <= l && f <= p.last) busy.emplace_back(p.off, p.off + p.size);
            std::sort(busy.begin(), busy.end());
            std::size_t cand = 0;
            for (const auto& [b0, b1] : busy) {
                if (cand + sz <= b0) break;
                cand = std::max(cand, b1);
            }
            offset_[id] = cand;
            placed.push_back({cand, sz, f, l});
            peak = std::max(peak, cand + sz);
        }
        arena_bytes_ = peak;
        arena_ = DeviceMem(peak);
        for (const auto& lp : launches_)
            if (lp->kind == Launch::kConv)
                workspace_bytes_ = std::max(workspace_bytes_, mlvc_hip_conv_workspace_bytes(&lp->conv));
        if (workspace_bytes_) workspace_ = DeviceMem(workspace_bytes_);
    }

    void allocate_io()
    {
        for (TensorId id : ext_in_) input_buf_.emplace(id, DeviceMem(desc_bytes(desc(id))));
        for (auto& b : bindings_)
            for (auto& buf : b.buf) buf = DeviceMem(b.bytes);
        for (TensorId id : ext_in_) in_stage_.emplace_back(desc_bytes(desc(id)));
        for (TensorId id : ext_out_) out_stage_.emplace_back(desc_bytes(desc(id)));
    }

    void upload_parameters()
    {
        for (auto& [dst, bytes] : pending_uploads_)
            hip_check(mlvc_hip_memcpy_h2d(dst, bytes.data(), bytes.size(), stream_), "parameter upload");
        hip_check(mlvc_hip_stream_synchronize(stream_), "stream sync");
        pending_uploads_.clear();
    }

    void* ptr(TensorId id, int parity)
    {
        if (auto it = state_in_.find(id); it != state_in_.end()) return bindings_[it->second].buf[parity].ptr;
        if (auto it = state_out_.find(id); it != state_out_.end()) return bindings_[it->second].buf[parity ^ 1].ptr;
        if (auto it = input_buf_.find(id); it != input_buf_.end()) return it->second.ptr;
        if (auto it = const_buf_.find(id); it != const_buf_.end()) return it->second.ptr;
        if (auto it = offset_.find(id); it != offset_.end()) return static_cast<char*>(arena_.ptr) + it->second;
        fail("tensor without device storage: " + desc(id).name);
    }

    void enqueue_one(Launch& l, int parity)
    {
        switch (l.kind) {
        case Launch::kConv: {
            mlvc_hip_conv_desc d = l.conv;
            d.x = ptr(l.x, parity);
            d.x2 = l.x2 ? ptr(l.x2, parity) : nullptr;
            d.residual = l.res ? ptr(l.res, parity) : nullptr;
            d.y = ptr(l.y, parity);
            d.packed_w = l.packed.ptr;
            d.bias = static_cast<const float*>(l.bias.ptr);
            d.workspace = workspace_.ptr;
            d.workspace_bytes = workspace_bytes_;
            hip_check(mlvc_hip_conv_launch(&d, stream_), "conv launch");
            break;
        }
        case Launch::kDepthwise:
            hip_check(mlvc_hip_depthwise(ptr(l.x, parity), static_cast<const std::uint16_t*>(l.packed.ptr),
                                         static_cast<const float*>(l.bias.ptr), ptr(l.y, parity), l.n, l.c, l.ih, l.iw, l.oh,
                                         l.ow, l.kh, l.kw, l.sh, l.sw, l.ph, l.pw, stream_),
                      "depthwise launch");
            break;
        case Launch::kDwBlock: {
            mlvc_hip_dwblock_desc d = l.blk;
            d.x = ptr(l.x, parity);
            d.y = ptr(l.y, parity);
            d.dw_w = static_cast<const std::uint16_t*>(l.packed.ptr);
            d.dw_b = static_cast<const float*>(l.bias.ptr);
            d.w1 = l.packed2.ptr;
            d.b1 = static_cast<const float*>(l.bias2.ptr);
            d.w2 = l.packed3.ptr;
            d.b2 = static_cast<const float*>(l.bias3.ptr);
            hip_check(mlvc_hip_dwblock_launch(&d, stream_), "dwblock launch");
            break;
        }
        case Launch::kPair: {
            mlvc_hip_convpair_desc d = l.pair;
            d.x = ptr(l.x, parity);
            d.r = ptr(l.x2, parity);
            d.y = ptr(l.y, parity);
            d.wa = l.packed.ptr;
            d.ba = static_cast<const float*>(l.bias.ptr);
            d.wb = l.packed2.ptr;
            d.bb = static_cast<const float*>(l.bias2.ptr);
            hip_check(mlvc_hip_convpair_launch(&d, stream_), "convpair launch");
            break;
        }
        case Launch::kLeaky:
            hip_check(mlvc_hip_leaky_relu(ptr(l.x, parity), ptr(l.y, parity), l.count, l.alpha, stream_), "leaky_relu launch");
            break;
        case Launch::kAdd:
            hip_check(mlvc_hip_add(ptr(l.x, parity), ptr(l.x2, parity), ptr(l.y, parity), l.count, stream_), "add launch");
            break;
        case Launch::kD2S:
            hip_check(mlvc_hip_depth_to_space(ptr(l.x, parity), ptr(l.y, parity), l.n, l.c, l.ih, l.iw, l.block, stream_),
                      "depth_to_space launch");
            break;
        case Launch::kS2D:
            hip_check(mlvc_hip_space_to_depth(ptr(l.x, parity), ptr(l.y, parity), l.n, l.c, l.ih, l.iw, l.block, stream_),
                      "space_to_depth launch");
            break;
        case Launch::kConcat:
            hip_check(mlvc_hip_concat_channels(ptr(l.x, parity), l.ca, ptr(l.x2, parity), l.cb, ptr(l.y, parity), l.n, l.hw,
                                               stream_),
                      "concat launch");
            break;
        case Launch::kUnary:
            hip_check(mlvc_hip_unary(ptr(l.x, parity), ptr(l.y, parity), l.count, l.op, l.lo, l.hi, stream_), "unary launch");
            break;
        case Launch::kBinary:
            hip_check(mlvc_hip_binary(ptr(l.x, parity), l.da, ptr(l.x2, parity), l.db, ptr(l.y, parity), l.dy, l.op, stream_),
                      "binary launch");
            break;
        case Launch::kSlice:
            hip_check(mlvc_hip_slice(ptr(l.x, parity), l.da, ptr(l.y, parity), l.dy, l.starts, l.steps, stream_), "slice launch");
            break;
        case Launch::kConcatAny: {
            auto* out = static_cast<std::uint16_t*>(ptr(l.y, parity));
            for (std::size_t k = 0; k < l.ins.size(); ++k) {
                const Launch::Piece& p = l.pieces[k];
                hip_check(mlvc_hip_copy_rows(ptr(l.ins[k], parity), out + p.y_offset, p.rows, p.row_elems, p.row_elems, p.y_stride,
                                             stream_),
                          "concat launch");
            }
            break;
        }
        case Launch::kGather:
            hip_check(mlvc_hip_gather(ptr(l.x, parity), ptr(l.x2, parity), l.idx64 ? 1 : 0, l.count, l.outer, l.dim, l.inner,
                                      ptr(l.y, parity), stream_),
                      "gather launch");
            break;
        case Launch::kReglu:
            hip_check(mlvc_hip_reglu(ptr(l.x, parity), ptr(l.y, parity), l.n, l.c, l.hw, l.lo, l.hi, stream_), "reglu launch");
            break;
        case Launch::kFeature:
            hip_check(mlvc_hip_feature_update(ptr(l.x, parity), ptr(l.ins[0], parity), ptr(l.ins[1], parity), ptr(l.y, parity),
                                              l.outs.empty() ? nullptr : ptr(l.outs[0], parity),
                                              l.outs.empty() ? nullptr : ptr(l.outs[1], parity), l.n, l.c, l.hw, stream_),
                      "feature update launch");
            break;
        case Launch::kY0: {
            mlvc_hip_y0_tail_desc d{};
            d.latent = ptr(l.ins[0], parity);
            d.prior = ptr(l.ins[1], parity);
            d.quant_scale = ptr(l.ins[2], parity);
            d.update_scale0 = ptr(l.ins[3], parity);
            d.update_scale1 = ptr(l.ins[4], parity);
            d.normalized = ptr(l.outs[0], parity);
            d.clipped = ptr(l.outs[1], parity);
            d.y_raw = ptr(l.outs[2], parity);
            d.concat2 = ptr(l.outs[3], parity);
            d.concat3 = ptr(l.y, parity);
            d.n = l.n;
            d.q = l.c;
            d.hw = l.hw;
            d.clip_min = l.lo;
            hip_check(mlvc_hip_y0_tail(&d, stream_), "y0 tail launch");
            break;
        }
        case Launch::kY1: {
            mlvc_hip_y1_tail_desc d{};
            d.normalized = ptr(l.ins[0], parity);
            d.prior = ptr(l.ins[1], parity);
            d.quant_scale = ptr(l.ins[2], parity);
            d.update_scale0 = ptr(l.ins[3], parity);
            d.update_scale1 = ptr(l.ins[4], parity);
            d.concat2 = ptr(l.ins[5], parity);
            d.clipped = ptr(l.ins[6], parity);
            d.y_raw = ptr(l.outs[0], parity);
            d.out = ptr(l.y, parity);
            d.n = l.n;
            d.q = l.c;
            d.hw = l.hw;
            hip_check(mlvc_hip_y1_tail(&d, stream_), "y1 tail launch");
            break;
        }
        }
    }

    // Fills every activation buffer (arena, graph inputs, state) with FP16
    // values in [-1, 1) (pattern = true: matrix cores fed zeros run cooler and
    // faster than on real data, which can rank tile variants differently) or
    // zeros.
    void fill_buffers(bool pattern)
    {
        unsigned seed = 1;
        auto fill = [&](void* p, std::size_t bytes, const char* what) {
            bytes &= ~std::size_t{1};
            if (!p || bytes == 0) return;
            hip_check(pattern ? mlvc_hip_fill_pattern(p, bytes, seed++, stream_) : mlvc_hip_zero(p, bytes, stream_), what);
        };
        fill(arena_.ptr, arena_bytes_, "arena fill");
        for (auto& [id, buf] : input_buf_) fill(buf.ptr, desc_bytes(desc(id)), "input fill");
        for (auto& b : bindings_)
            for (auto& buf : b.buf) fill(buf.ptr, b.bytes, "state fill");
    }

    // Measures every eligible tile variant of each conv launch on the real
    // buffers (filled with an FP16 pattern first, zeroed again afterwards) and
    // keeps the fastest. All variants of one kernel size share the K order, so
    // the choice changes timing, never results.
    void tune()
    {
        select();
        fill_buffers(true);
        constexpr int kWarm = 2, kReps = 5;
        // MLVC_HIP_TUNE_FILE=<path>: choices listed there ("<model>:<launch>
        // <variant>" per line) are taken without timing, so separate
        // processes (one counter pass each, or a benchmark and its profile)
        // run the same kernels. The file is only read, unless
        // MLVC_HIP_TUNE_WRITE=1 asks for every choice to be written back
        // (to a temporary file renamed into place, so a reader never sees a
        // partial file).
        const char* tune_file = std::getenv("MLVC_HIP_TUNE_FILE");
        const char* tune_write = std::getenv("MLVC_HIP_TUNE_WRITE");
        const bool write_back = tune_file && tune_write && std::string(tune_write) == "1";
        // MLVC_HIP_TUNE_VERBOSE=1 prints every candidate's time per launch.
        const char* verbose_env = std::getenv("MLVC_HIP_TUNE_VERBOSE");
        const bool tune_verbose = verbose_env && std::string(verbose_env) == "1";
        std::map<std::string, std::string> chosen;
        if (tune_file) {
            std::ifstream in(tune_file);
            std::string launch, variant;
            while (in >> launch >> variant) chosen[launch] = variant;
        }
        for (auto& lp : launches_) {
            Launch& L = *lp;
            if (L.kind != Launch::kConv || L.forced) continue;
            int count = 0;
            hip_check(mlvc_hip_conv_candidates(&L.conv, nullptr, 0, &count), "conv candidates");
            if (count < 2) continue;
            std::vector<int> cand(static_cast<std::size_t>(count));
            hip_check(mlvc_hip_conv_candidates(&L.conv, cand.data(), count, &count), "conv candidates");
            const mlvc_hip_conv_desc planned = L.conv;
            int best = planned.variant;
            float best_ms = -1.0F;
            const std::string key = model_ + ":" + L.name;
            if (const auto it = chosen.find(key); it != chosen.end()) {
                for (int v : cand)
                    if (it->second == mlvc_hip_conv_variant_name(v)) {
                        best = v;
                        best_ms = 0.0F;
                    }
                if (best_ms == 0.0F)
                    cand.clear();
                else
                    std::fprintf(stderr, "hip: tuning file names variant %s for %s, which cannot run it; timing the candidates\n",
                                 it->second.c_str(), key.c_str());
            }
            for (int v : cand) {
                mlvc_hip_conv_desc d = planned;
                d.variant = v;
                DeviceMem w, b;
                pack_conv(L, w, b, d);
                upload_parameters();
                std::swap(L.packed, w);
                std::swap(L.bias, b);
                L.conv = d;
                for (int r = 0; r < kWarm; ++r) enqueue_one(L, 0);
                hip_check(mlvc_hip_event_record(ev0_, stream_), "event record");
                for (int r = 0; r < kReps; ++r) enqueue_one(L, 0);
                hip_check(mlvc_hip_event_record(ev1_, stream_), "event record");
                hip_check(mlvc_hip_event_synchronize(ev1_), "event sync");
                float ms = 0.0F;
                hip_check(mlvc_hip_event_elapsed_ms(ev0_, ev1_, &ms), "event timing");
                std::swap(L.packed, w);
                std::swap(L.bias, b);
                if (tune_verbose)
                    std::fprintf(stderr, "hip tune %s %s %.2f us\n", key.c_str(), mlvc_hip_conv_variant_name(v),
                                 1e3 * ms / kReps);
                if (best_ms < 0.0F || ms < best_ms) {
                    best_ms = ms;
                    best = v;
                }
            }
            L.conv = planned;
            if (best != planned.variant) {
                L.conv.variant = best;
                pack_conv(L, L.packed, L.bias, L.conv);
                upload_parameters();
                const std::string old_name = mlvc_hip_conv_variant_name(planned.variant);
                L.kind_name = mlvc_hip_conv_variant_name(best) + L.kind_name.substr(old_name.size());
            }
            chosen[key] = mlvc_hip_conv_variant_name(best);
        }
        fill_buffers(false);
        hip_check(mlvc_hip_stream_synchronize(stream_), "stream sync");
        if (write_back) {
            const std::string tmp = std::string(tune_file) + ".tmp" + std::to_string(static_cast<long>(::getpid()));
            {
                std::ofstream out(tmp, std::ios::trunc);
                for (const auto& [launch, variant] : chosen) out << launch << ' ' << variant << '\n';
                if (!out.flush()) fail("cannot write tuning file " + tmp);
            }
            if (std::rename(tmp.c_str(), tune_file) != 0) {
                std::remove(tmp.c_str());
                fail(std::string("cannot replace tuning file ") + tune_file);
            }
        }
    }

    static bool tuning_enabled()
    {
        const char* e = std::getenv("MLVC_HIP_TUNE");
        return !(e && std::string(e) == "0");
    }

    void capture()
    {
        const int parities = bindings_.empty() ? 1 : 2;
        for (int p = 0; p < parities; ++p) {
            hip_check(mlvc_hip_capture_begin(stream_), "graph capture begin");
            try {
                for (auto& l : launches_) enqueue_one(*l, p);
            } catch (...) {
                mlvc_hip_graph g = nullptr;
                mlvc_hip_capture_end(stream_, &g);
                if (g) mlvc_hip_graph_destroy(g);
                throw;
            }
            mlvc_hip_graph g = nullptr;
            hip_check(mlvc_hip_capture_end(stream_, &g), "graph capture end");
            graphs_.push_back(g);
        }
    }

    void enqueue_downloads()
    {
        for (std::size_t i = 0; i < ext_out_.size(); ++i)
            hip_check(mlvc_hip_memcpy_d2h(out_stage_[i].ptr, ptr(ext_out_[i], parity_), desc_bytes(desc(ext_out_[i])), stream_),
                      "output download");
    }

    struct CodecSlot {
        HostMem frame;            // encoder input / decoder output frame (I420)
        std::vector<HostMem> io;  // encoder: external outputs; decoder: external inputs (not q)
        HostMem q;                // q_index_shifted staging
        mlvc_hip_event done = nullptr;
        bool pending = false;
    };

    static TensorDataType public_dtype(aot::DataType t)
    {
        return t == aot::DataType::INT32 ? TensorDataType::kInt32 : TensorDataType::kFloat16;
    }

    CodecSlot& idle_slot(std::size_t index, bool encoder, const char* side)
    {
        return const_cast<CodecSlot&>(static_cast<const Plan*>(this)->idle_slot(index, encoder, side));
    }

    const CodecSlot& idle_slot(std::size_t index, bool encoder, const char* side) const
    {
        if (!codec_on_ || codec_encoder_ != encoder) fail(std::string(side) + " codec I/O is unavailable");
        if (index >= slots_.size()) fail("codec slot is out of range");
        const CodecSlot& sl = slots_[index];
        if (sl.pending) fail(std::string(side) + " codec slot is pending");
        return sl;
    }

    MutableYuv420FrameView frame_view(CodecSlot& sl) const
    {
        auto* b = static_cast<std::uint8_t*>(sl.frame.ptr);
        const std::size_t ysz = static_cast<std::size_t>(codec_.width) * codec_.height, uvsz = ysz / 4;
        return MutableYuv420FrameView(codec_.width, codec_.height, std::span<std::uint8_t>(b, ysz),
                                      std::span<std::uint8_t>(b + ysz, uvsz), std::span<std::uint8_t>(b + ysz + uvsz, uvsz));
    }

    Yuv420FrameView frame_view(const CodecSlot& sl) const { return frame_view(const_cast<CodecSlot&>(sl)); }

    void enqueue_q(CodecSlot& sl, int shifted_q)
    {
        const std::int32_t q32 = static_cast<std::int32_t>(shifted_q);
        std::memcpy(sl.q.ptr, &q32, sizeof(q32));
        hip_check(mlvc_hip_memcpy_h2d(input_buf_.at(ext_in_[static_cast<std::size_t>(codec_q_)]).ptr, sl.q.ptr, sizeof(q32), stream_),
                  "q upload");
    }

    void finish_submit(CodecSlot& sl)
    {
        advance();
        hip_check(mlvc_hip_event_record(sl.done, stream_), "event record");
        sl.pending = true;
    }

    int device_;
    std::string model_;
    aot::LoadedGraph graph_;
    mlvc_hip_stream stream_ = nullptr;
    mlvc_hip_event ev0_ = nullptr, ev1_ = nullptr;
    void ensure_flush_buffer(std::size_t flush_bytes)
    {
        if (flush_bytes == 0 || flush_bytes == flush_bytes_) return;
        if (flush_buf_) hip_check(mlvc_hip_free(flush_buf_), "flush buffer release");
        flush_buf_ = nullptr;
        flush_bytes_ = 0;
        hip_check(mlvc_hip_malloc(&flush_buf_, flush_bytes), "flush buffer allocation");
        flush_bytes_ = flush_bytes;
    }

    std::vector<mlvc_hip_event> frame_evs_;  // time_frames_each: start/stop per frame
    void* flush_buf_ = nullptr;              // time_frames_each: cache-flush copy buffer
    std::size_t flush_bytes_ = 0;
    std::vector<Binding> bindings_;
    std::map<TensorId, std::size_t> state_in_, state_out_;
    std::vector<TensorId> ext_in_, ext_out_;
    std::vector<std::unique_ptr<Launch>> launches_;
    std::vector<std::pair<void*, std::vector<std::uint8_t>>> pending_uploads_;
    std::map<TensorId, std::size_t> offset_;
    std::size_t arena_bytes_ = 0;
    DeviceMem arena_;
    // FP32 partials of the split-K convs: one buffer for all of them (they
    // run one after another on the stream), sized for the largest.
    std::size_t workspace_bytes_ = 0;
    DeviceMem workspace_;
    std::map<TensorId, DeviceMem> input_buf_;
    std::map<TensorId, DeviceMem> const_buf_;  // initializers read by elementwise / layout operators
    std::map<TensorId, int> consumers_;
    std::vector<std::pair<std::size_t, std::size_t>> gather_checks_;  // (external input, axis length)
    std::vector<HostMem> in_stage_, out_stage_;
    std::vector<mlvc_hip_graph> graphs_;
    int parity_ = 0;
    bool initialized_ = false;
    // codec I/O
    bool codec_on_ = false, codec_encoder_ = false;
    CodecIoConfig codec_{};
    std::size_t codec_frame_bytes_ = 0;
    int codec_q_ = -1, codec_img_ = -1;  // external input index of q; of x (encoder) / output index of x_hat (decoder)
    DeviceMem codec_frame_, codec_lut_;
    std::vector<CodecSlot> slots_;
};

HipBackend::HipBackend(BackendOptions options) : options_(std::move(options))
{
    if (!options_.allow_cpu_fallback && (options_.execution_preference == ExecutionPreference::kCpu ||
                                         options_.execution_preference == ExecutionPreference::kNpu))
        fail("disallowed by strict non-GPU execution preference");
}

HipBackend::~HipBackend() = default;

Plan& HipBackend::require_plan(const char* caller) const
{
    if (!plan_) fail(std::string("load() must be called before ") + caller);
    return *plan_;
}

void HipBackend::load(const std::string& model_name, const ModelExecutionConfig& config)
{
    plan_.reset();
    plan_ = std::make_unique<Plan>(options_, model_name, config);
}

std::vector<Tensor> HipBackend::run(const std::vector<Tensor>& inputs) { return require_plan("run()").run(inputs); }
void HipBackend::reset_state() { require_plan("reset_state()").reset_state(); }
std::vector<std::vector<std::int64_t>> HipBackend::io_shapes(bool outputs) const { return require_plan("io_shapes()").io_shapes(outputs); }
void HipBackend::upload_inputs(const std::vector<const void*>& inputs) { require_plan("upload_inputs()").upload_inputs(inputs); }
std::vector<TensorDataType> HipBackend::io_dtypes(bool outputs) const { return require_plan("io_dtypes()").io_dtypes(outputs); }
void HipBackend::configure_codec_io(const CodecIoConfig& config) { require_plan("configure_codec_io()").configure_codec_io(config); }
std::size_t HipBackend::codec_slot_count() const noexcept { return plan_ ? plan_->codec_slot_count() : 0U; }
MutableYuv420FrameView HipBackend::encoder_input_yuv(std::size_t slot) { return require_plan("encoder_input_yuv()").encoder_input_yuv(slot); }
void HipBackend::submit_encoder(std::size_t slot, int q) { require_plan("submit_encoder()").submit_encoder(slot, q); }
std::vector<TensorView> HipBackend::encoder_outputs(std::size_t slot) const { return require_plan("encoder_outputs()").encoder_outputs(slot); }
std::vector<MutableTensorView> HipBackend::decoder_inputs(std::size_t slot) { return require_plan("decoder_inputs()").decoder_inputs(slot); }
void HipBackend::submit_decoder(std::size_t slot, int q) { require_plan("submit_decoder()").submit_decoder(slot, q); }
Yuv420FrameView HipBackend::decoder_output_yuv(std::size_t slot) const { return require_plan("decoder_output_yuv()").decoder_output_yuv(slot); }
void HipBackend::wait_codec_slot(std::size_t slot) { require_plan("wait_codec_slot()").wait_codec_slot(slot); }
float HipBackend::time_frames(int frames) { return require_plan("time_frames()").time_frames(frames); }
void HipBackend::time_frames_each(int frames, std::size_t flush_bytes, float* ms_each)
{
    require_plan("time_frames_each()").time_frames_each(frames, flush_bytes, ms_each);
}
void HipBackend::download_outputs(const std::vector<std::uint16_t*>& outputs) { require_plan("download_outputs()").download_outputs(outputs); }
std::size_t HipBackend::launch_count() const { return require_plan("launch_count()").launch_count(); }
LaunchInfo HipBackend::launch_info(std::size_t index) const { return require_plan("launch_info()").launch_info(index); }
float HipBackend::time_launch(std::size_t index, int reps) { return require_plan("time_launch()").time_launch(index, reps); }

void HipBackend::time_launch_cold(std::size_t index, int reps, std::size_t flush_bytes, float* ms_each)
{
    require_plan("time_launch_cold()").time_launch_cold(index, reps, flush_bytes, ms_each);
}

void register_hip_backend(bool make_default)
{
    register_backend(
        "hip", [](const BackendOptions& o) { return std::make_unique<HipBackend>(o); }, make_default);
}

}  // namespace mlvc::hip_backend
