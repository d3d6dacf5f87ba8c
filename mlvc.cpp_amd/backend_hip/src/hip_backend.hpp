#pragma once
// "hip" inference backend: runs schema-3 FP16 conv graphs on one MI355X.
//
// Sits beside the reference's backends/cpu and backends/driver_cubin behind
// mlvc::InferenceBackend. load() validates the graph, lowers it to a
// schedule of hand-written gfx950 kernels with fusions, plans device memory
// for that schedule and captures one hipGraph per state parity; run()
// uploads inputs, replays the frame's graph and downloads outputs.

#include "mlvc/runtime/aot_graph.hpp"
#include "mlvc/runtime/backend.hpp"

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace mlvc::hip_backend {

struct LaunchInfo {
    std::string name;
    std::string kind;
    double flops = 0.0;
    double bytes = 0.0;
};

class Plan;

class HipBackend final : public InferenceBackend, public BufferedCodecBackend {
public:
    explicit HipBackend(BackendOptions options);
    ~HipBackend() override;

    std::string_view name() const noexcept override { return "hip"; }
    void load(const std::string& model_name, const ModelExecutionConfig& config) override;
    std::vector<Tensor> run(const std::vector<Tensor>& inputs) override;
    void reset_state() override;

    // BufferedCodecBackend: pinned slots, GPU frame conversions around the
    // MLVCEncoder / MLVCDecoder graphs, stream-ordered submits.
    void configure_codec_io(const CodecIoConfig& config) override;
    std::size_t codec_slot_count() const noexcept override;
    MutableYuv420FrameView encoder_input_yuv(std::size_t slot) override;
    void submit_encoder(std::size_t slot, int shifted_q) override;
    std::vector<TensorView> encoder_outputs(std::size_t slot) const override;
    std::vector<MutableTensorView> decoder_inputs(std::size_t slot) override;
    void submit_decoder(std::size_t slot, int shifted_q) override;
    Yuv420FrameView decoder_output_yuv(std::size_t slot) const override;
    void wait_codec_slot(std::size_t slot) override;

    // External (non-state) graph inputs / outputs in graph order.
    std::vector<std::vector<std::int64_t>> io_shapes(bool outputs) const;
    std::vector<TensorDataType> io_dtypes(bool outputs) const;

    // Device-resident measurement helpers (inputs as raw host bytes).
    void upload_inputs(const std::vector<const void*>& inputs);
    float time_frames(int frames);
    void time_frames_each(int frames, std::size_t flush_bytes, float* ms_each);
    void download_outputs(const std::vector<std::uint16_t*>& outputs);
    std::size_t launch_count() const;
    LaunchInfo launch_info(std::size_t index) const;
    float time_launch(std::size_t index, int reps);
    // Per-launch times of `reps` single launches of kernel `index`, each after
    // a cache-evicting device copy of flush_bytes / 2 bytes outside its events.
    void time_launch_cold(std::size_t index, int reps, std::size_t flush_bytes, float* ms_each);

private:
    Plan& require_plan(const char* caller) const;

    BackendOptions options_;
    std::unique_ptr<Plan> plan_;
};

void register_hip_backend(bool make_default);

}  // namespace mlvc::hip_backend
