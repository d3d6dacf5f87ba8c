#pragma once
// Backend-agnostic fixed-shape graph execution and codec I/O contracts.
//
// Mirrors the reference's runtime/include/mlvc/runtime/backend.hpp:17-110 so
// that a backend written against it is a drop-in beside backends/cpu and
// backends/driver_cubin: BackendOptions, StateTensorBinding,
// ModelExecutionConfig, InferenceBackend (name/load/run/reset_state), the
// optional BufferedCodecBackend with CodecIoConfig, and the named factory
// registry (register_backend/create_backend).

#include "mlvc/core/assets.hpp"
#include "mlvc/core/tensor.hpp"
#include "mlvc/core/yuv.hpp"

#include <cstddef>
#include <cstdint>
#include <functional>
#include <memory>
#include <string>
#include <string_view>
#include <vector>

namespace mlvc {

enum class ExecutionPreference { kAuto, kCpu, kGpu, kNpu };

struct BackendOptions {
    std::string model_dir;
    int device_id = 0;
    int num_threads = 0;  // 0 = automatic
    ExecutionPreference execution_preference = ExecutionPreference::kAuto;
    bool allow_cpu_fallback = true;
    std::string backend_name;
    std::shared_ptr<const ModelAssetReader> asset_reader;
};

// Routes graph output `output_index` of one run() into graph input
// `input_index` of the next. Both disappear from run()'s tensor lists and
// reset_state() zeroes the carried value.
struct StateTensorBinding {
    std::size_t input_index = 0;
    std::size_t output_index = 0;
    TensorDataType data_type = TensorDataType::kFloat16;
    std::vector<std::int64_t> shape;
};

struct ModelExecutionConfig {
    std::vector<StateTensorBinding> state_bindings;
};

class InferenceBackend {
public:
    virtual ~InferenceBackend() = default;
    virtual std::string_view name() const noexcept = 0;
    virtual void load(const std::string& model_name, const ModelExecutionConfig& config) = 0;
    // Inputs and outputs keep graph order with bound state tensors removed.
    virtual std::vector<Tensor> run(const std::vector<Tensor>& inputs) = 0;
    virtual void reset_state() = 0;
};

// Optional fast path of fixed-shape backends (contract of the reference's
// backend.hpp:64-96): persistent pinned host slots and the frame <-> model
// image conversions run around inference in stream order. A slot's views
// stay valid until the slot is submitted again; a submitted slot must be
// waited before its buffers are read, written or resubmitted.
struct CodecIoConfig {
    int width = 0;
    int height = 0;
    int model_width = 0;
    int model_height = 0;
    float pixel_range = 1.0F;
    FramePadding padding;
    std::size_t slots = 2;
};

class BufferedCodecBackend {
public:
    virtual ~BufferedCodecBackend() = default;

    virtual void configure_codec_io(const CodecIoConfig& config) = 0;
    virtual std::size_t codec_slot_count() const noexcept = 0;

    virtual MutableYuv420FrameView encoder_input_yuv(std::size_t slot) = 0;
    virtual void submit_encoder(std::size_t slot, int shifted_q) = 0;
    virtual std::vector<TensorView> encoder_outputs(std::size_t slot) const = 0;

    virtual std::vector<MutableTensorView> decoder_inputs(std::size_t slot) = 0;
    virtual void submit_decoder(std::size_t slot, int shifted_q) = 0;
    virtual Yuv420FrameView decoder_output_yuv(std::size_t slot) const = 0;

    virtual void wait_codec_slot(std::size_t slot) = 0;
};

using BackendFactory =
    std::function<std::unique_ptr<InferenceBackend>(const BackendOptions&)>;

void register_backend(std::string name, BackendFactory factory, bool make_default = false);
std::vector<std::string> available_backends();
std::string_view default_backend_name() noexcept;
std::unique_ptr<InferenceBackend> create_backend(const BackendOptions& options);

}  // namespace mlvc
