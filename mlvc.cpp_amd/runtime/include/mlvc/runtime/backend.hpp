#pragma once
// Backend-agnostic fixed-shape graph execution contract.
//
// Mirrors the reference's runtime/include/mlvc/runtime/backend.hpp:17-110 so
// that a backend written against it is a drop-in beside backends/cpu and
// backends/driver_cubin: BackendOptions, StateTensorBinding,
// ModelExecutionConfig, InferenceBackend (name/load/run/reset_state) and the
// named factory registry (register_backend/create_backend).

#include "mlvc/core/assets.hpp"
#include "mlvc/core/tensor.hpp"

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

using BackendFactory =
    std::function<std::unique_ptr<InferenceBackend>(const BackendOptions&)>;

void register_backend(std::string name, BackendFactory factory, bool make_default = false);
std::vector<std::string> available_backends();
std::string_view default_backend_name() noexcept;
std::unique_ptr<InferenceBackend> create_backend(const BackendOptions& options);

}  // namespace mlvc
