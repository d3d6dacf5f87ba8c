#pragma once
// Writer for schema-3 model directories (aot/<model>/graph.pb, weights.bin,
// metadata.pb).
//
// Plays the role of the reference's offline graph writer
// (tools/python/mlvc_tools/aot.py:233-278, wire.py:100-137) for synthetic
// graphs: tensors get dense IDs, weights are placed at 256-byte offsets and
// activations get arena slots from a lifetime planner with the semantics of
// aot.py:45-87 (a slot is reusable once its last consumer has run;
// best-fit reuse of freed, coalesced blocks; graph outputs live to the end).

#include "mlvc/core/assets.hpp"
#include "mlvc/core/tensor.hpp"
#include "mlvc/runtime/aot_graph.hpp"
#include "mlvc/runtime/backend.hpp"
#include "mlvc/runtime/wire.hpp"

#include <array>
#include <cstdint>
#include <filesystem>
#include <memory>
#include <string>
#include <vector>

namespace mlvc::synth {

class GraphBuilder {
public:
    using Id = std::uint32_t;
    using Shape = std::vector<std::int64_t>;

    Id input(const std::string& name, const Shape& shape, aot::DataType dtype = aot::DataType::FP16);
    Id weight_fp16(const std::string& name, const Shape& shape, const std::vector<Float16Storage>& values);
    Id weight_int64(const std::string& name, const Shape& shape, const std::vector<std::int64_t>& values);

    // groups == 1 or depthwise (groups == Cin == Cout). Output shape is derived.
    Id conv(const std::string& name, Id x, Id w, Id b, std::array<int, 2> stride,
            std::array<int, 2> pad, int groups = 1);
    Id leaky_relu(const std::string& name, Id x, float alpha = 0.01F);
    Id binary(aot::Op op, const std::string& name, Id a, Id b);
    Id pixel(aot::Op op, const std::string& name, Id x, int block);
    Id concat(const std::string& name, const std::vector<Id>& xs, int axis);
    Id unary(aot::Op op, const std::string& name, Id x);
    // CLIP with FP16 scalar initializers `lo` / `hi` (0 = unbounded side).
    Id clip(const std::string& name, Id x, Id lo, Id hi);
    // SLICE with INT64 initializers; `axes` / `steps` may be empty (absent).
    Id slice(const std::string& name, Id x, const std::vector<std::int64_t>& starts, const std::vector<std::int64_t>& ends,
             const std::vector<std::int64_t>& axes = {}, const std::vector<std::int64_t>& steps = {});
    Id gather(const std::string& name, Id data, Id indices, int axis);

    void output(Id id) { outputs_.push_back(id); }
    // Model description written to metadata.pb (profile and checkpoint hash
    // are filled by build()); unset, a minimal placeholder is written.
    void set_metadata(const wire::ModelMetadata& m) { metadata_ = m; has_metadata_ = true; }
    const Shape& shape(Id id) const { return tensors_.at(id - 1).shape; }
    std::size_t node_count() const { return nodes_.size(); }

    struct Files {
        std::vector<std::byte> graph_pb, weights_bin, metadata_pb;
    };
    // Plans the arena, serialises the graph and computes SHA-256 provenance.
    Files build(const std::string& profile) const;
    // Writes aot/<model>/{graph.pb,weights.bin}, metadata.pb and
    // model_bundle.pb (the bundle's artifact list keeps the entries of other
    // graphs already written to the same directory).
    void write_directory(const std::filesystem::path& dir, const std::string& model_name,
                         const std::string& profile) const;
    std::shared_ptr<const ModelAssetReader> to_memory(const std::string& model_name,
                                                      const std::string& profile) const;

private:
    struct T {
        std::string name;
        aot::DataType dtype;
        Shape shape;
        bool is_weight = false;
        std::uint64_t w_offset = 0, w_bytes = 0;
    };
    struct N {
        aot::Op op = aot::Op::OP_UNSPECIFIED;
        std::vector<Id> inputs;
        Id output = 0;
        wire::AttrCase attr = wire::AttrCase::kNone;
        wire::ConvAttributes conv;
        int axis = 0;
        float alpha = 0.0F;
        int block = 0;
    };
    static N make_node(aot::Op op, std::vector<Id> inputs)
    {
        N n;
        n.op = op;
        n.inputs = std::move(inputs);
        return n;
    }
    Id add_tensor(const std::string& name, aot::DataType dtype, const Shape& shape);
    Id add_node(N node, const Shape& out_shape, const std::string& out_name);

    std::vector<T> tensors_;
    std::vector<N> nodes_;
    std::vector<Id> inputs_, outputs_;
    std::vector<std::byte> weights_;
    wire::ModelMetadata metadata_;
    bool has_metadata_ = false;
};

// SHA-256 (FIPS 180-4), used for the weights_sha256 provenance field.
std::array<std::uint8_t, 32> sha256(const void* data, std::size_t size);

// Deterministic generator: SplitMix64 stream, uniform doubles in [0,1) from
// the top 53 bits, normals by Box-Muller in double.
class Rng {
public:
    explicit Rng(std::uint64_t seed) : state_(seed) {}
    std::uint64_t next();
    double uniform();
    double normal();

private:
    std::uint64_t state_;
    bool have_spare_ = false;
    double spare_ = 0.0;
};

// Synthetic workloads. `config` is one of: "conv3x3_184x320" (single 3x3
// conv + bias + LeakyReLU), "conv_sweep_640x368", "dwblock_92x160_c128",
// "dwblock_46x80_c256", "mlvc_s_640x368", "mlvc_1920x1088", plus the
// scaled-down "mlvc_s_tiny" (same topology at 64x32) used for quick parity.
struct SyntheticModel {
    std::string model_name;
    std::string profile;  // metadata checkpoint id; graphs of one model directory share it
    std::vector<StateTensorBinding> state_bindings;
    std::vector<std::vector<std::int64_t>> external_inputs;  // graph order, bound state removed
    std::vector<std::string> external_input_names;
    std::vector<double> input_lo, input_hi;  // uniform range per external input
    int frames = 1;
};

GraphBuilder build_synthetic(const std::string& config, std::uint64_t seed, SyntheticModel* info);
std::vector<std::string> synthetic_configs();
SyntheticModel synthetic_info(const std::string& config);
// FP16 uniform input for (config, external input index, frame, seed).
std::vector<Float16Storage> synthetic_input(const std::string& config, std::size_t input_index,
                                            int frame, std::uint64_t seed);

}  // namespace mlvc::synth
