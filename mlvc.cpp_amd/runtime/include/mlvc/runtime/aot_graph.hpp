#pragma once
// AOT graph schema 3: typed operator schedule with integer tensor IDs,
// planned arena slots and 256-byte-aligned weights.
//
// The descriptor types and entry points keep the names and meaning of the
// reference's runtime/include/mlvc/runtime/aot_graph.hpp:16-125 (the operator
// contract that backends consume). decode_graph_binary applies the same
// validation rules as the reference's runtime/src/aot_graph.cpp:110-284 but
// parses the protobuf wire format with this library's own codec (wire.hpp), so
// no protobuf library is needed.

#include "mlvc/core/assets.hpp"

#include <array>
#include <cstddef>
#include <cstdint>
#include <filesystem>
#include <span>
#include <string>
#include <variant>
#include <vector>

namespace mlvc::aot {

using TensorId = std::uint32_t;

enum class Op {
    OP_UNSPECIFIED = 0,
    ADD = 1,
    SUB = 2,
    MUL = 3,
    CLIP = 4,
    CONCAT = 5,
    CONV = 6,
    DEPTH_TO_SPACE = 7,
    GATHER = 8,
    LEAKY_RELU = 9,
    RECIPROCAL = 10,
    ROUND = 11,
    SIGMOID = 12,
    SLICE = 13,
    SPACE_TO_DEPTH = 14,
};

enum class DataType { DATA_TYPE_UNSPECIFIED = 0, FP16 = 1, INT32 = 2, INT64 = 3 };

struct ConvAttributes {
    std::array<int, 2> strides{1, 1};
    std::array<int, 4> pads{0, 0, 0, 0};  // top, left, bottom, right
    std::array<int, 2> dilations{1, 1};
    int groups = 1;
};
struct AxisAttributes { int axis = 0; };
struct ActivationAttributes { float alpha = 0.01F; };
struct PixelAttributes { int block_size = 1; };

struct Node {
    std::size_t index = 0;
    Op op = Op::OP_UNSPECIFIED;
    std::vector<TensorId> inputs;
    std::vector<TensorId> outputs;
    std::variant<std::monostate, ConvAttributes, AxisAttributes, ActivationAttributes,
                 PixelAttributes>
        attributes;

    const ConvAttributes& conv() const { return std::get<ConvAttributes>(attributes); }
    int axis() const { return std::get<AxisAttributes>(attributes).axis; }
    float alpha() const { return std::get<ActivationAttributes>(attributes).alpha; }
    int block_size() const { return std::get<PixelAttributes>(attributes).block_size; }
};

struct ArenaSlot {
    std::size_t offset = 0;
    std::size_t bytes = 0;
    std::size_t birth = 0;
    std::size_t death = 0;
};

struct WeightLocation {
    std::size_t offset = 0;
    std::size_t bytes = 0;
};

struct TensorDescriptor {
    std::string name;  // empty = unused ID
    DataType dtype = DataType::DATA_TYPE_UNSPECIFIED;
    std::vector<std::int64_t> shape;
    std::variant<std::monostate, ArenaSlot, WeightLocation> storage;
};

struct GraphDescriptor {
    std::vector<Node> nodes;
    std::vector<TensorDescriptor> tensors;  // dense ID table; slot 0 is invalid
    std::vector<TensorId> inputs;
    std::vector<TensorId> outputs;
    std::size_t arena_bytes = 0;
    std::size_t weights_bytes = 0;
};

struct LoadedGraph {
    GraphDescriptor descriptor;
    std::vector<std::byte> weights;
};

std::size_t dtype_bytes(DataType dtype);

GraphDescriptor decode_graph_binary(std::span<const std::byte> bytes);
LoadedGraph load_aot_graph(const ModelAssetReader& assets, const std::string& model_name);
LoadedGraph load_aot_graph(const std::filesystem::path& model_dir,
                           const std::string& model_name);

}  // namespace mlvc::aot
