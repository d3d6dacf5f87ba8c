#pragma once
// Protobuf (proto3) wire codec for the schema-3 graph files, written without
// a protobuf library.
//
// Message and field numbers follow the reference schema
// proto/mlvc_model.proto:30-83 (Graph, TensorDescriptor, Node and the
// attribute/storage oneofs) and :85-107 (ModelMetadata). The reader accepts
// what a conforming protobuf parser accepts for these messages: fields in any
// order, unknown fields skipped, repeated scalars packed or unpacked, the
// last value winning for singular fields and the last-set member winning for
// a oneof. The writer emits the canonical deterministic encoding (fields in
// number order, packed repeated scalars, proto3 defaults omitted).

#include <cstddef>
#include <cstdint>
#include <optional>
#include <span>
#include <stdexcept>
#include <string>
#include <vector>

namespace mlvc::wire {

enum class AttrCase { kNone = 0, kConv = 4, kAxis = 5, kActivation = 6, kPixel = 7 };
enum class StorageCase { kNone = 0, kArena = 5, kWeight = 6 };

struct ConvAttributes {
    std::vector<std::uint32_t> strides, pads, dilations;
    std::uint32_t groups = 0;
};

struct Node {
    std::int32_t op = 0;
    std::vector<std::uint32_t> inputs, outputs;
    AttrCase attr_case = AttrCase::kNone;
    ConvAttributes conv;
    std::int32_t axis = 0;
    float alpha = 0.0F;
    std::uint32_t block_size = 0;
};

struct ArenaAllocation {
    std::uint64_t offset = 0, size_bytes = 0;
    std::uint32_t birth = 0, death = 0;
};

struct WeightLocation {
    std::uint64_t offset = 0, size_bytes = 0;
};

struct TensorDescriptor {
    std::uint32_t id = 0;
    std::string name;
    std::int32_t dtype = 0;
    std::vector<std::int64_t> shape;
    StorageCase storage_case = StorageCase::kNone;
    ArenaAllocation arena;
    WeightLocation weight;
};

struct Graph {
    std::uint32_t schema_version = 0;
    std::string checkpoint_sha256;
    std::vector<TensorDescriptor> tensors;
    std::vector<std::uint32_t> inputs, outputs;
    std::vector<Node> nodes;
    std::uint64_t arena_bytes = 0;
    std::uint32_t arena_alignment = 0;
    std::uint64_t weights_bytes = 0;
    std::string weights_sha256;
};

struct ModelMetadata {
    std::uint32_t schema_version = 0;
    std::string profile, model_version, checkpoint_sha256;
    std::uint32_t width = 0, height = 0;
    float pixel_range = 0.0F;
    std::uint32_t qp_num = 0, total_qp_num = 0;
    std::vector<std::uint32_t> frame_index_map;
    std::vector<std::int32_t> qp_shift;
    std::uint32_t feature_channels = 0, latent_channels = 0, hyperprior_channels = 0;
    std::uint32_t downsample_feature = 0, downsample_latent = 0, downsample_hyperprior = 0;
    std::uint32_t y_scale_repeat = 0;
    std::optional<std::uint32_t> iframe_period, reset_period;
    bool disable_feature_reset = false;
};

// model_bundle.pb (proto/mlvc_model.proto:135-161).
struct CodecContract {
    std::string container, entropy;
    std::uint32_t decoder_max_yuv_sample_error = 0;
    double decoder_min_psnr_db = 0.0;
};
struct Artifact {
    std::string path;
    std::uint64_t size_bytes = 0;
    std::string sha256;
};
struct ModelBundle {
    std::uint32_t schema_version = 0;
    std::string profile, model_version;
    std::uint32_t width = 0, height = 0;
    std::string checkpoint_sha256, entropy_model_sha256;
    CodecContract contract;
    std::vector<Artifact> artifacts;
};

// Throw std::runtime_error on malformed input.
Graph parse_graph(std::span<const std::byte> bytes);
ModelMetadata parse_metadata(std::span<const std::byte> bytes);
ModelBundle parse_bundle(std::span<const std::byte> bytes);

// A model file as the loaders read it (reference core/src/model_proto.hpp:11-23,
// runtime/src/aot_graph.cpp:95-106): empty or above 64 MiB is
// "invalid Protobuf model message size: <label>", a parse failure is
// "invalid Protobuf model message: <label>".
template <typename Parse>
auto parse_model_file(std::span<const std::byte> bytes, const std::string& label, Parse parse)
{
    constexpr std::size_t kLimit = 64U * 1024U * 1024U;
    if (bytes.empty() || bytes.size() > kLimit)
        throw std::runtime_error("invalid Protobuf model message size: " + label);
    try {
        return parse(bytes);
    } catch (const std::exception&) {
        throw std::runtime_error("invalid Protobuf model message: " + label);
    }
}

std::vector<std::byte> serialize(const Graph& graph);
std::vector<std::byte> serialize(const ModelMetadata& metadata);
std::vector<std::byte> serialize(const ModelBundle& bundle);

}  // namespace mlvc::wire
