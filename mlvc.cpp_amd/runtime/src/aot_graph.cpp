// Schema-3 graph decoding and validation.
//
// The acceptance rules restate the reference's runtime/src/aot_graph.cpp:
// schema == 3 and 32-byte SHA provenance (:112-115), tensor count (:116),
// non-empty graph (:118-120), arena alignment 256 (:121), dense unique
// tensor IDs and names (:129-135), rank <= 4 and positive extents
// (:139-148), weight extent and 256-byte offset alignment (:149-156), arena
// extent and lifetime bounds (:158-170), graph inputs without storage
// (:181-187), per-operator operand contracts (:196-255), absent-operand
// rules (:256-266), one arena output born at its producing node (:267-273)
// and unique graph outputs (:277-282). Loading follows :291-317: graph.pb
// and metadata.pb checkpoint SHAs must agree and weights.bin must have the
// declared size.

#include "mlvc/runtime/aot_graph.hpp"
#include "mlvc/runtime/wire.hpp"

#include <cmath>
#include <limits>
#include <stdexcept>
#include <unordered_set>

namespace mlvc::aot {
namespace {

void require(bool ok, const char* what)
{
    if (!ok)
        throw std::runtime_error(std::string("invalid AOT Protobuf graph: ") + what);
}

int positive_int(std::uint32_t v)
{
    require(v > 0 && v <= static_cast<std::uint32_t>(std::numeric_limits<int>::max()),
            "invalid positive attribute");
    return static_cast<int>(v);
}

template <std::size_t N>
std::array<int, N> dims(const std::vector<std::uint32_t>& v, bool positive)
{
    require(v.size() == N, "attribute dimension count");
    std::array<int, N> out{};
    for (std::size_t i = 0; i < N; ++i) {
        require(v[i] <= static_cast<std::uint32_t>(std::numeric_limits<int>::max()) &&
                    (!positive || v[i] > 0),
                "invalid attribute dimension");
        out[i] = static_cast<int>(v[i]);
    }
    return out;
}

DataType to_dtype(std::int32_t v)
{
    require(v >= 1 && v <= 3, "unsupported dtype");
    return static_cast<DataType>(v);
}

Op to_op(std::int32_t v)
{
    require(v >= 1 && v <= 14, "unknown operator");
    return static_cast<Op>(v);
}

GraphDescriptor decode(const wire::Graph& g)
{
    require(g.schema_version == 3, "unsupported schema");
    require(g.checkpoint_sha256.size() == 32 && g.weights_sha256.size() == 32,
            "missing SHA-256 provenance");
    require(!g.tensors.empty() && g.tensors.size() <= 1000000, "tensor count");
    require(!g.nodes.empty() && !g.inputs.empty() && !g.outputs.empty(), "empty graph");
    require(g.arena_alignment == 256 && g.arena_bytes > 0, "arena configuration");

    GraphDescriptor r;
    r.arena_bytes = g.arena_bytes;
    r.weights_bytes = g.weights_bytes;
    r.tensors.resize(g.tensors.size() + 1);
    std::unordered_set<std::string> names;
    for (const wire::TensorDescriptor& in : g.tensors) {
        require(in.id > 0 && in.id < r.tensors.size(), "tensor ID range");
        TensorDescriptor& t = r.tensors[in.id];
        require(t.name.empty() && !in.name.empty() && names.insert(in.name).second,
                "duplicate tensor ID or name");
        t.name = in.name;
        t.dtype = to_dtype(in.dtype);
        t.shape = in.shape;
        require(t.shape.size() <= 4, "tensor rank");
        std::size_t bytes = dtype_bytes(t.dtype);
        for (const std::int64_t d : t.shape) {
            require(d > 0 && static_cast<std::uint64_t>(d) <=
                                 std::numeric_limits<std::size_t>::max() / bytes,
                    "tensor extent overflow");
            bytes *= static_cast<std::size_t>(d);
        }
        if (in.storage_case == wire::StorageCase::kWeight) {
            const auto& w = in.weight;
            require(t.dtype != DataType::INT32 && w.offset % 256 == 0 && w.size_bytes == bytes &&
                        w.offset <= r.weights_bytes && w.size_bytes <= r.weights_bytes - w.offset,
                    "weight extent");
            t.storage = WeightLocation{w.offset, w.size_bytes};
        } else {
            require(t.dtype != DataType::INT64, "runtime int64 tensor");
            if (in.storage_case == wire::StorageCase::kArena) {
                const auto& a = in.arena;
                require(a.offset % 256 == 0 && a.size_bytes >= bytes && a.offset <= r.arena_bytes &&
                            a.size_bytes <= r.arena_bytes - a.offset && a.birth <= a.death &&
                            a.death <= g.nodes.size(),
                        "arena extent");
                t.storage = ArenaSlot{a.offset, a.size_bytes, a.birth, a.death};
            }
        }
    }

    auto valid = [&](TensorId id) {
        return id > 0 && id < r.tensors.size() && !r.tensors[id].name.empty();
    };
    std::unordered_set<TensorId> available;
    for (const wire::TensorDescriptor& in : g.tensors)
        if (in.storage_case == wire::StorageCase::kWeight)
            available.insert(in.id);
    for (const TensorId id : g.inputs) {
        require(valid(id) && std::holds_alternative<std::monostate>(r.tensors[id].storage) &&
                    available.insert(id).second,
                "input ID or storage");
        r.inputs.push_back(id);
    }

    for (const wire::Node& in : g.nodes) {
        Node n;
        n.index = r.nodes.size();
        n.op = to_op(in.op);
        n.inputs = in.inputs;
        n.outputs = in.outputs;
        const std::size_t count = n.inputs.size();
        const bool no_attr = in.attr_case == wire::AttrCase::kNone;
        switch (n.op) {
        case Op::CONV: {
            require(in.attr_case == wire::AttrCase::kConv && (count == 2 || count == 3),
                    "convolution contract");
            ConvAttributes c;
            c.strides = dims<2>(in.conv.strides, true);
            c.pads = dims<4>(in.conv.pads, false);
            c.dilations = dims<2>(in.conv.dilations, true);
            c.groups = positive_int(in.conv.groups);
            n.attributes = c;
            require(c.dilations == std::array<int, 2>{1, 1}, "unsupported dilation");
            require(c.pads[0] == c.pads[2] && c.pads[1] == c.pads[3],
                    "asymmetric convolution padding");
            break;
        }
        case Op::CONCAT:
        case Op::GATHER:
            require(in.attr_case == wire::AttrCase::kAxis &&
                        (n.op == Op::CONCAT ? count > 0 : count == 2),
                    "axis contract");
            n.attributes = AxisAttributes{in.axis};
            break;
        case Op::LEAKY_RELU:
            require(in.attr_case == wire::AttrCase::kActivation && count == 1 &&
                        std::isfinite(in.alpha),
                    "activation contract");
            n.attributes = ActivationAttributes{in.alpha};
            break;
        case Op::SPACE_TO_DEPTH:
        case Op::DEPTH_TO_SPACE:
            require(in.attr_case == wire::AttrCase::kPixel && count == 1, "pixel layout contract");
            n.attributes = PixelAttributes{positive_int(in.block_size)};
            break;
        case Op::ADD:
        case Op::SUB:
        case Op::MUL:
            require(no_attr && count == 2, "binary contract");
            break;
        case Op::CLIP:
            require(no_attr && count >= 1 && count <= 3, "clip contract");
            break;
        case Op::SLICE:
            require(no_attr && count >= 3 && count <= 5, "slice contract");
            break;
        case Op::RECIPROCAL:
        case Op::ROUND:
        case Op::SIGMOID:
            require(no_attr && count == 1, "unary contract");
            break;
        default:
            require(false, "unknown operator");
        }
        for (std::size_t i = 0; i < count; ++i) {
            if (n.inputs[i] == 0) {
                require((n.op == Op::CONV && i == 2) || (n.op == Op::CLIP && i > 0) ||
                            (n.op == Op::SLICE && i > 2),
                        "absent required operand");
            } else {
                require(valid(n.inputs[i]) && available.contains(n.inputs[i]), "unresolved operand");
            }
        }
        require(n.outputs.size() == 1 && valid(n.outputs[0]), "output ID");
        const TensorId out = n.outputs[0];
        require(std::holds_alternative<ArenaSlot>(r.tensors[out].storage) &&
                    available.insert(out).second,
                "duplicate output or missing arena");
        require(std::get<ArenaSlot>(r.tensors[out].storage).birth == n.index, "tensor birth");
        r.nodes.push_back(std::move(n));
    }

    std::unordered_set<TensorId> seen_outputs;
    for (const TensorId id : g.outputs) {
        require(valid(id) && available.contains(id) && seen_outputs.insert(id).second,
                "graph output");
        r.outputs.push_back(id);
    }
    return r;
}

}  // namespace

std::size_t dtype_bytes(DataType dtype)
{
    switch (dtype) {
    case DataType::FP16: return 2;
    case DataType::INT32: return 4;
    case DataType::INT64: return 8;
    default: throw std::runtime_error("unsupported AOT tensor data type");
    }
}

GraphDescriptor decode_graph_binary(std::span<const std::byte> bytes)
{
    return decode(wire::parse_model_file(bytes, "graph.pb", wire::parse_graph));
}

LoadedGraph load_aot_graph(const ModelAssetReader& assets, const std::string& model_name)
{
    const std::filesystem::path dir = std::filesystem::path("aot") / model_name;
    const auto graph_bytes = assets.read_binary(dir / "graph.pb");
    const wire::Graph graph =
        wire::parse_model_file(graph_bytes, (dir / "graph.pb").string(), wire::parse_graph);
    const auto meta_bytes = assets.read_binary("metadata.pb");
    const wire::ModelMetadata meta = wire::parse_model_file(meta_bytes, "metadata.pb", wire::parse_metadata);
    if (graph.checkpoint_sha256 != meta.checkpoint_sha256)
        throw std::runtime_error("AOT graph checkpoint differs from metadata (" +
                                 assets.location_label() + ")");
    LoadedGraph loaded;
    loaded.descriptor = decode(graph);
    loaded.weights = assets.read_binary(dir / "weights.bin");
    if (loaded.weights.size() != loaded.descriptor.weights_bytes)
        throw std::runtime_error("AOT weights size does not match graph (" +
                                 assets.location_label() + ")");
    return loaded;
}

LoadedGraph load_aot_graph(const std::filesystem::path& model_dir, const std::string& model_name)
{
    return load_aot_graph(*make_model_asset_reader(model_dir), model_name);  // "embedded:<profile>" too (:319-324)
}

}  // namespace mlvc::aot
