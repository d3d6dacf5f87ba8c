// Schema-3 graph writer, arena planner, SHA-256 and the seeded generator.

#include "mlvc/runtime/graph_builder.hpp"

#include <algorithm>
#include <bit>
#include <cmath>
#include <cstring>
#include <fstream>
#include <map>
#include <stdexcept>
#include <optional>

namespace mlvc::synth {
namespace {

constexpr std::uint64_t kAlign = 256;

std::uint64_t align_up(std::uint64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

std::size_t element_count(const GraphBuilder::Shape& s)
{
    std::size_t n = 1;
    for (auto d : s) n *= static_cast<std::size_t>(d);
    return n;
}

// ---- SHA-256 round constants, derived exactly from the primes ----------
// K[i] = first 32 fraction bits of cbrt(prime_i); H[i] likewise of sqrt.
using u128 = unsigned __int128;

std::uint64_t iroot(u128 x, int k)
{
    std::uint64_t lo = 0, hi = std::uint64_t{1} << 43;  // enough for both uses
    while (lo < hi) {
        const std::uint64_t mid = lo + (hi - lo + 1) / 2;
        u128 p = 1;
        for (int i = 0; i < k; ++i) p *= mid;
        if (p <= x) lo = mid; else hi = mid - 1;
    }
    return lo;
}

struct ShaConstants {
    std::uint32_t k[64];
    std::uint32_t h[8];
    ShaConstants()
    {
        int found = 0;
        for (std::uint64_t n = 2; found < 64; ++n) {
            bool prime = true;
            for (std::uint64_t d = 2; d * d <= n; ++d) if (n % d == 0) { prime = false; break; }
            if (!prime) continue;
            k[found] = static_cast<std::uint32_t>(iroot(static_cast<u128>(n) << 96, 3));
            if (found < 8) h[found] = static_cast<std::uint32_t>(iroot(static_cast<u128>(n) << 64, 2));
            ++found;
        }
    }
};

}  // namespace

std::array<std::uint8_t, 32> sha256(const void* data, std::size_t size)
{
    static const ShaConstants c;
    std::uint32_t h[8];
    std::memcpy(h, c.h, sizeof(h));
    const auto* bytes = static_cast<const std::uint8_t*>(data);
    std::vector<std::uint8_t> msg(bytes, bytes + size);
    msg.push_back(0x80);
    while (msg.size() % 64 != 56) msg.push_back(0);
    const std::uint64_t bits = static_cast<std::uint64_t>(size) * 8;
    for (int i = 7; i >= 0; --i) msg.push_back(static_cast<std::uint8_t>(bits >> (8 * i)));
    for (std::size_t off = 0; off < msg.size(); off += 64) {
        std::uint32_t w[64];
        for (int i = 0; i < 16; ++i)
            w[i] = (std::uint32_t{msg[off + 4 * i]} << 24) | (std::uint32_t{msg[off + 4 * i + 1]} << 16) |
                   (std::uint32_t{msg[off + 4 * i + 2]} << 8) | msg[off + 4 * i + 3];
        for (int i = 16; i < 64; ++i) {
            const std::uint32_t s0 = std::rotr(w[i - 15], 7) ^ std::rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const std::uint32_t s1 = std::rotr(w[i - 2], 17) ^ std::rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        std::uint32_t a = h[0], b = h[1], cc = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
        for (int i = 0; i < 64; ++i) {
            const std::uint32_t t1 = hh + (std::rotr(e, 6) ^ std::rotr(e, 11) ^ std::rotr(e, 25)) +
                                     ((e & f) ^ (~e & g)) + c.k[i] + w[i];
            const std::uint32_t t2 = (std::rotr(a, 2) ^ std::rotr(a, 13) ^ std::rotr(a, 22)) +
                                     ((a & b) ^ (a & cc) ^ (b & cc));
            hh = g; g = f; f = e; e = d + t1; d = cc; cc = b; b = a; a = t1 + t2;
        }
        h[0] += a; h[1] += b; h[2] += cc; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
    }
    std::array<std::uint8_t, 32> out{};
    for (int i = 0; i < 8; ++i)
        for (int j = 0; j < 4; ++j) out[4 * i + j] = static_cast<std::uint8_t>(h[i] >> (24 - 8 * j));
    return out;
}

// ---- RNG ----------------------------------------------------------------

std::uint64_t Rng::next()
{
    std::uint64_t z = (state_ += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

double Rng::uniform() { return static_cast<double>(next() >> 11) * 0x1.0p-53; }

double Rng::normal()
{
    if (have_spare_) {
        have_spare_ = false;
        return spare_;
    }
    double u1;
    do { u1 = uniform(); } while (u1 <= 0.0);
    const double u2 = uniform();
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double t = 2.0 * M_PI * u2;
    spare_ = r * std::sin(t);
    have_spare_ = true;
    return r * std::cos(t);
}

// ---- builder ------------------------------------------------------------

GraphBuilder::Id GraphBuilder::add_tensor(const std::string& name, aot::DataType dtype, const Shape& shape)
{
    for (const T& t : tensors_)
        if (t.name == name) throw std::runtime_error("duplicate tensor name: " + name);
    tensors_.push_back({name, dtype, shape});
    return static_cast<Id>(tensors_.size());
}

GraphBuilder::Id GraphBuilder::input(const std::string& name, const Shape& shape, aot::DataType dtype)
{
    const Id id = add_tensor(name, dtype, shape);
    inputs_.push_back(id);
    return id;
}

GraphBuilder::Id GraphBuilder::weight_fp16(const std::string& name, const Shape& shape,
                                           const std::vector<Float16Storage>& values)
{
    if (values.size() != element_count(shape)) throw std::runtime_error("weight size mismatch: " + name);
    const Id id = add_tensor(name, aot::DataType::FP16, shape);
    const std::uint64_t off = align_up(weights_.size());
    weights_.resize(off + values.size() * 2);
    std::memcpy(weights_.data() + off, values.data(), values.size() * 2);
    tensors_[id - 1].is_weight = true;
    tensors_[id - 1].w_offset = off;
    tensors_[id - 1].w_bytes = values.size() * 2;
    return id;
}

GraphBuilder::Id GraphBuilder::weight_int64(const std::string& name, const Shape& shape,
                                            const std::vector<std::int64_t>& values)
{
    if (values.size() != element_count(shape)) throw std::runtime_error("weight size mismatch: " + name);
    const Id id = add_tensor(name, aot::DataType::INT64, shape);
    const std::uint64_t off = align_up(weights_.size());
    weights_.resize(off + values.size() * 8);
    std::memcpy(weights_.data() + off, values.data(), values.size() * 8);
    tensors_[id - 1].is_weight = true;
    tensors_[id - 1].w_offset = off;
    tensors_[id - 1].w_bytes = values.size() * 8;
    return id;
}

GraphBuilder::Id GraphBuilder::add_node(N node, const Shape& out_shape, const std::string& out_name)
{
    node.output = add_tensor(out_name, aot::DataType::FP16, out_shape);
    nodes_.push_back(std::move(node));
    return nodes_.back().output;
}

GraphBuilder::Id GraphBuilder::conv(const std::string& name, Id x, Id w, Id b,
                                    std::array<int, 2> stride, std::array<int, 2> pad, int groups)
{
    const Shape& xs = shape(x);
    const Shape& ws = shape(w);
    const std::int64_t oh = (xs[2] + 2 * pad[0] - ws[2]) / stride[0] + 1;
    const std::int64_t ow = (xs[3] + 2 * pad[1] - ws[3]) / stride[1] + 1;
    N n = make_node(aot::Op::CONV, {x, w});
    if (b) n.inputs.push_back(b);
    n.attr = wire::AttrCase::kConv;
    n.conv.strides = {static_cast<std::uint32_t>(stride[0]), static_cast<std::uint32_t>(stride[1])};
    n.conv.pads = {static_cast<std::uint32_t>(pad[0]), static_cast<std::uint32_t>(pad[1]),
                   static_cast<std::uint32_t>(pad[0]), static_cast<std::uint32_t>(pad[1])};
    n.conv.dilations = {1, 1};
    n.conv.groups = static_cast<std::uint32_t>(groups);
    return add_node(std::move(n), {xs[0], ws[0], oh, ow}, name);
}

GraphBuilder::Id GraphBuilder::leaky_relu(const std::string& name, Id x, float alpha)
{
    N n = make_node(aot::Op::LEAKY_RELU, {x});
    n.attr = wire::AttrCase::kActivation;
    n.alpha = alpha;
    return add_node(std::move(n), shape(x), name);
}

GraphBuilder::Id GraphBuilder::binary(aot::Op op, const std::string& name, Id a, Id b)
{
    // Output shape: numpy broadcasting of the two operand shapes.
    const Shape& sa = shape(a);
    const Shape& sb = shape(b);
    const std::size_t r = std::max(sa.size(), sb.size());
    Shape out(r, 1);
    for (std::size_t i = 0; i < r; ++i) {
        const std::int64_t x = i + sa.size() >= r ? sa[i + sa.size() - r] : 1;
        const std::int64_t y = i + sb.size() >= r ? sb[i + sb.size() - r] : 1;
        if (x != y && x != 1 && y != 1) throw std::runtime_error("graph builder: operand shapes do not broadcast");
        out[i] = std::max(x, y);
    }
    return add_node(make_node(op, {a, b}), out, name);
}

GraphBuilder::Id GraphBuilder::clip(const std::string& name, Id x, Id lo, Id hi)
{
    std::vector<Id> ins{x, lo};
    if (hi) ins.push_back(hi);
    return add_node(make_node(aot::Op::CLIP, ins), shape(x), name);
}

GraphBuilder::Id GraphBuilder::slice(const std::string& name, Id x, const std::vector<std::int64_t>& starts,
                                     const std::vector<std::int64_t>& ends, const std::vector<std::int64_t>& axes,
                                     const std::vector<std::int64_t>& steps)
{
    // Output extent per sliced axis: ceil((clamp(end) - clamp(start)) / step)
    // for positive steps, the reverse range for negative ones.
    Shape out = shape(x);
    const auto n = static_cast<std::int64_t>(out.size());
    for (std::size_t a = 0; a < starts.size(); ++a) {
        std::int64_t ax = axes.empty() ? static_cast<std::int64_t>(a) : axes[a];
        if (ax < 0) ax += n;
        const std::int64_t dim = shape(x)[static_cast<std::size_t>(ax)];
        const std::int64_t step = steps.empty() ? 1 : steps[a];
        auto norm = [&](std::int64_t v, std::int64_t lo, std::int64_t hi) { return std::clamp(v < 0 ? v + dim : v, lo, hi); };
        std::int64_t len;
        if (step > 0) {
            len = (norm(ends[a], 0, dim) - norm(starts[a], 0, dim) + step - 1) / step;
        } else {
            len = (norm(starts[a], -1, dim - 1) - norm(ends[a], -1, dim - 1) + (-step) - 1) / (-step);
        }
        out[static_cast<std::size_t>(ax)] = std::max<std::int64_t>(len, 0);
    }
    const std::string p = name + "/";
    std::vector<Id> ins{x, weight_int64(p + "starts", {static_cast<std::int64_t>(starts.size())}, starts),
                        weight_int64(p + "ends", {static_cast<std::int64_t>(ends.size())}, ends)};
    if (!axes.empty()) ins.push_back(weight_int64(p + "axes", {static_cast<std::int64_t>(axes.size())}, axes));
    if (!steps.empty()) {
        if (axes.empty()) ins.push_back(0);
        ins.push_back(weight_int64(p + "steps", {static_cast<std::int64_t>(steps.size())}, steps));
    }
    return add_node(make_node(aot::Op::SLICE, ins), out, name);
}

GraphBuilder::Id GraphBuilder::gather(const std::string& name, Id data, Id indices, int axis)
{
    const Shape& ds = shape(data);
    const int ax = axis < 0 ? axis + static_cast<int>(ds.size()) : axis;
    Shape out(ds.begin(), ds.begin() + ax);
    for (auto d : shape(indices)) out.push_back(d);
    out.insert(out.end(), ds.begin() + ax + 1, ds.end());
    N n = make_node(aot::Op::GATHER, {data, indices});
    n.attr = wire::AttrCase::kAxis;
    n.axis = axis;
    return add_node(std::move(n), out, name);
}

GraphBuilder::Id GraphBuilder::unary(aot::Op op, const std::string& name, Id x)
{
    return add_node(make_node(op, {x}), shape(x), name);
}

GraphBuilder::Id GraphBuilder::pixel(aot::Op op, const std::string& name, Id x, int block)
{
    const Shape& s = shape(x);
    Shape out = s;
    if (op == aot::Op::DEPTH_TO_SPACE) {
        out = {s[0], s[1] / (block * block), s[2] * block, s[3] * block};
    } else {
        out = {s[0], s[1] * block * block, s[2] / block, s[3] / block};
    }
    N n = make_node(op, {x});
    n.attr = wire::AttrCase::kPixel;
    n.block = block;
    return add_node(std::move(n), out, name);
}

GraphBuilder::Id GraphBuilder::concat(const std::string& name, const std::vector<Id>& xs, int axis)
{
    Shape out = shape(xs.at(0));
    const int ax = axis < 0 ? axis + static_cast<int>(out.size()) : axis;
    for (std::size_t i = 1; i < xs.size(); ++i) out[static_cast<std::size_t>(ax)] += shape(xs[i])[static_cast<std::size_t>(ax)];
    N n = make_node(aot::Op::CONCAT, xs);
    n.attr = wire::AttrCase::kAxis;
    n.axis = axis;
    return add_node(std::move(n), out, name);
}

GraphBuilder::Files GraphBuilder::build(const std::string& profile) const
{
    // Lifetimes: birth = producing node; death = last consuming node, or the
    // node count for graph outputs.
    const std::size_t n_nodes = nodes_.size();
    std::vector<std::int64_t> birth(tensors_.size() + 1, -1), death(tensors_.size() + 1, -1);
    for (std::size_t i = 0; i < n_nodes; ++i) {
        birth[nodes_[i].output] = static_cast<std::int64_t>(i);
        death[nodes_[i].output] = std::max<std::int64_t>(death[nodes_[i].output], static_cast<std::int64_t>(i));
        for (Id in : nodes_[i].inputs) death[in] = std::max<std::int64_t>(death[in], static_cast<std::int64_t>(i));
    }
    for (Id o : outputs_) if (birth[o] >= 0) death[o] = static_cast<std::int64_t>(n_nodes);

    struct Interval { std::int64_t b, d; std::string name; std::uint64_t size; Id id; };
    std::vector<Interval> iv;
    for (Id id = 1; id <= tensors_.size(); ++id)
        if (birth[id] >= 0)
            iv.push_back({birth[id], death[id], tensors_[id - 1].name,
                          align_up(element_count(tensors_[id - 1].shape) * aot::dtype_bytes(tensors_[id - 1].dtype)), id});
    std::sort(iv.begin(), iv.end(), [](const Interval& a, const Interval& b) {
        return std::tie(a.b, a.d, a.name, a.size) < std::tie(b.b, b.d, b.name, b.size);
    });
    struct Block { std::uint64_t off, size; };
    std::vector<std::pair<std::int64_t, Block>> active;
    std::vector<Block> free_blocks;
    std::map<Id, std::pair<std::uint64_t, std::uint64_t>> placed;
    std::uint64_t arena_end = 0;
    for (const Interval& t : iv) {
        std::vector<std::pair<std::int64_t, Block>> keep;
        for (auto& a : active) (a.first < t.b ? free_blocks.push_back(a.second) : keep.push_back(a));
        active = std::move(keep);
        std::sort(free_blocks.begin(), free_blocks.end(), [](const Block& a, const Block& b) { return a.off < b.off; });
        std::vector<Block> merged;
        for (const Block& f : free_blocks) {
            if (!merged.empty() && merged.back().off + merged.back().size == f.off) merged.back().size += f.size;
            else merged.push_back(f);
        }
        free_blocks = std::move(merged);
        std::int64_t best = -1;
        for (std::size_t i = 0; i < free_blocks.size(); ++i)
            if (free_blocks[i].size >= t.size && (best < 0 || free_blocks[i].size < free_blocks[static_cast<std::size_t>(best)].size))
                best = static_cast<std::int64_t>(i);
        std::uint64_t off;
        if (best >= 0) {
            Block blk = free_blocks[static_cast<std::size_t>(best)];
            free_blocks.erase(free_blocks.begin() + best);
            off = blk.off;
            if (blk.size > t.size) free_blocks.push_back({blk.off + t.size, blk.size - t.size});
        } else {
            off = arena_end;
            arena_end += t.size;
        }
        active.push_back({t.d, {off, t.size}});
        placed[t.id] = {off, t.size};
    }

    wire::Graph g;
    g.schema_version = 3;
    const auto ck = sha256(profile.data(), profile.size());
    g.checkpoint_sha256.assign(reinterpret_cast<const char*>(ck.data()), 32);
    for (Id id = 1; id <= tensors_.size(); ++id) {
        const T& t = tensors_[id - 1];
        wire::TensorDescriptor td;
        td.id = id;
        td.name = t.name;
        td.dtype = static_cast<std::int32_t>(t.dtype);
        td.shape = t.shape;
        if (t.is_weight) {
            td.storage_case = wire::StorageCase::kWeight;
            td.weight = {t.w_offset, t.w_bytes};
        } else if (placed.count(id)) {
            td.storage_case = wire::StorageCase::kArena;
            td.arena = {placed[id].first, placed[id].second, static_cast<std::uint32_t>(birth[id]),
                        static_cast<std::uint32_t>(death[id])};
        }
        g.tensors.push_back(std::move(td));
    }
    g.inputs = inputs_;
    g.outputs = outputs_;
    for (const N& n : nodes_) {
        wire::Node wn;
        wn.op = static_cast<std::int32_t>(n.op);
        wn.inputs = n.inputs;
        wn.outputs = {n.output};
        wn.attr_case = n.attr;
        wn.conv = n.conv;
        wn.axis = n.axis;
        wn.alpha = n.alpha;
        wn.block_size = static_cast<std::uint32_t>(n.block);
        g.nodes.push_back(std::move(wn));
    }
    g.arena_bytes = std::max<std::uint64_t>(arena_end, kAlign);
    g.arena_alignment = 256;
    Files f;
    f.weights_bin = weights_;
    if (f.weights_bin.empty()) f.weights_bin.resize(kAlign);
    g.weights_bytes = f.weights_bin.size();
    const auto ws = sha256(f.weights_bin.data(), f.weights_bin.size());
    g.weights_sha256.assign(reinterpret_cast<const char*>(ws.data()), 32);
    f.graph_pb = wire::serialize(g);

    wire::ModelMetadata m;
    if (has_metadata_) {
        m = metadata_;
    } else {
        m.model_version = "synthetic";
        m.pixel_range = 255.0F;
        m.qp_num = 1;
        m.total_qp_num = 1;
    }
    m.schema_version = 1;
    m.profile = profile;
    m.checkpoint_sha256 = g.checkpoint_sha256;
    f.metadata_pb = wire::serialize(m);
    return f;
}

namespace {

// model_bundle.pb for a directory holding `files` (path -> bytes): schema 2,
// the metadata's identity, the codec contract, one artifact per file with
// its size and SHA-256, sorted by path. Entries of `previous` for other paths
// are kept. With no entropy model tables present, the entropy hash is the
// SHA-256 of nothing.
std::vector<std::byte> make_bundle(const wire::ModelMetadata& m, const std::map<std::string, const std::vector<std::byte>*>& files,
                                   const wire::ModelBundle* previous)
{
    wire::ModelBundle b;
    b.schema_version = 2;
    b.profile = m.profile;
    b.model_version = m.model_version;
    b.width = m.width;
    b.height = m.height;
    b.checkpoint_sha256 = m.checkpoint_sha256;
    const auto empty = sha256(nullptr, 0);
    b.entropy_model_sha256.assign(reinterpret_cast<const char*>(empty.data()), 32);
    b.contract.container = "mlvc-nalu-v0";
    b.contract.entropy = "canonical-pmf-v1";
    b.contract.decoder_max_yuv_sample_error = 1;
    b.contract.decoder_min_psnr_db = 60.0;
    std::map<std::string, wire::Artifact> arts;
    if (previous && previous->profile == m.profile && previous->checkpoint_sha256 == m.checkpoint_sha256)
        for (const auto& a : previous->artifacts) arts[a.path] = a;
    for (const auto& [path, bytes] : files) {
        wire::Artifact a;
        a.path = path;
        a.size_bytes = bytes->size();
        const auto d = sha256(bytes->data(), bytes->size());
        a.sha256.assign(reinterpret_cast<const char*>(d.data()), 32);
        arts[path] = a;
    }
    for (auto& [path, a] : arts) b.artifacts.push_back(a);
    return wire::serialize(b);
}

}  // namespace

void GraphBuilder::write_directory(const std::filesystem::path& dir, const std::string& model_name,
                                   const std::string& profile) const
{
    const Files f = build(profile);
    const auto gdir = dir / "aot" / model_name;
    std::filesystem::create_directories(gdir);
    auto put = [](const std::filesystem::path& p, const std::vector<std::byte>& b) {
        std::ofstream o(p, std::ios::binary | std::ios::trunc);
        o.write(reinterpret_cast<const char*>(b.data()), static_cast<std::streamsize>(b.size()));
        if (!o) throw std::runtime_error("cannot write " + p.string());
    };
    put(gdir / "graph.pb", f.graph_pb);
    put(gdir / "weights.bin", f.weights_bin);
    put(dir / "metadata.pb", f.metadata_pb);
    std::optional<wire::ModelBundle> previous;
    if (std::filesystem::is_regular_file(dir / "model_bundle.pb")) {
        try {
            previous = wire::parse_bundle(make_directory_asset_reader(dir)->read_binary("model_bundle.pb"));
        } catch (const std::exception&) {
            previous.reset();
        }
    }
    const std::string g = "aot/" + model_name + "/";
    const std::map<std::string, const std::vector<std::byte>*> files{
        {g + "graph.pb", &f.graph_pb}, {g + "weights.bin", &f.weights_bin}, {"metadata.pb", &f.metadata_pb}};
    put(dir / "model_bundle.pb", make_bundle(wire::parse_metadata(f.metadata_pb), files, previous ? &*previous : nullptr));
}

std::shared_ptr<const ModelAssetReader> GraphBuilder::to_memory(const std::string& model_name,
                                                                const std::string& profile) const
{
    const Files f = build(profile);
    auto r = std::make_shared<MemoryAssetReader>();
    const auto gdir = std::filesystem::path("aot") / model_name;
    r->add(gdir / "graph.pb", f.graph_pb);
    r->add(gdir / "weights.bin", f.weights_bin);
    r->add("metadata.pb", f.metadata_pb);
    const std::string g = "aot/" + model_name + "/";
    const std::map<std::string, const std::vector<std::byte>*> files{
        {g + "graph.pb", &f.graph_pb}, {g + "weights.bin", &f.weights_bin}, {"metadata.pb", &f.metadata_pb}};
    r->add("model_bundle.pb", make_bundle(wire::parse_metadata(f.metadata_pb), files, nullptr));
    return r;
}

}  // namespace mlvc::synth
