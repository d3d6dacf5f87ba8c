// Protobuf wire-format reader/writer for the schema-3 graph messages.
// Field numbers: reference proto/mlvc_model.proto:30-107.

#include "mlvc/runtime/wire.hpp"

#include <bit>
#include <cstring>
#include <stdexcept>

namespace mlvc::wire {
namespace {

constexpr int kVarint = 0, kFixed64 = 1, kLen = 2, kFixed32 = 5;

[[noreturn]] void fail(const char* what)
{
    throw std::runtime_error(std::string("malformed protobuf message: ") + what);
}

bool valid_utf8(std::span<const std::uint8_t> s)
{
    std::size_t i = 0;
    while (i < s.size()) {
        const std::uint8_t c = s[i];
        std::size_t n;
        std::uint32_t cp;
        if (c < 0x80) { ++i; continue; }
        if ((c & 0xE0) == 0xC0) { n = 1; cp = c & 0x1F; }
        else if ((c & 0xF0) == 0xE0) { n = 2; cp = c & 0x0F; }
        else if ((c & 0xF8) == 0xF0) { n = 3; cp = c & 0x07; }
        else return false;
        for (std::size_t k = 1; k <= n; ++k) {
            if (i + k >= s.size() || (s[i + k] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (s[i + k] & 0x3F);
        }
        // Reject overlong forms, surrogates and values past U+10FFFF.
        if ((n == 1 && cp < 0x80) || (n == 2 && cp < 0x800) || (n == 3 && cp < 0x10000) ||
            (cp >= 0xD800 && cp <= 0xDFFF) || cp > 0x10FFFF)
            return false;
        i += n + 1;
    }
    return true;
}

class Reader {
public:
    explicit Reader(std::span<const std::uint8_t> b) : p_(b.data()), end_(b.data() + b.size()) {}

    bool done() const { return p_ == end_; }

    std::uint64_t varint()
    {
        std::uint64_t v = 0;
        for (int shift = 0; shift < 70; shift += 7) {
            if (p_ == end_) fail("truncated varint");
            const std::uint8_t byte = *p_++;
            if (shift == 63 && byte > 1) fail("varint overflow");
            v |= static_cast<std::uint64_t>(byte & 0x7F) << shift;
            if (!(byte & 0x80)) return v;
        }
        fail("varint too long");
    }
    std::uint32_t fixed32()
    {
        if (end_ - p_ < 4) fail("truncated fixed32");
        std::uint32_t v;
        std::memcpy(&v, p_, 4);
        p_ += 4;
        return v;
    }
    std::uint64_t fixed64()
    {
        if (end_ - p_ < 8) fail("truncated fixed64");
        std::uint64_t v;
        std::memcpy(&v, p_, 8);
        p_ += 8;
        return v;
    }
    std::span<const std::uint8_t> len_delimited()
    {
        const std::uint64_t n = varint();
        if (n > static_cast<std::uint64_t>(end_ - p_)) fail("truncated length-delimited field");
        std::span<const std::uint8_t> s(p_, static_cast<std::size_t>(n));
        p_ += n;
        return s;
    }
    void skip(int wt)
    {
        switch (wt) {
        case kVarint: varint(); return;
        case kFixed64:
            if (end_ - p_ < 8) fail("truncated fixed64");
            p_ += 8;
            return;
        case kLen: len_delimited(); return;
        case kFixed32: fixed32(); return;
        default: fail("unsupported wire type");
        }
    }
    // Returns (field number, wire type).
    std::pair<std::uint32_t, int> tag()
    {
        const std::uint64_t t = varint();
        if (t > 0xFFFFFFFFULL) fail("tag out of range");
        const auto field = static_cast<std::uint32_t>(t >> 3);
        if (field == 0) fail("field number zero");
        return {field, static_cast<int>(t & 7)};
    }

private:
    const std::uint8_t* p_;
    const std::uint8_t* end_;
};

std::span<const std::uint8_t> as_u8(std::span<const std::byte> b)
{
    return {reinterpret_cast<const std::uint8_t*>(b.data()), b.size()};
}

std::string read_string(Reader& r, bool utf8)
{
    const auto s = r.len_delimited();
    if (utf8 && !valid_utf8(s)) fail("string field is not valid UTF-8");
    return std::string(reinterpret_cast<const char*>(s.data()), s.size());
}

// Repeated scalar: packed (wire type 2) or one element per tag (wire type 0).
template <typename T, typename Conv>
bool read_repeated(Reader& r, int wt, std::vector<T>& out, Conv conv)
{
    if (wt == kLen) {
        Reader sub(r.len_delimited());
        while (!sub.done()) out.push_back(conv(sub.varint()));
        return true;
    }
    if (wt == kVarint) {
        out.push_back(conv(r.varint()));
        return true;
    }
    return false;
}

auto as_u32 = [](std::uint64_t v) { return static_cast<std::uint32_t>(v); };
auto as_i32 = [](std::uint64_t v) { return static_cast<std::int32_t>(static_cast<std::uint32_t>(v)); };
auto as_i64 = [](std::uint64_t v) { return static_cast<std::int64_t>(v); };
auto zigzag32 = [](std::uint64_t v) {
    const auto u = static_cast<std::uint32_t>(v);
    return static_cast<std::int32_t>((u >> 1) ^ (~(u & 1U) + 1U));
};

void parse_conv(std::span<const std::uint8_t> b, ConvAttributes& m)
{
    Reader r(b);
    while (!r.done()) {
        const auto [f, wt] = r.tag();
        bool ok = true;
        switch (f) {
        case 1: ok = read_repeated(r, wt, m.strides, as_u32); break;
        case 2: ok = read_repeated(r, wt, m.pads, as_u32); break;
        case 3: ok = read_repeated(r, wt, m.dilations, as_u32); break;
        case 4: ok = wt == kVarint && (m.groups = as_u32(r.varint()), true); break;
        default: ok = false;
        }
        if (!ok) r.skip(wt);
    }
}

// Parses a one-field attribute message (AxisAttributes, ActivationAttributes
// or PixelAttributes) and applies `on_field` to field 1.
template <typename Fn>
void parse_single_field(std::span<const std::uint8_t> b, int want_wt, Fn on_field)
{
    Reader r(b);
    while (!r.done()) {
        const auto [f, wt] = r.tag();
        if (f == 1 && wt == want_wt)
            on_field(r);
        else
            r.skip(wt);
    }
}

void set_attr_case(Node& n, AttrCase c)
{
    if (n.attr_case != c) {
        n.conv = ConvAttributes{};
        n.axis = 0;
        n.alpha = 0.0F;
        n.block_size = 0;
        n.attr_case = c;
    }
}

void parse_node(std::span<const std::uint8_t> b, Node& n)
{
    Reader r(b);
    while (!r.done()) {
        const auto [f, wt] = r.tag();
        bool ok = true;
        switch (f) {
        case 1: ok = wt == kVarint && (n.op = as_i32(r.varint()), true); break;
        case 2: ok = read_repeated(r, wt, n.inputs, as_u32); break;
        case 3: ok = read_repeated(r, wt, n.outputs, as_u32); break;
        case 4:
            if ((ok = wt == kLen)) { set_attr_case(n, AttrCase::kConv); parse_conv(r.len_delimited(), n.conv); }
            break;
        case 5:
            if ((ok = wt == kLen)) {
                set_attr_case(n, AttrCase::kAxis);
                parse_single_field(r.len_delimited(), kVarint, [&](Reader& s) { n.axis = zigzag32(s.varint()); });
            }
            break;
        case 6:
            if ((ok = wt == kLen)) {
                set_attr_case(n, AttrCase::kActivation);
                parse_single_field(r.len_delimited(), kFixed32, [&](Reader& s) { n.alpha = std::bit_cast<float>(s.fixed32()); });
            }
            break;
        case 7:
            if ((ok = wt == kLen)) {
                set_attr_case(n, AttrCase::kPixel);
                parse_single_field(r.len_delimited(), kVarint, [&](Reader& s) { n.block_size = as_u32(s.varint()); });
            }
            break;
        default: ok = false;
        }
        if (!ok) r.skip(wt);
    }
}

void parse_tensor(std::span<const std::uint8_t> b, TensorDescriptor& t)
{
    Reader r(b);
    while (!r.done()) {
        const auto [f, wt] = r.tag();
        bool ok = true;
        switch (f) {
        case 1: ok = wt == kVarint && (t.id = as_u32(r.varint()), true); break;
        case 2: ok = wt == kLen && (t.name = read_string(r, true), true); break;
        case 3: ok = wt == kVarint && (t.dtype = as_i32(r.varint()), true); break;
        case 4: ok = read_repeated(r, wt, t.shape, as_i64); break;
        case 5:
            if ((ok = wt == kLen)) {
                if (t.storage_case != StorageCase::kArena) { t.weight = {}; t.arena = {}; }
                t.storage_case = StorageCase::kArena;
                Reader s(r.len_delimited());
                while (!s.done()) {
                    const auto [g, w] = s.tag();
                    if (w != kVarint) { s.skip(w); continue; }
                    const std::uint64_t v = s.varint();
                    if (g == 1) t.arena.offset = v;
                    else if (g == 2) t.arena.size_bytes = v;
                    else if (g == 3) t.arena.birth = as_u32(v);
                    else if (g == 4) t.arena.death = as_u32(v);
                }
            }
            break;
        case 6:
            if ((ok = wt == kLen)) {
                if (t.storage_case != StorageCase::kWeight) { t.weight = {}; t.arena = {}; }
                t.storage_case = StorageCase::kWeight;
                Reader s(r.len_delimited());
                while (!s.done()) {
                    const auto [g, w] = s.tag();
                    if (w != kVarint) { s.skip(w); continue; }
                    const std::uint64_t v = s.varint();
                    if (g == 1) t.weight.offset = v;
                    else if (g == 2) t.weight.size_bytes = v;
                }
            }
            break;
        default: ok = false;
        }
        if (!ok) r.skip(wt);
    }
}

// ---- writer ---------------------------------------------------------------

class Writer {
public:
    void varint(std::uint64_t v)
    {
        while (v >= 0x80) {
            out_.push_back(static_cast<std::uint8_t>(v | 0x80));
            v >>= 7;
        }
        out_.push_back(static_cast<std::uint8_t>(v));
    }
    void tag(std::uint32_t field, int wt) { varint((static_cast<std::uint64_t>(field) << 3) | static_cast<unsigned>(wt)); }
    void u64(std::uint32_t field, std::uint64_t v) { if (v) { tag(field, kVarint); varint(v); } }
    void i32(std::uint32_t field, std::int32_t v)
    {
        if (v) { tag(field, kVarint); varint(static_cast<std::uint64_t>(static_cast<std::int64_t>(v))); }
    }
    void sint32(std::uint32_t field, std::int32_t v)
    {
        const auto z = (static_cast<std::uint32_t>(v) << 1) ^ static_cast<std::uint32_t>(v >> 31);
        u64(field, z);
    }
    void boolean(std::uint32_t field, bool v) { u64(field, v ? 1 : 0); }
    void f64(std::uint32_t field, double v)
    {
        const auto bits = std::bit_cast<std::uint64_t>(v);
        if (bits) { tag(field, kFixed64); raw(&bits, 8); }
    }
    void f32(std::uint32_t field, float v)
    {
        const auto bits = std::bit_cast<std::uint32_t>(v);
        if (bits) { tag(field, kFixed32); raw(&bits, 4); }
    }
    void bytes(std::uint32_t field, const std::string& s, bool always = false)
    {
        if (s.empty() && !always) return;
        tag(field, kLen);
        varint(s.size());
        raw(s.data(), s.size());
    }
    template <typename T, typename Enc>
    void packed(std::uint32_t field, const std::vector<T>& v, Enc enc)
    {
        if (v.empty()) return;
        Writer body;
        for (const T& x : v) body.varint(enc(x));
        message(field, body);
    }
    void message(std::uint32_t field, const Writer& body)
    {
        tag(field, kLen);
        varint(body.out_.size());
        raw(body.out_.data(), body.out_.size());
    }
    void raw(const void* p, std::size_t n)
    {
        const auto* b = static_cast<const std::uint8_t*>(p);
        out_.insert(out_.end(), b, b + n);
    }
    std::vector<std::byte> take() const
    {
        std::vector<std::byte> r(out_.size());
        if (!out_.empty()) std::memcpy(r.data(), out_.data(), out_.size());
        return r;
    }

private:
    std::vector<std::uint8_t> out_;
};

auto enc_u32 = [](std::uint32_t v) { return static_cast<std::uint64_t>(v); };
auto enc_i64 = [](std::int64_t v) { return static_cast<std::uint64_t>(v); };
auto enc_i32 = [](std::int32_t v) { return static_cast<std::uint64_t>(static_cast<std::int64_t>(v)); };

}  // namespace

Graph parse_graph(std::span<const std::byte> bytes)
{
    Graph g;
    Reader r(as_u8(bytes));
    while (!r.done()) {
        const auto [f, wt] = r.tag();
        bool ok = true;
        switch (f) {
        case 1: ok = wt == kVarint && (g.schema_version = as_u32(r.varint()), true); break;
        case 2: ok = wt == kLen && (g.checkpoint_sha256 = read_string(r, false), true); break;
        case 3:
            if ((ok = wt == kLen)) { g.tensors.emplace_back(); parse_tensor(r.len_delimited(), g.tensors.back()); }
            break;
        case 4: ok = read_repeated(r, wt, g.inputs, as_u32); break;
        case 5: ok = read_repeated(r, wt, g.outputs, as_u32); break;
        case 6:
            if ((ok = wt == kLen)) { g.nodes.emplace_back(); parse_node(r.len_delimited(), g.nodes.back()); }
            break;
        case 7: ok = wt == kVarint && (g.arena_bytes = r.varint(), true); break;
        case 8: ok = wt == kVarint && (g.arena_alignment = as_u32(r.varint()), true); break;
        case 9: ok = wt == kVarint && (g.weights_bytes = r.varint(), true); break;
        case 10: ok = wt == kLen && (g.weights_sha256 = read_string(r, false), true); break;
        default: ok = false;
        }
        if (!ok) r.skip(wt);
    }
    return g;
}

ModelMetadata parse_metadata(std::span<const std::byte> bytes)
{
    ModelMetadata m;
    Reader r(as_u8(bytes));
    while (!r.done()) {
        const auto [f, wt] = r.tag();
        bool ok = true;
        auto u32 = [&](std::uint32_t& dst) { return wt == kVarint && (dst = as_u32(r.varint()), true); };
        switch (f) {
        case 1: ok = u32(m.schema_version); break;
        case 2: ok = wt == kLen && (m.profile = read_string(r, true), true); break;
        case 3: ok = wt == kLen && (m.model_version = read_string(r, true), true); break;
        case 4: ok = wt == kLen && (m.checkpoint_sha256 = read_string(r, false), true); break;
        case 5: ok = u32(m.width); break;
        case 6: ok = u32(m.height); break;
        case 7: ok = wt == kFixed32 && (m.pixel_range = std::bit_cast<float>(r.fixed32()), true); break;
        case 8: ok = u32(m.qp_num); break;
        case 9: ok = u32(m.total_qp_num); break;
        case 10: ok = read_repeated(r, wt, m.frame_index_map, as_u32); break;
        case 11: ok = read_repeated(r, wt, m.qp_shift, zigzag32); break;
        case 12: ok = u32(m.feature_channels); break;
        case 13: ok = u32(m.latent_channels); break;
        case 14: ok = u32(m.hyperprior_channels); break;
        case 15: ok = u32(m.downsample_feature); break;
        case 16: ok = u32(m.downsample_latent); break;
        case 17: ok = u32(m.downsample_hyperprior); break;
        case 18: ok = u32(m.y_scale_repeat); break;
        case 19: ok = wt == kVarint && (m.iframe_period = as_u32(r.varint()), true); break;
        case 20: ok = wt == kVarint && (m.reset_period = as_u32(r.varint()), true); break;
        case 21: ok = wt == kVarint && (m.disable_feature_reset = r.varint() != 0, true); break;
        default: ok = false;
        }
        if (!ok) r.skip(wt);
    }
    return m;
}

std::vector<std::byte> serialize(const Graph& g)
{
    Writer w;
    w.u64(1, g.schema_version);
    w.bytes(2, g.checkpoint_sha256);
    for (const TensorDescriptor& t : g.tensors) {
        Writer tw;
        tw.u64(1, t.id);
        tw.bytes(2, t.name);
        tw.i32(3, t.dtype);
        tw.packed(4, t.shape, enc_i64);
        if (t.storage_case == StorageCase::kArena) {
            Writer a;
            a.u64(1, t.arena.offset);
            a.u64(2, t.arena.size_bytes);
            a.u64(3, t.arena.birth);
            a.u64(4, t.arena.death);
            tw.message(5, a);
        } else if (t.storage_case == StorageCase::kWeight) {
            Writer a;
            a.u64(1, t.weight.offset);
            a.u64(2, t.weight.size_bytes);
            tw.message(6, a);
        }
        w.message(3, tw);
    }
    w.packed(4, g.inputs, enc_u32);
    w.packed(5, g.outputs, enc_u32);
    for (const Node& n : g.nodes) {
        Writer nw;
        nw.i32(1, n.op);
        nw.packed(2, n.inputs, enc_u32);
        nw.packed(3, n.outputs, enc_u32);
        Writer a;
        switch (n.attr_case) {
        case AttrCase::kConv:
            a.packed(1, n.conv.strides, enc_u32);
            a.packed(2, n.conv.pads, enc_u32);
            a.packed(3, n.conv.dilations, enc_u32);
            a.u64(4, n.conv.groups);
            nw.message(4, a);
            break;
        case AttrCase::kAxis: a.sint32(1, n.axis); nw.message(5, a); break;
        case AttrCase::kActivation: a.f32(1, n.alpha); nw.message(6, a); break;
        case AttrCase::kPixel: a.u64(1, n.block_size); nw.message(7, a); break;
        case AttrCase::kNone: break;
        }
        w.message(6, nw);
    }
    w.u64(7, g.arena_bytes);
    w.u64(8, g.arena_alignment);
    w.u64(9, g.weights_bytes);
    w.bytes(10, g.weights_sha256);
    return w.take();
}

std::vector<std::byte> serialize(const ModelMetadata& m)
{
    Writer w;
    w.u64(1, m.schema_version);
    w.bytes(2, m.profile);
    w.bytes(3, m.model_version);
    w.bytes(4, m.checkpoint_sha256);
    w.u64(5, m.width);
    w.u64(6, m.height);
    w.f32(7, m.pixel_range);
    w.u64(8, m.qp_num);
    w.u64(9, m.total_qp_num);
    w.packed(10, m.frame_index_map, enc_u32);
    w.packed(11, m.qp_shift, [](std::int32_t v) {
        return static_cast<std::uint64_t>((static_cast<std::uint32_t>(v) << 1) ^ static_cast<std::uint32_t>(v >> 31));
    });
    w.u64(12, m.feature_channels);
    w.u64(13, m.latent_channels);
    w.u64(14, m.hyperprior_channels);
    w.u64(15, m.downsample_feature);
    w.u64(16, m.downsample_latent);
    w.u64(17, m.downsample_hyperprior);
    w.u64(18, m.y_scale_repeat);
    if (m.iframe_period) { w.tag(19, kVarint); w.varint(*m.iframe_period); }
    if (m.reset_period) { w.tag(20, kVarint); w.varint(*m.reset_period); }
    w.boolean(21, m.disable_feature_reset);
    return w.take();
}

ModelBundle parse_bundle(std::span<const std::byte> bytes)
{
    ModelBundle b;
    Reader r(as_u8(bytes));
    while (!r.done()) {
        const auto [f, wt] = r.tag();
        bool ok = true;
        auto u32 = [&](std::uint32_t& dst) { return wt == kVarint && (dst = as_u32(r.varint()), true); };
        switch (f) {
        case 1: ok = u32(b.schema_version); break;
        case 2: ok = wt == kLen && (b.profile = read_string(r, true), true); break;
        case 3: ok = wt == kLen && (b.model_version = read_string(r, true), true); break;
        case 4: ok = u32(b.width); break;
        case 5: ok = u32(b.height); break;
        case 6: ok = wt == kLen && (b.checkpoint_sha256 = read_string(r, false), true); break;
        case 7: ok = wt == kLen && (b.entropy_model_sha256 = read_string(r, false), true); break;
        case 8: {
            if (wt != kLen) { ok = false; break; }
            Reader c(r.len_delimited());
            while (!c.done()) {
                const auto [cf, cwt] = c.tag();
                bool cok = true;
                if (cf == 1 && cwt == kLen) b.contract.container = read_string(c, true);
                else if (cf == 2 && cwt == kLen) b.contract.entropy = read_string(c, true);
                else if (cf == 3 && cwt == kVarint) b.contract.decoder_max_yuv_sample_error = as_u32(c.varint());
                else if (cf == 4 && cwt == kFixed64) b.contract.decoder_min_psnr_db = std::bit_cast<double>(c.fixed64());
                else cok = false;
                if (!cok) c.skip(cwt);
            }
            break;
        }
        case 9: {
            if (wt != kLen) { ok = false; break; }
            Artifact a;
            Reader c(r.len_delimited());
            while (!c.done()) {
                const auto [af, awt] = c.tag();
                bool aok = true;
                if (af == 1 && awt == kLen) a.path = read_string(c, true);
                else if (af == 2 && awt == kVarint) a.size_bytes = c.varint();
                else if (af == 3 && awt == kLen) a.sha256 = read_string(c, false);
                else aok = false;
                if (!aok) c.skip(awt);
            }
            b.artifacts.push_back(std::move(a));
            break;
        }
        default: ok = false;
        }
        if (!ok) r.skip(wt);
    }
    return b;
}

std::vector<std::byte> serialize(const ModelBundle& b)
{
    Writer w;
    w.u64(1, b.schema_version);
    w.bytes(2, b.profile);
    w.bytes(3, b.model_version);
    w.u64(4, b.width);
    w.u64(5, b.height);
    w.bytes(6, b.checkpoint_sha256);
    w.bytes(7, b.entropy_model_sha256);
    Writer c;
    c.bytes(1, b.contract.container);
    c.bytes(2, b.contract.entropy);
    c.u64(3, b.contract.decoder_max_yuv_sample_error);
    c.f64(4, b.contract.decoder_min_psnr_db);
    w.message(8, c);
    for (const Artifact& a : b.artifacts) {
        Writer aw;
        aw.bytes(1, a.path);
        aw.u64(2, a.size_bytes);
        aw.bytes(3, a.sha256);
        w.message(9, aw);
    }
    return w.take();
}

}  // namespace mlvc::wire
