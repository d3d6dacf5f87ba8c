// ModelConfig from metadata.pb checked against model_bundle.pb
// (contract of the reference's core/src/model.cpp:14-190), and the bundle's
// artifact hashes.

#include "mlvc/core/model.hpp"

#include "mlvc/runtime/graph_builder.hpp"
#include "mlvc/runtime/wire.hpp"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <limits>
#include <stdexcept>

namespace mlvc {
namespace {

// ceil(value / divisor) for positive operands (model.cpp:17-26).
int divide_up(int value, std::int64_t divisor)
{
    if (value <= 0 || divisor <= 0 || divisor > std::numeric_limits<int>::max())
        throw std::runtime_error("invalid model downsample dimensions");
    return static_cast<int>((static_cast<std::int64_t>(value) + divisor - 1) / divisor);
}

int checked_int(std::uint32_t value)
{
    if (value > static_cast<std::uint32_t>(std::numeric_limits<int>::max()))
        throw std::runtime_error("model integer exceeds runtime range");
    return static_cast<int>(value);
}

wire::ModelMetadata read_metadata(const ModelAssetReader& assets)
{
    return wire::parse_model_file(assets.read_binary("metadata.pb"), "metadata.pb", wire::parse_metadata);
}

// model.cpp:34-48: schema versions 1 / 2, the same profile, version,
// dimensions and checkpoint hash in both files, 32-byte hashes, and the
// container / entropy contract this runtime speaks.
void validate_bundle_manifest(const wire::ModelBundle& bundle, const wire::ModelMetadata& metadata)
{
    if (metadata.schema_version != 1 || bundle.schema_version != 2 || bundle.profile != metadata.profile ||
        bundle.model_version != metadata.model_version || bundle.width != metadata.width || bundle.height != metadata.height ||
        metadata.checkpoint_sha256.size() != 32 || bundle.entropy_model_sha256.size() != 32 ||
        bundle.checkpoint_sha256 != metadata.checkpoint_sha256 || bundle.contract.container != "mlvc-nalu-v0" ||
        bundle.contract.entropy != "canonical-pmf-v1")
        throw std::runtime_error("model bundle does not match Protobuf metadata");
}

}  // namespace

void ModelConfig::validate() const
{
    const bool bad_dims = model_width <= 0 || model_height <= 0 || feature_channels <= 0 || latent_channels <= 0 ||
                          hyperprior_channels <= 0 || downsample_feature <= 0 || downsample_latent <= 0 ||
                          downsample_hyperprior <= 0 || y_scale_repeat <= 0;
    if (name.empty() || model_version.empty() || bad_dims || !std::isfinite(pixel_range) || pixel_range <= 0.0F || qp_num <= 0 ||
        total_qp_num < qp_num || latent_channels % 2 != 0 || latent_channels % y_scale_repeat != 0 ||
        latent_channels / y_scale_repeat > hyperprior_channels || frame_index_map.empty() || qp_shift.empty())
        throw std::runtime_error("invalid fixed-shape model metadata");
    for (int index : frame_index_map)
        if (index < 0 || static_cast<std::size_t>(index) >= qp_shift.size())
            throw std::runtime_error("model QP shift mapping is out of range");
    for (int shift : qp_shift)
        if (shift < 0 || shift > total_qp_num - qp_num) throw std::runtime_error("model QP shift is outside the model range");
    if (iframe_period && *iframe_period <= 0) throw std::runtime_error("model I-frame period must be positive");
    if (reset_period && *reset_period <= 0) throw std::runtime_error("model reset period must be positive");
    if (static_cast<std::int64_t>(downsample_latent) * downsample_hyperprior > std::numeric_limits<int>::max())
        throw std::runtime_error("model downsample factor is too large");
    if (!disable_feature_reset || reset_period.has_value())
        throw std::runtime_error("this runtime currently requires the dmc61sbr_e1d1 no-reset profile");
}

int ModelConfig::feature_height() const { return divide_up(model_height, downsample_feature); }
int ModelConfig::feature_width() const { return divide_up(model_width, downsample_feature); }
int ModelConfig::latent_height() const { return divide_up(model_height, downsample_latent); }
int ModelConfig::latent_width() const { return divide_up(model_width, downsample_latent); }
int ModelConfig::hyperprior_height() const
{
    return divide_up(model_height, static_cast<std::int64_t>(downsample_latent) * downsample_hyperprior);
}
int ModelConfig::hyperprior_width() const
{
    return divide_up(model_width, static_cast<std::int64_t>(downsample_latent) * downsample_hyperprior);
}

ModelConfig load_model_config(const ModelAssetReader& assets)
{
    const wire::ModelMetadata m = read_metadata(assets);
    validate_bundle_manifest(wire::parse_model_file(assets.read_binary("model_bundle.pb"), "model_bundle.pb", wire::parse_bundle), m);
    ModelConfig c;
    c.name = m.profile;
    c.model_version = m.model_version;
    c.model_width = checked_int(m.width);
    c.model_height = checked_int(m.height);
    c.pixel_range = m.pixel_range;
    c.qp_num = checked_int(m.qp_num);
    c.total_qp_num = checked_int(m.total_qp_num);
    c.feature_channels = checked_int(m.feature_channels);
    c.latent_channels = checked_int(m.latent_channels);
    c.hyperprior_channels = checked_int(m.hyperprior_channels);
    c.downsample_feature = checked_int(m.downsample_feature);
    c.downsample_latent = checked_int(m.downsample_latent);
    c.downsample_hyperprior = checked_int(m.downsample_hyperprior);
    c.y_scale_repeat = checked_int(m.y_scale_repeat);
    for (std::uint32_t v : m.frame_index_map) c.frame_index_map.push_back(checked_int(v));
    c.qp_shift.assign(m.qp_shift.begin(), m.qp_shift.end());
    if (m.iframe_period) c.iframe_period = checked_int(*m.iframe_period);
    if (m.reset_period) c.reset_period = checked_int(*m.reset_period);
    c.disable_feature_reset = m.disable_feature_reset;
    try {
        c.validate();
    } catch (const std::exception& e) {
        throw std::runtime_error(std::string(e.what()) + ": " + assets.location_label() + "/metadata.pb");
    }
    return c;
}

ModelConfig load_model_config(const std::filesystem::path& model_dir)
{
    return load_model_config(*make_model_asset_reader(model_dir));
}

std::vector<std::string> embedded_model_profiles() { return list_embedded_model_profiles(); }

void verify_model_bundle(const ModelAssetReader& assets)
{
    const wire::ModelBundle b = wire::parse_model_file(assets.read_binary("model_bundle.pb"), "model_bundle.pb", wire::parse_bundle);
    for (const wire::Artifact& a : b.artifacts) {
        if (a.path.empty() || a.sha256.size() != 32) throw std::runtime_error("model bundle artifact entry is malformed");
        if (!assets.exists(a.path)) throw std::runtime_error("model bundle artifact is missing: " + a.path);
        const std::vector<std::byte> data = assets.read_binary(a.path);
        if (data.size() != a.size_bytes) throw std::runtime_error("model bundle artifact size mismatch: " + a.path);
        const auto digest = synth::sha256(data.data(), data.size());
        if (std::string(reinterpret_cast<const char*>(digest.data()), digest.size()) != a.sha256)
            throw std::runtime_error("model bundle artifact hash mismatch: " + a.path);
    }
}

}  // namespace mlvc
