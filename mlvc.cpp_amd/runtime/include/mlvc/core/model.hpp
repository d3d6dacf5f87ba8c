#pragma once
// Fixed-shape model configuration of an MLVC bundle, read from metadata.pb
// and checked against model_bundle.pb.
//
// Same contract as the reference's core/include/mlvc/core/model.hpp:10-46
// and core/src/model.cpp: ModelConfig (members, validate(), derived feature /
// latent / hyperprior dimensions), load_model_config and
// embedded_model_profiles. The reference's per-frame GOP and QP-shift
// schedule (frame_in_gop, q_index_shift) belongs to the codec pipeline, not
// to a backend, and is not declared here. verify_model_bundle is an
// addition: it checks the bundle's artifact list (path, size, SHA-256)
// against the files.

#include "mlvc/core/assets.hpp"

#include <filesystem>
#include <optional>
#include <string>
#include <vector>

namespace mlvc {

struct ModelConfig {
    std::string name;
    std::string model_version;
    int model_width = 0;
    int model_height = 0;
    float pixel_range = 1.0F;
    int qp_num = 0;
    int total_qp_num = 0;
    std::vector<int> frame_index_map;
    std::vector<int> qp_shift;
    int feature_channels = 0;
    int latent_channels = 0;
    int hyperprior_channels = 0;
    int downsample_feature = 0;
    int downsample_latent = 0;
    int downsample_hyperprior = 0;
    int y_scale_repeat = 0;
    std::optional<int> iframe_period;
    std::optional<int> reset_period;
    bool disable_feature_reset = false;

    void validate() const;
    int feature_height() const;
    int feature_width() const;
    int latent_height() const;
    int latent_width() const;
    int hyperprior_height() const;
    int hyperprior_width() const;
};

ModelConfig load_model_config(const ModelAssetReader& assets);
ModelConfig load_model_config(const std::filesystem::path& model_dir);
std::vector<std::string> embedded_model_profiles();

// Every artifact listed in model_bundle.pb exists with the recorded size and
// SHA-256; throws naming the first one that does not.
void verify_model_bundle(const ModelAssetReader& assets);

}  // namespace mlvc
