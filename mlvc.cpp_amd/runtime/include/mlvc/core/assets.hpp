#pragma once
// Read-only sources of model files (graph.pb, weights.bin, metadata.pb).
//
// Same interface as the reference's core/include/mlvc/core/assets.hpp:16-37
// (ModelAssetReader with location_label/exists/read_binary, the directory and
// embedded readers, "embedded:<profile>" locations and the default-location
// rule of core/src/model_assets.cpp:36-252), plus an in-memory reader. The
// embedded readers read the model image described in mlvc_embedded_models.h
// when one is linked; without one, the build behaves like the reference built
// without MLVC_HAS_EMBEDDED_MODELS: embedded readers hold no files and the
// profile list is empty.

#include <cstddef>
#include <filesystem>
#include <map>
#include <memory>
#include <string>
#include <string_view>
#include <vector>

namespace mlvc {

class ModelAssetReader {
public:
    virtual ~ModelAssetReader() = default;
    virtual std::string location_label() const = 0;
    virtual bool exists(const std::filesystem::path& relative_path) const = 0;
    virtual std::vector<std::byte> read_binary(
        const std::filesystem::path& relative_path) const = 0;
};

// Files keyed by their generic relative path ("aot/<model>/graph.pb").
class MemoryAssetReader final : public ModelAssetReader {
public:
    void add(const std::filesystem::path& relative_path, std::vector<std::byte> bytes);
    std::string location_label() const override { return "in-memory"; }
    bool exists(const std::filesystem::path& relative_path) const override;
    std::vector<std::byte> read_binary(
        const std::filesystem::path& relative_path) const override;

private:
    std::map<std::string, std::vector<std::byte>> files_;
};

std::shared_ptr<const ModelAssetReader> make_directory_asset_reader(
    std::filesystem::path directory);

// Reader of a profile compiled into the binary ("embedded:<profile>");
// profiles containing '/' or '\\' are rejected.
std::shared_ptr<const ModelAssetReader> make_embedded_asset_reader(std::string_view profile);

// "embedded:<profile>" -> embedded reader, anything else -> directory reader.
std::shared_ptr<const ModelAssetReader> make_model_asset_reader(const std::filesystem::path& location);

// `override_reader` when set, else a reader for `model_dir`, else the default
// embedded model (an error when none is linked).
std::shared_ptr<const ModelAssetReader> resolve_model_asset_reader(
    const std::filesystem::path& model_dir,
    std::shared_ptr<const ModelAssetReader> override_reader = nullptr);

std::vector<std::string> list_embedded_model_profiles();
// "embedded:mlvc-psnr-v1" when linked, else the first embedded profile, else empty.
std::filesystem::path default_model_location();

}  // namespace mlvc
