#pragma once
// Read-only sources of model files (graph.pb, weights.bin, metadata.pb).
//
// Same interface as the reference's core/include/mlvc/core/assets.hpp:16-37
// (ModelAssetReader with location_label/exists/read_binary); this build
// provides a directory reader and an in-memory reader. Embedded bundles are
// outside the inference path.

#include <cstddef>
#include <filesystem>
#include <map>
#include <memory>
#include <string>
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

// Returns `override_reader` when set, else a directory reader on `model_dir`.
std::shared_ptr<const ModelAssetReader> resolve_model_asset_reader(
    const std::filesystem::path& model_dir,
    std::shared_ptr<const ModelAssetReader> override_reader = nullptr);

}  // namespace mlvc
