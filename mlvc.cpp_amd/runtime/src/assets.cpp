// Directory and in-memory model asset readers.

#include "mlvc/core/assets.hpp"

#include <algorithm>
#include <fstream>
#include <stdexcept>

namespace mlvc {
namespace {

class DirectoryAssetReader final : public ModelAssetReader {
public:
    explicit DirectoryAssetReader(std::filesystem::path root) : root_(std::move(root)) {}

    std::string location_label() const override { return root_.string(); }

    bool exists(const std::filesystem::path& rel) const override
    {
        return std::filesystem::is_regular_file(root_ / rel);
    }

    std::vector<std::byte> read_binary(const std::filesystem::path& rel) const override
    {
        const auto path = root_ / rel;
        std::ifstream in(path, std::ios::binary | std::ios::ate);
        if (!in)
            throw std::runtime_error("cannot open model asset: " + path.string());
        const auto size = static_cast<std::size_t>(in.tellg());
        std::vector<std::byte> data(size);
        in.seekg(0);
        if (size && !in.read(reinterpret_cast<char*>(data.data()), static_cast<std::streamsize>(size)))
            throw std::runtime_error("cannot read model asset: " + path.string());
        return data;
    }

private:
    std::filesystem::path root_;
};

constexpr std::string_view kEmbeddedPrefix = "embedded:";

void check_profile(const std::string& profile)
{
    if (profile.empty() || profile.find('/') != std::string::npos || profile.find('\\') != std::string::npos)
        throw std::runtime_error("invalid embedded model profile: " + profile);
}

// No model image is linked into this build: every lookup misses.
class EmbeddedAssetReader final : public ModelAssetReader {
public:
    explicit EmbeddedAssetReader(std::string profile) : profile_(std::move(profile)) { check_profile(profile_); }

    std::string location_label() const override { return std::string(kEmbeddedPrefix) + profile_; }
    bool exists(const std::filesystem::path&) const override { return false; }
    std::vector<std::byte> read_binary(const std::filesystem::path&) const override
    {
        throw std::runtime_error("embedded models are disabled in this build (" + location_label() + ")");
    }

private:
    std::string profile_;
};

}  // namespace

void MemoryAssetReader::add(const std::filesystem::path& rel, std::vector<std::byte> bytes)
{
    files_[rel.generic_string()] = std::move(bytes);
}

bool MemoryAssetReader::exists(const std::filesystem::path& rel) const
{
    return files_.count(rel.generic_string()) != 0;
}

std::vector<std::byte> MemoryAssetReader::read_binary(const std::filesystem::path& rel) const
{
    const auto it = files_.find(rel.generic_string());
    if (it == files_.end())
        throw std::runtime_error("missing in-memory asset: " + rel.generic_string());
    return it->second;
}

std::shared_ptr<const ModelAssetReader> make_directory_asset_reader(std::filesystem::path directory)
{
    return std::make_shared<DirectoryAssetReader>(std::move(directory));
}

std::shared_ptr<const ModelAssetReader> make_embedded_asset_reader(std::string_view profile)
{
    return std::make_shared<EmbeddedAssetReader>(std::string(profile));
}

std::shared_ptr<const ModelAssetReader> make_model_asset_reader(const std::filesystem::path& location)
{
    const std::string s = location.generic_string();
    if (s.starts_with(kEmbeddedPrefix)) {
        const std::string profile = s.substr(kEmbeddedPrefix.size());
        check_profile(profile);
        return make_embedded_asset_reader(profile);
    }
    return make_directory_asset_reader(location);
}

std::shared_ptr<const ModelAssetReader> resolve_model_asset_reader(
    const std::filesystem::path& model_dir, std::shared_ptr<const ModelAssetReader> override_reader)
{
    if (override_reader)
        return override_reader;
    if (!model_dir.empty())
        return make_model_asset_reader(model_dir);
    const std::filesystem::path embedded = default_model_location();
    if (embedded.empty())
        throw std::runtime_error("no embedded model; supply --model-dir with an AOT bundle");
    return make_model_asset_reader(embedded);
}

std::vector<std::string> list_embedded_model_profiles() { return {}; }

std::filesystem::path default_model_location()
{
    const std::vector<std::string> profiles = list_embedded_model_profiles();
    if (profiles.empty()) return {};
    const auto it = std::find(profiles.begin(), profiles.end(), "mlvc-psnr-v1");
    return std::string(kEmbeddedPrefix) + (it == profiles.end() ? profiles.front() : *it);
}

}  // namespace mlvc
