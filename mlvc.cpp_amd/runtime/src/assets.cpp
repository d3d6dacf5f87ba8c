// Directory, embedded and in-memory model asset readers.

#include "mlvc/core/assets.hpp"

#include "mlvc_embedded_models.h"

#include <algorithm>
#include <cstdint>
#include <fstream>
#include <optional>
#include <span>
#include <stdexcept>

// The embedded image is optional: an image object defines these symbols
// (mlvc_embedded_models.h); without one they resolve to null.
extern "C" {
#pragma weak mlvc_embedded_models_start
#pragma weak mlvc_embedded_models_end
#pragma weak mlvc_embedded_models_index
#pragma weak mlvc_embedded_models_count
}

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

bool image_linked()
{
    return mlvc_embedded_models_start != nullptr && mlvc_embedded_models_end != nullptr &&
           mlvc_embedded_models_index != nullptr && &mlvc_embedded_models_count != nullptr;
}

std::span<const mlvc_embedded_model_asset> image_index()
{
    if (!image_linked()) return {};
    return {mlvc_embedded_models_index, static_cast<std::size_t>(mlvc_embedded_models_count)};
}

// The packed data, [start, end) (model_assets.cpp:50-61).
std::span<const std::byte> image_data()
{
    const auto begin = reinterpret_cast<std::uintptr_t>(mlvc_embedded_models_start);
    const auto end = reinterpret_cast<std::uintptr_t>(mlvc_embedded_models_end);
    if (end < begin) throw std::runtime_error("embedded model section is corrupt");
    return {reinterpret_cast<const std::byte*>(begin), static_cast<std::size_t>(end - begin)};
}

// First index entry of (profile, path), checked against the data
// (model_assets.cpp:63-76).
std::optional<std::span<const std::byte>> find_asset(std::string_view profile, std::string_view path)
{
    for (const auto& e : image_index()) {
        if (!e.profile || !e.path || profile != e.profile || path != e.path) continue;
        const auto data = image_data();
        if (e.offset > data.size() || e.size > data.size() - e.offset)
            throw std::runtime_error("embedded model index is corrupt");
        return data.subspan(static_cast<std::size_t>(e.offset), static_cast<std::size_t>(e.size));
    }
    return std::nullopt;
}

// Files of one profile of the linked image; without an image, every lookup
// misses and reads fail as in a build without embedded models.
class EmbeddedAssetReader final : public ModelAssetReader {
public:
    explicit EmbeddedAssetReader(std::string profile) : profile_(std::move(profile)) { check_profile(profile_); }

    std::string location_label() const override { return std::string(kEmbeddedPrefix) + profile_; }
    bool exists(const std::filesystem::path& rel) const override
    {
        return image_linked() && find_asset(profile_, rel.generic_string()).has_value();
    }
    std::vector<std::byte> read_binary(const std::filesystem::path& rel) const override
    {
        if (!image_linked())
            throw std::runtime_error("embedded models are disabled in this build (" + location_label() + ")");
        if (const auto a = find_asset(profile_, rel.generic_string())) return {a->begin(), a->end()};
        throw std::runtime_error("embedded model asset not found: " + profile_ + "/" + rel.generic_string());
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

std::vector<std::string> list_embedded_model_profiles()
{
    std::vector<std::string> out;
    for (const auto& e : image_index())
        if (e.profile && std::find(out.begin(), out.end(), e.profile) == out.end()) out.emplace_back(e.profile);
    return out;
}

std::filesystem::path default_model_location()
{
    const std::vector<std::string> profiles = list_embedded_model_profiles();
    if (profiles.empty()) return {};
    const auto it = std::find(profiles.begin(), profiles.end(), "mlvc-psnr-v1");
    return std::string(kEmbeddedPrefix) + (it == profiles.end() ? profiles.front() : *it);
}

}  // namespace mlvc
