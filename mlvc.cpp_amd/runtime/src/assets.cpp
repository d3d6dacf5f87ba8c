// Directory and in-memory model asset readers.

#include "mlvc/core/assets.hpp"

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

std::shared_ptr<const ModelAssetReader> resolve_model_asset_reader(
    const std::filesystem::path& model_dir, std::shared_ptr<const ModelAssetReader> override_reader)
{
    if (override_reader)
        return override_reader;
    if (model_dir.empty())
        throw std::runtime_error("no model directory or asset reader configured");
    return make_directory_asset_reader(model_dir);
}

}  // namespace mlvc
