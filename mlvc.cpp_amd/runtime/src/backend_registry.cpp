// Named backend factory registry.
//
// Behaviour follows the reference's runtime/src/backend_registry.cpp:32-113:
// re-registering a name replaces its factory, the first registration (or any
// with make_default) becomes the default, create_backend resolves an empty
// name to the default and fills in a directory asset reader when none is set.

#include "mlvc/runtime/backend.hpp"

#include <algorithm>
#include <mutex>
#include <stdexcept>

namespace mlvc {
namespace {

struct Registry {
    std::mutex mutex;
    std::vector<std::pair<std::string, BackendFactory>> entries;
    std::string default_name;
};

Registry& registry()
{
    static Registry instance;
    return instance;
}

}  // namespace

void register_backend(std::string name, BackendFactory factory, bool make_default)
{
    if (name.empty())
        throw std::runtime_error("backend name must not be empty");
    if (!factory)
        throw std::runtime_error("backend factory must not be null");
    Registry& r = registry();
    std::lock_guard<std::mutex> lock(r.mutex);
    auto it = std::find_if(r.entries.begin(), r.entries.end(),
                           [&](const auto& e) { return e.first == name; });
    if (it != r.entries.end())
        it->second = std::move(factory);
    else
        r.entries.emplace_back(name, std::move(factory));
    if (make_default || r.default_name.empty())
        r.default_name = std::move(name);
}

std::vector<std::string> available_backends()
{
    Registry& r = registry();
    std::lock_guard<std::mutex> lock(r.mutex);
    std::vector<std::string> names;
    for (const auto& e : r.entries)
        names.push_back(e.first);
    return names;
}

std::string_view default_backend_name() noexcept
{
    Registry& r = registry();
    std::lock_guard<std::mutex> lock(r.mutex);
    return r.default_name.empty() ? std::string_view("none") : std::string_view(r.default_name);
}

std::unique_ptr<InferenceBackend> create_backend(const BackendOptions& options)
{
    BackendFactory factory;
    std::string target;
    {
        Registry& r = registry();
        std::lock_guard<std::mutex> lock(r.mutex);
        target = options.backend_name.empty() ? r.default_name : options.backend_name;
        if (target.empty())
            throw std::runtime_error("no inference backend is registered in this build");
        auto it = std::find_if(r.entries.begin(), r.entries.end(),
                               [&](const auto& e) { return e.first == target; });
        if (it == r.entries.end())
            throw std::runtime_error("unknown inference backend: " + target);
        factory = it->second;
    }
    BackendOptions resolved = options;
    resolved.backend_name = target;
    if (!resolved.asset_reader)
        resolved.asset_reader = resolve_model_asset_reader(resolved.model_dir, nullptr);
    return factory(resolved);
}

}  // namespace mlvc
