// Static registration of the compiled-in backends, as the reference does in
// backends/selected_backends.cpp:1-32: this library provides "hip" and
// makes it the default.

#include "hip_backend.hpp"

namespace mlvc::detail {

extern bool g_hip_backend_registered;
bool g_hip_backend_registered = []() {
    hip_backend::register_hip_backend(true);
    return true;
}();

}  // namespace mlvc::detail
