// 1x1 (flattened pixels unless an unshuffle is fused) tile variants of the MFMA conv kernel (conv_kernel.hpp).

#include "conv_kernel.hpp"

namespace mlvc_hip {
namespace conv {

namespace {
const Variant kTable[] = {
    MLVC_VARIANT(32, 1, 256, 1, 1, 1, 32),
    MLVC_VARIANT(64, 1, 256, 1, 1, 1, 32),
    MLVC_VARIANT(64, 1, 128, 1, 1, 1, 32),
    MLVC_VARIANT(128, 1, 128, 1, 1, 1, 32),
    MLVC_VARIANT_S2D(64, 2, 64, 1, 1, 1, 32),
    MLVC_VARIANT_S2D(64, 4, 32, 1, 1, 1, 32),
};
}  // namespace

const Variant* variants_k1(int* n)
{
    *n = static_cast<int>(sizeof(kTable) / sizeof(kTable[0]));
    return kTable;
}

}  // namespace conv
}  // namespace mlvc_hip
