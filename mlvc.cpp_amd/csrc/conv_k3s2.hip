// 3x3 stride-2 tile variants of the MFMA conv kernel (conv_kernel.hpp) and of
// the weight-streaming kernel (conv_ws.hpp).

#include "conv_ws.hpp"

namespace mlvc_hip {
namespace conv {

namespace {
const Variant kTable[] = {
    MLVC_VARIANT_OCC(64, 4, 32, 3, 3, 2, 16, 4),
    MLVC_VARIANT_OCC(64, 8, 16, 3, 3, 2, 16, 4),
    MLVC_VARIANT_OCC(64, 2, 64, 3, 3, 2, 16, 4),
    MLVC_VARIANT_OCC(32, 4, 64, 3, 3, 2, 16, 4),
    MLVC_VARIANT(32, 4, 64, 3, 3, 2, 16),
    MLVC_VARIANT(64, 2, 64, 3, 3, 2, 16),
    MLVC_VARIANT(64, 4, 32, 3, 3, 2, 16),
    MLVC_VARIANT(64, 8, 16, 3, 3, 2, 16),
    MLVC_VARIANT(128, 2, 64, 3, 3, 2, 16),
    MLVC_VARIANT(64, 4, 32, 3, 3, 2, 32),
    MLVC_VARIANT(64, 8, 16, 3, 3, 2, 32),
    MLVC_VARIANT_WO(32, 2, 32, 3, 3, 2, 16, 1, 2, 4),
    MLVC_VARIANT_WO(64, 2, 32, 3, 3, 2, 16, 1, 2, 4),
    MLVC_VARIANT_WO(64, 2, 32, 3, 3, 2, 16, 2, 1, 4),
    MLVC_VARIANT_OCC(32, 2, 64, 3, 3, 2, 16, 4),
    MLVC_VARIANT_WS2(128, 4, 32, 32, 2, 4),
    MLVC_VARIANT_WS2(128, 2, 64, 32, 2, 4),
    MLVC_VARIANT_WS2(128, 2, 32, 64, 2, 4),
    MLVC_VARIANT_WS2(128, 4, 32, 64, 1, 4),
    MLVC_VARIANT_WS2(128, 2, 32, 32, 2, 4),
    MLVC_VARIANT_WS2(192, 4, 32, 32, 2, 3),
    MLVC_VARIANT_WS2(192, 2, 32, 64, 2, 3),
    // Deeper A rings, six waves over 192 output channels (one m-tile
    // each), and widths dividing 240 (24, 48).
    MLVC_VARIANT_WS2R(256, 2, 32, 64, 2, 8, 9),
    MLVC_VARIANT_WS2R(192, 2, 32, 64, 2, 6, 9),
    MLVC_VARIANT_WS2R(128, 4, 24, 32, 2, 4, 9),
    // Short, narrow tiles for deep convs onto few pixels (46x80 outputs).
    MLVC_VARIANT_WS2R(64, 2, 16, 64, 4, 2, 9),
    MLVC_VARIANT_WS2R(128, 2, 16, 64, 2, 4, 9),
    // All 192 output channels in one block over tiles dividing 136x240 (no
    // padded rows or columns), and one 32-pixel tile of all 256 channels per
    // CU at 68x120 (255 workgroups).
    MLVC_VARIANT_WS2R(192, 4, 24, 64, 2, 6, 9),
    MLVC_VARIANT_WS2R(192, 2, 48, 64, 2, 6, 9),
    MLVC_VARIANT_WS2R(256, 4, 8, 64, 2, 8, 9),
    // Four workgroups per CU (128 registers, 29 KB of LDS each): the
    // stride-2 convs wait on memory, and more waves keep more loads in flight.
    MLVC_VARIANT_WS2(128, 2, 32, 32, 4, 4),
    // One 8x16 tile of all 192 output channels per CU at 136x240 (255
    // workgroups of six waves, 109 KB of LDS for two halo buffers): each CU
    // streams the 442 KB weight set of a 128 -> 192 conv once, where the
    // 128-channel 2x32 tiles stream 1.25 MB per CU (4.25 workgroups of
    // 295 KB each).
    MLVC_VARIANT_WS2P(192, 8, 16, 32, 1, 6, 9),
};
}  // namespace

const Variant* variants_k3s2(int* n)
{
    *n = static_cast<int>(sizeof(kTable) / sizeof(kTable[0]));
    return kTable;
}

}  // namespace conv
}  // namespace mlvc_hip
