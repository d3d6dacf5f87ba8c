// 3x3 stride-1 tile variants of the MFMA conv kernel (conv_kernel.hpp).

#include "conv_ws.hpp"

namespace mlvc_hip {
namespace conv {

namespace {
const Variant kTable[] = {
    MLVC_VARIANT_OCC(32, 4, 64, 3, 3, 1, 16, 4),
    MLVC_VARIANT_OCC(32, 8, 32, 3, 3, 1, 16, 4),
    MLVC_VARIANT_OCC(64, 4, 32, 3, 3, 1, 16, 4),
    MLVC_VARIANT_S2D(32, 4, 64, 3, 3, 1, 16),
    MLVC_VARIANT_S2D(32, 8, 32, 3, 3, 1, 16),
    MLVC_VARIANT_S2D(64, 4, 64, 3, 3, 1, 16),
    MLVC_VARIANT_S2D(64, 8, 32, 3, 3, 1, 16),
    MLVC_VARIANT(64, 16, 16, 3, 3, 1, 16),
    MLVC_VARIANT(64, 2, 64, 3, 3, 1, 16),
    MLVC_VARIANT_S2D(64, 4, 32, 3, 3, 1, 16),
    MLVC_VARIANT_S2D(64, 8, 16, 3, 3, 1, 16),
    MLVC_VARIANT(128, 4, 64, 3, 3, 1, 16),
    MLVC_VARIANT(128, 8, 32, 3, 3, 1, 16),
    MLVC_VARIANT_W(128, 16, 32, 3, 3, 1, 16, 1, 8),
    MLVC_VARIANT_W(128, 8, 64, 3, 3, 1, 16, 1, 8),
    MLVC_VARIANT_W(256, 8, 32, 3, 3, 1, 16, 2, 4),
    MLVC_VARIANT_W(256, 4, 64, 3, 3, 1, 16, 2, 4),
    MLVC_VARIANT_W(64, 16, 32, 3, 3, 1, 16, 1, 8),
    MLVC_VARIANT_W(128, 16, 16, 3, 3, 1, 16, 2, 4),
    MLVC_VARIANT(128, 16, 16, 3, 3, 1, 16),
    MLVC_VARIANT(32, 8, 32, 3, 3, 1, 32),
    MLVC_VARIANT(64, 8, 32, 3, 3, 1, 32),
    MLVC_VARIANT(64, 4, 64, 3, 3, 1, 32),
    MLVC_VARIANT(64, 8, 16, 3, 3, 1, 32),
    MLVC_VARIANT_DB(64, 8, 32, 3, 3, 1, 16),
    MLVC_VARIANT_DB(32, 8, 32, 3, 3, 1, 16),
    MLVC_VARIANT_DB(128, 8, 32, 3, 3, 1, 16),
    MLVC_VARIANT_DB(128, 4, 64, 3, 3, 1, 16),
    MLVC_VARIANT_DB(64, 4, 64, 3, 3, 1, 16),
    MLVC_VARIANT_OCC(32, 2, 64, 3, 3, 1, 16, 4),
    MLVC_VARIANT_WO(32, 2, 32, 3, 3, 1, 16, 1, 2, 4),
    MLVC_VARIANT_WO(64, 2, 32, 3, 3, 1, 16, 1, 2, 4),
    MLVC_VARIANT_WS(256, 4, 32, 128, 2),
    MLVC_VARIANT_WS(128, 4, 32, 128, 2),
    MLVC_VARIANT_WS(256, 4, 32, 64, 2),
    MLVC_VARIANT_WS(128, 4, 32, 64, 2),
    MLVC_VARIANT_WS(256, 2, 32, 128, 2),
    MLVC_VARIANT_WSR(128, 4, 32, 64, 2, 9),
    MLVC_VARIANT_WSR(256, 2, 32, 128, 2, 9),
    // Widths that divide 120 and 240 (24, 40) or 240 and 480 (48), so the
    // 68x120 and 136x240 decoder convs run without padded columns.
    MLVC_VARIANT_WSR(128, 4, 24, 64, 2, 9),
    MLVC_VARIANT_WSR(128, 8, 24, 64, 2, 9),
    MLVC_VARIANT_WSR(128, 4, 40, 64, 2, 9),
    MLVC_VARIANT_WSR(128, 4, 48, 64, 2, 9),
    MLVC_VARIANT_WS(128, 8, 32, 64, 2),
    // Two m-tiles per wave with a 9-step ring.
    MLVC_VARIANT_WSR(256, 4, 24, 64, 2, 9),
    MLVC_VARIANT_WSR(256, 2, 48, 64, 2, 9),
    // Pipelined passes of 32 channels.
    MLVC_VARIANT_WSP(256, 4, 32, 32, 2, 3),
    MLVC_VARIANT_WSP(128, 8, 32, 32, 2, 3),
    MLVC_VARIANT_WSP(128, 4, 32, 32, 2, 9),
    MLVC_VARIANT_WSP(128, 4, 48, 32, 2, 9),
    MLVC_VARIANT_WSP(128, 4, 24, 32, 2, 9),
    // 64 output channels on two waves, more workgroups per CU.
    MLVC_VARIANT_WSW(64, 2, 32, 64, 4, 2, 9),
    MLVC_VARIANT_WSW(64, 4, 32, 64, 3, 2, 9),
    MLVC_VARIANT_WSW(64, 8, 32, 64, 2, 2, 9),
    // Short, narrow tiles: enough workgroups for deep convs over few pixels
    // (46x80 and 92x160 planes).
    MLVC_VARIANT_WSW(64, 2, 16, 64, 4, 2, 9),
    MLVC_VARIANT_WSR(128, 2, 16, 64, 2, 9),
    // 512 output channels at 136x240 in one round of two workgroups per CU:
    // 255 8x16 tiles x 2 channel blocks = 510 workgroups, where the 4x48
    // tiles' 680 take two rounds of 512 slots with the second a third full.
    // LDS for the channel-last DEPTH_TO_SPACE(2) output tile (72 KB).
    MLVC_VARIANT_WSPD(256, 8, 16, 32, 2, 3),
};
}  // namespace

const Variant* variants_k3s1(int* n)
{
    *n = static_cast<int>(sizeof(kTable) / sizeof(kTable[0]));
    return kTable;
}

}  // namespace conv
}  // namespace mlvc_hip
