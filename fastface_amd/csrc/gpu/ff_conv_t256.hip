// ff_conv_t256.hip -- the layers with 256 output channels (stage 3).
// (one translation unit per layer group, so the kernel instantiations
// compile in parallel; ff_conv.hip looks layers up in every group's table)
#include "ff_conv_table.h"

namespace {
const ConvEntry kTable[] = {
    FF_P(128, 256, 28, FF_S2_SPLIT),
    FF_S2(256, 256, 28, FF_S3S2_SPLIT, 128),
    FF_CBIG(128, 256, 1, 2, 28, 1),
    FF_PB(256, 256, 14, FF_S3_SPLIT),
    FF_CBIG(128, 256, 1, 1, 14, 1),         // shortcut over the compact block input
};
}  // namespace

const ConvEntry* ff_conv_table_c256(int* n) {
    *n = (int)(sizeof kTable / sizeof kTable[0]);
    return kTable;
}
