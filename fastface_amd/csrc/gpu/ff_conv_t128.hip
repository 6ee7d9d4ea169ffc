// ff_conv_t128.hip -- the layers with 128 output channels (stage 2).
// (one translation unit per layer group, so the kernel instantiations
// compile in parallel; ff_conv.hip looks layers up in every group's table)
#include "ff_conv_table.h"

namespace {
const ConvEntry kTable[] = {
    // 64 -> 128 at 56x56: one 64-channel run, so the patch kernel's single
    // input buffer fits two 256x128 workgroups per CU
    FF_P(64, 128, 56, 1),
    FF_S2(128, 128, 56, FF_S2_SPLIT, 64),
    FF_C128(64, 128, 1, 2, 56, 1),
    FF_P(128, 128, 28, FF_S2_SPLIT),
    FF_C128(64, 128, 1, 1, 28, 1),          // shortcut over the compact block input
};
}  // namespace

const ConvEntry* ff_conv_table_c128(int* n) {
    *n = (int)(sizeof kTable / sizeof kTable[0]);
    return kTable;
}
