// ff_conv_t64.hip -- the 64-channel layers (stage 1 at 112x112 and 56x56).
// (one translation unit per layer group, so the kernel instantiations
// compile in parallel; ff_conv.hip looks layers up in every group's table)
#include "ff_conv_table.h"

namespace {
const ConvEntry kTable[] = {
    FF_P64(64, 64, 112, 1),
    FF_S2_64(64, 64, 112, 1, 64),
    FF_C64(64, 64, 1, 2, 112, 1),
    FF_P64W(64, 64, 56, 1),
    // the 1x1 shortcut over a block input stored at its even pixels only
    // (FFK_OUT_X_EVEN): stride 1 over the compact tensor
    FF_C64(64, 64, 1, 1, 56, 1),
};
}  // namespace

const ConvEntry* ff_conv_table_c64(int* n) {
    *n = (int)(sizeof kTable / sizeof kTable[0]);
    return kTable;
}
