// ff_conv_t512.hip -- the layers with 512 output channels (stage 4).
// (one translation unit per layer group, so the kernel instantiations
// compile in parallel; ff_conv.hip looks layers up in every group's table)
#include "ff_conv_table.h"

namespace {
const ConvEntry kTable[] = {
    FF_PB(256, 512, 14, 3),
    // (not fused with its 256-channel shortcut: the shortcut's four K steps,
    // single-buffered after the main loop, made the pair 3 % slower than two
    // launches at 1024 faces)
    FF_S2(512, 512, 14, FF_S4_SPLIT, 0),
    FF_CBIG(256, 512, 1, 2, 14, 1),
    FF_PB(512, 512, 7, FF_S4_SPLIT),
    FF_CBIG(256, 512, 1, 1, 7, 1),          // shortcut over the compact block input
};
}  // namespace

const ConvEntry* ff_conv_table_c512(int* n) {
    *n = (int)(sizeof kTable / sizeof kTable[0]);
    return kTable;
}
