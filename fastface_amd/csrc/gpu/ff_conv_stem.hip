// ff_conv_stem.hip -- the input layer: 3 -> 64, 3x3, s1 at 112x112 with the
// fp32 (or uint8 RGB) input quantized on load, one kernel per epilogue
// variant (stem_kernel, ff_conv_kernels.h).
#include "ff_conv_table.h"

namespace {
typedef void (*stem_fn)(const ConvArgs&, int grid, int tiles_per_wg, hipStream_t);
template <bool RGB8, int EPI>
void launch_stem_as(const ConvArgs& a, int grid, int tiles_per_wg, hipStream_t s) {
    hipLaunchKernelGGL((stem_kernel<RGB8, EPI>), dim3(grid), dim3(STEM_NT), 0, s, a, tiles_per_wg);
}

void launch_stem(const ConvArgs& a, int grid, int, hipStream_t s) {
    (void)grid;
    const int tiles = a.M / (112 * 2);
    const int slots = 256 * STEM_WG_PER_CU;
    const int per_wg = (tiles + slots - 1) / slots;
    const int wgs = (tiles + per_wg - 1) / per_wg;
    int epi;
    if (a.out_i32) epi = STEM_EPI_RAW;
    else if (a.flags & FFK_EPI_INSCALE) epi = STEM_EPI_INSC;
    else epi = (a.flags & FFK_EPI_PRELU ? (a.flags & FFK_EPI_PRELU_LE1 ? 2 : 1) : 0) + (a.flags & FFK_EPI_BN ? 3 : 0) +
               (a.flags & FFK_EPI_IN_RANGE ? 8 : 0);
    // the one-rounding tail where the host proved it (FFK_EPI_FMA_TAIL): for
    // the in-range forms without the compare/select PReLU
    if (epi >= 8 && epi != 9 && epi != 12 && (a.flags & FFK_EPI_FMA_TAIL)) epi += 8;
    stem_fn fn;
    const bool rgb8 = (a.flags & FFK_IN_RGB8) != 0;
    switch (epi) {
#define FF_STEM_CASE(E) case E: fn = rgb8 ? &launch_stem_as<true, E> : &launch_stem_as<false, E>; break;
    FF_STEM_CASE(0) FF_STEM_CASE(1) FF_STEM_CASE(2) FF_STEM_CASE(3) FF_STEM_CASE(4) FF_STEM_CASE(5)
    FF_STEM_CASE(8) FF_STEM_CASE(9) FF_STEM_CASE(10) FF_STEM_CASE(11) FF_STEM_CASE(12) FF_STEM_CASE(13)
    FF_STEM_CASE(16) FF_STEM_CASE(18) FF_STEM_CASE(19) FF_STEM_CASE(21)
    FF_STEM_CASE(STEM_EPI_INSC)
    default: fn = rgb8 ? &launch_stem_as<true, STEM_EPI_RAW> : &launch_stem_as<false, STEM_EPI_RAW>; break;
#undef FF_STEM_CASE
    }
    fn(a, wgs, per_wg, s);
}

const ConvEntry kTable[] = {
    {3, 64, 3, 1, 112, 112, 224, 64, &launch_stem, 1, nullptr, nullptr, "stem"},
};
}  // namespace

const ConvEntry* ff_conv_table_stem(int* n) {
    *n = (int)(sizeof kTable / sizeof kTable[0]);
    return kTable;
}
