// ff_conv_table.h -- the launch-table machinery of the int8 conv kernels:
// host launchers of each kernel template, the table entry type, the tile
// configurations and the entry macros.  Each ff_conv_t*.hip unit
// instantiates the kernels of its layer geometries into a table of its own
// (separate units compile in parallel); ff_conv.hip looks layers up in them.
#pragma once
#include "ff_conv_kernels.h"

namespace ffconv {

// (split: the K ranges per tile choose_launch picked; only the small-tile
// launcher reads it)
typedef void (*launch_fn)(const ConvArgs&, int grid, int split, hipStream_t);

template <int CIN, int COUT, int KS, int STRIDE, int HIN, int WIN, int BM, int BN, int KB, int PF,
          int MI, int NJ, int OCC, int SPLIT>
void launch_conv(const ConvArgs& a, int grid, int, hipStream_t s) {
    hipLaunchKernelGGL((conv_i8_kernel<CIN, COUT, KS, STRIDE, HIN, WIN, BM, BN, KB, PF, MI, NJ, OCC, SPLIT>),
                       dim3(grid), dim3(256), 0, s, a);
}

template <int CIN, int COUT, int KS, int STRIDE, int HIN, int WIN, int WM, int WN, int MI, int NJ,
          int NST, int WPE>
void launch_conv_dma(const ConvArgs& a, int grid, int, hipStream_t s) {
    hipLaunchKernelGGL((conv_dma_kernel<CIN, COUT, KS, STRIDE, HIN, WIN, WM, WN, MI, NJ, NST, WPE>),
                       dim3(grid), dim3(WM * WN * 64), 0, s, a);
}

template <int CIN, int COUT, int H, int WM, int WN, int MI, int NJ, int WPE>
void launch_patch(const ConvArgs& a, int grid, int, hipStream_t s) {
    hipLaunchKernelGGL((conv3_patch_kernel<CIN, COUT, H, H, WM, WN, MI, NJ, WPE>), dim3(grid),
                       dim3(WM * WN * 64), 0, s, a);
}

template <int CIN, int COUT, int H, int WM, int WN, int MI, int NJ, int KG, int WPE, int D, int U>
void launch_patch_kg(const ConvArgs& a, int grid, int, hipStream_t s) {
    hipLaunchKernelGGL((conv3_patch_kg_kernel<CIN, COUT, H, H, WM, WN, MI, NJ, KG, WPE, D, U>), dim3(grid),
                       dim3(WM * WN * KG * 64), 0, s, a);
}

template <int CIN, int COUT, int H, int WM, int WN, int MI, int NJ, int WPE>
void launch_s2(const ConvArgs& a, int grid, int, hipStream_t s) {
    hipLaunchKernelGGL((conv3s2_phase_kernel<CIN, COUT, H, H, WM, WN, MI, NJ, WPE>), dim3(grid),
                       dim3(WM * WN * 64), 0, s, a);
}

// A stride-2 conv and the 1x1 shortcut that adds its output, in one launch
// (conv3s2_shortcut_kernel): the same tiles as launch_s2.
typedef void (*launch_pair_fn)(const ConvArgs&, const ConvArgs&, int grid, hipStream_t);

template <int CIN, int COUT, int H, int WM, int WN, int MI, int NJ, int WPE, int CX>
void launch_s2_shortcut(const ConvArgs& a, const ConvArgs& b, int grid, hipStream_t s) {
    hipLaunchKernelGGL((conv3s2_shortcut_kernel<CIN, COUT, H, H, WM, WN, MI, NJ, WPE, CX>), dim3(grid),
                       dim3(WM * WN * 64), 0, s, a, b);
}

// the fused launcher of a stride-2 layer, or none (CX = 0)
template <int CIN, int COUT, int H, int WM, int WN, int MI, int NJ, int WPE, int CX>
constexpr launch_pair_fn s2_pair() {
    if constexpr (CX > 0) return &launch_s2_shortcut<CIN, COUT, H, WM, WN, MI, NJ, WPE, CX>;
    else return nullptr;
}

// Small-batch split-K tiling: 64x64 workgroup tiles (one 32x32 MFMA tile per
// wave), the K stages of a tile shared by `split` workgroups.
constexpr int FF_SM_BM = 64, FF_SM_BN = 64;
// The split path is taken when the whole-K tiling leaves most CUs idle and the
// split grid stays at most FF_SPLIT_MAX_WG workgroups: past that the partial
// tiles' round trip through memory costs more than the shorter K chain saves
// (measured on the chain at 1-32 faces with limits of 160, 256, 320 and 400:
// 320 is fastest; against 160 it splits the long-K layers at 4 and 8 faces
// too, 0.518 -> 0.453 ms at 4 faces and 0.613 -> 0.582 at 8).
constexpr int FF_SPLIT_MIN_WG = 256;
constexpr int FF_SPLIT_MAX_WG = 320;
// The whole-K 64x64 tiles (no exchange) are taken up to this many
// workgroups, and up to FF_TILE64_MAX_WG_SHARED per half where two halves of
// a batch run at once (FFK_SHARED_GPU).  Measured on the chain at 1-64 faces
// with limits 0, 200, 320 and 640: 640 is fastest at 8 and 16 faces (8:
// 0.524 ms without these tiles, 0.486 with), 200 at the 48- and 64-face
// halves; b=1 takes them for every layer without a split (0.399 -> 0.374 ms).
#ifndef FF_TILE64_MAX_WG
#define FF_TILE64_MAX_WG 640
#endif
#ifndef FF_TILE64_MAX_WG_SHARED
#define FF_TILE64_MAX_WG_SHARED 200
#endif
// split-K workspace: [counter per tile, fixed size][int32 partial tiles]
constexpr size_t FF_SPLIT_COUNTER_BYTES = FF_SPLIT_MAX_WG * sizeof(unsigned);
static_assert(FF_SPLIT_COUNTER_BYTES <= FF_WS_COUNTER_AREA, "counters stay in the reserved area");

struct ConvEntry {
    int cin, cout, ks, stride, hin, win, bm, bn;
    launch_fn fn;
    int split;          // K split of the small-batch variant (1: no partial tiles)
    launch_fn small;    // 64x64-tile split-K variant, or none
    launch_fn mid;      // variant for grids too small for the big tiles (default:
                        // the 128x128-tile register-staged kernel), or none
    const char* kind;   // name of `fn` (ffk_conv_variant)
    int mid_bm, mid_bn; // tile of `mid` when it is not 128x128
    const char* mid_kind;
    int pair_cx;          // stride-2 layers: input channels of the 1x1 shortcut
    launch_pair_fn pair;  // that `fn` runs fused with (conv3s2_shortcut_kernel), or none
};

// A grid of fewer big tiles than this (one per CU) leaves CUs idle; the
// 128x128 variant (four times the workgroups) is taken instead.  Between one
// and two big tiles per CU the big tiles are kept: measured on the chain,
// 192 faces 1.68 -> 1.59 ms and 256 faces 2.25 -> 1.97 ms against a limit
// of 512 (1024 faces unchanged).
constexpr int FF_MID_MAX_WG = 256;

// Tile configurations: (BM, BN, MI, NJ, OCC) -- workgroup tile, wave tile in
// 32x32 MFMA blocks, workgroups per CU.
//   T64:  Cout = 64, 256x64 tiles of 64x64 waves
//   T128: 128x128 tiles of 64x64 waves
//   TBIG: the Cout >= 256 layers (stages 3-4)
#define FF_T64 256, 64, 2, 2, 2
#define FF_T128 128, 128, 2, 2, 2
#ifndef FF_TBIG
#define FF_TBIG 128, 128, 2, 2, 2
#endif
// 128-byte stages wherever Cin allows (twice the MFMA work per barrier)
#define FF_KB(CIN) ((CIN) % 128 == 0 ? 128 : 64)
#define FF_PFS(CIN) (FF_KB(CIN) == 128 ? FF_PF128 : FF_PF)
// The 128x128 mid-size variants of the 512-channel layers keep two stages in
// flight: with three their address registers spilled to scratch.
#define FF_PF_MID(CIN) ((CIN) >= 512 ? 2 : FF_PFS(CIN))
#ifdef FF_KB_BIG_V
#define FF_KB_BIG(CIN) FF_KB_BIG_V
#define FF_PF_BIG(CIN) FF_PF_BIG_V
#else
#define FF_KB_BIG(CIN) FF_KB(CIN)
#define FF_PF_BIG(CIN) FF_PFS(CIN)
#endif
// The 64x64-tile kernels of a geometry whose long K chain is split SPLIT
// ways at small batches: that split, 3 ranges where SPLIT is larger (for
// batches whose SPLIT-way grid would be too large), and the whole-K tiles
// (split 1: tiny grids of the layers without a split, or batches where no
// split grid fits).  `split` is the one choose_launch picked.
// (three K stages of loads in flight: 1-1.6 % faster chains at 1-16 faces
// than two; four, at two workgroups per CU, slower at 16 faces)
#ifndef FF_SM_PF
#define FF_SM_PF 3
#endif
#ifndef FF_SM_OCC
#define FF_SM_OCC 4
#endif
template <int CIN, int COUT, int KS, int S, int H, int SPLIT>
void launch_small(const ConvArgs& a, int grid, int split, hipStream_t s) {
#define FF_SMALL_CONV(SP) \
    launch_conv<CIN, COUT, KS, S, H, H, FF_SM_BM, FF_SM_BN, FF_KB(CIN), FF_SM_PF, 1, 1, FF_SM_OCC, SP>(a, grid, SP, s)
    if constexpr (SPLIT > 1) {
        if (split == SPLIT) { FF_SMALL_CONV(SPLIT); return; }
    }
    if constexpr (SPLIT > 3) {
        if (split == 3) { FF_SMALL_CONV(3); return; }
    }
    FF_SMALL_CONV(1);
#undef FF_SMALL_CONV
}
template <int CIN, int COUT, int KS, int S, int H, int SPLIT>
constexpr launch_fn split_launch() {
    return &launch_small<CIN, COUT, KS, S, H, SPLIT>;
}
#define FF_ENTRY(CIN, COUT, KS, S, H, SPLIT, KB, PF, BM, BN, MI, NJ, OCC)       \
    {CIN, COUT, KS, S, H, H, BM, BN,                                             \
     &launch_conv<CIN, COUT, KS, S, H, H, BM, BN, KB, PF, MI, NJ, OCC, 1>, SPLIT, \
     split_launch<CIN, COUT, KS, S, H, SPLIT>(), nullptr, "staged"}
#define FF_CONV(CIN, COUT, KS, S, H, SPLIT, TILE) \
    FF_ENTRY(CIN, COUT, KS, S, H, SPLIT, FF_KB(CIN), FF_PFS(CIN), TILE)
#define FF_CONV_K(CIN, COUT, KS, S, H, SPLIT, KB, PF, TILE) \
    FF_ENTRY(CIN, COUT, KS, S, H, SPLIT, KB, PF, TILE)
#define FF_CONVB(CIN, COUT, KS, S, H, SPLIT) \
    FF_CONV_K(CIN, COUT, KS, S, H, SPLIT, FF_KB_BIG(CIN), FF_PF_BIG(CIN), FF_TBIG)

// Direct-to-LDS tiles (WM, WN, MI, NJ, NST, WPE): 8 waves of 2x2 MFMA tiles
// -> 256x128, a 3-stage ring, 4 waves per SIMD (two workgroups per CU).
#ifndef FF_TDMA
#define FF_TDMA 4, 2, 2, 2, 3, 4
#endif
#define FF_DENTRY(CIN, COUT, KS, S, H, SPLIT, WM, WN, MI, NJ, NST, WPE)              \
    {CIN, COUT, KS, S, H, H, WM * MI * 32, WN * NJ * 32,                             \
     &launch_conv_dma<CIN, COUT, KS, S, H, H, WM, WN, MI, NJ, NST, WPE>, SPLIT,      \
     split_launch<CIN, COUT, KS, S, H, SPLIT>(),                                     \
     &launch_conv<CIN, COUT, KS, S, H, H, 128, 128, FF_KB(CIN), FF_PF_MID(CIN), 2, 2, 2, 1>, "direct"}
#define FF_CONVD_K(CIN, COUT, KS, S, H, SPLIT, TILE) FF_DENTRY(CIN, COUT, KS, S, H, SPLIT, TILE)
#define FF_CONVD(CIN, COUT, KS, S, H, SPLIT) FF_CONVD_K(CIN, COUT, KS, S, H, SPLIT, FF_TDMA)
#define FF_DENTRY_NOMID(CIN, COUT, KS, S, H, SPLIT, WM, WN, MI, NJ, NST, WPE)        \
    {CIN, COUT, KS, S, H, H, WM * MI * 32, WN * NJ * 32,                             \
     &launch_conv_dma<CIN, COUT, KS, S, H, H, WM, WN, MI, NJ, NST, WPE>, SPLIT,      \
     split_launch<CIN, COUT, KS, S, H, SPLIT>(), nullptr, "direct"}
#define FF_CONVD64_K(CIN, COUT, KS, S, H, SPLIT, TILE) FF_DENTRY_NOMID(CIN, COUT, KS, S, H, SPLIT, TILE)
// Cout = 64: 4 waves of 2x2 MFMA tiles -> 256x64, a 2-stage ring, 4 waves per
// SIMD (four workgroups per CU)
#ifndef FF_T64DMA
#define FF_T64DMA 4, 1, 2, 2, 2, 4
#endif
#ifdef FF_NO_DMA
#define FF_C64(CIN, COUT, KS, S, H, SPLIT) FF_CONV(CIN, COUT, KS, S, H, SPLIT, FF_T64)
#else
#define FF_C64(CIN, COUT, KS, S, H, SPLIT) FF_CONVD64_K(CIN, COUT, KS, S, H, SPLIT, FF_T64DMA)
#endif
#ifdef FF_NO_DMA
#define FF_C128(CIN, COUT, KS, S, H, SPLIT) FF_CONV(CIN, COUT, KS, S, H, SPLIT, FF_T128)
#define FF_CBIG(CIN, COUT, KS, S, H, SPLIT) FF_CONVB(CIN, COUT, KS, S, H, SPLIT)
#else
#define FF_C128(CIN, COUT, KS, S, H, SPLIT) FF_CONVD(CIN, COUT, KS, S, H, SPLIT)
#define FF_CBIG(CIN, COUT, KS, S, H, SPLIT) FF_CONVD(CIN, COUT, KS, S, H, SPLIT)
#endif

// 3x3 stride-1 layers: the patch kernel (WM, WN, MI, NJ, WPE).  8 waves of
// 2x2 MFMA tiles -> 256x128, two workgroups per CU; Cout = 64: 4 waves ->
// 256x64 and one 64-channel run, so a single patch buffer: three workgroups
// per CU at 56x56 and at 112x112.
#ifndef FF_TPATCH
#define FF_TPATCH 4, 2, 2, 2, 4
#endif
#ifndef FF_TPATCH64
#define FF_TPATCH64 4, 1, 2, 2, 3
#endif
// 64 -> 64 at 56x56: 8 waves -> 512x64 tiles, two workgroups per CU (4 waves
// per SIMD; half the per-tile setup and patch halo per output; only waves 0-3
// load a step's 4 KB of weights).  3 % faster there, slower at 112x112.
#ifndef FF_TPATCH64W
#define FF_TPATCH64W 8, 1, 2, 2, 4
#endif
// Cout >= 256 (stages 3-4)
#ifndef FF_TPATCH_BIG
#define FF_TPATCH_BIG FF_TPATCH
#endif
#define FF_PENTRY(CIN, COUT, H, SPLIT, MID, WM, WN, MI, NJ, WPE)                      \
    {CIN, COUT, 3, 1, H, H, WM * MI * 32, WN * NJ * 32,                              \
     &launch_patch<CIN, COUT, H, WM, WN, MI, NJ, WPE>, SPLIT,                         \
     split_launch<CIN, COUT, 3, 1, H, SPLIT>(), MID, "patch"}
#define FF_PENTRY_K(CIN, COUT, H, SPLIT, MID, TILE) FF_PENTRY(CIN, COUT, H, SPLIT, MID, TILE)
#ifdef FF_NO_PATCH
#define FF_P(CIN, COUT, H, SPLIT) FF_CBIG(CIN, COUT, 3, 1, H, SPLIT)
#define FF_PB(CIN, COUT, H, SPLIT) FF_CBIG(CIN, COUT, 3, 1, H, SPLIT)
#define FF_P64(CIN, COUT, H, SPLIT) FF_C64(CIN, COUT, 3, 1, H, SPLIT)
#define FF_P64W(CIN, COUT, H, SPLIT) FF_C64(CIN, COUT, 3, 1, H, SPLIT)
#else
// Grids too small for the 256-row tiles (small batches): 128x128 tiles of
// four 64x64 waves, the channel runs shared by two K-groups inside the
// workgroup where they divide evenly (conv3_patch_kg_kernel): eight waves,
// one workgroup per CU.
#ifndef FF_MID_KG_MAX
#define FF_MID_KG_MAX 2
#endif
// (four groups only where each takes one 64-channel run: with two runs per
// group the double-buffered patches of four groups exceed the LDS)
#define FF_MID_KG(CIN) ((CIN) == 256 && FF_MID_KG_MAX >= 4 ? 4 : (((CIN) / 64) % 2 == 0 && FF_MID_KG_MAX >= 2 ? 2 : 1))
#define FF_MID_WPE(CIN) (FF_MID_KG(CIN) == 2 ? 2 : 4)
// one barrier per FF_MID_STEPS taps (a small grid has one workgroup per CU:
// nothing else fills the SIMDs while its waves meet at a barrier); weights
// FF_MID_DEPTH taps ahead
#ifndef FF_MID_STEPS
#define FF_MID_STEPS 2
#endif
#ifndef FF_MID_DEPTH
#define FF_MID_DEPTH FF_MID_STEPS
#endif
#define FF_PMID(CIN, COUT, H)                                                        \
    (&launch_patch_kg<CIN, COUT, H, 2, 2, 2, 2, FF_MID_KG(CIN), FF_MID_WPE(CIN), FF_MID_DEPTH, FF_MID_STEPS>)
#define FF_PENTRY_MID(CIN, COUT, H, SPLIT, WM, WN, MI, NJ, WPE)                       \
    {CIN, COUT, 3, 1, H, H, WM * MI * 32, WN * NJ * 32,                              \
     &launch_patch<CIN, COUT, H, WM, WN, MI, NJ, WPE>, SPLIT,                         \
     split_launch<CIN, COUT, 3, 1, H, SPLIT>(), FF_PMID(CIN, COUT, H), "patch", 128, 128, "patch_kg"}
#define FF_PENTRY_MID_K(CIN, COUT, H, SPLIT, TILE) FF_PENTRY_MID(CIN, COUT, H, SPLIT, TILE)
#define FF_P(CIN, COUT, H, SPLIT) FF_PENTRY_MID_K(CIN, COUT, H, SPLIT, FF_TPATCH)
#define FF_PB(CIN, COUT, H, SPLIT) FF_PENTRY_MID_K(CIN, COUT, H, SPLIT, FF_TPATCH_BIG)
#define FF_P64(CIN, COUT, H, SPLIT) FF_PENTRY_K(CIN, COUT, H, SPLIT, nullptr, FF_TPATCH64)
// (small grids: the 256x64 tiles, twice the workgroups)
#define FF_P64W(CIN, COUT, H, SPLIT)                                                \
    {CIN, COUT, 3, 1, H, H, 512, 64, &launch_patch<CIN, COUT, H, FF_TPATCH64W>, SPLIT, \
     split_launch<CIN, COUT, 3, 1, H, SPLIT>(), &launch_patch<CIN, COUT, H, FF_TPATCH64>, "patch", \
     256, 64, "patch"}
#endif

// 3x3 stride-2 layers at large batches: the phase-split patch kernel
// (conv3s2_phase_kernel) -- 256x128 tiles of 8 waves, 256x64 of 4 waves for
// Cout = 64; small grids keep the register-staged 128x128 tiles / split-K.
#ifndef FF_S2_PHASE
#define FF_S2_PHASE 1
#endif
#ifndef FF_TS2
#define FF_TS2 4, 2, 2, 2, 4
#endif
#ifndef FF_TS2_64
#define FF_TS2_64 4, 1, 2, 2, 4
#endif
// CX: input channels of the block's 1x1 shortcut, which the phase kernel
// runs fused (conv3s2_shortcut_kernel), or 0: never fused
#define FF_S2ENTRY(CIN, COUT, H, SPLIT, MID, CX, WM, WN, MI, NJ, WPE)                \
    {CIN, COUT, 3, 2, H, H, WM * MI * 32, WN * NJ * 32,                              \
     &launch_s2<CIN, COUT, H, WM, WN, MI, NJ, WPE>, SPLIT,                            \
     split_launch<CIN, COUT, 3, 2, H, SPLIT>(), MID, "phase", 0, 0, nullptr,          \
     CX, s2_pair<CIN, COUT, H, WM, WN, MI, NJ, WPE, CX>()}
#define FF_S2ENTRY_K(CIN, COUT, H, SPLIT, MID, CX, TILE) FF_S2ENTRY(CIN, COUT, H, SPLIT, MID, CX, TILE)
#if FF_S2_PHASE
#define FF_S2(CIN, COUT, H, SPLIT, CX)                                              \
    FF_S2ENTRY_K(CIN, COUT, H, SPLIT,                                               \
                 (&launch_conv<CIN, COUT, 3, 2, H, H, 128, 128, FF_KB(CIN), FF_PF_MID(CIN), 2, 2, 2, 1>), CX, FF_TS2)
#define FF_S2_64(CIN, COUT, H, SPLIT, CX) FF_S2ENTRY_K(CIN, COUT, H, SPLIT, nullptr, CX, FF_TS2_64)
#else
#define FF_S2(CIN, COUT, H, SPLIT, CX) FF_CBIG(CIN, COUT, 3, 2, H, SPLIT)
#define FF_S2_64(CIN, COUT, H, SPLIT, CX) FF_C64(CIN, COUT, 3, 2, H, SPLIT)
#endif

#ifndef FF_S2_SPLIT
#define FF_S2_SPLIT 3
#endif
#ifndef FF_S3_SPLIT
#define FF_S3_SPLIT 3
#endif
#ifndef FF_S3S2_SPLIT
#define FF_S3S2_SPLIT 6
#endif
#ifndef FF_S4_SPLIT
#define FF_S4_SPLIT 9
#endif
// split: how many workgroups share the K stages of one small-batch tile (1:
// never split).  The 3x3 layers with 128 input channels or more gain from it
// (9, 18 or 36 stages of 128 bytes; the stage-2 layers measured 0.511 ->
// 0.486 ms for the b=1 chain with 3 ranges of 3 stages).  Each workgroup's
// partial tile makes a round trip through memory, so fewer splits can win:
// 256->256 @14 (12 launches at b=1) with 3 instead of 9 took the b=1 chain
// from 0.485 to 0.433 ms (and with the present exchange 0.399 ms against
// 0.414 with 6 and 0.442 with 9); 3 for the stride-2 and 512-channel layers
// measured the same as their 6 and 9, 2 (and 4) slower.
// One face gives 48-156 workgroups.  The 64-channel layers' 9 stages of 64
// bytes are too short to pay for the partial-sum exchange.
}  // namespace ffconv

using namespace ffconv;

// The tables of the ff_conv_t*.hip units (a ConvEntry array and its size).
const ConvEntry* ff_conv_table_stem(int* n);
const ConvEntry* ff_conv_table_c64(int* n);
const ConvEntry* ff_conv_table_c128(int* n);
const ConvEntry* ff_conv_table_c256(int* n);
const ConvEntry* ff_conv_table_c512(int* n);
// Any other conv geometry (ff_conv_generic.hip): one workgroup per 64x64
// output tile; a.M holds the launch's output pixels.
long long ff_conv_generic_grid(long long M, int cin, int cout);
int ff_conv_generic_launch(const ConvArgs& a, const ffk_conv_desc* d, hipStream_t s);
// FC head as an MFMA GEMM (ff_conv_fc.hip)
constexpr int FC_SPLIT = 8;
size_t ffk_fc_split_ws_bytes(int batch);
int ffk_fc_gemm_launch(const ffk_fc_desc* d, hipStream_t s);

