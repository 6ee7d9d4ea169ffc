// ff_conv.hip -- NHWC int8 convolution as implicit GEMM on gfx950 i8 MFMA
// (v_mfma_i32_32x32x32_i8, int32 accumulation) with the requantization
// epilogue fused into the store stage.
//
// GEMM view of one layer: M = batch*Hout*Wout output pixels, N = Cout,
// K = KH*KW*Cin in (kh, kw, ci) order.  The reference computes exactly these
// integers with im2col + a u8 x s8 VNNI GEMM and a -128*colsum correction
// (kernels/conv2d_nhwc.c:29-220, kernels/gemm_int8_v2.c:42-110); signed i8
// MFMA needs no correction, and integer sums do not depend on their order,
// so the accumulators are bit-identical.
//
// Two kernels share the epilogue: conv_dma_kernel (large grids: operands go
// straight from global into a swizzled LDS ring with global_load_lds_dwordx4)
// and conv_i8_kernel (small grids and split-K: register-staged operands).
//
// conv_i8_kernel K loop: workgroup = 4 wave64s computing a BM x BN tile (each
// wave MI x NJ MFMA 32x32 tiles).  Per K stage of KB = 64 or 128 bytes each thread fetches
// 16-byte pieces of the implicit im2col rows (one input pixel's channel run;
// padding taps read a zero page, so there are no branches) and of the packed
// weights.  PF stages of loads are in flight in registers; each stage goes
// through a double-buffered LDS tile whose KB+16-byte row pitch makes the
// ds_read_b128 MFMA operand reads conflict-free.  Small batches of the layers
// with long K chains split the stages of a tile over several workgroups
// (split-K, int32 partial tiles in a caller workspace).
//
// Epilogue straight from the accumulator registers: in the 32x32 MFMA result
// every lane owns one output channel (column) and 16 pixels (rows), so each
// lane needs the per-channel parameters of only NJ = 2 channels.  The int8
// results go through a small per-wave LDS byte tile only to leave as
// coalesced 16-byte stores.  The BN second output is a per-channel 256-entry
// table lookup (BN is a fixed function of the int8 value; the table is built
// bit-exactly on the host, ffk_make_bn_lut).
#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>

#include "ff_internal.h"
#include "ff_numerics.h"

// patch kernel: ask the scheduler to interleave LDS reads and MFMAs
// (__builtin_amdgcn_iglp_opt(1)) in every K step
#ifndef FF_PATCH_IGLP
#define FF_PATCH_IGLP 1
#endif
// the same hint in the direct-to-LDS kernel's K stages (neutral to 1.6 %
// faster on its layers)
#ifndef FF_DMA_IGLP
#define FF_DMA_IGLP 1
#endif

// stages of global loads kept in flight per thread (64- and 128-byte stages)
#ifndef FF_PF
#define FF_PF 4
#endif
#ifndef FF_PF128
#define FF_PF128 3
#endif

constexpr int FF_LUT_PITCH = 272;   // LDS row pitch of a 256-entry table

// 64 zero bytes: the source of every padding tap / out-of-range row load
__device__ __align__(64) int8_t ff_zero_page[64];

// Direct-to-LDS load of 16 bytes per lane: lane L of the wave writes
// lds_wave_base + 16 L (1 KB per wave load); counted by vmcnt.
__device__ __forceinline__ void dma16(const int8_t* g, int8_t* lds_wave_base) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds_wave_base, 16, 0, 0);
}

struct ConvArgs {
    const int8_t* in;
    const float* in_f32;
    const float* in_inv;
    const ffk_io* io;
    const int8_t* w;
    const float* params;
    const int8_t* add_src;
    const int8_t* bn_lut;
    int8_t* out;
    int8_t* out_bn;
    int32_t* out_i32;
    float* out_f32;
    const float* fc_ws;
    const float* fc_bias;
    const int8_t* in_lut;   // FFK_IN_RGB8: [3][256] input quantization table
    int32_t* ws;            // split-K partial tiles
    unsigned* counters;     // split-K arrival counters, one per tile (zero between launches)
    int M;
    int flags;
    float in_scale;
    int tiles_n;
};

// ---------------------------------------------------------------------------
// Epilogue of one wave's MI x NJ block of 32x32 MFMA tiles.
//   mrow0: global pixel index of the block's first row
//   ncol0: global output channel of the block's first column
//   Ws:    wave-private LDS byte tile [MI*32][NJ*32 + 16]
//   Lw:    BN table of channel ncol0 (row pitch FF_LUT_PITCH) or null
// ---------------------------------------------------------------------------
template <int MI, int NJ>
constexpr int wave_tile_bytes() { return MI * 32 * (NJ * 32 + 16); }

// Per-channel parameters of the NJ channels a lane owns (columns ncol0 +
// j*32 + lane%32).  Loaded separately so that a kernel walking several tiles
// of the same channels loads them once.
template <int NJ>
struct EpiParams {
    float ws[NJ], bias[NJ], slope[NJ], adds[NJ], inv[NJ];
};

template <int COUT, int NJ>
__device__ __forceinline__ EpiParams<NJ> load_epi_params(const ConvArgs& a, int ncol0) {
    EpiParams<NJ> P;
    const int lc = threadIdx.x & 31;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int c = ncol0 + j * 32 + lc;
        P.ws[j] = a.params[FFK_P_WS * COUT + c];
        P.bias[j] = a.params[FFK_P_BIAS * COUT + c];
        P.inv[j] = a.params[FFK_P_INV * COUT + c];
        P.slope[j] = a.params[FFK_P_SLOPE * COUT + c];
        P.adds[j] = a.params[FFK_P_ADDSCALE * COUT + c];
    }
    return P;
}

// Where output pixel m's X row goes: out + m*COUT, or with FFK_OUT_X_EVEN
// (HO x WO images, both even) its slot in the [HO/2][WO/2] tensor of the
// even-row, even-column pixels, and null for every other pixel.
template <int COUT, int HO, int WO>
__device__ __forceinline__ int8_t* x_row(const ConvArgs& a, int m) {
    if constexpr (HO % 2 == 0 && WO % 2 == 0) {
        if (a.flags & FFK_OUT_X_EVEN) {
            const int img = m / (HO * WO);
            const int rem = m - img * (HO * WO);
            const int oh = rem / WO, ow = rem - oh * WO;
            if ((oh | ow) & 1) return nullptr;
            return a.out + (((size_t)img * (HO / 2) + (oh >> 1)) * (WO / 2) + (ow >> 1)) * COUT;
        }
    }
    return a.out + (size_t)m * COUT;
}

// PRELU: 0 none, 1 f < 0 ? f*slope : f, 2 max(f, f*slope) (the same values
// when every slope is at most 1 and f is never infinite: FFK_EPI_PRELU_LE1).
// INSC: f = f * in_scale first (FFW2/FFW3 models; FFW4 skips the multiply).
// RANGE: every requant value is known in range (FFK_EPI_IN_RANGE).
// HO x WO: output image size (FFK_OUT_X_EVEN addressing).
// LUT_DMA: the BN table was issued as direct-to-LDS loads (issue_bn_lut) that
// may still be in flight; they are waited for before the flush.
template <int COUT, int MI, int NJ, int PRELU, bool ADD, bool BN2, bool INSC, bool RANGE, int HO, int WO,
          bool LUT_DMA = false>
__device__ __forceinline__ void wave_epi_i8(const v16i (&acc)[MI][NJ], const ConvArgs& a,
                                            const EpiParams<NJ>& prm, int mrow0, int ncol0, int8_t* Ws,
                                            const int8_t* Lw) {
    constexpr int P = NJ * 32 + 16;
    constexpr int ROWS = MI * 32;
    constexpr int CH = NJ * 2;          // 16-byte chunks per tile row
    constexpr int RPI = 64 / CH;        // tile rows per copy instruction
    constexpr int SPR = P / 16;         // 16-byte slots per tile row (the last one unused)
    constexpr int RSLOTS = ROWS * SPR;
    const int lane = threadIdx.x & 63;
    const int lc = lane & 31;
    const int lh = lane >> 5;
    const float* ws = prm.ws;
    const float* bias = prm.bias;
    const float* p2 = prm.slope;
    const float* adds = prm.adds;
    const float* inv = prm.inv;
    if (ADD && RSLOTS % 64 == 0) {
        // residual tile -> this wave's LDS tile as direct-to-LDS loads: slot s
        // of wave load k is tile row (64k+s)/SPR, piece (64k+s)%SPR; unused
        // pieces and rows past M fetch the zero page.  One wait covers them
        // and any BN-table loads issued before; the tile is this wave's own,
        // so no barrier.
        // (opaque: computed here, not folded into values kept across the
        // main loop)
        int lane_o = lane, m_o = mrow0;
        asm volatile("" : "+v"(lane_o), "+v"(m_o));
#pragma unroll
        for (int k = 0; k < RSLOTS / 64; k++) {
            const int slot = k * 64 + lane_o;
            const int row = slot / SPR;
            const int pc = slot - row * SPR;
            const int m = m_o + row;
            const int8_t* src = pc < CH && m < a.M ? a.add_src + (size_t)m * COUT + ncol0 + pc * 16 : ff_zero_page;
            dma16(src, Ws + k * 1024);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else if (ADD) {   // residual tile -> LDS (coalesced 16-byte loads)
#pragma unroll
        for (int k = 0; k < ROWS / RPI; k++) {
            const int row = lane / CH + k * RPI;
            const int ch = lane % CH;
            const int m = mrow0 + row;
            const int8_t* src = m < a.M ? a.add_src + (size_t)m * COUT + ncol0 + ch * 16 : ff_zero_page;
            *reinterpret_cast<v4i*>(Ws + row * P + ch * 16) = *reinterpret_cast<const v4i*>(src);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = i * 32 + (r >> 2) * 8 + lh * 4 + (r & 3);
                const int col = j * 32 + lc;
                float f = (float)acc[i][j][r];
                if (INSC) f = f * a.in_scale;
                f = f * ws[j];
                f = f + bias[j];
                if (ADD) f = ff::add_residual(f, (int32_t)Ws[row * P + col], adds[j]);
                if (PRELU == 1) f = ff::prelu(f, p2[j]);
                if (PRELU == 2) f = ff::prelu_le1(f, p2[j]);
                Ws[row * P + col] = (int8_t)(RANGE ? ff::requant_haz_in_range(f * inv[j])
                                                   : ff::requant_haz(f * inv[j]));
                // one 32x32 tile at a time: keeps the compiler from hoisting
                // every residual read of the wave tile into registers
                if (r == 15) asm volatile("" ::: "memory");
            }
    if (BN2 && LUT_DMA) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    // Flush: 16-byte chunks of the X tile go out as they are; the BN second
    // output maps each byte through its channel's table on the way.
#pragma unroll
    for (int k = 0; k < ROWS / RPI; k++) {
        const int row = lane / CH + k * RPI;
        const int ch = lane % CH;
        const int m = mrow0 + row;
        const v4i v = *reinterpret_cast<const v4i*>(Ws + row * P + ch * 16);
        if (m < a.M) {
            if (a.out) {
                int8_t* xo = x_row<COUT, HO, WO>(a, m);
                if (xo) *reinterpret_cast<v4i*>(xo + ncol0 + ch * 16) = v;
            }
            if (BN2) {
                const int8_t* L = Lw + (ch * 16) * FF_LUT_PITCH + 128;
                v4i o;
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    uint32_t packed = 0;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int q = (int8_t)((uint32_t)v[w] >> (e * 8));
                        packed |= (uint32_t)(uint8_t)L[(w * 4 + e) * FF_LUT_PITCH + q] << (e * 8);
                    }
                    o[w] = (int)packed;
                }
                *reinterpret_cast<v4i*>(a.out_bn + (size_t)m * COUT + ncol0 + ch * 16) = o;
            }
        }
        if (BN2) asm volatile("" ::: "memory");
    }
}

// raw int32 accumulators or the FC head's fp32 output (FC: the FC GEMM
// instantiation only): 4-byte elements are stored straight from registers (a
// half-wave writes 128 contiguous bytes)
template <int COUT, int MI, int NJ, bool FC>
__device__ __forceinline__ void wave_epi_wide(const v16i (&acc)[MI][NJ], const ConvArgs& a, int mrow0,
                                              int ncol0) {
    const int lane = threadIdx.x & 63;
    const int lc = lane & 31;
    const int lh = lane >> 5;
    if (!FC) {
#pragma unroll
        for (int i = 0; i < MI; i++)
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                int32_t* col = a.out_i32 + ncol0 + j * 32 + lc;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = mrow0 + i * 32 + (r >> 2) * 8 + lh * 4 + (r & 3);
                    if (m < a.M) col[(size_t)m * COUT] = acc[i][j][r];
                }
                asm volatile("" ::: "memory");
            }
        return;
    }
    float* out = a.out_f32 ? a.out_f32 : a.io->out;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int c = ncol0 + j * 32 + lc;
        const float ws = a.fc_ws[c], bias = a.fc_bias[c];
#pragma unroll
        for (int i = 0; i < MI; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int m = mrow0 + i * 32 + (r >> 2) * 8 + lh * 4 + (r & 3);
                if (m < a.M) out[(size_t)m * COUT + c] = ff::fc_out(acc[i][j][r], a.in_scale, ws, bias);
            }
    }
}

// int8 epilogue variants dispatched on the (uniform) flags, parameters given.
// FFK_EPI_PRELU_LE1 and FFK_EPI_IN_RANGE apply to the FFW4 path (no in-scale);
// the in-range variants exist for the PReLU forms FFW4 models use (none, or
// max(f, f*slope)).
template <int COUT, int MI, int NJ, bool INSC, int HO, int WO>
__device__ __forceinline__ void wave_epilogue_f(const v16i (&acc)[MI][NJ], const ConvArgs& a,
                                                const EpiParams<NJ>& P, int mrow0, int ncol0, int8_t* Ws,
                                                const int8_t* Lw) {
    const bool le1 = !INSC && (a.flags & FFK_EPI_PRELU_LE1);
    const bool rng = !INSC && (a.flags & FFK_EPI_IN_RANGE);
#define FF_EPI(PR, AD, BN, RG) \
    wave_epi_i8<COUT, MI, NJ, PR, AD, BN, INSC, RG, HO, WO, true>(acc, a, P, mrow0, ncol0, Ws, Lw)
    switch (a.flags & (FFK_EPI_PRELU | FFK_EPI_ADD | FFK_EPI_BN)) {
    case 0:
        if (rng) FF_EPI(0, false, false, true);
        else FF_EPI(0, false, false, false);
        break;
    case FFK_EPI_PRELU:
        if (le1 && rng) FF_EPI(2, false, false, true);
        else if (le1) FF_EPI(2, false, false, false);
        else FF_EPI(1, false, false, false);
        break;
    case FFK_EPI_ADD:
        if (rng) FF_EPI(0, true, false, true);
        else FF_EPI(0, true, false, false);
        break;
    case FFK_EPI_BN:
        if (rng) FF_EPI(0, false, true, true);
        else FF_EPI(0, false, true, false);
        break;
    case FFK_EPI_PRELU | FFK_EPI_BN:
        if (le1 && rng) FF_EPI(2, false, true, true);
        else if (le1) FF_EPI(2, false, true, false);
        else FF_EPI(1, false, true, false);
        break;
    case FFK_EPI_ADD | FFK_EPI_BN:
        if (rng) FF_EPI(0, true, true, true);
        else FF_EPI(0, true, true, false);
        break;
    case FFK_EPI_PRELU | FFK_EPI_ADD: FF_EPI(1, true, false, false); break;
    default: FF_EPI(1, true, true, false); break;
    }
#undef FF_EPI
}

template <int COUT, int MI, int NJ, int HO, int WO>
__device__ __forceinline__ void wave_epilogue_p(const v16i (&acc)[MI][NJ], const ConvArgs& a,
                                                const EpiParams<NJ>& P, int mrow0, int ncol0, int8_t* Ws,
                                                const int8_t* Lw) {
    if (a.out_i32) {
        wave_epi_wide<COUT, MI, NJ, false>(acc, a, mrow0, ncol0);
        return;
    }
    if (a.flags & FFK_EPI_INSCALE) wave_epilogue_f<COUT, MI, NJ, true, HO, WO>(acc, a, P, mrow0, ncol0, Ws, Lw);
    else wave_epilogue_f<COUT, MI, NJ, false, HO, WO>(acc, a, P, mrow0, ncol0, Ws, Lw);
}

template <int COUT, int MI, int NJ, int HO, int WO, bool FC = false>
__device__ __forceinline__ void wave_epilogue(const v16i (&acc)[MI][NJ], const ConvArgs& a, int mrow0,
                                              int ncol0, int8_t* Ws, const int8_t* Lw) {
    if (FC) {
        wave_epi_wide<COUT, MI, NJ, true>(acc, a, mrow0, ncol0);
        return;
    }
    if (a.out_i32) {
        wave_epi_wide<COUT, MI, NJ, false>(acc, a, mrow0, ncol0);
        return;
    }
    wave_epilogue_p<COUT, MI, NJ, HO, WO>(acc, a, load_epi_params<COUT, NJ>(a, ncol0), mrow0, ncol0, Ws, Lw);
}

// BN tables of channels [c0, c0 + NCH) -> LDS (pitch FF_LUT_PITCH) as
// direct-to-LDS loads, not waited for: wave load b fills LDS slots
// 64b .. 64b+63 of 16 bytes, slot s being piece s%17 of table s/17 (piece 16
// is the row padding and fetches the zero page).  The epilogue waits for them
// (vmcnt) and a barrier before it reads the tables.
template <int NW, int NCH>
__device__ __forceinline__ void issue_bn_lut(int8_t* Ls, const int8_t* lut, int c0) {
    constexpr int SPR = FF_LUT_PITCH / 16;
    constexpr int BLKS = NCH * SPR / 64;
    static_assert(FF_LUT_PITCH % 16 == 0 && (NCH * SPR) % 64 == 0, "whole wave loads");
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));           // (opaque, as in the residual loads)
    const int wave = tid >> 6;
    const int lane = tid & 63;
#pragma unroll
    for (int k = 0; k < (BLKS + NW - 1) / NW; k++) {
        const int blk = k * NW + wave;
        if (blk < BLKS) {                           // (uniform per wave)
            const int slot = blk * 64 + lane;
            const int c = slot / SPR;
            const int pc = slot - c * SPR;
            dma16(pc < 16 ? lut + (size_t)(c0 + c) * 256 + pc * 16 : ff_zero_page, Ls + blk * 1024);
        }
    }
}

// Workgroup index -> tile.  Workgroups are dispatched round-robin over the 8
// XCDs; give each XCD a contiguous run of tiles (N fastest) so the tiles that
// share an im2col row block sit in the same L2.
__device__ __forceinline__ int xcd_tile(int bid, int nb) {
    if ((nb & 7) == 0) return (bid & 7) * (nb >> 3) + (bid >> 3);
    return bid;
}

// ---------------------------------------------------------------------------
// Main conv kernel (Cin multiple of 64).
// ---------------------------------------------------------------------------
// KB: bytes of K per LDS stage (64 or 128: one or two 64-channel runs of one
// tap).  PF: stages of global loads kept in flight.  Each of the 4 waves
// computes MI x NJ MFMA tiles (MI*32 pixels x NJ*32 channels): bigger wave
// tiles read fewer LDS operand bytes per MFMA (MI+NJ reads per MI*NJ MFMAs).
// OCC: workgroups per CU the register/LDS budget is sized for.
// SPLIT > 1 (small batches): the K stages are cut into SPLIT ranges, one
// workgroup each; every workgroup stores its int32 partial tile and the last
// one to arrive at the tile (agent-scope counter) sums them and runs the
// epilogue.  Integer sums are exact, so the result does not depend on the
// order in which the partial tiles arrive.
template <int CIN, int COUT, int KS, int STRIDE, int HIN, int WIN, int BM, int BN, int KB, int PF,
          int MI, int NJ, int OCC, int SPLIT>
__global__ __launch_bounds__(256, OCC) void conv_i8_kernel(ConvArgs a) {
    constexpr int PAD = KS / 2;
    constexpr int HOUT = (HIN + 2 * PAD - KS) / STRIDE + 1;
    constexpr int WOUT = (WIN + 2 * PAD - KS) / STRIDE + 1;
    constexpr int HWO = HOUT * WOUT;
    constexpr int CSTEPS = CIN / KB;               // stages per tap
    constexpr int KALL = KS * KS * CSTEPS;         // stages of the whole reduction
    constexpr int KSTEPS = KALL / SPLIT;           // stages of this workgroup
    static_assert(KALL % SPLIT == 0, "split must divide the stages");
    constexpr int ROWB = KB + 16;                  // LDS row pitch (conflict-free b128 reads)
    constexpr int PPR = KB / 16;                   // 16-byte pieces per row and stage
    constexpr int A_LD = BM * PPR / 256;
    constexpr int B_LD = BN * PPR / 256;
    constexpr int WTM = MI * 32, WTN = NJ * 32;    // wave tile
    constexpr int WN = BN / WTN;                   // waves along N
    constexpr int LDS_K = 2 * (BM + BN) * ROWB;
    constexpr int LDS_E = 4 * wave_tile_bytes<MI, NJ>() + BN * FF_LUT_PITCH;
    constexpr int LDS = LDS_K > LDS_E ? LDS_K : LDS_E;
    static_assert(CIN % KB == 0 && KB % FF_KSTEP == 0, "Cin must be a multiple of the stage");
    static_assert((BM / WTM) * (BN / WTN) == 4, "4 waves");
    static_assert(COUT % BN == 0, "Cout must be a multiple of BN");

    __shared__ __align__(16) int8_t smem[LDS];
    int8_t* As = smem;
    int8_t* Bs = smem + 2 * BM * ROWB;

    const int tid = threadIdx.x;
    const int xbid = xcd_tile(blockIdx.x, gridDim.x);
    const int bid = xbid / SPLIT;                  // the splits of a tile are consecutive
    const int sp = xbid - bid * SPLIT;
    const int s_beg = sp * KSTEPS;
    const int tn = bid % a.tiles_n;
    const int tm = bid / a.tiles_n;
    const int m0 = tm * BM;

    // implicit-im2col row bookkeeping for this thread's A pieces
    const int8_t* a_img[A_LD];
    int a_ih0[A_LD], a_iw0[A_LD];
    bool a_ok[A_LD];
#pragma unroll
    for (int j = 0; j < A_LD; j++) {
        const int idx = tid + j * 256;
        const int m = m0 + idx / PPR;
        const bool ok = m < a.M;
        const int mm = ok ? m : 0;
        const int b = mm / HWO;
        const int r = mm - b * HWO;
        const int oh = r / WOUT;
        const int ow = r - oh * WOUT;
        a_img[j] = a.in + (size_t)b * (HIN * WIN * CIN) + (idx % PPR) * 16;
        a_ih0[j] = oh * STRIDE - PAD;
        a_iw0[j] = ow * STRIDE - PAD;
        a_ok[j] = ok;
    }
    // packed weights are [K/64][Cout][64]: piece p of a stage row n lies in
    // 64-byte K step (stage*KB/64 + p/4) at byte (p%4)*16
    int b_off[B_LD];
#pragma unroll
    for (int j = 0; j < B_LD; j++) {
        const int idx = tid + j * 256;
        const int n = idx / PPR, p = idx % PPR;
        b_off[j] = ((p / 4) * COUT + tn * BN + n) * FF_KSTEP + (p % 4) * 16;
    }

    // Prefetch queue: PF register sets, each holding one K step's global
    // loads, so PF steps of loads are in flight while the MFMAs of the
    // current step run out of LDS (memory latency is several times one
    // step's MFMA time).
    v4i ra[PF][A_LD], rb[PF][B_LD];
    auto gload = [&](int s, v4i (&qa)[A_LD], v4i (&qb)[B_LD]) {
        const int tap = s / CSTEPS;
        const int cs = s - tap * CSTEPS;
        const int kh = tap / KS;
        const int kw = tap - kh * KS;
#pragma unroll
        for (int j = 0; j < A_LD; j++) {
            const int ih = a_ih0[j] + kh;
            const int iw = a_iw0[j] + kw;
            const bool v = a_ok[j] && (unsigned)ih < (unsigned)HIN && (unsigned)iw < (unsigned)WIN;
            const int8_t* src = v ? a_img[j] + (ih * WIN + iw) * CIN + cs * KB : ff_zero_page;
            qa[j] = *reinterpret_cast<const v4i*>(src);
        }
        const int8_t* wst = a.w + (size_t)s * (KB / FF_KSTEP) * COUT * FF_KSTEP;
#pragma unroll
        for (int j = 0; j < B_LD; j++) qb[j] = *reinterpret_cast<const v4i*>(wst + b_off[j]);
    };
    auto sstore = [&](int buf, const v4i (&qa)[A_LD], const v4i (&qb)[B_LD]) {
#pragma unroll
        for (int j = 0; j < A_LD; j++) {
            const int idx = tid + j * 256;
            *reinterpret_cast<v4i*>(As + buf * BM * ROWB + (idx / PPR) * ROWB + (idx % PPR) * 16) = qa[j];
        }
#pragma unroll
        for (int j = 0; j < B_LD; j++) {
            const int idx = tid + j * 256;
            *reinterpret_cast<v4i*>(Bs + buf * BN * ROWB + (idx / PPR) * ROWB + (idx % PPR) * 16) = qb[j];
        }
    };

    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int wm = wave / WN;
    const int wn = wave % WN;
    const int8_t* a_rd = As + (wm * WTM + (lane & 31)) * ROWB + (lane >> 5) * 16;
    const int8_t* b_rd = Bs + (wn * WTN + (lane & 31)) * ROWB + (lane >> 5) * 16;

    v16i acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

    // prologue: steps 0 .. PF-1 in flight, step 0 staged in LDS
#pragma unroll
    for (int u = 0; u < PF; u++)
        if (u < KSTEPS) gload(s_beg + u, ra[u], rb[u]);
    sstore(0, ra[0], rb[0]);
    __syncthreads();
    // Step s lives in register set s % PF until it is staged into LDS buffer
    // s & 1; right after that the set is refilled with step s + PF.
    for (int s0 = 0; s0 < KSTEPS; s0 += PF) {
#pragma unroll
        for (int u = 0; u < PF; u++) {
            const int s = s0 + u;
            if (s < KSTEPS) {
                const int buf = s & 1;
                if (s + PF < KSTEPS) gload(s_beg + s + PF, ra[u], rb[u]);
#pragma unroll
                for (int ks = 0; ks < KB / 32; ks++) {
                    v4i af[MI], bf[NJ];
#pragma unroll
                    for (int i = 0; i < MI; i++)
                        af[i] = *reinterpret_cast<const v4i*>(a_rd + buf * BM * ROWB + i * 32 * ROWB + ks * 32);
#pragma unroll
                    for (int j = 0; j < NJ; j++)
                        bf[j] = *reinterpret_cast<const v4i*>(b_rd + buf * BN * ROWB + j * 32 * ROWB + ks * 32);
#pragma unroll
                    for (int i = 0; i < MI; i++)
#pragma unroll
                        for (int j = 0; j < NJ; j++)
                            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
                }
                if (s + 1 < KSTEPS) sstore(buf ^ 1, ra[(u + 1) % PF], rb[(u + 1) % PF]);
                __syncthreads();
            }
        }
    }

    if (SPLIT > 1) {
        // Partial tiles are exchanged with the documented agent-scope
        // release / acquire pattern, paid once per workgroup (the XCDs' L2s
        // are not coherent with each other): every thread stores its part
        // and waits for the stores; after the barrier one thread releases
        // (L2 write-back) and bumps the tile's arrival count; the workgroup
        // that arrives last acquires (L2 invalidate) and sums the partials.
        constexpr int NCH = MI * NJ * 4;            // 16-byte chunks per thread
        constexpr int PART = BM * BN * 4;           // bytes of one partial tile
        int8_t* part = reinterpret_cast<int8_t*>(a.ws + (size_t)bid * SPLIT * (BM * BN));
#pragma unroll
        for (int c = 0; c < NCH; c++) {             // chunk-major: a wave stores 1 KB runs
            const v16i& t = acc[c / (NJ * 4)][(c / 4) % NJ];
            const v4i v = {t[(c % 4) * 4], t[(c % 4) * 4 + 1], t[(c % 4) * 4 + 2], t[(c % 4) * 4 + 3]};
            *reinterpret_cast<v4i*>(part + sp * PART + (c * 256 + tid) * 16) = v;
        }
        __builtin_amdgcn_s_waitcnt(0);              // this wave's stores have reached L2
        __syncthreads();
        int* last = reinterpret_cast<int*>(smem);
        if (tid == 0) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            __builtin_amdgcn_s_waitcnt(0);          // write-back complete before the count moves
            const bool is_last = __hip_atomic_fetch_add(&a.counters[bid], 1u, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(SPLIT - 1);
            if (is_last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            __builtin_amdgcn_s_waitcnt(0);
            last[0] = is_last;
        }
        __syncthreads();
        if (!last[0]) return;                       // another workgroup finishes this tile
        // G partial tiles per round (NCH * G loads in flight) keep the
        // registers within the occupancy budget
        constexpr int G = SPLIT % 4 == 0 ? 4 : (SPLIT % 3 == 0 ? 3 : (SPLIT % 2 == 0 ? 2 : 1));
        v4i s[NCH];
#pragma unroll
        for (int c = 0; c < NCH; c++) s[c] = v4i{0, 0, 0, 0};
#pragma unroll 1
        for (int q0 = 0; q0 < SPLIT; q0 += G) {
            v4i t[NCH][G];
#pragma unroll
            for (int g = 0; g < G; g++)
#pragma unroll
                for (int c = 0; c < NCH; c++)
                    t[c][g] = *reinterpret_cast<const v4i*>(part + (q0 + g) * PART + (c * 256 + tid) * 16);
#pragma unroll
            for (int g = 0; g < G; g++)
#pragma unroll
                for (int c = 0; c < NCH; c++) s[c] += t[c][g];
        }
#pragma unroll
        for (int c = 0; c < NCH; c++) {
            v16i& t = acc[c / (NJ * 4)][(c / 4) % NJ];
#pragma unroll
            for (int e = 0; e < 4; e++) t[(c % 4) * 4 + e] = s[c][e];
        }
        if (tid == 0)                               // ready for the next launch
            __hip_atomic_store(&a.counters[bid], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
    }

    // epilogue (the loop's last barrier freed the K buffers)
    int8_t* Ws = smem + wave * wave_tile_bytes<MI, NJ>();
    int8_t* Ls = smem + 4 * wave_tile_bytes<MI, NJ>();
    if (a.flags & FFK_EPI_BN && !a.out_i32) issue_bn_lut<4, BN>(Ls, a.bn_lut, tn * BN);
    // the FC head runs this kernel as a 1x1 "conv" over a 1x1 image
    wave_epilogue<COUT, MI, NJ, HOUT, WOUT, HIN == 1 && WIN == 1>(acc, a, m0 + wm * WTM, tn * BN + wn * WTN, Ws,
                                Ls + (wn * WTN) * FF_LUT_PITCH);
}

// ---------------------------------------------------------------------------
// Conv kernel with direct-to-LDS operand loads (global_load_lds_dwordx4).
// ---------------------------------------------------------------------------
// WM x WN waves, each an MI x NJ block of 32x32 MFMA tiles: BM = WM*MI*32,
// BN = WN*NJ*32.  The K loop runs over 64-byte stages (one tap's 64-channel
// run).  Global loads go straight into an NST-deep LDS ring -- no register
// staging and no LDS store instructions, so the registers go to occupancy
// (WPE waves per SIMD) instead.  One wave load instruction writes 1 KB of LDS,
// lane L at byte 16*L.  A stage tile is a run of 256-byte lines of four
// 64-byte rows; the 16-byte slot of (row r, piece p) in line r/4 is
// ((r%4)*4 + p) XOR (r/4 % 4).  gfx950's LDS serves a ds_read_b128 in groups
// of 16 lanes over 64 banks (256 bytes), and the 16 rows such a group reads
// then land in 16 distinct slots: the operand reads are conflict-free.  The
// swizzle is realised by choosing which global piece each lane fetches: a
// line's 16 lanes still read four whole 64-byte rows.
// Per stage: wait for this thread's loads of the stage (vmcnt), barrier (every
// thread's loads landed; every wave is done with the stage the next loads
// overwrite), issue the loads of stage s+NST-1, then the MFMAs of stage s.
constexpr int DMA_KB = 64;

__device__ __forceinline__ int dma_slot(int r, int p) {
    const int line = r >> 2;
    return line * 256 + ((((r & 3) << 2) | p) ^ (line & 3)) * 16;
}

// Wait until at most N of this wave's global loads are in flight (and its LDS
// reads are done), then barrier.  Written as one asm block so that neither
// the compiler's waitcnt pass nor its scheduler moves LDS accesses across it.
template <int N>
__device__ __forceinline__ void dma_wait_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

template <int CIN, int COUT, int KS, int STRIDE, int HIN, int WIN, int WM, int WN, int MI, int NJ,
          int NST, int WPE>
__global__ __launch_bounds__(WM * WN * 64, WPE) void conv_dma_kernel(ConvArgs a) {
    constexpr int NW = WM * WN;
    constexpr int NT = NW * 64;
    constexpr int BM = WM * MI * 32, BN = WN * NJ * 32;
    constexpr int PAD = KS / 2;
    constexpr int HOUT = (HIN + 2 * PAD - KS) / STRIDE + 1;
    constexpr int WOUT = (WIN + 2 * PAD - KS) / STRIDE + 1;
    constexpr int HWO = HOUT * WOUT;
    constexpr int CSTEPS = CIN / DMA_KB;
    constexpr int KSTEPS = KS * KS * CSTEPS;
    constexpr int A_BYTES = BM * DMA_KB, B_BYTES = BN * DMA_KB;
    constexpr int STAGE = A_BYTES + B_BYTES;
    constexpr int A_LD = A_BYTES / (NT * 16), B_LD = B_BYTES / (NT * 16);
    constexpr int LPS = A_LD + B_LD;                        // loads per thread and stage
    constexpr int LDS_K = NST * STAGE;
    constexpr int LDS_E = NW * wave_tile_bytes<MI, NJ>() + BN * FF_LUT_PITCH;
    constexpr int LDS = LDS_K > LDS_E ? LDS_K : LDS_E;
    static_assert(CIN % DMA_KB == 0, "Cin must be a multiple of 64");
    static_assert(A_BYTES % (NT * 16) == 0 && B_BYTES % (NT * 16) == 0, "whole wave loads");
    static_assert(COUT % BN == 0, "Cout must be a multiple of BN");
    static_assert(NST >= 2 && (NST - 2) * LPS < 64, "ring depth");

    __shared__ __align__(1024) int8_t smem[LDS];
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int xbid = xcd_tile(blockIdx.x, gridDim.x);
    const int tn = xbid % a.tiles_n;
    const int tm = xbid / a.tiles_n;
    const int m0 = tm * BM;

    // This thread's pieces: wave load j of wave w fills lines (j*NW + w)*4 ..
    // +3 of the stage tile; lane L takes line +L/16, slot L%16.  Registers are
    // kept few (occupancy): a 32-bit image offset per piece, the piece's input
    // origin (a row past the tile's end gets an origin that fails every bounds
    // check), and its 16-byte slot in a 64-byte channel run.
    int a_off[A_LD], a_ih0[A_LD], a_iw0[A_LD], a_p[A_LD];
#pragma unroll
    for (int j = 0; j < A_LD; j++) {
        const int line = (j * NW + wave) * 4 + (lane >> 4);
        const int s = (lane & 15) ^ (line & 3);
        const int r = line * 4 + (s >> 2);
        const int p = s & 3;
        const int m = m0 + r;
        const bool ok = m < a.M;
        const int mm = ok ? m : 0;
        const int b = mm / HWO;
        const int rr = mm - b * HWO;
        const int oh = rr / WOUT;
        const int ow = rr - oh * WOUT;
        a_off[j] = b * (HIN * WIN * CIN) + p * 16;
        a_ih0[j] = ok ? oh * STRIDE - PAD : -4 * HIN;
        a_iw0[j] = ow * STRIDE - PAD;
        a_p[j] = p;
    }
    int b_off[B_LD];
#pragma unroll
    for (int j = 0; j < B_LD; j++) {
        const int line = (j * NW + wave) * 4 + (lane >> 4);
        const int s = (lane & 15) ^ (line & 3);
        const int n = line * 4 + (s >> 2);
        b_off[j] = (tn * BN + n) * FF_KSTEP + (s & 3) * 16;
    }
    auto issue = [&](int st, int buf) {
        const int tap = st / CSTEPS;
        const int cs = st - tap * CSTEPS;
        const int kh = tap / KS;
        const int kw = tap - kh * KS;
        int8_t* sb = smem + buf * STAGE;
#pragma unroll
        for (int j = 0; j < A_LD; j++) {
            const int ih = a_ih0[j] + kh;
            const int iw = a_iw0[j] + kw;
            const bool v = (unsigned)ih < (unsigned)HIN && (unsigned)iw < (unsigned)WIN;
            const int8_t* src = v ? a.in + (a_off[j] + (ih * WIN + iw) * CIN + cs * DMA_KB)
                                  : ff_zero_page + a_p[j] * 16;
            dma16(src, sb + (j * NW + wave) * 1024);
        }
        const int8_t* wst = a.w + (size_t)st * COUT * FF_KSTEP;
#pragma unroll
        for (int j = 0; j < B_LD; j++) dma16(wst + b_off[j], sb + A_BYTES + (j * NW + wave) * 1024);
    };

    const int wm = wave / WN;
    const int wn = wave % WN;
    // Fragment (i, ks) of this lane sits at a_rd + i*2048, XOR ks*32: 32 rows
    // are 8 lines (the swizzle key line%4 repeats), and the second 32-byte
    // k half flips bit 1 of the slot.
    const int a_rd = dma_slot(wm * MI * 32 + (lane & 31), lane >> 5);
    const int b_rd = A_BYTES + dma_slot(wn * NJ * 32 + (lane & 31), lane >> 5);

    v16i acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

#pragma unroll
    for (int u = 0; u < NST - 1; u++)
        if (u < KSTEPS) issue(u, u);
    int rbuf = 0;                          // ring slot of stage s
    for (int s = 0; s < KSTEPS; s++) {
        if (s + NST - 2 < KSTEPS) dma_wait_barrier<(NST - 2) * LPS>();
        else dma_wait_barrier<0>();
        if (s + NST - 1 < KSTEPS) issue(s + NST - 1, rbuf == 0 ? NST - 1 : rbuf - 1);
        const int8_t* sb = smem + rbuf * STAGE;
#if FF_DMA_IGLP
        __builtin_amdgcn_iglp_opt(1);
#endif
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            v4i af[MI], bf[NJ];
#pragma unroll
            for (int i = 0; i < MI; i++) af[i] = *reinterpret_cast<const v4i*>(sb + ((a_rd + i * 2048) ^ (ks * 32)));
#pragma unroll
            for (int j = 0; j < NJ; j++) bf[j] = *reinterpret_cast<const v4i*>(sb + ((b_rd + j * 2048) ^ (ks * 32)));
#pragma unroll
            for (int i = 0; i < MI; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        rbuf = rbuf == NST - 1 ? 0 : rbuf + 1;
    }
    __syncthreads();                       // every wave is done with the ring

    int8_t* Ws = smem + wave * wave_tile_bytes<MI, NJ>();
    int8_t* Ls = smem + NW * wave_tile_bytes<MI, NJ>();
    if (a.flags & FFK_EPI_BN && !a.out_i32) issue_bn_lut<NW, BN>(Ls, a.bn_lut, tn * BN);
    wave_epilogue<COUT, MI, NJ, HOUT, WOUT>(acc, a, m0 + wm * MI * 32, tn * BN + wn * NJ * 32, Ws,
                                Ls + (wn * NJ * 32) * FF_LUT_PITCH);
}

// ---------------------------------------------------------------------------
// 3x3 stride-1 conv with the input staged once per 64-channel run.
// ---------------------------------------------------------------------------
// A workgroup computes BM consecutive output pixels m0 .. m0+BM-1 (NHWC
// flattening over the whole batch) for BN channels.  With stride 1 the output
// and input pixel grids coincide, and tap (kh, kw) of output pixel m reads
// input pixel m + (kh-1)*W + (kw-1): for all nine taps these lie in one
// contiguous run, pixels m0-W-1 .. m0+BM+W, the tile's patch.  Each 64-channel
// run of the patch is loaded into LDS once (direct-to-LDS loads, double
// buffered: the next run loads during the nine taps of this one), instead of
// the 9 x BM rows a per-tap im2col tile would take, and tap (kh, kw) reads it
// at the fixed offset of kh*W + kw pixels.  A tap that falls into the zero
// padding (first / last row of an image, first / last pixel of a row) would
// read a neighbouring pixel of the run instead, so that lane's fragment address
// goes to a zero block.  Patch pixels are PATCH_PITCH = 80 bytes apart (64 data
// + 16 unused): the 16 consecutive pixels one 16-lane group of a ds_read_b128
// fetches then fall in 16 distinct bank slots (5 is odd), and every tap and
// K half is a constant offset.  The weights of each tap (BN x 64 bytes) go
// through a 3-stage ring with the conv_dma_kernel layout.
//
// Per step (one tap of one 64-channel run): wait for this step's weights (the
// in-order load counter also covers the patch, issued earlier), barrier,
// issue the weights of the step two ahead (and at tap 0 the next run's patch),
// then the MFMAs of the step.
constexpr int PATCH_PITCH = 80;

template <int CIN, int COUT, int H, int W, int WM, int WN, int MI, int NJ, int WPE>
__global__ __launch_bounds__(WM * WN * 64, WPE) void conv3_patch_kernel(ConvArgs a) {
    constexpr int NW = WM * WN;
    constexpr int NT = NW * 64;
    constexpr int BM = WM * MI * 32, BN = WN * NJ * 32;
    constexpr int CSTEPS = CIN / DMA_KB;                     // 64-channel runs
    constexpr int NP = BM + 2 * W + 2;                       // patch pixels
    constexpr int PSLOTS = NP * (PATCH_PITCH / 16);          // 16-byte slots of a patch
    constexpr int PLOADS = (PSLOTS + 63) / 64;               // 1 KB wave loads of a patch
    constexpr int LA = (PLOADS + NW - 1) / NW;               // patch loads per thread
    constexpr int PATCH_BYTES = PLOADS * 1024;
    constexpr int B_BYTES = BN * DMA_KB;
    // A step's weights are B_BYTES / 1 KB wave loads.  With fewer such loads
    // than waves (B_PART: 64 output channels over 8 waves) only waves
    // 0 .. BW-1 load weights, one each; the others load patches only.
    constexpr int BW = B_BYTES / 1024;
    constexpr bool B_PART = BW < NW;
    constexpr int B_LD = B_PART ? 1 : B_BYTES / (NT * 16);   // weight loads per loading thread and step
    constexpr int NSTB = 3;                                  // weight ring depth (9 % 3 == 0)
    constexpr int NPB = CSTEPS > 1 ? 2 : 1;                  // patch buffers (one run: no double buffer)
    constexpr int ZERO_OFF = NPB * PATCH_BYTES;              // 1 KB of zeros
    constexpr int RING_OFF = ZERO_OFF + 1024;
    constexpr int LDS_K = RING_OFF + NSTB * B_BYTES;
    constexpr int LDS_E = NW * wave_tile_bytes<MI, NJ>() + BN * FF_LUT_PITCH;
    constexpr int LDS = LDS_K > LDS_E ? LDS_K : LDS_E;
    static_assert(CIN % DMA_KB == 0, "Cin must be a multiple of 64");
    static_assert(B_BYTES % 1024 == 0 && (B_PART || B_BYTES % (NT * 16) == 0), "whole wave loads");
    static_assert(COUT % BN == 0, "Cout must be a multiple of BN");
    static_assert(B_LD + LA < 64, "load counter range");
    static_assert((2 * W + 2) * PATCH_PITCH + 32 + 16 < 65536, "tap offsets fit the ds_read offset field");

    __shared__ __align__(1024) int8_t smem[LDS];
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int xbid = xcd_tile(blockIdx.x, gridDim.x);
    const int tn = xbid % a.tiles_n;
    const int tm = xbid / a.tiles_n;
    const int m0 = tm * BM;
    const int first = m0 - W - 1;                            // input pixel of patch pixel 0

    // Zero block: masked taps read it.  Wave loads beyond the patch's PLOADS
    // (every thread issues LA, so that all waves count the same loads) fetch
    // the zero page into it as well.
    for (int i = tid; i < 64; i += NT) reinterpret_cast<v4i*>(smem + ZERO_OFF)[i] = v4i{0, 0, 0, 0};

    // Patch slots of this thread: wave load j of wave w is patch block j*NW + w,
    // lane L its slot L, i.e. patch pixel slot/5, piece slot%5 (piece 4 is the
    // unused 16 bytes).  Input offset of the slot at channel run 0, or -1 for
    // the zero page (unused piece, or a pixel outside the batch).
    int p_src[LA];
#pragma unroll
    for (int j = 0; j < LA; j++) {
        const int blk = j * NW + wave;
        const int slot = blk * 64 + lane;
        const int px = slot / 5;
        const int piece = slot - px * 5;
        const int g = first + px;
        const bool ok = blk < PLOADS && piece < 4 && g >= 0 && g < a.M;
        p_src[j] = ok ? g * CIN + piece * 16 : -1;
    }
    auto issue_patch = [&](int c, int buf) {
#pragma unroll
        for (int j = 0; j < LA; j++) {
            const int blk = j * NW + wave;
            const int8_t* src = p_src[j] >= 0 ? a.in + (p_src[j] + c * DMA_KB) : ff_zero_page;
            dma16(src, smem + (blk < PLOADS ? buf * PATCH_BYTES + blk * 1024 : ZERO_OFF));
        }
    };
    int b_off[B_LD];
#pragma unroll
    for (int j = 0; j < B_LD; j++) {
        const int line = (j * NW + wave) * 4 + (lane >> 4);
        const int sl = (lane & 15) ^ (line & 3);
        const int n = line * 4 + (sl >> 2);
        b_off[j] = (tn * BN + n) * FF_KSTEP + (sl & 3) * 16;
    }
    // step s = c*9 + t: tap t of channel run c, packed weight stage t*CSTEPS + c
    const bool loads_b = !B_PART || wave < BW;               // (uniform per wave)
    auto issue_b = [&](int c, int t, int slot) {
        if (!loads_b) return;
        const int8_t* wst = a.w + (size_t)(t * CSTEPS + c) * COUT * FF_KSTEP;
#pragma unroll
        for (int j = 0; j < B_LD; j++)
            dma16(wst + b_off[j], smem + RING_OFF + slot * B_BYTES + (j * NW + wave) * 1024);
    };

    const int wm = wave / WN;
    const int wn = wave % WN;
    // A fragment of row tile i: patch pixel (row + kh*W + kw) at PATCH_PITCH
    // bytes each, K piece lane/32 (+2 for the second 32-byte K half).  Edge
    // bits: 1 first row of its image, 2 last row, 4 first pixel of its row,
    // 8 last pixel.
    int a_base[MI], a_edge[MI];
#pragma unroll
    for (int i = 0; i < MI; i++) {
        const int r = wm * MI * 32 + i * 32 + (lane & 31);
        const int m = m0 + r;
        const int rr = m % (H * W);
        const int oh = rr / W;
        const int ow = rr - oh * W;
        a_edge[i] = (oh == 0 ? 1 : 0) | (oh == H - 1 ? 2 : 0) | (ow == 0 ? 4 : 0) | (ow == W - 1 ? 8 : 0);
        a_base[i] = r * PATCH_PITCH + (lane >> 5) * 16;
    }
    const int z_addr = ZERO_OFF + (lane >> 5) * 16;
    const int b_rd = RING_OFF + dma_slot(wn * NJ * 32 + (lane & 31), lane >> 5);

    v16i acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

    issue_patch(0, 0);
    issue_b(0, 0, 0);
    issue_b(0, 1, 1);
    for (int c = 0; c < CSTEPS; c++) {
        const bool more = c + 1 < CSTEPS;
        const int pb = (c & 1) * PATCH_BYTES;
        // (opaque per run: the nine taps' addresses are recomputed from these
        // instead of being kept live across the loop in 18 more registers)
#pragma unroll
        for (int i = 0; i < MI; i++) asm volatile("" : "+v"(a_base[i]), "+v"(a_edge[i]));
#pragma unroll
        for (int t = 0; t < 9; t++) {
            // loads issued after this step's weights: the next step's weights
            // and, at taps 1-2, the next run's patch (issued at tap 0)
            if (loads_b) {
                if (t == 1 || t == 2) {
                    if (more) dma_wait_barrier<B_LD + LA>();
                    else dma_wait_barrier<B_LD>();
                } else if (t == 8) {
                    if (more) dma_wait_barrier<B_LD>();
                    else dma_wait_barrier<0>();
                } else {
                    dma_wait_barrier<B_LD>();
                }
            } else {
                // patch loads only: the next run's (issued at tap 0) may still
                // be in flight at taps 1-2; from tap 3 on, like the weight
                // loaders' counts imply, nothing is
                if ((t == 1 || t == 2) && more) dma_wait_barrier<LA>();
                else dma_wait_barrier<0>();
            }
            if (t + 2 < 9) issue_b(c, t + 2, (t + 2) % NSTB);
            else if (more) issue_b(c + 1, t + 2 - 9, (t + 2) % NSTB);
            if (t == 0 && more) issue_patch(c + 1, (c + 1) & 1);

            const int kh = t / 3, kw = t % 3;
            const int emask = (kh == 0 ? 1 : 0) | (kh == 2 ? 2 : 0) | (kw == 0 ? 4 : 0) | (kw == 2 ? 8 : 0);
            const int toff = pb + (kh * W + kw) * PATCH_PITCH;
            int aa[MI];
#pragma unroll
            for (int i = 0; i < MI; i++) aa[i] = (a_edge[i] & emask) ? z_addr : a_base[i] + toff;
            const int br = b_rd + (t % NSTB) * B_BYTES;
            // scheduling hint: interleave the LDS reads with the MFMAs that
            // use them (measured 1-4% faster on every patch-kernel layer)
#if FF_PATCH_IGLP
            __builtin_amdgcn_iglp_opt(1);
#endif
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                v4i af[MI], bf[NJ];
#pragma unroll
                for (int i = 0; i < MI; i++) af[i] = *reinterpret_cast<const v4i*>(smem + aa[i] + ks * 32);
#pragma unroll
                for (int j = 0; j < NJ; j++) bf[j] = *reinterpret_cast<const v4i*>(smem + ((br + j * 2048) ^ (ks * 32)));
#pragma unroll
                for (int i = 0; i < MI; i++)
#pragma unroll
                    for (int j = 0; j < NJ; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
        }
    }
    __syncthreads();                       // every wave is done with the patch and the ring

    int8_t* Ws = smem + wave * wave_tile_bytes<MI, NJ>();
    int8_t* Ls = smem + NW * wave_tile_bytes<MI, NJ>();
    if (a.flags & FFK_EPI_BN && !a.out_i32) issue_bn_lut<NW, BN>(Ls, a.bn_lut, tn * BN);
    wave_epilogue<COUT, MI, NJ, H, W>(acc, a, m0 + wm * MI * 32, tn * BN + wn * NJ * 32, Ws,
                                Ls + (wn * NJ * 32) * FF_LUT_PITCH);
}

// ---------------------------------------------------------------------------
// Stem: 3 -> 64, 3x3, s1, p1 at 112x112, reading the fp32 faces.  One
// workgroup = two output rows of one face (224 pixels = 7 waves x 32 rows,
// all 64 channels).  The four input rows it needs are quantized once into
// LDS (quantize_fp32_nhwc_to_int8_per_channel fused into the conv,
// int8_epilogue.c:231-247); K = 27 is zero-padded to one 32-deep MFMA whose
// operands are gathered from that LDS patch.
// ---------------------------------------------------------------------------
constexpr int STEM_WAVES = 7;
constexpr int STEM_NT = STEM_WAVES * 64;

// Persistent: a workgroup loads the BN table and its weight fragments once and
// walks a contiguous run of tiles (neighbouring row pairs share input rows in
// cache); STEM_WG_PER_CU workgroups share a CU.
#ifndef FF_STEM_WG_PER_CU
#define FF_STEM_WG_PER_CU 2
#endif
constexpr int STEM_WG_PER_CU = FF_STEM_WG_PER_CU;

// Epilogue of a stem instantiation, chosen on the host (one variant per
// kernel keeps the register allocation to that variant's needs: with all of
// them in one kernel it spilled addresses to scratch and reloaded them in
// every tile's epilogue):
//   0-2  PReLU none / cmp-select / max form, X (and with BN) outputs
//   3-5  the same with the BN second output
//   6    FFK_EPI_INSCALE (FFW2/FFW3: flags dispatched inside)
//   7    raw int32 accumulators
//   8-13 0-5 with FFK_EPI_IN_RANGE
constexpr int STEM_EPI_INSC = 6, STEM_EPI_RAW = 7;

// (7 waves per workgroup over 4 SIMDs: STEM_WG_PER_CU * 7 / 4 waves per SIMD)
template <bool RGB8, int EPI>
__global__ __launch_bounds__(STEM_NT, (STEM_WG_PER_CU * STEM_WAVES + 3) / 4) void stem_kernel(ConvArgs a,
                                                                                        int tiles_per_wg) {
    constexpr int COUT = 64, H = 112, W = 112, HW = H * W;
    constexpr int PW = W + 2;                       // patch row: 114 pixels x 4 bytes
    constexpr int PATCH = 4 * PW * 4;
    __shared__ __align__(16) int8_t Ps[PATCH];
    __shared__ __align__(16) int8_t Es[STEM_WAVES * 32 * 80 + COUT * FF_LUT_PITCH];
    int8_t* Ls = Es + STEM_WAVES * 32 * 80;

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int ntiles = a.M / (2 * W);               // one tile = 2 output rows of one face
    const int t_beg = blockIdx.x * tiles_per_wg;
    const int t_end = t_beg + tiles_per_wg < ntiles ? t_beg + tiles_per_wg : ntiles;
    const void* x = a.in_f32 ? (const void*)a.in_f32 : (const void*)a.io->in;
    constexpr bool rgb8 = RGB8;
    const float inv0 = rgb8 ? 0.0f : a.in_inv[0];
    const float inv1 = rgb8 ? 0.0f : a.in_inv[1];
    const float inv2 = rgb8 ? 0.0f : a.in_inv[2];

    // tile-invariant: the BN table (direct-to-LDS loads, waited for at the
    // first tile and made visible by its barrier), the weight fragments, and
    // where this lane's A operand sits in the patch
    if (EPI != STEM_EPI_RAW && a.flags & FFK_EPI_BN) issue_bn_lut<STEM_WAVES, COUT>(Ls, a.bn_lut, 0);
    const int p = wave * 32 + (lane & 31);           // 0..223: pixel of the tile
    const int orow = p / W;
    const int ow = p - orow * W;
    const int g = lane >> 5;                         // K half
    // The MFMAs here take K in the order k' = 4*tap + c (c = 3 and taps past 8
    // carry zero weights): a tap's three channels and the patch's zero fourth
    // byte are then one aligned dword of the patch.  K' = 36 is zero-padded to
    // two 32-deep MFMAs.  Weight fragments in that order, built once from the
    // packed weights (k = 3*tap + c).
    auto bfrag = [&](int n, int kb) {
        v4i v;
#pragma unroll
        for (int w4 = 0; w4 < 4; w4++) {
            const int tap = kb / 4 + w4;
            uint32_t packed = 0;
            if (tap < 9)
#pragma unroll
                for (int c = 0; c < 3; c++) packed |= (uint32_t)(uint8_t)a.w[n * FF_KSTEP + tap * 3 + c] << (8 * c);
            v[w4] = (int)packed;
        }
        return v;
    };
    const v4i b0 = bfrag(lane & 31, g * 16), b1 = bfrag(32 + (lane & 31), g * 16);
    const v4i b0h = bfrag(lane & 31, 32 + g * 16), b1h = bfrag(32 + (lane & 31), 32 + g * 16);
    // this lane's four taps of the first MFMA (g*4 .. g*4+3) and tap 8 (second
    // MFMA; for g = 1 its weights are all zero, so the value read is unused)
    int a_off[5];
#pragma unroll
    for (int i = 0; i < 5; i++) {
        const int tap = i < 4 ? g * 4 + i : 8;
        a_off[i] = ((orow + tap / 3) * PW + ow + tap % 3) * 4;
    }
    // (raw int32 output: no parameter block is passed, a.params may be null)
    EpiParams<2> prm = {};
    if (EPI != STEM_EPI_RAW) prm = load_epi_params<COUT, 2>(a, 0);

    // The patch of tile t+1 is fetched into registers (PE elements per thread)
    // while tile t runs its MFMAs and epilogue: the loads' latency, not their
    // bytes, bounds this layer.
    constexpr int PE = (PATCH + STEM_NT - 1) / STEM_NT;
    float pv[RGB8 ? 1 : PE];                         // fp32 faces: the raw values
    int pq[RGB8 ? PE : 1];                           // uint8 pixels: the byte, or -1 for padding
    auto fetch = [&](int t) {
        const int b = t / (H / 2);
        const int oh0 = (t - b * (H / 2)) * 2;
#pragma unroll
        for (int j = 0; j < PE; j++) {
            const int e = tid + j * STEM_NT;
            const int pr = e / (PW * 4);
            const int rem = e - pr * (PW * 4);
            const int pc = rem >> 2;
            const int ci = rem & 3;
            const int ih = oh0 - 1 + pr;
            const int iw = pc - 1;
            const bool in = e < PATCH && ci < 3 && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;
            const size_t off = (size_t)b * HW * 3 + (ih * W + iw) * 3 + ci;
            if constexpr (RGB8) pq[j] = in ? (int)((const uint8_t*)x)[off] : -1;
            else pv[j] = in ? ((const float*)x)[off] : __builtin_nanf("");
        }
    };
    if (t_beg < t_end) fetch(t_beg);

    for (int t = t_beg; t < t_end; t++) {
        const int b = t / (H / 2);
        const int oh0 = (t - b * (H / 2)) * 2;
        const int m0 = b * HW + oh0 * W;
        __syncthreads();                             // the previous tile is done with Ps / Es

        // input rows oh0-1 .. oh0+2, columns -1 .. 112, channels 0..2 (+1 zero):
        // fp32 faces quantized in place, or uint8 pixels through the table;
        // padding and the fourth channel are zero
#pragma unroll
        for (int j = 0; j < PE; j++) {
            const int e = tid + j * STEM_NT;
            if (e < PATCH) {
                const int ci = e & 3;
                int8_t q = 0;
                if constexpr (RGB8) {
                    if (pq[j] >= 0) q = a.in_lut[ci * 256 + pq[j]];
                } else {
                    const int pr = e / (PW * 4);
                    const int pc = (e - pr * (PW * 4)) >> 2;
                    const int ih = oh0 - 1 + pr, iw = pc - 1;
                    if (ci < 3 && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W)
                        q = (int8_t)ff::quant_input(pv[j], ci == 0 ? inv0 : (ci == 1 ? inv1 : inv2));
                }
                Ps[e] = q;
            }
        }
        // the BN table's loads land before the first tile's barrier (nothing
        // else is in flight here: the next tile's fetch comes after)
        if (t == t_beg) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (t + 1 < t_end) fetch(t + 1);
        __syncthreads();

        // A operand: lane -> pixel (row of the MFMA tile) and K half g; one
        // dword of the patch per tap (the K' order above)
        const v4i av = {*reinterpret_cast<const int*>(Ps + a_off[0]), *reinterpret_cast<const int*>(Ps + a_off[1]),
                        *reinterpret_cast<const int*>(Ps + a_off[2]), *reinterpret_cast<const int*>(Ps + a_off[3])};
        const v4i ah = {*reinterpret_cast<const int*>(Ps + a_off[4]), 0, 0, 0};
        v16i acc[1][2];
#pragma unroll
        for (int r = 0; r < 16; r++) { acc[0][0][r] = 0; acc[0][1][r] = 0; }
        acc[0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b0, acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b1, acc[0][1], 0, 0, 0);
        acc[0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah, b0h, acc[0][0], 0, 0, 0);
        acc[0][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah, b1h, acc[0][1], 0, 0, 0);
        // the input layer has no residual input (ffk_conv rejects FFK_EPI_ADD here)
        int8_t* Ws = Es + wave * (32 * 80);
        const int mw = m0 + wave * 32;
        if constexpr (EPI == STEM_EPI_RAW) wave_epi_wide<COUT, 1, 2, false>(acc, a, mw, 0);
        else if constexpr (EPI == STEM_EPI_INSC) wave_epilogue_f<COUT, 1, 2, true, H, W>(acc, a, prm, mw, 0, Ws, Ls);
        else wave_epi_i8<COUT, 1, 2, (EPI & 7) % 3, false, ((EPI & 7) >= 3), false, (EPI >= 8), H, W>(
            acc, a, prm, mw, 0, Ws, Ls);
    }
}

// ---------------------------------------------------------------------------
// Dispatch table over the layer geometries of the IResNet family at 112x112
// (every IResNet-18/34/50/100 conv has one of these shapes).
// ---------------------------------------------------------------------------
namespace {

typedef void (*launch_fn)(const ConvArgs&, int grid, hipStream_t);

template <int CIN, int COUT, int KS, int STRIDE, int HIN, int WIN, int BM, int BN, int KB, int PF,
          int MI, int NJ, int OCC, int SPLIT>
void launch_conv(const ConvArgs& a, int grid, hipStream_t s) {
    hipLaunchKernelGGL((conv_i8_kernel<CIN, COUT, KS, STRIDE, HIN, WIN, BM, BN, KB, PF, MI, NJ, OCC, SPLIT>),
                       dim3(grid), dim3(256), 0, s, a);
}

template <int CIN, int COUT, int KS, int STRIDE, int HIN, int WIN, int WM, int WN, int MI, int NJ,
          int NST, int WPE>
void launch_conv_dma(const ConvArgs& a, int grid, hipStream_t s) {
    hipLaunchKernelGGL((conv_dma_kernel<CIN, COUT, KS, STRIDE, HIN, WIN, WM, WN, MI, NJ, NST, WPE>),
                       dim3(grid), dim3(WM * WN * 64), 0, s, a);
}

template <int CIN, int COUT, int H, int WM, int WN, int MI, int NJ, int WPE>
void launch_patch(const ConvArgs& a, int grid, hipStream_t s) {
    hipLaunchKernelGGL((conv3_patch_kernel<CIN, COUT, H, H, WM, WN, MI, NJ, WPE>), dim3(grid),
                       dim3(WM * WN * 64), 0, s, a);
}

typedef void (*stem_fn)(const ConvArgs&, int grid, int tiles_per_wg, hipStream_t);
template <bool RGB8, int EPI>
void launch_stem_as(const ConvArgs& a, int grid, int tiles_per_wg, hipStream_t s) {
    hipLaunchKernelGGL((stem_kernel<RGB8, EPI>), dim3(grid), dim3(STEM_NT), 0, s, a, tiles_per_wg);
}

void launch_stem(const ConvArgs& a, int grid, hipStream_t s) {
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
    stem_fn fn;
    const bool rgb8 = (a.flags & FFK_IN_RGB8) != 0;
    switch (epi) {
#define FF_STEM_CASE(E) case E: fn = rgb8 ? &launch_stem_as<true, E> : &launch_stem_as<false, E>; break;
    FF_STEM_CASE(0) FF_STEM_CASE(1) FF_STEM_CASE(2) FF_STEM_CASE(3) FF_STEM_CASE(4) FF_STEM_CASE(5)
    FF_STEM_CASE(8) FF_STEM_CASE(9) FF_STEM_CASE(10) FF_STEM_CASE(11) FF_STEM_CASE(12) FF_STEM_CASE(13)
    FF_STEM_CASE(STEM_EPI_INSC)
    default: fn = rgb8 ? &launch_stem_as<true, STEM_EPI_RAW> : &launch_stem_as<false, STEM_EPI_RAW>; break;
#undef FF_STEM_CASE
    }
    fn(a, wgs, per_wg, s);
}

// Small-batch split-K tiling: 64x64 workgroup tiles (one 32x32 MFMA tile per
// wave), the K stages of a tile shared by `split` workgroups.
constexpr int FF_SM_BM = 64, FF_SM_BN = 64;
// The split path is taken when the whole-K tiling leaves most CUs idle and the
// split grid stays small: every split workgroup pays one agent-scope L2
// write-back (~0.4 us, serialized per XCD), so a split grid much beyond ~20
// workgroups per XCD costs more than the shorter K chain saves.
constexpr int FF_SPLIT_MIN_WG = 256;
constexpr int FF_SPLIT_MAX_WG = 160;
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
};

// A grid of fewer big tiles than this leaves CUs idle; the 128x128 variant
// (four times the workgroups) is taken instead.
constexpr int FF_MID_MAX_WG = 512;

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
template <int CIN, int COUT, int KS, int S, int H, int SPLIT>
constexpr launch_fn split_launch() {
    if constexpr (SPLIT > 1)
        return &launch_conv<CIN, COUT, KS, S, H, H, FF_SM_BM, FF_SM_BN, FF_KB(CIN), 2, 1, 1, 4, SPLIT>;
    else
        return nullptr;
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
#define FF_P(CIN, COUT, H, SPLIT)                                                   \
    FF_PENTRY_K(CIN, COUT, H, SPLIT,                                                \
                (&launch_conv<CIN, COUT, 3, 1, H, H, 128, 128, FF_KB(CIN), FF_PF_MID(CIN), 2, 2, 2, 1>), \
                FF_TPATCH)
#define FF_PB(CIN, COUT, H, SPLIT)                                                  \
    FF_PENTRY_K(CIN, COUT, H, SPLIT,                                                \
                (&launch_conv<CIN, COUT, 3, 1, H, H, 128, 128, FF_KB(CIN), FF_PF_MID(CIN), 2, 2, 2, 1>), \
                FF_TPATCH_BIG)
#define FF_P64(CIN, COUT, H, SPLIT) FF_PENTRY_K(CIN, COUT, H, SPLIT, nullptr, FF_TPATCH64)
// (small grids: the 256x64 tiles, twice the workgroups)
#define FF_P64W(CIN, COUT, H, SPLIT)                                                \
    {CIN, COUT, 3, 1, H, H, 512, 64, &launch_patch<CIN, COUT, H, FF_TPATCH64W>, SPLIT, \
     split_launch<CIN, COUT, 3, 1, H, SPLIT>(), &launch_patch<CIN, COUT, H, FF_TPATCH64>, "patch", \
     256, 64, "patch"}
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
// partial tile costs an L2 write-back and those serialize per XCD, so fewer
// splits can win: 256->256 @14 (12 launches at b=1) with 3 instead of 9
// took the b=1 chain from 0.485 to 0.433 ms; 3 for the stride-2 and
// 512-channel layers measured the same as their 6 and 9, 2 (and 4) slower.
// One face gives 48-156 workgroups.  The 64-channel layers' 9 stages of 64
// bytes are too short to pay for the partial-sum exchange.
const ConvEntry kConvTable[] = {
    {3, 64, 3, 1, 112, 112, 224, 64, &launch_stem, 1, nullptr, nullptr, "stem"},
    FF_P64(64, 64, 112, 1),
    FF_C64(64, 64, 3, 2, 112, 1),
    FF_C64(64, 64, 1, 2, 112, 1),
    FF_P64W(64, 64, 56, 1),
    // 64 -> 128 at 56x56: one 64-channel run, so the patch kernel's single
    // input buffer fits two 256x128 workgroups per CU
    FF_P(64, 128, 56, 1),
    FF_C128(128, 128, 3, 2, 56, FF_S2_SPLIT),
    FF_C128(64, 128, 1, 2, 56, 1),
    FF_P(128, 128, 28, FF_S2_SPLIT),
    FF_P(128, 256, 28, FF_S2_SPLIT),
    FF_CBIG(256, 256, 3, 2, 28, FF_S3S2_SPLIT),
    FF_CBIG(128, 256, 1, 2, 28, 1),
    FF_PB(256, 256, 14, FF_S3_SPLIT),
    FF_PB(256, 512, 14, 3),
    FF_CBIG(512, 512, 3, 2, 14, FF_S4_SPLIT),
    FF_CBIG(256, 512, 1, 2, 14, 1),
    FF_PB(512, 512, 7, FF_S4_SPLIT),
    // the 1x1 shortcuts over a block input stored at its even pixels only
    // (FFK_OUT_X_EVEN): stride 1 over the compact tensor
    FF_C64(64, 64, 1, 1, 56, 1),
    FF_C128(64, 128, 1, 1, 28, 1),
    FF_CBIG(128, 256, 1, 1, 14, 1),
    FF_CBIG(256, 512, 1, 1, 7, 1),
};

const ConvEntry* find_conv(int cin, int cout, int kh, int kw, int stride, int pad, int hin, int win) {
    if (kh != kw || pad != kh / 2) return nullptr;
    for (const ConvEntry& e : kConvTable)
        if (e.cin == cin && e.cout == cout && e.ks == kh && e.stride == stride && e.hin == hin &&
            e.win == win)
            return &e;
    return nullptr;
}

// Launch choice for one layer at M output pixels.
struct ConvLaunch {
    launch_fn fn;
    const char* kind;
    int bn;             // workgroup tile width (tiles_n = cout / bn)
    int grid;
    int split;
    size_t counter_bytes, ws_bytes;   // split > 1: workspace layout
};

// ws_avail: workspace bytes the caller provides (a split > 1 variant that
// needs more falls back to the whole-K tiling).
ConvLaunch choose_launch(const ConvEntry* e, long long M, size_t ws_avail) {
    long long big = ((M + e->bm - 1) / e->bm) * (e->cout / e->bn);
    ConvLaunch l = {e->fn, e->kind, e->bn, (int)big, 1, 0, 0};
    if (e->mid && big < FF_MID_MAX_WG) {
        const int mbm = e->mid_bm ? e->mid_bm : 128, mbn = e->mid_bn ? e->mid_bn : 128;
        big = ((M + mbm - 1) / mbm) * (e->cout / mbn);
        l = {e->mid, e->mid_kind ? e->mid_kind : "staged128", mbn, (int)big, 1, 0, 0};
    }
    if (!e->small || big >= FF_SPLIT_MIN_WG) return l;
    const long long tiles = ((M + FF_SM_BM - 1) / FF_SM_BM) * (e->cout / FF_SM_BN);
    const long long wgs = tiles * e->split;
    if (wgs > FF_SPLIT_MAX_WG || wgs <= big) return l;
    if (e->split > 1) {
        // the counter area has the same size at every batch (tiles <= wgs), so
        // launches of different sizes never see each other's partial tiles
        // in their counters
        const size_t cnt = FF_SPLIT_COUNTER_BYTES;
        const size_t need = cnt + (size_t)wgs * FF_SM_BM * FF_SM_BN * sizeof(int32_t);
        if (need > ws_avail) return l;
        l.counter_bytes = cnt;
        l.ws_bytes = need;
    }
    l.fn = e->small;
    l.kind = "splitk";
    l.bn = FF_SM_BN;
    l.grid = (int)wgs;
    l.split = e->split;
    return l;
}

long long conv_pixels(const ffk_conv_desc* d) {
    const int hout = (d->hin + 2 * d->pad - d->kh) / d->stride + 1;
    const int wout = (d->win + 2 * d->pad - d->kw) / d->stride + 1;
    return (long long)d->batch * hout * wout;
}

}  // namespace

constexpr int FC_SPLIT = 7;
size_t ffk_fc_split_ws_bytes(int batch);

// FC head through the same kernel (a 1x1 "conv" over a 1x1 image with
// Cin = K): M = batch faces, N = 512, K = 25088.
int ffk_fc_gemm_launch(const ffk_fc_desc* d, hipStream_t s) {
    if (d->n != 512 || d->k != 25088) {
        ffk_set_error("fc gemm: unsupported shape (n must be 512, k 25088)%s%s", nullptr, nullptr);
        return FFK_ERR_UNSUPPORTED;
    }
    ConvArgs a = {};
    a.in = d->a;
    a.w = d->w;
    a.fc_ws = d->ws;
    a.fc_bias = d->bias;
    a.io = d->io;
    a.out_f32 = d->out;
    a.M = d->batch;
    a.flags = 0;
    a.in_scale = d->a_scale;
    a.tiles_n = 512 / 128;
    const int tiles = ((d->batch + 127) / 128) * a.tiles_n;
    const size_t need = ffk_fc_split_ws_bytes(d->batch);
    if (need && d->workspace && d->workspace_bytes >= need) {
        // split-K: FC_SPLIT workgroups per 128x128 output tile (the last to
        // arrive sums the int32 partial tiles and writes the fp32 outputs)
        a.counters = (unsigned*)d->workspace;
        a.ws = (int32_t*)((int8_t*)d->workspace + FF_SPLIT_COUNTER_BYTES);
        hipLaunchKernelGGL((conv_i8_kernel<25088, 512, 1, 1, 1, 1, 128, 128, 128, FF_PF128, 2, 2, 2, FC_SPLIT>),
                           dim3(tiles * FC_SPLIT), dim3(256), 0, s, a);
        return ffk_check_launch("fc gemm launch");
    }
    hipLaunchKernelGGL((conv_i8_kernel<25088, 512, 1, 1, 1, 1, 128, 128, 128, FF_PF128, 2, 2, 2, 1>),
                       dim3(tiles), dim3(256), 0, s, a);
    return ffk_check_launch("fc gemm launch");
}

// FC GEMM split-K: K = 25088 is 196 stages of 128 bytes; 7 ranges of 28.  A
// batch whose tiles fit the counter area and leave the GPU under-filled with
// one workgroup per tile (fewer than two per CU) splits.
size_t ffk_fc_split_ws_bytes(int batch) {
    const long long tiles = ((long long)(batch + 127) / 128) * (512 / 128);
    if (batch <= 0 || tiles > FF_SPLIT_MAX_WG || tiles >= 512) return 0;
    return FF_SPLIT_COUNTER_BYTES + (size_t)tiles * FC_SPLIT * 128 * 128 * sizeof(int32_t);
}

extern "C" {

int ffk_conv_supported(int cin, int cout, int kh, int kw, int stride, int pad, int hin, int win) {
    return find_conv(cin, cout, kh, kw, stride, pad, hin, win) != nullptr;
}

int ffk_prelu_le1_ok(const float* params, int cout, int ktotal, int with_add) {
    if (!params || cout <= 0 || ktotal <= 0) return 0;
    const double acc_max = (double)ktotal * 128.0 * 128.0;
    for (int c = 0; c < cout; c++) {
        const double s = params[FFK_P_SLOPE * cout + c];
        const double ws = params[FFK_P_WS * cout + c];
        const double bias = params[FFK_P_BIAS * cout + c];
        const double adds = with_add ? params[FFK_P_ADDSCALE * cout + c] : 0.0;
        if (!(s <= 1.0) || !std::isfinite(ws) || !std::isfinite(bias) || !std::isfinite(adds)) return 0;
        // each fp32 rounding is within a factor 1 + 2^-23 of its exact value
        const double bound = (acc_max * std::fabs(ws) + std::fabs(bias) + 128.0 * std::fabs(adds)) * 1.0001;
        if (!(bound < 3.0e38)) return 0;
    }
    return 1;
}

int ffk_requant_in_range(const float* params, int cout, int ktotal, int flags) {
    if (!params || cout <= 0 || ktotal <= 0 || (flags & FFK_EPI_INSCALE)) return 0;
    const double acc_max = (double)ktotal * 128.0 * 128.0;
    // each fp32 rounding is within a factor 1 + 2^-24 of its exact value;
    // five of them (conversion, ws, bias, residual, PReLU) before the inv one
    const double widen = 1.000001;
    for (int c = 0; c < cout; c++) {
        const double ws = params[FFK_P_WS * cout + c];
        const double bias = params[FFK_P_BIAS * cout + c];
        const double inv = params[FFK_P_INV * cout + c];
        const double adds = (flags & FFK_EPI_ADD) ? params[FFK_P_ADDSCALE * cout + c] : 0.0;
        const double slope = (flags & FFK_EPI_PRELU) ? params[FFK_P_SLOPE * cout + c] : 0.0;
        if (!std::isfinite(ws) || !std::isfinite(bias) || !std::isfinite(inv) || !std::isfinite(adds) ||
            !std::isfinite(slope))
            return 0;
        const double f = (acc_max * std::fabs(ws) + std::fabs(bias) + 128.0 * std::fabs(adds)) * widen;
        const double t = f * std::max(1.0, std::fabs(slope)) * std::fabs(inv) * widen;
        if (!(t < 2147483520.0)) return 0;              // 2^31 - 128
    }
    return 1;
}

size_t ffk_conv_packed_bytes(int cin, int cout, int kh, int kw) {
    const size_t ktot = (size_t)kh * kw * cin;
    const size_t steps = (ktot + FF_KSTEP - 1) / FF_KSTEP;
    return steps * (size_t)cout * FF_KSTEP;
}

int ffk_pack_conv_weights(const int8_t* w, int cout, int cin, int kh, int kw, int8_t* packed) {
    if (!w || !packed || cout <= 0 || cin <= 0 || kh <= 0 || kw <= 0) {
        ffk_set_error("pack_conv_weights: bad arguments%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    const int ktot = kh * kw * cin;
    const int steps = (ktot + FF_KSTEP - 1) / FF_KSTEP;
    for (int s = 0; s < steps; s++)
        for (int n = 0; n < cout; n++)
            for (int kk = 0; kk < FF_KSTEP; kk++) {
                const int k = s * FF_KSTEP + kk;
                int8_t v = 0;
                if (k < ktot) {
                    const int tap = k / cin, ci = k - tap * cin;
                    const int y = tap / kw, x = tap - y * kw;
                    v = w[(((size_t)n * cin + ci) * kh + y) * kw + x];
                }
                packed[((size_t)s * cout + n) * FF_KSTEP + kk] = v;
            }
    return FFK_OK;
}

int ffk_conv(const ffk_conv_desc* d, void* stream) {
    if (!d || d->batch < 0) {
        ffk_set_error("conv: bad descriptor%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    const ConvEntry* e = find_conv(d->cin, d->cout, d->kh, d->kw, d->stride, d->pad, d->hin, d->win);
    if (!e) {
        ffk_set_error("conv: no kernel for this layer geometry%s%s", nullptr, nullptr);
        return FFK_ERR_UNSUPPORTED;
    }
    const long long M = conv_pixels(d);
    if (M > 0x7fffffffLL) {
        ffk_set_error("conv: batch too large%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    const bool stem = d->cin == 3;
    const bool raw = d->out_i32 != nullptr;
    const bool rgb8 = stem && (d->flags & FFK_IN_RGB8);
    if (stem && (d->flags & FFK_EPI_ADD)) {
        ffk_set_error("conv: the 3-channel input layer takes no residual input%s%s", nullptr, nullptr);
        return FFK_ERR_UNSUPPORTED;
    }
    if ((d->flags & FFK_IN_RGB8) && !stem) {
        ffk_set_error("conv: FFK_IN_RGB8 applies to the 3-channel input layer only%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    bool bad = !d->w || (!raw && !d->params) || (stem && !rgb8 && !d->in_inv) || (rgb8 && !d->in_lut) ||
               (stem && !d->in && !d->io) ||
               (!stem && !d->in);
    if (!raw) {
        if ((d->flags & FFK_EPI_ADD) && !d->add_src) bad = true;
        if ((d->flags & FFK_EPI_BN) && (!d->out_bn || !d->bn_lut)) bad = true;
        if (!(d->flags & FFK_EPI_BN) && !d->out) bad = true;
    }
    if (bad) {
        ffk_set_error("conv: missing pointer for the requested flags%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    const bool x_even = (d->flags & FFK_OUT_X_EVEN) != 0;
    if (x_even) {
        const int hout = (d->hin + 2 * d->pad - d->kh) / d->stride + 1;
        const int wout = (d->win + 2 * d->pad - d->kw) / d->stride + 1;
        if (raw || !d->out || (hout & 1) || (wout & 1)) {
            ffk_set_error("conv: FFK_OUT_X_EVEN needs an int8 output X of even height and width%s%s",
                          nullptr, nullptr);
            return FFK_ERR_ARG;
        }
    }
    if (M == 0) return FFK_OK;
    if (d->flags & FFK_ALGO_WINOGRAD) return ffk_winograd_conv(d, (hipStream_t)stream);
    ConvArgs a = {};
    if (stem) a.in_f32 = (const float*)d->in;
    else a.in = (const int8_t*)d->in;
    a.in_inv = d->in_inv;
    a.in_lut = d->in_lut;
    a.io = d->io;
    a.w = d->w;
    a.params = d->params;
    a.add_src = d->add_src;
    a.bn_lut = d->bn_lut;
    a.out = d->out;
    a.out_bn = d->out_bn;
    a.out_i32 = d->out_i32;
    a.flags = d->flags & (FFK_EPI_PRELU | FFK_EPI_ADD | FFK_EPI_BN | FFK_EPI_BIAS | FFK_EPI_INSCALE |
                          FFK_EPI_PRELU_LE1 | FFK_OUT_X_EVEN | FFK_EPI_IN_RANGE |
                          FFK_IN_RGB8);
    a.in_scale = d->in_scale;
    // The direct-to-LDS kernels address the int8 input with 32-bit offsets:
    // a batch whose input tensor reaches 2 GiB runs as several launches over
    // consecutive image ranges (images are independent).
    const long long px_out = M / d->batch;
    const long long in_img = (long long)d->hin * d->win * d->cin;
    const int slice = stem ? d->batch : (int)std::min<long long>(d->batch, 0x7fffffffLL / in_img);
    for (int b0 = 0; b0 < d->batch; b0 += slice) {
        const int nb = std::min(slice, d->batch - b0);
        const long long ms = (long long)nb * px_out;
        ConvArgs as = a;
        if (!stem) as.in = a.in + (size_t)b0 * in_img;
        const size_t o = (size_t)b0 * px_out * d->cout;
        if (a.add_src) as.add_src = a.add_src + o;
        if (a.out) as.out = a.out + (x_even ? o / 4 : o);     // even/even pixels: a quarter
        if (a.out_bn) as.out_bn = a.out_bn + o;
        if (a.out_i32) as.out_i32 = a.out_i32 + o;
        as.M = (int)ms;
        const ConvLaunch l = choose_launch(e, ms, d->workspace ? d->workspace_bytes : 0);
        if (l.split > 1) {
            as.counters = (unsigned*)d->workspace;
            as.ws = (int32_t*)((int8_t*)d->workspace + l.counter_bytes);
        }
        as.tiles_n = d->cout / l.bn;
        l.fn(as, l.grid, (hipStream_t)stream);
        const int rc = ffk_check_launch("conv launch");
        if (rc != FFK_OK) return rc;
    }
    return FFK_OK;
}

// ---------------------------------------------------------------------------
// No-allocation variant of ffk_conv: the split-K workspace is a file-scope
// device array (each GPU holds its own copy, at its own address, for the life
// of the process) instead of caller memory.  Its size covers the largest
// split grid (FF_SPLIT_MAX_WG workgroups of 64x64 int32 partial tiles) behind
// the counter area.  In host code `scratch` names a host-side stand-in, not
// device memory: its device address comes from hipGetSymbolAddress, once per
// device, and only that address is passed on.
// ---------------------------------------------------------------------------
static_assert(FFK_NOALLOC_SCRATCH_BYTES == FF_WS_COUNTER_AREA + (size_t)FF_SPLIT_MAX_WG * FF_SM_BM * FF_SM_BN * 4,
              "the header's limit is the split-K workspace bound");
static __device__ __align__(256) int8_t scratch[FFK_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int FF_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_addr[FF_MAX_DEVICES];

// Device address of the current device's `scratch`.  First use on a device:
// look it up and clear the counter area with a fill kernel on `stream` (the
// array is zero when the code object loads; the clear does not rely on it).
int scratch_for_current_device(hipStream_t stream, void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return ffk_hip_fail(e, "hipGetDevice");
    if (dev < 0 || dev >= FF_MAX_DEVICES) {
        ffk_set_error("conv_noalloc: device index out of range%s%s", nullptr, nullptr);
        return FFK_ERR_UNSUPPORTED;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return ffk_hip_fail(e, "hipGetSymbolAddress(scratch)");
        const int rc = ffk_zero(p, FF_WS_COUNTER_AREA, stream);
        if (rc != FFK_OK) return rc;
        g_scratch_addr[dev] = p;
    }
    *out = g_scratch_addr[dev];
    return FFK_OK;
}
}  // namespace

int ffk_conv_noalloc(const ffk_conv_desc* d, void* stream) {
    if (!d) {
        ffk_set_error("conv_noalloc: bad descriptor%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    ffk_conv_desc dd = *d;
    dd.workspace = nullptr;
    dd.workspace_bytes = 0;
    const size_t need = ffk_conv_workspace_bytes(&dd);
    if (need > FFK_NOALLOC_SCRATCH_BYTES) {
        ffk_set_error("conv_noalloc: this layer needs a %s-byte workspace, above the %s-byte device scratch "
                      "(use ffk_conv with a workspace)",
                      std::to_string(need).c_str(), std::to_string(FFK_NOALLOC_SCRATCH_BYTES).c_str());
        return FFK_ERR_ARG;
    }
    void* p = nullptr;
    const int rc = scratch_for_current_device((hipStream_t)stream, &p);
    if (rc != FFK_OK) return rc;
    dd.workspace = p;
    dd.workspace_bytes = FFK_NOALLOC_SCRATCH_BYTES;
    return ffk_conv(&dd, stream);
}

size_t ffk_conv_workspace_bytes(const ffk_conv_desc* d) {
    if (!d || d->batch <= 0) return 0;
    const ConvEntry* e = find_conv(d->cin, d->cout, d->kh, d->kw, d->stride, d->pad, d->hin, d->win);
    if (!e) return 0;
    if (d->flags & FFK_ALGO_WINOGRAD) return ffk_winograd_ws_bytes(d);
    const long long M = conv_pixels(d);
    if (M > 0x7fffffffLL) return 0;
    return choose_launch(e, M, (size_t)-1).ws_bytes;
}

const char* ffk_conv_variant(const ffk_conv_desc* d) {
    if (!d || d->batch <= 0) return nullptr;
    const ConvEntry* e = find_conv(d->cin, d->cout, d->kh, d->kw, d->stride, d->pad, d->hin, d->win);
    if (!e) return nullptr;
    if (d->flags & FFK_ALGO_WINOGRAD) return ffk_winograd_eligible(d) ? "winograd" : nullptr;
    const long long M = conv_pixels(d);
    if (M > 0x7fffffffLL) return nullptr;
    return choose_launch(e, M, d->workspace ? d->workspace_bytes : 0).kind;
}

// BN second output as a table: lut[c][q + 128] = BN-requant of the int8
// value q for channel c, computed with the reference's fp32 sequence
// (bn_prelu_requant_int8 with bn != NULL, int8_epilogue.c:273-303):
//   f = fma(RN(q * s_in), bn_s, bn_o); round half away of RN(f * inv);
//   x86 cvttps2dq semantics; clamp to int8.
int ffk_make_bn_lut(const float* s_in, const float* bn_s, const float* bn_o, const float* bn_inv,
                    int cout, int8_t* lut) {
    if (!s_in || !bn_s || !bn_o || !bn_inv || !lut || cout <= 0) {
        ffk_set_error("make_bn_lut: bad arguments%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    for (int c = 0; c < cout; c++)
        for (int q = -128; q < 128; q++) {
            volatile float f = (float)q * s_in[c];
            f = __builtin_fmaf(f, bn_s[c], bn_o[c]);
            volatile float t = f * bn_inv[c];
            volatile float r = t + __builtin_copysignf(0.5f, t);
            int32_t v;
            if (r >= -2147483648.0f && r < 2147483648.0f) v = (int32_t)r;
            else v = INT32_MIN;
            v = v < -128 ? -128 : (v > 127 ? 127 : v);
            lut[(size_t)c * 256 + (q + 128)] = (int8_t)v;
        }
    return FFK_OK;
}

int ffk_make_rgb8_lut(const float* in_inv, int8_t* lut) {
    if (!in_inv || !lut) {
        ffk_set_error("make_rgb8_lut: bad arguments%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    for (int c = 0; c < 3; c++)
        for (int x = 0; x < 256; x++) {
            volatile float v = (float)x - 127.5f;      // exact
            v = v / 127.5f;                            // one correctly rounded division
            volatile float t = v * in_inv[c];
            long q = lrintf(t);                        // the reference's glibc call
            int32_t qi = (int32_t)q;
            qi = qi < -128 ? -128 : (qi > 127 ? 127 : qi);
            lut[c * 256 + x] = (int8_t)qi;
        }
    return FFK_OK;
}

}  // extern "C"
