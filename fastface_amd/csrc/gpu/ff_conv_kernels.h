// ff_conv_kernels.h -- NHWC int8 convolution kernels as implicit GEMM on gfx950 i8 MFMA
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
#pragma once
#include <algorithm>
#include <cmath>
#include <type_traits>

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
static __device__ __align__(64) int8_t ff_zero_page[64];

// Direct-to-LDS load of 16 bytes per lane: lane L of the wave writes
// lds_wave_base + 16 L (1 KB per wave load); counted by vmcnt.
__device__ __forceinline__ void dma16(const int8_t* g, int8_t* lds_wave_base) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds_wave_base, 16, 0, 0);
}

// The same through a buffer resource: byte voff (per lane) + soff (uniform)
// of the buffer.  A lane whose voff is at or past the buffer's size
// (FF_OOB) is out of range: the hardware returns zeros and reads no memory.
// Padding taps and rows past the batch use that instead of a zero page, so
// the per-lane address is one 32-bit offset (no 64-bit pointer select), and
// the uniform part stays in a scalar register.
constexpr unsigned FF_OOB = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t ff_rsrc(const void* base, unsigned bytes) {
    // raw (stride 0) buffer, 32-bit data format: the range check is offset < bytes
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ void bdma16(__amdgpu_buffer_rsrc_t r, unsigned voff, unsigned soff, int8_t* lds_wave_base) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_wave_base, 16, voff, soff, 0,
                                             0);
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
    int tiles_n;            // column tiles of the grid (cout / tile width); the
                            // kernels use their compile-time COUT / BN, the same value
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

// Pixel index of output pixel m's X row in the launch's X tensor: m, or
// with FFK_OUT_X_EVEN (HO x WO images, both even) its index in the
// [HO/2][WO/2] tensor of the even-row, even-column pixels, and FF_OOB for
// every other pixel.  Row r (0..31) of the 32-row block starting at pixel mb
// (uniform per wave); an image holding a whole number of 32-row blocks finds
// the block's image once (scalar work).  Pixels past the batch give indices
// past the tensor (a.M, or a.M / 4 even pixels).
template <int HO, int WO>
__device__ __forceinline__ unsigned x_pix_blk(const ConvArgs& a, int mb, int r) {
    if constexpr (HO % 2 == 0 && WO % 2 == 0) {
        if (a.flags & FFK_OUT_X_EVEN) {
            int img, rem;
            if constexpr ((HO * WO) % 32 == 0) {
                img = mb / (HO * WO);
                rem = mb - img * (HO * WO) + r;
            } else {
                img = (mb + r) / (HO * WO);
                rem = mb + r - img * (HO * WO);
            }
            const int oh = rem / WO, ow = rem - oh * WO;
            if ((oh | ow) & 1) return FF_OOB;
            return (unsigned)((img * (HO / 2) + (oh >> 1)) * (WO / 2) + (ow >> 1));
        }
    }
    return (unsigned)(mb + r);
}

// PRELU: 0 none, 1 f < 0 ? f*slope : f, 2 max(f, f*slope) (the same values
// when every slope is at most 1 and f is never infinite: FFK_EPI_PRELU_LE1).
// INSC: f = f * in_scale first (FFW2/FFW3 models; FFW4 skips the multiply).
// RANGE: 0 the general requant; 1 every requant value is known in range
// (FFK_EPI_IN_RANGE); 2 also its last two roundings taken as one fma
// (FFK_EPI_FMA_TAIL, proven per launch by the host; no residual).
// HO x WO: output image size (FFK_OUT_X_EVEN addressing).
// LUT_DMA: the BN table was issued as direct-to-LDS loads (issue_bn_lut) that
// may still be in flight; they are waited for before the flush.
// WG_SYNC: a workgroup barrier before the flush, which makes a BN table other
// waves loaded visible; without it (a table already visible, as in the
// persistent stem after its first tile) the flush reads only the wave's own
// staging tile, which the wave's in-order LDS accesses already order.
// STAGE (a conv fused with the 1x1 shortcut that adds its output): 1 leaves
// the int8 results in the wave's staging tile and stores nothing (the
// residual of the shortcut's epilogue); 2 (with ADD) takes the residual from
// the staging tile, where STAGE 1 left it, instead of loading it.  The same
// lane writes and reads each element, so no barrier orders the two.
// BN_PASS: the BN table lookups run as a pass of their own in which all
// lanes of a lookup instruction read the tables of one 16-channel chunk
// (lane -> tile row; with 32-row tiles two chunks, one per half-wave), so
// the reads of one table never meet another table's in a bank; the results
// go back into the staging tile and leave as coalesced 16-byte stores.
// Costs two more 16-byte LDS accesses per chunk: it pays only where the
// conflicts dominate the flush (the stem, measured 4 % faster; the
// 256-channel layers were up to 3 % slower).
// XOFF: the caller gives the X byte offset of each flush chunk k (tile row
// lane/CH + k*RPI, channels ncol0 + 16*(lane%CH); xoff[k], FF_OOB-based for
// chunks not stored), instead of the pixel arithmetic of
// x_pix_blk: a persistent kernel whose chunk offsets are a per-lane constant
// plus a per-tile step (the stem) computes them with one add.
template <int COUT, int MI, int NJ, int PRELU, bool ADD, bool BN2, bool INSC, int RANGE, int HO, int WO,
          bool LUT_DMA = false, bool WG_SYNC = true, int STAGE = 0, bool BN_PASS = false, bool XOFF = false>
__device__ __forceinline__ void wave_epi_i8(const v16i (&acc)[MI][NJ], const ConvArgs& a,
                                            const EpiParams<NJ>& prm, int mrow0, int ncol0, int8_t* Ws,
                                            const int8_t* Lw, const unsigned* xoff = nullptr) {
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
    static_assert(STAGE != 1 || !ADD, "a staged tile is an output, not a residual sum");
    static_assert(RANGE != 2 || (!ADD && !INSC), "the one-rounding tail is proven without a residual");
    if (ADD && STAGE != 2 && RSLOTS % 64 == 0) {
        // residual tile -> this wave's LDS tile as direct-to-LDS loads: slot s
        // of wave load k is tile row (64k+s)/SPR, piece (64k+s)%SPR; unused
        // pieces and rows past M fetch the zero page.  One wait covers them
        // and any BN-table loads issued before; the tile is this wave's own,
        // so no barrier.
        // (opaque: computed here, not folded into values kept across the
        // main loop)
        // (through a buffer resource: rows past the batch are out of range and
        // read as zeros, the unused piece of each row gets the FF_OOB offset)
        int lane_o = lane, m_o = mrow0;
        asm volatile("" : "+v"(lane_o), "+v"(m_o));
        const __amdgpu_buffer_rsrc_t r_add = ff_rsrc(a.add_src, (unsigned)a.M * COUT);
#pragma unroll
        for (int k = 0; k < RSLOTS / 64; k++) {
            const int slot = k * 64 + lane_o;
            const int row = slot / SPR;
            const int pc = slot - row * SPR;
            const unsigned off = pc < CH ? (unsigned)(m_o + row) * COUT + ncol0 + pc * 16 : FF_OOB;
            bdma16(r_add, off, 0, Ws + k * 1024);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else if (ADD && STAGE != 2) {   // residual tile -> LDS (coalesced 16-byte loads)
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
                Ws[row * P + col] = (int8_t)(RANGE == 2 ? ff::requant_fma_in_range(f, inv[j])
                                             : RANGE == 1 ? ff::requant_haz_in_range(f * inv[j])
                                                          : ff::requant_haz(f * inv[j]));
                // one 32x32 tile at a time: keeps the compiler from hoisting
                // every residual read of the wave tile into registers
                if (r == 15) asm volatile("" ::: "memory");
            }
    if constexpr (STAGE == 1) return;
    if (BN2 && LUT_DMA) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if constexpr (WG_SYNC) __syncthreads();
    else __builtin_amdgcn_wave_barrier();
    // Flush: 16-byte chunks of the X tile go out as they are; the BN second
    // output maps each byte through its channel's table on the way.  Both go
    // through buffer resources sized to the launch's tensors: rows past the
    // batch (and, for FFK_OUT_X_EVEN, X at odd pixels) get offsets out of
    // range and are dropped, so the flush has no branches and the table
    // reads of consecutive chunks can overlap.
    static_assert(32 % RPI == 0, "a copy instruction's rows lie in one 32-row block");
    static_assert(!XOFF || (CH == 4 && ROWS / RPI == 2), "xoff: the stem's two chunks, row lane/4 + 16k");
    const bool xe = (HO % 2 == 0 && WO % 2 == 0) && (a.flags & FFK_OUT_X_EVEN);
    const __amdgpu_buffer_rsrc_t r_x = ff_rsrc(a.out, a.out ? (unsigned)(xe ? a.M / 4 : a.M) * COUT : 0u);
    const __amdgpu_buffer_rsrc_t r_bn = ff_rsrc(a.out_bn, BN2 ? (unsigned)a.M * COUT : 0u);
    if constexpr (BN2 && BN_PASS) {
        // X as it is, then the table pass (results back into the tile), then
        // BN(X) from the tile
        constexpr int LR = ROWS >= 64 ? 64 : 32;          // tile rows per lookup instruction
        constexpr int CPI = 64 / LR;                      // 16-channel chunks per instruction
        static_assert(ROWS % LR == 0 && CH % CPI == 0, "whole passes");
#pragma unroll
        for (int k = 0; k < ROWS / RPI; k++) {
            const int row = lane / CH + k * RPI;
            const int ch = lane % CH;
            const v4i v = *reinterpret_cast<const v4i*>(Ws + row * P + ch * 16);
            unsigned xo;
            if constexpr (XOFF) {
                xo = xoff[k];
            } else {
                const unsigned xp = x_pix_blk<HO, WO>(a, mrow0 + (k * RPI / 32) * 32, row - (k * RPI / 32) * 32);
                xo = xp == FF_OOB ? FF_OOB : xp * COUT + ncol0 + ch * 16;
            }
            __builtin_amdgcn_raw_buffer_store_b128(v, r_x, xo, 0, 0);
        }
#pragma unroll
        for (int c0 = 0; c0 < CH; c0 += CPI) {
#pragma unroll
            for (int rb = 0; rb < ROWS / LR; rb++) {
                const int row = rb * LR + lane % LR;
                const int ch = c0 + lane / LR;
                int8_t* t = Ws + row * P + ch * 16;
                const v4i v = *reinterpret_cast<const v4i*>(t);
                const int8_t* L = Lw + (ch * 16) * FF_LUT_PITCH + 128;
                v4i o;
#pragma unroll
                for (int w = 0; w < 4; w++) {
                    uint32_t b[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const int q = (int8_t)((uint32_t)v[w] >> (e * 8));
                        b[e] = (uint8_t)L[(w * 4 + e) * FF_LUT_PITCH + q];
                    }
                    const uint32_t lo = __builtin_amdgcn_perm(b[1], b[0], 0x0c0c0400u);
                    const uint32_t hi = __builtin_amdgcn_perm(b[3], b[2], 0x0c0c0400u);
                    o[w] = (int)__builtin_amdgcn_perm(hi, lo, 0x05040100u);
                }
                *reinterpret_cast<v4i*>(t) = o;
            }
        }
#pragma unroll
        for (int k = 0; k < ROWS / RPI; k++) {
            const int row = lane / CH + k * RPI;
            const int ch = lane % CH;
            const v4i o = *reinterpret_cast<const v4i*>(Ws + row * P + ch * 16);
            __builtin_amdgcn_raw_buffer_store_b128(o, r_bn, (unsigned)(mrow0 + row) * COUT + ncol0 + ch * 16, 0, 0);
        }
        return;
    }
#pragma unroll
    for (int k = 0; k < ROWS / RPI; k++) {
        const int row = lane / CH + k * RPI;
        const int ch = lane % CH;
        const int m = mrow0 + row;
        const v4i v = *reinterpret_cast<const v4i*>(Ws + row * P + ch * 16);
        // (row = lane/CH + k*RPI: block k*RPI/32, a compile-time one)
        unsigned xo;
        if constexpr (XOFF) {
            xo = xoff[k];
        } else {
            const unsigned xp = x_pix_blk<HO, WO>(a, mrow0 + (k * RPI / 32) * 32, row - (k * RPI / 32) * 32);
            xo = xp == FF_OOB ? FF_OOB : xp * COUT + ncol0 + ch * 16;
        }
        __builtin_amdgcn_raw_buffer_store_b128(v, r_x, xo, 0, 0);
        if (BN2) {
            const int8_t* L = Lw + (ch * 16) * FF_LUT_PITCH + 128;
            v4i o;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                uint32_t b[4];
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int q = (int8_t)((uint32_t)v[w] >> (e * 8));
                    b[e] = (uint8_t)L[(w * 4 + e) * FF_LUT_PITCH + q];
                }
                // three byte permutes: (b0, b1), (b2, b3), then the two pairs
                // (v_perm_b32 selector bytes 0-3 pick the second operand's
                // bytes, 4-7 the first's, 0x0c a zero byte)
                const uint32_t lo = __builtin_amdgcn_perm(b[1], b[0], 0x0c0c0400u);
                const uint32_t hi = __builtin_amdgcn_perm(b[3], b[2], 0x0c0c0400u);
                o[w] = (int)__builtin_amdgcn_perm(hi, lo, 0x05040100u);
            }
            __builtin_amdgcn_raw_buffer_store_b128(o, r_bn, (unsigned)m * COUT + ncol0 + ch * 16, 0, 0);
        }
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
    const bool fma = rng && (a.flags & FFK_EPI_FMA_TAIL);
    constexpr int RF = INSC ? 1 : 2;   // (the in-scale instantiation never takes it)
#define FF_EPI(PR, AD, BN, RG) \
    wave_epi_i8<COUT, MI, NJ, PR, AD, BN, INSC, RG, HO, WO, true>(acc, a, P, mrow0, ncol0, Ws, Lw)
    switch (a.flags & (FFK_EPI_PRELU | FFK_EPI_ADD | FFK_EPI_BN)) {
    case 0:
        if (fma) FF_EPI(0, false, false, RF);
        else if (rng) FF_EPI(0, false, false, 1);
        else FF_EPI(0, false, false, 0);
        break;
    case FFK_EPI_PRELU:
        if (le1 && fma) FF_EPI(2, false, false, RF);
        else if (le1 && rng) FF_EPI(2, false, false, 1);
        else if (le1) FF_EPI(2, false, false, 0);
        else FF_EPI(1, false, false, 0);
        break;
    case FFK_EPI_ADD:
        if (rng) FF_EPI(0, true, false, 1);
        else FF_EPI(0, true, false, 0);
        break;
    case FFK_EPI_BN:
        if (fma) FF_EPI(0, false, true, RF);
        else if (rng) FF_EPI(0, false, true, 1);
        else FF_EPI(0, false, true, 0);
        break;
    case FFK_EPI_PRELU | FFK_EPI_BN:
        if (le1 && fma) FF_EPI(2, false, true, RF);
        else if (le1 && rng) FF_EPI(2, false, true, 1);
        else if (le1) FF_EPI(2, false, true, 0);
        else FF_EPI(1, false, true, 0);
        break;
    case FFK_EPI_ADD | FFK_EPI_BN:
        if (rng) FF_EPI(0, true, true, 1);
        else FF_EPI(0, true, true, 0);
        break;
    case FFK_EPI_PRELU | FFK_EPI_ADD: FF_EPI(1, true, false, 0); break;
    default: FF_EPI(1, true, true, 0); break;
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

// The two epilogues of a stride-2 conv fused with its block's 1x1 shortcut
// (the host fuses only these forms: the conv with bias and no PReLU,
// residual or BN; the shortcut with the residual add, optionally BN, no
// PReLU; neither with an in-scale).  First the conv's int8 tile into the
// wave's staging tile, no stores ...
template <int COUT, int MI, int NJ, int HO, int WO>
__device__ __forceinline__ void wave_epi_pair_stage(const v16i (&acc)[MI][NJ], const ConvArgs& a,
                                                    const EpiParams<NJ>& P, int mrow0, int ncol0, int8_t* Ws) {
    if ((a.flags & FFK_EPI_IN_RANGE) && (a.flags & FFK_EPI_FMA_TAIL))
        wave_epi_i8<COUT, MI, NJ, 0, false, false, false, 2, HO, WO, true, true, 1>(acc, a, P, mrow0, ncol0, Ws,
                                                                                   nullptr);
    else if (a.flags & FFK_EPI_IN_RANGE)
        wave_epi_i8<COUT, MI, NJ, 0, false, false, false, 1, HO, WO, true, true, 1>(acc, a, P, mrow0, ncol0, Ws,
                                                                                   nullptr);
    else
        wave_epi_i8<COUT, MI, NJ, 0, false, false, false, 0, HO, WO, true, true, 1>(acc, a, P, mrow0, ncol0, Ws,
                                                                                   nullptr);
}

// ... then the shortcut's, with that tile as its residual.
template <int COUT, int MI, int NJ, int HO, int WO>
__device__ __forceinline__ void wave_epi_pair_add(const v16i (&acc)[MI][NJ], const ConvArgs& b, int mrow0, int ncol0,
                                                  int8_t* Ws, const int8_t* Lw) {
    const EpiParams<NJ> P = load_epi_params<COUT, NJ>(b, ncol0);
    const bool rng = b.flags & FFK_EPI_IN_RANGE;
#define FF_EPI(BN, RG) \
    wave_epi_i8<COUT, MI, NJ, 0, true, BN, false, RG, HO, WO, true, true, 2>(acc, b, P, mrow0, ncol0, Ws, Lw)
    if (b.flags & FFK_EPI_BN) {
        if (rng) FF_EPI(true, 1);
        else FF_EPI(true, 0);
    } else {
        if (rng) FF_EPI(false, 1);
        else FF_EPI(false, 0);
    }
#undef FF_EPI
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
    // The FC head (a 1x1 image) split 8 ways takes split = XCD (workgroups
    // are dispatched round-robin over the 8 XCDs): each XCD streams one K
    // range of the activations and the weights for every tile, so both are
    // read from HBM about once (a row tile per XCD would read all the
    // weights on every XCD).  Elsewhere the splits of a tile are
    // consecutive within an XCD's contiguous run of tiles.
    constexpr bool SPLIT_BY_XCD = HIN == 1 && WIN == 1 && SPLIT == 8;
    const int xbid = SPLIT_BY_XCD ? (int)blockIdx.x : xcd_tile(blockIdx.x, gridDim.x);
    const int bid = SPLIT_BY_XCD ? xbid >> 3 : xbid / SPLIT;
    const int sp = SPLIT_BY_XCD ? xbid & 7 : xbid - bid * SPLIT;
    const int s_beg = sp * KSTEPS;
    const int tn = bid % (COUT / BN);              // (tiles_n = COUT / BN: a compile-time divisor)
    const int tm = bid / (COUT / BN);
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
        // Partial tiles are exchanged as agent-scope monotonic accesses: the
        // partial stores and the last workgroup's partial loads carry the sc1
        // cache policy (what gfx950 code for a relaxed agent-scope atomic
        // store or load uses: the store is written through the XCD's L2 and
        // complete only when visible device-wide, the load reads the
        // device-coherent value), every thread waits for its stores before the
        // barrier, and one thread then bumps the tile's agent-scope arrival
        // count.  The workgroup that arrives last sums the partials.  Only
        // the published bytes travel past the L2: no release / acquire fence,
        // which would write back or invalidate the whole L2 of the XCD (the
        // XCDs' L2s are not coherent with each other) once per workgroup.
        constexpr int NCH = MI * NJ * 4;            // 16-byte chunks per thread
        constexpr int PART = BM * BN * 4;           // bytes of one partial tile
        constexpr int CPOL_SC1 = 16;                // buffer cache policy: sc1 (device scope)
        const __amdgpu_buffer_rsrc_t r_ws = ff_rsrc(a.ws, (unsigned)gridDim.x * PART);
        const unsigned pbase = (unsigned)bid * SPLIT * PART;
#pragma unroll
        for (int c = 0; c < NCH; c++) {             // chunk-major: a wave stores 1 KB runs
            const v16i& t = acc[c / (NJ * 4)][(c / 4) % NJ];
            const v4i v = {t[(c % 4) * 4], t[(c % 4) * 4 + 1], t[(c % 4) * 4 + 2], t[(c % 4) * 4 + 3]};
            __builtin_amdgcn_raw_buffer_store_b128(v, r_ws, pbase + sp * PART + (c * 256 + tid) * 16, 0, CPOL_SC1);
        }
        __builtin_amdgcn_s_waitcnt(0);              // this wave's partial stores are complete
        __syncthreads();
        int* last = reinterpret_cast<int*>(smem);
        if (tid == 0)
            last[0] = __hip_atomic_fetch_add(&a.counters[bid], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                      (unsigned)(SPLIT - 1);
        __syncthreads();
        if (!last[0]) return;                       // another workgroup finishes this tile
        // G partial tiles per round (NCH * G loads in flight, at most 32
        // 16-byte chunks per thread) keep the registers within the
        // occupancy budget
        constexpr int G = (SPLIT % 4 == 0 && NCH * 4 <= 32) ? 4
                        : (SPLIT % 3 == 0 && NCH * 3 <= 32) ? 3
                        : (SPLIT % 2 == 0 && NCH * 2 <= 32) ? 2 : 1;
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
                    t[c][g] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(
                                                         r_ws, pbase + (q0 + g) * PART + (c * 256 + tid) * 16, 0,
                                                         CPOL_SC1));
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
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // (uniform: scalar)
    const int lane = tid & 63;
    // input (images x HIN x WIN x CIN, below 2 GiB) and packed weights as buffers
    const __amdgpu_buffer_rsrc_t r_in = ff_rsrc(a.in, (unsigned)(a.M / HWO) * (HIN * WIN * CIN));
    const __amdgpu_buffer_rsrc_t r_w = ff_rsrc(a.w, (unsigned)KSTEPS * COUT * FF_KSTEP);
    const int xbid = xcd_tile(blockIdx.x, gridDim.x);
    const int tn = xbid % (COUT / BN);             // (tiles_n = COUT / BN: a compile-time divisor)
    const int tm = xbid / (COUT / BN);
    const int m0 = tm * BM;

    // This thread's pieces: wave load j of wave w fills lines (j*NW + w)*4 ..
    // +3 of the stage tile; lane L takes line +L/16, slot L%16.  Registers are
    // kept few (occupancy): a 32-bit image offset per piece, the piece's input
    // origin (a row past the tile's end gets an origin that fails every bounds
    // check; such a piece, and every padding tap, is an out-of-range load that
    // returns zeros).
    int a_off[A_LD], a_ih0[A_LD], a_iw0[A_LD];
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
            bdma16(r_in, v ? (unsigned)(a_off[j] + (ih * WIN + iw) * CIN) : FF_OOB, (unsigned)(cs * DMA_KB),
                   sb + (j * NW + wave) * 1024);
        }
        const unsigned wst = (unsigned)(st * COUT * FF_KSTEP);
#pragma unroll
        for (int j = 0; j < B_LD; j++) bdma16(r_w, (unsigned)b_off[j], wst, sb + A_BYTES + (j * NW + wave) * 1024);
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
    // each patch buffer is followed by 1 KB of zeros: a masked tap's address
    // is the zero block's, and the second buffer's taps are the first's plus
    // PBUF, the zero block's included
    constexpr int PBUF = PATCH_BYTES + 1024;
    constexpr int ZERO_OFF = PATCH_BYTES;
    constexpr int RING_OFF = NPB * PBUF;
    constexpr int LDS_K = RING_OFF + NSTB * B_BYTES;
    constexpr int LDS_E = NW * wave_tile_bytes<MI, NJ>() + BN * FF_LUT_PITCH;
    constexpr int LDS = LDS_K > LDS_E ? LDS_K : LDS_E;
    static_assert(CIN % DMA_KB == 0, "Cin must be a multiple of 64");
    static_assert(B_BYTES % 1024 == 0 && (B_PART || B_BYTES % (NT * 16) == 0), "whole wave loads");
    static_assert(COUT % BN == 0, "Cout must be a multiple of BN");
    static_assert(B_LD + LA < 64, "load counter range");
    static_assert((NPB - 1) * PBUF + (2 * W + 2) * PATCH_PITCH + 32 + 16 < 65536,
                  "tap offsets fit the ds_read offset field");
    static_assert(NPB == 1 || CSTEPS % 2 == 0, "runs go in pairs over the two buffers");

    __shared__ __align__(1024) int8_t smem[LDS];
    const int tid = threadIdx.x;
    // (the wave index is uniform: kept in a scalar register, so the LDS
    // destinations of the direct-to-LDS loads are scalar arithmetic)
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int xbid = xcd_tile(blockIdx.x, gridDim.x);
    const int tn = xbid % (COUT / BN);             // (tiles_n = COUT / BN: a compile-time divisor)
    const int tm = xbid / (COUT / BN);
    const int m0 = tm * BM;
    const int first = m0 - W - 1;                            // input pixel of patch pixel 0
    // the input tensor (a.M pixels; the host keeps it below 2 GiB) and the
    // packed weights as buffers
    const __amdgpu_buffer_rsrc_t r_in = ff_rsrc(a.in, (unsigned)a.M * CIN);
    const __amdgpu_buffer_rsrc_t r_w = ff_rsrc(a.w, 9u * CSTEPS * COUT * FF_KSTEP);

    // Zero block: masked taps read it.  Wave loads beyond the patch's PLOADS
    // (every thread issues LA, so that all waves count the same loads) are
    // out-of-range loads into it.
    for (int i = tid; i < 64 * NPB; i += NT)
        reinterpret_cast<v4i*>(smem + ZERO_OFF + (i >> 6) * PBUF)[i & 63] = v4i{0, 0, 0, 0};

    // Patch slots of this thread: wave load j of wave w is patch block j*NW + w,
    // lane L its slot L, i.e. patch pixel slot/5, piece slot%5 (piece 4 is the
    // unused 16 bytes).  Input offset of the slot at channel run 0, or FF_OOB
    // for the unused piece.  A pixel outside the batch needs no test: past
    // the end its offset is at least the buffer's a.M * CIN bytes, before the
    // start (g >= -W-1) it is negative, i.e. at least 2^31 as the unsigned
    // offset the hardware checks (a.M * CIN < 2^31); either way the load is
    // out of range and returns zeros.  (The channel run's offset goes in the
    // scalar offset, which stays inside the pixel.)
    unsigned p_src[LA];
#pragma unroll
    for (int j = 0; j < LA; j++) {
        const int blk = j * NW + wave;
        const int slot = blk * 64 + lane;
        const int px = slot / 5;
        const int piece = slot - px * 5;
        const int g = first + px;
        const bool ok = blk < PLOADS && piece < 4;
        p_src[j] = ok ? (unsigned)g * CIN + piece * 16 : FF_OOB;        // (mod 2^32)
    }
    auto issue_patch = [&](int c, int buf) {
#pragma unroll
        for (int j = 0; j < LA; j++) {
            const int blk = j * NW + wave;
            bdma16(r_in, p_src[j], (unsigned)(c * DMA_KB), smem + (blk < PLOADS ? buf * PBUF + blk * 1024 : ZERO_OFF));
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
        const unsigned wst = (unsigned)((t * CSTEPS + c) * COUT * FF_KSTEP);
#pragma unroll
        for (int j = 0; j < B_LD; j++)
            bdma16(r_w, (unsigned)b_off[j], wst, smem + RING_OFF + slot * B_BYTES + (j * NW + wave) * 1024);
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

    // LDS address of every tap of every row tile of this lane, selected once
    // (masked taps: the zero block): no per-step address arithmetic
    int ta[9][MI];
#pragma unroll
    for (int i = 0; i < MI; i++) {
        // (four lane masks per row tile; a tap's mask is the OR of at most two)
        const bool top = a_edge[i] & 1, bot = a_edge[i] & 2, left = a_edge[i] & 4, right = a_edge[i] & 8;
#pragma unroll
        for (int t = 0; t < 9; t++) {
            const int kh = t / 3, kw = t % 3;
            const bool masked = (kh == 0 && top) || (kh == 2 && bot) || (kw == 0 && left) || (kw == 2 && right);
            ta[t][i] = masked ? z_addr : a_base[i] + (kh * W + kw) * PATCH_PITCH;
        }
    }

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
    // channel run c, its patch in buffer PB (c % 2: a compile-time offset)
    auto run = [&](const int c, auto pbc) {
        constexpr int PB = decltype(pbc)::value;
        const bool more = c + 1 < CSTEPS;
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
            if (t == 0 && more) issue_patch(c + 1, 1 - PB);

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
                for (int i = 0; i < MI; i++)
                    af[i] = *reinterpret_cast<const v4i*>(smem + ta[t][i] + PB * PBUF + ks * 32);
#pragma unroll
                for (int j = 0; j < NJ; j++) bf[j] = *reinterpret_cast<const v4i*>(smem + ((br + j * 2048) ^ (ks * 32)));
#pragma unroll
                for (int i = 0; i < MI; i++)
#pragma unroll
                    for (int j = 0; j < NJ; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
        }
    };
    for (int c = 0; c < CSTEPS; c += NPB) {
        run(c, std::integral_constant<int, 0>{});
        if constexpr (NPB == 2) run(c + 1, std::integral_constant<int, 1>{});
    }
    __syncthreads();                       // every wave is done with the patch and the ring

    int8_t* Ws = smem + wave * wave_tile_bytes<MI, NJ>();
    int8_t* Ls = smem + NW * wave_tile_bytes<MI, NJ>();
    if (a.flags & FFK_EPI_BN && !a.out_i32) issue_bn_lut<NW, BN>(Ls, a.bn_lut, tn * BN);
    wave_epilogue<COUT, MI, NJ, H, W>(acc, a, m0 + wm * MI * 32, tn * BN + wn * NJ * 32, Ws,
                                Ls + (wn * NJ * 32) * FF_LUT_PITCH);
}

// ---------------------------------------------------------------------------
// 3x3 stride-2 pad-1 conv with the input staged once per channel run, as four
// phase patches.  Phase (rp, cp) of the input is the image of its pixels
// (2i + rp, 2j + cp), HO x WO like the output, and indexed like it: tap
// (kh, kw) of output pixel (oh, ow) reads phase (kh != 1, kw != 1) at
// (oh + di, ow + dj), di = kh == 0 ? -1 : 0 (dj likewise).  So for a tile of
// BM consecutive output pixels every tap reads one phase's run of pixels
// m0 - WO - 1 .. m0 + BM - 1 at a constant offset (0, 1, WO or WO + 1), and a
// tap whose input row or column is -1 (oh == 0 with di = -1, ow == 0 with
// dj = -1) reads the zero block instead.  The steps go phase by phase --
// (1,1): 4 taps, (1,0): 2, (0,1): 2, (0,0): 1 -- and within a phase run by run
// (64 channels each), so the channel runs of one input pixel, which share its
// 128-byte L2 lines, are fetched one right after the other (run-major order
// re-fetched those lines from HBM for the second run: 1.57x the algorithmic
// bytes at 128 channels).  Each (phase, run) patch is staged once in LDS,
// double-buffered: the next one is issued at the barrier of the current one's
// first step, before that step's weights, and a one-tap phase waits for it at
// its own end.  The weights of each tap go through the 3-stage ring of
// conv3_patch_kernel; s2::Plan computes every barrier's load count at compile
// time.  Each input pixel is read about once per tile (the im2col gather of
// conv_dma_kernel reads each one for every tap that covers it).
// ---------------------------------------------------------------------------
namespace s2 {
// taps of the four phases, phase by phase: (1,1) taps 0-3, (1,0) 4-5, (0,1) 6-7, (0,0) 8
constexpr int first_tap[4] = {0, 4, 6, 8};
constexpr int len[4] = {4, 2, 2, 1};
constexpr int kh[9] = {0, 0, 2, 2, 0, 2, 1, 1, 1};
constexpr int kw[9] = {0, 2, 0, 2, 1, 1, 0, 2, 1};
constexpr int rp[4] = {1, 1, 0, 0};
constexpr int cp[4] = {1, 0, 1, 0};

// Step order and load waits of the phase kernel for C 64-channel runs.  The
// steps go phase-major: phase q's patch for run 0, its taps, then run 1's
// patch of the same phase and its taps, ...  (one input pixel's channel runs
// share 128-byte L2 lines, so the runs of a phase follow each other while the
// lines are still in L2).  Patch p = q*C + c; step s reads patch pat[s] at
// tap tap[s] of run run[s].  Loads are issued at step barriers, in this order:
// prologue: patch 0, weights 0, weights 1; at the barrier of step s: patch
// pat[s] + 1 if s is the first step of its patch, then weights s + 2.  wait[s]
// (wait_p[s] for a wave that loads no weights) is how many of this wave's
// loads may still be in flight at step s's barrier, with step s's weights and
// patch landed: everything issued after the later of the two.
template <int C, int LA, int BL>
struct Plan {
    static constexpr int N = 9 * C;
    int pat[N], tap[N], run[N], first[N], wait[N], wait_p[N];
    constexpr Plan() : pat(), tap(), run(), first(), wait(), wait_p() {
        int st = 0;
        for (int q = 0; q < 4; q++)
            for (int c = 0; c < C; c++)
                for (int t = 0; t < len[q]; t++) {
                    pat[st] = q * C + c;
                    tap[st] = first_tap[q] + t;
                    run[st] = c;
                    first[st] = t == 0;
                    st++;
                }
        // issue order: (kind, id, count) with kind 0 patch, 1 weights
        int kind[3 * N + 3] = {}, id[3 * N + 3] = {}, cnt[3 * N + 3] = {}, at[3 * N + 3] = {};
        int n = 0;
        auto add = [&](int k, int i, int c_, int barrier) { kind[n] = k; id[n] = i; cnt[n] = c_; at[n] = barrier; n++; };
        add(0, 0, LA, -1);
        add(1, 0, BL, -1);
        if (N > 1) add(1, 1, BL, -1);
        for (int b = 0; b < N; b++) {
            if (first[b] && pat[b] + 1 < 4 * C) add(0, pat[b] + 1, LA, b);
            if (b + 2 < N) add(1, b + 2, BL, b);
        }
        for (int s2 = 0; s2 < N; s2++) {
            int last_w = -1, last_p = -1;
            for (int i = 0; i < n; i++) {
                if (kind[i] == 1 && id[i] == s2) last_w = i;
                if (kind[i] == 0 && id[i] == pat[s2]) last_p = i;
            }
            const int lw = last_w > last_p ? last_w : last_p;
            int after = 0, after_p = 0;
            for (int i = 0; i < n; i++) {
                if (at[i] >= s2) continue;                   // not issued yet at this barrier
                if (i > lw) after += cnt[i];
                if (i > last_p && kind[i] == 0) after_p += cnt[i];
            }
            wait[s2] = after;
            wait_p[s2] = after_p;
        }
    }
};

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<I + 1, N>(f);
    }
}
}  // namespace s2

// CX > 0: the launch also runs the block's 1x1 shortcut conv b (CX input
// channels, over the compact block input: output pixel m reads its pixel m)
// whose epilogue adds this conv's int8 output.  That output stays in the
// waves' staging tiles and is never stored: after the main loop the conv's
// epilogue leaves it there, the shortcut's GEMM (CX/64 steps, its operands
// staged past the staging tiles; the first step's loads are issued before the
// conv's epilogue runs) reuses the accumulators, and the shortcut's epilogue
// reads its residual from the tiles.  The arithmetic of both epilogues is the
// same as in two separate launches.
template <int CIN, int COUT, int H, int W, int WM, int WN, int MI, int NJ, int CX>
__device__ __forceinline__ void conv3s2_phase_body(const ConvArgs& a, const ConvArgs& b) {
    constexpr int NW = WM * WN;
    constexpr int NT = NW * 64;
    constexpr int BM = WM * MI * 32, BN = WN * NJ * 32;
    constexpr int HO = H / 2, WO = W / 2;
    constexpr int CSTEPS = CIN / DMA_KB;
    constexpr int NSTEP = 9 * CSTEPS;
    constexpr int NP = BM + WO + 1;                          // phase patch pixels
    constexpr int PSLOTS = NP * (PATCH_PITCH / 16);
    constexpr int PLOADS = (PSLOTS + 63) / 64;
    constexpr int LA = (PLOADS + NW - 1) / NW;
    constexpr int PATCH_BYTES = PLOADS * 1024;
    constexpr int B_BYTES = BN * DMA_KB;
    constexpr int BW = B_BYTES / 1024;
    constexpr bool B_PART = BW < NW;
    constexpr int B_LD = B_PART ? 1 : B_BYTES / (NT * 16);
    constexpr int NSTB = 3;
    // each of the two patch buffers is followed by 1 KB of zeros: a masked
    // tap's address is the zero block's, the second buffer's taps are the
    // first's plus PBUF
    constexpr int PBUF = PATCH_BYTES + 1024;
    constexpr int ZERO_OFF = PATCH_BYTES;
    constexpr int RING_OFF = 2 * PBUF;
    constexpr int LDS_K = RING_OFF + NSTB * B_BYTES;
    constexpr int LDS_E = NW * wave_tile_bytes<MI, NJ>() + BN * FF_LUT_PITCH;
    // fused shortcut: its A operand (BM compact-input pixels at the patch
    // pitch) and B operand (one 64-channel run of its weights) past the
    // staging tiles; the BN table of the shortcut's epilogue goes over them
    // once its GEMM is done
    constexpr int A2_LOADS = (BM * (PATCH_PITCH / 16) + 63) / 64;
    constexpr int LA2 = (A2_LOADS + NW - 1) / NW;
    constexpr int A2_OFF = (NW * wave_tile_bytes<MI, NJ>() + 1023) / 1024 * 1024;
    constexpr int B2_OFF = A2_OFF + A2_LOADS * 1024;
    constexpr int LDS_SC = CX > 0 ? B2_OFF + B_BYTES : 0;
    constexpr int LDS_KE = LDS_K > LDS_E ? LDS_K : LDS_E;
    constexpr int LDS = LDS_KE > LDS_SC ? LDS_KE : LDS_SC;
    static_assert(CX % DMA_KB == 0, "shortcut input channels: a multiple of 64");
    static_assert(H % 2 == 0 && W % 2 == 0, "even input");
    static_assert(CIN % DMA_KB == 0, "Cin must be a multiple of 64");
    static_assert(B_BYTES % 1024 == 0 && (B_PART || B_BYTES % (NT * 16) == 0), "whole wave loads");
    static_assert(COUT % BN == 0, "Cout must be a multiple of BN");
    static_assert(B_LD + LA < 64, "load counter range");
    static_assert(PBUF + (WO + 1) * PATCH_PITCH + 32 + 16 < 65536, "tap offsets fit the ds_read offset field");

    __shared__ __align__(1024) int8_t smem[LDS];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // (uniform: scalar)
    const int lane = tid & 63;
    const int xbid = xcd_tile(blockIdx.x, gridDim.x);
    const int tn = xbid % (COUT / BN);             // (tiles_n = COUT / BN: a compile-time divisor)
    const int tm = xbid / (COUT / BN);
    const int m0 = tm * BM;
    const int first = m0 - WO - 1;                           // phase pixel of patch pixel 0
    // input (batch x H x W x CIN, below 2 GiB) and packed weights as buffers
    const int nimg = a.M / (HO * WO);
    const __amdgpu_buffer_rsrc_t r_in = ff_rsrc(a.in, (unsigned)nimg * (H * W * CIN));
    const __amdgpu_buffer_rsrc_t r_w = ff_rsrc(a.w, 9u * CSTEPS * COUT * FF_KSTEP);

    for (int i = tid; i < 128; i += NT)
        reinterpret_cast<v4i*>(smem + ZERO_OFF + (i >> 6) * PBUF)[i & 63] = v4i{0, 0, 0, 0};

    // patch slot -> input offset of the phase-(0,0) pixel (2i, 2j) of phase
    // pixel n = first + slot/5 (piece slot%5; piece 4 is the pitch padding),
    // or FF_OOB (the load returns zeros)
    unsigned p_src[LA];
#pragma unroll
    for (int j = 0; j < LA; j++) {
        const int blk = j * NW + wave;
        const int slot = blk * 64 + lane;
        const int px = slot / 5;
        const int piece = slot - px * 5;
        const int n = first + px;
        const bool ok = blk < PLOADS && piece < 4 && n >= 0 && n < a.M;
        const int nn = ok ? n : 0;
        const int b = nn / (HO * WO);
        const int rem = nn - b * (HO * WO);
        const int i = rem / WO;
        const int jj = rem - i * WO;
        p_src[j] = ok ? (unsigned)(((b * H + 2 * i) * W + 2 * jj) * CIN + piece * 16) : FF_OOB;
    }
    // patch P = q*CSTEPS + c (phase q of run c) into buffer P & 1
    auto issue_patch = [&](int P) {
        const int q = P / CSTEPS, c = P - q * CSTEPS;
        const int poff = (s2::rp[q] * W + s2::cp[q]) * CIN + c * DMA_KB;
#pragma unroll
        for (int j = 0; j < LA; j++) {
            const int blk = j * NW + wave;
            bdma16(r_in, p_src[j], (unsigned)poff, smem + (blk < PLOADS ? (P & 1) * PBUF + blk * 1024 : ZERO_OFF));
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
    const bool loads_b = !B_PART || wave < BW;
    // weights of step s (run PLAN.run[s], tap PLAN.tap[s]) into ring slot s % 3
    constexpr s2::Plan<CSTEPS, LA, B_LD> PLAN{};
    auto issue_b = [&](int s) {
        if (!loads_b) return;
        const int c = PLAN.run[s], k = PLAN.tap[s];
        const int tap = s2::kh[k] * 3 + s2::kw[k];
        const unsigned wst = (unsigned)((tap * CSTEPS + c) * COUT * FF_KSTEP);
#pragma unroll
        for (int j = 0; j < B_LD; j++)
            bdma16(r_w, (unsigned)b_off[j], wst, smem + RING_OFF + (s % NSTB) * B_BYTES + (j * NW + wave) * 1024);
    };

    const int wm = wave / WN;
    const int wn = wave % WN;
    // edge bits of this lane's output rows: 1 first output row, 4 first column
    int a_base[MI], a_edge[MI];
#pragma unroll
    for (int i = 0; i < MI; i++) {
        const int r = wm * MI * 32 + i * 32 + (lane & 31);
        const int m = m0 + r;
        const int rr = m % (HO * WO);
        const int oh = rr / WO;
        const int ow = rr - oh * WO;
        a_edge[i] = (oh == 0 ? 1 : 0) | (ow == 0 ? 4 : 0);
        a_base[i] = r * PATCH_PITCH + (lane >> 5) * 16;
    }
    const int z_addr = ZERO_OFF + (lane >> 5) * 16;
    const int b_rd = RING_OFF + dma_slot(wn * NJ * 32 + (lane & 31), lane >> 5);
    // LDS address of each row tile for the four tap offsets (di, dj) in
    // {-1, 0}^2 (index (di + 1) * 2 + dj + 1), selected once
    int ta[4][MI];
#pragma unroll
    for (int o = 0; o < 4; o++) {
        const int di = (o >> 1) - 1, dj = (o & 1) - 1;
        const int emask = (di ? 1 : 0) | (dj ? 4 : 0);
#pragma unroll
        for (int i = 0; i < MI; i++)
            ta[o][i] = (a_edge[i] & emask) ? z_addr : a_base[i] + ((WO + 1) + di * WO + dj) * PATCH_PITCH;
    }

    v16i acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

    // prologue: patch 0, weights of steps 0 and 1 (in that order)
    issue_patch(0);
    issue_b(0);
    issue_b(1);
    s2::static_for<0, NSTEP>([&](auto sc) {
        constexpr int s = decltype(sc)::value;
        constexpr int k = PLAN.tap[s];
        constexpr int P = PLAN.pat[s];
        // barrier before step s: its weights and its patch have landed
        if (loads_b) dma_wait_barrier<PLAN.wait[s]>();
        else dma_wait_barrier<PLAN.wait_p[s]>();
        // at a patch's first step: the next patch (into the buffer the patch
        // before this one used), then the weights two steps ahead
        if constexpr (PLAN.first[s] && P + 1 < 4 * CSTEPS) issue_patch(P + 1);
        if constexpr (s + 2 < NSTEP) issue_b(s + 2);

        constexpr int o = (s2::kh[k] == 0 ? 0 : 2) + (s2::kw[k] == 0 ? 0 : 1);
        constexpr int pbo = (P & 1) * PBUF;
        const int br = b_rd + (s % NSTB) * B_BYTES;
#if FF_PATCH_IGLP
        __builtin_amdgcn_iglp_opt(1);
#endif
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            v4i af[MI], bf[NJ];
#pragma unroll
            for (int i = 0; i < MI; i++) af[i] = *reinterpret_cast<const v4i*>(smem + ta[o][i] + pbo + ks * 32);
#pragma unroll
            for (int j = 0; j < NJ; j++) bf[j] = *reinterpret_cast<const v4i*>(smem + ((br + j * 2048) ^ (ks * 32)));
#pragma unroll
            for (int i = 0; i < MI; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    });
    __syncthreads();

    int8_t* Ws = smem + wave * wave_tile_bytes<MI, NJ>();
    int8_t* Ls = smem + NW * wave_tile_bytes<MI, NJ>();
    const int mrow0 = m0 + wm * MI * 32, ncol0 = tn * BN + wn * NJ * 32;
    if constexpr (CX == 0) {
        if (a.flags & FFK_EPI_BN && !a.out_i32) issue_bn_lut<NW, BN>(Ls, a.bn_lut, tn * BN);
        wave_epilogue<COUT, MI, NJ, HO, WO>(acc, a, mrow0, ncol0, Ws, Ls + (wn * NJ * 32) * FF_LUT_PITCH);
    } else {
        // the conv's epilogue parameters before the shortcut's loads, so that
        // waiting for them does not wait for those
        const EpiParams<NJ> P1 = load_epi_params<COUT, NJ>(a, ncol0);
        // shortcut operands of channel run c: A2 slot (pixel px, piece p) at
        // 16*(5*px + p) (piece 4 unused: FF_OOB, zeros), pixels past the batch
        // out of range (zeros); B2 as a weight ring slot.  (1x1 weights:
        // stage c of the packing is channel run c.)
        const __amdgpu_buffer_rsrc_t r_x2 = ff_rsrc(b.in, (unsigned)a.M * CX);
        const __amdgpu_buffer_rsrc_t r_w2 = ff_rsrc(b.w, (unsigned)(CX / DMA_KB) * COUT * FF_KSTEP);
        auto issue_sc = [&](int c) {
#pragma unroll
            for (int j = 0; j < LA2; j++) {
                const int blk = j * NW + wave;
                if (blk < A2_LOADS) {                        // (uniform per wave)
                    const int slot = blk * 64 + lane;
                    const int px = slot / 5;
                    const int piece = slot - px * 5;
                    const unsigned off = piece < 4 ? (unsigned)(m0 + px) * CX + piece * 16 : FF_OOB;
                    bdma16(r_x2, off, (unsigned)(c * DMA_KB), smem + A2_OFF + blk * 1024);
                }
            }
            if (loads_b) {
#pragma unroll
                for (int j = 0; j < B_LD; j++)
                    bdma16(r_w2, (unsigned)b_off[j], (unsigned)(c * COUT * FF_KSTEP),
                           smem + B2_OFF + (j * NW + wave) * 1024);
            }
        };
        issue_sc(0);
        wave_epi_pair_stage<COUT, MI, NJ, HO, WO>(acc, a, P1, mrow0, ncol0, Ws);
#pragma unroll
        for (int i = 0; i < MI; i++)
#pragma unroll
            for (int j = 0; j < NJ; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[i][j][r] = 0;
        const int a2_rd = A2_OFF + (wm * MI * 32 + (lane & 31)) * PATCH_PITCH + (lane >> 5) * 16;
        const int b2_rd = B2_OFF + dma_slot(wn * NJ * 32 + (lane & 31), lane >> 5);
#pragma unroll
        for (int c = 0; c < CX / DMA_KB; c++) {
            dma_wait_barrier<0>();                   // run c's operands landed
#pragma unroll
            for (int ks = 0; ks < 2; ks++) {
                v4i af[MI], bf[NJ];
#pragma unroll
                for (int i = 0; i < MI; i++)
                    af[i] = *reinterpret_cast<const v4i*>(smem + a2_rd + i * 32 * PATCH_PITCH + ks * 32);
#pragma unroll
                for (int j = 0; j < NJ; j++) bf[j] = *reinterpret_cast<const v4i*>(smem + ((b2_rd + j * 2048) ^ (ks * 32)));
#pragma unroll
                for (int i = 0; i < MI; i++)
#pragma unroll
                    for (int j = 0; j < NJ; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
            }
            if (c + 1 < CX / DMA_KB) {
                dma_wait_barrier<0>();               // every wave is done with run c
                issue_sc(c + 1);
            }
        }
        dma_wait_barrier<0>();                       // every wave is done with the operands
        if (b.flags & FFK_EPI_BN) issue_bn_lut<NW, BN>(Ls, b.bn_lut, tn * BN);
        wave_epi_pair_add<COUT, MI, NJ, HO, WO>(acc, b, mrow0, ncol0, Ws, Ls + (wn * NJ * 32) * FF_LUT_PITCH);
    }
}

template <int CIN, int COUT, int H, int W, int WM, int WN, int MI, int NJ, int WPE>
__global__ __launch_bounds__(WM * WN * 64, WPE) void conv3s2_phase_kernel(ConvArgs a) {
    conv3s2_phase_body<CIN, COUT, H, W, WM, WN, MI, NJ, 0>(a, a);
}

// the stride-2 conv a and the 1x1 shortcut b that adds a's output, one launch
template <int CIN, int COUT, int H, int W, int WM, int WN, int MI, int NJ, int WPE, int CX>
__global__ __launch_bounds__(WM * WN * 64, WPE) void conv3s2_shortcut_kernel(ConvArgs a, ConvArgs b) {
    conv3s2_phase_body<CIN, COUT, H, W, WM, WN, MI, NJ, CX>(a, b);
}

namespace ps1 {
// Load schedule of the small-grid patch kernel: RUNS channel runs of 9 taps
// (N = 9*RUNS steps), a barrier before every U-th step, weights D steps ahead
// in a ring of D + U slots.  Prologue: patch 0, then the weights of steps
// 0 .. D-1.  At the barrier before step b: the weights of steps b+D ..
// b+D+U-1, then the patch of run pnext[b/U] (-1: none).  Run r+1's patch goes
// into the buffer of run r-1, so it is issued at the first barrier at or
// after run r's first step (every step of run r-1 is done there).
// wait[k] (wait_p[k] for a wave that loads no weights) is how many of this
// wave's loads may still be in flight at barrier k with the weights and the
// patches of steps kU .. kU+U-1 landed.
template <int RUNS, int LA, int BL, int D, int U>
struct Plan {
    static constexpr int N = 9 * RUNS;
    static constexpr int NB = (N + U - 1) / U;
    int pnext[NB], wait[NB], wait_p[NB];
    constexpr Plan() : pnext(), wait(), wait_p() {
        for (int k = 0; k < NB; k++) pnext[k] = -1;
        for (int r = 0; r + 1 < RUNS; r++) pnext[(9 * r + U - 1) / U] = r + 1;
        constexpr int MAXI = 2 * N + RUNS + 2;
        int kind[MAXI] = {}, id[MAXI] = {}, cnt[MAXI] = {}, at[MAXI] = {};
        int n = 0;
        auto add = [&](int k, int i, int c, int bar) { kind[n] = k; id[n] = i; cnt[n] = c; at[n] = bar; n++; };
        add(0, 0, LA, -1);
        for (int w = 0; w < D && w < N; w++) add(1, w, BL, -1);
        for (int k = 0; k < NB; k++) {
            for (int i = 0; i < U; i++)
                if (k * U + D + i < N) add(1, k * U + D + i, BL, k);
            if (pnext[k] >= 0) add(0, pnext[k], LA, k);
        }
        for (int k = 0; k < NB; k++) {
            int last = -1, last_p = -1;
            for (int st = k * U; st < k * U + U && st < N; st++)
                for (int i = 0; i < n; i++) {
                    if (kind[i] == 1 && id[i] == st && i > last) last = i;
                    if (kind[i] == 0 && id[i] == st / 9 && i > last_p) last_p = i;
                }
            if (last_p > last) last = last_p;
            int after = 0, after_p = 0;
            for (int i = 0; i < n; i++) {
                if (at[i] >= k) continue;                    // not issued yet at this barrier
                if (i > last) after += cnt[i];
                if (i > last_p && kind[i] == 0) after_p += cnt[i];
            }
            wait[k] = after;
            wait_p[k] = after_p;
        }
    }
};
}  // namespace ps1

// ---------------------------------------------------------------------------
// Small-grid variant of the 3x3 stride-1 patch kernel: the channel runs of a
// tile are shared by KG groups of WM x WN waves inside the workgroup (group g
// takes runs g, g + KG, ...), each group with its own patch buffers and
// weight ring; all groups step in lockstep (one barrier per step).  At the
// end the int32 partial tiles are summed through LDS: the MI x NJ MFMA
// blocks of a wave position are divided among the groups (group g owns
// blocks g*T/KG .. (g+1)*T/KG - 1 in row-major order, T = MI*NJ); every
// other group writes its partial of those blocks, the owner adds them and
// runs the epilogue on its blocks.  Integer sums are exact, so the result is
// the whole-K kernel's.  This gives a small batch KG times the waves without
// the partial tiles' round trip through memory of split-K across workgroups.
// A small grid has one workgroup per CU, so no other workgroup fills the
// SIMDs while its waves meet at a barrier: the steps go U at a time between
// barriers, the weights D steps ahead in a ring of D + U slots (ps1::Plan);
// the epilogue's per-channel parameters are loaded before the main loop.
// ---------------------------------------------------------------------------
template <int CIN, int COUT, int H, int W, int WM, int WN, int MI, int NJ, int KG, int WPE, int D, int U>
__global__ __launch_bounds__(WM * WN * KG * 64, WPE) void conv3_patch_kg_kernel(ConvArgs a) {
    constexpr int NWG = WM * WN;                             // waves per group
    constexpr int NW = NWG * KG;
    constexpr int NTG = NWG * 64;
    constexpr int BM = WM * MI * 32, BN = WN * NJ * 32;
    constexpr int CSTEPS = CIN / DMA_KB;                     // 64-channel runs
    constexpr int RUNS = CSTEPS / KG;                        // runs of one group
    constexpr int NP = BM + 2 * W + 2;
    constexpr int PSLOTS = NP * (PATCH_PITCH / 16);
    constexpr int PLOADS = (PSLOTS + 63) / 64;
    constexpr int LA = (PLOADS + NWG - 1) / NWG;             // patch loads per thread
    constexpr int PATCH_BYTES = PLOADS * 1024;
    constexpr int B_BYTES = BN * DMA_KB;
    constexpr int BW = B_BYTES / 1024;
    constexpr bool B_PART = BW < NWG;
    constexpr int B_LD = B_PART ? 1 : B_BYTES / (NTG * 16);
    constexpr int NSTB = D + U;                              // weight ring slots
    constexpr int NSTEP = 9 * RUNS;
    constexpr int NPB = RUNS > 1 ? 2 : 1;
    // a group's patch buffers are each followed by 1 KB of zeros (masked
    // taps read them; the second buffer's taps are the first's plus PBUF)
    constexpr int PBUF = PATCH_BYTES + 1024;
    constexpr int GROUP_BYTES = NPB * PBUF + NSTB * B_BYTES;
    constexpr int ZERO_OFF = PATCH_BYTES;                    // (within each group)
    constexpr int LDS_K = KG * GROUP_BYTES;
    constexpr int T = MI * NJ;                               // MFMA blocks per wave
    constexpr int TO = T / KG;                               // blocks a group owns
    constexpr int PART = 64 * 64;                            // bytes of one block's partial (per wave)
    // partials are summed CHUNK blocks at a time: as many as fit beside the
    // main loop's LDS footprint (all of them when KG == 2)
    constexpr int BLOCK_X = (KG - 1) * NWG * PART;           // LDS of one block's partials
    constexpr int LDS_BASE = LDS_K > 64 * 1024 ? LDS_K : 64 * 1024;
    constexpr int CHUNK = KG == 1 ? 1 : (T * BLOCK_X <= LDS_BASE ? T : (LDS_BASE / BLOCK_X > 0 ? LDS_BASE / BLOCK_X : 1));
    constexpr int LDS_X = KG == 1 ? 0 : CHUNK * BLOCK_X;
    // owned blocks as an (MO x NO) sub-block at (i0, j0) of the wave tile
    constexpr int NO = TO >= NJ ? NJ : TO;
    constexpr int MO = TO >= NJ ? TO / NJ : 1;
    constexpr int LDS_E = NW * wave_tile_bytes<MO, NO>() + BN * FF_LUT_PITCH;
    constexpr int LDS = LDS_K > LDS_E ? (LDS_K > LDS_X ? LDS_K : LDS_X) : (LDS_E > LDS_X ? LDS_E : LDS_X);
    static_assert(CIN % DMA_KB == 0 && CSTEPS % KG == 0, "runs divide among the groups");
    static_assert(T % KG == 0 && (TO % NJ == 0 || NJ % TO == 0), "blocks divide among the groups");
    static_assert(B_BYTES % 1024 == 0 && (B_PART || B_BYTES % (NTG * 16) == 0), "whole wave loads");
    static_assert(COUT % BN == 0, "Cout must be a multiple of BN");
    static_assert(D >= U && U >= 1 && (D + U) * B_LD + 2 * LA < 64, "load counter range");
    static_assert((NPB - 1) * PBUF + (2 * W + 2) * PATCH_PITCH + 32 + 16 < 65536,
                  "tap offsets fit the ds_read offset field");
    static_assert(LDS <= 160 * 1024, "LDS");
    constexpr ps1::Plan<RUNS, LA, B_LD, D, U> PLAN{};

    __shared__ __align__(1024) int8_t smem[LDS];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // (uniform: scalar)
    const int lane = tid & 63;
    const int g = wave / NWG;                                // K group (uniform per wave)
    const int wg = wave - g * NWG;                           // wave within the group
    const int xbid = xcd_tile(blockIdx.x, gridDim.x);
    const int tn = xbid % (COUT / BN);             // (tiles_n = COUT / BN: a compile-time divisor)
    const int tm = xbid / (COUT / BN);
    const int m0 = tm * BM;
    const int first = m0 - W - 1;
    int8_t* gbase = smem + g * GROUP_BYTES;                   // this group's patches and ring
    const __amdgpu_buffer_rsrc_t r_in = ff_rsrc(a.in, (unsigned)a.M * CIN);
    const __amdgpu_buffer_rsrc_t r_w = ff_rsrc(a.w, 9u * CSTEPS * COUT * FF_KSTEP);

    for (int i = tid; i < 64 * NPB * KG; i += NW * 64)
        reinterpret_cast<v4i*>(smem + (i >> 6) / NPB * GROUP_BYTES + ZERO_OFF + (i >> 6) % NPB * PBUF)[i & 63] =
            v4i{0, 0, 0, 0};

    unsigned p_src[LA];
#pragma unroll
    for (int j = 0; j < LA; j++) {
        const int blk = j * NWG + wg;
        const int slot = blk * 64 + lane;
        const int px = slot / 5;
        const int piece = slot - px * 5;
        const int gp = first + px;
        const bool ok = blk < PLOADS && piece < 4;   // (outside the batch: out of range, as above)
        p_src[j] = ok ? (unsigned)gp * CIN + piece * 16 : FF_OOB;      // (mod 2^32)
    }
    // run r of this group is channel run g + KG*r
    auto issue_patch = [&](int r, int buf) {
        const int c = g + KG * r;
#pragma unroll
        for (int j = 0; j < LA; j++) {
            const int blk = j * NWG + wg;
            bdma16(r_in, p_src[j], (unsigned)(c * DMA_KB), gbase + (blk < PLOADS ? buf * PBUF + blk * 1024 : ZERO_OFF));
        }
    };
    int b_off[B_LD];
#pragma unroll
    for (int j = 0; j < B_LD; j++) {
        const int line = (j * NWG + wg) * 4 + (lane >> 4);
        const int sl = (lane & 15) ^ (line & 3);
        const int n = line * 4 + (sl >> 2);
        b_off[j] = (tn * BN + n) * FF_KSTEP + (sl & 3) * 16;
    }
    const bool loads_b = !B_PART || wg < BW;
    auto issue_b = [&](int r, int t, int slot) {
        if (!loads_b) return;
        const int c = g + KG * r;
        const unsigned wst = (unsigned)((t * CSTEPS + c) * COUT * FF_KSTEP);
#pragma unroll
        for (int j = 0; j < B_LD; j++)
            bdma16(r_w, (unsigned)b_off[j], wst, gbase + NPB * PBUF + slot * B_BYTES + (j * NWG + wg) * 1024);
    };

    const int wm = wg / WN;
    const int wn = wg % WN;
    int a_base[MI], a_edge[MI];
#pragma unroll
    for (int i = 0; i < MI; i++) {
        const int rr0 = wm * MI * 32 + i * 32 + (lane & 31);
        const int m = m0 + rr0;
        const int rr = m % (H * W);
        const int oh = rr / W;
        const int ow = rr - oh * W;
        a_edge[i] = (oh == 0 ? 1 : 0) | (oh == H - 1 ? 2 : 0) | (ow == 0 ? 4 : 0) | (ow == W - 1 ? 8 : 0);
        a_base[i] = g * GROUP_BYTES + rr0 * PATCH_PITCH + (lane >> 5) * 16;   // (absolute LDS offsets)
    }
    const int z_addr = g * GROUP_BYTES + ZERO_OFF + (lane >> 5) * 16;
    const int b_rd = g * GROUP_BYTES + NPB * PBUF + dma_slot(wn * NJ * 32 + (lane & 31), lane >> 5);
    // LDS address of every tap of every row tile, selected once
    int ta[9][MI];
#pragma unroll
    for (int i = 0; i < MI; i++) {
        // (four lane masks per row tile; a tap's mask is the OR of at most two)
        const bool top = a_edge[i] & 1, bot = a_edge[i] & 2, left = a_edge[i] & 4, right = a_edge[i] & 8;
#pragma unroll
        for (int t = 0; t < 9; t++) {
            const int kh = t / 3, kw = t % 3;
            const bool masked = (kh == 0 && top) || (kh == 2 && bot) || (kw == 0 && left) || (kw == 2 && right);
            ta[t][i] = masked ? z_addr : a_base[i] + (kh * W + kw) * PATCH_PITCH;
        }
    }

    v16i acc[MI][NJ];
#pragma unroll
    for (int i = 0; i < MI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

    // the epilogue's per-channel parameters (columns of the blocks this
    // group owns), loaded now so that their latency hides behind the main loop
    const int k0 = g * TO;                                   // first owned block
    const int i0 = k0 / NJ, j0 = k0 % NJ;
    const int ncol = wn * NJ * 32 + j0 * 32;
    EpiParams<NO> prm{};
    if (!a.out_i32) prm = load_epi_params<COUT, NO>(a, tn * BN + ncol);

    // prologue: run 0's patch, then the weights of steps 0 .. D-1
    issue_patch(0, 0);
    s2::static_for<0, (D < NSTEP ? D : NSTEP)>([&](auto wc) {
        constexpr int w = decltype(wc)::value;
        issue_b(w / 9, w % 9, w % NSTB);
    });
    s2::static_for<0, NSTEP>([&](auto sc) {
        constexpr int s = decltype(sc)::value;
        constexpr int r = s / 9, t = s % 9;
        if constexpr (s % U == 0) {
            // barrier before steps s .. s+U-1: their weights and their runs'
            // patches have landed
            constexpr int k = s / U;
            if (loads_b) dma_wait_barrier<PLAN.wait[k]>();
            else dma_wait_barrier<PLAN.wait_p[k]>();
            // the weights D steps ahead (into the slots of steps s-U .. s-1),
            // then the next run's patch where one is due
            s2::static_for<0, U>([&](auto ic) {
                constexpr int w = s + D + decltype(ic)::value;
                if constexpr (w < NSTEP) issue_b(w / 9, w % 9, w % NSTB);
            });
            if constexpr (PLAN.pnext[k] >= 0) issue_patch(PLAN.pnext[k], PLAN.pnext[k] & 1);
        }

        constexpr int pbo = (r & 1) * PBUF;
        const int br = b_rd + (s % NSTB) * B_BYTES;
#if FF_PATCH_IGLP
        __builtin_amdgcn_iglp_opt(1);
#endif
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            v4i af[MI], bf[NJ];
#pragma unroll
            for (int i = 0; i < MI; i++)
                af[i] = *reinterpret_cast<const v4i*>(smem + ta[t][i] + pbo + ks * 32);
#pragma unroll
            for (int j = 0; j < NJ; j++) bf[j] = *reinterpret_cast<const v4i*>(smem + ((br + j * 2048) ^ (ks * 32)));
#pragma unroll
            for (int i = 0; i < MI; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    });
    __syncthreads();                       // every wave is done with the patches and rings

    if constexpr (KG > 1) {
        // Block k (owner group o = k / TO) of wave position wg: the partial of
        // group g != o goes to slot ((k - c0)*(KG-1) + (g > o ? g - 1 : g))*NWG
        // + wg of the current chunk [c0, c0 + CHUNK), lane L's 16 ints as four
        // 16-byte pieces q at q*1024 + 16 L (conflict-free); the owner adds
        // the KG - 1 partials.
#pragma unroll
        for (int c0 = 0; c0 < T; c0 += CHUNK) {
#pragma unroll
            for (int k = c0; k < c0 + CHUNK && k < T; k++) {
                const int o = k / TO;
                if (g != o) {
                    const int src = g > o ? g - 1 : g;
                    int8_t* dst = smem + (((k - c0) * (KG - 1) + src) * NWG + wg) * PART + lane * 16;
                    const v16i& v = acc[k / NJ][k % NJ];
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        *reinterpret_cast<v4i*>(dst + q * 1024) = v4i{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
                }
            }
            __syncthreads();
#pragma unroll
            for (int k = c0; k < c0 + CHUNK && k < T; k++) {
                if (g == k / TO) {
                    v16i& v = acc[k / NJ][k % NJ];
#pragma unroll
                    for (int s2 = 0; s2 < KG - 1; s2++) {
                        const int8_t* srcp = smem + (((k - c0) * (KG - 1) + s2) * NWG + wg) * PART + lane * 16;
#pragma unroll
                        for (int q = 0; q < 4; q++) {
                            const v4i pv = *reinterpret_cast<const v4i*>(srcp + q * 1024);
#pragma unroll
                            for (int e = 0; e < 4; e++) v[4 * q + e] += pv[e];
                        }
                    }
                }
            }
            __syncthreads();               // the partial area is free again
        }
    }
    // the owned blocks (all of them when KG == 1) move to the front of the
    // array, so that one epilogue call with a runtime block offset serves
    // every group
    v16i own[MO][NO];
#pragma unroll
    for (int i = 0; i < MO; i++)
#pragma unroll
        for (int j = 0; j < NO; j++) own[i][j] = acc[i][j];
    if constexpr (KG > 1) {
#pragma unroll
        for (int gg = 1; gg < KG; gg++) {
            if (g == gg) {
#pragma unroll
                for (int i = 0; i < MO; i++)
#pragma unroll
                    for (int j = 0; j < NO; j++) {
                        const int k = gg * TO + i * NO + j;
                        own[i][j] = acc[k / NJ][k % NJ];
                    }
            }
        }
    }
    int8_t* Ws = smem + wave * wave_tile_bytes<MO, NO>();
    int8_t* Ls = smem + NW * wave_tile_bytes<MO, NO>();
    if (a.flags & FFK_EPI_BN && !a.out_i32) issue_bn_lut<NW, BN>(Ls, a.bn_lut, tn * BN);
    wave_epilogue_p<COUT, MO, NO, H, W>(own, a, prm, m0 + wm * MI * 32 + i0 * 32, tn * BN + ncol, Ws,
                                        Ls + ncol * FF_LUT_PITCH);
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
//   16, 18, 19, 21  8, 10, 11, 13 with FFK_EPI_FMA_TAIL
constexpr int STEM_EPI_INSC = 6, STEM_EPI_RAW = 7;
// The epilogue's workgroup barrier: the BN table is loaded once and waited
// for before the first tile's patch barrier, and each wave flushes only its
// own staging tile, so the stem needs none.
#ifndef FF_STEM_EPI_SYNC
#define FF_STEM_EPI_SYNC false
#endif

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
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // (uniform: scalar)
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
    // X byte offsets of this lane's two flush chunks: chunk k is the wave's
    // tile row lane/4 + 16k (pixel q = wave*32 + lane/4 + 16k of the tile's
    // 224), 16 bytes at channel 16*(lane%4).  Tile t is rows oh0, oh0 + 1 of
    // face b with t = 56b + oh0/2, so its pixel q is pixel 224t + q of the
    // batch, and with X at even pixels only (FFK_OUT_X_EVEN) pixel q is stored
    // iff q < 112 and q is even, at even-pixel index 56t + q/2.  Offset = a
    // per-lane constant + t * step; chunks not stored start at FF_OOB, which
    // stays out of the tensor's range (a.M * COUT < 2^31) after the step.
    const bool xev = a.flags & FFK_OUT_X_EVEN;
    unsigned xo0[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int q = wave * 32 + (lane >> 2) + 16 * k;
        const unsigned piece = (unsigned)(lane & 3) * 16;
        xo0[k] = !xev ? (unsigned)q * COUT + piece
                      : (q < W && !(q & 1)) ? (unsigned)(q >> 1) * COUT + piece : FF_OOB;
    }
    const unsigned xstep = (xev ? W / 2 : 2 * W) * COUT;

    // The patch of tile t+1 is fetched into registers while tile t runs its
    // MFMAs and epilogue: the loads' latency, not their bytes, bounds this
    // layer.  One thread per patch pixel (4 rows x 114 columns; the first PP
    // - 1 rounds cover every thread, the last the remainder): its three
    // channels, 0 for the zero padding (0 quantizes to 0 for any scale, and
    // the uint8 path marks padding with -1).
    constexpr int NPIX = 4 * PW;
    constexpr int PP = (NPIX + STEM_NT - 1) / STEM_NT;
    float pv[RGB8 ? 1 : PP][3];                      // fp32 faces: the raw values
    int pq[RGB8 ? PP : 1];                           // uint8 pixels: 3 bytes, or -1 for padding
    auto fetch = [&](int t) {
        const int b = t / (H / 2);
        const int oh0 = (t - b * (H / 2)) * 2;
#pragma unroll
        for (int j = 0; j < PP; j++) {
            const int px = tid + j * STEM_NT;
            const int pr = px / PW;
            const int pc = px - pr * PW;
            const int ih = oh0 - 1 + pr;
            const int iw = pc - 1;
            const bool in = px < NPIX && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;
            const size_t off = ((size_t)b * HW + ih * W + iw) * 3;
            // global-space loads: as generic-address (flat) loads, which the
            // compiler emits for a pointer read from the I/O descriptor, they
            // would count against the LDS wait counter, and the patch reads
            // of this tile would wait for the next tile's fetch
            if constexpr (RGB8) {
                const __attribute__((address_space(1))) uint8_t* src =
                    (const __attribute__((address_space(1))) uint8_t*)x + off;
                pq[j] = in ? (int)(src[0] | (src[1] << 8) | (src[2] << 16)) : -1;
            } else {
                const __attribute__((address_space(1))) float* src =
                    (const __attribute__((address_space(1))) float*)x + off;
#pragma unroll
                for (int c = 0; c < 3; c++) pv[j][c] = in ? src[c] : 0.0f;
            }
        }
    };
    if (t_beg < t_end) fetch(t_beg);

    for (int t = t_beg; t < t_end; t++) {
        const int b = t / (H / 2);
        const int oh0 = (t - b * (H / 2)) * 2;
        const int m0 = b * HW + oh0 * W;
        // the previous tile is done with the patch (a second patch buffer
        // instead of this barrier measured 7 % slower)
        __syncthreads();

        // input rows oh0-1 .. oh0+2, columns -1 .. 112: each pixel's three
        // channels quantized (fp32 faces) or mapped through the table (uint8),
        // with a zero fourth byte, as one dword
#pragma unroll
        for (int j = 0; j < PP; j++) {
            const int px = tid + j * STEM_NT;
            if (px < NPIX) {
                uint32_t packed = 0;
                if constexpr (RGB8) {
                    if (pq[j] >= 0)
#pragma unroll
                        for (int c = 0; c < 3; c++)
                            packed |= (uint32_t)(uint8_t)a.in_lut[c * 256 + ((pq[j] >> (8 * c)) & 255)] << (8 * c);
                } else {
                    const float inv[3] = {inv0, inv1, inv2};
                    float r[3];
                    bool fast = true;
#pragma unroll
                    for (int c = 0; c < 3; c++) {
                        r[c] = __builtin_rintf(pv[j][c] * inv[c]);
                        fast = fast && __builtin_fabsf(r[c]) < 2147483648.0f;
                    }
                    // every value of the wave in int32 range (real faces): the
                    // conversion is the clamp; otherwise the exact lrintf rule
                    if (__all(fast)) {
#pragma unroll
                        for (int c = 0; c < 3; c++)
                            packed |= (uint32_t)(uint8_t)(int)__builtin_amdgcn_fmed3f(r[c], -128.0f, 127.0f) << (8 * c);
                    } else {
#pragma unroll
                        for (int c = 0; c < 3; c++)
                            packed |= (uint32_t)(uint8_t)ff::quant_input(pv[j][c], inv[c]) << (8 * c);
                    }
                }
                reinterpret_cast<uint32_t*>(Ps)[px] = packed;
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
        else {
            const unsigned xoff[2] = {xo0[0] + (unsigned)t * xstep, xo0[1] + (unsigned)t * xstep};
            wave_epi_i8<COUT, 1, 2, (EPI & 7) % 3, false, ((EPI & 7) >= 3), false, EPI >= 16 ? 2 : (EPI >= 8 ? 1 : 0),
                        H, W, false, FF_STEM_EPI_SYNC, 0, true, true>(acc, a, prm, mw, 0, Ws, Ls, xoff);
        }
    }
}

