// ff_winograd.hip -- integer Winograd F(2,3) for the 64-channel 3x3 stride-1
// convolutions (stage 1 of IResNet at 56x56 and 112x112), exact on i8 MFMA.
//
// The reference's integer Winograd (kernels/winograd_int8_ref.c:36-179) uses
// G' = 2G so that every transform stays integral:
//   V = B^T d B (4x4 input window d), U = G' g G'^T (3x3 filter g),
//   M = sum_ci U (.) V,   Y = A^T M A = 4 x (the direct 3x3 conv, 2x2 outputs)
// with B^T = [1 0 -1 0; 0 1 1 0; 0 -1 1 0; 0 1 0 -1], G' = [2 0 0; 1 1 1;
// 1 -1 1; 0 0 2], A^T = [1 1 1 0; 0 1 -1 -1].  |v| <= 510 and |u| <= 1152 do
// not fit int8, so each operand is cut into two int8 limbs,
//   v = 64*v1 + v0,  u = 64*u1 + u0,  v0, u0 in [0, 63], v1 in [-8, 7],
//   u1 in [-18, 18],
// and  M = 64*(64*sum v1 u1 + sum (v1 u0 + v0 u1)) + sum v0 u0,  all in
// int32 (|M| <= 64*510*1152 < 2^26), evaluated Horner-style on one MFMA
// accumulator: 2 MFMAs, shift, 4 MFMAs, shift, 2 MFMAs per (cell, tile
// block).  Y / 4 is then the direct conv's int32 accumulator exactly, and
// the layer's usual requantization epilogue follows.
//
// Work: 16 cells x K' = 256 per 2x2 output block, i.e. 1024 int8 MACs per
// output and channel against the direct conv's 576 -- the limbs cost more
// than the transform saves, so this path is an exact alternative (BASELINE
// config 5 runs the stage-1 layers both ways), not the default.
//
// One kernel per layer (wino_conv_kernel), per 64-block x 64-channel tile:
// the input transform of the tile's 4x4 windows into LDS, one row of four
// cells at a time (V limbs [cell][block][K'], K' = [v1 of 64 channels | v0
// of 64 channels]), the cell GEMMs on MFMA, the output transform in
// registers, and the fused requant epilogue (PReLU / residual / BN second
// output).  The transformed input, 8x the int8 input, never leaves the CU.
#include <algorithm>

#include "ff_internal.h"
#include "ff_numerics.h"

namespace {

constexpr int WC = 64;              // Cin = Cout of the layers this path serves
constexpr int KP = 2 * WC;          // K' bytes per tile and cell: two limbs
constexpr int LUT_PITCH = 272;      // LDS row pitch of a 256-entry BN table
constexpr int PX_PITCH = 80;        // LDS bytes per output pixel (64 + 16)

__device__ __align__(64) int8_t wg_zero[64];

typedef short s16x16 __attribute__((ext_vector_type(16)));
typedef signed char c16 __attribute__((ext_vector_type(16)));

struct WinoArgs {
    const int8_t* x;          // int8 NHWC input
    const int8_t* U;          // packed weight limbs (ffk_pack_winograd_weights)
    const float* params;      // [FFK_NPARAM][64]
    const int8_t* add_src;
    const int8_t* bn_lut;
    int8_t* out;
    int8_t* out_bn;
    int32_t* out_i32;
    int n_tiles;              // 2x2 output blocks of the launch
    int flags;
    float in_scale;
};

// ---------------------------------------------------------------------------
// Input transform + cell GEMMs + output transform + epilogue.  Workgroup = 8
// waves: wave (wm, wn) takes output blocks t0 + wm*32 .. +31 (MFMA rows) and
// channels wn*32 .. +31 (MFMA columns).  Per row of four cells every thread
// transforms one block's 4x4 window for 16 channels (two of its input rows,
// 16-byte loads that the neighbouring blocks' windows share in L2) into the
// LDS A stage, and the cell row's U limbs (32 KB, contiguous in the packed
// weights) are copied into the LDS B stage; both operands are read from
// there in fragment order: lane (row/column lane%32, K half lane/32) holds
// 16 bytes of each 32-byte K step.  (Reading U straight from global memory
// in every wave cost a quarter of the layer's time: each 32x32 block
// re-read it from L2.)
// ---------------------------------------------------------------------------
constexpr int GW_TILES = 128;     // 2x2 output blocks per workgroup
constexpr int GW_NT = 512;        // threads per workgroup: 8 waves
constexpr int AT[2][4] = {{1, 1, 1, 0}, {0, 1, -1, -1}};

__device__ __forceinline__ v16i mfma(const v4i& a, const v4i& b, const v16i& c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

template <int H, int W, int PRELU, bool ADD>
__device__ __forceinline__ void wino_requant(const v16i (&y)[4], const WinoArgs& a, int8_t* T8, int c,
                                             int row0) {
    const int lane = threadIdx.x & 63;
    const bool insc = (a.flags & FFK_EPI_INSCALE) != 0;
    const float ws = a.params[FFK_P_WS * WC + c];
    const float bias = a.params[FFK_P_BIAS * WC + c];
    const float slope = a.params[FFK_P_SLOPE * WC + c];
    const float adds = a.params[FFK_P_ADDSCALE * WC + c];
    const float inv = a.params[FFK_P_INV * WC + c];
#pragma unroll
    for (int p = 0; p < 4; p++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int row = row0 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
            int8_t* e = T8 + (row * 4 + p) * PX_PITCH + c;
            float f = (float)y[p][r];
            if (insc) f = f * a.in_scale;
            f = f * ws;
            f = f + bias;
            if (ADD) f = ff::add_residual(f, (int32_t)*e, adds);
            if (PRELU == 1) f = ff::prelu(f, slope);
            if (PRELU == 2) f = ff::prelu_le1(f, slope);
            *e = (int8_t)ff::requant_haz(f * inv);
            if (r == 15) asm volatile("" ::: "memory");
        }
}

template <int H, int W>
__global__ __launch_bounds__(GW_NT, 1) void wino_conv_kernel(WinoArgs a) {
    constexpr int TH = H / 2, TW = W / 2;
    // the A operand of one cell row (4 cells x 128 blocks x K' bytes, row
    // pitch AP); the epilogue's byte tile reuses it after the last cell row
    constexpr int AP = KP + 16;
    static_assert(GW_TILES * 4 * PX_PITCH <= 4 * GW_TILES * AP, "the epilogue tile must fit the A stage");
    static_assert(GW_NT == GW_TILES * (WC / 16), "one thread per block and 16 channels");
    __shared__ __align__(16) int8_t As[4 * GW_TILES * AP];
    __shared__ __align__(16) int8_t Bs[4 * WC * AP];     // the B operand of one cell row
    __shared__ __align__(16) int8_t Ls[WC * LUT_PITCH];
    int8_t* T8 = As;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int lc = lane & 31, kh = lane >> 5;
    const int blk0 = blockIdx.x * GW_TILES;
    const int c = wn * 32 + lc;                            // this lane's B column (channel)
    const int8_t* brow = Bs + c * AP + kh * 16;            // ... in a cell of the B stage
    const int8_t* arow = As + (wm * 32 + lc) * AP + kh * 16;   // this lane's A row (block) in a cell

    // input transform: thread (tb, tg) = local block tb, channels 16*tg ..
    const int tb = tid >> 2, tg = tid & 3;
    const int gblk = blk0 + tb;
    const bool tvalid = gblk < a.n_tiles;
    int ib = 0, ty = 0, tx = 0;
    if (tvalid) {
        ib = gblk / (TH * TW);
        const int rr = gblk - ib * (TH * TW);
        ty = rr / TW;
        tx = rr - ty * TW;
    }
    // row r of the 4x4 window (input row 2ty - 1 + r), column j, this thread's
    // 16 channels as int16 (zero outside the image)
    auto win = [&](int r, int j) -> s16x16 {
        const int ih = 2 * ty - 1 + r, iw = 2 * tx - 1 + j;
        const bool in = tvalid && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W;
        const int8_t* src = in ? a.x + ((size_t)(ib * H + ih) * W + iw) * WC + tg * 16 : wg_zero;
        return __builtin_convertvector(*reinterpret_cast<const c16*>(src), s16x16);
    };

    v16i y[4];
#pragma unroll
    for (int p = 0; p < 4; p++)
#pragma unroll
        for (int r = 0; r < 16; r++) y[p][r] = 0;

#pragma unroll
    for (int ci = 0; ci < 4; ci++) {                       // cell row: cells 4ci .. 4ci+3
        // row ci of B^T d: d0 - d2, d1 + d2, d2 - d1, d1 - d3
        s16x16 e[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (ci == 0) e[j] = win(0, j) - win(2, j);
            if (ci == 1) e[j] = win(1, j) + win(2, j);
            if (ci == 2) e[j] = win(2, j) - win(1, j);
            if (ci == 3) e[j] = win(1, j) - win(3, j);
        }
        // columns: (B^T d) B, then the two limbs of each cell into the A stage
        s16x16 v[4];
        v[0] = e[0] - e[2];
        v[1] = e[1] + e[2];
        v[2] = e[2] - e[1];
        v[3] = e[1] - e[3];
        // the cell row's U limbs: 4 cells x 64 channels x K' bytes, contiguous
        // in the packed weights, 64 bytes per thread
        v4i u[4];
        const int8_t* usrc = a.U + (size_t)ci * 4 * WC * KP + (size_t)tid * 64;
#pragma unroll
        for (int q = 0; q < 4; q++) u[q] = *reinterpret_cast<const v4i*>(usrc + q * 16);
        __syncthreads();                                   // the previous cell row's fragments are read
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int byte = tid * 64 + q * 16;            // (cell, channel) row byte / KP, offset % KP
            *reinterpret_cast<v4i*>(Bs + (byte / KP) * AP + byte % KP) = u[q];
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const s16x16 v1 = v[j] >> (short)6;            // floor(v / 64)
            const s16x16 v0 = v[j] & (short)63;            // v - 64*v1
            int8_t* dst = As + (j * GW_TILES + tb) * AP + tg * 16;
            *reinterpret_cast<c16*>(dst) = __builtin_convertvector(v1, c16);
            *reinterpret_cast<c16*>(dst + WC) = __builtin_convertvector(v0, c16);
        }
        __syncthreads();
#pragma unroll
        for (int cj = 0; cj < 4; cj++) {
            const int8_t* ar = arow + cj * GW_TILES * AP;
            const int8_t* bc = brow + cj * WC * AP;
            v4i a1[2], a0[2], b1[2], b0[2];
#pragma unroll
            for (int s = 0; s < 2; s++) {
                a1[s] = *reinterpret_cast<const v4i*>(ar + s * 32);
                a0[s] = *reinterpret_cast<const v4i*>(ar + WC + s * 32);
                b1[s] = *reinterpret_cast<const v4i*>(bc + s * 32);
                b0[s] = *reinterpret_cast<const v4i*>(bc + WC + s * 32);
            }
            v16i m;
#pragma unroll
            for (int r = 0; r < 16; r++) m[r] = 0;
            m = mfma(a1[0], b1[0], m);
            m = mfma(a1[1], b1[1], m);
#pragma unroll
            for (int r = 0; r < 16; r++) m[r] <<= 6;
            m = mfma(a1[0], b0[0], m);
            m = mfma(a1[1], b0[1], m);
            m = mfma(a0[0], b1[0], m);
            m = mfma(a0[1], b1[1], m);
#pragma unroll
            for (int r = 0; r < 16; r++) m[r] <<= 6;
            m = mfma(a0[0], b0[0], m);
            m = mfma(a0[1], b0[1], m);
            // output transform: y(p, q) += A^T[p][ci] A^T[q][cj] M(ci, cj)
#pragma unroll
            for (int p = 0; p < 2; p++)
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const int k = AT[p][ci] * AT[q][cj];
                    if (k == 1) {
#pragma unroll
                        for (int r = 0; r < 16; r++) y[p * 2 + q][r] += m[r];
                    } else if (k == -1) {
#pragma unroll
                        for (int r = 0; r < 16; r++) y[p * 2 + q][r] -= m[r];
                    }
                }
        }
    }
    __syncthreads();                                       // the A stage becomes the epilogue tile
    // Y = 4 x the direct conv, exactly
#pragma unroll
    for (int p = 0; p < 4; p++)
#pragma unroll
        for (int r = 0; r < 16; r++) y[p][r] >>= 2;

    const int row0 = wm * 32;                              // block row of this wave in T8
    // output pixel of block row `row` (slice-relative), 2x2 position p
    auto pix = [&](int blk, int p) -> size_t {
        const int bimg = blk / (TH * TW);
        const int rr = blk - bimg * (TH * TW);
        const int ty = rr / TW, tx = rr - ty * TW;
        return ((size_t)bimg * H + 2 * ty + (p >> 1)) * W + 2 * tx + (p & 1);
    };
    if (a.out_i32) {
#pragma unroll
        for (int p = 0; p < 4; p++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int blk = blk0 + row0 + (r >> 2) * 8 + kh * 4 + (r & 3);
                if (blk < a.n_tiles) a.out_i32[pix(blk, p) * WC + c] = y[p][r];
            }
        return;
    }
    // 16-byte chunks of the block tile: chunk k of block row `row`, output
    // row `pr` (0/1) covers pixels (pr, 0..1) -- 128 contiguous bytes in NHWC
    auto chunk_lds = [&](int row, int pr, int k) { return (row * 4 + pr * 2 + (k >> 2)) * PX_PITCH + (k & 3) * 16; };
    const bool add = (a.flags & FFK_EPI_ADD) != 0;
    const bool bn = (a.flags & FFK_EPI_BN) != 0;
    const bool x_even = (a.flags & FFK_OUT_X_EVEN) != 0;
    if (bn)
        for (int i = tid; i < WC * 16; i += GW_NT)
            *reinterpret_cast<v4i*>(Ls + (i >> 4) * LUT_PITCH + (i & 15) * 16) =
                *reinterpret_cast<const v4i*>(a.bn_lut + (size_t)i * 16);
    if (add)
        for (int i = tid; i < GW_TILES * 2 * 8; i += GW_NT) {
            const int row = i >> 4, pr = (i >> 3) & 1, k = i & 7;
            const int blk = blk0 + row;
            const int8_t* src = blk < a.n_tiles ? a.add_src + pix(blk, pr * 2) * WC + k * 16 : wg_zero;
            *reinterpret_cast<v4i*>(T8 + chunk_lds(row, pr, k)) = *reinterpret_cast<const v4i*>(src);
        }
    __syncthreads();
    const int pf = a.flags & FFK_EPI_PRELU ? (a.flags & FFK_EPI_PRELU_LE1 && !(a.flags & FFK_EPI_INSCALE) ? 2 : 1) : 0;
    if (add) {
        if (pf == 0) wino_requant<H, W, 0, true>(y, a, T8, c, row0);
        else if (pf == 1) wino_requant<H, W, 1, true>(y, a, T8, c, row0);
        else wino_requant<H, W, 2, true>(y, a, T8, c, row0);
    } else {
        if (pf == 0) wino_requant<H, W, 0, false>(y, a, T8, c, row0);
        else if (pf == 1) wino_requant<H, W, 1, false>(y, a, T8, c, row0);
        else wino_requant<H, W, 2, false>(y, a, T8, c, row0);
    }
    __syncthreads();
    for (int i = tid; i < GW_TILES * 2 * 8; i += GW_NT) {
        const int row = i >> 4, pr = (i >> 3) & 1, k = i & 7;
        const int blk = blk0 + row;
        if (blk >= a.n_tiles) continue;
        const size_t off = pix(blk, pr * 2) * WC + k * 16;
        const v4i v = *reinterpret_cast<const v4i*>(T8 + chunk_lds(row, pr, k));
        if (a.out) {
            // FFK_OUT_X_EVEN keeps pixel (0, 0) of each 2x2 block (output row
            // pr = 0, chunks 0-3); the compact tensor's pixel index is `blk`
            if (!x_even) *reinterpret_cast<v4i*>(a.out + off) = v;
            else if (pr == 0 && k < 4) *reinterpret_cast<v4i*>(a.out + (size_t)blk * WC + k * 16) = v;
        }
        if (bn) {
            const int c0 = (k & 3) * 16;                   // first channel of the chunk
            const int8_t* L = Ls + c0 * LUT_PITCH + 128;
            v4i o;
#pragma unroll
            for (int w = 0; w < 4; w++) {
                uint32_t packed = 0;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int q = (int8_t)((uint32_t)v[w] >> (e * 8));
                    packed |= (uint32_t)(uint8_t)L[(w * 4 + e) * LUT_PITCH + q] << (e * 8);
                }
                o[w] = (int)packed;
            }
            *reinterpret_cast<v4i*>(a.out_bn + off) = o;
        }
    }
}

int eligible(const ffk_conv_desc* d) {
    return d && d->cin == WC && d->cout == WC && d->kh == 3 && d->kw == 3 && d->stride == 1 && d->pad == 1 &&
           d->hin == d->win && (d->hin == 56 || d->hin == 112);
}

template <int H, int W>
int launch(const ffk_conv_desc* d, hipStream_t s) {
    WinoArgs a = {};
    a.x = (const int8_t*)d->in;
    a.U = d->w;
    a.params = d->params;
    a.add_src = d->add_src;
    a.bn_lut = d->bn_lut;
    a.out = d->out;                 // FFK_OUT_X_EVEN: the top left pixel of each 2x2 block
    a.out_bn = d->out_bn;
    a.out_i32 = d->out_i32;
    a.n_tiles = d->batch * (H / 2) * (W / 2);
    a.flags = d->flags;
    a.in_scale = d->in_scale;
    hipLaunchKernelGGL((wino_conv_kernel<H, W>), dim3((a.n_tiles + GW_TILES - 1) / GW_TILES), dim3(GW_NT), 0, s, a);
    return ffk_check_launch("winograd conv");
}

}  // namespace

int ffk_winograd_eligible(const ffk_conv_desc* d) { return eligible(d); }

int ffk_winograd_conv(const ffk_conv_desc* d, hipStream_t s) {
    if (!eligible(d)) {
        ffk_set_error("conv: FFK_ALGO_WINOGRAD needs a 3x3 stride-1 64->64 layer at 56x56 or 112x112%s%s",
                      nullptr, nullptr);
        return FFK_ERR_UNSUPPORTED;
    }
    if (d->in == nullptr || (d->flags & FFK_IN_RGB8)) {
        ffk_set_error("conv: FFK_ALGO_WINOGRAD needs an int8 input tensor%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    if ((long long)d->batch * (d->hin / 2) * (d->win / 2) > 0x7fffffffLL - GW_TILES) {
        ffk_set_error("conv: batch too large for the Winograd path%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    return d->hin == 56 ? launch<56, 56>(d, s) : launch<112, 112>(d, s);
}

extern "C" {

int ffk_winograd_supported(int cin, int cout, int kh, int kw, int stride, int pad, int hin, int win) {
    ffk_conv_desc d = {};
    d.cin = cin; d.cout = cout; d.kh = kh; d.kw = kw; d.stride = stride; d.pad = pad; d.hin = hin; d.win = win;
    return eligible(&d);
}

size_t ffk_winograd_packed_bytes(int cin, int cout) {
    return (size_t)16 * (size_t)cout * 2 * (size_t)cin;
}

// U = G' g G'^T per (cell, co, ci) as in winograd_int8_transform_weights_ref
// (kernels/winograd_int8_ref.c:36-60), cut into limbs u = 64*u1 + u0:
// packed[((cell*Cout + co)*2 + limb)*Cin + ci], limb 0 = u1, limb 1 = u0.
int ffk_pack_winograd_weights(const int8_t* w, int cout, int cin, int8_t* packed) {
    if (!w || !packed || cout <= 0 || cin <= 0) {
        ffk_set_error("pack_winograd_weights: bad arguments%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    static const int G2[4][3] = {{2, 0, 0}, {1, 1, 1}, {1, -1, 1}, {0, 0, 2}};
    for (int co = 0; co < cout; co++)
        for (int ci = 0; ci < cin; ci++) {
            const int8_t* g = w + ((size_t)co * cin + ci) * 9;
            int tmp[4][3];
            for (int i = 0; i < 4; i++)
                for (int j = 0; j < 3; j++) {
                    int s = 0;
                    for (int k = 0; k < 3; k++) s += G2[i][k] * g[k * 3 + j];
                    tmp[i][j] = s;
                }
            for (int i = 0; i < 4; i++)
                for (int j = 0; j < 4; j++) {
                    int u = 0;
                    for (int k = 0; k < 3; k++) u += tmp[i][k] * G2[j][k];
                    const int u0 = u & 63;
                    const int u1 = (u - u0) / 64;
                    int8_t* dst = packed + ((size_t)(i * 4 + j) * cout + co) * 2 * cin;
                    dst[ci] = (int8_t)u1;
                    dst[cin + ci] = (int8_t)u0;
                }
        }
    return FFK_OK;
}

}  // extern "C"
