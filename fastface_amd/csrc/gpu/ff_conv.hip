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
// Workgroup = 4 wave64s computing a BM x BN tile (each wave a 64x64 block of
// 2x2 MFMA 32x32 tiles).  Per K step of 64 bytes each thread fetches 16-byte
// pieces of the implicit im2col rows (one input pixel's channel run, zero for
// padding) and of the packed weights, stages them through a double-buffered
// LDS tile (80-byte row pitch: conflict-free ds_read_b128 of MFMA operands),
// and the next step's global loads are in flight while MFMAs run.  After the
// K loop the int32 tile goes through LDS once more so that every thread
// requantizes 16 consecutive channels of one pixel and writes them with one
// 16-byte store (plus one for the BN second output).
#include "ff_internal.h"
#include "ff_numerics.h"

#define EPI_FC 0x100  // internal: FC head, fp32 output via ff::fc_out

// K steps of global loads kept in flight per thread
#ifndef FF_PF
#define FF_PF 4
#endif

struct ConvArgs {
    const int8_t* in;
    const float* in_f32;
    const float* in_inv;
    const ffk_io* io;
    const int8_t* w;
    const float* params;
    const int8_t* add_src;
    int8_t* out;
    int8_t* out_bn;
    int32_t* out_i32;
    float* out_f32;
    const float* fc_ws;
    const float* fc_bias;
    int M;
    int flags;
    float in_scale;
    int tiles_n;
};

// ---------------------------------------------------------------------------
// Epilogue: C tile (int32, LDS, row pitch BN+8) -> int8 / fp32 / int32 HBM.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void load16f(float (&d)[16], const float* p) {
    const float4* q = reinterpret_cast<const float4*>(p);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float4 v = q[i];
        d[4 * i + 0] = v.x; d[4 * i + 1] = v.y; d[4 * i + 2] = v.z; d[4 * i + 3] = v.w;
    }
}

template <int BM, int BN, int COUT, bool PRELU, bool ADD, bool BN2>
__device__ __forceinline__ void epi_requant(const int32_t* Cs, const ConvArgs& a, int m0, int nt0) {
    constexpr int CST = BN + 8;
    constexpr int GROUPS = BN / 16;
    constexpr int RSTEP = 256 / GROUPS;
    const int tid = threadIdx.x;
    const int cg = tid % GROUPS;
    const int n0 = nt0 + cg * 16;
    const bool inscale = (a.flags & FFK_EPI_INSCALE) != 0;
    const float in_scale = a.in_scale;
    float ws[16], bias[16], p2[16], inv[16];
    float bsin[16], bs[16], bo[16], binv[16];
    load16f(ws, a.params + FFK_P_WS * COUT + n0);
    load16f(bias, a.params + FFK_P_BIAS * COUT + n0);
    load16f(inv, a.params + FFK_P_INV * COUT + n0);
    if (PRELU) load16f(p2, a.params + FFK_P_SLOPE * COUT + n0);
    float adds[16];
    if (ADD) load16f(adds, a.params + FFK_P_ADDSCALE * COUT + n0);
    if (BN2) {
        load16f(bsin, a.params + FFK_P_BN_SIN * COUT + n0);
        load16f(bs, a.params + FFK_P_BN_S * COUT + n0);
        load16f(bo, a.params + FFK_P_BN_O * COUT + n0);
        load16f(binv, a.params + FFK_P_BN_INV * COUT + n0);
    }
    for (int row = tid / GROUPS; row < BM; row += RSTEP) {
        const int m = m0 + row;
        if (m >= a.M) break;
        int32_t acc[16];
        {
            const v4i* src = reinterpret_cast<const v4i*>(Cs + row * CST + cg * 16);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                v4i v = src[i];
                acc[4 * i] = v.x; acc[4 * i + 1] = v.y; acc[4 * i + 2] = v.z; acc[4 * i + 3] = v.w;
            }
        }
        const size_t off = (size_t)m * COUT + n0;
        v4i addv = {0, 0, 0, 0};
        if (ADD) addv = *reinterpret_cast<const v4i*>(a.add_src + off);
        uint32_t qw[4] = {0, 0, 0, 0}, bw[4] = {0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 16; e++) {
            float f = (float)acc[e];
            if (inscale) f = f * in_scale;
            f = f * ws[e];
            f = f + bias[e];
            if (ADD) {
                int32_t ai = (int32_t)(int8_t)((uint32_t)addv[e >> 2] >> ((e & 3) * 8));
                f = ff::add_residual(f, ai, adds[e]);
            }
            if (PRELU) f = ff::prelu(f, p2[e]);
            const int32_t q = ff::requant_haz(f * inv[e]);
            qw[e >> 2] |= ((uint32_t)q & 0xffu) << ((e & 3) * 8);
            if (BN2) {
                const int32_t q2 = ff::bn_requant(q, bsin[e], bs[e], bo[e], binv[e]);
                bw[e >> 2] |= ((uint32_t)q2 & 0xffu) << ((e & 3) * 8);
            }
        }
        if (a.out) {
            v4i o = {(int)qw[0], (int)qw[1], (int)qw[2], (int)qw[3]};
            *reinterpret_cast<v4i*>(a.out + off) = o;
        }
        if (BN2) {
            v4i o = {(int)bw[0], (int)bw[1], (int)bw[2], (int)bw[3]};
            *reinterpret_cast<v4i*>(a.out_bn + off) = o;
        }
    }
}

template <int BM, int BN, int COUT>
__device__ __forceinline__ void epi_raw_or_fc(const int32_t* Cs, const ConvArgs& a, int m0, int nt0) {
    constexpr int CST = BN + 8;
    constexpr int GROUPS = BN / 16;
    constexpr int RSTEP = 256 / GROUPS;
    const int tid = threadIdx.x;
    const int cg = tid % GROUPS;
    const int n0 = nt0 + cg * 16;
    if (a.out_i32) {
        for (int row = tid / GROUPS; row < BM; row += RSTEP) {
            const int m = m0 + row;
            if (m >= a.M) break;
            const v4i* src = reinterpret_cast<const v4i*>(Cs + row * CST + cg * 16);
            v4i* dst = reinterpret_cast<v4i*>(a.out_i32 + (size_t)m * COUT + n0);
#pragma unroll
            for (int i = 0; i < 4; i++) dst[i] = src[i];
        }
        return;
    }
    // FC head: out = fma(RN(dot * a_scale), ws, bias), fp32
    float ws[16], bias[16];
    load16f(ws, a.fc_ws + n0);
    load16f(bias, a.fc_bias + n0);
    float* out = a.out_f32 ? a.out_f32 : a.io->out;
    for (int row = tid / GROUPS; row < BM; row += RSTEP) {
        const int m = m0 + row;
        if (m >= a.M) break;
        const int32_t* src = Cs + row * CST + cg * 16;
        float r[16];
#pragma unroll
        for (int e = 0; e < 16; e++) r[e] = ff::fc_out(src[e], a.in_scale, ws[e], bias[e]);
        float4* dst = reinterpret_cast<float4*>(out + (size_t)m * COUT + n0);
#pragma unroll
        for (int i = 0; i < 4; i++) dst[i] = make_float4(r[4 * i], r[4 * i + 1], r[4 * i + 2], r[4 * i + 3]);
    }
}

template <int BM, int BN, int COUT>
__device__ __forceinline__ void tile_epilogue(const int32_t* Cs, const ConvArgs& a, int m0, int nt0) {
    if (a.out_i32 || (a.flags & EPI_FC)) {
        epi_raw_or_fc<BM, BN, COUT>(Cs, a, m0, nt0);
        return;
    }
    switch (a.flags & (FFK_EPI_PRELU | FFK_EPI_ADD | FFK_EPI_BN)) {
    case 0: epi_requant<BM, BN, COUT, false, false, false>(Cs, a, m0, nt0); break;
    case FFK_EPI_PRELU: epi_requant<BM, BN, COUT, true, false, false>(Cs, a, m0, nt0); break;
    case FFK_EPI_ADD: epi_requant<BM, BN, COUT, false, true, false>(Cs, a, m0, nt0); break;
    case FFK_EPI_BN: epi_requant<BM, BN, COUT, false, false, true>(Cs, a, m0, nt0); break;
    case FFK_EPI_PRELU | FFK_EPI_BN: epi_requant<BM, BN, COUT, true, false, true>(Cs, a, m0, nt0); break;
    case FFK_EPI_ADD | FFK_EPI_BN: epi_requant<BM, BN, COUT, false, true, true>(Cs, a, m0, nt0); break;
    case FFK_EPI_PRELU | FFK_EPI_ADD: epi_requant<BM, BN, COUT, true, true, false>(Cs, a, m0, nt0); break;
    default: epi_requant<BM, BN, COUT, true, true, true>(Cs, a, m0, nt0); break;
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
template <int CIN, int COUT, int KS, int STRIDE, int HIN, int WIN, int BM, int BN, int PF>
__global__ __launch_bounds__(256, 2) void conv_i8_kernel(ConvArgs a) {
    constexpr int PAD = KS / 2;
    constexpr int HOUT = (HIN + 2 * PAD - KS) / STRIDE + 1;
    constexpr int WOUT = (WIN + 2 * PAD - KS) / STRIDE + 1;
    constexpr int HWO = HOUT * WOUT;
    constexpr int CSTEPS = CIN / FF_KSTEP;
    constexpr int KSTEPS = KS * KS * CSTEPS;
    constexpr int ROWB = 80;
    constexpr int A_LD = BM * 4 / 256;
    constexpr int B_LD = BN * 4 / 256;
    constexpr int WN = BN / 64;
    constexpr int LDS_K = 2 * (BM + BN) * ROWB;
    constexpr int LDS_C = BM * (BN + 8) * 4;
    constexpr int LDS = LDS_K > LDS_C ? LDS_K : LDS_C;
    static_assert(CIN % FF_KSTEP == 0, "Cin must be a multiple of 64");
    static_assert((BM / 64) * (BN / 64) == 4, "4 waves of 64x64");
    static_assert(COUT % BN == 0, "Cout must be a multiple of BN");

    __shared__ __align__(16) int8_t smem[LDS];
    int8_t* As = smem;
    int8_t* Bs = smem + 2 * BM * ROWB;

    const int tid = threadIdx.x;
    const int bid = xcd_tile(blockIdx.x, gridDim.x);
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
        const int m = m0 + (idx >> 2);
        const bool ok = m < a.M;
        const int mm = ok ? m : 0;
        const int b = mm / HWO;
        const int r = mm - b * HWO;
        const int oh = r / WOUT;
        const int ow = r - oh * WOUT;
        a_img[j] = a.in + (size_t)b * (HIN * WIN * CIN) + (idx & 3) * 16;
        a_ih0[j] = oh * STRIDE - PAD;
        a_iw0[j] = ow * STRIDE - PAD;
        a_ok[j] = ok;
    }
    const int8_t* wbase = a.w + (size_t)tn * BN * FF_KSTEP + tid * 16;

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
            if (a_ok[j] && (unsigned)ih < (unsigned)HIN && (unsigned)iw < (unsigned)WIN)
                qa[j] = *reinterpret_cast<const v4i*>(a_img[j] + (ih * WIN + iw) * CIN + cs * FF_KSTEP);
            else
                qa[j] = v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < B_LD; j++)
            qb[j] = *reinterpret_cast<const v4i*>(wbase + (size_t)s * COUT * FF_KSTEP + j * 4096);
    };
    auto sstore = [&](int buf, const v4i (&qa)[A_LD], const v4i (&qb)[B_LD]) {
#pragma unroll
        for (int j = 0; j < A_LD; j++) {
            const int idx = tid + j * 256;
            *reinterpret_cast<v4i*>(As + buf * BM * ROWB + (idx >> 2) * ROWB + (idx & 3) * 16) = qa[j];
        }
#pragma unroll
        for (int j = 0; j < B_LD; j++) {
            const int idx = tid + j * 256;
            *reinterpret_cast<v4i*>(Bs + buf * BN * ROWB + (idx >> 2) * ROWB + (idx & 3) * 16) = qb[j];
        }
    };

    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int wm = wave / WN;
    const int wn = wave % WN;
    const int8_t* a_rd = As + (wm * 64 + (lane & 31)) * ROWB + (lane >> 5) * 16;
    const int8_t* b_rd = Bs + (wn * 64 + (lane & 31)) * ROWB + (lane >> 5) * 16;

    v16i acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

    // prologue: steps 0 .. PF-1 in flight, step 0 staged in LDS
#pragma unroll
    for (int u = 0; u < PF; u++)
        if (u < KSTEPS) gload(u, ra[u], rb[u]);
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
                if (s + PF < KSTEPS) gload(s + PF, ra[u], rb[u]);
#pragma unroll
                for (int ks = 0; ks < 2; ks++) {
                    const v4i a0 = *reinterpret_cast<const v4i*>(a_rd + buf * BM * ROWB + ks * 32);
                    const v4i a1 = *reinterpret_cast<const v4i*>(a_rd + buf * BM * ROWB + 32 * ROWB + ks * 32);
                    const v4i b0 = *reinterpret_cast<const v4i*>(b_rd + buf * BN * ROWB + ks * 32);
                    const v4i b1 = *reinterpret_cast<const v4i*>(b_rd + buf * BN * ROWB + 32 * ROWB + ks * 32);
                    acc[0][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b0, acc[0][0], 0, 0, 0);
                    acc[0][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a0, b1, acc[0][1], 0, 0, 0);
                    acc[1][0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b0, acc[1][0], 0, 0, 0);
                    acc[1][1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a1, b1, acc[1][1], 0, 0, 0);
                }
                if (s + 1 < KSTEPS) sstore(buf ^ 1, ra[(u + 1) % PF], rb[(u + 1) % PF]);
                __syncthreads();
            }
        }
    }

    // accumulators -> LDS tile (the loop's last barrier freed the K buffers)
    int32_t* Cs = reinterpret_cast<int32_t*>(smem);
    constexpr int CST = BN + 8;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = wm * 64 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                const int col = wn * 64 + j * 32 + (lane & 31);
                Cs[row * CST + col] = acc[i][j][r];
            }
    __syncthreads();
    tile_epilogue<BM, BN, COUT>(Cs, a, m0, tn * BN);
}

// ---------------------------------------------------------------------------
// Stem: 3 -> 64, 3x3, s1, p1 at 112x112 reading the fp32 faces directly and
// quantizing each tap on load (quantize_fp32_nhwc_to_int8_per_channel fused
// into the conv, int8_epilogue.c:231-247).  K = 27 is padded to one 32-deep
// MFMA; each lane gathers the 16 taps of its K half for its output pixel.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256, 2) void stem_kernel(ConvArgs a) {
    constexpr int BM = 128, BN = 64, COUT = 64, H = 112, W = 112, HW = H * W;
    constexpr int CST = BN + 8;
    __shared__ __align__(16) int32_t Cs[BM * CST];

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int m0 = xcd_tile(blockIdx.x, gridDim.x) * BM;
    const int m = m0 + wave * 32 + (lane & 31);
    const bool ok = m < a.M;
    const int mm = ok ? m : 0;
    const int b = mm / HW;
    const int r = mm - b * HW;
    const int oh = r / W;
    const int ow = r - oh * W;
    const float* x = a.in_f32 ? a.in_f32 : a.io->in;
    const float* img = x + (size_t)b * HW * 3;
    const float inv[3] = {a.in_inv[0], a.in_inv[1], a.in_inv[2]};
    const int g = lane >> 5;

    uint32_t aw[4] = {0, 0, 0, 0};
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const int k = g * 16 + e;
        if (k < 27) {
            const int tap = k / 3;
            const int ci = k - tap * 3;
            const int ih = oh - 1 + tap / 3;
            const int iw = ow - 1 + (tap - (tap / 3) * 3);
            if (ok && (unsigned)ih < (unsigned)H && (unsigned)iw < (unsigned)W) {
                const float v = img[(ih * W + iw) * 3 + ci];
                const float s = ci == 0 ? inv[0] : (ci == 1 ? inv[1] : inv[2]);
                const int32_t q = ff::quant_input(v, s);
                aw[e >> 2] |= ((uint32_t)q & 0xffu) << ((e & 3) * 8);
            }
        }
    }
    const v4i av = {(int)aw[0], (int)aw[1], (int)aw[2], (int)aw[3]};
    const v4i b0 = *reinterpret_cast<const v4i*>(a.w + (lane & 31) * FF_KSTEP + g * 16);
    const v4i b1 = *reinterpret_cast<const v4i*>(a.w + (32 + (lane & 31)) * FF_KSTEP + g * 16);
    v16i zero;
#pragma unroll
    for (int i = 0; i < 16; i++) zero[i] = 0;
    const v16i c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b0, zero, 0, 0, 0);
    const v16i c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, b1, zero, 0, 0, 0);
#pragma unroll
    for (int rr = 0; rr < 16; rr++) {
        const int row = wave * 32 + (rr >> 2) * 8 + (lane >> 5) * 4 + (rr & 3);
        Cs[row * CST + (lane & 31)] = c0[rr];
        Cs[row * CST + 32 + (lane & 31)] = c1[rr];
    }
    __syncthreads();
    tile_epilogue<BM, BN, COUT>(Cs, a, m0, 0);
}

// ---------------------------------------------------------------------------
// Dispatch table over the layer geometries of the IResNet family at 112x112
// (every IResNet-18/34/50/100 conv has one of these shapes).
// ---------------------------------------------------------------------------
namespace {

typedef void (*launch_fn)(const ConvArgs&, int grid, hipStream_t);

template <int CIN, int COUT, int KS, int STRIDE, int HIN, int WIN, int BM, int BN, int PF>
void launch_conv(const ConvArgs& a, int grid, hipStream_t s) {
    hipLaunchKernelGGL((conv_i8_kernel<CIN, COUT, KS, STRIDE, HIN, WIN, BM, BN, PF>), dim3(grid),
                       dim3(256), 0, s, a);
}

void launch_stem(const ConvArgs& a, int grid, hipStream_t s) {
    hipLaunchKernelGGL(stem_kernel, dim3(grid), dim3(256), 0, s, a);
}

struct ConvEntry {
    int cin, cout, ks, stride, hin, win, bm, bn;
    launch_fn fn;
};

#define FF_CONV(CIN, COUT, KS, S, H, BM, BN) \
    {CIN, COUT, KS, S, H, H, BM, BN, &launch_conv<CIN, COUT, KS, S, H, H, BM, BN, FF_PF>}

const ConvEntry kConvTable[] = {
    {3, 64, 3, 1, 112, 112, 128, 64, &launch_stem},
    FF_CONV(64, 64, 3, 1, 112, 256, 64),
    FF_CONV(64, 64, 3, 2, 112, 256, 64),
    FF_CONV(64, 64, 1, 2, 112, 256, 64),
    FF_CONV(64, 64, 3, 1, 56, 256, 64),
    FF_CONV(64, 128, 3, 1, 56, 128, 128),
    FF_CONV(128, 128, 3, 2, 56, 128, 128),
    FF_CONV(64, 128, 1, 2, 56, 128, 128),
    FF_CONV(128, 128, 3, 1, 28, 128, 128),
    FF_CONV(128, 256, 3, 1, 28, 128, 128),
    FF_CONV(256, 256, 3, 2, 28, 128, 128),
    FF_CONV(128, 256, 1, 2, 28, 128, 128),
    FF_CONV(256, 256, 3, 1, 14, 128, 128),
    FF_CONV(256, 512, 3, 1, 14, 128, 128),
    FF_CONV(512, 512, 3, 2, 14, 128, 128),
    FF_CONV(256, 512, 1, 2, 14, 128, 128),
    FF_CONV(512, 512, 3, 1, 7, 128, 128),
};

const ConvEntry* find_conv(int cin, int cout, int kh, int kw, int stride, int pad, int hin, int win) {
    if (kh != kw || pad != kh / 2) return nullptr;
    for (const ConvEntry& e : kConvTable)
        if (e.cin == cin && e.cout == cout && e.ks == kh && e.stride == stride && e.hin == hin &&
            e.win == win)
            return &e;
    return nullptr;
}

}  // namespace

// FC head through the same kernel (a 1x1 "conv" over a 1x1 image with
// Cin = K): M = batch faces, N = 512, K = 25088.
int ffk_fc_gemm_launch(const ffk_fc_desc* d, hipStream_t s) {
    if (d->n != 512 || d->k != 25088) {
        ffk_set_error("fc gemm: unsupported shape n=%s k=%s", "?", "?");
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
    a.flags = EPI_FC;
    a.in_scale = d->a_scale;
    a.tiles_n = 512 / 128;
    const int grid = ((d->batch + 127) / 128) * a.tiles_n;
    hipLaunchKernelGGL((conv_i8_kernel<25088, 512, 1, 1, 1, 1, 128, 128, FF_PF>), dim3(grid), dim3(256),
                       0, s, a);
    return ffk_check_launch("fc gemm launch");
}

extern "C" {

int ffk_conv_supported(int cin, int cout, int kh, int kw, int stride, int pad, int hin, int win) {
    return find_conv(cin, cout, kh, kw, stride, pad, hin, win) != nullptr;
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
    const int hout = (d->hin + 2 * d->pad - d->kh) / d->stride + 1;
    const int wout = (d->win + 2 * d->pad - d->kw) / d->stride + 1;
    const long long M = (long long)d->batch * hout * wout;
    if (M > 0x7fffffffLL) {
        ffk_set_error("conv: batch too large%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    const bool stem = d->cin == 3;
    const bool raw = d->out_i32 != nullptr;
    bool bad = !d->w || (!raw && !d->params) || (stem && !d->in_inv) || (stem && !d->in && !d->io) ||
               (!stem && !d->in);
    if (!raw) {
        if ((d->flags & FFK_EPI_ADD) && !d->add_src) bad = true;
        if ((d->flags & FFK_EPI_BN) && !d->out_bn) bad = true;
        if (!(d->flags & FFK_EPI_BN) && !d->out) bad = true;
    }
    if (bad) {
        ffk_set_error("conv: missing pointer for the requested flags%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    if (M == 0) return FFK_OK;
    ConvArgs a = {};
    if (stem) a.in_f32 = (const float*)d->in;
    else a.in = (const int8_t*)d->in;
    a.in_inv = d->in_inv;
    a.io = d->io;
    a.w = d->w;
    a.params = d->params;
    a.add_src = d->add_src;
    a.out = d->out;
    a.out_bn = d->out_bn;
    a.out_i32 = d->out_i32;
    a.M = (int)M;
    a.flags = d->flags & (FFK_EPI_PRELU | FFK_EPI_ADD | FFK_EPI_BN | FFK_EPI_BIAS | FFK_EPI_INSCALE);
    a.in_scale = d->in_scale;
    a.tiles_n = d->cout / e->bn;
    const int tiles_m = (int)((M + e->bm - 1) / e->bm);
    e->fn(a, tiles_m * a.tiles_n, (hipStream_t)stream);
    return ffk_check_launch("conv launch");
}

}  // extern "C"
