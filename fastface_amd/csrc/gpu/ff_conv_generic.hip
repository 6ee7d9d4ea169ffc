// ff_conv_generic.hip -- any conv geometry the tuned kernel table does not
// hold (the reference's im2col + GEMM path takes every shape:
// kernels/conv2d_nhwc.c:150-220): an implicit GEMM with the geometry in
// registers instead of template parameters.
//
// 64x64 output tiles, four waves of two 32x32x32 i8 MFMAs each per 64-byte
// K step; the A operand is gathered from the NHWC input in 16- or 8-byte
// channel runs where the channel count allows, byte by byte otherwise (any
// channel count, kernel size, stride and padding; the 3-channel input layer
// quantizes fp32 faces or maps uint8 pixels on the fly), the B operand read
// from the packed weights.  The epilogue is the general form of the tuned
// kernels' per element (in-scale, ws, bias, residual, PReLU, round half away
// with the x86 out-of-range case), then X, its even pixels only or BN(X)
// through the channel's table.  No LDS reuse of the input patch: each tap's
// run is read from L2 / HBM for every output pixel.
#include "ff_conv_table.h"
#include "ff_numerics.h"

namespace {

struct GenGeom {
    int cin, cout, kh, kw, stride, pad, hin, win, hout, wout;
    int ktot;       // kh * kw * cin
    int kpad;       // ktot rounded up to whole 64-byte weight steps
};

constexpr int GEN_PITCH = 80;    // LDS row pitch of the staged operands (one 64-byte K step + 16)

// The 16 A-operand bytes k .. k+15 of output pixel (b, ih0, iw0) (input
// pixel of tap (0, 0)), k in reduction order (kh*KW + kw)*Cin + ci.
// RUN 16: they are one tap's channel run (Cin % 16 == 0), one 16-byte load;
// RUN 8: two taps' 8-byte runs (Cin % 8 == 0); RUN 0: byte by byte (any Cin,
// and the 3-channel input layer, which quantizes fp32 faces or maps uint8
// pixels).  Padding, rows past the batch and k past K give zeros.
template <int RUN>
__device__ __forceinline__ v4i gather_a(const ConvArgs& a, const GenGeom& g, const void* x, bool mrow, int b,
                                        int ih0, int iw0, int k) {
    v4i v = {0, 0, 0, 0};
    if (!mrow) return v;
    if constexpr (RUN == 16 || RUN == 8) {
#pragma unroll
        for (int h = 0; h < 16 / RUN; h++) {
            const int kk = k + h * RUN;
            if (kk >= g.ktot) continue;
            const int tap = kk / g.cin, ci = kk - tap * g.cin;
            const int th = tap / g.kw;
            const int ih = ih0 + th, iw = iw0 + (tap - th * g.kw);
            if (ih < 0 || ih >= g.hin || iw < 0 || iw >= g.win) continue;
            const int8_t* src = (const int8_t*)x + (((size_t)b * g.hin + ih) * g.win + iw) * g.cin + ci;
            if constexpr (RUN == 16) {
                v = *reinterpret_cast<const v4i*>(src);
            } else {
                const uint2 u = *reinterpret_cast<const uint2*>(src);
                v[2 * h] = (int)u.x;
                v[2 * h + 1] = (int)u.y;
            }
        }
    } else {
        const bool stem = g.cin == 3;
        const bool rgb8 = stem && (a.flags & FFK_IN_RGB8);
        int tap = k / g.cin, ci = k - tap * g.cin;
        for (int e = 0; e < 16; e++, k++) {
            int q = 0;
            if (k < g.ktot) {
                const int th = tap / g.kw;
                const int ih = ih0 + th, iw = iw0 + (tap - th * g.kw);
                if (ih >= 0 && ih < g.hin && iw >= 0 && iw < g.win) {
                    const size_t off = (((size_t)b * g.hin + ih) * g.win + iw) * g.cin + ci;
                    if (!stem) q = ((const int8_t*)x)[off];
                    else if (rgb8) q = a.in_lut[ci * 256 + ((const uint8_t*)x)[off]];
                    else q = ff::quant_input(((const float*)x)[off], a.in_inv[ci]);
                }
            }
            v[e >> 2] |= (int)((uint32_t)(uint8_t)q << (8 * (e & 3)));
            if (++ci == g.cin) { ci = 0; tap++; }
        }
    }
    return v;
}

// 64x64 output tiles of four waves (one 32x32 block each); per 64-byte K
// step every thread stages 16 bytes of one A row (output pixel) and of one B
// row (output channel) in LDS, then each wave runs two 32x32x32 MFMAs; the
// next step's loads are in flight meanwhile.
template <int RUN>
__global__ __launch_bounds__(256) void conv_generic_kernel(ConvArgs a, GenGeom g) {
    __shared__ __align__(16) int8_t As[64 * GEN_PITCH];
    __shared__ __align__(16) int8_t Bs[64 * GEN_PITCH];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tiles_n = (g.cout + 63) / 64;
    const long long m0 = (long long)(blockIdx.x / tiles_n) * 64;
    const int n0 = (int)(blockIdx.x % tiles_n) * 64;
    const int hw = g.hout * g.wout;
    const void* x = g.cin != 3 ? (const void*)a.in : a.in_f32 ? (const void*)a.in_f32 : (const void*)a.io->in;

    const int r = tid >> 2, kq = (tid & 3) * 16;
    const long long m = m0 + r;
    const bool mrow = m < a.M;
    int b = 0, ih0 = 0, iw0 = 0;
    if (mrow) {
        b = (int)(m / hw);
        const int rem = (int)(m - (long long)b * hw);
        const int oh = rem / g.wout;
        ih0 = oh * g.stride - g.pad;
        iw0 = (rem - oh * g.wout) * g.stride - g.pad;
    }
    const int ncol = n0 + r;
    const int wr = (wave >> 1) * 32, wc = (wave & 1) * 32;
    auto load_b = [&](int k0) {
        v4i v = {0, 0, 0, 0};
        if (ncol < g.cout) v = *reinterpret_cast<const v4i*>(a.w + ((size_t)(k0 >> 6) * g.cout + ncol) * 64 + kq);
        return v;
    };

    v16i acc;
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = 0;
    v4i ra = gather_a<RUN>(a, g, x, mrow, b, ih0, iw0, kq);
    v4i rb = load_b(0);
    for (int k0 = 0; k0 < g.kpad; k0 += 64) {
        __syncthreads();                                  // the previous step's fragments are read
        *reinterpret_cast<v4i*>(As + r * GEN_PITCH + kq) = ra;
        *reinterpret_cast<v4i*>(Bs + r * GEN_PITCH + kq) = rb;
        __syncthreads();
        if (k0 + 64 < g.kpad) {
            ra = gather_a<RUN>(a, g, x, mrow, b, ih0, iw0, k0 + 64 + kq);
            rb = load_b(k0 + 64);
        }
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const v4i A = *reinterpret_cast<const v4i*>(As + (wr + (lane & 31)) * GEN_PITCH + h * 32 + (lane >> 5) * 16);
            const v4i B = *reinterpret_cast<const v4i*>(Bs + (wc + (lane & 31)) * GEN_PITCH + h * 32 + (lane >> 5) * 16);
            acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, acc, 0, 0, 0);
        }
    }

    // epilogue: lane owns column wc + lane%32 and 16 rows of the wave's block
    const int n = n0 + wc + (lane & 31);
    if (n >= g.cout) return;
    const int C = g.cout;
    const float* P = a.params;
    const bool raw = a.out_i32 != nullptr;
    float ws = 0.0f, bias = 0.0f, inv = 0.0f, slope = 0.0f, adds = 0.0f;
    if (!raw) {
        ws = P[FFK_P_WS * C + n];
        bias = P[FFK_P_BIAS * C + n];
        inv = P[FFK_P_INV * C + n];
        slope = P[FFK_P_SLOPE * C + n];
        adds = P[FFK_P_ADDSCALE * C + n];
    }
    const bool x_even = (a.flags & FFK_OUT_X_EVEN) != 0;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const long long mm = m0 + wr + (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3);
        if (mm >= a.M) continue;
        const size_t o = (size_t)mm * C + n;
        if (raw) {
            a.out_i32[o] = acc[i];
            continue;
        }
        float f = (float)acc[i];
        if (a.flags & FFK_EPI_INSCALE) f = f * a.in_scale;
        f = f * ws;
        f = f + bias;
        if (a.flags & FFK_EPI_ADD) f = ff::add_residual(f, (int32_t)a.add_src[o], adds);
        if (a.flags & FFK_EPI_PRELU) f = ff::prelu(f, slope);
        const int q = ff::requant_haz(f * inv);
        if (a.out) {
            if (!x_even) {
                a.out[o] = (int8_t)q;
            } else {
                const int bb = (int)(mm / hw);
                const int rem = (int)(mm - (long long)bb * hw);
                const int oh = rem / g.wout, ow = rem - oh * g.wout;
                if (!((oh | ow) & 1))
                    a.out[(((size_t)bb * (g.hout / 2) + (oh >> 1)) * (g.wout / 2) + (ow >> 1)) * C + n] = (int8_t)q;
            }
        }
        if (a.flags & FFK_EPI_BN) a.out_bn[o] = a.bn_lut[n * 256 + q + 128];
    }
}

}  // namespace

// Workgroups of the generic kernel for M output pixels (one per 64x64 tile).
long long ff_conv_generic_grid(long long M, int cout) { return ((M + 63) / 64) * ((cout + 63) / 64); }

int ff_conv_generic_launch(const ConvArgs& a, const ffk_conv_desc* d, hipStream_t s) {
    GenGeom g;
    g.cin = d->cin; g.cout = d->cout; g.kh = d->kh; g.kw = d->kw; g.stride = d->stride; g.pad = d->pad;
    g.hin = d->hin; g.win = d->win;
    g.hout = (d->hin + 2 * d->pad - d->kh) / d->stride + 1;
    g.wout = (d->win + 2 * d->pad - d->kw) / d->stride + 1;
    g.ktot = d->kh * d->kw * d->cin;
    g.kpad = (g.ktot + FF_KSTEP - 1) / FF_KSTEP * FF_KSTEP;
    const long long grid = ff_conv_generic_grid(a.M, d->cout);
    if (grid > 0x7fffffffLL) {
        ffk_set_error("conv: batch too large for the generic kernel%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    const dim3 gd((unsigned)grid), bd(256);
    // channel runs are read as 8- / 16-byte vectors: they need the run's
    // alignment in memory (a tensor base that is not 16-byte aligned takes
    // the byte gather)
    if (d->cin == 3 || d->cin % 8 || ((uintptr_t)d->in & 15))
        hipLaunchKernelGGL(conv_generic_kernel<0>, gd, bd, 0, s, a, g);
    else if (d->cin % 16) hipLaunchKernelGGL(conv_generic_kernel<8>, gd, bd, 0, s, a, g);
    else hipLaunchKernelGGL(conv_generic_kernel<16>, gd, bd, 0, s, a, g);
    return ffk_check_launch("generic conv launch");
}
