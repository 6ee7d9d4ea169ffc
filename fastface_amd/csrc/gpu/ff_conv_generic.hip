// ff_conv_generic.hip -- any conv geometry the tuned kernel table does not
// hold (the reference's im2col + GEMM path takes every shape:
// kernels/conv2d_nhwc.c:150-220): an implicit GEMM with the geometry in
// registers instead of template parameters.
//
// 64x64 output tiles, four waves of one 32x32x32 i8 MFMA each per 32-byte K
// step; the A operand is gathered byte by byte from the NHWC input (any
// channel count, kernel size, stride and padding; the 3-channel input layer
// quantizes fp32 faces or maps uint8 pixels on the fly), the B operand read
// from the packed weights.  The epilogue is the general form of the tuned
// kernels' per element (in-scale, ws, bias, residual, PReLU, round half away
// with the x86 out-of-range case), then X, its even pixels only or BN(X)
// through the channel's table.  A fallback for correctness: no LDS patch
// reuse, no double buffering.
#include "ff_conv_table.h"
#include "ff_numerics.h"

namespace {

struct GenGeom {
    int cin, cout, kh, kw, stride, pad, hin, win, hout, wout;
    int ktot;       // kh * kw * cin
    int kpad;       // ktot rounded up to whole 64-byte weight steps
};

constexpr int GEN_PITCH = 48;    // LDS row pitch of the staged operands (32 bytes + 16)

__global__ __launch_bounds__(256) void conv_generic_kernel(ConvArgs a, GenGeom g) {
    __shared__ __align__(16) int8_t As[64 * GEN_PITCH];
    __shared__ __align__(16) int8_t Bs[64 * GEN_PITCH];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tiles_n = (g.cout + 63) / 64;
    const long long m0 = (long long)(blockIdx.x / tiles_n) * 64;
    const int n0 = (int)(blockIdx.x % tiles_n) * 64;
    const int hw = g.hout * g.wout;
    const bool stem = g.cin == 3;
    const bool rgb8 = stem && (a.flags & FFK_IN_RGB8);
    const void* x = !stem ? (const void*)a.in : a.in_f32 ? (const void*)a.in_f32 : (const void*)a.io->in;

    // the A row (output pixel) and B row (output channel) this thread stages,
    // eight K bytes of each from byte kq of the step
    const int r = tid >> 2, kq = (tid & 3) * 8;
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

    v16i acc;
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = 0;
    for (int k0 = 0; k0 < g.kpad; k0 += 32) {
        uint32_t word[2] = {0, 0};
        int k = k0 + kq;
        int tap = k / g.cin, ci = k - tap * g.cin;
        for (int e = 0; e < 8; e++, k++) {
            int v = 0;
            if (mrow && k < g.ktot) {
                const int th = tap / g.kw;
                const int ih = ih0 + th, iw = iw0 + (tap - th * g.kw);
                if (ih >= 0 && ih < g.hin && iw >= 0 && iw < g.win) {
                    const size_t off = (((size_t)b * g.hin + ih) * g.win + iw) * g.cin + ci;
                    if (!stem) v = ((const int8_t*)x)[off];
                    else if (rgb8) v = a.in_lut[ci * 256 + ((const uint8_t*)x)[off]];
                    else v = ff::quant_input(((const float*)x)[off], a.in_inv[ci]);
                }
            }
            word[e >> 2] |= (uint32_t)(uint8_t)v << (8 * (e & 3));
            if (++ci == g.cin) { ci = 0; tap++; }
        }
        uint2 wv = {0u, 0u};
        if (ncol < g.cout)
            wv = *reinterpret_cast<const uint2*>(a.w + ((size_t)(k0 >> 6) * g.cout + ncol) * 64 + (k0 & 63) + kq);
        __syncthreads();                                  // the previous step's fragments are read
        *reinterpret_cast<uint2*>(As + r * GEN_PITCH + kq) = make_uint2(word[0], word[1]);
        *reinterpret_cast<uint2*>(Bs + r * GEN_PITCH + kq) = wv;
        __syncthreads();
        const v4i A = *reinterpret_cast<const v4i*>(As + (wr + (lane & 31)) * GEN_PITCH + (lane >> 5) * 16);
        const v4i B = *reinterpret_cast<const v4i*>(Bs + (wc + (lane & 31)) * GEN_PITCH + (lane >> 5) * 16);
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, acc, 0, 0, 0);
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
    hipLaunchKernelGGL(conv_generic_kernel, dim3((unsigned)grid), dim3(256), 0, s, a, g);
    return ffk_check_launch("generic conv launch");
}
