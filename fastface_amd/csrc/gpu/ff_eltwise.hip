// ff_eltwise.hip -- the reference's stand-alone elementwise ops on int8
// activations, for op sequences the conv epilogues cannot absorb: a BN or
// PReLU whose input is not a conv's output (libfastface.c:401-424,
// bn_prelu_requant_int8, kernels/int8_epilogue.c:253-318) and an Add that
// follows no conv (libfastface.c:429-434, add_requant_int8,
// kernels/int8_epilogue.c:116-131).
//
// Both are functions of int8 inputs only, so each becomes a table built on
// the host with the reference's fp32 sequence: a BN / PReLU a 256-entry table
// per channel, an Add (its scales are per tensor) one 256 x 256 table.  The
// kernels stream the tensor through a copy of the table in LDS: HBM-bound
// byte work, no arithmetic on the device.
#include <cmath>

#include "ff_internal.h"

namespace {

constexpr int MAP_CG = 64;                 // channels per workgroup (table slice 16 KB)
constexpr int MAP_PIX = 256 / (MAP_CG / 16);   // pixels per workgroup pass (4 lanes each)

// out[p][c] = lut[c][in[p][c] + 128] over n_pix pixels of C channels
// (C a multiple of 64, both tensors 16-byte aligned).  Workgroup (x, y) takes
// channels 64y .. 64y+63 of pixels x, x + gridDim.x, ... in passes of 64
// pixels; a lane owns 16 consecutive channels of one pixel.
__global__ __launch_bounds__(256) void map_lut_kernel(const int8_t* __restrict__ in, int8_t* __restrict__ out,
                                                      const int8_t* __restrict__ lut, long long n_pix, int C) {
    __shared__ __align__(16) uint8_t tab[MAP_CG * 256];
    const int tid = threadIdx.x;
    const int c0 = blockIdx.y * MAP_CG;
    const v4i* src = reinterpret_cast<const v4i*>(lut + (size_t)c0 * 256);
    for (int i = tid; i < MAP_CG * 256 / 16; i += 256) reinterpret_cast<v4i*>(tab)[i] = src[i];
    __syncthreads();
    const int q = tid & 3;                 // 16-channel chunk of the 64
    const uint8_t* t0 = tab + q * 16 * 256;
    for (long long p = (long long)blockIdx.x * MAP_PIX + (tid >> 2); p < n_pix;
         p += (long long)gridDim.x * MAP_PIX) {
        const size_t off = (size_t)p * C + c0 + q * 16;
        const v4i x = *reinterpret_cast<const v4i*>(in + off);
        v4i y;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const unsigned u = (unsigned)x[w] ^ 0x80808080u;      // bytes + 128
            unsigned r = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const unsigned v = (u >> (8 * b)) & 0xffu;
                r |= (unsigned)t0[(w * 4 + b) * 256 + v] << (8 * b);
            }
            y[w] = (int)r;
        }
        *reinterpret_cast<v4i*>(out + off) = y;
    }
}

// out[i] = lut[(a[i] + 128) * 256 + b[i] + 128] over n bytes (n a multiple
// of 16, all three 16-byte aligned).
__global__ __launch_bounds__(256) void add_lut_kernel(const int8_t* __restrict__ a, const int8_t* __restrict__ b,
                                                      int8_t* __restrict__ out, const int8_t* __restrict__ lut,
                                                      long long n16) {
    __shared__ __align__(16) uint8_t tab[256 * 256];
    const int tid = threadIdx.x;
    const v4i* src = reinterpret_cast<const v4i*>(lut);
    for (int i = tid; i < 256 * 256 / 16; i += 256) reinterpret_cast<v4i*>(tab)[i] = src[i];
    __syncthreads();
    for (long long i = (long long)blockIdx.x * 256 + tid; i < n16; i += (long long)gridDim.x * 256) {
        const v4i x = reinterpret_cast<const v4i*>(a)[i];
        const v4i z = reinterpret_cast<const v4i*>(b)[i];
        v4i y;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const unsigned ua = (unsigned)x[w] ^ 0x80808080u;
            const unsigned ub = (unsigned)z[w] ^ 0x80808080u;
            unsigned r = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const unsigned idx = (((ua >> (8 * k)) & 0xffu) << 8) | ((ub >> (8 * k)) & 0xffu);
                r |= (unsigned)tab[idx] << (8 * k);
            }
            y[w] = (int)r;
        }
        reinterpret_cast<v4i*>(out)[i] = y;
    }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// The reference's final requant of a BN / PReLU value (int8_epilogue.c:290-297):
// t + copysign(0.5, t) in fp32, then cvttps2dq (NaN and |r| >= 2^31 give
// INT32_MIN), then the clamp to int8.
int8_t requant_haz(float t) {
    volatile float r = t + std::copysign(0.5f, t);
    int32_t v;
    if (r >= -2147483648.0f && r < 2147483648.0f) v = (int32_t)r;
    else v = INT32_MIN;
    return (int8_t)(v < -128 ? -128 : (v > 127 ? 127 : v));
}

// (int)lrintf(v) as glibc computes it on x86-64 (int8_epilogue.c:126): round
// to nearest even into a 64-bit long (NaN and values beyond the long range
// give LONG_MIN), then the int conversion keeps the low 32 bits.
int32_t lrintf_low32(float v) {
    if (!(v >= -9223372036854775808.0f && v < 9223372036854775808.0f)) return 0;
    const long long r = (long long)std::nearbyint(v);
    return (int32_t)(uint32_t)(unsigned long long)r;
}

}  // namespace

extern "C" {

int ffk_make_map_lut(const float* s_in, const float* bn_s, const float* bn_o, const float* slope,
                     const float* inv, int c, int8_t* lut) {
    if (!s_in || !inv || !lut || c <= 0 || (!bn_s) != (!bn_o)) {
        ffk_set_error("make_map_lut: bad arguments%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    for (int ch = 0; ch < c; ch++)
        for (int q = -128; q < 128; q++) {
            volatile float f = (float)q * s_in[ch];
            if (bn_s) f = __builtin_fmaf(f, bn_s[ch], bn_o[ch]);
            if (slope) {
                volatile float neg = f * slope[ch];
                if (f < 0.0f) f = neg;
            }
            volatile float t = f * inv[ch];
            lut[(size_t)ch * 256 + (q + 128)] = requant_haz(t);
        }
    return FFK_OK;
}

int ffk_make_add_lut(float a_scale, float b_scale, float out_scale, int8_t* lut) {
    if (!lut) {
        ffk_set_error("make_add_lut: bad arguments%s%s", nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    volatile float den = out_scale + 1e-9f;
    const float inv = 1.0f / den;
    for (int a = -128; a < 128; a++)
        for (int b = -128; b < 128; b++) {
            volatile float pb = (float)b * b_scale;
            volatile float f = __builtin_fmaf((float)a, a_scale, pb);
            volatile float t = f * inv;
            int32_t q = lrintf_low32(t);
            q = q > 127 ? 127 : (q < -128 ? -128 : q);
            lut[(size_t)(a + 128) * 256 + (b + 128)] = (int8_t)q;
        }
    return FFK_OK;
}

int ffk_map_i8(const int8_t* in, int8_t* out, long long n_pix, int c, const int8_t* lut, void* stream) {
    if (!in || !out || !lut || n_pix < 0 || c <= 0 || c % MAP_CG || !aligned16(in) || !aligned16(out) ||
        !aligned16(lut)) {
        ffk_set_error("map_i8: bad arguments (channels a multiple of 64, 16-byte aligned tensors)%s%s",
                      nullptr, nullptr);
        return FFK_ERR_ARG;
    }
    if (n_pix == 0) return FFK_OK;
    const int groups = c / MAP_CG;
    long long gx = (n_pix + MAP_PIX - 1) / MAP_PIX;
    const long long cap = 2048 / groups > 0 ? 2048 / groups : 1;
    if (gx > cap) gx = cap;
    hipLaunchKernelGGL(map_lut_kernel, dim3((unsigned)gx, (unsigned)groups), dim3(256), 0, (hipStream_t)stream,
                       in, out, lut, n_pix, c);
    return ffk_check_launch("map_i8 launch");
}

int ffk_add_i8(const int8_t* a, const int8_t* b, int8_t* out, long long n, const int8_t* lut, void* stream) {
    if (!a || !b || !out || !lut || n < 0 || n % 16 || !aligned16(a) || !aligned16(b) || !aligned16(out) ||
        !aligned16(lut)) {
        ffk_set_error("add_i8: bad arguments (a multiple of 16 bytes, 16-byte aligned tensors)%s%s", nullptr,
                      nullptr);
        return FFK_ERR_ARG;
    }
    if (n == 0) return FFK_OK;
    const long long n16 = n / 16;
    long long g = (n16 + 255) / 256;
    if (g > 1024) g = 1024;
    hipLaunchKernelGGL(add_lut_kernel, dim3((unsigned)g), dim3(256), 0, (hipStream_t)stream, a, b, out, lut, n16);
    return ffk_check_launch("add_i8 launch");
}

}  // extern "C"
