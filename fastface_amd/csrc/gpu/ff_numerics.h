// ff_numerics.h -- device-side int8 requantization arithmetic.
//
// Every function reproduces, bit for bit, the fp32 sequence the reference
// executes on x86 (kernels/int8_epilogue.c, kernels/gemm_int8_matvec.c as
// compiled by gcc -O3 -mavx2 -mfma).  Rules that matter on gfx950:
//   * this file is compiled with -ffp-contract=off; the FMAs the x86 build
//     has (explicit _mm256_fmadd_ps, or GCC contraction) are written here as
//     __builtin_fmaf, everything else is one IEEE rounding per operation;
//   * fp32 denormals are kept (the kernel descriptors carry
//     float_denorm_mode_32 = 3): calibrated scales can be denormal;
//   * x86 cvttps2dq returns INT32_MIN for NaN or |r| >= 2^31, and that value
//     then clamps to -128 -- AMD's v_cvt_i32_f32 saturates instead, so the
//     out-of-range case is handled explicitly.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ff {

// x86 cvttps2dq followed by the [-128, 127] clamp (int8_epilogue.c:84-87).
// Clamping in fp32 first gives the same integers for every finite r below
// 2^31 (the bounds are integers, so truncation commutes with the clamp, and
// r <= -2^31 lands on -128 either way); NaN and r >= 2^31, where cvttps2dq
// returns INT32_MIN, fail the final compare and give -128.
__device__ __forceinline__ int32_t cvtt_clamp_i8(float r) {
    const int32_t q = (int32_t)__builtin_amdgcn_fmed3f(r, -128.0f, 127.0f);
    return r < 2147483648.0f ? q : -128;
}

// Round half away from zero in fp32: t + copysign(0.5, t), one rounding,
// then truncate (int8_epilogue.c:81-84).
__device__ __forceinline__ int32_t requant_haz(float t) {
    float r = t + copysignf(0.5f, t);
    return cvtt_clamp_i8(r);
}

// The same for t known finite with |t| < 2^31 - 128 (FFK_EPI_IN_RANGE): then
// |t| + 0.5 rounds to at most 2^31 - 128 (2^31 - 128 is a float), so
// cvttps2dq is in range and the clamp alone decides.
__device__ __forceinline__ int32_t requant_haz_in_range(float t) {
    float r = t + copysignf(0.5f, t);
    return (int32_t)__builtin_amdgcn_fmed3f(r, -128.0f, 127.0f);
}

// The last two roundings of the in-range requant taken as one (the host
// proves per launch that no value the launch can produce tells them apart:
// ffk_requant_fma_ok, FFK_EPI_FMA_TAIL): r = RN(f*inv + copysign(0.5, f)),
// the clamp and the truncation as above.  sign(f*inv) is sign(f) because
// inv > 0 there.
__device__ __forceinline__ int32_t requant_fma_in_range(float f, float inv) {
    const float r = __builtin_fmaf(f, inv, copysignf(0.5f, f));
    return (int32_t)__builtin_amdgcn_fmed3f(r, -128.0f, 127.0f);
}

// Conv epilogue for one element (int8_epilogue.c:52-93, FFW4 call site
// libfastface.c:389-392):
//   f = RN(RN(RN((float)acc * in_scale) * ws) + bias)
//   f = fma((float)add, add_scale, f)          [residual, GCC-contracted]
//   f = (f < 0) ? RN(f * slope) : f            [PReLU, ordered compare]
//   q = HAZ(RN(f * inv))
template <bool USE_IN_SCALE, bool HAS_BIAS>
__device__ __forceinline__ float conv_dequant(int32_t acc, float in_scale, float ws, float bias) {
    float f = (float)acc;
    if (USE_IN_SCALE) f = f * in_scale;
    f = f * ws;
    if (HAS_BIAS) f = f + bias;
    return f;
}

__device__ __forceinline__ float add_residual(float f, int32_t add_i8, float add_scale) {
    return __builtin_fmaf((float)add_i8, add_scale, f);
}

__device__ __forceinline__ float prelu(float f, float slope) {
    float neg = f * slope;
    return (f < 0.0f) ? neg : f;
}

// The same PReLU in two operations, max(f, RN(f * slope)), for slope <= 1
// and f never +-inf: for f < 0, f * slope >= f and RN is monotone, so the max
// is RN(f * slope); for f >= 0, f * slope <= f, so it is f (a zero may change
// sign, which no later step can tell apart: the int8 result of +-0 is 0);
// for NaN f both operands are NaN.
__device__ __forceinline__ float prelu_le1(float f, float slope) {
    return __builtin_fmaxf(f, f * slope);
}

// BN requant of an int8 value (bn_prelu_requant_int8 with bn != NULL,
// int8_epilogue.c:273-303): f = fma(RN(x * s_in), bn_s, bn_o); HAZ(RN(f*inv)).
__device__ __forceinline__ int32_t bn_requant(int32_t x, float s_in, float bn_s, float bn_o,
                                              float inv) {
    float f = (float)x * s_in;
    f = __builtin_fmaf(f, bn_s, bn_o);
    return requant_haz(f * inv);
}

// Input quantization (quantize_fp32_nhwc_to_int8_per_channel,
// int8_epilogue.c:231-247): q = clamp((int)lrintf(RN(x * inv)), -128, 127).
// glibc lrintf on x86-64 converts to a 64-bit long rounding to nearest even
// (NaN and |v| >= 2^63 give INT64_MIN); the (int) cast keeps the low 32 bits.
__device__ __forceinline__ int32_t quant_input(float x, float inv) {
    float v = x * inv;
    float r = __builtin_rintf(v);                  // RNE, exact for |v| >= 2^23
    int32_t q;
    if (r >= -2147483648.0f && r < 2147483648.0f) {
        q = (int32_t)r;
    } else if (r >= -9223372036854775808.0f && r < 9223372036854775808.0f) {
        q = (int32_t)(uint32_t)(uint64_t)(int64_t)r;   // low 32 bits of the long
    } else {
        q = 0;                                      // low 32 bits of INT64_MIN
    }
    q = q < -128 ? -128 : q;
    q = q > 127 ? 127 : q;
    return q;
}

// FC output (gemm_int8_matvec.c:79, contracted by GCC):
//   out = fma(RN((float)dot * a_scale), ws, bias)
__device__ __forceinline__ float fc_out(int32_t dot, float a_scale, float ws, float bias) {
    float t = (float)dot * a_scale;
    return __builtin_fmaf(t, ws, bias);
}

}  // namespace ff
