/* ff_oracle.h -- CPU restatement of FastFace's INT8 IResNet-50 path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (fastface_amd/) links,
 * loads or calls this code; only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg do, and only as the checker.
 *
 * Every function restates one reference function (file:line into the
 * bauratynov/fastface tree) in plain scalar C99.  Arithmetic order follows
 * the instruction sequence the reference compiles to with its Makefile flags
 * (gcc -O3 -mavx2 -mfma -mavxvnni): single IEEE fp32 roundings except where
 * GCC contracts a multiply-add into an FMA, which is written here as fmaf().
 * Build with -ffp-contract=off so that nothing else is fused.
 */
#ifndef FF_ORACLE_H
#define FF_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* x86 cvttps2dq: truncation, INT32_MIN ("integer indefinite") when the value
 * is NaN or outside [-2^31, 2^31). */
int32_t orc_cvtt_x86(float r);

/* kernels/int8_epilogue.c:231-247 quantize_fp32_nhwc_to_int8_per_channel */
void orc_quant_input_pc(const float* in, int n_pos, int C,
                        const float* inv_pc, int8_t* out);
/* kernels/int8_epilogue.c:218-227 quantize_fp32_nhwc_to_int8 (per-tensor) */
void orc_quant_input_pt(const float* in, int n, float scale, int8_t* out);

/* Exact signed int32 NHWC convolution.  Restates im2col_nhwc_u8 +
 * fastface_gemm_i8_fused (kernels/conv2d_nhwc.c:29-74,150-220,
 * kernels/gemm_int8_v2.c:42-110): (a+128)*w - 128*colsum(w) == a*w exactly,
 * zero padding, K order (kh,kw,ci).  in [B,H,W,Cin], w OIHW [Cout,Cin,KH,KW],
 * out [B*Ho*Wo, Cout]. */
void orc_conv_i32(const int8_t* in, int B, int H, int W, int Cin,
                  const int8_t* w_oihw, int Cout, int KH, int KW,
                  int stride, int pad, int Ho, int Wo, int32_t* out);

/* Integer Winograd F(2,3) for 3x3 s1 p1 convs (kernels/winograd_int8_ref.c:
 * 36-179).  Weight transform u = G' g G'^T with G' = 2G, int16, laid out
 * [16][Cout][Cin] (transform cell i*4+j) as the reference stores it; the conv
 * returns A^T[(G' g G'^T) .* (B^T d B)]A summed over Cin, which is exactly 4x
 * the direct convolution.  H and W even.  in [B,H,W,Cin], out [B,H,W,Cout]. */
void orc_winograd_f23_weights(const int8_t* w_oihw, int Cout, int Cin, int16_t* u);
void orc_conv_winograd_f23(const int8_t* in, int B, int H, int W, int Cin,
                           const int16_t* u, int Cout, int32_t* out);

/* kernels/int8_epilogue.c:25-112 fused_epilogue_int8 (AVX2 body; requires
 * Cout % 8 == 0, which holds for every IResNet-50 layer). */
void orc_fused_epilogue(const int32_t* acc, int n_pos, int Cout,
                        float in_scale, const float* ws, const float* bias,
                        const float* bn_scale, const float* bn_offset,
                        const float* prelu_slope,
                        const int8_t* add_src, float add_scale,
                        const float* add_scale_pc, const float* inv_out_pc,
                        float out_scale, int8_t* out);

/* kernels/int8_epilogue.c:253-318 bn_prelu_requant_int8 (AVX2 body; C%8==0) */
void orc_bn_prelu_requant(const int8_t* in, float in_scale,
                          const float* in_scale_pc,
                          const float* bn_scale, const float* bn_offset,
                          const float* prelu_slope, const float* inv_out_pc,
                          float out_scale, int8_t* out, int n_pos, int C);

/* kernels/int8_epilogue.c:116-131 add_requant_int8 (scalar, lrintf) */
void orc_add_requant(const int8_t* a, float a_scale, const int8_t* b,
                     float b_scale, int8_t* out, float out_scale, int n);

/* XOR-0x80 + kernels/gemm_int8_matvec.c:33-81 for one face:
 * out[n] = fma(RN((float)dot * A_scale), W_scale[n], bias[n]),
 * dot = exact sum_k a[k]*W[n,k].  a is the NCHW-flattened activation. */
void orc_fc(const int8_t* a, const int8_t* W, const float* W_scale,
            const float* bias, float A_scale, float* out, int N, int K);

/* ---------------- model files (FFW2/3/4, OPSC, OPSC2) ---------------- */
enum { ORC_CONV = 1, ORC_BN = 2, ORC_PRELU = 3, ORC_ADD = 4, ORC_GEMM = 5,
       ORC_FLATTEN = 6, ORC_SAVE_ID = 7, ORC_BLOCK_START = 8 };

typedef struct {
    int type;
    int Cin, Cout, Kh, Kw, stride, pad;
    const int8_t* conv_w; const float* conv_scales; const float* conv_bias;
    int bn_size; const float* bn_scale; const float* bn_offset;
    int prelu_size; const float* prelu_slope;
    uint32_t N, K; const int8_t* gemm_w; const float* gemm_scales; const float* gemm_bias;
} OrcOp;

typedef struct OrcModel OrcModel;

/* kernels/ffw2_loader.c:71-159 + libfastface.c:133-204,231-240.
 * Returns NULL on failure (same acceptance rules).  opsc2_path may be NULL. */
OrcModel* orc_model_load(const char* ffw_path, const char* opsc_path,
                         const char* opsc2_path);
void orc_model_free(OrcModel* m);
int orc_model_n_ops(const OrcModel* m);
int orc_model_version(const OrcModel* m);
const OrcOp* orc_model_op(const OrcModel* m, int i);
/* 1/(s+1e-9f) and s for op i of OPSC2 (NULL when absent / length 0). */
const float* orc_model_inv_pc(const OrcModel* m, int i, int* len);
const float* orc_model_scale_pc(const OrcModel* m, int i);
float orc_model_scale(const OrcModel* m, int i);

/* Dump callback: called after op `op_idx` (for a fused Conv+PReLU/Add, with
 * the index of the fused op) with the int8 activation tensor that the
 * reference interpreter holds in `A` at that point ([B, H, W, C] NHWC). */
typedef void (*orc_dump_fn)(void* user, int op_idx, const int8_t* act,
                            int B, int H, int W, int C);

/* The batched interpreter (arcface_forward_int8_batched.c:339-516, which is
 * libfastface.c:312-470 with positions scaled by B).  in: B faces of
 * [112,112,3] fp32, out: [B,512] fp32.  Returns 0 on success. */
int orc_forward(const OrcModel* m, const float* in, int B, float* out,
                orc_dump_fn dump, void* user);

#ifdef __cplusplus
}
#endif
#endif
