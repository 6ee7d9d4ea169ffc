/* ff_host.h -- host-side model formats and launch plan (C99, internal). */
#ifndef FF_HOST_H
#define FF_HOST_H

#include <stddef.h>
#include <stdint.h>

#include "fastface.h"
#include "fastface_kernels.h"

/* op codes of the FFW format (kernels/ffw2_loader.c:27-34) */
enum { FF_OP_CONV = 1, FF_OP_BN = 2, FF_OP_PRELU = 3, FF_OP_ADD = 4, FF_OP_GEMM = 5,
       FF_OP_FLATTEN = 6, FF_OP_SAVE_ID = 7, FF_OP_BLOCK_START = 8 };

typedef struct {
    int type;
    int Cin, Cout, Kh, Kw, stride, pad;
    const int8_t* conv_w;           /* OIHW, points into the mapping */
    const uint8_t* conv_scales;     /* f32[Cout], unaligned, in the mapping */
    const uint8_t* conv_bias;       /* f32[Cout] or NULL (FFW2) */
    int bn_size; const uint8_t* bn_scale; const uint8_t* bn_offset;
    int prelu_size; const uint8_t* prelu_slope;
    uint32_t N, K; const int8_t* gemm_w; const uint8_t* gemm_scales; const uint8_t* gemm_bias;
} FfOp;

typedef struct {
    void* map; size_t size; int version;
    int n_ops; FfOp* ops;
    /* OPSC (libfastface.c:116-129,193-204) */
    float input_scale; float* scales;
    /* OPSC2 (libfastface.c:133-191) */
    int has_v2; int n_in; float* in_scale_pc; float* in_inv_pc;
    uint32_t* pc_len; float** inv_pc; float** scale_pc;
} FfModel;

int  ff_model_load(FfModel* m, const char* ffw_path, const char* opsc_path, const char* opsc2_path);
void ff_model_free(FfModel* m);
float ff_read_f32(const uint8_t* p, int i);

/* ---- launch plan ---- */
#define FF_T_INPUT 0            /* tensor 0: the fp32 faces (quantized by the stem) */

typedef struct {
    int C, H, W;
    int def_step, last_use;     /* -1 when never read */
    int buf;                    /* buffer slot, -1 if none */
    int op;                     /* reference op index after which A holds it */
    int even;                   /* stored at its even-row, even-column pixels
                                   only (FFK_OUT_X_EVEN): every reader is a
                                   1x1 stride-2 conv, run at stride 1 */
} FfTensor;

/* step kinds: a conv (+PReLU | +Add, + BN second output), the FC head, a
 * stand-alone BN / PReLU (per-channel table over t_in), a stand-alone Add
 * (one table over the pairs of t_in and t_add) */
enum { FF_STEP_CONV = 1, FF_STEP_FC = 2, FF_STEP_MAP = 3, FF_STEP_ADD = 4 };

typedef struct {
    int kind;                   /* FF_STEP_*                                  */
    int op_first, op_last;
    int cin, cout, kh, kw, stride, pad, hin, win, hout, wout;
    int t_in, t_add, t_out, t_bn;
    int t_x;                    /* the conv's own output (t_out may drop it) */
    int flags; float in_scale;
    size_t w_off;               /* bytes into the weight arena */
    size_t p_off;               /* floats into the parameter arena */
    size_t lut_off;             /* bytes into the weight arena: BN table (conv),
                                   the map's or the Add's table */
    size_t wino_off;            /* bytes into the weight arena: Winograd-packed
                                   weights, or (size_t)-1 if the layer has none */
    /* fc */
    int fc_n, fc_k; float a_scale; size_t ws_off, bias_off;
} FfStep;

typedef struct {
    int n_steps; FfStep* steps;
    int n_tensors; FfTensor* tensors;
    int8_t* w_host; size_t w_bytes;         /* packed weights, all steps */
    float* p_host; size_t p_floats;         /* parameter blocks, all steps */
    float in_inv[4];                        /* stem input quantization */
    size_t max_face_bytes;                  /* largest int8 tensor per face */
    int n_buffers;                          /* buffer slots after liveness */
    int emb_n;                              /* embedding size */
    char err[256];
} FfPlan;

int  ff_plan_build(const FfModel* m, FfPlan* p);
/* keep_all: one buffer per tensor (debug) */
int  ff_plan_assign_buffers(FfPlan* p, int keep_all);
/* 1 if step s is a 3x3 stride-2 conv whose output only step s + 1 reads, as
 * the residual of its epilogue (a stage's 1x1 shortcut): the two may run as
 * one launch.  Valid after ff_plan_assign_buffers. */
int  ff_plan_pair(const FfPlan* p, int s);
void ff_plan_free(FfPlan* p);

#endif
