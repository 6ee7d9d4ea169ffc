/* fastface.h -- C API of the MI355X-native FastFace INT8 engine.
 *
 * Drop-in for the reference's fastface.h (bauratynov/fastface fastface.h:27-42):
 * same three entry points, same types, same constants, same conventions --
 * create returns NULL on any failure, embed returns 0 on success and non-zero
 * on error, results are bit-identical to the reference's int8 CPU path.
 *
 *     FastFace* ff = fastface_create("models/w600k_r50_ffw4.bin");
 *     float input[FASTFACE_INPUT_N];     // HWC fp32 face, [-1, 1]
 *     float embedding[FASTFACE_OUTPUT_N];
 *     fastface_embed(ff, input, embedding);
 *     fastface_destroy(ff);
 *
 * Side inputs, as in the reference (libfastface.c:236-240): per-op scales are
 * read from "models/op_scales.bin" relative to the working directory
 * (mandatory) and per-channel scales from $OPSC2_PATH or
 * "models/op_scales_v2.bin" (optional).
 *
 * Input layout:  HWC contiguous float32, 3*112*112 = 37632 floats per face.
 * Output layout: raw (not L2-normalized) float32 embedding, 512 per face.
 * Thread-safety: one context per thread (a context owns one HIP stream,
 * device buffers and captured graphs); contexts may run concurrently.
 */
#ifndef FASTFACE_H
#define FASTFACE_H

#include <stdint.h>

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct FastFace FastFace;

/* Reference fastface.h:31.  Loads FFW4 (also FFW3/FFW2) weights, builds the
 * fused launch plan, packs and uploads the weights once.  Any op list the
 * reference's interpreter runs is accepted (convs of any geometry, BN /
 * PReLU / Add with or without a conv before them), except ops on the fp32
 * input faces other than a 3-channel conv, ops after the GEMM head, and a
 * GEMM head whose K is not a multiple of 64 or whose N is not 512; those make
 * create return NULL with a message on stderr. */
FastFace* fastface_create(const char* ffw4_path);

/* Reference fastface.h:35.  One face: 37632 fp32 in, 512 fp32 out. */
int fastface_embed(FastFace* ff, const float* input_hwc, float* out_emb);

/* Reference fastface.h:38. */
void fastface_destroy(FastFace* ff);

#define FASTFACE_INPUT_N  37632   /* 3 * 112 * 112 */
#define FASTFACE_OUTPUT_N 512

/* ---------------- additive extensions (no reference counterpart) --------
 * fastface_create with the scale files named explicitly instead of found
 * relative to the working directory: opsc_path replaces
 * "models/op_scales.bin" (NULL: that default), opsc2_path replaces
 * $OPSC2_PATH / "models/op_scales_v2.bin" (NULL: those defaults).  For
 * callers that must not change the process's working directory (several
 * threads creating contexts).  fastface_create(p) is
 * fastface_create_with_scales(p, NULL, NULL). */
FastFace* fastface_create_with_scales(const char* ffw4_path, const char* opsc_path,
                                      const char* opsc2_path);

/* Batched embedding.  Face i of the batch gives exactly the embedding that
 * fastface_embed gives for face i alone (the reference's own invariant: its
 * batched driver, arcface_forward_int8_batched.c, is bit-identical per face).
 * Host buffers: batch*37632 floats in, batch*512 floats out.  A batch of
 * more than 512 faces streams: a first chunk of 256 faces, then chunks of
 * 768; the copy of the next chunk overlaps the compute of the current one
 * (same results).  The call returns when the embeddings are in out_b512. */
int fastface_embed_batch(FastFace* ff, const float* in_bhwc, int batch, float* out_b512);

/* Device-resident variant: d_in / d_out are device pointers (HBM), the work
 * is enqueued on `stream` (NULL: the context's stream) and not waited for. */
int fastface_embed_batch_device(FastFace* ff, const float* d_in, int batch, float* d_out,
                                void* stream);

/* uint8 RGB input, HWC [112][112][3] per face (batch*37632 bytes): gives
 * exactly the embedding fastface_embed gives for the face its SDKs build
 * from the same pixels, (float)x - 127.5f then / 127.5f (fastface.py:10,
 * README.md:152).  The input layer maps each pixel through a 256-entry table
 * per channel (normalization + the reference's input quantization), so a
 * quarter of the fp32 input bytes cross PCIe and HBM. */
/* (host buffers: batches of more than 512 faces stream in chunks of 512) */
int fastface_embed_batch_rgb8(FastFace* ff, const uint8_t* in_bhwc, int batch, float* out_b512);
int fastface_embed_batch_rgb8_device(FastFace* ff, const uint8_t* d_in, int batch, float* d_out,
                                     void* stream);

/* Pre-allocate device buffers for batches up to max_batch (default: grown on
 * demand; env FASTFACE_MAX_BATCH sets the initial reservation). */
int fastface_reserve(FastFace* ff, int max_batch);

/* The context's HIP stream (hipStream_t). */
void* fastface_stream(FastFace* ff);

/* Convolution algorithm of the 64-channel 3x3 stride-1 layers (stage 1 of
 * IResNet, at 56x56 and 112x112).  The integer Winograd F(2,3) path of the
 * reference (kernels/winograd_int8_ref.c, output 4x the direct conv, divided
 * back exactly) gives the same int32 accumulators, activations and
 * embeddings bit for bit as the direct implicit GEMM; it exists to run
 * those layers both ways, and is slower here (its int8 operand limbs cost
 * more MFMA work than the transform saves).  Returns the number of layers
 * the algorithm now runs, -1 on bad arguments, -2 if the larger workspace
 * cannot be allocated.  Captured launch chains are rebuilt on next use. */
#define FASTFACE_CONV_DIRECT       0
#define FASTFACE_CONV_WINOGRAD_F23 1
int fastface_set_conv_algo(FastFace* ff, int algo);

/* Epilogue forms of the convolutions.  At create time the plan gives a conv
 * launch the shorter requantization forms where its parameters prove them
 * value-identical (PReLU as max(f, f*slope); no x86 out-of-range case).
 * general = 1 launches every conv with the general forms instead (the
 * reference's compare/select PReLU and the cvttps2dq emulation), 0 restores
 * the plan's.  Embeddings are the same bit for bit either way; this exists
 * to measure and check the general forms, which models whose parameters do
 * not qualify run.  Returns the number of conv launches that have a
 * shorter form in the plan, -1 on bad arguments, -2 on allocation failure.
 * Captured launch chains are rebuilt on next use.  (No counterpart in the
 * reference, which has one form.) */
int fastface_set_epilogue_forms(FastFace* ff, int general);

/* Stride-2 blocks as one launch.  The last two convs of a stage's first
 * block (the 3x3 stride-2 conv and the 1x1 shortcut whose epilogue adds its
 * output) run as one kernel where one is compiled for the layer (IResNet
 * stages 1-3) and the batch uses the large-tile kernels
 * (ffk_conv_s2_shortcut): the conv's output stays on chip instead of going
 * through memory.  on = 1 (the default) fuses them, 0 runs them as two
 * launches.  Embeddings are the same bit for bit either way.  Returns the
 * number of such step pairs in the plan, -1 on bad arguments, -2 on
 * allocation failure.  Captured launch chains are rebuilt on next use.  (No
 * counterpart in the reference, which runs the two ops one after the
 * other.) */
int fastface_set_shortcut_fusion(FastFace* ff, int on);

/* ---------------- introspection (tests, bench) ---------------------------- */
typedef struct {
    int kind;                 /* 1 conv, 2 FC, 3 stand-alone BN / PReLU (a
                                 per-channel table), 4 stand-alone Add          */
    int op_first, op_last;    /* reference op indices this launch covers        */
    int cin, cout, kh, kw, stride, pad, hin, win, hout, wout;   /* as launched:
                                 a 1x1 stride-2 shortcut over a tensor stored
                                 at its even pixels runs at stride 1, hin/2  */
    int flags;                /* FFK_EPI_* / FFK_OUT_X_EVEN of the launch       */
    int stores_x;             /* writes the pre-BN tensor                       */
    double ops_per_face;      /* 2 * multiply-accumulates                       */
    double act_bytes_per_face;/* activation bytes read + written, algorithmic   */
    double weight_bytes;      /* packed weight bytes read per launch            */
} fastface_step_info;

int fastface_num_steps(const FastFace* ff);
int fastface_get_step(const FastFace* ff, int step, fastface_step_info* info);

/* Runs the launch chain `reps` times step by step with HIP events between
 * launches (no graph) on the context stream; step_ms[s] receives the mean
 * duration of step s.  The input buffer holds whatever the last embed left. */
int fastface_profile_steps(FastFace* ff, int batch, int reps, float* step_ms);

/* Debug: keep every intermediate tensor in its own buffer (call before the
 * first embed), then read the int8 NHWC tensor the reference interpreter
 * holds after op `op_idx` (a fused Conv+PReLU/Add is keyed by the fused op's
 * index).  Returns the number of bytes, or a negative error. */
int fastface_debug_keep_tensors(FastFace* ff, int on);
long long fastface_debug_read(FastFace* ff, int op_idx, int batch, void* host, size_t bytes);

#ifdef __cplusplus
}
#endif

#endif /* FASTFACE_H */
