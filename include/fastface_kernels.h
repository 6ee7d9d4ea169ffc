/* fastface_kernels.h -- kernel-level C ABI of the MI355X (gfx950) INT8 path.
 *
 * This is the thin layer between the C99 host code (libfastface's create /
 * embed, fastface.h) and the hand-written HIP kernels.  It is exported from
 * libfastface_amd.so so that the parity tests can drive every kernel on its
 * own, and so that a caller with its own buffers can run single layers.
 * Plain C types only: device pointers are `void*`/typed pointers obtained from
 * ffk_malloc, streams/events/graphs are opaque `void*` handles.
 *
 * All functions return FFK_OK (0) or a negative FFK_ERR_* code; the text of
 * the last error of the calling thread is available from ffk_last_error().
 */
#ifndef FASTFACE_KERNELS_H
#define FASTFACE_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FFK_OK              0
#define FFK_ERR_ARG        (-1)
#define FFK_ERR_UNSUPPORTED (-2)
#define FFK_ERR_HIP        (-3)
#define FFK_ERR_NOMEM      (-4)

const char* ffk_last_error(void);

/* ---- device memory, streams, events, graphs ------------------------- */
int   ffk_device_count(void);
void* ffk_malloc(size_t bytes);                 /* NULL on failure */
int   ffk_free(void* dptr);
void* ffk_host_alloc(size_t bytes);             /* pinned host memory */
int   ffk_host_free(void* hptr);
int   ffk_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int   ffk_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int   ffk_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
/* zero-fill with a kernel (safe inside graph capture; 16-byte aligned dst) */
int   ffk_zero(void* dst, size_t bytes, void* stream);
int   ffk_stream_create(void** stream);
int   ffk_stream_destroy(void* stream);
int   ffk_stream_sync(void* stream);            /* NULL: device-wide sync */
int   ffk_event_create(void** event);
int   ffk_event_destroy(void* event);
int   ffk_event_record(void* event, void* stream);
int   ffk_event_sync(void* event);              /* host waits for the event */
/* later work on `stream` waits for `event` (recorded on another stream) */
int   ffk_stream_wait_event(void* stream, void* event);
int   ffk_event_elapsed_ms(void* start, void* stop, float* ms);
int   ffk_graph_begin(void* stream);            /* start stream capture */
int   ffk_graph_end(void* stream, void** graph_exec);
int   ffk_graph_launch(void* graph_exec, void* stream);
int   ffk_graph_destroy(void* graph_exec);

/* ---- I/O descriptor ---------------------------------------------------
 * A captured launch chain reads its input faces (fp32, or uint8 RGB for the
 * FFK_IN_RGB8 chain) and writes its fp32 embeddings through this
 * device-resident pair of pointers, so the same
 * graph serves any caller buffers: update it (ffk_memcpy_h2d, same stream)
 * before the launch. */
typedef struct { const float* in; float* out; } ffk_io;

/* ---- convolution (implicit GEMM on i8 MFMA, fused requant epilogue) ----
 * Replaces, per layer, im2col_nhwc_u8 + fastface_gemm_i8_fused +
 * fused_epilogue_int8 (+ the following in-place bn_prelu_requant_int8 as a
 * second output) of the reference: kernels/conv2d_nhwc.c:150-220,
 * kernels/gemm_int8_v2.c:86-110, kernels/int8_epilogue.c:25-112,253-318.
 */
#define FFK_EPI_PRELU    0x01   /* f = f < 0 ? f*slope : f                   */
#define FFK_EPI_ADD      0x02   /* f = fma(add_src, add_scale, f)            */
#define FFK_EPI_BN       0x04   /* out_bn = BN-requant of the int8 output    */
#define FFK_EPI_BIAS     0x08   /* f = f + bias (FFW3/FFW4 always)           */
#define FFK_EPI_INSCALE  0x10   /* f = f * in_scale before ws (FFW2/FFW3)    */
#define FFK_IN_RGB8      0x20   /* cin == 3: `in` holds uint8 RGB pixels, each
                                   channel quantized through in_lut          */
#define FFK_EPI_PRELU_LE1 0x40  /* with FFK_EPI_PRELU: the caller guarantees
                                   every slope is <= 1 (not NaN) and the
                                   pre-activation value never reaches -inf,
                                   so the kernel may take PReLU as
                                   max(f, f*slope) -- the same values, one
                                   operation fewer (ffk_prelu_le1_ok)        */
#define FFK_OUT_X_EVEN   0x100  /* `out` receives X only at the output pixels
                                   of even row and even column, as int8
                                   [batch, hout/2, wout/2, cout] (hout and
                                   wout even; out_bn stays full size).  The
                                   one reader of a block input that feeds
                                   only a 1x1 stride-2 shortcut reads exactly
                                   these pixels, so it then runs as a 1x1
                                   stride-1 conv over the compact tensor.  No
                                   reference counterpart: the reference
                                   stores the whole tensor. */
#define FFK_EPI_IN_RANGE 0x200  /* the caller guarantees that every requant
                                   value RN(f*inv) is finite and below 2^31 -
                                   128 in magnitude (ffk_requant_in_range), so
                                   the kernel may skip the x86 out-of-range
                                   case (NaN or |r| >= 2^31 -> -128): the same
                                   values, two operations fewer.  Ignored with
                                   FFK_EPI_INSCALE. */
#define FFK_EPI_FMA_TAIL 0x800  /* with FFK_EPI_IN_RANGE, on a launch without
                                   FFK_EPI_ADD or FFK_EPI_INSCALE: the caller
                                   guarantees (ffk_requant_fma_ok) that the
                                   requant's last two roundings,
                                   RN(RN(f*inv) + copysign(0.5, f)), may be
                                   taken as one, fma(f, inv, copysign(0.5, f)),
                                   with the same int8 result for every value
                                   the launch can produce: one operation
                                   fewer.  No reference counterpart. */
#define FFK_SHARED_GPU   0x400  /* launch-choice hint, no effect on the
                                   values: another launch of the same size
                                   runs at the same time (the two halves of a
                                   split chain), so the tiling is chosen for
                                   the two launches' combined grid.  No
                                   reference counterpart. */

/* rows of the per-layer parameter block, each `cout` floats (device) */
enum {
    FFK_P_WS = 0,      /* weight scale                                  */
    FFK_P_BIAS,        /* conv bias                                     */
    FFK_P_SLOPE,       /* PReLU slope                                   */
    FFK_P_ADDSCALE,    /* residual per-channel scale                    */
    FFK_P_INV,         /* 1/(out_scale + 1e-9f)                         */
    FFK_P_BN_SIN,      /* BN input scale (forward scale of the output)  */
    FFK_P_BN_S,        /* BN scale                                      */
    FFK_P_BN_O,        /* BN offset                                     */
    FFK_P_BN_INV,      /* BN 1/(out_scale + 1e-9f)                      */
    FFK_NPARAM
};

typedef struct {
    int batch, cin, cout, kh, kw, stride, pad, hin, win;
    const void*    in;       /* int8 NHWC [batch,hin,win,cin]; cin == 3: fp32
                                faces [batch,112,112,3] quantized on load, or
                                uint8 RGB pixels with FFK_IN_RGB8             */
    const float*   in_inv;   /* cin == 3: 3 per-channel inverse input scales  */
    const ffk_io*  io;       /* cin == 3 and in == NULL: read io->in          */
    const int8_t*  w;        /* packed by ffk_pack_conv_weights               */
    const float*   params;   /* [FFK_NPARAM][cout]                            */
    const int8_t*  add_src;  /* FFK_EPI_ADD: int8 [batch,hout,wout,cout]      */
    const int8_t*  bn_lut;   /* FFK_EPI_BN: [cout][256] from ffk_make_bn_lut  */
    int8_t*        out;      /* int8 output X (FFK_OUT_X_EVEN: its even-row,
                                even-column pixels only), or NULL             */
    int8_t*        out_bn;   /* FFK_EPI_BN: BN(X), or NULL                    */
    int32_t*       out_i32;  /* non-NULL: store raw int32 accumulators only   */
    int            flags;
    float          in_scale;
    /* Optional split-K workspace (device memory) for small batches, where the
     * whole-K tiling would leave most CUs idle: the K reduction of each output
     * tile is shared by several workgroups that exchange int32 partial tiles
     * through it.  Zero-fill it once before its first use; every launch
     * leaves its counter area zero again.  Launches sharing one workspace
     * must be ordered (one stream).  NULL / too small: whole-K tiling. */
    void*          workspace;
    size_t         workspace_bytes;
    const int8_t*  in_lut;   /* FFK_IN_RGB8: [3][256] from ffk_make_rgb8_lut */
} ffk_conv_desc;

/* FFK_ALGO_WINOGRAD (flags): run a 3x3 stride-1 pad-1 layer with
 * cin == cout == 64 at 56x56 or 112x112 as integer Winograd F(2,3)
 * (kernels/winograd_int8_ref.c:36-179: G' = 2G, output = 4 x direct, here
 * divided back exactly) instead of the direct implicit GEMM.  Same int32
 * accumulators and outputs bit for bit; `w` must hold
 * ffk_pack_winograd_weights output; the transformed input stays on chip, so
 * the call needs no workspace.  ffk_conv_variant names it "winograd". */
#define FFK_ALGO_WINOGRAD 0x80
/* 1 if FFK_ALGO_WINOGRAD serves this layer geometry, else 0. */
int    ffk_winograd_supported(int cin, int cout, int kh, int kw, int stride, int pad,
                              int hin, int win);
/* Bytes of the Winograd-packed weights: 16 cells x cout x 2 int8 limbs x cin. */
size_t ffk_winograd_packed_bytes(int cin, int cout);
/* U = G' g G'^T per (cell, co, ci) (winograd_int8_ref.c:36-60) cut into
 * int8 limbs u = 64*u1 + u0 (u0 in [0,63]):
 * packed[((cell*cout + co)*2 + limb)*cin + ci], limb 0 = u1, 1 = u0. */
int    ffk_pack_winograd_weights(const int8_t* w_oihw, int cout, int cin, int8_t* packed);

/* 1 if a conv's parameter block (host memory, [FFK_NPARAM][cout]) allows
 * FFK_EPI_PRELU_LE1 for a reduction of ktotal = kh*kw*cin int8 products:
 * every PReLU slope is <= 1 and not NaN, every weight scale, bias and
 * residual scale is finite, and |acc|*|ws| + |bias| + 128*|add_scale| stays
 * below FLT_MAX for the largest |acc| = ktotal*128*128, so the
 * pre-activation value is never infinite.  Else 0. */
int    ffk_prelu_le1_ok(const float* params, int cout, int ktotal, int with_add);
/* 1 if a conv's parameter block (host memory) allows FFK_EPI_IN_RANGE for
 * a reduction of ktotal = kh*kw*cin int8 products with these epilogue flags
 * (FFK_EPI_PRELU / FFK_EPI_ADD select the rows that take part): every used
 * parameter is finite and (ktotal*128*128*|ws| + |bias| + 128*|add_scale|)
 * * max(1, |slope|) * |inv|, widened for the fp32 roundings, stays below
 * 2^31 - 128.  0 with FFK_EPI_INSCALE. */
int    ffk_requant_in_range(const float* params, int cout, int ktotal, int flags);

/* 1 if a conv's parameter block (host memory) allows FFK_EPI_FMA_TAIL for
 * a reduction of ktotal = kh*kw*cin int8 products with these epilogue flags
 * (FFK_EPI_PRELU selects the slope row; 0 with FFK_EPI_ADD or
 * FFK_EPI_INSCALE, or where ffk_requant_in_range fails).  With f the
 * pre-requant value and p = f*inv exact, one rounding of p + copysign(0.5, p)
 * truncates to another integer than the reference's two roundings only when
 * |p| lies strictly between 1/2 - 2^-25 - 2^-26 and 1/2 - 2^-25: there the
 * reference's first rounding lands on 1/2 - 2^-25 and its second one rounds
 * the tie up to 1 (at every other level the midpoint that separates the
 * two is not a float, and its exact ties round alike).  Per channel (inv
 * positive, slope >= 0): every float f whose product with inv falls in that
 * window is found, and the check fails if the channel's pre-requant value
 * reaches +-f for some accumulator in [-ktotal*128*128, ktotal*128*128]
 * (binary search: that value is monotone in the accumulator, constant for
 * a zero weight scale). */
int    ffk_requant_fma_ok(const float* params, int cout, int ktotal, int flags);

/* 1 if a tuned kernel is compiled for this layer geometry (the IResNet
 * layers at 112x112 input), else 0. */
int    ffk_conv_supported(int cin, int cout, int kh, int kw, int stride, int pad,
                          int hin, int win);
/* 1 if ffk_conv runs this geometry at all: a tuned kernel, or else the
 * generic implicit GEMM that takes any kernel size, stride, padding and
 * channel count (the reference's im2col path takes every shape,
 * kernels/conv2d_nhwc.c:150-220; the same integers and int8 results, at a
 * fraction of the tuned kernels' speed); 0 for an invalid geometry (a size
 * or stride below 1, negative padding, no output pixel). */
int    ffk_conv_runnable(int cin, int cout, int kh, int kw, int stride, int pad,
                         int hin, int win);
/* Bytes of the packed weights and the packing itself (host memory). */
size_t ffk_conv_packed_bytes(int cin, int cout, int kh, int kw);
int    ffk_pack_conv_weights(const int8_t* w_oihw, int cout, int cin, int kh, int kw,
                             int8_t* packed);
/* Workspace bytes ffk_conv would use for this descriptor's geometry and
 * batch (0: it takes the whole-K tiling and needs none); the workspace and
 * workspace_bytes fields are not read. */
size_t ffk_conv_workspace_bytes(const ffk_conv_desc* d);
int    ffk_conv(const ffk_conv_desc* d, void* stream);
/* A block's 3x3 stride-2 conv `c` and its 1x1 shortcut `s` (run at stride 1
 * over the compact block input, FFK_OUT_X_EVEN) whose residual is c's
 * output (s->add_src == c->out), as one launch: the results of
 * ffk_conv(c) then ffk_conv(s), bit for bit, except that c's output is
 * never stored (the caller guarantees nothing else reads it).  The
 * reference runs the two ops one after the other (libfastface.c:312-470,
 * the shortcut's epilogue adding the SAVE_ID'd conv output,
 * kernels/int8_epilogue.c:52-93); the fusion has no counterpart there.
 * Served forms: c with bias only (no PReLU, residual, BN or in-scale), s
 * with the residual add and optionally BN (no PReLU or in-scale), for the
 * stride-2 layers at 112, 56 and 28 pixels, at the batches where c would
 * run as the phase kernel.  Returns 1 when launched
 * (or nothing to do), 0 when the pair is not served (nothing launched, no
 * error set: run the two with ffk_conv), < 0 on an error. */
int    ffk_conv_s2_shortcut(const ffk_conv_desc* c, const ffk_conv_desc* s, void* stream);
/* ffk_conv without a caller workspace and without any allocation: no
 * counterpart in the reference.  For callers that cannot allocate device
 * memory -- code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  The small-batch split-K path takes its workspace from a
 * device array inside the library, FFK_NOALLOC_SCRATCH_BYTES per GPU, held
 * until the process ends (the descriptor's workspace fields are ignored).
 * Every layer the library runs fits it (the split-K grids are capped at its
 * size; larger batches, the Winograd and the generic paths need none); a
 * launch that would need more is rejected with FFK_ERR_ARG.  Every call on one GPU shares that GPU's array: calls that
 * overlap in time on one GPU (other streams, other threads) race and must be
 * ordered by the caller; each launch leaves the array's counter area zero for
 * the next.  Results are bit-identical to ffk_conv's. */
#define FFK_NOALLOC_SCRATCH_BYTES ((size_t)2048 + (size_t)320 * 64 * 64 * 4)
int    ffk_conv_noalloc(const ffk_conv_desc* d, void* stream);
/* Name of the kernel variant ffk_conv would run for this descriptor (its
 * geometry, batch and workspace): "stem", "patch" (3x3 stride-1 layers:
 * input patch staged once per channel run), "patch_kg" (the same with the
 * channel runs shared by K-groups of waves, small grids), "phase" (3x3
 * stride-2 layers as four phase images), "direct" (direct-to-LDS tiles),
 * "staged" / "staged128" (register-staged tiles), "splitk" (64x64 tiles
 * with the K reduction split over workgroups), "tile64" (64x64 tiles, whole
 * K: tiny grids), "winograd", "generic" (any other geometry); NULL when no
 * kernel applies.  No counterpart in the reference: it lets
 * tests and benchmarks name the code path they exercise. */
const char* ffk_conv_variant(const ffk_conv_desc* d);
/* Workgroups that launch would have (host function, no device involved);
 * -1 for the tuned input layer (a persistent grid sized at launch), Winograd
 * or invalid descriptors.  No counterpart in the reference: it lets a
 * launch list be built without a GPU. */
int         ffk_conv_grid(const ffk_conv_desc* d);

/* The BN second output as a table: lut[c*256 + q + 128] is the reference's
 * BN requant (kernels/int8_epilogue.c:273-303 with bn != NULL) of the int8
 * value q for channel c, from the FFK_P_BN_* rows (host function). */
int    ffk_make_bn_lut(const float* s_in, const float* bn_s, const float* bn_o,
                       const float* bn_inv, int cout, int8_t* lut);

/* ---- stand-alone elementwise ops --------------------------------------
 * A BN or PReLU whose input is not a conv's output, and an Add after no conv,
 * run as table lookups over int8 tensors (NHWC, 16-byte aligned).
 *
 * Replaces bn_prelu_requant_int8 (kernels/int8_epilogue.c:253-318, called by
 * libfastface.c:401-424): lut[c*256 + q + 128] is that function's output for
 * the int8 value q in channel c, with in-scale s_in[c], BN scale and offset
 * bn_s[c] / bn_o[c] (both NULL: no BN), PReLU slope[c] (NULL: no PReLU) and
 * output inverse scale inv[c] (host function; the reference's 8-channel
 * vector path, which every channel count that is a multiple of 8 takes). */
int    ffk_make_map_lut(const float* s_in, const float* bn_s, const float* bn_o,
                        const float* slope, const float* inv, int c, int8_t* lut);
/* Replaces add_requant_int8 (kernels/int8_epilogue.c:116-131, called by
 * libfastface.c:429-434): lut[(a + 128)*256 + b + 128] =
 * clamp((int)lrintf(fma(a, a_scale, b*b_scale) * (1/(out_scale + 1e-9f))))
 * as the reference computes it on x86-64 (host function, 65536 bytes). */
int    ffk_make_add_lut(float a_scale, float b_scale, float out_scale, int8_t* lut);
/* out[p*c + ch] = lut[ch*256 + in[p*c + ch] + 128] for n_pix pixels of c
 * channels (c a multiple of 64); `out` may not overlap `in`. */
int    ffk_map_i8(const int8_t* in, int8_t* out, long long n_pix, int c, const int8_t* lut,
                  void* stream);
/* out[i] = lut[(a[i] + 128)*256 + b[i] + 128] for n bytes (a multiple of 16). */
int    ffk_add_i8(const int8_t* a, const int8_t* b, int8_t* out, long long n, const int8_t* lut,
                  void* stream);

/* uint8 RGB input as a table: lut[c*256 + x] is the reference's input
 * quantization (quantize_fp32_nhwc_to_int8_per_channel,
 * kernels/int8_epilogue.c:231-247) of the pixel value its SDKs feed it,
 * (float)x - 127.5f then / 127.5f in fp32 (fastface.py:10, README.md:152),
 * with channel c's inverse scale in_inv[c] (host function). */
int    ffk_make_rgb8_lut(const float* in_inv, int8_t* lut);

/* ---- FC head ----------------------------------------------------------
 * Replaces the XOR-0x80 shift + fastface_gemm_i8_matvec_vnni of the reference
 * (libfastface.c:441-455, kernels/gemm_int8_matvec.c:33-81), batched:
 *   out[b][n] = fma(RN((float)dot(a[b], W[n]) * a_scale), ws[n], bias[n]).
 * a is the activation in the order W's columns are given in (the host permutes
 * the NCHW-flatten order of the reference to NHWC once, at create time). */
typedef struct {
    int batch, n, k;
    const int8_t*  a;        /* [batch][k] int8                               */
    const int8_t*  w;        /* packed by ffk_pack_fc_weights                 */
    const float*   ws;       /* [n] */
    const float*   bias;     /* [n] */
    float          a_scale;
    float*         out;      /* [batch][n] fp32, or NULL: io->out             */
    const ffk_io*  io;
    int            path;     /* 0 auto (the matvec up to 16 faces, the GEMM
                                above; a head other than 25088 -> 512 takes
                                the matvec, 16 faces per launch), 1 matvec,
                                2 MFMA GEMM (25088 -> 512 only)               */
    /* Optional workspace (device memory, zero-filled once, the same rules as
     * ffk_conv_desc.workspace; one workspace can serve both): the MFMA GEMM
     * path then shares each output tile's K reduction among several
     * workgroups, which fills the GPU at a few thousand faces.  NULL or too
     * small: one workgroup per output tile. */
    void*          workspace;
    size_t         workspace_bytes;
} ffk_fc_desc;

/* Workspace bytes ffk_fc would use for this descriptor's batch and path
 * (0: none); the workspace fields are not read. */
size_t ffk_fc_workspace_bytes(const ffk_fc_desc* d);
size_t ffk_fc_packed_bytes(int n, int k);
/* Packed FC weights: packed[(s*n + r)*64 + kk] = w_nk[r*k + s*64 + kk]
 * (k a multiple of 64); ffk_pack_fc_row packs row r alone (`row`: its k
 * bytes), so rows can be packed as they are produced, on several threads. */
int    ffk_pack_fc_weights(const int8_t* w_nk, int n, int k, int8_t* packed);
int    ffk_pack_fc_row(const int8_t* row, int n, int k, int r, int8_t* packed);
int    ffk_fc(const ffk_fc_desc* d, void* stream);

/* ---- self checks -------------------------------------------------------
 * Runs one 32x32x32 i8 MFMA on the device with the operand / result lane
 * layouts the conv kernels assume and compares with a host product.
 * Returns FFK_OK when they agree, FFK_ERR_UNSUPPORTED when they differ. */
int ffk_selftest_mfma(void);

#ifdef __cplusplus
}
#endif
#endif /* FASTFACE_KERNELS_H */
