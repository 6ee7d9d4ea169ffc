/* ff_oracle.c -- CPU restatement of FastFace's INT8 IResNet-50 path.
 *
 * TEST INFRASTRUCTURE ONLY (see ff_oracle.h).  Scalar C99 + OpenMP over
 * independent output positions; no cross-thread reductions, so results do
 * not depend on the thread count.
 *
 * Parity pins (what fixes each function, besides reading the reference):
 *   orc_cvtt_x86, orc_fused_epilogue, orc_bn_prelu_requant, orc_quant_input_pc,
 *   orc_fc        -> bit-compared with the reference's own functions compiled
 *                    from its sources (oracle/_ref) on seeded and special-case
 *                    inputs (ties, overflow, NaN, denormal scales, -0).
 *   orc_conv_i32  -> brute-force definition of convolution (tests/) and the
 *                    reference's im2col + VNNI GEMM from oracle/_ref.
 *   orc_forward   -> the reference's fastface_embed / batched binary from
 *                    oracle/_ref on the synthetic FFW4, bit-exact.
 */
#include "ff_oracle.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

int32_t orc_cvtt_x86(float r)
{
    if (r >= -2147483648.0f && r < 2147483648.0f) return (int32_t)r;
    return INT32_MIN;
}

static inline int8_t clamp_i8(int32_t q)
{
    if (q < -128) q = -128;
    if (q > 127) q = 127;
    return (int8_t)q;
}

/* Round half away from zero the way the reference's AVX2 code does it:
 * t + copysign(0.5, t) rounded to fp32, then cvttps2dq, then clamp
 * (kernels/int8_epilogue.c:81-87). */
static inline int8_t haz_requant(float t)
{
    float r = t + copysignf(0.5f, t);
    return clamp_i8(orc_cvtt_x86(r));
}

/* (int)lrintf(v): glibc on x86-64 converts to a 64-bit long with the current
 * (round-to-nearest-even) mode; the int cast keeps the low 32 bits. */
static inline int32_t lrintf_to_int(float v)
{
    return (int32_t)lrintf(v);
}

/* ---- kernels/int8_epilogue.c:231-247 ---------------------------------- */
void orc_quant_input_pc(const float* in, int n_pos, int C,
                        const float* inv_pc, int8_t* out)
{
    #pragma omp parallel for schedule(static) if (n_pos > 4096)
    for (int p = 0; p < n_pos; p++)
        for (int c = 0; c < C; c++) {
            float v = in[(size_t)p * C + c] * inv_pc[c];
            out[(size_t)p * C + c] = clamp_i8(lrintf_to_int(v));
        }
}

/* ---- kernels/int8_epilogue.c:218-227 ---------------------------------- */
void orc_quant_input_pt(const float* in, int n, float scale, int8_t* out)
{
    float inv = 1.0f / (scale + 1e-9f);
    for (int i = 0; i < n; i++) out[i] = clamp_i8(lrintf_to_int(in[i] * inv));
}

/* ---- exact convolution (conv2d_nhwc.c:29-220 + gemm_int8_v2.c:42-110) -- */
void orc_conv_i32(const int8_t* in, int B, int H, int W, int Cin,
                  const int8_t* w_oihw, int Cout, int KH, int KW,
                  int stride, int pad, int Ho, int Wo, int32_t* out)
{
    /* weights regrouped tap-major, output channel innermost */
    size_t K = (size_t)KH * KW * Cin;
    int16_t* wr = (int16_t*)malloc(K * Cout * sizeof(int16_t));
    for (int co = 0; co < Cout; co++)
        for (int ci = 0; ci < Cin; ci++)
            for (int kh = 0; kh < KH; kh++)
                for (int kw = 0; kw < KW; kw++)
                    wr[(((size_t)kh * KW + kw) * Cin + ci) * Cout + co] =
                        w_oihw[(((size_t)co * Cin + ci) * KH + kh) * KW + kw];
    long n_pos = (long)B * Ho * Wo;
    #pragma omp parallel for schedule(static)
    for (long m = 0; m < n_pos; m++) {
        int b = (int)(m / ((long)Ho * Wo));
        int rem = (int)(m % ((long)Ho * Wo));
        int oh = rem / Wo, ow = rem % Wo;
        int32_t* acc = out + (size_t)m * Cout;
        for (int co = 0; co < Cout; co++) acc[co] = 0;
        for (int kh = 0; kh < KH; kh++) {
            int ih = oh * stride - pad + kh;
            if (ih < 0 || ih >= H) continue;
            for (int kw = 0; kw < KW; kw++) {
                int iw = ow * stride - pad + kw;
                if (iw < 0 || iw >= W) continue;
                const int8_t* src = in + (((size_t)b * H + ih) * W + iw) * Cin;
                const int16_t* wt = wr + ((size_t)kh * KW + kw) * Cin * Cout;
                for (int ci = 0; ci < Cin; ci++) {
                    int32_t a = src[ci];
                    if (a == 0) continue;
                    const int16_t* wc = wt + (size_t)ci * Cout;
                    for (int co = 0; co < Cout; co++) acc[co] += a * (int32_t)wc[co];
                }
            }
        }
    }
    free(wr);
}

/* ---- kernels/winograd_int8_ref.c:36-179 -------------------------------- */
/* F(2,3) with G' = 2G keeps every transform in integers:
 *   B^T = [1 0 -1 0; 0 1 1 0; 0 -1 1 0; 0 1 0 -1]
 *   G'  = [2 0 0; 1 1 1; 1 -1 1; 0 0 2]
 *   A^T = [1 1 1 0; 0 1 -1 -1]
 * Written as plain small matrix products (rows x cols), not as the
 * reference's unrolled butterflies. */
static const int WG_BT[4][4] = {{1, 0, -1, 0}, {0, 1, 1, 0}, {0, -1, 1, 0}, {0, 1, 0, -1}};
static const int WG_G2[4][3] = {{2, 0, 0}, {1, 1, 1}, {1, -1, 1}, {0, 0, 2}};
static const int WG_AT[2][4] = {{1, 1, 1, 0}, {0, 1, -1, -1}};

void orc_winograd_f23_weights(const int8_t* w_oihw, int Cout, int Cin, int16_t* u)
{
    for (int co = 0; co < Cout; co++)
        for (int ci = 0; ci < Cin; ci++) {
            const int8_t* g = w_oihw + ((size_t)co * Cin + ci) * 9;
            int t[4][3];                       /* G' g */
            for (int i = 0; i < 4; i++)
                for (int j = 0; j < 3; j++) {
                    int acc = 0;
                    for (int k = 0; k < 3; k++) acc += WG_G2[i][k] * g[k * 3 + j];
                    t[i][j] = acc;
                }
            for (int i = 0; i < 4; i++)        /* (G' g) G'^T */
                for (int j = 0; j < 4; j++) {
                    int acc = 0;
                    for (int k = 0; k < 3; k++) acc += t[i][k] * WG_G2[j][k];
                    u[((size_t)(i * 4 + j) * Cout + co) * Cin + ci] = (int16_t)acc;
                }
        }
}

void orc_conv_winograd_f23(const int8_t* in, int B, int H, int W, int Cin,
                           const int16_t* u, int Cout, int32_t* out)
{
    const int TH = H / 2, TW = W / 2;
    const long n_tiles = (long)B * TH * TW;
    #pragma omp parallel
    {
        int32_t* V = (int32_t*)malloc((size_t)16 * Cin * sizeof(int32_t));
        int64_t* M = (int64_t*)malloc((size_t)16 * Cout * sizeof(int64_t));
        #pragma omp for schedule(static)
        for (long t = 0; t < n_tiles; t++) {
            const int b = (int)(t / ((long)TH * TW));
            const int r = (int)(t % ((long)TH * TW));
            const int oh = (r / TW) * 2, ow = (r % TW) * 2;
            /* V = B^T d B per input channel, d = the 4x4 input window at
             * (oh-1, ow-1) with zero padding */
            for (int ci = 0; ci < Cin; ci++) {
                int d[4][4], e[4][4];
                for (int i = 0; i < 4; i++)
                    for (int j = 0; j < 4; j++) {
                        const int ih = oh - 1 + i, iw = ow - 1 + j;
                        d[i][j] = (ih >= 0 && ih < H && iw >= 0 && iw < W)
                                      ? in[(((size_t)b * H + ih) * W + iw) * Cin + ci] : 0;
                    }
                for (int i = 0; i < 4; i++)
                    for (int j = 0; j < 4; j++) {
                        int acc = 0;
                        for (int k = 0; k < 4; k++) acc += WG_BT[i][k] * d[k][j];
                        e[i][j] = acc;
                    }
                for (int i = 0; i < 4; i++)
                    for (int j = 0; j < 4; j++) {
                        int acc = 0;
                        for (int k = 0; k < 4; k++) acc += e[i][k] * WG_BT[j][k];
                        V[(i * 4 + j) * Cin + ci] = acc;
                    }
            }
            /* M[cell][co] = sum_ci U[cell][co][ci] * V[cell][ci] (64-bit here;
             * the reference's int32 sums cannot overflow: |u|<=1152, |v|<=512) */
            for (int c = 0; c < 16; c++)
                for (int co = 0; co < Cout; co++) {
                    const int16_t* uc = u + ((size_t)c * Cout + co) * Cin;
                    const int32_t* vc = V + (size_t)c * Cin;
                    int64_t acc = 0;
                    for (int ci = 0; ci < Cin; ci++) acc += (int64_t)uc[ci] * vc[ci];
                    M[(size_t)c * Cout + co] = acc;
                }
            /* Y = A^T M A per output channel */
            for (int co = 0; co < Cout; co++)
                for (int i = 0; i < 2; i++)
                    for (int j = 0; j < 2; j++) {
                        int64_t acc = 0;
                        for (int p = 0; p < 4; p++)
                            for (int q = 0; q < 4; q++)
                                acc += (int64_t)WG_AT[i][p] * WG_AT[j][q] * M[(size_t)(p * 4 + q) * Cout + co];
                        out[(((size_t)b * H + oh + i) * W + ow + j) * Cout + co] = (int32_t)acc;
                    }
        }
        free(V);
        free(M);
    }
}

/* ---- kernels/int8_epilogue.c:25-112 ----------------------------------- */
void orc_fused_epilogue(const int32_t* acc, int n_pos, int Cout,
                        float in_scale, const float* ws, const float* bias,
                        const float* bn_scale, const float* bn_offset,
                        const float* prelu_slope,
                        const int8_t* add_src, float add_scale,
                        const float* add_scale_pc, const float* inv_out_pc,
                        float out_scale, int8_t* out)
{
    float inv_scalar = 1.0f / (out_scale + 1e-9f);
    int vec_end = Cout & ~7;
    #pragma omp parallel for schedule(static)
    for (int p = 0; p < n_pos; p++) {
        const int32_t* a_row = acc + (size_t)p * Cout;
        const int8_t* add_row = add_src ? add_src + (size_t)p * Cout : NULL;
        int8_t* o_row = out + (size_t)p * Cout;
        /* 8-wide AVX2 body: separately rounded mul, mul, add; the residual
         * product is contracted into an FMA by GCC; explicit BN FMA. */
        for (int co = 0; co < vec_end; co++) {
            float f = (float)a_row[co];
            f = f * in_scale;
            f = f * ws[co];
            if (bias) f = f + bias[co];
            if (add_row) {
                float as = add_scale_pc ? add_scale_pc[co] : add_scale;
                f = fmaf((float)add_row[co], as, f);
            }
            if (bn_scale) f = fmaf(f, bn_scale[co], bn_offset[co]);
            if (prelu_slope) {
                float neg = f * prelu_slope[co];
                if (f < 0.0f) f = neg;          /* _CMP_LT_OS: NaN, -0 keep f */
            }
            float inv = inv_out_pc ? inv_out_pc[co] : inv_scalar;
            o_row[co] = haz_requant(f * inv);
        }
        /* scalar tail (Cout % 8 != 0): never reached by IResNet-50, whose
         * channel counts are multiples of 8 -- parity unpinned. */
        for (int co = vec_end; co < Cout; co++) {
            float f = (float)a_row[co] * (in_scale * ws[co]);
            if (bias) f = f + bias[co];
            if (add_row) {
                float as = add_scale_pc ? add_scale_pc[co] : add_scale;
                f = f + (float)add_row[co] * as;
            }
            if (bn_scale) f = f * bn_scale[co] + bn_offset[co];
            if (prelu_slope && f < 0) f = f * prelu_slope[co];
            float inv = inv_out_pc ? inv_out_pc[co] : inv_scalar;
            o_row[co] = clamp_i8(lrintf_to_int(f * inv));
        }
    }
}

/* ---- kernels/int8_epilogue.c:253-318 ---------------------------------- */
void orc_bn_prelu_requant(const int8_t* in, float in_scale,
                          const float* in_scale_pc,
                          const float* bn_scale, const float* bn_offset,
                          const float* prelu_slope, const float* inv_out_pc,
                          float out_scale, int8_t* out, int n_pos, int C)
{
    float inv_scalar = 1.0f / (out_scale + 1e-9f);
    int vec_end = C & ~7;
    #pragma omp parallel for schedule(static)
    for (int p = 0; p < n_pos; p++) {
        const int8_t* i_row = in + (size_t)p * C;
        int8_t* o_row = out + (size_t)p * C;
        for (int c = 0; c < vec_end; c++) {
            float s = in_scale_pc ? in_scale_pc[c] : in_scale;
            float f = (float)i_row[c] * s;
            if (bn_scale) f = fmaf(f, bn_scale[c], bn_offset[c]);
            if (prelu_slope) {
                float neg = f * prelu_slope[c];
                if (f < 0.0f) f = neg;
            }
            float inv = inv_out_pc ? inv_out_pc[c] : inv_scalar;
            o_row[c] = haz_requant(f * inv);
        }
        for (int c = vec_end; c < C; c++) {     /* tail: parity unpinned */
            float s = in_scale_pc ? in_scale_pc[c] : in_scale;
            float f = (float)i_row[c] * s;
            if (bn_scale) f = f * bn_scale[c] + bn_offset[c];
            if (prelu_slope && f < 0) f = f * prelu_slope[c];
            float inv = inv_out_pc ? inv_out_pc[c] : inv_scalar;
            o_row[c] = clamp_i8(lrintf_to_int(f * inv));
        }
    }
}

/* ---- kernels/int8_epilogue.c:116-131 ---------------------------------- */
void orc_add_requant(const int8_t* a, float a_scale, const int8_t* b,
                     float b_scale, int8_t* out, float out_scale, int n)
{
    float inv = 1.0f / (out_scale + 1e-9f);
    for (int i = 0; i < n; i++) {
        float f = fmaf((float)a[i], a_scale, (float)b[i] * b_scale);
        out[i] = clamp_i8(lrintf_to_int(f * inv));
    }
}

/* ---- libfastface.c:441-455 + kernels/gemm_int8_matvec.c:33-81 ---------- */
void orc_fc(const int8_t* a, const int8_t* W, const float* W_scale,
            const float* bias, float A_scale, float* out, int N, int K)
{
    #pragma omp parallel for schedule(static)
    for (int n = 0; n < N; n++) {
        const int8_t* wr = W + (size_t)n * K;
        int32_t dot = 0;
        for (int k = 0; k < K; k++) dot += (int32_t)a[k] * (int32_t)wr[k];
        float t = (float)dot * A_scale;
        out[n] = fmaf(t, W_scale[n], bias[n]);
    }
}

/* ======================= model files ==================================== */
struct OrcModel {
    uint8_t* blob; size_t size; int version;
    int n_ops; OrcOp* ops;
    float input_scale; float* scales;           /* OPSC */
    int has_v2;                                 /* OPSC2 */
    int n_in; float* in_scale_pc; float* in_inv_pc;
    uint32_t* pc_len; float** inv_pc; float** scale_pc;
};

static uint8_t* read_file(const char* path, size_t* size)
{
    FILE* f = fopen(path, "rb");
    if (!f) return NULL;
    fseek(f, 0, SEEK_END);
    long n = ftell(f);
    fseek(f, 0, SEEK_SET);
    if (n < 0) { fclose(f); return NULL; }
    uint8_t* buf = (uint8_t*)malloc((size_t)n + 16);
    if (buf && fread(buf, 1, (size_t)n, f) != (size_t)n) { free(buf); buf = NULL; }
    fclose(f);
    *size = (size_t)n;
    return buf;
}

static uint16_t rd16(const uint8_t** p) { uint16_t v; memcpy(&v, *p, 2); *p += 2; return v; }
static uint32_t rd32(const uint8_t** p) { uint32_t v; memcpy(&v, *p, 4); *p += 4; return v; }

/* kernels/ffw2_loader.c:71-159 (the blob is read instead of mmapped; float
 * arrays are copied out so they are aligned) */
static int parse_ffw(OrcModel* m)
{
    const uint8_t* p = m->blob;
    if (m->size < 8) return -3;
    if (memcmp(p, "FFW4", 4) == 0) m->version = 4;
    else if (memcmp(p, "FFW3", 4) == 0) m->version = 3;
    else if (memcmp(p, "FFW2", 4) == 0) m->version = 2;
    else return -3;
    p += 4;
    m->n_ops = (int)rd32(&p);
    m->ops = (OrcOp*)calloc((size_t)m->n_ops, sizeof(OrcOp));
    for (int i = 0; i < m->n_ops; i++) {
        OrcOp* op = &m->ops[i];
        op->type = *p++;
        switch (op->type) {
        case ORC_CONV: {
            op->Cin = rd16(&p); op->Cout = rd16(&p); op->Kh = rd16(&p);
            op->Kw = rd16(&p); op->stride = rd16(&p); op->pad = rd16(&p);
            size_t nw = (size_t)op->Cout * op->Cin * op->Kh * op->Kw;
            op->conv_w = (const int8_t*)p; p += nw;
            float* s = (float*)malloc(op->Cout * sizeof(float));
            memcpy(s, p, op->Cout * sizeof(float)); p += op->Cout * sizeof(float);
            op->conv_scales = s;
            if (m->version >= 3) {
                float* b = (float*)malloc(op->Cout * sizeof(float));
                memcpy(b, p, op->Cout * sizeof(float)); p += op->Cout * sizeof(float);
                op->conv_bias = b;
            }
            break;
        }
        case ORC_BN: {
            op->bn_size = rd16(&p);
            float* s = (float*)malloc(op->bn_size * sizeof(float) + 4);
            float* o = (float*)malloc(op->bn_size * sizeof(float) + 4);
            memcpy(s, p, op->bn_size * sizeof(float)); p += op->bn_size * sizeof(float);
            memcpy(o, p, op->bn_size * sizeof(float)); p += op->bn_size * sizeof(float);
            op->bn_scale = s; op->bn_offset = o;
            break;
        }
        case ORC_PRELU: {
            op->prelu_size = rd16(&p);
            float* s = (float*)malloc(op->prelu_size * sizeof(float) + 4);
            memcpy(s, p, op->prelu_size * sizeof(float)); p += op->prelu_size * sizeof(float);
            op->prelu_slope = s;
            break;
        }
        case ORC_ADD: case ORC_FLATTEN: case ORC_SAVE_ID: case ORC_BLOCK_START:
            break;
        case ORC_GEMM: {
            op->N = rd32(&p); op->K = rd32(&p);
            op->gemm_w = (const int8_t*)p; p += (size_t)op->N * op->K;
            float* s = (float*)malloc(op->N * sizeof(float));
            float* b = (float*)malloc(op->N * sizeof(float));
            memcpy(s, p, op->N * sizeof(float)); p += op->N * sizeof(float);
            memcpy(b, p, op->N * sizeof(float)); p += op->N * sizeof(float);
            op->gemm_scales = s; op->gemm_bias = b;
            break;
        }
        default:
            return -4;
        }
    }
    return 0;
}

/* libfastface.c:193-204 */
static int load_opsc(OrcModel* m, const char* path)
{
    size_t n; uint8_t* d = read_file(path, &n);
    if (!d) return -1;
    if (n < 12 || memcmp(d, "OPSC", 4) != 0) { free(d); return -2; }
    const uint8_t* p = d + 4;
    uint32_t n_ops = rd32(&p);
    memcpy(&m->input_scale, p, 4); p += 4;
    m->scales = (float*)calloc(n_ops ? n_ops : 1, sizeof(float));
    size_t avail = (n - 12) / 4;
    memcpy(m->scales, p, (n_ops < avail ? n_ops : avail) * sizeof(float));
    free(d);
    if ((int)n_ops != m->n_ops) return -3;
    return 0;
}

/* libfastface.c:133-191: forward scales kept, inverses 1/(s+1e-9f) */
static int load_opsc2(OrcModel* m, const char* path)
{
    size_t n; uint8_t* d = read_file(path, &n);
    if (!d) return -1;
    if (n < 13 || memcmp(d, "OPSC2", 5) != 0) { free(d); return -2; }
    const uint8_t* p = d + 5;
    uint32_t n_ops = rd32(&p);
    if ((int)n_ops != m->n_ops) { free(d); return -3; }
    uint32_t n_in = rd32(&p);
    m->n_in = (int)n_in;
    m->in_scale_pc = (float*)malloc((n_in + 1) * sizeof(float));
    m->in_inv_pc = (float*)malloc((n_in + 1) * sizeof(float));
    memcpy(m->in_scale_pc, p, n_in * 4); p += n_in * 4;
    for (uint32_t c = 0; c < n_in; c++) m->in_inv_pc[c] = 1.0f / (m->in_scale_pc[c] + 1e-9f);
    m->pc_len = (uint32_t*)calloc(n_ops, sizeof(uint32_t));
    m->inv_pc = (float**)calloc(n_ops, sizeof(float*));
    m->scale_pc = (float**)calloc(n_ops, sizeof(float*));
    for (uint32_t i = 0; i < n_ops; i++) {
        uint32_t nch = rd32(&p);
        m->pc_len[i] = nch;
        if (nch == 0) continue;
        if (nch > 32768) { free(d); return -4; }
        m->inv_pc[i] = (float*)malloc(nch * sizeof(float));
        m->scale_pc[i] = (float*)malloc(nch * sizeof(float));
        for (uint32_t c = 0; c < nch; c++) {
            float s; memcpy(&s, p + 4 * c, 4);
            m->scale_pc[i][c] = s;
            m->inv_pc[i][c] = 1.0f / (s + 1e-9f);
        }
        p += nch * 4;
    }
    free(d);
    m->has_v2 = 1;
    return 0;
}

void orc_model_free(OrcModel* m)
{
    if (!m) return;
    for (int i = 0; m->ops && i < m->n_ops; i++) {
        free((void*)m->ops[i].conv_scales); free((void*)m->ops[i].conv_bias);
        free((void*)m->ops[i].bn_scale); free((void*)m->ops[i].bn_offset);
        free((void*)m->ops[i].prelu_slope);
        free((void*)m->ops[i].gemm_scales); free((void*)m->ops[i].gemm_bias);
        if (m->inv_pc) { free(m->inv_pc[i]); free(m->scale_pc[i]); }
    }
    free(m->ops); free(m->scales); free(m->in_scale_pc); free(m->in_inv_pc);
    free(m->pc_len); free(m->inv_pc); free(m->scale_pc); free(m->blob); free(m);
}

OrcModel* orc_model_load(const char* ffw_path, const char* opsc_path,
                         const char* opsc2_path)
{
    OrcModel* m = (OrcModel*)calloc(1, sizeof(OrcModel));
    m->blob = read_file(ffw_path, &m->size);
    if (!m->blob || parse_ffw(m) != 0) { orc_model_free(m); return NULL; }
    if (load_opsc(m, opsc_path) != 0) { orc_model_free(m); return NULL; }
    if (opsc2_path) load_opsc2(m, opsc2_path);   /* optional, non-fatal */
    return m;
}

int orc_model_n_ops(const OrcModel* m) { return m->n_ops; }
int orc_model_version(const OrcModel* m) { return m->version; }
const OrcOp* orc_model_op(const OrcModel* m, int i) { return &m->ops[i]; }
const float* orc_model_inv_pc(const OrcModel* m, int i, int* len)
{
    if (len) *len = m->has_v2 ? (int)m->pc_len[i] : 0;
    return m->has_v2 ? m->inv_pc[i] : NULL;
}
const float* orc_model_scale_pc(const OrcModel* m, int i)
{
    return m->has_v2 ? m->scale_pc[i] : NULL;
}
float orc_model_scale(const OrcModel* m, int i) { return m->scales[i]; }

/* ======================= interpreter ==================================== */
typedef struct { int C, H, W; } OShape;

int orc_forward(const OrcModel* m, const float* in, int B, float* out,
                orc_dump_fn dump, void* user)
{
    int n = m->n_ops;
    const int v4 = m->version >= 4;
    /* shortcut + shape pre-pass: libfastface.c:243-269 */
    uint8_t* is_sc = (uint8_t*)calloc((size_t)n, 1);
    OShape* sh_in = (OShape*)calloc((size_t)n, sizeof(OShape));
    OShape* sh_out = (OShape*)calloc((size_t)n, sizeof(OShape));
    for (int i = 1; i < n; i++)
        if (m->ops[i].type == ORC_CONV && m->ops[i - 1].type == ORC_SAVE_ID) is_sc[i] = 1;
    OShape cur = {3, 112, 112}, blk = cur;
    size_t max_act = (size_t)3 * 112 * 112;
    for (int i = 0; i < n; i++) {
        const OrcOp* op = &m->ops[i];
        OShape s = is_sc[i] ? blk : cur;
        sh_in[i] = s;
        if (op->type == ORC_CONV) {
            cur.C = op->Cout;
            cur.H = (s.H + 2 * op->pad - op->Kh) / op->stride + 1;
            cur.W = (s.W + 2 * op->pad - op->Kw) / op->stride + 1;
            size_t a = (size_t)cur.C * cur.H * cur.W;
            if (a > max_act) max_act = a;
        } else if (op->type == ORC_GEMM) {
            cur.C = (int)op->N; cur.H = 1; cur.W = 1;
        }
        sh_out[i] = cur;
        if (op->type == ORC_BLOCK_START) blk = cur;
    }
    size_t act_bytes = (size_t)B * max_act + 64;
    int8_t* bufA = (int8_t*)malloc(act_bytes);
    int8_t* bufB = (int8_t*)malloc(act_bytes);
    int8_t* block_buf = (int8_t*)malloc(act_bytes);
    int32_t* acc = (int32_t*)malloc(act_bytes * sizeof(int32_t));
    int8_t* id_slot[24] = {0};
    float id_scale[24] = {0};
    const float* id_scale_pc[24] = {0};

    /* initial quantization: libfastface.c:335-338 (batched: _batched.c:341-346) */
    if (v4 && m->has_v2 && m->in_inv_pc)
        orc_quant_input_pc(in, B * 112 * 112, 3, m->in_inv_pc, bufA);
    else
        orc_quant_input_pt(in, B * 3 * 112 * 112, m->input_scale, bufA);

    int8_t* A = bufA; int8_t* BB = bufB;
    float A_scale = m->input_scale;
    const float* A_scale_pc = v4 ? (m->has_v2 ? m->in_scale_pc : NULL) : NULL;
    float block_scale = m->input_scale;
    int save_idx = 0, add_idx = 0;
    memcpy(block_buf, bufA, (size_t)B * 3 * 112 * 112);
    int rc = 0;

    for (int i = 0; i < n; i++) {
        const OrcOp* op = &m->ops[i];
        OShape si = sh_in[i], so = sh_out[i];
        int HWi = si.H * si.W, HWo = so.H * so.W;
        float next_scale = m->scales[i];
        if (next_scale <= 0) next_scale = A_scale;
        switch (op->type) {
        case ORC_CONV: {    /* libfastface.c:359-400 */
            const int8_t* cin = is_sc[i] ? block_buf : A;
            float cin_scale = is_sc[i] ? block_scale : A_scale;
            if (v4) cin_scale = 1.0f;
            const float* f_prelu = NULL; const int8_t* f_add = NULL;
            float f_add_scale = 0.0f; const float* f_add_pc = NULL;
            float eff_scale = next_scale; int skip = 0, add_fused = 0, eff = i;
            if (i + 1 < n && m->ops[i + 1].type == ORC_PRELU) {
                f_prelu = m->ops[i + 1].prelu_slope;
                eff_scale = m->scales[i + 1];
                if (eff_scale <= 0) eff_scale = next_scale;
                skip = 1; eff = i + 1;
            } else if (i + 1 < n && m->ops[i + 1].type == ORC_ADD) {
                int k = add_idx % 24;
                if (!id_slot[k]) { rc = -10; goto done; }
                f_add = id_slot[k]; f_add_scale = id_scale[k];
                if (v4) f_add_pc = id_scale_pc[k];
                eff_scale = m->scales[i + 1];
                if (eff_scale <= 0) eff_scale = next_scale;
                skip = 1; add_fused = 1; eff = i + 1;
            }
            const float* inv = (v4 && m->has_v2) ? m->inv_pc[eff] : NULL;
            orc_conv_i32(cin, B, si.H, si.W, si.C, op->conv_w, op->Cout, op->Kh,
                         op->Kw, op->stride, op->pad, so.H, so.W, acc);
            orc_fused_epilogue(acc, B * HWo, op->Cout, cin_scale, op->conv_scales,
                               op->conv_bias, NULL, NULL, f_prelu, f_add, f_add_scale,
                               f_add_pc, inv, eff_scale, BB);
            { int8_t* t = A; A = BB; BB = t; }
            A_scale = eff_scale;
            if (v4 && m->has_v2 && m->scale_pc[eff]) A_scale_pc = m->scale_pc[eff];
            if (dump) dump(user, eff, A, B, so.H, so.W, so.C);
            if (skip) i++;
            if (add_fused) add_idx++;
            break;
        }
        case ORC_BN: {      /* libfastface.c:401-413 */
            const float* inv = (v4 && m->has_v2 && m->inv_pc[i] &&
                                m->pc_len[i] == (uint32_t)si.C) ? m->inv_pc[i] : NULL;
            const float* in_pc = (v4 && m->has_v2 && A_scale_pc) ? A_scale_pc : NULL;
            orc_bn_prelu_requant(A, A_scale, in_pc, op->bn_scale, op->bn_offset, NULL,
                                 inv, next_scale, A, B * HWi, si.C);
            A_scale = next_scale;
            if (v4 && m->has_v2 && m->scale_pc[i]) A_scale_pc = m->scale_pc[i];
            if (dump) dump(user, i, A, B, si.H, si.W, si.C);
            break;
        }
        case ORC_PRELU: {   /* libfastface.c:414-424 */
            const float* in_pc = (v4 && m->has_v2 && A_scale_pc) ? A_scale_pc : NULL;
            const float* inv = (v4 && m->has_v2 && m->inv_pc[i]) ? m->inv_pc[i] : NULL;
            orc_bn_prelu_requant(A, A_scale, in_pc, NULL, NULL, op->prelu_slope, inv,
                                 next_scale, A, B * HWi, si.C);
            A_scale = next_scale;
            if (v4 && m->has_v2 && m->scale_pc[i]) A_scale_pc = m->scale_pc[i];
            if (dump) dump(user, i, A, B, si.H, si.W, si.C);
            break;
        }
        case ORC_BLOCK_START:   /* libfastface.c:425-428 */
            memcpy(block_buf, A, (size_t)B * si.C * HWi);
            block_scale = A_scale;
            break;
        case ORC_ADD: {         /* libfastface.c:429-434 */
            int k = add_idx % 24;
            if (!id_slot[k]) { rc = -10; goto done; }
            orc_add_requant(A, A_scale, id_slot[k], id_scale[k], A, next_scale,
                            B * so.C * HWo);
            A_scale = next_scale; add_idx++;
            if (dump) dump(user, i, A, B, so.H, so.W, so.C);
            break;
        }
        case ORC_SAVE_ID: {     /* libfastface.c:435-440 */
            int k = save_idx % 24;
            if (!id_slot[k]) id_slot[k] = (int8_t*)malloc(act_bytes);
            memcpy(id_slot[k], A, (size_t)B * si.C * HWi);
            id_scale[k] = A_scale;
            id_scale_pc[k] = A_scale_pc;
            save_idx++;
            break;
        }
        case ORC_GEMM: {        /* libfastface.c:441-455, batched: per-face matvec */
            float a_sc = v4 ? 1.0f : A_scale;
            for (int b = 0; b < B; b++)
                orc_fc(A + (size_t)b * op->K, op->gemm_w, op->gemm_scales,
                       op->gemm_bias, a_sc, out + (size_t)b * 512, (int)op->N,
                       (int)op->K);
            break;
        }
        case ORC_FLATTEN: {     /* libfastface.c:456-464: NHWC -> NCHW per face */
            int Hf = si.H, Wf = si.W, Cf = si.C;
            size_t fs = (size_t)Cf * Hf * Wf;
            for (int b = 0; b < B; b++)
                for (int c = 0; c < Cf; c++)
                    for (int h = 0; h < Hf; h++)
                        for (int w = 0; w < Wf; w++)
                            BB[b * fs + (size_t)c * Hf * Wf + h * Wf + w] =
                                A[b * fs + ((size_t)h * Wf + w) * Cf + c];
            { int8_t* t = A; A = BB; BB = t; }
            break;
        }
        default:
            rc = -4; goto done;
        }
    }
done:
    for (int k = 0; k < 24; k++) free(id_slot[k]);
    free(bufA); free(bufB); free(block_buf); free(acc);
    free(is_sc); free(sh_in); free(sh_out);
    return rc;
}
