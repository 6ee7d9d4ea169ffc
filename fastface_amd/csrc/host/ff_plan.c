/* ff_plan.c -- turn the FFW op list into a fused launch plan, once.
 *
 * The reference re-interprets the op list on every embed
 * (libfastface.c:312-470; batched: arcface_forward_int8_batched.c:339-516):
 * Conv looks ahead to fuse the next PReLU or Add (:370-382), per-channel
 * forward/inverse scales are tracked op by op (:383-396, :402-411), BN
 * requantizes in place (:401-413), BLOCK_START / SAVE_ID copy the current
 * activation into the block buffer / one of 24 identity slots (:425-440),
 * and FLATTEN transposes NHWC to NCHW before the FC (:456-464).
 *
 * Here the same walk runs once at create time over immutable tensors:
 *   - every CONV (+PReLU | +Add) becomes one kernel launch;
 *   - a BN that follows it (through SAVE_ID / BLOCK_START) becomes a second
 *     output of that launch (the pre-BN tensor is still stored when the
 *     identity slot or the block buffer refers to it);
 *   - a BN or PReLU that no conv absorbs (after an Add, a PReLU, another BN)
 *     becomes a table lookup over its input tensor, and an Add that follows
 *     no conv a lookup over the pairs of its two inputs (the ops are
 *     functions of int8 values; libfastface.c:401-434); their outputs are
 *     new tensors, so earlier references to the input stay intact;
 *   - SAVE_ID / BLOCK_START become tensor references (no copies);
 *   - FLATTEN disappears: the FC weight columns are permuted from the
 *     reference's NCHW order (c*HW + hw) to NHWC (hw*C + c); the int32 dot
 *     product is order-independent, so results are unchanged;
 *   - every scalar fallback of the reference (no OPSC2 entry, length
 *     mismatch) is resolved into explicit per-channel parameter rows,
 *     computed in fp32 exactly as the reference computes them.
 * A conv geometry without a tuned kernel runs on the generic one.  Op
 * sequences outside this pattern (ops on the fp32 input faces other than a
 * 3-channel conv, invalid conv geometries, ops after the GEMM) are rejected
 * (create fails) instead of being run some other way.
 */
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "ff_host.h"

/* Weight-arena contents are produced after the walk, as independent jobs:
 * the walk only places them (offsets), the arena is then allocated once at
 * its final size and the jobs fill it on a few threads. */
enum { JOB_CONV, JOB_WINO, JOB_BN, JOB_FC, JOB_FMA_TAIL, JOB_MAP, JOB_ADD };
typedef struct {
    int kind;
    const int8_t* src;          /* conv / FC weights in the mapping */
    int cout, cin, kh, kw;      /* conv; FC: cout = N, cin = K; MAP: cout = C,
                                   kh = has BN, kw = has PReLU */
    int r0, r1;                 /* FC: rows of this job; FMA_TAIL: r0 the step */
    int fc_hw, fc_c, flat;      /* FC: NCHW flatten -> NHWC column order */
    size_t dst;                 /* bytes into the weight arena */
    size_t p_off;               /* BN, MAP, ADD: floats into the parameter arena */
} PackJob;

typedef struct {
    FfPlan* p;
    size_t p_cap;
    int s_cap, t_cap;
    PackJob* jobs;
    int n_jobs, j_cap;
} Builder;

static void add_job(Builder* b, PackJob j)
{
    if (b->n_jobs == b->j_cap) {
        b->j_cap = b->j_cap ? 2 * b->j_cap : 128;
        b->jobs = (PackJob*)realloc(b->jobs, (size_t)b->j_cap * sizeof(PackJob));
    }
    b->jobs[b->n_jobs++] = j;
}

static int fail(FfPlan* p, const char* msg, int op)
{
    snprintf(p->err, sizeof p->err, "%s (op %d)", msg, op);
    return -1;
}

static int new_tensor(Builder* b, int C, int H, int W, int op)
{
    FfPlan* p = b->p;
    if (p->n_tensors == b->t_cap) {
        b->t_cap = b->t_cap ? 2 * b->t_cap : 64;
        p->tensors = (FfTensor*)realloc(p->tensors, (size_t)b->t_cap * sizeof(FfTensor));
    }
    FfTensor* t = &p->tensors[p->n_tensors];
    t->C = C; t->H = H; t->W = W; t->def_step = p->n_steps; t->last_use = -1; t->buf = -1;
    t->op = op; t->even = 0;
    return p->n_tensors++;
}

static FfStep* new_step(Builder* b)
{
    FfPlan* p = b->p;
    if (p->n_steps == b->s_cap) {
        b->s_cap = b->s_cap ? 2 * b->s_cap : 64;
        p->steps = (FfStep*)realloc(p->steps, (size_t)b->s_cap * sizeof(FfStep));
    }
    FfStep* s = &p->steps[p->n_steps++];
    memset(s, 0, sizeof *s);
    s->t_in = s->t_add = s->t_out = s->t_bn = s->t_x = -1;
    return s;
}

static size_t alloc_params(Builder* b, size_t n)
{
    FfPlan* p = b->p;
    size_t off = (p->p_floats + 63) & ~(size_t)63;     /* 256-byte aligned rows */
    if (off + n > b->p_cap) {
        while (off + n > b->p_cap) b->p_cap = b->p_cap ? 2 * b->p_cap : 65536;
        p->p_host = (float*)realloc(p->p_host, b->p_cap * sizeof(float));
    }
    memset(p->p_host + p->p_floats, 0, (off + n - p->p_floats) * sizeof(float));
    p->p_floats = off + n;
    return off;
}

/* place n bytes in the weight arena (256-byte aligned); filled by a job */
static size_t alloc_weights(Builder* b, size_t n)
{
    FfPlan* p = b->p;
    size_t off = (p->w_bytes + 255) & ~(size_t)255;
    p->w_bytes = off + n;
    return off;
}

static void run_job(FfPlan* p, const PackJob* j, int8_t* row)
{
    int8_t* dst = p->w_host + j->dst;
    switch (j->kind) {
    case JOB_FMA_TAIL: {        /* (each job owns its step's flags) */
        FfStep* st = &p->steps[j->r0];
        if (ffk_requant_fma_ok(p->p_host + j->p_off, j->cout, j->cin, st->flags))
            st->flags |= FFK_EPI_FMA_TAIL;
        break;
    }
    case JOB_CONV:
        ffk_pack_conv_weights(j->src, j->cout, j->cin, j->kh, j->kw, dst);
        break;
    case JOB_WINO:
        ffk_pack_winograd_weights(j->src, j->cout, j->cin, dst);
        break;
    case JOB_BN: {
        const float* P = p->p_host + j->p_off;
        const int C = j->cout;
        ffk_make_bn_lut(P + FFK_P_BN_SIN * C, P + FFK_P_BN_S * C, P + FFK_P_BN_O * C,
                        P + FFK_P_BN_INV * C, C, dst);
        break;
    }
    case JOB_MAP: {             /* rows BN_SIN, BN_S, BN_O, SLOPE, BN_INV */
        const float* P = p->p_host + j->p_off;
        const int C = j->cout;
        ffk_make_map_lut(P + FFK_P_BN_SIN * C, j->kh ? P + FFK_P_BN_S * C : NULL,
                         j->kh ? P + FFK_P_BN_O * C : NULL, j->kw ? P + FFK_P_SLOPE * C : NULL,
                         P + FFK_P_BN_INV * C, C, dst);
        break;
    }
    case JOB_ADD: {             /* a_scale, b_scale, out_scale */
        const float* P = p->p_host + j->p_off;
        ffk_make_add_lut(P[0], P[1], P[2], dst);
        break;
    }
    case JOB_FC: {
        const int N = j->cout, K = j->cin, HW = j->fc_hw, Cc = j->fc_c;
        for (int r = j->r0; r < j->r1; r++) {
            const int8_t* src = j->src + (size_t)r * K;
            if (j->flat) {       /* reference column c*HW + hw -> NHWC column hw*C + c */
                for (int c = 0; c < Cc; c++)
                    for (int hw = 0; hw < HW; hw++) row[(size_t)hw * Cc + c] = src[(size_t)c * HW + hw];
                ffk_pack_fc_row(row, N, K, r, dst);
            } else {
                ffk_pack_fc_row(src, N, K, r, dst);
            }
        }
        break;
    }
    }
}

typedef struct {
    FfPlan* p;
    const PackJob* jobs;
    int n_jobs, next, row_bytes;
    pthread_mutex_t mu;
} JobQueue;

static void* job_worker(void* arg)
{
    JobQueue* q = (JobQueue*)arg;
    int8_t* row = q->row_bytes ? (int8_t*)malloc((size_t)q->row_bytes) : NULL;
    for (;;) {
        pthread_mutex_lock(&q->mu);
        const int k = q->next < q->n_jobs ? q->next++ : -1;
        pthread_mutex_unlock(&q->mu);
        if (k < 0) break;
        run_job(q->p, &q->jobs[k], row);
    }
    free(row);
    return NULL;
}

/* Allocate the weight arena and fill it: the jobs on up to 8 threads (the
 * caller's among them). */
static int run_jobs(Builder* b)
{
    FfPlan* p = b->p;
    p->w_host = (int8_t*)calloc(p->w_bytes ? p->w_bytes : 1, 1);   /* (alignment gaps stay zero) */
    if (!p->w_host) return -1;
    int row_bytes = 0;
    for (int k = 0; k < b->n_jobs; k++)
        if (b->jobs[k].kind == JOB_FC && b->jobs[k].cin > row_bytes) row_bytes = b->jobs[k].cin;
    JobQueue q;
    q.p = p; q.jobs = b->jobs; q.n_jobs = b->n_jobs; q.next = 0; q.row_bytes = row_bytes;
    pthread_mutex_init(&q.mu, NULL);
    long ncpu = sysconf(_SC_NPROCESSORS_ONLN);
    int nt = (int)(ncpu < 1 ? 1 : (ncpu > 8 ? 8 : ncpu));
    if (nt > b->n_jobs) nt = b->n_jobs > 0 ? b->n_jobs : 1;
    pthread_t th[8];
    int started = 0;
    for (int t = 1; t < nt; t++)
        if (pthread_create(&th[started], NULL, job_worker, &q) == 0) started++;
    job_worker(&q);
    for (int t = 0; t < started; t++) pthread_join(th[t], NULL);
    pthread_mutex_destroy(&q.mu);
    return 0;
}

static void fill_row(float* row, int n, const uint8_t* src, float scalar)
{
    for (int i = 0; i < n; i++) row[i] = src ? ff_read_f32(src, i) : scalar;
}
static void fill_rowf(float* row, int n, const float* src, float scalar)
{
    for (int i = 0; i < n; i++) row[i] = src ? src[i] : scalar;
}

/* inverse of a scalar scale the way the reference forms it
 * (int8_epilogue.c:39,122,262: 1.0f / (out_scale + 1e-9f)) */
static float inv_of(float s)
{
    volatile float t = s + 1e-9f;
    return 1.0f / t;
}

typedef struct { int C, H, W; } Shp;

/* A stand-alone BN / PReLU (libfastface.c:401-424, bn_prelu_requant_int8):
 * a per-channel table over the int8 tensor t_in, written to a new tensor.
 * s_in / inv: per-channel rows, or NULL for the scalar in-scale s_in_s and
 * the reference's 1/(out_s + 1e-9f).  Returns the new tensor, or -1. */
static int map_step(Builder* B, int op, int t_in, const float* s_in, float s_in_s,
                    const uint8_t* bn_s, const uint8_t* bn_o, const uint8_t* slope,
                    const float* inv, float out_s)
{
    FfPlan* p = B->p;
    if (t_in == FF_T_INPUT) return fail(p, "only the 3-channel stem conv may read the input faces", op);
    const int C = p->tensors[t_in].C, H = p->tensors[t_in].H, W = p->tensors[t_in].W;
    if (C % 64) return fail(p, "a stand-alone BN / PReLU needs a multiple of 64 channels", op);
    const int Y = new_tensor(B, C, H, W, op);
    FfStep* s = new_step(B);
    s->kind = FF_STEP_MAP; s->op_first = s->op_last = op;
    s->cin = s->cout = C; s->kh = s->kw = 1; s->stride = 1;
    s->hin = s->hout = H; s->win = s->wout = W;
    s->t_in = t_in; s->t_out = s->t_x = Y;
    s->wino_off = (size_t)-1;
    s->p_off = alloc_params(B, (size_t)FFK_NPARAM * C);
    float* P = p->p_host + s->p_off;
    fill_rowf(P + FFK_P_BN_SIN * C, C, s_in, s_in_s);
    if (bn_s) {
        fill_row(P + FFK_P_BN_S * C, C, bn_s, 0.0f);
        fill_row(P + FFK_P_BN_O * C, C, bn_o, 0.0f);
    }
    if (slope) fill_row(P + FFK_P_SLOPE * C, C, slope, 0.0f);
    fill_rowf(P + FFK_P_BN_INV * C, C, inv, inv_of(out_s));
    s->lut_off = alloc_weights(B, (size_t)C * 256);
    add_job(B, (PackJob){ JOB_MAP, NULL, C, 0, bn_s != NULL, slope != NULL, 0, 0, 0, 0, 0,
                          s->lut_off, s->p_off });
    return Y;
}

int ff_plan_build(const FfModel* m, FfPlan* p)
{
    memset(p, 0, sizeof *p);
    Builder B = { p, 0, 0, 0, NULL, 0, 0 };
    const int n = m->n_ops;
    const int v4 = m->version >= 4;
    const int pc = v4 && m->has_v2;

    /* input quantization (libfastface.c:335-338): per-channel for FFW4+OPSC2 */
    for (int c = 0; c < 3; c++)
        p->in_inv[c] = (pc && m->n_in >= 3) ? m->in_inv_pc[c] : inv_of(m->input_scale);
    if (pc && m->n_in < 3) return fail(p, "OPSC2 input scales need 3 channels", -1);
    new_tensor(&B, 3, 112, 112, -1);             /* FF_T_INPUT */

    /* shortcut + shape pre-pass (libfastface.c:243-269) */
    uint8_t* is_sc = (uint8_t*)calloc((size_t)n, 1);
    Shp* sh_in = (Shp*)calloc((size_t)n, sizeof(Shp));
    Shp* sh_out = (Shp*)calloc((size_t)n, sizeof(Shp));
    for (int i = 1; i < n; i++)
        if (m->ops[i].type == FF_OP_CONV && m->ops[i - 1].type == FF_OP_SAVE_ID) is_sc[i] = 1;
    Shp cur = {3, 112, 112}, blk = cur;
    for (int i = 0; i < n; i++) {
        const FfOp* op = &m->ops[i];
        Shp s = is_sc[i] ? blk : cur;
        sh_in[i] = s;
        if (op->type == FF_OP_CONV) {
            if (op->stride <= 0) { free(is_sc); free(sh_in); free(sh_out); return fail(p, "bad stride", i); }
            cur.C = op->Cout;
            cur.H = (s.H + 2 * op->pad - op->Kh) / op->stride + 1;
            cur.W = (s.W + 2 * op->pad - op->Kw) / op->stride + 1;
        } else if (op->type == FF_OP_GEMM) {
            cur.C = (int)op->N; cur.H = 1; cur.W = 1;
        }
        sh_out[i] = cur;
        if (op->type == FF_OP_BLOCK_START) blk = cur;
    }

    int rc = 0;
    int A = FF_T_INPUT;
    float A_scale = m->input_scale;
    const float* A_pc = pc ? m->in_scale_pc : NULL;
    int A_pc_len = pc ? m->n_in : 0;    /* floats A_pc holds */
    int blk_t = FF_T_INPUT;
    float blk_scale = m->input_scale;
    int slot_t[24]; float slot_scale[24]; const float* slot_pc[24]; int slot_pc_len[24];
    for (int k = 0; k < 24; k++) { slot_t[k] = -1; slot_scale[k] = 0.0f; slot_pc[k] = NULL; slot_pc_len[k] = 0; }
    int save_idx = 0, add_idx = 0;
    int last_conv = -1;         /* step whose output A currently is */
    int flat = 0, done = 0;

    for (int i = 0; i < n && !rc; i++) {
        const FfOp* op = &m->ops[i];
        float next_scale = m->scales[i];
        if (next_scale <= 0) next_scale = A_scale;
        if (done) { rc = fail(p, "ops after the GEMM are not supported", i); break; }
        switch (op->type) {
        case FF_OP_CONV: {
            const int in_t = is_sc[i] ? blk_t : A;
            const float in_scale = v4 ? 1.0f : (is_sc[i] ? blk_scale : A_scale);
            const Shp si = sh_in[i], so = sh_out[i];
            if (op->Cin != si.C) { rc = fail(p, "conv Cin does not match its input", i); break; }
            if ((in_t == FF_T_INPUT) != (op->Cin == 3)) {
                rc = fail(p, "only a 3-channel stem conv may read the input faces", i); break;
            }
            if (!ffk_conv_runnable(op->Cin, op->Cout, op->Kh, op->Kw, op->stride, op->pad, si.H, si.W)) {
                rc = fail(p, "invalid conv geometry", i); break;
            }
            const uint8_t* slope = NULL;
            int add_k = -1, eff = i, skip = 0;
            float eff_scale = next_scale;
            if (i + 1 < n && m->ops[i + 1].type == FF_OP_PRELU) {
                if (m->ops[i + 1].prelu_size != op->Cout) { rc = fail(p, "PReLU size != Cout", i + 1); break; }
                slope = m->ops[i + 1].prelu_slope;
                eff_scale = m->scales[i + 1];
                if (eff_scale <= 0) eff_scale = next_scale;
                eff = i + 1; skip = 1;
            } else if (i + 1 < n && m->ops[i + 1].type == FF_OP_ADD) {
                add_k = add_idx % 24;
                if (slot_t[add_k] < 0) { rc = fail(p, "Add before any SAVE_ID", i + 1); break; }
                const FfTensor* at = &p->tensors[slot_t[add_k]];
                if (at->C != op->Cout || at->H != so.H || at->W != so.W) {
                    rc = fail(p, "Add operands differ in shape", i + 1); break;
                }
                if (v4 && slot_pc[add_k] && slot_pc_len[add_k] < op->Cout) {
                    rc = fail(p, "OPSC2 entry too short", i + 1); break;
                }
                eff_scale = m->scales[i + 1];
                if (eff_scale <= 0) eff_scale = next_scale;
                eff = i + 1; skip = 1;
            }
            const float* inv_pc = pc ? m->inv_pc[eff] : NULL;
            if (inv_pc && m->pc_len[eff] < (uint32_t)op->Cout) { rc = fail(p, "OPSC2 entry too short", eff); break; }

            const int X = new_tensor(&B, op->Cout, so.H, so.W, eff);
            FfStep* s = new_step(&B);
            s->kind = FF_STEP_CONV; s->op_first = i; s->op_last = eff;
            s->cin = op->Cin; s->cout = op->Cout; s->kh = op->Kh; s->kw = op->Kw;
            s->stride = op->stride; s->pad = op->pad; s->hin = si.H; s->win = si.W;
            s->hout = so.H; s->wout = so.W;
            s->t_in = in_t; s->t_out = X; s->t_x = X;
            s->in_scale = in_scale;
            s->flags = FFK_EPI_BIAS | (in_scale != 1.0f ? FFK_EPI_INSCALE : 0);
            s->w_off = alloc_weights(&B, ffk_conv_packed_bytes(op->Cin, op->Cout, op->Kh, op->Kw));
            add_job(&B, (PackJob){ JOB_CONV, op->conv_w, op->Cout, op->Cin, op->Kh, op->Kw, 0, 0, 0, 0, 0,
                                   s->w_off, 0 });
            s->wino_off = (size_t)-1;
            if (ffk_winograd_supported(op->Cin, op->Cout, op->Kh, op->Kw, op->stride, op->pad, si.H, si.W)) {
                /* the same layer as integer Winograd F(2,3) (fastface_set_conv_algo) */
                s->wino_off = alloc_weights(&B, ffk_winograd_packed_bytes(op->Cin, op->Cout));
                add_job(&B, (PackJob){ JOB_WINO, op->conv_w, op->Cout, op->Cin, 3, 3, 0, 0, 0, 0, 0,
                                       s->wino_off, 0 });
            }
            s->p_off = alloc_params(&B, (size_t)FFK_NPARAM * op->Cout);
            float* P = p->p_host + s->p_off;
            const int C = op->Cout;
            fill_row(P + FFK_P_WS * C, C, op->conv_scales, 0.0f);
            fill_row(P + FFK_P_BIAS * C, C, op->conv_bias, 0.0f);   /* FFW2: no bias, +0 */
            fill_rowf(P + FFK_P_INV * C, C, inv_pc, inv_of(eff_scale));
            if (slope) {
                s->flags |= FFK_EPI_PRELU;
                fill_row(P + FFK_P_SLOPE * C, C, slope, 0.0f);
            }
            if (add_k >= 0) {
                s->flags |= FFK_EPI_ADD;
                s->t_add = slot_t[add_k];
                /* per-channel shortcut scale for FFW4 (libfastface.c:378), else scalar */
                fill_rowf(P + FFK_P_ADDSCALE * C, C, v4 ? slot_pc[add_k] : NULL, slot_scale[add_k]);
                add_idx++;
            }
            /* PReLU as max(f, f*slope) where the parameters allow it (same values) */
            if (slope && ffk_prelu_le1_ok(P, C, op->Kh * op->Kw * op->Cin, add_k >= 0))
                s->flags |= FFK_EPI_PRELU_LE1;
            /* requant values provably finite and below 2^31: no x86 out-of-range case */
            if (ffk_requant_in_range(P, C, op->Kh * op->Kw * op->Cin, s->flags)) {
                s->flags |= FFK_EPI_IN_RANGE;
                /* without a residual: its last two roundings as one, where no
                 * value of the layer tells them apart (a job: the proof
                 * searches per channel) */
                if (!(s->flags & (FFK_EPI_ADD | FFK_EPI_INSCALE)))
                    add_job(&B, (PackJob){ JOB_FMA_TAIL, NULL, C, op->Kh * op->Kw * op->Cin, 0, 0,
                                           p->n_steps - 1, 0, 0, 0, 0, 0, s->p_off });
            }
            A = X; A_scale = eff_scale;
            if (pc && m->scale_pc[eff]) { A_pc = m->scale_pc[eff]; A_pc_len = (int)m->pc_len[eff]; }
            last_conv = p->n_steps - 1;
            if (skip) i++;
            break;
        }
        case FF_OP_BN: {                 /* libfastface.c:401-413 */
            const Shp si = sh_in[i];
            const int C = si.C;
            if (op->bn_size != C) { rc = fail(p, "BN size != channels", i); break; }
            const float* bn_inv = (pc && m->inv_pc[i] && m->pc_len[i] == (uint32_t)C) ? m->inv_pc[i] : NULL;
            const float* bn_in = (pc && A_pc) ? A_pc : NULL;
            if (bn_in && A_pc_len < C) { rc = fail(p, "OPSC2 entry too short", i); break; }
            if (last_conv >= 0 && p->steps[last_conv].t_out == A && p->steps[last_conv].t_bn < 0) {
                /* the second output of the conv that produced A (through
                 * SAVE_ID / BLOCK_START only) */
                FfStep* s = &p->steps[last_conv];
                float* P = p->p_host + s->p_off;
                fill_rowf(P + FFK_P_BN_SIN * C, C, bn_in, A_scale);
                fill_row(P + FFK_P_BN_S * C, C, op->bn_scale, 0.0f);
                fill_row(P + FFK_P_BN_O * C, C, op->bn_offset, 0.0f);
                fill_rowf(P + FFK_P_BN_INV * C, C, bn_inv, inv_of(next_scale));
                s->flags |= FFK_EPI_BN;
                s->lut_off = alloc_weights(&B, (size_t)C * 256);
                add_job(&B, (PackJob){ JOB_BN, NULL, C, 0, 0, 0, 0, 0, 0, 0, 0, s->lut_off, s->p_off });
                const int Y = new_tensor(&B, C, si.H, si.W, i);
                p->tensors[Y].def_step = last_conv;
                s->t_bn = Y;
                s->op_last = i;
                A = Y;
            } else {
                const int Y = map_step(&B, i, A, bn_in, A_scale, op->bn_scale, op->bn_offset, NULL,
                                       bn_inv, next_scale);
                if (Y < 0) { rc = -1; break; }
                A = Y;
            }
            A_scale = next_scale;
            if (pc && m->scale_pc[i]) { A_pc = m->scale_pc[i]; A_pc_len = (int)m->pc_len[i]; }
            break;
        }
        case FF_OP_PRELU: {              /* libfastface.c:414-424 (not after a conv) */
            const int C = sh_in[i].C;
            if (op->prelu_size != C) { rc = fail(p, "PReLU size != channels", i); break; }
            const float* in_pc = (pc && A_pc) ? A_pc : NULL;
            const float* inv = (pc && m->inv_pc[i]) ? m->inv_pc[i] : NULL;
            if ((in_pc && A_pc_len < C) || (inv && m->pc_len[i] < (uint32_t)C)) {
                rc = fail(p, "OPSC2 entry too short", i); break;
            }
            const int Y = map_step(&B, i, A, in_pc, A_scale, NULL, NULL, op->prelu_slope, inv, next_scale);
            if (Y < 0) { rc = -1; break; }
            A = Y; A_scale = next_scale;
            if (pc && m->scale_pc[i]) { A_pc = m->scale_pc[i]; A_pc_len = (int)m->pc_len[i]; }
            break;
        }
        case FF_OP_ADD: {                /* libfastface.c:429-434 (not after a conv) */
            const int k = add_idx % 24;
            if (slot_t[k] < 0) { rc = fail(p, "Add before any SAVE_ID", i); break; }
            if (A == FF_T_INPUT || slot_t[k] == FF_T_INPUT) {
                rc = fail(p, "only the 3-channel stem conv may read the input faces", i); break;
            }
            const FfTensor* ta = &p->tensors[A];
            const FfTensor* tb = &p->tensors[slot_t[k]];
            if (ta->C != tb->C || ta->H != tb->H || ta->W != tb->W) {
                rc = fail(p, "Add operands differ in shape", i); break;
            }
            const int C = ta->C, H = ta->H, W = ta->W;
            if (C % 16) { rc = fail(p, "a stand-alone Add needs a multiple of 16 channels", i); break; }
            const int Y = new_tensor(&B, C, H, W, i);
            FfStep* s = new_step(&B);
            s->kind = FF_STEP_ADD; s->op_first = s->op_last = i;
            s->cin = s->cout = C; s->kh = s->kw = 1; s->stride = 1;
            s->hin = s->hout = H; s->win = s->wout = W;
            s->t_in = A; s->t_add = slot_t[k]; s->t_out = s->t_x = Y;
            s->wino_off = (size_t)-1;
            /* per-tensor scales even in FFW4 (add_requant_int8) */
            s->p_off = alloc_params(&B, 3);
            p->p_host[s->p_off] = A_scale;
            p->p_host[s->p_off + 1] = slot_scale[k];
            p->p_host[s->p_off + 2] = next_scale;
            s->lut_off = alloc_weights(&B, 65536);
            add_job(&B, (PackJob){ JOB_ADD, NULL, 0, 0, 0, 0, 0, 0, 0, 0, 0, s->lut_off, s->p_off });
            A = Y; A_scale = next_scale;        /* (the per-channel scales stay) */
            add_idx++;
            break;
        }
        case FF_OP_BLOCK_START:          /* libfastface.c:425-428 */
            blk_t = A; blk_scale = A_scale;
            break;
        case FF_OP_SAVE_ID: {            /* libfastface.c:435-440 */
            const int k = save_idx % 24;
            slot_t[k] = A; slot_scale[k] = A_scale; slot_pc[k] = A_pc; slot_pc_len[k] = A_pc_len;
            save_idx++;
            break;
        }
        case FF_OP_FLATTEN:
            flat = 1;
            break;
        case FF_OP_GEMM: {               /* libfastface.c:441-455 */
            const FfTensor* at = &p->tensors[A];
            const int K = (int)op->K, N = (int)op->N;
            if (A == FF_T_INPUT || (long long)at->C * at->H * at->W != K) {
                rc = fail(p, "GEMM K does not match its input", i); break;
            }
            if (K % 64 != 0) { rc = fail(p, "GEMM K must be a multiple of 64", i); break; }
            FfStep* s = new_step(&B);
            s->kind = FF_STEP_FC; s->op_first = i; s->op_last = i;
            s->t_in = A; s->fc_n = N; s->fc_k = K;
            s->a_scale = v4 ? 1.0f : A_scale;
            s->w_off = alloc_weights(&B, ffk_fc_packed_bytes(N, K));
            /* 16 rows per job: the rows are permuted and packed on the threads */
            for (int r0 = 0; r0 < N; r0 += 16)
                add_job(&B, (PackJob){ JOB_FC, op->gemm_w, N, K, 0, 0, r0, r0 + 16 < N ? r0 + 16 : N,
                                       at->H * at->W, at->C, flat, s->w_off, 0 });
            s->ws_off = alloc_params(&B, (size_t)N);
            fill_row(p->p_host + s->ws_off, N, op->gemm_scales, 0.0f);
            s->bias_off = alloc_params(&B, (size_t)N);
            fill_row(p->p_host + s->bias_off, N, op->gemm_bias, 0.0f);
            p->emb_n = N;
            done = 1;
            break;
        }
        default:
            rc = fail(p, "unknown op", i);
        }
    }
    free(is_sc); free(sh_in); free(sh_out);
    if (!rc && !done) rc = fail(p, "model has no GEMM head", n);
    if (!rc && p->emb_n != FASTFACE_OUTPUT_N) rc = fail(p, "embedding size must be 512", n);
    if (!rc && run_jobs(&B)) rc = fail(p, "out of host memory", n);
    free(B.jobs);
    return rc;
}

int ff_plan_pair(const FfPlan* p, int s)
{
    if (s < 0 || s + 1 >= p->n_steps) return 0;
    const FfStep* a = &p->steps[s];
    const FfStep* b = a + 1;
    return a->kind == FF_STEP_CONV && b->kind == FF_STEP_CONV && a->kh == 3 && a->stride == 2 && a->t_bn < 0 &&
           a->t_out >= 0 && b->t_add == a->t_out && b->t_in != a->t_out && p->tensors[a->t_out].last_use == s + 1;
}

int ff_plan_assign_buffers(FfPlan* p, int keep_all)
{
    for (int t = 0; t < p->n_tensors; t++) {
        p->tensors[t].last_use = -1; p->tensors[t].buf = -1; p->tensors[t].even = 0;
    }
    for (int s = 0; s < p->n_steps; s++) {
        const FfStep* st = &p->steps[s];
        if (st->t_in >= 0) p->tensors[st->t_in].last_use = s;
        if (st->t_add >= 0) p->tensors[st->t_add].last_use = s;
    }
    p->max_face_bytes = 0;
    for (int t = 1; t < p->n_tensors; t++) {
        size_t b = (size_t)p->tensors[t].C * p->tensors[t].H * p->tensors[t].W;
        if (b > p->max_face_bytes) p->max_face_bytes = b;
    }
    /* the pre-BN output of a dual-output step is stored only if read later */
    for (int s = 0; s < p->n_steps; s++) {
        FfStep* st = &p->steps[s];
        if (st->kind != FF_STEP_CONV) continue;
        st->t_out = st->t_x;
        if (st->t_bn >= 0 && p->tensors[st->t_x].last_use < 0 && !keep_all) st->t_out = -1;
    }
    /* A stored tensor whose every reader is a 1x1 stride-2 pad-0 conv (the
     * downsample shortcut of the next stage's first block, the only reader of
     * a stage's output X) is stored at its even pixels only: those readers
     * see nothing else, and run as 1x1 stride-1 convs over the compact tensor.
     * keep_all (debug reads) keeps every tensor whole. */
    for (int s = 0; s < p->n_steps && !keep_all; s++) {
        const FfStep* st = &p->steps[s];
        if (st->kind != FF_STEP_CONV || st->t_out < 0) continue;
        FfTensor* T = &p->tensors[st->t_out];
        if ((T->H & 1) || (T->W & 1)) continue;
        int readers = 0, ok = 1;
        for (int r = s + 1; r < p->n_steps && ok; r++) {
            const FfStep* rd = &p->steps[r];
            if (rd->t_add == st->t_out) ok = 0;
            if (rd->t_in != st->t_out) continue;
            readers++;
            ok = rd->kind == FF_STEP_CONV && rd->kh == 1 && rd->kw == 1 && rd->stride == 2 && rd->pad == 0 &&
                 ffk_conv_supported(rd->cin, rd->cout, 1, 1, 1, 0, T->H / 2, T->W / 2);
        }
        T->even = ok && readers > 0;
    }
    int* free_list = (int*)malloc((size_t)(p->n_tensors + 1) * sizeof(int));
    int n_free = 0, n_buf = 0;
    for (int s = 0; s < p->n_steps; s++) {
        FfStep* st = &p->steps[s];
        int outs[2] = { st->t_out, st->t_bn };
        for (int k = 0; k < 2; k++) {
            int t = outs[k];
            if (t < 0) continue;
            if (!keep_all && n_free > 0) p->tensors[t].buf = free_list[--n_free];
            else p->tensors[t].buf = n_buf++;
        }
        if (keep_all) continue;
        /* A pair that may run as one launch (ff_plan_pair) releases the
         * buffers its first step is done with only after the pair: the second
         * step's outputs must not take a buffer the first step still reads. */
        if (ff_plan_pair(p, s)) continue;
        const int from = ff_plan_pair(p, s - 1) ? s - 1 : s;
        /* release what is dead after this step (inputs, and outputs never read) */
        for (int t = 1; t < p->n_tensors; t++) {
            FfTensor* T = &p->tensors[t];
            if (T->buf < 0) continue;
            if (T->last_use >= from && T->last_use <= s) free_list[n_free++] = T->buf;
        }
    }
    free(free_list);
    p->n_buffers = n_buf;
    return 0;
}

void ff_plan_free(FfPlan* p)
{
    free(p->steps); free(p->tensors); free(p->w_host); free(p->p_host);
    memset(p, 0, sizeof *p);
}
