/* fastface.c -- the fastface.h C API on MI355X.
 *
 * create (reference libfastface.c:231-310): load FFW + OPSC/OPSC2, build the
 * fused launch plan, pack all weights into one device arena and all
 * per-channel parameters into another (two uploads), create the stream.
 * embed (libfastface.c:312-470): copy the faces in, replay the captured
 * launch chain for this batch size (one hipGraph per batch size, built on
 * first use over preallocated activation buffers), copy the embeddings out.
 * destroy (libfastface.c:472-490): free everything, including what the
 * reference leaks (the mapping and the scale arrays).
 *
 * Errors: NULL from create, non-zero from embed -- never an abort.  A HIP
 * failure message goes to stderr once, prefixed "fastface:".
 */
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "ff_host.h"

#define FF_MAX_GRAPHS 16

/* Host-buffer batches of at least two chunks stream: the host-to-device copy
 * of chunk k+1 (copy stream) runs while chunk k computes (context stream),
 * each chunk in its own region of the input buffer.  A chunk must fill the
 * GPU by itself, and the copy it hides must be worth a second launch chain:
 * uint8 batches stream in chunks of 512 faces (at 1024 faces ~122k faces/s,
 * against ~119k as one staged copy and one launch chain). */
#define FF_STREAM_CHUNK_U8 512
/* fp32 faces are four times the bytes: the first chunk's copy, the one
 * the GPU waits for, is kept short (256 faces), and the chunks after it
 * are larger (768), so that each copy still finishes while the chunk
 * before it computes (1024 faces as 256 + 768: ~111,000 faces/s against
 * ~106,000 as 512 + 512, same box).  Batches of up to FF_STREAM_MIN_F32
 * faces go in one copy. */
#define FF_STREAM_FIRST_F32 256
#define FF_STREAM_CHUNK_F32 768
#define FF_STREAM_MIN_F32 512
#define FF_MAX_CHUNKS 64

/* A streamed chunk reaches the device through two pinned staging buffers:
 * threads of the calling process copy one piece of the caller's (pageable)
 * faces into one buffer while the DMA of the previous piece runs from the
 * other.  A plain copy from pageable memory is staged by the runtime on one
 * host thread (~27 GB/s measured on the MI355X box); eight threads fill
 * pinned memory at ~64 GB/s and the DMA from it runs at ~57 GB/s. */
#ifndef FF_STAGE_MB
#define FF_STAGE_MB 16
#endif
#ifndef FF_STAGE_THREADS
#define FF_STAGE_THREADS 8
#endif
#define FF_STAGE_BYTES ((size_t)FF_STAGE_MB << 20)
/* a one-chunk host batch of at least this many bytes is staged too */
#define FF_STAGE_MIN_BYTES ((size_t)8 << 20)
/* Small host batches bounce through one pinned buffer instead (a DMA from
 * pinned memory skips the runtime's own staging of pageable memory): the
 * input up to FF_SMALL_IN bytes (one fp32 face, six uint8 faces), the
 * embeddings up to FF_SMALL_OUT bytes (eight faces).  Measured at b=1: the
 * 2 KB embedding 21.4 -> 11.9 us, the 147 KB face 14.7 -> 13.1 us. */
#define FF_SMALL_IN ((size_t)256 << 10)
#define FF_SMALL_OUT ((size_t)16 << 10)

/* Batches of FF_SPLIT_MIN faces or more run as two halves, each on its own
 * stream inside the one captured graph (a fork and a join), both launched
 * with FFK_SHARED_GPU (each layer takes the tiling the two halves' grids
 * together fill the GPU with).  A layer's kernel of one half fills the CUs
 * the other half's kernel leaves idle: the last, partly filled round of
 * workgroups at large batches, the partly empty grids at small ones.
 * Faces are independent, so the embeddings equal the one-chain path's bit
 * for bit.  Each half has its own region of every activation buffer, its
 * own I/O descriptor (d_io[part]) and its own half of the split-K
 * workspace.  Measured (ms per batch, one chain -> two halves, same box):
 * 16 0.677 -> 0.681, 32 0.754 -> 0.770, 48 0.891 -> 0.823, 96 1.42 -> 1.11,
 * 256 2.75 -> 2.33, 512 4.37 -> 3.76, 1024 7.86 -> 7.25; with the small-tile
 * kernels of small grids the halves win from 24 faces on: 16 0.516 -> 0.586,
 * 20 0.519 -> 0.566, 24 0.625 -> 0.588, 32 0.643 -> 0.637, 40 0.728 -> 0.684,
 * 47 0.872 -> 0.722. */
#define FF_SPLIT_MIN 24

/* one captured chain per (batch, input format: 0 fp32 faces, 1 uint8 RGB) */
typedef struct { int batch, fmt; void* exec; } GraphEntry;

/* Stream ordering.  A context's device state (the I/O descriptor, the
 * activation buffers, the split-K workspace and its counters, the captured
 * chains) is used by whatever stream the last call enqueued on: the context
 * stream, or a caller stream given to a *_device entry point.  After every
 * enqueue, ev_last is recorded on that stream.  A later enqueue on another
 * stream first makes that stream wait for ev_last (device-side ordering, no
 * host wait), and anything that rewrites or frees that state from the host
 * (the I/O staging slot, buffer growth, graph eviction, destroy) first waits
 * for ev_last on the host.  So calls on different streams never overlap on
 * one context's buffers. */

typedef struct Stager Stager;
static void stager_stop(Stager* s);

struct FastFace {
    FfModel model;
    FfPlan plan;
    void* stream;
    int8_t* d_weights;
    float* d_params;
    float* d_in_inv;
    int capacity;               /* faces the activation buffers hold */
    int8_t** d_bufs;            /* plan.n_buffers buffers */
    float* d_input;             /* capacity * 37632 */
    uint8_t* d_input_u8;        /* capacity * 37632 (uint8 RGB input) */
    int8_t* d_in_lut;           /* [3][256] uint8 pixel -> int8 input table */
    float* d_output;            /* capacity * 512 */
    void* d_ws;                 /* split-K workspaces of the small-batch convs */
    size_t ws_part;             /* bytes of each of d_ws's two halves */
    ffk_io* d_io;               /* device I/O descriptors of the two halves */
    ffk_io* h_io;               /* pinned staging, two descriptors each:
                                   [0..1] set_io, [2(1 + k)..] chunk k */
    void* cstream;              /* host-to-device copies of streamed chunks */
    void* sstream;              /* the second half of a split chain */
    void* ev_fork, *ev_join;    /* (recorded only inside graph capture) */
    void* ev_chunk[FF_MAX_CHUNKS];
    void* h_stage[2];           /* pinned staging of streamed input pieces (on first use) */
    void* h_small;              /* pinned bounce buffer of small host batches (on first use):
                                   FF_SMALL_IN input bytes, then FF_SMALL_OUT output bytes */
    void* ev_stage[2];          /* the last DMA out of each staging buffer */
    Stager* stager;             /* its copy threads (on first use), or NULL */
    ffk_io io_cur[2];           /* what d_io holds now */
    int keep_all;
    int algo;                   /* FASTFACE_CONV_* of the 64-channel 3x3 s1 layers */
    int general_epi;            /* launch every conv with the general epilogue forms */
    int no_fusion;              /* stride-2 convs and their shortcuts as two launches */
    GraphEntry graphs[FF_MAX_GRAPHS];
    int n_graphs, graph_rr;
    void* ev_last;              /* recorded after the last enqueue, on last_stream */
    void* last_stream;          /* stream of the last enqueue (NULL: none pending) */
};

static void report(const char* what, int rc)
{
    fprintf(stderr, "fastface: %s failed (%d): %s\n", what, rc, ffk_last_error());
}

/* host wait for everything this context enqueued (on any stream) */
static int drain(FastFace* ff)
{
    if (!ff->last_stream) return 0;
    int rc = ffk_event_sync(ff->ev_last);
    if (!rc) ff->last_stream = NULL;
    return rc;
}

/* order `stream` after the context's last enqueue on another stream */
static int order_after_last(FastFace* ff, void* stream)
{
    if (!ff->last_stream || ff->last_stream == stream) return 0;
    return ffk_stream_wait_event(stream, ff->ev_last);
}

/* record the end of an enqueue on `stream` */
static int mark_enqueued(FastFace* ff, void* stream)
{
    int rc = ffk_event_record(ff->ev_last, stream);
    if (!rc) ff->last_stream = stream;
    return rc;
}

static void drop_graphs(FastFace* ff)
{
    for (int i = 0; i < ff->n_graphs; i++) ffk_graph_destroy(ff->graphs[i].exec);
    ff->n_graphs = 0;
    ff->graph_rr = 0;
}

static void free_activations(FastFace* ff)
{
    drop_graphs(ff);
    if (ff->d_bufs) {
        for (int i = 0; i < ff->plan.n_buffers; i++) ffk_free(ff->d_bufs[i]);
        free(ff->d_bufs);
        ff->d_bufs = NULL;
    }
    ffk_free(ff->d_input); ff->d_input = NULL;
    ffk_free(ff->d_input_u8); ff->d_input_u8 = NULL;
    ffk_free(ff->d_output); ff->d_output = NULL;
    ffk_free(ff->d_ws); ff->d_ws = NULL;
    ff->ws_part = 0;
    ff->capacity = 0;
}

/* first face of the second half of a `batch` chain, or 0: one chain */
static int split_at(const FastFace* ff, int batch)
{
    return (!ff->keep_all && batch >= FF_SPLIT_MIN) ? batch / 2 : 0;
}

/* the I/O descriptors of the two halves of a `batch` chain over (in, out);
 * fmt 0: fp32 faces, 1: uint8 RGB */
static void io_pair(const FastFace* ff, ffk_io* io, const void* in, float* out, int batch, int fmt)
{
    const int na = split_at(ff, batch);
    const size_t face = (size_t)FASTFACE_INPUT_N * (fmt ? 1 : sizeof(float));
    io[0].in = (const float*)in;
    io[0].out = out;
    io[1].in = (const float*)((const int8_t*)in + (size_t)na * face);
    io[1].out = out + (size_t)na * FASTFACE_OUTPUT_N;
}

/* Point the device I/O descriptor at (in, out) for work enqueued next on
 * `stream`.  Unchanged pointers: nothing to do (the enqueue orders itself
 * after the last one).  Changed: every earlier enqueue of this context, on
 * any stream, may still read the descriptor or the staging slot, so wait for
 * them on the host first. */
static int set_io(FastFace* ff, const void* in, float* out, void* stream, int batch, int fmt)
{
    ffk_io want[2];
    io_pair(ff, want, in, out, batch, fmt);
    if (!memcmp(want, ff->io_cur, sizeof want)) return 0;
    int rc = drain(ff);
    if (!rc) rc = ffk_stream_sync(ff->stream);
    if (!rc && stream != ff->stream) rc = ffk_stream_sync(stream);
    if (rc) return rc;
    memcpy(ff->h_io, want, sizeof want);
    rc = ffk_memcpy_h2d(ff->d_io, ff->h_io, sizeof want, stream);
    if (!rc) rc = ffk_stream_sync(stream);
    if (rc) return rc;
    memcpy(ff->io_cur, want, sizeof want);
    return 0;
}

/* The epilogue flags a step launches with: the plan's, less the proven
 * fast forms when the context runs the general ones
 * (fastface_set_epilogue_forms). */
#define FF_FAST_EPI (FFK_EPI_PRELU_LE1 | FFK_EPI_IN_RANGE | FFK_EPI_FMA_TAIL)
static int step_flags(const FastFace* ff, const FfStep* st)
{
    return ff->general_epi ? st->flags & ~FF_FAST_EPI : st->flags;
}

static void step_desc(FastFace* ff, int s, int batch, int fmt, int part, size_t off, int shared, ffk_conv_desc* d);

/* Largest workspace any conv step asks for at 1..max_batch faces.  Only
 * small batches split K (the split grid is capped at FF_SPLIT_MAX_WG 64x64
 * tiles, far below 4096 faces for every layer); the Winograd and generic
 * paths need none.  max_batch itself is checked too (the FC head's split-K
 * workspace grows with the batch up to its own cap). */
static size_t workspace_bytes(FastFace* ff, int max_batch)
{
    size_t best = 0;
    const int top = max_batch < 4096 ? max_batch : 4096;
    for (int s = 0; s < ff->plan.n_steps; s++) {
        if (ff->plan.steps[s].kind == FF_STEP_FC) {          /* FC head: split-K of mid-size batches */
            for (int b = 1; b <= top + 1; b++) {
                ffk_fc_desc f;
                memset(&f, 0, sizeof f);
                f.batch = b <= top ? b : max_batch; f.n = ff->plan.steps[s].fc_n; f.k = ff->plan.steps[s].fc_k;
                const size_t n = ffk_fc_workspace_bytes(&f);
                if (n > best) best = n;
            }
            continue;
        }
        if (ff->plan.steps[s].kind != FF_STEP_CONV) continue;
        for (int b = 1; b <= top + 1; b++) {
            ffk_conv_desc d;
            step_desc(ff, s, b <= top ? b : max_batch, 0, 0, 0, 0, &d);
            const size_t n = ffk_conv_workspace_bytes(&d);
            if (n > best) best = n;
        }
    }
    return best;
}

static int ensure_capacity(FastFace* ff, int batch)
{
    if (batch <= ff->capacity) return 0;
    int rc = drain(ff);
    if (!rc) rc = ffk_stream_sync(ff->stream);
    if (rc) return rc;
    free_activations(ff);
    FfPlan* p = &ff->plan;
    ff->d_bufs = (int8_t**)calloc((size_t)p->n_buffers, sizeof(int8_t*));
    if (!ff->d_bufs) return FFK_ERR_NOMEM;
    const size_t buf_bytes = p->max_face_bytes * (size_t)batch + 256;
    for (int i = 0; i < p->n_buffers; i++) {
        ff->d_bufs[i] = (int8_t*)ffk_malloc(buf_bytes);
        if (!ff->d_bufs[i]) { free_activations(ff); return FFK_ERR_NOMEM; }
    }
    ff->d_input = (float*)ffk_malloc((size_t)batch * FASTFACE_INPUT_N * sizeof(float));
    ff->d_output = (float*)ffk_malloc((size_t)batch * FASTFACE_OUTPUT_N * sizeof(float));
    ff->d_input_u8 = (uint8_t*)ffk_malloc((size_t)batch * FASTFACE_INPUT_N);
    if (!ff->d_input || !ff->d_output || !ff->d_input_u8) { free_activations(ff); return FFK_ERR_NOMEM; }
    /* one workspace per half of a split chain (each covers any batch up to
     * the capacity); a one-chain launch uses the first */
    const size_t ws = workspace_bytes(ff, batch);
    if (ws) {
        ff->d_ws = ffk_malloc(2 * ws);
        if (!ff->d_ws) { free_activations(ff); return FFK_ERR_NOMEM; }
        rc = ffk_zero(ff->d_ws, 2 * ws, ff->stream);
        if (!rc) rc = ffk_stream_sync(ff->stream);
        if (rc) { free_activations(ff); return rc; }
        ff->ws_part = ws;
    }
    ff->capacity = batch;
    memset(ff->io_cur, 0, sizeof ff->io_cur);
    return 0;
}

/* tensor t of a half whose region starts `off` bytes into every buffer.
 * The plan reuses a buffer for tensors of different sizes once the earlier
 * one is dead, and the two halves of a split chain run different layers at
 * the same time, so each half has its own region of every buffer: the
 * second starts after the first half's faces at the largest tensor size. */
static int8_t* tensor_ptr(FastFace* ff, int t, size_t off)
{
    if (t < 0) return NULL;
    const FfTensor* T = &ff->plan.tensors[t];
    if (T->buf < 0) return NULL;
    return ff->d_bufs[T->buf] + off;
}

/* conv descriptor of step s (pointers are NULL while no activations exist);
 * fmt 1: the input layer reads uint8 RGB pixels through the input table */
/* A conv over a tensor stored at its even pixels only (a 1x1 stride-2
 * shortcut) runs at stride 1 over the compact tensor. */
static int reads_even(const FastFace* ff, const FfStep* st)
{
    return st->kind == FF_STEP_CONV && st->t_in > FF_T_INPUT && ff->plan.tensors[st->t_in].even;
}

static int writes_even(const FastFace* ff, const FfStep* st)
{
    return st->kind == FF_STEP_CONV && st->t_out >= 0 && ff->plan.tensors[st->t_out].even;
}

/* part / off: the half of a split chain (0 or 1) and its region's offset
 * into every activation buffer; shared: the other half runs at the same
 * time (FFK_SHARED_GPU) */
static void step_desc(FastFace* ff, int s, int batch, int fmt, int part, size_t off, int shared, ffk_conv_desc* d)
{
    const FfStep* st = &ff->plan.steps[s];
    memset(d, 0, sizeof *d);
    d->batch = batch; d->cin = st->cin; d->cout = st->cout; d->kh = st->kh; d->kw = st->kw;
    d->stride = st->stride; d->pad = st->pad; d->hin = st->hin; d->win = st->win;
    if (reads_even(ff, st)) { d->stride = 1; d->hin = st->hin / 2; d->win = st->win / 2; }
    if (st->t_in == FF_T_INPUT) {
        d->in = NULL;
        d->io = ff->d_io + part;
        d->in_inv = ff->d_in_inv;
        if (fmt) d->in_lut = ff->d_in_lut;
    } else {
        d->in = ff->d_bufs ? tensor_ptr(ff, st->t_in, off) : NULL;
    }
    d->w = ff->d_weights + st->w_off;
    d->params = ff->d_params + st->p_off;
    if (ff->d_bufs) {
        d->add_src = tensor_ptr(ff, st->t_add, off);
        d->out = tensor_ptr(ff, st->t_out, off);
        d->out_bn = tensor_ptr(ff, st->t_bn, off);
    }
    if (st->flags & FFK_EPI_BN) d->bn_lut = ff->d_weights + st->lut_off;
    d->flags = step_flags(ff, st) | ((fmt && st->t_in == FF_T_INPUT) ? FFK_IN_RGB8 : 0) |
               (writes_even(ff, st) ? FFK_OUT_X_EVEN : 0);
    if (ff->algo == FASTFACE_CONV_WINOGRAD_F23 && st->wino_off != (size_t)-1) {
        d->flags |= FFK_ALGO_WINOGRAD;
        d->w = ff->d_weights + st->wino_off;
    }
    if (shared) d->flags |= FFK_SHARED_GPU;
    d->in_scale = st->in_scale;
    d->workspace = ff->d_ws ? (int8_t*)ff->d_ws + (size_t)part * ff->ws_part : NULL;
    d->workspace_bytes = ff->ws_part;
}

static int launch_step(FastFace* ff, int s, int batch, void* stream, int fmt, int part, size_t off, int shared)
{
    const FfStep* st = &ff->plan.steps[s];
    if (st->kind == FF_STEP_CONV) {
        ffk_conv_desc d;
        step_desc(ff, s, batch, fmt, part, off, shared, &d);
        return ffk_conv(&d, stream);
    }
    if (st->kind == FF_STEP_MAP || st->kind == FF_STEP_ADD) {   /* stand-alone BN / PReLU / Add */
        const long long pix = (long long)batch * st->hout * st->wout;
        const int8_t* lut = ff->d_weights + st->lut_off;
        if (st->kind == FF_STEP_MAP)
            return ffk_map_i8(tensor_ptr(ff, st->t_in, off), tensor_ptr(ff, st->t_out, off), pix, st->cout,
                              lut, stream);
        return ffk_add_i8(tensor_ptr(ff, st->t_in, off), tensor_ptr(ff, st->t_add, off),
                          tensor_ptr(ff, st->t_out, off), pix * st->cout, lut, stream);
    }
    ffk_fc_desc f;
    memset(&f, 0, sizeof f);
    f.batch = batch; f.n = st->fc_n; f.k = st->fc_k;
    f.a = tensor_ptr(ff, st->t_in, off);
    f.w = ff->d_weights + st->w_off;
    f.ws = ff->d_params + st->ws_off;
    f.bias = ff->d_params + st->bias_off;
    f.a_scale = st->a_scale;
    f.out = NULL;
    f.io = ff->d_io + part;
    f.path = 0;
    f.workspace = ff->d_ws ? (int8_t*)ff->d_ws + (size_t)part * ff->ws_part : NULL;
    f.workspace_bytes = ff->ws_part;
    return ffk_fc(&f, stream);
}

/* Steps s and s + 1 may run as one launch (ff_plan_pair: a stride-2 conv
 * and the shortcut adding its output; the buffer plan keeps the first step's
 * inputs out of the second's outputs); ffk_conv_s2_shortcut decides per
 * batch.  Not with every tensor kept for debug reads. */
static int pair_at(const FastFace* ff, int s)
{
    return !ff->keep_all && ff_plan_pair(&ff->plan, s);
}

/* the chain of `batch` faces as half `part`, its activations `off` bytes
 * into every buffer */
static int run_part(FastFace* ff, int part, size_t off, int batch, void* stream, int fmt, int shared)
{
    for (int s = 0; s < ff->plan.n_steps; s++) {
        if (!ff->no_fusion && pair_at(ff, s)) {
            ffk_conv_desc c, sc;
            step_desc(ff, s, batch, fmt, part, off, shared, &c);
            step_desc(ff, s + 1, batch, fmt, part, off, shared, &sc);
            const int r = ffk_conv_s2_shortcut(&c, &sc, stream);
            if (r < 0) return r;
            if (r == 1) { s++; continue; }
        }
        int rc = launch_step(ff, s, batch, stream, fmt, part, off, shared);
        if (rc) return rc;
    }
    return 0;
}

static int run_direct(FastFace* ff, int batch, void* stream, int fmt)
{
    return run_part(ff, 0, 0, batch, stream, fmt, 0);
}

/* The chain as captured: one, or two halves forked onto the second stream
 * and joined back (the join is recorded even after an error, so that the
 * capture can end). */
static int run_captured(FastFace* ff, int batch, int fmt)
{
    const int na = split_at(ff, batch);
    if (!na) return run_direct(ff, batch, ff->stream, fmt);
    int rc = ffk_event_record(ff->ev_fork, ff->stream);
    if (rc) return rc;
    rc = ffk_stream_wait_event(ff->sstream, ff->ev_fork);
    if (!rc) rc = run_part(ff, 0, 0, na, ff->stream, fmt, 1);
    if (!rc) rc = run_part(ff, 1, (size_t)na * ff->plan.max_face_bytes, batch - na, ff->sstream, fmt, 1);
    int rj = ffk_event_record(ff->ev_join, ff->sstream);
    if (!rj) rj = ffk_stream_wait_event(ff->stream, ff->ev_join);
    return rc ? rc : rj;
}

/* The captured chain for (batch, fmt), capturing it on first use.  A full
 * cache evicts round-robin, never the entries holding `keep` or `keep2`
 * (chains the caller is about to launch); an evicted chain may still be in
 * flight, so the context's work is waited for before it is destroyed. */
static void* graph_for(FastFace* ff, int batch, int fmt, const void* keep, const void* keep2)
{
    for (int i = 0; i < ff->n_graphs; i++)
        if (ff->graphs[i].batch == batch && ff->graphs[i].fmt == fmt) return ff->graphs[i].exec;
    if (ffk_graph_begin(ff->stream)) return NULL;
    int rc = run_captured(ff, batch, fmt);
    void* exec = NULL;
    int rc2 = ffk_graph_end(ff->stream, &exec);
    if (rc || rc2) { if (exec) ffk_graph_destroy(exec); return NULL; }
    int slot;
    if (ff->n_graphs < FF_MAX_GRAPHS) {
        slot = ff->n_graphs++;
    } else {
        slot = ff->graph_rr;
        while (ff->graphs[slot].exec == keep || ff->graphs[slot].exec == keep2) slot = (slot + 1) % FF_MAX_GRAPHS;
        ff->graph_rr = (slot + 1) % FF_MAX_GRAPHS;
        if (drain(ff) || ffk_stream_sync(ff->stream)) { ffk_graph_destroy(exec); return NULL; }
        ffk_graph_destroy(ff->graphs[slot].exec);
    }
    ff->graphs[slot].batch = batch;
    ff->graphs[slot].fmt = fmt;
    ff->graphs[slot].exec = exec;
    return exec;
}

/* Enqueue one batch whose I/O pointers are already in d_io: ordered after
 * the context's last enqueue (whatever stream that was on), then marked as
 * the new last one.  `exec`: a chain already looked up, or NULL. */
static int enqueue_exec(FastFace* ff, int batch, void* stream, int fmt, void* exec)
{
    int rc = order_after_last(ff, stream);
    if (rc) return rc;
    if (ff->keep_all) {
        rc = run_direct(ff, batch, stream, fmt);
    } else {
        void* g = exec ? exec : graph_for(ff, batch, fmt, NULL, NULL);
        rc = g ? ffk_graph_launch(g, stream) : FFK_ERR_HIP;
    }
    if (!rc) rc = mark_enqueued(ff, stream);
    return rc;
}

static int enqueue(FastFace* ff, int batch, void* stream, int fmt)
{
    return enqueue_exec(ff, batch, stream, fmt, NULL);
}

FastFace* fastface_create(const char* ffw4_path)
{
    return fastface_create_with_scales(ffw4_path, NULL, NULL);
}

FastFace* fastface_create_with_scales(const char* ffw4_path, const char* opsc_path,
                                      const char* opsc2_path)
{
    if (!ffw4_path) return NULL;
    if (ffk_device_count() <= 0) {
        fprintf(stderr, "fastface: no HIP device\n");
        return NULL;
    }
    FastFace* ff = (FastFace*)calloc(1, sizeof(FastFace));
    if (!ff) return NULL;
    const char* v2 = opsc2_path ? opsc2_path : getenv("OPSC2_PATH");
    if (!v2) v2 = "models/op_scales_v2.bin";
    if (ff_model_load(&ff->model, ffw4_path, opsc_path ? opsc_path : "models/op_scales.bin", v2) != 0) {
        free(ff);
        return NULL;
    }
    if (ff_plan_build(&ff->model, &ff->plan) != 0) {
        fprintf(stderr, "fastface: unsupported model: %s\n", ff->plan.err);
        goto fail;
    }
    ff_plan_assign_buffers(&ff->plan, 0);
    if (ffk_stream_create(&ff->stream)) { report("stream", FFK_ERR_HIP); goto fail; }
    ff->d_weights = (int8_t*)ffk_malloc(ff->plan.w_bytes);
    ff->d_params = (float*)ffk_malloc(ff->plan.p_floats * sizeof(float));
    ff->d_in_inv = (float*)ffk_malloc(4 * sizeof(float));
    ff->d_in_lut = (int8_t*)ffk_malloc(3 * 256);
    ff->d_io = (ffk_io*)ffk_malloc(2 * sizeof(ffk_io));
    ff->h_io = (ffk_io*)ffk_host_alloc(2 * (1 + FF_MAX_CHUNKS) * sizeof(ffk_io));
    if (ffk_stream_create(&ff->cstream)) { report("stream", FFK_ERR_HIP); goto fail; }
    if (ffk_stream_create(&ff->sstream)) { report("stream", FFK_ERR_HIP); goto fail; }
    if (ffk_event_create(&ff->ev_fork) || ffk_event_create(&ff->ev_join)) { report("event", FFK_ERR_HIP); goto fail; }
    for (int k = 0; k < FF_MAX_CHUNKS; k++)
        if (ffk_event_create(&ff->ev_chunk[k])) { report("event", FFK_ERR_HIP); goto fail; }
    if (ffk_event_create(&ff->ev_last)) { report("event", FFK_ERR_HIP); goto fail; }
    if (ffk_event_create(&ff->ev_stage[0]) || ffk_event_create(&ff->ev_stage[1])) {
        report("event", FFK_ERR_HIP);
        goto fail;
    }
    if (!ff->d_weights || !ff->d_params || !ff->d_in_inv || !ff->d_in_lut || !ff->d_io || !ff->h_io) {
        report("device allocation", FFK_ERR_NOMEM);
        goto fail;
    }
    int8_t in_lut[3 * 256];
    if (ffk_make_rgb8_lut(ff->plan.in_inv, in_lut) ||
        ffk_memcpy_h2d(ff->d_weights, ff->plan.w_host, ff->plan.w_bytes, ff->stream) ||
        ffk_memcpy_h2d(ff->d_params, ff->plan.p_host, ff->plan.p_floats * sizeof(float), ff->stream) ||
        ffk_memcpy_h2d(ff->d_in_inv, ff->plan.in_inv, 4 * sizeof(float), ff->stream) ||
        ffk_memcpy_h2d(ff->d_in_lut, in_lut, sizeof in_lut, ff->stream) ||
        ffk_stream_sync(ff->stream)) {
        report("weight upload", FFK_ERR_HIP);
        goto fail;
    }
    /* host copies of the packed weights are no longer needed */
    free(ff->plan.w_host); ff->plan.w_host = NULL;
    {
        const char* e = getenv("FASTFACE_MAX_BATCH");
        int reserve = e ? atoi(e) : 1;
        if (reserve < 1) reserve = 1;
        if (ensure_capacity(ff, reserve)) { report("activation allocation", FFK_ERR_NOMEM); goto fail; }
    }
    return ff;
fail:
    fastface_destroy(ff);
    return NULL;
}

void fastface_destroy(FastFace* ff)
{
    if (!ff) return;
    if (ff->ev_last) drain(ff);
    if (ff->stream) ffk_stream_sync(ff->stream);
    free_activations(ff);
    ffk_free(ff->d_weights);
    ffk_free(ff->d_params);
    ffk_free(ff->d_in_inv);
    ffk_free(ff->d_in_lut);
    ffk_free(ff->d_io);
    ffk_host_free(ff->h_io);
    if (ff->cstream) { ffk_stream_sync(ff->cstream); ffk_stream_destroy(ff->cstream); }
    if (ff->sstream) { ffk_stream_sync(ff->sstream); ffk_stream_destroy(ff->sstream); }
    if (ff->ev_fork) ffk_event_destroy(ff->ev_fork);
    if (ff->ev_join) ffk_event_destroy(ff->ev_join);
    for (int k = 0; k < FF_MAX_CHUNKS; k++)
        if (ff->ev_chunk[k]) ffk_event_destroy(ff->ev_chunk[k]);
    if (ff->ev_last) ffk_event_destroy(ff->ev_last);
    if (ff->stager) { stager_stop(ff->stager); free(ff->stager); }
    for (int b = 0; b < 2; b++) {
        if (ff->ev_stage[b]) ffk_event_destroy(ff->ev_stage[b]);
        if (ff->h_stage[b]) ffk_host_free(ff->h_stage[b]);
    }
    if (ff->h_small) ffk_host_free(ff->h_small);
    if (ff->stream) ffk_stream_destroy(ff->stream);
    ff_plan_free(&ff->plan);
    ff_model_free(&ff->model);
    free(ff);
}

int fastface_reserve(FastFace* ff, int max_batch)
{
    if (!ff || max_batch < 1) return -1;
    return ensure_capacity(ff, max_batch) ? -2 : 0;
}

void* fastface_stream(FastFace* ff) { return ff ? ff->stream : NULL; }

/* A batch from host memory (fmt 0: fp32 faces, 1: uint8 RGB; face_bytes
 * each) to host embeddings.  Up to one chunk: copy in, replay the chain,
 * copy out.  More: chunk k's copy goes to its own region of the input buffer
 * on the copy stream; the context stream waits for it, points the I/O
 * descriptor at the chunk (a pinned slot per chunk, so no staging slot is
 * rewritten while a copy may still read it) and replays the chain for the
 * chunk's size.  Faces are independent: the results equal the one-shot
 * path's bit for bit. */
/* Copy threads of a context's streamed host calls (started on first use,
 * idle between calls, stopped when the context is destroyed): the calling
 * thread and n - 1 workers each copy one slice of the current piece.  A
 * piece starts when the caller bumps `gen` and ends when every worker has
 * counted itself in `finished`. */
typedef struct { Stager* s; int i; } StageSlot;
struct Stager {
    int n;                              /* copying threads, the caller included */
    pthread_t th[FF_STAGE_THREADS];
    StageSlot slot[FF_STAGE_THREADS];
    pthread_mutex_t mu;
    pthread_cond_t cv_go, cv_done;
    unsigned gen;
    int finished, quit;
    const int8_t* src;
    int8_t* dst;
    size_t bytes;
};

static void stage_slice(Stager* s, int i)
{
    const size_t per = ((s->bytes + s->n - 1) / s->n + 63) & ~(size_t)63;
    const size_t a = (size_t)i * per;
    if (a < s->bytes) memcpy(s->dst + a, s->src + a, s->bytes - a < per ? s->bytes - a : per);
}

static void* stage_worker(void* arg)
{
    StageSlot* t = (StageSlot*)arg;
    Stager* s = t->s;
    unsigned seen = 0;
    pthread_mutex_lock(&s->mu);
    for (;;) {
        while (s->gen == seen && !s->quit) pthread_cond_wait(&s->cv_go, &s->mu);
        if (s->quit) break;
        seen = s->gen;
        pthread_mutex_unlock(&s->mu);
        stage_slice(s, t->i);
        pthread_mutex_lock(&s->mu);
        if (++s->finished == s->n - 1) pthread_cond_signal(&s->cv_done);
    }
    pthread_mutex_unlock(&s->mu);
    return NULL;
}

/* 0 with s->n >= 2 copying threads running, or -1 (nothing to stop) */
static int stager_start(Stager* s)
{
    const long ncpu = sysconf(_SC_NPROCESSORS_ONLN);
    const int want = ncpu < FF_STAGE_THREADS ? (int)ncpu : FF_STAGE_THREADS;
    if (want < 2) return -1;
    if (pthread_mutex_init(&s->mu, NULL)) return -1;
    if (pthread_cond_init(&s->cv_go, NULL)) { pthread_mutex_destroy(&s->mu); return -1; }
    if (pthread_cond_init(&s->cv_done, NULL)) {
        pthread_cond_destroy(&s->cv_go);
        pthread_mutex_destroy(&s->mu);
        return -1;
    }
    s->gen = 0; s->finished = 0; s->quit = 0;
    s->n = 1;
    for (int i = 1; i < want; i++) {           /* (workers see s->n only after a piece starts) */
        s->slot[i].s = s;
        s->slot[i].i = i;
        if (pthread_create(&s->th[i], NULL, stage_worker, &s->slot[i])) break;
        s->n = i + 1;
    }
    if (s->n < 2) {
        pthread_cond_destroy(&s->cv_done);
        pthread_cond_destroy(&s->cv_go);
        pthread_mutex_destroy(&s->mu);
        return -1;
    }
    return 0;
}

static void stager_copy(Stager* s, int8_t* dst, const int8_t* src, size_t bytes)
{
    pthread_mutex_lock(&s->mu);
    s->dst = dst; s->src = src; s->bytes = bytes;
    s->finished = 0;
    s->gen++;
    pthread_cond_broadcast(&s->cv_go);
    pthread_mutex_unlock(&s->mu);
    stage_slice(s, 0);
    pthread_mutex_lock(&s->mu);
    while (s->finished < s->n - 1) pthread_cond_wait(&s->cv_done, &s->mu);
    pthread_mutex_unlock(&s->mu);
}

static void stager_stop(Stager* s)
{
    pthread_mutex_lock(&s->mu);
    s->quit = 1;
    pthread_cond_broadcast(&s->cv_go);
    pthread_mutex_unlock(&s->mu);
    for (int i = 1; i < s->n; i++) pthread_join(s->th[i], NULL);
    pthread_cond_destroy(&s->cv_done);
    pthread_cond_destroy(&s->cv_go);
    pthread_mutex_destroy(&s->mu);
}

/* The context's staging buffers and copy threads, set up on first use, or
 * NULL if they cannot be (the caller's memory is then copied directly). */
static Stager* staging(FastFace* ff)
{
    if (!ff->h_stage[0]) ff->h_stage[0] = ffk_host_alloc(FF_STAGE_BYTES);
    if (ff->h_stage[0] && !ff->h_stage[1]) ff->h_stage[1] = ffk_host_alloc(FF_STAGE_BYTES);
    if (!ff->h_stage[1]) return NULL;
    if (!ff->stager) {
        Stager* sg = (Stager*)calloc(1, sizeof *sg);
        if (sg && stager_start(sg) == 0) ff->stager = sg;
        else free(sg);
    }
    return ff->stager;
}

/* The input bytes [off, off + bytes) of a streamed call to d_in + off, on
 * the copy stream: through the pinned staging buffers when the stager runs
 * (piece p in buffer p % 2, after the DMA that last read that buffer),
 * else as one copy from the caller's memory.  *piece counts the pieces. */
static int stage_h2d(FastFace* ff, Stager* st, int8_t* d_in, const int8_t* in, size_t off, size_t bytes,
                     int* piece)
{
    if (!st) return ffk_memcpy_h2d(d_in + off, in + off, bytes, ff->cstream);
    for (size_t o = off; o < off + bytes; o += FF_STAGE_BYTES) {
        const size_t len = off + bytes - o < FF_STAGE_BYTES ? off + bytes - o : FF_STAGE_BYTES;
        const int b = *piece & 1;
        if (*piece >= 2) {
            int rc = ffk_event_sync(ff->ev_stage[b]);
            if (rc) return rc;
        }
        stager_copy(st, (int8_t*)ff->h_stage[b], in + o, len);
        int rc = ffk_memcpy_h2d(d_in + o, ff->h_stage[b], len, ff->cstream);
        if (!rc) rc = ffk_event_record(ff->ev_stage[b], ff->cstream);
        if (rc) return rc;
        ++*piece;
    }
    return 0;
}

/* the pinned bounce buffer of small host batches, NULL if it cannot be
 * had (the copies then go from and to the caller's memory directly) */
static int8_t* small_buffer(FastFace* ff)
{
    if (!ff->h_small) ff->h_small = ffk_host_alloc(FF_SMALL_IN + FF_SMALL_OUT);
    return (int8_t*)ff->h_small;
}

static int embed_host(FastFace* ff, const void* in, size_t face_bytes, int fmt, int batch, float* out)
{
    /* a host call is synchronous: first let any device call still running
     * on a caller stream finish with the context's buffers */
    int rc = drain(ff);
    if (!rc) rc = ensure_capacity(ff, batch);
    if (rc) { report("activation allocation", rc); return -2; }
    int8_t* d_in = fmt ? (int8_t*)ff->d_input_u8 : (int8_t*)ff->d_input;
    const size_t out_bytes = (size_t)batch * FASTFACE_OUTPUT_N * sizeof(float);
    /* chunks: `first` faces, then `chunk`-face chunks, the last one the rest */
    const int first = fmt ? FF_STREAM_CHUNK_U8 : FF_STREAM_FIRST_F32;
    int chunk = fmt ? FF_STREAM_CHUNK_U8 : FF_STREAM_CHUNK_F32;
    const int streamed = batch > (fmt ? FF_STREAM_CHUNK_U8 : FF_STREAM_MIN_F32);
    if (streamed && batch - first > chunk * (FF_MAX_CHUNKS - 1))
        chunk = (batch - first + FF_MAX_CHUNKS - 2) / (FF_MAX_CHUNKS - 1);
    const int n = streamed ? 1 + (batch - first + chunk - 1) / chunk : 1;
    if (n < 2 || ff->keep_all) {
        /* one chunk: a large one still goes through the staging buffers */
        const size_t bytes = (size_t)batch * face_bytes;
        Stager* st = bytes >= FF_STAGE_MIN_BYTES ? staging(ff) : NULL;
        int piece = 0;
        rc = set_io(ff, d_in, ff->d_output, ff->stream, batch, fmt);
        if (!rc && st) {
            rc = stage_h2d(ff, st, d_in, (const int8_t*)in, 0, bytes, &piece);
            if (!rc) rc = ffk_event_record(ff->ev_chunk[0], ff->cstream);
            if (!rc) rc = ffk_stream_wait_event(ff->stream, ff->ev_chunk[0]);
            if (rc) ffk_stream_sync(ff->cstream);
        } else if (!rc) {
            int8_t* hs = bytes <= FF_SMALL_IN ? small_buffer(ff) : NULL;
            /* (the stream is idle here after a completed call; the sync
             * covers a call that failed with its copy still in flight) */
            if (hs) rc = ffk_stream_sync(ff->stream);
            if (!rc && hs) {
                memcpy(hs, in, bytes);
                rc = ffk_memcpy_h2d(d_in, hs, bytes, ff->stream);
            } else if (!rc) {
                rc = ffk_memcpy_h2d(d_in, in, bytes, ff->stream);
            }
        }
        if (!rc) rc = enqueue(ff, batch, ff->stream, fmt);
    } else {
        /* capture the (up to three) chains before any copy is issued (a
         * lookup may not evict the chains looked up before it), and launch
         * them directly */
        const int last = batch - first - (n - 2) * chunk;
        void* g_first = graph_for(ff, first, fmt, NULL, NULL);
        void* g_chunk = g_first && n > 2 ? graph_for(ff, chunk, fmt, g_first, NULL) : g_first;
        void* g_last = g_chunk ? graph_for(ff, last, fmt, g_first, g_chunk) : NULL;
        if (!g_first || !g_chunk || !g_last) rc = FFK_ERR_HIP;
        Stager* st = rc ? NULL : staging(ff);
        int piece = 0;
        for (int k = 0; k < n && !rc; k++) {
            const size_t b0 = k ? (size_t)first + (size_t)(k - 1) * chunk : 0;
            const int nb = k == 0 ? first : (k + 1 < n ? chunk : last);
            rc = stage_h2d(ff, st, d_in, (const int8_t*)in, b0 * face_bytes, (size_t)nb * face_bytes, &piece);
            if (!rc) rc = ffk_event_record(ff->ev_chunk[k], ff->cstream);
            if (!rc) rc = ffk_stream_wait_event(ff->stream, ff->ev_chunk[k]);
            ffk_io* slot = &ff->h_io[2 * (1 + k)];
            io_pair(ff, slot, d_in + b0 * face_bytes, ff->d_output + b0 * FASTFACE_OUTPUT_N, nb, fmt);
            if (!rc) rc = ffk_memcpy_h2d(ff->d_io, slot, 2 * sizeof(ffk_io), ff->stream);
            if (!rc) rc = enqueue_exec(ff, nb, ff->stream, fmt, k == 0 ? g_first : (k + 1 < n ? g_chunk : g_last));
            if (!rc) memcpy(ff->io_cur, slot, sizeof ff->io_cur);
        }
        if (rc) {           /* leave no copy or chunk running into the buffers */
            ffk_stream_sync(ff->cstream);
            ffk_stream_sync(ff->stream);
            memset(ff->io_cur, 0, sizeof ff->io_cur);
        }
    }
    int8_t* ho = out_bytes <= FF_SMALL_OUT ? small_buffer(ff) : NULL;
    if (ho) ho += FF_SMALL_IN;
    if (!rc) rc = ffk_memcpy_d2h(ho ? (void*)ho : (void*)out, ff->d_output, out_bytes, ff->stream);
    if (!rc) rc = ffk_stream_sync(ff->stream);
    if (!rc && ho) memcpy(out, ho, out_bytes);
    if (!rc) ff->last_stream = NULL;        /* all of it has finished */
    if (rc) { report("embed", rc); return -3; }
    return 0;
}

int fastface_embed_batch(FastFace* ff, const float* in, int batch, float* out)
{
    if (!ff || !in || !out || batch < 0) return -1;
    if (batch == 0) return 0;
    return embed_host(ff, in, FASTFACE_INPUT_N * sizeof(float), 0, batch, out);
}

int fastface_embed(FastFace* ff, const float* input_hwc, float* out_emb)
{
    if (!ff || !input_hwc || !out_emb) return -1;
    return fastface_embed_batch(ff, input_hwc, 1, out_emb);
}

int fastface_embed_batch_device(FastFace* ff, const float* d_in, int batch, float* d_out, void* stream)
{
    if (!ff || !d_in || !d_out || batch < 0) return -1;
    if (batch == 0) return 0;
    if (!stream) stream = ff->stream;
    int rc = ensure_capacity(ff, batch);
    if (rc) { report("activation allocation", rc); return -2; }
    rc = set_io(ff, d_in, d_out, stream, batch, 0);
    if (!rc) rc = enqueue(ff, batch, stream, 0);
    if (rc) { report("embed_batch_device", rc); return -3; }
    return 0;
}

int fastface_embed_batch_rgb8(FastFace* ff, const uint8_t* in, int batch, float* out)
{
    if (!ff || !in || !out || batch < 0) return -1;
    if (batch == 0) return 0;
    return embed_host(ff, in, FASTFACE_INPUT_N, 1, batch, out);
}

int fastface_embed_batch_rgb8_device(FastFace* ff, const uint8_t* d_in, int batch, float* d_out,
                                     void* stream)
{
    if (!ff || !d_in || !d_out || batch < 0) return -1;
    if (batch == 0) return 0;
    if (!stream) stream = ff->stream;
    int rc = ensure_capacity(ff, batch);
    if (rc) { report("activation allocation", rc); return -2; }
    rc = set_io(ff, d_in, d_out, stream, batch, 1);
    if (!rc) rc = enqueue(ff, batch, stream, 1);
    if (rc) { report("embed_batch_rgb8_device", rc); return -3; }
    return 0;
}

int fastface_set_conv_algo(FastFace* ff, int algo)
{
    if (!ff || (algo != FASTFACE_CONV_DIRECT && algo != FASTFACE_CONV_WINOGRAD_F23)) return -1;
    int n = 0;
    if (algo == FASTFACE_CONV_WINOGRAD_F23)
        for (int s = 0; s < ff->plan.n_steps; s++)
            if (ff->plan.steps[s].kind == FF_STEP_CONV && ff->plan.steps[s].wino_off != (size_t)-1) n++;
    if (algo == ff->algo) return n;
    if (drain(ff) || ffk_stream_sync(ff->stream)) return -2;
    /* other launch chains, and another workspace size */
    const int cap = ff->capacity;
    free_activations(ff);
    ff->algo = algo;
    return ensure_capacity(ff, cap > 0 ? cap : 1) ? -2 : n;
}

int fastface_set_shortcut_fusion(FastFace* ff, int on)
{
    if (!ff || (on != 0 && on != 1)) return -1;
    int n = 0;
    for (int s = 0; s < ff->plan.n_steps; s++) n += pair_at(ff, s);
    if (on == !ff->no_fusion) return n;
    if (drain(ff) || ffk_stream_sync(ff->stream)) return -2;
    const int cap = ff->capacity;
    free_activations(ff);                 /* (the captured chains hold the old launches) */
    ff->no_fusion = !on;
    return ensure_capacity(ff, cap > 0 ? cap : 1) ? -2 : n;
}

int fastface_set_epilogue_forms(FastFace* ff, int general)
{
    if (!ff || (general != 0 && general != 1)) return -1;
    int n = 0;
    for (int s = 0; s < ff->plan.n_steps; s++)
        if (ff->plan.steps[s].kind == FF_STEP_CONV && (ff->plan.steps[s].flags & FF_FAST_EPI)) n++;
    if (general == ff->general_epi) return n;
    if (drain(ff) || ffk_stream_sync(ff->stream)) return -2;
    const int cap = ff->capacity;
    free_activations(ff);                 /* (the captured chains hold the old flags) */
    ff->general_epi = general;
    return ensure_capacity(ff, cap > 0 ? cap : 1) ? -2 : n;
}

int fastface_num_steps(const FastFace* ff) { return ff ? ff->plan.n_steps : -1; }

int fastface_get_step(const FastFace* ff, int s, fastface_step_info* info)
{
    if (!ff || !info || s < 0 || s >= ff->plan.n_steps) return -1;
    const FfStep* st = &ff->plan.steps[s];
    memset(info, 0, sizeof *info);
    info->kind = st->kind;
    info->op_first = st->op_first;
    info->op_last = st->op_last;
    if (st->kind == FF_STEP_CONV) {
        info->cin = st->cin; info->cout = st->cout; info->kh = st->kh; info->kw = st->kw;
        /* the geometry and flags of the launch (step_desc) */
        const int ev_in = reads_even(ff, st), ev_out = writes_even(ff, st);
        info->stride = ev_in ? 1 : st->stride; info->pad = st->pad;
        info->hin = ev_in ? st->hin / 2 : st->hin; info->win = ev_in ? st->win / 2 : st->win;
        info->hout = st->hout; info->wout = st->wout;
        info->flags = step_flags(ff, st) | (ev_out ? FFK_OUT_X_EVEN : 0);
        if (ff->algo == FASTFACE_CONV_WINOGRAD_F23 && st->wino_off != (size_t)-1)
            info->flags |= FFK_ALGO_WINOGRAD;
        info->stores_x = st->t_out >= 0;
        const double pix_out = (double)st->hout * st->wout;
        info->ops_per_face = 2.0 * pix_out * st->cout * st->kh * st->kw * st->cin;
        /* distinct input pixels a kernel must read */
        double pix_in = (st->kh == 1) ? pix_out : (double)st->hin * st->win;
        double in_bytes = pix_in * st->cin * (st->cin == 3 ? 4.0 : 1.0);
        double out_b = pix_out * st->cout;
        const double x_b = st->t_out < 0 ? 0.0 : (ev_out ? 0.25 : 1.0);
        info->act_bytes_per_face = in_bytes + out_b * (x_b + (st->t_bn >= 0) + (st->t_add >= 0));
        info->weight_bytes = (double)ffk_conv_packed_bytes(st->cin, st->cout, st->kh, st->kw);
    } else if (st->kind == FF_STEP_MAP || st->kind == FF_STEP_ADD) {
        info->cin = info->cout = st->cout; info->kh = info->kw = 1; info->stride = 1;
        info->hin = info->hout = st->hout; info->win = info->wout = st->wout;
        info->stores_x = 1;
        const double bytes = (double)st->hout * st->wout * st->cout;
        info->act_bytes_per_face = bytes * (st->kind == FF_STEP_ADD ? 3.0 : 2.0);
        info->weight_bytes = st->kind == FF_STEP_ADD ? 65536.0 : 256.0 * st->cout;
    } else {
        info->cin = st->fc_k; info->cout = st->fc_n; info->kh = info->kw = 1; info->stride = 1;
        info->hin = info->win = info->hout = info->wout = 1;
        info->ops_per_face = 2.0 * st->fc_k * st->fc_n;
        info->act_bytes_per_face = st->fc_k + 4.0 * st->fc_n;
        info->weight_bytes = (double)st->fc_k * st->fc_n;
    }
    return 0;
}

int fastface_profile_steps(FastFace* ff, int batch, int reps, float* step_ms)
{
    if (!ff || !step_ms || batch < 1 || reps < 1) return -1;
    int rc = drain(ff);
    if (!rc) rc = ensure_capacity(ff, batch);
    if (!rc) rc = set_io(ff, ff->d_input, ff->d_output, ff->stream, batch, 0);
    if (rc) return -2;
    const int n = ff->plan.n_steps;
    void** ev = (void**)calloc((size_t)n + 1, sizeof(void*));
    for (int s = 0; s <= n && !rc; s++) rc = ffk_event_create(&ev[s]);
    for (int s = 0; s < n; s++) step_ms[s] = 0.0f;
    for (int r = 0; r < reps && !rc; r++) {
        for (int s = 0; s < n && !rc; s++) {
            rc = ffk_event_record(ev[s], ff->stream);
            if (!rc) rc = launch_step(ff, s, batch, ff->stream, 0, 0, 0, 0);
        }
        if (!rc) rc = ffk_event_record(ev[n], ff->stream);
        if (!rc) rc = ffk_stream_sync(ff->stream);
        for (int s = 0; s < n && !rc; s++) {
            float ms = 0.0f;
            rc = ffk_event_elapsed_ms(ev[s], ev[s + 1], &ms);
            step_ms[s] += ms / (float)reps;
        }
    }
    for (int s = 0; s <= n; s++) if (ev[s]) ffk_event_destroy(ev[s]);
    free(ev);
    if (rc) { report("profile", rc); ffk_stream_sync(ff->stream); return -3; }
    return n;
}

int fastface_debug_keep_tensors(FastFace* ff, int on)
{
    if (!ff) return -1;
    int rc = drain(ff);
    if (!rc) rc = ffk_stream_sync(ff->stream);
    if (rc) return -3;
    int cap = ff->capacity;
    free_activations(ff);
    ff->keep_all = on ? 1 : 0;
    ff_plan_assign_buffers(&ff->plan, ff->keep_all);
    return ensure_capacity(ff, cap > 0 ? cap : 1) ? -2 : 0;
}

long long fastface_debug_read(FastFace* ff, int op_idx, int batch, void* host, size_t bytes)
{
    if (!ff || !host || batch < 1 || batch > ff->capacity) return -1;
    for (int t = ff->plan.n_tensors - 1; t > 0; t--) {
        const FfTensor* T = &ff->plan.tensors[t];
        if (T->op != op_idx || T->buf < 0) continue;
        size_t n = (size_t)T->C * T->H * T->W * (size_t)batch;
        if (n > bytes) return -4;
        if (drain(ff)) return -3;
        if (ffk_memcpy_d2h(host, ff->d_bufs[T->buf], n, ff->stream) || ffk_stream_sync(ff->stream))
            return -3;
        return (long long)n;
    }
    return -5;
}
