/* ff_model.c -- FFW2/3/4 weights (mmapped) and OPSC / OPSC2 scale files.
 *
 * Acceptance rules follow the reference: kernels/ffw2_loader.c:71-159
 * (magic -> version, op parsing, unknown op type is an error) and
 * libfastface.c:133-204 (OPSC mandatory with n_ops equal to the model's;
 * OPSC2 optional, inverses precomputed as 1/(s + 1e-9f) in fp32).
 * Unlike the reference, every read is bounds-checked against the file size.
 */
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include "ff_host.h"

float ff_read_f32(const uint8_t* p, int i)
{
    float v;
    memcpy(&v, p + 4 * (size_t)i, 4);
    return v;
}

typedef struct { const uint8_t* p; const uint8_t* end; int bad; } Cur;

static const uint8_t* take(Cur* c, size_t n)
{
    if (c->bad || (size_t)(c->end - c->p) < n) { c->bad = 1; return NULL; }
    const uint8_t* r = c->p;
    c->p += n;
    return r;
}
static uint32_t take_u32(Cur* c) { uint32_t v = 0; const uint8_t* q = take(c, 4); if (q) memcpy(&v, q, 4); return v; }
static uint16_t take_u16(Cur* c) { uint16_t v = 0; const uint8_t* q = take(c, 2); if (q) memcpy(&v, q, 2); return v; }
static uint8_t take_u8(Cur* c) { const uint8_t* q = take(c, 1); return q ? *q : 0; }

static int parse_ffw(FfModel* m)
{
    Cur c = { (const uint8_t*)m->map, (const uint8_t*)m->map + m->size, 0 };
    const uint8_t* magic = take(&c, 4);
    if (!magic) return -3;
    if (memcmp(magic, "FFW4", 4) == 0) m->version = 4;
    else if (memcmp(magic, "FFW3", 4) == 0) m->version = 3;
    else if (memcmp(magic, "FFW2", 4) == 0) m->version = 2;
    else return -3;
    uint32_t n = take_u32(&c);
    if (c.bad || n == 0 || n > 100000) return -3;
    m->n_ops = (int)n;
    m->ops = (FfOp*)calloc(n, sizeof(FfOp));
    if (!m->ops) return -5;
    for (uint32_t i = 0; i < n; i++) {
        FfOp* op = &m->ops[i];
        op->type = take_u8(&c);
        switch (op->type) {
        case FF_OP_CONV:
            op->Cin = take_u16(&c); op->Cout = take_u16(&c); op->Kh = take_u16(&c);
            op->Kw = take_u16(&c); op->stride = take_u16(&c); op->pad = take_u16(&c);
            op->conv_w = (const int8_t*)take(&c, (size_t)op->Cout * op->Cin * op->Kh * op->Kw);
            op->conv_scales = take(&c, (size_t)op->Cout * 4);
            if (m->version >= 3) op->conv_bias = take(&c, (size_t)op->Cout * 4);
            break;
        case FF_OP_BN:
            op->bn_size = take_u16(&c);
            op->bn_scale = take(&c, (size_t)op->bn_size * 4);
            op->bn_offset = take(&c, (size_t)op->bn_size * 4);
            break;
        case FF_OP_PRELU:
            op->prelu_size = take_u16(&c);
            op->prelu_slope = take(&c, (size_t)op->prelu_size * 4);
            break;
        case FF_OP_ADD: case FF_OP_FLATTEN: case FF_OP_SAVE_ID: case FF_OP_BLOCK_START:
            break;
        case FF_OP_GEMM:
            op->N = take_u32(&c); op->K = take_u32(&c);
            op->gemm_w = (const int8_t*)take(&c, (size_t)op->N * op->K);
            op->gemm_scales = take(&c, (size_t)op->N * 4);
            op->gemm_bias = take(&c, (size_t)op->N * 4);
            break;
        default:
            fprintf(stderr, "fastface: bad op type %d at op %u\n", op->type, i);
            return -4;
        }
        if (c.bad) { fprintf(stderr, "fastface: truncated weights file at op %u\n", i); return -4; }
    }
    return 0;
}

static uint8_t* slurp(const char* path, size_t* n)
{
    FILE* f = fopen(path, "rb");
    if (!f) return NULL;
    if (fseek(f, 0, SEEK_END) != 0) { fclose(f); return NULL; }
    long sz = ftell(f);
    if (sz < 0 || fseek(f, 0, SEEK_SET) != 0) { fclose(f); return NULL; }
    uint8_t* b = (uint8_t*)malloc((size_t)sz + 1);
    if (b && fread(b, 1, (size_t)sz, f) != (size_t)sz) { free(b); b = NULL; }
    fclose(f);
    *n = (size_t)sz;
    return b;
}

static int load_opsc(FfModel* m, const char* path)
{
    size_t n = 0;
    uint8_t* d = slurp(path, &n);
    if (!d) { fprintf(stderr, "open %s fail\n", path); return -1; }
    Cur c = { d, d + n, 0 };
    const uint8_t* magic = take(&c, 4);
    if (!magic || memcmp(magic, "OPSC", 4) != 0) { free(d); return -2; }
    uint32_t n_ops = take_u32(&c);
    const uint8_t* in = take(&c, 4);
    const uint8_t* arr = take(&c, (size_t)n_ops * 4);
    if (c.bad) { free(d); return -2; }
    memcpy(&m->input_scale, in, 4);
    m->scales = (float*)malloc((size_t)(n_ops ? n_ops : 1) * sizeof(float));
    memcpy(m->scales, arr, (size_t)n_ops * 4);
    free(d);
    return (int)n_ops == m->n_ops ? 0 : -3;
}

static int load_opsc2(FfModel* m, const char* path)
{
    size_t n = 0;
    uint8_t* d = slurp(path, &n);
    if (!d) return -1;
    Cur c = { d, d + n, 0 };
    const uint8_t* magic = take(&c, 5);
    if (!magic || memcmp(magic, "OPSC2", 5) != 0) { free(d); return -2; }
    uint32_t n_ops = take_u32(&c);
    if ((int)n_ops != m->n_ops) {
        fprintf(stderr, "OPSC2 n_ops mismatch: %u vs expected %d\n", n_ops, m->n_ops);
        free(d); return -3;
    }
    uint32_t n_in = take_u32(&c);
    const uint8_t* in = take(&c, (size_t)n_in * 4);
    if (c.bad || n_in > 64) { free(d); return -2; }
    m->n_in = (int)n_in;
    m->in_scale_pc = (float*)calloc(n_in + 1, sizeof(float));
    m->in_inv_pc = (float*)calloc(n_in + 1, sizeof(float));
    for (uint32_t i = 0; i < n_in; i++) {
        m->in_scale_pc[i] = ff_read_f32(in, (int)i);
        m->in_inv_pc[i] = 1.0f / (m->in_scale_pc[i] + 1e-9f);
    }
    m->pc_len = (uint32_t*)calloc(n_ops, sizeof(uint32_t));
    m->inv_pc = (float**)calloc(n_ops, sizeof(float*));
    m->scale_pc = (float**)calloc(n_ops, sizeof(float*));
    for (uint32_t i = 0; i < n_ops; i++) {
        uint32_t nch = take_u32(&c);
        const uint8_t* v = take(&c, (size_t)nch * 4);
        if (c.bad || nch > 32768) { free(d); return -4; }
        m->pc_len[i] = nch;
        if (nch == 0) continue;
        m->inv_pc[i] = (float*)malloc(nch * sizeof(float));
        m->scale_pc[i] = (float*)malloc(nch * sizeof(float));
        for (uint32_t k = 0; k < nch; k++) {
            float s = ff_read_f32(v, (int)k);
            m->scale_pc[i][k] = s;
            m->inv_pc[i][k] = 1.0f / (s + 1e-9f);
        }
    }
    free(d);
    m->has_v2 = 1;
    fprintf(stderr, "OPSC2: loaded per-channel scales (input_pc_ch=%u)\n", n_in);
    return 0;
}

void ff_model_free(FfModel* m)
{
    if (!m) return;
    if (m->map && m->map != MAP_FAILED) munmap(m->map, m->size);
    if (m->inv_pc)
        for (int i = 0; i < m->n_ops; i++) { free(m->inv_pc[i]); free(m->scale_pc[i]); }
    free(m->ops); free(m->scales); free(m->in_scale_pc); free(m->in_inv_pc);
    free(m->pc_len); free(m->inv_pc); free(m->scale_pc);
    memset(m, 0, sizeof *m);
}

int ff_model_load(FfModel* m, const char* ffw_path, const char* opsc_path, const char* opsc2_path)
{
    memset(m, 0, sizeof *m);
    int fd = open(ffw_path, O_RDONLY);
    if (fd < 0) { fprintf(stderr, "open fail\n"); return -1; }
    struct stat st;
    if (fstat(fd, &st) < 0 || st.st_size <= 0) { close(fd); return -1; }
    m->size = (size_t)st.st_size;
    m->map = mmap(NULL, m->size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m->map == MAP_FAILED) { m->map = NULL; return -2; }
    int rc = parse_ffw(m);
    if (rc) { ff_model_free(m); return rc; }
    rc = load_opsc(m, opsc_path);
    if (rc) { ff_model_free(m); return -10 + rc; }
    if (opsc2_path) load_opsc2(m, opsc2_path);      /* optional */
    return 0;
}
