/* ff_loader_check.c -- host-only driver of the model loader and the launch
 * planner (ff_model.c, ff_plan.c), built with AddressSanitizer and
 * UndefinedBehaviorSanitizer by `make -C fastface_amd/csrc san` for the CPU
 * tests, which feed it valid, truncated and corrupt weight and scale files.
 * It needs no GPU: the planner's packing and table helpers are host
 * functions of the library.
 *
 *   ff_loader_check <weights.ffw> <op_scales.bin> [<op_scales_v2.bin> | -] [<dump> | -]
 *                   [--launches <batch> ...]
 *
 * Prints "load <rc> version <v> ops <n> v2 <has_v2>" and, when the load
 * succeeded, "plan <rc> steps <n> buffers <n> weights <bytes>" and
 * "pairs <n> overlaps <n>": the steps that may run fused with the next one
 * (ff_plan_pair: a stride-2 conv and the shortcut adding its output, one
 * launch) and how many of them let the second step write a buffer the pair
 * still reads (its own input, the first step's input or output), which must
 * be none; "in_range <n> fma_tail <n> fma_bad <n>": the conv launches with
 * FFK_EPI_IN_RANGE and with FFK_EPI_FMA_TAIL, and those of the latter
 * without the former or with a residual / in-scale (must be none); exits 0
 * (a sanitizer finding aborts with its report and a
 * non-zero status).  With <dump>, the plan's weight arena goes to <dump>.bin
 * and, one line per region, "conv|wino|bn|map|add|fc <op> <offset> <bytes>" to
 * <dump>.txt, and the parameter arena to <dump>.params.bin.  With
 * --launches, the launch list of the chain at each batch, one line per
 * launch ("launch <batch>[/h<half>] <step> conv|fc <variant> <workgroups>
 * <geometry> <flags>", or "... map|add <channels> <pixels>" for a
 * stand-alone BN / PReLU / Add), built as fastface.c builds its descriptors (two
 * halves from 24 faces, FFK_SHARED_GPU) from the library's host-side
 * launch choice: no device is involved. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ff_host.h"

/* the chain of one half (or the whole batch) as fastface.c's run_part
 * launches it: conv descriptors as step_desc builds them, with a workspace
 * large enough for any split the launch may take */
static void print_launches(const FfPlan* p, const char* tag, int batch, int shared)
{
    for (int s = 0; s < p->n_steps; s++) {
        const FfStep* st = &p->steps[s];
        if (st->kind == FF_STEP_FC) {
            ffk_fc_desc f;
            memset(&f, 0, sizeof f);
            f.batch = batch; f.n = st->fc_n; f.k = st->fc_k;
            printf("launch %s %d fc %s %zu\n", tag, s, batch <= 16 ? "matvec" : "gemm", ffk_fc_workspace_bytes(&f));
            continue;
        }
        if (st->kind == FF_STEP_MAP || st->kind == FF_STEP_ADD) {
            printf("launch %s %d %s %d %lld\n", tag, s, st->kind == FF_STEP_MAP ? "map" : "add", st->cout,
                   (long long)batch * st->hout * st->wout);
            continue;
        }
        ffk_conv_desc d;
        memset(&d, 0, sizeof d);
        d.batch = batch; d.cin = st->cin; d.cout = st->cout; d.kh = st->kh; d.kw = st->kw;
        d.stride = st->stride; d.pad = st->pad; d.hin = st->hin; d.win = st->win;
        if (st->t_in > FF_T_INPUT && p->tensors[st->t_in].even) {     /* 1x1 s2 over a compact X */
            d.stride = 1; d.hin = st->hin / 2; d.win = st->win / 2;
        }
        d.flags = st->flags | ((st->t_out >= 0 && p->tensors[st->t_out].even) ? FFK_OUT_X_EVEN : 0) |
                  (shared ? FFK_SHARED_GPU : 0);
        d.workspace = (void*)(uintptr_t)4096;            /* (never dereferenced) */
        d.workspace_bytes = (size_t)1 << 30;
        const char* v = ffk_conv_variant(&d);
        printf("launch %s %d conv %s %d %d->%d k%d s%d @%d flags 0x%x\n", tag, s, v ? v : "none",
               ffk_conv_grid(&d), d.cin, d.cout, d.kh, d.stride, d.hin, d.flags);
    }
}

int main(int argc, char** argv)
{
    if (argc < 3) {
        fprintf(stderr, "usage: %s <ffw> <opsc> [<opsc2>|-]\n", argv[0]);
        return 2;
    }
    const char* v2 = (argc > 3 && strcmp(argv[3], "-") != 0) ? argv[3] : NULL;
    FfModel m;
    const int rc = ff_model_load(&m, argv[1], argv[2], v2);
    printf("load %d version %d ops %d v2 %d\n", rc, rc ? 0 : m.version, rc ? 0 : m.n_ops,
           rc ? 0 : m.has_v2);
    if (rc) return 0;
    FfPlan p;
    const int prc = ff_plan_build(&m, &p);
    if (!prc) ff_plan_assign_buffers(&p, 0);
    printf("plan %d steps %d buffers %d weights %zu%s%s\n", prc, prc ? 0 : p.n_steps,
           prc ? 0 : p.n_buffers, prc ? (size_t)0 : p.w_bytes, prc ? " err " : "", prc ? p.err : "");
    if (!prc) {
        int pairs = 0, overlaps = 0;
        for (int s = 0; s < p.n_steps; s++) {
            if (!ff_plan_pair(&p, s)) continue;
            const FfStep* a = &p.steps[s];
            const FfStep* b = &p.steps[s + 1];
            const int reads[3] = { a->t_in, b->t_in, a->t_out };
            const int writes[2] = { b->t_out, b->t_bn };
            pairs++;
            for (int w = 0; w < 2; w++)
                for (int r = 0; r < 3; r++)
                    if (writes[w] >= 0 && reads[r] >= 0 &&
                        p.tensors[writes[w]].buf == p.tensors[reads[r]].buf)
                        overlaps++;
        }
        printf("pairs %d overlaps %d\n", pairs, overlaps);
        int in_range = 0, fma = 0, fma_bad = 0;
        for (int s = 0; s < p.n_steps; s++) {
            const int f = p.steps[s].flags;
            if (p.steps[s].kind != FF_STEP_CONV) continue;
            in_range += (f & FFK_EPI_IN_RANGE) != 0;
            if (f & FFK_EPI_FMA_TAIL) {
                fma++;
                fma_bad += !(f & FFK_EPI_IN_RANGE) || (f & (FFK_EPI_ADD | FFK_EPI_INSCALE));
            }
        }
        printf("in_range %d fma_tail %d fma_bad %d\n", in_range, fma, fma_bad);
    }
    int la = 0;                                         /* first --launches batch */
    for (int i = 4; i < argc; i++)
        if (strcmp(argv[i], "--launches") == 0) { la = i + 1; break; }
    if (!prc && la)
        for (int i = la; i < argc; i++) {
            const int b = atoi(argv[i]);
            char tag[48];
            if (b <= 0) continue;
            if (b >= 24) {                                  /* fastface.c FF_SPLIT_MIN: two halves */
                snprintf(tag, sizeof tag, "%d/h0", b); print_launches(&p, tag, b / 2, 1);
                snprintf(tag, sizeof tag, "%d/h1", b); print_launches(&p, tag, b - b / 2, 1);
            } else {
                snprintf(tag, sizeof tag, "%d", b); print_launches(&p, tag, b, 0);
            }
        }
    if (!prc && argc > 4 && strcmp(argv[4], "-") != 0 && strcmp(argv[4], "--launches") != 0) {
        char path[4096];
        snprintf(path, sizeof path, "%s.bin", argv[4]);
        FILE* f = fopen(path, "wb");
        if (f) { fwrite(p.w_host, 1, p.w_bytes, f); fclose(f); }
        snprintf(path, sizeof path, "%s.params.bin", argv[4]);
        f = fopen(path, "wb");
        if (f) { fwrite(p.p_host, sizeof(float), p.p_floats, f); fclose(f); }
        snprintf(path, sizeof path, "%s.txt", argv[4]);
        f = fopen(path, "w");
        if (f) {
            for (int s = 0; s < p.n_steps; s++) {
                const FfStep* st = &p.steps[s];
                if (st->kind == FF_STEP_FC) {
                    fprintf(f, "fc %d %zu %zu\n", st->op_first, st->w_off, ffk_fc_packed_bytes(st->fc_n, st->fc_k));
                    continue;
                }
                if (st->kind == FF_STEP_MAP || st->kind == FF_STEP_ADD) {
                    fprintf(f, "%s %d %zu %zu %zu\n", st->kind == FF_STEP_MAP ? "map" : "add", st->op_first,
                            st->lut_off, st->kind == FF_STEP_MAP ? (size_t)st->cout * 256 : (size_t)65536,
                            st->p_off);
                    continue;
                }
                fprintf(f, "conv %d %zu %zu\n", st->op_first, st->w_off,
                        ffk_conv_packed_bytes(st->cin, st->cout, st->kh, st->kw));
                if (st->wino_off != (size_t)-1)
                    fprintf(f, "wino %d %zu %zu\n", st->op_first, st->wino_off,
                            ffk_winograd_packed_bytes(st->cin, st->cout));
                if (st->flags & FFK_EPI_BN)
                    fprintf(f, "bn %d %zu %zu %zu\n", st->op_first, st->lut_off, (size_t)st->cout * 256, st->p_off);
            }
            fclose(f);
        }
    }
    ff_plan_free(&p);
    ff_model_free(&m);
    return 0;
}
