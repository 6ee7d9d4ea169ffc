/* ff_loader_check.c -- host-only driver of the model loader and the launch
 * planner (ff_model.c, ff_plan.c), built with AddressSanitizer and
 * UndefinedBehaviorSanitizer by `make -C fastface_amd/csrc san` for the CPU
 * tests, which feed it valid, truncated and corrupt weight and scale files.
 * It needs no GPU: the planner's packing and table helpers are host
 * functions of the library.
 *
 *   ff_loader_check <weights.ffw> <op_scales.bin> [<op_scales_v2.bin> | -]
 *
 * Prints "load <rc> version <v> ops <n> v2 <has_v2>" and, when the load
 * succeeded, "plan <rc> steps <n> buffers <n> weights <bytes>"; exits 0 (a
 * sanitizer finding aborts with its report and a non-zero status). */
#include <stdio.h>
#include <string.h>

#include "ff_host.h"

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
    ff_plan_free(&p);
    ff_model_free(&m);
    return 0;
}
