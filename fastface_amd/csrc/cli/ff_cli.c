/* ff_cli.c -- wire-compatible replacements for the reference's CLIs
 * fastface_int8 (arcface_forward_int8.c:206-562) and fastface_int8_batched
 * (arcface_forward_int8_batched.c:206-600, built with -DFF_CLI_BATCHED), on
 * top of the fastface.h library.  The SDKs (fastface.py:77-90,
 * go/fastface/fastface.go:95) spawn these with --server and stream raw fp32
 * frames, so they run unchanged against the GPU.
 *
 *   <prog> [weights.ffw4] [--in IN --out OUT] [--server] [--threads N]
 *          [--batch N]            (batched build; env BATCH overrides)
 *
 * Modes and exit codes follow the reference:
 *   --in/--out : embed the B faces of IN (raw fp32), write B*512 fp32 to OUT;
 *                an unreadable IN exits 2.
 *   --server   : loop { read B*37632 fp32 from stdin; write B*512 fp32 to
 *                stdout; flush }.  EOF before a frame exits 0, a partial frame
 *                exits 4, a short write exits 5.  Banners go to stderr so that
 *                stdout carries frames only.
 *   otherwise  : benchmark, 5 trials x 30 passes over seeded faces, best.
 * Load failures exit 1.  --threads is accepted for compatibility (the work
 * runs on the GPU).  models/op_scales.bin is opened relative to the working
 * directory, as the reference does.
 */
#define _POSIX_C_SOURCE 200809L
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "fastface.h"

#ifdef FF_CLI_BATCHED
#define FF_CLI_DEFAULT_B 8
#define FF_CLI_NAME "FastFace INT8 batched (MI355X)"
#else
#define FF_CLI_DEFAULT_B 1
#define FF_CLI_NAME "FastFace INT8 (MI355X)"
#endif

static double now_s(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec + ts.tv_nsec * 1e-9;
}

/* seeded uniform faces in [-1, 1] for the first pass and the benchmark
 * (a 64-bit LCG: the reference's rand() sequence is libc-specific) */
static void fill_faces(float* x, size_t n)
{
    uint64_t s = 42;
    for (size_t i = 0; i < n; i++) {
        s = s * 6364136223846793005ULL + 1442695040888963407ULL;
        x[i] = (float)((int)((s >> 33) % 2001) - 1000) / 1000.0f;
    }
}

int main(int argc, char** argv)
{
    const char* path = (argc > 1) ? argv[1] : "models/w600k_r50_ffw4.bin";
    const char* in_path = NULL;
    const char* out_path = NULL;
    int server = 0;
    int B = FF_CLI_DEFAULT_B;
    for (int i = 2; i < argc; i++) {
        if (strcmp(argv[i], "--in") == 0 && i + 1 < argc) in_path = argv[++i];
        else if (strcmp(argv[i], "--out") == 0 && i + 1 < argc) out_path = argv[++i];
        else if (strcmp(argv[i], "--server") == 0) server = 1;
        else if (strcmp(argv[i], "--threads") == 0 && i + 1 < argc) ++i;
#ifdef FF_CLI_BATCHED
        else if (strcmp(argv[i], "--batch") == 0 && i + 1 < argc) B = atoi(argv[++i]);
#endif
    }
#ifdef FF_CLI_BATCHED
    {
        const char* e = getenv("BATCH");
        if (e) B = atoi(e);
    }
#endif
    if (B < 1) B = 1;
    const int validate = in_path && out_path;
    FILE* info = server ? stderr : stdout;

    FastFace* ff = fastface_create(path);
    if (!ff) {
        fprintf(stderr, "load fail\n");
        return 1;
    }
    fprintf(info, "%s  batch=%d\n", FF_CLI_NAME, B);
    if (fastface_reserve(ff, B) != 0) {
        fprintf(stderr, "device allocation failed\n");
        fastface_destroy(ff);
        return 1;
    }

    const size_t n_in = (size_t)B * FASTFACE_INPUT_N;
    const size_t n_out = (size_t)B * FASTFACE_OUTPUT_N;
    float* in = (float*)malloc(n_in * sizeof(float));
    float* out = (float*)malloc(n_out * sizeof(float));
    if (!in || !out) {
        fprintf(stderr, "out of memory\n");
        return 1;
    }
    if (validate) {
        FILE* f = fopen(in_path, "rb");
        if (!f) return 2;
        size_t got = fread(in, sizeof(float), n_in, f);
        fclose(f);
        if (got != n_in) memset(in + got, 0, (n_in - got) * sizeof(float));
    } else {
        fill_faces(in, n_in);
    }
    if (fastface_embed_batch(ff, in, B, out) != 0) {
        fprintf(stderr, "embed failed\n");
        return 1;
    }
    fprintf(stderr, "First pass OK\n");
    fprintf(stderr, "final_emb[0..4] = %g %g %g %g %g\n", out[0], out[1], out[2], out[3], out[4]);

    int rc = 0;
    if (validate) {
        FILE* f = fopen(out_path, "wb");
        if (!f || fwrite(out, sizeof(float), n_out, f) != n_out) rc = 5;
        if (f) fclose(f);
    } else if (server) {
        fprintf(stderr, "Server mode ready. Awaiting %zu-float frames (B=%d x 3x112x112).\n", n_in, B);
        for (;;) {
            size_t got = fread(in, sizeof(float), n_in, stdin);
            if (got == 0) break;
            if (got != n_in) {
                fprintf(stderr, "partial read (%zu/%zu floats) -- abort\n", got, n_in);
                rc = 4;
                break;
            }
            if (fastface_embed_batch(ff, in, B, out) != 0) {
                fprintf(stderr, "embed failed\n");
                rc = 1;
                break;
            }
            if (fwrite(out, sizeof(float), n_out, stdout) != n_out) {
                fprintf(stderr, "partial write\n");
                rc = 5;
                break;
            }
            fflush(stdout);
        }
    } else {
        double best = 1e9;
        for (int trial = 0; trial < 5; trial++) {
            double t0 = now_s();
            for (int it = 0; it < 30; it++) fastface_embed_batch(ff, in, B, out);
            double dt = (now_s() - t0) / 30;
            if (dt < best) best = dt;
            printf("Trial %d: %.2f ms/batch = %.2f ms/face  (%.1f face/s)\n", trial, dt * 1e3,
                   dt * 1e3 / B, B / dt);
        }
        printf("Best: %.2f ms/batch = %.2f ms/face  (%.1f face/s)\n", best * 1e3, best * 1e3 / B,
               B / best);
    }
    free(in);
    free(out);
    fastface_destroy(ff);
    return rc;
}
