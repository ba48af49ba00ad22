/*
 * The per-matvec backend plug as a maintainer adds it to the reference's
 * ss_matmul_dispatch (SlipStream/src/core/layer_scheduler.c:248-279): the
 * HIP branch is the INTEGRATION.md snippet, the CPU branch stands for
 * ss_dequant_matvec and only counts that it ran. Test infrastructure.
 *
 * usage: plug_snippet W.bin x.bin y.bin rows cols type [batch]
 * W.bin holds GGUF blocks (or F32 rows), x.bin cols fp32 values; y.bin receives rows fp32
 * values (two dispatches of the same matrix: the second reuses the upload).
 * With "batch": 17 dispatches inside one ss_hip_begin_batch / ss_hip_end_batch,
 * as the scheduler brackets Q/K/V (layer_scheduler.c:353-361), dispatch i
 * reading (i + 1) x; y.bin receives the 17 outputs in order.
 * Prints "fallbacks N".
 */
#include <stdbool.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ss_hip.h"

#define GGML_TYPE_F32 0
#define GGML_TYPE_Q4_0 2
#define GGML_TYPE_Q8_0 8
#define GGML_TYPE_Q4_K 12

typedef struct { ss_hip_ctx_t *hip_ctx; } sched_t;

static int cpu_fallbacks;

static void cpu_dequant_matvec(float *out, int32_t rows) {
    cpu_fallbacks++;
    for (int32_t r = 0; r < rows; r++) out[r] = -1.0f;
}

static void matmul_dispatch(sched_t *sched, float *out, const void *mat, const float *vec, int32_t rows,
                            int32_t cols, int32_t type) {
    if (sched->hip_ctx && ss_hip_should_use_gpu(rows, cols) &&
        (type == GGML_TYPE_Q4_0 || type == GGML_TYPE_Q8_0 || type == GGML_TYPE_Q4_K || type == GGML_TYPE_F32)) {
        /* true (nonzero) = out holds the result, as gpu_success for Metal */
        bool gpu_success = ss_hip_matvec_host(sched->hip_ctx, out, mat, vec, rows, cols, type) != 0;
        if (gpu_success) return;         /* else fall through to the CPU path */
    }
    cpu_dequant_matvec(out, rows);
}

static void *slurp(const char *path, size_t *n) {
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    fseek(f, 0, SEEK_END);
    long len = ftell(f);
    fseek(f, 0, SEEK_SET);
    void *p = malloc((size_t)len + 1);
    if (p && fread(p, 1, (size_t)len, f) != (size_t)len) { free(p); p = NULL; }
    fclose(f);
    *n = (size_t)len;
    return p;
}

int main(int argc, char **argv) {
    if (argc != 7 && argc != 8) return 2;
    size_t nw, nx;
    void *w = slurp(argv[1], &nw);
    float *x = (float *)slurp(argv[2], &nx);
    const int32_t rows = atoi(argv[4]), cols = atoi(argv[5]), type = atoi(argv[6]);
    if (!w || !x) return 3;
    float *y = (float *)calloc((size_t)rows, sizeof(float));
    float *y2 = (float *)calloc((size_t)rows, sizeof(float));
    sched_t sched = {ss_hip_init(0)};
    if (!sched.hip_ctx) {
        fprintf(stderr, "ss_hip_init: %s\n", ss_hip_last_error());
        return 4;
    }
    if (argc == 8 && strcmp(argv[7], "batch") == 0) {
        enum { N = 17 };
        float *ys = (float *)calloc((size_t)N * rows, sizeof(float));
        float *xs = (float *)malloc((size_t)N * cols * sizeof(float));
        if (!ys || !xs) return 3;
        for (int i = 0; i < N; i++)
            for (int32_t c = 0; c < cols; c++) xs[(size_t)i * cols + c] = (float)(i + 1) * x[c];
        ss_hip_begin_batch(sched.hip_ctx);
        for (int i = 0; i < N; i++)
            matmul_dispatch(&sched, ys + (size_t)i * rows, w, xs + (size_t)i * cols, rows, cols, type);
        if (ss_hip_end_batch(sched.hip_ctx) != 0) {
            fprintf(stderr, "ss_hip_end_batch: %s\n", ss_hip_last_error());
            return 7;
        }
        FILE *f = fopen(argv[3], "wb");
        if (!f || fwrite(ys, sizeof(float), (size_t)N * rows, f) != (size_t)N * rows) return 6;
        fclose(f);
        printf("fallbacks %d\n", cpu_fallbacks);
        ss_hip_free(sched.hip_ctx);
        return 0;
    }
    if (argc != 7) return 2;
    matmul_dispatch(&sched, y, w, x, rows, cols, type);
    matmul_dispatch(&sched, y2, w, x, rows, cols, type);
    if (memcmp(y, y2, (size_t)rows * sizeof(float)) != 0) return 5;
    FILE *f = fopen(argv[3], "wb");
    if (!f || fwrite(y, sizeof(float), (size_t)rows, f) != (size_t)rows) return 6;
    fclose(f);
    printf("fallbacks %d\n", cpu_fallbacks);
    ss_hip_free(sched.hip_ctx);
    return 0;
}
