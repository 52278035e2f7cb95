/*
 * A C host of the hyq C ABI (include/hyq.h), driving it the way a compiled
 * caller would -- the reference's Rust FFI shim in particular: opaque handles,
 * plain pointers and sizes, integer return codes and hyq_last_error(); no
 * Python and no torch in the process.
 *
 * Test program (tests/test_c_host.py). It links the oracle (test
 * infrastructure) to check the results it gets from libhyq.
 *
 *   hyq_host --no-gpu
 *       geometry queries, then a context request: on a machine without a
 *       GPU it fails with a negative code and a message.
 *   hyq_host DTYPE ROWS COLS WEIGHTS_FILE BATCH
 *       uploads the [ROWS x COLS] GGUF bytes, then
 *       - Weight::matmul at batch 1 from host pointers (hyq_matmul) against
 *         the oracle's f64 int8 GEMV, |err| <= 1e-5 * sum|terms|;
 *       - Weight::matmul at BATCH from device buffers (hyq_matmul_d) against
 *         the oracle's f64 product, |err| <= 2e-3 * sum|w x|;
 *       - a call with a wrong activation length: HYQ_EINVAL and a message;
 *       then releases everything. Exit status 0 when every check holds.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "hyq.h"
#include "hyq_oracle.h"

#define CHECK(cond, ...)                                                                       \
    do {                                                                                       \
        if (!(cond)) {                                                                         \
            fprintf(stderr, "hyq_host: " __VA_ARGS__);                                         \
            fprintf(stderr, " (last error: %s)\n", hyq_last_error());                          \
            return 1;                                                                          \
        }                                                                                      \
    } while (0)

static uint8_t *read_file(const char *path, size_t *len)
{
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    if (fseek(f, 0, SEEK_END) != 0) {
        fclose(f);
        return NULL;
    }
    long n = ftell(f);
    rewind(f);
    uint8_t *b = n > 0 ? malloc((size_t)n) : NULL;
    if (b && fread(b, 1, (size_t)n, f) != (size_t)n) {
        free(b);
        b = NULL;
    }
    fclose(f);
    *len = b ? (size_t)n : 0;
    return b;
}

/* N(0, 1) activations from a fixed 64-bit LCG and Box-Muller. */
static void fill_normal(float *x, size_t n, uint64_t seed)
{
    uint64_t s = seed * 6364136223846793005ull + 1442695040888963407ull;
    for (size_t i = 0; i < n; i += 2) {
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        const double u1 = ((double)(s >> 11) + 1.0) / 9007199254740993.0;
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        const double u2 = (double)(s >> 11) / 9007199254740992.0;
        const double r = sqrt(-2.0 * log(u1));
        x[i] = (float)(r * cos(6.283185307179586 * u2));
        if (i + 1 < n) x[i + 1] = (float)(r * sin(6.283185307179586 * u2));
    }
}

static int no_gpu(void)
{
    CHECK(hyq_block_len(HYQ_Q4_K) == 256 && hyq_block_bytes(HYQ_Q4_K) == 144,
          "Q4_K geometry");
    CHECK(hyq_block_len(HYQ_Q2_0C) == 512 && hyq_block_bytes(HYQ_STQ1_0) == 42,
          "Q2_0C / STQ1_0 geometry");
    CHECK(hyq_block_len(12345) == -1, "an unknown dtype has no geometry");
    hyq_ctx *ctx = NULL;
    const int rc = hyq_ctx_create(0, &ctx);
    if (rc == HYQ_OK) {
        hyq_ctx_destroy(ctx);
        printf("device present\n");
        return 0;
    }
    CHECK(rc < 0 && ctx == NULL && hyq_last_error()[0] != '\0',
          "a failed context request returns a negative code and a message");
    printf("no device: code %d, \"%s\"\n", rc, hyq_last_error());
    return 0;
}

int main(int argc, char **argv)
{
    if (argc == 2 && strcmp(argv[1], "--no-gpu") == 0) return no_gpu();
    if (argc != 6) {
        fprintf(stderr, "usage: hyq_host DTYPE ROWS COLS WEIGHTS_FILE BATCH | --no-gpu\n");
        return 2;
    }
    const int dtype = atoi(argv[1]);
    const size_t rows = (size_t)strtoull(argv[2], NULL, 10);
    const size_t cols = (size_t)strtoull(argv[3], NULL, 10);
    const size_t batch = (size_t)strtoull(argv[5], NULL, 10);
    size_t wlen = 0;
    uint8_t *w = read_file(argv[4], &wlen);
    CHECK(w != NULL, "cannot read %s", argv[4]);
    CHECK(rows > 0 && cols > 0 && batch > 1, "bad shape");

    hyq_ctx *ctx = NULL;
    CHECK(hyq_ctx_create(0, &ctx) == HYQ_OK, "context on device 0");
    const uint64_t dims[2] = {cols, rows}; /* GGUF order: innermost first */
    hyq_weight *W = NULL;
    CHECK(hyq_weight_upload(ctx, dtype, w, wlen, dims, 2, &W) == HYQ_OK, "weight upload");
    int got_dtype = -1, rank = 0;
    uint64_t got_dims[3] = {0, 0, 0};
    CHECK(hyq_weight_info(W, &got_dtype, got_dims, &rank) == HYQ_OK && got_dtype == dtype &&
              rank == 2 && got_dims[0] == cols && got_dims[1] == rows,
          "weight info");

    float *x = malloc(batch * cols * sizeof(float));
    float *y = malloc(batch * rows * sizeof(float));
    double *yr = malloc(batch * rows * sizeof(double));
    double *mag = malloc(batch * rows * sizeof(double));
    int8_t *q = malloc(cols);
    float *s = malloc((cols + 255) / 256 * sizeof(float));
    CHECK(x && y && yr && mag && q && s, "host allocation");
    fill_normal(x, batch * cols, 7);

    /* batch 1 from host pointers: the int8 GEMV */
    CHECK(hyq_matmul(ctx, W, x, 1, y) == HYQ_OK, "hyq_matmul at batch 1");
    hyqo_q8_quantize(x, cols, q, s);
    hyqo_gemv_q8_f64(dtype, w, rows, cols, q, s, yr, mag);
    double worst = 0.0;
    for (size_t r = 0; r < rows; ++r) {
        const double e = fabs((double)y[r] - yr[r]);
        CHECK(e <= 1e-5 * mag[r], "batch 1, row %zu: %.9g against %.9g", r, (double)y[r], yr[r]);
        if (mag[r] > 0 && e / mag[r] > worst) worst = e / mag[r];
    }
    printf("batch 1: %zu rows within 1e-5 * sum|terms| (worst %.2e)\n", rows, worst);

    /* BATCH from device buffers: the f16-MFMA product */
    void *xd = NULL, *yd = NULL;
    CHECK(hyq_device_alloc(ctx, batch * cols * sizeof(float), &xd) == HYQ_OK, "device x");
    CHECK(hyq_device_alloc(ctx, batch * rows * sizeof(float), &yd) == HYQ_OK, "device y");
    CHECK(hyq_memcpy_h2d(ctx, xd, x, batch * cols * sizeof(float)) == HYQ_OK, "copy x");
    CHECK(hyq_matmul_d(ctx, W, (const float *)xd, batch, (float *)yd) == HYQ_OK,
          "hyq_matmul_d at batch %zu", batch);
    CHECK(hyq_memcpy_d2h(ctx, y, yd, batch * rows * sizeof(float)) == HYQ_OK, "copy y");
    hyqo_matmul_f64(dtype, w, rows, cols, x, batch, yr, mag);
    worst = 0.0;
    for (size_t i = 0; i < batch * rows; ++i) {
        const double e = fabs((double)y[i] - yr[i]);
        CHECK(e <= 2e-3 * mag[i], "batch %zu, element %zu: %.9g against %.9g", batch, i,
              (double)y[i], yr[i]);
        if (mag[i] > 0 && e / mag[i] > worst) worst = e / mag[i];
    }
    printf("batch %zu: %zu elements within 2e-3 * sum|w x| (worst %.2e)\n", batch, batch * rows,
           worst);

    /* the error path: a wrong activation length for a Q8 vector */
    hyq_q8 *xq = NULL;
    CHECK(hyq_q8_create(ctx, cols + 256, &xq) == HYQ_OK, "Q8 vector");
    const int rc = hyq_gemv_q8_d(ctx, W, xq, NULL, (float *)yd);
    CHECK(rc == HYQ_EINVAL && strstr(hyq_last_error(), "length") != NULL,
          "a wrong activation length is HYQ_EINVAL (got %d)", rc);
    printf("wrong length: code %d, \"%s\"\n", rc, hyq_last_error());

    hyq_q8_release(xq);
    CHECK(hyq_device_free(ctx, xd) == HYQ_OK && hyq_device_free(ctx, yd) == HYQ_OK, "free");
    hyq_weight_release(W);
    CHECK(hyq_sync(ctx) == HYQ_OK, "sync");
    hyq_ctx_destroy(ctx);
    free(x);
    free(y);
    free(yr);
    free(mag);
    free(q);
    free(s);
    free(w);
    printf("ok\n");
    return 0;
}
