/*
 * abi_caller.c — a plain C (gnu11) consumer of include/qmm_hip.h, built with
 * gcc and linked against libqmm_hip.so by tests/test_c_caller.py: the way the
 * engine's own C code would bind the library (no C++, no HIP headers).
 *
 *   abi_caller sizes
 *       prints "key value" lines: row sizes, status strings, activation
 *       buffer sizes and offsets (host-only calls; no GPU needed)
 *   abi_caller dispatch DIR TYPE N K M
 *       reads DIR/w.bin (N rows of packed blocks) and DIR/x.bin (fp32 [M][K]),
 *       runs qmm_gemm_multi_dispatch on device 0 and writes DIR/y.bin
 *       (fp32 [M][N]); exits non-zero with the library's message on error
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qmm_hip.h"

static void *read_file(const char *dir, const char *name, size_t bytes) {
    char path[4096];
    snprintf(path, sizeof path, "%s/%s", dir, name);
    FILE *f = fopen(path, "rb");
    if (!f) return NULL;
    void *p = malloc(bytes ? bytes : 1);
    size_t got = p ? fread(p, 1, bytes, f) : 0;
    fclose(f);
    if (got != bytes) {
        free(p);
        return NULL;
    }
    return p;
}

static int sizes(void) {
    static const uint32_t types[] = {QMM_TYPE_F32, QMM_TYPE_F16, QMM_TYPE_Q8_0, QMM_TYPE_Q4_K, QMM_TYPE_Q5_K,
                                     QMM_TYPE_Q6_K, 3u /* not on this path */};
    static const int64_t cols[] = {256, 2560, 4096, 9728, 100};
    for (size_t i = 0; i < sizeof types / sizeof types[0]; ++i)
        for (size_t j = 0; j < sizeof cols / sizeof cols[0]; ++j)
            printf("row_bytes.%u.%lld %zu\n", types[i], (long long)cols[j], qmm_row_bytes(types[i], cols[j]));
    for (int s = QMM_OK; s <= QMM_ENOTFOUND; ++s) printf("status.%d %s\n", s, qmm_status_string(s));
    static const int mk[][2] = {{1, 2560}, {8, 2560}, {64, 9728}, {512, 4096}};
    for (size_t i = 0; i < sizeof mk / sizeof mk[0]; ++i) {
        const int M = mk[i][0], K = mk[i][1];
        printf("q8k_bytes.%d.%d %zu\n", M, K, qmm_q8k_bytes(M, K));
        printf("q8k_d_offset.%d.%d %zu\n", M, K, qmm_q8k_d_offset(M, K));
        printf("q8k_bsum_offset.%d.%d %zu\n", M, K, qmm_q8k_bsum_offset(M, K));
        printf("q8k_tile_offset.%d.%d %zu\n", M, K, qmm_q8k_tile_offset(M, K));
        printf("q8k_h_offset.%d.%d %zu\n", M, K, qmm_q8k_h_offset(M, K));
        printf("q8k_bh_offset.%d.%d %zu\n", M, K, qmm_q8k_bh_offset(M, K));
        printf("q8_0_bytes.%d.%d %zu\n", M, K, qmm_q8_0_bytes(M, K));
        printf("q8_0_d_offset.%d.%d %zu\n", M, K, qmm_q8_0_d_offset(M, K));
    }
    printf("noalloc_scratch_bytes %zu\n", qmm_noalloc_scratch_bytes());
    return 0;
}

#define CHECK(call)                                                                            \
    do {                                                                                       \
        const int rc_ = (call);                                                                \
        if (rc_ != QMM_OK) {                                                                   \
            fprintf(stderr, "%s: %s (%s)\n", #call, qmm_status_string(rc_),                    \
                    ctx ? qmm_last_error(ctx) : "");                                           \
            return 1;                                                                          \
        }                                                                                      \
    } while (0)

static int dispatch(const char *dir, uint32_t type, int N, int K, int M) {
    const size_t rb = qmm_row_bytes(type, K);
    if (rb == 0 || N <= 0 || M <= 0) {
        fprintf(stderr, "bad shape\n");
        return 1;
    }
    const size_t w_bytes = (size_t)N * rb, x_bytes = (size_t)M * K * sizeof(float);
    const size_t y_bytes = (size_t)M * N * sizeof(float);
    void *w = read_file(dir, "w.bin", w_bytes), *x = read_file(dir, "x.bin", x_bytes);
    float *y = malloc(y_bytes);
    if (!w || !x || !y) {
        fprintf(stderr, "cannot read the inputs from %s\n", dir);
        return 1;
    }
    qmm_context *ctx = NULL;
    CHECK(qmm_init(0, &ctx));
    void *wd = NULL, *xd = NULL, *yd = NULL;
    CHECK(qmm_weight_upload(ctx, w, type, N, K, &wd));
    CHECK(qmm_malloc(ctx, x_bytes, &xd));
    CHECK(qmm_malloc(ctx, y_bytes, &yd));
    CHECK(qmm_memcpy_h2d(ctx, xd, x, x_bytes));
    qmm_matrix_task t;
    memset(&t, 0, sizeof t);
    t.w_base = wd;
    t.type = type;
    t.row_bytes = rb;
    t.dst = (float *)yd;
    t.dst_stride = (size_t)N;
    t.residual = NULL;
    t.rows = N;
    t.cols = K;
    CHECK(qmm_gemm_multi_dispatch(ctx, (const float *)xd, M, K, &t, 1));
    CHECK(qmm_synchronize(ctx));
    CHECK(qmm_memcpy_d2h(ctx, y, yd, y_bytes));
    CHECK(qmm_free(ctx, wd));
    CHECK(qmm_free(ctx, xd));
    CHECK(qmm_free(ctx, yd));
    CHECK(qmm_destroy(ctx));
    char path[4096];
    snprintf(path, sizeof path, "%s/y.bin", dir);
    FILE *f = fopen(path, "wb");
    if (!f || fwrite(y, 1, y_bytes, f) != y_bytes) {
        fprintf(stderr, "cannot write %s\n", path);
        return 1;
    }
    fclose(f);
    free(w);
    free(x);
    free(y);
    printf("dispatch ok start_row %d\n", t.start_row);
    return 0;
}

int main(int argc, char **argv) {
    if (argc >= 2 && strcmp(argv[1], "sizes") == 0) return sizes();
    if (argc == 7 && strcmp(argv[1], "dispatch") == 0)
        return dispatch(argv[2], (uint32_t)strtoul(argv[3], NULL, 10), atoi(argv[4]), atoi(argv[5]), atoi(argv[6]));
    fprintf(stderr, "usage: %s sizes | dispatch DIR TYPE N K M\n", argv[0]);
    return 2;
}
