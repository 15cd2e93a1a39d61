/* Links libqlinear.a the way the reference's build.rs links its native library
 * (build.rs:13-67: a static archive pulled in whole, plus the runtime it needs).
 *
 *   static_link_test       argument checks that reject before any device work (no GPU)
 *   static_link_test gpu   kernels through the statically linked library: W4 weights from
 *                          [K, N] codes, an M=1 decode GEMV and an M=64 prefill GEMM through
 *                          qlin_run_f32 (the rk_npu_w4a8_run_f32 call, host buffers), and one
 *                          qlin_run_noalloc (device buffers, its static scratch array), each
 *                          checked bit for bit against the CPU oracle (oracle/qlin_oracle.c,
 *                          the restatement of src/npu.rs:1097-1121).
 * The GPU mode exercises what only a static link can get wrong: the code objects the
 * archive's constructors register, kernel launches from them, and the device address of
 * the no-alloc scratch array. */
#include <hip/hip_runtime_api.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/qlinear.h"
#include "../../oracle/qlin_oracle.h"

static int cpu_checks(void) {
    if (strcmp(qlin_strerror(QLIN_OK), "success") != 0) return 1;
    if (strcmp(qlin_strerror(QLIN_ERR_PARAM), "invalid parameter") != 0) return 2;
    if (strcmp(qlin_strerror(-99), "unknown error") != 0) return 3;
    qlin_weights* w = (qlin_weights*)&w;
    if (qlin_weights_create(NULL, NULL, NULL, &w) != QLIN_ERR_PARAM || w != NULL) return 4;
    qlin_weight_config bad_bits = {3, 8, 8};
    int8_t codes[64] = {0};
    float scales[8] = {1, 1, 1, 1, 1, 1, 1, 1};
    if (qlin_weights_create(&bad_bits, codes, scales, &w) != QLIN_ERR_PARAM || w != NULL) return 5;
    qlin_weight_config cfg = {4, 8, 8};
    codes[9] = 8; /* outside W4 [-8, 7] */
    if (qlin_weights_create(&cfg, codes, scales, &w) != QLIN_ERR_PARAM || w != NULL) return 6;
    codes[9] = 0;
    scales[3] = 0.0f; /* scales must be positive */
    if (qlin_weights_create(&cfg, codes, scales, &w) != QLIN_ERR_PARAM || w != NULL) return 7;
    if (qlin_run(NULL, NULL, 1, NULL, QLIN_F16, 8, NULL, QLIN_F16, 8, 0, NULL) != QLIN_ERR_PARAM) return 8;
    if (qlin_run_f32(NULL, NULL, 1, NULL, NULL) != QLIN_ERR_PARAM) return 9;
    qlin_weights_free(NULL);
    qlin_workspace_free(NULL);
    printf("static link ok\n");
    return 0;
}

/* splitmix64: seeded inputs without any library */
static uint64_t g_state = 42;
static uint64_t next_u64(void) {
    uint64_t z = (g_state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
static float next_unit(void) { return (float)(next_u64() >> 40) / (float)(1u << 24); } /* [0, 1) */

/* oracle output of the linear on f32 rows (src/npu.rs:1097-1121) */
static void oracle_out(const float* A, int M, int K, int N, const int8_t* codes_kn, const float* sc, float* out) {
    int8_t* q = malloc((size_t)M * K);
    float* s = malloc((size_t)M * sizeof(float));
    int32_t* acc = malloc((size_t)M * N * sizeof(int32_t));
    oracle_quantize(A, M, K, K, ORACLE_ROUND_AWAY, q, K, s);
    oracle_gemm_i32_kn(q, K, M, K, codes_kn, N, acc);
    oracle_dequant(acc, M, N, s, sc, out);
    free(q);
    free(s);
    free(acc);
}

static int same_bits(const float* a, const float* b, size_t n, const char* what) {
    if (memcmp(a, b, n * sizeof(float)) == 0) return 1;
    for (size_t i = 0; i < n; ++i)
        if (memcmp(a + i, b + i, sizeof(float)) != 0) {
            printf("FAIL %s: element %zu got %.9g expected %.9g\n", what, i, a[i], b[i]);
            break;
        }
    return 0;
}

static int gpu_checks(void) {
    enum { K = 2560, N = 2048, MMAX = 64 };
    int8_t* codes = malloc((size_t)K * N);
    float* sc = malloc(N * sizeof(float));
    float* A = malloc((size_t)MMAX * K * sizeof(float));
    float* got = malloc((size_t)MMAX * N * sizeof(float));
    float* want = malloc((size_t)MMAX * N * sizeof(float));
    for (size_t i = 0; i < (size_t)K * N; ++i) codes[i] = (int8_t)((int)(next_u64() % 16) - 8); /* W4 [-8, 7] */
    for (int n = 0; n < N; ++n) sc[n] = 0.01f + 0.09f * next_unit();
    for (size_t i = 0; i < (size_t)MMAX * K; ++i) {
        float v = 2.0f * next_unit() - 1.0f;
        if (i % 97 == 0) v *= 20.0f; /* outlier channels */
        A[i] = v;
    }
    qlin_weight_config cfg = {4, K, N};
    qlin_weights* w = NULL;
    qlin_workspace* ws = NULL;
    int rc = qlin_weights_create(&cfg, codes, sc, &w);
    if (rc == QLIN_OK) rc = qlin_workspace_create(MMAX, K, N, &ws);
    if (rc != QLIN_OK) {
        printf("FAIL create: %s\n", qlin_strerror(rc));
        return 10;
    }
    int ok = 1;
    const int rows[2] = {1, MMAX}; /* the fused decode GEMV, then quantize + the MFMA GEMM */
    for (int i = 0; i < 2 && ok; ++i) {
        const int M = rows[i];
        memset(got, 0, (size_t)M * N * sizeof(float));
        rc = qlin_run_f32(ws, w, M, A, got);
        if (rc != QLIN_OK) {
            printf("FAIL qlin_run_f32 M=%d: %s\n", M, qlin_strerror(rc));
            return 11;
        }
        oracle_out(A, M, K, N, codes, sc, want);
        ok &= same_bits(got, want, (size_t)M * N, M == 1 ? "qlin_run_f32 M=1" : "qlin_run_f32 M=64");
    }
    /* the entry point that allocates nothing, on device buffers */
    const int M = 4;
    void *dA = NULL, *dC = NULL;
    if (ok && (hipMalloc(&dA, (size_t)M * K * sizeof(float)) != hipSuccess ||
               hipMalloc(&dC, (size_t)M * N * sizeof(float)) != hipSuccess ||
               hipMemcpy(dA, A, (size_t)M * K * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)) {
        printf("FAIL device buffers\n");
        return 12;
    }
    if (ok) {
        rc = qlin_run_noalloc(w, M, dA, QLIN_F32, K, NULL, 0.0f, dC, QLIN_F32, N, 0, NULL, NULL);
        if (rc != QLIN_OK || hipDeviceSynchronize() != hipSuccess ||
            hipMemcpy(got, dC, (size_t)M * N * sizeof(float), hipMemcpyDeviceToHost) != hipSuccess) {
            printf("FAIL qlin_run_noalloc: %s\n", qlin_strerror(rc));
            return 13;
        }
        oracle_out(A, M, K, N, codes, sc, want);
        ok &= same_bits(got, want, (size_t)M * N, "qlin_run_noalloc M=4");
    }
    hipFree(dA);
    hipFree(dC);
    qlin_workspace_free(ws);
    qlin_weights_free(w);
    free(codes);
    free(sc);
    free(A);
    free(got);
    free(want);
    if (!ok) return 14;
    printf("static link gpu ok\n");
    return 0;
}

int main(int argc, char** argv) {
    if (argc > 1 && strcmp(argv[1], "gpu") == 0) return gpu_checks();
    return cpu_checks();
}
