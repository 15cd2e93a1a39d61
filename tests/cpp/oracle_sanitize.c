/*
 * Runs every function of the CPU oracle (oracle/qlin_oracle.c) on small inputs, edge
 * cases included, in a build with AddressSanitizer and UndefinedBehaviorSanitizer
 * (float-to-int overflow and float division by zero too): out-of-bounds accesses,
 * overflowing conversions and other undefined behaviour abort the run.  Test
 * infrastructure for the oracle, CPU only; tests/test_oracle_sanitize.py builds and runs it.
 *
 * Besides running clean, it checks what the oracle's own contracts fix: the three int32
 * GEMM routes agree, every finite fp16 pattern survives f16 -> f32 -> f16, quantized codes
 * stay in [-127, 127], a non-finite row is counted, and the unpacked compressed codes lie
 * in the signed range of their width.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../oracle/qlin_oracle.h"

static uint32_t rng = 12345u;
static uint32_t next_u32(void) {
    rng ^= rng << 13;
    rng ^= rng >> 17;
    rng ^= rng << 5;
    return rng;
}
static float next_f32(void) { return ((float)(next_u32() >> 8) / 16777216.0f) * 2.0f - 1.0f; }

#define CHECK(c)                                                      \
    do {                                                              \
        if (!(c)) {                                                   \
            fprintf(stderr, "check failed at line %d: %s\n", __LINE__, #c); \
            exit(1);                                                  \
        }                                                             \
    } while (0)

static void check_gemms(int64_t M, int64_t K, int64_t N, int bits) {
    const int lim = bits == 4 ? 8 : 127;
    int8_t* q = malloc((size_t)(M * K));
    int8_t* kn = malloc((size_t)(K * N));
    int8_t* nk = malloc((size_t)(N * K));
    int32_t* a0 = malloc(sizeof(int32_t) * (size_t)(M * N));
    int32_t* a1 = malloc(sizeof(int32_t) * (size_t)(M * N));
    int32_t* a2 = malloc(sizeof(int32_t) * (size_t)(M * N));
    for (int64_t i = 0; i < M * K; ++i) q[i] = (int8_t)((int)(next_u32() % 255) - 127);
    for (int64_t k = 0; k < K; ++k)
        for (int64_t n = 0; n < N; ++n) {
            const int8_t v = (int8_t)((int)(next_u32() % (uint32_t)(bits == 4 ? 16 : 255)) - (bits == 4 ? lim : 127));
            kn[k * N + n] = v;
            nk[n * K + k] = v;
        }
    oracle_gemm_i32_kn(q, K, M, K, kn, N, a0);
    oracle_gemm_i32_nk(q, K, M, K, nk, N, a1, 2);
    CHECK(memcmp(a0, a1, sizeof(int32_t) * (size_t)(M * N)) == 0);
    if (bits == 4) {
        oracle_gemm_i32_digit_split(q, K, M, K, kn, N, a2);
        CHECK(memcmp(a0, a2, sizeof(int32_t) * (size_t)(M * N)) == 0);
    }
    free(q), free(kn), free(nk), free(a0), free(a1), free(a2);
}

int main(void) {
    /* quantization: random rows, an all-zero row, a subnormal row, huge values, Inf / NaN */
    enum { M = 6, K = 100, LDA = 104 };
    float A[M * LDA];
    for (int i = 0; i < M * LDA; ++i) A[i] = next_f32() * 4.0f;
    for (int k = 0; k < K; ++k) A[1 * LDA + k] = 0.0f;
    for (int k = 0; k < K; ++k) A[2 * LDA + k] = 1e-45f * (float)(k % 3);
    A[3 * LDA + 5] = 3.0e38f;
    A[3 * LDA + 6] = -3.0e38f;
    A[4 * LDA + 7] = INFINITY;
    A[5 * LDA + 8] = NAN;
    int8_t q[M * K];
    float s[M];
    for (int mode = 0; mode < 2; ++mode) {
        const int64_t bad = oracle_quantize(A, M, K, LDA, mode, q, K, s);
        CHECK(bad == 2);
        for (int i = 0; i < M * K; ++i) CHECK(q[i] >= -127 && q[i] <= 127);
        CHECK(s[1] == 1.0f);
    }
    for (int m = 0; m < M; ++m) (void)oracle_row_scale(A + m * LDA, K);

    /* the three GEMM routes agree (W4 and W8, ragged sizes) */
    check_gemms(3, 64, 17, 4);
    check_gemms(5, 96, 33, 8);
    check_gemms(1, 2560, 8, 4);

    /* dequant, residual update, SiLU-gate with large gate values */
    {
        enum { DM = 3, DN = 10 };
        int32_t acc[DM * DN];
        float sc[DN], out[DM * DN], mid[DM * DN / 2], hid[DM * DN], srow[DM] = {0.5f, 1e-3f, 7.0f};
        for (int i = 0; i < DM * DN; ++i) acc[i] = (int32_t)(next_u32() % 2000001u) - 1000000;
        for (int n = 0; n < DN; ++n) sc[n] = 0.01f * (float)(n + 1);
        oracle_dequant(acc, DM, DN, srow, sc, out);
        out[0] = 200.0f;
        out[1] = -200.0f;
        oracle_swiglu(out, DM, DN, mid);
        for (int i = 0; i < DM * DN; ++i) hid[i] = next_f32();
        oracle_residual_add(hid, out, DM, DN, 0.5f);
        oracle_residual_add(hid, out, DM, DN, 1.0f);
    }

    /* RMSNorm in both summation orders, lengths around the 16-wide chains */
    {
        const int64_t Ks[] = {7, 16, 17, 100, 2560};
        for (int t = 0; t < 5; ++t) {
            const int64_t n = Ks[t];
            float* x = malloc(sizeof(float) * (size_t)(2 * n));
            float* w = malloc(sizeof(float) * (size_t)n);
            float* y = malloc(sizeof(float) * (size_t)(2 * n));
            for (int64_t i = 0; i < 2 * n; ++i) x[i] = next_f32();
            for (int64_t i = 0; i < n; ++i) w[i] = 1.0f + next_f32() * 0.1f;
            oracle_rmsnorm_neon16(x, 2, n, n, w, 1e-6f, y);
            oracle_rmsnorm_seq(x, 2, n, n, w, 1e-6f, y);
            free(x), free(w), free(y);
        }
    }

    /* binary16 conversions: every finite pattern round-trips; specials convert */
    for (uint32_t h = 0; h < 65536u; ++h) {
        const float f = oracle_f16_to_f32((uint16_t)h);
        if (isfinite(f)) CHECK(oracle_f32_to_f16(f) == (uint16_t)h);
    }
    {
        const float sp[] = {0.0f, -0.0f, 65504.0f, 65520.0f, 1e30f, -1e30f, 5.96e-8f, 2.9e-8f, INFINITY, NAN};
        uint16_t hb[10];
        float back[10];
        oracle_f32_to_f16_array(sp, 10, hb);
        oracle_f16_to_f32_array(hb, 10, back);
        CHECK(hb[4] == 0x7c00u && hb[5] == 0xfc00u);
    }

    /* the whole linear: W4 and W8, with and without RMSNorm and SiLU-gate */
    {
        enum { LM = 3, LK = 64, LN = 32 };
        uint16_t a16[LM * LK], o16[LM * LN];
        int8_t w[LN * LK];
        float sc[LN], g[LK];
        for (int i = 0; i < LM * LK; ++i) a16[i] = oracle_f32_to_f16(next_f32() * 3.0f);
        for (int k = 0; k < LK; ++k) g[k] = 1.0f + 0.05f * next_f32();
        for (int n = 0; n < LN; ++n) sc[n] = 0.02f + 0.01f * next_f32();
        for (int bits = 4; bits <= 8; bits += 4) {
            for (int i = 0; i < LN * LK; ++i)
                w[i] = (int8_t)((int)(next_u32() % (uint32_t)(bits == 4 ? 16 : 255)) - (bits == 4 ? 8 : 127));
            for (int v = 0; v < 8; ++v)  /* gamma, SiLU-gate, rounding mode */
                oracle_linear_f16(a16, LM, LK, (v & 1) ? g : NULL, 1e-6f, w, sc, LN, (v >> 1) & 1, (v >> 2) & 1, o16, 2);
        }
    }

    /* compressed-tensors decode, both widths, K not a multiple of the fields per word */
    for (int bits = 4; bits <= 8; bits += 4) {
        enum { CN = 5, CK = 37 };
        const int per = 32 / bits, words = (CK + per - 1) / per;
        uint32_t packed[CN * 10];
        int8_t codes[CK * CN];
        for (int i = 0; i < CN * words; ++i) packed[i] = next_u32();
        oracle_unpack_compressed(packed, CN, CK, bits, codes);
        const int lo = -(1 << (bits - 1)), hi = (1 << (bits - 1)) - 1;
        for (int i = 0; i < CK * CN; ++i) CHECK(codes[i] >= lo && codes[i] <= hi);
    }

    printf("oracle sanitize ok\n");
    return 0;
}
