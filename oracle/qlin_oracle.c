/*
 * CPU oracle for the W4A8 / W8A8 quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path, loaded by the test
 * suite, the smoke check and the benchmark's CPU-baseline leg.  Nothing in the
 * product links or calls it.  Built with -ffp-contract=off -fno-fast-math so each
 * f32 operation below rounds exactly once, as the Rust reference does.
 */
#include "qlin_oracle.h"

#include <float.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static void set_threads(int threads) {
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
}

/* src/npu.rs:1101-1106 */
float oracle_row_scale(const float* a, int64_t K) {
    float maximum = 0.0f;
    for (int64_t k = 0; k < K; ++k) maximum = fmaxf(maximum, fabsf(a[k])); /* f32::max ignores NaN */
    if (maximum == 0.0f) return 1.0f;
    float s = maximum / 127.0f;
    return s < FLT_MIN ? FLT_MIN : s; /* .max(f32::MIN_POSITIVE) */
}

static int8_t quantize_one(float x, float inv, int round_mode) {
    float v = x * inv;                                   /* src/npu.rs:1109 x * (1.0 / scale) */
    float r = round_mode == ORACLE_ROUND_EVEN ? rintf(v) : roundf(v);
    if (r != r) return 0;                                /* NaN: Rust `as i32` saturates NaN to 0 */
    if (r < -127.0f) r = -127.0f;                        /* .clamp(-127.0, 127.0) */
    if (r > 127.0f) r = 127.0f;
    return (int8_t)(int)r;
}

int64_t oracle_quantize(const float* A, int64_t M, int64_t K, int64_t lda, int round_mode,
                        int8_t* q, int64_t ldq, float* s) {
    int64_t bad = 0;
    for (int64_t m = 0; m < M; ++m) {
        const float* a = A + m * lda;
        float scale = oracle_row_scale(a, K);
        float inv = 1.0f / scale;
        int finite = 1;
        for (int64_t k = 0; k < K; ++k) {
            if (!isfinite(a[k])) finite = 0;
            q[m * ldq + k] = quantize_one(a[k], inv, round_mode);
        }
        s[m] = scale;
        bad += !finite;
    }
    return bad;
}

/* src/npu.rs:1112-1116 */
void oracle_gemm_i32_kn(const int8_t* q, int64_t ldq, int64_t M, int64_t K, const int8_t* codes,
                        int64_t N, int32_t* acc) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            int32_t sum = 0;
            for (int64_t k = 0; k < K; ++k) sum += (int32_t)q[m * ldq + k] * (int32_t)codes[k * N + n];
            acc[m * N + n] = sum;
        }
}

void oracle_gemm_i32_nk(const int8_t* q, int64_t ldq, int64_t M, int64_t K, const int8_t* w_nk,
                        int64_t N, int32_t* acc, int threads) {
    set_threads(threads);
#pragma omp parallel for schedule(static) collapse(2)
    for (int64_t n0 = 0; n0 < N; n0 += 16)
        for (int64_t m = 0; m < M; ++m) {
            const int8_t* qa = q + m * ldq;
            int64_t n1 = n0 + 16 < N ? n0 + 16 : N;
            for (int64_t n = n0; n < n1; ++n) {
                const int8_t* w = w_nk + n * K;
                int32_t sum = 0;
                for (int64_t k = 0; k < K; ++k) sum += (int32_t)qa[k] * (int32_t)w[k];
                acc[m * N + n] = sum;
            }
        }
}

/* QWEN3_W4A8_PIPELINE_REVIEW_20261020.md:17-30: q = 16h + l + 8, acc = 8*sum(B) + 16*P_hi + P_lo */
void oracle_gemm_i32_digit_split(const int8_t* q, int64_t ldq, int64_t M, int64_t K,
                                 const int8_t* codes, int64_t N, int32_t* acc) {
    for (int64_t n = 0; n < N; ++n) {
        int64_t correction = 0;
        for (int64_t k = 0; k < K; ++k) correction += 8 * (int64_t)codes[k * N + n];
        for (int64_t m = 0; m < M; ++m) {
            int64_t p_hi = 0, p_lo = 0;
            for (int64_t k = 0; k < K; ++k) {
                int u = (int)q[m * ldq + k] + 128; /* 1..255 */
                int h = u / 16 - 8, l = u % 16 - 8; /* both in [-8, 7] */
                p_hi += (int64_t)h * codes[k * N + n];
                p_lo += (int64_t)l * codes[k * N + n];
            }
            acc[m * N + n] = (int32_t)(correction + 16 * p_hi + p_lo);
        }
    }
}

/* src/npu.rs:1117 */
void oracle_dequant(const int32_t* acc, int64_t M, int64_t N, const float* s, const float* scales,
                    float* out) {
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) out[m * N + n] = ((float)acc[m * N + n] * s[m]) * scales[n];
}

/* src/model/dense.rs:486-489: scale (skipped at 1.0, src/model/cpu.rs:247-253), then
 * add_chunk's y[i] += x[i] (src/model/cpu.rs:68-85) */
void oracle_residual_add(float* hidden, const float* projected, int64_t M, int64_t N, float multiplier) {
    for (int64_t i = 0; i < M * N; ++i) {
        float p = projected[i];
        if (multiplier != 1.0f) p = p * multiplier;
        hidden[i] = hidden[i] + p;
    }
}

/* src/npu.rs:1202-1208 */
void oracle_swiglu(const float* out, int64_t M, int64_t N, float* mid) {
    int64_t F = N / 2;
    for (int64_t m = 0; m < M; ++m)
        for (int64_t j = 0; j < F; ++j) {
            float g = out[m * N + j], u = out[m * N + F + j];
            mid[m * F + j] = (g / (1.0f + expf(-g))) * u;
        }
}

/* src/model/cpu.rs:11-41 (aarch64 square_sum) */
static float square_sum_neon16(const float* x, int64_t K) {
    float acc[16] = {0};
    int64_t i = 0;
    for (; i + 16 <= K; i += 16)
        for (int j = 0; j < 16; ++j) acc[j] = fmaf(x[i + j], x[i + j], acc[j]); /* vfmaq_f32 */
    float t[4];
    for (int j = 0; j < 4; ++j) t[j] = (acc[j] + acc[4 + j]) + (acc[8 + j] + acc[12 + j]);
    float sum = (t[0] + t[1]) + (t[2] + t[3]); /* vaddvq_f32: faddp, faddp */
    for (; i < K; ++i) {
        float v2 = x[i] * x[i];
        sum += v2;
    }
    return sum;
}

static float square_sum_seq(const float* x, int64_t K) {
    float sum = 0.0f;
    for (int64_t i = 0; i < K; ++i) {
        float v2 = x[i] * x[i];
        sum += v2;
    }
    return sum;
}

/* src/model/cpu.rs:47-66 */
void oracle_rmsnorm_neon16(const float* x, int64_t M, int64_t K, int64_t ldx, const float* w,
                           float eps, float* y) {
    for (int64_t m = 0; m < M; ++m) {
        const float* r = x + m * ldx;
        float scale = 1.0f / sqrtf(square_sum_neon16(r, K) / (float)K + eps);
        for (int64_t k = 0; k < K; ++k) y[m * K + k] = (r[k] * scale) * w[k];
    }
}

/* src/ops/norm.rs:23-48 */
void oracle_rmsnorm_seq(const float* x, int64_t M, int64_t K, int64_t ldx, const float* w,
                        float eps, float* y) {
    for (int64_t m = 0; m < M; ++m) {
        const float* r = x + m * ldx;
        float scale = 1.0f / sqrtf(square_sum_seq(r, K) / (float)K + eps);
        for (int64_t k = 0; k < K; ++k) y[m * K + k] = (r[k] * scale) * w[k];
    }
}

uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                   /* below 2^-14: subnormal half */
        float v;
        memcpy(&v, &ax, 4);
        uint32_t n = (uint32_t)rintf(v * 16777216.0f); /* units of 2^-24, exact scaling */
        return (uint16_t)(sign | n);
    }
    uint32_t e = (ax >> 23) - 127 + 15, mant = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (mant >> 13), rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, mant = h & 0x3ffu, x;
    if (e == 0) {
        float v = (float)mant * (1.0f / 16777216.0f);
        memcpy(&x, &v, 4);
        x |= sign;
    } else if (e == 31) {
        x = sign | 0x7f800000u | (mant << 13);
    } else {
        x = sign | ((e - 15 + 127) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void oracle_f32_to_f16_array(const float* x, int64_t n, uint16_t* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f32_to_f16(x[i]);
}
void oracle_f16_to_f32_array(const uint16_t* h, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = oracle_f16_to_f32(h[i]);
}

void oracle_linear_f16(const uint16_t* A, int64_t M, int64_t K, const float* gamma, float eps,
                       const int8_t* w_nk, const float* scales, int64_t N, int swiglu,
                       int round_mode, uint16_t* out, int threads) {
    set_threads(threads);
    float* x = (float*)malloc((size_t)(M * K) * sizeof(float));
    int8_t* q = (int8_t*)malloc((size_t)(M * K));
    float* s = (float*)malloc((size_t)M * sizeof(float));
    int32_t* acc = (int32_t*)malloc((size_t)(M * N) * sizeof(int32_t));
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        float* r = x + m * K;
        for (int64_t k = 0; k < K; ++k) r[k] = oracle_f16_to_f32(A[m * K + k]);
        if (gamma) {
            float scale = 1.0f / sqrtf(square_sum_neon16(r, K) / (float)K + eps);
            for (int64_t k = 0; k < K; ++k) r[k] = (r[k] * scale) * gamma[k];
        }
        oracle_quantize(r, 1, K, K, round_mode, q + m * K, K, s + m);
    }
    oracle_gemm_i32_nk(q, K, M, K, w_nk, N, acc, threads);
    int64_t F = N / 2;
#pragma omp parallel for schedule(static)
    for (int64_t m = 0; m < M; ++m) {
        if (!swiglu) {
            for (int64_t n = 0; n < N; ++n)
                out[m * N + n] = oracle_f32_to_f16(((float)acc[m * N + n] * s[m]) * scales[n]);
        } else {
            for (int64_t j = 0; j < F; ++j) {
                float g = ((float)acc[m * N + j] * s[m]) * scales[j];
                float u = ((float)acc[m * N + F + j] * s[m]) * scales[F + j];
                out[m * F + j] = oracle_f32_to_f16((g / (1.0f + expf(-g))) * u);
            }
        }
    }
    free(x);
    free(q);
    free(s);
    free(acc);
}

/* src/model/checkpoint.rs:352-371 */
void oracle_unpack_compressed(const uint32_t* packed, int64_t N, int64_t K, int bits,
                              int8_t* codes) {
    int64_t factor = 32 / bits, columns = (K + factor - 1) / factor;
    uint32_t mask = (1u << bits) - 1u;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            uint32_t word = packed[n * columns + k / factor];
            int32_t field = (int32_t)((word >> ((k % factor) * bits)) & mask);
            codes[k * N + n] = (int8_t)(field - (1 << (bits - 1)));
        }
}
