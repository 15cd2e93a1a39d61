/*
 * CPU oracle for the W4A8 / W8A8 quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only the test suite,
 * the smoke check and the CPU-baseline leg of the benchmark may load it.  The
 * product (libqlinear.so) never links, loads or calls anything here.
 *
 * Every function restates the reference's arithmetic (HC-Zhou/open_rknpu2_lm_infer)
 * in plain C, citing the file:line it follows.  Build flags keep IEEE single
 * precision semantics: no fast-math, no FP contraction (the Rust reference never
 * contracts a*b+c unless it calls mul_add / vfmaq explicitly).
 *
 * Layouts:
 *   A      f32 [M, lda]           activations (row m starts at A + m*lda)
 *   q      i8  [M, ldq]           quantized activations
 *   s      f32 [M]                per-token scale
 *   codes  i8  [K, N]  K-major    reference QuantMatrix.codes, codes[k*N + n]
 *   w_nk   i8  [N, K]             same codes, output-channel-major
 *   scales f32 [N]                per-output-channel weight scale
 *   acc    i32 [M, N]
 */
#ifndef QLIN_ORACLE_H
#define QLIN_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* rounding of x*(1/s): 0 = half away from zero (Rust f32::round, the reference
 * default, src/npu.rs:1109), 1 = half to even (the rounding the W8A8 decode-GEMV
 * workload description names; the library's QLIN_ROUND_HALF_EVEN). */
#define ORACLE_ROUND_AWAY 0
#define ORACLE_ROUND_EVEN 1

/* src/npu.rs:1101-1106: absmax over the row, s = 1 for an all-zero row, else
 * max(absmax/127, FLT_MIN). */
float oracle_row_scale(const float* a, int64_t K);

/* src/npu.rs:1101-1110 for every row: s[m] and q[m,k] = clamp(round(x*(1/s)),-127,127);
 * NaN products map to 0 like Rust's saturating `as i32`.  Returns the number of
 * rows holding a non-finite value (the native library rejects such input). */
int64_t oracle_quantize(const float* A, int64_t M, int64_t K, int64_t lda, int round_mode,
                        int8_t* q, int64_t ldq, float* s);

/* src/npu.rs:1112-1116: exact int32 acc[m,n] = sum_k q[m,k]*codes[k*N+n]. */
void oracle_gemm_i32_kn(const int8_t* q, int64_t ldq, int64_t M, int64_t K, const int8_t* codes,
                        int64_t N, int32_t* acc);
/* Same sum over the [N,K] layout; OpenMP over rows and channels. */
void oracle_gemm_i32_nk(const int8_t* q, int64_t ldq, int64_t M, int64_t K, const int8_t* w_nk,
                        int64_t N, int32_t* acc, int threads);

/* The native library's digit split (QWEN3_W4A8_PIPELINE_REVIEW_20261020.md:17-30):
 * q = 16*h + l + 8 with h,l in [-8,7], acc = correction + 16*P_hi + P_lo where
 * correction[n] = 8*sum_k B[k,n].  Returns the same acc by a different route. */
void oracle_gemm_i32_digit_split(const int8_t* q, int64_t ldq, int64_t M, int64_t K,
                                 const int8_t* codes, int64_t N, int32_t* acc);

/* src/npu.rs:1117: out[m,n] = (f32(acc)*s[m]) * scales[n]. */
void oracle_dequant(const int32_t* acc, int64_t M, int64_t N, const float* s, const float* scales,
                    float* out);

/* src/model/dense.rs:486-489 and 534-537 (Cpu::scale then Cpu::add, src/model/cpu.rs:68-85,
 * 237-253): hidden[m,n] = hidden[m,n] + projected[m,n]*multiplier, in place, each an f32
 * rounding; Cpu::scale skips a multiplier of exactly 1 (x*1 == x, so the same result). */
void oracle_residual_add(float* hidden, const float* projected, int64_t M, int64_t N, float multiplier);

/* src/npu.rs:1202-1208 / src/model/cpu.rs:119-152: mid[m,j] = (g/(1+exp(-g)))*u
 * with g = out[m,j], u = out[m,j+N/2]; mid is [M, N/2]. */
void oracle_swiglu(const float* out, int64_t M, int64_t N, float* mid);

/* src/model/cpu.rs:11-41,47-66 (aarch64 build, the reference's production target):
 * sum of squares in 16 FMA accumulators (4 NEON vectors x 4 lanes), combined as
 * vaddvq(vaddq(vaddq(a,b),vaddq(c,d))), tail added as v*v; then
 * y = (x*scale)*w with scale = 1/sqrt(sum/len + eps). */
void oracle_rmsnorm_neon16(const float* x, int64_t M, int64_t K, int64_t ldx, const float* w,
                           float eps, float* y);
/* src/ops/norm.rs:23-48 (and cpu.rs on non-aarch64): sequential sum of v*v. */
void oracle_rmsnorm_seq(const float* x, int64_t M, int64_t K, int64_t ldx, const float* w,
                        float eps, float* y);

/* IEEE binary16 conversions, round to nearest even. */
uint16_t oracle_f32_to_f16(float x);
float oracle_f16_to_f32(uint16_t h);
void oracle_f32_to_f16_array(const float* x, int64_t n, uint16_t* out);
void oracle_f16_to_f32_array(const uint16_t* h, int64_t n, float* out);

/* Whole linear over the [N,K] layout with OpenMP (the timed CPU baseline):
 * quantize (optionally after RMSNorm when gamma != NULL, neon16 order), exact
 * int32 GEMM, dequant, optional SwiGLU.  Activations arrive as fp16 bits and the
 * result leaves as fp16 bits, like the GPU path.  bits = 4 or 8 only changes how
 * w_nk is interpreted (values already in [-8,7] or [-127,127]).  Output is
 * [M, N] or [M, N/2] with swiglu. */
void oracle_linear_f16(const uint16_t* A, int64_t M, int64_t K, const float* gamma, float eps,
                       const int8_t* w_nk, const float* scales, int64_t N, int swiglu,
                       int round_mode, uint16_t* out, int threads);

/* compressed-tensors pack-quantized decode (src/model/checkpoint.rs:352-371):
 * packed i32 words [N, ceil(K/(32/bits))], LSB-first fields, value = field - 2^(bits-1),
 * written K-major into codes[k*N+n]. */
void oracle_unpack_compressed(const uint32_t* packed, int64_t N, int64_t K, int bits,
                              int8_t* codes);

#ifdef __cplusplus
}
#endif
#endif
