// Per-row activation statistics shared by the quantize kernel and the GEMV prologue.
// All functions are called by every thread of a 256-thread workgroup.
//
// Bit-exactness: max is order independent, and every other f32 operation below is
// the same single-rounded operation, in the same order, as the reference:
//   RMSNorm  src/model/cpu.rs:11-41,47-66 (16 FMA accumulators) or src/ops/norm.rs:23-48
//   scale    src/npu.rs:1101-1106
//   quantize src/npu.rs:1107-1110
#pragma once

#include <hip/hip_fp16.h>

#include "qlin_internal.hpp"

namespace qlin {

constexpr int kRowThreads = 256;

template <typename T>
__device__ __forceinline__ float ld1(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ld1<float>(const float* p, int64_t i) {
    return p[i];
}
template <>
__device__ __forceinline__ float ld1<__half>(const __half* p, int64_t i) {
    return __half2float(p[i]);
}

// Loads x[k0 .. k0+8) as f32; VEC = 16-byte aligned, K % 8 == 0.  Out-of-range -> 0.
template <typename T, bool VEC>
__device__ __forceinline__ void load8(const T* row, int k0, int K, float v[8]) {
    if constexpr (VEC) {
        if (k0 >= K) {  // K % 8 == 0 here, so a group is either fully inside or outside
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = 0.0f;
            return;
        }
        if constexpr (sizeof(T) == 2) {
            uint4 raw = *reinterpret_cast<const uint4*>(row + k0);
            const __half2* h = reinterpret_cast<const __half2*>(&raw);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float2 f = __half22float2(h[i]);
                v[2 * i] = f.x;
                v[2 * i + 1] = f.y;
            }
        } else {
            float4 a = *reinterpret_cast<const float4*>(row + k0);
            float4 b = *reinterpret_cast<const float4*>(row + k0 + 4);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (k0 + i < K) ? ld1<T>(row, k0 + i) : 0.0f;
    }
}

__device__ __forceinline__ void load8_gamma(const float* g, int k0, int K, bool vec, float v[8]) {
    if (vec && k0 + 8 <= K) {
        float4 a = *reinterpret_cast<const float4*>(g + k0);
        float4 b = *reinterpret_cast<const float4*>(g + k0 + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = (k0 + i < K) ? g[k0 + i] : 0.0f;
    }
}

// RMSNorm scale 1/sqrt(sum(x^2)/K + eps) with the reference's summation order.
// lds: >= 1 float of shared scratch.  Result is returned to every thread.
template <typename T>
__device__ float block_rms_scale(const T* row, int K, float eps, bool sequential, float* lds) {
    const int t = threadIdx.x;
    if (sequential) {
        // src/ops/norm.rs:38: x.iter().map(|v| v * v).sum::<f32>(), one rounding per op
        if (t == 0) {
            float sum = 0.0f;
            for (int i = 0; i < K; ++i) {
                float x = ld1<T>(row, i);
                float v2 = x * x;
                sum = sum + v2;
            }
            lds[0] = 1.0f / __builtin_sqrtf(sum / (float)K + eps);
        }
    } else if (t < 64) {
        // src/model/cpu.rs:14-35: four float32x4 accumulators fed by vfmaq_f32
        float acc = 0.0f;
        const int j = t & 15;
        if (t < 16) {
            int i = 0;
            for (; i + 16 <= K; i += 16) {
                float x = ld1<T>(row, i + j);
                acc = __builtin_fmaf(x, x, acc);
            }
        }
        // vaddq(vaddq(a,b), vaddq(c,d)): lane j of the result
        float b = __shfl(acc, j + 4, 64);
        float c = __shfl(acc, j + 8, 64);
        float d = __shfl(acc, j + 12, 64);
        float tj = (acc + b) + (c + d);
        // vaddvq_f32 = faddp, faddp: (t0 + t1) + (t2 + t3)
        float t1 = __shfl(tj, 1, 64);
        float t2 = __shfl(tj, 2, 64);
        float t3 = __shfl(tj, 3, 64);
        if (t == 0) {
            float sum = (tj + t1) + (t2 + t3);
            for (int i = K & ~15; i < K; ++i) {  // scalar tail: sum += v * v
                float x = ld1<T>(row, i);
                float v2 = x * x;
                sum = sum + v2;
            }
            lds[0] = 1.0f / __builtin_sqrtf(sum / (float)K + eps);
        }
    }
    __syncthreads();
    float r = lds[0];
    __syncthreads();
    return r;
}

template <typename T>
__device__ __forceinline__ float lds_f32(const T* p, int i) {
    if constexpr (sizeof(T) == 2) return __half2float(p[i]);
    else return p[i];
}

// Sum of squares of a row held in LDS, in the order of src/ops/norm.rs:38
// (sum = sum + v*v, one rounding per operation).  One thread.  The loads of 16
// elements are issued before their additions, so LDS latency is paid once per 16.
template <typename T>
__device__ float lds_sumsq_seq(const T* x, int K) {
    float sum = 0.0f;
    int i = 0;
    for (; i + 16 <= K; i += 16) {
        float v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = lds_f32(x, i + u);
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const float v2 = v[u] * v[u];
            sum = sum + v2;
        }
    }
    for (; i < K; ++i) {
        const float v = lds_f32(x, i);
        const float v2 = v * v;
        sum = sum + v2;
    }
    return sum;
}

// Sum of squares of a row held in LDS, in the order of src/model/cpu.rs:14-35: 16
// fused-multiply-add chains (chain j takes elements j, j+16, ... in order), combined
// lanewise as (a+b)+(c+d), then (t0+t1)+(t2+t3), then the scalar tail sum += v*v.
// Called by all 64 lanes of one wave; the result is valid in lane 0.  Lane j runs
// chain j 32 steps (512 elements of the row) per loop trip, all 32 reads of a trip
// issued before its FMAs: with a loop of 16-element batches and a runtime K the reads
// waited one batch at a time (2560 fp16 values: 1.9 -> 1.1-1.2 us).  fp16 values are
// kept as fp16 so each conversion folds into its FMA (v_fma_mix_f32, exact).
template <typename T>
__device__ float lds_sumsq_neon16(const T* x, int K) {
    const int lane = threadIdx.x & 63, j = lane & 15;
    float acc = 0.0f;
    if (lane < 16) {
        const T* c = x + j;
        const int n16 = K & ~15;
        int i = 0;
        for (; i + 512 <= n16; i += 512) {
            T v[32];
#pragma unroll
            for (int u = 0; u < 32; ++u) v[u] = c[i + 16 * u];
#pragma unroll
            for (int u = 0; u < 32; ++u) {
                const float f = (float)v[u];
                acc = __builtin_fmaf(f, f, acc);
            }
        }
        for (; i < n16; i += 16) {
            const float f = (float)c[i];
            acc = __builtin_fmaf(f, f, acc);
        }
    }
    const float b = __shfl(acc, j + 4, 64), c = __shfl(acc, j + 8, 64), d = __shfl(acc, j + 12, 64);
    const float tj = (acc + b) + (c + d);
    const float t1 = __shfl(tj, 1, 64), t2 = __shfl(tj, 2, 64), t3 = __shfl(tj, 3, 64);
    float sum = (tj + t1) + (t2 + t3);
    if (lane == 0)
        for (int i = K & ~15; i < K; ++i) {
            const float v = (float)x[i];
            const float v2 = v * v;
            sum = sum + v2;
        }
    return sum;
}

// Block-wide max of non-negative values and OR of flags.  lds: >= 8 words.
__device__ __forceinline__ void block_max_or(float& v, int& f, float* lds) {
    v = wave_max(v);
    f = wave_or(f);
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int* ldsi = reinterpret_cast<int*>(lds);
    if (lane == 0) {
        lds[w] = v;
        ldsi[4 + w] = f;
    }
    __syncthreads();
    v = fmaxf(fmaxf(lds[0], lds[1]), fmaxf(lds[2], lds[3]));
    f = ldsi[4] | ldsi[5] | ldsi[6] | ldsi[7];
    __syncthreads();
}

// y = norm ? (x * nscale) * gamma : x for 8 values.
__device__ __forceinline__ void apply_norm8(float v[8], const float g[8], float nscale) {
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (v[i] * nscale) * g[i];
}

// Row statistics: returns s (per-token scale) and sets *bad when the row holds Inf/NaN.
// nscale is the RMSNorm scale (ignored without gamma).
template <typename T, bool VEC>
__device__ float block_row_scale(const T* row, int K, const float* gamma, bool gvec, float nscale,
                                 int* bad, float* lds) {
    float m = 0.0f;
    int f = 0;
    for (int k0 = threadIdx.x * 8; k0 < K; k0 += kRowThreads * 8) {
        float v[8];
        load8<T, VEC>(row, k0, K, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) f |= !__builtin_isfinite(v[i]);
        if (gamma) {
            float g[8];
            load8_gamma(gamma, k0, K, gvec, g);
            apply_norm8(v, g, nscale);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
    }
    block_max_or(m, f, lds);
    *bad = f;
    return qscale_from_absmax(m);
}

}  // namespace qlin
