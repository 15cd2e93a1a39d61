// Kernel (a): per-token activation quantization, optionally after RMSNorm.
//
// Without RMSNorm, rows of up to 40960 fp16 / 20480 f32 values are quantized from
// registers by four waves each.  Otherwise one 256-thread workgroup takes a row: rows of up to
// 60 KiB are copied into LDS once and every pass reads them there; longer rows take
// the two-pass kernel, whose pass 1
// (absmax + finiteness, with the norm applied on the fly) and pass 2 (quantize, 8
// values per thread per iteration, one 64-bit store) read global memory.
// The replaced library stage is the CPU scan + quantize of rk_npu_w4a8_quant.cpp
// (QWEN3_W4A8_PIPELINE_REVIEW_20261020.md:26-27); the arithmetic is the oracle's,
// src/npu.rs:1101-1110.
#include <algorithm>
#include <type_traits>

#include "qlin_rows.hpp"

namespace qlin {

// Four / eight values -> int8 codes packed little-endian.  `fast` (a finite row, the
// usual case) takes quant_finite; otherwise quant_one handles Inf / NaN.  The
// branches are uniform per row.
__device__ __forceinline__ uint32_t quant4(const float v[4], float inv, bool rne, bool fast) {
    int q[4];
    if (fast && rne) {
#pragma unroll
        for (int j = 0; j < 4; ++j) q[j] = quant_finite<true>(v[j], inv);
    } else if (fast) {
#pragma unroll
        for (int j = 0; j < 4; ++j) q[j] = quant_finite<false>(v[j], inv);
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) q[j] = quant_one(v[j], inv, rne);  // src/npu.rs:1107-1110
    }
    uint32_t w = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) w |= (uint32_t)(q[j] & 0xff) << (8 * j);
    return w;
}
__device__ __forceinline__ void quant8(const float v[8], float inv, bool rne, bool fast, uint32_t& w0, uint32_t& w1) {
    w0 = quant4(v, inv, rne, fast);
    w1 = quant4(v + 4, inv, rne, fast);
}


template <typename T, bool VEC>
__global__ __launch_bounds__(kRowThreads) void quant_rows_kernel(QuantParams p) {
    __shared__ float lds[8];
    const int row = blockIdx.x;
    const T* x = reinterpret_cast<const T*>(p.A) + (int64_t)row * p.lda;
    const bool gvec = VEC && ((reinterpret_cast<uintptr_t>(p.gamma) & 15) == 0);
    float nscale = 1.0f;
    if (p.gamma) nscale = block_rms_scale<T>(x, p.K, p.eps, (p.flags & kFlagNormSeq) != 0, lds);
    int bad = 0;
    const float s = block_row_scale<T, VEC>(x, p.K, p.gamma, gvec, nscale, &bad, lds);
    const float inv = 1.0f / s;
    const bool rne = (p.flags & kFlagRne) != 0;
    const bool fast = !bad && __builtin_isfinite(s);  // finite row: the short rounding sequence
    const bool qvec = ((reinterpret_cast<uintptr_t>(p.q) & 7) == 0) && (p.ldq % 8 == 0);
    int8_t* qrow = p.q + (int64_t)row * p.ldq;
    for (int k0 = threadIdx.x * 8; k0 < p.ldq; k0 += kRowThreads * 8) {
        float v[8];
        load8<T, VEC>(x, k0, p.K, v);  // zero beyond K
        if (p.gamma) {
            float g[8];
            load8_gamma(p.gamma, k0, p.K, gvec, g);
            apply_norm8(v, g, nscale);
        }
        uint32_t w0, w1;
        quant8(v, inv, rne, fast, w0, w1);
        if (qvec && k0 + 8 <= p.ldq) {
            *reinterpret_cast<uint2*>(qrow + k0) = make_uint2(w0, w1);
        } else {
            for (int i = 0; i < 8 && k0 + i < p.ldq; ++i)
                qrow[k0 + i] = (int8_t)((i < 4 ? w0 >> (8 * i) : w1 >> (8 * (i - 4))) & 0xff);
        }
    }
    if (threadIdx.x == 0) {
        p.s[row] = s;
        if (bad && p.err) atomicOr(p.err, 1u);
    }
}

// Row staged in LDS: one coalesced read of the row from global memory; the statistics
// and the quantize pass then read LDS.  NT threads per row: 256 spreads a row over four
// waves (the least latency per row); with many rows, 64 (one wave per row, many rows
// resident per CU) keeps more rows' sequential norm chains in flight at once, where
// 256-thread rows left three of four waves idle during the sum (M = 4096, K = 2560 with
// RMSNorm: 19.6 -> 14.6 us).  Many RMSNorm rows of up to 8 chunks per lane with 16-byte
// aligned weights take quant_norm_wave_kernel instead.  Rows of up to kStageBytes take this path (the
// default 64 KiB workgroup LDS limit, less the static reduction words).  Needs
// K % 8 == 0 and a 16-byte aligned row (16-byte copies).
constexpr int kStageBytes = 60 * 1024;

template <typename T>
__device__ __forceinline__ float lds_ld(const T* r, int i) {
    if constexpr (sizeof(T) == 2) return __half2float(r[i]);
    else return r[i];
}

// 8 consecutive values from LDS at a 16-byte aligned element index
template <typename T>
__device__ __forceinline__ void lds_ld8(const T* r, int k0, float v[8]) {
    if constexpr (sizeof(T) == 2) {
        const uint4 raw = *reinterpret_cast<const uint4*>(r + k0);
        const __half2* h = reinterpret_cast<const __half2*>(&raw);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float2 f = __half22float2(h[i]);
            v[2 * i] = f.x;
            v[2 * i + 1] = f.y;
        }
    } else {
        const float4 a = *reinterpret_cast<const float4*>(r + k0);
        const float4 b = *reinterpret_cast<const float4*>(r + k0 + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
}

template <typename T, int NT>
__global__ __launch_bounds__(NT) void quant_rows_staged_kernel(QuantParams p) {
    extern __shared__ __align__(16) uint8_t stage[];
    __shared__ float red[8];
    const int row = blockIdx.x, t = threadIdx.x;
    const T* x = reinterpret_cast<const T*>(p.A) + (int64_t)row * p.lda;
    T* xs = reinterpret_cast<T*>(stage);
    constexpr int E = 16 / sizeof(T);  // elements per 16-byte copy
    const int nchunks = p.K / E;
    // eight 16-byte loads in flight per thread before any is stored.  Loads and stores
    // are unconditional: past the end a lane copies the last chunk onto itself (same
    // data), so no load waits behind a branch.
    constexpr int B = 8;
    for (int c0 = t; c0 < nchunks; c0 += NT * B) {
        uint4 v[B];
#pragma unroll
        for (int i = 0; i < B; ++i) v[i] = reinterpret_cast<const uint4*>(x)[min(c0 + i * NT, nchunks - 1)];
#pragma unroll
        for (int i = 0; i < B; ++i) reinterpret_cast<uint4*>(xs)[min(c0 + i * NT, nchunks - 1)] = v[i];
    }
    __syncthreads();

    float nscale = 1.0f;
    if (p.gamma) {
        // RMSNorm scale with the reference's summation order (wave 0)
        if (t < 64) {
            const float sum = (p.flags & kFlagNormSeq) ? (t == 0 ? lds_sumsq_seq(xs, p.K) : 0.0f)
                                                       : lds_sumsq_neon16(xs, p.K);
            if (t == 0) red[0] = 1.0f / __builtin_sqrtf(sum / (float)p.K + p.eps);
        }
        __syncthreads();
        nscale = red[0];
        __syncthreads();
    }

    // absmax (after the norm) and finiteness (of the input), 8 values per step
    const bool gvec = (reinterpret_cast<uintptr_t>(p.gamma) & 15) == 0;
    float m = 0.0f;
    int f = 0;
    for (int k0 = t * 8; k0 < p.K; k0 += NT * 8) {
        float v[8];
        lds_ld8(xs, k0, v);
#pragma unroll
        for (int i = 0; i < 8; ++i) f |= !__builtin_isfinite(v[i]);
        if (p.gamma) {
            float g[8];
            load8_gamma(p.gamma, k0, p.K, gvec, g);
            apply_norm8(v, g, nscale);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
    }
    if constexpr (NT == 64) {
        m = wave_max(m);
        f = wave_or(f);
    } else {
        block_max_or(m, f, red);
    }
    const float s = qscale_from_absmax(m);
    const float inv = 1.0f / s;
    const bool rne = (p.flags & kFlagRne) != 0;
    const bool fast = !f && __builtin_isfinite(s);  // finite row: the short rounding sequence
    int8_t* qrow = p.q + (int64_t)row * p.ldq;
    // 8 codes per step; the zero tail [K, ldq) too (ldq % 8 == 0 on this path)
    for (int k0 = t * 8; k0 < p.ldq; k0 += NT * 8) {
        uint32_t w0 = 0, w1 = 0;
        if (k0 < p.K) {
            float v[8];
            lds_ld8(xs, k0, v);
            if (p.gamma) {
                float g[8];
                load8_gamma(p.gamma, k0, p.K, gvec, g);
                apply_norm8(v, g, nscale);
            }
            quant8(v, inv, rne, fast, w0, w1);
        }
        *reinterpret_cast<uint2*>(qrow + k0) = make_uint2(w0, w1);
    }
    if (t == 0) {
        p.s[row] = s;
        if (f && p.err) atomicOr(p.err, 1u);
    }
}

// RMSNorm rows, one wave per row, row and RMSNorm weights in registers: the lane's NC
// 16-byte row chunks and their weights are all loaded before any is used, the row is
// copied into LDS only for the norm sum (the reference's chain order reads it there),
// and the normalized values stay in registers for the absmax and the quantize pass.
// The staged kernel loads the weights again in both passes, a dependent global round
// trip per 8 values (M = 4096, K = 2560: 17.5 us there).  Same arithmetic as the staged
// kernel, value for value.  Needs K % 8 == 0, a 16-byte aligned row and weights, an
// 8-byte aligned q with ldq % 8 == 0, and 64 * NC chunks >= K / E.
// Sum of squares in the order of src/model/cpu.rs:14-35 (16 fused-multiply-add chains,
// chain j takes elements j, j+16, ... in order, combined lanewise as (a+b)+(c+d), then
// (t0+t1)+(t2+t3); K % 16 == 0 so there is no scalar tail), from a row stored
// chain-major in LDS: element k at cm[(k % 16) * ls + k / 16], ls = K / 16 + 8.  Lane j
// of the wave reads chain j 8 elements per 16-byte read (K / 128 reads instead of K / 16
// two-byte reads; with 16 rows per CU the two-byte reads held the sum at ~3.6 us per row
// against ~1.1 us alone).  The 8-element pad puts the 16 chains' reads, and the two
// chains written by one store instruction, in different banks.  Needs K % 512 == 0
// (trips of four reads).  Called by all 64 lanes; the result is valid in lane 0.
__device__ __forceinline__ float cm_sumsq_neon16(const _Float16* cm, int K) {
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int ls = K / 16 + 8;
    float acc = 0.0f;
    if (lane < 16) {
        const uint4* c = reinterpret_cast<const uint4*>(cm + j * ls);
        for (int r = 0; r < K / 128; r += 4) {
            uint4 v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = c[r + u];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const _Float16* h = reinterpret_cast<const _Float16*>(&v[u]);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float f = (float)h[e];
                    acc = __builtin_fmaf(f, f, acc);
                }
            }
        }
    }
    const float b = __shfl(acc, j + 4, 64), c = __shfl(acc, j + 8, 64), d = __shfl(acc, j + 12, 64);
    const float tj = (acc + b) + (c + d);
    const float t1 = __shfl(tj, 1, 64), t2 = __shfl(tj, 2, 64), t3 = __shfl(tj, 3, 64);
    return (tj + t1) + (t2 + t3);
}

template <typename T, int NC, bool CM>
__global__ __launch_bounds__(64) void quant_norm_wave_kernel(QuantParams p) {
    extern __shared__ __align__(16) uint8_t stage[];
    constexpr int E = 16 / sizeof(T);  // values per 16-byte chunk
    const int row = blockIdx.x, lane = threadIdx.x;
    const T* x = reinterpret_cast<const T*>(p.A) + (int64_t)row * p.lda;
    T* xs = reinterpret_cast<T*>(stage);
    const int nchunks = p.K / E;
    // (a clamped chunk repeats the last one: harmless for the max and the finiteness test,
    // and its LDS copy writes the same bytes to the same place)
    uint4 raw[NC];
    float v[NC][E];
#pragma unroll
    for (int i = 0; i < NC; ++i) raw[i] = reinterpret_cast<const uint4*>(x)[min(lane + 64 * i, nchunks - 1)];
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const float4* g = reinterpret_cast<const float4*>(p.gamma + (int64_t)min(lane + 64 * i, nchunks - 1) * E);
#pragma unroll
        for (int h = 0; h < E / 4; ++h) {
            const float4 a = g[h];
            v[i][4 * h] = a.x;
            v[i][4 * h + 1] = a.y;
            v[i][4 * h + 2] = a.z;
            v[i][4 * h + 3] = a.w;
        }
    }
    if constexpr (CM) {
        // chain-major copy: chunk c holds elements 8c .. 8c + 7, i.e. chains 8 (c & 1) + e at
        // position c >> 1
        _Float16* cm = reinterpret_cast<_Float16*>(stage);
        const int ls = p.K / 16 + 8;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const int c = min(lane + 64 * i, nchunks - 1);
            const _Float16* h = reinterpret_cast<const _Float16*>(&raw[i]);
#pragma unroll
            for (int e = 0; e < 8; ++e) cm[(8 * (c & 1) + e) * ls + (c >> 1)] = h[e];
        }
    } else {
#pragma unroll
        for (int i = 0; i < NC; ++i) reinterpret_cast<uint4*>(xs)[min(lane + 64 * i, nchunks - 1)] = raw[i];
    }
    __syncthreads();
    float sum;
    if constexpr (CM) sum = cm_sumsq_neon16(reinterpret_cast<const _Float16*>(stage), p.K);
    else sum = (p.flags & kFlagNormSeq) ? (lane == 0 ? lds_sumsq_seq(xs, p.K) : 0.0f) : lds_sumsq_neon16(xs, p.K);
    const float nscale = __shfl(1.0f / __builtin_sqrtf(sum / (float)p.K + p.eps), 0, 64);

    // normalized values (v: weight -> value), absmax (after the norm), finiteness (of the input)
    float m = 0.0f;
    int f = 0;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const T* e = reinterpret_cast<const T*>(&raw[i]);
#pragma unroll
        for (int j = 0; j < E; ++j) {
            const float xv = lds_ld(e, j);
            f |= !__builtin_isfinite(xv);
            v[i][j] = (xv * nscale) * v[i][j];
            m = fmaxf(m, fabsf(v[i][j]));
        }
    }
    m = wave_max(m);
    f = wave_or(f);
    const float s = qscale_from_absmax(m);
    const float inv = 1.0f / s;
    const bool rne = (p.flags & kFlagRne) != 0;
    const bool fast = !f && __builtin_isfinite(s);  // finite row: the short rounding sequence
    int8_t* qrow = p.q + (int64_t)row * p.ldq;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = lane + 64 * i;
        if (c < nchunks) {
            if constexpr (E == 8) {
                uint32_t w0, w1;
                quant8(v[i], inv, rne, fast, w0, w1);
                *reinterpret_cast<uint2*>(qrow + c * E) = make_uint2(w0, w1);
            } else {
                *reinterpret_cast<uint32_t*>(qrow + c * E) = quant4(v[i], inv, rne, fast);
            }
        }
    }
    for (int k0 = p.K + 8 * lane; k0 < p.ldq; k0 += 8 * 64) *reinterpret_cast<uint2*>(qrow + k0) = make_uint2(0, 0);
    if (lane == 0) {
        p.s[row] = s;
        if (f && p.err) atomicOr(p.err, 1u);
    }
}

template <typename T, bool CM>
static bool launch_quant_norm_wave_cm(const QuantParams& p, int rows, hipStream_t stream) {
    constexpr int E = 16 / sizeof(T);
    const int per_lane = (p.K / E + 63) / 64;
    const size_t lds = CM ? (size_t)(p.K + 128) * 2 : (size_t)p.K * sizeof(T);  // 16 chains of K / 16 + 8
    dim3 grid(rows), block(64);
    if (per_lane <= 2) quant_norm_wave_kernel<T, 2, CM><<<grid, block, lds, stream>>>(p);
    else if (per_lane <= 4) quant_norm_wave_kernel<T, 4, CM><<<grid, block, lds, stream>>>(p);
    else if (per_lane <= 5) quant_norm_wave_kernel<T, 5, CM><<<grid, block, lds, stream>>>(p);  // K = 2560 fp16
    else if (per_lane <= 8) quant_norm_wave_kernel<T, 8, CM><<<grid, block, lds, stream>>>(p);
    else return false;
    return true;
}

// fp16 rows in the reference's chain order with K % 512 == 0 take the chain-major sum
template <typename T>
static bool launch_quant_norm_wave(const QuantParams& p, int rows, hipStream_t stream) {
    if constexpr (sizeof(T) == 2) {
        if (!(p.flags & kFlagNormSeq) && p.K % 512 == 0) return launch_quant_norm_wave_cm<T, true>(p, rows, stream);
    }
    return launch_quant_norm_wave_cm<T, false>(p, rows, stream);
}

// Without RMSNorm: WPR waves per row (1 or 4) and 4 / WPR rows per 256-thread
// workgroup, the row held in registers (NC 16-byte chunks per lane, all loaded
// before any is used).  Absmax and finiteness come from one integer max over the
// sign-masked bit patterns: for non-negative fp16 / f32 values the bit order is the
// value order, and Inf / NaN are exactly the patterns at or above the all-ones
// exponent.  Needs K % 8 == 0, a 16-byte aligned row and an 8-byte aligned q with
// ldq % 8 == 0.
template <typename T, int NC, int WPR>
__global__ __launch_bounds__(256) void quant_rows_reg_kernel(QuantParams p, int rows) {
    __shared__ uint32_t red[4];
    constexpr int L = 64 * WPR;  // lanes per row
    const int lane = threadIdx.x % L;
    const int row = blockIdx.x * (4 / WPR) + threadIdx.x / L;
    if (WPR == 1 && row >= rows) return;  // whole wave; WPR 4 grids are exact
    constexpr int E = 16 / sizeof(T);
    const T* x = reinterpret_cast<const T*>(p.A) + (int64_t)row * p.lda;
    const int nchunks = p.K / E;
    uint4 raw[NC];
#pragma unroll
    for (int i = 0; i < NC; ++i) raw[i] = reinterpret_cast<const uint4*>(x)[min(lane + L * i, nchunks - 1)];
    // (clamped chunks repeat the last chunk: harmless for a max)
    uint32_t mx = 0;
    constexpr uint32_t kAbs = sizeof(T) == 2 ? 0x7FFF7FFFu : 0x7FFFFFFFu;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const uint32_t w[4] = {raw[i].x & kAbs, raw[i].y & kAbs, raw[i].z & kAbs, raw[i].w & kAbs};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if constexpr (sizeof(T) == 2) mx = max(mx, max(w[j] & 0xFFFFu, w[j] >> 16));
            else mx = max(mx, w[j]);
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = max(mx, (uint32_t)__shfl_xor((int)mx, o, 64));
    if constexpr (WPR > 1) {
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
        __syncthreads();
        mx = max(max(red[0], red[1]), max(red[2], red[3]));
    }
    float m;
    bool bad;
    if constexpr (sizeof(T) == 2) {
        bad = mx >= 0x7C00u;
        m = __half2float(__ushort_as_half((unsigned short)mx));
    } else {
        bad = mx >= 0x7F800000u;
        m = __uint_as_float(mx);
    }
    if (bad) {
        // rare: a row holding Inf / NaN takes the fmaxf absmax of the other kernels
        // (NaN ignored, Inf kept); the row is reported through the error word
        float fm = 0.0f;
#pragma unroll
        for (int i = 0; i < NC; ++i) {
            const T* e = reinterpret_cast<const T*>(&raw[i]);
#pragma unroll
            for (int j = 0; j < E; ++j) fm = fmaxf(fm, fabsf(lds_ld(e, j)));
        }
        fm = wave_max(fm);
        if constexpr (WPR > 1) {
            __syncthreads();
            if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = __float_as_uint(fm);
            __syncthreads();
            fm = fmaxf(fmaxf(__uint_as_float(red[0]), __uint_as_float(red[1])),
                       fmaxf(__uint_as_float(red[2]), __uint_as_float(red[3])));
        }
        m = fm;
    }
    const float s = qscale_from_absmax(m);
    const float inv = 1.0f / s;
    const bool rne = (p.flags & kFlagRne) != 0;
    const bool fast = !bad;  // finite row: the short rounding sequence
    int8_t* qrow = p.q + (int64_t)row * p.ldq;
#pragma unroll
    for (int i = 0; i < NC; ++i) {
        const int c = lane + L * i;
        if (c < nchunks) {
            const T* e = reinterpret_cast<const T*>(&raw[i]);
            uint32_t w[E / 4];
#pragma unroll
            for (int g = 0; g < E / 4; ++g) {
                float v[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = lds_ld(e, 4 * g + j);
                w[g] = quant4(v, inv, rne, fast);
            }
            if constexpr (E == 8)
                *reinterpret_cast<uint2*>(qrow + c * E) = make_uint2(w[0], w[1]);
            else
                *reinterpret_cast<uint32_t*>(qrow + c * E) = w[0];
        }
    }
    for (int k0 = p.K + 8 * lane; k0 < p.ldq; k0 += 8 * L) *reinterpret_cast<uint2*>(qrow + k0) = make_uint2(0, 0);
    if (lane == 0) {
        p.s[row] = s;
        if (bad && p.err) atomicOr(p.err, 1u);
    }
}

template <typename T, int WPR>
static bool launch_quant_reg_w(const QuantParams& p, int rows, hipStream_t stream) {
    constexpr int E = 16 / sizeof(T);
    const int per_lane = (p.K / E + 64 * WPR - 1) / (64 * WPR);
    dim3 grid((rows + 4 / WPR - 1) / (4 / WPR)), block(256);
    if (per_lane <= 2) quant_rows_reg_kernel<T, 2, WPR><<<grid, block, 0, stream>>>(p, rows);
    else if (per_lane <= 4) quant_rows_reg_kernel<T, 4, WPR><<<grid, block, 0, stream>>>(p, rows);
    else if (per_lane <= 6) quant_rows_reg_kernel<T, 6, WPR><<<grid, block, 0, stream>>>(p, rows);  // K = 9728
    else if (per_lane <= 8) quant_rows_reg_kernel<T, 8, WPR><<<grid, block, 0, stream>>>(p, rows);
    else if (per_lane <= 12) quant_rows_reg_kernel<T, 12, WPR><<<grid, block, 0, stream>>>(p, rows);
    else if (per_lane <= 20) quant_rows_reg_kernel<T, 20, WPR><<<grid, block, 0, stream>>>(p, rows);
    else return false;
    return true;
}

// Four waves per row measured faster than one at 512 and 4096 rows (more waves in
// flight, a quarter of the per-lane work).
template <typename T>
static bool launch_quant_reg(const QuantParams& p, int rows, hipStream_t stream) {
    return launch_quant_reg_w<T, 4>(p, rows, stream);
}

hipError_t launch_quant(const QuantParams& p, int rows, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    const bool vec = ((reinterpret_cast<uintptr_t>(p.A) & 15) == 0) && (p.lda % 8 == 0) &&
                     (p.K % 8 == 0);
    dim3 grid(rows), block(kRowThreads);
    const size_t row_bytes = (size_t)p.K * (p.a_f16 ? 2 : 4);
    const bool qvec = ((reinterpret_cast<uintptr_t>(p.q) & 7) == 0) && (p.ldq % 8 == 0);
    if (vec && qvec && !p.gamma) {
        const bool ok = p.a_f16 ? launch_quant_reg<__half>(p, rows, stream) : launch_quant_reg<float>(p, rows, stream);
        if (ok) return hipGetLastError();
    }
    if (vec && qvec && row_bytes <= (size_t)kStageBytes) {
        // many rows: one wave per row (see quant_rows_staged_kernel)
        const bool wave_rows = rows >= 1024;
        if (wave_rows && p.gamma && (reinterpret_cast<uintptr_t>(p.gamma) & 15) == 0) {
            const bool ok = p.a_f16 ? launch_quant_norm_wave<__half>(p, rows, stream)
                                    : launch_quant_norm_wave<float>(p, rows, stream);
            if (ok) return hipGetLastError();
        }
        const dim3 sblock(wave_rows ? 64 : kRowThreads);
        if (p.a_f16) {
            if (wave_rows) quant_rows_staged_kernel<__half, 64><<<grid, sblock, row_bytes, stream>>>(p);
            else quant_rows_staged_kernel<__half, kRowThreads><<<grid, sblock, row_bytes, stream>>>(p);
        } else {
            if (wave_rows) quant_rows_staged_kernel<float, 64><<<grid, sblock, row_bytes, stream>>>(p);
            else quant_rows_staged_kernel<float, kRowThreads><<<grid, sblock, row_bytes, stream>>>(p);
        }
        return hipGetLastError();
    }
    if (p.a_f16) {
        if (vec)
            hipLaunchKernelGGL((quant_rows_kernel<__half, true>), grid, block, 0, stream, p);
        else
            hipLaunchKernelGGL((quant_rows_kernel<__half, false>), grid, block, 0, stream, p);
    } else {
        if (vec)
            hipLaunchKernelGGL((quant_rows_kernel<float, true>), grid, block, 0, stream, p);
        else
            hipLaunchKernelGGL((quant_rows_kernel<float, false>), grid, block, 0, stream, p);
    }
    return hipGetLastError();
}

// SiLU-gate on the unfused layout: Y[m, j] = SiLU(X[m, j]) * X[m, F + j] for j < F, the
// gate block then the up block of each row (src/model/cpu.rs:119-152,327-351, Cpu::swiglu,
// the reference's fallback when run_swiglu declines).  The same silu_gate as the fused
// epilogues, so a caller that takes this route gets the fused path's bits.  Eight outputs
// per thread when the strides and bases allow 16-byte fp16 / 32-byte f32 accesses.
template <typename TY>
__device__ __forceinline__ TY swiglu_out(float v) {
    if constexpr (std::is_same<TY, _Float16>::value) return f16_of_f32(v);  // f32 result, then RNE to fp16
    else return v;
}

template <typename TX, typename TY>
__global__ void swiglu_kernel(int rows, int F, const TX* __restrict__ X, int64_t ldx, TY* __restrict__ Y, int64_t ldy,
                              int vec) {
    const int per = vec ? 8 : 1;
    const int64_t chunks = (F + per - 1) / per;
    const int64_t total = (int64_t)rows * chunks;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int m = (int)(i / chunks);
        const int j0 = (int)(i - (int64_t)m * chunks) * per;
        const TX* g = X + (int64_t)m * ldx + j0;
        const TX* u = g + F;
        TY* y = Y + (int64_t)m * ldy + j0;
        if (vec && j0 + 8 <= F) {
#pragma unroll
            for (int e = 0; e < 8; ++e) y[e] = swiglu_out<TY>(silu_gate((float)g[e], (float)u[e]));
        } else {
            for (int e = 0; e < per && j0 + e < F; ++e) y[e] = swiglu_out<TY>(silu_gate((float)g[e], (float)u[e]));
        }
    }
}

template <typename TX, typename TY>
static hipError_t launch_swiglu_t(int rows, int F, const void* X, int64_t ldx, void* Y, int64_t ldy, hipStream_t st) {
    const bool vec = F % 8 == 0 && ldx % 8 == 0 && ldy % 8 == 0 && (reinterpret_cast<uintptr_t>(X) & 31) == 0 &&
                     (reinterpret_cast<uintptr_t>(Y) & 31) == 0;
    const int64_t work = (int64_t)rows * (vec ? F / 8 : F);
    const int grid = (int)std::min<int64_t>((work + 255) / 256, 4096);
    hipLaunchKernelGGL((swiglu_kernel<TX, TY>), dim3(grid), dim3(256), 0, st, rows, F,
                       reinterpret_cast<const TX*>(X), ldx, reinterpret_cast<TY*>(Y), ldy, vec ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_swiglu(int rows, int F, const void* X, int x_f16, int64_t ldx, void* Y, int y_f16, int64_t ldy,
                         hipStream_t st) {
    if (x_f16) {
        return y_f16 ? launch_swiglu_t<_Float16, _Float16>(rows, F, X, ldx, Y, ldy, st)
                     : launch_swiglu_t<_Float16, float>(rows, F, X, ldx, Y, ldy, st);
    }
    return y_f16 ? launch_swiglu_t<float, _Float16>(rows, F, X, ldx, Y, ldy, st)
                 : launch_swiglu_t<float, float>(rows, F, X, ldx, Y, ldy, st);
}

}  // namespace qlin
