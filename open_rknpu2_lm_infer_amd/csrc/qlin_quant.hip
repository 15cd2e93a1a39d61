// Kernel (a): per-token activation quantization, optionally after RMSNorm.
//
// One 256-thread workgroup per row.  Pass 1 (absmax + finiteness, with the norm
// applied on the fly) and pass 2 (quantize, 8 values per thread per iteration,
// one 64-bit store) read the row from global memory; the second read hits L1/L2.
// The replaced library stage is the CPU scan + quantize of rk_npu_w4a8_quant.cpp
// (QWEN3_W4A8_PIPELINE_REVIEW_20261020.md:26-27); the arithmetic is the oracle's,
// src/npu.rs:1101-1110.
#include "qlin_rows.hpp"

namespace qlin {

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
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w0 |= (uint32_t)(quant_one(v[i], inv, rne) & 0xff) << (8 * i);
            w1 |= (uint32_t)(quant_one(v[4 + i], inv, rne) & 0xff) << (8 * i);
        }
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

hipError_t launch_quant(const QuantParams& p, int rows, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    const bool vec = ((reinterpret_cast<uintptr_t>(p.A) & 15) == 0) && (p.lda % 8 == 0) &&
                     (p.K % 8 == 0);
    dim3 grid(rows), block(kRowThreads);
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

}  // namespace qlin
