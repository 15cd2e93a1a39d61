// Kernel (b) + (d): decode GEMV for 1..16 rows with the dequant / SiLU-gate epilogue.
//
// Replaces the native library's per-call scan/quantize, NPU int4 GEMM and CPU
// reduce/dequant for small M (QWEN3_W4A8_PIPELINE_REVIEW_20261020.md:24-31).
//
// Mapping.  A workgroup (4 waves) owns one group of 16 output channels (plus the
// matching 16 "up" channels for SwiGLU) and one K slice; `splits` workgroups share
// a group along K and combine int32 partials with atomics, the last one to arrive
// running the epilogue and re-zeroing the partials and its counter.
//
// Streaming.  One wave step covers 16 weight rows x 128 bytes (a full 128-byte line
// per row): lane l loads 16 bytes of row l%16 at byte 16*(l/16) and 64 + 16*(l/16).
// For W8 those bytes are the B operand of v_mfma_i32_16x16x64_i8 directly; for W4
// each 16 bytes unpack in registers into two B operands.  The unpack keeps the
// nibble in the high half of each byte (w & 0xF0, w << 4 & 0xF0), i.e. 16*code as
// an exact int8, so the int32 sum is 16x the true one and is shifted back (exact)
// before dequant.  The two nibble halves come out as even-k / odd-k byte groups;
// the activation bytes are stored in LDS in that same order so the k index of A
// and B agree lane by lane.  Rows beyond M feed zeros to the matrix core.
//
// Activations.  The prologue quantizes (or copies) the rows for the workgroup's K
// slice into LDS.  In fused mode every workgroup scans the whole row for its absmax
// (and RMSNorm sum when gamma is given); max is order independent, so each
// workgroup derives the same s and q bit for bit.  The first batch of weight loads
// is issued before the prologue so the scan overlaps HBM latency.
#include "qlin_rows.hpp"

namespace qlin {

constexpr int kGemvThreads = 256;
constexpr int kGemvBatch = 4;  // wave steps in flight per buffer

template <int BITS, bool SWIGLU>
struct GemvTraits {
    static constexpr int KS = BITS == 4 ? 256 : 128;  // k per wave step
};

__device__ __forceinline__ v4i ld16(const uint8_t* p) {
    return *reinterpret_cast<const v4i*>(p);
}

__device__ __forceinline__ v4i lds16(const uint8_t* p) {
    return *reinterpret_cast<const v4i*>(p);
}

template <int BITS>
__device__ __forceinline__ void step_mfma(v4i& acc, const v4i b[2], const uint8_t* arow, bool live) {
    const v4i zero = {0, 0, 0, 0};
    if constexpr (BITS == 8) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            v4i a = live ? lds16(arow + 64 * j) : zero;
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b[j], acc, 0, 0, 0);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            v4i lo, hi;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                lo[d] = (b[j][d] << 4) & 0xF0F0F0F0;
                hi[d] = b[j][d] & 0xF0F0F0F0;
            }
            v4i b0 = {lo[0], hi[0], lo[1], hi[1]};
            v4i b1 = {lo[2], hi[2], lo[3], hi[3]};
            v4i a0 = live ? lds16(arow + 128 * j) : zero;
            v4i a1 = live ? lds16(arow + 128 * j + 16) : zero;
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, acc, 0, 0, 0);
        }
    }
}

// Packs 8 quantized values for LDS: natural order for W8, even-k then odd-k for W4.
template <int BITS>
__device__ __forceinline__ uint2 pack_q8(const int v[8]) {
    uint32_t w0 = 0, w1 = 0;
    if constexpr (BITS == 8) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w0 |= (uint32_t)(v[i] & 0xff) << (8 * i);
            w1 |= (uint32_t)(v[4 + i] & 0xff) << (8 * i);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w0 |= (uint32_t)(v[2 * i] & 0xff) << (8 * i);
            w1 |= (uint32_t)(v[2 * i + 1] & 0xff) << (8 * i);
        }
    }
    return make_uint2(w0, w1);
}

template <typename T, int BITS, bool VEC>
__device__ void stage_fused(const GemvParams& p, uint8_t* lds_a, int stride, int kb, int ke,
                            float* lds_s, float* lds_red) {
    const bool gvec = VEC && ((reinterpret_cast<uintptr_t>(p.gamma) & 15) == 0);
    const bool rne = (p.flags & kFlagRne) != 0;
    for (int m = 0; m < p.M; ++m) {
        const T* x = reinterpret_cast<const T*>(p.A) + (int64_t)m * p.lda;
        float nscale = 1.0f;
        if (p.gamma) nscale = block_rms_scale<T>(x, p.K, p.eps, (p.flags & kFlagNormSeq) != 0, lds_red);
        int bad = 0;
        const float s = block_row_scale<T, VEC>(x, p.K, p.gamma, gvec, nscale, &bad, lds_red);
        const float inv = 1.0f / s;
        if (threadIdx.x == 0) {
            lds_s[m] = s;
            if (bad && p.err && blockIdx.x == 0) atomicOr(p.err, 1u);
        }
        for (int k0 = kb + threadIdx.x * 8; k0 < ke; k0 += kGemvThreads * 8) {
            float v[8];
            load8<T, VEC>(x, k0, p.K, v);
            if (p.gamma) {
                float g[8];
                load8_gamma(p.gamma, k0, p.K, gvec, g);
                apply_norm8(v, g, nscale);
            }
            int qv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) qv[i] = quant_one(v[i], inv, rne);
            *reinterpret_cast<uint2*>(lds_a + m * stride + (k0 - kb)) = pack_q8<BITS>(qv);
        }
    }
}

template <int BITS>
__device__ void stage_quantized(const GemvParams& p, uint8_t* lds_a, int stride, int kb, int ke,
                                float* lds_s) {
    if (threadIdx.x < p.M) lds_s[threadIdx.x] = p.s ? p.s[threadIdx.x] : 0.0f;
    for (int m = 0; m < p.M; ++m) {
        const int8_t* qrow = p.q + (int64_t)m * p.ldq;
        for (int k0 = kb + threadIdx.x * 8; k0 < ke; k0 += kGemvThreads * 8) {
            uint2 raw = *reinterpret_cast<const uint2*>(qrow + k0);
            uint2 out = raw;
            if constexpr (BITS == 4) {
                // [k0..k7] -> [k0,k2,k4,k6 | k1,k3,k5,k7]
                out.x = __builtin_amdgcn_perm(raw.y, raw.x, 0x06040200u);
                out.y = __builtin_amdgcn_perm(raw.y, raw.x, 0x07050301u);
            }
            *reinterpret_cast<uint2*>(lds_a + m * stride + (k0 - kb)) = out;
        }
    }
}

template <int BITS, bool SWIGLU>
__device__ __forceinline__ void load_batch(v4i (&bg)[kGemvBatch][2], v4i (&bu)[kGemvBatch][2],
                                           const uint8_t* wg, const uint8_t* wu, int base, int end) {
#pragma unroll
    for (int i = 0; i < kGemvBatch; ++i) {
        const int st = base + 4 * i;
        if (st < end) {
            bg[i][0] = ld16(wg + (int64_t)st * 128);
            bg[i][1] = ld16(wg + (int64_t)st * 128 + 64);
            if constexpr (SWIGLU) {
                bu[i][0] = ld16(wu + (int64_t)st * 128);
                bu[i][1] = ld16(wu + (int64_t)st * 128 + 64);
            }
        }
    }
}

template <int BITS, bool SWIGLU>
__device__ __forceinline__ void compute_batch(v4i& ag, v4i& au, const v4i (&bg)[kGemvBatch][2],
                                              const v4i (&bu)[kGemvBatch][2], const uint8_t* arow,
                                              int base, int end, int step_begin, bool live) {
    constexpr int KS = GemvTraits<BITS, SWIGLU>::KS;
#pragma unroll
    for (int i = 0; i < kGemvBatch; ++i) {
        const int st = base + 4 * i;
        if (st < end) {
            const uint8_t* a = arow + (st - step_begin) * KS;
            step_mfma<BITS>(ag, bg[i], a, live);
            if constexpr (SWIGLU) step_mfma<BITS>(au, bu[i], a, live);
        }
    }
}

template <int BITS, bool SWIGLU>
__device__ __forceinline__ void gemv_finish(const GemvParams& p, int m, int n, int r0, int vg,
                                            int vu, const float* lds_s) {
    const int Nh = p.N >> 1;
    const int ag = BITS == 4 ? (vg >> 4) : vg;  // exact: W4 sums carry a factor 16
    if (p.c_kind == 2) {
        if (r0 + n < p.N) reinterpret_cast<int32_t*>(p.C)[(int64_t)m * p.ldc + r0 + n] = ag;
        return;
    }
    const float sm = lds_s[m];
    const int cg = r0 + n;
    float out = ((float)ag * sm) * p.wscale[cg];  // src/npu.rs:1117
    int col = cg;
    if constexpr (SWIGLU) {
        const int au = BITS == 4 ? (vu >> 4) : vu;
        const float up = ((float)au * sm) * p.wscale[Nh + cg];
        out = (out / (1.0f + expf(-out))) * up;  // src/npu.rs:1202-1208
    }
    const int ncols = SWIGLU ? Nh : p.N;
    if (col < ncols) {
        if (p.c_kind == 1)
            reinterpret_cast<_Float16*>(p.C)[(int64_t)m * p.ldc + col] = f16_of_f32(out);
        else
            reinterpret_cast<float*>(p.C)[(int64_t)m * p.ldc + col] = out;
    }
}

// MODE 0: q/s given; 1: fused quant of f16 rows; 2: fused quant of f32 rows.
template <int BITS, bool SWIGLU, int MODE, bool VEC>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(GemvParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int KS = GemvTraits<BITS, SWIGLU>::KS;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int rg = blockIdx.x / p.splits, z = blockIdx.x - rg * p.splits;
    const int total_steps = p.Kp / KS;
    const int step_begin = z * p.steps_per_split;
    const int step_end = min(step_begin + p.steps_per_split, total_steps);
    const int kb = step_begin * KS, ke = step_end * KS;
    const int stride = p.steps_per_split * KS + 16;

    uint8_t* lds_a = smem;
    float* lds_s = reinterpret_cast<float*>(smem + p.M * stride);
    float* lds_red = lds_s + kGemvMaxRows;              // 8 words of reduction scratch
    int* red = reinterpret_cast<int*>(lds_red + 8);     // [2][4 waves][64 lanes][4]
    __shared__ int last_flag;

    const int r0 = rg * 16;
    const int Nh = p.N >> 1;
    const uint8_t* wg = p.W + (int64_t)(r0 + (lane & 15)) * p.wrow + (lane >> 4) * 16;
    const uint8_t* wu = SWIGLU ? p.W + (int64_t)(Nh + r0 + (lane & 15)) * p.wrow + (lane >> 4) * 16
                               : nullptr;

    v4i bg0[kGemvBatch][2], bu0[kGemvBatch][2], bg1[kGemvBatch][2], bu1[kGemvBatch][2];
    int base = step_begin + wave;
    load_batch<BITS, SWIGLU>(bg0, bu0, wg, wu, base, step_end);

    if constexpr (MODE == 0) {
        stage_quantized<BITS>(p, lds_a, stride, kb, ke, lds_s);
    } else if constexpr (MODE == 1) {
        stage_fused<__half, BITS, VEC>(p, lds_a, stride, kb, ke, lds_s, lds_red);
    } else {
        stage_fused<float, BITS, VEC>(p, lds_a, stride, kb, ke, lds_s, lds_red);
    }
    __syncthreads();

    const int m_lane = lane & 15;
    const bool live = m_lane < p.M;
    // rows >= M read row M-1 (in bounds) and feed zeros instead
    const uint8_t* arow = lds_a + min(m_lane, p.M - 1) * stride + (lane >> 4) * (BITS == 4 ? 32 : 16);
    v4i ag = {0, 0, 0, 0}, au = {0, 0, 0, 0};
    while (base < step_end) {
        const int nb = base + 4 * kGemvBatch;
        load_batch<BITS, SWIGLU>(bg1, bu1, wg, wu, nb, step_end);
        compute_batch<BITS, SWIGLU>(ag, au, bg0, bu0, arow, base, step_end, step_begin, live);
        base = nb;
        if (base >= step_end) break;
        const int nb2 = base + 4 * kGemvBatch;
        load_batch<BITS, SWIGLU>(bg0, bu0, wg, wu, nb2, step_end);
        compute_batch<BITS, SWIGLU>(ag, au, bg1, bu1, arow, base, step_end, step_begin, live);
        base = nb2;
    }

    // cross-wave reduction: lane l holds D[4*(l/16)+i][l%16]
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        red[(wave * 64 + lane) * 4 + i] = ag[i];
        if constexpr (SWIGLU) red[1024 + (wave * 64 + lane) * 4 + i] = au[i];
    }
    __syncthreads();
    int vg = 0, vu = 0;
    const int m = tid >> 4, n = tid & 15;
    const bool owner = tid < 16 * p.M;
    if (owner) {
        const int src = (16 * (m >> 2) + n) * 4 + (m & 3);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            vg += red[w * 256 + src];
            if constexpr (SWIGLU) vu += red[1024 + w * 256 + src];
        }
    }
    if (p.splits == 1) {
        if (owner) gemv_finish<BITS, SWIGLU>(p, m, n, r0, vg, vu, lds_s);
        return;
    }
    int32_t* pg = p.part + (int64_t)m * p.Np + r0 + n;
    int32_t* pu = p.part + (int64_t)m * p.Np + Nh + r0 + n;
    if (owner) {
        atomicAdd(pg, vg);  // performed in L2 atomically; device-coherent
        if constexpr (SWIGLU) atomicAdd(pu, vu);
    }
    wait_all_memory();
    __syncthreads();
    if (tid == 0) last_flag = atomicAdd(&p.counters[rg], 1u) == (unsigned)(p.splits - 1);
    __syncthreads();
    if (!last_flag) return;
    if (owner) {  // atomic exchange reads every split's contribution and re-zeroes the slot
        vg = atomicExch(pg, 0);
        if constexpr (SWIGLU) vu = atomicExch(pu, 0);
        gemv_finish<BITS, SWIGLU>(p, m, n, r0, vg, vu, lds_s);
    }
    if (tid == 0) atomicExch(&p.counters[rg], 0u);
}

static size_t gemv_lds_bytes(int M, int steps_per_split, int KS) {
    return (size_t)M * (steps_per_split * KS + 16) + sizeof(float) * (kGemvMaxRows + 8) +
           sizeof(int) * 2 * 4 * 64 * 4;
}

template <int BITS, bool SWIGLU>
static hipError_t launch_gemv_t(const GemvParams& p, hipStream_t stream, size_t lds) {
    const int groups = (SWIGLU ? (p.N >> 1) : p.Np) / 16;
    dim3 grid(groups * p.splits), block(kGemvThreads);
    const bool vec = p.A && ((reinterpret_cast<uintptr_t>(p.A) & 15) == 0) && (p.lda % 8 == 0) &&
                     (p.K % 8 == 0);
    if (!p.A)
        hipLaunchKernelGGL((gemv_kernel<BITS, SWIGLU, 0, false>), grid, block, lds, stream, p);
    else if (p.a_f16 && vec)
        hipLaunchKernelGGL((gemv_kernel<BITS, SWIGLU, 1, true>), grid, block, lds, stream, p);
    else if (p.a_f16)
        hipLaunchKernelGGL((gemv_kernel<BITS, SWIGLU, 1, false>), grid, block, lds, stream, p);
    else if (vec)
        hipLaunchKernelGGL((gemv_kernel<BITS, SWIGLU, 2, true>), grid, block, lds, stream, p);
    else
        hipLaunchKernelGGL((gemv_kernel<BITS, SWIGLU, 2, false>), grid, block, lds, stream, p);
    return hipGetLastError();
}

hipError_t launch_gemv(const GemvParams& p, int bits, hipStream_t stream) {
    const int KS = bits == 4 ? 256 : 128;
    const size_t lds = gemv_lds_bytes(p.M, p.steps_per_split, KS);
    const bool sw = (p.flags & kFlagSwiglu) != 0;
    if (bits == 4) return sw ? launch_gemv_t<4, true>(p, stream, lds) : launch_gemv_t<4, false>(p, stream, lds);
    return sw ? launch_gemv_t<8, true>(p, stream, lds) : launch_gemv_t<8, false>(p, stream, lds);
}

size_t gemv_lds_bytes_for(int M, int steps_per_split, int bits) {
    return gemv_lds_bytes(M, steps_per_split, bits == 4 ? 256 : 128);
}

}  // namespace qlin
