// Decode chain: a sequence of quantized linears in one persistent launch (a decoder
// layer's projections, or a stack of layers), for 1..4 rows.  Each stage is the
// decode GEMV of one weight matrix (kernel (b) + (d)) with its activation quantization
// (kernel (a), after an optional RMSNorm) fused into the prologue, exactly as the
// single-linear entry points compute it.  Replaces the engine's per-linear calls of
// the decode step (src/model/dense.rs:470-530 driving src/npu.rs Linear::run).
//
// Grid.  One 512-thread workgroup per CU (all resident at once).  Stage s has
// groups_s items of 16 output channels over the whole K; workgroup b owns items
// b, b + G, b + 2G, ... and processes them in rounds of up to four, its 8 waves split
// evenly over the round's items and each item's waves splitting the K steps.
//
// Dependencies.  An item's weights do not depend on activations, so each wave issues
// its first batch of weight loads for a round before waiting for the previous stage:
// the weight stream keeps running while the stage boundary resolves.  A stage's
// outputs are written with device-coherent stores; after its last item a workgroup
// waits for its stores and adds its item count to the stage's counter.  The first
// round of the next stage waits (thread 0, bounded spin) until that counter reaches
// the stage's item count, then every workgroup loads the rows with device-coherent
// loads, applies the RMSNorm if configured, and quantizes them into LDS.  The
// workgroup completing the last stage resets the counters for the next launch.  A
// wait that exceeds the spin bound sets bit 1 of the error word and gives up, so every
// wave always reaches the end of the kernel.
#include <type_traits>

#include "qlin_chain.hpp"
#include "qlin_gemv_parts.hpp"
#include "qlin_rows.hpp"

namespace qlin {

constexpr int kChainWaves = 8;
constexpr int kChainThreads = 64 * kChainWaves;
static_assert(kChainThreads == kChainThreadsPerBlock, "host and kernel agree on the block size");
constexpr int kChainBatch = 2;  // wave steps per register buffer

typedef unsigned int u32x4c __attribute__((ext_vector_type(4)));
constexpr int kChainRsrc = 0x00020000;
constexpr int kSc1 = 16;  // cache policy: coherent at device scope

__device__ __forceinline__ __amdgpu_buffer_rsrc_t chain_rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kChainRsrc);
}

// Registers of one batch of wave steps: gate (or plain) and up weight blocks.
template <bool SWIGLU>
struct ChainBuf {
    v4i bg[kChainBatch][2];
    v4i bu[SWIGLU ? kChainBatch : 1][2];
};

// Unconditional loads: a step past the end re-reads the last one (an L2 hit).
template <int BITS, bool SWIGLU>
__device__ __forceinline__ void chain_load(ChainBuf<SWIGLU>& b, const uint8_t* wg, const uint8_t* wu, int first,
                                           int stride, int steps) {
#pragma unroll
    for (int i = 0; i < kChainBatch; ++i) {
        const int st = min(first + stride * i, steps - 1);
        b.bg[i][0] = ld16(wg + (int64_t)st * 128);
        b.bg[i][1] = ld16(wg + (int64_t)st * 128 + 64);
        if constexpr (SWIGLU) {
            b.bu[i][0] = ld16(wu + (int64_t)st * 128);
            b.bu[i][1] = ld16(wu + (int64_t)st * 128 + 64);
        }
    }
}

template <int BITS, bool SWIGLU>
__device__ __forceinline__ void chain_compute(v4i& ag, v4i& au, const ChainBuf<SWIGLU>& b, const uint8_t* arow,
                                              int first, int stride, int steps) {
    constexpr int KS = BITS == 4 ? 256 : 128;
#pragma unroll
    for (int i = 0; i < kChainBatch; ++i) {
        const int st = first + stride * i;
        if (st < steps) {
            v4i a[4];
            a_from_lds<BITS>(a, arow + st * KS);
            mfma_step<BITS>(ag, b.bg[i], a);
            if constexpr (SWIGLU) mfma_step<BITS>(au, b.bu[i], a);
        }
    }
}

// Thread 0 waits until *cnt >= target (bounded), then the workgroup proceeds.
__device__ __forceinline__ void chain_wait(const ChainParams& p, const uint32_t* cnt, uint32_t target) {
    if (threadIdx.x == 0) {
        int spins = 0;
        while (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            if (++spins > p.spin_limit) {
                atomicOr(p.err, 2u);
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __syncthreads();
}

// Activation prologue of one stage: rows [0, M) of the stage input (fp16) into LDS,
// RMSNorm scale, per-token scale, quantized rows in the order the stage's MFMA step
// expects, a zero row M.  Same arithmetic as the GEMV's fused prologue.
template <int BITS, int MR>
__device__ void chain_prologue(const ChainParams& p, const ChainStage& st, const __half* in, int64_t ld_in,
                               bool coherent, uint8_t* lds_q, int astride, __half* lds_x, float* s_rows,
                               float* s_inv, float (*s_red)[4], int* s_bad) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int M = p.M, K = st.K;
    const int ng = K >> 3;  // 8-value groups per row
    // 1. raw rows into LDS, 16 bytes per load, all loads of a thread issued together
    {
        const __amdgpu_buffer_rsrc_t r = chain_rsrc(in, (int64_t)(M - 1) * ld_in * 2 + (int64_t)K * 2);
        const int total = M * ng;
        constexpr int B = 4;
        for (int c0 = tid; c0 < total; c0 += kChainThreads * B) {
            u32x4c v[B];
#pragma unroll
            for (int i = 0; i < B; ++i) {
                const int c = min(c0 + kChainThreads * i, total - 1);
                const int m = c / ng, g = c - m * ng;
                const int off = (int)(((int64_t)m * ld_in + 8 * g) * 2);
                v[i] = coherent ? __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kSc1)
                                : __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < B; ++i) {
                const int c = min(c0 + kChainThreads * i, total - 1);
                const int m = c / ng, g = c - m * ng;
                *reinterpret_cast<u32x4c*>(lds_x + m * K + 8 * g) = v[i];
            }
        }
    }
    __syncthreads();
    // 2. RMSNorm scale per row (wave m computes row m), reference summation order
    if (st.gamma) {
        if (wave < M) {
            const __half* xr = lds_x + wave * K;
            float sum;
            if (st.flags & kFlagNormSeq)
                sum = lane == 0 ? lds_sumsq_seq(xr, K) : 0.0f;  // src/ops/norm.rs:38
            else
                sum = lds_sumsq_neon16(xr, K);  // src/model/cpu.rs:14-35
            if (lane == 0) s_inv[wave] = 1.0f / __builtin_sqrtf(sum / (float)K + st.eps);
        }
        __syncthreads();
    }
    float nscale[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) nscale[m] = (st.gamma && m < M) ? s_inv[m] : 1.0f;
    // 3. absmax (after the norm) and finiteness, per row
    float mx[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) mx[m] = 0.0f;
    int bad = 0;
    for (int c = tid; c < M * ng; c += kChainThreads) {
        const int m = c / ng, g = c - m * ng;
        float v[8];
        const uint4 raw = *reinterpret_cast<const uint4*>(lds_x + m * K + 8 * g);
        const __half2* h = reinterpret_cast<const __half2*>(&raw);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float2 f = __half22float2(h[i]);
            v[2 * i] = f.x;
            v[2 * i + 1] = f.y;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) bad |= !__builtin_isfinite(v[e]);
        float ns = 1.0f;
#pragma unroll
        for (int mm = 0; mm < MR; ++mm)
            if (mm == m) ns = nscale[mm];
        if (st.gamma) {
            const float4 ga = *reinterpret_cast<const float4*>(st.gamma + 8 * g);
            const float4 gb = *reinterpret_cast<const float4*>(st.gamma + 8 * g + 4);
            const float gg[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = (v[e] * ns) * gg[e];
        }
        float lm = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) lm = fmaxf(lm, fabsf(v[e]));
#pragma unroll
        for (int mm = 0; mm < MR; ++mm)
            if (mm == m) mx[mm] = fmaxf(mx[mm], lm);
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        const float w = wave_max_nonneg(mx[m]);
        if (lane == 0) s_red[wave][m] = w;
    }
    const bool any_bad = __ballot(bad) != 0;
    if (lane == 0) s_bad[wave] = any_bad;
    lds_barrier();
    // per-token scales, computed by every thread from the wave maxima
    int b = 0;
#pragma unroll
    for (int w = 0; w < kChainWaves; ++w) b |= s_bad[w];
    float inv[MR];
    bool finite = true;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        float am = 0.0f;
#pragma unroll
        for (int w = 0; w < kChainWaves; ++w) am = fmaxf(am, s_red[w][m]);
        const float s = qscale_from_absmax(am);  // src/npu.rs:1101-1106
        finite &= __builtin_isfinite(s);
        inv[m] = 1.0f / s;
        if (tid == 0 && m < M) s_rows[m] = s;
    }
    if (tid == 0 && b && blockIdx.x == 0) atomicOr(p.err, 1u);
    // 4. quantize into LDS (k order for both widths); a finite row (the usual case)
    // takes the short rounding sequence
    const bool rne = (st.flags & kFlagRne) != 0;
    const bool fast = !b && finite;
    for (int c = tid; c < M * ng; c += kChainThreads) {
        const int m = c / ng, g = c - m * ng;
        float v[8];
        const uint4 raw = *reinterpret_cast<const uint4*>(lds_x + m * K + 8 * g);
        const __half2* h = reinterpret_cast<const __half2*>(&raw);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float2 f = __half22float2(h[i]);
            v[2 * i] = f.x;
            v[2 * i + 1] = f.y;
        }
        if (st.gamma) {
            float ns = 1.0f;
#pragma unroll
            for (int mm = 0; mm < MR; ++mm)
                if (mm == m) ns = nscale[mm];
            const float4 ga = *reinterpret_cast<const float4*>(st.gamma + 8 * g);
            const float4 gb = *reinterpret_cast<const float4*>(st.gamma + 8 * g + 4);
            const float gg[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = (v[e] * ns) * gg[e];
        }
        float im = 1.0f;
#pragma unroll
        for (int mm = 0; mm < MR; ++mm)
            if (mm == m) im = inv[mm];
        int q[8];
        if (fast && rne) {
#pragma unroll
            for (int e = 0; e < 8; ++e) q[e] = quant_finite<true>(v[e], im);
        } else if (fast) {
#pragma unroll
            for (int e = 0; e < 8; ++e) q[e] = quant_finite<false>(v[e], im);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) q[e] = quant_one(v[e], im, rne);  // src/npu.rs:1107-1110
        }
        uint32_t w0 = 0, w1 = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            w0 |= (uint32_t)(q[e] & 0xff) << (8 * e);
            w1 |= (uint32_t)(q[4 + e] & 0xff) << (8 * e);
        }
        *reinterpret_cast<uint2*>(lds_q + m * astride + 8 * g) = make_uint2(w0, w1);
    }
    // zero the K..Kp tail of each row and the whole zero row M
    for (int m = 0; m < M; ++m)
        for (int k = K + tid * 8; k < st.Kp; k += kChainThreads * 8)
            *reinterpret_cast<uint2*>(lds_q + m * astride + k) = make_uint2(0, 0);
    for (int k = tid * 16; k < st.Kp; k += kChainThreads * 16)
        *reinterpret_cast<uint4*>(lds_q + M * astride + k) = make_uint4(0, 0, 0, 0);
    __syncthreads();
}

// All rounds of one stage for this workgroup.  Returns the number of items done.
template <int BITS, bool SWIGLU, int MR>
__device__ int chain_stage(const ChainParams& p, const ChainStage& st, int s, uint8_t* smem, float* s_rows,
                           float* s_inv, float (*s_red)[4], int* s_bad) {
    constexpr int KS = BITS == 4 ? 256 : 128;
    constexpr int LIVE_LANES = 16 * ((MR + 3) / 4);
    constexpr int REGS = MR < 4 ? MR : 4;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int G = gridDim.x;
    const int b = blockIdx.x;
    const int n_items = st.groups > b ? (st.groups - 1 - b) / G + 1 : 0;
    const int steps = st.Kp / KS;
    const int Nh = st.N >> 1;
    const int astride = p.kp_max + 16;
    uint8_t* lds_q = smem;
    int* red = reinterpret_cast<int*>(smem + p.lds_q_bytes);
    __half* lds_x = reinterpret_cast<__half*>(smem + p.lds_q_bytes + p.lds_red_bytes);
    const bool last = s == p.n_stages - 1;
    const bool from_x = st.in == nullptr;
    const __half* in = from_x ? p.x + st.x_offset : st.in;
    const int64_t ld_in = from_x ? p.ldx : st.ld_in;
    _Float16* out = last ? p.y : st.out;
    const int64_t ld_out = last ? p.ldy : st.ld_out;
    const int m_lane = lane & 15;
    const bool live = m_lane < p.M;

    if (n_items == 0) return 0;
    for (int r = 0; r < n_items; r += 4) {
        const int nr = min(4, n_items - r);
        const int wpi = kChainWaves / nr;
        const int item = wave / wpi;
        const bool active = item < nr;
        const int wave_in = wave - item * wpi;
        const int g = b + (r + min(item, nr - 1)) * G;
        const int r0 = 16 * g;
        const uint8_t* wg = st.W + (int64_t)(r0 + (lane & 15)) * st.wrow + (lane >> 4) * 16;
        const uint8_t* wu = SWIGLU ? st.W + (int64_t)(Nh + r0 + (lane & 15)) * st.wrow + (lane >> 4) * 16 : nullptr;
        ChainBuf<SWIGLU> b0, b1;
        int base = wave_in;
        if (active) chain_load<BITS, SWIGLU>(b0, wg, wu, base, wpi, steps);
        if (r == 0) {
            // first round: the weights above are in flight while the stage input resolves
            if (s > 0) chain_wait(p, p.counters + (s - 1), (uint32_t)p.stages[s - 1].groups);
            chain_prologue<BITS, MR>(p, st, in, ld_in, !from_x, lds_q, astride, lds_x, s_rows, s_inv, s_red, s_bad);
        }
        v4i ag = {0, 0, 0, 0}, au = {0, 0, 0, 0};
        if (active) {
            const uint8_t* arow = lds_q + (live ? m_lane : p.M) * astride + (lane >> 4) * (BITS == 4 ? 32 : 16);
            const int span = wpi * kChainBatch;
            while (base < steps) {
                const int nb = base + span;
                if (nb < steps) chain_load<BITS, SWIGLU>(b1, wg, wu, nb, wpi, steps);
                chain_compute<BITS, SWIGLU>(ag, au, b0, arow, base, wpi, steps);
                base = nb;
                if (base >= steps) break;
                const int nb2 = base + span;
                if (nb2 < steps) chain_load<BITS, SWIGLU>(b0, wg, wu, nb2, wpi, steps);
                chain_compute<BITS, SWIGLU>(ag, au, b1, arow, base, wpi, steps);
                base = nb2;
            }
        }
        // cross-wave reduction of each item's partial sums, then the epilogue
        if (active && lane < LIVE_LANES) {
#pragma unroll
            for (int i = 0; i < REGS; ++i) {
                red[(wave * LIVE_LANES + lane) * REGS + i] = ag[i];
                if constexpr (SWIGLU) red[kChainWaves * LIVE_LANES * REGS + (wave * LIVE_LANES + lane) * REGS + i] = au[i];
            }
        }
        __syncthreads();
        if (tid < nr * 16 * p.M) {
            const int j = tid / (16 * p.M), rem = tid - j * 16 * p.M;
            const int m = rem >> 4, n = rem & 15;
            const int src = (16 * (m >> 2) + n) * REGS + (m & 3);
            int vg = 0, vu = 0;
            for (int w = j * wpi; w < (j + 1) * wpi; ++w) {
                vg += red[w * LIVE_LANES * REGS + src];
                if constexpr (SWIGLU) vu += red[kChainWaves * LIVE_LANES * REGS + w * LIVE_LANES * REGS + src];
            }
            const int cg = 16 * (b + (r + j) * G) + n;
            const int ncols = SWIGLU ? Nh : st.N;
            if (cg < ncols) {
                const int a_g = BITS == 4 ? (vg >> 4) : vg;  // exact: W4 sums carry a factor 16
                float o = ((float)a_g * s_rows[m]) * st.wscale[cg];  // src/npu.rs:1117
                if constexpr (SWIGLU) {
                    const int a_u = BITS == 4 ? (vu >> 4) : vu;
                    const float up = ((float)a_u * s_rows[m]) * st.wscale[Nh + cg];
                    o = silu_gate(o, up);  // src/npu.rs:1202-1208
                } else if (st.res_kind) {
                    // src/model/dense.rs:486-489: hidden + projected * residual_multiplier; an
                    // earlier stage's rows are read device-coherently like a stage input
                    const float pr = o * st.rmult;
                    float hv;
                    if (st.res_kind == 1) {
                        hv = __half2float(p.x[(int64_t)m * p.ldx + st.res_x_offset + cg]);
                    } else {
                        const uint16_t bits = __hip_atomic_load(reinterpret_cast<const uint16_t*>(st.res) + (int64_t)m * st.ld_res + cg,
                                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        hv = (float)__builtin_bit_cast(_Float16, bits);
                    }
                    o = hv + pr;
                }
                const _Float16 h = f16_of_f32(o);
                __hip_atomic_store(reinterpret_cast<uint16_t*>(out) + (int64_t)m * ld_out + cg,
                                   __builtin_bit_cast(uint16_t, h), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __syncthreads();  // the reduction area is reused by the next round
    }
    return n_items;
}

template <int MR>
__global__ __launch_bounds__(kChainThreads) void chain_kernel(ChainParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float s_rows[4], s_inv[4];
    __shared__ float s_red[kChainWaves][4];
    __shared__ int s_bad[kChainWaves];
    for (int s = 0; s < p.n_stages; ++s) {
        const ChainStage& st = p.stages[s];
        const bool sw = (st.flags & kFlagSwiglu) != 0;
        int done;
        if (st.bits == 4)
            done = sw ? chain_stage<4, true, MR>(p, st, s, smem, s_rows, s_inv, s_red, s_bad)
                      : chain_stage<4, false, MR>(p, st, s, smem, s_rows, s_inv, s_red, s_bad);
        else
            done = sw ? chain_stage<8, true, MR>(p, st, s, smem, s_rows, s_inv, s_red, s_bad)
                      : chain_stage<8, false, MR>(p, st, s, smem, s_rows, s_inv, s_red, s_bad);
        if (done > 0) {
            wait_all_memory();  // this wave's coherent output stores have completed
            __syncthreads();
            if (threadIdx.x == 0) {
                const uint32_t old = atomicAdd(p.counters + s, (uint32_t)done);
                if (s == p.n_stages - 1 && old + done == (uint32_t)st.groups) {
                    // every item of every stage is complete: reset for the next launch
                    for (int i = 0; i < p.n_stages; ++i)
                        __hip_atomic_store(p.counters + i, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
    }
}

size_t chain_lds_bytes(int max_rows, int kp_max, int k_max, size_t* q_bytes, size_t* red_bytes) {
    const int mr = max_rows <= 1 ? 1 : 4;
    const size_t q = (size_t)(mr + 1) * (kp_max + 16);
    const size_t red = (size_t)2 * kChainWaves * 16 * (mr < 4 ? mr : 4) * sizeof(int);
    const size_t x = (size_t)mr * k_max * sizeof(__half);
    *q_bytes = (q + 15) & ~(size_t)15;
    *red_bytes = (red + 15) & ~(size_t)15;
    return *q_bytes + *red_bytes + x;
}

int chain_resident_per_cu(int max_rows, size_t lds) {
    int n = 0;
    const void* f = max_rows <= 1 ? reinterpret_cast<const void*>(&chain_kernel<1>)
                                  : reinterpret_cast<const void*>(&chain_kernel<4>);
    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kChainMaxLds) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, kChainThreads, lds) != hipSuccess) return 0;
    return n;
}

hipError_t launch_chain(const ChainParams& p, int grid, size_t lds, hipStream_t stream) {
    if (p.M <= 1) {
        static const hipError_t a1 = hipFuncSetAttribute(reinterpret_cast<const void*>(&chain_kernel<1>),
                                                         hipFuncAttributeMaxDynamicSharedMemorySize, kChainMaxLds);
        if (a1 != hipSuccess) return a1;
        chain_kernel<1><<<grid, kChainThreads, lds, stream>>>(p);
    } else {
        static const hipError_t a4 = hipFuncSetAttribute(reinterpret_cast<const void*>(&chain_kernel<4>),
                                                         hipFuncAttributeMaxDynamicSharedMemorySize, kChainMaxLds);
        if (a4 != hipSuccess) return a4;
        chain_kernel<4><<<grid, kChainThreads, lds, stream>>>(p);
    }
    return hipGetLastError();
}

}  // namespace qlin
