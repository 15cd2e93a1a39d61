// Decode chain: a sequence of quantized linears in one persistent launch (a decoder
// layer's projections, or a stack of layers), for 1..4 rows.  Each stage is the
// decode GEMV of one weight matrix (kernels (b) + (d)) with its activation
// quantization (kernel (a), after an optional RMSNorm) and optional residual update,
// exactly as the single-linear entry points compute it.  Replaces the engine's
// per-linear calls of the decode step (src/model/dense.rs:398-540 driving
// src/npu.rs Linear::run).
//
// Grid.  One workgroup per CU, all resident at once.  Each workgroup owns a fixed,
// contiguous range of output channels of every stage: ipw items of iw channels, sized
// on the host so the grid covers the stage's channels with the fewest channels per
// workgroup (e.g. 10 of N = 2560 on 256 CUs).  An item is one 16-row MFMA tile over
// the whole K; rows past the item's width re-read its last row and are not stored.
//
// Waves.  Four compute waves (one per SIMD) and four helper waves, eight for 2..4 rows
// (ChainShape).  The compute waves hold their workgroup's share of a stage's weights in
// registers (up to 40 x 16 bytes per lane, 32 for 2..4 rows) and issue no other global
// memory access, so the only thing they ever wait for is their own weight loads.  The
// helper waves do everything else: the first one (the I/O wave) polls the previous
// stage's completion flags, copies the stage input rows and the RMSNorm weights into
// LDS with direct global -> LDS copies and reads the per-channel scales and residual
// rows; all helpers compute the RMSNorm, per-token scale and quantized rows into LDS; after the products the I/O wave runs the epilogue and
// stores this workgroup's outputs.  The two groups never share a barrier: the compute
// waves wait for LDS words (input rows landed, quantized rows ready) and count
// themselves done in another; the helpers synchronize among themselves with an LDS
// counter.
//
// Per stage: (I/O) wait for stage s - 1, rows -> LDS | (compute) issue the stage's
// weight loads | (helpers) RMSNorm, per-token scale and quantized rows into LDS, same
// arithmetic as the GEMV prologue, then "rows ready" | (compute) MFMA over the weights
// in registers, int32 sums added into LDS, "done" | (I/O) dequant / SiLU-gate /
// residual epilogue, fp16 stores, then this workgroup's flag for stage s.  The weight
// loads start only once the input rows have landed: loads in flight during the
// exchange sit ahead of its polls, copies and stores in the CU's memory pipeline and
// delay every stage more than they save.
//
// Completion flags.  flags[s][b] holds the launch epoch in which workgroup b finished
// its part of stage s.  Workgroup b counts its launches in epochs[b]; all workgroups
// run every launch to its end, so they agree on the epoch and no flag or counter is
// ever reset (a graph replay is just the next epoch).  Outputs are written with
// device-coherent stores; the I/O wave waits for their completion before it stores the
// flag, and reads stage inputs with device-coherent loads after seeing every flag of
// the stage.  Every stage waits for the whole previous stage, so every earlier stage is
// complete as well.  A wait that exceeds the spin bound sets bit 1 of the error word
// and gives up, so every wave always reaches the end of the kernel.
#include "qlin_chain.hpp"
#include "qlin_gemv_parts.hpp"
#include "qlin_rows.hpp"

namespace qlin {

constexpr int kCW = kChainComputeWaves;
constexpr int kSc1 = 16;  // cache policy: coherent at device scope
constexpr int kRsrcFlags = 0x00020000;

typedef unsigned int u32x4c __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* chain_lds_ptr;

// Wave index as a wave-uniform (scalar) value: offsets derived from it stay in SGPRs.
__device__ __forceinline__ int c_wave() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Stage descriptors are read through the constant address space: scalar loads, which
// the compute waves can wait for without waiting for their weight loads.
typedef __attribute__((address_space(4))) const ChainStage ChainStageConst;
__device__ __forceinline__ ChainStage c_desc(const ChainParams& p, int s) {
#if defined(__HIP_DEVICE_COMPILE__)
    return ((ChainStageConst*)p.stages)[s];
#else
    return p.stages[s];  // the host pass never runs device code
#endif
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t c_rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcFlags);
}

// Items of stage st owned by workgroup b; item i covers output channels
// [c_first, c_first + c_width).
__device__ __forceinline__ int c_items(const ChainStage& st, int b) {
    const int c0 = b * st.ipw * st.iw;
    if (c0 >= st.ncols) return 0;
    const int n = (st.ncols - c0 + st.iw - 1) / st.iw;
    return n < st.ipw ? n : st.ipw;
}
__device__ __forceinline__ int c_first(const ChainStage& st, int b, int i) { return (b * st.ipw + i) * st.iw; }
__device__ __forceinline__ int c_width(const ChainStage& st, int b, int i) {
    const int w = st.ncols - c_first(st, b, i);
    return w < st.iw ? w : st.iw;
}

// Row items: with SwiGLU each channel item contributes a gate item (rows c) and an up
// item (rows N/2 + c), interleaved, so every stage streams plain 16-row items.
__device__ __forceinline__ int c_row_items(const ChainStage& st, int n_it) {
    return (st.flags & kFlagSwiglu) ? 2 * n_it : n_it;
}

// Weight steps f0 .. f0 + cnt - 1 of the workgroup's flat (row item, step) sequence
// into buf: lane (r, g) = (lane & 15, lane >> 4) loads bytes 16g and 64 + 16g of the
// 128-byte step of row r.  Every slot is loaded: slots past cnt read past the end of
// the buffer resource, which returns zeros without a memory access, so buf is written
// whole on one code path.
template <int E0, int E1, int NB>
__device__ __forceinline__ void c_load(v4i (&buf)[NB], const ChainStage& st, int b, int f0, int cnt) {
    const int lane = threadIdx.x & 63;
    const bool sw = (st.flags & kFlagSwiglu) != 0;
    const __amdgpu_buffer_rsrc_t r = c_rsrc(st.W, (int64_t)st.Np * st.wrow);
    const int wrow = (int)st.wrow, up_off = (st.N >> 1) * wrow, lo = (lane >> 4) * 16;
    int ri = (f0 + E0) / st.steps, t = (f0 + E0) - ri * st.steps;
    int off = 0;
#pragma unroll
    for (int e = E0; e < E1; ++e) {
        if (e == E0 || t == 0) {  // row offset of a new row item (one VALU multiply)
            const int i = sw ? ri >> 1 : ri;
            const int row = c_first(st, b, i) + min(lane & 15, c_width(st, b, i) - 1);
            off = row * wrow + lo + ((sw && (ri & 1)) ? up_off : 0);
        }
        const int o = e < cnt ? off : (int)0x80000000;  // past the resource: zeros, no access
        buf[2 * e] = __builtin_amdgcn_raw_buffer_load_b128(r, o, t * 128, 0);
        buf[2 * e + 1] = __builtin_amdgcn_raw_buffer_load_b128(r, o, t * 128 + 64, 0);
        if (++t == st.steps) {
            t = 0;
            ++ri;
        }
    }
}

// Sums of one row item into LDS: lanes 0..15 hold channel `lane`, rows 0..3 in acc[0..3].
template <int MR>
__device__ __forceinline__ void c_flush(const ChainStage& st, int b, int ri, const v4i& acc, int M, int* accg,
                                        int* accu) {
    const int lane = threadIdx.x & 63;
    const bool sw = (st.flags & kFlagSwiglu) != 0;
    const int i = sw ? ri >> 1 : ri;
    int* dst = (sw && (ri & 1)) ? accu : accg;
    if (lane < c_width(st, b, i)) {
#pragma unroll
        for (int r = 0; r < MR; ++r)
            if (r < M) atomicAdd(dst + (i * 16 + lane) * MR + r, acc[r]);
    }
}

// Matrix products of weight steps f0 .. f0 + cnt - 1 (already in buf) with the
// quantized rows in LDS.  One code path for both widths (a uniform branch per step),
// so the weight registers have a single consumer in the compute waves' loop.
template <int MR, int NB>
__device__ __forceinline__ void c_compute(const v4i (&buf)[NB], const ChainStage& st, int b, int f0, int cnt,
                                          const uint8_t* lds_q, int astride, int M, int* accg, int* accu) {
    const bool w4 = st.bits == 4;
    const int KS = w4 ? 256 : 128;
    const int lane = threadIdx.x & 63, ml = lane & 15;
    const uint8_t* arow = lds_q + (ml < M ? ml : M) * astride + (lane >> 4) * (w4 ? 32 : 16);
    int ri = f0 / st.steps, t = f0 - ri * st.steps;
    v4i acc = {0, 0, 0, 0};
    bool pending = false;
#pragma unroll
    for (int e = 0; e < NB / 2; ++e) {
        if (e < cnt) {
            const v4i w[2] = {buf[2 * e], buf[2 * e + 1]};
            v4i a[4];
            if (w4) {
                a_from_lds<4>(a, arow + t * KS);
                mfma_step<4>(acc, w, a);
            } else {
                a_from_lds<8>(a, arow + t * KS);
                mfma_step<8>(acc, w, a);
            }
            pending = true;
            if (++t == st.steps) {
                c_flush<MR>(st, b, ri, acc, M, accg, accu);
                acc = v4i{0, 0, 0, 0};
                pending = false;
                t = 0;
                ++ri;
            }
            // one step at a time: hoisting later steps' operand reads would need
            // registers the weight buffer holds
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    if (pending) c_flush<MR>(st, b, ri, acc, M, accg, accu);
}

// LDS words that order the waves of a workgroup (no s_barrier: the compute waves and
// the helpers never wait at the same barrier).
struct ChainSync {
    uint32_t rows_ready;  // stages whose quantized rows are in LDS
    uint32_t done;        // compute-wave completions, kCW per stage
    uint32_t helpers;     // helper arrivals, one per helper wave per helper barrier
    uint32_t io_mark;     // 2s once stage s's input rows are in LDS (releases the compute
                          // waves' weight loads of stage s)
};

__device__ __forceinline__ uint32_t lds_load(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Completes this wave's LDS accesses (not its global loads or stores).
__device__ __forceinline__ void wait_lds() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Waits until *w >= target.
__device__ __forceinline__ void lds_wait_ge(const uint32_t* w, uint32_t target) {
    while (lds_load(w) < target) __builtin_amdgcn_s_sleep(1);
}

// Barrier of the HW helper waves; k counts this wave's helper barriers.
template <int HW>
__device__ __forceinline__ void helper_sync(ChainSync* sy, uint32_t& k) {
    wait_lds();  // this wave's LDS writes are visible before it arrives
    ++k;
    if ((threadIdx.x & 63) == 0) atomicAdd(&sy->helpers, 1u);
    lds_wait_ge(&sy->helpers, HW * k);
}

// Waits until every workgroup has finished its part of stage s (all flags == e).
__device__ __forceinline__ void c_io_poll(const ChainParams& p, int s, uint32_t e) {
    const int lane = threadIdx.x & 63, G = gridDim.x;
    const __amdgpu_buffer_rsrc_t r = c_rsrc(p.flags + (int64_t)s * kChainFlagStride, kChainFlagStride * 4);
    for (int spins = 0;; ++spins) {
        bool ok = true;
        for (int j0 = 0; j0 < G; j0 += 256) {
            const int j = j0 + 4 * lane;
            const u32x4c v = __builtin_amdgcn_raw_buffer_load_b128(r, j * 4, 0, kSc1);
            ok &= (j >= G || v.x == e) && (j + 1 >= G || v.y == e) && (j + 2 >= G || v.z == e) &&
                  (j + 3 >= G || v.w == e);
        }
        if (__all(ok)) return;
        if (spins >= p.spin_limit) {
            if (lane == 0) atomicOr(p.err, 2u);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

__device__ __forceinline__ float c_residual(const ChainParams& p, const ChainStage& st, int m, int c) {
    if (st.res_kind == 1) return __half2float(p.x[(int64_t)m * p.ldx + st.res_x_offset + c]);
    const uint16_t bits = __hip_atomic_load(reinterpret_cast<const uint16_t*>(st.res) + (int64_t)m * st.ld_res + c,
                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return (float)__builtin_bit_cast(_Float16, bits);
}

// I/O wave, before the stage: per-channel scales and residual rows of this workgroup's
// outputs, the RMSNorm weights, the wait for stage s - 1, and the input rows.
template <bool SW, int MR>
__device__ __forceinline__ void c_io_input(const ChainParams& p, const ChainStage& st, int s, int b, int n_it,
                                           uint32_t e, uint8_t* smem, ChainSync* sy) {
    const int lane = threadIdx.x & 63, M = p.M;
    const int nch = n_it * 16;
    const int sc_up = p.ipw_max * 16;
    float* lsc = reinterpret_cast<float*>(smem + p.off_sc);
    float* lr = reinterpret_cast<float*>(smem + p.off_res);
    // 1. scales and (when their source is already complete) residual rows
    const bool small = nch <= 64;
    const bool res_early = st.res_kind == 1 || st.res_stage <= s - 2;
    const int ch = lane, ci = ch >> 4, cn = ch & 15;
    const bool own = small && ch < nch && cn < c_width(st, b, ci);
    const int cc = own ? c_first(st, b, ci) + cn : 0;
    float scg = 0.0f, scu = 0.0f, rv[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) rv[m] = 0.0f;
    if (own) {
        scg = st.wscale[cc];
        if constexpr (SW) scu = st.wscale[(st.N >> 1) + cc];
        if (st.res_kind && res_early) {
#pragma unroll
            for (int m = 0; m < MR; ++m)
                if (m < M) rv[m] = c_residual(p, st, m, cc);
        }
    }
    // 2. RMSNorm weights: direct copies into LDS, 1 KiB per instruction
    if (st.gamma) {
        const __amdgpu_buffer_rsrc_t r = c_rsrc(st.gamma, (int64_t)st.K * 4);
        const int chunks = (st.K * 4 + 1023) >> 10;
        for (int c = 0; c < chunks; ++c)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (chain_lds_ptr)(smem + p.off_g + c * 1024), 16, c * 1024 + lane * 16,
                                                     0, 0, 0);
    }
    // 3. wait for the previous stage
    if (s > 0) c_io_poll(p, s - 1, e);
    // 4. input rows: the chain input, or an earlier stage's output read device-coherently
    {
        const bool from_x = st.in == nullptr;
        const __half* in = from_x ? p.x + st.x_offset : st.in;
        const int64_t ld_in = from_x ? p.ldx : st.ld_in;
        const int chunks = (st.K * 2 + 1023) >> 10;
        for (int m = 0; m < M; ++m) {
            const __amdgpu_buffer_rsrc_t r = c_rsrc(in + (int64_t)m * ld_in, (int64_t)st.K * 2);
            uint8_t* dst = smem + p.off_x + m * p.xstride;
            if (from_x) {
                for (int c = 0; c < chunks; ++c)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (chain_lds_ptr)(dst + c * 1024), 16, c * 1024 + lane * 16, 0,
                                                             0, 0);
            } else {
                for (int c = 0; c < chunks; ++c)
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (chain_lds_ptr)(dst + c * 1024), 16, c * 1024 + lane * 16, 0,
                                                             0, kSc1);
            }
        }
    }
    if (own && st.res_kind && !res_early) {
#pragma unroll
        for (int m = 0; m < MR; ++m)
            if (m < M) rv[m] = c_residual(p, st, m, cc);
    }
    if (small) {
        if (ch < nch) {
            lsc[ch] = scg;
            if constexpr (SW) lsc[sc_up + ch] = scu;
            if (st.res_kind) {
#pragma unroll
                for (int m = 0; m < MR; ++m) lr[ch * MR + m] = rv[m];
            }
        }
    } else {
        // wide stages (more than 64 channels per workgroup): one pass per 64 channels
        for (int c2 = lane; c2 < nch; c2 += 64) {
            const int i = c2 >> 4, n = c2 & 15;
            if (n < c_width(st, b, i)) {
                const int c = c_first(st, b, i) + n;
                lsc[c2] = st.wscale[c];
                if constexpr (SW) lsc[sc_up + c2] = st.wscale[(st.N >> 1) + c];
                if (st.res_kind)
                    for (int m = 0; m < M; ++m) lr[c2 * MR + m] = c_residual(p, st, m, c);
            }
        }
    }
    wait_all_memory();  // the direct copies into LDS have landed
    if (lane == 0) __hip_atomic_store(&sy->io_mark, (uint32_t)(2 * s), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Sum of squares of a row of K fp16 values in LDS in the reference order (see
// lds_sumsq_neon16): one wave, result in lane 0.
__device__ __forceinline__ float c_sumsq_neon16(const __half* x, int K) {
    return lds_sumsq_neon16(reinterpret_cast<const _Float16*>(x), K);
}

__device__ __forceinline__ void c_unpack8(const uint4& raw, float v[8]) {
    const __half2* hv = reinterpret_cast<const __half2*>(&raw);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float2 f = __half22float2(hv[i]);
        v[2 * i] = f.x;
        v[2 * i + 1] = f.y;
    }
}

// RMSNorm (x * ns) * gamma of one group in place (src/model/cpu.rs:61-64).
__device__ __forceinline__ void c_norm8(float v[8], const float* lg, int g, float ns) {
    const float4 ga = *reinterpret_cast<const float4*>(lg + 8 * g);
    const float4 gb = *reinterpret_cast<const float4*>(lg + 8 * g + 4);
    const float gg[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (v[i] * ns) * gg[i];
}

__device__ __forceinline__ uint2 c_quant8(const float v[8], float im, bool fast, bool rne) {
    int q[8];
    if (fast && rne) {
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = quant_finite<true>(v[i], im);
    } else if (fast) {
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = quant_finite<false>(v[i], im);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = quant_one(v[i], im, rne);  // src/npu.rs:1107-1110
    }
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        w0 |= (uint32_t)(q[i] & 0xff) << (8 * i);
        w1 |= (uint32_t)(q[4 + i] & 0xff) << (8 * i);
    }
    return make_uint2(w0, w1);
}

// Helper waves: RMSNorm scale, per-token scale and the quantized rows of the stage
// input (raw fp16 rows in LDS at off_x) into lds_q.  Same arithmetic as the GEMV
// prologue.  h = helper thread index (0 .. 64 * helper waves - 1).
template <int MR>
__device__ __forceinline__ void c_prologue(const ChainParams& p, const ChainStage& st, uint8_t* smem, int astride,
                                           int h, ChainSync* sy, uint32_t& hk, float* s_inv, float* s_rows,
                                           float (*s_red)[ChainShape<MR>::kHelperWaves], int* s_bad) {
    constexpr int HW = ChainShape<MR>::kHelperWaves, HT = 64 * HW;
    const int hw = h >> 6, lane = h & 63;
    const int M = p.M, K = st.K, ng = K >> 3;
    const int xs = p.xstride >> 1;  // elements per LDS row
    const __half* lx = reinterpret_cast<const __half*>(smem + p.off_x);
    const float* lg = reinterpret_cast<const float*>(smem + p.off_g);
    uint8_t* lds_q = smem;
    const bool norm = st.gamma != nullptr;
    // 1. RMSNorm scale per row (helper wave m computes row m), reference summation order
    if (norm) {
        if (hw < M) {
            const __half* xrow = lx + hw * xs;
            float sum;
            if (st.flags & kFlagNormSeq)
                sum = lane == 0 ? lds_sumsq_seq(xrow, K) : 0.0f;  // src/ops/norm.rs:38
            else
                sum = c_sumsq_neon16(xrow, K);  // src/model/cpu.rs:14-35
            if (lane == 0) s_inv[hw] = 1.0f / __builtin_sqrtf(sum / (float)K + st.eps);
        }
        helper_sync<HW>(sy, hk);
    }
    float nsc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) nsc[m] = (norm && m < M) ? s_inv[m] : 1.0f;
    // 2. absmax (after the norm) and finiteness, per row
    float mx[MR];
    int bad = 0;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        mx[m] = 0.0f;
        if (m < M) {
            for (int g = h; g < ng; g += HT) {
                float v[8];
                c_unpack8(*reinterpret_cast<const uint4*>(lx + m * xs + 8 * g), v);
#pragma unroll
                for (int i = 0; i < 8; ++i) bad |= !__builtin_isfinite(v[i]);
                if (norm) c_norm8(v, lg, g, nsc[m]);
#pragma unroll
                for (int i = 0; i < 8; ++i) mx[m] = fmaxf(mx[m], fabsf(v[i]));
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        const float w = wave_max_nonneg(mx[m]);
        if (lane == 0) s_red[m][hw] = w;
    }
    const bool any_bad = __ballot(bad) != 0;
    if (lane == 0) s_bad[hw] = any_bad;
    helper_sync<HW>(sy, hk);
    // 3. per-token scales from the wave maxima, in every helper wave: lane m * HW + w
    // reads s_red[m][w] and each row's lanes meet by DPP, so one read and one division
    // sequence serve all rows (read row by row in every lane, the 36-layer stack at 4
    // rows ran 1737 us against 1665 us; at 1 row both take 1152-1154 us)
    const int b = __ballot(lane < HW && s_bad[lane & (HW - 1)] != 0) != 0;
    const float am_l = rows_max_lanes<HW, MR>(&s_red[0][0]);
    const float sc_l = qscale_from_absmax(am_l);  // src/npu.rs:1101-1106
    const float inv_l = 1.0f / sc_l;
    float inv[MR];
    bool finite = true;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        const float sc = lane_value(sc_l, m * HW);
        finite &= __builtin_isfinite(sc);
        inv[m] = lane_value(inv_l, m * HW);
        if (h == 0 && m < M) s_rows[m] = sc;
    }
    if (b && blockIdx.x == 0 && h == 0) atomicOr(p.err, 1u);
    // 4. quantize into LDS (k order for both widths); a finite row (the usual case)
    // takes the short rounding sequence
    const bool rne = (st.flags & kFlagRne) != 0;
    const bool fast = !b && finite;
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        if (m < M) {
            for (int g = h; g < ng; g += HT) {
                float v[8];
                c_unpack8(*reinterpret_cast<const uint4*>(lx + m * xs + 8 * g), v);
                if (norm) c_norm8(v, lg, g, nsc[m]);
                *reinterpret_cast<uint2*>(lds_q + m * astride + 8 * g) = c_quant8(v, inv[m], fast, rne);
            }
            // zeros in [K, Kp): a previous stage may have left a longer row here
            for (int k = K + h * 8; k < st.Kp; k += HT * 8)
                *reinterpret_cast<uint2*>(lds_q + m * astride + k) = make_uint2(0, 0);
        }
    }
    helper_sync<HW>(sy, hk);
}

// I/O wave, after the products: dequant / SiLU-gate / residual epilogue of this
// workgroup's outputs, fp16 device-coherent stores, then the completion flag.
template <int BITS, bool SW, int MR>
__device__ __forceinline__ void c_io_epilogue(const ChainParams& p, const ChainStage& st, int s, int b, int n_it,
                                              uint32_t e, uint8_t* smem, const float* s_rows) {
    const int lane = threadIdx.x & 63, M = p.M;
    int* accg = reinterpret_cast<int*>(smem + p.off_acc);
    int* accu = accg + p.ipw_max * 16 * MR;
    const float* lsc = reinterpret_cast<const float*>(smem + p.off_sc);
    const float* lr = reinterpret_cast<const float*>(smem + p.off_res);
    const int sc_up = p.ipw_max * 16;
    const bool last = s == p.n_stages - 1;
    uint16_t* out = reinterpret_cast<uint16_t*>(last ? p.y : st.out);
    const int64_t ld_out = last ? p.ldy : st.ld_out;
    for (int idx = lane; idx < n_it * 16 * MR; idx += 64) {
        const int ch = idx / MR, m = idx - ch * MR;
        const int i = ch >> 4, n = ch & 15;
        if (m < M && n < c_width(st, b, i)) {
            const int c = c_first(st, b, i) + n;
            const int vg = accg[idx];
            const int a_g = BITS == 4 ? (vg >> 4) : vg;  // exact: W4 sums carry a factor 16
            float o = ((float)a_g * s_rows[m]) * lsc[ch];  // src/npu.rs:1117
            if constexpr (SW) {
                const int vu = accu[idx];
                const int a_u = BITS == 4 ? (vu >> 4) : vu;
                const float up = ((float)a_u * s_rows[m]) * lsc[sc_up + ch];
                o = silu_gate(o, up);  // src/npu.rs:1202-1208
            } else if (st.res_kind) {
                // src/model/dense.rs:486-489: hidden + projected * residual_multiplier
                const float pr = o * st.rmult;
                o = lr[idx] + pr;
            }
            const _Float16 h = f16_of_f32(o);
            __hip_atomic_store(out + (int64_t)m * ld_out + c, __builtin_bit_cast(uint16_t, h), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
        accg[idx] = 0;
        if constexpr (SW) accu[idx] = 0;
    }
    if (!last) {
        wait_all_memory();  // this wave's coherent output stores have completed
        if (lane == 0)
            __hip_atomic_store(p.flags + (int64_t)s * kChainFlagStride + b, e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The helper waves' part of stage s.
template <int BITS, bool SW, int MR>
__device__ __forceinline__ void c_stage_helpers(const ChainParams& p, int s, uint32_t e, uint8_t* smem, ChainSync* sy,
                                                uint32_t& hk, float* s_inv, float* s_rows,
                                                float (*s_red)[ChainShape<MR>::kHelperWaves], int* s_bad) {
    const ChainStage st = c_desc(p, s);
    const int b = blockIdx.x;
    const int h = threadIdx.x - 64 * kCW;
    const bool io = h < 64;
    const int n_it = c_items(st, b);
    if (io) c_io_input<SW, MR>(p, st, s, b, n_it, e, smem, sy);
    helper_sync<ChainShape<MR>::kHelperWaves>(sy, hk);
    c_prologue<MR>(p, st, smem, p.kp_max + 16, h, sy, hk, s_inv, s_rows, s_red, s_bad);
    if (io) {
        if (h == 0) __hip_atomic_store(&sy->rows_ready, (uint32_t)(s + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        lds_wait_ge(&sy->done, (uint32_t)(kCW * (s + 1)));  // every compute wave has added its sums
        c_io_epilogue<BITS, SW, MR>(p, st, s, b, n_it, e, smem, s_rows);
    }
}

// A compute wave's part of stage s.  Its weight loads wait until the stage's input rows
// are in LDS: loads in flight during the exchange sit ahead of the exchange's own loads
// and stores in this CU's memory pipeline (issued right after the previous stage's
// products, or half of them then, the 36-layer stack ran 1.2x / 1.13x slower).  A share
// longer than the registers hold (e.g. a W8 SiLU-gate stage: K = 2560, N = 19456 is 120
// steps per CU) runs in rounds of NB / 2 steps, each loaded once the previous round's
// products are done.  The loads have one site in the code, so the weight registers have
// a single owner (a second site made the compiler spill them).
template <int MR, int NB>
__device__ __forceinline__ void c_stage_compute(const ChainParams& p, int s, v4i (&buf)[NB], uint8_t* smem,
                                                ChainSync* sy) {
    lds_wait_ge(&sy->io_mark, (uint32_t)(2 * s));  // the stage's input rows have landed
    const ChainStage st = c_desc(p, s);
    const int wave = c_wave(), b = blockIdx.x;
    const int astride = p.kp_max + 16;
    const int E = c_row_items(st, c_items(st, b)) * st.steps;
    int* accg = reinterpret_cast<int*>(smem + p.off_acc);
    int* accu = accg + p.ipw_max * 16 * MR;
    const int f0 = E * wave / kCW, f1 = E * (wave + 1) / kCW;
    for (int r0 = f0;;) {
        const int cnt = min(f1 - r0, NB / 2);
        c_load<0, NB / 2>(buf, st, b, r0, cnt);
        if (r0 == f0) lds_wait_ge(&sy->rows_ready, (uint32_t)(s + 1));
        c_compute<MR>(buf, st, b, r0, cnt, smem, astride, p.M, accg, accu);
        r0 += cnt;
        if (r0 >= f1) break;
    }
    wait_lds();  // the sums are in LDS before this wave counts itself done
    if ((threadIdx.x & 63) == 0) atomicAdd(&sy->done, 1u);
}

template <int MR>
__global__ __launch_bounds__(ChainShape<MR>::kThreads) void chain_kernel(ChainParams p) {
    constexpr int kCT = ChainShape<MR>::kThreads, kNB = ChainShape<MR>::kBufRegs;
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float s_inv[4], s_rows[4];
    __shared__ float s_red[4][ChainShape<MR>::kHelperWaves];  // [row][helper wave] maxima
    __shared__ int s_bad[ChainShape<MR>::kHelperWaves];
    __shared__ ChainSync sy;
    const int tid = threadIdx.x, b = blockIdx.x;
    const int astride = p.kp_max + 16;
    // zero rows of the quantized activations (row M is the MFMA's zero row) and the sums
    for (int i = tid * 16; i < (MR + 1) * astride; i += kCT * 16)
        *reinterpret_cast<uint4*>(smem + i) = make_uint4(0, 0, 0, 0);
    for (int i = tid; i < 2 * p.ipw_max * 16 * MR; i += kCT) reinterpret_cast<int*>(smem + p.off_acc)[i] = 0;
    if (tid == 0) {
        sy.rows_ready = 0;
        sy.done = 0;
        sy.helpers = 0;
        sy.io_mark = 0;
    }
    __syncthreads();  // the only workgroup barrier
    if (tid < 64 * kCW) {
        v4i buf[kNB];
        for (int s = 0; s < p.n_stages; ++s) {
            c_stage_compute<MR, kNB>(p, s, buf, smem, &sy);
        }
    } else {
        // the helpers' instructions (the exchange between stages) issue ahead of the
        // compute waves' weight loads
        __builtin_amdgcn_s_setprio(2);
        const bool io = tid < 64 * (kCW + 1);
        uint32_t e = 0, hk = 0;
        if (io) e = __hip_atomic_load(p.epochs + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
        for (int s = 0; s < p.n_stages; ++s) {
            const ChainStage st = c_desc(p, s);
            const bool sw = (st.flags & kFlagSwiglu) != 0;
            if (st.bits == 4) {
                if (sw)
                    c_stage_helpers<4, true, MR>(p, s, e, smem, &sy, hk, s_inv, s_rows, s_red, s_bad);
                else
                    c_stage_helpers<4, false, MR>(p, s, e, smem, &sy, hk, s_inv, s_rows, s_red, s_bad);
            } else {
                if (sw)
                    c_stage_helpers<8, true, MR>(p, s, e, smem, &sy, hk, s_inv, s_rows, s_red, s_bad);
                else
                    c_stage_helpers<8, false, MR>(p, s, e, smem, &sy, hk, s_inv, s_rows, s_red, s_bad);
            }
        }
        if (io && (tid & 63) == 0) __hip_atomic_store(p.epochs + b, e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

size_t chain_lds_layout(int max_rows, int kp_max, int k_max, int kg_max, int ipw_max, ChainParams* p) {
    const int mr = max_rows <= 1 ? 1 : 4;
    size_t off = align_up((size_t)(mr + 1) * (kp_max + 16), 16);
    p->xstride = (int)align_up((size_t)k_max * 2, 1024);
    p->off_x = (int)off;
    off += (size_t)mr * p->xstride;
    p->off_g = (int)off;
    off += align_up((size_t)kg_max * 4, 1024);
    p->off_acc = (int)off;
    off += (size_t)2 * ipw_max * 16 * mr * 4;
    p->off_sc = (int)off;
    off += (size_t)2 * ipw_max * 16 * 4;
    p->off_res = (int)off;
    off += (size_t)ipw_max * 16 * mr * 4;
    p->ipw_max = ipw_max;
    return off;
}

int chain_resident_per_cu(int max_rows, size_t lds) {
    int n = 0;
    const void* f = max_rows <= 1 ? reinterpret_cast<const void*>(&chain_kernel<1>)
                                  : reinterpret_cast<const void*>(&chain_kernel<4>);
    if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, kChainMaxLds) != hipSuccess) return 0;
    const int threads = max_rows <= 1 ? ChainShape<1>::kThreads : ChainShape<4>::kThreads;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, threads, lds) != hipSuccess) return 0;
    return n;
}

hipError_t launch_chain(const ChainParams& p, int grid, size_t lds, hipStream_t stream) {
    if (p.M <= 1) {
        static const hipError_t a1 = hipFuncSetAttribute(reinterpret_cast<const void*>(&chain_kernel<1>),
                                                         hipFuncAttributeMaxDynamicSharedMemorySize, kChainMaxLds);
        if (a1 != hipSuccess) return a1;
        chain_kernel<1><<<grid, ChainShape<1>::kThreads, lds, stream>>>(p);
    } else {
        static const hipError_t a4 = hipFuncSetAttribute(reinterpret_cast<const void*>(&chain_kernel<4>),
                                                         hipFuncAttributeMaxDynamicSharedMemorySize, kChainMaxLds);
        if (a4 != hipSuccess) return a4;
        chain_kernel<4><<<grid, ChainShape<4>::kThreads, lds, stream>>>(p);
    }
    return hipGetLastError();
}

}  // namespace qlin
