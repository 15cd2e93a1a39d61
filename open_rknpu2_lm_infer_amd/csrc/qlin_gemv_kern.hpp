// Decode GEMV kernels (gemv_kernel, gemv_items_kernel) and their launch templates,
// shared by the translation units that instantiate them: qlin_gemv_1row.hip holds the
// one-row instances and qlin_gemv.hip the multi-row ones and the dispatcher.
#pragma once

// Kernel (b) + (d): decode GEMV for 1..16 rows with the dequant / SiLU-gate epilogue.
//
// Replaces the native library's per-call scan/quantize, NPU int4 GEMM and CPU
// reduce/dequant for small M (QWEN3_W4A8_PIPELINE_REVIEW_20261020.md:24-31).
//
// Mapping.  One workgroup of WAVES waves owns a group of 16 output channels (plus the
// matching 16 "up" channels N/2 + j for SwiGLU) over the whole K; wave w takes wave
// steps w, w + WAVES, ...  Partial sums meet once, in LDS, at the end: no split-K,
// no atomics, no counters.  WAVES (4, 8 or 16) is picked per shape so that even
// N = 2560 puts a few thousand waves in flight.
//
// Streaming.  One wave step covers 16 weight rows x 128 bytes (a full 128-byte line
// per row): lane l loads 16 bytes of row l%16 at byte 16*(l/16) and 64 + 16*(l/16).
// For W8 those bytes are the B operand of v_mfma_i32_16x16x64_i8 directly; for W4
// each 16 bytes unpack in registers into two B operands.  The unpack keeps the
// nibble in the high half of each byte (w & 0xF0, w << 4 & 0xF0), i.e. 16*code as
// an exact int8, so the int32 sum is 16x the true one and is shifted back (exact)
// before dequant.  The device order of W4 codes (byte b of each word holds codes b
// and b + 4) makes the unpacked bytes come out in natural k order, so activation
// bytes are used as they are for both widths.  Rows beyond M feed zeros to the
// matrix core.
//
// Ordering.  Memory counters retire in issue order, so every activation load is
// issued before the first weight load; waiting for the activations then never
// waits for the weight stream, which is consumed only after the prologue.
//
// Activations.  FUSED (M <= 4): every workgroup loads the raw rows into registers,
// derives the per-token scale (and the RMSNorm scale) itself and quantizes into LDS;
// max is order independent, so every workgroup gets the same s and q bit for bit.
// Otherwise q and s come from the quantize kernel and each lane loads its A operand
// straight from L2.
#include <type_traits>

#include "qlin_gemv_parts.hpp"
#include "qlin_rows.hpp"

namespace qlin {

constexpr int kGemvRsrcFlags = 0x00020000;  // raw buffer, 32-bit data format (gfx9 word 3)

// Register budget per wave count (1024-thread workgroups get 128 VGPRs per lane):
// wave steps in flight per register buffer, and 8-element activation groups held
// per thread by the fused prologue.  With RMSNorm a thread also holds 8 gamma values per
// group: 2 slots at 16 waves and 4 below (the f32 rows of the RMSNorm fit 64 KiB of LDS,
// K <= 16384, i.e. at most 4 groups per thread at 512 threads), which keeps those
// kernels from spilling.
template <int WAVES, bool FUSED>
struct GemvCfg {
    static constexpr int BATCH = FUSED ? (WAVES >= 8 ? 2 : 4) : (WAVES >= 16 ? 1 : 2);
    static constexpr int XREGS = WAVES >= 16 ? 4 : 8;
    static constexpr int XREGS_NORM = WAVES >= 16 ? 2 : 4;
};
constexpr int fused_regs(int waves, bool norm) { return waves >= 16 ? (norm ? 2 : 4) : (norm ? 4 : 8); }
// Instances for one (or two) activation groups per thread per row, known at compile time:
// slot i holds group i % gpt of row i / gpt, so the slots' rows and groups are constants in
// the unrolled prologue loops.  One group: every shape but the longest rows; two: the down
// projection (K = 9728) at 16 waves.
constexpr int kOneGroupRegs = -1;
constexpr int kTwoGroupRegs = -2;
// Several rows without RMSNorm in 1024-thread workgroups may hold up to this many groups
// per thread, in instances of their own (rows of 3-4 groups per thread at 2 rows; the
// down projection, K = 9728, two groups per row, takes the two-group instances above);
// the 4-slot instances stay for the shorter rows, which ran slower with 8 slots (o at 2
// rows 5.01 -> 5.46 us).
constexpr int kWideRowsRegs = 8;
// Several rows with RMSNorm: fewer slots keep the prologue (gamma, the normalized values
// between its two passes) within the register file.
constexpr int kNormRowsRegs = 4;

// LDS of gemv_items_kernel: the quantized rows (and the f32 rows of the RMSNorm before
// them), then the partial-sum area [items][gate, up][WAVES][lanes][regs].
__host__ __device__ __forceinline__ size_t gemv_red_offset(int M, int Kp, int K, bool fused, bool norm) {
    size_t a = fused ? (size_t)(M + 1) * (Kp + 16) : 0;
    if (norm) a = a > (size_t)M * K * sizeof(float) ? a : (size_t)M * K * sizeof(float);
    return (a + 15) & ~(size_t)15;
}

template <int BITS>
__device__ __forceinline__ void a_from_global(v4i a[4], const int8_t* qrow, bool live) {
    const v4i zero = {0, 0, 0, 0};
    if constexpr (BITS == 8) {
        a[0] = live ? ld16(qrow) : zero;
        a[1] = live ? ld16(qrow + 64) : zero;
    } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            a[2 * j] = live ? ld16(qrow + 128 * j) : zero;           // k 0..15 of the lane's 32
            a[2 * j + 1] = live ? ld16(qrow + 128 * j + 16) : zero;  // k 16..31
        }
    }
}

// Registers of BATCH wave steps: weights (gate, up) and, when the rows arrive
// quantized, the matching A operands.
template <int BATCH, bool FUSED, int RB = 1>
struct StepBuf {
    v4i bg[BATCH][2], bu[BATCH][2];
    v4i a[FUSED ? 1 : BATCH][4];
    v4i a2[!FUSED && RB > 1 ? BATCH : 1][4];  // rows 16..31 (two row blocks of quantized rows)
};

// Issues the loads of one batch with no branches: steps past the end re-read the
// last step (an L2 hit), so the compiler can count outstanding loads exactly and
// never has to wait for more than it consumes.  In the quantized mode the A loads
// of a step are issued before its weights.
template <int BITS, bool SWIGLU, bool FUSED, int WAVES, int BATCH>
__device__ __forceinline__ void load_batch(StepBuf<BATCH, FUSED>& s, const uint8_t* wg, const uint8_t* wu,
                                           const int8_t* qrow, bool live, int base, int steps) {
    constexpr int KS = BITS == 4 ? 256 : 128;
#pragma unroll
    for (int i = 0; i < BATCH; ++i) {
        const int st = min(base + WAVES * i, steps - 1);
        if constexpr (!FUSED) a_from_global<BITS>(s.a[i], qrow + st * KS, live);
        s.bg[i][0] = ld16(wg + (int64_t)st * 128);
        s.bg[i][1] = ld16(wg + (int64_t)st * 128 + 64);
        if constexpr (SWIGLU) {
            s.bu[i][0] = ld16(wu + (int64_t)st * 128);
            s.bu[i][1] = ld16(wu + (int64_t)st * 128 + 64);
        }
    }
}

template <int BITS, bool SWIGLU, bool FUSED, int WAVES, int BATCH>
__device__ __forceinline__ void compute_batch(v4i& ag, v4i& au, const StepBuf<BATCH, FUSED>& s,
                                              const uint8_t* arow, int base, int steps) {
    constexpr int KS = BITS == 4 ? 256 : 128;
#pragma unroll
    for (int i = 0; i < BATCH; ++i) {
        const int st = base + WAVES * i;
        if (st < steps) {
            v4i a[4];
            if constexpr (FUSED) {
                a_from_lds<BITS>(a, arow + st * KS);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) a[j] = s.a[i][j];
            }
            mfma_step<BITS>(ag, s.bg[i], a);
            if constexpr (SWIGLU) mfma_step<BITS>(au, s.bu[i], a);
        }
    }
}

// Position in a wave's flat sequence of K steps: item j of the workgroup, step t.
// The sequence is the workgroup's flat step indices f = j * steps + t that are
// congruent to the wave index mod WAVES, in increasing order.
struct GemvPos {
    int j, t;
    __device__ __forceinline__ void advance(int waves, int steps) {
        t += waves;
        while (t >= steps) {
            t -= steps;
            ++j;
        }
    }
};

// Issues the loads of BATCH positions with no branches: positions past the end
// re-read the last one (an L2 hit), so the compiler can count outstanding loads
// exactly and never has to wait for more than it consumes.  In the quantized mode
// the A loads of a position are issued before its weights.
template <int BITS, bool SWIGLU, bool FUSED, int WAVES, int BATCH, int RB = 1>
__device__ __forceinline__ void load_batch_items(StepBuf<BATCH, FUSED, RB>& s, const GemvParams& p, GemvPos& pos, int& c,
                                           int total, GemvPos last, const uint8_t* wlane, int64_t up_off,
                                           const int8_t* qrow, bool live, int steps, int lrow, int ncols,
                                           const int8_t* qrow2 = nullptr, bool live2 = false) {
    constexpr int KS = BITS == 4 ? 256 : 128;
#pragma unroll
    for (int i = 0; i < BATCH; ++i) {
        const GemvPos q = c < total ? pos : last;
        // weight row of this lane: row lrow of the item, the last real row past the end
        const int row = min(p.iw * ((int)blockIdx.x + q.j * (int)gridDim.x) + lrow, ncols - 1);
        const uint8_t* wg = wlane + (int64_t)row * p.wrow + (int64_t)q.t * 128;
        if constexpr (!FUSED) a_from_global<BITS>(s.a[i], qrow + q.t * KS, live);
        if constexpr (!FUSED && RB > 1) a_from_global<BITS>(s.a2[i], qrow2 + q.t * KS, live2);
        s.bg[i][0] = ld16(wg);
        s.bg[i][1] = ld16(wg + 64);
        if constexpr (SWIGLU) {
            s.bu[i][0] = ld16(wg + up_off);
            s.bu[i][1] = ld16(wg + up_off + 64);
        }
        if (c < total) {
            pos.advance(WAVES, steps);
            ++c;
        }
    }
}

// Partial sums of the wave's current item to LDS (red[item][gate, up][wave]).
template <bool SWIGLU, int WAVES, int LIVE, int REGS>
__device__ __forceinline__ void gemv_flush(int* red, int j, int wave, int lane, v4i& ag, v4i& au) {
    if (lane < LIVE) {
#pragma unroll
        for (int i = 0; i < REGS; ++i) {
            red[(((j * 2) * WAVES + wave) * LIVE + lane) * REGS + i] = ag[i];
            if constexpr (SWIGLU) red[(((j * 2 + 1) * WAVES + wave) * LIVE + lane) * REGS + i] = au[i];
        }
    }
    ag = v4i{0, 0, 0, 0};
    au = v4i{0, 0, 0, 0};
}

// MFMAs of BATCH positions; cj is the item whose sums ag / au hold.  Moving to a later
// item flushes them (and zero sums for items this wave has no step of).
template <int BITS, bool SWIGLU, bool FUSED, int WAVES, int BATCH, int LIVE, int REGS, int RB = 1>
__device__ __forceinline__ void compute_batch_items(v4i& ag, v4i& au, const StepBuf<BATCH, FUSED, RB>& s, const uint8_t* arow,
                                              GemvPos& pos, int& c, int total, int& cj, int* red, int wave, int lane,
                                              int steps, v4i* ag2 = nullptr, v4i* au2 = nullptr) {
    constexpr int KS = BITS == 4 ? 256 : 128;
#pragma unroll
    for (int i = 0; i < BATCH; ++i) {
        if (c < total) {
            if constexpr (RB > 1) {
                // item j's row blocks take the sum slots 2j and 2j + 1
                while (cj < pos.j) {
                    gemv_flush<SWIGLU, WAVES, LIVE, REGS>(red, 2 * cj, wave, lane, ag, au);
                    gemv_flush<SWIGLU, WAVES, LIVE, REGS>(red, 2 * cj + 1, wave, lane, *ag2, *au2);
                    ++cj;
                }
            } else {
                while (cj < pos.j) gemv_flush<SWIGLU, WAVES, LIVE, REGS>(red, cj++, wave, lane, ag, au);
            }
            v4i a[4];
            if constexpr (FUSED) {
                a_from_lds<BITS>(a, arow + pos.t * KS);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) a[j] = s.a[i][j];
            }
            mfma_step<BITS>(ag, s.bg[i], a);
            if constexpr (SWIGLU) mfma_step<BITS>(au, s.bu[i], a);
            if constexpr (!FUSED && RB > 1) {
                v4i a2[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) a2[j] = s.a2[i][j];
                mfma_step<BITS>(*ag2, s.bg[i], a2);
                if constexpr (SWIGLU) mfma_step<BITS>(*au2, s.bu[i], a2);
            }
            pos.advance(WAVES, steps);
            ++c;
        }
    }
}

template <int BITS, bool SWIGLU>
__device__ __forceinline__ void gemv_store(const GemvParams& p, int m, int n, int r0, int vg, int vu, float sm,
                                           float wsg, float wsu) {
    const int Nh = p.N >> 1;
    const int ag = BITS == 4 ? (vg >> 4) : vg;  // exact: W4 sums carry a factor 16
    const int cg = r0 + n;
    if (p.c_kind == 2) {
        if (cg < p.N) reinterpret_cast<int32_t*>(p.C)[(int64_t)m * p.ldc + cg] = ag;
        return;
    }
    float out = ((float)ag * sm) * wsg;  // src/npu.rs:1117 (wsg = wscale[cg])
    if constexpr (SWIGLU) {
        const int au = BITS == 4 ? (vu >> 4) : vu;
        const float up = ((float)au * sm) * wsu;  // wsu = wscale[N/2 + cg]
        out = silu_gate(out, up);  // src/npu.rs:1202-1208
    }
    if (cg < (SWIGLU ? Nh : p.N)) {
        if (!SWIGLU && p.R) out = residual_add(p.R, p.ldr, p.r_f16, p.rmult, m, cg, out);  // src/model/dense.rs:486-489
        if (p.c_kind == 1)
            reinterpret_cast<_Float16*>(p.C)[(int64_t)m * p.ldc + cg] = f16_of_f32(out);
        else
            reinterpret_cast<float*>(p.C)[(int64_t)m * p.ldc + cg] = out;
    }
}

// Raw activation group of 8 values held in registers until quantization.
template <typename T>
struct XGroup;
template <>
struct XGroup<__half> {
    uint4 raw;
    __device__ __forceinline__ void load(const __half* p) { raw = *reinterpret_cast<const uint4*>(p); }
    __device__ __forceinline__ void get(float v[8]) const {
        const __half2* h = reinterpret_cast<const __half2*>(&raw);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float2 f = __half22float2(h[i]);
            v[2 * i] = f.x;
            v[2 * i + 1] = f.y;
        }
    }
};
template <>
struct XGroup<float> {
    float4 a, b;
    __device__ __forceinline__ void load(const float* p) {
        a = *reinterpret_cast<const float4*>(p);
        b = *reinterpret_cast<const float4*>(p + 4);
    }
    __device__ __forceinline__ void get(float v[8]) const {
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
};

// Register slot i of the fused prologue holds this thread's group j of row m, with
// i = m * gpt + j (gpt groups per thread per row).  The (m, j) of every slot come from a
// running count, wave-uniform values in scalar registers: i / gpt, with gpt known only
// at run time, cost an integer division sequence per slot in every loop over the slots.
template <int XR>
struct GemvSlots {
    int m[XR], j[XR];
    __device__ __forceinline__ explicit GemvSlots(int gpt) {
        int m0 = 0, j0 = 0;
#pragma unroll
        for (int i = 0; i < XR; ++i) {
            m[i] = m0;
            j[i] = j0;
            if (++j0 == gpt) {
                j0 = 0;
                ++m0;
            }
        }
    }
};

// The value of v[m] for a wave-uniform row index m < MR.  A chain of selects from a
// constant keeps the registers statically indexed (starting from v[0] the compiler
// turned the chain into an indexed load and moved v to scratch memory).
template <int MR>
__device__ __forceinline__ float row_pick(const float (&v)[MR], int m) {
    float r = 1.0f;
#pragma unroll
    for (int mm = 0; mm < MR; ++mm)
        if (mm == m) r = v[mm];
    return r;
}

// Activation groups of this thread into registers (and with RMSNorm the gamma values of
// each held group).  Only owned groups are loaded.  These loads may sit in branches
// because every weight load after them is unconditional: waits for them then count
// exactly the weight loads issued later.
template <int MR, int XR, int NT, bool NORM, typename T>
__device__ __forceinline__ void gemv_load_rows(const GemvParams& p, XGroup<T> (&xr)[XR], float (&gr)[NORM ? XR : 1][8],
                                               const GemvSlots<XR>& sl, int nreg, int ngroups) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < XR; ++i) {
        if (i < nreg) {
            const int g = tid + NT * sl.j[i];
            if (g < ngroups) xr[i].load(reinterpret_cast<const T*>(p.A) + (int64_t)sl.m[i] * p.lda + 8 * g);
        }
    }
    if constexpr (NORM) {
        // Rows share gamma: gr[j] holds the gamma values of this thread's group j, loaded by
        // row 0's slot j, and every row's slot takes them from there where it is used
        // (gemv_slot_gamma).  With at least two rows a thread holds at most XR / 2 groups.
        // Loading gamma for every slot issued the same bytes once per row (4 rows: a
        // quarter of the prologue's load issue time).  The loads are buffer loads with no
        // branch: a slot past the row reads beyond the buffer's range, which returns zeros
        // without a memory access.  (Loaded in branches, the registers were zeroed first
        // and moved after the loads, which made every wave wait for them before it issued
        // its first weights.)
        const __amdgpu_buffer_rsrc_t rg =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.gamma), (short)0, p.K * 4, kGemvRsrcFlags);
#pragma unroll
        for (int j = 0; j < (XR > 1 ? XR / 2 : 1); ++j) {
            const int g = tid + NT * j;
            const int off = sl.m[j] == 0 && g < ngroups ? 32 * g : p.K * 4;
            const float4 a = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rg, off, 0, 0));
            const float4 b = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rg, off + 16, 0, 0));
            gr[j][0] = a.x; gr[j][1] = a.y; gr[j][2] = a.z; gr[j][3] = a.w;
            gr[j][4] = b.x; gr[j][5] = b.y; gr[j][6] = b.z; gr[j][7] = b.w;
        }
    }
}

// The gamma values of slot i: gr[j[i]], j[i] < XR / 2 (a uniform choice among static
// registers).
template <int XR>
__device__ __forceinline__ void gemv_slot_gamma(const float (&gr)[XR][8], const GemvSlots<XR>& sl, int i,
                                                float (&gv)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) gv[e] = gr[0][e];
#pragma unroll
    for (int jj = 1; jj < XR / 2; ++jj)
        if (sl.j[i] == jj) {
#pragma unroll
            for (int e = 0; e < 8; ++e) gv[e] = gr[jj][e];
        }
}

// Per-token scales from the wave maxima s_red[m][w] and the wave flags s_bad[w]: lane
// m * WAVES + w reads s_red[m][w], the WAVES lanes of a row take their max by DPP, and
// every lane computes its row's scale and reciprocal, so one LDS read and one division
// sequence serve all rows (read row by row, 4 rows of 16 maxima took 64 words and four
// division pairs in every wave).  Wave 0 writes s_rows.  Returns whether any wave saw a
// value that is not finite.  The whole wave must be active.
template <int WAVES, int MR>
__device__ __forceinline__ bool gemv_row_scales(const float (*s_red)[WAVES], const int* s_bad, int M, float (&inv)[MR],
                                                float* s_rows) {
    const int lane = threadIdx.x & 63;
    const int bad = lane < WAVES ? s_bad[lane] : 0;
    const float am = rows_max_lanes<WAVES, MR>(&s_red[0][0]);
    const float sc = qscale_from_absmax(am);  // src/npu.rs:1101-1106
    const float iv = 1.0f / sc;
#pragma unroll
    for (int m = 0; m < MR; ++m) inv[m] = lane_value(iv, m * WAVES);
    const int row = lane / WAVES;
    if (threadIdx.x < 64 && lane == row * WAVES && row < M && row < MR) s_rows[row] = sc;
    return __ballot(bad) != 0;
}

// Quantized rows of the fused prologue into LDS for finite rows (quant_finite).
template <int BITS, bool NORM, bool RNE, int MR, int XR, typename XG>
__device__ __forceinline__ void gemv_quant_rows(const XG (&xr)[XR], const float (&gr)[NORM ? XR : 1][8],
                                                const float (&nsc)[MR], const float (&inv)[MR], uint8_t* lds_a,
                                                int astride, const GemvSlots<XR>& sl, int nreg, int ngroups, int tid,
                                                int NT) {
#pragma unroll
    for (int i = 0; i < XR; ++i) {
        if (i < nreg) {
            const int m = sl.m[i], g = tid + NT * sl.j[i];
            if (g < ngroups) {
                float v[8];
                xr[i].get(v);
                if constexpr (NORM) {
                    const float ns = row_pick(nsc, m);
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[e] = (v[e] * ns) * gr[i][e];
                }
                const float im = row_pick(inv, m);
                int q[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) q[e] = quant_finite<RNE>(v[e], im);  // src/npu.rs:1107-1110
                uint32_t w0 = 0, w1 = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    w0 |= (uint32_t)(q[e] & 0xff) << (8 * e);
                    w1 |= (uint32_t)(q[4 + e] & 0xff) << (8 * e);
                }
                *reinterpret_cast<uint2*>(lds_a + m * astride + 8 * g) = make_uint2(w0, w1);
            }
        }
    }
}

// Quantized rows into LDS from values already in registers (the normalized values of the
// RMSNorm prologue): FAST takes quant_finite (finite rows), else quant_one with rne.
template <bool RNE, bool FAST, int MR, int XR>
__device__ __forceinline__ void gemv_quant_vals(const float (&vn)[XR][8], const float (&inv)[MR], uint8_t* lds_a,
                                                int astride, const GemvSlots<XR>& sl, int nreg, int ngroups, int tid,
                                                int NT, bool rne = RNE) {
#pragma unroll
    for (int i = 0; i < XR; ++i) {
        if (i < nreg) {
            const int m = sl.m[i], g = tid + NT * sl.j[i];
            if (g < ngroups) {
                const float im = row_pick(inv, m);
                int q[8];
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    q[e] = FAST ? quant_finite<RNE>(vn[i][e], im) : quant_one(vn[i][e], im, rne);  // src/npu.rs:1107-1110
                uint32_t w0 = 0, w1 = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    w0 |= (uint32_t)(q[e] & 0xff) << (8 * e);
                    w1 |= (uint32_t)(q[4 + e] & 0xff) << (8 * e);
                }
                *reinterpret_cast<uint2*>(lds_a + m * astride + 8 * g) = make_uint2(w0, w1);
            }
        }
    }
}

// The fused prologue: (RMSNorm scale,) per-token scale and quantized rows in LDS.  LDS
// rows 0..M-1 hold the quantized activations; row M is all zeros and feeds the
// matrix-core rows M..15.  The caller's barrier after it publishes the rows.
template <int BITS, int MODE, bool NORM, int WAVES, int MR, int XR, typename T>
__device__ __forceinline__ void gemv_fused_prologue(const GemvParams& p, const XGroup<T> (&xr)[XR],
                                                    const float (&gr)[NORM ? XR : 1][8], const GemvSlots<XR>& sl,
                                                    int nreg, int ngroups, uint8_t* smem, int astride, float* s_inv,
                                                    float (*s_red)[WAVES], int* s_bad, float* s_rows) {
    constexpr int NT = 64 * WAVES;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    uint8_t* lds_a = smem;
    const bool rne = (p.flags & kFlagRne) != 0;
    float nsc[MR];  // RMSNorm scale per row
#pragma unroll
    for (int m = 0; m < MR; ++m) nsc[m] = 1.0f;
    if constexpr (NORM) {
        // the reference summation order needs each whole row in one place: f32 rows
        // [M][K] in LDS, one wave per row
        float* lds_x = reinterpret_cast<float*>(smem);
#pragma unroll
        for (int i = 0; i < XR; ++i) {
            const int m = MR == 1 ? 0 : sl.m[i], g = tid + NT * sl.j[i];
            if (i < nreg && g < ngroups) {
                float v[8];
                xr[i].get(v);
#pragma unroll
                for (int e = 0; e < 8; ++e) lds_x[m * p.K + 8 * g + e] = v[e];
            }
        }
        lds_barrier();
        if (wave < p.M) {
            const float* xm = lds_x + wave * p.K;
            const float sum = (p.flags & kFlagNormSeq) != 0 ? (lane == 0 ? lds_sumsq_seq(xm, p.K) : 0.0f)  // src/ops/norm.rs:38
                                                            : lds_sumsq_neon16(xm, p.K);  // src/model/cpu.rs:14-35
            if (lane == 0) s_inv[wave] = 1.0f / __builtin_sqrtf(sum / (float)p.K + p.eps);
        }
        lds_barrier();
#pragma unroll
        for (int m = 0; m < MR; ++m) nsc[m] = m < p.M ? s_inv[m] : 1.0f;
        lds_barrier();  // lds_x is overwritten by the quantized rows below
    }
    const bool owner_wave = wave * 64 < ngroups;  // waves holding activation groups (uniform)
    float vn[NORM ? XR : 1][8];  // RMSNorm: the normalized values, from the absmax pass to the quantize pass
    if (owner_wave) {
        float mx[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) mx[m] = 0.0f;
        int bad = 0;
#pragma unroll
        for (int i = 0; i < XR; ++i) {
            if (i < nreg) {
                const int m = sl.m[i], g = tid + NT * sl.j[i];  // m is uniform
                if (g < ngroups) {
                    float lm;
                    if constexpr (MODE == 1 && !NORM) {
                        // fp16 rows: absmax and finiteness from the bit patterns
                        const uint4 r = xr[i].raw;
                        const uint32_t mb = absmax_bits_f16x8(r.x, r.y, r.z, r.w);
                        bad |= mb > 0x7bffu;
                        lm = f32_of_f16_bits(mb > 0x7bffu ? 0u : mb);  // Inf / NaN: folded again below
                    } else {
                        float v[8];
                        xr[i].get(v);
#pragma unroll
                        for (int e = 0; e < 8; ++e) bad |= !__builtin_isfinite(v[e]);
                        if constexpr (NORM) {
                            const float ns = row_pick(nsc, m);
                            float gv[8];
                            gemv_slot_gamma(gr, sl, i, gv);
#pragma unroll
                            for (int e = 0; e < 8; ++e) {
                                v[e] = (v[e] * ns) * gv[e];
                                vn[i][e] = v[e];
                            }
                        }
                        lm = 0.0f;
#pragma unroll
                        for (int e = 0; e < 8; ++e) lm = fmaxf(lm, fabsf(v[e]));
                        bad |= !__builtin_isfinite(lm);  // the normalized values must stay finite too
                    }
#pragma unroll
                    for (int mm = 0; mm < MR; ++mm)
                        if (mm == m) mx[mm] = fmaxf(mx[mm], lm);
                }
            }
        }
        if constexpr (MODE == 1 && !NORM) {
            // A group holding Inf or NaN (rare) was left out of the maxima above: fold them
            // again as the reference does.  Wave-uniform: with several rows per thread the
            // branch-free fold of the one-row kernels costs more VALU in every launch.
            if (__builtin_expect(__ballot(bad) != 0, 0)) {
#pragma unroll
                for (int m = 0; m < MR; ++m) mx[m] = 0.0f;
#pragma unroll
                for (int i = 0; i < XR; ++i) {
                    const int m = sl.m[i], g = tid + NT * sl.j[i];
                    if (i < nreg && g < ngroups) {
                        bool nonfinite;
                        const float lm = f32_of_f16_bits(absmax_bits_f16x8_ref(xr[i].raw, nonfinite));
#pragma unroll
                        for (int mm = 0; mm < MR; ++mm)
                            if (mm == m) mx[mm] = fmaxf(mx[mm], lm);
                    }
                }
            }
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const float w = m < p.M ? wave_max_nonneg(mx[m]) : 0.0f;
            if (lane == 0) s_red[m][wave] = w;
        }
        const bool any_bad = __ballot(bad) != 0;
        if (lane == 0) s_bad[wave] = any_bad;
    } else if (lane == 0) {
#pragma unroll
        for (int m = 0; m < MR; ++m) s_red[m][wave] = 0.0f;
        s_bad[wave] = 0;
    }
    lds_barrier();
    // Per-token scales, computed by the waves that hold activation groups (the others
    // go straight to the barrier instead of spending the SIMDs on scales they do not
    // use) from all WAVES wave maxima (zeros, the identity of a max of magnitudes, from
    // the waves that own no group).
    if (owner_wave) {
        float inv[MR];
        const bool bad_rows = gemv_row_scales<WAVES, MR>(s_red, s_bad, p.M, inv, s_rows);
        if (tid == 0 && bad_rows && p.err && blockIdx.x == 0) atomicOr(p.err, 1u);
        if constexpr (NORM) {
            // from the normalized values of the absmax pass
            if (!bad_rows) {
                if (rne)
                    gemv_quant_vals<true, true, MR>(vn, inv, lds_a, astride, sl, nreg, ngroups, tid, NT);
                else
                    gemv_quant_vals<false, true, MR>(vn, inv, lds_a, astride, sl, nreg, ngroups, tid, NT);
            } else {
                gemv_quant_vals<false, false, MR>(vn, inv, lds_a, astride, sl, nreg, ngroups, tid, NT, rne);
            }
        } else if (!bad_rows) {
            // no RMSNorm: finite rows (the usual case) take the short rounding sequence
            if (rne)
                gemv_quant_rows<BITS, NORM, true, MR>(xr, gr, nsc, inv, lds_a, astride, sl, nreg, ngroups, tid, NT);
            else
                gemv_quant_rows<BITS, NORM, false, MR>(xr, gr, nsc, inv, lds_a, astride, sl, nreg, ngroups, tid, NT);
        } else {
#pragma unroll
            for (int i = 0; i < XR; ++i) {
                if (i < nreg) {
                    const int m = sl.m[i], g = tid + NT * sl.j[i];
                    if (g < ngroups) {
                        float v[8];
                        xr[i].get(v);
                        const float im = row_pick(inv, m);
                        int q[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) q[e] = quant_one(v[e], im, rne);  // src/npu.rs:1107-1110
                        uint32_t w0 = 0, w1 = 0;
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            w0 |= (uint32_t)(q[e] & 0xff) << (8 * e);
                            w1 |= (uint32_t)(q[4 + e] & 0xff) << (8 * e);
                        }
                        *reinterpret_cast<uint2*>(lds_a + m * astride + 8 * g) = make_uint2(w0, w1);
                    }
                }
            }
        }
    }
    // zero the K..Kp tail of each row and the whole zero row M
    for (int m = 0; m < p.M; ++m)
        for (int k = p.K + tid * 8; k < p.Kp; k += NT * 8)
            *reinterpret_cast<uint2*>(lds_a + m * astride + k) = make_uint2(0, 0);
    for (int k = tid * 16; k < p.Kp; k += NT * 16)
        *reinterpret_cast<uint4*>(lds_a + p.M * astride + k) = make_uint4(0, 0, 0, 0);
}

// Quantized rows into LDS for finite rows (quant_finite), for the one-row prologue the
// kernels keep written out: slot i holds group i - (i / gpt) * gpt of row i / gpt.
template <int BITS, bool NORM, bool RNE, int MR, int XR, typename XG>
__device__ __forceinline__ void gemv_quant_rows_1(const XG (&xr)[XR], const float (&gr)[NORM ? XR : 1][8],
                                                const float (&nsc)[MR], const float (&inv)[MR], uint8_t* lds_a, int astride, int nreg, int gpt,
                                                int ngroups, int tid, int NT) {
#pragma unroll
    for (int i = 0; i < XR; ++i) {
        if (i < nreg) {
            const int m = i / gpt, g = tid + NT * (i - m * gpt);
            if (g < ngroups) {
                float v[8];
                xr[i].get(v);
                if constexpr (NORM) {
                    float ns = 1.0f;
#pragma unroll
                    for (int mm = 0; mm < MR; ++mm)
                        if (mm == m) ns = nsc[mm];
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[e] = (v[e] * ns) * gr[i][e];
                }
                float im = 1.0f;
#pragma unroll
                for (int mm = 0; mm < MR; ++mm)
                    if (mm == m) im = inv[mm];
                int q[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) q[e] = quant_finite<RNE>(v[e], im);  // src/npu.rs:1107-1110
                uint32_t w0 = 0, w1 = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    w0 |= (uint32_t)(q[e] & 0xff) << (8 * e);
                    w1 |= (uint32_t)(q[4 + e] & 0xff) << (8 * e);
                }
                *reinterpret_cast<uint2*>(lds_a + m * astride + 8 * g) = make_uint2(w0, w1);
            }
        }
    }
}

// Brings the parameters a workgroup's prologue needs into scalar registers at once.
// Left to itself the compiler fetches them field by field as the code reaches them, and
// reuses their registers, so the prologue waited on 4-5 kernel-argument loads in series
// before its first global load; an empty asm that reads them all makes it issue the loads
// together and wait once.
__device__ __forceinline__ void gemv_fetch_params(const GemvParams& p) {
    asm volatile("" ::"s"(p.W), "s"(p.wscale), "s"(p.wrow), "s"(p.K), "s"(p.Kp), "s"(p.N), "s"(p.M), "s"(p.A),
                 "s"(p.lda), "s"(p.flags), "s"(p.grid), "s"(p.iw));
}

// MODE 0: q/s given.  MODE 1: fused quant of fp16 rows.  MODE 2: fused quant of f32 rows.
// MR: largest row count of the fused modes (1 or 4).  NORM: RMSNorm before the
// quantization (fused modes, one row).
template <int BITS, bool SWIGLU, int MODE, bool NORM, int WAVES, int MR, int XW>
__global__ __launch_bounds__(64 * WAVES) void gemv_kernel(GemvParams p) {
    using T = typename std::conditional<MODE == 2, float, __half>::type;
    constexpr bool FUSED = MODE != 0;
    constexpr int NT = 64 * WAVES;
    constexpr int KS = BITS == 4 ? 256 : 128;
    constexpr int BATCH = GemvCfg<WAVES, FUSED>::BATCH;
    constexpr int XR = XW > 0 ? XW
                       : XW < 0 ? MR * -XW
                       : NORM   ? (MR > 1 ? kNormRowsRegs : GemvCfg<WAVES, FUSED>::XREGS_NORM)
                                : GemvCfg<WAVES, FUSED>::XREGS;
    constexpr int ROWS = FUSED ? MR : kGemvMaxRows;  // rows whose sums leave the matrix core
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float s_rows[kGemvMaxRows];
    gemv_fetch_params(p);
    __shared__ float s_inv[kFusedMaxRows];
    __shared__ float s_red[kFusedMaxRows][WAVES];  // wave maxima per row (0 from waves owning no group)
    __shared__ int s_bad[WAVES];

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r0 = blockIdx.x * p.iw;  // first output channel of the item
    const int ncols = gemv_out_cols(p);
    const int Nh = p.N >> 1;
    const int steps = p.Kp / KS;
    const int m_lane = lane & 15;
    const bool live = m_lane < p.M;
    const int m_src = min(m_lane, p.M - 1);

    // ---- 1. channel scales and activation loads (before any weight load) ---------
    // the scales of this thread's epilogue outputs, so the epilogue needs no memory trip
    float wsg = 0.0f, wsu = 0.0f;
    if (tid < 16 * p.M) {
        const int cg = min(r0 + (tid & 15), ncols - 1);
        wsg = p.wscale[cg];
        if constexpr (SWIGLU) wsu = p.wscale[(p.N >> 1) + cg];
    }
    XGroup<T> xr[FUSED ? XR : 1];
    float gr[NORM ? XR : 1][8];
    const int ngroups = p.K >> 3;
    const int gpt = XW < 0 ? -XW : (ngroups + NT - 1) / NT;  // groups per thread per row
    const int nreg = FUSED ? p.M * gpt : 0;   // uniform
    // XW < 0: -XW groups per thread per row, known at compile time, so the slots' rows
    // and groups are constants in the unrolled loops and the per-slot row selects vanish
    // (the multi-row prologue is VALU-bound at 4 rows)
    const GemvSlots<FUSED ? XR : 1> sl(gpt);
    if constexpr (FUSED && MR == 1) {
        // Only owned groups are loaded.  These loads may sit in branches because every
        // weight load below is unconditional: waits for them then count exactly the
        // weight loads issued after them.
#pragma unroll
        for (int i = 0; i < XR; ++i) {
            if (i < nreg) {
                const int m = i / gpt, g = tid + NT * (i - m * gpt);
                if (g < ngroups) xr[i].load(reinterpret_cast<const T*>(p.A) + (int64_t)m * p.lda + 8 * g);
            }
        }
        if constexpr (NORM) {
            // gamma for every held group (rows share it: one copy per register slot keeps
            // the indexing static)
#pragma unroll
            for (int i = 0; i < XR; ++i) {
                const int m = MR == 1 ? 0 : i / gpt, g = tid + NT * (i - m * gpt);
                if (i < nreg && g < ngroups) {
                    const float4 a = *reinterpret_cast<const float4*>(p.gamma + 8 * g);
                    const float4 b = *reinterpret_cast<const float4*>(p.gamma + 8 * g + 4);
                    gr[i][0] = a.x; gr[i][1] = a.y; gr[i][2] = a.z; gr[i][3] = a.w;
                    gr[i][4] = b.x; gr[i][5] = b.y; gr[i][6] = b.z; gr[i][7] = b.w;
                }
            }
        }
    } else if constexpr (FUSED) {
        gemv_load_rows<MR, XR, NT, NORM>(p, xr, gr, sl, nreg, ngroups);
    } else {
        if (tid < p.M) s_rows[tid] = p.s ? p.s[tid] : 0.0f;
    }

    // Threads holding two or more activation groups (long rows): every wave's activation
    // loads enter the CU's memory queue before any wave's weight loads.  A barrier here
    // without waiting for the loads; the down GEMV (K = 9728) 7.05 -> 6.35 us per launch.
    // With one group per thread it measured slower (o 4.12 -> 4.22 us) and is skipped.
    if constexpr (FUSED) {
        if (nreg >= 2) issue_barrier();
    }

    // ---- 2. first weight batch ---------------------------------------------------
    // lane rows past the item's width (or past the last channel) re-read its last row
    const int wrow_l = min(r0 + min(lane & 15, p.iw - 1), ncols - 1);
    const uint8_t* wg = p.W + (int64_t)wrow_l * p.wrow + (lane >> 4) * 16;
    const uint8_t* wu = SWIGLU ? p.W + (int64_t)(Nh + wrow_l) * p.wrow + (lane >> 4) * 16 : nullptr;
    const int8_t* qrow = FUSED ? nullptr : p.q + (int64_t)m_src * p.ldq + (lane >> 4) * (BITS == 4 ? 32 : 16);
    StepBuf<BATCH, FUSED> b0, b1;
    int base = wave;
    load_batch<BITS, SWIGLU, FUSED, WAVES, BATCH>(b0, wg, wu, qrow, live, base, steps);

    // ---- 3. prologue: per-token scale and quantized rows in LDS ------------------
    // LDS rows 0..M-1 hold the quantized activations; row M is all zeros and feeds
    // the matrix-core rows M..15.  One row keeps its prologue written out here: the
    // shared gemv_fused_prologue, same arithmetic, measured slower at one row (qkv
    // 2560 x 6144 5.40 -> 5.70 us per launch, the 36-layer stack 1107 -> 1121 us), where
    // it saves little (one scale, few slot divisions).
    const int astride = p.Kp + 16;
    uint8_t* lds_a = smem;
    if constexpr (FUSED && MR == 1) {
        const bool rne = (p.flags & kFlagRne) != 0;
        float nsc[MR];  // RMSNorm scale per row
#pragma unroll
        for (int m = 0; m < MR; ++m) nsc[m] = 1.0f;
        if constexpr (NORM) {
            // the reference summation order needs each whole row in one place: f32 rows
            // [M][K] in LDS, one wave per row
            float* lds_x = reinterpret_cast<float*>(smem);
#pragma unroll
            for (int i = 0; i < XR; ++i) {
                const int m = MR == 1 ? 0 : i / gpt, g = tid + NT * (i - m * gpt);
                if (i < nreg && g < ngroups) {
                    float v[8];
                    xr[i].get(v);
#pragma unroll
                    for (int e = 0; e < 8; ++e) lds_x[m * p.K + 8 * g + e] = v[e];
                }
            }
            lds_barrier();
            if (wave < p.M) {
                const float* xm = lds_x + wave * p.K;
                const float sum = (p.flags & kFlagNormSeq) != 0 ? (lane == 0 ? lds_sumsq_seq(xm, p.K) : 0.0f)  // src/ops/norm.rs:38
                                                                : lds_sumsq_neon16(xm, p.K);  // src/model/cpu.rs:14-35
                if (lane == 0) s_inv[wave] = 1.0f / __builtin_sqrtf(sum / (float)p.K + p.eps);
            }
            lds_barrier();
#pragma unroll
            for (int m = 0; m < MR; ++m) nsc[m] = m < p.M ? s_inv[m] : 1.0f;
            lds_barrier();  // lds_x is overwritten by the quantized rows below
        }
        const bool owner_wave = wave * 64 < ngroups;  // waves holding activation groups (uniform)
        if (owner_wave) {
            float mx[MR];
#pragma unroll
            for (int m = 0; m < MR; ++m) mx[m] = 0.0f;
            int bad = 0;
#pragma unroll
            for (int i = 0; i < XR; ++i) {
                if (i < nreg) {
                    const int m = i / gpt, g = tid + NT * (i - m * gpt);  // m is uniform
                    if (g < ngroups) {
                        float lm;
                        if constexpr (MODE == 1 && !NORM) {
                            // fp16 rows: absmax and finiteness from the bit patterns
                            const uint4 r = xr[i].raw;
                            bool nonfinite;
                            const uint32_t mb = absmax_bits_f16x8_ref(r, nonfinite);
                            bad |= nonfinite;
                            lm = f32_of_f16_bits(mb);
                        } else {
                            float v[8];
                            xr[i].get(v);
#pragma unroll
                            for (int e = 0; e < 8; ++e) bad |= !__builtin_isfinite(v[e]);
                            if constexpr (NORM) {
                                float ns = 1.0f;
#pragma unroll
                                for (int mm = 0; mm < MR; ++mm)
                                    if (mm == m) ns = nsc[mm];
#pragma unroll
                                for (int e = 0; e < 8; ++e) v[e] = (v[e] * ns) * gr[i][e];
                            }
                            lm = 0.0f;
#pragma unroll
                            for (int e = 0; e < 8; ++e) lm = fmaxf(lm, fabsf(v[e]));
                            bad |= !__builtin_isfinite(lm);  // the normalized values must stay finite too
                        }
#pragma unroll
                        for (int mm = 0; mm < MR; ++mm)
                            if (mm == m) mx[mm] = fmaxf(mx[mm], lm);
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const float w = m < p.M ? wave_max_nonneg(mx[m]) : 0.0f;
                if (lane == 0) s_red[m][wave] = w;
            }
            const bool any_bad = __ballot(bad) != 0;
            if (lane == 0) s_bad[wave] = any_bad;
        } else if (lane == 0) {
#pragma unroll
            for (int m = 0; m < MR; ++m) s_red[m][wave] = 0.0f;
            s_bad[wave] = 0;
        }
        lds_barrier();
        // Per-token scales, computed by every thread of the waves that hold activation
        // groups (the others go straight to the barrier instead of spending the SIMDs on
        // scales they do not use) from all WAVES wave maxima (zeros, the identity of a max
        // of magnitudes, from the waves that own no group): a loop of fixed length lets
        // the reads issue back to back and wait once; one bounded by the number of owning
        // waves waited for each read in turn (about 1 us per launch).
        if (owner_wave) {
            int bad_rows = 0;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) bad_rows |= s_bad[w];
            float inv[MR];
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float am = 0.0f;
#pragma unroll
                for (int w = 0; w < WAVES; ++w) am = fmaxf(am, s_red[m][w]);
                const float s = qscale_from_absmax(am);  // src/npu.rs:1101-1106
                inv[m] = 1.0f / s;
                if (tid == 0 && m < p.M) s_rows[m] = s;
            }
            if (tid == 0 && bad_rows && p.err && blockIdx.x == 0) atomicOr(p.err, 1u);
            if (!bad_rows) {
                // finite rows (the usual case): the short rounding sequence
                if (rne)
                    gemv_quant_rows_1<BITS, NORM, true, MR>(xr, gr, nsc, inv, lds_a, astride, nreg, gpt, ngroups, tid, NT);
                else
                    gemv_quant_rows_1<BITS, NORM, false, MR>(xr, gr, nsc, inv, lds_a, astride, nreg, gpt, ngroups, tid, NT);
            } else {
#pragma unroll
                for (int i = 0; i < XR; ++i) {
                    if (i < nreg) {
                        const int m = i / gpt, g = tid + NT * (i - m * gpt);
                        if (g < ngroups) {
                            float v[8];
                            xr[i].get(v);
                            if constexpr (NORM) {
                                float ns = 1.0f;
#pragma unroll
                                for (int mm = 0; mm < MR; ++mm)
                                    if (mm == m) ns = nsc[mm];
#pragma unroll
                                for (int e = 0; e < 8; ++e) v[e] = (v[e] * ns) * gr[i][e];
                            }
                            float im = 1.0f;
#pragma unroll
                            for (int mm = 0; mm < MR; ++mm)
                                if (mm == m) im = inv[mm];
                            int q[8];
#pragma unroll
                            for (int e = 0; e < 8; ++e) q[e] = quant_one(v[e], im, rne);  // src/npu.rs:1107-1110
                            uint32_t w0 = 0, w1 = 0;
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                w0 |= (uint32_t)(q[e] & 0xff) << (8 * e);
                                w1 |= (uint32_t)(q[4 + e] & 0xff) << (8 * e);
                            }
                            *reinterpret_cast<uint2*>(lds_a + m * astride + 8 * g) = make_uint2(w0, w1);
                        }
                    }
                }
            }
        }
        // zero the K..Kp tail of each row and the whole zero row M
        for (int m = 0; m < p.M; ++m)
            for (int k = p.K + tid * 8; k < p.Kp; k += NT * 8)
                *reinterpret_cast<uint2*>(lds_a + m * astride + k) = make_uint2(0, 0);
        for (int k = tid * 16; k < p.Kp; k += NT * 16)
            *reinterpret_cast<uint4*>(lds_a + p.M * astride + k) = make_uint4(0, 0, 0, 0);
    } else if constexpr (FUSED) {
        gemv_fused_prologue<BITS, MODE, NORM, WAVES, MR>(p, xr, gr, sl, nreg, ngroups, smem, astride, s_inv, s_red,
                                                         s_bad, s_rows);
    }
    lds_barrier();

    // ---- 4. stream the weights through the matrix core ---------------------------
    const uint8_t* arow = lds_a + (live ? m_lane : p.M) * astride + (lane >> 4) * (BITS == 4 ? 32 : 16);
    v4i ag = {0, 0, 0, 0}, au = {0, 0, 0, 0};
    while (base < steps) {
        const int nb = base + WAVES * BATCH;
        if (nb < steps) load_batch<BITS, SWIGLU, FUSED, WAVES, BATCH>(b1, wg, wu, qrow, live, nb, steps);
        compute_batch<BITS, SWIGLU, FUSED, WAVES, BATCH>(ag, au, b0, arow, base, steps);
        base = nb;
        if (base >= steps) break;
        const int nb2 = base + WAVES * BATCH;
        if (nb2 < steps) load_batch<BITS, SWIGLU, FUSED, WAVES, BATCH>(b0, wg, wu, qrow, live, nb2, steps);
        compute_batch<BITS, SWIGLU, FUSED, WAVES, BATCH>(ag, au, b1, arow, base, steps);
        base = nb2;
    }

    // ---- 5. cross-wave reduction and epilogue ------------------------------------
    // lane l holds D[4*(l/16) + i][l%16]: only lanes < 16*ceil(ROWS/4) carry real rows
    constexpr int LIVE_LANES = 16 * ((ROWS + 3) / 4);
    constexpr int REGS = ROWS < 4 ? ROWS : 4;
    lds_barrier();  // the reduction area reuses the activation area
    int* red = reinterpret_cast<int*>(smem);  // [2][WAVES][LIVE_LANES][REGS]
    if (lane < LIVE_LANES) {
#pragma unroll
        for (int i = 0; i < REGS; ++i) {
            red[(wave * LIVE_LANES + lane) * REGS + i] = ag[i];
            if constexpr (SWIGLU) red[WAVES * LIVE_LANES * REGS + (wave * LIVE_LANES + lane) * REGS + i] = au[i];
        }
    }
    lds_barrier();
    if (tid < 16 * p.M && (tid & 15) < p.iw) {
        const int m = tid >> 4, n = tid & 15;
        const int src = (16 * (m >> 2) + n) * REGS + (m & 3);
        int vg = 0, vu = 0;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            vg += red[w * LIVE_LANES * REGS + src];
            if constexpr (SWIGLU) vu += red[WAVES * LIVE_LANES * REGS + w * LIVE_LANES * REGS + src];
        }
        gemv_store<BITS, SWIGLU>(p, m, n, r0, vg, vu, s_rows[m], wsg, wsu);
    }
}

// Several items per workgroup (fused modes with more items than CUs, or rows quantized
// beforehand with more items than one round of workgroups): the activation prologue as
// in gemv_kernel, then the flat K-step sequence of the workgroup's items.
template <int BITS, bool SWIGLU, int MODE, bool NORM, int WAVES, int MR, int XW>
__global__ __launch_bounds__(64 * WAVES) void gemv_items_kernel(GemvParams p) {
    using T = typename std::conditional<MODE == 2, float, __half>::type;
    constexpr bool FUSED = MODE != 0;
    constexpr int NT = 64 * WAVES;
    constexpr int KS = BITS == 4 ? 256 : 128;
    // (two row blocks of quantized rows: one step per batch, or the buffers would spill)
    constexpr int BATCH = !FUSED && MR > 1 ? 1 : GemvCfg<WAVES, FUSED>::BATCH;
    constexpr int XR = XW > 0 ? XW
                       : XW < 0 ? MR * -XW
                       : NORM   ? (MR > 1 ? kNormRowsRegs : GemvCfg<WAVES, FUSED>::XREGS_NORM)
                                : GemvCfg<WAVES, FUSED>::XREGS;
    constexpr int ROWS = FUSED ? MR : kGemvMaxRows;  // rows whose sums leave the matrix core
    // quantized rows (MODE 0) in MR blocks of 16: 17..32 rows take two blocks, each weight
    // fragment feeding one MFMA per block
    constexpr int RB = FUSED ? 1 : MR;
    static_assert(RB == 1 || RB == 2, "one or two row blocks");
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float s_rows[kGemvMaxRows * RB];
    gemv_fetch_params(p);
    __shared__ float s_inv[kFusedMaxRows];
    __shared__ float s_red[kFusedMaxRows][WAVES];  // wave maxima per row (0 from waves owning no group)
    __shared__ int s_bad[WAVES];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar registers
    const int Nh = p.N >> 1;
    const int steps = p.Kp / KS;
    const int groups = gemv_items(p);
    const int ncols = gemv_out_cols(p);
    const int n_items = ((groups - 1 - (int)blockIdx.x) / (int)gridDim.x) + 1;  // items of this workgroup
    const int flat = n_items * steps;                                             // K steps of the workgroup
    const int total = wave < flat ? (flat - 1 - wave) / WAVES + 1 : 0;          // of them, this wave's
    const int m_lane = lane & 15;
    const bool live = m_lane < p.M;
    const int m_src = min(m_lane, p.M - 1);

    // ---- 1. channel scales and activation loads (before any weight load) ---------
    // the scales of this thread's first epilogue output (the only one unless the
    // outputs outnumber the threads)
    float wsg = 0.0f, wsu = 0.0f;
    if (tid < n_items * 16 * p.M) {
        const int cg = min(p.iw * ((int)blockIdx.x + (tid / (16 * p.M)) * (int)gridDim.x) + (tid & 15), ncols - 1);
        wsg = p.wscale[cg];
        if constexpr (SWIGLU) wsu = p.wscale[Nh + cg];
    }
    XGroup<T> xr[FUSED ? XR : 1];
    float gr[NORM ? XR : 1][8];
    const int ngroups = p.K >> 3;
    const int gpt = XW < 0 ? -XW : (ngroups + NT - 1) / NT;  // groups per thread per row
    const int nreg = FUSED ? p.M * gpt : 0;   // uniform
    // XW < 0: -XW groups per thread per row, known at compile time, so the slots' rows
    // and groups are constants in the unrolled loops and the per-slot row selects vanish
    // (the multi-row prologue is VALU-bound at 4 rows)
    const GemvSlots<FUSED ? XR : 1> sl(gpt);
    if constexpr (FUSED && MR == 1) {
        // Only owned groups are loaded.  These loads may sit in branches because every
        // weight load below is unconditional: waits for them then count exactly the
        // weight loads issued after them.
#pragma unroll
        for (int i = 0; i < XR; ++i) {
            if (i < nreg) {
                const int m = i / gpt, g = tid + NT * (i - m * gpt);
                if (g < ngroups) xr[i].load(reinterpret_cast<const T*>(p.A) + (int64_t)m * p.lda + 8 * g);
            }
        }
        if constexpr (NORM) {
            // gamma for every held group (rows share it: one copy per register slot keeps
            // the indexing static)
#pragma unroll
            for (int i = 0; i < XR; ++i) {
                const int m = MR == 1 ? 0 : i / gpt, g = tid + NT * (i - m * gpt);
                if (i < nreg && g < ngroups) {
                    const float4 a = *reinterpret_cast<const float4*>(p.gamma + 8 * g);
                    const float4 b = *reinterpret_cast<const float4*>(p.gamma + 8 * g + 4);
                    gr[i][0] = a.x; gr[i][1] = a.y; gr[i][2] = a.z; gr[i][3] = a.w;
                    gr[i][4] = b.x; gr[i][5] = b.y; gr[i][6] = b.z; gr[i][7] = b.w;
                }
            }
        }
    } else if constexpr (FUSED) {
        gemv_load_rows<MR, XR, NT, NORM>(p, xr, gr, sl, nreg, ngroups);
    } else {
        if (tid < p.M) s_rows[tid] = p.s ? p.s[tid] : 0.0f;
    }

    // Threads holding two or more activation groups (long rows): every wave's activation
    // loads enter the CU's memory queue before any wave's weight loads.  A barrier here
    // without waiting for the loads; the down GEMV (K = 9728) 7.05 -> 6.35 us per launch.
    // With one group per thread it measured slower (o 4.12 -> 4.22 us) and is skipped.
    if constexpr (FUSED) {
        if (nreg >= 2) issue_barrier();
    }

    // ---- 2. first weight batch ---------------------------------------------------
    const int lrow = min(lane & 15, p.iw - 1);  // row of the item this lane loads
    const uint8_t* wlane = p.W + (lane >> 4) * 16;
    const int64_t up_off = SWIGLU ? (int64_t)Nh * p.wrow : 0;
    const int8_t* qrow = FUSED ? nullptr : p.q + (int64_t)m_src * p.ldq + (lane >> 4) * (BITS == 4 ? 32 : 16);
    const bool live2 = RB > 1 && 16 + m_lane < p.M;
    const int8_t* qrow2 = RB > 1 ? p.q + (int64_t)min(16 + m_lane, p.M - 1) * p.ldq + (lane >> 4) * (BITS == 4 ? 32 : 16)
                                 : nullptr;
    StepBuf<BATCH, FUSED, RB> b0, b1;
    // next position to load, and the last one of the sequence (item 0, step 0 for a
    // wave without steps, so that its loads below stay in bounds)
    const int f_last = wave + (total - 1) * WAVES;
    GemvPos lpos = total > 0 ? GemvPos{wave / steps, wave % steps} : GemvPos{0, 0};
    const GemvPos last = total > 0 ? GemvPos{f_last / steps, f_last % steps} : GemvPos{0, 0};
    int lc = 0;
    // PRE batches in flight during the prologue: two with up to 8 waves; one with 16,
    // whose 1024 threads already fill the CU's queue, and one with SwiGLU, whose steps
    // load twice the bytes (two batches there delayed the prologue: gate_up 2560x19456
    // 9.55 -> 8.89 us with one; with one activation group per thread 8.45 against 8.02
    // us).  Unconditional, so that the waits for the activation loads above count
    // exactly these loads after them.
    constexpr int PRE = WAVES <= 8 && !SWIGLU ? 2 : 1;
    load_batch_items<BITS, SWIGLU, FUSED, WAVES, BATCH, RB>(b0, p, lpos, lc, total, last, wlane, up_off, qrow, live, steps, lrow, ncols, qrow2, live2);
    if constexpr (PRE == 2) {
        asm volatile("" ::: "memory");  // keep batch 0's loads ahead of batch 1's
        load_batch_items<BITS, SWIGLU, FUSED, WAVES, BATCH, RB>(b1, p, lpos, lc, total, last, wlane, up_off, qrow, live, steps, lrow, ncols, qrow2, live2);
    }

    // ---- 3. prologue: per-token scale and quantized rows in LDS ------------------
    // LDS rows 0..M-1 hold the quantized activations; row M is all zeros and feeds
    // the matrix-core rows M..15.  One row keeps its prologue written out here: the
    // shared gemv_fused_prologue, same arithmetic, measured slower at one row (qkv
    // 2560 x 6144 5.40 -> 5.70 us per launch, the 36-layer stack 1107 -> 1121 us), where
    // it saves little (one scale, few slot divisions).
    const int astride = p.Kp + 16;
    uint8_t* lds_a = smem;
    if constexpr (FUSED && MR == 1) {
        const bool rne = (p.flags & kFlagRne) != 0;
        float nsc[MR];  // RMSNorm scale per row
#pragma unroll
        for (int m = 0; m < MR; ++m) nsc[m] = 1.0f;
        if constexpr (NORM) {
            // the reference summation order needs each whole row in one place: f32 rows
            // [M][K] in LDS, one wave per row
            float* lds_x = reinterpret_cast<float*>(smem);
#pragma unroll
            for (int i = 0; i < XR; ++i) {
                const int m = MR == 1 ? 0 : i / gpt, g = tid + NT * (i - m * gpt);
                if (i < nreg && g < ngroups) {
                    float v[8];
                    xr[i].get(v);
#pragma unroll
                    for (int e = 0; e < 8; ++e) lds_x[m * p.K + 8 * g + e] = v[e];
                }
            }
            lds_barrier();
            if (wave < p.M) {
                const float* xm = lds_x + wave * p.K;
                const float sum = (p.flags & kFlagNormSeq) != 0 ? (lane == 0 ? lds_sumsq_seq(xm, p.K) : 0.0f)  // src/ops/norm.rs:38
                                                                : lds_sumsq_neon16(xm, p.K);  // src/model/cpu.rs:14-35
                if (lane == 0) s_inv[wave] = 1.0f / __builtin_sqrtf(sum / (float)p.K + p.eps);
            }
            lds_barrier();
#pragma unroll
            for (int m = 0; m < MR; ++m) nsc[m] = m < p.M ? s_inv[m] : 1.0f;
            lds_barrier();  // lds_x is overwritten by the quantized rows below
        }
        const bool owner_wave = wave * 64 < ngroups;  // waves holding activation groups (uniform)
        if (owner_wave) {
            float mx[MR];
#pragma unroll
            for (int m = 0; m < MR; ++m) mx[m] = 0.0f;
            int bad = 0;
#pragma unroll
            for (int i = 0; i < XR; ++i) {
                if (i < nreg) {
                    const int m = i / gpt, g = tid + NT * (i - m * gpt);  // m is uniform
                    if (g < ngroups) {
                        float lm;
                        if constexpr (MODE == 1 && !NORM) {
                            // fp16 rows: absmax and finiteness from the bit patterns
                            const uint4 r = xr[i].raw;
                            bool nonfinite;
                            const uint32_t mb = absmax_bits_f16x8_ref(r, nonfinite);
                            bad |= nonfinite;
                            lm = f32_of_f16_bits(mb);
                        } else {
                            float v[8];
                            xr[i].get(v);
#pragma unroll
                            for (int e = 0; e < 8; ++e) bad |= !__builtin_isfinite(v[e]);
                            if constexpr (NORM) {
                                float ns = 1.0f;
#pragma unroll
                                for (int mm = 0; mm < MR; ++mm)
                                    if (mm == m) ns = nsc[mm];
#pragma unroll
                                for (int e = 0; e < 8; ++e) v[e] = (v[e] * ns) * gr[i][e];
                            }
                            lm = 0.0f;
#pragma unroll
                            for (int e = 0; e < 8; ++e) lm = fmaxf(lm, fabsf(v[e]));
                            bad |= !__builtin_isfinite(lm);  // the normalized values must stay finite too
                        }
#pragma unroll
                        for (int mm = 0; mm < MR; ++mm)
                            if (mm == m) mx[mm] = fmaxf(mx[mm], lm);
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const float w = m < p.M ? wave_max_nonneg(mx[m]) : 0.0f;
                if (lane == 0) s_red[m][wave] = w;
            }
            const bool any_bad = __ballot(bad) != 0;
            if (lane == 0) s_bad[wave] = any_bad;
        } else if (lane == 0) {
#pragma unroll
            for (int m = 0; m < MR; ++m) s_red[m][wave] = 0.0f;
            s_bad[wave] = 0;
        }
        lds_barrier();
        // Per-token scales, computed by every thread of the waves that hold activation
        // groups (the others go straight to the barrier instead of spending the SIMDs on
        // scales they do not use) from all WAVES wave maxima (zeros, the identity of a max
        // of magnitudes, from the waves that own no group): a loop of fixed length lets
        // the reads issue back to back and wait once; one bounded by the number of owning
        // waves waited for each read in turn (about 1 us per launch).
        if (owner_wave) {
            int bad_rows = 0;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) bad_rows |= s_bad[w];
            float inv[MR];
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float am = 0.0f;
#pragma unroll
                for (int w = 0; w < WAVES; ++w) am = fmaxf(am, s_red[m][w]);
                const float s = qscale_from_absmax(am);  // src/npu.rs:1101-1106
                inv[m] = 1.0f / s;
                if (tid == 0 && m < p.M) s_rows[m] = s;
            }
            if (tid == 0 && bad_rows && p.err && blockIdx.x == 0) atomicOr(p.err, 1u);
            if (!bad_rows) {
                // finite rows (the usual case): the short rounding sequence
                if (rne)
                    gemv_quant_rows_1<BITS, NORM, true, MR>(xr, gr, nsc, inv, lds_a, astride, nreg, gpt, ngroups, tid, NT);
                else
                    gemv_quant_rows_1<BITS, NORM, false, MR>(xr, gr, nsc, inv, lds_a, astride, nreg, gpt, ngroups, tid, NT);
            } else {
#pragma unroll
                for (int i = 0; i < XR; ++i) {
                    if (i < nreg) {
                        const int m = i / gpt, g = tid + NT * (i - m * gpt);
                        if (g < ngroups) {
                            float v[8];
                            xr[i].get(v);
                            if constexpr (NORM) {
                                float ns = 1.0f;
#pragma unroll
                                for (int mm = 0; mm < MR; ++mm)
                                    if (mm == m) ns = nsc[mm];
#pragma unroll
                                for (int e = 0; e < 8; ++e) v[e] = (v[e] * ns) * gr[i][e];
                            }
                            float im = 1.0f;
#pragma unroll
                            for (int mm = 0; mm < MR; ++mm)
                                if (mm == m) im = inv[mm];
                            int q[8];
#pragma unroll
                            for (int e = 0; e < 8; ++e) q[e] = quant_one(v[e], im, rne);  // src/npu.rs:1107-1110
                            uint32_t w0 = 0, w1 = 0;
#pragma unroll
                            for (int e = 0; e < 4; ++e) {
                                w0 |= (uint32_t)(q[e] & 0xff) << (8 * e);
                                w1 |= (uint32_t)(q[4 + e] & 0xff) << (8 * e);
                            }
                            *reinterpret_cast<uint2*>(lds_a + m * astride + 8 * g) = make_uint2(w0, w1);
                        }
                    }
                }
            }
        }
        // zero the K..Kp tail of each row and the whole zero row M
        for (int m = 0; m < p.M; ++m)
            for (int k = p.K + tid * 8; k < p.Kp; k += NT * 8)
                *reinterpret_cast<uint2*>(lds_a + m * astride + k) = make_uint2(0, 0);
        for (int k = tid * 16; k < p.Kp; k += NT * 16)
            *reinterpret_cast<uint4*>(lds_a + p.M * astride + k) = make_uint4(0, 0, 0, 0);
    } else if constexpr (FUSED) {
        gemv_fused_prologue<BITS, MODE, NORM, WAVES, MR>(p, xr, gr, sl, nreg, ngroups, smem, astride, s_inv, s_red,
                                                         s_bad, s_rows);
    }
    lds_barrier();

    // ---- 4. stream the weights through the matrix core ---------------------------
    // lane l holds D[4*(l/16) + i][l%16]: only lanes < 16*ceil(ROWS/4) carry real rows
    constexpr int LIVE_LANES = 16 * ((ROWS + 3) / 4);
    constexpr int REGS = ROWS < 4 ? ROWS : 4;
    int* red = reinterpret_cast<int*>(smem + gemv_red_offset(p.M, p.Kp, p.K, FUSED, NORM));
    const uint8_t* arow = lds_a + (live ? m_lane : p.M) * astride + (lane >> 4) * (BITS == 4 ? 32 : 16);
    v4i ag = {0, 0, 0, 0}, au = {0, 0, 0, 0};
    v4i ag2 = {0, 0, 0, 0}, au2 = {0, 0, 0, 0};  // the second row block
    GemvPos cpos{wave / steps, wave % steps};  // next position to multiply
    int cc = 0, cj = 0;
    while (cc < total) {
        if (PRE == 1 && lc < total)
            load_batch_items<BITS, SWIGLU, FUSED, WAVES, BATCH, RB>(b1, p, lpos, lc, total, last, wlane, up_off, qrow, live, steps, lrow, ncols, qrow2, live2);
        compute_batch_items<BITS, SWIGLU, FUSED, WAVES, BATCH, LIVE_LANES, REGS, RB>(ag, au, b0, arow, cpos, cc, total, cj,
                                                                               red, wave, lane, steps, &ag2, &au2);
        if (PRE == 2 && lc < total)
            load_batch_items<BITS, SWIGLU, FUSED, WAVES, BATCH, RB>(b0, p, lpos, lc, total, last, wlane, up_off, qrow, live, steps, lrow, ncols, qrow2, live2);
        if (cc >= total) break;
        if (PRE == 1 && lc < total)
            load_batch_items<BITS, SWIGLU, FUSED, WAVES, BATCH, RB>(b0, p, lpos, lc, total, last, wlane, up_off, qrow, live, steps, lrow, ncols, qrow2, live2);
        compute_batch_items<BITS, SWIGLU, FUSED, WAVES, BATCH, LIVE_LANES, REGS, RB>(ag, au, b1, arow, cpos, cc, total, cj,
                                                                               red, wave, lane, steps, &ag2, &au2);
        if (PRE == 2 && lc < total)
            load_batch_items<BITS, SWIGLU, FUSED, WAVES, BATCH, RB>(b1, p, lpos, lc, total, last, wlane, up_off, qrow, live, steps, lrow, ncols, qrow2, live2);
    }
    if constexpr (RB > 1) {
        for (; cj < n_items; ++cj) {
            gemv_flush<SWIGLU, WAVES, LIVE_LANES, REGS>(red, 2 * cj, wave, lane, ag, au);
            gemv_flush<SWIGLU, WAVES, LIVE_LANES, REGS>(red, 2 * cj + 1, wave, lane, ag2, au2);
        }
    } else {
        while (cj < n_items) gemv_flush<SWIGLU, WAVES, LIVE_LANES, REGS>(red, cj++, wave, lane, ag, au);
    }

    // ---- 5. cross-wave reduction and epilogue ------------------------------------
    lds_barrier();
    for (int o = tid; o < n_items * 16 * p.M; o += NT) {
        const int jj = o / (16 * p.M), rem = o - jj * 16 * p.M;
        const int m = rem >> 4, n = rem & 15;
        const int mb = RB > 1 ? m & 15 : m, slot = RB > 1 ? 2 * jj + (m >> 4) : jj;  // row in its block, sum slot
        const int src = (16 * (mb >> 2) + n) * REGS + (mb & 3);
        int vg = 0, vu = 0;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            vg += red[((slot * 2) * WAVES + w) * LIVE_LANES * REGS + src];
            if constexpr (SWIGLU) vu += red[((slot * 2 + 1) * WAVES + w) * LIVE_LANES * REGS + src];
        }
        const int r0 = p.iw * ((int)blockIdx.x + jj * (int)gridDim.x);
        if (n >= p.iw) continue;  // a re-read row, not an output
        if (o != tid) {
            wsg = p.wscale[min(r0 + n, ncols - 1)];
            if constexpr (SWIGLU) wsu = p.wscale[Nh + min(r0 + n, ncols - 1)];
        }
        gemv_store<BITS, SWIGLU>(p, m, n, r0, vg, vu, s_rows[m], wsg, wsu);
    }
}

template <int BITS, bool SWIGLU, int MODE, bool NORM, int MR, int WAVES, int XW = 0>
static hipError_t launch_k(const GemvParams& p, dim3 grid, bool items, size_t lds, hipStream_t st) {
    if (!items) {
        hipLaunchKernelGGL((gemv_kernel<BITS, SWIGLU, MODE, NORM, WAVES, MR, XW>), grid, dim3(64 * WAVES), lds, st, p);
        return hipGetLastError();
    }
    {
        const void* f = reinterpret_cast<const void*>(&gemv_items_kernel<BITS, SWIGLU, MODE, NORM, WAVES, MR, XW>);
        if (lds > 64 * 1024) {
            static const hipError_t a = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 159 * 1024);
            if (a != hipSuccess) return a;
        }
        hipLaunchKernelGGL((gemv_items_kernel<BITS, SWIGLU, MODE, NORM, WAVES, MR, XW>), grid, dim3(64 * WAVES), lds, st,
                           p);
        return hipGetLastError();
    }
}

template <int BITS, bool SWIGLU, int MODE, bool NORM, int MR>
static hipError_t launch_w(const GemvParams& p, int waves, size_t lds, hipStream_t st) {
    const int groups = gemv_items(p);
    const bool items = p.grid > 0 && p.grid < groups;
    const dim3 grid(items ? p.grid : groups);
    if constexpr (MODE != 0) {
        const int gpt = ((p.K >> 3) + 64 * waves - 1) / (64 * waves);  // groups per thread per row
        if constexpr (!NORM) {
            if (gpt == 2 && waves == 16)
                return launch_k<BITS, SWIGLU, MODE, NORM, MR, 16, kTwoGroupRegs>(p, grid, items, lds, st);
        }
        if (gpt == 1) {
            switch (waves) {
                case 4: return launch_k<BITS, SWIGLU, MODE, NORM, MR, 4, kOneGroupRegs>(p, grid, items, lds, st);
                case 8: return launch_k<BITS, SWIGLU, MODE, NORM, MR, 8, kOneGroupRegs>(p, grid, items, lds, st);
                case 16:
                    if constexpr (NORM && MR > 1) return hipErrorInvalidValue;  // as below
                    else return launch_k<BITS, SWIGLU, MODE, NORM, MR, 16, kOneGroupRegs>(p, grid, items, lds, st);
                default: return hipErrorInvalidValue;
            }
        }
    }
    switch (waves) {
        case 4: return launch_k<BITS, SWIGLU, MODE, NORM, MR, 4>(p, grid, items, lds, st);
        case 8: return launch_k<BITS, SWIGLU, MODE, NORM, MR, 8>(p, grid, items, lds, st);
        case 16:
            // several RMSNorm rows do not fit 1024-thread workgroups' registers (gemv_can_fuse
            // refuses them), so those kernels are not built
            if constexpr (NORM && MR > 1) {
                return hipErrorInvalidValue;
            } else {
                if constexpr (MR > 1 && MODE != 0) {
                    const int gpt = ((p.K >> 3) + 1023) / 1024;  // groups per thread per row
                    if (p.M * gpt > fused_regs(16, false))
                        return launch_k<BITS, SWIGLU, MODE, NORM, MR, 16, kWideRowsRegs>(p, grid, items, lds, st);
                }
                return launch_k<BITS, SWIGLU, MODE, NORM, MR, 16>(p, grid, items, lds, st);
            }
        default: return hipErrorInvalidValue;  // the LDS above was sized for `waves`
    }
}

// One-row instances (qlin_gemv_1row.hip).  They sit in a code object of their own, so
// their code addresses do not move when the multi-row kernels change: the one-row
// layer step measured 24.6 against 25.2 us for two builds whose one-row kernels were
// instruction for instruction the same and differed only in where they were placed.
hipError_t launch_gemv_1row(const GemvParams& p, int bits, bool swiglu, int mode, bool norm, int waves, size_t lds,
                            hipStream_t st);

// 5..8-row instances (qlin_gemv_8rows.hip): 8 waves, one activation group per thread per
// row, no RMSNorm.
hipError_t launch_gemv_8rows(const GemvParams& p, int bits, bool swiglu, int mode, int waves, size_t lds,
                             hipStream_t st);

}  // namespace qlin
