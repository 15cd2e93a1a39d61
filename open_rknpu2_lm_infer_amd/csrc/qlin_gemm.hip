// Kernel (c) + (d): prefill GEMM on gfx950 int8 MFMA with the dequant / SiLU-gate
// epilogue.  Replaces the native library's NPU int4 x int4 K-wave GEMM plus CPU
// int32 reduce (QWEN3_W4A8_PIPELINE_REVIEW_20261020.md:28-31); gfx950 multiplies
// the int8 codes directly, so no digit split or correction term is needed.
//
// Tile 128 (rows) x BN (channels, 128 or 256) x 128 (k); 256 threads as 2 x 2 waves,
// each wave 64 x BN/2 = 4 x BN/32 tiles of v_mfma_i32_16x16x64_i8 per 64-k half.
//
// Operands.  Quantized rows (A) and codes (B) go global -> registers -> LDS.  W4
// codes stay packed in LDS (half the LDS traffic of unpacked codes) and are unpacked
// per fragment: w & 0xF0 and (w << 4) & 0xF0 are 16*code as exact int8 values, in
// odd-k / even-k byte order, so the A rows are stored in LDS with each 8-byte group
// reordered evens-then-odds to match.  The int32 sums then carry a factor 16 that is
// shifted out exactly before the epilogue.  LDS granules are XOR-swizzled by row so
// the 16 rows one quarter-wave reads fall in distinct banks.
//
// Pipeline.  Two register buffers keep the global loads of k tiles t+1 and t+2 in
// flight while tile t is multiplied from one of two LDS buffers; one barrier per k
// tile.  All loads are unconditional (tile indices clamp at the end), so the compiler
// waits for exactly the tile it stores.  The k loop is unrolled by two so every LDS
// address is a per-lane base plus an immediate offset.
//
// SwiGLU: a tile of BN/2 output channels j loads B rows j (gate) and N/2 + j (up);
// each wave keeps gate and up accumulators for the same (row, j) in the same lane.
//
// Split-K: `splits` workgroups share a tile; each writes its int32 partial
// thread-major with device-coherent stores, waits for them, bumps the tile counter,
// and the last one sums the others, runs the epilogue and re-zeroes the counter.
#include <hip/hip_fp16.h>

#include "qlin_internal.hpp"

namespace qlin {

constexpr int BM = 128, BK = 128;
constexpr int kGemmThreads = 256;

template <int BITS, int BN>
struct GemmGeom {
    static constexpr int WN = BN / 2;                       // columns per wave
    static constexpr int NI = WN / 16;                      // B fragments per wave
    static constexpr int MI = 4;                            // A fragments per wave (64 rows)
    static constexpr int A_BYTES = BM * BK;                 // 16 KiB
    static constexpr int B_ROW = BITS == 4 ? BK / 2 : BK;   // bytes of one B row in LDS
    static constexpr int B_BYTES = BN * B_ROW;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int LDS = 2 * STAGE;
    static constexpr int NA = A_BYTES / 16 / kGemmThreads;  // 16-byte A loads per thread per k tile
    static constexpr int NB = B_BYTES / 16 / kGemmThreads;  // 16-byte B loads per thread per k tile
    static constexpr int REGS = MI * NI * 4;                // int32 accumulators per lane
};

__device__ __forceinline__ uint4 evens_odds(uint4 v) {
    // [k0..k7 | k8..k15] -> [k0 k2 k4 k6 k1 k3 k5 k7 | k8 ...]
    uint4 r;
    r.x = __builtin_amdgcn_perm(v.y, v.x, 0x06040200u);
    r.y = __builtin_amdgcn_perm(v.y, v.x, 0x07050301u);
    r.z = __builtin_amdgcn_perm(v.w, v.z, 0x06040200u);
    r.w = __builtin_amdgcn_perm(v.w, v.z, 0x07050301u);
    return r;
}

// LDS offsets.  A and W8 B rows: 128 bytes as 8 chunks of 16 swizzled by row & 7.
// W4 B rows: 64 bytes as 8 granules of 8 swizzled by (row & 7) ^ ((row >> 3) & 1).
__device__ __forceinline__ int off16(int row, int chunk) { return row * 128 + ((chunk ^ (row & 7)) << 4); }
__device__ __forceinline__ int off8(int row, int g) { return row * 64 + ((g ^ (row & 7) ^ ((row >> 3) & 1)) << 3); }

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
constexpr int kBufferFlags = 0x00020000;  // raw buffer, 32-bit data format (gfx9 word 3)

// Buffer loads: a per-tile descriptor whose size covers only the tile's valid rows,
// a per-lane row offset (VGPR) and the k offset in an SGPR.  A row beyond M or N lies
// past the descriptor's size and reads as zero, so every load is unconditional.
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, int64_t rows, int64_t ld) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)(rows * ld), kBufferFlags);
}

template <int BITS, bool SWIGLU, int BN>
struct Src {
    using G = GemmGeom<BITS, BN>;
    __amdgpu_buffer_rsrc_t ra, rg, ru;  // A rows; B (gate) rows; B up rows (SwiGLU)
    int aoff[G::NA], boff[G::NB];

    __device__ __forceinline__ Src(const GemmParams& p, int m0, int n0) {
        const int tid = threadIdx.x;
        ra = tile_rsrc(p.q + (int64_t)m0 * p.ldq, min(p.M - m0, BM), p.ldq);
        if constexpr (SWIGLU) {
            const int nh = p.N >> 1, rows = min(nh - n0, BN / 2);
            rg = tile_rsrc(p.W + (int64_t)n0 * p.wrow, rows, p.wrow);
            ru = tile_rsrc(p.W + (int64_t)(nh + n0) * p.wrow, rows, p.wrow);
        } else {
            rg = tile_rsrc(p.W + (int64_t)n0 * p.wrow, min(p.N - n0, BN), p.wrow);
            ru = rg;
        }
#pragma unroll
        for (int i = 0; i < G::NA; ++i) {
            const int c = tid + kGemmThreads * i;
            aoff[i] = (c >> 3) * (int)p.ldq + 16 * (c & 7);
        }
#pragma unroll
        for (int i = 0; i < G::NB; ++i) {
            const int c = tid + kGemmThreads * i;
            int row = BITS == 8 ? (c >> 3) : (c >> 2);
            const int ch = BITS == 8 ? (c & 7) : (c & 3);
            if (SWIGLU && i >= G::NB / 2) row -= BN / 2;  // load i < NB/2 covers gate rows [0, BN/2)
            boff[i] = row * (int)p.wrow + 16 * ch;
        }
    }
};

template <int BITS, bool SWIGLU, int BN>
struct Stage {
    using G = GemmGeom<BITS, BN>;
    uint4 ra[G::NA], rb[G::NB];

    // The scheduler barriers keep each stage's loads together and in program order:
    // the memory counter retires in issue order, so a stage stored while the other is
    // still in flight waits only for its own loads.
    __device__ __forceinline__ void load(const Src<BITS, SWIGLU, BN>& s, int kt) {
        const int k0 = kt * BK;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < G::NA; ++i) ra[i] = bload16(s.ra, s.aoff[i], k0);
#pragma unroll
        for (int i = 0; i < G::NB; ++i)
            rb[i] = bload16(SWIGLU && i >= G::NB / 2 ? s.ru : s.rg, s.boff[i], BITS == 8 ? k0 : k0 / 2);
        __builtin_amdgcn_sched_barrier(0);
    }

    __device__ __forceinline__ void store(uint8_t* As, uint8_t* Bs) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < G::NA; ++i) {
            const int c = tid + kGemmThreads * i, row = c >> 3, ch = c & 7;
            uint4 v = ra[i];
            if constexpr (BITS == 4) v = evens_odds(v);
            *reinterpret_cast<uint4*>(As + off16(row, ch)) = v;
        }
#pragma unroll
        for (int i = 0; i < G::NB; ++i) {
            const int c = tid + kGemmThreads * i;
            if constexpr (BITS == 8) {
                *reinterpret_cast<uint4*>(Bs + off16(c >> 3, c & 7)) = rb[i];
            } else {
                const int row = c >> 2, ch = c & 3;  // 16 packed bytes = granules 2ch, 2ch+1
                *reinterpret_cast<uint2*>(Bs + off8(row, 2 * ch)) = make_uint2(rb[i].x, rb[i].y);
                *reinterpret_cast<uint2*>(Bs + off8(row, 2 * ch + 1)) = make_uint2(rb[i].z, rb[i].w);
            }
        }
    }
};

template <bool SWIGLU, int BN>
__device__ __forceinline__ int b_frag_row(int wn, int ni) {
    constexpr int NI = BN / 32;
    if constexpr (SWIGLU) return (ni >= NI / 2 ? BN / 2 : 0) + wn * (BN / 4) + (ni % (NI / 2)) * 16;
    return wn * (BN / 2) + ni * 16;
}

template <int BITS, bool SWIGLU, int BN>
__device__ __forceinline__ void mma_tile(v4i (&acc)[4][BN / 32], const uint8_t* As, const uint8_t* Bs,
                                         const int (&abase)[2], const int (&bbase)[2], int wn) {
    using G = GemmGeom<BITS, BN>;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        v4i a[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const v4i*>(As + abase[h] + i * 16 * 128);
#pragma unroll
        for (int j = 0; j < G::NI; ++j) {
            v4i b;
            if constexpr (BITS == 8) {
                b = *reinterpret_cast<const v4i*>(Bs + bbase[h] + b_frag_row<SWIGLU, BN>(wn, j) * 128);
            } else {
                const uint2 w = *reinterpret_cast<const uint2*>(Bs + bbase[h] + b_frag_row<SWIGLU, BN>(wn, j) * 64);
                b[0] = (int)((w.x << 4) & 0xF0F0F0F0u);  // k 0 2 4 6
                b[1] = (int)(w.x & 0xF0F0F0F0u);         // k 1 3 5 7
                b[2] = (int)((w.y << 4) & 0xF0F0F0F0u);
                b[3] = (int)(w.y & 0xF0F0F0F0u);
            }
#pragma unroll
            // weights as the first operand: the 16x16 result is transposed, so each lane
            // holds 4 consecutive output channels of one row
            for (int i = 0; i < 4; ++i) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(b, a[i], acc[i][j], 0, 0, 0);
        }
    }
}

template <int BITS, bool SWIGLU, int OUT, int BN>
__global__ __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_kernel(GemmParams p) {
    using G = GemmGeom<BITS, BN>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;
    const int fr = lane & 15, fc = lane >> 4;

    const int tiles = p.m_tiles * p.n_tiles;
    const int NG = tiles * p.splits;
    int b = blockIdx.x;
    if ((NG & 7) == 0) b = (b & 7) * (NG >> 3) + (b >> 3);  // contiguous tile ranges per XCD
    const int z = b / tiles, tile = b - z * tiles;
    // groups of group_m m-tiles sweep all n tiles, m fastest: the workgroups resident on
    // one XCD share a few A row blocks and B column blocks in its L2
    const int per_group = p.group_m * p.n_tiles;
    const int g = tile / per_group, first_m = g * p.group_m;
    const int gm = min(p.m_tiles - first_m, p.group_m);
    const int r = tile - g * per_group;
    const int nt = r / gm, mt = first_m + (r - nt * gm);
    const int m0 = mt * BM;
    const int n0 = SWIGLU ? nt * (BN / 2) : nt * BN;
    const int ktiles = p.Kp / BK;
    const int kt_begin = z * p.ktiles_per_split;
    const int kt_end = min(kt_begin + p.ktiles_per_split, ktiles);
    const int T = kt_end - kt_begin;

    uint8_t* A0 = smem;
    uint8_t* B0 = smem + G::A_BYTES;
    uint8_t* A1 = smem + G::STAGE;
    uint8_t* B1 = smem + G::STAGE + G::A_BYTES;

    // per-lane LDS bases of the fragments (row & 7 == fr & 7 for every fragment row)
    int abase[2], bbase[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        abase[h] = off16(wm * 64 + fr, h * 4 + fc);
        bbase[h] = BITS == 8 ? off16(fr, h * 4 + fc) : off8(fr, h * 4 + fc);
    }

    v4i acc[4][G::NI];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < G::NI; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    if (T > 0) {
        // s0 / s1 carry k tiles t+2 / t+3 from global memory while tile t is multiplied;
        // past the end the tile index clamps, and the surplus tiles go to an LDS buffer
        // that is not read again.
        const int last = kt_end - 1;
        const Src<BITS, SWIGLU, BN> src(p, m0, n0);
        Stage<BITS, SWIGLU, BN> s0, s1;
        s0.load(src, kt_begin);
        s1.load(src, min(kt_begin + 1, last));
        s0.store(A0, B0);
        s0.load(src, min(kt_begin + 2, last));
        __syncthreads();
        for (int t = 0; t < T; t += 2) {
            mma_tile<BITS, SWIGLU, BN>(acc, A0, B0, abase, bbase, wn);  // tile t
            s1.store(A1, B1);                                           // tile t+1
            s1.load(src, min(kt_begin + t + 3, last));
            __syncthreads();
            if (t + 1 < T) mma_tile<BITS, SWIGLU, BN>(acc, A1, B1, abase, bbase, wn);
            s0.store(A0, B0);                                           // tile t+2
            s0.load(src, min(kt_begin + t + 4, last));
            __syncthreads();
        }
    }

    if (p.splits > 1) {
        const int64_t base = (int64_t)tile * p.splits * G::REGS * kGemmThreads;
        int32_t* mine = p.part + base + (int64_t)z * G::REGS * kGemmThreads;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < G::NI; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    store_coherent(mine + ((i * G::NI + j) * 4 + r) * kGemmThreads + tid, acc[i][j][r]);
        wait_all_memory();
        __syncthreads();
        int* flag = reinterpret_cast<int*>(smem);
        if (tid == 0) flag[0] = atomicAdd(&p.counters[tile], 1u) == (unsigned)(p.splits - 1);
        __syncthreads();
        if (!flag[0]) return;
        for (int zz = 0; zz < p.splits; ++zz) {
            if (zz == z) continue;
            const int32_t* other = p.part + base + (int64_t)zz * G::REGS * kGemmThreads;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < G::NI; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[i][j][r] += load_coherent(other + ((i * G::NI + j) * 4 + r) * kGemmThreads + tid);
        }
        if (tid == 0) atomicExch(&p.counters[tile], 0u);
    }

    // Epilogue.  Lane (fr, fc) holds, for A fragment i and B fragment j, row
    // m0 + 64 wm + 16 i + fr at the 4 consecutive channels cbase + 16 j + r.  All scales
    // are loaded first (one memory round trip), then each 4-channel group is written
    // with one vector store when the row stride and base allow it.
    constexpr int NJ = SWIGLU ? G::NI / 2 : G::NI;
    const int mrow = m0 + wm * 64 + fr;
    const int cbase = n0 + wn * (SWIGLU ? BN / 4 : BN / 2) + 4 * fc;
    const int ncols = SWIGLU ? (p.N >> 1) : p.N;
    const bool vec = (p.ldc & 3) == 0 && (reinterpret_cast<uintptr_t>(p.C) & 15) == 0;
    float sm[4];
    float4 sg[NJ], su[SWIGLU ? NJ : 1];
    if constexpr (OUT != 2) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sm[i] = p.s[min(mrow + 16 * i, p.M - 1)];
        const int cmax = (SWIGLU ? ncols : p.Np) - 4;  // scales hold Np entries
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int c = min(cbase + 16 * j, cmax);
            sg[j] = *reinterpret_cast<const float4*>(p.wscale + c);
            if constexpr (SWIGLU) su[j] = *reinterpret_cast<const float4*>(p.wscale + (p.N >> 1) + c);
        }
        // stores share the in-order memory counter with loads: wait for the scales
        // once here so no store below waits behind another
        wait_all_memory();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = mrow + 16 * i;
        if (m >= p.M) continue;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int c = cbase + 16 * j;
            if (c >= ncols) continue;
            const int64_t at = (int64_t)m * p.ldc + c;
            if constexpr (OUT == 2) {
                int o[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) o[r] = BITS == 4 ? acc[i][j][r] >> 4 : acc[i][j][r];
                int32_t* C = reinterpret_cast<int32_t*>(p.C) + at;
                if (vec && c + 3 < ncols) {
                    *reinterpret_cast<int4*>(C) = make_int4(o[0], o[1], o[2], o[3]);
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (c + r < ncols) C[r] = o[r];
                }
            } else {
                float o[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    int ag = acc[i][j][r];
                    if (BITS == 4) ag >>= 4;
                    const float g = ((float)ag * sm[i]) * sg[j][r];
                    if constexpr (SWIGLU) {
                        int au = acc[i][j + NJ][r];
                        if (BITS == 4) au >>= 4;
                        const float u = ((float)au * sm[i]) * su[j][r];
                        o[r] = (g / (1.0f + expf(-g))) * u;
                    } else {
                        o[r] = g;
                    }
                }
                if constexpr (OUT == 1) {
                    _Float16* C = reinterpret_cast<_Float16*>(p.C) + at;
                    if (vec && c + 3 < ncols) {
                        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                        h4 v;
#pragma unroll
                        for (int r = 0; r < 4; ++r) v[r] = f16_of_f32(o[r]);
                        *reinterpret_cast<h4*>(C) = v;
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (c + r < ncols) C[r] = f16_of_f32(o[r]);
                    }
                } else {
                    float* C = reinterpret_cast<float*>(p.C) + at;
                    if (vec && c + 3 < ncols) {
                        *reinterpret_cast<float4*>(C) = make_float4(o[0], o[1], o[2], o[3]);
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (c + r < ncols) C[r] = o[r];
                    }
                }
            }
        }
    }
}

template <int BITS, bool SWIGLU, int OUT, int BN>
static hipError_t launch_gemm_t(const GemmParams& p, hipStream_t stream) {
    dim3 grid(p.m_tiles * p.n_tiles * p.splits), block(kGemmThreads);
    constexpr size_t lds = GemmGeom<BITS, BN>::LDS;
    gemm_kernel<BITS, SWIGLU, OUT, BN><<<grid, block, lds, stream>>>(p);
    return hipGetLastError();
}

template <int BITS, int BN>
static hipError_t launch_gemm_b(const GemmParams& p, hipStream_t stream) {
    const bool sw = (p.flags & kFlagSwiglu) != 0;
    if (p.c_kind == 2) return launch_gemm_t<BITS, false, 2, BN>(p, stream);
    if (sw) return p.c_kind == 1 ? launch_gemm_t<BITS, true, 1, BN>(p, stream) : launch_gemm_t<BITS, true, 0, BN>(p, stream);
    return p.c_kind == 1 ? launch_gemm_t<BITS, false, 1, BN>(p, stream) : launch_gemm_t<BITS, false, 0, BN>(p, stream);
}

int gemm_tile_n(int bits, int N) {
    // W4 takes 256-channel tiles (packed codes keep the LDS stage at 32 KiB) when N
    // has enough of them; W8 and narrow W4 linears take 128.
    return (bits == 4 && N >= 4096) ? 256 : 128;
}

int gemm_regs_per_thread(int bn) { return 4 * (bn / 32) * 4; }

hipError_t launch_gemm(const GemmParams& p, int bits, int bn, hipStream_t stream) {
    if (bits == 4) return bn == 256 ? launch_gemm_b<4, 256>(p, stream) : launch_gemm_b<4, 128>(p, stream);
    return launch_gemm_b<8, 128>(p, stream);
}

}  // namespace qlin
