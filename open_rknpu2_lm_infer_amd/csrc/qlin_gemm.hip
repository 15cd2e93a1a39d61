// Kernel (c) + (d): prefill GEMM on gfx950 int8 MFMA with the dequant / SiLU-gate
// epilogue.  Replaces the native library's NPU int4 x int4 K-wave GEMM plus CPU
// int32 reduce (QWEN3_W4A8_PIPELINE_REVIEW_20261020.md:28-31); gfx950 multiplies
// the int8 codes directly, so no digit split or correction term is needed.
//
// Tile 128 (rows) x 128 (channels) x 128 (k), 256 threads as 2 x 2 waves, each wave
// 64 x 64 = 4 x 4 tiles of v_mfma_i32_16x16x64_i8 per 64-k half.  Operands go
// global -> registers -> LDS (double buffered, one barrier per k tile); 16-byte LDS
// chunks are XOR-swizzled by (row & 7) so the 16 rows a quarter-wave reads hit
// distinct banks.  W4 codes are unpacked while filling LDS: each byte's nibbles
// become 16*code int8 values in natural k order (v_perm_b32 interleave), so the int32
// sum is 16x the exact one and is shifted back before dequant.
//
// SwiGLU: a tile of 64 output channels j loads B rows j (gate) and N/2 + j (up);
// each wave keeps gate and up accumulators for the same (row, j) in the same lane.
//
// Split-K: `splits` workgroups share a tile; each writes its int32 partial
// thread-major into scratch, bumps the tile counter, and the last one sums the others,
// runs the epilogue and re-zeroes the counter.
#include <hip/hip_fp16.h>

#include "qlin_internal.hpp"

namespace qlin {

constexpr int BM = 128, BN = 128, BK = 128;
constexpr int kGemmThreads = 256;
constexpr size_t kGemmLds = 2 * (BM * BK + BN * BK);  // 64 KiB

__device__ __forceinline__ int swz(int row, int chunk) {
    return row * BK + ((chunk ^ (row & 7)) << 4);
}

// natural-order unpack of 8 nibbles (one dword) into two dwords of 16*code
__device__ __forceinline__ void unpack_w4(uint32_t w, uint32_t& n0, uint32_t& n1) {
    const uint32_t lo = (w << 4) & 0xF0F0F0F0u;  // k = 0,2,4,6
    const uint32_t hi = w & 0xF0F0F0F0u;         // k = 1,3,5,7
    n0 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);  // k0 k1 k2 k3
    n1 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);  // k4 k5 k6 k7
}

template <int BITS, bool SWIGLU>
struct GemmLoader {
    static constexpr int NA = 4;                  // 16-byte A loads per thread per k tile
    static constexpr int NB = BITS == 8 ? 4 : 2;  // 16-byte B loads per thread per k tile
    uint4 ra[NA], rb[NB];

    __device__ __forceinline__ int brow_global(const GemmParams& p, int n0, int r) const {
        if constexpr (SWIGLU) return r < 64 ? n0 + r : (p.N >> 1) + n0 + (r - 64);
        return n0 + r;
    }
    __device__ __forceinline__ bool brow_ok(const GemmParams& p, int n0, int r) const {
        if constexpr (SWIGLU) return n0 + (r & 63) < (p.N >> 1);
        return n0 + r < p.Np;
    }

    __device__ __forceinline__ void load(const GemmParams& p, int m0, int n0, int kt) {
        const int tid = threadIdx.x;
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int c = tid + kGemmThreads * i, row = c >> 3, ch = c & 7;
            if (m0 + row < p.M)
                ra[i] = *reinterpret_cast<const uint4*>(p.q + (int64_t)(m0 + row) * p.ldq + k0 + 16 * ch);
            else
                ra[i] = make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int c = tid + kGemmThreads * i;
            const int row = BITS == 8 ? (c >> 3) : (c >> 2), ch = BITS == 8 ? (c & 7) : (c & 3);
            if (brow_ok(p, n0, row)) {
                const int64_t off = (int64_t)brow_global(p, n0, row) * p.wrow +
                                    (BITS == 8 ? k0 : k0 / 2) + 16 * ch;
                rb[i] = *reinterpret_cast<const uint4*>(p.W + off);
            } else {
                rb[i] = make_uint4(0, 0, 0, 0);
            }
        }
    }

    __device__ __forceinline__ void store(uint8_t* As, uint8_t* Bs) const {
        const int tid = threadIdx.x;
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int c = tid + kGemmThreads * i, row = c >> 3, ch = c & 7;
            *reinterpret_cast<uint4*>(As + swz(row, ch)) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int c = tid + kGemmThreads * i;
            if constexpr (BITS == 8) {
                const int row = c >> 3, ch = c & 7;
                *reinterpret_cast<uint4*>(Bs + swz(row, ch)) = rb[i];
            } else {
                const int row = c >> 2, ch = c & 3;  // 16 packed bytes = k [32ch, 32ch+32)
                uint4 u0, u1;
                unpack_w4(rb[i].x, u0.x, u0.y);
                unpack_w4(rb[i].y, u0.z, u0.w);
                unpack_w4(rb[i].z, u1.x, u1.y);
                unpack_w4(rb[i].w, u1.z, u1.w);
                *reinterpret_cast<uint4*>(Bs + swz(row, 2 * ch)) = u0;
                *reinterpret_cast<uint4*>(Bs + swz(row, 2 * ch + 1)) = u1;
            }
        }
    }
};

template <bool SWIGLU>
__device__ __forceinline__ int b_frag_row(int wn, int ni) {
    if constexpr (SWIGLU) return (ni >> 1) * 64 + wn * 32 + (ni & 1) * 16;
    return wn * 64 + ni * 16;
}

template <int BITS, bool SWIGLU, int OUT>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(GemmParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wm = wave >> 1, wn = wave & 1;

    const int tiles = p.m_tiles * p.n_tiles;
    const int G = tiles * p.splits;
    int b = blockIdx.x;
    if ((G & 7) == 0) b = (b & 7) * (G >> 3) + (b >> 3);  // contiguous tile ranges per XCD
    const int z = b / tiles, tile = b - z * tiles;
    const int nt = tile / p.m_tiles, mt = tile - nt * p.m_tiles;
    const int m0 = mt * BM;
    const int n0 = SWIGLU ? nt * 64 : nt * BN;
    const int ktiles = p.Kp / BK;
    const int kt_begin = z * p.ktiles_per_split;
    const int kt_end = min(kt_begin + p.ktiles_per_split, ktiles);

    uint8_t* As0 = smem;
    uint8_t* Bs0 = smem + BM * BK;
    uint8_t* As1 = smem + BM * BK + BN * BK;
    uint8_t* Bs1 = As1 + BM * BK;

    v4i acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    GemmLoader<BITS, SWIGLU> ld;
    if (kt_begin < kt_end) {
        ld.load(p, m0, n0, kt_begin);
        ld.store(As0, Bs0);
    }
    __syncthreads();
    const int fr = lane & 15, fc = lane >> 4;
    for (int kt = kt_begin; kt < kt_end; ++kt) {
        const bool odd = (kt - kt_begin) & 1;
        const uint8_t* As = odd ? As1 : As0;
        const uint8_t* Bs = odd ? Bs1 : Bs0;
        const bool more = kt + 1 < kt_end;
        if (more) ld.load(p, m0, n0, kt + 1);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            v4i a[4], bb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int ra = wm * 64 + i * 16 + fr;
                a[i] = *reinterpret_cast<const v4i*>(As + swz(ra, h * 4 + fc));
                const int rb = b_frag_row<SWIGLU>(wn, i) + fr;
                bb[i] = *reinterpret_cast<const v4i*>(Bs + swz(rb, h * 4 + fc));
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[i], bb[j], acc[i][j], 0, 0, 0);
        }
        if (more) ld.store(odd ? As0 : As1, odd ? Bs0 : Bs1);
        __syncthreads();
    }

    if (p.splits > 1) {
        const int64_t base = ((int64_t)tile * p.splits) * 64 * kGemmThreads;
        int32_t* mine = p.part + base + (int64_t)z * 64 * kGemmThreads;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) store_coherent(mine + ((i * 4 + j) * 4 + r) * kGemmThreads + tid, acc[i][j][r]);
        wait_all_memory();
        __syncthreads();
        int* flag = reinterpret_cast<int*>(smem);
        if (tid == 0) flag[0] = atomicAdd(&p.counters[tile], 1u) == (unsigned)(p.splits - 1);
        __syncthreads();
        if (!flag[0]) return;
        for (int zz = 0; zz < p.splits; ++zz) {
            if (zz == z) continue;
            const int32_t* other = p.part + base + (int64_t)zz * 64 * kGemmThreads;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        acc[i][j][r] += load_coherent(other + ((i * 4 + j) * 4 + r) * kGemmThreads + tid);
        }
        if (tid == 0) atomicExch(&p.counters[tile], 0u);
    }

    // epilogue: lane holds D[4*(lane/16) + r][lane % 16] of each 16x16 tile
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + wm * 64 + i * 16 + 4 * fc + r;
            if (m >= p.M) continue;
            const float sm = OUT == 2 ? 0.0f : p.s[m];
            if constexpr (SWIGLU) {
                const int Nh = p.N >> 1;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int col = n0 + wn * 32 + j * 16 + fr;
                    if (col >= Nh) continue;
                    int ag = acc[i][j][r], au = acc[i][j + 2][r];
                    if (BITS == 4) {
                        ag >>= 4;
                        au >>= 4;
                    }
                    const float g = ((float)ag * sm) * p.wscale[col];
                    const float u = ((float)au * sm) * p.wscale[Nh + col];
                    const float o = (g / (1.0f + expf(-g))) * u;
                    if (OUT == 1)
                        reinterpret_cast<_Float16*>(p.C)[(int64_t)m * p.ldc + col] = f16_of_f32(o);
                    else
                        reinterpret_cast<float*>(p.C)[(int64_t)m * p.ldc + col] = o;
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int col = n0 + wn * 64 + j * 16 + fr;
                    if (col >= p.N) continue;
                    int a = acc[i][j][r];
                    if (BITS == 4) a >>= 4;
                    if (OUT == 2) {
                        reinterpret_cast<int32_t*>(p.C)[(int64_t)m * p.ldc + col] = a;
                    } else {
                        const float o = ((float)a * sm) * p.wscale[col];
                        if (OUT == 1)
                            reinterpret_cast<_Float16*>(p.C)[(int64_t)m * p.ldc + col] = f16_of_f32(o);
                        else
                            reinterpret_cast<float*>(p.C)[(int64_t)m * p.ldc + col] = o;
                    }
                }
            }
        }
    }
}

template <int BITS, bool SWIGLU, int OUT>
static hipError_t launch_gemm_t(const GemmParams& p, hipStream_t stream) {
    dim3 grid(p.m_tiles * p.n_tiles * p.splits), block(kGemmThreads);
    hipLaunchKernelGGL((gemm_kernel<BITS, SWIGLU, OUT>), grid, block, kGemmLds, stream, p);
    return hipGetLastError();
}

hipError_t launch_gemm(const GemmParams& p, int bits, hipStream_t stream) {
    const bool sw = (p.flags & kFlagSwiglu) != 0;
    if (p.c_kind == 2) {
        return bits == 4 ? launch_gemm_t<4, false, 2>(p, stream) : launch_gemm_t<8, false, 2>(p, stream);
    }
    if (bits == 4) {
        if (sw) return p.c_kind == 1 ? launch_gemm_t<4, true, 1>(p, stream) : launch_gemm_t<4, true, 0>(p, stream);
        return p.c_kind == 1 ? launch_gemm_t<4, false, 1>(p, stream) : launch_gemm_t<4, false, 0>(p, stream);
    }
    if (sw) return p.c_kind == 1 ? launch_gemm_t<8, true, 1>(p, stream) : launch_gemm_t<8, true, 0>(p, stream);
    return p.c_kind == 1 ? launch_gemm_t<8, false, 1>(p, stream) : launch_gemm_t<8, false, 0>(p, stream);
}

}  // namespace qlin
