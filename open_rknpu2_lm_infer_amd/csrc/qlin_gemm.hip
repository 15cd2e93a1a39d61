// Kernel (c) + (d): prefill GEMM on gfx950 int8 MFMA with the dequant / SiLU-gate
// epilogue.  Replaces the native library's NPU int4 x int4 K-wave GEMM plus CPU
// int32 reduce (QWEN3_W4A8_PIPELINE_REVIEW_20261020.md:28-31); gfx950 multiplies
// the int8 codes directly, so no digit split or correction term is needed.
//
// Tile 128 (rows) x BN (channels) x 128 (k); 128 * WN threads as 2 x WN waves, each
// wave 64 x BN/WN = 4 x BN/(16 WN) tiles of v_mfma_i32_16x16x64_i8 per 64-k half.
// WN = 4 (512 threads, the default) puts two waves on every SIMD even when a CU holds
// one workgroup: one wave's LDS reads and W4 unpack overlap the other's MFMAs (M = 512
// qkv 23.2 -> 20.9 us, the four layer linears 122.6 -> 114.5 us).  WN = 2 is the 2 x 2
// layout with 64 x 64 per wave (a quarter fewer LDS reads per MFMA, one wave per SIMD).
//
// Operands go from global memory straight into LDS (buffer_load_dwordx4 ... lds):
// one instruction fills 1 KiB of LDS in lane order, and which global 16-byte chunk a
// lane fetches sets the XOR swizzle that keeps fragment reads free of bank conflicts.
// gfx950 LDS has 64 banks of 4 bytes and a ds_read_b128 takes four cycles of 16 lanes;
// which lanes share a cycle was measured one access pattern at a time with calibration
// kernels under SQ_LDS_BANK_CONFLICT.  The swizzles used here read with zero conflicts there
// (and the counter reads 0 for this kernel):
// 128-byte rows (A, W8) XOR the chunk with bit 1 of the row into chunk bit 0 and bit 2
// into chunk bit 2; 64-byte rows (W4) XOR it with (row >> 1) & 3.
// A row beyond M or N lies past its buffer descriptor's size and arrives as zero.
// W4 codes stay packed in LDS; one 16-byte read gives a lane 32 codes, the k group it
// multiplies in both 64-k halves of the tile.  They are unpacked per fragment:
// (w << 4) & 0xF0 and w & 0xF0 are 16*code as exact int8 values, and the device order
// of the codes (byte b of each word holds codes b and b + 4) makes the unpacked bytes
// come out in natural k order, so activation fragments go to the matrix core as read.
// The int32 sums carry a factor 16 that is shifted out exactly at the end.
//
// Pipeline.  NST LDS stages: the copy of k tile t + NST - 1 is issued while tile t is
// multiplied.  Within a tile, the fragments of the second 64-k half are read while
// the first half's MFMAs run, and those of the next tile (after the one barrier per
// tile) while the second half's run.  Every k range has an even number of tiles (Kp is
// a multiple of 256 and splits are even), so the loop is unrolled by two with the two
// B fragment sets swapping roles and no register moves.
//
// SwiGLU: a tile of BN/2 output channels j loads B rows j (gate) and N/2 + j (up);
// each wave keeps gate and up accumulators for the same (row, j) in the same lane.
//
// Split-K: `splits` workgroups share a tile; each writes its int32 partial
// thread-major with device-coherent stores, waits for them, bumps the tile counter,
// and the last one sums the others, runs the epilogue and re-zeroes the counter.
// The splits of a tile are adjacent in the XCD-contiguous workgroup order, so when
// the grid divides among the 8 XCDs they run on one XCD (M = 512 o, 80 tiles x 2
// splits: 16.0 us against 17.8 with the splits of a tile on different XCDs).
#include <hip/hip_fp16.h>

#include "qlin_internal.hpp"

namespace qlin {

constexpr int BM = 128, BK = 128;
constexpr int kLdsBytes = 160 * 1024;  // LDS of one gfx950 CU

// W4 stages are 24 KiB: three of them let two workgroups share a CU, so one's MFMAs
// run while the other waits on LDS.  W8 stages are 32 KiB: one workgroup, four stages.
// WN: waves along N (2 x WN waves of 64 rows x BN / WN channels each).  WN = 4 puts two
// waves on every SIMD when the grid holds one workgroup per CU, so one wave's LDS reads
// and unpack overlap the other's MFMAs (a quarter more LDS reads per MFMA).
template <int BITS, int BN, int NSTAGES = (BITS == 4 ? 3 : 4), int WN = 2>
struct GemmGeom {
    static constexpr int THREADS = 128 * WN;
    static constexpr int NI = BN / (16 * WN);                  // B fragments per wave
    static constexpr int A_BYTES = BM * BK;                    // 16 KiB
    static constexpr int B_ROW = BITS == 4 ? BK / 2 : BK;      // bytes of one B row
    static constexpr int B_BYTES = BN * B_ROW;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int NST = kLdsBytes / STAGE < NSTAGES ? kLdsBytes / STAGE : NSTAGES;  // stages
    static constexpr int LDS = NST * STAGE;
    static constexpr int NA = A_BYTES / 1024 / (2 * WN);       // 1 KiB copies per wave per stage
    static constexpr int NB = B_BYTES / 1024 / (2 * WN);
    static_assert(NA >= 1 && NB >= 1 && NA * 1024 * 2 * WN == A_BYTES && NB * 1024 * 2 * WN == B_BYTES,
                  "copy plan");
    static constexpr int NL = NA + NB;
    static constexpr int REGS = 4 * NI * 4;                    // int32 accumulators per lane
    static_assert(NST >= 3, "pipeline needs three LDS stages");
};

typedef int v4i_t __attribute__((ext_vector_type(4)));
constexpr int kBufferFlags = 0x00020000;  // raw buffer, 32-bit data format (gfx9 word 3)
constexpr int kSc1 = 16;                   // buffer cache policy: coherent at device scope (sc1)
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const void* base, int64_t rows, int64_t ld) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)(rows * ld), kBufferFlags);
}

typedef __attribute__((address_space(3))) void* lds_ptr;

// chunk swizzle of a 128-byte LDS row (8 chunks of 16 bytes) from the row index
__device__ __forceinline__ int swz128(int row) { return ((row >> 1) & 1) | (((row >> 2) & 1) << 2); }

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds_block, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)lds_block, 16, voff, soff, 0, 0);
}

// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
template <int N>
__device__ __forceinline__ void wait_lgkm() {
    static_assert(N >= 0 && N < 16, "lgkmcnt range");
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4) | (N << 8));
}

// Workgroup barrier without a memory fence: the caller's explicit waits have already
// completed the LDS reads and copies it orders (a fence would also wait for the copies
// still meant to be in flight).  The empty asm statements keep the compiler from
// moving memory accesses across it.
__device__ __forceinline__ void barrier_no_fence() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// 16 packed codes (8 bytes, device order) -> 16*code as int8 in k order
__device__ __forceinline__ v4i unpack_w4(int x, int y) {
    const unsigned ux = (unsigned)x, uy = (unsigned)y;
    return v4i{(int)((ux << 4) & 0xF0F0F0F0u), (int)(ux & 0xF0F0F0F0u), (int)((uy << 4) & 0xF0F0F0F0u),
               (int)(uy & 0xF0F0F0F0u)};
}

template <bool SWIGLU, int BN, int WN>
__device__ __forceinline__ constexpr int b_frag_row(int wn, int j) {
    constexpr int NI = BN / (16 * WN);
    if constexpr (SWIGLU) return (j >= NI / 2 ? BN / 2 : 0) + wn * (BN / (2 * WN)) + (j % (NI / 2)) * 16;
    return wn * (BN / WN) + j * 16;
}

// Global -> LDS copy plan of one wave: NA activation blocks of 8 rows x 128 bytes and
// NB weight blocks (W8: 8 rows x 128 bytes; W4: 16 rows x 64 bytes).
template <int BITS, bool SWIGLU, int BN, int WN>
struct Copy {
    using G = GemmGeom<BITS, BN, 3, WN>;
    __amdgpu_buffer_rsrc_t ra, rg, ru;
    int aoff[G::NA], boff[G::NB];
    int wave;

    __device__ __forceinline__ Copy(const GemmParams& p, int m0, int n0, int wave_, int lane) : wave(wave_) {
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
            const int row = (wave * G::NA + i) * 8 + (lane >> 3);
            aoff[i] = row * (int)p.ldq + (((lane & 7) ^ swz128(row)) << 4);
        }
#pragma unroll
        for (int i = 0; i < G::NB; ++i) {
            const int blk = wave * G::NB + i;
            if constexpr (BITS == 8) {
                int row = blk * 8 + (lane >> 3);
                const int chunk = (lane & 7) ^ swz128(row);
                if (SWIGLU && row >= BN / 2) row -= BN / 2;
                boff[i] = row * (int)p.wrow + (chunk << 4);
            } else {
                int row = blk * 16 + (lane >> 2);
                const int chunk = (lane & 3) ^ ((row >> 1) & 3);
                if (SWIGLU && row >= BN / 2) row -= BN / 2;
                boff[i] = row * (int)p.wrow + (chunk << 4);
            }
        }
    }

    // copy k tile kt into the stage at LDS byte offset `stage`
    __device__ __forceinline__ void issue(uint8_t* smem, int stage, int kt) const {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < G::NA; ++i) dma16(ra, smem + stage + (wave * G::NA + i) * 1024, aoff[i], k0);
#pragma unroll
        for (int i = 0; i < G::NB; ++i) {
            const int blk = wave * G::NB + i;
            const int rows_per_blk = BITS == 8 ? 8 : 16;
            const bool up = SWIGLU && blk * rows_per_blk >= BN / 2;
            dma16(up ? ru : rg, smem + stage + G::A_BYTES + blk * 1024, boff[i], BITS == 8 ? k0 : k0 / 2);
        }
    }
};

// Fragment registers of one k tile: packed or int8 weight fragments for both halves.
template <int BITS, int BN, int WN>
struct BFrag {
    v4i v[BITS == 4 ? BN / (16 * WN) : 2 * (BN / (16 * WN))];
};

template <int BITS, bool SWIGLU, int BN, int WN>
__device__ __forceinline__ void read_b(BFrag<BITS, BN, WN>& b, const uint8_t* sb, int bbase0, int bbase1, int wn) {
    constexpr int NI = BN / (16 * WN);
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        if constexpr (BITS == 4) {
            b.v[j] = *reinterpret_cast<const v4i*>(sb + bbase0 + b_frag_row<SWIGLU, BN, WN>(wn, j) * 64);
        } else {
            b.v[2 * j] = *reinterpret_cast<const v4i*>(sb + bbase0 + b_frag_row<SWIGLU, BN, WN>(wn, j) * 128);
            b.v[2 * j + 1] = *reinterpret_cast<const v4i*>(sb + bbase1 + b_frag_row<SWIGLU, BN, WN>(wn, j) * 128);
        }
    }
}

__device__ __forceinline__ void read_a(v4i (&a)[4], const uint8_t* sa, int abase) {
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = *reinterpret_cast<const v4i*>(sa + abase + i * 16 * 128);
}

template <int BITS, int BN, int WN>
__device__ __forceinline__ void mma_half(v4i (&acc)[4][BN / (16 * WN)], const v4i (&a)[4], const BFrag<BITS, BN, WN>& b,
                                         int h) {
    constexpr int NI = BN / (16 * WN);
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        const v4i w = BITS == 4 ? (h == 0 ? unpack_w4(b.v[j][0], b.v[j][1]) : unpack_w4(b.v[j][2], b.v[j][3]))
                                : b.v[2 * j + h];
        // weights as the first operand: the 16x16 result is transposed, so each lane
        // holds 4 consecutive output channels of one row
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(w, a[i], acc[i][j], 0, 0, 0);
    }
}

// Instruction order of one half-tile region for the scheduler: the region's global-to-LDS
// copies and LDS reads first (they only queue work, and what they fetch is used one
// region later), then per B fragment its unpack VALU work followed by its 4 MFMAs.  A
// wave issues in order, so reads placed after a run of MFMAs would issue late and the
// next region would wait for them.
template <int J, int NJ, int VPJ>
__device__ __forceinline__ void order_mfma() {
    if constexpr (J < NJ) {
        if constexpr (VPJ > 0) __builtin_amdgcn_sched_group_barrier(0x002, VPJ, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        order_mfma<J + 1, NJ, VPJ>();
    }
}
template <int NJ, int VPJ, int NDS, int NVM>
__device__ __forceinline__ void order_region() {
    if constexpr (NVM > 0) __builtin_amdgcn_sched_group_barrier(0x010, NVM, 0);
    if constexpr (NDS > 0) __builtin_amdgcn_sched_group_barrier(0x100, NDS, 0);
    order_mfma<0, NJ, VPJ>();
}

// One k tile: multiply tile t (its first-half A fragments in a0, B in bc); read its
// second-half A fragments, then, after the barrier, the next tile's first-half A and
// its B fragments into bn.
template <int BITS, bool SWIGLU, int BN, int NSTG, int WN>
__device__ __forceinline__ void gemm_step(v4i (&acc)[4][BN / (16 * WN)], v4i (&a0)[4], v4i (&a1)[4],
                                          const BFrag<BITS, BN, WN>& bc, BFrag<BITS, BN, WN>& bn,
                                          const Copy<BITS, SWIGLU, BN, WN>& cp, uint8_t* smem, int t, int kt_begin,
                                          int last, int abase0, int abase1, int bbase0, int bbase1, int wn) {
    using G = GemmGeom<BITS, BN, NSTG, WN>;
    constexpr int NREAD_B = BITS == 4 ? G::NI : 2 * G::NI;     // 16-byte B reads per tile
    constexpr int VPJ = BITS == 4 ? 6 : 0;                     // unpack VALU work per B fragment
    const uint8_t* s0 = smem + (t % G::NST) * G::STAGE;
    read_a(a1, s0, abase1);
    mma_half<BITS, BN, WN>(acc, a0, bc, 0);
    order_region<G::NI, VPJ, 4, 0>();
    // Nothing moves across the two fences below: each half's MFMAs then use fragments
    // read one half (16 MFMAs) earlier instead of waiting on reads just issued.
    __builtin_amdgcn_sched_barrier(0);
    // Stage t-1 is refilled below.  This wave read it last in the previous step, and at
    // least 8 LDS reads were issued after those (LDS reads stay in program order around
    // the barrier's memory clobbers; their counter retires in order), so waiting until
    // at most the 4 reads of a1 are outstanding completes them without waiting for a1.
    wait_lgkm<4>();
    wait_vm<(G::NST - 3) * G::NL>();  // own copies of tile t+1 have landed
    barrier_no_fence();               // everyone's have, and stage t-1 is free
    const int fill = t + G::NST - 1;
    cp.issue(smem, (fill % G::NST) * G::STAGE, min(kt_begin + fill, last));
    const uint8_t* s1 = smem + ((t + 1) % G::NST) * G::STAGE;
    read_a(a0, s1, abase0);
    read_b<BITS, SWIGLU, BN, WN>(bn, s1 + G::A_BYTES, bbase0, bbase1, wn);
    mma_half<BITS, BN, WN>(acc, a1, bc, 1);
    order_region<G::NI, VPJ, 4 + NREAD_B, G::NL>();
    __builtin_amdgcn_sched_barrier(0);
}

template <int BITS, bool SWIGLU, int OUT, int BN, int NSTG, int WN>
__global__ __launch_bounds__(128 * WN) void gemm_kernel(GemmParams p) {
    using G = GemmGeom<BITS, BN, NSTG, WN>;
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const int wm = wave / WN, wn = wave % WN;
    const int fr = lane & 15, fc = lane >> 4;

    const int tiles = p.m_tiles * p.n_tiles;
    const int NG = tiles * p.splits;
    int b = blockIdx.x;
    if ((NG & 7) == 0) b = (b & 7) * (NG >> 3) + (b >> 3);  // contiguous tile ranges per XCD
    const int z = b % p.splits, tile = b / p.splits;  // the splits of a tile adjacent
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
    const int T = kt_end - kt_begin;  // even and >= 2
    const int last = kt_end - 1;

    // fragment read offsets: lane (fr, fc) multiplies k bytes [32 fc + 16 h, +16) of
    // the tile in half h, from rows whose low bits are those of fr
    const int sw = swz128(fr);
    const int abase0 = (wm * 64 + fr) * 128 + (((2 * fc) ^ sw) << 4);
    const int abase1 = (wm * 64 + fr) * 128 + (((2 * fc + 1) ^ sw) << 4);
    const int bbase0 = BITS == 4 ? fr * 64 + ((fc ^ ((fr >> 1) & 3)) << 4) : fr * 128 + (((2 * fc) ^ sw) << 4);
    const int bbase1 = BITS == 4 ? 0 : fr * 128 + (((2 * fc + 1) ^ sw) << 4);

    v4i acc[4][G::NI];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < G::NI; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    // Epilogue scales, loaded before the first copy so their round trip overlaps the k
    // loop.  Lane (fr, fc) holds, for A fragment i and B fragment j, row m0 + 64 wm + 16 i
    // + fr at the 4 consecutive channels cbase + 16 j + r.  (Older than every copy, they
    // retire before the first copy wait, which counts only copies issued after them.)
    constexpr int NJ = SWIGLU ? G::NI / 2 : G::NI;
    const int mrow = m0 + wm * 64 + fr;
    const int cbase = n0 + wn * (SWIGLU ? BN / (2 * WN) : BN / WN) + 4 * fc;
    const int ncols = SWIGLU ? (p.N >> 1) : p.N;
    float sm[4];
    float4 sg[NJ], su[SWIGLU ? NJ : 1];
    if constexpr (OUT != 2) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sm[i] = p.s[min(mrow + 16 * i, p.M - 1)];
        // per element and clamped: with SwiGLU, N / 2 (the up block's first scale) may be
        // any integer, so 16-byte loads would be misaligned
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int c = min(cbase + 16 * j + r, ncols - 1);
                sg[j][r] = p.wscale[c];
                if constexpr (SWIGLU) su[j][r] = p.wscale[(p.N >> 1) + c];
            }
        }
    }

    {
        const Copy<BITS, SWIGLU, BN, WN> cp(p, m0, n0, wave, lane);
#pragma unroll
        for (int s = 0; s < G::NST - 1; ++s) cp.issue(smem, s * G::STAGE, min(kt_begin + s, last));
        wait_vm<(G::NST - 2) * G::NL>();
        barrier_no_fence();

        v4i a0[4], a1[4];
        BFrag<BITS, BN, WN> bx, by;
        read_a(a0, smem, abase0);
        read_b<BITS, SWIGLU, BN, WN>(bx, smem + G::A_BYTES, bbase0, bbase1, wn);

        for (int t = 0; t < T; t += 2) {
            gemm_step<BITS, SWIGLU, BN, NSTG, WN>(acc, a0, a1, bx, by, cp, smem, t, kt_begin, last, abase0, abase1,
                                                  bbase0, bbase1, wn);
            gemm_step<BITS, SWIGLU, BN, NSTG, WN>(acc, a0, a1, by, bx, cp, smem, t + 1, kt_begin, last, abase0, abase1,
                                                  bbase0, bbase1, wn);
        }
        // drain the surplus copies before the LDS is reused or the workgroup ends
        wait_vm<0>();
        __syncthreads();
    }

    if (p.splits > 1) {
        // Each thread's 4 x NI accumulator fragments go out as 16-byte device-coherent
        // stores, fragment-major ((i * NI + j) * THREADS + tid): a quarter of the memory
        // instructions of one 4-byte store per register.
        constexpr int SLICE = G::REGS * G::THREADS * 4;  // bytes of one split's partial tile
        const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
            p.part + (int64_t)tile * p.splits * G::REGS * G::THREADS, (short)0, p.splits * SLICE, kBufferFlags);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < G::NI; ++j)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[i][j]), rp,
                                                       ((i * G::NI + j) * G::THREADS + tid) * 16, z * SLICE, kSc1);
        wait_all_memory();
        __syncthreads();
        int* flag = reinterpret_cast<int*>(smem);  // the LDS stages are drained
        if (tid == 0) flag[0] = atomicAdd(&p.counters[tile], 1u) == (unsigned)(p.splits - 1);
        __syncthreads();
        if (!flag[0]) return;
        for (int zz = 0; zz < p.splits; ++zz) {
            if (zz == z) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < G::NI; ++j)
                    acc[i][j] += __builtin_bit_cast(
                        v4i, __builtin_amdgcn_raw_buffer_load_b128(rp, ((i * G::NI + j) * G::THREADS + tid) * 16, zz * SLICE, kSc1));
        }
        if (tid == 0) atomicExch(&p.counters[tile], 0u);
    }

    // Epilogue: each 4-channel group is written with one vector store when the row
    // stride and base allow it (the scales were loaded before the k loop).
    const bool vec = (p.ldc & 3) == 0 && (reinterpret_cast<uintptr_t>(p.C) & 15) == 0;
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
                        o[r] = silu_gate(g, u);  // src/npu.rs:1202-1208
                    } else {
                        o[r] = g;
                    }
                }
                if (!SWIGLU && p.R) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)  // src/model/dense.rs:486-489
                        if (c + r < ncols) o[r] = residual_add(p.R, p.ldr, p.r_f16, p.rmult, m, c + r, o[r]);
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

template <int BITS, bool SWIGLU, int OUT, int BN, int NSTG, int WN>
static hipError_t launch_gemm_s(const GemmParams& p, hipStream_t stream) {
    using G = GemmGeom<BITS, BN, NSTG, WN>;
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&gemm_kernel<BITS, SWIGLU, OUT, BN, NSTG, WN>),
        hipFuncAttributeMaxDynamicSharedMemorySize, G::LDS);
    if (attr != hipSuccess) return attr;
    dim3 grid(p.m_tiles * p.n_tiles * p.splits), block(G::THREADS);
    gemm_kernel<BITS, SWIGLU, OUT, BN, NSTG, WN><<<grid, block, G::LDS, stream>>>(p);
    return hipGetLastError();
}

// Stage counts: the default lets two workgroups share a CU (W4); with p.deep (at most
// one workgroup per CU in the grid) more k tiles are in flight ahead of the matrix core.
template <int BITS, bool SWIGLU, int OUT, int BN>
static hipError_t launch_gemm_t(const GemmParams& p, hipStream_t stream) {
    // W4: four stages measured ahead of three, five and six at 512 tokens (qkv 18.7 / 16.3 /
    // 16.9 / 17.1 us, down 26.4 / 22.6 / 23.0 / 23.5 us)
    constexpr int DEEP = 4;
    if (p.deep) {
        if (p.wn == 4) return launch_gemm_s<BITS, SWIGLU, OUT, BN, DEEP, 4>(p, stream);
        return launch_gemm_s<BITS, SWIGLU, OUT, BN, DEEP, 2>(p, stream);
    }
    if (p.wn == 4) return launch_gemm_s<BITS, SWIGLU, OUT, BN, (BITS == 4 ? 3 : 4), 4>(p, stream);
    return launch_gemm_s<BITS, SWIGLU, OUT, BN, (BITS == 4 ? 3 : 4), 2>(p, stream);
}

template <int BITS, int BN>
static hipError_t launch_gemm_b(const GemmParams& p, hipStream_t stream) {
    const bool sw = (p.flags & kFlagSwiglu) != 0;
    if (p.c_kind == 2) return launch_gemm_t<BITS, false, 2, BN>(p, stream);
    if (sw) return p.c_kind == 1 ? launch_gemm_t<BITS, true, 1, BN>(p, stream) : launch_gemm_t<BITS, true, 0, BN>(p, stream);
    return p.c_kind == 1 ? launch_gemm_t<BITS, false, 1, BN>(p, stream) : launch_gemm_t<BITS, false, 0, BN>(p, stream);
}

int gemm_tile_n(int, int) { return 128; }


int gemm_regs_per_thread(int bn) { return 4 * (bn / 32) * 4; }

hipError_t launch_gemm(const GemmParams& p, int bits, int bn, hipStream_t stream) {
    if (bn != 128) return hipErrorInvalidValue;
    return bits == 4 ? launch_gemm_b<4, 128>(p, stream) : launch_gemm_b<8, 128>(p, stream);
}

}  // namespace qlin
