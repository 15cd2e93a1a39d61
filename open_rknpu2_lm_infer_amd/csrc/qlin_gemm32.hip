// Kernel (c) + (d): prefill GEMM on gfx950 int8 MFMA (v_mfma_i32_32x32x32_i8) with the
// dequant / SiLU-gate / residual epilogue.  Replaces the native library's NPU int4 x int4
// K-wave GEMM plus CPU int32 reduce (QWEN3_W4A8_PIPELINE_REVIEW_20261020.md:28-31); gfx950
// multiplies the int8 codes directly, so no digit split or correction term is needed.
//
// Why 32x32x32.  One v_mfma_i32_32x32x32_i8 takes a 16-byte A and a 16-byte B operand per
// lane for 32768 MACs, twice the MACs of v_mfma_i32_16x16x64_i8 for the same operand bytes,
// at the same rate (32 cycles per SIMD, 1024 MACs per clock; measured 4.2-4.3 POPS on 256
// CUs at the ~2.1 GHz the chip holds under MFMA load).  With a wave tile of TM tokens x TN
// channels the LDS bytes read per MAC are 1/TN + 1/(2 TM) (W4 B operands are packed), so a
// 64 x 128 wave tile reads 64 B per clock per CU at the MFMA rate, a quarter of the LDS
// bandwidth, where the 16x16x64 kernel with 64 x 32 wave tiles read 160 B per clock.
//
// Tile BM (tokens) x BN (weight rows) x 128 (k); WM x WN waves, each TM = BM/WM tokens x
// TN = BN/WN weight rows, MB x NB blocks of 32 x 32.  Weights are the first MFMA operand,
// so a lane of a 32 x 32 result block holds one token (lane % 32) and the channels
// 8 g + 4 (lane / 32) + i, g, i < 4: four groups of four consecutive channels.
//
// k order inside a 128-deep tile.  Lane half h (lane / 32) of the 32 x 32 x 32 instruction
// at k64 half t and step s multiplies k = 64 t + 32 h + 16 s + e, e < 16, for A and B alike
// (any common order gives the same sums).  A W4 lane then finds both steps' codes of a k64
// half in one 16-byte read: 32 codes k = 64 t + 32 h .. + 31 in device nibble order (byte b
// of each 32-bit word holds codes b and b + 4), which the unpack (x << 4) & 0xF0F0F0F0 and
// x & 0xF0F0F0F0 turns into 16 * code as exact int8 values in k order.  W4 sums carry a
// factor 16, shifted out exactly in the epilogue.
//
// Operands go from global memory straight into LDS (buffer_load_dwordx4 ... lds): one
// instruction fills 1 KiB in lane order, and which global 16-byte chunk a lane fetches
// sets the XOR swizzle that keeps the fragment reads free of bank conflicts.  Measured on
// gfx950 (8 waves, ds_read_b128, this read pattern): 128-byte rows (A, W8 B) with chunk ^
// (bit 1 of the row -> 1, bit 3 -> 2, bit 4 -> 4) and 64-byte rows (W4 B) with chunk ^
// ((row >> 3) & 3) read at 32 cycles per instruction per 8 waves, the bank limit; without
// the swizzle 8-way and 4-way conflicts.  A row beyond M or N lies past its buffer
// descriptor's size and arrives as zero, so every copy is unconditional.
//
// Pipeline.  NST LDS stages, all filled before the k loop.  One barrier per tile, at its end:
// by then every wave has read the tile out and tile t + 1 has landed, so the stage is
// refilled with tile t + NST and NST - 1 tiles stay in flight while the next is multiplied.
// Within a tile each k32 step's MFMAs use fragments read one step earlier (registers
// double-buffered), so the LDS latency hides under the previous step's MFMAs.
//
// SwiGLU: a tile of BN / 2 output channels j loads weight rows j (gate) and N / 2 + j (up);
// each wave keeps gate and up sums of the same (token, channel) in the same lane.
//
// Split-K: `splits` workgroups share a tile; each writes its int32 partial thread-major
// with device-coherent stores, waits for them, bumps the tile counter, and the last one
// sums the others, runs the epilogue and re-zeroes the counter (no memset in a graph).
// The splits of a tile are adjacent in the XCD-contiguous workgroup order, as in
// gemm_kernel.
#include <hip/hip_fp16.h>

#include "qlin_internal.hpp"

namespace qlin {

namespace g32 {

constexpr int BK = 128;
constexpr int kBufferFlags = 0x00020000;  // raw buffer, 32-bit data format (gfx9 word 3)
constexpr int kPastEnd = 0x7fff0000;      // a buffer offset past every operand (reads return zeros)
typedef int v16i __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void* lds_ptr;

template <int BITS, int BM, int BN, int WM, int WN, int NST>
struct Geom {
    static constexpr int NW = WM * WN;
    static constexpr int THREADS = 64 * NW;
    static constexpr int TM = BM / WM, TN = BN / WN;
    static constexpr int MB = TM / 32, NB = TN / 32;
    static constexpr int A_ROW = BK, B_ROW = BITS == 4 ? BK / 2 : BK;
    static constexpr int A_BYTES = BM * A_ROW, B_BYTES = BN * B_ROW;
    static constexpr int STAGE = A_BYTES + B_BYTES;
    static constexpr int A_BLK_ROWS = 1024 / A_ROW, B_BLK_ROWS = 1024 / B_ROW;  // rows per 1 KiB copy
    static constexpr int A_BLOCKS = A_BYTES / 1024, B_BLOCKS = B_BYTES / 1024;
    // copies per wave per stage; when the blocks do not divide among the waves, the last
    // slots read past their buffer (no memory access) into a scratch KiB after the stages,
    // so every wave issues the same number of copies and the copy waits stay uniform
    static constexpr int NA = (A_BLOCKS + NW - 1) / NW, NBC = (B_BLOCKS + NW - 1) / NW;
    static constexpr bool SPARE = NA * NW > A_BLOCKS || NBC * NW > B_BLOCKS;
    static constexpr int SCRATCH = NST * STAGE;  // byte offset of the scratch KiB
    static constexpr int NL = NA + NBC;
    static constexpr int LDS_ALL = NST * STAGE + (SPARE ? 1024 : 0);
    static constexpr int REGS = MB * NB * 16;  // int32 accumulators per lane
    static_assert(MB >= 1 && NB >= 1 && TM % 32 == 0 && TN % 32 == 0, "wave tile");
    static_assert(NA >= 1 && NBC >= 1 && A_BLOCKS * 1024 == A_BYTES && B_BLOCKS * 1024 == B_BYTES, "copy plan");
    static_assert(LDS_ALL <= 160 * 1024 && NST >= 3, "LDS stages");
};

__device__ __forceinline__ int swz128(int r) { return ((r >> 1) & 1) | (((r >> 3) & 1) << 1) | (((r >> 4) & 1) << 2); }
__device__ __forceinline__ int swz64(int r) { return (r >> 3) & 3; }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufferFlags);
}

__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint8_t* lds_block, int voff, int soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)lds_block, 16, voff, soff, 0, 0);
}

// s_waitcnt immediates (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8)
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier without a memory fence: the explicit waits before it have completed
// what it orders (a fence would also wait for the copies meant to stay in flight).
__device__ __forceinline__ void barrier_no_fence() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// 8 packed W4 codes (one 32-bit word, device order) -> two dwords of 16 * code as int8
__device__ __forceinline__ v4i unpack2(int x, int y) {
    const unsigned ux = (unsigned)x, uy = (unsigned)y;
    return v4i{(int)((ux << 4) & 0xF0F0F0F0u), (int)(ux & 0xF0F0F0F0u), (int)((uy << 4) & 0xF0F0F0F0u),
               (int)(uy & 0xF0F0F0F0u)};
}

// Instruction order of one k32 step for the scheduler: the next step's LDS reads first
// (they only queue work, and what they fetch is used one step later), then per B fragment
// its unpack VALU work (W4) followed by its MB MFMAs.  A wave issues in order, so reads
// placed after a run of MFMAs would issue late and the next step would wait for them.
template <int J, int NB, int MB, int VPJ>
__device__ __forceinline__ void order_mfma() {
    if constexpr (J < NB) {
        if constexpr (VPJ > 0) __builtin_amdgcn_sched_group_barrier(0x002, VPJ, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, MB, 0);
        order_mfma<J + 1, NB, MB, VPJ>();
    }
}
template <int NDS, int NB, int MB, int VPJ>
__device__ __forceinline__ void order_step() {
    if constexpr (NDS > 0) __builtin_amdgcn_sched_group_barrier(0x100, NDS, 0);
    order_mfma<0, NB, MB, VPJ>();
    __builtin_amdgcn_sched_barrier(0);
}

// First weight row of B block nb for wave column wn.
template <bool SWIGLU, int BN, int WN, int NB>
__device__ __forceinline__ constexpr int b_row0(int wn, int nb) {
    constexpr int TN = BN / WN;
    if constexpr (SWIGLU) return (nb >= NB / 2 ? BN / 2 : 0) + wn * (TN / 2) + (nb % (NB / 2)) * 32;
    return wn * TN + nb * 32;
}

// Global -> LDS copy plan of one wave: NA blocks of A (8 rows x 128 B) and NBC of B
// (W8: 8 rows x 128 B; W4: 16 rows x 64 B), each lane fetching the chunk its LDS slot
// holds under the swizzle.
template <int BITS, bool SWIGLU, int BM, int BN, int WM, int WN, int NST>
struct Copy {
    using G = Geom<BITS, BM, BN, WM, WN, NST>;
    __amdgpu_buffer_rsrc_t ra, rg, ru;
    int aoff[G::NA], boff[G::NBC];
    int wave;
    __device__ __forceinline__ Copy(const GemmParams& p, int m0, int n0, int wave_, int lane) : wave(wave_) {
        ra = rsrc(p.q + (int64_t)m0 * p.ldq, (int64_t)min(p.M - m0, BM) * p.ldq);
        if constexpr (SWIGLU) {
            const int nh = p.N >> 1, rows = min(nh - n0, BN / 2);
            rg = rsrc(p.W + (int64_t)n0 * p.wrow, (int64_t)rows * p.wrow);
            ru = rsrc(p.W + (int64_t)(nh + n0) * p.wrow, (int64_t)rows * p.wrow);
        } else {
            rg = rsrc(p.W + (int64_t)n0 * p.wrow, (int64_t)min(p.N - n0, BN) * p.wrow);
            ru = rg;
        }
#pragma unroll
        for (int i = 0; i < G::NA; ++i) {
            const int row = (wave * G::NA + i) * 8 + (lane >> 3);
            aoff[i] = row * (int)p.ldq + (((lane & 7) ^ swz128(row)) << 4);  // a spare slot: row >= BM, past ra
        }
#pragma unroll
        for (int i = 0; i < G::NBC; ++i) {
            const int blk = wave * G::NBC + i;
            int row, chunk;
            if constexpr (BITS == 8) {
                row = blk * 8 + (lane >> 3);
                chunk = (lane & 7) ^ swz128(row);
            } else {
                row = blk * 16 + (lane >> 2);
                chunk = (lane & 3) ^ swz64(row);
            }
            if (SWIGLU && row >= BN / 2) row -= BN / 2;
            boff[i] = blk < G::B_BLOCKS ? row * (int)p.wrow + (chunk << 4) : kPastEnd;
        }
    }

    // copy k tile kt into the stage at LDS byte offset `stage`
    __device__ __forceinline__ void issue(uint8_t* smem, int stage, int kt) const {
        const int k0 = kt * BK;
#pragma unroll
        for (int i = 0; i < G::NA; ++i) {
            const int blk = wave * G::NA + i;  // wave-uniform
            uint8_t* dst = G::SPARE && blk >= G::A_BLOCKS ? smem + G::SCRATCH : smem + stage + blk * 1024;
            dma16(ra, dst, aoff[i], k0);
        }
#pragma unroll
        for (int i = 0; i < G::NBC; ++i) {
            const int blk = wave * G::NBC + i;
            const bool up = SWIGLU && blk * G::B_BLK_ROWS >= BN / 2;
            uint8_t* dst = G::SPARE && blk >= G::B_BLOCKS ? smem + G::SCRATCH : smem + stage + G::A_BYTES + blk * 1024;
            dma16(up ? ru : rg, dst, boff[i], BITS == 8 ? k0 : k0 / 2);
        }
    }

};

template <int BITS, bool SWIGLU, int OUT, int BM, int BN, int WM, int WN, int NST>
__global__ __launch_bounds__(64 * WM * WN) void gemm32_kernel(GemmParams p) {
    using G = Geom<BITS, BM, BN, WM, WN, NST>;
    constexpr int MB = G::MB, NB = G::NB;
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int lr = lane & 31, lh = lane >> 5;

    const int tiles = p.m_tiles * p.n_tiles;
    const int NG = tiles * p.splits;
    int b = blockIdx.x;
    if ((NG & 7) == 0) b = (b & 7) * (NG >> 3) + (b >> 3);  // contiguous tile ranges per XCD
    const int z = b % p.splits, tile = b / p.splits;  // the splits of a tile adjacent
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
    const int last = kt_end - 1;

    // fragment read offsets inside a stage: A row wm*TM + 32 mb + lr; B row b_row0 + lr
    int a_row_off[MB], a_swz[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int row = wm * G::TM + 32 * mb + lr;
        a_row_off[mb] = row * G::A_ROW;
        a_swz[mb] = swz128(row);
    }
    int b_row_off[NB], b_swz[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
        const int row = b_row0<SWIGLU, BN, WN, NB>(wn, nb) + lr;
        b_row_off[nb] = row * G::B_ROW;
        b_swz[nb] = BITS == 4 ? swz64(row) : swz128(row);
    }

    v16i acc[MB][NB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[mb][nb][e] = 0;

    // Epilogue scales, loaded before the first copy so their round trip overlaps the k loop
    // (older than every copy, they retire before the first copy wait).  Lane (lr, lh) of
    // block (mb, nb) holds token m0 + wm*TM + 32 mb + lr and channels cb + 8 g + 4 lh + i.
    constexpr int NJ = SWIGLU ? NB / 2 : NB;  // output blocks per wave
    const int ncols = SWIGLU ? (p.N >> 1) : p.N;
    const int cwave = n0 + wn * (SWIGLU ? G::TN / 2 : G::TN);  // first output channel of the wave
    float sm[MB];
    float sg[NJ][16], su[SWIGLU ? NJ : 1][16];
    if constexpr (OUT != 2) {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) sm[mb] = p.s[min(m0 + wm * G::TM + 32 * mb + lr, p.M - 1)];
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int c = min(cwave + 32 * j + 8 * (e >> 2) + 4 * lh + (e & 3), ncols - 1);
                sg[j][e] = p.wscale[c];
                if constexpr (SWIGLU) su[j][e] = p.wscale[(p.N >> 1) + c];
            }
    }

    {
        const Copy<BITS, SWIGLU, BM, BN, WM, WN, NST> cp(p, m0, n0, wave, lane);
        // fragment reads of k32 step q (0..3: k64 half q / 2, step q % 2) of a stage
        auto read_a = [&](v4i (&a)[MB], const uint8_t* sa, int q) {
            const int chunk = 4 * (q >> 1) + 2 * lh + (q & 1);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
                a[mb] = *reinterpret_cast<const v4i*>(sa + a_row_off[mb] + ((chunk ^ a_swz[mb]) << 4));
        };
        // B: W4 the packed codes of k64 half q / 2 (both its steps), W8 step q
        auto read_b = [&](v4i (&bf)[NB], const uint8_t* sb, int q) {
            const int chunk = BITS == 4 ? 2 * (q >> 1) + lh : 4 * (q >> 1) + 2 * lh + (q & 1);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
                bf[nb] = *reinterpret_cast<const v4i*>(sb + b_row_off[nb] + ((chunk ^ b_swz[nb]) << 4));
        };
        auto mma = [&](const v4i (&a)[MB], const v4i (&bf)[NB], int s) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                v4i w;
                if constexpr (BITS == 4) w = s == 0 ? unpack2(bf[nb][0], bf[nb][1]) : unpack2(bf[nb][2], bf[nb][3]);
                else w = bf[nb];
#pragma unroll
                for (int mb = 0; mb < MB; ++mb)
                    acc[mb][nb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(w, a[mb], acc[mb][nb], 0, 0, 0);
            }
        };

        // every stage filled before the loop; afterwards NST - 1 tiles stay in flight while
        // one is multiplied
#pragma unroll
        for (int s = 0; s < NST; ++s) cp.issue(smem, s * G::STAGE, min(kt_begin + s, last));
        wait_vm<(NST - 1) * G::NL>();  // this wave's copies of tile 0 have landed
        barrier_no_fence();            // everyone's have
        v4i a0[MB], a1[MB], b0[NB], b1[NB];
        read_a(a0, smem, 0);
        read_b(b0, smem + G::A_BYTES, 0);
        constexpr int VPJ = BITS == 4 ? 6 : 0;  // unpack VALU instructions per B fragment
        for (int t = 0; t < T; ++t) {
            const uint8_t* sa = smem + (t % NST) * G::STAGE;
            const uint8_t* sb = sa + G::A_BYTES;
            // each step multiplies fragments read one step earlier and reads the next step's
            read_a(a1, sa, 1);
            if constexpr (BITS == 8) read_b(b1, sb, 1);
            mma(a0, b0, 0);
            order_step<BITS == 8 ? MB + NB : MB, NB, MB, VPJ>();
            read_a(a0, sa, 2);
            if constexpr (BITS == 4) read_b(b1, sb, 2);
            else read_b(b0, sb, 2);
            mma(a1, BITS == 4 ? b0 : b1, 1);
            order_step<MB + NB, NB, MB, VPJ>();
            read_a(a1, sa, 3);
            if constexpr (BITS == 8) read_b(b1, sb, 3);
            mma(a0, BITS == 4 ? b1 : b0, 0);
            order_step<BITS == 8 ? MB + NB : MB, NB, MB, VPJ>();
            // end of tile t: its stage is read out (the reads above have returned) and tile
            // t + 1 has landed; refill the stage with tile t + NST, read tile t + 1's first step
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            wait_vm<(NST - 2) * G::NL>();
            barrier_no_fence();
            cp.issue(smem, (t % NST) * G::STAGE, min(kt_begin + t + NST, last));
            const uint8_t* na = smem + ((t + 1) % NST) * G::STAGE;
            read_a(a0, na, 0);
            read_b(b0, na + G::A_BYTES, 0);
            mma(a1, b1, 1);
            order_step<MB + NB, NB, MB, VPJ>();
        }
        // drain the surplus copies before the LDS is reused or the workgroup ends
        wait_vm<0>();
        __syncthreads();
    }

    if (p.splits > 1) {
        const int64_t base = (int64_t)tile * p.splits * G::REGS * G::THREADS;
        int32_t* mine = p.part + base + (int64_t)z * G::REGS * G::THREADS;
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    store_coherent(mine + ((mb * NB + nb) * 16 + e) * G::THREADS + tid, acc[mb][nb][e]);
        wait_all_memory();
        __syncthreads();
        int* flag = reinterpret_cast<int*>(smem);  // the LDS stages are drained
        if (tid == 0) flag[0] = atomicAdd(&p.counters[tile], 1u) == (unsigned)(p.splits - 1);
        __syncthreads();
        if (!flag[0]) return;
        for (int zz = 0; zz < p.splits; ++zz) {
            if (zz == z) continue;
            const int32_t* other = p.part + base + (int64_t)zz * G::REGS * G::THREADS;
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        acc[mb][nb][e] += load_coherent(other + ((mb * NB + nb) * 16 + e) * G::THREADS + tid);
        }
        if (tid == 0) atomicExch(&p.counters[tile], 0u);
    }

    // Epilogue: per block, four groups of four consecutive channels of one token, each one
    // vector store when the row stride and base allow it.
    const bool vec = (p.ldc & 3) == 0 && (reinterpret_cast<uintptr_t>(p.C) & 15) == 0;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int m = m0 + wm * G::TM + 32 * mb + lr;
        if (m >= p.M) continue;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                const int c = cwave + 32 * j + 8 * gq + 4 * lh;
                if (c >= ncols) continue;
                const int64_t at = (int64_t)m * p.ldc + c;
                if constexpr (OUT == 2) {
                    int o[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) o[i] = BITS == 4 ? acc[mb][j][4 * gq + i] >> 4 : acc[mb][j][4 * gq + i];
                    int32_t* C = reinterpret_cast<int32_t*>(p.C) + at;
                    if (vec && c + 3 < ncols) {
                        *reinterpret_cast<int4*>(C) = make_int4(o[0], o[1], o[2], o[3]);
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (c + i < ncols) C[i] = o[i];
                    }
                } else {
                    float o[4];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        int ag = acc[mb][j][4 * gq + i];
                        if (BITS == 4) ag >>= 4;
                        const float gv = ((float)ag * sm[mb]) * sg[j][4 * gq + i];  // src/npu.rs:1117
                        if constexpr (SWIGLU) {
                            int au = acc[mb][j + NJ][4 * gq + i];
                            if (BITS == 4) au >>= 4;
                            const float uv = ((float)au * sm[mb]) * su[j][4 * gq + i];
                            o[i] = silu_gate(gv, uv);  // src/npu.rs:1202-1208
                        } else {
                            o[i] = gv;
                        }
                    }
                    if (!SWIGLU && p.R) {
#pragma unroll
                        for (int i = 0; i < 4; ++i)  // src/model/dense.rs:486-489
                            if (c + i < ncols) o[i] = residual_add(p.R, p.ldr, p.r_f16, p.rmult, m, c + i, o[i]);
                    }
                    if constexpr (OUT == 1) {
                        _Float16* C = reinterpret_cast<_Float16*>(p.C) + at;
                        if (vec && c + 3 < ncols) {
                            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                            h4 v;
#pragma unroll
                            for (int i = 0; i < 4; ++i) v[i] = f16_of_f32(o[i]);
                            *reinterpret_cast<h4*>(C) = v;
                        } else {
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                if (c + i < ncols) C[i] = f16_of_f32(o[i]);
                        }
                    } else {
                        float* C = reinterpret_cast<float*>(p.C) + at;
                        if (vec && c + 3 < ncols) {
                            *reinterpret_cast<float4*>(C) = make_float4(o[0], o[1], o[2], o[3]);
                        } else {
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                if (c + i < ncols) C[i] = o[i];
                        }
                    }
                }
            }
        }
    }
}

template <int BITS, bool SWIGLU, int OUT, int BM, int BN, int WM, int WN, int NST>
static hipError_t launch_s(const GemmParams& p, hipStream_t stream) {
    using G = Geom<BITS, BM, BN, WM, WN, NST>;
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&gemm32_kernel<BITS, SWIGLU, OUT, BM, BN, WM, WN, NST>),
        hipFuncAttributeMaxDynamicSharedMemorySize, G::LDS_ALL);
    if (attr != hipSuccess) return attr;
    dim3 grid(p.m_tiles * p.n_tiles * p.splits), block(G::THREADS);
    gemm32_kernel<BITS, SWIGLU, OUT, BM, BN, WM, WN, NST><<<grid, block, G::LDS_ALL, stream>>>(p);
    return hipGetLastError();
}

template <int BITS, int BM, int BN, int WM, int WN, int NST>
static hipError_t launch_cfg(const GemmParams& p, hipStream_t st) {
    const bool sw = (p.flags & kFlagSwiglu) != 0;
    if (p.c_kind == 2) return launch_s<BITS, false, 2, BM, BN, WM, WN, NST>(p, st);
    if (sw) return p.c_kind == 1 ? launch_s<BITS, true, 1, BM, BN, WM, WN, NST>(p, st)
                                 : launch_s<BITS, true, 0, BM, BN, WM, WN, NST>(p, st);
    return p.c_kind == 1 ? launch_s<BITS, false, 1, BM, BN, WM, WN, NST>(p, st)
                         : launch_s<BITS, false, 0, BM, BN, WM, WN, NST>(p, st);
}

}  // namespace g32

// Tile configurations of the 32x32x32 GEMM (tokens x weight rows, waves, stages):
//   W4 0: 128 x 128, 2 x 2 waves of 64 x 64, 3 x 24 KiB (two workgroups per CU), or 6 stages
//         when the grid holds at most one workgroup per CU
//   W4 1: 256 x 256, 2 x 4 waves of 128 x 64, 3 x 48 KiB
//   W4 2: 128 x 256, 2 x 4 waves of 64 x 64, 4 x 32 KiB
//   W4 3: 256 x 192, 4 x 3 waves of 64 x 64, 3 x 44 KiB (gate_up at 512 tokens: 204 tiles,
//         about one per CU; twelve waves keep the four SIMDs evenly loaded)
//   W8 0: 128 x 128, 2 x 2 waves of 64 x 64, 3 x 32 KiB, or 4 when at most one per CU
//   W8 1: 256 x 128, 2 x 2 waves of 128 x 64, 3 x 48 KiB
//   W8 2: 128 x 256, 2 x 4 waves of 64 x 64, 3 x 48 KiB
GemmTileCfg gemm32_tile(int bits, int cfg) {
    switch (cfg) {
        case 1: return bits == 4 ? GemmTileCfg{256, 256, 512, 128} : GemmTileCfg{256, 128, 256, 128};
        case 2: return GemmTileCfg{128, 256, 512, 64};
        case 3: return GemmTileCfg{256, 192, 768, 64};
        default: return GemmTileCfg{128, 128, 256, 64};
    }
}

hipError_t launch_gemm32(const GemmParams& p, int bits, int cfg, hipStream_t st) {
    if (bits == 4) {
        switch (cfg) {
            case 0: return p.deep ? g32::launch_cfg<4, 128, 128, 2, 2, 6>(p, st)
                                  : g32::launch_cfg<4, 128, 128, 2, 2, 3>(p, st);
            case 1: return g32::launch_cfg<4, 256, 256, 2, 4, 3>(p, st);
            case 2: return g32::launch_cfg<4, 128, 256, 2, 4, 4>(p, st);
            case 3: return g32::launch_cfg<4, 256, 192, 4, 3, 3>(p, st);
        }
    } else {
        switch (cfg) {
            case 0: return p.deep ? g32::launch_cfg<8, 128, 128, 2, 2, 4>(p, st)
                                  : g32::launch_cfg<8, 128, 128, 2, 2, 3>(p, st);
            case 1: return g32::launch_cfg<8, 256, 128, 2, 2, 3>(p, st);
            case 2: return g32::launch_cfg<8, 128, 256, 2, 4, 3>(p, st);
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace qlin
