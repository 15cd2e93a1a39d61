// Pieces of the MFMA matrix-vector product shared by the decode GEMV and the
// decode chain: 16-byte loads, the W4 unpack + MFMA step over one 16-row x 128-byte
// weight block, A operands from the quantized rows in LDS, and a DPP wave max.
#pragma once

#include "qlin_internal.hpp"

namespace qlin {

__device__ __forceinline__ v4i ld16(const void* p) {
    return *reinterpret_cast<const v4i*>(p);
}

template <int BITS>
__device__ __forceinline__ void mfma_step(v4i& acc, const v4i b[2], const v4i a[4]) {
    if constexpr (BITS == 8) {
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[0], b[0], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[1], b[1], acc, 0, 0, 0);
    } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            v4i lo, hi;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                lo[d] = (b[j][d] << 4) & 0xF0F0F0F0;
                hi[d] = b[j][d] & 0xF0F0F0F0;
            }
            const v4i b0 = {lo[0], hi[0], lo[1], hi[1]};
            const v4i b1 = {lo[2], hi[2], lo[3], hi[3]};
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[2 * j], b0, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[2 * j + 1], b1, acc, 0, 0, 0);
        }
    }
}

// A operand of one wave step: W8 uses a[0..1] (k 64j + 16g), W4 a[0..3] (k 128j + 32g + 16h).
template <int BITS>
__device__ __forceinline__ void a_from_lds(v4i a[4], const uint8_t* arow) {
    if constexpr (BITS == 8) {
        a[0] = ld16(arow);
        a[1] = ld16(arow + 64);
    } else {
        a[0] = ld16(arow);
        a[1] = ld16(arow + 16);
        a[2] = ld16(arow + 128);
        a[3] = ld16(arow + 144);
    }
}

// Wave-wide max of non-negative floats by DPP (no LDS traffic); valid in lane 63.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_max_step(float v) {
    const int o = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xf, false);
    return fmaxf(v, __builtin_bit_cast(float, o));
}
__device__ __forceinline__ float wave_max_nonneg(float v) {
    v = dpp_max_step<0x111, 0xf>(v);  // row_shr:1
    v = dpp_max_step<0x112, 0xf>(v);  // row_shr:2
    v = dpp_max_step<0x114, 0xf>(v);  // row_shr:4
    v = dpp_max_step<0x118, 0xf>(v);  // row_shr:8  -> lane 15 of each row holds the row max
    v = dpp_max_step<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v = dpp_max_step<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Per-row maxima of MR rows from per-wave maxima red[m * SEG + w] (SEG waves per row,
// non-negative values): lane m * SEG + w reads its word and the SEG lanes of each row
// meet by DPP, so every lane of row m's segment returns row m's max.  One LDS read for
// all rows instead of MR * SEG broadcast reads in every lane.  The whole wave must be
// active.
template <int SEG, int MR>
__device__ __forceinline__ float rows_max_lanes(const float* red) {
    static_assert(MR * SEG <= 64 && (SEG == 4 || SEG == 8 || SEG == 16), "segments of 4, 8 or 16 lanes");
    const int lane = threadIdx.x & 63;
    float v = lane < MR * SEG ? red[lane] : 0.0f;
    v = dpp_max_step<0xB1, 0xf>(v);  // quad_perm [1, 0, 3, 2]
    v = dpp_max_step<0x4E, 0xf>(v);  // quad_perm [2, 3, 0, 1]: every lane of a quad holds its max
    if constexpr (SEG >= 8) v = dpp_max_step<0x141, 0xf>(v);   // row_half_mirror: 8-lane max
    if constexpr (SEG >= 16) v = dpp_max_step<0x140, 0xf>(v);  // row_mirror: 16-lane max
    return v;
}

// v of lane `src` (a compile-time or wave-uniform lane index).
__device__ __forceinline__ float lane_value(float v, int src) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src));
}

}  // namespace qlin
