// Device-side description of a decode chain (see qlin_chain.hip).
#pragma once

#include <hip/hip_fp16.h>

#include "qlin_internal.hpp"

namespace qlin {

constexpr int kChainComputeWaves = 4;  // waves that stream weights (one per SIMD)
constexpr int kChainMaxLds = 159 * 1024;  // dynamic LDS cap: 160 KiB less the static words
constexpr int kChainFlagStride = 256;     // flag words per stage (>= grid, multiple of 256)

// Wave shape of the chain kernel for MR rows (1 or 4).  The 4-row instance quantizes four
// rows per stage, so it runs eight helper waves; three waves per SIMD then leave 168
// VGPRs a lane, and its compute waves hold 32 weight registers instead of 40 (measured
// on the 36-layer stack at 4 rows: 1746 us against 1866 us with four helpers; the 1-row
// instance ran slower with eight, 1180 us against 1155 us).
template <int MR>
struct ChainShape {
    static constexpr int kHelperWaves = MR > 1 ? 8 : 4;  // waves that exchange rows and quantize them
    static constexpr int kBufRegs = MR > 1 ? 32 : 40;    // 16-byte weight registers per compute lane
    static constexpr int kThreads = 64 * (kChainComputeWaves + kHelperWaves);
    static constexpr int kMaxSteps = kBufRegs / 2;  // weight steps a compute wave holds per round
};

struct ChainStage {
    const uint8_t* W;       // packed weights [Np, wrow]
    const float* wscale;    // [Np]
    int64_t wrow;
    int bits, K, Kp, N, Np;
    int flags;              // kFlagSwiglu | kFlagRne | kFlagNormSeq
    int ncols;              // output columns: N, or N/2 with SwiGLU
    int iw, ipw;            // output channels per item (1..16), items per workgroup
    int steps;              // 128-byte weight steps per row: Kp / 256 (W4) or Kp / 128 (W8)
    const float* gamma;     // RMSNorm weights [K] or null
    float eps;
    const __half* in;       // input rows: an earlier stage's output, or null for the chain input
    int64_t ld_in;
    int x_offset;           // first chain-input column read (when in is null)
    _Float16* out;          // stage output rows [rows, ncols]
    int64_t ld_out;
    // residual update (res_kind 1: the chain input from column res_x_offset; 2: an earlier
    // stage's output at res): out = R + y * rmult
    int res_kind;
    int res_stage;          // stage whose output res points into (-1: the chain input)
    const __half* res;
    int64_t ld_res;
    int res_x_offset;
    float rmult;
};

struct ChainParams {
    const ChainStage* stages;  // device array
    int n_stages;
    int M;                     // rows, 1..4
    const __half* x;           // chain input (stage 0) and output (last stage)
    int64_t ldx;
    _Float16* y;
    int64_t ldy;
    uint32_t* flags;           // [n_stages][kChainFlagStride]: launch epoch of each workgroup's
                               // finished part of each stage
    uint32_t* epochs;          // [grid]: launches each workgroup has completed
    uint32_t* err;             // bit 0: non-finite input; bit 1: a stage wait gave up
    int spin_limit;
    int kp_max;                // largest Kp over the stages
    int ipw_max;               // largest items per workgroup over the stages
    // LDS carve-up, byte offsets into the dynamic area
    int off_x, xstride;        // raw input rows (fp16), row stride in bytes (multiple of 1 KiB)
    int off_g;                 // RMSNorm weights (f32)
    int off_acc;               // int32 sums [2][ipw_max * 16][MR]
    int off_sc;                // per-channel scales [2][ipw_max * 16]
    int off_res;               // residual rows [ipw_max * 16][MR] (f32)
};

// LDS bytes of a chain (and the carve-up written into p).
size_t chain_lds_layout(int max_rows, int kp_max, int k_max, int kg_max, int ipw_max, ChainParams* p);
hipError_t launch_chain(const ChainParams& p, int grid, size_t lds, hipStream_t stream);
int chain_resident_per_cu(int max_rows, size_t lds);  // workgroups of the chain kernel per CU

}  // namespace qlin
