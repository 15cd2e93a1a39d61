// Device-side description of a decode chain (see qlin_chain.hip).
#pragma once

#include <hip/hip_fp16.h>

#include "qlin_internal.hpp"

namespace qlin {

struct ChainStage {
    const uint8_t* W;       // packed weights [Np, wrow]
    const float* wscale;    // [Np]
    int64_t wrow;
    int bits, K, Kp, N, Np;
    int flags;              // kFlagSwiglu | kFlagRne | kFlagNormSeq
    int groups;             // items: 16-channel groups ((SwiGLU ? N/2 : Np) / 16)
    const float* gamma;     // RMSNorm weights [K] or null
    float eps;
    const __half* in;       // input rows: an earlier stage's output, or null for the chain input
    int64_t ld_in;
    int x_offset;           // first chain-input column read (when in is null)
    _Float16* out;          // stage output rows [rows, N or N/2]
    int64_t ld_out;
    // residual update (res_kind 1: the chain input from column res_x_offset; 2: an earlier
    // stage's output at res): out = R + y * rmult
    int res_kind;
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
    uint32_t* counters;        // [n_stages], zero at rest
    uint32_t* err;             // bit 0: non-finite input; bit 1: a stage wait gave up
    int spin_limit;
    int kp_max;                // largest Kp over the stages
    int lds_q_bytes, lds_red_bytes;
};

size_t chain_lds_bytes(int max_rows, int kp_max, int k_max, size_t* q_bytes, size_t* red_bytes);
hipError_t launch_chain(const ChainParams& p, int grid, size_t lds, hipStream_t stream);
int chain_resident_per_cu(int max_rows, size_t lds);  // workgroups of the chain kernel per CU
constexpr int kChainThreadsPerBlock = 512;
constexpr int kChainMaxLds = 159 * 1024;  // dynamic LDS cap: 160 KiB less the static words

}  // namespace qlin
