// Decode GEMV dispatch: shapes, LDS sizing, and the multi-row kernel instances (the
// kernels themselves are in qlin_gemv_kern.hpp).
#include "qlin_gemv_kern.hpp"

namespace qlin {

// The multi-row decode kernels of a layer, instantiated first and in this order so that
// each layer's set sits together in the code object whatever else this file instantiates
// (their layer steps move with where the kernels sit relative to each other): the W4 layer
// at 2..4 rows (gate_up, qkv, o, down), then the mixed decode stack's (RMSNorm qkv, W8 o,
// W8 down, RMSNorm gate_up).  Measured
// against the compiler's order: W4 layer at 2 / 3 / 4 rows 26.9 / 29.9 / 31.7 -> 26.6 /
// 29.5 / 31.3 us, the 36-layer stack at 2 / 3 / 4 rows 1260 / 1333 / 1411 -> 1224 / 1308 /
// 1392 us.
template __global__ void gemv_items_kernel<4, true, 1, false, 8, 4, kOneGroupRegs>(GemvParams);
template __global__ void gemv_items_kernel<4, false, 1, false, 8, 4, kOneGroupRegs>(GemvParams);
template __global__ void gemv_kernel<4, false, 1, false, 16, 4, kOneGroupRegs>(GemvParams);
template __global__ void gemv_kernel<4, false, 1, false, 16, 4, kTwoGroupRegs>(GemvParams);
template __global__ void gemv_items_kernel<4, false, 1, true, 8, 4, kOneGroupRegs>(GemvParams);
template __global__ void gemv_kernel<8, false, 1, false, 16, 4, kOneGroupRegs>(GemvParams);
template __global__ void gemv_kernel<8, false, 1, false, 16, 4, kTwoGroupRegs>(GemvParams);
template __global__ void gemv_items_kernel<4, true, 1, true, 8, 4, kOneGroupRegs>(GemvParams);

size_t gemv_lds_bytes_for(int M, int Kp, int K, int waves, bool fused, bool norm, int items) {
    const size_t rb = !fused && M > kGemvMaxRows ? 2 : 1;  // row blocks: 17..32 take the items kernel
    if (items <= 1 && rb == 1) {
        // gemv_kernel: the reduction area reuses the activation area
        size_t a = fused ? (size_t)(M + 1) * (Kp + 16) : 0;
        if (norm) a = std::max(a, (size_t)M * K * sizeof(float));
        return std::max(a, (size_t)2 * waves * 64 * 4 * sizeof(int));
    }
    const size_t rows = fused ? (M == 1 ? 1 : M <= kFusedRowsWide ? 4 : 8) : kGemvMaxRows;  // rows leaving the matrix core
    const size_t live = 16 * ((rows + 3) / 4), regs = rows < 4 ? rows : 4;
    const size_t red = (size_t)(items > 1 ? items : 1) * rb * 2 * waves * live * regs * sizeof(int);
    return gemv_red_offset(M, Kp, K, fused, norm) + red;
}

int gemv_item_width(int cols, int cus) {
    // The busiest CU streams (items per CU) x iw weight rows; take the widest iw within 3%
    // of the fewest such rows (narrower items re-read rows, L2 hits, and add positions).
    auto rows_on_busiest = [&](int iw) { return ((cols + iw - 1) / iw + cus - 1) / cus * iw; };
    int least = rows_on_busiest(16);
    for (int iw = 15; iw >= 8; --iw) least = std::min(least, rows_on_busiest(iw));
    for (int iw = 16; iw > 8; --iw)
        if (rows_on_busiest(iw) * 100 <= least * 103) return iw;
    return 8;
}

int gemv_pick_waves(int groups, int steps) {
    int w = 4;
    while (w < 16 && groups * w < 3072 && 2 * w <= steps) w *= 2;
    return w;
}

bool gemv_can_fuse(int M, int K, int waves, bool norm) {
    const int nt = 64 * waves;
    const int gpt = (K / 8 + nt - 1) / nt;
    const int regs = waves >= 16 && !norm && M > 1 ? kWideRowsRegs : fused_regs(waves, norm);
    if (K % 8 || M > kFusedMaxRows || M * gpt > regs) return false;
    // 5..8 rows: the 8-row instances only (8 waves, one group per thread per row, no RMSNorm)
    if (M > kFusedRowsWide && (norm || waves != 8 || gpt != 1)) return false;
    if (norm && (size_t)M * K * 4 > 64 * 1024) return false;  // f32 rows of the RMSNorm in LDS
    // (1024-thread workgroups would spill the per-slot gamma registers)
    if (norm && M > 1 && (waves > 8 || M * gpt > kNormRowsRegs)) return false;
    return true;
}

template <int BITS, bool SWIGLU, int MODE>
static hipError_t launch_m(const GemvParams& p, int waves, size_t lds, hipStream_t st) {
    const bool norm = p.gamma != nullptr;  // fused RMSNorm
    if (p.M == 1) return launch_gemv_1row(p, BITS, SWIGLU, MODE, norm, waves, lds, st);
    if (p.M > kFusedRowsWide) return norm ? hipErrorInvalidValue : launch_gemv_8rows(p, BITS, SWIGLU, MODE, waves, lds, st);
    return norm ? launch_w<BITS, SWIGLU, MODE, true, 4>(p, waves, lds, st)
                : launch_w<BITS, SWIGLU, MODE, false, 4>(p, waves, lds, st);
}

// 17..32 quantized rows: two row blocks per weight fragment, always the items kernel (its
// partial sums of both blocks meet in LDS; one item per workgroup unless the plan groups them)
template <int BITS, bool SWIGLU, int WAVES>
static hipError_t launch_rows2_w(const GemvParams& p, size_t lds, hipStream_t st) {
    const int groups = gemv_items(p);
    const dim3 grid(p.grid > 0 && p.grid < groups ? p.grid : groups);
    const void* f = reinterpret_cast<const void*>(&gemv_items_kernel<BITS, SWIGLU, 0, false, WAVES, 2, 0>);
    if (lds > 64 * 1024) {
        static const hipError_t a = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 159 * 1024);
        if (a != hipSuccess) return a;
    }
    hipLaunchKernelGGL((gemv_items_kernel<BITS, SWIGLU, 0, false, WAVES, 2, 0>), grid, dim3(64 * WAVES), lds, st, p);
    return hipGetLastError();
}

template <int BITS, bool SWIGLU>
static hipError_t launch_rows2(const GemvParams& p, int waves, size_t lds, hipStream_t st) {
    switch (waves) {
        case 4: return launch_rows2_w<BITS, SWIGLU, 4>(p, lds, st);
        case 8: return launch_rows2_w<BITS, SWIGLU, 8>(p, lds, st);
        default: return hipErrorInvalidValue;  // 1024-thread workgroups would spill both blocks' buffers
    }
}

template <int BITS, bool SWIGLU>
static hipError_t launch_b(const GemvParams& p, int waves, size_t lds, hipStream_t st) {
    if (!p.A) {
        if (p.M > kGemvMaxRowsWide) return hipErrorInvalidValue;
        if (p.M > kGemvMaxRows) return launch_rows2<BITS, SWIGLU>(p, waves, lds, st);
        return launch_w<BITS, SWIGLU, 0, false, 1>(p, waves, lds, st);
    }
    return p.a_f16 ? launch_m<BITS, SWIGLU, 1>(p, waves, lds, st) : launch_m<BITS, SWIGLU, 2>(p, waves, lds, st);
}

hipError_t launch_gemv(const GemvParams& p, int bits, int waves, hipStream_t stream) {
    const bool fused = p.A != nullptr;
    if (p.iw < 1 || p.iw > 16 || (waves != 4 && waves != 8 && waves != 16)) return hipErrorInvalidValue;
    // a fused prologue holds the rows in registers: refuse a wave count that cannot
    if (fused && !gemv_can_fuse(p.M, p.K, waves, p.gamma != nullptr)) return hipErrorInvalidValue;
    const int groups = gemv_items(p);
    const int grid = p.grid > 0 && p.grid < groups ? p.grid : groups;
    const int items = (groups + grid - 1) / grid;
    const size_t lds = gemv_lds_bytes_for(p.M, p.Kp, p.K, waves, fused, fused && p.gamma != nullptr, items);
    const bool sw = (p.flags & kFlagSwiglu) != 0;
    if (bits == 4) return sw ? launch_b<4, true>(p, waves, lds, stream) : launch_b<4, false>(p, waves, lds, stream);
    return sw ? launch_b<8, true>(p, waves, lds, stream) : launch_b<8, false>(p, waves, lds, stream);
}

}  // namespace qlin
