// One-row instances of the fused decode GEMV kernels (activation rows quantized in the
// kernel), the decode path of a single sequence.
#include "qlin_gemv_kern.hpp"

namespace qlin {

// The one-row decode kernels of a layer, instantiated first and in this order so that
// they sit next to each other in the code object, whatever else this file instantiates.
// A layer step runs them back to back, and where they sit relative to each other changes
// its time: the W4 layer (gate_up, qkv, o / down) measured 24.15-24.22 us adjacent, and
// 24.4 / 24.8 / 25.1 us with 4 / 1 + 5 / 6 + 2 KiB of padding placed between them (same
// kernels, one box), consistent with the kernels' code evicting each other from the
// instruction cache.  The W4 layer: gate_up, qkv, o (one group per thread), down (two
// groups per thread); then the RMSNorm and W8 instances of the mixed decode stack.
template __global__ void gemv_items_kernel<4, true, 1, false, 8, 1, kOneGroupRegs>(GemvParams);
template __global__ void gemv_items_kernel<4, false, 1, false, 8, 1, kOneGroupRegs>(GemvParams);
template __global__ void gemv_kernel<4, false, 1, false, 16, 1, kOneGroupRegs>(GemvParams);
template __global__ void gemv_kernel<4, false, 1, false, 16, 1, kTwoGroupRegs>(GemvParams);
template __global__ void gemv_items_kernel<4, false, 1, true, 8, 1, kOneGroupRegs>(GemvParams);
template __global__ void gemv_kernel<8, false, 1, false, 16, 1, kOneGroupRegs>(GemvParams);
template __global__ void gemv_kernel<8, false, 1, false, 16, 1, kTwoGroupRegs>(GemvParams);
template __global__ void gemv_items_kernel<4, true, 1, true, 8, 1, kOneGroupRegs>(GemvParams);

template <int BITS, bool SWIGLU>
static hipError_t launch_1row_b(const GemvParams& p, int mode, bool norm, int waves, size_t lds, hipStream_t st) {
    if (mode == 1)
        return norm ? launch_w<BITS, SWIGLU, 1, true, 1>(p, waves, lds, st)
                    : launch_w<BITS, SWIGLU, 1, false, 1>(p, waves, lds, st);
    return norm ? launch_w<BITS, SWIGLU, 2, true, 1>(p, waves, lds, st)
                : launch_w<BITS, SWIGLU, 2, false, 1>(p, waves, lds, st);
}

hipError_t launch_gemv_1row(const GemvParams& p, int bits, bool swiglu, int mode, bool norm, int waves, size_t lds,
                            hipStream_t st) {
    if (p.M != 1 || (mode != 1 && mode != 2)) return hipErrorInvalidValue;
    if (bits == 4)
        return swiglu ? launch_1row_b<4, true>(p, mode, norm, waves, lds, st)
                      : launch_1row_b<4, false>(p, mode, norm, waves, lds, st);
    return swiglu ? launch_1row_b<8, true>(p, mode, norm, waves, lds, st)
                  : launch_1row_b<8, false>(p, mode, norm, waves, lds, st);
}

}  // namespace qlin
