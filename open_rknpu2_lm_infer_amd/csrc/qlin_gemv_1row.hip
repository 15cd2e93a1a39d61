// One-row instances of the fused decode GEMV kernels (activation rows quantized in the
// kernel), the decode path of a single sequence.
#include "qlin_gemv_kern.hpp"

namespace qlin {

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
