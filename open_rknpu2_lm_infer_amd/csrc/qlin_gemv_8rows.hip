// 5..8-row instances of the fused decode GEMV kernels (activation rows quantized in the
// kernel): speculative-decoding verification, one token plus up to seven drafts
// (src/model/speculation.rs:36,51).  512-thread workgroups with one activation group per
// thread per row (K <= 4096), no RMSNorm; the matrix core's 16 activation columns hold
// all 8 rows, so the weight stream and the MFMA count are those of one row.
#include "qlin_gemv_kern.hpp"

namespace qlin {

template <int BITS, bool SWIGLU, int MODE>
static hipError_t launch_8rows_m(const GemvParams& p, size_t lds, hipStream_t st) {
    const int groups = gemv_items(p);
    const bool items = p.grid > 0 && p.grid < groups;
    return launch_k<BITS, SWIGLU, MODE, false, 8, 8, kOneGroupRegs>(p, dim3(items ? p.grid : groups), items, lds, st);
}

template <int BITS, bool SWIGLU>
static hipError_t launch_8rows_b(const GemvParams& p, int mode, size_t lds, hipStream_t st) {
    return mode == 1 ? launch_8rows_m<BITS, SWIGLU, 1>(p, lds, st) : launch_8rows_m<BITS, SWIGLU, 2>(p, lds, st);
}

hipError_t launch_gemv_8rows(const GemvParams& p, int bits, bool swiglu, int mode, int waves, size_t lds,
                             hipStream_t st) {
    // the instances hold exactly one 8-value group of each row per thread
    if (p.M <= kFusedRowsWide || p.M > kFusedMaxRows || waves != 8 || p.gamma || (mode != 1 && mode != 2) ||
        (p.K >> 3) > 64 * 8)
        return hipErrorInvalidValue;
    if (bits == 4)
        return swiglu ? launch_8rows_b<4, true>(p, mode, lds, st) : launch_8rows_b<4, false>(p, mode, lds, st);
    return swiglu ? launch_8rows_b<8, true>(p, mode, lds, st) : launch_8rows_b<8, false>(p, mode, lds, st);
}

}  // namespace qlin
