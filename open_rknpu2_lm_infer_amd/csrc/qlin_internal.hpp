// Internal declarations shared by the HIP translation units of libqlinear.
//
// Device layout of the weights (see qlin_capi.hip for the repack):
//   W4: [Np, Kp/2] bytes of two's-complement 4-bit codes; each 32-bit word w of a row
//       holds k = 8w .. 8w+7, byte b with k = 8w+b in its low nibble and k = 8w+b+4 in
//       its high nibble (so the kernels' nibble unpack yields k order);
//   W8: [Np, Kp] int8;
//   scales: f32 [Np], zero in the padded rows.
// Kp = roundup(K, 256), Np = roundup(N, 64); pad codes are zero so they add nothing.
//
// Quantized activations: int8 [M, ldq] with ldq >= Kp and zeros in [K, Kp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qlin {

constexpr int kKAlign = 256;  // Kp alignment (one GEMV wave step of W4 spans 256 k)
constexpr int kNAlign = 64;   // Np alignment
constexpr int kMaxK = 131072; // int32 accumulators cannot overflow below this K (W4 codes x16)
constexpr int kGemvMaxRows = 16;      // rows of one matrix-core block of the decode GEMV
constexpr int kGemvMaxRowsWide = 32;  // rows the GEMV takes quantized: two blocks of 16
// Rows a fused GEMV prologue quantizes: up to 4 in every instance, 5..8 in the 8-row
// instances (512-thread workgroups, one activation group per thread per row, no RMSNorm).
constexpr int kFusedMaxRows = 8;
constexpr int kFusedRowsWide = 4;

typedef int v4i __attribute__((ext_vector_type(4)));

enum : uint32_t {
    kFlagRne = 0x1u,
    kFlagNormSeq = 0x2u,
    kFlagSwiglu = 0x4u,
    kFlagNoFusedQuant = 0x8u,
};

struct QuantParams {
    const void* A;
    int64_t lda;
    int a_f16;
    int K;
    int64_t ldq;     // q row stride; columns [K, ldq) are zero-filled
    int8_t* q;
    float* s;
    uint32_t* err;   // bit 0 set on non-finite input (may be null)
    const float* gamma;  // RMSNorm weight, null = no norm
    float eps;
    uint32_t flags;
};

struct GemvParams {
    const uint8_t* W;     // device layout
    const float* wscale;  // [Np]
    int64_t wrow;         // bytes per weight row
    int K, Kp, N, Np, M;
    // activations: either raw rows quantized in the prologue (A != null) ...
    const void* A;
    int64_t lda;
    int a_f16;
    const float* gamma;
    float eps;
    // ... or rows already quantized
    const int8_t* q;
    int64_t ldq;
    const float* s;
    void* C;
    int64_t ldc;
    int c_kind;         // 0 f32, 1 f16, 2 int32 acc (stage entry point)
    uint32_t flags;
    uint32_t* err;      // bit 0 set on non-finite input (fused quantization)
    int grid;           // workgroups (each takes items b, b + grid, ...); 0: one per item
    int iw;             // output channels per item, 1..16 (the MFMA tile's 16 rows; rows past
                        // iw re-read the item's last row and are not stored)
    // residual update of the epilogue (R != null): C = R + y * rmult, f32 roundings
    const void* R;
    int64_t ldr;
    int r_f16;
    float rmult;
};

// Items of a GEMV launch: output channels (N, or N/2 with SwiGLU) in groups of iw.
__host__ __device__ __forceinline__ int gemv_out_cols(const GemvParams& p) {
    return (p.flags & kFlagSwiglu) ? (p.N >> 1) : p.N;
}
__host__ __device__ __forceinline__ int gemv_items(const GemvParams& p) {
    return (gemv_out_cols(p) + p.iw - 1) / p.iw;
}

struct GemmParams {
    const uint8_t* W;
    const float* wscale;
    int64_t wrow;
    int K, Kp, N, Np, M;
    const int8_t* q;
    int64_t ldq;
    const float* s;       // null: write raw int32 acc (stage entry point)
    void* C;
    int64_t ldc;
    int c_kind;           // 0 f32, 1 f16, 2 int32 acc
    uint32_t flags;
    int m_tiles, n_tiles, splits, ktiles_per_split;
    int group_m;          // m tiles per group of the tile order
    int32_t* part;        // split-K partials, tile-major
    uint32_t* counters;   // [m_tiles * n_tiles], zero at rest
    int deep;             // 1: the most LDS stages (grid of at most one workgroup per CU)
    int wn;               // waves along N: 4 (2 x 4 waves, two per SIMD at one workgroup per CU) or 2
    // residual update of the epilogue (R != null): C = R + y * rmult, f32 roundings
    const void* R;
    int64_t ldr;
    int r_f16;
    float rmult;
};

// Residual update of an f32 epilogue value y at (m, c): R[m, c] + y * mult, each an f32
// rounding, the add in the reference's order hidden + projected (src/model/dense.rs:486-489,
// src/model/cpu.rs:68-85).  x * 1 is exact, so a multiplier of one equals the reference's
// skipped scale.
__device__ __forceinline__ float residual_add(const void* R, int64_t ldr, int r_f16, float mult, int m, int c, float y) {
    const float p = y * mult;
    const float h = r_f16 ? (float)reinterpret_cast<const _Float16*>(R)[(int64_t)m * ldr + c]
                          : reinterpret_cast<const float*>(R)[(int64_t)m * ldr + c];
    return h + p;
}

// Launchers (return hipError_t of the launch).
hipError_t launch_quant(const QuantParams& p, int rows, hipStream_t stream);
hipError_t launch_gemv(const GemvParams& p, int bits, int waves, hipStream_t stream);
int gemv_pick_waves(int groups, int steps);
int gemv_item_width(int cols, int cus);  // iw in 8..16 spreading cols / iw items best over the CUs
bool gemv_can_fuse(int M, int K, int waves, bool norm);
size_t gemv_lds_bytes_for(int M, int Kp, int K, int waves, bool fused, bool norm, int items);
hipError_t launch_gemm(const GemmParams& p, int bits, int bn, hipStream_t stream);
int gemm_tile_n(int bits, int N);          // channels of B per workgroup tile
int gemm_regs_per_thread(int bn);          // int32 accumulators per thread of one tile
// Tile of the 32x32x32 GEMM: tokens x weight rows, threads, int32 accumulators per thread.
struct GemmTileCfg {
    int bm, bn, threads, regs;
};
GemmTileCfg gemm32_tile(int bits, int cfg);
hipError_t launch_gemm32(const GemmParams& p, int bits, int cfg, hipStream_t stream);
hipError_t launch_swiglu(int rows, int F, const void* X, int x_f16, int64_t ldx, void* Y, int y_f16, int64_t ldy,
                         hipStream_t stream);
hipError_t launch_pack_w4(const int8_t* codes_nk, int N, int K, int Np, int Kp, uint8_t* out,
                          hipStream_t stream);

// ---- device helpers -------------------------------------------------------

__device__ __forceinline__ float qscale_from_absmax(float absmax) {
    // src/npu.rs:1102-1105
    if (absmax == 0.0f) return 1.0f;
    float s = absmax / 127.0f;  // IEEE division (correctly rounded build flag)
    return s < 1.17549435e-38f ? 1.17549435e-38f : s;
}

__device__ __forceinline__ int quant_one(float x, float inv, bool rne) {
    // src/npu.rs:1109: (x * (1.0 / scale)).round().clamp(-127.0, 127.0) as i32
    float v = x * inv;
    float r = rne ? __builtin_rintf(v) : __builtin_roundf(v);
    if (r != r) return 0;  // NaN -> 0, Rust's saturating cast
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    return (int)r;
}

// quant_one for a value known finite with |x * inv| < 256, the case of every element
// of a finite row (|x * inv| <= 127 * (1 + a few ulp)).  Round half away from zero is
// x + copysign(0.5 - 2^-25, x) truncated by the conversion: equal to Rust's f32::round
// for every float of magnitude below 256 (checked exhaustively, all 2^31 patterns of
// that range, against floor(|x| + 0.5) in double precision).  The clamp to +-127 is
// then a no-op and NaN cannot occur.
template <bool RNE>
__device__ __forceinline__ int quant_finite(float x, float inv) {
    const float v = x * inv;
    if constexpr (RNE) return (int)__builtin_rintf(v);
    else return (int)(v + __builtin_copysignf(0.49999997f, v));
}

// Largest |x| of eight fp16 values (one 16-byte group) as an fp16 bit pattern.
// Non-negative fp16 values order like their bit patterns, and Inf / NaN (>= 0x7c00)
// above every finite value, so one unsigned max also flags a non-finite group.
__device__ __forceinline__ uint32_t absmax_bits_f16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    u16x2 m = __builtin_bit_cast(u16x2, a & 0x7fff7fffu);
    m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, b & 0x7fff7fffu));
    m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, c & 0x7fff7fffu));
    m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, d & 0x7fff7fffu));
    return m.x > m.y ? m.x : m.y;
}
__device__ __forceinline__ float f32_of_f16_bits(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}
// Largest |x| of eight fp16 values (one 16-byte group) as the reference folds them
// (f32::max over |x|, src/npu.rs:1101-1106: NaN ignored, Inf kept), as an fp16 bit pattern,
// and whether any of them is Inf or NaN.  Each sign-masked pattern h is taken as the signed
// 16-bit value h + 0x3ff: finite values and Inf keep their order at 0x3ff..0x7fff, and NaN
// patterns (h > 0x7c00) wrap below zero, so one signed max passes over them.  A group of
// eight NaN gives 0.
__device__ __forceinline__ uint32_t absmax_bits_f16x8_ref(uint4 r, bool& nonfinite) {
    typedef short i16x2 __attribute__((ext_vector_type(2)));
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    const u16x2 off = {0x3ff, 0x3ff};
    const i16x2 b0 = __builtin_bit_cast(i16x2, __builtin_bit_cast(u16x2, r.x & 0x7fff7fffu) + off);
    const i16x2 b1 = __builtin_bit_cast(i16x2, __builtin_bit_cast(u16x2, r.y & 0x7fff7fffu) + off);
    const i16x2 b2 = __builtin_bit_cast(i16x2, __builtin_bit_cast(u16x2, r.z & 0x7fff7fffu) + off);
    const i16x2 b3 = __builtin_bit_cast(i16x2, __builtin_bit_cast(u16x2, r.w & 0x7fff7fffu) + off);
    const i16x2 m = __builtin_elementwise_max(__builtin_elementwise_max(b0, b1), __builtin_elementwise_max(b2, b3));
    const int top = m.x > m.y ? m.x : m.y;
    // a NaN wrapped below zero (sign bit set); an Inf is the top value 0x7c00 + 0x3ff
    const uint32_t signs = (__builtin_bit_cast(uint32_t, b0) | __builtin_bit_cast(uint32_t, b1) |
                            __builtin_bit_cast(uint32_t, b2) | __builtin_bit_cast(uint32_t, b3)) & 0x80008000u;
    nonfinite = signs != 0 || top == 0x7fff;
    return top < 0x3ff ? 0u : (uint32_t)(top - 0x3ff);
}

// SiLU(g) * u (src/npu.rs:1202-1208: g / (1 + e^-g) * u) with the hardware exp2 and
// reciprocal: e^-g = exp2(-g * log2 e), then g * rcp(1 + e^-g).  v_exp_f32 and v_rcp_f32
// are accurate to about 1 ulp, so the result stays within a few ulp of the IEEE
// expression, far inside the SwiGLU tolerance; this is 4 instructions where expf and the
// correctly rounded divide took about 30.  For g < -88, e^-g is +inf and the result is
// -0 * u, as in the IEEE form.
__device__ __forceinline__ float silu_gate(float g, float u) {
    const float e = __builtin_amdgcn_exp2f(-g * 1.44269504f);
    return (g * __builtin_amdgcn_rcpf(1.0f + e)) * u;
}

// fp16 store of an f32 result, rounded twice as specified (to f32 by the producing
// operation, then to fp16 to nearest even).  The empty asm pins x in a VGPR as a
// rounded f32 value; without it the backend folds the producing multiply into
// v_fma_mixlo_f16, which rounds the exact product once, straight to fp16.
__device__ __forceinline__ _Float16 f16_of_f32(float x) {
    __asm__ volatile("" : "+v"(x));
    return (_Float16)x;
}

// Waits until every memory operation this wave issued has completed (vmcnt,
// expcnt and lgkmcnt all zero).  Used before a workgroup barrier that precedes a
// split-K counter bump: partials are written with device-coherent (sc1) stores or
// L2 atomics, so completion is all the ordering needed, and the L2 writeback +
// invalidate of an agent-scope fence is avoided.
__device__ __forceinline__ void wait_all_memory() { __builtin_amdgcn_s_waitcnt(0); }

// Workgroup barrier that orders LDS accesses only: the caller's LDS operations
// complete before it, but unlike __syncthreads it does not wait for the caller's
// outstanding global loads (weight blocks already in flight for later steps).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
// A workgroup barrier that waits for no memory counter: orders instruction issue only.
__device__ __forceinline__ void issue_barrier() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ void store_coherent(int32_t* p, int32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t load_coherent(const int32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ int wave_or(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v |= __shfl_xor(v, o, 64);
    return v;
}

}  // namespace qlin
