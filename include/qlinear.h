/*
 * qlinear.h - C ABI of the MI355X (gfx950) W4A8 / W8A8 quantized linear.
 *
 * Symmetric per-output-channel int4/int8 weights times dynamic per-token int8
 * activations, as used by every Q/K/V/O and gate/up/down projection of the
 * HC-Zhou/open_rknpu2_lm_infer engine.  Each entry point below names the native
 * library call of the reference it replaces; the reference reaches those through
 * bindgen (build.rs:44-67) and calls them from src/npu.rs.
 *
 * Arithmetic (identical to the reference oracle, src/npu.rs:1097-1121):
 *   s[m]    = absmax_k |A[m,k]| == 0 ? 1 : max(absmax/127, FLT_MIN)
 *   q[m,k]  = clamp(round(A[m,k] * (1/s[m])), -127, 127)   round = half away from zero
 *   acc     = sum_k q[m,k] * codes[k,n]                      exact int32
 *   C[m,n]  = (float(acc) * s[m]) * scales[n]
 *   SwiGLU: C[m,j] = (g/(1+exp(-g))) * u, g = col j, u = col j + N/2 (src/npu.rs:1202-1208)
 *
 * Conventions: functions return 0 (QLIN_OK) or a negative QLIN_ERR_* code;
 * qlin_strerror() names it.  Handles are opaque and owned by the caller, who
 * frees them with the paired *_free.  Host buffers passed to *_create are copied.
 * Entry points taking `stream` are asynchronous and stream-ordered (stream is a
 * hipStream_t, NULL = default stream); pointers passed to them are device
 * pointers.
 *
 * A workspace holds shared scratch (quantized rows, per-token scales, the sticky error
 * word, split-K partial sums and self-resetting split-K counters): it serves one stream
 * at a time.  Two streams running on one workspace at once race on all of it, and a
 * split-K counter left mid-count corrupts later GEMMs; give each stream its own
 * workspace.  The output C of a run must not overlap its input A (the decode GEMV reads
 * A while other workgroups already store C); qlin_run_residual may update R in place.
 */
#ifndef QLINEAR_H
#define QLINEAR_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- return codes (src/npu.rs:138-151 maps them through rk_npu_strerror) ---- */
#define QLIN_OK 0
#define QLIN_ERR_PARAM (-1)       /* invalid argument, like RK_NPU_ERR_PARAM */
#define QLIN_ERR_NOMEM (-2)       /* device or pinned host allocation failed */
#define QLIN_ERR_DEVICE (-3)      /* a HIP runtime call failed */
#define QLIN_ERR_NONFINITE (-4)   /* activation row holds Inf/NaN (the native library rejects it) */
#define QLIN_ERR_UNSUPPORTED (-5) /* shape not supported by this entry point */
#define QLIN_ERR_NODEVICE (-6)    /* no gfx950 device visible */

/* ---- element types of activations / outputs ---- */
#define QLIN_F32 0
#define QLIN_F16 1

/* ---- flags ---- */
#define QLIN_ROUND_HALF_EVEN 0x1u /* q rounding half to even; default is half away (Rust f32::round) */
#define QLIN_NORM_SEQUENTIAL 0x2u /* RMSNorm sum order of src/ops/norm.rs:23-48 instead of the
                                     16-accumulator order of src/model/cpu.rs:11-41 */
#define QLIN_SWIGLU 0x4u          /* fused SiLU(gate)*up epilogue, output [M, N/2] */
#define QLIN_NO_FUSED_QUANT 0x8u  /* decode: quantize in a separate launch instead of in the GEMV */
#define QLIN_RESIDUAL 0x10u       /* chain stage: add a residual row after the linear (see qlin_chain_stage) */

typedef struct qlin_weights qlin_weights;
typedef struct qlin_workspace qlin_workspace;

/* Geometry of one linear (reference: rk_npu_i4_weight_config {K, N, k_tile} and
 * rk_npu_matmul_weight_config, src/npu.rs:392-396,432-436). */
typedef struct qlin_weight_config {
    int32_t bits; /* 4 or 8 */
    int32_t K;    /* in-features, 1..2^30 */
    int32_t N;    /* out-features, 1..2^30 */
} qlin_weight_config;

/* Reference: rk_npu_w4a8_weight_info / rk_npu_i4_weights_memory_query (src/npu.rs:408-423). */
typedef struct qlin_weight_info {
    int32_t bits, K, N;
    int32_t K_padded;      /* K rounded up to 256 (zero codes in the pad) */
    int32_t N_padded;      /* N rounded up to 64 (zero codes and scales in the pad) */
    int32_t device;        /* HIP device ordinal holding the weights */
    uint64_t device_bytes; /* packed codes + scales resident in HBM */
} qlin_weight_info;

/* Reference: rk_npu_w4a8_memory_info_ex / rk_npu_matmul_workspace_requirements (src/npu.rs:955-986). */
typedef struct qlin_workspace_info {
    int32_t max_rows;
    int32_t reserved;
    uint64_t device_bytes;      /* scratch: quantized rows, scales, split-K partials, counters */
    uint64_t pinned_host_bytes; /* staging for the host-buffer entry points */
} qlin_workspace_info;

/* Reference: rk_npu_strerror (src/npu.rs:138-144). */
const char* qlin_strerror(int rc);

/* Device and build facts used for roofline reporting: CU count, peak shader clock
 * (kHz), HBM bus width (bits), memory clock (kHz), and gfx arch number (950). */
typedef struct qlin_device_info {
    int32_t device, cu_count, arch, reserved;
    int64_t sclk_khz, mclk_khz, bus_width_bits, hbm_bytes;
} qlin_device_info;
int qlin_device_query(int32_t device, qlin_device_info* out);

/* ---- weights ----
 * Replaces rk_npu_w4a8_weights_create (W4, src/npu.rs:397-405) and
 * rk_npu_f32i8f32_weights_create (W8, src/npu.rs:439-447).  codes are the
 * reference QuantMatrix layout: int8 [K, N] K-major, codes[k*N + n], values in
 * [-8, 7] for bits = 4 and [-127, 127] for bits = 8; scales f32 [N], positive.
 * Both are host pointers, copied into the current HIP device's HBM as
 * [N, Kp/2] nibble-packed codes (each 32-bit word: byte b holds k = 8w+b low and
 * 8w+b+4 high, the order the kernels unpack into) or [N, Kp] int8.  Out-of-range
 * codes or non-positive / non-finite scales return QLIN_ERR_PARAM. */
int qlin_weights_create(const qlin_weight_config* config, const int8_t* codes_kn,
                        const float* scales, qlin_weights** out);

/* Same, from packed codes (host pointers): packed is [N, K/2] bytes with the low
 * nibble holding the even k (bits = 4, K even; reordered into the device nibble
 * order on the device) or [N, K] int8 (bits = 8).  Used by the benchmark. */
int qlin_weights_create_packed(const qlin_weight_config* config, const void* packed_nk,
                               const float* scales, qlin_weights** out);

/* Same as qlin_weights_create_packed, but packed_nk and scales are DEVICE pointers
 * (copied device-to-device on `stream`); no host round trip for large stacks. */
int qlin_weights_create_packed_device(const qlin_weight_config* config, const void* packed_nk,
                                      const float* scales, void* stream, qlin_weights** out);

/* compressed-tensors storage straight to the device layout.  Replaces QuantLoader::load's
 * unpack + [K,N] transpose (src/model/checkpoint.rs:320-390) and concatenate along N
 * (src/model/checkpoint.rs:392-423) for the engine's fused projections.
 * QLIN_PACK_QUANTIZED: data[i] is the I32 tensor weight_packed [part_n[i], ceil(K*bits/32)], fields
 *   LSB-first, code = field - 2^(bits-1) (checkpoint.rs:352-371).
 * QLIN_INT_QUANTIZED (bits = 8 only): data[i] is the I8 tensor weight [part_n[i], K] (checkpoint.rs:372-378).
 * The parts are stacked along N in order (q, k, v or gate, up); config->N = sum of part_n.  data and
 * scales are host pointers (e.g. the mmap'd tensors); scales[i] is f32 [part_n[i]], positive and finite.
 * Like the reference loader, code values are not range-checked (a W8 field 0 decodes to -128). */
#define QLIN_PACK_QUANTIZED 0
#define QLIN_INT_QUANTIZED 1
int qlin_weights_create_compressed(const qlin_weight_config* config, int32_t format, int32_t n_parts,
                                   const int32_t* part_n, const void* const* data,
                                   const float* const* scales, qlin_weights** out);

/* Replaces rk_npu_w4a8_weights_free / rk_npu_f32i8f32_weights_free (src/npu.rs:411,452). */
void qlin_weights_free(qlin_weights* weights);

/* Replaces rk_npu_w4a8_weights_query + rk_npu_i4_weights_memory_query (src/npu.rs:407-423). */
int qlin_weights_query(const qlin_weights* weights, qlin_weight_info* out);

/* ---- workspace ----
 * Replaces rk_npu_w4a8_workspace_create_ex / rk_npu_matmul_workspace_create
 * (src/npu.rs:964-991).  A workspace serves any weights with K <= max_k and
 * N <= max_n, at 1..max_rows rows.  The reference fixes M per workspace (its
 * bucket(), src/npu.rs:152-162); here any rows <= max_rows run. */
int qlin_workspace_create(int32_t max_rows, int32_t max_k, int32_t max_n, qlin_workspace** out);
void qlin_workspace_free(qlin_workspace* ws);
int qlin_workspace_query(const qlin_workspace* ws, qlin_workspace_info* out);

/* Sticky error word of asynchronous runs on this workspace: returns QLIN_OK or
 * QLIN_ERR_NONFINITE if any activation row seen since the last clear held Inf/NaN.
 * Synchronizes the workspace's last stream.  clear != 0 resets it. */
int qlin_workspace_status(qlin_workspace* ws, int32_t clear);

/* ---- host-buffer runs: the drop-in for the reference's synchronous calls ----
 * Replaces rk_npu_w4a8_run_f32 (src/npu.rs:1047-1049) and rk_npu_f32i8f32_run_dynamic
 * (src/npu.rs:1052-1061): A f32 [rows, K] and C f32 [rows, N] are host pointers;
 * the call returns after C is written.  Non-finite input returns QLIN_ERR_NONFINITE. */
int qlin_run_f32(qlin_workspace* ws, const qlin_weights* weights, int32_t rows, const float* A,
                 float* C);

/* Replaces rk_npu_w4a8_run_swiglu_f32 (src/npu.rs:1044-1046): C is [rows, N/2].
 * Any even N (the reference fuses only for N % 64 == 0, src/npu.rs:1011, and otherwise
 * falls back to its CPU SwiGLU; here every even N is fused).  Odd N returns
 * QLIN_ERR_UNSUPPORTED. */
int qlin_run_swiglu_f32(qlin_workspace* ws, const qlin_weights* weights, int32_t rows,
                        const float* A, float* C);

/* ---- device runs (MI355X-native, asynchronous) ----
 * A: device [rows, lda] of a_dtype; C: device [rows, ldc] of c_dtype, N columns
 * (N/2 with QLIN_SWIGLU).  flags: QLIN_ROUND_HALF_EVEN, QLIN_SWIGLU,
 * QLIN_NO_FUSED_QUANT.  Non-finite input sets the workspace's sticky error. */
int qlin_run(qlin_workspace* ws, const qlin_weights* weights, int32_t rows, const void* A,
             int32_t a_dtype, int64_t lda, void* C, int32_t c_dtype, int64_t ldc, uint32_t flags,
             void* stream);

/* RMSNorm -> quantize -> linear in one call (src/model/dense.rs:416-430,486-505:
 * Cpu::norm then Projection::run).  gamma: device f32 [K]; eps > 0.  The norm
 * output stays in f32 registers and is never rounded to fp16 before quantization,
 * as in the reference where norm_row writes f32.  flags as qlin_run plus
 * QLIN_NORM_SEQUENTIAL. */
int qlin_run_rmsnorm(qlin_workspace* ws, const qlin_weights* weights, int32_t rows,
                     const void* A, int32_t a_dtype, int64_t lda, const float* gamma, float eps,
                     void* C, int32_t c_dtype, int64_t ldc, uint32_t flags, void* stream);

/* Linear, then the decoder's residual update in the same epilogue (src/model/dense.rs:478-489
 * and 528-537: Projection::run, Cpu::scale(projected, residual_multiplier), Cpu::add(hidden,
 * projected)):  C[m,n] = R[m,n] + y[m,n] * multiplier, where y is what qlin_run computes, every
 * operation an f32 rounding (the add in the reference's order hidden + projected, add_chunk in
 * src/model/cpu.rs:68-85), then stored as c_dtype.  R: device [rows, ldr] of r_dtype (f32 or
 * fp16); R may equal C with ldr == ldc (the in-place hidden += of the reference).  Not with
 * QLIN_SWIGLU (QLIN_ERR_PARAM).  No counterpart in the native library: the reference runs the
 * scale and add on the CPU after rk_npu_w4a8_run_f32 / rk_npu_f32i8f32_run_dynamic return. */
int qlin_run_residual(qlin_workspace* ws, const qlin_weights* weights, int32_t rows, const void* A,
                      int32_t a_dtype, int64_t lda, const void* R, int32_t r_dtype, int64_t ldr,
                      float multiplier, void* C, int32_t c_dtype, int64_t ldc, uint32_t flags, void* stream);

/* qlin_run_rmsnorm (gamma != NULL) or qlin_run (gamma == NULL) without a workspace: no
 * counterpart in the reference.  For callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): it calls no hipMalloc,
 * hipFree or allocating routine.  Its scratch (quantized rows, per-token scales, split-K
 * partial sums and counters) is a 32.05 MiB static device array that each GPU the library
 * runs on holds until the process ends; every call on a GPU shares that GPU's array, so
 * calls that overlap on one GPU race (run them on one stream).  The first call on a device
 * also clears that array's counters with a kernel on `stream`.  Limits: rows <= 4096 and
 * rows * K_padded <= 16 MiB, else QLIN_ERR_UNSUPPORTED.  err (device uint32, may be NULL)
 * gets bit 0 set when an activation row holds Inf/NaN.  Otherwise as qlin_run_rmsnorm. */
int qlin_run_noalloc(const qlin_weights* weights, int32_t rows, const void* A, int32_t a_dtype, int64_t lda,
                     const float* gamma, float eps, void* C, int32_t c_dtype, int64_t ldc, uint32_t flags,
                     uint32_t* err, void* stream);

/* ---- stage entry points (parity checks and composition) ----
 * Per-token quantization alone (the library's scan + quantize,
 * QWEN3_W4A8_PIPELINE_REVIEW_20261020.md:26-27).  q: device int8 [rows, ldq], the
 * K..ldq-1 tail zero-filled; s: device f32 [rows].  gamma != NULL applies RMSNorm
 * first.  err (device uint32, may be NULL) gets bit 0 set on non-finite input. */
int qlin_quantize(int32_t rows, int32_t K, const void* A, int32_t a_dtype, int64_t lda,
                  const float* gamma, float eps, int8_t* q, int64_t ldq, float* s, uint32_t* err,
                  uint32_t flags, void* stream);

/* Exact int32 acc[rows, ldacc] = q[rows, :K] x codes over the whole N (the library's
 * integer GEMM + reduce, PIPELINE_REVIEW:28-30).  q: device int8 [rows, ldq] with
 * ldq >= K_padded and zeros in [K, K_padded). */
int qlin_gemm_i32(qlin_workspace* ws, const qlin_weights* weights, int32_t rows, const int8_t* q,
                  int64_t ldq, int32_t* acc, int64_t ldacc, void* stream);

/* Linear from already-quantized rows: the epilogue applies (float(acc)*s[m])*scales[n]
 * (and SwiGLU with QLIN_SWIGLU).  Lets a producer kernel hand over q and s directly. */
int qlin_run_quantized(qlin_workspace* ws, const qlin_weights* weights, int32_t rows,
                       const int8_t* q, int64_t ldq, const float* s, void* C, int32_t c_dtype,
                       int64_t ldc, uint32_t flags, void* stream);

/* SiLU-gate on the unfused layout, on the device: Y[m, j] = SiLU(X[m, j]) * X[m, F + j],
 * j < F, rows of X holding the gate block then the up block ([rows, 2F], stride ldx >= 2F)
 * and Y [rows, F] (stride ldy >= F), f32 or fp16 each.  Replaces the reference's CPU
 * fallback Cpu::swiglu / swiglu_block (src/model/cpu.rs:119-152,327-351), used when the
 * fused SwiGLU declines (src/model/dense.rs:508-522).  Same SiLU as the fused epilogue. */
int qlin_swiglu(int32_t rows, int32_t F, const void* X, int32_t x_dtype, int64_t ldx, void* Y, int32_t y_dtype,
                int64_t ldy, void* stream);

/* ---- launch plan (debug tap) ----
 * Describes the launches qlin_run (gamma NULL) or qlin_run_rmsnorm would make for these
 * arguments, without launching anything: A and gamma are only inspected for alignment.
 * No counterpart in the reference, whose library reports its strategy through
 * rk_npu_w4a8_query / backend stats (src/npu.rs:631-661). */
#define QLIN_PATH_GEMV_FUSED 0 /* one GEMV launch that quantizes (and normalizes) its rows itself */
#define QLIN_PATH_GEMV 1       /* a quantize launch, then the GEMV on the quantized rows */
#define QLIN_PATH_GEMM 2       /* a quantize launch, then the MFMA GEMM */
typedef struct qlin_plan {
    int32_t path;       /* QLIN_PATH_* */
    int32_t launches;   /* kernel launches of the call */
    int32_t waves;      /* waves per workgroup of the GEMV / GEMM */
    int32_t item_width; /* GEMV: output channels per item */
    int32_t items;      /* GEMV items, or GEMM output tiles */
    int32_t grid;       /* workgroups of the GEMV / GEMM launch */
    int32_t splits;     /* GEMM: k splits per tile */
    int32_t tile_m;     /* GEMM: rows per tile */
    int32_t tile_n;     /* GEMM: output channels per tile */
    int32_t reserved[3];
} qlin_plan;
int qlin_run_plan(const qlin_workspace* ws, const qlin_weights* weights, int32_t rows, const void* A, int64_t lda,
                  const float* gamma, uint32_t flags, qlin_plan* out);

/* ---- kernel-variant selection ----
 * Replaces the NPU strategy search and its on-disk cache (src/npu.rs:595-996, driven by
 * src/cli/tune.rs:10-59).  qlin_tune times, on `stream`, the variants of the path a run of
 * `rows` rows takes (decode GEMV: 4, 8 or 16 waves per channel group; GEMM: the 16x16x64
 * kernel and each tile configuration of the 32x32x32 kernel, each with 1..8 k splits),
 * checks that they all produce the same output, and records the fastest for the key (bits,
 * K, N, rows bucket, path, QLIN_SWIGLU); later runs with that key use it.  The table is
 * process-wide (all devices; tune on the device that runs).  QLIN_GEMV_WAVES,
 * QLIN_GEMM_SPLITS, QLIN_GEMM_KERNEL and QLIN_GEMM_CFG in the environment still take
 * precedence.  flags: 0 or QLIN_SWIGLU.  qlin_tune_load returns the number of entries read
 * (or an error code); the file is text, one entry per line: bits K N rows_bucket path swiglu
 * variant, the variant being the GEMV's waves (4, 8, 16) or, for a GEMM (path 2), splits +
 * 100 * kernel with splits 1..64 and kernel 0 (the planner's pick), 1 (16x16x64) or 2 + c
 * (32x32x32 in tile configuration c = 0..3; c = 3 for W4 only). */
int qlin_tune(qlin_workspace* ws, const qlin_weights* weights, int32_t rows, uint32_t flags, int32_t reps,
              void* stream);
int qlin_tune_count(void);
void qlin_tune_clear(void);
int qlin_tune_save(const char* path);
int qlin_tune_load(const char* path);

/* ---- decode chain: several linears in one launch (1..4 rows, fp16 activations) ----
 * Replaces the per-projection calls of the decode step, src/model/dense.rs:398-540
 * (Cpu::norm, then Projection::run / run_swiglu for qkv, o, gate_up, down, layer
 * after layer).  Each stage computes exactly what qlin_run_rmsnorm (gamma != NULL)
 * or qlin_run (gamma == NULL) computes for its input, with fp16 in and out: the
 * chain output equals those calls made one after another.  Attention and RoPE are not
 * part of it; a stage reads an earlier stage's output (or the chain input) from a column
 * offset, so a caller can route e.g. the q columns of qkv into o.  A stage with
 * QLIN_RESIDUAL computes what qlin_run_residual computes, with R = an earlier stage's
 * output or the chain input (the decoder's hidden += o(...) and hidden += down(...)). */
typedef struct qlin_chain qlin_chain;

typedef struct qlin_chain_stage {
    const qlin_weights* weights;
    uint32_t flags;       /* QLIN_SWIGLU, QLIN_ROUND_HALF_EVEN, QLIN_NORM_SEQUENTIAL */
    const float* gamma;   /* device RMSNorm weights [K], 16-byte aligned, or NULL */
    float eps;
    int32_t input;        /* -1: the chain input; j >= 0: the output of stage j (j < this) */
    int32_t input_offset; /* first column taken from that output (multiple of 8) */
    /* with QLIN_RESIDUAL in flags (not with QLIN_SWIGLU): */
    int32_t residual;     /* -1: the chain input; j >= 0: the output of stage j (j < this) */
    int32_t residual_offset;   /* first column of the residual rows (multiple of 8) */
    float residual_multiplier; /* the linear's output is scaled by this before the add */
} qlin_chain_stage;

/* Checks the stages (K of each stage = the columns it reads; K % 8 == 0) and
 * allocates the intermediate fp16 buffers for max_rows <= 4 rows.  The weights must
 * outlive the chain.  A CU holds up to 80 steps of 128 weight bytes of a stage in
 * registers at once (64 for 2..4 rows); a larger share (a W8 SiLU-gate stage K=2560,
 * N=19456 takes 120 on 256 CUs) streams in several rounds within the stage. */
int qlin_chain_create(const qlin_chain_stage* stages, int32_t n_stages, int32_t max_rows,
                      qlin_chain** out);
void qlin_chain_free(qlin_chain* chain);

/* x: device fp16 [rows, ldx] (K of stage 0 columns, 16-byte aligned rows); y: device
 * fp16 [rows, ldy] gets the last stage's output.  Asynchronous on `stream`. */
int qlin_chain_run(qlin_chain* chain, int32_t rows, const void* x, int64_t ldx, void* y, int64_t ldy,
                   void* stream);

/* Polls of the previous stage's completion flags (each followed by a short sleep)
 * before a workgroup gives up waiting and sets the QLIN_ERR_DEVICE bit of the chain's
 * error word.  Default 262144 (~0.3 s; QLIN_CHAIN_SPIN_LIMIT at chain creation overrides
 * it); 0 gives up at once, which tests use to exercise the failure path without any
 * kernel hanging. */
int qlin_chain_set_wait_limit(qlin_chain* chain, int32_t polls);

/* Device pointer and row stride (elements) of stage `stage`'s fp16 output from the
 * last run (the last stage writes y instead). */
int qlin_chain_stage_output(const qlin_chain* chain, int32_t stage, void** ptr, int64_t* ld);

/* Error word of the runs since the last clear: QLIN_OK, QLIN_ERR_NONFINITE (an input
 * row held Inf/NaN) or QLIN_ERR_DEVICE (a stage wait gave up: the grid was not fully
 * resident, e.g. other work occupied the GPU; that run's outputs are invalid).
 * Synchronizes the last run's stream.  clear != 0 resets the word.  A run that gave up
 * leaves no state behind: the next run is correct without any reset. */
int qlin_chain_status(qlin_chain* chain, int32_t clear);

#ifdef __cplusplus
}
#endif
#endif /* QLINEAR_H */
