// Host-side mirror of the reference's npu::{Backend, Linear, QuantMatrix}
// (src/npu.rs:112-118, 230-260, 310-661, 999-1071) over the C ABI in qlinear.h.
//
// Same names, argument meaning and error behaviour as the Rust surface, so an
// engine written against that surface switches by swapping the type:
//   Backend::create(options, domain)     <- Backend::new(&ModelOptions, domain_id)
//   Backend::load(QuantMatrix)           <- Backend::load(QuantMatrix, Option<Reload>)
//   Backend::prepare / retain_workspaces / weight_bytes / tune_operations / stats
//   Linear::k / n / run / run_swiglu
// Errors are thrown as npu::Error with the reference's messages (anyhow's ensure!).
// A Backend is used from one host thread (the reference's is Rc<RefCell<..>>, !Send).
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

struct qlin_weights;
struct qlin_workspace;

namespace npu {

struct Error : std::runtime_error {
    int rc;
    explicit Error(const std::string& what, int code = 0) : std::runtime_error(what), rc(code) {}
};

// The fields of ModelOptions (src/model.rs:35-50) that reach the linear path.
struct ModelOptions {
    size_t chunk = 128;   // ubatch rows, 1..256 (src/npu.rs:52-55)
    int device = 0;       // HIP device of this backend (the reference's NPU domain)
    bool tune = false;         // heuristic variant choice, no search (the reference's `tune`)
    bool tune_search = false;  // prepare() times the kernel variants of every live linear (src/npu.rs:728-940)
    std::string tune_cache;    // variant table file: read by create(), written after a search (src/npu.rs:665-680)
};

// src/npu.rs:112-118: codes int8 [K, N] K-major (codes[k*N + n]), scales f32 [N].
struct QuantMatrix {
    uint32_t bits = 0;
    size_t k = 0, n = 0;
    std::vector<int8_t> codes;
    std::vector<float> scales;
};

// src/npu.rs:152-162: rows 1..=128 -> next power of two; 129..=256 -> multiple of 64.
size_t bucket(size_t rows);

class Linear;

class Backend {
public:
    // src/npu.rs:310-366 (options checked like configure_cpu, src/npu.rs:46-55)
    static Backend create(const ModelOptions& options, uint32_t domain_id = 0);
    // src/npu.rs:368-484: validates bits/dims/lengths, copies the codes to HBM, and
    // prepares the one-row workspace.  The host codes are released on return.
    Linear load(QuantMatrix matrix);
    // src/npu.rs:595-615: workspaces for bucket(rows) of every loaded geometry; with
    // options.tune_search, also the variant search (qlin_tune) for bucket(rows) of every live
    // linear not searched yet (plain and, where N % 64 == 0, SwiGLU), saved to
    // options.tune_cache when set.
    void prepare(size_t rows);
    // src/npu.rs:616-623: drops workspaces whose bucket is not in `rows`.
    void retain_workspaces(const std::vector<size_t>& rows);
    uint64_t weight_bytes() const;
    size_t tune_operations() const;  // variant searches run (src/npu.rs:627)
    std::string stats() const;       // JSON, src/npu.rs:631-661

    struct Inner;
    std::shared_ptr<Inner> inner;
};

class Linear {
public:
    size_t k() const;
    size_t n() const;
    // src/npu.rs:1006-1008,1025-1071: input f32 [rows, K], output f32 [rows, N], host memory.
    void run(const float* input, size_t input_len, float* output, size_t output_len, size_t rows) const;
    // src/npu.rs:1009-1024: fused SiLU(gate) * up into output [rows, N/2]; false when the
    // shape cannot be fused (N % 64 != 0), leaving the caller to run() + its own SwiGLU.
    bool run_swiglu(const float* input, size_t input_len, float* output, size_t output_len, size_t rows) const;
    // Asynchronous device-pointer run on `stream` (a hipStream_t), any row count up to the
    // bucket workspace; a_dtype / c_dtype are QLIN_F32 or QLIN_F16.
    void run_device(const void* A, int a_dtype, int64_t lda, void* C, int c_dtype, int64_t ldc, size_t rows,
                    uint32_t flags, void* stream) const;

    struct State;
    std::shared_ptr<State> state;
};

// src/model/checkpoint.rs:392-423: modules joined along N in order (same bits and K).
QuantMatrix concatenate(std::vector<QuantMatrix> matrices);

// The quantized Projection of src/model/projection.rs:110-243: one Linear per run of
// consecutive same-bit modules (each run concatenated along N), outputs side by side in
// module order in rows of width() columns.
class Projection {
public:
    // src/model/projection.rs:141-188: modules in module order (e.g. q, k, v).
    static Projection load(Backend& backend, std::vector<QuantMatrix> modules);
    size_t width() const { return width_; }
    size_t parts() const { return parts_.size(); }
    size_t scratch_width() const;  // src/model/projection.rs:130-140
    // src/model/projection.rs:190-232: input f32 [rows, K]; output f32 [rows, width of the
    // suffix from part `first`]; scratch f32 [rows * scratch_width()] (unused at one row or
    // with one part).
    void run(const float* input, size_t input_len, float* output, size_t output_len, size_t rows,
             float* scratch, size_t scratch_len) const;
    void run_from(size_t first, const float* input, size_t input_len, float* output, size_t output_len, size_t rows,
                  float* scratch, size_t scratch_len) const;
    // src/model/projection.rs:233-243: fused only with a single part.
    bool run_swiglu(const float* input, size_t input_len, float* output, size_t output_len, size_t rows) const;
    // Device rows: every part writes its own columns of C [rows, ldc >= width()] directly
    // (no scratch copy); asynchronous on `stream`.
    void run_device(const void* A, int a_dtype, int64_t lda, void* C, int c_dtype, int64_t ldc, size_t rows,
                    void* stream) const;

private:
    std::vector<std::pair<Linear, size_t>> parts_;  // (linear, first output column)
    size_t width_ = 0;
};

}  // namespace npu
