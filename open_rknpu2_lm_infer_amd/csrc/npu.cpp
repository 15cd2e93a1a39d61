// Host-side mirror of the reference's npu::{Backend, Linear} over the C ABI.
// See npu.hpp for the correspondence with src/npu.rs.
#include "npu.hpp"

#include <algorithm>
#include <cstdio>
#include <sstream>

#include "../../include/qlinear.h"

namespace npu {

namespace {

void check(int rc, const char* name) {
    if (rc != QLIN_OK) throw Error(std::string(name) + ": " + qlin_strerror(rc) + " (" + std::to_string(rc) + ")", rc);
}

void ensure(bool ok, const char* msg) {
    if (!ok) throw Error(msg, QLIN_ERR_PARAM);
}

}  // namespace

size_t bucket(size_t rows) {
    ensure(rows >= 1 && rows <= 256, "linear batch must be within 1..256");
    if (rows <= 128) {
        size_t p = 1;
        while (p < rows) p <<= 1;
        return p;
    }
    return (rows + 63) / 64 * 64;
}

struct Weights {
    qlin_weights* raw = nullptr;
    ~Weights() { qlin_weights_free(raw); }
};

struct Workspace {
    qlin_workspace* raw = nullptr;
    int max_k = 0, max_n = 0;
    ~Workspace() { qlin_workspace_free(raw); }
};

struct Backend::Inner {
    ModelOptions options;
    uint32_t domain_id = 0;
    std::vector<std::weak_ptr<Weights>> linears;  // live weights, for the variant search
    std::vector<std::pair<const Weights*, size_t>> searched;  // (weights, bucket) already searched
    size_t tune_calls = 0;
    std::map<size_t, std::unique_ptr<Workspace>> work;  // bucket rows -> workspace
    int max_k = 0, max_n = 0;                           // largest loaded geometry
    size_t loaded_w4 = 0, loaded_w8 = 0, geometries = 0;
    uint64_t weight_bytes = 0;

    Workspace* get_work(size_t m) {
        auto it = work.find(m);
        if (it != work.end() && it->second->max_k >= max_k && it->second->max_n >= max_n) return it->second.get();
        auto ws = std::make_unique<Workspace>();
        ws->max_k = max_k;
        ws->max_n = max_n;
        check(qlin_workspace_create((int32_t)m, max_k, max_n, &ws->raw), "create workspace");
        Workspace* out = ws.get();
        work[m] = std::move(ws);
        return out;
    }
};

struct Linear::State {
    std::shared_ptr<Backend::Inner> owner;  // a Linear keeps its Backend alive (src/npu.rs:255-260)
    std::shared_ptr<Weights> weights;
    uint32_t bits = 0;
    size_t k = 0, n = 0;
};

Backend Backend::create(const ModelOptions& options, uint32_t domain_id) {
    ensure(options.chunk >= 1 && options.chunk <= 256, "ubatch-size must be within 1..256");
    ensure(options.device >= 0, "invalid device");
    Backend b;
    b.inner = std::make_shared<Inner>();
    b.inner->options = options;
    b.inner->domain_id = domain_id;
    if (!options.tune_cache.empty()) {
        // src/npu.rs:665-680: a missing cache file is not an error
        if (std::FILE* f = std::fopen(options.tune_cache.c_str(), "r")) {
            std::fclose(f);
            const int n = qlin_tune_load(options.tune_cache.c_str());
            check(n < 0 ? n : QLIN_OK, "load tune cache");
        }
    }
    return b;
}

Linear Backend::load(QuantMatrix matrix) {
    // src/npu.rs:369-383
    ensure(matrix.bits == 4 || matrix.bits == 8, "linear weights must use 4 or 8 bits");
    ensure(matrix.k > 0 && matrix.n > 0 && matrix.k <= INT32_MAX && matrix.n <= INT32_MAX,
           "invalid linear dimensions");
    ensure(matrix.codes.size() == matrix.k * matrix.n && matrix.scales.size() == matrix.n,
           "linear weight shape mismatch");
    Linear lin;
    lin.state = std::make_shared<Linear::State>();
    lin.state->owner = inner;
    lin.state->bits = matrix.bits;
    lin.state->k = matrix.k;
    lin.state->n = matrix.n;
    lin.state->weights = std::make_shared<Weights>();
    qlin_weight_config cfg{(int32_t)matrix.bits, (int32_t)matrix.k, (int32_t)matrix.n};
    check(qlin_weights_create(&cfg, matrix.codes.data(), matrix.scales.data(), &lin.state->weights->raw),
          matrix.bits == 4 ? "W4 weights" : "W8 weights");
    qlin_weight_info info{};
    check(qlin_weights_query(lin.state->weights->raw, &info), "weight query");
    inner->weight_bytes += info.device_bytes;
    (matrix.bits == 4 ? inner->loaded_w4 : inner->loaded_w8) += 1;
    inner->geometries += 1;
    inner->max_k = std::max(inner->max_k, (int)matrix.k);
    inner->max_n = std::max(inner->max_n, (int)matrix.n);
    inner->get_work(1);
    inner->linears.push_back(lin.state->weights);
    matrix.codes.clear();  // the device copy is the only one kept (src/npu.rs:459-477)
    matrix.codes.shrink_to_fit();
    return lin;
}

void Backend::prepare(size_t rows) {
    const size_t m = bucket(rows);
    Workspace* ws = inner->get_work(m);
    if (!inner->options.tune_search) return;
    size_t before = inner->tune_calls;
    for (auto& weak : inner->linears) {
        auto w = weak.lock();
        if (!w) continue;
        const std::pair<const Weights*, size_t> key{w.get(), m};
        if (std::find(inner->searched.begin(), inner->searched.end(), key) != inner->searched.end()) continue;
        qlin_weight_info info{};
        check(qlin_weights_query(w->raw, &info), "weight query");
        check(qlin_tune(ws->raw, w->raw, (int32_t)m, 0, 20, nullptr), "tune");
        ++inner->tune_calls;
        if (info.N % 64 == 0) {
            check(qlin_tune(ws->raw, w->raw, (int32_t)m, QLIN_SWIGLU, 20, nullptr), "tune");
            ++inner->tune_calls;
        }
        inner->searched.push_back(key);
    }
    if (inner->tune_calls != before && !inner->options.tune_cache.empty())
        check(qlin_tune_save(inner->options.tune_cache.c_str()), "save tune cache");
}

void Backend::retain_workspaces(const std::vector<size_t>& rows) {
    std::vector<size_t> keep;
    for (size_t r : rows) keep.push_back(bucket(r));
    for (auto it = inner->work.begin(); it != inner->work.end();) {
        if (std::find(keep.begin(), keep.end(), it->first) == keep.end())
            it = inner->work.erase(it);
        else
            ++it;
    }
}

uint64_t Backend::weight_bytes() const { return inner->weight_bytes; }

size_t Backend::tune_operations() const { return inner->tune_calls; }

std::string Backend::stats() const {
    uint64_t ws_bytes = 0;
    for (auto& kv : inner->work) {
        qlin_workspace_info info{};
        if (qlin_workspace_query(kv.second->raw, &info) == QLIN_OK) ws_bytes += info.device_bytes;
    }
    std::ostringstream o;
    o << "{\"backend\": \"qlinear-gfx950\", \"loaded_w4\": " << inner->loaded_w4
      << ", \"loaded_w8\": " << inner->loaded_w8 << ", \"weight_payload_bytes\": " << inner->weight_bytes
      << ", \"workspace_payload_bytes\": " << ws_bytes << ", \"workspace_count\": " << inner->work.size()
      << ", \"tune_calls\": " << inner->tune_calls << ", \"tune_entries\": " << qlin_tune_count()
      << ", \"strategy_fallbacks\": 0, \"strategy_fallback_calls\": 0, \"weight_reload_calls\": 0"
      << ", \"weight_geometries\": " << inner->geometries << ", \"device\": " << inner->options.device
      << ", \"domain_id\": " << inner->domain_id << "}";
    return o.str();
}

size_t Linear::k() const { return state->k; }
size_t Linear::n() const { return state->n; }

void Linear::run(const float* input, size_t input_len, float* output, size_t output_len, size_t rows) const {
    const size_t m = bucket(rows);
    ensure(input_len >= rows * k() && output_len >= rows * n(), "linear input/output shape mismatch");
    Workspace* ws = state->owner->get_work(m);
    check(qlin_run_f32(ws->raw, state->weights->raw, (int32_t)rows, input, output),
          state->bits == 4 ? "W4 run" : "W8 run");
}

bool Linear::run_swiglu(const float* input, size_t input_len, float* output, size_t output_len, size_t rows) const {
    if (n() % 64 != 0) return false;
    const size_t m = bucket(rows);
    ensure(input_len >= rows * k() && output_len >= rows * (n() / 2), "linear input/output shape mismatch");
    Workspace* ws = state->owner->get_work(m);
    check(qlin_run_swiglu_f32(ws->raw, state->weights->raw, (int32_t)rows, input, output),
          state->bits == 4 ? "W4 SwiGLU run" : "W8 SwiGLU run");
    return true;
}

void Linear::run_device(const void* A, int a_dtype, int64_t lda, void* C, int c_dtype, int64_t ldc, size_t rows,
                        uint32_t flags, void* stream) const {
    ensure(rows >= 1 && rows <= INT32_MAX, "linear batch must be positive");
    Workspace* ws = state->owner->get_work(std::max<size_t>(rows, 1));
    check(qlin_run(ws->raw, state->weights->raw, (int32_t)rows, A, a_dtype, lda, C, c_dtype, ldc, flags, stream),
          "device run");
}

QuantMatrix concatenate(std::vector<QuantMatrix> matrices) {
    ensure(!matrices.empty(), "empty fused projection");
    if (matrices.size() == 1) return std::move(matrices[0]);
    const uint32_t bits = matrices[0].bits;
    const size_t k = matrices[0].k;
    for (const QuantMatrix& m : matrices)
        ensure(m.bits == bits && m.k == k, "fused projections require identical bit widths and K");
    QuantMatrix out;
    out.bits = bits;
    out.k = k;
    for (const QuantMatrix& m : matrices) {
        out.n += m.n;
        out.scales.insert(out.scales.end(), m.scales.begin(), m.scales.end());
    }
    out.codes.resize(k * out.n);
    for (size_t ki = 0; ki < k; ++ki) {  // K-major rows: each row is the modules' rows side by side
        size_t offset = 0;
        for (const QuantMatrix& m : matrices) {
            std::copy(m.codes.begin() + ki * m.n, m.codes.begin() + (ki + 1) * m.n, out.codes.begin() + ki * out.n + offset);
            offset += m.n;
        }
    }
    return out;
}

Projection Projection::load(Backend& backend, std::vector<QuantMatrix> modules) {
    Projection result;
    size_t first = 0;
    while (first < modules.size()) {
        const uint32_t bits = modules[first].bits;
        size_t last = first + 1;
        while (last < modules.size() && modules[last].bits == bits) ++last;
        std::vector<QuantMatrix> group;
        for (size_t i = first; i < last; ++i) group.push_back(std::move(modules[i]));
        Linear linear = backend.load(concatenate(std::move(group)));
        const size_t n = linear.n();
        result.parts_.emplace_back(std::move(linear), result.width_);
        result.width_ += n;
        first = last;
    }
    return result;
}

size_t Projection::scratch_width() const {
    if (parts_.size() <= 1) return 0;
    size_t w = 0;
    for (const auto& p : parts_) w = std::max(w, p.first.n());
    return w;
}

void Projection::run(const float* input, size_t input_len, float* output, size_t output_len, size_t rows,
                     float* scratch, size_t scratch_len) const {
    run_from(0, input, input_len, output, output_len, rows, scratch, scratch_len);
}

void Projection::run_from(size_t first, const float* input, size_t input_len, float* output, size_t output_len,
                          size_t rows, float* scratch, size_t scratch_len) const {
    ensure(first < parts_.size(), "invalid projection suffix");
    const size_t base = parts_[first].second;
    const size_t width = width_ - base;
    ensure(output_len == rows * width, "projection suffix shape mismatch");
    if (parts_.size() - first == 1) {
        parts_[first].first.run(input, input_len, output, output_len, rows);
        return;
    }
    for (size_t i = first; i < parts_.size(); ++i) {
        const Linear& linear = parts_[i].first;
        const size_t offset = parts_[i].second - base, n = linear.n();
        if (rows == 1) {
            linear.run(input, input_len, output + offset, n, 1);
        } else {
            ensure(scratch && scratch_len >= rows * n, "projection scratch too small");
            linear.run(input, input_len, scratch, rows * n, rows);
            for (size_t r = 0; r < rows; ++r)
                std::copy(scratch + r * n, scratch + (r + 1) * n, output + r * width + offset);
        }
    }
}

bool Projection::run_swiglu(const float* input, size_t input_len, float* output, size_t output_len,
                            size_t rows) const {
    if (parts_.size() != 1) return false;
    return parts_[0].first.run_swiglu(input, input_len, output, output_len, rows);
}

void Projection::run_device(const void* A, int a_dtype, int64_t lda, void* C, int c_dtype, int64_t ldc, size_t rows,
                            void* stream) const {
    ensure(ldc >= (int64_t)width_, "projection output stride below its width");
    const size_t elem = c_dtype == QLIN_F16 ? 2 : 4;
    for (const auto& p : parts_)
        p.first.run_device(A, a_dtype, lda, static_cast<uint8_t*>(C) + p.second * elem, c_dtype, ldc, rows, 0, stream);
}

}  // namespace npu
