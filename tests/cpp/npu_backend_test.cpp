// The reference's board tests of the quantized linear, ported to the HIP backend
// through the npu::Backend / npu::Linear mirror:
//   quantized_linear_padding_and_swiglu       src/npu.rs:1161-1224
//   narrow_w8_gdn_gates_match_integer_oracle  src/npu/narrow_projection.rs:3-68
// plus the mixed-bit Projection (src/model/projection.rs:110-243) and concatenate
// (src/model/checkpoint.rs:392-423) of the mirror.
// Inputs are the tests' own closed forms; the checker is the CPU oracle
// (oracle/qlin_oracle.c) at the tests' own tolerances, plus bit-equality of the
// f32 outputs (both sides do the same singly-rounded f32 operations).
//
//   npu_backend_test cpu   -- host-side logic only (no GPU)
//   npu_backend_test gpu   -- the ported board tests on the GPU
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <functional>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/qlinear.h"
#include "../../oracle/qlin_oracle.h"
#include "../../open_rknpu2_lm_infer_amd/csrc/npu.hpp"

static int failures = 0;
#define EXPECT(cond, ...)                                  \
    do {                                                   \
        if (!(cond)) {                                     \
            std::printf("FAIL %s:%d: ", __FILE__, __LINE__); \
            std::printf(__VA_ARGS__);                      \
            std::printf("\n");                             \
            ++failures;                                    \
        }                                                  \
    } while (0)

// src/npu.rs:1097-1121
static std::vector<float> reference_oracle(const npu::QuantMatrix& m, const std::vector<float>& input, size_t rows) {
    std::vector<int8_t> q(rows * m.k);
    std::vector<float> s(rows), out(rows * m.n);
    std::vector<int32_t> acc(rows * m.n);
    oracle_quantize(input.data(), rows, m.k, m.k, ORACLE_ROUND_AWAY, q.data(), m.k, s.data());
    oracle_gemm_i32_kn(q.data(), m.k, rows, m.k, m.codes.data(), m.n, acc.data());
    oracle_dequant(acc.data(), rows, m.n, s.data(), m.scales.data(), out.data());
    return out;
}

// src/npu.rs:1125-1130
static void compare(const float* actual, const float* expected, size_t count, float tol, const char* what) {
    for (size_t i = 0; i < count; ++i) {
        const float a = actual[i], e = expected[i];
        if (!(std::isfinite(a) && std::fabs(a - e) <= tol * std::max(std::fabs(e), 1.0f))) {
            EXPECT(false, "%s element %zu: actual=%g expected=%g", what, i, a, e);
            return;
        }
    }
}

static void expect_error(const char* msg, const std::function<void()>& fn) {
    try {
        fn();
        EXPECT(false, "expected error '%s'", msg);
    } catch (const npu::Error& e) {
        EXPECT(std::string(e.what()).find(msg) != std::string::npos, "got '%s' expected '%s'", e.what(), msg);
    }
}

static int cpu_tests() {
    // bucket(): src/npu.rs:152-162
    const size_t in[] = {1, 2, 3, 5, 9, 17, 32, 33, 65, 127, 128, 129, 191, 192, 193, 255, 256};
    const size_t out[] = {1, 2, 4, 8, 16, 32, 32, 64, 128, 128, 128, 192, 192, 192, 256, 256, 256};
    for (size_t i = 0; i < sizeof(in) / sizeof(in[0]); ++i)
        EXPECT(npu::bucket(in[i]) == out[i], "bucket(%zu) = %zu", in[i], npu::bucket(in[i]));
    expect_error("linear batch must be within 1..256", [] { npu::bucket(0); });
    expect_error("linear batch must be within 1..256", [] { npu::bucket(257); });
    npu::ModelOptions opt;
    opt.chunk = 300;
    expect_error("ubatch-size must be within 1..256", [&] { npu::Backend::create(opt, 0); });
    opt.chunk = 64;
    auto backend = npu::Backend::create(opt, 0);
    // src/npu.rs:369-383: validated before any device work
    expect_error("linear weights must use 4 or 8 bits", [&] {
        backend.load(npu::QuantMatrix{3, 4, 4, std::vector<int8_t>(16), std::vector<float>(4, 1.0f)});
    });
    expect_error("invalid linear dimensions", [&] {
        backend.load(npu::QuantMatrix{8, 0, 4, std::vector<int8_t>(), std::vector<float>(4, 1.0f)});
    });
    expect_error("linear weight shape mismatch", [&] {
        backend.load(npu::QuantMatrix{8, 4, 4, std::vector<int8_t>(15), std::vector<float>(4, 1.0f)});
    });
    expect_error("linear weight shape mismatch", [&] {
        backend.load(npu::QuantMatrix{4, 4, 4, std::vector<int8_t>(16), std::vector<float>(3, 1.0f)});
    });
    EXPECT(backend.tune_operations() == 0, "tune operations");
    // concatenate (src/model/checkpoint.rs:392-423): K-major rows side by side, scales in order
    {
        npu::QuantMatrix a{8, 2, 2, {1, 2, 3, 4}, {0.5f, 0.25f}}, b{8, 2, 1, {9, 8}, {2.0f}};
        const npu::QuantMatrix c = npu::concatenate({a, b});
        const std::vector<int8_t> codes{1, 2, 9, 3, 4, 8};
        const std::vector<float> scales{0.5f, 0.25f, 2.0f};
        EXPECT(c.bits == 8 && c.k == 2 && c.n == 3 && c.codes == codes && c.scales == scales, "concatenate");
        expect_error("fused projections require identical bit widths and K", [&] {
            npu::concatenate({a, npu::QuantMatrix{4, 2, 1, {1, 2}, {1.0f}}});
        });
        expect_error("empty fused projection", [] { npu::concatenate({}); });
    }
    return failures;
}

// Projection of q (W4), k and v (W8): two parts (the W4 run, then k and v fused along N),
// outputs side by side; each module's columns equal the oracle of that module alone.
static void projection_tests(npu::Backend& backend) {
    const size_t K = 256, nq = 96, nk = 32, nv = 32;
    auto module = [&](uint32_t bits, size_t n, int salt) {
        npu::QuantMatrix m;
        m.bits = bits;
        m.k = K;
        m.n = n;
        const int lo = bits == 4 ? -8 : -127, span = bits == 4 ? 16 : 255;
        for (size_t i = 0; i < K * n; ++i) m.codes.push_back((int8_t)((long)(i * 29 + salt * 7 + i / n) % span + lo));
        for (size_t i = 0; i < n; ++i) m.scales.push_back(0.003f + (float)((i + salt) % 13) * 0.0007f);
        return m;
    };
    const std::vector<npu::QuantMatrix> mods{module(4, nq, 1), module(8, nk, 2), module(8, nv, 3)};
    npu::Projection proj = npu::Projection::load(backend, mods);
    EXPECT(proj.parts() == 2 && proj.width() == nq + nk + nv, "projection parts %zu width %zu", proj.parts(), proj.width());
    EXPECT(proj.scratch_width() == nq, "scratch width %zu", proj.scratch_width());
    for (size_t rows : {1u, 3u}) {
        std::vector<float> input(rows * K);
        for (size_t i = 0; i < input.size(); ++i) input[i] = (float)((i * 31 + 7) % 113) / 37.0f - 1.5f;
        std::vector<float> out(rows * proj.width()), scratch(rows * proj.scratch_width());
        proj.run(input.data(), input.size(), out.data(), out.size(), rows, scratch.data(), scratch.size());
        size_t col = 0;
        for (const npu::QuantMatrix& m : mods) {
            const std::vector<float> ref = reference_oracle(m, input, rows);
            for (size_t r = 0; r < rows; ++r)
                EXPECT(std::memcmp(out.data() + r * proj.width() + col, ref.data() + r * m.n, m.n * sizeof(float)) == 0,
                       "projection rows %zu: columns %zu.. differ from the module alone", rows, col);
            col += m.n;
        }
        // run_from(1): the k, v suffix only (src/model/projection.rs:198-232)
        std::vector<float> kv(rows * (nk + nv));
        proj.run_from(1, input.data(), input.size(), kv.data(), kv.size(), rows, scratch.data(), scratch.size());
        for (size_t r = 0; r < rows; ++r)
            EXPECT(std::memcmp(kv.data() + r * (nk + nv), out.data() + r * proj.width() + nq, (nk + nv) * sizeof(float)) == 0,
                   "run_from(1) rows %zu", rows);
        std::vector<float> mid(rows * proj.width() / 2);
        EXPECT(!proj.run_swiglu(input.data(), input.size(), mid.data(), mid.size(), rows), "two parts fused a SwiGLU");
        expect_error("projection suffix shape mismatch", [&] {
            proj.run_from(1, input.data(), input.size(), kv.data(), kv.size() - 1, rows, scratch.data(), scratch.size());
        });
        expect_error("invalid projection suffix", [&] {
            proj.run_from(2, input.data(), input.size(), kv.data(), kv.size(), rows, scratch.data(), scratch.size());
        });
    }
}

static npu::QuantMatrix padding_matrix(uint32_t bits) {
    npu::QuantMatrix m;
    m.bits = bits;
    m.k = m.n = 256;
    for (long i = 0; i < 256 * 256; ++i)  // src/npu.rs:1176-1182
        m.codes.push_back((int8_t)((i * 13 + i / 256 * 7) % (bits == 4 ? 16 : 255) - (bits == 4 ? 8 : 127)));
    for (int n = 0; n < 256; ++n) m.scales.push_back(0.002f + (float)(n % 11) * 0.0001f);
    return m;
}

static int gpu_tests() {
    npu::ModelOptions options;
    options.chunk = 256;
    options.tune = true;
    auto backend = npu::Backend::create(options, 15);
    std::vector<float> input;
    for (long i = 0; i < 256 * 256; ++i) input.push_back((float)((i * 17 + i / 256 * 3) % 127) / 63.0f - 1.0f);
    const size_t rows_list[] = {1, 2, 3, 5, 9, 17, 32, 33, 65, 127, 128, 129, 191, 192, 193, 255, 256};
    for (uint32_t bits : {4u, 8u}) {
        npu::QuantMatrix matrix = padding_matrix(bits);
        const std::vector<float> reference = reference_oracle(matrix, input, 256);
        npu::Linear linear = backend.load(matrix);
        for (size_t rows : rows_list) {
            std::vector<float> output(rows * 256);
            linear.run(input.data(), input.size(), output.data(), output.size(), rows);
            compare(output.data(), reference.data(), rows * 256, 2e-5f, "run");
            EXPECT(std::memcmp(output.data(), reference.data(), rows * 256 * sizeof(float)) == 0,
                   "W%u rows %zu: f32 outputs not bit-identical to the oracle", bits, rows);
            if (bits == 4 && rows >= 32) {
                std::vector<float> middle(rows * 128), expected(rows * 128);
                EXPECT(linear.run_swiglu(input.data(), input.size(), middle.data(), middle.size(), rows),
                       "run_swiglu declined");
                for (size_t r = 0; r < rows; ++r)
                    for (size_t n = 0; n < 128; ++n) {
                        const float gate = reference[r * 256 + n];
                        expected[r * 128 + n] = gate / (1.0f + std::exp(-gate)) * reference[r * 256 + 128 + n];
                    }
                compare(middle.data(), expected.data(), rows * 128, 3e-5f, "run_swiglu");
            }
        }
    }
    projection_tests(backend);
    // src/npu.rs:1213-1222: workspaces are bounded by retain_workspaces, no tuning at run time
    backend.retain_workspaces({1, 64});
    EXPECT(backend.stats().find("\"workspace_count\": 1") != std::string::npos ||
               backend.stats().find("\"workspace_count\": 2") != std::string::npos,
           "workspace count: %s", backend.stats().c_str());
    const size_t lookups = backend.tune_operations();
    backend.prepare(3);
    backend.retain_workspaces({1, 64});
    backend.prepare(3);
    EXPECT(backend.tune_operations() == lookups, "tune operations changed");
    EXPECT(backend.stats().find("\"tune_calls\": 0") != std::string::npos, "tune calls");
    EXPECT(backend.stats().find("\"weight_reload_calls\": 0") != std::string::npos, "reloads");

    // src/npu/narrow_projection.rs:3-68
    npu::ModelOptions narrow_opt;
    narrow_opt.chunk = 32;
    auto narrow = npu::Backend::create(narrow_opt, 15);
    const size_t k = 2560;
    for (size_t n : {32u, 64u}) {
        npu::QuantMatrix m;
        m.bits = 8;
        m.k = k;
        m.n = n;
        for (size_t i = 0; i < k * n; ++i) m.codes.push_back((int8_t)((i * 13 + i / n * 7) % 255 - 127));
        for (size_t i = 0; i < n; ++i) m.scales.push_back(0.001f + (float)(i % 11) * 0.0001f);
        const npu::QuantMatrix kept = m;
        npu::Linear linear = narrow.load(m);
        for (size_t rows : {1u, 2u, 3u, 5u, 7u}) {
            narrow.prepare(rows);
            std::vector<float> in(rows * k), outv(rows * n);
            for (size_t i = 0; i < rows * k; ++i) in[i] = (float)((i * 17 + i / k * 3) % 127) / 63.0f - 1.0f;
            linear.run(in.data(), in.size(), outv.data(), outv.size(), rows);
            for (size_t r = 0; r < rows; ++r) {
                float maxabs = 0.0f;
                for (size_t i = 0; i < k; ++i) maxabs = std::fmax(maxabs, std::fabs(in[r * k + i]));
                const float scale = maxabs / 127.0f, recip = 1.0f / scale;
                std::vector<int> quant(k);
                for (size_t i = 0; i < k; ++i) {
                    float v = std::round(in[r * k + i] * recip);
                    quant[i] = (int)std::fmin(std::fmax(v, -127.0f), 127.0f);
                }
                for (size_t col = 0; col < n; ++col) {
                    int sum = 0;
                    for (size_t i = 0; i < k; ++i) sum += quant[i] * kept.codes[i * n + col];
                    const float expected = ((float)sum * scale) * kept.scales[col];
                    const float actual = outv[r * n + col];
                    EXPECT(std::fabs(actual - expected) <= 2e-6f * std::max(std::fabs(expected), 1.0f),
                           "N=%zu M=%zu: %g != %g", n, rows, actual, expected);
                }
            }
        }
    }
    // variant search (the reference's tune_search + tune cache, src/npu.rs:595-615,665-680)
    {
        const char* tmp = std::getenv("TMPDIR");
        const std::string cache = std::string(tmp && *tmp ? tmp : "/tmp") + "/qlin_npu_tune_cache.txt";
        std::remove(cache.c_str());
        qlin_tune_clear();
        npu::ModelOptions topt;
        topt.chunk = 64;
        topt.tune_search = true;
        topt.tune_cache = cache;
        auto tb = npu::Backend::create(topt, 15);
        npu::QuantMatrix matrix = padding_matrix(4);
        std::vector<float> input;
        for (long i = 0; i < 256 * 256; ++i) input.push_back((float)((i * 17 + i / 256 * 3) % 127) / 63.0f - 1.0f);
        const std::vector<float> reference = reference_oracle(matrix, input, 256);
        npu::Linear linear = tb.load(matrix);
        tb.prepare(1);
        tb.prepare(64);
        EXPECT(tb.tune_operations() == 4, "tune operations %zu (plain + SwiGLU at two buckets)", tb.tune_operations());
        tb.prepare(64);
        EXPECT(tb.tune_operations() == 4, "a searched bucket was searched again");
        std::FILE* f = std::fopen(cache.c_str(), "r");
        EXPECT(f != nullptr, "tune cache not written");
        if (f) std::fclose(f);
        for (size_t rows : {1u, 64u}) {
            std::vector<float> output(rows * 256);
            linear.run(input.data(), input.size(), output.data(), output.size(), rows);
            EXPECT(std::memcmp(output.data(), reference.data(), rows * 256 * sizeof(float)) == 0,
                   "tuned rows %zu: f32 outputs not bit-identical to the oracle", rows);
        }
        qlin_tune_clear();
        npu::ModelOptions lopt;
        lopt.tune_cache = cache;
        auto lb = npu::Backend::create(lopt, 15);  // reads the cache
        EXPECT(qlin_tune_count() >= 2, "tune cache not loaded (%d entries)", qlin_tune_count());
        EXPECT(lb.tune_operations() == 0, "loading the cache ran a search");
        qlin_tune_clear();
        std::remove(cache.c_str());
    }
    return failures;
}

int main(int argc, char** argv) {
    const std::string mode = argc > 1 ? argv[1] : "cpu";
    try {
        if (mode == "cpu") cpu_tests();
        else if (mode == "gpu") gpu_tests();
        else {
            std::printf("usage: %s cpu|gpu\n", argv[0]);
            return 2;
        }
    } catch (const std::exception& e) {
        std::printf("FAIL exception: %s\n", e.what());
        return 1;
    }
    std::printf("%s %s tests: %d failure(s)\n", failures ? "FAIL" : "PASS", mode.c_str(), failures);
    return failures ? 1 : 0;
}
