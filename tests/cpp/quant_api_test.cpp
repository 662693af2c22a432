// quant_api_test.cpp -- the C++ Quant API (include/cllm/core/quant.hpp, libcllm_quant.so)
// exercised the way the reference's tests/quant_test.cpp exercises its own: fixed weight
// patterns with d = 1, matmul_quant against a dequantize-and-dot reference, the bias
// difference, batch against row-by-row. The expected values come from the C oracle
// (oracle/cllm_oracle.h), linked here as the oracle only.
//
//   quant_api_test --cpu   checks that need no GPU: size tables, has_vec_dot, the fp16
//                          conversions, and every argument error the API raises before it
//                          touches a device (message text included)
//   quant_api_test         all of the above, then the GPU computations
//
// Exit status 0 when every check passed. Each check prints its name before it runs.
#include "cllm/core/quant.hpp"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "cllm_oracle.h"

using namespace cllm;

namespace {

int g_pass = 0, g_fail = 0;

void expect(bool ok, const char* what) {
    if (ok) {
        ++g_pass;
    } else {
        ++g_fail;
        std::printf("  FAIL %s\n", what);
    }
}

// The call must throw std::runtime_error whose what() equals msg.
template <class F>
void expect_throw(F&& f, const char* msg) {
    std::string got = "(no exception)";
    try {
        f();
    } catch (const std::runtime_error& e) {
        got = e.what();
    }
    if (got == msg) {
        ++g_pass;
    } else {
        ++g_fail;
        std::printf("  FAIL expected \"%s\", got \"%s\"\n", msg, got.c_str());
    }
}

struct TypeCase {
    const char* name;
    GgmlType type;
};
const TypeCase kKernelTypes[] = {{"Q4_0", GgmlType::Q4_0}, {"Q5_0", GgmlType::Q5_0},
                                 {"Q8_0", GgmlType::Q8_0}, {"Q4_K", GgmlType::Q4_K},
                                 {"Q5_K", GgmlType::Q5_K}, {"Q6_K", GgmlType::Q6_K}};

// Every block: fp16 1.0 in its first two bytes, then the small repeating byte pattern
// (k + block + row) % 7 (the fill tests/quant_test.cpp:245-256 of the reference uses).
std::vector<uint8_t> pattern_weights(GgmlType t, int in_dim, int out_dim) {
    const int bs = block_size(t);
    const size_t ts = type_size(t), row_bytes = (size_t)(in_dim / bs) * ts;
    std::vector<uint8_t> w(row_bytes * out_dim, 0);
    for (int j = 0; j < out_dim; ++j)
        for (int b = 0; b < in_dim / bs; ++b) {
            uint8_t* p = &w[j * row_bytes + b * ts];
            p[0] = 0x00;
            p[1] = 0x3C;
            for (size_t k = 2; k < ts; ++k) p[k] = (uint8_t)((k + b + j) % 7);
        }
    return w;
}

// Deterministic pseudo-random bytes (xorshift64*), for weights with varied scales.
std::vector<uint8_t> random_bytes(size_t n, uint64_t seed) {
    std::vector<uint8_t> v(n);
    uint64_t s = seed * 0x9E3779B97F4A7C15ull + 1;
    for (auto& b : v) {
        s ^= s >> 12;
        s ^= s << 25;
        s ^= s >> 27;
        b = (uint8_t)((s * 0x2545F4914F6CDD1Dull) >> 56);
    }
    return v;
}

// Random weights whose fp16 scale fields are set to small finite values, so no block holds
// an infinity or NaN scale.
std::vector<uint8_t> random_weights(GgmlType t, int in_dim, int out_dim, uint64_t seed) {
    const int bs = block_size(t);
    const size_t ts = type_size(t), nblk = (size_t)(in_dim / bs) * out_dim;
    std::vector<uint8_t> w = random_bytes(nblk * ts, seed);
    std::vector<uint8_t> sc = random_bytes(nblk * 4, seed + 77);
    for (size_t b = 0; b < nblk; ++b) {
        uint8_t* p = &w[b * ts];
        // fp16 in [2^-9, 2^-6): exponent field 6..8, random mantissa
        auto put = [&](size_t off, int i) {
            const uint16_t h = (uint16_t)(((6 + sc[4 * b + i] % 3) << 10) |
                                          ((sc[4 * b + i + 1] << 2) & 0x3FF));
            p[off] = (uint8_t)(h & 0xFF);
            p[off + 1] = (uint8_t)(h >> 8);
        };
        if (t == GgmlType::Q6_K) {
            put(208, 0);
        } else if (t == GgmlType::Q4_K || t == GgmlType::Q5_K || t == GgmlType::Q4_1 ||
                   t == GgmlType::Q5_1) {
            put(0, 0);
            put(2, 2);
        } else if (t == GgmlType::Q2_K) {
            put(80, 0);
            put(82, 2);
        } else if (t == GgmlType::Q3_K) {
            put(108, 0);
        } else if (t == GgmlType::F16) {
            // fp16 values of either sign with exponent field 6..13
            const uint16_t h = (uint16_t)(((sc[4 * b] & 1) << 15) | ((6 + sc[4 * b + 1] % 8) << 10) |
                                          ((sc[4 * b + 2] << 2) & 0x3FF));
            p[0] = (uint8_t)(h & 0xFF);
            p[1] = (uint8_t)(h >> 8);
        } else if (t == GgmlType::F32) {
            const float v = (float)((int)(sc[4 * b] | (sc[4 * b + 1] << 8)) - 32768) * (1.0f / 65536.0f);
            std::memcpy(p, &v, 4);
        } else {
            put(0, 0);
        }
    }
    return w;
}

std::vector<float> activations(int n_rows, int in_dim, int variant) {
    std::vector<float> x((size_t)n_rows * in_dim);
    for (int t = 0; t < n_rows; ++t)
        for (int i = 0; i < in_dim; ++i) {
            float v = (float)(((i + t + variant) % 5) - 2) * 0.5f;
            if (variant > 0) v += 0.01f * (float)((i * 37 + t * 11 + variant) % 23) - 0.11f;
            x[(size_t)t * in_dim + i] = v;
        }
    return x;
}

// Largest |gpu - expected| / max(|expected|, 2^-10 * A) over all outputs, A being the sum of
// the absolute per-block terms of that output (the oracle's fp64 evaluation).
double floored_rel_err(const std::vector<float>& got, const float* x, const uint8_t* w,
                       GgmlType t, const float* bias, int in_dim, int out_dim, int n_rows) {
    std::vector<double> exact((size_t)n_rows * out_dim), abs_sum(exact.size());
    if (oracle_matmul_quant_f64(x, w, (uint32_t)t, bias, in_dim, out_dim, n_rows, exact.data(),
                                abs_sum.data()) != ORACLE_OK)
        return INFINITY;
    double worst = 0;
    for (size_t i = 0; i < exact.size(); ++i) {
        const double den = std::fmax(std::fabs(exact[i]), std::ldexp(abs_sum[i], -10));
        const double e = den > 0 ? std::fabs((double)got[i] - exact[i]) / den
                                 : std::fabs((double)got[i]);
        worst = std::fmax(worst, e);
    }
    return worst;
}

// ---- checks that need no device -------------------------------------------------------

void test_sizes() {
    std::printf("[sizes]\n");
    struct Row {
        GgmlType t;
        int bs;
        size_t ts;
        bool dot;
    };
    const Row rows[] = {{GgmlType::F32, 1, 4, false},     {GgmlType::F16, 1, 2, false},
                        {GgmlType::Q4_0, 32, 18, true},   {GgmlType::Q4_1, 32, 20, false},
                        {GgmlType::Q5_0, 32, 22, true},   {GgmlType::Q5_1, 32, 24, false},
                        {GgmlType::Q8_0, 32, 34, true},   {GgmlType::Q8_1, 32, 36, false},
                        {GgmlType::Q2_K, 256, 84, false}, {GgmlType::Q3_K, 256, 110, false},
                        {GgmlType::Q4_K, 256, 144, true}, {GgmlType::Q5_K, 256, 176, true},
                        {GgmlType::Q6_K, 256, 210, true}};
    for (const Row& r : rows) {
        expect(block_size(r.t) == r.bs, "block_size");
        expect(type_size(r.t) == r.ts, "type_size");
        expect(has_vec_dot(r.t) == r.dot, "has_vec_dot");
        expect(block_size(r.t) == oracle_block_size((uint32_t)r.t), "block_size vs oracle");
        expect(type_size(r.t) == oracle_type_size((uint32_t)r.t), "type_size vs oracle");
    }
}

void test_half_conversions() {
    std::printf("[half_to_float / float_to_half]\n");
    int bad = 0;
    for (uint32_t h = 0; h < 0x10000; ++h) {
        const float f = half_to_float((uint16_t)h), g = oracle_half_to_float((uint16_t)h);
        if (std::memcmp(&f, &g, 4) != 0) ++bad;
        const bool nan = ((h >> 10) & 0x1F) == 0x1F && (h & 0x3FF);
        if (!nan && float_to_half(f) != h) ++bad;  // every finite half and inf round-trips
    }
    expect(bad == 0, "fp16 round trip over all 65536 encodings");
    expect(float_to_half(65536.0f) == 0x7C00, "overflow to infinity");
    expect(float_to_half(std::ldexp(1.0f, -24)) == 0x0001, "smallest subnormal");
    expect(float_to_half(std::ldexp(1.0f, -26)) == 0x0000, "below half the smallest subnormal");
    expect(float_to_half(1.0f + std::ldexp(1.0f, -11)) == 0x3C00, "normal results truncate");
}

void test_argument_errors() {
    std::printf("[argument errors]\n");
    std::vector<float> x(300, 1.0f), y(8, 0.0f);
    std::vector<uint8_t> w(4096, 0);
    expect_throw([&] { matmul_quant(x.data(), w.data(), GgmlType::Q4_K, nullptr, 255, 1, y.data()); },
                 "matmul_quant: in_dim not divisible by block size");
    expect_throw([&] {
        matmul_quant_batch(x.data(), w.data(), GgmlType::Q8_0, nullptr, 33, 1, 2, y.data());
    }, "matmul_quant_batch: in_dim not divisible by block size");
    // one row is delegated to matmul_quant, whose message it then carries
    expect_throw([&] {
        matmul_quant_batch(x.data(), w.data(), GgmlType::Q8_0, nullptr, 33, 1, 1, y.data());
    }, "matmul_quant: in_dim not divisible by block size");
    expect_throw([&] {
        QuantizedQ8_0 q;
        quantize_row_q8_0(x.data(), q, 40);
    }, "quantize_row_q8_0: n not divisible by 32");
    expect_throw([&] {
        QuantizedQ8_0 q;
        q.n = 32;
        q.qs.assign(32, 0);
        q.scales.assign(1, 1.0f);
        q.bsums.assign(1, 0);
        vec_dot_row(w.data(), GgmlType::Q4_1, q, 32);
    }, "vec_dot_row: no kernel for this type");
    // n_rows <= 0 returns without writing y
    std::vector<float> keep(8, 7.0f);
    matmul_quant_batch(x.data(), w.data(), GgmlType::Q4_K, nullptr, 256, 8, 0, keep.data());
    bool untouched = true;
    for (float v : keep) untouched &= (v == 7.0f);
    expect(untouched, "n_rows = 0 leaves y untouched");
}

// ---- device checks ---------------------------------------------------------------------

void test_quantize_bit_exact() {
    std::printf("[quantize_row_q8_0 bit-exact]\n");
    for (int variant = 0; variant < 4; ++variant) {
        const int n = 1024;
        std::vector<float> x = activations(1, n, variant);
        if (variant == 2)
            for (int i = 0; i < n; ++i) x[i] *= (i % 64 == 5) ? 1e4f : 1.0f;
        if (variant == 3)
            for (int i = 0; i < 32; ++i) x[i] = (float)(i - 16) * 1e-42f;  // subnormal block
        QuantizedQ8_0 q;
        quantize_row_q8_0(x.data(), q, n);
        std::vector<int8_t> qs(n);
        std::vector<float> sc(n / 32);
        std::vector<int32_t> bs(n / 32);
        oracle_quantize_row_q8_0(x.data(), n, qs.data(), sc.data(), bs.data());
        expect(q.n == n && q.qs == qs && q.bsums == bs &&
                   std::memcmp(q.scales.data(), sc.data(), sc.size() * 4) == 0,
               "qs, scales, bsums identical to the oracle");
    }
}

void test_vec_dot_row() {
    std::printf("[vec_dot_row]\n");
    for (const TypeCase& c : kKernelTypes) {
        const int n = 512;
        std::vector<uint8_t> w = random_weights(c.type, n, 1, 11);
        std::vector<float> x = activations(1, n, 3);
        QuantizedQ8_0 q;
        quantize_row_q8_0(x.data(), q, n);
        const float got = vec_dot_row(w.data(), c.type, q, n);
        const double err = floored_rel_err({got}, x.data(), w.data(), c.type, nullptr, n, 1, 1);
        if (err > 1e-4) std::printf("  %s rel err %.3g\n", c.name, err);
        expect(err <= 1e-4, c.name);
    }
}

void test_matmul_quant_patterns() {
    for (const TypeCase& c : kKernelTypes) {
        std::printf("[matmul_quant %s]\n", c.name);
        const int bs = block_size(c.type);
        const int in_dim = bs <= 32 ? 64 : 256, out_dim = 40;
        const size_t row_bytes = (size_t)(in_dim / bs) * type_size(c.type);
        std::vector<uint8_t> w = pattern_weights(c.type, in_dim, out_dim);
        std::vector<float> x = activations(1, in_dim, 0);
        std::vector<float> y(out_dim);
        matmul_quant(x.data(), w.data(), c.type, nullptr, in_dim, out_dim, y.data());
        // the reference test's own bar: dequantized float weights . unquantized x, within
        // max(1e-2, 3%) for 32-element blocks and max(3e-2, 6%) for super-blocks
        int mism = 0;
        std::vector<float> row(in_dim);
        for (int j = 0; j < out_dim; ++j) {
            oracle_dequantize(&w[j * row_bytes], row.data(), (uint32_t)c.type, in_dim);
            double ref = 0;
            for (int i = 0; i < in_dim; ++i) ref += (double)x[i] * row[i];
            const double tol = std::fmax(bs <= 32 ? 1e-2 : 3e-2, (bs <= 32 ? 0.03 : 0.06) * std::fabs(ref));
            mism += std::fabs(ref - y[j]) > tol;
        }
        expect(mism == 0, "within the dequantize-and-dot tolerance");
        // the contract proper: the quantized computation within 1e-4
        expect(floored_rel_err(y, x.data(), w.data(), c.type, nullptr, in_dim, out_dim, 1) <= 1e-4,
               "within 1e-4 of the exact quantized result");
    }
}

// The types without vec_dot: the reference dequantizes each row and dots it with the fp32
// activations (quant.cpp:1404-1430); the bar is the same 1e-4 of the fp64 result.
void test_matmul_float_dot_types() {
    const TypeCase types[] = {{"F32", GgmlType::F32},   {"F16", GgmlType::F16},
                              {"Q4_1", GgmlType::Q4_1}, {"Q5_1", GgmlType::Q5_1},
                              {"Q8_1", GgmlType::Q8_1}, {"Q2_K", GgmlType::Q2_K},
                              {"Q3_K", GgmlType::Q3_K}};
    for (const TypeCase& c : types) {
        std::printf("[matmul_quant %s (float dot)]\n", c.name);
        const int in_dim = 512, out_dim = 300, n_rows = 3;
        std::vector<uint8_t> w = random_weights(c.type, in_dim, out_dim, 5 + (uint64_t)c.type);
        std::vector<float> x = activations(n_rows, in_dim, 2);
        std::vector<float> y((size_t)n_rows * out_dim), y1(out_dim);
        matmul_quant_batch(x.data(), w.data(), c.type, nullptr, in_dim, out_dim, n_rows, y.data());
        expect(floored_rel_err(y, x.data(), w.data(), c.type, nullptr, in_dim, out_dim, n_rows) <= 1e-4,
               "batch within 1e-4 of the fp64 result");
        matmul_quant(x.data() + in_dim, w.data(), c.type, nullptr, in_dim, out_dim, y1.data());
        expect(std::memcmp(y1.data(), y.data() + out_dim, out_dim * sizeof(float)) == 0,
               "batch row == single row, bit for bit");
    }
}

void test_matmul_quant_bias() {
    std::printf("[matmul_quant bias]\n");
    const int in_dim = 64, out_dim = 40;
    const size_t row_bytes = 2 * type_size(GgmlType::Q8_0);
    std::vector<uint8_t> w(row_bytes * out_dim, 0);
    for (int j = 0; j < out_dim; ++j)
        for (int b = 0; b < 2; ++b) {
            uint8_t* p = &w[j * row_bytes + b * 34];
            p[1] = 0x3C;
            for (int i = 0; i < 32; ++i) p[2 + i] = (uint8_t)(int8_t)((i + j) % 7 - 3);
        }
    std::vector<float> x = activations(1, in_dim, 0), y(out_dim), y2(out_dim), bias(out_dim);
    for (int j = 0; j < out_dim; ++j) bias[j] = (float)j;
    matmul_quant(x.data(), w.data(), GgmlType::Q8_0, nullptr, in_dim, out_dim, y.data());
    matmul_quant(x.data(), w.data(), GgmlType::Q8_0, bias.data(), in_dim, out_dim, y2.data());
    bool ok = true;
    for (int j = 0; j < out_dim; ++j) ok &= std::fabs((y2[j] - y[j]) - (float)j) <= 1e-4;
    expect(ok, "y(bias) - y == bias");
}

void test_matmul_quant_batch() {
    for (const TypeCase& c : kKernelTypes) {
        for (int n_rows : {3, 16, 40}) {
            std::printf("[matmul_quant_batch %s n_rows=%d]\n", c.name, n_rows);
            const int in_dim = 512, out_dim = 72;
            std::vector<uint8_t> w = random_weights(c.type, in_dim, out_dim, 5 + n_rows);
            std::vector<float> x = activations(n_rows, in_dim, 1), bias(out_dim);
            for (int j = 0; j < out_dim; ++j) bias[j] = 0.25f * (float)(j % 9) - 1.0f;
            std::vector<float> yb((size_t)n_rows * out_dim), y(out_dim);
            matmul_quant_batch(x.data(), w.data(), c.type, bias.data(), in_dim, out_dim, n_rows,
                               yb.data());
            // batch rows against one matmul_quant per row
            int mism = 0;
            for (int t = 0; t < n_rows; ++t) {
                matmul_quant(&x[(size_t)t * in_dim], w.data(), c.type, bias.data(), in_dim,
                             out_dim, y.data());
                for (int j = 0; j < out_dim; ++j)
                    mism += std::fabs(y[j] - yb[(size_t)t * out_dim + j]) >
                            1e-4 * std::fmax(1.0f, std::fabs(y[j]));
            }
            expect(mism == 0, "batch rows agree with single rows");
            const double err = floored_rel_err(yb, x.data(), w.data(), c.type, bias.data(),
                                               in_dim, out_dim, n_rows);
            if (err > 1e-4) std::printf("  rel err %.3g\n", err);
            expect(err <= 1e-4, "within 1e-4 of the exact quantized result");
        }
    }
}

}  // namespace

int main(int argc, char** argv) {
    const bool cpu_only = argc > 1 && std::strcmp(argv[1], "--cpu") == 0;
    try {
        test_sizes();
        test_half_conversions();
        test_argument_errors();
        if (!cpu_only) {
            test_quantize_bit_exact();
            test_vec_dot_row();
            test_matmul_quant_patterns();
            test_matmul_float_dot_types();
            test_matmul_quant_bias();
            test_matmul_quant_batch();
        }
    } catch (const std::exception& e) {
        std::printf("  FAIL unexpected exception: %s\n", e.what());
        ++g_fail;
    }
    std::printf("\n==== quant_api_test: %d passed, %d failed ====\n", g_pass, g_fail);
    return g_fail == 0 ? 0 : 1;
}
