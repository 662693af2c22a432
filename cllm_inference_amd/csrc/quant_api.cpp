// quant_api.cpp -- the cllm Quant API (include/cllm/core/quant.hpp) over the C ABI of
// libcllm_hip.so. Host-only C++20; every computation happens in the HIP kernels.
//
// Errors: each C-ABI failure becomes std::runtime_error carrying the library's message, which
// reproduces the reference's exception text where the reference has one
// (src/core/quant.cpp:387, 423, 1370, 1379, 1443).
#include "cllm/core/quant.hpp"
#include "cllm/core/tensor.hpp"

#include <stdexcept>
#include <string>

#include "cllm_hip.h"

namespace cllm {

namespace {
void check(int rc) {
    if (rc != CLLM_HIP_OK) throw std::runtime_error(cllm_hip_last_error());
}
}  // namespace

int block_size(GgmlType type) { return cllm_hip_block_size((uint32_t)type); }

size_t type_size(GgmlType type) { return cllm_hip_type_size((uint32_t)type); }

bool has_vec_dot(GgmlType type) { return cllm_hip_has_vec_dot((uint32_t)type) != 0; }

void dequantize_block(const void* src, float* dst, GgmlType type, int64_t n) {
    check(cllm_hip_dequantize_block(src, dst, (uint32_t)type, n));
}

void dequantize_block_f16(const void* src, uint16_t* dst, GgmlType type, int64_t n) {
    check(cllm_hip_dequantize_block_f16(src, dst, (uint32_t)type, n));
}

// quant.cpp:391-395 and 409-412 of the reference
std::vector<float> Tensor::dequantize() const {
    std::vector<float> out(numel());
    dequantize_block(data, out.data(), type, (int64_t)numel());
    return out;
}

std::vector<uint16_t> Tensor::dequantize_f16() const {
    std::vector<uint16_t> out(numel());
    dequantize_block_f16(data, out.data(), type, (int64_t)numel());
    return out;
}

void quantize_row_q8_0(const float* x, QuantizedQ8_0& out, int64_t n) {
    if (n % 32 != 0) throw std::runtime_error("quantize_row_q8_0: n not divisible by 32");
    out.n = n;
    out.scales.resize((size_t)(n / 32));
    out.qs.resize((size_t)n);
    out.bsums.resize((size_t)(n / 32));
    if (n == 0) return;
    check(cllm_hip_quantize_row_q8_0(x, n, 1, out.qs.data(), out.scales.data(), out.bsums.data()));
}

float vec_dot_row(const void* w_row, GgmlType w_type, const QuantizedQ8_0& qx, int64_t n) {
    float out = 0.0f;
    check(cllm_hip_vec_dot_rows(w_row, (uint32_t)w_type, n, 1, qx.qs.data(), qx.scales.data(),
                                qx.bsums.data(), &out));
    return out;
}

void matmul_quant(const float* x, const void* w, GgmlType type, const float* bias, int in_dim,
                  int out_dim, float* y, ThreadPool* /*pool*/) {
    check(cllm_hip_matmul_quant(x, w, (uint32_t)type, bias, in_dim, out_dim, y));
}

void matmul_quant_batch(const float* x, const void* w, GgmlType type, const float* bias,
                        int in_dim, int out_dim, int n_rows, float* y, ThreadPool* /*pool*/) {
    check(cllm_hip_matmul_quant_batch(x, w, (uint32_t)type, bias, in_dim, out_dim, n_rows, y));
}

}  // namespace cllm
