// quant.hpp -- the cllm Quant API, served by the MI355X (gfx950) kernels of libcllm_hip.so.
//
// Source-compatible with cllm_inference's include/cllm/core/quant.hpp (lines 13-151 there):
// same namespace, names, signatures, GgmlType ids and QuantizedQ8_0 layout. With
// include/cllm/core/tensor.hpp beside it, the reference's src/core/engine.cpp compiles
// against these headers unchanged and links against libcllm_quant.so: every Quant symbol the
// engine calls (matmul_quant, matmul_quant_batch at engine.cpp:237-238, 284; dequantize_block
// at 316; Tensor::dequantize / dequantize_f16 at 191-224) is defined there. Implemented in
// cllm_inference_amd/csrc/quant_api.cpp over the C ABI in cllm_hip.h.
//
// Differences a caller can observe:
//   - The ThreadPool* argument is accepted and ignored; the GPU grid replaces the pool.
//   - All thirteen types are computed on the GPU: the six with a vec_dot kernel (Q4_0, Q5_0,
//     Q8_0, Q4_K, Q5_K, Q6_K) on Q8_0 activations, the others (F32, F16, Q4_1, Q5_1, Q8_1,
//     Q2_K, Q3_K) as the reference's dequantize-and-float-dot fallback, on fp32 activations.
//   - dequantize_block / dequantize_block_f16 decode on the GPU (bit for bit the reference's
//     values) and copy the result back; they are meant for load time and single rows.
//   - Failures of the GPU runtime also surface as std::runtime_error.
#pragma once

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <vector>

namespace cllm {

class ThreadPool;

// GGUF tensor type ids.
enum class GgmlType : uint32_t {
    F32 = 0,
    F16 = 1,
    Q4_0 = 2,
    Q4_1 = 3,
    Q5_0 = 6,
    Q5_1 = 7,
    Q8_0 = 8,
    Q8_1 = 9,
    Q2_K = 10,
    Q3_K = 11,
    Q4_K = 12,
    Q5_K = 13,
    Q6_K = 14,
};

// IEEE binary16 bits -> float, exact for every input (subnormals, infinities, NaN payloads).
inline float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0x1Fu) {
        bits = sign | 0x7F800000u | (man << 13);
    } else if (exp != 0) {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {
        // subnormal: shift the leading one up to bit 10, lowering the exponent each step
        uint32_t e = 113;
        while (!(man & 0x400u)) {
            man <<= 1;
            --e;
        }
        bits = sign | (e << 23) | ((man & 0x3FFu) << 13);
    }
    float f;
    std::memcpy(&f, &bits, sizeof f);
    return f;
}

// float -> binary16 bits. Normal results keep the top 10 mantissa bits (truncation);
// results below the normal range are rounded; overflow gives infinity and NaN a quiet NaN.
// This is the conversion the reference header defines (its quant.hpp:58-87).
inline uint16_t float_to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t biased = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (biased == 0xFFu) return (uint16_t)(sign | (man ? 0x7E00u : 0x7C00u));
    const int32_t e = (int32_t)biased - 112;  // rebias 127 -> 15
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e > 0) return (uint16_t)(sign | ((uint32_t)e << 10) | (man >> 13));
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    const uint32_t shift = (uint32_t)(14 - e);
    const uint32_t half_ulp_minus_one = (1u << (shift - 1)) - 1u;
    const uint32_t odd = (man >> shift) & 1u;
    return (uint16_t)(sign | ((man + half_ulp_minus_one + odd) >> shift));
}

// Elements per block, and bytes per block.
int block_size(GgmlType type);
size_t type_size(GgmlType type);

// The first n elements of the blocks at src, dequantized to float dst[n]. A partial last
// block is read whole and written up to n. Throws "unsupported ggml type for dequantize" for
// an id that is no GGML type.
void dequantize_block(const void* src, float* dst, GgmlType type, int64_t n);

// The same values as binary16 bits (float_to_half of each; F16 blocks are copied as they are).
void dequantize_block_f16(const void* src, uint16_t* dst, GgmlType type, int64_t n);

// A Q8_0-quantized activation row: 32-element blocks, one fp32 scale and one int32 sum of
// the quantized values per block.
struct QuantizedQ8_0 {
    std::vector<float> scales;   // n / 32
    std::vector<int8_t> qs;      // n
    std::vector<int32_t> bsums;  // n / 32
    int64_t n = 0;
};

// fp32 -> Q8_0 (absmax scale per 32-element block). n must be a multiple of 32.
void quantize_row_q8_0(const float* x, QuantizedQ8_0& out, int64_t n);

// True for the weight types with an integer-dot kernel: Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K.
bool has_vec_dot(GgmlType type);

// Dot product of one quantized weight row with a quantized activation row of length n.
float vec_dot_row(const void* w_row, GgmlType w_type, const QuantizedQ8_0& qx, int64_t n);

// y[out_dim] = x[in_dim] . W[out_dim, in_dim]^T (+ bias). in_dim must be a multiple of the
// type's block size. pool is ignored.
void matmul_quant(const float* x, const void* w, GgmlType type, const float* bias, int in_dim,
                  int out_dim, float* y, ThreadPool* pool = nullptr);

// Weight-stationary batch: X[n_rows, in_dim] . W^T -> y[n_rows, out_dim], row-major.
void matmul_quant_batch(const float* x, const void* w, GgmlType type, const float* bias,
                        int in_dim, int out_dim, int n_rows, float* y,
                        ThreadPool* pool = nullptr);

}  // namespace cllm
