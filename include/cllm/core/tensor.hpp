// tensor.hpp -- a weight tensor of a loaded GGUF file, as the cllm engine holds it.
//
// The same struct as cllm_inference's include/cllm/core/tensor.hpp (its lines 11-29): same
// members, order and types, so the reference's gguf.cpp and engine.cpp compile against it
// unchanged. Its two member functions belong to the Quant API (the reference defines them in
// src/core/quant.cpp:391-412) and are implemented in libcllm_quant.so over
// dequantize_block / dequantize_block_f16, which decode on the GPU.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "cllm/core/quant.hpp"

namespace cllm {

struct Tensor {
    std::vector<uint32_t> shape;  // GGUF order: the innermost dimension first
    GgmlType type = GgmlType::F32;
    const void* data = nullptr;   // the tensor's blocks inside the mapped file (read-only)
    uint64_t offset = 0;          // byte offset of the blocks in the file's data section

    // Product of the dimensions.
    uint64_t numel() const {
        uint64_t count = 1;
        for (uint32_t d : shape) count *= d;
        return count;
    }

    // Every element as float (dequantize_block over numel() elements).
    std::vector<float> dequantize() const;

    // Every element as binary16 bits (dequantize_block_f16 over numel() elements).
    std::vector<uint16_t> dequantize_f16() const;
};

}  // namespace cllm
