// ggml_blocks.h -- GGUF block geometry of the six vec_dot weight types, usable from host
// and device code.
//
// Byte layouts (offsets within one block) follow the reference's readers in
// src/core/quant.cpp: Q8_0 40-51, Q4_0 55-68, Q4_K 82-108, Q5_0 113-132, Q6_K 135-161,
// Q5_K 302-336; sizes 340-369; type ids include/cllm/core/quant.hpp:13-27.
#pragma once

#include <stddef.h>
#include <stdint.h>

#if defined(__HIPCC__)
#define CLLM_HD __host__ __device__
#else
#define CLLM_HD
#endif

namespace cllm_hip {

enum GgmlTypeId : uint32_t {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7, T_Q8_0 = 8,
    T_Q8_1 = 9, T_Q2_K = 10, T_Q3_K = 11, T_Q4_K = 12, T_Q5_K = 13, T_Q6_K = 14,
};

// Activation blocks are always 32 elements (Q8_0, quant.cpp:421).
constexpr int QK8 = 32;

// Q8_0: [d f16][qs i8 x32]
constexpr int Q8_0_BYTES = 34;
// Q4_0: [d f16][qs 16 B]; byte j: low nibble = elem j, high nibble = elem j + 16
constexpr int Q4_0_BYTES = 18;
// Q5_0: [d f16][qh u32 LE][qs 16 B]; bit j of qh = bit 4 of elem j
constexpr int Q5_0_BYTES = 22;
// Q4_K: [d f16][dmin f16][scales 12 B][qs 128 B]; 8 sub-blocks of 32
constexpr int Q4_K_BYTES = 144;
constexpr int Q4_K_QS = 16;
// Q5_K: [d][dmin][scales 12][qh 32][qs 128]; bit k of qh[l] = bit 4 of elem 32k + l
constexpr int Q5_K_BYTES = 176;
constexpr int Q5_K_QH = 16;
constexpr int Q5_K_QS = 48;
// Q6_K: [ql 128][qh 64][sc i8 x16][d f16]
constexpr int Q6_K_BYTES = 210;
constexpr int Q6_K_QH = 128;
constexpr int Q6_K_SC = 192;
constexpr int Q6_K_D = 208;

CLLM_HD inline int block_elems(uint32_t t) {
    switch (t) {
        case T_F32: case T_F16: return 1;
        case T_Q4_0: case T_Q4_1: case T_Q5_0: case T_Q5_1: case T_Q8_0: case T_Q8_1: return 32;
        case T_Q2_K: case T_Q3_K: case T_Q4_K: case T_Q5_K: case T_Q6_K: return 256;
        default: return 1;
    }
}

CLLM_HD inline size_t block_bytes(uint32_t t) {
    switch (t) {
        case T_F32: return 4;
        case T_F16: return 2;
        case T_Q4_0: return 18;
        case T_Q4_1: return 20;
        case T_Q5_0: return 22;
        case T_Q5_1: return 24;
        case T_Q8_0: return 34;
        case T_Q8_1: return 36;
        case T_Q2_K: return 84;
        case T_Q3_K: return 110;
        case T_Q4_K: return 144;
        case T_Q5_K: return 176;
        case T_Q6_K: return 210;
        default: return 0;
    }
}

CLLM_HD inline bool has_kernel(uint32_t t) {
    return t == T_Q4_0 || t == T_Q5_0 || t == T_Q8_0 || t == T_Q4_K || t == T_Q5_K ||
           t == T_Q6_K;
}

}  // namespace cllm_hip
