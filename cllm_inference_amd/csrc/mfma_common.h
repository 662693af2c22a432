// mfma_common.h -- building blocks of the MFMA prefill kernels (k_gemmw.hip): fragment vector
// types, direct-to-LDS loads, the fp16 magic-number unpacking of weight bytes and the Q4_K /
// Q5_K scale unpacking.
#pragma once

#include "device_utils.h"

namespace cllm_hip {

typedef _Float16 wh2 __attribute__((ext_vector_type(2)));
typedef _Float16 wh8 __attribute__((ext_vector_type(8)));
typedef __bf16 wbf8 __attribute__((ext_vector_type(8)));
typedef float wf16 __attribute__((ext_vector_type(16)));
typedef uint32_t wu4 __attribute__((ext_vector_type(4)));

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ void lds_load16(const void* g, uint8_t* lds_base) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_base, 16, 0, 0);
}
__device__ __forceinline__ void lds_load4(const void* g, uint8_t* lds_base) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_base, 4, 0, 0);
}

// Waits for this wave's outstanding vector-memory loads (including direct-to-LDS ones).
__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Returns v unchanged, but opaque to the optimizer: arithmetic on a value loaded for the next
// stage cannot be hoisted to where its load is issued, which would make the wave wait there
// for all of that stage's loads instead of after the current stage's MFMA work.
template <typename T>
__device__ __forceinline__ T pinned(T v) {
    asm volatile("" : "+v"(v));
    return v;
}


// fp16 pairs (1024 + b0, 1024 + b1) from bytes 0,1 (pair 0) or 2,3 (pair 1) of x.
__device__ __forceinline__ wh2 magic_pair(uint32_t x, int pair) {
    return __builtin_bit_cast(wh2, __builtin_amdgcn_perm(0x64646464u, x, pair ? 0x04030402u : 0x04010400u));
}

// Eight fp16 values from 8 bytes (d0, d1) holding v (or 16 v): fma(1024 + byte, s, c) with
// c = -1024 s is byte * s, exact because the result is an integer of at most 11 significant
// bits and the FMA rounds once.
__device__ __forceinline__ wh8 scaled8(uint32_t d0, uint32_t d1, wh2 s, wh2 c) {
    const wh2 a = __builtin_elementwise_fma(magic_pair(d0, 0), s, c);
    const wh2 b = __builtin_elementwise_fma(magic_pair(d0, 1), s, c);
    const wh2 e = __builtin_elementwise_fma(magic_pair(d1, 0), s, c);
    const wh2 f = __builtin_elementwise_fma(magic_pair(d1, 1), s, c);
    return wh8{a.x, a.y, b.x, b.y, e.x, e.y, f.x, f.y};
}

// Eight signed int8 values (two dwords) as exact fp16: (q ^ 0x80) = q + 128 as a byte, so the
// magic pair is 1152 + q, minus 1152.
__device__ __forceinline__ wu4 int8x8_to_h8(uint32_t d0, uint32_t d1) {
    const wh2 off = {(_Float16)-1152.0f, (_Float16)-1152.0f};
    const uint32_t u0 = d0 ^ 0x80808080u, u1 = d1 ^ 0x80808080u;
    const wh2 a = magic_pair(u0, 0) + off, b = magic_pair(u0, 1) + off;
    const wh2 e = magic_pair(u1, 0) + off, f = magic_pair(u1, 1) + off;
    return wu4{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
               __builtin_bit_cast(uint32_t, e), __builtin_bit_cast(uint32_t, f)};
}

// 6-bit scale and minimum of sub-block j of a Q4_K super-block (get_scale_min_k4,
// quant.cpp:72-80) from the 12 packed bytes in s0 (bytes 0-3), s1 (4-7), s2 (8-11).
__device__ __forceinline__ void k4_sm(int j, uint32_t s0, uint32_t s1, uint32_t s2, int& sc, int& mn) {
    if (j < 4) {
        sc = (s0 >> (8 * j)) & 63;
        mn = (s1 >> (8 * j)) & 63;
    } else {
        const int i = j - 4;
        sc = ((s2 >> (8 * i)) & 0xF) | (((s0 >> (8 * i + 6)) & 3) << 4);
        mn = ((s2 >> (8 * i + 4)) & 0xF) | (((s1 >> (8 * i + 6)) & 3) << 4);
    }
}

}  // namespace cllm_hip
