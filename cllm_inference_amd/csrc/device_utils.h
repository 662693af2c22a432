// device_utils.h -- small gfx950 building blocks shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cllm_hip {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// Same vectors with only 4-byte alignment promised: global_load_dwordx{2,4} need dword
// alignment, not natural alignment.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));

__device__ __forceinline__ float f16_to_f32(uint32_t bits16) {
    // v_cvt_f32_f16: exact for every fp16 value, subnormals included, like
    // half_to_float (include/cllm/core/quant.hpp:31-56).
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
}

__device__ __forceinline__ u32x4 ld_u32x4(const void* p) { return *(const u32x4*)p; }
__device__ __forceinline__ u32x4 ld_u32x4_nt(const void* p) {
    return __builtin_nontemporal_load((const u32x4*)p);
}

// NDW dwords starting at a 2-byte aligned address p, for blocks whose size is not a multiple
// of 4 (Q8_0 34 B, Q4_0 18 B, Q5_0 22 B, Q6_K 210 B). One dword-aligned vector load of
// [p - s, p - s + 4*NDW) with s = p & 3 in {0, 2}, plus the 2 bytes at p + 4*NDW - 2, then a
// funnel shift. Every byte read lies in [p - 2, p + 4*NDW); when s == 2 the two bytes before
// p exist because p is then at least 2 bytes past a 4-aligned base.
template <int NDW>
__device__ __forceinline__ void ld_a2(const uint8_t* p, uint32_t (&out)[NDW]) {
    const uint32_t s = (uint32_t)((uintptr_t)p & 3u);
    const uint32_t* q = (const uint32_t*)(p - s);  // pointer arithmetic keeps the address space
    uint32_t v[NDW + 1];
    if constexpr (NDW % 4 == 0) {
#pragma unroll
        for (int i = 0; i < NDW; i += 4) {
            const u32x4_a4 t = *(const u32x4_a4*)(q + i);
            v[i] = t.x; v[i + 1] = t.y; v[i + 2] = t.z; v[i + 3] = t.w;
        }
    } else if constexpr (NDW == 2) {
        const u32x2_a4 t = *(const u32x2_a4*)q;
        v[0] = t.x; v[1] = t.y;
    } else {
#pragma unroll
        for (int i = 0; i < NDW; ++i) v[i] = q[i];
    }
    v[NDW] = *(const uint16_t*)(p + 4 * NDW - 2);
    const uint32_t sel = s;
#pragma unroll
    for (int i = 0; i < NDW; ++i) out[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], sel);
}

__device__ __forceinline__ uint32_t ld_u16(const uint8_t* p) { return *(const uint16_t*)p; }

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// (scale, min) of sub-block j (0..7) from the 12 packed bytes held as dwords s0 = bytes 0-3,
// s1 = bytes 4-7, s2 = bytes 8-11 (get_scale_min_k4, src/core/quant.cpp:72-80):
//   j < 4 : sc = q[j] & 63,                          m = q[j+4] & 63
//   j >= 4: sc = (q[j+4] & 15) | ((q[j-4] >> 6) << 4), m = (q[j+4] >> 4) | ((q[j] >> 6) << 4)
__device__ __forceinline__ void k4_scale_min(uint32_t s0, uint32_t s1, uint32_t s2, int j,
                                             int& sc, int& m) {
    const uint32_t sh = 8u * (uint32_t)(j & 3);
    const uint32_t b0 = (s0 >> sh) & 0xFFu; // q[j & 3]
    const uint32_t b1 = (s1 >> sh) & 0xFFu; // q[4 + (j & 3)]
    const uint32_t b2 = (s2 >> sh) & 0xFFu; // q[8 + (j & 3)]
    const int sc_lo = (int)(b0 & 63u), m_lo = (int)(b1 & 63u);
    const int sc_hi = (int)((b2 & 15u) | ((b0 >> 6) << 4));
    const int m_hi = (int)((b2 >> 4) | ((b1 >> 6) << 4));
    sc = j < 4 ? sc_lo : sc_hi;
    m = j < 4 ? m_lo : m_hi;
}

// Q8_0 quantization of 4 consecutive elements of a 32-element block whose |x| maximum is
// amax (quantize_row_q8_0, src/core/quant.cpp:431-450, bit for bit):
//   d = amax / 127 and id = 1 / d (correctly rounded divisions), q = clamp(rint(x * id)).
// When amax is tiny enough that 1/d overflows, x * id is +-inf (or NaN for 0 * inf); the
// reference's (int) conversion of such values is x86's cvttss2si result, INT_MIN, which the
// clamp turns into -128, so that value is produced here too (v_cvt_i32_f32 would saturate).
// Returns the four int8 values packed little-endian; `sum` receives their sum.
__device__ __forceinline__ uint32_t q8_quant4(float x0, float x1, float x2, float x3, float id,
                                              int& sum) {
    const float e[4] = {x0, x1, x2, x3};
    int q[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float r = __builtin_rintf(__fmul_rn(e[i], id));
        int t = (fabsf(r) < 2147483648.0f) ? (int)r : INT32_MIN;
        t = t > 127 ? 127 : t;
        t = t < -128 ? -128 : t;
        q[i] = t;
    }
    sum = q[0] + q[1] + q[2] + q[3];
    return (uint32_t)(q[0] & 0xFF) | ((uint32_t)(q[1] & 0xFF) << 8) |
           ((uint32_t)(q[2] & 0xFF) << 16) | ((uint32_t)(q[3] & 0xFF) << 24);
}

__device__ __forceinline__ float q8_scale(float amax) { return __fdiv_rn(amax, 127.0f); }
__device__ __forceinline__ float q8_inv_scale(float d) {
    return (d != 0.0f) ? __fdiv_rn(1.0f, d) : 0.0f;
}

// fp32 -> bf16 bits, round to nearest even (finite inputs).
__device__ __forceinline__ uint32_t bf16_bits(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_val(uint32_t b) { return __builtin_bit_cast(float, b << 16); }

// dx * bsum of one Q8_0 block as three bf16 parts hi + mid + lo (24 significant bits: the
// fp32 value exactly), the token operand of the K-quant minimum term on bf16 MFMA. Stored in
// a super-block record of 32 bf16: hi at j, mid at 8 + j, lo at 16 + j and 0 at 24 + j for the
// record's block j.
__device__ __forceinline__ void xq_store(uint16_t* rec, int j, float pv) {
    const uint32_t hi = bf16_bits(pv);
    const float r1 = pv - bf16_val(hi);
    const uint32_t mid = bf16_bits(r1);
    const uint32_t lo = bf16_bits(r1 - bf16_val(mid));
    rec[j] = (uint16_t)hi;
    rec[8 + j] = (uint16_t)mid;
    rec[16 + j] = (uint16_t)lo;
    rec[24 + j] = 0;
}

// Cross-lane moves inside a row of 16 lanes (DPP; no LDS traffic).
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                 CTRL, 0xF, 0xF, false));
}
constexpr int DPP_QUAD_SWAP1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_SWAP2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;

// Sum over all 64 lanes; the result is valid in every lane.
// silu(g) * u, silu(v) = v / (1 + exp(-v)) (the reference engine's SwiGLU, engine.cpp:38),
// with IEEE division and product and the device expf.
__device__ __forceinline__ float silu_mul(float g, float u) {
    return __fmul_rn(__fdiv_rn(g, 1.0f + expf(-g)), u);
}

// Q8_0 quantization of one 32-element block held by a DPP quad of lanes, 8 consecutive
// elements e[] per lane (lane 4g + p holds elements 8p .. 8p+7), bit for bit as
// quantize_row_q8_0 (src/core/quant.cpp:431-450): q receives the lane's 8 int8 values packed
// little-endian, d the block's scale (the same in the four lanes), s8 the sum of the lane's 8
// values. All four lanes of the quad must be active.
//
// Fast path, for blocks with no inf / NaN and a finite 1/d (every real activation): amax is
// the largest (bits << 1), which orders finite floats by |x|, so it is the reference's amax;
// since fl(amax * id) < 127.5 bounds every |fl(x * id)|, rint(v) lies in [-127, 127] and is
// the low byte of fl(v + 1.5 * 2^23) (the sum lands in [2^23, 2^24), where the ulp is 1 and
// round-to-nearest-even rounds exactly as rint; the clamp cannot act). The four lanes of a
// block take the same path. Other blocks run q8_quant4, which reproduces the reference's NaN
// handling of amax and the x86 INT_MIN conversion of out-of-range values.
// fl(x * id) must be rounded before the 1.5 * 2^23 is added, so the function is compiled with
// contraction off (with it, the compiler fuses the two into one FMA, which rounds the exact
// product instead and moves a quant by one for about one value in 10^5). The product and the
// sum are written as plain * and + in this scope: HIP's __fmul_rn and __fadd_rn are plain
// operations compiled in the header's own scope, where contraction stays on.
__device__ __forceinline__ void q8_quant_quad(const float (&e)[8], uint32_t (&q)[2], float& d,
                                              int& s8) {
#pragma clang fp contract(off)
    uint32_t mb = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) mb = max(mb, __builtin_bit_cast(uint32_t, e[j]) << 1);
    mb = max(mb, (uint32_t)dpp_i32<DPP_QUAD_SWAP1>((int)mb));
    mb = max(mb, (uint32_t)dpp_i32<DPP_QUAD_SWAP2>((int)mb));
    float id = 0.0f;
    d = 0.0f;
    bool fast = mb < 0xFF000000u;  // no inf or NaN in the block
    if (fast) {
        const float amax = __builtin_bit_cast(float, mb >> 1);
        d = q8_scale(amax);
        id = q8_inv_scale(d);
        fast = __fmul_rn(amax, id) < 127.5f;  // false when 1/d overflowed to inf
    }
    s8 = 0;
    if (fast) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            uint32_t rb[4];
#pragma unroll
            for (int t = 0; t < 4; ++t)
                rb[t] = __builtin_bit_cast(uint32_t, e[4 * j + t] * id + 12582912.0f);
            const uint32_t lo = __builtin_amdgcn_perm(rb[1], rb[0], 0x0C0C0400u);
            const uint32_t hi = __builtin_amdgcn_perm(rb[3], rb[2], 0x0C0C0400u);
            q[j] = lo | (hi << 16);
            s8 = sdot4(q[j], 0x01010101u, s8);
        }
    } else {
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(e[j]));
        amax = fmaxf(amax, dpp_f32<DPP_QUAD_SWAP1>(amax));
        amax = fmaxf(amax, dpp_f32<DPP_QUAD_SWAP2>(amax));
        d = q8_scale(amax);
        id = q8_inv_scale(d);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            int sm;
            q[j] = q8_quant4(e[4 * j], e[4 * j + 1], e[4 * j + 2], e[4 * j + 3], id, sm);
            s8 += sm;
        }
    }
}

// A zero the compiler cannot see through, and a fence for it: the asm statement has side
// effects, clobbers memory and takes the base pointers of the loads issued before it (a, b, c:
// wave-uniform, or null), so for the compiler it may write their memory and no load of theirs
// moves below it, not even with __restrict__ pointers or into a later branch; adding the zero
// to a later address keeps that load below it. Every load stays one the compiler counts in its
// own vmcnt waits.
__device__ __forceinline__ uint32_t opaque_zero(const void* a = nullptr, const void* b = nullptr,
                                                const void* c = nullptr) {
    uint32_t z;
    asm volatile("v_mov_b32 %0, 0" : "=v"(z) : "s"(a), "s"(b), "s"(c) : "memory");
    return z;
}

// Sum over all 64 lanes, valid in lane 63 only: row sums by quad and mirror moves, then
// row_bcast:15 and row_bcast:31 carry them up (DPP only, no LDS-path permutes).
__device__ __forceinline__ float wave_sum63(float v) {
    v += dpp_f32<DPP_QUAD_SWAP1>(v);
    v += dpp_f32<DPP_QUAD_SWAP2>(v);
    v += dpp_f32<DPP_ROW_HALF_MIRROR>(v);
    v += dpp_f32<DPP_ROW_MIRROR>(v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142, 0xA, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143, 0xC, 0xF, false));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f32<DPP_QUAD_SWAP1>(v);
    v += dpp_f32<DPP_QUAD_SWAP2>(v);
    v += dpp_f32<DPP_ROW_HALF_MIRROR>(v);
    v += dpp_f32<DPP_ROW_MIRROR>(v);
    // four row sums -> all lanes
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

}  // namespace cllm_hip
