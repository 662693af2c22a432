// k_gemv_f.hip -- float-dot GEMV for the weight types without a vec_dot kernel: F32, F16,
// Q4_1, Q5_1, Q8_1, Q2_K and Q3_K.
//
// The reference routes these through the fallback of matmul_quant (src/core/quant.cpp:
// 1404-1430; matmul_quant_batch runs it row by row, 1471-1474): each weight row is
// dequantized to fp32 and dotted with the fp32 activation row, which is NOT quantized to
// Q8_0. So here
//     y[t, j] = bias[j] + sum_i x[t, i] * deq(W[j, i])
// in fp32. F32 and F16 take one fma per element and activation row. The quantized types
// dequantize as w = A q + B over groups of 16 or 32 elements (q the element's small
// non-negative or int8 code, A and B the group's scale and offset as the reference's deq_*
// functions form them, quant.cpp:28-298), so the dot is regrouped per group:
//     sum_i x_i w_i = A * sum_i x_i q_i + B * sum_i x_i,
// one fma per element on the exact code, then two per group; the group sums of x are formed
// once, with the activation rows' staging. Only the rounding order differs from the
// reference (an exact product per element, a few roundings per group of 16 or 32): lanes own
// 32-element units of a row and the partial sums are added across lanes.
//
// Work split. A unit is 32 consecutive elements of a row: 32 fp32 or fp16 values, one
// Q4_1 / Q5_1 / Q8_1 block, or one eighth of a Q2_K / Q3_K super-block. A row's units are
// spread over L lanes (L = 64, or the power of two covering the units of a short row, so a
// wave then works on 64 / L rows at once); each lane loads the raw bytes of two units before
// decoding the first, and many waves per CU keep the HBM stream busy.
//
// Activations. The MR activation rows of a workgroup's token group are staged in LDS as fp32
// with 16 bytes of padding after every 32 values, so the 16-byte reads of the lanes (units at
// a stride of 144 bytes) spread over all 64 banks, followed by the rows' sums of every 16
// values (for the grouped types). Rows too long for the LDS budget (80 KB, two workgroups per
// CU) are read from global memory instead (they stay in L2), and the quantized types then
// take the per-element form: decode w, one fma per element.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "device_utils.h"
#include "ggml_blocks.h"
#include "launch.h"

namespace cllm_hip {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr size_t kLdsBudget = 80 * 1024;  // two workgroups per CU

// byte b (0..3) of dword v as a float: v_cvt_f32_ubyte{0..3}
__device__ __forceinline__ float ubyte_f(uint32_t v, int b) {
    return (float)((v >> (8 * b)) & 0xFFu);
}

// The 16 codes held in the bytes of v[0..3] (element order; unsigned, or int8 when SIGNED) as
// floats. The words pass through an empty asm first: the compiler knows which bits the
// callers' masks clear and would otherwise turn each byte into a narrower bit-field extract
// plus v_cvt_f32_ubyte0, instead of one v_cvt_f32_ubyte{0..3}.
template <bool SIGNED>
__device__ __forceinline__ void codes16(const uint32_t (&v)[4], float (&c)[16]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t w = v[i];
        asm volatile("" : "+v"(w));
#pragma unroll
        for (int b = 0; b < 4; ++b)
            c[4 * i + b] = SIGNED ? (float)(int8_t)((w >> (8 * b)) & 0xFFu) : ubyte_f(w, b);
    }
}

// sum over 16 elements of x[e] * c[e], x 16 consecutive floats (16-byte aligned), in order
__device__ __forceinline__ float dot16(const float (&c)[16], const float* x) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 xv = *(const float4*)(x + 4 * i);
        s = __builtin_fmaf(xv.x, c[4 * i], s);
        s = __builtin_fmaf(xv.y, c[4 * i + 1], s);
        s = __builtin_fmaf(xv.z, c[4 * i + 2], s);
        s = __builtin_fmaf(xv.w, c[4 * i + 3], s);
    }
    return s;
}

// bits 0..3 of h (h < 16) to bit 4 of bytes 0..3: h * 0x204081 puts bit j at bit 8 j
__device__ __forceinline__ uint32_t spread4_bit4(uint32_t h) {
    return ((h * 0x00204081u) & 0x01010101u) << 4;
}

// ------------------------------------------------------------------------- unit decoders
// Each FUnit<T> loads the raw bytes of unit u of a row (load) and turns them into the 32
// fp32 weights of that unit, in element order (decode).

template <uint32_t T> struct FUnit;

// F32: 128 bytes (quant.cpp:29-31)
template <> struct FUnit<T_F32> {
    struct Raw { u32x4 v[8]; };
    __device__ __forceinline__ static Raw load(const uint8_t* row, int u) {
        Raw r;
        const u32x4* p = (const u32x4*)(row + (size_t)u * 128);
#pragma unroll
        for (int i = 0; i < 8; ++i) r.v[i] = p[i];
        return r;
    }
    __device__ __forceinline__ static void decode(const Raw& r, int, float (&w)[32]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            // element values are copied out first: __builtin_bit_cast applied to a vector
            // element expression reads element 0 with this compiler
            const uint32_t e[4] = {r.v[i].x, r.v[i].y, r.v[i].z, r.v[i].w};
#pragma unroll
            for (int c = 0; c < 4; ++c) w[4 * i + c] = __builtin_bit_cast(float, e[c]);
        }
    }
};

// F16: 64 bytes, exact conversion (quant.cpp:34-37)
template <> struct FUnit<T_F16> {
    struct Raw { u32x4 v[4]; };
    __device__ __forceinline__ static Raw load(const uint8_t* row, int u) {
        Raw r;
        const u32x4* p = (const u32x4*)(row + (size_t)u * 64);
#pragma unroll
        for (int i = 0; i < 4; ++i) r.v[i] = p[i];
        return r;
    }
    __device__ __forceinline__ static void decode(const Raw& r, int, float (&w)[32]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t d[4] = {r.v[i].x, r.v[i].y, r.v[i].z, r.v[i].w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                w[8 * i + 2 * k] = f16_to_f32(d[k] & 0xFFFFu);
                w[8 * i + 2 * k + 1] = f16_to_f32(d[k] >> 16);
            }
        }
    }
};

// Q8_1: [d f16][s f16][qs i8 x32], 36 bytes, value d * q; s is not used (quant.cpp:203-214)
template <> struct FUnit<T_Q8_1> {
    struct Raw { u32x4_a4 a, b; uint32_t c; };
    __device__ __forceinline__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* p = row + (size_t)u * 36;
        Raw r;
        r.a = *(const u32x4_a4*)p;
        r.b = *(const u32x4_a4*)(p + 16);
        r.c = *(const uint32_t*)(p + 32);
        return r;
    }
    __device__ __forceinline__ static void decode(const Raw& r, int, float (&w)[32]) {
        const float d = f16_to_f32(r.a.x & 0xFFFFu);
        const uint32_t q[8] = {r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w, r.c};
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int b = 0; b < 4; ++b)
                w[4 * i + b] = d * (float)(int8_t)((q[i] >> (8 * b)) & 0xFFu);
    }
    // w = d q: A = d, no offset
    template <int MR>
    __device__ __forceinline__ static void gdot(const Raw& r, int, const float* xp, int xstride,
                                                const float*, int, float (&acc)[MR]) {
        const float d = f16_to_f32(r.a.x & 0xFFFFu);
        const uint32_t q0[4] = {r.a.y, r.a.z, r.a.w, r.b.x}, q1[4] = {r.b.y, r.b.z, r.b.w, r.c};
        float c0[16], c1[16];
        codes16<true>(q0, c0);
        codes16<true>(q1, c1);
#pragma unroll
        for (int t = 0; t < MR; ++t) {
            const float* xt = xp + (size_t)t * xstride;
            acc[t] = __builtin_fmaf(d, dot16(c0, xt) + dot16(c1, xt + 16), acc[t]);
        }
    }
};

// Q4_1: [d][m][qs 16 B], 20 bytes; byte j: low nibble = element j, high = element j + 16;
// value d * q + m (quant.cpp:164-177)
template <> struct FUnit<T_Q4_1> {
    struct Raw { uint32_t dm; u32x4_a4 qs; };
    __device__ __forceinline__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* p = row + (size_t)u * 20;
        Raw r;
        r.dm = *(const uint32_t*)p;
        r.qs = *(const u32x4_a4*)(p + 4);
        return r;
    }
    __device__ __forceinline__ static void decode(const Raw& r, int, float (&w)[32]) {
        const float d = f16_to_f32(r.dm & 0xFFFFu), m = f16_to_f32(r.dm >> 16);
        const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = q[i] & 0x0F0F0F0Fu, hi = (q[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                w[4 * i + b] = __builtin_fmaf(d, ubyte_f(lo, b), m);
                w[16 + 4 * i + b] = __builtin_fmaf(d, ubyte_f(hi, b), m);
            }
        }
    }
    // w = d q + m over the 32 elements: A = d, B = m
    template <int MR>
    __device__ __forceinline__ static void gdot(const Raw& r, int, const float* xp, int xstride,
                                                const float* xg, int gstride, float (&acc)[MR]) {
        const float d = f16_to_f32(r.dm & 0xFFFFu), m = f16_to_f32(r.dm >> 16);
        const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lo[i] = q[i] & 0x0F0F0F0Fu;
            hi[i] = (q[i] >> 4) & 0x0F0F0F0Fu;
        }
        float c0[16], c1[16];
        codes16<false>(lo, c0);
        codes16<false>(hi, c1);
#pragma unroll
        for (int t = 0; t < MR; ++t) {
            const float* xt = xp + (size_t)t * xstride;
            const float s = dot16(c0, xt) + dot16(c1, xt + 16);
            const float xsum = xg[(size_t)t * gstride] + xg[(size_t)t * gstride + 1];
            acc[t] = __builtin_fmaf(m, xsum, __builtin_fmaf(d, s, acc[t]));
        }
    }
};

// Q5_1: [d][m][qh u32][qs 16 B], 24 bytes; bit j of qh is bit 4 of element j
// (quant.cpp:182-200)
template <> struct FUnit<T_Q5_1> {
    struct Raw { u32x2_a4 dmh; u32x4_a4 qs; };
    __device__ __forceinline__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* p = row + (size_t)u * 24;
        Raw r;
        r.dmh = *(const u32x2_a4*)p;
        r.qs = *(const u32x4_a4*)(p + 8);
        return r;
    }
    __device__ __forceinline__ static void decode(const Raw& r, int, float (&w)[32]) {
        const float d = f16_to_f32(r.dmh.x & 0xFFFFu), m = f16_to_f32(r.dmh.x >> 16);
        const uint32_t qh = r.dmh.y;
        const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // bit 4 of elements 4i..4i+3 and 16+4i..: qh bits 4i.. and 16+4i.. moved to bit 4
            // of each byte
            const uint32_t h0 = (qh >> (4 * i)) & 0xFu, h1 = (qh >> (16 + 4 * i)) & 0xFu;
            const uint32_t s0 = ((h0 & 1u) | ((h0 & 2u) << 7) | ((h0 & 4u) << 14) | ((h0 & 8u) << 21)) << 4;
            const uint32_t s1 = ((h1 & 1u) | ((h1 & 2u) << 7) | ((h1 & 4u) << 14) | ((h1 & 8u) << 21)) << 4;
            const uint32_t lo = (q[i] & 0x0F0F0F0Fu) | s0, hi = ((q[i] >> 4) & 0x0F0F0F0Fu) | s1;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                w[4 * i + b] = __builtin_fmaf(d, ubyte_f(lo, b), m);
                w[16 + 4 * i + b] = __builtin_fmaf(d, ubyte_f(hi, b), m);
            }
        }
    }
    // w = d q + m over the 32 elements (q 5 bits): A = d, B = m
    template <int MR>
    __device__ __forceinline__ static void gdot(const Raw& r, int, const float* xp, int xstride,
                                                const float* xg, int gstride, float (&acc)[MR]) {
        const float d = f16_to_f32(r.dmh.x & 0xFFFFu), m = f16_to_f32(r.dmh.x >> 16);
        const uint32_t qh = r.dmh.y;
        const uint32_t q[4] = {r.qs.x, r.qs.y, r.qs.z, r.qs.w};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lo[i] = (q[i] & 0x0F0F0F0Fu) | spread4_bit4((qh >> (4 * i)) & 0xFu);
            hi[i] = ((q[i] >> 4) & 0x0F0F0F0Fu) | spread4_bit4((qh >> (16 + 4 * i)) & 0xFu);
        }
        float c0[16], c1[16];
        codes16<false>(lo, c0);
        codes16<false>(hi, c1);
#pragma unroll
        for (int t = 0; t < MR; ++t) {
            const float* xt = xp + (size_t)t * xstride;
            const float s = dot16(c0, xt) + dot16(c1, xt + 16);
            const float xsum = xg[(size_t)t * gstride] + xg[(size_t)t * gstride + 1];
            acc[t] = __builtin_fmaf(m, xsum, __builtin_fmaf(d, s, acc[t]));
        }
    }
};

// Q2_K: [scales 16][qs 64][d][dmin], 84 bytes. Unit v = 4 h + j of a super-block: elements
// 32 v + l take bits 2j..2j+1 of qs[32 h + l], with scale byte 8 h + 2 j for l < 16 and
// 8 h + 2 j + 1 for l >= 16 (low nibble scale, high nibble min); value
// d * sc * q - dmin * m (quant.cpp:218-248).
template <> struct FUnit<T_Q2_K> {
    struct Raw { u32x4_a4 q0, q1; uint32_t sc; uint32_t dd; };
    __device__ __forceinline__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)(u >> 3) * 84;
        const int v = u & 7, h = v >> 2, j = v & 3;
        Raw r;
        r.q0 = *(const u32x4_a4*)(blk + 16 + 32 * h);
        r.q1 = *(const u32x4_a4*)(blk + 32 + 32 * h);
        r.sc = ld_u16(blk + 8 * h + 2 * j);
        r.dd = *(const uint32_t*)(blk + 80);
        return r;
    }
    __device__ __forceinline__ static void decode(const Raw& r, int u, float (&w)[32]) {
        const int sh = 2 * (u & 3);
        const float d = f16_to_f32(r.dd & 0xFFFFu), dmin = f16_to_f32(r.dd >> 16);
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const uint32_t scb = (r.sc >> (8 * g)) & 0xFFu;
            const float dl = d * (float)(scb & 0xFu), ml = dmin * (float)(scb >> 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t v = (q[4 * g + i] >> sh) & 0x03030303u;
#pragma unroll
                for (int b = 0; b < 4; ++b) w[16 * g + 4 * i + b] = __builtin_fmaf(dl, ubyte_f(v, b), -ml);
            }
        }
    }
};

// Q3_K: [hmask 32][qs 64][scales 12][d], 110 bytes (2-byte aligned blocks). Unit v = 4 h + j:
// elements 32 v + l take bits 2j..2j+1 of qs[32 h + l] minus 4 unless bit 4h + j of
// hmask[l] is set, with the signed 6-bit scale 8 h + 2 j (l < 16) or 8 h + 2 j + 1 (l >= 16);
// value d * (scale - 32) * q (quant.cpp:252-298).
template <> struct FUnit<T_Q3_K> {
    struct Raw { uint32_t hm[8], q[8], sc[3], d; };
    __device__ __forceinline__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)(u >> 3) * 110;
        const int h = (u & 7) >> 2;
        Raw r;
        ld_a2<8>(blk, r.hm);
        ld_a2<8>(blk + 32 + 32 * h, r.q);
        ld_a2<3>(blk + 96, r.sc);
        r.d = ld_u16(blk + 108);
        return r;
    }
    // Scale i (0..15) of the 12 packed bytes b (as dwords s[0..2]): low four bits from byte
    // i (i < 8, low nibble) or byte i - 8 (i >= 8, high nibble), top two bits from byte
    // 8 + i % 4 at bit 2 (i / 4) (the aux shuffle of quant.cpp:259-265).
    __device__ __forceinline__ static int scale(const uint32_t (&s)[3], int i) {
        const int grp = i >> 2, ii = i & 3;
        // bytes 0-7 as one 64-bit value, shifted (an indexed pick of s[0] / s[1] would be
        // lowered to a scratch-memory load)
        const uint64_t s01 = (uint64_t)s[0] | ((uint64_t)s[1] << 32);
        const uint32_t src = (uint32_t)(s01 >> (32 * (grp & 1) + 8 * ii));
        const uint32_t lo = (grp < 2 ? src : src >> 4) & 0xFu;
        const uint32_t hi = (s[2] >> (8 * ii + 2 * grp)) & 3u;
        return (int)(lo | (hi << 4)) - 32;
    }
    __device__ __forceinline__ static void decode(const Raw& r, int u, float (&w)[32]) {
        const int v = u & 7, h = v >> 2, j = v & 3;
        const float d = f16_to_f32(r.d);
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const float dl = d * (float)scale(r.sc, 8 * h + 2 * j + g);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                // q2 | hbit << 2 per byte, so value = byte - 4
                const uint32_t q2 = (r.q[4 * g + i] >> (2 * j)) & 0x03030303u;
                const uint32_t hb = ((r.hm[4 * g + i] >> (4 * h + j)) & 0x01010101u) << 2;
                const uint32_t qv = q2 | hb;
#pragma unroll
                for (int b = 0; b < 4; ++b) w[16 * g + 4 * i + b] = dl * (ubyte_f(qv, b) - 4.0f);
            }
        }
    }
};

// The six vec_dot types, for the row dequantization below (the GEMV keeps their integer
// kernels). Values as the reference's deq_* produce them (quant.cpp:39-161, 302-336).

// Q8_0: [d][qs i8 x32], 34 bytes (2-byte aligned blocks): d * q
template <> struct FUnit<T_Q8_0> {
    struct Raw { uint32_t d; uint32_t q[8]; };
    __device__ __forceinline__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)u * 34;
        Raw r;
        r.d = ld_u16(blk);
        ld_a2<8>(blk + 2, r.q);
        return r;
    }
    __device__ __forceinline__ static void decode(const Raw& r, int, float (&w)[32]) {
        const float d = f16_to_f32(r.d);
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int b = 0; b < 4; ++b) w[4 * i + b] = d * (float)(int8_t)((r.q[i] >> (8 * b)) & 0xFFu);
    }
};

// Q4_0: [d][qs 16 B], 18 bytes: d * (q - 8), low nibble element j, high nibble j + 16
template <> struct FUnit<T_Q4_0> {
    struct Raw { uint32_t d; uint32_t q[4]; };
    __device__ __forceinline__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)u * 18;
        Raw r;
        r.d = ld_u16(blk);
        ld_a2<4>(blk + 2, r.q);
        return r;
    }
    __device__ __forceinline__ static void decode(const Raw& r, int, float (&w)[32]) {
        const float d = f16_to_f32(r.d);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = r.q[i] & 0x0F0F0F0Fu, hi = (r.q[i] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                w[4 * i + b] = d * (ubyte_f(lo, b) - 8.0f);
                w[16 + 4 * i + b] = d * (ubyte_f(hi, b) - 8.0f);
            }
        }
    }
};

// Q5_0: [d][qh u32][qs 16 B], 22 bytes: d * (q - 16), bit j of qh = bit 4 of element j
template <> struct FUnit<T_Q5_0> {
    struct Raw { uint32_t d; uint32_t qh[1]; uint32_t q[4]; };
    __device__ __forceinline__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)u * 22;
        Raw r;
        r.d = ld_u16(blk);
        ld_a2<1>(blk + 2, r.qh);
        ld_a2<4>(blk + 6, r.q);
        return r;
    }
    __device__ __forceinline__ static void decode(const Raw& r, int, float (&w)[32]) {
        const float d = f16_to_f32(r.d);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int j = 4 * i + b;
                const uint32_t byte = (r.q[i] >> (8 * b)) & 0xFFu;
                const uint32_t q0 = (byte & 0xFu) | (((r.qh[0] >> j) & 1u) << 4);
                const uint32_t q1 = (byte >> 4) | (((r.qh[0] >> (j + 16)) & 1u) << 4);
                w[j] = d * ((float)q0 - 16.0f);
                w[j + 16] = d * ((float)q1 - 16.0f);
            }
        }
    }
};

// Q4_K / Q5_K: unit u = sub-block u of the super-block: low (u even) or high (u odd)
// nibbles of the 32-byte chunk u / 2, Q5_K adding bit u of qh[l] as bit 4; value
// d * sc_u * q - dmin * m_u (quant.cpp:82-108, 302-336).
template <bool Q5>
struct FUnitK45 {
    struct Raw { uint32_t dd; uint32_t s[3]; u32x4 q0, q1, h0, h1; };
    __device__ __forceinline__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)(u >> 3) * (Q5 ? 176 : 144);
        const int c = (u & 7) >> 1;
        Raw r;
        r.dd = *(const uint32_t*)blk;
        r.s[0] = *(const uint32_t*)(blk + 4);
        r.s[1] = *(const uint32_t*)(blk + 8);
        r.s[2] = *(const uint32_t*)(blk + 12);
        const u32x4* qs = (const u32x4*)(blk + (Q5 ? 48 : 16) + 32 * c);
        r.q0 = qs[0];
        r.q1 = qs[1];
        if constexpr (Q5) {
            r.h0 = *(const u32x4*)(blk + 16);
            r.h1 = *(const u32x4*)(blk + 32);
        }
        return r;
    }
    __device__ __forceinline__ static void decode(const Raw& r, int u, float (&w)[32]) {
        const int k = u & 7;
        int sc, m;
        k4_scale_min(r.s[0], r.s[1], r.s[2], k, sc, m);
        const float d1 = f16_to_f32(r.dd & 0xFFFFu) * (float)sc;
        const float m1 = f16_to_f32(r.dd >> 16) * (float)m;
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        const uint32_t h[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t v = (k & 1) ? (q[i] >> 4) & 0x0F0F0F0Fu : q[i] & 0x0F0F0F0Fu;
            if constexpr (Q5) v |= ((h[i] >> k) & 0x01010101u) << 4;
#pragma unroll
            for (int b = 0; b < 4; ++b) w[4 * i + b] = __builtin_fmaf(d1, ubyte_f(v, b), -m1);
        }
    }
};
template <> struct FUnit<T_Q4_K> : FUnitK45<false> {};
template <> struct FUnit<T_Q5_K> : FUnitK45<true> {};

// Q6_K: [ql 128][qh 64][sc i8 x16][d], 210 bytes (2-byte aligned). Unit u = 4 g + i (half g,
// quarter i): element l takes the low (i < 2) or high nibble of ql[64 g + 32 (i & 1) + l],
// bits 2i..2i+1 of qh[32 g + l] as bits 4-5, scale sc[8 g + 2 i + l / 16]; value
// d * sc * (q - 32) (quant.cpp:135-161).
template <> struct FUnit<T_Q6_K> {
    struct Raw { uint32_t ql[8], qh[8], sc, d; };
    __device__ __forceinline__ static Raw load(const uint8_t* row, int u) {
        const uint8_t* blk = row + (size_t)(u >> 3) * 210;
        const int g = (u & 7) >> 2, i = u & 3;
        Raw r;
        ld_a2<8>(blk + 64 * g + 32 * (i & 1), r.ql);
        ld_a2<8>(blk + 128 + 32 * g, r.qh);
        r.sc = ld_u16(blk + 192 + 8 * g + 2 * i);
        r.d = ld_u16(blk + 208);
        return r;
    }
    __device__ __forceinline__ static void decode(const Raw& r, int u, float (&w)[32]) {
        const int i = u & 3;
        const float d = f16_to_f32(r.d);
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
            const float ds = d * (float)(int8_t)((r.sc >> (8 * hb)) & 0xFFu);  // exact
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t lo = (i < 2 ? r.ql[4 * hb + j] : r.ql[4 * hb + j] >> 4) & 0x0F0F0F0Fu;
                const uint32_t hi = ((r.qh[4 * hb + j] >> (2 * i)) & 0x03030303u) << 4;
                const uint32_t v = lo | hi;
#pragma unroll
                for (int b = 0; b < 4; ++b) w[16 * hb + 4 * j + b] = ds * (ubyte_f(v, b) - 32.0f);
            }
        }
    }
};

// ------------------------------------------------------------------------------ kernel


__host__ __device__ constexpr int xpad_row(int k) { return k + k / 8; }  // floats per LDS row

// Types whose dot is regrouped per 32 elements (gdot), from the LDS-staged activations.
// Q2_K and Q3_K keep the per-element form: regrouped per 16 elements they measured no faster
// on one activation row at 14336 x 4096 (Q2_K 12.6 us either way; Q3_K 15.8, with whole
// half-super-block items per lane 14.1) and, as half-super-block items, slower on four
// (63 / 65 us against 52 / 56). A batch row and the same row alone must take one path.
__host__ __device__ constexpr bool grouped(uint32_t T) {
    return T == T_Q4_1 || T == T_Q5_1 || T == T_Q8_1;
}
// LDS floats per staged activation row: the padded row, and the sums of its 16-value groups
__host__ __device__ constexpr int xlds_row(uint32_t T, int k) { return xpad_row(k) + (grouped(T) ? k / 16 : 0); }

// Workgroups per CU of the pipelined kernel for one activation row, 0 where the per-row
// kernel is faster (MI355X, 14336 x 4096, cold weights, us, per-row kernel against the
// pipelined one at 3 / 4 / 8 workgroups per CU: Q4_1 12.9 against 12.4 / 11.7 / 12.3, Q5_1
// 14.2 against 13.8 / 13.5 / 14.1; Q8_1 15.3 against 15.5 / 15.9 / 16.2)
template <uint32_t T>
constexpr int fp_wgs_per_cu() {
    return T == T_Q4_1 || T == T_Q5_1 ? 4 : 0;
}

template <int MR>
__device__ __forceinline__ void fma_unit(const float (&w)[32], const float* xp, int xstride,
                                         float (&acc)[MR]) {
#pragma unroll
    for (int t = 0; t < MR; ++t) {
        const float4* p = (const float4*)(xp + (size_t)t * xstride);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 xv = p[q];
            acc[t] = __builtin_fmaf(xv.x, w[4 * q], acc[t]);
            acc[t] = __builtin_fmaf(xv.y, w[4 * q + 1], acc[t]);
            acc[t] = __builtin_fmaf(xv.z, w[4 * q + 2], acc[t]);
            acc[t] = __builtin_fmaf(xv.w, w[4 * q + 3], acc[t]);
        }
    }
}

// Stages the MR activation rows from t0 (zeros past m) in LDS with the 16-byte pad per 32
// values; with GS a quad of lanes (16 consecutive values, never across rows: k / 4 is a
// multiple of 4) also forms the group's sum, in a fixed order, into xg[t][k / 16]. Ends with
// a workgroup barrier.
template <int MR, bool GS, int NT = kThreads>
__device__ __forceinline__ void stage_rows(const float* __restrict__ x, int k, int m, int t0, float* xs,
                                           float* xg) {
    const int q4 = k / 4;
    const int srow = xpad_row(k), gstride = k / 16;
    for (int i = threadIdx.x; i < MR * q4; i += NT) {
        const int t = i / q4, e = 4 * (i - t * q4);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t0 + t < m) v = *(const float4*)(x + (size_t)(t0 + t) * k + e);
        *(float4*)(xs + t * srow + e + (e >> 5) * 4) = v;
        if constexpr (GS) {
            float p = (v.x + v.y) + (v.z + v.w);
            p += dpp_f32<DPP_QUAD_SWAP1>(p);
            p += dpp_f32<DPP_QUAD_SWAP2>(p);
            if ((i & 3) == 0) xg[t * gstride + (e >> 4)] = p;
        }
    }
    __syncthreads();
}

// grid (row workgroups, token groups of MR), NT threads. lpr_log2 = log2(lanes per row).
template <uint32_t T, int MR, bool XG, int NT = kThreads>
__global__ __launch_bounds__(NT) void k_gemv_f(const uint8_t* __restrict__ w,
                                                     size_t row_bytes, int k, int n, int m,
                                                     const float* __restrict__ x,
                                                     const float* __restrict__ bias,
                                                     float* __restrict__ y, int lpr_log2) {
    using U = FUnit<T>;
    constexpr bool GDOT = grouped(T) && !XG;
    extern __shared__ __align__(16) float xs[];
    const int t0 = blockIdx.y * MR;
    const int units = k / 32;
    const int srow = xpad_row(k);
    const int gstride = k / 16;
    float* xg = xs + MR * srow;  // GDOT: [t][k / 16] sums of 16 activations
    if constexpr (!XG) stage_rows<MR, GDOT, NT>(x, k, m, t0, xs, xg);
    const int lane = threadIdx.x & 63;
    const int lpr = 1 << lpr_log2;
    const int sub = lane & (lpr - 1);
    const int rpw = 64 >> lpr_log2;  // rows per wave
    const int gw = blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
    const int nw = gridDim.x * (NT / 64);
    // activation source: LDS rows, or global rows clamped to the last valid one
    const float* xbase = XG ? x + (size_t)min(t0, m - 1) * k : xs;
    const int xstride = XG ? k : srow;
    auto xptr = [&](int u) { return XG ? xbase + 32 * u : xbase + 36 * u; };

    for (int rb = gw * rpw; rb < n; rb += nw * rpw) {
        const int j = rb + (lane >> lpr_log2);
        const uint8_t* row = w + (size_t)min(j, n - 1) * row_bytes;
        float acc[MR];
#pragma unroll
        for (int t = 0; t < MR; ++t) acc[t] = 0.0f;
        if constexpr (GDOT) {
            // each lane two units at a time. Both units' loads go out before either is used:
            // when some lane of the wave has a second unit (u - sub is wave-uniform), every
            // lane computes one (a lane without one takes unit u again and keeps its sums).
            // Under a per-lane branch the second unit's loads would be issued after the first
            // one's arithmetic, and each row would take two round trips.
            for (int u = sub; u < units; u += 2 * lpr) {
                const bool two = u + lpr < units;
                if (u - sub + lpr < units) {
                    const int u1 = two ? u + lpr : u;
                    const typename U::Raw r0 = U::load(row, u);
                    const typename U::Raw r1 = U::load(row, u1);
                    U::template gdot<MR>(r0, u, xptr(u), xstride, xg + 2 * u, gstride, acc);
                    float acc1[MR];
#pragma unroll
                    for (int t = 0; t < MR; ++t) acc1[t] = acc[t];
                    U::template gdot<MR>(r1, u1, xptr(u1), xstride, xg + 2 * u1, gstride, acc1);
#pragma unroll
                    for (int t = 0; t < MR; ++t) acc[t] = two ? acc1[t] : acc[t];
                } else {
                    U::template gdot<MR>(U::load(row, u), u, xptr(u), xstride, xg + 2 * u, gstride, acc);
                }
            }
        } else {
            for (int u = sub; u < units; u += 2 * lpr) {
                const bool two = u + lpr < units;
                const typename U::Raw r0 = U::load(row, u);
                const typename U::Raw r1 = U::load(row, two ? u + lpr : u);
                float wv[32];
                U::decode(r0, u, wv);
                fma_unit<MR>(wv, xptr(u), xstride, acc);
                if (two) {
                    U::decode(r1, u + lpr, wv);
                    fma_unit<MR>(wv, xptr(u + lpr), xstride, acc);
                }
            }
        }
#pragma unroll
        for (int t = 0; t < MR; ++t)
            for (int off = lpr >> 1; off > 0; off >>= 1) acc[t] += __shfl_xor(acc[t], off, 64);
        if (sub == 0 && j < n) {
            const float b = bias ? bias[j] : 0.0f;
#pragma unroll
            for (int t = 0; t < MR; ++t)
                if (t0 + t < m) y[(size_t)(t0 + t) * n + j] = acc[t] + b;
        }
    }
}

// The grouped types on rows of at most two units per lane, activations in LDS (staged as for
// k_gemv_f). Each wave walks rows rb, rb + step, .. and issues the next row's loads before
// the current row's arithmetic, unconditionally (rows past the matrix read the last row
// again, units past a short row the last unit), so that a wave keeps a row of loads in
// flight while it computes. (k_gemv_f gives every wave about one row at these sizes: the
// whole matrix is requested at once and no arithmetic overlaps the transfer.) The per-row
// arithmetic is k_gemv_f's, in the same order, so the two kernels agree bit for bit.
// grid (row workgroups, token groups of MR), 256 threads.
template <uint32_t T, int MR>
__global__ __launch_bounds__(kThreads) void k_gemv_fp(const uint8_t* __restrict__ w,
                                                      size_t row_bytes, int k, int n, int m,
                                                      const float* __restrict__ x,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ y, int lpr_log2) {
    using U = FUnit<T>;
    static_assert(grouped(T), "the grouped types only");
    extern __shared__ __align__(16) float xs[];
    const int t0 = blockIdx.y * MR;
    const int srow = xpad_row(k);
    const int gstride = k / 16;
    float* xg = xs + MR * srow;
    stage_rows<MR, true>(x, k, m, t0, xs, xg);

    const int lane = threadIdx.x & 63;
    const int lpr = 1 << lpr_log2;
    const int sub = lane & (lpr - 1);
    const int rpw = 64 >> lpr_log2;
    const int step = (int)gridDim.x * kWaves * rpw;
    const int units = k / 32;
    const bool has0 = sub < units, has1 = sub + lpr < units;
    const int u0 = min(sub, units - 1), u1 = min(sub + lpr, units - 1);
    auto row_at = [&](int rb) {
        return w + (size_t)min(rb + (lane >> lpr_log2), n - 1) * row_bytes;
    };
    const int rb0 = (blockIdx.x * kWaves + (threadIdx.x >> 6)) * rpw;
    if (rb0 >= n) return;  // wave-uniform, after the last barrier
    // NI units per lane (2 when some lane's row has a second one, else 1: uniform)
    auto walk = [&]<int NI>() {
        typename U::Raw a0 = U::load(row_at(rb0), u0);
        typename U::Raw a1 = U::load(row_at(rb0), NI == 2 ? u1 : u0);
        for (int rb = rb0; rb < n; rb += step) {
            const typename U::Raw c0 = a0;
            const typename U::Raw c1 = a1;
            a0 = U::load(row_at(rb + step), u0);
            if constexpr (NI == 2) a1 = U::load(row_at(rb + step), u1);
            float acc[MR], acc1[MR];
#pragma unroll
            for (int t = 0; t < MR; ++t) acc[t] = 0.0f;
            U::template gdot<MR>(c0, u0, xs + 36 * u0, srow, xg + 2 * u0, gstride, acc);
            if constexpr (NI == 2) {
#pragma unroll
                for (int t = 0; t < MR; ++t) acc1[t] = acc[t];
                U::template gdot<MR>(c1, u1, xs + 36 * u1, srow, xg + 2 * u1, gstride, acc1);
            }
#pragma unroll
            for (int t = 0; t < MR; ++t) acc[t] = (NI == 2 && has1) ? acc1[t] : (has0 ? acc[t] : 0.0f);
#pragma unroll
            for (int t = 0; t < MR; ++t)
                for (int off = lpr >> 1; off > 0; off >>= 1) acc[t] += __shfl_xor(acc[t], off, 64);
            const int j = rb + (lane >> lpr_log2);
            if (sub == 0 && j < n) {
                const float b = bias ? bias[j] : 0.0f;
#pragma unroll
                for (int t = 0; t < MR; ++t)
                    if (t0 + t < m) y[(size_t)(t0 + t) * n + j] = acc[t] + b;
            }
        }
    };
    if (lpr < units)
        walk.template operator()<2>();
    else
        walk.template operator()<1>();
}

// F32 / F16 rows whose length is not a multiple of 32: one wave per row, lanes stride over
// the elements, activations from global memory, every token of the batch in turn.
template <uint32_t T>
__global__ __launch_bounds__(kThreads) void k_gemv_f_any(const uint8_t* __restrict__ w,
                                                         size_t row_bytes, int k, int n, int m,
                                                         const float* __restrict__ x,
                                                         const float* __restrict__ bias,
                                                         float* __restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const int nw = gridDim.x * kWaves;
    for (int j = gw; j < n; j += nw) {
        const uint8_t* row = w + (size_t)j * row_bytes;
        for (int t = 0; t < m; ++t) {
            const float* xt = x + (size_t)t * k;
            float acc = 0.0f;
            for (int e = lane; e < k; e += 64) {
                const float wv = T == T_F32 ? ((const float*)row)[e]
                                            : f16_to_f32(((const uint16_t*)row)[e]);
                acc = __builtin_fmaf(xt[e], wv, acc);
            }
            acc = wave_sum(acc);
            if (lane == 0) y[(size_t)t * n + j] = acc + (bias ? bias[j] : 0.0f);
        }
    }
}

int device_cus_f() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            cus = v;
        else
            cus = 256;
    }
    return cus;
}

template <uint32_t T, int MR, bool XG>
hipError_t launch_mr(const uint8_t* w, size_t row_bytes, int k, int n, int m, const float* x,
                     const float* bias, float* y, hipStream_t stream) {
    const int units = k / 32;
    int lpr_log2 = 6;
    while (lpr_log2 > 0 && (1 << (lpr_log2 - 1)) >= units) --lpr_log2;
    const int rpw = 64 >> lpr_log2;
    const int64_t row_groups = ((int64_t)n + rpw - 1) / rpw;
    const int64_t wgs = std::min<int64_t>((row_groups + kWaves - 1) / kWaves,
                                          (int64_t)device_cus_f() * 8);
    const int groups = (m + MR - 1) / MR;
    if (groups > 65535) return hipErrorInvalidConfiguration;
    const size_t lds = XG ? 0 : (size_t)MR * xlds_row(T, k) * sizeof(float);
    if constexpr (grouped(T) && !XG && MR == 1) {
        // rows of at most two units per lane take the pipelined kernel where it is the
        // faster one, on fp_wgs_per_cu workgroups per CU (fewer if the rows run out). The
        // tuning knob "gemv_fp_wgs" forces it at 1 to 8 workgroups per CU, or (9) the per-row
        // kernel.
        const int knob = tuning().gemv_fp_wgs.load(std::memory_order_relaxed);
        const int per_cu = knob == 0 ? fp_wgs_per_cu<T>() : knob == 9 ? 0 : knob;
        if (units <= 2 * (1 << lpr_log2) && per_cu > 0) {
            const int64_t fwgs = std::min<int64_t>((row_groups + kWaves - 1) / kWaves,
                                                   (int64_t)device_cus_f() * per_cu);
            hipLaunchKernelGGL((k_gemv_fp<T, MR>), dim3((unsigned)fwgs, (unsigned)groups),
                               dim3(kThreads), lds, stream, w, row_bytes, k, n, m, x, bias, y, lpr_log2);
            return hipGetLastError();
        }
    }
    if constexpr (MR >= 2 && !XG) {
        // Several activation rows whose staging takes more than 20 KB of LDS run on 1024-thread
        // workgroups. LDS then holds fewer than eight 256-thread workgroups per CU (four rows
        // of 4096, ~78 KB: two), which left each wave's row loads exposed (MI355X, 14336 x
        // 4096 at 4 rows, cold weights, us, 256 / 1024 threads: Q2_K 51.3 / 21.8, Q4_1 50.5 /
        // 25.8, Q8_1 54.6 / 28.3, F16 56.4 / 32.9, F32 78.2 / 57.7). Shorter rows keep 256
        // threads (the F16 151936 x 896 head at 4 rows, 16 KB: 61.9 against 78.4 us). The
        // grid is the workgroups resident at once (two per CU; waves walk further rows): more
        // would restage the rows in every later workgroup. Same bits either way: a row's
        // additions do not depend on the workgroup size.
        if (lds > 20 * 1024) {
            constexpr int NT = 1024;
            const int64_t wgs_nt = std::min<int64_t>((row_groups + NT / 64 - 1) / (NT / 64),
                                                     (int64_t)device_cus_f() * 2);
            hipLaunchKernelGGL((k_gemv_f<T, MR, XG, NT>), dim3((unsigned)wgs_nt, (unsigned)groups),
                               dim3(NT), lds, stream, w, row_bytes, k, n, m, x, bias, y, lpr_log2);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((k_gemv_f<T, MR, XG>), dim3((unsigned)wgs, (unsigned)groups),
                       dim3(kThreads), lds, stream, w, row_bytes, k, n, m, x, bias, y, lpr_log2);
    return hipGetLastError();
}

template <uint32_t T>
hipError_t launch_type(const uint8_t* w, int k, int n, int m, const float* x, const float* bias,
                       float* y, hipStream_t stream) {
    const size_t row_bytes = (size_t)(k / block_elems(T)) * block_bytes(T);
    if constexpr (T == T_F32 || T == T_F16) {
        if (k % 32 != 0) {
            const int64_t wgs = std::min<int64_t>(((int64_t)n + kWaves - 1) / kWaves,
                                                  (int64_t)device_cus_f() * 8);
            hipLaunchKernelGGL((k_gemv_f_any<T>), dim3((unsigned)wgs), dim3(kThreads), 0, stream,
                               w, row_bytes, k, n, m, x, bias, y);
            return hipGetLastError();
        }
    }
    const size_t row_lds = (size_t)xlds_row(T, k) * sizeof(float);
    if (m >= 3 && 4 * row_lds <= kLdsBudget)
        return launch_mr<T, 4, false>(w, row_bytes, k, n, m, x, bias, y, stream);
    if (m >= 2 && 2 * row_lds <= kLdsBudget)
        return launch_mr<T, 2, false>(w, row_bytes, k, n, m, x, bias, y, stream);
    if (row_lds <= kLdsBudget)
        return launch_mr<T, 1, false>(w, row_bytes, k, n, m, x, bias, y, stream);
    if (m >= 3) return launch_mr<T, 4, true>(w, row_bytes, k, n, m, x, bias, y, stream);
    return launch_mr<T, 1, true>(w, row_bytes, k, n, m, x, bias, y, stream);
}

// Rows ids[i] of a weight matrix dequantized to fp32 (get_embedding's dequantize_block,
// engine.cpp:310-317, quant.cpp:371-389): one thread per 32-element unit.
template <uint32_t T>
__global__ __launch_bounds__(kThreads) void k_dequant_rows(const uint8_t* __restrict__ w,
                                                           size_t row_bytes, int k,
                                                           const int32_t* __restrict__ ids,
                                                           int n_ids, float* __restrict__ out) {
    const int units = k / 32;
    const int64_t g = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (g >= (int64_t)n_ids * units) return;
    const int r = (int)(g / units), u = (int)(g - (int64_t)r * units);
    float v[32];
    FUnit<T>::decode(FUnit<T>::load(w + (size_t)ids[r] * row_bytes, u), u, v);
    f32x4* o = (f32x4*)(out + (size_t)r * k + 32 * u);
#pragma unroll
    for (int q = 0; q < 8; ++q) o[q] = f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
}

// F32 / F16 rows of any length, one element per thread.
template <uint32_t T>
__global__ __launch_bounds__(kThreads) void k_dequant_rows_any(const uint8_t* __restrict__ w,
                                                               size_t row_bytes, int k,
                                                               const int32_t* __restrict__ ids,
                                                               int n_ids, float* __restrict__ out) {
    const int64_t g = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (g >= (int64_t)n_ids * k) return;
    const int r = (int)(g / k), e = (int)(g - (int64_t)r * k);
    const uint8_t* row = w + (size_t)ids[r] * row_bytes;
    out[(size_t)r * k + e] = T == T_F32 ? ((const float*)row)[e] : f16_to_f32(((const uint16_t*)row)[e]);
}

// binary16 bits -> float by integer operations only: exact for every encoding, and a NaN keeps
// its payload and signalling bit (half_to_float, include/cllm/core/quant.hpp:31-56), which the
// hardware conversion would quiet.
__device__ __forceinline__ float f16_to_f32_exact(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
    if (e == 0x1Fu) return __builtin_bit_cast(float, sign | 0x7F800000u | (man << 13));
    if (e != 0) return __builtin_bit_cast(float, sign | ((e + 112u) << 23) | (man << 13));
    // zero or subnormal: man * 2^-24, exact in fp32
    return __builtin_bit_cast(float, sign | __builtin_bit_cast(uint32_t, (float)man * 0x1p-24f));
}

// float -> binary16 bits by the rule of the reference header's float_to_half (its
// include/cllm/core/quant.hpp:58-87): results in the normal range keep the top 10 mantissa
// bits (truncation), results below it are rounded to nearest with ties to even, results
// below 2^-25 or so become signed zero, overflow becomes infinity and NaN a quiet NaN.
__device__ __forceinline__ uint32_t f32_to_f16_trunc(float f) {
    const uint32_t x = __builtin_bit_cast(uint32_t, f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t biased = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (biased == 0xFFu) return sign | (man ? 0x7E00u : 0x7C00u);
    const int e = (int)biased - 112;  // rebias 127 -> 15
    if (e >= 31) return sign | 0x7C00u;
    if (e > 0) return sign | ((uint32_t)e << 10) | (man >> 13);
    if (e < -10) return sign;
    man |= 0x800000u;
    const uint32_t shift = (uint32_t)(14 - e);
    return sign | ((man + ((1u << (shift - 1)) - 1u) + ((man >> shift) & 1u)) >> shift);
}

// Elements [0, n) of a run of blocks (dequantize_block, quant.cpp:371-389, and
// dequantize_block_f16, 398-407): thread u decodes the 32-element unit u; the elements at and
// past n of a partial last block are not written, as the reference's loops guard them. H: the
// values go out as binary16 bits (f32_to_f16_trunc) instead of fp32.
template <uint32_t T, bool H>
__global__ __launch_bounds__(kThreads) void k_dequant_span(const uint8_t* __restrict__ src,
                                                           int64_t n, float* __restrict__ out,
                                                           uint16_t* __restrict__ out16) {
    const int64_t u = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (u >= (n + 31) / 32) return;
    float v[32];
    if constexpr (T == T_F16) {
        // integer conversion, so NaN payloads pass unchanged as in half_to_float
        const u32x4* p = (const u32x4*)(src + 64 * u);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4 r = p[q];
            const uint32_t d[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[8 * q + 2 * i] = f16_to_f32_exact(d[i] & 0xFFFFu);
                v[8 * q + 2 * i + 1] = f16_to_f32_exact(d[i] >> 16);
            }
        }
    } else {
        FUnit<T>::decode(FUnit<T>::load(src, (int)u), (int)u, v);
    }
    const int64_t e0 = 32 * u;
    if (e0 + 32 <= n) {
        if constexpr (H) {
            u32x4* o = (u32x4*)(out16 + e0);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t p[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    p[i] = f32_to_f16_trunc(v[8 * q + 2 * i]) | (f32_to_f16_trunc(v[8 * q + 2 * i + 1]) << 16);
                o[q] = u32x4{p[0], p[1], p[2], p[3]};
            }
        } else {
            f32x4* o = (f32x4*)(out + e0);
#pragma unroll
            for (int q = 0; q < 8; ++q) o[q] = f32x4{v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]};
        }
    } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            if (e0 + i < n) {
                if constexpr (H)
                    out16[e0 + i] = (uint16_t)f32_to_f16_trunc(v[i]);
                else
                    out[e0 + i] = v[i];
            }
        }
    }
}

// F32 / F16 runs of any length, one element per thread.
template <uint32_t T, bool H>
__global__ __launch_bounds__(kThreads) void k_dequant_span_any(const uint8_t* __restrict__ src,
                                                               int64_t n, float* __restrict__ out,
                                                               uint16_t* __restrict__ out16) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const float v = T == T_F32 ? ((const float*)src)[i] : f16_to_f32_exact(((const uint16_t*)src)[i]);
    if constexpr (H)
        out16[i] = (uint16_t)f32_to_f16_trunc(v);
    else
        out[i] = v;
}

template <uint32_t T>
hipError_t launch_span_t(const uint8_t* src, int64_t n, float* out, uint16_t* out16,
                         hipStream_t stream) {
    if ((T == T_F32 || T == T_F16) && n % 32 != 0) {
        const unsigned grid = (unsigned)((n + kThreads - 1) / kThreads);
        if (out16)
            hipLaunchKernelGGL((k_dequant_span_any<T, true>), dim3(grid), dim3(kThreads), 0, stream, src, n, out, out16);
        else
            hipLaunchKernelGGL((k_dequant_span_any<T, false>), dim3(grid), dim3(kThreads), 0, stream, src, n, out, out16);
    } else {
        const unsigned grid = (unsigned)(((n + 31) / 32 + kThreads - 1) / kThreads);
        if (out16)
            hipLaunchKernelGGL((k_dequant_span<T, true>), dim3(grid), dim3(kThreads), 0, stream, src, n, out, out16);
        else
            hipLaunchKernelGGL((k_dequant_span<T, false>), dim3(grid), dim3(kThreads), 0, stream, src, n, out, out16);
    }
    return hipGetLastError();
}

template <uint32_t T>
hipError_t launch_dequant_t(const uint8_t* w, int k, const int32_t* ids, int n, float* out,
                            hipStream_t stream) {
    const size_t row_bytes = (size_t)(k / block_elems(T)) * block_bytes(T);
    if ((T == T_F32 || T == T_F16) && k % 32 != 0) {
        const int64_t threads = (int64_t)n * k;
        hipLaunchKernelGGL((k_dequant_rows_any<T>), dim3((unsigned)((threads + kThreads - 1) / kThreads)),
                           dim3(kThreads), 0, stream, w, row_bytes, k, ids, n, out);
    } else {
        const int64_t threads = (int64_t)n * (k / 32);
        hipLaunchKernelGGL((k_dequant_rows<T>), dim3((unsigned)((threads + kThreads - 1) / kThreads)),
                           dim3(kThreads), 0, stream, w, row_bytes, k, ids, n, out);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_dequantize_rows(uint32_t type, const uint8_t* w, int k, const int32_t* ids,
                                  int n, float* out, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    if (k <= 0 || k % block_elems(type) != 0) return hipErrorInvalidValue;
    switch (type) {
        case T_F32: return launch_dequant_t<T_F32>(w, k, ids, n, out, stream);
        case T_F16: return launch_dequant_t<T_F16>(w, k, ids, n, out, stream);
        case T_Q4_0: return launch_dequant_t<T_Q4_0>(w, k, ids, n, out, stream);
        case T_Q4_1: return launch_dequant_t<T_Q4_1>(w, k, ids, n, out, stream);
        case T_Q5_0: return launch_dequant_t<T_Q5_0>(w, k, ids, n, out, stream);
        case T_Q5_1: return launch_dequant_t<T_Q5_1>(w, k, ids, n, out, stream);
        case T_Q8_0: return launch_dequant_t<T_Q8_0>(w, k, ids, n, out, stream);
        case T_Q8_1: return launch_dequant_t<T_Q8_1>(w, k, ids, n, out, stream);
        case T_Q2_K: return launch_dequant_t<T_Q2_K>(w, k, ids, n, out, stream);
        case T_Q3_K: return launch_dequant_t<T_Q3_K>(w, k, ids, n, out, stream);
        case T_Q4_K: return launch_dequant_t<T_Q4_K>(w, k, ids, n, out, stream);
        case T_Q5_K: return launch_dequant_t<T_Q5_K>(w, k, ids, n, out, stream);
        case T_Q6_K: return launch_dequant_t<T_Q6_K>(w, k, ids, n, out, stream);
        default: return hipErrorNotSupported;
    }
}

hipError_t launch_dequantize_span(uint32_t type, const uint8_t* src, int64_t n, float* out,
                                  uint16_t* out16, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    if ((out == nullptr) == (out16 == nullptr) || n > ((int64_t)1 << 36)) return hipErrorInvalidValue;
    switch (type) {
        case T_F32: return launch_span_t<T_F32>(src, n, out, out16, stream);
        case T_F16: return launch_span_t<T_F16>(src, n, out, out16, stream);
        case T_Q4_0: return launch_span_t<T_Q4_0>(src, n, out, out16, stream);
        case T_Q4_1: return launch_span_t<T_Q4_1>(src, n, out, out16, stream);
        case T_Q5_0: return launch_span_t<T_Q5_0>(src, n, out, out16, stream);
        case T_Q5_1: return launch_span_t<T_Q5_1>(src, n, out, out16, stream);
        case T_Q8_0: return launch_span_t<T_Q8_0>(src, n, out, out16, stream);
        case T_Q8_1: return launch_span_t<T_Q8_1>(src, n, out, out16, stream);
        case T_Q2_K: return launch_span_t<T_Q2_K>(src, n, out, out16, stream);
        case T_Q3_K: return launch_span_t<T_Q3_K>(src, n, out, out16, stream);
        case T_Q4_K: return launch_span_t<T_Q4_K>(src, n, out, out16, stream);
        case T_Q5_K: return launch_span_t<T_Q5_K>(src, n, out, out16, stream);
        case T_Q6_K: return launch_span_t<T_Q6_K>(src, n, out, out16, stream);
        default: return hipErrorNotSupported;
    }
}

bool gemv_f_supported(uint32_t type) {
    return type == T_F32 || type == T_F16 || type == T_Q4_1 || type == T_Q5_1 ||
           type == T_Q8_1 || type == T_Q2_K || type == T_Q3_K;
}

hipError_t launch_gemv_f(uint32_t type, const uint8_t* w, int k, int n, int m, const float* x,
                         const float* bias, float* y, hipStream_t stream) {
    if (n <= 0 || m <= 0) return hipSuccess;
    if (k <= 0 || k % block_elems(type) != 0) return hipErrorInvalidValue;
    switch (type) {
        case T_F32: return launch_type<T_F32>(w, k, n, m, x, bias, y, stream);
        case T_F16: return launch_type<T_F16>(w, k, n, m, x, bias, y, stream);
        case T_Q4_1: return launch_type<T_Q4_1>(w, k, n, m, x, bias, y, stream);
        case T_Q5_1: return launch_type<T_Q5_1>(w, k, n, m, x, bias, y, stream);
        case T_Q8_1: return launch_type<T_Q8_1>(w, k, n, m, x, bias, y, stream);
        case T_Q2_K: return launch_type<T_Q2_K>(w, k, n, m, x, bias, y, stream);
        case T_Q3_K: return launch_type<T_Q3_K>(w, k, n, m, x, bias, y, stream);
        default: return hipErrorNotSupported;
    }
}

}  // namespace cllm_hip
