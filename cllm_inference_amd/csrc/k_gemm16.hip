// k_gemm16.hip -- batched prefill GEMM on the fp16 matrix cores, used as an exact integer
// dot-product engine.
//
// y[m, n] = sum_b dx[m,b] * (ws[n,b] * I[m,n,b] - wm[n,b] * bsum[m,b]) (+ bias[n]) -- the
// reference's per-block terms (src/core/quant.cpp:1453-1464 over the vec_dot kernels).
//
// Why fp16 MFMA. Every Q8_0 activation value q_x (|q_x| <= 128) and every weight integer the
// block layouts produce is exact in fp16, and so are the K-quant products sc * q (<= 63 * 31)
// and the split Q6_K products below. v_mfma_f32_32x32x16_f16 multiplies exactly and, for
// these magnitudes (32-element sums < 2^24), accumulates exactly in fp32. So one block's MFMA
// result F[m,n] is the reference's exact integer bracket:
//   Q4_K / Q5_K : F = sc_b * I            (B operand holds sc_b * q)
//   Q6_K        : F = sc_a*I_a + sc_b*I_b (B holds sc*(q-32) as 16*sc_hi*(q-32) + sc_lo*(q-32),
//                                          sc = 16 sc_hi + sc_lo, each part exact; quant.cpp:677)
//   Q8_0 / Q4_0 / Q5_0 : F = I            (B holds q - offset)
// leaving one fp32 FMA per output per block (acc += dx * F) instead of the int8 path's
// convert-scale-accumulate, with d applied once per 256-element super-block. The K-quant
// minimum term sum_b (dx*bsum)[m,b] * (dmin*m)[n,b] runs on v_mfma_f32_32x32x2_f32, two blocks
// (one K step) per instruction, accumulated over all of K.
//
// Tiling: a 512-thread workgroup owns a 128 x 128 output tile (activation rows x weight rows);
// each of its 8 waves a 32 x 64 sub-tile (two 32x32 MFMA tiles). K advances 64 elements (two
// blocks) per step through double-buffered LDS: while step s is computed, step s+1's weights
// and activations are loaded into registers, then unpacked into the other buffer.
#include "device_utils.h"
#include "ggml_blocks.h"
#include "launch.h"

namespace cllm_hip {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int FBM = 128;   // activation rows per workgroup
constexpr int FBN = 128;   // weight rows per workgroup
constexpr int FKS = 64;    // elements per K step (two 32-element blocks)
constexpr int FROW = 144;  // LDS row stride in bytes: 64 fp16 + 16 bytes padding
constexpr int FNT = 512;   // threads per workgroup

template <uint32_t T> struct Gemm16Traits {
    static constexpr bool KQ = T == T_Q4_K || T == T_Q5_K;   // minimum term
    static constexpr bool SUPER = KQ || T == T_Q6_K;          // d per 256-element super-block
    static constexpr bool SPLIT = T == T_Q6_K;                // two B operands per block
};

// fp16 pairs (1024 + b0, 1024 + b1) from bytes 0,1 (pair 0) or 2,3 (pair 1) of x, for byte
// values b <= 1023: 0x64 as the high byte of a binary16 is 1024 with unit spacing.
__device__ __forceinline__ h2 bias1024(uint32_t x, int pair) {
    return __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, x, pair ? 0x04030402u : 0x04010400u));
}

// 4 unsigned bytes (each <= 63) -> 4 fp16 values (byte - off) * scale, exact when the results
// are integers of at most 11 significant bits.
__device__ __forceinline__ void bytes_to_h4(uint32_t x, float off, _Float16 scale, h2& lo, h2& hi) {
    const h2 o = {(_Float16)(-(1024.0f + off)), (_Float16)(-(1024.0f + off))};
    const h2 s = {scale, scale};
    lo = (bias1024(x, 0) + o) * s;
    hi = (bias1024(x, 1) + o) * s;
}

struct StepRegs {
    // activation tile: two 16-byte pieces of the fp16 values per thread
    u32x4 a0, a1;
    float dxp;          // dx (threads 0-255) or dx * bsum (threads 256-511) of one (row, block)
    // weight bytes (meaning depends on the type)
    uint32_t w[6];
    u32x4 hdr;          // K-quant super-block header (d, dmin, 12 scale bytes)
    uint32_t dbits;     // fp16 d (Q6_K / 32-element types)
    uint32_t sh;        // byte misalignment of 2-byte-aligned blocks
};

template <uint32_t T>
__device__ __forceinline__ void load_step(StepRegs& g, const uint8_t* __restrict__ w,
                                          int64_t row_bytes, int k, int n, int m, int n0, int m0,
                                          int s, const _Float16* __restrict__ xh,
                                          const float* __restrict__ xs,
                                          const float* __restrict__ xp) {
    const int tid = threadIdx.x;
    const int nb = k / 32;
    // activations: 128 rows x 64 fp16 = 1024 pieces of 16 bytes, two per thread
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = tid + FNT * j;
        const int r = i >> 3, part = i & 7;
        const int mm = min(m0 + r, m - 1);
        const u32x4 v = ld_u32x4(xh + (size_t)mm * k + (size_t)s * FKS + 8 * part);
        if (j == 0) g.a0 = v; else g.a1 = v;
    }
    {
        const int which = tid >> 8;          // 0: dx, 1: dx * bsum
        const int r = (tid & 255) >> 1, j = tid & 1;
        const int mm = min(m0 + r, m - 1);
        const size_t ix = (size_t)mm * nb + (size_t)s * 2 + j;
        g.dxp = (which == 0) ? xs[ix] : (Gemm16Traits<T>::KQ ? xp[ix] : 0.0f);
    }
    // weights: thread (row r, quarter q4)
    const int r = tid >> 2, q4 = tid & 3;
    const uint8_t* row = w + (int64_t)min(n0 + r, n - 1) * row_bytes;
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        constexpr int BYTES = T == T_Q5_K ? Q5_K_BYTES : Q4_K_BYTES;
        const int sb = s >> 2, c = s & 3;
        const uint8_t* blk = row + (size_t)sb * BYTES;
        const u32x2 q = *(const u32x2*)(blk + (T == T_Q5_K ? Q5_K_QS : Q4_K_QS) + 32 * c + 8 * q4);
        g.w[0] = q.x;
        g.w[1] = q.y;
        if constexpr (T == T_Q5_K) {
            const u32x2 h = *(const u32x2*)(blk + Q5_K_QH + 8 * q4);
            g.w[2] = h.x;
            g.w[3] = h.y;
        }
        g.hdr = ld_u32x4(blk);
    } else if constexpr (T == T_Q6_K) {
        const int sb = s >> 2, c = s & 3, gg = c >> 1;
        const uint8_t* blk = row + (size_t)sb * Q6_K_BYTES;
        g.sh = (uint32_t)((uintptr_t)blk & 3u);
        // ql for sub-block 2(c&1) and 2(c&1)+1, qh, of elements l = 8 q4 .. 8 q4 + 7
        const uint8_t* p0 = blk + 64 * gg + 8 * q4;
        const uint8_t* p1 = blk + 64 * gg + 32 + 8 * q4;
        const uint8_t* p2 = blk + Q6_K_QH + 32 * gg + 8 * q4;
        const uint8_t* p3 = blk + Q6_K_SC + 8 * gg + 4 * (c & 1);
        const uint32_t* a0 = (const uint32_t*)(p0 - g.sh);
        const uint32_t* a1 = (const uint32_t*)(p1 - g.sh);
        const uint32_t* a2 = (const uint32_t*)(p2 - g.sh);
        const uint32_t* a3 = (const uint32_t*)(p3 - g.sh);
        // 8 bytes at p: dwords at p - sh (+4) and the last two bytes at p + 6
        g.w[0] = a0[0]; g.w[1] = a0[1]; g.w[2] = a1[0]; g.w[3] = a1[1];
        g.w[4] = a2[0]; g.w[5] = a2[1];
        g.hdr.x = ld_u16(p0 + 6);
        g.hdr.y = ld_u16(p1 + 6);
        g.hdr.z = ld_u16(p2 + 6);
        g.hdr.w = a3[0] | 0u;  // 4 scale bytes at p3 (aligned part)
        g.dbits = (uint32_t)ld_u16(p3 + 2) | ((uint32_t)ld_u16(blk + Q6_K_D) << 16);
    } else {
        constexpr int BYTES = T == T_Q8_0 ? Q8_0_BYTES : T == T_Q4_0 ? Q4_0_BYTES : Q5_0_BYTES;
        const int j = q4 >> 1, half = q4 & 1;
        const uint8_t* blk = row + (size_t)(s * 2 + j) * BYTES;
        const uint8_t* p = blk + (T == T_Q5_0 ? 6 : 2) + (T == T_Q8_0 ? 16 * half : 0);
        g.sh = (uint32_t)((uintptr_t)p & 3u);
        const u32x4 v = *(const u32x4_a4*)(p - g.sh);
        g.w[0] = v.x; g.w[1] = v.y; g.w[2] = v.z; g.w[3] = v.w;
        g.w[4] = ld_u16(p + 14);
        if constexpr (T == T_Q5_0) {
            const uint8_t* ph = blk + 2;
            g.w[5] = ((const uint32_t*)(ph - g.sh))[0] | 0u;
            g.hdr.x = ld_u16(ph + 2);
        }
        g.dbits = ld_u16(blk);
    }
}

struct Bufs {
    uint8_t* A;   // [FBM][FROW]
    uint8_t* B;   // [FBN][FROW]
    uint8_t* B2;  // [FBN][FROW] (Q6_K low part)
    float* dx;    // [2][FBM]
    float* px;    // [2][FBM]
    float* wm;    // [2][FBN]  (K-quants: dmin*m; 32-element types: d)
    float* d;     // [FBN]     (K-quants and Q6_K: d of the super-block)
};

template <uint32_t T>
__device__ __forceinline__ void store_step(const StepRegs& g, const Bufs& L, int s) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = tid + FNT * j;
        const int r = i >> 3, part = i & 7;
        *(u32x4*)(L.A + r * FROW + 16 * part) = j == 0 ? g.a0 : g.a1;
    }
    {
        const int which = tid >> 8;
        const int r = (tid & 255) >> 1, j = tid & 1;
        if (which == 0) L.dx[j * FBM + r] = g.dxp;
        else if (Gemm16Traits<T>::KQ) L.px[j * FBM + r] = g.dxp;
    }
    const int r = tid >> 2, q4 = tid & 3;
    uint8_t* brow = L.B + r * FROW;
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        const int c = s & 3;
        // scales / mins of sub-blocks 2c, 2c+1 (get_scale_min_k4, quant.cpp:72-80)
        const uint32_t sh = 16u * (uint32_t)(c & 1);
        const uint32_t w0 = g.hdr.y >> sh, w1 = g.hdr.z >> sh, w2 = g.hdr.w >> sh;
        const uint32_t sc2 = c < 2 ? (w0 & 0x3F3Fu) : ((w2 & 0x0F0Fu) | ((w0 >> 2) & 0x3030u));
        const uint32_t mn2 = c < 2 ? (w1 & 0x3F3Fu) : (((w2 >> 4) & 0x0F0Fu) | ((w1 >> 2) & 0x3030u));
        const _Float16 sc0 = (_Float16)(float)(sc2 & 0xFFu), sc1 = (_Float16)(float)(sc2 >> 8);
#pragma unroll
        for (int d = 0; d < 2; ++d) {
            uint32_t lo = g.w[d] & 0x0F0F0F0Fu, hi = (g.w[d] >> 4) & 0x0F0F0F0Fu;
            if constexpr (T == T_Q5_K) {
                lo |= ((g.w[2 + d] >> (2 * c)) & 0x01010101u) << 4;
                hi |= ((g.w[2 + d] >> (2 * c + 1)) & 0x01010101u) << 4;
            }
            h2 l0, l1, h0, h1;
            bytes_to_h4(lo, 0.0f, sc0, l0, l1);
            bytes_to_h4(hi, 0.0f, sc1, h0, h1);
            // block 0 (sub-block 2c): elements 8 q4 + 4 d ..; block 1: 32 + ...
            *(u32x2*)(brow + 2 * (8 * q4 + 4 * d)) =
                u32x2{__builtin_bit_cast(uint32_t, l0), __builtin_bit_cast(uint32_t, l1)};
            *(u32x2*)(brow + 2 * (32 + 8 * q4 + 4 * d)) =
                u32x2{__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1)};
        }
        if (q4 < 2) {
            const float dmin = f16_to_f32(g.hdr.x >> 16);
            L.wm[q4 * FBN + r] = dmin * (float)((mn2 >> (8 * q4)) & 0xFFu);
        } else if (q4 == 2) {
            L.d[r] = f16_to_f32(g.hdr.x & 0xFFFFu);
        }
    } else if constexpr (T == T_Q6_K) {
        const int c = s & 3;
        const uint32_t sh = g.sh;
        const uint32_t ql0a = __builtin_amdgcn_alignbyte(g.w[1], g.w[0], sh);
        const uint32_t ql0b = __builtin_amdgcn_alignbyte(g.hdr.x, g.w[1], sh);
        const uint32_t ql1a = __builtin_amdgcn_alignbyte(g.w[3], g.w[2], sh);
        const uint32_t ql1b = __builtin_amdgcn_alignbyte(g.hdr.y, g.w[3], sh);
        const uint32_t qha = __builtin_amdgcn_alignbyte(g.w[5], g.w[4], sh);
        const uint32_t qhb = __builtin_amdgcn_alignbyte(g.hdr.z, g.w[5], sh);
        const uint32_t sc4 = __builtin_amdgcn_alignbyte(g.dbits & 0xFFFFu, g.hdr.w, sh);
        const uint32_t lsh = (c & 1) ? 4u : 0u;  // sub-blocks 2,3 of a half use high nibbles
        const uint8_t* brow2 = L.B2 + r * FROW;
#pragma unroll
        for (int t = 0; t < 2; ++t) {  // sub-block i = 2(c&1) + t -> block t of the step
            const int i = 2 * (c & 1) + t;
            const int h16 = q4 >> 1;   // 16-element group of elements 8 q4 ..
            const int scv = (int)(int8_t)((sc4 >> (8 * (2 * t + h16))) & 0xFFu);
            const _Float16 s_hi = (_Float16)(float)(16 * (scv >> 4));
            const _Float16 s_lo = (_Float16)(float)(scv & 15);
#pragma unroll
            for (int d = 0; d < 2; ++d) {
                const uint32_t qlw = t == 0 ? (d ? ql0b : ql0a) : (d ? ql1b : ql1a);
                const uint32_t qhw = d ? qhb : qha;
                const uint32_t v = ((qlw >> lsh) & 0x0F0F0F0Fu) | (((qhw >> (2 * i)) & 0x03030303u) << 4);
                h2 a0, a1, b0, b1;
                bytes_to_h4(v, 32.0f, s_hi, a0, a1);
                bytes_to_h4(v, 32.0f, s_lo, b0, b1);
                const int e = 32 * t + 8 * q4 + 4 * d;
                *(u32x2*)(brow + 2 * e) =
                    u32x2{__builtin_bit_cast(uint32_t, a0), __builtin_bit_cast(uint32_t, a1)};
                *(u32x2*)(brow2 + 2 * e) =
                    u32x2{__builtin_bit_cast(uint32_t, b0), __builtin_bit_cast(uint32_t, b1)};
            }
        }
        if (q4 == 0) L.d[r] = f16_to_f32(g.dbits >> 16);
    } else {
        const int j = q4 >> 1, half = q4 & 1;
        uint32_t q[4];
#pragma unroll
        for (int i = 0; i < 3; ++i) q[i] = __builtin_amdgcn_alignbyte(g.w[i + 1], g.w[i], g.sh);
        q[3] = __builtin_amdgcn_alignbyte(g.w[4], g.w[3], g.sh);
        uint32_t v[4];
        if constexpr (T == T_Q8_0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = q[i] ^ 0x80808080u;  // q + 128, unsigned
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = (q[i] >> (4 * half)) & 0x0F0F0F0Fu;
            if constexpr (T == T_Q5_0) {
                const uint32_t qh = __builtin_amdgcn_alignbyte(g.hdr.x, g.w[5], g.sh) >> (16 * half);
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    v[i] |= ((((qh >> (4 * i)) & 0xFu) * 0x00204081u) & 0x01010101u) << 4;
            }
        }
        const float off = T == T_Q8_0 ? 128.0f : T == T_Q4_0 ? 8.0f : 16.0f;
        const _Float16 one = (_Float16)1.0f;
        const int e0 = 32 * j + 16 * half;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            h2 a, b;
            bytes_to_h4(v[i], off, one, a, b);
            *(u32x2*)(brow + 2 * (e0 + 4 * i)) =
                u32x2{__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b)};
        }
        if (half == 0) L.wm[j * FBN + r] = f16_to_f32(g.dbits);
    }
}

template <uint32_t T>
__global__ __launch_bounds__(FNT) void k_gemm16(const uint8_t* __restrict__ w, int64_t row_bytes,
                                                 int k, int n, int m,
                                                 const _Float16* __restrict__ xh,
                                                 const float* __restrict__ xs,
                                                 const float* __restrict__ xp,
                                                 const float* __restrict__ bias,
                                                 float* __restrict__ y) {
    using Tr = Gemm16Traits<T>;
    constexpr int BUF = FBM * FROW + FBN * FROW * (Tr::SPLIT ? 2 : 1) + 4 * (2 * FBM + 2 * FBM + 2 * FBN + FBN);
    __shared__ __align__(16) uint8_t lds[2 * BUF];
    Bufs bufs[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        uint8_t* base = lds + i * BUF;
        bufs[i].A = base;
        bufs[i].B = base + FBM * FROW;
        bufs[i].B2 = bufs[i].B + FBN * FROW;
        uint8_t* f = bufs[i].B + FBN * FROW * (Tr::SPLIT ? 2 : 1);
        bufs[i].dx = (float*)f;
        bufs[i].px = bufs[i].dx + 2 * FBM;
        bufs[i].wm = bufs[i].px + 2 * FBM;
        bufs[i].d = bufs[i].wm + 2 * FBN;
    }

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wmi = wave >> 1;  // 32-row slice of the activation tile (0..3)
    const int wni = wave & 1;   // 64-row slice of the weight tile (0..1)
    const int n0 = blockIdx.x * FBN;
    const int m0 = blockIdx.y * FBM;
    const int steps = k / FKS;

    f32x16 yacc[2], sacc[2], macc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) yacc[t][r] = sacc[t][r] = macc[t][r] = 0.0f;

    StepRegs g;
    load_step<T>(g, w, row_bytes, k, n, m, n0, m0, 0, xh, xs, xp);
    store_step<T>(g, bufs[0], 0);
    __syncthreads();

    const int arow = 32 * wmi + (lane & 31);  // A fragment row (activation)
    const int k8 = lane >> 5;                 // which 8-element half of a K16 step
    const int orow0 = 32 * wmi + 4 * k8;      // first output row of this lane (+ 8a + c)

    for (int s = 0; s < steps; ++s) {
        const Bufs& L = bufs[s & 1];
        if (s + 1 < steps) load_step<T>(g, w, row_bytes, k, n, m, n0, m0, s + 1, xh, xs, xp);

#pragma unroll
        for (int j = 0; j < 2; ++j) {  // block j of the step
            const h8 a0 = *(const h8*)(L.A + arow * FROW + 2 * (32 * j + 8 * k8));
            const h8 a1 = *(const h8*)(L.A + arow * FROW + 2 * (32 * j + 16 + 8 * k8));
            float dxr[16];
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                const float4 d4 = *(const float4*)(L.dx + j * FBM + orow0 + 8 * a4);
                dxr[4 * a4] = d4.x; dxr[4 * a4 + 1] = d4.y; dxr[4 * a4 + 2] = d4.z; dxr[4 * a4 + 3] = d4.w;
            }
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int brow = 64 * wni + 32 * t + (lane & 31);
                const h8 b0 = *(const h8*)(L.B + brow * FROW + 2 * (32 * j + 8 * k8));
                const h8 b1 = *(const h8*)(L.B + brow * FROW + 2 * (32 * j + 16 + 8 * k8));
                f32x16 F = {};
                F = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b0, F, 0, 0, 0);
                F = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b1, F, 0, 0, 0);
                if constexpr (Tr::SPLIT) {
                    const h8 c0 = *(const h8*)(L.B2 + brow * FROW + 2 * (32 * j + 8 * k8));
                    const h8 c1 = *(const h8*)(L.B2 + brow * FROW + 2 * (32 * j + 16 + 8 * k8));
                    F = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, c0, F, 0, 0, 0);
                    F = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, c1, F, 0, 0, 0);
                }
                if constexpr (Tr::SUPER) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) sacc[t][r] = fmaf(dxr[r], F[r], sacc[t][r]);
                } else {
                    const float d = L.wm[j * FBN + brow];
#pragma unroll
                    for (int r = 0; r < 16; ++r) yacc[t][r] = fmaf(dxr[r] * d, F[r], yacc[t][r]);
                }
            }
        }
        if constexpr (Tr::KQ) {
            // minimum term of both blocks: K = 2 fp32 MFMA (lane k = lane / 32 = block j)
            const float pa = L.px[k8 * FBM + arow];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const float wb = L.wm[k8 * FBN + 64 * wni + 32 * t + (lane & 31)];
                macc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(pa, wb, macc[t], 0, 0, 0);
            }
        }
        if constexpr (Tr::SUPER) {
            if ((s & 3) == 3) {  // end of a 256-element super-block: apply d
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const float d = L.d[64 * wni + 32 * t + (lane & 31)];
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        yacc[t][r] = fmaf(d, sacc[t][r], yacc[t][r]);
                        sacc[t][r] = 0.0f;
                    }
                }
            }
        }
        if (s + 1 < steps) store_step<T>(g, bufs[(s + 1) & 1], s + 1);
        __syncthreads();
    }

#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int col = n0 + 64 * wni + 32 * t + (lane & 31);
        if (col >= n) continue;
        const float bj = bias ? bias[col] : 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + orow0 + 8 * (r >> 2) + (r & 3);
            if (row < m) {
                float v = yacc[t][r];
                if constexpr (Tr::KQ) v -= macc[t][r];
                if (bias) v += bj;
                y[(size_t)row * n + col] = v;
            }
        }
    }
}

template <uint32_t T>
static hipError_t launch16_t(const uint8_t* w, int k, int n, int m, const _Float16* xh,
                             const float* xs, const float* xp, const float* bias, float* y,
                             hipStream_t stream) {
    const int64_t row_bytes = (int64_t)(k / block_elems(T)) * (int64_t)block_bytes(T);
    const dim3 grid((unsigned)((n + FBN - 1) / FBN), (unsigned)((m + FBM - 1) / FBM));
    hipLaunchKernelGGL(k_gemm16<T>, grid, dim3(FNT), 0, stream, w, row_bytes, k, n, m, xh, xs, xp,
                       bias, y);
    return hipGetLastError();
}

hipError_t launch_gemm16(uint32_t type, const uint8_t* w, int k, int n, int m,
                         const _Float16* xh, const float* xs, const float* xp, const float* bias,
                         float* y, hipStream_t stream) {
    if (k % 256 != 0) return hipErrorNotSupported;
    switch (type) {
        case T_Q4_K: return launch16_t<T_Q4_K>(w, k, n, m, xh, xs, xp, bias, y, stream);
        case T_Q5_K: return launch16_t<T_Q5_K>(w, k, n, m, xh, xs, xp, bias, y, stream);
        case T_Q6_K: return launch16_t<T_Q6_K>(w, k, n, m, xh, xs, xp, bias, y, stream);
        case T_Q8_0: return launch16_t<T_Q8_0>(w, k, n, m, xh, xs, xp, bias, y, stream);
        case T_Q4_0: return launch16_t<T_Q4_0>(w, k, n, m, xh, xs, xp, bias, y, stream);
        case T_Q5_0: return launch16_t<T_Q5_0>(w, k, n, m, xh, xs, xp, bias, y, stream);
        default: return hipErrorNotSupported;
    }
}

}  // namespace cllm_hip
