// k_gemv.hip -- weight-streaming GEMV kernels (decode, small n_rows) on gfx950.
//
// y[t, j] = vec_dot(W row j, Q8_0 activation row t) (+ bias[j]): the inner loops of
// matmul_quant / matmul_quant_batch (src/core/quant.cpp:1388-1397, 1453-1464) for the six
// weight types with a vec_dot kernel.
//
// Work split. A row is cut into "units" that one lane handles:
//   Q4_K, Q5_K : a quarter super-block = one 32-byte qs chunk = sub-blocks 2c and 2c+1
//   Q6_K       : a quarter super-block = half g, element half h of four sub-blocks
//   Q8_0, Q4_0, Q5_0 : one 32-element block
// Lanes stride over the units of a row, so neighbouring lanes read neighbouring bytes and
// every weight byte is loaded once, in place, from the GGUF blocks. A row's units form one or
// more "items" (64 units each) for the wave.
//
// Streaming. The grid is persistent: each wave walks rows j = wave, wave + n_waves, ... and
// keeps a ring of P items whose weight loads are in flight while it computes the oldest one
// (s_waitcnt vmcnt counts in issue order, so only the oldest item's loads are waited for).
// The Q8_0 activation rows are staged once per workgroup in LDS, together with the
// activation-only terms the kernels need (dx * bsum for the K-quant minimum, 16-element sums
// for Q6_K), so no vector-memory load other than the weight ring sits in the wave's queue.
//
// Arithmetic. Integer dots use v_dot4_i32_i8 and are exact; the fp32 per-block terms follow
// the reference (quant.cpp:545, 582-583, 621-622, 677-678, 775, 891):
//   acc += (ws * dx) * dot       and, for Q4_K / Q5_K, acc -= wm * (dx * bsum)
// Lane partial sums are reduced across the wave, so only the fp32 summation order (and the
// association of the minimum term's product) differs from the reference.
#include <algorithm>
#include <climits>
#include <atomic>
#include <cstdio>
#include <cstdlib>

#include "device_utils.h"
#include "ggml_blocks.h"
#include "launch.h"

namespace cllm_hip {

// Activation qs rows in LDS carry 16 bytes of padding after every 256 bytes: the lanes of a
// wave read 16-byte pieces at strides of 64 B (Q4_K / Q5_K), 32 B (32-element blocks) or
// 256 B + 32 B (Q6_K), which without padding land on 16 of the 64 banks; with it every access
// pattern spreads over all banks.
__host__ __device__ constexpr int lds_qs_off(int off) { return off + ((off >> 8) << 4); }
__host__ __device__ constexpr int lds_qs_row(int k) { return lds_qs_off(k); }

// Activation rows staged in LDS.
struct ActLds {
    const int8_t* qs;  // [MR][lds_qs_row(k)], padded as above
    const float* xd;   // [MR][nb] dx
    const float* xm;   // [MR][nb] dx * bsum (K-quants)
    const int32_t* xb; // [MR][nb] bsum (Q4_0 / Q5_0)
    const int32_t* hs; // [MR][2][nb] sums of 16 qs (Q6_K): index r*2nb + h*nb + b
    int k, nb;
};

// 16 activation bytes of row r at element offset e (e % 16 == 0).
__device__ __forceinline__ u32x4 lds_x16(const ActLds& a, int r, int e) {
    return *(const u32x4*)(a.qs + r * lds_qs_row(a.k) + lds_qs_off(e));
}

__device__ __forceinline__ void lds_x32(const ActLds& a, int r, int b, uint32_t (&x)[8]) {
    const u32x4 x0 = lds_x16(a, r, b * 32), x1 = lds_x16(a, r, b * 32 + 16);
    x[0] = x0.x; x[1] = x0.y; x[2] = x0.z; x[3] = x0.w;
    x[4] = x1.x; x[5] = x1.y; x[6] = x1.z; x[7] = x1.w;
}

// Raw bytes of a 2-byte-aligned field of NDW dwords: the dword-aligned vector at p & ~3 and
// the field's last two bytes. Every byte read lies in [p - 2, p + 4 NDW), and p - 2 is inside
// the buffer whenever p & 3 == 2 (see ld_a2).
template <int NDW>
struct A2 {
    uint32_t v[NDW];
    uint32_t tail;
};

template <int NDW>
__device__ __forceinline__ A2<NDW> load_a2(const uint8_t* p) {
    // Pointer arithmetic (not an integer round trip) keeps the global address space, so these
    // stay global_load_* rather than flat loads that would also count against lgkmcnt.
    const uint32_t* q = (const uint32_t*)(p - ((uintptr_t)p & 3u));
    A2<NDW> r;
    if constexpr (NDW % 4 == 0) {
#pragma unroll
        for (int i = 0; i < NDW; i += 4) {
            const u32x4_a4 t = *(const u32x4_a4*)(q + i);
            r.v[i] = t.x; r.v[i + 1] = t.y; r.v[i + 2] = t.z; r.v[i + 3] = t.w;
        }
    } else if constexpr (NDW == 2) {
        const u32x2_a4 t = *(const u32x2_a4*)q;
        r.v[0] = t.x; r.v[1] = t.y;
    } else {
#pragma unroll
        for (int i = 0; i < NDW; ++i) r.v[i] = q[i];
    }
    r.tail = *(const uint16_t*)(p + 4 * NDW - 2);
    return r;
}



template <int NDW>
__device__ __forceinline__ void align_a2(const A2<NDW>& r, uint32_t sh, uint32_t (&out)[NDW]) {
#pragma unroll
    for (int i = 0; i < NDW - 1; ++i) out[i] = __builtin_amdgcn_alignbyte(r.v[i + 1], r.v[i], sh);
    out[NDW - 1] = __builtin_amdgcn_alignbyte(r.tail, r.v[NDW - 1], sh);
}

// The same field read from a weight piece staged in LDS at byte offset off of buf (any
// alignment of 2): the aligned dwords at off & ~3 and the last two bytes.
template <int NDW>
__device__ __forceinline__ A2<NDW> lds_a2(const uint8_t* buf, int off) {
    const uint32_t* q = (const uint32_t*)(buf + (off & ~3));
    A2<NDW> r;
    if constexpr (NDW % 4 == 0) {
#pragma unroll
        for (int i = 0; i < NDW; i += 4) {
            const u32x4_a4 t = *(const u32x4_a4*)(q + i);
            r.v[i] = t.x; r.v[i + 1] = t.y; r.v[i + 2] = t.z; r.v[i + 3] = t.w;
        }
    } else if constexpr (NDW == 2) {
        const u32x2_a4 t = *(const u32x2_a4*)q;
        r.v[0] = t.x; r.v[1] = t.y;
    } else {
#pragma unroll
        for (int i = 0; i < NDW; ++i) r.v[i] = q[i];
    }
    r.tail = *(const uint16_t*)(buf + off + 4 * NDW - 2);
    return r;
}

// ------------------------------------------------------------------------------ Q4_K / Q5_K
// Unit u = 4 s + c of super-block s: the low nibbles of qs[32c .. 32c+31] are sub-block 2c,
// the high nibbles sub-block 2c+1 (quant.cpp:549-590; Q5_K adds bit k of qh[l], 592-628).
template <bool Q5>
struct TraitsK45 {
    static constexpr int UNIT = 64;
    static constexpr int BLK_BYTES = Q5 ? Q5_K_BYTES : Q4_K_BYTES, UNITS_PER_BLK = 4;
    static constexpr bool ALIGN16 = true;  // every field is a whole 16-byte piece
    static constexpr bool NEED_XM = true, NEED_XB = false, NEED_HS = false;
    struct Raw {
        u32x4 h, qa, qb;
        u32x4 hha, hhb;  // Q5_K high bits (unused for Q4_K)
    };
    static __device__ __forceinline__ Raw load(const uint8_t* row, int u) {
        const int s = u >> 2, c = u & 3;
        const uint8_t* blk = row + (size_t)s * (Q5 ? Q5_K_BYTES : Q4_K_BYTES);
        const uint8_t* qp = blk + (Q5 ? Q5_K_QS : Q4_K_QS) + 32 * c;
        Raw r;
        r.h = ld_u32x4(blk);
        r.qa = ld_u32x4(qp);
        r.qb = ld_u32x4(qp + 16);
        if constexpr (Q5) {
            r.hha = ld_u32x4(blk + Q5_K_QH);
            r.hhb = ld_u32x4(blk + Q5_K_QH + 16);
        }
        return r;
    }
    // Unit u (its quarter c = u & 3) of the super-block staged at byte o of buf.
    static __device__ __forceinline__ Raw load_lds(const uint8_t* buf, int o, int u) {
        const int c = u & 3;
        const uint8_t* blk = buf + o;
        const uint8_t* qp = blk + (Q5 ? Q5_K_QS : Q4_K_QS) + 32 * c;
        Raw r;
        r.h = *(const u32x4*)blk;
        r.qa = *(const u32x4*)qp;
        r.qb = *(const u32x4*)(qp + 16);
        if constexpr (Q5) {
            r.hha = *(const u32x4*)(blk + Q5_K_QH);
            r.hhb = *(const u32x4*)(blk + Q5_K_QH + 16);
        }
        return r;
    }
    // The weight side of unit u: nibbles (plus the Q5_K bit) and the two sub-blocks' scale and
    // minimum products.
    struct W {
        uint32_t lo[8], hi[8];
        float ws0, ws1, wm0, wm1;
    };
    // The activation side of unit u for row t: the 64 quantized values, dx and dx * bsum of its
    // two blocks.
    struct X {
        uint32_t x0[8], x1[8];
        float2 xd, xm;
    };
    static __device__ __forceinline__ W wdec(const Raw& r, int u) {
        const int c = u & 3;
        W w;
        const uint32_t q[8] = {r.qa.x, r.qa.y, r.qa.z, r.qa.w, r.qb.x, r.qb.y, r.qb.z, r.qb.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            w.lo[i] = q[i] & 0x0F0F0F0Fu;
            w.hi[i] = (q[i] >> 4) & 0x0F0F0F0Fu;
        }
        if constexpr (Q5) {
            const uint32_t qh[8] = {r.hha.x, r.hha.y, r.hha.z, r.hha.w,
                                    r.hhb.x, r.hhb.y, r.hhb.z, r.hhb.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                w.lo[i] |= ((qh[i] >> (2 * c)) & 0x01010101u) << 4;
                w.hi[i] |= ((qh[i] >> (2 * c + 1)) & 0x01010101u) << 4;
            }
        }
        // 6-bit scales / mins of sub-blocks 2c and 2c+1 (get_scale_min_k4, quant.cpp:72-80).
        // Both use bytes 2(c&1) and 2(c&1)+1 of each packed dword, so they decode as a pair of
        // bytes: for c < 2 the low 6 bits of bytes 0-3 / 4-7, for c >= 2 a nibble of bytes
        // 8-11 plus the top two bits of bytes 0-3 / 4-7.
        const uint32_t sh = 16u * (uint32_t)(c & 1);
        const uint32_t w0 = r.h.y >> sh, w1 = r.h.z >> sh, w2 = r.h.w >> sh;
        const uint32_t sc2 = c < 2 ? (w0 & 0x3F3Fu) : ((w2 & 0x0F0Fu) | ((w0 >> 2) & 0x3030u));
        const uint32_t mn2 = c < 2 ? (w1 & 0x3F3Fu) : (((w2 >> 4) & 0x0F0Fu) | ((w1 >> 2) & 0x3030u));
        const float d = f16_to_f32(r.h.x & 0xFFFFu), dmin = f16_to_f32(r.h.x >> 16);
        w.ws0 = d * (float)(sc2 & 0xFFu);
        w.ws1 = d * (float)(sc2 >> 8);
        w.wm0 = dmin * (float)(mn2 & 0xFFu);
        w.wm1 = dmin * (float)(mn2 >> 8);
        return w;
    }
    static __device__ __forceinline__ X x_of(const ActLds& a, int t, int u) {
        const int b0 = 8 * (u >> 2) + 2 * (u & 3);
        X x;
        lds_x32(a, t, b0, x.x0);
        lds_x32(a, t, b0 + 1, x.x1);
        x.xd = *(const float2*)(a.xd + (size_t)t * a.nb + b0);
        x.xm = *(const float2*)(a.xm + (size_t)t * a.nb + b0);
        return x;
    }
    static __device__ __forceinline__ float fin(const W& w, const X& x, float v, int) {
        int d0 = 0, d1 = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            d0 = sdot4(w.lo[i], x.x0[i], d0);
            d1 = sdot4(w.hi[i], x.x1[i], d1);
        }
        v = fmaf(w.ws0 * x.xd.x, (float)d0, v);
        v = fmaf(-w.wm0, x.xm.x, v);
        v = fmaf(w.ws1 * x.xd.y, (float)d1, v);
        v = fmaf(-w.wm1, x.xm.y, v);
        return v;
    }
    template <int MR>
    static __device__ __forceinline__ void compute(const Raw& r, int u, const ActLds& a,
                                                   float (&acc)[MR]) {
        const W w = wdec(r, u);
#pragma unroll
        for (int t = 0; t < MR; ++t) acc[t] = fin(w, x_of(a, t, u), acc[t], u);
    }
};

// ------------------------------------------------------------------------------------ Q6_K
// Unit u = 4 s + 2 g + h: half g (elements 128g .. 128g+127) of super-block s, element half h
// (l in [16h, 16h+16)) of its four sub-blocks i. Element l of sub-block i:
//   low4 = ql[64g + 32(i&1) + l], low nibble for i < 2, high nibble for i >= 2
//   hi2  = (qh[32g + l] >> 2i) & 3;   q6 = (low4 | hi2 << 4) - 32
// scaled by sc[8g + 2i + h] (quant.cpp:630-687). The kernel dots the unsigned 6-bit values and
// subtracts 32 * (sum of the 16 activation values), which is exact. The two lanes h = 0, 1 of
// a sub-block form the reference's integer sc_a*dot_a + sc_b*dot_b with one DPP move.
struct TraitsQ6K {
    static constexpr int UNIT = 64;
    static constexpr int BLK_BYTES = Q6_K_BYTES, UNITS_PER_BLK = 4;
    static constexpr bool ALIGN16 = false;
    static constexpr bool NEED_XM = false, NEED_XB = false, NEED_HS = true;
    struct Raw {
        A2<4> qa, qb, qh;
        A2<2> sc;
        uint32_t d;
        uint32_t sh;
    };
    static __device__ __forceinline__ Raw load(const uint8_t* row, int u) {
        const int s = u >> 2, g = (u >> 1) & 1, h = u & 1;
        const uint8_t* blk = row + (size_t)s * Q6_K_BYTES;
        Raw r;
        r.qa = load_a2<4>(blk + 64 * g + 16 * h);
        r.qb = load_a2<4>(blk + 64 * g + 32 + 16 * h);
        r.qh = load_a2<4>(blk + Q6_K_QH + 32 * g + 16 * h);
        r.sc = load_a2<2>(blk + Q6_K_SC + 8 * g);
        r.d = ld_u16(blk + Q6_K_D);
        r.sh = (uint32_t)((uintptr_t)blk & 3u);  // every field offset is a multiple of 4
        return r;
    }
    static __device__ __forceinline__ Raw load_lds(const uint8_t* buf, int o, int u) {
        const int g = (u >> 1) & 1, h = u & 1;
        Raw r;
        r.qa = lds_a2<4>(buf, o + 64 * g + 16 * h);
        r.qb = lds_a2<4>(buf, o + 64 * g + 32 + 16 * h);
        r.qh = lds_a2<4>(buf, o + Q6_K_QH + 32 * g + 16 * h);
        r.sc = lds_a2<2>(buf, o + Q6_K_SC + 8 * g);
        r.d = *(const uint16_t*)(buf + o + Q6_K_D);
        r.sh = (uint32_t)o & 3u;
        return r;
    }
    struct W {
        uint32_t v[4][4];  // [sub-block i][dword]: unsigned 6-bit values
        int scv[4];
        float d;
    };
    struct X {
        u32x4 x[4];   // the 16 quantized values of sub-block i the unit covers
        int hs[4];    // their sums
        float2 xd;    // dx of blocks bb + 2h, bb + 2h + 1
    };
    static __device__ __forceinline__ W wdec(const Raw& r, int u) {
        const int h = u & 1;
        uint32_t la[4], lb[4], qh[4], sc[2];
        align_a2<4>(r.qa, r.sh, la);
        align_a2<4>(r.qb, r.sh, lb);
        align_a2<4>(r.qh, r.sh, qh);
        align_a2<2>(r.sc, r.sh, sc);
        W w;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            w.v[0][t] = (la[t] & 0x0F0F0F0Fu) | ((qh[t] & 0x03030303u) << 4);
            w.v[1][t] = (lb[t] & 0x0F0F0F0Fu) | ((qh[t] & 0x0C0C0C0Cu) << 2);
            w.v[2][t] = ((la[t] >> 4) & 0x0F0F0F0Fu) | (qh[t] & 0x30303030u);
            w.v[3][t] = ((lb[t] >> 4) & 0x0F0F0F0Fu) | ((qh[t] >> 2) & 0x30303030u);
        }
        // sc[8g + 2i + h]: byte h (i = 0), 2 + h (i = 1) of dword 0, same of dword 1 (i = 2, 3)
        w.scv[0] = __builtin_amdgcn_sbfe((int)sc[0], 8 * h, 8);
        w.scv[1] = __builtin_amdgcn_sbfe((int)sc[0], 16 + 8 * h, 8);
        w.scv[2] = __builtin_amdgcn_sbfe((int)sc[1], 8 * h, 8);
        w.scv[3] = __builtin_amdgcn_sbfe((int)sc[1], 16 + 8 * h, 8);
        w.d = f16_to_f32(r.d);
        return w;
    }
    static __device__ __forceinline__ X x_of(const ActLds& a, int t, int u) {
        const int g = (u >> 1) & 1, h = u & 1;
        const int bb = 8 * (u >> 2) + 4 * g;
        X x;
        const u32x4 hs = *(const u32x4*)(a.hs + (size_t)t * 2 * a.nb + (size_t)h * a.nb + bb);
        x.hs[0] = (int)hs.x;
        x.hs[1] = (int)hs.y;
        x.hs[2] = (int)hs.z;
        x.hs[3] = (int)hs.w;
#pragma unroll
        for (int i = 0; i < 4; ++i) x.x[i] = lds_x16(a, t, (bb + i) * 32 + 16 * h);
        x.xd = *(const float2*)(a.xd + (size_t)t * a.nb + bb + 2 * h);
        return x;
    }
    // The two lanes h = 0, 1 of a sub-block form the reference's integer
    // sc_a * dot_a + sc_b * dot_b with one DPP move; lane h finishes sub-blocks 2h and 2h + 1.
    static __device__ __forceinline__ float fin(const W& w, const X& x, float vacc, int u) {
        const int h = u & 1;
        int tot[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            int dot = sdot4(w.v[i][0], x.x[i].x, 0);
            dot = sdot4(w.v[i][1], x.x[i].y, dot);
            dot = sdot4(w.v[i][2], x.x[i].z, dot);
            dot = sdot4(w.v[i][3], x.x[i].w, dot);
            const int part = w.scv[i] * (dot - 32 * x.hs[i]);
            tot[i] = part + dpp_i32<DPP_QUAD_SWAP1>(part);  // + partner lane h ^ 1
        }
        const int ia = h ? tot[2] : tot[0];
        const int ib = h ? tot[3] : tot[1];
        vacc = fmaf(w.d * x.xd.x, (float)ia, vacc);
        vacc = fmaf(w.d * x.xd.y, (float)ib, vacc);
        return vacc;
    }
    template <int MR>
    static __device__ __forceinline__ void compute(const Raw& r, int u, const ActLds& a,
                                                   float (&acc)[MR]) {
        const W w = wdec(r, u);
#pragma unroll
        for (int t = 0; t < MR; ++t) acc[t] = fin(w, x_of(a, t, u), acc[t], u);
    }
};

// ------------------------------------------------------------------------------------ Q8_0
struct TraitsQ80 {
    static constexpr int UNIT = 32;
    static constexpr int BLK_BYTES = Q8_0_BYTES, UNITS_PER_BLK = 1;
    static constexpr bool ALIGN16 = false;
    static constexpr bool NEED_XM = false, NEED_XB = false, NEED_HS = false;
    struct Raw {
        A2<8> q;
        uint32_t d, sh;
    };
    static __device__ __forceinline__ Raw load(const uint8_t* row, int b) {
        const uint8_t* blk = row + (size_t)b * Q8_0_BYTES;
        Raw r;
        r.q = load_a2<8>(blk + 2);
        r.d = ld_u16(blk);
        r.sh = (uint32_t)((uintptr_t)(blk + 2) & 3u);
        return r;
    }
    static __device__ __forceinline__ Raw load_lds(const uint8_t* buf, int o, int) {
        Raw r;
        r.q = lds_a2<8>(buf, o + 2);
        r.d = *(const uint16_t*)(buf + o);
        r.sh = (uint32_t)(o + 2) & 3u;
        return r;
    }
    struct W {
        uint32_t q[8];
        float d;
    };
    struct X {
        uint32_t x[8];
        float xd;
    };
    static __device__ __forceinline__ W wdec(const Raw& r, int) {
        W w;
        align_a2<8>(r.q, r.sh, w.q);
        w.d = f16_to_f32(r.d);
        return w;
    }
    static __device__ __forceinline__ X x_of(const ActLds& a, int t, int b) {
        X x;
        lds_x32(a, t, b, x.x);
        x.xd = a.xd[(size_t)t * a.nb + b];
        return x;
    }
    static __device__ __forceinline__ float fin(const W& w, const X& x, float acc, int) {
        int dot = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) dot = sdot4(w.q[i], x.x[i], dot);
        return fmaf(w.d * x.xd, (float)dot, acc);
    }
    template <int MR>
    static __device__ __forceinline__ void compute(const Raw& r, int b, const ActLds& a,
                                                   float (&acc)[MR]) {
        const W w = wdec(r, b);
#pragma unroll
        for (int t = 0; t < MR; ++t) acc[t] = fin(w, x_of(a, t, b), acc[t], b);
    }
};

// ----------------------------------------------------------------------------- Q4_0 / Q5_0
// Byte j of qs: low nibble = element j, high nibble = element j + 16. Q5_0 adds bit j of
// the little-endian u32 qh as bit 4 of element j. The bracket dot - off * bsum is an exact
// integer (quant.cpp:757-777, 863-893).
template <bool Q5>
struct TraitsQ450 {
    static constexpr int UNIT = 32;
    static constexpr int BLK_BYTES = Q5 ? Q5_0_BYTES : Q4_0_BYTES, UNITS_PER_BLK = 1;
    static constexpr bool ALIGN16 = false;
    static constexpr bool NEED_XM = false, NEED_XB = true, NEED_HS = false;
    struct Raw {
        A2<4> q;
        A2<1> qh;
        uint32_t d, sh;
    };
    // bits 0..3 of x4 -> bit 4 of bytes 0..3
    static __device__ __forceinline__ uint32_t spread4(uint32_t x4) {
        return ((x4 * 0x00204081u) & 0x01010101u) << 4;
    }
    static __device__ __forceinline__ Raw load(const uint8_t* row, int b) {
        const uint8_t* blk = row + (size_t)b * (Q5 ? Q5_0_BYTES : Q4_0_BYTES);
        Raw r;
        r.q = load_a2<4>(blk + (Q5 ? 6 : 2));
        if constexpr (Q5) r.qh = load_a2<1>(blk + 2);
        r.d = ld_u16(blk);
        r.sh = (uint32_t)((uintptr_t)(blk + 2) & 3u);  // qh (+2) and qs (+6) share it
        return r;
    }
    static __device__ __forceinline__ Raw load_lds(const uint8_t* buf, int o, int) {
        Raw r;
        r.q = lds_a2<4>(buf, o + (Q5 ? 6 : 2));
        if constexpr (Q5) r.qh = lds_a2<1>(buf, o + 2);
        r.d = *(const uint16_t*)(buf + o);
        r.sh = (uint32_t)(o + 2) & 3u;
        return r;
    }
    struct W {
        uint32_t lo[4], hi[4];
        float d;
    };
    struct X {
        uint32_t x[8];
        float xd;
        int xb;
    };
    static __device__ __forceinline__ W wdec(const Raw& r, int) {
        uint32_t q[4];
        align_a2<4>(r.q, r.sh, q);
        uint32_t qh = 0;
        if constexpr (Q5) {
            uint32_t t1[1];
            align_a2<1>(r.qh, r.sh, t1);
            qh = t1[0];
        }
        W w;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            w.lo[t] = q[t] & 0x0F0F0F0Fu;
            w.hi[t] = (q[t] >> 4) & 0x0F0F0F0Fu;
            if constexpr (Q5) {
                w.lo[t] |= spread4((qh >> (4 * t)) & 0xFu);
                w.hi[t] |= spread4((qh >> (16 + 4 * t)) & 0xFu);
            }
        }
        w.d = f16_to_f32(r.d);
        return w;
    }
    static __device__ __forceinline__ X x_of(const ActLds& a, int t, int b) {
        X x;
        lds_x32(a, t, b, x.x);
        const size_t ix = (size_t)t * a.nb + b;
        x.xd = a.xd[ix];
        x.xb = a.xb[ix];
        return x;
    }
    static __device__ __forceinline__ float fin(const W& w, const X& x, float acc, int) {
        int dot = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            dot = sdot4(w.lo[i], x.x[i], dot);
            dot = sdot4(w.hi[i], x.x[4 + i], dot);
        }
        const int inner = dot - (Q5 ? 16 : 8) * x.xb;
        return fmaf(w.d * x.xd, (float)inner, acc);
    }
    template <int MR>
    static __device__ __forceinline__ void compute(const Raw& r, int b, const ActLds& a,
                                                   float (&acc)[MR]) {
        const W w = wdec(r, b);
#pragma unroll
        for (int t = 0; t < MR; ++t) acc[t] = fin(w, x_of(a, t, b), acc[t], b);
    }
};

template <uint32_t T> struct TraitsOf;
template <> struct TraitsOf<T_Q4_K> { using type = TraitsK45<false>; };
template <> struct TraitsOf<T_Q5_K> { using type = TraitsK45<true>; };
template <> struct TraitsOf<T_Q6_K> { using type = TraitsQ6K; };
template <> struct TraitsOf<T_Q8_0> { using type = TraitsQ80; };
template <> struct TraitsOf<T_Q4_0> { using type = TraitsQ450<false>; };
template <> struct TraitsOf<T_Q5_0> { using type = TraitsQ450<true>; };

__host__ __device__ constexpr size_t align16(size_t v) { return (v + 15) & ~(size_t)15; }

// LDS bytes of the staged activation rows: qs | xd | xm or xb | hs.
template <uint32_t T>
__host__ __device__ constexpr size_t act_lds_bytes(int mr, int k) {
    using Tr = typename TraitsOf<T>::type;
    const size_t nb = (size_t)k / 32;
    size_t b = align16((size_t)mr * lds_qs_row(k)) + align16((size_t)mr * nb * 4);
    if (Tr::NEED_XM || Tr::NEED_XB) b += align16((size_t)mr * nb * 4);
    if (Tr::NEED_HS) b += align16((size_t)mr * 2 * nb * 4);
    return b;
}

// Carves the LDS block into the staged activation arrays (layout of act_lds_bytes).
template <uint32_t T, int MR>
__device__ __forceinline__ ActLds act_layout(uint8_t* lds, int k) {
    using Tr = typename TraitsOf<T>::type;
    const int nb = k / 32;
    ActLds a;
    a.k = k;
    a.nb = nb;
    size_t off = 0;
    a.qs = (const int8_t*)(lds + off);
    off += align16((size_t)MR * lds_qs_row(k));
    a.xd = (const float*)(lds + off);
    off += align16((size_t)MR * nb * 4);
    a.xm = (const float*)(lds + off);
    a.xb = (const int32_t*)(lds + off);
    if (Tr::NEED_XM || Tr::NEED_XB) off += align16((size_t)MR * nb * 4);
    a.hs = (const int32_t*)(lds + off);
    return a;
}

// Activation staging runs in two phases around the first weight loads. issue() loads the
// first kPre slots of this thread into registers before the weight ring is filled, so the
// in-order vmcnt lets them land without waiting for weight bytes; commit() writes them to LDS
// after the ring loads are out; any slots beyond kPre per thread (long or many rows) are
// loaded and written by rest(), after the ring loads. Loads are unconditional with clamped
// indices (so the compiler counts them exactly); only valid slots are stored.
constexpr int kPre = 2;

// Workgroup barrier that orders LDS only: the weight loads still in flight are not waited for.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Copy of an already-quantized Q8_0 batch: slot i < MR*k/16 is 16 qs bytes (plus its
// 16-element sum for Q6_K); slot j < MR*nb is one block's dx and bsum.
template <uint32_t T, int MR>
struct StageCopy {
    using Tr = typename TraitsOf<T>::type;
    const int8_t* __restrict__ qs;
    const float* __restrict__ xs;
    const int32_t* __restrict__ xb;
    int k;
    u32x4 q[kPre];
    float d[kPre];
    int32_t b[kPre];

    __device__ __forceinline__ int chunks() const { return MR * k / 16; }
    __device__ __forceinline__ int blocks() const { return MR * (k / 32); }

    __device__ __forceinline__ void load_slot(int i, u32x4& qv, float& dv, int32_t& bv) const {
        const int ic = min(i, chunks() - 1), jc = min(i, blocks() - 1);
        qv = ld_u32x4(qs + (size_t)ic * 16);
        dv = xs[jc];
        bv = Tr::NEED_XM || Tr::NEED_XB ? xb[jc] : 0;
    }
    __device__ __forceinline__ void store_slot(const ActLds& a, int i, const u32x4& v, float dv,
                                               int32_t bv) const {
        const int nb = k / 32;
        if (i < chunks()) {
            const int r = i / (k / 16), c = i - r * (k / 16);
            *(u32x4*)(const_cast<int8_t*>(a.qs) + r * lds_qs_row(k) + lds_qs_off(c * 16)) = v;
            if constexpr (Tr::NEED_HS) {
                int sm = sdot4(v.x, 0x01010101u, 0);
                sm = sdot4(v.y, 0x01010101u, sm);
                sm = sdot4(v.z, 0x01010101u, sm);
                sm = sdot4(v.w, 0x01010101u, sm);
                const_cast<int32_t*>(a.hs)[(size_t)r * 2 * nb + (size_t)(c & 1) * nb + (c >> 1)] = sm;
            }
        }
        if (i < blocks()) {
            const_cast<float*>(a.xd)[i] = dv;
            if constexpr (Tr::NEED_XM) const_cast<float*>(a.xm)[i] = dv * (float)bv;
            if constexpr (Tr::NEED_XB) const_cast<int32_t*>(a.xb)[i] = bv;
        }
    }
    __device__ __forceinline__ void issue() {
#pragma unroll
        for (int p = 0; p < kPre; ++p) load_slot(threadIdx.x + p * blockDim.x, q[p], d[p], b[p]);
    }
    __device__ __forceinline__ void commit(const ActLds& a) const {
#pragma unroll
        for (int p = 0; p < kPre; ++p) store_slot(a, threadIdx.x + p * blockDim.x, q[p], d[p], b[p]);
    }
    __device__ __forceinline__ void rest(const ActLds& a) const {
        const int n = max(chunks(), blocks());
        for (int i = threadIdx.x + kPre * blockDim.x; i < n; i += blockDim.x) {
            u32x4 qv;
            float dv;
            int32_t bv;
            load_slot(i, qv, dv, bv);
            store_slot(a, i, qv, dv, bv);
        }
    }
};

// Fused decode: quantize MR fp32 activation rows straight into the LDS layout, bit for bit as
// k_quantize_q8_0 (q8_quant_quad). Slot i = lanes 4g + p of the workgroup: elements 8p .. 8p+7
// of activation block g (row-major over the rows); the four lanes of a block are one DPP quad.
//
// With NORM (one row of at most 4096 elements, 512 threads) the row first goes through the
// RMSNorm h = (x * rms) * nw (engine.cpp:23-28) and h is quantized. The sum of squares is
// reduced in the order of k_rmsnorm_q8_0_reg<1> (1024 threads of one 4-element chunk each, a
// wave sum, then the 16 wave sums in order), so h and its blocks are bit-identical to that
// kernel's: thread t holds chunks 2t and 2t + 1, and their sum followed by butterflies over
// 2, 4, .., 32 lanes adds the same pairs of values as that kernel's wave sum (float addition
// is commutative), leaving its wave sums 2w and 2w + 1 in lanes 0 and 32 of wave w; waves
// past the eighth hold no elements. RAWBAR: the workgroup barrier waits for LDS writes only
// (k_gemv_st, whose LDS-DMA weight loads a fenced barrier would wait for too).
//
// SP slots per thread go out with issue_all() and are quantized by commit() (SP = 2: both
// before the caller's next loads, so a batch of up to 2 x blockDim slots is staged after
// one round trip); rest() takes the slots past SP x blockDim.
template <uint32_t T, int MR, bool NORM = false, bool RAWBAR = false, int SP = 1>
struct StageQuant {
    using Tr = typename TraitsOf<T>::type;
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    static_assert(SP == 1 || (SP == 2 && !NORM), "two slots per thread without the RMSNorm");
    const float* __restrict__ x;
    int k;
    f32x4 v[2];
    f32x4 v2[2] = {};  // SP = 2: the thread's second slot
    const float* __restrict__ nw = nullptr;  // NORM: the norm weight
    float eps = 0.0f;
    float* part = nullptr;                   // NORM: 16 floats of LDS
    f32x4 wv[2] = {};

    __device__ __forceinline__ int slots() const { return MR * (k / 8); }
    __device__ __forceinline__ void load_slot(int i, f32x4 (&r)[2]) const {
        const f32x4* p = (const f32x4*)(x + (size_t)min(i, slots() - 1) * 8);
        r[0] = p[0];
        r[1] = p[1];
    }
    // Quantizes slot i (the caller keeps i < slots(); slots() is a multiple of 4, so the quad
    // of a live lane is live).
    __device__ __forceinline__ void quant_slot(const ActLds& a, int i, const f32x4 (&r)[2]) const {
        const int nb = a.nb;
        const int g = i >> 2, part = i & 3;
        const int row = MR == 1 ? 0 : g / nb, b = g - row * nb;
        const float e[8] = {r[0].x, r[0].y, r[0].z, r[0].w, r[1].x, r[1].y, r[1].z, r[1].w};
        uint32_t q[2];
        float d;
        int s8;
        q8_quant_quad(e, q, d, s8);
        *(u32x2*)(const_cast<int8_t*>(a.qs) + row * lds_qs_row(a.k) + lds_qs_off(b * 32 + part * 8)) =
            u32x2{q[0], q[1]};
        const int s16 = s8 + dpp_i32<DPP_QUAD_SWAP1>(s8);  // this half block's sum
        if constexpr (Tr::NEED_HS) {
            if ((part & 1) == 0)
                const_cast<int32_t*>(a.hs)[(size_t)row * 2 * nb + (size_t)(part >> 1) * nb + b] = s16;
        }
        const int bsum = s16 + dpp_i32<DPP_QUAD_SWAP2>(s16);
        if (part == 0) {
            const_cast<float*>(a.xd)[g] = d;
            if constexpr (Tr::NEED_XM) const_cast<float*>(a.xm)[g] = d * (float)bsum;
            if constexpr (Tr::NEED_XB) const_cast<int32_t*>(a.xb)[g] = bsum;
        }
    }
    // Waves with no slot load nothing; lanes of a partly used wave load a clamped slot.
    __device__ __forceinline__ bool wave_live() const {
        return (int)(threadIdx.x & ~63u) < slots();
    }
    __device__ __forceinline__ void issue() {
        if (wave_live()) {
            load_slot(threadIdx.x, v);
            if constexpr (NORM) {
                const f32x4* p = (const f32x4*)(nw + (size_t)min((int)threadIdx.x, slots() - 1) * 8);
                wv[0] = p[0];
                wv[1] = p[1];
            }
        }
    }
    // issue() in every wave, with no branch (waves past the slots load the last slot again):
    // loads issued after these on one straight path leave the compiler's wait before their
    // first use at vmcnt(loads issued since), so those loads stay in flight meanwhile.
    __device__ __forceinline__ void issue_all() {
        load_slot(threadIdx.x, v);
        if constexpr (SP == 2) load_slot(threadIdx.x + blockDim.x, v2);
        if constexpr (NORM) {
            const f32x4* p = (const f32x4*)(nw + (size_t)min((int)threadIdx.x, slots() - 1) * 8);
            wv[0] = p[0];
            wv[1] = p[1];
        }
    }
    // NORM: every thread of the workgroup takes part (one LDS barrier).
    __device__ __forceinline__ void normalize() {
        float sa = 0.0f, sb = 0.0f;
        if ((int)threadIdx.x < slots()) {
            sa = __builtin_fmaf(v[0].x, v[0].x, sa);
            sa = __builtin_fmaf(v[0].y, v[0].y, sa);
            sa = __builtin_fmaf(v[0].z, v[0].z, sa);
            sa = __builtin_fmaf(v[0].w, v[0].w, sa);
            sb = __builtin_fmaf(v[1].x, v[1].x, sb);
            sb = __builtin_fmaf(v[1].y, v[1].y, sb);
            sb = __builtin_fmaf(v[1].z, v[1].z, sb);
            sb = __builtin_fmaf(v[1].w, v[1].w, sb);
        }
        float s = sa + sb;
        s += dpp_f32<DPP_QUAD_SWAP1>(s);
        s += dpp_f32<DPP_QUAD_SWAP2>(s);
        s += dpp_f32<DPP_ROW_HALF_MIRROR>(s);
        s += dpp_f32<DPP_ROW_MIRROR>(s);
        s += __shfl_xor(s, 16, 64);
        if ((threadIdx.x & 31) == 0 && (threadIdx.x >> 5) < 16) part[threadIdx.x >> 5] = s;
        if constexpr (RAWBAR) {
            __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
            asm volatile("s_barrier" ::: "memory");
        } else {
            lds_barrier();
        }
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) sum += part[i];
        const float rms = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(sum, (float)k) + eps));
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            v[j].x = __fmul_rn(__fmul_rn(v[j].x, rms), wv[j].x);
            v[j].y = __fmul_rn(__fmul_rn(v[j].y, rms), wv[j].y);
            v[j].z = __fmul_rn(__fmul_rn(v[j].z, rms), wv[j].z);
            v[j].w = __fmul_rn(__fmul_rn(v[j].w, rms), wv[j].w);
        }
    }
    __device__ __forceinline__ void commit(const ActLds& a) {
        if constexpr (NORM) normalize();
        if (wave_live() && (int)threadIdx.x < slots()) quant_slot(a, threadIdx.x, v);
        if constexpr (SP == 2) {
            const int i = (int)(threadIdx.x + blockDim.x);
            if (i < slots()) quant_slot(a, i, v2);
        }
    }
    __device__ __forceinline__ void rest(const ActLds& a) const {
        for (int base = SP * blockDim.x; base < slots(); base += blockDim.x) {
            const int i = base + threadIdx.x;
            if (i < slots()) {
                f32x4 r[2];
                load_slot(i, r);
                quant_slot(a, i, r);
            }
        }
    }
};

// Up to three weight matrices of one type and row length that read the same activation rows
// (q, k and v; gate and up) run as one launch: virtual row j belongs to segment s with
// start[s] <= j < start[s + 1] and is row j - start[s] of w[s], its results going to y[s]
// (row stride rows[s]) plus bias[s]. Unused segments start at INT_MAX. The segment of a row
// is wave-uniform, so the picks below are scalar selects (an indexed read of the argument
// arrays would go through scratch memory).
struct GemvSegs {
    const uint8_t* w[3];
    float* y[3];
    const float* bias[3];
    int start[3];
    int rows[3];
    const float* norm_w;  // the RMSNorm weight of the NORM kernels, else null
    float eps;
};

__device__ __forceinline__ int seg_of(const GemvSegs& sg, int j) {
    return (j >= sg.start[1] ? 1 : 0) + (j >= sg.start[2] ? 1 : 0);
}
template <class V>
__device__ __forceinline__ V seg_pick(int s, V a, V b, V c) {
    return s == 0 ? a : (s == 1 ? b : c);
}

// Persistent GEMV: wave w owns rows j = w, w + n_waves, ...; items (row, 64-unit slice) are
// streamed through a P-deep ring of in-flight weight loads.
// Workgroup size: 8 waves share one staged (or quantized) activation batch for decode-sized
// batches (on MI355X 512 threads beat 1024 and 256 on the Q4_K 14336x4096 and Q6_K
// 128256x4096 decode shapes); with 4 or 8 activation rows the per-wave registers need the
// 256-VGPR budget of 4-wave workgroups.
template <int MR>
constexpr int gemv_threads() { return MR <= 2 ? 512 : 256; }

// With SW (the gate and up projections of a SwiGLU feed-forward, engine.cpp:509-512): segment 0
// is the gate matrix, segment 1 the up matrix, both of n rows; a wave takes row p of both in
// turn (row p of gate, then row p of up) and writes h[p] = silu(gate_p) * up_p to y[0] instead
// of the two projections, so the SwiGLU needs no launch of its own.
//
// With NORM (MR = 1, k <= 4096): the fp32 row x_f32 goes through the RMSNorm with weight
// sg.norm_w in the staging (StageQuant) before it is quantized.
template <uint32_t T, int MR, int P, bool SW = false, bool NORM = false>
__global__ __launch_bounds__(gemv_threads<MR>()) void k_gemv(GemvSegs sg, int64_t row_bytes,
                                              int k, int n, const int8_t* __restrict__ qs,
                                              const float* __restrict__ xs,
                                              const int32_t* __restrict__ xb,
                                              const float* __restrict__ x_f32, int accumulate) {
    using Tr = typename TraitsOf<T>::type;
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    constexpr int kWaves = gemv_threads<MR>() / 64;
    const int n_waves = gridDim.x * kWaves;
    const int wid = blockIdx.x * kWaves + wave;
    const int units = k / Tr::UNIT;
    const int iters = (units + 63) / 64;
    const int my_rows = (wid < n ? (n - 1 - wid) / n_waves + 1 : 0) * (SW ? 2 : 1);
    const int n_items = my_rows * iters;

    // Item i of this wave is row wid + (i / iters) * n_waves, unit slice i % iters (with SW,
    // row slot t = i / iters is row wid + (t / 2) n_waves of gate (t even) or up). Refills are
    // issued for every slot, with the item, row and unit clamped to valid memory (a wave with
    // no rows reads row n - 1), so the number of loads in flight is the same on every path
    // and the compiler's vmcnt waits only ever wait for the oldest slot.
    auto slot_addr = [&](int item, const uint8_t*& row, int& u) {
        const int c = max(0, min(item, n_items - 1));
        const int t = c / iters, it = c - t * iters;
        if constexpr (SW) {
            const int p = min(wid + (t >> 1) * n_waves, n - 1);
            row = ((t & 1) ? sg.w[1] : sg.w[0]) + (int64_t)p * row_bytes;
        } else {
            const int jr = min(wid + t * n_waves, n - 1);
            const int s = seg_of(sg, jr);
            row = seg_pick(s, sg.w[0], sg.w[1], sg.w[2]) +
                  (int64_t)(jr - seg_pick(s, sg.start[0], sg.start[1], sg.start[2])) * row_bytes;
        }
        u = min(lane + 64 * it, units - 1);
    };

    // Activation loads go out first, then the weight ring; the activations are written to LDS
    // once their own loads land (vmcnt counts in issue order), and the barrier orders LDS only,
    // so no wave waits for weight bytes before the first item's compute.
    const ActLds a = act_layout<T, MR>(lds, k);
    StageCopy<T, MR> sc{qs, xs, xb, k, {}, {}, {}};
    StageQuant<T, MR, NORM> sq{x_f32, k, {}};
    static_assert(!NORM || MR == 1, "the RMSNorm staging takes one row");
    __shared__ float norm_part[16];
    if constexpr (NORM) {
        sq.nw = sg.norm_w;
        sq.eps = sg.eps;
        sq.part = norm_part;
    }
    const bool fused = NORM || x_f32 != nullptr;
    if (fused)
        sq.issue();
    else
        sc.issue();
    __builtin_amdgcn_sched_barrier(0);

    typename Tr::Raw ring[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const uint8_t* row;
        int u;
        slot_addr(p, row, u);
        ring[p] = Tr::load(row, u);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (fused) {
        sq.commit(a);
        sq.rest(a);
    } else {
        sc.commit(a);
        sc.rest(a);
    }
    lds_barrier();
    if (n_items == 0) return;

    float acc[MR], gate_v[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[r] = gate_v[r] = 0.0f;

    const int n_pad = ((n_items + P - 1) / P) * P;
    for (int base = 0; base < n_pad; base += P) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int item = base + p;
            const int t = item / iters, it = item - t * iters;
            const int u = lane + 64 * it;
            {
                // Straight-line for every slot: padded items and lanes past the row's last
                // unit compute on clamped (valid) data and their result is dropped.
                float nacc[MR];
#pragma unroll
                for (int r = 0; r < MR; ++r) nacc[r] = acc[r];
                Tr::template compute<MR>(ring[p], min(u, units - 1), a, nacc);
                const bool keep = item < n_items && u < units;
#pragma unroll
                for (int r = 0; r < MR; ++r) acc[r] = keep ? nacc[r] : acc[r];
            }
            // With one slot every wait is vmcnt(0) anyway, so the refill is skipped past the
            // wave's last item instead of re-reading a clamped row (whose return would hold
            // the wave, and so the kernel's tail, for one more memory round trip).
            if (P > 1 || item + P < n_items) {
                const uint8_t* row;
                int u2;
                slot_addr(item + P, row, u2);
                ring[p] = Tr::load(row, u2);
            }
            if (SW && item < n_items && it == iters - 1) {
                const int j = __builtin_amdgcn_readfirstlane(wid + (t >> 1) * n_waves);
                const bool up = t & 1;
                const float* bias = up ? sg.bias[1] : sg.bias[0];
                const float bj = bias ? bias[j] : 0.0f;
#pragma unroll
                for (int r = 0; r < MR; ++r) {
                    float v = wave_sum(acc[r]);
                    if (bias) v += bj;
                    if (!up) {
                        gate_v[r] = v;
                    } else if (lane == r) {
                        sg.y[0][(size_t)r * sg.rows[0] + j] = silu_mul(gate_v[r], v);
                    }
                    acc[r] = 0.0f;
                }
            } else if (item < n_items && it == iters - 1) {
                const int jv = __builtin_amdgcn_readfirstlane(wid + t * n_waves);
                const int s = seg_of(sg, jv);
                const int j = jv - seg_pick(s, sg.start[0], sg.start[1], sg.start[2]);
                const float* bias = seg_pick(s, sg.bias[0], sg.bias[1], sg.bias[2]);
                float* y = seg_pick(s, sg.y[0], sg.y[1], sg.y[2]);
                const int ny = seg_pick(s, sg.rows[0], sg.rows[1], sg.rows[2]);
                const float bj = bias ? bias[j] : 0.0f;
#pragma unroll
                for (int r = 0; r < MR; ++r) {
                    float v = wave_sum(acc[r]);
                    if (bias) v += bj;
                    if (lane == r) {
                        float* yp = y + (size_t)r * ny + j;
                        *yp = accumulate ? *yp + v : v;  // residual add: x += (W a + b)
                    }
                    acc[r] = 0.0f;
                }
            }
        }
    }
}

// ------------------------------------------------------------ weight stream staged in LDS
// The same GEMV with the weight bytes routed through LDS. An item (a row's slice of 64 units:
// 16 K-quant super-blocks or 64 32-element blocks) is read as whole, aligned 16-byte pieces
// straight into one of the wave's S LDS slots (global_load_lds: piece 64 L + l of the item
// goes to lane l of wave-load L and lands at byte 16 (64 L + l) of the slot), so each load
// instruction reads 1 KB of contiguous memory, where k_gemv's per-unit field loads spread each
// instruction over 16 to 64 separate places of a row. The lanes then read their unit's fields
// from the slot and compute exactly as k_gemv. Items are cut into pieces starting at the
// 16-byte boundary at or below the item, so every read stays within 16-byte pieces that hold
// bytes of the matrix; lanes past an item's last piece stay idle, except lane 0, which reads
// the last piece again (into its own place, past the item) so that every item issues the
// same NL load instructions.
//
// The slots are private to their wave: no barrier orders them, only this wave's vmcnt. The
// loads of an item are its NL wave-loads, in order, and every item issues NL (the last items
// of a wave refill their slots with clamped, repeated items), so waiting until at most
// (S - 1) NL vector-memory operations are outstanding means the oldest slot has landed;
// stores issued in between only make that wait stricter.
template <class Tr>
__host__ __device__ constexpr int item_blocks() { return 64 / Tr::UNITS_PER_BLK; }
template <class Tr>
__host__ __device__ constexpr int item_pieces() {  // 16-byte pieces, a misaligned start included
    return (15 + item_blocks<Tr>() * Tr::BLK_BYTES - 1) / 16 + 1;
}
template <class Tr>
__host__ __device__ constexpr int item_loads() { return (item_pieces<Tr>() + 63) / 64; }
template <class Tr>
__host__ __device__ constexpr int slot_bytes() {
    return 16 * (item_pieces<Tr>() > 64 * (item_loads<Tr>() - 1) + 1 ? item_pieces<Tr>()
                                                                     : 64 * (item_loads<Tr>() - 1) + 1);
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt in bits 3:0 and 15:14, the other counters at max).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

// One wave-load of 16 bytes per lane from g into LDS at lds + 16 * lane (global_load_lds).
// Written as inline assembly so that the compiler does not track it: it would otherwise wait
// for every load in flight before each LDS read of the kernel, since it cannot tell which LDS
// bytes a load writes. The caller orders the reads with wait_vmcnt.
__device__ __forceinline__ void dma16(const void* g, const uint8_t* lds) {
    const uint32_t m0 = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)lds;
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" : : "v"(g), "s"(m0) : "memory", "m0");
}

template <uint32_t T, int MR, int S, int WV, bool NORM = false>
__global__ __launch_bounds__(64 * WV) void k_gemv_st(GemvSegs sg, int64_t row_bytes, int k, int n,
                                                     const int8_t* __restrict__ qs,
                                                     const float* __restrict__ xs,
                                                     const int32_t* __restrict__ xb,
                                                     const float* __restrict__ x_f32,
                                                     int accumulate) {
    using Tr = typename TraitsOf<T>::type;
    constexpr int NL = item_loads<Tr>();
    constexpr int BPI = item_blocks<Tr>();
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int n_waves = gridDim.x * WV;
    const int wid = blockIdx.x * WV + wave;
    const int units = k / Tr::UNIT;
    const int iters = (units + 63) / 64;
    const int nblk = units / Tr::UNITS_PER_BLK;
    const int my_rows = wid < n ? (n - 1 - wid) / n_waves + 1 : 0;
    const int n_items = my_rows * iters;
    constexpr int SLOT = slot_bytes<Tr>();
    __shared__ __align__(16) uint8_t slots[S * WV * SLOT];
    auto slot_ptr = [&](int p) { return slots + (p * WV + wave) * SLOT; };

    // First byte of item `item` (clamped to the wave's items; a wave with none reads row n-1).
    auto item_first = [&](int item, int& it) {
        const int c = max(0, min(item, n_items - 1));
        const int t = c / iters;
        it = c - t * iters;
        const int jr = min(wid + t * n_waves, n - 1);
        const int s = seg_of(sg, jr);
        const uint8_t* row = seg_pick(s, sg.w[0], sg.w[1], sg.w[2]) +
                             (int64_t)(jr - seg_pick(s, sg.start[0], sg.start[1], sg.start[2])) * row_bytes;
        return row + (size_t)(it * BPI) * Tr::BLK_BYTES;
    };
    auto issue = [&](int item, int slot) {
        int it;
        const uint8_t* first = item_first(item, it);
        const int mis = (int)((uintptr_t)first & 15u);
        const int last = (mis + min(BPI, nblk - it * BPI) * Tr::BLK_BYTES - 1) >> 4;
        const uint8_t* base = first - mis;
#pragma unroll
        for (int L = 0; L < NL; ++L) {
            const int c = 64 * L + lane;
            if (c <= last || lane == 0) dma16(base + 16 * min(c, last), slot_ptr(slot) + L * 1024);
        }
    };

    const ActLds a = act_layout<T, MR>(lds, k);
    StageCopy<T, MR> sc{qs, xs, xb, k, {}, {}, {}};
    StageQuant<T, MR, NORM, true> sq{x_f32, k, {}};
    static_assert(!NORM || MR == 1, "the RMSNorm staging takes one row");
    __shared__ float norm_part[16];
    if constexpr (NORM) {
        sq.nw = sg.norm_w;
        sq.eps = sg.eps;
        sq.part = norm_part;
    }
    const bool fused = NORM || x_f32 != nullptr;
    if (fused)
        sq.issue();
    else
        sc.issue();
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int p = 0; p < S; ++p) issue(p, p);
    __builtin_amdgcn_sched_barrier(0);
    if (fused) {
        sq.commit(a);
        sq.rest(a);
    } else {
        sc.commit(a);
        sc.rest(a);
    }
    // The activation rows are complete in LDS once every wave's LDS writes have: a fenced
    // barrier would also wait for the ring loads (LDS writes of this wave too).
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
    if (n_items == 0) {
        wait_vmcnt<0>();
        return;
    }

    float acc[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[r] = 0.0f;

    const int n_pad = ((n_items + S - 1) / S) * S;
    for (int base = 0; base < n_pad; base += S) {
#pragma unroll
        for (int p = 0; p < S; ++p) {
            const int item = base + p;
            const int t = item / iters, it = item - t * iters;
            const int u = lane + 64 * it;
            const bool row_end = item < n_items && it == iters - 1;
            wait_vmcnt<(S - 1) * NL>();
            __builtin_amdgcn_sched_barrier(0);
            {
                int itc;
                const int mis = (int)((uintptr_t)item_first(item, itc) & 15u);
                const int uc = min(u, units - 1) - 64 * itc;  // unit within the item
                const typename Tr::Raw raw = Tr::load_lds(
                    slot_ptr(p), mis + (uc / Tr::UNITS_PER_BLK) * Tr::BLK_BYTES, uc);
                float nacc[MR];
#pragma unroll
                for (int r = 0; r < MR; ++r) nacc[r] = acc[r];
                Tr::template compute<MR>(raw, min(u, units - 1), a, nacc);
                const bool keep = item < n_items && u < units;
#pragma unroll
                for (int r = 0; r < MR; ++r) acc[r] = keep ? nacc[r] : acc[r];
            }
            __builtin_amdgcn_sched_barrier(0);
            issue(item + S, p);
            // No vector-memory load in the loop but the ring's: one would have to be waited for
            // behind the refill just issued. The bias is read by a scalar load (the constant
            // address space; it is never written here) and the residual add is an atomic add
            // of the result (one wave owns the row, so it is the plain sum y + v).
            if (row_end) {
                const int jv = __builtin_amdgcn_readfirstlane(wid + t * n_waves);
                const int s = seg_of(sg, jv);
                const int j = jv - seg_pick(s, sg.start[0], sg.start[1], sg.start[2]);
                const float* bias = seg_pick(s, sg.bias[0], sg.bias[1], sg.bias[2]);
                float* y = seg_pick(s, sg.y[0], sg.y[1], sg.y[2]);
                const int ny = seg_pick(s, sg.rows[0], sg.rows[1], sg.rows[2]);
                const float bj = bias ? ((const __attribute__((address_space(4))) float*)bias)[j] : 0.0f;
#pragma unroll
                for (int r = 0; r < MR; ++r) {
                    const float v = wave_sum(acc[r]) + bj;
                    if (lane == r) {
                        float* yp = y + (size_t)r * ny + j;
                        if (accumulate)
                            __hip_atomic_fetch_add(yp, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        else
                            *yp = v;
                    }
                    acc[r] = 0.0f;
                }
            }
        }
    }
    wait_vmcnt<0>();  // the refills past the wave's last item land before its LDS is released
}

// ---------------------------------------------- decode stream, one item in flight per wave
// One activation row against a long weight stream, shaped for the HBM queues rather than for
// occupancy. A cold one-launch read of a matrix is bound by how many bytes are in flight:
// with F bytes requested the loads return after about max(L0, F / BW), so a whole matrix
// requested at once comes back all at the end (nothing for the arithmetic to overlap), and an
// activation row requested beside it waits its turn in the same queues. Here each wave keeps
// exactly one item in flight (one 16-wave workgroup per CU, the LDS request keeps a second one
// off: ~8 MB in flight over the device, about the bandwidth-latency product), the activation
// row goes out with the first item, and each step issues the next item's loads before it
// computes the current one.
//
// An item's bytes are read as whole, contiguous 16-byte pieces (nontemporal: each line is used
// once, by this load) into registers, then written to the wave's LDS slot, from which each lane
// reads its unit's fields as k_gemv does. The activation slices of the lane's units (one per
// item of a row, XR of them) are read from LDS once and kept in registers; XR = 0 reads them per
// unit. Measured on the Q4_K 14336 x 4096 decode step against the same kernel with
// direct-to-LDS item loads and per-unit activation reads: 7.8 against 9.9 us.
// FUSED: fp32 activation rows quantized here (x_f32), else a Q8_0 batch (qs, xs, xb). With
// XR > 0 the row is at most 8192 elements and the 1024 threads stage it in one pass; only
// XR = 0 has the staging's second pass (rest()), whose loads would otherwise make the compiler
// wait for every load in flight, the first item's included, after the staging.
//
// Rows are handed out inside the workgroup: workgroup b owns rows [b rpw, (b + 1) rpw), wave w
// starts with row b rpw + w and takes each further row from an LDS counter, one row ahead. A
// fixed share per wave would leave the workgroup waiting on its slowest waves: the CU does not
// serve its SIMDs' memory requests evenly (per-wave timestamps on the Q4_K 14336 x 4096 step:
// the last four waves of a workgroup ended 2.5 us after the first four).
//
// MR > 1: that many activation rows (a small batch) against the same stream, each lane keeping
// MR sums and reading the rows' slices of its unit from LDS per item (XR = 0).
template <uint32_t T, int WV, int XR, bool NORM, bool FUSED, int MR = 1>
__global__ __launch_bounds__(64 * WV) void k_gemv_str(GemvSegs sg, int64_t row_bytes, int k, int n,
                                                      int rpw, const int8_t* __restrict__ qs,
                                                      const float* __restrict__ xs,
                                                      const int32_t* __restrict__ xb,
                                                      const float* __restrict__ x_f32,
                                                      int accumulate) {
    using Tr = typename TraitsOf<T>::type;
    constexpr int NL = item_loads<Tr>();
    constexpr int BPI = item_blocks<Tr>();
    constexpr int SLOT = slot_bytes<Tr>();
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int next_row;  // rows of this workgroup handed out so far
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int units = k / Tr::UNIT;
    const int iters = (units + 63) / 64;
    const int nblk = units / Tr::UNITS_PER_BLK;
    static_assert(MR == 1 || (XR == 0 && !NORM), "several rows: slices read per unit, no RMSNorm");
    const int r0 = blockIdx.x * rpw;
    const int r_end = min(n, r0 + rpw);
    uint8_t* slot = lds + align16(act_lds_bytes<T>(MR, k)) + (size_t)wave * SLOT;

    // First byte of item `it` of row jr.
    auto item_first = [&](int jr, int it) {
        const int s = seg_of(sg, jr);
        const uint8_t* row = seg_pick(s, sg.w[0], sg.w[1], sg.w[2]) +
                             (int64_t)(jr - seg_pick(s, sg.start[0], sg.start[1], sg.start[2])) * row_bytes;
        return row + (size_t)(it * BPI) * Tr::BLK_BYTES;
    };
    // The item's 16-byte pieces from the one at or below its first byte: piece 64 L + lane to
    // pc[L] (lanes past the last piece load the last one again: straight-line loads, so the
    // compiler counts exactly NL per item in its waits). dep is an opaque zero.
    u32x4 pc[NL];
    auto load_item = [&](int jr, int it, uint32_t dep) {
        const uint8_t* first = item_first(jr, it);
        const int mis = (int)((uintptr_t)first & 15u);
        const int last = (mis + min(BPI, nblk - it * BPI) * Tr::BLK_BYTES - 1) >> 4;
        const u32x4* base = (const u32x4*)(first - mis + dep);
#pragma unroll
        for (int L = 0; L < NL; ++L)
            pc[L] = __builtin_nontemporal_load(base + min(64 * L + lane, last));
    };
    auto to_slot = [&](int jr, int it) {
        const uint8_t* first = item_first(jr, it);
        const int mis = (int)((uintptr_t)first & 15u);
        const int last = (mis + min(BPI, nblk - it * BPI) * Tr::BLK_BYTES - 1) >> 4;
#pragma unroll
        for (int L = 0; L < NL; ++L)
            if (64 * L + lane <= last) *(u32x4*)(slot + 16 * (64 * L + lane)) = pc[L];
        return mis;
    };
    // The next row of this workgroup, -1 when they are all handed out.
    auto grab = [&]() {
        int c = 0;
        if (lane == 0) c = __hip_atomic_fetch_add(&next_row, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        c = __builtin_amdgcn_readfirstlane(c);
        return r0 + c < r_end ? r0 + c : -1;
    };

    const ActLds a = act_layout<T, MR>(lds, k);
    // several rows, or rows longer than 8192, stage two slots per thread up front: a second
    // pass would issue its loads after item 0's, and waiting for them would wait for the item
    // too (the RMSNorm staging takes rows of at most 4096)
    StageQuant<T, MR, NORM, false, ((MR >= 2 || XR == 0) && !NORM ? 2 : 1)> sq{x_f32, k, {}};
    StageCopy<T, MR> sc{qs, xs, xb, k, {}, {}, {}};
    __shared__ float norm_part[16];
    if constexpr (NORM) {
        sq.nw = sg.norm_w;
        sq.eps = sg.eps;
        sq.part = norm_part;
    }
    if (threadIdx.x == 0) next_row = WV;
    int row = r0 + wave < r_end ? r0 + wave : -1;
    // The activation loads and item 0 fly together; the activation is waited for alone. Every
    // wave loads an item 0 (a wave with no row that of row r0, which every workgroup owns),
    // so the path to the staging has no branch: behind the fence the item loads are the last
    // NL issued, and the compiler's wait before the staging reads the activation is vmcnt(NL).
    static_assert(!NORM || FUSED, "the RMSNorm staging quantizes an fp32 row");
    if constexpr (FUSED)
        sq.issue_all();
    else
        sc.issue();
    // LATE: item 0 goes out once the activation is staged, so that the staging's loads do not
    // share the device's first burst of weight requests (the fused quantization, several
    // rows, and rows longer than 8192 gained; one pre-quantized row of 4096 lost, and so did
    // one fused Q5_K row of 4096 by 0.1 us)
    constexpr bool LATE = (FUSED || MR >= 2 || XR == 0) && !NORM && !(T == T_Q5_K && MR == 1 && XR > 0);
    const uint32_t dep0 = FUSED ? opaque_zero(x_f32, sg.norm_w) : opaque_zero(qs, xs, xb);
    if constexpr (!LATE) load_item(row >= 0 ? row : r0, 0, dep0);
    if constexpr (FUSED) {
        sq.commit(a);
        if constexpr (XR == 0) sq.rest(a);
    } else {
        sc.commit(a);
        if constexpr (XR == 0) sc.rest(a);
    }
    if constexpr (LATE) load_item(row >= 0 ? row : r0, 0, dep0);
    lds_barrier();  // also publishes next_row
    if (row < 0) return;

    // the activation slices of this lane's units, one per item of a row
    typename Tr::X xr[XR > 0 ? XR : 1];
#pragma unroll
    for (int i = 0; i < XR; ++i) xr[i] = Tr::x_of(a, 0, min(lane + 64 * i, units - 1));

    int it = 0;
    int nrow = grab();  // the row after the current one
    float acc[MR];
#pragma unroll
    for (int t = 0; t < MR; ++t) acc[t] = 0.0f;
    while (row >= 0) {
        const int u = min(lane + 64 * it, units - 1);
        const int mis = to_slot(row, it);
        // issue the next item: the current row's next one, or the first of the next row
        const bool last_item = it == iters - 1;
        const int frow = last_item ? nrow : row, fit = last_item ? 0 : it + 1;
        if (frow >= 0) load_item(frow, fit, 0u);
        int nnrow = nrow;
        if (last_item && nrow >= 0) nnrow = grab();
        {
            const int uc = u - 64 * it;  // unit within the item
            const typename Tr::Raw raw =
                Tr::load_lds(slot, mis + (uc / Tr::UNITS_PER_BLK) * Tr::BLK_BYTES, uc);
            const typename Tr::W w = Tr::wdec(raw, u);
            float v[MR];
            if constexpr (XR > 0) {
                typename Tr::X x = xr[0];
#pragma unroll
                for (int i = 1; i < XR; ++i)
                    if (it == i) x = xr[i];
                v[0] = Tr::fin(w, x, acc[0], u);
            } else {
#pragma unroll
                for (int t = 0; t < MR; ++t) v[t] = Tr::fin(w, Tr::x_of(a, t, u), acc[t], u);
            }
#pragma unroll
            for (int t = 0; t < MR; ++t) acc[t] = lane + 64 * it < units ? v[t] : acc[t];
        }
        if (last_item) {
            const int s = seg_of(sg, row);
            const int j = row - seg_pick(s, sg.start[0], sg.start[1], sg.start[2]);
            const float* bias = seg_pick(s, sg.bias[0], sg.bias[1], sg.bias[2]);
            float* y = seg_pick(s, sg.y[0], sg.y[1], sg.y[2]);
            const int ny = seg_pick(s, sg.rows[0], sg.rows[1], sg.rows[2]);
            const float bj = bias ? ((const __attribute__((address_space(4))) float*)bias)[j] : 0.0f;
#pragma unroll
            for (int t = 0; t < MR; ++t) {
                float v = wave_sum63(acc[t]);  // the same additions as wave_sum's, in lane 63
                if (bias) v += bj;
                // the residual add as an atomic (one wave owns the row, so it is the plain sum
                // y + v): a load of y here would wait behind the next item's loads
                if (lane == 63) {
                    float* yp = y + (size_t)t * ny + j;
                    if (accumulate)
                        __hip_atomic_fetch_add(yp, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    else
                        *yp = v;
                }
                acc[t] = 0.0f;
            }
            row = nrow;
            nrow = nnrow;
            it = 0;
        } else {
            ++it;
        }
    }
}

static int g_cu_count = 0;

static int cu_count() {
    if (g_cu_count == 0) {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
            cus > 0)
            g_cu_count = cus;
        else
            g_cu_count = 256;
    }
    return g_cu_count;
}

// Launch shape, from sweeps on MI355X (cold HBM, fused quantization). With one or two
// activation rows, one item in flight per wave and as many waves as stay resident beat every
// deeper ring, on the short stream and on the long one: Q4_K 14336x4096 took 8.0 us against
// 8.8-10.6 us for 2- and 4-deep rings (rows strided or blocked per wave), the Q6_K
// 128256x4096 head 81 us against 88-96 us for the 2-deep ring at 4 waves per SIMD. More
// loads in flight per wave lost even when every extra load was useful. With 4 or 8 rows,
// streams longer than 32 items per SIMD use the 2-deep ring at 4 waves per SIMD.
// The tuning knob "gemv_waves" (cllm_hip_tune) caps the waves per SIMD of the two rings for
// sweeps. The grid never exceeds the waves resident at once.
struct GemvTuning {
    int short_wps = 8;
    int deep_wps = 4;
};

static GemvTuning gemv_tuning() {
    GemvTuning r;
    const int a = tuning().gemv_short_wps.load(std::memory_order_relaxed);
    const int b = tuning().gemv_deep_wps.load(std::memory_order_relaxed);
    if (a >= 1 && a <= 16) r.short_wps = a;
    if (b >= 1 && b <= 16) r.deep_wps = b;
    return r;
}

// Waves of k_gemv<T, MR, P> resident on the whole device with `shmem` bytes of LDS per
// workgroup (cached per instantiation for the last LDS size asked).
template <uint32_t T, int MR, int P, bool SW = false, bool NORM = false>
static int64_t resident_waves(size_t shmem) {
    static std::atomic<uint64_t> cache{0};  // (shmem << 16) | workgroups per CU, 0 = empty
    uint64_t c = cache.load(std::memory_order_relaxed);
    int blocks;
    if (c != 0 && (c >> 16) == shmem) {
        blocks = (int)(c & 0xFFFFu);
    } else {
        blocks = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, reinterpret_cast<const void*>(&k_gemv<T, MR, P, SW, NORM>),
                                                         gemv_threads<MR>(), shmem) != hipSuccess ||
            blocks < 1)
            blocks = 1;
        cache.store(((uint64_t)shmem << 16) | (uint64_t)(blocks & 0xFFFF), std::memory_order_relaxed);
    }
    return (int64_t)blocks * (gemv_threads<MR>() / 64) * cu_count();
}

// The LDS-staged stream, one slot per wave, 16 waves per workgroup (from sweeps on MI355X,
// cold HBM, fused quantization: the Q6_K 128256x4096 head 72 us against 73-78 us for 8-wave
// workgroups at 3-4 per CU and 78-81 us with two slots; the register-ring k_gemv 81-88 us on
// the same boxes). Grid: the workgroups resident at once, or fewer if the rows run out.
template <uint32_t T, int S, int WV, bool NORM = false>
static int64_t resident_st_wgs(size_t shmem) {
    static std::atomic<uint64_t> cache{0};
    uint64_t c = cache.load(std::memory_order_relaxed);
    int blocks;
    if (c != 0 && (c >> 16) == shmem) {
        blocks = (int)(c & 0xFFFFu);
    } else {
        blocks = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, reinterpret_cast<const void*>(&k_gemv_st<T, 1, S, WV, NORM>),
                                                         64 * WV, shmem) != hipSuccess ||
            blocks < 1)
            blocks = 1;
        cache.store(((uint64_t)shmem << 16) | (uint64_t)(blocks & 0xFFFF), std::memory_order_relaxed);
    }
    return (int64_t)blocks * cu_count();
}

template <uint32_t T, int S, int WV, bool NORM = false>
static hipError_t launch_st(const GemvSegs& sg, int k, int n, const int8_t* qs, const float* xs,
                            const int32_t* xb, const float* x_f32, int accumulate, int64_t items,
                            hipStream_t stream) {
    const int64_t row_bytes = (int64_t)(k / block_elems(T)) * (int64_t)block_bytes(T);
    const size_t shmem = act_lds_bytes<T>(1, k);
    const int64_t grid = std::min((items + WV - 1) / WV, resident_st_wgs<T, S, WV, NORM>(shmem));
    hipLaunchKernelGGL((k_gemv_st<T, 1, S, WV, NORM>), dim3((unsigned)grid), dim3(64 * WV), shmem,
                       stream, sg, row_bytes, k, n, qs, xs, xb, x_f32, accumulate);
    return hipGetLastError();
}

// The streaming kernel: 16-wave workgroups, at most one per CU (the LDS request is at least
// kStrMinLds, more than half a CU's 160 KB), the rows split evenly over them.
constexpr int kStrWaves = 16;
constexpr int kStrMaxRows = 8;  // activation rows of one streaming launch
constexpr size_t kStrMinLds = 96 * 1024;

template <uint32_t T>
__host__ constexpr size_t str_lds_bytes(int k, int mr = 1) {
    using Tr = typename TraitsOf<T>::type;
    return align16(act_lds_bytes<T>(mr, k)) + (size_t)kStrWaves * slot_bytes<Tr>();
}

template <uint32_t T, int XR, bool NORM, bool FUSED, int MR = 1>
static hipError_t launch_str_k(const GemvSegs& sg, int k, int n, const int8_t* qs, const float* xs,
                               const int32_t* xb, const float* x_f32, int accumulate,
                               hipStream_t stream) {
    const int64_t row_bytes = (int64_t)(k / block_elems(T)) * (int64_t)block_bytes(T);
    const size_t shmem = std::max(str_lds_bytes<T>(k, MR), kStrMinLds);
    // the attribute covers the largest LDS request this instantiation makes (k up to what
    // str_fits admits)
    static bool attr_set = false;
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute((const void*)k_gemv_str<T, kStrWaves, XR, NORM, FUSED, MR>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, 150 * 1024);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    // one workgroup per CU (fewer for a short matrix: at least one row per wave), rows split
    // evenly (the tuning knob "gemv_str_grid" overrides the count)
    int64_t grid = std::min<int64_t>(cu_count(), (n + kStrWaves - 1) / kStrWaves);
    const int force = tuning().gemv_str_grid.load(std::memory_order_relaxed);
    if (force > 0) grid = force;
    const int rpw = (int)((n + grid - 1) / grid);
    grid = (n + rpw - 1) / rpw;
    hipLaunchKernelGGL((k_gemv_str<T, kStrWaves, XR, NORM, FUSED, MR>), dim3((unsigned)grid),
                       dim3(64 * kStrWaves), shmem, stream, sg, row_bytes, k, n, rpw, qs, xs, xb,
                       x_f32, accumulate);
    return hipGetLastError();
}

template <uint32_t T, int XR, bool NORM>
static hipError_t launch_str_x(const GemvSegs& sg, int k, int n, const int8_t* qs, const float* xs,
                               const int32_t* xb, const float* x_f32, int accumulate,
                               hipStream_t stream) {
    if (NORM || x_f32 != nullptr)
        return launch_str_k<T, XR, NORM, true>(sg, k, n, qs, xs, xb, x_f32, accumulate, stream);
    if constexpr (!NORM)
        return launch_str_k<T, XR, false, false>(sg, k, n, qs, xs, xb, x_f32, accumulate, stream);
    return hipErrorInvalidValue;
}

// Rows of one or two items keep the activation slices in registers; longer rows read them per
// unit (their slices would not fit beside the item pieces).
template <uint32_t T, bool NORM = false>
static hipError_t launch_str(const GemvSegs& sg, int k, int n, const int8_t* qs, const float* xs,
                             const int32_t* xb, const float* x_f32, int accumulate, int64_t,
                             hipStream_t stream) {
    using Tr = typename TraitsOf<T>::type;
    const int iters = (k / Tr::UNIT + 63) / 64;
    if (iters == 1) return launch_str_x<T, 1, NORM>(sg, k, n, qs, xs, xb, x_f32, accumulate, stream);
    if (iters == 2) return launch_str_x<T, 2, NORM>(sg, k, n, qs, xs, xb, x_f32, accumulate, stream);
    return launch_str_x<T, 0, NORM>(sg, k, n, qs, xs, xb, x_f32, accumulate, stream);
}

template <uint32_t T>
static bool str_fits(int k, int mr = 1) { return str_lds_bytes<T>(k, mr) <= 150 * 1024; }

// A small batch (2 to kStrMaxRows rows) on the streaming kernel, from fp32 rows or a
// quantized batch.
template <uint32_t T, int MR>
static hipError_t launch_str_rows(const GemvSegs& sg, int k, int n, const int8_t* qs,
                                  const float* xs, const int32_t* xb, const float* x_f32,
                                  int accumulate, hipStream_t stream) {
    if (x_f32 != nullptr)
        return launch_str_k<T, 0, false, true, MR>(sg, k, n, qs, xs, xb, x_f32, accumulate, stream);
    return launch_str_k<T, 0, false, false, MR>(sg, k, n, qs, xs, xb, x_f32, accumulate, stream);
}

// The streaming kernel takes one activation row over a stream of at least 4 MiB; shorter
// streams fill too few workgroups of 16 rows each and keep the register ring (MI355X, cold
// HBM: Q4_K 1024x4096, 2.4 MB, 3.85 against 3.24 us; Q8_0 4864x896, 4.7 MB, 3.90 against
// 4.37 us).
template <uint32_t T>
static bool use_str(int k, int n) {
    const int64_t bytes = (int64_t)n * (k / block_elems(T)) * block_bytes(T);
    return bytes >= (4ll << 20) && str_fits<T>(k);
}

// Decode streams of at least this many weight bytes take the LDS-staged kernel: its contiguous
// nontemporal loads win on long streams and lose on short ones, where its extra startup shows.
// Q6_K: the 128256x4096 head (431 MB) 72-80 against 81-88 us, the 4096x14336 FFN down matrix
// (48 MB) 15.5 against 18.2 us, 4096x4096 (14 MB) 6.5 against 6.1 us. Q4_K: 128256x4096
// (295 MB) 52 against 57 us, 14336x4096 (33 MB) 10.1 against 9.1 us. More slots per wave
// (all of a short stream's items in flight from the start) lost everywhere: Q4_K 14336x4096
// took 12.8 / 15.4 / 13.7 us with 2 / 3 / 4 slots.
template <uint32_t T>
constexpr int64_t staged_min_bytes() { return T == T_Q6_K ? 32ll << 20 : T == T_Q4_K ? 96ll << 20 : INT64_MAX; }

// One activation row over a long Q6_K / Q4_K stream takes the staged kernel (Q4_K's LDS field
// reads are whole 16-byte pieces: its rows must start 16-byte aligned).
template <uint32_t T>
static bool use_staged(const GemvSegs& sg, int k, int n) {
    if constexpr (T != T_Q6_K && T != T_Q4_K) return false;
    const int64_t bytes = (int64_t)n * (k / block_elems(T)) * block_bytes(T);
    bool aligned = true;
    if constexpr (T == T_Q4_K)
        for (int i = 0; i < 3; ++i) aligned = aligned && ((uintptr_t)sg.w[i] & 15u) == 0;
    return bytes >= staged_min_bytes<T>() && aligned && act_lds_bytes<T>(1, k) <= 64 * 1024;
}

template <uint32_t T, int MR, int P, bool SW, bool NORM = false>
static hipError_t launch_t(const GemvSegs& sg, int k, int n, const int8_t* qs, const float* xs,
                           const int32_t* xb, const float* x_f32, int accumulate, int waves,
                           hipStream_t stream) {
    const int64_t row_bytes = (int64_t)(k / block_elems(T)) * (int64_t)block_bytes(T);
    if (waves > n) waves = n;
    constexpr int kWaves = gemv_threads<MR>() / 64;
    const int grid = (waves + kWaves - 1) / kWaves;
    const size_t shmem = act_lds_bytes<T>(MR, k);
    hipLaunchKernelGGL((k_gemv<T, MR, P, SW, NORM>), dim3(grid), dim3(gemv_threads<MR>()), shmem, stream, sg,
                       row_bytes, k, n, qs, xs, xb, x_f32, accumulate);
    return hipGetLastError();
}

// Most activation rows one launch stages in LDS for this type and k (1, 2, 4 or 8).
template <uint32_t T>
static int max_rows_per_launch(int k) {
    constexpr size_t kLdsBudget = 48 * 1024;
    int mr = 8;
    while (mr > 1 && act_lds_bytes<T>(mr, k) > kLdsBudget) mr /= 2;
    return mr;
}

// SW: n is the row count of each of the two matrices (gate and up), whose rows pair up.
template <uint32_t T, int MR, bool SW>
static hipError_t launch_mr(const GemvSegs& sg, int k, int n, const int8_t* qs, const float* xs,
                            const int32_t* xb, const float* x_f32, int accumulate,
                            hipStream_t stream) {
    using Tr = typename TraitsOf<T>::type;
    const int iters = (k / Tr::UNIT + 63) / 64;
    const int64_t items = (int64_t)n * iters * (SW ? 2 : 1);
    const int64_t simds = (int64_t)cu_count() * 4;
    const GemvTuning tu = gemv_tuning();
    const size_t shmem = act_lds_bytes<T>(MR, k);
    // one activation row: the streaming kernel (tuning knob "gemv_kernel": 0 the default,
    // 1 the register ring k_gemv, 2 the staged k_gemv_st, 3 k_gemv_str)
    const int kind = tuning().gemv_kind.load(std::memory_order_relaxed);
    if constexpr (MR == 1 && !SW) {
        if ((kind == 0 && use_str<T>(k, n)) || (kind == 3 && str_fits<T>(k))) {
            if (sg.norm_w) return launch_str<T, true>(sg, k, n, qs, xs, xb, x_f32, accumulate, items, stream);
            return launch_str<T, false>(sg, k, n, qs, xs, xb, x_f32, accumulate, items, stream);
        }
    }
    if constexpr (MR == 1) {
        if (sg.norm_w) {  // the RMSNorm rides in the staging (one row)
            if constexpr ((T == T_Q6_K || T == T_Q4_K) && !SW)
                if (kind == 2 || (kind == 0 && use_staged<T>(sg, k, n)))
                    return launch_st<T, 1, 16, true>(sg, k, n, qs, xs, xb, x_f32, accumulate, items,
                                                     stream);
            const int64_t waves =
                std::min({items, simds * tu.short_wps, resident_waves<T, 1, 1, SW, true>(shmem)});
            return launch_t<T, 1, 1, SW, true>(sg, k, n, qs, xs, xb, x_f32, accumulate, (int)waves,
                                               stream);
        }
    }
    if constexpr ((T == T_Q6_K || T == T_Q4_K) && MR == 1 && !SW)
        if (kind == 2 || (kind == 0 && use_staged<T>(sg, k, n)))
            return launch_st<T, 1, 16>(sg, k, n, qs, xs, xb, x_f32, accumulate, items, stream);
    if (MR > 2 && items > simds * 32) {
        const int64_t waves = std::min(simds * tu.deep_wps, resident_waves<T, MR, 2, SW>(shmem));
        return launch_t<T, MR, 2, SW>(sg, k, n, qs, xs, xb, x_f32, accumulate, (int)waves, stream);
    }
    const int64_t waves = std::min({items, simds * tu.short_wps, resident_waves<T, MR, 1, SW>(shmem)});
    return launch_t<T, MR, 1, SW>(sg, k, n, qs, xs, xb, x_f32, accumulate, (int)waves, stream);
}

template <uint32_t T, bool SW>
static hipError_t launch_rows(const GemvSegs& sg, int k, int n, int mr, const int8_t* qs,
                              const float* xs, const int32_t* xb, const float* x_f32, int acc,
                              hipStream_t stream) {
    switch (mr) {
        case 1: return launch_mr<T, 1, SW>(sg, k, n, qs, xs, xb, x_f32, acc, stream);
        case 2: return launch_mr<T, 2, SW>(sg, k, n, qs, xs, xb, x_f32, acc, stream);
        case 4: return launch_mr<T, 4, SW>(sg, k, n, qs, xs, xb, x_f32, acc, stream);
        default: return launch_mr<T, 8, SW>(sg, k, n, qs, xs, xb, x_f32, acc, stream);
    }
}

// Rows of the next launch with `left` activation rows to go: 8, 4, 2 or 1, halved down to
// what one launch's LDS holds (`lim`, max_rows_per_launch).
static int next_launch_rows(int left, int lim) {
    int mr = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
    while (mr > lim) mr /= 2;
    return mr;
}

// 2 to 8 activation rows over a long stream run as one launch of the streaming kernel with
// that many sums per lane (MI355X, cold HBM, us, against the register ring k_gemv: Q5_K
// 14336x4096 at 2 / 4 rows 11.0 / 15.6 against 13.1 / 17.7, Q8_0 4096x4096 6.1 / 8.6 against
// 7.6 / 10.1, Q6_K 4096x14336 at 2 rows 15.1 against 20.1; results bit for bit the same).
template <uint32_t T>
static bool str_whole_batch(int k, int n, int m) {
    if (m < 2 || m > kStrMaxRows || !str_fits<T>(k, m)) return false;
    const int kind = tuning().gemv_kind.load(std::memory_order_relaxed);
    return (kind == 0 && use_str<T>(k, n)) || kind == 3;
}

template <uint32_t T>
static hipError_t launch_str_batch(const GemvSegs& sg, int k, int n, int m, const int8_t* qs,
                                   const float* xs, const int32_t* xb, const float* x_f32,
                                   int acc, hipStream_t stream) {
    switch (m) {
        case 2: return launch_str_rows<T, 2>(sg, k, n, qs, xs, xb, x_f32, acc, stream);
        case 3: return launch_str_rows<T, 3>(sg, k, n, qs, xs, xb, x_f32, acc, stream);
        case 4: return launch_str_rows<T, 4>(sg, k, n, qs, xs, xb, x_f32, acc, stream);
        case 5: return launch_str_rows<T, 5>(sg, k, n, qs, xs, xb, x_f32, acc, stream);
        case 6: return launch_str_rows<T, 6>(sg, k, n, qs, xs, xb, x_f32, acc, stream);
        case 7: return launch_str_rows<T, 7>(sg, k, n, qs, xs, xb, x_f32, acc, stream);
        case 8: return launch_str_rows<T, 8>(sg, k, n, qs, xs, xb, x_f32, acc, stream);
        default: return hipErrorInvalidValue;
    }
}

// Runs every activation row through the GEMV, MR rows per launch (or all of a small batch in
// one streaming launch). With x_f32 set, the rows are fp32 and each launch quantizes its rows
// itself (qs / scales / bsums unused).
template <uint32_t T, bool SW = false>
static hipError_t gemv_all_rows(const GemvSegs& sg0, int k, int n, int m, const int8_t* qs,
                                const float* scales, const int32_t* bsums, const float* x_f32,
                                int acc, hipStream_t stream) {
    if (!SW && !sg0.norm_w && str_whole_batch<T>(k, n, m))
        return launch_str_batch<T>(sg0, k, n, m, qs, scales, bsums, x_f32, acc, stream);
    const int nb = k / 32;
    const int cap = max_rows_per_launch<T>(k);
    int t = 0;
    while (t < m) {
        const int mr = next_launch_rows(m - t, cap);
        GemvSegs sg = sg0;
        for (int i = 0; i < 3; ++i) sg.y[i] = sg0.y[i] + (size_t)t * sg0.rows[i];
        const hipError_t e = launch_rows<T, SW>(
            sg, k, n, mr, qs ? qs + (size_t)t * k : nullptr, scales ? scales + (size_t)t * nb : nullptr,
            bsums ? bsums + (size_t)t * nb : nullptr, x_f32 ? x_f32 + (size_t)t * k : nullptr, acc,
            stream);
        if (e != hipSuccess) return e;
        t += mr;
    }
    return hipSuccess;
}

// Launches gemv_all_rows makes for m activation rows (each streams the whole matrix) when it
// takes the register ring (k_gemv).
template <uint32_t T>
static int launches_for(int k, int m) {
    const int lim = max_rows_per_launch<T>(k);
    int launches = 0;
    for (int t = 0; t < m; ++launches) t += next_launch_rows(m - t, lim);
    return launches;
}

// The kernel gemv_all_rows runs first for m activation rows, and its launch count; weights
// taken as 16-byte aligned.
template <uint32_t T>
static void plan_rows(const char* tname, int k, int n, int m, char* buf, size_t cap) {
    if (str_whole_batch<T>(k, n, m)) {
        snprintf(buf, cap, "k_gemv_str<%s,%d> launches=1", tname, m);
        return;
    }
    const int mr0 = m > 0 ? next_launch_rows(m, max_rows_per_launch<T>(k)) : 0;
    const int launches = launches_for<T>(k, m);
    const int kind = tuning().gemv_kind.load(std::memory_order_relaxed);
    const int64_t bytes = (int64_t)n * (k / block_elems(T)) * block_bytes(T);
    const char* name = "k_gemv";
    if (mr0 == 1 && ((kind == 0 && use_str<T>(k, n)) || (kind == 3 && str_fits<T>(k))))
        name = "k_gemv_str";
    else if (mr0 == 1 && (T == T_Q6_K || T == T_Q4_K) &&
             (kind == 2 || (kind == 0 && bytes >= staged_min_bytes<T>() &&
                            act_lds_bytes<T>(1, k) <= 64 * 1024)))
        name = "k_gemv_st";
    snprintf(buf, cap, "%s<%s,%d> launches=%d", name, tname, mr0, launches);
}

bool gemv_streams_batch(uint32_t type, int k, int n, int m) {
    switch (type) {
        case T_Q4_K: return str_whole_batch<T_Q4_K>(k, n, m);
        case T_Q5_K: return str_whole_batch<T_Q5_K>(k, n, m);
        case T_Q6_K: return str_whole_batch<T_Q6_K>(k, n, m);
        case T_Q8_0: return str_whole_batch<T_Q8_0>(k, n, m);
        case T_Q4_0: return str_whole_batch<T_Q4_0>(k, n, m);
        case T_Q5_0: return str_whole_batch<T_Q5_0>(k, n, m);
        default: return false;
    }
}

int gemv_launch_count(uint32_t type, int k, int m) {
    switch (type) {
        case T_Q4_K: return launches_for<T_Q4_K>(k, m);
        case T_Q5_K: return launches_for<T_Q5_K>(k, m);
        case T_Q6_K: return launches_for<T_Q6_K>(k, m);
        case T_Q8_0: return launches_for<T_Q8_0>(k, m);
        case T_Q4_0: return launches_for<T_Q4_0>(k, m);
        case T_Q5_0: return launches_for<T_Q5_0>(k, m);
        default: return 1;
    }
}

void gemv_plan_name(uint32_t type, int k, int n, int m, char* buf, size_t cap) {
    switch (type) {
        case T_Q4_K: return plan_rows<T_Q4_K>("Q4_K", k, n, m, buf, cap);
        case T_Q5_K: return plan_rows<T_Q5_K>("Q5_K", k, n, m, buf, cap);
        case T_Q6_K: return plan_rows<T_Q6_K>("Q6_K", k, n, m, buf, cap);
        case T_Q8_0: return plan_rows<T_Q8_0>("Q8_0", k, n, m, buf, cap);
        case T_Q4_0: return plan_rows<T_Q4_0>("Q4_0", k, n, m, buf, cap);
        case T_Q5_0: return plan_rows<T_Q5_0>("Q5_0", k, n, m, buf, cap);
        default: snprintf(buf, cap, "none");
    }
}

static hipError_t gemv_dispatch(uint32_t type, const GemvSegs& sg, int k, int n, int m,
                                const int8_t* qs, const float* scales, const int32_t* bsums,
                                const float* x_f32, int acc, hipStream_t stream) {
    switch (type) {
        case T_Q4_K: return gemv_all_rows<T_Q4_K>(sg, k, n, m, qs, scales, bsums, x_f32, acc, stream);
        case T_Q5_K: return gemv_all_rows<T_Q5_K>(sg, k, n, m, qs, scales, bsums, x_f32, acc, stream);
        case T_Q6_K: return gemv_all_rows<T_Q6_K>(sg, k, n, m, qs, scales, bsums, x_f32, acc, stream);
        case T_Q8_0: return gemv_all_rows<T_Q8_0>(sg, k, n, m, qs, scales, bsums, x_f32, acc, stream);
        case T_Q4_0: return gemv_all_rows<T_Q4_0>(sg, k, n, m, qs, scales, bsums, x_f32, acc, stream);
        case T_Q5_0: return gemv_all_rows<T_Q5_0>(sg, k, n, m, qs, scales, bsums, x_f32, acc, stream);
        default: return hipErrorInvalidValue;
    }
}

static GemvSegs one_segment(const uint8_t* w, int n, const float* bias, float* y) {
    GemvSegs sg;
    for (int i = 0; i < 3; ++i) {
        sg.w[i] = w;
        sg.y[i] = y;
        sg.bias[i] = bias;
        sg.start[i] = i == 0 ? 0 : INT_MAX;
        sg.rows[i] = n;
    }
    sg.norm_w = nullptr;
    sg.eps = 0.0f;
    return sg;
}

hipError_t launch_gemv(uint32_t type, const uint8_t* w, int k, int n, int m, const int8_t* qs,
                       const float* scales, const int32_t* bsums, const float* bias, float* y,
                       hipStream_t stream, bool accumulate) {
    return gemv_dispatch(type, one_segment(w, n, bias, y), k, n, m, qs, scales, bsums, nullptr,
                         accumulate ? 1 : 0, stream);
}

// q/k/v (or any 1 to 3 matrices) as segments of one launch.
static hipError_t multi_segs(int n_mats, const uint8_t* const* w, const int* n,
                             const float* const* bias, float* const* y, GemvSegs& sg, int& total) {
    if (n_mats < 1 || n_mats > 3) return hipErrorInvalidValue;
    sg = one_segment(w[0], n[0], bias ? bias[0] : nullptr, y[0]);
    total = 0;
    for (int i = 0; i < n_mats; ++i) {
        sg.w[i] = w[i];
        sg.y[i] = y[i];
        sg.bias[i] = bias ? bias[i] : nullptr;
        sg.start[i] = total;
        sg.rows[i] = n[i];
        if (n[i] < 0 || (int64_t)total + n[i] > INT_MAX / 2) return hipErrorInvalidValue;
        total += n[i];
    }
    return hipSuccess;
}

hipError_t launch_gemv_multi(uint32_t type, int k, int n_mats, const uint8_t* const* w,
                             const int* n, const float* const* bias, float* const* y, int m,
                             const int8_t* qs, const float* scales, const int32_t* bsums,
                             hipStream_t stream) {
    GemvSegs sg;
    int total;
    const hipError_t e = multi_segs(n_mats, w, n, bias, y, sg, total);
    if (e != hipSuccess) return e;
    if (total == 0) return hipSuccess;
    return gemv_dispatch(type, sg, k, total, m, qs, scales, bsums, nullptr, 0, stream);
}

hipError_t launch_rmsnorm_gemv_multi(uint32_t type, int k, int n_mats, const uint8_t* const* w,
                                     const int* n, const float* const* bias, float* const* y,
                                     const float* x, const float* norm_w, float eps,
                                     hipStream_t stream) {
    if (k <= 0 || k > 4096 || k % 32 != 0 || norm_w == nullptr) return hipErrorInvalidValue;
    GemvSegs sg;
    int total;
    const hipError_t e = multi_segs(n_mats, w, n, bias, y, sg, total);
    if (e != hipSuccess) return e;
    if (total == 0) return hipSuccess;
    sg.norm_w = norm_w;
    sg.eps = eps;
    return gemv_dispatch(type, sg, k, total, 1, nullptr, nullptr, nullptr, x, 0, stream);
}

static hipError_t swiglu_dispatch(uint32_t type, const GemvSegs& sg, int k, int n, int m,
                                  const int8_t* qs, const float* scales, const int32_t* bsums,
                                  const float* x_f32, hipStream_t stream) {
    switch (type) {
        case T_Q4_K: return gemv_all_rows<T_Q4_K, true>(sg, k, n, m, qs, scales, bsums, x_f32, 0, stream);
        case T_Q5_K: return gemv_all_rows<T_Q5_K, true>(sg, k, n, m, qs, scales, bsums, x_f32, 0, stream);
        case T_Q6_K: return gemv_all_rows<T_Q6_K, true>(sg, k, n, m, qs, scales, bsums, x_f32, 0, stream);
        case T_Q8_0: return gemv_all_rows<T_Q8_0, true>(sg, k, n, m, qs, scales, bsums, x_f32, 0, stream);
        case T_Q4_0: return gemv_all_rows<T_Q4_0, true>(sg, k, n, m, qs, scales, bsums, x_f32, 0, stream);
        case T_Q5_0: return gemv_all_rows<T_Q5_0, true>(sg, k, n, m, qs, scales, bsums, x_f32, 0, stream);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_swiglu(uint32_t type, int k, int n, const uint8_t* w_gate,
                              const uint8_t* w_up, const float* bias_gate, const float* bias_up,
                              float* h, int m, const int8_t* qs, const float* scales,
                              const int32_t* bsums, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    GemvSegs sg = one_segment(w_gate, n, bias_gate, h);
    sg.w[1] = w_up;
    sg.bias[1] = bias_up;
    return swiglu_dispatch(type, sg, k, n, m, qs, scales, bsums, nullptr, stream);
}

hipError_t launch_rmsnorm_gemv_swiglu(uint32_t type, int k, int n, const uint8_t* w_gate,
                                      const uint8_t* w_up, const float* bias_gate,
                                      const float* bias_up, const float* x, const float* norm_w,
                                      float eps, float* h, hipStream_t stream) {
    if (k <= 0 || k > 4096 || k % 32 != 0 || norm_w == nullptr) return hipErrorInvalidValue;
    if (n <= 0) return hipSuccess;
    GemvSegs sg = one_segment(w_gate, n, bias_gate, h);
    sg.w[1] = w_up;
    sg.bias[1] = bias_up;
    sg.norm_w = norm_w;
    sg.eps = eps;
    return swiglu_dispatch(type, sg, k, n, 1, nullptr, nullptr, nullptr, x, stream);
}

hipError_t launch_gemv_fused(uint32_t type, const uint8_t* w, int k, int n, int m,
                             const float* x, const float* bias, float* y, hipStream_t stream,
                             bool accumulate) {
    return gemv_dispatch(type, one_segment(w, n, bias, y), k, n, m, nullptr, nullptr, nullptr, x,
                         accumulate ? 1 : 0, stream);
}

}  // namespace cllm_hip
