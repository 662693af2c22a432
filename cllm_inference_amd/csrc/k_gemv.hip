// k_gemv.hip -- weight-streaming GEMV kernels (decode, small n_rows) on gfx950.
//
// y[t, j] = vec_dot(W row j, Q8_0 activation row t) (+ bias[j]): the inner loops of
// matmul_quant / matmul_quant_batch (src/core/quant.cpp:1388-1397, 1453-1464) for the six
// weight types with a vec_dot kernel.
//
// Work split. One wave64 owns R consecutive weight rows. A row is cut into "units" that one
// lane handles at a time:
//   Q4_K, Q5_K : a quarter super-block = one 32-byte qs chunk = sub-blocks 2c and 2c+1
//   Q6_K       : a quarter super-block = half g, element half h of four sub-blocks
//   Q8_0, Q4_0, Q5_0 : one 32-element block
// Lanes stride over the units of the row, so consecutive lanes read consecutive bytes and
// every weight byte is loaded exactly once, in place, straight from the GGUF blocks. Integer
// dots use v_dot4_i32_i8; the fp32 per-block terms are the reference's:
//   acc += (ws * dx) * dot      and, for Q4_K / Q5_K, acc -= (wm * dx) * bsum
// (quant.cpp:545, 582-583, 621-622, 677-678, 775, 891). Lane partial sums are reduced across
// the wave, so only the fp32 summation order differs from the reference.
//
// Activations (Q8_0 rows: int8 qs, fp32 scales, int32 block sums) are small and re-read from
// L1/L2 by every wave; for m > 1 each weight unit is dotted with up to MR activation rows
// while it sits in registers.
#include "device_utils.h"
#include "ggml_blocks.h"
#include "launch.h"

namespace cllm_hip {

struct ActRows {
    const int8_t* qs;
    const float* sc;
    const int32_t* bs;
    int k;   // elements per activation row
    int nb;  // 32-element blocks per activation row
};

__device__ __forceinline__ void ld_act32(const ActRows& a, int r, int b, uint32_t (&x)[8]) {
    const int8_t* p = a.qs + (size_t)r * a.k + (size_t)b * 32;
    const u32x4 x0 = ld_u32x4(p), x1 = ld_u32x4(p + 16);
    x[0] = x0.x; x[1] = x0.y; x[2] = x0.z; x[3] = x0.w;
    x[4] = x1.x; x[5] = x1.y; x[6] = x1.z; x[7] = x1.w;
}

// ------------------------------------------------------------------------------ Q4_K / Q5_K
// Unit u = 4 s + c of super-block s: the low nibbles of qs[32c .. 32c+31] are sub-block 2c,
// the high nibbles sub-block 2c+1 (quant.cpp:549-590; Q5_K adds bit k of qh[l], 592-628).
template <bool Q5>
struct TraitsK45 {
    static constexpr int UNIT = 64;
    struct Prep {
        uint32_t lo[8], hi[8];
        float ws0, wm0, ws1, wm1;
    };
    static __device__ __forceinline__ Prep load(const uint8_t* row, int u) {
        const int s = u >> 2, c = u & 3;
        const uint8_t* blk = row + (size_t)s * (Q5 ? Q5_K_BYTES : Q4_K_BYTES);
        const u32x4 h = ld_u32x4(blk);
        const uint8_t* qp = blk + (Q5 ? Q5_K_QS : Q4_K_QS) + 32 * c;
        const u32x4 qa = ld_u32x4(qp), qb = ld_u32x4(qp + 16);
        const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        Prep p;
        if constexpr (Q5) {
            const u32x4 ha = ld_u32x4(blk + Q5_K_QH), hb = ld_u32x4(blk + Q5_K_QH + 16);
            const uint32_t qh[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                p.lo[i] = (q[i] & 0x0F0F0F0Fu) | (((qh[i] >> (2 * c)) & 0x01010101u) << 4);
                p.hi[i] = ((q[i] >> 4) & 0x0F0F0F0Fu) | (((qh[i] >> (2 * c + 1)) & 0x01010101u) << 4);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                p.lo[i] = q[i] & 0x0F0F0F0Fu;
                p.hi[i] = (q[i] >> 4) & 0x0F0F0F0Fu;
            }
        }
        const float d = f16_to_f32(h.x & 0xFFFFu), dmin = f16_to_f32(h.x >> 16);
        int sc0, m0, sc1, m1;
        k4_scale_min(h.y, h.z, h.w, 2 * c, sc0, m0);
        k4_scale_min(h.y, h.z, h.w, 2 * c + 1, sc1, m1);
        p.ws0 = d * (float)sc0;
        p.wm0 = dmin * (float)m0;
        p.ws1 = d * (float)sc1;
        p.wm1 = dmin * (float)m1;
        return p;
    }
    template <int R, int MR>
    static __device__ __forceinline__ void accum(const Prep (&p)[R], int u, const ActRows& a,
                                                 float (&acc)[R][MR]) {
        const int b0 = 8 * (u >> 2) + 2 * (u & 3);
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            uint32_t x0[8], x1[8];
            ld_act32(a, r, b0, x0);
            ld_act32(a, r, b0 + 1, x1);
            const float* xs = a.sc + (size_t)r * a.nb + b0;
            const int32_t* xb = a.bs + (size_t)r * a.nb + b0;
            const float dx0 = xs[0], dx1 = xs[1];
            const float bs0 = (float)xb[0], bs1 = (float)xb[1];
#pragma unroll
            for (int rr = 0; rr < R; ++rr) {
                int d0 = 0, d1 = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    d0 = sdot4(p[rr].lo[i], x0[i], d0);
                    d1 = sdot4(p[rr].hi[i], x1[i], d1);
                }
                float v = acc[rr][r];
                v = fmaf(p[rr].ws0 * dx0, (float)d0, v);
                v = fmaf(-(p[rr].wm0 * dx0), bs0, v);
                v = fmaf(p[rr].ws1 * dx1, (float)d1, v);
                v = fmaf(-(p[rr].wm1 * dx1), bs1, v);
                acc[rr][r] = v;
            }
        }
    }
};

// ------------------------------------------------------------------------------------ Q6_K
// Unit u = 4 s + 2 g + h: half g (elements 128g .. 128g+127) of super-block s, element half h
// (l in [16h, 16h+16)) of its four sub-blocks i. Element l of sub-block i:
//   low4 = ql[64g + 32(i&1) + l], low nibble for i < 2, high nibble for i >= 2
//   hi2  = (qh[32g + l] >> 2i) & 3;   q6 = (low4 | hi2 << 4) - 32
// and it is scaled by sc[8g + 2i + h] (quant.cpp:630-687). The two lanes h = 0, 1 of a
// sub-block form the reference's exact integer sc_a*dot_a + sc_b*dot_b with one DPP move.
struct TraitsQ6K {
    static constexpr int UNIT = 64;
    struct Prep {
        uint32_t q[4][4];  // [sub-block i][dword]: signed bytes q6 - 32
        int sc[4];
        float d;
    };
    static __device__ __forceinline__ Prep load(const uint8_t* row, int u) {
        const int s = u >> 2, g = (u >> 1) & 1, h = u & 1;
        const uint8_t* blk = row + (size_t)s * Q6_K_BYTES;
        uint32_t qa[4], qb[4], qh[4], sc[2];
        ld_a2<4>(blk + 64 * g + 16 * h, qa);
        ld_a2<4>(blk + 64 * g + 32 + 16 * h, qb);
        ld_a2<4>(blk + Q6_K_QH + 32 * g + 16 * h, qh);
        ld_a2<2>(blk + Q6_K_SC + 8 * g, sc);
        const uint32_t dbits = ld_u16(blk + Q6_K_D);
        Prep p;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t l0 = qa[t] & 0x0F0F0F0Fu, l2 = (qa[t] >> 4) & 0x0F0F0F0Fu;
            const uint32_t l1 = qb[t] & 0x0F0F0F0Fu, l3 = (qb[t] >> 4) & 0x0F0F0F0Fu;
            const uint32_t h0 = (qh[t] & 0x03030303u) << 4;
            const uint32_t h1 = (qh[t] & 0x0C0C0C0Cu) << 2;
            const uint32_t h2 = qh[t] & 0x30303030u;
            const uint32_t h3 = (qh[t] & 0xC0C0C0C0u) >> 2;
            // bytes v in [0, 63]: (v + 0x60) ^ 0x80 is the int8 byte of v - 32, no carries.
            p.q[0][t] = (l0 + h0 + 0x60606060u) ^ 0x80808080u;
            p.q[1][t] = (l1 + h1 + 0x60606060u) ^ 0x80808080u;
            p.q[2][t] = (l2 + h2 + 0x60606060u) ^ 0x80808080u;
            p.q[3][t] = (l3 + h3 + 0x60606060u) ^ 0x80808080u;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
            p.sc[i] = (int)(int8_t)((sc[i >> 1] >> (8 * (2 * (i & 1) + h))) & 0xFFu);
        p.d = f16_to_f32(dbits);
        return p;
    }
    template <int R, int MR>
    static __device__ __forceinline__ void accum(const Prep (&p)[R], int u, const ActRows& a,
                                                 float (&acc)[R][MR]) {
        const int s = u >> 2, g = (u >> 1) & 1, h = u & 1;
        const int bb = 8 * s + 4 * g;
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            uint32_t x[4][4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const u32x4 v = ld_u32x4(a.qs + (size_t)r * a.k + (size_t)(bb + i) * 32 + 16 * h);
                x[i][0] = v.x; x[i][1] = v.y; x[i][2] = v.z; x[i][3] = v.w;
            }
            const float* xs = a.sc + (size_t)r * a.nb + bb;
            const float dxa = xs[2 * h], dxb = xs[2 * h + 1];
#pragma unroll
            for (int rr = 0; rr < R; ++rr) {
                int tot[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    int dot = 0;
#pragma unroll
                    for (int t = 0; t < 4; ++t) dot = sdot4(p[rr].q[i][t], x[i][t], dot);
                    const int part = p[rr].sc[i] * dot;
                    tot[i] = part + dpp_i32<DPP_QUAD_SWAP1>(part);  // + partner lane h ^ 1
                }
                // lane h finishes sub-blocks 2h and 2h + 1
                const int ia = h ? tot[2] : tot[0];
                const int ib = h ? tot[3] : tot[1];
                float v = acc[rr][r];
                v = fmaf(p[rr].d * dxa, (float)ia, v);
                v = fmaf(p[rr].d * dxb, (float)ib, v);
                acc[rr][r] = v;
            }
        }
    }
};

// ------------------------------------------------------------------------------------ Q8_0
struct TraitsQ80 {
    static constexpr int UNIT = 32;
    struct Prep {
        uint32_t q[8];
        float d;
    };
    static __device__ __forceinline__ Prep load(const uint8_t* row, int b) {
        const uint8_t* blk = row + (size_t)b * Q8_0_BYTES;
        Prep p;
        ld_a2<8>(blk + 2, p.q);
        p.d = f16_to_f32(ld_u16(blk));
        return p;
    }
    template <int R, int MR>
    static __device__ __forceinline__ void accum(const Prep (&p)[R], int b, const ActRows& a,
                                                 float (&acc)[R][MR]) {
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            uint32_t x[8];
            ld_act32(a, r, b, x);
            const float dx = a.sc[(size_t)r * a.nb + b];
#pragma unroll
            for (int rr = 0; rr < R; ++rr) {
                int dot = 0;
#pragma unroll
                for (int i = 0; i < 8; ++i) dot = sdot4(p[rr].q[i], x[i], dot);
                acc[rr][r] = fmaf(p[rr].d * dx, (float)dot, acc[rr][r]);
            }
        }
    }
};

// ----------------------------------------------------------------------------- Q4_0 / Q5_0
// Byte j of qs: low nibble = element j, high nibble = element j + 16. Q5_0 adds bit j of
// the little-endian u32 qh as bit 4 of element j. The bracket dot - off * bsum is an exact
// integer (quant.cpp:757-777, 863-893).
template <bool Q5>
struct TraitsQ450 {
    static constexpr int UNIT = 32;
    struct Prep {
        uint32_t lo[4], hi[4];
        float d;
    };
    // bits 0..3 of x4 -> bit 4 of bytes 0..3
    static __device__ __forceinline__ uint32_t spread4(uint32_t x4) {
        return ((x4 * 0x00204081u) & 0x01010101u) << 4;
    }
    static __device__ __forceinline__ Prep load(const uint8_t* row, int b) {
        const uint8_t* blk = row + (size_t)b * (Q5 ? Q5_0_BYTES : Q4_0_BYTES);
        uint32_t q[4];
        ld_a2<4>(blk + (Q5 ? 6 : 2), q);
        Prep p;
        uint32_t qh = 0;
        if constexpr (Q5) {
            uint32_t t[1];
            ld_a2<1>(blk + 2, t);
            qh = t[0];
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            p.lo[t] = q[t] & 0x0F0F0F0Fu;
            p.hi[t] = (q[t] >> 4) & 0x0F0F0F0Fu;
            if constexpr (Q5) {
                p.lo[t] |= spread4((qh >> (4 * t)) & 0xFu);
                p.hi[t] |= spread4((qh >> (16 + 4 * t)) & 0xFu);
            }
        }
        p.d = f16_to_f32(ld_u16(blk));
        return p;
    }
    template <int R, int MR>
    static __device__ __forceinline__ void accum(const Prep (&p)[R], int b, const ActRows& a,
                                                 float (&acc)[R][MR]) {
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            uint32_t x[8];
            ld_act32(a, r, b, x);
            const float dx = a.sc[(size_t)r * a.nb + b];
            const int off = (Q5 ? 16 : 8) * a.bs[(size_t)r * a.nb + b];
#pragma unroll
            for (int rr = 0; rr < R; ++rr) {
                int dot = 0;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    dot = sdot4(p[rr].lo[t], x[t], dot);
                    dot = sdot4(p[rr].hi[t], x[4 + t], dot);
                }
                acc[rr][r] = fmaf(p[rr].d * dx, (float)(dot - off), acc[rr][r]);
            }
        }
    }
};

template <uint32_t T> struct TraitsOf;
template <> struct TraitsOf<T_Q4_K> { using type = TraitsK45<false>; };
template <> struct TraitsOf<T_Q5_K> { using type = TraitsK45<true>; };
template <> struct TraitsOf<T_Q6_K> { using type = TraitsQ6K; };
template <> struct TraitsOf<T_Q8_0> { using type = TraitsQ80; };
template <> struct TraitsOf<T_Q4_0> { using type = TraitsQ450<false>; };
template <> struct TraitsOf<T_Q5_0> { using type = TraitsQ450<true>; };

// One wave per R consecutive weight rows; 4 waves per workgroup.
template <uint32_t T, int R, int MR>
__global__ __launch_bounds__(256) void k_gemv(const uint8_t* __restrict__ w, int64_t row_bytes,
                                              int k, int n, const int8_t* __restrict__ qs,
                                              const float* __restrict__ xs,
                                              const int32_t* __restrict__ xb,
                                              const float* __restrict__ bias,
                                              float* __restrict__ y) {
    using Tr = typename TraitsOf<T>::type;
    const int lane = threadIdx.x & 63;
    const int j0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
    if (j0 >= n) return;  // wave-uniform
    const ActRows a{qs, xs, xb, k, k / 32};
    const int units = k / Tr::UNIT;

    float acc[R][MR];
#pragma unroll
    for (int rr = 0; rr < R; ++rr)
#pragma unroll
        for (int r = 0; r < MR; ++r) acc[rr][r] = 0.0f;

    for (int u = lane; u < units; u += 64) {
        typename Tr::Prep p[R];
#pragma unroll
        for (int rr = 0; rr < R; ++rr) {
            const int j = min(j0 + rr, n - 1);  // rows past n repeat row n-1 and are not stored
            p[rr] = Tr::load(w + (int64_t)j * row_bytes, u);
        }
        Tr::template accum<R, MR>(p, u, a, acc);
    }

#pragma unroll
    for (int rr = 0; rr < R; ++rr) {
#pragma unroll
        for (int r = 0; r < MR; ++r) {
            float v = wave_sum(acc[rr][r]);
            const int j = j0 + rr;
            if (lane == r && j < n) {
                if (bias) v += bias[j];
                y[(size_t)r * n + j] = v;
            }
        }
    }
}

template <uint32_t T, int R, int MR>
static hipError_t launch_t(const uint8_t* w, int k, int n, const int8_t* qs, const float* xs,
                           const int32_t* xb, const float* bias, float* y, hipStream_t stream) {
    const int64_t row_bytes = (int64_t)(k / block_elems(T)) * (int64_t)block_bytes(T);
    const int waves = (n + R - 1) / R;
    const int grid = (waves + 3) / 4;
    hipLaunchKernelGGL((k_gemv<T, R, MR>), dim3(grid), dim3(256), 0, stream, w, row_bytes, k, n,
                       qs, xs, xb, bias, y);
    return hipGetLastError();
}

template <uint32_t T>
static hipError_t launch_rows(const uint8_t* w, int k, int n, int mr, const int8_t* qs,
                              const float* xs, const int32_t* xb, const float* bias, float* y,
                              hipStream_t stream) {
    switch (mr) {
        case 1: return launch_t<T, 2, 1>(w, k, n, qs, xs, xb, bias, y, stream);
        case 2: return launch_t<T, 2, 2>(w, k, n, qs, xs, xb, bias, y, stream);
        case 4: return launch_t<T, 1, 4>(w, k, n, qs, xs, xb, bias, y, stream);
        default: return launch_t<T, 1, 8>(w, k, n, qs, xs, xb, bias, y, stream);
    }
}

hipError_t launch_gemv(uint32_t type, const uint8_t* w, int k, int n, int m, const int8_t* qs,
                       const float* scales, const int32_t* bsums, const float* bias, float* y,
                       hipStream_t stream) {
    const int nb = k / 32;
    int t = 0;
    while (t < m) {
        const int left = m - t;
        const int mr = left >= 8 ? 8 : left >= 4 ? 4 : left >= 2 ? 2 : 1;
        const int8_t* q = qs + (size_t)t * k;
        const float* s = scales + (size_t)t * nb;
        const int32_t* b = bsums + (size_t)t * nb;
        float* yy = y + (size_t)t * n;
        hipError_t e;
        switch (type) {
            case T_Q4_K: e = launch_rows<T_Q4_K>(w, k, n, mr, q, s, b, bias, yy, stream); break;
            case T_Q5_K: e = launch_rows<T_Q5_K>(w, k, n, mr, q, s, b, bias, yy, stream); break;
            case T_Q6_K: e = launch_rows<T_Q6_K>(w, k, n, mr, q, s, b, bias, yy, stream); break;
            case T_Q8_0: e = launch_rows<T_Q8_0>(w, k, n, mr, q, s, b, bias, yy, stream); break;
            case T_Q4_0: e = launch_rows<T_Q4_0>(w, k, n, mr, q, s, b, bias, yy, stream); break;
            case T_Q5_0: e = launch_rows<T_Q5_0>(w, k, n, mr, q, s, b, bias, yy, stream); break;
            default: return hipErrorInvalidValue;
        }
        if (e != hipSuccess) return e;
        t += mr;
    }
    return hipSuccess;
}

}  // namespace cllm_hip
