// k_gemm.hip -- int8-MFMA GEMM for batched prefill (matmul_quant_batch with many rows).
//
// y[m, n] = sum_b dx[m,b] * (ws[n,b] * I[m,n,b] - wm[n,b] * bsum[m,b]) (+ bias[n]), the
// reference's per-block terms (src/core/quant.cpp:1453-1464 over the vec_dot kernels), with
// I[m,n,b] = sum over the 32 elements of block b of qx[m,k] * q[n,k], computed exactly by
// v_mfma_i32_32x32x32_i8 (one instruction = one 32x32 tile of one activation block). Q6_K
// scales every 16 elements, so it runs two v_mfma_i32_32x32x16_i8 per block and combines
// sc_a * I_a + sc_b * I_b exactly in int32, as the reference does (quant.cpp:677-678).
//
// Weights are read in place from the GGUF blocks and unpacked once per workgroup tile into
// signed int8 in LDS, with their offsets (-8 / -16 / -32) applied, so Q4_0 / Q5_0 / Q6_K need
// no activation-sum term; Q4_K / Q5_K keep the reference's separate minimum term.
//
// Tiling: a 256-thread workgroup owns a BM x BN = 64 x 128 output tile and walks K in steps of
// 256 elements (one super-block, or eight 32-element blocks). Each of the 4 waves computes a
// 32 x 64 sub-tile: two 32x32 MFMA tiles per activation block, followed by the fp32 epilogue.
#include "device_utils.h"
#include "ggml_blocks.h"
#include "launch.h"

namespace cllm_hip {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

constexpr int GBM = 64;    // activation rows per workgroup
constexpr int GBN = 128;   // weight rows per workgroup
constexpr int GKS = 256;   // elements per K step
constexpr int GROW = 272;  // LDS row stride in bytes (256 + 16 padding against bank conflicts)

// Signed int8 bytes v - off for unsigned bytes v <= 2 * off - 1, without carries between
// bytes: (v + (128 - off)) ^ 0x80 per byte.
__device__ __forceinline__ uint32_t sub_off(uint32_t v, uint32_t off) {
    return (v + (0x80808080u - off * 0x01010101u)) ^ 0x80808080u;
}

// 16 bytes of a 2-byte-aligned field (see ld_a2 in device_utils.h).
__device__ __forceinline__ u32x4 ld16_a2(const uint8_t* p) {
    uint32_t o[4];
    ld_a2<4>(p, o);
    return u32x4{o[0], o[1], o[2], o[3]};
}

// Chunk c (elements 16c .. 16c+15 of a 256-element K step) of weight row `row`, K step ks, as
// signed int8 with the type's offset applied.
template <uint32_t T>
__device__ __forceinline__ u32x4 unpack_chunk(const uint8_t* row, int ks, int c) {
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        const uint8_t* blk = row + (size_t)ks * (T == T_Q5_K ? Q5_K_BYTES : Q4_K_BYTES);
        const int b = c >> 1, h = c & 1;  // sub-block, element half
        const u32x4 q = ld_u32x4(blk + (T == T_Q5_K ? Q5_K_QS : Q4_K_QS) + 32 * (b >> 1) + 16 * h);
        const uint32_t sh = 4u * (uint32_t)(b & 1);
        u32x4 v;
        v.x = (q.x >> sh) & 0x0F0F0F0Fu;
        v.y = (q.y >> sh) & 0x0F0F0F0Fu;
        v.z = (q.z >> sh) & 0x0F0F0F0Fu;
        v.w = (q.w >> sh) & 0x0F0F0F0Fu;
        if constexpr (T == T_Q5_K) {
            const u32x4 qh = ld_u32x4(blk + Q5_K_QH + 16 * h);
            v.x |= ((qh.x >> b) & 0x01010101u) << 4;
            v.y |= ((qh.y >> b) & 0x01010101u) << 4;
            v.z |= ((qh.z >> b) & 0x01010101u) << 4;
            v.w |= ((qh.w >> b) & 0x01010101u) << 4;
        }
        return v;
    } else if constexpr (T == T_Q6_K) {
        const uint8_t* blk = row + (size_t)ks * Q6_K_BYTES;
        const int g = c >> 3, i = (c & 7) >> 1, h = c & 1;
        const u32x4 ql = ld16_a2(blk + 64 * g + 32 * (i & 1) + 16 * h);
        const u32x4 qh = ld16_a2(blk + Q6_K_QH + 32 * g + 16 * h);
        const uint32_t lsh = i < 2 ? 0u : 4u, hsh = 2u * (uint32_t)i;
        u32x4 v;
        v.x = sub_off(((ql.x >> lsh) & 0x0F0F0F0Fu) | (((qh.x >> hsh) & 0x03030303u) << 4), 32);
        v.y = sub_off(((ql.y >> lsh) & 0x0F0F0F0Fu) | (((qh.y >> hsh) & 0x03030303u) << 4), 32);
        v.z = sub_off(((ql.z >> lsh) & 0x0F0F0F0Fu) | (((qh.z >> hsh) & 0x03030303u) << 4), 32);
        v.w = sub_off(((ql.w >> lsh) & 0x0F0F0F0Fu) | (((qh.w >> hsh) & 0x03030303u) << 4), 32);
        return v;
    } else if constexpr (T == T_Q8_0) {
        const uint8_t* blk = row + (size_t)(ks * 8 + (c >> 1)) * Q8_0_BYTES;
        return ld16_a2(blk + 2 + 16 * (c & 1));
    } else {  // Q4_0 / Q5_0
        constexpr bool Q5 = T == T_Q5_0;
        const uint8_t* blk = row + (size_t)(ks * 8 + (c >> 1)) * (Q5 ? Q5_0_BYTES : Q4_0_BYTES);
        const int h = c & 1;  // element half: low nibbles (0-15) or high nibbles (16-31)
        const u32x4 q = ld16_a2(blk + (Q5 ? 6 : 2));
        const uint32_t sh = 4u * (uint32_t)h;
        uint32_t w[4] = {(q.x >> sh) & 0x0F0F0F0Fu, (q.y >> sh) & 0x0F0F0F0Fu,
                         (q.z >> sh) & 0x0F0F0F0Fu, (q.w >> sh) & 0x0F0F0F0Fu};
        if constexpr (Q5) {
            uint32_t t[1];
            ld_a2<1>(blk + 2, t);
            const uint32_t bits = t[0] >> (16 * h);
#pragma unroll
            for (int d = 0; d < 4; ++d)
                w[d] |= (((bits >> (4 * d)) & 0xFu) * 0x00204081u & 0x01010101u) << 4;
        }
        const uint32_t off = Q5 ? 16u : 8u;
        return u32x4{sub_off(w[0], off), sub_off(w[1], off), sub_off(w[2], off), sub_off(w[3], off)};
    }
}

// Per-block weight scales of row `row`, K step ks, block b (0..7): ws multiplies dx * I,
// wm multiplies dx * bsum (K-quant minimum). For Q6_K, sc16 returns the two int8 scales of the
// block's halves and ws = d.
template <uint32_t T>
__device__ __forceinline__ void block_scales(const uint8_t* row, int ks, int b, float& ws,
                                             float& wm, int& sca, int& scb) {
    wm = 0.0f;
    sca = scb = 0;
    if constexpr (T == T_Q4_K || T == T_Q5_K) {
        const uint8_t* blk = row + (size_t)ks * (T == T_Q5_K ? Q5_K_BYTES : Q4_K_BYTES);
        const u32x4 h = ld_u32x4(blk);
        int sc, m;
        k4_scale_min(h.y, h.z, h.w, b, sc, m);
        ws = f16_to_f32(h.x & 0xFFFFu) * (float)sc;
        wm = f16_to_f32(h.x >> 16) * (float)m;
    } else if constexpr (T == T_Q6_K) {
        const uint8_t* blk = row + (size_t)ks * Q6_K_BYTES;
        ws = f16_to_f32(ld_u16(blk + Q6_K_D));
        const uint32_t pair = ld_u16(blk + Q6_K_SC + 2 * b);  // sc[2b], sc[2b+1]
        sca = (int)(int8_t)(pair & 0xFFu);
        scb = (int)(int8_t)(pair >> 8);
    } else {
        constexpr int bytes = T == T_Q8_0 ? Q8_0_BYTES : T == T_Q4_0 ? Q4_0_BYTES : Q5_0_BYTES;
        ws = f16_to_f32(ld_u16(row + (size_t)(ks * 8 + b) * bytes));
    }
}

template <uint32_t T>
__global__ __launch_bounds__(256) void k_gemm_i8(const uint8_t* __restrict__ w, int64_t row_bytes,
                                                 int k, int n, int m,
                                                 const int8_t* __restrict__ qs,
                                                 const float* __restrict__ xs,
                                                 const int32_t* __restrict__ xb,
                                                 const float* __restrict__ bias,
                                                 float* __restrict__ y) {
    constexpr bool KMIN = T == T_Q4_K || T == T_Q5_K;
    constexpr bool Q6 = T == T_Q6_K;
    __shared__ __align__(16) int8_t sA[GBM * GROW];
    __shared__ __align__(16) int8_t sB[GBN * GROW];
    __shared__ __align__(16) float sDx[8][GBM];   // dx
    __shared__ __align__(16) float sPx[8][GBM];   // dx * bsum (K-quants)
    __shared__ __align__(16) float sWs[8][GBN];   // ws (Q6_K: d)
    __shared__ __align__(16) float sWm[8][GBN];   // wm (K-quants)
    __shared__ __align__(16) int sSc[16][GBN];    // Q6_K 16-element scales

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int n0 = blockIdx.x * GBN;
    const int m0 = blockIdx.y * GBM;
    const int nb = k / 32;
    const int wm_ = wave >> 1;  // 32-row half of the activation tile
    const int wn_ = wave & 1;   // 64-row half of the weight tile

    float acc[2][16];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;

    const int steps = k / GKS;
    for (int ks = 0; ks < steps; ++ks) {
        // ---- stage the activation tile: GBM rows x 256 int8, scales and sums
        for (int i = tid; i < GBM * 16; i += 256) {
            const int r = i >> 4, c = i & 15;
            const int mm = min(m0 + r, m - 1);  // rows past m repeat row m-1; never stored
            *(u32x4*)(sA + r * GROW + 16 * c) =
                ld_u32x4(qs + (size_t)mm * k + (size_t)ks * GKS + 16 * c);
        }
        for (int i = tid; i < GBM * 8; i += 256) {
            const int r = i >> 3, b = i & 7;
            const int mm = min(m0 + r, m - 1);
            const size_t ix = (size_t)mm * nb + (size_t)ks * 8 + b;
            const float dx = xs[ix];
            sDx[b][r] = dx;
            if constexpr (KMIN) sPx[b][r] = dx * (float)xb[ix];
        }
        // ---- unpack the weight tile: GBN rows x 16 chunks of 16 elements, and block scales
        for (int i = tid; i < GBN * 16; i += 256) {
            const int r = i >> 4, c = i & 15;
            const int nn = min(n0 + r, n - 1);
            *(u32x4*)(sB + r * GROW + 16 * c) = unpack_chunk<T>(w + (int64_t)nn * row_bytes, ks, c);
        }
        for (int i = tid; i < GBN * 8; i += 256) {
            const int r = i >> 3, b = i & 7;
            const int nn = min(n0 + r, n - 1);
            float ws, wmv;
            int sca, scb;
            block_scales<T>(w + (int64_t)nn * row_bytes, ks, b, ws, wmv, sca, scb);
            sWs[b][r] = ws;
            if constexpr (KMIN) sWm[b][r] = wmv;
            if constexpr (Q6) {
                sSc[2 * b][r] = sca;
                sSc[2 * b + 1][r] = scb;
            }
        }
        __syncthreads();

        // ---- MFMA + epilogue, one 32-element activation block at a time
        const int am = 32 * wm_ + (lane & 31);   // A fragment row
        const int kh = lane >> 5;                // k half held by this lane
        const int mrow0 = 32 * wm_ + 4 * kh;     // first output row of this lane (+ 8a + c)
#pragma unroll 1
        for (int b = 0; b < 8; ++b) {
            // dx (and dx * bsum) of the 16 output rows of this lane: rows mrow0 + 8a + c
            float dxr[16], pxr[16];
#pragma unroll
            for (int a4 = 0; a4 < 4; ++a4) {
                const float4 d4 = *(const float4*)&sDx[b][mrow0 + 8 * a4];
                dxr[4 * a4] = d4.x; dxr[4 * a4 + 1] = d4.y; dxr[4 * a4 + 2] = d4.z; dxr[4 * a4 + 3] = d4.w;
                if constexpr (KMIN) {
                    const float4 p4 = *(const float4*)&sPx[b][mrow0 + 8 * a4];
                    pxr[4 * a4] = p4.x; pxr[4 * a4 + 1] = p4.y; pxr[4 * a4 + 2] = p4.z; pxr[4 * a4 + 3] = p4.w;
                }
            }
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int bn = 64 * wn_ + 32 * t + (lane & 31);  // B fragment row = output col
                i32x16 I;
                if constexpr (Q6) {
                    // two K=16 MFMAs: halves of the block, 8 bytes per lane
                    i32x16 zero = {};
                    const long a0 = *(const long*)(sA + am * GROW + 32 * b + 8 * kh);
                    const long b0 = *(const long*)(sB + bn * GROW + 32 * b + 8 * kh);
                    const long a1 = *(const long*)(sA + am * GROW + 32 * b + 16 + 8 * kh);
                    const long b1 = *(const long*)(sB + bn * GROW + 32 * b + 16 + 8 * kh);
                    const i32x16 Ia = __builtin_amdgcn_mfma_i32_32x32x16_i8(a0, b0, zero, 0, 0, 0);
                    const i32x16 Ib = __builtin_amdgcn_mfma_i32_32x32x16_i8(a1, b1, zero, 0, 0, 0);
                    const int sca = sSc[2 * b][bn], scb = sSc[2 * b + 1][bn];
#pragma unroll
                    for (int r = 0; r < 16; ++r) I[r] = sca * Ia[r] + scb * Ib[r];
                } else {
                    i32x16 zero = {};
                    const i32x4 av = *(const i32x4*)(sA + am * GROW + 32 * b + 16 * kh);
                    const i32x4 bv = *(const i32x4*)(sB + bn * GROW + 32 * b + 16 * kh);
                    I = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bv, zero, 0, 0, 0);
                }
                const float ws = sWs[b][bn];
                const float wmv = KMIN ? sWm[b][bn] : 0.0f;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float v = fmaf(ws * dxr[r], (float)I[r], acc[t][r]);
                    if constexpr (KMIN) v = fmaf(-wmv, pxr[r], v);
                    acc[t][r] = v;
                }
            }
        }
        __syncthreads();
    }

    // ---- store: lane holds rows mrow0 + 8a + c (a, c < 4), column 32t + lane % 32
    const int kh = lane >> 5;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int col = n0 + 64 * wn_ + 32 * t + (lane & 31);
        if (col >= n) continue;
        const float bj = bias ? bias[col] : 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int row = m0 + 32 * wm_ + 8 * (r >> 2) + 4 * kh + (r & 3);
            if (row < m) {
                float v = acc[t][r];
                if (bias) v += bj;
                y[(size_t)row * n + col] = v;
            }
        }
    }
}

bool gemm_supported(uint32_t type) { return has_kernel(type); }

template <uint32_t T>
static hipError_t launch_gemm_t(const uint8_t* w, int k, int n, int m, const int8_t* qs,
                                const float* xs, const int32_t* xb, const float* bias, float* y,
                                hipStream_t stream) {
    const int64_t row_bytes = (int64_t)(k / block_elems(T)) * (int64_t)block_bytes(T);
    const dim3 grid((unsigned)((n + GBN - 1) / GBN), (unsigned)((m + GBM - 1) / GBM));
    hipLaunchKernelGGL(k_gemm_i8<T>, grid, dim3(256), 0, stream, w, row_bytes, k, n, m, qs, xs,
                       xb, bias, y);
    return hipGetLastError();
}

hipError_t launch_gemm(uint32_t type, const uint8_t* w, int k, int n, int m, const int8_t* qs,
                       const float* scales, const int32_t* bsums, const float* bias, float* y,
                       hipStream_t stream) {
    if (k % GKS != 0) return hipErrorNotSupported;
    switch (type) {
        case T_Q4_K: return launch_gemm_t<T_Q4_K>(w, k, n, m, qs, scales, bsums, bias, y, stream);
        case T_Q5_K: return launch_gemm_t<T_Q5_K>(w, k, n, m, qs, scales, bsums, bias, y, stream);
        case T_Q6_K: return launch_gemm_t<T_Q6_K>(w, k, n, m, qs, scales, bsums, bias, y, stream);
        case T_Q8_0: return launch_gemm_t<T_Q8_0>(w, k, n, m, qs, scales, bsums, bias, y, stream);
        case T_Q4_0: return launch_gemm_t<T_Q4_0>(w, k, n, m, qs, scales, bsums, bias, y, stream);
        case T_Q5_0: return launch_gemm_t<T_Q5_0>(w, k, n, m, qs, scales, bsums, bias, y, stream);
        default: return hipErrorNotSupported;
    }
}

}  // namespace cllm_hip
