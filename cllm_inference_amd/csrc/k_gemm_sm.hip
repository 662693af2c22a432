// Small batches (a few to 64 activation rows): the weight stream read once for the whole
// batch, dot products on int8 MFMA.
//
// matmul_quant_batch (src/core/quant.cpp:1433-1475) with M rows is M vec_dots per weight row.
// At M <= 64 the weights (tens of MB) still dominate the bytes, so the kernel is shaped like
// the decode GEMV's streaming kernel: one 16-wave workgroup per CU, each wave keeping one item
// of weights in flight while it computes the previous one. An item is 16 weight rows x 256
// elements (one super-block of a row, or eight 32-element blocks), read as contiguous
// nontemporal 16-byte pieces into the wave's LDS slot.
//
// Arithmetic, per 32-element block b of weight row r and activation row t:
//   - v_mfma_i32_16x16x32_i8 gives the exact integer dot of the 16 rows' weight quants with
//     the 16 activation rows' Q8_0 quants (tiles of 16 activation rows);
//   - Q4_K / Q5_K: y += d_r * sum_b (float)(sc_rb * dot) * dx_tb, then the minimum term
//     dmin_r * sum_b m_rb * (dx_tb * bsum_tb), which is a 16 x 8 x 16 product done by two
//     v_mfma_f32_16x16x4_f32 (fp32 operands, so each term is the fp32 product);
//   - Q8_0: y += (float)dot * (d_rb * dx_tb).
// The same terms as the reference's vec_dot_q4_K_q8_0 / vec_dot_q5_K_q8_0 / vec_dot_q8_0_q8_0
// (quant.cpp:549-590, 591-629, 507-548), summed in another order.
//
// Work split: a workgroup owns 16 / kp row groups (16 rows each) and one range of K (the
// split, blockIdx.y); within it wave w takes row group w / kp and the w % kp-th part of the
// split's super-blocks. The int8 activations of the split's K range sit in LDS for all waves
// (at most 64 KB, so 16 rows can span K = 4096 and 64 rows K = 1024); longer K is split over
// workgroups, whose partial tiles the last one to finish adds in split order (the cross-XCD
// protocol of the weight-row GEMM). The kp parts of a row group are added in LDS, in order.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "device_utils.h"
#include "ggml_blocks.h"
#include "launch.h"

namespace cllm_hip {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kSmWaves = 16;
constexpr int kSmActBytes = 64 * 1024;  // int8 activations of a split: 16 MT rows x kc

__host__ __device__ constexpr size_t sm_align16(size_t v) { return (v + 15) & ~(size_t)15; }

// Bytes of an item's row in its LDS slot: 256 elements of one weight row. A Q6_K super-block
// (210 bytes, 2-byte aligned) comes as the 224-byte window from the 16-byte boundary at or
// below it; with rows of a multiple of 16 bytes (k a multiple of 2048) the window of the
// row's last super-block ends exactly at the row's end, and no window leaves its row.
template <uint32_t T>
__host__ __device__ constexpr int sm_sb_bytes() {
    return T == T_Q8_0 ? 8 * Q8_0_BYTES : T == T_Q4_0 ? 8 * Q4_0_BYTES : T == T_Q5_0 ? 8 * Q5_0_BYTES
         : T == T_Q5_K ? 176 : T == T_Q6_K ? 224 : 144;
}
template <uint32_t T>
__host__ __device__ constexpr bool sm_kq() { return T == T_Q4_K || T == T_Q5_K; }
// Per-wave exchange table: Q4_K / Q5_K, the 6-bit scales [16 rows][8 blocks] as bytes; Q6_K,
// the 16 int8 scales of each row [16 rows][16]; the 32-element block types, the blocks' d as
// floats [8 blocks][16 rows].
template <uint32_t T>
__host__ __device__ constexpr int sm_tab_bytes() { return sm_kq<T>() ? 128 : T == T_Q6_K ? 256 : 512; }

// LDS layout of a workgroup: activations qs [16 MT][kc + 8] (the reduction area after the main
// loop), dx [16 MT][kc / 32], for the K-quants dx * bsum [16 MT][kc / 32], the waves' weight
// slots (16 rows x sb bytes each), the waves' exchange tables.
struct SmLayout {
    size_t xd, xm, slots, tab, total;
};
template <uint32_t T, int MT>
__host__ __device__ constexpr SmLayout sm_layout(int kc) {
    constexpr int MP = 16 * MT;
    SmLayout l{};
    const size_t q = (size_t)MP * (kc + 8), red = (size_t)kSmWaves * MT * 1024;
    l.xd = sm_align16(q > red ? q : red);
    l.xm = l.xd + (size_t)MP * (kc / 32) * 4;
    l.slots = sm_align16(l.xm + (sm_kq<T>() ? (size_t)MP * (kc / 32) * 4 : 0));
    l.tab = l.slots + (size_t)kSmWaves * 16 * sm_sb_bytes<T>();
    l.total = l.tab + (size_t)kSmWaves * sm_tab_bytes<T>();
    return l;
}

// Workgroup barrier that orders LDS only (weight loads in flight are not waited for).
__device__ __forceinline__ void sm_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ long as_long(u32x2 v) { return __builtin_bit_cast(long, v); }

// FUSED: x holds fp32 activation rows [m][k], quantized here (q8_quant_quad, bit for bit as
// quantize_row_q8_0); else qs / xs / xb hold the Q8_0 batch. Activation rows past m are zeros.
// LATE (from a quantized batch, one item per wave): item 0 is issued after the staging.
template <uint32_t T, int MT, bool FUSED, bool LATE>
__global__ __launch_bounds__(64 * kSmWaves) void k_gemm_sm(
    const uint8_t* __restrict__ w, int64_t row_bytes, int k, int n, int m, int kc, int kp,
    const float* __restrict__ x, const int8_t* __restrict__ qs, const float* __restrict__ xs,
    const int32_t* __restrict__ xb, const float* __restrict__ bias, float* __restrict__ y,
    float* __restrict__ part, int* __restrict__ counters) {
    constexpr int SB = sm_sb_bytes<T>();
    constexpr int PPR = SB / 16;         // 16-byte pieces per row of an item
    constexpr int NP = 16 * PPR;         // pieces per item
    constexpr int NL = (NP + 63) / 64;   // loads per lane per item
    constexpr int MP = 16 * MT;
    constexpr bool KQ = sm_kq<T>();
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int last_split;

    const SmLayout L = sm_layout<T, MT>(kc);
    const int QSR = kc + 8;  // activation row stride: 16 rows' 8-byte fragments hit distinct banks
    const int nb = kc / 32;
    int8_t* aq = (int8_t*)lds;
    float* axd = (float*)(lds + L.xd);
    float* axm = (float*)(lds + L.xm);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15, g = lane >> 4;
    const int rgw = kSmWaves / kp;
    const int n_rg = (n + 15) / 16;
    const int rg = blockIdx.x * rgw + wave / kp;
    const int kpart = wave % kp;
    const int k0 = blockIdx.y * kc;
    const int kce = min(kc, k - k0);    // this split's elements (a multiple of 256)
    const int nsb = kce / 256;
    // K part kpart takes super-blocks kpart, kpart + kp, ..: at each step the kp waves of a row
    // group read neighbouring super-blocks of the same rows
    const int items = rg < n_rg && kpart < nsb ? (nsb - kpart + kp - 1) / kp : 0;
    uint8_t* slot = lds + L.slots + (size_t)wave * 16 * SB;
    uint8_t* tab = lds + L.tab + (size_t)wave * sm_tab_bytes<T>();

    // ---- item loads: piece p = 64 L + lane is piece p % PPR of item row p / PPR ----
    u32x4 pc[NL];
    auto load_item = [&](int it, uint32_t dep) {
        const int sbg = min(k0 / 256 + kpart + kp * it, k / 256 - 1);
        // the item's bytes within each row (Q6_K: the 16-byte boundary at or below the block)
        const int64_t at = T == T_Q6_K ? ((int64_t)sbg * Q6_K_BYTES) & ~(int64_t)15 : (int64_t)sbg * SB;
#pragma unroll
        for (int l = 0; l < NL; ++l) {
            const int p = min(64 * l + lane, NP - 1);
            const int rr = p / PPR, c = p - rr * PPR;
            const int row = min(rg * 16 + rr, n - 1);
            const uint8_t* src = w + (int64_t)row * row_bytes + at + 16 * c + dep;
            pc[l] = __builtin_nontemporal_load((const u32x4*)src);
        }
    };
    auto to_slot = [&]() {
#pragma unroll
        for (int l = 0; l < NL; ++l)
            if (64 * l + lane < NP) *(u32x4*)(slot + 16 * (64 * l + lane)) = pc[l];
    };

    // ---- activation staging, its loads issued before item 0's ----
    const int n8 = kce / 8;  // 8-element groups per activation row of this split
    uint32_t dep;
    if constexpr (FUSED) {
        // groups i = threadIdx.x + 1024 j of the MP x n8 grid (MP x kc <= 64K elements, so
        // j < 8); a quad of lanes holds one 32-element block
        f32x4 xv[8][2];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = min((int)threadIdx.x + 1024 * j, MP * n8 - 1);
            const int t = min(i / n8, m - 1), g8 = i % n8;
            const f32x4* src = (const f32x4*)(x + (size_t)t * k + k0 + 8 * g8);
            xv[j][0] = src[0];
            xv[j][1] = src[1];
        }
        dep = opaque_zero(x);
        load_item(0, dep);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int i = threadIdx.x + 1024 * j;
            if (i < MP * n8) {  // whole quads: MP * n8 and 1024 are multiples of 4
                const int t = i / n8, g8 = i % n8;
                const bool live = t < m;
                const float e[8] = {live ? xv[j][0].x : 0.0f, live ? xv[j][0].y : 0.0f,
                                    live ? xv[j][0].z : 0.0f, live ? xv[j][0].w : 0.0f,
                                    live ? xv[j][1].x : 0.0f, live ? xv[j][1].y : 0.0f,
                                    live ? xv[j][1].z : 0.0f, live ? xv[j][1].w : 0.0f};
                uint32_t q[2];
                float d;
                int s8;
                q8_quant_quad(e, q, d, s8);
                *(u32x2*)(aq + (size_t)t * QSR + 8 * g8) = u32x2{q[0], q[1]};
                const int s16 = s8 + dpp_i32<DPP_QUAD_SWAP1>(s8);
                const int bsum = s16 + dpp_i32<DPP_QUAD_SWAP2>(s16);
                if ((g8 & 3) == 0) {
                    axd[t * nb + (g8 >> 2)] = d;
                    if constexpr (KQ) axm[t * nb + (g8 >> 2)] = d * (float)bsum;
                }
            }
        }
    } else {
        // the Q8_0 batch: 16-byte pieces of qs (MP x kce / 16 <= 4096, 4 per thread) and the
        // blocks' dx and bsum (MP x kce / 32 <= 2048, 2 per thread)
        const int n16 = kce / 16, n32 = kce / 32;
        u32x4 qv[4];
        float dv[2];
        int32_t bv[2];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = min((int)threadIdx.x + 1024 * j, MP * n16 - 1);
            const int t = min(i / n16, m - 1), c = i % n16;
            qv[j] = *(const u32x4*)(qs + (size_t)t * k + k0 + 16 * c);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int i = min((int)threadIdx.x + 1024 * j, MP * n32 - 1);
            const int t = min(i / n32, m - 1), b = i % n32;
            dv[j] = xs[(size_t)t * (k / 32) + k0 / 32 + b];
            bv[j] = KQ ? xb[(size_t)t * (k / 32) + k0 / 32 + b] : 0;
        }
        dep = opaque_zero(qs, xs, xb);
        if constexpr (!LATE) load_item(0, dep);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int i = threadIdx.x + 1024 * j;
            if (i < MP * n16) {
                const int t = i / n16, c = i % n16;
                *(u32x4*)(aq + (size_t)t * QSR + 16 * c) = t < m ? qv[j] : u32x4{0, 0, 0, 0};
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int i = threadIdx.x + 1024 * j;
            if (i < MP * n32) {
                const int t = i / n32, b = i % n32;
                axd[t * nb + b] = t < m ? dv[j] : 0.0f;
                if constexpr (KQ) axm[t * nb + b] = t < m ? dv[j] * (float)bv[j] : 0.0f;
            }
        }
        // LATE (one item per wave): its weights go out once the activations are in. Issued
        // beside them they share the first burst's queues, and the staging, which every wave
        // waits for, returns later. With more items the early item 0 starts the wave's chain
        // of round trips sooner.
        if constexpr (LATE) load_item(0, dep);
    }
    sm_barrier();

    // ---- main loop: this wave's items (row group rg, super-blocks kpart, kpart + kp, ..) ----
    f32x4 acc[MT];
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const i32x4 izero = {0, 0, 0, 0};
    const f32x4 fzero = {0.0f, 0.0f, 0.0f, 0.0f};
    auto compute_item = [&](int it) {
        const int sbl = kpart + kp * it;  // super-block within the split
        const uint8_t* rowp = slot + r * SB;  // this lane's A-fragment row
        u32x2 A[8];
        if constexpr (T == T_Q6_K) {
            // the super-block sits at byte sh of each slot row (even, the same for every row)
            const int sh = ((k0 / 256 + sbl) * Q6_K_BYTES) & 15;
            // 8 bytes at rowp + o (o even): two dword reads, or three realigned
            auto rd8 = [&](const uint8_t* base, int o) -> u32x2 {
                const uint8_t* q = base + o;  // 4-byte aligned when sh is, not 8
                if ((sh & 2) == 0) return u32x2{*(const uint32_t*)q, *(const uint32_t*)(q + 4)};
                const uint32_t d0 = *(const uint32_t*)(q - 2), d1 = *(const uint32_t*)(q + 2),
                               d2 = *(const uint32_t*)(q + 6);
                return u32x2{__builtin_amdgcn_alignbyte(d1, d0, 2), __builtin_amdgcn_alignbyte(d2, d1, 2)};
            };
            // block b = 4 half + jj holds elements 128 half + 32 jj + l (l < 32): low (jj < 2) or
            // high nibble of ql[64 half + 32 (jj & 1) + l], bits 2 jj of qh[32 half + l]; the
            // lane's 8 elements l = 8 g .. 8 g + 7 share the scale sc[2 b + g / 2]. As int8,
            // 4 (q - 32) = (q << 2) ^ 0x80 per byte, exact (|4 (q - 32)| <= 128).
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const u32x2 qh8 = rd8(rowp, sh + 128 + 32 * half + 8 * g);
#pragma unroll
                for (int jo = 0; jo < 2; ++jo) {
                    const u32x2 ql8 = rd8(rowp, sh + 64 * half + 32 * jo + 8 * g);
#pragma unroll
                    for (int hi = 0; hi < 2; ++hi) {
                        const int jj = jo + 2 * hi;
                        const u32x2 nib = hi ? ((ql8 >> 4) & 0x0F0F0F0Fu) : (ql8 & 0x0F0F0F0Fu);
                        const u32x2 hb = (qh8 >> (2 * jj)) & 0x03030303u;
                        A[4 * half + jj] = ((nib << 2) | (hb << 6)) ^ 0x80808080u;
                    }
                }
            }
            // the row's 16 scales to the table (lanes of g = 0), then the result rows' scales
            if (g == 0) {
                *(u32x2*)(tab + r * 16) = rd8(rowp, sh + 192);
                *(u32x2*)(tab + r * 16 + 8) = rd8(rowp, sh + 200);
            }
            u32x4 scr[4];
            float dq[4];  // the result rows' d / 4 (the weight operand holds 4 (q - 32))
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                scr[i] = *(const u32x4*)(tab + (4 * g + i) * 16);
                dq[i] = 0.25f * f16_to_f32(*(const uint16_t*)(slot + (4 * g + i) * SB + sh + 208));
            }
            const u32x2 zero2 = {0u, 0u};
#pragma unroll
            for (int j = 0; j < MT; ++j) {
                const int tok = 16 * j + r;
                const f32x4 dx0 = *(const f32x4*)(axd + tok * nb + sbl * 8);
                const f32x4 dx1 = *(const f32x4*)(axd + tok * nb + sbl * 8 + 4);
                const float dx[8] = {dx0.x, dx0.y, dx0.z, dx0.w, dx1.x, dx1.y, dx1.z, dx1.w};
                f32x4 sacc = fzero;
#pragma unroll
                for (int b = 0; b < 8; ++b) {
                    const u32x2 bq = *(const u32x2*)(aq + tok * QSR + sbl * 256 + 32 * b + 8 * g);
                    // the two 16-element halves of the block apart: lanes g < 2 hold the first
                    const i32x4 d0 = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                        as_long(g < 2 ? A[b] : zero2), as_long(bq), izero, 0, 0, 0);
                    const i32x4 d1 = __builtin_amdgcn_mfma_i32_16x16x32_i8(
                        as_long(g < 2 ? zero2 : A[b]), as_long(bq), izero, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t wsc = scr[i][b >> 1];
                        const int sc0 = __builtin_amdgcn_sbfe(wsc, 16 * (b & 1), 8);
                        const int sc1 = __builtin_amdgcn_sbfe(wsc, 16 * (b & 1) + 8, 8);
                        // |4 dot| <= 2^20 and |sc| <= 128: the 24-bit products are exact
                        const int v = __mul24(sc0, d0[i]) + __mul24(sc1, d1[i]);
                        sacc[i] = __builtin_fmaf((float)v, dx[b], sacc[i]);
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[j][i] = __builtin_fmaf(dq[i], sacc[i], acc[j][i]);
            }
        } else if constexpr (KQ) {
            constexpr int QS = T == T_Q5_K ? 48 : 16;
            u32x2 h = {0, 0};
            if constexpr (T == T_Q5_K) h = *(const u32x2*)(rowp + 16 + 8 * g);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u32x2 v = *(const u32x2*)(rowp + QS + 32 * j + 8 * g);
                A[2 * j] = v & 0x0F0F0F0Fu;
                A[2 * j + 1] = (v >> 4) & 0x0F0F0F0Fu;
                if constexpr (T == T_Q5_K) {
                    A[2 * j] |= ((h >> (2 * j)) & 0x01010101u) << 4;
                    A[2 * j + 1] |= ((h >> (2 * j + 1)) & 0x01010101u) << 4;
                }
            }
            // header: d | dmin, then the 12 scale bytes (get_scale_min_k4)
            const u32x4 hd = *(const u32x4*)rowp;
            int sc0, sc1, mg, mg4, unused;
            k4_scale_min(hd.y, hd.z, hd.w, 2 * g, sc0, unused);
            k4_scale_min(hd.y, hd.z, hd.w, 2 * g + 1, sc1, unused);
            k4_scale_min(hd.y, hd.z, hd.w, g, unused, mg);
            k4_scale_min(hd.y, hd.z, hd.w, g + 4, unused, mg4);
            const float dmin = f16_to_f32(hd.x >> 16);
            const float fa0 = dmin * (float)mg, fa1 = dmin * (float)mg4;
            *(uint16_t*)(tab + r * 8 + 2 * g) = (uint16_t)(sc0 | (sc1 << 8));
            // the result rows of this lane: 4 g + i; their d and their eight scales
            float dc[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) dc[i] = f16_to_f32(*(const uint16_t*)(slot + (4 * g + i) * SB));
            const u32x4 sa = *(const u32x4*)(tab + 32 * g), sb = *(const u32x4*)(tab + 32 * g + 16);
            const uint32_t scw[8] = {sa.x, sa.y, sa.z, sa.w, sb.x, sb.y, sb.z, sb.w};
#pragma unroll
            for (int j = 0; j < MT; ++j) {
                const int tok = 16 * j + r;
                const f32x4 dx0 = *(const f32x4*)(axd + tok * nb + sbl * 8);
                const f32x4 dx1 = *(const f32x4*)(axd + tok * nb + sbl * 8 + 4);
                const float dx[8] = {dx0.x, dx0.y, dx0.z, dx0.w, dx1.x, dx1.y, dx1.z, dx1.w};
                f32x4 s = fzero;
#pragma unroll
                for (int b = 0; b < 8; ++b) {
                    const u32x2 bq = *(const u32x2*)(aq + tok * QSR + sbl * 256 + 32 * b + 8 * g);
                    const i32x4 dd = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(A[b]), as_long(bq),
                                                                          izero, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int sc = (int)((scw[2 * i + (b >> 2)] >> (8 * (b & 3))) & 0xFFu);
                        // |dot| < 2^17 and sc < 64: the 24-bit multiply is exact (full rate)
                        s[i] = __builtin_fmaf((float)__mul24(dd[i], sc), dx[b], s[i]);
                    }
                }
                const float xm0 = axm[tok * nb + sbl * 8 + g], xm1 = axm[tok * nb + sbl * 8 + 4 + g];
                f32x4 mn = __builtin_amdgcn_mfma_f32_16x16x4f32(fa0, xm0, fzero, 0, 0, 0);
                mn = __builtin_amdgcn_mfma_f32_16x16x4f32(fa1, xm1, mn, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[j][i] = __builtin_fmaf(dc[i], s[i], acc[j][i]) - mn[i];
            }
        } else {
            // 32-element blocks: block b of row r at BB b, d (fp16) first. This lane's 8
            // elements are 8 g .. 8 g + 7 of each block:
            //   Q8_0: the 8 quant bytes at 2 + 8 g;
            //   Q4_0 / Q5_0: the low (g < 2) or high nibbles of the 8 qs bytes at QB + 8 (g & 1)
            //   (byte j holds elements j and j + 16); Q5_0 adds bit 8 g + i of its 4 qh bytes at
            //   2 as bit 4 of element i. As int8, q - 8 = (q + 0x78) ^ 0x80 and q - 16 =
            //   (q + 0x70) ^ 0x80 per byte (no carry leaves a byte), exact.
            // Every block starts 2 bytes past a 4-byte boundary when b is even (BB = 2 mod 4),
            // so even blocks' 8 bytes are realigned from three dword reads.
            constexpr int BB = T == T_Q8_0 ? Q8_0_BYTES : T == T_Q4_0 ? Q4_0_BYTES : Q5_0_BYTES;
            constexpr int QB = T == T_Q5_0 ? 6 : 2;  // quant bytes within a block
#pragma unroll
            for (int b = 0; b < 8; ++b) {
                const int a = BB * b + QB + (T == T_Q8_0 ? 8 * g : 8 * (g & 1));
                u32x2 v;
                if ((b & 1) != 0) {
                    v = u32x2{*(const uint32_t*)(rowp + a), *(const uint32_t*)(rowp + a + 4)};
                } else {
                    const uint32_t d0 = *(const uint32_t*)(rowp + a - 2);
                    const uint32_t d1 = *(const uint32_t*)(rowp + a + 2);
                    const uint32_t d2 = *(const uint32_t*)(rowp + a + 6);
                    v = u32x2{__builtin_amdgcn_alignbyte(d1, d0, 2), __builtin_amdgcn_alignbyte(d2, d1, 2)};
                }
                if constexpr (T == T_Q8_0) {
                    A[b] = v;
                } else {
                    u32x2 q = g < 2 ? (v & 0x0F0F0F0Fu) : ((v >> 4) & 0x0F0F0F0Fu);
                    if constexpr (T == T_Q5_0) {
                        // bits i of the qh byte to bit 4 of byte i: x * 0x00204081 puts bit i of
                        // a 4-bit x at bit 8 i (among others off those positions)
                        const uint32_t hb = rowp[BB * b + 2 + g];
                        const uint32_t s0 = ((hb & 0xFu) * 0x00204081u) & 0x01010101u;
                        const uint32_t s1 = ((hb >> 4) * 0x00204081u) & 0x01010101u;
                        q = q | (u32x2{s0, s1} << 4);
                        A[b] = (q + 0x70707070u) ^ 0x80808080u;
                    } else {
                        A[b] = (q + 0x78787878u) ^ 0x80808080u;
                    }
                }
            }
            // the blocks' d: this lane converts those of row r, blocks 2 g and 2 g + 1, into
            // the table [block][row]; the result rows 4 g + i read theirs back per block
            float* dt = (float*)tab;
            dt[(2 * g) * 16 + r] = f16_to_f32(*(const uint16_t*)(rowp + BB * (2 * g)));
            dt[(2 * g + 1) * 16 + r] = f16_to_f32(*(const uint16_t*)(rowp + BB * (2 * g + 1)));
            f32x4 dcb[8];
#pragma unroll
            for (int b = 0; b < 8; ++b) dcb[b] = *(const f32x4*)(dt + b * 16 + 4 * g);
#pragma unroll
            for (int j = 0; j < MT; ++j) {
                const int tok = 16 * j + r;
                const f32x4 dx0 = *(const f32x4*)(axd + tok * nb + sbl * 8);
                const f32x4 dx1 = *(const f32x4*)(axd + tok * nb + sbl * 8 + 4);
                const float dx[8] = {dx0.x, dx0.y, dx0.z, dx0.w, dx1.x, dx1.y, dx1.z, dx1.w};
#pragma unroll
                for (int b = 0; b < 8; ++b) {
                    const u32x2 bq = *(const u32x2*)(aq + tok * QSR + sbl * 256 + 32 * b + 8 * g);
                    const i32x4 dd = __builtin_amdgcn_mfma_i32_16x16x32_i8(as_long(A[b]), as_long(bq),
                                                                          izero, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[j][i] = __builtin_fmaf((float)dd[i], dcb[b][i] * dx[b], acc[j][i]);
                }
            }
        }
    };
    for (int it = 0; it < items; ++it) {
        to_slot();
        if (it + 1 < items) load_item(it + 1, 0u);
        compute_item(it);
    }

    // ---- the kp parts of each row group, added in part order ----
    // The group's tile is MT x 64 entries e = 64 j + l (token tile j, accumulator lane l: token
    // 16 j + l % 16, rows 4 (l / 16) .. + 3 of the row group), one f32x4 each. Thread
    // t = 64 kpart + lane of the group owns entries t, t + 64 kp, ..; it adds the kp parts of
    // each in part order (bit for bit the order of one wave adding them one by one) and writes
    // the result, or its split's partial.
    sm_barrier();  // every wave is past its activation reads: the qs area becomes the sums
    f32x4* red = (f32x4*)lds;
    if (kp > 1) {
#pragma unroll
        for (int j = 0; j < MT; ++j) red[(wave * MT + j) * 64 + lane] = acc[j];
        sm_barrier();
    }
    const int t_own = 64 * kpart + lane;
    const int gw = wave - kpart;  // the group's first wave
    const bool live = rg < n_rg;
    f32x4 ev[MT];
    bool own[MT];
#pragma unroll
    for (int q = 0; q < MT; ++q) {
        const int e = t_own + 64 * kp * q;
        own[q] = live && e < 64 * MT;
        ev[q] = fzero;
        if (kp == 1) {
            ev[q] = acc[q];  // t_own = lane: entry 64 q + lane is this wave's tile j = q
        } else if (own[q]) {
            f32x4 v = red[gw * MT * 64 + e];
            for (int pq = 1; pq < kp; ++pq) v += red[(gw + pq) * MT * 64 + e];
            ev[q] = v;
        }
    }
    // writes entry q's values (token and rows from its entry index) plus the bias
    auto write_out = [&](const f32x4 (&v)[MT]) {
#pragma unroll
        for (int q = 0; q < MT; ++q) {
            if (!own[q]) continue;
            const int e = t_own + 64 * kp * q;
            const int tok = 16 * (e >> 6) + (e & 15);
            const int row0 = rg * 16 + 4 * ((e >> 4) & 3);
            if (tok >= m) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = row0 + i;
                if (row < n) y[(size_t)tok * n + row] = bias ? v[q][i] + bias[row] : v[q][i];
            }
        }
    };
    const int splits = (int)gridDim.y;
    if (splits == 1) {
        write_out(ev);
        return;
    }
    // split-K: this split's tile of sums to part[split][rg][e], as relaxed agent-scope 64-bit
    // atomic stores (coherent across XCDs by themselves); the last split of the row tile to
    // arrive adds all splits in split order
    uint64_t* pp = (uint64_t*)part;
    const size_t stride = (size_t)n_rg * MT * 128;  // 8-byte pairs per split
#pragma unroll
    for (int q = 0; q < MT; ++q) {
        if (!own[q]) continue;
        const size_t o = (size_t)blockIdx.y * stride + (size_t)rg * MT * 128 + 2 * (t_own + 64 * kp * q);
        const uint64_t a = (uint64_t)__float_as_uint(ev[q][0]) | ((uint64_t)__float_as_uint(ev[q][1]) << 32);
        const uint64_t b = (uint64_t)__float_as_uint(ev[q][2]) | ((uint64_t)__float_as_uint(ev[q][3]) << 32);
        __hip_atomic_store(pp + o, a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pp + o + 1, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores have completed
    __syncthreads();
    if (threadIdx.x == 0) {
        const int arrived = __hip_atomic_fetch_add(&counters[blockIdx.x], 1, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
        last_split = arrived == splits - 1;
        if (arrived == splits - 1)
            __hip_atomic_store(&counters[blockIdx.x], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last_split) return;
    f32x4 sum[MT];
#pragma unroll
    for (int q = 0; q < MT; ++q) sum[q] = fzero;
    for (int sp = 0; sp < splits; ++sp) {
#pragma unroll
        for (int q = 0; q < MT; ++q) {
            if (!own[q]) continue;
            f32x4 v = ev[q];
            if (sp != (int)blockIdx.y) {
                const size_t o = (size_t)sp * stride + (size_t)rg * MT * 128 + 2 * (t_own + 64 * kp * q);
                const uint64_t a = __hip_atomic_load(pp + o, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const uint64_t b = __hip_atomic_load(pp + o + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                v = f32x4{__uint_as_float((uint32_t)a), __uint_as_float((uint32_t)(a >> 32)),
                          __uint_as_float((uint32_t)b), __uint_as_float((uint32_t)(b >> 32))};
            }
            sum[q] = sp == 0 ? v : sum[q] + v;
        }
    }
    write_out(sum);
}

// ---- host side -----------------------------------------------------------------------

int sm_cus() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0, c = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && c > 0)
            cus = c;
        else
            cus = 256;
    }
    return cus;
}

struct SmPlan {
    int mt, kc, splits, kp, grid_x;
};

// Token tiles of 16; K split over workgroups in ranges that fit kSmActBytes (16 MT rows of
// int8 activations); the K parts per workgroup that bring the workgroup count closest to one
// per CU without exceeding it. From a batch quantized once a range may fill the activation LDS
// (16 rows span K = 4096 in one split: no split-K tail); the fused form (quantization inside
// every workgroup, of its K range) caps ranges at 1024 elements, since that redundant work
// grows with the range. Measured on MI355X (cold weights, us): from a quantized batch,
// Q5_K 14336x4096 at 16 rows 16.0 (1 split x 4 parts) against 18.6 (4 x 1); Q8_0 4096x4096 at
// 16 rows 9.7 (1 x 16) against 10.6 (4 x 4). Fused, at 16 rows: Q5_K 20.7 (4 x 1) against
// 21.2 (1 x 4), Q8_0 12.4 (4 x 4) against 14.0 (1 x 16).
SmPlan sm_plan(uint32_t type, int k, int n, int m, bool fused) {
    SmPlan p{};
    p.mt = (m + 15) / 16;
    const int nsb = k / 256;
    const int sb_act = std::max(1, kSmActBytes / (16 * p.mt) / 256);
    const int sb_max = fused ? std::min(4, sb_act) : sb_act;
    p.splits = (nsb + sb_max - 1) / sb_max;
    // the tuning knob "gemm_small_plan" (splits, K parts per workgroup) overrides the plan,
    // within what the activation LDS holds
    const int fs = tuning().gemm_small_splits.load(std::memory_order_relaxed);
    const int fk = tuning().gemm_small_kp.load(std::memory_order_relaxed);
    if (fs >= (nsb + sb_act - 1) / sb_act && fs <= nsb) p.splits = fs;
    p.kc = ((nsb + p.splits - 1) / p.splits) * 256;
    p.splits = (nsb * 256 + p.kc - 1) / p.kc;
    const int n_rg = (n + 15) / 16;
    const int cus = sm_cus();
    p.kp = 1;
    p.grid_x = n_rg;
    int best = -1;
    for (int kp = 1; kp <= kSmWaves; kp *= 2) {
        if (kp > p.kc / 256) break;
        const int gx = (n_rg + kSmWaves / kp - 1) / (kSmWaves / kp);
        const int wgs = gx * p.splits;
        if (wgs <= cus && wgs > best) {
            best = wgs;
            p.kp = kp;
            p.grid_x = gx;
        }
    }
    if (best < 0) {
        p.kp = 1;
        p.grid_x = (n_rg + kSmWaves - 1) / kSmWaves;
    }
    if (fk == 1 || fk == 2 || fk == 4 || fk == 8 || fk == 16) {
        if (fk <= p.kc / 256) {
            p.kp = fk;
            p.grid_x = (n_rg + kSmWaves / fk - 1) / (kSmWaves / fk);
        }
    }
    return p;
}

constexpr size_t kSmCounterBytes = 64 * 1024;  // the split-K region's tile counters

size_t sm_slices_bytes(const SmPlan& p, int n) {
    return (size_t)p.splits * ((n + 15) / 16) * p.mt * 1024;
}

template <uint32_t T, int MT, bool FUSED, bool LATE>
hipError_t launch_sm_k(const uint8_t* w, int k, int n, int m, const SmPlan& p, const float* x,
                        const int8_t* qs, const float* xs, const int32_t* xb, const float* bias,
                        float* y, float* part, int* counters, hipStream_t stream) {
    const size_t shmem = sm_layout<T, MT>(p.kc).total;
    static bool attr_set = false;
    if (!attr_set) {
        const hipError_t e = hipFuncSetAttribute((const void*)k_gemm_sm<T, MT, FUSED, LATE>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                                 (int)sm_layout<T, MT>(kSmActBytes / (16 * MT)).total);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const int64_t row_bytes = (int64_t)(k / block_elems(T)) * block_bytes(T);
    hipLaunchKernelGGL((k_gemm_sm<T, MT, FUSED, LATE>), dim3((unsigned)p.grid_x, (unsigned)p.splits),
                       dim3(64 * kSmWaves), shmem, stream, w, row_bytes, k, n, m, p.kc, p.kp, x, qs,
                       xs, xb, bias, y, part, counters);
    return hipGetLastError();
}


template <uint32_t T, bool FUSED>
hipError_t launch_sm_mt(const uint8_t* w, int k, int n, int m, const SmPlan& p, const float* x,
                        const int8_t* qs, const float* xs, const int32_t* xb, const float* bias,
                        float* y, float* part, int* counters, hipStream_t stream) {
    // from a quantized batch with one item per wave, item 0 goes out after the staging
    // (Q8_0 4096x4096, us: 16 rows 11.71 -> 11.39, 64 rows 19.39 -> 19.06; with four items per
    // wave, Q5_K 14336x4096 at 16 rows, the late issue lost: 17.94 -> 18.50)
    if constexpr (!FUSED) {
        if (p.kc <= 256 * p.kp) {
            switch (p.mt) {
                case 1: return launch_sm_k<T, 1, false, true>(w, k, n, m, p, x, qs, xs, xb, bias, y, part, counters, stream);
                case 2: return launch_sm_k<T, 2, false, true>(w, k, n, m, p, x, qs, xs, xb, bias, y, part, counters, stream);
                case 3: return launch_sm_k<T, 3, false, true>(w, k, n, m, p, x, qs, xs, xb, bias, y, part, counters, stream);
                case 4: return launch_sm_k<T, 4, false, true>(w, k, n, m, p, x, qs, xs, xb, bias, y, part, counters, stream);
                default: return hipErrorInvalidValue;
            }
        }
    }
    switch (p.mt) {
        case 1: return launch_sm_k<T, 1, FUSED, false>(w, k, n, m, p, x, qs, xs, xb, bias, y, part, counters, stream);
        case 2: return launch_sm_k<T, 2, FUSED, false>(w, k, n, m, p, x, qs, xs, xb, bias, y, part, counters, stream);
        case 3: return launch_sm_k<T, 3, FUSED, false>(w, k, n, m, p, x, qs, xs, xb, bias, y, part, counters, stream);
        case 4: return launch_sm_k<T, 4, FUSED, false>(w, k, n, m, p, x, qs, xs, xb, bias, y, part, counters, stream);
        default: return hipErrorInvalidValue;
    }
}

template <bool FUSED>
hipError_t launch_sm(uint32_t type, const uint8_t* w, int k, int n, int m, const float* x,
                     const int8_t* qs, const float* xs, const int32_t* xb, const float* bias,
                     float* y, float* part, size_t part_bytes, hipStream_t stream) {
    if (!gemm_sm_supported(type, k, m)) return hipErrorNotSupported;
    const SmPlan p = sm_plan(type, k, n, m, FUSED);
    int* counters = nullptr;
    float* slices = nullptr;
    if (p.splits > 1) {
        if (part == nullptr || part_bytes < kSmCounterBytes + sm_slices_bytes(p, n) ||
            (size_t)p.grid_x * 4 > kSmCounterBytes)
            return hipErrorInvalidValue;
        counters = (int*)part;
        slices = (float*)((char*)part + kSmCounterBytes);
    }
    switch (type) {
        case T_Q4_K: return launch_sm_mt<T_Q4_K, FUSED>(w, k, n, m, p, x, qs, xs, xb, bias, y, slices, counters, stream);
        case T_Q5_K: return launch_sm_mt<T_Q5_K, FUSED>(w, k, n, m, p, x, qs, xs, xb, bias, y, slices, counters, stream);
        case T_Q8_0: return launch_sm_mt<T_Q8_0, FUSED>(w, k, n, m, p, x, qs, xs, xb, bias, y, slices, counters, stream);
        case T_Q4_0:  // Q4_0 / Q5_0 from a quantized batch only
            if constexpr (!FUSED)
                return launch_sm_mt<T_Q4_0, false>(w, k, n, m, p, x, qs, xs, xb, bias, y, slices, counters, stream);
            return hipErrorNotSupported;
        case T_Q5_0:
            if constexpr (!FUSED)
                return launch_sm_mt<T_Q5_0, false>(w, k, n, m, p, x, qs, xs, xb, bias, y, slices, counters, stream);
            return hipErrorNotSupported;
        case T_Q6_K:  // from a quantized batch only (the fused form would spill registers)
            if constexpr (!FUSED)
                return launch_sm_mt<T_Q6_K, false>(w, k, n, m, p, x, qs, xs, xb, bias, y, slices, counters, stream);
            return hipErrorNotSupported;
        default: return hipErrorNotSupported;
    }
}

}  // namespace

bool gemm_sm_supported(uint32_t type, int k, int m) {
    // Q6_K rows must be whole 16-byte pieces: k a multiple of 2048 (8 super-blocks)
    return (type == T_Q4_K || type == T_Q5_K || type == T_Q8_0 || type == T_Q4_0 || type == T_Q5_0 ||
            (type == T_Q6_K && k % 2048 == 0)) && k % 256 == 0 && k > 0 && m >= 1 && m <= 64;
}

// The split-K region of either plan (fused or from a quantized batch).
size_t gemm_sm_partial_bytes(uint32_t type, int k, int n, int m) {
    if (!gemm_sm_supported(type, k, m)) return 0;
    size_t bytes = 0;
    for (const bool fused : {false, true}) {
        const SmPlan p = sm_plan(type, k, n, m, fused);
        if (p.splits > 1) bytes = std::max(bytes, kSmCounterBytes + sm_slices_bytes(p, n));
    }
    return bytes;
}

void gemm_sm_plan_name(uint32_t type, int k, int n, int m, bool fused, char* buf, size_t cap) {
    const SmPlan p = sm_plan(type, k, n, m, fused);
    snprintf(buf, cap, "k_gemm_sm<%s,%d> splits=%d kp=%d",
             type == T_Q8_0 ? "Q8_0" : type == T_Q5_K ? "Q5_K" : type == T_Q6_K ? "Q6_K"
             : type == T_Q4_0 ? "Q4_0" : type == T_Q5_0 ? "Q5_0" : "Q4_K",
             p.mt, p.splits, p.kp);
}

hipError_t launch_gemm_sm_f32(uint32_t type, const uint8_t* w, int k, int n, int m, const float* x,
                              const float* bias, float* y, float* part, size_t part_bytes,
                              hipStream_t stream) {
    return launch_sm<true>(type, w, k, n, m, x, nullptr, nullptr, nullptr, bias, y, part,
                           part_bytes, stream);
}

hipError_t launch_gemm_sm_q8(uint32_t type, const uint8_t* w, int k, int n, int m,
                             const int8_t* qs, const float* xs, const int32_t* xb,
                             const float* bias, float* y, float* part, size_t part_bytes,
                             hipStream_t stream) {
    return launch_sm<false>(type, w, k, n, m, nullptr, qs, xs, xb, bias, y, part, part_bytes,
                            stream);
}

}  // namespace cllm_hip
