// k_gemmw.hip -- prefill GEMM with the weights as the MFMA row operand (gfx950).
//
// y[m, n] = sum_s [ d[n,s] * sum_{b in s} dx[m,b] * sc[n,b] * I[m,n,b]
//                 - dmin[n,s] * sum_{b in s} mn[n,b] * (dx * bsum)[m,b] ]   (+ bias[n])
// -- the reference's per-block terms for Q4_K (src/core/quant.cpp:549-590, accumulated over
// rows in 1453-1464), with I[m,n,b] the exact integer dot of block b.
//
// Exact-integer fp16 MFMA. Weight operand A holds sc * q (q <= 15, sc <= 63: at most 945,
// exact in fp16), activation operand B holds the Q8_0 integers (|q_x| <= 128, exact), so one
// block's v_mfma_f32_32x32x16_f16 pair returns sc * I exactly (32-element sums < 2^24). With
// the weight rows on the MFMA's row side every lane's output column is one token, so the
// activation scale dx[m, b] is one scalar per lane and the per-block epilogue is a single FMA
// per output (sacc += dx * F). d is applied once per super-block, the minimum term once per
// half super-block on v_mfma_f32_32x32x16_bf16: the 4 block minima (6-bit integers, exact in
// bf16) against dx*bsum split into three bf16 parts (hi + mid + lo, 24 significant bits).
//
// Tiling. A workgroup of W waves owns 32 W weight rows x 32 MT tokens; wave w owns weight rows
// 32w .. 32w+31 (one MFMA tile) against all MT token tiles, so each wave unpacks only its own
// rows, straight from the raw bytes in LDS into MFMA fragments, and the token fragments in LDS
// are shared by all waves. K advances half a super-block (128 elements) per stage through two
// LDS buffers, filled one stage ahead: the raw Q4_K bytes of the half (header + 64 quant
// bytes per row) and dx by direct-to-LDS loads (global_load_lds); the int8 activations
// through registers, widened to fp16 (16-byte chunks XOR-swizzled by token) on the way in;
// dx * bsum likewise, split into bf16 parts.
#include <cstdio>
#include <cstdlib>

#include "device_utils.h"
#include "ggml_blocks.h"
#include "launch.h"

namespace cllm_hip {

namespace {

typedef _Float16 wh2 __attribute__((ext_vector_type(2)));
typedef _Float16 wh8 __attribute__((ext_vector_type(8)));
typedef __bf16 wbf8 __attribute__((ext_vector_type(8)));
typedef float wf16 __attribute__((ext_vector_type(16)));
typedef uint32_t wu4 __attribute__((ext_vector_type(4)));

constexpr int kKS = 128;        // K elements per stage
constexpr int kWRow = 80;       // LDS bytes per weight row per stage: header + 64 qs bytes
constexpr int kWChunks = kWRow / 16;
constexpr int kXpStride = 48;   // bytes per token: hi[4] mid[4] lo[4] 0[4] bf16 + 16 pad

template <int W, int NT, int MT>
struct Cfg {
    static constexpr int THREADS = 64 * W;
    static constexpr int BN = 32 * NT * W;
    static constexpr int BM = 32 * MT;
    // LDS layout of one stage
    static constexpr int ACT = BM * 256;          // [token][16 chunks of 8 fp16], swizzled
    static constexpr int DX = 4 * BM * 4;         // [block][token] fp32
    static constexpr int XP = BM * kXpStride;     // [token][...]
    static constexpr int WB = BN * kWRow;         // [row][80]
    static constexpr int OFF_DX = ACT;
    static constexpr int OFF_XP = OFF_DX + DX;
    static constexpr int OFF_W = OFF_XP + XP;
    static constexpr int STAGE = OFF_W + WB;
    static constexpr int SCRATCH = W * NT * 64 * 4;  // per wave and tile: d[32], dmin[32]
    static constexpr int LDS = 2 * STAGE + SCRATCH;
    static_assert(LDS <= 160 * 1024, "LDS budget");
    // loader work per stage
    static constexpr int A_CHUNKS = BM * 8;       // 16-byte int8 chunks of activations
    static constexpr int A_SLOTS = (A_CHUNKS + THREADS - 1) / THREADS;
    static constexpr int W_LOADS = BN * kWChunks / 64;   // wave-loads of raw weights
    static constexpr int W_SLOTS = (W_LOADS + W - 1) / W;
    static constexpr int DX_LOADS = 4 * BM / 64;          // wave-loads of dx
    static constexpr int DX_SLOTS = (DX_LOADS + W - 1) / W;
    static constexpr int P_VALS = 4 * BM;                 // dx * bsum values
    static constexpr int P_SLOTS = (P_VALS + THREADS - 1) / THREADS;
};

typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ void lds_load16(const void* g, uint8_t* lds_base) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_base, 16, 0, 0);
}
__device__ __forceinline__ void lds_load4(const void* g, uint8_t* lds_base) {
    __builtin_amdgcn_global_load_lds(g, (lds_void*)lds_base, 4, 0, 0);
}

// Waits for this wave's outstanding vector-memory loads (including direct-to-LDS ones).
__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// fp32 -> bf16 bits, round to nearest even (finite inputs).
__device__ __forceinline__ uint32_t bf16_bits(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}
__device__ __forceinline__ float bf16_val(uint32_t b) { return __builtin_bit_cast(float, b << 16); }

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

}  // namespace

template <int W, int NT, int MT>
__global__ __launch_bounds__(64 * W) void k_gemmw_q4k(const uint8_t* __restrict__ w,
                                                      uint32_t row_bytes, int k, int n, int m,
                                                      const int8_t* __restrict__ qs,
                                                      const float* __restrict__ xs,
                                                      const int32_t* __restrict__ xb,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ y) {
    using C = Cfg<W, NT, MT>;
    constexpr int BM = C::BM;
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    const int r32 = lane & 31;

    // Workgroup -> (weight block, token block). Hardware hands consecutive workgroups to the
    // 8 XCDs in turn; renumber so the token blocks of one weight block share an XCD's L2.
    const int mb_count = (m + BM - 1) / BM;
    const int g = gridDim.x;
    const int bid = blockIdx.x;
    const int lin = (g % 8 == 0) ? (bid % 8) * (g / 8) + bid / 8 : bid;
    const int nblk = lin / mb_count, mblk = lin - nblk * mb_count;
    const int n0 = nblk * C::BN, m0 = mblk * BM;
    const int nb = k / 32;
    const int stages = k / kKS;

    // ---- per-lane load offsets (stage 0); each stage adds a uniform step -----------------
    uint32_t a_off[C::A_SLOTS];     // activation chunk: byte offset into qs
    int a_dst[C::A_SLOTS];          // LDS byte offset of its low fp16 chunk (-1: none)
#pragma unroll
    for (int j = 0; j < C::A_SLOTS; ++j) {
        const int i = tid + j * C::THREADS;
        const int ic = min(i, C::A_CHUNKS - 1);
        const int tok = ic >> 3, c8 = ic & 7;
        a_off[j] = (uint32_t)min(m0 + tok, m - 1) * (uint32_t)k + 16u * c8;
        a_dst[j] = i < C::A_CHUNKS ? tok * 256 + 16 * ((2 * c8) ^ (tok & 15)) : -1;
    }
    uint32_t w_off[C::W_SLOTS];     // raw weight chunk: byte offset into w
    bool w_q[C::W_SLOTS];           // quant bytes (the offset moves with the stage half)
#pragma unroll
    for (int j = 0; j < C::W_SLOTS; ++j) {
        const int p = min((wave * C::W_SLOTS + j) * 64 + lane, C::W_LOADS * 64 - 1);
        const int row = p / kWChunks, piece = p - row * kWChunks;
        w_off[j] = (uint32_t)min(n0 + row, n - 1) * row_bytes +
                   (piece == 0 ? 0u : (uint32_t)(Q4_K_QS + 16 * (piece - 1)));
        w_q[j] = piece != 0;
    }
    uint32_t dx_off[C::DX_SLOTS];   // dx: [block][token], wave-load wave + j W
#pragma unroll
    for (int j = 0; j < C::DX_SLOTS; ++j) {
        const int p = min(wave + j * W, C::DX_LOADS - 1) * 64 + lane;
        const int b = p / BM, tok = p - b * BM;
        dx_off[j] = (uint32_t)min(m0 + tok, m - 1) * (uint32_t)nb + b;
    }
    uint32_t p_off[C::P_SLOTS];     // dx * bsum value: element offset into xs / xb
#pragma unroll
    for (int j = 0; j < C::P_SLOTS; ++j) {
        const int i = min(tid + j * C::THREADS, C::P_VALS - 1);
        const int tok = i >> 2, b = i & 3;
        p_off[j] = (uint32_t)min(m0 + tok, m - 1) * (uint32_t)nb + b;
    }

    struct Pending {
        wu4 a[C::A_SLOTS];
        float d[C::P_SLOTS];
        int32_t bs[C::P_SLOTS];
    };
    auto issue_stage = [&](int s, uint8_t* st, Pending& pd) {
        const int sb = s >> 1, half = s & 1;
#pragma unroll
        for (int j = 0; j < C::A_SLOTS; ++j)
            pd.a[j] = *(const wu4*)(qs + a_off[j] + (uint32_t)s * kKS);
#pragma unroll
        for (int j = 0; j < C::W_SLOTS; ++j) {
            const int slot = wave * C::W_SLOTS + j;
            if (C::W_LOADS % W == 0 || slot < C::W_LOADS)
                lds_load16(w + w_off[j] + (uint32_t)sb * Q4_K_BYTES + (w_q[j] ? 64u * half : 0u),
                           st + C::OFF_W + slot * 1024);
        }
#pragma unroll
        for (int j = 0; j < C::DX_SLOTS; ++j) {
            const int wl = wave + j * W;
            if (C::DX_LOADS % W == 0 || wl < C::DX_LOADS)
                lds_load4(xs + dx_off[j] + (uint32_t)s * 4, st + C::OFF_DX + wl * 256);
        }
#pragma unroll
        for (int j = 0; j < C::P_SLOTS; ++j) {
            pd.d[j] = xs[p_off[j] + (uint32_t)s * 4];
            pd.bs[j] = xb[p_off[j] + (uint32_t)s * 4];
        }
    };
    auto commit_stage = [&](uint8_t* st, const Pending& pd) {
#pragma unroll
        for (int j = 0; j < C::A_SLOTS; ++j) {
            if (a_dst[j] >= 0) {
                // logical chunks 2 c8 and 2 c8 + 1 of the token: swizzled indices differ in bit 0
                *(wu4*)(st + a_dst[j]) = int8x8_to_h8(pd.a[j].x, pd.a[j].y);
                *(wu4*)(st + (a_dst[j] ^ 16)) = int8x8_to_h8(pd.a[j].z, pd.a[j].w);
            }
        }
#pragma unroll
        for (int j = 0; j < C::P_SLOTS; ++j) {
            const int i = tid + j * C::THREADS;
            if (i < C::P_VALS) {
                const int tok = i >> 2, b = i & 3;
                const float pv = pd.d[j] * (float)pd.bs[j];
                const uint32_t hi = bf16_bits(pv);
                const float r1 = pv - bf16_val(hi);
                const uint32_t mid = bf16_bits(r1);
                const uint32_t lo = bf16_bits(r1 - bf16_val(mid));
                uint16_t* p = (uint16_t*)(st + C::OFF_XP + tok * kXpStride);
                p[b] = (uint16_t)hi;
                p[4 + b] = (uint16_t)mid;
                p[8 + b] = (uint16_t)lo;
                p[12 + b] = 0;
            }
        }
    };

    wf16 sacc[NT][MT], yacc[NT][MT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int a = 0; a < MT; ++a)
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[t][a][r] = yacc[t][a][r] = 0.0f;

    float* scratch = (float*)(lds + 2 * C::STAGE) + wave * NT * 64;

    {
        Pending pd;
        issue_stage(0, lds, pd);
        wait_vm();
        commit_stage(lds, pd);
    }
    __syncthreads();

    for (int s = 0; s < stages; ++s) {
        uint8_t* cur = lds + (s & 1) * C::STAGE;
        uint8_t* nxt = lds + ((s + 1) & 1) * C::STAGE;
        Pending pd;
        const bool more = s + 1 < stages;
        if (more) issue_stage(s + 1, nxt, pd);
        const int half = s & 1;

        // this lane's weight rows: row r32 of each of the wave's NT tiles
        const uint8_t* wr[NT];
        wu4 hdr[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            wr[t] = cur + C::OFF_W + ((wave * NT + t) * 32 + r32) * kWRow;
            hdr[t] = *(const wu4*)wr[t];
        }
        const uint8_t* act = cur;
        const float* dxl = (const float*)(cur + C::OFF_DX);

#pragma unroll 1
        for (int pc = 0; pc < 2; ++pc) {
            const int c = 2 * half + pc;
            // A fragments: sub-block 2c (low nibbles) and 2c+1 (high nibbles), K steps j = 0, 1
            wh8 afr[NT][2][2];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const wu4 q = *(const wu4*)(wr[t] + 16 * (1 + 2 * pc + h));
                int sa, ma, sb, mb;
                k4_sm(2 * c, hdr[t].y, hdr[t].z, hdr[t].w, sa, ma);
                k4_sm(2 * c + 1, hdr[t].y, hdr[t].z, hdr[t].w, sb, mb);
                const _Float16 fa = (_Float16)sa, fb = (_Float16)(sb * 0.0625f);
                const _Float16 ca = (_Float16)(-1024.0f * sa), cb = (_Float16)(-64.0f * sb);
                const wh2 s_lo = {fa, fa}, c_lo = {ca, ca};
                const wh2 s_hi = {fb, fb}, c_hi = {cb, cb};
                afr[t][0][0] = scaled8(q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu, s_lo, c_lo);
                afr[t][0][1] = scaled8(q.z & 0x0F0F0F0Fu, q.w & 0x0F0F0F0Fu, s_lo, c_lo);
                afr[t][1][0] = scaled8(q.x & 0xF0F0F0F0u, q.y & 0xF0F0F0F0u, s_hi, c_hi);
                afr[t][1][1] = scaled8(q.z & 0xF0F0F0F0u, q.w & 0xF0F0F0F0u, s_hi, c_hi);
            }
#pragma unroll
            for (int blk = 0; blk < 2; ++blk) {
                const int b = 2 * pc + blk;  // block within the stage
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const int tok = mt * 32 + r32;
                    const wh8 b0 = *(const wh8*)(act + tok * 256 + 16 * ((4 * b + 2 * h) ^ (tok & 15)));
                    const wh8 b1 = *(const wh8*)(act + tok * 256 + 16 * ((4 * b + 2 * h + 1) ^ (tok & 15)));
                    const float dxv = dxl[b * BM + tok];
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        wf16 f = {};
                        f = __builtin_amdgcn_mfma_f32_32x32x16_f16(afr[t][blk][0], b0, f, 0, 0, 0);
                        f = __builtin_amdgcn_mfma_f32_32x32x16_f16(afr[t][blk][1], b1, f, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 16; ++r) sacc[t][mt][r] = fmaf(dxv, f[r], sacc[t][mt][r]);
                    }
                }
            }
        }

        // minimum term of this half: minima of sub-blocks 4 half .. 4 half + 3; d at the end
        // of the super-block
        {
            const uint8_t* xpl = cur + C::OFF_XP;
            wbf8 xbv[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                xbv[mt] = *(const wbf8*)(xpl + (mt * 32 + r32) * kXpStride + 16 * h);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                uint32_t mq[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    int scj, mnj;
                    k4_sm(4 * half + j, hdr[t].y, hdr[t].z, hdr[t].w, scj, mnj);
                    mq[j] = bf16_bits((float)mnj);
                }
                const uint32_t m01 = mq[0] | (mq[1] << 16), m23 = mq[2] | (mq[3] << 16);
                const wbf8 amq = __builtin_bit_cast(wbf8, wu4{m01, m23, m01, m23});
                float* sc_t = scratch + t * 64;
                if (h == 0) {
                    sc_t[r32] = f16_to_f32(hdr[t].x & 0xFFFFu);
                    sc_t[32 + r32] = f16_to_f32(hdr[t].x >> 16);
                }
                float dmr[16];
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const float4 mv = *(const float4*)(sc_t + 32 + 8 * q4 + 4 * h);
                    dmr[4 * q4] = mv.x; dmr[4 * q4 + 1] = mv.y; dmr[4 * q4 + 2] = mv.z; dmr[4 * q4 + 3] = mv.w;
                }
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    wf16 fm = {};
                    fm = __builtin_amdgcn_mfma_f32_32x32x16_bf16(amq, xbv[mt], fm, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; ++r) yacc[t][mt][r] = fmaf(-dmr[r], fm[r], yacc[t][mt][r]);
                }
                if (half == 1) {
                    float dr[16];
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4) {
                        const float4 dv = *(const float4*)(sc_t + 8 * q4 + 4 * h);
                        dr[4 * q4] = dv.x; dr[4 * q4 + 1] = dv.y; dr[4 * q4 + 2] = dv.z; dr[4 * q4 + 3] = dv.w;
                    }
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                        for (int r = 0; r < 16; ++r) {
                            yacc[t][mt][r] = fmaf(dr[r], sacc[t][mt][r], yacc[t][mt][r]);
                            sacc[t][mt][r] = 0.0f;
                        }
                }
            }
        }

        if (more) {
            wait_vm();
            commit_stage(nxt, pd);
        }
        __syncthreads();
    }

    // ---- output: lane holds rows 8q + 4h + (0..3) of each tile, token column r32 ----------
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int tok = m0 + mt * 32 + r32;
            if (tok >= m) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = n0 + (wave * NT + t) * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row < n) {
                    float v = yacc[t][mt][r];
                    if (bias) v += bias[row];
                    y[(size_t)tok * n + row] = v;
                }
            }
        }
}

bool gemmw_supported(uint32_t type) { return type == T_Q4_K; }

template <int W, int NT, int MT>
static hipError_t launch_cfg(const uint8_t* w, int k, int n, int m, const int8_t* qs,
                             const float* xs, const int32_t* xb, const float* bias, float* y,
                             hipStream_t stream) {
    using C = Cfg<W, NT, MT>;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)k_gemmw_q4k<W, NT, MT>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const uint32_t row_bytes = (uint32_t)(k / 256) * Q4_K_BYTES;
    const int tiles = ((n + C::BN - 1) / C::BN) * ((m + C::BM - 1) / C::BM);
    hipLaunchKernelGGL((k_gemmw_q4k<W, NT, MT>), dim3((unsigned)tiles), dim3(C::THREADS), C::LDS,
                       stream, w, row_bytes, k, n, m, qs, xs, xb, bias, y);
    return hipGetLastError();
}

hipError_t launch_gemmw(uint32_t type, const uint8_t* w, int k, int n, int m, const int8_t* qs,
                        const float* xs, const int32_t* xb, const float* bias, float* y,
                        hipStream_t stream) {
    if (type != T_Q4_K || k % 256 != 0) return hipErrorNotSupported;
    // the kernel indexes with 32-bit offsets
    if ((uint64_t)n * (uint64_t)(k / 256) * Q4_K_BYTES >= (1ull << 32) ||
        (uint64_t)m * (uint64_t)k >= (1ull << 32))
        return hipErrorNotSupported;
    // Tile shape: CLLM_HIP_GEMMW_CFG="<waves>,<weight tiles per wave>,<token tiles>" (for
    // sweeps), else by the grid size.
    int wv = 0, nt = 0, mt = 0;
    if (const char* e = getenv("CLLM_HIP_GEMMW_CFG")) {
        if (sscanf(e, "%d,%d,%d", &wv, &nt, &mt) != 3) wv = nt = mt = 0;
    }
    if (wv == 0) {
        // Measured on MI355X at m = 512: 256 x 128 tiles (8 waves) when they fill the CUs
        // (n = 14336: 163 us), else 128 x 32 tiles (4 waves; n = 4096: 74 us against 137 us).
        int cus = 256, dev = 0, c = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && c > 0)
            cus = c;
        const int big = ((n + 255) / 256) * ((m + 127) / 128);
        if (big >= cus * 3 / 4) {
            wv = 8, nt = 1, mt = 4;
        } else {
            wv = 4, nt = 1, mt = 1;
        }
    }
#define CLLM_GEMMW_CASE(A, B, D) \
    if (wv == A && nt == B && mt == D) return launch_cfg<A, B, D>(w, k, n, m, qs, xs, xb, bias, y, stream);
    CLLM_GEMMW_CASE(8, 1, 4)
    CLLM_GEMMW_CASE(8, 1, 2)
    CLLM_GEMMW_CASE(8, 2, 2)
    CLLM_GEMMW_CASE(4, 2, 4)
    CLLM_GEMMW_CASE(4, 2, 2)
    CLLM_GEMMW_CASE(4, 1, 2)
    CLLM_GEMMW_CASE(4, 1, 1)
#undef CLLM_GEMMW_CASE
    return hipErrorNotSupported;
}

}  // namespace cllm_hip
