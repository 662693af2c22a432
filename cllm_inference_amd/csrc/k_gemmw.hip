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
// LDS buffers, filled one stage ahead, every operand by direct-to-LDS loads (global_load_lds):
// the raw Q4_K bytes of the half (header + 64 quant bytes per row), dx, the activations as
// fp16 integers (16-byte chunks swizzled by token, so the fragment reads of 16 consecutive
// tokens fall on distinct banks) and dx * bsum split into bf16 parts.
#include <cstdio>
#include <cstdlib>

#include "ggml_blocks.h"
#include "launch.h"
#include "mfma_common.h"

namespace cllm_hip {

namespace {

constexpr int kKS = 128;        // K elements per stage
// LDS bytes per weight row per stage: the 16-byte header, for Q5_K the super-block's 32 qh
// bytes, and the half super-block's 64 qs bytes
template <bool Q5>
constexpr int wrow_bytes() { return Q5 ? 112 : 80; }
constexpr int kActRow = 272;    // Q6_K kernel: LDS bytes per token, 128 fp16 + 16 of padding
constexpr int kXqRow = 64;      // bytes per token and super-block of the minimum operand

// Q4_K kernel. Every operand reaches LDS by direct-to-LDS loads (no register staging):
//   ACT  [token][16 chunks of 8 fp16], chunk c of token t stored at slot c ^ (t & 15), so the
//        16-byte fragment reads of 16 consecutive tokens fall on distinct banks;
//   DX   [token][4 blocks] fp32 (at least one wave-load);
//   XQ   [token][hi 8 | mid 8 | lo 8 | 0 8] bf16 for the super-block (stages of half 1 only);
//   W    [row][80] raw Q4_K bytes: 16-byte header, then the half super-block's 64 quant bytes
//        (Q5_K: [row][112], the 32 qh bytes between the two).
template <int W, int NT, int MT, bool Q5>
struct Cfg {
    static constexpr int THREADS = 64 * W;
    static constexpr int BN = 32 * NT * W;
    static constexpr int BM = 32 * MT;
    static constexpr int ACT = BM * 256;
    static constexpr int DX = BM * 16 < 1024 ? 1024 : BM * 16;
    static constexpr int XQ = BM * kXqRow;
    static constexpr int WROW = wrow_bytes<Q5>();
    static constexpr int WB = BN * WROW;
    static constexpr int OFF_DX = ACT;
    static constexpr int OFF_XQ = OFF_DX + DX;
    static constexpr int OFF_W = OFF_XQ + XQ;
    static constexpr int STAGE = OFF_W + WB;
    static constexpr int SCRATCH = W * NT * 64 * 4;  // per wave and tile: d[32], dmin[32]
    static constexpr int LDS = 2 * STAGE + SCRATCH;
    static_assert(LDS <= 160 * 1024, "LDS budget");
    // wave-loads (64 lanes x 16 or 4 bytes) per stage, spread over the W waves
    static constexpr int A_LOADS = ACT / 1024;
    static constexpr int A_SLOTS = (A_LOADS + W - 1) / W;
    static constexpr int W_LOADS = WB / 1024;
    static_assert(WB % 1024 == 0, "whole wave-loads of weight chunks");
    static constexpr int W_SLOTS = (W_LOADS + W - 1) / W;
    static constexpr int DX_LOADS = DX / 1024;
    static constexpr int DX_SLOTS = (DX_LOADS + W - 1) / W;
    static constexpr int XQ_LOADS = XQ / 1024;
    static constexpr int XQ_SLOTS = (XQ_LOADS + W - 1) / W;
};

// Output of a workgroup's tile: lane values val(i, r) for token tok(i) and weight row row(i, r),
// i < NI, r < 16. Without split-K they go to y (plus the bias). With split-K (gridDim.y > 1)
// each wave writes its whole share of the tile, bounds ignored, to its slot of split
// blockIdx.y in part, laid out [i][r / 2][lane] in 8-byte pairs so that every store
// instruction covers 512 contiguous bytes; the last split to finish the tile, found by a
// per-tile arrival counter that it resets, adds the slots in split order (its own from
// registers, so the sum does not depend on which split finished last), plus the bias, into y.
// No split waits for another.
//
// The slots cross XCDs, whose L2 caches are not coherent with each other. They are written
// and read as relaxed agent-scope atomics (loads and stores that are coherent device-wide by
// themselves), so no agent-scope fence is needed: such a fence writes back and invalidates
// the whole L2 of the XCD, under the feet of every other workgroup streaming through it.
// Each wave waits for its slot stores to complete before the workgroup barrier, and the
// counter is bumped after that barrier; the workgroup's LDS (free once every wave has left
// its main loop) carries the verdict.
template <int NI, int W, class Val, class Tok, class Row>
__device__ __forceinline__ void store_tile(int n, int m, const float* __restrict__ bias,
                                           float* __restrict__ y, float* __restrict__ part,
                                           int* __restrict__ counters, uint8_t* lds, int wave,
                                           Val val, Tok tok, Row row) {
    const int splits = (int)gridDim.y;
    // y (plus the bias): a token tile's 16 bias values are loaded together (rows past n
    // clamped), not one dependent load per output
    auto write_out = [&](auto get) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int t = tok(i);
            if (t >= m) continue;
            float bv[16];
            if (bias) {
#pragma unroll
                for (int r = 0; r < 16; ++r) bv[r] = bias[min(row(i, r), n - 1)];
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int j = row(i, r);
                if (j < n) y[(size_t)t * n + j] = bias ? get(i, r) + bv[r] : get(i, r);
            }
        }
    };
    if (splits == 1) {
        write_out(val);
        return;
    }
    constexpr int SLOT = NI * 8 * 64;  // 8-byte pairs per wave slot
    const size_t split_pairs = (size_t)gridDim.x * W * SLOT;
    const size_t slot = ((size_t)blockIdx.x * W + wave) * SLOT + (threadIdx.x & 63);
    uint64_t* __restrict__ pairs = (uint64_t*)part;
    auto pack = [&](int i, int r2) {
        return (uint64_t)__float_as_uint(val(i, 2 * r2)) |
               ((uint64_t)__float_as_uint(val(i, 2 * r2 + 1)) << 32);
    };
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int r2 = 0; r2 < 8; ++r2)
            __hip_atomic_store(pairs + blockIdx.y * split_pairs + slot + (i * 8 + r2) * 64,
                               pack(i, r2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's slot stores have completed
    __syncthreads();
    int* last = (int*)lds;
    if (threadIdx.x == 0) {
        const int arrived = __hip_atomic_fetch_add(&counters[blockIdx.x], 1, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
        *last = arrived == splits - 1;
        if (arrived == splits - 1)
            __hip_atomic_store(&counters[blockIdx.x], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!*last) return;
    float acc[NI][16];
    for (int sp = 0; sp < splits; ++sp) {
        const bool own = sp == (int)blockIdx.y;
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int r2 = 0; r2 < 8; ++r2) {
                float x0, x1;
                if (own) {
                    x0 = val(i, 2 * r2);
                    x1 = val(i, 2 * r2 + 1);
                } else {
                    const uint64_t b = __hip_atomic_load(
                        pairs + sp * split_pairs + slot + (i * 8 + r2) * 64, __ATOMIC_RELAXED,
                        __HIP_MEMORY_SCOPE_AGENT);
                    x0 = __uint_as_float((uint32_t)b);
                    x1 = __uint_as_float((uint32_t)(b >> 32));
                }
                acc[i][2 * r2] = sp == 0 ? x0 : acc[i][2 * r2] + x0;
                acc[i][2 * r2 + 1] = sp == 0 ? x1 : acc[i][2 * r2 + 1] + x1;
            }
    }
    write_out([&](int i, int r) { return acc[i][r]; });
}

}  // namespace

// Up to kMaxSegs weight matrices of one type and K over one activation batch, in one launch
// (the q, k and v projections, or gate and up): segment i has n[i] rows, its own bias and
// output, and owns the workgroups [tile_end[i - 1], tile_end[i]) of the grid's x dimension.
constexpr int kMaxSegs = 3;
struct Segs {
    const uint8_t* w[kMaxSegs];
    const float* bias[kMaxSegs];
    float* y[kMaxSegs];
    int n[kMaxSegs];
    int tile_end[kMaxSegs];
    int count;
};

template <int W, int NT, int MT, bool Q5>
__global__ __launch_bounds__(64 * W) void k_gemmw_q4k(Segs segs, uint32_t row_bytes, int k, int m,
                                                      const _Float16* __restrict__ qh,
                                                      const float* __restrict__ xs,
                                                      const uint16_t* __restrict__ xq,
                                                      float* __restrict__ part,
                                                      int* __restrict__ counters, int split_stages) {
    using C = Cfg<W, NT, MT, Q5>;
    constexpr int BM = C::BM;
    constexpr int WCH = C::WROW / 16;             // 16-byte pieces per weight row and stage
    constexpr int QS_AT = Q5 ? 48 : 16;           // qs bytes within an LDS row
    constexpr uint32_t SB_BYTES = Q5 ? Q5_K_BYTES : Q4_K_BYTES;
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane >> 5;
    const int r32 = lane & 31;

    // Workgroup -> (weight block, token block), token blocks fastest. Hardware hands
    // consecutive workgroups to the 8 XCDs in turn, so an XCD holds few token blocks of many
    // weight blocks. (Renumbering so that the token blocks of one weight block share an XCD,
    // as the Q6_K kernel does, measured slower here at M = 512: gate 127.3 against 125.2 us,
    // wq 52.9 against 51.9, wk 26.2 against 24.9.)
    const int mb_count = (m + BM - 1) / BM;
    // the workgroup's segment (wave-uniform), then its tile within the segment
    int seg = 0;
    while (seg + 1 < segs.count && (int)blockIdx.x >= segs.tile_end[seg]) ++seg;
    const int lin = (int)blockIdx.x - (seg ? segs.tile_end[seg - 1] : 0);
    const uint8_t* __restrict__ w = segs.w[seg];
    const float* __restrict__ bias = segs.bias[seg];
    float* __restrict__ y = segs.y[seg];
    const int n = segs.n[seg];
    const int nblk = lin / mb_count, mblk = lin - nblk * mb_count;
    const int n0 = nblk * C::BN, m0 = mblk * BM;
    const int nb = k / 32;
    // split-K: blockIdx.y owns stages [s_begin, s_end) (an even count: whole super-blocks);
    // store_tile completes the tile (the last split to arrive adds the partials and the bias)
    const int s_begin = blockIdx.y * split_stages;
    const int s_end = min(s_begin + split_stages, k / kKS);

    // ---- per-lane source offsets of this wave's load slots (stage 0; stages add a step) ----
    // Rows and tokens past the matrix are clamped to the last one (their results are dropped).
    uint32_t a_off[C::A_SLOTS];   // bytes into qh: token, swizzled 16-byte chunk
#pragma unroll
    for (int j = 0; j < C::A_SLOTS; ++j) {
        const int L = min(wave + j * W, C::A_LOADS - 1);
        const int t = 4 * L + (lane >> 4);                 // 4 tokens per wave-load
        const int c = (lane & 15) ^ (t & 15);              // chunk stored at slot lane & 15
        a_off[j] = ((uint32_t)min(m0 + t, m - 1) * (uint32_t)k + 8u * (uint32_t)c) * 2u;
    }
    uint32_t w_off[C::W_SLOTS];   // bytes into w
    bool w_q[C::W_SLOTS];         // quant bytes (the offset moves with the stage half)
#pragma unroll
    for (int j = 0; j < C::W_SLOTS; ++j) {
        const int L = min(wave + j * W, C::W_LOADS - 1);
        const int p = L * 64 + lane;
        const int row = p / WCH, piece = p - row * WCH;
        // header, (Q5_K) qh, then the qs bytes, which move with the stage half
        w_off[j] = (uint32_t)min(n0 + row, n - 1) * row_bytes + 16u * (uint32_t)piece;
        w_q[j] = 16 * piece >= QS_AT;
    }
    uint32_t dx_off[C::DX_SLOTS];  // elements into xs: a token's 4 blocks of the stage
#pragma unroll
    for (int j = 0; j < C::DX_SLOTS; ++j) {
        const int t = min(wave + j * W, C::DX_LOADS - 1) * 64 + lane;
        dx_off[j] = (uint32_t)min(m0 + t, m - 1) * (uint32_t)nb;
    }
    uint32_t q_off[C::XQ_SLOTS];   // bytes into xq: 16 tokens x 64 bytes per wave-load
#pragma unroll
    for (int j = 0; j < C::XQ_SLOTS; ++j) {
        const int L = min(wave + j * W, C::XQ_LOADS - 1);
        const int t = 16 * L + (lane >> 2);
        q_off[j] = (uint32_t)min(m0 + t, m - 1) * (uint32_t)(k / 256) * (uint32_t)kXqRow + 16u * (lane & 3);
    }

    // A stage's direct-to-LDS loads, in two parts issued before each half of the stage's MFMA
    // work: a wave's address unit accepts about one 16-byte wave-load per 16 cycles, so the
    // whole stage issued at once (right after a barrier, by every wave) stalls the waves for
    // ~1000 cycles. Offsets pass through pinned() so their address arithmetic is not hoisted
    // out of the MFMA loop (where it would hold registers the loop needs).
    auto issue_part = [&](int s, uint8_t* st, int part) {
        const int sb = s >> 1, half = s & 1;
        constexpr int AH = (C::A_SLOTS + 1) / 2, WH = (C::W_SLOTS + 1) / 2;
#pragma unroll
        for (int j = 0; j < C::A_SLOTS; ++j) {
            const int L = wave + j * W;
            if ((j < AH) == (part == 0) && (C::A_LOADS % W == 0 || L < C::A_LOADS))
                lds_load16((const uint8_t*)qh + pinned(a_off[j]) + (uint32_t)s * (2u * kKS), st + L * 1024);
        }
#pragma unroll
        for (int j = 0; j < C::W_SLOTS; ++j) {
            const int L = wave + j * W;
            if ((j < WH) == (part == 0) && (C::W_LOADS % W == 0 || L < C::W_LOADS))
                lds_load16(w + pinned(w_off[j]) + (uint32_t)sb * SB_BYTES + (w_q[j] ? 64u * half : 0u),
                           st + C::OFF_W + L * 1024);
        }
        if (part == 0) {
#pragma unroll
            for (int j = 0; j < C::DX_SLOTS; ++j) {
                const int L = wave + j * W;
                if (C::DX_LOADS % W == 0 || L < C::DX_LOADS)
                    lds_load16(xs + pinned(dx_off[j]) + (uint32_t)s * 4, st + C::OFF_DX + L * 1024);
            }
        } else if (half == 1) {
#pragma unroll
            for (int j = 0; j < C::XQ_SLOTS; ++j) {
                const int L = wave + j * W;
                if (C::XQ_LOADS % W == 0 || L < C::XQ_LOADS)
                    lds_load16((const uint8_t*)xq + pinned(q_off[j]) + (uint32_t)sb * kXqRow,
                               st + C::OFF_XQ + L * 1024);
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

    // this lane's weight row r32 of the wave's first tile, as an offset into a stage buffer
    const uint32_t woff = (uint32_t)C::OFF_W + (uint32_t)((wave * NT * 32 + r32) * C::WROW);

    // One stage: half HALF of a super-block. The host keeps every split's stage range even and
    // super-block aligned, so stage s sits in LDS buffer HALF = s & 1; the first block of each
    // super-block starts the scaled sums (sacc = dx * F), its last stage folds them into the
    // output sums (times d, minus the minimum term).
    auto run_stage = [&]<int HALF>(int s) {
        uint8_t* cur = lds + HALF * C::STAGE;
        uint8_t* nxt = lds + (1 - HALF) * C::STAGE;

        // this lane's weight rows: row r32 of each of the wave's NT tiles. The rows' d and dmin
        // go to this wave's scratch before the next stage's direct-to-LDS loads are issued: an
        // LDS store while those are in flight would make the compiler wait for all of them.
        wu4 hdr[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            hdr[t] = *(const wu4*)(cur + woff + t * 32 * C::WROW);
            if (h == 0 && HALF == 1) {
                float* sc_t = scratch + t * 64;
                sc_t[r32] = f16_to_f32(hdr[t].x & 0xFFFFu);
                sc_t[32 + r32] = f16_to_f32(hdr[t].x >> 16);
            }
        }
        const bool more = s + 1 < s_end;

        // blocks 2 PC and 2 PC + 1 of the stage (sub-blocks 2c and 2c + 1, c = 2 HALF + PC)
        auto blocks = [&](int PC) {
            const int c = 2 * HALF + PC;
            // A fragments: sub-block 2c (low nibbles) and 2c+1 (high nibbles), K steps j = 0, 1
            wh8 afr[NT][2][2];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const uint8_t* wr = cur + woff + t * 32 * C::WROW;
                const wu4 q = *(const wu4*)(wr + QS_AT + 32 * PC + 16 * h);
                int sa, ma, sb, mb;
                k4_sm(2 * c, hdr[t].y, hdr[t].z, hdr[t].w, sa, ma);
                k4_sm(2 * c + 1, hdr[t].y, hdr[t].z, hdr[t].w, sb, mb);
                const _Float16 fa = (_Float16)sa;
                const wh2 s_lo = {fa, fa};
                if constexpr (Q5) {
                    // 5-bit values: bit 2c (sub-block 2c) or 2c+1 of qh[l] above the nibble;
                    // sc * q <= 63 * 31 stays exact in fp16
                    const wu4 hb = *(const wu4*)(wr + 16 + 16 * h);
                    const uint32_t q4[4] = {q.x, q.y, q.z, q.w}, h4[4] = {hb.x, hb.y, hb.z, hb.w};
                    uint32_t lo[4], hi[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        lo[e] = (q4[e] & 0x0F0F0F0Fu) | (((h4[e] >> (2 * c)) & 0x01010101u) << 4);
                        hi[e] = ((q4[e] >> 4) & 0x0F0F0F0Fu) | (((h4[e] >> (2 * c + 1)) & 0x01010101u) << 4);
                    }
                    const _Float16 fb = (_Float16)sb;
                    const wh2 s_hi = {fb, fb};
                    const wh2 c_lo = {(_Float16)(-1024.0f * sa), (_Float16)(-1024.0f * sa)};
                    const wh2 c_hi = {(_Float16)(-1024.0f * sb), (_Float16)(-1024.0f * sb)};
                    afr[t][0][0] = scaled8(lo[0], lo[1], s_lo, c_lo);
                    afr[t][0][1] = scaled8(lo[2], lo[3], s_lo, c_lo);
                    afr[t][1][0] = scaled8(hi[0], hi[1], s_hi, c_hi);
                    afr[t][1][1] = scaled8(hi[2], hi[3], s_hi, c_hi);
                } else {
                    const _Float16 fb = (_Float16)(sb * 0.0625f);
                    const _Float16 ca = (_Float16)(-1024.0f * sa), cb = (_Float16)(-64.0f * sb);
                    const wh2 c_lo = {ca, ca};
                    const wh2 s_hi = {fb, fb}, c_hi = {cb, cb};
                    afr[t][0][0] = scaled8(q.x & 0x0F0F0F0Fu, q.y & 0x0F0F0F0Fu, s_lo, c_lo);
                    afr[t][0][1] = scaled8(q.z & 0x0F0F0F0Fu, q.w & 0x0F0F0F0Fu, s_lo, c_lo);
                    afr[t][1][0] = scaled8(q.x & 0xF0F0F0F0u, q.y & 0xF0F0F0F0u, s_hi, c_hi);
                    afr[t][1][1] = scaled8(q.z & 0xF0F0F0F0u, q.w & 0xF0F0F0F0u, s_hi, c_hi);
                }
            }
            auto block = [&]<int BLK, bool FRESH>() {
                const int b = 2 * PC + BLK;  // block within the stage
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const uint8_t* arow = cur + (mt * 32 + r32) * 256;
                    const int sw = r32 & 15;
                    const wh8 b0 = *(const wh8*)(arow + (((4 * b + 2 * h) ^ sw) << 4));
                    const wh8 b1 = *(const wh8*)(arow + (((4 * b + 2 * h + 1) ^ sw) << 4));
                    const float dxv = *(const float*)(cur + C::OFF_DX + (mt * 32 + r32) * 16 + 4 * b);
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        wf16 f = {};
                        f = __builtin_amdgcn_mfma_f32_32x32x16_f16(afr[t][BLK][0], b0, f, 0, 0, 0);
                        f = __builtin_amdgcn_mfma_f32_32x32x16_f16(afr[t][BLK][1], b1, f, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 16; ++r)
                            sacc[t][mt][r] = FRESH ? dxv * f[r] : fmaf(dxv, f[r], sacc[t][mt][r]);
                    }
                }
            };
            // the super-block's first block starts the scaled sums (PC is wave-uniform)
            if (HALF == 0 && PC == 0)
                block.template operator()<0, true>();
            else
                block.template operator()<0, false>();
            block.template operator()<1, false>();
        };
        // (a rolled loop: unrolled, the compiler interleaves the two block pairs and spills)
#pragma unroll 1
        for (int pc = 0; pc < 2; ++pc) {
            if (more) issue_part(s + 1, nxt, pc);
            blocks(pc);
        }

        // The next stage's loads have landed before the scratch is read (an LDS read while
        // direct-to-LDS loads are in flight waits for all of them anyway).
        if (more) wait_vm();

        // End of the super-block: the minimum term of its 8 sub-blocks, then d.
        //   fm = sum_b mn_b * (hi_b + mid_b + lo_b) as two bf16 MFMAs: the weight operand holds
        //   the 8 minima in both K halves, the token operand hi | mid, then lo | 0.
        if constexpr (HALF == 1) {
            const uint8_t* xql = cur + C::OFF_XQ;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                uint32_t mq[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    int scj, mnj;
                    k4_sm(j, hdr[t].y, hdr[t].z, hdr[t].w, scj, mnj);
                    mq[j] = bf16_bits((float)mnj);
                }
                const wbf8 amq = __builtin_bit_cast(
                    wbf8, wu4{mq[0] | (mq[1] << 16), mq[2] | (mq[3] << 16), mq[4] | (mq[5] << 16),
                              mq[6] | (mq[7] << 16)});
                const float* sc_t = scratch + t * 64;
                float dr[16], dmr[16];
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const float4 dv = *(const float4*)(sc_t + 8 * q4 + 4 * h);
                    const float4 mv = *(const float4*)(sc_t + 32 + 8 * q4 + 4 * h);
                    dr[4 * q4] = dv.x; dr[4 * q4 + 1] = dv.y; dr[4 * q4 + 2] = dv.z; dr[4 * q4 + 3] = dv.w;
                    dmr[4 * q4] = mv.x; dmr[4 * q4 + 1] = mv.y; dmr[4 * q4 + 2] = mv.z; dmr[4 * q4 + 3] = mv.w;
                }
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const uint8_t* q = xql + (mt * 32 + r32) * kXqRow + 16 * h;
                    wf16 fm = {};
                    fm = __builtin_amdgcn_mfma_f32_32x32x16_bf16(amq, *(const wbf8*)q, fm, 0, 0, 0);
                    fm = __builtin_amdgcn_mfma_f32_32x32x16_bf16(amq, *(const wbf8*)(q + 32), fm, 0, 0, 0);
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        yacc[t][mt][r] = fmaf(-dmr[r], fm[r], fmaf(dr[r], sacc[t][mt][r], yacc[t][mt][r]));
                }
            }
        }
        __syncthreads();
    };

    // An empty split range (the host rounds the stages per split up to whole super-blocks)
    // loads nothing and contributes zeros. Stage ranges are even: stage pairs are the halves
    // of one super-block.
    if (s_begin < s_end) {
        issue_part(s_begin, lds, 0);
        issue_part(s_begin, lds, 1);
        wait_vm();
        __syncthreads();
        for (int s = s_begin; s < s_end; s += 2) {
            run_stage.template operator()<0>(s);
            run_stage.template operator()<1>(s + 1);
        }
    }

    // ---- output: lane holds rows 8q + 4h + (0..3) of each tile, token column r32 ----------
    store_tile<NT * MT, W>(
        n, m, bias, y, part, counters, lds, wave, [&](int i, int r) { return yacc[i / MT][i % MT][r]; },
        [&](int i) { return m0 + (i % MT) * 32 + r32; },
        [&](int i, int r) { return n0 + (wave * NT + i / MT) * 32 + 8 * (r >> 2) + 4 * h + (r & 3); });
}

// ------------------------------------------------------------------------------------ Q6_K
// Same scheme for Q6_K (src/core/quant.cpp:630-687): the block b = 4g + i of a super-block is
// elements 128g + 32i + l; with lane half h taking l = 16h .. 16h+15, its 16 values share the
// one 16-element scale sc[8g + 2i + h]. The weight operand holds sc * (q - 32) as two exact
// fp16 parts, 16 sc_hi (q - 32) and sc_lo (q - 32) with sc = 16 sc_hi + sc_lo, so a block costs
// four MFMAs per token tile and F = sc * I (exact while the partial sums stay below 2^24, else
// within one fp32 rounding). No minimum term; d is applied once per super-block.
//
// A stage is half a super-block (g = stage parity). Q6_K super-blocks (210 bytes) sit at
// 2-byte alignment, so a row's bytes of the half come by 4-byte direct-to-LDS loads of
// dword-aligned windows around them, each inside the super-block at byte offset base of the
// matrix (sh = base & 3, 0 or 2: the weights are 16-byte aligned):
//   ql: 80 bytes from base + 64 g - sh, qh: 48 bytes from base + 128 + 32 g - sh,
//   scales: 16 bytes from base + 192 - sh (g = 0) or base + 192 + sh (g = 1).
// LDS holds them as nine 16-byte chunks per row, chunk-major ([chunk][row][16 bytes]), so
// that one wave-load fills one chunk of 16 rows (256 contiguous bytes) and the lanes' 16-byte
// reads of consecutive rows fall on distinct banks; each lane realigns its row's bytes with
// v_alignbyte. d comes by a 2-byte register load in the stage of half 0.
constexpr int kQ6Ch = 9;                  // 16-byte chunks per row and stage
constexpr int kQ6QhCh = 5, kQ6ScCh = 8;   // first chunk of the qh window, the scale chunk

template <int W, int MT>
struct Cfg6 {
    static constexpr int THREADS = 64 * W;
    static constexpr int BN = 32 * W;
    static constexpr int BM = 32 * MT;
    static constexpr int ACT = BM * 256;          // swizzled fp16 activations, as for Q4_K
    static constexpr int DX = 4 * BM * 4;
    static constexpr int WB = kQ6Ch * BN * 16;  // [chunk][row][16 bytes]
    static constexpr int OFF_DX = ACT;
    static constexpr int OFF_W = OFF_DX + DX;
    static constexpr int STAGE = OFF_W + WB;
    static constexpr int SCRATCH = W * 32 * 4;  // per wave: d[32]
    static constexpr int LDS = 2 * STAGE + SCRATCH;
    static_assert(LDS <= 160 * 1024, "LDS budget");
    static constexpr int A_LOADS = ACT / 1024;    // direct-to-LDS wave-loads
    static constexpr int A_SLOTS = (A_LOADS + W - 1) / W;
    static constexpr int DX_LOADS = DX / 256;
    static constexpr int DX_SLOTS = (DX_LOADS + W - 1) / W;
    // weight wave-loads: chunk c of 16 rows; BN / 16 = 2 W of them per chunk, so wave w's
    // slot j loads chunk j / 2 of rows 16 (w + W (j & 1)) ..
    static_assert(BN / 16 == 2 * W, "two row groups of 16 per wave and chunk");
    static constexpr int W_SLOTS = 2 * kQ6Ch;
};

template <int W, int MT>
__global__ __launch_bounds__(64 * W) void k_gemmw_q6k(const uint8_t* __restrict__ w,
                                                      uint32_t row_bytes, int k, int n, int m,
                                                      const _Float16* __restrict__ qh,
                                                      const float* __restrict__ xs,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ y, float* __restrict__ part,
                                                      int* __restrict__ counters, int split_stages) {
    using C = Cfg6<W, MT>;
    constexpr int BM = C::BM;
    extern __shared__ __align__(16) uint8_t lds[];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    const int r32 = lane & 31;

    // Workgroup -> (weight block, token block), renumbered so that the token blocks of one
    // weight block share an XCD (hardware hands consecutive workgroups to the 8 XCDs in
    // turn), whose L2 then serves the weight tile's rereads (Q6_K down, M = 512: 198 us,
    // 212 without the renumbering).
    const int mb_count = (m + BM - 1) / BM;
    const int g = gridDim.x;
    const int bid = blockIdx.x;
    const int lin = (g % 8 == 0) ? (bid % 8) * (g / 8) + bid / 8 : bid;
    const int nblk = lin / mb_count, mblk = lin - nblk * mb_count;
    const int n0 = nblk * C::BN, m0 = mblk * BM;
    const int nb = k / 32;
    const int s_begin = blockIdx.y * split_stages;
    const int s_end = min(s_begin + split_stages, k / kKS);

    // per-lane offsets for stage 0 (rows and tokens past the matrix are clamped to the last one)
    uint32_t a_off[C::A_SLOTS];   // bytes into qh: token, swizzled 16-byte chunk
#pragma unroll
    for (int j = 0; j < C::A_SLOTS; ++j) {
        const int L = min(wave + j * W, C::A_LOADS - 1);
        const int t = 4 * L + (lane >> 4);
        const int c = (lane & 15) ^ (t & 15);
        a_off[j] = ((uint32_t)min(m0 + t, m - 1) * (uint32_t)k + 8u * (uint32_t)c) * 2u;
    }
    // weight windows: this lane loads dword lane & 3 of a chunk of row 16 q + (lane >> 2);
    // rows past the matrix are clamped to the last one (their results are dropped). A tile
    // with all its rows inside the matrix takes each row's offset from rowoff0.
    const int lrow = lane >> 2;
    const uint32_t rowoff0 = (uint32_t)(n0 + lrow) * row_bytes;
    const bool full_tile = n0 + C::BN <= n;
    const int wrow = wave * 32 + r32;
    const uint32_t ro_own = (uint32_t)min(n0 + wrow, n - 1) * row_bytes;
    uint32_t dx_off[C::DX_SLOTS];  // elements into xs: [block][token] in LDS
#pragma unroll
    for (int j = 0; j < C::DX_SLOTS; ++j) {
        const int p = min(wave + j * W, C::DX_LOADS - 1) * 64 + lane;
        const int b = p / BM, tok = p - b * BM;
        dx_off[j] = (uint32_t)min(m0 + tok, m - 1) * (uint32_t)nb + b;
    }

    // every operand goes straight to LDS (direct-to-LDS loads); GH = s & 1. A stage's loads
    // go out in two parts (PART < 0: both), each before half of the stage's MFMA work, as
    // for Q4_K: part 0 the activations, dx and the first half of the weight wave-loads.
    auto issue_stage = [&]<int GH, int PART>(int s, uint8_t* st) {
        const int sb = s >> 1;
        if (PART <= 0) {
#pragma unroll
            for (int j = 0; j < C::A_SLOTS; ++j) {
                const int L = wave + j * W;
                if (C::A_LOADS % W == 0 || L < C::A_LOADS)
                    lds_load16((const uint8_t*)qh + a_off[j] + (uint32_t)s * (2u * kKS), st + L * 1024);
            }
#pragma unroll
            for (int j = 0; j < C::DX_SLOTS; ++j) {
                const int L = wave + j * W;
                if (C::DX_LOADS % W == 0 || L < C::DX_LOADS)
                    lds_load4(xs + dx_off[j] + (uint32_t)s * 4, st + C::OFF_DX + L * 256);
            }
        }
        const uint32_t sbo = (uint32_t)sb * Q6_K_BYTES;
        // a full tile: rows 16 q + lrow at rowoff0 + 16 q row_bytes, all with the shift of
        // the lane's own row (16 q row_bytes is a multiple of 4)
        const uint32_t sh0 = (rowoff0 + sbo) & 3u;
        const uint32_t lb = rowoff0 + sbo + 4u * (uint32_t)(lane & 3) - sh0;  // ql, qh, scales of half 0
        const uint32_t lbs = lb + 2u * sh0;                                   // scales of half 1
#pragma unroll
        for (int j = 0; j < C::W_SLOTS; ++j) {
            if (PART == 0 && j >= C::W_SLOTS / 2) continue;
            if (PART == 1 && j < C::W_SLOTS / 2) continue;
            const int c = j >> 1;
            const int q = wave + W * (j & 1);
            const uint32_t win = c < kQ6QhCh ? 64u * GH + 16u * c
                               : c < kQ6ScCh ? 128u + 32u * GH + 16u * (c - kQ6QhCh) : 192u;
            uint32_t src;
            if (full_tile) {
                src = (c == kQ6ScCh && GH == 1 ? lbs : lb) + (uint32_t)(16 * q) * row_bytes + win;
            } else {
                const uint32_t base = (uint32_t)min(n0 + 16 * q + lrow, n - 1) * row_bytes + sbo;
                const uint32_t sh = base & 3u;
                src = base + 4u * (uint32_t)(lane & 3) + win +
                      ((c == kQ6ScCh && GH == 1) ? sh : 0u - sh);
            }
            lds_load4(w + src, st + C::OFF_W + (c * C::BN + 16 * q) * 16);
        }
    };

    wf16 sacc[MT], yacc[MT];
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[a][r] = yacc[a][r] = 0.0f;

    float* scratch = (float*)(lds + 2 * C::STAGE) + wave * 32;
    uint32_t dbits = 0;  // d of the wave row's super-block, loaded in the stage of its half 0

    // One stage: half GH of a super-block (stage ranges are even and super-block aligned, so
    // stage s sits in LDS buffer GH and the first block of GH = 0 starts the scaled sums).
    auto run_stage = [&]<int GH>(int s) {
        uint8_t* cur = lds + GH * C::STAGE;
        uint8_t* nxt = lds + (1 - GH) * C::STAGE;
        // chunk c of the lane's weight row: wr + c * BN * 16
        const uint8_t* wr = cur + C::OFF_W + wrow * 16;
        const uint32_t own = ro_own + (uint32_t)(s >> 1) * Q6_K_BYTES;
        const uint32_t sh = own & 3u;  // the windows' lead before the row's bytes
        // 16 bytes at byte sh of the window from chunk c: the chunk, the next one's first
        // dword, realigned
        auto window16 = [&](int c) {
            const wu4 a = *(const wu4*)(wr + c * (C::BN * 16));
            const uint32_t e = *(const uint32_t*)(wr + (c + 1) * (C::BN * 16));
            return wu4{__builtin_amdgcn_alignbyte(a.y, a.x, sh), __builtin_amdgcn_alignbyte(a.z, a.y, sh),
                       __builtin_amdgcn_alignbyte(a.w, a.z, sh), __builtin_amdgcn_alignbyte(e, a.w, sh)};
        };
        // d for the lane's output rows goes to the wave's scratch; half 0 loads the next one
        if (GH == 1 && h == 0) scratch[r32] = f16_to_f32(dbits);
        if (GH == 0) dbits = *(const uint16_t*)(w + own + Q6_K_D);
        const bool more = s + 1 < s_end;
        if (more) issue_stage.template operator()<1 - GH, 0>(s + 1, nxt);

        const wu4 qhb = window16(kQ6QhCh + h);
        // the half's 8 scales: at byte sh (half 0) or 8 - sh (half 1) of the scale chunk
        uint32_t scx, scy;
        {
            const wu4 c = *(const wu4*)(wr + kQ6ScCh * (C::BN * 16));
            if (GH == 0) {
                scx = __builtin_amdgcn_alignbyte(c.y, c.x, sh);
                scy = __builtin_amdgcn_alignbyte(c.z, c.y, sh);
            } else {
                scx = sh ? __builtin_amdgcn_alignbyte(c.z, c.y, 2u) : c.z;
                scy = sh ? __builtin_amdgcn_alignbyte(c.w, c.z, 2u) : c.w;
            }
        }
        const uint8_t* act = cur;
        const float* dxl = (const float*)(cur + C::OFF_DX);

        auto block = [&]<bool FRESH>(int i) {
            const wu4 ql = window16(2 * (i & 1) + h);
            const uint32_t lsh = i >= 2 ? 4u : 0u;
            // bits 2i, 2i+1 of every qh byte to bits 4, 5 of the same byte: a rotation right by
            // 2i - 4 (mod 32); the bits it carries across bytes are masked off
            const uint32_t rot = (uint32_t)(2 * i - 4) & 31u;
            const uint32_t qhv[4] = {qhb.x, qhb.y, qhb.z, qhb.w}, qlv[4] = {ql.x, ql.y, ql.z, ql.w};
            uint32_t q6[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
                q6[e] = ((qlv[e] >> lsh) & 0x0F0F0F0Fu) |
                        (__builtin_amdgcn_alignbit(qhv[e], qhv[e], rot) & 0x30303030u);
            // scale of this lane's 16 values: sc[8 g + 2 i + h], local index 2 i + h
            const int si = 2 * i + h;
            const uint32_t scw = si < 4 ? scx : scy;
            const int sc = (int)(int8_t)((scw >> (8 * (si & 3))) & 0xFFu);
            const int s_hi = sc >> 4, s_lo = sc & 15;
            const wh2 off = {(_Float16)-1056.0f, (_Float16)-1056.0f};
            const wh2 m1 = {(_Float16)(16 * s_hi), (_Float16)(16 * s_hi)};
            const wh2 m2 = {(_Float16)s_lo, (_Float16)s_lo};
            wh8 a1[2], a2[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const wh2 v0 = magic_pair(q6[2 * j], 0) + off, v1 = magic_pair(q6[2 * j], 1) + off;
                const wh2 v2 = magic_pair(q6[2 * j + 1], 0) + off, v3 = magic_pair(q6[2 * j + 1], 1) + off;
                const wh2 p0 = v0 * m1, p1 = v1 * m1, p2 = v2 * m1, p3 = v3 * m1;
                const wh2 q0 = v0 * m2, q1 = v1 * m2, q2 = v2 * m2, q3 = v3 * m2;
                a1[j] = wh8{p0.x, p0.y, p1.x, p1.y, p2.x, p2.y, p3.x, p3.y};
                a2[j] = wh8{q0.x, q0.y, q1.x, q1.y, q2.x, q2.y, q3.x, q3.y};
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int tok = mt * 32 + r32;
                const uint8_t* arow = act + tok * 256;
                const int sw = tok & 15;
                const wh8 b0 = *(const wh8*)(arow + (((4 * i + 2 * h) ^ sw) << 4));
                const wh8 b1 = *(const wh8*)(arow + (((4 * i + 2 * h + 1) ^ sw) << 4));
                const float dxv = dxl[i * BM + tok];
                wf16 f = {};
                f = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1[0], b0, f, 0, 0, 0);
                f = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1[1], b1, f, 0, 0, 0);
                f = __builtin_amdgcn_mfma_f32_32x32x16_f16(a2[0], b0, f, 0, 0, 0);
                f = __builtin_amdgcn_mfma_f32_32x32x16_f16(a2[1], b1, f, 0, 0, 0);
                if constexpr (FRESH) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) sacc[mt][r] = dxv * f[r];
                } else {
#pragma unroll
                    for (int r = 0; r < 16; ++r) sacc[mt][r] = fmaf(dxv, f[r], sacc[mt][r]);
                }
            }
        };
        if constexpr (GH == 0)
            block.template operator()<true>(0);
        else
            block.template operator()<false>(0);
        block.template operator()<false>(1);
        if (more) issue_stage.template operator()<1 - GH, 1>(s + 1, nxt);
#pragma unroll 1
        for (int i = 2; i < 4; ++i) block.template operator()<false>(i);
        if (more) wait_vm();
        if constexpr (GH == 1) {
            float dr[16];
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const float4 dv = *(const float4*)(scratch + 8 * q4 + 4 * h);
                dr[4 * q4] = dv.x; dr[4 * q4 + 1] = dv.y; dr[4 * q4 + 2] = dv.z; dr[4 * q4 + 3] = dv.w;
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) yacc[mt][r] = fmaf(dr[r], sacc[mt][r], yacc[mt][r]);
        }
        __syncthreads();
    };

    // An empty split range (stages per split are rounded up to whole super-blocks) loads
    // nothing and contributes zeros.
    if (s_begin < s_end) {
        issue_stage.template operator()<0, -1>(s_begin, lds);
        wait_vm();
        __syncthreads();
        for (int s = s_begin; s < s_end; s += 2) {
            run_stage.template operator()<0>(s);
            run_stage.template operator()<1>(s + 1);
        }
    }

    store_tile<MT, W>(
        n, m, bias, y, part, counters, lds, wave, [&](int i, int r) { return yacc[i][r]; },
        [&](int i) { return m0 + i * 32 + r32; },
        [&](int i, int r) { return n0 + wave * 32 + 8 * (r >> 2) + 4 * h + (r & 3); });
}

// ------------------------------------------------------------------ Q8_0 / Q4_0 / Q5_0
// 32-element blocks with one fp16 scale d each (quant.cpp: Q8_0 and Q4_0 vec_dot 706-724,
// Q5_0 its analogue). The weight operand holds the block's integers (q, q - 8 or q - 16, exact
// in fp16), so a block's MFMA pair returns the reference's integer dot I exactly and
//   y += dx * (d * I)
// costs two VALU operations per output and block (d belongs to the weight row, dx to the
// token). A stage is 4 blocks (128 elements); the rows' stage bytes (4 blocks of 34 / 18 / 22
// bytes, 4-byte aligned because k % 256 == 0) arrive by 4-byte direct-to-LDS loads in the
// blocks' own layout, and each lane realigns its 2-byte-aligned fields from 4-byte LDS reads.
template <uint32_t T>
constexpr int b32_bytes() { return T == T_Q8_0 ? Q8_0_BYTES : T == T_Q4_0 ? Q4_0_BYTES : Q5_0_BYTES; }

template <uint32_t T, int W, int MT>
struct CfgB {
    static constexpr int THREADS = 64 * W;
    static constexpr int BN = 32 * W;
    static constexpr int BM = 32 * MT;
    static constexpr int SROW = 4 * b32_bytes<T>();   // bytes per weight row per stage
    static constexpr int SDW = SROW / 4;
    static constexpr int ACT = BM * 256;                // swizzled fp16, as for the K-quants
    static constexpr int DX = BM * 16 < 1024 ? 1024 : BM * 16;
    static constexpr int WB = (BN * SROW + 255) / 256 * 256 + 64;  // + slack for the last lane's 5th dword
    static constexpr int OFF_DX = ACT;
    static constexpr int OFF_W = OFF_DX + DX;
    static constexpr int STAGE = OFF_W + WB;
    static constexpr int SCRATCH = W * 4 * 32 * 4;      // per wave: d[4 blocks][32 rows]
    static constexpr int LDS = 2 * STAGE + SCRATCH;
    static_assert(LDS <= 160 * 1024, "LDS budget");
    static constexpr int A_LOADS = ACT / 1024;
    static constexpr int A_SLOTS = (A_LOADS + W - 1) / W;
    static constexpr int DX_LOADS = DX / 1024;
    static constexpr int DX_SLOTS = (DX_LOADS + W - 1) / W;
    static constexpr int W_DW = BN * SDW;               // weight dwords per stage
    static constexpr int W_LOADS = (W_DW + 63) / 64;    // 4-byte wave-loads
    static constexpr int W_SLOTS = (W_LOADS + W - 1) / W;
};

// Bytes [o, o + 4 N) of an LDS row whose base is 4-byte aligned, o even: N + 1 aligned dword
// reads and a funnel shift.
template <int N>
__device__ __forceinline__ void lds_unaligned(const uint8_t* row, int o, uint32_t (&out)[N]) {
    const uint32_t* p = (const uint32_t*)(row + (o & ~3));
    const uint32_t sh = (uint32_t)(o & 3);
    uint32_t v[N + 1];
#pragma unroll
    for (int i = 0; i <= N; ++i) v[i] = p[i];
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], sh);
}

// Four bits b0..b3 of x (at bit positions 0..3) moved to bit 4 of bytes 0..3.
__device__ __forceinline__ uint32_t bits_to_byte_bit4(uint32_t x) {
    x &= 0xFu;
    return ((x | (x << 7) | (x << 14) | (x << 21)) & 0x01010101u) << 4;
}

template <uint32_t T, int W, int MT>
__global__ __launch_bounds__(64 * W) void k_gemmw_b32(const uint8_t* __restrict__ w,
                                                      uint32_t row_bytes, int k, int n, int m,
                                                      const _Float16* __restrict__ qh,
                                                      const float* __restrict__ xs,
                                                      const float* __restrict__ bias,
                                                      float* __restrict__ y, float* __restrict__ part,
                                                      int* __restrict__ counters, int split_stages) {
    using C = CfgB<T, W, MT>;
    constexpr int BM = C::BM;
    constexpr int BS = b32_bytes<T>();
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane >> 5;
    const int r32 = lane & 31;

    // Workgroup -> (weight block, token block), renumbered so that the token blocks of one
    // weight block share an XCD (hardware hands consecutive workgroups to the 8 XCDs in
    // turn), whose L2 then serves the weight tile's rereads (Q6_K down, M = 512: 198 us,
    // 212 without the renumbering).
    const int mb_count = (m + BM - 1) / BM;
    const int g = gridDim.x;
    const int bid = blockIdx.x;
    const int lin = (g % 8 == 0) ? (bid % 8) * (g / 8) + bid / 8 : bid;
    const int nblk = lin / mb_count, mblk = lin - nblk * mb_count;
    const int n0 = nblk * C::BN, m0 = mblk * BM;
    const int nb = k / 32;
    const int s_begin = blockIdx.y * split_stages;
    const int s_end = min(s_begin + split_stages, k / kKS);

    // per-lane source offsets (stage 0); rows and tokens past the matrix are clamped
    uint32_t a_off[C::A_SLOTS];
#pragma unroll
    for (int j = 0; j < C::A_SLOTS; ++j) {
        const int L = min(wave + j * W, C::A_LOADS - 1);
        const int t = 4 * L + (lane >> 4);
        const int c = (lane & 15) ^ (t & 15);
        a_off[j] = ((uint32_t)min(m0 + t, m - 1) * (uint32_t)k + 8u * (uint32_t)c) * 2u;
    }
    uint32_t dx_off[C::DX_SLOTS];
#pragma unroll
    for (int j = 0; j < C::DX_SLOTS; ++j) {
        const int t = min(wave + j * W, C::DX_LOADS - 1) * 64 + lane;
        dx_off[j] = (uint32_t)min(m0 + t, m - 1) * (uint32_t)nb;
    }
    uint32_t w_off[C::W_SLOTS];   // flat dword f of [row][SDW]: row f / SDW, dword f % SDW
#pragma unroll
    for (int j = 0; j < C::W_SLOTS; ++j) {
        const int f = min(min(wave + j * W, C::W_LOADS - 1) * 64 + lane, C::W_DW - 1);
        const int row = f / C::SDW, dw = f - row * C::SDW;
        w_off[j] = (uint32_t)min(n0 + row, n - 1) * row_bytes + 4u * (uint32_t)dw;
    }

    auto issue_stage = [&](int s, uint8_t* st) {
#pragma unroll
        for (int j = 0; j < C::A_SLOTS; ++j) {
            const int L = wave + j * W;
            if (C::A_LOADS % W == 0 || L < C::A_LOADS)
                lds_load16((const uint8_t*)qh + a_off[j] + (uint32_t)s * (2u * kKS), st + L * 1024);
        }
#pragma unroll
        for (int j = 0; j < C::DX_SLOTS; ++j) {
            const int L = wave + j * W;
            if (C::DX_LOADS % W == 0 || L < C::DX_LOADS)
                lds_load16(xs + dx_off[j] + (uint32_t)s * 4, st + C::OFF_DX + L * 1024);
        }
#pragma unroll
        for (int j = 0; j < C::W_SLOTS; ++j) {
            const int L = wave + j * W;
            if (C::W_LOADS % W == 0 || L < C::W_LOADS)
                lds_load4(w + w_off[j] + (uint32_t)s * (uint32_t)C::SROW, st + C::OFF_W + L * 256);
        }
    };

    wf16 yacc[MT];
#pragma unroll
    for (int a = 0; a < MT; ++a)
#pragma unroll
        for (int r = 0; r < 16; ++r) yacc[a][r] = 0.0f;

    float* scratch = (float*)(lds + 2 * C::STAGE) + wave * 128;
    const int wrow = wave * 32 + r32;

    auto run_stage = [&](int s) {
        const int buf = (s - s_begin) & 1;
        uint8_t* cur = lds + buf * C::STAGE;
        uint8_t* nxt = lds + (1 - buf) * C::STAGE;
        const uint8_t* wr = cur + C::OFF_W + wrow * C::SROW;

        // d of blocks 2h and 2h + 1 of this lane's row -> scratch, then each lane's 16 output
        // rows' d for all 4 blocks into registers, before the next stage's direct-to-LDS loads
        // are issued (LDS accesses while they fly would make the compiler wait for them)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int b = 2 * h + e;
            const uint32_t dw = *(const uint32_t*)(wr + ((b * BS) & ~3));
            scratch[b * 32 + r32] = f16_to_f32(((b * BS) & 2) ? (dw >> 16) : (dw & 0xFFFFu));
        }
        float dr[4][16];
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const float4 dv = *(const float4*)(scratch + b * 32 + 8 * q4 + 4 * h);
                dr[b][4 * q4] = dv.x; dr[b][4 * q4 + 1] = dv.y; dr[b][4 * q4 + 2] = dv.z; dr[b][4 * q4 + 3] = dv.w;
            }
        const bool more = s + 1 < s_end;
        if (more) issue_stage(s + 1, nxt);

        const uint8_t* act = cur;
        const float* dxl = (const float*)(cur + C::OFF_DX);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            // A fragments: elements 16h + 8j + e of block b (K steps j = 0, 1)
            wh8 afr[2];
            if constexpr (T == T_Q8_0) {
                uint32_t u[4];
                lds_unaligned<4>(wr, b * BS + 2 + 16 * h, u);
                afr[0] = __builtin_bit_cast(wh8, int8x8_to_h8(u[0], u[1]));
                afr[1] = __builtin_bit_cast(wh8, int8x8_to_h8(u[2], u[3]));
            } else {
                uint32_t u[4], hb = 0;
                if constexpr (T == T_Q4_0) {
                    lds_unaligned<4>(wr, b * BS + 2, u);
                } else {
                    uint32_t v[5];
                    lds_unaligned<5>(wr, b * BS + 2, v);
                    hb = v[0] >> (16 * h);
                    u[0] = v[1]; u[1] = v[2]; u[2] = v[3]; u[3] = v[4];
                }
                // byte j: low nibble = element j, high nibble = element 16 + j
                uint32_t q[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    q[e] = h ? ((u[e] >> 4) & 0x0F0F0F0Fu) : (u[e] & 0x0F0F0F0Fu);
                    if constexpr (T == T_Q5_0) q[e] |= bits_to_byte_bit4(hb >> (4 * e));
                }
                const _Float16 off = (_Float16)(T == T_Q4_0 ? -1032.0f : -1040.0f);
                const wh2 one = {(_Float16)1.0f, (_Float16)1.0f}, c = {off, off};
                afr[0] = scaled8(q[0], q[1], one, c);
                afr[1] = scaled8(q[2], q[3], one, c);
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int tok = mt * 32 + r32;
                const uint8_t* arow = act + tok * 256;
                const int sw = tok & 15;
                const wh8 b0 = *(const wh8*)(arow + (((4 * b + 2 * h) ^ sw) << 4));
                const wh8 b1 = *(const wh8*)(arow + (((4 * b + 2 * h + 1) ^ sw) << 4));
                const float dxv = dxl[tok * 4 + b];
                wf16 f = {};
                f = __builtin_amdgcn_mfma_f32_32x32x16_f16(afr[0], b0, f, 0, 0, 0);
                f = __builtin_amdgcn_mfma_f32_32x32x16_f16(afr[1], b1, f, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 16; ++r) yacc[mt][r] = fmaf(dxv, dr[b][r] * f[r], yacc[mt][r]);
            }
        }
        if (more) wait_vm();
        __syncthreads();
    };

    if (s_begin < s_end) {
        issue_stage(s_begin, lds);
        wait_vm();
        __syncthreads();
        for (int s = s_begin; s < s_end; ++s) run_stage(s);
    }

    store_tile<MT, W>(
        n, m, bias, y, part, counters, lds, wave, [&](int i, int r) { return yacc[i][r]; },
        [&](int i) { return m0 + i * 32 + r32; },
        [&](int i, int r) { return n0 + wave * 32 + 8 * (r >> 2) + 4 * h + (r & 3); });
}

bool gemmw_supported(uint32_t type) {
    return type == T_Q4_K || type == T_Q5_K || type == T_Q6_K || type == T_Q8_0 || type == T_Q4_0 ||
           type == T_Q5_0;
}

// The kernels index the weights and the fp16 activations with 32-bit byte offsets.
bool gemmw_fits(uint32_t type, int k, int n, int m) {
    const uint64_t wbytes = (uint64_t)n * (uint64_t)(k / block_elems(type)) * (uint64_t)block_bytes(type);
    return wbytes < (1ull << 32) && 2ull * (uint64_t)m * (uint64_t)k < (1ull << 32);
}

bool is_b32(uint32_t type) { return type == T_Q8_0 || type == T_Q4_0 || type == T_Q5_0; }

namespace {

int device_cus() {
    static int cached = 0;
    if (cached == 0) {
        int dev = 0, c = 0;
        cached = (hipGetDevice(&dev) == hipSuccess &&
                  hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && c > 0)
                     ? c
                     : 256;
    }
    return cached;
}

// Split-K factor: workgroups up to `target`, at least min_stages stages per split.
int choose_splits(int tiles, int stages, int target, int min_stages = 8) {
    int sp = 1;
    while (sp < 8 && tiles * sp * 2 <= target && stages / (sp * 2) >= min_stages) sp *= 2;
    return sp;
}

struct Plan {
    int wv, nt, mt, splits;
};

Plan plan_for(uint32_t type, int k, int n, int m) {
    Plan p{};
    // the tuning overrides (cllm_hip_tune "gemm_tiles" / "gemm_splits"): any compiled tile
    // shape of the K-quant kernels, and the split-K factor
    const Tuning& tu = tuning();
    const int wv = tu.gemm_waves.load(std::memory_order_relaxed);
    const int nt = tu.gemm_wtiles.load(std::memory_order_relaxed);
    const int mt = tu.gemm_ttiles.load(std::memory_order_relaxed);
    const int cus = device_cus();
    int target = 2 * cus;  // workgroups to aim for
    int min_stages = 8;    // stages per split at least
    if (is_b32(type)) {
        // 32-element block types: 128 x 32 tiles up to 32 rows, else 128 x 64 (the per-block
        // d of the 16 output rows a lane holds stays in registers, which larger token tiles
        // would spill); split K to about two workgroups per CU
        p.wv = 4, p.nt = 1, p.mt = m <= 32 ? 1 : 2;
    } else if (type == T_Q6_K) {
        // 128 weight rows x 64 tokens (4 waves, two workgroups per CU), x 32 tokens up to 32
        // rows; the tuning override takes the other compiled shapes (256 x 64 on 8 waves,
        // 128 x 128)
        p.wv = 4, p.nt = 1, p.mt = m <= 32 ? 1 : 2;
        if ((wv == 8 && nt == 1 && mt == 2) || (wv == 4 && nt == 1 && (mt == 1 || mt == 2 || mt == 4)))
            p.wv = wv, p.mt = mt;
    } else if (wv != 0 && (type == T_Q4_K ||
                           (wv == 8 && nt == 1 && (mt == 4 || mt == 2)) ||
                           (wv == 4 && nt == 1 && (mt == 2 || mt == 1)))) {
        // Q5_K has the four shapes of the default plan compiled
        p.wv = wv, p.nt = nt, p.mt = mt;
    } else {
        // From sweeps on MI355X over n = 14336 / 4096 / 1024 and m = 64 .. 512 (k = 4096):
        // - 256 x 128 tiles (8 waves, one workgroup per CU) when they fill the CUs: 14336 x
        //   4096 at m = 512 runs its 224 tiles unsplit in 129 us (152 for the best 128 x 64);
        // - else 128 x 64 tiles (4 waves, two workgroups per CU) above 32 rows when there are
        //   at least 3/8 as many as CUs, split to about two workgroups per CU (4096 at m = 512:
        //   50 us against 53 for 256 x 64; 14336 at m = 64: 33 against 39 for 128 x 32);
        // - else 128 x 32 tiles split to about two workgroups per CU, down to 4 stages per
        //   split (4096 at m = 64: 21 us for 8 splits against 22 for 4; 1024 at m = 128: 20
        //   against 22).
        // - long K (at least 24 stages per split): 256 x 128 tiles on 2 or 4 splits when that
        //   fills 3/4 of the CUs. Q4_K 4096 x 14336 at m = 384 / 512 / 768 / 1024: 122 / 128 /
        //   210 / 224 us against 134 / 137 / 249 / 256 on 128 x 64 tiles (Q5_K and K = 11008
        //   alike; 3 splits were slower than 2 and 4 throughout, and K = 4096 has too few
        //   stages: wq 4096 x 4096 at m = 512 took 58.5 us on 4 splits against 48.3).
        const int t84 = ((n + 255) / 256) * ((m + 127) / 128);
        const int t42 = ((n + 127) / 128) * ((m + 63) / 64);
        constexpr int kLongKStages = 24;
        const int s84 = choose_splits(t84, k / kKS, cus, kLongKStages);
        if (t84 >= cus * 3 / 4) {
            p.wv = 8, p.nt = 1, p.mt = 4;
            target = cus;
        } else if (s84 >= 2 && t84 * s84 >= cus * 3 / 4) {
            p.wv = 8, p.nt = 1, p.mt = 4;
            target = cus;
            min_stages = kLongKStages;
        } else if (m > 32 && t42 >= cus * 3 / 8) {
            p.wv = 4, p.nt = 1, p.mt = 2;
        } else {
            p.wv = 4, p.nt = 1, p.mt = 1;
            min_stages = 4;
        }
    }
    const int bn = 32 * p.nt * p.wv, bm = 32 * p.mt;
    const int tiles = ((n + bn - 1) / bn) * ((m + bm - 1) / bm);
    p.splits = choose_splits(tiles, k / kKS, target, min_stages);
    // Above 256 rows on 128 x 64 tiles, while the tiles make fewer than two rounds of the
    // CUs' resident workgroups (1 per CU for the 32-element block types' tile at 306 VGPRs, 2
    // for the K-quants'): the split count (1, 2 or 4) whose workgroups run in the fewest
    // stage-rounds,
    // ceil(workgroups / slots) x ceil(stages / splits); on a tie, more splits only while the CUs
    // are not yet filled. Measured at m = 384 .. 1024: on 4096 x 14336 and 4096 x 4096 this
    // picks the fastest of 1 / 2 / 4 splits (within 1 %), e.g. Q8_0 4096 x 14336 at m = 384 /
    // 768 took 175 / 329 us against 218 / 425 for the at-most-two-per-CU rule above, Q6_K
    // 4096 x 14336 147 / 275 against 169 / 334. With more tiles the extra splits cost more
    // than the rounds save (Q8_0 14336 x 4096 at m = 768: 405 us on 4 splits, 386 unsplit).
    // Q4_K alike: 4096 x 4096 at m = 768 73 us on 4 splits against 81 unsplit, 11008 x 4096
    // at m = 384 109 against 130.
    const int slots = cus * (is_b32(type) ? 1 : 2);
    if (m > 256 && p.wv == 4 && p.nt == 1 && p.mt == 2 && tiles < 2 * slots) {
        const int stages = k / kKS;
        int best = 1;
        long best_cost = -1;
        for (int s = 1; s <= 4 && stages / s >= min_stages; s *= 2) {
            const long wgs = (long)tiles * s;
            const long cost = (wgs + slots - 1) / slots * ((stages + s - 1) / s);
            if (best_cost < 0 || cost < best_cost || (cost == best_cost && (long)tiles * best < slots)) {
                best = s;
                best_cost = cost;
            }
        }
        p.splits = best;
    }
    const int sp = tu.gemm_splits.load(std::memory_order_relaxed);
    if (sp >= 1 && sp <= 16 && sp <= k / kKS) p.splits = sp;
    return p;
}

template <int W, int NT, int MT, bool Q5>
hipError_t launch_q4(Segs segs, int k, int m, const _Float16* qh, const float* xs,
                     const uint16_t* xq, float* part, int* counters, int splits,
                     hipStream_t stream) {
    using C = Cfg<W, NT, MT, Q5>;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)k_gemmw_q4k<W, NT, MT, Q5>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const uint32_t row_bytes = (uint32_t)(k / 256) * (Q5 ? Q5_K_BYTES : Q4_K_BYTES);
    const int mb = (m + C::BM - 1) / C::BM;
    int tiles = 0;
    for (int i = 0; i < segs.count; ++i) {
        tiles += ((segs.n[i] + C::BN - 1) / C::BN) * mb;
        segs.tile_end[i] = tiles;
    }
    const int stages = k / kKS, per = 2 * ((stages / 2 + splits - 1) / splits);
    hipLaunchKernelGGL((k_gemmw_q4k<W, NT, MT, Q5>), dim3((unsigned)tiles, (unsigned)splits),
                       dim3(C::THREADS), C::LDS, stream, segs, row_bytes, k, m, qh, xs, xq, part,
                       counters, per);
    return hipGetLastError();
}

template <int W, int MT>
hipError_t launch_q6(const uint8_t* w, int k, int n, int m, const _Float16* qh, const float* xs,
                     const float* bias, float* y, float* part, int* counters, int splits,
                     hipStream_t stream) {
    using C = Cfg6<W, MT>;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)k_gemmw_q6k<W, MT>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const uint32_t row_bytes = (uint32_t)(k / 256) * Q6_K_BYTES;
    const int tiles = ((n + C::BN - 1) / C::BN) * ((m + C::BM - 1) / C::BM);
    const int stages = k / kKS, per = 2 * ((stages / 2 + splits - 1) / splits);
    hipLaunchKernelGGL((k_gemmw_q6k<W, MT>), dim3((unsigned)tiles, (unsigned)splits),
                       dim3(C::THREADS), C::LDS, stream, w, row_bytes, k, n, m, qh, xs, bias, y,
                       part, counters, per);
    return hipGetLastError();
}

template <uint32_t T, int W, int MT>
hipError_t launch_b32(const uint8_t* w, int k, int n, int m, const _Float16* qh, const float* xs,
                      const float* bias, float* y, float* part, int* counters, int splits,
                      hipStream_t stream) {
    using C = CfgB<T, W, MT>;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)k_gemmw_b32<T, W, MT>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, C::LDS);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const uint32_t row_bytes = (uint32_t)(k / 32) * (uint32_t)b32_bytes<T>();
    const int tiles = ((n + C::BN - 1) / C::BN) * ((m + C::BM - 1) / C::BM);
    const int stages = k / kKS, per = 2 * ((stages / 2 + splits - 1) / splits);
    hipLaunchKernelGGL((k_gemmw_b32<T, W, MT>), dim3((unsigned)tiles, (unsigned)splits),
                       dim3(C::THREADS), C::LDS, stream, w, row_bytes, k, n, m, qh, xs, bias, y, part,
                       counters, per);
    return hipGetLastError();
}

}  // namespace

// Split-K workspace: one arrival counter per tile at its start (a fixed block of ints that must
// be zero before the first launch; each launch leaves it zero, and no launch writes anything
// else there whatever its shape), then the partial sums: per split, one whole tile of fp32 per
// workgroup (rows and tokens past the matrix included).
int64_t plan_tiles(const Plan& p, int n, int m) {
    return (int64_t)((n + 32 * p.nt * p.wv - 1) / (32 * p.nt * p.wv)) *
           ((m + 32 * p.mt - 1) / (32 * p.mt));
}
size_t slices_bytes(const Plan& p, int n, int m) {
    const size_t tile = (size_t)(32 * p.nt * p.wv) * (size_t)(32 * p.mt) * sizeof(float);
    return (size_t)p.splits * (size_t)plan_tiles(p, n, m) * tile;
}
constexpr size_t kCounterBytes = 64 * 1024;  // 16384 tiles

size_t gemmw_counter_bytes() { return kCounterBytes; }

size_t gemmw_partial_bytes(uint32_t type, int k, int n, int m) {
    if (!gemmw_supported(type) || k % 256 != 0) return 0;
    const Plan p = plan_for(type, k, n, m);
    return p.splits > 1 ? slices_bytes(p, n, m) + kCounterBytes : 0;
}

__global__ void k_zero_words(uint32_t* __restrict__ p, size_t words) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < words) p[i] = 0;
}

hipError_t gemmw_workspace_init(void* part, size_t bytes, hipStream_t stream) {
    const size_t words = bytes / 4;
    if (words == 0) return hipSuccess;
    hipLaunchKernelGGL(k_zero_words, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, stream,
                       (uint32_t*)part, words);
    return hipGetLastError();
}

namespace {

// Tiles of a launch over the segments: whole tiles per segment.
int64_t segs_tiles(const Plan& p, const Segs& sg, int m) {
    const int bn = 32 * p.nt * p.wv;
    int64_t t = 0;
    for (int i = 0; i < sg.count; ++i) t += (sg.n[i] + bn - 1) / bn;
    return t * ((m + 32 * p.mt - 1) / (32 * p.mt));
}

int segs_rows(const Segs& sg) {
    int n = 0;
    for (int i = 0; i < sg.count; ++i) n += sg.n[i];
    return n;
}

// One launch of the weight-row kernel over the segments (several only for Q4_K / Q5_K), on
// the plan of their rows together.
hipError_t gemmw_dispatch(uint32_t type, const Segs& sg, int k, int m, const float* xs,
                          const _Float16* qh, const uint16_t* xq, float* part, size_t part_bytes,
                          hipStream_t stream) {
    if (!gemmw_supported(type) || k % 256 != 0 || sg.count < 1 || sg.count > kMaxSegs)
        return hipErrorNotSupported;
    if (sg.count > 1 && type != T_Q4_K && type != T_Q5_K) return hipErrorNotSupported;
    for (int i = 0; i < sg.count; ++i)
        if (!gemmw_fits(type, k, sg.n[i], m)) return hipErrorNotSupported;
    Plan p = plan_for(type, k, segs_rows(sg), m);
    const int64_t tiles = segs_tiles(p, sg, m);
    const size_t tile_bytes = (size_t)(32 * p.nt * p.wv) * (size_t)(32 * p.mt) * sizeof(float);
    if (p.splits > 1 && (part == nullptr ||
                         part_bytes < (size_t)p.splits * (size_t)tiles * tile_bytes + kCounterBytes ||
                         tiles * 4 > (int64_t)kCounterBytes))
        p.splits = 1;
    int* counters = p.splits > 1 ? (int*)part : nullptr;
    part = p.splits > 1 ? (float*)((char*)part + kCounterBytes) : nullptr;
    const uint8_t* w = sg.w[0];
    const int n = sg.n[0];
    const float* bias = sg.bias[0];
    float* y = sg.y[0];
    hipError_t e = hipErrorNotSupported;
    if (type == T_Q6_K) {
        if (p.wv == 8)
            e = launch_q6<8, 2>(w, k, n, m, qh, xs, bias, y, part, counters, p.splits, stream);
        else if (p.mt == 4)
            e = launch_q6<4, 4>(w, k, n, m, qh, xs, bias, y, part, counters, p.splits, stream);
        else if (p.mt == 1)
            e = launch_q6<4, 1>(w, k, n, m, qh, xs, bias, y, part, counters, p.splits, stream);
        else
            e = launch_q6<4, 2>(w, k, n, m, qh, xs, bias, y, part, counters, p.splits, stream);
    } else if (is_b32(type)) {
#define CLLM_GEMMW_B32(TT)                                                                    \
        if (type == TT) {                                                                      \
            if (p.mt == 2)                                                                     \
                e = launch_b32<TT, 4, 2>(w, k, n, m, qh, xs, bias, y, part, counters, p.splits, stream); \
            else                                                                               \
                e = launch_b32<TT, 4, 1>(w, k, n, m, qh, xs, bias, y, part, counters, p.splits, stream); \
        }
        CLLM_GEMMW_B32(T_Q8_0)
        CLLM_GEMMW_B32(T_Q4_0)
        CLLM_GEMMW_B32(T_Q5_0)
#undef CLLM_GEMMW_B32
    } else if (type == T_Q5_K) {
        // the four shapes of the default plan (the only ones the tuning override takes)
        if (p.wv == 8 && p.nt == 1 && p.mt == 4)
            e = launch_q4<8, 1, 4, true>(sg, k, m, qh, xs, xq, part, counters, p.splits, stream);
        else if (p.wv == 8 && p.nt == 1 && p.mt == 2)
            e = launch_q4<8, 1, 2, true>(sg, k, m, qh, xs, xq, part, counters, p.splits, stream);
        else if (p.wv == 4 && p.nt == 1 && p.mt == 2)
            e = launch_q4<4, 1, 2, true>(sg, k, m, qh, xs, xq, part, counters, p.splits, stream);
        else
            e = launch_q4<4, 1, 1, true>(sg, k, m, qh, xs, xq, part, counters, p.splits, stream);
    } else {
#define CLLM_GEMMW_CASE(A, B, D)                                                              \
        if (p.wv == A && p.nt == B && p.mt == D)                                               \
            e = launch_q4<A, B, D, false>(sg, k, m, qh, xs, xq, part, counters, p.splits, stream);
        CLLM_GEMMW_CASE(8, 1, 4)
        CLLM_GEMMW_CASE(8, 1, 2)
        CLLM_GEMMW_CASE(8, 2, 2)
        CLLM_GEMMW_CASE(4, 2, 4)
        CLLM_GEMMW_CASE(4, 2, 2)
        CLLM_GEMMW_CASE(4, 1, 2)
        CLLM_GEMMW_CASE(4, 1, 1)
#undef CLLM_GEMMW_CASE
    }
    return e;
}

Segs one_seg(const uint8_t* w, int n, const float* bias, float* y) {
    Segs sg{};
    sg.w[0] = w;
    sg.n[0] = n;
    sg.bias[0] = bias;
    sg.y[0] = y;
    sg.count = 1;
    return sg;
}

}  // namespace

hipError_t launch_gemmw(uint32_t type, const uint8_t* w, int k, int n, int m, const float* xs,
                        const _Float16* qh, const uint16_t* xq,
                        const float* bias, float* y, float* part, size_t part_bytes,
                        hipStream_t stream) {
    return gemmw_dispatch(type, one_seg(w, n, bias, y), k, m, xs, qh, xq, part, part_bytes, stream);
}

bool gemmw_multi_supported(uint32_t type, int count) {
    return (type == T_Q4_K || type == T_Q5_K) && count >= 1 && count <= kMaxSegs;
}

size_t gemmw_multi_partial_bytes(uint32_t type, int k, int count, const int* n, int m) {
    if (!gemmw_supported(type) || k % 256 != 0 || !gemmw_multi_supported(type, count)) return 0;
    Segs sg{};
    sg.count = count;
    for (int i = 0; i < count; ++i) sg.n[i] = n[i];
    const Plan p = plan_for(type, k, segs_rows(sg), m);
    if (p.splits <= 1) return 0;
    const size_t tile_bytes = (size_t)(32 * p.nt * p.wv) * (size_t)(32 * p.mt) * sizeof(float);
    return (size_t)p.splits * (size_t)segs_tiles(p, sg, m) * tile_bytes + kCounterBytes;
}

hipError_t launch_gemmw_multi(uint32_t type, int k, int m, int count, const uint8_t* const* w,
                              const int* n, const float* const* bias, float* const* y,
                              const float* xs, const _Float16* qh, const uint16_t* xq,
                              float* part, size_t part_bytes, hipStream_t stream) {
    if (!gemmw_multi_supported(type, count)) return hipErrorNotSupported;
    Segs sg{};
    sg.count = count;
    for (int i = 0; i < count; ++i) {
        sg.w[i] = w[i];
        sg.n[i] = n[i];
        sg.bias[i] = bias ? bias[i] : nullptr;
        sg.y[i] = y[i];
    }
    return gemmw_dispatch(type, sg, k, m, xs, qh, xq, part, part_bytes, stream);
}

void gemmw_multi_plan_name(uint32_t type, int k, int count, const int* n, int m, char* buf,
                           size_t cap) {
    int rows = 0;
    for (int i = 0; i < count; ++i) rows += n[i];
    gemmw_plan_name(type, k, rows, m, buf, cap);
}

void gemmw_plan_name(uint32_t type, int k, int n, int m, char* buf, size_t cap) {
    if (!gemmw_supported(type) || k % 256 != 0) {
        snprintf(buf, cap, "none");
        return;
    }
    const Plan p = plan_for(type, k, n, m);
    if (type == T_Q6_K)
        snprintf(buf, cap, "k_gemmw_q6k<%d,%d> splits=%d", p.wv, p.mt, p.splits);
    else if (is_b32(type))
        snprintf(buf, cap, "k_gemmw_b32<%s,4,%d> splits=%d",
                 type == T_Q8_0 ? "Q8_0" : type == T_Q4_0 ? "Q4_0" : "Q5_0", p.mt, p.splits);
    else
        snprintf(buf, cap, "k_gemmw_q4k<%d,%d,%d,%s> splits=%d", p.wv, p.nt, p.mt,
                 type == T_Q5_K ? "Q5_K" : "Q4_K", p.splits);
}

}  // namespace cllm_hip
