// k_attention.hip -- the float ops between the linear layers on the device: NEOX RoPE and
// grouped-query attention over a KV cache (decode and prefill).
//
// Reference (src/core/engine.cpp):
//   apply_rope (41-56): per head, pairs (i, i + half), theta = pos / base^(i / half),
//     x_i' = x_i cos - x_{i+half} sin, x_{i+half}' = x_i sin + x_{i+half} cos;
//   attention (114-146): per query head h (KV head h / n_rep), s_t = dot(q_h, k_t) / sqrt(d)
//     over the t < seq cached positions, softmax (max subtracted, exp, sum), then
//     out_h = sum_t (e_t / sum) v_t; decode (495) and prefill (581-583, query t of the
//     batch sees pos0 + t + 1 positions).
//
// Two attention kernels: k_attention (below; decode, and a few rows over a long cache) and
// k_attention_mfma (many query rows, on fp32 MFMA; its layout is described above it).
//
// Attention layout. One workgroup per (KV head, query row, sequence split); it serves the
// n_rep query heads of that KV head, so every K and V row is loaded once for all of them.
// Positions go in chunks of 64: sixteen lanes per position read the K row (16-byte pieces,
// coalesced), each lane dots its slice with every query head held in registers, a 16-lane
// reduction gives the scores; the softmax is online (running max and sum per head, the
// partial output rescaled when the max grows); each wave adds p_t v_t for its 16 positions
// of the chunk into per-lane partial outputs (lane l owns dims l + 64 e of every head), with
// every K and V load of a chunk issued before the arithmetic that needs it; the four waves'
// partials are added at the end.
// Long sequences are split over several workgroups whose (max, sum, unnormalised output)
// partials the last of them to finish combines (a per-(row, KV head) arrival counter), so a
// decode step (one query row) still spreads over the device in one launch. The summation
// order differs from the reference's (per-chunk and per-split partial sums, output divided
// by the sum once); the arithmetic is otherwise the same
// fp32 operations with the device's expf, sinf, cosf and powf.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "device_utils.h"
#include "launch.h"

namespace cllm_hip {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------------- RoPE

// grid (rows, n_heads + n_heads2), half = head_dim / 2 threads (up to 256): row t has
// position pos0 + t; heads past n_heads belong to the second tensor x2 (the keys), so the
// queries and keys of a layer turn in one launch.
__global__ __launch_bounds__(256) void k_rope_neox(float* __restrict__ x, int n_heads,
                                                   float* __restrict__ x2, int n_heads2,
                                                   int head_dim, int pos0, float base) {
    const int t = blockIdx.x, i = threadIdx.x;
    const int half = head_dim / 2;
    if (i >= half) return;
    const bool second = (int)blockIdx.y >= n_heads;
    const int h = second ? blockIdx.y - n_heads : blockIdx.y;
    float* xh = (second ? x2 + (size_t)t * n_heads2 * head_dim : x + (size_t)t * n_heads * head_dim) +
                (size_t)h * head_dim;
    const float theta = __fdiv_rn((float)(pos0 + t), powf(base, __fdiv_rn((float)i, (float)half)));
    const float c = cosf(theta), s = sinf(theta);
    const float x0 = xh[i], x1 = xh[i + half];
    xh[i] = __builtin_fmaf(x0, c, -__fmul_rn(x1, s));
    xh[i + half] = __builtin_fmaf(x0, s, __fmul_rn(x1, c));
}

// ----------------------------------------------------------------------------- attention

constexpr int kThreads = 256;
constexpr int kChunk = 64;       // positions per online-softmax step
constexpr int kLanesPerPos = 16; // lanes sharing one K row
constexpr int kMaxRep = 8;       // query heads per KV head
constexpr int kAttnCounters = 1024;  // (row, KV head) pairs a split launch may have
constexpr int kMaxSplits = 256;      // sequence splits per (row, KV head)

// HD = head_dim (multiple of 64, at most 256). Partials of split z for query head hq of row
// t: part[((t * n_head + hq) * S + z) * (HD + 4) + ...] = unnormalised output [HD], max, sum
// (two floats of padding keep every row 16-byte aligned for the combine's vector loads).
// With one split, the normalised output goes straight to out.
//
// rope_base > 0 (one query row, a decode step): the queries and the key row at pos0 arrive
// unrotated and the kernel applies the NEOX rotation of k_rope_neox itself, to the queries in
// registers and to the key row as it loads it, writing the rotated key row back to k_new (the
// cache row pos0, read by no other workgroup: only the split holding pos0 covers it). k_new
// points into the key cache, so kc carries no __restrict__: the compiler may not treat the
// cache as unwritten by this kernel.
template <int HD>
__global__ __launch_bounds__(kThreads) void k_attention(
    const float* __restrict__ q, const float* kc, const float* __restrict__ vc,
    int n_head, int n_kv, int pos0, int split_len, float scale, float* __restrict__ part,
    int* __restrict__ counters, float* __restrict__ out, float rope_base, float* k_new) {
    constexpr int PER = HD / kLanesPerPos;  // K elements per lane (4 .. 16)
    __shared__ float sc[kMaxRep][kChunk];
    __shared__ float m_run[kMaxRep], l_run[kMaxRep], corr[kMaxRep];

    const int kvh = blockIdx.x, t = blockIdx.y, z = blockIdx.z, S = gridDim.z;
    const int n_rep = n_head / n_kv;
    const int kv_dim = n_kv * HD;
    const int L = pos0 + t + 1;
    const int begin = z * split_len;
    const int end = min(L, begin + split_len);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int seg = lane % kLanesPerPos, sub = lane / kLanesPerPos;  // sub: position in wave

    // this lane's slice of every query head of the group
    float qv[kMaxRep][PER];
#pragma unroll
    for (int r = 0; r < kMaxRep; ++r) {
        const float* qh = q + ((size_t)t * n_head + kvh * n_rep + min(r, n_rep - 1)) * HD + seg * PER;
#pragma unroll
        for (int e = 0; e < PER; e += 4) {
            const f32x4 v = *(const f32x4*)(qh + e);
            qv[r][e] = v.x; qv[r][e + 1] = v.y; qv[r][e + 2] = v.z; qv[r][e + 3] = v.w;
        }
    }
    // NEOX rotation at position pos0: dims seg * PER + e pair with the partner lane seg ^ 8
    // (the other half of the head); lanes seg < 8 hold x0 (dims i < HD / 2), the others x1.
    const bool rope = rope_base > 0.0f;
    const bool lo_half = seg < 8;
    float rc[PER], rs[PER];
    auto rotate = [&](float (&x)[PER]) {
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            const float other = __shfl_xor(x[e], 8, 16);
            const float x0 = lo_half ? x[e] : other, x1 = lo_half ? other : x[e];
            x[e] = lo_half ? __builtin_fmaf(x0, rc[e], -__fmul_rn(x1, rs[e]))
                           : __builtin_fmaf(x0, rs[e], __fmul_rn(x1, rc[e]));
        }
    };
    // the angles of the HD / 2 pairs, one per thread, shared through LDS
    __shared__ float rope_cs[2][HD / 2];
    if (rope && threadIdx.x < HD / 2) {
        const int i = threadIdx.x;
        const float theta = __fdiv_rn((float)pos0, powf(rope_base, __fdiv_rn((float)i, (float)(HD / 2))));
        rope_cs[0][i] = cosf(theta);
        rope_cs[1][i] = sinf(theta);
    }
    // Each wave accumulates the output of its own 16 positions of every chunk: lane l owns
    // dims l + 64 e (e < HD / 64) of every query head of the group; the four waves' partials
    // are added at the end.
    constexpr int DE = HD / 64;
    float acc[kMaxRep][DE];
#pragma unroll
    for (int r = 0; r < kMaxRep; ++r)
#pragma unroll
        for (int e = 0; e < DE; ++e) acc[r][e] = 0.0f;
    if (threadIdx.x < kMaxRep) {
        m_run[threadIdx.x] = -INFINITY;
        l_run[threadIdx.x] = 0.0f;
    }
    __syncthreads();
    if (rope) {
#pragma unroll
        for (int e = 0; e < PER; ++e) {
            rc[e] = rope_cs[0][(seg & 7) * PER + e];
            rs[e] = rope_cs[1][(seg & 7) * PER + e];
        }
#pragma unroll
        for (int r = 0; r < kMaxRep; ++r) rotate(qv[r]);
    }

    for (int c0 = begin; c0 < end; c0 += kChunk) {
        // scores of the chunk: each wave takes 4 positions per round, 4 rounds; all the K
        // loads of the chunk are issued before the first dot
        float kv[kChunk / 16][PER];
#pragma unroll
        for (int round = 0; round < kChunk / 16; ++round) {
            const int pc = min(c0 + round * 16 + wave * 4 + sub, end - 1);
            const float* kr = kc + (size_t)pc * kv_dim + kvh * HD + seg * PER;
#pragma unroll
            for (int e = 0; e < PER; e += 4) {
                const f32x4 v = *(const f32x4*)(kr + e);
                kv[round][e] = v.x; kv[round][e + 1] = v.y; kv[round][e + 2] = v.z;
                kv[round][e + 3] = v.w;
            }
        }
        // the new key row (clamped positions past the end repeat it, and rotate it alike)
        bool knew[kChunk / 16];
        if (rope) {
#pragma unroll
            for (int round = 0; round < kChunk / 16; ++round) {
                knew[round] = min(c0 + round * 16 + wave * 4 + sub, end - 1) == pos0;
                float rot[PER];
#pragma unroll
                for (int e = 0; e < PER; ++e) rot[e] = kv[round][e];
                rotate(rot);
                if (knew[round]) {
#pragma unroll
                    for (int e = 0; e < PER; ++e) kv[round][e] = rot[e];
                }
            }
        }
        // this wave's V rows, issued with the K rows so both latencies overlap the score and softmax
        // work (rows past the end are clamped, their probability is zero)
        float vv[16][DE];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int pc = min(c0 + wave * 16 + j, end - 1);
            const float* vr = vc + (size_t)pc * kv_dim + kvh * HD + lane;
#pragma unroll
            for (int e = 0; e < DE; ++e) vv[j][e] = vr[64 * e];
        }
#pragma unroll
        for (int round = 0; round < kChunk / 16; ++round) {
            const int slot = round * 16 + wave * 4 + sub;
            const int p = c0 + slot;
#pragma unroll
            for (int r = 0; r < kMaxRep; ++r) {
                if (r >= n_rep) break;
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < PER; ++e) d = __builtin_fmaf(qv[r][e], kv[round][e], d);
                d += __shfl_xor(d, 8, 16);
                d += __shfl_xor(d, 4, 16);
                d += __shfl_xor(d, 2, 16);
                d += __shfl_xor(d, 1, 16);
                if (seg == 0) sc[r][slot] = p < end ? __fmul_rn(d, scale) : -INFINITY;
            }
        }
        __syncthreads();
        // every K load of the workgroup has been consumed: the rotated row can go back
        if (rope) {
#pragma unroll
            for (int round = 0; round < kChunk / 16; ++round) {
                if (knew[round]) {
                    float* kw = k_new + kvh * HD + seg * PER;
#pragma unroll
                    for (int e = 0; e < PER; e += 4)
                        *(f32x4*)(kw + e) = f32x4{kv[round][e], kv[round][e + 1], kv[round][e + 2], kv[round][e + 3]};
                }
            }
        }
        // one wave per query head (lane i = position i of the chunk): the running max, the
        // probabilities relative to it in place of the scores, their sum, and the factor that
        // rescales what is already summed
        static_assert(kChunk == 64, "a chunk is one wave's lanes");
        for (int r = wave; r < n_rep; r += kThreads / 64) {
            const float s = sc[r][lane];
            float cm = s;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) cm = fmaxf(cm, __shfl_xor(cm, o, 64));
            const float mo = m_run[r], mn = fmaxf(mo, cm);
            const float pr = s == -INFINITY ? 0.0f : expf(s - mn);
            float ps = pr;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) ps += __shfl_xor(ps, o, 64);
            sc[r][lane] = pr;
            if (lane == 0) {
                const float cr = mo == -INFINITY ? 0.0f : expf(mo - mn);
                corr[r] = cr;
                m_run[r] = mn;
                l_run[r] = __builtin_fmaf(l_run[r], cr, ps);
            }
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < kMaxRep; ++r) {
            if (r >= n_rep) break;
            const float cr = corr[r];
#pragma unroll
            for (int e = 0; e < DE; ++e) {
                float a = acc[r][e] * cr;
#pragma unroll
                for (int j = 0; j < 16; ++j) a = __builtin_fmaf(sc[r][wave * 16 + j], vv[j][e], a);
                acc[r][e] = a;
            }
        }
        __syncthreads();
    }

    // the four waves' partial outputs, added through LDS (reusing nothing else: a separate
    // buffer), then the split's partial or the normalised output
    __shared__ float wpart[kThreads / 64][kMaxRep * HD];
#pragma unroll
    for (int r = 0; r < kMaxRep; ++r) {
        if (r >= n_rep) break;
#pragma unroll
        for (int e = 0; e < DE; ++e) wpart[wave][r * HD + lane + 64 * e] = acc[r][e];
    }
    __syncthreads();
    if (S == 1) {
        for (int o = threadIdx.x; o < n_rep * HD; o += kThreads) {
            const int r = o / HD, d = o - r * HD;
            const float v = (wpart[0][o] + wpart[1][o]) + (wpart[2][o] + wpart[3][o]);
            out[((size_t)t * n_head + kvh * n_rep + r) * HD + d] = __fdiv_rn(v, l_run[r]);
        }
        return;
    }
    // Several splits: write this split's partial; the last split of (row, KV head) to
    // arrive, found by a counter it resets, combines them all. The partials cross XCDs, whose
    // L2s are not coherent with each other, so they are stored and loaded as relaxed
    // agent-scope atomics (coherent device-wide by themselves; no L2-wide fence).
    for (int o = threadIdx.x; o < n_rep * HD; o += kThreads) {
        const int r = o / HD, d = o - r * HD;
        const float v = (wpart[0][o] + wpart[1][o]) + (wpart[2][o] + wpart[3][o]);
        float* pp = part + (((size_t)t * n_head + kvh * n_rep + r) * S + z) * (HD + 4);
        __hip_atomic_store(pp + d, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (d == 0) {
            __hip_atomic_store(pp + HD, m_run[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(pp + HD + 1, l_run[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
    __syncthreads();
    __shared__ int last;
    if (threadIdx.x == 0) {
        int* cnt = counters + (size_t)t * n_kv + kvh;
        const int arrived = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = arrived == S - 1;
        if (arrived == S - 1) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last) return;
    // out = sum_z e^(m_z - M) o_z / sum_z e^(m_z - M) l_z, per head of the group. The maxima
    // and sums of all splits are loaded at once (one per thread) into LDS; each output then
    // reads its S values sixteen loads at a time.
    auto ld = [](const float* a) {
        return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    __shared__ float wz[kMaxRep][kMaxSplits], lsum[kMaxRep];
    float* mz = &wpart[0][0];  // the wave partials are consumed: reuse as [kMaxRep][S] maxima
    for (int i = threadIdx.x; i < n_rep * S; i += kThreads) {
        const int r = i / S, zz = i - r * S;
        const float* pz = part + (((size_t)t * n_head + kvh * n_rep + r) * S + zz) * (HD + 4);
        mz[r * S + zz] = ld(pz + HD);
        wz[r][zz] = ld(pz + HD + 1);  // the sums for now
    }
    __syncthreads();
    if (threadIdx.x < n_rep) {
        const int r = threadIdx.x;
        float M = -INFINITY;
        for (int zz = 0; zz < S; ++zz) M = fmaxf(M, mz[r * S + zz]);
        float den = 0.0f;
        for (int zz = 0; zz < S; ++zz) {
            const float m = mz[r * S + zz];
            const float wgt = m == -INFINITY ? 0.0f : expf(m - M);
            den = __builtin_fmaf(wgt, wz[r][zz], den);
            wz[r][zz] = wgt;
        }
        lsum[r] = den;
    }
    __syncthreads();
    // Each thread takes four consecutive dims of one head and reads them as one 16-byte
    // load per split: a buffer load with the SC1 bit, the same device-scope cache policy as
    // the agent-scope atomic loads above, over this (row, KV head)'s partial rows. Sixteen
    // splits at a time are in flight; per output the additions are in split order.
    typedef float f32x4v __attribute__((ext_vector_type(4)));
    const float* pg = part + ((size_t)t * n_head + kvh * n_rep) * S * (HD + 4);
    const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)pg, (short)0, (int)((size_t)n_rep * S * (HD + 4) * sizeof(float)), 0x00020000);
    auto ld4 = [&](uint32_t off) {
        return __builtin_bit_cast(f32x4v, __builtin_amdgcn_raw_buffer_load_b128(prs, off, 0, 16));
    };
    constexpr int Q = HD / 4;
    for (int o = threadIdx.x; o < n_rep * Q; o += kThreads) {
        const int r = o / Q, d = 4 * (o - r * Q);
        const uint32_t off0 = (uint32_t)((r * S * (HD + 4) + d) * sizeof(float));
        const uint32_t zstep = (uint32_t)((HD + 4) * sizeof(float));
        f32x4v num = {0.0f, 0.0f, 0.0f, 0.0f};
        auto add = [&](float wgt, f32x4v v) {
            num.x = __builtin_fmaf(wgt, v.x, num.x);
            num.y = __builtin_fmaf(wgt, v.y, num.y);
            num.z = __builtin_fmaf(wgt, v.z, num.z);
            num.w = __builtin_fmaf(wgt, v.w, num.w);
        };
        int zz = 0;
        for (; zz + 16 <= S; zz += 16) {
            f32x4v v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) v[u] = ld4(off0 + (uint32_t)(zz + u) * zstep);
#pragma unroll
            for (int u = 0; u < 16; ++u) add(wz[r][zz + u], v[u]);
        }
        if (zz < S) {  // the last S % 16, also loaded together (one round trip, same order)
            f32x4v v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u)
                v[u] = zz + u < S ? ld4(off0 + (uint32_t)(zz + u) * zstep) : f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int u = 0; u < 16; ++u)
                if (zz + u < S) add(wz[r][zz + u], v[u]);
        }
        float* op = out + ((size_t)t * n_head + kvh * n_rep + r) * HD + d;
        op[0] = __fdiv_rn(num.x, lsum[r]);
        op[1] = __fdiv_rn(num.y, lsum[r]);
        op[2] = __fdiv_rn(num.z, lsum[r]);
        op[3] = __fdiv_rn(num.w, lsum[r]);
    }
}

// The split kernel's sequence splits for these rows: enough workgroups for the device, at
// least one chunk per split (one split when the rows' arrival counters would not fit).
int attention_splits(int rows, int pos0, int n_kv) {
    const int L_max = pos0 + rows;
    const int64_t base = (int64_t)n_kv * rows;
    int S = (int)std::min<int64_t>(std::max<int64_t>(1, (1024 + base - 1) / base),
                                   (L_max + kChunk - 1) / kChunk);
    S = std::min(S, kMaxSplits);
    if ((int64_t)rows * n_kv > kAttnCounters) S = 1;
    const int split_len = ((L_max + S - 1) / S + kChunk - 1) / kChunk * kChunk;
    return (L_max + split_len - 1) / split_len;
}

template <int HD>
hipError_t launch_attention_hd(const float* q, const float* kc, const float* vc, int rows,
                               int pos0, int n_head, int n_kv, float* out, float* part,
                               size_t part_floats, int* counters, float rope_base, float* k_new,
                               hipStream_t stream) {
    const int L_max = pos0 + rows;
    int S = attention_splits(rows, pos0, n_kv);
    if ((size_t)rows * n_head * S * (HD + 4) > part_floats || !counters) S = 1;
    const int split_len = ((L_max + S - 1) / S + kChunk - 1) / kChunk * kChunk;
    S = (L_max + split_len - 1) / split_len;
    const float scale = 1.0f / std::sqrt((float)HD);  // engine.cpp:121, IEEE on the host
    hipLaunchKernelGGL((k_attention<HD>), dim3((unsigned)n_kv, (unsigned)rows, (unsigned)S),
                       dim3(kThreads), 0, stream, q, kc, vc, n_head, n_kv, pos0, split_len, scale,
                       part, counters, out, rope_base, k_new);
    return hipGetLastError();
}

// ------------------------------------------------------------- many query rows on MFMA

// Prefill attention on the fp32 matrix cores (v_mfma_f32_16x16x4f32: the same fp32 products
// and sums as the split kernel's FMAs, in another order).
//
// Columns. A query block is COLS = 16 * CT (row, head) pairs of one KV head: column c is
// query head c % n_rep of row r0 + c / n_rep, so the n_rep heads of a row and several rows
// share every K and V row loaded.
//
// Balance. Row block b needs pos0 + (its last row + 1) positions, so causal work grows with
// b; a workgroup takes blocks p and n_blocks - 1 - p, and the 16-position steps of the two
// form one list that its W waves split evenly (the wave whose share straddles the two blocks
// works on both). Each wave's part of a block leaves a (max, sum, unnormalised output) partial
// in LDS; one combine at the end adds each block's partials in slot order. The KV head is the
// fastest grid index, which keeps a KV head's workgroups on one XCD (blockIdx modulo 8) and
// its K and V rows in that XCD's L2 when n_kv is 8. Two waves per SIMD (W = 8 up to head_dim
// 128).
//
// One step, per 16-column tile: the scores come out transposed, S^T (16 positions x 16
// columns) = K Q^T over HD / 4 MFMAs (lane l holds K row l % 16 and Q column l % 16 at
// dims (HD / 4) (l / 16) + j for MFMA j; even and odd j in two accumulators added at the end,
// which halves the longest rounding chain), so lane l holds column l % 16's scores of
// positions 4 (l / 16) + i in its four result registers. That is the B operand of
// O^T (HD x 16 columns) = V^T P^T, one MFMA per (i, 16-dim tile dt): the A operand is
// V[4 (l / 16) + i][(HD / 16) (l % 16) + dt], dims permuted so each lane reads HD / 16
// consecutive values of a row. The online softmax is per lane: a column's running max and
// sum live in the four lanes l % 16 of its tile, reduced with v_permlane32_swap and
// v_permlane16_swap (lanes l ^ 32, l ^ 16).
//
// Pipeline. A wave issues the next step's score MFMAs interleaved with this step's softmax
// (an MFMA every few VALU instructions, so the matrix pipe stays busy through the softmax),
// then this step's P.V MFMAs; K rows are requested two steps ahead and V rows one step
// ahead. Loads past a part's last step are clamped to rows in bounds instead of branched, so
// a step is one basic block.

// x combined with its value in lanes l ^ 16, l ^ 32 and l ^ 48 (max or sum)
template <bool MAX>
__device__ __forceinline__ float quad_reduce(float x) {
    const unsigned u = __float_as_uint(x);
    const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    const float a0 = __uint_as_float(a[0]), a1 = __uint_as_float(a[1]);
    x = MAX ? fmaxf(a0, a1) : a0 + a1;
    const unsigned v = __float_as_uint(x);
    const auto b = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    const float b0 = __uint_as_float(b[0]), b1 = __uint_as_float(b[1]);
    return MAX ? fmaxf(b0, b1) : b0 + b1;
}

template <int HD, int CT, int W>
__global__ __launch_bounds__(W * 64) void k_attention_mfma(
    const float* __restrict__ q, const float* __restrict__ kc, const float* __restrict__ vc,
    int n_head, int n_kv, int rows, int pos0, int n_blocks, float scale, float* __restrict__ out) {
    constexpr int COLS = 16 * CT;
    constexpr int DQ = HD / 4;   // K and Q values per lane and row
    constexpr int DV = HD / 16;  // V values per lane and row
    constexpr int PAD = HD + 4;  // LDS row stride of the partial outputs
    constexpr int NS = W + 1;    // partial slots: one per wave, one more for the straddling wave
    __shared__ float o_sm[NS][COLS][PAD];
    __shared__ float m_sm[NS][COLS], l_sm[NS][COLS];
    __shared__ float den_sm[2][COLS];
    __shared__ int slot_blk[NS];  // the block (0 or 1) whose partial a slot holds, -1: none

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col16 = lane & 15, quad = lane >> 4;
    const int g = blockIdx.x % n_kv, pair = blockIdx.x / n_kv;
    const int n_rep = n_head / n_kv, rpb = COLS / n_rep, used = rpb * n_rep;
    const size_t kv_dim = (size_t)n_kv * HD;
    const float* kg = kc + (size_t)g * HD + DQ * quad;
    const float* vg = vc + (size_t)g * HD + DV * col16;

    const int blk_row[2] = {pair * rpb, (n_blocks - 1 - pair) * rpb};
    const bool two = n_blocks - 1 - pair > pair;
    const int len[2] = {pos0 + min(rows, blk_row[0] + rpb), two ? pos0 + min(rows, blk_row[1] + rpb) : 0};
    const int nA = (len[0] + 15) / 16, T = nA + (len[1] + 15) / 16;
    const int g0 = wave * T / W, g1 = (wave + 1) * T / W;
    if (lane == 0) {
        slot_blk[wave] = g0 >= g1 ? -1 : g1 > nA ? 1 : 0;
        if (wave == 0) {
            bool straddle = false;
            for (int w = 0; w < W; ++w) straddle |= w * T / W < nA && nA < (w + 1) * T / W;
            slot_blk[W] = straddle ? 0 : -1;
        }
    }

    for (int part = 0; part < 2; ++part) {
        const int s0 = part == 0 ? g0 : max(g0, nA) - nA;
        const int s1 = part == 0 ? min(g1, nA) : g1 - nA;
        if (s0 >= s1) continue;
        const int r0 = blk_row[part], L = len[part];
        const int slot = part == 0 && g1 > nA ? W : wave;

        // the queries of this lane's columns (unused columns: zeros from a row in bounds);
        // lim = the last position a column sees (-1: an unused column, every score masked)
        float qf[CT][DQ];
        int lim[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            const int c = ct * 16 + col16;
            const int t = r0 + c / n_rep;
            const bool valid = c < used && t < rows;
            lim[ct] = valid ? pos0 + t : -1;
            const float* qr = q + ((size_t)min(t, rows - 1) * n_head + g * n_rep + c % n_rep) * HD + DQ * quad;
#pragma unroll
            for (int j = 0; j < DQ; j += 4) {
                const f32x4 v = *(const f32x4*)(qr + j);
                qf[ct][j] = valid ? v.x : 0.0f;
                qf[ct][j + 1] = valid ? v.y : 0.0f;
                qf[ct][j + 2] = valid ? v.z : 0.0f;
                qf[ct][j + 3] = valid ? v.w : 0.0f;
            }
        }
        f32x4 o[CT][DV];
        float m_run[CT], l_run[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            m_run[ct] = -INFINITY;
            l_run[ct] = 0.0f;
#pragma unroll
            for (int dt = 0; dt < DV; ++dt) o[ct][dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }

        // K row 16 s + l % 16 and V rows 16 s + 4 (l / 16) + i of step s, positions clamped
        // to the block's last (their scores are masked) and steps to the part's last
        float kf[DQ], vf[4][DV];
        auto load_k = [&](int s) {
            const float* kr = kg + (size_t)min(min(s, s1 - 1) * 16 + col16, L - 1) * kv_dim;
#pragma unroll
            for (int j = 0; j < DQ; j += 4) {
                const f32x4 v = *(const f32x4*)(kr + j);
                kf[j] = v.x; kf[j + 1] = v.y; kf[j + 2] = v.z; kf[j + 3] = v.w;
            }
        };
        auto load_v = [&](int s) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float* vr = vg + (size_t)min(min(s, s1 - 1) * 16 + 4 * quad + i, L - 1) * kv_dim;
#pragma unroll
                for (int e = 0; e < DV; e += 4) {
                    const f32x4 v = *(const f32x4*)(vr + e);
                    vf[i][e] = v.x; vf[i][e + 1] = v.y; vf[i][e + 2] = v.z; vf[i][e + 3] = v.w;
                }
            }
        };
        auto scores = [&](f32x4 (&sa)[CT][2]) {
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) sa[ct][0] = sa[ct][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < DQ; ++j)
#pragma unroll
                for (int ct = 0; ct < CT; ++ct)
                    sa[ct][j & 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[j], qf[ct][j], sa[ct][j & 1], 0, 0, 0);
        };
        // the online softmax of step s's scores: probabilities into pr, the running max, sum
        // and output rescaled (by exactly 1 while a column's max stands)
        float pr[CT][4];
        auto softmax = [&](int s, const f32x4 (&sa)[CT][2]) {
            const int pq = s * 16 + 4 * quad;  // position of result register 0
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                const f32x4 sc = sa[ct][0] + sa[ct][1];
                float sv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) sv[i] = pq + i <= lim[ct] ? __fmul_rn(sc[i], scale) : -INFINITY;
                const float mx = quad_reduce<true>(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])));
                const float mo = m_run[ct], mn = fmaxf(mo, mx);
                float ps = 0.0f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float e = expf(sv[i] - mn);
                    pr[ct][i] = sv[i] == -INFINITY ? 0.0f : e;
                    ps += pr[ct][i];
                }
                ps = quad_reduce<false>(ps);
                const float e = expf(mo - mn);
                const float cr = mo == -INFINITY ? 0.0f : e;
                m_run[ct] = mn;
                l_run[ct] = __builtin_fmaf(l_run[ct], cr, ps);
#pragma unroll
                for (int dt = 0; dt < DV; ++dt) o[ct][dt] *= cr;
            }
        };
        auto pv = [&]() {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int dt = 0; dt < DV; ++dt)
#pragma unroll
                    for (int ct = 0; ct < CT; ++ct)
                        o[ct][dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[i][dt], pr[ct][i], o[ct][dt], 0, 0, 0);
        };

        f32x4 sa[CT][2];
        load_k(s0);
        load_v(s0);
        scores(sa);
        load_k(s0 + 1);
        for (int s = s0; s < s1 - 1; ++s) {
            f32x4 sn[CT][2];
            scores(sn);        // step s + 1 (K rows requested a step ago)
            load_k(s + 2);
            softmax(s, sa);    // step s, beside the score MFMAs
#pragma unroll
            for (int i = 0; i < DQ * CT; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);  // five VALU
            }
            pv();
            load_v(s + 1);     // V rows a step ahead of their P.V MFMAs
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
                sa[ct][0] = sn[ct][0];
                sa[ct][1] = sn[ct][1];
            }
        }
        softmax(s1 - 1, sa);
        pv();

        // the part's partial: result register r of dim tile dt is dim DV (4 (l / 16) + r) + dt
        // of column l % 16, so each lane stores HD / 4 consecutive dims
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            const int c = ct * 16 + col16;
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int dt = 0; dt < DV; ++dt) o_sm[slot][c][DV * (4 * quad + r) + dt] = o[ct][dt][r];
            if (quad == 0) {
                m_sm[slot][c] = m_run[ct];
                l_sm[slot][c] = l_run[ct];
            }
        }
    }
    __syncthreads();
    // per (block, column): the partials' weights e^(m - M) in place of their maxima, and the sum
    if (threadIdx.x < 2 * COLS) {
        const int blk = threadIdx.x / COLS, c = threadIdx.x % COLS;
        float M = -INFINITY;
        for (int z = 0; z < NS; ++z)
            if (slot_blk[z] == blk) M = fmaxf(M, m_sm[z][c]);
        float den = 0.0f;
        for (int z = 0; z < NS; ++z) {
            if (slot_blk[z] != blk) continue;
            const float m = m_sm[z][c];
            const float e = expf(m - M);
            const float wgt = m == -INFINITY ? 0.0f : e;
            den = __builtin_fmaf(wgt, l_sm[z][c], den);
            m_sm[z][c] = wgt;
        }
        den_sm[blk][c] = den;
    }
    __syncthreads();
    for (int o4 = threadIdx.x; o4 < 2 * COLS * (HD / 4); o4 += W * 64) {
        const int blk = o4 / (COLS * (HD / 4));
        const int c = (o4 / (HD / 4)) % COLS, d = (o4 % (HD / 4)) * 4;
        const int t = blk_row[blk] + c / n_rep;
        if ((blk == 1 && !two) || c >= used || t >= rows) continue;
        f32x4 num = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        for (int z = 0; z < NS; ++z) {
            if (slot_blk[z] != blk) continue;
            const float wgt = m_sm[z][c];
            const f32x4 v = *(const f32x4*)&o_sm[z][c][d];
            num.x = __builtin_fmaf(wgt, v.x, num.x);
            num.y = __builtin_fmaf(wgt, v.y, num.y);
            num.z = __builtin_fmaf(wgt, v.z, num.z);
            num.w = __builtin_fmaf(wgt, v.w, num.w);
        }
        const float den = den_sm[blk][c];
        float* orow = out + ((size_t)t * n_head + g * n_rep + c % n_rep) * HD + d;
        orow[0] = __fdiv_rn(num.x, den);  // out is 4-byte aligned only
        orow[1] = __fdiv_rn(num.y, den);
        orow[2] = __fdiv_rn(num.z, den);
        orow[3] = __fdiv_rn(num.w, den);
    }
}

template <int HD, int CT, int W>
hipError_t launch_attention_mfma_hd(const float* q, const float* kc, const float* vc, int rows,
                                    int pos0, int n_head, int n_kv, float* out, hipStream_t stream) {
    const int rpb = 16 * CT / (n_head / n_kv);
    const int n_blocks = (rows + rpb - 1) / rpb;
    const int pairs = (n_blocks + 1) / 2;
    const float scale = 1.0f / std::sqrt((float)HD);  // engine.cpp:121, IEEE on the host
    hipLaunchKernelGGL((k_attention_mfma<HD, CT, W>), dim3((unsigned)(n_kv * pairs)), dim3(W * 64),
                       0, stream, q, kc, vc, n_head, n_kv, rows, pos0, n_blocks, scale, out);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_rope_neox(float* x, int rows, int n_heads, float* x2, int n_heads2,
                            int head_dim, int pos0, float base, hipStream_t stream) {
    if (!x2) n_heads2 = 0;
    if (rows <= 0 || n_heads + n_heads2 <= 0) return hipSuccess;
    if (head_dim <= 0 || head_dim % 2 != 0 || head_dim > 512) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_rope_neox, dim3((unsigned)rows, (unsigned)(n_heads + n_heads2)), dim3(256),
                       0, stream, x, n_heads, x2, n_heads2, head_dim, pos0, base);
    return hipGetLastError();
}

size_t attention_workspace_bytes(int rows, int n_head, int head_dim) {
    // at most 1024 / (n_kv * rows) + 1 splits, n_kv >= 1
    const size_t splits = (size_t)(1024 / std::max(rows, 1) + 1);
    return kAttnCounters * sizeof(int) + (size_t)rows * n_head * splits * (head_dim + 4) * sizeof(float);
}

namespace {

// Workgroups of the MFMA kernel: n_kv x pairs of row blocks (16 CT columns per block).
int attention_mfma_groups(int rows, int n_head, int n_kv, int head_dim) {
    const int ct = head_dim == 256 ? 1 : 2;
    const int rpb = 16 * ct / (n_head / n_kv);
    const int n_blocks = (rows + rpb - 1) / rpb;
    return n_kv * ((n_blocks + 1) / 2);
}

}  // namespace

// Many query rows go to the MFMA kernel (no workspace, no sequence split); with fewer than 32
// of its workgroups (under 49 rows at 8 KV heads of 4 query heads each) the split kernel,
// which spreads each row's positions over the device, is as fast or faster (MI355X, head_dim
// 128: 32 rows at pos0 1024 89.9 us split / 94.5 MFMA, 64 rows 168 / 97).
bool attention_uses_mfma(int rows, int pos0, int n_head, int n_kv, int head_dim) {
    const int kind = tuning().attention_kind.load();
    if (kind != 0) return kind == 2;
    (void)pos0;
    return attention_mfma_groups(rows, n_head, n_kv, head_dim) >= 32;
}

void attention_plan_name(int rows, int pos0, int n_head, int n_kv, int head_dim, char* buf,
                         size_t cap) {
    if (attention_uses_mfma(rows, pos0, n_head, n_kv, head_dim)) {
        const int ct = head_dim == 256 ? 1 : 2, w = head_dim == 256 ? 4 : 8;
        snprintf(buf, cap, "k_attention_mfma<%d,%d,%d> workgroups=%d", head_dim, ct, w,
                 attention_mfma_groups(rows, n_head, n_kv, head_dim));
    } else {
        snprintf(buf, cap, "k_attention<%d> splits=%d", head_dim, attention_splits(rows, pos0, n_kv));
    }
}

bool attention_supported(int head_dim, int n_head, int n_kv) {
    return (head_dim == 64 || head_dim == 128 || head_dim == 256) && n_kv > 0 &&
           n_head % n_kv == 0 && n_head / n_kv <= kMaxRep;
}

// The workspace: kAttnCounters arrival counters (zero when allocated, left zero by every
// launch), then the split partials.
hipError_t launch_attention(const float* q, const float* kc, const float* vc, int rows, int pos0,
                            int n_head, int n_kv, int head_dim, float* out, void* ws,
                            size_t ws_bytes, hipStream_t stream, float rope_base) {
    if (rows <= 0) return hipSuccess;
    if (!attention_supported(head_dim, n_head, n_kv)) return hipErrorInvalidValue;
    if (rope_base > 0.0f && rows != 1) return hipErrorInvalidValue;
    if (rope_base <= 0.0f && attention_uses_mfma(rows, pos0, n_head, n_kv, head_dim)) {
        switch (head_dim) {
            case 64: return launch_attention_mfma_hd<64, 2, 8>(q, kc, vc, rows, pos0, n_head, n_kv, out, stream);
            case 128: return launch_attention_mfma_hd<128, 2, 8>(q, kc, vc, rows, pos0, n_head, n_kv, out, stream);
            default: return launch_attention_mfma_hd<256, 1, 4>(q, kc, vc, rows, pos0, n_head, n_kv, out, stream);
        }
    }
    float* k_new = rope_base > 0.0f ? const_cast<float*>(kc) + (size_t)pos0 * n_kv * head_dim : nullptr;
    constexpr size_t kCountBytes = kAttnCounters * sizeof(int);
    int* counters = ws && ws_bytes > kCountBytes ? (int*)ws : nullptr;
    float* part = counters ? (float*)((char*)ws + kCountBytes) : nullptr;
    const size_t part_floats = counters ? (ws_bytes - kCountBytes) / sizeof(float) : 0;
    switch (head_dim) {
        case 64: return launch_attention_hd<64>(q, kc, vc, rows, pos0, n_head, n_kv, out, part, part_floats, counters, rope_base, k_new, stream);
        case 128: return launch_attention_hd<128>(q, kc, vc, rows, pos0, n_head, n_kv, out, part, part_floats, counters, rope_base, k_new, stream);
        default: return launch_attention_hd<256>(q, kc, vc, rows, pos0, n_head, n_kv, out, part, part_floats, counters, rope_base, k_new, stream);
    }
}

}  // namespace cllm_hip
