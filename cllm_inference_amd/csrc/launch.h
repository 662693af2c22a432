// launch.h -- host-side launchers of the kernels (internal to libcllm_hip.so).
//
// Every launcher validates nothing: capi.hip checks shapes, types and alignment before it
// calls one, so the grid of each launch matches what its kernel indexes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace cllm_hip {

// Process-wide kernel-choice overrides for tests and tuning sweeps (cllm_hip_tune). Zero
// everywhere means the planners' own choices; the product never sets them itself.
struct Tuning {
    std::atomic<int> gemm_kind{0};  // 0 planner, 1 int8 MFMA (k_gemm), 2 activation-row fp16 (k_gemm16)
    std::atomic<int> gemm_waves{0}, gemm_wtiles{0}, gemm_ttiles{0};  // weight-row GEMM tile
    std::atomic<int> gemm_splits{0};                                   // weight-row GEMM K splits
    std::atomic<int> gemv_short_wps{0}, gemv_deep_wps{0};              // GEMV waves per SIMD
    std::atomic<int> gemv_kind{0};  // one-row GEMV: 0 planner, 1 k_gemv, 2 k_gemv_st, 3 k_gemv_str
    std::atomic<int> gemv_str_grid{0};  // workgroups of k_gemv_str (0 = one per CU)
    std::atomic<int> gemm_small{0};  // small-batch GEMM: 0 planner, 1 from 3 rows, 2 never
    std::atomic<int> gemm_small_splits{0}, gemm_small_kp{0};  // its plan (0 = planner's)
    std::atomic<int> gemm_small_q8{0};    // fp32 batches: 0 planner, 1 quantized once first, 2 in-kernel
    std::atomic<int> gemv_fused_rows{0};  // streamed GEMV batches quantized in-kernel up to this many rows
    std::atomic<int> attention_kind{0};   // attention: 0 planner, 1 split kernel, 2 MFMA kernel
    std::atomic<int> gemv_fp_wgs{0};  // one-row float-dot GEMV: 0 planner, 1-8 pipelined kernel at that many workgroups per CU, 9 per-row kernel
};
Tuning& tuning();

// n_blocks consecutive 32-element fp32 blocks -> Q8_0 (qs, fp32 scales, int32 block sums).
hipError_t launch_quantize_q8_0(const float* x, int64_t n_blocks, int8_t* qs, float* scales,
                                int32_t* bsums, hipStream_t stream);

// The MFMA path's activation format: fp32 -> Q8_0 as above, kept as dx (scales), the
// quantized values as exact fp16 (qh[m * k]) and dx * bsum (px[m * k / 32]).
hipError_t launch_quantize_mfma(const float* x, int64_t n_blocks, float* scales,
                                _Float16* qh, float* px, hipStream_t stream);
// Same format from an already-quantized Q8_0 batch.
hipError_t launch_q8_to_mfma(const int8_t* qs, const float* scales, const int32_t* bsums,
                             int64_t n_blocks, _Float16* qh, float* px, hipStream_t stream);

// The weight-row GEMM's activation format: dx (scales), the quantized values as exact fp16
// (qh[m * k]) and (xq, may be null) dx * bsum split into bf16 parts, one 64-byte record per
// 8 blocks (xq[m * k / 8]); rows of k % 256 == 0 elements. From fp32 or from a Q8_0 batch.
hipError_t launch_quantize_w(const float* x, int64_t n_blocks, float* scales, _Float16* qh,
                             uint16_t* xq, hipStream_t stream);
// (The Q8_0 variant also copies the scales to scales_out: the GEMM loads them 16 bytes at a
// time, so they must sit in a 16-byte-aligned buffer of the library's own.)
hipError_t launch_q8_to_w(const int8_t* qs, const float* scales, const int32_t* bsums,
                          int64_t n_blocks, float* scales_out, _Float16* qh, uint16_t* xq,
                          hipStream_t stream);

// The decode kernel launch_gemv runs first for m activation rows of a k x n matrix ("none"
// for a type with no vec_dot kernel): name<type,rows per launch> launches=count.
void gemv_plan_name(uint32_t type, int k, int n, int m, char* buf, size_t cap);
// Launches the multi-row GEMV makes for m activation rows (each reads the whole matrix) on
// its register-ring kernel.
int gemv_launch_count(uint32_t type, int k, int m);
// Whether the GEMV takes all m rows (2 to 8) in one launch of its streaming kernel.
bool gemv_streams_batch(uint32_t type, int k, int n, int m);

// y[t, j] = vec_dot(W row j, activation row t) (+ bias[j]) for t < m, j < n.
// Activation rows are Q8_0: qs[t * k], scales / bsums[t * k / 32]. Any m >= 1.
// With accumulate, y[t, j] += vec_dot (+ bias[j]) instead of y[t, j] = ... (the residual add
// that follows a matmul in the engine, fused).
hipError_t launch_gemv(uint32_t type, const uint8_t* w, int k, int n, int m, const int8_t* qs,
                       const float* scales, const int32_t* bsums, const float* bias, float* y,
                       hipStream_t stream, bool accumulate = false);

// launch_gemv over up to three matrices of one type and row length k that read the same
// activation rows (q / k / v, gate / up), in one launch: matrix i has n[i] rows, results
// go to y[i] ([m][n[i]]) plus bias[i] (bias may be null, as may its entries).
hipError_t launch_gemv_multi(uint32_t type, int k, int n_mats, const uint8_t* const* w,
                             const int* n, const float* const* bias, float* const* y, int m,
                             const int8_t* qs, const float* scales, const int32_t* bsums,
                             hipStream_t stream);

// launch_gemv_multi on one fp32 row x[k] (k <= 4096, k % 32 == 0) put through the RMSNorm
// with weight norm_w first, inside the launch: bit-identical to launch_rmsnorm_q8_0 followed
// by launch_gemv_multi.
hipError_t launch_rmsnorm_gemv_multi(uint32_t type, int k, int n_mats, const uint8_t* const* w,
                                     const int* n, const float* const* bias, float* const* y,
                                     const float* x, const float* norm_w, float eps,
                                     hipStream_t stream);

// SwiGLU feed-forward input: h[t, j] = silu(gate_j . a_t + bg_j) * (up_j . a_t + bu_j) for the
// n rows of the gate and up matrices (biases may be null), one launch, on Q8_0 activation rows.
hipError_t launch_gemv_swiglu(uint32_t type, int k, int n, const uint8_t* w_gate,
                              const uint8_t* w_up, const float* bias_gate, const float* bias_up,
                              float* h, int m, const int8_t* qs, const float* scales,
                              const int32_t* bsums, hipStream_t stream);

// launch_gemv_swiglu on one fp32 row x[k] put through the RMSNorm first, inside the launch
// (same limits and result as launch_rmsnorm_gemv_multi).
hipError_t launch_rmsnorm_gemv_swiglu(uint32_t type, int k, int n, const uint8_t* w_gate,
                                      const uint8_t* w_up, const float* bias_gate,
                                      const float* bias_up, const float* x, const float* norm_w,
                                      float eps, float* h, hipStream_t stream);

// Same as launch_gemv with fp32 activation rows x[m][k]: each launch quantizes its rows to
// Q8_0 in LDS (bit-identical to launch_quantize_q8_0) instead of reading a quantized batch,
// so a decode step is a single kernel.
hipError_t launch_gemv_fused(uint32_t type, const uint8_t* w, int k, int n, int m,
                             const float* x, const float* bias, float* y, hipStream_t stream,
                             bool accumulate = false);

// Same contract as launch_gemv, on the int8 MFMA path (m >= 1, any n; k % 256 == 0 for the
// K-quants, k % 32 == 0 otherwise). Returns hipErrorNotSupported for types without an MFMA
// kernel.
hipError_t launch_gemm(uint32_t type, const uint8_t* w, int k, int n, int m, const int8_t* qs,
                       const float* scales, const int32_t* bsums, const float* bias, float* y,
                       hipStream_t stream);
bool gemm_supported(uint32_t type);

// The fp16-MFMA GEMM (k_gemm16.hip), same contract, on the MFMA activation format: qh[m*k]
// fp16 quantized values, xs[m*k/32] dx, xp[m*k/32] dx*bsum. k % 256 == 0.
hipError_t launch_gemm16(uint32_t type, const uint8_t* w, int k, int n, int m,
                         const _Float16* qh, const float* xs, const float* xp, const float* bias,
                         float* y, hipStream_t stream);

// The weight-row fp16-MFMA GEMM (k_gemmw.hip), same contract as launch_gemm, on the activation
// format of launch_quantize_w: dx (xs), fp16 values (qh) and, for Q4_K, the minimum operand
// (xq). All six types; k % 256 == 0. When its plan splits K it needs a workspace part of at
// least gemmw_partial_bytes(type, k, n, m) bytes (else K is not split), zeroed once by
// gemmw_workspace_init when allocated: the splits write partial sums there and the last split
// of each tile adds them into y inside the same launch.
hipError_t launch_gemmw(uint32_t type, const uint8_t* w, int k, int n, int m, const float* xs,
                        const _Float16* qh, const uint16_t* xq,
                        const float* bias, float* y, float* part, size_t part_bytes,
                        hipStream_t stream);
size_t gemmw_partial_bytes(uint32_t type, int k, int n, int m);
// The tile-counter block at the start of that region (the bytes that must be zero).
size_t gemmw_counter_bytes();
// Name of the weight-row kernel instantiation and its split count for this shape, e.g.
// "k_gemmw_q4k<8,1,2,Q5_K> splits=1" (written into buf).
void gemmw_plan_name(uint32_t type, int k, int n, int m, char* buf, size_t cap);

// Producers of the linear layers' activations (k_producers.hip): RMSNorm of `rows` rows of n
// and SwiGLU (silu(gate) * up) over `total` elements, each writing h (fp32, may be null)
// and, when qs is not null and n (total) is a multiple of 32, its Q8_0 blocks; x += d.
// qh / xq (null, or both): the Q8_0 blocks also in the weight-row kernels' format (fp16
// codes, minimum-term operand; the rows whole 256-element super-blocks).
hipError_t launch_rmsnorm_q8_0(const float* x, const float* w, float eps, int n, int rows,
                               float* h, int8_t* qs, float* scales, int32_t* bsums,
                               hipStream_t stream, _Float16* qh = nullptr, uint16_t* xq = nullptr);
hipError_t launch_swiglu_q8_0(const float* gate, const float* up, int64_t total, float* h,
                              int8_t* qs, float* scales, int32_t* bsums, hipStream_t stream,
                              _Float16* qh = nullptr, uint16_t* xq = nullptr);
hipError_t launch_add(float* x, const float* d, int64_t n, hipStream_t stream);

// Float ops between the linear layers (k_attention.hip): NEOX RoPE in place on `rows` rows
// of n_heads x head_dim (row t at position pos0 + t), optionally on a second tensor x2 of
// n_heads2 heads per row in the same launch (queries and keys), and grouped-query attention of `rows`
// query rows (n_head x head_dim each) over KV caches of n_kv x head_dim per position, query
// row t seeing positions [0, pos0 + t]. `ws` (attention_workspace_bytes, zeroed when first
// allocated; null for no sequence split) holds the splits' arrival counters and partials.
hipError_t launch_rope_neox(float* x, int rows, int n_heads, float* x2, int n_heads2,
                            int head_dim, int pos0, float base, hipStream_t stream);
bool attention_supported(int head_dim, int n_head, int n_kv);
// Which attention kernel launch_attention runs for these rows (true: k_attention_mfma), and
// its name with the launch's workgroups or sequence splits.
bool attention_uses_mfma(int rows, int pos0, int n_head, int n_kv, int head_dim);
void attention_plan_name(int rows, int pos0, int n_head, int n_kv, int head_dim, char* buf,
                         size_t cap);
size_t attention_workspace_bytes(int rows, int n_head, int head_dim);
// With rope_base > 0 (rows == 1 only), q and the key row at pos0 are unrotated: the kernel
// applies launch_rope_neox's rotation to both (the key row in place in kc).
hipError_t launch_attention(const float* q, const float* kc, const float* vc, int rows, int pos0,
                            int n_head, int n_kv, int head_dim, float* out, void* ws,
                            size_t ws_bytes, hipStream_t stream, float rope_base = 0.0f);

// Rows ids[0..n) of a weight matrix of any GGML type, dequantized to fp32 out[n][k] exactly
// as the reference's dequantize_block (the embedding lookup). k_gemv_f.hip.
hipError_t launch_dequantize_rows(uint32_t type, const uint8_t* w, int k, const int32_t* ids,
                                  int n, float* out, hipStream_t stream);

// Elements [0, n) of the run of blocks at src (16-byte aligned), dequantized bit for bit as
// dequantize_block (to fp32 out) or dequantize_block_f16 (to binary16 bits out16; exactly one
// of the two outputs is given). A partial last block is read whole, written up to n.
hipError_t launch_dequantize_span(uint32_t type, const uint8_t* src, int64_t n, float* out,
                                  uint16_t* out16, hipStream_t stream);

// Float-dot GEMV (k_gemv_f.hip) for the types without a vec_dot kernel (F32, F16, Q4_1,
// Q5_1, Q8_1, Q2_K, Q3_K): y[t, j] = bias[j] + sum_i x[t, i] * deq(W[j, i]) on fp32
// activation rows x[m][k], as the reference's dequantize fallback computes it.
bool gemv_f_supported(uint32_t type);
hipError_t launch_gemv_f(uint32_t type, const uint8_t* w, int k, int n, int m, const float* x,
                         const float* bias, float* y, hipStream_t stream);
hipError_t gemmw_workspace_init(void* part, size_t bytes, hipStream_t stream);
bool gemmw_supported(uint32_t type);
// Several matrices of one type and K over one activation batch in one weight-row launch
// (Q4_K / Q5_K, up to 3): the same contract as launch_gemmw per matrix, the split-K region
// sized by gemmw_multi_partial_bytes.
bool gemmw_multi_supported(uint32_t type, int count);
size_t gemmw_multi_partial_bytes(uint32_t type, int k, int count, const int* n, int m);
hipError_t launch_gemmw_multi(uint32_t type, int k, int m, int count, const uint8_t* const* w,
                              const int* n, const float* const* bias, float* const* y,
                              const float* xs, const _Float16* qh, const uint16_t* xq,
                              float* part, size_t part_bytes, hipStream_t stream);
void gemmw_multi_plan_name(uint32_t type, int k, int count, const int* n, int m, char* buf,
                           size_t cap);
// false when the shape's weights (4 GiB and up) or fp16 activations (2 m k bytes, 4 GiB and
// up) are past the weight-row kernels' 32-bit offsets; such shapes take the int8 kernel
bool gemmw_fits(uint32_t type, int k, int n, int m);

// Reads `bytes` (a multiple of 16) at the 16-byte-aligned device address p once and computes
// nothing: the one-launch read ceiling of that stream (k_read.hip). cus = the device's CUs.
hipError_t launch_read_stream(const void* p, int64_t bytes, int cus, hipStream_t stream);

// Small-batch GEMM (k_gemm_sm.hip): the same contract as launch_gemv for 1 <= m <= 64 rows of
// Q4_K / Q5_K / Q8_0 weights with k % 256 == 0, on int8 MFMA, the weights streamed once for the
// whole batch. From fp32 rows x[m][k] (quantized in the kernel) or from a Q8_0 batch. part /
// part_bytes: the split-K region (gemm_sm_partial_bytes; its first 64 KB are tile counters that
// must be zero, and every launch leaves them zero).
bool gemm_sm_supported(uint32_t type, int k, int m);
size_t gemm_sm_partial_bytes(uint32_t type, int k, int n, int m);
// fused: the plan of launch_gemm_sm_f32 (quantization inside the kernel), else launch_gemm_sm_q8's
void gemm_sm_plan_name(uint32_t type, int k, int n, int m, bool fused, char* buf, size_t cap);
hipError_t launch_gemm_sm_f32(uint32_t type, const uint8_t* w, int k, int n, int m, const float* x,
                              const float* bias, float* y, float* part, size_t part_bytes,
                              hipStream_t stream);
hipError_t launch_gemm_sm_q8(uint32_t type, const uint8_t* w, int k, int n, int m,
                             const int8_t* qs, const float* xs, const int32_t* xb,
                             const float* bias, float* y, float* part, size_t part_bytes,
                             hipStream_t stream);

}  // namespace cllm_hip
