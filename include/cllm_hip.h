/*
 * cllm_hip.h -- C ABI of the MI355X (gfx950) quantized linear-layer path.
 *
 * This library replaces the compute behind cllm_inference's Quant API
 * (include/cllm/core/quant.hpp:90-151, implemented in src/core/quant.cpp:415-1475). Plain
 * pointers and sizes only: no C++ types, no torch types. The C++20 Quant API itself
 * (include/cllm/core/quant.hpp in this repository, cllm_inference_amd/csrc/quant_api.cpp)
 * is a thin wrapper over these functions, and Python reaches them through ctypes.
 *
 * Conventions
 *   - Every function returns CLLM_HIP_OK (0) or one of the CLLM_HIP_E_* codes; the message
 *     of the last failure on the calling thread is returned by cllm_hip_last_error(). The
 *     messages of the reference's exceptions are reproduced verbatim where one exists.
 *   - "type" is a GgmlType id (F32 = 0 ... Q6_K = 14, include/cllm/core/quant.hpp:13-27).
 *     The six types with a vec_dot kernel in the reference (Q4_0, Q5_0, Q8_0, Q4_K, Q5_K,
 *     Q6_K; src/core/quant.cpp:1347-1357) are computed on Q8_0-quantized activations, like
 *     the reference's fast path; the other seven (F32, F16, Q4_1, Q5_1, Q8_1, Q2_K, Q3_K) on
 *     the fp32 activations, like its dequantize-and-float-dot fallback (1404-1430). The
 *     vec_dot and Q8_0 entry points (cllm_hip_vec_dot_rows, cllm_hip_gemv_q8_dev) take
 *     the six types only.
 *   - Weights are GGUF blocks read in place, row-major: out_dim rows of
 *     (in_dim / block_size) * type_size bytes (src/core/quant.cpp:1381).
 *   - Functions without the _dev suffix take host pointers and are synchronous, like the
 *     reference. Functions with the _dev suffix take device pointers, enqueue on the given
 *     HIP stream (NULL = the null stream) and return without waiting.
 *   - Device weight pointers must be 16-byte aligned (GGUF data sections are 32-byte
 *     aligned, gguf.cpp:171-172); device activation and output pointers 16-byte aligned.
 */
#ifndef CLLM_HIP_H
#define CLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CLLM_HIP_OK 0
#define CLLM_HIP_E_SHAPE 1   /* a dimension is not a multiple of the block size */
#define CLLM_HIP_E_TYPE 2    /* no kernel for this weight type */
#define CLLM_HIP_E_ARG 3     /* null or misaligned pointer, negative size */
#define CLLM_HIP_E_RUNTIME 4 /* HIP runtime failure (allocation, copy, launch) */
#define CLLM_HIP_E_NODEV 5   /* no usable gfx950 device */
#define CLLM_HIP_E_BUSY 6    /* the fixed scratch of the GPU is in use by a call on another stream */

/* Selects the device used by this thread's later calls and builds its per-device state.
 * Calling it is optional: the first call on a thread uses device 0. No reference
 * counterpart (the reference is CPU-only). */
int cllm_hip_init(int device);

/* Message of the last failure on this thread ("" if none). */
const char* cllm_hip_last_error(void);

/* block_size / type_size: include/cllm/core/quant.hpp:90-93, src/core/quant.cpp:340-369. */
int cllm_hip_block_size(uint32_t type);
size_t cllm_hip_type_size(uint32_t type);

/* has_vec_dot: include/cllm/core/quant.hpp:130, src/core/quant.cpp:1347-1357. */
int cllm_hip_has_vec_dot(uint32_t type);

/* quantize_row_q8_0 over n_rows rows of length n (n % 32 == 0): qs[n_rows * n],
 * scales[n_rows * n / 32] (fp32), bsums[n_rows * n / 32]. Bit-exact with the reference.
 * Replaces include/cllm/core/quant.hpp:127 / src/core/quant.cpp:420-452 (which handles one
 * row; n_rows = 1 is that call). Host buffers. */
int cllm_hip_quantize_row_q8_0(const float* x, int64_t n, int n_rows, int8_t* qs,
                               float* scales, int32_t* bsums);

/* vec_dot_row for n_w_rows consecutive weight rows against one Q8_0 activation row:
 * out[j] = vec_dot_row(w + j * row_bytes, type, qx, n). Replaces
 * include/cllm/core/quant.hpp:135-136 / src/core/quant.cpp:1359-1372. Host buffers. */
int cllm_hip_vec_dot_rows(const void* w, uint32_t type, int64_t n, int n_w_rows,
                          const int8_t* qs, const float* scales, const int32_t* bsums,
                          float* out);

/* matmul_quant: y[out_dim] = x[in_dim] . W^T (+ bias). Replaces
 * include/cllm/core/quant.hpp:143-145 / src/core/quant.cpp:1374-1402. Host buffers; w may
 * also be a device pointer or lie inside a region given to cllm_hip_register_weights. */
int cllm_hip_matmul_quant(const float* x, const void* w, uint32_t type, const float* bias,
                          int in_dim, int out_dim, float* y);

/* matmul_quant_batch: y[n_rows, out_dim] row-major. n_rows <= 0 returns without writing y.
 * Replaces include/cllm/core/quant.hpp:149-151 / src/core/quant.cpp:1433-1469. */
int cllm_hip_matmul_quant_batch(const float* x, const void* w, uint32_t type,
                                const float* bias, int in_dim, int out_dim, int n_rows,
                                float* y);

/* Uploads [host_base, host_base + bytes) -- typically the mmap'd GGUF data section
 * (gguf.cpp:178-189) -- to the current device once. Later host weight pointers inside the
 * region resolve to the device copy by offset instead of being copied per call. No
 * reference counterpart: the reference reads the mmap directly (engine.cpp:189). */
int cllm_hip_register_weights(const void* host_base, size_t bytes);
int cllm_hip_unregister_weights(const void* host_base);

/* Weights inside a read-only private file mapping (the engine's mmap'd GGUF, gguf.cpp:178)
 * are copied to the device once per mapping, and each later call first checks that the
 * mapping and its file are unchanged: one kernel mapping query and one fstat. This returns
 * what that check compares, for the mapping holding p: info[0..8] = mapping start, end,
 * file offset, inode, device (major << 32 | minor), then the file's size, mtime and ctime
 * (ns) and 1 if the file is reachable by its path (else the mapping alone is checked).
 * CLLM_HIP_E_ARG if p lies in no read-only private file mapping. Needs no GPU. No reference
 * counterpart: a diagnostic of the device copy's validation. */
int cllm_hip_file_mapping_identity(const void* p, uint64_t info[9]);

/* dequantize_block: the first n elements of the run of blocks at src (ceil(n / block_size)
 * blocks of any of the thirteen types) to fp32 dst[n], bit for bit. A partial last block is
 * read whole and written up to n, as the reference's loops do. src is a host pointer (it may
 * lie in a registered region) or a device pointer, of any alignment; dst is host memory.
 * Decoded on the GPU. Replaces include/cllm/core/quant.hpp:99 / src/core/quant.cpp:371-389
 * (the engine's embedding lookup, engine.cpp:316, and Tensor::dequantize, quant.cpp:391-395). */
int cllm_hip_dequantize_block(const void* src, float* dst, uint32_t type, int64_t n);

/* dequantize_block_f16: the same values as binary16 bits, converted with the reference
 * header's float_to_half rule (normal results truncated); F16 blocks are copied as they are.
 * Replaces include/cllm/core/quant.hpp:105 / src/core/quant.cpp:398-407 (and
 * Tensor::dequantize_f16, 409-412). */
int cllm_hip_dequantize_block_f16(const void* src, uint16_t* dst, uint32_t type, int64_t n);

/* ---- device-pointer entry points (stream-ordered) ------------------------------------ */

/* quantize_row_q8_0 on device buffers (same layout as cllm_hip_quantize_row_q8_0). */
int cllm_hip_quantize_q8_0_dev(const float* x, int64_t n, int n_rows, int8_t* qs,
                               float* scales, int32_t* bsums, void* stream);

/* The vec_dot kernels on an already-quantized activation batch:
 * y[t, j] = vec_dot_row(w row j, type, qx row t, in_dim) (+ bias[j]), t < n_rows.
 * This is the inner loop of src/core/quant.cpp:1388-1397 and 1453-1464. */
int cllm_hip_gemv_q8_dev(const void* w, uint32_t type, int in_dim, int out_dim, int n_rows,
                         const int8_t* qs, const float* scales, const int32_t* bsums,
                         const float* bias, float* y, void* stream);

/* cllm_hip_gemv_q8_dev over n_mats (1 to 3) matrices of one type and in_dim that read the
 * same quantized activation rows, in one launch: the q, k and v projections of one norm's
 * output (src/core/engine.cpp:476-478), or gate and up (509-510). Matrix i has
 * out_dims[i] rows, writes y[i] ([n_rows][out_dims[i]]) and adds bias[i] when bias and
 * bias[i] are not null. */
int cllm_hip_gemv_q8_multi_dev(uint32_t type, int in_dim, int n_mats, const void* const* w,
                               const int* out_dims, const float* const* bias, float* const* y,
                               int n_rows, const int8_t* qs, const float* scales,
                               const int32_t* bsums, void* stream);

/* The gate and up projections of a SwiGLU feed-forward and the product after them in one
 * launch (src/core/engine.cpp:509-512, 38-39): h[t, j] = silu(g) * u with
 * g = vec_dot_row(w_gate row j, qx row t) (+ bias_gate[j]), u likewise for w_up, silu(v) =
 * v / (1 + exp(-v)); both matrices have n_ff rows of in_dim, h is [n_rows][n_ff]. The same
 * values as cllm_hip_gemv_q8_multi_dev on the two matrices followed by cllm_hip_swiglu_q8_0_dev,
 * bit for bit. Biases may be null. */
int cllm_hip_gemv_q8_swiglu_dev(uint32_t type, int in_dim, int n_ff, const void* w_gate,
                                const void* w_up, const float* bias_gate, const float* bias_up,
                                int n_rows, const int8_t* qs, const float* scales,
                                const int32_t* bsums, float* h, void* stream);

/* The RMSNorm before the q, k and v projections and the projections in one launch, for one
 * activation row (decode): rms_norm_ptr(x, norm_w, eps) (src/core/engine.cpp:23-28, 475),
 * its Q8_0 quantization and cllm_hip_gemv_q8_multi_dev on it (476-478). x and norm_w are
 * in_dim fp32 values on the device, in_dim a multiple of 32 up to 4096. The outputs are
 * bit-identical to cllm_hip_rmsnorm_q8_0_dev followed by cllm_hip_gemv_q8_multi_dev. */
int cllm_hip_rmsnorm_gemv_multi_dev(uint32_t type, int in_dim, int n_mats, const void* const* w,
                                    const int* out_dims, const float* const* bias,
                                    float* const* y, const float* x, const float* norm_w,
                                    float eps, void* stream);

/* The RMSNorm before the feed-forward and cllm_hip_gemv_q8_swiglu_dev on its output in one
 * launch, for one activation row (src/core/engine.cpp:23-28, 508-512); same limits as
 * cllm_hip_rmsnorm_gemv_multi_dev, bit-identical to cllm_hip_rmsnorm_q8_0_dev followed by
 * cllm_hip_gemv_q8_swiglu_dev. */
int cllm_hip_rmsnorm_gemv_swiglu_dev(uint32_t type, int in_dim, int n_ff, const void* w_gate,
                                     const void* w_up, const float* bias_gate,
                                     const float* bias_up, const float* x, const float* norm_w,
                                     float eps, float* h, void* stream);

/* cllm_hip_gemv_q8_dev fused with the residual add that follows the matmul in the engine
 * (x += mm(...), src/core/engine.cpp:505-506, 512-513): y[t, j] += vec_dot_row(...)
 * (+ bias[j]), so y holds the residual stream on entry. Always the GEMV kernels (meant for
 * decode and small batches). */
int cllm_hip_gemv_q8_residual_dev(const void* w, uint32_t type, int in_dim, int out_dim,
                                  int n_rows, const int8_t* qs, const float* scales,
                                  const int32_t* bsums, const float* bias, float* y,
                                  void* stream);

/* cllm_hip_matmul_quant_dev followed by the residual add (x += mm(...),
 * src/core/engine.cpp:505-506, 512-513): y[t, j] += (row t of x . W row j) (+ bias[j]).
 * Small batches of the vec_dot types quantize their rows in the GEMV and add in its
 * epilogue (one launch); other shapes and types add a separate pass. */
int cllm_hip_matmul_quant_residual_dev(const float* x, const void* w, uint32_t type,
                                       const float* bias, int in_dim, int out_dim, int n_rows,
                                       float* y, void* stream);

/* matmul_quant_batch on device buffers. vec_dot types, small n_rows: one GEMV launch that
 * quantizes its activation rows itself; large n_rows: quantizes x into a library-owned
 * per-stream workspace, then runs the MFMA GEMM. Other types: the float-dot GEMV on x. */
int cllm_hip_matmul_quant_dev(const float* x, const void* w, uint32_t type, const float* bias,
                              int in_dim, int out_dim, int n_rows, float* y, void* stream);

/* cllm_hip_matmul_quant_dev for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. Same routes, kernels and results (bit for bit); the scratch the routes need
 * (quantized activations, the MFMA formats, split-K partial sums) is carved from a fixed
 * array of cllm_hip_static_scratch_bytes() (64 MiB) per GPU, held from library load to process
 * end, and nothing is allocated or freed (call cllm_hip_init first: it builds the per-device
 * state once). A batch whose scratch exceeds the array fails with CLLM_HIP_E_ARG (M = 512
 * rows of 14336 need ~27 MB; split larger batches). Every call on one GPU shares that GPU's
 * array, which keeps the last call's contents. Calls on one stream are ordered by it; a call
 * on another stream while the last eager call's work may still be running fails with
 * CLLM_HIP_E_BUSY instead of overwriting its scratch. Under graph capture nothing is checked:
 * replays of captured calls on different streams must be ordered by the caller. */
int cllm_hip_matmul_quant_static_dev(const float* x, const void* w, uint32_t type,
                                     const float* bias, int in_dim, int out_dim, int n_rows,
                                     float* y, void* stream);
size_t cllm_hip_static_scratch_bytes(void);
/* Device (and pinned host) allocations the library has made since it was loaded. No
 * reference counterpart: lets a caller check that cllm_hip_matmul_quant_static_dev
 * allocated nothing. */
uint64_t cllm_hip_allocation_count(void);

/* Reads `bytes` bytes at the device address p (16-byte aligned, bytes a multiple of 16) once,
 * by 16-byte nontemporal loads in a grid-stride loop over four 512-thread workgroups per CU,
 * and computes nothing from them: the one-launch HBM read ceiling of that stream, which a
 * GEMV over the same bytes is measured against. For benchmarks; no reference counterpart. */
int cllm_hip_read_stream_dev(const void* p, uint64_t bytes, void* stream);

/* ---- producers of a device-resident layer's activations (stream-ordered) -------------- */

/* RMSNorm of n_rows rows of n floats fused with the Q8_0 quantization matmul_quant applies
 * to its input: h = x * (1 / sqrt(sum(x^2) / n + eps)) * w (rms_norm_ptr,
 * src/core/engine.cpp:23-28), then quantize_row_q8_0(h) (src/core/quant.cpp:420-452) into
 * qs / scales / bsums (the layout of cllm_hip_quantize_q8_0_dev). h (fp32) may be null, or
 * qs, scales and bsums may all be null; n % 32 == 0 when they are given. The Q8_0 blocks are
 * exactly those of h; the sum of squares is reduced in parallel, so h can differ from the
 * reference's in the last bits. Feed qs/scales/bsums to cllm_hip_gemv_q8_dev. */
int cllm_hip_rmsnorm_q8_0_dev(const float* x, const float* w, float eps, int n, int n_rows,
                              float* h, int8_t* qs, float* scales, int32_t* bsums,
                              void* stream);

/* h = silu(gate) * up, silu(v) = v / (1 + exp(-v)) (src/core/engine.cpp:38, 511, 596),
 * over n_rows rows of n, fused with its Q8_0 quantization as above. */
int cllm_hip_swiglu_q8_0_dev(const float* gate, const float* up, int n, int n_rows, float* h,
                             int8_t* qs, float* scales, int32_t* bsums, void* stream);

/* x[i] += d[i], i < n: the residual adds (src/core/engine.cpp:506, 513, 587, 598). */
int cllm_hip_add_dev(float* x, const float* d, int64_t n, void* stream);

/* ---- the prefill linear layer, device-resident (stream-ordered) ------------------------
 * The reference's prefill quantizes each projection's input inside every matmul_quant_batch
 * call, the same rows once per matrix (q, k and v on h: src/core/engine.cpp:564-566; gate and
 * up on h2: 594-595; mm_batch, 276-285). Here a producer writes the Q8_0 blocks of an input
 * once, in the format the weight-row MFMA kernels read (act: the block scales, the codes as
 * exact fp16 and the K-quant minimum term's operand; cllm_hip_mfma_act_bytes bytes of device
 * memory, 16-byte aligned, in_dim a multiple of 256), and the matrices on that input run
 * from it, q/k/v or gate/up in one launch. The codes and scales are quantize_row_q8_0's,
 * bit for bit, of the producer's fp32 output. */
size_t cllm_hip_mfma_act_bytes(int in_dim, int n_rows);
/* Q8_0 of n_rows rows of x[n_rows][in_dim] into act. */
int cllm_hip_quantize_mfma_dev(const float* x, int in_dim, int n_rows, void* act, void* stream);
/* RMSNorm of each row (rms_norm_ptr, src/core/engine.cpp:23-28, 558-562, 590-592), as
 * cllm_hip_rmsnorm_q8_0_dev, into h (fp32, may be null) and act. */
int cllm_hip_rmsnorm_mfma_dev(const float* x, const float* norm_w, float eps, int in_dim,
                              int n_rows, float* h, void* act, void* stream);
/* h = silu(gate) * up (src/core/engine.cpp:596), as cllm_hip_swiglu_q8_0_dev, into h (fp32,
 * may be null) and act; n a multiple of 256. */
int cllm_hip_swiglu_mfma_dev(const float* gate, const float* up, int n, int n_rows, float* h,
                             void* act, void* stream);
/* matmul_quant_batch of n_mats matrices of one type (Q4_0/Q5_0/Q8_0/Q4_K/Q5_K/Q6_K) and
 * in_dim over the n_rows activation rows in act: y[i][n_rows][out_dims[i]] (+ bias[i], which
 * may be null, as may bias). Q4_K / Q5_K run up to 3 matrices in one weight-row launch; other
 * types, or more matrices, one launch per matrix. Split-K scratch comes from the library's
 * workspace of the stream. Replaces the mm_batch calls above (engine.cpp:276-285). */
int cllm_hip_matmul_mfma_dev(uint32_t type, int in_dim, int n_mats, const void* const* w,
                             const int* out_dims, const float* const* bias, float* const* y,
                             int n_rows, const void* act, void* stream);
/* The kernel instantiation, split and launch count cllm_hip_matmul_mfma_dev would run. */
const char* cllm_hip_matmul_mfma_plan(uint32_t type, int in_dim, int n_mats, const int* out_dims,
                                      int n_rows);

/* ---- float ops between the linear layers (stream-ordered) ----------------------------- */

/* Rows ids[0..n_ids) of a weight matrix of any GGML type (device pointers), dequantized
 * to fp32 out[n_ids][in_dim] bit for bit like dequantize_block (src/core/quant.cpp:
 * 371-389): the embedding lookup of get_embedding (src/core/engine.cpp:306-322). */
int cllm_hip_dequantize_rows_dev(const void* w, uint32_t type, int in_dim, const int32_t* ids,
                                 int n_ids, float* out, void* stream);

/* NEOX RoPE in place (apply_rope, src/core/engine.cpp:41-56): x holds n_rows rows of
 * n_heads x head_dim; row t sits at position pos0 + t; pair (i, i + head_dim / 2) of each
 * head turns by (pos0 + t) / theta_base^(i / (head_dim / 2)). */
int cllm_hip_rope_neox_dev(float* x, int n_rows, int n_heads, int head_dim, int pos0,
                           float theta_base, void* stream);

/* The same on the queries q (n_rows x n_head heads) and the keys k (n_rows x n_head_kv
 * heads, e.g. the cache rows just written) in one launch (engine.cpp:481-482). */
int cllm_hip_rope_neox2_dev(float* q, int n_head, float* k, int n_head_kv, int n_rows,
                            int head_dim, int pos0, float theta_base, void* stream);

/* Grouped-query attention (attention, src/core/engine.cpp:114-146): q holds n_rows rows of
 * n_head x head_dim; the caches hold n_head_kv x head_dim per position, positions
 * [0, pos0 + n_rows) filled; query row t sees positions [0, pos0 + t] (decode: n_rows = 1,
 * pos0 = the new token's position; prefill: engine.cpp:581-583). out: n_rows rows of
 * n_head x head_dim. head_dim 64, 128 or 256; n_head / n_head_kv at most 8. */
int cllm_hip_attention_dev(const float* q, const float* k_cache, const float* v_cache,
                           int n_rows, int pos0, int n_head, int n_head_kv, int head_dim,
                           float* out, void* stream);

/* The attention kernel cllm_hip_attention_dev would run for this shape: "k_attention_mfma<HD,
 * CT,W> workgroups=N" (many query rows) or "k_attention<HD> splits=S"; for tests and
 * benchmarks. No reference counterpart. */
const char* cllm_hip_attention_plan(int n_rows, int pos0, int n_head, int n_head_kv,
                                    int head_dim);

/* One decode step's RoPE and attention in one launch (engine.cpp:486-495): q holds one row of
 * n_head unrotated query heads, k_cache row pos0 the unrotated new key; both get the NEOX
 * rotation of cllm_hip_rope_neox2_dev at position pos0 (the queries in registers, q is not
 * written; the key row in place in k_cache), then the attention of cllm_hip_attention_dev over
 * the pos0 + 1 cached positions. The same output and key row as those two calls, bit for bit. */
int cllm_hip_attention_rope_dev(const float* q, float* k_cache, const float* v_cache, int pos0,
                                int n_head, int n_head_kv, int head_dim, float theta_base,
                                float* out, void* stream);

/* ---- GGUF files ------------------------------------------------------------------------ */

/* A GGUF file mapped read-only, parsed like GgufLoader::load (src/core/gguf.cpp:122-275):
 * version 2 or 3, the tensor table, the data section at the next multiple of 32 bytes after
 * the table, and the hyper-parameters under "<arch>." (falling back to "llama.").
 * Errors carry the reference's messages ("cannot open model file: ...", "invalid GGUF
 * magic", "unsupported GGUF version: N", "read_u32", ...). */
typedef struct cllm_hip_gguf cllm_hip_gguf;

/* ModelConfig (include/cllm/core/gguf.hpp:13-34), head_dim resolved, plus the file's layout. */
typedef struct {
    char arch[64];
    uint32_t n_layers, n_embd, n_head, n_head_kv, n_ctx, n_ff, vocab_size, head_dim;
    float rope_theta, norm_eps;
    uint32_t version;
    uint64_t data_offset, data_bytes;
} cllm_hip_model_config;

/* Opens and parses path. With upload != 0 the data section is copied to the current device
 * once (pinned, double-buffered) and registered like cllm_hip_register_weights, so host
 * tensor pointers of this file resolve to the device copy in every matmul call. Replaces
 * the engine's zero-copy mmap use (engine.cpp:182-199) for the GPU. */
int cllm_hip_gguf_open(const char* path, int upload, cllm_hip_gguf** out);
/* Unregisters and frees the device copy, unmaps the file. */
int cllm_hip_gguf_close(cllm_hip_gguf* g);
int cllm_hip_gguf_tensor_count(const cllm_hip_gguf* g);
/* Index of the tensor called name, -1 if none. */
int cllm_hip_gguf_find(const cllm_hip_gguf* g, const char* name);
/* Tensor i: name, GgmlType id, dims rows-first (up to 4, the file's order reversed like
 * Tensor::shape, gguf.cpp:163-165), offset in the data section, host address in the
 * mapping, device address (null without upload). Any output may be null. */
int cllm_hip_gguf_tensor(const cllm_hip_gguf* g, int i, const char** name, uint32_t* type,
                         int* n_dims, uint64_t* dims, uint64_t* offset, const void** host,
                         const void** dev);
int cllm_hip_gguf_config(const cllm_hip_gguf* g, cllm_hip_model_config* cfg);

/* Name of the kernel family cllm_hip_matmul_quant_dev would run for this shape: "gemv",
 * "small" (the small-batch int8 MFMA kernel) or "mfma" (vec_dot types), "fdot" (the float-dot
 * kernels of the other types), "none" (no GGML type); for tests and benchmarks. */
const char* cllm_hip_matmul_route(uint32_t type, int in_dim, int out_dim, int n_rows);

/* The kernel instantiation and launch plan cllm_hip_matmul_quant_dev would run for this shape,
 * e.g. "k_gemmw_q4k<8,1,2,Q5_K> splits=1" (MFMA route), "k_gemv_str<Q4_K,1> launches=1" (GEMV
 * route: kernel, activation rows per launch, launches), or the route name for the float-dot
 * route; for tests and benchmarks. No reference counterpart. */
const char* cllm_hip_matmul_plan(uint32_t type, int in_dim, int out_dim, int n_rows);

/* Process-wide kernel-choice overrides for tests and tuning sweeps; no reference counterpart.
 * The library itself never sets them, and nothing reads the environment. Knobs:
 *   "gemm_kernel"  values[0]: 0 the planner's MFMA kernel, 1 the int8 MFMA kernel, 2 the
 *                  activation-row fp16 MFMA kernel (from 16 rows, every vec_dot type)
 *   "gemm_tiles"   waves, weight tiles per wave, token tiles of the weight-row GEMM (a shape
 *                  it has compiled; 0, 0, 0 = the planner's)
 *   "gemm_splits"  K splits of the weight-row GEMM (0 = the planner's)
 *   "gemv_waves"   waves per SIMD of the one-deep and two-deep GEMV rings (0 = defaults)
 *   "gemv_kernel"  kernel of one-activation-row GEMVs: 0 the default, 1 the register ring,
 *                  2 the LDS-staged stream, 3 the one-item-in-flight stream
 *   "gemv_str_grid" workgroups of the one-item-in-flight stream (0 = one per CU)
 *   "gemm_small"   the small-batch kernel (Q4_K / Q5_K / Q8_0, up to 64 rows): 0 the default
 *                  rows, 1 every batch of 3 to 64 rows, 2 never (it is also off while
 *                  "gemm_kernel" forces a kernel)
 *   "gemm_small_plan" K splits (more than the planner's) and K parts per workgroup (1, 2, 4,
 *                  8 or 16) of the small-batch kernel (0, 0 = the planner's)
 *   "gemm_small_q8" fp32 batches on the small-batch kernel: 0 the default, 1 quantized once by
 *                  a separate launch, 2 quantized inside the kernel
 *   "gemv_fused_rows" batches of up to this many rows (1 to 8) on the streaming GEMV are
 *                  quantized inside its launch (0 = the default)
 *   "attention_kernel" 0 the default, 1 the sequence-split kernel, 2 the many-row MFMA kernel
 *                  (decode with fused RoPE always takes the split kernel)
 *   "gemv_fp_wgs"  one activation row of Q4_1 / Q5_1 / Q8_1 (float dot), rows of up to two
 *                  blocks per lane: 0 the default, 1 to 8 the pipelined row walk at that many
 *                  workgroups per CU, 9 the per-row kernel
 * Missing values count as 0, so n_values = 0 resets a knob. Takes effect on the next call. */
int cllm_hip_tune(const char* knob, const int* values, int n_values);

#ifdef __cplusplus
}
#endif
#endif
