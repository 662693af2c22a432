/*
 * cllm_oracle.h -- CPU restatement of cllm_inference's quantized linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py may load this library, and only as the oracle. The product path
 * (libcllm_hip.so) never links, loads or calls it.
 *
 * Every function restates one piece of the reference (citations are path:line into the
 * reference tree):
 *   oracle_half_to_float        include/cllm/core/quant.hpp:31-56
 *   oracle_block_size/type_size src/core/quant.cpp:340-369
 *   oracle_dequantize           src/core/quant.cpp:28-336 (Q8_0 40-51, Q4_0 55-68,
 *                               Q4_K 82-108, Q5_0 113-132, Q6_K 135-161, Q5_K 302-336 and
 *                               the seven fallback types)
 *   oracle_dequantize_block     src/core/quant.cpp:371-389
 *   oracle_float_to_half        include/cllm/core/quant.hpp:58-87
 *   oracle_dequantize_block_f16 src/core/quant.cpp:398-407
 *   oracle_quantize_row_q8_0    src/core/quant.cpp:420-452
 *   oracle_vec_dot_row          src/core/quant.cpp:1359-1372 dispatching to the AVX2 forms
 *                               Q8_0 534-547, Q4_K 549-590, Q5_K 592-628, Q6_K 630-687,
 *                               Q4_0 757-777, Q5_0 863-893
 *   oracle_matmul_quant         src/core/quant.cpp:1374-1402 (vec_dot fast path only)
 *   oracle_matmul_quant_batch   src/core/quant.cpp:1433-1469 (vec_dot fast path only)
 *   thread chunking             src/core/thread_pool.cpp:44-89
 *
 * Pinning (what checks each function against something other than itself) is listed in
 * the header of oracle/cllm_oracle.c.
 */
#ifndef CLLM_ORACLE_H
#define CLLM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (include/cllm/core/quant.hpp:13-27). */
enum {
    ORACLE_F32 = 0, ORACLE_F16 = 1, ORACLE_Q4_0 = 2, ORACLE_Q4_1 = 3, ORACLE_Q5_0 = 6,
    ORACLE_Q5_1 = 7, ORACLE_Q8_0 = 8, ORACLE_Q8_1 = 9, ORACLE_Q2_K = 10, ORACLE_Q3_K = 11,
    ORACLE_Q4_K = 12, ORACLE_Q5_K = 13, ORACLE_Q6_K = 14
};

/* Return codes. */
enum { ORACLE_OK = 0, ORACLE_ERR_SHAPE = 1, ORACLE_ERR_TYPE = 2, ORACLE_ERR_SYS = 3 };

float oracle_half_to_float(uint16_t h);
int oracle_block_size(uint32_t type);
size_t oracle_type_size(uint32_t type);

/* Scalar dequantization of the thirteen types (the layout oracle); n % block_size == 0. */
int oracle_dequantize(const void* src, float* dst, uint32_t type, int64_t n);

/* dequantize_block (src/core/quant.cpp:371-389): any n, a partial last block read whole. */
int oracle_dequantize_block(const void* src, float* dst, uint32_t type, int64_t n);

/* float_to_half of the reference header (include/cllm/core/quant.hpp:58-87). */
uint16_t oracle_float_to_half(float f);

/* dequantize_block_f16 (src/core/quant.cpp:398-407). */
int oracle_dequantize_block_f16(const void* src, uint16_t* dst, uint32_t type, int64_t n);

/* fp32 -> Q8_0: qs[n], scales[n/32], bsums[n/32]. Bit-exact restatement. */
int oracle_quantize_row_q8_0(const float* x, int64_t n, int8_t* qs, float* scales,
                             int32_t* bsums);

int oracle_has_vec_dot(uint32_t type);

/* One weight row against one Q8_0 activation row of length n. */
int oracle_vec_dot_row(const void* w_row, uint32_t type, const int8_t* qs,
                       const float* scales, const int32_t* bsums, int64_t n, float* out);

/* y[out_dim] = x[in_dim] . W^T (+ bias). n_threads <= 1 runs serially; otherwise rows are
 * split the way ThreadPool::parallel_for splits them, when out_dim >= 256. */
int oracle_matmul_quant(const float* x, const void* w, uint32_t type, const float* bias,
                        int in_dim, int out_dim, float* y, int n_threads);

/* y[n_rows, out_dim] row-major. */
int oracle_matmul_quant_batch(const float* x, const void* w, uint32_t type,
                              const float* bias, int in_dim, int out_dim, int n_rows,
                              float* y, int n_threads);

/* Same blocks, same quantized activations, evaluated in fp64. Also returns abs_sum[t,j],
 * the sum of the absolute values of every per-block term (and |bias|), which the tests use
 * to floor the relative-error denominator of rows whose output nearly cancels. */
int oracle_matmul_quant_f64(const float* x, const void* w, uint32_t type, const float* bias,
                            int in_dim, int out_dim, int n_rows, double* y, double* abs_sum);

const char* oracle_last_error(void);

/* Producers of the linear layers' inputs in the reference engine (next to the path):
 *   oracle_rms_norm   src/core/engine.cpp:23-28 (rms_norm_ptr), row by row
 *   oracle_swiglu     src/core/engine.cpp:38 (silu) and 511 / 596 (gate * up) */
int oracle_rms_norm(const float* x, const float* w, int n, int rows, float eps, float* out);
int oracle_swiglu(const float* gate, const float* up, int64_t n, float* out);

#ifdef __cplusplus
}
#endif
#endif
