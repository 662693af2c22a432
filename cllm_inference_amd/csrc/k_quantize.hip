// k_quantize.hip -- fp32 -> Q8_0 activation quantization on gfx950.
//
// Restates quantize_row_q8_0 (src/core/quant.cpp:420-452) bit for bit (q8_scale,
// q8_inv_scale and q8_quant4 in device_utils.h hold the arithmetic); bsum is the sum of the
// block's q. amax is a max, so the order of the cross-lane reduction cannot change it.
//
// Mapping: the input is n_blocks contiguous 32-element blocks (M rows of K, K % 32 == 0, are
// exactly M*K/32 consecutive blocks). A DPP quad of lanes owns one block, eight elements each,
// loaded as two 16-byte vectors, and quantizes it with q8_quant_quad (the reductions over the
// quad are DPP moves, no LDS); a 256-thread workgroup quantizes 64 blocks.
#include "device_utils.h"
#include "launch.h"

namespace cllm_hip {

// Besides the Q8_0 row (qs, scales, bsums, any of which may be null), the MFMA paths ask for
// the quantized values as fp16 (qh, exact: |q| <= 128) and dx * bsum, the K-quant minimum
// term's activation factor, as fp32 (px) or split into bf16 parts per super-block (xq, see
// xq_store; its record of block blk is xq + 32 (blk / 8), rows of k % 256 == 0 elements).
__global__ __launch_bounds__(256) void k_quantize_q8_0(const float* __restrict__ x,
                                                       int64_t n_blocks,
                                                       int8_t* __restrict__ qs,
                                                       float* __restrict__ scales,
                                                       int32_t* __restrict__ bsums,
                                                       _Float16* __restrict__ qh,
                                                       float* __restrict__ px,
                                                       uint16_t* __restrict__ xq) {
    const int64_t gt = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = gt >> 2;
    const int part = (int)(gt & 3);
    if (blk >= n_blocks) return;  // whole quads leave together

    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4* src = (const f32x4*)(x + blk * 32 + part * 8);
    const f32x4 v0 = src[0], v1 = src[1];
    const float e[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    uint32_t q[2];
    float d;
    int s8;
    q8_quant_quad(e, q, d, s8);
    if (qs) *(u32x2*)(qs + blk * 32 + part * 8) = u32x2{q[0], q[1]};
    if (qh) {
        typedef _Float16 h8 __attribute__((ext_vector_type(8)));
        h8 hv;
#pragma unroll
        for (int j = 0; j < 8; ++j) hv[j] = (_Float16)(int8_t)((q[j >> 2] >> (8 * (j & 3))) & 0xFFu);
        *(h8*)(qh + blk * 32 + part * 8) = hv;
    }
    const int s16 = s8 + dpp_i32<DPP_QUAD_SWAP1>(s8);
    const int s = s16 + dpp_i32<DPP_QUAD_SWAP2>(s16);
    if (part == 0) {
        if (scales) scales[blk] = d;
        if (bsums) bsums[blk] = s;
        if (px) px[blk] = d * (float)s;
        if (xq) xq_store(xq + (blk >> 3) * 32, (int)(blk & 7), d * (float)s);
    }
}

// int8 qs / fp32 scales / int32 bsums (an already-quantized batch) -> the MFMA paths' fp16
// values and dx * bsum, and (scales_out, may be null) a copy of the scales.
__global__ __launch_bounds__(256) void k_q8_to_mfma(const int8_t* __restrict__ qs,
                                                    const float* __restrict__ scales,
                                                    const int32_t* __restrict__ bsums,
                                                    int64_t n_blocks, _Float16* __restrict__ qh,
                                                    float* __restrict__ px,
                                                    uint16_t* __restrict__ xq,
                                                    float* __restrict__ scales_out) {
    const int64_t gt = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = gt >> 3;
    const int part = (int)(gt & 7);
    if (blk >= n_blocks) return;
    const uint32_t packed = *(const uint32_t*)(qs + blk * 32 + part * 4);
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 hv = {(_Float16)(int8_t)(packed & 0xFF), (_Float16)(int8_t)(packed >> 8),
                   (_Float16)(int8_t)(packed >> 16), (_Float16)(int8_t)(packed >> 24)};
    *(h4*)(qh + blk * 32 + part * 4) = hv;
    if (part == 0) {
        const float pv = scales[blk] * (float)bsums[blk];
        if (scales_out) scales_out[blk] = scales[blk];
        if (px) px[blk] = pv;
        if (xq) xq_store(xq + (blk >> 3) * 32, (int)(blk & 7), pv);
    }
}

hipError_t launch_quantize_q8_0(const float* x, int64_t n_blocks, int8_t* qs, float* scales,
                                int32_t* bsums, hipStream_t stream) {
    if (n_blocks <= 0) return hipSuccess;
    const int64_t grid = (n_blocks * 4 + 255) / 256;
    hipLaunchKernelGGL(k_quantize_q8_0, dim3((unsigned)grid), dim3(256), 0, stream, x, n_blocks,
                       qs, scales, bsums, (_Float16*)nullptr, (float*)nullptr, (uint16_t*)nullptr);
    return hipGetLastError();
}

hipError_t launch_quantize_mfma(const float* x, int64_t n_blocks, float* scales,
                                _Float16* qh, float* px, hipStream_t stream) {
    if (n_blocks <= 0) return hipSuccess;
    const int64_t grid = (n_blocks * 4 + 255) / 256;
    hipLaunchKernelGGL(k_quantize_q8_0, dim3((unsigned)grid), dim3(256), 0, stream, x, n_blocks,
                       (int8_t*)nullptr, scales, (int32_t*)nullptr, qh, px, (uint16_t*)nullptr);
    return hipGetLastError();
}

hipError_t launch_q8_to_mfma(const int8_t* qs, const float* scales, const int32_t* bsums,
                             int64_t n_blocks, _Float16* qh, float* px, hipStream_t stream) {
    if (n_blocks <= 0) return hipSuccess;
    const int64_t grid = (n_blocks * 8 + 255) / 256;
    hipLaunchKernelGGL(k_q8_to_mfma, dim3((unsigned)grid), dim3(256), 0, stream, qs, scales,
                       bsums, n_blocks, qh, px, (uint16_t*)nullptr, (float*)nullptr);
    return hipGetLastError();
}

hipError_t launch_quantize_w(const float* x, int64_t n_blocks, float* scales, _Float16* qh,
                             uint16_t* xq, hipStream_t stream) {
    if (n_blocks <= 0) return hipSuccess;
    const int64_t grid = (n_blocks * 4 + 255) / 256;
    hipLaunchKernelGGL(k_quantize_q8_0, dim3((unsigned)grid), dim3(256), 0, stream, x, n_blocks,
                       (int8_t*)nullptr, scales, (int32_t*)nullptr, qh, (float*)nullptr, xq);
    return hipGetLastError();
}

hipError_t launch_q8_to_w(const int8_t* qs, const float* scales, const int32_t* bsums,
                          int64_t n_blocks, float* scales_out, _Float16* qh, uint16_t* xq,
                          hipStream_t stream) {
    if (n_blocks <= 0) return hipSuccess;
    const int64_t grid = (n_blocks * 8 + 255) / 256;
    hipLaunchKernelGGL(k_q8_to_mfma, dim3((unsigned)grid), dim3(256), 0, stream, qs, scales,
                       bsums, n_blocks, qh, (float*)nullptr, xq, scales_out);
    return hipGetLastError();
}

}  // namespace cllm_hip
