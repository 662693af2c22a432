// k_quantize.hip -- fp32 -> Q8_0 activation quantization on gfx950.
//
// Restates quantize_row_q8_0 (src/core/quant.cpp:420-452) bit for bit:
//   amax = max |x| over the 32-element block
//   d    = amax / 127.0f          (IEEE division, correctly rounded)
//   id   = d != 0 ? 1.0f / d : 0  (IEEE division, correctly rounded)
//   q    = clamp(rint(x * id), -128, 127)   (rint = nearbyint in round-to-nearest-even)
//   bsum = sum of the block's q
// amax is a max, so the order of the cross-lane reduction cannot change it.
//
// Mapping: the input is n_blocks contiguous 32-element blocks (M rows of K, K % 32 == 0, are
// exactly M*K/32 consecutive blocks). Eight lanes own one block, four elements each, loaded as
// one 16-byte vector; a 256-thread workgroup quantizes 32 blocks.
#include "device_utils.h"
#include "launch.h"

namespace cllm_hip {

__global__ __launch_bounds__(256) void k_quantize_q8_0(const float* __restrict__ x,
                                                       int64_t n_blocks,
                                                       int8_t* __restrict__ qs,
                                                       float* __restrict__ scales,
                                                       int32_t* __restrict__ bsums) {
    const int64_t gt = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = gt >> 3;
    const int part = (int)(gt & 7);
    if (blk >= n_blocks) return;  // whole 8-lane groups leave together

    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4 v = *(const f32x4*)(x + blk * 32 + part * 4);

    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 8));

    const float d = __fdiv_rn(amax, 127.0f);
    const float id = (d != 0.0f) ? __fdiv_rn(1.0f, d) : 0.0f;

    int q[4];
    const float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float r = __builtin_rintf(__fmul_rn(e[i], id));
        // When amax is tiny enough that 1/d overflows, x * id is +-inf (or NaN for 0 * inf).
        // The reference's (int) conversion of such values is x86's cvttss2si result, INT_MIN,
        // which the clamp then turns into -128; v_cvt_i32_f32 would saturate instead.
        int t = (fabsf(r) < 2147483648.0f) ? (int)r : INT32_MIN;
        t = t > 127 ? 127 : t;
        t = t < -128 ? -128 : t;
        q[i] = t;
    }
    const uint32_t packed = (uint32_t)(q[0] & 0xFF) | ((uint32_t)(q[1] & 0xFF) << 8) |
                            ((uint32_t)(q[2] & 0xFF) << 16) | ((uint32_t)(q[3] & 0xFF) << 24);
    *(uint32_t*)(qs + blk * 32 + part * 4) = packed;

    int s = q[0] + q[1] + q[2] + q[3];
    s += __shfl_xor(s, 1, 8);
    s += __shfl_xor(s, 2, 8);
    s += __shfl_xor(s, 4, 8);
    if (part == 0) {
        scales[blk] = d;
        bsums[blk] = s;
    }
}

hipError_t launch_quantize_q8_0(const float* x, int64_t n_blocks, int8_t* qs, float* scales,
                                int32_t* bsums, hipStream_t stream) {
    if (n_blocks <= 0) return hipSuccess;
    const int64_t threads = n_blocks * 8;
    const int64_t grid = (threads + 255) / 256;
    hipLaunchKernelGGL(k_quantize_q8_0, dim3((unsigned)grid), dim3(256), 0, stream, x, n_blocks,
                       qs, scales, bsums);
    return hipGetLastError();
}

}  // namespace cllm_hip
