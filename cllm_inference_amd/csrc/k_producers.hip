// k_producers.hip -- the producers of the linear layers' activations, fused with their Q8_0
// quantization, so a device-resident layer hands the GEMV its quantized rows directly.
//
// The reference engine computes, per token (src/core/engine.cpp):
//   RMSNorm   h = x * (1 / sqrt(sum(x^2) / n + eps)) * w        (rms_norm_ptr, 23-28)
//   SwiGLU    h = silu(gate) * up, silu(v) = v / (1 + exp(-v))  (38, 511, 596)
//   residual  x += tmp / x += down                              (506, 513, 587, 598)
// and every matmul_quant then quantizes h to Q8_0 (quant.cpp:1386-1387, 420-452). Here the
// producer writes h and its Q8_0 blocks in one pass.
//
// Arithmetic. Given the sum of squares, rms and h are bit-identical to the reference's
// (IEEE division and square root, h = (x * rms) * w with no contraction), and the Q8_0 blocks
// are exactly quantize_row_q8_0(h). The sum of squares is reduced in parallel, so it differs
// from the reference's sequential fp32 sum in the last bits (a relative 1e-7 or so); silu uses
// the device's expf (within 1 ulp). The quantized codes then agree except where a value sits
// at a rounding boundary.
#include "device_utils.h"
#include "launch.h"

namespace cllm_hip {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Where a producer writes the Q8_0 blocks of its output (any pointer may be null): the Q8_0
// row (codes qs, scales, bsums) and the weight-row MFMA kernels' format (the codes as exact
// fp16 qh, and the minimum term's operand xq, whose record of block blk is xq + 32 (blk / 8),
// rows of whole 256-element super-blocks).
struct Q8Out {
    int8_t* qs = nullptr;
    float* scales = nullptr;
    int32_t* bsums = nullptr;
    _Float16* qh = nullptr;
    uint16_t* xq = nullptr;
    __host__ __device__ bool any() const { return qs || qh; }
};

// Q8_0 of the 32-element block held by 8 consecutive lanes (4 elements each, lane part):
// writes the lane's 4 codes and, from part 0, the block's d and bsum.
__device__ __forceinline__ void quantize_block8(f32x4 v, int part, int64_t blk, const Q8Out& o) {
    float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
    const float d = q8_scale(amax);
    const float id = q8_inv_scale(d);
    int s;
    const uint32_t packed = q8_quant4(v.x, v.y, v.z, v.w, id, s);
    if (o.qs) *(uint32_t*)(o.qs + blk * 32 + part * 4) = packed;
    if (o.qh) {
        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
        const h4 hv = {(_Float16)(int8_t)(packed & 0xFF), (_Float16)(int8_t)(packed >> 8),
                       (_Float16)(int8_t)(packed >> 16), (_Float16)(int8_t)(packed >> 24)};
        *(h4*)(o.qh + blk * 32 + part * 4) = hv;
    }
    s += __shfl_xor(s, 1, 8);
    s += __shfl_xor(s, 2, 8);
    s += __shfl_xor(s, 4, 8);
    if (part == 0) {
        if (o.scales) o.scales[blk] = d;
        if (o.bsums) o.bsums[blk] = s;
        if (o.xq) xq_store(o.xq + (blk >> 3) * 32, (int)(blk & 7), d * (float)s);
    }
}

constexpr int kThreads = 256;

// One workgroup per row. Pass 1: sum of squares (fma per element, then a wave and a
// workgroup reduction). Pass 2: eight lanes per 32-element block form h and quantize it.
__global__ __launch_bounds__(kThreads) void k_rmsnorm_q8_0(const float* __restrict__ x,
                                                           const float* __restrict__ w,
                                                           float eps, int n,
                                                           float* __restrict__ h, Q8Out o) {
    __shared__ float part_sums[kThreads / 64];
    const int row = blockIdx.x;
    const float* xr = x + (size_t)row * n;
    float ss = 0.0f;
    if (n % 4 == 0) {
        for (int c = threadIdx.x; c < n / 4; c += kThreads) {
            const f32x4 v = *(const f32x4*)(xr + 4 * c);
            ss = __builtin_fmaf(v.x, v.x, ss);
            ss = __builtin_fmaf(v.y, v.y, ss);
            ss = __builtin_fmaf(v.z, v.z, ss);
            ss = __builtin_fmaf(v.w, v.w, ss);
        }
    } else {
        for (int i = threadIdx.x; i < n; i += kThreads) ss = __builtin_fmaf(xr[i], xr[i], ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) part_sums[threadIdx.x >> 6] = ss;
    __syncthreads();
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < kThreads / 64; ++i) sum += part_sums[i];
    // 1 / sqrt(sum / n + eps), each operation correctly rounded as in the reference
    const float rms = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(sum, (float)n) + eps));

    float* hr = h ? h + (size_t)row * n : nullptr;
    if (!o.any() || n % 32 != 0) {
        for (int i = threadIdx.x; i < n; i += kThreads)
            if (hr) hr[i] = __fmul_rn(__fmul_rn(xr[i], rms), w[i]);
        return;
    }
    const int nb = n / 32;
    const int part = threadIdx.x & 7;
    // whole 8-lane groups stay together through the loop (the shuffles need them)
    for (int b = threadIdx.x >> 3; b < ((nb + 31) / 32) * 32; b += kThreads / 8) {
        const int bb = b < nb ? b : nb - 1;
        const f32x4 xv = *(const f32x4*)(xr + bb * 32 + part * 4);
        const f32x4 wv = *(const f32x4*)(w + bb * 32 + part * 4);
        f32x4 hv;
        hv.x = __fmul_rn(__fmul_rn(xv.x, rms), wv.x);
        hv.y = __fmul_rn(__fmul_rn(xv.y, rms), wv.y);
        hv.z = __fmul_rn(__fmul_rn(xv.z, rms), wv.z);
        hv.w = __fmul_rn(__fmul_rn(xv.w, rms), wv.w);
        if (b < nb) {
            if (hr) *(f32x4*)(hr + b * 32 + part * 4) = hv;
            quantize_block8(hv, part, (int64_t)row * nb + b, o);
        }
    }
}

// The same with the row held in registers: 1024 threads, CPT 16-byte chunks per thread
// (n <= 4096 * CPT, n % 32 == 0), so the row is read once and no thread loops long.
// Chunk c = t + 1024 i of the row; the 8 consecutive lanes of a group share t / 8 and hold
// the 8 chunks of one 32-element block.
constexpr int kRegThreads = 1024;

template <int CPT>
__global__ __launch_bounds__(kRegThreads) void k_rmsnorm_q8_0_reg(const float* __restrict__ x,
                                                                  const float* __restrict__ w,
                                                                  float eps, int n,
                                                                  float* __restrict__ h, Q8Out o) {
    __shared__ float part_sums[kRegThreads / 64];
    const int row = blockIdx.x;
    const float* xr = x + (size_t)row * n;
    const int chunks = n / 4;
    f32x4 v[CPT], wv[CPT];
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = threadIdx.x + kRegThreads * i;
        // the weight row is loaded with x, so its latency hides behind the reduction
        wv[i] = c < chunks ? *(const f32x4*)(w + 4 * c) : f32x4{0.f, 0.f, 0.f, 0.f};
        v[i] = c < chunks ? *(const f32x4*)(xr + 4 * c) : f32x4{0.f, 0.f, 0.f, 0.f};
        ss = __builtin_fmaf(v[i].x, v[i].x, ss);
        ss = __builtin_fmaf(v[i].y, v[i].y, ss);
        ss = __builtin_fmaf(v[i].z, v[i].z, ss);
        ss = __builtin_fmaf(v[i].w, v[i].w, ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) part_sums[threadIdx.x >> 6] = ss;
    __syncthreads();
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < kRegThreads / 64; ++i) sum += part_sums[i];
    const float rms = __fdiv_rn(1.0f, __fsqrt_rn(__fdiv_rn(sum, (float)n) + eps));
    const int part = threadIdx.x & 7;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = threadIdx.x + kRegThreads * i;
        if (c >= chunks) break;  // whole 8-lane groups (chunks % 8 == 0)
        f32x4 hv;
        hv.x = __fmul_rn(__fmul_rn(v[i].x, rms), wv[i].x);
        hv.y = __fmul_rn(__fmul_rn(v[i].y, rms), wv[i].y);
        hv.z = __fmul_rn(__fmul_rn(v[i].z, rms), wv[i].z);
        hv.w = __fmul_rn(__fmul_rn(v[i].w, rms), wv[i].w);
        if (h) *(f32x4*)(h + (size_t)row * n + 4 * c) = hv;
        if (o.any()) quantize_block8(hv, part, (int64_t)row * (n / 32) + c / 8, o);
    }
}

// silu(g) * u over n_blocks 32-element blocks, eight lanes per block.
__global__ __launch_bounds__(kThreads) void k_swiglu_q8_0(const float* __restrict__ gate,
                                                          const float* __restrict__ up,
                                                          int64_t n_blocks,
                                                          float* __restrict__ h, Q8Out o) {
    const int64_t gt = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t blk = gt >> 3;
    const int part = (int)(gt & 7);
    if (blk >= n_blocks) return;  // whole 8-lane groups leave together
    const int64_t at = blk * 32 + part * 4;
    const f32x4 g = *(const f32x4*)(gate + at);
    const f32x4 u = *(const f32x4*)(up + at);
    f32x4 hv;
    hv.x = silu_mul(g.x, u.x);
    hv.y = silu_mul(g.y, u.y);
    hv.z = silu_mul(g.z, u.z);
    hv.w = silu_mul(g.w, u.w);
    if (h) *(f32x4*)(h + at) = hv;
    if (o.any()) quantize_block8(hv, part, blk, o);
}

// silu(g) * u for lengths that are not whole blocks (fp32 output only)
__global__ __launch_bounds__(kThreads) void k_swiglu_f32(const float* __restrict__ gate,
                                                         const float* __restrict__ up,
                                                         int64_t total, float* __restrict__ h) {
    const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i < total) h[i] = silu_mul(gate[i], up[i]);
}

// x += d (the residual adds), four elements per thread where aligned
__global__ __launch_bounds__(kThreads) void k_add(float* __restrict__ x, const float* __restrict__ d,
                                                  int64_t n) {
    const int64_t i = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * 4;
    if (i + 4 <= n) {
        f32x4 a = *(f32x4*)(x + i);
        const f32x4 b = *(const f32x4*)(d + i);
        a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
        *(f32x4*)(x + i) = a;
    } else {
        for (int64_t j = i; j < n; ++j) x[j] += d[j];
    }
}

}  // namespace

hipError_t launch_rmsnorm_q8_0(const float* x, const float* w, float eps, int n, int rows,
                               float* h, int8_t* qs, float* scales, int32_t* bsums,
                               hipStream_t stream, _Float16* qh, uint16_t* xq) {
    if (rows <= 0 || n <= 0) return hipSuccess;
    Q8Out o;
    o.qs = qs, o.scales = scales, o.bsums = bsums, o.qh = qh, o.xq = xq;
    if (n % 32 == 0 && n <= 4 * 4 * kRegThreads) {
        const int cpt = (n + 4 * kRegThreads - 1) / (4 * kRegThreads);
        if (cpt == 1)
            hipLaunchKernelGGL(k_rmsnorm_q8_0_reg<1>, dim3((unsigned)rows), dim3(kRegThreads), 0,
                               stream, x, w, eps, n, h, o);
        else if (cpt == 2)
            hipLaunchKernelGGL(k_rmsnorm_q8_0_reg<2>, dim3((unsigned)rows), dim3(kRegThreads), 0,
                               stream, x, w, eps, n, h, o);
        else
            hipLaunchKernelGGL(k_rmsnorm_q8_0_reg<4>, dim3((unsigned)rows), dim3(kRegThreads), 0,
                               stream, x, w, eps, n, h, o);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_rmsnorm_q8_0, dim3((unsigned)rows), dim3(kThreads), 0, stream, x, w, eps,
                       n, h, o);
    return hipGetLastError();
}

hipError_t launch_swiglu_q8_0(const float* gate, const float* up, int64_t total, float* h,
                              int8_t* qs, float* scales, int32_t* bsums, hipStream_t stream,
                              _Float16* qh, uint16_t* xq) {
    if (total <= 0) return hipSuccess;
    Q8Out o;
    o.qs = qs, o.scales = scales, o.bsums = bsums, o.qh = qh, o.xq = xq;
    if (!o.any() || total % 32 != 0) {
        hipLaunchKernelGGL(k_swiglu_f32, dim3((unsigned)((total + kThreads - 1) / kThreads)),
                           dim3(kThreads), 0, stream, gate, up, total, h);
        return hipGetLastError();
    }
    // one wave per workgroup: a decode row (14336 elements) then spreads over 224 CUs
    const int64_t n_blocks = total / 32;
    hipLaunchKernelGGL(k_swiglu_q8_0, dim3((unsigned)((n_blocks * 8 + 63) / 64)), dim3(64), 0,
                       stream, gate, up, n_blocks, h, o);
    return hipGetLastError();
}

hipError_t launch_add(float* x, const float* d, int64_t n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int64_t threads = (n + 3) / 4;
    hipLaunchKernelGGL(k_add, dim3((unsigned)((threads + kThreads - 1) / kThreads)), dim3(kThreads),
                       0, stream, x, d, n);
    return hipGetLastError();
}

}  // namespace cllm_hip
