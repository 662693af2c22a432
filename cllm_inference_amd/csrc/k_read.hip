// One-launch HBM read ceiling: the stream a decode GEMV reads, read once by the simplest
// pattern that came out fastest on MI355X for a cold 33 MB matrix (graph-timed, 17 rotated
// copies): a grid-stride loop of 16-byte nontemporal loads, four 512-thread workgroups per CU,
// one load in flight per lane per step. 6.08 us against 6.2-7.1 us for every other shape
// tried (two or four loads per step, eight per CU, every load of a workgroup's contiguous
// chunk issued up front, the Q4_K GEMV's own per-unit load pattern). A GEMV over the same
// bytes is measured against this figure.
#include <hip/hip_runtime.h>

#include "device_utils.h"
#include "launch.h"

namespace cllm_hip {

// The loaded words are folded into one value per lane that is stored only if it equals a
// constant (so the loads cannot be removed); it lands in g_read_sink then.
__device__ uint32_t g_read_sink[64];

__global__ __launch_bounds__(512) void k_read_stream(const u32x4* __restrict__ p, int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    uint32_t acc = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
        const u32x4 v = __builtin_nontemporal_load(p + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) g_read_sink[threadIdx.x & 63] = acc;
}

hipError_t launch_read_stream(const void* p, int64_t bytes, int cus, hipStream_t stream) {
    const int64_t n16 = bytes / 16;
    const int64_t grid = std::min<int64_t>(4ll * cus, (n16 + 511) / 512);
    hipLaunchKernelGGL(k_read_stream, dim3((unsigned)std::max<int64_t>(grid, 1)), dim3(512), 0,
                       stream, (const u32x4*)p, n16);
    return hipGetLastError();
}

}  // namespace cllm_hip
