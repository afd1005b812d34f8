/*
 * expf_kernel.hip -- elementwise expf, bit-identical to the host libm expf the
 * reference's softmax calls (src/sampler.c:179); see expf_glibc.h.
 */
#include "dlk_device.h"
#include "../../../include/diskllm_amd.h"

namespace dlk {

__constant__ uint64_t kExpTabC[32] = DLK_EXP2_TAB_INIT;

__global__ __launch_bounds__(256) void expf_kernel(const float *__restrict__ x, float *__restrict__ y, int64_t n) {
    __shared__ uint64_t tab[32];
    if (threadIdx.x < 32) tab[threadIdx.x] = kExpTabC[threadIdx.x];
    __syncthreads();
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = dlk_expf_glibc(x[i], tab);
}

}  // namespace dlk

extern "C" int dlk_expf(const float *x, float *y, int64_t n, hipStream_t stream) {
    if (!x || !y || n < 0) return DLK_ERR_INVALID;
    if (n == 0) return DLK_OK;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(dlk::expf_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, x, y, n);
    return hipGetLastError() == hipSuccess ? DLK_OK : DLK_ERR_HIP;
}
