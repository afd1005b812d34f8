/*
 * softcap.hip -- the reference's logit soft-cap on the device, in place:
 * logits[i] = cap * tanhf(logits[i] / cap) over each row
 * (src/core/context.c:604-606 after a prefill, :873-876 after a decode step,
 * where it is a host loop over the vocabulary).  tanhf is bit-identical to the
 * host libm's (tanhf_glibc.h).
 *
 * HBM-bound elementwise work: 8 bytes per element (read + write).  Rows whose
 * stride and base allow it are processed as float4 (16-byte loads and stores);
 * a workgroup covers 4 * 256 * kSoftcapVec4 elements of one row.
 */
#include <hip/hip_runtime.h>

#include "tanhf_glibc.h"
#include "../../../include/diskllm_amd.h"

namespace dlk {

constexpr int kSoftcapThreads = 256;
constexpr int kSoftcapVec4 = 2;             /* float4 groups per thread */

__global__ __launch_bounds__(kSoftcapThreads) void softcap_vec_kernel(float *__restrict__ logits, int64_t ld,
                                                                      int vocab, float cap) {
    float *row = logits + (int64_t)blockIdx.y * ld;
    const int base = (blockIdx.x * kSoftcapVec4 * kSoftcapThreads + threadIdx.x) * 4;
    float4 v[kSoftcapVec4];
#pragma unroll
    for (int k = 0; k < kSoftcapVec4; k++) {
        const int i = base + k * kSoftcapThreads * 4;
        if (i + 3 < vocab) v[k] = *(const float4 *)(row + i);
    }
#pragma unroll
    for (int k = 0; k < kSoftcapVec4; k++) {
        const int i = base + k * kSoftcapThreads * 4;
        if (i + 3 < vocab) {
            float4 o;
            o.x = dlk_softcap_glibc(v[k].x, cap);
            o.y = dlk_softcap_glibc(v[k].y, cap);
            o.z = dlk_softcap_glibc(v[k].z, cap);
            o.w = dlk_softcap_glibc(v[k].w, cap);
            *(float4 *)(row + i) = o;
        } else {
            for (int c = 0; c < 4 && i + c < vocab; c++) row[i + c] = dlk_softcap_glibc(row[i + c], cap);
        }
    }
}

__global__ __launch_bounds__(kSoftcapThreads) void softcap_scalar_kernel(float *__restrict__ logits, int64_t ld,
                                                                         int vocab, float cap) {
    float *row = logits + (int64_t)blockIdx.y * ld;
    for (int i = blockIdx.x * kSoftcapThreads + threadIdx.x; i < vocab; i += gridDim.x * kSoftcapThreads)
        row[i] = dlk_softcap_glibc(row[i], cap);
}

}  // namespace dlk

extern "C" int dlk_softcap(float *logits, int64_t ld, int rows, int vocab, float cap, hipStream_t stream) {
    if (!logits || rows < 0 || vocab < 0 || ld < vocab) return DLK_ERR_INVALID;
    if (rows > 65535 || vocab > 0x7fffffff - 8192) return DLK_ERR_UNSUPPORTED;   /* grid rows; int indices */
    /* the reference caps only when the model's cap is positive (a NaN cap too is no cap) */
    if (rows == 0 || vocab == 0 || !(cap > 0.0f)) return DLK_OK;
    const bool vec = ld % 4 == 0 && ((uintptr_t)logits & 15u) == 0;
    if (vec) {
        const int per = 4 * dlk::kSoftcapVec4 * dlk::kSoftcapThreads;
        const dim3 grid((unsigned)((vocab + per - 1) / per), (unsigned)rows);
        hipLaunchKernelGGL(dlk::softcap_vec_kernel, grid, dim3(dlk::kSoftcapThreads), 0, stream, logits, ld, vocab,
                           cap);
    } else {
        int bx = (vocab + dlk::kSoftcapThreads - 1) / dlk::kSoftcapThreads;
        if (bx > 1024) bx = 1024;
        hipLaunchKernelGGL(dlk::softcap_scalar_kernel, dim3((unsigned)bx, (unsigned)rows),
                           dim3(dlk::kSoftcapThreads), 0, stream, logits, ld, vocab, cap);
    }
    return hipGetLastError() == hipSuccess ? DLK_OK : DLK_ERR_HIP;
}
