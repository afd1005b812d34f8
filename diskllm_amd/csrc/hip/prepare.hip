/*
 * prepare.hip -- the logits sampler_sample would see, written to a scratch
 * copy: the soft-cap (src/core/context.c:604-606, :873-876), then the grammar's
 * -INFINITY writes as a packed allow-mask (src/core/grammar.c:285-305), in the
 * reference's order.  dlk_sample runs this (and then the penalties in place on
 * the copy) for calls whose per-row state does not fit its fused kernels: a
 * history longer than the LDS staging.
 *
 * Elementwise, 8 bytes per element (read + write); grid (chunks, rows).
 */
#include <hip/hip_runtime.h>

#include "tanhf_glibc.h"
#include "../../../include/diskllm_amd.h"

namespace dlk {

constexpr int kPrepThreads = 256;
constexpr int kPrepPer = 4;              /* elements per thread */

__global__ __launch_bounds__(kPrepThreads) void prepare_rows_kernel(const float *__restrict__ src, int64_t ld,
                                                                    float *__restrict__ dst, int64_t dld, int V,
                                                                    const uint32_t *__restrict__ mask, int64_t mask_ld,
                                                                    const int32_t *__restrict__ mask_row, float cap) {
    const int row = blockIdx.y;
    const float *s = src + (int64_t)row * ld;
    float *d = dst + (int64_t)row * dld;
    const uint32_t *mk = nullptr;
    if (mask) mk = mask + (int64_t)(mask_row ? mask_row[row] : row) * mask_ld;
    const int base = blockIdx.x * kPrepThreads * kPrepPer + threadIdx.x;
#pragma unroll
    for (int k = 0; k < kPrepPer; k++) {
        const int i = base + k * kPrepThreads;
        if (i >= V) break;
        float x = s[i];
        if (cap > 0.0f) x = dlk_softcap_glibc(x, cap);
        if (mk && !((mk[i >> 5] >> (i & 31)) & 1u)) x = -INFINITY;
        d[i] = x;
    }
}

}  // namespace dlk

extern "C" int dlk_launch_prepare_rows(const float *src, int64_t ld, float *dst, int64_t dld, int rows, int vocab,
                                       const uint32_t *mask, int64_t mask_ld, const int32_t *mask_row, float cap,
                                       hipStream_t stream) {
    if (rows <= 0 || vocab <= 0 || rows > 65535) return -1;
    const int per = dlk::kPrepThreads * dlk::kPrepPer;
    const dim3 grid((unsigned)((vocab + per - 1) / per), (unsigned)rows);
    hipLaunchKernelGGL(dlk::prepare_rows_kernel, grid, dim3(dlk::kPrepThreads), 0, stream, src, ld, dst, dld, vocab,
                       mask, mask_ld, mask_row, cap);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
