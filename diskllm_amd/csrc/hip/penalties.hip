/*
 * penalties.hip -- repetition / frequency / presence penalties in place on device
 * logits (src/sampler.c:21-52 and the frequency form of the batched path).
 * One workgroup per row; each distinct in-range history id is handled by the
 * thread of its first occurrence, which counts the occurrences and applies the
 * ops in order, so no two threads touch one logit.
 */
#include <hip/hip_runtime.h>

#include "../../../include/diskllm_amd.h"

namespace dlk {

constexpr int kPenThreads = 256;
constexpr int kPenLds = 16384;         /* history entries staged in LDS; longer ones are read from memory */

__device__ __forceinline__ float penalize_ops(float x, int cnt, uint32_t order, float rep, float freq, float pres) {
    for (int s = 0; s < 8; s++) {
        const uint32_t op = (order >> (4 * s)) & 0xFu;
        if (op == 0) break;
        if (op == DLK_OP_REPETITION) {
            if (rep > 1.0f)
                for (int k = 0; k < cnt; k++) x = x < 0.0f ? x * rep : x / rep;
        } else if (op == DLK_OP_FREQUENCY) {
            if (freq != 0.0f) { const float d = freq * (float)cnt; x = x - d; }
        } else if (op == DLK_OP_PRESENCE) {
            if (pres != 0.0f) x = x - pres;
        }
    }
    return x;
}

__global__ __launch_bounds__(kPenThreads) void penalties_kernel(float *logits, int64_t ld, int V,
                                                                const int32_t *hist_off, const int32_t *hist_ids,
                                                                uint32_t order, float rep, float freq, float pres) {
    __shared__ int32_t h[kPenLds];
    const int row = blockIdx.x;
    const int32_t *hr = hist_ids + hist_off[row];
    const int n = hist_off[row + 1] - hist_off[row];
    const bool staged = n <= kPenLds;
    if (staged)
        for (int i = threadIdx.x; i < n; i += kPenThreads) h[i] = hr[i];
    __syncthreads();
    const int32_t *hh = staged ? h : hr;
    float *lr = logits + (int64_t)row * ld;
    for (int i = threadIdx.x; i < n; i += kPenThreads) {
        const int32_t id = hh[i];
        if (id < 0 || id >= V) continue;
        bool first = true;
        for (int j = 0; j < i && first; j++) first = hh[j] != id;
        if (!first) continue;
        int cnt = 1;
        for (int j = i + 1; j < n; j++) cnt += hh[j] == id;
        lr[id] = penalize_ops(lr[id], cnt, order, rep, freq, pres);
    }
}

}  // namespace dlk

extern "C" int dlk_apply_penalties(float *logits, int64_t ld, int rows, int vocab, const int32_t *hist_off,
                                   const int32_t *hist_ids, uint32_t order, float rep, float freq, float pres,
                                   hipStream_t stream) {
    if (!logits || rows < 0 || vocab <= 0 || ld < vocab) return DLK_ERR_INVALID;
    if (rows == 0 || !hist_off) return DLK_OK;
    if (!hist_ids) return DLK_ERR_INVALID;
    hipLaunchKernelGGL(dlk::penalties_kernel, dim3(rows), dim3(dlk::kPenThreads), 0, stream, logits, ld, vocab,
                       hist_off, hist_ids, order, rep, freq, pres);
    return hipGetLastError() == hipSuccess ? DLK_OK : DLK_ERR_HIP;
}
