/*
 * grammar_mask.hip -- diskllm_grammar_apply_mask (src/core/grammar.c:275-308) for
 * a batch of sequences over one vocabulary: one thread per token resumes its
 * row's validator from the state after the buffer (grammar_scan.h) and feeds
 * the token's bytes, so a step costs O(V * token length) instead of the
 * reference's O(V * (buffer + token length)).
 */
#include <hip/hip_runtime.h>
#include <math.h>

#include "grammar_scan.h"

namespace dlk {

constexpr int kMaskThreads = 256;

__global__ void zero_i32(int32_t *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

/* grid (ceil(V / 256), rows); a wave covers 64 consecutive tokens = 2 mask words */
__global__ __launch_bounds__(kMaskThreads) void grammar_mask_kernel(const uint32_t *__restrict__ off,
                                                                    const uint8_t *__restrict__ bytes, int V,
                                                                    const dlk_grammar_row *__restrict__ states,
                                                                    int eos_id, uint32_t *mask, int64_t mask_ld,
                                                                    float *logits, int64_t ld, int32_t *valid) {
    const int row = blockIdx.y;
    const int t = blockIdx.x * kMaskThreads + threadIdx.x;
    const dlk_grammar_row st = states[row];
    bool ok = false;
    if (t < V) {
        if (t == eos_id) {
            ok = dlk_balance_finished(&st.bal) != 0;                     /* :285-291 */
        } else {
            const uint32_t b0 = off[t], b1 = off[t + 1];
            if (b1 > b0 && bytes[b0] != 0) {                             /* :294-298 */
                dlk_scan_state s = st.scan;
                uint32_t i = b0;
                for (; i < b1; i++) {
                    const uint8_t c = bytes[i];
                    if (c == 0) break;
                    dlk_scan_step(&s, c);
                    if (!dlk_scan_ok(&s)) break;
                }
                uint32_t len = i - b0;                                   /* strlen, unless rejected early */
                if (dlk_scan_ok(&s))
                    ok = (int64_t)st.bal.len + len < DLK_GRAMMAR_BUF - 1; /* :233 */
            }
        }
        if (!ok && logits) logits[(int64_t)row * ld + t] = -INFINITY;
    }
    const uint64_t bal = __ballot(ok);
    const int lane = threadIdx.x & 63;
    const int w0 = (blockIdx.x * kMaskThreads + (threadIdx.x & ~63)) >> 5;
    const int nw = (V + 31) >> 5;
    if (lane == 0 && w0 < nw) mask[(int64_t)row * mask_ld + w0] = (uint32_t)bal;
    if (lane == 32 && w0 + 1 < nw) mask[(int64_t)row * mask_ld + w0 + 1] = (uint32_t)(bal >> 32);
    if (valid && lane == 0 && bal) atomicAdd(&valid[row], (int32_t)__popcll(bal));
}

}  // namespace dlk

extern "C" int dlk_grammar_mask(const uint32_t *off, const uint8_t *bytes, int vocab, const dlk_grammar_row *states,
                                int rows, int eos_id, uint32_t *mask, int64_t mask_ld, float *logits, int64_t ld,
                                int32_t *valid, hipStream_t stream) {
    using namespace dlk;
    if (!off || !bytes || !states || !mask || vocab <= 0 || rows <= 0 || rows > 65535) return DLK_ERR_INVALID;
    if (mask_ld < (vocab + 31) / 32 || (logits && ld < vocab)) return DLK_ERR_INVALID;
    if (valid) hipLaunchKernelGGL(zero_i32, dim3((rows + 255) / 256), dim3(256), 0, stream, valid, rows);
    hipLaunchKernelGGL(grammar_mask_kernel, dim3((vocab + kMaskThreads - 1) / kMaskThreads, rows),
                       dim3(kMaskThreads), 0, stream, off, bytes, vocab, states, eos_id, mask, mask_ld, logits, ld,
                       valid);
    return hipGetLastError() == hipSuccess ? DLK_OK : DLK_ERR_HIP;
}
