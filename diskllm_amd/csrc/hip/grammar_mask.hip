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

/* diskllm_grammar_advance (src/core/grammar.c:248-256) as diskllm_sample_grammar
 * calls it after the draw (src/core/sampler_api.c:65-70): unless the token is
 * the EOS id, its string (up to its first NUL) is appended when buffer + string
 * stays below 8191 bytes; here the row's validator and balance states take
 * those bytes.  One thread per row. */
__global__ void grammar_advance_kernel(const uint32_t *__restrict__ off, const uint8_t *__restrict__ bytes, int V,
                                       dlk_grammar_row *states, const int32_t *__restrict__ tokens, int rows,
                                       int eos_id) {
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= rows) return;
    const int tok = tokens[row];
    if (tok < 0 || tok >= V || tok == eos_id) return;
    const uint32_t b0 = off[tok], b1 = off[tok + 1];
    uint32_t len = 0;
    while (b0 + len < b1 && bytes[b0 + len] != 0) len++;
    dlk_grammar_row st = states[row];
    if ((int64_t)st.bal.len + len >= DLK_GRAMMAR_BUF - 1) return;
    for (uint32_t i = 0; i < len; i++) {
        const uint8_t c = bytes[b0 + i];
        dlk_scan_step(&st.scan, c);
        dlk_balance_step(&st.bal, c);
    }
    states[row] = st;
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

extern "C" int dlk_grammar_advance(const uint32_t *off, const uint8_t *bytes, int vocab, dlk_grammar_row *states,
                                   const int32_t *tokens, int rows, int eos_id, hipStream_t stream) {
    using namespace dlk;
    if (!off || !bytes || !states || !tokens || vocab <= 0 || rows <= 0) return DLK_ERR_INVALID;
    hipLaunchKernelGGL(grammar_advance_kernel, dim3((rows + 63) / 64), dim3(64), 0, stream, off, bytes, vocab, states,
                       tokens, rows, eos_id);
    return hipGetLastError() == hipSuccess ? DLK_OK : DLK_ERR_HIP;
}

extern "C" int dlk_sample_grammar(const dlk_batch *b, int rows, int vocab, const dlk_sample_params *params,
                                  const uint32_t *off, const uint8_t *bytes, dlk_grammar_row *states, int eos_id,
                                  hipStream_t stream) {
    if (!b || !params || !b->mask || b->mask_row) return DLK_ERR_INVALID;
    /* the batch's mask buffer is written here, then read by the draw */
    int rc = dlk_grammar_mask(off, bytes, vocab, states, rows, eos_id, (uint32_t *)b->mask, b->mask_ld, nullptr, 0,
                              nullptr, stream);
    if (rc != DLK_OK) return rc;
    rc = dlk_sample(b, rows, vocab, params, stream);
    if (rc != DLK_OK) return rc;
    return dlk_grammar_advance(off, bytes, vocab, states, b->out_ids, rows, eos_id, stream);
}
