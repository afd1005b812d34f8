/*
 * dfa_mask.hip -- byte-DFA allow-masks across the vocabulary.
 *
 * No reference counterpart: the reference validates buffer+piece from scratch
 * for every token through the accept_str callback (src/core/grammar.c:284-306);
 * for a byte-level automaton the same per-token decision is a walk of the token's
 * bytes from the current state.  The transition table (<= 64 KB) sits in LDS; one
 * thread walks one token for every row of its row group, and a wave ballot packs
 * 64 decisions into two mask words (bit t%32 of word t/32, 1 = allowed).
 */
#include "dlk_device.h"
#include "../../../include/diskllm_amd.h"

namespace dlk {

constexpr int kDfaRowsPerBlock = 16;

__global__ __launch_bounds__(256) void dfa_mask_kernel(const uint32_t *__restrict__ off,
                                                       const uint8_t *__restrict__ bytes, int V,
                                                       const uint8_t *__restrict__ trans, int n_states,
                                                       const int32_t *__restrict__ states, int n_rows, int eos_id,
                                                       uint64_t accept, uint32_t *__restrict__ out, int64_t ld) {
    extern __shared__ uint8_t tt[];
    const int n_tt = n_states * 256;
    for (int i = threadIdx.x * 4; i < n_tt; i += blockDim.x * 4) {
        *(uint32_t *)(tt + i) = *(const uint32_t *)(trans + i);
    }
    __syncthreads();
    const int tok = blockIdx.x * blockDim.x + threadIdx.x;
    const int lane = lane_id();
    const int W = (V + 31) >> 5;
    uint32_t b0 = 0, b1 = 0;
    if (tok < V) { b0 = off[tok]; b1 = off[tok + 1]; }
    const int r0 = blockIdx.y * kDfaRowsPerBlock;
    const int r1 = min(n_rows, r0 + kDfaRowsPerBlock);
    for (int r = r0; r < r1; r++) {
        const int s0 = states[r];
        bool ok = false;
        if (tok < V) {
            if (tok == eos_id) {
                ok = s0 > 0 && s0 < 64 && ((accept >> s0) & 1ull);
            } else {
                int s = s0;
                ok = s > 0 && s < n_states && b1 > b0;
                for (uint32_t j = b0; ok && j < b1; j++) {
                    s = tt[s * 256 + bytes[j]];
                    ok = s != 0 && s < n_states;
                }
            }
        }
        uint64_t bal = ballot(ok);
        const int wbase = (tok - lane) >> 5;          /* first word of this wave's 64 tokens */
        if (lane == 0 && wbase < W) out[(int64_t)r * ld + wbase] = (uint32_t)bal;
        if (lane == 32 && wbase + 1 < W) out[(int64_t)r * ld + wbase + 1] = (uint32_t)(bal >> 32);
    }
}

}  // namespace dlk

extern "C" int dlk_dfa_mask(const uint32_t *off, const uint8_t *bytes, int vocab, const uint8_t *trans,
                            int n_states, const int32_t *states, int n_rows, int eos_id, uint64_t accept_mask,
                            uint32_t *out_mask, int64_t mask_ld, hipStream_t stream) {
    if (!off || !bytes || !trans || !states || !out_mask || vocab <= 0 || n_rows <= 0) return DLK_ERR_INVALID;
    if (n_states <= 0 || n_states > 256) return DLK_ERR_UNSUPPORTED;
    if (mask_ld < (vocab + 31) / 32) return DLK_ERR_INVALID;
    if (((uintptr_t)trans & 3) != 0) return DLK_ERR_INVALID;
    dim3 grid((vocab + 255) / 256, (n_rows + dlk::kDfaRowsPerBlock - 1) / dlk::kDfaRowsPerBlock);
    hipLaunchKernelGGL(dlk::dfa_mask_kernel, grid, dim3(256), (size_t)n_states * 256, stream, off, bytes, vocab,
                       trans, n_states, states, n_rows, eos_id, accept_mask, out_mask, mask_ld);
    return hipGetLastError() == hipSuccess ? DLK_OK : DLK_ERR_HIP;
}
