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

constexpr int kDfaRegBytes = 16;          /* token bytes held in registers; longer tokens read the rest */
constexpr int kDfaStageWords = 16;        /* table words a thread loads at once while staging */

/* One thread per token; the rows in groups of R (R = 8 for up to 16 rows, 16
 * above: 13.2 against 15.3 us for 16 rows over 151,936 tokens, 39.7 against
 * 44.6 us for 64 rows over 262,144), gpb groups per block one after another
 * (grid.y: the blocks of groups).  A block stages the table and reads its
 * tokens' bytes once for all its groups, so the host gives a block as many
 * groups as keep the grid at about 1,024 blocks or more (64 rows over 262,144
 * tokens: all four groups in one block, 35.6 against 40.2 us).  The rows are
 * stepped together: at each byte position every row takes one table lookup
 * (independent of the other rows'), so a step is 16 LDS reads in flight rather
 * than one dependent chain per row.  The table is staged with state 0's row all
 * zeros and every entry outside the table mapped to 0, so a rejected walk stays
 * at 0 by itself; the walk ends when no row of any lane of the wave is alive. */
template <int R>
__global__ __launch_bounds__(256) void dfa_mask_kernel(const uint32_t *__restrict__ off,
                                                       const uint8_t *__restrict__ bytes, int V,
                                                       const uint8_t *__restrict__ trans, int n_states,
                                                       const int32_t *__restrict__ states, int n_rows, int gpb,
                                                       int eos_id, uint64_t accept, uint32_t *__restrict__ out,
                                                       int64_t ld) {
    extern __shared__ uint8_t tt[];
    const int n_tt = n_states * 256;
    const int tok = blockIdx.x * blockDim.x + threadIdx.x;
    const int lane = lane_id();
    const int W = (V + 31) >> 5;
    uint32_t b0 = 0, len = 0;
    if (tok < V) {
        b0 = off[tok];
        len = off[tok + 1] - b0;
    }
    /* the token's first bytes, every load issued at once (they land while the
     * table is staged) */
    uint32_t by[kDfaRegBytes];
#pragma unroll
    for (int j = 0; j < kDfaRegBytes; j++) by[j] = (uint32_t)j < len ? bytes[b0 + j] : 0u;
    /* the table: kDfaStageWords words per thread loaded before any is stored,
     * so one round trip stages up to 64 states */
    for (int i0 = threadIdx.x * 4; i0 < n_tt; i0 += blockDim.x * 4 * kDfaStageWords) {
        uint32_t w[kDfaStageWords];
#pragma unroll
        for (int u = 0; u < kDfaStageWords; u++) {
            const int i = i0 + u * (int)blockDim.x * 4;
            w[u] = i >= 256 && i < n_tt ? *(const uint32_t *)(trans + i) : 0u;
        }
#pragma unroll
        for (int u = 0; u < kDfaStageWords; u++) {
            const int i = i0 + u * (int)blockDim.x * 4;
            if (i >= n_tt) break;
            uint32_t x = w[u];
            if (n_states < 256)
                for (int k = 0; k < 4; k++)
                    if (((x >> (8 * k)) & 255u) >= (uint32_t)n_states) x &= ~(255u << (8 * k));
            *(uint32_t *)(tt + i) = x;
        }
    }
    const bool walk = tok < V && tok != eos_id && len > 0;
    /* steps every lane of the wave may need: the wave's longest token, up to kDfaRegBytes */
    uint32_t wl = len < (uint32_t)kDfaRegBytes ? len : (uint32_t)kDfaRegBytes;
    for (int m = 32; m >= 1; m >>= 1) wl = max(wl, (uint32_t)shfl_xor((int)wl, m));
    const int wbase = (tok - lane) >> 5;          /* first word of this wave's 64 tokens */
    __syncthreads();
    const int r_end = min(n_rows, (int)(blockIdx.y + 1) * gpb * R);
    for (int r0 = blockIdx.y * gpb * R; r0 < r_end; r0 += R) {
        const int nr = min(n_rows - r0, R);
        uint32_t st[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int s0 = r < nr ? states[r0 + r] : 0;
            st[r] = walk && s0 > 0 && s0 < n_states ? (uint32_t)s0 : 0u;
        }
#pragma unroll
        for (int j = 0; j < kDfaRegBytes; j++) {
            uint32_t any = 0;
#pragma unroll
            for (int r = 0; r < R; r++) any |= st[r];
            if ((uint32_t)j >= wl || !ballot(any != 0u && (uint32_t)j < len)) break;
            const bool act = (uint32_t)j < len;
#pragma unroll
            for (int r = 0; r < R; r++) {
                const uint32_t nx = tt[st[r] * 256u + by[j]];
                st[r] = act ? nx : st[r];
            }
        }
        for (uint32_t j = kDfaRegBytes; j < len; j++) {     /* the rest of a long token */
            const uint32_t b = bytes[b0 + j];
#pragma unroll
            for (int r = 0; r < R; r++) st[r] = tt[st[r] * 256u + b];
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            if (r >= nr) break;
            bool ok = st[r] != 0u;
            if (tok == eos_id) {
                const int s0 = states[r0 + r];
                ok = s0 > 0 && s0 < 64 && ((accept >> s0) & 1ull);
            }
            ok = ok && tok < V;
            const uint64_t bal = ballot(ok);
            if (lane == 0 && wbase < W) out[(int64_t)(r0 + r) * ld + wbase] = (uint32_t)bal;
            if (lane == 32 && wbase + 1 < W) out[(int64_t)(r0 + r) * ld + wbase + 1] = (uint32_t)(bal >> 32);
        }
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
    const int R = n_rows <= 16 ? 8 : 16;
    const int n_groups = (n_rows + R - 1) / R, tok_blocks = (vocab + 255) / 256;
    int gpb = (int)std::min<int64_t>(n_groups, std::max<int64_t>(1, (int64_t)tok_blocks * n_groups / 1024));
    dim3 grid(tok_blocks, (n_groups + gpb - 1) / gpb);
    if (R == 8)
        hipLaunchKernelGGL(dlk::dfa_mask_kernel<8>, grid, dim3(256), (size_t)n_states * 256, stream, off, bytes, vocab,
                           trans, n_states, states, n_rows, gpb, eos_id, accept_mask, out_mask, mask_ld);
    else
        hipLaunchKernelGGL(dlk::dfa_mask_kernel<16>, grid, dim3(256), (size_t)n_states * 256, stream, off, bytes,
                           vocab, trans, n_states, states, n_rows, gpb, eos_id, accept_mask, out_mask, mask_ld);
    return hipGetLastError() == hipSuccess ? DLK_OK : DLK_ERR_HIP;
}
