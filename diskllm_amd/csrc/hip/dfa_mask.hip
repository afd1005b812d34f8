/*
 * dfa_mask.hip -- byte-DFA allow-masks across the vocabulary.
 *
 * No reference counterpart: the reference validates buffer+piece from scratch
 * for every token through the accept_str callback (src/core/grammar.c:284-306);
 * for a byte-level automaton the same per-token decision is a walk of the token's
 * bytes from the current state.
 *
 * Two kernels.  Automata of up to 64 states (dfa_walk_kernel): a wave's lanes
 * are the distinct start states of the rows (rows in one state share one mask,
 * so a batch of any size walks at most 64 of them) and the tokens are shared by
 * the wave, so every step of every lane reads the same row of a byte-major
 * table -- one LDS row of 68 bytes, no bank conflicts -- and the token's bytes
 * come from LDS as broadcast reads.  Larger automata (dfa_mask_kernel): one
 * thread per token walking it for every row of its row group.
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

/* ---- automata of up to 64 states ------------------------------------------
 *
 * LDS table tt[c * kWalkNsp + s], c = 0..255 a byte and c = 256 the end of a
 * token, s = 0..63 a state and s = kWalkAcc (64) "accepted":
 *   tt[c][s] = trans[s][c] for a byte (0 for s = 0 or an entry outside the table),
 *   tt[256][s] = kWalkAcc for a live s, 0 for s = 0,
 *   tt[c][kWalkAcc] = kWalkAcc.
 * So a walk is one lookup per entry of the token's entry list (its bytes, then
 * the end entry), both 0 and kWalkAcc absorb, and the token is allowed iff the
 * walk ends at kWalkAcc.  A state is still walking iff its low 6 bits are set.
 *
 * A block covers a range of mask words (32 tokens each) for every row.  The
 * rows' keys -- the start state if in [0, 64), else 0, which behaves as state 0
 * (dead, no EOS) -- are collected into a 64-bit set; key index k is the k-th
 * key of the set, and RW >= the number of keys.  The block stages its tokens'
 * entry lists in LDS as table offsets c * kWalkNsp, back to back, each
 * closed by the end entry (each entry held as a u32 together with the next,
 * so that a step of two entries is one LDS read), and the list start of every token (bit 31: not
 * walked -- empty, the EOS id, or past the vocabulary).  Lane l of a wave walks
 * key index l % RW for token slot l / RW (64 / RW slots), kWalkTpl tokens at
 * once (independent lookups in flight); the slots' bits are OR-ed across lanes
 * into one word per key, kept in LDS, and the block then writes every row's
 * words from its key's: a row's kWalkWpb words are one 64-byte line.
 * Walks of one group step together until no lane of the wave is walking: a
 * lane reads past its own end entry into the next lists or the padding of end
 * entries after the last (as long as the block's longest list), harmlessly,
 * since its state then absorbs.  A block whose lists exceed the staging
 * capacity reads the bytes from global memory instead. */
constexpr int kWalkThreads = 512;            /* one token per thread while staging */
constexpr int kWalkAcc = 64;
constexpr int kWalkNsp = 68;                   /* bytes per table row: 64 states, accepted, padding */
constexpr int kWalkTabBytes = ((257 * kWalkNsp) + 15) & ~15;
constexpr int kWalkTplMax = 8;                /* tokens walked at once per lane (at most) */
constexpr int kWalkWpb = kWalkThreads / 32;    /* mask words per block */
constexpr int kWalkRawPer = 16;                /* token bytes staged per thread (coalesced byte loads) */
constexpr int kWalkRawCap = kWalkRawPer * kWalkThreads;
constexpr int kWalkStageEntries = 10240;       /* entries staged per block (u32 pairs) */
constexpr uint32_t kWalkSkip = 0x80000000u;
constexpr size_t kWalkLds = kWalkTabBytes + kWalkWpb * 32 * 4 + kWalkRawCap + kWalkStageEntries * 4;

/* byte k of x if it is a state of the automaton, else 0 */
__device__ __forceinline__ uint32_t live_byte(uint32_t x, int k, uint32_t n_states) {
    const uint32_t v = (x >> (8 * k)) & 255u;
    return v < n_states ? v : 0u;
}

/* A row's key: its start state if in [0, 64) (a state at or above n_states is
 * dead but keeps its accept bit for the EOS rule), else 0. */
DLK_DEV int walk_key(int s) { return s >= 0 && s < 64 ? s : 0; }

template <int RW>
__global__ __launch_bounds__(kWalkThreads) void dfa_walk_kernel(const uint32_t *__restrict__ off,
                                                                const uint8_t *__restrict__ bytes, int V,
                                                                const uint8_t *__restrict__ trans, int n_states,
                                                                const int32_t *__restrict__ states, int n_rows,
                                                                int eos_id, uint64_t accept,
                                                                uint32_t *__restrict__ out, int64_t ld) {
    constexpr int P = 64 / RW;                 /* token slots per wave */
    constexpr int kWalkTpl = 32 / P < kWalkTplMax ? 32 / P : kWalkTplMax;   /* tokens per lane */
    constexpr int TPI = P * kWalkTpl;          /* tokens per wave iteration (divides 32) */
    static_assert(32 % TPI == 0, "an iteration's tokens lie in one mask word");
    extern __shared__ __align__(16) uint8_t sm[];
    __shared__ uint32_t s_maxlen, s_keys[2];
    __shared__ uint8_t s_key[64];                 /* the state of each key index */
    __shared__ uint32_t kb[kWalkWpb * 64];        /* [word][key index] */
    uint8_t *tt = sm;
    uint32_t *tpos = (uint32_t *)(sm + kWalkTabBytes);                     /* [kWalkWpb * 32] */
    uint8_t *raw = sm + kWalkTabBytes + kWalkWpb * 32 * 4;                 /* [kWalkRawCap] */
    uint32_t *ent = (uint32_t *)(raw + kWalkRawCap);                       /* [kWalkStageEntries] */
    const int t = threadIdx.x;
    const int W = (V + 31) >> 5;
    const int w0 = blockIdx.x * kWalkWpb, w1 = min(W, w0 + kWalkWpb);
    const int t0 = w0 * 32, t1 = min(V, w1 * 32);
    const uint32_t ns = (uint32_t)n_states;
    /* ---- every global load first: the table as 4x4 byte squares (states 4a..,
     *      bytes 4q..; two squares per thread, coalesced over q), the token's
     *      offsets, and the block's token bytes (coalesced bytes) ------------- */
    uint32_t sq[2][4];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int i = t + h * kWalkThreads, a = i >> 6, q = i & 63;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int st = 4 * a + k;
            sq[h][k] = (st > 0 && st < n_states) ? *(const uint32_t *)(trans + st * 256 + 4 * q) : 0u;
        }
    }
    const int tk = t0 + t;                     /* this thread's token (kWalkWpb * 32 == kWalkThreads) */
    uint32_t b0 = 0, len = 0;
    if (tk < t1) {
        b0 = off[tk];
        len = off[tk + 1] - b0;
    }
    const uint32_t B = off[t0];
    const uint32_t n_raw = off[t1] - B;
    uint32_t rb[kWalkRawPer];
#pragma unroll
    for (int m = 0; m < kWalkRawPer; m++) {
        const uint32_t i = (uint32_t)t + (uint32_t)m * kWalkThreads;
        rb[m] = i < n_raw ? bytes[B + i] : 0u;
    }
    const int st0 = t < n_rows ? states[t] : 0;     /* the first rows' start states, with the other loads */
    /* ---- LDS: the table byte-major, the bytes, the longest entry list -------- */
    if (t == 0) { s_maxlen = 0; s_keys[0] = 0u; s_keys[1] = 0u; }
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int i = t + h * kWalkThreads, a = i >> 6, q = i & 63;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const uint32_t x = live_byte(sq[h][0], m, ns) | (live_byte(sq[h][1], m, ns) << 8) |
                               (live_byte(sq[h][2], m, ns) << 16) | (live_byte(sq[h][3], m, ns) << 24);
            *(uint32_t *)(tt + (4 * q + m) * kWalkNsp + 4 * a) = x;
        }
    }
    if (t < 257) *(uint32_t *)(tt + t * kWalkNsp + kWalkAcc) = (uint32_t)kWalkAcc;   /* accepted absorbs */
    if (t < 16) {                                                                    /* the end row */
        uint32_t x = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int st = 4 * t + k;
            x |= (st > 0 && st < n_states ? (uint32_t)kWalkAcc : 0u) << (8 * k);
        }
        *(uint32_t *)(tt + 256 * kWalkNsp + 4 * t) = x;
    }
#pragma unroll
    for (int m = 0; m < kWalkRawPer; m++) {
        const uint32_t i = (uint32_t)t + (uint32_t)m * kWalkThreads;
        if (i < n_raw && i < (uint32_t)kWalkRawCap) raw[i] = (uint8_t)rb[m];
    }
    __syncthreads();
    /* the longest entry list and the rows' key set: reduced over each wave
     * first, then one LDS atomic per wave (512 lanes on one word serialise) */
    {
        uint32_t ml = tk < t1 ? len + 1 : 0u;
        uint64_t ks = 0;
        for (int r = t; r < n_rows; r += kWalkThreads) ks |= 1ull << walk_key(r == t ? st0 : states[r]);
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            ml = max(ml, (uint32_t)shfl_xor((int)ml, m));
            ks |= ((uint64_t)(uint32_t)shfl_xor((int)(uint32_t)(ks >> 32), m) << 32) |
                  (uint32_t)shfl_xor((int)(uint32_t)ks, m);
        }
        if ((t & 63) == 0) {
            atomicMax(&s_maxlen, ml);
            if ((uint32_t)ks) atomicOr(&s_keys[0], (uint32_t)ks);
            if ((uint32_t)(ks >> 32)) atomicOr(&s_keys[1], (uint32_t)(ks >> 32));
        }
    }
    __syncthreads();
    const uint64_t keys = ((uint64_t)s_keys[1] << 32) | s_keys[0];
    const int n_keys = __popcll(keys);
    if (t < 64 && ((keys >> t) & 1ull)) s_key[__popcll(keys & ((1ull << t) - 1ull))] = (uint8_t)t;
    /* ---- each token's entry list: its bytes as table rows, then the end row --- */
    const uint32_t n_ent = n_raw + (uint32_t)(t1 - t0);
    const uint32_t pad = s_maxlen;       /* a walk reads at most this far past a list start */
    const bool staged = n_raw <= (uint32_t)kWalkRawCap && (uint64_t)n_ent + pad <= (uint64_t)kWalkStageEntries;
    const uint32_t p0 = b0 - B + (uint32_t)t;
    /* each entry together with the next one (the end entry's partner is the
     * end entry again), so that a step of two entries is one LDS read */
    constexpr uint32_t kEnd = 256u * kWalkNsp;
    if (staged) {
        uint32_t cur = len > 0 ? (uint32_t)raw[b0 - B] * kWalkNsp : kEnd;
#pragma unroll 4
        for (uint32_t j = 0; j < len; j++) {
            const uint32_t nx = j + 1 < len ? (uint32_t)raw[b0 - B + j + 1] * kWalkNsp : kEnd;
            ent[p0 + j] = cur | (nx << 16);
            cur = nx;
        }
        if (tk < t1) ent[p0 + len] = kEnd | (kEnd << 16);
        for (uint32_t i = (uint32_t)t; i < pad; i += kWalkThreads) ent[n_ent + i] = kEnd | (kEnd << 16);
    }
    tpos[t] = (tk >= t1 || len == 0 || tk == eos_id) ? kWalkSkip : p0;
    __syncthreads();
    /* ---- the walks -------------------------------------------------------------- */
    const int lane = lane_id(), wv = t >> 6, slot = lane / RW, kx = lane % RW;
    const int s_row = kx < n_keys ? (int)s_key[kx] : 0;
    const uint32_t s_init = (s_row > 0 && s_row < n_states) ? (uint32_t)s_row : 0u;
    const bool eos_ok = s_row > 0 && s_row < 64 && ((accept >> s_row) & 1ull);
    for (int w = w0 + wv; w < w1; w += kWalkThreads / 64) {
        uint32_t bits = 0;
#pragma unroll 1
        for (int it = 0; it < 32; it += TPI) {
            const int tb = w * 32 + it + slot * kWalkTpl;          /* this lane's first token */
            uint32_t st[kWalkTpl], pos[kWalkTpl];
            /* the list starts of the lane's tokens, 16 bytes at a time (tb - t0
             * is a multiple of kWalkTpl, and kWalkTpl of 4) */
            static_assert(kWalkTpl % 4 == 0, "list starts read four at a time");
            uint32_t pps[kWalkTpl];
#pragma unroll
            for (int i = 0; i < kWalkTpl; i += 4) {
                const uint4 q4 = *(const uint4 *)&tpos[tb + i - t0];
                pps[i] = q4.x;
                pps[i + 1] = q4.y;
                pps[i + 2] = q4.z;
                pps[i + 3] = q4.w;
            }
#pragma unroll
            for (int i = 0; i < kWalkTpl; i++) {
                const uint32_t pp = pps[i];
                pos[i] = pp & ~kWalkSkip;
                st[i] = (pp & kWalkSkip) ? 0u : s_init;
            }
            if (staged) {
                /* two steps per check: a walk that has absorbed stays where it is */
                while (true) {
                    uint32_t act = 0;
#pragma unroll
                    for (int i = 0; i < kWalkTpl; i++) act |= st[i];
                    if (ballot((act & 63u) != 0u) == 0) break;
#pragma unroll
                    for (int i = 0; i < kWalkTpl; i++) {
                        const uint32_t pr = ent[pos[i]];
                        st[i] = tt[(pr >> 16) + tt[(pr & 0xffffu) + st[i]]];
                        pos[i] += 2;
                    }
                }
            } else {
                uint32_t tb0[kWalkTpl], tlen[kWalkTpl];
#pragma unroll
                for (int i = 0; i < kWalkTpl; i++) {
                    const int tq = tb + i;
                    tb0[i] = tq < t1 ? off[tq] : 0u;
                    tlen[i] = tq < t1 ? off[tq + 1] - tb0[i] : 0u;
                }
                for (uint32_t j = 0;; j++) {
                    uint32_t act = 0;
#pragma unroll
                    for (int i = 0; i < kWalkTpl; i++) act |= st[i];
                    if (ballot((act & 63u) != 0u) == 0) break;
#pragma unroll
                    for (int i = 0; i < kWalkTpl; i++) {
                        const uint32_t c = j < tlen[i] ? (uint32_t)bytes[tb0[i] + j] : (j == tlen[i] ? 256u : 0u);
                        const uint32_t nx = tt[c * kWalkNsp + st[i]];
                        st[i] = j <= tlen[i] ? nx : st[i];
                    }
                }
            }
            /* (the EOS id is not walked: its state is 0 here, its bit set below) */
            uint32_t nib = 0;
#pragma unroll
            for (int i = 0; i < kWalkTpl; i++) nib |= (st[i] == (uint32_t)kWalkAcc ? 1u : 0u) << i;
            bits |= nib << (it + slot * kWalkTpl);
        }
#pragma unroll
        for (int m = RW; m < 64; m <<= 1) bits |= (uint32_t)shfl_xor((int)bits, m);
        if (eos_id >= w * 32 && eos_id < w * 32 + 32 && eos_id < V && eos_ok) bits |= 1u << (eos_id & 31);
        if (slot == 0 && kx < n_keys) kb[(w - w0) * 64 + kx] = bits;
    }
    __syncthreads();
    /* every row's words from its key's: 16 lanes per row, one line each */
    const int nw = w1 - w0;
    for (int64_t i = t; i < (int64_t)n_rows * kWalkWpb; i += kWalkThreads) {
        const int r = (int)(i / kWalkWpb), j = (int)(i % kWalkWpb);
        if (j >= nw) continue;
        const int kr = walk_key(states[r]);
        out[(int64_t)r * ld + w0 + j] = kb[j * 64 + __popcll(keys & ((1ull << kr) - 1ull))];
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
    if (n_states <= 64) {
        /* the state-per-lane walk (dfa_walk_kernel): lanes for as many keys as
         * the rows can hold (at most 64) */
        const int W = (vocab + 31) / 32;
        const int RW = n_rows <= 8 ? 8 : n_rows <= 16 ? 16 : n_rows <= 32 ? 32 : 64;
        const dim3 grid((unsigned)((W + dlk::kWalkWpb - 1) / dlk::kWalkWpb));
        const size_t lds = dlk::kWalkLds;
        auto launch = [&](const void *fn) -> int {
            static int attr[4] = {0, 0, 0, 0};
            const int ai = RW == 8 ? 0 : RW == 16 ? 1 : RW == 32 ? 2 : 3;
            if (!attr[ai]) {
                if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
                    return DLK_ERR_HIP;
                attr[ai] = 1;
            }
            return DLK_OK;
        };
        int rc;
        switch (RW) {
        case 8:
            if ((rc = launch((const void *)dlk::dfa_walk_kernel<8>)) != DLK_OK) return rc;
            hipLaunchKernelGGL(dlk::dfa_walk_kernel<8>, grid, dim3(dlk::kWalkThreads), lds, stream, off, bytes, vocab,
                               trans, n_states, states, n_rows, eos_id, accept_mask, out_mask, mask_ld);
            break;
        case 16:
            if ((rc = launch((const void *)dlk::dfa_walk_kernel<16>)) != DLK_OK) return rc;
            hipLaunchKernelGGL(dlk::dfa_walk_kernel<16>, grid, dim3(dlk::kWalkThreads), lds, stream, off, bytes,
                               vocab, trans, n_states, states, n_rows, eos_id, accept_mask, out_mask, mask_ld);
            break;
        case 32:
            if ((rc = launch((const void *)dlk::dfa_walk_kernel<32>)) != DLK_OK) return rc;
            hipLaunchKernelGGL(dlk::dfa_walk_kernel<32>, grid, dim3(dlk::kWalkThreads), lds, stream, off, bytes,
                               vocab, trans, n_states, states, n_rows, eos_id, accept_mask, out_mask, mask_ld);
            break;
        default:
            if ((rc = launch((const void *)dlk::dfa_walk_kernel<64>)) != DLK_OK) return rc;
            hipLaunchKernelGGL(dlk::dfa_walk_kernel<64>, grid, dim3(dlk::kWalkThreads), lds, stream, off, bytes,
                               vocab, trans, n_states, states, n_rows, eos_id, accept_mask, out_mask, mask_ld);
            break;
        }
        return hipGetLastError() == hipSuccess ? DLK_OK : DLK_ERR_HIP;
    }
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
