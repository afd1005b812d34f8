/*
 * sampler_topk.hip -- single-pass top-k sampling path (top-k active or greedy).
 *
 * One row is split over G workgroups.  Each streams its contiguous slice once
 * into registers (128-bit loads), applies the allow-mask and the penalty patches
 * of the ids in its slice, and keeps its local candidates: the first K' = k + 16
 * elements under (prepared logit desc, index asc).  The last workgroup of the row
 * to finish (relaxed agent-scope atomics: no cache flushes, no spin waits) merges
 * the G candidate lists.  Because s = (l - M) * (1/T) is monotone in l but not
 * injective, the merge re-sorts on s and certifies that no unseen element of any
 * slice can tie the k-th s; rows it cannot certify (long runs of equal s) rerun
 * the exact selection over the whole row in the same workgroup.  The merged top-k
 * then goes through the exact softmax / top-p / draw pipeline.
 *
 * Reference: src/sampler.c:109-134 (top-k order), :136-234 (pipeline),
 * src/sampler.c:9-19 (greedy), src/core/sampler_api.c:51-61 (mask, penalties).
 */
#include "sampler_common.h"
#include "sampler_topk.h"

namespace dlk {

constexpr float kFltMax = 3.40282347e38f;

DLK_DEV uint32_t asc_key(float l) {          /* ascending orderable key, -0 == +0 */
    return ~desc_key(l);
}

DLK_DEV void pub32(uint32_t *a, uint32_t v) { __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DLK_DEV void pub64(uint64_t *a, uint64_t v) { __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DLK_DEV uint32_t get32(const uint32_t *a) {
    return __hip_atomic_load((uint32_t *)a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DLK_DEV uint64_t get64(const uint64_t *a) {
    return __hip_atomic_load((uint64_t *)a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

/* Penalised value of token id: mask first, then the ops in order; the
 * occurrence count is read from the whole history (src/sampler.c:21-52). */
DLK_DEV float penalised(const RowParams &p, float x, int cnt) {
    for (int s = 0; s < 8; s++) {
        uint32_t op = (p.order >> (4 * s)) & 0xFu;
        if (op == 0) break;
        if (op == DLK_OP_REPETITION) {
            if (p.rep > 1.0f)
                for (int k = 0; k < cnt; k++) x = x < 0.0f ? x * p.rep : x / p.rep;
        } else if (op == DLK_OP_FREQUENCY) {
            if (p.freq != 0.0f) {
                float d = p.freq * (float)cnt;
                x = x - d;
            }
        } else if (op == DLK_OP_PRESENCE) {
            if (p.pres != 0.0f) x = x - p.pres;
        }
    }
    return x;
}

/* Soft-cap (CAP): y = cap * tanhf(x / cap) is non-decreasing in x (tanhf is
 * non-decreasing from float to float: tests/native/tanhf_monotone_check.c), so a
 * slice is streamed and thresholded on its raw logits -- with +-inf clamped to
 * +-FLT_MAX, which the cap maps to the same +-cap -- and only the candidates it
 * collects are capped; the penalty patches are capped values, handled from
 * their LDS list.  Ties that the cap creates are resolved by the order
 * (y desc, index asc) of the collected candidates and the merge's certificate. */

/* Key of the r-th largest of the 128 ascending keys a, b held two per lane: the
 * largest K with at least r keys >= K, found bit by bit from ballots (no LDS, no
 * barrier).  Every lane returns it. */
DLK_DEV uint32_t wave_rth_key(uint32_t a, uint32_t b, int r) {
    uint32_t K = 0;
#pragma unroll
    for (int bit = 31; bit >= 0; bit--) {
        const uint32_t c = K | (1u << bit);
        const int n = __popcll(ballot(a >= c)) + __popcll(ballot(b >= c));
        if (n >= r) K = c;
    }
    return K;
}

/* The value of an ascending key from wave_rth_key, -inf for keys at or below -inf's. */
DLK_DEV float asc_value(uint32_t K) { return K > asc_key(-INFINITY) ? key_value(~K) : -INFINITY; }

/* x where bit c of `live` is set, else -inf (a bitfield extract and insert). */
DLK_DEV float live_or_ninf(float x, uint32_t live, int c) {
    const int m = (int)(live << (31 - c)) >> 31;
    return __int_as_float((__float_as_int(x) & m) | ((int)0xff800000 & ~m));
}

/* The 16-byte group of row elements i0 .. i0 + 3 (i0 a multiple of 4), -inf past s1. */
DLK_DEV float4 load_group(const float *lg, int i0, int s1) {
    if (i0 + 3 < s1) return *(const float4 *)(lg + i0);
    float4 x = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    if (i0 < s1) x.x = lg[i0];
    if (i0 + 1 < s1) x.y = lg[i0 + 1];
    if (i0 + 2 < s1) x.z = lg[i0 + 2];
    return x;
}

/* Bits of the group at i0 whose entries come from the stream: inside the slice,
 * allowed by the mask word bits `mw` (already shifted to i0), not penalised.  A
 * penalised id sets its group's bit in gbits; such groups look their ids up in
 * the slice's patch list (pid[0 .. np)). */
DLK_DEV uint32_t group_live(uint32_t mw, const uint32_t *gbits, const int *pid, int np, int i0, int s0, int s1) {
    uint32_t live = mw;
    if (i0 + 4 > s1) live &= i0 < s1 ? (1u << (s1 - i0)) - 1u : 0u;
    const int gr = (i0 - s0) >> 2;
    if ((gbits[gr >> 5] >> (gr & 31)) & 1u)
        for (int k = 0; k < np; k++) {
            const unsigned d = (unsigned)(pid[k] - i0);
            if (d < 4u) live &= ~(1u << d);
        }
    return live & 0xFu;
}

/* Whether id (inside the slice) is one of the penalised ids. */
DLK_DEV bool is_patched(const uint32_t *gbits, const int *pid, int np, int id, int s0) {
    const int gr = (id - s0) >> 2;
    if (!((gbits[gr >> 5] >> (gr & 31)) & 1u)) return false;
    for (int k = 0; k < np; k++)
        if (pid[k] == id) return true;
    return false;
}

/* Bits of the group at i0 allowed by the mask word bits `mw` and inside the slice. */
DLK_DEV uint32_t range_live(uint32_t mw, int i0, int s1) {
    uint32_t live = mw;
    if (i0 + 4 > s1) live &= i0 < s1 ? (1u << (s1 - i0)) - 1u : 0u;
    return live & 0xFu;
}

DLK_DEV int lanes_below(uint64_t bal) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
}

/* Of the n <= blockDim.x <= 256 entries of buf (sort keys: high word first),
 * moves those whose high word is at or below the r-th smallest high word (r <= n)
 * to the front and returns their count (r, plus any ties): the r-th high word
 * by a bitwise search on one wave, four keys a lane.  slot: two LDS words. */
DLK_DEV int keep_best(uint64_t *buf, int n, int r, int *slot) {
    const int t = threadIdx.x, lane = lane_id();
    const uint64_t mine = t < n ? buf[t] : ~0ull;
    if (wave_id() == 0) {
        uint32_t kk[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int i = lane + 64 * q;
            kk[q] = i < n ? (uint32_t)(buf[i] >> 32) : 0xffffffffu;
        }
        uint32_t K = 0;
        for (int bit = 31; bit >= 0; bit--) {
            const uint32_t c = K | (1u << bit);
            int cnt = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) cnt += (int)__popcll(ballot(kk[q] < c));
            if (cnt < r) K = c;
        }
        if (lane == 0) { slot[0] = (int)K; slot[1] = 0; }
    }
    __syncthreads();
    const uint32_t Ks = (uint32_t)slot[0];
    const bool keep = t < n && (uint32_t)(mine >> 32) <= Ks;
    const uint64_t bk = ballot(keep);
    int b2 = 0;
    if (lane == 0 && bk) b2 = atomicAdd(&slot[1], (int)__popcll(bk));
    b2 = shfl(b2, 0);
    if (keep) buf[b2 + lanes_below(bk)] = mine;
    __syncthreads();
    return slot[1];
}

/* The slice of a row that one workgroup streams: groups of four elements at
 * s0 + 4 * (t + j * T), j = 0 .. S/(4T) - 1, in batches of four groups per thread
 * with the next batch's loads in flight.
 *   - The penalised ids of the slice are patched from an LDS list (their stream
 *     entries count as -inf and the list is folded in afterwards).
 *   - Threshold: after batch 0 each wave takes the ceil(KP/4)-th largest of its
 *     lanes' two best group maxima (distinct entries, so the wave holds at least
 *     that many entries at or above it); the smallest of the four is a valid
 *     bound for the slice's KP-th largest entry.  Refreshed the same way after the
 *     last batch, from every batch's maxima.
 *   - Groups whose maximum reaches the threshold are listed in LDS; afterwards
 *     they are reloaded (from cache) and their entries at or above the final
 *     threshold become the candidates, of which the first KP under (value desc,
 *     index asc) are published.
 *   - Finite counts come from the mask bits; a non-finite raw logit anywhere in
 *     the slice sends it through an exact recount (NaN / +inf make the row
 *     irregular, -inf is not finite).
 * GREEDY keeps only the maximum and its lowest index. */
template <bool CAP, bool GREEDY>
__global__ __launch_bounds__(kTopkThreads, 8) void topk_kernel(TopkParams f) {
    extern __shared__ __align__(16) unsigned char smem[];
    const RowParams &p = f.p;
    /* With several blocks per CU, the later blocks on a CU stream behind the
     * earlier ones (older waves win issue and the memory queues): spread,
     * every row takes its slices from every dispatch slot, rather than the
     * rows of the last slot all finishing last */
    const int g = f.spread ? (int)blockIdx.y : (int)blockIdx.x;
    const int row = f.spread ? (int)blockIdx.x : (int)blockIdx.y;
    const int t = threadIdx.x, lane = lane_id(), w = wave_id();
    const int T = kTopkThreads, V = p.V, G = f.G;
    const int s0 = g * f.S, s1 = min(V, s0 + f.S);
    const float *lg = p.logits + (int64_t)row * p.ld;
    const uint32_t *mk = nullptr;
    if (p.mask) mk = p.mask + (int64_t)(p.mask_row ? p.mask_row[row] : row) * p.mask_ld;
    constexpr int kSpecial = CAP ? (1 | 2) : (1 | 2 | 4 | 512);     /* class bits: NaN (and -inf, +inf) */

    /* LDS: the row-kernel layout (for the in-workgroup fallback), a few words,
     * then one region the slice and the merge use in turn */
    Lds L = make_lds(smem, p.plan);
    unsigned char *q = L.region;
    int *misc = (int *)carve(q, 64 * 4);
    int *selh = (int *)carve(q, kSelWords * 4);                           /* radix-select histogram */
    uint32_t *sk = (uint32_t *)carve(q, (size_t)(3 * G + 2) * 4);          /* merge: per-slice words, tau */
    unsigned char *work = q;
    uint32_t *gbits = (uint32_t *)carve(q, (size_t)(f.S / 128) * 4);       /* slice: groups holding penalised ids */
    uint32_t *grp = (uint32_t *)carve(q, (size_t)f.grp_cap * 4);           /* slice: listed groups */
    float *gmx = (float *)carve(q, (size_t)f.grp_cap * 4);                 /* slice: their maxima */
    uint64_t *cbuf = (uint64_t *)carve(q, (size_t)f.cand_cap * 8);         /* slice: candidates */
    uint64_t *buf = (uint64_t *)work;                                       /* merge: f.buf_cap entries, then aggregates */
    if (t < 32) L.tab[t] = kExp2Tab[t];
    const uint64_t rng0 = p.greedy ? 0ull : p.rng[row];     /* read early: only the merge uses (and writes) it */

    auto gpos = [&](int b, int j) { return s0 + 4 * (t + (4 * b + j) * T); };
    float4 xa[4];
    uint32_t ma[4];
    /* A batch's loads: the mask words unshifted (the shift waits for the
     * load, and a wait here would keep one group in flight instead of the
     * batch); a batch wholly inside the slice without per-lane guards. */
    const int msh = (s0 + 4 * t) & 31;             /* bit of a group's first entry in its mask word */
    auto load_batch = [&](float4 (&x)[4], uint32_t (&m)[4], int b) {
        if (gpos(b, 0) - 4 * t + 16 * T <= s1) {
#pragma unroll
            for (int j = 0; j < 4; j++) x[j] = *(const float4 *)(lg + gpos(b, j));
#pragma unroll
            for (int j = 0; j < 4; j++) m[j] = mk ? mk[gpos(b, j) >> 5] : 0xffffffffu;
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int i0 = gpos(b, j);
                x[j] = load_group(lg, i0, s1);
                m[j] = (mk && i0 < s1) ? mk[i0 >> 5] : 0xffffffffu;
            }
        }
    };
    /* batch 0 first: in flight while the history is read (one register set:
     * the other resident waves keep loads in flight) */
    load_batch(xa, ma, 0);

    const int32_t *hist = nullptr;
    int nh = 0;
    if (p.hist_off) {
        hist = p.hist_ids + p.hist_off[row];
        nh = p.hist_off[row + 1] - p.hist_off[row];
    }
    if (DLK_COLD(nh > p.plan.hcap)) {
        if (g == 0 && t == 0) {
            p.out_ids[row] = -1;
            if (p.status) atomicOr(p.status, DLK_STATUS_HISTORY_TOO_LONG);
        }
        return;
    }
    int hid = t < nh ? hist[t] : -1;               /* the first T history ids, read early */
    /* and, for those inside the slice, their logit and mask word (in flight
     * during the stream) */
    float hval = 0.0f;
    uint32_t hmw = 0xffffffffu;
    if (hid >= s0 && hid < s1) {
        hval = lg[hid];
        if (mk) hmw = mk[hid >> 5];
    }
    for (int i = t; i < f.S / 128; i += T) gbits[i] = 0;
    if (t < 16) misc[t] = 0;                       /* (16.. are written before they are read) */

    /* penalty patches of the ids inside this slice: misc[0] entries of
     * (pid, pval), their groups' bits in gbits, misc[11] of them allowed by the
     * mask.  The slice's history entries are counted in an LDS hash table of
     * their ids (open addressing over 2 * hcap >= 2 * nh slots, so every id has
     * its slot and probes stay short); the entry that inserted an id computes
     * its patch once every count is in: the patch depends only on the id, its
     * count, its logit and its mask word, so any one occurrence may compute it.
     * Keys span hsort and pid, counts pval and pcnt (carved back to back, each
     * hcap words, a multiple of 16 bytes); pid and pval are reused for the
     * patch list only after the counts have been read. */
    int *hkey = (int *)L.hsort;
    int *hcnt = (int *)L.pval;
    const int hslots = 2 * p.plan.hcap;            /* a power of two */
    const int hshift = 32 - (31 - __clz(hslots));
    constexpr int kPer = kTopkHcapMax / kTopkThreads;   /* history entries per thread (nh <= hcap) */
    auto stage_history = [&]() {
        for (int i = t; i < hslots; i += T) { hkey[i] = -1; hcnt[i] = 0; }
        __syncthreads();
    };
    auto count_patches = [&]() {
        int oslot[kPer], oid[kPer];
        float ov[kPer];
        uint32_t om[kPer];
        /* the first T entries from registers (read early), the rest loaded here */
#pragma unroll
        for (int k = 0; k < kPer; k++) {
            const int i = t + k * T;
            oslot[k] = -1;
            oid[k] = -1;
            ov[k] = 0.0f;
            om[k] = 0xffffffffu;
            if (i >= nh) continue;
            const int id = k == 0 ? hid : hist[i];
            if (id < s0 || id >= s1) continue;
            oid[k] = id;
            if (k == 0) {
                ov[k] = hval;
                om[k] = hmw;
            } else {
                ov[k] = lg[id];
                om[k] = mk ? mk[id >> 5] : 0xffffffffu;
            }
            uint32_t h = ((uint32_t)id * 0x9E3779B1u) >> hshift;
            bool found = false;
            for (int probe = 0; probe < hslots && !found; probe++) {
                const int old = atomicCAS(&hkey[h], -1, id);
                if (old == -1) oslot[k] = (int)h;
                if (old == -1 || old == id) found = true;
                else h = (h + 1) & (uint32_t)(hslots - 1);
            }
            if (found) atomicAdd(&hcnt[h], 1);
        }
        __syncthreads();
        int cnt[kPer];
#pragma unroll
        for (int k = 0; k < kPer; k++) cnt[k] = oslot[k] >= 0 ? hcnt[oslot[k]] : 0;
        __syncthreads();                           /* counts read: pid and pval are free */
#pragma unroll
        for (int k = 0; k < kPer; k++) {
            if (oslot[k] < 0) continue;
            const int id = oid[k];
            float v = ov[k];
            const bool allowed = (om[k] >> (id & 31)) & 1u;
            if (CAP) v = dlk_softcap_glibc(v, p.cap);  /* the soft-cap first (src/core/context.c:873-876) */
            if (!allowed) v = -INFINITY;
            v = penalised(p, v, cnt[k]);
            const int at = atomicAdd(&misc[0], 1);
            if (at < p.plan.hcap) { L.pid[at] = id; L.pval[at] = v; }
            if (allowed) atomicAdd(&misc[11], 1);
            atomicOr(&gbits[(id - s0) >> 7], 1u << (((id - s0) >> 2) & 31));
        }
        __syncthreads();
    };
    if (GREEDY) {                                  /* greedy streams exact values */
        stage_history();
        count_patches();
    }
    int np = GREEDY ? min(misc[0], p.plan.hcap) : 0;

    /* ---- 2. stream the slice -------------------------------------------- */
    float m1 = -INFINITY, m2 = -INFINITY;          /* the lane's two best group maxima */
    int gi = -1;                                   /* GREEDY: first group holding m1 */
    int nfl = 0;                                   /* stream entries allowed by the mask */
    uint64_t spc = 0;                              /* ballot: a non-finite raw logit seen */
    float thr = -INFINITY;
    const int nb = f.S / (16 * T);                 /* batches of four groups per thread */
    auto batch = [&](const float4 (&x)[4], const uint32_t (&m)[4], int b) {
        float gm[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i0 = gpos(b, j);
            /* (non-greedy: the penalised ids stream their raw logits; the
             * patches come after the stream) */
            const uint32_t mw = m[j] >> msh;
            const uint32_t live = GREEDY ? group_live(mw, gbits, L.pid, np, i0, s0, s1) : range_live(mw, i0, s1);
            const float4 v = x[j];
            float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                if (!GREEDY) spc |= ballot(__builtin_amdgcn_class(e[c], kSpecial));
                float y = e[c];
                if (CAP) y = fminf(fmaxf(y, -kFltMax), kFltMax);   /* raw stand-in of cap(x) */
                e[c] = live_or_ninf(y, live, c);
            }
            gm[j] = fmaxf(fmaxf(e[0], e[1]), fmaxf(e[2], e[3]));
            if (GREEDY) {
                if (gm[j] > m1) { m1 = gm[j]; gi = i0; }
            } else {
                nfl += __popc(live);
                m2 = fmaxf(m2, fminf(m1, gm[j]));
                m1 = fmaxf(m1, gm[j]);
            }
        }
        if (!GREEDY) {
            /* the threshold after batches 0, 1, 3, 7, ...: every slot holds a
             * valid bound at all times (each only grows), so after the first
             * barrier a wave reads them as they are */
            if (((b + 1) & b) == 0) {
                const uint32_t K = wave_rth_key(asc_key(m1), asc_key(m2), (f.KP + 3) / 4);
                if (lane == 0) misc[16 + w] = (int)K;
                if (b == 0) __syncthreads();
                uint32_t Km = (uint32_t)misc[16];
                for (int u = 1; u < T / 64; u++) Km = min(Km, (uint32_t)misc[16 + u]);
                thr = asc_value(Km);
            }
            /* list the groups whose maximum reaches the threshold: one LDS
             * reservation per wave and batch */
            const float te = thr > -INFINITY ? thr : -kFltMax;
            uint64_t bal[4];
            int tot = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                bal[j] = ballot(gm[j] >= te);
                tot += (int)__popcll(bal[j]);
            }
            if (tot) {
                int base = 0;
                if (lane == 0) base = atomicAdd(&misc[1], tot);
                base = __builtin_amdgcn_readfirstlane(base);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int at = base + lanes_below(bal[j]);
                    if (gm[j] >= te && at < f.grp_cap) {
                        grp[at] = (uint32_t)gpos(b, j);
                        gmx[at] = gm[j];
                    }
                    base += (int)__popcll(bal[j]);
                }
            }
        }
    };
#pragma clang loop unroll(disable)
    for (int b = 0; b < nb; b++) {
        batch(xa, ma, b);
        if (b + 1 < nb) load_batch(xa, ma, b + 1);
    }

    /* several blocks per CU: a slice past its stream takes issue ahead of the
     * blocks still streaming (which wait on memory), so its tail runs sooner */
    if (f.spread) __builtin_amdgcn_s_setprio(2);
    float bm;
    int bi = 0x7fffffff, nf = 0, irr = 0, kept = 0, complete = 1;
    uint32_t last_key = 0, fnan = 0;
    if (GREEDY) {
        /* ---- 3g. slice maximum and its lowest index --------------------- */
        if (gi >= 0) {
            const float4 v = load_group(lg, gi, s1);
            const uint32_t mwg = mk ? mk[gi >> 5] >> (gi & 31) : 0xFu;
            const uint32_t live = group_live(mwg, gbits, L.pid, np, gi, s0, s1);
            const float e[4] = {v.x, v.y, v.z, v.w};
            for (int c = 3; c >= 0; c--)
                if (live_or_ninf(e[c], live, c) == m1) bi = gi + c;
        }
        bm = m1;
        for (int k2 = t; k2 < np; k2 += T) {
            const float y = L.pval[k2];
            const int id = L.pid[k2];
            /* (a row whose maximum is -inf samples index 0: no index is taken then) */
            if (y > bm || (y == bm && y > -INFINITY && id < bi)) { bm = y; bi = id; }
        }
        block_argmax(bm, bi, L);
        if (g == 0 && t == 0) {
            /* the reference compares from logits[0] (src/sampler.c:10-17): NaN there wins */
            float x0 = lg[0];
            if (mk && !(mk[0] & 1u)) x0 = -INFINITY;
            for (int k2 = 0; k2 < np; k2++)
                if (L.pid[k2] == 0) x0 = L.pval[k2];
            fnan = isnan(x0) ? 1u : 0u;
        }
    } else {
        /* ---- 3. patches, finite count; an exact pass when needed -------- */
        {
            /* the final threshold, from every batch (read after the patches' barriers) */
            const uint32_t K = wave_rth_key(asc_key(m1), asc_key(m2), (f.KP + 3) / 4);
            if (lane == 0) misc[16 + w] = (int)K;
        }
        int wn = nfl;
        for (int m = 32; m >= 1; m >>= 1) wn += shfl_xor(wn, m);
        if (lane == 0) {
            atomicAdd(&misc[3], wn);
            if (spc) misc[8] = 1;
        }
        stage_history();
        count_patches();
        np = min(misc[0], p.plan.hcap);
        float pmax = -INFINITY;
        int pn = 0, pirr = 0;
        for (int k2 = t; k2 < np; k2 += T) {       /* the patches: capped values under CAP */
            const float y = L.pval[k2];
            pn += y > -INFINITY;
            pirr |= !(y < INFINITY) && !(y == -INFINITY);
            pmax = fmaxf(pmax, y);
        }
        if (pn) atomicAdd(&misc[4], pn);
        if (pirr) misc[5] = 1;
        if (pmax > -INFINITY) atomicMax((unsigned *)&misc[7], asc_key(pmax));
        __syncthreads();
        nf = misc[3] - misc[11] + misc[4];         /* allowed stream entries, penalised ones replaced */
        {
            uint32_t Km = (uint32_t)misc[16];
            for (int u = 1; u < T / 64; u++) Km = min(Km, (uint32_t)misc[16 + u]);
            thr = asc_value(Km);
        }
        irr = misc[5];
        const float pmv = asc_value((uint32_t)misc[7]);
        /* the exact pass (at most once): every group of the slice with the
         * penalised ids left out -- finite count and irregular entries (under CAP
         * after the clamp), the stream maximum, and a valid threshold from the
         * exact group maxima */
        bool exact_done = false;
        float smax = -INFINITY, ethr = -INFINITY;
        auto exact_pass = [&]() {
            int c2 = 0, ir = 0;
            float e1 = -INFINITY, e2 = -INFINITY;
            for (int k2 = t; k2 < f.S / 4; k2 += T) {
                const int i0 = s0 + 4 * k2;
                const float4 v = load_group(lg, i0, s1);
                const uint32_t live =
                    group_live(mk && i0 < s1 ? mk[i0 >> 5] >> (i0 & 31) : 0xFu, gbits, L.pid, np, i0, s0, s1);
                const float e[4] = {v.x, v.y, v.z, v.w};
                float gmx = -INFINITY;
                for (int c = 0; c < 4; c++) {
                    if (!((live >> c) & 1u)) continue;
                    float y = e[c];
                    if (CAP && !(y != y)) y = fminf(fmaxf(y, -kFltMax), kFltMax);
                    c2 += y > -INFINITY;
                    ir |= !(y < INFINITY) && !(y == -INFINITY);
                    gmx = fmaxf(gmx, y);
                }
                e2 = fmaxf(e2, fminf(e1, gmx));
                e1 = fmaxf(e1, gmx);
            }
            float wmx = e1;
            for (int m = 32; m >= 1; m >>= 1) {
                c2 += shfl_xor(c2, m);
                ir |= shfl_xor(ir, m);
                wmx = fmaxf(wmx, shfl_xor(wmx, m));
            }
            const uint32_t K = wave_rth_key(asc_key(e1), asc_key(e2), (f.KP + 3) / 4);
            if (lane == 0) {
                atomicAdd(&misc[12], c2);
                if (ir) misc[13] = 1;
                atomicMax((unsigned *)&misc[14], asc_key(wmx));
                misc[16 + w] = (int)K;
            }
            __syncthreads();
            nf = misc[12] + misc[4];
            irr |= misc[13];
            smax = asc_value((uint32_t)misc[14]);
            uint32_t Km = (uint32_t)misc[16];
            for (int u = 1; u < T / 64; u++) Km = min(Km, (uint32_t)misc[16 + u]);
            ethr = asc_value(Km);
            exact_done = true;
        };
        if (DLK_COLD(misc[8])) exact_pass();
        /* ---- 4. candidates: the entries at or above the threshold -------- */
        bool all_groups = false, over = false;
        int C = 0;
        for (int attempt = 0; attempt < 2; attempt++) {
            const float te = thr > -INFINITY ? thr : -kFltMax;
            const float cte = !CAP ? te : thr > -INFINITY ? dlk_softcap_glibc(thr, p.cap) : -INFINITY;
            const int ng = misc[1];
            const int lim = all_groups ? f.S / 4 : min(ng, f.grp_cap);
            for (int k2 = t; k2 < lim; k2 += T) {
                /* (a listed group below the final threshold holds no candidate) */
                if (!all_groups && !(gmx[k2] >= te)) continue;
                const int i0 = all_groups ? s0 + 4 * k2 : (int)grp[k2];
                if (i0 >= s1) continue;
                const float4 v = load_group(lg, i0, s1);
                const uint32_t live = group_live(mk ? mk[i0 >> 5] >> (i0 & 31) : 0xFu, gbits, L.pid, np, i0, s0, s1);
                const float e[4] = {v.x, v.y, v.z, v.w};
                for (int c = 0; c < 4; c++) {
                    float y = e[c];
                    if (CAP) y = fminf(fmaxf(y, -kFltMax), kFltMax);
                    if (((live >> c) & 1u) && y >= te) {
                        const int at = atomicAdd(&misc[10], 1);
                        if (at < f.cand_cap) cbuf[at] = ((uint64_t)desc_key(y) << 32) | (uint32_t)(i0 + c);
                    }
                }
            }
            for (int k2 = t; k2 < np; k2 += T) {
                const float y = L.pval[k2];
                if (y > -INFINITY && y >= cte) {
                    const int at = atomicAdd(&misc[10], 1);
                    if (at < f.cand_cap) cbuf[at] = ((uint64_t)desc_key(y) << 32) | (uint32_t)L.pid[k2];
                }
            }
            __syncthreads();
            C = misc[10];
            over = (!all_groups && ng > f.grp_cap) || C > f.cand_cap;
            if (DLK_COLD(over && !exact_done)) exact_pass();  /* the row falls back: its maximum must be exact */
            if (DLK_HOT(over || C >= f.KP || C >= nf)) break;
            /* fewer than KP entries reach a threshold taken from raw logits
             * (penalties lowered some of them): the exact threshold, every group */
            if (!exact_done) exact_pass();
            thr = ethr;
            all_groups = true;
            if (t == 0) misc[10] = 0;
            __syncthreads();
        }
        bm = -INFINITY;
        if (exact_done) {
            bm = smax;
            if (CAP && bm > -INFINITY) bm = dlk_softcap_glibc(bm, p.cap);
            bm = fmaxf(bm, pmv);
        }
        if (over) {
            complete = -1;                         /* overflow: the merge falls back */
        } else if (C > 0) {
            if (CAP) {
                /* cap the streamed entries (the patches' values are capped already) */
                for (int i = t; i < C; i += T) {
                    const uint64_t e = cbuf[i];
                    const uint32_t id = (uint32_t)e;
                    if (!is_patched(gbits, L.pid, np, (int)id, s0)) {
                        const float y = dlk_softcap_glibc(key_value((uint32_t)(e >> 32)), p.cap);
                        cbuf[i] = ((uint64_t)desc_key(y) << 32) | id;
                    }
                }
                __syncthreads();
            }
            int n = C;
            /* only the KP best are sorted (KP, plus any ties at the KP-th key) */
            if (n > f.KP + 16 && n <= T) n = keep_best(cbuf, n, f.KP, &misc[20]);
            if (n <= T) {
                rank_sort_distinct(cbuf, n);
            } else {
                int P = 64;
                while (P < n) P <<= 1;
                for (int i = n + t; i < P; i += T) cbuf[i] = ~0ull;
                __syncthreads();
                bitonic_sort(cbuf, P);
            }
            /* every entry at or above the threshold is here, so the first is the
             * slice maximum */
            if (!exact_done) bm = key_value((uint32_t)(cbuf[0] >> 32));
            kept = min(f.KP, n);
            complete = kept == nf ? 1 : 0;
            last_key = (uint32_t)(cbuf[kept - 1] >> 32);
            uint64_t *cands = f.cands + ((int64_t)row * G + g) * f.KP;
            for (int j = t; j < kept; j += T) pub64(&cands[j], cbuf[j]);
        } else {
            complete = nf == 0 ? 1 : 0;
        }
    }
    TopkSlot *slot = f.slots + ((int64_t)row * G + g);
    /* ---- 5. publish and elect the merging workgroup --------------------- */
    if (t == 0) {
        pub32(&slot->max_bits, f2u(bm));
        pub32(&slot->argmax, (uint32_t)bi);
        pub32(&slot->nfin, (uint32_t)nf);
        pub32(&slot->kept, (uint32_t)kept);
        pub32(&slot->complete, (uint32_t)complete);
        pub32(&slot->last_key, last_key);
        pub32(&slot->first_nan, fnan | (irr ? 2u : 0u));
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t == 0) {
        uint32_t old = __hip_atomic_fetch_add(&f.counters[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        misc[2] = old == (uint32_t)(G - 1);
    }
    __syncthreads();
    if (!misc[2]) return;

    /* ===================== merge (last workgroup of the row) ============== */
    /* one round trip: every slice's words and every candidate slot (slot j of
     * slice h holds its (j+1)-th best entry when j < kept_h) */
    const int KP = f.KP, GK = G * KP;
    const uint64_t *crow = f.cands + (int64_t)row * GK;
    uint64_t cv[kMergePerThread];
#pragma unroll
    for (int u = 0; u < kMergePerThread; u++) {
        const int i = t + u * T;
        cv[u] = i < GK ? get64(&crow[i]) : ~0ull;
    }
    uint32_t *sw = (uint32_t *)selh;               /* max, argmax, nfin, first_nan per slice (G <= 64) */
    if (t < G) {
        /* every word loaded before any is stored (one round trip, not seven) */
        const TopkSlot *s = f.slots + ((int64_t)row * G + t);
        const uint32_t kept_h = get32(&s->kept), complete_h = get32(&s->complete), last_h = get32(&s->last_key);
        const uint32_t max_h = get32(&s->max_bits), arg_h = get32(&s->argmax), nfin_h = get32(&s->nfin);
        const uint32_t nan_h = get32(&s->first_nan);
        sk[3 * t + 0] = kept_h;
        sk[3 * t + 1] = complete_h;
        sk[3 * t + 2] = last_h;
        sw[t] = max_h;
        sw[64 + t] = arg_h;
        sw[128 + t] = nfin_h;
        sw[192 + t] = nan_h;
    }
    uint32_t *tau = sk + 3 * G, *tau2 = sk + 3 * G + 1;
    if (t == 0) { pub32(&f.counters[row], 0u); *tau = 0xffffffffu; *tau2 = 0u; misc[46] = 0; }
    __syncthreads();
    /* every wave reduces the slices itself (the argmax keeps the larger value,
     * ties to the lower index, as in order) */
    float M = -INFINITY;
    int amax = 0x7fffffff, NF = 0, total = 0, overflow = 0, first_nan = 0, irregular = 0;
    if (lane < G) {
        M = u2f(sw[lane]);
        amax = (int)sw[64 + lane];
        NF = (int)sw[128 + lane];
        first_nan = (int)(sw[192 + lane] & 1u);
        irregular = (int)(sw[192 + lane] & 2u);
        total = (int)sk[3 * lane];
        overflow = (int)sk[3 * lane + 1] == -1;
    }
    for (int m2 = 32; m2 >= 1; m2 >>= 1) {
        const float om = shfl_xor(M, m2);
        const int oa = shfl_xor(amax, m2);
        if (om > M || (om == M && oa < amax)) { M = om; amax = oa; }
        NF += shfl_xor(NF, m2);
        first_nan |= shfl_xor(first_nan, m2);
        irregular |= shfl_xor(irregular, m2);
        total += shfl_xor(total, m2);
        overflow |= shfl_xor(overflow, m2);
    }
    const int n_out = p.n_out;
    auto out_cands_empty = [&](float pr, float lpv, bool ids_idx, int kk) {
        for (int j = t; j < n_out; j += T) {
            int64_t o = (int64_t)row * n_out + j;
            if (p.out_cand_ids) p.out_cand_ids[o] = ids_idx ? (j < kk ? j : -1) : -1;
            if (p.out_cand_probs) p.out_cand_probs[o] = pr;
            if (p.out_cand_logprobs) p.out_cand_logprobs[o] = lpv;
        }
    };
    if (p.greedy) {
        if (t == 0) p.out_ids[row] = (first_nan || amax == 0x7fffffff) ? 0 : amax;
        out_cands_empty(0.0f, -INFINITY, false, 0);
        return;
    }
    uint64_t st = xorshift64(rng0);
    const float r = rand_f32_from(st);
    if (t == 0) p.rng[row] = st;
    const int k = p.top_k;
    if (DLK_COLD(irregular)) {
        /* NaN or +inf in the row: the reference's sequence on one thread */
        Row R;
        R.lg = lg; R.mk = mk; R.V = V; R.pid = L.pid; R.pval = L.pval; R.pflag = L.pflag;
        R.M = 0.0f; R.inv_t = p.inv_temp; R.maxv = 0.0f; R.tab = L.tab; R.cap = p.cap;
        R.np = build_patches(p, row, lg, mk, L, p.plan, V);
        if (t == 0) emulate_topk_row(p, R, k, r, buf, row);
        return;
    }
    if (DLK_COLD(NF == 0)) {                 /* every entry -inf (see sampler_row.hip) */
        if (t == 0) p.out_ids[row] = k - 1;
        out_cands_empty(NAN, NAN, true, k);
        return;
    }

    Row R;
    R.lg = lg; R.mk = mk; R.V = V; R.pid = L.pid; R.pval = L.pval; R.np = 0; R.pflag = L.pflag;
    R.M = M; R.inv_t = p.inv_temp; R.maxv = 0.0f; R.tab = L.tab; R.cap = p.cap;

    /* candidates re-keyed on s, the ones that can be in the top k gathered and
     * sorted (s desc, index asc) */
    bool ok = !overflow;
    if (ok) {
        /* bounds for the sort: list h is in logit order and s is monotone in
         * the logit, so at least k entries have s >= the s of any list's k-th
         * entry (tau), and when every list holds cq = ceil(k / G) entries, at
         * least G * cq >= k have s >= the smallest s among the lists' cq-th
         * entries (tau2); anything whose s is below the better bound is not in
         * the top k */
        const int cq = (k + G - 1) / G;
        const bool all_cq = __popcll(ballot(lane < G && (int)sk[3 * lane] >= cq)) == (unsigned)G;
        /* (list h, slot j) of entry i = t + u * T, stepped without a division;
         * tau and tau2 reduced in the wave first (one LDS atomic per wave) */
        const int qT = T / KP, rT = T - qT * KP;
        int h = t / KP, j = t - h * KP;
        uint32_t kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
        for (int u = 0; u < kMergePerThread; u++) {
            const int i = t + u * T;
            if (i < GK && j < (int)sk[3 * h]) {
                cv[u] = ((uint64_t)desc_key((key_value((uint32_t)(cv[u] >> 32)) - M) * R.inv_t) << 32) |
                        (cv[u] & 0xffffffffull);
                if (j == k - 1) kmin = min(kmin, (uint32_t)(cv[u] >> 32));
                if (j == cq - 1) kmax = max(kmax, (uint32_t)(cv[u] >> 32));
            } else {
                cv[u] = ~0ull;
            }
            h += qT;
            j += rT;
            if (j >= KP) { j -= KP; h++; }
        }
        kmin = wave_minmax_u32<true>(kmin);
        kmax = wave_minmax_u32<false>(kmax);
        if (lane == 0) {
            if (kmin != 0xffffffffu) atomicMin(tau, kmin);
            if (kmax != 0u) atomicMax(tau2, kmax);
        }
        __syncthreads();
        const uint32_t tk = all_cq ? min(*tau, *tau2) : *tau;
        /* the survivors to LDS: one reservation per wave */
        uint64_t balu[kMergePerThread];
        int tot = 0;
#pragma unroll
        for (int u = 0; u < kMergePerThread; u++) {
            balu[u] = ballot(cv[u] != ~0ull && (uint32_t)(cv[u] >> 32) <= tk);
            tot += (int)__popcll(balu[u]);
        }
        int base = 0;
        if (lane == 0 && tot) base = atomicAdd(&misc[46], tot);
        base = shfl(base, 0);
#pragma unroll
        for (int u = 0; u < kMergePerThread; u++) {
            const int at = base + lanes_below(balu[u]);
            if (((balu[u] >> lane) & 1ull) && at < f.buf_cap) buf[at] = cv[u];
            base += (int)__popcll(balu[u]);
        }
        __syncthreads();
        int nsort = misc[46];
        if (DLK_COLD(nsort > f.buf_cap)) {
            ok = false;
        } else {
            /* only the k best are sorted (k, plus any ties at the k-th s-key) */
            if (nsort > k + 16 && nsort <= T) nsort = keep_best(buf, nsort, k, &misc[48]);
            if (DLK_HOT(nsort <= T)) {
                rank_sort_distinct(buf, nsort);
            } else {
                int P = 64;
                while (P < nsort) P <<= 1;
                for (int i = nsort + t; i < P; i += T) buf[i] = ~0ull;
                __syncthreads();
                bitonic_sort(buf, P);
            }
            if (NF >= k) {
                /* certify: every slice that kept only part of its finite
                 * elements must have its last kept candidate strictly below
                 * the k-th s (one wave: G <= 64) */
                const uint32_t kth = (uint32_t)(buf[k - 1] >> 32);
                bool bad = false;
                if (lane < G && (int)sk[3 * lane + 1] != 1)
                    bad = !(desc_key((key_value(sk[3 * lane + 2]) - M) * R.inv_t) > kth);
                if (ballot(bad)) ok = false;
            } else {
                /* fewer finite entries than k: all of them plus the first k-NF
                 * entries that are -inf, in index order */
                if (total != NF) ok = false;
            }
        }
    }
    __syncthreads();
    if (DLK_COLD(!ok)) {
        /* exact selection over the whole row in this workgroup */
        int np_row = build_patches(p, row, lg, mk, L, p.plan, V);
        R.np = np_row;
        uint32_t *hist2 = (uint32_t *)(buf + p.plan.kp);
        select_top_k(R, k, buf, p.plan.kp, hist2, L);
    } else if (DLK_COLD(NF < k)) {
        /* append the first k-NF -inf entries in index order */
        int need = k - NF, found = 0;
        int np_row = build_patches(p, row, lg, mk, L, p.plan, V);
        R.np = np_row;
        for (int i0 = 0; i0 < V && found < need; i0 += T) {
            int i = i0 + t;
            bool ninf = i < V && !(prepared(R, i) > -INFINITY);
            uint64_t bal = ballot(ninf);
            if (lane == 0) misc[8 + w] = __popcll(bal);
            __syncthreads();
            int before = 0, tot = 0;
            for (int u = 0; u < n_waves(); u++) { if (u < w) before += misc[8 + u]; tot += misc[8 + u]; }
            int rank = found + before + __popcll(bal & ((1ull << lane) - 1));
            if (ninf && rank < need) buf[NF + rank] = ((uint64_t)desc_key(-INFINITY) << 32) | (uint32_t)i;
            __syncthreads();
            found += tot;
        }
        __syncthreads();
    }
    CandBase cb{&R, buf};
    R.maxv = cb.s(0);
    Scal S;
    int pos;
    if (DLK_HOT(k <= 64)) {
        /* a few candidates: one wave runs the reference's loops literally */
        if (w == 0) {
            pos = pipeline_small(p, cb, k, r, S);
            if (lane == 0) {
                misc[40] = pos;
                misc[41] = (int)f2u(S.inv); misc[42] = (int)f2u(S.inv2); misc[43] = (int)f2u(S.inv3);
                misc[44] = S.minp_all; misc[45] = S.cut;
            }
        }
        __syncthreads();
        pos = misc[40];
        S.inv = u2f((uint32_t)misc[41]); S.inv2 = u2f((uint32_t)misc[42]); S.inv3 = u2f((uint32_t)misc[43]);
        S.min_p = p.min_p; S.minp_on = p.minp_on; S.minp_all = misc[44]; S.topp_on = p.topp_on; S.cut = misc[45];
    } else {
        unsigned char *reg = (unsigned char *)(buf + f.buf_cap);
        pos = pipeline(p, cb, k, r, reg, L, S);
    }
    if (t == 0) p.out_ids[row] = cb.token(pos);
    for (int j = t; j < n_out; j += T) {
        int64_t o = (int64_t)row * n_out + j;
        if (j < k) {
            float pj = cb.e(j) * S.inv;
            QDraw<CandBase> qd{&cb, &S};
            float fj = qd(j);
            if (p.out_cand_ids) p.out_cand_ids[o] = cb.token(j);
            if (p.out_cand_probs) p.out_cand_probs[o] = pj;
            if (p.out_cand_logprobs) p.out_cand_logprobs[o] = fj > 0.0f ? (float)log((double)fj) : -INFINITY;
        } else {
            if (p.out_cand_ids) p.out_cand_ids[o] = -1;
            if (p.out_cand_probs) p.out_cand_probs[o] = 0.0f;
            if (p.out_cand_logprobs) p.out_cand_logprobs[o] = -INFINITY;
        }
    }
}

}  // namespace dlk

namespace {
template <bool CAP, bool GREEDY>
const void *topk_fn() {
    return (const void *)dlk::topk_kernel<CAP, GREEDY>;
}

const void *topk_kind(int kind) {
    return kind == 1 ? topk_fn<true, false>() : kind == 2 ? topk_fn<false, true>() : topk_fn<false, false>();
}
}  // namespace

/* Workgroups of the top-k kernel of this kind (0 plain, 1 soft-cap, 2 greedy)
 * resident per CU with `lds` bytes of dynamic LDS. */
extern "C" int dlk_topk_kernel_occupancy(int kind, size_t lds) {
    int n = 0;
    if (hipFuncSetAttribute(topk_kind(kind), hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess)
        return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, topk_kind(kind), dlk::kTopkThreads, lds) != hipSuccess)
        return 0;
    return n;
}

extern "C" int dlk_launch_topk_kernel(const dlk::TopkParams *f, int rows, size_t lds, hipStream_t stream) {
    using namespace dlk;
    static int set[3] = {0, 0, 0};
    const int cap = f->p.cap > 0.0f ? 1 : 0, greedy = f->p.greedy ? 1 : 0;
    if ((cap && greedy) || f->S % (16 * kTopkThreads) != 0) return -1;
    const int kind = cap ? 1 : greedy ? 2 : 0;
    const void *fn = topk_kind(kind);
    if (!set[kind]) {
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess) return -1;
        set[kind] = 1;
    }
    TopkParams fp = *f;
    void *args[] = {&fp};
    /* blocks are dispatched x-fastest: (rows, G) puts a row's slices a row-count apart */
    const dim3 grid = f->spread ? dim3(rows, f->G) : dim3(f->G, rows);
    if (hipLaunchKernel(fn, grid, dim3(kTopkThreads), args, lds, stream) != hipSuccess) return -1;
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
