/*
 * sampler_common.h -- device code shared by the sampling kernels: the prepared
 * row view (mask + penalties), LDS carving, block helpers, penalty patches, the
 * exact top-k selection and the softmax / min-p / top-p / draw pipeline.
 *
 * Reference map:
 *   penalties          src/sampler.c:21-52 (+ builder frequency), order src/core/sampler_api.c:55-61
 *   packed mask        -INFINITY writes of src/core/grammar.c:285-305
 *   greedy             src/sampler.c:9-19, :140-142
 *   temperature / max  src/sampler.c:153-162
 *   top-k              src/sampler.c:109-134, :165-170 (first k under (value desc, index asc))
 *   softmax            src/sampler.c:172-185
 *   min-p              src/sampler.c:188-202
 *   top-p              src/sampler.c:205-222
 *   draw               src/sampler.c:225-233
 */
#ifndef DLK_SAMPLER_COMMON_H
#define DLK_SAMPLER_COMMON_H

#include <math.h>

#include "dlk_device.h"
#include "exact_scan.h"
#include "sampler_params.h"
#include "tanhf_glibc.h"

namespace dlk {

static __constant__ uint64_t kExp2Tab[32] = DLK_EXP2_TAB_INIT;

/* ------------------------------------------------------------------ row view */

struct Row {
    const float *lg;
    const uint32_t *mk;      /* packed allow-mask of this row or nullptr */
    int V;
    const int *pid;          /* sorted distinct penalised ids */
    const float *pval;       /* their penalised values (mask applied first) */
    int np;
    const uint32_t *pflag;   /* bit per 64-element chunk holding a penalised id */
    float M, inv_t, maxv;
    const uint64_t *tab;
    float cap;               /* > 0: the soft-cap, applied first */
};

/* The logit sampler_sample sees: soft-capped (src/core/context.c:873-876), then
 * the mask's -INFINITY (src/core/grammar.c:285-305), then the penalties. */
DLK_DEV float prepared_from(const Row &R, int i, float x) {    /* x: the raw logit R.lg[i] */
    if (R.cap > 0.0f) x = dlk_softcap_glibc(x, R.cap);
    if (R.mk && !((R.mk[i >> 5] >> (i & 31)) & 1u)) x = -INFINITY;
    if (R.np && ((R.pflag[i >> 11] >> ((i >> 6) & 31)) & 1u)) {
        int lo = 0, hi = R.np;
        while (lo < hi) {
            int mid = (lo + hi) >> 1;
            if (R.pid[mid] < i) lo = mid + 1;
            else hi = mid;
        }
        if (lo < R.np && R.pid[lo] == i) x = R.pval[lo];
    }
    return x;
}
DLK_DEV float prepared(const Row &R, int i) { return prepared_from(R, i, R.lg[i]); }

DLK_DEV float scaled(const Row &R, int i) { return (prepared(R, i) - R.M) * R.inv_t; }
DLK_DEV float expo(const Row &R, float s) { return dlk_expf_glibc(s - R.maxv, R.tab); }

/* --------------------------------------------------------------- LDS layout */

struct Lds {
    uint64_t *tab;      /* 32 */
    double *red;        /* 64 doubles of reduction scratch */
    double *bd;         /* 16 doubles: broadcast slots */
    int *bi;            /* 64 ints: broadcast slots */
    uint32_t *hsort;    /* hcap: history ids (sort buffer) */
    int *pid;           /* hcap */
    float *pval;        /* hcap */
    int *pcnt;          /* hcap */
    uint32_t *pflag;    /* flag words */
    unsigned char *region;
};

DLK_DEV unsigned char *carve(unsigned char *&p, size_t bytes) {
    unsigned char *r = p;
    p += (bytes + 15) & ~(size_t)15;
    return r;
}

DLK_DEV Lds make_lds(unsigned char *base, const LdsPlan &pl) {
    Lds L;
    unsigned char *p = base;
    L.tab = (uint64_t *)carve(p, 32 * 8);
    L.red = (double *)carve(p, 64 * 8);
    L.bd = (double *)carve(p, 16 * 8);
    L.bi = (int *)carve(p, 64 * 4);
    L.hsort = (uint32_t *)carve(p, (size_t)pl.hcap * 4);
    L.pid = (int *)carve(p, (size_t)pl.hcap * 4);
    L.pval = (float *)carve(p, (size_t)pl.hcap * 4);
    L.pcnt = (int *)carve(p, (size_t)pl.hcap * 4);
    L.pflag = (uint32_t *)carve(p, (size_t)pl.flag_words * 4);
    L.region = p;
    return L;
}

DLK_DEV Aggs make_aggs(unsigned char *p, int n) {
    const int nch = (n + 63) >> 6, ngr = (nch + 63) >> 6;
    Aggs A;
    A.a0 = (uint64_t *)carve(p, (size_t)nch * 8);
    A.a1 = (uint64_t *)carve(p, (size_t)nch * 8);
    A.bh = (int *)carve(p, (size_t)nch * 4);
    A.ga0 = (uint64_t *)carve(p, (size_t)ngr * 8);
    A.ga1 = (uint64_t *)carve(p, (size_t)ngr * 8);
    A.gbh = (int *)carve(p, (size_t)ngr * 4);
    A.P = (double *)carve(p, (size_t)(nch + 1) * 8);
    return A;
}

/* ------------------------------------------------------------ block helpers */

/* Bitonic sort (ascending) of n = power of two 64-bit keys in LDS. */
template <class K>
__device__ __forceinline__ void bitonic_sort(K *a, int n) {
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < n; i += blockDim.x) {
                int l = i ^ j;
                if (l > i) {
                    K x = a[i], y = a[l];
                    bool up = (i & k) == 0;
                    if ((x > y) == up) { a[i] = y; a[l] = x; }
                }
            }
            __syncthreads();
        }
    }
}

/* Ascending sort of n <= blockDim.x distinct 64-bit keys a[0..n) in LDS, by
 * rank: thread i counts the keys below a[i] (broadcast reads, no barrier per
 * step) and stores a[i] at that position.  Two barriers, where a bitonic network
 * over the next power of two takes one per pass.  Keys at and past n are not
 * touched. */
template <class K>
__device__ __forceinline__ void rank_sort_distinct(K *a, int n) {
    const int i = threadIdx.x;
    K key = K();
    int r = 0;
    if (i < n) {
        key = a[i];
#pragma unroll 8
        for (int j = 0; j < n; j++) r += a[j] < key ? 1 : 0;
    }
    __syncthreads();
    if (i < n) a[r] = key;
    __syncthreads();
}

/* The key of rank r (0-based, ascending) among the n 32-bit keys key(i),
 * i < n, 0 <= r < n: four rounds of 8-bit digits over an LDS histogram of 256
 * counters (hist) and two broadcast words (bc); a handful of barriers where a
 * bitonic sort of n keys takes log2(n)^2 / 2.  Every thread returns it. */
template <class KF>
__device__ __forceinline__ uint32_t block_select_u32(int n, int r, const KF &key, int *hist, int *bc) {
    const int T = blockDim.x, t = threadIdx.x, lane = lane_id();
    uint32_t prefix = 0;
#pragma unroll 1
    for (int round = 0; round < 4; round++) {
        const int shift = 24 - 8 * round;
        for (int i = t; i < 256; i += T) hist[i] = 0;
        __syncthreads();
        for (int i = t; i < n; i += T) {
            const uint32_t k = key(i);
            if (round == 0 || (k >> (shift + 8)) == prefix) atomicAdd(&hist[(k >> shift) & 255], 1);
        }
        __syncthreads();
        if (t < 64) {
            const int c0 = hist[4 * lane], c1 = hist[4 * lane + 1], c2 = hist[4 * lane + 2], c3 = hist[4 * lane + 3];
            const uint32_t sum4 = (uint32_t)(c0 + c1 + c2 + c3);
            const uint32_t incl = wave_scan_sat_u32(sum4, 0xffffffffu);
            const int excl = (int)(incl - sum4);
            if (excl <= r && r < (int)incl) {
                int rr = r - excl, d = 4 * lane;
                if (rr >= c0) {
                    rr -= c0; d++;
                    if (rr >= c1) {
                        rr -= c1; d++;
                        if (rr >= c2) { rr -= c2; d++; }
                    }
                }
                bc[0] = d;
                bc[1] = rr;
            }
        }
        __syncthreads();
        prefix = (prefix << 8) | (uint32_t)bc[0];
        r = bc[1];
    }
    return prefix;
}

/* Block reduce of (value, index): larger value wins, ties to the lower index;
 * NaN never wins (src/sampler.c:13 compares with '>'). */
__device__ __forceinline__ void block_argmax(float &v, int &i, Lds &L) {
    const int lane = lane_id(), w = wave_id();
    for (int m = 32; m >= 1; m >>= 1) {
        float ov = shfl_xor(v, m);
        int oi = shfl_xor(i, m);
        if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
    }
    float *rv = (float *)L.red;
    int *ri = (int *)(L.red + 32);
    if (lane == 0) { rv[w] = v; ri[w] = i; }
    __syncthreads();
    if (w == 0) {
        int nw = n_waves();
        v = lane < nw ? rv[lane] : -INFINITY;
        i = lane < nw ? ri[lane] : 0x7fffffff;
        for (int m = 32; m >= 1; m >>= 1) {
            float ov = shfl_xor(v, m);
            int oi = shfl_xor(i, m);
            if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }
        }
        if (lane == 0) { rv[0] = v; ri[0] = i; }
    }
    __syncthreads();
    v = rv[0];
    i = ri[0];
    __syncthreads();
}

__device__ __forceinline__ int block_sum_int(int v, Lds &L) {
    const int lane = lane_id(), w = wave_id();
    for (int m = 32; m >= 1; m >>= 1) v += shfl_xor(v, m);
    int *r = (int *)L.red;
    if (lane == 0) r[w] = v;
    __syncthreads();
    int s = 0;
    for (int k = 0; k < n_waves(); k++) s += r[k];
    __syncthreads();
    return s;
}

/* ----------------------------------------------------- penalties (patches) */

/* Deduplicate the row's history and compute each distinct id's penalised value:
 * the mask first (grammar runs before the penalties, src/core/sampler_api.c:51-61),
 * then the ops in `order`; repetition is applied once per occurrence
 * (src/sampler.c:23-31), presence and frequency once per distinct id. */
/* Penalties of one logit whose id occurs `cnt` times in the history, in the
 * configured order (src/sampler.c:19-63 and the builder's frequency/presence
 * pass): repetition divides positive / multiplies negative logits once per
 * occurrence; frequency subtracts freq * count; presence subtracts pres once. */
DLK_DEV float penalize(float x, int cnt, const RowParams &p) {
    for (int s = 0; s < 8; s++) {
        uint32_t op = (p.order >> (4 * s)) & 0xFu;
        if (op == 0) break;
        if (op == DLK_OP_REPETITION) {
            if (p.rep > 1.0f)
                for (int k = 0; k < cnt; k++) x = x < 0.0f ? x * p.rep : x / p.rep;
        } else if (op == DLK_OP_FREQUENCY) {
            if (p.freq != 0.0f) { float d = p.freq * (float)cnt; x = x - d; }
        } else if (op == DLK_OP_PRESENCE) {
            if (p.pres != 0.0f) x = x - p.pres;
        }
    }
    return x;
}

__device__ __forceinline__ int build_patches(const RowParams &p, int row, const float *lg, const uint32_t *mk, Lds &L,
                             const LdsPlan &pl, int V) {
    const int t = threadIdx.x, T = blockDim.x;
    int np = 0;
    for (int w = t; w < pl.flag_words; w += T) L.pflag[w] = 0;
    if (!p.hist_off) return 0;
    const int h0 = p.hist_off[row], h1 = p.hist_off[row + 1];
    const int nh = h1 - h0;
    if (nh <= 0) { __syncthreads(); return 0; }
    for (int i = t; i < pl.hcap; i += T) {
        uint32_t v = 0xffffffffu;
        if (i < nh) {
            int id = p.hist_ids[h0 + i];
            if (id >= 0 && id < V) v = (uint32_t)id;
        }
        L.hsort[i] = v;
    }
    __syncthreads();
    bitonic_sort(L.hsort, pl.hcap);
    /* run lengths at run starts */
    for (int i = t; i < pl.hcap; i += T) {
        uint32_t v = L.hsort[i];
        int c = 0;
        if (v != 0xffffffffu && (i == 0 || L.hsort[i - 1] != v)) {
            int j = i;
            while (j < pl.hcap && L.hsort[j] == v) j++;
            c = j - i;
        }
        L.pcnt[i] = c;
    }
    __syncthreads();
    if (wave_id() == 0) {
        const int lane = lane_id();
        int base = 0;
        for (int i0 = 0; i0 < pl.hcap; i0 += 64) {
            int i = i0 + lane;
            int c = L.pcnt[i];
            uint32_t v = L.hsort[i];
            uint64_t bal = ballot(c > 0);
            int at = base + __popcll(bal & ((1ull << lane) - 1));
            if (c > 0) { L.pid[at] = (int)v; L.pval[at] = (float)c; }
            base += __popcll(bal);
        }
        if (lane == 0) L.bi[0] = base;
    }
    __syncthreads();
    np = L.bi[0];
    for (int j = t; j < np; j += T) {
        int id = L.pid[j];
        int cnt = (int)L.pval[j];
        float x = lg[id];
        if (p.cap > 0.0f) x = dlk_softcap_glibc(x, p.cap);
        if (mk && !((mk[id >> 5] >> (id & 31)) & 1u)) x = -INFINITY;
        x = penalize(x, cnt, p);
        L.pval[j] = x;
        atomicOr(&L.pflag[id >> 11], 1u << ((id >> 6) & 31));
    }
    __syncthreads();
    return np;
}

/* ------------------------------------------------------------- exact top-k */

/* The key of the k-th element (1-based) under (s desc, index asc), as
 * desc_key(s): radix select on the 32-bit key (11/11/10 bits).  Also returns
 * how many keys are below it and how many equal it. */
struct KthKey {
    uint32_t key;
    int below, equal;
};
template <class KeyFn>
__device__ __forceinline__ KthKey radix_kth_keys(KeyFn key_of, int V, int k, uint32_t *hist, Lds &L) {
    const int t = threadIdx.x, T = blockDim.x, lane = lane_id();
    uint32_t prefix = 0;
    int krem = k, below_total = 0, eq_count = 0;
    for (int rd = 0; rd < 3; rd++) {
        const int sh = rd == 0 ? 21 : rd == 1 ? 10 : 0;
        const int width = rd == 2 ? 10 : 11;
        const int nb = 1 << width;
        const int hsh = rd == 0 ? 32 : rd == 1 ? 21 : 10;
        for (int b = t; b < nb; b += T) hist[b] = 0;
        __syncthreads();
        for (int i = t; i < V; i += T) {
            uint32_t key = key_of(i);
            bool in = rd == 0 || (key >> hsh) == prefix;
            if (in) atomicAdd(&hist[(key >> sh) & (nb - 1)], 1u);
        }
        __syncthreads();
        if (wave_id() == 0) {
            const int per = nb / 64;
            uint32_t loc = 0;
            for (int b = 0; b < per; b++) loc += hist[lane * per + b];
            const uint32_t inc = wave_scan_sat_u32(loc, 0xffffffffu);
            uint32_t exc = inc - loc;
            bool hit = exc < (uint32_t)krem && inc >= (uint32_t)krem;
            uint64_t bal = ballot(hit);
            int hl = first_lane(bal);
            if (lane == hl) {
                uint32_t run = exc;
                int b = 0;
                for (; b < per; b++) {
                    uint32_t c = hist[lane * per + b];
                    if (run + c >= (uint32_t)krem) break;
                    run += c;
                }
                L.bi[4] = lane * per + b;
                L.bi[5] = (int)run;
                L.bi[6] = (int)hist[lane * per + b];
            }
        }
        __syncthreads();
        int d = L.bi[4], below = L.bi[5];
        eq_count = L.bi[6];
        __syncthreads();
        prefix = (rd == 0) ? (uint32_t)d : ((prefix << width) | (uint32_t)d);
        krem -= below;
        below_total += below;
    }
    return KthKey{prefix, below_total, eq_count};
}

__device__ __forceinline__ KthKey radix_kth(const Row &R, int k, uint32_t *hist, Lds &L) {
    return radix_kth_keys([&](int i) { return desc_key(scaled(R, i)); }, R.V, k, hist, L);
}

/* desc_key with every NaN last (key 0xffffffff, past -inf): the order the
 * reference's top-k gives the entries it can take when no NaN sits among the
 * first k (a NaN past them never enters, src/sampler.c:122). */
DLK_DEV uint32_t key_nan_last(float s) { return s != s ? 0xffffffffu : desc_key(s); }

/* Index of the need-th (1-based) element i < V, in index order, with
 * key_of(i) == key; the block's count of such elements must reach need. */
template <class KeyFn>
__device__ __forceinline__ int nth_index_with_key(KeyFn key_of, int V, uint32_t key, int need, Lds &L) {
    const int t = threadIdx.x, T = blockDim.x, lane = lane_id();
    int *wcnt = (int *)L.red;
    int taken = 0, found = -1;
    for (int i0 = 0; i0 < V && found < 0; i0 += T) {
        const int i = i0 + t;
        const bool hit = i < V && key_of(i) == key;
        const uint64_t bal = ballot(hit);
        if (lane == 0) wcnt[wave_id()] = __popcll(bal);
        __syncthreads();
        int before = 0, tot = 0;
        for (int w = 0; w < n_waves(); w++) {
            if (w < wave_id()) before += wcnt[w];
            tot += wcnt[w];
        }
        const int rank = taken + before + __popcll(bal & ((1ull << lane) - 1));
        if (hit && rank == need - 1) L.bi[12] = i;
        taken += tot;
        __syncthreads();
        if (taken >= need) found = L.bi[12];
        __syncthreads();
    }
    return found;
}

/* First k elements under (s desc, index asc), sorted, into cand[0..k) as
 * (desc_key << 32 | index): the k-th key by radix select, then collection;
 * ties at the k-th key are taken in index order. */
__device__ __forceinline__ void select_top_k(const Row &R, int k, uint64_t *cand, int kp, uint32_t *hist, Lds &L) {
    const int t = threadIdx.x, T = blockDim.x, V = R.V, lane = lane_id();
    const KthKey kk = radix_kth(R, k, hist, L);
    const int below_total = kk.below, eq_count = kk.equal;
    const uint32_t kstar = kk.key;
    const int need = k - below_total;     /* >= 1 elements with key == kstar */
    int *cnt = L.bi + 8;                  /* [0] appended, [1] ties taken */
    if (t == 0) { cnt[0] = 0; cnt[1] = 0; }
    __syncthreads();
    const bool ordered_ties = eq_count > need;
    for (int i = t; i < V; i += T) {
        uint32_t key = desc_key(scaled(R, i));
        bool take = key < kstar || (!ordered_ties && key == kstar);
        if (take) {
            int at = atomicAdd(&cnt[0], 1);
            cand[at] = ((uint64_t)key << 32) | (uint32_t)i;
        }
    }
    __syncthreads();
    if (ordered_ties) {
        /* index-ordered pass over the ties, stopping after `need` of them */
        int *wcnt = (int *)L.red;
        for (int i0 = 0; i0 < V; i0 += T) {
            int taken = cnt[1];
            if (taken >= need) break;
            int i = i0 + t;
            bool tie = i < V && desc_key(scaled(R, i)) == kstar;
            uint64_t bal = ballot(tie);
            if (lane == 0) wcnt[wave_id()] = __popcll(bal);
            __syncthreads();
            int before = 0;
            for (int w = 0; w < wave_id(); w++) before += wcnt[w];
            int rank = taken + before + __popcll(bal & ((1ull << lane) - 1));
            if (tie && rank < need) cand[below_total + rank] = ((uint64_t)kstar << 32) | (uint32_t)i;
            __syncthreads();
            if (t == 0) {
                int tot = 0;
                for (int w = 0; w < n_waves(); w++) tot += wcnt[w];
                cnt[1] = taken + tot;
            }
            __syncthreads();
        }
    }
    for (int i = k + t; i < kp; i += T) cand[i] = ~0ull;
    __syncthreads();
    bitonic_sort(cand, kp);
}

/* Inclusive block prefix of per-thread u32 values in thread order; `total` is
 * the block's sum (red: one word per wave). */
DLK_DEV uint32_t block_incl_prefix_u32t(uint32_t v, uint32_t *red, uint32_t &total) {
    const int lane = lane_id(), w = wave_id(), nw = n_waves();
    const uint32_t inc = wave_scan_sat_u32(v, 0xffffffffu);
    if (lane == 63) red[w] = inc;
    __syncthreads();
    const uint32_t wt = wave_scan_sat_u32(lane < nw ? red[lane] : 0u, 0xffffffffu);
    const uint32_t base = w > 0 ? (uint32_t)__builtin_amdgcn_readlane((int)wt, w - 1) : 0u;
    total = (uint32_t)__builtin_amdgcn_readlane((int)wt, nw - 1);
    __syncthreads();
    return base + inc;
}

/* LDS words select_top_k_global needs (bucket bases and per-wave digit counts). */
constexpr int kLsdWords = 256 + 16 * 256 + 16;

/* select_top_k for a k too large for LDS: the first k elements under (s desc,
 * index asc), sorted, into a[0..k) (global memory; b[0..k) is the sort's second
 * buffer).  The k-th key by radix select; the candidates collected in index
 * order (ties at the k-th key: the first ones in index order, as the
 * reference's insertion sort keeps them, src/sampler.c:122,127); then a stable
 * LSD radix sort on the 32-bit s key, 4 passes of 8 bits, which keeps equal keys
 * in index order.  Needs blockDim.x <= 1024. */
__device__ __forceinline__ void select_top_k_global(const Row &R, int k, uint64_t *a, uint64_t *b, uint32_t *hist,
                                                    uint32_t *lsd, Lds &L) {
    const int t = threadIdx.x, T = blockDim.x, V = R.V, lane = lane_id(), w = wave_id(), nw = n_waves();
    /* (NaN keys last: a row reaching here holds no NaN among its first k) */
    const KthKey kk = radix_kth_keys([&](int i) { return key_nan_last(scaled(R, i)); }, V, k, hist, L);
    const int need = k - kk.below;                 /* ties at the k-th key to take, >= 1 */
    uint32_t *red = lsd + 256 + 16 * 256;
    /* ---- collection in index order: a tile of T elements at a time -------- */
    int base_lt = 0, base_tie = 0;
    for (int i0 = 0; i0 < V; i0 += T) {
        const int i = i0 + t;
        const uint32_t key = i < V ? key_nan_last(scaled(R, i)) : 0xffffffffu;
        const bool lt = i < V && key < kk.key, tie = i < V && key == kk.key;
        const uint32_t v = (lt ? 1u : 0u) | (tie ? 0x10000u : 0u);
        uint32_t tot = 0;
        const uint32_t ex = block_incl_prefix_u32t(v, red, tot) - v;
        const int lt_before = base_lt + (int)(ex & 0xffffu), tie_before = base_tie + (int)(ex >> 16);
        if (lt || (tie && tie_before < need))
            a[lt_before + min(tie_before, need)] = ((uint64_t)key << 32) | (uint32_t)i;
        base_lt += (int)(tot & 0xffffu);
        base_tie += (int)(tot >> 16);
    }
    __syncthreads();
    /* ---- stable LSD radix sort of a[0..k) on bits 32..63 ------------------- */
    uint32_t *cnt = lsd, *wc = lsd + 256;
    uint64_t *src = a, *dst = b;
    const uint64_t lt_mask = (1ull << lane) - 1ull;
    for (int pass = 0; pass < 4; pass++) {
        const int sh = 32 + 8 * pass;
        for (int d = t; d < 256; d += T) cnt[d] = 0;
        __syncthreads();
        for (int i = t; i < k; i += T) atomicAdd(&cnt[(uint32_t)(src[i] >> sh) & 255u], 1u);
        __syncthreads();
        if (w == 0) {
            const uint32_t c0 = cnt[4 * lane], c1 = cnt[4 * lane + 1], c2 = cnt[4 * lane + 2], c3 = cnt[4 * lane + 3];
            const uint32_t s4 = c0 + c1 + c2 + c3;
            const uint32_t ex = wave_scan_sat_u32(s4, 0xffffffffu) - s4;
            cnt[4 * lane] = ex;
            cnt[4 * lane + 1] = ex + c0;
            cnt[4 * lane + 2] = ex + c0 + c1;
            cnt[4 * lane + 3] = ex + c0 + c1 + c2;
        }
        __syncthreads();
        for (int i0 = 0; i0 < k; i0 += T) {
            const int i = i0 + t;
            const bool valid = i < k;
            const uint64_t e = valid ? src[i] : 0ull;
            const uint32_t d = (uint32_t)(e >> sh) & 255u;
            for (int j = t; j < 16 * 256; j += T) wc[j] = 0;
            /* lanes of this wave holding the same digit (8 ballots) */
            uint64_t m = ballot(valid);
#pragma unroll
            for (int bit = 0; bit < 8; bit++) {
                const uint64_t bb = ballot(valid && ((d >> bit) & 1u));
                m &= ((d >> bit) & 1u) ? bb : ~bb;
            }
            const int rank = __popcll(m & lt_mask);
            __syncthreads();
            if (valid && rank == 0) wc[w * 256 + d] = (uint32_t)__popcll(m);
            __syncthreads();
            /* per digit: the waves' offsets in order, then the bucket moves on */
            for (int dd = t; dd < 256; dd += T) {
                uint32_t acc = cnt[dd];
                for (int ww = 0; ww < nw; ww++) {
                    const uint32_t c = wc[ww * 256 + dd];
                    wc[ww * 256 + dd] = acc;
                    acc += c;
                }
                cnt[dd] = acc;
            }
            __syncthreads();
            if (valid) dst[wc[w * 256 + d] + (uint32_t)rank] = e;
            __syncthreads();
        }
        uint64_t *tmp = src;
        src = dst;
        dst = tmp;
    }
    /* four passes: the sorted keys are back in a */
}

/* -------------------------------------------------------- sampling pipeline */

/* Base sequence of the softmax: e_j over candidate positions j < n. */
struct FullBase {           /* k = V: position j is token j */
    const Row *R;
    DLK_DEV float e(int j) const { return expo(*R, scaled(*R, j)); }
    DLK_DEV int token(int j) const { return j; }
};
struct CandBase {           /* top-k: position j is cand[j] */
    const Row *R;
    const uint64_t *cand;
    DLK_DEV float s(int j) const { return key_value((uint32_t)(cand[j] >> 32)); }
    DLK_DEV float e(int j) const { return expo(*R, s(j)); }
    DLK_DEV int token(int j) const { return (int)(uint32_t)cand[j]; }
};

struct Scal {               /* row scalars of the later stages */
    float inv, inv2, inv3, min_p;
    int minp_on, minp_all, topp_on, cut;     /* cut: last kept position */
};

template <class B>
struct QSoft {              /* p_j = e_j * inv_sum (src/sampler.c:183-185) */
    const B *b; const Scal *S;
    DLK_DEV float operator()(int j) const { return b->e(j) * S->inv; }
};
template <class B>
struct QExp {
    const B *b;
    DLK_DEV float operator()(int j) const { return b->e(j); }
};
template <class B>
struct QSurv {              /* min-p survivors (src/sampler.c:191-195) */
    const B *b; const Scal *S;
    DLK_DEV float operator()(int j) const {
        float pj = b->e(j) * S->inv;
        return (S->minp_all || pj >= S->min_p) ? pj : 0.0f;
    }
};
template <class B>
struct QTopP {              /* input of the top-p cumulation */
    const B *b; const Scal *S;
    DLK_DEV float operator()(int j) const {
        float pj = b->e(j) * S->inv;
        if (!S->minp_on) return pj;
        if (!(S->minp_all || pj >= S->min_p)) return 0.0f;
        return pj * S->inv2;
    }
};
template <class B>
struct QDraw {              /* final probabilities (src/sampler.c:221, :228) */
    const B *b; const Scal *S;
    DLK_DEV float operator()(int j) const {
        QTopP<B> tp{b, S};
        float v = tp(j);
        if (!S->topp_on) return v;
        return j <= S->cut ? v * S->inv3 : 0.0f;
    }
};

/* Runs one exact sum: block builds aggregates, wave 0 resolves, all threads get
 * (pos, value). */
template <int MB, class QF>
__device__ __forceinline__ ResolveOut<MB> exact_sum(int n, const QF &q, const Aggs &A, double scale, double cut, bool has_thr,
                                    double thr, Lds &L) {
    build_aggs<MB>(n, q, A, scale, cut);
    if (wave_id() == 0) {
        ResolveOut<MB> o = resolve<MB>(n, q, A, has_thr, thr);
        if (lane_id() == 0) { L.bi[16] = o.pos; L.bd[8] = (double)o.value; }
    }
    __syncthreads();
    ResolveOut<MB> o;
    o.pos = L.bi[16];
    o.value = (typename Fmt<MB>::T)L.bd[8];
    __syncthreads();
    return o;
}

/* The reference's softmax/min-p/top-p/draw over n candidate positions.
 * Returns the sampled position; fills S. */
/* ------------------------------------------------- rows holding NaN or +inf */

/* Largest k for which a row whose s holds NaN runs emulate_topk_row (the
 * reference's O(V k) insertion sort on one thread). */
constexpr int kEmulateMaxK = 4096;

/* Top-k rows holding NaN or +inf after the mask and penalties: once NaN takes
 * part, the reference's insertion sort keeps NaN entries in place and stops
 * other entries at them, and its sums and comparisons turn NaN, so the outcome
 * depends on the order of every step.  One thread therefore runs the
 * reference's own sequence (src/sampler.c:155-233): the row max (:155-158),
 * s = (l - max) * (1/T) (:160-162), the insertion partial sort (:109-134), the
 * softmax over the k candidates (:173-185), min-p (:188-202), top-p (:205-222)
 * and the draw (:225-233).  cand holds k (value bits << 32 | index) entries.
 * Writes the token and the candidate outputs; call from thread 0 only. */
__device__ __forceinline__ void emulate_topk_row(const RowParams &p, const Row &R, int k, float r, uint64_t *cand,
                                                 int row) {
    auto ent = [](int i, float v) { return ((uint64_t)f2u(v) << 32) | (uint32_t)i; };
    auto val = [](uint64_t e) { return u2f((uint32_t)(e >> 32)); };
    const int V = R.V;
    float mx = prepared(R, 0);
    for (int i = 1; i < V; i++) {
        const float x = prepared(R, i);
        if (x > mx) mx = x;
    }
    const float inv_t = R.inv_t;
    for (int i = 0; i < k; i++) cand[i] = ent(i, (prepared(R, i) - mx) * inv_t);
    for (int i = 1; i < k; i++) {
        const uint64_t tmp = cand[i];
        int j = i;
        while (j > 0 && val(cand[j - 1]) < val(tmp)) { cand[j] = cand[j - 1]; j--; }
        cand[j] = tmp;
    }
    for (int i = k; i < V; i++) {
        const float v = (prepared(R, i) - mx) * inv_t;
        if (v > val(cand[k - 1])) {
            const uint64_t tmp = ent(i, v);
            int j = k - 1;
            while (j > 0 && val(cand[j - 1]) < v) { cand[j] = cand[j - 1]; j--; }
            cand[j] = tmp;
        }
    }
    /* softmax over the k candidates */
    float mv = val(cand[0]);
    for (int i = 1; i < k; i++)
        if (val(cand[i]) > mv) mv = val(cand[i]);
    double sum = 0.0;
    for (int i = 0; i < k; i++) {
        const float e = dlk_expf_glibc(val(cand[i]) - mv, R.tab);
        cand[i] = ent((int)(uint32_t)cand[i], e);
        sum += e;
    }
    const float inv = (float)(1.0 / sum);
    for (int i = 0; i < k; i++) cand[i] = ent((int)(uint32_t)cand[i], val(cand[i]) * inv);
    /* min-p: the list is the entries >= min_p when any is, else all k */
    const bool minp = p.min_p > 0.0f;
    int nmin = 0;
    if (minp)
        for (int i = 0; i < k; i++) nmin += val(cand[i]) >= p.min_p;
    const bool all = !minp || nmin == 0;
    auto member = [&](int i) { return all || val(cand[i]) >= p.min_p; };
    float inv2 = 1.0f;
    if (minp) {
        double s2 = 0.0;
        for (int i = 0; i < k; i++)
            if (member(i)) s2 += val(cand[i]);
        inv2 = (float)(1.0 / s2);
    }
    auto w = [&](int i) { return minp ? val(cand[i]) * inv2 : val(cand[i]); };
    /* top-p over the list: nk members kept */
    int nk = all ? k : nmin;
    float inv3 = 1.0f;
    const bool topp = p.top_p < 1.0f;
    if (topp) {
        double cum = 0.0;
        int rank = 0;
        for (int i = 0; i < k; i++) {
            if (!member(i)) continue;
            cum += w(i);
            rank++;
            if ((float)cum >= p.top_p) { nk = rank; break; }
        }
        double s3 = 0.0;
        rank = 0;
        for (int i = 0; i < k && rank < nk; i++) {
            if (!member(i)) continue;
            s3 += w(i);
            rank++;
        }
        inv3 = (float)(1.0 / s3);
    }
    auto q = [&](int i) { return topp ? w(i) * inv3 : w(i); };
    /* the draw */
    float cum = 0.0f;
    int tok = -1, last = -1, rank = 0;
    for (int i = 0; i < k && rank < nk; i++) {
        if (!member(i)) continue;
        cum += q(i);
        rank++;
        last = (int)(uint32_t)cand[i];
        if (r < cum) { tok = last; break; }
    }
    p.out_ids[row] = tok >= 0 ? tok : last;
    /* candidate outputs: softmax probabilities and log of the final ones */
    rank = 0;
    for (int j = 0; j < p.n_out; j++) {
        const int64_t o = (int64_t)row * p.n_out + j;
        if (j < k) {
            const bool in = member(j) && rank < nk;
            if (member(j)) rank++;
            const float fj = in ? q(j) : 0.0f;
            if (p.out_cand_ids) p.out_cand_ids[o] = (int)(uint32_t)cand[j];
            if (p.out_cand_probs) p.out_cand_probs[o] = val(cand[j]);
            if (p.out_cand_logprobs) p.out_cand_logprobs[o] = fj > 0.0f ? (float)log((double)fj) : -INFINITY;
        } else {
            if (p.out_cand_ids) p.out_cand_ids[o] = -1;
            if (p.out_cand_probs) p.out_cand_probs[o] = 0.0f;
            if (p.out_cand_logprobs) p.out_cand_logprobs[o] = -INFINITY;
        }
    }
}

template <class B>
__device__ __forceinline__ int pipeline(const RowParams &p, const B &base, int n, float r, unsigned char *region, Lds &L, Scal &S) {
    Aggs A = make_aggs(region, n);
    S.inv2 = 1.0f; S.inv3 = 1.0f; S.min_p = p.min_p;
    S.minp_on = p.minp_on; S.minp_all = 0; S.topp_on = p.topp_on; S.cut = n - 1;
    /* softmax sum, src/sampler.c:177-182 */
    QExp<B> qe{&base};
    chunk_prefix(n, qe, A.P, L.red);
    ResolveOut<53> s1 = exact_sum<53>(n, qe, A, 1.0, INFINITY, false, 0.0, L);
    S.inv = (float)(1.0 / s1.value);
    double scale = S.inv;
    if (S.minp_on) {
        /* src/sampler.c:188-202: survivors p >= min_p, all kept if none. */
        int cnt = 0, last = -1;
        for (int j = threadIdx.x; j < n; j += blockDim.x) {
            if (base.e(j) * S.inv >= S.min_p) { cnt++; last = max(last, j); }
        }
        cnt = block_sum_int(cnt, L);
        for (int m = 32; m >= 1; m >>= 1) last = max(last, shfl_xor(last, m));
        if (lane_id() == 0) L.bi[32 + wave_id()] = last;
        __syncthreads();
        int lastall = -1;
        for (int w = 0; w < n_waves(); w++) lastall = max(lastall, L.bi[32 + w]);
        __syncthreads();
        S.minp_all = cnt == 0;
        S.cut = S.minp_all ? n - 1 : lastall;
        QSurv<B> qs{&base, &S};
        chunk_prefix(n, qs, A.P, L.red);
        ResolveOut<53> s2 = exact_sum<53>(n, qs, A, 1.0, INFINITY, false, 0.0, L);
        S.inv2 = (float)(1.0 / s2.value);
        scale = S.inv2;
    }
    int last_kept = S.cut;
    if (S.topp_on) {
        QTopP<B> qt{&base, &S};
        double s3;
        int x;
        if (p.top_p <= 0.0f) {
            /* cumul after the first kept entry is that entry: nk = 1 */
            x = 0;
            if (S.minp_on && !S.minp_all) {
                int first = n;
                for (int j = threadIdx.x; j < n; j += blockDim.x)
                    if (base.e(j) * S.inv >= S.min_p) first = min(first, j);
                for (int m = 32; m >= 1; m >>= 1) first = min(first, shfl_xor(first, m));
                if (lane_id() == 0) L.bi[32 + wave_id()] = first;
                __syncthreads();
                x = n;
                for (int w = 0; w < n_waves(); w++) x = min(x, L.bi[32 + w]);
                __syncthreads();
            }
            s3 = (double)qt(x);
        } else {
            ResolveOut<53> o = exact_sum<53>(n, qt, A, scale, INFINITY, true, p.topp_thr, L);
            x = o.pos >= 0 ? o.pos : last_kept;
            s3 = o.value;
        }
        S.inv3 = (float)(1.0 / s3);
        S.cut = x;
        last_kept = x;
        scale = scale * (double)S.inv3;
    }
    /* draw, src/sampler.c:225-233: first j with r < cumul (cumul >= nextafter(r)) */
    QDraw<B> qd{&base, &S};
    double cutP = A.P[min((n + 63) >> 6, (last_kept >> 6) + 1)];
    double vthr = (double)u2f(f2u(r) + 1u);
    ResolveOut<24> d = exact_sum<24>(n, qd, A, scale, cutP, true, vthr, L);
    return d.pos >= 0 ? d.pos : last_kept;
}

/* The reference's running double sum of the lanes' values in lane order
 * (finite, non-negative; a 0 adds nothing), as an inclusive prefix in every
 * lane -- by a wave scan, when that is provably the same: if every value is a
 * whole multiple of U = 2^(k-52), where 2^k > 64 * max >= every prefix, each
 * prefix is a multiple of U below 2^(k+1), so a double, every addition of the
 * sequential loop is exact, and a scan in any order gives the same numbers.
 * Returns false when the condition fails (the caller runs the loop). */
DLK_DEV bool exact_prefix_d(float v, double &pre) {
    const float mx = wave_max_dpp(v);
    if (!(mx < INFINITY)) return false;
    int k = 0;
    (void)frexp(64.0 * (double)mx, &k);       /* 64 * max < 2^k */
    const double sc = ldexp((double)v, 52 - k);
    if (ballot(!(sc == trunc(sc))) != 0) return false;
    pre = wave_incl_scan_d((double)v);
    return true;
}

/* pipeline for n <= 64 candidates, by one wave (lane j holds candidate j): the
 * reference's sequential sums (src/sampler.c:177-233) in the same order -- a
 * double sum by exact_prefix_d's scan where that gives the same number, else
 * literally, every lane repeating it on values read lane by lane; the draw's
 * float sum literally.  No block barrier; the caller broadcasts pos and S. */
template <class B>
__device__ __forceinline__ int pipeline_small(const RowParams &p, const B &base, int n, float r, Scal &S) {
    const int lane = lane_id();
    S.inv2 = 1.0f; S.inv3 = 1.0f; S.min_p = p.min_p;
    S.minp_on = p.minp_on; S.minp_all = 0; S.topp_on = p.topp_on; S.cut = n - 1;
    const float e = lane < n ? base.e(lane) : 0.0f;
    /* softmax, :177-185 */
    double sum = 0.0, pre = 0.0;
    if (exact_prefix_d(e, pre)) {
        sum = u2d(readlane64(d2u(pre), 63));
    } else {
        for (int j = 0; j < n; j++) sum += (double)readlanef(e, j);
    }
    S.inv = (float)(1.0 / sum);
    const float pj = e * S.inv;
    /* min-p, :188-202: survivors in order, all kept if none survives */
    float t = pj;
    if (S.minp_on) {
        const uint64_t surv = ballot(lane < n && pj >= S.min_p);
        S.minp_all = surv == 0;
        S.cut = S.minp_all ? n - 1 : 63 - __builtin_clzll(surv);
        const bool kept = lane < n && (S.minp_all || ((surv >> lane) & 1ull));
        double s2 = 0.0;
        if (exact_prefix_d(kept ? pj : 0.0f, pre)) {
            s2 = u2d(readlane64(d2u(pre), 63));
        } else {
            for (int j = 0; j < n; j++)
                if (S.minp_all || ((surv >> j) & 1ull)) s2 += (double)readlanef(pj, j);
        }
        S.inv2 = (float)(1.0 / s2);
        t = kept ? pj * S.inv2 : 0.0f;
    }
    int last_kept = S.cut;
    /* top-p, :205-222: the first position whose cumulative (float) reaches top_p */
    if (S.topp_on) {
        int x = last_kept;
        double s3 = 0.0;
        if (p.top_p <= 0.0f) {
            x = S.minp_on && !S.minp_all ? __builtin_ctzll(ballot(lane < n && pj >= S.min_p)) : 0;
            s3 = (double)readlanef(t, x);
        } else if (exact_prefix_d(lane <= last_kept ? t : 0.0f, pre)) {
            /* the first position whose prefix reaches top_p, else all kept */
            const uint64_t hit = ballot(lane <= last_kept && (float)pre >= p.top_p);
            x = hit ? __builtin_ctzll(hit) : last_kept;
            s3 = u2d(readlane64(d2u(pre), x));
        } else {
            double cumul = 0.0;
            for (int j = 0; j <= last_kept; j++) {
                cumul += (double)readlanef(t, j);
                if ((float)cumul >= p.top_p) { x = j; break; }
            }
            s3 = cumul;
        }
        S.inv3 = (float)(1.0 / s3);
        S.cut = x;
        last_kept = x;
        t = lane <= x ? t * S.inv3 : 0.0f;
    }
    /* draw, :225-233: the first position with r < cumul, else the last kept */
    float cumul = 0.0f;
    for (int j = 0; j <= last_kept; j++) {
        cumul += readlanef(t, j);
        if (r < cumul) return j;
    }
    return last_kept;
}

}  // namespace dlk

#endif
