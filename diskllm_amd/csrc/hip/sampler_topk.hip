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
 * +-FLT_MAX, which the cap maps to the same +-cap -- and only the elements it
 * collects are capped; the penalty patches are capped values, handled from
 * their LDS list.  Ties that the cap creates are resolved by the order
 * (y desc, index asc) of the collected candidates and the merge's certificate. */
template <int EPT, bool CAP>
__global__ __launch_bounds__(kTopkThreads, 4) void topk_kernel(TopkParams f) {
    extern __shared__ __align__(16) unsigned char smem[];
    const RowParams &p = f.p;
    const int g = blockIdx.x, row = blockIdx.y, t = threadIdx.x, lane = lane_id(), w = wave_id();
    const int T = kTopkThreads, V = p.V, G = f.G;
    const int s0 = g * f.S, s1 = min(V, s0 + f.S);
    const float *lg = p.logits + (int64_t)row * p.ld;
    const uint32_t *mk = nullptr;
    if (p.mask) mk = p.mask + (int64_t)(p.mask_row ? p.mask_row[row] : row) * p.mask_ld;

    /* LDS: the row-kernel layout (for the in-workgroup fallback) + fast-path buffers */
    Lds L = make_lds(smem, p.plan);
    unsigned char *q = L.region;
    uint32_t *sbits = (uint32_t *)carve(q, (size_t)(f.S / 32) * 4);          /* patched positions in slice */
    float *tmax = (float *)carve(q, (size_t)T * 4);
    int *misc = (int *)carve(q, 64 * 4);
    int *selh = (int *)carve(q, kSelWords * 4);                           /* radix-select histogram */
    uint64_t *buf = (uint64_t *)carve(q, (size_t)f.buf_cap * 8);           /* collect / merge / fallback (+ aggs) */
    if (t < 32) L.tab[t] = kExp2Tab[t];
    const uint64_t rng0 = p.greedy ? 0ull : p.rng[row];     /* read early: only the merge uses (and writes) it */

    const int32_t *hist = nullptr;
    int nh = 0;
    if (p.hist_off) {
        hist = p.hist_ids + p.hist_off[row];
        nh = p.hist_off[row + 1] - p.hist_off[row];
    }

    if (nh > p.plan.hcap) {
        if (g == 0 && t == 0) {
            p.out_ids[row] = -1;
            if (p.status) atomicOr(p.status, DLK_STATUS_HISTORY_TOO_LONG);
        }
        return;
    }
    /* ---- 1. penalty patches of the ids inside this slice ---------------- */
    for (int i = t; i < f.S / 32; i += T) sbits[i] = 0;
    if (t == 0) misc[0] = 0;
    __syncthreads();
    int *hl = (int *)L.hsort;                      /* the row's history, staged in LDS */
    for (int i = t; i < nh; i += T) hl[i] = hist[i];
    __syncthreads();
    for (int i = t; i < nh; i += T) {             /* in-slice occurrences, first occurrence only */
        int id = hl[i];
        if (id < s0 || id >= s1) continue;
        bool first = true;
        int cnt = 0;
        for (int j = 0; j < nh; j++) {
            int o = hl[j];
            if (o == id) { cnt++; if (j < i) first = false; }
        }
        if (!first) continue;
        float x = lg[id];
        if (CAP) x = dlk_softcap_glibc(x, p.cap);  /* the soft-cap first (src/core/context.c:873-876) */
        if (mk && !((mk[id >> 5] >> (id & 31)) & 1u)) x = -INFINITY;
        x = penalised(p, x, cnt);
        int at = atomicAdd(&misc[0], 1);
        if (at < p.plan.hcap) { L.pid[at] = id; L.pval[at] = x; }
        atomicOr(&sbits[(id - s0) >> 5], 1u << ((id - s0) & 31));
    }
    __syncthreads();
    const int np = min(misc[0], p.plan.hcap);

    /* ---- 2. stream the slice into registers ---------------------------- */
    float v[EPT];
    float tm = -INFINITY;
    int targ = 0x7fffffff, nfin = 0, irr = 0;
#pragma unroll
    for (int j4 = 0; j4 < EPT / 4; j4++) {
        const int i0 = s0 + 4 * (t + j4 * T);
        float4 x4 = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        if (i0 + 3 < s1) {
            x4 = *(const float4 *)(lg + i0);
        } else {
            if (i0 < s1) x4.x = lg[i0];
            if (i0 + 1 < s1) x4.y = lg[i0 + 1];
            if (i0 + 2 < s1) x4.z = lg[i0 + 2];
        }
        float xs[4] = {x4.x, x4.y, x4.z, x4.w};
        uint32_t mw = 0xffffffffu;
        if (mk && i0 < s1) mw = mk[i0 >> 5] >> (i0 & 31);
        uint32_t pb = 0;
        if (i0 < s1) pb = (sbits[(i0 - s0) >> 5] >> ((i0 - s0) & 31)) & 0xFu;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int i = i0 + c;
            float x = xs[c];
            if (CAP && !(x != x)) x = fminf(fmaxf(x, -kFltMax), kFltMax);   /* raw stand-in of cap(x) */
            if (!((mw >> c) & 1u)) x = -INFINITY;
            if ((pb >> c) & 1u) {
                if (CAP) {
                    x = -INFINITY;                 /* a capped patch: from the LDS list below */
                } else {
                    for (int k = 0; k < np; k++)
                        if (L.pid[k] == i) x = L.pval[k];
                }
            }
            if (i >= s1) x = -INFINITY;
            v[j4 * 4 + c] = x;
            if (i < s1) {
                if (x > tm || (x == tm && i < targ)) { tm = x; targ = i; }
                nfin += (x > -INFINITY);
                irr |= !(x < INFINITY) && !(x == -INFINITY);
            }
        }
    }
    float pmax = -INFINITY;                        /* CAP: largest capped patch */
    if (CAP) {
        for (int k = t; k < np; k += T) {
            const float y = L.pval[k];
            nfin += y > -INFINITY;
            irr |= !(y < INFINITY) && !(y == -INFINITY);
            pmax = fmaxf(pmax, y);
        }
    }
    /* ---- 3. workgroup max / argmax / finite count ----------------------- */
    float bm = tm;
    int bi = targ;
    block_argmax(bm, bi, L);
    int nf = block_sum_int(nfin, L);
    irr = block_sum_int(irr, L);
    if (CAP) {
        /* the slice maximum of the capped row (the argmax serves greedy
         * sampling, which does not take this path under a cap) */
        uint32_t pbits = asc_key(pmax);             /* ascending keys: the largest key is the maximum */
        for (int m2 = 32; m2 >= 1; m2 >>= 1) pbits = max(pbits, (uint32_t)shfl_xor((int)pbits, m2));
        if (lane == 0) misc[24 + w] = (int)pbits;
        __syncthreads();
        for (int u = 0; u < T / 64; u++) pbits = max(pbits, (uint32_t)misc[24 + u]);
        __syncthreads();
        const float pm = key_value(~pbits);
        const float cm = bm > -INFINITY ? dlk_softcap_glibc(bm, p.cap) : bm;
        bm = fmaxf(cm, pm);
    }
    TopkSlot *slot = f.slots + ((int64_t)row * G + g);
    uint64_t *cands = f.cands + ((int64_t)row * G + g) * f.KP;

    int kept = 0, complete = 1;
    uint32_t last_key = 0;
    if (!p.greedy && nf > 0) {
        /* ---- 4. threshold: the KP-th largest thread maximum ------------- */
        ((uint32_t *)tmax)[t] = asc_key(tm);
        __syncthreads();
        const int KP = f.KP;
        const uint32_t *tk32 = (const uint32_t *)tmax;
        const uint32_t thr_key = block_select_u32(T, T - min(KP, T), [&](int i) { return tk32[i]; }, selh, selh + 256);
        float thr = key_value(~thr_key);
        if (!(thr > -INFINITY)) thr = -INFINITY;
        /* CAP: the patches at or above the capped threshold join the candidates */
        const float cthr = CAP && thr > -INFINITY ? dlk_softcap_glibc(thr, p.cap) : -INFINITY;
        /* ---- 5. collect finite elements >= thr ------------------------- */
        /* a count per thread, one block prefix, then the writes */
        uint32_t cnt = 0;
#pragma unroll
        for (int j = 0; j < EPT; j++) cnt += (v[j] > -INFINITY && v[j] >= thr) ? 1u : 0u;
        if (CAP)
            for (int k = t; k < np; k += T) cnt += (L.pval[k] > -INFINITY && L.pval[k] >= cthr) ? 1u : 0u;
        const uint32_t incl = wave_scan_sat_u32(cnt, 0xffffffffu);
        if (lane == 63) misc[8 + w] = (int)incl;
        __syncthreads();
        int at = (int)(incl - cnt), C = 0;
        for (int u = 0; u < T / 64; u++) {
            if (u < w) at += misc[8 + u];
            C += misc[8 + u];
        }
#pragma unroll
        for (int j = 0; j < EPT; j++) {
            const float x = v[j];
            if (x > -INFINITY && x >= thr) {
                const float y = CAP ? dlk_softcap_glibc(x, p.cap) : x;
                if (at < f.buf_cap) buf[at] = ((uint64_t)desc_key(y) << 32) | (uint32_t)(s0 + 4 * (t + (j / 4) * T) + (j & 3));
                at++;
            }
        }
        if (CAP) {
            for (int k = t; k < np; k += T) {
                const float y = L.pval[k];
                if (y > -INFINITY && y >= cthr) {
                    if (at < f.buf_cap) buf[at] = ((uint64_t)desc_key(y) << 32) | (uint32_t)L.pid[k];
                    at++;
                }
            }
        }
        __syncthreads();
        if (C > f.buf_cap) {
            complete = -1;                     /* overflow: the merge falls back */
        } else {
            int P = 64;
            while (P < C) P <<= 1;
            for (int i = C + t; i < P; i += T) buf[i] = ~0ull;
            __syncthreads();
            /* keys carry their index: distinct, so a rank sort when they fit */
            if (C <= T) rank_sort_distinct(buf, C);
            else bitonic_sort(buf, P);
            kept = min(KP, C);
            complete = (C == nf) ? 1 : 0;
            last_key = (uint32_t)(buf[kept - 1] >> 32);
            for (int j = t; j < kept; j += T) pub64(&cands[j], buf[j]);
        }
    }
    /* ---- 6. publish and elect the merging workgroup --------------------- */
    if (t == 0) {
        pub32(&slot->max_bits, f2u(bm));
        pub32(&slot->argmax, (uint32_t)bi);
        pub32(&slot->nfin, (uint32_t)nf);
        pub32(&slot->kept, (uint32_t)kept);
        pub32(&slot->complete, (uint32_t)complete);
        pub32(&slot->last_key, last_key);
        pub32(&slot->first_nan, ((g == 0 && isnan(v[0])) ? 1u : 0u) | (irr ? 2u : 0u));
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
    if (t == 0) pub32(&f.counters[row], 0u);
    /* slot h -> LDS (misc[16..]: kept, complete, last_key per slice; up to 64 slices per pass) */
    uint32_t *sk = (uint32_t *)tmax;                 /* tmax is free now: 3 words per slice */
    float M = -INFINITY;
    int amax = 0x7fffffff, NF = 0, total = 0, overflow = 0, first_nan = 0, irregular = 0;
    for (int h = t; h < G; h += T) {
        TopkSlot *s = f.slots + ((int64_t)row * G + h);
        sk[3 * h + 0] = get32(&s->kept);
        sk[3 * h + 1] = get32(&s->complete);
        sk[3 * h + 2] = get32(&s->last_key);
        buf[h] = ((uint64_t)get32(&s->max_bits) << 32) | get32(&s->argmax);
        buf[G + h] = ((uint64_t)get32(&s->nfin) << 32) | get32(&s->first_nan);
    }
    __syncthreads();
    if (w == 0) {
        /* one wave: slices lane, lane + 64, ...; then lane reductions (the
         * argmax keeps the larger value, ties to the lower index, as in order) */
        for (int h = lane; h < G; h += 64) {
            const float m = u2f((uint32_t)(buf[h] >> 32));
            const int a = (int)(uint32_t)buf[h];
            if (m > M || (m == M && a < amax)) { M = m; amax = a; }
            NF += (int)(buf[G + h] >> 32);
            first_nan |= (int)((uint32_t)buf[G + h] & 1u);
            irregular |= (int)((uint32_t)buf[G + h] & 2u);
            total += (int)sk[3 * h];
            overflow |= (int)sk[3 * h + 1] == -1;
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
        if (lane == 0) {
            misc[48] = (int)f2u(M); misc[49] = amax; misc[50] = NF; misc[51] = first_nan;
            misc[52] = irregular; misc[53] = total; misc[54] = overflow;
        }
    }
    __syncthreads();
    M = u2f((uint32_t)misc[48]); amax = misc[49]; NF = misc[50]; first_nan = misc[51];
    irregular = misc[52]; total = misc[53]; overflow = misc[54];
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
    __syncthreads();
    if (t == 0) p.rng[row] = st;
    const int k = p.top_k;
    if (irregular) {
        /* NaN or +inf in the row: the reference's sequence on one thread */
        Row R;
        R.lg = lg; R.mk = mk; R.V = V; R.pid = L.pid; R.pval = L.pval; R.pflag = L.pflag;
        R.M = 0.0f; R.inv_t = p.inv_temp; R.maxv = 0.0f; R.tab = L.tab; R.cap = p.cap;
        R.np = build_patches(p, row, lg, mk, L, p.plan, V);
        if (t == 0) emulate_topk_row(p, R, k, r, buf, row);
        return;
    }
    if (NF == 0) {                           /* every entry -inf (see sampler_row.hip) */
        if (t == 0) p.out_ids[row] = k - 1;
        out_cands_empty(NAN, NAN, true, k);
        return;
    }

    Row R;
    R.lg = lg; R.mk = mk; R.V = V; R.pid = L.pid; R.pval = L.pval; R.np = 0; R.pflag = L.pflag;
    R.M = M; R.inv_t = p.inv_temp; R.maxv = 0.0f; R.tab = L.tab; R.cap = p.cap;

    /* gather candidates re-keyed on s, sorted (s desc, index asc) */
    bool ok = !overflow && total <= f.buf_cap;
    int P = 64;
    if (ok) {
        /* every candidate read at once: thread t takes the slots t + u * T of
         * the G x KP candidate array (slot j of slice h holds its (j+1)-th best
         * logit when j < kept_h) */
        uint32_t *tau = (uint32_t *)(sk + 3 * G);
        if (t == 0) { *tau = 0xffffffffu; misc[46] = 0; }
        __syncthreads();
        const int KP = f.KP, GK = G * KP;
        const uint64_t *crow = f.cands + (int64_t)row * GK;
        uint64_t cv[kMergePerThread];
#pragma unroll
        for (int u = 0; u < kMergePerThread; u++) {
            const int i = t + u * T;
            const int h = i / KP, j = i - h * KP;
            cv[u] = (i < GK && j < (int)sk[3 * h]) ? get64(&crow[i]) : ~0ull;
        }
        /* a bound for the sort: list h is in logit order and s is monotone in
         * the logit, so at least k entries have s >= the s of its k-th entry;
         * anything whose s is below the best such bound is not in the top k */
#pragma unroll
        for (int u = 0; u < kMergePerThread; u++) {
            const int i = t + u * T;
            if (cv[u] != ~0ull) {
                cv[u] = ((uint64_t)desc_key((key_value((uint32_t)(cv[u] >> 32)) - M) * R.inv_t) << 32) |
                        (cv[u] & 0xffffffffull);
                if (i % KP == k - 1) atomicMin(tau, (uint32_t)(cv[u] >> 32));
            }
        }
        __syncthreads();
        const uint32_t tk = *tau;
#pragma unroll
        for (int u = 0; u < kMergePerThread; u++) {
            const bool take = cv[u] != ~0ull && (uint32_t)(cv[u] >> 32) <= tk;
            const uint64_t bal = ballot(take);
            int base = 0;
            if (lane == 0 && bal) base = atomicAdd(&misc[46], __popcll(bal));
            base = shfl(base, 0);
            if (take) buf[base + __popcll(bal & ((1ull << lane) - 1))] = cv[u];
        }
        __syncthreads();
        int nsort = misc[46];
        if (nsort > 64 && nsort >= k) {
            /* only the k best are needed: the k-th smallest s-key by radix
             * select, then the entries at or below it (k plus any ties) */
            const uint32_t K = block_select_u32(nsort, k - 1, [&](int i) { return (uint32_t)(buf[i] >> 32); }, selh,
                                                selh + 256);
            uint64_t mine[kMergePerThread];
#pragma unroll
            for (int u = 0; u < kMergePerThread; u++) {
                const int i = t + u * T;
                mine[u] = i < nsort ? buf[i] : ~0ull;
            }
            if (t == 0) misc[47] = 0;
            __syncthreads();
#pragma unroll
            for (int u = 0; u < kMergePerThread; u++) {
                const bool take = (uint32_t)(mine[u] >> 32) <= K && mine[u] != ~0ull;
                const uint64_t bal = ballot(take);
                int base = 0;
                if (lane == 0 && bal) base = atomicAdd(&misc[47], __popcll(bal));
                base = shfl(base, 0);
                if (take) buf[base + __popcll(bal & ((1ull << lane) - 1))] = mine[u];
            }
            __syncthreads();
            nsort = misc[47];
        }
        while (P < nsort) P <<= 1;
        for (int i = nsort + t; i < P; i += T) buf[i] = ~0ull;
        __syncthreads();
        if (nsort <= T) rank_sort_distinct(buf, nsort);
        else bitonic_sort(buf, P);
        if (NF >= k) {
            /* certify: every slice that kept only part of its finite elements
             * must have its last kept candidate strictly below the k-th s */
            const uint32_t kth = (uint32_t)(buf[k - 1] >> 32);
            if (t == 0) misc[55] = 0;
            __syncthreads();
            for (int h = t; h < G; h += T) {
                if ((int)sk[3 * h + 1] == 1) continue;
                const float l = key_value(sk[3 * h + 2]);
                if (!(desc_key((l - M) * R.inv_t) > kth)) misc[55] = 1;
            }
            __syncthreads();
            if (misc[55]) ok = false;
        } else {
            /* fewer finite entries than k: all of them plus the first k-NF
             * entries that are -inf, in index order */
            if (total != NF) ok = false;
        }
    }
    __syncthreads();
    if (!ok) {
        /* exact selection over the whole row in this workgroup */
        int np_row = build_patches(p, row, lg, mk, L, p.plan, V);
        R.np = np_row;
        uint32_t *hist2 = (uint32_t *)(buf + p.plan.kp);
        select_top_k(R, k, buf, p.plan.kp, hist2, L);
    } else if (NF < k) {
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
    if (k <= 64) {
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
template <bool CAP>
const void *topk_fn(int which) {
    using namespace dlk;
    switch (which) {
        case 0: return (const void *)topk_kernel<4, CAP>;
        case 1: return (const void *)topk_kernel<8, CAP>;
        case 2: return (const void *)topk_kernel<16, CAP>;
        case 3: return (const void *)topk_kernel<32, CAP>;
        default: return (const void *)topk_kernel<64, CAP>;
    }
}
}  // namespace

extern "C" int dlk_launch_topk_kernel(const dlk::TopkParams *f, int rows, int ept, size_t lds, hipStream_t stream) {
    using namespace dlk;
    static int set[2][5] = {{0, 0, 0, 0, 0}, {0, 0, 0, 0, 0}};
    const int which = ept == 4 ? 0 : ept == 8 ? 1 : ept == 16 ? 2 : ept == 32 ? 3 : ept == 64 ? 4 : -1;
    const int cap = f->p.cap > 0.0f ? 1 : 0;
    if (which < 0) return -1;
    const void *fn = cap ? topk_fn<true>(which) : topk_fn<false>(which);
    if (!set[cap][which]) {
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess) return -1;
        set[cap][which] = 1;
    }
    TopkParams fp = *f;
    void *args[] = {&fp};
    if (hipLaunchKernel(fn, dim3(f->G, rows), dim3(kTopkThreads), args, lds, stream) != hipSuccess) return -1;
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
