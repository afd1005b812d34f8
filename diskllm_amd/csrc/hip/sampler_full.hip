/*
 * sampler_full.hip -- fused full-vocabulary sampling (top-k off; min-p and
 * top-p on or off): src/sampler.c:136-234 with k = V, bit-exact, one HBM pass.
 *
 * A row is split over G workgroups of 512 threads, two per CU, all resident at
 * once (see dlk_launch_full_kernel); each keeps its slice in registers.  The
 * row is tied together by row barriers through relaxed agent-scope atomics
 * (every shared word is an atomic store/load; each writer waits for its stores
 * before it signals, so no cache-flushing fences are needed on this path; only
 * the split sums' bulk stores take an agent-scope release and acquire), and
 * finished by the last workgroup to arrive:
 *
 *   A  slice maxima            -> M (src/sampler.c:155-158)
 *   B  slice sums of e         -> inv = (float)(1/sum), certified: the sequential
 *                                 double sum (:177-181) lies within a proven
 *                                 relative bound of our sum, and inv is taken only
 *                                 if every value in that interval gives the same
 *                                 float (:182)
 *   B2 (min-p) slice sums of the survivors -> inv2, certified as inv is
 *                                 (:188-202)
 *   C  slice sums of p -> the slice holding the top-p crossing finds the
 *                                 certified cut x and inv3 from its candidate
 *                                 chunks and hands them to the others (:207-220)
 *   D  each slice's predicted contribution to the draw's float running sum
 *                              -> each workgroup's predicted exact start value
 *   last  every workgroup runs the draw's exact float running sum (:226-232,
 *         exact_scan.h) over its slice for 64 candidate start values around its
 *         prediction; the last workgroup of the row composes the slices from the
 *         row's exact start 0 and writes the token.
 *
 * A sum whose bound straddles a float rounding boundary (probability ~1e-3
 * per row) is found exactly by all G workgroups of the row (split_sum53: the
 * slices' exact_scan.h aggregates from registers, one walk by workgroup 0),
 * and the row goes on; a slice whose candidate chains do not cover the value
 * the composition reaches is walked by the last workgroup itself from that
 * value (draw_fix), and the composition resumes after it.  Only a wait that
 * gave up leaves a row undecided (DLK_STATUS_SYNC_TIMEOUT).
 */
#include "sampler_common.h"
#include "sampler_full.h"

namespace dlk {

DLK_DEV void at_st32(uint32_t *a, uint32_t v) { __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DLK_DEV void at_st64(uint64_t *a, uint64_t v) { __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
DLK_DEV uint32_t at_ld32(const uint32_t *a) {
    return __hip_atomic_load((uint32_t *)a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
DLK_DEV uint64_t at_ld64(const uint64_t *a) {
    return __hip_atomic_load((uint64_t *)a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}



/* Issues the loads of a slice: 16-byte groups of logits (an out-of-range group
 * reads the slice start instead) and, with a mask, each group's mask word. */
template <int EPT, int J0, int J1>
__device__ __forceinline__ void load_slice(const float *lg, const uint32_t *mk, int s0, int s1, int t, int T,
                                           float4 *raw, uint32_t *mwd) {
#pragma unroll
    for (int j4 = J0; j4 < J1; j4++) {
        const int i0 = s0 + 4 * (t + j4 * T);
        raw[j4] = *(const float4 *)(lg + (i0 < s1 ? i0 : s0));
        mwd[j4] = (mk && i0 < s1) ? mk[i0 >> 5] : 0xffffffffu;
    }
}


constexpr int kClassNanPosInf = 1 | 2 | 512;       /* signalling NaN, quiet NaN, +inf */

DLK_DEV float wave_max(float v) { return wave_max_dpp(v); }

/* Published words carry kReady (bit 63; every value stored in them leaves it
 * clear) once written, so a reader polls the data itself instead of a separate
 * arrival counter: one round trip less per barrier.  The row's words are zero
 * between launches. */
constexpr uint64_t kReady = 1ull << 63;

/* A draw range that starts past the top-p cut (no candidate base is this value:
 * a base is the bits of a non-negative float less 32, or 0). */
constexpr uint32_t kPastX = 0xffffffffu;

/* Waits until word idx[k] (k < K) of every workgroup of the row carries kReady
 * and copies it, flag cleared, into pc[h * kPubWords + idx[k]] for the whole
 * workgroup.  Wave 0 polls, a word per lane; the wait is bounded. */
template <uint32_t LIMIT, int K>
__device__ __forceinline__ void row_gather(const uint64_t *pubrow, int G, const int (&idx)[K], uint64_t *pc,
                                           uint32_t *status, int *tflag) {
    if (wave_id() == 0) {
        const int lane = lane_id(), n = G * K;
        for (int b = 0; b < n; b += 64) {
            const int q = b + lane;
            const bool act = q < n;
            const int off = act ? (q / K) * kPubWords + idx[q % K] : 0;
            uint64_t w = 0;
            uint32_t spins = 0;
            while (true) {
                if (act && !(w & kReady)) w = at_ld64(&pubrow[off]);
                if (ballot(act && !(w & kReady)) == 0) break;
                if (++spins > LIMIT) {
                    if (lane == 0) {
                        if (status) atomicOr(status, DLK_STATUS_SYNC_TIMEOUT);
                        *tflag = 1;
                    }
                    break;
                }
            }
            if (act) pc[off] = w & ~kReady;
        }
    }
    __syncthreads();
}

/* Last workgroup of the row to leave returns the row's sync and published words to zero. */
__device__ __forceinline__ void row_exit(uint32_t *sync, uint64_t *pubrow, int G) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x < 64) {
        uint32_t old = 0;
        if (threadIdx.x == 0) old = __hip_atomic_fetch_add(&sync[kSyncExit], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = (uint32_t)__builtin_amdgcn_readfirstlane((int)old);
        if (old == (uint32_t)(G - 1)) {
            for (int i = threadIdx.x; i < G * kPubWords; i += 64) at_st64(&pubrow[i], 0ull);
            for (int i = threadIdx.x; i < kSyncWords; i += 64) at_st32(&sync[i], 0u);
        }
    }
}

/* Exclusive scan of P[0..n) in place, P[n] = total (deterministic order). */
__device__ __forceinline__ void block_excl_scan(double *P, int n, double *red) {
    const int lane = lane_id(), w = wave_id(), T = blockDim.x, t = threadIdx.x;
    const int per = (n + T - 1) / T;
    const int b0 = t * per, b1 = min(n, b0 + per);
    double loc = 0.0;
    for (int c = b0; c < b1; c++) loc += P[c];
    const double inc = wave_incl_scan_d(loc);
    if (lane == 63) red[w] = inc;
    __syncthreads();
    /* wave bases: a scan of the wave totals, one per lane */
    const double wt = wave_incl_scan_d(lane < T / 64 ? red[lane] : 0.0);
    const double wbase = w > 0 ? __longlong_as_double((long long)readlane64((uint64_t)__double_as_longlong(wt), w - 1)) : 0.0;
    double run = wbase + inc - loc;
    __syncthreads();
    for (int c = b0; c < b1; c++) { double v = P[c]; P[c] = run; run += v; }
    if (t == T - 1) P[n] = run;
    __syncthreads();
}

/* e = expf((v - M) * inv_t) in place; returns the thread's e total in double
 * and stores each
 * chunk's e sum, rounded to float and summed in float, at ce[chunk]
 * (relative error below 5 * 2^-24). */
template <int EPT>
__device__ __forceinline__ double exp_slice(float (&v)[EPT], float M, float inv_t, const uint64_t *tab, double *ce,
                                            int t, int T) {
    const int lane = lane_id();
    double tsum = 0.0;
#pragma unroll
    for (int j4 = 0; j4 < EPT / 4; j4++) {
        /* four at a time, each group summed at once: enough independent work
         * to hide latency without widening live ranges into spills */
        double d = 0.0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float e = dlk_expf_glibc_core(fmaxf((v[4 * j4 + k] - M) * inv_t, -200.0f), tab);
            v[4 * j4 + k] = e;
            d = k == 0 ? (double)e : d + (double)e;
        }
        tsum += d;
        const float fs = row_scan_f((float)d);
        if ((lane & 15) == 15) ce[(t + j4 * T) >> 4] = (double)fs;
        __builtin_amdgcn_sched_barrier(0);
    }
    return tsum;
}

/* Inclusive prefix of per-thread 64-bit values in thread order (red: 16 words). */
DLK_DEV uint64_t block_incl_prefix_u64(uint64_t v, uint64_t *red) {
    const int lane = lane_id(), w = wave_id();
    const uint64_t inc = wave_incl_scan_u64(v);
    if (lane == 63) red[w] = inc;
    __syncthreads();
    const uint64_t wt = wave_incl_scan_u64(lane < (int)(blockDim.x / 64) ? red[lane] : 0ull);
    const uint64_t base = w > 0 ? readlane64(wt, w - 1) : 0ull;
    __syncthreads();
    return base + inc;
}

/* The draw's per-slice data in LDS (see full_kernel): segments, run
 * increments, staged chunks and candidate tables. */
struct DrawView {
    const int4 *seg;
    const uint64_t *rtot;
    const int *smap;
    const uint32_t *spx;
    const int2 *tab;
    const uint32_t *tbase;
    int ntab, nch_loc, s0;
    float thr_f;
};

/* One segment s of the draw for the lane's running value (bits cb): a run adds
 * its increments (exact while the value stays in the run's binade), an
 * element-level chunk is a table lookup.  tok becomes the token on a crossing,
 * or -2 when unresolved (a value outside what the prediction covers).  (Code
 * that let a lane sum a chunk outside its table itself, even out of this path
 * and never run, made every launch 17 us slower, so a value outside a table is
 * unresolved here and the tables are recentred on the refined starts.) */
__device__ __forceinline__ void draw_step(const DrawView &dv, int s, uint32_t &cb, int &tok) {
    const int4 sg = dv.seg[s];
    const int sx = sg.x, sy = sg.y, sz = sg.z, sw = sg.w;
    const float thr_f = dv.thr_f;
    if (sx == kZeroBinade) return;
    if (sx != kInvalidBinade) {
        /* run [sy, sw) on the grid of binade sx: exact integer steps
         * on the value's bits while it stays in the binade */
        const uint32_t R = (uint32_t)sz;
        const bool inb = (cb >> 23) == (uint32_t)(sx + 127) && (cb & 0x7fffffu) + R < 0x800000u;
        if (!inb) {
            tok = -2;
        } else if (u2f(cb + R) >= thr_f) {
            /* the crossing is in this run: its chunk by bisection on
             * the increments to the run's end, then its element */
            const uint64_t R0 = dv.rtot[sy];
            int lo = sy, hi = sw - 1;
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                const uint64_t after = mid + 1 < sw ? dv.rtot[mid + 1] : 0ull;
                if (u2f(cb + (uint32_t)(R0 - after)) >= thr_f) hi = mid;
                else lo = mid + 1;
            }
            const int sl = dv.smap[lo];
            tok = -2;
            if (sl >= 0) {
                /* the first element whose running value (the chunk's
                 * start plus its increment prefix, on one grid) reaches
                 * thr_f: a bisection on the prefixes */
                const uint32_t need = f2u(thr_f) - (cb + (uint32_t)(R0 - dv.rtot[lo]));
                const uint32_t *px = dv.spx + sl * 64;
                int ea = 0, eb = 63;
                while (ea < eb) {
                    const int em = (ea + eb) >> 1;
                    if (px[em] >= need) eb = em;
                    else ea = em + 1;
                }
                tok = dv.s0 + 64 * lo + ea;
            }
        } else {
            cb += R;
        }
    } else {
        /* element-level chunk sy: its table sz */
        const uint32_t bse = sz < dv.ntab ? dv.tbase[sz] : 0xffffffffu;
        const uint32_t d = cb - bse;
        if (bse == 0xffffffffu || d >= 64u) {
            tok = -2;
        } else {
            const int2 te = dv.tab[sz * 64 + (int)d];
            if (te.y >= 0) tok = dv.s0 + 64 * sy + te.y;
            else cb = (uint32_t)te.x;
        }
    }
}

/* Values of the row for the element-level steps of the split sum's walk. */
struct QRow {
    const float *q;
    DLK_DEV float operator()(int i) const { return q[i]; }
};

/* A double running sum over the whole row (the softmax sum, src/sampler.c:
 * 177-181, or the top-p cumulation, :207-215) that the certified bound could
 * not decide, run by all G workgroups of the row: each builds the exact_scan.h
 * aggregates of its slice from the values v in its registers (a chunk is 16
 * lanes of 4 values: a pair scan over a DPP row; a group is 64 chunks, from
 * LDS) under binades predicted from the approximate prefix Pb + pk * ce[c],
 * stores them and the values in the row's fallback region and signals on
 * sync[sw]; workgroup 0 then walks the row (resolve) and publishes the running
 * value after the threshold element (has_thr) or after the last, and the
 * position, in its words pw and pw + 1.  The stores are plain: each workgroup
 * waits for them and makes them visible at agent scope before it signals, and
 * the walker acquires after the signals are in.  Every workgroup returns the
 * same (pos, value), or false when a wait gave up (status flagged, misc[6]). */
template <uint32_t LIMIT, int EPT, bool POS = false>
__device__ __forceinline__ bool split_sum53(const float (&v)[EPT], double Pb, double pk, const double *ce,
                                            const FullParams &f, int row, int g, int s0, int s1, bool has_thr,
                                            double thr, int sw, int pw, uint32_t *sync, uint64_t *pubrow,
                                            uint64_t *la0, uint64_t *la1, int *lbh, int *misc, double *md,
                                            int &pos, double &value) {
    const int t = threadIdx.x, lane = lane_id(), w = wave_id(), T = kFullThreads;
    const int V = f.p.V, G = f.G;
    unsigned char *fbr = f.fb + (int64_t)row * f.fb_bytes;
    const Aggs A = make_aggs(fbr, V);
    float *qb = (float *)(fbr + f.fb_q_off);
    const int nchr = (V + 63) >> 6, ngr = (nchr + 63) >> 6, cb0 = s0 >> 6;
    /* POS: the positive part of v (the caller negates the entries that count as 0) */
    auto val = [](float a) { return POS ? (a > 0.0f ? a : 0.0f) : a; };
#pragma unroll
    for (int j4 = 0; j4 < EPT / 4; j4++) {
        const int u = t + j4 * T, lc = u >> 4;
        const float q0 = val(v[4 * j4]), q1 = val(v[4 * j4 + 1]), q2 = val(v[4 * j4 + 2]), q3 = val(v[4 * j4 + 3]);
        if (s0 + 4 * u < s1) *(float4 *)&qb[s0 + 4 * u] = make_float4(q0, q1, q2, q3);
        const int bs = predict_binade<53>(Pb + pk * ce[lc]);
        const int be = predict_binade<53>(Pb + pk * ce[lc + 1]);
        const int ue = bs - 52;
        Pair x = increment(q0, ue);
        x = compose(x, increment(q1, ue));
        x = compose(x, increment(q2, ue));
        x = compose(x, increment(q3, ue));
        x = compose(dpp_pair<kDppRowShr1>(x), x);
        x = compose(dpp_pair<kDppRowShr2>(x), x);
        x = compose(dpp_pair<kDppRowShr4>(x), x);
        x = compose(dpp_pair<kDppRowShr8>(x), x);
        if ((lane & 15) == 15) {
            const int b = bs == be ? bs : kInvalidBinade;
            la0[lc] = x.a0; la1[lc] = x.a1; lbh[lc] = b;
            if (cb0 + lc < nchr) { A.a0[cb0 + lc] = x.a0; A.a1[cb0 + lc] = x.a1; A.bh[cb0 + lc] = b; }
        }
    }
    __syncthreads();
    for (int lg = w; lg < EPT * T / 4096; lg += T / 64) {
        const int gg = (s0 >> 12) + lg;
        if (gg >= ngr) continue;
        const int c = lg * 64 + lane;
        const bool in = cb0 + c < nchr;
        const int b0 = lbh[lg * 64];
        if (ballot(in && lbh[c] != b0) != 0 || b0 == kInvalidBinade) {
            if (lane == 0) A.gbh[gg] = kInvalidBinade;
            continue;
        }
        Pair x = in ? Pair{la0[c], la1[c]} : Pair{0, 0};
        x = wave_incl_scan(x, lane);
        if (lane == 63) { A.ga0[gg] = x.a0; A.ga1[gg] = x.a1; A.gbh[gg] = b0; }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        __hip_atomic_fetch_add(&sync[sw], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (w == 0) {
        uint64_t wv = kReady | 0x7ff8000000000000ull, wp = kReady;
        uint32_t spins = 0;
        bool got = true;
        if (g == 0) {
            while (at_ld32(&sync[sw]) < (uint32_t)G)
                if (++spins > LIMIT) { got = false; break; }
            if (got) {
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
                const ResolveOut<53> o = resolve<53>(V, QRow{qb}, A, has_thr, thr);
                wv = d2u(o.value) | kReady;
                wp = (uint64_t)(uint32_t)o.pos | kReady;
            }
            if (lane == 0) { at_st64(&pubrow[pw + 1], wp); at_st64(&pubrow[pw], wv); }
        } else {
            while (!((wv = at_ld64(&pubrow[pw])) & kReady))
                if (++spins > LIMIT) { got = false; break; }
            if (got) wp = at_ld64(&pubrow[pw + 1]);
        }
        if (lane == 0) {
            const double val = u2d(wv & ~kReady);
            if (!got) {
                if (f.p.status) atomicOr(f.p.status, DLK_STATUS_SYNC_TIMEOUT);
                misc[6] = 1;
            }
            misc[31] = got && !__builtin_isnan(val);
            misc[30] = (int)(uint32_t)wp;
            md[2] = val;
        }
    }
    __syncthreads();
    pos = misc[30];
    value = md[2];
    const bool ok = misc[31] != 0;
    __syncthreads();
    return ok;
}

/* The draw's float running sum (src/sampler.c:225-233) over slice h alone from
 * its exact start value cb (float bits), for the row's last workgroup when the
 * slice's candidate chains do not cover the value its composition reached.
 * The slice's final probabilities are recomputed from the logits as the slice
 * computed them (its patches from the row's history list), the exact_scan.h
 * aggregates built from registers into LDS (la0/la1/lbh: a chunk per DPP row of
 * 16 lanes; groups in gm) under binades predicted from cb plus the chunks'
 * float sums (cs: nch + 1 doubles), the values stored at the row's value
 * region for the walk's element steps, and wave 0 walks the slice up to x
 * (resolve).  pos: the first slice index whose running value reaches thr_f,
 * or -1; endb: the running value's bits after the slice's last entry up to x. */
template <int EPT, bool CAP>
__device__ __forceinline__ void draw_fix(const FullParams &f, int row, int h, uint32_t cb, int x, float M, float inv,
                                         bool keep_all, float inv2, float inv3, float thr_f, Lds &L, const float *lg,
                                         const uint32_t *mk, double *cs, uint64_t *la0, uint64_t *la1, int *lbh,
                                         unsigned char *gm, int *misc, int &pos, uint32_t &endb) {
    const RowParams &p = f.p;
    const int t = threadIdx.x, lane = lane_id(), w = wave_id(), T = kFullThreads;
    const int V = p.V, S = f.S, nch = S / 64;
    const int s0 = h * S, s1 = min(V, s0 + S);
    const int n = min(s1, x + 1) - s0;
    Row R;
    R.lg = lg; R.mk = mk; R.V = V; R.pid = L.pid; R.pval = L.pval; R.pflag = L.pflag;
    R.M = M; R.inv_t = p.inv_temp; R.maxv = 0.0f; R.tab = L.tab; R.cap = CAP ? p.cap : 0.0f;
    R.np = build_patches(p, row, lg, mk, L, p.plan, V);
    /* each group's values (a thread reads back its own stores below) and the
     * chunks' float sums, two groups' loads in flight at a time */
    float *qb = (float *)(f.fb + (int64_t)row * f.fb_bytes + f.fb_q_off);
#pragma unroll 1
    for (int jb = 0; jb < EPT / 4; jb += 2) {
        float4 raw[2];
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int i0 = s0 + 4 * (t + (jb + k) * T);
            raw[k] = i0 < s1 ? *(const float4 *)(lg + i0) : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        }
#pragma unroll
        for (int k = 0; k < 2; k++) {
            const int u = t + (jb + k) * T, i0 = s0 + 4 * u;
            const float xs[4] = {raw[k].x, raw[k].y, raw[k].z, raw[k].w};
            float q[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int i = i0 + c;
                const float y = i < s1 ? prepared_from(R, i, xs[c]) : -INFINITY;
                float v = dlk_expf_glibc_core(fmaxf((y - M) * p.inv_temp, -200.0f), L.tab) * inv;
                if (p.minp_on) v = keep_all || v >= p.min_p ? v * inv2 : 0.0f;
                q[c] = i <= x ? (p.topp_on ? v * inv3 : v) : 0.0f;
            }
            *(float4 *)&qb[4 * u] = make_float4(q[0], q[1], q[2], q[3]);
            const float fs = row_scan_f((q[0] + q[1]) + (q[2] + q[3]));
            if ((lane & 15) == 15) cs[u >> 4] = (double)fs;
        }
    }
    __syncthreads();
    block_excl_scan(cs, nch, L.red);
    const double c0 = (double)u2f(cb);
#pragma unroll 1
    for (int j4 = 0; j4 < EPT / 4; j4++) {
        const int u = t + j4 * T, lc = u >> 4;
        const float4 q4 = *(const float4 *)&qb[4 * u];
        const int bs = predict_binade<24>(c0 + cs[lc]);
        const int be = predict_binade<24>(c0 + cs[lc + 1]);
        const Pair xp = row_chunk_pair(q4.x, q4.y, q4.z, q4.w, bs - 23);
        if ((lane & 15) == 15) { la0[lc] = xp.a0; la1[lc] = xp.a1; lbh[lc] = bs == be ? bs : kInvalidBinade; }
    }
    __syncthreads();
    uint64_t *ga0 = (uint64_t *)gm, *ga1 = ga0 + 16;
    int *gbh = (int *)(ga1 + 16);
    const int nchn = (n + 63) >> 6, ngn = (nchn + 63) >> 6;
    for (int gi = w; gi < ngn; gi += T / 64) {
        const int c = gi * 64 + lane;
        const bool in = c < nchn;
        const int b0 = lbh[gi * 64];
        if (ballot(in && lbh[c] != b0) != 0 || b0 == kInvalidBinade) {
            if (lane == 0) gbh[gi] = kInvalidBinade;
            continue;
        }
        Pair xp = in ? Pair{la0[c], la1[c]} : Pair{0, 0};
        xp = wave_incl_scan(xp, lane);
        if (lane == 63) { ga0[gi] = xp.a0; ga1[gi] = xp.a1; gbh[gi] = b0; }
    }
    /* the values are read back by wave 0: every store done, the cache lines
     * this compute unit may hold of the region dropped */
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (w == 0) {
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        Aggs A;
        A.a0 = la0; A.a1 = la1; A.bh = lbh; A.ga0 = ga0; A.ga1 = ga1; A.gbh = gbh; A.P = cs;
        ResolveOut<24> o{-1, u2f(cb)};
        if (n > 0) o = resolve<24>(n, QRow{qb}, A, true, (double)thr_f, u2f(cb));
        if (lane == 0) { misc[26] = o.pos; misc[27] = (int)f2u(o.value); }
    }
    __syncthreads();
    pos = misc[26];
    endb = (uint32_t)misc[27];
    __syncthreads();
}

/* NOWAIT (a test instance): every wait gives up at its first poll that finds a
 * word not yet written, which sets DLK_STATUS_SYNC_TIMEOUT. */
/* HP: history ids per thread (1 up to kFullThreads ids; 2 up to twice that,
 * an instance of its own so that the common case keeps its registers). */
template <int EPT, bool CAP, bool NOWAIT = false, int HP = 1>
__global__ __launch_bounds__(kFullThreads) void full_kernel(FullParams f) {
    constexpr uint32_t kLimit = NOWAIT ? 0u : kFullSpinLimit;
    extern __shared__ __align__(16) unsigned char smem[];
    const RowParams &p = f.p;
    const int G = f.G, T = kFullThreads;
    /* a row's workgroups on one XCD: dispatch deals workgroup b to XCD b % 8,
     * so when the grid holds whole groups of eight rows, the rows of b % 8 are
     * those of XCD b % 8.  Among an XCD's blocks, the first half are the first
     * block of their CU and the second half the second (two per CU), and the
     * second block of a CU runs behind the first (older waves win issue): so a
     * row takes half its slices from each half, rather than all of a row's
     * slices running behind.  The first half takes slice 0 (the start of the
     * draw, the row's longest draw phase) and the last G/2 - 1 slices (where
     * the top-p crossing of a spread-out row lies, which the others wait for) */
    int row, g;
    if (gridDim.x % (8 * G) == 0 && (G & 1) == 0) {
        /* k: the block's place among its XCD's blocks; the first and second
         * halves of them are the first and second block of their CUs: each row
         * takes G/2 slices from each half */
        const int k = blockIdx.x >> 3, R = (int)(gridDim.x >> 4), h = G >> 1;
        const int k2 = k < R ? k : k - R;
        row = (k2 / h) * 8 + (blockIdx.x & 7);
        const int i = k2 % h;
        g = k < R ? (i == 0 ? 0 : G - h + i) : 1 + i;
    } else if (gridDim.x % (8 * G) == 0) {
        const int k = blockIdx.x >> 3;
        row = (k / G) * 8 + (blockIdx.x & 7);
        g = k % G;
    } else {
        row = blockIdx.x / G;
        g = blockIdx.x % G;
    }
    const int t = threadIdx.x, lane = lane_id();
    const int V = p.V, S = f.S, nch = S / 64;
    const int s0 = g * S, s1 = min(V, s0 + S);
    const float *lg = p.logits + (int64_t)row * p.ld;
    const uint32_t *mk = nullptr;
    if (p.mask) mk = p.mask + (int64_t)(p.mask_row ? p.mask_row[row] : row) * p.mask_ld;
    uint32_t *sync = f.sync + (int64_t)row * kSyncWords;
    uint64_t *pubrow = f.pub + (int64_t)row * G * kPubWords;
    uint64_t *mypub = pubrow + (int64_t)g * kPubWords;

    Lds L = make_lds(smem, p.plan);
    unsigned char *q = L.region;
    uint32_t *sbits = (uint32_t *)carve(q, (size_t)(S / 32) * 4);
    double *ce = (double *)carve(q, (size_t)(nch + 1) * 8);      /* e prefix; later the contributions' prefix */
    int *cbh = (int *)carve(q, (size_t)nch * 4);                 /* chunk binade, kInvalidBinade or kZeroBinade */
    uint32_t *ca = (uint32_t *)carve(q, (size_t)nch * 4);        /* chunk increments on that grid */
    uint64_t *rtot = (uint64_t *)carve(q, (size_t)nch * 8);      /* increments to the end of the run */
    int *rend = (int *)carve(q, (size_t)nch * 4);                /* scratch: last chunk of segment s */
    uint64_t *rpre = (uint64_t *)carve(q, (size_t)nch * 8);      /* scratch: increments up to it */
    double *Pc = (double *)carve(q, (size_t)(nch + 1) * 8);      /* predicted running value */
    int *smap = (int *)carve(q, (size_t)nch * 4);                /* staged slot of each chunk or -1 */
    float *svals = (float *)carve(q, (size_t)f.stage_cap * 64 * 4);
    uint32_t *spx = (uint32_t *)carve(q, (size_t)f.stage_cap * 64 * 4);   /* staged run chunks: increment prefixes */
    int2 *elist = (int2 *)carve(q, (size_t)nch * 8);             /* element-level chunks {chunk, slot} */
    int *elc = (int *)carve(q, (size_t)nch * 4);                 /* element-level chunks before chunk c */
    int4 *seg = (int4 *)carve(q, (size_t)nch * 16);              /* the draw's segments */
    int2 *tab = (int2 *)carve(q, (size_t)kMaxTabs * 64 * 8);     /* candidate tables {end bits, crossing} */
    uint32_t *tbase = (uint32_t *)carve(q, (size_t)kMaxTabs * 4);  /* each table's first candidate */
    int2 *rres = (int2 *)carve(q, (size_t)(kFullThreads / 64) * 64 * 8);   /* each wave's range: {end bits, token} */
    uint32_t *rbase = (uint32_t *)carve(q, (size_t)(kFullThreads / 64) * 4);  /* each range's first candidate */
    uint64_t *pc = (uint64_t *)carve(q, (size_t)G * kPubWords * 8);   /* published words, cached */
    int *misc = (int *)carve(q, 64 * 4);
    double *md = (double *)carve(q, 16 * 8);
    if (t < 32) L.tab[t] = kExp2Tab[t];

    /* ---- history first: the row's ids (HP per thread; the host keeps the
     *      direct history within the workgroup) and, for an id inside this
     *      slice, its logit and mask word, gathered before the bulk loads ----- */
    const int32_t *hist = nullptr;
    int nh = 0;
    if (p.hist_off) {
        hist = p.hist_ids + p.hist_off[row];
        nh = p.hist_off[row + 1] - p.hist_off[row];
    }
    int hid[HP];
    float gx[HP];
    uint32_t gm[HP];
#pragma unroll
    for (int k = 0; k < HP; k++) {
        hid[k] = t + k * T < nh ? hist[t + k * T] : -1;
        gx[k] = 0.0f;
        gm[k] = 0xffffffffu;
        if (hid[k] >= s0 && hid[k] < s1) {
            gx[k] = lg[hid[k]];
            if (mk) gm[k] = mk[hid[k] >> 5];
        }
    }

    /* ---- stream the slice into registers: every load issued before any use */
    float4 raw[EPT / 4];
    uint32_t mwd[EPT / 4];
    load_slice<EPT, 0, EPT / 4>(lg, mk, s0, s1, t, T, raw, mwd);

    if (DLK_COLD(nh > p.plan.hcap || nh > HP * T)) {    /* (the host keeps both) */
        if (g == 0 && t == 0) {
            p.out_ids[row] = -1;
            if (p.status) atomicOr(p.status, DLK_STATUS_HISTORY_TOO_LONG);
        }
        row_exit(sync, pubrow, G);
        return;
    }
    /* ---- penalty patches of the ids inside this slice ------------------- */
    /* The slice's history entries are counted in an LDS hash table of their
     * ids (open addressing over 2 * hcap >= 2 * nh slots: every id has its
     * slot and probes stay short; keys span hsort and pid, counts pval and
     * pcnt, carved back to back), and a bit per slice element marks the ids.
     * A patch depends only on the id's count, its logit and its mask word, so
     * the entry that inserted the id computes it once every count is in, from
     * the logit and mask word it gathered before the bulk loads, and leaves it
     * in the slot in place of the count (in straight-line code: the use of the
     * gathered values then waits only for those loads, and the merge below
     * takes the slice as it lands).  Two block barriers, where ranking the
     * marked ids by a scan of the bitmap took six. */
    const int nw = S / 32;
    int *hkey = (int *)L.hsort;
    uint32_t *hcnt = (uint32_t *)L.pval;
    const int hslots = 2 * p.plan.hcap;            /* a power of two */
    const int hshift = 32 - (31 - __clz(hslots));
    for (int i = t; i < nw; i += T) sbits[i] = 0;
    for (int i = t; i < hslots; i += T) { hkey[i] = -1; hcnt[i] = 0u; }
    if (t == 0) { misc[5] = 0; misc[6] = 0; }     /* a NaN / +inf entry; a wait that gave up */
    __syncthreads();
    int oslot[HP];
#pragma unroll
    for (int k = 0; k < HP; k++) {
        oslot[k] = -1;
        const int id = hid[k];
        if (id >= s0 && id < s1) {
            uint32_t h = ((uint32_t)id * 0x9E3779B1u) >> hshift;
            for (int probe = 0; probe < hslots; probe++) {
                const int old = atomicCAS(&hkey[h], -1, id);
                if (old == -1) { oslot[k] = (int)h; atomicOr(&sbits[(id - s0) >> 5], 1u << ((id - s0) & 31)); }
                if (old == -1 || old == id) break;
                h = (h + 1) & (uint32_t)(hslots - 1);
            }
            atomicAdd(&hcnt[h], 1u);
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < HP; k++) {
        if (oslot[k] >= 0) {
            float x = gx[k];
            if (CAP) x = dlk_softcap_glibc(x, p.cap);
            if (!((gm[k] >> (hid[k] & 31)) & 1u)) x = -INFINITY;
            hcnt[oslot[k]] = __float_as_uint(penalize(x, (int)hcnt[oslot[k]], p));
        }
    }
    /* the patch of a marked id */
    auto hpatch = [&](int id) {
        uint32_t h = ((uint32_t)id * 0x9E3779B1u) >> hshift;
        while (hkey[h] != id) h = (h + 1) & (uint32_t)(hslots - 1);
        return __uint_as_float(hcnt[h]);
    };
    const uint64_t st = xorshift64(p.rng[row]);     /* one uniform per sampled row (src/sampler.c:225) */
    const float r = rand_f32_from(st);
    __syncthreads();

    /* masked entries -inf, patched entries their penalised value; the row is a
     * whole number of 4-element groups (the host routes other rows elsewhere) */
    float v[EPT];
    float tm = -INFINITY;
    bool bad = false;                              /* NaN or +inf after penalties */
#pragma unroll
    for (int j4 = 0; j4 < EPT / 4; j4++) {
        const int i0 = s0 + 4 * (t + j4 * T);
        float xs[4] = {raw[j4].x, raw[j4].y, raw[j4].z, raw[j4].w};
        if (CAP) {
#pragma unroll
            for (int c = 0; c < 4; c++) xs[c] = dlk_softcap_glibc(xs[c], p.cap);
        }
        if (i0 >= s1) xs[0] = xs[1] = xs[2] = xs[3] = -INFINITY;
        if (mk) {
            const uint32_t mw = mwd[j4] >> (i0 & 31);
#pragma unroll
            for (int c = 0; c < 4; c++)
                if (!((mw >> c) & 1u)) xs[c] = -INFINITY;
        }
        const int li0 = i0 - s0;
        const uint32_t pb = i0 < s1 ? (sbits[li0 >> 5] >> (li0 & 31)) & 0xFu : 0u;
        if (pb) {
            /* the patched ids of the group (src/sampler.c:21-52) */
#pragma unroll
            for (int c = 0; c < 4; c++)
                if ((pb >> c) & 1u) xs[c] = hpatch(i0 + c);
        }
#pragma unroll
        for (int c = 0; c < 4; c++) {
            v[j4 * 4 + c] = xs[c];
            tm = fmaxf(tm, xs[c]);
            bad |= __builtin_amdgcn_class(xs[c], kClassNanPosInf);
        }
    }
    if (ballot(bad) != 0 && lane == 0) misc[5] = 1;

    /* ---- A: row maximum -------------------------------------------------- */
    tm = wave_max(tm);
    if (lane == 0) ((float *)L.red)[wave_id()] = tm;
    __syncthreads();
    if (wave_id() == 0) {
        tm = wave_max_dpp(lane < T / 64 ? ((const float *)L.red)[lane] : -INFINITY);
        if (lane == 0) at_st64(&mypub[kPubMax], (uint64_t)f2u(tm) | ((uint64_t)(misc[5] != 0) << 32) | kReady);
    }
    {
        const int idx[1] = {kPubMax};
        row_gather<kLimit>(pubrow, G, idx, pc, p.status, &misc[6]);
    }
    float M = -INFINITY;
    bool row_bad = false;
    for (int h = 0; h < G; h++) {
        M = fmaxf(M, u2f((uint32_t)pc[h * kPubWords + kPubMax]));
        row_bad |= (pc[h * kPubWords + kPubMax] >> 32) != 0;
    }
    if (g == 0 && t == 0) p.rng[row] = st;                  /* every workgroup has read it */
    const int n_out = p.n_out;
    if (DLK_COLD(row_bad || !(M > -INFINITY))) {
        /* every entry -inf, or a NaN / +inf entry: the softmax sum is NaN, no
         * comparison with it holds, and the draw falls through to index V-1 */
        if (g == 0) {
            if (t == 0) p.out_ids[row] = V - 1;
            for (int j = t; j < n_out; j += T) {
                int64_t o = (int64_t)row * n_out + j;
                if (p.out_cand_ids) p.out_cand_ids[o] = j < V ? j : -1;
                if (p.out_cand_probs) p.out_cand_probs[o] = NAN;
                if (p.out_cand_logprobs) p.out_cand_logprobs[o] = NAN;
            }
        }
        row_exit(sync, pubrow, G);
        return;
    }

    /* ---- e and its slice sums ------------------------------------------- */
    /* e in place; the slice's e total in double (a bound-certified sum, any
     * order), and float chunk sums, which only predict the top-p candidates */
    const float inv_t = p.inv_temp;
    double tsum = exp_slice<EPT>(v, M, inv_t, L.tab, ce, t, T);
    tsum = wave_incl_scan_d(tsum);
    if (lane == 63) L.red[32 + wave_id()] = tsum;
    __syncthreads();
    /* the slice's total is published first; the chunk prefix is built while
     * the other slices' totals arrive */
    if (t == 0) {
        double e_tot = 0.0;
        for (int w2 = 0; w2 < T / 64; w2++) e_tot += L.red[32 + w2];
        at_st64(&mypub[kPubE], d2u(e_tot) | kReady);
    }
    block_excl_scan(ce, nch, L.red);                        /* ce[c]: approximate e prefix at chunk c */

    /* ---- B: softmax normaliser ------------------------------------------ */
    {
        const int idx[1] = {kPubE};
        row_gather<kLimit>(pubrow, G, idx, pc, p.status, &misc[6]);
    }
    double Sapx = 0.0;
    for (int h = 0; h < G; h++) Sapx += u2d(pc[h * kPubWords + kPubE]);
    /* |sequential - exact| <= V u sum; |ours - exact| <= 64 u sum (summation depth) */
    const double U = 0x1p-53;
    const double eps_s = ((double)V + 64.0) * U * 1.01 + 4.0 * U;
    const float inv_a = (float)(1.0 / (Sapx * (1.0 + eps_s)));
    const float inv_b = (float)(1.0 / (Sapx * (1.0 - eps_s)));
    bool ok = inv_a == inv_b && !f.force_exact;
    float inv = inv_a;
    if (DLK_COLD((inv_a != inv_b || f.force_exact) && !misc[6])) {
        /* the bound straddles a float rounding boundary: the sequential sum
         * itself, split over the row's workgroups */
        double Eb = 0.0;
        for (int h = 0; h < g; h++) Eb += u2d(pc[h * kPubWords + kPubE]);
        int pos;
        double s1v;
        ok = split_sum53<kLimit, EPT>(v, Eb, 1.0, ce, f, row, g, s0, s1, false, 0.0, kSyncSplitE, kPubSplitE, sync,
                                      pubrow, rtot, rpre, cbh, misc, md, pos, s1v);
        inv = (float)(1.0 / s1v);
    }

    float inv3 = 1.0f;
    int x = V - 1;
    const bool topp = p.topp_on;
    double RWg = 0.0;                              /* exact-bounded p prefix before this slice */
    float pk = inv;                                /* prefix of the values at chunk c ~ pk * ce[c] */
    bool mp_all = true;                            /* min-p: every entry kept (none reaches min_p) */
    float mp_inv2 = 1.0f;                          /* min-p: the survivors' normaliser */
    if (ok) {
        /* ---- p and the slice's p total (double, any order) ------------------ */
#pragma unroll
        for (int j = 0; j < EPT; j++) v[j] = v[j] * inv;
        const bool want_cands = g == 0 && n_out > 0 && (p.out_cand_ids != nullptr || p.out_cand_probs != nullptr);
        if (DLK_COLD(want_cands)) {
#pragma unroll
            for (int j = 0; j < EPT; j++) {
                const int i = 4 * (t + (j / 4) * T) + (j & 3);
                if (i < n_out && i < V) {
                    int64_t o = (int64_t)row * n_out + i;
                    if (p.out_cand_ids) p.out_cand_ids[o] = i;
                    if (p.out_cand_probs) p.out_cand_probs[o] = v[j];
                }
            }
        }
        if (DLK_COLD(p.minp_on)) {
            /* ---- B2: min-p (src/sampler.c:188-202): the entries with p >= min_p
             *      survive, in index order (none: every entry stays); their
             *      double sum, certified as inv is, gives inv2.  v becomes
             *      p * inv2 for the entries kept and 0 for the others (a 0 moves
             *      neither the top-p sum nor the draw's), and ce the chunk prefix
             *      of v ------------------------------------------------------ */
            double s_sv = 0.0, s_all = 0.0;
            int n_sv = 0;
#pragma unroll
            for (int j = 0; j < EPT; j++) {
                const double d = (double)v[j];
                s_all += d;
                if (v[j] >= p.min_p) { s_sv += d; n_sv++; }
            }
            s_sv = wave_incl_scan_d(s_sv);
            s_all = wave_incl_scan_d(s_all);
            for (int m = 32; m >= 1; m >>= 1) n_sv += shfl_xor(n_sv, m);
            if (t == 0) misc[12] = 0;
            if (lane == 63) { L.red[wave_id()] = s_sv; L.red[32 + wave_id()] = s_all; }
            __syncthreads();
            if (lane == 0 && n_sv) atomicAdd(&misc[12], n_sv);
            __syncthreads();
            if (t == 0) {
                double a = 0.0, b = 0.0;
                for (int w2 = 0; w2 < T / 64; w2++) { a += L.red[w2]; b += L.red[32 + w2]; }
                at_st64(&mypub[kPubS2], d2u(a) | kReady);
                at_st64(&mypub[kPubA2], d2u(b) | kReady);
                at_st64(&mypub[kPubN2], (uint64_t)(uint32_t)misc[12] | kReady);
            }
            {
                const int idx[3] = {kPubS2, kPubA2, kPubN2};
                row_gather<kLimit>(pubrow, G, idx, pc, p.status, &misc[6]);
            }
            double S2 = 0.0, SA = 0.0;
            int64_t nkeep = 0;
            for (int h = 0; h < G; h++) {
                S2 += u2d(pc[h * kPubWords + kPubS2]);
                SA += u2d(pc[h * kPubWords + kPubA2]);
                nkeep += (int64_t)(uint32_t)pc[h * kPubWords + kPubN2];
            }
            const bool keep_all = nkeep == 0;
            const double Sx = keep_all ? SA : S2;
            const float i2a = (float)(1.0 / (Sx * (1.0 + eps_s)));
            const float i2b = (float)(1.0 / (Sx * (1.0 - eps_s)));
            float inv2 = i2a;
            if (DLK_COLD((i2a != i2b || f.force_exact) && !misc[6])) {
                /* the survivors' sum itself (src/sampler.c:198-199), split over
                 * the row's workgroups: an entry min-p drops adds 0 (negated
                 * here, the split takes the positive part), predicted from the
                 * survivors' chunk sums (in Pc, free until the draw) */
#pragma unroll
                for (int j = 0; j < EPT; j++)
                    if (!(keep_all || v[j] >= p.min_p)) v[j] = -v[j];
#pragma unroll
                for (int j4 = 0; j4 < EPT / 4; j4++) {
                    const float d = (fmaxf(v[4 * j4], 0.0f) + fmaxf(v[4 * j4 + 1], 0.0f)) +
                                    (fmaxf(v[4 * j4 + 2], 0.0f) + fmaxf(v[4 * j4 + 3], 0.0f));
                    const float fs = row_scan_f(d);
                    if ((lane & 15) == 15) Pc[(t + j4 * T) >> 4] = (double)fs;
                }
                __syncthreads();
                block_excl_scan(Pc, nch, L.red);
                double Sb = 0.0;
                for (int h = 0; h < g; h++) Sb += u2d(pc[h * kPubWords + (keep_all ? kPubA2 : kPubS2)]);
                int pos;
                double s2v;
                ok = split_sum53<kLimit, EPT, true>(v, Sb, 1.0, Pc, f, row, g, s0, s1, false, 0.0, kSyncSplitM,
                                                    kPubSplitM, sync, pubrow, rtot, rpre, cbh, misc, md, pos, s2v);
                inv2 = (float)(1.0 / s2v);
#pragma unroll
                for (int j = 0; j < EPT; j++) v[j] = fabsf(v[j]);
            } else if (i2a != i2b) {
                ok = false;
            }
            mp_all = keep_all;
            mp_inv2 = inv2;
#pragma unroll
            for (int j = 0; j < EPT; j++) v[j] = keep_all || v[j] >= p.min_p ? v[j] * inv2 : 0.0f;
#pragma unroll
            for (int j4 = 0; j4 < EPT / 4; j4++) {
                const float d = (v[4 * j4] + v[4 * j4 + 1]) + (v[4 * j4 + 2] + v[4 * j4 + 3]);
                const float fs = row_scan_f(d);
                if ((lane & 15) == 15) ce[(t + j4 * T) >> 4] = (double)fs;
            }
            __syncthreads();
            block_excl_scan(ce, nch, L.red);
            pk = 1.0f;
        }
        {
            double ps = 0.0;
#pragma unroll
            for (int j4 = 0; j4 < EPT / 4; j4++)
                ps += ((double)v[4 * j4] + (double)v[4 * j4 + 1]) + ((double)v[4 * j4 + 2] + (double)v[4 * j4 + 3]);
            ps = wave_incl_scan_d(ps);
            if (lane == 63) L.red[wave_id()] = ps;
            __syncthreads();
            if (t == 0) {
                double tot = 0.0;
                for (int w2 = 0; w2 < T / 64; w2++) tot += L.red[w2];
                at_st64(&mypub[kPubP], d2u(tot) | kReady);
                at_st64(&mypub[kPubP0], (g == 0 ? (uint64_t)f2u(v[0]) : 0ull) | kReady);
            }
        }

        /* ---- C: the slices' p totals -> the top-p cut x and its normaliser
         *      inv3 (src/sampler.c:205-220): the slice holding the crossing finds
         *      and certifies them and hands them to the others ----------------- */
        {
            const int idx[2] = {kPubP, kPubP0};
            row_gather<kLimit>(pubrow, G, idx, pc, p.status, &misc[6]);
        }
        for (int h = 0; h < g; h++) RWg += u2d(pc[h * kPubWords + kPubP]);
        const double U = 0x1p-53;
        int hx = -1;                               /* the slice that finds x */
        if (!topp) {
            /* no renormalisation (src/sampler.c:205) */
        } else if (p.top_p <= 0.0f) {
            x = 0;                                 /* cumul after the first entry */
            inv3 = (float)(1.0 / (double)u2f((uint32_t)pc[kPubP0]));
        } else {
            /* the first slice whose end prefix may reach tau; |ours - sequential|
             * within the bound e of the reference's double sum (src/sampler.c:209) */
            const double tau = p.topp_thr;
            double R = 0.0;
            bool amb = false;
            for (int h = 0; h < G && hx < 0; h++) {
                R += u2d(pc[h * kPubWords + kPubP]);
                const double e = ((double)min(V, (h + 1) * S) + 256.0) * U * 1.01 + 4.0 * U;
                if (R * (1.0 + e) >= tau) {
                    hx = h;
                    amb = R * (1.0 - e) < tau;     /* the crossing may be at its very end or beyond */
                }
            }
            if (hx < 0) {
                /* the whole row stays below top_p: nk = k (src/sampler.c:208-215) */
                const double e = ((double)V + 256.0) * U * 1.01 + 4.0 * U;
                const float a = (float)(1.0 / (R * (1.0 + e))), b = (float)(1.0 / (R * (1.0 - e)));
                if (a == b) inv3 = a;
                else ok = false;
            } else if (amb) {
                ok = false;
            }
        }
        if (ok && hx == g) {
            /* this slice holds the crossing: the chunks that may hold it, from the
             * e prefix (|p - e*inv| <= 2^-24 p each, the float chunk sums within
             * 5 * 2^-24, inv within 2^-24) */
            const double tau = p.topp_thr, dl = 0x1p-20;
            if (t == 0) misc[1] = 0;
            __syncthreads();
            for (int c = t; c < nch; c += T) {
                if (s0 + 64 * c >= s1) continue;
                const double lo = RWg + (double)pk * ce[c] * (1.0 - dl);
                const double hi = RWg + (double)pk * ce[c + 1] * (1.0 + dl);
                if (lo <= tau && tau <= hi) {
                    const int sl = atomicAdd(&misc[1], 1);
                    if (sl < kCandSlots) misc[2 + sl] = c;
                }
            }
            __syncthreads();
            const int ncand = misc[1];
            int okc = ncand >= 1 && ncand <= kCandSlots;
            int c0 = okc ? misc[2] : 0, c1 = okc && ncand == 2 ? misc[3] : -1;
            if (c1 >= 0 && c1 < c0) { const int tmp = c0; c0 = c1; c1 = tmp; }
            /* each candidate's exact prefix: the slice's values before it, summed
             * per thread and over the block; and its 64 values into LDS */
            double m0 = 0.0, m1 = 0.0;
            float *cv = svals;
#pragma unroll
            for (int j4 = 0; j4 < EPT / 4; j4++) {
                const int u = t + j4 * T;           /* 4-element group index */
                const double d = ((double)v[4 * j4] + (double)v[4 * j4 + 1]) + ((double)v[4 * j4 + 2] + (double)v[4 * j4 + 3]);
                if (u < 16 * c0) m0 += d;
                if (u < 16 * c1) m1 += d;
                const int cg = u >> 4;
                if (okc && (cg == c0 || cg == c1))
                    *(float4 *)&cv[(cg == c0 ? 0 : 64) + (u & 15) * 4] =
                        make_float4(v[4 * j4], v[4 * j4 + 1], v[4 * j4 + 2], v[4 * j4 + 3]);
            }
            m0 = wave_incl_scan_d(m0);
            m1 = wave_incl_scan_d(m1);
            if (lane == 63) { L.red[wave_id()] = m0; L.red[32 + wave_id()] = m1; }
            __syncthreads();
            if (wave_id() == 0) {
                double P0 = 0.0, P1 = 0.0;
                for (int w2 = 0; w2 < T / 64; w2++) { P0 += L.red[w2]; P1 += L.red[32 + w2]; }
                int xx = V - 1;
                double s3 = 0.0, eps3 = 0.0;
                bool found = false;
                for (int k = 0; k < 2 && okc && !found; k++) {
                    const int cg = k == 0 ? c0 : c1;
                    if (cg < 0) break;
                    const int i = s0 + cg * 64 + lane;
                    double Rv = i < V ? (double)cv[k * 64 + lane] : 0.0;
                    Rv = wave_incl_scan_d(Rv) + RWg + (k == 0 ? P0 : P1);
                    const double e = ((double)(i + 1) + 256.0) * U * 1.01 + 4.0 * U;
                    const int fl = first_lane(ballot(i < V && Rv * (1.0 + e) >= tau));
                    if (fl < 64) {
                        const double Rf = u2d(readlane64(d2u(Rv), fl));
                        const double ef = ((double)(s0 + cg * 64 + fl + 1) + 256.0) * U * 1.01 + 4.0 * U;
                        if (Rf * (1.0 - ef) >= tau) { found = true; xx = s0 + cg * 64 + fl; s3 = Rf; eps3 = ef; }
                        else okc = 0;
                    }
                }
                float i3 = 1.0f;
                if (!found) okc = 0;
                if (okc) {
                    const float a = (float)(1.0 / (s3 * (1.0 + eps3)));
                    const float b = (float)(1.0 / (s3 * (1.0 - eps3)));
                    if (a == b) i3 = a;
                    else okc = 0;
                }
                if (lane == 0) {
                    misc[8] = okc;
                    misc[9] = xx;
                    md[0] = (double)i3;
                    /* x in bits 0-30 (0x7fffffff: not certified), inv3 in 31-62 */
                    at_st64(&mypub[kPubX], (uint64_t)(okc ? (uint32_t)xx : 0x7fffffffu) |
                                               ((uint64_t)f2u(i3) << 31) | kReady);
                }
            }
            __syncthreads();
            ok = misc[8] != 0;
            x = misc[9];
            inv3 = (float)md[0];
        } else if (ok && hx >= 0) {
            /* another slice holds the crossing: its word (one wave polls, bounded) */
            if (wave_id() == 0) {
                uint64_t wv = 0;
                uint32_t spins = 0;
                const uint64_t *src = &pubrow[hx * kPubWords + kPubX];
                while (!((wv = at_ld64(src)) & kReady)) {
                    if (++spins > kLimit) {
                        if (lane == 0) {
                            if (p.status) atomicOr(p.status, DLK_STATUS_SYNC_TIMEOUT);
                            misc[6] = 1;
                        }
                        wv = kReady | 0x7fffffffull;
                        break;
                    }
                }
                if (lane == 0) misc[10] = (int)(uint32_t)(wv & 0x7fffffffull);
                if (lane == 0) misc[11] = (int)(uint32_t)(wv >> 31);
            }
            __syncthreads();
            const uint32_t xw = (uint32_t)misc[10];
            ok = xw != 0x7fffffffu;
            x = (int)xw;
            inv3 = u2f((uint32_t)misc[11]);
            __syncthreads();
        }
        if (DLK_COLD(topp && p.top_p > 0.0f && (!ok || f.force_exact) && !misc[6])) {
            /* the cut or its normaliser is undecided: the cumulation itself
             * (src/sampler.c:207-215), split over the row's workgroups; no
             * crossing keeps every entry (nk = k) */
            int pos;
            double s3;
            ok = split_sum53<kLimit, EPT>(v, RWg, (double)pk, ce, f, row, g, s0, s1, true, p.topp_thr, kSyncSplitP,
                                          kPubSplitP, sync, pubrow, rtot, rpre, cbh, misc, md, pos, s3);
            x = pos >= 0 ? pos : V - 1;
            inv3 = (float)(1.0 / s3);
        }
    }

    /* thread 0 composes from slice h0 and value cb: misc[23] the token
     * (-1: none up to x), misc[24] the first slice whose chains do not
     * cover the value reached (-1: none), misc[25] that value */
    const uint64_t *ent = (const uint64_t *)tab;   /* (the composition's copy of the row's chains) */
    auto compose = [&](int h0, uint32_t cb) {
        if (t == 0) {
            int tk_out = -1, fh = -1;
            for (int h = h0; h < G && h * S <= x; h++) {
                if (DLK_COLD(f.force_exact)) { fh = h; break; }
                uint32_t d = 0;
                if (h > 0) {
                    d = cb - (uint32_t)ent[h * kLaneWords + 64];
                    if (d >= 64u) { fh = h; break; }
                }
                const uint64_t e = ent[h * kLaneWords + d];
                const int tk = (int)(uint32_t)(e >> 32);
                if (tk == -2) { fh = h; break; }
                if (tk >= 0) { tk_out = tk; break; }
                cb = (uint32_t)e;
            }
            misc[23] = tk_out;
            misc[24] = fh;
            misc[25] = (int)cb;
        }
        __syncthreads();
    };
    bool run_exact = !ok && g == 0;        /* a wait gave up before the row's sums were decided */
    bool rewalk = false;                   /* a slice's chains miss the composition's value */
    float thr_fx = 0.0f;
    if (ok) {
    /* ---- final probabilities, draw aggregates, staged chunks -------------- */
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        const int i = s0 + 4 * (t + (j / 4) * T) + (j & 3);
        v[j] = i <= x ? (topp ? v[j] * inv3 : v[j]) : 0.0f;
    }
    /* (a uniform test first: the log must not be evaluated speculatively when
     * no log-probabilities are asked for) */
    const bool want_logp = g == 0 && n_out > 0 && p.out_cand_logprobs != nullptr;
    if (DLK_COLD(want_logp)) {
#pragma unroll
        for (int j = 0; j < EPT; j++) {
            const int i = 4 * (t + (j / 4) * T) + (j & 3);
            if (i < n_out && i < V)
                p.out_cand_logprobs[(int64_t)row * n_out + i] = v[j] > 0.0f ? (float)log((double)v[j]) : -INFINITY;
        }
    }
    /* predicted running value at chunk starts (the p prefix, cut at x, scaled) */
    const double scale = topp ? (double)inv3 : 1.0;
    double Rx;
    {
        /* p prefix at x: bounded by the prefix at the end of x's chunk */
        int cx = (x - s0) >> 6;
        Rx = (x < s0) ? RWg : (x >= s1 ? 1e300 : RWg + (double)pk * ce[min(nch, cx + 1)]);
    }
    /* each chunk's predicted binade: that of its start value when it and its
     * end value, widened by a margin far beyond the float sum's accumulated
     * rounding (2^-12 relative), share one; kInvalidBinade otherwise; and
     * kZeroBinade for a chunk that adds nothing (every value 0, or absorbed by
     * the double prefix, so certainly by the float sum) */
    const double mu = 0x1p-12;
    for (int c = t; c <= nch; c += T) {
        const double a = fmin(RWg + (double)pk * ce[c], Rx) * scale;
        Pc[c] = a;
        if (c < nch) {
            const double b = fmin(RWg + (double)pk * ce[c + 1], Rx) * scale;
            const bool zero = ce[c + 1] == ce[c] || s0 + 64 * c > x;
            const int bh = predict_binade<24>(a * (1.0 - mu));
            const bool valid = bh == predict_binade<24>(b * (1.0 + mu)) && bh >= -100;
            cbh[c] = zero ? kZeroBinade : valid ? bh : kInvalidBinade;
        }
    }
    __syncthreads();
    /* every lane reads its chunks' predicted binades before any is replaced: a
     * chunk belongs to one 16-lane row of one wave, whose lane 15 replaces it
     * below (all reads up front where the registers allow it) */
    constexpr bool kPreload = EPT <= 40;
    int pbh[EPT / 4];
    if (kPreload) {
#pragma unroll
        for (int j4 = 0; j4 < EPT / 4; j4++) pbh[j4] = cbh[(t + j4 * T) >> 4];
    }
#pragma unroll
    for (int j4 = 0; j4 < EPT / 4; j4++) {
        const int u = t + j4 * T;
        const int c = u >> 4;
        const int bh = kPreload ? pbh[j4] : cbh[c];
        /* the increments are integers below 2^24 wherever the prediction holds,
         * so their float sum is exact; where it does not the sum still reaches
         * 2^24 (non-negative terms, monotone rounding) and the chunk becomes an
         * element-level one.  Computed for every lane (no branch: an invalid or
         * zero chunk's scale 2^(23 - bh) underflows to 0); a tie saturates the
         * lane's sum, so a chunk whose total reaches 2^24 -- a tie, or a sum
         * that leaves the binade -- is element-level. */
        float xs[4], n[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            xs[k] = ldexpf(v[4 * j4 + k], 23 - bh);
            n[k] = rintf(xs[k]);
        }
        const float fsum = ((n[0] + n[1]) + n[2]) + n[3];
        /* largest distance to the rounded value: 0.5 exactly iff one term is a tie */
        const float fr = fmaxf(fmaxf(fabsf(xs[0] - n[0]), fabsf(xs[1] - n[1])),
                               fmaxf(fabsf(xs[2] - n[2]), fabsf(xs[3] - n[3])));
        uint32_t sum = fr == 0.5f ? (1u << 25) : (uint32_t)fminf(fsum, 0x1p25f);
        sum = row_scan_u32(sum);
        if ((lane & 15) == 15) {
            ca[c] = bh == kZeroBinade ? 0u : sum;
            cbh[c] = (bh == kZeroBinade || (bh != kInvalidBinade && sum < (1u << 24))) ? bh : kInvalidBinade;
        }
    }
    if (t == 0) misc[10] = 0;
    __syncthreads();
    /* the draw's segments, in order: each maximal run of chunks of one binade
     * (their values add exactly their increments on its grid), and each
     * element-level chunk on its own.  One scan (nch <= T): increments in bits
     * 0-39 (below 2^24 per chunk), segment ends in 40-51, element-level chunks
     * in 52-63 (counts at most nch <= 4095).  seg[s] = {binade, first chunk,
     * the run's increments (saturated at 2^24) or the chunk's table, next chunk}. */
    int elpos = -1;
    {
        const int c = t;
        const bool in = c < nch;
        const int bc = in ? cbh[c] : kInvalidBinade;
        const bool vld = bc != kInvalidBinade;
        const bool end = in && (!vld || c == nch - 1 || cbh[c + 1] != bc);
        const uint64_t a = vld ? (uint64_t)ca[c] : 0;
        const bool isel = in && !vld;
        const uint64_t all = block_incl_prefix_u64(a | ((uint64_t)end << 40) | ((uint64_t)isel << 52),
                                                   (uint64_t *)L.red);
        const uint64_t ainc = all & ((1ull << 40) - 1);
        const uint32_t run = (uint32_t)((all >> 40) & 0xfffu) - (end ? 1u : 0u);
        if (isel) elpos = (int)(all >> 52) - 1;
        if (in) elc[c] = (int)(all >> 52) - (isel ? 1 : 0);
        if (t == T - 1) {
            misc[17] = (int)(all >> 52);
            misc[21] = (int)((all >> 40) & 0xfffu);
        }
        if (end) { rend[run] = c; rpre[run] = ainc; }
        __syncthreads();
        if (in) rtot[c] = vld ? rpre[run] - (ainc - a) : 0;
        if (end) {
            if (vld) {
                const int first = run == 0 ? 0 : rend[run - 1] + 1;
                const uint64_t R = rpre[run] - (run == 0 ? 0ull : rpre[run - 1]);
                seg[run] = make_int4(bc, first, (int)(R < (1ull << 24) ? R : (1ull << 24)), c + 1);
            } else {
                seg[run] = make_int4(kInvalidBinade, c, elpos, c + 1);
            }
        }
    }
    __syncthreads();
    /* each chunk's predicted contribution to the exact float running sum: its
     * increments on its binade's grid (exact while the prediction holds), or
     * the real sum of an element-level chunk (off by that chunk's rounding, a
     * few of its ulps); the chunks staged in LDS here: the element-level ones
     * and x's (those that may hold r's crossing follow barrier D) */
    double *fpre = ce;                             /* ce is free again */
    const float thr_f = u2f(f2u(r) + 1u);          /* r < cumul  <=>  cumul >= thr_f */
    const double vthr = (double)thr_f;
    if (t < nch) {
        const int c = t;
        const int bh = cbh[c];
        fpre[c] = bh != kInvalidBinade ? ldexp((double)ca[c], bh - 23) : Pc[c + 1] - Pc[c];
        const bool want = bh == kInvalidBinade || (x >= s0 + 64 * c && x < s0 + 64 * c + 64);
        int sl = -1;
        if (want && s0 + 64 * c <= x) {
            sl = atomicAdd(&misc[10], 1);
            if (sl >= f.stage_cap) sl = -1;
        }
        smap[c] = sl;
        if (elpos >= 0) elist[elpos] = make_int2(c, sl);
    }
    __syncthreads();
    block_excl_scan(fpre, nch, L.red);             /* fpre[c]: before chunk c; fpre[nch]: the slice */
    if (t == 0) at_st64(&mypub[kPubF], d2u(fpre[nch]) | kReady);
    /* a staged chunk's values, and for a chunk of a run the inclusive prefix of
     * its increments on the run's grid (a chunk is one 16-lane row); slot_of
     * gives the chunk's slot, or -1 for a chunk not staged by this pass */
    auto stage = [&](const int *slot_of) {
#pragma unroll
        for (int j4 = 0; j4 < EPT / 4; j4++) {
            const int u = t + j4 * T;
            const int c = u >> 4;
            const int sl = slot_of[c];
            if (ballot(sl >= 0) != 0) {
                const int bh = cbh[c];
                const bool run = bh != kInvalidBinade && bh != kZeroBinade;
                uint32_t n[4];
#pragma unroll
                for (int k = 0; k < 4; k++) n[k] = run ? (uint32_t)rintf(ldexpf(v[4 * j4 + k], 23 - bh)) : 0u;
                const uint32_t s4 = ((n[0] + n[1]) + n[2]) + n[3];
                const uint32_t ex = row_scan_u32(s4) - s4;
                if (sl >= 0) {
                    *(float4 *)&svals[sl * 64 + (u & 15) * 4] =
                        make_float4(v[4 * j4], v[4 * j4 + 1], v[4 * j4 + 2], v[4 * j4 + 3]);
                    *(uint4 *)&spx[sl * 64 + (u & 15) * 4] =
                        make_uint4(ex + n[0], ex + n[0] + n[1], ex + n[0] + n[1] + n[2], ex + s4);
                }
            }
        }
    };
    stage(smap);

    /* ---- D: the slices' predicted contributions -> this slice's predicted
     *      exact start value (exact for slice 0: the sum starts at 0) ------- */
    {
        const int idx[1] = {kPubF};
        row_gather<kLimit>(pubrow, G, idx, pc, p.status, &misc[6]);
    }
    double Phat = 0.0;
    for (int h = 0; h < g; h++) Phat += u2d(pc[h * kPubWords + kPubF]);

    /* ---- the chunks that may hold r's crossing, from the float prediction
     *      (this slice's predicted start plus its contributions, off by a few
     *      tens of its ulps at most on sharp rows): a chunk that adds something
     *      and whose predicted running values come within 128 ulps of thr_f.
     *      (A window on the double prefix, whose drift from the float sum is
     *      some 10^-4 relative, took hundreds of nearly empty chunks of sharp
     *      rows and overflowed the staging.)  rend (free after the segments)
     *      holds the slots of this pass. ---------------------------------- */
    {
        const uint32_t ex_thr = (f2u(thr_f) >> 23) & 255u;
        const double mg = 128.0 * ldexp(1.0, (int)(ex_thr > 0u ? ex_thr : 1u) - 150);
        /* (a slice whose predicted span misses thr_f by more than the margin
         * stages nothing here: every workgroup evaluates the same test) */
        const bool span = Phat + fpre[0] - mg <= vthr && vthr <= Phat + fpre[nch] + mg && s0 <= x;
        if (span && t < nch) {
            const int c = t;
            int sl = -1;
            if (smap[c] < 0 && s0 + 64 * c <= x && cbh[c] != kZeroBinade) {
                const double a = Phat + fpre[c], b = Phat + fpre[c + 1];
                if (a - mg <= vthr && vthr <= b + mg) {
                    sl = atomicAdd(&misc[10], 1);
                    if (sl >= f.stage_cap) sl = -1;
                    else smap[c] = sl;
                }
            }
            rend[c] = sl;
        }
        if (span) {
            __syncthreads();
            stage(rend);
        }
    }

    /* ---- candidate tables: each element-level chunk summed in order from the
     *      64 consecutive floats around its predicted start, one wave per chunk
     *      (src/sampler.c:226-232); lane k keeps the end value and the first
     *      position whose running value reaches thr_f ------------------------ */
    const int ntab = min(misc[17], kMaxTabs);
    /* table ti for the 64 starts from `base`: lane k's end value and crossing
     * (returned: the lane's end value) */
    auto build_table = [&](int ti, const int2 e, uint32_t base) -> float {
        float c = u2f(base + (uint32_t)lane);
        int below = 0;
        const float4 *q4 = (const float4 *)(svals + e.y * 64);
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const float4 qv = q4[k];
            c = c + qv.x;
            below += c < thr_f ? 1 : 0;
            c = c + qv.y;
            below += c < thr_f ? 1 : 0;
            c = c + qv.z;
            below += c < thr_f ? 1 : 0;
            c = c + qv.w;
            below += c < thr_f ? 1 : 0;
        }
        tab[ti * 64 + lane] = make_int2((int)f2u(c), below < 64 ? below : -1);
        return c;
    };
    /* each table's correction to its chunk's predicted contribution: lane 32
     * starts at the chunk's predicted value, so its end value less that start
     * is the chunk's float contribution (the same for any start on that grid,
     * ties and binade changes aside), where the prediction took the chunk's
     * real sum, off by its additions' roundings (L.red is free from here to
     * the end of the ranges) */
    double *tdelta = L.red;
    for (int ti = wave_id(); ti < ntab; ti += T / 64) {
        const int2 e = elist[ti];
        uint32_t base = 0xffffffffu;
        double dl = 0.0;
        if (e.y >= 0) {
            const uint32_t pb = f2u((float)(Phat + fpre[e.x]));
            base = pb >= 32u ? pb - 32u : 0u;
            const float cend = build_table(ti, e, base);
            dl = (double)cend - (double)u2f(base + 32u) - (fpre[e.x + 1] - fpre[e.x]);
        }
        if (lane == 0) tbase[ti] = base;
        if (lane == 32) tdelta[ti] = dl;
    }
    __syncthreads();
    /* ---- the slice's draw for 64 candidate start values (slice 0: its exact
     *      start 0 in every lane).  The segments are split into one contiguous
     *      range per wave; wave w runs its range for the 64 consecutive floats
     *      around the range's predicted start, segment by segment: a run adds
     *      its increments (exact while the value stays in the run's binade), an
     *      element-level chunk is a table lookup.  A lane that leaves what the
     *      prediction covers (another binade, a value outside a table, a crossing
     *      in an unstaged chunk) is marked -2.  Wave 0 then composes the ranges:
     *      each range's lane for the value the previous range ended with; a
     *      range that starts past x adds nothing to any start value and is
     *      passed over (its window would only test the prediction at x) ----- */
    const int nch_loc = x < s0 ? 0 : min(nch, ((x - s0) >> 6) + 1);
    const int nseg = misc[21];
    const int per = (nseg + T / 64 - 1) / (T / 64);
    const int nrng = per > 0 ? (nseg + per - 1) / per : 0;
    if (wave_id() < nrng) {
        const int w = wave_id();
        const int sa = w * per, sb = min(nseg, sa + per);
        const int c0 = seg[sa].y;
        /* refined start: the corrections of the tables before the range (they
         * add up over a slice's element-level chunks; without them a range's
         * start fell outside its 64 candidates on sharper rows, T 0.7-0.8) */
        const double dlt = lane < ntab ? tdelta[lane] : 0.0;
        const double dex = wave_incl_scan_d(dlt) - dlt;
        const double pstart = Phat + fpre[c0] + u2d(readlane64(d2u(dex), min(elc[c0], ntab)));
        /* this wave alone reads the tables of its range: one whose refined start
         * (the corrections of the tables before it) lies more than 24 candidates
         * from its window's centre is built again around it, here, with no
         * barrier (the corrections do not depend on where the windows lie).
         * One lane per segment of the range; a range holds at most 64. */
        {
            int ti = -1;
            uint32_t nb = 0;
            if (sa + lane < sb) {
                const int4 sg = seg[sa + lane];
                if (sg.x == kInvalidBinade && sg.y < nch_loc && sg.z < ntab) ti = sg.z;
            }
            const double dti = u2d(((uint64_t)(uint32_t)__shfl((int)(uint32_t)(d2u(dex) >> 32), max(ti, 0), 64) << 32) |
                                   (uint32_t)__shfl((int)(uint32_t)d2u(dex), max(ti, 0), 64));
            bool re = false;
            if (ti >= 0) {
                const int2 e = elist[ti];
                const uint32_t ob = tbase[ti];
                if (e.y >= 0 && ob != 0xffffffffu) {
                    const uint32_t pb = f2u((float)(Phat + fpre[e.x] + dti));
                    nb = pb >= 32u ? pb - 32u : 0u;
                    const int dd = (int)(nb - ob);
                    re = dd < -24 || dd > 24;
                }
            }
            uint64_t todo = ballot(re);
            while (DLK_COLD(todo != 0)) {
                const int l = first_lane(todo);
                todo &= todo - 1;
                const int tj = __builtin_amdgcn_readlane(ti, l);
                const uint32_t nbj = (uint32_t)__builtin_amdgcn_readlane((int)nb, l);
                build_table(tj, elist[tj], nbj);
                if (lane == 0) tbase[tj] = nbj;
            }
        }
        uint32_t rb = 0, cb = 0;
        if (g > 0 || w > 0) {
            const uint32_t pb = f2u((float)pstart);
            rb = pb >= 32u ? pb - 32u : 0u;
            cb = rb + (uint32_t)lane;
        }
        int tok = -1;                              /* -1 no crossing yet; >= 0 token; -2 unresolved */
        if (c0 >= nch_loc) {
            /* past x: every value is 0 and the range adds nothing */
        } else if (pstart > vthr * (1.0 + 0x1p-9)) {
            tok = -3;                              /* r's crossing lies before this range */
        } else {
            const DrawView dv{seg, rtot, smap, spx, tab, tbase, ntab, nch_loc, s0, thr_f};
            for (int s = sa; s < sb; s++) {
                const int sy = seg[s].y;
                if (sy >= nch_loc || ballot(tok == -1) == 0) break;
                if (tok != -1) continue;
                draw_step(dv, s, cb, tok);
            }
        }
        rres[w * 64 + lane] = make_int2((int)cb, tok);
        if (lane == 0) rbase[w] = c0 >= nch_loc ? kPastX : rb;
    }
    __syncthreads();
    if (wave_id() == 0) {
        uint32_t wbase = 0;
        if (g > 0) {
            const uint32_t pb = f2u((float)Phat);
            wbase = pb >= 32u ? pb - 32u : 0u;
        }
        uint32_t cb = g > 0 ? wbase + (uint32_t)lane : 0u;
        int tok = -1;
        if (g == 0) {
            /* the row's first slice starts at exactly 0: every lane follows the
             * same value, so the chain is uniform.  Every range's entries are
             * loaded at once and each step reads its entry across lanes
             * (v_readlane) instead of waiting on an LDS read per range: the
             * first slice holds the draw's early binade changes, so it is the
             * row's slowest and its chain of up to 16 dependent reads (about
             * 2.3 us) was on the launch's critical path */
            constexpr int kW = kFullThreads / 64;
            int2 ent[kW];
            uint32_t rbw[kW];
#pragma unroll
            for (int w = 0; w < kW; w++) {
                ent[w] = w < nrng ? rres[w * 64 + lane] : make_int2(0, -2);
                rbw[w] = w < nrng ? rbase[w] : kPastX;
            }
            uint32_t cu = 0;
            int tu = -1;
#pragma unroll
            for (int w = 0; w < kW; w++) {
                const uint32_t rb = (uint32_t)__builtin_amdgcn_readfirstlane((int)rbw[w]);
                if (tu != -1 || w >= nrng || rb == kPastX) continue;
                const uint32_t d = cu - rb;
                if (d >= 64u) {
                    tu = -2;
                } else {
                    const int ey = __builtin_amdgcn_readlane(ent[w].y, (int)d);
                    const uint32_t ex = (uint32_t)__builtin_amdgcn_readlane(ent[w].x, (int)d);
                    if (ey == -1) cu = ex;
                    else tu = ey == -3 ? -2 : ey;
                }
            }
            cb = cu;
            tok = tu;
        } else {
            for (int w = 0; w < nrng; w++) {
                if (ballot(tok == -1) == 0) break;
                if (tok != -1 || rbase[w] == kPastX) continue;
                const uint32_t d = cb - rbase[w];
                if (d >= 64u) {
                    tok = -2;
                } else {
                    const int2 e = rres[w * 64 + (int)d];
                    if (e.y == -1) cb = (uint32_t)e.x;
                    else tok = e.y == -3 ? -2 : e.y;
                }
            }
        }
        uint64_t *lw = f.lanes + ((int64_t)row * G + g) * kLaneWords;
        at_st64(&lw[lane], (uint64_t)cb | ((uint64_t)(uint32_t)tok << 32));
        if (lane == 0) at_st64(&lw[64], (uint64_t)wbase);
    }
    /* the chains are stored before the count that announces them */
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (t == 0) {
        const uint32_t old = __hip_atomic_fetch_add(&sync[kSyncLanes], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        misc[22] = old == (uint32_t)(G - 1);
    }
    __syncthreads();
    if (misc[22]) {
        /* ---- the last workgroup of the row composes the slices from the
         *      row's exact start 0: slice h's lane for the value slice h-1 ended
         *      with gives slice h's end value or the token ---------------------- */
        uint64_t *entw = (uint64_t *)tab;
        const uint64_t *lrow = f.lanes + (int64_t)row * G * kLaneWords;
        for (int i = t; i < G * kLaneWords; i += T) entw[i] = at_ld64(&lrow[i]);
        __syncthreads();
        compose(0, 0u);
        /* nothing crossed r up to x: the last kept entry (src/sampler.c:233) */
        int token = misc[23] >= 0 ? misc[23] : x;
        rewalk = misc[24] >= 0;
        thr_fx = thr_f;
        if (DLK_HOT(!rewalk) && t == 0) p.out_ids[row] = token;
    }
    }

    if (DLK_COLD(rewalk)) {
        /* a slice whose chains do not cover the value the composition reached
         * is walked itself from that value (draw_fix), and the composition
         * resumes after it */
        int token = x;
        while (true) {
            const int fh = misc[24];
            int pos;
            uint32_t endb;
            draw_fix<EPT, CAP>(f, row, fh, (uint32_t)misc[25], x, M, inv, mp_all, mp_inv2, inv3, thr_fx, L, lg, mk, Pc,
                               rtot, rpre, cbh, (unsigned char *)seg, misc, pos, endb);
            if (pos >= 0) { token = fh * S + pos; break; }
            if (fh + 1 >= G || (fh + 1) * S > x) break;
            compose(fh + 1, endb);
            if (misc[24] < 0) { token = misc[23] >= 0 ? misc[23] : x; break; }
        }
        if (t == 0) p.out_ids[row] = token;
    }
    if (DLK_COLD(run_exact) && t == 0) {
        /* only a wait that gave up leaves a sum undecided (the status word
         * flags the launch; the row's id stays inside the vocabulary) */
        p.out_ids[row] = V - 1;
        if (p.status) atomicOr(p.status, DLK_STATUS_SYNC_TIMEOUT);
    }
    /* a wait of this workgroup gave up (the status word flags the launch): the
     * row's workgroups may disagree on whether its sums were certified, so no
     * workgroup may compose it; this one leaves an id inside the vocabulary */
    if (misc[6] && t == 0) p.out_ids[row] = V - 1;
    row_exit(sync, pubrow, G);
}

}  // namespace dlk

namespace {
template <bool CAP, int HP>
const void *full_fn_hp(int which) {
    using namespace dlk;
    switch (which) {
        case 0: return (const void *)full_kernel<16, CAP, false, HP>;
        case 1: return (const void *)full_kernel<24, CAP, false, HP>;
        case 2: return (const void *)full_kernel<32, CAP, false, HP>;
        case 3: return (const void *)full_kernel<40, CAP, false, HP>;
        default: return (const void *)full_kernel<48, CAP, false, HP>;
    }
}
/* the instance for (elements per thread, soft-cap, history ids per thread) */
const void *full_fn(int which, int cap, int hp) {
    if (cap) return hp > 1 ? full_fn_hp<true, 2>(which) : full_fn_hp<true, 1>(which);
    return hp > 1 ? full_fn_hp<false, 2>(which) : full_fn_hp<false, 1>(which);
}
int ept_index(int ept) { return ept == 16 ? 0 : ept == 24 ? 1 : ept == 32 ? 2 : ept == 40 ? 3 : ept == 48 ? 4 : -1; }
}  // namespace

extern "C" int dlk_launch_full_kernel(const dlk::FullParams *f, int rows, int ept, size_t lds, hipStream_t stream) {
    using namespace dlk;
    static int set[2][2][5];
    static int set_nw = 0;
    const int which = ept_index(ept), cap = f->p.cap > 0.0f ? 1 : 0;
    const int hp = f->p.plan.hcap > kFullThreads ? 2 : 1;
    if (which < 0) return -1;
    const void *fn = full_fn(which, cap, hp);
    if (f->no_wait) {
        /* the test instance exists for 24 elements per thread, no soft-cap */
        if (ept != 24 || cap || hp != 1) return -2;
        fn = (const void *)full_kernel<24, false, true>;
        if (!set_nw) {
            if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess) return -1;
            set_nw = 1;
        }
    } else if (!set[cap][hp - 1][which]) {
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess) return -1;
        set[cap][hp - 1][which] = 1;
    }
    /* An ordinary launch: the grid fits the device's resident workgroups
     * (checked by the host against dlk_full_kernel_capacity), and the row
     * waits only on workgroups of its own row.  Workgroups are dispatched in
     * index order and a row's workgroups are consecutive, so every row below
     * the dispatch frontier is fully resident and finishes, which frees room
     * for the rest: the barriers make progress without a cooperative launch
     * (which costs ~12 us of launch latency here), and every wait is bounded. */
    FullParams fp = *f;
    void *args[] = {&fp};
    if (hipLaunchKernel(fn, dim3(rows * f->G), dim3(kFullThreads), args, lds, stream) != hipSuccess) return -1;
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

extern "C" int dlk_full_kernel_capacity(int ept, size_t lds, int cap, int hp) {
    using namespace dlk;
    const int which = ept_index(ept);
    if (which < 0) return 0;
    const void *fn = full_fn(which, cap, hp);
    if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess) return 0;
    int per_cu = 0, dev = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kFullThreads, lds) != hipSuccess) return 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    return per_cu * cus;
}
