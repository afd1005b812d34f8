/*
 * exact_scan.h -- bit-exact emulation of a sequential floating-point running sum
 * on one wavefront, with the bulk of the work done in parallel.
 *
 * The reference accumulates probabilities one at a time (src/sampler.c:177-181,
 * :198-199, :207-215, :218-219 in double; :226-232 in float).  A tree or
 * prefix sum rounds differently, and the sampled token depends on those bits,
 * so the order-dependent sum has to be reproduced exactly.
 *
 * Method.  Let the running value c lie in binade b, i.e. c in [2^b, 2^(b+1))
 * (the lowest binade also holds 0 and the subnormals, which share its grid), and
 * let u = 2^(b - MB + 1) be its ulp, MB = 24 (float) or 53 (double).  Then c = m*u
 * for an integer m < 2^MB, and for a non-negative float q whose sum stays in the
 * binade, fl(c + q) = u * RNE(m + q/u) = u * (m + n(q, m mod 2)): n is q/u rounded
 * to nearest, and only when q/u is exactly halfway does the result depend on m's
 * parity (ties go to the even m).  So inside one binade the sum is an integer
 * prefix sum over pair-valued increments (A0, A1) -- the increment for an even and
 * an odd start -- and pairs compose associatively:
 *      (A then B)_p = A_p + B_{(p + A_p) mod 2}.
 * A step that leaves the binade (m + n >= 2^MB) is done as a real IEEE addition.
 *
 * Data.  The block precomputes aggregates per chunk (64 elements) and per group
 * (64 chunks = 4096 elements), each under a *predicted* binade taken from an
 * approximate prefix sum (wrong predictions only cost time: the resolver checks
 * every aggregate against the true binade and descends into it otherwise).
 *
 * Resolve.  One wave walks the sequence: 64 aggregates (or elements) per step,
 * an inclusive pair scan across lanes, and a ballot for the first lane whose
 * aggregate is invalid for the current binade, leaves the binade, or crosses the
 * caller's threshold; it advances to that lane and descends one level, down to
 * single elements, where exits become real additions.  Every step consumes at
 * least one element or descends one of three levels, so the walk ends.
 *
 * Thresholds.  A threshold v stops the walk at the first element after which
 * c >= v (the draw r < cumul uses v = nextafter(r); top-p (float)cumul >= top_p
 * uses the smallest double that rounds to >= top_p).  In binade b this is the
 * integer test m >= ceil(v / u).
 */
#ifndef DLK_EXACT_SCAN_H
#define DLK_EXACT_SCAN_H

#include <type_traits>

#include "dlk_device.h"

namespace dlk {

constexpr uint64_t kCap = 1ull << 62;       /* saturation: far above any binade */
constexpr int kInvalidBinade = 0x7fff;
constexpr int kEmptyRun = 0x7ffe;          /* walk_pairs: consecutive element chunks */
constexpr int kZeroBinade = 0x7ffd;        /* a chunk that adds nothing to the running value */

struct Pair {
    uint64_t a0, a1;
};

DLK_DEV uint64_t sat_add(uint64_t a, uint64_t b) {
    uint64_t s = a + b;                      /* a, b <= 2^62: no wrap */
    return s > kCap ? kCap : s;
}

DLK_DEV Pair compose(Pair A, Pair B) {
    Pair C;
    C.a0 = sat_add(A.a0, (A.a0 & 1) ? B.a1 : B.a0);
    C.a1 = sat_add(A.a1, (A.a1 & 1) ? B.a0 : B.a1);
    return C;
}

template <int MB>
struct Fmt;
template <>
struct Fmt<24> {
    static constexpr int EMIN = -126;
    using T = float;
};
template <>
struct Fmt<53> {
    static constexpr int EMIN = -1022;
    using T = double;
};

/* Increment of a non-negative float q on the grid 2^ue. */
DLK_DEV Pair increment(float q, int ue) {
    uint32_t u = f2u(q);
    uint32_t ex = u >> 23;
    uint32_t mq = u & 0x7fffffu;
    int eq;
    if (ex == 0) {
        eq = -149;
    } else {
        mq |= 0x800000u;
        eq = (int)ex - 150;
    }
    if (mq == 0) return Pair{0, 0};
    int sh = eq - ue;
    if (sh >= 0) {
        uint64_t n = sh >= 38 ? kCap : ((uint64_t)mq << sh);
        return Pair{n, n};
    }
    int s = -sh;
    if (s >= 26) return Pair{0, 0};          /* q/u < 1/4 */
    uint64_t n = mq >> s;
    uint32_t rem = mq & ((1u << s) - 1u);
    uint32_t half = 1u << (s - 1);
    if (rem > half) n += 1;
    if (rem == half) return Pair{n + (n & 1), n + ((n + 1) & 1)};
    return Pair{n, n};
}

/* Binade of a running value / its integer significand on that binade's grid. */
DLK_DEV void split(float c, int &b, uint64_t &m) {
    uint32_t u = f2u(c), ex = u >> 23;
    if (ex <= 1) { b = -126; m = u; }
    else { b = (int)ex - 127; m = (u & 0x7fffffu) | 0x800000u; }
}
DLK_DEV void split(double c, int &b, uint64_t &m) {
    uint64_t u = d2u(c), ex = u >> 52;
    if (ex <= 1) { b = -1022; m = u; }
    else { b = (int)ex - 1023; m = (u & 0xfffffffffffffull) | (1ull << 52); }
}
DLK_DEV float join_f(int b, uint64_t m) {
    if (m >= (1ull << 24)) return u2f((uint32_t)(b + 128) << 23);   /* exactly 2^(b+1) */
    if (b == -126) return u2f((uint32_t)m);
    return u2f(((uint32_t)(b + 127) << 23) | ((uint32_t)m & 0x7fffffu));
}
DLK_DEV double join_d(int b, uint64_t m) {
    if (m >= (1ull << 53)) return u2d((uint64_t)(b + 1024) << 52);
    if (b == -1022) return u2d(m);
    return u2d(((uint64_t)(b + 1023) << 52) | (m & 0xfffffffffffffull));
}
template <int MB>
DLK_DEV typename Fmt<MB>::T join(int b, uint64_t m);
template <>
DLK_DEV float join<24>(int b, uint64_t m) { return join_f(b, m); }
template <>
DLK_DEV double join<53>(int b, uint64_t m) { return join_d(b, m); }

/* Predicted binade of a running value approximated by the double v >= 0. */
template <int MB>
DLK_DEV int predict_binade(double v) {
    uint64_t u = d2u(v);
    int ex = (int)(u >> 52) - 1023;
    return ex <= Fmt<MB>::EMIN ? Fmt<MB>::EMIN : ex;
}

/* Smallest integer t with t * 2^ue >= v (v >= 0 finite double); saturating. */
DLK_DEV uint64_t ceil_div_pow2(double v, int ue) {
    uint64_t u = d2u(v);
    uint64_t ex = u >> 52, mv = u & 0xfffffffffffffull;
    if (ex == 0 && mv == 0) return 0;
    int ev;
    if (ex == 0) ev = -1074;
    else { mv |= 1ull << 52; ev = (int)ex - 1075; }
    int sh = ev - ue;
    if (sh >= 0) return sh >= 9 ? kCap : (mv << sh);
    int s = -sh;
    if (s >= 64) return 1;
    return (mv >> s) + ((mv & ((1ull << s) - 1)) != 0);
}

/* The lanes' pairs composed in lane order, inclusive: DPP row shifts, then row
 * broadcasts (a lane with no source receives {0, 0}, the identity of
 * compose; the left operand is always the lower lanes' part, so the order of
 * the composition is kept). */
template <int CTRL, int ROWS = 0xf, bool BC = true>
DLK_DEV Pair dpp_pair(Pair x) {
    return Pair{dpp_u64<CTRL, ROWS, BC>(x.a0), dpp_u64<CTRL, ROWS, BC>(x.a1)};
}
DLK_DEV Pair wave_incl_scan(Pair x, int lane) {
    (void)lane;
    x = compose(dpp_pair<kDppRowShr1>(x), x);
    x = compose(dpp_pair<kDppRowShr2>(x), x);
    x = compose(dpp_pair<kDppRowShr4>(x), x);
    x = compose(dpp_pair<kDppRowShr8>(x), x);
    x = compose(dpp_pair<kDppRowBcast15, 0xa, false>(x), x);
    x = compose(dpp_pair<kDppRowBcast31, 0xc, false>(x), x);
    return x;
}

/* The pair of a 64-element chunk held by a 16-lane row, four values per lane
 * in order (q0..q3, non-negative floats), on the grid 2^ue: every lane gets
 * the inclusive composition of its row's increments, lane 15 the chunk's.
 * When no value of the wave lies exactly halfway between two grid points, no
 * increment depends on the running value's parity: the pair is (n, n) with n
 * the sum of the values rounded to the grid, taken in double (exact while
 * below 2^53; a sum at or past 2^53 is past any binade's top, so it only has
 * to stay there, and is saturated at kCap).  Otherwise the wave composes the
 * pairs (increment()). */
DLK_DEV Pair row_chunk_pair(float q0, float q1, float q2, float q3, int ue) {
    const double d0 = ldexp((double)q0, -ue), d1 = ldexp((double)q1, -ue);
    const double d2 = ldexp((double)q2, -ue), d3 = ldexp((double)q3, -ue);
    const double n0 = rint(d0), n1 = rint(d1), n2 = rint(d2), n3 = rint(d3);
    const bool tie = fabs(d0 - n0) == 0.5 || fabs(d1 - n1) == 0.5 || fabs(d2 - n2) == 0.5 || fabs(d3 - n3) == 0.5;
    if (ballot(tie) == 0) {
        const double sum = row_scan_d((n0 + n1) + (n2 + n3));
        const uint64_t a = sum >= 0x1p62 ? kCap : (uint64_t)sum;
        return Pair{a, a};
    }
    Pair x = increment(q0, ue);
    x = compose(x, increment(q1, ue));
    x = compose(x, increment(q2, ue));
    x = compose(x, increment(q3, ue));
    x = compose(dpp_pair<kDppRowShr1>(x), x);
    x = compose(dpp_pair<kDppRowShr2>(x), x);
    x = compose(dpp_pair<kDppRowShr4>(x), x);
    x = compose(dpp_pair<kDppRowShr8>(x), x);
    return x;
}

/* Aggregates of one sequence: chunk (64) and group (4096) level.  Flat
 * pointers, so they may live in LDS or in global memory. */
struct Aggs {
    uint64_t *a0, *a1;
    int *bh;
    uint64_t *ga0, *ga1;
    int *gbh;
    double *P;      /* [nch + 1] approximate prefix sums at chunk starts */
};

/* Block-wide: P[c] = approximate exclusive prefix of q over chunks, P[nch] = total.
 * Uses `red` (>= blockDim/64 doubles of LDS) as scratch. */
template <class QF>
__device__ __forceinline__ void chunk_prefix(int n, const QF &q, double *P, double *red) {
    const int lane = lane_id(), w = wave_id(), nw = n_waves();
    const int nch = (n + 63) >> 6;
    for (int c = w; c < nch; c += nw) {
        int i = c * 64 + lane;
        double v = i < n ? (double)q(i) : 0.0;
        v = wave_incl_scan_d(v);                /* (any order: P only predicts binades) */
        if (lane == 63) P[c] = v;
    }
    __syncthreads();
    /* exclusive scan over nch values: each thread a contiguous run. */
    const int T = blockDim.x, t = threadIdx.x;
    const int per = (nch + T - 1) / T;
    const int b0 = t * per, b1 = min(nch, b0 + per);
    double loc = 0.0;
    for (int c = b0; c < b1; c++) loc += P[c];
    const double inc = wave_incl_scan_d(loc);
    if (lane == 63) red[w] = inc;
    __syncthreads();
    double wbase = 0.0;
    for (int k = 0; k < w; k++) wbase += red[k];
    double run = wbase + inc - loc;
    __syncthreads();
    for (int c = b0; c < b1; c++) { double v = P[c]; P[c] = run; run += v; }
    if (t == T - 1) P[nch] = run;
    __syncthreads();
}

/* Block-wide: chunk and group aggregates of q under binades predicted from
 * scale * min(P, cut). */
template <int MB, class QF>
__device__ __forceinline__ void build_aggs(int n, const QF &q, const Aggs &A, double scale, double cut) {
    const int lane = lane_id(), w = wave_id(), nw = n_waves();
    const int nch = (n + 63) >> 6, ngr = (nch + 63) >> 6;
    for (int c = w; c < nch; c += nw) {
        int bs = predict_binade<MB>(fmin(A.P[c], cut) * scale);
        int be = predict_binade<MB>(fmin(A.P[c + 1], cut) * scale);
        if (bs != be) {
            if (lane == 0) A.bh[c] = kInvalidBinade;
            continue;
        }
        int i = c * 64 + lane;
        Pair x = i < n ? increment(q(i), bs - (MB - 1)) : Pair{0, 0};
        x = wave_incl_scan(x, lane);
        if (lane == 63) { A.a0[c] = x.a0; A.a1[c] = x.a1; A.bh[c] = bs; }
    }
    __syncthreads();
    for (int g = w; g < ngr; g += nw) {
        int c = g * 64 + lane;
        bool in = c < nch;
        int b0 = A.bh[g * 64];
        bool ok = !in || A.bh[c] == b0;
        ok = (ballot(!ok) == 0) && b0 != kInvalidBinade;
        if (!ok) {
            if (lane == 0) A.gbh[g] = kInvalidBinade;
            continue;
        }
        Pair x = in ? Pair{A.a0[c], A.a1[c]} : Pair{0, 0};
        x = wave_incl_scan(x, lane);
        if (lane == 63) { A.ga0[g] = x.a0; A.ga1[g] = x.a1; A.gbh[g] = b0; }
    }
    __syncthreads();
}

template <int MB>
struct ResolveOut {
    int pos;                        /* first element reaching the threshold, or -1 */
    typename Fmt<MB>::T value;      /* running value after `pos` (or after the last element) */
};

DLK_DEV uint64_t readlane64(uint64_t v, int l) {
    uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
    uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
    return ((uint64_t)hi << 32) | lo;
}
DLK_DEV float readlanef(float v, int l) { return u2f((uint32_t)__builtin_amdgcn_readlane((int)f2u(v), l)); }

/* Inclusive scan of the lanes' increments, added to m: the running significand
 * after each lane's element/aggregate (saturating; exact below 2^MB). */
template <int MB>
DLK_DEV uint64_t scan_from(uint64_t m, Pair x, int lane) {
    if (MB == 24 && ballot(x.a0 != x.a1) == 0) {
        const uint32_t cap32 = 1u << 30;
        return m + wave_scan_sat_u32((uint32_t)min(x.a0, (uint64_t)cap32), cap32);
    }
    x = wave_incl_scan(x, lane);
    return sat_add(m, (m & 1) ? x.a1 : x.a0);
}

/* One wave: walk the sequence with the aggregates, starting from the running
 * value c0.  has_thr selects a stop at the first element after which c >= thr_v.
 * All lanes return the same result. */
template <int MB, class QF>
__device__ __forceinline__ ResolveOut<MB> resolve(int n, const QF &q, const Aggs &A, bool has_thr, double thr_v,
                                                  typename Fmt<MB>::T c0 = 0) {
    using T = typename Fmt<MB>::T;
    const int lane = lane_id();
    const uint64_t top = 1ull << MB;
    const int nch = (n + 63) >> 6, ngr = (nch + 63) >> 6;
    int b;
    uint64_t m;
    split(c0, b, m);
    uint64_t thr = has_thr ? ceil_div_pow2(thr_v, b - (MB - 1)) : kCap;
    int pos = 0, cap = 2;
    while (pos < n) {
        int L = 0;
        if (cap >= 2 && (pos & 4095) == 0) L = 2;
        else if (cap >= 1 && (pos & 63) == 0) L = 1;
        if (L == 0) {
            /* single elements up to the end of the chunk; each exit from the
             * binade is one real addition and a re-scan of the remaining lanes */
            const int count = min(64 - (pos & 63), n - pos);
            const bool act = lane < count;
            const float qv = act ? q(pos + lane) : 0.0f;
            int from = 0;
            while (true) {
                Pair x = (act && lane >= from) ? increment(qv, b - (MB - 1)) : Pair{0, 0};
                uint64_t ma = scan_from<MB>(m, x, lane);
                bool ev = act && lane >= from && (ma >= top || ma >= thr);
                int f = first_lane(ballot(ev));
                if (f >= count) {
                    if (count > from) m = readlane64(ma, count - 1);
                    break;
                }
                if (f > from) m = readlane64(ma, f - 1);
                const uint64_t maf = readlane64(ma, f);
                if (maf < top) return ResolveOut<MB>{pos + f, join<MB>(b, maf)};
                T c = join<MB>(b, m) + (T)readlanef(qv, f);
                if (has_thr && (double)c >= thr_v) return ResolveOut<MB>{pos + f, c};
                split(c, b, m);
                thr = has_thr ? ceil_div_pow2(thr_v, b - (MB - 1)) : kCap;
                from = f + 1;
            }
            pos += count;
            cap = 2;
            continue;
        }
        const int item = pos >> (6 * L);
        const int count = L == 2 ? min(64, ngr - item) : min(64 - (item & 63), nch - item);
        const bool act = lane < count;
        Pair x{0, 0};
        bool valid = true;
        if (act) {
            if (L == 1) {
                int c = item + lane;
                valid = A.bh[c] == b;
                x = Pair{A.a0[c], A.a1[c]};
            } else {
                int g = item + lane;
                valid = A.gbh[g] == b;
                x = Pair{A.ga0[g], A.ga1[g]};
            }
        }
        if (!valid) x = Pair{0, 0};
        uint64_t ma = scan_from<MB>(m, x, lane);
        bool ev = act && (!valid || ma >= top || ma >= thr);
        int f = first_lane(ballot(ev));
        if (f > count) f = count;
        if (f > 0) m = readlane64(ma, f - 1);
        pos = min(n, pos + (f << (6 * L)));
        if (f == count) { cap = 2; continue; }
        cap = L - 1;                         /* descend into item f */
    }
    return ResolveOut<MB>{-1, join<MB>(b, m)};
}

/* ---- run-skipping float resolver ------------------------------------------
 * The draw (src/sampler.c:226-232) accumulates in float.  Chunks (64 elements)
 * whose running value provably stays in one binade b add exact integers on the
 * grid 2^(b-23); consecutive such chunks of one binade form a run, and for each
 * chunk the integer total from it to the end of its run is precomputed, so the
 * walk crosses a run in one step.  Every other chunk (binade change, halfway
 * case, misprediction) is summed element by element in float.
 *
 * Each chunk has one 16-byte record, read by the walk in one LDS access:
 *   x = (binade & 0xffff) | (staged slot << 16)   binade = kInvalidBinade for an
 *                                                  element-level chunk, slot -1
 *                                                  when the values are not staged
 *   y = first chunk after the chunk's run
 *   z, w = low / high word of the increments from the chunk to the end of its run */
DLK_DEV int4 make_rec(int bh, int slot, int next, uint64_t tot) {
    return make_int4((bh & 0xffff) | (slot << 16), next, (int)(uint32_t)tot, (int)(uint32_t)(tot >> 32));
}
DLK_DEV int rec_bh(int x) { return (int)(short)(x & 0xffff); }
DLK_DEV int rec_slot(int x) { return x >> 16; }
DLK_DEV uint64_t rec_tot(int4 r) { return ((uint64_t)(uint32_t)r.w << 32) | (uint32_t)r.z; }

/* f(std::integral_constant<int, 0>) ... f(std::integral_constant<int, N-1>) */
template <int N, int I = 0, class F>
DLK_DEV void static_for(F &&f) {
    if constexpr (I < N) {
        f(std::integral_constant<int, I>{});
        static_for<N, I + 1>(f);
    }
}

/* r = lane == K ? y : cur: the one-lane mask is made in VCC by a scalar
 * shift (no scalar register held, no lane compare), then one v_cndmask. */
template <int K>
DLK_DEV float select_lane(float cur, float y) {
    float r;
    asm("s_lshl_b64 vcc, 1, %3\n\tv_cndmask_b32_e32 %0, %1, %2, vcc" : "=v"(r) : "v"(cur), "v"(y), "n"(K) : "vcc");
    return r;
}

/* c + q[0] + ... in order in every lane (the whole chunk read by every lane,
 * an LDS broadcast), lane k keeping the running value after q[k]; returns the
 * first of the first `count` positions whose value reaches thr_f (64 if none)
 * and that value, and the chunk's end value in `fin`.  Values past count must
 * be zero. */
DLK_DEV int chunk_serial_find(float c, const float *q, float thr_f, int count, float &val, float &fin) {
    const float4 *src = (const float4 *)q;
    float4 a[16];
#pragma unroll
    for (int k = 0; k < 16; k++) a[k] = src[k];
    float mine = 0.0f;
    static_for<16>([&](auto kk) {
        constexpr int k = decltype(kk)::value;
        c = c + a[k].x;
        mine = select_lane<4 * k>(mine, c);
        c = c + a[k].y;
        mine = select_lane<4 * k + 1>(mine, c);
        c = c + a[k].z;
        mine = select_lane<4 * k + 2>(mine, c);
        c = c + a[k].w;
        mine = select_lane<4 * k + 3>(mine, c);
    });
    fin = c;
    const int f = first_lane(ballot(lane_id() < count && mine >= thr_f));
    val = f < 64 ? readlanef(mine, f) : c;
    return f;
}

/* Staged values of one element-level chunk as chunk_split_sum reads them:
 * lane 0 the first 32, every other lane the last 32; and the first half's sum. */
struct HalfChunk {
    float4 a[8];
    double shalf;
};
DLK_DEV void load_half_chunk(const float *q, double shalf, HalfChunk &h) {
    const float4 *src = (const float4 *)(q + (lane_id() == 0 ? 0 : 32));
#pragma unroll
    for (int k = 0; k < 8; k++) h.a[k] = src[k];
    h.shalf = shalf;
}

/* c0 + q[0] + ... + q[63] in order, with half the dependent additions: lane 0
 * adds q[0..32) to c0; lanes 1..63 each add q[32..64) to one of the 63
 * consecutive floats around the predicted midpoint c0 + shalf.  32 float
 * additions move the running value at most 16 of its ulps from the real sum,
 * so the exact midpoint is among the starts -29 .. +33 floats from the
 * prediction (the upward side allows for the ulp doubling at a binade edge);
 * lane 0's result picks the lane that started there.  Should the midpoint
 * ever fall outside, the second half is added in order from it (q in LDS). */
DLK_DEV float chunk_split_sum(float c0, const HalfChunk &h, const float *q) {
    const int lane = lane_id();
    const uint32_t pu = f2u((float)((double)c0 + h.shalf));
    float c = lane == 0 ? c0 : u2f(pu + (uint32_t)(lane - 30));
#pragma unroll
    for (int k = 0; k < 8; k++) {
        c = c + h.a[k].x;
        c = c + h.a[k].y;
        c = c + h.a[k].z;
        c = c + h.a[k].w;
    }
    const uint32_t mid = (uint32_t)__builtin_amdgcn_readlane((int)f2u(c), 0);
    const int d = (int)(mid - pu) + 30;
    if (d >= 1 && d <= 63) return u2f((uint32_t)__builtin_amdgcn_readlane((int)f2u(c), d));
    float r = u2f(mid);
    for (int k = 32; k < 64; k++) r = r + q[k];
    return r;
}

/* Exact state of a walk between chunks: next chunk j, running value join_f(b, m). */
struct WalkState {
    int j;
    int b;
    uint32_t m;
};
/* pos >= 0: the first position whose running value reaches the threshold, and
 * that value; pos == -1: no position up to n (value = final running value);
 * need >= 0: the walk stopped at chunk `need`, which is not staged. */
struct WalkOut {
    int pos;
    float value;
    int need;
};

DLK_DEV int sreadi(int v) { return __builtin_amdgcn_readfirstlane(v); }

/* Smallest m on the grid of binade b with join_f(b, m) >= thr_v, saturated at 2^25. */
DLK_DEV uint32_t grid_threshold(double thr_v, int b) {
    const uint64_t t64 = ceil_div_pow2(thr_v, b - 23);
    return t64 < (1ull << 25) ? (uint32_t)t64 : (1u << 25);
}

/* Walks the running float sum c + q(0) + ... from state st over n elements
 * (one wave, uniform control flow): runs are crossed with their integer
 * totals, any other chunk is summed element by element from its staged values
 * (svals[slot * 64 ...], 16-byte aligned).  The record of the chunk after an
 * element-level chunk is read while that chunk is summed.  Elements past n in
 * the last chunk and in run totals must be zero. */
__device__ __forceinline__ WalkOut walk_recs(int n, const int4 *recs, const float *svals, double thr_v,
                                             WalkState &st) {
    const int lane = lane_id();
    const int nch = (n + 63) >> 6;
    int b = sreadi(st.b), j = sreadi(st.j);
    uint32_t m = (uint32_t)sreadi((int)st.m);
    uint32_t thr = grid_threshold(thr_v, b);
    if (j >= nch) return WalkOut{-1, join_f(b, m), -1};
    int4 r = recs[j];
    while (true) {
        int x = sreadi(r.x);
        if (rec_bh(x) == b) {
            const uint32_t lim = thr < (1u << 24) ? thr : (1u << 24);
            uint64_t tot = ((uint64_t)(uint32_t)sreadi(r.w) << 32) | (uint32_t)sreadi(r.z);
            const int nx = sreadi(r.y);
            if ((uint64_t)m + tot < lim) {
                m += (uint32_t)tot;
                j = nx;
                if (j >= nch) break;
                r = recs[j];
                continue;
            }
            /* the limit is reached inside the run: find the chunk, first the
             * segment of ceil(len / 64) chunks that holds it (one ballot over
             * the segment ends), then the chunk */
            {
                const int len = nx - j, step = (len + 63) >> 6;
                if (step > 1) {
                    const int nseg = (len + step - 1) / step;
                    const int k1 = j + min((lane + 1) * step, len);
                    const uint64_t t1 = lane < nseg && k1 < nx ? rec_tot(recs[k1]) : 0;
                    const int sg = min(first_lane(ballot(lane < nseg && (uint64_t)m + (tot - t1) >= lim)), nseg - 1);
                    if (sg > 0) {
                        const uint64_t ts = readlane64(t1, sg - 1);     /* suffix total at the segment's start */
                        m += (uint32_t)(tot - ts);
                        tot = ts;
                        j += sg * step;
                    }
                }
            }
            while (true) {
                const int k = j + lane;
                const uint64_t tk = k < nx ? rec_tot(recs[k]) : 0;
                const uint64_t tk1 = k + 1 < nx ? rec_tot(recs[k + 1]) : 0;
                const int f = first_lane(ballot(k < nx && (uint64_t)m + (tot - tk1) >= lim));
                if (f < 64) {
                    m += (uint32_t)(tot - readlane64(tk, f));
                    j += f;
                    break;
                }
                const uint64_t tn = readlane64(tk1, 63);
                m += (uint32_t)(tot - tn);
                tot = tn;
                j += 64;
            }
            r = recs[j];
            x = sreadi(r.x);
        }
        const int sl = rec_slot(x);
        if (sl < 0) {
            st.j = j;
            st.b = b;
            st.m = m;
            return WalkOut{-1, 0.0f, j};
        }
        const float *q = svals + sl * 64;
        const int4 rn = recs[j + 1 < nch ? j + 1 : j];
        const float c0 = join_f(b, m);
        float fin, val;
        const int f = chunk_serial_find(c0, q, (float)thr_v, min(64, n - j * 64), val, fin);
        if (f < 64) return WalkOut{j * 64 + f, val, -1};   /* the threshold is crossed in this chunk */
        uint64_t m64;
        split(fin, b, m64);
        b = sreadi(b);
        m = (uint32_t)sreadi((int)(uint32_t)m64);
        thr = grid_threshold(thr_v, b);
        if (++j >= nch) break;
        r = rn;
    }
    st.j = j;
    st.b = b;
    st.m = m;
    return WalkOut{-1, join_f(b, m), -1};
}

/* chunk_split_sum for the walk's inner loop, without a branch: the candidate
 * lane that started at the exact midpoint is read with a lane read at a scalar
 * index (the candidates start from the prediction while it is still in vector
 * registers; only the window offset goes through a scalar register).  mid:
 * the exact running value after 32 elements; inw false when the midpoint fell
 * outside the candidate window (the result is then not the chunk's end value). */
DLK_DEV float split_step(float c, const HalfChunk &h, float &mid, bool &inw) {
    const int lane = lane_id();
    const uint32_t pv = f2u((float)((double)c + h.shalf));
    float y = lane == 0 ? c : u2f(pv + (uint32_t)(lane - 30));
#pragma unroll
    for (int k = 0; k < 8; k++) {
        y = y + h.a[k].x;
        y = y + h.a[k].y;
        y = y + h.a[k].z;
        y = y + h.a[k].w;
    }
    const uint32_t pu = (uint32_t)sreadi((int)pv);
    mid = readlanef(y, 0);
    const uint32_t d = f2u(mid) - pu + 30u;
    inw = d - 1u < 63u;
    return readlanef(y, inw ? (int)d : 0);
}

/* The common shape of a walk: run, element-level chunk, run, element-level
 * chunk, ...  el[0..ne) lists the slice's element-level chunks in order with
 * their staged slots (-1: not staged; the walk hands over to walk_recs before
 * it).  Lane l holds list entry l and the run after it as one exact float
 * step: R = its integer increments on the grid of its binade b, valid while the
 * running value stays in [2^b, 2^(b+1)) (then every addition inside the run is
 * exact on that grid, so the run adds exactly R).  A step sums the element
 * chunk with split_step, whose values were read during the previous step, and
 * crosses the run after it.  Branches cost far more than arithmetic here (a
 * uniform branch about 60 cycles against 5.5 for a dependent add), so the
 * checks are combined without short-circuits and the loop test is the step's
 * only branch; the state advances by selects.  Anything else (a run
 * of another binade, the threshold inside a run or chunk, a chunk not in the
 * list, the list's end) leaves the loop: the threshold inside the chunk is
 * resolved here, the rest continues in walk_recs from the exact state reached. */
__device__ __forceinline__ WalkOut walk_pairs(int n, const int4 *recs, const float *svals, const double *shalf,
                                              const int2 *el, int ne, double thr_v, WalkState &st) {
    const int lane = lane_id();
    const int nch = (n + 63) >> 6;
    const float thr_f = (float)thr_v;
    int j = sreadi(st.j);
    float c = join_f(sreadi(st.b), (uint32_t)sreadi((int)st.m));
    const int cnt = min(64, ne);
    if (cnt <= 0) goto general;
    {
        const int2 my_el = lane < cnt ? el[lane] : make_int2(nch, -1);
        /* the run after entry `lane`: fl 1 = it ends at the next entry, 2 = it
         * ends at the slice's end; R, [lo, hi) as above (lo = +inf: unusable) */
        float R = 0.0f, lo = INFINITY, hi = 0.0f;
        int fl = 0;
        {
            const int nx = __shfl_down(my_el.x, 1, 64), nsl = __shfl_down(my_el.y, 1, 64);
            const int c1 = my_el.x + 1;
            const bool has_next = lane + 1 < cnt && nx < nch && nsl >= 0;
            const int stop = has_next ? nx : nch;
            if (my_el.x < nch && (has_next || lane + 1 == cnt)) {
                if (c1 == stop) {
                    lo = 0.0f;
                    hi = INFINITY;
                    fl = has_next ? 1 : 2;
                } else if (c1 < stop) {
                    const int4 rr = recs[c1];
                    const int rb = rec_bh(rr.x);
                    const uint64_t tt = rec_tot(rr);
                    if (rr.y == stop && rb != kInvalidBinade && rb > -126 && tt < (1ull << 24)) {
                        R = ldexpf((float)tt, rb - 23);
                        lo = ldexpf(1.0f, rb);
                        hi = ldexpf(1.0f, rb + 1);
                        fl = has_next ? 1 : 2;
                    }
                }
            }
        }
        int i = 0;
        while (i < cnt && __builtin_amdgcn_readlane(my_el.x, i) < j) i++;
        if (i == cnt) goto general;
        {
            const int e = __builtin_amdgcn_readlane(my_el.x, i);
            if (e >= nch) goto general;
            if (j < e) {
                /* the run from j to the first entry */
                const int4 rr = recs[j];
                const int rb = rec_bh(sreadi(rr.x));
                const uint64_t tt = ((uint64_t)(uint32_t)sreadi(rr.w) << 32) | (uint32_t)sreadi(rr.z);
                if (sreadi(rr.y) != e || rb == kInvalidBinade || rb <= -126 || tt >= (1ull << 24)) goto general;
                const float R0 = ldexpf((float)tt, rb - 23);
                if (!(c >= ldexpf(1.0f, rb) && c + R0 < fminf(ldexpf(1.0f, rb + 1), thr_f))) goto general;
                c = c + R0;
                j = e;
            }
        }
        if (__builtin_amdgcn_readlane(my_el.y, i) < 0) goto general;
        /* one buffer: the next chunk's values are read once this chunk's
         * additions have consumed the registers, while the step finishes */
        HalfChunk H;
        {
            const int sl = __builtin_amdgcn_readlane(my_el.y, i);
            load_half_chunk(svals + sl * 64, shalf[sl], H);
            /* nothing outstanding at the loop head, so the compiler's wait
             * counting at the back edge starts from an empty count */
            __builtin_amdgcn_s_waitcnt(0xc07f);
        }
        float ce, mid;
        bool inw, ok;
        int fi;
        /* one uniform branch per step: the loop test */
        do {
            fi = __builtin_amdgcn_readlane(fl, i);
            ce = split_step(c, H, mid, inw);
            {
                /* the next entry's values (this entry's again at the list's end) */
                const int sl2 = __builtin_amdgcn_readlane(my_el.y, fi == 1 ? i + 1 : i);
                load_half_chunk(svals + sl2 * 64, shalf[sl2], H);
            }
            const float Ri = readlanef(R, i), loi = readlanef(lo, i), hii = readlanef(hi, i);
            const float cn = ce + Ri;
            ok = inw & (ce < thr_f) & (ce >= loi) & (cn < fminf(hii, thr_f));
            const bool go = ok & (fi == 1);
            c = go ? cn : c;
            i = go ? i + 1 : i;
            if (!go) break;
        } while (true);
        __builtin_amdgcn_s_waitcnt(0xc07f);
        if (ok) return WalkOut{-1, ce + readlanef(R, i), -1};      /* the slice's end */
        {
            /* entry i's chunk was summed from c; ce is its end value if inw */
            const int e = __builtin_amdgcn_readlane(my_el.x, i);
            const int sl = __builtin_amdgcn_readlane(my_el.y, i);
            const float *q = svals + sl * 64;
            if (!inw) {
                float r = mid;
                for (int k = 32; k < 64; k++) r = r + q[k];
                ce = r;
            }
            if (ce >= thr_f) {
                float fin, val;
                const int f = chunk_serial_find(c, q, thr_f, min(64, n - e * 64), val, fin);
                return WalkOut{e * 64 + f, val, -1};
            }
            c = ce;
            j = e + 1;
        }
    }
general:
    {
        int b;
        uint64_t m64;
        split(c, b, m64);
        st.j = j;
        st.b = sreadi(b);
        st.m = (uint32_t)sreadi((int)(uint32_t)m64);
    }
    return walk_recs(n, recs, svals, thr_v, st);
}

}  // namespace dlk

#endif
