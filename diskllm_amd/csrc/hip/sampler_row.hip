/*
 * sampler_row.hip -- one workgroup per row: the whole src/sampler.c pipeline
 * (penalties -> temperature -> top-k -> softmax -> min-p -> top-p -> draw) for
 * one row of logits, bit-exact with the reference.
 *
 * This kernel is the general path: every configuration can run through it, and
 * the multi-workgroup fast paths fall back to it for rows they cannot certify.
 * It streams the row from global memory several times (the row stays in L2/MALL
 * after the first pass) and keeps everything else in LDS.
 */
#include "sampler_common.h"

namespace dlk {

/* ------------------------------------------------------------------- kernel */

__global__ __launch_bounds__(1024) void row_kernel(RowParams p) {
    extern __shared__ __align__(16) unsigned char smem[];
    const LdsPlan pl = p.plan;
    Lds L = make_lds(smem, pl);
    const int row = blockIdx.x, t = threadIdx.x, lane = lane_id();
    const int V = p.V;
    const float *lg = p.logits + (int64_t)row * p.ld;
    const uint32_t *mk = nullptr;
    if (p.mask) mk = p.mask + (int64_t)(p.mask_row ? p.mask_row[row] : row) * p.mask_ld;
    if (t < 32) L.tab[t] = kExp2Tab[t];

    if (p.hist_off && p.hist_off[row + 1] - p.hist_off[row] > pl.hcap) {
        if (t == 0) {
            p.out_ids[row] = -1;
            if (p.status) atomicOr(p.status, DLK_STATUS_HISTORY_TOO_LONG);
        }
        return;
    }
    int np = build_patches(p, row, lg, mk, L, pl, V);

    Row R;
    R.lg = lg; R.mk = mk; R.V = V; R.pid = L.pid; R.pval = L.pval; R.np = np; R.pflag = L.pflag;
    R.M = 0.0f; R.inv_t = p.inv_temp; R.maxv = 0.0f; R.tab = L.tab; R.cap = p.cap;

    /* max / argmax over the prepared row (src/sampler.c:9-19, :155-158) */
    float bv = -INFINITY;
    int bidx = 0x7fffffff;
    int irr = 0;                                  /* NaN or +inf after the mask and penalties */
    for (int i = t; i < V; i += blockDim.x) {
        float x = prepared(R, i);
        if (x > bv || (x == bv && i < bidx)) { bv = x; bidx = i; }
        irr |= !(x < INFINITY) && !(x == -INFINITY);
    }
    block_argmax(bv, bidx, L);
    irr = block_sum_int(irr, L);
    const bool first_nan = isnan(prepared(R, 0));

    const int n_out = p.n_out;
    if (p.greedy) {
        if (t == 0) p.out_ids[row] = (first_nan || bidx == 0x7fffffff) ? 0 : bidx;
        for (int j = t; j < n_out; j += blockDim.x) {
            if (p.out_cand_ids) p.out_cand_ids[(int64_t)row * n_out + j] = -1;
            if (p.out_cand_probs) p.out_cand_probs[(int64_t)row * n_out + j] = 0.0f;
            if (p.out_cand_logprobs) p.out_cand_logprobs[(int64_t)row * n_out + j] = -INFINITY;
        }
        return;
    }
    /* one uniform per non-greedy sample (src/sampler.c:225) */
    uint64_t st = xorshift64(p.rng[row]);
    const float r = rand_f32_from(st);
    __syncthreads();
    if (t == 0) p.rng[row] = st;

    const int k = p.topk_on ? p.top_k : V;
    /* s = (l - max) * (1/T) holding NaN (snan) or +inf (spinf): with 1/T in
     * (0, inf) exactly when a prepared logit is NaN or +inf; otherwise checked
     * on s itself, whose maximum (src/sampler.c:173-176) is then not 0 */
    bool snan = irr != 0, spinf = false;
    float maxs = 0.0f;
    R.M = bv;
    if (p.s_general && !irr && bv > -INFINITY) {
        float m = -INFINITY;
        int fl = 0;
        for (int i = t; i < V; i += blockDim.x) {
            const float s = scaled(R, i);
            if (s != s) fl |= 1;
            else if (s == INFINITY) fl |= 2;
            else m = fmaxf(m, s);
        }
        m = wave_max_dpp(m);
        for (int o = 32; o >= 1; o >>= 1) fl |= shfl_xor(fl, o);
        float *rm = (float *)L.red;
        int *rf = (int *)(L.red + 32);
        if (lane == 0) { rm[wave_id()] = m; rf[wave_id()] = fl; }
        __syncthreads();
        m = -INFINITY;
        fl = 0;
        for (int w2 = 0; w2 < n_waves(); w2++) { m = fmaxf(m, rm[w2]); fl |= rf[w2]; }
        __syncthreads();
        snan = (fl & 1) != 0;
        spinf = (fl & 2) != 0;
        maxs = m;
    }
    if (snan && p.topk_on && (k <= kEmulateMaxK || bv > -INFINITY)) {
        if (k <= kEmulateMaxK) {
            if (t == 0) emulate_topk_row(p, R, k, r, (uint64_t *)L.region, row);
            return;
        }
        /* k too large for the one-thread emulation: the reference's insertion
         * sort with NaN keys in closed form (src/sampler.c:109-134).  A NaN never
         * moves (every comparison with it is false) and stops any element moving
         * past it, and no entry past the first k replaces a NaN at k-1 or enters
         * as a NaN.  So with q the last NaN among the first k: if q = k-1 the
         * buffer ends with it; otherwise the entries after q form a window that
         * ends up holding the best k-1-q entries, under (s desc, index asc), of
         * the window's own entries and the non-NaN entries past k.  Any NaN among
         * the first k makes the softmax sum NaN, every comparison of the draw
         * false, and the draw falls through to buf[k-1] (:226-233).  With no NaN
         * among the first k the NaN entries never enter and the ordinary path
         * below selects among the others (NaN keys last). */
        R.M = first_nan ? NAN : bv;               /* the reference's max loop (:155-158) */
        int q = -1;
        for (int i = t; i < k; i += blockDim.x)
            if (isnan(scaled(R, i))) q = i;
        for (int m = 32; m >= 1; m >>= 1) q = max(q, shfl_xor(q, m));
        if (lane == 0) L.bi[32 + wave_id()] = q;
        __syncthreads();
        for (int w2 = 0; w2 < n_waves(); w2++) q = max(q, L.bi[32 + w2]);
        __syncthreads();
        if (q >= 0) {
            int tok = k - 1;
            if (q < k - 1) {
                const int win = k - 1 - q;
                auto key_of = [&](int i) {
                    const float s = scaled(R, i);
                    return (i <= q || s != s) ? 0xffffffffu : desc_key(s);
                };
                const KthKey kk = radix_kth_keys(key_of, V, win, (uint32_t *)L.region, L);
                tok = nth_index_with_key(key_of, V, kk.key, win - kk.below, L);
            }
            if (t == 0) p.out_ids[row] = tok;
            /* every probability is NaN; the buffer order is not produced */
            for (int j = t; j < n_out; j += blockDim.x) {
                if (p.out_cand_ids) p.out_cand_ids[(int64_t)row * n_out + j] = -1;
                if (p.out_cand_probs) p.out_cand_probs[(int64_t)row * n_out + j] = NAN;
                if (p.out_cand_logprobs) p.out_cand_logprobs[(int64_t)row * n_out + j] = NAN;
            }
            return;
        }
    }
    if (((snan || spinf) && !p.topk_on) || !(bv > -INFINITY)) {
        /* without top-k a NaN or +inf entry of s makes the softmax sum NaN (+inf -
         * max is NaN): as for a row of -inf, no comparison with it holds and the
         * draw falls through to the last candidate, which is index k-1 in index
         * order (every s of a row of -inf is NaN, so the top-k sort moves nothing) */
        if (t == 0) p.out_ids[row] = k - 1;
        for (int j = t; j < n_out; j += blockDim.x) {
            if (p.out_cand_ids) p.out_cand_ids[(int64_t)row * n_out + j] = j < k ? j : -1;
            if (p.out_cand_probs) p.out_cand_probs[(int64_t)row * n_out + j] = NAN;
            if (p.out_cand_logprobs) p.out_cand_logprobs[(int64_t)row * n_out + j] = NAN;
        }
        return;
    }
    Scal S;
    int pos, tok;
    if (p.topk_on) {
        uint64_t *cand;
        unsigned char *reg;
        if (p.gcand) {
            /* k too large for LDS: candidates and aggregates in global memory */
            cand = p.gcand + (int64_t)row * p.gcand_stride;
            reg = p.gregion + (int64_t)row * p.gregion_stride;
            uint32_t *hist = (uint32_t *)L.region;
            select_top_k_global(R, k, cand, cand + p.gcand_stride / 2, hist, hist + 2048, L);
        } else {
            const int kp = pl.kp;
            cand = (uint64_t *)L.region;
            uint32_t *hist = (uint32_t *)(L.region + (size_t)kp * 8);
            select_top_k(R, k, cand, kp, hist, L);
            reg = L.region + (size_t)kp * 8;
        }
        CandBase cb{&R, cand};
        R.maxv = cb.s(0);                 /* sorted: buf[0] is the maximum (src/sampler.c:173-176) */
        if (spinf || !(R.maxv > -INFINITY)) {
            /* +inf at the top of the sorted candidates, or every candidate -inf (1/T
             * infinite leaves -inf below the NaN at the maximum): e = expf(s - max_v)
             * is NaN there, so the sum, every probability and every comparison of the
             * draw are NaN and the draw falls through to buf[k-1] (src/sampler.c:233) */
            if (t == 0) p.out_ids[row] = cb.token(k - 1);
            for (int j = t; j < n_out; j += blockDim.x) {
                int64_t o = (int64_t)row * n_out + j;
                if (p.out_cand_ids) p.out_cand_ids[o] = j < k ? cb.token(j) : -1;
                if (p.out_cand_probs) p.out_cand_probs[o] = j < k ? NAN : 0.0f;
                if (p.out_cand_logprobs) p.out_cand_logprobs[o] = -INFINITY;
            }
            return;
        }
        pos = pipeline(p, cb, k, r, reg, L, S);
        tok = cb.token(pos);
        if (t == 0) p.out_ids[row] = tok;
        for (int j = t; j < n_out; j += blockDim.x) {
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
    } else {
        R.maxv = maxs;                    /* 0 unless 1/T is outside (0, inf) */
        FullBase fb{&R};
        pos = pipeline(p, fb, V, r, L.region, L, S);
        if (t == 0) p.out_ids[row] = pos;
        for (int j = t; j < n_out; j += blockDim.x) {
            int64_t o = (int64_t)row * n_out + j;
            float pj = fb.e(j) * S.inv;
            QDraw<FullBase> qd{&fb, &S};
            float fj = qd(j);
            if (p.out_cand_ids) p.out_cand_ids[o] = j;
            if (p.out_cand_probs) p.out_cand_probs[o] = pj;
            if (p.out_cand_logprobs) p.out_cand_logprobs[o] = fj > 0.0f ? (float)log((double)fj) : -INFINITY;
        }
    }
    (void)lane;
}

}  // namespace dlk

/* ---------------------------------------------------------------- launcher */

extern "C" int dlk_launch_row_kernel(const dlk::RowParams *p, int rows, size_t lds_bytes, hipStream_t stream) {
    static int attr_set = 0;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void *)dlk::row_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                160 * 1024) != hipSuccess)
            return -1;
        attr_set = 1;
    }
    hipLaunchKernelGGL(dlk::row_kernel, dim3(rows), dim3(1024), lds_bytes, stream, *p);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
