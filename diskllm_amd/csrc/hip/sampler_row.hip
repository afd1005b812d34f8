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
    R.M = 0.0f; R.inv_t = p.inv_temp; R.maxv = 0.0f; R.tab = L.tab;

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
    if (irr && p.topk_on) {
        if (t == 0) emulate_topk_row(p, R, k, r, (uint64_t *)L.region, row);
        return;
    }
    if (irr || !(bv > -INFINITY)) {
        /* without top-k a NaN or +inf entry makes the softmax sum NaN (+inf - max
         * is NaN): as for a row of -inf, no comparison with it holds and the draw
         * falls through to the last candidate */
        /* every entry -inf: the softmax is NaN throughout and the draw falls
         * through to the last candidate, which is index k-1 in index order */
        if (t == 0) p.out_ids[row] = k - 1;
        for (int j = t; j < n_out; j += blockDim.x) {
            if (p.out_cand_ids) p.out_cand_ids[(int64_t)row * n_out + j] = j < k ? j : -1;
            if (p.out_cand_probs) p.out_cand_probs[(int64_t)row * n_out + j] = NAN;
            if (p.out_cand_logprobs) p.out_cand_logprobs[(int64_t)row * n_out + j] = NAN;
        }
        return;
    }
    R.M = bv;
    Scal S;
    int pos, tok;
    if (p.topk_on) {
        const int kp = pl.kp;
        uint64_t *cand = (uint64_t *)L.region;
        uint32_t *hist = (uint32_t *)(L.region + (size_t)kp * 8);
        select_top_k(R, k, cand, kp, hist, L);
        CandBase cb{&R, cand};
        R.maxv = cb.s(0);                 /* sorted: buf[0] is the maximum (src/sampler.c:173-176) */
        unsigned char *reg = L.region + (size_t)kp * 8;
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
