/*
 * capi.hip -- host side of the batched C ABI (include/diskllm_amd.h): argument
 * checks, the scalars the reference computes on the host side of its loops
 * (1/temperature, the top-p threshold), LDS planning and the launch.
 */
#include <math.h>
#include <string.h>

#include <hip/hip_runtime.h>

#include "sampler_params.h"

extern "C" int dlk_launch_row_kernel(const dlk::RowParams *p, int rows, size_t lds_bytes, hipStream_t stream);

namespace {

constexpr size_t kMaxLds = 160 * 1024;
constexpr int kMaxTopK = 4096;

size_t r16(size_t b) { return (b + 15) & ~(size_t)15; }

int pow2_at_least(int v, int lo) {
    int p = lo;
    while (p < v) p <<= 1;
    return p;
}

size_t aggs_bytes(int n) {
    size_t nch = ((size_t)n + 63) / 64, ngr = (nch + 63) / 64;
    return 2 * r16(nch * 8) + r16(nch * 4) + 2 * r16(ngr * 8) + r16(ngr * 4) + r16((nch + 1) * 8);
}

/* Smallest double d with (float)d >= tp, for tp > 0 finite: the boundary of the
 * test (float)cumul >= top_p (src/sampler.c:211). */
double topp_threshold(float tp) {
    float lo = nextafterf(tp, 0.0f);
    double mid = ((double)lo + (double)tp) * 0.5;
    if ((float)mid >= tp) return mid;
    return nextafter(mid, INFINITY);
}

}  // namespace

extern "C" uint64_t dlk_seed_state(uint64_t seed) { return seed ? seed : 0xDEADBEEF12345678ULL; }

extern "C" int dlk_sample(const dlk_batch *b, int rows, int vocab, const dlk_sample_params *prm,
                          hipStream_t stream) {
    if (!b || !prm || rows <= 0 || vocab <= 0 || !b->logits || !b->out_ids || b->ld < vocab) return DLK_ERR_INVALID;
    if (prm->n_out < 0) return DLK_ERR_INVALID;
    if ((b->hist_off == nullptr) != (b->hist_ids == nullptr)) return DLK_ERR_INVALID;
    if (b->mask && b->mask_ld < (vocab + 31) / 32) return DLK_ERR_INVALID;
    dlk::RowParams p;
    memset(&p, 0, sizeof(p));
    p.logits = b->logits; p.ld = b->ld; p.V = vocab;
    p.hist_off = b->hist_off; p.hist_ids = b->hist_ids;
    p.mask = b->mask; p.mask_ld = b->mask_ld; p.mask_row = b->mask_row;
    p.rng = b->rng; p.out_ids = b->out_ids;
    p.out_cand_ids = b->out_cand_ids; p.out_cand_probs = b->out_cand_probs; p.out_cand_logprobs = b->out_cand_logprobs;
    p.n_out = prm->n_out; p.status = b->status;
    p.top_p = prm->top_p; p.min_p = prm->min_p;
    p.rep = prm->repeat_penalty; p.freq = prm->frequency_penalty; p.pres = prm->presence_penalty;
    p.order = prm->penalty_order;
    p.greedy = prm->temperature == 0.0f;                        /* src/sampler.c:140 */
    if (!p.greedy) {
        if (!b->rng) return DLK_ERR_INVALID;
        p.inv_temp = 1.0f / prm->temperature;                   /* src/sampler.c:154 */
        if (!(p.inv_temp > 0.0f) || isinf(p.inv_temp)) return DLK_ERR_UNSUPPORTED;
    }
    p.topk_on = prm->top_k > 0 && prm->top_k < vocab;           /* src/sampler.c:166 */
    p.top_k = prm->top_k;
    if (p.topk_on && prm->top_k > kMaxTopK) return DLK_ERR_UNSUPPORTED;
    p.topp_on = prm->top_p < 1.0f;                              /* src/sampler.c:205 */
    p.topp_thr = (p.topp_on && prm->top_p > 0.0f) ? topp_threshold(prm->top_p) : 0.0;
    p.minp_on = prm->min_p > 0.0f;                              /* src/sampler.c:188 */

    dlk::LdsPlan &pl = p.plan;
    int max_hist = prm->max_history > 0 ? prm->max_history : 1024;
    pl.hcap = b->hist_off ? pow2_at_least(max_hist, 64) : 64;
    int nch = (vocab + 63) / 64;
    pl.flag_words = (nch + 31) / 32;
    pl.kp = p.topk_on ? pow2_at_least(p.top_k, 64) : 0;
    size_t fixed = r16(32 * 8) + r16(64 * 8) + r16(16 * 8) + r16(64 * 4) + 4 * r16((size_t)pl.hcap * 4) +
                   r16((size_t)pl.flag_words * 4);
    size_t region = 0;
    if (!p.greedy) {
        if (p.topk_on) region = r16((size_t)pl.kp * 8) + (aggs_bytes(p.top_k) > 8192 ? aggs_bytes(p.top_k) : 8192);
        else region = aggs_bytes(vocab);
    }
    size_t total = fixed + region;
    if (total > kMaxLds) return DLK_ERR_UNSUPPORTED;
    pl.bytes = (int)total;
    return dlk_launch_row_kernel(&p, rows, total, stream) == 0 ? DLK_OK : DLK_ERR_HIP;
}
