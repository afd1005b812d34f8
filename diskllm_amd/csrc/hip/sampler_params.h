/*
 * sampler_params.h -- kernel parameter block shared by the host launchers and
 * the device code (passed by value to the kernels).
 */
#ifndef DLK_SAMPLER_PARAMS_H
#define DLK_SAMPLER_PARAMS_H

#include <stdint.h>

#include "../../../include/diskllm_amd.h"

namespace dlk {

/* LDS layout of the one-workgroup-per-row kernel. */
struct LdsPlan {
    int hcap;        /* history sort capacity (power of two >= 64) */
    int flag_words;  /* words of the per-64-element "has a penalised id" bitmap */
    int kp;          /* top-k candidate capacity (power of two >= k), 0 if top-k is off */
    int bytes;       /* total dynamic LDS */
};

struct RowParams {
    const float *logits;
    int64_t ld;
    int V;
    const int32_t *hist_off;
    const int32_t *hist_ids;
    const uint32_t *mask;
    int64_t mask_ld;
    const int32_t *mask_row;
    uint64_t *rng;
    int32_t *out_ids;
    int32_t *out_cand_ids;
    float *out_cand_probs;
    float *out_cand_logprobs;
    int n_out;
    uint32_t *status;
    float inv_temp, top_p, min_p, rep, freq, pres;
    int top_k;
    uint32_t order;
    double topp_thr;     /* smallest double d with (float)d >= top_p */
    int greedy, topk_on, topp_on, minp_on;
    float cap;           /* > 0: logits soft-capped, cap * tanhf(l / cap), before everything else */
    /* 1/temperature outside (0, inf): s = (l - max) * (1/T) may hold NaN or +inf
     * and its maximum is not 0 (row kernel only) */
    int s_general;
    /* top-k too large for LDS (row kernel only): per row, 2 * gcand_stride/2
     * candidate entries (sort ping-pong) and the pipeline's aggregates */
    uint64_t *gcand;
    int64_t gcand_stride;
    unsigned char *gregion;
    int64_t gregion_stride;
    LdsPlan plan;
};

}  // namespace dlk

#endif
