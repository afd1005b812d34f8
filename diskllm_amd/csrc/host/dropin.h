/*
 * dropin.h -- device staging shared by the host-pointer drop-ins (sampler.h,
 * grammar.h): one stream and grow-only device buffers per context.
 */
#ifndef DLK_DROPIN_H
#define DLK_DROPIN_H

#include <stdint.h>

#include <hip/hip_runtime_api.h>

typedef struct {
    hipStream_t stream;
    float *logits;       /* [cap] */
    int cap;
    int32_t *hist;       /* [hist_cap] */
    int hist_cap;
    int32_t *hoff;       /* [2] */
    uint64_t *rng;       /* [1] */
    int32_t *ids;        /* [2]: token, valid count */
    uint32_t *status;    /* [1] */
    uint32_t *mask;      /* [mask_cap] words */
    int mask_cap;
} dlk_dropin_ctx;

int dlk_dropin_init(dlk_dropin_ctx *c);
void dlk_dropin_release(dlk_dropin_ctx *c);
int dlk_dropin_reserve(dlk_dropin_ctx *c, int vocab, int hist);

/* The process-wide context of the stateless calls, locked while in use. */
dlk_dropin_ctx *dlk_dropin_shared_lock(void);
void dlk_dropin_shared_unlock(void);

#endif
