/*
 * dropin_ctx.c -- device staging for the host-pointer drop-ins.
 */
#include <pthread.h>
#include <string.h>

#include "diskllm_amd.h"
#include "dropin.h"

int dlk_dropin_init(dlk_dropin_ctx *c) {
    memset(c, 0, sizeof(*c));
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) return -1;
    if (hipMalloc((void **)&c->hoff, 2 * sizeof(int32_t)) != hipSuccess) goto fail;
    if (hipMalloc((void **)&c->rng, sizeof(uint64_t)) != hipSuccess) goto fail;
    if (hipMalloc((void **)&c->ids, 2 * sizeof(int32_t)) != hipSuccess) goto fail;
    if (hipMalloc((void **)&c->status, sizeof(uint32_t)) != hipSuccess) goto fail;
    return 0;
fail:
    dlk_dropin_release(c);
    return -1;
}

void dlk_dropin_release(dlk_dropin_ctx *c) {
    if (c->stream) {
        hipStreamSynchronize(c->stream);
        (void)dlk_release_stream(c->stream);
    }
    hipFree(c->logits);
    hipFree(c->hist);
    hipFree(c->hoff);
    hipFree(c->rng);
    hipFree(c->ids);
    hipFree(c->status);
    hipFree(c->mask);
    if (c->stream) hipStreamDestroy(c->stream);
    memset(c, 0, sizeof(*c));
}

int dlk_dropin_reserve(dlk_dropin_ctx *c, int vocab, int hist) {
    if (vocab > c->cap) {
        hipStreamSynchronize(c->stream);
        hipFree(c->logits);
        hipFree(c->mask);
        c->logits = NULL;
        c->mask = NULL;
        c->cap = c->mask_cap = 0;
        if (hipMalloc((void **)&c->logits, (size_t)vocab * sizeof(float)) != hipSuccess) return -1;
        if (hipMalloc((void **)&c->mask, (size_t)((vocab + 31) / 32) * sizeof(uint32_t)) != hipSuccess) return -1;
        c->cap = vocab;
        c->mask_cap = (vocab + 31) / 32;
    }
    if (hist > c->hist_cap) {
        hipStreamSynchronize(c->stream);
        hipFree(c->hist);
        c->hist = NULL;
        c->hist_cap = 0;
        if (hipMalloc((void **)&c->hist, (size_t)hist * sizeof(int32_t)) != hipSuccess) return -1;
        c->hist_cap = hist;
    }
    return 0;
}

static pthread_mutex_t g_lock = PTHREAD_MUTEX_INITIALIZER;
static dlk_dropin_ctx g_ctx;
static int g_ready;

dlk_dropin_ctx *dlk_dropin_shared_lock(void) {
    pthread_mutex_lock(&g_lock);
    if (!g_ready) {
        if (dlk_dropin_init(&g_ctx) != 0) {
            pthread_mutex_unlock(&g_lock);
            return NULL;
        }
        g_ready = 1;
    }
    return &g_ctx;
}

void dlk_dropin_shared_unlock(void) { pthread_mutex_unlock(&g_lock); }
