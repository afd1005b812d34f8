/*
 * dropin_sampler.c -- include/sampler.h on the GPU: the reference's single-row
 * host API (include/sampler.h:19-34, src/sampler.c) as copies around the
 * batched entry points of diskllm_amd.h.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "diskllm_amd.h"
#include "sampler.h"
#include "dropin.h"

struct sampler {
    sampler_config cfg;
    uint64_t rng;            /* host copy of the xorshift state (src/sampler.c:63) */
    int path;                /* DLK_PATH_* of the first attempt (DLK_DROPIN_PATH, tests) */
    dlk_dropin_ctx dev;
};

sampler *sampler_create(const sampler_config *cfg) {
    if (!cfg) return NULL;
    sampler *s = calloc(1, sizeof(*s));
    if (!s) return NULL;
    s->cfg = *cfg;
    s->rng = dlk_seed_state(cfg->seed);                      /* src/sampler.c:87 */
    /* test hook: the implementation the first attempt of each draw uses (e.g.
     * DLK_PATH_FULL_NO_WAIT to force the sync-timeout recovery below) */
    const char *ps = getenv("DLK_DROPIN_PATH");
    s->path = ps ? atoi(ps) : DLK_PATH_AUTO;
    if (dlk_dropin_init(&s->dev) != 0) {
        free(s);
        return NULL;
    }
    return s;
}

void sampler_free(sampler *s) {
    if (!s) return;
    dlk_dropin_release(&s->dev);
    free(s);
}

/* A device failure the reference API has no channel for: said once on stderr. */
static void report_device_failure(const char *what) {
    static int said;
    if (!said) {
        said = 1;
        fprintf(stderr, "libdiskllm_amd: %s could not reach the GPU; continuing as the reference does "
                        "without its resources (src/sampler.c:145-147)\n", what);
    }
}

/* The reference's greedy_sample (src/sampler.c:9-19) on the host row: the
 * answer of sampler_sample and greedy_sample when the device cannot be reached,
 * as the reference degrades to greedy when it cannot get its work buffer
 * (src/sampler.c:145-147, no random number drawn). */
static int host_greedy(const float *logits, int vocab) {
    int best = 0;
    float bv = logits[0];
    for (int i = 1; i < vocab; i++)
        if (logits[i] > bv) { bv = logits[i]; best = i; }
    return best;
}

/* One row through dlk_sample on `c` with the rng state *rng; on success the
 * token, the status word in *status and the advanced state in *rng_out (not
 * greedy); -1 when a device call fails. */
static int sample_one(dlk_dropin_ctx *c, const float *logits, int vocab, float temperature, int top_k, float top_p,
                      float min_p, int path, const uint64_t *rng, uint64_t *rng_out, uint32_t *status) {
    if (dlk_dropin_reserve(c, vocab, 0) != 0) return -1;
    const int greedy = temperature == 0.0f;
    if (hipMemcpyAsync(c->logits, logits, (size_t)vocab * sizeof(float), hipMemcpyHostToDevice, c->stream) !=
        hipSuccess)
        return -1;
    if (!greedy &&
        hipMemcpyAsync(c->rng, rng, sizeof(uint64_t), hipMemcpyHostToDevice, c->stream) != hipSuccess)
        return -1;
    dlk_batch b;
    memset(&b, 0, sizeof(b));
    b.logits = c->logits;
    b.ld = vocab;
    b.rng = c->rng;
    b.out_ids = c->ids;
    b.status = c->status;
    dlk_sample_params p;
    memset(&p, 0, sizeof(p));
    p.temperature = temperature;
    p.top_k = top_k;
    p.top_p = top_p;
    p.min_p = min_p;
    p.repeat_penalty = 1.0f;
    p.path = path;
    if (hipMemsetAsync(c->status, 0, sizeof(uint32_t), c->stream) != hipSuccess) return -1;
    if (dlk_sample(&b, 1, vocab, &p, c->stream) != DLK_OK) return -1;
    int32_t id = -1;
    uint32_t st = 0;
    if (hipMemcpyAsync(&id, c->ids, sizeof(int32_t), hipMemcpyDeviceToHost, c->stream) != hipSuccess) return -1;
    if (hipMemcpyAsync(&st, c->status, sizeof(uint32_t), hipMemcpyDeviceToHost, c->stream) != hipSuccess) return -1;
    uint64_t r = 0;
    if (!greedy && hipMemcpyAsync(&r, c->rng, sizeof(uint64_t), hipMemcpyDeviceToHost, c->stream) != hipSuccess)
        return -1;
    if (hipStreamSynchronize(c->stream) != hipSuccess) return -1;
    *status = st;
    if (!greedy) *rng_out = r;
    return id;
}

/* The reference always returns a token (src/sampler.c:136-234): its caller
 * feeds it straight to the next decode step (src/cli/main.c:386-388).  A
 * launch whose cross-workgroup wait gave up (another kernel holding the GPU)
 * is run again on the row kernel, which has no such waits, from the same rng
 * state, so the token and the state are the reference's; if the device
 * cannot be reached at all the row is sampled greedily on the host, without
 * drawing, as the reference does when it has no work buffer. */
int sampler_sample(sampler *s, float *logits, int vocab_size) {
    if (!s || !logits || vocab_size <= 0) return -1;
    const sampler_config *cf = &s->cfg;
    uint64_t next = s->rng;
    uint32_t st = 0;
    int id = sample_one(&s->dev, logits, vocab_size, cf->temperature, cf->top_k, cf->top_p, cf->min_p, s->path,
                        &s->rng, &next, &st);
    if (id >= 0 && (st & DLK_STATUS_SYNC_TIMEOUT)) {
        st = 0;
        id = sample_one(&s->dev, logits, vocab_size, cf->temperature, cf->top_k, cf->top_p, cf->min_p, DLK_PATH_ROW,
                        &s->rng, &next, &st);
    }
    if (id < 0 || st != 0 || id >= vocab_size) {
        report_device_failure("sampler_sample");
        return host_greedy(logits, vocab_size);
    }
    if (cf->temperature != 0.0f) s->rng = next;
    return id;
}

int greedy_sample(const float *logits, int vocab_size) {
    if (!logits || vocab_size <= 0) return 0;
    dlk_dropin_ctx *c = dlk_dropin_shared_lock();
    int id = -1;
    uint32_t st = 0;
    if (c) {
        const uint64_t unused = 1;
        uint64_t out = 1;
        id = sample_one(c, logits, vocab_size, 0.0f, 0, 1.0f, 0.0f, DLK_PATH_AUTO, &unused, &out, &st);
        dlk_dropin_shared_unlock();
    }
    if (id < 0 || st != 0 || id >= vocab_size) {
        report_device_failure("greedy_sample");
        return host_greedy(logits, vocab_size);
    }
    return id;
}

/* One penalty op in place on the host row.  Only the touched entries cross
 * PCIe: the logits of the distinct in-range ids (ids outside [0, vocab) are
 * skipped, as the reference skips them) go up as a compact row, the history as
 * slots of that row, the device applies the op there, and the compact row comes
 * back to be written over those ids: 12 bytes per id each way in place of the
 * whole row.  The order of a history does not matter to either op: repetition
 * scales an entry once per occurrence (its sign never changes), presence
 * subtracts once per distinct id. */
typedef struct { int32_t id, pos; } id_pos;

static int cmp_id_pos(const void *a, const void *b) {
    const id_pos *x = (const id_pos *)a, *y = (const id_pos *)b;
    if (x->id != y->id) return x->id < y->id ? -1 : 1;
    return x->pos < y->pos ? -1 : x->pos > y->pos;
}

static void report_penalty_failure(uint32_t op) {
    fprintf(stderr, "libdiskllm_amd: sampler_apply_%s_penalty could not reach the GPU; the row was not "
                    "penalised\n", op == DLK_OP_REPETITION ? "repetition" : "presence");
}

static void penalty_one(float *logits, int vocab, const int *seen, int n, uint32_t op, float value) {
    id_pos *ip = malloc((size_t)n * sizeof(id_pos));
    int32_t *slots = malloc((size_t)n * sizeof(int32_t));
    int32_t *ids = malloc((size_t)n * sizeof(int32_t));
    float *vals = malloc((size_t)n * sizeof(float));
    int m = 0, nd = 0;
    if (ip && slots && ids && vals) {
        for (int i = 0; i < n; i++)
            if (seen[i] >= 0 && seen[i] < vocab) ip[m++] = (id_pos){seen[i], i};
        qsort(ip, (size_t)m, sizeof(id_pos), cmp_id_pos);
        for (int j = 0; j < m; j++) {
            if (j == 0 || ip[j].id != ip[j - 1].id) {
                ids[nd] = ip[j].id;
                vals[nd] = logits[ip[j].id];
                nd++;
            }
            slots[j] = nd - 1;
        }
    }
    int done = nd == 0 && (ip && slots && ids && vals);
    dlk_dropin_ctx *c = nd ? dlk_dropin_shared_lock() : NULL;
    if (c) {
        if (dlk_dropin_reserve(c, nd, m) == 0) {
            const int32_t hoff[2] = {0, m};
            const size_t bytes = (size_t)nd * sizeof(float);
            int ok = hipMemcpyAsync(c->logits, vals, bytes, hipMemcpyHostToDevice, c->stream) == hipSuccess &&
                     hipMemcpyAsync(c->hist, slots, (size_t)m * sizeof(int32_t), hipMemcpyHostToDevice,
                                    c->stream) == hipSuccess &&
                     hipMemcpyAsync(c->hoff, hoff, sizeof(hoff), hipMemcpyHostToDevice, c->stream) == hipSuccess;
            if (ok)
                ok = dlk_apply_penalties(c->logits, nd, 1, nd, c->hoff, c->hist, op,
                                         op == DLK_OP_REPETITION ? value : 1.0f, 0.0f,
                                         op == DLK_OP_PRESENCE ? value : 0.0f, c->stream) == DLK_OK;
            if (ok) ok = hipMemcpyAsync(vals, c->logits, bytes, hipMemcpyDeviceToHost, c->stream) == hipSuccess;
            if (hipStreamSynchronize(c->stream) == hipSuccess && ok) {
                for (int d = 0; d < nd; d++) logits[ids[d]] = vals[d];
                done = 1;
            }
        }
        dlk_dropin_shared_unlock();
    }
    /* the reference's penalties cannot fail (src/sampler.c:21-52); these can
     * only when host or device memory runs out or the GPU is gone: said on
     * stderr rather than passed over in silence */
    if (!done) report_penalty_failure(op);
    free(ip);
    free(slots);
    free(ids);
    free(vals);
}

void sampler_apply_repetition_penalty(float *logits, int vocab_size, const int *seen_tokens, int num_seen,
                                      float penalty) {
    if (penalty <= 1.0f || !seen_tokens || num_seen <= 0 || !logits || vocab_size <= 0) return;   /* :22 */
    penalty_one(logits, vocab_size, seen_tokens, num_seen, DLK_OP_REPETITION, penalty);
}

void sampler_apply_presence_penalty(float *logits, int vocab_size, const int *seen_tokens, int num_seen,
                                    float presence_penalty) {
    if (presence_penalty == 0.0f || !seen_tokens || num_seen <= 0 || !logits || vocab_size <= 0) return;  /* :36 */
    penalty_one(logits, vocab_size, seen_tokens, num_seen, DLK_OP_PRESENCE, presence_penalty);
}
