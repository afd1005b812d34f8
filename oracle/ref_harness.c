/*
 * ref_harness.c -- TEST INFRASTRUCTURE ONLY.
 *
 * Compiled by oracle/Makefile together with the reference's own src/sampler.c
 * (included below from the reference tree via -I<reference>/src) into
 * oracle/_ref/.  It adds two entry points the reference lacks:
 *   refh_sample_trace: one sampler_sample() call that also copies out the first n
 *     work-buffer entries (src/sampler.c:64), which hold the softmax probabilities
 *     when top_p >= 1 and min_p == 0 (src/sampler.c:183-185);
 *   refh_time_batch: the CPU baseline -- rows split over pthreads, one sampler per
 *     thread (instances are not thread-safe), CLOCK_MONOTONIC around penalties +
 *     sampler_sample for every row of the batch.
 * Nothing here changes the reference's arithmetic.
 */
#define _POSIX_C_SOURCE 200809L   /* clock_gettime, pthread barriers */
#include "sampler.c"

#include <pthread.h>
#include <time.h>

int refh_sample_trace(const sampler_config *cfg, uint64_t *rng_inout, float *logits, int vocab,
                      int n, int *out_idx, float *out_val) {
    sampler *s = sampler_create(cfg);
    if (!s) return -1;
    if (rng_inout) s->rng_state = *rng_inout;
    int tok = sampler_sample(s, logits, vocab);
    for (int i = 0; i < n && s->work_buf && i < s->work_cap; i++) {
        out_idx[i] = s->work_buf[i].index;
        out_val[i] = s->work_buf[i].value;
    }
    if (rng_inout) *rng_inout = s->rng_state;
    sampler_free(s);
    return tok;
}

/* Builder-defined frequency penalty (the reference has none): once per distinct
 * id, l -= f * (float)count. */
static void refh_frequency(float *logits, int vocab, const int *seen, int n, float f) {
    if (f == 0.0f || !seen || n <= 0) return;
    for (int i = 0; i < n; i++) {
        int t = seen[i], first = 1, count = 0;
        if (t < 0 || t >= vocab) continue;
        for (int j = 0; j < i; j++) if (seen[j] == t) { first = 0; break; }
        if (!first) continue;
        for (int j = i; j < n; j++) count += (seen[j] == t);
        float d = f * (float)count;
        logits[t] -= d;
    }
}

typedef struct {
    float *work;                 /* rows x vocab, mutated in place */
    int r0, r1, vocab;
    const int *hist_off, *hist_ids;
    const uint32_t *mask;        /* rows x mask_words or NULL */
    int mask_words;
    uint32_t order;
    float rep, freq, pres;
    sampler_config cfg;
    const uint64_t *seeds;
    int *out_ids;
    pthread_barrier_t *bar;
    sampler *smp;
    struct timespec *t0, *t1;    /* worker 0 only: after the start and end barriers */
} refh_job;

static void *refh_worker(void *arg) {
    refh_job *j = (refh_job *)arg;
    pthread_barrier_wait(j->bar);
    if (j->t0) clock_gettime(CLOCK_MONOTONIC, j->t0);
    for (int r = j->r0; r < j->r1; r++) {
        float *l = j->work + (size_t)r * j->vocab;
        if (j->mask) {
            const uint32_t *m = j->mask + (size_t)r * j->mask_words;
            for (int i = 0; i < j->vocab; i++) if (!((m[i >> 5] >> (i & 31)) & 1u)) l[i] = -INFINITY;
        }
        const int *seen = j->hist_ids ? j->hist_ids + j->hist_off[r] : NULL;
        int n = j->hist_ids ? j->hist_off[r + 1] - j->hist_off[r] : 0;
        for (int s = 0; s < 8; s++) {
            uint32_t op = (j->order >> (4 * s)) & 0xF;
            if (op == 0) break;
            if (op == 1) sampler_apply_repetition_penalty(l, j->vocab, seen, n, j->rep);
            else if (op == 2) refh_frequency(l, j->vocab, seen, n, j->freq);
            else if (op == 3) sampler_apply_presence_penalty(l, j->vocab, seen, n, j->pres);
        }
        j->smp->rng_state = j->seeds[r] ? j->seeds[r] : 0xDEADBEEF12345678ULL;
        j->out_ids[r] = sampler_sample(j->smp, l, j->vocab);
    }
    pthread_barrier_wait(j->bar);
    if (j->t1) clock_gettime(CLOCK_MONOTONIC, j->t1);
    return NULL;
}

/* Times `runs` passes over the batch; out_ms[run] = wall ms of one pass, from
 * the moment every worker has started to the moment the last one is done, read
 * by worker 0 after each of two barriers among the workers only (a timing
 * thread beside them would need a core of its own: on a host with exactly
 * `threads` cores it can be scheduled late and read a start time after work
 * has begun). */
int refh_time_batch(const float *logits, int rows, int vocab, const int *hist_off,
                    const int *hist_ids, const uint32_t *mask, int mask_words, uint32_t order,
                    float rep, float freq, float pres, const sampler_config *cfg,
                    const uint64_t *seeds, int threads, int runs, double *out_ms, int *out_ids) {
    size_t total = (size_t)rows * vocab;
    float *work = malloc(total * sizeof(float));
    refh_job *jobs = calloc((size_t)threads, sizeof(refh_job));
    pthread_t *th = calloc((size_t)threads, sizeof(pthread_t));
    if (!work || !jobs || !th) return -1;
    for (int t = 0; t < threads; t++) jobs[t].smp = sampler_create(cfg);
    pthread_barrier_t bar;
    for (int run = 0; run < runs; run++) {
        memcpy(work, logits, total * sizeof(float));
        pthread_barrier_init(&bar, NULL, (unsigned)threads);
        struct timespec a, b;
        for (int t = 0; t < threads; t++) {
            refh_job *j = &jobs[t];
            j->work = work; j->vocab = vocab;
            j->r0 = (int)((long)rows * t / threads); j->r1 = (int)((long)rows * (t + 1) / threads);
            j->hist_off = hist_off; j->hist_ids = hist_ids; j->mask = mask; j->mask_words = mask_words;
            j->order = order; j->rep = rep; j->freq = freq; j->pres = pres; j->cfg = *cfg;
            j->seeds = seeds; j->out_ids = out_ids; j->bar = &bar;
            j->t0 = t == 0 ? &a : NULL;
            j->t1 = t == 0 ? &b : NULL;
            pthread_create(&th[t], NULL, refh_worker, j);
        }
        for (int t = 0; t < threads; t++) pthread_join(th[t], NULL);
        pthread_barrier_destroy(&bar);
        out_ms[run] = (b.tv_sec - a.tv_sec) * 1e3 + (b.tv_nsec - a.tv_nsec) * 1e-6;
    }
    for (int t = 0; t < threads; t++) sampler_free(jobs[t].smp);
    free(work); free(jobs); free(th);
    return 0;
}

/* expf of the host libm, for the exhaustive libm-agreement checks. */
void refh_expf_many(const float *x, float *y, long n) {
    for (long i = 0; i < n; i++) y[i] = expf(x[i]);
}

/* The decode step's final-logit soft-cap, in place (src/core/context.c:604-606 and
 * :873-876; context.c itself needs the whole model runtime to compile, so its
 * one-line loop is restated here).  Compiled with each build's flags, so the fast
 * build shows what the reference Makefile's -O3 -ffast-math makes of it
 * (x * (1/cap) and gcc's vectorised libmvec tanhf). */
void refh_softcap(float *logits, int n, float cap) {
    for (int i = 0; i < n; i++) logits[i] = cap * tanhf(logits[i] / cap);
}
