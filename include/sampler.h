/*
 * sampler.h -- drop-in for DiskLLM's include/sampler.h (same types, names and
 * signatures; include/sampler.h:7-34 of the reference), implemented by
 * libdiskllm_amd.so on the GPU: sampler_sample copies the caller's host row to
 * the device and runs the batched kernels of diskllm_amd.h on it; the penalty
 * functions send only the logits of the history's ids and write them back.
 * Results are bit-identical to the reference built as strict ISO C.
 *
 * Each sampler owns a HIP stream and device buffers (its own kernel workspace
 * too), so separate samplers may be used from separate threads at once; one
 * sampler, like the reference's, is not thread-safe.  greedy_sample and the two
 * penalty functions take no sampler and share one lazily created per-process
 * context guarded by a mutex.
 */
#ifndef SAMPLER_H
#define SAMPLER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Opaque sampler state (reference: src/sampler.c:61-66). */
typedef struct sampler sampler;

/* Sampling configuration (reference include/sampler.h:10-16). */
typedef struct {
    float temperature;   /* 0 = greedy; otherwise logits are scaled by 1/temperature */
    int top_k;           /* 0 (or >= vocab) = no top-k */
    float top_p;         /* >= 1 = no nucleus cut */
    float min_p;         /* <= 0 = no min-p cut (absolute probability threshold) */
    uint64_t seed;       /* xorshift64 seed; 0 selects 0xDEADBEEF12345678 */
} sampler_config;

/* A sampler with its own rng state; NULL on failure (no GPU, no memory). */
sampler *sampler_create(const sampler_config *cfg);

void sampler_free(sampler *s);

/* In place on the host row: once per occurrence, negative logits multiplied by
 * `penalty`, others divided; nothing unless penalty > 1 (src/sampler.c:21-33).
 * If the device cannot be reached the row is left as it is and stderr says so
 * (the reference's penalties cannot fail; these have no error channel either). */
void sampler_apply_repetition_penalty(float *logits, int vocab_size, const int *seen_tokens, int num_seen,
                                      float penalty);

/* In place on the host row: presence_penalty subtracted once per distinct
 * seen id (src/sampler.c:35-52). */
void sampler_apply_presence_penalty(float *logits, int vocab_size, const int *seen_tokens, int num_seen,
                                    float presence_penalty);

/* One token from the row (src/sampler.c:136-234); advances the rng state once
 * unless temperature == 0.  The row is not modified.  Every configuration of the
 * reference is served (any non-zero temperature, any 0 < top_k < vocab_size,
 * NaN and infinite logits).  Like the reference it always returns a token in
 * [0, vocab_size): a launch whose cross-workgroup wait gave up (another kernel
 * holding the GPU) is run again on the one-workgroup-per-row kernel from the same
 * rng state, and if the device cannot be reached the row is sampled greedily on
 * the host without drawing, as the reference does when it cannot get its work
 * buffer (src/sampler.c:145-147); that case is reported once on stderr.
 * -1 only for a NULL sampler or row, or vocab_size <= 0. */
int sampler_sample(sampler *s, float *logits, int vocab_size);

/* First index of the maximum; 0 when logits[0] is NaN (src/sampler.c:9-19).
 * On the host if the device cannot be reached (reported once on stderr). */
int greedy_sample(const float *logits, int vocab_size);

#ifdef __cplusplus
}
#endif

#endif
