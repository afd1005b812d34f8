/* Exhaustive agreement check: dlk_tanhf_glibc (the GPU's restatement, compiled
 * for the host) against the host libm tanhf over every non-NaN float bit pattern
 * in [lo, hi) with the given stride.  With a fifth argument "cap=<c>" it checks
 * dlk_softcap_glibc(x, c) against c * tanhf(x / c) instead (the reference's
 * soft-cap, src/core/context.c:604-606).  Prints "<checked> <mismatches>" and the
 * first few mismatching inputs.  Test infrastructure. */
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "../../diskllm_amd/csrc/hip/tanhf_glibc.h"

static uint64_t lo_, hi_, stride_;
static int nth_, use_cap_;
static float cap_;
static unsigned long long checked_[64], bad_[64];

static void *work(void *arg) {
    long t = (long)arg;
    for (uint64_t u = lo_ + (uint64_t)t * stride_; u < hi_; u += (uint64_t)nth_ * stride_) {
        float x = dlk_th_u2f((uint32_t)u);
        if (isnan(x)) continue;
        checked_[t]++;
        float a = use_cap_ ? cap_ * tanhf(x / cap_) : tanhf(x);
        float b = use_cap_ ? dlk_softcap_glibc(x, cap_) : dlk_tanhf_glibc(x);
        if (dlk_th_f2u(a) != dlk_th_f2u(b)) {
            if (bad_[t] < 4) fprintf(stderr, "mismatch x=%a libm=%08x mine=%08x\n", x, dlk_th_f2u(a), dlk_th_f2u(b));
            bad_[t]++;
        }
    }
    return NULL;
}

int main(int argc, char **argv) {
    lo_ = argc > 1 ? strtoull(argv[1], 0, 0) : 0;
    hi_ = argc > 2 ? strtoull(argv[2], 0, 0) : (1ull << 32);
    stride_ = argc > 3 ? strtoull(argv[3], 0, 0) : 1;
    nth_ = argc > 4 ? atoi(argv[4]) : 8;
    if (argc > 5 && strncmp(argv[5], "cap=", 4) == 0) {
        use_cap_ = 1;
        cap_ = strtof(argv[5] + 4, NULL);
    }
    if (nth_ < 1) nth_ = 1;
    if (nth_ > 64) nth_ = 64;
    pthread_t th[64];
    for (long t = 0; t < nth_; t++) pthread_create(&th[t], NULL, work, (void *)t);
    unsigned long long c = 0, b = 0;
    for (int t = 0; t < nth_; t++) { pthread_join(th[t], NULL); c += checked_[t]; b += bad_[t]; }
    printf("%llu %llu\n", c, b);
    return b != 0;
}
