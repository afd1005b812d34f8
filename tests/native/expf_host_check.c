/* Exhaustive agreement check: dlk_expf_glibc (the GPU's restatement, compiled for
 * the host) against the host libm expf over every non-NaN float bit pattern in
 * [lo, hi) with the given stride.  With a fifth argument "core" it checks the
 * unscreened dlk_expf_glibc_core on max(x, -200) instead, for the inputs x <= 0
 * (and -inf) the fused kernel feeds it.  Prints "<checked> <mismatches>" and the
 * first few mismatching inputs.  Test infrastructure. */
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "../../diskllm_amd/csrc/hip/expf_glibc.h"

static const uint64_t TAB[32] = DLK_EXP2_TAB_INIT;
static uint64_t lo_, hi_, stride_;
static int nth_, core_;
static unsigned long long checked_[64], bad_[64];

static void *work(void *arg) {
    long t = (long)arg;
    for (uint64_t u = lo_ + (uint64_t)t * stride_; u < hi_; u += (uint64_t)nth_ * stride_) {
        float x = dlk_u2f((uint32_t)u);
        if (isnan(x)) continue;
        if (core_ && !(x <= 0.0f)) continue;
        checked_[t]++;
        float a = expf(x), b = core_ ? dlk_expf_glibc_core(fmaxf(x, -200.0f), TAB) : dlk_expf_glibc(x, TAB);
        if (dlk_f2u(a) != dlk_f2u(b)) {
            if (bad_[t] < 4) fprintf(stderr, "mismatch x=%a libm=%08x mine=%08x\n", x, dlk_f2u(a), dlk_f2u(b));
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
    core_ = argc > 5 && strcmp(argv[5], "core") == 0;
    if (nth_ < 1) nth_ = 1;
    if (nth_ > 64) nth_ = 64;
    pthread_t th[64];
    for (long t = 0; t < nth_; t++) pthread_create(&th[t], NULL, work, (void *)t);
    unsigned long long c = 0, b = 0;
    for (int t = 0; t < nth_; t++) { pthread_join(th[t], NULL); c += checked_[t]; b += bad_[t]; }
    printf("%llu %llu\n", c, b);
    return b != 0;
}
