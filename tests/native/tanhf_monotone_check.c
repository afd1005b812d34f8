/* Monotonicity check of the soft-cap: dlk_tanhf_glibc (bit-identical to the host
 * libm tanhf, which tanhf_host_check.c checks exhaustively) is non-decreasing
 * over every pair of consecutive non-NaN floats from -inf to +inf, visited in
 * numeric order.  Then x -> cap * tanhf(x / cap) is non-decreasing for every
 * cap > 0, since x / cap and cap * y are correctly rounded and so non-decreasing
 * in x and y.  With a fourth argument "cap=<c>" the composite itself is checked
 * the same way.  Arguments: stride (1 = every float), threads.  Prints
 * "<pairs checked> <decreases>" and the first few decreases.  Test
 * infrastructure: the sampling kernels select top-k candidates on raw logits
 * under a soft-cap only because this holds. */
#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include "../../diskllm_amd/csrc/hip/tanhf_glibc.h"

/* ascending order key of a non-NaN float and its inverse */
static uint32_t from_key(uint32_t k) { return (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k; }

static const uint32_t kFirst = 0x007fffffu;   /* key of -inf */
static const uint32_t kLast = 0xff800000u;    /* key of +inf */
static uint64_t stride_;
static int nth_, use_cap_;
static float cap_;
static unsigned long long checked_[64], bad_[64];

static float f(float x) { return use_cap_ ? dlk_softcap_glibc(x, cap_) : dlk_tanhf_glibc(x); }

static void *work(void *arg) {
    long t = (long)arg;
    const uint64_t span = (uint64_t)kLast - kFirst;
    for (uint64_t o = (uint64_t)t * stride_; o < span; o += (uint64_t)nth_ * stride_) {
        const uint32_t k = (uint32_t)(kFirst + o);
        const float a = dlk_th_u2f(from_key(k)), b = dlk_th_u2f(from_key(k + 1));
        checked_[t]++;
        if (f(b) < f(a)) {
            if (bad_[t] < 4) fprintf(stderr, "decrease: f(%a) = %a > f(%a) = %a\n", a, f(a), b, f(b));
            bad_[t]++;
        }
    }
    return NULL;
}

int main(int argc, char **argv) {
    stride_ = argc > 1 ? strtoull(argv[1], 0, 0) : 1;
    nth_ = argc > 2 ? atoi(argv[2]) : 8;
    if (argc > 3 && strncmp(argv[3], "cap=", 4) == 0) {
        use_cap_ = 1;
        cap_ = strtof(argv[3] + 4, NULL);
    }
    if (stride_ < 1) stride_ = 1;
    if (nth_ < 1) nth_ = 1;
    if (nth_ > 64) nth_ = 64;
    pthread_t th[64];
    for (long t = 0; t < nth_; t++) pthread_create(&th[t], NULL, work, (void *)t);
    unsigned long long c = 0, b = 0;
    for (int t = 0; t < nth_; t++) { pthread_join(th[t], NULL); c += checked_[t]; b += bad_[t]; }
    printf("%llu %llu\n", c, b);
    return b != 0;
}
