/*
 * oracle.c -- CPU restatement of DiskLLM's token-sampling and grammar-mask path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: only tests/, the smoke
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py load it.  The
 * product (diskllm_amd/) never links, loads or calls anything here.
 *
 * Build (see oracle/Makefile): gcc -std=c11 -O2 -ffp-contract=off, no -march, so
 * every float/double operation is a single IEEE-754 round-to-nearest operation in
 * source order and expf() is the host glibc libm routine -- the same arithmetic the
 * reference's src/sampler.c performs in a strict -std=c11 -O2 build.
 *
 * Every function names the reference lines it restates.  Where the reference has
 * no counterpart (frequency penalty, packed-bitmask apply, the byte-DFA mask), the
 * function says "builder-defined" and states the convention.
 *
 * Pinning (how each part is checked independently of this file):
 *   - orc_rand_f32 / xorshift: closed form + differential vs oracle/_ref build.
 *   - orc_greedy, penalties: closed form per id + differential vs oracle/_ref.
 *   - orc_sample: differential vs the reference src/sampler.c compiled from its own
 *     sources into oracle/_ref (tests/test_oracle.py), plus invariants.
 *   - grammar validators: the reference KATs (tools/test_grammar_unit.c:17-24)
 *     and differential vs the reference grammar.c compiled into oracle/_ref.
 *   - DFA mask: no reference counterpart; pinned by an independent numpy walk
 *     (tests/test_oracle.py) and hand-built tiny DFAs.
 */
#define _POSIX_C_SOURCE 200809L
#include <math.h>
#include <stdbool.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <pthread.h>

#include "oracle.h"

/* ---- RNG: src/sampler.c:69-81, seeding src/sampler.c:87 ---------------------- */

uint64_t orc_seed_state(uint64_t seed) { return seed ? seed : 0xDEADBEEF12345678ULL; }

uint64_t orc_xorshift64(uint64_t *state) {
    uint64_t x = *state;
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    *state = x;
    return x;
}

float orc_rand_f32(uint64_t *state) {
    /* u64 -> float conversion rounds to nearest even; 2^-53 scaling is exact. */
    return (float)(orc_xorshift64(state) >> 11) * (1.0f / (float)(1ULL << 53));
}

/* ---- greedy: src/sampler.c:9-19 ---------------------------------------------- */

int orc_greedy(const float *logits, int vocab) {
    int best = 0;
    float bv = logits[0];
    for (int i = 1; i < vocab; i++)
        if (logits[i] > bv) { bv = logits[i]; best = i; }
    return best;
}

/* ---- penalties ---------------------------------------------------------------- */

/* src/sampler.c:21-33: once per occurrence, l<0 ? l*=p : l/=p. */
void orc_repetition(float *logits, int vocab, const int *seen, int n, float penalty) {
    if (penalty <= 1.0f || !seen || n <= 0) return;
    for (int i = 0; i < n; i++) {
        int t = seen[i];
        if (t < 0 || t >= vocab) continue;
        if (logits[t] < 0.0f) logits[t] *= penalty;
        else logits[t] /= penalty;
    }
}

/* src/sampler.c:35-52: once per distinct id, l -= pp (first-occurrence test). */
void orc_presence(float *logits, int vocab, const int *seen, int n, float pp) {
    if (pp == 0.0f || !seen || n <= 0) return;
    for (int i = 0; i < n; i++) {
        int t = seen[i];
        if (t < 0 || t >= vocab) continue;
        int first = 1;
        for (int j = 0; j < i; j++)
            if (seen[j] == t) { first = 0; break; }
        if (first) logits[t] -= pp;
    }
}

/* Builder-defined (absent from the reference): once per distinct id,
 * l -= f * (float)count, the product rounded to float before the subtraction. */
void orc_frequency(float *logits, int vocab, const int *seen, int n, float f) {
    if (f == 0.0f || !seen || n <= 0) return;
    for (int i = 0; i < n; i++) {
        int t = seen[i];
        if (t < 0 || t >= vocab) continue;
        int first = 1, count = 0;
        for (int j = 0; j < i; j++)
            if (seen[j] == t) { first = 0; break; }
        if (!first) continue;
        for (int j = i; j < n; j++) count += (seen[j] == t);
        float d = f * (float)count;
        logits[t] -= d;
    }
}

/* Apply the penalties in the order packed into `order` (ORC_OP_* nibbles, lowest
 * nibble first, a zero nibble ends the list).  The reference caller order is
 * presence then repetition (src/core/sampler_api.c:55-61). */
void orc_penalties(float *logits, int vocab, const int *seen, int n, uint32_t order,
                   float repeat, float frequency, float presence) {
    for (int s = 0; s < 8; s++) {
        uint32_t op = (order >> (4 * s)) & 0xF;
        if (op == 0) break;
        if (op == ORC_OP_REPETITION) orc_repetition(logits, vocab, seen, n, repeat);
        else if (op == ORC_OP_FREQUENCY) orc_frequency(logits, vocab, seen, n, frequency);
        else if (op == ORC_OP_PRESENCE) orc_presence(logits, vocab, seen, n, presence);
    }
}

/* Builder-defined packed allow-mask (bit i%32 of word i/32, 1 = allowed); masked
 * entries become -INFINITY, the write the reference grammar mask performs
 * (src/core/grammar.c:285-305). Returns the allowed count. */
int orc_apply_packed_mask(float *logits, int vocab, const uint32_t *mask) {
    int valid = 0;
    for (int i = 0; i < vocab; i++) {
        if ((mask[i >> 5] >> (i & 31)) & 1u) valid++;
        else logits[i] = -INFINITY;
    }
    return valid;
}

/* ---- sampler_sample: src/sampler.c:136-234 ------------------------------------ */

/* src/sampler.c:109-134, partial insertion sort of the first k by value desc.
 * Restated step for step because its NaN behaviour (all-masked rows) is part of
 * the observable result. */
static void select_top_k(int *idx, float *val, int n, int k) {
    for (int i = 1; i < n && i < k; i++) {
        int j = i, ti = idx[i];
        float tv = val[i];
        while (j > 0 && val[j - 1] < tv) { idx[j] = idx[j - 1]; val[j] = val[j - 1]; j--; }
        idx[j] = ti; val[j] = tv;
    }
    for (int i = k; i < n; i++) {
        if (val[i] > val[k - 1]) {
            int j = k - 1, ti = idx[i];
            float tv = val[i];
            while (j > 0 && val[j - 1] < tv) { idx[j] = idx[j - 1]; val[j] = val[j - 1]; j--; }
            idx[j] = ti; val[j] = tv;
        }
    }
}

int orc_sample(const orc_cfg *cfg, uint64_t *rng, const float *logits, int vocab,
               orc_trace *tr) {
    /* tr->idx / tr->val: caller arrays of length >= vocab (the work buffer). */
    int *idx = tr->idx;
    float *val = tr->val;
    tr->greedy = 0;
    tr->k = 0; tr->k_minp = 0; tr->nk = 0; tr->r = 0.0f;
    tr->sum = tr->s2 = tr->s3 = 0.0;
    tr->inv_sum = tr->inv_s2 = tr->inv_s3 = 0.0f;

    float temp = cfg->temperature;
    if (temp == 0.0f) {                                    /* :140-142 */
        tr->greedy = 1;
        return orc_greedy(logits, vocab);
    }
    for (int i = 0; i < vocab; i++) { idx[i] = i; val[i] = logits[i]; }   /* :148-151 */
    float inv_temp = 1.0f / temp;                          /* :154 */
    float mx = val[0];                                     /* :155-158 */
    for (int i = 1; i < vocab; i++) if (val[i] > mx) mx = val[i];
    for (int i = 0; i < vocab; i++) val[i] = (val[i] - mx) * inv_temp;   /* :160-162 */

    int k = vocab;                                         /* :165-170 */
    if (cfg->top_k > 0 && cfg->top_k < vocab) { k = cfg->top_k; select_top_k(idx, val, vocab, k); }
    tr->k = k;

    float mv = val[0];                                     /* :173-176 */
    for (int i = 1; i < k; i++) if (val[i] > mv) mv = val[i];
    double sum = 0.0;                                      /* :177-181 */
    for (int i = 0; i < k; i++) { val[i] = expf(val[i] - mv); sum += val[i]; }
    float inv_sum = (float)(1.0 / sum);                    /* :182-185 */
    for (int i = 0; i < k; i++) val[i] *= inv_sum;
    tr->sum = sum; tr->inv_sum = inv_sum;
    if (tr->p) for (int i = 0; i < k; i++) tr->p[i] = val[i];

    if (cfg->min_p > 0.0f) {                               /* :188-202 */
        float min_prob = cfg->min_p;
        int nk = 0;
        for (int i = 0; i < k; i++)
            if (val[i] >= min_prob) { idx[nk] = idx[i]; val[nk] = val[i]; nk++; }
        if (nk > 0) k = nk;
        double s2 = 0.0;
        for (int i = 0; i < k; i++) s2 += val[i];
        float inv_s2 = (float)(1.0 / s2);
        for (int i = 0; i < k; i++) val[i] *= inv_s2;
        tr->s2 = s2; tr->inv_s2 = inv_s2;
    }
    tr->k_minp = k;

    if (cfg->top_p < 1.0f) {                               /* :205-222 */
        double cumul = 0.0;
        int nk = k;
        for (int i = 0; i < k; i++) {
            cumul += val[i];
            if ((float)cumul >= cfg->top_p) { nk = i + 1; break; }
        }
        k = nk;
        double s3 = 0.0;
        for (int i = 0; i < k; i++) s3 += val[i];
        float inv_s3 = (float)(1.0 / s3);
        for (int i = 0; i < k; i++) val[i] *= inv_s3;
        tr->s3 = s3; tr->inv_s3 = inv_s3;
    }
    tr->nk = k;

    float r = orc_rand_f32(rng);                           /* :225-233 */
    tr->r = r;
    float cumul = 0.0f;
    for (int i = 0; i < k; i++) {
        cumul += val[i];
        if (r < cumul) { tr->pos = i; return idx[i]; }
    }
    tr->pos = k - 1;
    return idx[k - 1];
}

/* ---- byte-DFA mask (builder-defined; no reference counterpart) --------------- */

/* Token t (bytes[off[t]..off[t+1])) is allowed from `state` iff the state is not
 * the dead state 0, the token is non-empty, and walking its bytes through
 * trans[state*256 + byte] never reaches state 0.  Optional EOS rule: the eos id is
 * allowed iff bit `state` of accept_mask is set (mirrors the EOS/is_finished rule
 * of src/core/grammar.c:285-292). Writes the packed allow-mask; returns count. */
int orc_dfa_mask(const uint32_t *off, const uint8_t *bytes, int vocab, const uint8_t *trans,
                 int state, int eos_id, uint64_t accept_mask, uint32_t *out_mask) {
    int words = (vocab + 31) / 32, valid = 0;
    memset(out_mask, 0, (size_t)words * 4);
    for (int t = 0; t < vocab; t++) {
        int ok;
        if (t == eos_id) {
            ok = state > 0 && state < 64 && ((accept_mask >> state) & 1u);
        } else {
            uint32_t b = off[t], e = off[t + 1];
            ok = (state != 0) && (e > b);
            int s = state;
            for (uint32_t j = b; ok && j < e; j++) {
                s = trans[s * 256 + bytes[j]];
                if (s == 0) ok = 0;
            }
        }
        if (ok) { out_mask[t >> 5] |= 1u << (t & 31); valid++; }
    }
    return valid;
}

/* ---- grammar validators: src/core/grammar.c ------------------------------------ */

static int is_ws(unsigned char c) { return c == ' ' || c == '\t' || c == '\n' || c == '\v' || c == '\f' || c == '\r'; }
static int is_dig(unsigned char c) { return c >= '0' && c <= '9'; }

/* src/core/grammar.c:68-194, restated as the same left-to-right scan. */
bool orc_receipt_prefix(const char *s, int len) {
    int i = 0;
    while (i < len && is_ws((unsigned char)s[i])) i++;
    if (i >= len) return true;
    if (s[i] != '{') return false;
    i++;
    static const char key1[] = "\"bbox_2d\":";
    int k1 = (int)sizeof(key1) - 1;
    while (i < len && is_ws((unsigned char)s[i])) i++;
    if (i >= len) return true;
    for (int m = 0; i < len && m < k1; m++, i++) {
        if (s[i] != key1[m] && !(key1[m] == ':' && is_ws((unsigned char)s[i]))) return false;
    }
    if (i >= len) return true;
    while (i < len && is_ws((unsigned char)s[i])) i++;
    if (i >= len) return true;
    if (s[i] != '[') return false;
    i++;
    for (int num = 0; num < 4; num++) {
        while (i < len && is_ws((unsigned char)s[i])) i++;
        if (i >= len) return true;
        bool dig = false;
        while (i < len && is_dig((unsigned char)s[i])) { dig = true; i++; }
        if (i >= len) return true;
        if (!dig && s[i] != ']' && s[i] != ',') return false;
        while (i < len && is_ws((unsigned char)s[i])) i++;
        if (i >= len) return true;
        char want = num < 3 ? ',' : ']';
        if (s[i] == want) i++;
        else if (!is_dig((unsigned char)s[i])) return false;
    }
    if (i >= len) return true;
    while (i < len && is_ws((unsigned char)s[i])) i++;
    if (i >= len) return true;
    if (s[i] != ',') return false;
    i++;
    while (i < len && is_ws((unsigned char)s[i])) i++;
    if (i >= len) return true;
    static const char key2[] = "\"text_content\":";
    int k2 = (int)sizeof(key2) - 1;
    for (int m = 0; i < len && m < k2; m++, i++)
        if (s[i] != key2[m]) return false;
    if (i >= len) return true;
    while (i < len && is_ws((unsigned char)s[i])) i++;
    if (i >= len) return true;
    if (s[i] != '"') return false;
    i++;
    bool closed = false;
    while (i < len) {
        if (s[i] == '"' && (i == 0 || s[i - 1] != '\\')) { closed = true; i++; break; }
        i++;
    }
    if (i >= len) return true;
    if (closed) {
        while (i < len && is_ws((unsigned char)s[i])) i++;
        if (i >= len) return true;
        if (s[i] != '}') return false;
        i++;
        while (i < len && is_ws((unsigned char)s[i])) i++;
        return i >= len;
    }
    return true;
}

/* src/core/grammar.c:197-226. */
bool orc_json_prefix(const char *s, int len) {
    if (len == 0) return true;
    int i = 0;
    while (i < len && is_ws((unsigned char)s[i])) i++;
    if (i >= len) return true;
    if (s[i] != '{' && s[i] != '[') return false;
    int braces = 0, brackets = 0;
    bool in_str = false;
    for (; i < len; i++) {
        char c = s[i];
        if (c == '"' && (i == 0 || s[i - 1] != '\\')) in_str = !in_str;
        else if (!in_str) {
            if (c == '{') braces++;
            else if (c == '}') { if (--braces < 0) return false; }
            else if (c == '[') brackets++;
            else if (c == ']') { if (--brackets < 0) return false; }
        }
    }
    return true;
}

/* Grammar mode and buffer, src/core/grammar.c:8-14, :16-28 (mode by substring). */
void orc_grammar_init(orc_grammar *g, const char *text) {
    memset(g, 0, sizeof(*g));
    if (!text) return;
    g->is_receipt = strstr(text, "bbox_2d") != NULL;
    g->is_json = strstr(text, "object") != NULL || strstr(text, "value") != NULL;
}

/* src/core/grammar.c:228-246. */
bool orc_grammar_accept(const orc_grammar *g, const char *piece) {
    if (!g || !piece) return true;
    int cur = g->len, plen = (int)strlen(piece);
    if (cur + plen >= ORC_GRAMMAR_BUF - 1) return false;
    char tmp[ORC_GRAMMAR_BUF];
    memcpy(tmp, g->buf, (size_t)cur);
    memcpy(tmp + cur, piece, (size_t)plen);
    tmp[cur + plen] = 0;
    if (g->is_receipt) return orc_receipt_prefix(tmp, cur + plen);
    if (g->is_json) return orc_json_prefix(tmp, cur + plen);
    return true;
}

/* src/core/grammar.c:248-256 (a piece that does not fit is dropped silently). */
void orc_grammar_advance(orc_grammar *g, const char *piece) {
    if (!g || !piece) return;
    int plen = (int)strlen(piece);
    if (g->len + plen < ORC_GRAMMAR_BUF - 1) {
        memcpy(g->buf + g->len, piece, (size_t)plen);
        g->len += plen;
        g->buf[g->len] = 0;
    }
}

/* src/core/grammar.c:258-273. */
bool orc_grammar_finished(const orc_grammar *g) {
    if (!g || g->len == 0) return false;
    int braces = 0, brackets = 0;
    bool in_str = false;
    for (int i = 0; i < g->len; i++) {
        char c = g->buf[i];
        if (c == '"' && (i == 0 || g->buf[i - 1] != '\\')) in_str = !in_str;
        if (!in_str) {
            if (c == '{') braces++;
            else if (c == '}') braces--;
            else if (c == '[') brackets++;
            else if (c == ']') brackets--;
        }
    }
    return braces == 0 && brackets == 0 && !in_str && g->len > 1;
}

/* src/core/grammar.c:275-308 over a CSR table of token strings (off[t]..off[t+1]).
 * A zero-length entry stands for a NULL string; a piece is read up to its first
 * NUL byte, as the reference's strlen() would. */
int orc_grammar_mask(const orc_grammar *g, float *logits, int vocab, const uint32_t *off,
                     const uint8_t *bytes, int eos_id) {
    int valid = 0;
    bool fin = orc_grammar_finished(g);
    char piece[ORC_GRAMMAR_BUF + 1];
    for (int i = 0; i < vocab; i++) {
        if (i == eos_id) {
            if (!fin) logits[i] = -INFINITY;
            else valid++;
            continue;
        }
        uint32_t b = off[i], e = off[i + 1];
        if (e == b || bytes[b] == 0) { logits[i] = -INFINITY; continue; }   /* :294-298 */
        uint32_t n = e - b;
        if (n > ORC_GRAMMAR_BUF) n = ORC_GRAMMAR_BUF;
        memcpy(piece, bytes + b, n);
        piece[n] = 0;
        if (!orc_grammar_accept(g, piece)) logits[i] = -INFINITY;
        else valid++;
    }
    return valid;
}

/* ---- host libm expf over a range of bit patterns (for the device expf check) -- */

typedef struct { uint32_t first; long n; float *out; } orc_expf_job;

static void *orc_expf_worker(void *arg) {
    orc_expf_job *j = (orc_expf_job *)arg;
    for (long i = 0; i < j->n; i++) {
        uint32_t u = j->first + (uint32_t)i;
        float x;
        memcpy(&x, &u, 4);
        j->out[i] = expf(x);
    }
    return NULL;
}

/* out[i] = expf(bits(first + i)) with the host libm, over `threads` threads. */
void orc_expf_bits(uint32_t first, long n, float *out, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t th[64];
    orc_expf_job jobs[64];
    long per = (n + threads - 1) / threads;
    for (int t = 0; t < threads; t++) {
        long a = t * per, b = a + per < n ? a + per : n;
        jobs[t].first = first + (uint32_t)(a > n ? n : a);
        jobs[t].n = b > a ? b - a : 0;
        jobs[t].out = out + (a > n ? n : a);
        pthread_create(&th[t], NULL, orc_expf_worker, &jobs[t]);
    }
    for (int t = 0; t < threads; t++) pthread_join(th[t], NULL);
}

/* The reference's logit soft-cap (src/core/context.c:604-606 and :873-876):
 * y[i] = cap * tanhf(x[i] / cap) with the host libm, applied only when cap > 0;
 * y may equal x. */
void orc_softcap(const float *x, float *y, long n, float cap) {
    if (!(cap > 0.0f)) {
        if (y != x) memmove(y, x, (size_t)n * sizeof(float));
        return;
    }
    for (long i = 0; i < n; i++) y[i] = cap * tanhf(x[i] / cap);
}

typedef struct { uint32_t first; long n; float *out; } orc_tanhf_job;

static void *orc_tanhf_worker(void *arg) {
    orc_tanhf_job *j = (orc_tanhf_job *)arg;
    for (long i = 0; i < j->n; i++) {
        uint32_t u = j->first + (uint32_t)i;
        float x;
        memcpy(&x, &u, 4);
        j->out[i] = tanhf(x);
    }
    return NULL;
}

/* out[i] = tanhf(bits(first + i)) with the host libm, over `threads` threads. */
void orc_tanhf_bits(uint32_t first, long n, float *out, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t th[64];
    orc_tanhf_job jobs[64];
    long per = (n + threads - 1) / threads;
    for (int t = 0; t < threads; t++) {
        long a = t * per, b = a + per < n ? a + per : n;
        jobs[t].first = first + (uint32_t)(a > n ? n : a);
        jobs[t].n = b > a ? b - a : 0;
        jobs[t].out = out + (a > n ? n : a);
        pthread_create(&th[t], NULL, orc_tanhf_worker, &jobs[t]);
    }
    for (int t = 0; t < threads; t++) pthread_join(th[t], NULL);
}
