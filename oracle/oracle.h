/* oracle.h -- CPU restatement of DiskLLM's sampling + grammar-mask path.
 * TEST INFRASTRUCTURE ONLY (see oracle.c). */
#ifndef DISKLLM_ORACLE_H
#define DISKLLM_ORACLE_H
#include <stdbool.h>
#include <stdint.h>

#define ORC_OP_REPETITION 1u
#define ORC_OP_FREQUENCY 2u
#define ORC_OP_PRESENCE 3u
#define ORC_GRAMMAR_BUF 8192

typedef struct {
    float temperature;
    int top_k;
    float top_p;
    float min_p;
} orc_cfg;

typedef struct {
    int *idx;      /* work buffer indices, length >= vocab */
    float *val;    /* work buffer values,  length >= vocab */
    float *p;      /* optional: softmax probabilities of the k candidates (A9) */
    int greedy, k, k_minp, nk, pos;
    float r, inv_sum, inv_s2, inv_s3;
    double sum, s2, s3;
} orc_trace;

typedef struct {
    char buf[ORC_GRAMMAR_BUF];
    int len;
    bool is_json, is_receipt;
} orc_grammar;

uint64_t orc_seed_state(uint64_t seed);
uint64_t orc_xorshift64(uint64_t *state);
float orc_rand_f32(uint64_t *state);
int orc_greedy(const float *logits, int vocab);
void orc_repetition(float *logits, int vocab, const int *seen, int n, float penalty);
void orc_presence(float *logits, int vocab, const int *seen, int n, float pp);
void orc_frequency(float *logits, int vocab, const int *seen, int n, float f);
void orc_penalties(float *logits, int vocab, const int *seen, int n, uint32_t order,
                   float repeat, float frequency, float presence);
int orc_apply_packed_mask(float *logits, int vocab, const uint32_t *mask);
int orc_sample(const orc_cfg *cfg, uint64_t *rng, const float *logits, int vocab, orc_trace *tr);
int orc_dfa_mask(const uint32_t *off, const uint8_t *bytes, int vocab, const uint8_t *trans,
                 int state, int eos_id, uint64_t accept_mask, uint32_t *out_mask);
bool orc_receipt_prefix(const char *s, int len);
bool orc_json_prefix(const char *s, int len);
void orc_grammar_init(orc_grammar *g, const char *text);
bool orc_grammar_accept(const orc_grammar *g, const char *piece);
void orc_grammar_advance(orc_grammar *g, const char *piece);
bool orc_grammar_finished(const orc_grammar *g);
int orc_grammar_mask(const orc_grammar *g, float *logits, int vocab, const uint32_t *off,
                     const uint8_t *bytes, int eos_id);
void orc_expf_bits(uint32_t first, long n, float *out, int threads);
void orc_softcap(const float *x, float *y, long n, float cap);
void orc_tanhf_bits(uint32_t first, long n, float *out, int threads);
#endif
