/*
 * dropin_grammar.c -- include/grammar.h on the GPU.  The grammar object keeps the
 * reference's text buffer (src/core/grammar.c:8-14) and the validator state
 * after it; apply_mask rebuilds the token-string table through the caller's
 * callback (as the reference reads it on every call), uploads it only when it
 * changed, and masks every token on the device from the buffer's state; only the
 * packed mask comes back (one bit per token), and the disallowed logits are set
 * to -inf from it in place.
 */
#define _POSIX_C_SOURCE 200809L
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "diskllm_amd.h"
#include "grammar.h"
#include "dropin.h"
#include "../hip/grammar_scan.h"

struct diskllm_grammar {
    char buffer[DLK_GRAMMAR_BUF];
    int buf_len;
    int mode;
    dlk_grammar_row row;         /* validator + balance state after buffer[0..buf_len) */
    /* token table of the last apply_mask: host copy and its device upload */
    uint32_t *off;
    uint8_t *bytes;
    int tab_vocab;
    size_t tab_bytes, bytes_cap;
    uint32_t *d_off;
    uint8_t *d_bytes;
    size_t d_bytes_cap;
    int d_vocab_cap;
    dlk_grammar_row *d_row;
    uint32_t *hmask;             /* host copy of the last mask */
    int hmask_cap;
    dlk_dropin_ctx dev;
    int dev_ready;
};

diskllm_grammar *diskllm_grammar_init_from_str(const char *grammar_str) {
    if (!grammar_str) return NULL;
    diskllm_grammar *g = calloc(1, sizeof(*g));
    if (!g) return NULL;
    g->mode = dlk_grammar_mode_of(grammar_str);
    dlk_grammar_row_init(&g->row, g->mode);
    return g;
}

diskllm_grammar *diskllm_grammar_init_from_file(const char *filepath) {
    if (!filepath) return NULL;
    FILE *f = fopen(filepath, "rb");
    if (!f) return NULL;
    if (fseek(f, 0, SEEK_END) != 0) { fclose(f); return NULL; }
    const long sz = ftell(f);
    if (sz < 0 || fseek(f, 0, SEEK_SET) != 0) { fclose(f); return NULL; }
    char *text = malloc((size_t)sz + 1);
    if (!text) { fclose(f); return NULL; }
    const size_t got = fread(text, 1, (size_t)sz, f);
    text[got] = '\0';
    fclose(f);
    diskllm_grammar *g = diskllm_grammar_init_from_str(text);
    free(text);
    return g;
}

diskllm_grammar *diskllm_grammar_init_json(void) {
    diskllm_grammar *g = diskllm_grammar_init_from_str("root ::= object | array\n");
    if (g && g->mode == DLK_GRAMMAR_NONE) {
        g->mode = DLK_GRAMMAR_JSON;
        dlk_grammar_row_init(&g->row, g->mode);
    }
    return g;
}

void diskllm_grammar_free(diskllm_grammar *g) {
    if (!g) return;
    if (g->dev_ready) {
        hipStreamSynchronize(g->dev.stream);
        hipFree(g->d_off);
        hipFree(g->d_bytes);
        hipFree(g->d_row);
        dlk_dropin_release(&g->dev);
    }
    free(g->off);
    free(g->bytes);
    free(g->hmask);
    free(g);
}

void diskllm_grammar_reset(diskllm_grammar *g) {
    if (!g) return;
    g->buf_len = 0;
    g->buffer[0] = '\0';
    dlk_grammar_row_init(&g->row, g->mode);
}

bool diskllm_grammar_accept_str(const diskllm_grammar *g, const char *piece) {
    if (!g || !piece) return true;
    const size_t plen = strlen(piece);
    if ((size_t)g->buf_len + plen >= DLK_GRAMMAR_BUF - 1) return false;        /* src/core/grammar.c:233 */
    dlk_scan_state s = g->row.scan;
    for (size_t i = 0; i < plen && dlk_scan_ok(&s); i++) dlk_scan_step(&s, (uint8_t)piece[i]);
    return dlk_scan_ok(&s) != 0;
}

void diskllm_grammar_advance(diskllm_grammar *g, const char *piece) {
    if (!g || !piece) return;
    const size_t plen = strlen(piece);
    if ((size_t)g->buf_len + plen < DLK_GRAMMAR_BUF - 1) {                     /* src/core/grammar.c:251 */
        memcpy(g->buffer + g->buf_len, piece, plen);
        g->buf_len += (int)plen;
        g->buffer[g->buf_len] = '\0';
        dlk_grammar_row_feed(&g->row, piece, (int)plen);
    }
}

bool diskllm_grammar_is_finished(const diskllm_grammar *g) {
    if (!g || g->buf_len == 0) return false;
    return dlk_balance_finished(&g->row.bal) != 0;
}

/* The token table through the callback; returns 1 if it differs from the last. */
static int read_table(diskllm_grammar *g, int vocab, void *ctx, const char *(*get)(void *, int)) {
    uint32_t *off = malloc(((size_t)vocab + 1) * sizeof(uint32_t));
    if (!off) return -1;
    size_t cap = g->bytes_cap ? g->bytes_cap : (size_t)vocab * 8 + 64;
    uint8_t *bytes = malloc(cap);
    if (!bytes) { free(off); return -1; }
    size_t n = 0;
    for (int t = 0; t < vocab; t++) {
        off[t] = (uint32_t)n;
        const char *s = get(ctx, t);
        if (!s) continue;                        /* NULL: an empty entry (masked, :295) */
        const size_t len = strlen(s);
        if (n + len > cap) {
            while (n + len > cap) cap *= 2;
            uint8_t *nb = realloc(bytes, cap);
            if (!nb) { free(off); free(bytes); return -1; }
            bytes = nb;
        }
        memcpy(bytes + n, s, len);
        n += len;
    }
    off[vocab] = (uint32_t)n;
    const int same = g->off && g->tab_vocab == vocab && g->tab_bytes == n &&
                     memcmp(g->off, off, ((size_t)vocab + 1) * sizeof(uint32_t)) == 0 &&
                     memcmp(g->bytes, bytes, n) == 0;
    free(g->off);
    free(g->bytes);
    g->off = off;
    g->bytes = bytes;
    g->bytes_cap = cap;
    g->tab_vocab = vocab;
    g->tab_bytes = n;
    return !same;
}

int diskllm_grammar_apply_mask(diskllm_grammar *g, float *logits, int vocab_size, void *tok_ctx,
                               const char *(*get_token_str)(void *ctx, int token_id), int eos_token_id) {
    if (!g || !logits || vocab_size <= 0 || !get_token_str) return vocab_size;    /* src/core/grammar.c:279 */
    if (!g->dev_ready) {
        if (dlk_dropin_init(&g->dev) != 0) return -1;
        if (hipMalloc((void **)&g->d_row, sizeof(dlk_grammar_row)) != hipSuccess) return -1;
        g->dev_ready = 1;
    }
    const int changed = read_table(g, vocab_size, tok_ctx, get_token_str);
    if (changed < 0 || dlk_dropin_reserve(&g->dev, vocab_size, 0) != 0) return -1;
    hipStream_t st = g->dev.stream;
    if (changed) {
        hipStreamSynchronize(st);
        if (vocab_size + 1 > g->d_vocab_cap) {
            hipFree(g->d_off);
            g->d_off = NULL;
            g->d_vocab_cap = 0;
            if (hipMalloc((void **)&g->d_off, ((size_t)vocab_size + 1) * sizeof(uint32_t)) != hipSuccess) return -1;
            g->d_vocab_cap = vocab_size + 1;
        }
        const size_t nb = g->tab_bytes ? g->tab_bytes : 1;
        if (nb > g->d_bytes_cap) {
            hipFree(g->d_bytes);
            g->d_bytes = NULL;
            g->d_bytes_cap = 0;
            if (hipMalloc((void **)&g->d_bytes, nb) != hipSuccess) return -1;
            g->d_bytes_cap = nb;
        }
        if (hipMemcpyAsync(g->d_off, g->off, ((size_t)vocab_size + 1) * sizeof(uint32_t), hipMemcpyHostToDevice,
                           st) != hipSuccess)
            return -1;
        if (g->tab_bytes &&
            hipMemcpyAsync(g->d_bytes, g->bytes, g->tab_bytes, hipMemcpyHostToDevice, st) != hipSuccess)
            return -1;
    }
    const int words = (vocab_size + 31) / 32;
    if (words > g->hmask_cap) {
        uint32_t *nm = realloc(g->hmask, (size_t)words * sizeof(uint32_t));
        if (!nm) return -1;
        g->hmask = nm;
        g->hmask_cap = words;
    }
    if (hipMemcpyAsync(g->d_row, &g->row, sizeof(g->row), hipMemcpyHostToDevice, st) != hipSuccess) return -1;
    if (dlk_grammar_mask(g->d_off, g->d_bytes, vocab_size, g->d_row, 1, eos_token_id, g->dev.mask, g->dev.mask_cap,
                         NULL, 0, g->dev.ids, st) != DLK_OK)
        return -1;
    int32_t valid = 0;
    if (hipMemcpyAsync(g->hmask, g->dev.mask, (size_t)words * sizeof(uint32_t), hipMemcpyDeviceToHost, st) !=
        hipSuccess)
        return -1;
    if (hipMemcpyAsync(&valid, g->dev.ids, sizeof(int32_t), hipMemcpyDeviceToHost, st) != hipSuccess) return -1;
    if (hipStreamSynchronize(st) != hipSuccess) return -1;
    /* the mask's cleared bits: logits[t] = -INFINITY (src/core/grammar.c:295-305) */
    for (int w = 0; w < words; w++) {
        uint32_t off = ~g->hmask[w];
        while (off) {
            const int t = 32 * w + __builtin_ctz(off);
            off &= off - 1u;
            if (t < vocab_size) logits[t] = -INFINITY;
        }
    }
    return valid;
}
