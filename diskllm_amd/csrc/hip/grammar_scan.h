/*
 * grammar_scan.h -- the reference's grammar validators as resumable byte scanners,
 * shared by the host library and the mask kernel (gfx950).
 *
 * The reference checks a candidate token by re-running a validator over
 * buffer + piece from the start (diskllm_grammar_accept_str, src/core/grammar.c:
 * 228-246).  Both validators read left to right, look at most one byte back, and
 * answer "true" wherever the input runs out (every `if (i >= len) return true`),
 * so they are streaming machines: the state after the buffer is computed once and
 * each token only feeds its own bytes.  A prefix is accepted iff no byte is
 * rejected.  The program points below follow the source line by line:
 *
 *   receipt  src/core/grammar.c:68-194  {"bbox_2d": [n, n, n, n], "text_content": "..."}
 *   json     src/core/grammar.c:197-226 leading whitespace, then '{' or '[', then
 *            quote toggling (previous byte not '\') and brace / bracket depth >= 0
 *   finished src/core/grammar.c:258-273 balanced, not in a string, length > 1
 *
 * isspace / isdigit are those of the "C" locale.
 */
#ifndef DLK_GRAMMAR_SCAN_H
#define DLK_GRAMMAR_SCAN_H

#include <stdint.h>

#include "../../../include/diskllm_amd.h"

#if defined(__HIPCC__)
#define DLK_GHD __host__ __device__ inline
#else
#define DLK_GHD static inline
#endif

/* program points of the receipt validator */
enum {
    DLK_RC_WS0 = 0,     /* :70-75   leading whitespace, then '{' */
    DLK_RC_WS1,         /* :81-82   whitespace before the first key */
    DLK_RC_KEY1,        /* :85-97   "\"bbox_2d\":" (n = matched; ':' may be a space) */
    DLK_RC_WS2,         /* :99-103  whitespace, then '[' */
    DLK_RC_NUM_A,       /* :107-108 whitespace before number n */
    DLK_RC_DIGITS,      /* :111-117 digits of number n (flag = had a digit) */
    DLK_RC_NUM_B,       /* :119-138 whitespace, then ',' / ']' / a digit */
    DLK_RC_AFTER,       /* :140-146 whitespace, then ',' */
    DLK_RC_WS3,         /* :148-149 whitespace before the second key */
    DLK_RC_KEY2,        /* :152-160 "\"text_content\":" (n = matched) */
    DLK_RC_WS4,         /* :162-166 whitespace, then '"' */
    DLK_RC_STR,         /* :169-177 string body up to an unescaped '"' */
    DLK_RC_WS5,         /* :181-183 whitespace, then '}' */
    DLK_RC_WS6,         /* :185-187 whitespace only */
    DLK_JS_WS = 16,     /* :199-204 leading whitespace, then '{' or '[' */
    DLK_JS_BODY,        /* :209-224 */
    DLK_SCAN_REJECT = 255
};

DLK_GHD int dlk_isspace(uint8_t c) { return c == ' ' || (c >= 9 && c <= 13); }
DLK_GHD int dlk_isdigit(uint8_t c) { return c >= '0' && c <= '9'; }

DLK_GHD uint8_t dlk_key1(int k) {
    /* "bbox_2d": */
    const uint8_t s[10] = {'"', 'b', 'b', 'o', 'x', '_', '2', 'd', '"', ':'};
    return s[k];
}
DLK_GHD uint8_t dlk_key2(int k) {
    /* "text_content": */
    const uint8_t s[15] = {'"', 't', 'e', 'x', 't', '_', 'c', 'o', 'n', 't', 'e', 'n', 't', '"', ':'};
    return s[k];
}

/* One byte of the receipt validator.  A byte that leaves its program point
 * without being consumed is handed to the next point (the `continue`). */
DLK_GHD void dlk_receipt_step(dlk_scan_state *s, uint8_t c) {
    while (1) {
        switch (s->pc) {
            case DLK_RC_WS0:
                if (dlk_isspace(c)) break;
                if (c != '{') { s->pc = DLK_SCAN_REJECT; break; }
                s->pc = DLK_RC_WS1;
                break;
            case DLK_RC_WS1:
                if (dlk_isspace(c)) break;
                s->pc = DLK_RC_KEY1;
                s->n = 0;
                continue;
            case DLK_RC_KEY1: {
                const uint8_t want = dlk_key1(s->n);
                if (c != want && !(want == ':' && dlk_isspace(c))) { s->pc = DLK_SCAN_REJECT; break; }
                if (++s->n == 10) s->pc = DLK_RC_WS2;
                break;
            }
            case DLK_RC_WS2:
                if (dlk_isspace(c)) break;
                if (c != '[') { s->pc = DLK_SCAN_REJECT; break; }
                s->pc = DLK_RC_NUM_A;
                s->n = 0;
                break;
            case DLK_RC_NUM_A:
                if (dlk_isspace(c)) break;
                s->pc = DLK_RC_DIGITS;
                s->flag = 0;
                continue;
            case DLK_RC_DIGITS:
                if (dlk_isdigit(c)) { s->flag = 1; break; }
                if (!s->flag && c != ']' && c != ',') { s->pc = DLK_SCAN_REJECT; break; }
                s->pc = DLK_RC_NUM_B;
                continue;
            case DLK_RC_NUM_B:
                if (dlk_isspace(c)) break;
                if (s->n < 3) {
                    if (c == ',') { s->pc = DLK_RC_NUM_A; s->n++; break; }
                    if (dlk_isdigit(c)) { s->pc = DLK_RC_NUM_A; s->n++; continue; }
                } else {
                    if (c == ']') { s->pc = DLK_RC_AFTER; break; }
                    if (dlk_isdigit(c)) { s->pc = DLK_RC_AFTER; continue; }
                }
                s->pc = DLK_SCAN_REJECT;
                break;
            case DLK_RC_AFTER:
                if (dlk_isspace(c)) break;
                s->pc = c == ',' ? DLK_RC_WS3 : DLK_SCAN_REJECT;
                break;
            case DLK_RC_WS3:
                if (dlk_isspace(c)) break;
                s->pc = DLK_RC_KEY2;
                s->n = 0;
                continue;
            case DLK_RC_KEY2:
                if (c != dlk_key2(s->n)) { s->pc = DLK_SCAN_REJECT; break; }
                if (++s->n == 15) s->pc = DLK_RC_WS4;
                break;
            case DLK_RC_WS4:
                if (dlk_isspace(c)) break;
                s->pc = c == '"' ? DLK_RC_STR : DLK_SCAN_REJECT;
                break;
            case DLK_RC_STR:
                if (c == '"' && s->prev != '\\') s->pc = DLK_RC_WS5;
                break;
            case DLK_RC_WS5:
                if (dlk_isspace(c)) break;
                s->pc = c == '}' ? DLK_RC_WS6 : DLK_SCAN_REJECT;
                break;
            case DLK_RC_WS6:
                if (!dlk_isspace(c)) s->pc = DLK_SCAN_REJECT;
                break;
            default:
                break;
        }
        break;
    }
    s->prev = c;
}

/* One byte of the JSON validator. */
DLK_GHD void dlk_json_step(dlk_scan_state *s, uint8_t c) {
    if (s->pc == DLK_JS_WS) {
        if (dlk_isspace(c)) { s->prev = c; return; }
        if (c != '{' && c != '[') { s->pc = DLK_SCAN_REJECT; s->prev = c; return; }
        s->pc = DLK_JS_BODY;
    }
    if (s->pc == DLK_JS_BODY) {
        if (c == '"' && s->prev != '\\') {
            s->flag ^= 1;                            /* in string */
        } else if (!s->flag) {
            if (c == '{') s->n++;
            else if (c == '}') { if (--s->n < 0) s->pc = DLK_SCAN_REJECT; }
            else if (c == '[') s->m++;
            else if (c == ']') { if (--s->m < 0) s->pc = DLK_SCAN_REJECT; }
        }
    }
    s->prev = c;
}

/* Balance of the whole buffer for is_finished (src/core/grammar.c:258-273);
 * the reference's `char c` compares equal to the same ASCII bytes. */
DLK_GHD void dlk_balance_step(dlk_balance_state *b, uint8_t c) {
    if (c == '"' && (b->len == 0 || b->prev != '\\')) b->in_str ^= 1;
    if (!b->in_str) {
        if (c == '{') b->braces++;
        else if (c == '}') b->braces--;
        else if (c == '[') b->brackets++;
        else if (c == ']') b->brackets--;
    }
    b->prev = c;
    b->len++;
}

DLK_GHD int dlk_balance_finished(const dlk_balance_state *b) {
    /* len > 1 (and so also len != 0) */
    return b->braces == 0 && b->brackets == 0 && !b->in_str && b->len > 1;
}

DLK_GHD void dlk_scan_init(dlk_scan_state *s, int mode) {
    s->mode = mode;
    s->pc = mode == DLK_GRAMMAR_JSON ? DLK_JS_WS : DLK_RC_WS0;
    s->prev = 0;
    s->flag = 0;
    s->n = 0;
    s->m = 0;
}

DLK_GHD void dlk_scan_step(dlk_scan_state *s, uint8_t c) {
    if (s->pc == DLK_SCAN_REJECT) return;
    if (s->mode == DLK_GRAMMAR_RECEIPT) dlk_receipt_step(s, c);
    else if (s->mode == DLK_GRAMMAR_JSON) dlk_json_step(s, c);
}

DLK_GHD int dlk_scan_ok(const dlk_scan_state *s) { return s->mode == DLK_GRAMMAR_NONE || s->pc != DLK_SCAN_REJECT; }

#endif
