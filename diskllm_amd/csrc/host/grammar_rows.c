/*
 * grammar_rows.c -- host side of the grammar rows of diskllm_amd.h: the mode a
 * grammar text selects and the validator state after appended bytes.  The byte
 * steps are the ones the mask kernel runs (hip/grammar_scan.h).
 */
#include <string.h>

#include "diskllm_amd.h"
#include "../hip/grammar_scan.h"

int dlk_grammar_mode_of(const char *text) {
    if (!text) return DLK_GRAMMAR_NONE;
    if (strstr(text, "bbox_2d")) return DLK_GRAMMAR_RECEIPT;                   /* src/core/grammar.c:21, :240 */
    if (strstr(text, "object") || strstr(text, "value")) return DLK_GRAMMAR_JSON;   /* :24 */
    return DLK_GRAMMAR_NONE;
}

void dlk_grammar_row_init(dlk_grammar_row *row, int mode) {
    memset(row, 0, sizeof(*row));
    dlk_scan_init(&row->scan, mode);
}

void dlk_grammar_row_feed(dlk_grammar_row *row, const char *bytes, int n) {
    for (int i = 0; i < n; i++) {
        const uint8_t c = (uint8_t)bytes[i];
        dlk_scan_step(&row->scan, c);
        dlk_balance_step(&row->bal, c);
    }
}
