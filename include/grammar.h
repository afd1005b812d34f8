/*
 * grammar.h -- drop-in for DiskLLM's include/grammar.h (same names and
 * signatures; include/grammar.h:12-41 of the reference), implemented by
 * libdiskllm_amd.so.  The grammar keeps the reference's 8 KiB text buffer and,
 * beside it, the validator state after the buffer (dlk_grammar_row in
 * diskllm_amd.h), updated as tokens are appended, so that apply_mask resumes
 * every token from that state on the GPU instead of rescanning the buffer; only
 * the packed mask (a bit per token) comes back, and the disallowed logits are
 * set to -inf in place from it.
 */
#ifndef DISKLLM_GRAMMAR_H
#define DISKLLM_GRAMMAR_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct diskllm_grammar diskllm_grammar;

/* Mode from the grammar text (src/core/grammar.c:16-52): receipt when it names
 * bbox_2d, JSON when it names object or value, otherwise unconstrained. */
diskllm_grammar *diskllm_grammar_init_from_file(const char *filepath);
diskllm_grammar *diskllm_grammar_init_from_str(const char *grammar_str);
diskllm_grammar *diskllm_grammar_init_json(void);

void diskllm_grammar_free(diskllm_grammar *g);

/* Empty the buffer (src/core/grammar.c:58-63). */
void diskllm_grammar_reset(diskllm_grammar *g);

/* Would buffer + piece still be a valid prefix (src/core/grammar.c:228-246)? */
bool diskllm_grammar_accept_str(const diskllm_grammar *g, const char *piece);

/* Append a chosen token's string; dropped when it would not fit (src/core/grammar.c:248-256). */
void diskllm_grammar_advance(diskllm_grammar *g, const char *piece);

/* Balanced, outside a string and longer than one byte (src/core/grammar.c:258-273). */
bool diskllm_grammar_is_finished(const diskllm_grammar *g);

/* Set every token that may not follow to -INFINITY in the host row and return
 * the number allowed (src/core/grammar.c:275-308).  The token strings are read
 * through get_token_str on every call, as the reference does; the table is only
 * re-uploaded to the device when it changed. */
int diskllm_grammar_apply_mask(diskllm_grammar *g, float *logits, int vocab_size, void *tok_ctx,
                               const char *(*get_token_str)(void *ctx, int token_id), int eos_token_id);

#ifdef __cplusplus
}
#endif

#endif
