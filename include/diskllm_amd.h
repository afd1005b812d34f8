/*
 * diskllm_amd.h -- batched, device-resident C ABI of the MI355X sampling and
 * grammar-mask path.
 *
 * The drop-in headers include/sampler.h and include/grammar.h keep DiskLLM's
 * single-row host API; this header adds the batched entry points they are built
 * on.  All pointers below are device pointers unless stated otherwise; every
 * call is asynchronous on `stream` and returns a DLK_* status.
 *
 * Row semantics are those of the reference caller diskllm_sample_grammar()
 * (src/core/sampler_api.c:48-73) with the allow-mask in place of the grammar
 * callback: mask -> penalties (in `penalty_order`) -> sampler_sample()
 * (src/sampler.c:136-234).  Token ids are bit-identical to the reference built
 * as strict ISO C (-std=c11 -O2) on the same inputs and the same xorshift state.
 */
#ifndef DISKLLM_AMD_H
#define DISKLLM_AMD_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DLK_OK 0
#define DLK_ERR_INVALID (-1)      /* bad argument */
#define DLK_ERR_UNSUPPORTED (-2)  /* shape or parameter outside the supported range */
#define DLK_ERR_HIP (-3)          /* a HIP runtime call failed */
#define DLK_ERR_FORMAT (-4)       /* a file that cannot be opened, is truncated or is not in the format read */

/* Device status bits written by the kernels (dlk_batch.status). */
#define DLK_STATUS_HISTORY_TOO_LONG 1u  /* a row's history exceeded max_history: its id is -1 */
#define DLK_STATUS_SYNC_TIMEOUT 2u      /* a cross-workgroup wait gave up: the call's ids are invalid,
                                           though each stays inside [0, vocab) */
#define DLK_STATUS_UNSUPPORTED_ROW 4u   /* reserved: no row kind is refused any more (rows whose
                                           s = (l - max) / T holds NaN with top_k > 4096 are served) */

/* Penalty ops, packed low nibble first into dlk_sample_params.penalty_order. */
#define DLK_OP_REPETITION 1u  /* src/sampler.c:21-33, once per occurrence */
#define DLK_OP_FREQUENCY 2u   /* builder-defined: l -= f * count, once per distinct id */
#define DLK_OP_PRESENCE 3u    /* src/sampler.c:35-52, once per distinct id */
/* Reference caller order: presence then repetition (src/core/sampler_api.c:55-61). */
#define DLK_ORDER_REFERENCE (DLK_OP_PRESENCE | (DLK_OP_REPETITION << 4))
/* repetition -> frequency -> presence. */
#define DLK_ORDER_REP_FREQ_PRES (DLK_OP_REPETITION | (DLK_OP_FREQUENCY << 4) | (DLK_OP_PRESENCE << 8))

typedef struct {
    /* sampler_config (include/sampler.h:10-16) without the seed: */
    float temperature;        /* 0 = greedy; any other value as the reference uses it (1/temperature
                                 negative, zero or infinite included, src/sampler.c:154) */
    int top_k;                /* active when 0 < top_k < vocab */
    float top_p;              /* active when < 1 */
    float min_p;              /* active when > 0 (absolute threshold, src/sampler.c:189) */
    /* penalties (diskllm_sampler_params, include/diskllm.h:48-56, plus frequency): */
    float repeat_penalty;     /* active when > 1 */
    float frequency_penalty;  /* active when != 0 */
    float presence_penalty;   /* active when != 0 */
    uint32_t penalty_order;   /* DLK_ORDER_* or any packing of DLK_OP_* */
    int max_history;          /* upper bound on any row's history length (0 = 1024); above 1024 the
                                 penalties are applied to a scratch copy of the rows first */
    int n_out;                /* candidate outputs per row (0 = none) */
    int path;                 /* DLK_PATH_AUTO; the others force one implementation (tests) */
    float softcap;            /* > 0: logits = softcap * tanhf(logits / softcap) first, as the
                                 reference's decode step does (src/core/context.c:873-876); else none */
} dlk_sample_params;

#define DLK_PATH_AUTO 0        /* fastest path that covers the configuration */
#define DLK_PATH_ROW 1         /* one workgroup per row, every sum emulated exactly */
#define DLK_PATH_FULL_EXACT 2  /* fused full-vocabulary kernel with every row finished by its exact
                                  fallbacks: the softmax, min-p and top-p sums found by the split exact
                                  sums and the draw walked slice by slice from each slice's exact start,
                                  as for a row whose certified bounds or candidate chains do not decide
                                  them (tests) */
#define DLK_PATH_FULL_NO_WAIT 3  /* fused full-vocabulary kernel whose cross-workgroup waits give up at the
                                   first poll that finds a word not yet written: forces the
                                   DLK_STATUS_SYNC_TIMEOUT path (tests; the ids are then invalid).
                                   Shapes whose slices hold 24 entries per thread, no soft-cap;
                                   others return DLK_ERR_UNSUPPORTED */

typedef struct {
    const float *logits;      /* [rows, ld] fp32, read only */
    int64_t ld;               /* row stride in elements (>= vocab) */
    const int32_t *hist_off;  /* [rows+1] CSR offsets into hist_ids, or NULL */
    const int32_t *hist_ids;  /* previously seen token ids (out-of-range ids are skipped) */
    const uint32_t *mask;     /* packed allow-masks, bit i%32 of word i/32 (1 = allowed), or NULL */
    int64_t mask_ld;          /* words between mask rows */
    const int32_t *mask_row;  /* [rows] mask row used by each row (e.g. a DFA state), or NULL = row */
    uint64_t *rng;            /* [rows] xorshift64 states (non-zero), advanced once per sampled row */
    int32_t *out_ids;         /* [rows] sampled token ids */
    int32_t *out_cand_ids;    /* [rows, n_out] first n_out candidates in buffer order, or NULL */
    float *out_cand_probs;    /* [rows, n_out] their softmax probabilities (src/sampler.c:183-185) */
    float *out_cand_logprobs; /* [rows, n_out] log of their final sampling probability (-inf if cut) */
    uint32_t *status;         /* one word of DLK_STATUS_* bits, OR-ed by the kernels, or NULL */
} dlk_batch;

/* Initial xorshift state for a seed (src/sampler.c:87): seed 0 -> 0xDEADBEEF12345678. */
uint64_t dlk_seed_state(uint64_t seed);

/* Sample one token per row.  Replaces, for a batch of rows, the sequence
 * diskllm_grammar_apply_mask (as a packed mask) -> sampler_apply_*_penalty ->
 * sampler_sample of the reference (src/core/sampler_api.c:48-63). */
int dlk_sample(const dlk_batch *batch, int rows, int vocab, const dlk_sample_params *params,
               hipStream_t stream);

/* Workspace lifetime.  dlk_sample and the calls built on it keep one lazily
 * grown device workspace per (device, stream) they are called on (kernels queued
 * on one stream run in order and share it; calls on different streams never
 * do).  It is held until the process ends or until this call, which waits for
 * the stream's queued work and frees the stream's workspaces on the current
 * device.  Call it before destroying a stream that was passed to dlk_sample; a
 * later call on the stream allocates afresh.  No counterpart in the reference,
 * whose sampler owns a host work buffer freed by sampler_free
 * (src/sampler.c:91-95). */
int dlk_release_stream(hipStream_t stream);

/* dlk_sample without any allocation.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops and harnesses that forbid hipMalloc).  Same arguments, kernels
 * and results as dlk_sample; its workspace is a fixed 64 MiB scratch array per
 * device (held until the process ends), whose counter words each call clears
 * with a fill kernel on `stream`.  Every call on a device shares that device's
 * array, so calls that overlap on one device race.  DLK_ERR_UNSUPPORTED when the
 * call needs more than the array holds or a second buffer: max_history > 1024
 * (the penalties then run on a scratch copy of the rows), or a batch whose
 * kernels' workspace exceeds the array (the fused full-vocabulary kernel takes
 * as many rows per launch as the array holds, about 680 KB per row at a
 * vocabulary of 151,936). */
#define DLK_NOALLOC_SCRATCH_BYTES (64u << 20)
int dlk_sample_noalloc(const dlk_batch *batch, int rows, int vocab, const dlk_sample_params *params,
                       hipStream_t stream);

/* Byte-DFA allow-masks (no reference counterpart; replaces the accept_str
 * callback loop of src/core/grammar.c:284-306 for byte-level automata).
 * Token t = bytes[off[t] .. off[t+1]) is allowed from state s iff s != 0, the
 * token is non-empty and no prefix walk through trans[s*256 + byte] reaches
 * state 0; the EOS id (if >= 0) is allowed iff bit s of accept_mask is set.
 * Writes out_mask[r * mask_ld + w] for the n_rows states in `states`. */
int dlk_dfa_mask(const uint32_t *off, const uint8_t *bytes, int vocab, const uint8_t *trans, int n_states,
                 const int32_t *states, int n_rows, int eos_id, uint64_t accept_mask, uint32_t *out_mask,
                 int64_t mask_ld, hipStream_t stream);

/* y[i] = expf(x[i]) for i < n, bit-identical to the host libm expf that the
 * reference's softmax calls (src/sampler.c:179; glibc 2.35, x86-64 FMA variant). */
int dlk_expf(const float *x, float *y, int64_t n, hipStream_t stream);

/* Penalties in place on device logits [rows, ld], history as in dlk_batch
 * (hist_off [rows+1], hist_ids).  One call replaces, per row,
 * sampler_apply_presence_penalty (src/sampler.c:35-52: `pres` subtracted once
 * per distinct in-range id) and sampler_apply_repetition_penalty (:21-33: once
 * per occurrence, negative logits multiplied, others divided, only when
 * rep > 1), plus the frequency penalty (freq * count once per distinct id), in
 * `order` (DLK_OP_* nibbles, low first). */
int dlk_apply_penalties(float *logits, int64_t ld, int rows, int vocab, const int32_t *hist_off,
                        const int32_t *hist_ids, uint32_t order, float rep, float freq, float pres,
                        hipStream_t stream);

/* ---- grammar masks (src/core/grammar.c) ------------------------------------ */

/* Grammar modes, chosen from the grammar text as diskllm_grammar_init_from_str
 * does (src/core/grammar.c:21-26): receipt when it names bbox_2d (checked
 * first, :240), else JSON when it names object or value, else no constraint. */
#define DLK_GRAMMAR_NONE 0
#define DLK_GRAMMAR_JSON 1
#define DLK_GRAMMAR_RECEIPT 2
#define DLK_GRAMMAR_BUF 8192      /* the reference's buffer: buffer + piece must stay < 8191 bytes */

/* State of one validator after the bytes fed so far (a resumable form of
 * is_valid_receipt_prefix / is_valid_json_prefix, src/core/grammar.c:68-226). */
typedef struct {
    int32_t mode;             /* DLK_GRAMMAR_* */
    int32_t pc;               /* program point; 255 = rejected */
    int32_t n, m;             /* receipt: key / number position; JSON: brace / bracket depth */
    uint8_t prev;             /* previous byte */
    uint8_t flag;             /* receipt: the number had a digit; JSON: inside a string */
    uint8_t pad[2];
} dlk_scan_state;

/* Balance of the whole buffer (diskllm_grammar_is_finished, src/core/grammar.c:258-273). */
typedef struct {
    int32_t braces, brackets;
    int32_t len;              /* bytes in the buffer */
    uint8_t in_str, prev, pad[2];
} dlk_balance_state;

/* One sequence's grammar position: everything the mask needs about its buffer. */
typedef struct {
    dlk_scan_state scan;
    dlk_balance_state bal;
} dlk_grammar_row;

/* Host helpers (plain C, no device work): the mode a grammar text selects, a
 * fresh row, and a row advanced by n appended buffer bytes. */
int dlk_grammar_mode_of(const char *grammar_text);
void dlk_grammar_row_init(dlk_grammar_row *row, int mode);
void dlk_grammar_row_feed(dlk_grammar_row *row, const char *bytes, int n);

/* Grammar allow-masks for `rows` sequences (states: device array of
 * dlk_grammar_row) over one vocabulary of token strings in CSR form, token t =
 * bytes[off[t] .. off[t+1]) read up to its first NUL (strlen).  Per token, as
 * diskllm_grammar_apply_mask (src/core/grammar.c:275-308): the EOS id is
 * allowed iff the buffer is finished; an empty string is not allowed; any other
 * token iff buffer + token fits the buffer and is still a valid prefix.
 * Writes mask[r * mask_ld + w] (bit t%32 of word t/32, 1 = allowed); when
 * `logits` is not NULL sets disallowed logits[r * ld + t] to -inf; when `valid`
 * is not NULL writes each row's allowed count (the reference's return value). */
int dlk_grammar_mask(const uint32_t *off, const uint8_t *bytes, int vocab, const dlk_grammar_row *states,
                     int rows, int eos_id, uint32_t *mask, int64_t mask_ld, float *logits, int64_t ld,
                     int32_t *valid, hipStream_t stream);

/* The device form of diskllm_grammar_advance (src/core/grammar.c:248-256) as
 * diskllm_sample_grammar applies it after the draw (src/core/sampler_api.c:
 * 65-70): for each row whose token (device array) is not eos_id, that token's
 * string (up to its first NUL) is appended to the row's buffer when buffer +
 * string stays below 8191 bytes, i.e. the row's states take those bytes. */
int dlk_grammar_advance(const uint32_t *off, const uint8_t *bytes, int vocab, dlk_grammar_row *states,
                        const int32_t *tokens, int rows, int eos_id, hipStream_t stream);

/* One constrained decoding step for a batch, on the device, replacing
 * diskllm_sample_grammar (src/core/sampler_api.c:48-73) per row: the grammar
 * mask of each row's state (written to batch->mask, which must be a
 * [rows, mask_ld] buffer, and mask_row NULL), penalties and the draw as
 * dlk_sample (params->order DLK_ORDER_REFERENCE gives the reference's order),
 * then the rows' states advanced by the drawn tokens.
 * Unlike the reference it does not write -inf into the caller's logits. */
int dlk_sample_grammar(const dlk_batch *batch, int rows, int vocab, const dlk_sample_params *params,
                       const uint32_t *off, const uint8_t *bytes, dlk_grammar_row *states, int eos_id,
                       hipStream_t stream);

/* The reference's logit soft-cap, in place: logits[r * ld + i] = cap *
 * tanhf(logits[r * ld + i] / cap) for i < vocab (src/core/context.c:604-606
 * after a prefill, :873-876 after a decode step, a host loop there), with tanhf
 * bit-identical to the host libm's.  No-op unless cap > 0, as in the reference. */
int dlk_softcap(float *logits, int64_t ld, int rows, int vocab, float cap, hipStream_t stream);

/* The vocabulary table of the calls above (token t = bytes[off[t] .. off[t+1]),
 * read up to its first NUL) from a GGUF file's `tokenizer.ggml.tokens` string
 * array: the strings tokenizer_init loads (src/tokenizer.c:247-300) and
 * tokenizer_decode_raw returns (src/tokenizer.c:377-380).  Host memory, no
 * device work.  The table covers ids 0 .. vocab-1 (vocab <= 0: one id per
 * string); ids past the file's strings get empty entries, which the mask
 * disallows as the reference does the NULL string it gets for them.  A file
 * with no tokens array gives an all-empty table (the reference's tokenizer
 * has vocab_size 0 then).  Call once with off = NULL to get *n_tokens (the
 * array's length) and *n_bytes (bytes the table needs), then with off
 * ([vocab+1] entries) and bytes ([bytes_cap] bytes) to fill them.
 * DLK_ERR_FORMAT: the file cannot be opened, is truncated, is not GGUF, or its
 * tokens array does not hold strings; DLK_ERR_INVALID: bytes_cap too small. */
int dlk_vocab_csr_from_gguf(const char *path, int vocab, uint32_t *off, uint8_t *bytes, int64_t bytes_cap,
                            int32_t *n_tokens, int64_t *n_bytes);

/* The token-string callback of diskllm_grammar_apply_mask (include/grammar.h,
 * src/core/grammar.c:275-308: NUL-terminated strings, NULL for no string) over a
 * table in the form above, for callers that hold the vocabulary as that table
 * rather than as a tokenizer (no counterpart in the reference, whose caller
 * passes tokenizer_decode_raw, src/core/sampler_api.c:42-46).  ctx points to a
 * dlk_csr_vocab; the string is copied into its scratch buffer (scratch_cap
 * bytes; longer entries are cut there), so one ctx serves one thread at a time.
 * NULL for ids outside [0, vocab). */
typedef struct {
    const uint32_t *off;      /* [vocab+1] */
    const uint8_t *bytes;
    int vocab;
    char *scratch;            /* [scratch_cap] */
    int scratch_cap;
} dlk_csr_vocab;
const char *dlk_csr_token_str(void *ctx, int token_id);

#ifdef __cplusplus
}
#endif

#endif
