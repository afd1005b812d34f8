/*
 * gguf_vocab.c -- the vocabulary table the grammar kernels read, taken from a
 * GGUF file's `tokenizer.ggml.tokens` string array (the strings DiskLLM's
 * tokenizer_init loads, src/tokenizer.c:247-300, and tokenizer_decode_raw
 * hands to the grammar, src/tokenizer.c:377-380).
 *
 * Only the metadata section is read: the header, then key/value pairs until the
 * tokens array.  A pair of any other key is stepped over by its type's size
 * (arrays element by element, nested arrays included).  Buffered stdio, one
 * pass per call; the first call (off == NULL) only sizes the table.
 */
#define _FILE_OFFSET_BITS 64
#define _POSIX_C_SOURCE 200809L
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "diskllm_amd.h"

enum {
    GGUF_U8 = 0, GGUF_I8, GGUF_U16, GGUF_I16, GGUF_U32, GGUF_I32, GGUF_F32, GGUF_BOOL,
    GGUF_STRING = 8, GGUF_ARRAY = 9, GGUF_U64 = 10, GGUF_I64, GGUF_F64
};

static const char kTokensKey[] = "tokenizer.ggml.tokens";

static int rd(FILE *f, void *p, size_t n) { return fread(p, 1, n, f) == n ? 0 : -1; }

static int skip(FILE *f, uint64_t n) {
    /* fseeko past the end succeeds; the next read then fails, which is what
     * reports a truncated file. */
    return n > (uint64_t)INT64_MAX ? -1 : (fseeko(f, (off_t)n, SEEK_CUR) == 0 ? 0 : -1);
}

static int scalar_size(uint32_t type) {
    switch (type) {
    case GGUF_U8: case GGUF_I8: case GGUF_BOOL: return 1;
    case GGUF_U16: case GGUF_I16: return 2;
    case GGUF_U32: case GGUF_I32: case GGUF_F32: return 4;
    case GGUF_U64: case GGUF_I64: case GGUF_F64: return 8;
    default: return 0;
    }
}

/* Steps over one value of `type`; depth bounds nested arrays. */
static int skip_value(FILE *f, uint32_t type, int depth) {
    const int sz = scalar_size(type);
    if (sz) return skip(f, (uint64_t)sz);
    if (type == GGUF_STRING) {
        uint64_t len;
        return rd(f, &len, 8) ? -1 : skip(f, len);
    }
    if (type != GGUF_ARRAY || depth > 8) return -1;
    uint32_t et;
    uint64_t n;
    if (rd(f, &et, 4) || rd(f, &n, 8)) return -1;
    const int esz = scalar_size(et);
    if (esz) return n > (uint64_t)INT64_MAX / (uint64_t)esz ? -1 : skip(f, n * (uint64_t)esz);
    for (uint64_t i = 0; i < n; i++)
        if (skip_value(f, et, depth + 1)) return -1;
    return 0;
}

/* Positions f at the first string of the tokens array and returns its length
 * in *count; 1 when the file holds no such array, -1 on a read or format error. */
static int seek_tokens(FILE *f, uint64_t *count) {
    char magic[4];
    uint32_t version;
    uint64_t n_tensors, n_kv;
    if (rd(f, magic, 4) || memcmp(magic, "GGUF", 4) || rd(f, &version, 4) || rd(f, &n_tensors, 8) ||
        rd(f, &n_kv, 8))
        return -1;
    char key[sizeof(kTokensKey)];
    for (uint64_t i = 0; i < n_kv; i++) {
        uint64_t klen;
        uint32_t type;
        if (rd(f, &klen, 8)) return -1;
        int match = 0;
        if (klen == sizeof(kTokensKey) - 1) {
            if (rd(f, key, klen)) return -1;
            match = memcmp(key, kTokensKey, klen) == 0;
        } else if (skip(f, klen)) {
            return -1;
        }
        if (rd(f, &type, 4)) return -1;
        if (match && type == GGUF_ARRAY) {
            uint32_t et;
            if (rd(f, &et, 4) || rd(f, count, 8)) return -1;
            if (et != GGUF_STRING) return -1;
            return 0;
        }
        if (skip_value(f, type, 0)) return -1;
    }
    return 1;
}

int dlk_vocab_csr_from_gguf(const char *path, int vocab, uint32_t *off, uint8_t *bytes, int64_t bytes_cap,
                            int32_t *n_tokens, int64_t *n_bytes) {
    if (!path || (off && !bytes && bytes_cap > 0) || bytes_cap < 0) return DLK_ERR_INVALID;
    FILE *f = fopen(path, "rb");
    if (!f) return DLK_ERR_FORMAT;
    setvbuf(f, NULL, _IOFBF, 1 << 20);
    uint64_t count = 0;
    const int found = seek_tokens(f, &count);
    if (found < 0 || count > (uint64_t)INT32_MAX) {
        fclose(f);
        return found < 0 ? DLK_ERR_FORMAT : DLK_ERR_UNSUPPORTED;
    }
    if (found == 1) count = 0;    /* no tokens array: every id decodes to nothing */
    const int64_t ids = vocab > 0 ? vocab : (int64_t)count;
    const uint64_t take = count < (uint64_t)ids ? count : (uint64_t)ids;
    uint64_t total = 0;
    for (uint64_t t = 0; t < take; t++) {
        uint64_t len;
        if (rd(f, &len, 8)) {
            fclose(f);
            return DLK_ERR_FORMAT;
        }
        if (len > UINT32_MAX - total) {    /* offsets are 32-bit */
            fclose(f);
            return DLK_ERR_UNSUPPORTED;
        }
        if (off) {
            off[t] = (uint32_t)total;
            if ((int64_t)(total + len) > bytes_cap || rd(f, bytes + total, len)) {
                fclose(f);
                return (int64_t)(total + len) > bytes_cap ? DLK_ERR_INVALID : DLK_ERR_FORMAT;
            }
        } else if (skip(f, len)) {
            fclose(f);
            return DLK_ERR_FORMAT;
        }
        total += len;
    }
    if (!off && take) {
        /* The sizing pass stepped over the strings with seeks only; reading
         * the last byte they span shows the file holds them all. */
        uint8_t b;
        if (fseeko(f, -1, SEEK_CUR) || rd(f, &b, 1)) {
            fclose(f);
            return DLK_ERR_FORMAT;
        }
    }
    fclose(f);
    if (off)
        for (int64_t t = (int64_t)take; t <= ids; t++) off[t] = (uint32_t)total;
    if (n_tokens) *n_tokens = (int32_t)count;
    if (n_bytes) *n_bytes = (int64_t)total;
    return DLK_OK;
}

const char *dlk_csr_token_str(void *ctx, int token_id) {
    const dlk_csr_vocab *v = (const dlk_csr_vocab *)ctx;
    if (!v || !v->off || !v->scratch || v->scratch_cap <= 0 || token_id < 0 || token_id >= v->vocab) return NULL;
    size_t n = (size_t)(v->off[token_id + 1] - v->off[token_id]);
    if (n > (size_t)v->scratch_cap - 1) n = (size_t)v->scratch_cap - 1;
    memcpy(v->scratch, v->bytes + v->off[token_id], n);
    v->scratch[n] = '\0';
    return v->scratch;
}
