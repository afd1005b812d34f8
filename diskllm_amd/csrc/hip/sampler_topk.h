/*
 * sampler_topk.h -- parameters and workspace slots of the single-pass top-k path.
 */
#ifndef DLK_SAMPLER_TOPK_H
#define DLK_SAMPLER_TOPK_H

#include "sampler_params.h"

namespace dlk {

constexpr int kTopkThreads = 256;
constexpr int kSelWords = 260;              /* radix-select histogram (256) + broadcast words */
constexpr int kMergePerThread = 8;          /* merge: candidates per thread (G * KP <= 2048) */
constexpr int kTopkGroupCap = 1024;         /* listed 16-byte groups per slice at most (more: the row falls back) */
constexpr int kTopkMaxG = 64;               /* workgroups per row */
constexpr int kTopkMaxS = 65536;            /* slice length */
constexpr int kTopkMaxK = 496;              /* four waves' thresholds need KP = k + 16 <= 4 * 128 */
constexpr int kTopkHcapMax = 1024;          /* history capacity of a launch (longer histories take the pre-pass) */

/* What each slice workgroup publishes (relaxed agent-scope atomic stores). */
struct TopkSlot {
    uint32_t max_bits;   /* slice maximum of the prepared logits */
    uint32_t argmax;     /* its lowest index */
    uint32_t nfin;       /* finite entries in the slice */
    uint32_t kept;       /* candidates published */
    uint32_t complete;   /* 1: every finite entry published; 0: partial; 0xffffffff: overflow */
    uint32_t last_key;   /* desc key of the last published candidate */
    uint32_t first_nan;  /* bit 0 (slice 0): prepared logit 0 is NaN; bit 1: NaN or +inf in the slice */
    uint32_t pad;
};

struct TopkParams {
    RowParams p;
    int G;               /* workgroups per row */
    int S;               /* slice length: a multiple of 16 * kTopkThreads, at most kTopkMaxS */
    int KP;              /* candidates kept per slice: min(k + 16, ...) */
    int buf_cap;         /* merge buffer entries (LDS) */
    int grp_cap;         /* listed groups per slice (LDS) */
    int cand_cap;        /* slice candidates (LDS) */
    int spread;          /* 1: grid (rows, G), row blockIdx.x, slice blockIdx.y (a row's slices spread
                            over the CUs' dispatch slots); 0: grid (G, rows), slice blockIdx.x of row
                            blockIdx.y */
    uint32_t *counters;  /* [rows], zero between launches */
    TopkSlot *slots;     /* [rows * G] */
    uint64_t *cands;     /* [rows * G * KP] */
};

}  // namespace dlk

#endif
