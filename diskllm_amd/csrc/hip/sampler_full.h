/*
 * sampler_full.h -- parameters of the fused full-vocabulary path (top-k off).
 */
#ifndef DLK_SAMPLER_FULL_H
#define DLK_SAMPLER_FULL_H

#include "sampler_params.h"

namespace dlk {

constexpr int kFullThreads = 1024;
constexpr int kFullMaxG = 16;        /* workgroups per row */
constexpr int kPubWords = 16;        /* 64-bit words each workgroup publishes */
constexpr int kCandSlots = 2;        /* predicted top-p crossing chunks per workgroup */
constexpr int kSyncWords = 64;       /* per-row synchronisation words */

/* per-row sync words (all zero between launches) */
enum : int {
    kSyncExit = 3,     /* workgroups finished */
    kSyncDone = 4,     /* token written */
    kSyncChain = 16,   /* + w: running value for workgroup w is ready */
    kSyncChainVal = 32,/* + w: that running value (float bits) */
    kSyncWalk = 48     /* + w: walk data of slice w published for workgroup 0 */
};

/* published words per workgroup */
enum : int {
    kPubMax = 0,       /* float bits of the slice maximum */
    kPubE = 1,         /* double: slice sum of e */
    kPubP = 2,         /* double: slice sum of p */
    kPubNCand = 3,     /* number of crossing-candidate chunks */
    kPubCandChunk = 4, /* + s: global chunk index */
    kPubCandPre = 6,   /* + s: double, slice-local exclusive p prefix at that chunk */
    kPubP0 = 8,        /* float bits of p_0 (workgroup 0) */
    kPubStaged = 9,    /* staged chunks in the published walk data */
    kPubNElem = 10,    /* entries of the published element-chunk list */
};

struct FullParams {
    RowParams p;
    int G;             /* workgroups per row */
    int S;             /* slice length = EPT * kFullThreads */
    int stage_cap;     /* chunks of final probabilities kept in LDS per workgroup */
    int pf_slices;     /* later slices whose walk data workgroup 0 prefetches into LDS */
    int pf_cap;        /* staged chunks of a prefetched slice that fit its buffer */
    uint32_t *sync;    /* [rows][kSyncWords] */
    uint64_t *pub;     /* [rows][G][kPubWords], in the zeroed counter region: a word that readers
                          poll carries kReady (bit 63) once written; all zero between launches */
    float *cvals;      /* [rows][G][kCandSlots][64] */
    int4 *wrecs;       /* [rows][G][nch]: each chunk's walk record (make_rec in exact_scan.h), stored as
                          two arrays of 64-bit halves {x | y << 32}[nch] then {z | w << 32}[nch] */
    float *wsvals;     /* [rows][G][stage_cap * 64]: staged chunks */
    double *wshalf;    /* [rows][G][stage_cap]: first-half sum of each staged chunk */
    int2 *wel;         /* [rows][G][stage_cap]: element-level chunks {chunk, slot} in order */
    unsigned char *fb; /* [rows][fb_bytes]: global aggregates for the exact fallback */
    size_t fb_bytes;
    int force_exact;   /* test hook: send every row through the exact fallback */
};

}  // namespace dlk

#endif
