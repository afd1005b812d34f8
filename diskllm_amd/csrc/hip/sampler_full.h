/*
 * sampler_full.h -- parameters of the fused full-vocabulary path (top-k off).
 */
#ifndef DLK_SAMPLER_FULL_H
#define DLK_SAMPLER_FULL_H

#include "sampler_params.h"

namespace dlk {

constexpr int kFullThreads = 512;    /* two workgroups per CU */
constexpr int kFullMaxG = 16;        /* workgroups per row */
constexpr int kPubWords = 16;        /* 64-bit words each workgroup publishes */
constexpr int kCandSlots = 2;        /* predicted top-p crossing chunks per workgroup */
constexpr int kSyncWords = 64;       /* per-row synchronisation words */
constexpr uint32_t kFullSpinLimit = 1u << 22;   /* polls before a cross-workgroup wait gives up: a few seconds */

/* per-row sync words (all zero between launches) */
enum : int {
    kSyncExit = 3,     /* workgroups finished */
    kSyncLanes = 5,    /* workgroups that published their candidate chains */
    kSyncSplitE = 6,   /* workgroups that stored their slice of the split softmax sum */
    kSyncSplitP = 7,   /* workgroups that stored their slice of the split top-p cumulation */
    kSyncSplitM = 8    /* workgroups that stored their slice of the split min-p survivors' sum */
};

/* published words per workgroup */
enum : int {
    kPubMax = 0,       /* float bits of the slice maximum */
    kPubE = 1,         /* double: slice sum of e */
    kPubP = 2,         /* double: slice sum of p (min-p: of the kept p * inv2) */
    kPubS2 = 3,        /* min-p: double, slice sum of the surviving p */
    kPubA2 = 4,        /* min-p: double, slice sum of every p */
    kPubN2 = 5,        /* min-p: surviving entries in the slice */
    kPubSplitM = 6,    /* workgroup 0: the split min-p survivors' sum (double bits; NaN: a wait gave
                          up); word 7 its (unused) position */
    kPubP0 = 8,        /* float bits of p_0 (workgroup 0) */
    kPubF = 9,         /* double: the slice's predicted contribution to the draw's float sum */
    kPubX = 10,        /* from the slice holding the top-p crossing: x (bits 0-30, 0x7fffffff: not
                          certified) and the float bits of inv3 (bits 31-62) */
    kPubSplitE = 11,   /* workgroup 0: the split softmax sum (double bits; NaN: a wait gave up) */
    kPubSplitP = 13    /* workgroup 0: the split top-p cumulation's value (double bits) and, in
                          the next word, its threshold position (-1: none) */
};

constexpr int kMaxTabs = 32;         /* element-level chunks with a candidate table per workgroup */
constexpr int kLaneWords = 65;       /* per workgroup: 64 candidate chain results + the window base */

struct FullParams {
    RowParams p;
    int G;             /* workgroups per row */
    int S;             /* slice length = EPT * kFullThreads */
    int stage_cap;     /* chunks of final probabilities kept in LDS per workgroup */
    uint32_t *sync;    /* [rows][kSyncWords] */
    uint64_t *pub;     /* [rows][G][kPubWords], in the zeroed counter region: a word that readers
                          poll carries kReady (bit 63) once written; all zero between launches */
    uint64_t *lanes;   /* [rows][G][kLaneWords]: per candidate start of the slice, its end value
                          (low word) and crossing token (high word: -1 none, -2 unresolved);
                          word 64: float bits of candidate 0 */
    unsigned char *fb; /* [rows][fb_bytes]: global aggregates for the exact fallback and the split
                          sums, then (at fb_q_off) the row's values for the split sums or a slice's
                          for a re-walked draw */
    size_t fb_bytes, fb_q_off;
    int force_exact;   /* test hook: every row runs the split sums (as if no bound had decided
                          them) and re-walks the draw of every slice from its exact start (as if
                          no chain covered it) */
    int no_wait;       /* test hook: launch the instance whose waits give up at their first poll
                          that finds a word not yet written (DLK_STATUS_SYNC_TIMEOUT) */
};

}  // namespace dlk

#endif
