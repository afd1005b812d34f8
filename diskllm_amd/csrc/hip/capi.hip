/*
 * capi.hip -- host side of the batched C ABI (include/diskllm_amd.h): argument
 * checks, the scalars the reference computes on the host side of its loops
 * (1/temperature, the top-p threshold), LDS planning, workspace and the launch.
 */
#include <math.h>
#include <string.h>

#include <hip/hip_runtime.h>

#include <mutex>
#include <algorithm>
#include <vector>

#include "sampler_params.h"
#include "sampler_topk.h"
#include "sampler_full.h"

extern "C" int dlk_launch_row_kernel(const dlk::RowParams *p, int rows, size_t lds_bytes, hipStream_t stream);
extern "C" int dlk_launch_topk_kernel(const dlk::TopkParams *f, int rows, size_t lds, hipStream_t stream);
extern "C" int dlk_topk_kernel_occupancy(int kind, size_t lds);
extern "C" int dlk_launch_full_kernel(const dlk::FullParams *f, int rows, int ept, size_t lds, hipStream_t stream);
extern "C" int dlk_full_kernel_capacity(int ept, size_t lds, int cap, int hp);
extern "C" int dlk_launch_long_history_penalties(float *logits, int64_t ld, int rows, int vocab,
                                                 const int32_t *hist_off, const int32_t *hist_ids, uint32_t order,
                                                 float rep, float freq, float pres, int max_hist, int32_t *too_long,
                                                 const uint64_t *rng, uint64_t *rng_saved, hipStream_t stream);
extern "C" int dlk_launch_long_history_fixup(int rows, const int32_t *too_long, const uint64_t *rng_saved,
                                             uint64_t *rng, int32_t *out_ids, uint32_t *status, hipStream_t stream);
extern "C" int dlk_launch_prepare_rows(const float *src, int64_t ld, float *dst, int64_t dld, int rows, int vocab,
                                       const uint32_t *mask, int64_t mask_ld, const int32_t *mask_row, float cap,
                                       hipStream_t stream);

namespace {

constexpr size_t kMaxLds = 160 * 1024;
constexpr int kMaxTopKLds = 4096;          /* larger top-k: candidates in global memory */
constexpr int kHcapDirect = 1024;          /* longer histories: penalties applied to a scratch copy first */
constexpr size_t kGlobalTopkBudget = (size_t)256 << 20;   /* workspace per launch of the large-k row kernel */
constexpr int kLsdWords = 256 + 16 * 256 + 16;            /* select_top_k_global's LDS words */

size_t r16(size_t b) { return (b + 15) & ~(size_t)15; }

int pow2_at_least(int v, int lo) {
    int p = lo;
    while (p < v) p <<= 1;
    return p;
}

size_t aggs_bytes(int n) {
    size_t nch = ((size_t)n + 63) / 64, ngr = (nch + 63) / 64;
    return 2 * r16(nch * 8) + r16(nch * 4) + 2 * r16(ngr * 8) + r16(ngr * 4) + r16((nch + 1) * 8);
}

/* Smallest double d with (float)d >= tp, for tp > 0 finite: the boundary of the
 * test (float)cumul >= top_p (src/sampler.c:211). */
double topp_threshold(float tp) {
    float lo = nextafterf(tp, 0.0f);
    double mid = ((double)lo + (double)tp) * 0.5;
    if ((float)mid >= tp) return mid;
    return nextafter(mid, INFINITY);
}

/* ---- workspace --------------------------------------------------------------
 * Device scratch of the kernels, one lazily grown buffer per (device, stream,
 * kind): kernels queued on one stream run in order, so they may share it, and
 * calls on different streams never do.  Kind 0 starts with a counter region
 * that is zero between launches (each launch returns its counters to zero),
 * then scratch; kind 1 holds the prepared logits of dlk_sample's pre-pass.
 * g_mu guards the table and is held by each entry point from its first
 * workspace() through its last launch, so no buffer is regrown (freed) between
 * the moment a call takes its pointers and the moment its kernels are queued. */
struct WsBuf {
    int dev;
    hipStream_t stream;
    int kind;
    void *ptr;
    size_t ctr_cap;      /* counter words */
    size_t data_bytes;   /* scratch bytes after the counters */
};
std::mutex g_mu;
std::vector<WsBuf> g_ws;

struct WsView {
    uint32_t *counters;
    unsigned char *data;
};

/* ---- the no-allocation entry point's scratch ----------------------------------
 * dlk_sample_noalloc takes its workspace from this fixed array instead: every
 * device the library runs on holds one copy of it until the process ends.  The
 * first kScratchCtrWords words are the counter region, the rest is scratch.  In
 * host code `scratch` names a host-side stand-in, never the device memory: the
 * device address comes from hipGetSymbolAddress, once per device, with that
 * device current (scratch_ptr), and only that address is handed to kernels. */
constexpr size_t kScratchBytes = (size_t)DLK_NOALLOC_SCRATCH_BYTES;
constexpr size_t kScratchCtrWords = (size_t)1 << 16;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
unsigned char *g_scratch_dev[64];     /* per device: the address of its copy */
bool g_noalloc = false;               /* set (under g_mu) for a dlk_sample_noalloc call */
int g_ws_err = DLK_ERR_HIP;           /* why the last workspace() failed */

__global__ void zero_words_kernel(uint32_t *p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

unsigned char *scratch_ptr() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    if (!g_scratch_dev[dev]) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) return nullptr;
        g_scratch_dev[dev] = (unsigned char *)ptr;
    }
    return g_scratch_dev[dev];
}

/* The no-allocation workspace: the scratch array, its counter words this call
 * uses cleared by a fill kernel on the call's stream (a kernel, not a memset
 * node, so that the call may be captured into a graph). */
bool workspace_noalloc(hipStream_t stream, int kind, size_t counters, size_t data_bytes, WsView &out) {
    g_ws_err = DLK_ERR_UNSUPPORTED;
    if (kind != 0 || counters > kScratchCtrWords || data_bytes > kScratchBytes - kScratchCtrWords * 4) return false;
    unsigned char *base = scratch_ptr();
    g_ws_err = DLK_ERR_HIP;
    if (!base) return false;
    if (counters > 0) {
        unsigned blocks = (unsigned)((counters + 255) / 256);
        if (blocks > 1024) blocks = 1024;
        hipLaunchKernelGGL(zero_words_kernel, dim3(blocks), dim3(256), 0, stream, (uint32_t *)base, counters);
        if (hipGetLastError() != hipSuccess) return false;
    }
    out.counters = (uint32_t *)base;
    out.data = base + kScratchCtrWords * 4;
    return true;
}

bool workspace(hipStream_t stream, int kind, size_t counters, size_t data_bytes, WsView &out) {
    if (g_noalloc) return workspace_noalloc(stream, kind, counters, data_bytes, out);
    g_ws_err = DLK_ERR_HIP;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    WsBuf *w = nullptr;
    for (auto &e : g_ws)
        if (e.dev == dev && e.stream == stream && e.kind == kind) { w = &e; break; }
    if (!w) {
        g_ws.push_back(WsBuf{dev, stream, kind, nullptr, 0, 0});
        w = &g_ws.back();
    }
    if (w->ctr_cap < counters || w->data_bytes < data_bytes) {
        size_t cc = w->ctr_cap > counters ? w->ctr_cap : counters;
        if (kind == 0 && cc < 4096) cc = 4096;
        cc = (cc + 63) & ~(size_t)63;
        size_t db = w->data_bytes > data_bytes ? w->data_bytes : data_bytes;
        if (db < (1u << 20)) db = 1u << 20;
        if (w->ptr) {
            /* the stream's earlier kernels may still use the old buffer */
            if (hipStreamSynchronize(stream) != hipSuccess) return false;
            (void)hipFree(w->ptr);
            w->ptr = nullptr;
            w->ctr_cap = w->data_bytes = 0;
        }
        if (hipMalloc(&w->ptr, cc * 4 + db) != hipSuccess) { w->ptr = nullptr; return false; }
        if (cc > 0 && hipMemset(w->ptr, 0, cc * 4) != hipSuccess) return false;
        w->ctr_cap = cc;
        w->data_bytes = db;
    }
    out.counters = (uint32_t *)w->ptr;
    out.data = (unsigned char *)w->ptr + w->ctr_cap * 4;
    return true;
}

size_t fixed_lds(const dlk::LdsPlan &pl) {
    return r16(32 * 8) + r16(64 * 8) + r16(16 * 8) + r16(64 * 4) + 4 * r16((size_t)pl.hcap * 4) +
           r16((size_t)pl.flag_words * 4);
}

/* The parameter block for rows r0.. of the batch: every per-row pointer moved on. */
dlk::RowParams rows_from(const dlk::RowParams &p, int r0) {
    dlk::RowParams q = p;
    q.logits = p.logits + (int64_t)r0 * p.ld;
    if (p.hist_off) q.hist_off = p.hist_off + r0;
    if (p.mask) {
        if (p.mask_row) q.mask_row = p.mask_row + r0;
        else q.mask = p.mask + (int64_t)r0 * p.mask_ld;
    }
    if (p.rng) q.rng = p.rng + r0;
    q.out_ids = p.out_ids + r0;
    if (p.out_cand_ids) q.out_cand_ids = p.out_cand_ids + (int64_t)r0 * p.n_out;
    if (p.out_cand_probs) q.out_cand_probs = p.out_cand_probs + (int64_t)r0 * p.n_out;
    if (p.out_cand_logprobs) q.out_cand_logprobs = p.out_cand_logprobs + (int64_t)r0 * p.n_out;
    return q;
}

/* Single-pass top-k path (sampler_topk.hip): returns DLK_OK, or 1 when the
 * configuration is outside its range (the caller then uses the row kernel). */
int launch_topk(dlk::RowParams &p, int rows, int vocab, hipStream_t stream) {
    using namespace dlk;
    const int T = kTopkThreads;
    if (((uintptr_t)p.logits & 15) != 0 || (p.ld & 3) != 0) return 1;
    const int k = p.greedy ? 1 : p.top_k;
    if (k > kTopkMaxK) return 1;
    if (p.plan.hcap > kTopkHcapMax) return 1;     /* (the host stages longer histories elsewhere) */
    if (p.greedy && p.cap > 0.0f) return 1;
    const int KP = k + 16;
    const int kind = p.cap > 0.0f ? 1 : p.greedy ? 2 : 0;
    const int unit = 16 * T;                          /* slices are whole batches of 4 groups per thread */
    const int gmax = std::min(kTopkMaxG, kMergePerThread * T / KP);
    const int gmin = (vocab + kTopkMaxS - 1) / kTopkMaxS;
    if (gmin > gmax) return 1;
    int cc = 512;
    while (cc < 2 * KP) cc <<= 1;
    /* LDS of a launch with slices of S: the kernel's carve order -- misc, select
     * histogram, merge words, then one region for the slice (penalised-group
     * bits, listed groups and their maxima, candidates) and the merge (entries, pipeline aggregates;
     * the fallback's kp entries + 2048-word histogram) */
    auto lds_for = [&](int S, int G) {
        const int gc = S / 4 < kTopkGroupCap ? S / 4 : kTopkGroupCap;
        const size_t slice_b = r16((size_t)(S / 128) * 4) + 2 * r16((size_t)gc * 4) + r16((size_t)cc * 8);
        const size_t merge_b = r16((size_t)cc * 8) + (p.greedy ? 0 : aggs_bytes(k));
        const size_t fall_b = (size_t)p.plan.kp * 8 + 2048 * 4;
        size_t work = slice_b > merge_b ? slice_b : merge_b;
        if (fall_b > work) work = fall_b;
        return fixed_lds(p.plan) + r16(64 * 4) + r16((size_t)kSelWords * 4) + r16((size_t)(3 * G + 2) * 4) + work;
    };
    /* the most workgroups per row that still run as one resident round (each
     * workgroup's post-stream latency is then paid once), else the fewest */
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return DLK_ERR_HIP;
    static int n_cu[64];
    if (dev < 0 || dev >= 64) return DLK_ERR_HIP;
    if (!n_cu[dev] && hipDeviceGetAttribute(&n_cu[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return DLK_ERR_HIP;
    /* occupancy per (device, kind, LDS): a fixed table, so that no call
     * allocates host memory either (past its size a query is simply repeated) */
    struct Occ { int dev, kind; size_t lds; int n; };
    static Occ occ_cache[256];
    static int n_occ = 0;
    auto resident = [&](size_t lds) {
        for (int i = 0; i < n_occ; i++) {
            const Occ &e = occ_cache[i];
            if (e.dev == dev && e.kind == kind && e.lds == lds) return e.n * n_cu[dev];
        }
        const int n = dlk_topk_kernel_occupancy(kind, lds);
        if (n_occ < 256) occ_cache[n_occ++] = Occ{dev, kind, lds, n};
        return n * n_cu[dev];
    };
    auto slice_of = [&](int g) { return ((vocab + g - 1) / g + unit - 1) / unit * unit; };
    int S = slice_of(gmin);
    for (int g = gmax; g >= gmin; g--) {
        const int s = slice_of(g), gr = (vocab + s - 1) / s;
        if ((int64_t)rows * gr <= resident(lds_for(s, gr))) { S = s; break; }
    }
    const int G = (vocab + S - 1) / S;
    TopkParams f;
    memset(&f, 0, sizeof(f));
    f.p = p;
    f.G = G;
    f.S = S;
    f.KP = KP;
    f.grp_cap = S / 4 < kTopkGroupCap ? S / 4 : kTopkGroupCap;
    f.cand_cap = cc;
    f.buf_cap = cc;
    f.spread = (int64_t)rows * G >= 4 * (int64_t)n_cu[dev] ? 1 : 0;   /* four or more blocks per CU */
    const size_t lds = lds_for(S, G);
    size_t n_slot = r16((size_t)rows * G * sizeof(TopkSlot));
    size_t n_cand = (size_t)rows * G * KP * 8;
    WsView ws;
    if (!workspace(stream, 0, (size_t)rows, n_slot + n_cand, ws)) return g_ws_err;
    f.counters = ws.counters;
    f.slots = (TopkSlot *)ws.data;
    f.cands = (uint64_t *)(ws.data + n_slot);
    return dlk_launch_topk_kernel(&f, rows, lds, stream) == 0 ? DLK_OK : DLK_ERR_HIP;
}

/* Fused full-vocabulary path (sampler_full.hip): DLK_OK, or 1 when outside its
 * range (the caller then uses the row kernel). */
int launch_full(dlk::RowParams &p, int rows, int vocab, int force_exact, int no_wait, hipStream_t stream) {
    using namespace dlk;
    const int T = kFullThreads;
    if (p.greedy || p.topk_on || p.s_general) return 1;
    /* min-p with the cut after the first kept entry (it may lie in any slice): the row kernel */
    if (p.minp_on && p.topp_on && p.top_p <= 0.0f) return 1;
    if (!(p.inv_temp < INFINITY)) return 1;            /* (v - M) * inv_t is NaN at the maximum */
    if (p.plan.hcap > 2 * T) return 1;                 /* one or two history ids per thread, loaded first */
    if (((uintptr_t)p.logits & 15) != 0 || (p.ld & 3) != 0) return 1;
    if (vocab < 8192 || (vocab & 3) != 0) return 1;   /* whole 16-byte groups per row */
    /* about 512 workgroups: two per CU on 256 CUs */
    int G = (512 + rows - 1) / rows;
    if (G > kFullMaxG) G = kFullMaxG;
    if (G < 1) G = 1;
    int ept = (vocab + G * T - 1) / (G * T);
    ept = ept <= 16 ? 16 : ept <= 24 ? 24 : ept <= 32 ? 32 : ept <= 40 ? 40 : 48;
    G = (vocab + ept * T - 1) / (ept * T);
    if (G > kFullMaxG) return 1;
    const int S = ept * T;
    if (p.n_out > S) return 1;
    /* (the no-wait test instance: 24 elements per thread, no soft-cap) */
    if (no_wait && (ept != 24 || p.cap > 0.0f)) return DLK_ERR_UNSUPPORTED;
    const int nch = S / 64;
    FullParams f;
    memset(&f, 0, sizeof(f));
    f.G = G;
    f.S = S;
    f.force_exact = force_exact;
    f.no_wait = no_wait;
    /* carve order of full_kernel: sbits, ce, cbh, ca, rtot, rend, rpre, Pc, smap, svals, spx, elist, elc, seg,
     * tab, tbase, rres, rbase, pc, misc, md; 48 chunks staged per workgroup (sharp rows stage many: every
     * chunk with a tie and those around r's crossing) */
    auto lds_for = [&](int stage_cap) {
        return fixed_lds(p.plan) + r16((size_t)(S / 32) * 4) + r16((size_t)(nch + 1) * 8) +
               2 * r16((size_t)nch * 4) + r16((size_t)nch * 8) + r16((size_t)nch * 4) + r16((size_t)nch * 8) +
               r16((size_t)(nch + 1) * 8) + r16((size_t)nch * 4) + 2 * r16((size_t)stage_cap * 64 * 4) +
               r16((size_t)nch * 8) + r16((size_t)nch * 4) + r16((size_t)nch * 16) + r16((size_t)kMaxTabs * 64 * 8) +
               r16((size_t)kMaxTabs * 4) + r16((size_t)(kFullThreads / 64) * 64 * 8) +
               r16((size_t)(kFullThreads / 64) * 4) + r16((size_t)G * kPubWords * 8) + r16(64 * 4) + r16(16 * 8);
    };
    f.stage_cap = 48;
    const size_t lds = lds_for(f.stage_cap);
    if (lds > kMaxLds) return 1;
    /* resident workgroups of this instance: queried once per (device, ept, LDS, instance) */
    struct CapEntry { int dev, ept; size_t lds; int softcap, hp, cap; };
    static CapEntry cap_cache[256];       /* fixed, as occ_cache above */
    static int n_cap = 0;
    const int softcap = p.cap > 0.0f ? 1 : 0;
    const int hp = p.plan.hcap > kFullThreads ? 2 : 1;    /* history ids per thread */
    int dev = 0, cap = -1;
    if (hipGetDevice(&dev) != hipSuccess) return DLK_ERR_HIP;
    for (int i = 0; i < n_cap; i++) {
        const CapEntry &e = cap_cache[i];
        if (e.dev == dev && e.ept == ept && e.lds == lds && e.softcap == softcap && e.hp == hp) { cap = e.cap; break; }
    }
    if (cap < 0) {
        cap = dlk_full_kernel_capacity(ept, lds, softcap, hp);
        if (n_cap < 256) cap_cache[n_cap++] = CapEntry{dev, ept, lds, softcap, hp, cap};
    }
    int rows_per = cap / G;
    if (rows_per < 1) return 1;
    if (rows_per > rows) rows_per = rows;
    /* per row: the fallback's aggregates, then the row's values for the split
     * sums (V) or one slice's for a re-walked draw (S, which may exceed V) */
    const size_t fb_q_off = r16(aggs_bytes(vocab));
    const size_t fb_bytes = fb_q_off + r16((size_t)(vocab > S ? vocab : S) * 4);
    if (g_noalloc) {
        /* the fixed scratch array: as many rows per launch as it holds */
        const size_t room = kScratchBytes - kScratchCtrWords * 4 - 256;
        const size_t per = fb_bytes + (size_t)G * kLaneWords * 8;
        if (room / per < (size_t)rows_per) rows_per = (int)(room / per);
        if (rows_per < 1) return DLK_ERR_UNSUPPORTED;
    }
    const size_t n_ln = r16((size_t)rows_per * G * kLaneWords * 8);
    WsView ws;
    /* the published words live in the zeroed counter region: they are zero
     * between launches (the kernel returns them to zero) */
    if (!workspace(stream, 0, (size_t)rows_per * kSyncWords + (size_t)rows_per * G * kPubWords * 2,
                   n_ln + (size_t)rows_per * fb_bytes, ws))
        return g_ws_err;
    f.sync = ws.counters;
    f.pub = (uint64_t *)(ws.counters + (size_t)rows_per * kSyncWords);
    f.lanes = (uint64_t *)ws.data;
    f.fb = ws.data + n_ln;
    f.fb_bytes = fb_bytes;
    f.fb_q_off = fb_q_off;
    for (int r0 = 0; r0 < rows; r0 += rows_per) {
        const int nr = rows - r0 < rows_per ? rows - r0 : rows_per;
        f.p = rows_from(p, r0);
        if (dlk_launch_full_kernel(&f, nr, ept, lds, stream) != 0) return DLK_ERR_HIP;
    }
    return DLK_OK;
}

/* The row kernel with a top-k too large for LDS: candidates (two buffers for
 * the sort) and the pipeline's aggregates in workspace, rows in chunks. */
int launch_row_global_topk(dlk::RowParams &p, int rows, hipStream_t stream) {
    const int64_t kpad = ((int64_t)p.top_k + 63) & ~(int64_t)63;
    const size_t cand_bytes = (size_t)kpad * 2 * 8;
    const size_t reg_bytes = r16(aggs_bytes(p.top_k));
    const size_t per_row = cand_bytes + reg_bytes;
    const size_t budget = g_noalloc ? kScratchBytes - kScratchCtrWords * 4 : kGlobalTopkBudget;
    int rows_per = (int)(budget / per_row);
    if (rows_per < 1) rows_per = 1;
    if (rows_per > rows) rows_per = rows;
    WsView ws;
    if (!workspace(stream, 0, 0, (size_t)rows_per * per_row, ws)) return g_ws_err;
    p.gcand = (uint64_t *)ws.data;
    p.gcand_stride = kpad * 2;
    p.gregion = ws.data + (size_t)rows_per * cand_bytes;
    p.gregion_stride = (int64_t)reg_bytes;
    const size_t total = fixed_lds(p.plan) + r16(2048 * 4) + r16((size_t)kLsdWords * 4);
    if (total > kMaxLds) return DLK_ERR_UNSUPPORTED;
    p.plan.bytes = (int)total;
    for (int r0 = 0; r0 < rows; r0 += rows_per) {
        const int nr = rows - r0 < rows_per ? rows - r0 : rows_per;
        dlk::RowParams q = rows_from(p, r0);
        if (dlk_launch_row_kernel(&q, nr, total, stream) != 0) return DLK_ERR_HIP;
    }
    return DLK_OK;
}

int sample_impl(const dlk_batch *b, int rows, int vocab, const dlk_sample_params *prm, hipStream_t stream) {
    if (!b || !prm || rows <= 0 || vocab <= 0 || !b->logits || !b->out_ids || b->ld < vocab) return DLK_ERR_INVALID;
    if (prm->n_out < 0) return DLK_ERR_INVALID;
    if ((b->hist_off == nullptr) != (b->hist_ids == nullptr)) return DLK_ERR_INVALID;
    if (b->mask && b->mask_ld < (vocab + 31) / 32) return DLK_ERR_INVALID;
    const bool greedy = prm->temperature == 0.0f;               /* src/sampler.c:140 */
    if (!greedy && !b->rng) return DLK_ERR_INVALID;
    const int max_hist = prm->max_history > 0 ? prm->max_history : 1024;
    const bool cap_on = prm->softcap > 0.0f;                    /* src/core/context.c:604 */
    if (b->hist_off && pow2_at_least(max_hist, 64) > kHcapDirect) {
        /* a history too long to stage in LDS: the rows as sampler_sample would
         * see them -- soft-cap, mask, penalties (src/core/sampler_api.c:51-61) --
         * in a scratch copy; then the sampling alone over the copy.  A row whose
         * history exceeds max_history is flagged by the penalty pass (its rng
         * state kept) and given id -1 and the status bit after the sampling,
         * as the sampling kernels do for the histories they stage */
        if (rows > 65535) return DLK_ERR_UNSUPPORTED;
        const int64_t ldp = ((int64_t)vocab + 63) & ~(int64_t)63;
        const size_t prep_b = r16((size_t)rows * ldp * 4), flag_b = r16((size_t)rows * 4);
        WsView ws;
        if (!workspace(stream, 1, 0, prep_b + flag_b + (size_t)rows * 8, ws)) return g_ws_err;
        float *prep = (float *)ws.data;
        int32_t *too_long = (int32_t *)(ws.data + prep_b);
        uint64_t *rng_saved = (uint64_t *)(ws.data + prep_b + flag_b);
        if (dlk_launch_prepare_rows(b->logits, b->ld, prep, ldp, rows, vocab, b->mask, b->mask_ld, b->mask_row,
                                    cap_on ? prm->softcap : 0.0f, stream) != 0)
            return DLK_ERR_HIP;
        int rc = dlk_launch_long_history_penalties(prep, ldp, rows, vocab, b->hist_off, b->hist_ids,
                                                   prm->penalty_order, prm->repeat_penalty, prm->frequency_penalty,
                                                   prm->presence_penalty, max_hist, too_long,
                                                   greedy ? nullptr : b->rng, rng_saved, stream);
        if (rc != DLK_OK) return rc;
        dlk_batch b2 = *b;
        b2.logits = prep;
        b2.ld = ldp;
        b2.hist_off = b2.hist_ids = nullptr;
        b2.mask = nullptr;
        b2.mask_row = nullptr;
        b2.mask_ld = 0;
        dlk_sample_params p2 = *prm;
        p2.softcap = 0.0f;
        p2.max_history = 0;
        rc = sample_impl(&b2, rows, vocab, &p2, stream);
        if (rc != DLK_OK) return rc;
        return dlk_launch_long_history_fixup(rows, too_long, rng_saved, greedy ? nullptr : b->rng, b->out_ids,
                                             b->status, stream);
    }

    dlk::RowParams p;
    memset(&p, 0, sizeof(p));
    p.logits = b->logits; p.ld = b->ld; p.V = vocab;
    p.hist_off = b->hist_off; p.hist_ids = b->hist_ids;
    p.mask = b->mask; p.mask_ld = b->mask_ld; p.mask_row = b->mask_row;
    p.rng = b->rng; p.out_ids = b->out_ids;
    p.out_cand_ids = b->out_cand_ids; p.out_cand_probs = b->out_cand_probs; p.out_cand_logprobs = b->out_cand_logprobs;
    p.n_out = prm->n_out; p.status = b->status;
    p.top_p = prm->top_p; p.min_p = prm->min_p;
    p.rep = prm->repeat_penalty; p.freq = prm->frequency_penalty; p.pres = prm->presence_penalty;
    p.order = prm->penalty_order;
    p.greedy = greedy;
    p.cap = cap_on ? prm->softcap : 0.0f;          /* applied inside the sampling kernels */
    if (!p.greedy) {
        p.inv_temp = 1.0f / prm->temperature;                   /* src/sampler.c:154 */
        /* 1/T negative, zero or infinite: s = (l - max) * (1/T) may be NaN or +inf
         * and its maximum is not 0; the row kernel handles it */
        p.s_general = !(p.inv_temp > 0.0f && p.inv_temp < INFINITY);
    }
    p.topk_on = prm->top_k > 0 && prm->top_k < vocab;           /* src/sampler.c:166 */
    p.top_k = prm->top_k;
    p.topp_on = prm->top_p < 1.0f;                              /* src/sampler.c:205 */
    p.topp_thr = (p.topp_on && prm->top_p > 0.0f) ? topp_threshold(prm->top_p) : 0.0;
    p.minp_on = prm->min_p > 0.0f;                              /* src/sampler.c:188 */

    dlk::LdsPlan &pl = p.plan;
    pl.hcap = b->hist_off ? pow2_at_least(max_hist, 64) : 64;
    int nch = (vocab + 63) / 64;
    pl.flag_words = (nch + 31) / 32;
    const bool big_k = p.topk_on && !p.greedy && p.top_k > kMaxTopKLds;
    pl.kp = p.topk_on && !big_k ? pow2_at_least(p.top_k, 64) : 0;
    if (big_k) return launch_row_global_topk(p, rows, stream);
    size_t fixed = fixed_lds(pl);
    size_t region = 0;
    if (!p.greedy) {
        if (p.topk_on) region = r16((size_t)pl.kp * 8) + (aggs_bytes(p.top_k) > 8192 ? aggs_bytes(p.top_k) : 8192);
        else region = aggs_bytes(vocab);
    }
    size_t total = fixed + region;
    /* (greedy under a cap: the row kernel, whose argmax is taken on the capped row) */
    if (prm->path == DLK_PATH_AUTO && (p.greedy || p.topk_on) && !p.s_general && !(p.greedy && cap_on)) {
        int rc = launch_topk(p, rows, vocab, stream);
        if (rc <= 0) return rc;
    }
    if ((prm->path == DLK_PATH_AUTO || prm->path == DLK_PATH_FULL_EXACT || prm->path == DLK_PATH_FULL_NO_WAIT) &&
        !p.greedy && !p.topk_on) {
        int rc = launch_full(p, rows, vocab, prm->path == DLK_PATH_FULL_EXACT, prm->path == DLK_PATH_FULL_NO_WAIT,
                             stream);
        if (rc <= 0) return rc;
    }
    if (total > kMaxLds) return DLK_ERR_UNSUPPORTED;
    pl.bytes = (int)total;
    return dlk_launch_row_kernel(&p, rows, total, stream) == 0 ? DLK_OK : DLK_ERR_HIP;
}

}  // namespace

extern "C" uint64_t dlk_seed_state(uint64_t seed) { return seed ? seed : 0xDEADBEEF12345678ULL; }

extern "C" int dlk_sample(const dlk_batch *b, int rows, int vocab, const dlk_sample_params *prm,
                          hipStream_t stream) {
    std::lock_guard<std::mutex> lock(g_mu);
    return sample_impl(b, rows, vocab, prm, stream);
}

/* Frees the workspace buffers of `stream` on the current device, after the
 * stream's queued work has finished with them (include/diskllm_amd.h). */
extern "C" int dlk_release_stream(hipStream_t stream) {
    std::lock_guard<std::mutex> lock(g_mu);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return DLK_ERR_HIP;
    int rc = DLK_OK;
    bool synced = false;
    for (size_t i = 0; i < g_ws.size();) {
        if (g_ws[i].dev == dev && g_ws[i].stream == stream) {
            if (!synced) {
                if (hipStreamSynchronize(stream) != hipSuccess) rc = DLK_ERR_HIP;
                synced = true;
            }
            if (g_ws[i].ptr && hipFree(g_ws[i].ptr) != hipSuccess) rc = DLK_ERR_HIP;
            g_ws.erase(g_ws.begin() + (long)i);
        } else {
            i++;
        }
    }
    return rc;
}

/* dlk_sample with its workspace in the fixed per-device scratch array: no
 * allocation of any kind.  The scratch is shared by every call on the device,
 * so calls that overlap on one device race. */
extern "C" int dlk_sample_noalloc(const dlk_batch *b, int rows, int vocab, const dlk_sample_params *prm,
                                  hipStream_t stream) {
    std::lock_guard<std::mutex> lock(g_mu);
    g_noalloc = true;
    const int rc = sample_impl(b, rows, vocab, prm, stream);
    g_noalloc = false;
    return rc;
}
