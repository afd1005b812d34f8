/*
 * penalties.hip -- repetition / frequency / presence penalties in place on device
 * logits (src/sampler.c:21-52 and the frequency form of the batched path).
 *
 * One workgroup per row.  The row's history is counted in an LDS hash table of
 * its in-range ids (open addressing, one compare-and-swap per entry); the
 * thread that finds an occupied slot after the counts are in applies the ops
 * for that id with its count, so no two threads touch one logit.  A penalty
 * depends only on the id's count (repetition acts once per occurrence and never
 * changes the sign, presence and frequency once per distinct id), not on where
 * the occurrences lie.  A history with more distinct ids than the table holds
 * is counted by a scan instead (O(n^2) per row).
 *
 * The same kernel serves dlk_sample's long-history pre-pass: there a row whose
 * history exceeds max_history is flagged and left alone, and a second kernel
 * after the sampling gives such a row id -1, DLK_STATUS_HISTORY_TOO_LONG and its
 * rng state from before the call, as the sampling kernels do for the histories
 * they stage themselves.
 */
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../../include/diskllm_amd.h"

namespace dlk {

constexpr int kPenThreads = 1024;
constexpr int kPenMaxSlots = 16384;    /* LDS hash slots (key + count: 128 KiB) */

__device__ __forceinline__ float penalize_ops(float x, int cnt, uint32_t order, float rep, float freq, float pres) {
    for (int s = 0; s < 8; s++) {
        const uint32_t op = (order >> (4 * s)) & 0xFu;
        if (op == 0) break;
        if (op == DLK_OP_REPETITION) {
            if (rep > 1.0f)
                for (int k = 0; k < cnt; k++) x = x < 0.0f ? x * rep : x / rep;
        } else if (op == DLK_OP_FREQUENCY) {
            if (freq != 0.0f) { const float d = freq * (float)cnt; x = x - d; }
        } else if (op == DLK_OP_PRESENCE) {
            if (pres != 0.0f) x = x - pres;
        }
    }
    return x;
}

/* slots: a power of two <= kPenMaxSlots (dynamic LDS of 8 * slots bytes).
 * max_hist >= 0: rows with more history entries are flagged in too_long[row]
 * (their rng state saved) and not penalised. */
__global__ __launch_bounds__(kPenThreads) void penalties_kernel(float *logits, int64_t ld, int V,
                                                                const int32_t *hist_off, const int32_t *hist_ids,
                                                                uint32_t order, float rep, float freq, float pres,
                                                                int slots, int max_hist, int32_t *too_long,
                                                                const uint64_t *rng, uint64_t *rng_saved) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int full;
    int *key = (int *)smem;
    uint32_t *cnt = (uint32_t *)(smem + (size_t)slots * 4);
    const int row = blockIdx.x, t = threadIdx.x;
    const int32_t *hr = hist_ids + hist_off[row];
    const int n = hist_off[row + 1] - hist_off[row];
    if (max_hist >= 0) {
        const bool over = n > max_hist;
        if (t == 0) {
            too_long[row] = over ? 1 : 0;
            if (over && rng) rng_saved[row] = rng[row];
        }
        if (over) return;
    }
    if (n <= 0) return;
    float *lr = logits + (int64_t)row * ld;
    for (int i = t; i < slots; i += kPenThreads) { key[i] = -1; cnt[i] = 0u; }
    if (t == 0) full = 0;
    __syncthreads();
    const uint32_t mask = (uint32_t)slots - 1u;
    const int shift = 32 - (31 - __clz(slots));
    for (int i = t; i < n; i += kPenThreads) {
        const int32_t id = hr[i];
        if (id < 0 || id >= V) continue;
        uint32_t h = slots > 1 ? ((uint32_t)id * 0x9E3779B1u) >> shift : 0u;
        bool placed = false;
        for (int probe = 0; probe < slots; probe++) {
            const int old = atomicCAS(&key[h], -1, id);
            if (old == -1 || old == id) {
                atomicAdd(&cnt[h], 1u);
                placed = true;
                break;
            }
            h = (h + 1u) & mask;
        }
        if (!placed) full = 1;
    }
    __syncthreads();
    if (!full) {
        for (int h = t; h < slots; h += kPenThreads) {
            const int id = key[h];
            if (id >= 0) lr[id] = penalize_ops(lr[id], (int)cnt[h], order, rep, freq, pres);
        }
        return;
    }
    /* more distinct ids than slots: the thread of an id's first occurrence
     * counts its occurrences */
    for (int i = t; i < n; i += kPenThreads) {
        const int32_t id = hr[i];
        if (id < 0 || id >= V) continue;
        bool first = true;
        for (int j = 0; j < i && first; j++) first = hr[j] != id;
        if (!first) continue;
        int c = 1;
        for (int j = i + 1; j < n; j++) c += hr[j] == id;
        lr[id] = penalize_ops(lr[id], c, order, rep, freq, pres);
    }
}

/* After the sampling of a long-history call: the flagged rows get id -1, the
 * status bit and their rng state back (the sampling drew for them). */
__global__ void long_history_fixup_kernel(int rows, const int32_t *too_long, const uint64_t *rng_saved,
                                          uint64_t *rng, int32_t *out_ids, uint32_t *status) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows || !too_long[r]) return;
    out_ids[r] = -1;
    if (rng) rng[r] = rng_saved[r];
    if (status) atomicOr(status, DLK_STATUS_HISTORY_TOO_LONG);
}

/* Hash slots for the longest history a launch may meet: at least twice the
 * entries (short probes), at most kPenMaxSlots. */
inline int pen_slots(int max_entries) {
    int s = 64;
    while (s < 2 * max_entries && s < kPenMaxSlots) s <<= 1;
    return s;
}

inline int launch_penalties(float *logits, int64_t ld, int rows, int vocab, const int32_t *hist_off,
                            const int32_t *hist_ids, uint32_t order, float rep, float freq, float pres, int slots,
                            int max_hist, int32_t *too_long, const uint64_t *rng, uint64_t *rng_saved,
                            hipStream_t stream) {
    static std::once_flag once;
    static hipError_t attr = hipSuccess;
    std::call_once(once, [] {
        attr = hipFuncSetAttribute((const void *)penalties_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                   kPenMaxSlots * 8);
    });
    if (attr != hipSuccess) return DLK_ERR_HIP;
    hipLaunchKernelGGL(penalties_kernel, dim3(rows), dim3(kPenThreads), (size_t)slots * 8, stream, logits, ld, vocab,
                       hist_off, hist_ids, order, rep, freq, pres, slots, max_hist, too_long, rng, rng_saved);
    return hipGetLastError() == hipSuccess ? DLK_OK : DLK_ERR_HIP;
}

}  // namespace dlk

extern "C" int dlk_apply_penalties(float *logits, int64_t ld, int rows, int vocab, const int32_t *hist_off,
                                   const int32_t *hist_ids, uint32_t order, float rep, float freq, float pres,
                                   hipStream_t stream) {
    if (!logits || rows < 0 || vocab <= 0 || ld < vocab) return DLK_ERR_INVALID;
    if (rows == 0 || !hist_off) return DLK_OK;
    if (!hist_ids) return DLK_ERR_INVALID;
    /* the history lengths live on the device: the table is sized for the most
     * distinct ids LDS holds, and a row with more falls back to the scan */
    return dlk::launch_penalties(logits, ld, rows, vocab, hist_off, hist_ids, order, rep, freq, pres,
                                 dlk::kPenMaxSlots, -1, nullptr, nullptr, nullptr, stream);
}

/* dlk_sample's long-history pre-pass (capi.hip): penalties in place on the
 * prepared copy, rows over max_hist flagged in too_long with their rng state
 * saved; then, after the sampling, the fix-up of the flagged rows. */
extern "C" int dlk_launch_long_history_penalties(float *logits, int64_t ld, int rows, int vocab,
                                                 const int32_t *hist_off, const int32_t *hist_ids, uint32_t order,
                                                 float rep, float freq, float pres, int max_hist, int32_t *too_long,
                                                 const uint64_t *rng, uint64_t *rng_saved, hipStream_t stream) {
    return dlk::launch_penalties(logits, ld, rows, vocab, hist_off, hist_ids, order, rep, freq, pres,
                                 dlk::pen_slots(max_hist), max_hist, too_long, rng, rng_saved, stream);
}

extern "C" int dlk_launch_long_history_fixup(int rows, const int32_t *too_long, const uint64_t *rng_saved,
                                             uint64_t *rng, int32_t *out_ids, uint32_t *status, hipStream_t stream) {
    hipLaunchKernelGGL(dlk::long_history_fixup_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream,
                       rows, too_long, rng_saved, rng, out_ids, status);
    return hipGetLastError() == hipSuccess ? DLK_OK : DLK_ERR_HIP;
}
