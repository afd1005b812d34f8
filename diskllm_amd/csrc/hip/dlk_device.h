/*
 * dlk_device.h -- device helpers shared by the sampling kernels (gfx950, wave64).
 */
#ifndef DLK_DEVICE_H
#define DLK_DEVICE_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "expf_glibc.h"

#define DLK_DEV __device__ __forceinline__

namespace dlk {

constexpr int kWave = 64;

DLK_DEV int lane_id() { return __lane_id(); }
DLK_DEV int wave_id() { return threadIdx.x >> 6; }
DLK_DEV int n_waves() { return blockDim.x >> 6; }

DLK_DEV uint32_t f2u(float f) { return __float_as_uint(f); }
DLK_DEV float u2f(uint32_t u) { return __uint_as_float(u); }
DLK_DEV uint64_t d2u(double d) { return (uint64_t)__double_as_longlong(d); }
DLK_DEV double u2d(uint64_t u) { return __longlong_as_double((long long)u); }

DLK_DEV uint64_t ballot(bool p) { return __ballot(p); }
DLK_DEV int first_lane(uint64_t m) { return m ? __builtin_ctzll(m) : 64; }

template <class T>
DLK_DEV T shfl(T v, int src) { return __shfl(v, src, 64); }
template <class T>
DLK_DEV T shfl_up(T v, int d) { return __shfl_up(v, (unsigned)d, 64); }
template <class T>
DLK_DEV T shfl_xor(T v, int m) { return __shfl_xor(v, m, 64); }

/* Orderable descending key of a float: ascending key <=> descending value, with
 * -0 and +0 made equal (C's '<' treats them as equal, src/sampler.c:114,:122). */
DLK_DEV uint32_t desc_key(float s) {
    uint32_t u = f2u(s);
    if (u == 0x80000000u) u = 0;
    uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ~ord;
}
DLK_DEV float key_value(uint32_t key) {
    uint32_t ord = ~key;
    return u2f((ord & 0x80000000u) ? (ord & 0x7fffffffu) : ~ord);
}

/* Round-to-nearest-even conversion of an integer v < 2^53 to float, written out
 * so it does not depend on the compiler's u64->f32 lowering. */
DLK_DEV float u53_to_f32_rn(uint64_t v) {
    if (v == 0) return 0.0f;
    int msb = 63 - __clzll((long long)v);
    if (msb <= 23) return (float)(uint32_t)v;
    int sh = msb - 23;
    uint64_t mant = v >> sh;
    uint64_t rem = v & ((1ull << sh) - 1);
    uint64_t half = 1ull << (sh - 1);
    if (rem > half || (rem == half && (mant & 1))) mant++;
    return ldexpf((float)(uint32_t)mant, sh);
}

/* xorshift64 + rand_f32, src/sampler.c:69-81. */
DLK_DEV uint64_t xorshift64(uint64_t x) {
    x ^= x << 13;
    x ^= x >> 7;
    x ^= x << 17;
    return x;
}
DLK_DEV float rand_f32_from(uint64_t x) { return u53_to_f32_rn(x >> 11) * (1.0f / 9007199254740992.0f); }

/* DPP controls (gfx9 encoding). */
constexpr int kDppRowShr1 = 0x111, kDppRowShr2 = 0x112, kDppRowShr4 = 0x114, kDppRowShr8 = 0x118;
constexpr int kDppRowBcast15 = 0x142, kDppRowBcast31 = 0x143;

/* Inclusive prefix sum within each 16-lane row (lane 15 holds the row total). */
DLK_DEV uint32_t row_scan_u32(uint32_t x) {
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, kDppRowShr1, 0xf, 0xf, true);
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, kDppRowShr2, 0xf, 0xf, true);
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, kDppRowShr4, 0xf, 0xf, true);
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, kDppRowShr8, 0xf, 0xf, true);
    return x;
}
/* Inclusive prefix sum of floats within each 16-lane row. */
DLK_DEV float row_scan_f(float x) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kDppRowShr1, 0xf, 0xf, true));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kDppRowShr2, 0xf, 0xf, true));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kDppRowShr4, 0xf, 0xf, true));
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), kDppRowShr8, 0xf, 0xf, true));
    return x;
}
template <int CTRL>
DLK_DEV double dpp_row_d(double v) {
    uint64_t u = (uint64_t)__double_as_longlong(v);
    int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xf, 0xf, true);
    int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xf, 0xf, true);
    return __longlong_as_double((long long)(((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo));
}
/* Inclusive prefix sum of doubles within each 16-lane row. */
DLK_DEV double row_scan_d(double x) {
    x += dpp_row_d<kDppRowShr1>(x);
    x += dpp_row_d<kDppRowShr2>(x);
    x += dpp_row_d<kDppRowShr4>(x);
    x += dpp_row_d<kDppRowShr8>(x);
    return x;
}
/* 64-bit lane exchange by DPP: lanes the control leaves without a source (or
 * rows outside row_mask) get `old`. */
template <int CTRL, int ROWS = 0xf, bool BC = true>
DLK_DEV uint64_t dpp_u64(uint64_t v, uint64_t old = 0) {
    const int lo = __builtin_amdgcn_update_dpp((int)(uint32_t)old, (int)(uint32_t)v, CTRL, ROWS, 0xf, BC);
    const int hi = __builtin_amdgcn_update_dpp((int)(uint32_t)(old >> 32), (int)(uint32_t)(v >> 32), CTRL, ROWS, 0xf, BC);
    return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}
/* Inclusive prefix over the 64 lanes by DPP (row shifts, then row broadcasts). */
DLK_DEV double wave_incl_scan_d(double x) {
    x += __longlong_as_double((long long)dpp_u64<kDppRowShr1>((uint64_t)__double_as_longlong(x)));
    x += __longlong_as_double((long long)dpp_u64<kDppRowShr2>((uint64_t)__double_as_longlong(x)));
    x += __longlong_as_double((long long)dpp_u64<kDppRowShr4>((uint64_t)__double_as_longlong(x)));
    x += __longlong_as_double((long long)dpp_u64<kDppRowShr8>((uint64_t)__double_as_longlong(x)));
    x += __longlong_as_double((long long)dpp_u64<kDppRowBcast15, 0xa, false>((uint64_t)__double_as_longlong(x)));
    x += __longlong_as_double((long long)dpp_u64<kDppRowBcast31, 0xc, false>((uint64_t)__double_as_longlong(x)));
    return x;
}
DLK_DEV uint64_t wave_incl_scan_u64(uint64_t x) {
    x += dpp_u64<kDppRowShr1>(x);
    x += dpp_u64<kDppRowShr2>(x);
    x += dpp_u64<kDppRowShr4>(x);
    x += dpp_u64<kDppRowShr8>(x);
    x += dpp_u64<kDppRowBcast15, 0xa, false>(x);
    x += dpp_u64<kDppRowBcast31, 0xc, false>(x);
    return x;
}
/* Maximum over the 64 lanes (every lane gets it). */
DLK_DEV float wave_max_dpp(float v) {
    const int ninf = (int)0xff800000u;
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), kDppRowShr1, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), kDppRowShr2, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), kDppRowShr4, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), kDppRowShr8, 0xf, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), kDppRowBcast15, 0xa, 0xf, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(ninf, __float_as_int(v), kDppRowBcast31, 0xc, 0xf, false)));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
/* Wave-wide minimum and maximum of a u32 (DPP row shifts, then row
 * broadcasts; lanes with no source take the identity). */
template <bool MIN>
DLK_DEV uint32_t wave_minmax_u32(uint32_t v) {
    const int id = MIN ? -1 : 0;
    uint32_t o;
    o = (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, kDppRowShr1, 0xf, 0xf, false); v = MIN ? min(v, o) : max(v, o);
    o = (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, kDppRowShr2, 0xf, 0xf, false); v = MIN ? min(v, o) : max(v, o);
    o = (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, kDppRowShr4, 0xf, 0xf, false); v = MIN ? min(v, o) : max(v, o);
    o = (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, kDppRowShr8, 0xf, 0xf, false); v = MIN ? min(v, o) : max(v, o);
    o = (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, kDppRowBcast15, 0xa, 0xf, false); v = MIN ? min(v, o) : max(v, o);
    o = (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, kDppRowBcast31, 0xc, 0xf, false); v = MIN ? min(v, o) : max(v, o);
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
/* Inclusive wave prefix with saturation at `cap` (values <= cap). */
DLK_DEV uint32_t wave_scan_sat_u32(uint32_t x, uint32_t cap) {
    uint32_t t;
    t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, kDppRowShr1, 0xf, 0xf, true); x = min(x + t, cap);
    t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, kDppRowShr2, 0xf, 0xf, true); x = min(x + t, cap);
    t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, kDppRowShr4, 0xf, 0xf, true); x = min(x + t, cap);
    t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, kDppRowShr8, 0xf, 0xf, true); x = min(x + t, cap);
    t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, kDppRowBcast15, 0xa, 0xf, false); x = min(x + t, cap);
    t = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, kDppRowBcast31, 0xc, 0xf, false); x = min(x + t, cap);
    return x;
}

}  // namespace dlk

/* Branch hints for kernel code layout: a block behind DLK_COLD is taken rarely
 * (or only on request) and is placed after the kernel's main path, which then
 * stays contiguous and small enough for the instruction cache across launches;
 * DLK_HOT marks the usual side of a branch. */
#define DLK_COLD(c) __builtin_expect(!!(c), 0)
#define DLK_HOT(c) __builtin_expect(!!(c), 1)

#endif
