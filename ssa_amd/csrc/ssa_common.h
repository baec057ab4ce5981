// ssa_common.h -- shared device helpers for the gfx950 SparseAttention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ssa_amd.h"

#define SSA_WAVE 64

// ---------------------------------------------------------------- error text
void ssa_set_error(const char *fmt, ...);

#define SSA_CHECK_ARG(cond, ...)                 \
    do {                                         \
        if (!(cond)) {                           \
            ssa_set_error(__VA_ARGS__);          \
            return SSA_E_ARG;                    \
        }                                        \
    } while (0)

// A failed call's error is also taken off the runtime's last-error slot, so
// the caller's next HIP call (torch's included) does not report it again: the
// library reports it once, through its return code and ssa_last_error.
#define SSA_CHECK_HIP(expr)                                                        \
    do {                                                                           \
        hipError_t e_ = (expr);                                                    \
        if (e_ != hipSuccess) {                                                    \
            ssa_set_error("%s failed: %s", #expr, hipGetErrorString(e_));          \
            (void)hipGetLastError();                                               \
            return SSA_E_HIP;                                                      \
        }                                                                          \
    } while (0)

#define SSA_CHECK_LAUNCH() SSA_CHECK_HIP(hipGetLastError())

// ---------------------------------------------------------------- dtypes
// 16-bit storage types as raw bits: bf16 = upper half of an fp32, fp16 = IEEE
// binary16.  Conversions are written out so the numerics are explicit.
struct bf16_t { uint16_t x; };
struct f16_t  { uint16_t x; };

__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(bf16_t v) {
    return __uint_as_float(((uint32_t)v.x) << 16);
}
__device__ __forceinline__ float to_f32(f16_t v) {
    _Float16 h;
    __builtin_memcpy(&h, &v.x, 2);
    return (float)h;
}

// round-to-nearest-even fp32 -> bf16 (NaN kept quiet)
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u) return (uint16_t)((u >> 16) | ((u & 0xffff) ? 0x40 : 0));
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

template <typename T> struct Cvt;
template <> struct Cvt<float> {
    static __device__ __forceinline__ float round(float v) { return v; }
    static __device__ __forceinline__ void store(float *p, float v) { *p = v; }
};
template <> struct Cvt<bf16_t> {
    static __device__ __forceinline__ float round(float v) {
        return __uint_as_float(((uint32_t)f32_to_bf16_bits(v)) << 16);
    }
    static __device__ __forceinline__ void store(bf16_t *p, float v) { p->x = f32_to_bf16_bits(v); }
};
template <> struct Cvt<f16_t> {
    static __device__ __forceinline__ float round(float v) { return (float)(_Float16)v; }
    static __device__ __forceinline__ void store(f16_t *p, float v) {
        _Float16 h = (_Float16)v;
        __builtin_memcpy(&p->x, &h, 2);
    }
};

// ---------------------------------------------------------------- wave ops
__device__ __forceinline__ int lane_id() {
    const unsigned l = __lane_id();
    __builtin_assume(l < SSA_WAVE);
    return (int)l;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, SSA_WAVE);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, SSA_WAVE));
    return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, SSA_WAVE);
    return v;
}

// wave-wide max / min of an unsigned value through DPP row operations
// (quad swaps, row mirrors, row broadcasts 15 and 31), read from lane 63: a
// wave-uniform result with no LDS traffic.  Every lane must be active.
// The moved operand's "old" value is the identity of the operation (lanes of
// rows outside a broadcast's row mask see it), which also lets the compiler
// fold the move into the max / min as a DPP operand.
template <bool MAX>
__device__ __forceinline__ uint32_t wave_reduce_dpp(uint32_t v) {
    constexpr int id = MAX ? 0 : -1;
    auto op = [](uint32_t a, uint32_t b) { return MAX ? (a > b ? a : b) : (a < b ? a : b); };
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0xB1, 0xF, 0xF, false));
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x4E, 0xF, 0xF, false));
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x141, 0xF, 0xF, false));
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x140, 0xF, 0xF, false));
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x142, 0xA, 0xF, false));
    v = op(v, (uint32_t)__builtin_amdgcn_update_dpp(id, (int)v, 0x143, 0xC, 0xF, false));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, SSA_WAVE - 1);
}
__device__ __forceinline__ uint32_t wave_max_u(uint32_t v) { return wave_reduce_dpp<true>(v); }
__device__ __forceinline__ uint32_t wave_min_u(uint32_t v) { return wave_reduce_dpp<false>(v); }

// orders one wavefront's own LDS accesses across its lanes
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ballot over the 64-lane wave
__device__ __forceinline__ uint64_t wave_ballot(bool p) { return __ballot(p); }

// lane predicate from a wave-uniform lane mask (becomes the exec mask itself)
__device__ __forceinline__ bool in_mask(uint64_t m) { return __builtin_amdgcn_inverse_ballot_w64(m); }

// word 3 of a raw buffer resource on gfx950: 32-bit data format, reads past
// num_records return 0
#define SSA_BUF_FLAGS 0x00020000

// wave-uniform mask of lanes [0, L)
__device__ __forceinline__ uint64_t lanes_mask(int L) {
    return L >= 64 ? ~0ull : (L <= 0 ? 0ull : ((1ull << L) - 1ull));
}

// number of set bits of m in lanes below this one
__device__ __forceinline__ int lanes_below(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0));
}

// Swap count of a Hoare partition from its stopper lists: TL[f ..] holds the
// numL left stoppers in ascending position, TR[f ..] the numR right stoppers
// in ascending position; pair k couples the k-th left stopper with the k-th
// right stopper from the end, and the pairs that swap (left one left of the
// right one) are a prefix.  The largest s with TL[f + s - 1] < TR[f + numR - s]
// is found by a 64-ary search: each round the wave tests 64 evenly spaced
// candidates at once and keeps the range between the last true and the first
// false, so the answer takes one or two rounds of parallel LDS reads.  Every
// lane must be active; the result is wave-uniform.
template <typename Pos>
__device__ __forceinline__ int hoare_swap_count(const Pos *TL, const Pos *TR, int f,
                                                int numL, int numR) {
    const int lane = (int)__lane_id();
    int lo = 0, hi = numL < numR ? numL : numR;     // the answer lies in [lo, hi]
    while (hi > lo) {
        const int span = hi - lo;
        // lane j tests lo + ceil(span (j + 1) / 64): non-decreasing, the last is hi,
        // and every value of (lo, hi] appears once span <= 64
        const int mid = lo + (span * (lane + 1) + 63) / 64;
        const bool t = (int)TL[f + mid - 1] < (int)TR[f + numR - mid];
        const int c = __popcll(__ballot(t));        // lanes 0 .. c-1 hold true
        const int nlo = c > 0 ? __builtin_amdgcn_readlane(mid, c - 1) : lo;
        const int nhi = c < 64 ? __builtin_amdgcn_readlane(mid, c < 64 ? c : 63) - 1 : hi;
        lo = nlo;
        hi = nhi;
    }
    return lo;
}

// Bucket id and probe ids of one row from its P <= 12 hyperplane projections
// pr[0..P-1] (sparse_attention.py:559-646): bit j = pr[j] > 0 (+0, -0 and NaN
// give 0), id = sum of bit j << j; probe t flips, in the base id, the plane
// with the t-th smallest |pr| in the order of a stable ascending argsort
// (ties by plane index, NaN after every number).  Writes o[0] = id and
// o[1 + t] for t < Tp.  The projections are read into registers once and each
// probe picks its plane in one pass over them: O(P) per probe.
__device__ __forceinline__ bool abs_before(float a, int ja, float b, int jb) {
    // |a| before |b| in a stable ascending sort (a, b already absolute)
    if (a != a) return (b != b) && ja < jb;
    return (b != b) || a < b || (a == b && ja < jb);
}
__device__ __forceinline__ void ssa_write_ids(const float *pr, int P, int Tp, uint16_t *o) {
    float v[12];
#pragma unroll
    for (int j = 0; j < 12; ++j) v[j] = j < P ? pr[j] : 0.f;
    int id = 0;
#pragma unroll
    for (int j = 0; j < 12; ++j)
        if (j < P && v[j] > 0.f) id |= 1 << j;
    o[0] = (uint16_t)id;
    int picked = 0;
    for (int t = 0; t < Tp; ++t) {
        int pos = -1;
        float best = 0.f;
#pragma unroll
        for (int j = 0; j < 12; ++j) {
            const float a = fabsf(v[j]);
            if (j < P && !((picked >> j) & 1) && (pos < 0 || abs_before(a, j, best, pos))) {
                best = a;
                pos = j;
            }
        }
        picked |= 1 << pos;
        o[1 + t] = (uint16_t)(id ^ (1 << pos));
    }
}

// order-preserving map fp32 -> uint32 (larger float -> larger key); all
// finite values and +/-inf map above 0, so 0 can mark "no score".
__device__ __forceinline__ uint32_t score_key(float f) {
    // -0 and +0 compare equal (one key); every NaN ranks above +inf, as the
    // top-k comparator "NaN first, then >" orders them
    if (f != f) return 0xffffffffu;
    const uint32_t u = __float_as_uint(f == 0.f ? 0.f : f);
    const uint32_t k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return k == 0 ? 1u : k;
}
// 16-bit score code: a monotone map of the score onto [0, 65535], with
// `scale` taking +-(a bound of the query's scores) to the ends of the range and
// NaN above everything.  Monotone (fma, clamp and truncation all are), so a
// larger code means a larger score and equal scores share a code; scores that
// share a code are told apart by their exact keys.  The code is 65535 minus
// the clamped, truncated -s * scale + 32767: fmaxf(NaN, 0) is 0, so a NaN
// score gets 65535 with no test of its own (the clamp is one v_med3_f32).
__device__ __forceinline__ uint32_t score_neg_code(float s, float scale) {
    return (uint32_t)fminf(fmaxf(fmaf(-s, scale, 32767.f), 0.f), 65535.f);
}
__device__ __forceinline__ uint32_t score_code(float s, float scale) {
    return 65535u - score_neg_code(s, scale);
}
// scale of a query with |q|^2 = q2 against keys with max |k|^2 = k2: every
// score q.k lies within +-sqrt(q2 k2), which maps onto +-32767 (any positive
// scale is correct, only how often codes tie depends on it)
__device__ __forceinline__ float code_scale(float q2, float k2) {
    const float sc = 32767.f / (sqrtf(q2) * sqrtf(k2));
    return (sc > 0.f && sc < 3.0e38f) ? sc : 1.f;
}
__device__ __forceinline__ float key_score(uint32_t k) {
    uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(u);
}

__host__ __device__ __forceinline__ int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Head dims the kernels take: 4..256, whole vectors of the element type (8
// elements of a 16-bit type, 4 of fp32: rows are read in 16-byte pieces) or a
// power of two.  A kernel instance for head dim D serves every d <= D: lanes
// and elements past d read zeros and store nothing.
inline bool ssa_head_dim_ok(int d, int dtype) {
    const int vec = dtype == SSA_F32 ? 4 : 8;
    return d >= 4 && d <= 1024 && ((d & (d - 1)) == 0 || d % vec == 0);
}
// the smallest power-of-two instance (4..1024) that covers d
inline int ssa_pow2_instance(int d) {
    int D = 4;
    while (D < d) D <<= 1;
    return D;
}

// XCD-aware block order: the dispatcher sends workgroup i to XCD i % 8.  Map
// physical block id -> logical id so that each XCD walks one contiguous range
// of logical blocks (consecutive logical blocks share K/V rows in L2).
__device__ __forceinline__ int64_t xcd_logical_block(int64_t phys, int64_t nlogical) {
    const int64_t per = (nlogical + 7) / 8;
    return (phys % 8) * per + phys / 8;
}
