// ssa_apply.hip -- gather attention over a fixed neighbor graph (gfx950).
//
// Replaces sparse_gather_attention (sparse_attention.py:1096-1199).
//
// One wavefront per query row (b, h, n).  The row's neighbour ids are staged
// once in LDS as int32.  A row of d elements is covered by LPR lanes with
// 16-byte loads, so one load instruction brings RPI = 64/LPR whole K (or V)
// rows; with U rows in flight per lane the wave keeps U*RPI*row_bytes of
// gathers outstanding.  Scores go to LDS, the fp32 softmax is a wave
// reduction that turns them into the weights p in place (one exp per slot),
// and P.V accumulates in fp32 registers, reduced across the RPI row groups at
// the end.
//
// Numerics follow the reference: s = fp32(q.k) * fp32(scale); -inf where
// !valid; p = exp(s - max) / sum in fp32; 16-bit models round p to the value
// dtype before P.V (fp32_attn_weights keeps it fp32); P.V accumulates in fp32
// and is rounded once to the output dtype.
#include <type_traits>

#include "ssa_common.h"

namespace {

struct ApplyP {
    int32_t B, Hq, Hkv, N, M, K, rep;
    int32_t d;             // head dim (<= the kernel's D; lanes past it load zeros, store nothing)
    const void *q, *k, *v;
    int64_t qsb, qsh, qsn, ksb, ksh, ksn, vsb, vsh, vsn;
    const int64_t *nb;
    const uint8_t *valid;
    const int32_t *nb32;   // or the graph as int32 ids, negative = invalid
    int32_t *row_inv;      // optional: per row, its count of invalid slots
    float scale;
    int32_t fp32w;
    float drop_p;
    float drop_scale;
    uint64_t seed;
    void *out;
    int64_t osb, osh, osn;
    int64_t rows;          // B*Hq*N
    int64_t nblocks;       // logical blocks
    // backward
    const float *dout;
    float *dq, *dk, *dv;
    // deterministic backward (workspace): per (row, slot) the two weights the
    // key and value gradients take, per key row its slot count and largest
    // weights (float bits), the largest |q| and |dout| (float bits), and the
    // fixed-point sums
    float *wdraw, *wpw;
    uint32_t *kcnt, *kmaxd, *kmaxp, *gmax;
    unsigned long long *acck, *accv;
};

constexpr int WAVES = 4;   // waves per workgroup

template <typename T> struct VecOf;
template <> struct VecOf<float> { static constexpr int n = 4; };
template <> struct VecOf<bf16_t> { static constexpr int n = 8; };
template <> struct VecOf<f16_t> { static constexpr int n = 8; };

template <typename T, int D> struct Geo {
    // elements per lane: a 16-byte load, more when the row is wider than a
    // wave holds that way (fp32 beyond 256)
    static constexpr int VEC = (VecOf<T>::n < D) ? (VecOf<T>::n * SSA_WAVE < D ? D / SSA_WAVE
                                                                              : VecOf<T>::n)
                                                 : D;
    static constexpr int LPR = D / VEC;                                // lanes per row
    static constexpr int RPI = SSA_WAVE / LPR;                         // rows per wave load
    static_assert(D % VEC == 0, "head dim must be a multiple of the vector width");
    static_assert(LPR <= SSA_WAVE, "row wider than a wave");
};

template <typename T, int VEC>
__device__ __forceinline__ void load_vec(const T *p, float (&f)[VEC]) {
    if constexpr (sizeof(T) * VEC == 32) {
        uint4 u[2] = {reinterpret_cast<const uint4 *>(p)[0], reinterpret_cast<const uint4 *>(p)[1]};
        const T *e = reinterpret_cast<const T *>(u);
#pragma unroll
        for (int i = 0; i < VEC; ++i) f[i] = to_f32(e[i]);
    } else if constexpr (sizeof(T) * VEC == 16) {
        uint4 u = *reinterpret_cast<const uint4 *>(p);
        const T *e = reinterpret_cast<const T *>(&u);
#pragma unroll
        for (int i = 0; i < VEC; ++i) f[i] = to_f32(e[i]);
    } else if constexpr (sizeof(T) * VEC == 8) {
        uint2 u = *reinterpret_cast<const uint2 *>(p);
        const T *e = reinterpret_cast<const T *>(&u);
#pragma unroll
        for (int i = 0; i < VEC; ++i) f[i] = to_f32(e[i]);
    } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) f[i] = to_f32(p[i]);
    }
}

// counter-based uniform in [0, 1): 64-bit mix of (seed, row, slot)
__device__ __forceinline__ float drop_uniform(uint64_t seed, int64_t row, int j) {
    uint64_t x = seed ^ (uint64_t)row * 0x9E3779B97F4A7C15ull ^ ((uint64_t)j << 32);
    x ^= x >> 33; x *= 0xff51afd7ed558ccdull;
    x ^= x >> 33; x *= 0xc4ceb9fe1a85ec53ull;
    x ^= x >> 33;
    return (float)(x >> 40) * (1.0f / 16777216.0f);
}

// The factor kept weights are multiplied by: the reference's dropout runs on
// the weights in their own dtype (the value dtype, or fp32 with
// fp32_attn_weights), whose noise tensor holds 1 / (1 - p) rounded to that
// dtype (sparse_attention.py:1193-1194).
template <typename T>
__device__ __forceinline__ float drop_scale_of(const ApplyP &p) {
    return p.fp32w ? p.drop_scale : Cvt<T>::round(p.drop_scale);
}

// A query row's graph slots j0 + u * 64 + lane (u < NB): the ids (int32 graph,
// or int64 ids and the mask) of all NB groups are loaded before any is used,
// so the row pays one memory latency for them instead of one per group.  The
// loads are unconditional (lanes past the row read its last slot) and the
// graph's layout is a template parameter, so no branch separates a load from
// the others.
constexpr int APPLY_SLOT_BATCH = 4;
template <int NB, bool I32>
struct RowSlots {
    int64_t y[NB];
    uint8_t v[NB];
    __device__ __forceinline__ void load(const ApplyP &p, int64_t row, const int64_t *nb,
                                         const uint8_t *va, int j0, int lane) {
#pragma unroll
        for (int u = 0; u < NB; ++u) {
            const int j = min(j0 + u * SSA_WAVE + lane, p.K - 1);
            if constexpr (I32) {
                y[u] = p.nb32[row * p.K + j];
            } else {
                y[u] = nb[j];
                v[u] = va ? va[j] : (uint8_t)1;
            }
        }
    }
    // the slot is marked invalid: mask false, or a negative id in an int32 graph
    __device__ __forceinline__ bool marked(int u) const {
        if constexpr (I32) return y[u] < 0;
        else return v[u] == 0;
    }
};

template <typename T, int D, int U>
__global__ void __launch_bounds__(WAVES * SSA_WAVE)
apply_fwd_kernel(ApplyP p) {
    using G = Geo<T, D>;
    constexpr int VEC = G::VEC, LPR = G::LPR, RPI = G::RPI;
    extern __shared__ float smem[];
    const int64_t blk = xcd_logical_block(blockIdx.x, p.nblocks);
    if (blk >= p.nblocks) return;
    const int wid = threadIdx.x / SSA_WAVE;
    const int64_t row = blk * WAVES + wid;
    if (row >= p.rows) return;
    const int lane = lane_id();
    const int sub = lane / LPR, li = lane % LPR;
    int32_t *ix = reinterpret_cast<int32_t *>(smem) + (int64_t)wid * 2 * p.K;   // key ids, -1 = masked
    float *sc = reinterpret_cast<float *>(ix + p.K);                          // scores, then p

    const int n = (int)(row % p.N);
    const int64_t bh = row / p.N;
    const int h = (int)(bh % p.Hq);
    const int b = (int)(bh / p.Hq);
    const int g = h / p.rep;

    const T *qrow = (const T *)p.q + b * p.qsb + h * p.qsh + (int64_t)n * p.qsn;
    const T *kb = (const T *)p.k + b * p.ksb + g * p.ksh;
    const T *vb = (const T *)p.v + b * p.vsb + g * p.vsh;
    const int64_t *nb = p.nb ? p.nb + row * p.K : nullptr;
    const uint8_t *va = p.valid ? p.valid + row * p.K : nullptr;

    // lanes whose elements lie past the head dim hold zeros and store nothing
    const bool live = li * VEC < p.d;
    const int lofs = live ? li * VEC : 0;
    // the q row is loaded first, beside the row's graph slots below
    float qf[VEC];
    load_vec<T, VEC>(qrow + lofs, qf);

    // neighbour ids once, as int32 in LDS; masked or out-of-range slots -> -1.
    // The row's padding count is the reference's (sparse_attention.py:1508):
    // slots the graph marks invalid (mask false, or a negative id in an int32
    // graph); an out-of-range id marked valid is skipped here but not counted
    int ninv = 0;
    auto slots = [&](auto i32) __attribute__((always_inline)) {
        for (int j0 = 0; j0 < p.K; j0 += APPLY_SLOT_BATCH * SSA_WAVE) {
            RowSlots<APPLY_SLOT_BATCH, decltype(i32)::value> rs;
            rs.load(p, row, nb, va, j0, lane);
#pragma unroll
            for (int u = 0; u < APPLY_SLOT_BATCH; ++u) {
                const int j = j0 + u * SSA_WAVE + lane;
                const bool in = j < p.K;
                const bool marked = in && rs.marked(u);
                const int64_t x = rs.y[u];
                if (in) ix[j] = (!marked && x >= 0 && x < p.M) ? (int)x : -1;
                ninv += __popcll(wave_ballot(marked));
            }
        }
    };
    if (p.nb32) slots(std::true_type{});
    else slots(std::false_type{});
    if (p.row_inv && lane == 0) p.row_inv[row] = ninv;
#pragma unroll
    for (int e = 0; e < VEC; ++e) qf[e] = live ? qf[e] : 0.f;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- scores
    for (int j0 = 0; j0 < p.K; j0 += RPI * U) {
        int xi[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = j0 + u * RPI + sub;
            xi[u] = j < p.K ? ix[j] : -1;
        }
        float kf[U][VEC];
#pragma unroll
        for (int u = 0; u < U; ++u)
            load_vec<T, VEC>(kb + (int64_t)(xi[u] < 0 ? 0 : xi[u]) * p.ksn + lofs, kf[u]);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float part = 0.f;
#pragma unroll
            for (int e = 0; e < VEC; ++e) part = fmaf(qf[e], kf[u][e], part);
#pragma unroll
            for (int o = LPR / 2; o > 0; o >>= 1) part += __shfl_xor(part, o, SSA_WAVE);
            const int j = j0 + u * RPI + sub;
            if (li == 0 && j < p.K) sc[j] = xi[u] >= 0 ? part * p.scale : -INFINITY;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- fp32 softmax, p computed once per slot (rounded to the value dtype
    // unless fp32_attn_weights; inverted dropout applied to p)
    float m = -INFINITY;
    for (int j = lane; j < p.K; j += SSA_WAVE) m = fmaxf(m, sc[j]);
    m = wave_max(m);
    float l = 0.f;
    for (int j = lane; j < p.K; j += SSA_WAVE) l += expf(sc[j] - m);
    l = wave_sum(l);
    const float inv = 1.f / l;
    for (int j = lane; j < p.K; j += SSA_WAVE) {
        float w = expf(sc[j] - m) * inv;
        if (!p.fp32w) w = Cvt<T>::round(w);
        if (p.drop_p > 0.f) {
            w = (drop_uniform(p.seed, row, j) < p.drop_p) ? 0.f : w * drop_scale_of<T>(p);
            if (!p.fp32w) w = Cvt<T>::round(w);
        }
        sc[j] = w;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- P.V
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
    for (int j0 = 0; j0 < p.K; j0 += RPI * U) {
        int xi[U];
        float pj[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = j0 + u * RPI + sub;
            const bool in = j < p.K;
            xi[u] = in ? ix[j] : -1;
            pj[u] = in ? sc[j] : 0.f;
        }
        float vf[U][VEC];
#pragma unroll
        for (int u = 0; u < U; ++u)
            load_vec<T, VEC>(vb + (int64_t)(xi[u] < 0 ? 0 : xi[u]) * p.vsn + lofs, vf[u]);
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int e = 0; e < VEC; ++e) acc[e] = fmaf(pj[u], vf[u][e], acc[e]);
    }
#pragma unroll
    for (int o = LPR; o < SSA_WAVE; o <<= 1)
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] += __shfl_xor(acc[e], o, SSA_WAVE);
    if (sub == 0 && live) {
        T *orow = (T *)p.out + b * p.osb + h * p.osh + (int64_t)n * p.osn + li * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) Cvt<T>::store(orow + e, acc[e]);
    }
}

// ---------------------------------------------------------------- rows beyond LDS
// Rows of more than APPLY_KLDS slots (whose scores do not fit a wave's share
// of LDS): nothing is kept per slot.  The scores are computed again in each
// pass over the row (same products, same order, so the same values): first
// the softmax maximum and sum online (a slot raising the maximum rescales the
// sum), then the weights, whose arithmetic is the kernels' above.
constexpr int APPLY_KLDS = 4096;

template <typename T, int VEC, int LPR>
struct LongRow {
    const ApplyP &p;
    int64_t row;
    const T *kb, *vb;
    const int64_t *nb;
    const uint8_t *va;
    int lofs;
    // key id of slot j, -1 when masked or out of range
    __device__ int id(int j, bool *marked = nullptr) const {
        const int64_t x = p.nb32 ? (int64_t)p.nb32[row * p.K + j] : nb[j];
        const bool mk = p.nb32 ? x < 0 : (va ? va[j] == 0 : false);
        if (marked) *marked = mk;
        return (!mk && x >= 0 && x < p.M) ? (int)x : -1;
    }
    // score of slot j (key id x, -1: -inf), every lane of the slot's group
    __device__ float score(const float (&qf)[VEC], int x) const {
        float kf[VEC];
        load_vec<T, VEC>(kb + (int64_t)(x < 0 ? 0 : x) * p.ksn + lofs, kf);
        float part = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) part = fmaf(qf[e], kf[e], part);
#pragma unroll
        for (int o = LPR / 2; o > 0; o >>= 1) part += __shfl_xor(part, o, SSA_WAVE);
        return x >= 0 ? part * p.scale : -INFINITY;
    }
    // dout . v of key x (row 0 for -1), every lane of the slot's group
    __device__ float dotv(const float (&dof)[VEC], int x) const {
        float vf[VEC];
        load_vec<T, VEC>(vb + (int64_t)(x < 0 ? 0 : x) * p.vsn + lofs, vf);
        float part = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) part = fmaf(dof[e], vf[e], part);
#pragma unroll
        for (int o = LPR / 2; o > 0; o >>= 1) part += __shfl_xor(part, o, SSA_WAVE);
        return part;
    }
};

// online softmax statistics of one lane group, then merged over the wave
__device__ __forceinline__ void online_add(float s, float &m, float &l) {
    if (s == -INFINITY) return;
    if (s > m) { l = l * expf(m - s) + 1.f; m = s; }
    else l += expf(s - m);
}

__device__ __forceinline__ void online_merge(bool lead, float m, float l, float &mm, float &ll) {
    mm = wave_max(lead ? m : -INFINITY);
    ll = wave_sum((lead && m != -INFINITY) ? l * expf(m - mm) : 0.f);
}

template <typename T, int D>
__global__ void __launch_bounds__(WAVES * SSA_WAVE)
apply_fwd_long_kernel(ApplyP p) {
    using G = Geo<T, D>;
    constexpr int VEC = G::VEC, LPR = G::LPR, RPI = G::RPI;
    const int64_t blk = xcd_logical_block(blockIdx.x, p.nblocks);
    if (blk >= p.nblocks) return;
    const int wid = threadIdx.x / SSA_WAVE;
    const int64_t row = blk * WAVES + wid;
    if (row >= p.rows) return;
    const int lane = lane_id();
    const int sub = lane / LPR, li = lane % LPR;
    const int n = (int)(row % p.N);
    const int64_t bh = row / p.N;
    const int h = (int)(bh % p.Hq);
    const int b = (int)(bh / p.Hq);
    const int g = h / p.rep;
    const T *qrow = (const T *)p.q + b * p.qsb + h * p.qsh + (int64_t)n * p.qsn;
    const bool live = li * VEC < p.d;
    const LongRow<T, VEC, LPR> R{p, row, (const T *)p.k + b * p.ksb + g * p.ksh,
                                 (const T *)p.v + b * p.vsb + g * p.vsh,
                                 p.nb ? p.nb + row * p.K : nullptr,
                                 p.valid ? p.valid + row * p.K : nullptr, live ? li * VEC : 0};
    if (p.row_inv) {
        int ninv = 0;
        for (int j0 = 0; j0 < p.K; j0 += SSA_WAVE) {
            bool mk = false;
            if (j0 + lane < p.K) (void)R.id(j0 + lane, &mk);
            ninv += __popcll(wave_ballot(mk));
        }
        if (lane == 0) p.row_inv[row] = ninv;
    }
    float qf[VEC];
    load_vec<T, VEC>(qrow + R.lofs, qf);
#pragma unroll
    for (int e = 0; e < VEC; ++e) qf[e] = live ? qf[e] : 0.f;
    float m = -INFINITY, l = 0.f;
    for (int j0 = 0; j0 < p.K; j0 += RPI) {
        const int j = j0 + sub;
        const float sj = R.score(qf, j < p.K ? R.id(j) : -1);
        if (j < p.K) online_add(sj, m, l);
    }
    float mm, ll;
    online_merge(li == 0, m, l, mm, ll);
    const float inv = 1.f / ll;
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
    for (int j0 = 0; j0 < p.K; j0 += RPI) {
        const int j = j0 + sub;
        const int x = j < p.K ? R.id(j) : -1;
        const float sj = R.score(qf, x);
        float w = expf(sj - mm) * inv;
        if (!p.fp32w) w = Cvt<T>::round(w);
        if (p.drop_p > 0.f) {
            w = (drop_uniform(p.seed, row, j) < p.drop_p) ? 0.f : w * drop_scale_of<T>(p);
            if (!p.fp32w) w = Cvt<T>::round(w);
        }
        w = j < p.K ? w : 0.f;
        float vf[VEC];
        load_vec<T, VEC>(R.vb + (int64_t)(x < 0 ? 0 : x) * p.vsn + R.lofs, vf);
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] = fmaf(w, vf[e], acc[e]);
    }
#pragma unroll
    for (int o = LPR; o < SSA_WAVE; o <<= 1)
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] += __shfl_xor(acc[e], o, SSA_WAVE);
    if (sub == 0 && live) {
        T *orow = (T *)p.out + b * p.osb + h * p.osh + (int64_t)n * p.osn + li * VEC;
#pragma unroll
        for (int e = 0; e < VEC; ++e) Cvt<T>::store(orow + e, acc[e]);
    }
}

// ---------------------------------------------------------------- 16-bit forward
// Packed 16-bit arithmetic for bf16 / fp16 models whose attention weights are
// rounded to the value dtype (fp32_attn_weights off):
//  * q.k: four v_dot2 (pairs of 16-bit products, fp32 accumulate) per lane,
//    then a sum over the LPR lanes of a row by DPP row permutations;
//  * P.V: the weights are exact in the value dtype, so two neighbours j, j'
//    go through one v_dot2 per element: {p_j, p_j'} . {v_j[e], v_j'[e]},
//    with the element pairs gathered by v_perm;
//  * rows are addressed by 32-bit byte offsets from a wave-uniform base.
template <typename T> struct Dot2;
template <> struct Dot2<bf16_t> {
    typedef __bf16 __attribute__((ext_vector_type(2))) v2;
    static __device__ __forceinline__ float dot(uint32_t a, uint32_t b, float c) {
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b),
                                               c, false);
    }
    // two bf16-exact fp32 values as a pair (a low, b high): their upper halves
    static __device__ __forceinline__ uint32_t pack(float a, float b) {
        return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
    }
    static __device__ __forceinline__ uint32_t bits(float v) { return f32_to_bf16_bits(v); }
};
template <> struct Dot2<f16_t> {
    typedef _Float16 __attribute__((ext_vector_type(2))) v2;
    static __device__ __forceinline__ float dot(uint32_t a, uint32_t b, float c) {
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(v2, a), __builtin_bit_cast(v2, b), c,
                                      false);
    }
    static __device__ __forceinline__ uint32_t pack(float a, float b) {
        const v2 h = {(_Float16)a, (_Float16)b};       // exact: both are fp16 values
        return __builtin_bit_cast(uint32_t, h);
    }
    static __device__ __forceinline__ uint32_t bits(float v) {
        const _Float16 h = (_Float16)v;
        return (uint32_t)__builtin_bit_cast(uint16_t, h);
    }
};

template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
    // every source lane of these patterns exists: old (0) is never used, and
    // an identity old lets the move fold into the add as a DPP operand
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF,
                                                          false));
}

// sum over the L lanes of each aligned group (L a power of two <= 32); every
// lane of the group gets the sum
template <int L>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (L >= 16) v = dpp_add<0x140>(v);   // row mirror
    if constexpr (L >= 8) v = dpp_add<0x141>(v);    // row half mirror
    if constexpr (L >= 2) v = dpp_add<0xB1>(v);     // quad perm [1,0,3,2]
    if constexpr (L >= 4) v = dpp_add<0x4E>(v);     // quad perm [2,3,0,1]
    if constexpr (L >= 32) v += __shfl_xor(v, 16, SSA_WAVE);
    return v;
}

template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Reduce U per-lane partials (one per row) over the 2U lanes of a row group
// by a butterfly: at each step a lane pair splits its rows, each lane sending
// the half it drops and adding the half it keeps (row mirror, half mirror,
// quad swaps as the pairings).  Afterwards lanes li and li ^ 1 both hold the
// total of row r = 4 [li >= 8] + 2 [li & 4] + [li & 2] (U = 8), or
// r = 2 [li & 4] + [li & 2] (U = 4).
template <int U>
__device__ __forceinline__ float butterfly_rows(float (&v)[U], int li) {
    static_assert(U == 4 || U == 8, "butterfly over 8 or 16 lanes");
    float w[4];
    if constexpr (U == 8) {
        const bool hi = li >= 8;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float send = hi ? v[k] : v[k + 4], keep = hi ? v[k + 4] : v[k];
            w[k] = keep + dpp_move<0x140>(send);        // row mirror: li <-> 15 - li
        }
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = v[k];
    }
    float x[2];
    {
        const bool hi = (li & 4) != 0;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const float send = hi ? w[k] : w[k + 2], keep = hi ? w[k + 2] : w[k];
            x[k] = keep + dpp_move<0x141>(send);        // half mirror: li <-> 7 - li (in 8)
        }
    }
    const bool hi = (li & 2) != 0;
    const float send = hi ? x[0] : x[1], keep = hi ? x[1] : x[0];
    float y = keep + dpp_move<0x4E>(send);              // quad perm [2,3,0,1]: li ^ 2
    return y + dpp_move<0xB1>(y);                       // quad perm [1,0,3,2]: li ^ 1
}

template <typename T, int D, int U>
__global__ void __launch_bounds__(WAVES * SSA_WAVE)
apply_fwd16_kernel(ApplyP p) {
    constexpr int LPR = D / 8;                 // lanes per row, 16 bytes each
    constexpr int RPI = SSA_WAVE / LPR;        // rows per wave load
    constexpr int STEP = RPI * U;              // slots per loop step
    constexpr bool BFLY = 2 * U == LPR;        // head dims 64 and 128
    static_assert(sizeof(T) == 2 && D % 8 == 0 && LPR <= 32 && U % 2 == 0, "16-bit path");
    extern __shared__ float smem[];
    const int64_t blk = xcd_logical_block(blockIdx.x, p.nblocks);
    if (blk >= p.nblocks) return;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / SSA_WAVE);
    const int64_t row = blk * WAVES + wid;
    if (row >= p.rows) return;
    const int lane = lane_id();
    const int sub = lane / LPR, li = lane % LPR;
    const int Kp = (p.K + STEP - 1) / STEP * STEP;                               // padded slots
    // key ids; masked, out-of-range and padding slots hold INT_MIN, whose low
    // 24 bits (all a 24-bit multiply reads) address row 0
    int32_t *ix = reinterpret_cast<int32_t *>(smem) + (int64_t)wid * 2 * Kp;
    float *sc = reinterpret_cast<float *>(ix + Kp);                           // scores, then p

    const int n = (int)(row % p.N);
    const int64_t bh = row / p.N;
    const int h = (int)(bh % p.Hq);
    const int b = (int)(bh / p.Hq);
    const int g = h / p.rep;
    const T *qrow = (const T *)p.q + b * p.qsb + h * p.qsh + (int64_t)n * p.qsn;
    const char *kb = (const char *)((const T *)p.k + b * p.ksb + g * p.ksh);
    const char *vb = (const char *)((const T *)p.v + b * p.vsb + g * p.vsh);
    const uint32_t krb = (uint32_t)(p.ksn * 2), vrb = (uint32_t)(p.vsn * 2);   // row bytes < 2^24
    // lanes whose 8 elements lie past the head dim hold zeros and store nothing
    const bool live = li * 8 < p.d;
    const uint32_t lio = live ? (uint32_t)li * 16u : 0u;
    const int64_t *nb = p.nb ? p.nb + row * p.K : nullptr;
    const uint8_t *va = p.valid ? p.valid + row * p.K : nullptr;

    // the q row is loaded first, beside the row's graph slots below
    uint4 q4 = *reinterpret_cast<const uint4 *>(qrow + (live ? li * 8 : 0));

    // neighbour ids as int32 in LDS (ids < 2^24, checked at dispatch); the
    // padding count takes the slots the graph marks invalid, as above
    int ninv = 0;
    auto slots = [&](auto i32) __attribute__((always_inline)) {
        for (int j0 = 0; j0 < Kp; j0 += APPLY_SLOT_BATCH * SSA_WAVE) {
            RowSlots<APPLY_SLOT_BATCH, decltype(i32)::value> rs;
            rs.load(p, row, nb, va, j0, lane);
#pragma unroll
            for (int u = 0; u < APPLY_SLOT_BATCH; ++u) {
                const int j = j0 + u * SSA_WAVE + lane;
                const bool in = j < p.K;
                const bool marked = in && rs.marked(u);
                const int64_t y = rs.y[u];
                const int x = (in && !marked && y >= 0 && y < p.M) ? (int)y : INT32_MIN;
                if (j < Kp) ix[j] = x;
                ninv += __popcll(wave_ballot(marked));
            }
        }
    };
    if (p.nb32) slots(std::true_type{});
    else slots(std::false_type{});
    if (p.row_inv && lane == 0) p.row_inv[row] = ninv;
    if (!live) q4 = make_uint4(0, 0, 0, 0);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- scores q.k * scale (masked slots are set to -inf by the softmax)
    for (int j0 = 0; j0 < Kp; j0 += STEP) {
        int xi[U];
#pragma unroll
        for (int u = 0; u < U; ++u) xi[u] = ix[j0 + u * RPI + sub];
        uint4 kv[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            kv[u] = *reinterpret_cast<const uint4 *>(kb + (__umul24((uint32_t)xi[u], krb) + lio));
        float part[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            part[u] = Dot2<T>::dot(q4.x, kv[u].x, 0.f);
            part[u] = Dot2<T>::dot(q4.y, kv[u].y, part[u]);
            part[u] = Dot2<T>::dot(q4.z, kv[u].z, part[u]);
            part[u] = Dot2<T>::dot(q4.w, kv[u].w, part[u]);
        }
        if constexpr (BFLY) {
            const float tot = butterfly_rows<U>(part, li);
            const int r = (U == 8 ? 4 * (li >= 8) : 0) + 2 * ((li & 4) != 0) + ((li & 2) != 0);
            if ((li & 1) == 0) sc[j0 + r * RPI + sub] = tot * p.scale;
        } else {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const float tot = group_sum<LPR>(part[u]);
                if (li == 0) sc[j0 + u * RPI + sub] = tot * p.scale;
            }
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // the first P.V step's V rows (they need only the ids) load while the
    // softmax runs
    uint4 vv0[U];
    {
        int xi[U];
#pragma unroll
        for (int u = 0; u < U; ++u) xi[u] = ix[u * RPI + sub];
#pragma unroll
        for (int u = 0; u < U; ++u)
            vv0[u] = *reinterpret_cast<const uint4 *>(vb + (__umul24((uint32_t)xi[u], vrb) + lio));
    }

    // ---- fp32 softmax; p rounded to the value dtype (inverted dropout on p);
    // padding slots get p = 0
    float m = -INFINITY;
    for (int j = lane; j < p.K; j += SSA_WAVE) {
        const float s = ix[j] >= 0 ? sc[j] : -INFINITY;
        sc[j] = s;
        m = fmaxf(m, s);
    }
    m = wave_max(m);
    float l = 0.f;
    for (int j = lane; j < p.K; j += SSA_WAVE) l += expf(sc[j] - m);
    l = wave_sum(l);
    const float inv = 1.f / l;
    for (int j = lane; j < Kp; j += SSA_WAVE) {
        float w = 0.f;
        if (j < p.K) {
            w = Cvt<T>::round(expf(sc[j] - m) * inv);
            if (p.drop_p > 0.f)
                w = (drop_uniform(p.seed, row, j) < p.drop_p) ? 0.f
                                                              : Cvt<T>::round(w * drop_scale_of<T>(p));
        }
        sc[j] = w;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // ---- P.V, neighbours in pairs
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.f;
    auto vstep = [&](int j0, const uint4 (&vv)[U]) __attribute__((always_inline)) {
        float pj[U];
#pragma unroll
        for (int u = 0; u < U; ++u) pj[u] = sc[j0 + u * RPI + sub];
#pragma unroll
        for (int u = 0; u < U; u += 2) {
            const uint32_t pp = Dot2<T>::pack(pj[u], pj[u + 1]);
            const uint32_t a[4] = {vv[u].x, vv[u].y, vv[u].z, vv[u].w};
            const uint32_t c[4] = {vv[u + 1].x, vv[u + 1].y, vv[u + 1].z, vv[u + 1].w};
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                acc[2 * r] = Dot2<T>::dot(pp, __builtin_amdgcn_perm(c[r], a[r], 0x05040100u),
                                          acc[2 * r]);
                acc[2 * r + 1] = Dot2<T>::dot(pp, __builtin_amdgcn_perm(c[r], a[r], 0x07060302u),
                                              acc[2 * r + 1]);
            }
        }
    };
    vstep(0, vv0);
    for (int j0 = STEP; j0 < Kp; j0 += STEP) {
        int xi[U];
#pragma unroll
        for (int u = 0; u < U; ++u) xi[u] = ix[j0 + u * RPI + sub];
        uint4 vv[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            vv[u] = *reinterpret_cast<const uint4 *>(vb + (__umul24((uint32_t)xi[u], vrb) + lio));
        vstep(j0, vv);
    }
#pragma unroll
    for (int o = LPR; o < SSA_WAVE; o <<= 1)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[e] += __shfl_xor(acc[e], o, SSA_WAVE);
    if (sub == 0 && live) {
        T *orow = (T *)p.out + b * p.osb + h * p.osh + (int64_t)n * p.osn + li * 8;
        uint4 o4;
        o4.x = Dot2<T>::bits(acc[0]) | (Dot2<T>::bits(acc[1]) << 16);
        o4.y = Dot2<T>::bits(acc[2]) | (Dot2<T>::bits(acc[3]) << 16);
        o4.z = Dot2<T>::bits(acc[4]) | (Dot2<T>::bits(acc[5]) << 16);
        o4.w = Dot2<T>::bits(acc[6]) | (Dot2<T>::bits(acc[7]) << 16);
        *reinterpret_cast<uint4 *>(orow) = o4;
    }
}

// Backward: recompute p, then dp = dO.v, ds = p (dp - sum p dp), draw = ds*scale,
// dq = sum draw k (direct store), dk += draw q, dv += p' dO (fp32 atomics).
// DET (the deterministic backward's first pass): instead of the atomics, each
// slot's draw and p' go to the workspace, and its key row's slot count and
// largest |draw| and |p'| are raised (integer atomics, whose results do not
// depend on their order), as are the largest |q| and |dout|.
template <typename T, int D, bool DET>
__global__ void __launch_bounds__(WAVES * SSA_WAVE)
apply_bwd_kernel(ApplyP p) {
    using G = Geo<T, D>;
    constexpr int VEC = G::VEC, LPR = G::LPR, RPI = G::RPI;
    extern __shared__ float smem[];
    const int64_t blk = xcd_logical_block(blockIdx.x, p.nblocks);
    if (blk >= p.nblocks) return;
    const int wid = threadIdx.x / SSA_WAVE;
    const int64_t row = blk * WAVES + wid;
    if (row >= p.rows) return;
    const int lane = lane_id();
    const int sub = lane / LPR, li = lane % LPR;
    float *sc = smem + wid * 2 * p.K;     // scores, then p'
    float *dpv = sc + p.K;                // dp per slot

    const int n = (int)(row % p.N);
    const int64_t bh = row / p.N;
    const int h = (int)(bh % p.Hq);
    const int b = (int)(bh / p.Hq);
    const int g = h / p.rep;
    const T *qrow = (const T *)p.q + b * p.qsb + h * p.qsh + (int64_t)n * p.qsn;
    const T *kb = (const T *)p.k + b * p.ksb + g * p.ksh;
    const T *vb = (const T *)p.v + b * p.vsb + g * p.vsh;
    const int64_t *nb = p.nb + row * p.K;
    const uint8_t *va = p.valid ? p.valid + row * p.K : nullptr;
    // gradients are (rows, d) fp32; lanes past the head dim hold zeros and
    // write nothing
    const bool live = li * VEC < p.d;
    const int lofs = live ? li * VEC : 0;
    const float *dorow = p.dout + row * p.d + lofs;

    float qf[VEC], dof[VEC];
    load_vec<T, VEC>(qrow + lofs, qf);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
        dof[e] = live ? dorow[e] : 0.f;
        qf[e] = live ? qf[e] : 0.f;
    }

    for (int j0 = 0; j0 < p.K; j0 += RPI) {
        const int j = j0 + sub;
        int64_t x = 0;
        bool o = false;
        if (j < p.K) { x = nb[j]; o = va ? (va[j] != 0) : true; }
        if (x < 0 || x >= p.M) { x = 0; o = false; }
        float kf[VEC], vf[VEC];
        load_vec<T, VEC>(kb + x * p.ksn + lofs, kf);
        load_vec<T, VEC>(vb + x * p.vsn + lofs, vf);
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) { s = fmaf(qf[e], kf[e], s); dp = fmaf(dof[e], vf[e], dp); }
#pragma unroll
        for (int off = LPR / 2; off > 0; off >>= 1) {
            s += __shfl_xor(s, off, SSA_WAVE);
            dp += __shfl_xor(dp, off, SSA_WAVE);
        }
        if (li == 0 && j < p.K) { sc[j] = o ? s * p.scale : -INFINITY; dpv[j] = dp; }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float m = -INFINITY;
    for (int j = lane; j < p.K; j += SSA_WAVE) m = fmaxf(m, sc[j]);
    m = wave_max(m);
    float l = 0.f;
    for (int j = lane; j < p.K; j += SSA_WAVE) l += expf(sc[j] - m);
    l = wave_sum(l);
    // dp w.r.t. softmax output includes the dropout mask/scale
    float pdp = 0.f;
    for (int j = lane; j < p.K; j += SSA_WAVE) {
        float pj = expf(sc[j] - m) / l;
        float mask = 1.f;
        if (p.drop_p > 0.f) mask = (drop_uniform(p.seed, row, j) < p.drop_p) ? 0.f : drop_scale_of<T>(p);
        float dpj = dpv[j] * mask;
        pdp += pj * dpj;
        sc[j] = pj;          // keep p
        dpv[j] = dpj;        // keep dp (softmax-output side)
    }
    pdp = wave_sum(pdp);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    if (DET) {
        // the largest |q| and |dout| bound every slot's contributions
        float qm = 0.f, dm = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            qm = fmaxf(qm, fabsf(qf[e]));
            dm = fmaxf(dm, fabsf(dof[e]));
        }
        qm = wave_max(qm);
        dm = wave_max(dm);
        if (lane == 0) {
            atomicMax(&p.gmax[0], __float_as_uint(qm));
            atomicMax(&p.gmax[1], __float_as_uint(dm));
        }
    }
    float dqa[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) dqa[e] = 0.f;
    for (int j0 = 0; j0 < p.K; j0 += RPI) {
        const int j = j0 + sub;
        if (j >= p.K) continue;
        int64_t x = nb[j];
        if (x < 0 || x >= p.M) {
            if (DET && li == 0) { p.wdraw[row * p.K + j] = 0.f; p.wpw[row * p.K + j] = 0.f; }
            continue;
        }
        const float pj = sc[j];
        const float draw = pj * (dpv[j] - pdp) * p.scale;
        float mask = 1.f;
        if (p.drop_p > 0.f) mask = (drop_uniform(p.seed, row, j) < p.drop_p) ? 0.f : drop_scale_of<T>(p);
        const float pw = pj * mask;
        float kf[VEC];
        load_vec<T, VEC>(kb + x * p.ksn + lofs, kf);
        const int64_t kr = ((int64_t)b * p.Hkv + g) * p.M + x;
        if (DET) {
            if (li == 0) {
                p.wdraw[row * p.K + j] = draw;
                p.wpw[row * p.K + j] = pw;
                atomicAdd(&p.kcnt[kr], 1u);
                atomicMax(&p.kmaxd[kr], __float_as_uint(fabsf(draw)));
                atomicMax(&p.kmaxp[kr], __float_as_uint(fabsf(pw)));
            }
#pragma unroll
            for (int e = 0; e < VEC; ++e) dqa[e] = fmaf(draw, kf[e], dqa[e]);
        } else {
            float *dkr = p.dk + kr * p.d + lofs;
            float *dvr = p.dv + kr * p.d + lofs;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                dqa[e] = fmaf(draw, kf[e], dqa[e]);
                if (live && draw != 0.f) unsafeAtomicAdd(dkr + e, draw * qf[e]);
                if (live && pw != 0.f) unsafeAtomicAdd(dvr + e, pw * dof[e]);
            }
        }
    }
#pragma unroll
    for (int o = LPR; o < SSA_WAVE; o <<= 1)
#pragma unroll
        for (int e = 0; e < VEC; ++e) dqa[e] += __shfl_xor(dqa[e], o, SSA_WAVE);
    if (sub == 0 && live) {
        float *dqr = p.dq + row * p.d + lofs;
#pragma unroll
        for (int e = 0; e < VEC; ++e) dqr[e] = dqa[e];
    }
}

// Backward of rows beyond LDS: the softmax statistics online, then
// sum p dp, then each slot's draw and p' (the arithmetic of apply_bwd_kernel,
// with the scores and dout . v computed again in each pass).
template <typename T, int D, bool DET>
__global__ void __launch_bounds__(WAVES * SSA_WAVE)
apply_bwd_long_kernel(ApplyP p) {
    using G = Geo<T, D>;
    constexpr int VEC = G::VEC, LPR = G::LPR, RPI = G::RPI;
    const int64_t blk = xcd_logical_block(blockIdx.x, p.nblocks);
    if (blk >= p.nblocks) return;
    const int wid = threadIdx.x / SSA_WAVE;
    const int64_t row = blk * WAVES + wid;
    if (row >= p.rows) return;
    const int lane = lane_id();
    const int sub = lane / LPR, li = lane % LPR;
    const int n = (int)(row % p.N);
    const int64_t bh = row / p.N;
    const int h = (int)(bh % p.Hq);
    const int b = (int)(bh / p.Hq);
    const int g = h / p.rep;
    const T *qrow = (const T *)p.q + b * p.qsb + h * p.qsh + (int64_t)n * p.qsn;
    const bool live = li * VEC < p.d;
    const LongRow<T, VEC, LPR> R{p, row, (const T *)p.k + b * p.ksb + g * p.ksh,
                                 (const T *)p.v + b * p.vsb + g * p.vsh, p.nb + row * p.K,
                                 p.valid ? p.valid + row * p.K : nullptr, live ? li * VEC : 0};
    const float *dorow = p.dout + row * p.d + R.lofs;
    float qf[VEC], dof[VEC];
    load_vec<T, VEC>(qrow + R.lofs, qf);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
        dof[e] = live ? dorow[e] : 0.f;
        qf[e] = live ? qf[e] : 0.f;
    }
    if (DET) {
        float qm = 0.f, dm = 0.f;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            qm = fmaxf(qm, fabsf(qf[e]));
            dm = fmaxf(dm, fabsf(dof[e]));
        }
        qm = wave_max(qm);
        dm = wave_max(dm);
        if (lane == 0) {
            atomicMax(&p.gmax[0], __float_as_uint(qm));
            atomicMax(&p.gmax[1], __float_as_uint(dm));
        }
    }
    // the ids are read from the graph in each pass (the graph's validity and
    // range rules of the forward; the backward takes int64 ids only)
    float m = -INFINITY, l = 0.f;
    for (int j0 = 0; j0 < p.K; j0 += RPI) {
        const int j = j0 + sub;
        const float sj = R.score(qf, j < p.K ? R.id(j) : -1);
        if (j < p.K) online_add(sj, m, l);
    }
    float mm, ll;
    online_merge(li == 0, m, l, mm, ll);
    auto mask_of = [&](int j) {
        return p.drop_p > 0.f ? ((drop_uniform(p.seed, row, j) < p.drop_p) ? 0.f : drop_scale_of<T>(p))
                              : 1.f;
    };
    float pdp = 0.f;
    for (int j0 = 0; j0 < p.K; j0 += RPI) {
        const int j = j0 + sub;
        const int x = j < p.K ? R.id(j) : -1;
        const float pj = expf(R.score(qf, x) - mm) / ll;
        const float dpj = R.dotv(dof, x) * mask_of(j);
        if (j < p.K && li == 0) pdp += pj * dpj;
    }
    pdp = wave_sum(pdp);
    float dqa[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) dqa[e] = 0.f;
    for (int j0 = 0; j0 < p.K; j0 += RPI) {
        const int j = j0 + sub;
        if (j >= p.K) continue;
        const int64_t xr = R.nb[j];
        if (xr < 0 || xr >= p.M) {
            if (DET && li == 0) { p.wdraw[row * p.K + j] = 0.f; p.wpw[row * p.K + j] = 0.f; }
            continue;
        }
        const int x = R.id(j);
        const float pj = expf(R.score(qf, x) - mm) / ll;
        const float mask = mask_of(j);
        const float draw = pj * (R.dotv(dof, x) * mask - pdp) * p.scale;
        const float pw = pj * mask;
        float kf[VEC];
        load_vec<T, VEC>(R.kb + xr * p.ksn + R.lofs, kf);
        const int64_t kr = ((int64_t)b * p.Hkv + g) * p.M + xr;
        if (DET) {
            if (li == 0) {
                p.wdraw[row * p.K + j] = draw;
                p.wpw[row * p.K + j] = pw;
                atomicAdd(&p.kcnt[kr], 1u);
                atomicMax(&p.kmaxd[kr], __float_as_uint(fabsf(draw)));
                atomicMax(&p.kmaxp[kr], __float_as_uint(fabsf(pw)));
            }
#pragma unroll
            for (int e = 0; e < VEC; ++e) dqa[e] = fmaf(draw, kf[e], dqa[e]);
        } else {
            float *dkr = p.dk + kr * p.d + R.lofs;
            float *dvr = p.dv + kr * p.d + R.lofs;
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
                dqa[e] = fmaf(draw, kf[e], dqa[e]);
                if (live && draw != 0.f) unsafeAtomicAdd(dkr + e, draw * qf[e]);
                if (live && pw != 0.f) unsafeAtomicAdd(dvr + e, pw * dof[e]);
            }
        }
    }
#pragma unroll
    for (int o = LPR; o < SSA_WAVE; o <<= 1)
#pragma unroll
        for (int e = 0; e < VEC; ++e) dqa[e] += __shfl_xor(dqa[e], o, SSA_WAVE);
    if (sub == 0 && live) {
        float *dqr = p.dq + row * p.d + R.lofs;
#pragma unroll
        for (int e = 0; e < VEC; ++e) dqr[e] = dqa[e];
    }
}

// ---- deterministic backward: fixed-point sums
// A key row's gradient is a sum over the (query row, slot) pairs that hold it.
// Its terms are rounded to a fixed-point grid of that key row and summed as
// 64-bit integers, whose sum does not depend on the order the atomics land
// in; the grid 2^-s is the finest for which the sum cannot overflow: count x
// largest weight x largest |q| (or |dout|) below 2^(61 - s).  Returns -1
// when the key row has no term, -2 when a bound is not finite.
__device__ __forceinline__ int fx_shift(uint32_t cnt, uint32_t wbits, uint32_t xbits) {
    const double bound = (double)cnt * (double)__uint_as_float(wbits) * (double)__uint_as_float(xbits);
    if (!(bound == bound) || bound > 1e300) return -2;
    if (!(bound > 0.0)) return -1;
    int e = 0;
    (void)frexp(bound, &e);                 // bound < 2^e
    return 61 - e;
}

__device__ __forceinline__ unsigned long long fx_of(float c, int s) {
    return (unsigned long long)(long long)rint(ldexp((double)c, s));
}

// second pass: per query row, each slot's terms draw * q and p' * dout added
// to its key row's fixed-point sums
template <typename T, int D>
__global__ void __launch_bounds__(WAVES * SSA_WAVE)
apply_bwd_fx_kernel(ApplyP p) {
    using G = Geo<T, D>;
    constexpr int VEC = G::VEC, LPR = G::LPR, RPI = G::RPI;
    const int64_t blk = xcd_logical_block(blockIdx.x, p.nblocks);
    if (blk >= p.nblocks) return;
    const int wid = threadIdx.x / SSA_WAVE;
    const int64_t row = blk * WAVES + wid;
    if (row >= p.rows) return;
    const int lane = lane_id();
    const int sub = lane / LPR, li = lane % LPR;
    const int n = (int)(row % p.N);
    const int64_t bh = row / p.N;
    const int h = (int)(bh % p.Hq);
    const int b = (int)(bh / p.Hq);
    const int g = h / p.rep;
    const T *qrow = (const T *)p.q + b * p.qsb + h * p.qsh + (int64_t)n * p.qsn;
    const int64_t *nb = p.nb + row * p.K;
    const bool live = li * VEC < p.d;
    const int lofs = live ? li * VEC : 0;
    const float *dorow = p.dout + row * p.d + lofs;
    float qf[VEC], dof[VEC];
    load_vec<T, VEC>(qrow + lofs, qf);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
        dof[e] = live ? dorow[e] : 0.f;
        qf[e] = live ? qf[e] : 0.f;
    }
    const uint32_t qmax = p.gmax[0], dmax = p.gmax[1];
    for (int j0 = 0; j0 < p.K; j0 += RPI) {
        const int j = j0 + sub;
        if (j >= p.K) continue;
        const int64_t x = nb[j];
        if (x < 0 || x >= p.M) continue;
        const float draw = p.wdraw[row * p.K + j], pw = p.wpw[row * p.K + j];
        const int64_t kr = ((int64_t)b * p.Hkv + g) * p.M + x;
        const uint32_t cnt = p.kcnt[kr];
        const int sk = fx_shift(cnt, p.kmaxd[kr], qmax);
        const int sv = fx_shift(cnt, p.kmaxp[kr], dmax);
        unsigned long long *ak = p.acck + kr * p.d + lofs;
        unsigned long long *av = p.accv + kr * p.d + lofs;
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
            if (live && draw != 0.f && sk >= 0) atomicAdd(ak + e, fx_of(draw * qf[e], sk));
            if (live && pw != 0.f && sv >= 0) atomicAdd(av + e, fx_of(pw * dof[e], sv));
        }
    }
}

// last pass: dk += sum * 2^-s, dv likewise, per element (NaN where a bound
// was not finite)
__global__ void __launch_bounds__(256) apply_bwd_finish_kernel(ApplyP p, int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= total) return;
    const int64_t kr = i / p.d;
    const uint32_t cnt = p.kcnt[kr];
    const int sk = fx_shift(cnt, p.kmaxd[kr], p.gmax[0]);
    const int sv = fx_shift(cnt, p.kmaxp[kr], p.gmax[1]);
    if (sk >= 0) p.dk[i] += (float)ldexp((double)(long long)p.acck[i], -sk);
    else if (sk == -2) p.dk[i] = __builtin_nanf("");
    if (sv >= 0) p.dv[i] += (float)ldexp((double)(long long)p.accv[i], -sv);
    else if (sv == -2) p.dv[i] = __builtin_nanf("");
}

__global__ void __launch_bounds__(256) apply_zero_kernel(uint32_t *w, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        w[i] = 0u;
}

// The 16-bit path needs weights in the value dtype, 16-byte aligned rows,
// byte offsets of every K / V row (and q row slice) within 32 bits, and key
// ids below 2^24 (rows are addressed by 24-bit multiplies).
bool fwd16_ok(const ApplyP &p, int elem, int D) {
    const int64_t v = 16 / elem;
    const bool aligned = ((uintptr_t)p.q % 16 == 0) && ((uintptr_t)p.k % 16 == 0) &&
                         ((uintptr_t)p.v % 16 == 0) && ((uintptr_t)p.out % 16 == 0) &&
                         p.qsb % v == 0 && p.qsh % v == 0 && p.qsn % v == 0 && p.ksb % v == 0 &&
                         p.ksh % v == 0 && p.ksn % v == 0 && p.vsb % v == 0 && p.vsh % v == 0 &&
                         p.vsn % v == 0 && p.osb % v == 0 && p.osh % v == 0 && p.osn % v == 0;
    const int64_t lim = (int64_t)1 << 24;
    const bool small = p.M < lim && p.ksn * elem < lim && p.vsn * elem < lim &&
                       ((int64_t)p.M * p.ksn + D) * elem < ((int64_t)1 << 31) &&
                       ((int64_t)p.M * p.vsn + D) * elem < ((int64_t)1 << 31);
    return !p.fp32w && aligned && small;
}

template <typename T, int D>
int launch_apply(const ApplyP &p, hipStream_t st, bool bwd) {
    const int64_t grid = 8 * ceil_div(p.nblocks, 8);
    const bool lng = p.K > APPLY_KLDS;
    if (lng && !bwd) {
        hipLaunchKernelGGL((apply_fwd_long_kernel<T, D>), dim3((unsigned)grid),
                           dim3(WAVES * SSA_WAVE), 0, st, p);
        SSA_CHECK_LAUNCH();
        return SSA_OK;
    }
    if (lng && !p.wdraw) {
        hipLaunchKernelGGL((apply_bwd_long_kernel<T, D, false>), dim3((unsigned)grid),
                           dim3(WAVES * SSA_WAVE), 0, st, p);
        SSA_CHECK_LAUNCH();
        return SSA_OK;
    }
    if (bwd && p.wdraw) {
        // deterministic: rows (dq, weights, bounds), fixed-point sums, finish
        if (lng) {
            hipLaunchKernelGGL((apply_bwd_long_kernel<T, D, true>), dim3((unsigned)grid),
                               dim3(WAVES * SSA_WAVE), 0, st, p);
        } else {
            const size_t lds = (size_t)WAVES * 2 * p.K * sizeof(float);
            if (lds > 65536)
                SSA_CHECK_HIP(hipFuncSetAttribute((const void *)apply_bwd_kernel<T, D, true>,
                                                  hipFuncAttributeMaxDynamicSharedMemorySize,
                                                  (int)lds));
            hipLaunchKernelGGL((apply_bwd_kernel<T, D, true>), dim3((unsigned)grid),
                               dim3(WAVES * SSA_WAVE), lds, st, p);
        }
        SSA_CHECK_LAUNCH();
        hipLaunchKernelGGL((apply_bwd_fx_kernel<T, D>), dim3((unsigned)grid),
                           dim3(WAVES * SSA_WAVE), 0, st, p);
        SSA_CHECK_LAUNCH();
        const int64_t total = (int64_t)p.B * p.Hkv * p.M * p.d;
        if (total > 0) {
            hipLaunchKernelGGL(apply_bwd_finish_kernel, dim3((unsigned)ceil_div(total, 256)),
                               dim3(256), 0, st, p, total);
        }
    } else if (bwd) {
        const size_t lds = (size_t)WAVES * 2 * p.K * sizeof(float);
        if (lds > 65536)
            SSA_CHECK_HIP(hipFuncSetAttribute((const void *)apply_bwd_kernel<T, D, false>,
                                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        hipLaunchKernelGGL((apply_bwd_kernel<T, D, false>), dim3((unsigned)grid),
                           dim3(WAVES * SSA_WAVE), lds, st, p);
    } else {
        const size_t lds = (size_t)WAVES * 2 * p.K * sizeof(float);
        // slot batches of 8 row loads, 4 where a load covers 16 rows or more
        // (64 slots a step at 8 rows a load: 64-wide bf16 heads 1% faster)
        constexpr int U = (Geo<T, D>::RPI >= 16) ? 4 : 8;
        if constexpr (sizeof(T) == 2 && D >= 8 && D <= 256) {   // two rows per wave at least
            if (fwd16_ok(p, (int)sizeof(T), D)) {
                constexpr int STEP = (SSA_WAVE / (D / 8)) * U;
                const size_t lds16 = (size_t)WAVES * 2 * ceil_div(p.K, STEP) * STEP * sizeof(float);
                if (lds16 > 65536)
                    SSA_CHECK_HIP(hipFuncSetAttribute((const void *)apply_fwd16_kernel<T, D, U>,
                                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                                      (int)lds16));
                hipLaunchKernelGGL((apply_fwd16_kernel<T, D, U>), dim3((unsigned)grid),
                                   dim3(WAVES * SSA_WAVE), lds16, st, p);
                SSA_CHECK_LAUNCH();
                return SSA_OK;
            }
        }
        if (lds > 65536)
            SSA_CHECK_HIP(hipFuncSetAttribute((const void *)apply_fwd_kernel<T, D, U>,
                                              hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        hipLaunchKernelGGL((apply_fwd_kernel<T, D, U>), dim3((unsigned)grid),
                           dim3(WAVES * SSA_WAVE), lds, st, p);
    }
    SSA_CHECK_LAUNCH();
    return SSA_OK;
}

template <typename T>
int dispatch_d(const ApplyP &p, int d, hipStream_t st, bool bwd) {
    if (!ssa_head_dim_ok(d, std::is_same<T, float>::value ? SSA_F32 : SSA_BF16)) {
        ssa_set_error("sparse_gather_attention: head dim %d unsupported (4..1024: a power of two "
                      "or a multiple of %d)", d, std::is_same<T, float>::value ? 4 : 8);
        return SSA_E_UNSUP;
    }
    switch (ssa_pow2_instance(d)) {
        case 4: return launch_apply<T, 4>(p, st, bwd);
        case 8: return launch_apply<T, 8>(p, st, bwd);
        case 16: return launch_apply<T, 16>(p, st, bwd);
        case 32: return launch_apply<T, 32>(p, st, bwd);
        case 64: return launch_apply<T, 64>(p, st, bwd);
        case 128: return launch_apply<T, 128>(p, st, bwd);
        case 256: return launch_apply<T, 256>(p, st, bwd);
        case 512: return launch_apply<T, 512>(p, st, bwd);
        case 1024: return launch_apply<T, 1024>(p, st, bwd);
        default:
            ssa_set_error("sparse_gather_attention: head dim %d has no kernel instance", d);
            return SSA_E_UNSUP;
    }
}

int check_view(const ssa_tensor4 &t, int dtype, const char *name) {
    if (!t.ptr) { ssa_set_error("%s: null pointer", name); return SSA_E_ARG; }
    if (t.dtype != dtype) { ssa_set_error("%s: dtype mismatch", name); return SSA_E_ARG; }
    return SSA_OK;
}

int apply_common(const ssa_apply_args *a, ApplyP &p) {
    SSA_CHECK_ARG(a != nullptr, "sparse_gather_attention: null args");
    SSA_CHECK_ARG(a->B >= 0 && a->Hq > 0 && a->Hkv > 0 && a->N >= 0 && a->M > 0 && a->K >= 0,
                  "sparse_gather_attention: bad sizes B=%d Hq=%d Hkv=%d N=%d M=%d K=%d", a->B,
                  a->Hq, a->Hkv, a->N, a->M, a->K);
    SSA_CHECK_ARG(a->Hq % a->Hkv == 0, "sparse_gather_attention: Hq %% Hkv != 0");
    SSA_CHECK_ARG((int64_t)a->B * a->Hq * a->N * a->K < ((int64_t)1 << 62),
                  "sparse_gather_attention: too many slots");
    SSA_CHECK_ARG(a->q.dtype >= 0 && a->q.dtype <= 2, "sparse_gather_attention: bad dtype");
    int rc;
    if ((rc = check_view(a->q, a->q.dtype, "q"))) return rc;
    if ((rc = check_view(a->k, a->q.dtype, "k"))) return rc;
    if ((rc = check_view(a->v, a->q.dtype, "v"))) return rc;
    SSA_CHECK_ARG((a->neighbors != nullptr || a->neighbors32 != nullptr) && a->out != nullptr,
                  "sparse_gather_attention: null");
    SSA_CHECK_ARG(a->dropout_p >= 0.f && a->dropout_p < 1.f, "dropout p must be in [0, 1)");
    p = ApplyP{};
    p.B = a->B; p.Hq = a->Hq; p.Hkv = a->Hkv; p.N = a->N; p.M = a->M; p.K = a->K;
    p.rep = a->Hq / a->Hkv;
    p.d = a->d;
    p.q = a->q.ptr; p.k = a->k.ptr; p.v = a->v.ptr;
    p.qsb = a->q.sb; p.qsh = a->q.sh; p.qsn = a->q.sn;
    p.ksb = a->k.sb; p.ksh = a->k.sh; p.ksn = a->k.sn;
    p.vsb = a->v.sb; p.vsh = a->v.sh; p.vsn = a->v.sn;
    p.nb = a->neighbors; p.valid = a->valid; p.nb32 = a->neighbors32;
    p.row_inv = a->row_invalid;
    p.scale = a->scale; p.fp32w = a->fp32_weights;
    p.drop_p = a->dropout_p;
    // inverted dropout scales kept weights by 1 / (1 - p), the keep rate taken
    // in double and rounded to fp32 as torch's dropout divides its noise
    p.drop_scale = a->dropout_p > 0.f ? 1.f / (float)(1.0 - (double)a->dropout_p) : 1.f;
    p.seed = a->seed;
    p.out = a->out; p.osb = a->out_sb; p.osh = a->out_sh; p.osn = a->out_sn;
    p.rows = (int64_t)a->B * a->Hq * a->N;
    p.nblocks = ceil_div(p.rows, WAVES);
    return SSA_OK;
}

int run_apply(const ApplyP &p, int dtype, int d, hipStream_t st, bool bwd) {
    if (p.rows == 0) return SSA_OK;
    switch (dtype) {
        case SSA_F32: return dispatch_d<float>(p, d, st, bwd);
        case SSA_BF16: return dispatch_d<bf16_t>(p, d, st, bwd);
        case SSA_F16: return dispatch_d<f16_t>(p, d, st, bwd);
    }
    ssa_set_error("sparse_gather_attention: bad dtype %d", dtype);
    return SSA_E_ARG;
}

}  // namespace

extern "C" int ssa_sparse_gather_attention(const ssa_apply_args *a, void *stream) {
    ApplyP p;
    int rc = apply_common(a, p);
    if (rc) return rc;
    return run_apply(p, a->q.dtype, a->d, (hipStream_t)stream, false);
}

namespace {

int bwd_common(const ssa_apply_bwd_args *a, ApplyP &p) {
    SSA_CHECK_ARG(a != nullptr, "sparse_gather_attention_bwd: null args");
    int rc = apply_common(&a->fwd, p);
    if (rc) return rc;
    SSA_CHECK_ARG(a->dout && a->dq && a->dk && a->dv, "sparse_gather_attention_bwd: null grad");
    SSA_CHECK_ARG(a->fwd.neighbors32 == nullptr && a->fwd.neighbors != nullptr,
                  "sparse_gather_attention_bwd: needs the int64 neighbours");
    p.dout = a->dout; p.dq = a->dq; p.dk = a->dk; p.dv = a->dv;
    p.row_inv = nullptr;
    return SSA_OK;
}

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

// workspace of the deterministic backward: the per-slot weights, then (zeroed
// together) the key rows' counts and bounds, the two maxima and the sums
struct DetLayout {
    int64_t wdraw, wpw, zero_at, kcnt, kmaxd, kmaxp, gmax, acck, accv, total;
};

DetLayout det_layout(const ApplyP &p) {
    DetLayout L{};
    const int64_t slots = p.rows * p.K, keys = (int64_t)p.B * p.Hkv * p.M;
    int64_t o = 0;
    auto take = [&](int64_t bytes) { const int64_t at = o; o += align256(bytes); return at; };
    L.wdraw = take(slots * 4);
    L.wpw = take(slots * 4);
    L.zero_at = o;
    L.kcnt = take(keys * 4);
    L.kmaxd = take(keys * 4);
    L.kmaxp = take(keys * 4);
    L.gmax = take(8);
    L.acck = take(keys * p.d * 8);
    L.accv = take(keys * p.d * 8);
    L.total = o;
    return L;
}

}  // namespace

extern "C" int ssa_sparse_gather_attention_bwd(const ssa_apply_bwd_args *a, void *stream) {
    ApplyP p;
    const int rc = bwd_common(a, p);
    if (rc) return rc;
    return run_apply(p, a->fwd.q.dtype, a->fwd.d, (hipStream_t)stream, true);
}

extern "C" int64_t ssa_sparse_gather_attention_bwd_det_workspace_bytes(const ssa_apply_bwd_args *a) {
    ApplyP p;
    const int rc = bwd_common(a, p);
    if (rc) return rc;
    return det_layout(p).total;
}

extern "C" int ssa_sparse_gather_attention_bwd_det(const ssa_apply_bwd_args *a, void *workspace,
                                                   int64_t workspace_bytes, void *stream) {
    ApplyP p;
    const int rc = bwd_common(a, p);
    if (rc) return rc;
    const DetLayout L = det_layout(p);
    SSA_CHECK_ARG(workspace != nullptr && workspace_bytes >= L.total,
                  "sparse_gather_attention_bwd_det: workspace of %lld bytes, %lld needed",
                  (long long)workspace_bytes, (long long)L.total);
    SSA_CHECK_ARG((uintptr_t)workspace % 256 == 0,
                  "sparse_gather_attention_bwd_det: workspace must be 256-byte aligned");
    if (p.rows == 0) return SSA_OK;
    char *ws = (char *)workspace;
    p.wdraw = (float *)(ws + L.wdraw);
    p.wpw = (float *)(ws + L.wpw);
    p.kcnt = (uint32_t *)(ws + L.kcnt);
    p.kmaxd = (uint32_t *)(ws + L.kmaxd);
    p.kmaxp = (uint32_t *)(ws + L.kmaxp);
    p.gmax = (uint32_t *)(ws + L.gmax);
    p.acck = (unsigned long long *)(ws + L.acck);
    p.accv = (unsigned long long *)(ws + L.accv);
    const hipStream_t st = (hipStream_t)stream;
    const int64_t nz = (L.total - L.zero_at) / 4;
    hipLaunchKernelGGL(apply_zero_kernel, dim3((unsigned)std::min<int64_t>(ceil_div(nz, 256), 4096)),
                       dim3(256), 0, st, (uint32_t *)(ws + L.zero_at), nz);
    SSA_CHECK_LAUNCH();
    return run_apply(p, a->fwd.q.dtype, a->fwd.d, st, true);
}
