// ssa_proj.hip -- the q and k/v projections of SparseAttention.forward with the
// LSH hash of the graph build in their epilogue (gfx950, bf16).
//
// Replaces, for bf16 models, the projections q = x Wq^T and k, v = src Wk^T,
// src Wv^T (sparse_attention.py:1484-1486) together with the hash of the
// projected rows (`_hash_proj` / `_hash` / `_probe_ids`, :559-646, as
// `_single_round` calls them, :775-779).  One launch per projection:
//
//  * the GEMM Y = X W^T (X: token rows of d_model bf16, W: output rows of
//    d_model bf16) on v_mfma_f32_32x32x16_bf16, fp32 accumulation, one
//    round-to-nearest-even to bf16 -- the arithmetic of hipBLASLt's bf16 GEMM
//    (the result is bit-identical to torch's F.linear on the tested shapes);
//  * its epilogue takes each 16-row x head block of the rounded tile (the
//    values the rest of the build reads back from Y) and computes what the
//    separate hash / aux passes computed from a second read of q and k:
//      KEYS     bucket ids of the key rows per round (key layout) and the
//               largest |k|^2 of each 16 rows (the code scale's key norm);
//      QUERIES  bucket and probe ids per round, the query's code scale from
//               |q|^2 and the per-(batch, kv head) max |k|^2, and the aux
//               scores q.k_n (causal) and q.k_glob[j], q.k_0 with exactly the
//               rescore's arithmetic (16x16x32 k steps), so equal keys keep
//               equal scores.
//    The hyperplane projections run on v_mfma_f32_16x16x32_bf16 against the
//    fp32 hyperplanes split into three bf16 terms (hi + lo + lo2 = the fp32
//    value exactly): the products are exact and accumulate in fp32, so a
//    projection is an fp32 dot product of the bf16 row with the fp32 plane, as
//    the reference's `x.float() @ rand_proj.T` is; only the summation order
//    differs (the reference leaves it to its BLAS).  Sign rule: bit = proj > 0.
//
// Main loop: 256 (or 128) token rows x 256 output features per workgroup of 4
// waves (each 128 (64) x 128 in 32x32 blocks), k stages of 32 in four LDS
// buffers filled straight from global memory (buffer_load_dwordx4 ... lds, 16
// rows of 64 bytes per wave load, chunks XOR-swizzled by row so 8 lanes reading
// one chunk of 8 rows hit 8 bank groups), loads three stages ahead, the next
// stage's fragments read between the current stage's products, one barrier
// per stage.  Tiles go to XCDs in contiguous ranges, grouped 4 token tiles x
// the feature tiles so an XCD's L2 serves the rows its tiles share.
#include <algorithm>

#include "ssa_common.h"
#include "ssa_graph_internal.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int PJ_BK = 32;                  // k per stage
constexpr int PJ_NST = 4;                  // LDS stages
constexpr int PJ_GM = 4;                   // token tiles per tile group
constexpr int PJ_SCR = (4 * 16 * 65 + 16) * 4;   // projection rows of the 4 waves (<= 64 planes),
                                                // + 16 floats: ids read 12 values past any row start

template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

__device__ __forceinline__ f32x4_t mma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ids of one row from its projections pr[0..P-1] as ssa_write_ids computes
// them, with all 12 values read unconditionally (pr[P..11] must be readable:
// the scratch rows are padded), so the reads issue together and one wait
// covers them
__device__ __forceinline__ void pj_write_ids(const float *pr, int P, int Tp, uint16_t *o) {
    float v[12];
#pragma unroll
    for (int j = 0; j < 12; ++j) v[j] = pr[j];
#pragma unroll
    for (int j = 0; j < 12; ++j) v[j] = j < P ? v[j] : 0.f;
    int id = 0;
#pragma unroll
    for (int j = 0; j < 12; ++j) id |= (j < P && v[j] > 0.f) ? 1 << j : 0;
    o[0] = (uint16_t)id;
    int picked = 0;
    for (int t = 0; t < Tp; ++t) {
        int pos = -1;
        float best = 0.f;
#pragma unroll
        for (int j = 0; j < 12; ++j) {
            const float a = fabsf(v[j]);
            const bool take = j < P && !((picked >> j) & 1) && (pos < 0 || abs_before(a, j, best, pos));
            best = take ? a : best;
            pos = take ? j : pos;
        }
        picked |= 1 << pos;
        o[1 + t] = (uint16_t)(id ^ (1 << pos));
    }
}

// key bucket id of one row (no probes), the 12 values read unconditionally
__device__ __forceinline__ int pj_key_id(const float *pr, int P) {
    float v[12];
#pragma unroll
    for (int j = 0; j < 12; ++j) v[j] = pr[j];
    int id = 0;
#pragma unroll
    for (int j = 0; j < 12; ++j) id |= (j < P && v[j] > 0.f) ? 1 << j : 0;
    return id;
}

// The fp32 hyperplanes as three bf16 terms, zero-padded to whole 16-plane
// tiles and to the head dim: out[term][j][e], j < NT * 16, e < d.
__global__ void __launch_bounds__(256) plane_split_kernel(const float *planes, int R, int maxP, int P,
                                                          int d, int np16, uint16_t *out) {
    const int n = np16 * d;
    for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) {
        const int j = i / d, e = i % d;
        float v = 0.f;
        if (j < R * P) v = planes[((int64_t)(j / P) * maxP + (j % P)) * d + e];
        const __bf16 hi = (__bf16)v;
        const float r1 = v - (float)hi;
        const __bf16 lo = (__bf16)r1;
        const __bf16 lo2 = (__bf16)(r1 - (float)lo);
        out[i] = __builtin_bit_cast(uint16_t, hi);
        out[n + i] = __builtin_bit_cast(uint16_t, lo);
        out[2 * n + i] = __builtin_bit_cast(uint16_t, lo2);
    }
}

// ---------------------------------------------------------------------------
// Hash epilogue.  The rounded tile sits in LDS (rows of 512 bytes, 16-byte
// chunk c of row r at c ^ (r % 32)).  Its blocks are 16 rows x one head; wave
// w takes blocks w, w + 4, ... (block u: rows 16 (u % NRG) .., head slot
// u / NRG of the tile).  Lane (li, lg) holds, as the B operand of a 16x16x32
// step s, elements 32 s + 8 lg .. +7 of row li.  The global operands (the
// hyperplane terms, the keys of the aux scores) are loaded for all of a
// wave's blocks before the first block is scored, so their latency is paid
// once: one wave per SIMD has no other wave to hide it behind.
template <int BM, int MODE, int D>
struct HashEpi {
    static constexpr int KS = D / 32;              // 16x16x32 steps over a head
    static constexpr int HT = 256 / D;             // heads per tile
    static constexpr int NRG = BM / 16;            // 16-row groups per tile
    static constexpr int NSW = NRG * HT / 4;       // blocks per wave
    static constexpr int CH = NSW < 8 ? NSW : 8;   // blocks per group of prefetched keys
    static constexpr int NTM = 12 / KS < 4 ? 12 / KS : 4;   // 16-plane tiles held
    bf16x8_t pl[3][NTM][KS];                       // hyperplane terms (A operand)
    int gkey;                                      // QUERIES: glob[li] (li < G), else key 0

    __device__ __forceinline__ static bf16x8_t zero8() {
        return __builtin_bit_cast(bf16x8_t, make_uint4(0, 0, 0, 0));
    }

    // block i of wave w is block u = w + 4 i of the tile: rows 16 (u % NRG) ..,
    // head slot u / NRG (w < 4 and NRG a multiple of 4)
    __device__ __forceinline__ static int hslot(int i, int wid) { return (wid + 4 * i) / NRG; }
    __device__ __forceinline__ static int rgrp(int i, int wid) { return (wid + 4 * i) % NRG; }

    // after the main loop (its fragment registers are dead): the hyperplane terms
    __device__ __forceinline__ void prefetch(const ProjP &p, int lane) {
        const int li = lane & 15, lg = lane >> 4;
        const int NT = (p.R * p.P + 15) / 16;
        const int np16 = NT * 16;
#pragma unroll
        for (int c = 0; c < 3; ++c)
#pragma unroll
            for (int t = 0; t < NTM; ++t)
#pragma unroll
                for (int s = 0; s < KS; ++s)
                    pl[c][t][s] = t < NT ? *reinterpret_cast<const bf16x8_t *>(
                                               p.psplit + ((int64_t)c * np16 + 16 * t + li) * D + 32 * s + 8 * lg)
                                         : zero8();
        if constexpr (MODE == SSA_PROJ_QUERIES) gkey = li < p.G ? (int)p.glob[li] : 0;
    }

    // QUERIES: for the CH blocks from block i0 of this wave, the key rows of the
    // aux scores (each row's own key when causal, glob[li] / key 0) and the key
    // norm of the block's (batch, kv head).  A block's 16 rows share a batch
    // (L % 16 == 0), so its batch and first position are wave-uniform.
    __device__ __forceinline__ void load_keys(const ProjP &p, int m0, int n0, int wid, int lane, int i0,
                                              int key, bf16x8_t (&ks)[CH][KS], bf16x8_t (&kg)[CH][KS],
                                              float (&kn)[CH]) {
        const int li = lane & 15, lg = lane >> 4;
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            // every load is in bounds (blocks past the rows read block 0's, non-causal
            // rows read key 0), so none waits behind a branch
            const int i = i0 + j;
            const int grow0 = m0 + 16 * rgrp(i, wid);
            const int gi = i < NSW && grow0 < p.rows ? grow0 : 0;
            const int g = (n0 / D + hslot(i, wid)) / p.rep;
            const int b = gi / p.L;
            const int n = p.causal ? min(gi % p.L + li, p.Lk - 1) : 0;
            const bf16_t *kb = (const bf16_t *)p.k + b * p.ksb + g * p.ksh;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                ks[j][s] = *reinterpret_cast<const bf16x8_t *>(kb + (int64_t)n * p.ksn + 32 * s + 8 * lg);
                kg[j][s] = *reinterpret_cast<const bf16x8_t *>(kb + (int64_t)key * p.ksn + 32 * s + 8 * lg);
            }
            kn[j] = __uint_as_float(p.knorm[b * p.Hkv + g]);
        }
    }

    // one 16-row x head block: ids (and for queries the aux row) from the tile
    __device__ __forceinline__ void block(const ProjP &p, unsigned char *sm, float *pw, int pst, int m0,
                                          int n0, int wid, int lane, int i, const bf16x8_t *ksb,
                                          const bf16x8_t *kgb, float knorm) {
        const int li = lane & 15, lg = lane >> 4;
        const int NT = (p.R * p.P + 15) / 16;
        const int rg = rgrp(i, wid), hl = hslot(i, wid);
        const int hh = n0 / D + hl;                  // head index in the output
        const int grow0 = m0 + 16 * rg;              // global token row of the block
        if (MODE == SSA_PROJ_KEYS && hh >= p.heads) return;    // value columns
        if (grow0 >= p.rows) return;                 // rows % 16 == 0: whole blocks only
        const int b = grow0 / p.L, n0r = grow0 % p.L;
        bf16x8_t qa[KS];
        {
            const int r = 16 * rg + li;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const int ch = (hl * D + 32 * s + 8 * lg) / 8;
                qa[s] = *reinterpret_cast<const bf16x8_t *>(sm + r * 512 + ((ch ^ (r & 31)) * 16));
            }
        }
        // |x|^2 of row li (lanes lg hold quarters of it)
        float x2 = 0.f;
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v = (float)qa[s][e];
                x2 = fmaf(v, v, x2);
            }
        x2 += __shfl_xor(x2, 16, SSA_WAVE);
        x2 += __shfl_xor(x2, 32, SSA_WAVE);
        // Projections as Q . planes^T: lane (li, lg) receives row 4 lg + r, plane
        // 16 t + li in acc[t][r] (the three terms of a plane in turn, the
        // smaller ones last).  ballot(acc[t][r] > 0) holds, in bits 16 lg' ..
        // 16 lg' + 15, the signs of planes 16 t .. 16 t + 15 of row 4 lg' + r.
        f32x4_t acc[NTM];
#pragma unroll
        for (int t = 0; t < NTM; ++t) {
            acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
            if (t < NT) {
#pragma unroll
                for (int c = 0; c < 3; ++c)
#pragma unroll
                    for (int s = 0; s < KS; ++s) acc[t] = mma16(qa[s], pl[c][t][s], acc[t]);
            }
        }
        // sign bits of every plane of row li (bit j = proj_j > 0), built from
        // the ballots: the row's 16-bit field of each tile's mask for r = li % 4
        uint64_t rowbits = 0;
#pragma unroll
        for (int t = 0; t < NTM; ++t) {
            if (t < NT) {
                uint64_t m = 0;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint64_t b = wave_ballot(acc[t][r] > 0.f);
                    m = (li & 3) == r ? b : m;
                }
                rowbits |= ((m >> (16 * (li >> 2))) & 0xffffull) << (16 * t);
            }
        }
        if constexpr (MODE == SSA_PROJ_KEYS) {
            // key layout: id of key n of (batch, kv head) hh in round r at
            // ids[((b * heads + hh) * R + r) * L + n]; lane (li, lg) takes rounds
            // lg, lg + 4, ...
            const int64_t bk = (int64_t)b * p.heads + hh;
            const uint32_t pm = (1u << p.P) - 1u;
            for (int r = lg; r < p.R; r += 4)
                p.ids[(bk * p.R + r) * p.L + n0r + li] = (uint16_t)((rowbits >> (r * p.P)) & pm);
            // largest |k|^2 of the 16 rows (non-negative floats order as bits)
            const uint32_t mx = wave_max_u(__float_as_uint(x2));
            if (lane == 0) p.kpart[(bk * p.L + n0r) / 16] = mx;
        } else {
            // query layout: ids[((bh * L + n) * R + r) * NS + t]
            const int64_t bh = (int64_t)b * p.Hq + hh;
            const uint32_t pm = (1u << p.P) - 1u;
            if (p.Tp == 0) {
                for (int r = lg; r < p.R; r += 4)
                    p.ids[((bh * p.L + n0r + li) * p.R + r) * p.NS] = (uint16_t)((rowbits >> (r * p.P)) & pm);
            } else {
                // probes rank |proj| within a round: the projections go through
                // this wave's LDS rows, one (row, round) pair per lane
#pragma unroll
                for (int t = 0; t < NTM; ++t)
                    if (t < NT)
#pragma unroll
                        for (int r = 0; r < 4; ++r) pw[(4 * lg + r) * pst + 16 * t + li] = acc[t][r];
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                for (int x0 = 0; x0 < 16 * p.R; x0 += SSA_WAVE) {
                    const int x = x0 + lane;
                    const int rl = x / p.R, r = x - rl * p.R;
                    if (rl < 16)
                        pj_write_ids(pw + rl * pst + r * p.P, p.P, p.Tp,
                                     p.ids + ((bh * p.L + n0r + rl) * p.R + r) * p.NS);
                }
            }
            // aux row (bh, n): q.k_n (causal), q.k_glob[0..G-1], q.k_0, code scale
            const int g = hh / p.rep;
            float *ob = p.aux + (bh * p.L + n0r) * p.NA;
            if (lg == 0)
                ob[(int64_t)li * p.NA + p.NA - 1] = code_scale(x2, knorm);
            if (p.causal) {
                // key row li is key n0r + li: the diagonal is q_n . k_n
                f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < KS; ++s) sc = mma16(ksb[s], qa[s], sc);
#pragma unroll
                for (int rr = 0; rr < 4; ++rr)
                    if (4 * lg + rr == li) ob[(int64_t)li * p.NA] = sc[rr];
            }
            for (int j0 = 0; j0 <= p.G; j0 += 16) {   // key rows glob[0..G-1], then key 0
                bf16x8_t kb[KS];
                if (j0 == 0) {
#pragma unroll
                    for (int s = 0; s < KS; ++s) kb[s] = kgb[s];
                } else {
                    const int j = j0 + li;
                    const int key = j < p.G ? (int)p.glob[j] : 0;
                    const bf16_t *kr = (const bf16_t *)p.k + b * p.ksb + g * p.ksh + (int64_t)key * p.ksn;
#pragma unroll
                    for (int s = 0; s < KS; ++s) kb[s] = *reinterpret_cast<const bf16x8_t *>(kr + 32 * s + 8 * lg);
                }
                f32x4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < KS; ++s) sc = mma16(kb[s], qa[s], sc);
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int jj = j0 + 4 * lg + rr;
                    if (jj <= p.G) ob[(int64_t)li * p.NA + 1 + jj] = sc[rr];
                }
            }
        }
        // this wave's projection rows are rewritten by its next block
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // After the tile went to LDS: the keys of the first group of blocks are
    // loaded, then `store` (the tile's global store) runs while they arrive,
    // then the blocks; each later group's keys are loaded before it.
    template <typename Store>
    __device__ __forceinline__ void run(const ProjP &p, unsigned char *sm, int m0, int n0, int wid,
                                        int lane, Store store) {
        const int NT = (p.R * p.P + 15) / 16;
        const int pst = NT * 16 + 1;
        float *pw = reinterpret_cast<float *>(sm + BM * 512) + wid * 16 * pst;
        bf16x8_t ks[CH][KS], kg[CH][KS];
        float kn[CH];
        if constexpr (MODE == SSA_PROJ_QUERIES) load_keys(p, m0, n0, wid, lane, 0, gkey, ks, kg, kn);
        store();
        if (p.zero1 && blockIdx.x == 0 && threadIdx.x == 0) *p.zero1 = 0;
        for (int i0 = 0; i0 < NSW; i0 += CH) {
            if (MODE == SSA_PROJ_QUERIES && i0 > 0) load_keys(p, m0, n0, wid, lane, i0, gkey, ks, kg, kn);
#pragma unroll
            for (int j = 0; j < CH; ++j)
                block(p, sm, pw, pst, m0, n0, wid, lane, i0 + j, ks[j], kg[j], kn[j]);
        }
    }
};

// ---------------------------------------------------------------------------
template <int BM, int MODE, int D>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
proj_kernel(ProjP p) {
    constexpr int RB = PJ_BK * 2;                  // LDS row bytes of a stage
    constexpr int ABYTES = BM * RB, SB = (BM + 256) * RB;
    constexpr int LA = ABYTES / 4096, LB = 256 * RB / 4096;    // wave loads per stage and wave
    constexpr int PER_STAGE = LA + LB;
    constexpr int RPL = 16;                        // rows per 1 KB wave load
    constexpr int TM = BM / 64;                    // 32-row blocks per wave
    constexpr int KS = PJ_BK / 16;                 // k16 steps per stage
    constexpr int EPI = BM * 512 + (MODE == SSA_PROJ_PLAIN ? 0 : PJ_SCR);
    constexpr int SMB = PJ_NST * SB > EPI ? PJ_NST * SB : EPI;
    __shared__ __align__(1024) unsigned char sm[SMB];
    const int tid = threadIdx.x;
    const int wid = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63;
    const int wm = wid >> 1, wn = wid & 1;
    const int ntm = (p.rows + BM - 1) / BM, ntn = p.cols / 256;
    const int ntiles = ntm * ntn;
    // XCD-contiguous tile ranges (the dispatcher sends block i to XCD i % 8),
    // tiles ordered in groups of PJ_GM token tiles x all feature tiles
    const int per = (ntiles + 7) / 8;
    const int L = (blockIdx.x % 8) * per + blockIdx.x / 8;
    if (L >= ntiles) return;
    const int gfull = PJ_GM * ntn;
    const int grp = L / gfull;
    const int fm = grp * PJ_GM;
    const int gm = min(PJ_GM, ntm - fm);
    const int inner = L - grp * gfull;
    const int mt = fm + inner % gm, nt = inner / gm;
    const int m0 = mt * BM, n0 = nt * 256;
    const int mrows = min(BM, p.rows - m0);
    // buffer resources over the tile's rows: loads past them return zeros
    const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const uint16_t *)p.x + (int64_t)m0 * p.ldx), (short)0,
        (int)((int64_t)mrows * p.ldx * 2), SSA_BUF_FLAGS);
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        (void *)((const uint16_t *)p.w + (int64_t)n0 * p.ldw), (short)0,
        (int)((int64_t)256 * p.ldw * 2), SSA_BUF_FLAGS);
    // chunk c of LDS stage row r holds global chunk c ^ ((r / 2) % 4): 8 lanes
    // reading one chunk of 8 consecutive rows hit 8 different bank groups
    auto key = [](int r) { return (r >> 1) & 3; };
    const int lr = lane >> 2;
    const int lc = (lane & 3) ^ key(lr);
    const uint32_t vx = (uint32_t)(((LA * RPL * wid + lr) * p.ldx + 8 * lc) * 2);
    const uint32_t vw = (uint32_t)(((LB * RPL * wid + lr) * p.ldw + 8 * lc) * 2);
    const uint32_t sx = (uint32_t)(RPL * p.ldx * 2), sw = (uint32_t)(RPL * p.ldw * 2);
    auto stage = [&](int st, int k0) __attribute__((always_inline)) {
        unsigned char *sb = sm + st * SB;
#pragma unroll
        for (int t = 0; t < LA; ++t)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void_t *)(sb + 1024 * (LA * wid + t)), 16,
                                                     vx, k0 * 2 + t * sx, 0, 0);
#pragma unroll
        for (int t = 0; t < LB; ++t)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_void_t *)(sb + ABYTES + 1024 * (LB * wid + t)),
                                                     16, vw, k0 * 2 + t * sw, 0, 0);
    };
    f32x16_t acc[4][TM];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    // 32x32x16 operands: lane l gives row l % 32 with k 8 (l / 32) .. +7 of the step
    const int fr = lane & 31, fh = lane >> 5;
    uint32_t fx[KS], fw[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        fx[s] = (uint32_t)((BM / 2 * wm + fr) * RB + (((2 * s + fh) ^ key(fr)) * 16));
        fw[s] = (uint32_t)(ABYTES + (128 * wn + fr) * RB + (((2 * s + fh) ^ key(fr)) * 16));
    }
    bf16x8_t xf[2][KS][TM], wf[2][KS][4];
    auto rd = [&](int st, int b) __attribute__((always_inline)) {
        const unsigned char *sb = sm + st * SB;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
#pragma unroll
            for (int j = 0; j < TM; ++j)
                xf[b][s][j] = *reinterpret_cast<const bf16x8_t *>(sb + fx[s] + 32 * RB * j);
#pragma unroll
            for (int i = 0; i < 4; ++i)
                wf[b][s][i] = *reinterpret_cast<const bf16x8_t *>(sb + fw[s] + 32 * RB * i);
        }
    };
    auto mm = [&](int b) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[b][s][i], xf[b][s][j], acc[i][j],
                                                                        0, 0, 0);
    };
    const int nk = p.K / PJ_BK;                    // even (K % 64 == 0)
    constexpr int NMF = KS * 4 * TM;               // MFMAs per stage and wave
    constexpr int NRD = KS * (4 + TM);             // fragment reads per stage and wave
#pragma unroll
    for (int s = 0; s < PJ_NST - 1; ++s) stage(s, PJ_BK * min(s, nk - 1));
    // stage 0 landed; the stages after it may stay in flight
    wait_vm<(PJ_NST - 2) * PER_STAGE>();
    asm volatile("s_barrier" ::: "memory");
    rd(0, 0);
    // Stage k: its products (fragment set k % 2) with the fragment reads of stage
    // k + 1 and the loads of stage k + 3 (into the buffer of stage k - 1, whose
    // reads ended before this stage's barrier) spread between them.  Past the
    // last stage the loads repeat the last stage into buffers no longer read and
    // the reads fill registers no longer used: no branches, so the reads and
    // loads interleave with the products.
    for (int kt = 0; kt < nk; kt += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int k = kt + u;
            __builtin_amdgcn_sched_barrier(0);
            // stage k + 1 landed (stage k + 2's loads may stay in flight)
            asm volatile("" ::: "memory");
            wait_vm<PER_STAGE>();
            asm volatile("s_barrier" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
            rd((k + 1) % PJ_NST, u ^ 1);
            stage((k + PJ_NST - 1) % PJ_NST, PJ_BK * min(k + PJ_NST - 1, nk - 1));
            mm(u);
#pragma unroll
            for (int q = 0; q < NRD; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
#pragma unroll
            for (int q = 0; q < PER_STAGE; ++q) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            }
            // (128-row tiles have fewer products than reads + loads: the last
            // groups then take what is left)
            __builtin_amdgcn_sched_group_barrier(0x008, NMF > NRD + PER_STAGE ? NMF - NRD - PER_STAGE : 0,
                                                 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt vmcnt(0)\n s_barrier" ::: "memory");
    HashEpi<BM, MODE, D> epi;
    if constexpr (MODE != SSA_PROJ_PLAIN) epi.prefetch(p, lane);
    // The tile rounded to bf16 (round to nearest even) into LDS: rows of 512
    // bytes, 16-byte chunk c of row r at c ^ (r % 32).  Lane l of block (i, j)
    // holds row 32 j + l % 32 and features 32 i + 8 g + 4 (l / 32) + 0..3 in
    // accumulators 4 g .. 4 g + 3.
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int row = BM / 2 * wm + 32 * j + fr;
                const int ch = 16 * wn + 4 * i + g;
                const f2_t v0 = {acc[i][j][4 * g], acc[i][j][4 * g + 1]};
                const f2_t v1 = {acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
                const uint32_t lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(v0, bf16x2_t));
                const uint32_t hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(v1, bf16x2_t));
                *reinterpret_cast<uint2 *>(sm + row * 512 + ((ch ^ (row & 31)) * 16) + fh * 8) =
                    make_uint2(lo, hi);
            }
    __syncthreads();
    uint16_t *Y = (uint16_t *)p.y;
    auto store = [&]() __attribute__((always_inline)) {
#pragma unroll 4
        for (int it = 0; it < BM / 8; ++it) {
            const int idx = it * 256 + tid;
            const int row = idx >> 5, c = idx & 31;
            const uint4 v = *reinterpret_cast<const uint4 *>(sm + row * 512 + ((c ^ (row & 31)) * 16));
            if (row < mrows) *reinterpret_cast<uint4 *>(Y + (int64_t)(m0 + row) * p.ldy + n0 + 8 * c) = v;
        }
    };
    if constexpr (MODE == SSA_PROJ_PLAIN) store();
    else epi.run(p, sm, m0, n0, wid, lane, store);
}

template <int BM, int MODE>
int launch_bm_mode(const ProjP &p, hipStream_t st) {
    const int ntiles = ((p.rows + BM - 1) / BM) * (p.cols / 256);
    const dim3 grid((unsigned)(8 * ((ntiles + 7) / 8)));
#define SSA_PJ(DD) hipLaunchKernelGGL((proj_kernel<BM, MODE, DD>), grid, dim3(256), 0, st, p)
    if (MODE == SSA_PROJ_PLAIN) SSA_PJ(128);
    else if (p.d == 32) SSA_PJ(32);
    else if (p.d == 64) SSA_PJ(64);
    else SSA_PJ(128);
#undef SSA_PJ
    SSA_CHECK_LAUNCH();
    return SSA_OK;
}

}  // namespace

bool ssa_project_supported(int rows, int cols, int K, int d, int np) {
    // the epilogue holds at most 12 / (d / 32) (and 4) tiles of 16 hyperplanes
    const int nt = (np + 15) / 16, ntm = std::min(4, 12 / (d / 32));
    return rows >= 1 && rows % 16 == 0 && cols % 256 == 0 && K >= 64 && K % 64 == 0 &&
           (d == 32 || d == 64 || d == 128) && np >= 1 && nt <= ntm &&
           (int64_t)256 * K * 2 < ((int64_t)1 << 31);
}

int64_t ssa_plane_split_bytes(int np, int d) { return (int64_t)3 * ((np + 15) / 16 * 16) * d * 2; }

int ssa_launch_plane_split(const float *planes, int R, int maxP, int P, int d, uint16_t *out,
                           hipStream_t st) {
    const int np16 = (R * P + 15) / 16 * 16;
    const int n = np16 * d;
    hipLaunchKernelGGL(plane_split_kernel, dim3((unsigned)std::min(64, (n + 255) / 256)), dim3(256), 0,
                       st, planes, R, maxP, P, d, np16, out);
    SSA_CHECK_LAUNCH();
    return SSA_OK;
}

int ssa_launch_project(const ProjP &p, hipStream_t st) {
    SSA_CHECK_ARG(p.x && p.w && p.y, "project: null operand");
    SSA_CHECK_ARG(p.rows >= 1 && p.cols % 256 == 0 && p.K % 64 == 0 && p.ldx >= p.K && p.ldw >= p.K &&
                      p.ldy >= p.cols,
                  "project: rows %d, cols %d, K %d, ldx %lld, ldw %lld, ldy %lld", p.rows, p.cols, p.K,
                  (long long)p.ldx, (long long)p.ldw, (long long)p.ldy);
    SSA_CHECK_ARG((int64_t)256 * p.ldx * 2 < ((int64_t)1 << 31) &&
                      (int64_t)256 * p.ldw * 2 < ((int64_t)1 << 31),
                  "project: a tile's rows exceed 2 GiB");
    if (p.mode != SSA_PROJ_PLAIN) {
        SSA_CHECK_ARG(ssa_project_supported(p.rows, p.cols, p.K, p.d, p.R * p.P) && p.L >= 16 &&
                          p.L % 16 == 0 && p.rows % p.L == 0 && p.ids && p.psplit && p.P <= 12,
                      "project: hash epilogue for rows %d, L %d, d %d, %d planes", p.rows, p.L, p.d,
                      p.R * p.P);
        SSA_CHECK_ARG(p.mode == SSA_PROJ_KEYS ? (p.kpart != nullptr && p.heads * p.d <= p.cols)
                                               : (p.k && p.aux && p.knorm && p.rep >= 1 &&
                                                  p.Hq * p.d == p.cols && (p.G == 0 || p.glob)),
                      "project: epilogue operands");
    }
    // 256 feature tiles on all CUs: 256-row tiles when they give the chip at
    // least one tile per CU, else 128-row tiles
    const int64_t t256 = (int64_t)((p.rows + 255) / 256) * (p.cols / 256);
    const bool big = t256 >= 256;
    switch (p.mode) {
        case SSA_PROJ_PLAIN:
            return big ? launch_bm_mode<256, SSA_PROJ_PLAIN>(p, st) : launch_bm_mode<128, SSA_PROJ_PLAIN>(p, st);
        case SSA_PROJ_KEYS:
            return big ? launch_bm_mode<256, SSA_PROJ_KEYS>(p, st) : launch_bm_mode<128, SSA_PROJ_KEYS>(p, st);
        case SSA_PROJ_QUERIES:
            return big ? launch_bm_mode<256, SSA_PROJ_QUERIES>(p, st)
                       : launch_bm_mode<128, SSA_PROJ_QUERIES>(p, st);
    }
    ssa_set_error("project: mode %d", p.mode);
    return SSA_E_ARG;
}
