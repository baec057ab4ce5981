// ssa_graph.hip -- neighbor-graph build for SparseAttention on gfx950.
//
// Replaces SparseAttention.build_graph (sparse_attention.py:1325-1390) and
// LSHGraphBuilder.forward (:814-959).  Pipeline per call:
//
//  1. hash_kernel      fp32 projections of every q row (B*Hq*N) and every
//                      UN-expanded k row (B*Hkv*M) on the first P planes of
//                      each round; bit j = (proj_j > 0) (+0, -0, NaN -> 0),
//                      plane j = bit j; probe t flips the t-th least |proj|
//                      bit of the base id (ties by plane order) (:575-646).
//  2. bucket sort      introsort-exact permutation per (kv head, round), see
//                      ssa_sort.hip (:781-792).  Shared by the kv_rep query
//                      heads of a GQA group.
//  3. query bucketing  counting sort of the N queries of each (head, round,
//                      id set) by bucket id, and a tile list of up to 64
//                      queries that share one bucket.
//  4. rescore          a query's candidate list depends only on its bucket
//                      (:668-696): the C candidate rows of bucket u are scored
//                      against up to 64 queries of the bucket per tile (MFMA
//                      for 16-bit inputs, fp32 fma chains otherwise; q.k
//                      unscaled, :909-916).  Scores go to S[row][slot], slot =
//                      stream position.  aux_*_kernel scores, with the same
//                      arithmetic, the keys the lists do not carry: the query
//                      itself (causal substitution) and glob ++ 0.
//  5. select_kernel    one wavefront per query walks its candidate stream in
//                      the reference's concatenation order (round, id set,
//                      slot, :869-877) with a seen-bitmap of M bits in LDS:
//                      a slot is kept iff valid and its key was not met at an
//                      earlier stream position, valid or not (:884-890);
//                      causal future keys become the query itself (:698-709);
//                      empty buckets read glob ++ 0 (:711-737).  The kept
//                      scores above a running lower bound are buffered in LDS
//                      and the exact kk-th is found by a bitwise search of
//                      the order-preserving score keys.  Slots without a
//                      candidate take glob[t] / 0 by position (:948-957).
//                      FULL mode then merges window, globals and the LSH set
//                      into a key bitmap and reads it out in ascending order
//                      (:966-1089).
//  6. topk_replay      rows whose result depends on the order of equal scores
//                      (a tied kk-th score; in LSH mode any equal selected
//                      scores) are rebuilt and run through an exact replay of
//                      the reference's chunked nth_element + sort (:904-922).
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <type_traits>

#include "ssa_common.h"
#include "ssa_graph_internal.h"
#include "ssa_sort_dev.h"

// ------------------------------------------------------------------ checked build
// Built with SSA_CHECKED (`make checked`: libssa_amd_checked.so), the
// data-dependent indices of the select, tie replay and merge paths are
// compared with the length of what they index: key ids with the key count,
// list and bucket positions with the sorted arrays, tie rows with the row
// count, output slots with the output.  An index outside is recorded in
// ssa_oob (word 0: one bit per site; words 1-3: the last offender's site,
// index and length) and replaced by 0, so no access leaves its buffer; the
// host reads and clears the record with ssa_checked_oob.  The product build
// compiles SSA_IDX to the index itself.
#ifdef SSA_CHECKED
static __device__ uint32_t ssa_oob[4];
__device__ __attribute__((noinline)) int64_t ssa_idx_bad(int64_t i, int64_t n, int site) {
    atomicOr(&ssa_oob[0], 1u << site);
    ssa_oob[1] = (uint32_t)site;
    ssa_oob[2] = (uint32_t)i;
    ssa_oob[3] = (uint32_t)n;
    return 0;
}
__device__ __forceinline__ int64_t ssa_idx(int64_t i, int64_t n, int site) {
    return (i >= 0 && i < n) ? i : ssa_idx_bad(i, n, site);
}
#define SSA_IDX(i, n, site) ssa_idx((int64_t)(i), (int64_t)(n), (site))
#else
#define SSA_IDX(i, n, site) (i)
#endif

namespace {

constexpr int TQ = 64;         // queries per rescore tile
constexpr int TC = 64;         // candidates per rescore sub-tile
constexpr int SEL_WAVES = 4;   // waves per select workgroup

struct Dims {
    int B, Hq, Hkv, rep, N, M, d, R, maxP, P, Tp, NS, NB, C, CPL, nlists, G, kk, Kw, Kout;
    int64_t Call, BH, BK;
    int nbh_chunk;
    int chunk;         // width of the reference's running top-k chunks (:903)
    int Cs;            // score row stride: min(C, M) rounded up to 64 members
    int rpw_blocks;    // blocks of the workgroup tie replay (0: the per-wave replay)
    int rpw_nsim;      // its replaying waves per block
    int rp_glb_blocks; // blocks of the per-wave replay when its arrays live in the workspace
    int ctab;          // the list sort writes the cut's rank table (causal only)
    int fused;         // the projections hashed the rows (ssa_project_build_graph): no
                       // hash or aux pass, aux rows for every head, split hyperplanes
    int cbits;         // width of the cut entries' size and cutoff fields
    int swaves;        // rows (waves) per select workgroup, as many as its LDS allows
};

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------ hashing
struct HashP {
    const void *x;
    int64_t sb, sh, sn;
    int nh, L, d;
    const float *planes;
    int R, maxP, P, Tp, NS;
    const float *inj;
    uint16_t *out;
    int key_layout;
    int vec16;          // rows 16-byte aligned: quarter rows load with 16-byte loads
    int64_t rows;
    int pl16;           // planes 16-byte aligned with d % 4 == 0: planes load with 16-byte loads
    uint32_t *zero;     // block 0 clears zero[0..nzero) and *zero1 (later kernels'
    int nzero;          // accumulator and counter; either may be null)
    int32_t *zero1;
    uint32_t *kpart;    // key hash: max |k|^2 of each 16-row tile as float bits, or null
};

__device__ __forceinline__ void hash_clear(const HashP &p) {
    if (blockIdx.x == 0) {
        for (int i = threadIdx.x; i < p.nzero; i += blockDim.x) p.zero[i] = 0u;
        if (p.zero1 && threadIdx.x == 0) *p.zero1 = 0;
    }
}

template <typename T>
__global__ void __launch_bounds__(256) hash_kernel(HashP p) {
    hash_clear(p);
    const int64_t row = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= p.rows) return;
    const int i = (int)(row % p.L);
    const int64_t bh = row / p.L;
    const int h = (int)(bh % p.nh);
    const int64_t b = bh / p.nh;
    const T *x = (const T *)p.x + b * p.sb + h * p.sh + (int64_t)i * p.sn;
    for (int r = 0; r < p.R; ++r) {
        float pr[12];
#pragma unroll
        for (int j = 0; j < 12; ++j) pr[j] = 0.f;
        if (p.inj) {
            const float *ip = p.inj + ((bh * p.R + r) * p.L + i) * p.P;
            for (int j = 0; j < p.P; ++j) pr[j] = ip[j];
        } else {
            const float *pl = p.planes + (int64_t)r * p.maxP * p.d;
            for (int e = 0; e < p.d; ++e) {
                const float xv = to_f32(x[e]);
#pragma unroll
                for (int j = 0; j < 12; ++j)
                    if (j < p.P) pr[j] = fmaf(xv, pl[j * p.d + e], pr[j]);
            }
        }
        int id = 0;
#pragma unroll
        for (int j = 0; j < 12; ++j)
            if (j < p.P && pr[j] > 0.f) id |= 1 << j;
        if (p.key_layout) {
            p.out[(bh * p.R + r) * p.L + i] = (uint16_t)id;
        } else {
            uint16_t *o = p.out + ((bh * p.L + i) * p.R + r) * p.NS;
            o[0] = (uint16_t)id;
            if (p.Tp > 0) {
                int ord[12];
#pragma unroll
                for (int j = 0; j < 12; ++j) ord[j] = 0;
                for (int j = 0; j < p.P; ++j) {       // stable rank of |proj_j|
                    const float aj = fabsf(pr[j]);
                    int rank = 0;
                    for (int q = 0; q < p.P; ++q) {
                        const float aq = fabsf(pr[q]);
                        rank += (aq < aj) || (aq == aj && q < j);
                    }
                    for (int t = 0; t < 12; ++t)
                        if (t == rank) ord[t] = j;
                }
                for (int t = 0; t < p.Tp; ++t) {
                    int pos = 0;
#pragma unroll
                    for (int q = 0; q < 12; ++q)
                        if (q == t) pos = ord[q];
                    o[1 + t] = (uint16_t)(id ^ (1 << pos));
                }
            }
        }
    }
}

// Projection on the matrix cores: v_mfma_f32_16x16x4f32 computes a 16 x 16 block
// of rows x planes, lane l feeding row (l % 16) and plane (l % 16) with the
// element k = l / 16 of the step.  The reduction over the head dim is split so
// that lane group g = l / 16 walks the contiguous quarter [g*d/4, (g+1)*d/4):
// every lane loads its quarter row once with wide loads, and quarter lg of
// plane 16 t + li straight from global memory into registers (the planes are
// L2-resident after the first waves): no staging loop and no barrier precede
// the products.  Each wavefront takes one tile of 16 rows.  D is the
// instance's head dim; the rows' own d <= D: elements past d are zero in the
// rows and the planes.
template <typename T, int D>
__global__ void __launch_bounds__(256) hash_mfma_kernel(HashP p) {
    constexpr int DQ = D / 4;
    constexpr int CH = DQ < 32 ? DQ : 32;             // plane elements loaded per group
    extern __shared__ float hs[];
    const int NP = p.R * p.P;
    const int NT = (NP + 15) / 16;
    float *proj = hs;                                 // [4 waves][16][NT*16 + 1]
    const int pst = NT * 16 + 1;
    hash_clear(p);
    const int wid = threadIdx.x / SSA_WAVE;
    const int lane = lane_id();
    const int li = lane % 16, lg = lane / 16;
    {
        // the block's 4 waves take adjacent 16-row tiles
        const int64_t row0 = ((int64_t)blockIdx.x * 4 + wid) * 16;
        if (row0 >= p.rows) return;
        const int64_t row = row0 + li;
        float xs[DQ];
        if (row < p.rows) {
            const int i = (int)(row % p.L);
            const int64_t bh = row / p.L;
            const T *x = (const T *)p.x + (bh / p.nh) * p.sb + (bh % p.nh) * p.sh + (int64_t)i * p.sn +
                         lg * DQ;
            const int dq = p.d - lg * DQ;             // this quarter's elements below d
            constexpr int PER16 = 16 / (int)sizeof(T);
            if constexpr (DQ % PER16 == 0) {
                if (p.vec16) {
                    // d fills whole 16-byte pieces (a multiple of PER16)
#pragma unroll
                    for (int e0 = 0; e0 < DQ; e0 += PER16) {
                        uint4 w = make_uint4(0, 0, 0, 0);
                        if (e0 < dq) w = *reinterpret_cast<const uint4 *>(x + e0);
                        const T *tv = reinterpret_cast<const T *>(&w);
#pragma unroll
                        for (int e = 0; e < PER16; ++e) xs[e0 + e] = to_f32(tv[e]);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < DQ; ++e) xs[e] = e < dq ? to_f32(x[e]) : 0.f;
                }
            } else {
#pragma unroll
                for (int e = 0; e < DQ; ++e) xs[e] = e < dq ? to_f32(x[e]) : 0.f;
            }
        } else {
#pragma unroll
            for (int e = 0; e < DQ; ++e) xs[e] = 0.f;
        }
        if (p.kpart) {
            // |k|^2 of the tile's rows (lane groups hold quarters; rows past the
            // end are 0), maximised over the tile: non-negative floats order as
            // their bit patterns
            float s2 = 0.f;
#pragma unroll
            for (int e = 0; e < DQ; ++e) s2 = fmaf(xs[e], xs[e], s2);
            s2 += __shfl_xor(s2, 16, SSA_WAVE);
            s2 += __shfl_xor(s2, 32, SSA_WAVE);
            const uint32_t m = wave_max_u(__float_as_uint(s2));
            if (lane == 0) p.kpart[row0 / 16] = m;
        }
        float *pw = proj + wid * 16 * pst;
        const int dq = p.d - lg * DQ;                 // this quarter's elements below d
        for (int t = 0; t < NT; ++t) {
            // plane j = 16 t + li: round j / P, hash j % P; zero past the R*P planes
            const int j = t * 16 + li;
            const bool real = j < NP;
            const float *wr =
                p.planes + (real ? ((int64_t)(j / p.P) * p.maxP + (j % p.P)) * p.d : 0) + lg * DQ;
            f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s0 = 0; s0 < DQ; s0 += CH) {
                float wv[CH];
                bool wide = false;
                if constexpr (CH % 4 == 0) {
                    // 16-byte aligned rows of a multiple of 4 floats: a piece
                    // starting below d lies wholly below it
                    wide = p.pl16 != 0;
                    if (wide) {
#pragma unroll
                        for (int u = 0; u < CH; u += 4) {
                            float4 w = make_float4(0.f, 0.f, 0.f, 0.f);
                            if (real && s0 + u < dq) w = *reinterpret_cast<const float4 *>(wr + s0 + u);
                            wv[u] = w.x; wv[u + 1] = w.y; wv[u + 2] = w.z; wv[u + 3] = w.w;
                        }
                    }
                }
                if (!wide) {
#pragma unroll
                    for (int u = 0; u < CH; ++u) wv[u] = (real && s0 + u < dq) ? wr[s0 + u] : 0.f;
                }
#pragma unroll
                for (int u = 0; u < CH; ++u)
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xs[s0 + u], wv[u], acc, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) pw[(4 * lg + r) * pst + t * 16 + li] = acc[r];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (p.key_layout) {
            // one (round, row) pair per lane, the 16 rows of a round on
            // consecutive lanes (consecutive ids in the key layout)
            for (int x0 = 0; x0 < 16 * p.R; x0 += SSA_WAVE) {
                const int x = x0 + lane;
                const int r = x / 16, rl = x % 16;
                const int64_t rw = row0 + rl;
                if (r < p.R && rw < p.rows) {
                    const float *pr = pw + rl * pst + r * p.P;
                    int id = 0;
                    for (int j = 0; j < p.P; ++j)
                        if (pr[j] > 0.f) id |= 1 << j;
                    p.out[((rw / p.L) * p.R + r) * p.L + rw % p.L] = (uint16_t)id;
                }
            }
        } else {
            // query layout: one (row, round) pair per lane, in the ids' memory
            // order (row-major over the tile's rows, then rounds)
            for (int x0 = 0; x0 < 16 * p.R; x0 += SSA_WAVE) {
                const int x = x0 + lane;
                const int rl = x / p.R, r = x - rl * p.R;
                if (rl < 16 && row0 + rl < p.rows)
                    ssa_write_ids(pw + rl * pst + r * p.P, p.P, p.Tp, p.out + ((row0 + rl) * p.R + r) * p.NS);
            }
        }
    }
}

// ------------------------------------------------------------------ small utilities
__global__ void fill_i32_kernel(int32_t *p, int64_t n, int32_t v) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

// max |k|^2 over the keys of each (batch, kv head), as float bits (non-negative
// floats order as their bit patterns); out must start at zero.  Block
// (c, bk) takes rows [c * per, (c + 1) * per) of head bk and issues one atomic.
struct KnP {
    const void *k;
    int64_t ksb, ksh, ksn;
    int Hkv, M, d, per;
    uint32_t *out;     // (B * Hkv)
};

// SEG > 0: rows of SEG 16-byte segments, one per lane (64 / SEG rows per
// wavefront step); SEG == 0: one row per lane, element by element.
template <typename T, int SEG>
__global__ void __launch_bounds__(256) knorm_kernel(KnP p) {
    __shared__ uint32_t red[4];
    const int lane = lane_id(), wid = threadIdx.x / SSA_WAVE;
    const int bk = blockIdx.y;
    const int m0 = blockIdx.x * p.per, m1 = min(m0 + p.per, p.M);
    const T *kh = (const T *)p.k + (bk / p.Hkv) * p.ksb + (bk % p.Hkv) * p.ksh;
    float mx = 0.f;
    if constexpr (SEG > 0) {
        constexpr int RPW = SSA_WAVE / SEG;           // rows per wavefront step
        constexpr int E = 16 / (int)sizeof(T);        // elements per segment
        // (not unrolled: the row sum's lane exchanges sit inside the loop)
        for (int m = m0 + wid * RPW + lane / SEG; m < m1; m += 4 * RPW) {
            T ev[E];
            const uint4 w = *reinterpret_cast<const uint4 *>(kh + (int64_t)m * p.ksn + (lane % SEG) * E);
            __builtin_memcpy(ev, &w, sizeof(w));
            float s2 = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) s2 = fmaf(to_f32(ev[e]), to_f32(ev[e]), s2);
            // the row's sum, over its group of SEG lanes
#pragma unroll
            for (int o = 1; o < SEG; o <<= 1) s2 += __shfl_xor(s2, o, SSA_WAVE);
            mx = fmaxf(mx, s2);
        }
    } else {
        for (int m = m0 + (int)threadIdx.x; m < m1; m += 256) {
            const T *row = kh + (int64_t)m * p.ksn;
            float s2 = 0.f;
            for (int c = 0; c < p.d; ++c) s2 = fmaf(to_f32(row[c]), to_f32(row[c]), s2);
            mx = fmaxf(mx, s2);
        }
    }
    const uint32_t wm = wave_max_u(__float_as_uint(mx));
    if (lane == 0) red[wid] = wm;
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t b = max(max(red[0], red[1]), max(red[2], red[3]));
        atomicMax(&p.out[bk], b);
    }
}

// ------------------------------------------------------------------ query bucketing
struct QbP {
    const uint16_t *qid;
    const int32_t *bsize;   // key bucket sizes (BK*R, NB)
    const int32_t *bstart;  // key bucket starts (BK*R, NB)
    int32_t *cnt, *off, *cur, *qlist, *tiles, *ntiles;
    int32_t *tcnt;          // tiles per instance
    int32_t *kbase;         // first tile of each order key
    int32_t *hcnt;          // per (instance, query block, bucket): count, then first position
    int N, R, NS, NB, Hq, Hkv, rep, bh0, ninst, C;
    int64_t heads;          // (kv head, group head) pairs the order keys span
    int rmajor;             // tile order by (round, id set) first (see qb_order_key)
};

// Rescore tiles are stored in launch order: the dispatcher sends block i to
// XCD i % 8, and XCD x is to take the contiguous tile range [x * per,
// (x + 1) * per) in order, so that its L2 keeps the candidate rows adjacent
// tiles share.  Tile L therefore sits in slot (L % per) * 8 + L / per, and a
// block reads its slot and the tile count together (no dependent read).
__device__ __forceinline__ int rs_tile_slot(int L, int ntiles) {
    const int per = (ntiles + 7) / 8;
    return (L % per) * 8 + L / per;
}

__device__ __forceinline__ void inst_decode(const QbP &p, int inst, int &bh, int &r, int &t) {
    t = inst % p.NS;
    r = (inst / p.NS) % p.R;
    bh = p.bh0 + inst / (p.NS * p.R);
}

// Query block bx (256 queries) of nbx of instance inst: its count per bucket
// (hist: NB words of the workgroup's LDS; 256 threads)
__device__ void qb_hist_block(const QbP &p, int inst, int bx, int nbx, int32_t *hist) {
    int bh, r, t;
    inst_decode(p, inst, bh, r, t);
    for (int u = threadIdx.x; u < p.NB; u += blockDim.x) hist[u] = 0;
    __syncthreads();
    const int n = bx * (int)blockDim.x + (int)threadIdx.x;
    if (n < p.N) {
        const int u = p.qid[(((int64_t)bh * p.N + n) * p.R + r) * p.NS + t];
        atomicAdd(&hist[u], 1);
    }
    __syncthreads();
    int32_t *hb = p.hcnt + ((int64_t)inst * nbx + bx) * p.NB;
    for (int u = threadIdx.x; u < p.NB; u += blockDim.x) hb[u] = hist[u];
}

__global__ void __launch_bounds__(256) qb_hist_kernel(QbP p) {
    extern __shared__ int32_t hist[];
    qb_hist_block(p, (int)blockIdx.y, (int)blockIdx.x, (int)gridDim.x, hist);
}

// one block per instance: bucket totals and offsets, the first position of
// each query block's queries in each bucket (so queries stay in position
// order inside a bucket), and the instance's tile count
__device__ void qb_scan_block(const QbP &p, int inst) {
    // thread = (bucket column, query-block group): with NB <= 256 the NB
    // columns are split over 256 / NB groups of query blocks; with more
    // buckets a thread takes NB / 256 columns over every block
    __shared__ int32_t part[256];          // per thread: its sum, then its starting offset
    __shared__ int32_t sq[256], st[256];   // per column: bucket count, tile count (scanned)
    const int tid = threadIdx.x;
    int bh, r, t;
    inst_decode(p, inst, bh, r, t);
    const int b = bh / p.Hq, h = bh % p.Hq, g = h / p.rep;
    const int64_t krow = ((int64_t)b * p.Hkv + g) * p.R + r;
    const int nblk = (p.N + 255) / 256;
    int32_t *hb = p.hcnt + (int64_t)inst * nblk * p.NB;
    const int ncol = p.NB < 256 ? p.NB : 256;           // NB is a power of two
    const int per = p.NB / ncol;                        // buckets per column
    const int ngrp = 256 / ncol;                        // query-block groups per column
    const int col = tid % ncol, grp = tid / ncol;
    const int kper = (nblk + ngrp - 1) / ngrp;
    const int k0 = min(grp * kper, nblk), k1 = min(k0 + kper, nblk);
    // 1: each thread's sum over its blocks (per == 1 whenever ngrp > 1)
    if (per == 1) {
        int s = 0;
        for (int k = k0; k < k1; ++k) s += hb[(int64_t)k * p.NB + col];
        part[tid] = s;
    }
    __syncthreads();
    // 2: per column, bucket counts, tile counts and the groups' offsets within
    // their bucket
    if (tid < ncol) {
        int cq = 0, ct = 0;
        if (per == 1) {
            for (int gg = 0; gg < ngrp; ++gg) {
                const int v = part[gg * ncol + tid];
                part[gg * ncol + tid] = cq;
                cq += v;
            }
            p.cnt[(int64_t)inst * p.NB + tid] = cq;
            if (cq > 0 && p.bsize[krow * p.NB + tid] > 0) ct = (cq + TQ - 1) / TQ;
        } else {
            for (int u = tid * per; u < tid * per + per; ++u) {
                int c = 0;
                for (int k = 0; k < nblk; ++k) c += hb[(int64_t)k * p.NB + u];
                p.cnt[(int64_t)inst * p.NB + u] = c;
                cq += c;
                if (c > 0 && p.bsize[krow * p.NB + u] > 0) ct += (c + TQ - 1) / TQ;
            }
        }
        sq[tid] = cq;
        st[tid] = ct;
    } else {
        sq[tid] = 0;
        st[tid] = 0;
    }
    __syncthreads();
    // 3: inclusive scans of the column counts (Hillis-Steele over 256)
    for (int o = 1; o < 256; o <<= 1) {
        const int yq = tid >= o ? sq[tid - o] : 0;
        const int yt = tid >= o ? st[tid - o] : 0;
        __syncthreads();
        sq[tid] += yq;
        st[tid] += yt;
        __syncthreads();
    }
    if (tid == 0) p.tcnt[inst] = st[255];
    // 4: bucket offsets and each block's first position in its bucket
    const int cstart = col > 0 ? sq[col - 1] : 0;
    if (per == 1) {
        if (grp == 0) p.off[(int64_t)inst * p.NB + col] = cstart;
        int base = cstart + part[tid];
        for (int k = k0; k < k1; ++k) {
            const int c = hb[(int64_t)k * p.NB + col];
            hb[(int64_t)k * p.NB + col] = base;
            base += c;
        }
    } else if (tid < ncol) {
        int aq = cstart;
        for (int u = tid * per; u < tid * per + per; ++u) {
            p.off[(int64_t)inst * p.NB + u] = aq;
            int base = aq;
            for (int k = 0; k < nblk; ++k) {
                const int c = hb[(int64_t)k * p.NB + u];
                hb[(int64_t)k * p.NB + u] = base;
                base += c;
            }
            aq = base;
        }
    }
}

__global__ void __launch_bounds__(256) qb_scan_kernel(QbP p) { qb_scan_block(p, (int)blockIdx.x); }

// Position of an instance in the tile list: ordered by (kv head, query head
// within the GQA group, round, id set).  An XCD takes a contiguous range of
// tiles, so it works through one query head's rounds back to back while that
// head's q rows (N * d elements) and the kv head's K rows stay in its L2; with
// the rounds outside the query heads, every round re-read the group's q rows.
// When a head's q rows are larger than that (rmajor: the 32k MQA workload's
// 8 MB per head), the order is (round, id set, kv head, query head): each XCD
// then shares its rounds' tiles of every head with the others (rescore 8%
// faster there, 3% slower at 1 MB per head).
__device__ __forceinline__ int64_t qb_order_key(const QbP &p, int inst, int64_t bk_first) {
    int bh, r, t;
    inst_decode(p, inst, bh, r, t);
    const int b = bh / p.Hq, h = bh % p.Hq;
    const int64_t bk = (int64_t)b * p.Hkv + h / p.rep - bk_first;
    if (p.rmajor) return ((int64_t)r * p.NS + t) * p.heads + bk * p.rep + h % p.rep;
    return ((bk * p.rep + h % p.rep) * p.R + r) * p.NS + t;
}

// one block: the first tile of each instance in that order (kbase), and the
// tile count
__global__ void __launch_bounds__(256) qb_order_kernel(QbP p, int64_t nkeys) {
    __shared__ int32_t part[256];
    const int64_t bk_first = (int64_t)(p.bh0 / p.Hq) * p.Hkv + (p.bh0 % p.Hq) / p.rep;
    // dense per-key tile counts, then an exclusive scan over keys
    for (int64_t k = threadIdx.x; k < nkeys; k += 256) p.kbase[k] = 0;
    __syncthreads();
    for (int inst = threadIdx.x; inst < p.ninst; inst += 256)
        p.kbase[qb_order_key(p, inst, bk_first)] = p.tcnt[inst];
    __syncthreads();
    const int64_t per = (nkeys + 255) / 256;
    const int64_t k0 = threadIdx.x * per;
    int sum = 0;
    for (int64_t k = k0; k < k0 + per && k < nkeys; ++k) sum += p.kbase[k];
    part[threadIdx.x] = sum;
    __syncthreads();
    if (threadIdx.x == 0) {
        int acc = 0;
        for (int i = 0; i < 256; ++i) { const int v = part[i]; part[i] = acc; acc += v; }
        p.ntiles[0] = acc;
    }
    __syncthreads();
    int acc = part[threadIdx.x];
    for (int64_t k = k0; k < k0 + per && k < nkeys; ++k) {
        const int v = p.kbase[k];
        p.kbase[k] = acc;
        acc += v;
    }
}

// The tiles of one instance from its first tile (kbase): buckets in order,
// up to TQ queries per tile; buckets without keys or queries have none.
__device__ void qb_write_tiles(const QbP &p, int inst, int bh, int r, int t, int32_t *scan) {
    const int b = bh / p.Hq, h = bh % p.Hq, g = h / p.rep;
    const int64_t krow = ((int64_t)b * p.Hkv + g) * p.R + r;
    const int64_t bk_first = (int64_t)(p.bh0 / p.Hq) * p.Hkv + (p.bh0 % p.Hq) / p.rep;
    int carry = p.kbase[qb_order_key(p, inst, bk_first)];
    for (int u0 = 0; u0 < p.NB; u0 += blockDim.x) {
        const int u = u0 + threadIdx.x;
        int c = 0, nt = 0;
        if (u < p.NB) {
            c = p.cnt[(int64_t)inst * p.NB + u];
            nt = (c > 0 && p.bsize[krow * p.NB + u] > 0) ? (c + TQ - 1) / TQ : 0;
        }
        scan[threadIdx.x] = nt;
        __syncthreads();
        for (int o = 1; o < (int)blockDim.x; o <<= 1) {      // inclusive scan
            const int y = threadIdx.x >= (unsigned)o ? scan[threadIdx.x - o] : 0;
            __syncthreads();
            scan[threadIdx.x] += y;
            __syncthreads();
        }
        int at = carry + scan[threadIdx.x] - nt;
        if (nt > 0) {
            const int aq = p.off[(int64_t)inst * p.NB + u];
            const int bst = p.bstart[krow * p.NB + u];
            const int nva = min(p.bsize[krow * p.NB + u], p.C);
            const int ntiles = p.ntiles[0];
            for (int k = 0; k < nt; ++k)
                reinterpret_cast<int4 *>(p.tiles)[rs_tile_slot(at + k, ntiles)] =
                    make_int4(inst, aq + k * TQ, bst, min(TQ, c - k * TQ) | (nva << 8));
        }
        carry += scan[blockDim.x - 1];
        __syncthreads();
    }
}

constexpr int LS_RANK_MIN = 128;   // lists at least this long are ranked through a bitmap
static_assert(LS_RANK_MIN <= 128, "shorter lists pack their slots in 7 bits");

struct CutP {
    const int32_t *perm, *bstart, *bsize, *sid, *smin;
    const int64_t *glob;
    int4 *cut;
    int32_t *srix;     // per (row, list): offset of the query's score row in its head's
                       // region of S (lists * N * C elements), in elements
    const uint2 *ctab; // optional: the list sort's rank table of long lists
    int N, M, R, NS, NB, C, Cs, Hq, Hkv, rep, bh0, G, causal, nlists;
    int cbits;         // width of a cut entry's size and cutoff fields (the filler
                       // key and the bucket start take the bits above them)
    int64_t rows;
};

// The cut entry of query row rloc (chunk-relative) and list `list` (round,
// id set), whose bucket is u and whose position in its bucket's query list
// is pos: written by the query scatter, which has both at hand.
__device__ void cut_entry(const CutP &p, int64_t rloc, int list, int u, int pos) {
    const int64_t x = rloc * p.nlists + list;
    const int n = (int)(rloc % p.N);
    const int bh = p.bh0 + (int)(rloc / p.N);
    const int b = bh / p.Hq, h = bh % p.Hq, g = h / p.rep;
    const int64_t prow = ((int64_t)b * p.Hkv + g) * p.R + list / p.NS;
    const int st = p.bstart[prow * p.NB + u];
    const int sz = p.bsize[prow * p.NB + u];
    const int f = p.perm[prow * p.M + p.M - 1];   // key of the overflow filler slots
    int cutoff = 0, first = p.C, real = 0;
    if (sz == 0) {
        if (p.causal) {
            const int gl = min(p.G, p.C);
            for (int j = 0; j < gl; ++j)
                if ((int)p.glob[j] == n) { first = j; break; }
            if (first == p.C && n == 0 && p.G < p.C) first = p.G;
            real = 1;
        }
    } else {
        const int nv = min(sz, p.C);
        if (p.causal) {
            if (p.ctab && nv >= LS_RANK_MIN) {
                // members with id < n: those below n's 32-id word, then its bits
                const uint2 e = p.ctab[(prow * p.NB + u) * (int64_t)((p.M + 31) / 32) + (n >> 5)];
                cutoff = (int)e.x + __popc(e.y & ((1u << (n & 31)) - 1u));
            } else {
                const int32_t *sd = p.sid + prow * p.M + st;
                int lo = 0, hi = nv;               // members with id < n
                while (lo < hi) {
                    const int mid = (lo + hi) >> 1;
                    if (sd[mid] < n) lo = mid + 1; else hi = mid;
                }
                cutoff = lo;
            }
            const int a = cutoff < nv ? p.smin[prow * p.M + st + cutoff] : p.C;
            const int fb = (sz < p.C && f >= n) ? sz : p.C;
            first = min(a, fb);
            real = a < fb ? 1 : 0;
        } else {
            cutoff = nv;
        }
    }
    // Packed fields, read back as unsigned: the list size capped at C (every
    // use compares it with 0 and C or takes min(size, C)) and the cutoff in
    // the low cbits bits, the filler key and the bucket start (both below M)
    // above them; cbits is 16 up to 65,536 keys, and the host refuses sizes
    // whose fields do not fit 32 bits
    p.cut[x] = make_int4((int)(prow * p.M) + st,
                         (int)((uint32_t)min(sz, p.C) | ((uint32_t)f << p.cbits)),
                         (int)((uint32_t)cutoff | ((uint32_t)st << p.cbits)), first * 2 + real);
    p.srix[x] = (int32_t)(((int64_t)list * p.N + pos) * p.Cs);
}


__global__ void __launch_bounds__(256) qb_scatter_kernel(QbP p, CutP c) {
    // rank of each query among the block's queries of its bucket, in position
    // order: per wave the lanes of one bucket matched bit by bit (log2 NB
    // ballots), then the waves in order
    extern __shared__ int32_t sc_smem[];   // [4][NB] per-wave counts, then a scan buffer
    const int inst = blockIdx.y;
    int bh, r, t;
    inst_decode(p, inst, bh, r, t);
    if (blockIdx.x == 0) {
        qb_write_tiles(p, inst, bh, r, t, sc_smem);
        __syncthreads();
    }
    const int wid = threadIdx.x / SSA_WAVE;
    for (int x = threadIdx.x; x < 4 * p.NB; x += blockDim.x) sc_smem[x] = 0;
    __syncthreads();
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    const bool in = n < p.N;
    const int u = in ? p.qid[(((int64_t)bh * p.N + n) * p.R + r) * p.NS + t] : -1;
    uint64_t same = wave_ballot(in);
    for (int b = 0; (1 << b) < p.NB; ++b) {
        const bool bit = ((u >> b) & 1) != 0;
        const uint64_t m = wave_ballot(in && bit);
        same &= bit ? m : ~m;
    }
    const int local = lanes_below(same);
    // the lowest lane of each bucket gives the wave's count for it
    if (in && local == 0) sc_smem[wid * p.NB + u] = __popcll(same);
    __syncthreads();
    if (in) {
        int pos = p.hcnt[((int64_t)inst * gridDim.x + blockIdx.x) * p.NB + u] + local;
        for (int w = 0; w < wid; ++w) pos += sc_smem[w * p.NB + u];
        p.qlist[(int64_t)inst * p.N + pos] = n;
        cut_entry(c, (int64_t)(bh - p.bh0) * p.N + n, r * p.NS + t, u, pos);
    }
}

// ------------------------------------------------------------------ rescore
struct RsP {
    const int32_t *tiles, *ntiles, *qlist, *sid, *bstart, *bsize;
    const void *q, *k;
    int64_t qsb, qsh, qsn, ksb, ksh, ksn;
    uint16_t *S;       // 16-bit score codes (score_code): row (instance * N + qlist
                       // position) of Cs
    const float *aux;  // per query row: NA floats, the last the query's code scale
    int NA;
    int N, M, R, NS, NB, C, Hq, Hkv, rep, bh0, causal;
    int d;             // head dim (<= the instance's D; elements past it are zero)
    int Cs;            // score row stride (a multiple of 64)
    int k32;           // byte offsets of the K rows of a (batch, kv head) fit 32 bits
    int64_t Call;
};

// This block's tile (slot blockIdx.x, see rs_tile_slot): instance, first
// position in the instance's query list, the bucket's first sorted member,
// query count and member count (the bucket size clamped to C).  False: the
// slot holds no tile.
struct RsTile { int inst, qb, st, qc, nva; };
__device__ __forceinline__ bool rs_tile_fetch(const RsP &p, RsTile &t) {
    const int slot = (int)blockIdx.x;
    const int4 e = reinterpret_cast<const int4 *>(p.tiles)[slot];
    const int ntiles = *p.ntiles;
    const int per = (ntiles + 7) / 8, x = slot % 8, k = slot / 8;
    if (k >= per || x * per + k >= ntiles) return false;
    t.inst = e.x; t.qb = e.y; t.st = e.z; t.qc = e.w & 0xff; t.nva = e.w >> 8;
    return true;
}

// Sorted members a tile needs: a causal query only uses members below its own
// position, so the tile needs those below its last query (all otherwise).
// sd: the bucket's member ids in ascending order; nq: tile queries in nidx.
__device__ __forceinline__ int rs_tile_cutoff(const int32_t *sd, int nv, const int *nidx, int nq,
                                              bool causal) {
    if (!causal) return nv;
    const int lane = lane_id();
    const int nmax = (int)wave_max_u(lane < nq ? (uint32_t)nidx[lane] : 0u);
    int cnt = 0;
    for (int c0 = 0; c0 < nv; c0 += SSA_WAVE) {
        const int c = c0 + lane;
        const int m = __popcll(wave_ballot(c < nv && sd[c] < nmax));
        cnt += m;
        if (m < SSA_WAVE) break;
    }
    return cnt;
}

template <typename T, int D>
__global__ void __launch_bounds__(256) rescore_kernel(RsP p) {
    // head dims beyond 256 are staged 256 columns at a time (the q slice then
    // again for every candidate chunk); each score's fmaf chain still runs
    // over the columns in order
    constexpr int DS = D < 256 ? D : 256;
    constexpr bool ONE = D <= DS;
    constexpr int LD = DS + 1;
    extern __shared__ float rs_smem[];
    float *Qs = rs_smem;                // [TQ][LD]
    float *Ks = Qs + TQ * LD;           // [TC][LD]
    int *nidx = (int *)(Ks + TC * LD);  // [TQ]
    int *kidx = nidx + TQ;              // [TC]
    RsTile tl;
    if (!rs_tile_fetch(p, tl)) return;
    const int inst = tl.inst, qb = tl.qb, qc = tl.qc, st = tl.st;
    const int r = (inst / p.NS) % p.R, bhl = inst / (p.NS * p.R);
    const int bh = p.bh0 + bhl;
    const int b = bh / p.Hq, h = bh % p.Hq, g = h / p.rep;
    const int64_t prow = ((int64_t)b * p.Hkv + g) * p.R + r;
    const int tid = threadIdx.x;
    const T *qbase = (const T *)p.q + b * p.qsb + h * p.qsh;
    const T *kbase = (const T *)p.k + b * p.ksb + g * p.ksh;
    const int32_t *sd = p.sid + prow * p.M + st;

    if (tid < TQ) nidx[tid] = tid < qc ? p.qlist[(int64_t)inst * p.N + qb + tid] : 0;
    __syncthreads();
    const int nv = rs_tile_cutoff(sd, tl.nva, nidx, qc, p.causal);
    auto load_q = [&](int ds0) {
        for (int x = tid; x < TQ * DS; x += 256) {
            const int i = x / DS, c = x % DS;
            Qs[i * LD + c] = (i < qc && ds0 + c < p.d)
                                 ? to_f32(qbase[(int64_t)nidx[i] * p.qsn + ds0 + c]) : 0.f;
        }
    };
    if (ONE) load_q(0);
    const int ty = tid / 16, tx = tid % 16;
    for (int c0 = 0; c0 < nv; c0 += TC) {
        __syncthreads();
        if (tid < TC) kidx[tid] = (c0 + tid < nv) ? sd[c0 + tid] : 0;
        float acc[4][4];
#pragma unroll
        for (int a = 0; a < 4; ++a)
#pragma unroll
            for (int bb = 0; bb < 4; ++bb) acc[a][bb] = 0.f;
        for (int ds0 = 0; ds0 < p.d; ds0 += DS) {
            __syncthreads();
            if (!ONE) load_q(ds0);
            for (int x = tid; x < TC * DS; x += 256) {
                const int j = x / DS, c = x % DS;
                Ks[j * LD + c] = (c0 + j < nv && ds0 + c < p.d)
                                     ? to_f32(kbase[(int64_t)kidx[j] * p.ksn + ds0 + c]) : 0.f;
            }
            __syncthreads();
            // one fmaf chain over the head dim, as the select's exact keys run it
            const int cn = min(DS, p.d - ds0);
            for (int c = 0; c < cn; ++c) {
                float qa[4], kb[4];
#pragma unroll
                for (int a = 0; a < 4; ++a) qa[a] = Qs[(ty * 4 + a) * LD + c];
#pragma unroll
                for (int bb = 0; bb < 4; ++bb) kb[bb] = Ks[(tx + 16 * bb) * LD + c];
#pragma unroll
                for (int a = 0; a < 4; ++a)
#pragma unroll
                    for (int bb = 0; bb < 4; ++bb) acc[a][bb] = fmaf(qa[a], kb[bb], acc[a][bb]);
            }
        }
#pragma unroll
        for (int a = 0; a < 4; ++a) {
            const int i = ty * 4 + a;
            if (i >= qc) continue;
            uint16_t *srow = p.S + ((int64_t)inst * p.N + qb + i) * p.Cs + c0;
            const float sc = p.aux[((int64_t)bhl * p.N + nidx[i]) * p.NA + p.NA - 1];
#pragma unroll
            for (int bb = 0; bb < 4; ++bb) {
                const int cc = tx + 16 * bb;
                if (c0 + cc < nv) srow[cc] = (uint16_t)score_code(acc[a][bb], sc);
            }
        }
    }
}

// Matrix-core rescore for 16-bit q/k.  v_mfma_f32_16x16x32_{bf16,f16}: lane l
// supplies row (l % 16) of A and column (l % 16) of B, each with the 8
// elements k = 8*(l/16) .. +7; result element (4*(l/16) + r, l % 16) lands in
// accumulator r.  Products of 16-bit values are exact in fp32 and accumulate
// in fp32, so a score equals an fp32 dot product up to summation order.
// Each wave keeps the fragments of the tile's 64 queries in registers and
// streams slices of 64 candidate rows (4 x 4 blocks of 16 x 16).

template <typename T> struct Mfma16;
template <> struct Mfma16<bf16_t> {
    typedef bf16x8_t vec;
    static __device__ __forceinline__ f32x4_t mma(vec a, vec b, f32x4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
};
template <> struct Mfma16<f16_t> {
    typedef f16x8_t vec;
    static __device__ __forceinline__ f32x4_t mma(vec a, vec b, f32x4_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
};

// MFMA rescore of one tile (up to 64 queries of one bucket x the bucket's
// candidates in ascending id order, up to the tile's cutoff).  The K rows of
// each 32-candidate slice go from global memory straight into LDS (one
// global_load_lds_dwordx4 per 1 KB: lane l of a wave load writes bytes
// 16 l .. 16 l + 15 of it), in three buffers so slices j + 1 and j + 2 are in
// flight while slice j is scored; wave w scores queries 16w..16w+15 against
// the slice as K . Q^T, so each lane holds 8 consecutive candidates of one
// query and writes their 16-bit score codes with one 16-byte store.  About
// 26 KB of LDS and at most 80 registers per lane: 6 blocks per CU.
constexpr int RS_SLICE = 32;   // candidates per staged K slice

template <int D>
struct RsStage {
    static constexpr int SEGS = D / 8;                          // 16-byte pieces per K row
    static constexpr int RB = D * 2;                            // LDS bytes per row
    static constexpr int NI = (RS_SLICE * SEGS + 63) / 64;      // 1 KB wave loads per slice
    static constexpr int NIW = (NI + 3) / 4;                    // of them per wave (at most)
    static constexpr int BUF = NI * 1024;                       // LDS bytes per slice buffer
    static constexpr int W1 = SEGS >= 8 ? 1 : 8 / SEGS;        // rows per 128 bytes
    // Rows are stored unpadded with their pieces rotated: piece x of LDS row R
    // sits in slot (x + rot(R)) % SEGS.  A fragment read takes one piece of
    // 16 consecutive rows 16 ct .. 16 ct + 15; with this rotation its 16 lanes
    // hit 16 different 16-byte bank groups, and any 8 consecutive of them 8
    static __device__ __forceinline__ int rot(int R) {
        const int r = R % 16;
        return (r / W1 + r / (W1 * SEGS)) % SEGS;
    }
};

// Slice member held by LDS row R.  Tile ct of a slice multiplies LDS rows
// 16 ct .. 16 ct + 15 and lane (li, lg) receives rows 16 ct + 4 lg .. + 3;
// storing member 8 a + 4 b + c at row 16 b + 4 a + c hands lane (li, lg) the 8
// consecutive members 8 lg .. 8 lg + 7 (tiles 0 and 1).
__device__ __forceinline__ int rs_row_member(int R) {
    return ((R & 12) << 1) | ((R & 16) >> 2) | (R & 3);
}

// two 16-bit score codes, a at the lower address
__device__ __forceinline__ uint32_t code_pair(float a, float b, float sc) {
    // both complements at once: 65535 - x is ~x in 16 bits
    return ~(score_neg_code(a, sc) | (score_neg_code(b, sc) << 16));
}

typedef __attribute__((address_space(3))) void lds_void_t;

template <typename T, int D>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(6)))
rescore_mfma_kernel(RsP p) {
    using V = typename Mfma16<T>::vec;
    using S = RsStage<D>;
    constexpr int KS = (D + 31) / 32;          // k steps of 32
    constexpr int SEGS = S::SEGS;
    __shared__ int nidx[TQ];
    // the slice buffers are separate arrays, so the compiler can tell a load
    // into one from the reads of another
    __shared__ __align__(1024) unsigned char kb0[S::BUF], kb1[S::BUF], kb2[S::BUF];
    extern __shared__ int32_t prl[];           // the tile's candidate ids
    RsTile tl;
    if (!rs_tile_fetch(p, tl)) return;
    const int inst = tl.inst, qb = tl.qb, qc = tl.qc, st = tl.st, nva = tl.nva;
    const int r = (inst / p.NS) % p.R, bhl = inst / (p.NS * p.R);
    const int bh = p.bh0 + bhl;
    const int b = bh / p.Hq, h = bh % p.Hq, g = h / p.rep;
    const int64_t prow = ((int64_t)b * p.Hkv + g) * p.R + r;
    const int tid = threadIdx.x;
    const int wid = __builtin_amdgcn_readfirstlane(tid / SSA_WAVE);
    const int lane = lane_id();
    const int li = lane % 16, lg = lane / 16;
    const T *qbase = (const T *)p.q + b * p.qsb + h * p.qsh;
    const T *kbase = (const T *)p.k + b * p.ksb + g * p.ksh;
    const int32_t *pr = p.sid + prow * p.M + st;
    // the tile's queries and candidate ids (the list's members, ascending,
    // then INT_MAX up to a whole slice) load together, before one barrier
    if (tid < TQ) nidx[tid] = tid < qc ? p.qlist[(int64_t)inst * p.N + qb + tid] : 0;
    const int nvp = (nva + RS_SLICE - 1) / RS_SLICE * RS_SLICE;
    for (int c = tid; c < nvp; c += 256) prl[c] = c < nva ? pr[c] : INT_MAX;
    __syncthreads();

    // this wave's 16 queries as the B operand (column li = query 16*wid + li)
    const int qrow = 16 * wid + li;
    const bool qok = qrow < qc;
    V qf[KS];
    {
        const T *src = qbase + (int64_t)nidx[qok ? qrow : 0] * p.qsn;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const int e0 = 32 * s + 8 * lg;
            qf[s] = (qok && e0 < p.d) ? __builtin_bit_cast(V, *reinterpret_cast<const uint4 *>(src + e0))
                                      : __builtin_bit_cast(V, make_uint4(0, 0, 0, 0));
        }
    }
    const bool active = 16 * wid < qc;
    // the query's code scale (written by the aux kernel)
    const float qsc = qok ? p.aux[((int64_t)bhl * p.N + nidx[qrow]) * p.NA + p.NA - 1] : 1.f;
    const int nv = rs_tile_cutoff(prl, nva, nidx, qc, p.causal);
    const int nsl = (nv + RS_SLICE - 1) / RS_SLICE;

    // This lane's part of the wave's slice loads: wave load i = wid + 4 t
    // fills bytes 1024 i .. of a buffer, its lane the 16-byte slot
    // g = 64 i + lane, i.e. slot g % SEGS of LDS row g / SEGS (rows past the
    // slice, only at D = 8, land in the buffer's unused half).  Rows are
    // addressed by 32-bit byte offsets from the head's base (the dispatcher
    // picks this kernel only when they fit); pieces past the head dim load
    // piece 0 and slots past the list the last row (neither is used).
    const uint32_t rowb = (uint32_t)(p.ksn * (int64_t)sizeof(T));
    int lmem[S::NIW];
    uint32_t lseg[S::NIW];
#pragma unroll
    for (int t = 0; t < S::NIW; ++t) {
        const int gs = 64 * (wid + 4 * t) + lane;
        const int R = gs / SEGS;
        const int x = (gs % SEGS + SEGS - S::rot(R)) % SEGS;
        lmem[t] = rs_row_member(R % RS_SLICE);
        lseg[t] = (uint32_t)(x * 8 < p.d ? x : 0) * 16u;
    }
    // (the member ids are read before the first load: a read of LDS after a
    // load into LDS waits for that load)
    auto stage = [&](unsigned char *buf, int c0) __attribute__((always_inline)) {
        uint32_t ro[S::NIW];
#pragma unroll
        for (int t = 0; t < S::NIW; ++t)
            ro[t] = __umul24(min((uint32_t)prl[c0 + lmem[t]], (uint32_t)(p.M - 1)), rowb) + lseg[t];
#pragma unroll
        for (int t = 0; t < S::NIW; ++t) {
            const int i = wid + 4 * t;
            if (S::NI % 4 == 0 || i < S::NI)
                __builtin_amdgcn_global_load_lds((const void *)((const char *)kbase + ro[t]),
                                                 (lds_void_t *)(buf + 1024 * i), 16, 0, 0);
        }
    };
    if (nsl > 0) stage(kb0, 0);
    if (nsl > 1) stage(kb1, RS_SLICE);

    // Each lane stores its 8 score codes as a 16-byte vector through a raw
    // buffer over the instance's rows (rows are padded to a multiple of 64
    // members).  A group of 8 members is stored only when its first member is
    // below the lane's query (causal; the select kernel reads no further), is
    // on the list (not INT_MAX) and the lane has a query: other lanes give an
    // offset past the buffer's end, which the hardware drops.  So every slice
    // issues exactly one store per wave after its loads, and waiting for a
    // slice's loads leaves the last store in flight.
    const int nqe = !qok ? INT_MIN : p.causal ? nidx[qrow] : INT_MAX;
    const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(p.S + (int64_t)inst * p.N * p.Cs), (short)0, (int)((int64_t)p.N * p.Cs * 2),
        SSA_BUF_FLAGS);
    // make_dims keeps an instance's rows (N * Cs * 2 bytes) below 2^31
    const uint32_t sbase = ((uint32_t)(qb + qrow) * (uint32_t)p.Cs + 8u * lg) * 2u;
    // TAIL: k steps reach past the head dim, so the pieces there are zeroed
    // (they hold piece 0 of the row; its product with the zero q pieces would
    // still turn an infinite element into NaN)
    const int rrot = S::rot(li);
    auto score = [&](const unsigned char *kl, int c0, auto tail) __attribute__((always_inline)) {
        constexpr bool TAIL = decltype(tail)::value;
        u32x4_t kq = {};
        if (active) {
            f32x4_t acc[2] = {f32x4_t{0.f, 0.f, 0.f, 0.f}, f32x4_t{0.f, 0.f, 0.f, 0.f}};
            // rows li and 16 + li share their rotation
            const unsigned char *kr = kl + li * S::RB;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const int x = 4 * s + lg;      // the lane's 16-byte piece of the k step
                const int slot = (x + rrot) % SEGS;
#pragma unroll
                for (int ct = 0; ct < 2; ++ct) {
                    uint4 kv = *reinterpret_cast<const uint4 *>(kr + 16 * ct * S::RB + slot * 16);
                    if constexpr (TAIL) {
                        const uint32_t m = 8 * x < p.d ? ~0u : 0u;
                        kv = make_uint4(kv.x & m, kv.y & m, kv.z & m, kv.w & m);
                    }
                    acc[ct] = Mfma16<T>::mma(__builtin_bit_cast(V, kv), qf[s], acc[ct]);
                }
            }
            // lane (li, lg) holds members c0 + 8 lg + 4 ct + rr of query li in acc[ct][rr]
            kq = u32x4_t{code_pair(acc[0][0], acc[0][1], qsc), code_pair(acc[0][2], acc[0][3], qsc),
                         code_pair(acc[1][0], acc[1][1], qsc), code_pair(acc[1][2], acc[1][3], qsc)};
        }
        // every wave issues the same store (dropped where out of range)
        const uint32_t off = prl[c0 + 8 * lg] < nqe ? sbase : 0x80000000u;
        __builtin_amdgcn_raw_buffer_store_b128(kq, srs, off, 2 * c0, 0);
    };
    // The barrier before slice j: each wave first waits for its own loads of
    // the slice (the hardware writes a load's data to LDS before it counts
    // the load done), so after the barrier the whole slice is in LDS; the
    // reads of the buffer the next loads overwrite (slice j - 1's) were
    // consumed by the MFMAs before it.  A wave's vector memory operations
    // issue in the order: loads of slice j, store of slice j - 2, loads of
    // slice j + 1, store of slice j - 1, and complete in order, so the wait
    // leaves the ones after the loads of slice j in flight: at least NW loads
    // per slice and wave (waves with more wait a little longer than they
    // need).  Before slice 0 everything is waited for (the q rows and slice 1
    // too: the compiler then knows the q rows have landed).  The wait is
    // the builtin (so the compiler counts it and adds none of its own),
    // fenced by empty asm statements that keep memory operations on their
    // side of it, and the barrier a bare s_barrier: the workgroup fence of
    // __syncthreads would also wait for the score stores.
    constexpr int NW = S::NI / 4;
    auto slice_barrier = [&](int j) __attribute__((always_inline)) {
        const int after = j == 0 ? 0 : (j >= 2) + (j + 1 < nsl ? NW : 0) + 1;
        asm volatile("" ::: "memory");
        // vmcnt(after); lgkmcnt and expcnt not waited for
        if (after == 0) __builtin_amdgcn_s_waitcnt(0x0F70);
        else if (after == 1) __builtin_amdgcn_s_waitcnt(0x0F71);
        else if (after == 2) __builtin_amdgcn_s_waitcnt(0x0F72);
        else if (after == 3) __builtin_amdgcn_s_waitcnt(0x0F73);
        else __builtin_amdgcn_s_waitcnt(0x0F74);
        asm volatile("s_barrier" ::: "memory");
    };
    static_assert(NW <= 2, "vmcnt immediates above cover at most 4 operations");
    auto slices = [&](auto tail) __attribute__((always_inline)) {
        for (int j = 0; j < nsl; j += 3) {
            // slice j is in kb0, j + 1 in kb1, j + 2 in kb2; the buffer a
            // stage fills was last read by the slice before the barrier
            slice_barrier(j);
            if (j + 2 < nsl) stage(kb2, RS_SLICE * (j + 2));
            score(kb0, RS_SLICE * j, tail);
            if (j + 1 >= nsl) break;
            slice_barrier(j + 1);
            if (j + 3 < nsl) stage(kb0, RS_SLICE * (j + 3));
            score(kb1, RS_SLICE * (j + 1), tail);
            if (j + 2 >= nsl) break;
            slice_barrier(j + 2);
            if (j + 4 < nsl) stage(kb1, RS_SLICE * (j + 4));
            score(kb2, RS_SLICE * (j + 2), tail);
        }
    };
    // below D = 32 the k steps also cover pieces past the row (at piece 0)
    if (p.d == D && D % 32 == 0) slices(std::false_type{});
    else slices(std::true_type{});
}

// ------------------------------------------------------------------ sorted candidate lists
// A bucket's candidate list is its first C members in permutation order
// (:668-696).  Only the order-free parts of the stream are rescored and
// scanned in key order: with the members of each list sorted by key id, the
// members a causal query can use (ids below its own position) are a prefix.
// Per (kv head, round) row of M permutation positions:
//   sid[st + i]  i-th smallest member id of the bucket starting at st (i < nv)
//   rnk[st + c]  sorted index of the member at list slot c
//   smin[st + i] smallest list slot among sorted members i.. (first future slot)
//   inv[key]     permutation position of every key

struct LsP {
    const int32_t *perm, *bstart, *bsize;
    int32_t *sid, *rnk, *smin, *inv;
    int M, NB, C;
    // with kpart: block (kv head bk, round 0, bucket 0) also writes knorm[bk], the
    // max of the key hash's M / 16 tile maxima of |k|^2 for that head
    const uint32_t *kpart;
    uint32_t *knorm;
    int R;
    // optional, per (row, bucket, 32-id word) of a long list: (members with a
    // smaller id, the word's member bits) -- the cut's count of members below
    // a query without a search
    uint2 *ctab;
};

// Workgroup blk: list (kv head / round row blk / NB, bucket blk % NB);
// ls_key: the workgroup's dynamic LDS (256 threads)
__device__ void list_sort_block(const LsP &p, int64_t blk, uint32_t *ls_key) {
    const int64_t prow = blk / p.NB;
    const int u = (int)(blk % p.NB);
    if (p.kpart && u == 0 && prow % p.R == 0) {
        __shared__ uint32_t kred[4];
        const int64_t bk = prow / p.R;
        const int nt = p.M / 16;
        uint32_t m = 0u;
        for (int i = threadIdx.x; i < nt; i += 256) m = max(m, p.kpart[bk * nt + i]);
        m = wave_max_u(m);
        if (lane_id() == 0) kred[threadIdx.x / SSA_WAVE] = m;
        __syncthreads();
        if (threadIdx.x == 0) p.knorm[bk] = max(max(kred[0], kred[1]), max(kred[2], kred[3]));
    }
    const int st = p.bstart[prow * p.NB + u];
    const int sz = p.bsize[prow * p.NB + u];
    if (sz == 0) return;
    const int nv = min(sz, p.C);
    int P2 = 1;
    while (P2 < nv) P2 <<= 1;
    const int tid = threadIdx.x;
    const int64_t base = prow * p.M;
    const int32_t *pr = p.perm + base;
    for (int i = tid; i < sz; i += 256) p.inv[base + pr[st + i]] = st + i;
    if (nv >= LS_RANK_MIN) {
        // long lists: the rank of a member is the number of member ids below
        // it, read off an M-bit map of the list with per-word prefix counts
        const int W = (p.M + 31) / 32;
        uint32_t *bmp = ls_key;                       // [W]
        int32_t *pre = (int32_t *)(bmp + W);          // [W]
        int32_t *sor = pre + W;                       // [nv] list slot of each rank
        int32_t *wsum = sor + min(p.C, p.M);          // [4]
        for (int w = tid; w < W; w += 256) bmp[w] = 0u;
        __syncthreads();
        for (int i = tid; i < nv; i += 256) {
            const int id = pr[st + i];
            atomicOr(&bmp[id >> 5], 1u << (id & 31));
        }
        __syncthreads();
        const int per = (W + 255) / 256, w0 = tid * per;
        int c = 0;
        for (int w = w0; w < w0 + per && w < W; ++w) c += __popc(bmp[w]);
        const int lane = lane_id(), wv = tid / SSA_WAVE;
        int x = c;
#pragma unroll
        for (int o = 1; o < SSA_WAVE; o <<= 1) {
            const int y = __shfl_up(x, o, SSA_WAVE);
            if (lane >= o) x += y;
        }
        if (lane == SSA_WAVE - 1) wsum[wv] = x;
        __syncthreads();
        int acc = x - c;
        for (int k = 0; k < wv; ++k) acc += wsum[k];
        uint2 *ct = p.ctab ? p.ctab + (prow * p.NB + u) * (int64_t)W : nullptr;
        for (int w = w0; w < w0 + per && w < W; ++w) {
            pre[w] = acc;
            if (ct) ct[w] = make_uint2((uint32_t)acc, bmp[w]);
            acc += __popc(bmp[w]);
        }
        __syncthreads();
        for (int i = tid; i < nv; i += 256) {
            const int id = pr[st + i];
            const int r = pre[id >> 5] + __popc(bmp[id >> 5] & ((1u << (id & 31)) - 1u));
            p.sid[base + st + r] = id;
            p.rnk[base + st + i] = r;
            sor[r] = i;
        }
        __syncthreads();
        if (tid < SSA_WAVE) {                      // suffix minimum of the list slots
            int carry = p.C;
            for (int hi = nv; hi > 0; hi -= SSA_WAVE) {
                const int i = hi - SSA_WAVE + lane;
                int cs = i >= 0 ? sor[i] : p.C;
#pragma unroll
                for (int o = 1; o < SSA_WAVE; o <<= 1) {
                    const int y = __shfl_down(cs, o, SSA_WAVE);
                    if (lane + o < SSA_WAVE) cs = min(cs, y);
                }
                cs = min(cs, carry);
                if (i >= 0) p.smin[base + st + i] = cs;
                carry = __shfl(cs, 0, SSA_WAVE);
            }
        }
        return;
    }
    // key id << 7 | list slot: lists this short have slots below 128, and
    // key ids (below M <= 2^20) leave the packed keys below the padding
    for (int i = tid; i < P2; i += 256)
        ls_key[i] = i < nv ? (((uint32_t)pr[st + i] << 7) | (uint32_t)i) : 0xffffffffu;
    __syncthreads();
    for (int k = 2; k <= P2; k <<= 1) {            // bitonic sort, ascending
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < P2; i += 256) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const uint32_t a = ls_key[i], b = ls_key[ixj];
                    if ((a > b) == ((i & k) == 0)) { ls_key[i] = b; ls_key[ixj] = a; }
                }
            }
            __syncthreads();
        }
    }
    for (int i = tid; i < nv; i += 256) {
        const uint32_t key = ls_key[i];
        p.sid[base + st + i] = (int32_t)(key >> 7);
        p.rnk[base + st + (int)(key & 127u)] = i;
    }
    if (tid < SSA_WAVE) {                          // suffix minimum of the list slots
        const int lane = tid;
        int carry = p.C;
        for (int hi = nv; hi > 0; hi -= SSA_WAVE) {
            const int i = hi - SSA_WAVE + lane;
            int c = i >= 0 ? (int)(ls_key[i] & 127u) : p.C;
#pragma unroll
            for (int o = 1; o < SSA_WAVE; o <<= 1) {
                const int y = __shfl_down(c, o, SSA_WAVE);
                if (lane + o < SSA_WAVE) c = min(c, y);
            }
            c = min(c, carry);
            if (i >= 0) p.smin[base + st + i] = c;
            carry = __shfl(c, 0, SSA_WAVE);
        }
    }
}

__global__ void __launch_bounds__(256) list_sort_kernel(LsP p) {
    extern __shared__ uint32_t ls_key[];
    list_sort_block(p, (int64_t)blockIdx.x, ls_key);
}

// Launches shared by independent work of the first head chunk, whose query
// ids the launch of the sort's top levels computed: the sort's segment
// kernel (workgroups [0, nseg)) beside that chunk's query histogram (the
// rest, nqb per instance), and the list sort (workgroups [0, nls)) beside
// the chunk's bucket scan (one per instance).  Each pair reads and writes
// disjoint data, and the segment kernel and the list sort leave most CUs
// idle on their own.
__global__ void __launch_bounds__(SEG_WAVES * SSA_WAVE)
sort_seg_hist_kernel(SortTopArgs s, QbP qp, int nseg, int nqb) {
    extern __shared__ uint32_t sh_lds[];       // the segment waves' arrays, or NB counts
    const int blk = (int)blockIdx.x;
    if (blk < nseg) {
        sort_seg_blocks<uint16_t>(s.gkv, s.n, s.segs, s.segcount, s.perm, sh_lds, blk, nseg);
    } else {
        const int b = blk - nseg;
        qb_hist_block(qp, b / nqb, b % nqb, nqb, (int32_t *)sh_lds);
    }
}

__global__ void __launch_bounds__(256) list_sort_scan_kernel(LsP lp, QbP qp, int nls) {
    extern __shared__ uint32_t ls_key[];
    if ((int)blockIdx.x < nls) list_sort_block(lp, (int64_t)blockIdx.x, ls_key);
    else qb_scan_block(qp, (int)blockIdx.x - nls);
}

// Per (query row, list): the number of sorted members below the query
// (causal; all of them otherwise), and where the query's own key first occurs
// in the list -- a member at or past the query (causal substitution, :698-709),
// an overflow filler (invalid) when the filler key is at or past the query, or
// an entry of glob ++ 0 for an empty bucket (:711-737) -- as
// {row offset of the bucket (kv-head/round row * M + start), size | filler
// key << cbits, cutoff | start << cbits, first slot * 2 + (that slot is
// valid)}; first slot C: none.
// ------------------------------------------------------------------ extra scores
// Per query row: q.k_n (the key that replaces future candidates when causal,
// :698-709) and q.k_glob[j], q.k_0 (the empty-bucket list, :711-737).  They
// are computed with exactly the arithmetic of the rescore kernel the same
// call uses (MFMA k-steps of 32, or one fmaf chain over d), so a key scores
// the same wherever it appears -- the reference's single einsum gives equal
// keys equal scores, and ties among them must survive.
struct AuxP {
    const void *q, *k;
    int64_t qsb, qsh, qsn, ksb, ksh, ksn;
    const int64_t *glob;
    const uint32_t *knorm;   // max |k|^2 per (batch, kv head), float bits
    int N, Hq, Hkv, rep, bh0, nbh, G, NA, causal, d;
    float *out;        // (nbh * N, NA): q.k_n, q.k_glob[0..G-1], q.k_0, code scale
    // aux_mfma_kernel with qid set also hashes its query rows (the query hash
    // of hash_mfma_kernel on the q rows it has loaded anyway): planes as
    // HashP's (16-byte aligned), ids in the query layout; zero1, if set, is
    // cleared by block 0 (the select kernels' tie-row counter)
    const float *planes;
    int R, maxP, P, Tp, NS;
    uint16_t *qid;
    int32_t *zero1;
    // when set (the launch beside the key sort, before the list sort reduces
    // them): each wave takes max |k|^2 of its kv head from the key hash's
    // 16-row tile maxima (kp_n per kv head) instead of knorm
    const uint32_t *kpart;
    int kp_n;
};

// LDS floats a wave of aux_mfma_rows needs for the fused query hash
__host__ __device__ inline int aux_wave_floats(int R, int P) {
    return 16 * (((R * P + 15) / 16) * 16 + 1);
}

// One wavefront's 16 query rows of the aux pass (wg: the wave's index over
// the launch; pw: its LDS region of aux_wave_floats floats).
template <typename T, int D>
__device__ void aux_mfma_rows(const AuxP &p, int64_t wg, float *pw) {
    using V = typename Mfma16<T>::vec;
    constexpr int KS = (D + 31) / 32;
    const int lane = lane_id();
    const int li = lane % 16, lg = lane / 16;
    const int nblk = (p.N + 15) / 16;
    if (wg >= (int64_t)p.nbh * nblk) return;
    const int bhl = (int)(wg / nblk);
    const int n0 = (int)(wg % nblk) * 16;
    const int bh = p.bh0 + bhl;
    const int b = bh / p.Hq, h = bh % p.Hq, g = h / p.rep;
    const T *qbase = (const T *)p.q + b * p.qsb + h * p.qsh;
    const T *kbase = (const T *)p.k + b * p.ksb + g * p.ksh;
    // k steps of 32 over the head dim d <= D, elements past d zero (as the
    // rescore and the select's exact keys take them)
    auto frag = [&](const T *src, bool ok, int s) {
        const int e0 = 32 * s + 8 * lg;
        if (ok && e0 < p.d) return __builtin_bit_cast(V, *reinterpret_cast<const uint4 *>(src + e0));
        return __builtin_bit_cast(V, make_uint4(0, 0, 0, 0));
    };
    const int nq = n0 + li;
    const bool okq = nq < p.N;
    V qa[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) qa[s] = frag(qbase + (int64_t)(okq ? nq : 0) * p.qsn, okq, s);
    if (p.qid) {
        // bucket and probe ids of the 16 rows (sparse_attention.py:559-646):
        // fp32 projections on v_mfma_f32_16x16x4f32, lane (li, lg) feeding row
        // li and plane li with element 32 s + 8 lg + e at step (s, e) -- the
        // elements its bf16/f16 fragments hold -- then through LDS to one lane
        // per row, which writes the ids as the query hash does
        if (p.zero1 && wg == 0 && lane == 0) *p.zero1 = 0;
        const int NP = p.R * p.P;
        const int NT = (NP + 15) / 16;
        const int pst = NT * 16 + 1;
        for (int t = 0; t < NT; ++t) {
            const int j = t * 16 + li;
            const bool real = j < NP;
            const float *pl = p.planes + (real ? ((int64_t)(j / p.P) * p.maxP + (j % p.P)) * p.d : 0);
            f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                const int e0 = 32 * s + 8 * lg;
                float4 w0 = make_float4(0.f, 0.f, 0.f, 0.f), w1 = w0;
                if (real && e0 < p.d) {
                    w0 = *reinterpret_cast<const float4 *>(pl + e0);
                    w1 = *reinterpret_cast<const float4 *>(pl + e0 + 4);
                }
                const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
                T qe[8];
                __builtin_memcpy(qe, &qa[s], sizeof(qe));
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(to_f32(qe[e]), wv[e], acc, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) pw[(4 * lg + r) * pst + t * 16 + li] = acc[r];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // one (row, round) pair per lane, in the ids' memory order
        for (int x0 = 0; x0 < 16 * p.R; x0 += SSA_WAVE) {
            const int x = x0 + lane;
            const int rl = x / p.R, r = x - rl * p.R;
            if (rl < 16 && n0 + rl < p.N)
                ssa_write_ids(pw + rl * pst + r * p.P, p.P, p.Tp,
                          p.qid + (((int64_t)bh * p.N + n0 + rl) * p.R + r) * p.NS);
        }
    }
    // operand roles as in the rescore (keys as A, queries as B): lane (li, lg)
    // receives C[4 lg + rr][li] = score of key row 4 lg + rr for query n0 + li
    float *ob = p.out + ((int64_t)bhl * p.N + n0) * p.NA;
    {
        // the query's code scale from |q|^2 (lanes lg hold quarters of the row)
        float q2 = 0.f;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            T qe[8];
            __builtin_memcpy(qe, &qa[s], sizeof(qe));
#pragma unroll
            for (int e = 0; e < 8; ++e) q2 = fmaf(to_f32(qe[e]), to_f32(qe[e]), q2);
        }
        q2 += __shfl_xor(q2, 16, SSA_WAVE);
        q2 += __shfl_xor(q2, 32, SSA_WAVE);
        uint32_t kn;
        if (p.kpart) {
            // max over the tile maxima, as the list sort reduces them
            const uint32_t *kt = p.kpart + (int64_t)(b * p.Hkv + g) * p.kp_n;
            uint32_t m = 0u;
            for (int i = lane; i < p.kp_n; i += SSA_WAVE) m = max(m, kt[i]);
            kn = wave_max_u(m);
        } else {
            kn = p.knorm[b * p.Hkv + g];
        }
        if (lg == 0 && okq) ob[(int64_t)li * p.NA + p.NA - 1] = code_scale(q2, __uint_as_float(kn));
    }
    if (p.causal) {            // key row li is key n0 + li: the diagonal is q_n . k_n
        V kb[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) kb[s] = frag(kbase + (int64_t)(okq ? nq : 0) * p.ksn, okq, s);
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s) acc = Mfma16<T>::mma(kb[s], qa[s], acc);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
            if (4 * lg + rr == li && okq) ob[(int64_t)li * p.NA] = acc[rr];
    }
    for (int j0 = 0; j0 <= p.G; j0 += 16) {       // key rows: glob[0..G-1], then key 0
        const int j = j0 + li;
        const int key = j < p.G ? (int)p.glob[j] : 0;
        V kb[KS];
#pragma unroll
        for (int s = 0; s < KS; ++s) kb[s] = frag(kbase + (int64_t)key * p.ksn, true, s);
        f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s) acc = Mfma16<T>::mma(kb[s], qa[s], acc);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int jj = j0 + 4 * lg + rr;
            if (okq && jj <= p.G) ob[(int64_t)li * p.NA + 1 + jj] = acc[rr];
        }
    }
}

template <typename T, int D>
__global__ void __launch_bounds__(256) aux_mfma_kernel(AuxP p) {
    extern __shared__ float aux_proj[];
    const int wid = threadIdx.x / SSA_WAVE;
    aux_mfma_rows<T, D>(p, (int64_t)blockIdx.x * 4 + wid,
                        aux_proj + (p.qid ? wid * aux_wave_floats(p.R, p.P) : 0));
}

// The key sort's top levels (workgroups 0 .. s.rows - 1, one row each) and the
// first head chunk's aux pass with its query hash (the other workgroups, 16
// waves of aux_mfma_rows each) in one launch: the sort keeps only s.rows
// CUs busy, and the query side needs only q, the hyperplanes and the key
// hash's norm tiles.
template <typename T, int D>
__global__ void __launch_bounds__(SORT_THREADS) sort_aux_kernel(SortTopArgs s, AuxP p) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    __shared__ TopShared sh;
    if ((int)blockIdx.x < s.rows) {
        sort_top_row<uint16_t>((int)blockIdx.x, s.ids, s.n, s.NB, s.perm, s.bstart, s.bsize, s.gkv,
                               s.segs, s.segcount, s.glb, s.tl_in_lds, s.cap, smem_raw, sh);
        return;
    }
    const int wid = threadIdx.x / SSA_WAVE;
    aux_mfma_rows<T, D>(p, ((int64_t)blockIdx.x - s.rows) * SORT_WAVES + wid,
                        (float *)smem_raw + wid * aux_wave_floats(p.R, p.P));
}

template <typename T, int D>
__global__ void __launch_bounds__(256) aux_valu_kernel(AuxP p) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)p.nbh * p.N * p.NA) return;
    const int a = (int)(idx % p.NA);
    const int64_t rloc = idx / p.NA;
    const int n = (int)(rloc % p.N);
    const int bh = p.bh0 + (int)(rloc / p.N);
    const int b = bh / p.Hq, h = bh % p.Hq, g = h / p.rep;
    if (a == 0 && !p.causal) return;
    const T *qr = (const T *)p.q + b * p.qsb + h * p.qsh + (int64_t)n * p.qsn;
    if (a == p.NA - 1) {               // the query's code scale
        float q2 = 0.f;
        for (int c = 0; c < p.d; ++c) q2 = fmaf(to_f32(qr[c]), to_f32(qr[c]), q2);
        p.out[idx] = code_scale(q2, __uint_as_float(p.knorm[b * p.Hkv + g]));
        return;
    }
    const int key = a == 0 ? n : (a - 1 < p.G ? (int)p.glob[a - 1] : 0);
    const T *kr = (const T *)p.k + b * p.ksb + g * p.ksh + (int64_t)key * p.ksn;
    float acc = 0.f;
    for (int c = 0; c < p.d; ++c) acc = fmaf(to_f32(qr[c]), to_f32(kr[c]), acc);
    p.out[idx] = acc;
}

// ------------------------------------------------------------------ select + merge
struct SelP {
    const uint16_t *qid;
    const int32_t *perm, *bstart, *bsize;
    const int32_t *sid, *rnk, *inv;   // sorted list members, their ranks, key positions
    const int4 *cut;       // per (row, list): bucket offset, size/filler, cutoff/start, first
    const int32_t *srix;   // per (row, list): offset of the query's score row in its head's
                           // region of S
    uint32_t head_bytes;   // bytes of one head's region of S (< 2^32)
    uint32_t nl_magic;     // ceil(2^32 / nlists): pair index / nlists as a high product
    const uint16_t *S;     // score-key prefixes (score_key >> 16), rows as the rescore wrote
    int mfma;              // the rescore used MFMA k-steps (else one fmaf chain over d)
    const void *q, *k;
    int64_t qsb, qsh, qsn, ksb, ksh, ksn;
    const int64_t *glob;
    int N, M, d, R, NS, NB, C, Cs, CPL, nlists, Hq, Hkv, rep, G, kk, window, causal, cross, mode,
        total_k, Kw, Kout, bh0, words;
    int cbits;             // width of a cut entry's size and cutoff fields
    int waves;             // rows (one per wave) of a select workgroup
    int64_t Call, rows;
    int64_t rows_all;      // query rows of every head (B * Hq * N): tie rows and output rows
    int64_t *out_idx;
    uint8_t *out_valid;
    int32_t *out_idx32;    // FULL mode: the graph as int32 ids (-1 = invalid) instead
    int32_t *ties;
    int32_t *tie_list;     // rows (bh * N + n) handed to the exact top-k replay
    int32_t *tie_count;
    const float *aux;      // per row: q.k_n, then q.k_glob[j] (j < G), then q.k_0
    int NA;
    int perm_bytes;        // size of the permutation array (B*Hkv*R*M*4 < 2^31)
    int64_t nblocks;
};

__device__ __forceinline__ void bm_set(uint32_t *bm, int v) { atomicOr(&bm[v >> 5], 1u << (v & 31)); }

// index of the k-th (0-based) set bit of b (k < popcount(b))
__device__ __forceinline__ int nth_set_bit(uint32_t b, int k) {
    int pos = 0;
#pragma unroll
    for (int sh = 16; sh >= 1; sh >>= 1) {
        const int c = __popc(b & ((1u << sh) - 1u));
        const bool up = k >= c;
        k = up ? k - c : k;
        b = up ? b >> sh : b;
        pos = up ? pos + sh : pos;
    }
    return pos;
}

// Exact score keys of one query row qr against the keys v of the lanes with
// `want` set (0 elsewhere), computed with the arithmetic of the rescore that
// wrote the table, whose 16-bit prefixes they extend: MFMA k-steps of 32 with
// the keys as A rows and the query as every B column (the wanted lanes taken 16
// at a time, in lane order), or one fmaf chain over d.  kb: the kv head's K rows.
template <typename T>
__device__ uint32_t exact_keys(const SelP &p, const T *qr, const T *kb, int v, bool want) {
    const int lane = lane_id();
    if constexpr (!std::is_same<T, float>::value) {
        if (p.mfma) {
            using V = typename Mfma16<T>::vec;
            const uint64_t wm = wave_ballot(want);
            const int li = lane & 15, lg = lane >> 4;
            const int KS = (p.d + 31) >> 5;
            const int rank = lanes_below(wm);
            const int total = __popcll(wm);
            const uint32_t wlo = (uint32_t)wm, whi = (uint32_t)(wm >> 32);
            const int clo = __popc(wlo);
            uint32_t out = 0u;
            for (int g0 = 0; g0 < total; g0 += 16) {
                const int j = g0 + li;             // A row li: the j-th wanted lane
                const bool ok = j < total;
                const int src = !ok ? 0 : (j < clo ? nth_set_bit(wlo, j)
                                                   : 32 + nth_set_bit(whi, j - clo));
                const int vid = __shfl(v, src, SSA_WAVE);
                const T *kr = kb + (int64_t)SSA_IDX(ok ? vid : 0, p.M, 0) * p.ksn;
                f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
                for (int s = 0; s < KS; ++s) {
                    const int e0 = 32 * s + 8 * lg;
                    const V a = (ok && e0 < p.d)
                                    ? __builtin_bit_cast(V, *reinterpret_cast<const uint4 *>(kr + e0))
                                    : __builtin_bit_cast(V, make_uint4(0, 0, 0, 0));
                    const V b = e0 < p.d
                                    ? __builtin_bit_cast(V, *reinterpret_cast<const uint4 *>(qr + e0))
                                    : __builtin_bit_cast(V, make_uint4(0, 0, 0, 0));
                    acc = Mfma16<T>::mma(a, b, acc);
                }
                // lane (li, lg) holds rows 4 lg .. 4 lg + 3, every column alike:
                // row r is read from lane 16 (r / 4) + r % 4, which offers acc[li % 4]
                const int sel = li & 3;
                const float x = sel == 0 ? acc[0] : sel == 1 ? acc[1] : sel == 2 ? acc[2] : acc[3];
                const int r = (rank - g0) & 15;
                const float y = __shfl(x, 16 * (r >> 2) + (r & 3), SSA_WAVE);
                if (want && rank >= g0 && rank < g0 + 16) out = score_key(y);
            }
            return out;
        }
    }
    float acc = 0.f;
    if (want) {
        const T *kr = kb + (int64_t)SSA_IDX(v, p.M, 0) * p.ksn;
        for (int c = 0; c < p.d; ++c) acc = fmaf(to_f32(qr[c]), to_f32(kr[c]), acc);
    }
    return want ? score_key(acc) : 0u;
}


// exact_keys for up to 64 wanted lanes with every round's K rows in flight
// before the first product (the same MFMA k steps, operand placement and
// results as exact_keys): for callers with registers to spare, whose rounds
// would otherwise wait on their loads one after another.  KSM: k steps the
// instance holds (>= ceil(d / 32)).
template <typename T, int KSM>
__device__ uint32_t exact_keys_wide(const SelP &p, const T *qr, const T *kb, int v, bool want) {
    if constexpr (std::is_same<T, float>::value || KSM == 0) {
        return exact_keys<T>(p, qr, kb, v, want);
    } else {
        if (!p.mfma) return exact_keys<T>(p, qr, kb, v, want);
        using V = typename Mfma16<T>::vec;
        const int lane = lane_id();
        const uint64_t wm = wave_ballot(want);
        const int li = lane & 15, lg = lane >> 4;
        const int KS = (p.d + 31) >> 5;
        const int rank = lanes_below(wm);
        const int total = __popcll(wm);
        const uint32_t wlo = (uint32_t)wm, whi = (uint32_t)(wm >> 32);
        const int clo = __popc(wlo);
        V a[4][KSM];
        V b[KSM];
#pragma unroll
        for (int s = 0; s < KSM; ++s) {
            const int e0 = 32 * s + 8 * lg;
            b[s] = (s < KS && e0 < p.d)
                       ? __builtin_bit_cast(V, *reinterpret_cast<const uint4 *>(qr + e0))
                       : __builtin_bit_cast(V, make_uint4(0, 0, 0, 0));
        }
        // A rows of round g: the (16 g + li)-th wanted lane's key
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int j = 16 * g + li;
            const bool ok = j < total;
            const int src = !ok ? 0 : (j < clo ? nth_set_bit(wlo, j) : 32 + nth_set_bit(whi, j - clo));
            const int vid = __shfl(v, src, SSA_WAVE);
            const T *kr = kb + (int64_t)SSA_IDX(ok ? vid : 0, p.M, 0) * p.ksn;
#pragma unroll
            for (int s = 0; s < KSM; ++s) {
                const int e0 = 32 * s + 8 * lg;
                a[g][s] = (16 * g < total && ok && s < KS && e0 < p.d)
                              ? __builtin_bit_cast(V, *reinterpret_cast<const uint4 *>(kr + e0))
                              : __builtin_bit_cast(V, make_uint4(0, 0, 0, 0));
            }
        }
        uint32_t out = 0u;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            if (16 * g >= total) break;
            f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < KSM; ++s)
                if (s < KS) acc = Mfma16<T>::mma(a[g][s], b[s], acc);
            const int sel = li & 3;
            const float x = sel == 0 ? acc[0] : sel == 1 ? acc[1] : sel == 2 ? acc[2] : acc[3];
            const int r = (rank - 16 * g) & 15;
            const float y = __shfl(x, 16 * (r >> 2) + (r & 3), SSA_WAVE);
            if (want && rank >= 16 * g && rank < 16 * g + 16) out = score_key(y);
        }
        return out;
    }
}

// Inclusive prefix scans over the 64 lanes with DPP: row shifts by 1, 2, 4
// and 8 scan each row of 16 lanes, then row broadcasts 15 (into rows 1 and
// 3) and 31 (into rows 2 and 3) carry the row totals -- VALU only, no LDS
// round trips.  Lanes a shift or broadcast leaves out see the identity.
// Every lane must be active.
__device__ __forceinline__ int wave_incl_sum(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);   // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);   // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);   // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);   // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);   // row_bcast:15
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);   // row_bcast:31
    return v;
}
// values >= -1 (-1 is the identity)
__device__ __forceinline__ int wave_incl_max(int v) {
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x111, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x112, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x114, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x118, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x142, 0xA, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(-1, v, 0x143, 0xC, 0xF, false));
    return v;
}
// exclusive prefix sum and the wave total
__device__ __forceinline__ int wave_excl_scan(int v, int &total) {
    const int x = wave_incl_sum(v);
    total = __builtin_amdgcn_readlane(x, SSA_WAVE - 1);
    return x - v;
}

__device__ __forceinline__ void wave_compiler_fence() {
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
}

// Keys kept in LDS for the exact threshold search (CAP): 384, or 512 when kk
// is above SEL_CAP_LARGE_KK -- a buffer filled to CAP - 128 then holds more
// than kk keys, so its lower bound is raised once or twice per row instead
// of every few chunks (the larger buffer costs LDS, hence occupancy).
constexpr int SEL_CAP_SMALL = 384, SEL_CAP_LARGE = 512, SEL_CAP_LARGE_KK = 160;

// Per-wave LDS of the select kernel, in 32-bit words:
//   lch   [4*nlists]  per list, for its 64-member chunks: index of its first
//                     member id, score slot of its first member, members below
//                     the query (the cutoff), index of its first chunk in the
//                     row's chunk sequence
//   lst   [4*nlists]  per list: bucket start, size, offset of its kv-head/round
//                     row, overflow filler key (after the filler rule: the key
//                     if it is marked seen, else -1)
//   bm    [words]     seen bitmap, later the merge bitmap
//   ckey  [CAP+64]    kept keys >= the lower bound; the last 64 entries take
//                     the stores of lanes that append nothing
//   cval  [CAP+64]    key id of each compacted key (ckey and cval together span
//                     at least `words`: the overflow path's second bitmap)
//   LSH mode: ekey/eval/eslot [kk] the selected entries
constexpr int SEL_PIPE = 2;            // chunks per group in pass 1
// ckey + cval, which also hold the overflow path's second seen bitmap
// seen bitmap over M key ids, in 32-bit words rounded up to an even count
// (at M = 8192 the select kernel's per-wave words then come to 1,280: 8 waves
// per SIMD fill the 160 KB of LDS exactly)
__host__ __device__ inline int sel_bitmap_words(int M) { return ((M + 31) / 32 + 1) & ~1; }
__host__ __device__ inline int sel_buf_words(int words, int cap) {
    return 2 * (cap + 64) > words ? 2 * (cap + 64) : words;
}
__host__ __device__ inline int sel_lds_words(int words, int kk, bool lsh, int nlists, int cap) {
    return (8 * nlists + words + sel_buf_words(words, cap) + (lsh ? 3 * kk : 0) + 1) & ~1;
}

// Dedup one chunk of members (lanes in Min) against the seen bitmap, count the
// kept ones, and append the kept keys >= lo to the compacted buffer.  Every
// lane stores: lanes that append nothing (or would pass the capacity) write
// to their own slot past CAP, which is never read.
template <int CAP>
__device__ __forceinline__ void sel_absorb(uint32_t *bm, uint32_t *ckey, uint32_t *cval,
                                           uint64_t Min, int v, uint32_t kv, uint32_t lo,
                                           int &cnt, int &nkept) {
    const int lane = lane_id();
    const uint32_t bit = 1u << (v & 31);
    uint32_t old = 0u;
    if (in_mask(Min)) old = atomicOr(&bm[v >> 5], bit);
    const uint64_t km = Min & wave_ballot((old & bit) == 0u);
    nkept += __popcll(km);
    const uint64_t am = km & wave_ballot(kv >= lo);
    const int pos = cnt + lanes_below(am);
    const int dst = (in_mask(am) & (pos < CAP)) ? pos : CAP + lane;
    ckey[dst] = kv;
    cval[dst] = (uint32_t)v;
    cnt += __popcll(am);
}

// Largest t (resolved down to bit lo_bit) such that at least kk of the wave's
// keys k[0..NK) per lane are >= t, given base <= answer <= top: the answer shares
// the bit prefix of base and top, so only the bits below their highest
// difference are searched.  Stops early once exactly kk keys are >= t.
template <int NK>
__device__ __forceinline__ uint32_t kth_search(const uint32_t (&k)[NK], int kk, uint32_t base,
                                               uint32_t top, int lo_bit) {
    if (base >= top) return base;
    const int hb = 31 - __clz(base ^ top);
    uint32_t thr = hb >= 31 ? 0u : (base & ~((2u << hb) - 1u));
#pragma unroll 1
    for (int bit = hb; bit >= lo_bit; --bit) {
        const uint32_t cand = thr | (1u << bit);
        int tot = 0;                   // one compare-to-mask + scalar popcount per slot
#pragma unroll
        for (int i = 0; i < NK; ++i) tot += __popcll(wave_ballot(k[i] >= cand));
        if (tot >= kk) {
            thr = cand;
            if (tot == kk) break;
        }
    }
    return thr;
}


// FULL mode tail (merge_neighbors, sparse_attention.py:966-1089): `bm` holds
// the selected LSH keys; adds the window (:368-376), the globals, key 0 when a
// -inf slot at or past G falls back to it (:948-957), removes the query itself
// and writes [self] ++ the ascending union, zero-padded and marked invalid.
// scr: LDS scratch of scr_cap ints (free at this point).
__device__ void full_merge_emit(uint32_t *bm, const SelP &p, int n, int64_t row, int f,
                                int32_t *scr, int scr_cap) {
    const int lane = lane_id();
    const int kk = p.kk;
    if (!p.cross) {
        // the window {clamp(n + o) : |o| <= window, o <= 0 if causal} is the
        // range [a, e]: one mask per word
        const int a = min(max(n - p.window, 0), p.M - 1);
        const int e = min(max(p.causal ? n : n + p.window, 0), p.M - 1);
        for (int w = (a >> 5) + lane; w <= (e >> 5); w += SSA_WAVE) {
            const int lo = max(a - 32 * w, 0), hi = min(e - 32 * w, 31);
            const uint32_t m = (hi == 31 ? 0xffffffffu : ((2u << hi) - 1u)) & ~((1u << lo) - 1u);
            atomicOr(&bm[w], m);
        }
    }
    for (int j = lane; j < p.G; j += SSA_WAVE) bm_set(bm, (int)p.glob[j]);
    if (lane == 0 && (f > p.G ? f : p.G) < kk) bm_set(bm, 0);
    wave_lds_sync();
    if (!p.cross && lane == 0) atomicAnd(&bm[n >> 5], ~(1u << (n & 31)));
    wave_lds_sync();

    const int self = p.cross ? 0 : 1;
    const int ks = p.Kout - self;
    // slot i gets key id v (valid) or the padding; as int64 + valid byte, or
    // as one int32 with -1 for padding
    auto put = [&](int i, int v, bool valid) {
        const int64_t o = SSA_IDX(row * p.Kout + SSA_IDX(i, p.Kout, 4), p.rows_all * p.Kout, 4);
        if (p.out_idx32) {
            p.out_idx32[o] = valid ? v : -1;
        } else {
            p.out_idx[o] = valid ? (int64_t)v : 0;
            p.out_valid[o] = valid ? 1 : 0;
        }
    };
    const int wpl = (p.words + SSA_WAVE - 1) / SSA_WAVE;
    const int w0 = lane * wpl;
    int cntb = 0;
    for (int w = w0; w < w0 + wpl && w < p.words; ++w) cntb += __popc(bm[w]);
    int total;
    const int pos = wave_excl_scan(cntb, total);
    const int filled = total < ks ? total : ks;
    if (ks <= scr_cap) {
        // output slot t holds the (t - s)-th key of the word whose first key
        // is at slot s, the last word start at or before t: mark word starts,
        // then a running max over the slots finds s
        for (int t = lane; t < ks; t += SSA_WAVE) scr[t] = -1;
        wave_lds_sync();
        int q = pos;
        for (int w = w0; w < w0 + wpl && w < p.words; ++w) {
            const int c = __popc(bm[w]);
            if (c > 0 && q < ks) scr[q] = w;
            q += c;
        }
        wave_lds_sync();
        int carry = -1;
        for (int t0 = 0; t0 < filled; t0 += SSA_WAVE) {
            const int t = t0 + lane;
            const bool in = t < filled;
            int s = wave_incl_max((in && scr[t] >= 0) ? t : -1);
            s = max(s, carry);
            carry = __builtin_amdgcn_readlane(s, SSA_WAVE - 1);
            if (in) {
                const int w = scr[s];
                put(self + t, w * 32 + nth_set_bit(bm[w], t - s), true);
            }
        }
    } else {
        int q = pos;
        for (int w = w0; w < w0 + wpl && w < p.words && q < ks; ++w) {
            uint32_t word = bm[w];
            while (word && q < ks) {
                const int bitp = __ffs(word) - 1;
                word &= word - 1;
                put(self + q, w * 32 + bitp, true);
                ++q;
            }
        }
    }
    for (int i = self + filled + lane; i < p.Kout; i += SSA_WAVE) {
        put(i, 0, false);
    }
    if (self && lane == 0) {
        put(0, n, true);
    }
}

// kk-th largest of the cnt compacted keys, known to lie in [lo, hi] and
// resolved down to bit lo_bit: the threshold thr, how many keys equal to it
// are needed (need), and whether more equal keys than needed exist (btie).
// NK keys per lane cover cnt.
template <int NK>
__device__ __forceinline__ void sel_threshold(const uint32_t *ckey, int cnt, int kk, uint32_t lo,
                                              uint32_t hi, int lo_bit, uint32_t &thr, int &need,
                                              bool &btie) {
    const int lane = lane_id();
    uint32_t cv[NK];
#pragma unroll
    for (int i = 0; i < NK; ++i) cv[i] = ckey[lane + SSA_WAVE * i];
#pragma unroll
    for (int i = 0; i < NK; ++i) cv[i] = lane + SSA_WAVE * i < cnt ? cv[i] : 0u;
    uint32_t mx = 0u, mn = 0xffffffffu;
#pragma unroll
    for (int i = 0; i < NK; ++i) {
        mx = cv[i] > mx ? cv[i] : mx;
        mn = (cv[i] != 0u && cv[i] < mn) ? cv[i] : mn;
    }
    mx = wave_max_u(mx);
    mn = wave_min_u(mn);
    thr = kth_search(cv, kk, lo > mn ? lo : mn, hi < mx ? hi : mx, lo_bit);
    int ge = 0, gt = 0;
#pragma unroll
    for (int i = 0; i < NK; ++i) {
        ge += __popcll(wave_ballot(cv[i] >= thr));
        gt += __popcll(wave_ballot(cv[i] > thr));
    }
    need = kk - gt;
    btie = ge - gt > need;
}

// Entries of the buffer whose codes tie at the kk-th place (bit i of ebits:
// entry lane + 64 i is one, and now holds its exact key): the need-th largest
// exact key among them decides.  Each such entry is rewritten to
// pf | 2 / 1 / 0 (above / equal to / below that key), and the threshold
// becomes pf | 1 with `need` of those equal to it taken, so the selection
// compares codes everywhere else.
template <int NK>
__device__ __forceinline__ void sel_boundary(uint32_t *ckey, int ebits, uint32_t pf, int &need,
                                             bool &btie) {
    const int lane = lane_id();
    uint32_t xv[NK];
    uint32_t mx = 0u, mn = 0xffffffffu;
#pragma unroll
    for (int i = 0; i < NK; ++i) {
        xv[i] = ((ebits >> i) & 1) ? ckey[lane + SSA_WAVE * i] : 0u;
        mx = xv[i] > mx ? xv[i] : mx;
        mn = (xv[i] != 0u && xv[i] < mn) ? xv[i] : mn;
    }
    mx = wave_max_u(mx);
    mn = wave_min_u(mn);
    const uint32_t xthr = kth_search(xv, need, mn, mx, 0);
    int gt = 0, eq = 0;
#pragma unroll
    for (int i = 0; i < NK; ++i) {
        gt += __popcll(wave_ballot(xv[i] > xthr));
        eq += __popcll(wave_ballot(xv[i] == xthr));
    }
#pragma unroll
    for (int i = 0; i < NK; ++i)
        if ((ebits >> i) & 1)
            ckey[lane + SSA_WAVE * i] = pf | (xv[i] > xthr ? 2u : (xv[i] == xthr ? 1u : 0u));
    need -= gt;
    btie = eq > need;
}

// One wavefront per query row.  The reference scans the query's candidate
// stream (round, id set, slot) and keeps each key at its first occurrence,
// valid or not (:884-890).  Real members of a list all carry their own score,
// so which of their occurrences comes first does not change the selection:
// only the query's own key (every future member becomes the query when
// causal, :698-709) and the overflow filler keys (invalid slots, :691-696)
// depend on the stream order, and both are settled up front:
//  query   kept with its own score when its first occurrence (from the cut
//          table, earliest list first) is valid;
//  filler  a filler key whose first occurrence is a filler slot is marked seen
//          (never kept); the real occurrences before it are found through the
//          key's permutation position in each list's round.
// What remains is order-free, so each list contributes only its members below
// the query (causal; all otherwise) in ascending id order, whose scores the
// rescore wrote contiguously, plus glob ++ 0 for an empty bucket:
//  pass 1  members whose key is below a running lower bound are dropped
//          first (a key scores the same in every list, so each of its
//          occurrences is dropped alike); the rest are deduplicated by a
//          test-and-set of the key's bit in LDS, and the kept ones compacted
//          (key, id) into LDS.  The count of kept keys is exact while the
//          bound is 0; once it is raised, at least kk distinct keys lie above
//          it, which is all the selection needs of the count;
//  bound   the kk-th largest buffered key over the top 16 bits raises the
//          lower bound whenever the buffer fills (the buffer is a subset of the
//          stream);
//  search  exact kk-th largest over the compacted keys (bitwise, early exit);
//  emit    selected = key > thr, or key == thr for the first `need`; rows where
//          that choice matters (a tied kk-th key, equal selected keys in LSH
//          mode) are handed to the exact replay.  LSH mode writes the selected
//          keys by descending score, FULL mode merges them with the window and
//          the globals through a key bitmap.
// WIDE: the cut entries' field width and the rows per workgroup come from
// p.cbits and p.waves (beyond 65,536 keys, or when fewer than SEL_WAVES rows
// fit a workgroup's LDS); else they are 16 and SEL_WAVES, as constants.
template <typename T, bool LSH_MODE, bool CAUSAL, int CAP, bool WIDE>
// Registers are held to what 8 waves per SIMD allow (the kernel waits on
// memory and LDS; the bench workload's 5 KB of LDS per wave fits 8 as well).
// The 512-key buffer's rows (large kk, whose LDS allows fewer waves anyway)
// take the register budget of 7, which spills fewer scalar registers.
__global__ void __launch_bounds__(SEL_WAVES * SSA_WAVE)
__attribute__((amdgpu_waves_per_eu(CAP >= SEL_CAP_LARGE ? 7 : 8, 8)))
select_kernel(SelP p) {
    extern __shared__ uint32_t sel_smem[];
    const int64_t blk = xcd_logical_block(blockIdx.x, p.nblocks);
    if (blk >= p.nblocks) return;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / SSA_WAVE);   // wave-uniform
    const int64_t rd = blk * (WIDE ? p.waves : SEL_WAVES) + wid;
    if (rd >= p.rows) return;
    // causal rows cost more the later their position (more members below the
    // query): a head's rows go in descending position, so the launch ends on
    // its cheapest rows instead of its dearest
    const int64_t rloc =
        CAUSAL ? (int64_t)((uint32_t)rd / (uint32_t)p.N) * p.N + (p.N - 1 - (int)((uint32_t)rd % (uint32_t)p.N))
               : rd;
    const int lane = lane_id();
    const int nl = p.nlists;
    int4 *lch = (int4 *)(sel_smem + (int64_t)wid * sel_lds_words(p.words, p.kk, LSH_MODE, nl, CAP));
    int4 *lst = lch + nl;
    uint32_t *bm = (uint32_t *)(lst + nl);
    uint32_t *ckey = bm + p.words;
    uint32_t *cval = ckey + CAP + 64;
    uint32_t *ekey = ckey + sel_buf_words(p.words, CAP);
    uint32_t *eval = ekey + p.kk;
    uint32_t *eslot = eval + p.kk;

    const int n = (int)((uint32_t)rloc % (uint32_t)p.N);     // rows of a chunk < 2^31
    const int bhl = (int)((uint32_t)rloc / (uint32_t)p.N);
    const uint16_t *shead = p.S + (int64_t)bhl * nl * p.N * p.Cs;
    const int64_t row = (int64_t)p.bh0 * p.N + rloc;
    // exact keys (where codes tie) of this query row: its q row and its kv
    // head's K rows are located only on those rare paths
    auto exact = [&](int v, bool want) {
        const int bh = p.bh0 + bhl;
        const int hq = bh % p.Hq;
        const T *qr = (const T *)p.q + (bh / p.Hq) * p.qsb + hq * p.qsh + (int64_t)n * p.qsn;
        const T *kb = (const T *)p.k + (bh / p.Hq) * p.ksb + (hq / p.rep) * p.ksh;
        return exact_keys<T>(p, qr, kb, v, want);
    };
    // scores the candidate lists do not carry (computed with the rescore's
    // arithmetic, so equal keys get equal scores): the query's own key and the
    // empty-bucket list glob ++ 0
    const float *arow = p.aux + rloc * p.NA;
    const float qsc = arow[p.NA - 1];          // the query's code scale
    const uint32_t kself = CAUSAL ? score_key(arow[0]) : 0u;
    const uint32_t cself = CAUSAL ? score_code(arow[0], qsc) : 0u;
    // the empty-bucket list glob ++ 0: its first nge entries (the rest are
    // further zeros, never first occurrences), 64 at a time
    const int nge = min(p.G + 1, p.C);
    for (int w = lane; w < p.words; w += SSA_WAVE) bm[w] = 0u;

    // ---- per-list chunk data of the sorted prefixes, one lane per list
    int nch = 0;
    bool any_empty = false;            // some bucket is empty: glob ++ 0 (same for all)
    bool nkeep = false;                // the query's own key is kept
    bool nfound = !CAUSAL;
    bool any_fill = false;             // some list has an overflow filler below the query
    const int4 *crow = p.cut + rloc * nl;
    const int32_t *xrow = p.srix + rloc * nl;
    for (int l0 = 0; l0 < nl; l0 += SSA_WAVE) {
        const int list = l0 + lane;
        const bool in = list < nl;
        const int4 ct = in ? crow[list] : make_int4(0, 0, 0, 0);
        const int so = in ? xrow[list] : 0;
        const int cb = WIDE ? p.cbits : 16;
        const uint32_t cmask = (1u << cb) - 1u;
        const int sz = (int)(ct.y & cmask), cutoff = (int)(ct.z & cmask);
        const int st = (int)((uint32_t)ct.z >> cb), fk = (int)((uint32_t)ct.y >> cb);
        // a filler that cannot matter (no overflow, or past the query) is -1
        const bool fl = in && sz > 0 && sz < p.C && (!CAUSAL || fk < n);
        if (in) lst[list] = make_int4(st, sz, ct.x - st, fl ? fk : -1);
        any_fill = any_fill || wave_ballot(fl) != 0ull;
        const int nc = (in && sz > 0) ? (cutoff + SSA_WAVE - 1) / SSA_WAVE : 0;
        int ncs;
        const int at = nch + wave_excl_scan(nc, ncs);
        if (in) lch[list] = make_int4(ct.x, so, cutoff, at);
        nch += ncs;
        any_empty = any_empty || wave_ballot(in && sz == 0) != 0ull;
        if (!nfound) {
            // earliest list holding the query's key: its first slot decides
            const uint64_t fm = wave_ballot(in && (ct.w >> 1) < p.C);
            if (fm != 0ull) {
                const uint64_t vm = wave_ballot(in && (ct.w & 1));
                nkeep = ((vm >> (__ffsll((long long)fm) - 1)) & 1ull) != 0ull;
                nfound = true;
            }
        }
    }
    nch = __builtin_amdgcn_readfirstlane(nch);
    // glob ++ 0 (:711-737), entries c0 .. c0 + 63: lane j's id, code and key
    // (its score from the aux row: glob scores, then key 0's)
    auto glob_entry = [&](int c0, int &id, uint32_t &code, uint32_t &key) {
        const int c = c0 + lane;
        id = 0; code = 0u; key = 0u;
        if (c < nge) {
            key = score_key(arow[1 + c]);
            code = score_code(arow[1 + c], qsc);
            id = c < p.G ? (int)p.glob[c] : 0;
        }
        uint64_t Min = wave_ballot(c < nge);
        if (CAUSAL) Min &= ~wave_ballot(c < nge && id == n);   // the query's own key is settled
        return Min;
    };
    // glob slots 1 .. nge; the chunks' stream slots follow
    const int slot0 = 1 + SSA_WAVE * (int)((nge + SSA_WAVE - 1) / SSA_WAVE);
    wave_lds_sync();

    // ---- overflow fillers: list L (0 < size < C) holds its round's filler key
    // f at slots size..C-1, invalid.  Lane pairs (L, L2 <= L) look for a real
    // occurrence of f in list L2 or a filler of f in an earlier list; with
    // neither, f's first occurrence is L's filler and f is never kept.  The
    // table marked such lists by a filler key >= 0 (else -1, which every
    // later use of the key reads as "no filler").
    if (any_fill) {
        uint32_t *fhit = ckey;         // per list: f occurs earlier (scratch before pass 1)
        for (int w = lane; w < (nl + 31) / 32; w += SSA_WAVE) fhit[w] = 0u;
        wave_lds_sync();
        const int np = nl * nl;
        for (int p0 = 0; p0 < np; p0 += SSA_WAVE) {
            const int pi = p0 + lane;
            const int L = nl <= 1024 ? (int)__umulhi((uint32_t)pi, p.nl_magic) : pi / nl;
            const int L2 = pi - L * nl;
            if (pi < np && L2 <= L) {
                const int4 a = lst[L];
                const int v = a.w;                     // >= 0: L's filler can matter
                if (v >= 0) {
                    const int4 c2 = lst[L2];
                    bool hit;
                    if (c2.y == 0) {                   // glob ++ 0, all valid
                        hit = v == 0 && p.G < p.C;
                        const int gl = min(p.G, p.C);
                        for (int j = 0; j < gl; ++j) hit |= (int)p.glob[j] == v;
                    } else {
                        hit = L2 < L && c2.y < p.C && c2.w == v;
                        if (!hit) {
                            const int pos = p.inv[SSA_IDX(c2.z + v, p.perm_bytes / 4, 1)];
                            hit = pos >= c2.x && pos < c2.x + min(c2.y, p.C);
                        }
                    }
                    if (hit) atomicOr(&fhit[L >> 5], 1u << (L & 31));
                }
            }
        }
        wave_lds_sync();
        for (int L = lane; L < nl; L += SSA_WAVE) {
            const int4 a = lst[L];
            const bool mark = a.w >= 0 && !((fhit[L >> 5] >> (L & 31)) & 1u);
            if (mark) bm_set(bm, a.w);
            lst[L].w = mark ? a.w : -1;
        }
        wave_lds_sync();
    }

    // Descriptor of chunk dwin + lane: index of its first member id, lane mask
    // (low), score slot of its first member, lane mask (high); zero past the
    // last chunk.  Its list is the last one whose first chunk is at or before
    // it (lists without chunks share the next list's first chunk index).
    const int lstep = nl > 1 ? 1 << (31 - __clz(nl - 1)) : 0;
    auto desc_window = [&](int dwin) {
        const int ci = dwin + lane;
        int4 d = make_int4(0, 0, 0, 0);
        if (ci < nch) {
            int L = 0;
            for (int step = lstep; step > 0; step >>= 1)
                if (L + step < nl && lch[L + step].w <= ci) L += step;
            const int4 e = lch[L];
            const int c0 = (ci - e.w) * SSA_WAVE;
            const uint64_t m = lanes_mask(e.z - c0);
            d = make_int4(e.x + c0, (int)(uint32_t)m, e.y + c0, (int)(uint32_t)(m >> 32));
        }
        return d;
    };

    // ---- pass 1: dedup, and the kept keys >= lo into LDS.  lo is a lower
    // bound of the final threshold: whenever the buffer nears its capacity, lo
    // is raised to (a 16-bit floor of) the kk-th largest key in the buffer --
    // a subset of the stream -- and the buffer is filtered in place.
    const int kk = p.kk;
    // checked once per group of SEL_PIPE chunks: a group adds at most 64 * SEL_PIPE keys
    const int fill = CAP - SEL_PIPE * SSA_WAVE;
    int nkept = nkeep ? 1 : 0, cnt = 0;
    uint32_t lo = 0u;
    bool overflow = false;
    // the buffer holds 16-bit score codes in the high half of each key
    if (nkeep) {
        if (lane == 0) { ckey[0] = cself << 16; cval[0] = (uint32_t)n; }
        cnt = 1;
    }
    if (any_empty) {                   // glob ++ 0; the query's own key is settled
        for (int c0 = 0; c0 < nge; c0 += SSA_WAVE) {
            int gid;
            uint32_t gc, gk;
            const uint64_t Min = glob_entry(c0, gid, gc, gk);
            sel_absorb<CAP>(bm, ckey, cval, Min, gid, gc << 16, lo, cnt, nkept);
        }
    }
    // Chunks are processed PIPE at a time; the loads of the next group are
    // issued before the current group is deduplicated, so a wave always has
    // one group of member ids and scores in flight (two register sets, A and
    // B, alternate so that no loaded value is copied).  Loads are unconditional
    // raw buffer loads (scalar chunk offset, constant lane offset): lanes past
    // a chunk's members read in-range data or 0.  The group's bitmap
    // test-and-sets are issued back to back: LDS operations of a wave
    // complete in order, so each chunk still sees the bits the chunks before
    // it set.
    constexpr int PIPE = SEL_PIPE;
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc((void *)p.sid, (short)0, p.perm_bytes, SSA_BUF_FLAGS);
    const __amdgpu_buffer_rsrc_t srs =
        __builtin_amdgcn_make_buffer_rsrc((void *)shead, (short)0, (int)p.head_bytes, SSA_BUF_FLAGS);
    const int lane4 = lane * 4, lane2 = lane * 2;
    uint64_t mA[PIPE], mB[PIPE];
    int rA[PIPE], rB[PIPE];
    uint32_t sA[PIPE], sB[PIPE];
    // descriptors of 64 chunks at a time, lane j holding chunk (window + j);
    // a chunk's fields are read with a lane select, so no LDS read waits in
    // front of each group's loads.  Chunks past the last read as empty.
    int dwin = 0;
    int4 dl = desc_window(0);
    auto fetch = [&](int ci0, uint64_t (&m)[PIPE], int (&raw)[PIPE], uint32_t (&sk)[PIPE])
        __attribute__((always_inline)) {
        if ((ci0 & ~(SSA_WAVE - 1)) != dwin) {      // groups never straddle a window
            dwin = ci0 & ~(SSA_WAVE - 1);
            dl = desc_window(dwin);
        }
#pragma unroll
        for (int u = 0; u < PIPE; ++u) {
            const int j = (ci0 + u) & (SSA_WAVE - 1);
            m[u] = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(dl.w, j) << 32) |
                   (uint32_t)__builtin_amdgcn_readlane(dl.y, j);
            const int x = __builtin_amdgcn_readlane(dl.x, j);
            const int z = __builtin_amdgcn_readlane(dl.z, j);
            raw[u] = __builtin_amdgcn_raw_buffer_load_b32(prs, lane4, x * 4, 0);
            sk[u] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(srs, lane2, (int)((uint32_t)z << 1), 0)
                    << 16;
        }
    };
    auto absorb = [&](const uint64_t (&cm)[PIPE], const int (&craw)[PIPE],
                      const uint32_t (&csk)[PIPE]) __attribute__((always_inline)) {
        uint32_t old[PIPE], bit[PIPE];
        uint64_t lm[PIPE];
#pragma unroll
        for (int u = 0; u < PIPE; ++u) {
            bit[u] = 1u << (craw[u] & 31);
            old[u] = 0u;
            lm[u] = cm[u] & wave_ballot(csk[u] >= lo);
            if (in_mask(lm[u])) old[u] = atomicOr(&bm[craw[u] >> 5], bit[u]);
        }
#pragma unroll
        for (int u = 0; u < PIPE; ++u) {
            const uint64_t am = lm[u] & wave_ballot((old[u] & bit[u]) == 0u);
            nkept += __popcll(am);
            const int pos = cnt + lanes_below(am);
            const int dst = (in_mask(am) & (pos < CAP)) ? pos : CAP + lane;
            ckey[dst] = csk[u];
            cval[dst] = (uint32_t)craw[u];
            cnt += __popcll(am);
        }
        if (cnt >= fill && cnt >= kk && !overflow) {
            wave_lds_sync();
            const int m0 = cnt < CAP ? cnt : CAP;
            uint32_t sv[CAP / SSA_WAVE];
#pragma unroll
            for (int i = 0; i < CAP / SSA_WAVE; ++i) sv[i] = ckey[lane + SSA_WAVE * i];
#pragma unroll
            for (int i = 0; i < CAP / SSA_WAVE; ++i)
                sv[i] = lane + SSA_WAVE * i < m0 ? sv[i] : 0u;   // slots past the count are stale
            uint32_t mx = 0u, mn = 0xffffffffu;
#pragma unroll
            for (int i = 0; i < CAP / SSA_WAVE; ++i) {
                mx = sv[i] > mx ? sv[i] : mx;
                mn = (sv[i] != 0u && sv[i] < mn) ? sv[i] : mn;
            }
            mx = wave_max_u(mx);
            mn = wave_min_u(mn);
            const uint32_t base0 = lo > mn ? lo : mn;     // every buffered key >= lo
            // any lower bound of the kk-th key will do: the search stops 6 bits
            // below the highest bit in which the buffer's keys differ
            const int hbit = base0 >= mx ? 16 : 31 - __clz(base0 ^ mx);
            const uint32_t nlo = kth_search(sv, kk, base0, mx, max(16, hbit - 5));
            lo = nlo > lo ? nlo : lo;
            uint32_t sl[CAP / SSA_WAVE];
#pragma unroll
            for (int i = 0; i < CAP / SSA_WAVE; ++i) sl[i] = cval[lane + SSA_WAVE * i];
            wave_lds_sync();
            int nc = 0;
#pragma unroll
            for (int i = 0; i < CAP / SSA_WAVE; ++i) {
                const bool t = sv[i] >= lo && sv[i] != 0u;
                const uint64_t m = wave_ballot(t);
                if (t) { ckey[nc + lanes_below(m)] = sv[i]; cval[nc + lanes_below(m)] = sl[i]; }
                nc += __popcll(m);
            }
            overflow = cnt > CAP;
            cnt = nc;
            wave_lds_sync();
        }
    };
    // Fetches past the last chunk are unconditional (they read the empty tail
    // chunks), so every path into a group sees the same loads in flight and
    // waits only for its own.
    fetch(0, mA, rA, sA);
    for (int ci0 = 0; ci0 < nch; ci0 += 2 * PIPE) {
        fetch(ci0 + PIPE, mB, rB, sB);
        absorb(mA, rA, sA);
        if (ci0 + PIPE >= nch) break;
        fetch(ci0 + 2 * PIPE, mA, rA, sA);
        absorb(mB, rB, sB);
    }
    overflow = overflow || cnt > CAP;
    wave_lds_sync();
    // with the bound raised, nkept misses the keys below it, but at least kk
    // distinct keys lie above it
    const int nk = (lo > 0u && nkept <= kk) ? kk + 1 : nkept;

    // re-walk the kept keys (rare path: the buffer overflowed, so it is free
    // to hold a fresh seen bitmap).  A key comes as (xm 0) its code << 16;
    // (1) its exact key if its code is pfx, else 0; (2) its code << 16, with
    // the low bits 2 / 1 / 0 if its code is pfx and its exact key is above /
    // equal to / below xthr; (3) its exact key.
    auto walk_kept = [&](int xm, uint32_t pfx, uint32_t xthr, auto &&fn) {
        auto kv_of = [&](uint32_t c, uint32_t x) -> uint32_t {
            if (xm == 3) return x;
            if (xm == 1) return c == pfx ? x : 0u;
            if (xm == 2 && c == pfx) return (c << 16) | (x > xthr ? 2u : (x == xthr ? 1u : 0u));
            return c << 16;
        };
        uint32_t *bm2 = ckey;
        wave_lds_sync();
        for (int w = lane; w < p.words; w += SSA_WAVE) bm2[w] = 0u;
        wave_lds_sync();
        for (int L = lane; L < nl; L += SSA_WAVE)
            if (lst[L].w >= 0) bm_set(bm2, lst[L].w);
        wave_lds_sync();
        if (nkeep) fn(lane == 0, kv_of(cself, kself), n, 0);
        auto walk_chunk = [&](uint64_t Min, int v, uint32_t kv, int slot) {
            const uint32_t bit = 1u << (v & 31);
            uint32_t old = 0u;
            if (in_mask(Min)) old = atomicOr(&bm2[v >> 5], bit);
            fn(in_mask(Min) && !(old & bit), kv, v, slot);
        };
        if (any_empty) {
            for (int c0 = 0; c0 < nge; c0 += SSA_WAVE) {
                int gid;
                uint32_t gc, gk;
                const uint64_t Min = glob_entry(c0, gid, gc, gk);
                walk_chunk(Min, gid, kv_of(gc, gk), 1 + c0 + lane);
            }
        }
        int4 dw = make_int4(0, 0, 0, 0);
        for (int ci = 0; ci < nch; ++ci) {
            const int j = ci & (SSA_WAVE - 1);
            if (j == 0) dw = desc_window(ci);
            const uint64_t Min = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(dw.w, j) << 32) |
                                 (uint32_t)__builtin_amdgcn_readlane(dw.y, j);
            int v = 0;
            uint32_t c = 0u;
            if (in_mask(Min)) {
                v = p.sid[SSA_IDX(__builtin_amdgcn_readlane(dw.x, j) + lane, p.perm_bytes / 4, 2)];
                c = shead[SSA_IDX((int64_t)(uint32_t)__builtin_amdgcn_readlane(dw.z, j) + lane,
                                  p.head_bytes / 2, 3)];
            }
            const bool xw = in_mask(Min) && (xm == 3 || (xm != 0 && c == pfx));
            uint32_t x = 0u;
            if (wave_ballot(xw) != 0ull) x = exact(v, xw);
            walk_chunk(Min, v, kv_of(c, x), slot0 + ci * SSA_WAVE + lane);
        }
    };
    // kk2-th largest key of the kept stream as walk mode xm gives it, over bits
    // hi_bit .. lo_bit (above them: t0), with how many keys lie above it and on it
    auto walk_search = [&](int xm, uint32_t pfx, int kk2, uint32_t t0, int hi_bit, int lo_bit,
                           int &gt, int &ge) {
        for (int bit = hi_bit; bit >= lo_bit; --bit) {
            const uint32_t cand = t0 | (1u << bit);
            int c = 0;
            walk_kept(xm, pfx, 0u, [&](bool keep, uint32_t kv, int, int) {
                c += __popcll(wave_ballot(keep & (kv >= cand)));
            });
            if (c >= kk2) t0 = cand;
        }
        ge = 0;
        gt = 0;
        walk_kept(xm, pfx, 0u, [&](bool keep, uint32_t kv, int, int) {
            ge += __popcll(wave_ballot(keep & (kv >= t0)));
            gt += __popcll(wave_ballot(keep & (kv > t0)));
        });
        return t0;
    };

    // ---- threshold
    uint32_t thr = 0u;                 // 0: every kept key is selected
    int need = 0;
    bool btie = false;                 // several kept keys equal the kk-th one
    const bool compacted = !overflow;  // every key >= the threshold is in ckey
    uint32_t wpfx = 0x10000u, wxthr = 0u;   // overflow path: the code resolved by exact keys
    // kk-th largest buffered key in [base, top], resolved down to bit lo_bit;
    // keys held per lane: as few as the buffer needs
    auto threshold = [&](uint32_t base, uint32_t top, int lo_bit) {
        if (cnt <= 2 * SSA_WAVE)
            sel_threshold<2>(ckey, cnt, kk, base, top, lo_bit, thr, need, btie);
        else if (cnt <= 4 * SSA_WAVE)
            sel_threshold<4>(ckey, cnt, kk, base, top, lo_bit, thr, need, btie);
        else
            sel_threshold<CAP / SSA_WAVE>(ckey, cnt, kk, base, top, lo_bit, thr, need, btie);
    };
    // exact keys of the buffered entries whose key is `only` (every entry: 0);
    // bit i of the result: lane's entry lane + 64 i now holds its exact key
    auto exact_buffer = [&](uint32_t only) {
        int ebits = 0;
        for (int i = 0; i * SSA_WAVE < cnt; ++i) {
            const int e = lane + SSA_WAVE * i;
            const bool in = e < cnt && (only == 0u || ckey[e] == only);
            if (wave_ballot(in) == 0ull) continue;
            const uint32_t x = exact(in ? (int)cval[e] : 0, in);
            if (in) {
                ckey[e] = x;
                ebits |= 1 << i;
            }
        }
        wave_lds_sync();
        return ebits;
    };
    if (compacted) {
        if (LSH_MODE) {
            // LSH mode ranks the selected keys by score: exact keys throughout
            exact_buffer(0u);
            if (nk > kk) threshold(0u, 0xffffffffu, 0);
        } else if (nk > kk) {
            threshold(lo, 0xffffffffu, 16);
            if (btie) {
                // more buffered codes equal the kk-th than are needed: the
                // exact keys of those entries decide among them
                const int ebits = exact_buffer(thr);
                if (cnt <= 2 * SSA_WAVE)
                    sel_boundary<2>(ckey, ebits, thr, need, btie);
                else if (cnt <= 4 * SSA_WAVE)
                    sel_boundary<4>(ckey, ebits, thr, need, btie);
                else
                    sel_boundary<CAP / SSA_WAVE>(ckey, ebits, thr, need, btie);
                thr |= 1u;
                wave_lds_sync();
            }
        }
    } else if (nk > kk) {
        // rare: search the whole kept stream, one walk per bit
        int gt, ge;
        if (LSH_MODE) {
            thr = walk_search(3, 0u, kk, 0u, 31, 0, gt, ge);
            need = kk - gt;
            btie = ge - gt > need;
        } else {
            thr = walk_search(0, 0u, kk, 0u, 31, 16, gt, ge);      // over the codes
            need = kk - gt;
            if (ge - gt > need) {
                // codes tie at the kk-th place: exact keys among that code
                wpfx = thr >> 16;
                wxthr = walk_search(1, wpfx, need, 0u, 31, 0, gt, ge);
                need -= gt;
                btie = ge - gt > need;
                thr |= 1u;
            }
        }
    }
    if (btie && lane == 0 && p.ties) atomicAdd(p.ties, 1);
    const int f = nk < kk ? nk : kk;

    // ---- emit the selected slots
    if (!LSH_MODE) {
        for (int w = lane; w < p.words; w += SSA_WAVE) bm[w] = 0u;
        wave_lds_sync();
    }
    int nsel = 0, eq_before = 0;
    auto take = [&](bool sel, uint32_t kv, int v, int slot) {
        if (!LSH_MODE) {
            atomicOr(&bm[v >> 5], sel ? (1u << (v & 31)) : 0u);
        } else {
            const uint64_t sm = wave_ballot(sel);
            if (sel) {
                const int pos = nsel + lanes_below(sm);
                ekey[pos] = kv;
                eval[pos] = (uint32_t)v;
                eslot[pos] = (uint32_t)slot;
            }
            nsel += __popcll(sm);
        }
    };
    auto decide = [&](bool keep, uint32_t kv) {
        const bool is_eq = keep & (kv == thr) & (thr != 0u);
        const uint64_t eqm = wave_ballot(is_eq);
        const bool sel = keep & ((kv > thr) | (is_eq & (eq_before + lanes_below(eqm) < need)));
        eq_before += __popcll(eqm);
        return sel;
    };
    if (compacted) {
        for (int e0 = 0; e0 < cnt; e0 += SSA_WAVE) {
            const int e = e0 + lane;
            const bool in = e < cnt;
            const uint32_t kv = in ? ckey[e] : 0u;
            const bool sel = decide(in, kv);
            const int v = in ? (int)cval[e] : 0;
            take(sel, kv, v, e);           // compacted index: increasing in stream order
        }
    } else {
        walk_kept(LSH_MODE ? 3 : 2, wpfx, wxthr, [&](bool keep, uint32_t kv, int v, int slot) {
            take(decide(keep, kv), kv, v, slot);
        });
    }
    wave_lds_sync();

    if (LSH_MODE) {
        int64_t *orow = p.out_idx + row * kk;
        bool dup = false;
        for (int e = lane; e < f; e += SSA_WAVE) {
            const uint32_t k0 = ekey[e], s0 = eslot[e];
            int rank = 0;
            for (int e2 = 0; e2 < f; ++e2) {
                const uint32_t k2 = ekey[e2];
                rank += (k2 > k0) || (k2 == k0 && eslot[e2] < s0);
                dup |= (k2 == k0) && (e2 != e);
            }
            orow[SSA_IDX(rank, kk, 9)] = (int64_t)eval[e];
        }
        for (int t = f + lane; t < kk; t += SSA_WAVE) orow[t] = t < p.G ? p.glob[t] : 0;
        // the order among equal scores (and a tied kk-th place) follows the
        // reference's nth_element / sort internals: replayed exactly later
        if ((btie || wave_ballot(dup)) && lane == 0 && p.tie_list)
            p.tie_list[atomicAdd(p.tie_count, 1)] = (int)row;
        return;
    }
    if (btie && lane == 0 && p.tie_list) p.tie_list[atomicAdd(p.tie_count, 1)] = (int)row;

    full_merge_emit(bm, p, n, row, f, (int32_t *)ckey, sel_buf_words(p.words, CAP));
}

// ------------------------------------------------------------------ exact top-k replay
// A row whose kk-th kept score is tied, or (LSH mode) whose selected scores are
// not all distinct, depends on how the reference's running top-k orders equal
// scores: torch.topk on the CPU is std::nth_element(kk-1) followed by
// std::sort of the first kk-1, over best ++ chunk, chunk by chunk (:904-922).
// Such rows are replayed here, one wavefront per row: the candidate stream is
// rebuilt chunk by chunk (same keys, scores and first-occurrence rule as the
// select kernel), and every nth_element / sort runs as libstdc++ runs it:
// median-of-three Hoare partitions (data-parallel, as in the bucket sort),
// heap fallbacks at the depth limit and final insertion sorts, all on keys
// ordered by the top-k comparator ("NaN first, then >").
constexpr int RP_WAVES = 2;
constexpr uint32_t RP_NEGINF = 0xff800000u;   // rank key of -inf: ~score_key(-inf)
constexpr int RP_STACK = 64;

// The per-wave replay carries key ids as 16-bit values up to 65,536 keys (a
// seen bitmap of at most 2,048 words), as 32-bit values beyond
__host__ __device__ inline bool rp_wide_ids(int words) { return words > 2048; }
__host__ __device__ inline int rp_cand_words(int W, int words) {
    return rp_wide_ids(words) ? W : (W + 1) / 2;
}
// words of one row of the per-wave replay: rank keys (W), key ids, TL/TR
// (two 16-bit lists), leaf bits, stack, bitmap, glob scores
__host__ __device__ inline int rp_lds_words(int W, int words) {
    return (2 * W + rp_cand_words(W, words) + (W + 31) / 32 + 1 + 3 * RP_STACK + words + 1) & ~1;
}

__device__ __forceinline__ void rp_sync() {
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// CT: 32-bit key ids (the per-wave replay) or 16-bit positions (the
// workgroup replay, whose rows hold fewer than 2^16 slots)
template <typename CT>
struct RpArr {
    uint32_t *key;     // rank keys: smaller = earlier in top-k order
    CT *cand;          // key ids (or positions) carried along
};

template <class A>
__device__ __forceinline__ void rp_swap(const A &a, int i, int j) {
    const uint32_t tk = a.key[i];
    const int32_t tc = a.cand[i];
    a.key[i] = a.key[j]; a.cand[i] = a.cand[j];
    a.key[j] = tk; a.cand[j] = tc;
}

// ---- single-lane heap routines (depth-limit fallbacks, partial_sort)
template <class A>
__device__ void rp_push_up(const A &a, int base, int hole, int top, uint32_t vk, int32_t vc) {
    int parent = (hole - 1) / 2;
    while (hole > top && a.key[base + parent] < vk) {
        a.key[base + hole] = a.key[base + parent];
        a.cand[base + hole] = a.cand[base + parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    a.key[base + hole] = vk;
    a.cand[base + hole] = vc;
}

template <class A>
__device__ void rp_adjust(const A &a, int base, int hole, int len, uint32_t vk, int32_t vc) {
    const int top = hole;
    int child = hole;
    while (child < (len - 1) / 2) {
        child = 2 * (child + 1);
        if (a.key[base + child] < a.key[base + child - 1]) child--;
        a.key[base + hole] = a.key[base + child];
        a.cand[base + hole] = a.cand[base + child];
        hole = child;
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
        child = 2 * (child + 1);
        a.key[base + hole] = a.key[base + child - 1];
        a.cand[base + hole] = a.cand[base + child - 1];
        hole = child - 1;
    }
    rp_push_up(a, base, hole, top, vk, vc);
}

// heap_select(f, mid, l): [f, mid) becomes a max-heap of the mid-f smallest
template <class A>
__device__ void rp_heap_select(const A &a, int f, int mid, int l) {
    const int len = mid - f;
    if (len >= 2) {
        for (int parent = (len - 2) / 2;; --parent) {
            rp_adjust(a, f, parent, len, a.key[f + parent], a.cand[f + parent]);
            if (parent == 0) break;
        }
    }
    for (int i = mid; i < l; ++i) {
        if (a.key[i] < a.key[f]) {
            const uint32_t vk = a.key[i];
            const int32_t vc = a.cand[i];
            a.key[i] = a.key[f];
            a.cand[i] = a.cand[f];
            rp_adjust(a, f, 0, len, vk, vc);
        }
    }
}

template <class A>
__device__ void rp_heap_sort(const A &a, int f, int l) {
    while (l - f > 1) {
        --l;
        const uint32_t vk = a.key[l];
        const int32_t vc = a.cand[l];
        a.key[l] = a.key[f];
        a.cand[l] = a.cand[f];
        rp_adjust(a, f, 0, l - f, vk, vc);
    }
}

template <class A>
__device__ void rp_insertion(const A &a, int f, int l) {
    for (int i = f + 1; i < l; ++i) {
        const uint32_t vk = a.key[i];
        const int32_t vc = a.cand[i];
        int j = i;
        while (j > f && vk < a.key[j - 1]) {
            a.key[j] = a.key[j - 1];
            a.cand[j] = a.cand[j - 1];
            --j;
        }
        a.key[j] = vk;
        a.cand[j] = vc;
    }
}

// ---- one wavefront partitions [f, l) (median of f+1, middle, l-1 moved to f,
// then the unguarded Hoare scan, done from the stopper lists); returns the cut
template <class A>
__device__ int rp_partition(const A &a, uint16_t *TL, uint16_t *TR, int f, int l) {
    const int lane = lane_id();
    const int n = l - f;
    const int ia = f + 1, ib = f + n / 2, ic = l - 1;
    const uint32_t ka = a.key[ia], kb = a.key[ib], kc = a.key[ic];
    int x;
    if (ka < kb) {
        if (kb < kc) x = ib;
        else if (ka < kc) x = ic;
        else x = ia;
    } else if (ka < kc) x = ia;
    else if (kb < kc) x = ic;
    else x = ib;
    const uint32_t pv = a.key[x];
    rp_sync();
    if (lane == 0) rp_swap(a, f, x);
    rp_sync();
    int numL = 0, numR = 0;
    for (int base = f; base < l; base += SSA_WAVE) {
        const int i = base + lane;
        const bool in = i < l;
        const uint32_t kv = in ? a.key[i] : 0u;
        const bool isL = in && i > f && kv >= pv;
        const bool isR = in && kv <= pv;
        const uint64_t bL = wave_ballot(isL), bR = wave_ballot(isR);
        if (isL) TL[f + numL + lanes_below(bL)] = (uint16_t)i;
        if (isR) TR[f + numR + lanes_below(bR)] = (uint16_t)i;
        numL += __popcll(bL);
        numR += __popcll(bR);
    }
    rp_sync();
    const int sw = hoare_swap_count(TL, TR, f, numL, numR);
    for (int k0 = 0; k0 < sw; k0 += SSA_WAVE) {
        const int k = k0 + lane;
        if (k < sw) rp_swap(a, TL[f + k], TR[f + numR - 1 - k]);
    }
    int cut = 0x7fffffff;
    if (sw < numL) cut = TL[f + sw];
    if (sw > 0) { const int r = TR[f + numR - sw]; cut = r < cut ? r : cut; }
    rp_sync();
    return cut;
}

__device__ __forceinline__ int rp_log2(int n) { return 31 - __clz(n); }

// std::nth_element(f, nth, l)
template <class A>
__device__ void rp_nth_element(const A &a, uint16_t *TL, uint16_t *TR, int f, int nth, int l) {
    if (f == l || nth == l) return;
    int depth = 2 * rp_log2(l - f);
    while (l - f > 3) {
        if (depth == 0) {
            if (lane_id() == 0) {
                rp_heap_select(a, f, nth + 1, l);
                rp_swap(a, f, nth);
            }
            rp_sync();
            return;
        }
        --depth;
        const int cut = rp_partition(a, TL, TR, f, l);
        if (cut <= nth) f = cut; else l = cut;
    }
    if (lane_id() == 0) rp_insertion(a, f, l);
    rp_sync();
}

// std::sort(f, l): introsort loop over an explicit stack, then the final
// insertion sort, which stops at every partition cut, so it runs per leaf
template <class A>
__device__ void rp_sort(const A &a, uint16_t *TL, uint16_t *TR, uint32_t *lbits,
                        int32_t *stk, int f, int l) {
    const int lane = lane_id();
    if (l - f < 2) return;
    for (int w = lane; w < (l + 31) / 32 + 1; w += SSA_WAVE) lbits[w] = 0u;
    rp_sync();
    if (lane == 0) atomicOr(&lbits[f >> 5], 1u << (f & 31));
    int top = 0;
    if (l - f > 16) {
        if (lane == 0) { stk[0] = f; stk[RP_STACK] = l; stk[2 * RP_STACK] = 2 * rp_log2(l - f); }
        top = 1;
    }
    rp_sync();
    while (top > 0) {
        --top;
        const int sf = stk[top], sl = stk[RP_STACK + top], sd = stk[2 * RP_STACK + top];
        rp_sync();
        if (sd == 0) {
            if (lane == 0) {
                rp_heap_select(a, sf, sl, sl);
                rp_heap_sort(a, sf, sl);
            }
            rp_sync();
            continue;
        }
        const int cut = rp_partition(a, TL, TR, sf, sl);
        if (lane == 0) {
            atomicOr(&lbits[cut >> 5], 1u << (cut & 31));
            int t = top;
            if (sl - cut > 16) { stk[t] = cut; stk[RP_STACK + t] = sl; stk[2 * RP_STACK + t] = sd - 1; ++t; }
            if (cut - sf > 16) { stk[t] = sf; stk[RP_STACK + t] = cut; stk[2 * RP_STACK + t] = sd - 1; ++t; }
        }
        top += (sl - cut > 16) + (cut - sf > 16);
        rp_sync();
    }
    // leaf starts in order, then one leaf per lane
    int nl = 0;
    for (int base = f; base < l; base += SSA_WAVE) {
        const int i = base + lane;
        const bool st = i < l && ((lbits[i >> 5] >> (i & 31)) & 1u);
        const uint64_t m = wave_ballot(st);
        if (st) TL[nl + lanes_below(m)] = (uint16_t)i;
        nl += __popcll(m);
    }
    rp_sync();
    for (int i = lane; i < nl; i += SSA_WAVE) {
        const int s0 = TL[i];
        const int e = i + 1 < nl ? (int)TL[i + 1] : l;
        // a leaf above 16 entries was heap-sorted (the insertion sort leaves it)
        rp_insertion(a, s0, e);
    }
    rp_sync();
}

// GLB: the per-wave arrays live in a device buffer (`gscr`, rp_lds_words(W)
// words per resident wave) instead of LDS, for rows whose kk + chunk slots do
// not fit; the same code runs on either (all accesses of a wave's arrays come
// from that wave, whose stores its own later loads see after rp_sync).
// Rows are taken only when more than `skip_max` are tied (fewer go to the
// workgroup replay; skip_max < 0: always).  Six waves per SIMD (80 VGPRs):
// with many rows the launch runs in rounds of resident rows.
// CT: the key ids' type, uint32_t exactly when rp_wide_ids(p.words)
template <typename T, bool LSH_MODE, bool GLB, typename CT>
__global__ void __launch_bounds__(RP_WAVES * SSA_WAVE) __attribute__((amdgpu_waves_per_eu(6)))
topk_replay_kernel(SelP p, int chunk, int W, uint32_t *gscr, int skip_max) {
    extern __shared__ uint32_t rp_smem[];
    const int wid = threadIdx.x / SSA_WAVE;
    const int lane = lane_id();
    // rp_cand_words and rp_lds_words, given that CT is 32-bit exactly when
    // rp_wide_ids(p.words)
    const int cw = sizeof(CT) == 4 ? W : (W + 1) / 2;
    const int64_t wave_words = (2 * W + cw + (W + 31) / 32 + 1 + 3 * RP_STACK + p.words + 1) & ~1;
    uint32_t *base = GLB ? gscr + ((int64_t)blockIdx.x * RP_WAVES + wid) * wave_words
                         : rp_smem + (int64_t)wid * wave_words;
    RpArr<CT> A;
    A.key = base;
    A.cand = (CT *)(base + W);
    uint16_t *TL = (uint16_t *)(base + W + cw);
    uint16_t *TR = TL + W;
    uint32_t *lbits = base + 2 * W + cw;
    int32_t *stk = (int32_t *)(lbits + (W + 31) / 32 + 1);
    uint32_t *bm = (uint32_t *)(stk + 3 * RP_STACK);

    const int total = (int)gridDim.x * RP_WAVES;
    const int cnt = *p.tie_count;
    if (cnt <= skip_max) return;
    const int kk = p.kk;
    for (int it = (int)blockIdx.x * RP_WAVES + wid; it < cnt; it += total) {
        // bh * N + n, over all query heads
        const int64_t row = SSA_IDX(p.tie_list[SSA_IDX(it, p.rows_all, 6)], p.rows_all, 6);
        const int n = (int)(row % p.N);
        const int bh = (int)(row / p.N);
        const int b = bh / p.Hq, h = bh % p.Hq, g = h / p.rep;
        const int bk = b * p.Hkv + g;
        const T *qr = (const T *)p.q + b * p.qsb + h * p.qsh + (int64_t)n * p.qsn;
        const T *kb = (const T *)p.k + b * p.ksb + g * p.ksh;
        // the scores the candidate lists do not carry, with the rescore's
        // arithmetic (as the aux kernel computes them): the query's own key,
        // and glob ++ 0 for an empty bucket (lane j: entry j)
        const uint32_t kq = exact_keys<T>(p, qr, kb, n, p.causal && lane == 0);
        const uint32_t kself = (uint32_t)__builtin_amdgcn_readfirstlane((int)kq);
        for (int w = lane; w < p.words; w += SSA_WAVE) bm[w] = 0u;
        for (int t = lane; t < kk; t += SSA_WAVE) { A.key[t] = RP_NEGINF; A.cand[t] = 0; }
        const uint16_t *qids = p.qid + row * p.R * p.NS;
        rp_sync();

        for (int64_t s0 = 0; s0 < p.Call; s0 += chunk) {
            const int64_t s1 = s0 + chunk < p.Call ? s0 + chunk : p.Call;
            // rebuild the stream slots [s0, s1) in groups that stay inside one list
            for (int64_t j0 = s0; j0 < s1;) {
                const int list = (int)(j0 / p.C);
                const int c0 = (int)(j0 - (int64_t)list * p.C);
                int nl = p.C - c0;
                nl = nl < SSA_WAVE ? nl : SSA_WAVE;
                nl = (int64_t)nl < s1 - j0 ? nl : (int)(s1 - j0);
                const int u = qids[list];
                const int64_t prow = (int64_t)bk * p.R + list / p.NS;
                const int st = p.bstart[prow * p.NB + SSA_IDX(u, p.NB, 7)];
                const int sz = p.bsize[prow * p.NB + SSA_IDX(u, p.NB, 7)];
                const int c = c0 + lane;
                const bool in = lane < nl;
                int v = 0;
                bool keep = false;
                uint32_t sk = 0u;
                if (sz > 0) {
                    const bool real = in && c < min(sz, p.C);
                    const int raw =
                        in ? p.perm[prow * p.M + SSA_IDX(real ? st + c : p.M - 1, p.M, 8)] : 0;
                    v = (p.causal && raw > n) ? n : raw;
                    const uint32_t bit = 1u << (v & 31);
                    const uint32_t old = atomicOr(&bm[v >> 5], real ? bit : 0u);
                    const bool fill = in && !real;
                    if (wave_ballot(fill)) atomicOr(&bm[v >> 5], fill ? bit : 0u);
                    keep = real && !(old & bit);
                    if (p.causal) {
                        // several slots of this group became the query itself:
                        // the earliest one is the first occurrence
                        const uint64_t nm = wave_ballot(real && v == n);
                        if (__popcll(nm) > 1) {
                            const bool clr = real && v == n && !(old & bit);
                            const bool seen = wave_ballot(clr) == 0ull;
                            if (real && v == n)
                                keep = !seen && lane == (int)(__ffsll((long long)nm) - 1);
                        }
                    }
                    // exact keys with the rescore's arithmetic (the table holds
                    // only their prefixes); the query itself scores as in aux
                    const bool xk = keep && !(p.causal && v == n);
                    const uint32_t ex = exact_keys<T>(p, qr, kb, v, xk);
                    if (keep) sk = xk ? ex : kself;
                } else {
                    // empty bucket: glob ++ 0, all valid; duplicates resolved in slot order
                    v = (c < p.G) ? (int)p.glob[c < p.G ? c : 0] : 0;
                    bool pending = in;
                    uint64_t pm = wave_ballot(pending);
                    while (pm) {
                        const int leader = (int)(__ffsll((long long)pm) - 1);
                        const int vl = __shfl(v, leader, SSA_WAVE);
                        const bool same = pending && v == vl;
                        if (lane == leader) {
                            const uint32_t bit = 1u << (v & 31);
                            const uint32_t old = atomicOr(&bm[v >> 5], bit);
                            keep = !(old & bit);
                        }
                        pending = pending && !same;
                        pm = wave_ballot(pending);
                    }
                    // the glob entries' keys with the exact-key arithmetic
                    // (the query's own key included), as the aux rows hold them
                    const uint32_t ex = exact_keys<T>(p, qr, kb, v, keep);
                    if (keep) sk = ex;
                }
                if (in) {
                    const int at = kk + (int)(j0 - s0) + lane;
                    A.key[at] = keep ? ~sk : RP_NEGINF;
                    A.cand[at] = (CT)v;
                }
                rp_sync();
                j0 += nl;
            }
            // torch.topk(best ++ chunk, kk): partial_sort when 64*kk <= width,
            // else nth_element(kk-1) + sort(kk-1)
            const int w = kk + (int)(s1 - s0);
            if ((int64_t)kk * 64 <= w) {
                if (lane == 0) {
                    rp_heap_select(A, 0, kk, w);
                    rp_heap_sort(A, 0, kk);
                }
                rp_sync();
            } else {
                rp_nth_element(A, TL, TR, 0, kk - 1, w);
                rp_sort(A, TL, TR, lbits, stk, 0, kk - 1);
            }
        }
        // A[0, kk) is the reference's best list: finite entries first
        int fcount = 0;
        for (int t0 = 0; t0 < kk; t0 += SSA_WAVE) {
            const int t = t0 + lane;
            fcount += __popcll(wave_ballot(t < kk && A.key[t] != RP_NEGINF));
        }
        if (LSH_MODE) {
            int64_t *orow = p.out_idx + row * kk;
            for (int t = lane; t < kk; t += SSA_WAVE)
                orow[t] = t < fcount ? (int64_t)A.cand[t] : (t < p.G ? p.glob[t] : 0);
        } else {
            for (int w = lane; w < p.words; w += SSA_WAVE) bm[w] = 0u;
            rp_sync();
            for (int t = lane; t < fcount; t += SSA_WAVE) bm_set(bm, A.cand[t]);
            rp_sync();
            full_merge_emit(bm, p, n, row, fcount, (int32_t *)A.key, W);
        }
        rp_sync();
    }
}

// ---- tie replay, one workgroup per row
// The running top-k of the reference (sparse_attention.py:904-922) holds after
// chunk s the kk smallest rank keys of chunks 0..s in sorted order (nth_element
// + sort of the first kk - 1, or partial_sort): the key array of every state
// S_s follows from the stream alone.  Only which candidate sits in which of
// several equal keys depends on the comparisons and swaps made, and those look
// at keys only.  So chunk s replays by itself, on S_{s-1}'s keys ++ the chunk's
// keys with input positions as payload, into a map pi_s from output slot to
// input position; where the first kk + 1 merged keys of a chunk hold no two
// equal finite keys, the sorted merge gives the same map.  For a graph (a set)
// only the ties at the final kk-th key matter: other equal keys are all kept
// or all dropped, so only the chunks where that key is tied are replayed.  A
// row runs as
//   1. the stream: each slot's key id and validity, its first occurrence (the
//      smallest slot holding the id, by atomicMin: the reference's stable sort
//      by id, :884-890), then per chunk the exact keys and the chunk's finite
//      keys sorted -- all waves;
//   2. the states' keys by merging each state with its chunk's sorted head,
//      noting the tied keys per chunk -- wave 0;
//   3. the chunks to replay, replayed as the reference runs them, one wave each;
//   4. every finite output slot followed back through the maps to its stream
//      slot, then the emit -- wave 0.
// For many tied rows the per-wave replay (one row per wave, more rows in
// flight) is faster; a launch takes its rows only when at most `cap` are tied.
constexpr int RPW_WAVES = 16;
constexpr int RPW_THREADS = RPW_WAVES * SSA_WAVE;
constexpr int RPW_MAX_BLOCKS = 1024;
constexpr int RPW_TV = 4;            // tied key values noted per chunk
constexpr uint32_t RPW_VALID = 1u << 31, RPW_EMPTY = 1u << 30, RPW_OWNER = 1u << 29,
                   RPW_VMASK = RPW_OWNER - 1u;

// LDS of one replaying wave: keys (W), 16-bit positions, TL/TR, leaf bits,
// stack (the first 2 W words also hold a chunk's keys and tags while sorting)
__host__ __device__ inline int rpw_slot_words(int W) {
    return (2 * W + (W + 1) / 2 + (W + 31) / 32 + 1 + 3 * RP_STACK + 1) & ~1;
}
// LDS shared by the workgroup: bitmap, glob scores, list table, state keys,
// merge output, per chunk (head length, tie count, tied keys, input state,
// marked list), misc, keep bits, the maps (u16)
__host__ __device__ inline int rpw_shared_words(int words, int nls, int kk, int nch, int64_t Call) {
    return (int)((words + 2 * nls + kk + 2 * (kk + 1) + (int64_t)nch * (4 + RPW_TV) + 8 +
                  (Call + 31) / 32 + ((int64_t)nch * kk + 1) / 2 + 1) & ~1);
}
// workspace words of one block: stream keys and ids, first occurrences, the
// tied chunks' input state keys, each chunk's sorted head (kk + 1 keys, tags)
__host__ __device__ inline int64_t rpw_scratch_words(int64_t Call, int M, int kk, int nch) {
    return (2 * Call + M + (int64_t)nch * kk + 2 * (int64_t)nch * (kk + 1) + 63) / 64 * 64;
}

// a wave's LDS stores seen by its later loads, without waiting for its
// global loads (rp_sync waits for every counter)
__device__ __forceinline__ void rpw_lsync() {
    __builtin_amdgcn_s_waitcnt(0xC07F);    // lgkmcnt(0)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// one wave sorts k[0, e) ascending, t alongside (bitonic with a mirrored first
// step, which sorts any e when pairs reaching past e are skipped).  The pairs
// of a step are disjoint: four rows of 64 are read before any is written.
__device__ void rpw_sort(uint32_t *k, uint32_t *t, int e) {
    const int lane = lane_id();
    for (int size = 2; size < 2 * e; size <<= 1) {
        for (int j = size >> 1; j > 0; j >>= 1) {
            for (int i0 = 0; i0 < e; i0 += 4 * SSA_WAVE) {
                int ii[4], pp[4];
                bool on[4];
                uint32_t a[4], b[4], ta[4], tb[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    ii[u] = i0 + u * SSA_WAVE + lane;
                    pp[u] = j == (size >> 1) ? (ii[u] ^ (size - 1)) : (ii[u] ^ j);
                    on[u] = ii[u] < e && pp[u] > ii[u] && pp[u] < e;
                    a[u] = on[u] ? k[ii[u]] : 0u;
                    b[u] = on[u] ? k[pp[u]] : 0u;
                    ta[u] = on[u] ? t[ii[u]] : 0u;
                    tb[u] = on[u] ? t[pp[u]] : 0u;
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (on[u] && b[u] < a[u]) {
                        k[ii[u]] = b[u];
                        k[pp[u]] = a[u];
                        t[ii[u]] = tb[u];
                        t[pp[u]] = ta[u];
                    }
                }
            }
            rp_sync();
        }
    }
}

// entries of sorted k[0, n) below x (or at most x)
__device__ __forceinline__ int rpw_rank(const uint32_t *k, int n, uint32_t x, bool incl) {
    int lo = 0, hi = n;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        const uint32_t y = k[mid];
        if (incl ? y <= x : y < x) lo = mid + 1;
        else hi = mid;
    }
    return lo;
}

template <typename T, bool LSH_MODE>
__global__ void __launch_bounds__(RPW_THREADS)
topk_replay_wg_kernel(SelP p, int chunk, int W, int nsim, uint32_t *gscr, int64_t scr_words,
                      int cap) {
    extern __shared__ uint32_t rp_smem[];
    const int wid = threadIdx.x / SSA_WAVE;
    const int lane = lane_id();
    const int cnt = *p.tie_count;
    if (cnt > cap || (int)blockIdx.x >= cnt) return;
    const int kk = p.kk;
    const int nls = p.R * p.NS;
    const int nch = (int)((p.Call + chunk - 1) / chunk);
    const int sw = rpw_slot_words(W);
    uint32_t *slot = rp_smem + (int64_t)(wid < nsim ? wid : 0) * sw;
    uint32_t *sh = rp_smem + (int64_t)nsim * sw;
    uint32_t *bm = sh;
    int32_t *lst = (int32_t *)(bm + p.words);
    int32_t *lsz = lst + nls;
    uint32_t *Sk = (uint32_t *)(lsz + nls);
    uint32_t *Sn = Sk + kk;
    uint32_t *Tn = Sn + kk + 1;
    int32_t *chd = (int32_t *)(Tn + kk + 1);    // per chunk: sorted head length
    int32_t *ctc = chd + nch;                   // tied key values
    int32_t *csi = ctc + nch;                   // its input state's index in SK
    int32_t *mk = csi + nch;                    // the chunks to replay
    uint32_t *ctv = (uint32_t *)(mk + nch);     // RPW_TV tied keys per chunk
    int32_t *misc = (int32_t *)(ctv + (int64_t)nch * RPW_TV);
    uint32_t *kbits = (uint32_t *)(misc + 8);   // kept slots
    uint16_t *PI = (uint16_t *)(kbits + (p.Call + 31) / 32);

    uint32_t *g = gscr + (int64_t)blockIdx.x * scr_words;
    uint32_t *skey = g;
    uint32_t *svs = g + p.Call;
    uint32_t *first = svs + p.Call;
    uint32_t *SK = first + p.M;
    uint32_t *SS = SK + (int64_t)nch * kk;
    uint32_t *ST = SS + (int64_t)nch * (kk + 1);
    for (int i = threadIdx.x; i < p.M; i += RPW_THREADS) first[i] = 0xffffffffu;

    for (int it = (int)blockIdx.x; it < cnt; it += (int)gridDim.x) {
        // bh * N + n, over all query heads
        const int64_t row = SSA_IDX(p.tie_list[SSA_IDX(it, p.rows_all, 6)], p.rows_all, 6);
        const int n = (int)(row % p.N);
        const int bh = (int)(row / p.N);
        const int b = bh / p.Hq, h = bh % p.Hq, gq = h / p.rep;
        const int bk = b * p.Hkv + gq;
        const T *qr = (const T *)p.q + b * p.qsb + h * p.qsh + (int64_t)n * p.qsn;
        const T *kb = (const T *)p.k + b * p.ksb + gq * p.ksh;
        const uint16_t *qids = p.qid + row * p.R * p.NS;
        for (int l = threadIdx.x; l < nls; l += RPW_THREADS) {
            const int u = qids[l];
            const int64_t prow = (int64_t)bk * p.R + l / p.NS;
            lst[l] = p.bstart[prow * p.NB + SSA_IDX(u, p.NB, 7)];
            lsz[l] = p.bsize[prow * p.NB + SSA_IDX(u, p.NB, 7)];
        }
        for (int64_t w = threadIdx.x; w < (p.Call + 31) / 32; w += RPW_THREADS) kbits[w] = 0u;
        if (wid == 0) {
            // the scores the stream does not carry, with the rescore's arithmetic
            // (as the aux kernel computes them): the query's own key, and
            // glob ++ 0 for an empty bucket (lane j: entry j)
            const uint32_t kq = exact_keys<T>(p, qr, kb, n, p.causal && lane == 0);
            if (lane == 0) misc[0] = (int)kq;
        }
        __syncthreads();

        // 1a. key ids and validity of every slot; first occurrences
        for (int64_t j0 = threadIdx.x; j0 < p.Call; j0 += 8 * RPW_THREADS) {
            int v[8];
            uint32_t fl[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int64_t j = j0 + (int64_t)u * RPW_THREADS;
                v[u] = 0;
                fl[u] = 0u;
                if (j < p.Call) {
                    const int list = (int)(j / p.C);
                    const int c = (int)(j - (int64_t)list * p.C);
                    const int sz = lsz[list];
                    if (sz > 0) {
                        const bool real = c < min(sz, p.C);
                        const int64_t prow = (int64_t)bk * p.R + list / p.NS;
                        const int raw =
                            p.perm[prow * p.M + SSA_IDX(real ? lst[list] + c : p.M - 1, p.M, 8)];
                        v[u] = (p.causal && raw > n) ? n : raw;
                        fl[u] = real ? RPW_VALID : 0u;
                    } else {
                        // empty bucket: glob ++ 0, all valid
                        v[u] = c < p.G ? (int)p.glob[c < p.G ? c : 0] : 0;
                        fl[u] = RPW_VALID | RPW_EMPTY;
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                // a wave's slots are consecutive: a run of one id needs only its
                // first slot's atomic, and so do the slots clamped to the query
                const int64_t j = j0 + (int64_t)u * RPW_THREADS;
                const bool in = j < p.Call;
                const int vu = in ? v[u] : -1;
                const int vprev = __shfl_up(vu, 1, SSA_WAVE);
                const uint64_t nm = wave_ballot(in && vu == n);
                bool need = in && !(lane > 0 && vprev == vu);
                if (in && vu == n) need = lane == (int)(__ffsll((long long)nm) - 1);
                if (need) atomicMin(&first[SSA_IDX(vu, p.M, 10)], (uint32_t)j);
                if (in) svs[j] = (uint32_t)vu | fl[u];
            }
        }
        __syncthreads();

        // 1b. the first occurrences own their ids; valid owners are kept
        for (int64_t j0 = threadIdx.x; j0 < p.Call; j0 += 8 * RPW_THREADS) {
            uint32_t vs[8], fv[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int64_t j = j0 + (int64_t)u * RPW_THREADS;
                vs[u] = j < p.Call ? svs[j] : 0u;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int64_t j = j0 + (int64_t)u * RPW_THREADS;
                fv[u] = j < p.Call ? __hip_atomic_load(&first[SSA_IDX(vs[u] & RPW_VMASK, p.M, 10)],
                                                       __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT)
                                   : 0xffffffffu;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int64_t j = j0 + (int64_t)u * RPW_THREADS;
                if (j < p.Call && fv[u] == (uint32_t)j) {
                    svs[j] = vs[u] | RPW_OWNER;
                    if (vs[u] & RPW_VALID) atomicOr(&kbits[j >> 5], 1u << (j & 31));
                }
            }
        }
        __syncthreads();

        // 1c. per chunk: the first-occurrence table back to empty, the kept
        // slots' exact keys (the query itself scores as in aux), the finite
        // keys sorted
        const uint32_t kself = (uint32_t)misc[0];
        if (wid < nsim) {
            uint32_t *Ek = slot, *Et = slot + W;
            for (int s = wid; s < nch; s += nsim) {
                const int64_t s0 = (int64_t)s * chunk;
                const int c = (int)min((int64_t)chunk, p.Call - s0);
                // the kept slots, compacted: ids into Ek, positions into Et
                int e = 0;
                for (int j0 = 0; j0 < c; j0 += 4 * SSA_WAVE) {
                    uint32_t vs[4];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int jl = j0 + u * SSA_WAVE + lane;
                        vs[u] = jl < c ? svs[s0 + jl] : 0u;
                    }
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int jl = j0 + u * SSA_WAVE + lane;
                        const int64_t j = s0 + jl;
                        const bool in = jl < c;
                        const bool keep = in && ((kbits[j >> 5] >> (j & 31)) & 1u);
                        if (in && (vs[u] & RPW_OWNER))
                            first[SSA_IDX(vs[u] & RPW_VMASK, p.M, 10)] = 0xffffffffu;
                        if (in && !keep) skey[j] = RP_NEGINF;
                        const uint64_t m = wave_ballot(keep);
                        if (keep) {
                            const int at = e + lanes_below(m);
                            Ek[at] = vs[u] & RPW_VMASK;
                            Et[at] = (uint32_t)(kk + jl);
                        }
                        e += __popcll(m);
                    }
                }
                rp_sync();
                for (int g0 = 0; g0 < e; g0 += SSA_WAVE) {
                    const int t = g0 + lane;
                    const bool in = t < e;
                    const int v = in ? (int)Ek[t] : 0;
                    const int64_t j = s0 + (in ? (int)Et[t] - kk : 0);
                    const int list = (int)(j / p.C);
                    const bool empty = lsz[list] == 0;
                    // glob ++ 0 entries (empty buckets) take the exact-key
                    // arithmetic even for the query's own key, as the aux rows do
                    const bool xk = in && (empty || !(p.causal && v == n));
                    const uint32_t ex = exact_keys_wide<T, 4>(p, qr, kb, v, xk);
                    if (in) {
                        const uint32_t key = ~(xk ? ex : kself);
                        Ek[t] = key;
                        skey[j] = key;
                    }
                }
                rp_sync();
                // the sorted head: the first kk + 1 finite keys (-inf sorts last)
                int hl;
                if (e > kk + 1 && e <= 16 * SSA_WAVE) {
                    // the (kk + 1)-th smallest key first (a bitwise search over
                    // the keys in registers), then only the head is sorted; of
                    // several keys equal to it any may complete the head (equal
                    // keys that reach a state are ties, and tied chunks replay)
                    uint32_t kv[16], tv[16];
                    int nf = 0;
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int t = i * SSA_WAVE + lane;
                        kv[i] = t < e ? Ek[t] : 0xffffffffu;
                        tv[i] = t < e ? Et[t] : 0u;
                        nf += __popcll(wave_ballot(t < e && kv[i] != RP_NEGINF));
                    }
                    hl = min(nf, kk + 1);
                    uint32_t tau = 0u;
                    for (int bit = 31; bit >= 0; --bit) {
                        const uint32_t probe = tau | ((1u << bit) - 1u);
                        int c = 0;
#pragma unroll
                        for (int i = 0; i < 16; ++i) c += __popcll(wave_ballot(kv[i] <= probe));
                        if (c < hl) tau |= 1u << bit;
                    }
                    rp_sync();
                    int nlt = 0;
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const bool lt = kv[i] < tau;
                        const uint64_t m = wave_ballot(lt);
                        if (lt) {
                            Ek[nlt + lanes_below(m)] = kv[i];
                            Et[nlt + lanes_below(m)] = tv[i];
                        }
                        nlt += __popcll(m);
                    }
                    int neq = nlt;
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const bool eq = kv[i] == tau;
                        const uint64_t m = wave_ballot(eq);
                        const int at = neq + lanes_below(m);
                        if (eq && at < hl) {
                            Ek[at] = kv[i];
                            Et[at] = tv[i];
                        }
                        neq += __popcll(m);
                    }
                    rp_sync();
                    rpw_sort(Ek, Et, hl);
                } else {
                    rpw_sort(Ek, Et, e);
                    hl = min(rpw_rank(Ek, e, RP_NEGINF, false), kk + 1);
                }
                for (int t = lane; t < hl; t += SSA_WAVE) {
                    SS[(int64_t)s * (kk + 1) + t] = Ek[t];
                    ST[(int64_t)s * (kk + 1) + t] = Et[t];
                }
                if (lane == 0) chd[s] = hl;
                rp_sync();
            }
        }
        __syncthreads();

        if (wid == 0) {
            // 2. the states' keys: S_s = the kk smallest of S_{s-1} ++ chunk s
            uint32_t *Ek = slot, *Et = slot + W;
            for (int t = lane; t < kk; t += SSA_WAVE) Sk[t] = RP_NEGINF;
            int a = 0;       // finite keys in Sk
            int nst = 0;     // input states kept
            // the next chunk's head, its first 4 * 64 entries loaded a step ahead
            uint32_t hk[4], ht[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int t = u * SSA_WAVE + lane;
                hk[u] = t < chd[0] ? SS[t] : 0u;
                ht[u] = t < chd[0] ? ST[t] : 0u;
            }
            rpw_lsync();
            for (int s = 0; s < nch; ++s) {
                const int hl = chd[s];
                const uint32_t thr = a == kk ? Sk[kk - 1] : RP_NEGINF;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int t = u * SSA_WAVE + lane;
                    if (t < hl) { Ek[t] = hk[u]; Et[t] = ht[u]; }
                }
                for (int t = 4 * SSA_WAVE + lane; t < hl; t += SSA_WAVE) {
                    Ek[t] = SS[(int64_t)s * (kk + 1) + t];
                    Et[t] = ST[(int64_t)s * (kk + 1) + t];
                }
                if (s + 1 < nch) {
                    const int hn = chd[s + 1];
#pragma unroll
                    for (int u = 0; u < 4; ++u) {
                        const int t = u * SSA_WAVE + lane;
                        hk[u] = t < hn ? SS[(int64_t)(s + 1) * (kk + 1) + t] : 0u;
                        ht[u] = t < hn ? ST[(int64_t)(s + 1) * (kk + 1) + t] : 0u;
                    }
                }
                rpw_lsync();
                // the head's keys that enter (at most the state's worst): counted
                // with ballots, the head being sorted
                int e = 0;
                for (int t0 = 0; t0 < hl; t0 += SSA_WAVE) {
                    const int t = t0 + lane;
                    e += __popcll(wave_ballot(t < hl && Ek[t] <= thr));
                }
                // merge: state entries before chunk entries of the same key; the
                // two rank searches of a lane run side by side
                const int nout = min(kk + 1, a + e);
                const int em = min(e, nout);
                for (int t = lane; t < a || t < em; t += SSA_WAVE) {
                    const bool ds = t < a, de = t < em;
                    const uint32_t xs = ds ? Sk[t] : 0u, xe = de ? Ek[t] : 0u;
                    const int rs = t + (ds ? rpw_rank(Ek, e, xs, false) : 0);
                    const int re = t + (de ? rpw_rank(Sk, a, xe, true) : 0);
                    if (ds && rs < nout) { Sn[rs] = xs; Tn[rs] = (uint32_t)t; }
                    if (de && re < nout) { Sn[re] = xe; Tn[re] = Et[t]; }
                }
                rpw_lsync();
                // equal finite keys among the first kk + 1: note each tied value
                int ntv = 0;
                for (int t0 = 0; t0 < kk && t0 + 1 < nout; t0 += SSA_WAVE) {
                    const int t = t0 + lane;
                    const bool run = t < kk && t + 1 < nout && Sn[t] == Sn[t + 1] &&
                                     (t == 0 || Sn[t - 1] != Sn[t]);
                    const uint64_t m = wave_ballot(run);
                    if (run) {
                        const int at = ntv + lanes_below(m);
                        if (at < RPW_TV) ctv[(int64_t)s * RPW_TV + at] = Sn[t];
                    }
                    ntv += __popcll(m);
                }
                if (ntv > 0) {
                    for (int t = lane; t < kk; t += SSA_WAVE) SK[(int64_t)nst * kk + t] = Sk[t];
                    if (lane == 0) csi[s] = nst;
                    ++nst;
                }
                if (lane == 0) ctc[s] = ntv;
                const int an = min(kk, a + e);
                for (int t = lane; t < kk; t += SSA_WAVE) {
                    Sk[t] = t < an ? Sn[t] : RP_NEGINF;
                    PI[(int64_t)s * kk + t] = (uint16_t)(t < an ? Tn[t] : 0u);
                }
                a = an;
                rpw_lsync();
            }
            // the chunks to replay: every tie for an ordered list; for a set,
            // the chunks where the final kk-th key is tied (none when fewer
            // than kk keys are finite: all of them are kept)
            const uint32_t vstar = Sk[kk - 1];
            int nmark = 0;
            for (int s0 = 0; s0 < nch; s0 += SSA_WAVE) {
                const int s = s0 + lane;
                bool mark = false;
                if (s < nch && ctc[s] > 0) {
                    if (LSH_MODE || ctc[s] > RPW_TV) {
                        mark = LSH_MODE || a == kk;
                    } else if (a == kk) {
                        for (int u = 0; u < ctc[s]; ++u) mark |= ctv[(int64_t)s * RPW_TV + u] == vstar;
                    }
                }
                const uint64_t m = wave_ballot(mark);
                if (mark) mk[nmark + lanes_below(m)] = s;
                nmark += __popcll(m);
            }
            if (lane == 0) { misc[1] = nmark; misc[2] = a; }
        }
        __syncthreads();

        // 3. the chunks to replay, replayed as the reference runs them
        const int nmark = misc[1];
        if (wid < nsim) {
            RpArr<uint16_t> A;
            A.key = slot;
            A.cand = (uint16_t *)(slot + W);
            uint16_t *TL = (uint16_t *)(slot + W + (W + 1) / 2);
            uint16_t *TR = TL + W;
            uint32_t *lbits = slot + 2 * W + (W + 1) / 2;
            int32_t *stk = (int32_t *)(lbits + (W + 31) / 32 + 1);
            for (int f = wid; f < nmark; f += nsim) {
                const int s = mk[f];
                const int64_t s0 = (int64_t)s * chunk;
                const int c = (int)min((int64_t)chunk, p.Call - s0);
                const int si = csi[s];
                for (int t = lane; t < kk; t += SSA_WAVE) {
                    A.key[t] = SK[(int64_t)si * kk + t];
                    A.cand[t] = (uint16_t)t;
                }
                for (int t = lane; t < c; t += SSA_WAVE) {
                    A.key[kk + t] = skey[s0 + t];
                    A.cand[kk + t] = (uint16_t)(kk + t);
                }
                rp_sync();
                // torch.topk(best ++ chunk, kk): partial_sort when 64*kk <= width,
                // else nth_element(kk-1) + sort(kk-1)
                const int w = kk + c;
                if ((int64_t)kk * 64 <= w) {
                    if (lane == 0) {
                        rp_heap_select(A, 0, kk, w);
                        rp_heap_sort(A, 0, kk);
                    }
                    rp_sync();
                } else {
                    rp_nth_element(A, TL, TR, 0, kk - 1, w);
                    rp_sort(A, TL, TR, lbits, stk, 0, kk - 1);
                }
                for (int t = lane; t < kk; t += SSA_WAVE) PI[(int64_t)s * kk + t] = (uint16_t)A.cand[t];
                rp_sync();
            }
        }
        __syncthreads();

        if (wid == 0) {
            // 4. each finite output slot back to its stream slot
            const int fcount = misc[2];
            int32_t *cand = (int32_t *)(slot + W);
            for (int t = lane; t < fcount; t += SSA_WAVE) {
                int pos = t;
                int64_t js = -1;
                for (int s = nch - 1; s >= 0; --s) {
                    const int tg = PI[(int64_t)s * kk + pos];
                    if (tg >= kk) { js = (int64_t)s * chunk + (tg - kk); break; }
                    pos = tg;
                }
                cand[t] = js >= 0 ? (int32_t)(svs[SSA_IDX(js, p.Call, 11)] & RPW_VMASK) : 0;
            }
            rp_sync();
            if (LSH_MODE) {
                int64_t *orow = p.out_idx + row * kk;
                for (int t = lane; t < kk; t += SSA_WAVE)
                    orow[t] = t < fcount ? (int64_t)cand[t] : (t < p.G ? p.glob[t] : 0);
            } else {
                for (int w = lane; w < p.words; w += SSA_WAVE) bm[w] = 0u;
                rp_sync();
                for (int t = lane; t < fcount; t += SSA_WAVE) bm_set(bm, cand[t]);
                rp_sync();
                full_merge_emit(bm, p, n, row, fcount, (int32_t *)slot, W);
            }
        }
        __syncthreads();
    }
}

// ------------------------------------------------------------------ host side
// Instance of the matrix-core rescore / aux kernels for head dim d (8..128,
// whole 8-element pieces): k steps of 32, so ceil(d / 32) steps as the select's
// exact keys take them
int mfma_instance(int d) { return d <= 8 ? 8 : d <= 16 ? 16 : (d + 31) / 32 * 32; }

// Whether RP_WAVES replayed rows of W = kk + chunk slots fit one workgroup's LDS.
bool replay_fits_lds(int W, int words) {
    return (int64_t)RP_WAVES * rp_lds_words(W, words) * 4 <= SSA_LDS_BYTES;
}

// Blocks of the replay whose per-wave arrays live in the workspace: as many as
// keep that region within `budget` bytes (at least one, at most 256; each
// block loops over its rows).
int64_t replay_glb_blocks(int W, int words, int64_t budget) {
    const int64_t per_block = (int64_t)RP_WAVES * rp_lds_words(W, words) * 4;
    return std::max<int64_t>(1, std::min<int64_t>(256, budget / per_block));
}

struct Layout {
    int64_t kid, qid, perm, bstart, bsize, sorttmp, sid, rnk, smin, inv, cut, srix, cnt, off,
        cur,
        qlist, tiles, ntiles, tcnt, kbase, S,
        tie_list, tie_count, aux, psplit, knorm, kpart, rpscr, rpw, ctab, total;
};

int64_t align256(int64_t x) { return (x + 255) / 256 * 256; }

Layout plan(const Dims &D) {
    Layout L{};
    int64_t o = 0;
    auto take = [&](int64_t bytes) { int64_t at = o; o += align256(bytes); return at; };
    const int64_t nbh = D.nbh_chunk;
    const int64_t ninst = nbh * D.R * D.NS;
    L.kid = take(D.BK * D.R * D.M * 2);
    L.qid = take(D.BH * D.N * D.R * D.NS * 2);
    L.perm = take(D.BK * D.R * D.M * 4);
    L.bstart = take(D.BK * D.R * D.NB * 4);
    L.bsize = take(D.BK * D.R * D.NB * 4);
    L.sorttmp = take(ssa_sort_tmp_bytes((int)(D.BK * D.R), D.M));
    L.sid = take(D.BK * D.R * D.M * 4);
    L.rnk = take(D.BK * D.R * D.M * 4);
    L.smin = take(D.BK * D.R * D.M * 4);
    L.inv = take(D.BK * D.R * D.M * 4);
    L.cut = take(nbh * D.N * D.nlists * 16);
    L.srix = take(nbh * D.N * D.nlists * 4);
    L.cnt = take(ninst * D.NB * 4);
    L.off = take(ninst * D.NB * 4);
    L.cur = take(ninst * ceil_div(D.N, 256) * D.NB * 4);   // per-block counts / bases
    L.qlist = take(ninst * D.N * 4);
    // one 16-byte slot per block of the rescore grid (a multiple of 8)
    L.tiles = take(8 * ceil_div(ninst * (ceil_div(D.N, TQ) + D.NB), 8) * 16);
    L.ntiles = take(4);
    L.tcnt = take(ninst * 4);
    L.kbase = take((nbh / D.rep + 2) * D.R * D.NS * D.rep * 4);
    L.S = take(nbh * D.N * D.nlists * D.Cs * 2);
    L.tie_list = take(D.BH * D.N * 4);
    L.tie_count = take(4);
    L.aux = take((D.fused ? D.BH : nbh) * D.N * (D.G + 3) * 4);
    L.psplit = take(D.fused ? ssa_plane_split_bytes(D.R * D.P, D.d) : 0);
    L.knorm = take(D.BK * 4);
    L.ctab = take(D.ctab ? D.BK * D.R * D.NB * (int64_t)((D.M + 31) / 32) * 8 : 0);
    L.kpart = take(D.BK * (D.M / 16) * 4);
    {
        // the replay's per-wave arrays, when they do not fit LDS
        const int W = D.kk + D.chunk;
        const int words = sel_bitmap_words(D.M);
        L.rpscr = take(replay_fits_lds(W, words)
                           ? 0
                           : (int64_t)D.rp_glb_blocks * RP_WAVES * rp_lds_words(W, words) * 4);
        L.rpw = take((int64_t)D.rpw_blocks *
                     rpw_scratch_words(D.Call, D.M, D.kk, (int)ceil_div(D.Call, D.chunk)) * 4);
    }
    L.total = o;
    return L;
}

Layout plan(const Dims &D);

// ws_cap > 0: query heads go in chunks small enough that the workspace stays
// within ws_cap bytes (the build without allocation runs in a fixed scratch
// array); SSA_E_WORKSPACE when even one head per chunk needs more.
int make_dims(const ssa_graph_args *a, Dims &D, bool need_q = true, int64_t ws_cap = 0,
              bool fused = false) {
    SSA_CHECK_ARG(a != nullptr, "build_graph: null args");
    SSA_CHECK_ARG(a->mode == SSA_GRAPH_FULL || a->mode == SSA_GRAPH_LSH, "build_graph: bad mode");
    SSA_CHECK_ARG(a->B >= 1 && a->Hq >= 1 && a->Hkv >= 1 && a->N >= 1 && a->M >= 1,
                  "build_graph: bad sizes B=%d Hq=%d Hkv=%d N=%d M=%d", a->B, a->Hq, a->Hkv,
                  a->N, a->M);
    SSA_CHECK_ARG(a->Hq % a->Hkv == 0, "build_graph: Hq %% Hkv != 0");
    SSA_CHECK_ARG(a->P >= 1 && a->P <= 12 && a->P <= a->max_p, "build_graph: P=%d", a->P);
    SSA_CHECK_ARG(a->R >= 1 && a->C >= 1 && a->top_k >= 1 && a->T >= 0, "build_graph: R/C/top_k/T");
    SSA_CHECK_ARG(a->C <= (1 << 24), "build_graph: C=%d above 2^24", a->C);
    SSA_CHECK_ARG(a->G >= 0 && a->G <= a->M, "build_graph: G=%d outside 0..M (%d)", a->G, a->M);
    SSA_CHECK_ARG(a->rand_proj || (a->q_proj && a->k_proj), "build_graph: no hyperplanes");
    SSA_CHECK_ARG((a->q.ptr || !need_q) && a->k.ptr, "build_graph: null q/k");
    SSA_CHECK_ARG(a->q.dtype == a->k.dtype && a->q.dtype >= 0 && a->q.dtype <= 2,
                  "build_graph: q/k dtype");
    SSA_CHECK_ARG(a->G == 0 || a->glob, "build_graph: glob is null");
    if (!ssa_head_dim_ok(a->d, a->q.dtype)) {
        ssa_set_error("build_graph: head dim %d unsupported (4..1024: a power of two or a multiple "
                      "of %d)", a->d, a->q.dtype == SSA_F32 ? 4 : 8);
        return SSA_E_UNSUP;
    }
    // a cut entry packs a list's size (capped at C) and cutoff, both at most
    // min(C, M), with a key id and a bucket start, both below M, into 32 bits
    // each: 16 + 16 bits up to 65,536 keys, else as many bits as min(C, M)
    // needs for the first two
    if (!ssa_sort_supported(a->M)) {
        ssa_set_error("build_graph: key length %d unsupported (1..1048576)", a->M);
        return SSA_E_UNSUP;
    }
    {
        auto width = [](int64_t v) { int b = 0; while (((int64_t)1 << b) <= v) ++b; return b; };
        const int cb = width(std::min<int64_t>(a->C, a->M)), mb = width(a->M - 1);
        D.cbits = cb <= 16 && mb <= 16 ? 16 : cb;
        if (D.cbits + mb > 32) {
            ssa_set_error("build_graph: %d keys with lists of up to %d members exceed the 32-bit "
                          "fields of a list cut (%d + %d bits)", a->M, a->C, cb, mb);
            return SSA_E_UNSUP;
        }
    }
    SSA_CHECK_ARG((int64_t)a->B * a->Hkv * a->R * a->M < ((int64_t)1 << 29),
                  "build_graph: B*Hkv*R*M must stay below 2^29 (bucket permutation bytes)");
    D.fused = fused ? 1 : 0;
    D.B = a->B; D.Hq = a->Hq; D.Hkv = a->Hkv; D.rep = a->Hq / a->Hkv;
    D.N = a->N; D.M = a->M; D.d = a->d; D.R = a->R; D.maxP = a->max_p; D.P = a->P;
    D.Tp = a->T < a->P ? a->T : a->P;
    D.NS = 1 + D.Tp;
    D.NB = 1 << a->P;
    D.C = a->C;
    D.Cs = (int)ceil_div(std::min<int64_t>(a->C, a->M), 64) * 64;
    D.CPL = (int)ceil_div(a->C, SSA_WAVE);
    D.nlists = a->R * D.NS;
    D.G = a->G;
    D.Call = (int64_t)a->R * D.NS * a->C;
    D.kk = (int)(a->top_k < D.Call ? a->top_k : D.Call);
    {
        int64_t ch = 4 * (int64_t)D.kk;
        if (ch < 256) ch = 256;
        if (ch > D.Call) ch = D.Call;
        D.chunk = (int)ch;
    }
    D.BH = (int64_t)a->B * a->Hq;
    D.BK = (int64_t)a->B * a->Hkv;
    const int self = a->is_cross ? 0 : 1;
    D.Kw = a->is_cross ? 0 : 2 * a->window + 1;
    const int64_t Kall = (int64_t)D.Kw + a->G + D.kk;
    if (a->mode == SSA_GRAPH_FULL) {
        SSA_CHECK_ARG(a->total_k >= 1, "build_graph: total_k");
        SSA_CHECK_ARG(a->is_cross || a->N == a->M, "build_graph: self-attention needs N == M");
        SSA_CHECK_ARG(a->window >= 0, "build_graph: window");
        const int64_t ks = self ? (a->total_k - 1 < Kall ? a->total_k - 1 : Kall)
                                : (a->total_k < Kall ? a->total_k : Kall);
        D.Kout = (int)(self + ks);
    } else {
        D.Kout = D.kk;
    }
    SSA_CHECK_ARG(!a->causal || a->N <= a->M, "build_graph: causal needs N <= M");
    if (D.kk + D.chunk > 65535) {
        // the replay of tied rows indexes best ++ chunk with 16-bit positions
        ssa_set_error("build_graph: LSH top-k %d with stream chunks of %d slots exceeds the "
                      "65535 slots the exact tie replay supports", D.kk, D.chunk);
        return SSA_E_UNSUP;
    }
    {
        // one select row (its seen bitmap and buffer grow with the key length)
        // and the list sort's ranking of a long list must fit a workgroup's LDS
        const int cap = D.kk > SEL_CAP_LARGE_KK ? SEL_CAP_LARGE : SEL_CAP_SMALL;
        const int64_t sel = (int64_t)sel_lds_words(sel_bitmap_words(D.M), D.kk,
                                                   a->mode == SSA_GRAPH_LSH, D.nlists, cap) * 4;
        const int64_t lsr = (2 * (int64_t)((D.M + 31) / 32) + std::min(D.C, D.M) + 4) * 4;
        if (sel > SSA_LDS_BYTES || lsr > SSA_LDS_BYTES) {
            ssa_set_error("build_graph: key length %d unsupported here (a select row needs %lld "
                          "bytes of LDS, the list ranking %lld; at most %d)", D.M, (long long)sel,
                          (long long)lsr, SSA_LDS_BYTES);
            return SSA_E_UNSUP;
        }
    }
    // chunk the query heads so the score buffer stays near 8 GiB (a chunk's
    // select and rescore grids grow with it: one head of the 32k MQA workload
    // per chunk leaves a long tail per launch)
    const int64_t per_bh = (int64_t)a->N * D.nlists * D.Cs * 2;
    if (per_bh >= ((int64_t)4 << 30)) {
        ssa_set_error("build_graph: one head's score table (N * R * id sets * C * 2 = %lld bytes) "
                      "must stay below 4 GiB", (long long)per_bh);
        return SSA_E_UNSUP;
    }
    if ((int64_t)a->N * D.Cs * 2 >= ((int64_t)1 << 31)) {
        // the rescore addresses one (head, round, id set) instance's score rows
        // through 32-bit buffer offsets
        ssa_set_error("build_graph: one instance's score rows (N * C * 2 = %lld bytes) must stay "
                      "below 2 GiB", (long long)a->N * D.Cs * 2);
        return SSA_E_UNSUP;
    }
    {
        // the workgroup replay: as many blocks as 256 MiB of workspace hold (a
        // quarter of ws_cap without allocation), when its LDS fits
        const int nch = (int)ceil_div(D.Call, D.chunk);
        const int W = D.kk + D.chunk;
        const int shared = rpw_shared_words(sel_bitmap_words(D.M), D.nlists, D.kk, nch, D.Call);
        D.rpw_nsim = std::min<int>(RPW_WAVES, (SSA_LDS_BYTES / 4 - shared) / rpw_slot_words(W));
        const int64_t per = rpw_scratch_words(D.Call, D.M, D.kk, nch) * 4;
        const int64_t budget = ws_cap > 0 ? ws_cap / 4 : ((int64_t)256 << 20);
        D.rpw_blocks = (int)std::min<int64_t>(RPW_MAX_BLOCKS, budget / per);
        if (D.rpw_nsim < 1 || D.M >= (1 << 29) || D.Call >= ((int64_t)1 << 31)) D.rpw_blocks = 0;
    }
    // the per-wave replay's arrays, when they do not fit LDS: 64 MiB of
    // workspace (a sixteenth of ws_cap without allocation)
    D.rp_glb_blocks = (int)replay_glb_blocks(
        D.kk + D.chunk, sel_bitmap_words(D.M),
        ws_cap > 0 ? std::min<int64_t>(ws_cap / 16, (int64_t)64 << 20) : ((int64_t)64 << 20));
    {
        // the cut's rank table: 8 bytes per (kv head, round, bucket, 32 key
        // ids), when causal and within 256 MiB (a sixteenth of ws_cap)
        const int64_t tb = D.BK * D.R * D.NB * (int64_t)((D.M + 31) / 32) * 8;
        D.ctab = a->causal && tb <= (ws_cap > 0 ? ws_cap / 16 : ((int64_t)256 << 20)) ? 1 : 0;
    }
    int64_t nbh = ((int64_t)8 << 30) / per_bh;
    if (nbh < 1) nbh = 1;
    if (nbh > D.BH) nbh = D.BH;
    D.nbh_chunk = (int)nbh;
    if (ws_cap > 0 && plan(D).total > ws_cap) {
        // the workspace grows with the chunk's head count: the largest count
        // in [1, nbh) that fits, by bisection
        int lo = 1, hi = D.nbh_chunk - 1;
        while (lo < hi) {
            D.nbh_chunk = (lo + hi + 1) / 2;
            if (plan(D).total <= ws_cap) lo = D.nbh_chunk;
            else hi = D.nbh_chunk - 1;
        }
        D.nbh_chunk = lo;
        const int64_t need = plan(D).total;
        if (need > ws_cap) {
            ssa_set_error("build_graph: this problem needs %lld bytes of workspace with one query "
                          "head per chunk; the scratch array holds %lld",
                          (long long)need, (long long)ws_cap);
            return SSA_E_WORKSPACE;
        }
    }
    return SSA_OK;
}

template <typename T, int Dh>
int launch_hash_mfma(const HashP &hp, hipStream_t st) {
    const int NT = (hp.R * hp.P + 15) / 16;
    const size_t lds = (size_t)4 * 16 * (NT * 16 + 1) * 4;
    if (lds > SSA_LDS_BYTES) {
        ssa_set_error("hash: %d planes need %zu bytes of LDS", hp.R * hp.P, lds);
        return SSA_E_UNSUP;
    }
    SSA_CHECK_HIP(hipFuncSetAttribute((const void *)hash_mfma_kernel<T, Dh>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL((hash_mfma_kernel<T, Dh>), dim3((unsigned)ceil_div(hp.rows, 64)), dim3(256),
                       lds, st, hp);
    SSA_CHECK_LAUNCH();
    return SSA_OK;
}

template <typename T>
int launch_hash_one(const HashP &hp, int d, hipStream_t st) {
    if (hp.rows == 0) return SSA_OK;
    if (hp.inj) {
        hipLaunchKernelGGL(hash_kernel<T>, dim3((unsigned)ceil_div(hp.rows, 256)), dim3(256), 0,
                           st, hp);
        SSA_CHECK_LAUNCH();
        return SSA_OK;
    }
    switch (ssa_pow2_instance(d)) {
        case 4: return launch_hash_mfma<T, 4>(hp, st);
        case 8: return launch_hash_mfma<T, 8>(hp, st);
        case 16: return launch_hash_mfma<T, 16>(hp, st);
        case 32: return launch_hash_mfma<T, 32>(hp, st);
        case 64: return launch_hash_mfma<T, 64>(hp, st);
        case 128: return launch_hash_mfma<T, 128>(hp, st);
        case 256: return launch_hash_mfma<T, 256>(hp, st);
        case 512: return launch_hash_mfma<T, 512>(hp, st);
        case 1024: return launch_hash_mfma<T, 1024>(hp, st);
    }
    ssa_set_error("hash: head dim %d", d);
    return SSA_E_UNSUP;
}

bool view_aligned16(const ssa_tensor4 &t, int elem) {
    const int64_t v = 16 / elem;
    return (uintptr_t)t.ptr % 16 == 0 && t.sb % v == 0 && t.sh % v == 0 && t.sn % v == 0;
}

// The key hash can also give max |k|^2 per kv head when it reads the key rows
// itself (no injected projections) and 16-row tiles never straddle two heads.
bool key_norm_in_hash(const Dims &D, const ssa_graph_args *a) {
    return !a->k_proj && D.M % 16 == 0 && D.BK * D.M > 0;
}

template <typename T>
int launch_hash(const Dims &D, const ssa_graph_args *a, const Layout &L, char *ws,
                hipStream_t st, bool keys) {
    HashP hp{};
    hp.planes = a->rand_proj;
    hp.R = D.R; hp.maxP = D.maxP; hp.P = D.P; hp.Tp = D.Tp; hp.NS = D.NS; hp.d = D.d;
    hp.pl16 = (a->rand_proj && (uintptr_t)a->rand_proj % 16 == 0 && D.d % 4 == 0) ? 1 : 0;
    if (keys) {
        hp.x = a->k.ptr; hp.sb = a->k.sb; hp.sh = a->k.sh; hp.sn = a->k.sn;
        hp.nh = D.Hkv; hp.L = D.M; hp.inj = a->k_proj; hp.key_layout = 1;
        hp.vec16 = view_aligned16(a->k, (int)sizeof(T)) ? 1 : 0;
        hp.out = (uint16_t *)(ws + L.kid);
        hp.rows = D.BK * D.M;
        // the bucket sort's segment counter starts at zero
        hp.zero1 = ssa_sort_counter((uint16_t *)(ws + L.sorttmp), (int)(D.BK * D.R), D.M);
        if (key_norm_in_hash(D, a)) {
            // max |k|^2 per tile here, per kv head in the list sort
            hp.kpart = (uint32_t *)(ws + L.kpart);
        } else {
            // the max |k|^2 accumulators of knorm_kernel start at zero
            hp.zero = (uint32_t *)(ws + L.knorm);
            hp.nzero = (int)D.BK;
        }
        return launch_hash_one<T>(hp, D.d, st);
    }
    hp.x = a->q.ptr; hp.sb = a->q.sb; hp.sh = a->q.sh; hp.sn = a->q.sn;
    hp.nh = D.Hq; hp.L = D.N; hp.inj = a->q_proj; hp.key_layout = 0;
    hp.vec16 = view_aligned16(a->q, (int)sizeof(T)) ? 1 : 0;
    hp.out = (uint16_t *)(ws + L.qid);
    hp.rows = D.BH * D.N;
    // the tie-row counter of the select kernels (replayed once, after every chunk)
    hp.zero1 = (int32_t *)(ws + L.tie_count);
    return launch_hash_one<T>(hp, D.d, st);
}

template <typename T, int Dh>
int launch_rescore(const RsP &rp, int64_t grid, hipStream_t st) {
    const size_t lds = (size_t)(TQ + TC) * ((Dh < 256 ? Dh : 256) + 1) * 4 + (TQ + TC) * 4;
    SSA_CHECK_HIP(hipFuncSetAttribute((const void *)rescore_kernel<T, Dh>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL((rescore_kernel<T, Dh>), dim3((unsigned)grid), dim3(256), lds, st, rp);
    SSA_CHECK_LAUNCH();
    return SSA_OK;
}

template <typename T, int Dh>
int launch_rescore_mfma(const RsP &rp, int64_t grid, hipStream_t st) {
    // the member ids, rounded up to a whole slice (the slice buffers are static)
    const size_t lds = (size_t)ceil_div(rp.C, RS_SLICE) * RS_SLICE * 4;
    SSA_CHECK_HIP(hipFuncSetAttribute((const void *)rescore_mfma_kernel<T, Dh>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL((rescore_mfma_kernel<T, Dh>), dim3((unsigned)grid), dim3(256), lds, st, rp);
    SSA_CHECK_LAUNCH();
    return SSA_OK;
}

// 16-byte fragment loads need 16-byte aligned rows
bool rows_aligned16(const RsP &rp, int elem) {
    const int64_t v = 16 / elem;
    return ((uintptr_t)rp.q % 16 == 0) && ((uintptr_t)rp.k % 16 == 0) && rp.qsb % v == 0 &&
           rp.qsh % v == 0 && rp.qsn % v == 0 && rp.ksb % v == 0 && rp.ksh % v == 0 &&
           rp.ksn % v == 0;
}

template <typename T>
bool rescore_uses_mfma(int d, const RsP &rp) {
    return !std::is_same<T, float>::value && d >= 8 && d <= 128 && rows_aligned16(rp, 2) &&
           rp.k32;
}

template <typename T>
int rescore_dispatch(int d, const RsP &rp, int64_t grid, hipStream_t st) {
    if constexpr (!std::is_same<T, float>::value) {
        if (rescore_uses_mfma<T>(d, rp)) {
            switch (mfma_instance(d)) {
                case 8: return launch_rescore_mfma<T, 8>(rp, grid, st);
                case 16: return launch_rescore_mfma<T, 16>(rp, grid, st);
                case 32: return launch_rescore_mfma<T, 32>(rp, grid, st);
                case 64: return launch_rescore_mfma<T, 64>(rp, grid, st);
                case 96: return launch_rescore_mfma<T, 96>(rp, grid, st);
                case 128: return launch_rescore_mfma<T, 128>(rp, grid, st);
            }
        }
    }
    switch (ssa_pow2_instance(d)) {
        case 4: return launch_rescore<T, 4>(rp, grid, st);
        case 8: return launch_rescore<T, 8>(rp, grid, st);
        case 16: return launch_rescore<T, 16>(rp, grid, st);
        case 32: return launch_rescore<T, 32>(rp, grid, st);
        case 64: return launch_rescore<T, 64>(rp, grid, st);
        case 128: return launch_rescore<T, 128>(rp, grid, st);
        case 256: return launch_rescore<T, 256>(rp, grid, st);
        case 512: return launch_rescore<T, 512>(rp, grid, st);
        case 1024: return launch_rescore<T, 1024>(rp, grid, st);
    }
    ssa_set_error("rescore: head dim %d", d);
    return SSA_E_UNSUP;
}

template <typename T, bool LSH, bool CAUSAL, int CAP, bool WIDE>
int launch_select_w(const SelP &sp, size_t lds, hipStream_t st) {
    SSA_CHECK_HIP(hipFuncSetAttribute((const void *)select_kernel<T, LSH, CAUSAL, CAP, WIDE>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    const int64_t grid = 8 * ceil_div(sp.nblocks, 8);
    hipLaunchKernelGGL((select_kernel<T, LSH, CAUSAL, CAP, WIDE>), dim3((unsigned)grid),
                       dim3(sp.waves * SSA_WAVE), lds, st, sp);
    SSA_CHECK_LAUNCH();
    return SSA_OK;
}

template <typename T, bool LSH, bool CAUSAL, int CAP>
int launch_select(const SelP &sp0, hipStream_t st) {
    // SEL_WAVES rows per workgroup, fewer where a row's LDS (its seen bitmap
    // and buffer grow with the key length) leaves room for fewer
    const size_t per = (size_t)sel_lds_words(sp0.words, sp0.kk, LSH, sp0.nlists, CAP) * 4;
    const int waves = (int)std::min<size_t>(SEL_WAVES, SSA_LDS_BYTES / per);
    if (waves < 1) {
        ssa_set_error("build_graph: a select row needs %zu bytes of LDS (%d keys)", per, sp0.M);
        return SSA_E_UNSUP;
    }
    SelP sp = sp0;
    sp.waves = waves;
    sp.nblocks = ceil_div(sp.rows, waves);
    const size_t lds = (size_t)waves * per;
    return sp.cbits != 16 || waves != SEL_WAVES
               ? launch_select_w<T, LSH, CAUSAL, CAP, true>(sp, lds, st)
               : launch_select_w<T, LSH, CAUSAL, CAP, false>(sp, lds, st);
}

// Extra scores with the arithmetic of the rescore kernel rescore_dispatch picks
template <typename T>
int aux_dispatch(int d, bool mfma, const AuxP &ap, hipStream_t st) {
    const int64_t rows = (int64_t)ap.nbh * ap.N;
    if constexpr (!std::is_same<T, float>::value) {
        if (mfma) {
            const int64_t waves = (int64_t)ap.nbh * ((ap.N + 15) / 16);
            const dim3 grid((unsigned)ceil_div(waves, 4));
            // fused query hash: 16 projection rows of every plane tile per wave
            const size_t lds =
                ap.qid ? (size_t)4 * 16 * (ceil_div((int64_t)ap.R * ap.P, 16) * 16 + 1) * 4 : 0;
#define SSA_AUX_MFMA(DD) \
    case DD: hipLaunchKernelGGL((aux_mfma_kernel<T, DD>), grid, dim3(256), lds, st, ap); break;
            switch (mfma_instance(d)) {
                SSA_AUX_MFMA(8) SSA_AUX_MFMA(16) SSA_AUX_MFMA(32) SSA_AUX_MFMA(64)
                SSA_AUX_MFMA(96) SSA_AUX_MFMA(128)
                default: ssa_set_error("aux scores: head dim %d", d); return SSA_E_UNSUP;
            }
#undef SSA_AUX_MFMA
            SSA_CHECK_LAUNCH();
            return SSA_OK;
        }
    }
    const dim3 grid((unsigned)ceil_div(rows * ap.NA, 256));
#define SSA_AUX_VALU(DD) \
    case DD: hipLaunchKernelGGL((aux_valu_kernel<T, DD>), grid, dim3(256), 0, st, ap); break;
    switch (ssa_pow2_instance(d)) {
        SSA_AUX_VALU(4) SSA_AUX_VALU(8) SSA_AUX_VALU(16) SSA_AUX_VALU(32) SSA_AUX_VALU(64)
        SSA_AUX_VALU(128) SSA_AUX_VALU(256) SSA_AUX_VALU(512) SSA_AUX_VALU(1024)
        default: ssa_set_error("aux scores: head dim %d", d); return SSA_E_UNSUP;
    }
#undef SSA_AUX_VALU
    SSA_CHECK_LAUNCH();
    return SSA_OK;
}

// Exact top-k replay of the rows select flagged.  Up to `cap` tied rows go
// to the workgroup replay (rpw_blocks blocks at most, its arrays in LDS and in
// the workspace region `rpwscr`); more go to the per-wave replay, whose arrays
// (rp_lds_words(kk + chunk) words per row) live in LDS when RP_WAVES of them
// fit, else in the workspace region `rpscr` (replay_glb_blocks blocks).  Both
// are launched: each reads the tie count on the device and exits at once when
// the rows are the other's.
// the per-wave replay, its arrays in LDS or (when two rows do not fit) in
// the workspace; CT: the key ids' type
template <typename T, bool LSH, typename CT>
int launch_replay_pw(const SelP &sp, const Dims &D, int W, uint32_t *rpscr, int cap,
                     hipStream_t st) {
    const int chunk = D.chunk;
    if (!replay_fits_lds(W, sp.words)) {
        const int64_t blocks = D.rp_glb_blocks;
        hipLaunchKernelGGL((topk_replay_kernel<T, LSH, true, CT>), dim3((unsigned)blocks),
                           dim3(RP_WAVES * SSA_WAVE), 0, st, sp, chunk, W, rpscr, cap);
        SSA_CHECK_LAUNCH();
        return SSA_OK;
    }
    const size_t lds = (size_t)RP_WAVES * rp_lds_words(W, sp.words) * 4;
    SSA_CHECK_HIP(hipFuncSetAttribute((const void *)topk_replay_kernel<T, LSH, false, CT>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    // enough blocks for every resident wave to take a row (the rest exit at once)
    const int64_t blocks = std::min<int64_t>(ceil_div(sp.rows, RP_WAVES), 8192);
    hipLaunchKernelGGL((topk_replay_kernel<T, LSH, false, CT>), dim3((unsigned)blocks),
                       dim3(RP_WAVES * SSA_WAVE), lds, st, sp, chunk, W, (uint32_t *)nullptr, cap);
    SSA_CHECK_LAUNCH();
    return SSA_OK;
}

template <typename T, bool LSH>
int launch_replay(const SelP &sp, const Dims &D, uint32_t *rpscr, uint32_t *rpwscr,
                  hipStream_t st) {
    const int chunk = D.chunk;
    const int W = sp.kk + chunk;
    int cap = -1;
    if (D.rpw_blocks > 0) {
        const int nch = (int)ceil_div(sp.Call, chunk);
        const int lds = (D.rpw_nsim * rpw_slot_words(W) +
                         rpw_shared_words(sp.words, sp.R * sp.NS, sp.kk, nch, sp.Call)) * 4;
        int dev = 0, cus = 0;
        SSA_CHECK_HIP(hipGetDevice(&dev));
        SSA_CHECK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        SSA_CHECK_HIP(hipFuncSetAttribute((const void *)topk_replay_wg_kernel<T, LSH>,
                                          hipFuncAttributeMaxDynamicSharedMemorySize, lds));
        // the blocks resident at once (registers and LDS): each loops over its
        // rows; up to four rows per block beat the per-wave replay
        int per_cu = 0;
        SSA_CHECK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, (const void *)topk_replay_wg_kernel<T, LSH>, RPW_THREADS, lds));
        const int64_t blocks = std::min<int64_t>(
            std::min<int64_t>(D.rpw_blocks, (int64_t)cus * std::max(1, per_cu)), sp.rows);
        cap = (int)std::min<int64_t>(4 * blocks, sp.rows);
        hipLaunchKernelGGL((topk_replay_wg_kernel<T, LSH>), dim3((unsigned)blocks),
                           dim3(RPW_THREADS), (size_t)lds, st, sp, chunk, W, D.rpw_nsim, rpwscr,
                           rpw_scratch_words(sp.Call, sp.M, sp.kk, nch), cap);
        SSA_CHECK_LAUNCH();
    }
    return rp_wide_ids(sp.words) ? launch_replay_pw<T, LSH, uint32_t>(sp, D, W, rpscr, cap, st)
                                  : launch_replay_pw<T, LSH, uint16_t>(sp, D, W, rpscr, cap, st);
}

template <typename T, bool LSH>
int sel_dispatch_cap(const SelP &sp, hipStream_t st) {
    if (sp.kk > SEL_CAP_LARGE_KK)
        return sp.causal ? launch_select<T, LSH, true, SEL_CAP_LARGE>(sp, st)
                         : launch_select<T, LSH, false, SEL_CAP_LARGE>(sp, st);
    return sp.causal ? launch_select<T, LSH, true, SEL_CAP_SMALL>(sp, st)
                     : launch_select<T, LSH, false, SEL_CAP_SMALL>(sp, st);
}

template <typename T>
int select_dispatch(const SelP &sp, hipStream_t st) {
    if (sp.mode == SSA_GRAPH_LSH)
        return sel_dispatch_cap<T, true>(sp, st);
    return sel_dispatch_cap<T, false>(sp, st);
}

// Key phase: bucket ids of the keys, the bucket permutation and tables and
// the sorted candidate lists -- everything that needs k but not q.
// the rescore's parameters that hold for every head chunk
RsP rescore_common(const Dims &D, const ssa_graph_args *a, const Layout &L, char *ws) {
    RsP rp{};
    rp.sid = (const int32_t *)(ws + L.sid);
    rp.bstart = (const int32_t *)(ws + L.bstart);
    rp.bsize = (const int32_t *)(ws + L.bsize);
    rp.q = a->q.ptr; rp.k = a->k.ptr;
    rp.qsb = a->q.sb; rp.qsh = a->q.sh; rp.qsn = a->q.sn;
    rp.ksb = a->k.sb; rp.ksh = a->k.sh; rp.ksn = a->k.sn;
    rp.S = (uint16_t *)(ws + L.S);
    rp.N = D.N; rp.M = D.M; rp.R = D.R; rp.NS = D.NS; rp.NB = D.NB; rp.C = D.C;
    rp.Hq = D.Hq; rp.Hkv = D.Hkv; rp.rep = D.rep; rp.Call = D.Call;
    rp.causal = a->causal ? 1 : 0;
    rp.Cs = D.Cs;
    rp.d = D.d;
    {
        const int64_t el = a->q.dtype == SSA_F32 ? 4 : 2;
        rp.k32 = (rp.ksn * el < ((int64_t)1 << 24) &&
                  ((int64_t)D.M * rp.ksn + D.d) * el < ((int64_t)1 << 31)) ? 1 : 0;
    }
    return rp;
}

// With aux on the matrix cores, aux_mfma_kernel also hashes the queries (one
// pass over q): without injected projections, with 16-byte aligned planes and
// their projection rows within 48 KB of LDS per block
template <typename T>
bool aux_hashes_queries(const Dims &D, const ssa_graph_args *a, bool mfma) {
    const int np16 = (int)ceil_div((int64_t)D.R * D.P, 16) * 16;
    return mfma && !a->q_proj && (uintptr_t)a->rand_proj % 16 == 0 &&
           (size_t)4 * 16 * (np16 + 1) * 4 <= 48 * 1024;
}

// The first head chunk's aux pass runs beside the key sort's top levels
// (sort_aux_kernel) when it hashes the queries, the key hash left its norm
// tiles and the sort keeps its rows in LDS
template <typename T>
bool sort_beside_aux(const Dims &D, const ssa_graph_args *a, const Layout &L, char *ws) {
    if constexpr (std::is_same<T, float>::value) {
        return false;
    } else {
        const RsP rp = rescore_common(D, a, L, ws);
        const bool mfma = rescore_uses_mfma<T>(D.d, rp);
        return !D.fused && aux_hashes_queries<T>(D, a, mfma) && key_norm_in_hash(D, a) &&
               D.M <= 32768 && D.BH * D.N > 0;
    }
}

AuxP aux_params(const Dims &D, const ssa_graph_args *a, const Layout &L, char *ws, int64_t bh0,
                int nbh, bool qhash) {
    AuxP ap{};
    ap.q = a->q.ptr; ap.k = a->k.ptr;
    ap.qsb = a->q.sb; ap.qsh = a->q.sh; ap.qsn = a->q.sn;
    ap.ksb = a->k.sb; ap.ksh = a->k.sh; ap.ksn = a->k.sn;
    ap.glob = a->glob;
    ap.knorm = (const uint32_t *)(ws + L.knorm);
    ap.N = D.N; ap.Hq = D.Hq; ap.Hkv = D.Hkv; ap.rep = D.rep; ap.bh0 = (int)bh0;
    ap.nbh = nbh; ap.G = D.G; ap.NA = D.G + 3; ap.causal = a->causal; ap.d = D.d;
    // (fused: the query projection wrote every head's aux rows and ids)
    ap.out = (float *)(ws + L.aux) + (D.fused ? bh0 * (int64_t)D.N * ap.NA : 0);
    if (qhash) {
        ap.planes = a->rand_proj;
        ap.R = D.R; ap.maxP = D.maxP; ap.P = D.P; ap.Tp = D.Tp; ap.NS = D.NS;
        ap.qid = (uint16_t *)(ws + L.qid);
        // the tie-row counter of the select kernels (replayed once, after every chunk)
        ap.zero1 = bh0 == 0 ? (int32_t *)(ws + L.tie_count) : nullptr;
    }
    return ap;
}

// Query bucketing parameters of the head chunk [bh0, bh0 + nbh)
QbP qb_params(const Dims &D, const ssa_graph_args *a, const Layout &L, char *ws, int64_t bh0,
              int nbh) {
    QbP qp{};
    qp.qid = (const uint16_t *)(ws + L.qid);
    qp.bsize = (const int32_t *)(ws + L.bsize);
    qp.bstart = (const int32_t *)(ws + L.bstart);
    qp.cnt = (int32_t *)(ws + L.cnt);
    qp.off = (int32_t *)(ws + L.off);
    qp.cur = nullptr;
    qp.hcnt = (int32_t *)(ws + L.cur);
    qp.qlist = (int32_t *)(ws + L.qlist);
    qp.tiles = (int32_t *)(ws + L.tiles);
    qp.ntiles = (int32_t *)(ws + L.ntiles);
    qp.tcnt = (int32_t *)(ws + L.tcnt);
    qp.kbase = (int32_t *)(ws + L.kbase);
    qp.N = D.N; qp.R = D.R; qp.NS = D.NS; qp.NB = D.NB; qp.Hq = D.Hq; qp.Hkv = D.Hkv;
    qp.rep = D.rep; qp.bh0 = (int)bh0; qp.ninst = nbh * D.R * D.NS; qp.C = D.C;
    // round-major tiles when a head's q rows exceed half an XCD's 4 MB L2
    qp.rmajor = (int64_t)D.N * D.d * (a->q.dtype == SSA_F32 ? 4 : 2) > ((int64_t)2 << 20);
    return qp;
}

// Static LDS of the list sort's and the bucket scan's workgroup bodies (kred,
// part, sq, st), with room to spare
constexpr size_t LS_SCAN_STATIC_LDS = 4096;

template <typename T>
int launch_sort_aux(const Dims &D, const ssa_graph_args *a, const Layout &L, char *ws,
                    hipStream_t st) {
    SortTopArgs sa{};
    int rc = ssa_sort_top_setup((const uint16_t *)(ws + L.kid), (int)(D.BK * D.R), D.M, D.P,
                                (int32_t *)(ws + L.perm), (int32_t *)(ws + L.bstart),
                                (int32_t *)(ws + L.bsize), (uint16_t *)(ws + L.sorttmp), &sa);
    if (rc) return rc;
    const int nbh = (int)std::min<int64_t>(D.BH, D.nbh_chunk);
    AuxP ap = aux_params(D, a, L, ws, 0, nbh, true);
    ap.kpart = (const uint32_t *)(ws + L.kpart);
    ap.kp_n = D.M / 16;
    const int64_t waves = (int64_t)nbh * ceil_div(D.N, 16);
    const int64_t grid = sa.rows + ceil_div(waves, SORT_WAVES);
    const size_t lds = std::max<size_t>((size_t)sa.lds,
                                        (size_t)SORT_WAVES * aux_wave_floats(D.R, D.P) * 4);
    SSA_CHECK_ARG(lds <= SORT_LDS_BYTES, "build_graph: sort and aux need %zu bytes of LDS", lds);
    const void *fn = nullptr;
    switch (mfma_instance(D.d)) {
        case 8: fn = (const void *)sort_aux_kernel<T, 8>; break;
        case 16: fn = (const void *)sort_aux_kernel<T, 16>; break;
        case 32: fn = (const void *)sort_aux_kernel<T, 32>; break;
        case 64: fn = (const void *)sort_aux_kernel<T, 64>; break;
        case 96: fn = (const void *)sort_aux_kernel<T, 96>; break;
        case 128: fn = (const void *)sort_aux_kernel<T, 128>; break;
        default: ssa_set_error("sort and aux: head dim %d", D.d); return SSA_E_UNSUP;
    }
    SSA_CHECK_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    switch (mfma_instance(D.d)) {
#define SSA_SORT_AUX(DD)                                                                     \
    case DD:                                                                                 \
        hipLaunchKernelGGL((sort_aux_kernel<T, DD>), dim3((unsigned)grid), dim3(SORT_THREADS), \
                           lds, st, sa, ap);                                                 \
        break;
        SSA_SORT_AUX(8) SSA_SORT_AUX(16) SSA_SORT_AUX(32) SSA_SORT_AUX(64) SSA_SORT_AUX(96)
        SSA_SORT_AUX(128)
#undef SSA_SORT_AUX
    }
    SSA_CHECK_LAUNCH();
    // the segments, beside the first chunk's query histogram (its ids came
    // from the launch above)
    static_assert(SEG_WAVES * SSA_WAVE == 256, "the query histogram takes 256 queries a block");
    const QbP qp = qb_params(D, a, L, ws, 0, nbh);
    const int nseg = ssa_sort_seg_blocks(sa.rows, sa.n);
    const int nqb = (int)ceil_div(D.N, 256);
    const size_t hl = std::max<size_t>((size_t)SEG_WAVES * seg_lds_words<uint16_t>() * 4,
                                       (size_t)D.NB * 4);
    SSA_CHECK_HIP(hipFuncSetAttribute((const void *)sort_seg_hist_kernel,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)hl));
    hipLaunchKernelGGL(sort_seg_hist_kernel, dim3((unsigned)(nseg + (int64_t)qp.ninst * nqb)),
                       dim3(256), hl, st, sa, qp, nseg, nqb);
    SSA_CHECK_LAUNCH();
    return SSA_OK;
}

template <typename T>
int keys_typed(const Dims &D, const ssa_graph_args *a, const Layout &L, char *ws,
               hipStream_t st, bool sort_aux) {
    int rc = SSA_OK;
    {
        // (fused: the key projection wrote the key ids and the 16-row norm maxima)
        if (!D.fused) rc = launch_hash<T>(D, a, L, ws, st, true);
        if (rc) return rc;
        // max |k|^2 per (batch, kv head): the query code scales derive from it
        KnP kp{};
        kp.k = a->k.ptr; kp.ksb = a->k.sb; kp.ksh = a->k.sh; kp.ksn = a->k.sn;
        kp.Hkv = D.Hkv; kp.M = D.M; kp.d = D.d;
        kp.out = (uint32_t *)(ws + L.knorm);
        if (key_norm_in_hash(D, a)) {
            // the list sort reduces the key hash's tile maxima
        } else if (D.BK * D.M == 0) {  // else the key hash cleared it
            hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(256), 0, st, (int32_t *)kp.out,
                               (int64_t)D.BK, 0);
            SSA_CHECK_LAUNCH();
        } else {
            const int seg = (int)((int64_t)D.d * (int64_t)sizeof(T) / 16);
            const bool vec = view_aligned16(a->k, (int)sizeof(T)) && D.d * (int)sizeof(T) % 16 == 0 &&
                             seg >= 4 && seg <= 32;
            // about 256 blocks, at least 64 rows each
            const int64_t nc = std::max<int64_t>(
                1, std::min<int64_t>(ceil_div(256, D.BK), ceil_div(D.M, 64)));
            kp.per = (int)ceil_div(D.M, nc);
            const dim3 grid((unsigned)ceil_div(D.M, kp.per), (unsigned)D.BK);
            if (vec && seg == 4) hipLaunchKernelGGL((knorm_kernel<T, 4>), grid, dim3(256), 0, st, kp);
            else if (vec && seg == 8) hipLaunchKernelGGL((knorm_kernel<T, 8>), grid, dim3(256), 0, st, kp);
            else if (vec && seg == 16) hipLaunchKernelGGL((knorm_kernel<T, 16>), grid, dim3(256), 0, st, kp);
            else if (vec && seg == 32) hipLaunchKernelGGL((knorm_kernel<T, 32>), grid, dim3(256), 0, st, kp);
            else hipLaunchKernelGGL((knorm_kernel<T, 0>), grid, dim3(256), 0, st, kp);
            SSA_CHECK_LAUNCH();
        }
    }
    // the key hash cleared the sort's counter
    bool done = false;
    if constexpr (!std::is_same<T, float>::value) {
        if (sort_aux) {
            rc = launch_sort_aux<T>(D, a, L, ws, st);
            done = true;
        }
    }
    if (!done) {
        rc = ssa_launch_bucket_sort((const uint16_t *)(ws + L.kid), (int)(D.BK * D.R), D.M, D.P,
                                    (int32_t *)(ws + L.perm), (int32_t *)(ws + L.bstart),
                                    (int32_t *)(ws + L.bsize), (uint16_t *)(ws + L.sorttmp), st,
                                    false);
    }
    if (rc) return rc;
    {
        LsP lp{};
        lp.perm = (const int32_t *)(ws + L.perm);
        lp.bstart = (const int32_t *)(ws + L.bstart);
        lp.bsize = (const int32_t *)(ws + L.bsize);
        lp.sid = (int32_t *)(ws + L.sid);
        lp.rnk = (int32_t *)(ws + L.rnk);
        lp.smin = (int32_t *)(ws + L.smin);
        lp.inv = (int32_t *)(ws + L.inv);
        lp.M = D.M; lp.NB = D.NB; lp.C = D.C;
        lp.ctab = D.ctab ? (uint2 *)(ws + L.ctab) : nullptr;
        if (key_norm_in_hash(D, a)) {
            lp.kpart = (const uint32_t *)(ws + L.kpart);
            lp.knorm = (uint32_t *)(ws + L.knorm);
            lp.R = D.R;
        }
        int p2 = 1;
        while (p2 < std::min(D.C, D.M)) p2 <<= 1;
        const size_t lds = std::max((size_t)p2 * 4,
                                    (size_t)(2 * ((D.M + 31) / 32) + std::min(D.C, D.M) + 4) * 4);
        if (lds > SSA_LDS_BYTES) {
            ssa_set_error("build_graph: ranking lists of up to %d members over %d keys needs %zu "
                          "bytes of LDS", D.C, D.M, lds);
            return SSA_E_UNSUP;
        }
        const int64_t nls = D.BK * D.R * D.NB;
        if (sort_aux && lds + LS_SCAN_STATIC_LDS <= SSA_LDS_BYTES) {
            // beside the first chunk's bucket scan (its histogram ran beside
            // the segments)
            const QbP qp = qb_params(D, a, L, ws, 0, (int)std::min<int64_t>(D.BH, D.nbh_chunk));
            SSA_CHECK_HIP(hipFuncSetAttribute((const void *)list_sort_scan_kernel,
                                              hipFuncAttributeMaxDynamicSharedMemorySize,
                                              (int)lds));
            hipLaunchKernelGGL(list_sort_scan_kernel, dim3((unsigned)(nls + qp.ninst)), dim3(256),
                               lds, st, lp, qp, (int)nls);
            SSA_CHECK_LAUNCH();
            return SSA_OK;
        }
        SSA_CHECK_HIP(hipFuncSetAttribute((const void *)list_sort_kernel,
                                          hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        hipLaunchKernelGGL(list_sort_kernel, dim3((unsigned)nls), dim3(256), lds, st, lp);
        SSA_CHECK_LAUNCH();
        if (sort_aux) {
            const QbP qp = qb_params(D, a, L, ws, 0, (int)std::min<int64_t>(D.BH, D.nbh_chunk));
            hipLaunchKernelGGL(qb_scan_kernel, dim3((unsigned)qp.ninst), dim3(256), 0, st, qp);
            SSA_CHECK_LAUNCH();
        }
    }
    return SSA_OK;
}

// Query phase: everything else, given the key phase's results in ws.
template <typename T>
int queries_typed(const Dims &D, const ssa_graph_args *a, const Layout &L, char *ws,
                  hipStream_t st, bool sort_aux) {
    RsP rp = rescore_common(D, a, L, ws);
    const bool mfma = rescore_uses_mfma<T>(D.d, rp);
    const bool fuse_qhash = aux_hashes_queries<T>(D, a, mfma);
    int rc = SSA_OK;
    if (!fuse_qhash && !D.fused) {
        rc = launch_hash<T>(D, a, L, ws, st, false);
        if (rc) return rc;
    }
    SelP last{};
    for (int64_t bh0 = 0; bh0 < D.BH; bh0 += D.nbh_chunk) {
        const int nbh = (int)((D.BH - bh0) < D.nbh_chunk ? (D.BH - bh0) : D.nbh_chunk);
        const int ninst = nbh * D.R * D.NS;
        // aux first: the rescore codes its scores with the query scales it
        // writes, and the query buckets need the ids it writes when fused
        // (the first chunk's ran beside the key sort when sort_aux)
        const AuxP ap = aux_params(D, a, L, ws, bh0, nbh, fuse_qhash);
        if (!D.fused && !(sort_aux && bh0 == 0)) rc = aux_dispatch<T>(D.d, mfma, ap, st);
        if (rc) return rc;
        QbP qp = qb_params(D, a, L, ws, bh0, nbh);
        const dim3 gq((unsigned)ceil_div(D.N, 256), (unsigned)ninst);
        // (the first chunk's histogram and scan ran in the key phase when sort_aux)
        if (!(sort_aux && bh0 == 0)) {
            hipLaunchKernelGGL(qb_hist_kernel, gq, dim3(256), (size_t)D.NB * 4, st, qp);
            SSA_CHECK_LAUNCH();
            hipLaunchKernelGGL(qb_scan_kernel, dim3((unsigned)ninst), dim3(256), 0, st, qp);
            SSA_CHECK_LAUNCH();
        }
        {
            auto bk_of = [&](int64_t bh) { return (bh / D.Hq) * D.Hkv + (bh % D.Hq) / D.rep; };
            qp.heads = (bk_of(bh0 + nbh - 1) - bk_of(bh0) + 1) * D.rep;
            const int64_t nkeys = qp.heads * D.R * D.NS;
            hipLaunchKernelGGL(qb_order_kernel, dim3(1), dim3(256), 0, st, qp, nkeys);
            SSA_CHECK_LAUNCH();
        }
        // the query scatter also writes each (query, list) cut entry: it has
        // the query's bucket and its position in the bucket's query list
        CutP cp{};
        cp.perm = (const int32_t *)(ws + L.perm);
        cp.bstart = rp.bstart; cp.bsize = rp.bsize; cp.sid = rp.sid;
        cp.smin = (const int32_t *)(ws + L.smin);
        cp.glob = a->glob;
        cp.cut = (int4 *)(ws + L.cut);
        cp.srix = (int32_t *)(ws + L.srix);
        cp.ctab = D.ctab ? (const uint2 *)(ws + L.ctab) : nullptr;
        cp.N = D.N; cp.M = D.M; cp.R = D.R; cp.NS = D.NS; cp.NB = D.NB; cp.C = D.C; cp.Cs = D.Cs;
        cp.Hq = D.Hq; cp.Hkv = D.Hkv; cp.rep = D.rep; cp.bh0 = (int)bh0; cp.G = D.G;
        cp.causal = a->causal ? 1 : 0; cp.nlists = D.nlists; cp.rows = (int64_t)nbh * D.N;
        cp.cbits = D.cbits;
        hipLaunchKernelGGL(qb_scatter_kernel, gq, dim3(256), (size_t)std::max(D.NB * 16, 256 * 4),
                           st, qp, cp);
        SSA_CHECK_LAUNCH();

        rp.tiles = qp.tiles; rp.ntiles = qp.ntiles; rp.qlist = qp.qlist;
        rp.bh0 = (int)bh0;
        rp.aux = ap.out;
        rp.NA = ap.NA;
        const int64_t grid = 8 * ceil_div((int64_t)ninst * (ceil_div(D.N, TQ) + D.NB), 8);
        rc = rescore_dispatch<T>(D.d, rp, grid, st);
        if (rc) return rc;

        SelP sp{};
        sp.qid = qp.qid; sp.perm = cp.perm; sp.bstart = rp.bstart; sp.bsize = rp.bsize;
        sp.sid = rp.sid; sp.rnk = (const int32_t *)(ws + L.rnk);
        sp.inv = (const int32_t *)(ws + L.inv); sp.cut = cp.cut; sp.srix = cp.srix;
        sp.head_bytes = (uint32_t)((int64_t)D.N * D.nlists * D.Cs * 2);
        sp.mfma = mfma ? 1 : 0;
        sp.nl_magic = (uint32_t)((((uint64_t)1 << 32) + D.nlists - 1) / D.nlists);
        sp.S = rp.S; sp.q = a->q.ptr; sp.k = a->k.ptr;
        sp.qsb = a->q.sb; sp.qsh = a->q.sh; sp.qsn = a->q.sn;
        sp.ksb = a->k.sb; sp.ksh = a->k.sh; sp.ksn = a->k.sn;
        sp.glob = a->glob;
        sp.N = D.N; sp.M = D.M; sp.d = D.d; sp.R = D.R; sp.NS = D.NS; sp.NB = D.NB; sp.C = D.C;
        sp.Cs = D.Cs;
        sp.CPL = D.CPL; sp.nlists = D.nlists; sp.Hq = D.Hq; sp.Hkv = D.Hkv; sp.rep = D.rep;
        sp.G = D.G; sp.kk = D.kk; sp.window = a->window; sp.causal = a->causal;
        sp.cross = a->is_cross; sp.mode = a->mode; sp.total_k = a->total_k; sp.Kw = D.Kw;
        sp.Kout = D.Kout; sp.bh0 = (int)bh0; sp.words = sel_bitmap_words(D.M);
        sp.Call = D.Call; sp.rows = (int64_t)nbh * D.N; sp.rows_all = D.BH * D.N;
        sp.out_idx = a->out_idx; sp.out_valid = a->out_valid; sp.ties = a->out_ties;
        sp.out_idx32 = a->mode == SSA_GRAPH_FULL ? a->out_idx32 : nullptr;
        sp.tie_list = (int32_t *)(ws + L.tie_list);
        sp.tie_count = (int32_t *)(ws + L.tie_count);
        sp.aux = ap.out;
        sp.NA = ap.NA;
        sp.perm_bytes = (int)(D.BK * D.R * D.M * 4);
        sp.cbits = D.cbits;
        rc = select_dispatch<T>(sp, st);
        if (rc) return rc;
        last = sp;
    }
    if (D.BH * D.N == 0) return SSA_OK;
    // the rows every chunk flagged, in one launch: each row's replay is a long
    // chain of dependent steps, so rows from all chunks run side by side
    SelP xp = last;
    xp.bh0 = 0;
    xp.rows = D.BH * D.N;
    uint32_t *rpscr = (uint32_t *)(ws + L.rpscr);
    uint32_t *rpwscr = (uint32_t *)(ws + L.rpw);
    return xp.mode == SSA_GRAPH_LSH ? launch_replay<T, true>(xp, D, rpscr, rpwscr, st)
                                    : launch_replay<T, false>(xp, D, rpscr, rpwscr, st);
}

}  // namespace

extern "C" int64_t ssa_graph_out_width(const ssa_graph_args *a) {
    Dims D;
    if (make_dims(a, D, false)) return -1;
    return D.Kout;
}

extern "C" int64_t ssa_graph_workspace_bytes(const ssa_graph_args *a) {
    Dims D;
    if (make_dims(a, D, false)) return -1;
    return plan(D).total;
}

namespace {
int build_impl(const ssa_graph_args *a, void *workspace, int64_t workspace_bytes, void *stream,
               int64_t ws_cap = 0) {
    Dims D;
    int rc = make_dims(a, D, true, ws_cap);
    if (rc) return rc;
    {
        const bool i32 = a->mode == SSA_GRAPH_FULL && a->out_idx32;
        SSA_CHECK_ARG(i32 || a->out_idx, "build_graph: out_idx is null");
        SSA_CHECK_ARG(i32 || a->mode != SSA_GRAPH_FULL || a->out_valid,
                      "build_graph: out_valid is null");
    }
    const Layout L = plan(D);
    if (workspace_bytes < L.total || !workspace) {
        ssa_set_error("build_graph: workspace %lld < %lld bytes", (long long)workspace_bytes,
                      (long long)L.total);
        return SSA_E_WORKSPACE;
    }
    hipStream_t st = (hipStream_t)stream;
    char *ws = (char *)workspace;
    switch (a->k.dtype) {
        case SSA_F32:
        {
            const bool sa = sort_beside_aux<float>(D, a, L, ws);
            if ((rc = keys_typed<float>(D, a, L, ws, st, sa))) return rc;
            return queries_typed<float>(D, a, L, ws, st, sa);
        }
        case SSA_BF16:
        {
            const bool sa = sort_beside_aux<bf16_t>(D, a, L, ws);
            if ((rc = keys_typed<bf16_t>(D, a, L, ws, st, sa))) return rc;
            return queries_typed<bf16_t>(D, a, L, ws, st, sa);
        }
        case SSA_F16:
        {
            const bool sa = sort_beside_aux<f16_t>(D, a, L, ws);
            if ((rc = keys_typed<f16_t>(D, a, L, ws, st, sa))) return rc;
            return queries_typed<f16_t>(D, a, L, ws, st, sa);
        }
    }
    return SSA_E_ARG;
}
}  // namespace

extern "C" int ssa_build_graph(const ssa_graph_args *a, void *workspace, int64_t workspace_bytes,
                               void *stream) {
    return build_impl(a, workspace, workspace_bytes, stream);
}

int64_t ssa_graph_workspace_bytes_capped(const ssa_graph_args *a, int64_t ws_cap) {
    Dims D;
    const int rc = make_dims(a, D, false, ws_cap);
    if (rc) return rc;
    return plan(D).total;
}

int ssa_build_graph_capped(const ssa_graph_args *a, void *workspace, int64_t ws_cap,
                           void *stream) {
    return build_impl(a, workspace, ws_cap, stream, ws_cap);
}

// ---------------------------------------------------------------------------
// Projections and graph build in one call (bf16): the projections' epilogue
// hashes the rows it writes (ssa_proj.hip), so the build reads q and k only
// for the rescore, the exact keys and the apply.
namespace {

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// The fused path's conditions beyond make_dims'; with `why`, the reason it is
// refused goes to the error text.
int project_check(const ssa_project_graph_args *pa, Dims &D, bool why) {
    auto refuse = [&](const char *msg) {
        if (why) ssa_set_error("project_build_graph: %s", msg);
        return SSA_E_UNSUP;
    };
    if (!pa) return refuse("null args");
    const ssa_graph_args *a = &pa->graph;
    if (make_dims(a, D, true, 0, true)) return why ? SSA_E_ARG : SSA_E_UNSUP;
    if (a->q.dtype != SSA_BF16 || a->k.dtype != SSA_BF16) return refuse("bf16 only");
    if (a->q_proj || a->k_proj || !a->rand_proj) return refuse("injected projections");
    if (!pa->x || !pa->src || !pa->wq || !pa->wkv || !pa->q_out || !pa->kv_out)
        return refuse("null operand");
    if (!aligned16(pa->x) || !aligned16(pa->src) || !aligned16(pa->wq) || !aligned16(pa->wkv) ||
        !aligned16(pa->q_out) || !aligned16(pa->kv_out))
        return refuse("operands must be 16-byte aligned");
    const int d = D.d, qc = D.Hq * d, kc = 2 * D.Hkv * d;
    if (a->q.ptr != pa->q_out || a->q.sb != (int64_t)D.N * qc || a->q.sh != d || a->q.sn != qc)
        return refuse("graph.q is not the (B, Hq, N, d) view of q_out");
    if (a->k.ptr != pa->kv_out || a->k.sb != (int64_t)D.M * kc || a->k.sh != d || a->k.sn != kc)
        return refuse("graph.k is not the (B, Hkv, M, d) view of kv_out");
    if (D.N % 16 || D.M % 16) return refuse("N and M must be multiples of 16");
    const int np = D.R * D.P;
    if (!ssa_project_supported((int)(D.B * (int64_t)D.N), qc, pa->d_model, d, np) ||
        !ssa_project_supported((int)(D.B * (int64_t)D.M), kc, pa->d_model, d, np) ||
        D.B * (int64_t)std::max(D.N, D.M) >= ((int64_t)1 << 31))
        return refuse("sizes outside the projection kernel's (d 32/64/128, d_model a multiple "
                      "of 64, Hq*d and 2*Hkv*d multiples of 256, few enough hyperplanes)");
    // the aux scores repeat the matrix-core rescore's arithmetic
    if ((int64_t)kc * 2 >= ((int64_t)1 << 24) ||
        ((int64_t)D.M * kc + d) * 2 >= ((int64_t)1 << 31))
        return refuse("key rows beyond the matrix-core rescore's 32-bit offsets");
    return SSA_OK;
}

int project_build_impl(const ssa_project_graph_args *pa, void *workspace, int64_t workspace_bytes,
                       void *stream) {
    Dims D;
    int rc = project_check(pa, D, true);
    if (rc) return rc;
    const ssa_graph_args *a = &pa->graph;
    {
        const bool i32 = a->mode == SSA_GRAPH_FULL && a->out_idx32;
        SSA_CHECK_ARG(i32 || a->out_idx, "project_build_graph: out_idx is null");
        SSA_CHECK_ARG(i32 || a->mode != SSA_GRAPH_FULL || a->out_valid,
                      "project_build_graph: out_valid is null");
    }
    const Layout L = plan(D);
    if (workspace_bytes < L.total || !workspace) {
        ssa_set_error("project_build_graph: workspace %lld < %lld bytes",
                      (long long)workspace_bytes, (long long)L.total);
        return SSA_E_WORKSPACE;
    }
    hipStream_t st = (hipStream_t)stream;
    char *ws = (char *)workspace;
    const int d = D.d;
    uint16_t *psplit = (uint16_t *)(ws + L.psplit);
    if ((rc = ssa_launch_plane_split(a->rand_proj, D.R, D.maxP, D.P, d, psplit, st))) return rc;
    ProjP kp{};
    kp.x = pa->src; kp.ldx = pa->d_model;
    kp.w = pa->wkv; kp.ldw = pa->d_model;
    kp.y = pa->kv_out; kp.ldy = 2 * D.Hkv * d;
    kp.rows = (int)(D.B * (int64_t)D.M); kp.cols = 2 * D.Hkv * d; kp.K = pa->d_model;
    kp.mode = SSA_PROJ_KEYS; kp.L = D.M; kp.d = d; kp.heads = D.Hkv;
    kp.psplit = psplit; kp.R = D.R; kp.P = D.P; kp.Tp = D.Tp; kp.NS = D.NS;
    kp.ids = (uint16_t *)(ws + L.kid);
    kp.kpart = (uint32_t *)(ws + L.kpart);
    // the bucket sort's segment counter starts at zero
    kp.zero1 = ssa_sort_counter((uint16_t *)(ws + L.sorttmp), (int)(D.BK * D.R), D.M);
    if ((rc = ssa_launch_project(kp, st))) return rc;
    if ((rc = keys_typed<bf16_t>(D, a, L, ws, st, false))) return rc;
    ProjP qp{};
    qp.x = pa->x; qp.ldx = pa->d_model;
    qp.w = pa->wq; qp.ldw = pa->d_model;
    qp.y = pa->q_out; qp.ldy = D.Hq * d;
    qp.rows = (int)(D.B * (int64_t)D.N); qp.cols = D.Hq * d; qp.K = pa->d_model;
    qp.mode = SSA_PROJ_QUERIES; qp.L = D.N; qp.Lk = D.M; qp.d = d; qp.heads = D.Hq;
    qp.psplit = psplit; qp.R = D.R; qp.P = D.P; qp.Tp = D.Tp; qp.NS = D.NS;
    qp.ids = (uint16_t *)(ws + L.qid);
    // the tie-row counter of the select kernels (replayed once, after every chunk)
    qp.zero1 = (int32_t *)(ws + L.tie_count);
    qp.k = a->k.ptr; qp.ksb = a->k.sb; qp.ksh = a->k.sh; qp.ksn = a->k.sn;
    qp.glob = a->glob; qp.G = D.G; qp.NA = D.G + 3; qp.causal = a->causal ? 1 : 0;
    qp.Hq = D.Hq; qp.Hkv = D.Hkv; qp.rep = D.rep;
    qp.knorm = (const uint32_t *)(ws + L.knorm);
    qp.aux = (float *)(ws + L.aux);
    if ((rc = ssa_launch_project(qp, st))) return rc;
    return queries_typed<bf16_t>(D, a, L, ws, st, false);
}

}  // namespace

extern "C" int ssa_project_graph_supported(const ssa_project_graph_args *a) {
    Dims D;
    return project_check(a, D, false) == SSA_OK ? 1 : 0;
}

extern "C" int64_t ssa_project_graph_workspace_bytes(const ssa_project_graph_args *a) {
    Dims D;
    const int rc = project_check(a, D, true);
    if (rc) return rc;
    return plan(D).total;
}

extern "C" int ssa_project_build_graph(const ssa_project_graph_args *a, void *workspace,
                                       int64_t workspace_bytes, void *stream) {
    return project_build_impl(a, workspace, workspace_bytes, stream);
}

extern "C" int ssa_project_gemm(const void *x, int64_t ldx, const void *w, int64_t ldw, void *y,
                                int64_t ldy, int32_t rows, int32_t cols, int32_t K, void *stream) {
    ProjP p{};
    p.x = x; p.ldx = ldx; p.w = w; p.ldw = ldw; p.y = y; p.ldy = ldy;
    p.rows = rows; p.cols = cols; p.K = K;
    p.mode = SSA_PROJ_PLAIN;
    SSA_CHECK_ARG(x && w && y && aligned16(x) && aligned16(w) && aligned16(y) && ldx % 8 == 0 &&
                      ldw % 8 == 0 && ldy % 8 == 0,
                  "project_gemm: operands must be 16-byte aligned rows");
    return ssa_launch_project(p, (hipStream_t)stream);
}

extern "C" int ssa_checked_oob(uint32_t *record) {
#ifdef SSA_CHECKED
    SSA_CHECK_ARG(record != nullptr, "checked_oob: record");
    SSA_CHECK_HIP(hipDeviceSynchronize());
    SSA_CHECK_HIP(hipMemcpyFromSymbol(record, HIP_SYMBOL(ssa_oob), sizeof(uint32_t) * 4));
    const uint32_t zero[4] = {0u, 0u, 0u, 0u};
    SSA_CHECK_HIP(hipMemcpyToSymbol(HIP_SYMBOL(ssa_oob), zero, sizeof(zero)));
    return 1;
#else
    (void)record;
    return 0;
#endif
}
