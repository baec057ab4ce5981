// ssa_sort_dev.h -- device side of the bucket sort's top levels (kernel A),
// shared by ssa_sort.hip and by the graph build, which runs the top levels of
// its key sort side by side with the first head chunk's query hash in one
// launch.  See ssa_sort.hip for the algorithm.
#pragma once
#include <type_traits>

#include "ssa_common.h"

namespace {

constexpr int SORT_THREADS = 1024;
constexpr int SORT_WAVES = SORT_THREADS / SSA_WAVE;
constexpr int LEAF = 16;

// Orders one wavefront's own LDS / global accesses across lanes: wait for all
// outstanding memory operations, then fence at wavefront scope.
__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ int floor_log2_i(int n) { return 31 - __clz(n); }

// ---- heap sort of [f, l) by key, one lane (rare: only at the depth limit)
template <typename Pos>
__device__ void heap_push_up(uint16_t *key, Pos *idx, int base, int hole, int top,
                             uint16_t vk, Pos vi) {
    int parent = (hole - 1) / 2;
    while (hole > top && key[base + parent] < vk) {
        key[base + hole] = key[base + parent];
        idx[base + hole] = idx[base + parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    key[base + hole] = vk;
    idx[base + hole] = vi;
}

template <typename Pos>
__device__ void heap_adjust(uint16_t *key, Pos *idx, int base, int hole, int len,
                            uint16_t vk, Pos vi) {
    const int top = hole;
    int child = hole;
    while (child < (len - 1) / 2) {
        child = 2 * (child + 1);
        if (key[base + child] < key[base + child - 1]) child--;
        key[base + hole] = key[base + child];
        idx[base + hole] = idx[base + child];
        hole = child;
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
        child = 2 * (child + 1);
        key[base + hole] = key[base + child - 1];
        idx[base + hole] = idx[base + child - 1];
        hole = child - 1;
    }
    heap_push_up(key, idx, base, hole, top, vk, vi);
}

template <typename Pos>
__device__ void heap_sort_range(uint16_t *key, Pos *idx, int f, int l) {
    const int len = l - f;
    if (len < 2) return;
    for (int parent = (len - 2) / 2;; --parent) {
        heap_adjust(key, idx, f, parent, len, key[f + parent], idx[f + parent]);
        if (parent == 0) break;
    }
    for (int last = len - 1; last > 0; --last) {
        const uint16_t vk = key[f + last];
        const Pos vi = idx[f + last];
        key[f + last] = key[f];
        idx[f + last] = idx[f];
        heap_adjust(key, idx, f, 0, last, vk, vi);
    }
}

// ---- one wavefront partitions [f, l); returns the cut
template <typename Pos>
__device__ int wave_partition(uint16_t *key, Pos *idx, Pos *TL, Pos *TR, int f, int l) {
    const int lane = lane_id();
    const int n = l - f;
    const int a = f + 1, b = f + n / 2, c = l - 1;
    const int ka = key[a], kb = key[b], kc = key[c];
    int x, p;
    if (ka < kb) {
        if (kb < kc) { x = b; p = kb; }
        else if (ka < kc) { x = c; p = kc; }
        else { x = a; p = ka; }
    } else if (ka < kc) { x = a; p = ka; }
    else if (kb < kc) { x = c; p = kc; }
    else { x = b; p = kb; }
    if (lane == 0) {
        const uint16_t tk = key[f];
        const Pos ti = idx[f];
        key[f] = key[x]; idx[f] = idx[x];
        key[x] = tk; idx[x] = ti;
    }
    wave_sync_lds();

    int numL = 0, numR = 0;
    for (int base = f; base < l; base += SSA_WAVE) {
        const int i = base + lane;
        const bool in = i < l;
        const int kv = in ? (int)key[i] : 0;
        const bool isL = in && i > f && kv >= p;
        const bool isR = in && kv <= p;
        const uint64_t bL = wave_ballot(isL), bR = wave_ballot(isR);
        if (isL) TL[f + numL + lanes_below(bL)] = (Pos)i;
        if (isR) TR[f + numR + lanes_below(bR)] = (Pos)i;
        numL += __popcll(bL);
        numR += __popcll(bR);
    }
    wave_sync_lds();

    // s = number of k (1-based) with L_k < R_k, where R_k = TR[numR - k]
    const int s = hoare_swap_count(TL, TR, f, numL, numR);
    for (int k0 = 0; k0 < s; k0 += SSA_WAVE) {
        const int k = k0 + lane;
        if (k < s) {
            const int pa = TL[f + k], pb = TR[f + numR - 1 - k];
            const uint16_t tk = key[pa];
            const Pos ti = idx[pa];
            key[pa] = key[pb]; idx[pa] = idx[pb];
            key[pb] = tk; idx[pb] = ti;
        }
    }
    int cut = 0x7fffffff;
    if (s < numL) cut = TL[f + s];
    if (s > 0) { const int r = TR[f + numR - s]; cut = r < cut ? r : cut; }
    wave_sync_lds();
    return cut;
}

// index of the k-th (0-based) set bit of a 32 / 64-bit mask (k < popcount)
__device__ __forceinline__ int nth_set_bit32(uint32_t b, int k) {
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
__device__ __forceinline__ int nth_set_bit64(uint64_t m, int k) {
    const int c = __popc((uint32_t)m);
    const bool up = k >= c;
    return (up ? 32 : 0) + nth_set_bit32(up ? (uint32_t)(m >> 32) : (uint32_t)m, up ? k - c : k);
}

// The whole introsort subtree of a segment of at most 64 keys, in one
// wavefront's registers (lane i holds position f + i).  Each partition is the
// same median-of-three + Hoare scan as wave_partition, computed with ballots:
// L_k / R_k are the k-th set bits of the stopper masks (from the bottom / the
// top), every lane finds its swap partner with one shuffle, and the cut is
// read from lane s.  Pending segments are bits of a mask (segment starts), so
// the order in which independent segments are split does not matter.
template <typename Pos>
__device__ void wave_small_sort(uint16_t *key, Pos *idx, uint32_t *bits, int f, int n,
                                int depth0) {
    const int lane = lane_id();
    int kv = lane < n ? (int)key[f + lane] : 0;
    int xv = lane < n ? (int)idx[f + lane] : 0;
    int dep = lane == 0 ? depth0 : 0;          // depth of the segment starting at this lane
    uint64_t bnd = 1ull;                       // segment starts
    uint64_t pend = n > LEAF ? 1ull : 0ull;    // starts of segments still to split
    while (pend) {
        const int a = __ffsll((long long)pend) - 1;
        pend &= pend - 1ull;
        const uint64_t above = bnd & ~((2ull << a) - 1ull);
        const int b = above ? __ffsll((long long)above) - 1 : n;
        const int d = __builtin_amdgcn_readlane(dep, a);
        if (d == 0) {                          // depth limit: heap sort through LDS
            if (lane < n) { key[f + lane] = (uint16_t)kv; idx[f + lane] = (Pos)xv; }
            wave_sync_lds();
            if (lane == 0) heap_sort_range(key, idx, f + a, f + b);
            wave_sync_lds();
            if (lane < n) { kv = key[f + lane]; xv = idx[f + lane]; }
            continue;
        }
        const int m = b - a;
        const int ia = a + 1, ib = a + m / 2, ic = b - 1;
        const int ka = __builtin_amdgcn_readlane(kv, ia), kb = __builtin_amdgcn_readlane(kv, ib),
                  kc = __builtin_amdgcn_readlane(kv, ic);
        int x, p;
        if (ka < kb) {
            if (kb < kc) { x = ib; p = kb; }
            else if (ka < kc) { x = ic; p = kc; }
            else { x = ia; p = ka; }
        } else if (ka < kc) { x = ia; p = ka; }
        else if (kb < kc) { x = ic; p = kc; }
        else { x = ib; p = kb; }
        {                                       // pivot to the front
            const int kx = __builtin_amdgcn_readlane(kv, x), xx = __builtin_amdgcn_readlane(xv, x);
            const int k0 = __builtin_amdgcn_readlane(kv, a), x0 = __builtin_amdgcn_readlane(xv, a);
            if (lane == a) { kv = kx; xv = xx; }
            else if (lane == x) { kv = k0; xv = x0; }
        }
        const bool in = lane >= a && lane < b;
        const uint64_t bL = wave_ballot(in && lane > a && kv >= p);
        const uint64_t bR = wave_ballot(in && kv <= p);
        const int nL = __popcll(bL), nR = __popcll(bR);
        const int Lj = nth_set_bit64(bL, lane);                                   // lane < nL
        const int Rj = 63 - nth_set_bit64(__builtin_bitreverse64(bR), lane);      // lane < nR
        const int mn = nL < nR ? nL : nR;
        const int sw = __popcll(wave_ballot(lane < mn && Lj < Rj));               // a prefix
        const int rl = lanes_below(bL);
        const int rr = __popcll(bR & ~((2ull << lane) - 1ull));
        const int tR = __shfl(Rj, rl, SSA_WAVE);   // R_rl
        const int tL = __shfl(Lj, rr, SSA_WAVE);   // L_rr
        int partner = lane;
        if (((bL >> lane) & 1ull) && rl < sw) partner = tR;
        else if (((bR >> lane) & 1ull) && rr < sw) partner = tL;
        kv = __shfl(kv, partner, SSA_WAVE);
        xv = __shfl(xv, partner, SSA_WAVE);
        const int cL = sw < nL ? __builtin_amdgcn_readlane(Lj, sw) : 0x7fffffff;
        const int cR = sw > 0 ? __builtin_amdgcn_readlane(Rj, sw - 1) : 0x7fffffff;
        const int c = cL < cR ? cL : cR;
        if (lane == 0) atomicOr(&bits[(f + c) >> 5], 1u << ((f + c) & 31));
        bnd |= 1ull << c;
        dep = (lane == a || lane == c) ? d - 1 : dep;
        if (c - a > LEAF) pend |= 1ull << a;
        if (b - c > LEAF) pend |= 1ull << c;
    }
    if (lane < n) { key[f + lane] = (uint16_t)kv; idx[f + lane] = (Pos)xv; }
    wave_sync_lds();
}

// ---------------------------------------------------------------- top levels
// Kernel A, one workgroup of SORT_WAVES waves per row: loads the row, writes the
// bucket tables from a histogram (bstart[u] = #keys < u, bsize[u] = #keys
// == u: what binary searches on the sorted row give), and splits segments
// larger than SEG_T.  While a level has few segments, the waves of a group
// cooperate on one segment (each wave finds the stoppers of its stretch; the
// stopper lists are concatenated by prefix counts); with many segments each
// wave partitions its own.  Children of at most SEG_T keys (and leaves) are
// appended to a global segment list for kernel B, and the row as it stands
// (keys | ids << 16) is written out; so is `perm`, which kernel B overwrites
// for every listed segment (a segment heap-sorted here keeps these values).
constexpr int SEG_T = 256;                 // segments handed to kernel B
constexpr int SORT_NW = SORT_WAVES;
// A row's segments for kernel B are gathered in LDS (up to SEG_STAGE of them)
// and appended to the global list with one atomic per row at the end: a
// device-scope atomic on the list's one counter per segment made the top
// levels 10% slower.  Segments past SEG_STAGE take that atomic each.
constexpr int SEG_STAGE = 256;
// dynamic LDS of kernel A: the static TopShared below takes the rest
constexpr int SORT_LDS_BYTES = SSA_LDS_BYTES - SEG_STAGE * 16;

struct TopShared {
    int ncur, nnxt, nseg, base;
    int piv[SORT_NW], cnt[SORT_NW][2], s[SORT_NW], cut[SORT_NW], nL[SORT_NW], nR[SORT_NW];
    int4 stage[SEG_STAGE];
};

__device__ __forceinline__ void emit_segment(TopShared &sh, int4 *segs, int *segcount, int row,
                                             int f, int l, int depth) {
    const int4 e = make_int4(row, f, l - f, depth);
    const int k = atomicAdd(&sh.nseg, 1);
    if (k < SEG_STAGE) sh.stage[k] = e;
    else segs[atomicAdd(segcount, 1)] = e;
}

// Pos: uint16_t (rows of up to 32768 keys, the row in LDS) or uint32_t (longer
// rows: keys, positions and stopper lists in `glb`, per row 2 + 3 * 4 bytes
// per key).  A segment word holds f | l << (8 * sizeof(Pos)).
// workspace bytes of one row beyond LDS: positions, stopper lists, keys
__host__ __device__ inline int64_t sort_glb_row_bytes(int n) {
    return ((int64_t)n * 14 + 15) / 16 * 16;
}

template <typename Pos> struct SortWords {
    using W = typename std::conditional<sizeof(Pos) == 2, uint32_t, uint64_t>::type;
    static constexpr int SH = 8 * (int)sizeof(Pos);
};

// One workgroup of SORT_THREADS threads sorts row `row` (the body of kernel A;
// smem_raw is the dynamic LDS sort_plan sizes, sh the workgroup's shared
// state).  Every thread of the workgroup calls it.
template <typename Pos>
__device__ void sort_top_row(int row, const uint16_t *ids, int n, int NB, int32_t *perm,
                             int32_t *bstart, int32_t *bsize, typename SortWords<Pos>::W *gkv,
                             int4 *segs, int *segcount, unsigned char *glb, int tl_in_lds, int cap,
                             unsigned char *smem_raw, TopShared &sh) {
    using W = typename SortWords<Pos>::W;
    constexpr int SH = SortWords<Pos>::SH;
    constexpr bool GLB = sizeof(Pos) == 4;
    const int tid = threadIdx.x;
    const int wid = tid / SSA_WAVE;
    const int lane = lane_id();
    const uint16_t *src = ids + (int64_t)row * n;

    uint16_t *key;
    Pos *idx, *TL, *TR;
    int32_t *hist;
    if (GLB) {
        unsigned char *g = glb + (int64_t)row * sort_glb_row_bytes(n);
        idx = (Pos *)g;
        TL = idx + n;
        TR = TL + n;
        key = (uint16_t *)(TR + n);
        hist = (int32_t *)smem_raw;
    } else {
        key = (uint16_t *)smem_raw;
        idx = (Pos *)(key + n);
        hist = (int32_t *)(smem_raw + ((size_t)4 * n + 15) / 16 * 16);
    }
    W *segA = (W *)(hist + NB);
    W *segB = segA + cap;
    uint8_t *depA = (uint8_t *)(segB + cap);
    uint8_t *depB = depA + cap;
    if (!GLB) {
        if (tl_in_lds) {
            const size_t off = ((size_t)((unsigned char *)(depB + cap) - smem_raw) + 15) / 16 * 16;
            TL = (Pos *)(smem_raw + off);
        } else {
            TL = (Pos *)glb + (int64_t)row * 2 * n;
        }
        TR = TL + n;
    }

    for (int u = tid; u < NB; u += SORT_THREADS) hist[u] = 0;
    __syncthreads();
    for (int i = tid; i < n; i += SORT_THREADS) {
        const uint16_t k = src[i];
        key[i] = k;
        idx[i] = (Pos)i;
        if (k < NB) atomicAdd(&hist[k], 1);
    }
    const int depth0 = 2 * floor_log2_i(n);
    if (tid == 0) {
        sh.ncur = 0;
        sh.nnxt = 0;
        sh.nseg = 0;
        if (n > SEG_T) {
            segA[0] = (W)n << SH;
            depA[0] = (uint8_t)depth0;
            sh.ncur = 1;
        } else {
            emit_segment(sh, segs, segcount, row, 0, n, depth0);
        }
    }
    __syncthreads();
    if (wid == 0) {                                // bucket tables: exclusive scan of hist
        int carry = 0;
        for (int u0 = 0; u0 < NB; u0 += SSA_WAVE) {
            const int u = u0 + lane;
            const int c = u < NB ? hist[u] : 0;
            int x = c;
#pragma unroll
            for (int o = 1; o < SSA_WAVE; o <<= 1) {
                const int y = __shfl_up(x, o, SSA_WAVE);
                if (lane >= o) x += y;
            }
            if (u < NB) {
                bstart[(int64_t)row * NB + u] = carry + x - c;
                bsize[(int64_t)row * NB + u] = c;
            }
            carry += __shfl(x, SSA_WAVE - 1, SSA_WAVE);
        }
    }

    W *cur = segA, *nxt = segB;
    uint8_t *dcur = depA, *dnxt = depB;
    constexpr W LOW = ((W)1 << SH) - 1;
    auto child = [&](int f, int l, int depth) {
        if (l - f > SEG_T) {
            const int slot = atomicAdd(&sh.nnxt, 1);
            nxt[slot] = (W)f | ((W)l << SH);
            dnxt[slot] = (uint8_t)depth;
        } else {
            emit_segment(sh, segs, segcount, row, f, l, depth);
        }
    };
    for (int level = 0; level < 64; ++level) {
        __syncthreads();
        const int ncur = sh.ncur;
        if (ncur == 0) break;
        if (2 * ncur <= SORT_NW) {
            // ---- group mode: gw waves per segment, gi = index in the group
            const int gw = SORT_NW / ncur;
            const int g = wid / gw, gi = wid - g * gw;
            const bool act = g < ncur;
            int f = 0, l = 0, depth = 1;
            if (act) {
                f = (int)(cur[g] & LOW);
                l = (int)(cur[g] >> SH);
                depth = dcur[g];
            }
            // a segment at the depth limit is heap-sorted by its group's first lane
            if (act && depth == 0) {
                if (gi == 0 && lane == 0) heap_sort_range(key, idx, f, l);
            } else if (act && gi == 0) {               // median of three to the front
                const int nn = l - f;
                const int a = f + 1, b = f + nn / 2, c = l - 1;
                const int ka = key[a], kb = key[b], kc = key[c];
                int x, p;
                if (ka < kb) {
                    if (kb < kc) { x = b; p = kb; }
                    else if (ka < kc) { x = c; p = kc; }
                    else { x = a; p = ka; }
                } else if (ka < kc) { x = a; p = ka; }
                else if (kb < kc) { x = c; p = kc; }
                else { x = b; p = kb; }
                if (lane == 0) {
                    const uint16_t tk = key[f];
                    const Pos ti = idx[f];
                    key[f] = key[x]; idx[f] = idx[x];
                    key[x] = tk; idx[x] = ti;
                    sh.piv[g] = p;
                }
            }
            __syncthreads();
            const bool part = act && depth > 0;
            // stretch of this wave: [f + gi*per, ...), per a multiple of 64
            const int per = part ? ((l - f + gw - 1) / gw + SSA_WAVE - 1) / SSA_WAVE * SSA_WAVE : 0;
            const int s0 = f + gi * per, s1 = min(s0 + per, l);
            const int p = part ? sh.piv[g] : 0;
            if (part) {
                int cL = 0, cR = 0;
                for (int base = s0; base < s1; base += SSA_WAVE) {
                    const int i = base + lane;
                    const bool in = i < s1;
                    const int kv = in ? (int)key[i] : 0;
                    cL += __popcll(wave_ballot(in && i > f && kv >= p));
                    cR += __popcll(wave_ballot(in && kv <= p));
                }
                if (lane == 0) { sh.cnt[wid][0] = cL; sh.cnt[wid][1] = cR; }
            }
            __syncthreads();
            if (part) {
                int oL = 0, oR = 0, tL = 0, tR = 0;
                for (int w = 0; w < gw; ++w) {
                    const int cl = sh.cnt[g * gw + w][0], cr = sh.cnt[g * gw + w][1];
                    if (w < gi) { oL += cl; oR += cr; }
                    tL += cl;
                    tR += cr;
                }
                int numL = oL, numR = oR;
                for (int base = s0; base < s1; base += SSA_WAVE) {
                    const int i = base + lane;
                    const bool in = i < s1;
                    const int kv = in ? (int)key[i] : 0;
                    const bool isL = in && i > f && kv >= p;
                    const bool isR = in && kv <= p;
                    const uint64_t bL = wave_ballot(isL), bR = wave_ballot(isR);
                    if (isL) TL[f + numL + lanes_below(bL)] = (Pos)i;
                    if (isR) TR[f + numR + lanes_below(bR)] = (Pos)i;
                    numL += __popcll(bL);
                    numR += __popcll(bR);
                }
                if (gi == 0 && lane == 0) { sh.nL[g] = tL; sh.nR[g] = tR; }
            }
            __syncthreads();
            if (part && gi == 0) {                    // s = #k with L_k < R_k
                const int numL = sh.nL[g], numR = sh.nR[g];
                const int lo = hoare_swap_count(TL, TR, f, numL, numR);
                int cut = 0x7fffffff;
                if (lo < numL) cut = TL[f + lo];
                if (lo > 0) { const int r = TR[f + numR - lo]; cut = r < cut ? r : cut; }
                if (lane == 0) { sh.s[g] = lo; sh.cut[g] = cut; }
            }
            __syncthreads();
            if (part) {
                const int sw = sh.s[g], numR = sh.nR[g];
                for (int k = gi * SSA_WAVE + lane; k < sw; k += gw * SSA_WAVE) {
                    const int pa = TL[f + k], pb = TR[f + numR - 1 - k];
                    const uint16_t tk = key[pa];
                    const Pos ti = idx[pa];
                    key[pa] = key[pb]; idx[pa] = idx[pb];
                    key[pb] = tk; idx[pb] = ti;
                }
                if (gi == 0 && lane == 0) {
                    const int cut = sh.cut[g];
                    child(f, cut, depth - 1);
                    child(cut, l, depth - 1);
                }
            }
        } else {
            // ---- wave mode: one wave per segment
            for (int sgi = wid; sgi < ncur; sgi += SORT_NW) {
                const int f = (int)(cur[sgi] & LOW);
                const int l = (int)(cur[sgi] >> SH);
                const int depth = dcur[sgi];
                if (depth == 0) {
                    if (lane == 0) heap_sort_range(key, idx, f, l);
                    wave_sync_lds();
                    continue;
                }
                const int cut = wave_partition(key, idx, TL, TR, f, l);
                if (lane == 0) {
                    child(f, cut, depth - 1);
                    child(cut, l, depth - 1);
                }
            }
        }
        __syncthreads();
        if (tid == 0) { sh.ncur = sh.nnxt; sh.nnxt = 0; }
        W *t = cur; cur = nxt; nxt = t;
        uint8_t *td = dcur; dcur = dnxt; dnxt = td;
    }
    __syncthreads();
    // the gathered segments into the global list, one atomic for all of them
    const int ns = min(sh.nseg, SEG_STAGE);
    if (tid == 0 && ns > 0) sh.base = atomicAdd(segcount, ns);
    W *okv = gkv + (int64_t)row * n;
    int32_t *pout = perm + (int64_t)row * n;
    for (int i = tid; i < n; i += SORT_THREADS) {
        okv[i] = (W)key[i] | ((W)idx[i] << SH);
        pout[i] = (int32_t)idx[i];
    }
    __syncthreads();
    for (int i = tid; i < ns; i += SORT_THREADS) segs[sh.base + i] = sh.stage[i];
}

// ---------------------------------------------------------------- segments
// Kernel B, one wavefront per listed segment (<= SEG_T keys), anywhere on the
// chip: the segment's remaining introsort subtree (wave partitions above 64
// keys, the register path below), then the final insertion sort of each leaf
// (one leaf per lane; partitions leave max(left) <= min(right), so this equals
// the reference's final insertion pass over the row), and its slice of perm.
constexpr int SEG_WAVES = 4;
constexpr int SEG_STACK = SEG_T / (LEAF + 1) + 2;
constexpr int SEG_PER_LANE = SEG_T / SSA_WAVE;

// A segment whose keys are all equal: libstdc++'s partitions then depend on
// its length alone.  The median of three (first + 1, middle, last - 1) is the
// middle element, moved to the front; the unguarded scan stops at every
// element, so it swaps positions k and n - k for 1 <= k < n / 2 and cuts at
// ceil(n / 2); both halves recurse the same way down to leaves of LEAF, whose
// insertion sort moves nothing.  So an element's final slot follows from its
// position in O(log n) steps, and the subtree is one permutation.
__device__ __forceinline__ int eq_final_pos(int n, int i) {
    int base = 0;
    while (n > LEAF) {
        const int h = n >> 1;
        i = i == 0 ? h : (i == h ? 0 : i);
        if (i != 0 && 2 * i != n) i = n - i;
        const int c = (n + 1) >> 1;
        if (i < c) {
            n = c;
        } else {
            base += c;
            i -= c;
            n -= c;
        }
    }
    return base + i;
}
// partition levels the closed form takes (the larger half each time): the
// subtree reaches no depth limit when the segment's depth is at least this
__device__ __forceinline__ int eq_levels(int n) {
    int l = 0;
    for (; n > LEAF; n = (n + 1) >> 1) ++l;
    return l;
}

template <typename Pos>
__host__ __device__ constexpr int seg_lds_words() {
    // key (u16), idx, TL, TR (Pos) x SEG_T each, bits, stack
    return (SEG_T * (2 + 3 * (int)sizeof(Pos))) / 4 + (SEG_T / 32 + 1) + 2 * SEG_STACK;
}

// The body of kernel B for workgroup `block` of `nblocks` (SEG_WAVES waves
// each); lds: SEG_WAVES * seg_lds_words<Pos>() words of the workgroup's LDS.
template <typename Pos>
__device__ void sort_seg_blocks(const typename SortWords<Pos>::W *gkv, int n, const int4 *segs,
                                const int *segcount, int32_t *perm, uint32_t *lds, int block,
                                int nblocks) {
    using W = typename SortWords<Pos>::W;
    constexpr int SH = SortWords<Pos>::SH;
    const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x / SSA_WAVE);
    const int lane = lane_id();
    uint32_t *w0 = lds + wid * seg_lds_words<Pos>();
    Pos *idx = (Pos *)w0;
    Pos *TL = idx + SEG_T;
    Pos *TR = TL + SEG_T;
    uint16_t *key = (uint16_t *)(TR + SEG_T);
    uint32_t *bits = (uint32_t *)(key + SEG_T);
    uint32_t *stk = bits + (SEG_T / 32 + 1);
    uint32_t *sdep = stk + SEG_STACK;
    const int count = *segcount;
    const int stride = nblocks * SEG_WAVES;
    for (int sgi = block * SEG_WAVES + wid; sgi < count; sgi += stride) {
        const int4 e = segs[sgi];
        const int row = e.x, f0 = e.y, m = e.z, depth0 = e.w;
        const W *src = gkv + (int64_t)row * n + f0;
        int32_t *pout = perm + (int64_t)row * n + f0;
        W rv[SEG_PER_LANE];
        uint32_t kmin = 0xffffu, kmax = 0u;
#pragma unroll
        for (int u = 0; u < SEG_PER_LANE; ++u) {
            const int i = lane + SSA_WAVE * u;
            rv[u] = src[min(i, m - 1)];
            const uint32_t k = (uint32_t)(rv[u] & 0xffffu);
            kmin = min(kmin, k);
            kmax = max(kmax, k);
        }
        if (wave_min_u(kmin) == wave_max_u(kmax) && depth0 >= eq_levels(m)) {
            // every key equal: the segment's permutation in closed form
#pragma unroll
            for (int u = 0; u < SEG_PER_LANE; ++u) {
                const int i = lane + SSA_WAVE * u;
                if (i < m) pout[eq_final_pos(m, i)] = (int32_t)(Pos)(rv[u] >> SH);
            }
            continue;
        }
#pragma unroll
        for (int u = 0; u < SEG_PER_LANE; ++u) {
            const int i = lane + SSA_WAVE * u;
            if (i < m) {
                key[i] = (uint16_t)(rv[u] & 0xffffu);
                idx[i] = (Pos)(rv[u] >> SH);
            }
        }
        for (int w = lane; w < SEG_T / 32 + 1; w += SSA_WAVE) bits[w] = w == 0 ? 1u : 0u;
        wave_sync_lds();
        if (m > LEAF) {
            int top = 1;
            if (lane == 0) { stk[0] = (uint32_t)m << 16; sdep[0] = (uint32_t)depth0; }
            wave_sync_lds();
            while (top > 0) {
                --top;
                const uint32_t se = stk[top];
                const int a = (int)(se & 0xffffu), b = (int)(se >> 16);
                const int d = (int)sdep[top];
                wave_sync_lds();
                {
                    // a sub-segment whose keys are all equal: its subtree in
                    // closed form, each slot then a leaf of its own
                    uint32_t smin = 0xffffu, smax = 0u;
#pragma unroll
                    for (int u = 0; u < SEG_PER_LANE; ++u) {
                        const int i = a + lane + SSA_WAVE * u;
                        if (i < b) {
                            const uint32_t k = key[i];
                            smin = min(smin, k);
                            smax = max(smax, k);
                        }
                    }
                    if (wave_min_u(smin) == wave_max_u(smax) && d >= eq_levels(b - a)) {
                        Pos iv[SEG_PER_LANE];
#pragma unroll
                        for (int u = 0; u < SEG_PER_LANE; ++u) {
                            const int i = a + lane + SSA_WAVE * u;
                            iv[u] = i < b ? idx[i] : (Pos)0;
                        }
                        wave_sync_lds();
#pragma unroll
                        for (int u = 0; u < SEG_PER_LANE; ++u) {
                            const int i = lane + SSA_WAVE * u;
                            if (a + i < b) {
                                idx[a + eq_final_pos(b - a, i)] = iv[u];
                                atomicOr(&bits[(a + i) >> 5], 1u << ((a + i) & 31));
                            }
                        }
                        wave_sync_lds();
                        continue;
                    }
                }
                if (d == 0) {
                    if (lane == 0) heap_sort_range(key, idx, a, b);
                    wave_sync_lds();
                    continue;
                }
                if (b - a <= SSA_WAVE) {
                    wave_small_sort(key, idx, bits, a, b - a, d);
                    continue;
                }
                const int cut = wave_partition(key, idx, TL, TR, a, b);
                if (lane == 0) {
                    atomicOr(&bits[cut >> 5], 1u << (cut & 31));
                    if (cut - a > LEAF) { stk[top] = (uint32_t)a | ((uint32_t)cut << 16); sdep[top] = d - 1; }
                }
                if (cut - a > LEAF) ++top;
                if (lane == 0 && b - cut > LEAF) {
                    stk[top] = (uint32_t)cut | ((uint32_t)b << 16);
                    sdep[top] = d - 1;
                }
                if (b - cut > LEAF) ++top;
                wave_sync_lds();
            }
        }
        // final insertion sort, one leaf per lane
        for (int s0 = lane; s0 < m; s0 += SSA_WAVE) {
            if (!((bits[s0 >> 5] >> (s0 & 31)) & 1u)) continue;
            int e1 = s0 + 1;
            while (e1 < m && !((bits[e1 >> 5] >> (e1 & 31)) & 1u)) ++e1;
            for (int i = s0 + 1; i < e1; ++i) {
                const uint16_t vk = key[i];
                const Pos vi = idx[i];
                int j = i;
                while (j > s0 && key[j - 1] > vk) {
                    key[j] = key[j - 1];
                    idx[j] = idx[j - 1];
                    --j;
                }
                key[j] = vk;
                idx[j] = vi;
            }
        }
        wave_sync_lds();
        for (int i = lane; i < m; i += SSA_WAVE) pout[i] = (int32_t)idx[i];
        wave_sync_lds();
    }
}

}  // namespace
