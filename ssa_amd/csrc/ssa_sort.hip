// ssa_sort.hip -- bucket permutation identical to torch.sort(ids, dim=-1) on the CPU.
//
// The reference sorts each row of bucket ids with torch.sort(stable=False)
// (sparse_attention.py:781), which on the CPU is libstdc++'s introsort over
// (key, position) pairs compared on the key only.  The candidate lists take
// the FIRST C members of a bucket in that order, so the permutation itself,
// not just the sortedness, must be reproduced.
//
// Introsort as a data-parallel program (one workgroup per row):
//   * the recursion is run level by level; every active segment [f, l) with
//     l - f > 16 is partitioned by one wavefront;
//   * partition = median-of-three (first+1, middle, last-1) moved to f, then
//     the unguarded Hoare scan.  The scan's swaps are fixed by the ORIGINAL
//     array: with L_k the k-th position in (f, l) holding key >= p (ascending)
//     and R_k the k-th position in [f, l) holding key <= p (descending), the
//     scan swaps (L_k, R_k) for every k with L_k < R_k (a prefix k <= s) and
//     stops at cut = min(L_{s+1}, R_s).  A wave finds the stoppers with
//     ballots, s by a 64-ary search, then performs all s swaps in parallel;
//   * both children inherit depth - 1; a segment reaching depth 0 is heap-
//     sorted by one lane (the depth limit is 2*floor(log2 n));
//   * a segment of at most 64 elements is finished (down to its leaves) by one
//     wavefront in registers;
//   * segments of <= 16 elements are left for the final insertion sort.
//     Because every partition leaves max(left) <= min(right), that final pass
//     equals a stable insertion sort inside each leaf, done one leaf per thread.
// The bucket start/size tables come from binary searches on the sorted keys.
//
// Rows of up to 32768 keys keep keys and 16-bit positions in LDS.  Longer rows
// (up to SORT_MAX_KEYS) run the same program with 32-bit positions and the
// row's keys, positions and stopper lists in the workspace (the top levels'
// memory traffic then goes to the L2 / HBM instead of LDS); kernel B's
// segments stay in LDS either way.
#include <algorithm>
#include <type_traits>

#include "ssa_common.h"
#include "ssa_graph_internal.h"

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
// Kernel A, one workgroup of NW waves per row: loads the row, writes the
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
constexpr int NW = SORT_WAVES;

struct TopShared {
    int ncur, nnxt;
    int piv[NW], cnt[NW][2], s[NW], cut[NW], nL[NW], nR[NW];
};

__device__ __forceinline__ void emit_segment(int4 *segs, int *segcount, int row, int f, int l,
                                             int depth) {
    segs[atomicAdd(segcount, 1)] = make_int4(row, f, l - f, depth);
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

template <typename Pos>
__global__ void __launch_bounds__(SORT_THREADS)
sort_top_kernel(const uint16_t *ids, int n, int NB, int32_t *perm, int32_t *bstart, int32_t *bsize,
                typename SortWords<Pos>::W *gkv, int4 *segs, int *segcount, unsigned char *glb,
                int tl_in_lds, int cap) {
    using W = typename SortWords<Pos>::W;
    constexpr int SH = SortWords<Pos>::SH;
    constexpr bool GLB = sizeof(Pos) == 4;
    extern __shared__ __align__(16) unsigned char smem_raw[];
    __shared__ TopShared sh;
    const int row = blockIdx.x;
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
        if (n > SEG_T) {
            segA[0] = (W)n << SH;
            depA[0] = (uint8_t)depth0;
            sh.ncur = 1;
        } else {
            emit_segment(segs, segcount, row, 0, n, depth0);
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
            emit_segment(segs, segcount, row, f, l, depth);
        }
    };
    for (int level = 0; level < 64; ++level) {
        __syncthreads();
        const int ncur = sh.ncur;
        if (ncur == 0) break;
        if (2 * ncur <= NW) {
            // ---- group mode: gw waves per segment, gi = index in the group
            const int gw = NW / ncur;
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
            for (int sgi = wid; sgi < ncur; sgi += NW) {
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
    W *okv = gkv + (int64_t)row * n;
    int32_t *pout = perm + (int64_t)row * n;
    for (int i = tid; i < n; i += SORT_THREADS) {
        okv[i] = (W)key[i] | ((W)idx[i] << SH);
        pout[i] = (int32_t)idx[i];
    }
}

// ---------------------------------------------------------------- segments
// Kernel B, one wavefront per listed segment (<= SEG_T keys), anywhere on the
// chip: the segment's remaining introsort subtree (wave partitions above 64
// keys, the register path below), then the final insertion sort of each leaf
// (one leaf per lane; partitions leave max(left) <= min(right), so this equals
// the reference's final insertion pass over the row), and its slice of perm.
constexpr int SEG_WAVES = 4;
constexpr int SEG_STACK = SEG_T / (LEAF + 1) + 2;

template <typename Pos>
__host__ __device__ constexpr int seg_lds_words() {
    // key (u16), idx, TL, TR (Pos) x SEG_T each, bits, stack
    return (SEG_T * (2 + 3 * (int)sizeof(Pos))) / 4 + (SEG_T / 32 + 1) + 2 * SEG_STACK;
}

template <typename Pos>
__global__ void __launch_bounds__(SEG_WAVES * SSA_WAVE)
sort_seg_kernel(const typename SortWords<Pos>::W *gkv, int n, const int4 *segs,
                const int *segcount, int32_t *perm) {
    using W = typename SortWords<Pos>::W;
    constexpr int SH = SortWords<Pos>::SH;
    __shared__ uint32_t lds[SEG_WAVES * seg_lds_words<Pos>()];
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
    const int stride = (int)gridDim.x * SEG_WAVES;
    for (int sgi = (int)blockIdx.x * SEG_WAVES + wid; sgi < count; sgi += stride) {
        const int4 e = segs[sgi];
        const int row = e.x, f0 = e.y, m = e.z, depth0 = e.w;
        const W *src = gkv + (int64_t)row * n + f0;
        for (int i = lane; i < m; i += SSA_WAVE) {
            const W v = src[i];
            key[i] = (uint16_t)(v & 0xffffu);
            idx[i] = (Pos)(v >> SH);
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
        int32_t *pout = perm + (int64_t)row * n + f0;
        for (int i = lane; i < m; i += SSA_WAVE) pout[i] = (int32_t)idx[i];
        wave_sync_lds();
    }
}

__global__ void sort_zero_kernel(int *p) {
    if (threadIdx.x == 0) *p = 0;
}

}  // namespace

// Rows longer than this keep their keys and positions in the workspace
constexpr int SORT_LDS_KEYS = 32768;
// ... up to this many keys (kernel A's segment lists stay in LDS)
constexpr int SORT_MAX_KEYS = 1 << 20;

// LDS plan of kernel A for a row of n keys and NB buckets
static void sort_plan(int n, int NB, int *cap, int *tl_in_lds, size_t *lds) {
    const int c = n / (SEG_T + 1) + 2;
    *cap = c;
    if (n > SORT_LDS_KEYS) {                   // hist and 64-bit segment words only
        *tl_in_lds = 0;
        *lds = (size_t)NB * 4 + (size_t)c * 16 + (size_t)c * 2;
        return;
    }
    const size_t base = ((size_t)4 * n + 15) / 16 * 16 + (size_t)NB * 4 + (size_t)c * 8 +
                        (size_t)c * 2;
    const size_t with_tl = (base + 15) / 16 * 16 + (size_t)4 * n;
    if (with_tl <= SSA_LDS_BYTES) { *tl_in_lds = 1; *lds = with_tl; }
    else { *tl_in_lds = 0; *lds = base; }
}

// scratch: the rows after kernel A (4 B per key, 8 beyond LDS), the segment
// list (16 B per key at most), its counter, and the stopper lists when they do
// not fit LDS (beyond LDS: the rows' keys, positions and stopper lists)
static int64_t al256(int64_t x) { return (x + 255) / 256 * 256; }

static int64_t sort_row_bytes(int n) { return n > SORT_LDS_KEYS ? 8 : 4; }

int64_t ssa_sort_tmp_bytes(int rows, int n) {
    int cap, tl;
    size_t lds;
    sort_plan(n, 4096, &cap, &tl, &lds);
    const int64_t rn = (int64_t)rows * n;
    const int64_t rest = n > SORT_LDS_KEYS ? rows * sort_glb_row_bytes(n) : (tl ? 0 : rn * 4);
    return al256(rn * sort_row_bytes(n)) + al256(rn * 16) + 256 + rest;
}

int ssa_sort_supported(int n) {
    int cap, tl;
    size_t lds;
    if (n < 1 || n > SORT_MAX_KEYS) return 0;
    sort_plan(n, 4096, &cap, &tl, &lds);
    return lds <= SSA_LDS_BYTES;
}

int32_t *ssa_sort_counter(uint16_t *tmp, int rows, int n) {
    const int64_t rn = (int64_t)rows * n;
    return (int32_t *)((char *)tmp + al256(rn * sort_row_bytes(n)) + al256(rn * 16));
}

template <typename Pos>
static int launch_sort(const uint16_t *ids, int rows, int n, int NB, int32_t *perm,
                       int32_t *bstart, int32_t *bsize, char *t, hipStream_t st) {
    using W = typename SortWords<Pos>::W;
    int cap, tl;
    size_t lds;
    sort_plan(n, NB, &cap, &tl, &lds);
    const int64_t rn = (int64_t)rows * n;
    W *gkv = (W *)t;
    int4 *segs = (int4 *)(t + al256(rn * (int64_t)sizeof(W)));
    int *segcount = ssa_sort_counter((uint16_t *)t, rows, n);
    unsigned char *glb = (unsigned char *)t + al256(rn * (int64_t)sizeof(W)) + al256(rn * 16) + 256;
    SSA_CHECK_HIP(hipFuncSetAttribute((const void *)sort_top_kernel<Pos>,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL((sort_top_kernel<Pos>), dim3(rows), dim3(SORT_THREADS), lds, st, ids, n, NB,
                       perm, bstart, bsize, gkv, segs, segcount, glb, tl, cap);
    SSA_CHECK_LAUNCH();
    const int64_t waves = std::max<int64_t>(1, std::min<int64_t>(rn / 128, 8192));
    hipLaunchKernelGGL((sort_seg_kernel<Pos>), dim3((unsigned)ceil_div(waves, SEG_WAVES)),
                       dim3(SEG_WAVES * SSA_WAVE), 0, st, gkv, n, segs, segcount, perm);
    SSA_CHECK_LAUNCH();
    return SSA_OK;
}

int ssa_launch_bucket_sort(const uint16_t *ids, int rows, int n, int P, int32_t *perm,
                           int32_t *bstart, int32_t *bsize, uint16_t *tmp, hipStream_t st,
                           bool counter_clear) {
    if (!ssa_sort_supported(n)) {
        ssa_set_error("bucket sort: key length %d unsupported (1..%d)", n, SORT_MAX_KEYS);
        return SSA_E_UNSUP;
    }
    if (rows == 0) return SSA_OK;
    const int NB = 1 << P;
    if (counter_clear) {
        hipLaunchKernelGGL(sort_zero_kernel, dim3(1), dim3(64), 0, st,
                           ssa_sort_counter(tmp, rows, n));
        SSA_CHECK_LAUNCH();
    }
    return n > SORT_LDS_KEYS
               ? launch_sort<uint32_t>(ids, rows, n, NB, perm, bstart, bsize, (char *)tmp, st)
               : launch_sort<uint16_t>(ids, rows, n, NB, perm, bstart, bsize, (char *)tmp, st);
}

extern "C" int64_t ssa_bucket_sort_workspace_bytes(int32_t rows, int32_t n) {
    return ssa_sort_tmp_bytes(rows, n);
}

extern "C" int ssa_bucket_sort(const uint16_t *ids, int32_t rows, int32_t n, int32_t P,
                               int32_t *perm, int32_t *bstart, int32_t *bsize, void *workspace,
                               int64_t workspace_bytes, void *stream) {
    SSA_CHECK_ARG(ids && perm && bstart && bsize, "bucket_sort: null pointer");
    SSA_CHECK_ARG(rows >= 0 && n >= 1, "bucket_sort: bad sizes");
    SSA_CHECK_ARG(P >= 1 && P <= 12, "bucket_sort: P=%d outside 1..12", P);
    const int64_t need = ssa_sort_tmp_bytes(rows, n);
    if (workspace_bytes < need) {
        ssa_set_error("bucket_sort: workspace %lld < %lld bytes", (long long)workspace_bytes,
                      (long long)need);
        return SSA_E_WORKSPACE;
    }
    return ssa_launch_bucket_sort(ids, rows, n, P, perm, bstart, bsize, (uint16_t *)workspace,
                                  (hipStream_t)stream);
}
