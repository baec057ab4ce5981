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
//     ballots, s by binary search, then performs all s swaps in parallel;
//   * both children inherit depth - 1; a segment reaching depth 0 is heap-
//     sorted by one lane (the depth limit is 2*floor(log2 n));
//   * a segment of at most 64 elements is finished (down to its leaves) by one
//     wavefront in registers;
//   * segments of <= 16 elements are left for the final insertion sort.
//     Because every partition leaves max(left) <= min(right), that final pass
//     equals a stable insertion sort inside each leaf, done one leaf per thread.
// The bucket start/size tables come from binary searches on the sorted keys.
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
__device__ void heap_push_up(uint16_t *key, uint16_t *idx, int base, int hole, int top,
                             uint16_t vk, uint16_t vi) {
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

__device__ void heap_adjust(uint16_t *key, uint16_t *idx, int base, int hole, int len,
                            uint16_t vk, uint16_t vi) {
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

__device__ void heap_sort_range(uint16_t *key, uint16_t *idx, int f, int l) {
    const int len = l - f;
    if (len < 2) return;
    for (int parent = (len - 2) / 2;; --parent) {
        heap_adjust(key, idx, f, parent, len, key[f + parent], idx[f + parent]);
        if (parent == 0) break;
    }
    for (int last = len - 1; last > 0; --last) {
        const uint16_t vk = key[f + last], vi = idx[f + last];
        key[f + last] = key[f];
        idx[f + last] = idx[f];
        heap_adjust(key, idx, f, 0, last, vk, vi);
    }
}

// ---- one wavefront partitions [f, l); returns the cut
__device__ int wave_partition(uint16_t *key, uint16_t *idx, uint16_t *TL, uint16_t *TR, int f,
                              int l) {
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
        const uint16_t tk = key[f], ti = idx[f];
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
        if (isL) TL[f + numL + lanes_below(bL)] = (uint16_t)i;
        if (isR) TR[f + numR + lanes_below(bR)] = (uint16_t)i;
        numL += __popcll(bL);
        numR += __popcll(bR);
    }
    wave_sync_lds();

    // s = number of k (1-based) with L_k < R_k, where R_k = TR[numR - k]
    int lo = 0, hi = numL < numR ? numL : numR;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if ((int)TL[f + mid - 1] < (int)TR[f + numR - mid]) lo = mid; else hi = mid - 1;
    }
    const int s = lo;
    for (int k0 = 0; k0 < s; k0 += SSA_WAVE) {
        const int k = k0 + lane;
        if (k < s) {
            const int pa = TL[f + k], pb = TR[f + numR - 1 - k];
            const uint16_t tk = key[pa], ti = idx[pa];
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
__device__ void wave_small_sort(uint16_t *key, uint16_t *idx, uint32_t *bits, int f, int n,
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
            if (lane < n) { key[f + lane] = (uint16_t)kv; idx[f + lane] = (uint16_t)xv; }
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
    if (lane < n) { key[f + lane] = (uint16_t)kv; idx[f + lane] = (uint16_t)xv; }
    wave_sync_lds();
}

struct SortShared {
    int ncur, nnxt;
};

// ids: rows x n (uint16); perm rows x n (int32); bstart/bsize rows x NB.
// tmp: rows x 2n uint16 scratch for the stopper lists when they do not fit LDS.
__global__ void __launch_bounds__(SORT_THREADS)
bucket_sort_kernel(const uint16_t *ids, int n, int NB, int32_t *perm, int32_t *bstart,
                   int32_t *bsize, uint16_t *tmp, int tl_in_lds, int cap) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    __shared__ SortShared sh;
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const int wid = tid / SSA_WAVE;
    const int lane = lane_id();
    const uint16_t *src = ids + (int64_t)row * n;

    // LDS layout
    uint16_t *key = (uint16_t *)smem_raw;
    uint16_t *idx = key + n;
    uint32_t *bits = (uint32_t *)(smem_raw + ((size_t)4 * n + 15) / 16 * 16);
    const int nwords = (n + 31) / 32 + 1;
    uint32_t *segA = bits + nwords;
    uint32_t *segB = segA + cap;
    uint8_t *depA = (uint8_t *)(segB + cap);
    uint8_t *depB = depA + cap;
    uint16_t *TL, *TR;
    if (tl_in_lds) {
        const size_t off = ((size_t)((unsigned char *)(depB + cap) - smem_raw) + 15) / 16 * 16;
        TL = (uint16_t *)(smem_raw + off);
        TR = TL + n;
    } else {
        TL = tmp + (int64_t)row * 2 * n;
        TR = TL + n;
    }

    for (int i = tid; i < n; i += SORT_THREADS) { key[i] = src[i]; idx[i] = (uint16_t)i; }
    for (int i = tid; i < nwords; i += SORT_THREADS) bits[i] = 0;
    if (tid == 0) {
        sh.ncur = 0;
        sh.nnxt = 0;
        if (n > LEAF) {
            segA[0] = 0u | ((uint32_t)n << 16);
            depA[0] = (uint8_t)(2 * floor_log2_i(n));
            sh.ncur = 1;
        }
    }
    __syncthreads();
    if (tid == 0) bits[0] = 1u;

    uint32_t *cur = segA, *nxt = segB;
    uint8_t *dcur = depA, *dnxt = depB;
    for (int level = 0; level < 64; ++level) {
        __syncthreads();
        const int ncur = sh.ncur;
        if (ncur == 0) break;
        for (int s = wid; s < ncur; s += SORT_WAVES) {
            const int f = (int)(cur[s] & 0xffffu);
            const int l = (int)(cur[s] >> 16);
            const int depth = dcur[s];
            if (depth == 0) {
                if (lane == 0) heap_sort_range(key, idx, f, l);
                wave_sync_lds();
                continue;
            }
            if (l - f <= SSA_WAVE) {           // the rest of this subtree in registers
                wave_small_sort(key, idx, bits, f, l - f, depth);
                continue;
            }
            const int cut = wave_partition(key, idx, TL, TR, f, l);
            if (lane == 0) {
                atomicOr(&bits[cut >> 5], 1u << (cut & 31));
                if (cut - f > LEAF) {
                    const int slot = atomicAdd(&sh.nnxt, 1);
                    nxt[slot] = (uint32_t)f | ((uint32_t)cut << 16);
                    dnxt[slot] = (uint8_t)(depth - 1);
                }
                if (l - cut > LEAF) {
                    const int slot = atomicAdd(&sh.nnxt, 1);
                    nxt[slot] = (uint32_t)cut | ((uint32_t)l << 16);
                    dnxt[slot] = (uint8_t)(depth - 1);
                }
            }
        }
        __syncthreads();
        if (tid == 0) { sh.ncur = sh.nnxt; sh.nnxt = 0; }
        uint32_t *t = cur; cur = nxt; nxt = t;
        uint8_t *td = dcur; dcur = dnxt; dnxt = td;
    }
    __syncthreads();

    // final insertion sort: one leaf (run between consecutive boundary bits) per thread
    for (int w = tid; w < (n + 31) / 32; w += SORT_THREADS) {
        uint32_t word = bits[w];
        while (word) {
            const int bpos = __ffs(word) - 1;
            word &= word - 1;
            const int s0 = w * 32 + bpos;
            if (s0 >= n) break;
            // end = next boundary after s0
            int e = n;
            uint32_t rest = word;
            if (rest) {
                e = w * 32 + __ffs(rest) - 1;
            } else {
                for (int w2 = w + 1; w2 < (n + 31) / 32; ++w2) {
                    if (bits[w2]) { e = w2 * 32 + __ffs(bits[w2]) - 1; break; }
                }
            }
            if (e > n) e = n;
            for (int i = s0 + 1; i < e; ++i) {
                const uint16_t vk = key[i], vi = idx[i];
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
    }
    __syncthreads();

    int32_t *pout = perm + (int64_t)row * n;
    for (int i = tid; i < n; i += SORT_THREADS) pout[i] = idx[i];
    for (int u = tid; u < NB; u += SORT_THREADS) {
        int lo = 0, hi = n;          // lower_bound(u)
        while (lo < hi) { const int mid = (lo + hi) >> 1; if (key[mid] < u) lo = mid + 1; else hi = mid; }
        const int st = lo;
        hi = n;                      // upper_bound(u)
        while (lo < hi) { const int mid = (lo + hi) >> 1; if (key[mid] <= u) lo = mid + 1; else hi = mid; }
        bstart[(int64_t)row * NB + u] = st;
        bsize[(int64_t)row * NB + u] = lo - st;
    }
}

}  // namespace

// LDS plan for a row of n keys
static void sort_plan(int n, int *cap, int *tl_in_lds, size_t *lds) {
    const int c = n / (LEAF + 1) + 2;
    const size_t base = ((size_t)4 * n + 15) / 16 * 16 + ((size_t)(n + 31) / 32 + 1) * 4 +
                        (size_t)c * 8 + (size_t)c * 2;
    const size_t with_tl = (base + 15) / 16 * 16 + (size_t)4 * n;
    *cap = c;
    if (with_tl <= SSA_LDS_BYTES) { *tl_in_lds = 1; *lds = with_tl; }
    else { *tl_in_lds = 0; *lds = base; }
}

int64_t ssa_sort_tmp_bytes(int rows, int n) {
    int cap, tl;
    size_t lds;
    sort_plan(n, &cap, &tl, &lds);
    return tl ? 0 : (int64_t)rows * 2 * n * (int64_t)sizeof(uint16_t);
}

int ssa_sort_supported(int n) {
    int cap, tl;
    size_t lds;
    if (n < 1 || n > 32768) return 0;
    sort_plan(n, &cap, &tl, &lds);
    return lds <= SSA_LDS_BYTES;
}

int ssa_launch_bucket_sort(const uint16_t *ids, int rows, int n, int P, int32_t *perm,
                           int32_t *bstart, int32_t *bsize, uint16_t *tmp, hipStream_t st) {
    if (!ssa_sort_supported(n)) {
        ssa_set_error("bucket sort: key length %d unsupported (1..32768)", n);
        return SSA_E_UNSUP;
    }
    if (rows == 0) return SSA_OK;
    int cap, tl;
    size_t lds;
    sort_plan(n, &cap, &tl, &lds);
    SSA_CHECK_HIP(hipFuncSetAttribute((const void *)bucket_sort_kernel,
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    hipLaunchKernelGGL(bucket_sort_kernel, dim3(rows), dim3(SORT_THREADS), lds, st, ids, n,
                       1 << P, perm, bstart, bsize, tmp, tl, cap);
    SSA_CHECK_LAUNCH();
    return SSA_OK;
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
