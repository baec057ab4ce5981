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

#include "ssa_sort_dev.h"

namespace {

template <typename Pos>
__global__ void __launch_bounds__(SORT_THREADS)
sort_top_kernel(const uint16_t *ids, int n, int NB, int32_t *perm, int32_t *bstart, int32_t *bsize,
                typename SortWords<Pos>::W *gkv, int4 *segs, int *segcount, unsigned char *glb,
                int tl_in_lds, int cap) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    __shared__ TopShared sh;
    sort_top_row<Pos>((int)blockIdx.x, ids, n, NB, perm, bstart, bsize, gkv, segs, segcount, glb,
                      tl_in_lds, cap, smem_raw, sh);
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
    if (with_tl <= SORT_LDS_BYTES) { *tl_in_lds = 1; *lds = with_tl; }
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
    return lds <= SORT_LDS_BYTES;
}

int32_t *ssa_sort_counter(uint16_t *tmp, int rows, int n) {
    const int64_t rn = (int64_t)rows * n;
    return (int32_t *)((char *)tmp + al256(rn * sort_row_bytes(n)) + al256(rn * 16));
}

int ssa_sort_top_setup(const uint16_t *ids, int rows, int n, int P, int32_t *perm,
                       int32_t *bstart, int32_t *bsize, uint16_t *tmp, SortTopArgs *a) {
    if (n > SORT_LDS_KEYS || !ssa_sort_supported(n)) {
        ssa_set_error("bucket sort: the shared top-level launch takes 1..%d keys", SORT_LDS_KEYS);
        return SSA_E_UNSUP;
    }
    size_t lds;
    a->NB = 1 << P;
    sort_plan(n, a->NB, &a->cap, &a->tl_in_lds, &lds);
    a->lds = (int)lds;
    const int64_t rn = (int64_t)rows * n;
    char *t = (char *)tmp;
    a->ids = ids; a->rows = rows; a->n = n;
    a->perm = perm; a->bstart = bstart; a->bsize = bsize;
    a->gkv = (uint32_t *)t;
    a->segs = (int4 *)(t + al256(rn * 4));
    a->segcount = ssa_sort_counter(tmp, rows, n);
    a->glb = (unsigned char *)t + al256(rn * 4) + al256(rn * 16) + 256;
    return SSA_OK;
}

template <typename Pos>
static int launch_seg(const typename SortWords<Pos>::W *gkv, int rows, int n, const int4 *segs,
                      const int *segcount, int32_t *perm, hipStream_t st) {
    const int64_t waves = std::max<int64_t>(1, std::min<int64_t>((int64_t)rows * n / 128, 8192));
    hipLaunchKernelGGL((sort_seg_kernel<Pos>), dim3((unsigned)ceil_div(waves, SEG_WAVES)),
                       dim3(SEG_WAVES * SSA_WAVE), 0, st, gkv, n, segs, segcount, perm);
    SSA_CHECK_LAUNCH();
    return SSA_OK;
}

int ssa_launch_sort_seg(const SortTopArgs &a, hipStream_t st) {
    return launch_seg<uint16_t>(a.gkv, a.rows, a.n, a.segs, a.segcount, a.perm, st);
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
    return launch_seg<Pos>(gkv, rows, n, segs, segcount, perm, st);
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
