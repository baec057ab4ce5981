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

template <typename Pos>
__global__ void __launch_bounds__(SEG_WAVES * SSA_WAVE)
sort_seg_kernel(const typename SortWords<Pos>::W *gkv, int n, const int4 *segs,
                const int *segcount, int32_t *perm) {
    __shared__ uint32_t lds[SEG_WAVES * seg_lds_words<Pos>()];
    sort_seg_blocks<Pos>(gkv, n, segs, segcount, perm, lds, (int)blockIdx.x, (int)gridDim.x);
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

int ssa_sort_seg_blocks(int rows, int n) {
    const int64_t waves = std::max<int64_t>(1, std::min<int64_t>((int64_t)rows * n / 128, 8192));
    return (int)ceil_div(waves, SEG_WAVES);
}

template <typename Pos>
static int launch_seg(const typename SortWords<Pos>::W *gkv, int rows, int n, const int4 *segs,
                      const int *segcount, int32_t *perm, hipStream_t st) {
    hipLaunchKernelGGL((sort_seg_kernel<Pos>), dim3((unsigned)ssa_sort_seg_blocks(rows, n)),
                       dim3(SEG_WAVES * SSA_WAVE), 0, st, gkv, n, segs, segcount, perm);
    SSA_CHECK_LAUNCH();
    return SSA_OK;
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
