// ssa_merge.hip -- merge of arbitrary window / global / LSH index lists.
//
// Replaces merge_neighbors (sparse_attention.py:966-1089) when it is called
// with caller-supplied lists (the fused build_graph path merges through a key
// bitmap instead).  The semantics are kept exactly, including the single
// sentinel = max(all inputs) + 1 (:1036-1037): self entries become the
// sentinel, the row is sorted, duplicates become the sentinel, the row is
// sorted again, self-attention prepends n; entries above the global max are
// invalid and written as 0; the result is clamped to [0, max].
//
// One wavefront per (bh, n) row sorts its Kall values with a bitonic network
// in LDS (Kall <= 1024).
#include "ssa_common.h"

namespace {

constexpr int MW = 4;   // waves per workgroup

__device__ __forceinline__ unsigned long long ord64(int64_t v) {
    return (unsigned long long)v ^ 0x8000000000000000ull;
}
__device__ __forceinline__ int64_t unord64(unsigned long long u) {
    return (int64_t)(u ^ 0x8000000000000000ull);
}

__global__ void merge_init_kernel(unsigned long long *tmax) { *tmax = ord64(INT64_MIN); }

__global__ void __launch_bounds__(256)
merge_max_kernel(const int64_t *win, int64_t nwin, const int64_t *glob, int G, const int64_t *lsh,
                 int64_t nlsh, unsigned long long *tmax) {
    int64_t m = INT64_MIN;
    const int64_t tot = nwin + G + nlsh;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < tot;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t v = i < nwin ? win[i] : (i < nwin + G ? glob[i - nwin] : lsh[i - nwin - G]);
        m = v > m ? v : m;
    }
    // wave max then one atomic per wave
    for (int o = 32; o > 0; o >>= 1) {
        const int64_t y = __shfl_xor(m, o, SSA_WAVE);
        m = y > m ? y : m;
    }
    if (lane_id() == 0 && m != INT64_MIN) atomicMax(tmax, ord64(m));
}

__device__ void wave_bitonic(int64_t *s, int n2) {
    const int lane = lane_id();
    for (int k = 2; k <= n2; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = lane; i < n2; i += SSA_WAVE) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const int64_t a = s[i], b = s[ixj];
                    const bool up = (i & k) == 0;
                    if ((a > b) == up) { s[i] = b; s[ixj] = a; }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
    }
}

__global__ void __launch_bounds__(MW * SSA_WAVE)
merge_rows_kernel(const int64_t *win, int Kw, const int64_t *glob, int G, const int64_t *lsh,
                  int Kl, int64_t BH, int N, int has_self, int Kout, int n2,
                  const unsigned long long *tmax_p, int64_t *out, uint8_t *valid) {
    extern __shared__ int64_t mg_smem[];
    const int wid = threadIdx.x / SSA_WAVE;
    const int64_t row = (int64_t)blockIdx.x * MW + wid;
    if (row >= BH * (int64_t)N) return;
    const int lane = lane_id();
    const int n = (int)(row % N);
    int64_t *s = mg_smem + (int64_t)wid * n2;
    const int Kall = Kw + G + Kl;
    const int64_t tmax = unord64(*tmax_p);
    const int64_t sentinel = tmax + 1;
    for (int i = lane; i < n2; i += SSA_WAVE) {
        int64_t v = INT64_MAX;
        if (i < Kw) v = win[(int64_t)n * Kw + i];
        else if (i < Kw + G) v = glob[i - Kw];
        else if (i < Kall) v = lsh[row * Kl + (i - Kw - G)];
        if (has_self && i < Kall && v == n) v = sentinel;
        s[i] = v;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    wave_bitonic(s, n2);
    // duplicates -> sentinel (decide on the sorted row first, then write)
    bool dup[16];
    for (int c = 0; c < 16; ++c) {
        const int i = lane + c * SSA_WAVE;
        dup[c] = i > 0 && i < Kall && i < n2 && s[i] == s[i - 1];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (int c = 0; c < 16; ++c) {
        const int i = lane + c * SSA_WAVE;
        if (dup[c]) s[i] = sentinel;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    wave_bitonic(s, n2);
    int64_t *orow = out + row * Kout;
    uint8_t *vrow = valid + row * Kout;
    const int self = has_self ? 1 : 0;
    for (int i = lane; i < Kout; i += SSA_WAVE) {
        int64_t v = (self && i == 0) ? (int64_t)n : s[i - self];
        bool ok = v <= tmax;
        if (self && i == 0) ok = true;
        if (v > tmax) v = 0;
        if (v < 0) v = 0;
        if (v > tmax) v = tmax;
        orow[i] = v;
        vrow[i] = ok ? 1 : 0;
    }
}

}  // namespace

extern "C" int ssa_merge_neighbors(const int64_t *win, int32_t Kw, const int64_t *glob, int32_t G,
                                   const int64_t *lsh, int32_t Kl, int32_t BH, int32_t N,
                                   int32_t has_self, int32_t total_k, int64_t *out,
                                   uint8_t *valid, void *workspace, void *stream) {
    SSA_CHECK_ARG(Kw >= 0 && G >= 0 && Kl >= 0 && BH >= 0 && N >= 0 && total_k >= 1,
                  "merge_neighbors: bad sizes");
    SSA_CHECK_ARG(out && valid && workspace, "merge_neighbors: null output/workspace");
    SSA_CHECK_ARG((Kw == 0 || win) && (G == 0 || glob) && (Kl == 0 || lsh),
                  "merge_neighbors: null input");
    const int Kall = Kw + G + Kl;
    SSA_CHECK_ARG(Kall >= 1 && Kall <= 1024, "merge_neighbors: Kall=%d outside 1..1024", Kall);
    const int ks = has_self ? (total_k - 1 < Kall ? total_k - 1 : Kall)
                            : (total_k < Kall ? total_k : Kall);
    const int Kout = (has_self ? 1 : 0) + ks;
    if ((int64_t)BH * N == 0 || Kout == 0) return SSA_OK;
    int n2 = 64;
    while (n2 < Kall) n2 <<= 1;
    hipStream_t st = (hipStream_t)stream;
    unsigned long long *tmax = (unsigned long long *)workspace;
    hipLaunchKernelGGL(merge_init_kernel, dim3(1), dim3(1), 0, st, tmax);
    SSA_CHECK_LAUNCH();
    const int64_t nlsh = (int64_t)BH * N * Kl;
    const int64_t tot = (int64_t)N * Kw + G + nlsh;
    const unsigned g = (unsigned)std::min<int64_t>(ceil_div(tot, 256), 2048);
    hipLaunchKernelGGL(merge_max_kernel, dim3(g), dim3(256), 0, st, win, (int64_t)N * Kw, glob, G,
                       lsh, nlsh, tmax);
    SSA_CHECK_LAUNCH();
    const int64_t rows = (int64_t)BH * N;
    const size_t lds = (size_t)MW * n2 * sizeof(int64_t);
    hipLaunchKernelGGL(merge_rows_kernel, dim3((unsigned)ceil_div(rows, MW)), dim3(MW * SSA_WAVE),
                       lds, st, win, Kw, glob, G, lsh, Kl, (int64_t)BH, N, has_self, Kout, n2,
                       (const unsigned long long *)tmax, out, valid);
    SSA_CHECK_LAUNCH();
    return SSA_OK;
}
