// ssa_measure.hip -- a reference kernel for the cache path the gather attention
// is bound by (no counterpart in the reference; used by the benchmark).
//
// The gather attention reads each query's neighbour rows of K and V; those
// rows repeat across queries, so they come from the L2 (and the MALL behind
// it), not from HBM, and the kernel's ceiling is how fast the L2 delivers
// lines to the CUs.  ssa_measure_l2_read measures that delivery rate: every
// workgroup streams the same small buffer (it stays in each XCD's L2 after the
// first touch, and it is far larger than a CU's L1, so nearly every load is an
// L1 miss served by the L2) with 16-byte loads, as the gather kernels load.
#include "ssa_common.h"
#include "../../include/ssa_amd.h"

namespace {

constexpr int L2R_THREADS = 256;
constexpr int L2R_UNROLL = 8;

__global__ void __launch_bounds__(L2R_THREADS)
l2_read_kernel(const uint4 *__restrict__ buf, uint32_t mask16, int iters, uint32_t *out) {
    // each block starts at its own offset so that the channels stay balanced
    uint32_t i = (blockIdx.x * 4099u * L2R_THREADS + threadIdx.x) & mask16;
    uint32_t acc = 0u;
    const uint32_t step = L2R_THREADS;
    const uint32_t per_iter = (mask16 + 1u) / (step * L2R_UNROLL);
    for (int it = 0; it < iters; ++it) {
        for (uint32_t j = 0; j < per_iter; ++j) {
            uint4 v[L2R_UNROLL];
#pragma unroll
            for (int u = 0; u < L2R_UNROLL; ++u) v[u] = buf[(i + u * step) & mask16];
#pragma unroll
            for (int u = 0; u < L2R_UNROLL; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
            i = (i + L2R_UNROLL * step) & mask16;
        }
    }
    // the result is written only when it equals a value the caller chose never
    // to match, which keeps every load live without a store per block
    if (acc == 0x9e3779b9u) out[blockIdx.x] = acc;
}

}  // namespace

extern "C" int ssa_measure_l2_read(const void *buf, int64_t bytes, int32_t blocks, int32_t iters,
                                   uint32_t *sink, void *stream) {
    SSA_CHECK_ARG(buf && sink, "measure_l2_read: null buffer");
    SSA_CHECK_ARG(bytes >= (int64_t)16 * L2R_THREADS * L2R_UNROLL && bytes <= ((int64_t)1 << 31) &&
                      (bytes & (bytes - 1)) == 0,
                  "measure_l2_read: bytes must be a power of two in [32 KiB, 2 GiB]");
    SSA_CHECK_ARG(blocks >= 1 && iters >= 1, "measure_l2_read: blocks %d iters %d", blocks, iters);
    SSA_CHECK_ARG(((uintptr_t)buf & 15) == 0, "measure_l2_read: buffer not 16-byte aligned");
    const uint32_t mask16 = (uint32_t)(bytes / 16 - 1);
    hipLaunchKernelGGL(l2_read_kernel, dim3((unsigned)blocks), dim3(L2R_THREADS), 0,
                       (hipStream_t)stream, (const uint4 *)buf, mask16, iters, sink);
    SSA_CHECK_LAUNCH();
    return SSA_OK;
}
