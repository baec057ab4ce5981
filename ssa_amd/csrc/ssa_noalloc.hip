// ssa_noalloc.hip -- the neighbour-graph build without any device allocation.
//
// For callers that cannot allocate (code under HIP graph capture, tight
// serving loops, harnesses that forbid hipMalloc): ssa_build_graph's work runs
// over `scratch`, a fixed array of SSA_NOALLOC_SCRATCH_BYTES in device memory
// that every GPU the library runs on holds from module load until the process
// ends, instead of a caller-sized workspace.  Query heads go in chunks small
// enough for the array (the same kernels and results as ssa_build_graph);
// problems that do not fit with one head per chunk are refused with
// SSA_E_WORKSPACE before anything is launched.
//
// Host code never passes `scratch` itself to a kernel: in host code the name
// is a stand-in registered with the runtime, not a device address.  The device
// address comes from hipGetSymbolAddress, once per device with that device
// current, and only that pointer is used.  Every call on one GPU shares the
// array and it keeps the last call's contents: the build clears what it needs
// cleared itself (its counters, with kernels), and calls that overlap on one
// GPU (different streams, different host threads) race on it.
#include <mutex>

#include "ssa_graph_internal.h"

static __device__ __align__(256) unsigned char scratch[SSA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_scratch[kMaxDevices];   // device address of `scratch` per device (null = not yet)

// Device address of this device's scratch array.  The stream, when given, must
// belong to the current device: the address is looked up with it current.
int scratch_address(void *stream, void **out) {
    int dev = -1;
    SSA_CHECK_HIP(hipGetDevice(&dev));
    SSA_CHECK_ARG(dev >= 0 && dev < kMaxDevices, "build_graph_noalloc: device %d", dev);
    if (stream) {
        hipDevice_t sdev = -1;
        SSA_CHECK_HIP(hipStreamGetDevice((hipStream_t)stream, &sdev));
        SSA_CHECK_ARG(sdev == dev,
                      "build_graph_noalloc: the stream belongs to device %d, the current device "
                      "is %d", (int)sdev, dev);
    }
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_scratch[dev]) {
        void *ptr = nullptr;
        SSA_CHECK_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        SSA_CHECK_ARG(ptr != nullptr, "build_graph_noalloc: no address for the scratch array");
        g_scratch[dev] = ptr;
    }
    *out = g_scratch[dev];
    return SSA_OK;
}

}  // namespace

extern "C" int ssa_build_graph_noalloc(const ssa_graph_args *a, void *stream) {
    // refuse what does not fit before touching the device
    const int64_t need = ssa_graph_workspace_bytes_capped(a, (int64_t)SSA_NOALLOC_SCRATCH_BYTES);
    if (need < 0) return (int)need;
    void *ws = nullptr;
    const int rc = scratch_address(stream, &ws);
    if (rc) return rc;
    return ssa_build_graph_capped(a, ws, (int64_t)SSA_NOALLOC_SCRATCH_BYTES, stream);
}
