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
// cleared itself (its counters, with kernels).
//
// Calls on one GPU are ordered: each call's stream first waits for an event
// recorded at the end of the previous call's work on that GPU (whatever its
// stream or host thread), and the enqueue itself holds a lock, so calls from
// several streams or threads run one after another on the device instead of
// racing on the array.  The event is created once per device at the first
// call (no device memory).  A call made while its stream is under graph
// capture neither waits nor records (an event recorded outside a capture
// cannot be waited on inside it): replays of such a graph are ordered only
// by the stream they are launched on, so a caller must not replay one on a
// stream that runs beside another call of this entry point on the same GPU.
#include <mutex>

#include "ssa_graph_internal.h"

static __device__ __align__(256) unsigned char scratch[SSA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_scratch[kMaxDevices];   // device address of `scratch` per device (null = not yet)
hipEvent_t g_done[kMaxDevices]; // end of the last call's work per device
bool g_done_set[kMaxDevices];   // g_done has been recorded
std::mutex g_order_mu;          // held while a call is enqueued

// Device address of this device's scratch array.  The stream, when given, must
// belong to the current device: the address is looked up with it current.
int scratch_address(void *stream, void **out, int *dev_out) {
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
        SSA_CHECK_HIP(hipEventCreateWithFlags(&g_done[dev], hipEventDisableTiming));
        g_scratch[dev] = ptr;
    }
    *out = g_scratch[dev];
    *dev_out = dev;
    return SSA_OK;
}

}  // namespace

extern "C" int ssa_build_graph_noalloc(const ssa_graph_args *a, void *stream) {
    // refuse what does not fit before touching the device
    const int64_t need = ssa_graph_workspace_bytes_capped(a, (int64_t)SSA_NOALLOC_SCRATCH_BYTES);
    if (need < 0) return (int)need;
    void *ws = nullptr;
    int dev = -1;
    int rc = scratch_address(stream, &ws, &dev);
    if (rc) return rc;
    const hipStream_t st = (hipStream_t)stream;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    SSA_CHECK_HIP(hipStreamIsCapturing(st, &cs));
    const bool ordered = cs == hipStreamCaptureStatusNone;
    std::lock_guard<std::mutex> lk(g_order_mu);
    if (ordered && g_done_set[dev]) SSA_CHECK_HIP(hipStreamWaitEvent(st, g_done[dev], 0));
    rc = ssa_build_graph_capped(a, ws, (int64_t)SSA_NOALLOC_SCRATCH_BYTES, stream);
    if (ordered) {
        // recorded after a failed call too: whatever it enqueued is covered
        SSA_CHECK_HIP(hipEventRecord(g_done[dev], st));
        g_done_set[dev] = true;
    }
    return rc;
}
