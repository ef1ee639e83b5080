// Device scratch of the allocation-free fused entry point
// (dcn_forward_f16_prepacked_noalloc_dev): the padded channel-block copy of the input
// lives in a file-scope device array instead of the context's hipMalloc'd workspace.
//
// The array is one per device (each device that loads the library holds it until the
// process ends). Host code never uses the array's name as an address: its device
// address is resolved once per device with hipGetSymbolAddress, with that device
// current, and cached here; kernels receive that address as an argument.
//
// Calls on one device share its array, so they are ordered here: each call records an
// event on its stream after its work, and a call on another stream first makes its stream
// wait for that event (hipStreamWaitEvent allocates nothing). Calls from several host
// threads take the same lock while they enqueue. Under graph capture the call neither
// waits nor records (the caller orders captured calls).
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "dcn_internal.hpp"

namespace dcn {
namespace {

static __device__ __align__(256) uint8_t scratch[DCN_NOALLOC_SCRATCH_BYTES];

// Per device: the device address of `scratch`, an event recorded after the last call's
// work and the stream it was recorded on.
struct ScratchState {
    void* ptr = nullptr;
    hipEvent_t done = nullptr;
    hipStream_t last = nullptr;
    bool used = false;
};
std::mutex g_scratch_mu;
std::vector<ScratchState> g_scratch;

bool capturing(hipStream_t stream) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    // (An error here, e.g. the null stream while another stream captures globally, is
    // treated as capture: the call then leaves the ordering to its caller.)
    return hipStreamIsCapturing(stream, &st) != hipSuccess || st != hipStreamCaptureStatusNone;
}

}  // namespace

hipError_t noalloc_scratch_init(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device < 0) return hipErrorInvalidDevice;
    if (g_scratch.size() <= (size_t)device) g_scratch.resize((size_t)device + 1);
    ScratchState& d = g_scratch[(size_t)device];
    if (d.ptr) return hipSuccess;
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    hipEvent_t ev = nullptr;
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) return e;
    d.ptr = ptr;
    d.done = ev;
    return hipSuccess;
}

NoallocScratchUse::NoallocScratchUse(int device, hipStream_t stream)
    : lock_(g_scratch_mu), device_(device), stream_(stream) {
    if (device < 0 || (size_t)device >= g_scratch.size() || !g_scratch[(size_t)device].ptr) return;
    ScratchState& d = g_scratch[(size_t)device];
    ptr_ = d.ptr;
    ordered_ = !capturing(stream);
    // The previous call on another stream may still read the array: this stream waits
    // for it (on the device; the host does not block).
    if (ordered_ && d.used && d.last != stream) error_ = hipStreamWaitEvent(stream, d.done, 0);
}

NoallocScratchUse::~NoallocScratchUse() {
    if (!ptr_ || !ordered_) return;
    ScratchState& d = g_scratch[(size_t)device_];
    if (hipEventRecord(d.done, stream_) == hipSuccess) {
        d.last = stream_;
        d.used = true;
    }
}

}  // namespace dcn
