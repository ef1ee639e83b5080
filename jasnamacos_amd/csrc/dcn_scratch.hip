// Device scratch of the allocation-free fused entry point
// (dcn_forward_f16_prepacked_noalloc_dev): the padded channel-block copy of the input
// lives in a file-scope device array instead of the context's hipMalloc'd workspace.
//
// The array is one per device (each device that loads the library holds it until the
// process ends). Host code never uses the array's name as an address: its device
// address is resolved once per device with hipGetSymbolAddress, with that device
// current, and cached here; kernels receive that address as an argument.
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "dcn_internal.hpp"

namespace dcn {
namespace {

static __device__ __align__(256) uint8_t scratch[DCN_NOALLOC_SCRATCH_BYTES];

std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;  // device address of `scratch`, per device index

}  // namespace

hipError_t noalloc_scratch_init(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (device < 0) return hipErrorInvalidDevice;
    if (g_scratch_ptr.size() <= (size_t)device) g_scratch_ptr.resize((size_t)device + 1, nullptr);
    if (g_scratch_ptr[(size_t)device]) return hipSuccess;
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[(size_t)device] = ptr;
    return hipSuccess;
}

void* noalloc_scratch(int device) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    return device >= 0 && (size_t)device < g_scratch_ptr.size() ? g_scratch_ptr[(size_t)device] : nullptr;
}

}  // namespace dcn
