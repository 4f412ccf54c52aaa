// Workspace of the allocation-free batch search: a file-scope device array,
// one copy per GPU, whose address is looked up once per device.
//
// Host code never passes `scratch` itself to a kernel or a copy: on the host
// the name is a stand-in for the symbol, not a device address.  Only the
// pointer hipGetSymbolAddress returns for the current device is used.
#include <mutex>

#include "vgpu_runtime.h"

namespace vgpu {

static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[kMaxDevices] = {};
// Serialises the synchronous calls that share one device's array.
std::mutex g_call_mu[kMaxDevices];
}  // namespace

std::mutex& noalloc_call_mutex(int device) {
    if (device < 0 || device >= kMaxDevices)
        throw Error(VGPU_ERR_DEVICE, "device ordinal " + std::to_string(device) + " out of range");
    return g_call_mu[device];
}

uint8_t* noalloc_scratch(int device) {
    if (device < 0 || device >= kMaxDevices)
        throw Error(VGPU_ERR_DEVICE, "device ordinal " + std::to_string(device) + " out of range");
    int cur = -1;
    VGPU_HIP(hipGetDevice(&cur));
    if (cur != device)
        throw Error(VGPU_ERR_INVALID_PARAMETER, "the index's device (" + std::to_string(device) +
                                                    ") must be current, not device " + std::to_string(cur));
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void* p = nullptr;
        VGPU_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) throw Error(VGPU_ERR_DEVICE, "hipGetSymbolAddress returned a null scratch address");
        g_scratch_ptr[device] = static_cast<uint8_t*>(p);
    }
    return g_scratch_ptr[device];
}

}  // namespace vgpu
