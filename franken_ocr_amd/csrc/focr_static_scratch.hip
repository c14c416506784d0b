// focr_static_scratch.hip — the device scratch of the allocation-free entry
// points (focr_hip_moe_decode_noalloc): one statically allocated array per
// GPU, resolved to a device address once per device when a context is
// created, so those entry points never call hipMalloc or hipFree.
//
// In host code the array's name is only a host-side stand-in for the symbol:
// a kernel handed `scratch` itself would fault. The address every host path
// uses is the one hipGetSymbolAddress returns with the device current, kept
// per device (each GPU holds its own copy of the array at its own address).
#include "focr_internal.hpp"

static __device__ __align__(256) unsigned char scratch[focr::kStaticScratchBytes];

namespace focr {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices];
hipError_t g_err[kMaxDevices];
bool g_done[kMaxDevices];

}  // namespace

hipError_t static_scratch_init(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_done[device]) {
        void* p = nullptr;
        g_err[device] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));  // the caller made `device` current
        g_ptr[device] = g_err[device] == hipSuccess ? p : nullptr;
        g_done[device] = true;
    }
    *out = g_ptr[device];
    return g_err[device];
}

}  // namespace focr
