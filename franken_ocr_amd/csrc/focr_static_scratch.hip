// focr_static_scratch.hip — the device scratch of the allocation-free entry
// points (focr_hip_moe_decode_noalloc): one statically allocated array per
// GPU, resolved to a device address once per device when a context is
// created, so those entry points never call hipMalloc or hipFree.
//
// In host code the array's name is only a host-side stand-in for the symbol:
// a kernel handed `scratch` itself would fault. The address every host path
// uses is the one hipGetSymbolAddress returns with the device current, kept
// per device (each GPU holds its own copy of the array at its own address).
//
// Every call on a GPU shares that GPU's array, so calls are ordered per
// device: each call's stream first waits for the previous call's completion
// event, and the call records its own at the end (StaticScratchOrder). The
// event is created once, with the address, at context creation; a call
// creates and allocates nothing. Calls issued while their stream is being
// captured into a graph are not ordered this way (the graph's own
// dependencies order them).
#include "focr_internal.hpp"

static __device__ __align__(256) unsigned char scratch[focr::kStaticScratchBytes];

namespace focr {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;                    // guards the tables below
void* g_ptr[kMaxDevices];           // resolved address (null until resolved)
hipEvent_t g_last[kMaxDevices];     // completion of the last call on the device
bool g_recorded[kMaxDevices];       // g_last has been recorded at least once
std::mutex g_call_mu[kMaxDevices];  // held from a call's wait to its record

}  // namespace

hipError_t static_scratch_init(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[device]) {
        // nothing is cached on failure: a later context, or the entry point
        // itself, resolves again
        void* p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));  // the caller made `device` current
        if (e != hipSuccess) return e;
        if (!g_last[device]) {
            hipEvent_t ev = nullptr;
            e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
            if (e != hipSuccess) return e;
            g_last[device] = ev;
        }
        g_ptr[device] = p;
    }
    *out = g_ptr[device];
    return hipSuccess;
}

StaticScratchOrder::StaticScratchOrder(int device, hipStream_t stream) : device_(device), stream_(stream) {
    if (device < 0 || device >= kMaxDevices) {
        err_ = hipErrorInvalidDevice;
        return;
    }
    g_call_mu[device].lock();
    locked_ = true;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    err_ = hipStreamIsCapturing(stream, &cs);
    if (err_ != hipSuccess) return;
    capturing_ = cs != hipStreamCaptureStatusNone;
    if (capturing_) return;
    bool recorded;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        ev_ = g_last[device];
        recorded = g_recorded[device];
    }
    if (ev_ && recorded) err_ = hipStreamWaitEvent(stream, ev_, 0);
}

StaticScratchOrder::~StaticScratchOrder() {
    if (!locked_) return;
    if (err_ == hipSuccess && ev_ && hipEventRecord(ev_, stream_) == hipSuccess) {
        std::lock_guard<std::mutex> lk(g_mu);
        g_recorded[device_] = true;
    }
    g_call_mu[device_].unlock();
}

}  // namespace focr
