// Per-device static scratch of the allocation-free paged decode (fa_paged_decode_noalloc).
//
// The array is ordinary device memory that the code object carries: every GPU the library
// runs on holds its own copy at its own address until the process ends. Host code never passes
// the array's name to a kernel or a copy (in host code that name is a host-side stand-in, not a
// device address); it asks noalloc_scratch() for the device's address, resolved once per device
// with hipGetSymbolAddress while that device is current.
#include <mutex>

#include "kernels.hpp"

static __device__ __align__(256) unsigned char scratch[fa::kNoAllocScratchBytes];

namespace fa {
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
// Calls on one device are ordered through the scratch: each call holds the device's mutex
// while it enqueues, makes its stream wait for the event the previous user recorded, and
// records its own completion into that event. Stream-ordered, no host wait, no allocation.
std::mutex g_order_mu[kMaxDevices];
hipEvent_t g_last_user[kMaxDevices] = {};
}  // namespace

hipError_t noalloc_order_begin(int device, hipStream_t s) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    g_order_mu[device].lock();
    hipError_t e = hipSuccess;
    if (!g_last_user[device])
        e = hipEventCreateWithFlags(&g_last_user[device], hipEventDisableTiming);
    else
        e = hipStreamWaitEvent(s, g_last_user[device], 0);
    if (e != hipSuccess) g_order_mu[device].unlock();
    return e;
}

hipError_t noalloc_order_end(int device, hipStream_t s, bool enqueued) {
    hipError_t e = hipSuccess;
    if (enqueued) e = hipEventRecord(g_last_user[device], s);
    g_order_mu[device].unlock();
    return e;
}

hipError_t noalloc_scratch(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        int current = -1;
        hipError_t e = hipGetDevice(&current);
        if (e != hipSuccess) return e;
        if (current != device && (e = hipSetDevice(device)) != hipSuccess) return e;
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (current != device) (void)hipSetDevice(current);
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return hipSuccess;
}

}  // namespace fa
