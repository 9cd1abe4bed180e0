// Fixed device scratch for rfxq_gemm_no_alloc: a file-scope device array of
// kScratchBytes that the HIP runtime places in each device's memory when this
// object's code is loaded there. Its device address comes from
// hipGetSymbolAddress once per device, with that device current, and is kept
// per device here: in host code the array's name is only a host-side handle,
// never a device address, so nothing passes `scratch` itself to a kernel or a
// copy. Every call on one device shares its array (calls that overlap on one
// device race) and finds the previous call's contents in it.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>

#include "scratch.hpp"

namespace {

static __device__ __align__(256) unsigned char scratch[rfxq_scratch::kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

}  // namespace

namespace rfxq_scratch {

hipError_t setup(int device, void** out) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e != hipSuccess) return e;
        if (cur != device) return hipErrorInvalidDevice;  // the device must be current
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return hipSuccess;
}

void* address(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    return g_scratch_ptr[device];
}

}  // namespace rfxq_scratch
