// The scratch memory of sl_hip_dispatch_noalloc: one file-scope device array
// per GPU (the code object's own data, resident from module load until the
// process ends), so that entry point never allocates.
//
// In host code `scratch` names a host-side stand-in, not a device address:
// its per-GPU address comes from hipGetSymbolAddress, called once per device
// with that device current, and only that address is used.
#include <mutex>

#include "common.h"
#include "kernels.h"

namespace slhip {
namespace {

static __device__ __align__(256) float scratch[kStaticScratchFloats];

constexpr int kMaxOrdinals = 64;
std::mutex g_lock;
float* g_addr[kMaxOrdinals] = {};

}  // namespace

hipError_t static_scratch_address(int ordinal, float** out) {
    *out = nullptr;
    if (ordinal < 0 || ordinal >= kMaxOrdinals) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> hold(g_lock);
    if (g_addr[ordinal] == nullptr) {
        int current = -1;
        hipError_t e = hipGetDevice(&current);
        if (e != hipSuccess) return e;
        if (current != ordinal) return hipErrorInvalidDevice;  // the caller makes `ordinal` current
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_addr[ordinal] = static_cast<float*>(p);
    }
    *out = g_addr[ordinal];
    return hipSuccess;
}

}  // namespace slhip
