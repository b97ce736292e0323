// noalloc.hip — the scratch memory of the entry point that allocates nothing
// (mgh_gemm_h16_f32in_noalloc, include/mgh.h): a file-scope device array of a fixed size that
// every GPU the library runs on holds until the process ends.
//
// Host code never uses the array's name as an address (in host code it is a host-side
// stand-in): the device address comes from hipGetSymbolAddress, looked up once per device with
// that device current, and kept per device. Calls on one GPU share that GPU's array; calls that
// overlap on one GPU (two streams, two threads) race on it.
#include <mutex>

#include "mgh_common.h"
#include "mgh_kernels.h"

namespace mgh {

namespace {

constexpr size_t kNoallocScratchBytes = (size_t)64 << 20;

__device__ __align__(256) uint8_t scratch[kNoallocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

}  // namespace

size_t noalloc_scratch_bytes() { return kNoallocScratchBytes; }

hipError_t noalloc_scratch(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[device]) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e != hipSuccess) return e;
        if (cur != device && (e = hipSetDevice(device)) != hipSuccess) return e;
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != device) (void)hipSetDevice(cur);
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_ptr[device] = p;
    }
    *out = g_ptr[device];
    return hipSuccess;
}

}  // namespace mgh
