// noalloc.hip — the scratch memory of the entry point that allocates nothing
// (mgh_gemm_h16_f32in_noalloc, include/mgh.h): a file-scope device array of a fixed size that
// every GPU the library runs on holds until the process ends.
//
// Host code never uses the array's name as an address (in host code it is a host-side
// stand-in): the device address comes from hipGetSymbolAddress, looked up once per device with
// that device current, and kept per device. Calls on one GPU share that GPU's array. They are
// ordered on the device by one event per GPU (created at the same set-up): each call waits for
// the previous call's launches, on whatever stream they ran, then records the event after its
// own (noalloc_order_begin / _end, under a host mutex so two threads cannot interleave). Under
// stream capture the event is not used: the captured graph's launches are ordered by the graph,
// and replays of it must not overlap other calls on the same GPU.
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
hipEvent_t g_ev[kMaxDevices] = {};
std::mutex g_order_mu;

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
        hipEvent_t ev = nullptr;
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (cur != device) (void)hipSetDevice(cur);
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_ptr[device] = p;
        g_ev[device] = ev;
    }
    *out = g_ptr[device];
    return hipSuccess;
}

hipError_t noalloc_order_begin(int device, hipStream_t s, bool* capturing) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(s, &st);
    if (e != hipSuccess) return e;
    *capturing = st != hipStreamCaptureStatusNone;
    if (*capturing) return hipSuccess;
    g_order_mu.lock();
    // waiting on an event no call has recorded yet returns at once
    e = hipStreamWaitEvent(s, g_ev[device], 0);
    if (e != hipSuccess) g_order_mu.unlock();
    return e;
}

hipError_t noalloc_order_end(int device, hipStream_t s, bool capturing) {
    if (capturing) return hipSuccess;
    const hipError_t e = hipEventRecord(g_ev[device], s);
    g_order_mu.unlock();
    return e;
}

}  // namespace mgh
