// noalloc.hip -- the static device scratch of lbt_ternary_linear_dev_noalloc,
// the entry point that allocates nothing (for callers that cannot call
// hipMalloc: code under HIP graph capture, tight serving loops).
//
// The quantized activations of the several-row paths (int8 rows padded to
// the LB2 width, then s_a and sum(q) per row) live in one file-scope device
// array.  Each device holds its own copy until the process ends; its address
// on a device is looked up once (hipGetSymbolAddress, with that device
// current) and only that address is handed to kernels and copies -- in host
// code the array's name is a host-side stand-in, not a device address.
// Every call on a device shares the array and leaves its contents behind;
// the quantizer writes every byte a later kernel reads (padding included),
// so nothing needs clearing.  Calls on one device are ordered: each call runs
// under the device's host mutex and, when the previous call came from
// another stream, first makes its stream wait (on the device) for that call's
// completion event.  Under stream capture no event is waited for or recorded
// (a captured stream cannot wait on work outside its capture): captured calls
// that overlap other streams' calls on the device race.
#include <functional>
#include <mutex>

#include "lbt_internal.h"

namespace {

constexpr size_t kNoAllocScratchBytes = 4u << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

// per device: the order of calls
struct DevOrder {
    std::mutex mu;
    hipEvent_t done = nullptr;      // recorded after the last call's kernels
    hipStream_t last = nullptr;     // the stream of the last call
};
DevOrder g_order[kMaxDevices];

}  // namespace

namespace lbt {

int noalloc_scratch_init(int device, void** out, size_t* bytes) {
    *out = nullptr;
    *bytes = 0;
    if (device < 0 || device >= kMaxDevices) return LBT_E_INVALID;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[device]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return LBT_E_DEVICE;
        hipEvent_t ev = nullptr;
        if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) return LBT_E_DEVICE;
        g_order[device].done = ev;
        g_ptr[device] = p;
    }
    *out = g_ptr[device];
    *bytes = kNoAllocScratchBytes;
    return LBT_OK;
}

int noalloc_ordered(int device, hipStream_t s, const std::function<int()>& launch) {
    if (device < 0 || device >= kMaxDevices || !g_order[device].done) return LBT_E_DEVICE;
    DevOrder& o = g_order[device];
    std::lock_guard<std::mutex> lk(o.mu);
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess) return LBT_E_DEVICE;
    const bool capturing = cs != hipStreamCaptureStatusNone;
    if (!capturing && o.last && o.last != s && hipStreamWaitEvent(s, o.done, 0) != hipSuccess) return LBT_E_DEVICE;
    const int rc = launch();
    if (rc || capturing) return rc;
    if (hipEventRecord(o.done, s) != hipSuccess) return LBT_E_DEVICE;
    o.last = s;
    return LBT_OK;
}

}  // namespace lbt
