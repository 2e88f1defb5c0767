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
// so nothing needs clearing.  Calls that overlap on one device (two
// contexts' streams, several host threads) race.
#include <mutex>

#include "lbt_internal.h"

namespace {

constexpr size_t kNoAllocScratchBytes = 4u << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

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
        g_ptr[device] = p;
    }
    *out = g_ptr[device];
    *bytes = kNoAllocScratchBytes;
    return LBT_OK;
}

}  // namespace lbt
