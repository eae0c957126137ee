// lgx_scratch.hip -- the fixed device scratch of lgx_q8_gemm_noalloc.
//
// One file-scope device array, LGX_NOALLOC_SCRATCH_BYTES long, that the HIP
// runtime places on every device the library runs on when it loads this
// translation unit's code object, and keeps until the process ends.  Host
// code never uses the array's name as an address (on the host it is only a
// stand-in for the symbol): lgxi_scratch_ptr resolves this device's copy once
// with hipGetSymbolAddress, with the device current, and every later use
// (kernel arguments, copies) goes through the returned pointer.
//
// Every call of the no-alloc entry point on one device shares that device's
// copy; nothing in it has to start at zero (each launch writes every byte it
// later reads), and calls that overlap on one device race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../../include/lgx.h"

static __device__ __align__(256) unsigned char scratch[LGX_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_addr[kMaxDevices] = {};   // this library's scratch on each device, once resolved
}  // namespace

// Device address of `device`'s copy of the scratch array; the caller has
// made `device` current.  Resolved on the first call per device.
extern "C" hipError_t lgxi_scratch_ptr(int device, void** out) {
    if (device < 0 || device >= kMaxDevices || !out) return hipErrorInvalidValue;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_addr[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_addr[device] = p;
    }
    *out = g_addr[device];
    return hipSuccess;
}
