// Fixed device scratch of the no-allocation entry point (brik_matmul_t_q4_noalloc).
//
// Callers that cannot allocate device memory (code under HIP graph capture, serving loops that must
// not call hipMalloc) still need the matmul's staging memory: the f16 activation rows of the MFMA
// path and the staged activation image of a large M = 1 GEMV. That memory is this file-scope array,
// one copy per device, held until the process ends. It is never named in device code: the kernels
// take its device address as an argument, exactly as they take a context workspace.
//
// The array's name in host code is a host-side stand-in, not a device address, so it is never passed
// to a kernel or a copy. Its address on a device comes from hipGetSymbolAddress with that device
// current, resolved once per device (brik_create calls brik_scratch_resolve) and kept in a table.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <mutex>

#include "../../include/brik.h"

namespace {

static __device__ __align__(256) unsigned char scratch[BRIK_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_lock;
void* g_addr[kMaxDevices] = {};

}  // namespace

// Device address of the scratch array on `device`, which must be the current device. Resolved with
// hipGetSymbolAddress on the first call for a device and cached after that. Returns a hipError_t
// value (hipSuccess = 0), or hipErrorInvalidDevice for a device index beyond the table.
extern "C" __attribute__((visibility("hidden"))) int brik_scratch_resolve(int device, void** out, size_t* bytes)
{
    *out = nullptr;
    *bytes = 0;
    if (device < 0 || device >= kMaxDevices) return (int)hipErrorInvalidDevice;
    std::lock_guard<std::mutex> guard(g_lock);
    if (!g_addr[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        if (!p) return (int)hipErrorInvalidSymbol;
        g_addr[device] = p;
    }
    *out = g_addr[device];
    *bytes = sizeof(scratch);
    return (int)hipSuccess;
}
