// noalloc.hip -- the fixed device scratch of gncx_hip_decode_step_noalloc.
//
// The native decode step keeps two scratch buffers: the split-K partials of
// each layer's attention (written by the chunk kernel, read by the merge) and
// the per-chunk maxima of the greedy argmax.  Both are fully written before
// they are read, so nothing in them has to start at zero.  The no-allocation
// entry point takes them from one file-scope device array instead of device
// memory the library allocates: each GPU the library runs on holds its own
// copy of the array (kNoAllocScratchBytes) until the process ends.  Its
// device address is looked up once per device, with that device current;
// host code passes that address, never the array's name (which is a
// host-side stand-in, not a device address).  Calls that overlap on one GPU
// share the array and race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "gncx_launch.h"

static __device__ __align__(256) uint8_t scratch[gncx::kNoAllocScratchBytes];

namespace gncx {
namespace {

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;

}  // namespace

hipError_t noalloc_scratch(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        int cur = -1;
        hipError_t e = hipGetDevice(&cur);
        if (e != hipSuccess) return e;
        if (cur != device && (e = hipSetDevice(device)) != hipSuccess) return e;
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (cur != device) (void)hipSetDevice(cur);
        if (e != hipSuccess) return e;
        if (!p || (reinterpret_cast<uintptr_t>(p) & 255u) != 0) return hipErrorInvalidSymbol;
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return hipSuccess;
}

}  // namespace gncx
