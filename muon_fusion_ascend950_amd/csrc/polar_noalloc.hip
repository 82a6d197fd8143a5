// polar_noalloc.hip — the scratch memory of muon_polar_step_noalloc, for callers
// that cannot allocate device memory (code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc).
//
// `scratch` is a file-scope device array: the runtime gives every GPU that loads
// this code object its own copy, at its own address, held until the process
// ends.  Host code never passes the array's name to a kernel or a copy (in host
// code it names a host-side stand-in); it asks the runtime for this device's
// address once (hipGetSymbolAddress with the device current) and uses that.
//
// The kernels need nothing in it to start at zero: A, P and the padded copy of X
// are written before they are read, stream-K partials are written before their
// arrival counts, and the arrival words carry a per-launch token, so words left
// by earlier calls count as zero.  Calls that overlap on one GPU share the array
// and race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "polar_kernels.h"

static __device__ __align__(256) unsigned char scratch[muon_polar::kNoAllocScratchBytes];

namespace muon_polar {

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch[kMaxDevices];  // device address of `scratch` on each device, once known
}  // namespace

hipError_t noalloc_scratch(int device, void **ptr) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch[device] == nullptr) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (p == nullptr) return hipErrorInvalidSymbol;
        g_scratch[device] = p;
    }
    *ptr = g_scratch[device];
    return hipSuccess;
}

}  // namespace muon_polar
