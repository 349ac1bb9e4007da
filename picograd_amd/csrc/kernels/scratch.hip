// Fixed device workspace of pg_amd_gemm_ex_noalloc: a file-scope array that
// every device the library runs on holds until the process ends, so that
// entry point allocates nothing (for callers under HIP graph capture or in
// loops that must not call hipMalloc).
//
// In host code `scratch` names a host-side stand-in, not device memory: it
// is never passed to a kernel or a copy.  pgk_noalloc_scratch_init asks the
// runtime for the array's address on the current device once per device
// (hipGetSymbolAddress) and keeps it; every use goes through that address.
// The library runs its work on one stream from one host thread, so calls
// that share the array are ordered on the stream; two callers that
// launched on the same device concurrently (the library is not thread-safe)
// would race on it.
#include <hip/hip_runtime.h>

#include "launch.h"

namespace {

constexpr size_t kNoallocScratchBytes = (size_t)32 << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

void *g_scratch_dev[kMaxDevices];

} // namespace

extern "C" size_t pgk_noalloc_scratch_bytes(void) { return kNoallocScratchBytes; }

extern "C" int pgk_noalloc_scratch_init(void)
{
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return (int)e;
    if (dev < 0 || dev >= kMaxDevices)
        return (int)hipErrorInvalidDevice;
    if (g_scratch_dev[dev])
        return 0;
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess)
        return (int)e;
    if (!p)
        return (int)hipErrorInvalidSymbol;
    g_scratch_dev[dev] = p;
    return 0;
}

extern "C" void *pgk_noalloc_scratch(void)
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return nullptr;
    if (!g_scratch_dev[dev] && pgk_noalloc_scratch_init() != 0)
        return nullptr;
    return g_scratch_dev[dev];
}
