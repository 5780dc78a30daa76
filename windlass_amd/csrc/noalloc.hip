// noalloc.hip — the library's static device scratch, used by the entry point
// that allocates nothing (wl_run_moe_batched_noalloc): callers under HIP graph
// capture or in loops that may not call hipMalloc get the batched layer's
// scratch from this array instead of a context allocation.
//
// `scratch` is a file-scope device array: every GPU the library runs on holds
// its own copy, at its own address, until the process ends. In host code the
// array's name is not a device address, so its address is looked up once per
// device (hipGetSymbolAddress, with that device current) and only that
// pointer is ever handed to kernels or copies.
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "internal.h"

namespace wl {

// 64 MiB: the batched layer's scratch for 169 tokens per chunk at the GLM shape
// (hidden 6144, inter 2048, 8 of 256 experts).
constexpr size_t kScratchBytes = 64ull << 20;

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
struct DevicePtr {
    int device;
    void* ptr;
};
std::mutex g_mu;
std::vector<DevicePtr> g_ptrs;
}  // namespace

int noalloc_scratch(int device, void** ptr) {
    std::lock_guard<std::mutex> lk(g_mu);
    for (const DevicePtr& d : g_ptrs)
        if (d.device == device) {
            *ptr = d.ptr;
            return 0;
        }
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) return e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
    g_ptrs.push_back({device, p});
    *ptr = p;
    return 0;
}

size_t noalloc_scratch_bytes() { return kScratchBytes; }

}  // namespace wl
