// static_scratch.hip — the device scratch of the allocation-free entry point
// (holo_hip_dispatch_noalloc): a file-scope device array that every GPU the
// library runs on holds from module load until the process ends.
//
// In host code the array's name is only a stand-in for the symbol, not a
// device address, so nothing outside this file touches it: at backend
// creation, with the backend's device current, static_scratch_init() asks the
// runtime for this device's address of the array once and keeps it per
// device; every later use goes through static_scratch().
#include <hip/hip_runtime.h>

#include <mutex>

#include "holo_kernels.h"

static __device__ __align__(256) unsigned char scratch[holo::kStaticScratchBytes];

namespace holo {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void *g_ptr[kMaxDevices] = {};

}  // namespace

hipError_t static_scratch_init(int device) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    if (g_ptr[device]) return hipSuccess;
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_ptr[device] = p;
    return hipSuccess;
}

void *static_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_mu);
    return g_ptr[device];
}

}  // namespace holo
