// holo_device.h — small device-side helpers shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace holo {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Streaming 16-byte load/store (non-temporal: the data is touched once).
__device__ __forceinline__ u32x4 ld_stream(const u32x4 *p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st_stream(u32x4 v, u32x4 *p) { __builtin_nontemporal_store(v, p); }

}  // namespace holo
