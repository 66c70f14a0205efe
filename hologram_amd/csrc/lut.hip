// lut.hip — bf16/f16 activation as a gather through the 65536-entry table
// (the device form of unary_lut, crates/hologram-compute/src/cpu/lut.rs:76-98).
//
// Every workgroup first stages the whole 128 KiB table in LDS (gfx950 gives a
// workgroup up to 160 KiB), then streams the input with 16-byte loads and
// stores: 8 patterns per load, 8 LDS lookups, one 16-byte store. The grid is
// one workgroup per CU, persistent, so the table is staged 256 times (32 MiB
// of L2/MALL reads) for any n. HBM traffic is 2 bytes read + 2 bytes written
// per element.
#include <hip/hip_runtime.h>

#include "holo_device.h"
#include "holo_kernels.h"

namespace holo {
namespace {

constexpr int kThreads = 1024;
constexpr int kUnroll = 4;  // 16-byte vectors in flight per thread

__device__ __forceinline__ uint32_t look2(const uint16_t *t, uint32_t w) {
    return static_cast<uint32_t>(t[w & 0xffffu]) | (static_cast<uint32_t>(t[w >> 16]) << 16);
}

__device__ __forceinline__ u32x4 look8(const uint16_t *t, u32x4 v) {
    u32x4 r;
    r.x = look2(t, v.x);
    r.y = look2(t, v.y);
    r.z = look2(t, v.z);
    r.w = look2(t, v.w);
    return r;
}

// nvec: number of 16-byte vectors handled by the vector loop (0 when the
// pointers are not both 16-byte aligned); elements [nvec*8, n) take the
// scalar loop.
__global__ __launch_bounds__(kThreads) void lut_gather_kernel(const uint16_t *__restrict__ table,
                                                             const uint16_t *__restrict__ in,
                                                             uint16_t *__restrict__ out,
                                                             uint64_t n, uint64_t nvec) {
    __shared__ u32x4 lds4[65536 * 2 / 16];
    const u32x4 *tab4 = reinterpret_cast<const u32x4 *>(table);
#pragma unroll
    for (int i = 0; i < 65536 * 2 / 16 / kThreads; ++i)
        lds4[threadIdx.x + i * kThreads] = tab4[threadIdx.x + i * kThreads];
    __syncthreads();
    const uint16_t *t = reinterpret_cast<const uint16_t *>(lds4);

    const u32x4 *in4 = reinterpret_cast<const u32x4 *>(in);
    u32x4 *out4 = reinterpret_cast<u32x4 *>(out);
    const uint64_t stride = uint64_t(gridDim.x) * kThreads;
    uint64_t i = uint64_t(blockIdx.x) * kThreads + threadIdx.x;
    // main loop: kUnroll independent 16-byte loads before any lookup
    for (; i + (kUnroll - 1) * stride < nvec; i += kUnroll * stride) {
        u32x4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) v[u] = ld_stream(&in4[i + u * stride]);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) st_stream(look8(t, v[u]), &out4[i + u * stride]);
    }
    for (; i < nvec; i += stride) out4[i] = look8(t, in4[i]);
    for (uint64_t e = nvec * 8 + uint64_t(blockIdx.x) * kThreads + threadIdx.x; e < n; e += stride)
        out[e] = t[in[e]];
}

}  // namespace

hipError_t launch_lut_u16(const uint16_t *table, const uint16_t *in, uint16_t *out, uint64_t n,
                          hipStream_t stream) {
    if (n == 0) return hipSuccess;
    const bool aligned = ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    const uint64_t nvec = aligned ? n / 8 : 0;
    int dev = 0, cus = 256;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    // one persistent workgroup per CU; fewer when n is small
    const uint64_t work = aligned ? nvec : n;
    uint64_t blocks = (work + kThreads - 1) / kThreads;
    if (blocks > uint64_t(cus)) blocks = cus;
    if (blocks == 0) blocks = 1;
    hipLaunchKernelGGL(lut_gather_kernel, dim3(unsigned(blocks)), dim3(kThreads), 0, stream, table,
                       in, out, n, nvec);
    return hipGetLastError();
}

}  // namespace holo
