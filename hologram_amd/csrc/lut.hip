// lut.hip — bf16/f16 activation as a gather through the 65536-entry table
// (the device form of unary_lut, crates/hologram-compute/src/cpu/lut.rs:76-98).
//
// Large inputs: one persistent workgroup per CU holds the whole 128 KiB table in LDS (gfx950
// gives a workgroup up to 160 KiB). Each thread first issues the 16-byte loads
// of its first input vectors, then helps stage the table, so the table's L2
// reads overlap the HBM reads; after the barrier it looks up 8 patterns per
// vector in LDS and streams the results out. A workgroup's vectors are one
// contiguous span per pass (DRAM page locality). HBM traffic: 2 bytes read +
// 2 bytes written per element; the table adds one 128 KiB L2 read per CU.
#include <hip/hip_runtime.h>

#include <stdlib.h>

#include "holo_device.h"
#include "holo_kernels.h"

namespace holo {
namespace {

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

// TPB threads, VPT 16-byte vectors per thread per pass. nvec: vectors handled
// by the vector path (0 when the pointers are not both 16-byte aligned);
// elements [nvec*8, n) take the scalar tail.
template <int TPB, int VPT>
__global__ __launch_bounds__(TPB) void lut_gather_kernel(const uint16_t *__restrict__ table,
                                                        const uint16_t *__restrict__ in,
                                                        uint16_t *__restrict__ out, uint64_t n,
                                                        uint64_t nvec) {
    __shared__ u32x4 lds4[65536 * 2 / 16];
    const u32x4 *in4 = reinterpret_cast<const u32x4 *>(in);
    u32x4 *out4 = reinterpret_cast<u32x4 *>(out);
    constexpr uint64_t kSpan = uint64_t(TPB) * VPT;          // vectors per workgroup pass
    const uint64_t pass = uint64_t(gridDim.x) * kSpan;

    uint64_t base = blockIdx.x * kSpan + threadIdx.x;
    u32x4 v[VPT];
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
        const uint64_t i = base + uint64_t(u) * TPB;
        if (i < nvec) v[u] = ld_stream(&in4[i]);
    }
    const u32x4 *tab4 = reinterpret_cast<const u32x4 *>(table);
#pragma unroll
    for (int i = 0; i < 65536 * 2 / 16 / TPB; ++i) lds4[threadIdx.x + i * TPB] = tab4[threadIdx.x + i * TPB];
    __syncthreads();
    const uint16_t *t = reinterpret_cast<const uint16_t *>(lds4);

    while (base < nvec) {
        const uint64_t next = base + pass;
        u32x4 w[VPT];
#pragma unroll
        for (int u = 0; u < VPT; ++u) {   // next pass's loads go out before this pass's stores
            const uint64_t i = next + uint64_t(u) * TPB;
            if (i < nvec) w[u] = ld_stream(&in4[i]);
        }
#pragma unroll
        for (int u = 0; u < VPT; ++u) {
            const uint64_t i = base + uint64_t(u) * TPB;
            if (i < nvec) st_stream(look8(t, v[u]), &out4[i]);
        }
#pragma unroll
        for (int u = 0; u < VPT; ++u) v[u] = w[u];
        base = next;
    }
    for (uint64_t e = nvec * 8 + uint64_t(blockIdx.x) * TPB + threadIdx.x; e < n;
         e += uint64_t(gridDim.x) * TPB)
        out[e] = t[in[e]];
}

// Few elements: staging the 128 KiB table in LDS costs more than the whole
// gather, and a persistent grid would be a handful of workgroups. Each thread
// takes one 16-byte vector and looks its 8 patterns up in the table in global
// memory (L2-resident after the first touches).
__global__ __launch_bounds__(256) void lut_direct_kernel(const uint16_t *__restrict__ table,
                                                         const uint16_t *__restrict__ in,
                                                         uint16_t *__restrict__ out, uint64_t n,
                                                         uint64_t nvec) {
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i < nvec) reinterpret_cast<u32x4 *>(out)[i] = look8(table, reinterpret_cast<const u32x4 *>(in)[i]);
    const uint64_t e = nvec * 8 + i;              // the n % 8 tail, one element per thread
    if (i < 8 && e < n) out[e] = table[in[e]];
}

int cu_count() {
    static const int cus = [] {
        int dev = 0, c = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
            c = 256;
        return c;
    }();
    return cus;
}

template <int TPB, int VPT>
hipError_t launch(const uint16_t *table, const uint16_t *in, uint16_t *out, uint64_t n,
                  uint64_t nvec, hipStream_t stream) {
    // one workgroup per CU at most (the table fills the CU's LDS)
    const uint64_t work = nvec ? (nvec + uint64_t(TPB) * VPT - 1) / (uint64_t(TPB) * VPT)
                               : (n + TPB - 1) / TPB;
    uint64_t blocks = work < uint64_t(cu_count()) ? work : uint64_t(cu_count());
    if (blocks == 0) blocks = 1;
    hipLaunchKernelGGL((lut_gather_kernel<TPB, VPT>), dim3(unsigned(blocks)), dim3(TPB), 0, stream,
                       table, in, out, n, nvec);
    return hipGetLastError();
}

}  // namespace

// Up to this many 16-byte vectors (2M elements) the direct kernel runs.
constexpr uint64_t kDirectMaxVec = 256 * 1024;

hipError_t launch_lut_u16(const uint16_t *table, const uint16_t *in, uint16_t *out, uint64_t n,
                          hipStream_t stream) {
    if (n == 0) return hipSuccess;
    const bool aligned = ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    const uint64_t nvec = aligned ? n / 8 : 0;
    if (nvec && nvec <= kDirectMaxVec) {
        hipLaunchKernelGGL(lut_direct_kernel, dim3(unsigned((nvec + 255) / 256)), dim3(256), 0,
                           stream, table, in, out, n, nvec);
        return hipGetLastError();
    }
    return launch<1024, 8>(table, in, out, n, nvec, stream);
}

}  // namespace holo
