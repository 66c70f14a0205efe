// lut.hip — bf16/f16 activation as a gather through the 65536-entry table
// (the device form of unary_lut, crates/hologram-compute/src/cpu/lut.rs:76-98).
//
// Large inputs: one persistent workgroup per CU holds the whole 128 KiB table in LDS (gfx950
// gives a workgroup up to 160 KiB). Each thread issues its share of the table
// rows and its first input vectors together, so the table's L2 reads overlap
// the HBM reads; it looks up 8 patterns per vector in LDS and streams the
// results out as the vectors arrive. A workgroup's vectors are one contiguous
// span per pass (DRAM page locality). HBM traffic: 2 bytes read +
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

// A workgroup barrier over LDS only: each wave waits for its own LDS accesses
// (lgkmcnt 0), then s_barrier. __syncthreads() would also wait for every
// input load in flight, so no lookup could start before the last vector of
// the pass had landed.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));   // lgkmcnt(0); vmcnt, expcnt untouched
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Buffer resource over `bytes` bytes at `base` (at most 2^31): loads past the
// range read 0 and stores past it are dropped, so partial spans need no
// per-load branch (a branch around a load also makes the compiler wait for
// every load in flight at the join).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t span_rsrc(const void *base, uint64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, int(bytes), 0x00020000);
}

// TPB threads, VPT 16-byte vectors per thread per pass. A pass of a workgroup
// is TPB * VPT consecutive vectors; wave w owns the w-th run of 64 * VPT of
// them and lane l takes vectors l, l + 64, ... of that run, so each load
// instruction of a wave reads one contiguous KiB. nvec: vectors handled by the
// vector path (0 when the pointers are not both 16-byte aligned); elements
// [nvec*8, n) take the scalar tail.
//
// Order per thread: its share of the table's 16-byte rows, then its first
// pass's input vectors, all in flight together. The table rows come first in
// the load queue (and are L2 hits), so they go to LDS while the inputs are
// still arriving; after an LDS-only barrier each vector is looked up and
// stored as soon as it lands. Input loads use the normal cache policy and
// output stores the nontemporal one: on this part that pairing copies 32 MiB
// (read and written) in 11.3 us, against 12.4 us with both nontemporal and
// 13.0 us with neither.
template <int TPB, int VPT>
__global__ __launch_bounds__(TPB) void lut_gather_kernel(const uint16_t *__restrict__ table,
                                                        const uint16_t *__restrict__ in,
                                                        uint16_t *__restrict__ out, uint64_t n,
                                                        uint64_t nvec) {
    constexpr int kRows = 65536 * 2 / 16 / TPB;              // table rows per thread
    static_assert(kRows * TPB * 16 == 65536 * 2, "the table splits evenly over the threads");
    constexpr uint64_t kSpan = uint64_t(TPB) * VPT;          // vectors per workgroup pass
    static_assert(kSpan * 16 < (1u << 31), "a pass fits one buffer range");
    constexpr int kNt = 2;                                   // cache policy: nontemporal
    __shared__ u32x4 lds4[65536 * 2 / 16];
    const uint64_t pass = uint64_t(gridDim.x) * kSpan;
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int off = int((wave * 64 * VPT + lane) * 16);      // byte offset within the span

    const u32x4 *tab4 = reinterpret_cast<const u32x4 *>(table);
    u32x4 rows[kRows];
#pragma unroll
    for (int i = 0; i < kRows; ++i) rows[i] = tab4[threadIdx.x + i * TPB];
    // this workgroup's span of pass p starts at vector blk0
    auto span_bytes = [&](uint64_t blk0) -> uint64_t {
        const uint64_t left = nvec > blk0 ? nvec - blk0 : 0;
        return (left < kSpan ? left : kSpan) * 16;
    };
    uint64_t blk0 = uint64_t(blockIdx.x) * kSpan;
    uint64_t sb = span_bytes(blk0);
    auto ri = span_rsrc(reinterpret_cast<const u32x4 *>(in) + blk0, sb);
    auto ro = span_rsrc(reinterpret_cast<u32x4 *>(out) + blk0, sb);
    u32x4 v[VPT];
#pragma unroll
    for (int u = 0; u < VPT; ++u) v[u] = __builtin_amdgcn_raw_buffer_load_b128(ri, off, 1024 * u, 0);
#pragma unroll
    for (int i = 0; i < kRows; ++i) lds4[threadIdx.x + i * TPB] = rows[i];
    lds_barrier();
    const uint16_t *t = reinterpret_cast<const uint16_t *>(lds4);
#pragma unroll
    for (int u = 0; u < VPT; ++u)
        __builtin_amdgcn_raw_buffer_store_b128(look8(t, v[u]), ro, off, 1024 * u, kNt);

    for (blk0 += pass; blk0 < nvec; blk0 += pass) {   // inputs beyond one pass of the grid
        sb = span_bytes(blk0);
        ri = span_rsrc(reinterpret_cast<const u32x4 *>(in) + blk0, sb);
        ro = span_rsrc(reinterpret_cast<u32x4 *>(out) + blk0, sb);
#pragma unroll
        for (int u = 0; u < VPT; ++u) v[u] = __builtin_amdgcn_raw_buffer_load_b128(ri, off, 1024 * u, 0);
#pragma unroll
        for (int u = 0; u < VPT; ++u)
            __builtin_amdgcn_raw_buffer_store_b128(look8(t, v[u]), ro, off, 1024 * u, kNt);
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
