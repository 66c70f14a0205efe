// kv.hip — KV-cache kernels: the honest-copy byte stream, KvCacheWrite's ring
// row placement (crates/hologram-compute/src/cpu/kernels.rs:455-501), and the
// int8 quantize+append that applies quantize_row_i8
// (src/cpu/simd.rs:4755-4785) to each appended row on the device.
//
// The write position `pos` is content: a device-resident 4-byte u32 read by
// the kernels themselves, so a decode step never syncs to the host for it.
#include <hip/hip_runtime.h>

#include "holo_device.h"
#include "holo_kernels.h"

namespace holo {
namespace {

constexpr int kCopyThreads = 256;

// 16-byte copy: a workgroup takes runs of kCopyThreads * kCopyVec vectors, each
// thread kCopyVec of them kCopyThreads apart, all loads issued before the
// stores. Loads use the normal cache policy and stores the nontemporal one:
// on this part that pairing, with enough workgroups for one run each, copies
// 32 MiB in 11.3 us, against 12.2-13.4 us for a grid-stride loop with both
// nontemporal.
constexpr int kCopyVec = 4;
constexpr uint64_t kCopyRun = uint64_t(kCopyThreads) * kCopyVec;

__global__ __launch_bounds__(kCopyThreads) void copy16_kernel(const u32x4 *__restrict__ src,
                                                             u32x4 *__restrict__ dst, uint64_t nvec) {
    for (uint64_t c = uint64_t(blockIdx.x) * kCopyRun + threadIdx.x; c < nvec;
         c += uint64_t(gridDim.x) * kCopyRun) {
        u32x4 v[kCopyVec];
#pragma unroll
        for (int u = 0; u < kCopyVec; ++u) {
            const uint64_t i = c + uint64_t(u) * kCopyThreads;
            if (i < nvec) v[u] = src[i];
        }
#pragma unroll
        for (int u = 0; u < kCopyVec; ++u) {
            const uint64_t i = c + uint64_t(u) * kCopyThreads;
            if (i < nvec) st_stream(v[u], &dst[i]);
        }
    }
}

unsigned copy16_blocks(uint64_t nvec) {
    const uint64_t b = (nvec + kCopyRun - 1) / kCopyRun;
    return unsigned(b < (1u << 24) ? (b ? b : 1) : (1u << 24));
}

__global__ __launch_bounds__(kCopyThreads) void copy1_kernel(const uint8_t *__restrict__ src,
                                                            uint8_t *__restrict__ dst, uint64_t n) {
    const uint64_t stride = uint64_t(gridDim.x) * kCopyThreads;
    for (uint64_t i = uint64_t(blockIdx.x) * kCopyThreads + threadIdx.x; i < n; i += stride)
        dst[i] = src[i];
}

__global__ __launch_bounds__(kCopyThreads) void zero1_kernel(uint8_t *__restrict__ dst, uint64_t n) {
    const uint64_t stride = uint64_t(gridDim.x) * kCopyThreads;
    for (uint64_t i = uint64_t(blockIdx.x) * kCopyThreads + threadIdx.x; i < n; i += stride) dst[i] = 0;
}

unsigned copy_blocks(uint64_t items) {
    uint64_t b = (items + kCopyThreads - 1) / kCopyThreads;
    const uint64_t cap = 256 * 16;  // 16 workgroups per CU, grid-stride beyond
    if (b > cap) b = cap;
    return unsigned(b ? b : 1);
}

// One workgroup per (plane, new row): out[p][(pos + j) % bucket] = new[p][j].
__global__ __launch_bounds__(kCopyThreads) void place_rows_kernel(const uint8_t *__restrict__ nw,
                                                                 const uint32_t *__restrict__ posp,
                                                                 uint8_t *__restrict__ out,
                                                                 uint32_t bucket, uint32_t new_rows,
                                                                 uint32_t row_bytes) {
    const uint32_t p = blockIdx.x / new_rows, j = blockIdx.x % new_rows;
    const uint64_t pos = *posp % bucket;
    const uint64_t dst = (uint64_t(p) * bucket + (pos + j) % bucket) * row_bytes;
    const uint64_t src = (uint64_t(p) * new_rows + j) * row_bytes;
    for (uint32_t c = threadIdx.x; c < row_bytes; c += kCopyThreads) out[dst + c] = nw[src + c];
}

__device__ __forceinline__ float widen16(uint32_t b, uint8_t dtype);

__device__ __forceinline__ float widen(const void *base, uint8_t dtype, uint64_t i) {
    if (dtype == 8) return reinterpret_cast<const float *>(base)[i];
    return widen16(reinterpret_cast<const uint16_t *>(base)[i], dtype);
}

// A 16-bit element (bf16, else f16) widened to f32.
__device__ __forceinline__ float widen16(uint32_t b, uint8_t dtype) {
    if (dtype == 7) return __uint_as_float(b << 16);
    // f16 -> f32 by bits, as src/cpu/dtype.rs:94-118 (exact; NaN payload kept)
    const uint32_t s = (b >> 15) << 31, e = (b >> 10) & 0x1fu, m = b & 0x3ffu;
    if (e == 0x1fu) return __uint_as_float(s | 0x7f800000u | (m << 13));
    if (e != 0) return __uint_as_float(s | ((e + 112u) << 23) | (m << 13));
    if (m == 0) return __uint_as_float(s);
    const int sh = __clz(m) - 21;  // left shifts until the implicit bit (0x400) is set
    return __uint_as_float(s | (uint32_t(113 - sh) << 23) | (((m << sh) & 0x3ffu) << 13));
}

// Rust's `f32 as i32` then clamp(-127, 127): NaN -> 0; any out-of-range value
// saturates, so clamping in the float domain first gives the same integer.
__device__ __forceinline__ int8_t to_q(float r) {
    if (r != r) return 0;
    r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
    return static_cast<int8_t>(static_cast<int32_t>(r));
}

// One wavefront per (plane, new row). The row max is a wave reduction of
// |x| (NaN never wins a `>` comparison, as in the reference's scan; max is
// exact, so the order of the reduction does not matter). Divisions are the
// correctly rounded IEEE ones and the file is built without contraction, so
// t = x * inv and t +- 0.5 round exactly as the reference's two steps.
template <int kMaxPerLane>
__device__ __forceinline__ void quant_row_wave(const void *__restrict__ nw, uint8_t dtype,
                                               uint64_t pos, int8_t *__restrict__ cq,
                                               float *__restrict__ cs, uint32_t wave,
                                               uint32_t lane, uint32_t bucket, uint32_t new_rows,
                                               uint32_t d) {
    const uint32_t p = wave / new_rows, j = wave % new_rows;
    const uint64_t row = uint64_t(p) * bucket + (pos + j) % bucket;
    const uint64_t src = (uint64_t(p) * new_rows + j) * d;

    float x[kMaxPerLane];
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < kMaxPerLane; ++e) {
        const uint32_t c = lane + 64u * e;
        x[e] = c < d ? widen(nw, dtype, src + c) : 0.0f;
        const float v = x[e];
        const float av = v < 0.0f ? -v : v;
        if (av > amax) amax = av;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(amax, off, 64);
        if (o > amax) amax = o;
    }
    int8_t *dst = cq + row * d;
    if (amax == 0.0f) {
#pragma unroll
        for (int e = 0; e < kMaxPerLane; ++e) {
            const uint32_t c = lane + 64u * e;
            if (c < d) dst[c] = 0;
        }
        if (lane == 0) cs[row] = 0.0f;
        return;
    }
    const float inv = 127.0f / amax;
#pragma unroll
    for (int e = 0; e < kMaxPerLane; ++e) {
        const uint32_t c = lane + 64u * e;
        if (c < d) {
            const float t = x[e] * inv;
            const float r = t >= 0.0f ? truncf(t + 0.5f) : truncf(t - 0.5f);
            dst[c] = to_q(r);
        }
    }
    if (lane == 0) cs[row] = amax / 127.0f;
}

template <int kMaxPerLane>
__global__ __launch_bounds__(256) void quant_append_kernel(const void *__restrict__ nw, uint8_t dtype,
                                                          const uint32_t *__restrict__ posp,
                                                          int8_t *__restrict__ cq,
                                                          float *__restrict__ cs, uint32_t planes,
                                                          uint32_t bucket, uint32_t new_rows,
                                                          uint32_t d) {
    const uint32_t wave = (blockIdx.x * 256u + threadIdx.x) >> 6;
    if (wave >= planes * new_rows) return;
    quant_row_wave<kMaxPerLane>(nw, dtype, *posp % bucket, cq, cs, wave, threadIdx.x & 63u, bucket,
                                new_rows, d);
}

// The same quantization for 16-bit rows of d = 8 kL elements (64 or 128):
// kL lanes a row, eight elements a lane from one 16-byte load, the row max
// over the kL lanes, eight int8 values stored at once.
template <uint32_t kL>
__global__ __launch_bounds__(256) void quant_append_vec_kernel(const u32x4 *__restrict__ nw,
                                                              uint8_t dtype,
                                                              const uint32_t *__restrict__ posp,
                                                              int8_t *__restrict__ cq,
                                                              float *__restrict__ cs, uint32_t planes,
                                                              uint32_t bucket, uint32_t new_rows) {
    constexpr uint32_t d = 8 * kL;
    const uint64_t t = uint64_t(blockIdx.x) * 256u + threadIdx.x;
    const uint64_t r = t / kL;
    const uint32_t c = uint32_t(t % kL);
    const bool live = r < uint64_t(planes) * new_rows;
    const u32x4 v = live ? nw[t] : u32x4{0u, 0u, 0u, 0u};
    float x[8];
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        x[e] = widen16((v[e / 2] >> ((e & 1) * 16)) & 0xffffu, dtype);
        const float av = x[e] < 0.0f ? -x[e] : x[e];
        if (av > amax) amax = av;
    }
#pragma unroll
    for (uint32_t off = kL / 2; off >= 1; off >>= 1) {
        const float o = __shfl_xor(amax, int(off), 64);
        if (o > amax) amax = o;
    }
    if (!live) return;
    const uint32_t p = uint32_t(r / new_rows), j = uint32_t(r % new_rows);
    const uint64_t row = uint64_t(p) * bucket + (uint64_t(*posp % bucket) + j) % bucket;
    uint32_t lo = 0, hi = 0;
    if (amax != 0.0f) {
        const float inv = 127.0f / amax;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float q = x[e] * inv;
            const float rq = q >= 0.0f ? truncf(q + 0.5f) : truncf(q - 0.5f);
            const uint32_t by = uint32_t(uint8_t(to_q(rq))) << (8 * (e & 3));
            if (e < 4) lo |= by; else hi |= by;
        }
    }
    reinterpret_cast<uint2 *>(cq + row * d)[c] = make_uint2(lo, hi);
    if (c == 0) cs[row] = amax == 0.0f ? 0.0f : amax / 127.0f;
}

// Buffer resource over `bytes` bytes (< 2^31) at `base`: loads past the range
// read 0 and stores past it are dropped, so a skipped store is an offset out
// of range rather than a branch (a branch around memory operations makes the
// compiler wait for every load in flight where it joins).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, int(bytes), 0x00020000);
}

// The copy form of KvQuantAppend in one launch: the int8 planes and the scale
// planes are copied to the outputs, except the rows being appended, which
// the first workgroups quantize and place (one wavefront per new row, the
// arithmetic above). No byte is written twice, so the three parts need no
// order among themselves. Block roles, in block order:
//   [0, qblocks)                      quantize + place the new rows
//   [qblocks, + planes * runs)        int8 plane p, run r: kCopyRun vectors
//   [.., + scale runs)                the scale planes, flat, 4 rows a vector
// Requires d % 16 == 0, bucket % 4 == 0, 16-byte aligned caches and planes
// under 2 GiB, so a 16-byte int8 vector lies in one row, a scale vector in
// one plane, and a plane is one buffer range. vshift: log2(d / 16) when d / 16
// is a power of two, else -1 (divide).
constexpr uint32_t kNoStore = 0x80000000u;   // past every range below

template <int kMaxPerLane>
__global__ __launch_bounds__(kCopyThreads) void quant_copy_append_kernel(
    const void *__restrict__ nw, uint8_t dtype, const uint32_t *__restrict__ posp,
    const u32x4 *__restrict__ cq, const u32x4 *__restrict__ cs, int8_t *__restrict__ oq,
    float *__restrict__ os, uint32_t planes, uint32_t bucket, uint32_t new_rows, uint32_t d,
    uint32_t qblocks, uint32_t runs, uint32_t plane_vecs, uint32_t scale_vecs, int vshift) {
    uint32_t bid = blockIdx.x;
    if (bid < qblocks) {
        const uint32_t wave = bid * 4u + (threadIdx.x >> 6);
        if (wave < planes * new_rows)
            quant_row_wave<kMaxPerLane>(nw, dtype, *posp % bucket, oq, os, wave, threadIdx.x & 63u,
                                        bucket, new_rows, d);
        return;
    }
    bid -= qblocks;
    const uint32_t pos = *posp % bucket;
    // row r of a plane is being appended when (r - pos) mod bucket < new_rows
    auto appended = [&](uint32_t r) { return (r >= pos ? r - pos : r + bucket - pos) < new_rows; };
    if (bid < planes * runs) {
        const uint32_t p = bid / runs;
        const uint32_t v0 = (bid % runs) * uint32_t(kCopyRun) + threadIdx.x;
        const auto rs = rsrc_of(cq + uint64_t(p) * plane_vecs, plane_vecs * 16u);
        const auto rd = rsrc_of(reinterpret_cast<u32x4 *>(oq) + uint64_t(p) * plane_vecs,
                                plane_vecs * 16u);
        u32x4 v[kCopyVec];
#pragma unroll
        for (int u = 0; u < kCopyVec; ++u)
            v[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, 16u * (v0 + uint32_t(u) * kCopyThreads),
                                                         0, 0);
        const uint32_t vpr = d / 16;
#pragma unroll
        for (int u = 0; u < kCopyVec; ++u) {
            const uint32_t i = v0 + uint32_t(u) * kCopyThreads;
            const uint32_t row = vshift >= 0 ? i >> vshift : i / vpr;
            __builtin_amdgcn_raw_buffer_store_b128(v[u], rd, appended(row) ? kNoStore : 16u * i, 0, 2);
        }
        return;
    }
    bid -= planes * runs;
    const uint32_t v0 = bid * uint32_t(kCopyRun) + threadIdx.x;
    const auto rs = rsrc_of(cs, scale_vecs * 16u), rd = rsrc_of(os, scale_vecs * 16u);
    u32x4 v[kCopyVec];
#pragma unroll
    for (int u = 0; u < kCopyVec; ++u)
        v[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, 16u * (v0 + uint32_t(u) * kCopyThreads), 0, 0);
#pragma unroll
    for (int u = 0; u < kCopyVec; ++u) {
        const uint32_t i = v0 + uint32_t(u) * kCopyThreads;
        const uint32_t r0 = (4u * i) % bucket;          // the vector's rows r0 .. r0 + 3
        bool a[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) a[e] = appended(r0 + uint32_t(e));
        const bool any = a[0] || a[1] || a[2] || a[3];
        // whole vector when no row of it is appended, else its other rows one by one
        __builtin_amdgcn_raw_buffer_store_b128(v[u], rd, any ? kNoStore : 16u * i, 0, 2);
#pragma unroll
        for (int e = 0; e < 4; ++e)
            __builtin_amdgcn_raw_buffer_store_b32(v[u][e], rd,
                                                  any && !a[e] ? 16u * i + 4u * e : kNoStore, 0, 0);
    }
}

}  // namespace

hipError_t launch_copy_bytes(const void *src, void *dst, uint64_t bytes, hipStream_t stream) {
    if (bytes == 0) return hipSuccess;
    const bool aligned =
        ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0;
    if (aligned) {
        const uint64_t nvec = bytes / 16, tail = bytes - nvec * 16;
        if (nvec)
            hipLaunchKernelGGL(copy16_kernel, dim3(copy16_blocks(nvec)), dim3(kCopyThreads), 0, stream,
                               static_cast<const u32x4 *>(src), static_cast<u32x4 *>(dst), nvec);
        if (tail)
            hipLaunchKernelGGL(copy1_kernel, dim3(1), dim3(kCopyThreads), 0, stream,
                               static_cast<const uint8_t *>(src) + nvec * 16,
                               static_cast<uint8_t *>(dst) + nvec * 16, tail);
    } else {
        hipLaunchKernelGGL(copy1_kernel, dim3(copy_blocks(bytes)), dim3(kCopyThreads), 0, stream,
                           static_cast<const uint8_t *>(src), static_cast<uint8_t *>(dst), bytes);
    }
    return hipGetLastError();
}

hipError_t launch_fill_zero(void *dst, uint64_t bytes, hipStream_t stream) {
    if (bytes == 0) return hipSuccess;
    hipLaunchKernelGGL(zero1_kernel, dim3(copy_blocks(bytes)), dim3(kCopyThreads), 0, stream,
                       static_cast<uint8_t *>(dst), bytes);
    return hipGetLastError();
}

hipError_t launch_kv_place_rows(const uint8_t *nw, const uint32_t *pos, uint8_t *out, uint32_t planes,
                                uint32_t bucket, uint32_t new_rows, uint32_t row_bytes,
                                hipStream_t stream) {
    const uint64_t blocks = uint64_t(planes) * new_rows;
    if (blocks == 0) return hipSuccess;
    if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
    hipLaunchKernelGGL(place_rows_kernel, dim3(unsigned(blocks)), dim3(kCopyThreads), 0, stream, nw,
                       pos, out, bucket, new_rows, row_bytes);
    return hipGetLastError();
}

bool kv_quant_copy_fusable(const void *cq, const void *cs, const void *oq, const void *os,
                           uint32_t planes, uint32_t bucket, uint32_t d) {
    const uintptr_t al = reinterpret_cast<uintptr_t>(cq) | reinterpret_cast<uintptr_t>(cs) |
                         reinterpret_cast<uintptr_t>(oq) | reinterpret_cast<uintptr_t>(os);
    return (al & 15) == 0 && d % 16 == 0 && d != 0 && d <= 8192 && bucket % 4 == 0 &&
           uint64_t(bucket) * d < (1ull << 31) && uint64_t(planes) * bucket * 4 < (1ull << 31);
}

hipError_t launch_kv_quant_copy_append(const void *nw, uint8_t dtype, const uint32_t *pos,
                                       const int8_t *cq, const float *cs, int8_t *oq, float *os,
                                       uint32_t planes, uint32_t bucket, uint32_t new_rows,
                                       uint32_t d, hipStream_t stream) {
    if (!kv_quant_copy_fusable(cq, cs, oq, os, planes, bucket, d)) return hipErrorInvalidValue;
    if (planes == 0) return hipSuccess;
    const uint32_t plane_vecs = bucket * (d / 16);
    const uint32_t runs = uint32_t((plane_vecs + kCopyRun - 1) / kCopyRun);
    const uint32_t vpr = d / 16;
    const int vshift = (vpr & (vpr - 1)) == 0 ? __builtin_ctz(vpr) : -1;
    const uint32_t scale_vecs = planes * (bucket / 4);
    const uint64_t qblocks = (uint64_t(planes) * new_rows + 3) / 4;
    const uint64_t sblocks = (scale_vecs + kCopyRun - 1) / kCopyRun;
    const uint64_t blocks = qblocks + uint64_t(planes) * runs + sblocks;
    if (blocks > 0x7fffffffull || uint64_t(planes) * new_rows > 0xffffffffull / 64)
        return hipErrorInvalidValue;
    const auto *q4 = reinterpret_cast<const u32x4 *>(cq);
    const auto *s4 = reinterpret_cast<const u32x4 *>(cs);
#define HOLO_QCA(K)                                                                              \
    hipLaunchKernelGGL(quant_copy_append_kernel<K>, dim3(unsigned(blocks)), dim3(kCopyThreads), 0, \
                       stream, nw, dtype, pos, q4, s4, oq, os, planes, bucket, new_rows, d,       \
                       uint32_t(qblocks), runs, plane_vecs, scale_vecs, vshift)
    if (d <= 128) HOLO_QCA(2);
    else if (d <= 512) HOLO_QCA(8);
    else if (d <= 2048) HOLO_QCA(32);
    else HOLO_QCA(128);
#undef HOLO_QCA
    return hipGetLastError();
}

hipError_t launch_kv_quant_append(const void *nw, uint8_t dtype, const uint32_t *pos, int8_t *cq,
                                  float *cs, uint32_t planes, uint32_t bucket, uint32_t new_rows,
                                  uint32_t d, hipStream_t stream) {
    const uint64_t waves = uint64_t(planes) * new_rows;
    if (waves == 0) return hipSuccess;
    const uint64_t blocks = (waves + 3) / 4;
    if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
    const dim3 g{unsigned(blocks), 1, 1}, b{256, 1, 1};
    if (dtype != 8 && (d == 64 || d == 128) && (reinterpret_cast<uintptr_t>(nw) & 15) == 0 &&
        (reinterpret_cast<uintptr_t>(cq) & 7) == 0) {
        const uint64_t vblocks = (waves * (d / 8) + 255) / 256;
        if (vblocks > 0x7fffffffull) return hipErrorInvalidValue;
        if (d == 64)
            hipLaunchKernelGGL(quant_append_vec_kernel<8>, dim3(unsigned(vblocks)), b, 0, stream,
                               static_cast<const u32x4 *>(nw), dtype, pos, cq, cs, planes, bucket, new_rows);
        else
            hipLaunchKernelGGL(quant_append_vec_kernel<16>, dim3(unsigned(vblocks)), b, 0, stream,
                               static_cast<const u32x4 *>(nw), dtype, pos, cq, cs, planes, bucket, new_rows);
        return hipGetLastError();
    }
    if (d <= 128)
        hipLaunchKernelGGL(quant_append_kernel<2>, g, b, 0, stream, nw, dtype, pos, cq, cs, planes,
                           bucket, new_rows, d);
    else if (d <= 512)
        hipLaunchKernelGGL(quant_append_kernel<8>, g, b, 0, stream, nw, dtype, pos, cq, cs, planes,
                           bucket, new_rows, d);
    else if (d <= 2048)
        hipLaunchKernelGGL(quant_append_kernel<32>, g, b, 0, stream, nw, dtype, pos, cq, cs, planes,
                           bucket, new_rows, d);
    else if (d <= 8192)
        hipLaunchKernelGGL(quant_append_kernel<128>, g, b, 0, stream, nw, dtype, pos, cq, cs, planes,
                           bucket, new_rows, d);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace holo
