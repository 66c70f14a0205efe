// decoder_ops.hip — the remaining ops of a Llama-style decode step on the
// device: Add / Mul, RmsNorm, rotary embedding, Gather (embedding rows) and
// ArgMax (the greedy pick). Each is memory-bound at decode shapes; each keeps
// the reference's per-element arithmetic (widen to f32, the same IEEE
// operations in the same order, narrow bf16 by truncation), so Add, Mul, RoPE
// and Gather are bit-exact with the reference CPU kernels, and RmsNorm differs
// only by the order of its sum of squares (a tree here, sequential there).
#include <hip/hip_runtime.h>
#include <type_traits>

#include <math.h>

#include "holo_device.h"
#include "holo_kernels.h"

namespace holo {
namespace {

__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) { return uint16_t(__float_as_uint(f) >> 16); }

// Element access by dtype tag (f16 6, bf16 7, f32 8): widen exactly; narrow
// bf16 by truncation and f16 by the reference's rounding (read_float /
// write_float, src/cpu/dtype.rs:69-153).
constexpr int kF16 = 6, kBF16 = 7, kF32 = 8;

template <int DT>
__device__ __forceinline__ float wid(uint32_t h) {
    return DT == kBF16 ? bf2f(uint16_t(h)) : f16_bits_to_f32(h);
}
template <int DT>
__device__ __forceinline__ uint32_t nar(float v) {
    return DT == kBF16 ? f2bf(v) : f32_to_f16_bits(v);
}

template <int DT>
__device__ __forceinline__ float ld(const void *p, uint64_t i) {
    if constexpr (DT == kF32)
        return static_cast<const float *>(p)[i];
    else
        return wid<DT>(static_cast<const uint16_t *>(p)[i]);
}

template <int DT>
__device__ __forceinline__ void st(void *p, uint64_t i, float v) {
    if constexpr (DT == kF32)
        static_cast<float *>(p)[i] = v;
    else
        static_cast<uint16_t *>(p)[i] = uint16_t(nar<DT>(v));
}

constexpr int kOpAdd = 0, kOpMul = 1;

template <int kOp>
__device__ __forceinline__ float bin(float a, float b) {
    return kOp == kOpAdd ? a + b : a * b;
}

// Add / Mul: 16-byte vectors (8 bf16/f16 or 4 f32 per lane) when every
// operand is 16-byte aligned, element tail after; grid-stride.
template <int DT, int kOp>
__global__ __launch_bounds__(256) void binary_kernel(const void *__restrict__ a,
                                                     const void *__restrict__ b,
                                                     void *__restrict__ out, uint64_t n,
                                                     uint64_t nvec) {
    constexpr int E = DT == kF32 ? 4 : 8;
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    const u32x4 *a4 = static_cast<const u32x4 *>(a);
    const u32x4 *b4 = static_cast<const u32x4 *>(b);
    u32x4 *o4 = static_cast<u32x4 *>(out);
    for (uint64_t v = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; v < nvec; v += stride) {
        const u32x4 x = a4[v], y = b4[v];
        u32x4 r;
        if constexpr (DT == kBF16) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float lo = bin<kOp>(__uint_as_float(x[w] << 16), __uint_as_float(y[w] << 16));
                const float hi = bin<kOp>(__uint_as_float(x[w] & 0xFFFF0000u),
                                          __uint_as_float(y[w] & 0xFFFF0000u));
                r[w] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
            }
        } else if constexpr (DT == kF16) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const float lo = bin<kOp>(wid<DT>(x[w] & 0xFFFFu), wid<DT>(y[w] & 0xFFFFu));
                const float hi = bin<kOp>(wid<DT>(x[w] >> 16), wid<DT>(y[w] >> 16));
                r[w] = nar<DT>(lo) | (nar<DT>(hi) << 16);
            }
        } else {
#pragma unroll
            for (int w = 0; w < 4; ++w)
                r[w] = __float_as_uint(bin<kOp>(__uint_as_float(x[w]), __uint_as_float(y[w])));
        }
        o4[v] = r;
    }
    for (uint64_t i = nvec * E + uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        st<DT>(out, i, bin<kOp>(ld<DT>(a, i), ld<DT>(b, i)));
}

// RmsNorm: one workgroup per row. Sum of squares in f32 (tree order), then
// out = (x * inv_rms) * gamma as the reference evaluates it.
template <int DT>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const void *__restrict__ x,
                                                      const void *__restrict__ gamma,
                                                      void *__restrict__ out, uint32_t feature,
                                                      float eps) {
    __shared__ float part[8];
    const uint64_t row = uint64_t(blockIdx.x) * feature;
    float ss = 0.0f;
    for (uint32_t j = threadIdx.x; j < feature; j += 256) {
        const float v = ld<DT>(x, row + j);
        ss = fmaf(v, v, ss);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float sumsq = part[0] + part[1] + part[2] + part[3];
    const float inv = 1.0f / sqrtf(sumsq / float(feature) + eps);
    for (uint32_t j = threadIdx.x; j < feature; j += 256) {
        float v = ld<DT>(x, row + j) * inv;
        if (gamma) v = v * ld<DT>(gamma, j);
        st<DT>(out, row + j, v);
    }
}

// AddRmsNorm: one workgroup per row over v = x + residual, the sum taken in
// f32 and never narrowed (add_rms_norm_float, float_kernels.rs:1566-1672).
// The reference's f32 rows with a residual scale in place by (inv * g); every
// other form writes (v * inv) * g; the sum of squares is in tree order.
template <int DT>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(const void *__restrict__ x,
                                                          const void *__restrict__ res,
                                                          const void *__restrict__ gamma,
                                                          void *__restrict__ out, uint32_t feature,
                                                          float eps) {
    __shared__ float part[4];
    const uint64_t row = uint64_t(blockIdx.x) * feature;
    float ss = 0.0f;
    for (uint32_t j = threadIdx.x; j < feature; j += 256) {
        float v = ld<DT>(x, row + j);
        if (res) v = v + ld<DT>(res, row + j);
        ss = fmaf(v, v, ss);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float sumsq = part[0] + part[1] + part[2] + part[3];
    const float inv = 1.0f / sqrtf(sumsq / float(feature) + eps);
    for (uint32_t j = threadIdx.x; j < feature; j += 256) {
        float v = ld<DT>(x, row + j);
        if (res) v = v + ld<DT>(res, row + j);
        float o;
        if (DT == kF32 && res) {
            o = gamma ? v * (inv * ld<DT>(gamma, j)) : v * inv;
        } else {
            o = v * inv;
            if (gamma) o = o * ld<DT>(gamma, j);
        }
        st<DT>(out, row + j, o);
    }
}

// RmsNorm for bf16 rows of feature % 8 == 0, feature <= 8 * 256 * 4: one
// workgroup per row, every 16-byte vector of x and gamma loaded once, up
// front, and kept in registers through the reduction (rmsnorm_vec_row).
__global__ __launch_bounds__(256) void rmsnorm_bf16_vec_kernel(const uint16_t *__restrict__ x,
                                                               const uint16_t *__restrict__ gamma,
                                                               uint16_t *__restrict__ out,
                                                               uint32_t feature, float eps) {
    constexpr int kMaxVec = 4;
    __shared__ float part[4];
    const uint32_t nv = feature / 8;
    const u32x4 *xr = reinterpret_cast<const u32x4 *>(x + uint64_t(blockIdx.x) * feature);
    const u32x4 *gr = reinterpret_cast<const u32x4 *>(gamma);
    u32x4 xv[kMaxVec], gv[kMaxVec];
#pragma unroll
    for (int u = 0; u < kMaxVec; ++u) {
        const uint32_t v = threadIdx.x + 256u * u;
        if (v < nv) {
            xv[u] = xr[v];
            gv[u] = gamma ? gr[v] : u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
        }
    }
    rmsnorm_vec_row<kMaxVec>(xv, gv, nv, feature, eps, part,
                             reinterpret_cast<u32x4 *>(out + uint64_t(blockIdx.x) * feature));
}

// Rotary embedding, rotate-half form over heads of head_dim elements.
template <int DT>
__global__ __launch_bounds__(256) void rope_kernel(const void *__restrict__ x,
                                                   const void *__restrict__ cs,
                                                   const void *__restrict__ sn,
                                                   void *__restrict__ out, uint32_t head_dim,
                                                   uint64_t n) {
    const uint32_t half = head_dim / 2;
    for (uint64_t e = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < n;
         e += uint64_t(gridDim.x) * blockDim.x) {
        const uint32_t pos = uint32_t(e % head_dim);
        const float xe = ld<DT>(x, e), ce = ld<DT>(cs, e), se = ld<DT>(sn, e);
        float v;
        if (pos < half)
            v = xe * ce - ld<DT>(x, e + half) * se;
        else
            v = xe * ce + ld<DT>(x, e - half) * se;
        st<DT>(out, e, v);
    }
}

// The bf16 form eight elements a lane (head_dim a multiple of 16, operands
// 16-byte aligned, n a multiple of 8): the same per-element arithmetic, with
// 16-byte loads of x, its rotate-half partner, cos and sin.
__global__ __launch_bounds__(256) void rope_bf16_vec_kernel(const u32x4 *__restrict__ x,
                                                            const u32x4 *__restrict__ cs,
                                                            const u32x4 *__restrict__ sn,
                                                            u32x4 *__restrict__ out, uint32_t head_dim,
                                                            uint64_t n8) {
    const uint32_t half8 = head_dim / 16, hd8 = head_dim / 8;
    for (uint64_t e = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < n8;
         e += uint64_t(gridDim.x) * blockDim.x) {
        const bool lo = uint32_t(e % hd8) < half8;
        const u32x4 xv = x[e], pv = x[lo ? e + half8 : e - half8], cv = cs[e], sv = sn[e];
        u32x4 o;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t sh = (j & 1) * 16;
            const float xe = bf2f((xv[j / 2] >> sh) & 0xffffu), xp = bf2f((pv[j / 2] >> sh) & 0xffffu);
            const float ce = bf2f((cv[j / 2] >> sh) & 0xffffu), se = bf2f((sv[j / 2] >> sh) & 0xffffu);
            const float v = lo ? xe * ce - xp * se : xe * ce + xp * se;
            const uint32_t b = f2bf(v);
            o[j / 2] = (j & 1) ? (o[j / 2] | (b << 16)) : b;
        }
        out[e] = o;
    }
}

// Gather rows of `row_bytes` (a multiple of 4 when `words`): one workgroup per
// (outer, index) row. An index outside [-axis_dim, axis_dim) zeroes its row
// and raises *err.
template <bool kI64>
__global__ __launch_bounds__(256) void gather_kernel(const uint8_t *__restrict__ data,
                                                     const void *__restrict__ idx,
                                                     uint8_t *__restrict__ out, uint64_t axis_dim,
                                                     uint64_t num_idx, uint64_t row_bytes,
                                                     int *__restrict__ err) {
    const uint64_t o = blockIdx.y, k = blockIdx.x;
    int64_t i = kI64 ? static_cast<const int64_t *>(idx)[k] : static_cast<const int32_t *>(idx)[k];
    if (i < 0) i += int64_t(axis_dim);
    uint8_t *dst = out + (o * num_idx + k) * row_bytes;
    const bool ok = i >= 0 && uint64_t(i) < axis_dim;
    if (!ok && threadIdx.x == 0) atomicOr(err, 1);
    const uint8_t *src = data + (o * axis_dim + (ok ? uint64_t(i) : 0)) * row_bytes;
    if ((row_bytes & 15) == 0 && ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0) {
        const u32x4 *s4 = reinterpret_cast<const u32x4 *>(src);
        u32x4 *d4 = reinterpret_cast<u32x4 *>(dst);
        for (uint64_t w = threadIdx.x; w < row_bytes / 16; w += 256)
            d4[w] = ok ? s4[w] : u32x4{0, 0, 0, 0};
    } else {
        for (uint64_t w = threadIdx.x; w < row_bytes; w += 256) dst[w] = ok ? src[w] : uint8_t(0);
    }
}

// ArgMax per row: one workgroup per row; each thread keeps the first index of
// its largest value, then a (value, index) reduction that prefers the lower
// index on equal values. NaN never compares greater.
template <int DT>
__global__ __launch_bounds__(1024) void argmax_kernel(const void *__restrict__ in,
                                                      int32_t *__restrict__ out, uint32_t cols) {
    constexpr int kW = 16;                       // wavefronts
    constexpr bool kBf16 = DT == kBF16;
    constexpr int E = kBf16 ? 8 : 4;             // elements per 16-byte vector
    __shared__ float sv[kW];
    __shared__ int si[kW];
    const uint64_t row = uint64_t(blockIdx.x) * cols;
    float best = -INFINITY;
    int bi = -1;
    auto take = [&](float v, int j) {
        if (v > best || (bi < 0 && v == best)) {
            best = v;
            bi = j;
        }
    };
    // 16-byte vectors when the row start is aligned; each thread's vectors are
    // ascending in index, so a strict > keeps the first index of its maximum.
    // Four vectors a thread are loaded before any is compared (one memory
    // round trip per 4096 vectors, not one per 1024); a vector past the row
    // reads zero from its buffer range and is not compared.
    const bool vec = ((reinterpret_cast<uintptr_t>(in) + row * (kBf16 ? 2 : 4)) & 15) == 0 &&
                     uint64_t(cols / E) * 16u < (uint64_t(1) << 32);   // a 32-bit buffer range
    uint32_t j0 = 0;
    if (vec) {
        const uint32_t nv = cols / E;
        const auto rr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<char *>(static_cast<const char *>(in) + row * (kBf16 ? 2 : 4)), 0,
            int(nv * 16u), 0x00020000);
        for (uint32_t v0 = threadIdx.x; v0 < nv; v0 += 4 * 1024) {
            u32x4 x[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t v = v0 + 1024u * u;
                x[u] = __builtin_amdgcn_raw_buffer_load_b128(rr, v < nv ? 16u * v : 0x80000000u, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const uint32_t v = v0 + 1024u * u;
                if (v >= nv) break;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    if constexpr (kBf16) {
                        take(__uint_as_float(x[u][w] << 16), int(v * E + 2 * w));
                        take(__uint_as_float(x[u][w] & 0xFFFF0000u), int(v * E + 2 * w + 1));
                    } else {
                        take(__uint_as_float(x[u][w]), int(v * E + w));
                    }
                }
            }
        }
        j0 = nv * E;
    }
    for (uint32_t j = j0 + threadIdx.x; j < cols; j += 1024) take(ld<DT>(in, row + j), int(j));
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (oi >= 0 && (bi < 0 || ov > best || (ov == best && oi < bi))) {
            best = ov;
            bi = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = best;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < kW; ++w)
            if (si[w] >= 0 && (bi < 0 || sv[w] > best || (sv[w] == best && si[w] < bi))) {
                best = sv[w];
                bi = si[w];
            }
        out[blockIdx.x] = bi < 0 ? 0 : bi;
    }
}

// Transpose (transpose_float, src/cpu/float_kernels.rs:2980-3028): output
// axis i is input axis perm[i]. The copy unit is a piece of an output row of
// the last axis when that axis stays last (16 bytes when rows and bases allow,
// else one element), one element otherwise; each thread finds its input
// offset from the output coordinates.
struct TransposeArgs {
    const uint8_t *in;
    uint8_t *out;
    uint32_t lead;                 // output axes decomposed per unit
    uint64_t out_dims[8];
    uint64_t in_stride[8];         // bytes per step of output axis i in the input
    uint64_t unit_bytes, units_per_row, units;
};

// kNarrow: unit counts and output dims below 2^32, so the coordinates come
// from 32-bit divisions (a 64-bit one is a long instruction sequence).
template <bool kNarrow>
__global__ __launch_bounds__(256) void transpose_kernel(const TransposeArgs a) {
    using idx_t = typename std::conditional<kNarrow, uint32_t, uint64_t>::type;
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t u = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; u < a.units; u += stride) {
        const idx_t row = idx_t(u) / idx_t(a.units_per_row), piece = idx_t(u) % idx_t(a.units_per_row);
        idx_t rem = row;
        uint64_t src = uint64_t(piece) * a.unit_bytes;
        for (int i = int(a.lead) - 1; i >= 0; --i) {
            src += uint64_t(rem % idx_t(a.out_dims[i])) * a.in_stride[i];
            rem /= idx_t(a.out_dims[i]);
        }
        const uint8_t *s = a.in + src;
        uint8_t *d = a.out + u * a.unit_bytes;
        if (a.unit_bytes == 16)
            *reinterpret_cast<u32x4 *>(d) = *reinterpret_cast<const u32x4 *>(s);
        else
            for (uint64_t b = 0; b < a.unit_bytes; ++b) d[b] = s[b];
    }
}

unsigned grid_for(uint64_t work, unsigned cap = 4096) {
    const uint64_t g = (work + 255) / 256;
    return unsigned(g == 0 ? 1 : (g < cap ? g : cap));
}

}  // namespace

hipError_t launch_binary(int op, const void *a, const void *b, void *out, uint64_t n, uint8_t dtype,
                         hipStream_t stream) {
    const bool vec = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                       reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    const uint64_t nvec = vec ? n / (dtype == kF32 ? 4 : 8) : 0;
    const unsigned grid = grid_for(nvec ? nvec : n);
#define HOLO_BIN(D)                                                                              \
    do {                                                                                         \
        if (op == 0)                                                                             \
            hipLaunchKernelGGL((binary_kernel<D, kOpAdd>), dim3(grid), dim3(256), 0, stream, a, b, \
                               out, n, nvec);                                                    \
        else                                                                                     \
            hipLaunchKernelGGL((binary_kernel<D, kOpMul>), dim3(grid), dim3(256), 0, stream, a, b, \
                               out, n, nvec);                                                    \
    } while (0)
    switch (dtype) {
        case kBF16: HOLO_BIN(kBF16); break;
        case kF16: HOLO_BIN(kF16); break;
        case kF32: HOLO_BIN(kF32); break;
        default: return hipErrorInvalidValue;
    }
#undef HOLO_BIN
    return hipGetLastError();
}

hipError_t launch_add_rmsnorm(const void *x, const void *residual, const void *gamma, void *out,
                              uint32_t batch, uint32_t feature, float eps, uint8_t dtype,
                              hipStream_t stream) {
    if (batch == 0 || feature == 0) return hipSuccess;
    switch (dtype) {
        case kBF16:
            hipLaunchKernelGGL((add_rmsnorm_kernel<kBF16>), dim3(batch), dim3(256), 0, stream, x,
                               residual, gamma, out, feature, eps);
            break;
        case kF16:
            hipLaunchKernelGGL((add_rmsnorm_kernel<kF16>), dim3(batch), dim3(256), 0, stream, x,
                               residual, gamma, out, feature, eps);
            break;
        case kF32:
            hipLaunchKernelGGL((add_rmsnorm_kernel<kF32>), dim3(batch), dim3(256), 0, stream, x,
                               residual, gamma, out, feature, eps);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const void *x, const void *gamma, void *out, uint32_t batch,
                          uint32_t feature, float eps, uint8_t dtype, hipStream_t stream) {
    const bool vec = dtype == kBF16 && feature % 8 == 0 && feature <= 8 * 256 * 4 &&
                     ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gamma) |
                       reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    if (vec) {
        hipLaunchKernelGGL(rmsnorm_bf16_vec_kernel, dim3(batch), dim3(256), 0, stream,
                           static_cast<const uint16_t *>(x), static_cast<const uint16_t *>(gamma),
                           static_cast<uint16_t *>(out), feature, eps);
        return hipGetLastError();
    }
    switch (dtype) {
        case kBF16:
            hipLaunchKernelGGL((rmsnorm_kernel<kBF16>), dim3(batch), dim3(256), 0, stream, x, gamma,
                               out, feature, eps);
            break;
        case kF16:
            hipLaunchKernelGGL((rmsnorm_kernel<kF16>), dim3(batch), dim3(256), 0, stream, x, gamma,
                               out, feature, eps);
            break;
        case kF32:
            hipLaunchKernelGGL((rmsnorm_kernel<kF32>), dim3(batch), dim3(256), 0, stream, x, gamma,
                               out, feature, eps);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_rope(const void *x, const void *cs, const void *sn, void *out, uint32_t head_dim,
                       uint64_t n, uint8_t dtype, hipStream_t stream) {
    if (dtype == kBF16 && head_dim % 16 == 0 && n % 8 == 0 &&
        ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(cs) |
          reinterpret_cast<uintptr_t>(sn) | reinterpret_cast<uintptr_t>(out)) & 15) == 0) {
        hipLaunchKernelGGL(rope_bf16_vec_kernel, dim3(grid_for(n / 8)), dim3(256), 0, stream,
                           static_cast<const u32x4 *>(x), static_cast<const u32x4 *>(cs),
                           static_cast<const u32x4 *>(sn), static_cast<u32x4 *>(out), head_dim, n / 8);
        return hipGetLastError();
    }
    const unsigned grid = grid_for(n);
    switch (dtype) {
        case kBF16:
            hipLaunchKernelGGL((rope_kernel<kBF16>), dim3(grid), dim3(256), 0, stream, x, cs, sn, out,
                               head_dim, n);
            break;
        case kF16:
            hipLaunchKernelGGL((rope_kernel<kF16>), dim3(grid), dim3(256), 0, stream, x, cs, sn, out,
                               head_dim, n);
            break;
        case kF32:
            hipLaunchKernelGGL((rope_kernel<kF32>), dim3(grid), dim3(256), 0, stream, x, cs, sn, out,
                               head_dim, n);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// The multi-row attention's precondition, checked where the lengths live: a
// prompt's earlier rows need cache slots that a ring wrap (lens > bucket) has
// already overwritten with later rows, so such a length raises bit 2 of *err.
__global__ __launch_bounds__(256) void lens_within_kernel(const uint32_t *__restrict__ lens,
                                                          uint32_t n, uint32_t bucket,
                                                          int *__restrict__ err) {
    bool bad = false;
    for (uint32_t i = threadIdx.x; i < n; i += 256) bad = bad || lens[i] > bucket;
    if (bad) atomicOr(err, 2);
}

hipError_t launch_lens_within(const uint32_t *lens, uint32_t n, uint32_t bucket, int *err,
                              hipStream_t stream) {
    hipLaunchKernelGGL(lens_within_kernel, dim3(1), dim3(256), 0, stream, lens, n, bucket, err);
    return hipGetLastError();
}

// Unary activations over f32: the reference computes these per element
// (unary_act, src/cpu/kernels.rs:1586-1598), with the same scalar functions.
__global__ __launch_bounds__(256) void act_f32_kernel(const float *__restrict__ in,
                                                      float *__restrict__ out, uint64_t n,
                                                      uint32_t act) {
    const uint64_t stride = uint64_t(gridDim.x) * 256;
    for (uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride)
        out[i] = act_f32(act, in[i]);
}

// The fused MatMul epilogues over an f16 product already in `c` (narrowed
// with the reference's rounding), as matmul_activation_float /
// matmul_add_float / matmul_add_activation_float compute 16-bit rows
// (src/cpu/float_kernels.rs:816-935): v = widen(c[i]) (+ widen(res[i]) in
// f32), the scalar fused activation on the f32 value, one narrowing.
// kind: 1 = activation, 2 = residual add, 3 = add then activation.
__global__ __launch_bounds__(256) void epilogue_f16_kernel(uint16_t *__restrict__ c,
                                                           const uint16_t *__restrict__ res,
                                                           uint64_t n, uint32_t kind, uint32_t act) {
    const uint64_t stride = uint64_t(gridDim.x) * 256;
    for (uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) {
        float v = f16_bits_to_f32(c[i]);
        if (kind >= 2) v = v + f16_bits_to_f32(res[i]);
        if (kind != 2) v = act_f32(act, v);
        c[i] = f32_to_f16_bits(v);
    }
}

hipError_t launch_epilogue_f16(uint16_t *c, const uint16_t *res, uint64_t n, uint32_t kind,
                               uint32_t act, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    const uint64_t b = (n + 255) / 256;
    hipLaunchKernelGGL(epilogue_f16_kernel, dim3(unsigned(b < 8192 ? b : 8192)), dim3(256), 0,
                       stream, c, res, n, kind, act);
    return hipGetLastError();
}

hipError_t launch_act_f32(const float *in, float *out, uint64_t n, uint32_t act,
                          hipStream_t stream) {
    if (n == 0) return hipSuccess;
    const uint64_t b = (n + 255) / 256;
    hipLaunchKernelGGL(act_f32_kernel, dim3(unsigned(b < 8192 ? b : 8192)), dim3(256), 0, stream,
                       in, out, n, act);
    return hipGetLastError();
}

hipError_t launch_gather(const void *data, const void *idx, void *out, uint64_t outer,
                         uint64_t axis_dim, uint64_t num_idx, uint64_t row_bytes, bool i64,
                         int *err, hipStream_t stream) {
    const dim3 grid{unsigned(num_idx), unsigned(outer), 1u};
    if (i64)
        hipLaunchKernelGGL((gather_kernel<true>), grid, dim3(256), 0, stream,
                           static_cast<const uint8_t *>(data), idx, static_cast<uint8_t *>(out),
                           axis_dim, num_idx, row_bytes, err);
    else
        hipLaunchKernelGGL((gather_kernel<false>), grid, dim3(256), 0, stream,
                           static_cast<const uint8_t *>(data), idx, static_cast<uint8_t *>(out),
                           axis_dim, num_idx, row_bytes, err);
    return hipGetLastError();
}

hipError_t launch_transpose(const void *in, void *out, uint32_t rank, const uint32_t *dims,
                            const uint8_t *perm, uint32_t es, hipStream_t stream) {
    if (rank == 0 || rank > 8) return hipErrorInvalidValue;
    uint64_t in_stride[8], total = 1;
    for (int i = int(rank) - 1; i >= 0; --i) {
        in_stride[i] = total * es;
        total *= dims[i];
    }
    if (total == 0) return hipSuccess;
    TransposeArgs a{};
    a.in = static_cast<const uint8_t *>(in);
    a.out = static_cast<uint8_t *>(out);
    for (uint32_t i = 0; i < rank; ++i) {
        a.out_dims[i] = dims[perm[i]];
        a.in_stride[i] = in_stride[perm[i]];
    }
    const bool keep_last = perm[rank - 1] == rank - 1;
    const uint64_t row_bytes = keep_last ? uint64_t(dims[rank - 1]) * es : es;
    a.lead = keep_last ? rank - 1 : rank;
    const bool vec = keep_last && row_bytes % 16 == 0 &&
                     ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15) == 0;
    a.unit_bytes = vec ? 16 : es;
    a.units_per_row = row_bytes / a.unit_bytes;
    a.units = total * es / a.unit_bytes;
    bool narrow = a.units < (1ull << 32) && a.units_per_row < (1ull << 32);
    for (uint32_t i = 0; i < a.lead; ++i) narrow = narrow && a.out_dims[i] < (1ull << 32);
    if (narrow)
        hipLaunchKernelGGL(transpose_kernel<true>, dim3(grid_for(a.units, 16384)), dim3(256), 0, stream, a);
    else
        hipLaunchKernelGGL(transpose_kernel<false>, dim3(grid_for(a.units, 16384)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_argmax(const void *in, int32_t *out, uint32_t rows, uint32_t cols, bool bf16,
                         hipStream_t stream) {
    if (bf16)
        hipLaunchKernelGGL((argmax_kernel<kBF16>), dim3(rows), dim3(1024), 0, stream, in, out, cols);
    else
        hipLaunchKernelGGL((argmax_kernel<kF32>), dim3(rows), dim3(1024), 0, stream, in, out, cols);
    return hipGetLastError();
}

}  // namespace holo
