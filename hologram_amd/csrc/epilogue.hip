// epilogue.hip — the end of a few-row MatMul on the device: the fp32 split-K
// partials of one launch (gemm_skinny.hip, launch_skinny_partials) summed in
// ks order, narrowed, and finished per output segment with the ops that
// consume the product in a decode step, so those ops cost no launch of their
// own and their inputs never round-trip through HBM:
//
//   base      the product itself; + a residual (MatMulAdd, float_kernels.rs:
//             846-888); an activation (MatMulActivation, :816-844; bf16 through
//             the same 65536-entry table the standalone op uses, f32 through
//             exp_f32_det as gelu_f/silu_f/sigmoid_f/tanh_f, :3537-3566); both
//             (MatMulAddActivation, :890-935)
//   rope      rotate-half rotary embedding of each head (rope_float, :3123-3186)
//   quant     int8 quantize + ring append of each head row (quantize_row_i8,
//             src/cpu/simd.rs:4755-4785; placement as kernels.rs:455-501)
//   pair      the element-wise product with another segment's value
//             (binary_float Mul, float_kernels.rs:238-300: SwiGLU's silu(g)*u)
//
// Every step is the same IEEE operation in the same order as the standalone
// kernel it replaces (the partials summed sequentially in ks order as
// skinny_reduce_kernel does, bf16 narrowed by truncation between ops), so a
// fused walk gives the same bits as the unfused one.

#include <hip/hip_runtime.h>

#include <math.h>

#include "holo_device.h"
#include "holo_kernels.h"
#include "epilogue_math.h"

namespace holo {
namespace {

using namespace epi;

typedef float f32x4 __attribute__((ext_vector_type(4)));

// One wavefront per workgroup: the epilogue of a decode step is a few
// thousand threads, spread over as many CUs as possible.
constexpr uint32_t kEpiThreads = 64;

// Segment of this workgroup (workgroup-uniform, chosen with selects).
__device__ __forceinline__ int pick(const EpiArgs &g, uint32_t *first_block) {
    int s = 0;
    uint32_t b0 = 0;
#pragma unroll
    for (int i = 1; i < kSkinnyMaxSeg; ++i)
        if (uint32_t(i) < g.nseg && blockIdx.x >= g.blk_end[i - 1]) {
            s = i;
            b0 = g.blk_end[i - 1];
        }
    *first_block = b0;
    return s;
}

// 4 consecutive columns (c a multiple of 4), as 16-byte loads.
__device__ __forceinline__ f32x4 product4(const EpiArgs &g, uint32_t m, uint32_t c) {
    return sum_partials(reinterpret_cast<const f32x4 *>(g.P + uint64_t(m) * g.ntot + c),
                        uint64_t(g.m) * g.ntot / 4, g.ks);
}

// Element-wise segments: 4 consecutive columns of one row per thread. The
// residual and both segments' partials are loaded before any arithmetic.
template <bool kBf16>
__device__ __forceinline__ void elem_segment(const EpiArgs &g, const EpiSeg &sg, const EpiSeg &pr, uint32_t blk) {
    const uint64_t i = (uint64_t(blk) * kEpiThreads + threadIdx.x) * 4;
    if (i >= uint64_t(g.m) * sg.n) return;
    const uint32_t m = uint32_t(i / sg.n), c = uint32_t(i % sg.n);
    const uint64_t e0 = uint64_t(m) * sg.n + c;
    float ra[4], rb[4];
    const bool pair = sg.pair >= 0;
    const auto rra = opt_rsrc(sg.residual, has_residual(sg));
    const auto rrb = opt_rsrc(pr.residual, pair && has_residual(pr));
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
        ra[j] = opt_load<kBf16>(rra, e0 + j);
        rb[j] = opt_load<kBf16>(rrb, e0 + j);
    }
    f32x4 va, vb = f32x4{0.f, 0.f, 0.f, 0.f};
    if (!pair) {
        va = product4(g, m, sg.col0 + c);
    } else {
        // both segments' partials in flight together
        const uint64_t plane = uint64_t(g.m) * g.ntot / 4;
        const f32x4 *pa = reinterpret_cast<const f32x4 *>(g.P + uint64_t(m) * g.ntot + sg.col0 + c);
        const f32x4 *pb = reinterpret_cast<const f32x4 *>(g.P + uint64_t(m) * g.ntot + pr.col0 + c);
        for (uint32_t k0 = 0; k0 < g.ks; k0 += kBatch / 2) {
            f32x4 xa[kBatch / 2], xb[kBatch / 2];
#pragma unroll
            for (uint32_t u = 0; u < kBatch / 2; ++u) {
                const uint64_t kk = clamp_ks(k0 + u, g.ks);
                xa[u] = pa[kk * plane];
                xb[u] = pb[kk * plane];
            }
            if (k0 == 0) {
                va = xa[0];
                vb = xb[0];
            }
#pragma unroll
            for (uint32_t u = 0; u < kBatch / 2; ++u)
                if (k0 + u < g.ks && (k0 | u) != 0) {
                    va += xa[u];
                    vb += xb[u];
                }
        }
    }
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
        va[j] = base_value<kBf16>(sg, va[j], ra[j]);
        if (sg.out) store<kBf16>(sg.out, e0 + j, va[j]);
    }
    if (!pair) return;
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) {
        vb[j] = base_value<kBf16>(pr, vb[j], rb[j]);
        if (pr.out) store<kBf16>(pr.out, e0 + j, vb[j]);
        store<kBf16>(sg.mul_out, e0 + j, va[j] * vb[j]);
    }
}

// Head-wise segments (rope and/or quant): a head of D = head_dim columns is
// D/2 lanes, lane d holding the rotate-half pair (d, d + D/2).
template <bool kBf16>
__device__ __forceinline__ void head_segment(const EpiArgs &g, const EpiSeg &sg, uint32_t blk) {
    const uint32_t D = sg.head_dim, half = D / 2;
    const uint32_t heads_per_block = kEpiThreads / half;
    const uint32_t hl = threadIdx.x / half, d = threadIdx.x % half;
    const uint32_t heads_row = sg.n / D;
    const uint64_t head = uint64_t(blk) * heads_per_block + hl;
    const uint64_t nheads = uint64_t(g.m) * heads_row;
    const bool live = head < nheads;
    // every lane loads (a lane past the last head reads the last head), so no
    // load sits behind a branch; only live lanes store
    const uint64_t hc = live ? head : nheads - 1;
    head_finish<kBf16>(g, sg, uint32_t(hc / heads_row), uint32_t(hc % heads_row), d, live);
}

// A group of one element-wise bf16 segment that also leaves the RmsNorm
// statistics of each result row. The standalone bf16 RmsNorm kernel (one 256-thread workgroup per
// row) has thread t sum the squares of its 16-byte vectors t + 256u in order,
// then reduces each wave with a xor tree, then adds the four wave sums. Here
// four one-wave workgroups per row each play one of those waves exactly: lane
// l of wave w holds vectors 64w + l + 256u, computes the same per-lane sum and
// the same tree, and stores the wave's sum; the reader adds the four in order.
constexpr uint32_t kStatVec = 4;   // vectors per lane: n <= 8 * 256 * 4
constexpr uint32_t kStatBatch = 16;  // partials per column pair in flight at once

__global__ __launch_bounds__(kEpiThreads) void epilogue_stat_kernel(const EpiArgs g) {
    const EpiSeg &sg = g.seg[0];
    const uint32_t r = blockIdx.x / 4, w = blockIdx.x % 4, l = threadIdx.x;
    const uint32_t nv = sg.n / 8;
    const uint64_t plane = uint64_t(g.m) * g.ntot / 4;
    const bool add = has_residual(sg);
    float ss = 0.0f;
#pragma unroll
    for (uint32_t u = 0; u < kStatVec; ++u) {
        const uint32_t v = 64 * w + l + 256 * u;
        if (v >= nv) break;
        const uint64_t e0 = uint64_t(r) * sg.n + 8ull * v;
        const u32x4 res = __builtin_amdgcn_raw_buffer_load_b128(
            opt_rsrc(sg.residual, add), uint32_t(e0) * 2u, 0, 0);
        // columns 8v .. 8v+3 and 8v+4 .. 8v+7: the residual and both halves'
        // partials (up to 16 of each) in flight together, summed in ks order
        const f32x4 *pa = reinterpret_cast<const f32x4 *>(g.P + uint64_t(r) * g.ntot + sg.col0 + 8 * v);
        f32x4 va, vb;
        for (uint32_t k0 = 0; k0 < g.ks; k0 += kStatBatch) {
            f32x4 xa[kStatBatch], xb[kStatBatch];
#pragma unroll
            for (uint32_t i = 0; i < kStatBatch; ++i) {
                const uint64_t kk = clamp_ks(k0 + i, g.ks);
                xa[i] = pa[kk * plane];
                xb[i] = pa[kk * plane + 1];
            }
            if (k0 == 0) {
                va = xa[0];
                vb = xb[0];
            }
#pragma unroll
            for (uint32_t i = 0; i < kStatBatch; ++i)
                if (k0 + i < g.ks && (k0 | i) != 0) {
                    va += xa[i];
                    vb += xb[i];
                }
        }
        u32x4 x;
#pragma unroll
        for (uint32_t h = 0; h < 4; ++h) {
            const float p0 = h < 2 ? va[2 * h] : vb[2 * h - 4];
            const float p1 = h < 2 ? va[2 * h + 1] : vb[2 * h - 3];
            const float lo = base_value<true>(sg, p0, bf2f(res[h] & 0xffffu));
            const float hi = base_value<true>(sg, p1, bf2f(res[h] >> 16));
            x[h] = f2bf(lo) | (f2bf(hi) << 16);
        }
        if (sg.out) reinterpret_cast<u32x4 *>(sg.out)[e0 / 8] = x;
#pragma unroll
        for (uint32_t h = 0; h < 4; ++h) {
            const float lo = bf2f(x[h] & 0xffffu), hi = __uint_as_float(x[h] & 0xFFFF0000u);
            ss = fmaf(lo, lo, ss);
            ss = fmaf(hi, hi, ss);
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if (l == 0) sg.ssq[4 * r + w] = ss;
}

template <bool kBf16>
__global__ __launch_bounds__(kEpiThreads) void epilogue_kernel(const EpiArgs g) {
    uint32_t b0;
    const int s = pick(g, &b0);
    const EpiSeg sg = seg_of(g, uint32_t(s));
    const uint32_t blk = blockIdx.x - b0;
    if (sg.head_dim) {
        head_segment<kBf16>(g, sg, blk);
    } else {
        const int p = sg.pair < 0 ? 0 : sg.pair;
        const EpiSeg pr = seg_of(g, uint32_t(p));
        elem_segment<kBf16>(g, sg, pr, blk);
    }
}

}  // namespace

// In-place epilogue over a tiled MatMul's output: 8 bf16 (or 4 f32) per
// thread as one 16-byte load and store when the operands allow, element by
// element otherwise; grid-stride.
template <bool kBf16, bool kVec>
__global__ __launch_bounds__(256) void tile_epilogue_kernel(void *__restrict__ c,
                                                           const void *__restrict__ res,
                                                           const uint16_t *__restrict__ lut,
                                                           uint64_t count, uint8_t kind,
                                                           uint32_t act) {
    constexpr uint32_t E = kVec ? (kBf16 ? 8 : 4) : 1;
    const uint64_t stride = uint64_t(gridDim.x) * blockDim.x;
    for (uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x; i * E < count; i += stride) {
        float v[E], r[E];
        if constexpr (kVec) {
            const u32x4 x = reinterpret_cast<const u32x4 *>(c)[i];
            const u32x4 y = kind >= 2 ? reinterpret_cast<const u32x4 *>(res)[i]
                                      : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
            for (uint32_t j = 0; j < E; ++j) {
                if constexpr (kBf16) {
                    v[j] = bf2f(j & 1 ? x[j / 2] >> 16 : x[j / 2] & 0xffffu);
                    r[j] = bf2f(j & 1 ? y[j / 2] >> 16 : y[j / 2] & 0xffffu);
                } else {
                    v[j] = __uint_as_float(x[j]);
                    r[j] = __uint_as_float(y[j]);
                }
            }
        } else {
            v[0] = load<kBf16>(c, i);
            r[0] = kind >= 2 ? load<kBf16>(res, i) : 0.0f;
        }
        EpiSeg sg;
        sg.base = kind;
        sg.act = act;
        sg.lut = lut;
#pragma unroll
        for (uint32_t j = 0; j < E; ++j) v[j] = base_value<kBf16>(sg, v[j], r[j]);
        if constexpr (kVec) {
            u32x4 o;
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j)
                o[j] = kBf16 ? (f2bf(v[2 * j]) | (f2bf(v[2 * j + 1]) << 16)) : __float_as_uint(v[j]);
            reinterpret_cast<u32x4 *>(c)[i] = o;
        } else {
            store<kBf16>(c, i, v[0]);
        }
    }
}

uint32_t epilogue_blocks(const EpiSeg &sg, uint32_t m) {
    if (sg.skip) return 0;
    if (sg.head_dim) {
        const uint32_t heads_per_block = kEpiThreads / (sg.head_dim / 2);
        const uint64_t heads = uint64_t(m) * (sg.n / sg.head_dim);
        return uint32_t((heads + heads_per_block - 1) / heads_per_block);
    }
    const uint64_t threads = uint64_t(m) * sg.n / 4;
    return uint32_t((threads + kEpiThreads - 1) / kEpiThreads);
}

hipError_t launch_tile_epilogue(void *c, uint64_t count, bool bf16, const TileEpi &epi,
                                hipStream_t stream) {
    if (count == 0 || epi.kind == kEpiStore) return hipSuccess;
    const uint64_t E = bf16 ? 8 : 4;
    const bool vec = count % E == 0 && ((reinterpret_cast<uintptr_t>(c) |
                                         reinterpret_cast<uintptr_t>(epi.residual)) & 15) == 0;
    const uint64_t items = vec ? count / E : count;
    uint64_t blocks = (items + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    const dim3 grid{unsigned(blocks)}, block{256u};
#define HOLO_TILE_EPI(BF, VEC)                                                                   \
    hipLaunchKernelGGL((tile_epilogue_kernel<BF, VEC>), grid, block, 0, stream, c, epi.residual, \
                       epi.lut, count, epi.kind, epi.act)
    if (bf16) {
        if (vec) HOLO_TILE_EPI(true, true);
        else HOLO_TILE_EPI(true, false);
    } else {
        if (vec) HOLO_TILE_EPI(false, true);
        else HOLO_TILE_EPI(false, false);
    }
#undef HOLO_TILE_EPI
    return hipGetLastError();
}

hipError_t launch_epilogue(EpiArgs g, hipStream_t stream) {
    if (g.nseg < 1 || g.nseg > uint32_t(kSkinnyMaxSeg)) return hipErrorInvalidValue;
    // side operands are read through 32-bit buffer offsets
    for (uint32_t i = 0; i < g.nseg; ++i)
        if (uint64_t(g.m) * g.seg[i].n * (g.bf16 ? 2 : 4) > 0x7fffffffull) return hipErrorInvalidValue;
    if (g.seg[0].ssq) {
        const EpiSeg &s = g.seg[0];
        if (g.nseg != 1 || !g.bf16 || s.head_dim || s.pair >= 0 || s.skip || s.n % 8 != 0 ||
            s.n > 8 * 256 * kStatVec || g.ntot != s.n || g.ks < 1 ||
            ((reinterpret_cast<uintptr_t>(s.out) | reinterpret_cast<uintptr_t>(s.residual) |
              reinterpret_cast<uintptr_t>(s.ssq)) & 15) != 0)
            return hipErrorInvalidValue;
        hipLaunchKernelGGL(epilogue_stat_kernel, dim3(4 * g.m), dim3(kEpiThreads), 0, stream, g);
        return hipGetLastError();
    }
    uint32_t total = 0;
    for (uint32_t i = 0; i < g.nseg; ++i) {
        if (g.seg[i].ssq) return hipErrorInvalidValue;
        total += epilogue_blocks(g.seg[i], g.m);
        g.blk_end[i] = total;
    }
    if (total == 0) return hipSuccess;
    if (g.bf16)
        hipLaunchKernelGGL(epilogue_kernel<true>, dim3(total), dim3(kEpiThreads), 0, stream, g);
    else
        hipLaunchKernelGGL(epilogue_kernel<false>, dim3(total), dim3(kEpiThreads), 0, stream, g);
    return hipGetLastError();
}

}  // namespace holo
