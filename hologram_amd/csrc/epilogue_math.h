// epilogue_math.h — the per-element finish of a few-row MatMul product, shared
// by the split-K epilogue (epilogue.hip) and the single-launch group over
// packed weights (gemv_packed.hip): the same IEEE operations in the same
// order, so both give the bits the standalone kernels give.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "holo_device.h"
#include "holo_kernels.h"

namespace holo {
namespace epi {

__device__ __forceinline__ float bf2f(uint32_t b) { return __uint_as_float(b << 16); }
__device__ __forceinline__ uint32_t f2bf(float f) { return __float_as_uint(f) >> 16; }

// Segment i, copied out of the kernel arguments field by field with
// constant indices: a reference picked at run time makes the compiler copy
// the whole argument block to scratch memory on entry.
template <class Args>
__device__ __forceinline__ EpiSeg seg_of(const Args &g, uint32_t i) {
    EpiSeg s;
#define HOLO_SEG_FIELD(F) \
    s.F = i == 0 ? g.seg[0].F : i == 1 ? g.seg[1].F : i == 2 ? g.seg[2].F : g.seg[3].F
    HOLO_SEG_FIELD(n);
    HOLO_SEG_FIELD(col0);
    HOLO_SEG_FIELD(base);
    HOLO_SEG_FIELD(act);
    HOLO_SEG_FIELD(lut);
    HOLO_SEG_FIELD(residual);
    HOLO_SEG_FIELD(out);
    HOLO_SEG_FIELD(head_dim);
    HOLO_SEG_FIELD(rope);
    HOLO_SEG_FIELD(cos);
    HOLO_SEG_FIELD(sin);
    HOLO_SEG_FIELD(rope_out);
    HOLO_SEG_FIELD(quant);
    HOLO_SEG_FIELD(pos);
    HOLO_SEG_FIELD(cq);
    HOLO_SEG_FIELD(cs);
    HOLO_SEG_FIELD(bucket);
    HOLO_SEG_FIELD(new_rows);
    HOLO_SEG_FIELD(pair);
    HOLO_SEG_FIELD(mul_out);
    HOLO_SEG_FIELD(skip);
    HOLO_SEG_FIELD(ssq);
#undef HOLO_SEG_FIELD
    return s;
}

// An optional side operand (residual, cos, sin) read through a buffer range
// that is empty when the operand is absent: the load then reads 0 without a
// memory access, so it needs no branch.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t opt_rsrc(const void *p, bool present) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, present ? 0x7fffffff : 0,
                                             0x00020000);
}
template <bool kBf16>
__device__ __forceinline__ float opt_load(__amdgpu_buffer_rsrc_t r, uint64_t e) {
    if constexpr (kBf16)
        return bf2f(__builtin_amdgcn_raw_buffer_load_b16(r, uint32_t(e) * 2u, 0, 0));
    else
        return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, uint32_t(e) * 4u, 0, 0));
}

// The segment's base value from its product v and (for the add forms) the
// residual r (bf16: the result is a bf16 bit pattern widened back to f32, so
// later steps see exactly the stored value).
template <bool kBf16>
__device__ __forceinline__ float base_value(const EpiSeg &sg, float v, float r) {
    if constexpr (kBf16) {
        uint32_t x = f2bf(v);
        if (sg.base == kEpiAct) x = sg.lut[x];   // f(widen(x)) narrowed: the table entry
        if (sg.base == kEpiAdd || sg.base == kEpiAddAct) {
            const float s = bf2f(x) + r;
            // MatMulAddActivation applies f to the f32 sum before narrowing
            x = f2bf(sg.base == kEpiAddAct ? act_f32_call(sg.act, s) : s);
        }
        return bf2f(x);
    } else {
        if (sg.base == kEpiAdd || sg.base == kEpiAddAct) v = v + r;
        if (sg.base == kEpiAct || sg.base == kEpiAddAct) v = act_f32_call(sg.act, v);
        return v;
    }
}

__device__ __forceinline__ bool has_residual(const EpiSeg &sg) {
    return sg.base == kEpiAdd || sg.base == kEpiAddAct;
}

template <bool kBf16>
__device__ __forceinline__ void store(void *p, uint64_t e, float v) {
    if constexpr (kBf16)
        static_cast<uint16_t *>(p)[e] = uint16_t(f2bf(v));
    else
        static_cast<float *>(p)[e] = v;
}

template <bool kBf16>
__device__ __forceinline__ float load(const void *p, uint64_t e) {
    if constexpr (kBf16)
        return bf2f(static_cast<const uint16_t *>(p)[e]);
    else
        return static_cast<const float *>(p)[e];
}

// Rust's `f32 as i32` then clamp(-127, 127) (NaN -> 0, saturating).
__device__ __forceinline__ int8_t to_q(float r) {
    if (r != r) return 0;
    r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
    return static_cast<int8_t>(static_cast<int32_t>(r));
}

// The product at (row m, column c) of P's column space: partials summed in
// ks order. Up to kBatch loads go out before the first add, so a split of up
// to kBatch partials costs one memory round trip; the adds keep ks order.
// No load sits behind a branch: a batch past ks reloads partial ks - 1 (its
// value is not added), since a branch around a load makes the compiler wait
// for every load in flight where the branch joins.
constexpr uint32_t kBatch = 32;

__device__ __forceinline__ uint32_t clamp_ks(uint32_t k, uint32_t ks) { return k < ks ? k : ks - 1; }

template <class T>
__device__ __forceinline__ T sum_partials(const T *p, uint64_t plane, uint32_t ks) {
    T s{};
    for (uint32_t k0 = 0; k0 < ks; k0 += kBatch) {
        T v[kBatch];
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u) v[u] = p[clamp_ks(k0 + u, ks) * plane];
        if (k0 == 0) s = v[0];
#pragma unroll
        for (uint32_t u = 0; u < kBatch; ++u)
            if (k0 + u < ks && (k0 | u) != 0) s += v[u];
    }
    return s;
}

// Two columns (c, c + off) of one row, their partials in flight together.
__device__ __forceinline__ void product2(const EpiArgs &g, uint32_t m, uint32_t c, uint32_t off,
                                        float *x1, float *x2) {
    const uint64_t plane = uint64_t(g.m) * g.ntot;
    const float *p = g.P + uint64_t(m) * g.ntot + c;
    float s1 = 0.0f, s2 = 0.0f;
    for (uint32_t k0 = 0; k0 < g.ks; k0 += kBatch / 2) {
        float v1[kBatch / 2], v2[kBatch / 2];
#pragma unroll
        for (uint32_t u = 0; u < kBatch / 2; ++u) {
            const uint64_t kk = clamp_ks(k0 + u, g.ks);
            v1[u] = p[kk * plane];
            v2[u] = p[kk * plane + off];
        }
        if (k0 == 0) {
            s1 = v1[0];
            s2 = v2[0];
        }
#pragma unroll
        for (uint32_t u = 0; u < kBatch / 2; ++u)
            if (k0 + u < g.ks && (k0 | u) != 0) {
                s1 += v1[u];
                s2 += v2[u];
            }
    }
    *x1 = s1;
    *x2 = s2;
}

// One head of a head-wise segment (rope and/or quant) at row m, head h of the
// row: lane d < D/2 of the head's D/2 consecutive lanes holds the rotate-half
// pair (d, d + D/2). The head's lanes run this together (the int8 scale is a
// shuffle reduction over them). `live` false: the lane loads and computes but
// stores nothing.
template <bool kBf16>
__device__ __forceinline__ void head_finish(const EpiArgs &g, const EpiSeg &sg, uint32_t m, uint32_t h,
                                            uint32_t d, bool live) {
    const uint32_t D = sg.head_dim, half = D / 2;
    const uint32_t c1 = h * D + d;
    const uint64_t e1 = uint64_t(m) * sg.n + c1;
    // side operands first: their loads overlap the partials'
    const auto rc = opt_rsrc(sg.cos, sg.rope), rs = opt_rsrc(sg.sin, sg.rope);
    const auto rr = opt_rsrc(sg.residual, has_residual(sg));
    const float c1v = opt_load<kBf16>(rc, e1), s1v = opt_load<kBf16>(rs, e1);
    const float c2v = opt_load<kBf16>(rc, e1 + half), s2v = opt_load<kBf16>(rs, e1 + half);
    const float r1 = opt_load<kBf16>(rr, e1), r2 = opt_load<kBf16>(rr, e1 + half);
    float p1, p2;
    product2(g, m, sg.col0 + c1, half, &p1, &p2);
    float x1 = base_value<kBf16>(sg, p1, r1);
    float x2 = base_value<kBf16>(sg, p2, r2);
    if (live) {
        if (sg.out) {
            store<kBf16>(sg.out, e1, x1);
            store<kBf16>(sg.out, e1 + half, x2);
        }
        if (sg.rope) {
            float y1 = x1 * c1v - x2 * s1v;
            float y2 = x2 * c2v + x1 * s2v;
            if constexpr (kBf16) {
                y1 = bf2f(f2bf(y1));
                y2 = bf2f(f2bf(y2));
            }
            x1 = y1;
            x2 = y2;
            if (sg.rope_out) {
                store<kBf16>(sg.rope_out, e1, x1);
                store<kBf16>(sg.rope_out, e1 + half, x2);
            }
        }
    }
    if (!sg.quant) return;
    // row max of |x| over the head's lanes (NaN never wins a `>`); exact, so
    // the order of the reduction does not matter
    float amax = 0.0f;
    const float a1 = x1 < 0.0f ? -x1 : x1, a2 = x2 < 0.0f ? -x2 : x2;
    if (a1 > amax) amax = a1;
    if (a2 > amax) amax = a2;
    for (uint32_t off = half / 2; off >= 1; off >>= 1) {
        const float o = __shfl_xor(amax, int(off), 64);
        if (o > amax) amax = o;
    }
    if (!live) return;
    const uint64_t r = e1 / D;   // the row of the appended [planes, new_rows, D] block
    const uint32_t plane = uint32_t(r / sg.new_rows), j = uint32_t(r % sg.new_rows);
    const uint64_t pos = *sg.pos % sg.bucket;
    const uint64_t row = uint64_t(plane) * sg.bucket + (pos + j) % sg.bucket;
    int8_t *dst = sg.cq + row * D;
    if (amax == 0.0f) {
        dst[d] = 0;
        dst[d + half] = 0;
        if (d == 0) sg.cs[row] = 0.0f;
        return;
    }
    const float inv = 127.0f / amax;
    const float t1 = x1 * inv, t2 = x2 * inv;
    dst[d] = to_q(t1 >= 0.0f ? truncf(t1 + 0.5f) : truncf(t1 - 0.5f));
    dst[d + half] = to_q(t2 >= 0.0f ? truncf(t2 + 0.5f) : truncf(t2 - 0.5f));
    if (d == 0) sg.cs[row] = amax / 127.0f;
}

}  // namespace epi
}  // namespace holo
