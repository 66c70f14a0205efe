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

}  // namespace epi
}  // namespace holo
