// holo_device.h — small device-side helpers shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace holo {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Streaming 16-byte load/store (non-temporal: the data is touched once).
__device__ __forceinline__ u32x4 ld_stream(const u32x4 *p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st_stream(u32x4 v, u32x4 *p) { __builtin_nontemporal_store(v, p); }

// exp_f32_det (src/cpu/simd.rs:4191-4239): clamp, k = trunc(x*log2e +- 1/2),
// Cody-Waite reduction, degree-6 Horner, scale by 2^k. IEEE basic operations
// only; the files that include this are built without contraction.
__device__ inline float exp_det(float x) {
    const float LO = -87.33654f, HI = 88.0f;
    const float LOG2E = 1.44269504088896340736f;
    const float LN2_HI = __uint_as_float(0x3F318000u);
    const float LN2_LO = -2.1219444e-4f;
    const float C6 = 1.0f / 720.0f, C5 = 1.0f / 120.0f, C4 = 1.0f / 24.0f, C3 = 1.0f / 6.0f,
                C2 = 0.5f;
    if (x != x || x < LO) return 0.0f;
    if (x > HI) x = HI;
    const float t = x * LOG2E;
    const int32_t k = t >= 0.0f ? int32_t(t + 0.5f) : int32_t(t - 0.5f);
    const float kf = float(k);
    const float r = (x - kf * LN2_HI) - kf * LN2_LO;
    float p = C6;
    p = p * r + C5;
    p = p * r + C4;
    p = p * r + C3;
    p = p * r + C2;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    uint32_t sb = uint32_t(k + 127) << 23;
    if (sb > 0x7f000000u) sb = 0x7f000000u;
    return p * __uint_as_float(sb);
}

// f32 activations of the fused MatMul epilogues, by fused_activation id
// (kernel_call.rs:861-870): gelu_f, silu_f, sigmoid_f, tanh_f
// (src/cpu/float_kernels.rs:3549-3566), same operation order.
__device__ inline float act_f32(uint32_t act, float x) {
    switch (act) {
        case 2: {   // GELU
            const float cube = ((0.044715f * x) * x) * x;
            const float u = 0.7978846f * (x + cube);
            const float e = exp_det(2.0f * u);
            return (0.5f * x) * (1.0f + (e - 1.0f) / (e + 1.0f));
        }
        case 3: return x * (1.0f / (1.0f + exp_det(-x)));   // SILU
        case 4: return 1.0f / (1.0f + exp_det(-x));         // SIGMOID
        case 5: {                                            // TANH
            const float e = exp_det(2.0f * x);
            return (e - 1.0f) / (e + 1.0f);
        }
        default: return x;
    }
}

}  // namespace holo
