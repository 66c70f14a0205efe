// lut_tables.cpp — host construction of the 65536-entry activation tables the
// GPU gather stages in LDS.
//
// The reference builds T[b] = narrow(f(widen(b))) once per (activation, dtype)
// on the host (crates/hologram-compute/src/cpu/lut.rs:43-72) from
// lut_act_ref (src/cpu/float_kernels.rs:3628-3638). The table is part of the
// result's definition: its NaN entries follow x86-64 SSE semantics (an invalid
// operation yields the default NaN 0xFFC00000, a NaN operand propagates
// quieted), so it is built here on the x86-64 host, compiled without FMA
// contraction, and uploaded to the device once per backend. Every f32
// operation below is in the reference's order.
#include <stdint.h>
#include <string.h>

#include <cmath>

namespace holo {
namespace {

inline uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
inline float float_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

// Rust `f32 as i32`: truncation toward zero, saturating, NaN -> 0.
inline int32_t trunc_sat_i32(float t) {
    if (std::isnan(t)) return 0;
    if (t >= 2147483648.0f) return INT32_MAX;
    if (t <= -2147483904.0f) return INT32_MIN;
    return static_cast<int32_t>(t);
}

// exp_f32_det, src/cpu/simd.rs:4191-4239 (Cody-Waite split + degree-6 Taylor).
float det_exp(float x) {
    if (std::isnan(x) || x < -87.33654f) return 0.0f;
    if (x > 88.0f) x = 88.0f;
    const float t = x * 1.44269504088896340736f;
    const int32_t k = t >= 0.0f ? trunc_sat_i32(t + 0.5f) : trunc_sat_i32(t - 0.5f);
    const float kf = static_cast<float>(k);
    const float r = (x - kf * float_of(0x3F318000u)) - kf * -2.1219444e-4f;
    static const float coeff[5] = {1.0f / 120.0f, 1.0f / 24.0f, 1.0f / 6.0f, 0.5f, 1.0f};
    float p = 1.0f / 720.0f;
    for (float c : coeff) p = p * r + c;
    p = p * r + 1.0f;
    uint32_t scale = static_cast<uint32_t>(k + 127) << 23;
    if (scale > 0x7f000000u) scale = 0x7f000000u;
    return p * float_of(scale);
}

// scalbnf of the libm crate (musl): exact pre-scaling, one final rounding.
float scale_by_pow2(float y, int32_t n) {
    const float two127 = float_of(0x7f000000u);
    const float two_m102 = float_of(0x00800000u) * float_of(0x4b800000u);
    for (int step = 0; step < 2; ++step) {
        if (n > 127) {
            y *= two127;
            n -= 127;
        } else if (n < -126) {
            y *= two_m102;
            n += 102;
        } else {
            break;
        }
    }
    if (n > 127) n = 127;
    if (n < -126) n = -126;
    return y * float_of(static_cast<uint32_t>(0x7f + n) << 23);
}

// libm 0.2.16 expf (the lut_act::EXP entry, float_kernels.rs:3498-3500): the
// published FreeBSD e_expf.c reduction and rational approximation.
float libm_expf(float x) {
    uint32_t ax = bits_of(x);
    const int neg = static_cast<int>(ax >> 31);
    ax &= 0x7fffffffu;
    if (ax >= 0x42aeac50u) {
        if (ax > 0x7f800000u) return x;
        if (!neg && ax >= 0x42b17218u) return x * float_of(0x7f000000u);
        if (neg && ax >= 0x42cff1b5u) return 0.0f;
    }
    int32_t k = 0;
    float hi = x, lo = 0.0f;
    if (ax > 0x3eb17218u) {
        k = ax > 0x3f851592u ? trunc_sat_i32(1.4426950216e+00f * x + (neg ? -0.5f : 0.5f))
                             : 1 - 2 * neg;
        const float kf = static_cast<float>(k);
        hi = x - kf * 6.9314575195e-01f;
        lo = kf * 1.4286067653e-06f;
        x = hi - lo;
    } else if (ax <= 0x39000000u) {
        return 1.0f + x;
    }
    const float xx = x * x;
    const float c = x - xx * (1.6666625440e-1f + xx * -2.7667332906e-3f);
    const float y = 1.0f + (((x * c) / (2.0f - c) - lo) + hi);
    return k == 0 ? y : scale_by_pow2(y, k);
}

float act_sigmoid(float x) { return 1.0f / (1.0f + det_exp(-x)); }
float act_tanh(float x) {
    const float e = det_exp(2.0f * x);
    return (e - 1.0f) / (e + 1.0f);
}
float act_gelu(float x) {
    const float inner = 0.7978846f * (x + ((0.044715f * x) * x) * x);
    return (0.5f * x) * (1.0f + act_tanh(inner));
}
float act_silu(float x) { return x * act_sigmoid(x); }
// relu_f, elu_f, selu_f (src/cpu/float_kernels.rs:3448, 3641-3656). relu is
// x.max(0.0): a NaN or a zero of either sign gives +0.0.
float act_relu(float x) { return x > 0.0f ? x : 0.0f; }
float act_elu(float x) { return x >= 0.0f ? x : libm_expf(x) - 1.0f; }
float act_selu(float x) {
    const float alpha = 1.6732632f, scale = 1.050701f;
    return x >= 0.0f ? scale * x : scale * alpha * (libm_expf(x) - 1.0f);
}

// IEEE binary16 -> binary32 (src/cpu/dtype.rs:94-118).
float half_to_float(uint16_t h) {
    const uint32_t s = static_cast<uint32_t>(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0x1f) return float_of(s | 0x7f800000u | (m << 13));
    if (e != 0) return float_of(s | ((e + 112u) << 23) | (m << 13));
    if (m == 0) return float_of(s);
    int32_t ex = 1;
    while (!(m & 0x400u)) {
        m <<= 1;
        --ex;
    }
    return float_of(s | (static_cast<uint32_t>(112 + ex) << 23) | ((m & 0x3ffu) << 13));
}

// binary32 -> binary16 with the reference's rounding (src/cpu/dtype.rs:121-153):
// add half an ulp of the destination and truncate; overflow saturates to Inf.
uint16_t float_to_half(float f) {
    const uint32_t u = bits_of(f);
    const uint16_t s = static_cast<uint16_t>((u >> 16) & 0x8000u);
    const int32_t e = static_cast<int32_t>((u >> 23) & 0xffu) - 112;
    const uint32_t m = u & 0x7fffffu;
    if (e == 0xff - 112) return static_cast<uint16_t>(s | 0x7c00u | (m ? 0x200u : 0u));
    if (e >= 0x1f) return static_cast<uint16_t>(s | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return s;
        const uint32_t shift = static_cast<uint32_t>(14 - e);
        return static_cast<uint16_t>(s | ((m | 0x800000u) + (1u << (shift - 1))) >> shift);
    }
    const uint32_t r = (m + 0x1000u) >> 13;
    if (r & 0x400u) {
        return e + 1 >= 0x1f ? static_cast<uint16_t>(s | 0x7c00u)
                             : static_cast<uint16_t>(s | ((e + 1) << 10));
    }
    return static_cast<uint16_t>(s | (e << 10) | (r & 0x3ffu));
}

}  // namespace

// Returns false for an activation id this build has no table for. Ids 0-4
// are lut_act's (kernel_call.rs:877-885); 6-8 are this backend's tables for
// the fused epilogues' Relu, Elu and Selu on 16-bit products (the reference
// computes narrow(f(widen(x))) per element, which is the table entry).
bool build_lut_table(int act, bool f16, uint16_t *t) {
    float (*fn)(float) = nullptr;
    switch (act) {
        case 0: fn = act_sigmoid; break;
        case 1: fn = act_tanh; break;
        case 2: fn = act_gelu; break;
        case 3: fn = act_silu; break;
        case 4: fn = libm_expf; break;
        case 6: fn = act_relu; break;
        case 7: fn = act_elu; break;
        case 8: fn = act_selu; break;
        default: return false;
    }
    for (uint32_t b = 0; b < 65536u; ++b) {
        const float x = f16 ? half_to_float(static_cast<uint16_t>(b)) : float_of(b << 16);
        const float y = fn(x);
        t[b] = f16 ? float_to_half(y) : static_cast<uint16_t>(bits_of(y) >> 16);
    }
    return true;
}

// f(x) for lut_act id `act` (lut_act_ref, src/cpu/float_kernels.rs:3628-3638):
// the DequantActivation table's entries. False for an id with no restatement.
bool lut_act_value(int act, float x, float *y) {
    switch (act) {
        case 0: *y = act_sigmoid(x); return true;
        case 1: *y = act_tanh(x); return true;
        case 2: *y = act_gelu(x); return true;
        case 3: *y = act_silu(x); return true;
        case 4: *y = libm_expf(x); return true;
        default: return false;
    }
}

}  // namespace holo
