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

// libm 0.2.16 erff (the lut_act::ERF entry, float_kernels.rs:3534-3536): musl's
// erff.c, from FreeBSD's s_erff.c (fdlibm's rational approximations of erf in
// float). Polynomials nest innermost-first as the source writes them.
struct ErfCoeffs {
    static constexpr float erx = 8.4506291151e-01f, efx8 = 1.0270333290e+00f;
    static constexpr float pp[5] = {1.2837916613e-01f, -3.2504209876e-01f, -2.8481749818e-02f,
                                    -5.7702702470e-03f, -2.3763017452e-05f};
    static constexpr float qq[5] = {3.9791721106e-01f, 6.5022252500e-02f, 5.0813062117e-03f,
                                    1.3249473704e-04f, -3.9602282413e-06f};
    static constexpr float pa[7] = {-2.3621185683e-03f, 4.1485610604e-01f, -3.7220788002e-01f,
                                    3.1834661961e-01f, -1.1089469492e-01f, 3.5478305072e-02f,
                                    -2.1663755178e-03f};
    static constexpr float qa[6] = {1.0642088205e-01f, 5.4039794207e-01f, 7.1828655899e-02f,
                                    1.2617121637e-01f, 1.3637083583e-02f, 1.1984500103e-02f};
    static constexpr float ra[8] = {-9.8649440333e-03f, -6.9385856390e-01f, -1.0558626175e+01f,
                                    -6.2375331879e+01f, -1.6239666748e+02f, -1.8460508728e+02f,
                                    -8.1287437439e+01f, -9.8143291473e+00f};
    static constexpr float sa[8] = {1.9651271820e+01f, 1.3765776062e+02f, 4.3456588745e+02f,
                                    6.4538726807e+02f, 4.2900814819e+02f, 1.0863500214e+02f,
                                    6.5702495575e+00f, -6.0424413532e-02f};
    static constexpr float rb[7] = {-9.8649431020e-03f, -7.9928326607e-01f, -1.7757955551e+01f,
                                    -1.6063638306e+02f, -6.3756646729e+02f, -1.0250950928e+03f,
                                    -4.8351919556e+02f};
    static constexpr float sb[7] = {3.0338060379e+01f, 3.2579251099e+02f, 1.5367296143e+03f,
                                    3.1998581543e+03f, 2.5530502930e+03f, 4.7452853394e+02f,
                                    -2.2440952301e+01f};
};

template <int N>
float poly(const float (&c)[N], float t) {
    float v = c[N - 1];
    for (int i = N - 2; i >= 0; --i) v = c[i] + t * v;
    return v;
}

float libm_erff(float x) {
    using C = ErfCoeffs;
    uint32_t ix = bits_of(x);
    const bool neg = (ix >> 31) != 0;
    ix &= 0x7fffffffu;
    if (ix >= 0x7f800000u) return 1.0f - 2.0f * (neg ? 1.0f : 0.0f) + 1.0f / x;
    if (ix < 0x3f580000u) {                       // |x| < 0.84375
        if (ix < 0x31800000u) return 0.125f * (8.0f * x + C::efx8 * x);
        const float z = x * x;
        const float y = poly(C::pp, z) / (1.0f + z * poly(C::qq, z));
        return x + x * y;
    }
    float erfc;
    if (ix >= 0x40c00000u) {                      // |x| >= 6
        const float y = 1.0f - float_of(0x03800000u);
        return neg ? -y : y;
    }
    if (ix < 0x3fa00000u) {                       // |x| < 1.25
        const float s = std::fabs(x) - 1.0f;
        erfc = 1.0f - C::erx - poly(C::pa, s) / (1.0f + s * poly(C::qa, s));
    } else {
        const float ax = std::fabs(x), s = 1.0f / (ax * ax);
        float r, big_s;
        if (ix < 0x4036db6du) {                   // |x| < 1/0.35
            r = poly(C::ra, s);
            big_s = 1.0f + s * poly(C::sa, s);
        } else {
            r = poly(C::rb, s);
            big_s = 1.0f + s * poly(C::sb, s);
        }
        const float z = float_of(bits_of(ax) & 0xffffe000u);
        erfc = libm_expf(-z * z - 0.5625f) * libm_expf((z - ax) * (z + ax) + r / big_s) / ax;
    }
    const float y = 1.0f - erfc;
    return neg ? -y : y;
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

// Returns false for an activation id this build has no table for. Ids 0-5
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
        case 5: fn = libm_erff; break;
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
// the DequantActivation table's entries; Erf for 5 and any id past it.
bool lut_act_value(int act, float x, float *y) {
    switch (act) {
        case 0: *y = act_sigmoid(x); return true;
        case 1: *y = act_tanh(x); return true;
        case 2: *y = act_gelu(x); return true;
        case 3: *y = act_silu(x); return true;
        case 4: *y = libm_expf(x); return true;
        default:
            if (act < 0) return false;
            *y = libm_erff(x);
            return true;
    }
}

}  // namespace holo
