// holo_device.h — small device-side helpers shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "holo_kernels.h"

namespace holo {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Streaming 16-byte load/store (non-temporal: the data is touched once).
__device__ __forceinline__ u32x4 ld_stream(const u32x4 *p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ void st_stream(u32x4 v, u32x4 *p) { __builtin_nontemporal_store(v, p); }

// f16 -> f32 by bits (src/cpu/dtype.rs:94-118): exact, NaN payload kept.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
    const uint32_t s = (b >> 15) << 31, e = (b >> 10) & 0x1fu, m = b & 0x3ffu;
    if (e == 0x1fu) return __uint_as_float(s | 0x7f800000u | (m << 13));
    if (e != 0) return __uint_as_float(s | ((e + 112u) << 23) | (m << 13));
    if (m == 0) return __uint_as_float(s);
    const int sh = __clz(m) - 21;  // left shifts until the implicit bit (0x400) is set
    return __uint_as_float(s | (uint32_t(113 - sh) << 23) | (((m << sh) & 0x3ffu) << 13));
}

// f32 -> f16 bits with the reference's rule (src/cpu/dtype.rs:121-153): the
// magnitude rounded half up at the cut, overflow to Inf, NaN as the quiet
// NaN of its sign, subnormals by the same half-up shift.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float v) {
    const uint32_t bits = __float_as_uint(v);
    const uint32_t sign = (bits >> 31) & 1u;
    const int32_t ex = int32_t((bits >> 23) & 0xffu);
    const uint32_t mant = bits & 0x7fffffu;
    if (ex == 0xff) return uint16_t((sign << 15) | (0x1fu << 10) | (mant != 0 ? 0x200u : 0u));
    const int32_t ne = ex - 127 + 15;
    if (ne >= 0x1f) return uint16_t((sign << 15) | (0x1fu << 10));
    if (ne <= 0) {
        if (ne < -10) return uint16_t(sign << 15);
        const uint32_t m = mant | 0x800000u;
        const uint32_t shift = uint32_t(1 - ne) + 13;
        return uint16_t((sign << 15) | ((m + (1u << (shift - 1))) >> shift));
    }
    const uint32_t rm = (mant + 0x1000u) >> 13;
    if (rm & 0x400u) {
        const int32_t be = ne + 1;
        if (be >= 0x1f) return uint16_t((sign << 15) | (0x1fu << 10));
        return uint16_t((sign << 15) | (uint32_t(be) << 10));
    }
    return uint16_t((sign << 15) | (uint32_t(ne) << 10) | (rm & 0x3ffu));
}

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

// libm 0.2.16 expf (exp_f, src/cpu/float_kernels.rs:3498-3500): the
// published FreeBSD e_expf.c reduction and rational approximation, then the
// musl scalbnf scaling, with the same operation order as the host table
// builder's restatement (IEEE basic operations, no contraction).
__device__ inline float scale_by_pow2_dev(float y, int32_t n) {
    const float two127 = __uint_as_float(0x7f000000u);
    const float two_m102 = __uint_as_float(0x00800000u) * __uint_as_float(0x4b800000u);
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
    return y * __uint_as_float(uint32_t(0x7f + n) << 23);
}

__device__ inline int32_t trunc_sat_i32_dev(float v) {
    if (v != v) return 0;
    if (v >= 2147483648.0f) return 2147483647;
    if (v < -2147483648.0f) return int32_t(-2147483647 - 1);
    return int32_t(v);
}

__device__ inline float libm_expf_dev(float x) {
    uint32_t ax = __float_as_uint(x);
    const int neg = int(ax >> 31);
    ax &= 0x7fffffffu;
    if (ax >= 0x42aeac50u) {
        if (ax > 0x7f800000u) return x;
        if (!neg && ax >= 0x42b17218u) return x * __uint_as_float(0x7f000000u);
        if (neg && ax >= 0x42cff1b5u) return 0.0f;
    }
    int32_t k = 0;
    float hi = x, lo = 0.0f;
    if (ax > 0x3eb17218u) {
        k = ax > 0x3f851592u ? trunc_sat_i32_dev(1.4426950216e+00f * x + (neg ? -0.5f : 0.5f))
                             : 1 - 2 * neg;
        const float kf = float(k);
        hi = x - kf * 6.9314575195e-01f;
        lo = kf * 1.4286067653e-06f;
        x = hi - lo;
    } else if (ax <= 0x39000000u) {
        return 1.0f + x;
    }
    const float xx = x * x;
    const float c = x - xx * (1.6666625440e-1f + xx * -2.7667332906e-3f);
    const float y = 1.0f + (((x * c) / (2.0f - c) - lo) + hi);
    return k == 0 ? y : scale_by_pow2_dev(y, k);
}

// libm 0.2.16 erff (lut_act::ERF, float_kernels.rs:3534-3536; musl erff.c from
// FreeBSD s_erff.c): the published fdlibm coefficients, nested as written.
__device__ inline float erf_poly(const float *c, int n, float t) {
    float v = c[n - 1];
    for (int i = n - 2; i >= 0; --i) v = c[i] + t * v;
    return v;
}

__device__ inline float libm_erff_dev(float x) {
    constexpr float erx = 8.4506291151e-01f, efx8 = 1.0270333290e+00f;
    const float pp[5] = {1.2837916613e-01f, -3.2504209876e-01f, -2.8481749818e-02f,
                         -5.7702702470e-03f, -2.3763017452e-05f};
    const float qq[5] = {3.9791721106e-01f, 6.5022252500e-02f, 5.0813062117e-03f,
                         1.3249473704e-04f, -3.9602282413e-06f};
    uint32_t ix = __float_as_uint(x);
    const bool neg = (ix >> 31) != 0;
    ix &= 0x7fffffffu;
    if (ix >= 0x7f800000u) return 1.0f - 2.0f * (neg ? 1.0f : 0.0f) + 1.0f / x;
    if (ix < 0x3f580000u) {                       // |x| < 0.84375
        if (ix < 0x31800000u) return 0.125f * (8.0f * x + efx8 * x);
        const float z = x * x;
        const float y = erf_poly(pp, 5, z) / (1.0f + z * erf_poly(qq, 5, z));
        return x + x * y;
    }
    if (ix >= 0x40c00000u) {                      // |x| >= 6: 1 - 2^-120
        const float y = 1.0f - __uint_as_float(0x03800000u);
        return neg ? -y : y;
    }
    float erfc;
    if (ix < 0x3fa00000u) {                       // |x| < 1.25
        const float pa[7] = {-2.3621185683e-03f, 4.1485610604e-01f, -3.7220788002e-01f,
                             3.1834661961e-01f, -1.1089469492e-01f, 3.5478305072e-02f,
                             -2.1663755178e-03f};
        const float qa[6] = {1.0642088205e-01f, 5.4039794207e-01f, 7.1828655899e-02f,
                             1.2617121637e-01f, 1.3637083583e-02f, 1.1984500103e-02f};
        const float s = fabsf(x) - 1.0f;
        erfc = 1.0f - erx - erf_poly(pa, 7, s) / (1.0f + s * erf_poly(qa, 6, s));
    } else {
        const float ax = fabsf(x), s = 1.0f / (ax * ax);
        float r, big_s;
        if (ix < 0x4036db6du) {                   // |x| < 1/0.35
            const float ra[8] = {-9.8649440333e-03f, -6.9385856390e-01f, -1.0558626175e+01f,
                                 -6.2375331879e+01f, -1.6239666748e+02f, -1.8460508728e+02f,
                                 -8.1287437439e+01f, -9.8143291473e+00f};
            const float sa[8] = {1.9651271820e+01f, 1.3765776062e+02f, 4.3456588745e+02f,
                                 6.4538726807e+02f, 4.2900814819e+02f, 1.0863500214e+02f,
                                 6.5702495575e+00f, -6.0424413532e-02f};
            r = erf_poly(ra, 8, s);
            big_s = 1.0f + s * erf_poly(sa, 8, s);
        } else {
            const float rb[7] = {-9.8649431020e-03f, -7.9928326607e-01f, -1.7757955551e+01f,
                                 -1.6063638306e+02f, -6.3756646729e+02f, -1.0250950928e+03f,
                                 -4.8351919556e+02f};
            const float sb[7] = {3.0338060379e+01f, 3.2579251099e+02f, 1.5367296143e+03f,
                                 3.1998581543e+03f, 2.5530502930e+03f, 4.7452853394e+02f,
                                 -2.2440952301e+01f};
            r = erf_poly(rb, 7, s);
            big_s = 1.0f + s * erf_poly(sb, 7, s);
        }
        const float z = __uint_as_float(__float_as_uint(ax) & 0xffffe000u);
        erfc = libm_expf_dev(-z * z - 0.5625f) * libm_expf_dev((z - ax) * (z + ax) + r / big_s) / ax;
    }
    const float y = 1.0f - erfc;
    return neg ? -y : y;
}

// f32 activations of the fused MatMul epilogues, by fused_activation id
// (kernel_call.rs:861-870, fused_act_fn float_kernels.rs:768-780): relu_f
// (:3448), gelu_f, silu_f, sigmoid_f, tanh_f (:3549-3566), elu_f and selu_f
// (:3641-3656), exp_f (libm expf); same operation order.
__device__ inline float act_f32(uint32_t act, float x) {
    switch (act) {
        case 1: return x > 0.0f ? x : 0.0f;                  // RELU: x.max(0.0), NaN -> +0
        case 6: return x >= 0.0f ? x : libm_expf_dev(x) - 1.0f;   // ELU
        case 7: {                                            // SELU
            const float alpha = 1.6732632f, scale = 1.050701f;
            return x >= 0.0f ? scale * x : scale * alpha * (libm_expf_dev(x) - 1.0f);
        }
        case 8: return libm_expf_dev(x);                     // EXP
        case kActErf: return libm_erff_dev(x);               // the Erf unary (f32)
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

// The same, out of line: for epilogues that unroll many elements, where an
// inlined copy per element (the switch with its exp / expf / erff bodies)
// would multiply the kernel's code size (tens of KiB per kernel, re-fetched
// into the instruction cache at every launch) for a path most launches never
// take. The call needs no stack.
__device__ __attribute__((noinline)) inline float act_f32_call(uint32_t act, float x) {
    return act_f32(act, x);
}

// RmsNorm of one bf16 row held as 16-byte vectors: thread t of a 256-thread
// group (waves 0-3 of its workgroup) holds vectors t + 256u (u < kMaxVec, v <
// nv) of x and of gamma. Sum of squares: per thread in vector order with fmaf,
// then a xor tree in each wave, then the four wave sums in order; then
// out = (x * inv) * gamma narrowed by truncation (rms_norm_float,
// src/cpu/float_kernels.rs:1683-1755). The standalone kernel and the fused
// MatMul epilogue share this, so both give the same bits. `part` is 4 floats
// of LDS; every thread of the workgroup must call it (it synchronises).
template <int kMaxVec>
__device__ __forceinline__ void rmsnorm_vec_row(const u32x4 (&xv)[kMaxVec],
                                                const u32x4 (&gv)[kMaxVec], uint32_t nv,
                                                uint32_t feature, float eps, float *part,
                                                u32x4 *__restrict__ orow) {
    const uint32_t t = threadIdx.x;
    float ss = 0.0f;
    if (t < 256) {
#pragma unroll
        for (int u = 0; u < kMaxVec; ++u)
            if (t + 256u * u < nv)
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const float lo = __uint_as_float(xv[u][w] << 16),
                                hi = __uint_as_float(xv[u][w] & 0xFFFF0000u);
                    ss = fmaf(lo, lo, ss);
                    ss = fmaf(hi, hi, ss);
                }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if (t < 256 && (t & 63) == 0) part[t >> 6] = ss;
    __syncthreads();
    if (t >= 256) return;
    const float inv = 1.0f / sqrtf((part[0] + part[1] + part[2] + part[3]) / float(feature) + eps);
#pragma unroll
    for (int u = 0; u < kMaxVec; ++u) {
        const uint32_t v = t + 256u * u;
        if (v >= nv) continue;
        u32x4 r;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float lo = (__uint_as_float(xv[u][w] << 16) * inv) * __uint_as_float(gv[u][w] << 16);
            const float hi = (__uint_as_float(xv[u][w] & 0xFFFF0000u) * inv) *
                             __uint_as_float(gv[u][w] & 0xFFFF0000u);
            r[w] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
        }
        orow[v] = r;
    }
}

}  // namespace holo
