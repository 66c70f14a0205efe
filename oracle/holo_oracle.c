/*
 * holo_oracle.c — CPU restatement of the reference hot path (TEST INFRASTRUCTURE).
 *
 * Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg, as the checker. Build: oracle/Makefile (-O2 -ffp-contract=off
 * -fno-fast-math, x86-64 SSE2). Each function cites the reference file:line it
 * restates (paths under crates/hologram-compute/ unless stated). The pins that
 * check each function are listed in holo_oracle.h.
 */
#include "holo_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* bit helpers                                                              */
/* ------------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Rust's `f32 as i32`: truncate toward zero, saturate, NaN -> 0. */
static inline int32_t rust_f32_as_i32(float t)
{
    if (t != t) return 0;
    if (t >= 2147483648.0f) return INT32_MAX;
    if (t <= -2147483904.0f) return INT32_MIN;
    return (int32_t)t;
}

/* ------------------------------------------------------------------------ */
/* codecs: src/cpu/dtype.rs:69-153                                          */
/* ------------------------------------------------------------------------ */
float or_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }          /* :69-73 */
uint16_t or_f32_to_bf16(float v) { return (uint16_t)(f2u(v) >> 16); }        /* :75-79 */

float or_f16_to_f32(uint16_t bits)                                            /* :94-118 */
{
    uint32_t sign = (bits >> 15) & 1u, ex = (bits >> 10) & 0x1fu, mant = bits & 0x3ffu;
    uint32_t out;
    if (ex == 0) {
        if (mant == 0) {
            out = sign << 31;
        } else {
            uint32_t m = mant;
            int32_t e = 1;
            while ((m & 0x400u) == 0) { m <<= 1; e -= 1; }
            out = (sign << 31) | ((uint32_t)(127 - 15 + e) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (ex == 0x1f) {
        out = (sign << 31) | (0xffu << 23) | (mant << 13);
    } else {
        out = (sign << 31) | ((ex + 127 - 15) << 23) | (mant << 13);
    }
    return u2f(out);
}

uint16_t or_f32_to_f16(float v)                                               /* :121-153 */
{
    uint32_t bits = f2u(v);
    uint16_t sign = (uint16_t)((bits >> 31) & 1u);
    int32_t ex = (int32_t)((bits >> 23) & 0xffu);
    uint32_t mant = bits & 0x7fffffu;
    if (ex == 0xff) {
        uint16_t nan_bit = mant != 0 ? 0x200 : 0;
        return (uint16_t)((sign << 15) | (0x1f << 10) | nan_bit);
    }
    int32_t ne = ex - 127 + 15;
    if (ne >= 0x1f) return (uint16_t)((sign << 15) | (0x1f << 10));
    if (ne <= 0) {
        if (ne < -10) return (uint16_t)(sign << 15);
        uint32_t m = mant | 0x800000u;
        uint32_t shift = (uint32_t)(1 - ne) + 13;
        uint32_t rounded = (m + (1u << (shift - 1))) >> shift;
        return (uint16_t)((sign << 15) | (uint16_t)rounded);
    }
    uint16_t rm = (uint16_t)((mant + 0x1000u) >> 13);
    if (rm & 0x400) {
        int32_t be = ne + 1;
        if (be >= 0x1f) return (uint16_t)((sign << 15) | (0x1f << 10));
        return (uint16_t)((sign << 15) | ((uint16_t)be << 10));
    }
    return (uint16_t)((sign << 15) | ((uint16_t)ne << 10) | (rm & 0x3ff));
}

/* ------------------------------------------------------------------------ */
/* deterministic exp: src/cpu/simd.rs:4191-4239                             */
/* ------------------------------------------------------------------------ */
float or_exp_f32_det(float x)
{
    const float LO = -87.33654f, HI = 88.0f;
    const float LOG2E = 1.44269504088896340736f;     /* core::f32::consts::LOG2_E */
    const float LN2_HI = u2f(0x3F318000u);
    const float LN2_LO = -2.1219444e-4f;
    const float C6 = 1.0f / 720.0f, C5 = 1.0f / 120.0f, C4 = 1.0f / 24.0f,
                C3 = 1.0f / 6.0f, C2 = 0.5f;
    if (x != x || x < LO) return 0.0f;
    if (x > HI) x = HI;
    float t = x * LOG2E;
    int32_t k = t >= 0.0f ? rust_f32_as_i32(t + 0.5f) : rust_f32_as_i32(t - 0.5f);
    float kf = (float)k;
    float r = (x - kf * LN2_HI) - kf * LN2_LO;
    float p = C6;
    p = p * r + C5;
    p = p * r + C4;
    p = p * r + C3;
    p = p * r + C2;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    uint32_t sb = (uint32_t)(k + 127) << 23;
    if (sb > 0x7f000000u) sb = 0x7f000000u;
    return p * u2f(sb);
}

/* ------------------------------------------------------------------------ */
/* libm 0.2.16 `expf` (Cargo.lock:2471-2473; call site float_kernels.rs:3498-3500).
 * The crate is not vendored in the reference. Its expf is the published
 * FreeBSD msun e_expf.c algorithm (as carried by musl): special-case cutoffs,
 * ln2 hi/lo reduction with k = trunc(x/ln2 +- 1/2), the degree-2 rational
 * remez form y = 1 + (x*c/(2-c) - lo + hi), then scalbnf. Restated here from
 * that published algorithm; pinned against a correctly rounded exp.        */
/* ------------------------------------------------------------------------ */
static float or_scalbnf(float x, int32_t n)
{
    const float x1p127 = u2f(0x7f000000u), x1p_126 = u2f(0x00800000u), x1p24 = u2f(0x4b800000u);
    if (n > 127) {
        x *= x1p127;
        n -= 127;
        if (n > 127) {
            x *= x1p127;
            n -= 127;
            if (n > 127) n = 127;
        }
    } else if (n < -126) {
        x *= x1p_126 * x1p24;
        n += 126 - 24;
        if (n < -126) {
            x *= x1p_126 * x1p24;
            n += 126 - 24;
            if (n < -126) n = -126;
        }
    }
    return x * u2f((uint32_t)(0x7f + n) << 23);
}

float or_libm_expf(float x)
{
    const float HALF[2] = {0.5f, -0.5f};
    const float LN2_HI = 6.9314575195e-01f;  /* 0x3f317200 */
    const float LN2_LO = 1.4286067653e-06f;  /* 0x35bfbe8e */
    const float INV_LN2 = 1.4426950216e+00f; /* 0x3fb8aa3b */
    const float P1 = 1.6666625440e-1f;       /* 0xaaaa8f.0p-26 */
    const float P2 = -2.7667332906e-3f;      /* -0xb55215.0p-32 */
    const float x1p127 = u2f(0x7f000000u);
    uint32_t hx = f2u(x);
    int32_t sign = (int32_t)(hx >> 31);
    hx &= 0x7fffffffu;
    if (hx >= 0x42aeac50u) {                 /* |x| >= 87.33655 or NaN */
        if (hx > 0x7f800000u) return x;      /* NaN: returned unchanged */
        if (hx >= 0x42b17218u && !sign) return x * x1p127;   /* overflow */
        if (sign && hx >= 0x42cff1b5u) return 0.0f;          /* x <= -103.97 */
    }
    int32_t k;
    float hi, lo;
    if (hx > 0x3eb17218u) {                  /* |x| > 0.5 ln2 */
        if (hx > 0x3f851592u)                /* |x| > 1.5 ln2 */
            k = rust_f32_as_i32(INV_LN2 * x + HALF[sign]);
        else
            k = 1 - sign - sign;
        float kf = (float)k;
        hi = x - kf * LN2_HI;
        lo = kf * LN2_LO;
        x = hi - lo;
    } else if (hx > 0x39000000u) {           /* |x| > 2^-14 */
        k = 0;
        hi = x;
        lo = 0.0f;
    } else {
        return 1.0f + x;
    }
    float xx = x * x;
    float c = x - xx * (P1 + xx * P2);
    float y = 1.0f + (((x * c) / (2.0f - c) - lo) + hi);
    return k == 0 ? y : or_scalbnf(y, k);
}

/* ------------------------------------------------------------------------ */
/* activations: src/cpu/float_kernels.rs:3537-3566, op order kept, no FMA   */
/* ------------------------------------------------------------------------ */
float or_sigmoid_f(float x) { return 1.0f / (1.0f + or_exp_f32_det(-x)); }
float or_tanh_f(float x)
{
    float e = or_exp_f32_det(2.0f * x);
    return (e - 1.0f) / (e + 1.0f);
}
float or_gelu_f(float x)
{
    /* 0.5 * x * (1.0 + tanh_f(0.797_884_6 * (x + 0.044_715 * x * x * x))) */
    float cube = ((0.044715f * x) * x) * x;
    float u = 0.7978846f * (x + cube);
    return (0.5f * x) * (1.0f + or_tanh_f(u));
}
float or_silu_f(float x) { return x * or_sigmoid_f(x); }

/* fused_act_fn (src/cpu/float_kernels.rs:768-780) over a slice, the f32
 * epilogue of MatMulActivation / MatMulAddActivation. ids: fused_activation
 * (src/kernel_call.rs:861-870). Relu, Elu and Selu are not restated (-1). */
/* relu_f (float_kernels.rs:3448, x.max(0.0): NaN and -0.0 give +0.0), elu_f
 * and selu_f (:3641-3656) */
static float relu_f(float x) { return x > 0.0f ? x : 0.0f; }
static float elu_f(float x) { return x >= 0.0f ? x : or_libm_expf(x) - 1.0f; }
static float selu_f(float x)
{
    const float alpha = 1.6732632f, scale = 1.050701f;
    return x >= 0.0f ? scale * x : scale * alpha * (or_libm_expf(x) - 1.0f);
}

int or_fused_act_f32(int act, const float *in, float *out, size_t n)
{
    for (size_t i = 0; i < n; ++i) {
        switch (act) {
        case 1: out[i] = relu_f(in[i]); break;
        case 6: out[i] = elu_f(in[i]); break;
        case 7: out[i] = selu_f(in[i]); break;
        case 2: out[i] = or_gelu_f(in[i]); break;
        case 3: out[i] = or_silu_f(in[i]); break;
        case 4: out[i] = or_sigmoid_f(in[i]); break;
        case 5: out[i] = or_tanh_f(in[i]); break;
        case 8: out[i] = or_libm_expf(in[i]); break;
        default: return -1;
        }
    }
    return 0;
}

/* libm 0.2.16 erff (the lut_act::ERF entry, float_kernels.rs:3534-3536): the
 * crate ports musl's src/math/erff.c, itself FreeBSD's s_erff.c (fdlibm's
 * erf rational approximations in float). Four ranges of |x|: [0, 0.84375)
 * x + x*P(x^2)/Q(x^2); [0.84375, 1.25) 1 - ((1 - erx) - P(s)/Q(s)) with
 * s = |x| - 1; [1.25, 6) 1 - exp(-z^2 - 0.5625) exp((z - x)(z + x) + R/S) / x
 * with z = x truncated to 11 mantissa bits and R/S in 1/x^2; beyond, 1 - 2^-120.
 * The coefficients are the published ones (each also given as its bits). */
static const float ERF_ERX = 8.4506291151e-01f;   /* 0x3f58560b */
static const float ERF_EFX8 = 1.0270333290e+00f;  /* 0x3f8375d4 */
static const float ERF_PP[5] = {1.2837916613e-01f, -3.2504209876e-01f, -2.8481749818e-02f,
                                -5.7702702470e-03f, -2.3763017452e-05f};
static const float ERF_QQ[5] = {3.9791721106e-01f, 6.5022252500e-02f, 5.0813062117e-03f,
                                1.3249473704e-04f, -3.9602282413e-06f};
static const float ERF_PA[7] = {-2.3621185683e-03f, 4.1485610604e-01f, -3.7220788002e-01f,
                                3.1834661961e-01f, -1.1089469492e-01f, 3.5478305072e-02f,
                                -2.1663755178e-03f};
static const float ERF_QA[6] = {1.0642088205e-01f, 5.4039794207e-01f, 7.1828655899e-02f,
                                1.2617121637e-01f, 1.3637083583e-02f, 1.1984500103e-02f};
static const float ERF_RA[8] = {-9.8649440333e-03f, -6.9385856390e-01f, -1.0558626175e+01f,
                                -6.2375331879e+01f, -1.6239666748e+02f, -1.8460508728e+02f,
                                -8.1287437439e+01f, -9.8143291473e+00f};
static const float ERF_SA[8] = {1.9651271820e+01f, 1.3765776062e+02f, 4.3456588745e+02f,
                                6.4538726807e+02f, 4.2900814819e+02f, 1.0863500214e+02f,
                                6.5702495575e+00f, -6.0424413532e-02f};
static const float ERF_RB[7] = {-9.8649431020e-03f, -7.9928326607e-01f, -1.7757955551e+01f,
                                -1.6063638306e+02f, -6.3756646729e+02f, -1.0250950928e+03f,
                                -4.8351919556e+02f};
static const float ERF_SB[7] = {3.0338060379e+01f, 3.2579251099e+02f, 1.5367296143e+03f,
                                3.1998581543e+03f, 2.5530502930e+03f, 4.7452853394e+02f,
                                -2.2440952301e+01f};

/* c[0] + t*(c[1] + t*(... + t*c[n-1])), innermost first, as the source nests it */
static float horner(const float *c, int n, float t)
{
    float v = c[n - 1];
    for (int i = n - 2; i >= 0; --i) v = c[i] + t * v;
    return v;
}

/* 1 + t*(c[0] + t*(c[1] + ...)) */
static float horner1(const float *c, int n, float t) { return 1.0f + t * horner(c, n, t); }

static float erfc_mid(float x)          /* |x| in [0.84375, 1.25) */
{
    float s = fabsf(x) - 1.0f;
    float p = horner(ERF_PA, 7, s);
    float q = horner1(ERF_QA, 6, s);
    return 1.0f - ERF_ERX - p / q;
}

static float erfc_tail(uint32_t ix, float x)   /* |x| in [0.84375, 6) */
{
    if (ix < 0x3fa00000u) return erfc_mid(x);
    x = fabsf(x);
    float s = 1.0f / (x * x);
    float r, big_s;
    if (ix < 0x4036db6du) {             /* |x| < 1/0.35 */
        r = horner(ERF_RA, 8, s);
        big_s = horner1(ERF_SA, 8, s);
    } else {
        r = horner(ERF_RB, 7, s);
        big_s = horner1(ERF_SB, 7, s);
    }
    float z = u2f(f2u(x) & 0xffffe000u);
    return or_libm_expf(-z * z - 0.5625f) * or_libm_expf((z - x) * (z + x) + r / big_s) / x;
}

float or_libm_erff(float x)
{
    uint32_t ix = f2u(x);
    int sign = (int)(ix >> 31);
    ix &= 0x7fffffffu;
    if (ix >= 0x7f800000u) return 1.0f - 2.0f * (float)sign + 1.0f / x;   /* NaN, +-Inf */
    if (ix < 0x3f580000u) {             /* |x| < 0.84375 */
        if (ix < 0x31800000u) return 0.125f * (8.0f * x + ERF_EFX8 * x);  /* |x| < 2^-28 */
        float z = x * x;
        float y = horner(ERF_PP, 5, z) / horner1(ERF_QQ, 5, z);
        return x + x * y;
    }
    float y = ix < 0x40c00000u ? 1.0f - erfc_tail(ix, x) : 1.0f - u2f(0x03800000u);
    return sign ? -y : y;
}

float or_lut_act_ref(int act, float x)
{
    switch (act) {
    case OR_ACT_SIGMOID: return or_sigmoid_f(x);
    case OR_ACT_TANH: return or_tanh_f(x);
    case OR_ACT_GELU: return or_gelu_f(x);
    case OR_ACT_SILU: return or_silu_f(x);
    case OR_ACT_EXP: return or_libm_expf(x);
    default: return or_libm_erff(x);          /* lut_act::ERF and any other id */
    }
}

/* ------------------------------------------------------------------------ */
/* LUT build / gather: src/cpu/lut.rs:43-67, 76-98                          */
/* ------------------------------------------------------------------------ */
int or_build_table(int act, int dtype, uint16_t *t)
{
    if (act < 0 || act > OR_ACT_ERF) return -1;
    if (dtype != OR_DTYPE_BF16 && dtype != OR_DTYPE_F16) return -1;
    for (uint32_t bits = 0; bits < 65536u; ++bits) {
        float x = dtype == OR_DTYPE_F16 ? or_f16_to_f32((uint16_t)bits)
                                        : or_bf16_to_f32((uint16_t)bits);
        float y = or_lut_act_ref(act, x);
        t[bits] = dtype == OR_DTYPE_F16 ? or_f32_to_f16(y) : or_f32_to_bf16(y);
    }
    return 0;
}

void or_unary_lut(const uint16_t *t, const uint16_t *in, uint16_t *out, size_t n)
{
    for (size_t i = 0; i < n; ++i) out[i] = t[in[i]];
}

/* ------------------------------------------------------------------------ */
/* int8 scheme: src/cpu/simd.rs:4755-4785                                   */
/* ------------------------------------------------------------------------ */
float or_quantize_row_i8(const float *a, int8_t *q, size_t k)
{
    float amax = 0.0f;
    for (size_t i = 0; i < k; ++i) {
        float v = a[i];
        float av = v < 0.0f ? -v : v;
        if (av > amax) amax = av;
    }
    if (amax == 0.0f) return 0.0f;           /* q left untouched, as the reference */
    float inv = 127.0f / amax;
    for (size_t i = 0; i < k; ++i) {
        float t = a[i] * inv;
        int32_t r = t >= 0.0f ? rust_f32_as_i32(t + 0.5f) : rust_f32_as_i32(t - 0.5f);
        if (r < -127) r = -127;
        if (r > 127) r = 127;
        q[i] = (int8_t)r;
    }
    return amax / 127.0f;
}

/* simd.rs:5295-5480 with the portable inner of :5203-5215: exact i32 dot,
 * out = (acc as f32) * (scale_a * scales[j]); an all-zero row writes zeros. */
/* The output-major weight's integer level at (column j, row kk), per tier:
 * i8 one byte (quant_tier.rs I8); i4 packed nibbles, unit u = j*k + kk in the
 * low nibble of byte u/2 when u is even, sign-extended from bit 3
 * (omajor_repack :117-131, ScalarQuant::read float_kernels.rs:440-455); e8cb a
 * codebook index per 8-row group, the level codebook[idx*8 + kk%8]
 * (matmul_e8cb_omajor simd.rs:6867-6900). */
static int32_t omajor_level(int tier, const uint8_t *bq, const int8_t *cb, size_t j, size_t kk,
                            size_t k)
{
    if (tier == OR_DTYPE_I4) {
        size_t u = j * k + kk;
        int32_t v = (u & 1) ? (bq[u >> 1] >> 4) : (bq[u >> 1] & 0x0F);
        return v >= 8 ? v - 16 : v;
    }
    if (tier == OR_DTYPE_E8CB) return cb[(size_t)bq[j * (k / 8) + kk / 8] * 8 + kk % 8];
    return (int8_t)bq[j * k + kk];
}

int or_matmul_q_omajor(int tier, const float *a, const uint8_t *bq, const int8_t *codebook,
                       const float *scales, float *out, size_t m, size_t k, size_t n)
{
    if (tier != OR_DTYPE_I8 && tier != OR_DTYPE_I4 && tier != OR_DTYPE_E8CB) return 3;
    if ((tier == OR_DTYPE_I4 && k % 2) || (tier == OR_DTYPE_E8CB && k % 8)) return 3;
    if (k > OR_I8_DOT_K_MAX) return 3;
    int8_t *q = (int8_t *)malloc(k ? k : 1);
    for (size_t i = 0; i < m; ++i) {
        memset(q, 0, k);
        float sa = or_quantize_row_i8(a + i * k, q, k);
        if (sa == 0.0f) {
            for (size_t j = 0; j < n; ++j) out[i * n + j] = 0.0f;
            continue;
        }
        for (size_t j = 0; j < n; ++j) {
            int32_t acc = 0;
            for (size_t kk = 0; kk < k; ++kk)
                acc += (int32_t)q[kk] * omajor_level(tier, bq, codebook, j, kk, k);
            out[i * n + j] = (float)acc * (sa * scales[j]);
        }
    }
    free(q);
    return 0;
}

void or_matmul_i8_pc_omajor(const float *a, const int8_t *bq, const float *scales,
                            float *out, size_t m, size_t k, size_t n)
{
    or_matmul_q_omajor(OR_DTYPE_I8, a, (const uint8_t *)bq, NULL, scales, out, m, k, n);
}

/* ------------------------------------------------------------------------ */
/* dequantize: src/cpu/kernels.rs:185-296; dequant_activation :311-388        */
/* ------------------------------------------------------------------------ */
/* The stored level of element i: i8 two's complement, u8 the raw byte, i4 a
 * nibble (low first) sign-extended from bit 3 (kernels.rs:247-270). */
static int32_t scalar_level(int quant, const uint8_t *in, uint64_t i)
{
    if (quant == OR_DTYPE_I8) return (int32_t)(int8_t)in[i];
    if (quant == OR_DTYPE_U8) return (int32_t)in[i];
    uint8_t nib = (i % 2 == 0) ? (in[i / 2] & 0x0f) : (in[i / 2] >> 4);
    return nib >= 8 ? (int32_t)nib - 16 : (int32_t)nib;
}

/* (q - zp) in two's complement i32, as the reference's release build wraps */
static int32_t wrap_sub(int32_t a, int32_t b) { return (int32_t)((uint32_t)a - (uint32_t)b); }

int or_dequantize(const uint8_t *in, uint64_t n, int quant, const float *scales,
                  const int32_t *zps, uint32_t channels, uint32_t inner, float scale,
                  int32_t zp, int dtype, void *out)
{
    if (quant != OR_DTYPE_I8 && quant != OR_DTYPE_U8 && quant != OR_DTYPE_I4) return 1;
    if (dtype != OR_DTYPE_F32 && dtype != OR_DTYPE_BF16 && dtype != OR_DTYPE_F16) return 1;
    int per_ch = channels > 0 && scales != NULL;
    uint64_t in_step = inner ? inner : 1;
    for (uint64_t i = 0; i < n; ++i) {
        float s = scale;
        int32_t z = zp;
        if (per_ch) {
            uint64_t ch = (i / in_step) % channels;
            s = scales[ch];
            z = zps[ch];
        }
        float v = (float)wrap_sub(scalar_level(quant, in, i), z) * s;
        if (dtype == OR_DTYPE_F32) ((float *)out)[i] = v;
        else if (dtype == OR_DTYPE_BF16) ((uint16_t *)out)[i] = or_f32_to_bf16(v);
        else ((uint16_t *)out)[i] = or_f32_to_f16(v);
    }
    return 0;
}

int or_dequant_activation(const uint8_t *in, uint64_t n, int quant, int act, float scale,
                          int32_t zp, float *out)
{
    if (quant != OR_DTYPE_I8 && quant != OR_DTYPE_U8 && quant != OR_DTYPE_I4) return 1;
    float table[256];
    int levels = quant == OR_DTYPE_I4 ? 16 : 256;
    for (int raw = 0; raw < levels; ++raw) {
        int32_t q = quant == OR_DTYPE_I8 ? (int32_t)(int8_t)(uint8_t)raw
                  : quant == OR_DTYPE_U8 ? raw : (raw >= 8 ? raw - 16 : raw);
        table[raw] = or_lut_act_ref(act, (float)wrap_sub(q, zp) * scale);
    }
    for (uint64_t i = 0; i < n; ++i) {
        int raw = quant == OR_DTYPE_I4 ? ((i % 2 == 0) ? (in[i / 2] & 0x0f) : (in[i / 2] >> 4))
                                       : in[i];
        out[i] = table[raw];
    }
    return 0;
}

/* FNV-1a over the LE bytes of each f32 (simd.rs:8237-8246). */
uint64_t or_fnv1a_f32(const float *v, size_t n)
{
    uint64_t h = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < n; ++i) {
        uint32_t u = f2u(v[i]);
        for (int b = 0; b < 4; ++b) {
            h ^= (u >> (8 * b)) & 0xffu;
            h *= 0x100000001b3ull;
        }
    }
    return h;
}

/* ------------------------------------------------------------------------ */
/* KV write: src/cpu/kernels.rs:455-501                                     */
/* ------------------------------------------------------------------------ */
int or_kv_cache_write(const uint8_t *cache, const uint8_t *nw, uint32_t posv, uint8_t *out,
                      uint32_t planes, uint32_t bucket, uint32_t new_rows, uint32_t row)
{
    if (bucket == 0 || row == 0) return 3;   /* UnsupportedOp */
    if (new_rows > bucket) return 3;
    size_t plane_bytes = (size_t)bucket * row;
    size_t pos = (size_t)posv % bucket;
    memcpy(out, cache, (size_t)planes * plane_bytes);
    for (size_t p = 0; p < planes; ++p) {
        size_t ob = p * plane_bytes, nb = p * (size_t)new_rows * row;
        for (size_t j = 0; j < new_rows; ++j) {
            size_t dst = ob + ((pos + j) % bucket) * row;
            memcpy(out + dst, nw + nb + j * row, row);
        }
    }
    return 0;
}

static float widen(const void *base, int dtype, size_t i)
{
    if (dtype == OR_DTYPE_BF16) return or_bf16_to_f32(((const uint16_t *)base)[i]);
    if (dtype == OR_DTYPE_F16) return or_f16_to_f32(((const uint16_t *)base)[i]);
    return ((const float *)base)[i];
}

int or_kv_quant_append(const void *nw, int dtype, uint32_t posv, int8_t *cq, float *cs,
                       uint32_t planes, uint32_t bucket, uint32_t new_rows, uint32_t d)
{
    float row[8192];
    if (bucket == 0 || d == 0 || d > 8192) return 3;
    if (new_rows > bucket) return 3;
    if (dtype != OR_DTYPE_BF16 && dtype != OR_DTYPE_F16 && dtype != OR_DTYPE_F32) return 3;
    size_t pos = (size_t)posv % bucket;
    for (size_t p = 0; p < planes; ++p) {
        for (size_t j = 0; j < new_rows; ++j) {
            size_t src = (p * new_rows + j) * (size_t)d;
            for (size_t c = 0; c < d; ++c) row[c] = widen(nw, dtype, src + c);
            size_t r = p * (size_t)bucket + (pos + j) % bucket;
            int8_t *dst = cq + r * d;
            memset(dst, 0, d);                 /* all-zero row: q defined as 0 */
            cs[r] = or_quantize_row_i8(row, dst, d);
        }
    }
    return 0;
}

void or_dequant_i8(const int8_t *q, const float *scales, float *out, size_t rows, size_t len)
{
    for (size_t r = 0; r < rows; ++r)
        for (size_t c = 0; c < len; ++c)
            out[r * len + c] = (float)q[r * len + c] * scales[r];   /* kernels.rs:270 */
}

/* ------------------------------------------------------------------------ */
/* decode attention: src/cpu/float_kernels.rs:3834-3957, 4192-4307          */
/* ------------------------------------------------------------------------ */
float or_attn_scale(uint32_t d, uint32_t scale_bits)             /* :4256-4266 */
{
    float dflt = sqrtf((float)d);
    if (dflt < 1.0f) dflt = 1.0f;
    if (scale_bits == 0) return dflt;
    float sm = u2f(scale_bits);
    return sm > 0.0f ? 1.0f / sm : dflt;
}

/* one (b, h, q-row): :3834-3883. The dot is a sequential scalar sum here; the
 * reference's SIMD lane order differs in the last bits (tolerance metric). */
static void valid_row(const float *q, const float *kp, const float *vp, const float *kn,
                      const float *vn, float *out, size_t vis_past, size_t new_vis, size_t d,
                      float scale, float *sc)
{
    size_t vis = vis_past + new_vis;
    for (size_t c = 0; c < d; ++c) out[c] = 0.0f;
    if (vis == 0) return;
    for (size_t j = 0; j < vis; ++j) {
        const float *kr = j < vis_past ? kp + j * d : kn + (j - vis_past) * d;
        float s = 0.0f;
        for (size_t c = 0; c < d; ++c) s += q[c] * kr[c];
        sc[j] = s / scale;
    }
    float mx = -INFINITY;
    for (size_t j = 0; j < vis; ++j) mx = fmaxf(mx, sc[j]);
    for (size_t j = 0; j < vis; ++j) sc[j] = or_exp_f32_det(sc[j] - mx);
    float sum = 0.0f;
    for (size_t j = 0; j < vis; ++j) sum += sc[j];
    float denom = sum > 1e-30f ? sum : 1e-30f;
    for (size_t j = 0; j < vis; ++j) {
        float p = sc[j] / denom;
        const float *vr = j < vis_past ? vp + j * d : vn + (j - vis_past) * d;
        for (size_t c = 0; c < d; ++c) out[c] += p * vr[c];
    }
}

#include <stdlib.h>
void or_decode_attention_valid_f32(const float *q, const float *kp, const float *vp,
                                   const float *kn, const float *vn, float *out,
                                   uint32_t b, uint32_t h, uint32_t hkv, uint32_t m,
                                   uint32_t past, uint32_t nnew, uint32_t d, float scale,
                                   uint32_t vis_past)
{
    /* :3899-3957: row r -> (bi, hi, qi); kvh = bi*hkv + hi/group */
    if (hkv == 0) hkv = h;
    size_t group = h / hkv;
    if (vis_past > past) vis_past = past;
    float *sc = (float *)malloc(sizeof(float) * ((size_t)past + nnew + 1));
    size_t rows = (size_t)b * h * m;
    for (size_t r = 0; r < rows; ++r) {
        size_t bi = r / ((size_t)h * m), hi = (r / m) % h, qi = r % m;
        size_t kvh = bi * hkv + hi / group;
        size_t new_vis = qi + 1 < nnew ? qi + 1 : nnew;
        valid_row(q + r * d, kp + kvh * (size_t)past * d, vp + kvh * (size_t)past * d,
                  kn + kvh * (size_t)nnew * d, vn + kvh * (size_t)nnew * d, out + r * d,
                  vis_past, new_vis, d, scale, sc);
    }
    free(sc);
}

static float *widen_all(const void *src, int dtype, size_t n)
{
    float *o = (float *)malloc(sizeof(float) * (n ? n : 1));
    for (size_t i = 0; i < n; ++i) o[i] = widen(src, dtype, i);
    return o;
}

int or_decode_attention_valid(const void *q, const void *k_past, const void *v_past,
                              const void *k_new, const void *v_new, uint32_t valid_len, void *out,
                              uint32_t b, uint32_t h, uint32_t hkv, uint32_t m, uint32_t past,
                              uint32_t nnew, uint32_t d, uint32_t scale_bits, int dtype)
{
    /* :4199-4216: empty shapes, the q_rows == new_len >= 1 law, the GQA map */
    if (b == 0 || h == 0 || d == 0) return 0;
    if (m == 0 || m != nnew) return 3;
    if (hkv == 0) hkv = h;
    if (h % hkv != 0) return 3;
    if (dtype != OR_DTYPE_F32 && dtype != OR_DTYPE_BF16 && dtype != OR_DTYPE_F16) return 3;
    size_t qn = (size_t)b * h * m * d, pn = (size_t)b * hkv * past * d, nn = (size_t)b * hkv * nnew * d;
    float *q32 = widen_all(q, dtype, qn), *kp = widen_all(k_past, dtype, pn);
    float *vp = widen_all(v_past, dtype, pn), *kn = widen_all(k_new, dtype, nn);
    float *vn = widen_all(v_new, dtype, nn);
    float *o = (float *)malloc(sizeof(float) * qn);
    uint32_t vis = valid_len < past ? valid_len : past;              /* :4254 */
    or_decode_attention_valid_f32(q32, kp, vp, kn, vn, o, b, h, hkv, m, past, nnew, d,
                                  or_attn_scale(d, scale_bits), vis);
    for (size_t i = 0; i < qn; ++i) {
        if (dtype == OR_DTYPE_F32) ((float *)out)[i] = o[i];
        else if (dtype == OR_DTYPE_BF16) ((uint16_t *)out)[i] = or_f32_to_bf16(o[i]);
        else ((uint16_t *)out)[i] = or_f32_to_f16(o[i]);
    }
    free(q32); free(kp); free(vp); free(kn); free(vn); free(o);
    return 0;
}

/* DecodeAttention, the mask form. One (b, h, q-row), :2420-2477: scores over
 * past then new keys, each dot / scale + the row's mask entry; a row whose
 * largest score is -inf is the zero row; then max-shift, exp_f32_det, the
 * sequential sum, denom = max(sum, 1e-30), out = sum_j (e_j / denom) v_j. */
static void mask_row(const float *q, const float *kp, const float *vp, const float *kn,
                     const float *vn, const float *mrow, float *out, size_t past, size_t nnew,
                     size_t d, float scale, float *sc)
{
    size_t l = past + nnew;
    for (size_t j = 0; j < l; ++j) {
        const float *kr = j < past ? kp + j * d : kn + (j - past) * d;
        float s = 0.0f;
        for (size_t c = 0; c < d; ++c) s += q[c] * kr[c];
        sc[j] = s / scale + mrow[j];
    }
    float mx = -INFINITY;
    for (size_t j = 0; j < l; ++j) mx = fmaxf(mx, sc[j]);
    for (size_t c = 0; c < d; ++c) out[c] = 0.0f;
    if (mx == -INFINITY) return;
    for (size_t j = 0; j < l; ++j) sc[j] = or_exp_f32_det(sc[j] - mx);
    float sum = 0.0f;
    for (size_t j = 0; j < l; ++j) sum += sc[j];
    float denom = sum > 1e-30f ? sum : 1e-30f;
    for (size_t j = 0; j < l; ++j) {
        float p = sc[j] / denom;
        const float *vr = j < past ? vp + j * d : vn + (j - past) * d;
        for (size_t c = 0; c < d; ++c) out[c] += p * vr[c];
    }
}

/* serial engine, :2606-2660: row r -> (bi, hi, qi), kv head bi*hkv + hi/group,
 * mask row qi of [m][past + nnew] (shared by batch and heads) */
void or_decode_attention_mask_f32(const float *q, const float *kp, const float *vp,
                                  const float *kn, const float *vn, const float *mask, float *out,
                                  uint32_t b, uint32_t h, uint32_t hkv, uint32_t m,
                                  uint32_t past, uint32_t nnew, uint32_t d, float scale)
{
    if (hkv == 0) hkv = h;
    size_t group = h / hkv, l = (size_t)past + nnew;
    float *sc = (float *)malloc(sizeof(float) * (l + 1));
    size_t rows = (size_t)b * h * m;
    for (size_t r = 0; r < rows; ++r) {
        size_t bi = r / ((size_t)h * m), hi = (r / m) % h, qi = r % m;
        size_t kvh = bi * hkv + hi / group;
        mask_row(q + r * d, kp + kvh * (size_t)past * d, vp + kvh * (size_t)past * d,
                 kn + kvh * (size_t)nnew * d, vn + kvh * (size_t)nnew * d, mask + qi * l,
                 out + r * d, past, nnew, d, scale, sc);
    }
    free(sc);
}

int or_decode_attention(const void *q, const void *k_past, const void *v_past, const void *k_new,
                        const void *v_new, const float *mask, void *out, uint32_t b, uint32_t h,
                        uint32_t hkv, uint32_t m, uint32_t past, uint32_t nnew, uint32_t d,
                        uint32_t scale_bits, int dtype)
{
    /* :2489-2511 and :2576-2580: empty shapes, an empty key list, the GQA map,
     * then the compute dtypes */
    if (b == 0 || h == 0 || m == 0 || d == 0) return 0;
    if ((size_t)past + nnew == 0) return 3;
    if (hkv == 0) hkv = h;
    if (h % hkv != 0) return 3;
    if (dtype != OR_DTYPE_F32 && dtype != OR_DTYPE_BF16 && dtype != OR_DTYPE_F16) return 3;
    size_t qn = (size_t)b * h * m * d, pn = (size_t)b * hkv * past * d, nn = (size_t)b * hkv * nnew * d;
    float *q32 = widen_all(q, dtype, qn), *kp = widen_all(k_past, dtype, pn);
    float *vp = widen_all(v_past, dtype, pn), *kn = widen_all(k_new, dtype, nn);
    float *vn = widen_all(v_new, dtype, nn);
    float *o = (float *)malloc(sizeof(float) * qn);
    or_decode_attention_mask_f32(q32, kp, vp, kn, vn, mask, o, b, h, hkv, m, past, nnew, d,
                                 or_attn_scale(d, scale_bits));
    for (size_t i = 0; i < qn; ++i) {
        if (dtype == OR_DTYPE_F32) ((float *)out)[i] = o[i];
        else if (dtype == OR_DTYPE_BF16) ((uint16_t *)out)[i] = or_f32_to_bf16(o[i]);
        else ((uint16_t *)out)[i] = or_f32_to_f16(o[i]);
    }
    free(q32); free(kp); free(vp); free(kn); free(vn); free(o);
    return 0;
}

void or_decode_attention_i8(const float *q, const int8_t *kq, const float *ks,
                            const int8_t *vq, const float *vs, const uint32_t *lens,
                            float *out, uint32_t B, uint32_t H, uint32_t Hkv,
                            uint32_t bucket, uint32_t D, float scale)
{
    size_t group = H / Hkv;
    float *kd = (float *)malloc(sizeof(float) * (size_t)bucket * D);
    float *vd = (float *)malloc(sizeof(float) * (size_t)bucket * D);
    float *sc = (float *)malloc(sizeof(float) * ((size_t)bucket + 1));
    for (size_t b = 0; b < B; ++b) {
        size_t L = lens[b] < bucket ? lens[b] : bucket;
        for (size_t kh = 0; kh < Hkv; ++kh) {
            size_t plane = b * Hkv + kh;
            or_dequant_i8(kq + plane * (size_t)bucket * D, ks + plane * (size_t)bucket, kd, L, D);
            or_dequant_i8(vq + plane * (size_t)bucket * D, vs + plane * (size_t)bucket, vd, L, D);
            for (size_t g = 0; g < group; ++g) {
                size_t hh = kh * group + g;
                const float *qr = q + (b * H + hh) * D;
                float *orow = out + (b * H + hh) * D;
                if (L == 0) {
                    for (size_t c = 0; c < D; ++c) orow[c] = 0.0f;
                    continue;
                }
                /* past = L-1 dequantized rows, new = the last row (q_rows = new = 1) */
                valid_row(qr, kd, vd, kd + (L - 1) * D, vd + (L - 1) * D, orow, L - 1, 1, D,
                          scale, sc);
            }
        }
    }
    free(kd);
    free(vd);
    free(sc);
}

/* ------------------------------------------------------------------------ */
/* MatMul reference: tests/conformance.rs:100-112, metric :138-144          */
/* ------------------------------------------------------------------------ */
void or_matmul_ref_f64(const float *a, const float *b, float *out, size_t m, size_t k, size_t n)
{
    double *acc = (double *)malloc(sizeof(double) * n);
    for (size_t i = 0; i < m; ++i) {
        for (size_t j = 0; j < n; ++j) acc[j] = 0.0;
        for (size_t p = 0; p < k; ++p) {
            double av = (double)a[i * k + p];
            const float *br = b + p * n;
            for (size_t j = 0; j < n; ++j) acc[j] += av * (double)br[j];
        }
        for (size_t j = 0; j < n; ++j) out[i * n + j] = (float)acc[j];
    }
    free(acc);
}

double or_max_rel_err(const float *got, const float *want, size_t n)
{
    double scale = 0.0, worst = 0.0;
    for (size_t i = 0; i < n; ++i) {
        double w = fabs((double)want[i]);
        if (w > scale) scale = w;
    }
    scale += 1e-9;
    for (size_t i = 0; i < n; ++i) {
        double e = fabs((double)got[i] - (double)want[i]) / scale;
        if (e > worst || e != e) worst = e != e ? INFINITY : e;
    }
    return worst;
}

/* ------------------------------------------------------------------------ */
/* Decode-step ops. Element access widens bf16 and f16 (exact) and narrows  */
/* bf16 by truncation and f16 by the reference's rounding, as read_float /  */
/* write_float do (src/cpu/dtype.rs:69-153).                                */
static float rd(const void *p, size_t i, int dtype)
{
    if (dtype == OR_DTYPE_BF16) return or_bf16_to_f32(((const uint16_t *)p)[i]);
    if (dtype == OR_DTYPE_F16) return or_f16_to_f32(((const uint16_t *)p)[i]);
    return ((const float *)p)[i];
}

static void wr(void *p, size_t i, float v, int dtype)
{
    if (dtype == OR_DTYPE_BF16)
        ((uint16_t *)p)[i] = or_f32_to_bf16(v);
    else if (dtype == OR_DTYPE_F16)
        ((uint16_t *)p)[i] = or_f32_to_f16(v);
    else
        ((float *)p)[i] = v;
}

/* binary_float, src/cpu/float_kernels.rs:238-300 (scalar loop :290-298) */
void or_binary(int op, const void *a, const void *b, void *out, size_t n, int dtype)
{
    for (size_t i = 0; i < n; ++i) {
        const float va = rd(a, i, dtype), vb = rd(b, i, dtype);
        wr(out, i, op == 0 ? va + vb : va * vb, dtype);
    }
}

/* rms_norm_float generic path, src/cpu/float_kernels.rs:1737-1754;
 * epsilon rule :1324-1336. Returns -1 for an invalid epsilon. */
int or_rms_norm(const void *x, const void *gamma, void *out, uint32_t batch, uint32_t feature,
                uint64_t epsilon_bits, int dtype)
{
    float eps = 1e-9f;
    if (epsilon_bits != 0) {
        eps = u2f((uint32_t)epsilon_bits);
        if (!(isfinite(eps) && eps > 0.0f)) return -1;
    }
    for (uint32_t bi = 0; bi < batch; ++bi) {
        const size_t row = (size_t)bi * feature;
        float sumsq = 0.0f;
        for (uint32_t j = 0; j < feature; ++j) {
            const float v = rd(x, row + j, dtype);
            sumsq += v * v;
        }
        const float inv_rms = 1.0f / sqrtf(sumsq / (float)feature + eps);
        for (uint32_t j = 0; j < feature; ++j) {
            const float g = gamma ? rd(gamma, j, dtype) : 1.0f;
            wr(out, row + j, rd(x, row + j, dtype) * inv_rms * g, dtype);
        }
    }
    return 0;
}

/* add_rms_norm_float, src/cpu/float_kernels.rs:1566-1672: v = x + residual in
 * f32 (never narrowed), sequential f32 sum of squares; the f32 rows with a
 * residual scale in place by (inv * g) (:1625-1634), every other form writes
 * (v * inv) * g (:1636-1650, 1656-1671). residual may be NULL. */
int or_add_rms_norm(const void *x, const void *res, const void *gamma, void *out, uint32_t batch,
                    uint32_t feature, uint64_t epsilon_bits, int dtype)
{
    float eps = 1e-9f;
    if (epsilon_bits != 0) {
        eps = u2f((uint32_t)epsilon_bits);
        if (!(isfinite(eps) && eps > 0.0f)) return -1;
    }
    for (uint32_t bi = 0; bi < batch; ++bi) {
        const size_t row = (size_t)bi * feature;
        float sumsq = 0.0f;
        for (uint32_t j = 0; j < feature; ++j) {
            const float v = rd(x, row + j, dtype) + (res ? rd(res, row + j, dtype) : 0.0f);
            sumsq += v * v;
        }
        const float inv = 1.0f / sqrtf(sumsq / (float)feature + eps);
        for (uint32_t j = 0; j < feature; ++j) {
            const float v = rd(x, row + j, dtype) + (res ? rd(res, row + j, dtype) : 0.0f);
            float o;
            if (dtype == OR_DTYPE_F32 && res)
                o = gamma ? v * (inv * rd(gamma, j, dtype)) : v * inv;
            else
                o = v * inv * (gamma ? rd(gamma, j, dtype) : 1.0f);
            wr(out, row + j, o, dtype);
        }
    }
    return 0;
}

/* rope_float scalar path, src/cpu/float_kernels.rs:3171-3184 */
int or_rope(const void *x, const void *cs, const void *sn, void *out, uint32_t head_dim, size_t n,
            int dtype)
{
    if (head_dim == 0 || head_dim % 2 != 0 || n % head_dim != 0) return -1;
    const size_t half = head_dim / 2;
    for (size_t e = 0; e < n; ++e) {
        const size_t pos = e % head_dim, base = e - pos;
        const float xe = rd(x, e, dtype), ce = rd(cs, e, dtype), se = rd(sn, e, dtype);
        const float v = pos < half ? xe * ce - rd(x, base + pos + half, dtype) * se
                                   : xe * ce + rd(x, base + pos - half, dtype) * se;
        wr(out, e, v, dtype);
    }
    return 0;
}

/* gather, src/cpu/kernels.rs:389-447 (rows of row_bytes). 0 ok, -1 an index
 * is out of range (the reference's SlotOutOfRange(indices)). */
int or_gather(const uint8_t *data, const void *idx, uint8_t *out, uint64_t outer,
              uint64_t axis_dim, uint64_t row_bytes, uint64_t num_idx, int idx_i64)
{
    for (uint64_t o = 0; o < outer; ++o)
        for (uint64_t k = 0; k < num_idx; ++k) {
            int64_t i = idx_i64 ? ((const int64_t *)idx)[k] : (int64_t)((const int32_t *)idx)[k];
            if (i < 0) i += (int64_t)axis_dim;
            if (i < 0 || (uint64_t)i >= axis_dim) return -1;
            memcpy(out + (o * num_idx + k) * row_bytes, data + (o * axis_dim + (uint64_t)i) * row_bytes,
                   row_bytes);
        }
    return 0;
}

/* argmax (new op 124): the lowest index of the largest value per row; NaN is
 * never larger; a row with no comparable value gives 0. */
void or_argmax(const void *in, int32_t *out, uint32_t rows, uint32_t cols, int dtype)
{
    for (uint32_t r = 0; r < rows; ++r) {
        int best_i = -1;
        float best = 0.0f;
        for (uint32_t j = 0; j < cols; ++j) {
            const float v = rd(in, (size_t)r * cols + j, dtype);
            if (v != v) continue;
            if (best_i < 0 || v > best) {
                best = v;
                best_i = (int)j;
            }
        }
        out[r] = best_i < 0 ? 0 : best_i;
    }
}
