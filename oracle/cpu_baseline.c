/*
 * cpu_baseline.c — multi-threaded CPU timing engines (TEST INFRASTRUCTURE).
 *
 * bench.py's cpu_baseline leg times these on the GPU box's host cores, beside
 * the HIP kernels. They restate the reference CPU backend's engines, not just
 * its arithmetic, so the baseline is a fair stand-in for the Rust binary that
 * cannot be built here:
 *   LUT      scalar u16 gather (src/cpu/lut.rs:93-96), rows split over threads
 *   MatMul   4x16 AVX2/FMA register tile (src/cpu/simd.rs:709-800) under the
 *            cache-oblivious bisection with a 64^3 leaf (:994-1061); output
 *            row tiles across threads (src/cpu/parallel.rs output_tiles);
 *            bf16 widens A and B to f32 and narrows by truncation
 *            (src/cpu/float_kernels.rs:368-392)
 *   KV       honest copy + quantize_row_i8 per new row (kernels.rs:455-501,
 *            simd.rs:4761-4785)
 *   Attn     dequantize the realized rows, then the two-pass row of
 *            float_kernels.rs:3834-3883 with AVX2 dot/axpy, (b, kv-head)
 *            tasks across threads
 * Built with -O3 -mavx2 -mfma -pthread (oracle/Makefile).
 */
#include "holo_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

typedef void (*cb_task_fn)(void *ctx, size_t lo, size_t hi);
typedef struct { cb_task_fn fn; void *ctx; size_t lo, hi; } cb_range;

static void *cb_thread(void *p)
{
    cb_range *r = (cb_range *)p;
    r->fn(r->ctx, r->lo, r->hi);
    return NULL;
}

/* Split [0, n) into `threads` contiguous ranges and run them concurrently. */
static void cb_parallel(cb_task_fn fn, void *ctx, size_t n, int threads)
{
    if (threads < 1) threads = 1;
    if ((size_t)threads > n) threads = (int)(n ? n : 1);
    pthread_t tid[256];
    cb_range rg[256];
    if (threads > 256) threads = 256;
    for (int t = 0; t < threads; ++t) {
        rg[t].fn = fn;
        rg[t].ctx = ctx;
        rg[t].lo = n * (size_t)t / (size_t)threads;
        rg[t].hi = n * (size_t)(t + 1) / (size_t)threads;
    }
    for (int t = 1; t < threads; ++t) pthread_create(&tid[t], NULL, cb_thread, &rg[t]);
    cb_thread(&rg[0]);
    for (int t = 1; t < threads; ++t) pthread_join(tid[t], NULL);
}

/* ---------------------------------------------------------------- LUT --- */
typedef struct { const uint16_t *t, *in; uint16_t *out; } lut_ctx;
static void lut_task(void *c, size_t lo, size_t hi)
{
    lut_ctx *x = (lut_ctx *)c;
    for (size_t i = lo; i < hi; ++i) x->out[i] = x->t[x->in[i]];
}
void cb_lut(const uint16_t *table, const uint16_t *in, uint16_t *out, size_t n, int threads)
{
    lut_ctx c = {table, in, out};
    cb_parallel(lut_task, &c, n, threads);
}

/* ------------------------------------------------------------- MatMul --- */
static void fma_strided(const float *a, const float *b, float *out, size_t m, size_t k,
                        size_t n, size_t lda, size_t ldb, size_t ldc, int acc)
{
    enum { MR = 4, NR = 16 };
    size_t i = 0;
    for (; i + MR <= m; i += MR) {
        size_t j = 0;
        for (; j + NR <= n; j += NR) {
            __m256 c[MR][2];
            for (int r = 0; r < MR; ++r) {
                float *o = out + (i + r) * ldc + j;
                c[r][0] = acc ? _mm256_loadu_ps(o) : _mm256_setzero_ps();
                c[r][1] = acc ? _mm256_loadu_ps(o + 8) : _mm256_setzero_ps();
            }
            for (size_t kk = 0; kk < k; ++kk) {
                const float *br = b + kk * ldb + j;
                __m256 b0 = _mm256_loadu_ps(br), b1 = _mm256_loadu_ps(br + 8);
                for (int r = 0; r < MR; ++r) {
                    __m256 av = _mm256_set1_ps(a[(i + r) * lda + kk]);
                    c[r][0] = _mm256_fmadd_ps(av, b0, c[r][0]);
                    c[r][1] = _mm256_fmadd_ps(av, b1, c[r][1]);
                }
            }
            for (int r = 0; r < MR; ++r) {
                float *o = out + (i + r) * ldc + j;
                _mm256_storeu_ps(o, c[r][0]);
                _mm256_storeu_ps(o + 8, c[r][1]);
            }
        }
        for (; j + 8 <= n; j += 8) {
            __m256 c[MR];
            for (int r = 0; r < MR; ++r)
                c[r] = acc ? _mm256_loadu_ps(out + (i + r) * ldc + j) : _mm256_setzero_ps();
            for (size_t kk = 0; kk < k; ++kk) {
                __m256 bv = _mm256_loadu_ps(b + kk * ldb + j);
                for (int r = 0; r < MR; ++r)
                    c[r] = _mm256_fmadd_ps(_mm256_set1_ps(a[(i + r) * lda + kk]), bv, c[r]);
            }
            for (int r = 0; r < MR; ++r) _mm256_storeu_ps(out + (i + r) * ldc + j, c[r]);
        }
        for (; j < n; ++j) {
            for (int r = 0; r < MR; ++r) {
                float s = acc ? out[(i + r) * ldc + j] : 0.0f;
                for (size_t kk = 0; kk < k; ++kk) s += a[(i + r) * lda + kk] * b[kk * ldb + j];
                out[(i + r) * ldc + j] = s;
            }
        }
    }
    for (; i < m; ++i) {           /* row remainder: same column tiers */
        size_t j = 0;
        for (; j + 8 <= n; j += 8) {
            __m256 c = acc ? _mm256_loadu_ps(out + i * ldc + j) : _mm256_setzero_ps();
            for (size_t kk = 0; kk < k; ++kk)
                c = _mm256_fmadd_ps(_mm256_set1_ps(a[i * lda + kk]), _mm256_loadu_ps(b + kk * ldb + j), c);
            _mm256_storeu_ps(out + i * ldc + j, c);
        }
        for (; j < n; ++j) {
            float s = acc ? out[i * ldc + j] : 0.0f;
            for (size_t kk = 0; kk < k; ++kk) s += a[i * lda + kk] * b[kk * ldb + j];
            out[i * ldc + j] = s;
        }
    }
}

static void mm_recursive(const float *a, const float *b, float *out, size_t m, size_t k,
                         size_t n, size_t lda, size_t ldb, size_t ldc, int acc)
{
    const size_t LEAF = 64;
    if (m <= LEAF && k <= LEAF && n <= LEAF) {
        fma_strided(a, b, out, m, k, n, lda, ldb, ldc, acc);
        return;
    }
    if (m >= n && m >= k) {
        size_t h = m / 2;
        mm_recursive(a, b, out, h, k, n, lda, ldb, ldc, acc);
        mm_recursive(a + h * lda, b, out + h * ldc, m - h, k, n, lda, ldb, ldc, acc);
    } else if (n >= m && n >= k) {
        size_t h = n / 2;
        mm_recursive(a, b, out, m, k, h, lda, ldb, ldc, acc);
        mm_recursive(a, b + h, out + h, m, k, n - h, lda, ldb, ldc, acc);
    } else {
        size_t h = k / 2;
        mm_recursive(a, b, out, m, h, n, lda, ldb, ldc, acc);
        mm_recursive(a + h, b + h * ldb, out, m, k - h, n, lda, ldb, ldc, 1);
    }
}

typedef struct { const float *a, *b; float *out; size_t m, k, n, rows_per; } mm_ctx;
static void mm_task(void *c, size_t lo, size_t hi)
{
    mm_ctx *x = (mm_ctx *)c;
    for (size_t t = lo; t < hi; ++t) {
        size_t r0 = t * x->rows_per, r1 = r0 + x->rows_per;
        if (r1 > x->m) r1 = x->m;
        if (r0 < r1)
            mm_recursive(x->a + r0 * x->k, x->b, x->out + r0 * x->n, r1 - r0, x->k, x->n,
                         x->k, x->n, x->n, 0);
    }
}
void cb_matmul_f32(const float *a, const float *b, float *out, size_t m, size_t k, size_t n,
                   int threads)
{
    size_t tiles = (size_t)(threads > 0 ? threads : 1) * 4;
    size_t rows_per = (m + tiles - 1) / tiles;
    if (rows_per < 4) rows_per = 4;
    rows_per = (rows_per + 3) / 4 * 4;
    mm_ctx c = {a, b, out, m, k, n, rows_per};
    cb_parallel(mm_task, &c, (m + rows_per - 1) / rows_per, threads);
}

typedef struct { const uint16_t *src; float *dst; } widen_ctx;
static void widen_task(void *c, size_t lo, size_t hi)
{
    widen_ctx *x = (widen_ctx *)c;
    for (size_t i = lo; i < hi; ++i) {
        uint32_t u = (uint32_t)x->src[i] << 16;
        memcpy(&x->dst[i], &u, 4);
    }
}
typedef struct { const float *src; uint16_t *dst; } narrow_ctx;
static void narrow_task(void *c, size_t lo, size_t hi)
{
    narrow_ctx *x = (narrow_ctx *)c;
    for (size_t i = lo; i < hi; ++i) {
        uint32_t u;
        memcpy(&u, &x->src[i], 4);
        x->dst[i] = (uint16_t)(u >> 16);
    }
}
/* bf16 path: widen A and B, f32 engine, truncate (float_kernels.rs:368-392). */
void cb_matmul_bf16(const uint16_t *a, const uint16_t *b, uint16_t *out, size_t m, size_t k,
                    size_t n, int threads)
{
    float *a32 = (float *)malloc(sizeof(float) * m * k);
    float *b32 = (float *)malloc(sizeof(float) * k * n);
    float *o32 = (float *)malloc(sizeof(float) * m * n);
    widen_ctx wa = {a, a32}, wb = {b, b32};
    cb_parallel(widen_task, &wa, m * k, threads);
    cb_parallel(widen_task, &wb, k * n, threads);
    cb_matmul_f32(a32, b32, o32, m, k, n, threads);
    narrow_ctx nc = {o32, out};
    cb_parallel(narrow_task, &nc, m * n, threads);
    free(a32);
    free(b32);
    free(o32);
}

/* Few-row bf16 path (m <= 8, float_kernels.rs:369-379; matmul_lowp_gemv,
 * simd.rs:3808-3858): B is streamed once and widened in registers, never
 * materialized; a is widened up front; output truncated. Threads take
 * 64-column blocks of B. */
typedef struct { const float *a; const uint16_t *b; float *out; size_t m, k, n; } gemv_ctx;
static void gemv_task(void *c, size_t lo, size_t hi)
{
    gemv_ctx *x = (gemv_ctx *)c;
    for (size_t blk = lo; blk < hi; ++blk) {
        size_t c0 = blk * 64, c1 = c0 + 64 < x->n ? c0 + 64 : x->n;
        for (size_t j = c0; j < c1; j += 8) {
            if (j + 8 <= c1) {
                __m256 acc[8];
                for (size_t r = 0; r < x->m; ++r) acc[r] = _mm256_setzero_ps();
                for (size_t kk = 0; kk < x->k; ++kk) {
                    __m128i h = _mm_loadu_si128((const __m128i *)(x->b + kk * x->n + j));
                    __m256 bv = _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(h), 16));
                    for (size_t r = 0; r < x->m; ++r)
                        acc[r] = _mm256_fmadd_ps(_mm256_set1_ps(x->a[r * x->k + kk]), bv, acc[r]);
                }
                for (size_t r = 0; r < x->m; ++r) _mm256_storeu_ps(x->out + r * x->n + j, acc[r]);
            } else {
                for (size_t jj = j; jj < c1; ++jj)
                    for (size_t r = 0; r < x->m; ++r) {
                        float s = 0.0f;
                        for (size_t kk = 0; kk < x->k; ++kk) {
                            uint32_t u = (uint32_t)x->b[kk * x->n + jj] << 16;
                            float bf;
                            memcpy(&bf, &u, 4);
                            s += x->a[r * x->k + kk] * bf;
                        }
                        x->out[r * x->n + jj] = s;
                    }
            }
        }
    }
}
void cb_matmul_bf16_gemv(const uint16_t *a, const uint16_t *b, uint16_t *out, size_t m, size_t k,
                         size_t n, int threads)
{
    float *a32 = (float *)malloc(sizeof(float) * m * k);
    float *o32 = (float *)malloc(sizeof(float) * m * n);
    for (size_t i = 0; i < m * k; ++i) {
        uint32_t u = (uint32_t)a[i] << 16;
        memcpy(&a32[i], &u, 4);
    }
    gemv_ctx c = {a32, b, o32, m, k, n};
    cb_parallel(gemv_task, &c, (n + 63) / 64, threads);
    for (size_t i = 0; i < m * n; ++i) {
        uint32_t u;
        memcpy(&u, &o32[i], 4);
        out[i] = (uint16_t)(u >> 16);
    }
    free(a32);
    free(o32);
}

/* ----------------------------------------------------------------- KV --- */
typedef struct { const uint8_t *src; uint8_t *dst; size_t chunk, total; } copy_ctx;
static void copy_task(void *c, size_t lo, size_t hi)
{
    copy_ctx *x = (copy_ctx *)c;
    for (size_t t = lo; t < hi; ++t) {
        size_t b0 = t * x->chunk, b1 = b0 + x->chunk;
        if (b1 > x->total) b1 = x->total;
        memcpy(x->dst + b0, x->src + b0, b1 - b0);
    }
}
static void par_copy(const void *src, void *dst, size_t bytes, int threads)
{
    copy_ctx c = {(const uint8_t *)src, (uint8_t *)dst, 1u << 20, bytes};
    cb_parallel(copy_task, &c, (bytes + c.chunk - 1) / c.chunk, threads);
}
/* Honest-copy quantize+append of one cache (data + scales). */
int cb_kv_quant_append_copy(const void *nw, int dtype, uint32_t pos, const int8_t *cq,
                            const float *cs, int8_t *oq, float *os, uint32_t planes,
                            uint32_t bucket, uint32_t new_rows, uint32_t d, int threads)
{
    par_copy(cq, oq, (size_t)planes * bucket * d, threads);
    par_copy(cs, os, (size_t)planes * bucket * sizeof(float), threads);
    return or_kv_quant_append(nw, dtype, pos, oq, os, planes, bucket, new_rows, d);
}

/* --------------------------------------------------------------- Attn --- */
static float dot_avx2(const float *a, const float *b, size_t n)
{
    __m256 acc = _mm256_setzero_ps();
    size_t i = 0;
    for (; i + 8 <= n; i += 8) acc = _mm256_fmadd_ps(_mm256_loadu_ps(a + i), _mm256_loadu_ps(b + i), acc);
    float t[8];
    _mm256_storeu_ps(t, acc);
    float s = ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
    for (; i < n; ++i) s += a[i] * b[i];
    return s;
}
static void axpy_avx2(float *o, float s, const float *b, size_t n)
{
    __m256 sv = _mm256_set1_ps(s);
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        _mm256_storeu_ps(o + i, _mm256_fmadd_ps(sv, _mm256_loadu_ps(b + i), _mm256_loadu_ps(o + i)));
    for (; i < n; ++i) o[i] += s * b[i];
}

typedef struct {
    const float *q;
    const int8_t *kq, *vq;
    const float *ks, *vs;
    const uint32_t *lens;
    float *out;
    uint32_t B, H, Hkv, bucket, D;
    float scale;
} attn_ctx;

static void attn_task(void *c, size_t lo, size_t hi)
{
    attn_ctx *x = (attn_ctx *)c;
    size_t D = x->D, group = x->H / x->Hkv;
    float *kd = (float *)malloc(sizeof(float) * (size_t)x->bucket * D);
    float *vd = (float *)malloc(sizeof(float) * (size_t)x->bucket * D);
    float *sc = (float *)malloc(sizeof(float) * ((size_t)x->bucket + 1));
    for (size_t t = lo; t < hi; ++t) {
        size_t b = t / x->Hkv, kh = t % x->Hkv;
        size_t L = x->lens[b] < x->bucket ? x->lens[b] : x->bucket;
        size_t plane = b * x->Hkv + kh;
        or_dequant_i8(x->kq + plane * (size_t)x->bucket * D, x->ks + plane * (size_t)x->bucket, kd, L, D);
        or_dequant_i8(x->vq + plane * (size_t)x->bucket * D, x->vs + plane * (size_t)x->bucket, vd, L, D);
        for (size_t g = 0; g < group; ++g) {
            size_t hh = kh * group + g;
            const float *qr = x->q + (b * x->H + hh) * D;
            float *o = x->out + (b * x->H + hh) * D;
            memset(o, 0, sizeof(float) * D);
            if (L == 0) continue;
            for (size_t j = 0; j < L; ++j) sc[j] = dot_avx2(qr, kd + j * D, D) / x->scale;
            float mx = -INFINITY;
            for (size_t j = 0; j < L; ++j) mx = fmaxf(mx, sc[j]);
            float sum = 0.0f;
            for (size_t j = 0; j < L; ++j) {
                sc[j] = or_exp_f32_det(sc[j] - mx);
                sum += sc[j];
            }
            float denom = sum > 1e-30f ? sum : 1e-30f;
            for (size_t j = 0; j < L; ++j) axpy_avx2(o, sc[j] / denom, vd + j * D, D);
        }
    }
    free(kd);
    free(vd);
    free(sc);
}
void cb_decode_attention_i8(const float *q, const int8_t *kq, const float *ks, const int8_t *vq,
                            const float *vs, const uint32_t *lens, float *out, uint32_t B,
                            uint32_t H, uint32_t Hkv, uint32_t bucket, uint32_t D, float scale,
                            int threads)
{
    attn_ctx c = {q, kq, vq, ks, vs, lens, out, B, H, Hkv, bucket, D, scale};
    cb_parallel(attn_task, &c, (size_t)B * Hkv, threads);
}
