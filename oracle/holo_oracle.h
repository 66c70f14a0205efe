/*
 * holo_oracle.h — CPU restatement of the Hologram reference's hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker that the HIP backend
 * (hologram_amd/) is compared against, and the CPU baseline bench.py times
 * beside it. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it. The product never links, loads or calls anything here.
 *
 * Every function restates one reference function (Rust, crates/hologram-compute)
 * in plain C with the same IEEE-754 binary32 operation order, built with
 * -ffp-contract=off -fno-fast-math on x86-64 SSE2 (no x87, no FMA), which is
 * the target the reference's LUT tables are defined against.
 *
 * Parity pins (what checks each function; see tests/test_oracle_pins.py):
 *   bf16/f16 codecs ............ closed form (exhaustive round trips, RNE rules)
 *   or_exp_f32_det ............. closed form (|rel err| <= 2e-6 vs long double)
 *   or_gelu/silu/sigmoid/tanh .. reference test tolerances (tests/lut.rs:67-132)
 *                                 and f64 closed forms within 1 bf16 ulp
 *   or_libm_expf ............... correctly-rounded exp (<= 1 ulp everywhere,
 *                                 bit-equal on all non-fragile bf16 entries)
 *   or_quantize_row_i8 ......... reference golden FNV 0x787ccdc172029f9b
 *                                 (simd.rs:8236-8259) through or_matmul_i8_pc_omajor
 *   or_kv_cache_write .......... closed form (ring placement, brute force)
 *   or_decode_attention_* ...... f64 softmax closed form, zero-visible row = 0
 *   or_matmul_ref_f64 .......... closed form (identity / permutation products)
 *   or_binary .................. closed form (f32 add/mul then truncation,
 *                                 numpy float32 arithmetic on the same inputs)
 *   or_rms_norm ................ f64 closed form within 2 bf16 ulp; unit rows
 *   or_rope .................... f64 rotation of each pair (cos/sin of an angle
 *                                 preserve the pair's norm); angle 0 = identity
 *   or_gather .................. brute-force row indexing, negative wrap
 *   or_argmax .................. numpy argmax (NaN-free rows), first-index ties
 *   or_libm_erff ............... correctly-rounded erf (<= 1 ulp on every finite
 *                                 bf16 input and 450,000 sampled f32), odd
 *                                 symmetry, special values
 *   or_matmul_q_omajor ......... reference goldens for the i8, i4 and e8cb tiers
 *                                 (simd.rs:8236-8283)
 *   or_dequantize .............. reference known answers (conformance.rs:936-1009),
 *                                 exact (q - zp) * scale, nibble order, i32 wrap
 *   or_dequant_activation ...... the unfused pair (or_dequantize then the
 *                                 activation) bit for bit; f64 GELU tracking
 *   or_add_rms_norm ............ RmsNorm bit for bit without a residual; the
 *                                 unnarrowed f32 sum; f64 closed form (f32)
 *   or_decode_attention_valid .. f64 softmax law over the causal visible set
 *   or_decode_attention (mask) . bit-equal to or_decode_attention_valid when the
 *                                 mask states the same visibility (0 / -inf over
 *                                 finite K/V: decode_attention_valid.rs:1-13);
 *                                 f64 softmax law with the mask added; a fully
 *                                 masked row is exactly zero
 *   pack_b_panels (Python) ..... the layout formula (layout.rs:16-45)
 *
 * Parity unpinned: the 126 signaling-NaN inputs of the bf16/f16 SiLU tables
 * and NaN payloads of the Exp table (IEEE quieting assumed); Erf table entries
 * are pinned to within one ulp of the correctly rounded erf, not bit for bit
 * against libm 0.2.16 (not vendored in the reference).
 */
#ifndef HOLO_ORACLE_H
#define HOLO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype tags: crates/hologram-types/src/dtype_id.rs:52-61 */
enum { OR_DTYPE_I8 = 2, OR_DTYPE_F16 = 6, OR_DTYPE_BF16 = 7, OR_DTYPE_F32 = 8 };
/* lut_act ids: crates/hologram-compute/src/kernel_call.rs:877-885 */
enum { OR_ACT_SIGMOID = 0, OR_ACT_TANH = 1, OR_ACT_GELU = 2, OR_ACT_SILU = 3, OR_ACT_EXP = 4,
       OR_ACT_ERF = 5 };

/* ---- codecs: src/cpu/dtype.rs:69-153 ---- */
float    or_bf16_to_f32(uint16_t b);
uint16_t or_f32_to_bf16(float v);          /* truncation, NaN payload kept */
float    or_f16_to_f32(uint16_t b);
uint16_t or_f32_to_f16(float v);           /* the reference's own rounding */

/* ---- transcendental restatements ---- */
float or_exp_f32_det(float x);             /* src/cpu/simd.rs:4217-4239 */
float or_libm_expf(float x);               /* libm 0.2.16 expf (FreeBSD e_expf.c) */
float or_sigmoid_f(float x);               /* src/cpu/float_kernels.rs:3549-3551 */
float or_tanh_f(float x);                  /* :3553-3558 */
float or_gelu_f(float x);                  /* :3560-3562 */
float or_silu_f(float x);                  /* :3564-3566 */
int or_fused_act_f32(int act, const float *in, float *out, size_t n); /* fused_act_fn :768-780 */
float or_libm_erff(float x);               /* libm 0.2.16 erff (musl erff.c, FreeBSD s_erff.c) */
float or_lut_act_ref(int act, float x);    /* :3628-3638 */

/* ---- LUT: src/cpu/lut.rs:43-67 (build) and :76-98 (gather) ---- */
int  or_build_table(int act, int dtype, uint16_t *table /* [65536] */);
void or_unary_lut(const uint16_t *table, const uint16_t *in, uint16_t *out, size_t n);

/* ---- int8 scheme: src/cpu/simd.rs:4755-4785 ---- */
float or_quantize_row_i8(const float *a, int8_t *q, size_t k);
/* W8A8 output-major GEMV, simd.rs:5295-5480 (golden carrier, simd.rs:8236-8259) */
/* Output-major W8A8 GEMV for the i8 (2), i4 (10) and e8cb (11) tiers
 * (simd.rs:5295-5480, :6172-6230, :6867-6950): per-token symmetric activation
 * quantization, exact i32 dot, out = (acc as f32) * (scale_a * scales[j]).
 * codebook: 256 x 8 i8 (e8cb only). Returns 3 for an unknown tier, a k the
 * tier cannot split, or k above the exact-i32 bound. */
#define OR_DTYPE_I4 10
#define OR_DTYPE_E8CB 11
#define OR_DTYPE_U8 1
/* dequantize (src/cpu/kernels.rs:185-296): out[i] = ((q[i] - zp) as f32 * s)
 * as dtype, per-channel (scales/zps [channels], channel (i / inner) %
 * channels) when scales is non-null and channels > 0. 0, or 1 for an
 * unknown quant/output dtype. */
int or_dequantize(const uint8_t *in, uint64_t n, int quant, const float *scales,
                  const int32_t *zps, uint32_t channels, uint32_t inner, float scale,
                  int32_t zp, int dtype, void *out);
/* dequant_activation (kernels.rs:311-388): f32 out[i] = f((q - zp) as f32 *
 * scale), f = lut_act_ref(act) (0-4, and erff for 5 and any other id). */
int or_dequant_activation(const uint8_t *in, uint64_t n, int quant, int act, float scale,
                          int32_t zp, float *out);
#define OR_I8_DOT_K_MAX 133144   /* i32::MAX / (127 * 127), kernel_call.rs:103 */
int or_matmul_q_omajor(int tier, const float *a, const uint8_t *bq, const int8_t *codebook,
                       const float *scales, float *out, size_t m, size_t k, size_t n);
void or_matmul_i8_pc_omajor(const float *a, const int8_t *bq, const float *scales,
                            float *out, size_t m, size_t k, size_t n);
uint64_t or_fnv1a_f32(const float *v, size_t n);

/* ---- KV write: src/cpu/kernels.rs:455-501 (honest copy) ---- */
int or_kv_cache_write(const uint8_t *cache, const uint8_t *newrows, uint32_t pos,
                      uint8_t *out, uint32_t planes, uint32_t bucket_rows,
                      uint32_t new_rows, uint32_t row_bytes);
/* int8 quantize+append (new op): widen each new row (dtype of `newrows`),
 * quantize it with or_quantize_row_i8, place the int8 row and its f32 scale at
 * ring row (pos + j) % bucket of the int8 cache and the scale cache. Writes in
 * place into cache_q / cache_s (the caller copies first for the copy form). */
int or_kv_quant_append(const void *newrows, int dtype, uint32_t pos,
                       int8_t *cache_q, float *cache_s, uint32_t planes,
                       uint32_t bucket_rows, uint32_t new_rows, uint32_t head_dim);
/* dequantize: src/cpu/kernels.rs:246-271, symmetric zp = 0 */
void or_dequant_i8(const int8_t *q, const float *scales, float *out,
                   size_t rows, size_t row_len);

/* ---- decode attention: src/cpu/float_kernels.rs:3834-3957, 4192-4307 ---- */
float or_attn_scale(uint32_t head_dim, uint32_t scale_bits);
void or_decode_attention_valid_f32(const float *q, const float *k_past, const float *v_past,
                                   const float *k_new, const float *v_new, float *out,
                                   uint32_t b, uint32_t h, uint32_t hkv, uint32_t m,
                                   uint32_t past, uint32_t nnew, uint32_t d, float scale,
                                   uint32_t vis_past);
/* DecodeAttentionValid over any of bf16/f16/f32 (:4192-4307): the declared
 * buffers widened whole, the f32 engine, the output narrowed. valid_len is
 * the u32 operand's value. Returns 0, or 3 (UnsupportedOp) for q_rows !=
 * new_len, q_rows == 0, heads % kv_heads != 0 or another dtype. */
int or_decode_attention_valid(const void *q, const void *k_past, const void *v_past,
                              const void *k_new, const void *v_new, uint32_t valid_len, void *out,
                              uint32_t b, uint32_t h, uint32_t hkv, uint32_t m, uint32_t past,
                              uint32_t nnew, uint32_t d, uint32_t scale_bits, int dtype);
/* DecodeAttention, the mask form (:2420-2477 row, :2482-2660 call): every
 * past row then every new row is a key, query row qi adds mask[qi][j]
 * (f32 [m][past + nnew]) to the score of key j, a row with no finite score
 * maximum (all -inf) is zero. or_decode_attention returns 0, or 3
 * (UnsupportedOp) for past + nnew == 0, heads % kv_heads != 0 or another
 * dtype. */
void or_decode_attention_mask_f32(const float *q, const float *k_past, const float *v_past,
                                  const float *k_new, const float *v_new, const float *mask,
                                  float *out, uint32_t b, uint32_t h, uint32_t hkv, uint32_t m,
                                  uint32_t past, uint32_t nnew, uint32_t d, float scale);
int or_decode_attention(const void *q, const void *k_past, const void *v_past, const void *k_new,
                        const void *v_new, const float *mask, void *out, uint32_t b, uint32_t h,
                        uint32_t hkv, uint32_t m, uint32_t past, uint32_t nnew, uint32_t d,
                        uint32_t scale_bits, int dtype);
/* int8-cache decode attention (new op), stated as the reference's per-sequence
 * DecodeAttentionValid{b=1, past=L-1, valid=L-1, q=new=1} over the dequantized
 * rows.  q: [B,H,D] f32 (widened), caches [B,Hkv,bucket,D] int8 + [B,Hkv,bucket]
 * f32 scales, lens[B] (clamped to bucket), out [B,H,D] f32. */
void or_decode_attention_i8(const float *q, const int8_t *kq, const float *ks,
                            const int8_t *vq, const float *vs, const uint32_t *lens,
                            float *out, uint32_t B, uint32_t H, uint32_t Hkv,
                            uint32_t bucket, uint32_t D, float scale);

/* ---- decode-step ops (bf16 or f32 operands) ---- */
/* binary_float, src/cpu/float_kernels.rs:238-300: op 0 = Add, 1 = Mul */
void or_binary(int op, const void *a, const void *b, void *out, size_t n, int dtype);
/* rms_norm_float generic path, float_kernels.rs:1683-1755 (gamma NULL: none) */
int or_rms_norm(const void *x, const void *gamma, void *out, uint32_t batch, uint32_t feature,
                uint64_t epsilon_bits, int dtype);
int or_add_rms_norm(const void *x, const void *res, const void *gamma, void *out, uint32_t batch,
                    uint32_t feature, uint64_t epsilon_bits, int dtype);
/* rope_float scalar path, float_kernels.rs:3123-3186 */
int or_rope(const void *x, const void *cs, const void *sn, void *out, uint32_t head_dim, size_t n,
            int dtype);
/* gather, src/cpu/kernels.rs:389-447; -1 = index out of range */
int or_gather(const uint8_t *data, const void *idx, uint8_t *out, uint64_t outer,
              uint64_t axis_dim, uint64_t row_bytes, uint64_t num_idx, int idx_i64);
/* argmax (new op 124) */
void or_argmax(const void *in, int32_t *out, uint32_t rows, uint32_t cols, int dtype);

/* ---- MatMul references: tests/conformance.rs:100-144 ---- */
void or_matmul_ref_f64(const float *a, const float *b, float *out,
                       size_t m, size_t k, size_t n);
double or_max_rel_err(const float *got, const float *want, size_t n);

#ifdef __cplusplus
}
#endif
#endif
