/*
 * holo_hip.h — C ABI of the MI355X (gfx950) compute backend for Hologram.
 *
 * The reference's operator API is the Rust trait
 *     Backend::dispatch(&mut self, &KernelCall, &mut Workspace) -> Result<(), BackendError>
 * (crates/hologram-compute/src/backend.rs:8-15). This header is that boundary as
 * a C ABI: a Rust `Backend` impl binds these functions one to one, falling
 * back to the CPU backend for UnsupportedOp. Buffers are device-resident: the caller's content-addressed
 * pool (crates/hologram-exec/src/buffer.rs:149-207) binds each slot to a device
 * allocation it owns, and kernels read/write the slots in place — no per-call
 * host round trip.
 *
 * All entry points return a holo_status; on failure a human-readable message is
 * available from holo_hip_last_error_message() on the same thread
 * (the convention of crates/hologram-ffi/src/lib.rs:47-48).
 */
#ifndef HOLO_HIP_H
#define HOLO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* BackendError, crates/hologram-compute/src/error.rs:6-20 (0 = Ok). */
typedef enum holo_status {
    HOLO_OK = 0,
    HOLO_ERR_SLOT_OUT_OF_RANGE = 1, /* BackendError::SlotOutOfRange(slot) */
    HOLO_ERR_SHAPE_MISMATCH = 2,    /* BackendError::ShapeMismatch        */
    HOLO_ERR_UNSUPPORTED_OP = 3,    /* BackendError::UnsupportedOp(..)    */
    HOLO_ERR_INIT = 4,              /* BackendError::Init(..)             */
    HOLO_ERR_DISPATCH = 5           /* BackendError::Dispatch(..)         */
} holo_status;

/* dtype tags, crates/hologram-types/src/dtype_id.rs:52-61 */
#define HOLO_DTYPE_I8 2u
#define HOLO_DTYPE_F16 6u
#define HOLO_DTYPE_BF16 7u
#define HOLO_DTYPE_F32 8u

#define HOLO_DTYPE_I32 4u
#define HOLO_DTYPE_I64 5u
#define HOLO_DTYPE_F64 9u     /* storage only: no op computes in it (kernels.rs:1611-1615) */
#define HOLO_DTYPE_U8 1u
#define HOLO_DTYPE_I4 10u     /* packed signed 4-bit, two per byte, low nibble first */
#define HOLO_DTYPE_E8CB 11u   /* one u8 codebook index per 8-element group */

/* lut_act ids, crates/hologram-compute/src/kernel_call.rs:877-885 */
#define HOLO_ACT_SIGMOID 0
#define HOLO_ACT_TANH 1
#define HOLO_ACT_GELU 2
#define HOLO_ACT_SILU 3
#define HOLO_ACT_EXP 4
#define HOLO_ACT_ERF 5

/* fused_activation ids of the fused MatMul epilogues,
 * crates/hologram-compute/src/kernel_call.rs:861-870 */
#define HOLO_FUSED_RELU 1
#define HOLO_FUSED_GELU 2
#define HOLO_FUSED_SILU 3
#define HOLO_FUSED_SIGMOID 4
#define HOLO_FUSED_TANH 5
#define HOLO_FUSED_ELU 6
#define HOLO_FUSED_SELU 7
#define HOLO_FUSED_EXP 8

/* KernelCall tags = the archive wire discriminants,
 * crates/hologram-archive/src/kernel_codec.rs:18-128. 122 and 123 are new
 * capabilities and take new discriminants (kernel_codec.rs:124-128). */
#define HOLO_OP_ADD 5u
#define HOLO_OP_MUL 7u
#define HOLO_OP_RELU 11u
#define HOLO_OP_SIGMOID 12u
#define HOLO_OP_TANH 13u
#define HOLO_OP_GELU 14u
#define HOLO_OP_SILU 15u
#define HOLO_OP_ELU 16u
#define HOLO_OP_SELU 17u
#define HOLO_OP_EXP 18u
#define HOLO_OP_ERF 32u                   /* Erf: libm erff (bf16/f16 table, f32 computed) */
#define HOLO_OP_DEQUANTIZE 105u           /* Dequantize (wire 105; 118 carries the extended fields) */
#define HOLO_OP_MATMUL_DEQUANT 111u       /* MatMulDequant (wire 111; 116 / 117 the extended forms) */
#define HOLO_OP_DEQUANT_ACT 113u          /* DequantActivation */
#define HOLO_OP_MATMUL 46u
#define HOLO_OP_MATMUL_ACT 106u           /* MatMulActivation (kernel_codec.rs:102)    */
#define HOLO_OP_MATMUL_ADD 107u           /* MatMulAdd (kernel_codec.rs:103)           */
#define HOLO_OP_MATMUL_ADD_ACT 108u       /* MatMulAddActivation (kernel_codec.rs:104) */
#define HOLO_OP_RMS_NORM 51u
#define HOLO_OP_ADD_RMS_NORM 54u          /* AddRmsNorm: rms_norm(x + residual) */
#define HOLO_OP_ROTARY 75u
#define HOLO_OP_GATHER 114u
#define HOLO_OP_DECODE_ATTN 119u          /* DecodeAttention, mask form (kernel_codec.rs D_DECATTN) */
#define HOLO_OP_KV_CACHE_WRITE 120u
#define HOLO_OP_DECODE_ATTN_VALID 121u    /* DecodeAttentionValid (kernel_codec.rs D_DAVL) */
#define HOLO_OP_KV_QUANT_APPEND 122u      /* new: int8 quantize + ring append   */
#define HOLO_OP_DECODE_ATTN_I8 123u       /* new: GQA decode over an int8 cache */
#define HOLO_OP_ARGMAX 124u               /* new: per-row argmax (greedy pick)  */
#define HOLO_OP_ATTN_I8_ROWS 125u         /* new: multi-row (prefill) form of 123 */
#define HOLO_OP_TRANSPOSE 61u             /* Transpose (kernel_codec.rs:80)     */
#define HOLO_OP_RESHAPE 60u               /* Reshape (kernel_codec.rs:79, D_RESHAPE) */
#define HOLO_OP_SLICE 63u                 /* Slice (kernel_codec.rs:82, D_SLICE)     */

/* BufferRef, crates/hologram-compute/src/workspace.rs:16-24.
 * length == 0 means "to the end of the slot"; slot == HOLO_SLOT_ABSENT marks an
 * absent operand (kernel_call.rs:217-228). */
typedef struct holo_buffer_ref {
    uint32_t slot;
    uint64_t offset;
    uint64_t length;
} holo_buffer_ref;
#define HOLO_SLOT_ABSENT 0xFFFFFFFFu

/* UnaryCall, kernel_call.rs:28-36. Sigmoid/Tanh/Gelu/Silu/Exp over bf16/f16
 * run as a gather through the 65536-entry table (src/cpu/lut.rs:76-98); Relu,
 * Elu and Selu over bf16/f16 through the same kind of table of
 * narrow(f(widen(x))); every one of them over f32 is computed per element with
 * the reference's scalar function (exp_f32_det, libm expf for Exp/Elu/Selu). */
typedef struct holo_unary_call {
    holo_buffer_ref input;
    holo_buffer_ref output;
    uint64_t element_count;
    uint16_t witt_bits;
    uint8_t dtype;
} holo_unary_call;

/* BinaryCall, kernel_call.rs:38-46. Add / Mul over f16, bf16 or f32: widen, one
 * IEEE f32 operation, narrow (bf16 by truncation, f16 by the reference's
 * rounding, src/cpu/dtype.rs:121-153) — binary_float,
 * src/cpu/float_kernels.rs:238-300. */
typedef struct holo_binary_call {
    holo_buffer_ref a;
    holo_buffer_ref b;
    holo_buffer_ref output;
    uint64_t element_count;
    uint16_t witt_bits;
    uint8_t dtype;
} holo_binary_call;

/* NormCall, kernel_call.rs:422-446, as RmsNorm (src/cpu/float_kernels.rs:
 * 1683-1755): per row of `feature` values, out = x * (1 / sqrtf(mean(x^2) +
 * eps)) * gamma (gamma absent: 1). eps = f32(epsilon_bits), 0 selects 1e-9
 * (float_kernels.rs:1324-1336). beta and residual must be absent; channels and
 * num_groups must be 0. dtype f16, bf16 or f32.
 * As AddRmsNorm (tag 54, add_rms_norm_float, float_kernels.rs:1566-1672): the
 * rows are v = x + residual (residual optional), summed in f32 and never
 * narrowed; beta, channels and num_groups are ignored. */
typedef struct holo_norm_call {
    holo_buffer_ref x;
    holo_buffer_ref gamma;
    holo_buffer_ref beta;
    holo_buffer_ref residual;
    holo_buffer_ref output;
    uint32_t batch, feature, channels, num_groups;
    uint64_t epsilon_bits;
    uint8_t dtype;
} holo_norm_call;

/* RoPECall, kernel_call.rs:500-515 (rope_float, float_kernels.rs:3123-3186):
 * rotate-half over heads of head_dim; cos/sin tables have x's element layout;
 * f16, bf16 or f32. */
typedef struct holo_rope_call {
    holo_buffer_ref x;
    holo_buffer_ref cos;
    holo_buffer_ref sin;
    holo_buffer_ref output;
    uint32_t head_dim;
    uint64_t element_count;
    uint8_t dtype;
} holo_rope_call;

/* GatherCall, kernel_call.rs:380-404 (gather, src/cpu/kernels.rs:389-447):
 * out[o][k] = data[o][idx[k]] rows of `inner` elements; i32/i64 indices with
 * negative wrap. An index out of range is a SlotOutOfRange(indices) error; the
 * device reports it at the next holo_hip_synchronize (its row is zeroed). */
typedef struct holo_gather_call {
    holo_buffer_ref data;
    holo_buffer_ref indices;
    holo_buffer_ref output;
    uint64_t outer, axis_dim, inner, num_indices;
    uint8_t idx_dtype;
    uint8_t dtype;
} holo_gather_call;

/* New (tag 124): per-row argmax, the greedy token pick of a decode step,
 * kept on the device so the next step's Gather reads the ids in place.
 * out[r] = the lowest index of the largest value of row r (NaN never wins;
 * a row with no comparable value gives 0), as i32. input bf16 or f32
 * [rows, cols]. */
typedef struct holo_argmax_call {
    holo_buffer_ref input;
    holo_buffer_ref output;
    uint32_t rows, cols;
    uint8_t dtype;
} holo_argmax_call;

/* MatMulCall, kernel_call.rs:49-65. Row-major A[m,k] * B[k,n] -> C[m,n];
 * f32, bf16 or f16 (fp32 accumulation; a bf16 result narrowed by truncation,
 * an f16 one with the reference's rounding, src/cpu/dtype.rs:121-153;
 * src/cpu/float_kernels.rs:368-392). b_packed = 1 (f32 only) reads B in the
 * reference compiler's panel layout, f32[ceil(n/16)][k][16] (src/layout.rs:16-45). */
typedef struct holo_matmul_call {
    holo_buffer_ref a;
    holo_buffer_ref b;
    holo_buffer_ref output;
    uint32_t m, k, n;
    uint8_t dtype;
    uint8_t b_packed;
} holo_matmul_call;

/* The fused MatMul epilogues the reference's loader produces from
 * `matmul -> activation` and `matmul -> add(residual)` (fuse_matmul_epilogue,
 * crates/hologram-exec/src/session.rs:2150-2373), kernel_call.rs:892-929:
 *   MatMulActivation     out = f(A*B)           (float_kernels.rs:816-844)
 *   MatMulAdd            out = A*B + residual   (:846-888)
 *   MatMulAddActivation  out = f(A*B + residual) (:890-935)
 * bf16 results are narrowed after the product (and again after the add), as
 * the separate kernels would. Served activations: bf16 GELU/SILU/SIGMOID/TANH/
 * EXP for MatMulActivation (through the same 65536-entry tables as the unary
 * ops); GELU/SILU/SIGMOID/TANH otherwise (exp_f32_det); the rest return
 * UnsupportedOp. The residual must not overlap the output (split_borrow). */
typedef struct holo_matmul_act_call {
    holo_matmul_call mm;
    uint8_t act;
} holo_matmul_act_call;
typedef struct holo_matmul_add_call {
    holo_matmul_call mm;
    holo_buffer_ref residual;
} holo_matmul_add_call;
typedef struct holo_matmul_add_act_call {
    holo_matmul_call mm;
    holo_buffer_ref residual;
    uint8_t act;
} holo_matmul_add_act_call;

/* KvCacheWriteCall, kernel_call.rs:742-759 (byte rows, honest copy:
 * src/cpu/kernels.rs:455-501). `pos` is a device-resident 4-byte LE u32. */
typedef struct holo_kv_cache_write_call {
    holo_buffer_ref cache;
    holo_buffer_ref new_rows_buf;
    holo_buffer_ref pos;
    holo_buffer_ref output;
    uint32_t planes, bucket_rows, new_rows, row_bytes;
} holo_kv_cache_write_call;

/* DecodeAttentionValidCall, kernel_call.rs:691-716 (decode_attention_valid_float,
 * src/cpu/float_kernels.rs:4192-4307), the reference's decode attention:
 * q [batch, heads, q_rows, head_dim]; k/v_past [batch, kv_heads, past_len,
 * head_dim] of which the first min(valid_len, past_len) rows are realized;
 * k/v_new [batch, kv_heads, new_len, head_dim]; valid_len a 4-byte LE u32 read
 * by the device (content, one graph serves every step); out like q. Query row
 * qi of head h (kv head h / (heads / kv_heads)) sees the realized past rows,
 * then new rows 0..min(qi + 1, new_len). Scores dot(q, k) / s with s =
 * sqrtf(head_dim) (at least 1) or 1 / f32(scale_bits); f32 softmax; no
 * visible key gives the zero row. dtype bf16, f16 or f32 (all operands);
 * q_rows must equal new_len >= 1; kv_heads 0 means heads; head_dim <= 4096. */
typedef struct holo_decode_attention_valid_call {
    holo_buffer_ref q;
    holo_buffer_ref k_past;
    holo_buffer_ref v_past;
    holo_buffer_ref k_new;
    holo_buffer_ref v_new;
    holo_buffer_ref valid_len;
    holo_buffer_ref output;
    uint32_t batch, heads, kv_heads, q_rows, past_len, new_len, head_dim, scale_bits;
    uint8_t dtype;
} holo_decode_attention_valid_call;

/* DecodeAttentionCall, kernel_call.rs:632-656 (decode_attention_float,
 * src/cpu/float_kernels.rs:2482-2600, row function :2420-2477), the mask form
 * of decode attention: the same operands as DecodeAttentionValid with the
 * additive mask, f32 [q_rows, past_len + new_len] shared by batch and heads,
 * in place of valid_len. Every past row, then every new row, is a key; query
 * row qi scores key j as dot(q, k_j) / s + mask[qi][j] (s as in
 * DecodeAttentionValid); f32 softmax; a row whose every score is -inf is the
 * zero row. Any q_rows >= 1 and new_len >= 0 pair; past_len + new_len >= 1;
 * dtype bf16, f16 or f32 for q, K, V and out; kv_heads 0 means heads;
 * head_dim <= 4096. */
typedef struct holo_decode_attention_call {
    holo_buffer_ref q;
    holo_buffer_ref k_past;
    holo_buffer_ref v_past;
    holo_buffer_ref k_new;
    holo_buffer_ref v_new;
    holo_buffer_ref mask;
    holo_buffer_ref output;
    uint32_t batch, heads, kv_heads, q_rows, past_len, new_len, head_dim, scale_bits;
    uint8_t dtype;
} holo_decode_attention_call;

/* DequantizeCall, kernel_call.rs:782-818 (dequantize, src/cpu/kernels.rs:185-296):
 * out[i] = (q[i] - zp) as f32 * scale, per tensor (scale_bits, zero_point) or
 * per channel (channels > 0 and scales present: channel (i / inner) % channels
 * reads scales[ch] f32 and zero_points[ch] i32). quant_dtype i8, u8 or i4
 * (nibbles, low first, sign-extended); dtype f32, bf16 or f16. The extended
 * wire form (118) adds weight_layout, act_quant and codebook, which the
 * loader's dequant -> matmul fusion reads; the standalone op ignores them. */
typedef struct holo_dequantize_call {
    holo_buffer_ref input;
    holo_buffer_ref scales;
    holo_buffer_ref zero_points;
    holo_buffer_ref output;
    uint64_t element_count;
    uint32_t channels, inner;
    uint8_t quant_dtype;
    uint8_t dtype;
    uint32_t scale_bits;
    int32_t zero_point;
    holo_buffer_ref codebook;   /* HOLO_SLOT_ABSENT unless 118 carries one */
    uint8_t weight_layout;      /* 0 row-major [k,n], 1 output-major [n,k] */
    uint8_t act_quant;          /* 0 W8A32, 1 W8A8 per-token symmetric */
} holo_dequantize_call;

/* MatMulDequantCall, kernel_call.rs:162-273 (matmul_dequant_float +
 * matmul_dequant_epilogue, src/cpu/float_kernels.rs:459-760): out = act(A .
 * dequant(Bq) [+ residual]), f32 A and output.
 *   bq_omajor = 1 with act_quant = 1 (W8A8): Bq output-major, symmetric
 *   per-channel (channels == n, inner == 1, zero points 0, which the device
 *   checks and reports at the next holo_hip_synchronize), i8 / i4 / e8cb
 *   (codebook: 256 x 8 i8); each A row quantized per token, exact int32 dots,
 *   out = (acc as f32) * (scale_a * scales[j]): bit-exact.
 *   otherwise (W8A32): Bq [k,n] i8 / u8 / i4, per tensor or per channel,
 *   dequantized to f32 and multiplied in f32 (within 1e-5).
 * act: fused_activation id (0 none); residual: HOLO_SLOT_ABSENT for none. */
typedef struct holo_matmul_dequant_call {
    holo_buffer_ref a;
    holo_buffer_ref bq;
    holo_buffer_ref scales;
    holo_buffer_ref zero_points;
    holo_buffer_ref output;
    uint32_t m, k, n, channels, inner;
    uint8_t quant_dtype;
    uint8_t dtype;
    uint32_t scale_bits;
    int32_t zero_point;
    uint8_t bq_omajor;
    uint8_t act_quant;
    uint8_t act;
    holo_buffer_ref residual;
    holo_buffer_ref codebook;
} holo_matmul_dequant_call;

/* DequantActivationCall, kernel_call.rs:275-290 (dequant_activation,
 * src/cpu/kernels.rs:311-388): out[i] = f((q[i] - zp) as f32 * scale) as f32,
 * the table of the <= 256 levels built once per call with the reference's
 * scalar function f of lut_act id `act` (0-4). i8 / u8 / i4 input. */
typedef struct holo_dequant_activation_call {
    holo_buffer_ref input;
    holo_buffer_ref output;
    uint64_t element_count;
    uint8_t quant_dtype;
    uint8_t act;
    uint8_t dtype;
    uint32_t scale_bits;
    int32_t zero_point;
} holo_dequant_activation_call;

/* New (tag 122): int8 KV quantize + append. Each new row (head_dim values of
 * `dtype` in {bf16, f16, f32}) is quantized with the reference's per-row
 * symmetric scheme (src/cpu/simd.rs:4755-4785: scale = max|x|/127,
 * q = clamp(round-half-away(x * (127/max|x|)), -127, 127); an all-zero row is
 * q = 0, scale = 0) and placed at ring row (pos + j) % bucket_rows of plane p,
 * as KvCacheWrite places rows. Caches: int8 [planes, bucket_rows, head_dim] and
 * f32 scales [planes, bucket_rows].
 *   output == cache and output_scales == cache_scales (same slot and offset):
 *       in-place form (the executor's O(new_rows) move, session.rs:1313-1370);
 *   otherwise: honest-copy form, outputs must not overlap any input. */
typedef struct holo_kv_quant_append_call {
    holo_buffer_ref new_rows_buf;
    holo_buffer_ref pos;
    holo_buffer_ref cache;
    holo_buffer_ref cache_scales;
    holo_buffer_ref output;
    holo_buffer_ref output_scales;
    uint32_t planes, bucket_rows, new_rows, head_dim;
    uint8_t dtype;
} holo_kv_quant_append_call;

/* New (tag 123): single-token GQA decode attention over int8 K/V caches laid
 * out as holo_kv_quant_append_call writes them. For sequence b the visible keys
 * are rows [0, min(lens[b], bucket_rows)) of each kv-head plane; query head h
 * reads kv head h / (heads / kv_heads) (kernel_call.rs:691-716). Scores are
 * dot(q, k_dequant) / scale with scale = sqrtf(head_dim) (or 1/f32(scale_bits)),
 * fp32 softmax; the result equals the reference DecodeAttentionValid
 * {b=1, past=L-1, valid=L-1, q_rows=new=1} over the dequantized rows
 * (src/cpu/float_kernels.rs:4192-4307) within tolerance. A sequence with no
 * visible key produces the exact zero vector. q/output dtype: bf16 or f32
 * ([batch, heads, head_dim]); lens: u32 [batch], device-resident. */
typedef struct holo_decode_attention_i8_call {
    holo_buffer_ref q;
    holo_buffer_ref k_cache;
    holo_buffer_ref v_cache;
    holo_buffer_ref k_scales;
    holo_buffer_ref v_scales;
    holo_buffer_ref lens;
    holo_buffer_ref output;
    uint32_t batch, heads, kv_heads, bucket_rows, head_dim, scale_bits;
    uint8_t dtype;
} holo_decode_attention_i8_call;

/* New (tag 125): the multi-row form of tag 123, a prompt's rows against the
 * int8 cache they were appended to (prefill). q / output are
 * [batch, q_rows, heads, head_dim]; lens[b] is the visible length of sequence
 * b's last row, and row t sees the first lens[b] - (q_rows - 1 - t) rows of its
 * planes (none when that is not positive), at most bucket_rows: the causal
 * visibility of DecodeAttentionValid's new rows, past prefix then min(qi + 1, new)
 * (src/cpu/float_kernels.rs:3926). q_rows = 1 is tag 123. With q_rows > 1 every
 * lens[b] must be at most bucket_rows: once a multi-row append wraps the ring,
 * later rows have overwritten slots the earlier rows must see. The lengths
 * live on the device, so a violation is reported (UnsupportedOp) by the next
 * holo_hip_synchronize. */
typedef struct holo_attention_i8_rows_call {
    holo_decode_attention_i8_call attn;
    uint32_t q_rows;
} holo_attention_i8_rows_call;

/* TransposeCall, kernel_call.rs:487-499 (transpose_float,
 * src/cpu/float_kernels.rs:2980-3028): output axis i is input axis perm[i] of
 * the row-major input of shape dims[0..rank). rank 1..8; f16/bf16/f32 elements;
 * perm must be a permutation of 0..rank-1. */
typedef struct holo_transpose_call {
    holo_buffer_ref input;
    holo_buffer_ref output;
    uint8_t rank;
    uint32_t dims[8];
    uint8_t perm[8];
    uint8_t dtype;
} holo_transpose_call;

/* LayoutCall, kernel_call.rs:479-485, as Reshape (tag 60) and Slice (tag 63):
 * the first element_count elements of the input view copied to the output
 * view — element_count x the element width bytes for f16/bf16/f32
 * (layout_float, src/cpu/float_kernels.rs:2939-2954), element_count bytes for
 * the byte-domain dtypes (layout_copy, src/cpu/kernels.rs:688-701); f64 is
 * refused (kernels.rs:1611-1615). A Slice's input view is the field it
 * projects. Inside a session an interior Reshape or Slice moves nothing: its
 * output slot is bound to its input's memory (session.rs:1106-1150); only one
 * that writes an output port copies. */
typedef struct holo_layout_call {
    holo_buffer_ref input;
    holo_buffer_ref output;
    uint64_t element_count;
    uint8_t dtype;
} holo_layout_call;

/* KernelCall (kernel_call.rs:1146-1276): tag + the variant's payload. */
typedef struct holo_kernel_call {
    uint32_t tag;
    union {
        holo_unary_call unary;
        holo_binary_call binary;
        holo_norm_call norm;
        holo_rope_call rope;
        holo_gather_call gather;
        holo_argmax_call argmax;
        holo_matmul_call matmul;
        holo_matmul_act_call matmul_act;
        holo_matmul_add_call matmul_add;
        holo_matmul_add_act_call matmul_add_act;
        holo_kv_cache_write_call kv_write;
        holo_kv_quant_append_call kv_quant_append;
        holo_decode_attention_valid_call attn_valid;
        holo_decode_attention_call attn_mask;
        holo_dequantize_call dequantize;
        holo_matmul_dequant_call matmul_dequant;
        holo_dequant_activation_call dequant_act;
        holo_decode_attention_i8_call attn_i8;
        holo_attention_i8_rows_call attn_i8_rows;
        holo_transpose_call transpose;
        holo_layout_call layout;
    } u;
} holo_kernel_call;

typedef struct holo_backend holo_backend;

/* Create a backend on HIP device `device`, enqueueing on `stream` (a
 * hipStream_t; NULL = the device's null stream). Replaces CpuBackend::new()
 * (crates/hologram-compute/src/cpu.rs:55-87). */
int holo_hip_backend_create(int device, void *stream, holo_backend **out);
int holo_hip_backend_destroy(holo_backend *be);
/* Change the stream later dispatches enqueue on. */
int holo_hip_set_stream(holo_backend *be, void *stream);

/* Bind slot -> device range (pool-owned memory; the backend never frees it).
 * The slot table is the device form of BufferArena's binding table
 * (crates/hologram-exec/src/buffer.rs:312-335). */
int holo_hip_slot_bind(holo_backend *be, uint32_t slot, void *device_ptr, uint64_t bytes);
int holo_hip_slot_unbind(holo_backend *be, uint32_t slot);

/* Backend::dispatch (backend.rs:8-15): validate, then enqueue the call's
 * kernels on the backend's stream. Asynchronous: call holo_hip_synchronize
 * before the host reads any output. Unsupported tags return
 * HOLO_ERR_UNSUPPORTED_OP so the caller can route the call elsewhere, as the
 * reference's GPU backends do (src/metal_backend/mod.rs:172-180). */
int holo_hip_dispatch(holo_backend *be, const holo_kernel_call *call);
/* No counterpart in the reference: the allocation-free variant of
 * holo_hip_dispatch, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). It serves DecodeAttentionI8 (123) and AttentionI8Rows (125),
 * whose kernels need split-K scratch, from a fixed 16 MiB device array per GPU
 * (held until the process ends) instead of the backend's grown scratch; it
 * calls no hipMalloc/hipFree. A call needing more scratch than 16 MiB is
 * refused with HOLO_ERR_UNSUPPORTED_OP (config 4's batch needs about 2 MiB).
 * All calls on one GPU share that array: calls that overlap in time on one
 * GPU (other streams, other threads, other backends) race; serialize them.
 * Results are bit-identical to holo_hip_dispatch of the same call. */
int holo_hip_dispatch_noalloc(holo_backend *be, const holo_kernel_call *call);
/* Same, from one call in the archive wire format (u16 LE discriminant + LE
 * payload, crates/hologram-archive/src/kernel_codec.rs:130-137, 557-813).
 * *consumed receives the encoded length. */
int holo_hip_dispatch_encoded(holo_backend *be, const uint8_t *wire, size_t len,
                              size_t *consumed);
int holo_hip_synchronize(holo_backend *be);

/* Host-side checks of one call against slot sizes, with no device work
 * (the refusals of src/cpu/kernels.rs, float_kernels.rs; split_borrow's
 * overlap rule, buffer.rs:974-998). slot_bytes[i] = size of slot i. */
int holo_hip_validate(const holo_kernel_call *call, const uint64_t *slot_bytes, uint32_t nslots);
/* Decode one wire-format call into *out (no device work). */
int holo_hip_decode_call(const uint8_t *wire, size_t len, holo_kernel_call *out, size_t *consumed);

/* The 65536-entry table the backend stages in LDS for (act, dtype):
 * T[b] = narrow(f(widen(b))), src/cpu/lut.rs:43-67. */
int holo_hip_lut_table(int act, int dtype, uint16_t *out65536);

/* ---- Session: a `.holo` archive run over device-resident slots ----------
 * The InferenceSession of crates/hologram-exec/src/session.rs (load :428-797,
 * execute :846-932, the node walk compute_and_label :1052-1289) with this
 * backend behind every node. Load checks the header, version 2..=3 and the
 * BLAKE3 footer (crates/hologram-archive/src/loader.rs:141-185), decodes the
 * KernelCalls, Inputs/Outputs, ExecPlan, Constants and Weights sections,
 * uploads every constant once, and gives every other slot a device buffer.
 * A KV write whose cache no other node reads runs as the in-place move
 * (session.rs:1163-1190): its output port then aliases the cache buffer. */
typedef struct holo_session holo_session;

/* be == NULL loads dry: the archive is parsed, sized and every call validated,
 * but nothing is allocated and the session cannot execute (host-only checks). */
int holo_hip_session_load(holo_backend *be, const uint8_t *archive, size_t len,
                          holo_session **out);
/* Load with options. By default a load runs the reference's loader passes in
 * its order (session.rs:493-504): fuse_dequant_matmul (a Dequantize read only
 * as an f32 MatMul's B becomes a MatMulDequant; an output-major weight
 * declaration nothing can read refuses the load), fuse_matmul_epilogue
 * (session.rs:2150-2373), fuse_dequant_activation (a per-tensor f32 Dequantize
 * read only by an f32 transcendental becomes a DequantActivation), and then
 * this backend's device
 * fusion: few-row MatMuls that share their A operand run as one launch, and
 * the ops that only consume such a product (rotary embedding, int8
 * quantize+append, the SwiGLU product) run inside the launch that finishes
 * it. A bf16 RmsNorm between two such MatMuls is split between them: the
 * first leaves each row's sums of squares, the second normalizes its A as it
 * reads it, and the norm's own launch and output go away. All of these give
 * the same bits as the unfused walk; the flags turn them off
 * (NO_DEVICE_FUSION also turns off the norm fusion; NO_DEQUANT_FUSION the two
 * dequant passes). A bf16 group of at most 16 rows whose weights are
 * constants of the archive runs as one launch: at load each such weight is
 * copied once into the matrix cores' operand order (the archive's own copy
 * stays), a workgroup owns a 16-column tile (a SwiGLU tile pair, a head) over
 * the whole of K, and a fused RmsNorm's statistics are taken in that launch;
 * the few-row product's summation order is fixed by K alone, so this too is
 * bit-identical. NO_WEIGHT_PACKING keeps the split-K launches. A decode
 * step's q/k/v group (every product head-wise: RoPE and / or the int8 append)
 * followed by the int8 decode attention over what it wrote leaves its split-K
 * epilogue to that attention's launch, each workgroup finishing its own
 * plane's heads first (the same device code, so the same bits);
 * NO_ATTN_PROLOGUE keeps the epilogue a launch of its own. */
#define HOLO_SESSION_NO_EPILOGUE_FUSION 1u
#define HOLO_SESSION_NO_DEVICE_FUSION 2u
#define HOLO_SESSION_NO_NORM_FUSION 4u
#define HOLO_SESSION_NO_DEQUANT_FUSION 8u
#define HOLO_SESSION_NO_WEIGHT_PACKING 16u
#define HOLO_SESSION_NO_ATTN_PROLOGUE 32u
int holo_hip_session_load_ex(holo_backend *be, const uint8_t *archive, size_t len, uint32_t flags,
                             holo_session **out);
/* Steps of one walk after fusion (each a call or a fused MatMul group), and
 * how many of them are fused groups. Steps bound at load instead of run (an
 * interior Reshape or Slice, a repeat of a value the walk already holds) are
 * not counted. */
int holo_hip_session_nodes(const holo_session *s, uint32_t *n_nodes, uint32_t *n_groups);
/* The last walk's steps dispatched and skipped (last_dispatched /
 * last_skipped, session.rs:1291-1310): skipped counts the steps bound at load,
 * the steps a memo-on holo_hip_session_execute_bytes found unchanged since
 * the previous walk, and every step on a whole-graph memo hit. */
int holo_hip_session_last_walk(const holo_session *s, uint32_t *dispatched, uint32_t *skipped);
/* Fused groups that run as one launch over packed weights, and the device
 * bytes the packed copies of their weights hold (no counterpart in the
 * reference: its CPU kernels read weights in place). */
int holo_hip_session_packed(const holo_session *s, uint32_t *groups, uint64_t *bytes);
/* Fused groups that leave their split-K epilogue to the int8 decode attention
 * after them (NO_ATTN_PROLOGUE; no counterpart in the reference). Decided at
 * load; a launch shape the fused kernel does not take (more than one chunk a
 * plane, the balanced form, head_dim other than 64 / 128, f32) runs the
 * epilogue on its own at dispatch. */
int holo_hip_session_attn_prologues(const holo_session *s, uint32_t *n);
/* The index-th kernel call of the loaded schedule, after the reference's
 * loader passes (the calls the reference's Session counts with
 * dequant_fused_count and its siblings, session.rs:1390-1437). */
int holo_hip_session_call(const holo_session *s, uint32_t index, holo_kernel_call *out);
/* The output ports' κ-labels for the given input-port labels (n_inputs x
 * HOLO_LABEL_LEN bytes in, n_outputs x HOLO_LABEL_LEN out), derived through
 * the loaded schedule as the reference's compute_and_label does
 * (session.rs:1052-1289): constants are labelled by their content, each call
 * by derive_label over its op signature and its operands' labels (buffers()
 * order, kernel_call.rs:1526-1660; Add and Mul sort theirs), a Reshape by its
 * input's label; the call that writes an output port gives that port the
 * boundary form, derive_label_boundary (address.rs:197-221), while later
 * calls derive from its plain label; a port no call writes carries its
 * input's or constant's label. Works on a dry load. */
int holo_hip_session_output_labels(const holo_session *s, const char *input_labels, char *out);
/* Execute from host bytes with the reference's whole-graph memo
 * (session.rs:841-905): each input is labelled by its bytes (a port whose
 * bytes repeat is not hashed again); when the labels equal the last walk's
 * and nothing has touched the session since (no bind, write, execute,
 * capture or replay in between), the outputs already in place are those of
 * these inputs and the walk is skipped (*memo_hit = 1). Writing session
 * memory through a pointer from holo_hip_session_output is outside what the
 * memo sees: turn it off first. `sizes[i]` bytes of input i are used, at most
 * its port's size. */
int holo_hip_session_execute_bytes(holo_session *s, const void *const *inputs, const uint64_t *sizes,
                                   uint32_t n, int *memo_hit);
/* Turn the memo's hits on (the default) or off (benchmarks: every call walks). */
int holo_hip_session_set_memo(holo_session *s, int enabled);
int holo_hip_session_close(holo_session *s);
int holo_hip_session_info(const holo_session *s, uint32_t *n_inputs, uint32_t *n_outputs,
                          uint32_t *n_calls, uint32_t *n_slots);
/* Port `index` of the inputs (is_output = 0) or outputs: its slot, element
 * count, dtype tag and byte size. */
int holo_hip_session_port(const holo_session *s, int is_output, uint32_t index, uint32_t *slot,
                          uint64_t *element_count, uint8_t *dtype, uint64_t *bytes);
/* The verified 32-byte footer fingerprint (HoloLoader::fingerprint). */
int holo_hip_session_fingerprint(const holo_session *s, uint8_t out32[32]);
/* Bind input port `index` to caller-owned device memory (zero copy, the
 * execute_addressed form, session.rs:942-984); NULL restores the session's
 * own buffer. */
int holo_hip_session_bind_input(holo_session *s, uint32_t index, void *device_ptr, uint64_t bytes);
/* Copy host bytes into input port `index`'s current buffer (the execute form). */
int holo_hip_session_write_input(holo_session *s, uint32_t index, const void *host, uint64_t bytes);
/* One walk of the plan, enqueued on the session's stream (asynchronous). */
int holo_hip_session_execute(holo_session *s);
/* Record the walk once into a HIP graph (after one eager walk), then replay it.
 * Replay refuses if an input was rebound since the capture. */
int holo_hip_session_capture(holo_session *s);
int holo_hip_session_replay(holo_session *s);
/* Wait for the session's stream; reports device-side refusals (Gather range). */
int holo_hip_session_synchronize(holo_session *s);
int holo_hip_session_stream(const holo_session *s, void **stream);
/* Device view of output port `index`, or a host copy of it (waits first). */
int holo_hip_session_output(const holo_session *s, uint32_t index, void **device_ptr,
                            uint64_t *bytes);
int holo_hip_session_read_output(holo_session *s, uint32_t index, void *host, uint64_t bytes);

/* BLAKE3 (default mode, 32-byte digest): the archive footer and weight
 * fingerprint hash (crates/hologram-archive/src/weight.rs WeightFingerprint). */
int holo_hip_blake3(const void *data, size_t len, uint8_t out32[32]);

/* κ-labels (crates/hologram-archive/src/address.rs): "blake3:" followed by the
 * 64 lowercase hex digits of a BLAKE3 digest, HOLO_LABEL_LEN ASCII bytes
 * (`out` receives them and a terminating NUL). */
#define HOLO_LABEL_LEN 71
/* derive_label_boundary (address.rs:197-221): the label an output port
 * receives from the call that writes it: the op's own label (address_bytes of
 * opcode u16 LE || params) composed left to right with each operand label,
 * each composition address_bytes(digest(acc) || digest(operand))
 * (compose.rs:154-164); with no operand, the op label composed with itself. */
int holo_hip_derive_label_boundary(uint16_t opcode, const uint8_t *params, uint64_t n_params,
                                   const char *labels, uint64_t n_labels, char out[72]);
/* address_bytes (address.rs:96-99): the label of opaque bytes. */
int holo_hip_address_bytes(const void *bytes, uint64_t len, char out[72]);
/* derive_label (address.rs:108-116): the label of a computed value, the digest
 * of opcode (u16 LE) || params || each operand label in order; `labels` holds
 * n_labels labels back to back (HOLO_LABEL_LEN bytes each). */
int holo_hip_derive_label(uint16_t opcode, const uint8_t *params, uint64_t n_params,
                          const char *labels, uint64_t n_labels, char out[72]);
/* KernelCall::op_signature (crates/hologram-compute/src/kernel_call.rs:
 * 1321-1500): the opcode and LE parameter bytes a call's label is derived
 * with. The new calls (122-125) take their discriminant as opcode and their
 * scalar fields in struct order. UnsupportedOp for a call not served here. */
int holo_hip_op_signature(const holo_kernel_call *call, uint16_t *opcode, uint8_t params[64],
                          uint32_t *n_params);

/* Message of the last failed call on this thread ("" if none). */
const char *holo_hip_last_error_message(void);

#ifdef __cplusplus
}
#endif
#endif
