// holo_kernels.h — launchers the host dispatcher calls; each is defined in the
// .hip file that holds its kernels. Pointers are device pointers already
// resolved and bounds-checked by the dispatcher; every launcher only enqueues
// on `stream` and returns the launch status.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace holo {

// lut.hip — out[i] = table[in[i]] for n u16 patterns; table is 65536 u16 in
// device memory, staged into LDS by every workgroup.
hipError_t launch_lut_u16(const uint16_t *table, const uint16_t *in, uint16_t *out,
                          uint64_t n, hipStream_t stream);

// kv.hip — byte copy (the honest-copy half of KvCacheWrite / KvQuantAppend).
hipError_t launch_copy_bytes(const void *src, void *dst, uint64_t bytes, hipStream_t stream);
// kv.hip — zero `bytes` bytes with a fill kernel (graph-capture safe).
hipError_t launch_fill_zero(void *dst, uint64_t bytes, hipStream_t stream);
// kv.hip — KvCacheWrite row placement: out[p][(pos+j)%bucket] = new[p][j].
hipError_t launch_kv_place_rows(const uint8_t *nw, const uint32_t *pos, uint8_t *out,
                                uint32_t planes, uint32_t bucket, uint32_t new_rows,
                                uint32_t row_bytes, hipStream_t stream);
// kv.hip — the copy form of the int8 quantize + ring append in one launch:
// caches copied to the outputs except the appended rows, which are quantized
// into place (requires kv_quant_copy_fusable).
bool kv_quant_copy_fusable(const void *cq, const void *cs, const void *oq, const void *os,
                           uint32_t planes, uint32_t bucket, uint32_t d);
hipError_t launch_kv_quant_copy_append(const void *nw, uint8_t dtype, const uint32_t *pos,
                                       const int8_t *cq, const float *cs, int8_t *oq, float *os,
                                       uint32_t planes, uint32_t bucket, uint32_t new_rows,
                                       uint32_t d, hipStream_t stream);
// kv.hip — int8 quantize + ring append into (cache_q, cache_s) in place.
hipError_t launch_kv_quant_append(const void *nw, uint8_t dtype, const uint32_t *pos,
                                  int8_t *cache_q, float *cache_s, uint32_t planes,
                                  uint32_t bucket, uint32_t new_rows, uint32_t head_dim,
                                  hipStream_t stream);

// static_scratch.hip — the fixed device scratch of holo_hip_dispatch_noalloc:
// kStaticScratchBytes per GPU, held until the process ends. init records this
// device's address of the array (call with `device` current, once per device);
// static_scratch returns it (nullptr before init).
constexpr size_t kStaticScratchBytes = size_t(16) << 20;
hipError_t static_scratch_init(int device);
void *static_scratch(int device);

// attn.hip — int8-KV GQA decode attention. `scratch` holds the split-K
// partials; attn_i8_scratch_bytes() gives its size. Calls sharing one scratch
// must not overlap.
struct AttnI8Args {
    const void *q;          // [B, H, D] bf16 or f32
    const int8_t *kq, *vq;  // [B, Hkv, bucket, D]
    const float *ks, *vs;   // [B, Hkv, bucket]
    const uint32_t *lens;   // [B]
    void *out;              // [B, H, D] bf16 or f32
    uint32_t B, H, Hkv, bucket, D;
    float score_scale;      // the divisor: sqrtf(D) or 1/scale_multiplier
    uint8_t dtype;
    uint32_t q_rows = 1;    // query rows per sequence (q/out [B, q_rows, H, D]); row t
                            // sees min(lens[b] - (q_rows - 1 - t), bucket) keys
};
size_t attn_i8_scratch_bytes(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t bucket, uint32_t D,
                             uint32_t q_rows = 1);
bool attn_i8_supported(uint32_t H, uint32_t Hkv, uint32_t D, uint32_t bucket);
hipError_t launch_attn_i8(const AttnI8Args &a, void *scratch, hipStream_t stream);
// The decode step's grid form with a few-row group's split-K epilogue in
// front (attn_pro_kernel): every segment head-wise at head_dim D, its heads a
// multiple of Hkv, one row per sequence, one appended row; q_rows 1, bf16, one
// chunk a plane. Needs no scratch. Declared after EpiArgs below.
struct EpiArgs;
bool attn_i8_pro_applies(const AttnI8Args &a, const EpiArgs &pro);
hipError_t launch_attn_i8_pro(const AttnI8Args &a, const EpiArgs &pro, hipStream_t stream);
// attn_valid.hip — the same op for every other head_dim (up to 4096) and any
// query-head group: a blocked split-K walk with each K/V block dequantized
// into LDS, then the merge of the shares.
bool attn_i8_any_supported(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t q_rows, uint32_t D);
size_t attn_i8_any_scratch_bytes(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t q_rows,
                                 uint32_t bucket, uint32_t D);
hipError_t launch_attn_i8_any(const AttnI8Args &a, void *scratch, hipStream_t stream);

// attn_valid.hip — DecodeAttentionValid (discriminant 121) over bf16/f16/f32
// K/V: q/out [B, H, M, D], k/v_past [B, Hkv, past, D], k/v_new [B, Hkv, nnew, D]
// (M == nnew), valid_len a 4-byte LE u32 on the device.
struct AttnValidArgs {
    const void *q, *kp, *vp, *kn, *vn;
    const uint8_t *valid_len;   // 121; null in the mask form
    const float *mask = nullptr;  // 119: f32 [M, past + nnew] added to the scores
    void *out;
    uint32_t B, H, Hkv, M, past, nnew, D;
    float scale;            // the divisor: sqrtf(D) (>= 1) or 1/scale_multiplier
    uint8_t dtype;          // 7 bf16, 6 f16, 8 f32
};
bool attn_valid_supported(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t M, uint32_t D);
size_t attn_valid_scratch_bytes(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t M, uint32_t past,
                                uint32_t nnew, uint32_t D);
hipError_t launch_attn_valid(const AttnValidArgs &a, void *scratch, hipStream_t stream);

// quant.hip — MatMulDequant's output-major W8A8 GEMM (f32 A quantized per
// row on the device, exact int32 dots, (acc as f32) * (scale_a * scales[j]),
// then + residual and the fused activation), Dequantize and
// DequantActivation. `scratch` holds the quantized rows
// (q_omajor_scratch_bytes).
struct QOmajorArgs {
    const float *a;           // [m][k] f32
    const void *bq;           // output-major weight: i8 [n][k], i4 [n][k/2], e8cb [n][k/8]
    const int8_t *codebook;   // e8cb: 256 x 8 i8
    const float *scales;      // [n]
    const float *residual;    // [m][n] f32 or null
    float *out;               // [m][n] f32
    uint32_t m, k, n;
    uint8_t tier;             // 2 i8, 10 i4, 11 e8cb
    uint32_t act;             // fused_activation id, 0 none
};
constexpr uint32_t kI8DotKMax = 133144;   // i32::MAX / (127 * 127), kernel_call.rs:103
size_t q_omajor_scratch_bytes(uint32_t m, uint32_t k);
hipError_t launch_matmul_q_omajor(const QOmajorArgs &a, void *scratch, hipStream_t stream);
struct DequantArgs {
    const void *in;           // i8 / u8 bytes, or i4 nibbles (low first)
    const float *scales;      // per-channel [channels], or null (per-tensor)
    const int32_t *zps;       // per-channel [channels]
    void *out;                // n elements of dtype
    uint64_t n;
    uint32_t channels, inner;
    uint8_t quant;            // 2 i8, 1 u8, 10 i4
    uint8_t dtype;            // 8 f32, 7 bf16, 6 f16
    float scale;
    int32_t zp;
};
hipError_t launch_dequantize(const DequantArgs &a, hipStream_t stream);
// Raise bit 4 of *err if any of the `count` little-endian i32 zero points at
// zps (any alignment) is nonzero (W8A8 symmetry).
hipError_t launch_zero_points_check(const void *zps, uint64_t count, int *err, hipStream_t stream);
// out[i] = table[level(i)]: i8/u8 index by the raw byte, i4 by the nibble.
hipError_t launch_dequant_act(const uint8_t *in, float *out, uint64_t n, bool i4,
                              const float table[256], hipStream_t stream);

// decoder_ops.hip — the other ops of a decode step; `dtype` is the element
// tag (f16 6, bf16 7, f32 8). op 0 = Add, 1 = Mul.
hipError_t launch_binary(int op, const void *a, const void *b, void *out, uint64_t n, uint8_t dtype,
                         hipStream_t stream);
// The fused MatMul epilogues over an f16 product in place: kind 1 = act,
// 2 = + residual, 3 = act(+ residual), computed in f32, narrowed once.
hipError_t launch_epilogue_f16(uint16_t *c, const uint16_t *res, uint64_t n, uint32_t kind,
                               uint32_t act, hipStream_t stream);
// out[i] = f(in[i]) over f32, f = act_f32(act) (a fused_activation id).
hipError_t launch_act_f32(const float *in, float *out, uint64_t n, uint32_t act,
                          hipStream_t stream);
// gamma == nullptr: no affine scale.
// AddRmsNorm: rows of x + residual (residual may be null), in f32.
hipError_t launch_add_rmsnorm(const void *x, const void *residual, const void *gamma, void *out,
                              uint32_t batch, uint32_t feature, float eps, uint8_t dtype,
                              hipStream_t stream);
hipError_t launch_rmsnorm(const void *x, const void *gamma, void *out, uint32_t batch,
                          uint32_t feature, float eps, uint8_t dtype, hipStream_t stream);
hipError_t launch_rope(const void *x, const void *cs, const void *sn, void *out, uint32_t head_dim,
                       uint64_t n, uint8_t dtype, hipStream_t stream);
// Row gather; an out-of-range index zeroes its row and sets *err (device int).
// Raise bit 2 of *err if any of lens[0..n) exceeds bucket (multi-row attention).
hipError_t launch_lens_within(const uint32_t *lens, uint32_t n, uint32_t bucket, int *err,
                              hipStream_t stream);
hipError_t launch_gather(const void *data, const void *idx, void *out, uint64_t outer,
                         uint64_t axis_dim, uint64_t num_idx, uint64_t row_bytes, bool i64,
                         int *err, hipStream_t stream);
hipError_t launch_argmax(const void *in, int32_t *out, uint32_t rows, uint32_t cols, bool bf16,
                         hipStream_t stream);
// Axis permutation of a row-major [dims[0], .., dims[rank-1]] tensor of es-byte
// elements: output axis i is input axis perm[i] (perm a permutation of 0..rank-1).
hipError_t launch_transpose(const void *in, void *out, uint32_t rank, const uint32_t *dims,
                            const uint8_t *perm, uint32_t es, hipStream_t stream);

// gemm.hip — C = A*B row-major, fp32 accumulation. dtype f32 or bf16 (bf16
// result narrowed by truncation). `scratch` holds split-K partials of the
// few-row path, matmul_scratch_bytes() bytes (0: none needed). Calls sharing
// one scratch must not overlap.
// An element-wise epilogue over a tiled MatMul's output, in place (kind as
// EpiSeg::base: 1 activation, 2 + residual, 3 + residual then activation); the
// same arithmetic as the separate kernels.
struct TileEpi {
    uint8_t kind = 0;
    uint32_t act = 0;                  // fused_activation id (f32, and bf16 kind 3)
    const uint16_t *lut = nullptr;     // bf16 kind 1: the activation's table
    const void *residual = nullptr;    // kinds 2, 3: [count], same dtype
};
hipError_t launch_tile_epilogue(void *c, uint64_t count, bool bf16, const TileEpi &epi,
                                hipStream_t stream);
size_t matmul_scratch_bytes(uint32_t m, uint32_t k, uint32_t n, uint8_t dtype);
hipError_t launch_matmul(const void *a, const void *b, void *c, uint32_t m, uint32_t k,
                         uint32_t n, uint8_t dtype, void *scratch, hipStream_t stream);
// f32 C = A * B with B in the reference's panel-packed layout (src/layout.rs:
// 16-45): [ceil(n/16)][k][16] floats, columns past n zero.
hipError_t launch_matmul_f32_packed(const float *a, const float *b_packed, float *c, uint32_t m,
                                   uint32_t k, uint32_t n, hipStream_t stream);
// The packed layout's length in elements (layout::packed_len).
inline uint64_t packed_len(uint32_t k, uint32_t n) { return uint64_t((n + 15) / 16) * k * 16; }

// gemm_skinny.hip — the few-row (m <= 64) path that launch_matmul takes when
// it applies (16-byte aligned operands required by the caller).
constexpr int kSkinnyMaxSeg = 4;
struct SkinnyPlan {
    int mt = 0, steps = 0;             // 16-row tiles of A; k steps per wave (0: does not apply)
    uint32_t kc = 0, ks = 0, strips = 0;   // K rows per workgroup, K ranges, column strips
};
SkinnyPlan matmul_skinny_plan(uint32_t m, uint32_t k, uint32_t n, uint8_t dtype);
bool matmul_skinny_applies(uint32_t m, uint32_t k, uint32_t n, uint8_t dtype);
size_t matmul_skinny_scratch_bytes(uint32_t m, uint32_t k, uint32_t n, uint8_t dtype);
hipError_t launch_matmul_skinny(const void *a, const void *b, void *c, uint32_t m, uint32_t k,
                                uint32_t n, uint8_t dtype, void *scratch, hipStream_t stream);
// One launch over up to kSkinnyMaxSeg products sharing A[m, k]: segment s is
// B_s [k, n_s]. Every segment's fp32 partials go to P [plan.ks][m][ntot]
// (ntot = sum of n_s), segment s at columns sum(n_0 .. n_{s-1}); `plan` must be
// the plan each segment has on its own (the sums then match a single call).
// epilogue.hip — the finish of a few-row MatMul group: partials summed in ks
// order, then per segment the base value (the product, + residual, activation),
// and optionally rotary embedding, int8 quantize + append, and the product with
// another segment's value. The same operations in the same order as the
// standalone kernels they stand in for.
constexpr uint8_t kEpiStore = 0, kEpiAct = 1, kEpiAdd = 2, kEpiAddAct = 3;
// fused_activation ids (crates/hologram-compute/src/kernel_call.rs:861-870)
constexpr uint32_t kFusedRelu = 1, kFusedGelu = 2, kFusedSilu = 3, kFusedSigmoid = 4,
                   kFusedTanh = 5, kFusedElu = 6, kFusedSelu = 7, kFusedExp = 8;
// The f32 Erf unary's id in act_f32 (Erf has no fused_activation id, so no
// fusion produces it).
constexpr uint32_t kActErf = 9;
// Table ids of the 16-bit fused Relu/Elu/Selu (beyond lut_act's 0-5).
constexpr int kTableRelu = 6, kTableElu = 7, kTableSelu = 8;
struct EpiSeg {
    uint32_t n = 0, col0 = 0;          // columns; first column in the partials' column space
    uint8_t base = kEpiStore;
    uint32_t act = 0;                  // f32: fused_activation id
    const uint16_t *lut = nullptr;     // bf16: the activation's table (same as the unary op's)
    const void *residual = nullptr;    // [m, n]
    void *out = nullptr;               // [m, n] base value, or null (not materialized)
    uint32_t head_dim = 0;             // > 0: head-wise (rope and/or quant), power of 2 <= 128
    bool rope = false;
    const void *cos = nullptr, *sin = nullptr;
    void *rope_out = nullptr;          // null: the rotated value is not materialized
    bool quant = false;                // in-place append of each head row
    const uint32_t *pos = nullptr;
    int8_t *cq = nullptr;
    float *cs = nullptr;
    uint32_t bucket = 0, new_rows = 0;
    int pair = -1;                     // element-wise product with segment `pair`'s value
    void *mul_out = nullptr;
    bool skip = false;                 // consumed through another segment's pair; no blocks
    // bf16, element-wise, n % 8 == 0, n <= 8192: also the RmsNorm statistics
    // of each result row, [m][4] floats (the four wave sums of squares of the
    // standalone bf16 RmsNorm kernel, in its order); out and residual must be
    // 16-byte aligned. The normalization itself happens where the row is read
    // (SkinnyNormA).
    float *ssq = nullptr;
};
struct EpiArgs {
    const float *P = nullptr;          // [ks][m][ntot], ks >= 1
    uint32_t m = 0, ks = 0, ntot = 0, nseg = 0;
    bool bf16 = true;
    EpiSeg seg[kSkinnyMaxSeg];
    uint32_t blk_end[kSkinnyMaxSeg] = {};
};
hipError_t launch_epilogue(EpiArgs g, hipStream_t stream);

// gemv_packed.hip — a few-row bf16 group (m <= 16) over weights packed into
// MFMA fragment order (launch_pack_b): every product and its epilogue (the
// EpiSeg fields, except `ssq`: a group that reads A through a fused RmsNorm
// computes the statistics itself) in one launch, a workgroup per 16-column
// tile, SwiGLU tile pair or head. Same bits as the split-K launch and
// launch_epilogue over the same segments.
struct PackedGroup {
    const void *a = nullptr;               // [m, k] bf16, 16-byte aligned
    const uint16_t *gamma = nullptr;       // norm: [k] (null: the identity)
    float eps = 0.0f;
    bool norm = false;                     // A read as RmsNorm(A) (SkinnyNormA's arithmetic)
    uint32_t m = 0, k = 0;
    int nseg = 0;
    uint32_t tw = 16;                      // element-wise tile width (8 or 16): as the weights were packed
    uint32_t tpu = 0;                      // tiles per element-wise workgroup (0: chosen)
    int occupancy = 0;                     // workgroups a CU: 2 for one-tile units, else 1
    const void *bp[kSkinnyMaxSeg] = {};   // B_s [k, n_s] in fragment order
    EpiSeg seg[kSkinnyMaxSeg];
};
bool packed_group_applies(uint32_t m, uint32_t k, const EpiSeg *segs, int nseg, bool norm);
hipError_t launch_packed_group(const PackedGroup &pg, hipStream_t stream);
// B [k, n] row-major bf16 -> fragment order in tiles of tw = 8 or 16 columns
// (k % 32 == 0, n % tw == 0): packed_b_bytes(k, n, tw) (= k * n * 2) bytes at bp.
// rope_d > 0: a rotary-only head-wise segment over heads of rope_d, packed in
// rope tiles (tile column q < 8: head element 8t + q; q >= 8: its rotate-half
// partner), the layout the launch expects for such a segment.
hipError_t launch_pack_b(const void *b, void *bp, uint32_t k, uint32_t n, uint32_t tw, uint32_t rope_d,
                         hipStream_t stream);
uint64_t packed_b_bytes(uint32_t k, uint32_t n, uint32_t tw);
// The tile width a group's weights are packed with.
uint32_t packed_tile_width(uint32_t m, uint32_t k, const EpiSeg *segs, int nseg);

struct SkinnySegment {
    const void *b;
    uint32_t n;
};
// bf16 A read as RmsNorm(A) (feature = k): each element becomes
// ((a * inv) * gamma) narrowed by truncation, inv = 1 / sqrt(sum / k + eps)
// from the four wave sums an epilogue's `ssq` left for the row, the same bits
// the standalone bf16 RmsNorm kernel writes. gamma null: the identity.
struct SkinnyNormA {
    const float *ssq = nullptr;        // [m][4], 16-byte aligned
    const uint16_t *gamma = nullptr;   // [k], 16-byte aligned
    float eps = 0.0f;
};
// Large-M bf16 products sharing A [m, k] (segment s: B_s [k, n_s] into c[s]),
// one launch of the tiled DMA kernel. Applies when each product alone would
// take that kernel (launch_matmul), so each result is bit for bit the single
// call's. res (optional, per segment, null for none): a residual [m, n_s]
// added as MatMulAdd does (product narrowed, added in f32, narrowed; n_s <
// 2^21). Operands 16-byte aligned.
bool matmul_group_tiled_applies(uint32_t m, uint32_t k, const uint32_t *n, int nseg);
hipError_t launch_matmul_group_tiled(const void *a, uint32_t m, uint32_t k,
                                     const SkinnySegment *segs, void *const *c, int nseg,
                                     hipStream_t stream, const void *const *res = nullptr);
// SwiGLU-shaped pair on the tiled kernel: out = f(A*Bg) * (A*Bu), each
// product narrowed to bf16, gate passed through its activation table when
// given (the bf16 unary op's 65536-entry table), the product narrowed again.
// Applies where matmul_group_tiled_applies does for [m, k] x [k, n]; bit for
// bit the two single calls, gate's epilogue and the Mul.
hipError_t launch_matmul_pair_tiled(const void *a, uint32_t m, uint32_t k, const void *b_gate,
                                    const void *b_up, uint32_t n, void *out,
                                    const uint16_t *lut_gate, hipStream_t stream);
hipError_t launch_skinny_partials(const void *a, uint32_t m, uint32_t k, uint8_t dtype,
                                  const SkinnySegment *segs, int nseg, const SkinnyPlan &plan,
                                  float *P, hipStream_t stream, const SkinnyNormA *norm = nullptr);

}  // namespace holo
