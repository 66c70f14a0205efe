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
// kv.hip — int8 quantize + ring append into (cache_q, cache_s) in place.
hipError_t launch_kv_quant_append(const void *nw, uint8_t dtype, const uint32_t *pos,
                                  int8_t *cache_q, float *cache_s, uint32_t planes,
                                  uint32_t bucket, uint32_t new_rows, uint32_t head_dim,
                                  hipStream_t stream);

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
};
size_t attn_i8_scratch_bytes(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t bucket, uint32_t D);
bool attn_i8_supported(uint32_t H, uint32_t Hkv, uint32_t D, uint32_t bucket);
hipError_t launch_attn_i8(const AttnI8Args &a, void *scratch, hipStream_t stream);

// decoder_ops.hip — the other ops of a decode step (bf16 or f32 operands).
// op 0 = Add, 1 = Mul.
hipError_t launch_binary(int op, const void *a, const void *b, void *out, uint64_t n, bool bf16,
                         hipStream_t stream);
// gamma == nullptr: no affine scale.
hipError_t launch_rmsnorm(const void *x, const void *gamma, void *out, uint32_t batch,
                          uint32_t feature, float eps, bool bf16, hipStream_t stream);
hipError_t launch_rope(const void *x, const void *cs, const void *sn, void *out, uint32_t head_dim,
                       uint64_t n, bool bf16, hipStream_t stream);
// Row gather; an out-of-range index zeroes its row and sets *err (device int).
hipError_t launch_gather(const void *data, const void *idx, void *out, uint64_t outer,
                         uint64_t axis_dim, uint64_t num_idx, uint64_t row_bytes, bool i64,
                         int *err, hipStream_t stream);
hipError_t launch_argmax(const void *in, int32_t *out, uint32_t rows, uint32_t cols, bool bf16,
                         hipStream_t stream);

// gemm.hip — C = A*B row-major, fp32 accumulation. dtype f32 or bf16 (bf16
// result narrowed by truncation). `scratch` holds split-K partials of the
// few-row path, matmul_scratch_bytes() bytes (0: none needed). Calls sharing
// one scratch must not overlap.
size_t matmul_scratch_bytes(uint32_t m, uint32_t k, uint32_t n, uint8_t dtype);
hipError_t launch_matmul(const void *a, const void *b, void *c, uint32_t m, uint32_t k,
                         uint32_t n, uint8_t dtype, void *scratch, hipStream_t stream);

// gemm_skinny.hip — the few-row (m <= 64) path that launch_matmul takes when
// it applies (16-byte aligned operands required by the caller).
bool matmul_skinny_applies(uint32_t m, uint32_t k, uint32_t n, uint8_t dtype);
size_t matmul_skinny_scratch_bytes(uint32_t m, uint32_t k, uint32_t n, uint8_t dtype);
hipError_t launch_matmul_skinny(const void *a, const void *b, void *c, uint32_t m, uint32_t k,
                                uint32_t n, uint8_t dtype, void *scratch, hipStream_t stream);

}  // namespace holo
