// quant.hip — the quantized-weight ops: Dequantize (src/cpu/kernels.rs:185-296),
// DequantActivation (:311-388) and MatMulDequant's output-major W8A8 GEMM
// (matmul_i8_pc_omajor / matmul_i4_pc_omajor / matmul_e8cb_omajor,
// src/cpu/simd.rs:5295-5480, 6172-6230, 6867-6950).
//
// The W8A8 GEMM is exact integer arithmetic, so any tiling gives the
// reference's bits: each activation row is quantized once (quantize_row_i8,
// the same operations as the KV quantizer), the dot products accumulate in
// int32 on v_mfma_i32_16x16x64_i8 (four wavefronts split K and add their
// int32 tiles), and the writeback is the reference's expression,
// (acc as f32) * (scale_a * scales[j]).
//
// Layout of the GEMM: a workgroup owns 16 output columns and MT 16-row tiles
// of A. The output-major weight keeps each column's k-vector contiguous, so a
// lane's 16-byte B fragment (k .. k+15 of its column) is one load; lane
// (r, g) of a wavefront holds column r and k-chunk g of each 64-deep step, and
// A row r's chunk g from the quantized rows, so both operands agree on which k
// each byte is. i4 columns unpack 8 bytes to 16 sign-extended levels; e8cb
// columns read two codebook blocks (the 2 KiB codebook staged in LDS).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "holo_device.h"
#include "holo_kernels.h"

namespace holo {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Rust's `f32 as i32`, then clamp(-127, 127) (NaN -> 0), as the KV quantizer.
__device__ __forceinline__ int8_t to_q8(float r) {
    if (r != r) return 0;
    r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
    return static_cast<int8_t>(static_cast<int32_t>(r));
}

// ---------------------------------------------------------- per-token quant --
// One workgroup per row of A (f32): amax with `>` (NaN never wins), then
// q = clamp(round-half-away(x * (127 / amax))), scale amax / 127 (0 for an
// all-zero row, whose q is 0). Row stride kpad >= k; the padding is zeroed so
// the GEMM's whole 64-deep steps read zeros there.
__global__ __launch_bounds__(256) void quant_rows_kernel(const float *__restrict__ a, uint32_t k,
                                                         uint32_t kpad, int8_t *__restrict__ q,
                                                         float *__restrict__ sa) {
    __shared__ float red[4];
    const uint64_t row = blockIdx.x;
    const float *x = a + row * k;
    float amax = 0.0f;
    for (uint32_t c = threadIdx.x; c < k; c += 256) {
        const float v = x[c];
        const float av = v < 0.0f ? -v : v;
        if (av > amax) amax = av;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(amax, off, 64);
        if (o > amax) amax = o;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = red[0];
    for (int w = 1; w < 4; ++w)
        if (red[w] > amax) amax = red[w];
    int8_t *dst = q + row * kpad;
    if (amax == 0.0f) {
        for (uint32_t c = threadIdx.x; c < kpad; c += 256) dst[c] = 0;
        if (threadIdx.x == 0) sa[row] = 0.0f;
        return;
    }
    const float inv = 127.0f / amax;
    for (uint32_t c = threadIdx.x; c < kpad; c += 256) {
        if (c < k) {
            const float t = x[c] * inv;
            dst[c] = to_q8(t >= 0.0f ? truncf(t + 0.5f) : truncf(t - 0.5f));
        } else {
            dst[c] = 0;
        }
    }
    if (threadIdx.x == 0) sa[row] = amax / 127.0f;
}

// ------------------------------------------------------------- W8A8 GEMM ----
struct QGemm {
    const int8_t *q;          // [m][kpad] quantized activation rows
    const float *sa;          // [m] their scales
    const uint8_t *bq;        // output-major weight (tier layout)
    const int8_t *codebook;   // e8cb: 256 x 8
    const float *scales;      // [n] per-column scales
    const float *residual;    // [m][n] or null
    float *out;               // [m][n]
    uint32_t m, k, n, kpad;
    uint32_t act;             // fused_activation id (0: none)
};

// 16 consecutive k of column j starting at k0 (a multiple of 16) as 16 int8
// levels, zero past k or past the last column.
template <int TIER>
__device__ __forceinline__ i32x4 b_fragment(const QGemm &g, const int8_t *cb, uint32_t j,
                                            uint32_t k0) {
    i32x4 r = {0, 0, 0, 0};
    if (j >= g.n || k0 >= g.k) return r;
    const uint32_t k = g.k;
    if constexpr (TIER == 2) {   // i8: bytes j*k + k0 ..
        const uint8_t *p = g.bq + uint64_t(j) * k + k0;
        if (k0 + 16 <= k && ((reinterpret_cast<uintptr_t>(p) & 15) == 0)) {
            const u32x4 v = *reinterpret_cast<const u32x4 *>(p);
            r = i32x4{int32_t(v[0]), int32_t(v[1]), int32_t(v[2]), int32_t(v[3])};
        } else {
            uint32_t w[4] = {0, 0, 0, 0};
            for (int e = 0; e < 16; ++e)
                if (k0 + e < k) w[e >> 2] |= uint32_t(p[e]) << (8 * (e & 3));
            r = i32x4{int32_t(w[0]), int32_t(w[1]), int32_t(w[2]), int32_t(w[3])};
        }
    } else if constexpr (TIER == 10) {   // i4: unit u = j*k + kk, low nibble first
        const uint64_t u0 = uint64_t(j) * k + k0;   // even (k even, k0 % 16 == 0)
        const uint8_t *p = g.bq + (u0 >> 1);
        uint32_t w[4] = {0, 0, 0, 0};
        for (int e = 0; e < 8; ++e) {
            if (k0 + 2 * e >= k) break;
            const uint32_t byte = p[e];
            const int32_t lo = int32_t(byte & 0x0Fu), hi = int32_t(byte >> 4);
            const uint32_t l8 = uint32_t(uint8_t(int8_t(lo >= 8 ? lo - 16 : lo)));
            const uint32_t h8 = uint32_t(uint8_t(int8_t(hi >= 8 ? hi - 16 : hi)));
            w[(2 * e) >> 2] |= l8 << (8 * ((2 * e) & 3));
            w[(2 * e + 1) >> 2] |= h8 << (8 * ((2 * e + 1) & 3));
        }
        r = i32x4{int32_t(w[0]), int32_t(w[1]), int32_t(w[2]), int32_t(w[3])};
    } else {   // e8cb: two 8-row groups, codebook blocks of 8 i8
        const uint8_t *p = g.bq + uint64_t(j) * (k / 8) + k0 / 8;
        uint32_t w[4] = {0, 0, 0, 0};
        for (int h = 0; h < 2; ++h) {
            if (k0 + 8 * h >= k) break;
            const int8_t *blk = cb + uint32_t(p[h]) * 8;
            for (int e = 0; e < 8; ++e) w[2 * h + (e >> 2)] |= uint32_t(uint8_t(blk[e])) << (8 * (e & 3));
        }
        r = i32x4{int32_t(w[0]), int32_t(w[1]), int32_t(w[2]), int32_t(w[3])};
    }
    return r;
}

template <int TIER, int MT>
__global__ __launch_bounds__(256) void gemm_q_omajor_kernel(QGemm g) {
    __shared__ int8_t cb[TIER == 11 ? 256 * 8 : 16];
    __shared__ i32x4 red[3][MT][64];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r = lane & 15, gq = lane >> 4;
    if constexpr (TIER == 11) {
        for (int i = tid; i < 256 * 8; i += 256) cb[i] = g.codebook[i];
        __syncthreads();
    }
    const uint32_t n0 = blockIdx.x * 16, m0 = blockIdx.y * 16 * MT;
    const uint32_t steps = g.kpad / 64;
    const uint32_t per = (steps + 3) / 4;
    const uint32_t s0 = per * wave, s1 = s0 + per < steps ? s0 + per : steps;
    i32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = i32x4{0, 0, 0, 0};
    for (uint32_t s = s0; s < s1; ++s) {
        const uint32_t k0 = s * 64 + 16 * gq;
        const i32x4 bf = b_fragment<TIER>(g, cb, n0 + r, k0);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const uint32_t row = m0 + 16 * t + r;
            i32x4 af = {0, 0, 0, 0};
            if (row < g.m) {
                const u32x4 v = *reinterpret_cast<const u32x4 *>(g.q + uint64_t(row) * g.kpad + k0);
                af = i32x4{int32_t(v[0]), int32_t(v[1]), int32_t(v[2]), int32_t(v[3])};
            }
            acc[t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf, acc[t], 0, 0, 0);
        }
    }
    // the four wavefronts' int32 tiles (exact, so any order)
    if (wave > 0)
#pragma unroll
        for (int t = 0; t < MT; ++t) red[wave - 1][t][lane] = acc[t];
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        i32x4 v = acc[t];
        for (int w = 0; w < 3; ++w) v += red[w][t][lane];
        // C layout of the 16x16 tile: lane holds rows 4*(lane/16) + e, column lane % 16
        const uint32_t j = n0 + r;
        if (j >= g.n) continue;
        const float sj = g.scales[j];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t i = m0 + 16 * t + 4 * gq + e;
            if (i >= g.m) continue;
            const float si = g.sa[i];
            float o = si == 0.0f ? 0.0f : float(v[e]) * (si * sj);
            if (g.residual) o = o + g.residual[uint64_t(i) * g.n + j];
            if (g.act) o = act_f32_call(g.act, o);
            g.out[uint64_t(i) * g.n + j] = o;
        }
    }
}

// ----------------------------------------------------- W8A8 decode GEMV ----
// Few rows (m <= 4): the dot products on v_dot4c_i32_i8 instead of MFMA, so
// the weight stream is fully coalesced: a wavefront owns kGemvCols columns
// and its 64 lanes sweep each column's k-vector in consecutive chunks (lane
// l takes chunks l, l + 64, ...), one 16-byte (e8cb: 8-byte) load per column
// per chunk; the int32 sums are exact, so the order of the lanes' partial sums
// and of the cross-lane reduction does not matter. Chunks: i8 16 levels
// (16 bytes), i4 32 levels (16 bytes: word t holds levels 8t .. 8t+7, even
// levels in the low nibbles), e8cb 64 levels (8 codebook indices).
constexpr int kGemvCols = 8;
// Workgroups of the GEMV: each loops over column blocks (4 waves x kGemvCols
// columns) with a grid stride, so the e8cb codebook is staged once per
// workgroup and every wavefront streams several blocks.
constexpr uint32_t kGemvGrid = 2048;

// Reduce-scatter of N int32 values (N a power of two, <= 64) over the 64
// lanes: each xor step halves the values a lane holds (it keeps the half its
// lane bit selects and adds its partner's copy of that half), then plain xor
// sums finish the strides left. Lane l ends with the wavefront's total of
// value `index` (the bits the halving steps selected); integer sums are exact,
// so the result is the plain total.
template <int N, int S>
struct Scatter {
    static __device__ __forceinline__ void run(int32_t *v, int lane, int &index) {
        constexpr int H = N / 2;
        const bool up = (lane & S) != 0;
#pragma unroll
        for (int i = 0; i < H; ++i) {
            const int32_t send = up ? v[i] : v[i + H];
            const int32_t recv = __shfl_xor(send, S, 64);
            v[i] = (up ? v[i + H] : v[i]) + recv;
        }
        if (up) index += H;
        Scatter<H, S / 2>::run(v, lane, index);
    }
};
template <int S>
struct Scatter<1, S> {
    static __device__ __forceinline__ void run(int32_t *v, int lane, int &index) {
        v[0] += __shfl_xor(v[0], S, 64);
        Scatter<1, S / 2>::run(v, lane, index);
    }
};
template <>
struct Scatter<1, 0> {
    static __device__ __forceinline__ void run(int32_t *, int, int &) {}
};

template <int TIER>
struct GemvChunk {
    static constexpr uint32_t elems = TIER == 2 ? 16 : (TIER == 10 ? 32 : 64);
    static constexpr uint32_t bytes = TIER == 11 ? 8 : 16;
};

template <int TIER, int M>
__global__ __launch_bounds__(256) void gemv_q_omajor_kernel(QGemm g) {
    using Ch = GemvChunk<TIER>;
    __shared__ __attribute__((aligned(16))) int8_t cbb[TIER == 11 ? 256 * 8 : 16];
    if constexpr (TIER == 11) {
        for (int i = threadIdx.x; i < 256 * 8; i += 256) cbb[i] = g.codebook[i];
        __syncthreads();
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t nchunk = g.k / Ch::elems;
    const uint64_t col_bytes = uint64_t(g.k) * Ch::bytes / Ch::elems;
    const uint32_t nblk = (g.n + 4 * kGemvCols - 1) / (4 * kGemvCols);
    for (uint32_t blk = blockIdx.x; blk < nblk; blk += gridDim.x) {
    const uint32_t j0 = (blk * 4 + wave) * kGemvCols;
    int32_t acc[M][kGemvCols];
    int32_t corr[M];   // i4: the sum of the activation levels (the nibble bias)
#pragma unroll
    for (int r = 0; r < M; ++r) {
        corr[r] = 0;
#pragma unroll
        for (int c = 0; c < kGemvCols; ++c) acc[r][c] = 0;
    }
    for (uint32_t ch = lane; ch < nchunk; ch += 64) {
        // every column's chunk first, so the loads are in flight together
        u32x4 w[kGemvCols];
        uint64_t wi[kGemvCols];
#pragma unroll
        for (int c = 0; c < kGemvCols; ++c) {
            const uint32_t j = j0 + c < g.n ? j0 + c : g.n - 1;   // a clamped column is never stored
            const uint8_t *p = g.bq + uint64_t(j) * col_bytes + uint64_t(ch) * Ch::bytes;
            if constexpr (TIER == 11) wi[c] = *reinterpret_cast<const uint64_t *>(p);
            else w[c] = ld_stream(reinterpret_cast<const u32x4 *>(p));
        }
#pragma unroll
        for (int r = 0; r < M; ++r) {
            const u32x4 *qa = reinterpret_cast<const u32x4 *>(g.q + uint64_t(r) * g.kpad +
                                                             uint64_t(ch) * Ch::elems);
            if constexpr (TIER == 2) {
                const u32x4 x = qa[0];
#pragma unroll
                for (int c = 0; c < kGemvCols; ++c)
#pragma unroll
                    for (int t = 0; t < 4; ++t)
                        acc[r][c] = __builtin_amdgcn_sdot4(int(x[t]), int(w[c][t]), acc[r][c], false);
            } else if constexpr (TIER == 10) {
                const u32x4 x0 = qa[0], x1 = qa[1];
                const uint32_t xa[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    // levels 8t .. 8t+7: even ones (low nibbles) and odd ones (high)
                    const uint32_t lo = __builtin_amdgcn_perm(xa[2 * t + 1], xa[2 * t], 0x06040200u);
                    const uint32_t hi = __builtin_amdgcn_perm(xa[2 * t + 1], xa[2 * t], 0x07050301u);
                    corr[r] = __builtin_amdgcn_sdot4(int(xa[2 * t]), 0x01010101, corr[r], false);
                    corr[r] = __builtin_amdgcn_sdot4(int(xa[2 * t + 1]), 0x01010101, corr[r], false);
#pragma unroll
                    for (int c = 0; c < kGemvCols; ++c) {
                        // a nibble u, as (u ^ 8) in 0..15: its signed level is (u ^ 8) - 8
                        const uint32_t b = w[c][t] ^ 0x88888888u;
                        acc[r][c] = __builtin_amdgcn_sdot4(int(lo), int(b & 0x0F0F0F0Fu), acc[r][c], false);
                        acc[r][c] = __builtin_amdgcn_sdot4(int(hi), int((b >> 4) & 0x0F0F0F0Fu), acc[r][c],
                                                           false);
                    }
                }
            } else {
                const u32x4 x0 = qa[0], x1 = qa[1], x2 = qa[2], x3 = qa[3];
                const uint32_t xa[16] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3],
                                         x2[0], x2[1], x2[2], x2[3], x3[0], x3[1], x3[2], x3[3]};
#pragma unroll
                for (int c = 0; c < kGemvCols; ++c)
#pragma unroll
                    for (int h = 0; h < 8; ++h) {
                        const uint32_t half = h < 4 ? uint32_t(wi[c]) : uint32_t(wi[c] >> 32);
                        const uint32_t idx = (half >> (8 * (h & 3))) & 0xffu;
                        const uint64_t v = *reinterpret_cast<const uint64_t *>(cbb + idx * 8);
                        acc[r][c] = __builtin_amdgcn_sdot4(int(xa[2 * h]), int(uint32_t(v)), acc[r][c], false);
                        acc[r][c] = __builtin_amdgcn_sdot4(int(xa[2 * h + 1]), int(uint32_t(v >> 32)),
                                                           acc[r][c], false);
                    }
            }
        }
    }
    // exact int32 totals over the wavefront (the i4 bias folded in first: the
    // totals are linear in the lanes' sums); M = 3 is padded to four rows
    constexpr int MP = M == 3 ? 4 : M;
    int32_t v[MP * kGemvCols];
#pragma unroll
    for (int r = 0; r < MP; ++r)
#pragma unroll
        for (int c = 0; c < kGemvCols; ++c)
            v[r * kGemvCols + c] = r < M ? (TIER == 10 ? acc[r][c] - 8 * corr[r] : acc[r][c]) : 0;
    int index = 0;
    Scatter<MP * kGemvCols, 32>::run(v, lane, index);
    if ((lane & (64 / (MP * kGemvCols) - 1)) == 0) {
        const int r = index / kGemvCols, c = index % kGemvCols;
        const int32_t tot = v[0];
        const uint32_t j = j0 + c;
        if (uint32_t(r) < g.m && j < g.n) {
            const float si = g.sa[r], sj = g.scales[j];
            float o = si == 0.0f ? 0.0f : float(tot) * (si * sj);
            if (g.residual) o = o + g.residual[uint64_t(r) * g.n + j];
            if (g.act) o = act_f32_call(g.act, o);
            g.out[uint64_t(r) * g.n + j] = o;
        }
    }
    }
}

// ------------------------------------------------------------- Dequantize ----
struct DqArgs {
    const uint8_t *in;
    const float *scales;      // per-channel, or null
    const int32_t *zps;       // per-channel, or null
    void *out;
    uint64_t n;
    uint32_t channels, inner;
    uint8_t quant;            // 2 i8, 1 u8, 10 i4
    uint8_t dtype;            // 8 f32, 7 bf16, 6 f16
    float scale;
    int32_t zp;
};

__device__ __forceinline__ int32_t level_at(const DqArgs &d, uint64_t i) {
    if (d.quant == 2) return int32_t(int8_t(d.in[i]));
    if (d.quant == 1) return int32_t(d.in[i]);
    const uint32_t byte = d.in[i >> 1];
    const int32_t v = int32_t((i & 1) ? (byte >> 4) : (byte & 0x0Fu));
    return v >= 8 ? v - 16 : v;
}

__global__ __launch_bounds__(256) void dequant_kernel(DqArgs d) {
    const uint64_t stride = uint64_t(gridDim.x) * 256;
    for (uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x; i < d.n; i += stride) {
        float s = d.scale;
        int32_t z = d.zp;
        if (d.scales) {
            const uint32_t ch = uint32_t((i / d.inner) % d.channels);
            s = d.scales[ch];
            z = d.zps[ch];
        }
        // (q - zp) in wrapping i32, then `as f32`, then * scale (kernels.rs:270)
        const int32_t qz = int32_t(uint32_t(level_at(d, i)) - uint32_t(z));
        const float v = float(qz) * s;
        if (d.dtype == 8) static_cast<float *>(d.out)[i] = v;
        else if (d.dtype == 7) static_cast<uint16_t *>(d.out)[i] = uint16_t(__float_as_uint(v) >> 16);
        else static_cast<uint16_t *>(d.out)[i] = f32_to_f16_bits(v);
    }
}

// ------------------------------------------------------- DequantActivation --
struct DqActTable {
    float t[256];
};

__global__ __launch_bounds__(256) void dequant_act_kernel(const uint8_t *__restrict__ in,
                                                          float *__restrict__ out, uint64_t n,
                                                          bool i4, DqActTable tab) {
    const uint64_t stride = uint64_t(gridDim.x) * 256;
    for (uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += stride) {
        uint32_t idx;
        if (i4) {
            const uint32_t byte = in[i >> 1];
            idx = (i & 1) ? (byte >> 4) : (byte & 0x0Fu);
        } else {
            idx = in[i];
        }
        out[i] = tab.t[idx];
    }
}

// W8A8 needs symmetric weights: any nonzero zero point raises bit 4 of *err
// (reported at the next synchronize as UnsupportedOp).
// Byte-wise, so the zero points need no alignment: an i32 is zero exactly when
// its four bytes are.
__global__ __launch_bounds__(256) void zp_zero_kernel(const uint8_t *__restrict__ zps, uint64_t bytes,
                                                      int *__restrict__ err) {
    bool bad = false;
    for (uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x; i < bytes; i += uint64_t(gridDim.x) * 256)
        bad = bad || zps[i] != 0;
    if (bad) atomicOr(err, 4);
}

uint32_t grid_for(uint64_t n) {
    const uint64_t b = (n + 255) / 256;
    return uint32_t(b < 4096 ? (b ? b : 1) : 4096);
}

}  // namespace

size_t q_omajor_scratch_bytes(uint32_t m, uint32_t k) {
    const uint64_t kpad = (uint64_t(k) + 63) / 64 * 64;
    return size_t(m) * kpad + size_t(m) * 4 + 256;
}

hipError_t launch_matmul_q_omajor(const QOmajorArgs &a, void *scratch, hipStream_t stream) {
    const uint32_t kpad = (a.k + 63) / 64 * 64;
    int8_t *q = static_cast<int8_t *>(scratch);
    float *sa = reinterpret_cast<float *>(static_cast<uint8_t *>(scratch) +
                                          (uint64_t(a.m) * kpad + 255) / 256 * 256);
    hipLaunchKernelGGL(quant_rows_kernel, dim3(a.m), dim3(256), 0, stream, a.a, a.k, kpad, q, sa);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    QGemm g;
    g.q = q;
    g.sa = sa;
    g.bq = static_cast<const uint8_t *>(a.bq);
    g.codebook = a.codebook;
    g.scales = a.scales;
    g.residual = a.residual;
    g.out = a.out;
    g.m = a.m;
    g.k = a.k;
    g.n = a.n;
    g.kpad = kpad;
    g.act = a.act;
    // the decode GEMV when its whole chunks tile k and the loads are aligned
    const uint32_t ce = a.tier == 2 ? 16 : (a.tier == 10 ? 32 : 64);
    const uintptr_t bal = a.tier == 11 ? 7 : 15;
    if (a.m <= 4 && a.k % ce == 0 && (reinterpret_cast<uintptr_t>(a.bq) & bal) == 0) {
        const uint32_t nblk = (a.n + 4 * kGemvCols - 1) / (4 * kGemvCols);
        const dim3 gg(nblk < kGemvGrid ? nblk : kGemvGrid);
#define HOLO_QV(T, M) hipLaunchKernelGGL((gemv_q_omajor_kernel<T, M>), gg, dim3(256), 0, stream, g)
#define HOLO_QVM(T)                         \
    do {                                    \
        switch (a.m) {                      \
            case 1: HOLO_QV(T, 1); break;   \
            case 2: HOLO_QV(T, 2); break;   \
            case 3: HOLO_QV(T, 3); break;   \
            default: HOLO_QV(T, 4); break;  \
        }                                   \
    } while (0)
        switch (a.tier) {
            case 2: HOLO_QVM(2); break;
            case 10: HOLO_QVM(10); break;
            case 11: HOLO_QVM(11); break;
            default: return hipErrorInvalidValue;
        }
#undef HOLO_QVM
#undef HOLO_QV
        return hipGetLastError();
    }
    const bool tall = a.m > 16;
    const dim3 grid((a.n + 15) / 16, tall ? (a.m + 63) / 64 : 1);
#define HOLO_QG(T)                                                                            \
    do {                                                                                      \
        if (tall) hipLaunchKernelGGL((gemm_q_omajor_kernel<T, 4>), grid, dim3(256), 0, stream, g); \
        else hipLaunchKernelGGL((gemm_q_omajor_kernel<T, 1>), grid, dim3(256), 0, stream, g); \
    } while (0)
    switch (a.tier) {
        case 2: HOLO_QG(2); break;
        case 10: HOLO_QG(10); break;
        case 11: HOLO_QG(11); break;
        default: return hipErrorInvalidValue;
    }
#undef HOLO_QG
    return hipGetLastError();
}

hipError_t launch_zero_points_check(const void *zps, uint64_t count, int *err, hipStream_t stream) {
    if (count == 0) return hipSuccess;
    const uint64_t bytes = count * 4;
    hipLaunchKernelGGL(zp_zero_kernel, dim3(grid_for(bytes)), dim3(256), 0, stream,
                       static_cast<const uint8_t *>(zps), bytes, err);
    return hipGetLastError();
}

hipError_t launch_dequantize(const DequantArgs &a, hipStream_t stream) {
    if (a.n == 0) return hipSuccess;
    DqArgs d;
    d.in = static_cast<const uint8_t *>(a.in);
    d.scales = a.scales;
    d.zps = a.zps;
    d.out = a.out;
    d.n = a.n;
    d.channels = a.channels;
    d.inner = a.inner ? a.inner : 1;
    d.quant = a.quant;
    d.dtype = a.dtype;
    d.scale = a.scale;
    d.zp = a.zp;
    hipLaunchKernelGGL(dequant_kernel, dim3(grid_for(a.n)), dim3(256), 0, stream, d);
    return hipGetLastError();
}

hipError_t launch_dequant_act(const uint8_t *in, float *out, uint64_t n, bool i4,
                              const float table[256], hipStream_t stream) {
    if (n == 0) return hipSuccess;
    DqActTable t;
    for (int i = 0; i < 256; ++i) t.t[i] = table[i];
    hipLaunchKernelGGL(dequant_act_kernel, dim3(grid_for(n)), dim3(256), 0, stream, in, out, n, i4,
                       t);
    return hipGetLastError();
}

}  // namespace holo
