// attn.hip — single-token GQA decode attention over int8 K/V caches.
//
// Semantics: for sequence b and query head h (kv head kh = h / G), the visible
// keys are rows [0, L_b) with L_b = min(lens[b], bucket) of plane (b, kh);
//   s_j = dot(q, k_j * kscale_j) / scale,  p = softmax(s),  out = sum_j p_j v_j * vscale_j
// which is the reference's DecodeAttentionValid row
// (crates/hologram-compute/src/cpu/float_kernels.rs:3834-3883) over the
// dequantized rows (kernels.rs:270). Softmax is fp32 (exp2 of log2e-scaled
// scores, online); no key with j >= L_b contributes.
//
// Work split (balanced form, the default): the planes' keys, in 128-key quads,
// are laid end to end and cut into as many equal shares as the GPU holds
// workgroups at once, so a ragged batch (lengths 512..32768) runs as a single
// round with every workgroup streaming the same number of bytes. A share may
// end inside a plane or span several; each (plane, share) segment leaves a
// partial (m, l, O[D]) per head unless it is the whole plane, and
// attn_merge_kernel merges a plane's partials in a fixed order. The quad
// offsets are scanned from `lens` on the device, so a decode step never waits
// on the host. Batches beyond the scan's LDS use the grid form: one workgroup
// per 2048-key chunk of each plane, merged by attn_combine_kernel.
//
// Inside a segment (attn_segment), four wavefronts own all G <= 16 query heads
// of the group, so each K/V byte is read from HBM once. Each wavefront takes
// every 4th 32-key block:
//     S^T[32 keys x 16 heads] = K . Q^T   v_mfma_i32_16x16x64_i8 on the raw K
//                                         bytes; Q as exact int8 hi/lo halves
//     online softmax over the block       fp32, per head = per lane column
//     O^T[D x 16] += V^T . P^T            v_mfma_f32_16x16x32_f16; P^T is
//                                         exactly the lane's own 8 scores, V^T
//                                         is gathered byte-transposed from 8
//                                         key rows
// and the four wavefront states merge in LDS. (Merging across workgroups is a
// second kernel: the kernel boundary makes every partial visible across the
// XCDs' separate L2s; a same-kernel merge would need agent-scope fences per
// workgroup, which write back and invalidate L2.)
//
// Exactness: Q is scaled by a power of two per head so its largest |q| sits in
// [2^13, 2^14), rounded to an integer q_s (relative error <= 2^-14 of the
// head's max) and split q_s = 256 qh + ql with int8 halves, so the int32 QK
// dot products are exact. For PV, an int8 v is the f16 1152 + (v ^ 0x80) - 1152
// built by byte placement under the f16 exponent of 1024 (every integer
// -128..127 is an exact f16); P' = p * vscale / 2^ve with 2^ve
// >= every vscale seen so far keeps P' in [0, 1] (ve is tracked per 512-key
// super-block and the accumulator rescaled when it grows). MFMA products are
// exact and accumulate in fp32.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>

#include "epilogue_math.h"
#include "holo_device.h"
#include "holo_kernels.h"

namespace holo {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// Wavefronts per SIMD the registers are budgeted for. Two (about 176 VGPRs,
// 512 workgroups in the balanced form) run config 4's decode attention 5-7%
// faster than three (168 VGPRs, 768 workgroups): 133k vs 125-127k tok/s.
constexpr int kWps = 2;
constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kBlock = 32;     // keys per wavefront step
constexpr uint32_t kQuad = kWaves * kBlock;   // keys per pass of the four wavefronts
constexpr float kLog2e = 1.4426950408889634f;

typedef int i32x4 __attribute__((ext_vector_type(4)));

// A workgroup barrier over LDS only: each wave waits for its own LDS accesses
// (lgkmcnt 0), then s_barrier, without __syncthreads' release fence, which
// would also wait for every load in flight (the prefetched key blocks).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));   // lgkmcnt(0); vmcnt, expcnt untouched
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// V^T operand of the PV MFMA: dim t of the lane's 4-byte segment, for the
// lane's 8 keys (words w[0..7], bytes already xor 0x80), as 8 exact f16.
// Two byte permutes interleave a key pair, two more place each byte under the
// f16 exponent of 1024 (0x64xx = 1024 + byte), and one packed subtract of
// 1152 leaves the signed int8 value.
__device__ __forceinline__ void pair_dims(uint32_t a, uint32_t b, uint32_t *f4) {
    const uint32_t kMagic = 0x64646464u;
    const uint32_t x01 = __builtin_amdgcn_perm(b, a, 0x05010400u);   // a0 b0 a1 b1
    const uint32_t x23 = __builtin_amdgcn_perm(b, a, 0x07030602u);   // a2 b2 a3 b3
    f4[0] = __builtin_amdgcn_perm(kMagic, x01, 0x04010400u);         // a0 64 b0 64
    f4[1] = __builtin_amdgcn_perm(kMagic, x01, 0x04030402u);         // a1 64 b1 64
    f4[2] = __builtin_amdgcn_perm(kMagic, x23, 0x04010400u);
    f4[3] = __builtin_amdgcn_perm(kMagic, x23, 0x04030402u);
}

__device__ __forceinline__ f16x8 words_to_f16(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
    u32x4 m;
    m.x = w0;
    m.y = w1;
    m.z = w2;
    m.w = w3;
    return __builtin_bit_cast(f16x8, m) - (f16x8)(_Float16)1152.0f;
}

// A value every lane holds alike, moved to a scalar register.
__device__ __forceinline__ uint32_t uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, int(bytes), 0x00020000);
}


// The exact zero rows of plane (b, kh): no visible key (pinned_semantics.rs).
template <bool kF32Q>
__device__ __forceinline__ void zero_rows(void *out, uint32_t b, uint32_t kh, uint32_t H,
                                          uint32_t G, uint32_t D, uint32_t tid, uint32_t nthreads) {
    for (uint32_t idx = tid; idx < G * D; idx += nthreads) {
        const uint64_t oi = (uint64_t(b) * H + kh * G) * D + idx;
        if constexpr (kF32Q)
            static_cast<float *>(out)[oi] = 0.0f;
        else
            static_cast<uint16_t *>(out)[oi] = 0;
    }
}

// LDS of one workgroup's segment: the wavefront merge and the super-block
// scale buffers. k-scales are stored pre-multiplied by log2(e)/scale.
// W wavefronts per workgroup (4, or 8 for the grid form over few planes):
// a pass of the wavefronts covers W * 32 keys, a scale super-block four passes.
template <int W>
constexpr uint32_t super_keys() { return 4u * W * kBlock; }

template <int D, int W = kWaves>
struct SegLds {
    float red_m[W][16], red_l[W][16];
    float red_o[W][16][D];
    float sk[2][super_keys<W>()], sv[2][super_keys<W>()];
    float svmax[2][W / 2];
    i32x4 qop[2][D / 64][64];   // Q int8 hi/lo MFMA operands, per lane of a wavefront
    float smul[16];             // 2^-qe per head
};

// One workgroup's share of a plane: keys [c0, c1) of plane (b, kh) with
// c0 a multiple of 128 and c0 < c1 <= L_b, for all G query heads of the group.
// `single`: the range is the whole plane, so the merged state is the answer and
// goes to `out`; otherwise it is a partial (m, l, O[D]) per head at `dst`.
// b, kh, c0, c1 and single must be uniform over the workgroup; every wavefront
// of the workgroup calls this together (it synchronises through LDS).
//
// Per 512-key super-block the workgroup loads the k- and v-scales in one
// 16-byte load per thread (one load ahead, staged through registers into a
// double buffer in LDS), so the scales travel as large requests rather than
// one 128-byte line per block and stream; invisible keys get scale 0. The
// super-block's largest v-scale sets ve, shared by the four wavefronts:
// P' = p * vscale / 2^ve <= 1 is fed to the f16 MFMA, and the softmax state is
// kept in units of 2^-ve (p' = exp2(s - m - ve), l' = sum p').
//
// kPack (prompt rows, whole-plane segments only): the 16 MFMA columns hold
// `prow` consecutive query rows x G heads, column r = row r / G, head r % G,
// each row with its own visible-key limit lim0 + r / G (clamped to
// [0, bucket]); c1 is the largest. Keys past a column's limit score -inf, and
// a column that has seen no visible key yet keeps exact zeros (its rescale
// and weights are guarded); a row with no visible key at all is written as
// zeros.
template <int D, bool kF32Q, bool kPack = false, int W = kWaves>
__device__ __forceinline__ void attn_segment(
    const void *__restrict__ q, const int8_t *__restrict__ kq, const int8_t *__restrict__ vq,
    const float *__restrict__ ks, const float *__restrict__ vs, float *__restrict__ dst,
    void *__restrict__ out, uint32_t b, uint32_t qrow, uint32_t kh, uint32_t c0, uint32_t c1,
    bool single, uint32_t H, uint32_t Hkv, uint32_t G, uint32_t bucket, float log2e_over_scale,
    SegLds<D, W> &lds, uint32_t prow = 1, int64_t lim0 = 0) {
    constexpr uint32_t kQ = W * kBlock;         // keys per pass of the wavefronts
    constexpr uint32_t kS = super_keys<W>();    // keys per scale super-block
    constexpr int kNT = 64 * W;
    constexpr int KB = D / 4;          // K bytes per lane per key row (QK k-slots)
    constexpr int NKS = D / 64;        // i8 MFMA k-steps (64 dims each)
    constexpr int NDB = D / 16;        // 16-row dim blocks of O^T
    constexpr int VW = NDB / 4;        // V u32 words per lane per key row
    constexpr int kVeMin = -100;       // 2^ve floor: keeps l' = sum p' finite
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int r = lane & 15, g = lane >> 4;
    // the wavefront index is uniform: keep block offsets in scalar registers
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    const uint64_t plane = uint64_t(b) * Hkv + kh;
    // One buffer resource per plane: uniform base, 32-bit lane offsets, and
    // hardware range checking (reads past the plane return 0).
    const auto rk = rsrc(kq + plane * bucket * D, bucket * D);
    const auto rv = rsrc(vq + plane * bucket * D, bucket * D);
    const auto rks = rsrc(ks + plane * bucket, bucket * 4);
    const auto rvs = rsrc(vs + plane * bucket, bucket * 4);

    // Per-lane byte offsets inside a 32-key block; the block base is a uniform
    // soffset and the per-row parts are instruction immediates. K rows 16mb + r
    // (KB bytes at KB*g); V rows kappa(g, j) = 16(j/4) + 4g + j%4 (NDB bytes at
    // NDB*r).
    const int koff = r * D + KB * g;
    const int voff = 4 * g * D + NDB * r;

    struct Blk {
        u32x4 k[2][NKS];
        uint32_t v[8][VW];
    };
    // The per-row constants ride in the scalar offset: only koff and voff stay
    // in vector registers across the loop. A block that is not `live` loads
    // nothing: its scalar offset starts at the end of the plane's buffer range,
    // where buffer loads return 0 without a memory access. So no load sits
    // behind a branch, and the compiler keeps an exact count of the loads in
    // flight (a branch around a load makes it wait for all of them at the
    // join, and the prefetched block would be waited for at once). K and V are
    // read once: their loads are non-temporal (cache policy nt), which took
    // config 4 from 0.234 to 0.214 ms (the scales gained nothing from it).
    const int kvs_none = int(bucket * D);
    constexpr int kNt = 2;   // the nt bit of the buffer load's cache policy
    auto load = [&](uint32_t blk, bool live, Blk &o) {
        const int kvs = live ? int(blk * D) : kvs_none;
#pragma unroll
        for (int mb = 0; mb < 2; ++mb)
#pragma unroll
            for (int s = 0; s < NKS; ++s)
                o.k[mb][s] = __builtin_amdgcn_raw_buffer_load_b128(rk, koff, kvs + 16 * mb * D + 16 * s, kNt);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int row = (16 * (j >> 2) + (j & 3)) * D;
            if constexpr (VW == 2) {
                const auto w = __builtin_amdgcn_raw_buffer_load_b64(rv, voff, kvs + row, kNt);
                o.v[j][0] = w[0];
                o.v[j][1] = w[1];
            } else {
                o.v[j][0] = __builtin_amdgcn_raw_buffer_load_b32(rv, voff, kvs + row, kNt);
            }
        }
    };
    // Super-block scales: wavefronts 0-1 load the 512 k-scales, 2-3 the
    // v-scales, four keys per thread.
    const uint32_t nsb = (c1 - c0 + kS - 1) / kS;
    const uint32_t st = uint32_t(tid) & (32u * W - 1u);
    auto load_sc = [&](uint32_t sb) -> u32x4 {   // sb >= nsb loads nothing
        const int so = sb < nsb ? int((c0 + sb * kS) * 4) : int(bucket * 4);
        return wv < W / 2 ? __builtin_amdgcn_raw_buffer_load_b128(rks, int(16 * st), so, 0)
                      : __builtin_amdgcn_raw_buffer_load_b128(rvs, int(16 * st), so, 0);
    };
    auto store_sc = [&](uint32_t sb, u32x4 v) {
        const uint32_t key0 = c0 + sb * kS + 4 * st;
        float f[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) f[t] = key0 + t < c1 ? __uint_as_float(v[t]) : 0.0f;
        if (wv < W / 2) {
            *reinterpret_cast<float4 *>(&lds.sk[sb & 1][4 * st]) =
                float4{f[0] * log2e_over_scale, f[1] * log2e_over_scale,
                       f[2] * log2e_over_scale, f[3] * log2e_over_scale};
        } else {
            *reinterpret_cast<float4 *>(&lds.sv[sb & 1][4 * st]) = float4{f[0], f[1], f[2], f[3]};
            float m = fmaxf(fmaxf(f[0], f[1]), fmaxf(f[2], f[3]));
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
            if (lane == 0) lds.svmax[sb & 1][wv - W / 2] = m;
        }
    };

    // Wavefront 0 turns Q into the MFMA operands (in LDS, shared by the four
    // wavefronts); its loads go out first. Lanes of padding heads (r >= G)
    // read head 0 and zero it.
    if (wv == 0) {
        float qv[KB];
        const uint32_t cols = kPack ? G * prow : G;
        const bool live = uint32_t(r) < cols;
        const uint32_t col = live ? uint32_t(r) : 0u;
        const uint64_t qi = kPack ? ((uint64_t(qrow) + col / G) * H + kh * G + col % G) * D + KB * g
                                  : (uint64_t(qrow) * H + kh * G + col) * D + KB * g;
        if constexpr (kF32Q) {
            const u32x4 *src = reinterpret_cast<const u32x4 *>(static_cast<const float *>(q) + qi);
#pragma unroll
            for (int w = 0; w < KB / 4; ++w) {
                const u32x4 v = src[w];
                qv[4 * w] = __uint_as_float(v.x);
                qv[4 * w + 1] = __uint_as_float(v.y);
                qv[4 * w + 2] = __uint_as_float(v.z);
                qv[4 * w + 3] = __uint_as_float(v.w);
            }
        } else {
            const u32x4 *src = reinterpret_cast<const u32x4 *>(static_cast<const uint16_t *>(q) + qi);
#pragma unroll
            for (int w = 0; w < KB / 8; ++w) {
                const u32x4 v = src[w];
                const uint32_t e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    qv[8 * w + 2 * t] = __uint_as_float(e[t] << 16);
                    qv[8 * w + 2 * t + 1] = __uint_as_float(e[t] & 0xFFFF0000u);
                }
            }
        }
#pragma unroll
        for (int e = 0; e < KB; ++e) qv[e] = live ? qv[e] : 0.0f;
        // Q as a 15-bit integer per head, q * 2^qe with max |.| in [2^13, 2^14),
        // split exactly into int8 halves: q_s = 256 qh + ql, ql in [-128, 127].
        float qmax = 0.0f;
#pragma unroll
        for (int e = 0; e < KB; ++e) qmax = fmaxf(qmax, fabsf(qv[e]));
        qmax = fmaxf(qmax, __shfl_xor(qmax, 16, 64));
        qmax = fmaxf(qmax, __shfl_xor(qmax, 32, 64));
        int qe = 0;
        if (qmax > 0.0f && qmax <= 3.0e38f) {
            (void)frexpf(qmax, &qe);          // qmax < 2^qe
            qe = 14 - qe;
        }
#pragma unroll
        for (int s = 0; s < NKS; ++s) {
            i32x4 qh, ql;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint32_t hw = 0, lw = 0;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int qs = int(rintf(ldexpf(qv[16 * s + 4 * w + t], qe)));
                    const int hi = (qs + 128) >> 8;
                    const int lo = qs - hi * 256;
                    hw |= uint32_t(hi & 0xFF) << (8 * t);
                    lw |= uint32_t(lo & 0xFF) << (8 * t);
                }
                qh[w] = int(hw);
                ql[w] = int(lw);
            }
            lds.qop[0][s][lane] = qh;
            lds.qop[1][s][lane] = ql;
        }
        if (g == 0) lds.smul[r] = ldexpf(1.0f, -qe);   // the k-scales carry log2(e)/scale
    }
    u32x4 sreg = load_sc(0);
    // Wavefront wv takes every fourth 32-key block of the segment, with its
    // next PD - 1 blocks in flight while one is computed: at head_dim 64 a
    // decode step's short contexts give a wavefront only a few blocks, which
    // one block in flight would fetch one latency at a time. The blocks sit in
    // a ring indexed by the block's position in its 4-block super-block pass,
    // a constant once that loop is unrolled, so no register is moved while its
    // load is in flight.
    constexpr int PD = D <= 64 ? 4 : 2;
    Blk ring[PD];
#pragma unroll
    for (int p = 0; p < PD - 1; ++p) {
        const uint32_t bb = c0 + uint32_t(p) * kQ + wv * kBlock;
        load(bb, bb < c1, ring[p]);
    }

    f32x4 acc_o[NDB];
#pragma unroll
    for (int i = 0; i < NDB; ++i) acc_o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_run = 0.0f, mv = -INFINITY;   // mv = m_run + ve
    int ve = kVeMin;

    store_sc(0, sreg);
    lds_barrier();   // Q operands and the first scales; the blocks stay in flight
    const float smul = lds.smul[r];
    // kPack: this lane's column limit, and the smallest limit (blocks ending
    // past it need the per-key test)
    int64_t lim_r = lim0 + int64_t(uint32_t(r) / (G ? G : 1));
    lim_r = lim_r < 0 ? 0 : (lim_r > int64_t(bucket) ? int64_t(bucket) : lim_r);
    const uint32_t lim_lane = kPack ? uint32_t(lim_r) : c1;
    const uint32_t lim_min = kPack ? uint32_t(lim0 < 0 ? 0 : (lim0 > int64_t(bucket) ? int64_t(bucket) : lim0)) : c1;

    // One 32-key block: lane (r, g) holds keys 16mb + 4g + i for head r.
    // masked: keys at or beyond c1 are invisible (the segment's last block;
    // wave-uniform, so the masking is a branch the full blocks skip).
    auto block = [&](bool masked, const Blk &cb, uint32_t blk, const float *skp,
                     const float *svp) __attribute__((always_inline)) {
        float ksc[8], vsc[8];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float4 k4 = *reinterpret_cast<const float4 *>(skp + 16 * h + 4 * g);
            const float4 v4 = *reinterpret_cast<const float4 *>(svp + 16 * h + 4 * g);
            ksc[4 * h] = k4.x; ksc[4 * h + 1] = k4.y; ksc[4 * h + 2] = k4.z; ksc[4 * h + 3] = k4.w;
            vsc[4 * h] = v4.x; vsc[4 * h + 1] = v4.y; vsc[4 * h + 2] = v4.z; vsc[4 * h + 3] = v4.w;
        }
        // -- S^T = K . Q^T on the int8 MFMA, exact in int32
        float sc[8];
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            i32x4 ah = {0, 0, 0, 0}, al = {0, 0, 0, 0};
#pragma unroll
            for (int s = 0; s < NKS; ++s) {
                const i32x4 kf = __builtin_bit_cast(i32x4, cb.k[mb][s]);
                ah = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf, lds.qop[0][s][lane], ah, 0, 0, 0);
                al = __builtin_amdgcn_mfma_i32_16x16x64_i8(kf, lds.qop[1][s][lane], al, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) sc[4 * mb + i] = (float(ah[i] * 256 + al[i]) * ksc[4 * mb + i]) * smul;
        }
        if (masked) {
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (blk + 16 * (j >> 2) + 4 * g + (j & 3) >= lim_lane) sc[j] = -INFINITY;
        }
        float m_blk = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])),
                            fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
        {   // across the four key groups g: lanes r, r+16, r+32, r+48
            const auto x16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(m_blk), __float_as_uint(m_blk), false, false);
            m_blk = fmaxf(__uint_as_float(x16[0]), __uint_as_float(x16[1]));
            const auto x32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(m_blk), __float_as_uint(m_blk), false, false);
            m_blk = fmaxf(__uint_as_float(x32[0]), __uint_as_float(x32[1]));
        }
        if (__any(m_blk > m_run)) {        // rescale only when some head's max grew
            const float m_new = fmaxf(m_run, m_blk);
            // kPack: a column with no visible key so far stays at -inf, exact 0
            const float alpha = kPack && m_new == -INFINITY ? 1.0f : exp2f(m_run - m_new);
            m_run = m_new;
            mv = m_run + float(ve);
            l_run *= alpha;
#pragma unroll
            for (int i = 0; i < NDB; ++i) acc_o[i] *= alpha;
        }
        f16x8 pf;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float p = exp2f(sc[j] - mv);         // p * 2^-ve; masked keys: exp2(-inf) = 0
            if (kPack && sc[j] == -INFINITY) p = 0.0f;
            l_run += p;
            pf[j] = (_Float16)(p * vsc[j]);      // invisible keys carry scale 0
        }
        // -- O^T += V^T . P^T : dim block mb = 4w + t, row m holds dim NDB*m + mb
#pragma unroll
        for (int w = 0; w < VW; ++w) {
            uint32_t f[4][4];   // [dim t][key pair]
#pragma unroll
            for (int pr = 0; pr < 4; ++pr) {
                uint32_t f4[4];
                pair_dims(cb.v[2 * pr][w] ^ 0x80808080u, cb.v[2 * pr + 1][w] ^ 0x80808080u, f4);
#pragma unroll
                for (int t = 0; t < 4; ++t) f[t][pr] = f4[t];
            }
#pragma unroll
            for (int t = 0; t < 4; ++t)
                acc_o[4 * w + t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                    words_to_f16(f[t][0], f[t][1], f[t][2], f[t][3]), pf, acc_o[4 * w + t], 0, 0, 0);
        }
    };

    // Every wavefront walks the same nsb super-blocks of 4 quads (the barriers
    // must match); its block of a quad past c1 is skipped.
    for (uint32_t sb = 0; sb < nsb; ++sb) {
        sreg = load_sc(sb + 1);
        {   // 2^ve bounds every v-scale of this super-block (all wavefronts alike)
            float vb = lds.svmax[sb & 1][0];
#pragma unroll
            for (int i = 1; i < W / 2; ++i) vb = fmaxf(vb, lds.svmax[sb & 1][i]);
            if (vb > ldexpf(1.0f, ve) && vb <= 3.0e38f) {
                int ve_new;
                (void)frexpf(vb, &ve_new);                     // vb < 2^ve_new
                const float shrink = ldexpf(1.0f, ve - ve_new);
                l_run *= shrink;
#pragma unroll
                for (int i = 0; i < NDB; ++i) acc_o[i] *= shrink;
                ve = ve_new;
                mv = m_run + float(ve);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t blk = c0 + (4 * sb + uint32_t(i)) * kQ + wv * kBlock;
            const uint32_t nb = blk + (PD - 1) * kQ;
            load(nb, nb < c1, ring[(i + PD - 1) % PD]);
            if (blk < c1) {
                const uint32_t so = uint32_t(i) * kQ + wv * kBlock;
                const float *skp = lds.sk[sb & 1] + so, *svp = lds.sv[sb & 1] + so;
                block(blk + kBlock > lim_min, ring[i % PD], blk, skp, svp);
            }
        }
        if (sb + 1 < nsb) store_sc(sb + 1, sreg);
        lds_barrier();
    }

    // ---- wavefront state -> LDS, merge the four wavefronts per head
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    if (g == 0) {
        lds.red_m[wave][r] = m_run;
        lds.red_l[wave][r] = l_run;
    }
#pragma unroll
    for (int mb = 0; mb < NDB; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            lds.red_o[wave][r][NDB * (4 * g + i) + mb] = acc_o[mb][i];
    __syncthreads();

    // The whole plane: the merged state is the answer (o / l does not depend on
    // the common 2^ve). Otherwise write the partial, scaled back by 2^ve.
    const float v_rescale = ldexpf(1.0f, ve);
    const uint32_t ncol = kPack ? G * prow : G;
    for (uint32_t idx = tid; idx < ncol * D; idx += kNT) {
        const uint32_t h = idx / D, d = idx % D;
        float m = -INFINITY;
#pragma unroll
        for (int w = 0; w < W; ++w) m = fmaxf(m, lds.red_m[w][h]);
        float o = 0.0f, l = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float sc = lds.red_m[w][h] == -INFINITY ? 0.0f : exp2f(lds.red_m[w][h] - m);
            o = fmaf(lds.red_o[w][h][d], sc, o);
            l = fmaf(lds.red_l[w][h], sc, l);
        }
        if (single) {
            const uint64_t oi = kPack ? ((uint64_t(qrow) + h / G) * H + kh * G + h % G) * D + d
                                      : (uint64_t(qrow) * H + kh * G + h) * D + d;
            const float res = kPack && l == 0.0f ? 0.0f : o / l;   // kPack: a row with no key
            if constexpr (kF32Q)
                static_cast<float *>(out)[oi] = res;
            else
                static_cast<uint16_t *>(out)[oi] = uint16_t(__float_as_uint(res) >> 16);
            continue;
        }
        dst[h * (D + 2) + 2 + d] = o * v_rescale;
        if (d == 0) {
            dst[h * (D + 2)] = m;
            dst[h * (D + 2) + 1] = l * v_rescale;
        }
    }
    __syncthreads();   // the caller may reuse the LDS next
}

// Keys visible to a query row `back` rows before the last of its sequence:
// the sequence's visible length less `back` (none if that is not positive),
// at most the bucket.
__device__ __forceinline__ uint32_t visible_keys(uint32_t len, uint32_t back, uint32_t bucket) {
    const uint32_t L = len > back ? len - back : 0u;
    return L < bucket ? L : bucket;
}

// Grid form for very large batches: grid (chunks, Hkv, B), one workgroup per
// kChunk-key chunk of a plane; chunks at or beyond L_b exit at once, and chunk
// 0 of a plane with no visible key writes the exact zero rows. Partial of
// (plane, chunk) at index plane * nchunks + chunk. W wavefronts a workgroup:
// 8 when the grid is too small to fill the GPU (a decode step's 64 planes of
// one chunk each), so each wavefront walks an eighth of its plane, not a
// quarter.
template <int D, bool kF32Q, int W>
__global__ __launch_bounds__(64 * W, W == kWaves ? kWps : 1) void attn_chunk_kernel(
    const void *__restrict__ q, const int8_t *__restrict__ kq, const int8_t *__restrict__ vq,
    const float *__restrict__ ks, const float *__restrict__ vs, const uint32_t *__restrict__ lens,
    float *__restrict__ part, void *__restrict__ out, uint32_t H, uint32_t Hkv, uint32_t G,
    uint32_t bucket, uint32_t kChunk, uint32_t nchunks, float log2e_over_scale, uint32_t q_rows) {
    __shared__ SegLds<D, W> lds;
    const uint32_t v = blockIdx.z, kh = blockIdx.y, chunk = blockIdx.x;
    const uint32_t b = v / q_rows;
    const uint32_t L = visible_keys(lens[b], q_rows - 1 - v % q_rows, bucket);
    const uint32_t c0 = chunk * kChunk;
    if (c0 >= L) {
        if (L == 0 && chunk == 0) zero_rows<kF32Q>(out, v, kh, H, G, D, threadIdx.x, 64 * W);
        return;
    }
    const uint32_t c1 = L - c0 < kChunk ? L : c0 + kChunk;
    const uint64_t row_plane = uint64_t(v) * Hkv + kh;
    float *dst = part + (row_plane * nchunks + chunk) * G * (D + 2);
    attn_segment<D, kF32Q, false, W>(q, kq, vq, ks, vs, dst, out, b, v, kh, c0, c1, L <= kChunk, H,
                                     Hkv, G, bucket, log2e_over_scale, lds);
}

// The grid form of a decode step (one chunk a plane, one bf16 query row) with
// the q/k/v group's split-K epilogue in front: workgroup (b, kh) first
// finishes, from the partials, every head of the group's head-wise segments
// that belongs to kv head kh of row b (segment s holds n_s / D heads a row,
// n_s / (D Hkv) of them per kv head: its query heads, or its one k or v head),
// storing the rotated q and the appended int8 k / v rows exactly as the
// epilogue launch does (the same head_finish), then attends. A workgroup reads
// back only what it stored itself (its plane's query heads and cache rows),
// after its stores have completed (s_waitcnt) and a workgroup barrier, so no
// other workgroup's order matters.
template <int D, int W>
__global__ __launch_bounds__(64 * W, W == kWaves ? kWps : 1) void attn_pro_kernel(
    const uint16_t *__restrict__ q, const int8_t *__restrict__ kq, const int8_t *__restrict__ vq,
    const float *__restrict__ ks, const float *__restrict__ vs, const uint32_t *__restrict__ lens,
    void *__restrict__ out, uint32_t H, uint32_t Hkv, uint32_t G, uint32_t bucket,
    float log2e_over_scale, const EpiArgs pro) {
    __shared__ SegLds<D, W> lds;
    const uint32_t b = blockIdx.z, kh = blockIdx.y;
    const uint32_t len_b = lens[b];   // read before the prologue: it does not write lens
    {
        constexpr uint32_t half = D / 2, slots = 64 * W / half;
        const uint32_t slot = threadIdx.x / half, d = threadIdx.x % half;
        uint32_t hp[kSkinnyMaxSeg], total = 0;
#pragma unroll
        for (int s = 0; s < kSkinnyMaxSeg; ++s) {
            hp[s] = uint32_t(s) < pro.nseg ? pro.seg[s].n / (D * Hkv) : 0u;
            total += hp[s];
        }
        // a head's D/2 lanes take the same heads (the quantizer's shuffles)
        for (uint32_t t = slot; t < total; t += slots) {
            uint32_t si = 0, first = 0, acc = hp[0];
#pragma unroll
            for (int s = 1; s < kSkinnyMaxSeg; ++s)
                if (t >= acc) {
                    si = uint32_t(s);
                    first = acc;
                    acc += hp[s];
                }
            const EpiSeg sg = epi::seg_of(pro, si);
            epi::head_finish<true>(pro, sg, b, kh * (sg.n / (D * Hkv)) + (t - first), d, true);
        }
        __builtin_amdgcn_s_waitcnt(0);   // every store of this workgroup has completed
        __syncthreads();
    }
    const uint32_t L = visible_keys(len_b, 0, bucket);
    if (L == 0) {
        zero_rows<false>(out, b, kh, H, G, D, threadIdx.x, 64 * W);
        return;
    }
    attn_segment<D, false, false, W>(q, kq, vq, ks, vs, nullptr, out, b, b, kh, 0, L, true, H, Hkv, G,
                                     bucket, log2e_over_scale, lds);
}

// Packed prompt form: grid (1, Hkv, B * ceil(T / R)). A workgroup takes R
// consecutive query rows of one sequence for one kv head (R * G <= 16 MFMA
// columns), so each K/V byte of the plane is read once per R rows. Each plane
// fits one chunk (the whole visible range is one segment; no merge).
template <int D, bool kF32Q>
__global__ __launch_bounds__(kThreads, kWps) void attn_rows_packed_kernel(
    const void *__restrict__ q, const int8_t *__restrict__ kq, const int8_t *__restrict__ vq,
    const float *__restrict__ ks, const float *__restrict__ vs, const uint32_t *__restrict__ lens,
    void *__restrict__ out, uint32_t H, uint32_t Hkv, uint32_t G, uint32_t bucket,
    float log2e_over_scale, uint32_t T, uint32_t R) {
    __shared__ SegLds<D> lds;
    const uint32_t nt = (T + R - 1) / R;
    const uint32_t kh = blockIdx.y, b = blockIdx.z / nt, t0 = (blockIdx.z % nt) * R;
    const uint32_t rows = T - t0 < R ? T - t0 : R;
    const int64_t lim0 = int64_t(lens[b]) - int64_t(T - 1 - t0);    // first packed row
    int64_t last = lim0 + rows - 1;
    last = last < 0 ? 0 : (last > int64_t(bucket) ? int64_t(bucket) : last);
    const uint32_t qrow = b * T + t0;
    if (last == 0) {   // no packed row sees a key: exact zeros
        for (uint32_t ro = 0; ro < rows; ++ro)
            zero_rows<kF32Q>(out, qrow + ro, kh, H, G, D, threadIdx.x, kThreads);
        return;
    }
    attn_segment<D, kF32Q, true>(q, kq, vq, ks, vs, nullptr, out, b, qrow, kh, 0, uint32_t(last),
                                 true, H, Hkv, G, bucket, log2e_over_scale, lds, rows, lim0);
}

// Prompt form for G = 4, D = 64, bf16 rows: grid (ceil(T / 64), Hkv, B).
// A workgroup takes 64 consecutive query rows of one sequence; wave w owns
// query head 4 kh + w. Each 64-key tile of the plane is staged in LDS once for
// all four heads: K as bf16 [key][dim] (int8 values are exact) and V
// transposed as f16 [dim][key] with the key's scale applied (v * vscale, an
// f16 rounding of 2^-11 relative). Per tile and wave:
//     S^T[64 keys x 64 rows] = K . Q^T   v_mfma_f32_32x32x16_bf16
//     scale by kscale * log2e / scale, causal mask per row (only in tiles
//     some row of the block does not fully see), online softmax (fp32, exp2;
//     a row is a lane column, its keys in the lane and the lane 32 apart),
//     p as f16
//     O^T[64 dims x 64 rows] += V'^T . P^T   v_mfma_f32_32x32x16_f16
// A lane's 8 scores of a 16-key step are exactly its B operand when the
// step's keys are taken in the order the S^T layout holds them (rows
// 4 lg + 0..3 and 8 + 4 lg + 0..3 of each 16); V^T is read in that order.
// Row t sees the first clamp(lens[b] - (T - 1 - t), 0, bucket) keys; a row
// that sees none is written as zeros. Later row blocks see more keys; the
// upper half of the workgroups takes the blocks in reverse order, so the two
// workgroups a CU holds at once tend to pair a long block with a short one.
constexpr uint32_t kPT = 64;    // query rows per workgroup, keys per tile
constexpr uint32_t kPLd = 72;   // LDS row stride of the staged tiles (16-bit elements)
typedef __bf16 pbf16x8 __attribute__((ext_vector_type(8)));
typedef float pf32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ uint32_t bf16_of_int(int v) {
    return __float_as_uint(float(v)) >> 16;   // exact: |v| <= 128
}
__device__ __forceinline__ uint32_t f16_of_int(int v) {
    const _Float16 h = _Float16(float(v));
    return __builtin_bit_cast(uint16_t, h);
}

__global__ __launch_bounds__(kThreads, 2) void attn_prompt_kernel(
    const uint16_t *__restrict__ q, const int8_t *__restrict__ kq, const int8_t *__restrict__ vq,
    const float *__restrict__ ks, const float *__restrict__ vs, const uint32_t *__restrict__ lens,
    uint16_t *__restrict__ out, uint32_t H, uint32_t Hkv, uint32_t bucket, float mul, uint32_t T) {
    __shared__ __attribute__((aligned(16))) uint16_t kl[kPT * kPLd];   // K tile, bf16 [key][dim]
    __shared__ __attribute__((aligned(16))) uint16_t vt[kPT * kPLd];   // V tile, f16 [dim][key]
    __shared__ float ksl[kPT];
    const uint32_t nqb = gridDim.x;
    const uint32_t lin = blockIdx.x + nqb * (blockIdx.y + gridDim.y * blockIdx.z);
    const uint32_t xb = 2 * lin >= nqb * gridDim.y * gridDim.z ? nqb - 1 - blockIdx.x : blockIdx.x;
    const uint32_t b = blockIdx.z, kh = blockIdx.y, t0 = xb * kPT;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, lr = lane & 31, lg = lane >> 5;
    const uint32_t h = kh * 4 + wave;
    const uint64_t plane = uint64_t(b) * Hkv + kh;
    const int8_t *kp = kq + plane * bucket * 64, *vp = vq + plane * bucket * 64;
    const float *ksp = ks + plane * bucket, *vsp = vs + plane * bucket;
    const int64_t len = lens[b];
    auto visible = [&](uint32_t t) -> uint32_t {
        const int64_t L = len - int64_t(T - 1 - t);
        return L < 0 ? 0u : (L > int64_t(bucket) ? bucket : uint32_t(L));
    };
    const uint32_t tl = (t0 + kPT < T ? t0 + kPT : T) - 1;   // the block's last row sees most
    const uint32_t kmax = visible(tl);
    const uint32_t kmin = visible(t0);   // ... and its first row least: keys < kmin need no mask

    // this lane's rows t0 + 32 qb + lr: their key limits and Q^T fragments
    // (dims 16 kk + 8 lg .. +7)
    uint32_t lim[2];
    pbf16x8 qf[2][4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const uint32_t t = t0 + 32 * qb + lr;
        lim[qb] = t < T ? visible(t) : 0u;
        const uint16_t *qr = q + ((uint64_t(b) * T + t) * H + h) * 64 + 8 * lg;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            u32x4 v = u32x4{0u, 0u, 0u, 0u};
            if (t < T) v = *reinterpret_cast<const u32x4 *>(qr + 16 * kk);
            qf[qb][kk] = __builtin_bit_cast(pbf16x8, v);
        }
    }
    pf32x16 o[2][2];
#pragma unroll
    for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int r = 0; r < 16; ++r) o[db][qb][r] = 0.0f;
    float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.0f, 0.0f};

    // A tile's K, V and scales come into registers one tile ahead (branch-free
    // buffer loads: a key past the bucket reads zero), so the loads of tile
    // j0 + 64 are in flight while tile j0 is computed. Thread: key tid / 4,
    // dims 16 (tid % 4) .. +15; threads below 64 also take one k-scale.
    const auto rk = rsrc(kp, bucket * 64u), rv = rsrc(vp, bucket * 64u);
    const auto rks = rsrc(ksp, bucket * 4u), rvs = rsrc(vsp, bucket * 4u);
    const uint32_t fkey = uint32_t(tid) >> 2, fd0 = (uint32_t(tid) & 3u) * 16u;
    u32x4 kr, vr;
    float vsc, ksv;
    auto fetch = [&](uint32_t j0) {
        const uint32_t j = j0 + fkey;
        kr = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, j * 64u + fd0, 0, 0));
        vr = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rv, j * 64u + fd0, 0, 0));
        vsc = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rvs, j * 4u, 0, 0));
        ksv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                            rks, tid < int(kPT) ? (j0 + uint32_t(tid)) * 4u : 0x80000000u, 0, 0));
    };
    fetch(0);
    for (uint32_t j0 = 0; j0 < kmax; j0 += kPT) {
        __syncthreads();   // the previous tile's readers are done
        {
            const uint32_t key = fkey, d0 = fd0;
            u32x4 k0, k1;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const uint32_t x = kr[w];
                const uint32_t lo = bf16_of_int(int8_t(x & 0xff)) | (bf16_of_int(int8_t((x >> 8) & 0xff)) << 16);
                const uint32_t hi = bf16_of_int(int8_t((x >> 16) & 0xff)) | (bf16_of_int(int8_t(x >> 24)) << 16);
                if (w < 2) {
                    k0[2 * w] = lo;
                    k0[2 * w + 1] = hi;
                } else {
                    k1[2 * w - 4] = lo;
                    k1[2 * w - 3] = hi;
                }
            }
            *reinterpret_cast<u32x4 *>(kl + key * kPLd + d0) = k0;
            *reinterpret_cast<u32x4 *>(kl + key * kPLd + d0 + 8) = k1;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const _Float16 vh = _Float16(float(int8_t((vr[i / 4] >> (8 * (i % 4))) & 0xff)) * vsc);
                vt[(d0 + i) * kPLd + key] = __builtin_bit_cast(uint16_t, vh);
            }
            if (tid < int(kPT)) ksl[tid] = ksv * mul;
        }
        fetch(j0 + kPT);   // the next tile (past kmax: loads nobody stages)
        __syncthreads();

        // S^T for key blocks kb and row blocks qb
        pf32x16 s[2][2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            pbf16x8 kf[4];
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
                kf[kk] = *reinterpret_cast<const pbf16x8 *>(kl + (32 * kb + lr) * kPLd + 16 * kk + 8 * lg);
#pragma unroll
            for (int qb = 0; qb < 2; ++qb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) s[kb][qb][r] = 0.0f;
#pragma unroll
                for (int kk = 0; kk < 4; ++kk)
                    s[kb][qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[kk], qf[qb][kk], s[kb][qb], 0, 0, 0);
            }
        }
        // scale, mask, online softmax; s becomes p
        float ksc[2][16];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) ksc[kb][r] = ksl[32 * kb + 8 * (r >> 2) + 4 * lg + (r & 3)];
        const bool full = j0 + kPT <= kmin;   // every row of the block sees the whole tile
#pragma unroll
        for (int qb = 0; qb < 2; ++qb) {
            float mt = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const uint32_t kt = 32 * kb + 8 * (r >> 2) + 4 * lg + (r & 3);
                    float x = s[kb][qb][r] * ksc[kb][r];
                    if (!full) x = j0 + kt < lim[qb] ? x : -INFINITY;
                    s[kb][qb][r] = x;
                    mt = x > mt ? x : mt;
                }
            const float mo = __shfl_xor(mt, 32, 64);
            mt = mo > mt ? mo : mt;
            const float mn = m[qb] > mt ? m[qb] : mt;
            // v_exp_f32 directly: it differs from exp2f only below 2^-126
            const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m[qb] - mn);
            const float mref = mn == -INFINITY ? 0.0f : mn;   // all masked: exp2(-inf) = 0
            float rs = 0.0f;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float p = __builtin_amdgcn_exp2f(s[kb][qb][r] - mref);
                    rs += p;
                    s[kb][qb][r] = p;
                }
            rs += __shfl_xor(rs, 32, 64);
            l[qb] = l[qb] * alpha + rs;
            m[qb] = mn;
#pragma unroll
            for (int db = 0; db < 2; ++db) o[db][qb] *= alpha;
        }
        // O^T += V^T . P'^T over four 16-key steps
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const int kb = st >> 1, hh = st & 1;
            f16x8 pf[2];
#pragma unroll
            for (int qb = 0; qb < 2; ++qb)
#pragma unroll
                for (int i = 0; i < 8; ++i) pf[qb][i] = _Float16(s[kb][qb][8 * hh + i]);
#pragma unroll
            for (int db = 0; db < 2; ++db) {
                const uint16_t *vrow = vt + (32 * db + lr) * kPLd + 32 * kb + 16 * hh + 4 * lg;
                const uint2 lo = *reinterpret_cast<const uint2 *>(vrow);
                const uint2 hi = *reinterpret_cast<const uint2 *>(vrow + 8);
                const u32x4 w = u32x4{lo.x, lo.y, hi.x, hi.y};
                const f16x8 vf = __builtin_bit_cast(f16x8, w);
#pragma unroll
                for (int qb = 0; qb < 2; ++qb)
                    o[db][qb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf, pf[qb], o[db][qb], 0, 0, 0);
            }
        }
    }
    // O^T: lane holds dims 32 db + 8 (r/4) + 4 lg + r%4 of row t0 + 32 qb + lr
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        const uint32_t t = t0 + 32 * qb + lr;
        if (t >= T) continue;
        const float inv = l[qb] > 0.0f ? 1.0f / l[qb] : 0.0f;
        uint16_t *orow = out + ((uint64_t(b) * T + t) * H + h) * 64;
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int r = 0; r < 16; ++r)
                orow[32 * db + 8 * (r >> 2) + 4 * lg + (r & 3)] =
                    uint16_t(__float_as_uint(o[db][qb][r] * inv) >> 16);
    }
}

// Balanced form: the planes' 128-key quads laid end to end, plane (b, kh) in
// (b, kh) order, and cut into `P` equal shares, one per workgroup (P is the
// number of workgroups the GPU holds at once, so the whole batch is one round
// with no tail). Each workgroup first scans ceil(L_b / 128) into quad offsets
// (in LDS; workgroup 0 also stores them for the merge), then walks the planes
// its share touches. Segment (plane p, workgroup w) has partial index p + w,
// which is unique because along the quad line either p or w grows at every
// segment boundary; a plane's partials are contiguous. Shares are at least
// kMinQuads quads, so a small batch uses fewer workgroups.
constexpr uint32_t kScanMax = 1024;   // sequences the balanced form scans in LDS
constexpr uint32_t kMinQuads = 4;
constexpr uint32_t kMaxSplit = 1024;  // workgroups of the balanced form

__device__ __forceinline__ uint32_t split_count(uint64_t quads, uint32_t P) {
    const uint64_t cap = (quads + kMinQuads - 1) / kMinQuads;
    return uint32_t(cap < P ? (cap ? cap : 1) : P);
}

template <int D, bool kF32Q>
__global__ __launch_bounds__(kThreads, kWps) void attn_split_kernel(
    const void *__restrict__ q, const int8_t *__restrict__ kq, const int8_t *__restrict__ vq,
    const float *__restrict__ ks, const float *__restrict__ vs, const uint32_t *__restrict__ lens,
    float *__restrict__ part, uint32_t *__restrict__ qoff_out, void *__restrict__ out, uint32_t B,
    uint32_t H, uint32_t Hkv, uint32_t G, uint32_t bucket, uint32_t P, float log2e_over_scale) {
    __shared__ SegLds<D> lds;
    __shared__ uint32_t qoff[kScanMax + 1];
    __shared__ uint32_t wsum[kWaves];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    // quads of sequence i = ceil(min(lens[i], bucket) / 128); each thread owns
    // four consecutive sequences, then a workgroup-wide exclusive scan
    uint32_t nq[4], t = 0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const uint32_t i = 4 * tid + u;
        uint32_t L = i < B ? lens[i] : 0u;
        L = L > bucket ? bucket : L;
        nq[u] = (L + kQuad - 1) / kQuad;
        t += nq[u];
    }
    uint32_t incl = t;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t v = __shfl_up(incl, d, 64);
        if (lane >= d) incl += v;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    uint32_t ex = incl - t, total = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
        ex += w < wave ? wsum[w] : 0u;
        total += wsum[w];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const uint32_t i = 4 * tid + u;
        if (i < B) qoff[i] = ex;
        ex += nq[u];
    }
    if (tid == 0) qoff[B] = total;
    __syncthreads();
    if (blockIdx.x == 0)
        for (uint32_t i = tid; i <= B; i += kThreads) qoff_out[i] = qoff[i];

    // Everything below is uniform: keep it in scalar registers (the segment's
    // inner loop needs the vector registers).
    const uint32_t tot = uni(total);
    const uint64_t qt = uint64_t(Hkv) * tot;
    const uint32_t Pe = split_count(qt, P);
    const uint32_t w = blockIdx.x;
    if (w >= Pe) return;
    uint64_t x = uint64_t(w) * qt / Pe;
    const uint64_t x1 = uint64_t(w + 1) * qt / Pe;
    if (x >= x1) return;
    // the sequence holding quad x: the largest b with Hkv * qoff[b] <= x
    uint32_t lo = 0, hi = B;
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (uint64_t(Hkv) * uni(qoff[mid]) <= x) lo = mid; else hi = mid;
    }
    uint32_t b = lo;
    uint32_t q0 = uni(qoff[b]), q1 = uni(qoff[b + 1]);
    uint32_t kh = uint32_t((x - uint64_t(Hkv) * q0) / (q1 - q0));
    while (x < x1) {
        const uint32_t nqb = q1 - q0;
        const uint64_t ps = uint64_t(Hkv) * q0 + uint64_t(kh) * nqb, pe = ps + nqb;
        const uint64_t se = x1 < pe ? x1 : pe;
        uint32_t L = lens[b];
        L = L > bucket ? bucket : L;
        const uint32_t c0 = uint32_t(x - ps) * kQuad;
        const uint32_t c1e = uint32_t(se - ps) * kQuad;
        const uint32_t c1 = c1e < L ? c1e : L;
        const bool single = x == ps && se == pe;
        const uint64_t p = uint64_t(b) * Hkv + kh;
        float *dst = part + (p + w) * G * (D + 2);
        attn_segment<D, kF32Q>(q, kq, vq, ks, vs, dst, out, b, b, kh, c0, c1, single, H, Hkv, G,
                               bucket, log2e_over_scale, lds);
        x = se;
        if (++kh == Hkv) {
            kh = 0;
            do {
                ++b;
                q0 = q1;
                q1 = b < B ? uni(qoff[b + 1]) : q0;
            } while (b < B && q1 == q0);
        }
    }
}

// Merge `nseg` consecutive partials (m, l, O[D]) per head at `src` into the G
// output rows of plane (b, kh): 256 threads, the per-(segment, head) weights
// first, then each (head, dim) output as one weighted sum whose loads are
// issued eight at a time. nseg <= kMaxSeg.
constexpr uint32_t kMaxSeg = 1024;
constexpr uint32_t kFastSeg = 8;   // up to this many segments merge in one round trip

template <int D, bool kF32Q>
__device__ __forceinline__ void merge_partials(const float *__restrict__ src, uint32_t nseg,
                                               void *__restrict__ out, uint32_t b, uint32_t kh,
                                               uint32_t H, uint32_t G, float (&wgt)[kMaxSeg][16],
                                               float (&inv_l)[16]) {
    const uint32_t tid = threadIdx.x;
    const uint64_t cstride = uint64_t(G) * (D + 2);
    if (nseg <= kFastSeg && G * D <= 2 * 256) {
        // Few segments: each thread loads m, l and O of every segment for its
        // (head, dim) outputs in one go (one memory round trip instead of
        // three), then weighs them in segment order. Clamped indices keep
        // every load unconditional.
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint32_t idx = tid + 256u * t;
            const uint32_t h = idx < G * D ? idx / D : 0u, d = idx % D;
            float mc[kFastSeg], lc[kFastSeg], oc[kFastSeg];
#pragma unroll
            for (int c = 0; c < int(kFastSeg); ++c) {
                const float *ps = src + (uint32_t(c) < nseg ? c : nseg - 1) * cstride + h * (D + 2);
                mc[c] = ps[0];
                lc[c] = ps[1];
                oc[c] = ps[2 + d];
            }
            float m = -INFINITY;
#pragma unroll
            for (int c = 0; c < int(kFastSeg); ++c) m = uint32_t(c) < nseg ? fmaxf(m, mc[c]) : m;
            float o = 0.0f, l = 0.0f;
#pragma unroll
            for (int c = 0; c < int(kFastSeg); ++c) {
                if (uint32_t(c) >= nseg) continue;
                const float w = mc[c] == -INFINITY ? 0.0f : exp2f(mc[c] - m);
                o = fmaf(oc[c], w, o);
                l = fmaf(lc[c], w, l);
            }
            if (idx >= G * D) continue;
            const float res = o * (1.0f / l);
            const uint64_t oi = (uint64_t(b) * H + kh * G + h) * D + d;
            if constexpr (kF32Q)
                static_cast<float *>(out)[oi] = res;
            else
                static_cast<uint16_t *>(out)[oi] = uint16_t(__float_as_uint(res) >> 16);
        }
        return;
    }
    // per head: M = max_c m_c; wgt[c] = 2^(m_c - M); 1 / sum_c wgt[c] l_c
    if (tid < 64) {
        const uint32_t h = tid & 15, c4 = tid >> 4;    // 4 segment lanes per head
        float m = -INFINITY;
        if (h < G)
            for (uint32_t c = c4; c < nseg; c += 4) m = fmaxf(m, src[c * cstride + h * (D + 2)]);
        m = fmaxf(m, __shfl_xor(m, 16, 64));
        m = fmaxf(m, __shfl_xor(m, 32, 64));
        float l = 0.0f;
        if (h < G)
            for (uint32_t c = c4; c < nseg; c += 4) {
                const float mc = src[c * cstride + h * (D + 2)];
                const float w = mc == -INFINITY ? 0.0f : exp2f(mc - m);
                wgt[c][h] = w;
                l = fmaf(src[c * cstride + h * (D + 2) + 1], w, l);
            }
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        if (c4 == 0 && h < G) inv_l[h] = 1.0f / l;
    }
    __syncthreads();
    for (uint32_t idx = tid; idx < G * D; idx += 256) {
        const uint32_t h = idx / D, d = idx % D;
        const float *ph = src + h * (D + 2) + 2 + d;
        float o = 0.0f;
        for (uint32_t c0 = 0; c0 < nseg; c0 += 8) {
            float v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t c = c0 + u < nseg ? c0 + u : nseg - 1;
                v[u] = ph[c * cstride];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u)
                if (c0 + u < nseg) o = fmaf(v[u], wgt[c0 + u][h], o);
        }
        const float res = o * inv_l[h];
        const uint64_t oi = (uint64_t(b) * H + kh * G + h) * D + d;
        if constexpr (kF32Q)
            static_cast<float *>(out)[oi] = res;
        else
            static_cast<uint16_t *>(out)[oi] = uint16_t(__float_as_uint(res) >> 16);
    }
}

// Merge for the grid form: grid (Hkv, B); planes of one chunk were written directly.
template <int D, bool kF32Q>
__global__ __launch_bounds__(256) void attn_combine_kernel(const float *__restrict__ part,
                                                          const uint32_t *__restrict__ lens,
                                                          void *__restrict__ out, uint32_t H,
                                                          uint32_t Hkv, uint32_t G,
                                                          uint32_t bucket, uint32_t kChunk,
                                                          uint32_t nchunks, uint32_t q_rows) {
    __shared__ float wgt[kMaxSeg][16];
    __shared__ float inv_l[16];
    const uint32_t kh = blockIdx.x, v = blockIdx.y;
    const uint32_t L = visible_keys(lens[v / q_rows], q_rows - 1 - v % q_rows, bucket);
    const uint32_t nch = (L + kChunk - 1) / kChunk;
    if (nch <= 1) return;
    const uint64_t row_plane = uint64_t(v) * Hkv + kh;
    merge_partials<D, kF32Q>(part + row_plane * nchunks * G * (D + 2), nch, out, v, kh, H, G, wgt,
                             inv_l);
}

// Merge for the balanced form: grid (Hkv, B). A plane with no visible key gets
// the exact zero rows; a plane inside one workgroup's share was written
// directly; otherwise its partials p + wa .. p + wb are merged.
template <int D, bool kF32Q>
__global__ __launch_bounds__(256) void attn_merge_kernel(const float *__restrict__ part,
                                                        const uint32_t *__restrict__ qoff,
                                                        const uint32_t *__restrict__ lens,
                                                        void *__restrict__ out, uint32_t B,
                                                        uint32_t H, uint32_t Hkv, uint32_t G,
                                                        uint32_t bucket, uint32_t P) {
    __shared__ float wgt[kMaxSeg][16];
    __shared__ float inv_l[16];
    const uint32_t kh = blockIdx.x, b = blockIdx.y;
    const uint32_t L = lens[b];
    if (L == 0 || bucket == 0) {
        zero_rows<kF32Q>(out, b, kh, H, G, D, threadIdx.x, 256);
        return;
    }
    const uint64_t qt = uint64_t(Hkv) * qoff[B];
    const uint32_t Pe = split_count(qt, P);
    const uint32_t nqb = qoff[b + 1] - qoff[b];
    const uint64_t ps = uint64_t(Hkv) * qoff[b] + uint64_t(kh) * nqb, pe = ps + nqb;
    // workgroup holding quad x: ((x + 1) * Pe - 1) / qt
    const uint32_t wa = uint32_t(((ps + 1) * Pe - 1) / qt);
    const uint32_t wb = uint32_t((pe * Pe - 1) / qt);
    if (wa == wb) return;
    const uint64_t p = uint64_t(b) * Hkv + kh;
    merge_partials<D, kF32Q>(part + (p + wa) * G * (D + 2), wb - wa + 1, out, b, kh, H, G, wgt,
                             inv_l);
}

// Keys per workgroup of the grid form: a multiple of the 128 keys one pass of
// the four wavefronts covers.
uint32_t chunk_keys(uint32_t bucket) {
    uint32_t c = 2048;
    while ((bucket + c - 1) / c > kMaxSeg) c *= 2;
    return c;
}

uint32_t chunks_of(uint32_t bucket) {
    const uint32_t c = chunk_keys(bucket);
    return (bucket + c - 1) / c;
}

int cu_count() {
    static const int cus = [] {
        int dev = 0, c = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
            c = 256;
        return c;
    }();
    return cus;
}

// Workgroups of the balanced form: as many as the GPU runs at once (CUs x
// resident workgroups per CU of this kernel), at most kMaxSplit.
template <int D, bool kF32Q>
uint32_t split_wgs() {
    static const uint32_t n = [] {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &per_cu, reinterpret_cast<const void *>(&attn_split_kernel<D, kF32Q>), kThreads, 0) !=
                hipSuccess || per_cu <= 0)
            per_cu = 1;
        const uint64_t v = uint64_t(per_cu) * cu_count();
        return uint32_t(v < kMaxSplit ? v : kMaxSplit);
    }();
    return n;
}

// The balanced form is taken whenever the batch fits its LDS scan, except when
// every plane fits one chunk and there are enough planes to spread over the
// GPU: then the grid form is one workgroup per plane and needs no merge
// launch (a decode step's short contexts: 64 planes of <= 1024 keys run in
// 8-9 us against 11.5 + 4.4 us for split + merge).
constexpr uint32_t kGridMinPlanes = 32;

// A grid form of at most this many workgroups (fewer than the GPU's CUs) runs
// them wide, kWideWaves wavefronts each.
constexpr uint64_t kWideMaxWgs = 128;
constexpr int kWideWaves = 8;

uint32_t chunks_of(uint32_t bucket);

bool use_split(uint32_t B, uint32_t Hkv, uint32_t bucket) {
    if (B > kScanMax) return false;
    return !(chunks_of(bucket) == 1 && uint64_t(B) * Hkv >= kGridMinPlanes);
}

// scratch: partials first, then (balanced form) the B + 1 quad offsets
size_t split_part_floats(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t D, uint32_t P) {
    return (size_t(B) * Hkv + P) * (H / Hkv) * (D + 2);
}

template <int D, bool kF32Q>
hipError_t run_t(const AttnI8Args &a, void *scratch, hipStream_t stream) {
    const uint32_t G = a.H / a.Hkv;
    float *part = static_cast<float *>(scratch);
    const float mul = kLog2e / a.score_scale;
    if (a.q_rows == 1 && use_split(a.B, a.Hkv, a.bucket)) {
        const uint32_t P = split_wgs<D, kF32Q>();
        uint32_t *qoff = reinterpret_cast<uint32_t *>(part + split_part_floats(a.B, a.H, a.Hkv, D, P));
        hipLaunchKernelGGL((attn_split_kernel<D, kF32Q>), dim3(P), dim3(kThreads), 0, stream, a.q,
                           a.kq, a.vq, a.ks, a.vs, a.lens, part, qoff, a.out, a.B, a.H, a.Hkv, G,
                           a.bucket, P, mul);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL((attn_merge_kernel<D, kF32Q>), dim3(a.Hkv, a.B), dim3(256), 0, stream,
                           part, qoff, a.lens, a.out, a.B, a.H, a.Hkv, G, a.bucket, P);
        return hipGetLastError();
    }
    if constexpr (D == 64 && !kF32Q) {
        const uintptr_t al = reinterpret_cast<uintptr_t>(a.q) | reinterpret_cast<uintptr_t>(a.kq) |
                             reinterpret_cast<uintptr_t>(a.vq) | reinterpret_cast<uintptr_t>(a.out);
        if (a.q_rows > 1 && G == 4 && (al & 15) == 0) {
            hipLaunchKernelGGL(attn_prompt_kernel, dim3((a.q_rows + kPT - 1) / kPT, a.Hkv, a.B),
                               dim3(kThreads), 0, stream, static_cast<const uint16_t *>(a.q), a.kq,
                               a.vq, a.ks, a.vs, a.lens, static_cast<uint16_t *>(a.out), a.H, a.Hkv,
                               a.bucket, mul, a.q_rows);
            return hipGetLastError();
        }
    }
    const uint32_t ck = chunk_keys(a.bucket);
    const uint32_t nch = chunks_of(a.bucket);
    if (a.q_rows > 1 && nch == 1 && G <= 8) {
        const uint32_t R = 16 / G;
        const uint32_t nt = (a.q_rows + R - 1) / R;
        hipLaunchKernelGGL((attn_rows_packed_kernel<D, kF32Q>), dim3(1, a.Hkv, a.B * nt),
                           dim3(kThreads), 0, stream, a.q, a.kq, a.vq, a.ks, a.vs, a.lens, a.out,
                           a.H, a.Hkv, G, a.bucket, mul, a.q_rows, R);
        return hipGetLastError();
    }
    const uint32_t rows = a.B * a.q_rows;
    if (uint64_t(nch) * a.Hkv * rows <= kWideMaxWgs)
        hipLaunchKernelGGL((attn_chunk_kernel<D, kF32Q, kWideWaves>), dim3(nch, a.Hkv, rows),
                           dim3(64 * kWideWaves), 0, stream, a.q, a.kq, a.vq, a.ks, a.vs, a.lens,
                           part, a.out, a.H, a.Hkv, G, a.bucket, ck, nch, mul, a.q_rows);
    else
        hipLaunchKernelGGL((attn_chunk_kernel<D, kF32Q, kWaves>), dim3(nch, a.Hkv, rows),
                           dim3(kThreads), 0, stream, a.q, a.kq, a.vq, a.ks, a.vs, a.lens, part,
                           a.out, a.H, a.Hkv, G, a.bucket, ck, nch, mul, a.q_rows);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || nch == 1) return e;
    hipLaunchKernelGGL((attn_combine_kernel<D, kF32Q>), dim3(a.Hkv, rows), dim3(256), 0, stream,
                       part, a.lens, a.out, a.H, a.Hkv, G, a.bucket, ck, nch, a.q_rows);
    return hipGetLastError();
}

template <int D>
hipError_t run(const AttnI8Args &a, void *scratch, hipStream_t stream) {
    return a.dtype == 8 ? run_t<D, true>(a, scratch, stream) : run_t<D, false>(a, scratch, stream);
}

template <int D, bool kF32Q>
size_t scratch_t(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t bucket, uint32_t q_rows) {
    if (q_rows == 1 && use_split(B, Hkv, bucket))
        return split_part_floats(B, H, Hkv, D, split_wgs<D, kF32Q>()) * sizeof(float) +
               size_t(B + 1) * sizeof(uint32_t);
    return size_t(B) * q_rows * H * chunks_of(bucket) * (D + 2) * sizeof(float);
}

}  // namespace

size_t attn_i8_scratch_bytes(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t bucket, uint32_t D,
                             uint32_t q_rows) {
    // the larger of the bf16 and f32 instantiations' needs (their occupancy may differ)
    size_t n = 0;
    if (D == 128)
        n = std::max(scratch_t<128, false>(B, H, Hkv, bucket, q_rows),
                     scratch_t<128, true>(B, H, Hkv, bucket, q_rows));
    if (D == 64)
        n = std::max(scratch_t<64, false>(B, H, Hkv, bucket, q_rows),
                     scratch_t<64, true>(B, H, Hkv, bucket, q_rows));
    return n;
}

bool attn_i8_supported(uint32_t H, uint32_t Hkv, uint32_t D, uint32_t bucket) {
    if (Hkv == 0 || H % Hkv) return false;
    return (D == 64 || D == 128) && H / Hkv <= 16 && bucket <= (1u << 30) / D;
}

hipError_t launch_attn_i8(const AttnI8Args &a, void *scratch, hipStream_t stream) {
    if (a.D == 128) return run<128>(a, scratch, stream);
    if (a.D == 64) return run<64>(a, scratch, stream);
    return hipErrorInvalidValue;
}

bool attn_i8_pro_applies(const AttnI8Args &a, const EpiArgs &pro) {
    if (a.q_rows != 1 || a.dtype == 8 || !attn_i8_supported(a.H, a.Hkv, a.D, a.bucket) ||
        a.B == 0 || a.B > 65535 || a.Hkv > 65535 || use_split(a.B, a.Hkv, a.bucket) ||
        chunks_of(a.bucket) != 1)
        return false;
    if (!pro.bf16 || pro.m != a.B || pro.ks == 0 || pro.nseg == 0 || pro.nseg > uint32_t(kSkinnyMaxSeg))
        return false;
    for (uint32_t i = 0; i < pro.nseg; ++i) {
        const EpiSeg &s = pro.seg[i];
        if (s.head_dim != a.D || s.pair >= 0 || s.skip || s.ssq || s.n % (a.D * a.Hkv) != 0 ||
            (s.quant && s.new_rows != 1))
            return false;
    }
    return true;
}

hipError_t launch_attn_i8_pro(const AttnI8Args &a, const EpiArgs &pro, hipStream_t stream) {
    if (!attn_i8_pro_applies(a, pro)) return hipErrorInvalidValue;
    const uint32_t G = a.H / a.Hkv;
    const float mul = kLog2e / a.score_scale;
    const bool wide = uint64_t(a.Hkv) * a.B <= kWideMaxWgs;
    const auto *q = static_cast<const uint16_t *>(a.q);
    const dim3 grid(1, a.Hkv, a.B);
    if (a.D == 64 && wide)
        hipLaunchKernelGGL((attn_pro_kernel<64, kWideWaves>), grid, dim3(64 * kWideWaves), 0, stream, q,
                           a.kq, a.vq, a.ks, a.vs, a.lens, a.out, a.H, a.Hkv, G, a.bucket, mul, pro);
    else if (a.D == 64)
        hipLaunchKernelGGL((attn_pro_kernel<64, kWaves>), grid, dim3(kThreads), 0, stream, q, a.kq,
                           a.vq, a.ks, a.vs, a.lens, a.out, a.H, a.Hkv, G, a.bucket, mul, pro);
    else if (wide)
        hipLaunchKernelGGL((attn_pro_kernel<128, kWideWaves>), grid, dim3(64 * kWideWaves), 0, stream, q,
                           a.kq, a.vq, a.ks, a.vs, a.lens, a.out, a.H, a.Hkv, G, a.bucket, mul, pro);
    else
        hipLaunchKernelGGL((attn_pro_kernel<128, kWaves>), grid, dim3(kThreads), 0, stream, q, a.kq,
                           a.vq, a.ks, a.vs, a.lens, a.out, a.H, a.Hkv, G, a.bucket, mul, pro);
    return hipGetLastError();
}

}  // namespace holo
