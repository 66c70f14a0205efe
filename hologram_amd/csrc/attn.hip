// attn.hip — single-token GQA decode attention over int8 K/V caches.
//
// Semantics: for sequence b and query head h (kv head kh = h / G), the visible
// keys are rows [0, L_b) with L_b = min(lens[b], bucket) of plane (b, kh);
//   s_j = dot(q, k_j * kscale_j) / scale,  p = softmax(s),  out = sum_j p_j v_j * vscale_j
// which is the reference's DecodeAttentionValid row
// (crates/hologram-compute/src/cpu/float_kernels.rs:3834-3883) over the
// dequantized rows (kernels.rs:270). Softmax is fp32 (exp2 of log2e-scaled
// scores, online across chunks); no key with j >= L_b is ever read.
//
// Structure (split-K flash decoding):
//   attn_chunk_kernel  grid (chunks, Hkv, B), 256 threads. One workgroup
//                      owns one (b, kh, 256-key chunk) and all G query heads
//                      of the group, so each K/V byte is read from HBM once
//                      for the whole group. Pass 1 scores the chunk (int8 K
//                      dequantized in registers), the chunk max and sum are
//                      taken in LDS, pass 2 accumulates p * v. It writes the
//                      partial (m, l, acc[D]) per head.
//   attn_combine_kernel grid (H, B), D threads: merges the chunk partials of
//                      one (b, h) and writes the output row (bf16 by
//                      truncation, as the reference narrows, or f32).
// Workgroups whose chunk starts at or beyond L_b exit at once, so the
// ragged batch costs only the keys that exist.
#include <hip/hip_runtime.h>

#include "holo_kernels.h"

namespace holo {
namespace {

constexpr int kChunk = 256;   // keys per workgroup
constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float load_q(const void *q, uint8_t dtype, uint64_t i) {
    if (dtype == 8) return reinterpret_cast<const float *>(q)[i];
    return __uint_as_float(uint32_t(reinterpret_cast<const uint16_t *>(q)[i]) << 16);
}

// 4 int8 in a 32-bit word -> 4 floats (sign-extending byte extracts).
__device__ __forceinline__ void i8x4_to_f32(uint32_t w, float *f) {
    f[0] = static_cast<float>(static_cast<int32_t>(w << 24) >> 24);
    f[1] = static_cast<float>(static_cast<int32_t>(w << 16) >> 24);
    f[2] = static_cast<float>(static_cast<int32_t>(w << 8) >> 24);
    f[3] = static_cast<float>(static_cast<int32_t>(w) >> 24);
}

template <int DPT>
__device__ __forceinline__ void load_row(const int8_t *p, float *f) {
    if constexpr (DPT == 16) {
        const uint4 v = *reinterpret_cast<const uint4 *>(p);
        i8x4_to_f32(v.x, f);
        i8x4_to_f32(v.y, f + 4);
        i8x4_to_f32(v.z, f + 8);
        i8x4_to_f32(v.w, f + 12);
    } else {
        const uint2 v = *reinterpret_cast<const uint2 *>(p);
        i8x4_to_f32(v.x, f);
        i8x4_to_f32(v.y, f + 4);
    }
}

// D: head_dim; G: query heads per kv head; DPT: dims per thread.
template <int D, int G, int DPT>
__global__ __launch_bounds__(kThreads) void attn_chunk_kernel(
    const void *__restrict__ q, uint8_t dtype, const int8_t *__restrict__ kq,
    const int8_t *__restrict__ vq, const float *__restrict__ ks, const float *__restrict__ vs,
    const uint32_t *__restrict__ lens, float *__restrict__ part, uint32_t H, uint32_t Hkv,
    uint32_t bucket, uint32_t nchunks, float inv_scale_log2e) {
    constexpr int TPK = D / DPT;          // threads cooperating on one key row
    constexpr int KPP = kThreads / TPK;   // keys per pass of the workgroup
    static_assert(64 % TPK == 0, "a key's threads must share a wavefront");

    __shared__ float sc[G][kChunk];       // scores, then probabilities
    __shared__ float red[G][D];           // p.v accumulation across key slots
    __shared__ float stat[G][2];          // chunk max, chunk sum

    const uint32_t b = blockIdx.z, kh = blockIdx.y, chunk = blockIdx.x;
    uint32_t L = lens[b];
    if (L > bucket) L = bucket;
    const uint32_t c0 = chunk * kChunk;
    if (c0 >= L) return;
    const uint32_t nk = L - c0 < uint32_t(kChunk) ? L - c0 : uint32_t(kChunk);

    const int tid = threadIdx.x;
    const int dg = tid % TPK;             // dim group
    const int slot = tid / TPK;           // key slot
    const uint64_t plane = uint64_t(b) * Hkv + kh;
    const int8_t *kbase = kq + (plane * bucket + c0) * D + dg * DPT;
    const int8_t *vbase = vq + (plane * bucket + c0) * D + dg * DPT;
    const float *ksb = ks + plane * bucket + c0;
    const float *vsb = vs + plane * bucket + c0;

    for (int i = tid; i < G * D; i += kThreads) (&red[0][0])[i] = 0.0f;

    float qr[G][DPT];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < DPT; ++e)
            qr[g][e] = load_q(q, dtype, (uint64_t(b) * H + kh * G + g) * D + dg * DPT + e);

    // pass 1: s2 = (q . k_int) * kscale * log2e / scale
    for (uint32_t kk = slot; kk < nk; kk += KPP) {
        float kf[DPT];
        load_row<DPT>(kbase + uint64_t(kk) * D, kf);
        float dot[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float a = 0.0f;
#pragma unroll
            for (int e = 0; e < DPT; ++e) a = fmaf(qr[g][e], kf[e], a);
            dot[g] = a;
        }
#pragma unroll
        for (int off = TPK / 2; off >= 1; off >>= 1)
#pragma unroll
            for (int g = 0; g < G; ++g) dot[g] += __shfl_xor(dot[g], off, 64);
        if (dg == 0) {
            const float kscale = ksb[kk];
#pragma unroll
            for (int g = 0; g < G; ++g) sc[g][kk] = (dot[g] * kscale) * inv_scale_log2e;
        }
    }
    __syncthreads();

    // chunk max and sum per head: wavefront w takes heads w, w + 4, ...
    {
        const int w = tid >> 6, lane = tid & 63;
        for (int g = w; g < G; g += kThreads / 64) {
            float m = -INFINITY;
            for (uint32_t j = lane; j < nk; j += 64) m = fmaxf(m, sc[g][j]);
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
            float l = 0.0f;
            for (uint32_t j = lane; j < nk; j += 64) {
                const float p = exp2f(sc[g][j] - m);
                sc[g][j] = p;
                l += p;
            }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) l += __shfl_xor(l, off, 64);
            if (lane == 0) {
                stat[g][0] = m;
                stat[g][1] = l;
            }
        }
    }
    __syncthreads();

    // pass 2: acc[g][dims] += p_g * vscale * v_int
    float acc[G][DPT];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < DPT; ++e) acc[g][e] = 0.0f;
    for (uint32_t kk = slot; kk < nk; kk += KPP) {
        float vf[DPT];
        load_row<DPT>(vbase + uint64_t(kk) * D, vf);
        const float vscale = vsb[kk];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float pw = sc[g][kk] * vscale;
#pragma unroll
            for (int e = 0; e < DPT; ++e) acc[g][e] = fmaf(pw, vf[e], acc[g][e]);
        }
    }
    // fold the key slots of one wavefront (lanes dg, dg+TPK, ...), then LDS
#pragma unroll
    for (int off = TPK; off < 64; off <<= 1)
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < DPT; ++e) acc[g][e] += __shfl_xor(acc[g][e], off, 64);
    if ((tid & 63) < TPK) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < DPT; ++e) atomicAdd(&red[g][dg * DPT + e], acc[g][e]);
    }
    __syncthreads();

    float *dst = part + ((plane * nchunks + chunk) * G) * (D + 2);
    for (int i = tid; i < G * D; i += kThreads) {
        const int g = i / D, d = i % D;
        dst[g * (D + 2) + 2 + d] = red[g][d];
    }
    if (tid < G) {
        dst[tid * (D + 2)] = stat[tid][0];
        dst[tid * (D + 2) + 1] = stat[tid][1];
    }
}

template <int D, int G>
__global__ __launch_bounds__(D) void attn_combine_kernel(const float *__restrict__ part,
                                                        const uint32_t *__restrict__ lens,
                                                        void *__restrict__ out, uint8_t dtype,
                                                        uint32_t H, uint32_t Hkv, uint32_t bucket,
                                                        uint32_t nchunks) {
    const uint32_t h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const uint32_t kh = h / G, g = h % G;
    uint32_t L = lens[b];
    if (L > bucket) L = bucket;
    const uint32_t nch = (L + kChunk - 1) / kChunk;
    const float *src = part + ((uint64_t(b) * Hkv + kh) * nchunks * G + g) * (D + 2);
    const uint64_t stride = uint64_t(G) * (D + 2);
    float m = -INFINITY;
    for (uint32_t c = 0; c < nch; ++c) m = fmaxf(m, src[c * stride]);
    float l = 0.0f, o = 0.0f;
    for (uint32_t c = 0; c < nch; ++c) {
        const float w = exp2f(src[c * stride] - m);
        l = fmaf(src[c * stride + 1], w, l);
        o = fmaf(src[c * stride + 2 + d], w, o);
    }
    const float r = nch ? o / l : 0.0f;   // no visible key: the exact zero row
    const uint64_t oi = (uint64_t(b) * H + h) * D + d;
    if (dtype == 8)
        reinterpret_cast<float *>(out)[oi] = r;
    else
        reinterpret_cast<uint16_t *>(out)[oi] = uint16_t(__float_as_uint(r) >> 16);
}

uint32_t chunks_of(uint32_t bucket) { return (bucket + kChunk - 1) / kChunk; }

}  // namespace

size_t attn_i8_scratch_bytes(uint32_t B, uint32_t H, uint32_t bucket, uint32_t D) {
    return size_t(B) * H * chunks_of(bucket) * (D + 2) * sizeof(float);
}

bool attn_i8_supported(uint32_t H, uint32_t Hkv, uint32_t D) {
    if (Hkv == 0 || H % Hkv) return false;
    const uint32_t G = H / Hkv;
    return (D == 64 || D == 128) && (G == 1 || G == 2 || G == 4 || G == 8);
}

template <int D, int G, int DPT>
static hipError_t run(const AttnI8Args &a, float *part, hipStream_t stream) {
    const uint32_t nch = chunks_of(a.bucket);
    const float inv_scale_log2e = kLog2e / a.score_scale;
    hipLaunchKernelGGL((attn_chunk_kernel<D, G, DPT>), dim3(nch, a.Hkv, a.B), dim3(kThreads), 0,
                       stream, a.q, a.dtype, a.kq, a.vq, a.ks, a.vs, a.lens, part, a.H, a.Hkv,
                       a.bucket, nch, inv_scale_log2e);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((attn_combine_kernel<D, G>), dim3(a.H, a.B), dim3(D), 0, stream, part,
                       a.lens, a.out, a.dtype, a.H, a.Hkv, a.bucket, nch);
    return hipGetLastError();
}

hipError_t launch_attn_i8(const AttnI8Args &a, void *scratch, hipStream_t stream) {
    float *part = static_cast<float *>(scratch);
    const uint32_t G = a.H / a.Hkv;
    if (a.D == 128) {
        switch (G) {
            case 1: return run<128, 1, 16>(a, part, stream);
            case 2: return run<128, 2, 16>(a, part, stream);
            case 4: return run<128, 4, 16>(a, part, stream);
            case 8: return run<128, 8, 8>(a, part, stream);
        }
    } else if (a.D == 64) {
        switch (G) {
            case 1: return run<64, 1, 16>(a, part, stream);
            case 2: return run<64, 2, 16>(a, part, stream);
            case 4: return run<64, 4, 16>(a, part, stream);
            case 8: return run<64, 8, 8>(a, part, stream);
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace holo
