// attn_valid.hip — DecodeAttentionValid (discriminant 121) over 16-bit or f32
// K/V: the reference's own decode-attention op, as its compiler lowers
// attention (crates/hologram-compiler/src/lower.rs:817), with the semantics
// of decode_attention_valid_float (src/cpu/float_kernels.rs:4192-4307) and its
// row function (:3834-3957). The same kernels serve the mask form,
// DecodeAttention (discriminant 119, decode_attention_float :2482-2600, row
// function :2420-2477): the list is every past row then every new row, and
// query row qi adds mask[qi][j] (f32 [q_rows, past + new]) to the score of
// list entry j; a key the mask erases (-inf) weighs exactly 0, and a row
// whose every key is erased is the zero row.
//
// Visible keys of a plane (batch b, kv head) form one list: the realized past
// prefix, rows [0, vis_past) of k_past / v_past (vis_past = min(valid_len,
// past_len), read on the device), then the new rows [0, new_len) of k_new /
// v_new. Query row qi of head h sees the first vis_past + min(qi + 1, new_len)
// entries. Scores are dot(q, k) / scale, softmax in f32 with the reference's
// deterministic exp (exp_f32_det), zero visible keys give the exact zero row.
//
// Layout of the work. The G*M query rows of one plane are contiguous in q
// ([B, H, M, D], heads kvh*G .. kvh*G+G-1), so a workgroup owns a tile of RT
// of them and walks a share of the plane's key list in blocks of KB keys.
// Each block of K and V is widened to f32 into LDS once and serves all RT
// rows (the GQA reuse): scores from LDS, an online softmax per row, then the
// PV accumulation with each thread owning fixed (row, column) slots. The list
// is cut into `nsplit` equal shares (from the realized length, so a short
// valid_len does not leave most workgroups idle); the shares' partials
// (m, l, acc[D]) are merged in share order by a second launch.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "holo_device.h"
#include "holo_kernels.h"

namespace holo {
namespace {

constexpr int kThreads = 256;
constexpr int kNacc = 16;     // acc slots per thread: RT * D <= 4096

// element widening / narrowing by dtype tag (bf16 7, f16 6, f32 8)
template <int DT>
__device__ __forceinline__ float ld_elem(const void *p, uint64_t i) {
    if constexpr (DT == 8) return static_cast<const float *>(p)[i];
    else if constexpr (DT == 7) return __uint_as_float(uint32_t(static_cast<const uint16_t *>(p)[i]) << 16);
    else return f16_bits_to_f32(static_cast<const uint16_t *>(p)[i]);
}

template <int DT>
__device__ __forceinline__ void st_elem(void *p, uint64_t i, float v) {
    if constexpr (DT == 8) static_cast<float *>(p)[i] = v;
    else if constexpr (DT == 7) static_cast<uint16_t *>(p)[i] = uint16_t(__float_as_uint(v) >> 16);
    else static_cast<uint16_t *>(p)[i] = f32_to_f16_bits(v);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ uint32_t read_u32_le(const uint8_t *p) {
    return uint32_t(p[0]) | (uint32_t(p[1]) << 8) | (uint32_t(p[2]) << 16) | (uint32_t(p[3]) << 24);
}

// grid (nsplit, row tiles, planes). LDS: q tile [RT][D], K block [KB][D+1]
// (padded: a wave's lanes read one column of consecutive keys), V block
// [KB][D], scores [RT][KB], per-row running max, sum and rescale factor.
template <int DT>
__global__ __launch_bounds__(kThreads) void attn_valid_split_kernel(AttnValidArgs a, uint32_t RT,
                                                                    uint32_t KB, uint32_t nsplit,
                                                                    float *__restrict__ part) {
    extern __shared__ float lds[];
    const uint32_t D = a.D, Dp = D + 1;
    float *qs = lds;
    float *ks = qs + RT * D;
    float *vs = ks + KB * Dp;
    float *sc = vs + KB * D;
    float *mrow = sc + RT * KB;
    float *lrow = mrow + RT;
    float *alpha = lrow + RT;

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t split = blockIdx.x, tile = blockIdx.y, plane = blockIdx.z;
    const uint32_t G = a.H / a.Hkv, R = G * a.M;
    const uint32_t b = plane / a.Hkv, kvh = plane % a.Hkv;
    const uint32_t r0 = tile * RT, nr = R - r0 < RT ? R - r0 : RT;
    const uint64_t qrow0 = (uint64_t(b) * a.H + uint64_t(kvh) * G) * a.M + r0;

    // mask form: every past row is in the list, visibility is the mask's
    uint32_t vis_past = a.mask ? a.past : read_u32_le(a.valid_len);
    if (vis_past > a.past) vis_past = a.past;
    const uint32_t total = vis_past + a.nnew;
    const uint32_t share = (total + nsplit - 1) / nsplit;
    const uint32_t chunk = (share + KB - 1) / KB * KB;
    const uint32_t j0 = split * chunk < total ? split * chunk : total;
    const uint32_t j1 = j0 + chunk < total ? j0 + chunk : total;

    for (uint32_t e = tid; e < nr * D; e += kThreads) qs[e] = ld_elem<DT>(a.q, qrow0 * D + e);
    if (tid < RT) {
        mrow[tid] = -INFINITY;
        lrow[tid] = 0.0f;
    }
    float acc[kNacc];
#pragma unroll
    for (int i = 0; i < kNacc; ++i) acc[i] = 0.0f;
    const uint64_t kp_base = uint64_t(plane) * a.past * D, kn_base = uint64_t(plane) * a.nnew * D;
    __syncthreads();

    for (uint32_t jb = j0; jb < j1; jb += KB) {
        const uint32_t nk = j1 - jb < KB ? j1 - jb : KB;
        // stage the block: list entry j is past row j, or new row j - vis_past
        for (uint32_t e = tid; e < nk * D; e += kThreads) {
            const uint32_t key = e / D, c = e % D, j = jb + key;
            float kv, vv;
            if (j < vis_past) {
                kv = ld_elem<DT>(a.kp, kp_base + uint64_t(j) * D + c);
                vv = ld_elem<DT>(a.vp, kp_base + uint64_t(j) * D + c);
            } else {
                kv = ld_elem<DT>(a.kn, kn_base + uint64_t(j - vis_past) * D + c);
                vv = ld_elem<DT>(a.vn, kn_base + uint64_t(j - vis_past) * D + c);
            }
            ks[key * Dp + c] = kv;
            vs[key * D + c] = vv;
        }
        __syncthreads();
        // scores of (row, key); a key past the row's causal limit is -inf
        for (uint32_t pi = tid; pi < nr * KB; pi += kThreads) {
            const uint32_t rr = pi / KB, key = pi % KB;
            const uint32_t qi = (r0 + rr) % a.M;
            const uint32_t lim = a.mask ? total : vis_past + (qi + 1 < a.nnew ? qi + 1 : a.nnew);
            float s = -INFINITY;
            if (key < nk && jb + key < lim) {
                const float *qr = qs + rr * D, *kr = ks + key * Dp;
                float d0 = 0.0f, d1 = 0.0f, d2 = 0.0f, d3 = 0.0f;
                uint32_t c = 0;
                for (; c + 4 <= D; c += 4) {
                    d0 = fmaf(qr[c], kr[c], d0);
                    d1 = fmaf(qr[c + 1], kr[c + 1], d1);
                    d2 = fmaf(qr[c + 2], kr[c + 2], d2);
                    d3 = fmaf(qr[c + 3], kr[c + 3], d3);
                }
                for (; c < D; ++c) d0 = fmaf(qr[c], kr[c], d0);
                s = ((d0 + d1) + (d2 + d3)) / a.scale;
                if (a.mask) s = s + a.mask[uint64_t(qi) * total + jb + key];
            }
            sc[rr * KB + key] = s;
        }
        __syncthreads();
        // online softmax: one wave per row, one key per lane (KB <= 64)
        for (uint32_t rr = wave; rr < nr; rr += kThreads / 64) {
            const float v = lane < KB ? sc[rr * KB + lane] : -INFINITY;
            const float m_old = mrow[rr];
            const float m_new = fmaxf(m_old, wave_max(v));
            float p = 0.0f, al = 1.0f;
            if (m_new != -INFINITY) {
                p = v == -INFINITY ? 0.0f : exp_det(v - m_new);
                al = m_old == -INFINITY ? 0.0f : exp_det(m_old - m_new);
            }
            const float psum = wave_sum(p);
            if (lane < KB) sc[rr * KB + lane] = p;
            if (lane == 0) {
                lrow[rr] = lrow[rr] * al + psum;
                mrow[rr] = m_new;
                alpha[rr] = al;
            }
        }
        __syncthreads();
        // PV: slot i of this thread is (row, column) = divmod(tid + 256 i, D).
        // A valid-form row's list ends at its causal limit: keys past it are
        // not in the row's list at all (not even as 0 * v, which a non-finite
        // v would turn into NaN). The mask form's list is every key.
#pragma unroll
        for (int i = 0; i < kNacc; ++i) {
            const uint32_t idx = tid + kThreads * uint32_t(i);
            if (idx < nr * D) {
                const uint32_t rr = idx / D, c = idx % D;
                uint32_t kend = nk;
                if (!a.mask) {
                    const uint32_t qi = (r0 + rr) % a.M;
                    const uint32_t lim = vis_past + (qi + 1 < a.nnew ? qi + 1 : a.nnew);
                    const uint32_t room = lim > jb ? lim - jb : 0;
                    kend = room < nk ? room : nk;
                }
                float x = acc[i] * alpha[rr];
                const float *pr = sc + rr * KB;
                for (uint32_t key = 0; key < kend; ++key) x = fmaf(pr[key], vs[key * D + c], x);
                acc[i] = x;
            }
        }
        __syncthreads();
    }
    // a single share finishes the rows; several leave (m, l, acc) partials.
    // A row with no visible key (every score -inf) is the exact zero row
    // (float_kernels.rs:2446-2453, :3849-3852), whatever its keys' v rows hold.
    if (nsplit == 1) {
#pragma unroll
        for (int i = 0; i < kNacc; ++i) {
            const uint32_t idx = tid + kThreads * uint32_t(i);
            if (idx < nr * D) {
                const uint32_t rr = idx / D;
                const float l = lrow[rr];
                const float o = mrow[rr] == -INFINITY ? 0.0f : acc[i] / (l > 1e-30f ? l : 1e-30f);
                st_elem<DT>(a.out, qrow0 * D + idx, o);
            }
        }
        return;
    }
    const uint32_t planes = a.B * a.Hkv, ntiles = gridDim.y;
    float *pp = part + ((uint64_t(split) * planes + plane) * ntiles + tile) * uint64_t(RT) * (D + 2);
#pragma unroll
    for (int i = 0; i < kNacc; ++i) {
        const uint32_t idx = tid + kThreads * uint32_t(i);
        if (idx < nr * D) {
            const uint32_t rr = idx / D, c = idx % D;
            pp[uint64_t(rr) * (D + 2) + 2 + c] = acc[i];
        }
    }
    if (tid < nr) {
        pp[uint64_t(tid) * (D + 2)] = mrow[tid];
        pp[uint64_t(tid) * (D + 2) + 1] = lrow[tid];
    }
}

// One workgroup per query row: the shares' weights exp(m_s - M) first (share
// order), then out = sum_s w_s acc_s / max(sum_s w_s l_s, 1e-30). Every share
// enters the sum, so a share whose keys the row weighs 0 still passes on
// 0 * v (a non-finite v reaches the output, as in the reference's axpy); a row
// with no visible key in any share is the exact zero row.
template <int DT>
__global__ __launch_bounds__(kThreads) void attn_valid_merge_kernel(AttnValidArgs a, uint32_t RT,
                                                                    uint32_t nsplit, uint32_t ntiles,
                                                                    const float *__restrict__ part) {
    __shared__ float w[256];
    __shared__ float denom, mxs;
    const uint32_t D = a.D, G = a.H / a.Hkv, R = G * a.M;
    const uint32_t plane = blockIdx.x / R, r = blockIdx.x % R;
    const uint32_t tile = r / RT, rr = r % RT;
    const uint32_t b = plane / a.Hkv, kvh = plane % a.Hkv;
    const uint64_t qrow = (uint64_t(b) * a.H + uint64_t(kvh) * G) * a.M + r;
    const uint32_t planes = a.B * a.Hkv;
    auto row_of = [&](uint32_t s) {
        return part + (((uint64_t(s) * planes + plane) * ntiles + tile) * RT + rr) * uint64_t(D + 2);
    };
    if (threadIdx.x == 0) {
        float mx = -INFINITY;
        for (uint32_t s = 0; s < nsplit; ++s) mx = fmaxf(mx, row_of(s)[0]);
        float l = 0.0f;
        for (uint32_t s = 0; s < nsplit; ++s) {
            const float ms = row_of(s)[0];
            const float ws = (mx == -INFINITY || ms == -INFINITY) ? 0.0f : exp_det(ms - mx);
            w[s] = ws;
            l = l + ws * row_of(s)[1];
        }
        denom = l > 1e-30f ? l : 1e-30f;
        mxs = mx;
    }
    __syncthreads();
    const bool none = mxs == -INFINITY;
    for (uint32_t c = threadIdx.x; c < D; c += kThreads) {
        float x = 0.0f;
        if (!none)
            for (uint32_t s = 0; s < nsplit; ++s) x = fmaf(w[s], row_of(s)[2 + c], x);
        st_elem<DT>(a.out, qrow * D + c, x / denom);
    }
}

struct Plan {
    uint32_t RT, KB, ntiles, nsplit;
    size_t lds;
};

int cu_count() {
    static const int n = [] {
        int dev = 0, c = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
            c = 256;
        return c;
    }();
    return n;
}

Plan plan_of(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t M, uint32_t past, uint32_t nnew, uint32_t D) {
    Plan p;
    p.RT = 4096 / D < 16 ? 4096 / D : 16;
    if (p.RT == 0) p.RT = 1;
    // the largest key block (<= 64, a multiple of 8 when >= 8) whose LDS,
    // with the q tile, stays within 64 KiB
    const int64_t avail = 16384 - int64_t(p.RT) * D - 3 * int64_t(p.RT);
    int64_t kb = avail / (2 * int64_t(D) + 1 + p.RT);
    if (kb > 64) kb = 64;
    if (kb >= 8) kb &= ~int64_t(7);
    p.KB = kb < 1 ? 1 : uint32_t(kb);
    const uint32_t R = (H / Hkv) * M;
    p.ntiles = (R + p.RT - 1) / p.RT;
    const uint64_t groups = uint64_t(B) * Hkv * p.ntiles;
    const uint64_t blocks = (uint64_t(past) + nnew + p.KB - 1) / p.KB;
    uint64_t ns = (2ull * cu_count() + groups - 1) / groups;
    if (ns > blocks) ns = blocks;
    if (ns > 256) ns = 256;
    if (ns < 1) ns = 1;
    p.nsplit = uint32_t(ns);
    p.lds = (size_t(p.RT) * D + size_t(p.KB) * (D + 1) + size_t(p.KB) * D + size_t(p.RT) * p.KB +
             3 * size_t(p.RT)) * sizeof(float);
    return p;
}

template <int DT>
hipError_t run(const AttnValidArgs &a, void *scratch, hipStream_t stream) {
    const Plan p = plan_of(a.B, a.H, a.Hkv, a.M, a.past, a.nnew, a.D);
    float *part = static_cast<float *>(scratch);
    hipLaunchKernelGGL(attn_valid_split_kernel<DT>, dim3(p.nsplit, p.ntiles, a.B * a.Hkv),
                       dim3(kThreads), p.lds, stream, a, p.RT, p.KB, p.nsplit, part);
    if (p.nsplit == 1) return hipGetLastError();
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint32_t rows = a.B * a.Hkv * (a.H / a.Hkv) * a.M;
    hipLaunchKernelGGL(attn_valid_merge_kernel<DT>, dim3(rows), dim3(kThreads), 0, stream, a,
                       p.RT, p.nsplit, p.ntiles, part);
    return hipGetLastError();
}

// ------------------------------------------------ int8 cache, any head_dim --
// Ops 123 / 125 over the int8 cache for the shapes attn.hip's MFMA kernels do
// not take (head_dim other than 64 / 128, more than 16 query heads per kv
// head): the same blocked split-K walk as above, each K/V block dequantized
// into LDS with one f32 multiply per element, q * scale (the Dequantize law,
// src/cpu/kernels.rs:270). A plane's rows are (t, g), t < q_rows, g < G, row
// r = t G + g, q / out [B, q_rows, H, D]; row (t, g) of sequence b sees the
// first clamp(lens[b] - (q_rows - 1 - t), 0, bucket) cache rows.
template <int DT>
__device__ __forceinline__ uint64_t i8_row_index(const AttnI8Args &a, uint32_t b, uint32_t kvh,
                                                 uint32_t G, uint32_t r) {
    const uint32_t t = r / G, g = r % G;
    return (uint64_t(b) * a.q_rows + t) * a.H + uint64_t(kvh) * G + g;
}

__device__ __forceinline__ uint32_t i8_row_limit(const AttnI8Args &a, uint32_t len, uint32_t G,
                                                 uint32_t r) {
    const int64_t v = int64_t(len) - int64_t(a.q_rows - 1 - r / G);
    return v <= 0 ? 0u : (uint64_t(v) < a.bucket ? uint32_t(v) : a.bucket);
}

template <int DT>
__global__ __launch_bounds__(kThreads) void attn_i8_any_split_kernel(AttnI8Args a, uint32_t RT,
                                                                     uint32_t KB, uint32_t nsplit,
                                                                     float *__restrict__ part) {
    extern __shared__ float lds[];
    const uint32_t D = a.D, Dp = D + 1;
    float *qs = lds;
    float *ks = qs + RT * D;
    float *vs = ks + KB * Dp;
    float *sc = vs + KB * D;
    float *mrow = sc + RT * KB;
    float *lrow = mrow + RT;
    float *alpha = lrow + RT;

    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t split = blockIdx.x, tile = blockIdx.y, plane = blockIdx.z;
    const uint32_t G = a.H / a.Hkv, R = G * a.q_rows;
    const uint32_t b = plane / a.Hkv, kvh = plane % a.Hkv;
    const uint32_t r0 = tile * RT, nr = R - r0 < RT ? R - r0 : RT;
    const uint32_t len = a.lens[b];
    const uint32_t total = i8_row_limit(a, len, G, R - 1);   // the last row sees the most
    const uint32_t share = (total + nsplit - 1) / nsplit;
    const uint32_t chunk = (share + KB - 1) / KB * KB;
    const uint32_t j0 = split * chunk < total ? split * chunk : total;
    const uint32_t j1 = j0 + chunk < total ? j0 + chunk : total;

    for (uint32_t e = tid; e < nr * D; e += kThreads)
        qs[e] = ld_elem<DT>(a.q, i8_row_index<DT>(a, b, kvh, G, r0 + e / D) * D + e % D);
    if (tid < RT) {
        mrow[tid] = -INFINITY;
        lrow[tid] = 0.0f;
    }
    float acc[kNacc];
#pragma unroll
    for (int i = 0; i < kNacc; ++i) acc[i] = 0.0f;
    const uint64_t row_base = uint64_t(plane) * a.bucket;
    __syncthreads();

    for (uint32_t jb = j0; jb < j1; jb += KB) {
        const uint32_t nk = j1 - jb < KB ? j1 - jb : KB;
        for (uint32_t e = tid; e < nk * D; e += kThreads) {
            const uint32_t key = e / D, c = e % D;
            const uint64_t row = row_base + jb + key;
            ks[key * Dp + c] = float(a.kq[row * D + c]) * a.ks[row];
            vs[key * D + c] = float(a.vq[row * D + c]) * a.vs[row];
        }
        __syncthreads();
        for (uint32_t pi = tid; pi < nr * KB; pi += kThreads) {
            const uint32_t rr = pi / KB, key = pi % KB;
            const uint32_t lim = i8_row_limit(a, len, G, r0 + rr);
            float s = -INFINITY;
            if (key < nk && jb + key < lim) {
                const float *qr = qs + rr * D, *kr = ks + key * Dp;
                float d0 = 0.0f, d1 = 0.0f, d2 = 0.0f, d3 = 0.0f;
                uint32_t c = 0;
                for (; c + 4 <= D; c += 4) {
                    d0 = fmaf(qr[c], kr[c], d0);
                    d1 = fmaf(qr[c + 1], kr[c + 1], d1);
                    d2 = fmaf(qr[c + 2], kr[c + 2], d2);
                    d3 = fmaf(qr[c + 3], kr[c + 3], d3);
                }
                for (; c < D; ++c) d0 = fmaf(qr[c], kr[c], d0);
                s = ((d0 + d1) + (d2 + d3)) / a.score_scale;
            }
            sc[rr * KB + key] = s;
        }
        __syncthreads();
        for (uint32_t rr = wave; rr < nr; rr += kThreads / 64) {
            const float v = lane < KB ? sc[rr * KB + lane] : -INFINITY;
            const float m_old = mrow[rr];
            const float m_new = fmaxf(m_old, wave_max(v));
            float p = 0.0f, al = 1.0f;
            if (m_new != -INFINITY) {
                p = v == -INFINITY ? 0.0f : exp_det(v - m_new);
                al = m_old == -INFINITY ? 0.0f : exp_det(m_old - m_new);
            }
            const float psum = wave_sum(p);
            if (lane < KB) sc[rr * KB + lane] = p;
            if (lane == 0) {
                lrow[rr] = lrow[rr] * al + psum;
                mrow[rr] = m_new;
                alpha[rr] = al;
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kNacc; ++i) {
            const uint32_t idx = tid + kThreads * uint32_t(i);
            if (idx < nr * D) {
                const uint32_t rr = idx / D, c = idx % D;
                const uint32_t lim = i8_row_limit(a, len, G, r0 + rr);
                const uint32_t room = lim > jb ? lim - jb : 0;
                const uint32_t kend = room < nk ? room : nk;
                float x = acc[i] * alpha[rr];
                const float *pr = sc + rr * KB;
                for (uint32_t key = 0; key < kend; ++key) x = fmaf(pr[key], vs[key * D + c], x);
                acc[i] = x;
            }
        }
        __syncthreads();
    }
    if (nsplit == 1) {   // one share finishes its rows; no visible key: the zero row
#pragma unroll
        for (int i = 0; i < kNacc; ++i) {
            const uint32_t idx = tid + kThreads * uint32_t(i);
            if (idx < nr * D) {
                const uint32_t rr = idx / D, c = idx % D;
                const float l = lrow[rr];
                const float o = mrow[rr] == -INFINITY ? 0.0f : acc[i] / (l > 1e-30f ? l : 1e-30f);
                st_elem<DT>(a.out, i8_row_index<DT>(a, b, kvh, G, r0 + rr) * D + c, o);
            }
        }
        return;
    }
    const uint32_t planes = a.B * a.Hkv, ntiles = gridDim.y;
    float *pp = part + ((uint64_t(split) * planes + plane) * ntiles + tile) * uint64_t(RT) * (D + 2);
#pragma unroll
    for (int i = 0; i < kNacc; ++i) {
        const uint32_t idx = tid + kThreads * uint32_t(i);
        if (idx < nr * D) {
            const uint32_t rr = idx / D, c = idx % D;
            pp[uint64_t(rr) * (D + 2) + 2 + c] = acc[i];
        }
    }
    if (tid < nr) {
        pp[uint64_t(tid) * (D + 2)] = mrow[tid];
        pp[uint64_t(tid) * (D + 2) + 1] = lrow[tid];
    }
}

// One workgroup per query row: the shares merged in share order, as the
// valid form's merge; a row with no visible key is the zero row.
template <int DT>
__global__ __launch_bounds__(kThreads) void attn_i8_any_merge_kernel(AttnI8Args a, uint32_t RT,
                                                                     uint32_t nsplit, uint32_t ntiles,
                                                                     const float *__restrict__ part) {
    __shared__ float w[256];
    __shared__ float denom, mxs;
    const uint32_t D = a.D, G = a.H / a.Hkv, R = G * a.q_rows;
    const uint32_t plane = blockIdx.x / R, r = blockIdx.x % R;
    const uint32_t tile = r / RT, rr = r % RT;
    const uint32_t b = plane / a.Hkv, kvh = plane % a.Hkv;
    const uint64_t orow = i8_row_index<DT>(a, b, kvh, G, r);
    const uint32_t planes = a.B * a.Hkv;
    auto row_of = [&](uint32_t s) {
        return part + (((uint64_t(s) * planes + plane) * ntiles + tile) * RT + rr) * uint64_t(D + 2);
    };
    if (threadIdx.x == 0) {
        float mx = -INFINITY;
        for (uint32_t s = 0; s < nsplit; ++s) mx = fmaxf(mx, row_of(s)[0]);
        float l = 0.0f;
        for (uint32_t s = 0; s < nsplit; ++s) {
            const float ms = row_of(s)[0];
            const float ws = (mx == -INFINITY || ms == -INFINITY) ? 0.0f : exp_det(ms - mx);
            w[s] = ws;
            l = l + ws * row_of(s)[1];
        }
        denom = l > 1e-30f ? l : 1e-30f;
        mxs = mx;
    }
    __syncthreads();
    const bool none = mxs == -INFINITY;
    for (uint32_t c = threadIdx.x; c < D; c += kThreads) {
        float x = 0.0f;
        if (!none)
            for (uint32_t s = 0; s < nsplit; ++s) x = fmaf(w[s], row_of(s)[2 + c], x);
        st_elem<DT>(a.out, orow * D + c, x / denom);
    }
}

Plan plan_i8_any(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t q_rows, uint32_t bucket, uint32_t D) {
    Plan p = plan_of(B, H, Hkv, q_rows, 0, bucket, D);
    return p;
}

template <int DT>
hipError_t run_i8_any(const AttnI8Args &a, void *scratch, hipStream_t stream) {
    const Plan p = plan_i8_any(a.B, a.H, a.Hkv, a.q_rows, a.bucket, a.D);
    float *part = static_cast<float *>(scratch);
    hipLaunchKernelGGL(attn_i8_any_split_kernel<DT>, dim3(p.nsplit, p.ntiles, a.B * a.Hkv),
                       dim3(kThreads), p.lds, stream, a, p.RT, p.KB, p.nsplit, part);
    if (p.nsplit == 1) return hipGetLastError();
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const uint32_t rows = a.B * a.Hkv * (a.H / a.Hkv) * a.q_rows;
    hipLaunchKernelGGL(attn_i8_any_merge_kernel<DT>, dim3(rows), dim3(kThreads), 0, stream, a, p.RT,
                       p.nsplit, p.ntiles, part);
    return hipGetLastError();
}

}  // namespace

bool attn_i8_any_supported(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t q_rows, uint32_t D) {
    if (D == 0 || D > 4096 || Hkv == 0 || H % Hkv != 0 || q_rows == 0) return false;
    const Plan p = plan_i8_any(B, H, Hkv, q_rows, 1, D);
    return p.ntiles <= 65535 && uint64_t(B) * Hkv <= 65535 &&
           uint64_t(B) * H * q_rows <= 0x7fffffffull && p.lds <= 64 * 1024;
}

size_t attn_i8_any_scratch_bytes(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t q_rows,
                                 uint32_t bucket, uint32_t D) {
    const Plan p = plan_i8_any(B, H, Hkv, q_rows, bucket, D);
    if (p.nsplit == 1) return 0;
    return size_t(p.nsplit) * B * Hkv * p.ntiles * p.RT * (size_t(D) + 2) * sizeof(float);
}

hipError_t launch_attn_i8_any(const AttnI8Args &a, void *scratch, hipStream_t stream) {
    switch (a.dtype) {
        case 7: return run_i8_any<7>(a, scratch, stream);
        case 8: return run_i8_any<8>(a, scratch, stream);
        default: return hipErrorInvalidValue;
    }
}

bool attn_valid_supported(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t M, uint32_t D) {
    if (D == 0 || D > 4096 || Hkv == 0 || H % Hkv != 0) return false;
    const Plan p = plan_of(B, H, Hkv, M, 0, M, D);
    // grid y (row tiles) and z (planes), and one merge workgroup per query row
    return p.ntiles <= 65535 && uint64_t(B) * Hkv <= 65535 &&
           uint64_t(B) * H * M <= 0x7fffffffull && p.lds <= 64 * 1024;
}

size_t attn_valid_scratch_bytes(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t M, uint32_t past,
                                uint32_t nnew, uint32_t D) {
    const Plan p = plan_of(B, H, Hkv, M, past, nnew, D);
    if (p.nsplit == 1) return 0;
    return size_t(p.nsplit) * B * Hkv * p.ntiles * p.RT * (size_t(D) + 2) * sizeof(float);
}

hipError_t launch_attn_valid(const AttnValidArgs &a, void *scratch, hipStream_t stream) {
    switch (a.dtype) {
        case 7: return run<7>(a, scratch, stream);
        case 6: return run<6>(a, scratch, stream);
        case 8: return run<8>(a, scratch, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace holo
