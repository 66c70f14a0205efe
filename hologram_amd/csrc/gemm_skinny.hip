// gemm_skinny.hip — C = A * B for a few rows of A (M <= 64), the decode-shaped
// MatMul (one token's activations against a weight): B's K*N elements are the
// whole cost, so the kernels are built to stream B once at HBM rate.
//
// Same arithmetic contract as the tiled kernels (matmul_float,
// crates/hologram-compute/src/cpu/float_kernels.rs:298-399): fp32 accumulate,
// bf16 results narrowed by truncation (src/cpu/dtype.rs:75-79).
//
// Summation order (bf16). K is cut into 32-deep steps; chain c = 0..63
// accumulates the steps s = c, c + 64, c + 128, ... in ascending order on the
// MFMA; group g = 0..15 adds its chains 4g .. 4g + 3 in order; the product is
// the groups added in order. The order depends on K alone, so a call, a
// grouped launch and the single-launch form over packed weights
// (gemv_packed.hip) give the same bits.
//
// Work split (bf16). A workgroup owns a strip of 128 columns and one group:
// its four wavefronts are the group's four chains, each issuing all of its
// steps' B loads up front (up to four steps a batch), and their partial tiles
// are added through LDS in chain order. Each group's fp32 partials go to
// [group][M][N] and a second kernel adds the groups in order. f32 keeps
// contiguous K ranges of KC rows, the four waves interleaving over a range in
// k steps, the ranges summed in order by the same second kernel.
//
// B operand without LDS. B is row-major, the MFMA B operand wants consecutive
// k per lane. A lane loads an 8 (k) x 8 (n) bf16 block as eight 16-byte rows
// and transposes it with byte permutes into eight k-vectors, one per column;
// MFMA number c then covers columns 8j + c of the strip (j = lane % 16), so the
// accumulators of one lane hold 8 consecutive columns. f32 does the same with
// 4 x 4 blocks and 16x16x4 MFMAs, with the k order chosen so the A operand of
// four MFMAs is one 16-byte load.
#include <hip/hip_runtime.h>

#include "holo_device.h"
#include "holo_kernels.h"

namespace holo {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, int(bytes), 0x00020000);
}

// Column c (0..7) of an 8x8 bf16 block held as 8 rows of 4 dwords: the 8 k
// values as 4 dwords of k pairs.
__device__ __forceinline__ u32x4 column8(const u32x4 *rows, int c) {
    const uint32_t sel = (c & 1) ? 0x07060302u : 0x05040100u;
    u32x4 o;
    o.x = __builtin_amdgcn_perm(rows[1][c >> 1], rows[0][c >> 1], sel);
    o.y = __builtin_amdgcn_perm(rows[3][c >> 1], rows[2][c >> 1], sel);
    o.z = __builtin_amdgcn_perm(rows[5][c >> 1], rows[4][c >> 1], sel);
    o.w = __builtin_amdgcn_perm(rows[7][c >> 1], rows[6][c >> 1], sel);
    return o;
}

// A launch covers one or more segments that share A: segment s owns its own
// B [K, n_s] and output, and grid.x runs over the strips of every segment in
// turn (strip_end is the running total). Partials of all segments share one
// fp32 buffer [ks][M][ntot], segment s at columns col0_s.
struct SkinnyArgs {
    const void *a;
    float *p;
    uint32_t m, k, ntot, nseg;
    uint32_t direct;                         // 1: one K range, narrow straight into c
    uint32_t strip_end[kSkinnyMaxSeg];
    const void *b[kSkinnyMaxSeg];
    void *c[kSkinnyMaxSeg];
    uint32_t n[kSkinnyMaxSeg], col0[kSkinnyMaxSeg];
    SkinnyNormA norm;                        // bf16: ssq non-null reads A as RmsNorm(A)
};

// Segment of this workgroup and its first strip (workgroup-uniform, picked
// from the kernel arguments with selects so nothing is indexed dynamically).
struct SegPick {
    const void *b;
    void *c;
    uint32_t n, col0, strip;
};

__device__ __forceinline__ SegPick pick_segment(const SkinnyArgs &g) {
    const uint32_t bx = blockIdx.x;
    SegPick r{g.b[0], g.c[0], g.n[0], g.col0[0], bx};
#pragma unroll
    for (int i = 1; i < kSkinnyMaxSeg; ++i)
        if (uint32_t(i) < g.nseg && bx >= g.strip_end[i - 1]) {
            r.b = g.b[i];
            r.c = g.c[i];
            r.n = g.n[i];
            r.col0 = g.col0[i];
            r.strip = bx - g.strip_end[i - 1];
        }
    return r;
}

// ---------------------------------------------------------------- bf16 ----
// MT 16-row tiles of A; each wave (chain 4 * blockIdx.y + w) takes its steps
// STEPS at a time, all of a batch's loads issued before its MFMAs.
template <int MT, int STEPS>
__global__ __launch_bounds__(256) void skinny_bf16_kernel(const SkinnyArgs g) {
    __shared__ f32x4 red[kWaves - 1][MT][8][64];
    const SegPick sg = pick_segment(g);
    const uint16_t *__restrict__ A = static_cast<const uint16_t *>(g.a);
    const uint16_t *__restrict__ B = static_cast<const uint16_t *>(sg.b);
    const uint32_t M = g.m, N = sg.n, K = g.k, S = K / 32;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, grp = lane >> 4, q = lane & 15;
    const uint32_t n0 = sg.strip * 128 + 8 * q;
    const uint32_t chain = 4 * blockIdx.y + w;
    // steps of this chain: chain, chain + 64, ...
    const uint32_t nsteps = chain < S ? (S - chain + 63) / 64 : 0;
    // All of B as one buffer range; columns past N are sent out of range,
    // where buffer loads return zero.
    const auto rb = rsrc(B, K * N * 2u);
    const auto ra = rsrc(A, M * K * 2u);   // rows >= M read zero
    const uint32_t bcol = n0 < N ? n0 * 2u : 0x80000000u;

    // RmsNorm of A on the way in: the producer's four wave sums of each of
    // this lane's rows and gamma at the lane's k values, loaded ahead of B.
    // No load sits behind a branch: a step past the chain, a row past M or an
    // absent gamma loads from an out-of-range offset (zero, no memory access),
    // so the compiler counts the loads in flight exactly and each step waits
    // only for its own.
    const bool norm = g.norm.ssq != nullptr;
    const auto rs = rsrc(g.norm.ssq, norm ? M * 16u : 0u);
    const auto rg = rsrc(g.norm.gamma, norm && g.norm.gamma ? K * 2u : 0u);
    f32x4 ssq[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
        ssq[mt] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                rs, (mt * 16 + q) * 16u, 0, 0));
    f32x4 acc[MT][8];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int c = 0; c < 8; ++c) acc[mt][c] = f32x4{0.f, 0.f, 0.f, 0.f};
    float inv[MT] = {};
    for (uint32_t t0 = 0; t0 < nsteps; t0 += STEPS) {
        u32x4 b[STEPS][8], a[STEPS][MT], gam[STEPS];
#pragma unroll
        for (int t = 0; t < STEPS; ++t) {
            const bool live = t0 + t < nsteps;
            const uint32_t kr = (chain + 64 * (t0 + t)) * 32;   // the step's first row of B
            gam[t] = __builtin_amdgcn_raw_buffer_load_b128(rg, live ? (kr + 8 * grp) * 2u : 0x80000000u,
                                                           0, 0);
            const uint32_t vo = live ? bcol + (kr + 8 * grp) * N * 2u : 0x80000000u;
#pragma unroll
            for (int r = 0; r < 8; ++r)
                b[t][r] = __builtin_amdgcn_raw_buffer_load_b128(rb, vo, int(N * 2u) * r, 0);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                a[t][mt] = __builtin_amdgcn_raw_buffer_load_b128(
                    ra, live ? ((mt * 16 + q) * K + kr + 8 * grp) * 2u : 0x80000000u, 0, 0);
        }
        if (norm) {
            // inv of each row: the four wave sums added in the standalone kernel's order
            if (!g.norm.gamma)   // no gamma: scale 1
#pragma unroll
                for (int t = 0; t < STEPS; ++t)
                    gam[t] = u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const f32x4 s = ssq[mt];
                inv[mt] = 1.0f / sqrtf((s[0] + s[1] + s[2] + s[3]) / float(K) + g.norm.eps);
            }
        }
#pragma unroll
        for (int t = 0; t < STEPS; ++t) {
            if (t0 + t < nsteps) {
                if (norm) {
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        u32x4 r;
#pragma unroll
                        for (int h = 0; h < 4; ++h) {
                            const uint32_t x = a[t][mt][h], y = gam[t][h];
                            const float lo = (__uint_as_float(x << 16) * inv[mt]) * __uint_as_float(y << 16);
                            const float hi = (__uint_as_float(x & 0xFFFF0000u) * inv[mt]) *
                                             __uint_as_float(y & 0xFFFF0000u);
                            r[h] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
                        }
                        a[t][mt] = r;
                    }
                }
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const u32x4 o = column8(b[t], c);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        acc[mt][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            __builtin_bit_cast(bf16x8, a[t][mt]), __builtin_bit_cast(bf16x8, o),
                            acc[mt][c], 0, 0, 0);
                }
            }
        }
    }

    // waves 1..3 hand their partials to wave 0 (lane-contiguous, conflict-free)
    if (w > 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int c = 0; c < 8; ++c) red[w - 1][mt][c][lane] = acc[mt][c];
    }
    __syncthreads();
    if (w != 0) return;
#pragma unroll
    for (int v = 0; v < kWaves - 1; ++v)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int c = 0; c < 8; ++c) acc[mt][c] += red[v][mt][c][lane];

    // D layout: acc[mt][c][i] is row mt*16 + 4*grp + i, column n0 + c
    if (n0 >= N) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t m = mt * 16 + 4 * grp + i;
            if (m >= M) continue;
            if (g.direct) {
                u32x4 o;
#pragma unroll
                for (int h = 0; h < 4; ++h)
                    o[h] = (__float_as_uint(acc[mt][2 * h][i]) >> 16) |
                           (__float_as_uint(acc[mt][2 * h + 1][i]) & 0xffff0000u);
                *reinterpret_cast<u32x4 *>(static_cast<uint16_t *>(sg.c) + uint64_t(m) * N + n0) = o;
            } else {
                float *p = g.p + (uint64_t(blockIdx.y) * M + m) * g.ntot + sg.col0 + n0;
                *reinterpret_cast<f32x4 *>(p) =
                    f32x4{acc[mt][0][i], acc[mt][1][i], acc[mt][2][i], acc[mt][3][i]};
                *reinterpret_cast<f32x4 *>(p + 4) =
                    f32x4{acc[mt][4][i], acc[mt][5][i], acc[mt][6][i], acc[mt][7][i]};
            }
        }
}

// ----------------------------------------------------------------- f32 ----
// MT 16-row tiles of A, STEPS 16-deep k steps per wave: KC = 4 * STEPS * 16.
// Lane (grp, q) of a step loads rows kr + 4*grp + r (r = 0..3), columns
// 4q..4q+3 of the strip, and A[m][kr + 4*grp .. kr + 4*grp + 3]; MFMA (r, c)
// pairs k-group grp with row kr + 4*grp + r in both operands.
template <int MT, int STEPS>
__global__ __launch_bounds__(256) void skinny_f32_kernel(const SkinnyArgs g) {
    constexpr uint32_t KC = kWaves * STEPS * 16;
    __shared__ f32x4 red[kWaves - 1][MT][4][64];
    const SegPick sg = pick_segment(g);
    const float *__restrict__ A = static_cast<const float *>(g.a);
    const float *__restrict__ B = static_cast<const float *>(sg.b);
    const uint32_t M = g.m, N = sg.n, K = g.k;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, grp = lane >> 4, q = lane & 15;
    const uint32_t n0 = sg.strip * 64 + 4 * q;
    const uint32_t kb0 = blockIdx.y * KC;
    const uint32_t krows = K - kb0 < KC ? K - kb0 : KC;
    const auto rb = rsrc(B + uint64_t(kb0) * N, krows * N * 4u);
    const auto ra = rsrc(A, M * K * 4u);
    const uint32_t bcol = n0 < N ? n0 * 4u : 0x80000000u;

    // steps past the range load from an out-of-range offset (no branch)
    u32x4 b[STEPS][4], a[STEPS][MT];
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
        const uint32_t kr = uint32_t(t * kWaves + w) * 16;
        const bool live = kr < krows;
        const uint32_t vo = live ? bcol + (kr + 4 * grp) * N * 4u : 0x80000000u;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            b[t][r] = __builtin_amdgcn_raw_buffer_load_b128(rb, vo, int(N * 4u) * r, 0);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
            a[t][mt] = __builtin_amdgcn_raw_buffer_load_b128(
                ra, live ? ((mt * 16 + q) * K + kb0 + kr + 4 * grp) * 4u : 0x80000000u, 0, 0);
    }
    f32x4 acc[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[mt][c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
        if (uint32_t(t * kWaves + w) * 16 < krows) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int c = 0; c < 4; ++c)
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        acc[mt][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(
                            __uint_as_float(a[t][mt][r]), __uint_as_float(b[t][r][c]), acc[mt][c],
                            0, 0, 0);
        }
    }

    if (w > 0) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int c = 0; c < 4; ++c) red[w - 1][mt][c][lane] = acc[mt][c];
    }
    __syncthreads();
    if (w != 0) return;
#pragma unroll
    for (int v = 0; v < kWaves - 1; ++v)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[mt][c] += red[v][mt][c][lane];

    if (n0 >= N) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t m = mt * 16 + 4 * grp + i;
            if (m >= M) continue;
            float *dst = g.direct ? static_cast<float *>(sg.c) + uint64_t(m) * N + n0
                                  : g.p + (uint64_t(blockIdx.y) * M + m) * g.ntot + sg.col0 + n0;
            *reinterpret_cast<f32x4 *>(dst) =
                f32x4{acc[mt][0][i], acc[mt][1][i], acc[mt][2][i], acc[mt][3][i]};
        }
}

// Sum of the ks partials in ks order; 4 consecutive outputs per thread.
template <bool kBf16>
__global__ __launch_bounds__(256) void skinny_reduce_kernel(const float *__restrict__ P,
                                                            void *__restrict__ C, uint32_t M,
                                                            uint32_t N, uint32_t KS) {
    const uint64_t quads = uint64_t(M) * N / 4;
    const uint64_t i = uint64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= quads) return;
    const uint64_t plane = uint64_t(M) * N;
    const f32x4 *p = reinterpret_cast<const f32x4 *>(P + 4 * i);
    const uint64_t step = plane / 4;
    f32x4 s = p[0];
    uint32_t ks = 1;
    for (; ks + 8 <= KS; ks += 8) {   // eight loads in flight, added in ks order
        f32x4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = p[(ks + u) * step];
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; ks < KS; ++ks) s += p[ks * step];
    if (kBf16) {
        uint2 o;
        o.x = (__float_as_uint(s[0]) >> 16) | (__float_as_uint(s[1]) & 0xffff0000u);
        o.y = (__float_as_uint(s[2]) >> 16) | (__float_as_uint(s[3]) & 0xffff0000u);
        reinterpret_cast<uint2 *>(C)[i] = o;
    } else {
        reinterpret_cast<f32x4 *>(C)[i] = s;
    }
}

int skinny_cus() {
    static const int cus = [] {
        int dev = 0, c = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
            c = 256;
        return c;
    }();
    return cus;
}

hipError_t launch_skinny(const SkinnyArgs &g, uint8_t dtype, int mt, int steps, uint32_t strips,
                         uint32_t ks, hipStream_t stream) {
    const dim3 grid(strips, ks), block(256);
#define HOLO_SKINNY(KER, MT, ST) hipLaunchKernelGGL((KER<MT, ST>), grid, block, 0, stream, g)
    if (dtype == 7) {
        if (mt == 1) {
            if (steps == 4) HOLO_SKINNY(skinny_bf16_kernel, 1, 4);
            else if (steps == 2) HOLO_SKINNY(skinny_bf16_kernel, 1, 2);
            else HOLO_SKINNY(skinny_bf16_kernel, 1, 1);
        } else if (mt == 2) {
            if (steps == 4) HOLO_SKINNY(skinny_bf16_kernel, 2, 4);
            else if (steps == 2) HOLO_SKINNY(skinny_bf16_kernel, 2, 2);
            else HOLO_SKINNY(skinny_bf16_kernel, 2, 1);
        } else {
            if (steps == 2) HOLO_SKINNY(skinny_bf16_kernel, 4, 2);
            else HOLO_SKINNY(skinny_bf16_kernel, 4, 1);
        }
    } else {
        if (mt == 1) {
            if (steps == 8) HOLO_SKINNY(skinny_f32_kernel, 1, 8);
            else if (steps == 4) HOLO_SKINNY(skinny_f32_kernel, 1, 4);
            else if (steps == 2) HOLO_SKINNY(skinny_f32_kernel, 1, 2);
            else HOLO_SKINNY(skinny_f32_kernel, 1, 1);
        } else if (mt == 2) {
            if (steps == 8) HOLO_SKINNY(skinny_f32_kernel, 2, 8);
            else if (steps == 4) HOLO_SKINNY(skinny_f32_kernel, 2, 4);
            else if (steps == 2) HOLO_SKINNY(skinny_f32_kernel, 2, 2);
            else HOLO_SKINNY(skinny_f32_kernel, 2, 1);
        } else {
            if (steps == 4) HOLO_SKINNY(skinny_f32_kernel, 4, 4);
            else if (steps == 2) HOLO_SKINNY(skinny_f32_kernel, 4, 2);
            else HOLO_SKINNY(skinny_f32_kernel, 4, 1);
        }
    }
#undef HOLO_SKINNY
    return hipGetLastError();
}

}  // namespace

// The split of a few-row MatMul: 16-row tiles of A, the k steps per wave and
// the K ranges (bf16: the groups of the summation order). For f32 it fixes
// the order of every fp32 sum (within a wave, across the four waves, then
// across K ranges in ks order), so a call and a grouped launch with the same
// plan give the same bits; for bf16 the order depends on K alone. mt = 0: the
// few-row kernels do not apply.
// f32 workgroups per CU the K split aims for: one gave config 5's decode
// step 1.068 ms against 1.091 with two (fewer partials for the epilogues to
// sum) and 1.128 with four.
constexpr uint32_t kSkinnyWgPerCu = 1;
SkinnyPlan matmul_skinny_plan(uint32_t m, uint32_t k, uint32_t n, uint8_t dtype) {
    SkinnyPlan p;
    if (m == 0 || m > 64 || k == 0 || n == 0) return p;
    const bool bf16 = dtype == 7;
    if (dtype != 7 && dtype != 8) return p;
    if (bf16 ? (n % 8 != 0 || k % 32 != 0) : (n % 4 != 0 || k % 16 != 0)) return p;
    p.mt = m <= 16 ? 1 : m <= 32 ? 2 : 4;
    p.strips = (n + (bf16 ? 127 : 63)) / (bf16 ? 128 : 64);
    if (bf16) {
        // 32-bit buffer ranges over all of A and all of B (plus the
        // out-of-range column offset 2^31 on top of a row offset)
        if (uint64_t(m) * k * 2 >= (1ull << 31) || uint64_t(k) * n * 2 >= (1ull << 31) ||
            p.strips > (1u << 31)) {
            p.mt = 0;
            return p;
        }
        const uint32_t S = k / 32, per_chain = (S + 63) / 64;
        const int max_steps = p.mt == 4 ? 2 : 4;
        p.steps = 1;
        while (p.steps < max_steps && uint32_t(p.steps) < per_chain) p.steps *= 2;
        p.ks = S / 4 + (S % 4 != 0);
        if (p.ks > 16) p.ks = 16;
        p.kc = 0;
        return p;
    }
    // k steps per wave: the most that still gives every CU its workgroups
    // (a long K range per workgroup keeps its loads streaming; a short one
    // fills the GPU when B is small)
    const int kstep = 16;
    const int max_steps = p.mt == 4 ? 4 : 8;
    p.steps = max_steps;
    while (p.steps > 1 &&
           uint64_t(p.strips) * ((k + kWaves * p.steps * kstep - 1) / (kWaves * p.steps * kstep)) <
               uint64_t(kSkinnyWgPerCu) * skinny_cus())
        p.steps /= 2;
    p.kc = kWaves * p.steps * kstep;
    // 32-bit buffer ranges: all of A, and KC rows of B (plus the out-of-range
    // column offset 2^31 on top of a row offset)
    if (uint64_t(m) * k * 4 >= (1ull << 31) || uint64_t(p.kc) * n * 4 >= (1ull << 31)) {
        p.mt = 0;
        return p;
    }
    p.ks = (k + p.kc - 1) / p.kc;
    if (p.ks > 65535 || p.strips > (1u << 31)) p.mt = 0;
    return p;
}

size_t matmul_skinny_scratch_bytes(uint32_t m, uint32_t k, uint32_t n, uint8_t dtype) {
    const SkinnyPlan p = matmul_skinny_plan(m, k, n, dtype);
    if (p.mt == 0 || p.ks <= 1) return 0;
    return size_t(p.ks) * m * n * 4;
}

bool matmul_skinny_applies(uint32_t m, uint32_t k, uint32_t n, uint8_t dtype) {
    return matmul_skinny_plan(m, k, n, dtype).mt != 0;
}

hipError_t launch_matmul_skinny(const void *a, const void *b, void *c, uint32_t m, uint32_t k,
                                uint32_t n, uint8_t dtype, void *scratch, hipStream_t stream) {
    const SkinnyPlan p = matmul_skinny_plan(m, k, n, dtype);
    if (p.mt == 0 || (p.ks > 1 && scratch == nullptr)) return hipErrorInvalidValue;
    SkinnyArgs g{};
    g.a = a;
    g.p = static_cast<float *>(scratch);
    g.m = m;
    g.k = k;
    g.ntot = n;
    g.nseg = 1;
    g.direct = p.ks <= 1;
    g.strip_end[0] = p.strips;
    g.b[0] = b;
    g.c[0] = c;
    g.n[0] = n;
    g.col0[0] = 0;
    hipError_t e = launch_skinny(g, dtype, p.mt, p.steps, p.strips, p.ks, stream);
    if (e != hipSuccess || p.ks <= 1) return e;
    const uint64_t quads = uint64_t(m) * n / 4;
    const dim3 rgrid(unsigned((quads + 255) / 256)), block(256);
    if (dtype == 7)
        hipLaunchKernelGGL(skinny_reduce_kernel<true>, rgrid, block, 0, stream, g.p, c, m, n, p.ks);
    else
        hipLaunchKernelGGL(skinny_reduce_kernel<false>, rgrid, block, 0, stream, g.p, c, m, n, p.ks);
    return hipGetLastError();
}

hipError_t launch_skinny_partials(const void *a, uint32_t m, uint32_t k, uint8_t dtype,
                                  const SkinnySegment *segs, int nseg, const SkinnyPlan &plan,
                                  float *P, hipStream_t stream, const SkinnyNormA *norm) {
    if (plan.mt == 0 || nseg < 1 || nseg > kSkinnyMaxSeg || P == nullptr) return hipErrorInvalidValue;
    if (norm && norm->ssq && dtype != 7) return hipErrorInvalidValue;
    SkinnyArgs g{};
    if (norm) g.norm = *norm;
    g.a = a;
    g.p = P;
    g.m = m;
    g.k = k;
    g.nseg = uint32_t(nseg);
    g.direct = 0;
    const uint32_t sw = dtype == 7 ? 128 : 64;
    uint32_t strips = 0, col = 0;
    for (int i = 0; i < nseg; ++i) {
        strips += (segs[i].n + sw - 1) / sw;
        g.strip_end[i] = strips;
        g.b[i] = segs[i].b;
        g.c[i] = nullptr;
        g.n[i] = segs[i].n;
        g.col0[i] = col;
        col += segs[i].n;
    }
    g.ntot = col;
    return launch_skinny(g, dtype, plan.mt, plan.steps, strips, plan.ks, stream);
}

}  // namespace holo
