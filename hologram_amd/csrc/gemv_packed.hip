// gemv_packed.hip — a few-row bf16 MatMul group (A: m <= 16 rows) over
// constant weights, each product and its epilogue in one launch.
//
// Weights in fragment order. At session load each constant B [K, N] that such
// a group reads is copied once into the order the MFMA consumes it
// (launch_pack_b): tile j (16 columns) by step s (32 k) is one 1 KiB block in
// which lane (grp, q) holds B[32s + 8grp + e][16j + q] for e = 0..7; the blocks
// of a tile are consecutive in step order, the tiles in column order. One
// wave's load of a block is 1 KiB of consecutive bytes, so a workgroup can own
// a 16-column tile over the whole of K without the short strided rows a
// row-major 16-column strip would read.
//
// Work split. A workgroup owns one unit over the whole of K: a 16-column tile;
// for a SwiGLU product the gate tile and the up tile at the same columns; for
// the head-wise epilogues (rotary embedding, int8 append) every tile of one
// head. No partial leaves the workgroup, so the epilogue runs in the same
// launch. Its sixteen wavefronts are the sixteen groups of the few-row
// product's fixed summation order (gemm_skinny.hip): chain c = 0..63
// accumulates the steps s = c, c + 64, ... in ascending order on the MFMA, a
// group adds its four chains in order, the groups are added in order through
// LDS. The split-K kernels compute the same sums with one workgroup per group,
// so both give the same bits.
//
// RmsNorm of A. A group that reads A through a fused RmsNorm computes each
// row's sum of squares itself, as the standalone bf16 RmsNorm kernel
// (decoder_ops.hip, rmsnorm_vec_row) does: thread t of 256 sums the squares of
// the row's 16-byte vectors t + 256u in order, each wave reduces by a xor
// tree, the four wave sums are added in order. For each row, four of the
// sixteen wavefronts play those four waves exactly.
#include <hip/hip_runtime.h>

#include <math.h>

#include <type_traits>

#include "epilogue_math.h"
#include "holo_device.h"
#include "holo_kernels.h"

namespace holo {
namespace {

using namespace epi;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kPkWaves = 16;            // = the groups of the summation order

constexpr uint32_t kNoLoad = 0x80000000u;   // an offset past every buffer range

struct PackedArgs {
    const uint16_t *a;
    const uint16_t *gamma;              // norm: [k] (null: the identity)
    float eps;
    uint32_t norm;                      // A read as RmsNorm(A)
    uint32_t m, k, nseg;
    uint32_t tpu;                       // tiles per element-wise unit (pairs: tile pairs)
    uint32_t tw;                        // element-wise tile width: 16 or 8 columns
    uint32_t unit_end[kSkinnyMaxSeg];   // running total of units per segment
    const u32x4 *bp[kSkinnyMaxSeg];     // each segment's B in fragment order
    EpiSeg seg[kSkinnyMaxSeg];
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, int(bytes), 0x00020000);
}

// The launch's arguments read in place from the kernel argument segment:
// indexing the by-value struct with a workgroup-uniform segment number would
// make the compiler copy the whole struct to scratch memory; through this
// pointer the same fields are scalar loads.
typedef const __attribute__((address_space(4))) PackedArgs *KArgs;
typedef const __attribute__((address_space(4))) EpiSeg *KSeg;

__device__ __forceinline__ KArgs kargs() { return (KArgs)__builtin_amdgcn_kernarg_segment_ptr(); }

// Segment of this workgroup and its unit index.
__device__ __forceinline__ int pick_unit(KArgs g, uint32_t *unit) {
    int s = 0;
    uint32_t u0 = 0;
#pragma unroll
    for (int i = 1; i < kSkinnyMaxSeg; ++i)
        if (uint32_t(i) < g->nseg && blockIdx.x >= g->unit_end[i - 1]) {
            s = i;
            u0 = g->unit_end[i - 1];
        }
    *unit = blockIdx.x - u0;
    return s;
}

// The fields base_value reads.
__device__ __forceinline__ EpiSeg value_form(KSeg s) {
    EpiSeg e;
    e.base = s->base;
    e.act = s->act;
    e.lut = s->lut;
    return e;
}

// NT: most tiles a unit of this launch holds; SPC: most steps a chain holds
// (ceil(K / 32 / 64)); NORM: A is read through the RmsNorm (needs LDSA);
// LDSA: A is staged in LDS (dynamic shared memory, M rows of K + 8
// elements); MP: passes of four rows over A's rows when staging.
//
// Every global load of the workgroup goes out before the first wait, none
// behind a branch (an unused load reads an out-of-range offset: zero, no
// memory access): the epilogue's side operands, A (or its rows for the LDS
// copy) and gamma, then B. A and gamma arrive first (loads complete in
// order), so the LDS copy and the norm's statistics overlap B's stream.
template <int NT, int SPC, bool NORM, bool LDSA, int MP>
__device__ __forceinline__ void gemv_packed_body(const PackedArgs &g) {
    __shared__ f32x4 red[kPkWaves][NT][64];
    __shared__ float ssq_l[16][4];
    extern __shared__ u32x4 alds[];           // LDSA: row r at r * (K / 8 + 1) vectors
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, grp = lane >> 4, q = lane & 15;
    const uint32_t M = g.m, K = g.k, S = K / 32, nv = K / 8, pitch = nv + 1;
    const KArgs ka = kargs();
    uint32_t unit;
    const int si = pick_unit(ka, &unit);
    const KSeg sg = &ka->seg[si];
    const int pair = sg->pair;
    const int pi = pair < 0 ? si : pair;
    const KSeg pr = &ka->seg[pi];
    const uint32_t head_dim = sg->head_dim;
    const uint32_t n = sg->n;
    // A rotary head-wise segment runs in 16-column rope tiles: its weights are
    // packed so that tile column q < 8 is head element 8t + q and q >= 8 its
    // rotate-half partner 8t + q - 8 + D/2, so the pair meets in lanes q and
    // q ^ 8 of one workgroup.
    const bool rtile = head_dim != 0;
    // B: tpu consecutive tiles of the segment (rb0); for a pair, the up
    // segment's tiles at the same columns follow (rb1). Tiles past the unit or
    // the segment fall past the ranges. An element-wise tile of 8 columns is a
    // 512-byte block a step (lanes q < 8 of the MFMA's B operand; the others
    // read zero).
    const uint32_t tpu = rtile ? 1u : g.tpu;
    const uint32_t tw = rtile ? 16u : g.tw, blk = tw * 64u;      // columns, bytes a block
    const uint32_t ts = S * blk;                                   // bytes a tile
    const uint32_t first = unit * tpu;
    const uint32_t left = n / tw - first;                          // the segment's tiles from `first`
    const uint32_t own = left < tpu ? left : tpu;
    const auto rb0 = rsrc(reinterpret_cast<const uint8_t *>(ka->bp[si]) + uint64_t(first) * ts, own * ts);
    const auto rb1 = rsrc(reinterpret_cast<const uint8_t *>(ka->bp[pi]) + uint64_t(first) * ts,
                          pair >= 0 ? own * ts : 0u);
    const bool qin = uint32_t(q) < tw;                              // this lane's column is in the tile
    const auto ra = rsrc(g.a, M * K * 2u);   // rows >= M read zero

    // (1) the epilogue's side operands: wave t < own finishes tile `first +
    // t`, lane (grp, q) holding rows 4grp + i at its column ecol (a rope
    // tile's columns are the head's pairs, see above). ra_: the residual; rb_:
    // the pair's residual, or a rope tile's cos; rs_: a rope tile's sin (a
    // rope tile has no pair).
    const EpiSeg vf = value_form(sg), pf = value_form(pr);
    const uint32_t rt_h = rtile ? unit / (head_dim / 16) : 0, rt_t = rtile ? unit % (head_dim / 16) : 0;
    const uint32_t ecol = rtile ? rt_h * head_dim + 8 * rt_t + (q < 8 ? uint32_t(q) : uint32_t(q) - 8 + head_dim / 2)
                                : tw * (first + uint32_t(w)) + uint32_t(q);
    float ra_[4] = {}, rb_[4] = {}, rs_[4] = {};
    {
        const bool mine = uint32_t(w) < own && qin;
        const auto rra = opt_rsrc(sg->residual, has_residual(vf) && mine);
        const auto rrb = rtile ? opt_rsrc(sg->cos, mine) : opt_rsrc(pr->residual, pair >= 0 && has_residual(pf) && mine);
        const auto rrs = opt_rsrc(sg->sin, rtile && mine);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t m = 4 * grp + i;
            const uint64_t e = m < M && qin ? uint64_t(m) * n + ecol : uint64_t(kNoLoad) / 2;
            ra_[i] = opt_load<true>(rra, e);
            rb_[i] = opt_load<true>(rrb, e);
            rs_[i] = opt_load<true>(rrs, e);
        }
    }

    // (2) A. Staged: thread tau = 256p + t of pass p holds the vectors
    // t + 256u of row 4p' + tau / 256 (p' the pass), exactly the vectors the
    // standalone RmsNorm kernel's thread t sums for that row, in the same
    // waves. Direct: each lane loads its own fragments (chain 4w + cc, step
    // 4w + cc + 64i, row q, k 32s + 8grp .. + 7).
    constexpr int kPass = MP;                // passes of four rows
    constexpr int kVec = SPC;                // vectors a thread per row (K <= 2048 SPC)
    const uint32_t t256 = threadIdx.x & 255, r0 = threadIdx.x >> 8;
    u32x4 xv[LDSA ? kPass : 1][kVec], gv[LDSA && NORM ? kVec : 1];
    u32x4 a[LDSA ? 1 : 4][SPC];
    auto load_a = [&]() {
        if constexpr (!LDSA) {
#pragma unroll
            for (int cc = 0; cc < 4; ++cc)
#pragma unroll
                for (int i = 0; i < SPC; ++i) {
                    const uint32_t s = uint32_t(4 * w + cc) + 64 * i;
                    a[cc][i] = __builtin_amdgcn_raw_buffer_load_b128(
                        ra, s < S ? (q * K + 32 * s + 8 * grp) * 2u : kNoLoad, 0, 0);
                }
        }
    };
    if constexpr (LDSA) {
#pragma unroll
        for (int p = 0; p < kPass; ++p)
#pragma unroll
            for (int u = 0; u < kVec; ++u) {
                const uint32_t r = 4 * p + r0, v = t256 + 256 * u;
                xv[p][u] = __builtin_amdgcn_raw_buffer_load_b128(ra, r < M && v < nv ? (r * K + 8 * v) * 2u : kNoLoad,
                                                                 0, 0);
            }
        if constexpr (NORM) {
            const auto rg = rsrc(g.gamma, g.gamma ? K * 2u : 0u);
#pragma unroll
            for (int u = 0; u < kVec; ++u) {
                const uint32_t v = t256 + 256 * u;
                gv[u] = __builtin_amdgcn_raw_buffer_load_b128(rg, v < nv ? 16u * v : kNoLoad, 0, 0);
            }
        }
    } else {
        load_a();
    }
    // (3) B at this wave's steps
    u32x4 b[4][SPC][NT];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc)
#pragma unroll
        for (int i = 0; i < SPC; ++i) {
            const uint32_t s = uint32_t(4 * w + cc) + 64 * i;
            const bool live = s < S;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const bool up = pair >= 0 && uint32_t(t) >= tpu;   // a pair's up tile
                const uint32_t tt = up ? uint32_t(t) - tpu : uint32_t(t);
                const uint32_t li = tw == 16 ? uint32_t(lane) : uint32_t(grp) * 8 + uint32_t(q);
                const uint32_t off = live && qin ? tt * ts + s * blk + li * 16u : kNoLoad;
                b[cc][i][t] = __builtin_amdgcn_raw_buffer_load_b128(up ? rb1 : rb0, off, 0, 0);
            }
        }

    // (4) the LDS copy of A: the norm's statistics (the standalone kernel's
    // per-thread sums, xor tree per wave, four wave sums in order), then each
    // vector normalized as the standalone kernel writes it
    if constexpr (LDSA) {
        if constexpr (NORM) {
#pragma unroll
            for (int p = 0; p < kPass; ++p) {
                const uint32_t r = 4 * p + r0;
                float ss = 0.0f;
#pragma unroll
                for (int u = 0; u < kVec; ++u)
#pragma unroll
                    for (int h = 0; h < 4; ++h) {
                        const float lo = __uint_as_float(xv[p][u][h] << 16),
                                    hi = __uint_as_float(xv[p][u][h] & 0xFFFF0000u);
                        ss = fmaf(lo, lo, ss);
                        ss = fmaf(hi, hi, ss);
                    }
#pragma unroll
                for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
                if (lane == 0 && r < 16) ssq_l[r][t256 >> 6] = ss;
            }
            __syncthreads();
#pragma unroll
            for (int p = 0; p < kPass; ++p) {
                const uint32_t r = 4 * p + r0;
                if (r >= M) continue;
                const float inv =
                    1.0f / sqrtf((ssq_l[r][0] + ssq_l[r][1] + ssq_l[r][2] + ssq_l[r][3]) / float(K) + g.eps);
#pragma unroll
                for (int u = 0; u < kVec; ++u) {
                    const uint32_t v = t256 + 256 * u;
                    if (v >= nv) continue;
                    const u32x4 y = g.gamma ? gv[u] : u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
                    u32x4 o;
#pragma unroll
                    for (int h = 0; h < 4; ++h) {
                        const uint32_t x = xv[p][u][h];
                        const float lo = (__uint_as_float(x << 16) * inv) * __uint_as_float(y[h] << 16);
                        const float hi = (__uint_as_float(x & 0xFFFF0000u) * inv) * __uint_as_float(y[h] & 0xFFFF0000u);
                        o[h] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
                    }
                    alds[r * pitch + v] = o;
                }
            }
        } else {
#pragma unroll
            for (int p = 0; p < kPass; ++p) {
                const uint32_t r = 4 * p + r0;
                if (r >= M) continue;
#pragma unroll
                for (int u = 0; u < kVec; ++u) {
                    const uint32_t v = t256 + 256 * u;
                    if (v < nv) alds[r * pitch + v] = xv[p][u];
                }
            }
        }
        __syncthreads();
    }

    // (5) this wave's group: four chains, each over its steps in order, then
    // the chains added in order
    f32x4 grp_sum[NT];
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
        u32x4 av[SPC];
#pragma unroll
        for (int i = 0; i < SPC; ++i) {
            const uint32_t s = uint32_t(4 * w + cc) + 64 * i;
            if constexpr (LDSA) {   // rows >= M are zero
                const u32x4 x = alds[(q < int(M) ? uint32_t(q) : 0u) * pitch + (s < S ? 4 * s + grp : 0u)];
                av[i] = q < int(M) ? x : u32x4{0u, 0u, 0u, 0u};
            } else {
                av[i] = a[cc][i];
            }
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            f32x4 c = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < SPC; ++i)
                if (uint32_t(4 * w + cc) + 64 * i < S)
                    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, av[i]),
                                                                __builtin_bit_cast(bf16x8, b[cc][i][t]), c,
                                                                0, 0, 0);
            if (cc == 0)
                grp_sum[t] = c;
            else
                grp_sum[t] += c;
        }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) red[w][t][lane] = grp_sum[t];
    __syncthreads();

    // (6) the groups added in order, then the epilogue
    const uint32_t groups = S / 4 + (S % 4 != 0), G = groups > 16 ? 16 : groups;
    {
        // wave t < own: tile `first + t` (and its up tile at t + tpu)
        if (uint32_t(w) >= own) return;
        const uint32_t wt = uint32_t(w) < NT ? uint32_t(w) : 0;
        const uint32_t tu = wt + tpu < NT ? wt + tpu : 0;
        f32x4 va = red[0][wt][lane], vb = red[0][tu][lane];
        for (uint32_t v = 1; v < G; ++v) {
            va += red[v][wt][lane];
            if (pair >= 0) vb += red[v][tu][lane];
        }
        if (rtile) {
            // rotate-half: y = x c - x' s (first half), x c + x' s (second),
            // x' the partner in lane q ^ 8, as the standalone rotary kernel
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t m = 4 * grp + i;
                const float x = base_value<true>(vf, va[i], ra_[i]);
                const float xp = __shfl_xor(x, 8, 64);
                const float y = bf2f(f2bf(q < 8 ? x * rb_[i] - xp * rs_[i] : x * rb_[i] + xp * rs_[i]));
                if (m >= M) continue;
                const uint64_t e = uint64_t(m) * n + ecol;
                if (sg->out) store<true>(sg->out, e, x);
                if (sg->rope_out) store<true>(sg->rope_out, e, y);
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t m = 4 * grp + i;
            if (m >= M || !qin) continue;
            const uint64_t e = uint64_t(m) * n + ecol;
            const float xa = base_value<true>(vf, va[i], ra_[i]);
            if (sg->out) store<true>(sg->out, e, xa);
            if (pair >= 0) {
                const float xb = base_value<true>(pf, vb[i], rb_[i]);
                if (pr->out) store<true>(pr->out, e, xb);
                store<true>(sg->mul_out, e, xa * xb);
            }
        }
        return;
    }
}

// One workgroup of sixteen waves per CU at a time, or two (at most 64
// registers a lane: a workgroup's latency then overlaps the other's stream).
template <int NT, int SPC, bool NORM, bool LDSA, int MP>
__global__ __launch_bounds__(1024) void gemv_packed_kernel(const PackedArgs g) {
    gemv_packed_body<NT, SPC, NORM, LDSA, MP>(g);
}
template <int NT, int SPC, bool NORM, bool LDSA, int MP>
__global__ __launch_bounds__(1024) __attribute__((amdgpu_waves_per_eu(8, 8))) void gemv_packed2_kernel(
    const PackedArgs g) {
    gemv_packed_body<NT, SPC, NORM, LDSA, MP>(g);
}

// B [K, N] row-major -> fragment order; one 16-byte block lane per thread.
// Tile width tw = 16: block (j, s) is 64 lanes (grp, q) holding B[32s + 8grp
// + e][16j + q]; tw = 8: 32 lanes (grp, q < 8) holding B[32s + 8grp + e][8j + q];
// rope_d > 0 (tw 16): the columns of rope tiles over heads of rope_d.
__global__ __launch_bounds__(256) void pack_b_kernel(const uint16_t *__restrict__ B,
                                                     uint8_t *__restrict__ Bp, uint32_t K, uint32_t N,
                                                     uint32_t tw, uint32_t rope_d) {
    const uint32_t S = K / 32, lanes = 4 * tw;
    const uint64_t ts = uint64_t(S) * tw * 64;
    const uint64_t total = uint64_t(N / tw) * S * lanes;
    for (uint64_t idx = uint64_t(blockIdx.x) * 256 + threadIdx.x; idx < total;
         idx += uint64_t(gridDim.x) * 256) {
        const uint32_t ln = uint32_t(idx % lanes), grp = ln / tw, q = ln % tw;
        const uint64_t js = idx / lanes;
        const uint64_t s = js % S, j = js / S;
        // rope_d: tile j is rope tile t of head h, its columns the head's
        // elements 8t + q (q < 8) and their rotate-half partners
        const uint64_t hj = rope_d ? j / (rope_d / 16) : 0, tj = rope_d ? j % (rope_d / 16) : 0;
        const uint64_t col = rope_d ? hj * rope_d + 8 * tj + (q < 8 ? q : q - 8 + rope_d / 2)
                                    : uint64_t(tw) * j + q;
        const uint64_t row0 = 32 * s + 8 * grp;
        u32x4 o;
#pragma unroll
        for (int h = 0; h < 4; ++h)
            o[h] = uint32_t(B[(row0 + 2 * h) * N + col]) | (uint32_t(B[(row0 + 2 * h + 1) * N + col]) << 16);
        *reinterpret_cast<u32x4 *>(Bp + j * ts + s * tw * 64 + ln * 16) = o;
    }
}

}  // namespace

// Tiles one unit of a segment holds (0: no unit of its own), at tpu tiles
// (pairs: tile pairs) of tw columns per element-wise unit; and the segment's
// units.
uint32_t packed_unit_tiles(const EpiSeg &s, uint32_t tpu) {
    if (s.skip) return 0;
    if (s.head_dim) return 1;   // a rope tile
    return s.pair >= 0 ? 2 * tpu : tpu;
}
uint32_t packed_units(const EpiSeg &s, uint32_t tpu, uint32_t tw) {
    if (s.skip) return 0;
    if (s.head_dim) return s.n / 16;
    return (s.n / tw + tpu - 1) / tpu;
}

// A staged in LDS: M rows of K + 8 elements, within the default dynamic LDS.
constexpr uint32_t kMaxDynLds = 65536;
uint32_t packed_lds_bytes(uint32_t m, uint32_t k) { return m * (k / 8 + 1) * 16; }

bool packed_group_applies(uint32_t m, uint32_t k, const EpiSeg *segs, int nseg, bool norm) {
    // At most two 32-k steps a chain (K <= 4096): four (K = 8192, Wd) would
    // hold a chain's B and A operands in 128 registers at 1024 threads only by
    // spilling, and a workgroup owning all of such a K also reads the whole of
    // A (as many bytes as its weights), so K beyond 4096 stays split-K.
    if (m == 0 || m > 16 || k == 0 || k % 32 != 0 || k > 4096 || nseg < 1 || nseg > kSkinnyMaxSeg)
        return false;
    // the norm is taken on the LDS copy of A
    if (norm && packed_lds_bytes(m, k) > kMaxDynLds) return false;
    // Where a workgroup owning all of K loses to the split-K launch and its
    // epilogue (measured per decode shape on one box, weights streamed from
    // HBM): more than 1024 sixteen-column tiles (an LM head of 32000 columns:
    // 35.9 against 34.1 us), and the int8 append, whose row maximum needs a
    // whole head in one workgroup (q/k/v: 11.3 against 9.7 us). It wins where
    // the epilogue's launch is a large share: Wo + residual 6.5 against 7.7
    // us, gate/up + SwiGLU 20.4 against 21.3 us.
    if (uint64_t(m) * k * 2 >= (1ull << 31)) return false;
    uint32_t units = 0, tiles = 0;
    for (int i = 0; i < nseg; ++i) {
        const EpiSeg &s = segs[i];
        if (s.n == 0 || s.n % 8 != 0 || uint64_t(k) * s.n * 2 >= (1ull << 31) ||
            uint64_t(m) * s.n * 2 >= (1ull << 31) || s.quant)
            return false;
        if (s.head_dim) {   // rope tiles
            if (!s.rope || !(s.head_dim == 16 || s.head_dim == 32 || s.head_dim == 64 || s.head_dim == 128) ||
                s.n % s.head_dim != 0 || s.pair >= 0)
                return false;
        }
        if (s.pair >= 0) {
            if (s.pair >= nseg || s.pair == i || segs[s.pair].n != s.n || segs[s.pair].head_dim) return false;
        }
        units += packed_units(s, 1, 16);
        tiles += s.n / 16 + (s.n % 16 != 0);
    }
    return units > 0 && tiles <= 1024;
}

hipError_t launch_packed_group(const PackedGroup &pg, hipStream_t stream) {
    if (!packed_group_applies(pg.m, pg.k, pg.seg, pg.nseg, pg.norm) || pg.a == nullptr)
        return hipErrorInvalidValue;
    PackedArgs g{};
    g.a = static_cast<const uint16_t *>(pg.a);
    g.gamma = pg.gamma;
    g.eps = pg.eps;
    g.norm = pg.norm ? 1u : 0u;
    g.m = pg.m;
    g.k = pg.k;
    g.nseg = uint32_t(pg.nseg);
    const uint32_t spc = (pg.k / 32 + 63) / 64;
    const uint32_t spc_t = spc <= 1 ? 1 : spc <= 2 ? 2 : 4;
    // element-wise tile width: as the weights were packed (launch_pack_b)
    const uint32_t tw = pg.tw == 8 ? 8u : 16u;
    // tiles per element-wise unit: the most (up to 4) that keeps every unit's
    // B in registers and leaves at least one workgroup a CU (fewer, larger
    // units pay each workgroup's fixed latency fewer times)
    constexpr uint32_t kMinUnits = 256;
    uint32_t tpu = pg.tpu;
    if (tpu == 0) {
        tpu = 1;
        for (uint32_t c = 2; c <= 4; c *= 2) {
            uint32_t units = 0, nt = 1;
            for (int i = 0; i < pg.nseg; ++i) {
                units += packed_units(pg.seg[i], c, tw);
                const uint32_t t = packed_unit_tiles(pg.seg[i], c);
                nt = t > nt ? t : nt;
            }
            if (nt * spc_t <= 4 && units >= kMinUnits) tpu = c;
        }
    }
    g.tpu = tpu;
    g.tw = tw;
    uint32_t units = 0, nt = 1;
    for (int i = 0; i < pg.nseg; ++i) {
        const EpiSeg &s = pg.seg[i];
        if (pg.bp[i] == nullptr) return hipErrorInvalidValue;
        g.bp[i] = static_cast<const u32x4 *>(pg.bp[i]);
        g.seg[i] = s;
        const uint32_t t = packed_unit_tiles(s, tpu);
        nt = t > nt ? t : nt;
        units += packed_units(s, tpu, tw);
        g.unit_end[i] = units;
    }
    // the kernels are instantiated for at most two steps a chain (K <= 4096)
    if (spc_t > 2 || nt * spc_t > 4) return hipErrorInvalidValue;
    const uint32_t lds = packed_lds_bytes(pg.m, pg.k);
    const bool ldsa = lds <= kMaxDynLds && spc_t <= 2;
    if (g.norm && !ldsa) return hipErrorInvalidValue;
    const dim3 grid(units), block(1024);
    // two workgroups a CU (the compiler then holds a lane to 64 registers,
    // spilling) only when asked: one measured faster on every decode shape
    const bool two = pg.occupancy == 2 && nt == 1 && spc_t == 1;
    const int mp = pg.m > 8 ? 4 : 2;
    auto go = [&](auto nt_c, auto spc_c) {
        constexpr int NT = decltype(nt_c)::value, SPC = decltype(spc_c)::value;
        if (!ldsa) {
            hipLaunchKernelGGL((gemv_packed_kernel<NT, SPC, false, false, 1>), grid, block, 0, stream, g);
            return;
        }
        auto with = [&](auto norm_c, auto mp_c) {
            constexpr bool NORM = decltype(norm_c)::value;
            constexpr int MP = decltype(mp_c)::value;
            if constexpr (NT == 1 && SPC == 1) {
                if (two) {
                    hipLaunchKernelGGL((gemv_packed2_kernel<NT, SPC, NORM, true, MP>), grid, block, lds, stream, g);
                    return;
                }
            }
            hipLaunchKernelGGL((gemv_packed_kernel<NT, SPC, NORM, true, MP>), grid, block, lds, stream, g);
        };
        using T = std::true_type;
        using F = std::false_type;
        using I2 = std::integral_constant<int, 2>;
        using I4 = std::integral_constant<int, 4>;
        if (g.norm) {
            if (mp == 4) with(T{}, I4{});
            else with(T{}, I2{});
        } else {
            if (mp == 4) with(F{}, I4{});
            else with(F{}, I2{});
        }
    };
    using C1 = std::integral_constant<int, 1>;
    using C2 = std::integral_constant<int, 2>;
    using C4 = std::integral_constant<int, 4>;
    if (nt <= 1) {
        if (spc_t == 1) go(C1{}, C1{});
        else go(C1{}, C2{});
    } else if (nt <= 2) {
        if (spc_t == 1) go(C2{}, C1{});
        else go(C2{}, C2{});
    } else {
        go(C4{}, C1{});
    }
    return hipGetLastError();
}

hipError_t launch_pack_b(const void *b, void *bp, uint32_t k, uint32_t n, uint32_t tw, uint32_t rope_d,
                         hipStream_t stream) {
    if (k == 0 || n == 0 || k % 32 != 0 || (tw != 8 && tw != 16) || n % tw != 0) return hipErrorInvalidValue;
    if (rope_d && (tw != 16 || rope_d % 16 != 0 || n % rope_d != 0)) return hipErrorInvalidValue;
    const uint64_t total = uint64_t(n / tw) * (k / 32) * 4 * tw;
    uint64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(pack_b_kernel, dim3(unsigned(blocks)), dim3(256), 0, stream,
                       static_cast<const uint16_t *>(b), static_cast<uint8_t *>(bp), k, n, tw, rope_d);
    return hipGetLastError();
}

uint64_t packed_b_bytes(uint32_t k, uint32_t n, uint32_t tw) {
    return uint64_t(n / tw) * uint64_t(k / 32) * tw * 64;
}

// Element-wise tile width for a group: 8 columns when a product's width is
// not a multiple of 16, or when 16-column units would leave the GPU
// under-filled (fewer workgroups than CUs); else 16. Head-wise segments always
// use 16 (a head is whole tiles).
uint32_t packed_tile_width(uint32_t m, uint32_t k, const EpiSeg *segs, int nseg) {
    (void)m;
    (void)k;
    uint32_t units = 0;
    bool heads = false, odd = false;
    for (int i = 0; i < nseg; ++i) {
        if (segs[i].skip) continue;
        units += segs[i].head_dim ? 0 : (segs[i].n + 15) / 16;
        heads = heads || segs[i].head_dim;
        odd = odd || (!segs[i].head_dim && segs[i].n % 16 != 0);
    }
    return odd || (!heads && units < 256) ? 8u : 16u;
}

}  // namespace holo
