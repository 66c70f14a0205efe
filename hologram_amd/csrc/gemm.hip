// gemm.hip — C = A * B on MFMA (row-major A[M,K], B[K,N], C[M,N]).
//
// The reference MatMul (crates/hologram-compute/src/cpu/float_kernels.rs:298-399)
// accumulates in f32; bf16 operands are exact in f32, and the bf16 result is
// narrowed by truncation (write_bf16, src/cpu/dtype.rs:75-79). Here:
//   bf16: v_mfma_f32_16x16x32_bf16 (fp32 accumulate), truncating store
//   f32 : v_mfma_f32_16x16x4_f32
// Workgroup tile 32*WT square (four wavefronts, 16*WT square each as WT x WT
// MFMA tiles): 128 (WT = 4), or 64 (WT = 2) when 128-tiles would leave CUs
// idle. K staged through LDS in double-buffered slabs: the next slab's global
// loads are issued before the current slab's MFMAs.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "holo_device.h"
#include "holo_kernels.h"

namespace holo {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;

// ---------------------------------------------------------------- bf16 ----
// LDS: A slab [BM][BK + pad], B slab [BK][BN + pad] (both as u16).
constexpr int BK16 = 64;
constexpr int APAD16 = 8, BPAD16 = 8;

template <bool kFast, int BM>
__device__ __forceinline__ void load_slab_bf16(const uint16_t *__restrict__ A,
                                               const uint16_t *__restrict__ B, uint32_t M,
                                               uint32_t N, uint32_t K, uint32_t m0, uint32_t n0,
                                               uint32_t k0, uint4 *ra, uint4 *rb) {
    constexpr int BN = BM, kChunks = BM / 32;   // 16-byte chunks per thread per operand
    const int t = threadIdx.x;
    // A: BM x BK16 u16 in chunks of 8
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
        const int c = t + i * kThreads;
        const int r = c / (BK16 / 8), kc = (c % (BK16 / 8)) * 8;
        const uint32_t gm = m0 + r, gk = k0 + kc;
        if (kFast) {
            ra[i] = gm < M ? *reinterpret_cast<const uint4 *>(A + uint64_t(gm) * K + gk)
                           : make_uint4(0, 0, 0, 0);
        } else {
            uint16_t v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)
                v[e] = (gm < M && gk + e < K) ? A[uint64_t(gm) * K + gk + e] : uint16_t(0);
            ra[i] = make_uint4(v[0] | (uint32_t(v[1]) << 16), v[2] | (uint32_t(v[3]) << 16),
                               v[4] | (uint32_t(v[5]) << 16), v[6] | (uint32_t(v[7]) << 16));
        }
    }
    // B: BK16 x BN u16 in chunks of 8 along n
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
        const int c = t + i * kThreads;
        const int r = c / (BN / 8), nc = (c % (BN / 8)) * 8;
        const uint32_t gk = k0 + r, gn = n0 + nc;
        if (kFast) {
            rb[i] = gn < N ? *reinterpret_cast<const uint4 *>(B + uint64_t(gk) * N + gn)
                           : make_uint4(0, 0, 0, 0);
        } else {
            uint16_t v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)
                v[e] = (gk < K && gn + e < N) ? B[uint64_t(gk) * N + gn + e] : uint16_t(0);
            rb[i] = make_uint4(v[0] | (uint32_t(v[1]) << 16), v[2] | (uint32_t(v[3]) << 16),
                               v[4] | (uint32_t(v[5]) << 16), v[6] | (uint32_t(v[7]) << 16));
        }
    }
}

template <int BM>
__device__ __forceinline__ void store_slab_bf16(uint16_t (*As)[BK16 + APAD16],
                                                uint16_t (*Bs)[BM + BPAD16], const uint4 *ra,
                                                const uint4 *rb) {
    constexpr int BN = BM, kChunks = BM / 32;
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
        const int c = t + i * kThreads;
        const int r = c / (BK16 / 8), kc = (c % (BK16 / 8)) * 8;
        *reinterpret_cast<uint4 *>(&As[r][kc]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
        const int c = t + i * kThreads;
        const int r = c / (BN / 8), nc = (c % (BN / 8)) * 8;
        *reinterpret_cast<uint4 *>(&Bs[r][nc]) = rb[i];
    }
}

// kF16: f16 operands on v_mfma_f32_16x16x32_f16 (products exact in f32, f32
// accumulation), each result narrowed with the reference's f16 rounding
// (write_float, src/cpu/dtype.rs:121-153); the lowp MatMul serves f16 as it
// serves bf16 (float_kernels.rs:356-392).
template <bool kFast, int WT, bool kF16>
__device__ __forceinline__ void gemm16_tile(const uint16_t *__restrict__ A,
                                            const uint16_t *__restrict__ B,
                                            uint16_t *__restrict__ C, uint32_t M, uint32_t N,
                                            uint32_t K) {
    constexpr int BM = 32 * WT, BN = BM;
    __shared__ uint16_t As[2][BM][BK16 + APAD16];
    __shared__ uint16_t Bs[2][BK16][BN + BPAD16];

    const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm = (wave >> 1) * 16 * WT, wn = (wave & 1) * 16 * WT;
    const int lr = lane & 15, lg = lane >> 4;

    f32x4 acc[WT][WT];
#pragma unroll
    for (int i = 0; i < WT; ++i)
#pragma unroll
        for (int j = 0; j < WT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const uint32_t nk = (K + BK16 - 1) / BK16;
    uint4 ra[BM / 32], rb[BM / 32];
    load_slab_bf16<kFast, BM>(A, B, M, N, K, m0, n0, 0, ra, rb);
    store_slab_bf16<BM>(As[0], Bs[0], ra, rb);
    __syncthreads();

    for (uint32_t s = 0; s < nk; ++s) {
        const int cur = s & 1;
        if (s + 1 < nk) load_slab_bf16<kFast, BM>(A, B, M, N, K, m0, n0, (s + 1) * BK16, ra, rb);
#pragma unroll
        for (int kk = 0; kk < BK16; kk += 32) {
            bf16x8 af[WT], bfr[WT];
#pragma unroll
            for (int i = 0; i < WT; ++i)
                af[i] = *reinterpret_cast<const bf16x8 *>(&As[cur][wm + i * 16 + lr][kk + lg * 8]);
#pragma unroll
            for (int j = 0; j < WT; ++j) {
                uint16_t v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = Bs[cur][kk + lg * 8 + e][wn + j * 16 + lr];
                bfr[j] = *reinterpret_cast<const bf16x8 *>(v);
            }
#pragma unroll
            for (int i = 0; i < WT; ++i)
#pragma unroll
                for (int j = 0; j < WT; ++j) {
                    if constexpr (kF16)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            __builtin_bit_cast(f16x8, af[i]), __builtin_bit_cast(f16x8, bfr[j]),
                            acc[i][j], 0, 0, 0);
                    else
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
                }
        }
        if (s + 1 < nk) store_slab_bf16<BM>(As[cur ^ 1], Bs[cur ^ 1], ra, rb);
        __syncthreads();
    }

    // D layout: lane holds rows 4*lg + r, column lr of each 16x16 tile
#pragma unroll
    for (int i = 0; i < WT; ++i)
#pragma unroll
        for (int j = 0; j < WT; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t gm = m0 + wm + i * 16 + lg * 4 + r, gn = n0 + wn + j * 16 + lr;
                if (gm < M && gn < N)
                    C[uint64_t(gm) * N + gn] = kF16 ? f32_to_f16_bits(acc[i][j][r])
                                                    : uint16_t(__float_as_uint(acc[i][j][r]) >> 16);
            }
}

template <bool kFast, int WT>
__global__ __launch_bounds__(kThreads) void gemm_bf16_kernel(const uint16_t *__restrict__ A,
                                                            const uint16_t *__restrict__ B,
                                                            uint16_t *__restrict__ C, uint32_t M,
                                                            uint32_t N, uint32_t K) {
    gemm16_tile<kFast, WT, false>(A, B, C, M, N, K);
}

template <bool kFast, int WT>
__global__ __launch_bounds__(kThreads) void gemm_f16_kernel(const uint16_t *__restrict__ A,
                                                           const uint16_t *__restrict__ B,
                                                           uint16_t *__restrict__ C, uint32_t M,
                                                           uint32_t N, uint32_t K) {
    gemm16_tile<kFast, WT, true>(A, B, C, M, N, K);
}

// ----------------------------------------------------------------- f32 ----
constexpr int BK32 = 32;
constexpr int APAD32 = 4, BPAD32 = 4;

// kPacked: B is the reference's panel-packed weight (src/layout.rs:16-45),
// [ceil(N/16)][K][16] with zero-padded columns: element (k, n) sits at
// ((n / 16) * K + k) * 16 + n % 16, so four columns n..n+3 (n % 4 == 0) of one
// k-row are still one 16-byte load, and a load past N reads panel padding.
template <bool kPacked>
__device__ __forceinline__ uint64_t b_index(uint32_t gk, uint32_t gn, uint32_t N, uint32_t K) {
    return kPacked ? (uint64_t(gn >> 4) * K + gk) * 16 + (gn & 15) : uint64_t(gk) * N + gn;
}

template <bool kFast, int WT, bool kPacked = false>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(const float *__restrict__ A,
                                                           const float *__restrict__ B,
                                                           float *__restrict__ C, uint32_t M,
                                                           uint32_t N, uint32_t K) {
    constexpr int BM = 32 * WT, BN = BM, kChunks = BM / 32;   // float4 per thread per operand
    __shared__ float As[2][BM][BK32 + APAD32];
    __shared__ float Bs[2][BK32][BN + BPAD32];

    const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int t = threadIdx.x;
    const int wave = t >> 6, lane = t & 63;
    const int wm = (wave >> 1) * 16 * WT, wn = (wave & 1) * 16 * WT;
    const int lr = lane & 15, lg = lane >> 4;

    f32x4 acc[WT][WT];
#pragma unroll
    for (int i = 0; i < WT; ++i)
#pragma unroll
        for (int j = 0; j < WT; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    float4 ra[kChunks], rb[kChunks];
    auto load = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {  // A: BM x 32 floats
            const int c = t + i * kThreads;
            const int r = c / (BK32 / 4), kc = (c % (BK32 / 4)) * 4;
            const uint32_t gm = m0 + r, gk = k0 + kc;
            if (kFast) {
                ra[i] = gm < M ? *reinterpret_cast<const float4 *>(A + uint64_t(gm) * K + gk)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    v[e] = (gm < M && gk + e < K) ? A[uint64_t(gm) * K + gk + e] : 0.0f;
                ra[i] = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {  // B: 32 x BN floats
            const int c = t + i * kThreads;
            const int r = c / (BN / 4), nc = (c % (BN / 4)) * 4;
            const uint32_t gk = k0 + r, gn = n0 + nc;
            if (kFast) {
                rb[i] = gn < N ? *reinterpret_cast<const float4 *>(B + b_index<kPacked>(gk, gn, N, K))
                               : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    v[e] = (gk < K && gn + e < N) ? B[b_index<kPacked>(gk, gn + e, N, K)] : 0.0f;
                rb[i] = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const int c = t + i * kThreads;
            const int r = c / (BK32 / 4), kc = (c % (BK32 / 4)) * 4;
            *reinterpret_cast<float4 *>(&As[buf][r][kc]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const int c = t + i * kThreads;
            const int r = c / (BN / 4), nc = (c % (BN / 4)) * 4;
            *reinterpret_cast<float4 *>(&Bs[buf][r][nc]) = rb[i];
        }
    };

    const uint32_t nk = (K + BK32 - 1) / BK32;
    load(0);
    store(0);
    __syncthreads();
    for (uint32_t s = 0; s < nk; ++s) {
        const int cur = s & 1;
        if (s + 1 < nk) load((s + 1) * BK32);
#pragma unroll
        for (int kk = 0; kk < BK32; kk += 4) {
            float af[WT], bfv[WT];
#pragma unroll
            for (int i = 0; i < WT; ++i) af[i] = As[cur][wm + i * 16 + lr][kk + lg];
#pragma unroll
            for (int j = 0; j < WT; ++j) bfv[j] = Bs[cur][kk + lg][wn + j * 16 + lr];
#pragma unroll
            for (int i = 0; i < WT; ++i)
#pragma unroll
                for (int j = 0; j < WT; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bfv[j], acc[i][j], 0, 0, 0);
        }
        if (s + 1 < nk) store(cur ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < WT; ++i)
#pragma unroll
        for (int j = 0; j < WT; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t gm = m0 + wm + i * 16 + lg * 4 + r, gn = n0 + wn + j * 16 + lr;
                if (gm < M && gn < N) C[uint64_t(gm) * N + gn] = acc[i][j][r];
            }
}


// ------------------------------------------------------ bf16, large tiles ----
// 256x256 workgroup tile, K slabs of 64, four wavefronts of 128x128 on
// v_mfma_f32_32x32x16_bf16 (4x4 tiles, 256 fp32 accumulators per lane). B is
// row-major [K, N]; the MFMA B operand wants 8 consecutive k per lane, so each
// thread loads an 8(k) x 8(n) block, transposes it in registers with byte
// permutes and stores it n-major (Bt[n][k]) into LDS: both operands are then
// 16-byte, k-contiguous LDS reads. LDS rows are padded to 72 elements (144 B)
// so the 32 rows one fragment read touches fall on distinct banks. The next
// slab's global loads are issued before the current slab's MFMAs.
typedef float f32x16 __attribute__((ext_vector_type(16)));
constexpr int kBigM = 256, kBigN = 256, kBigK = 64, kLdk = kBigK + 8;
// The large-tile kernels are used from this many 256x256 tiles up. Measured
// with the DMA kernel's 256x128 tiles against the 128x128 / 64x64 kernel:
// 4096x2048x512 (32 tiles) 26.2 vs 34.4 us, 2048^3 (64 tiles) 28.1 vs 46.8 us;
// at 16 tiles it no longer pays (2048x8192x512: 89.0 vs 83.9 us).
constexpr uint64_t kBigMinTiles = 32;
// the DMA kernel takes 256x128 tiles when there are at most this many of them
// (one per CU)
constexpr uint64_t kDmaNarrowMax = 256;

__device__ __forceinline__ void tile_coords(uint32_t wg, uint32_t nwg, uint32_t tiles_m,
                                            uint32_t tiles_n, uint32_t *tm, uint32_t *tn) {
    // Workgroups are dispatched round-robin over the 8 XCDs (wg % 8). Give each
    // XCD a contiguous run of tile ids, so neighbouring tiles share its L2.
    const uint32_t tile = nwg % 8 == 0 ? (wg % 8) * (nwg / 8) + wg / 8 : wg;
    // Grouped order: 8 tile rows per group, columns walked within the group.
    constexpr uint32_t kGroup = 8;
    const uint32_t per_group = kGroup * tiles_n;
    const uint32_t first_m = (tile / per_group) * kGroup;
    const uint32_t gsize = tiles_m - first_m < kGroup ? tiles_m - first_m : kGroup;
    const uint32_t in_group = tile % per_group;
    *tm = first_m + in_group % gsize;
    *tn = in_group / gsize;
}

// ------------------------------------------- bf16, large tiles, LDS DMA ----
// 256 x BN workgroup tiles (BN = 256, or 128 when 256-wide tiles would leave
// CUs idle), four wavefronts of 128 x BN/2 on v_mfma_f32_32x32x16_bf16, 32-deep
// K slabs in kDmaStages LDS stages. Both operands go from global memory into
// LDS by DMA (buffer_load ... lds: lane l of a load writes the 16 bytes at
// LDS base + 16 l) in their own layouts, A [m][k] and B [k][n], each 16-byte
// chunk of a row at a swizzled place (chunk ^ f(row)) so fragment reads hit
// distinct banks. The A operand is a 16-byte LDS read. The B operand (8
// consecutive k of one column per lane) is two ds_read_b64_tr_b16: within
// each 16-lane group, lane r addresses row k0 + r/4, columns n0 + 4(r%4) ..+3,
// and lane j receives rows k0 .. k0+3 of column n0 + j. No operand passes
// through registers on its way to LDS. One barrier per slab, placed between
// the slab's two k-steps so the MFMAs already issued cover it. The MFMA order
// per output element is k ascending in steps of 16.
constexpr int kDmaK = 32, kDmaStages = 4;

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;
typedef __attribute__((address_space(3))) uint8_t lds_u8;

__device__ __forceinline__ uint32_t swz_a(uint32_t row) { return ((row >> 1) ^ (row >> 2)) & 3u; }
// B rows of BN/8 chunks: the 4-chunk group of a chunk is XORed with a
// function of the k-row, so the eight k-rows one transposing read touches
// (k0..k0+3, k0+8..k0+11) spread over the banks
template <int BN>
__device__ __forceinline__ uint32_t swz_b(uint32_t k) {
    if constexpr (BN == 256) return 4u * ((k & 3u) | (((k >> 3) & 1u) << 2));
    else return 4u * (k & 3u);
}
// s_waitcnt with vmcnt <= n and no wait on the other counters (gfx9 encoding)
template <int n>
__device__ __forceinline__ void wait_vm() {
    __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8));
}
// The slab barrier: each wave has waited (wait_vm) for its own share of the
// DMA loads the next reads need, and its reads of the stage about to be
// refilled have been consumed by MFMAs already issued. __syncthreads' release
// fence would also wait for the DMA loads still meant to be in flight, so the
// barrier is bare, with compiler barriers on both sides.
__device__ __forceinline__ void slab_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// A launch over up to kSkinnyMaxSeg products sharing A [M, K]: segment s has
// B_s [K, n_s] and C_s [M, n_s]; the tile columns of every segment are laid
// end to end (tiles_end: running totals of BN-wide columns) and each
// workgroup's tile belongs to one segment.
// Pair form (one segment): b[0] and b[1] are two products' B of the same
// shape [K, n[0]] (SwiGLU's gate and up); the workgroup tile is 256 rows x
// 128 columns of both, and c[0] receives f(gate) * up per element, each
// product narrowed to bf16, gate passed through its activation table lut[0]
// when given, the product narrowed again (the standalone kernels'
// arithmetic).
struct DmaGroup {
    const uint16_t *a;
    uint32_t m, k, nseg;
    uint32_t tiles_end[kSkinnyMaxSeg];
    const uint16_t *b[kSkinnyMaxSeg];
    uint16_t *c[kSkinnyMaxSeg];
    uint32_t n[kSkinnyMaxSeg];
    const uint16_t *res[kSkinnyMaxSeg];   // plain form: residual [M, n_s] added, or null
    const uint16_t *lut[1];
};

template <int BN, bool kPair = false>
__device__ __forceinline__ void gemm_bf16_dma(const DmaGroup &g) {
    static_assert(!kPair || BN == 256, "the pair form fills a 256-wide tile from two B tiles");
    constexpr int NJ = BN / 64;                  // 32-column MFMA blocks per wave
    constexpr int BW = kPair ? 128 : BN;         // columns of one B matrix in the tile
    constexpr uint32_t kBytesB = 64u * BN;       // one stage of B: 32 k-rows
    constexpr uint32_t kStage = 16384u + kBytesB, kOffB = 16384u;
    constexpr int kLoadsB = BN / 64;             // 1 KiB DMA loads of B per wave per slab
    constexpr int kLoads = 4 + kLoadsB;          // ... of A and B
    constexpr int kMfma = 4 * NJ, kReads = 4 + 2 * NJ;   // per k-step
    // one array per stage: the compiler then knows a DMA into one stage does
    // not feed reads of another, and waits only where a read needs the data
    __shared__ __attribute__((aligned(1024))) uint8_t lds0[kStage], lds1[kStage], lds2[kStage],
        lds3[kStage];
    auto stage = [&](auto st) -> lds_u8 * {
        constexpr int kS = decltype(st)::value % kDmaStages;
        return kS == 0 ? (lds_u8 *)lds0 : kS == 1 ? (lds_u8 *)lds1 : kS == 2 ? (lds_u8 *)lds2 : (lds_u8 *)lds3;
    };
    const uint16_t *__restrict__ A = g.a;
    const uint32_t M = g.m, K = g.k;
    const uint32_t tiles_m = M / kBigM, tiles_n = g.tiles_end[g.nseg - 1];
    uint32_t tm, tn;
    tile_coords(blockIdx.x, gridDim.x, tiles_m, tiles_n, &tm, &tn);
    // this tile's segment (workgroup-uniform, chosen with selects)
    const uint16_t *__restrict__ B = g.b[0];
    uint16_t *__restrict__ C = g.c[0];
    const uint16_t *Rs = g.res[0];
    uint32_t N = g.n[0], first = 0;
#pragma unroll
    for (int i = 1; i < kSkinnyMaxSeg; ++i)
        if (uint32_t(i) < g.nseg && tn >= g.tiles_end[i - 1]) {
            B = g.b[i];
            C = g.c[i];
            Rs = g.res[i];
            N = g.n[i];
            first = g.tiles_end[i - 1];
        }
    const uint32_t m0 = tm * kBigM, n0 = (tn - first) * BW;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    // wave tile: 128 rows x BN/2 columns; in the pair form its columns are
    // 64 of gate and the same 64 of up
    const int wm = (wave >> 1) * 128, wn = (wave & 1) * (BW / 2);
    const int lr = lane & 31, lg = lane >> 5;

    // DMA: each load of a wave fills 1 KiB of a stage. A (4 per wave): rows
    // 64 wave + 16 t + lane/4, physical chunk lane%4. B (BN/64 per wave):
    // k-rows of BN/8 chunks, lane/(BN/8) of 512/BN rows per load, physical
    // chunk lane%(BN/8). Each lane fetches the logical chunk stored there.
    const uint32_t arow = 64u * wave + lane / 4;
    const uint32_t a_voff = (arow * K + 8u * ((lane & 3) ^ swz_a(arow))) * 2u;
    // (pair form: each of the two B matrices as a BW-wide tile, kLoadsB / 2
    // loads each, gate's tile first)
    constexpr int kLoadsM = kPair ? kLoadsB / 2 : kLoadsB;   // loads per B matrix
    uint32_t b_voff[kLoadsM];
#pragma unroll
    for (int t = 0; t < kLoadsM; ++t) {
        const uint32_t k = (kLoadsM * wave + t) * (512u / BW) + lane / (BW / 8);
        b_voff[t] = (k * N + 8u * ((lane % (BW / 8)) ^ swz_b<BW>(k))) * 2u;
    }
    auto dma = [&](uint32_t slab, auto st) {
        const uint32_t k0 = slab * kDmaK;
        const auto ra = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t *>(A + uint64_t(m0) * K + k0), 0, int(512u * K), 0x00020000);
        lds_u8 *sa = stage(st) + wave * 4096u;
#pragma unroll
        for (int t = 0; t < 4; ++t)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, sa + 1024 * t, 16, a_voff, 32u * K * t, 0, 0);
#pragma unroll
        for (int mi = 0; mi < (kPair ? 2 : 1); ++mi) {
            const uint16_t *Bm = kPair && mi == 1 ? g.b[1] : B;
            const auto rb = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<uint16_t *>(Bm + uint64_t(k0) * N + n0), 0, int(64u * N), 0x00020000);
            lds_u8 *sb = stage(st) + kOffB + mi * (64u * BW) + wave * (1024u * kLoadsM);
#pragma unroll
            for (int t = 0; t < kLoadsM; ++t)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, sb + 1024 * t, 16, b_voff[t], 0, 0, 0);
        }
    };

    // fragment offsets within a stage. A: row wm + 32i + lr, logical chunk
    // kk/8 + lg (the swizzle depends on lr only); B: per j, lane (g, r) of
    // its 16-lane group addresses k-row 8(g/2) + r/4 (+ kk + 4h), column
    // wn + 32j + 16(g%2) + 4(r%4) (the swizzle is the same for every kk, h)
    const uint32_t a_frag = (wm + lr) * 64u + ((lg ^ swz_a(lr)) * 16u);
    uint32_t b_frag[NJ];
    {
        const uint32_t g = lane >> 4, r = lane & 15;
        const uint32_t k = 8u * (g >> 1) + (r >> 2);
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int mi = kPair ? j / 2 : 0, jj = kPair ? j % 2 : j;
            const uint32_t n = wn + 32u * jj + 16u * (g & 1) + 4u * (r & 3);
            b_frag[j] = kOffB + mi * (64u * BW) + k * (2u * BW) +
                        (((n >> 3) ^ swz_b<BW>(k)) * 16u) + (n & 7u) * 2u;
        }
    }
    bf16x8 af[2][4], bfr[2][NJ];
    auto fload = [&](auto st, int kk, int fb) {
        const lds_u8 *base = stage(st);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            af[fb][i] = *reinterpret_cast<const __attribute__((address_space(3))) bf16x8 *>(
                base + ((a_frag + 2048u * i) ^ (kk == 16 ? 32u : 0u)));
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const lds_u8 *p = base + b_frag[j] + (2u * BW) * kk;
            const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                reinterpret_cast<lds_v4i16 *>(const_cast<lds_u8 *>(p)));
            const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                reinterpret_cast<lds_v4i16 *>(const_cast<lds_u8 *>(p + 8u * BW)));
            bfr[fb][j] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
    };

    f32x16 acc[4][NJ];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    auto mfmas = [&](int fb) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[fb][i], bfr[fb][j], acc[i][j], 0, 0, 0);
    };
    // interleave into the k-step's MFMAs: after each, one DMA load (while
    // any are left) and one fragment read (while any are left)
    auto mix = [](auto loads) {
        constexpr int kL = decltype(loads)::value;
#pragma unroll
        for (int i = 0; i < kMfma; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            if (i < kL) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
            if (i < kReads) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
    };
    using n0_ = std::integral_constant<int, 0>;
    using nl_ = std::integral_constant<int, kLoads>;

    // One slab s in stage s % kDmaStages. kNext: slab s+1 exists (wait for its
    // DMA and pass the barrier mid-slab, then read its first fragments);
    // kWait: the DMA loads allowed to stay in flight at that point; kLoad: slab
    // s + kDmaStages - 1 exists (its DMA goes into the stage slab s-1 used).
    auto slab = [&](uint32_t s, auto st, auto next, auto wait, auto load) {
        constexpr bool kNext = decltype(next)::value, kLoad = decltype(load)::value;
        constexpr int kWait = decltype(wait)::value, kS = decltype(st)::value;
        fload(st, 16, 1);
        mfmas(0);
        mix(n0_{});
        __builtin_amdgcn_sched_barrier(0);
        if (kNext) {
            wait_vm<kWait>();
            slab_barrier();
            if (kLoad) dma(s + kDmaStages - 1, std::integral_constant<int, kS + kDmaStages - 1>{});
            fload(std::integral_constant<int, kS + 1>{}, 0, 0);
        }
        mfmas(1);
        if (kNext) {
            if (kLoad) mix(nl_{});
            else mix(n0_{});
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    using yes = std::integral_constant<bool, true>;
    using no = std::integral_constant<bool, false>;
    // While slab s+1 is awaited, the slabs issued after it (up to
    // s + kDmaStages - 2) may stay in flight.
    using w_steady = std::integral_constant<int, kLoads * (kDmaStages - 3)>;
    using w_drain = std::integral_constant<int, 0>;
    static_assert(kDmaStages == 4, "the loop below is written for four stages");
    using s0 = std::integral_constant<int, 0>;
    using s1 = std::integral_constant<int, 1>;
    using s2 = std::integral_constant<int, 2>;
    using s3 = std::integral_constant<int, 3>;

    const uint32_t nk = K / kDmaK;   // a multiple of 4, >= 8
    dma(0, s0{});
    dma(1, s1{});
    dma(2, s2{});
    wait_vm<2 * kLoads>();
    slab_barrier();
    fload(s0{}, 0, 0);
    // slab s uses stage s % 4; every slab but the last three issues the DMA
    // of slab s + 3
    for (uint32_t s = 0; s + 4 < nk; s += 4) {
        slab(s, s0{}, yes{}, w_steady{}, yes{});
        slab(s + 1, s1{}, yes{}, w_steady{}, yes{});
        slab(s + 2, s2{}, yes{}, w_steady{}, yes{});
        slab(s + 3, s3{}, yes{}, w_steady{}, yes{});
    }
    slab(nk - 4, s0{}, yes{}, w_steady{}, yes{});
    slab(nk - 3, s1{}, yes{}, w_steady{}, no{});
    slab(nk - 2, s2{}, yes{}, w_drain{}, no{});
    slab(nk - 1, s3{}, no{}, w_drain{}, no{});

    // 32x32 D layout: acc[r] is row 8(r/4) + 4*lg + r%4, column lr
    uint16_t *cbase = C + uint64_t(m0 + wm + 4 * lg) * N + n0 + wn + lr;
    if constexpr (kPair) {
        static_assert(kStage == 32768, "the table fills the four stages");
        // gate's activation table (65536 bf16 = the four 32 KiB stages, which
        // the last slab's reads have left) comes into LDS for the lookups:
        // wave w fills stage w with entries 16384 w .. 16384 w + 16383
        const uint16_t *lut = g.lut[0];
        if (lut) {
            slab_barrier();
            const auto rl = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(lut), 0,
                                                              131072, 0x00020000);
            const uint32_t wu = __builtin_amdgcn_readfirstlane(wave);   // in an SGPR
            lds_u8 *dst = wu == 0 ? stage(s0{}) : wu == 1 ? stage(s1{}) : wu == 2 ? stage(s2{}) : stage(s3{});
#pragma unroll
            for (int t = 0; t < 32; ++t)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rl, dst + 1024 * t, 16, lane * 16u,
                                                         wu * 32768u + t * 1024u, 0, 0);
            wait_vm<0>();
            slab_barrier();
        }
        auto lookup = [&](uint32_t x) -> uint32_t {
            const uint32_t part = x >> 14, off = (x & 16383u) * 2u;
            const lds_u8 *base = part == 0 ? stage(s0{}) : part == 1 ? stage(s1{})
                               : part == 2 ? stage(s2{}) : stage(s3{});
            return *reinterpret_cast<const __attribute__((address_space(3))) uint16_t *>(base + off);
        };
        // acc[i][jj] is gate and acc[i][jj + 2] up at the same element
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                uint16_t *ct = cbase + uint64_t(32 * i) * N + 32 * jj;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    uint32_t x = __float_as_uint(acc[i][jj][r]) >> 16;
                    const uint32_t y = __float_as_uint(acc[i][jj + 2][r]) >> 16;
                    if (lut) x = lookup(x);
                    const float v = __uint_as_float(x << 16) * __uint_as_float(y << 16);
                    ct[uint64_t(8 * (r >> 2) + (r & 3)) * N] = uint16_t(__float_as_uint(v) >> 16);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
    } else {
        // + residual (MatMulAdd): each wave brings the residual of its own
        // 128 x BW/2 quadrant into its LDS stage (the main loop has left the
        // stages; the one barrier waits out the last slab's reads), then adds
        // it block row by block row as the loads land: product narrowed,
        // residual added in f32, narrowed again (the standalone epilogue's
        // arithmetic)
        constexpr uint32_t kQc = BW / 2, kLanesRow = kQc / 8, kRows = 64 / kLanesRow;
        constexpr uint32_t kLoadsI = 32 / kRows;   // 1 KiB loads per 32-row block row
        const uint32_t wu = __builtin_amdgcn_readfirstlane(wave);   // the wave index, in an SGPR
        lds_u8 *qres = wu == 0 ? stage(s0{}) : wu == 1 ? stage(s1{}) : wu == 2 ? stage(s2{}) : stage(s3{});
        if (Rs) {
            static_assert(128 * kQc * 2 <= kStage, "a stage holds a wave's residual quadrant");
            slab_barrier();
            const uint64_t q0 = uint64_t(m0 + (wu >> 1) * 128u) * N + n0 + (wu & 1u) * kQc;
            const auto rr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(Rs + q0), 0,
                                                              int(256u * N), 0x00020000);
            const uint32_t voff = ((lane / kLanesRow) * N + 8u * (lane % kLanesRow)) * 2u;
#pragma unroll
            for (uint32_t t = 0; t < 4 * kLoadsI; ++t)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, qres + 1024 * t, 16, voff, kRows * t * N * 2u, 0, 0);
        }
        auto res_at = [&](uint32_t qr, uint32_t qc) -> uint32_t {
            return *reinterpret_cast<const __attribute__((address_space(3))) uint16_t *>(
                qres + (qr * kQc + qc) * 2u);
        };
        if (Rs) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (i == 0) wait_vm<3 * kLoadsI>();
                else if (i == 1) wait_vm<2 * kLoadsI>();
                else if (i == 2) wait_vm<kLoadsI>();
                else wait_vm<0>();
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    uint16_t *ct = cbase + uint64_t(32 * i) * N + 32 * j;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const uint32_t x = __float_as_uint(acc[i][j][r]) >> 16;
                        const uint32_t y = res_at(32 * i + 8 * (r >> 2) + 4 * lg + (r & 3), 32 * j + lr);
                        ct[uint64_t(8 * (r >> 2) + (r & 3)) * N] = uint16_t(
                            __float_as_uint(__uint_as_float(x << 16) + __uint_as_float(y << 16)) >> 16);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    uint16_t *ct = cbase + uint64_t(32 * i) * N + 32 * j;
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        ct[uint64_t(8 * (r >> 2) + (r & 3)) * N] =
                            uint16_t(__float_as_uint(acc[i][j][r]) >> 16);
                    __builtin_amdgcn_sched_barrier(0);
                }
        }
    }
}

__global__ __launch_bounds__(256, 1) void gemm_bf16_dma256_kernel(const DmaGroup g) {
    gemm_bf16_dma<256>(g);
}
__global__ __launch_bounds__(256, 1) void gemm_bf16_dma128_kernel(const DmaGroup g) {
    gemm_bf16_dma<128>(g);
}
__global__ __launch_bounds__(256, 1) void gemm_bf16_dma_pair_kernel(const DmaGroup g) {
    gemm_bf16_dma<256, true>(g);
}

// Whether the DMA kernel takes a product (bf16, 16-byte aligned operands
// checked by the caller): K a multiple of 128 and >= 256, at least
// kBigMinTiles 256x256 tiles, and 256 rows of A / 32 rows of B within
// a 32-bit buffer range.
// ------------------------------------------- bf16, 64x64 tiles, LDS DMA ----
// Mid-size products (fewer than 256 128x128 tiles, e.g. 1024^3): one 64x64
// tile per workgroup, so 1024^3 runs 256 workgroups, one per CU. Each wave
// owns a 32x32 block on v_mfma_f32_32x32x16_bf16. With so little MFMA work
// per K step the tile is bound by how many operand bytes it keeps in flight,
// so A [64][64 k] and B [64 k][64] slabs go by DMA into an 8-stage LDS ring
// (16 KiB per stage, 128 KiB): seven slabs (112 KiB) are in flight while one
// is multiplied. Slab layouts are the large-tile kernel's with 128-byte rows:
// A row r holds its eight 16-byte k-chunks at chunk ^ ((r >> 1) & 7), so the
// 16-byte fragment reads of 8 consecutive rows hit distinct banks; B k-row k
// holds its eight column chunks at chunk ^ 4 ((k >> 1) & 1), so the
// transposing reads of k-rows k0..k0+3 fill one 256-byte bank row. The loop is
// unrolled by the ring depth (stage indices are constants, no load behind a
// branch); a slab past K loads nothing (its buffer range is empty). MFMA order
// per output element: k ascending in steps of 16.
constexpr int kD64K = 64, kD64Stages = 8;
constexpr uint32_t kD64Stage = 16384, kD64OffB = 8192;

__device__ __forceinline__ uint32_t swz_a64(uint32_t row) { return (row >> 1) & 7u; }
__device__ __forceinline__ uint32_t swz_b64(uint32_t k) { return 4u * ((k >> 1) & 1u); }

__global__ __launch_bounds__(kThreads, 1) void gemm_bf16_dma64_kernel(const uint16_t *__restrict__ A,
                                                                      const uint16_t *__restrict__ B,
                                                                      uint16_t *__restrict__ C,
                                                                      uint32_t M, uint32_t N,
                                                                      uint32_t K) {
    __shared__ __attribute__((aligned(1024))) uint8_t l0[kD64Stage], l1[kD64Stage], l2[kD64Stage],
        l3[kD64Stage], l4[kD64Stage], l5[kD64Stage], l6[kD64Stage], l7[kD64Stage];
    auto stage = [&](auto st) -> lds_u8 * {
        constexpr int kS = decltype(st)::value % kD64Stages;
        return kS == 0 ? (lds_u8 *)l0 : kS == 1 ? (lds_u8 *)l1 : kS == 2 ? (lds_u8 *)l2
             : kS == 3 ? (lds_u8 *)l3 : kS == 4 ? (lds_u8 *)l4 : kS == 5 ? (lds_u8 *)l5
             : kS == 6 ? (lds_u8 *)l6 : (lds_u8 *)l7;
    };
    uint32_t tm, tn;
    tile_coords(blockIdx.x, gridDim.x, M / 64, N / 64, &tm, &tn);
    const uint32_t m0 = tm * 64, n0 = tn * 64;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const uint32_t wu = __builtin_amdgcn_readfirstlane(wave);
    const int lr = lane & 31, lg = lane >> 5;

    // DMA: per slab each wave fills 2 KiB of A (rows 16 w .. 16 w + 15) and
    // 2 KiB of B (k-rows 16 w .. 16 w + 15), 8 rows of 8 chunks per load.
    uint32_t a_voff[2], b_voff[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const uint32_t row = 16u * wave + 8u * t + lane / 8;
        a_voff[t] = (row * K + 8u * ((lane & 7) ^ swz_a64(row))) * 2u;
        b_voff[t] = (row * N + 8u * ((lane & 7) ^ swz_b64(row))) * 2u;
    }
    const uint32_t nk = K / kD64K;
    auto dma = [&](uint32_t slab, auto st) {
        const bool live = slab < nk;
        const uint32_t k0 = live ? slab * kD64K : 0u;
        const auto ra = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t *>(A + uint64_t(m0) * K + k0), 0, live ? int(128u * K) : 0, 0x00020000);
        const auto rb = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint16_t *>(B + uint64_t(k0) * N + n0), 0, live ? int(128u * N) : 0, 0x00020000);
        lds_u8 *sa = stage(st) + wu * 2048u;
        lds_u8 *sb = stage(st) + kD64OffB + wu * 2048u;
#pragma unroll
        for (int t = 0; t < 2; ++t)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, sa + 1024 * t, 16, a_voff[t], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < 2; ++t)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, sb + 1024 * t, 16, b_voff[t], 0, 0, 0);
    };

    // fragment offsets within a stage. A: row 32 (w / 2) + lr, logical chunk
    // kk/8 + lg. B: lane (g, r) of its 16-lane group addresses k-row
    // 8 (g / 2) + r / 4 (+ kk, and + 4 for the second read), column
    // 32 (w % 2) + 16 (g % 2) + 4 (r % 4).
    const uint32_t arow = 32u * (wave >> 1) + lr;
    uint32_t a_frag[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) a_frag[q] = arow * 128u + (((2u * q + lg) ^ swz_a64(arow)) * 16u);
    uint32_t b_frag;
    {
        const uint32_t g = lane >> 4, r = lane & 15;
        const uint32_t k = 8u * (g >> 1) + (r >> 2);
        const uint32_t n = 32u * (wave & 1) + 16u * (g & 1) + 4u * (r & 3);
        b_frag = kD64OffB + k * 128u + (((n >> 3) ^ swz_b64(k)) * 16u) + (n & 7u) * 2u;
    }
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;

    // Slab s in stage s % 8: wait for its DMA (the six slabs issued after it
    // may stay in flight), barrier (every wave's share landed, and every wave
    // is done reading the stage refilled next), issue slab s + 7 into the
    // stage slab s - 1 used, then four k-steps.
    auto step = [&](uint32_t s, auto st) {
        constexpr int kS = decltype(st)::value;
        wait_vm<4 * (kD64Stages - 2)>();
        slab_barrier();
        dma(s + kD64Stages - 1, std::integral_constant<int, kS + kD64Stages - 1>{});
        const lds_u8 *base = stage(st);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const bf16x8 af = *reinterpret_cast<const __attribute__((address_space(3))) bf16x8 *>(base + a_frag[q]);
            const lds_u8 *p = base + b_frag + 128u * 16u * q;
            const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                reinterpret_cast<lds_v4i16 *>(const_cast<lds_u8 *>(p)));
            const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                reinterpret_cast<lds_v4i16 *>(const_cast<lds_u8 *>(p + 512u)));
            const bf16x8 bf = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bf, acc, 0, 0, 0);
        }
    };
#pragma unroll
    for (int p = 0; p < kD64Stages - 1; ++p) {
        // prologue: slabs 0..6 (constant stage indices through the switch)
        switch (p) {
        case 0: dma(0, std::integral_constant<int, 0>{}); break;
        case 1: dma(1, std::integral_constant<int, 1>{}); break;
        case 2: dma(2, std::integral_constant<int, 2>{}); break;
        case 3: dma(3, std::integral_constant<int, 3>{}); break;
        case 4: dma(4, std::integral_constant<int, 4>{}); break;
        case 5: dma(5, std::integral_constant<int, 5>{}); break;
        default: dma(6, std::integral_constant<int, 6>{}); break;
        }
    }
    for (uint32_t s = 0; s < nk; s += kD64Stages) {   // nk is a multiple of 8
        step(s + 0, std::integral_constant<int, 0>{});
        step(s + 1, std::integral_constant<int, 1>{});
        step(s + 2, std::integral_constant<int, 2>{});
        step(s + 3, std::integral_constant<int, 3>{});
        step(s + 4, std::integral_constant<int, 4>{});
        step(s + 5, std::integral_constant<int, 5>{});
        step(s + 6, std::integral_constant<int, 6>{});
        step(s + 7, std::integral_constant<int, 7>{});
    }
    // 32x32 D layout: acc[r] is row 8 (r / 4) + 4 lg + r % 4, column lr;
    // bf16 by truncation
    uint16_t *cb = C + uint64_t(m0 + 32u * (wave >> 1) + 4u * lg) * N + n0 + 32u * (wave & 1) + lr;
#pragma unroll
    for (int r = 0; r < 16; ++r)
        cb[uint64_t(8 * (r >> 2) + (r & 3)) * N] = uint16_t(__float_as_uint(acc[r]) >> 16);
}

bool dma64_applies(uint32_t m, uint32_t k, uint32_t n) {
    return m % 64 == 0 && n % 64 == 0 && k % (kD64K * kD64Stages) == 0 && k < (1u << 23) &&
           n < (1u << 23) && m >= 64 && n >= 64;
}

bool dma_applies(uint32_t m, uint32_t k, uint32_t n) {
    return m % kBigM == 0 && n % kBigN == 0 && k % (2 * kBigK) == 0 && k >= 4 * kBigK &&
           k < (1u << 22) && n < (1u << 24) &&
           uint64_t(m / kBigM) * (n / kBigN) >= kBigMinTiles;
}

hipError_t launch_dma(DmaGroup g, hipStream_t stream) {
    uint32_t wide = 0;
    for (uint32_t i = 0; i < g.nseg; ++i) wide += g.n[i] / kBigN;
    // 256x128 tiles when they all fit in one round of workgroups: a 256x128
    // workgroup takes about 0.82 of a 256x256 one's time for half the work
    // (4096x2048x2048: 40 us on 256 CUs vs 49 us on 128), so they pay only
    // when twice as many tiles still need no second round
    const bool narrow = 2 * uint64_t(g.m / kBigM) * wide <= kDmaNarrowMax;
    uint32_t cols = 0;
    for (uint32_t i = 0; i < g.nseg; ++i) {
        cols += g.n[i] / (narrow ? 128u : 256u);
        g.tiles_end[i] = cols;
    }
    const dim3 grid{(g.m / kBigM) * cols}, block{256u};
    if (narrow)
        hipLaunchKernelGGL(gemm_bf16_dma128_kernel, grid, block, 0, stream, g);
    else
        hipLaunchKernelGGL(gemm_bf16_dma256_kernel, grid, block, 0, stream, g);
    return hipGetLastError();
}

}  // namespace

size_t matmul_scratch_bytes(uint32_t m, uint32_t k, uint32_t n, uint8_t dtype) {
    return matmul_skinny_scratch_bytes(m, k, n, dtype);
}

hipError_t launch_matmul(const void *a, const void *b, void *c, uint32_t m, uint32_t k, uint32_t n,
                         uint8_t dtype, void *scratch, hipStream_t stream) {
    const uintptr_t al = reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b);
    // few rows: stream B once (16-byte aligned operands, output included)
    if (dtype != 6 && ((al | reinterpret_cast<uintptr_t>(c)) & 15) == 0 &&
        matmul_skinny_applies(m, k, n, dtype))
        return launch_matmul_skinny(a, b, c, m, k, n, dtype, scratch, stream);
    // 64-tiles when 128-tiles would not give every CU a workgroup
    const uint64_t tiles128 = uint64_t((m + 127) / 128) * ((n + 127) / 128);
    const bool small = tiles128 < 256;
    const uint32_t bt = small ? 64 : 128;
    const dim3 grid((n + bt - 1) / bt, (m + bt - 1) / bt);
#define HOLO_GEMM_LAUNCH(KERNEL, T)                                                              \
    do {                                                                                         \
        const T *A_ = static_cast<const T *>(a);                                                 \
        const T *B_ = static_cast<const T *>(b);                                                 \
        T *C_ = static_cast<T *>(c);                                                             \
        if (fast) {                                                                              \
            if (small)                                                                           \
                hipLaunchKernelGGL((KERNEL<true, 2>), grid, dim3(kThreads), 0, stream, A_, B_, C_, \
                                   m, n, k);                                                     \
            else                                                                                 \
                hipLaunchKernelGGL((KERNEL<true, 4>), grid, dim3(kThreads), 0, stream, A_, B_, C_, \
                                   m, n, k);                                                     \
        } else {                                                                                 \
            if (small)                                                                           \
                hipLaunchKernelGGL((KERNEL<false, 2>), grid, dim3(kThreads), 0, stream, A_, B_,  \
                                   C_, m, n, k);                                                 \
            else                                                                                 \
                hipLaunchKernelGGL((KERNEL<false, 4>), grid, dim3(kThreads), 0, stream, A_, B_,  \
                                   C_, m, n, k);                                                 \
        }                                                                                        \
    } while (0)
    if (dtype == 7) {
        // large aligned problems: at least kBigMinTiles 256x256 tiles, K a
        // multiple of 128 and >= 256, and 256 rows of A / 64 rows of B within a
        // 32-bit buffer range
        if ((al & 15) == 0 && dma_applies(m, k, n)) {
            DmaGroup g{};
            g.a = static_cast<const uint16_t *>(a);
            g.m = m;
            g.k = k;
            g.nseg = 1;
            g.b[0] = static_cast<const uint16_t *>(b);
            g.c[0] = static_cast<uint16_t *>(c);
            g.n[0] = n;
            return launch_dma(g, stream);
        }
        // mid-size aligned problems: 64x64 tiles fed by LDS DMA
        if (small && ((al | reinterpret_cast<uintptr_t>(c)) & 15) == 0 && dma64_applies(m, k, n)) {
            hipLaunchKernelGGL(gemm_bf16_dma64_kernel, dim3((m / 64) * (n / 64)), dim3(kThreads), 0,
                               stream, static_cast<const uint16_t *>(a),
                               static_cast<const uint16_t *>(b), static_cast<uint16_t *>(c), m, n, k);
            return hipGetLastError();
        }
        const bool fast = (al & 15) == 0 && k % BK16 == 0 && n % 8 == 0;
        HOLO_GEMM_LAUNCH(gemm_bf16_kernel, uint16_t);
    } else if (dtype == 8) {
        const bool fast = (al & 15) == 0 && k % BK32 == 0 && n % 4 == 0;
        HOLO_GEMM_LAUNCH(gemm_f32_kernel, float);
    } else if (dtype == 6) {
        const bool fast = (al & 15) == 0 && k % BK16 == 0 && n % 8 == 0;
        HOLO_GEMM_LAUNCH(gemm_f16_kernel, uint16_t);
    } else {
        return hipErrorInvalidValue;
    }
#undef HOLO_GEMM_LAUNCH
    return hipGetLastError();
}

hipError_t launch_matmul_f32_packed(const float *a, const float *b_packed, float *c, uint32_t m,
                                   uint32_t k, uint32_t n, hipStream_t stream) {
    const uint64_t tiles128 = uint64_t((m + 127) / 128) * ((n + 127) / 128);
    const bool small = tiles128 < 256;
    const uint32_t bt = small ? 64 : 128;
    const dim3 grid((n + bt - 1) / bt, (m + bt - 1) / bt);
    // the fast loads need 16-byte aligned A and B rows and whole K slabs; the
    // packed B's panel padding covers any n
    const bool fast = ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b_packed)) & 15) == 0 &&
                      k % BK32 == 0;
    if (fast && small)
        hipLaunchKernelGGL((gemm_f32_kernel<true, 2, true>), grid, dim3(kThreads), 0, stream, a,
                           b_packed, c, m, n, k);
    else if (fast)
        hipLaunchKernelGGL((gemm_f32_kernel<true, 4, true>), grid, dim3(kThreads), 0, stream, a,
                           b_packed, c, m, n, k);
    else if (small)
        hipLaunchKernelGGL((gemm_f32_kernel<false, 2, true>), grid, dim3(kThreads), 0, stream, a,
                           b_packed, c, m, n, k);
    else
        hipLaunchKernelGGL((gemm_f32_kernel<false, 4, true>), grid, dim3(kThreads), 0, stream, a,
                           b_packed, c, m, n, k);
    return hipGetLastError();
}

hipError_t launch_matmul_pair_tiled(const void *a, uint32_t m, uint32_t k, const void *b_gate,
                                    const void *b_up, uint32_t n, void *out,
                                    const uint16_t *lut_gate, hipStream_t stream) {
    const uintptr_t al = reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b_gate) |
                         reinterpret_cast<uintptr_t>(b_up) | reinterpret_cast<uintptr_t>(out);
    if ((al & 15) != 0 || !matmul_group_tiled_applies(m, k, &n, 1)) return hipErrorInvalidValue;
    DmaGroup g{};
    g.a = static_cast<const uint16_t *>(a);
    g.m = m;
    g.k = k;
    g.nseg = 1;
    g.b[0] = static_cast<const uint16_t *>(b_gate);
    g.b[1] = static_cast<const uint16_t *>(b_up);
    g.c[0] = static_cast<uint16_t *>(out);
    g.n[0] = n;
    g.tiles_end[0] = n / 128;
    g.lut[0] = lut_gate;
    const dim3 grid{(m / kBigM) * (n / 128)}, block{256u};
    hipLaunchKernelGGL(gemm_bf16_dma_pair_kernel, grid, block, 0, stream, g);
    return hipGetLastError();
}

bool matmul_group_tiled_applies(uint32_t m, uint32_t k, const uint32_t *n, int nseg) {
    if (nseg < 1 || nseg > kSkinnyMaxSeg) return false;
    for (int i = 0; i < nseg; ++i)
        if (!dma_applies(m, k, n[i])) return false;
    return true;
}

hipError_t launch_matmul_group_tiled(const void *a, uint32_t m, uint32_t k,
                                     const SkinnySegment *segs, void *const *c, int nseg,
                                     hipStream_t stream, const void *const *res) {
    uint32_t n[kSkinnyMaxSeg] = {};
    uintptr_t al = reinterpret_cast<uintptr_t>(a);
    for (int i = 0; i < nseg && i < kSkinnyMaxSeg; ++i) {
        n[i] = segs[i].n;
        al |= reinterpret_cast<uintptr_t>(segs[i].b) | reinterpret_cast<uintptr_t>(c[i]);
        if (res && res[i]) {
            al |= reinterpret_cast<uintptr_t>(res[i]);
            if (n[i] >= (1u << 21)) return hipErrorInvalidValue;   // 256 rows within 2^31 bytes
        }
    }
    if ((al & 15) != 0 || !matmul_group_tiled_applies(m, k, n, nseg)) return hipErrorInvalidValue;
    DmaGroup g{};
    g.a = static_cast<const uint16_t *>(a);
    g.m = m;
    g.k = k;
    g.nseg = uint32_t(nseg);
    for (int i = 0; i < nseg; ++i) {
        g.b[i] = static_cast<const uint16_t *>(segs[i].b);
        g.c[i] = static_cast<uint16_t *>(c[i]);
        g.n[i] = n[i];
        g.res[i] = res ? static_cast<const uint16_t *>(res[i]) : nullptr;
    }
    return launch_dma(g, stream);
}

}  // namespace holo
