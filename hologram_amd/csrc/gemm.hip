// gemm.hip — C = A * B on MFMA (row-major A[M,K], B[K,N], C[M,N]).
//
// The reference MatMul (crates/hologram-compute/src/cpu/float_kernels.rs:298-399)
// accumulates in f32; bf16 operands are exact in f32, and the bf16 result is
// narrowed by truncation (write_bf16, src/cpu/dtype.rs:75-79). Here:
//   bf16: v_mfma_f32_16x16x32_bf16 (fp32 accumulate), truncating store
//   f32 : v_mfma_f32_16x16x4_f32
// Workgroup tile 128x128 (four wavefronts, 64x64 each as 4x4 MFMA tiles),
// K staged through LDS in double-buffered slabs: the next slab's global loads
// are issued before the current slab's MFMAs.
#include <hip/hip_runtime.h>

#include "holo_kernels.h"

namespace holo {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128;
constexpr int kThreads = 256;

// ---------------------------------------------------------------- bf16 ----
// LDS: A slab [BM][BK + pad], B slab [BK][BN + pad] (both as u16).
constexpr int BK16 = 64;
constexpr int APAD16 = 8, BPAD16 = 8;

template <bool kFast>
__device__ __forceinline__ void load_slab_bf16(const uint16_t *__restrict__ A,
                                               const uint16_t *__restrict__ B, uint32_t M,
                                               uint32_t N, uint32_t K, uint32_t m0, uint32_t n0,
                                               uint32_t k0, uint4 *ra, uint4 *rb) {
    const int t = threadIdx.x;
    // A: BM x BK16 = 128 x 64 u16 = 1024 chunks of 8; 4 per thread
#pragma unroll
    for (int i = 0; i < 4; ++i) {
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
    // B: BK16 x BN = 64 x 128 u16 = 1024 chunks of 8 along n; 4 per thread
#pragma unroll
    for (int i = 0; i < 4; ++i) {
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

__device__ __forceinline__ void store_slab_bf16(uint16_t (*As)[BK16 + APAD16],
                                                uint16_t (*Bs)[BN + BPAD16], const uint4 *ra,
                                                const uint4 *rb) {
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = t + i * kThreads;
        const int r = c / (BK16 / 8), kc = (c % (BK16 / 8)) * 8;
        *reinterpret_cast<uint4 *>(&As[r][kc]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = t + i * kThreads;
        const int r = c / (BN / 8), nc = (c % (BN / 8)) * 8;
        *reinterpret_cast<uint4 *>(&Bs[r][nc]) = rb[i];
    }
}

template <bool kFast>
__global__ __launch_bounds__(kThreads) void gemm_bf16_kernel(const uint16_t *__restrict__ A,
                                                            const uint16_t *__restrict__ B,
                                                            uint16_t *__restrict__ C, uint32_t M,
                                                            uint32_t N, uint32_t K) {
    __shared__ uint16_t As[2][BM][BK16 + APAD16];
    __shared__ uint16_t Bs[2][BK16][BN + BPAD16];

    const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int lr = lane & 15, lg = lane >> 4;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    const uint32_t nk = (K + BK16 - 1) / BK16;
    uint4 ra[4], rb[4];
    load_slab_bf16<kFast>(A, B, M, N, K, m0, n0, 0, ra, rb);
    store_slab_bf16(As[0], Bs[0], ra, rb);
    __syncthreads();

    for (uint32_t s = 0; s < nk; ++s) {
        const int cur = s & 1;
        if (s + 1 < nk) load_slab_bf16<kFast>(A, B, M, N, K, m0, n0, (s + 1) * BK16, ra, rb);
#pragma unroll
        for (int kk = 0; kk < BK16; kk += 32) {
            bf16x8 af[4], bfr[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                af[i] = *reinterpret_cast<const bf16x8 *>(&As[cur][wm + i * 16 + lr][kk + lg * 8]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint16_t v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = Bs[cur][kk + lg * 8 + e][wn + j * 16 + lr];
                bfr[j] = *reinterpret_cast<const bf16x8 *>(v);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        if (s + 1 < nk) store_slab_bf16(As[cur ^ 1], Bs[cur ^ 1], ra, rb);
        __syncthreads();
    }

    // D layout: lane holds rows 4*lg + r, column lr of each 16x16 tile
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t gm = m0 + wm + i * 16 + lg * 4 + r, gn = n0 + wn + j * 16 + lr;
                if (gm < M && gn < N)
                    C[uint64_t(gm) * N + gn] = uint16_t(__float_as_uint(acc[i][j][r]) >> 16);
            }
}

// ----------------------------------------------------------------- f32 ----
constexpr int BK32 = 32;
constexpr int APAD32 = 4, BPAD32 = 4;

template <bool kFast>
__global__ __launch_bounds__(kThreads) void gemm_f32_kernel(const float *__restrict__ A,
                                                           const float *__restrict__ B,
                                                           float *__restrict__ C, uint32_t M,
                                                           uint32_t N, uint32_t K) {
    __shared__ float As[2][BM][BK32 + APAD32];
    __shared__ float Bs[2][BK32][BN + BPAD32];

    const uint32_t m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int t = threadIdx.x;
    const int wave = t >> 6, lane = t & 63;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int lr = lane & 15, lg = lane >> 4;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    float4 ra[4], rb[4];
    auto load = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // A: 128 x 32 floats = 1024 float4
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
        for (int i = 0; i < 4; ++i) {  // B: 32 x 128 floats = 1024 float4
            const int c = t + i * kThreads;
            const int r = c / (BN / 4), nc = (c % (BN / 4)) * 4;
            const uint32_t gk = k0 + r, gn = n0 + nc;
            if (kFast) {
                rb[i] = gn < N ? *reinterpret_cast<const float4 *>(B + uint64_t(gk) * N + gn)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    v[e] = (gk < K && gn + e < N) ? B[uint64_t(gk) * N + gn + e] : 0.0f;
                rb[i] = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = t + i * kThreads;
            const int r = c / (BK32 / 4), kc = (c % (BK32 / 4)) * 4;
            *reinterpret_cast<float4 *>(&As[buf][r][kc]) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
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
            float af[4], bfv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) af[i] = As[cur][wm + i * 16 + lr][kk + lg];
#pragma unroll
            for (int j = 0; j < 4; ++j) bfv[j] = Bs[cur][kk + lg][wn + j * 16 + lr];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bfv[j], acc[i][j], 0, 0, 0);
        }
        if (s + 1 < nk) store(cur ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t gm = m0 + wm + i * 16 + lg * 4 + r, gn = n0 + wn + j * 16 + lr;
                if (gm < M && gn < N) C[uint64_t(gm) * N + gn] = acc[i][j][r];
            }
}

}  // namespace

hipError_t launch_matmul(const void *a, const void *b, void *c, uint32_t m, uint32_t k, uint32_t n,
                         uint8_t dtype, hipStream_t stream) {
    const dim3 grid((n + BN - 1) / BN, (m + BM - 1) / BM);
    const uintptr_t al = reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b);
    if (dtype == 7) {
        const bool fast = (al & 15) == 0 && k % BK16 == 0 && n % 8 == 0;
        if (fast)
            hipLaunchKernelGGL(gemm_bf16_kernel<true>, grid, dim3(kThreads), 0, stream,
                               static_cast<const uint16_t *>(a), static_cast<const uint16_t *>(b),
                               static_cast<uint16_t *>(c), m, n, k);
        else
            hipLaunchKernelGGL(gemm_bf16_kernel<false>, grid, dim3(kThreads), 0, stream,
                               static_cast<const uint16_t *>(a), static_cast<const uint16_t *>(b),
                               static_cast<uint16_t *>(c), m, n, k);
    } else if (dtype == 8) {
        const bool fast = (al & 15) == 0 && k % BK32 == 0 && n % 4 == 0;
        if (fast)
            hipLaunchKernelGGL(gemm_f32_kernel<true>, grid, dim3(kThreads), 0, stream,
                               static_cast<const float *>(a), static_cast<const float *>(b),
                               static_cast<float *>(c), m, n, k);
        else
            hipLaunchKernelGGL(gemm_f32_kernel<false>, grid, dim3(kThreads), 0, stream,
                               static_cast<const float *>(a), static_cast<const float *>(b),
                               static_cast<float *>(c), m, n, k);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace holo
