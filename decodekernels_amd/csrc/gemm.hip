// C[M,N] = A[M,K] * B[N,K]^T (+ bias[N]) for gfx950 -- the nn.Linear "TN"
// GEMM of every decoder projection. Same contract as DecodeKernels'
// dk::launch_gemm_tn (csrc/gemm_wmma.cuh:191-219): fp32 accumulation, bias
// added in fp32, one rounding to the model dtype; K, lda, ldb multiples of 8;
// A and B 16-byte aligned; any M, N and ldc.
//
// Two kernels, both on v_mfma_f32_16x16x32_{bf16,f16}:
//
// * skinny (M <= 64, decode): the op streams the weight matrix once, so it is
//   bound by HBM bandwidth. A workgroup owns 16 output columns and all M rows;
//   its 4 waves split K into interleaved 32-column steps, each lane loading 16
//   bytes of a weight row per step straight into its MFMA operand, U steps in
//   flight per wave. The activations (<= 64 rows) are read through L2, where
//   they stay resident. The 4 partial tiles are summed through LDS.
// * tiled (M > 64, prefill): 128x128 output tile per 256-thread workgroup,
//   2x2 waves of 64x64, K in 64-column stages double-buffered in LDS (rows
//   padded by 16 bytes against bank conflicts); the next stage's global loads
//   are in flight while the current stage is multiplied.
#include "../../include/decodekernels_amd.h"
#include "dk_device.h"
#include "dk_host.h"

namespace dk {
namespace gemm {

// MFMA operand fragment: 8 consecutive K elements of one row.
__device__ __forceinline__ u32x4 frag_or_zero(const uint16_t* base, int64_t ld, int row, int rows, int k, int K) {
  if (row < rows && k < K) return *reinterpret_cast<const u32x4*>(base + row * ld + k);
  return u32x4{0u, 0u, 0u, 0u};
}

// ---------------------------------------------------------------------------
// Skinny kernel
// ---------------------------------------------------------------------------
constexpr int kSkinnyWaves = 4;
constexpr int kSkinnyThreads = kSkinnyWaves * kWave;

template <typename E, int MT, int U>
__global__ __launch_bounds__(kSkinnyThreads) void gemm_skinny_kernel(const uint16_t* __restrict__ A,
                                                                     const uint16_t* __restrict__ B,
                                                                     const uint16_t* __restrict__ bias,
                                                                     uint16_t* __restrict__ C, int M, int N, int K,
                                                                     int lda, int ldb, int ldc) {
  __shared__ f32x4 red[kSkinnyWaves][MT][kWave];
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int l16 = lane % 16;
  const int lg = lane / 16;
  const int n0 = blockIdx.x * 16;

  f32x4 acc[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int ksteps = (K + 31) / 32;
  const int brow = n0 + l16;
  // Round j of wave w covers k-steps (j * kSkinnyWaves + w) * U + u, u < U.
  for (int base = wave * U; base < ksteps; base += kSkinnyWaves * U) {
    u32x4 bf[U];
    u32x4 af[U][MT];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = (base + u) * 32 + 8 * lg;
      bf[u] = frag_or_zero(B, ldb, brow, N, k, K);
#pragma unroll
      for (int i = 0; i < MT; ++i) af[u][i] = frag_or_zero(A, lda, 16 * i + l16, M, k, K);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
#pragma unroll
      for (int i = 0; i < MT; ++i) acc[i] = E::mfma_16x16x32(af[u][i], bf[u], acc[i]);
    }
  }

#pragma unroll
  for (int i = 0; i < MT; ++i) red[wave][i][lane] = acc[i];
  __syncthreads();

  // Output element e of this tile: row m = e / 16, column n0 + e % 16.
  for (int e = threadIdx.x; e < MT * 16 * 16; e += kSkinnyThreads) {
    const int m = e / 16;
    const int n = n0 + e % 16;
    if (m >= M || n >= N) continue;
    // acc layout: tile i = m / 16, lane = 16 * ((m % 16) / 4) + (n % 16), reg (m % 4).
    const int i = m / 16;
    const int src_lane = 16 * ((m % 16) / 4) + (e % 16);
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < kSkinnyWaves; ++w) v += red[w][i][src_lane][m % 4];
    if (bias != nullptr) v += E::to_float(bias[n]);
    C[static_cast<int64_t>(m) * ldc + n] = E::from_float(v);
  }
}

// ---------------------------------------------------------------------------
// Tiled kernel (128 x 128 x 64)
// ---------------------------------------------------------------------------
constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kLdsRow = kBK + 8;  // padded LDS row, in elements
constexpr int kTiledThreads = 256;

template <typename E>
__global__ __launch_bounds__(kTiledThreads) void gemm_tiled_kernel(const uint16_t* __restrict__ A,
                                                                   const uint16_t* __restrict__ B,
                                                                   const uint16_t* __restrict__ bias,
                                                                   uint16_t* __restrict__ C, int M, int N, int K,
                                                                   int lda, int ldb, int ldc) {
  __shared__ uint16_t As[2][kBM * kLdsRow];
  __shared__ uint16_t Bs[2][kBN * kLdsRow];
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int wm = wave / 2;
  const int wn = wave % 2;
  const int l16 = lane % 16;
  const int lg = lane / 16;
  const int m0 = blockIdx.y * kBM;
  const int n0 = blockIdx.x * kBN;

  // Global -> register staging: each thread moves 4 A and 4 B vectors per stage.
  constexpr int kVecPerRow = kBK / 8;                          // 8
  constexpr int kLoads = kBM * kVecPerRow / kTiledThreads;     // 4
  u32x4 ra[kLoads], rb[kLoads];
  auto gload = [&](int k0) {
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const int v = tid + j * kTiledThreads;
      const int row = v / kVecPerRow;
      const int col = (v % kVecPerRow) * 8;
      ra[j] = frag_or_zero(A, lda, m0 + row, M, k0 + col, K);
      rb[j] = frag_or_zero(B, ldb, n0 + row, N, k0 + col, K);
    }
  };
  auto lstore = [&](int stage) {
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const int v = tid + j * kTiledThreads;
      const int row = v / kVecPerRow;
      const int col = (v % kVecPerRow) * 8;
      *reinterpret_cast<u32x4*>(&As[stage][row * kLdsRow + col]) = ra[j];
      *reinterpret_cast<u32x4*>(&Bs[stage][row * kLdsRow + col]) = rb[j];
    }
  };

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int stages = (K + kBK - 1) / kBK;
  gload(0);
  lstore(0);
  __syncthreads();
  for (int s = 0; s < stages; ++s) {
    const int cur = s & 1;
    if (s + 1 < stages) gload((s + 1) * kBK);
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 32) {
      u32x4 af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        af[i] = *reinterpret_cast<const u32x4*>(&As[cur][(wm * 64 + 16 * i + l16) * kLdsRow + kk + 8 * lg]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        bf[j] = *reinterpret_cast<const u32x4*>(&Bs[cur][(wn * 64 + 16 * j + l16) * kLdsRow + kk + 8 * lg]);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = E::mfma_16x16x32(af[i], bf[j], acc[i][j]);
    }
    if (s + 1 < stages) lstore(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: acc[i][j] lane l reg r -> C[m0 + wm*64 + 16i + 4*lg + r][n0 + wn*64 + 16j + l16].
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int n = n0 + wn * 64 + 16 * j + l16;
    if (n >= N) continue;
    const float b = bias != nullptr ? E::to_float(bias[n]) : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 64 + 16 * i + 4 * lg + r;
        if (m < M) C[static_cast<int64_t>(m) * ldc + n] = E::from_float(acc[i][j][r] + b);
      }
    }
  }
}

template <typename E>
hipError_t launch(const uint16_t* A, const uint16_t* B, const uint16_t* bias, uint16_t* C, int M, int N, int K,
                  int lda, int ldb, int ldc, hipStream_t s) {
  if (M <= 64) {
    const dim3 grid(static_cast<unsigned>(ceil_div64(N, 16)));
    const dim3 block(kSkinnyThreads);
    if (M <= 16) {
      hipLaunchKernelGGL((gemm_skinny_kernel<E, 1, 8>), grid, block, 0, s, A, B, bias, C, M, N, K, lda, ldb, ldc);
    } else if (M <= 32) {
      hipLaunchKernelGGL((gemm_skinny_kernel<E, 2, 4>), grid, block, 0, s, A, B, bias, C, M, N, K, lda, ldb, ldc);
    } else {
      hipLaunchKernelGGL((gemm_skinny_kernel<E, 4, 4>), grid, block, 0, s, A, B, bias, C, M, N, K, lda, ldb, ldc);
    }
    return hipGetLastError();
  }
  if (ceil_div64(M, kBM) > 65535) return hipErrorInvalidValue;
  const dim3 grid(static_cast<unsigned>(ceil_div64(N, kBN)), static_cast<unsigned>(ceil_div64(M, kBM)));
  hipLaunchKernelGGL((gemm_tiled_kernel<E>), grid, dim3(kTiledThreads), 0, s, A, B, bias, C, M, N, K, lda, ldb, ldc);
  return hipGetLastError();
}

}  // namespace gemm
}  // namespace dk

extern "C" int dk_gemm_tn(int dtype, const void* A, const void* B, const void* bias, void* C, int M, int N, int K,
                          int lda, int ldb, int ldc, void* stream) {
  using namespace dk;
  clear_error();
  if (dtype != DK_FLOAT16 && dtype != DK_BFLOAT16)
    return fail("gemm_tn: expected float16 or bfloat16, got dtype code %d", dtype);
  if (M < 0 || N < 0 || K < 0) return fail("gemm_tn: M, N and K must be non-negative");
  if (M == 0 || N == 0) return hipSuccess;
  if (K % 8 != 0 || lda % 8 != 0 || ldb % 8 != 0)
    return fail("gemm_tn: K and row strides of a/b must be multiples of 8");
  if (!aligned_to(A, 16) || !aligned_to(B, 16)) return fail("gemm_tn: a and b must be 16-byte aligned");
  if (C == nullptr || (K > 0 && (A == nullptr || B == nullptr))) return fail("gemm_tn: pointers must not be NULL");
  if (M > 64 && ceil_div64(M, gemm::kBM) > 65535) return fail("gemm_tn: M is too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* a = static_cast<const uint16_t*>(A);
  const auto* b = static_cast<const uint16_t*>(B);
  const auto* bi = static_cast<const uint16_t*>(bias);
  auto* c = static_cast<uint16_t*>(C);
  const hipError_t e = dtype == DK_BFLOAT16 ? gemm::launch<Bf16>(a, b, bi, c, M, N, K, lda, ldb, ldc, s)
                                            : gemm::launch<F16>(a, b, bi, c, M, N, K, lda, ldb, ldc, s);
  return static_cast<int>(e);
}
