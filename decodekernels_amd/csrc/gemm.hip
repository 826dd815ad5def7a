// C[M,N] = A[M,K] * B[N,K]^T (+ bias[N]) for gfx950 -- the nn.Linear "TN"
// GEMM of every decoder projection. Same contract as DecodeKernels'
// dk::launch_gemm_tn (csrc/gemm_wmma.cuh:191-219): fp32 accumulation, bias
// added in fp32, one rounding to the model dtype; K, lda, ldb multiples of 8;
// A and B 16-byte aligned; any M, N and ldc.
//
// Two kernels, both on v_mfma_f32_16x16x32_{bf16,f16}:
//
// * skinny (M <= 64, decode): the op streams the weight matrix once, so it is
//   bound by HBM bandwidth -- and, per CU, by how many cache lines its loads
//   touch: an MFMA fragment load of 16 rows touches 16 lines. Weight fragments
//   therefore go straight to registers (each weight byte is used once), while
//   activation tiles are loaded once per workgroup with contiguous 16-byte
//   loads into LDS and shared by the waves that own different output columns.
//   8 waves per workgroup, split between N (16 columns each) and K so that a
//   launch keeps >= 192 workgroups; buffer loads with descriptor bounds make
//   rows past M/N and columns past K read as zero, and a DEPTH-deep register
//   ring keeps weight loads in flight across the per-step barrier.
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
// Word 3 of a gfx9-family buffer resource for raw (untyped) loads.
constexpr int kRsrcWord3 = 0x00020000;
// Byte offset that is outside every buffer resource used here: loads there
// return zero without touching memory.
constexpr int kOutOfRange = 0x7fffffff;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0,
                                           static_cast<int>(bytes < kOutOfRange ? bytes : kOutOfRange), kRsrcWord3);
}

// ---------------------------------------------------------------------------
// Skinny kernel (M <= 64) with LDS-shared activations
// ---------------------------------------------------------------------------
// Workgroup = WN x WK waves: wave (wn, wk) owns output columns n0 + 16 wn ...
// and K chunks c = j * WK + wk (BK = 64 columns each). The activation tile
// of a chunk (16 MT rows x 64) is loaded once per K-group with contiguous
// 16-byte loads (8 lanes cover a 128-byte row segment), written to LDS and
// read by the WN waves of that group, so each activation byte crosses the
// L1 once per workgroup instead of once per wave. Weight fragments go
// straight from HBM to registers through a DEPTH-deep ring. All waves step
// through the chunks together (one barrier per step); the WK partial tiles
// are summed through LDS at the end.
constexpr int kLdsBK = 64;
constexpr int kLdsARow = kLdsBK + 8;  // padded LDS row (elements)

template <int MT, int WN>
struct ARegs {
  static constexpr int kVecs = 16 * MT * kLdsBK / 8;                             // 16-byte vectors per tile
  static constexpr int kPerLane = (kVecs + WN * kWave - 1) / (WN * kWave);     // per lane of the K-group
  static constexpr bool kPartial = kVecs % (WN * kWave) != 0;                  // some lanes idle
  u32x4 v[kPerLane];
};

template <typename E, int MT, int WN, int WK, int DEPTH>
__global__ __launch_bounds__(WN * WK * kWave) void gemm_skinny_lds_kernel(const uint16_t* __restrict__ A,
                                                                          const uint16_t* __restrict__ B,
                                                                          const uint16_t* __restrict__ bias,
                                                                          uint16_t* __restrict__ C, int M, int N,
                                                                          int K, int lda, int ldb, int ldc) {
  constexpr int NT = WN * WK * kWave;
  constexpr int KS = kLdsBK / 32;  // k-steps per chunk
  using AR = ARegs<MT, WN>;
  static_assert(!AR::kPartial || AR::kPerLane == 1, "a partial activation load is one vector per lane");
  // The activation tiles and, after the K loop's last barrier, the partial
  // output tiles share one LDS allocation.
  constexpr size_t kBytesA = sizeof(uint16_t) * WK * 2 * 16 * MT * kLdsARow;
  constexpr size_t kBytesRed = sizeof(f32x4) * WK * WN * MT * kWave;
  __shared__ __attribute__((aligned(16))) unsigned char smem[kBytesA > kBytesRed ? kBytesA : kBytesRed];
  auto lds_a = reinterpret_cast<uint16_t(*)[2][16 * MT * kLdsARow]>(smem);
  auto red = reinterpret_cast<f32x4(*)[WN][MT][kWave]>(smem);

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wn = wave % WN;
  const int wk = wave / WN;
  const int gl = wn * kWave + lane;  // lane index inside the K-group
  const int l16 = lane % 16;
  const int lg = lane / 16;
  const int n0 = blockIdx.x * (16 * WN);
  const int ncol0 = n0 + 16 * wn;

  const __amdgpu_buffer_rsrc_t rb =
      rsrc(B + static_cast<int64_t>(ncol0) * ldb, static_cast<int64_t>(max(0, min(16, N - ncol0))) * ldb * 2);
  const __amdgpu_buffer_rsrc_t ra = rsrc(A, static_cast<int64_t>(M) * lda * 2);
  const __amdgpu_buffer_rsrc_t r_none = rsrc(A, 0);
  const int boff = l16 * ldb * 2 + 16 * lg;

  const int n_chunks = (K + kLdsBK - 1) / kLdsBK;
  const int steps = (n_chunks + WK - 1) / WK;  // chunk steps of the whole workgroup

  // Activation tile of chunk c: vector v of the group covers row v / 8, columns 8 (v % 8) ...
  auto load_a = [&](int step, AR& r) {
    const int c = step * WK + wk;
    const bool live = step < steps && c < n_chunks;
    const __amdgpu_buffer_rsrc_t rr = live ? ra : r_none;
#pragma unroll
    for (int j = 0; j < AR::kPerLane; ++j) {
      const int v = gl + j * WN * kWave;
      const int row = v / 8;
      const int k = c * kLdsBK + 8 * (v % 8);
      const bool in = k < K && (!AR::kPartial || v < AR::kVecs);
      r.v[j] = __builtin_amdgcn_raw_buffer_load_b128(rr, in ? row * lda * 2 + 2 * k : kOutOfRange, 0, 0);
    }
  };
  auto store_a = [&](int buf, const AR& r) {
#pragma unroll
    for (int j = 0; j < AR::kPerLane; ++j) {
      const int v = gl + j * WN * kWave;
      if (!AR::kPartial || v < AR::kVecs) *reinterpret_cast<u32x4*>(&lds_a[wk][buf][(v / 8) * kLdsARow + 8 * (v % 8)]) = r.v[j];
    }
  };
  // Weight fragments of chunk step `step` for this wave: KS k-steps.
  auto load_b = [&](int step, u32x4 (&bf)[KS]) {
    const int c = step * WK + wk;
    const bool live = step < steps && c < n_chunks;
    const __amdgpu_buffer_rsrc_t rr = live ? rb : r_none;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int k = c * kLdsBK + 32 * s + 8 * lg;
      bf[s] = __builtin_amdgcn_raw_buffer_load_b128(rr, k < K ? boff + 2 * (c * kLdsBK + 32 * s) : kOutOfRange, 0, 0);
    }
  };

  f32x4 acc[MT];
#pragma unroll
  for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 bring[DEPTH][KS];
  AR areg;
  load_a(0, areg);
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) load_b(d, bring[d]);
  store_a(0, areg);
  load_a(1, areg);
  __syncthreads();

  for (int base = 0; base < steps; base += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int step = base + d;
      if (step < steps) {
        const uint16_t* at = lds_a[wk][step & 1];
#pragma unroll
        for (int s = 0; s < KS; ++s) {
#pragma unroll
          for (int i = 0; i < MT; ++i) {
            const u32x4 af = *reinterpret_cast<const u32x4*>(&at[(16 * i + l16) * kLdsARow + 32 * s + 8 * lg]);
            acc[i] = E::mfma_16x16x32(af, bring[d][s], acc[i]);
          }
        }
      }
      load_b(step + DEPTH, bring[d]);
      if (step + 1 < steps) store_a((step + 1) & 1, areg);
      load_a(step + 2, areg);
      __syncthreads();
    }
  }

#pragma unroll
  for (int i = 0; i < MT; ++i) red[wk][wn][i][lane] = acc[i];
  __syncthreads();

  // acc[i] of wave (wn, *) lane l, reg r: C[16 i + 4 (l/16) + r][n0 + 16 wn + l % 16].
  for (int e = threadIdx.x; e < MT * 16 * 16 * WN; e += NT) {
    const int cn = e % (16 * WN);
    const int m = e / (16 * WN);
    const int n = n0 + cn;
    if (m >= M || n >= N) continue;
    const int i = m / 16;
    const int src_lane = 16 * ((m % 16) / 4) + (cn % 16);
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < WK; ++w) v += red[w][cn / 16][i][src_lane][m % 4];
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
    {
      // 8 waves; as many along N as keep >= 192 workgroups (more columns per
      // workgroup share each activation tile), the rest split K.
      const int wn = (M > 32 && N >= 24576) ? 8 : (N >= 64 * 192 ? 4 : (N >= 32 * 192 ? 2 : 1));
      const int mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
      const dim3 g2(static_cast<unsigned>(ceil_div64(N, 16 * wn)));
      const dim3 b2(8 * kWave);
#define DK_SKINNY_LDS(MT_, WN_)                                                                               \
  hipLaunchKernelGGL((gemm_skinny_lds_kernel<E, MT_, WN_, 8 / WN_, 3>), g2, b2, 0, s, A, B, bias, C, M, N, K, lda, \
                     ldb, ldc)
      switch (mt * 10 + wn) {
        case 11: DK_SKINNY_LDS(1, 1); break;
        case 12: DK_SKINNY_LDS(1, 2); break;
        case 14: DK_SKINNY_LDS(1, 4); break;
        case 21: DK_SKINNY_LDS(2, 1); break;
        case 22: DK_SKINNY_LDS(2, 2); break;
        case 24: DK_SKINNY_LDS(2, 4); break;
        case 18: DK_SKINNY_LDS(1, 8); break;
        case 28: DK_SKINNY_LDS(2, 8); break;
        case 41: DK_SKINNY_LDS(4, 1); break;
        case 42: DK_SKINNY_LDS(4, 2); break;
        case 44: DK_SKINNY_LDS(4, 4); break;
        default: DK_SKINNY_LDS(4, 8); break;
      }
#undef DK_SKINNY_LDS
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
  if (M <= 64 && (static_cast<int64_t>(M) * lda * 2 >= (int64_t{1} << 31) || int64_t{16} * ldb * 2 >= (int64_t{1} << 31)))
    return fail("gemm_tn: row strides too large for 32-bit buffer offsets");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* a = static_cast<const uint16_t*>(A);
  const auto* b = static_cast<const uint16_t*>(B);
  const auto* bi = static_cast<const uint16_t*>(bias);
  auto* c = static_cast<uint16_t*>(C);
  const hipError_t e = dtype == DK_BFLOAT16 ? gemm::launch<Bf16>(a, b, bi, c, M, N, K, lda, ldb, ldc, s)
                                            : gemm::launch<F16>(a, b, bi, c, M, N, K, lda, ldb, ldc, s);
  return static_cast<int>(e);
}
