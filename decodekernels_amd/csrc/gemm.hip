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
//   launch keeps >= 384 (M <= 16) or >= 192 workgroups; buffer loads with
//   descriptor bounds make rows past M/N and columns past K read as zero, and
//   DEPTH-deep register rings of weights and activations keep loads in flight
//   across the per-step barrier.
// * LDS-DMA (M > 64, batched decode and prefill): A and B tiles go from HBM
//   straight into LDS (buffer_load ... lds), bank-conflict-free XOR-swizzled,
//   through a multi-stage ring; five tile shapes from 256x256 down to 64x64,
//   picked per call by a throughput model so that batches of a few hundred
//   rows still fill all 256 CUs.
#include "../../include/decodekernels_amd.h"
#include "dk_device.h"
#include "dk_host.h"

namespace dk {
namespace gemm {

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
// straight from HBM to registers; weights and activations both run through
// DEPTH-deep register rings. All waves step through the chunks together (one
// barrier per step); the WK partial tiles are summed through LDS at the end.
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

  // Step j's weight fragments and activation vectors live in ring slot
  // j % DEPTH; both are issued DEPTH steps ahead. Loads complete in issue
  // order, so the wait for step j + 1's activations (stored to LDS during
  // step j) covers only loads issued up to step j + 1 - DEPTH: DEPTH - 1
  // steps of both operands stay in flight across each barrier.
  u32x4 bring[DEPTH][KS];
  AR aring[DEPTH];
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) {
    load_a(d, aring[d]);
    load_b(d, bring[d]);
  }
  store_a(0, aring[0]);
  load_a(DEPTH, aring[0]);
  __syncthreads();

  for (int base = 0; base < steps; base += DEPTH) {
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
      const int step = base + d;
      const int d1 = (d + 1) % DEPTH;
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
      if (step + 1 < steps) store_a((step + 1) & 1, aring[d1]);
      load_a(step + 1 + DEPTH, aring[d1]);
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
// LDS-DMA kernel (M > 64)
// ---------------------------------------------------------------------------
// BM x BN output tile per workgroup of WM x WN waves. K advances in 64-column
// slices; a slice of A (BM rows) and of B (BN rows) goes from HBM straight into
// LDS with buffer_load ... lds (16 bytes per lane, one 1 KB instruction per 8
// rows, no registers), through a STAGES-deep ring: slice t + STAGES - 1 is in
// flight while slice t is multiplied. A slice row is 128 bytes = 8 chunks of 16
// bytes, and chunk c of row r is stored at position c ^ (r & 7). gfx950's LDS
// has 64 banks of 4 bytes and serves a ds_read_b128 in four cycles of 16 lanes:
// the lanes that share bit 5 and the parity of bits 2..4 of the lane id
// (measured with SQ_LDS_BANK_CONFLICT on pairs of active lanes). A fragment
// read (lane l: row l % 16, chunk 2 (l / 32) + (l / 16) % 2 + 4 h) puts 8 rows
// with chunk c and 8 rows with chunk c ^ 1 in each such group, and the XOR
// sends those 16 reads to 16 distinct 16-byte bank groups; unswizzled or
// 16-byte-padded rows conflict 2-way. The load lanes fetch the permuted chunks,
// so global reads stay whole 128-byte row segments.
//
// Tiles are numbered so that each XCD (workgroups go to the 8 XCDs round
// robin) takes a contiguous run of them, walked in groups of kGroupM tile rows:
// the ~32 workgroups resident on one XCD share A rows and B rows in its L2.
constexpr int kDmaBK = 64;
constexpr int kXcds = 8;
#ifndef DK_GEMM_GROUP_M
#define DK_GEMM_GROUP_M 4  // tile rows per group of the XCD-contiguous tile order
#endif
constexpr int kGroupM = DK_GEMM_GROUP_M;

__device__ __forceinline__ int swz(int r) { return r & 7; }

template <int BM, int BN>
__device__ __forceinline__ void dma_tile_of(int id, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  int pid = id;
  if (total % kXcds == 0) pid = (id % kXcds) * (total / kXcds) + id / kXcds;
  const int per_group = kGroupM * tiles_n;
  const int first_m = (pid / per_group) * kGroupM;
  const int gm = min(tiles_m - first_m, kGroupM);
  tm = first_m + (pid % per_group) % gm;
  tn = (pid % per_group) / gm;
}

template <typename E, int BM, int BN, int WM, int WN, int STAGES>
__global__ __launch_bounds__(WM * WN * kWave) void gemm_dma_kernel(const uint16_t* __restrict__ A,
                                                                   const uint16_t* __restrict__ B,
                                                                   const uint16_t* __restrict__ bias,
                                                                   uint16_t* __restrict__ C, int M, int N, int K,
                                                                   int lda, int ldb, int ldc, int vec_store) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM / 16;  // 16-row fragments per wave
  constexpr int TN = BN / WN / 16;
  constexpr int LA = BM / 8 / NW;   // 1 KB DMA loads per wave per slice
  constexpr int LB = BN / 8 / NW;
  constexpr int kSlice = (BM + BN) * 8;  // u32x4 per slice
  static_assert(BM % (8 * NW) == 0 && BN % (8 * NW) == 0 && TM >= 1 && TN >= 1, "tile shape");
  static_assert(STAGES >= 2 && (STAGES - 2) * (LA + LB) < 64, "vmcnt range");
  __shared__ u32x4 lds[STAGES * kSlice];

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wm = wave % WM;
  const int wn = wave / WM;
  const int l16 = lane % 16;
  const int lg = lane / 16;

  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  int tm, tn;
  dma_tile_of<BM, BN>(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM;
  const int n0 = tn * BN;
  const int rows_a = min(BM, M - m0);
  const int rows_b = min(BN, N - n0);
  // Rows past M (N) lie past num_records and read as zero.
  const __amdgpu_buffer_rsrc_t ra =
      rsrc(A + static_cast<int64_t>(m0) * lda, (static_cast<int64_t>(rows_a - 1) * lda + K) * 2);
  const __amdgpu_buffer_rsrc_t rb =
      rsrc(B + static_cast<int64_t>(n0) * ldb, (static_cast<int64_t>(rows_b - 1) * ldb + K) * 2);

  // DMA lane roles: load j of this wave fills tile rows 8 g .. 8 g + 7 (g = wave + j NW);
  // lane l writes position l % 8 of row 8 g + l / 8, i.e. chunk (l % 8) ^ swz(row).
  int offa[LA], ka[LA], offb[LB], kb[LB];
#pragma unroll
  for (int j = 0; j < LA; ++j) {
    const int r = 8 * (wave + j * NW) + lane / 8;
    const int c = (lane % 8) ^ swz(r);
    ka[j] = 8 * c;
    offa[j] = r < rows_a ? r * lda * 2 + 16 * c : kOutOfRange;
  }
#pragma unroll
  for (int j = 0; j < LB; ++j) {
    const int r = 8 * (wave + j * NW) + lane / 8;
    const int c = (lane % 8) ^ swz(r);
    kb[j] = 8 * c;
    offb[j] = r < rows_b ? r * ldb * 2 + 16 * c : kOutOfRange;
  }
  // Issued for every slice index, also past the last one (those lanes are out
  // of range and move no data), so each wave always has the same count in flight.
  auto issue = [&](int t, int buf) {
    const int k0 = t * kDmaBK;
    u32x4* base = lds + buf * kSlice;
#pragma unroll
    for (int j = 0; j < LA; ++j) {
      const int off = (offa[j] != kOutOfRange && k0 + ka[j] < K) ? offa[j] + 2 * k0 : kOutOfRange;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ra, (__attribute__((address_space(3))) void*)(base + (wave + j * NW) * 64), 16, off, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < LB; ++j) {
      const int off = (offb[j] != kOutOfRange && k0 + kb[j] < K) ? offb[j] + 2 * k0 : kOutOfRange;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rb, (__attribute__((address_space(3))) void*)(base + BM * 8 + (wave + j * NW) * 64), 16, off, 0, 0, 0);
    }
  };

  // Fragment read offsets (u32x4) inside a slice, for the two 32-column halves.
  int ia[TM][2], ib[TN][2];
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int r = wm * (BM / WM) + 16 * i + l16;
    ia[i][0] = r * 8 + (lg ^ swz(r));
    ia[i][1] = r * 8 + ((4 + lg) ^ swz(r));
  }
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int r = wn * (BN / WN) + 16 * j + l16;
    ib[j][0] = BM * 8 + r * 8 + (lg ^ swz(r));
    ib[j][1] = BM * 8 + r * 8 + ((4 + lg) ^ swz(r));
  }

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int ktiles = (K + kDmaBK - 1) / kDmaBK;
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s) issue(s, s);

  // vmcnt(n) with expcnt / lgkmcnt left at their maxima (gfx9 encoding).
  constexpr int kWaitN = (STAGES - 2) * (LA + LB);
  constexpr int kWaitImm = (kWaitN & 15) | ((kWaitN >> 4) << 14) | (7 << 4) | (15 << 8);

  for (int t0 = 0; t0 < ktiles; t0 += STAGES) {
#pragma unroll
    for (int u = 0; u < STAGES; ++u) {
      if (t0 + u < ktiles) {
        // This wave's loads of slice t0 + u have landed; the barrier extends that
        // to every wave and ensures all reads of the buffer refilled next are done.
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(kWaitImm);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        issue(t0 + u + STAGES - 1, (u + STAGES - 1) % STAGES);
        const u32x4* sl = lds + u * kSlice;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          u32x4 af[TM], bf[TN];
#pragma unroll
          for (int i = 0; i < TM; ++i) af[i] = sl[ia[i][h]];
#pragma unroll
          for (int j = 0; j < TN; ++j) bf[j] = sl[ib[j][h]];
          // A wave that has its fragments issues its MFMAs ahead of the other
          // wave on the SIMD, which meanwhile reads its own: the two drift
          // out of phase instead of reading and multiplying in lockstep
          // (measured 1-4% at M = 1024 / 4096).
          __builtin_amdgcn_s_setprio(1);
#pragma unroll
          for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = E::mfma_16x16x32(bf[j], af[i], acc[i][j]);
          __builtin_amdgcn_s_setprio(0);
        }
      }
    }
  }

  // The loads issued past the last slice move no data, but none may still be
  // in flight into this workgroup's LDS when it exits.
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));

  // acc[i][j] lane l, reg r = C[m0 + wm BM/WM + 16 i + l % 16][n0 + wn BN/WN + 16 j + 4 (l / 16) + r].
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int m = m0 + wm * (BM / WM) + 16 * i + l16;
    if (m >= M) continue;
    uint16_t* crow = C + static_cast<int64_t>(m) * ldc;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * (BN / WN) + 16 * j + 4 * lg;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r)
        v[r] = acc[i][j][r] + (bias != nullptr && n + r < N ? E::to_float(bias[n + r]) : 0.0f);
      if (vec_store && n + 3 < N) {
        *reinterpret_cast<u32x2*>(crow + n) = u32x2{pack2<E>(v[0], v[1]), pack2<E>(v[2], v[3])};
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < N) crow[n + r] = E::from_float(v[r]);
      }
    }
  }
}

template <typename E, int BM, int BN, int WM, int WN, int STAGES>
hipError_t launch_dma(const uint16_t* A, const uint16_t* B, const uint16_t* bias, uint16_t* C, int M, int N, int K,
                      int lda, int ldb, int ldc, hipStream_t s) {
  const int64_t tiles = ceil_div64(M, BM) * ceil_div64(N, BN);
  const int vec = (ldc % 4 == 0 && aligned_to(C, 8)) ? 1 : 0;
  hipLaunchKernelGGL((gemm_dma_kernel<E, BM, BN, WM, WN, STAGES>), dim3(static_cast<unsigned>(tiles)),
                     dim3(WM * WN * kWave), 0, s, A, B, bias, C, M, N, K, lda, ldb, ldc, vec);
  return hipGetLastError();
}

#ifndef DK_SKINNY_WAVES
#define DK_SKINNY_WAVES 8  // waves per skinny workgroup
#endif
#ifndef DK_SKINNY_DEPTH
#define DK_SKINNY_DEPTH 2  // k-steps of weights and activations in flight per wave
#endif
#ifndef DK_SKINNY_MIN_WGS
#define DK_SKINNY_MIN_WGS 192  // fewest workgroups the N split may leave, M > 16
#endif
#ifndef DK_SKINNY_MIN_WGS_M16
#define DK_SKINNY_MIN_WGS_M16 384  // the same for M <= 16
#endif

template <typename E>
hipError_t launch(const uint16_t* A, const uint16_t* B, const uint16_t* bias, uint16_t* C, int M, int N, int K,
                  int lda, int ldb, int ldc, hipStream_t s) {
  if (M <= 64) {
    {
      // DK_SKINNY_WAVES waves; as many along N as keep enough workgroups
      // (more columns per workgroup share each activation tile), the rest
      // split K. Measured: with one 16-row activation tile (M <= 16) the
      // activation traffic is small and 384 workgroups beat 192 (qkv, N =
      // 6144); with 32 or 64 rows the activation tile reloads cost more.
      constexpr int kW = DK_SKINNY_WAVES;
      const int mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
      const int min_wgs = mt == 1 ? DK_SKINNY_MIN_WGS_M16 : DK_SKINNY_MIN_WGS;
      int wn = (M > 32 && N >= 24576) ? 8 : (N >= 64 * min_wgs ? 4 : (N >= 32 * min_wgs ? 2 : 1));
      wn = wn > kW ? kW : wn;
      const dim3 g2(static_cast<unsigned>(ceil_div64(N, 16 * wn)));
#define DK_SKINNY_LDS(MT_, WN_)                                                                          \
  hipLaunchKernelGGL((gemm_skinny_lds_kernel<E, MT_, WN_, (kW / WN_ > 0 ? kW / WN_ : 1), DK_SKINNY_DEPTH>), g2, \
                     dim3(WN_ * (kW / WN_ > 0 ? kW / WN_ : 1) * kWave), 0, s, A, B, bias, C, M, N, K, lda, ldb, ldc)
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
  // Tile shape by a throughput model fitted to measured bf16 runs at K = 4096
  // and 14336: time ~ ceil(tiles / 256 CUs) x tile flops / per-CU rate of the
  // shape (TFLOP/s). Large tiles move fewer bytes per flop through L2 and LDS;
  // small ones keep all 256 CUs busy when M is a few hundred rows.
  struct Shape {
    int bm, bn;
    double rate;
    hipError_t (*fn)(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int, int, int,
                     hipStream_t);
  };
  static const Shape shapes[] = {
      {256, 256, 4.7, launch_dma<E, 256, 256, 4, 2, 2>},
      {256, 128, 4.2, launch_dma<E, 256, 128, 4, 2, 3>},
      {128, 128, 3.2, launch_dma<E, 128, 128, 4, 2, 3>},
      {128, 64, 2.2, launch_dma<E, 128, 64, 2, 2, 4>},
      {64, 64, 1.4, launch_dma<E, 64, 64, 2, 2, 4>},
  };
  const Shape* best = nullptr;
  double best_t = 0.0;
  for (const Shape& sh : shapes) {
    const double rounds = static_cast<double>(ceil_div64(ceil_div64(M, sh.bm) * ceil_div64(N, sh.bn), 256));
    const double t = rounds * sh.bm * sh.bn / sh.rate;
    if (best == nullptr || t < best_t) {
      best = &sh;
      best_t = t;
    }
  }
  return best->fn(A, B, bias, C, M, N, K, lda, ldb, ldc, s);
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
  if (M > 64 && ceil_div64(M, 64) * ceil_div64(N, 64) >= (int64_t{1} << 31)) return fail("gemm_tn: M x N is too large");
  if (M > 64 && int64_t{256} * std::max(lda, ldb) * 2 >= (int64_t{1} << 31))
    return fail("gemm_tn: row strides too large for 32-bit buffer offsets");
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
