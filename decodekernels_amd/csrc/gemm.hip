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
//   Up to 14 waves per workgroup, split between N (16 columns each) and K; the
//   grid is planned at one workgroup per CU, with wide column tiles to cut the
//   activation re-reads and, given a workspace, the K reduction split over
//   workgroups (fp32 partial tiles summed in order by a second kernel). Buffer
//   loads with descriptor bounds make rows past M/N and columns past K read as
//   zero, and DEPTH-deep register rings of weights and activations keep loads
//   in flight across the per-step barrier.
// * LDS-DMA (M > 64, batched decode and prefill): A and B tiles go from HBM
//   straight into LDS (buffer_load ... lds), bank-conflict-free XOR-swizzled,
//   through a multi-stage ring; nine tile shapes from 256x256 down to 64x64,
//   picked per call by a throughput model so that batches of a few hundred
//   rows still fill all 256 CUs. The output tile leaves through the freed
//   ring, read back row by row for 16-byte stores. At M <= 64 its 64-row
//   tiles (64 or 128 columns, K split) replace the skinny kernel from M = 32
//   where they fill the CUs, and for N > 32768 (decode_dma_plan).
#include <algorithm>

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
#ifndef DK_SKINNY_ROT
#define DK_SKINNY_ROT 5  // unsplit K walk of workgroup x starts at chunk (x * DK_SKINNY_ROT) mod chunks
#endif
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
                                                                          int K, int lda, int ldb, int ldc,
                                                                          float* __restrict__ part, int k_split) {
  constexpr int NT = WN * WK * kWave;
  constexpr int KS = kLdsBK / 32;  // k-steps per chunk
  // Split-K (part != nullptr): workgroup row blockIdx.y covers K columns
  // [kb, ke) (k_split a multiple of kLdsBK) and writes its fp32 partial tile to
  // part[blockIdx.y][M][N], without the bias; a second kernel sums the splits.
  const int kb = part != nullptr ? static_cast<int>(blockIdx.y) * k_split : 0;
  const int ke = part != nullptr ? min(K, kb + k_split) : K;
  using AR = ARegs<MT, WN>;
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

  const int n_chunks = (ke - kb + kLdsBK - 1) / kLdsBK;
  const int steps = (n_chunks + WK - 1) / WK;  // chunk steps of the whole workgroup
  // Unsplit, every workgroup walks the whole K range in lockstep with the
  // others: at a given moment they read the same column offset of rows a
  // fixed stride apart, which at some base addresses lands on few HBM
  // channels (measured: qkv M=1 18.3 us at 11 of 12 weight placements, 14.9 at
  // the twelfth). Starting workgroup x's walk at chunk x * DK_SKINNY_ROT mod
  // n_chunks spreads the concurrent reads: 14.3-14.6 us at every placement,
  // gate_up M=16 54.5 -> 44.0 us. Split workgroups already start at different
  // K offsets (rotating them measured 1-5% slower). Chunk c of the walk reads
  // K chunk (c + rot) mod n_chunks; the partial sums are deterministic.
  const int rot = DK_SKINNY_ROT > 0 && part == nullptr && n_chunks > 0
                      ? static_cast<int>((blockIdx.x * static_cast<unsigned>(DK_SKINNY_ROT)) % n_chunks)
                      : 0;
  auto chunk = [&](int c) { return c + rot >= n_chunks ? c + rot - n_chunks : c + rot; };

  // Activation tile of chunk c: vector v of the group covers row v / 8, columns 8 (v % 8) ...
  auto load_a = [&](int step, AR& r) {
    const int c = step * WK + wk;
    const bool live = step < steps && c < n_chunks;
    const __amdgpu_buffer_rsrc_t rr = live ? ra : r_none;
    const int cc = chunk(c);
#pragma unroll
    for (int j = 0; j < AR::kPerLane; ++j) {
      const int v = gl + j * WN * kWave;
      const int row = v / 8;
      const int k = kb + cc * kLdsBK + 8 * (v % 8);
      const bool in = k < ke && (!AR::kPartial || v < AR::kVecs);
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
    const int cc = chunk(c);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const int k = kb + cc * kLdsBK + 32 * s + 8 * lg;
      bf[s] = __builtin_amdgcn_raw_buffer_load_b128(rr, k < ke ? boff + 2 * (kb + cc * kLdsBK + 32 * s) : kOutOfRange, 0,
                                                    0);
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
    if (part != nullptr) {
      part[(static_cast<int64_t>(blockIdx.y) * M + m) * N + n] = v;
      continue;
    }
    if (bias != nullptr) v += E::to_float(bias[n]);
    C[static_cast<int64_t>(m) * ldc + n] = E::from_float(v);
  }
}

// Sums the split-K partial tiles (of either kernel) in split order, adds the
// bias in fp32 and rounds once: C[m][n] = round(sum_s part[s][m][n] + bias[n]).
// One thread per 4 consecutive columns of a row; 16-byte loads when N % 4 == 0
// (every partial row then starts 16-byte aligned). With S > 0 (= splits) the
// S partial loads and the bias load are issued together before the in-order
// sum: loaded one split at a time, each waited for in turn, the reduce took
// S round trips. S = 0 is the general runtime-count loop.
template <typename E, int S>
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(const float* __restrict__ part, int splits, int M,
                                                                 int N, const uint16_t* __restrict__ bias,
                                                                 uint16_t* __restrict__ C, int ldc, int vec_store) {
  const int n4 = (N + 3) / 4;
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (idx >= static_cast<int64_t>(M) * n4) return;
  const int m = static_cast<int>(idx / n4);
  const int n = static_cast<int>(idx % n4) * 4;
  const int64_t plane = static_cast<int64_t>(M) * N;
  const float* p = part + static_cast<int64_t>(m) * N + n;
  auto load_bias = [&](float (&b)[4]) {  // columns past N are not stored: clamped addresses
    if (bias != nullptr) {
#pragma unroll
      for (int r = 0; r < 4; ++r) b[r] = E::to_float(bias[min(n + r, N - 1)]);
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) b[r] = 0.0f;
    }
  };
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  float b[4];
  if (S > 0 && N % 4 == 0) {
    f32x4 x[S > 0 ? S : 1];
#pragma unroll
    for (int sp = 0; sp < S; ++sp) x[sp] = *reinterpret_cast<const f32x4*>(p + sp * plane);
    load_bias(b);
#pragma unroll
    for (int sp = 0; sp < S; ++sp)
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] += x[sp][r];
  } else if (N % 4 == 0) {
    for (int sp = 0; sp < splits; ++sp) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(p + sp * plane);
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] += x[r];
    }
    load_bias(b);
  } else {
    for (int sp = 0; sp < splits; ++sp) {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (n + r < N) v[r] += p[sp * plane + r];
    }
    load_bias(b);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) v[r] += b[r];
  uint16_t* c = C + static_cast<int64_t>(m) * ldc + n;
  if (vec_store && n + 3 < N) {
    *reinterpret_cast<u32x2*>(c) = u32x2{pack2<E>(v[0], v[1]), pack2<E>(v[2], v[3])};
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r)
      if (n + r < N) c[r] = E::from_float(v[r]);
  }
}

template <typename E>
void launch_splitk_reduce(const float* part, int splits, int M, int N, const uint16_t* bias, uint16_t* C, int ldc,
                          hipStream_t s) {
  const int64_t threads = static_cast<int64_t>(M) * ((N + 3) / 4);
  const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
  const int vec = (ldc % 4 == 0 && aligned_to(C, 8)) ? 1 : 0;
#define DK_REDUCE_CASE(S_)                                                                                 \
  case S_:                                                                                                 \
    hipLaunchKernelGGL((gemm_splitk_reduce_kernel<E, S_>), grid, dim3(256), 0, s, part, splits, M, N, bias, C, \
                       ldc, vec);                                                                          \
    return;
  switch (splits) {
    DK_REDUCE_CASE(2)
    DK_REDUCE_CASE(3)
    DK_REDUCE_CASE(4)
    DK_REDUCE_CASE(5)
    DK_REDUCE_CASE(6)
    DK_REDUCE_CASE(7)
    DK_REDUCE_CASE(8)
    default:
      hipLaunchKernelGGL((gemm_splitk_reduce_kernel<E, 0>), grid, dim3(256), 0, s, part, splits, M, N, bias, C, ldc,
                         vec);
  }
#undef DK_REDUCE_CASE
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
                                                                   int lda, int ldb, int ldc, int vec_store,
                                                                   float* __restrict__ part, int k_split) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM / 16;  // 16-row fragments per wave
  constexpr int TN = BN / WN / 16;
  constexpr int LA = BM / 8 / NW;   // 1 KB DMA loads per wave per slice
  // B's 8-row load groups need not divide among the waves (256 x 224: 28 groups
  // for 8 waves); the waves past the last group skip their final load.
  constexpr int kGroupsB = BN / 8;
  constexpr int LB = (kGroupsB + NW - 1) / NW;
  constexpr bool kTailB = kGroupsB % NW != 0;
  constexpr int kSlice = (BM + BN) * 8;  // u32x4 per slice
  static_assert(BM % (8 * NW) == 0 && BN % 8 == 0 && TM >= 1 && TN >= 1 && BN % (16 * WN) == 0, "tile shape");
  static_assert(STAGES >= 2 && (STAGES - 2) * (LA + LB) < 64, "vmcnt range");
  // With uneven B loads the waves have different counts in flight, which only
  // a 2-stage ring's vmcnt(0) waits allow.
  static_assert(!kTailB || STAGES == 2, "uneven B loads need STAGES == 2");
  constexpr int kStagePitch = BN / WN * 2 + 16;         // bytes per staged output row
  constexpr int kStageWave = BM / WM * kStagePitch;     // bytes of one wave's staged tile
  constexpr int kLdsU4 = STAGES * kSlice > NW * kStageWave / 16 ? STAGES * kSlice : NW * kStageWave / 16;
  static_assert(kLdsU4 * 16 <= 160 * 1024, "LDS of one workgroup (gfx950: 160 KB)");
  __shared__ u32x4 lds[kLdsU4];

  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int wm = wave % WM;
  const int wn = wave / WM;
  const int l16 = lane % 16;
  const int lg = lane / 16;

  // Split-K (part != nullptr): workgroup row blockIdx.y covers K columns
  // [kb, ke) (k_split a multiple of kDmaBK) and writes its fp32 partial tile to
  // part[blockIdx.y][M][N], without the bias; gemm_splitk_reduce_kernel sums them.
  const int kb = part != nullptr ? static_cast<int>(blockIdx.y) * k_split : 0;
  const int ke = part != nullptr ? min(K, kb + k_split) : K;
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
  int offa[LA], ka[LA], offb[LB], kbc[LB];
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
    kbc[j] = 8 * c;
    offb[j] = r < rows_b && r < BN ? r * ldb * 2 + 16 * c : kOutOfRange;
  }
  // Issued for every slice index, also past the last one (those lanes are out
  // of range and move no data), so each wave keeps the same count in flight
  // from slice to slice.
  auto issue = [&](int t, int buf) {
    const int k0 = kb + t * kDmaBK;
    u32x4* base = lds + buf * kSlice;
#pragma unroll
    for (int j = 0; j < LA; ++j) {
      const int off = (offa[j] != kOutOfRange && k0 + ka[j] < ke) ? offa[j] + 2 * k0 : kOutOfRange;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ra, (__attribute__((address_space(3))) void*)(base + (wave + j * NW) * 64), 16, off, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < LB; ++j) {
      // A wave past B's last load group issues nothing (its LDS target would be past the slice).
      if (kTailB && j == LB - 1 && wave + j * NW >= kGroupsB) break;
      const int off = (offb[j] != kOutOfRange && k0 + kbc[j] < ke) ? offb[j] + 2 * k0 : kOutOfRange;
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

  const int ktiles = (ke - kb + kDmaBK - 1) / kDmaBK;
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
  if (part != nullptr) {  // fp32 partial tile, no bias
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * (BN / WN) + 16 * j + 4 * lg;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int m = m0 + wm * (BM / WM) + 16 * i + l16;
        if (m >= M) continue;
        float* prow = part + (static_cast<int64_t>(blockIdx.y) * M + m) * N;
        if (N % 4 == 0 && n + 3 < N) {
          *reinterpret_cast<f32x4*>(prow + n) = acc[i][j];
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < N) prow[n + r] = acc[i][j][r];
        }
      }
    }
    return;
  }

  // Every bias value this lane adds, loaded before any store, with clamped
  // addresses and no branch per element so that the loads issue together.
  // (Loaded one at a time under a bounds branch, each was waited for behind
  // the stores before it: up to 6 us at M = N = 4096.) Columns past N are
  // never stored, so their clamped values do not matter.
  float bj[TN][4];
  if (bias != nullptr) {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn * (BN / WN) + 16 * j + 4 * lg;
#pragma unroll
      for (int r = 0; r < 4; ++r) bj[j][r] = E::to_float(bias[min(n + r, N - 1)]);
    }
  } else {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) bj[j][r] = 0.0f;
  }

  // The output goes through LDS: each wave writes its (BM/WM) x (BN/WN) tile
  // into its own part of the ring in the MFMA layout (8 bytes per lane), then
  // reads it back row by row, 16 bytes per lane, so a store writes whole row
  // segments instead of 32-byte pieces of 16 rows. Rows are padded by 16 bytes.
  constexpr int kNc = BN / WN / 8;  // 16-byte chunks per tile row
  char* stg = reinterpret_cast<char*>(lds) + wave * kStageWave;
  __syncthreads();  // every wave is done with the ring
#pragma unroll
  for (int j = 0; j < TN; ++j) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int row = 16 * i + l16;
      const int c = 2 * j + lg / 2;
      float v[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] = acc[i][j][r] + bj[j][r];
      *reinterpret_cast<u32x2*>(stg + row * kStagePitch + c * 16 + (lg % 2) * 8) =
          u32x2{pack2<E>(v[0], v[1]), pack2<E>(v[2], v[3])};
    }
  }
  __syncthreads();  // the tile's rows come from the other lanes of the wave
  constexpr int kChunks = (BM / WM) * kNc;  // 16-byte chunks of a wave's tile
#pragma unroll
  for (int it = 0; it < (kChunks + kWave - 1) / kWave; ++it) {
    const int idx = it * kWave + lane;
    if (kChunks % kWave != 0 && idx >= kChunks) break;  // last pass part-filled (192 x 224: 10.5 passes)
    const int row = idx / kNc;
    const int c = idx % kNc;
    const u32x4 val = *reinterpret_cast<const u32x4*>(stg + row * kStagePitch + c * 16);
    const int m = m0 + wm * (BM / WM) + row;
    const int n = n0 + wn * (BN / WN) + 8 * c;
    if (m >= M) continue;
    uint16_t* crow = C + static_cast<int64_t>(m) * ldc;
    if (vec_store == 2 && n + 7 < N) {
      *reinterpret_cast<u32x4*>(crow + n) = val;
    } else if (vec_store == 1 && n + 7 < N) {
      *reinterpret_cast<u32x2*>(crow + n) = u32x2{val[0], val[1]};
      *reinterpret_cast<u32x2*>(crow + n + 4) = u32x2{val[2], val[3]};
    } else {
#pragma unroll
      for (int r = 0; r < 8; ++r)
        if (n + r < N) crow[n + r] = static_cast<uint16_t>(val[r / 2] >> (16 * (r % 2)));
    }
  }
}

// With part != nullptr the K splits write fp32 partial tiles; `reduce` then
// launches gemm_splitk_reduce_kernel, otherwise the caller consumes them.
template <typename E, int BM, int BN, int WM, int WN, int STAGES>
hipError_t launch_dma(const uint16_t* A, const uint16_t* B, const uint16_t* bias, uint16_t* C, int M, int N, int K,
                      int lda, int ldb, int ldc, hipStream_t s, float* part, int splits, int k_split, bool reduce) {
  const int64_t tiles = ceil_div64(M, BM) * ceil_div64(N, BN);
  // Output stores of 16 bytes, or 8 where C's rows allow only that.
  const int vec = (ldc % 8 == 0 && aligned_to(C, 16)) ? 2 : (ldc % 4 == 0 && aligned_to(C, 8)) ? 1 : 0;
  hipLaunchKernelGGL((gemm_dma_kernel<E, BM, BN, WM, WN, STAGES>),
                     dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(part != nullptr ? splits : 1)),
                     dim3(WM * WN * kWave), 0, s, A, B, bias, C, M, N, K, lda, ldb, ldc, vec, part,
                     part != nullptr ? k_split : K);
  if (part == nullptr || !reduce) return hipGetLastError();
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  launch_splitk_reduce<E>(part, splits, M, N, bias, C, ldc, s);
  return hipGetLastError();
}

using DmaLauncher = hipError_t (*)(const uint16_t*, const uint16_t*, const uint16_t*, uint16_t*, int, int, int, int,
                                   int, int, hipStream_t, float*, int, int, bool);

// Launchers of kDmaShapes' tile shapes, in the same order.
template <typename E>
const DmaLauncher* dma_launchers() {
  static const DmaLauncher fns[] = {
      launch_dma<E, 256, 256, 4, 2, 2>, launch_dma<E, 256, 224, 4, 2, 2>, launch_dma<E, 256, 192, 4, 2, 2>,
      launch_dma<E, 256, 128, 4, 2, 3>, launch_dma<E, 192, 224, 4, 2, 2>, launch_dma<E, 192, 192, 4, 2, 3>,
      launch_dma<E, 128, 128, 4, 2, 3>, launch_dma<E, 128, 64, 2, 2, 4>,  launch_dma<E, 64, 64, 2, 2, 4>,
  };
  return fns;
}

#ifndef DK_SKINNY_DEPTH
#define DK_SKINNY_DEPTH 2  // k-steps of weights and activations in flight per wave
#endif
#ifndef DK_SKINNY_MIN_WGS
#define DK_SKINNY_MIN_WGS 192  // wide plan (N > 32768): fewest workgroups the N split may leave, M > 16
#endif
#ifndef DK_SKINNY_MIN_WGS_M16
#define DK_SKINNY_MIN_WGS_M16 384  // the same for M <= 16
#endif

// Launch shape of the skinny kernel: MT 16-row activation tiles, WN x WK
// waves per workgroup (WN along N, 16 columns each; WK along K), and, with a
// workspace, the K reduction split over `splits` workgroup rows of k_split
// columns each.
struct SkinnyPlan {
  int mt, wn, wk, splits, k_split;
};

// Plan of grids with more than one workgroup per CU (N > 32768): as many waves
// along N as keep >= 384 (M <= 16) or >= 192 workgroups, the rest along K.
inline SkinnyPlan skinny_plan_wide(int M, int N, int K) {
  SkinnyPlan p{};
  p.mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  const int min_wgs = p.mt == 1 ? DK_SKINNY_MIN_WGS_M16 : DK_SKINNY_MIN_WGS;
  p.wn = (M > 32 && N >= 24576) ? 8 : (N >= 64 * min_wgs ? 4 : (N >= 32 * min_wgs ? 2 : 1));
  p.wk = 8 / p.wn;
  p.splits = 1;
  p.k_split = K;
  return p;
}

// Workgroup shapes (WN, WK) of the plans below, narrowest first.
constexpr int kSkinnyShapes[][2] = {{1, 8}, {2, 4}, {4, 2}, {6, 2}, {7, 2}, {8, 1}};
constexpr int kSkinnyCus = 256;

// The widest unsplit grid that fits one workgroup per CU (the narrowest shape
// with <= 256 column tiles); wn = 0 when none does.
inline SkinnyPlan skinny_plan_unsplit(int M, int N, int K) {
  SkinnyPlan p{};
  p.mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  p.splits = 1;
  p.k_split = K;
  for (const auto& sh : kSkinnyShapes) {
    if (ceil_div64(N, 16 * sh[0]) <= kSkinnyCus) {
      p.wn = sh[0];
      p.wk = sh[1];
      return p;
    }
  }
  return p;
}

// Every workgroup re-reads the activation rows of its K range (M x k_split
// elements) for its 16 WN x k_split weights, so wide column tiles cut that
// traffic; splitting K over workgroup rows then keeps the grid at the CU
// count, at the price of an fp32 partial tile per split and a second kernel
// that sums them. The plan, fitted to interleaved cold timings of every
// candidate shape at M = 1 ... 64 on the Llama-3-8B projections (bf16,
// MI355X):
//  1. the widest unsplit grid of at most one workgroup per CU, if it fills
//     >= 3/4 of the CUs and each workgroup re-reads <= 256 KiB of activations;
//  2. else, with a workspace, the grids of 2 ... 8 K splits (>= 512 columns
//     each, <= 256 workgroups) within 10% of the fullest one: the fewest
//     splits whose workgroups re-read at most max(128 KiB, half their weight
//     bytes) of activations, or failing that the fewest activation bytes;
//  3. else the unsplit grid of 1, or for N > 32768 (no grid of one workgroup
//     per CU) the wide plan.
// Picks (waves along N x along K, splits), with the unsplit K-walk rotation;
// us cold, interleaved with hipBLASLt, ratio to it:
//   qkv (N 6144, K 4096): M <= 32 2 x 4 unsplit, 14.4 (M=1, 0.86x) ... 18.7
//     (M=32, 1.05x); M = 48/64 6 x 2 with 4 splits, 21.3 (M=64, 1.00x);
//   o (N 4096): M <= 32 1 x 8 unsplit, 11.3 ... 14.6 (0.62 ... 0.93x);
//     M = 48/64 4 x 2 with 4 splits, 16.6 (M=64, 0.93x);
//   gate_up (N 28672): 7 x 2 unsplit, 43.9 (M=1, 0.71x) ... 51.4 (M=64, 0.92x);
//   down (N 4096, K 14336): M <= 8 1 x 8, 24.4 (0.88x); M = 16 / 32 2 x 4 / 4 x 2
//     with 2 / 4 splits, 29.3 (M=32, 0.86x); M = 48/64 8 x 1 with 8 splits,
//     33.0 (M=64, 0.65x).
// Each pick was the fastest candidate of its shape and M, except gate_up at
// M <= 32 before the rotation: there 4 x 2 (448 workgroups) was 6-8% faster on
// one of four machines and 7 x 2 7% faster on two. A 257th workgroup puts two
// on one CU and doubles that CU's time.
inline SkinnyPlan skinny_plan(int M, int N, int K, bool split_ok) {
  constexpr int64_t kKiB = 1024;
  SkinnyPlan u = skinny_plan_unsplit(M, N, K);
  if (u.wn > 0 && static_cast<int64_t>(M) * K * 2 <= 256 * kKiB &&
      4 * ceil_div64(N, 16 * u.wn) >= 3 * kSkinnyCus)
    return u;
  if (split_ok && K > 0) {
    struct Cand {
      int wn, wk, splits, k_split;
      int64_t wgs;
    };
    Cand cand[sizeof(kSkinnyShapes) / sizeof(kSkinnyShapes[0]) * 7];
    int nc = 0;
    int64_t max_wgs = 0;
    for (const auto& sh : kSkinnyShapes) {
      const int64_t tiles = ceil_div64(N, 16 * sh[0]);
      for (int s = 2; s <= 8; ++s) {
        if (K / s < 512) break;
        const int per = (K + s - 1) / s;
        const int ks = (per + kLdsBK - 1) / kLdsBK * kLdsBK;
        if ((K + ks - 1) / ks != s) continue;  // every split non-empty
        if (tiles * s > kSkinnyCus) break;
        cand[nc++] = Cand{sh[0], sh[1], s, ks, tiles * s};
        max_wgs = std::max(max_wgs, tiles * s);
      }
    }
    const Cand* best = nullptr;
    bool best_ok = false;
    for (int i = 0; i < nc; ++i) {
      const Cand& c = cand[i];
      if (10 * c.wgs < 9 * max_wgs) continue;  // within 10% of the fullest grid
      const int64_t act = static_cast<int64_t>(M) * c.k_split * 2;
      const int64_t wts = int64_t{16} * c.wn * c.k_split * 2;
      const bool ok = act <= std::max<int64_t>(128 * kKiB, wts / 2);
      if (best == nullptr || (ok && !best_ok)) {
        best = &c;
        best_ok = ok;
        continue;
      }
      if (ok != best_ok) continue;
      const int64_t best_act = static_cast<int64_t>(M) * best->k_split;
      const bool better = ok ? (c.splits < best->splits)
                             : (static_cast<int64_t>(M) * c.k_split < best_act ||
                                (static_cast<int64_t>(M) * c.k_split == best_act && c.splits < best->splits));
      if (better) best = &c;
    }
    if (best != nullptr) {
      SkinnyPlan p = u;
      p.wn = best->wn;
      p.wk = best->wk;
      p.splits = best->splits;
      p.k_split = best->k_split;
      return p;
    }
  }
  return u.wn > 0 ? u : skinny_plan_wide(M, N, K);
}

inline int64_t skinny_workspace_bytes(const SkinnyPlan& p, int M, int N) {
  return p.splits > 1 ? static_cast<int64_t>(p.splits) * M * N * static_cast<int64_t>(sizeof(float)) : 0;
}

// Plan of the LDS-DMA kernel (M > 64): tile shape and, with a workspace, K
// split over workgroup rows. Time model fitted to interleaved cold timings of
// every shape x {1, 2, 4, 8} splits on the Llama-3-8B projections at M = 128,
// 256 and 512 (mean 1.5% from the fastest, picks identical to the previous
// unsplit model at M >= 1000):
//   rounds(tiles x splits over 256 CUs) x tile flops per split / rate(shape)
//   + [splits > 1] (1.84 us + splits x M x N x 8 B / 4.68 TB/s),
// the last term the fp32 partials written and read back plus the reduce
// launch. Splits are considered only when the unsplit grid leaves CUs idle
// (< 256 tiles). Measured (us, cold): down (N 4096, K 14336) M = 128 73.2 ->
// 36.6 (128 x 128, 8 splits; hipBLASLt 83.6), M = 256 73.3 -> 50.9 (256 x 128,
// 8; 69.0), M = 512 105.3 -> 75.8 (256 x 128, 4; 100.4); o M = 128 24.6 ->
// 19.3 (64 x 64, 2); qkv M = 256 35.8 -> 33.5 (128 x 128, 2). The 256 x 192
// tile (rate placed between its neighbours from the qkv M = 4096 timing) fills
// whole rounds where 256 x 256 leaves the last one part-empty: qkv (N 6144)
// M = 1536 / 3072 / 4096 / 6000 103.9 / 188.3 / 194.1 / 298.7 -> 93.5 / 175.7
// / 182.2 / 258.1, N 3072 and 5120 at M = 4096 105.2 / 185.9 -> 98.3 / 175.3
// (each pick the fastest of the three 256-row tiles). The 256 x 224 tile does
// the same for N = 28672 (128 column tiles; its rate fitted to gate_up at
// M = 384 ... 4096, where 256 x 256 leaves the last round part-empty):
// gate_up M = 384 / 512 / 1024 / 1536 / 2048 / 3072 102.7 / 110.0 / 206.7 /
// 306.0 / 411.7 / 604.3 -> 96.9 / 104.3 / 197.0 / 289.5 / 378.0 / 570.7 (at
// M = 768 it ties 256 x 192, and the 192 x 224 tile below beats both; M = 4096
// keeps 256 x 256, measured faster).
// The 192 x 192 tile (8 waves, 3 stages; N = 6144 is 32 of its columns, so
// M = 1536 is one full round): its rate is the one, on a grid search over
// every (tile, split) candidate timed for six projections at M = 128 ... 6144,
// that adds no pick more than 2% slower than the plan before it. It takes qkv
// (N 6144) at M = 384 / 768 / 1536 / 3072 from 43.8 / 62.3 / 90.8 / 159.5 to
// 38.0 / 53.6 / 70.8 / 133.1 us (hipBLASLt 40.1 / 52.8 / 78.1 / 141.0).
// The 192 x 224 tile (2 stages, 106 KB; its last epilogue pass is half
// filled) got its rate the same way, on eight projections (Qwen2.5-7B's
// gate_up and down added): every rate in 4.51 ... 4.60 picks it for 12 shapes,
// none more than 0.4% slower, and from 4.61 on it displaces 192 x 192 at
// 7-32% cost. Gains: Llama gate_up M = 768 182.1 -> 166.1 us; Qwen2.5-7B down
// M = 384 ... 6144 4.5-7.5%, gate_up M = 512 5%, o M = 3072 6%, qkv M = 2048 7%.
struct DmaPlan {
  int shape, splits, k_split;
};

// Largest split-K workspace the plan asks for (bytes); larger splits are not considered.
constexpr int64_t kDmaMaxWorkspace = int64_t{64} << 20;

struct DmaShape {
  int bm, bn;
  double rate;  // TFLOP/s per CU
};
constexpr DmaShape kDmaShapes[] = {
    {256, 256, 5.355}, {256, 224, 4.95}, {256, 192, 5.15}, {256, 128, 4.776}, {192, 224, 4.55},
    {192, 192, 3.95},  {128, 128, 3.48}, {128, 64, 2.398}, {64, 64, 2.007},
};

inline DmaPlan dma_plan(int M, int N, int K, bool split_ok) {
  DmaPlan best{0, 1, K};
  double best_t = -1.0;
  for (int i = 0; i < static_cast<int>(sizeof(kDmaShapes) / sizeof(kDmaShapes[0])); ++i) {
    const DmaShape& sh = kDmaShapes[i];
    const int64_t tiles = ceil_div64(M, sh.bm) * ceil_div64(N, sh.bn);
    for (int s = 1; s <= 8; s *= 2) {
      int ks = K, sp = 1;
      if (s > 1) {
        if (!split_ok || tiles >= kSkinnyCus || K / s < 512) break;
        const int per = (K + s - 1) / s;
        ks = (per + kDmaBK - 1) / kDmaBK * kDmaBK;
        sp = (K + ks - 1) / ks;
        if (sp < 2) continue;
        if (static_cast<int64_t>(sp) * M * N * static_cast<int64_t>(sizeof(float)) > kDmaMaxWorkspace) break;
      }
      const double rounds = static_cast<double>(ceil_div64(tiles * sp, kSkinnyCus));
      double t = rounds * sh.bm * sh.bn * 2.0 * ks / 1e6 / sh.rate;
      if (sp > 1) t += 1.84 + static_cast<double>(sp) * M * N * 8 / 4.68e6;
      if (best_t < 0 || t < best_t) {
        best = DmaPlan{i, sp, ks};
        best_t = t;
      }
    }
  }
  return best;
}

inline int64_t dma_workspace_bytes(const DmaPlan& d, int M, int N) {
  return d.splits > 1 ? static_cast<int64_t>(d.splits) * M * N * static_cast<int64_t>(sizeof(float)) : 0;
}

// The LDS-DMA kernel at decode sizes (M <= 64), on one 64-row tile: column
// tiles of bn = 64 (4 waves, two workgroups per CU) or 128 (4 waves, one per
// CU), K split over workgroup rows. Where it applies it replaces the skinny
// plan; bn = 0 keeps the skinny kernel. Fitted to interleaved cold timings
// of both kernels at M = 1 ... 64 on the Llama-3-8B, Qwen2.5-7B and
// Qwen2.5-0.5B projections (every candidate below, bf16, with the split
// reduce):
//  * candidates: bn in {128, 64} x 1, 2, 4, 8 splits of >= 768 columns, at
//    most 256 workgroups; the pick streams the fewest weight bytes per
//    workgroup (bn x k_split), bn = 128 on a tie;
//  * it replaces the skinny plan when M >= 32 and the pick fills at least half
//    of the CUs: the skinny kernel's per-step activation work grows with M
//    while the tile's stays flat. Llama-3-8B at M = 64: qkv 20.9 -> 18.7 us
//    (128 x 4 splits), o 17.1 -> 14.9 (64 x 4), down 32.7 -> 30.1 (128 x 8);
//    qkv at M = 32 18.7 -> 17.2 (hipBLASLt 18.0). Below M = 32 the skinny
//    plans are 5-10% faster on the 8B shapes, and with fewer than 128
//    workgroups (the 0.5B model's small matrices) at every M. An unsplit
//    pick replaces only a skinny grid that leaves over a quarter of the CUs
//    idle (0.5B gate_up, 152 workgroups: 12.8 -> 10.4 us at M = 64), not a
//    full one (8B gate_up: 64 x 128 unsplit 56.4 against 51.8 us);
//  * for N > 32768, where no skinny grid fits one workgroup per CU, 64 x 64
//    unsplit at every M: Qwen2.5-7B gate_up (N 37888) 57.7 -> 56.0 us at
//    M = 1, 80.3 -> 65.6 at M = 64. At N <= 32768 the skinny kernel's full
//    one-per-CU grid stays (Llama-3-8B gate_up: 43.9 against 47.6 us).
struct DecodeDmaPlan {
  int bn, splits, k_split;
};

inline DecodeDmaPlan decode_dma_plan(int M, int N, int K, bool split_ok) {
  DecodeDmaPlan none{0, 1, K};
  if (M > 64 || K <= 0) return none;
  if (skinny_plan_unsplit(M, N, K).wn == 0) return DecodeDmaPlan{64, 1, K};
  if (M < 32) return none;
  DecodeDmaPlan best = none;
  int64_t best_bytes = -1, best_wgs = 0;
  for (const int bn : {128, 64}) {
    const int64_t tiles = ceil_div64(N, bn);
    for (int s = 1; s <= 8; s *= 2) {
      int ks = K, sp = 1;
      if (s > 1) {
        if (!split_ok) break;
        const int per = (K + s - 1) / s;
        ks = (per + kDmaBK - 1) / kDmaBK * kDmaBK;
        sp = (K + ks - 1) / ks;
        if (ks < 768) break;
        if (sp < 2) continue;
      }
      if (tiles * sp > kSkinnyCus) break;
      const int64_t bytes = static_cast<int64_t>(bn) * ks;
      if (best_bytes < 0 || bytes < best_bytes) {
        best = DecodeDmaPlan{bn, sp, ks};
        best_bytes = bytes;
        best_wgs = tiles * sp;
      }
    }
  }
  if (2 * best_wgs < kSkinnyCus) return none;
  if (best.splits == 1) {
    // Unsplit, a tile streams about the bytes per workgroup of the skinny
    // kernel's full grid, which its 14-wave workgroups stream faster.
    const SkinnyPlan u = skinny_plan_unsplit(M, N, K);
    if (4 * ceil_div64(N, 16 * u.wn) >= 3 * kSkinnyCus) return none;
  }
  return best;
}

inline int64_t decode_dma_workspace_bytes(const DecodeDmaPlan& d, int M, int N) {
  return d.bn > 0 && d.splits > 1 ? static_cast<int64_t>(d.splits) * M * N * static_cast<int64_t>(sizeof(float)) : 0;
}

// Launches C = A B^T (+ bias) with the plan for (M, N, K) and the workspace
// given. With deferred_splits != nullptr, a plan that splits K stops after the
// main kernel, leaving splits x M x N fp32 partial tiles (no bias) in the
// workspace for the caller to sum in split order, and reports the split count
// there (1: C was written directly). dma_ok: the row strides allow the LDS-DMA
// kernel's 32-bit offsets (M <= 64 then keeps to the skinny kernel without).
template <typename E>
hipError_t launch(const uint16_t* A, const uint16_t* B, const uint16_t* bias, uint16_t* C, int M, int N, int K,
                  int lda, int ldb, int ldc, void* workspace, int64_t workspace_bytes, hipStream_t s,
                  int* deferred_splits, bool dma_ok) {
  if (M <= 64) {
    constexpr DecodeDmaPlan kNone{0, 1, 0};
    DecodeDmaPlan d = dma_ok ? decode_dma_plan(M, N, K, true) : kNone;
    SkinnyPlan p = skinny_plan(M, N, K, true);
    // A workspace smaller than the plan's needs runs exactly the plan
    // without one (both kernels' choices then exclude splits).
    const int64_t need = d.bn > 0 ? decode_dma_workspace_bytes(d, M, N) : skinny_workspace_bytes(p, M, N);
    if (need > 0 && (workspace == nullptr || need > workspace_bytes)) {
      d = dma_ok ? decode_dma_plan(M, N, K, false) : kNone;
      p = skinny_plan(M, N, K, false);
    }
    if (d.bn > 0) {
      if (deferred_splits != nullptr) *deferred_splits = d.splits;
      const DmaLauncher fn = d.bn == 64 ? launch_dma<E, 64, 64, 2, 2, 4> : launch_dma<E, 64, 128, 2, 2, 4>;
      return fn(A, B, bias, C, M, N, K, lda, ldb, ldc, s, d.splits > 1 ? static_cast<float*>(workspace) : nullptr,
                d.splits, d.k_split, deferred_splits == nullptr);
    }
    float* part = p.splits > 1 ? static_cast<float*>(workspace) : nullptr;
    if (deferred_splits != nullptr) *deferred_splits = p.splits;
    const dim3 g2(static_cast<unsigned>(ceil_div64(N, 16 * p.wn)), static_cast<unsigned>(p.splits));
#define DK_SKINNY_LDS(MT_, WN_, WK_)                                                                 \
  case MT_ * 100 + WN_ * 10 + WK_:                                                                   \
    hipLaunchKernelGGL((gemm_skinny_lds_kernel<E, MT_, WN_, WK_, DK_SKINNY_DEPTH>), g2, dim3(WN_ * WK_ * kWave), 0, s, \
                       A, B, bias, C, M, N, K, lda, ldb, ldc, part, p.k_split);                            \
    break;
#define DK_SKINNY_MT(MT_)                                                                                 \
  DK_SKINNY_LDS(MT_, 1, 8) DK_SKINNY_LDS(MT_, 2, 4) DK_SKINNY_LDS(MT_, 4, 2) DK_SKINNY_LDS(MT_, 6, 2)     \
  DK_SKINNY_LDS(MT_, 7, 2) DK_SKINNY_LDS(MT_, 8, 1)
    switch (p.mt * 100 + p.wn * 10 + p.wk) {
      DK_SKINNY_MT(1)
      DK_SKINNY_MT(2)
      DK_SKINNY_MT(4)
      default: return hipErrorInvalidValue;  // not a shape the plans produce
    }
#undef DK_SKINNY_MT
#undef DK_SKINNY_LDS
    if (part != nullptr && deferred_splits == nullptr) {
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      launch_splitk_reduce<E>(part, p.splits, M, N, bias, C, ldc, s);
    }
    return hipGetLastError();
  }
  const DmaPlan d = dma_plan(M, N, K, workspace != nullptr);
  const bool split = d.splits > 1 && dma_workspace_bytes(d, M, N) <= workspace_bytes;
  const DmaPlan u = split ? d : dma_plan(M, N, K, false);
  if (deferred_splits != nullptr) *deferred_splits = u.splits;
  return dma_launchers<E>()[u.shape](A, B, bias, C, M, N, K, lda, ldb, ldc, s,
                                     split ? static_cast<float*>(workspace) : nullptr, u.splits, u.k_split,
                                     deferred_splits == nullptr);
}

}  // namespace gemm
}  // namespace dk

namespace {

int gemm_tn_checked(int dtype, const void* A, const void* B, const void* bias, void* C, int M, int N, int K, int lda,
                    int ldb, int ldc, void* workspace, int64_t workspace_bytes, void* stream,
                    int* deferred_splits = nullptr) {
  using namespace dk;
  clear_error();
  if (dtype != DK_FLOAT16 && dtype != DK_BFLOAT16)
    return fail("gemm_tn: expected float16 or bfloat16, got dtype code %d", dtype);
  if (M < 0 || N < 0 || K < 0) return fail("gemm_tn: M, N and K must be non-negative");
  if (M == 0 || N == 0) return hipSuccess;
  // A lone row's stride is never used: take the row length. Otherwise a row
  // stride below the row length would overlap rows, cut the last rows off the
  // load descriptors' extents (read as zeros) and write C out of bounds.
  if (M == 1) {
    lda = K;
    ldc = N;
  }
  if (N == 1) ldb = K;
  if (lda < K || ldb < K || ldc < N)
    return fail("gemm_tn: row strides must be at least the row lengths (lda, ldb >= K, ldc >= N)");
  if (K % 8 != 0 || lda % 8 != 0 || ldb % 8 != 0)
    return fail("gemm_tn: K and row strides of a/b must be multiples of 8");
  if (!aligned_to(A, 16) || !aligned_to(B, 16)) return fail("gemm_tn: a and b must be 16-byte aligned");
  if (C == nullptr || (K > 0 && (A == nullptr || B == nullptr))) return fail("gemm_tn: pointers must not be NULL");
  if (workspace != nullptr && !aligned_to(workspace, 16)) return fail("gemm_tn: workspace must be 16-byte aligned");
  if (workspace_bytes < 0) return fail("gemm_tn: workspace_bytes must be non-negative");
  if (M > 64 && ceil_div64(M, 64) * ceil_div64(N, 64) >= (int64_t{1} << 31)) return fail("gemm_tn: M x N is too large");
  const bool dma_ok = int64_t{256} * std::max(lda, ldb) * 2 < (int64_t{1} << 31);
  if (M > 64 && !dma_ok) return fail("gemm_tn: row strides too large for 32-bit buffer offsets");
  if (M <= 64 && (static_cast<int64_t>(M) * lda * 2 >= (int64_t{1} << 31) || int64_t{16} * ldb * 2 >= (int64_t{1} << 31)))
    return fail("gemm_tn: row strides too large for 32-bit buffer offsets");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const auto* a = static_cast<const uint16_t*>(A);
  const auto* b = static_cast<const uint16_t*>(B);
  const auto* bi = static_cast<const uint16_t*>(bias);
  auto* c = static_cast<uint16_t*>(C);
  const hipError_t e =
      dtype == DK_BFLOAT16
          ? gemm::launch<Bf16>(a, b, bi, c, M, N, K, lda, ldb, ldc, workspace, workspace_bytes, s, deferred_splits,
                               dma_ok)
          : gemm::launch<F16>(a, b, bi, c, M, N, K, lda, ldb, ldc, workspace, workspace_bytes, s, deferred_splits,
                              dma_ok);
  return static_cast<int>(e);
}

}  // namespace

extern "C" int dk_gemm_tn(int dtype, const void* A, const void* B, const void* bias, void* C, int M, int N, int K,
                          int lda, int ldb, int ldc, void* stream) {
  return gemm_tn_checked(dtype, A, B, bias, C, M, N, K, lda, ldb, ldc, nullptr, 0, stream);
}

extern "C" int64_t dk_gemm_tn_workspace_bytes(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  if (M > 64) return dk::gemm::dma_workspace_bytes(dk::gemm::dma_plan(M, N, K, true), M, N);
  const dk::gemm::DecodeDmaPlan d = dk::gemm::decode_dma_plan(M, N, K, true);
  if (d.bn > 0) return dk::gemm::decode_dma_workspace_bytes(d, M, N);
  const dk::gemm::SkinnyPlan p = dk::gemm::skinny_plan(M, N, K, true);
  return dk::gemm::skinny_workspace_bytes(p, M, N);
}

extern "C" int dk_gemm_tn_plan(int M, int N, int K, int with_workspace, int* plan) {
  dk::clear_error();
  if (plan == nullptr) return dk::fail("gemm_tn_plan: plan must not be NULL");
  if (M <= 0 || N <= 0 || K < 0) return dk::fail("gemm_tn_plan: M and N must be positive, K non-negative");
  if (M > 64) {
    const dk::gemm::DmaPlan d = dk::gemm::dma_plan(M, N, K, with_workspace != 0);
    plan[0] = dk::gemm::kDmaShapes[d.shape].bm;
    plan[1] = dk::gemm::kDmaShapes[d.shape].bn;
    plan[2] = d.splits;
    plan[3] = d.k_split;
    return hipSuccess;
  }
  const dk::gemm::DecodeDmaPlan d = dk::gemm::decode_dma_plan(M, N, K, with_workspace != 0);
  if (d.bn > 0) {
    plan[0] = 64;
    plan[1] = d.bn;
    plan[2] = d.splits;
    plan[3] = d.k_split;
    return hipSuccess;
  }
  const dk::gemm::SkinnyPlan p = dk::gemm::skinny_plan(M, N, K, with_workspace != 0);
  plan[0] = p.wn;
  plan[1] = p.wk;
  plan[2] = p.splits;
  plan[3] = p.k_split;
  return hipSuccess;
}

extern "C" int dk_gemm_tn_ws(int dtype, const void* A, const void* B, const void* bias, void* C, int M, int N, int K,
                             int lda, int ldb, int ldc, void* workspace, int64_t workspace_bytes, void* stream) {
  return gemm_tn_checked(dtype, A, B, bias, C, M, N, K, lda, ldb, ldc, workspace, workspace_bytes, stream);
}

// gemm_tn followed by fused_add_rms_norm on its output, with the split-K sum
// of decode-size plans done inside the norm's kernel (one launch fewer, the
// GEMM output never written before the norm). Results equal dk_gemm_tn_ws into
// `out` followed by dk_fused_add_rms_norm(out, residual, weight, eps) bit for
// bit; rows whose norm cannot take its vector path run exactly that pair.
extern "C" int dk_gemm_tn_add_rms_norm(int dtype, const void* A, const void* B, const void* bias, void* out,
                                       void* residual, const void* weight, float eps, int M, int N, int K, int lda,
                                       int ldb, int ld_out, int ld_res, void* workspace, int64_t workspace_bytes,
                                       void* stream) {
  using namespace dk;
  clear_error();
  if (dtype != DK_FLOAT16 && dtype != DK_BFLOAT16)
    return fail("gemm_tn_add_rms_norm: expected float16 or bfloat16, got dtype code %d", dtype);
  if (M < 0 || N < 0 || K < 0) return fail("gemm_tn: M, N and K must be non-negative");
  if (M == 0 || N == 0) return hipSuccess;
  if (out == nullptr || residual == nullptr || weight == nullptr)
    return fail("gemm_tn_add_rms_norm: out, residual and weight must not be NULL");
  if (ld_out < N || ld_res < N) return fail("gemm_tn_add_rms_norm: row strides of out and residual must be >= N");
  const bool fused = fused_add_rms_norm_vectorizable(N, ld_out, ld_res, out, residual, weight);
  int splits = 1;
  const int rc = gemm_tn_checked(dtype, A, B, bias, out, M, N, K, lda, ldb, ld_out, workspace, workspace_bytes,
                                 stream, fused ? &splits : nullptr);
  if (rc != hipSuccess) return rc;
  if (splits > 1)
    return launch_splitk_fused_add_rms_norm(dtype, static_cast<const float*>(workspace), splits, bias, out, ld_out,
                                            residual, ld_res, weight, M, N, eps, static_cast<hipStream_t>(stream));
  return dk_fused_add_rms_norm(dtype, out, residual, weight, M, N, ld_out, ld_res, eps, stream);
}

namespace {

int gemm_tn_rope_cache(const char* op, int dtype, const void* A, const void* B, const void* bias, void* C, int M, int N,
                       int K, int lda, int ldb, int ldc, const dk_rotary_params* r, const dk_cache_write_params* c,
                       bool fp8, float k_scale, float v_scale, void* workspace, int64_t workspace_bytes,
                       void* stream) {
  using namespace dk;
  clear_error();
  if (dtype != DK_FLOAT16 && dtype != DK_BFLOAT16) return fail("%s: expected float16 or bfloat16, got dtype code %d", op, dtype);
  if (M < 0 || N < 0 || K < 0) return fail("gemm_tn: M, N and K must be non-negative");
  if (M == 0 || N == 0) return hipSuccess;
  if (C == nullptr) return fail("gemm_tn: pointers must not be NULL");
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Everything is checked before the GEMM runs, so a bad rotary / cache
  // argument leaves C untouched.
  if (const int rc = rotary_and_cache_on_rows(op, r, c, dtype, fp8, k_scale, v_scale, nullptr, 1, bias, C, ldc, M, N,
                                              true, s))
    return rc;
  int splits = 1;
  const int rc = gemm_tn_checked(dtype, A, B, bias, C, M, N, K, lda, ldb, ldc, workspace, workspace_bytes, stream,
                                 &splits);
  if (rc != hipSuccess) return rc;
  return rotary_and_cache_on_rows(op, r, c, dtype, fp8, k_scale, v_scale,
                                  splits > 1 ? static_cast<const float*>(workspace) : nullptr, splits, bias, C, ldc, M, N,
                                  false, s);
}

}  // namespace

// gemm_tn into C (e.g. a fused q | k | v projection) followed by
// rotary_embedding_and_cache on q / k / v views of C's rows; a plan that
// splits K forms each token's row of C from the partial tiles inside the
// rotary / cache kernel (one launch fewer). Results equal dk_gemm_tn_ws then
// dk_rotary_embedding_and_cache bit for bit.
extern "C" int dk_gemm_tn_rotary_embedding_and_cache(int dtype, const void* A, const void* B, const void* bias, void* C,
                                                     int M, int N, int K, int lda, int ldb, int ldc,
                                                     const dk_rotary_params* r, const dk_cache_write_params* c,
                                                     void* workspace, int64_t workspace_bytes, void* stream) {
  return gemm_tn_rope_cache("gemm_tn_rotary_embedding_and_cache", dtype, A, B, bias, C, M, N, K, lda, ldb, ldc, r, c,
                            false, 1.0f, 1.0f, workspace, workspace_bytes, stream);
}

// The same into fp8 (e4m3fn) caches (dk_rotary_embedding_and_cache_fp8).
extern "C" int dk_gemm_tn_rotary_embedding_and_cache_fp8(int dtype, const void* A, const void* B, const void* bias,
                                                         void* C, int M, int N, int K, int lda, int ldb, int ldc,
                                                         const dk_rotary_params* r, const dk_cache_write_params* c,
                                                         float k_scale, float v_scale, void* workspace,
                                                         int64_t workspace_bytes, void* stream) {
  return gemm_tn_rope_cache("gemm_tn_rotary_embedding_and_cache_fp8", dtype, A, B, bias, C, M, N, K, lda, ldb, ldc, r,
                            c, true, k_scale, v_scale, workspace, workspace_bytes, stream);
}
