// Paged decode attention for gfx950: one query token per sequence attends
// over a paged KV cache, with flash-decoding split-K for long contexts.
//
// Semantics follow DecodeKernels' dk::launch_paged_attention_decode
// (csrc/paged_attention.cuh:73-333): GQA-aware work units (one KV head and
// its whole query-head group), 512-token partitions when max_seq_len > 512,
// each writing its normalised partial output plus (max logit, exp-sum) to a
// caller-owned fp32 workspace, then a log-sum-exp merge. Empty sequences
// give exact zeros.
//
// The decomposition is CDNA4-specific:
//
// * A work unit is a token range of one KV head x one sequence with the
//   KV head's whole query-head group; its tokens form 16-token tiles, wave w
//   of the workgroup takes tiles w, w + NW, ... (NW = 4, 2 at head_dim > 128)
//   with its own online-softmax state, and the waves merge through LDS (the
//   split-K log-sum-exp rule). Two drivers run units: the grid kernel (one
//   workgroup per 1024-token unit, two 512-token workspace slots) and the
//   balanced kernel (a resident-sized grid; each workgroup takes an equal
//   share of all tiles and writes one workspace row per piece). The reduce
//   kernel merges the rows of each query head.
// * Q.K^T for a tile is 16 tokens x 16 (padded) query heads x head_dim on
//   v_mfma_f32_16x16x32_{bf16,f16}. Lane l feeds K row (l % 16) with one
//   16-byte load per 32-column step, and the query fragment of head (l % 16)
//   in the model dtype (exact); the fp32 logits come out as
//   S[token 4*(l/16)+r][head l%16], r = 0..3.
// * P.V on v_mfma_f32_16x16x16, whose A operand is P exactly as Q.K^T leaves
//   it; P is split into hi + lo parts in the model dtype (two MFMAs per
//   16-column block keep the products accurate to ~2^-17 relative). V is
//   loaded like K and brought into the B-operand layout through the wave's
//   LDS tile with ds_read_b64_tr_b16 transpose reads (or, DK_ATTN_VTR=0, by
//   MFMAs against an identity operand; the same bits). Accumulators: lane l
//   holds O[head 4*(l/16)+i][column 16n + l%16].
// * Logits are kept in log2 units (scale * log2 e folded into one multiply)
//   and exponentiated with v_exp_f32 against a lazily moved reference max;
//   max_logits are stored in natural-log units so the workspace means what
//   the reference's does.
// * K/V tiles run through DEPTH-deep register rings of raw buffer loads.
// * An fp8 (e4m3fn) cache takes the same path: K with 16-byte loads of 64
//   columns per lane group, V row-contiguous (whole 128-byte lines, as the
//   16-bit row loads), both converted exactly to the model dtype when a tile
//   is consumed; k_scale folds into the logit scale, v_scale into the output.
#include <algorithm>
#include <atomic>
#include <climits>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "../../include/decodekernels_amd.h"
#include "dk_device.h"
#include "dk_host.h"

namespace dk {
namespace attn {

constexpr int kPart = DK_PARTITION_SIZE;  // workspace slot (tokens), as the reference's partition
constexpr int kUnit = 2 * kPart;          // split-K work unit: two slots (its block-table entries fit one per lane)
// Tuning constants of the main kernel (compile-time; defaults are the tuned values).
#ifndef DK_ATTN_WAVES
#define DK_ATTN_WAVES 4  // waves per workgroup, head_dim <= 128
#endif
#ifndef DK_ATTN_WAVES_D256
#define DK_ATTN_WAVES_D256 2  // waves per workgroup, head_dim 256
#endif
#ifndef DK_ATTN_DEPTH
#define DK_ATTN_DEPTH 2  // tiles in flight per wave (head_dim <= 128)
#endif
#ifndef DK_ATTN_DEPTH_D256
#define DK_ATTN_DEPTH_D256 2  // tiles in flight per wave (head_dim 256)
#endif
#ifndef DK_ATTN_DEPTH_FP8
#define DK_ATTN_DEPTH_FP8 2  // tiles in flight per wave with an fp8 cache
#endif
#ifndef DK_ATTN_VTR
#define DK_ATTN_VTR 1  // V into the P.V operand layout: 1 LDS transpose reads, 0 identity MFMAs
#endif
#ifndef DK_ATTN_OCC_FP8_D128
#define DK_ATTN_OCC_FP8_D128 3  // waves per SIMD targeted at head_dim 128 with an fp8 cache
#endif
#ifndef DK_ATTN_OCC_FP8_D256
#define DK_ATTN_OCC_FP8_D256 1  // waves per SIMD targeted at head_dim 256 with an fp8 cache
#endif
#ifndef DK_ATTN_LOAD_AUX
#define DK_ATTN_LOAD_AUX 0  // cache-policy bits of the K/V buffer loads in the MFMA-operand layout
#endif
#ifndef DK_ATTN_FP8_K_AUX
#define DK_ATTN_FP8_K_AUX 2  // cache-policy bits of the fp8 K loads (2 = nt; measured 0.5-2% faster than 0)
#endif
#ifndef DK_ATTN_ROWLOAD
#define DK_ATTN_ROWLOAD 1  // 16-bit caches: K and V tiles load row-contiguous (whole 128-byte lines) through LDS
#endif
#ifndef DK_REDUCE_PRE
#define DK_REDUCE_PRE 2  // workspace rows per wave loaded in the reduce's first round trip
#endif
#ifndef DK_ATTN_ROW_AUX
#define DK_ATTN_ROW_AUX 2  // cache-policy bits of the row-contiguous K/V loads (2 = nt, non-temporal)
#endif
#ifndef DK_ATTN_OCC_D128
#define DK_ATTN_OCC_D128 2  // waves per SIMD targeted at head_dim 128
#endif
#ifndef DK_ATTN_OCC_D256
#define DK_ATTN_OCC_D256 1  // waves per SIMD targeted at head_dim 192 / 256
#endif
#ifndef DK_ATTN_OCC_D64
#define DK_ATTN_OCC_D64 4  // waves per SIMD targeted at head_dim 64
#endif
constexpr int kWaves = DK_ATTN_WAVES;
constexpr int kTile = 16;
constexpr int kMaxGroup = DK_MAX_GQA_GROUP;  // 16: the MFMA tile's padded head count
constexpr int kMergeHeads = 8;               // heads per LDS merge pass (two passes above 8)
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct KParams {
  uint16_t* out;
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* block_tables;
  const int32_t* seq_lens;
  float* tmp_out;
  float* max_logits;
  float* exp_sums;
  // Element strides, each below 2^31 (checked by the host); every address
  // computed from them is formed in 64 bits. As 32-bit kernel arguments they
  // take half the scalar registers, which the balanced kernel's schedule state
  // needs (with 64-bit strides it spilled scalar registers to VGPR lanes).
  int32_t q_ss, q_sh, o_ss, o_sh;
  int32_t k_sb, k_st, k_sh, v_sb, v_st, v_sh;
  int32_t bt_stride;
  int num_q_heads, group, block_size, max_partitions;
  int num_seqs, num_kv_heads;
  int num_units;  // split-K grid: unit positions per sequence, ceil(max_partitions / 2)
  int unit512;    // split-K grid: one 512-token unit per workspace row instead (small grids)
  int pair_ratio;  // balanced kernel: share of workgroups [0, grid/2) over the others', x100
  int lockstep;    // balanced kernel: groups of num_kv_heads workgroups share one token range (grid % heads == 0)
  float scale_log2;  // softmax scale x log2(e) (x k_scale for an fp8 cache)
  float v_scale;     // multiplies the output (fp8 cache's v_scale; 1 otherwise)
};


// Word 3 of a gfx9-family buffer resource for raw (untyped) loads.
constexpr int kRsrcWord3 = 0x00020000;

// Raw buffer loads of 8 / 4 consecutive 16-bit elements at byte offset `off`
// of the resource; the resource's num_records bounds the access (0 = none).
template <int ALIGN, int A = DK_ATTN_LOAD_AUX>
__device__ __forceinline__ u32x4 bload8(__amdgpu_buffer_rsrc_t r, int off) {
  if constexpr (ALIGN >= 16) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, A);
  } else if constexpr (ALIGN == 8) {
    const u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, A);
    const u32x2 b = __builtin_amdgcn_raw_buffer_load_b64(r, off + 8, 0, A);
    return u32x4{a[0], a[1], b[0], b[1]};
  } else {
    return u32x4{__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, A), __builtin_amdgcn_raw_buffer_load_b32(r, off + 4, 0, A),
                 __builtin_amdgcn_raw_buffer_load_b32(r, off + 8, 0, A), __builtin_amdgcn_raw_buffer_load_b32(r, off + 12, 0, A)};
  }
}

// Raw buffer load of 16 bytes at byte offset `off`, aligned to ALIGN (16 or 8).
template <int ALIGN, int A = DK_ATTN_LOAD_AUX>
__device__ __forceinline__ u32x4 bload16b(__amdgpu_buffer_rsrc_t r, int off) {
  if constexpr (ALIGN >= 16) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, A);
  } else {
    const u32x2 a = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, A);
    const u32x2 b = __builtin_amdgcn_raw_buffer_load_b64(r, off + 8, 0, A);
    return u32x4{a[0], a[1], b[0], b[1]};
  }
}

template <int ALIGN>
__device__ __forceinline__ u32x2 bload4(__amdgpu_buffer_rsrc_t r, int off) {
  constexpr int A = DK_ATTN_LOAD_AUX;
  if constexpr (ALIGN >= 8) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, A);
  } else {
    return u32x2{__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, A), __builtin_amdgcn_raw_buffer_load_b32(r, off + 4, 0, A)};
  }
}

// One 16-token tile in registers: lane l holds 8 consecutive elements
// (columns 8*(l/16) + 32*c ...) of K row l%16 and of V row l%16, for every
// 32-column chunk c -- the A-operand layout of v_mfma_f32_16x16x32.
template <int CHUNKS, bool KV8>
struct TileRegs {
  u32x4 k[CHUNKS];
  u32x4 v[CHUNKS];
};

// An fp8 (e4m3fn) cache tile. K: lane l holds 16 contiguous bytes of row
// l % 16 per 64 columns (columns 64 j + 16 (l / 16) ...), one 16-byte load
// each -- 64 bytes of every row per load, as the 16-bit tiles. The columns of
// MFMA chunk c are then 64 (c / 2) + 16 (l / 16) + 8 (c % 2) ...; the query
// fragments use the same columns, so Q.K^T is unchanged. V goes through the
// wave's LDS tile for the transpose reads, so its loads need no MFMA layout:
// load j holds bytes [1024 j + 16 l, +16) of the tile's rows laid end to end,
// whole lines of consecutive rows (tiles inside one cache block; tiles across
// blocks load V like K).
template <int CHUNKS>
struct TileRegs<CHUNKS, true> {
  u32x4 k[CHUNKS / 2];
  u32x4 v[CHUNKS / 2];
};

// 16 bytes at an 8-byte-aligned address (fp8 rows are 8-byte aligned).
__device__ __forceinline__ u32x4 load16_8b(const uint8_t* p) {
  const u32x2 a = reinterpret_cast<const u32x2*>(p)[0];
  const u32x2 b = reinterpret_cast<const u32x2*>(p)[1];
  return u32x4{a[0], a[1], b[0], b[1]};
}

// 8 e4m3fn bytes -> 8 elements of E, exactly (every e4m3fn value is a bf16
// and an fp16 value); v_cvt_pk_f32_fp8 matches torch.float8_e4m3fn on all
// 256 encodings (checked on the device).
template <typename E>
__device__ __forceinline__ u32x4 fp8x8_to(u32x2 w) {
  const auto a = __builtin_amdgcn_cvt_pk_f32_fp8(w[0], false);
  const auto b = __builtin_amdgcn_cvt_pk_f32_fp8(w[0], true);
  const auto c = __builtin_amdgcn_cvt_pk_f32_fp8(w[1], false);
  const auto d = __builtin_amdgcn_cvt_pk_f32_fp8(w[1], true);
  return u32x4{pack2<E>(a[0], a[1]), pack2<E>(b[0], b[1]), pack2<E>(c[0], c[1]), pack2<E>(d[0], d[1])};
}

// Log2-units headroom of the lazy running max: exponentials are taken
// against a reference max that only moves when a tile exceeds it by more
// than this, so accumulators are rescaled rarely (weights stay <= 2^8).
constexpr float kLazyMax = 8.0f;

// Waves per SIMD the register allocation targets: head_dim 64 fits four and
// head_dim 128 three without spilling; head_dim 256 keeps its natural
// allocation (one wave, no spills).
template <int D, bool KV8 = false>
constexpr int attn_occupancy() {
  // Classes: D <= 64, 64 < D <= 128 (96, 128), D > 128 (192, 256).
  if constexpr (KV8) return D > 128 ? DK_ATTN_OCC_FP8_D256 : (D > 64 ? DK_ATTN_OCC_FP8_D128 : DK_ATTN_OCC_D64);
  return D > 128 ? DK_ATTN_OCC_D256 : (D > 64 ? DK_ATTN_OCC_D128 : DK_ATTN_OCC_D64);
}

// LDS of one work unit: per-wave softmax state and partial outputs, merged at the end.
// Row pitch (16-bit elements) of a wave's V tile in LDS: 32 bytes of padding
// put the 16 rows' 8-byte transpose reads of one 16-lane group on distinct
// banks (rows start 8 banks apart).
template <int D>
constexpr int vt_pitch() {
  return D + 16;
}

// Row-contiguous tile loads (whole 128-byte lines per load instruction, K
// brought into the MFMA layout through LDS) apply when a 16-token tile lies
// inside one cache block.
template <bool BS16, bool KV8>
constexpr bool row_load() {
  return DK_ATTN_ROWLOAD && BS16 && !KV8;
}

template <int D, int NW, bool ROW = false>
struct UnitSmem {
  float m[NW][16];  // reference max per head (log2 units)
  float t[NW][16];  // true max per head
  float l[NW][16];  // exp-sum against the reference max
  // A wave's current tiles (model dtype), 16-byte aligned rows.
  struct __attribute__((aligned(16))) Tiles {
    uint16_t vt[DK_ATTN_VTR ? 16 * vt_pitch<D>() : 1];  // V tile
    uint16_t kt[ROW ? 16 * vt_pitch<D>() : 1];          // K tile (row loads)
  };
  // At head_dim 64 a wave's partial outputs of a merge pass share its region
  // with its tiles, which keeps four workgroups per CU: a wave writes its
  // outputs only after its last tile's LDS reads were issued (LDS operations
  // of one wave complete in order) and the merge ends with a barrier before
  // any wave writes tiles again. Larger head dims keep them apart (two
  // workgroups per CU either way).
  struct __attribute__((aligned(16))) Shared {
    union {
      float o[kMergeHeads][D];
      Tiles tile;
    };
  };
  struct __attribute__((aligned(16))) Separate {
    float o[kMergeHeads][D];
    Tiles tile;
  };
  typename std::conditional<(D <= 64), Shared, Separate>::type w[NW];
};
static_assert(sizeof(UnitSmem<96, 4, false>::Tiles) % 16 == 0 && sizeof(UnitSmem<64, 4, true>::Shared) % 16 == 0,
              "tile rows must stay 16-byte aligned in every wave's region");

// A work unit: tokens [start, end) of sequence `seq` (end > start, at most
// 1024 tokens) for KV head `kv_head` and its query-head group. Split-K writes
// its result to workspace slot `slot`; a unit of more than 512 tokens marks
// slot + 1 empty (max logit -inf, exp-sum 0), so the reduce walks 512-token
// slots exactly as the reference's partitions.
struct Unit {
  int kv_head, seq, start, end, slot;
  bool two_slots;
};

__device__ __forceinline__ Unit make_unit(int kv_head, int seq, int start, int unit_tokens, int seq_len, int slot) {
  return Unit{kv_head, seq, start, min(start + unit_tokens, seq_len), slot, unit_tokens > kPart};
}

// Barrier for data exchanged through LDS only: global loads issued before it
// stay in flight (a full __syncthreads fence would wait for them).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Runs work units on NW waves: wave w takes tiles w, w + NW, ... of a unit,
// keeps DEPTH tiles of loads in flight and its own online-softmax state; the
// waves merge through LDS. The steps are separate so that the balanced
// kernel can issue the next unit's loads before merging the current one.
template <typename E, int D, bool SPLIT, bool BS16, int ALIGN, int NW, bool KV8>
struct UnitEngine {
  static constexpr int CH = D / 32;  // 32-column chunks per row
  static constexpr int NB = D / 16;  // 16-column output blocks
  static constexpr int DEPTH = KV8 ? DK_ATTN_DEPTH_FP8 : (D > 128 ? DK_ATTN_DEPTH_D256 : DK_ATTN_DEPTH);
  static constexpr int NT = NW * kWave;
  static constexpr bool ROW = row_load<BS16, KV8>();
  static constexpr int RB = KV8 ? D : 2 * D;     // bytes of one K (or V) row
  static constexpr int NI = 16 * RB / 1024;      // row-contiguous 1 KB loads per K (or V) tile
  static_assert(!ROW || DK_ATTN_VTR, "row loads bring V into LDS for the transpose read");
  using Tile = TileRegs<CH, KV8>;

  const KParams& p;
  UnitSmem<D, NW, ROW>& sm;
  int tid, lane, wave, l16, lg;
  u32x4 eye0, eye1;  // identity fragments (see process)
  u32x4 qf[CH];      // query fragments of the current unit
  Tile buf[DEPTH];   // tiles in flight
  f32x4 acc[NB];
  float m_ref;   // reference max (log2 units) of head l16
  float m_true;  // exact running max of head l16
  float l_run;   // this lane's share of the exp-sum against m_ref

  __device__ __forceinline__ UnitEngine(const KParams& params, UnitSmem<D, NW, ROW>& smem) : p(params), sm(smem) {
    tid = threadIdx.x;
    lane = tid % kWave;
    wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    l16 = lane % 16;  // K/V row of the tile, head of the logits, output column
    lg = lane / 16;   // lane group 0..3
    // Identity fragments (B operand of a 16x16x32 MFMA): with them, an MFMA
    // whose A operand is a V chunk returns V transposed into the B-operand
    // layout of v_mfma_f32_16x16x16 -- lane l: V[token 4*lg + r][column l16 (+16)].
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int k0 = 8 * lg + 2 * e;
      eye0[e] = (k0 == l16 ? E::kOne : 0u) | ((k0 + 1 == l16 ? E::kOne : 0u) << 16);
      eye1[e] = (k0 == l16 + 16 ? E::kOne : 0u) | ((k0 + 1 == l16 + 16 ? E::kOne : 0u) << 16);
    }
    reset();
  }

  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int n = 0; n < NB; ++n) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
    m_ref = -__builtin_huge_valf();
    m_true = -__builtin_huge_valf();
    l_run = 0.0f;
  }

  __device__ __forceinline__ int n_tiles(const Unit& u) const { return (u.end - u.start + kTile - 1) / kTile; }

  // Block-table entries of a unit (lane e holds entry start / block_size + e)
  // when every 16-token tile lies inside one cache block.
  __device__ __forceinline__ int load_bt(const Unit& u) const {
    int v = 0;
    if constexpr (BS16) {
      const int lb0 = u.start / p.block_size;
      const int lb_last = (u.end - 1) / p.block_size;
      if (lb0 + lane <= lb_last) v = p.block_tables[static_cast<int64_t>(u.seq) * p.bt_stride + lb0 + lane];
    }
    return v;
  }

  // Query fragments (B operand of Q·Kᵀ): head l16, columns 8*lg + 32*c ... +7,
  // in the model dtype; heads past the group are zero.
  // First column of this lane's 8 columns of MFMA chunk c.
  __device__ __forceinline__ int chunk_col(int c) const {
    return KV8 && !ROW ? 64 * (c / 2) + 16 * lg + 8 * (c % 2) : 32 * c + 8 * lg;
  }

  __device__ __forceinline__ void load_q(const Unit& u) { load_q(u, p.q_ss, p.q_sh); }
  __device__ __forceinline__ void load_q(const Unit& u, int32_t q_ss, int32_t q_sh) {
    const uint16_t* qrow =
        p.q + static_cast<int64_t>(u.seq) * q_ss + static_cast<int64_t>(u.kv_head * p.group + l16) * q_sh;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (l16 < p.group) {
        const uint16_t* src = qrow + chunk_col(c);
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = static_cast<uint32_t>(src[2 * e]) | (static_cast<uint32_t>(src[2 * e + 1]) << 16);
      }
      qf[c] = w;
    }
  }

  // Issues the loads of one tile. Tiles past the end are still "loaded" so
  // every wave runs the same load sequence (the compiler then waits for
  // exactly the oldest tile): with whole-tile blocks their buffer resource
  // has num_records = 0 and nothing is read; otherwise the last tile is
  // re-read (an L2 hit). Rows past the sequence end are clamped to its last
  // row, so V never contributes uninitialised cache contents.
  __device__ __forceinline__ void load_tile(const Unit& u, int bt_lane, int tile, Tile& r) const {
    const int nt = n_tiles(u);
    const bool live = tile < nt;
    const int tt = live ? tile : nt - 1;
    const int t0 = u.start + tt * kTile;
    const int row = min(l16, u.end - 1 - t0);
    // Element pointers of the K / V cache (bytes for fp8, 16-bit otherwise).
    using KvT = typename std::conditional<KV8, uint8_t, uint16_t>::type;
    constexpr int kElt = sizeof(KvT);
    const KvT* kbase = reinterpret_cast<const KvT*>(p.k) + static_cast<int64_t>(u.kv_head) * p.k_sh;
    const KvT* vbase = reinterpret_cast<const KvT*>(p.v) + static_cast<int64_t>(u.kv_head) * p.v_sh;
    if constexpr (BS16) {
      const int lb = t0 / p.block_size;
      const int phys = __builtin_amdgcn_readlane(bt_lane, lb - u.start / p.block_size);
      const int off = t0 - lb * p.block_size;
      const KvT* kt = kbase + static_cast<int64_t>(phys) * p.k_sb + static_cast<int64_t>(off) * p.k_st;
      const KvT* vt = vbase + static_cast<int64_t>(phys) * p.v_sb + static_cast<int64_t>(off) * p.v_st;
      const int nrec = live ? 0x7fffffff : 0;
      const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<KvT*>(kt), 0, nrec, kRsrcWord3);
      const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<KvT*>(vt), 0, nrec, kRsrcWord3);
      if constexpr (ROW) {
        // Load j covers bytes [1024 j, 1024 j + 1024) of the tile's rows laid
        // end to end: lane l reads 16 bytes of row (1024 j + 16 l) / RB, so
        // every instruction reads whole lines of consecutive rows. Rows past
        // the sequence end re-read its last row.
        const int last = u.end - 1 - t0;
        const int kst = kElt * p.k_st;  // 16 rows of either fit 2^31 bytes (host)
        const int vst = kElt * p.v_st;
#pragma unroll
        for (int j = 0; j < NI; ++j) {
          const int o = 1024 * j + 16 * lane;
          const int rr = min(o / RB, last);
          if constexpr (KV8) r.k[j] = bload16b<ALIGN, DK_ATTN_ROW_AUX>(rk, rr * kst + o % RB);
          else r.k[j] = bload8<ALIGN, DK_ATTN_ROW_AUX>(rk, rr * kst + o % RB);
        }
#pragma unroll
        for (int j = 0; j < NI; ++j) {
          const int o = 1024 * j + 16 * lane;
          const int rr = min(o / RB, last);
          if constexpr (KV8) r.v[j] = bload16b<ALIGN, DK_ATTN_ROW_AUX>(rv, rr * vst + o % RB);
          else r.v[j] = bload8<ALIGN, DK_ATTN_ROW_AUX>(rv, rr * vst + o % RB);
        }
      } else if constexpr (KV8) {
        const int koff = row * p.k_st + 16 * lg;
#pragma unroll
        for (int j = 0; j < CH / 2; ++j) r.k[j] = bload16b<ALIGN, DK_ATTN_FP8_K_AUX>(rk, koff + 64 * j);
        // V row-contiguous; rows past the sequence end re-read its last row.
        const int last = u.end - 1 - t0;
        const int vst = p.v_st;
#pragma unroll
        for (int j = 0; j < CH / 2; ++j) {
          const int o = 1024 * j + 16 * lane;
          r.v[j] = bload16b<ALIGN, DK_ATTN_ROW_AUX>(rv, min(o / RB, last) * vst + o % RB);
        }
      } else {
        const int koff = kElt * (row * p.k_st + 8 * lg);
        const int voff = kElt * (row * p.v_st + 8 * lg);
#pragma unroll
        for (int c = 0; c < CH; ++c) r.k[c] = bload8<ALIGN>(rk, koff + 64 * c);
#pragma unroll
        for (int c = 0; c < CH; ++c) r.v[c] = bload8<ALIGN>(rv, voff + 64 * c);
      }
    } else {
      const int t = t0 + row;
      const int lb = t / p.block_size;
      const int64_t phys = p.block_tables[static_cast<int64_t>(u.seq) * p.bt_stride + lb];
      const int64_t off = t - lb * p.block_size;
      if constexpr (KV8) {
        const KvT* kp = kbase + phys * p.k_sb + off * p.k_st + 16 * lg;
        const KvT* vp = vbase + phys * p.v_sb + off * p.v_st + 16 * lg;
#pragma unroll
        for (int j = 0; j < CH / 2; ++j) r.k[j] = load16_8b(kp + 64 * j);
#pragma unroll
        for (int j = 0; j < CH / 2; ++j) r.v[j] = load16_8b(vp + 64 * j);
      } else {
        const KvT* kp = kbase + phys * p.k_sb + off * p.k_st + 8 * lg;
        const KvT* vp = vbase + phys * p.v_sb + off * p.v_st + 8 * lg;
#pragma unroll
        for (int c = 0; c < CH; ++c) r.k[c] = load8<ALIGN>(kp + 32 * c);
#pragma unroll
        for (int c = 0; c < CH; ++c) r.v[c] = load8<ALIGN>(vp + 32 * c);
      }
    }
  }

  // K chunk c of a tile as an MFMA operand in the model dtype.
  __device__ __forceinline__ static u32x4 k_operand(const Tile& r, int c) {
    if constexpr (KV8) {
      const u32x4 w = r.k[c / 2];
      return c % 2 == 0 ? fp8x8_to<E>(u32x2{w[0], w[1]}) : fp8x8_to<E>(u32x2{w[2], w[3]});
    } else {
      return r.k[c];
    }
  }

  // The first DEPTH tiles of this wave. The scheduling barriers keep the
  // tiles' load groups in program order, so the oldest outstanding loads are
  // always those of the next tile consumed.
  __device__ __forceinline__ void prologue(const Unit& u, int bt_lane) {
#pragma unroll
    for (int i = 0; i < DEPTH; ++i) {
      load_tile(u, bt_lane, wave + i * NW, buf[i]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Online softmax + P·V for one live tile held in `r`.
  __device__ __forceinline__ void process(const Unit& u, int tile, const Tile& r) {
    // Q·Kᵀ: S[token 4*lg + i][head l16].
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    if constexpr (ROW) {
      // Both row-contiguous tiles go to this wave's LDS tiles at their
      // [row][column] places (fp8 converted to the model dtype); K comes back
      // in the A-operand layout of v_mfma_f32_16x16x32 (row l16, columns
      // 8 lg + 32 c ...), V through the transpose reads below.
      uint16_t* kt = sm.w[wave].tile.kt;
      uint16_t* vt = sm.w[wave].tile.vt;
#pragma unroll
      for (int j = 0; j < NI; ++j) {
        const int o = 1024 * j + 16 * lane;
        const int at = (o / RB) * vt_pitch<D>() + (KV8 ? o % RB : (o % RB) / 2);
        if constexpr (KV8) {
          *reinterpret_cast<u32x4*>(kt + at) = fp8x8_to<E>(u32x2{r.k[j][0], r.k[j][1]});
          *reinterpret_cast<u32x4*>(kt + at + 8) = fp8x8_to<E>(u32x2{r.k[j][2], r.k[j][3]});
          *reinterpret_cast<u32x4*>(vt + at) = fp8x8_to<E>(u32x2{r.v[j][0], r.v[j][1]});
          *reinterpret_cast<u32x4*>(vt + at + 8) = fp8x8_to<E>(u32x2{r.v[j][2], r.v[j][3]});
        } else {
          *reinterpret_cast<u32x4*>(kt + at) = r.k[j];
          *reinterpret_cast<u32x4*>(vt + at) = r.v[j];
        }
      }
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        const u32x4 ka = *reinterpret_cast<const u32x4*>(kt + l16 * vt_pitch<D>() + 8 * lg + 32 * c);
        s = E::mfma_16x16x32(ka, qf[c], s);
      }
    } else {
#pragma unroll
      for (int c = 0; c < CH; ++c) s = E::mfma_16x16x32(k_operand(r, c), qf[c], s);
    }

    const int t0 = u.start + tile * kTile;
    float x[4];
    float tmax = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool valid = t0 + 4 * lg + i < u.end;
      x[i] = valid ? s[i] * p.scale_log2 : -__builtin_huge_valf();
      tmax = fmaxf(tmax, x[i]);
    }
    tmax = rows_max(tmax);  // over the tile's 16 tokens
    m_true = fmaxf(m_true, tmax);
    if (__any(tmax > m_ref + kLazyMax)) {
      const float m_new = fmaxf(m_ref, tmax);
      const float alpha = __builtin_amdgcn_exp2f(m_ref - m_new);
      m_ref = m_new;
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = __shfl(alpha, 4 * lg + i, kWave);
#pragma unroll
        for (int n = 0; n < NB; ++n) acc[n][i] *= a;
      }
    }
    float pr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pr[i] = __builtin_amdgcn_exp2f(x[i] - m_ref);
      l_run += pr[i];
    }
    // P = P_hi + P_lo in the model dtype: two 16x16x16 MFMAs per block keep
    // the products accurate to ~2^-17 relative (fp32-like).
    const u32x2 p_hi = {pack2<E>(pr[0], pr[1]), pack2<E>(pr[2], pr[3])};
    const u32x2 p_lo = {pack2<E>(pr[0] - E::lo(p_hi[0]), pr[1] - E::hi(p_hi[0])),
                        pack2<E>(pr[2] - E::lo(p_hi[1]), pr[3] - E::hi(p_hi[1]))};
#if DK_ATTN_VTR
    // V through this wave's LDS tile: lane l writes its row (token l16,
    // columns 8 lg + 32 c ...) and reads back, with ds_read_b64_tr_b16, the
    // B operand of v_mfma_f32_16x16x16 for 16-column block nb -- V[token
    // 4 lg + e][column 16 nb + l16], e = 0..3. The transpose read hands lane
    // j of a 16-lane group element j % 4 of group lane 4 k + (j % 16) / 4 as
    // its element k (measured on the device), so group lane s reads the four
    // columns 16 nb + 4 (s % 4) ... of token 4 lg + (s % 16) / 4.
    uint16_t* vt = sm.w[wave].tile.vt;
    if constexpr (ROW) {
      // written above with K
    } else if constexpr (KV8) {
      // Whole-block tiles load V row-contiguous (lane l of load j holds row
      // (1024 j + 16 l) / RB); tiles across blocks load it in the K layout.
#pragma unroll
      for (int j = 0; j < CH / 2; ++j) {
        const u32x4 w = r.v[j];
        const int o = 1024 * j + 16 * lane;
        uint16_t* dst = BS16 ? vt + (o / RB) * vt_pitch<D>() + o % RB : vt + l16 * vt_pitch<D>() + 64 * j + 16 * lg;
        *reinterpret_cast<u32x4*>(dst) = fp8x8_to<E>(u32x2{w[0], w[1]});
        *reinterpret_cast<u32x4*>(dst + 8) = fp8x8_to<E>(u32x2{w[2], w[3]});
      }
    } else {
#pragma unroll
      for (int c = 0; c < CH; ++c) *reinterpret_cast<u32x4*>(vt + l16 * vt_pitch<D>() + 8 * lg + 32 * c) = r.v[c];
    }
    const int tr_row = 4 * lg + l16 / 4;
    const int tr_col = 4 * (l16 % 4);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      using lds_v4i16 = __attribute__((address_space(3))) s16x4;
      // (a C-style cast is the generic -> LDS address-space conversion)
      const auto src = (lds_v4i16*)(vt + tr_row * vt_pitch<D>() + 16 * nb + tr_col);
      const u32x2 vb = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(src));
      acc[nb] = E::mfma_16x16x16(p_hi, vb, acc[nb]);
      acc[nb] = E::mfma_16x16x16(p_lo, vb, acc[nb]);
    }
#else
    static_assert(!KV8, "the fp8 cache path reads V through the LDS transpose");
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
      const u32x4 vc = r.v[c];
      const f32x4 t_lo = E::mfma_16x16x32(vc, eye0, z);  // columns 32c + l16
      const f32x4 t_hi = E::mfma_16x16x32(vc, eye1, z);  // columns 32c + 16 + l16
      const u32x2 v_lo = {pack2<E>(t_lo[0], t_lo[1]), pack2<E>(t_lo[2], t_lo[3])};
      const u32x2 v_hi = {pack2<E>(t_hi[0], t_hi[1]), pack2<E>(t_hi[2], t_hi[3])};
      acc[2 * c] = E::mfma_16x16x16(p_hi, v_lo, acc[2 * c]);
      acc[2 * c] = E::mfma_16x16x16(p_lo, v_lo, acc[2 * c]);
      acc[2 * c + 1] = E::mfma_16x16x16(p_hi, v_hi, acc[2 * c + 1]);
      acc[2 * c + 1] = E::mfma_16x16x16(p_lo, v_hi, acc[2 * c + 1]);
    }
#endif
  }

  // Steady state: consume the oldest tile, refill its registers DEPTH tiles
  // ahead. Loads are issued on every path, so the wait before each tile is
  // for exactly that tile's loads.
  __device__ __forceinline__ void run_tiles(const Unit& u, int bt_lane) {
    const int nt = n_tiles(u);
    for (int base = wave; base < nt; base += DEPTH * NW) {
#pragma unroll
      for (int i = 0; i < DEPTH; ++i) {
        const int t = base + i * NW;
        if (t < nt) process(u, t, buf[i]);
        load_tile(u, bt_lane, t + DEPTH * NW, buf[i]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  // Merges the waves' states through LDS and writes the unit's result; ends
  // with a barrier, after which the LDS may be reused.
  __device__ __forceinline__ void merge(const Unit& u) {
    // The outputs below overwrite this wave's tile region. The hardware runs a
    // wave's LDS operations in order, but the compiler sees float stores and
    // 16-bit tile reads of other types and could move them past each other:
    // keep program order here.
    __asm__ volatile("" ::: "memory");
    const int group = p.group;
    // Exp-sum of head l16 over all four lane groups.
    const float l_tot = rows_sum(l_run);
    // The lane test is made here, per merge: hoisted out of the balanced
    // kernel's piece loop, its 64-bit mask (like the one below) stayed live in
    // scalar registers for the whole loop and was spilled.
    if (fresh_vgpr(lane) < 16) {
      sm.m[wave][lane] = m_ref;
      sm.t[wave][lane] = m_true;
      sm.l[wave][lane] = l_tot;
    }
    // Heads in passes of kMergeHeads (one pass up to 8, two up to 16); the
    // group has at least one head (host), so the first pass needs no test.
    int h0 = 0;
    do {
      const int hn = min(kMergeHeads, group - h0);
      // acc[n] lane l: O[head 4*lg + i][column 16n + l16].
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int h = 4 * lg + i - h0;
        if (h >= 0 && h < hn) {
#pragma unroll
          for (int n = 0; n < NB; ++n) sm.w[wave].o[h][16 * n + l16] = acc[n][i];
        }
      }
      lds_barrier();
      merge_pass(u, h0, hn);
      lds_barrier();
      h0 += kMergeHeads;
    } while (h0 < group);
  }

  // Combines the waves' partial outputs of heads h0 .. h0 + hn - 1 (in LDS)
  // and writes them.
  __device__ __forceinline__ void merge_pass(const Unit& u, int h0, int hn) {
    const int group = p.group;
    for (int idx = tid; idx < hn * D; idx += NT) {
      const int hh = idx / D;
      const int d = idx - hh * D;
      const int h = h0 + hh;
      float M = sm.m[0][h];
#pragma unroll
      for (int w = 1; w < NW; ++w) M = fmaxf(M, sm.m[w][h]);
      float L = 0.0f;
      float O = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float f = __builtin_amdgcn_exp2f(sm.m[w][h] - M);
        L += f * sm.l[w][h];
        O += f * sm.w[w].o[hh][d];
      }
      const float res = O / L * p.v_scale;
      const int q_head = u.kv_head * group + h;
      if constexpr (SPLIT) {
        const int64_t row = (static_cast<int64_t>(u.seq) * p.num_q_heads + q_head) * p.max_partitions + u.slot;
        p.tmp_out[row * D + d] = res;
        if (d == 0) {
          // Report (max logit, exp-sum) against the unit's true max.
          float T = sm.t[0][h];
#pragma unroll
          for (int w = 1; w < NW; ++w) T = fmaxf(T, sm.t[w][h]);
          p.max_logits[row] = T * kLn2;
          p.exp_sums[row] = L * __builtin_amdgcn_exp2f(M - T);
          if (u.two_slots && u.slot + 1 < p.max_partitions) {
            p.max_logits[row + 1] = -__builtin_huge_valf();
            p.exp_sums[row + 1] = 0.0f;
          }
        }
      } else {
        p.out[static_cast<int64_t>(u.seq) * p.o_ss + static_cast<int64_t>(q_head) * p.o_sh + d] = E::from_float(res);
      }
    }
  }
};

// Grid kernel: one workgroup per work unit. The units at one token position
// form a plane of num_seqs x num_kv_heads. Split-K planes run from the last
// 1024-token position down; the first 1024 tokens of every sequence come last
// as two planes of 512-token units, so the units still running when the grid
// drains are short. Plane k is rotated by k positions: workgroup i runs on XCD
// i mod 8, and without the rotation every unit of a (sequence, KV head) would
// land on one XCD, where a few long sequences would keep it busy long after
// the others are idle.
template <typename E, int D, bool SPLIT, bool BS16, int ALIGN, int NW, bool KV8>
__global__ __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(attn_occupancy<D, KV8>(),
                                                                            attn_occupancy<D, KV8>())))
void paged_attention_kernel(const KParams p) {
  __shared__ UnitSmem<D, NW, row_load<BS16, KV8>()> sm;
  const int per_plane = p.num_seqs * p.num_kv_heads;
  const int plane = static_cast<int>(blockIdx.x) / per_plane;
  const int rot = static_cast<int>(blockIdx.x) - plane * per_plane;
  const int unit = (rot + per_plane - plane % per_plane) % per_plane;
  const int seq = unit / p.num_kv_heads;
  const int kv_head = unit - seq * p.num_kv_heads;
  int start = 0;
  int unit_tokens = kPart;
  int seq_len = p.seq_lens[seq];
  if constexpr (SPLIT) {
    if (p.unit512) {
      start = (p.max_partitions - 1 - plane) * kPart;  // planes walk the 512-token positions from the last down
    } else {
      const int full_planes = p.num_units - 1;  // positions 1 .. num_units - 1, 1024 tokens each
      if (plane < full_planes) {
        start = (full_planes - plane) * kUnit;
        unit_tokens = kUnit;
      } else {
        start = plane == full_planes ? kPart : 0;
      }
    }
    seq_len = min(seq_len, p.max_partitions * kPart);  // tokens past the workspace are ignored
  }
  if (start >= seq_len) {
    if (!SPLIT) {
      for (int idx = threadIdx.x; idx < p.group * D; idx += NW * kWave) {
        const int h = idx / D;
        const int d = idx - h * D;
        p.out[static_cast<int64_t>(seq) * p.o_ss + static_cast<int64_t>(kv_head * p.group + h) * p.o_sh + d] = 0;
      }
    }
    return;
  }
  UnitEngine<E, D, SPLIT, BS16, ALIGN, NW, KV8> eng(p, sm);
  Unit u = make_unit(kv_head, seq, start, unit_tokens, seq_len, start / kPart);
  // 512-token units: rows 0 .. n-1 hold the sequence's partitions and the
  // last one marks row n empty (if n < max_partitions) -- the layout the
  // balanced schedule's reduce reads. (two_slots: "mark the next row empty".)
  if (SPLIT && p.unit512) u.two_slots = start + kPart >= seq_len;
  const int bt = eng.load_bt(u);
  eng.load_q(u);
  eng.prologue(u, bt);
  eng.run_tiles(u, bt);
  eng.merge(u);
}

// Balanced split-K kernel: a resident-sized grid in which every workgroup
// gets an equal share of the work, known up front.
//
// Per-workgroup bandwidth is latency-bound (each workgroup moves ~1/500 of
// the chip's bandwidth), so a 1024-token unit takes tens of microseconds and a
// grid of whole units ends with a long tail of the last ones. Here the
// (sequence, KV head) streams are laid end to end (sequences in order, KV
// heads innermost) on a line where each stream costs its 16-token tiles plus
// a fixed overhead (its query load and partial-result merge, counted as
// kStreamCost tiles), and workgroup w takes cost range [w s, w s + s),
// s = max(64, ceil(total / grid)). Since a workgroup knows its whole list, the
// next piece's block-table entries, query and first tiles load while the
// current one finishes: no piece start waits on a round trip, no atomics.
//
// Lockstep variant (16-bit caches): the line holds sequences only, each
// costing its tiles plus the overhead once, and its shares go to groups of
// num_kv_heads consecutive workgroups; workgroup h of a group runs KV head h
// of the group's share, so a sequence's KV heads read the same tokens at
// about the same time. Everything below holds with "group" for "workgroup".
//
// A piece is one stream's tiles inside a workgroup's share (run as sub-units
// of at most 64 tiles sharing one softmax state). Its partial result goes to
// workspace row (w - workgroup of the stream's first tile) of the stream's
// query heads: rows are numbered by piece, not by token position. A stream of
// n tiles meets at most ceil(n / 64) + 1 shares, which is at most
// max(2, ceil(L / 512)) <= max_partitions rows; the workgroup holding a
// stream's last tile marks the row after its piece empty (exp-sum 0), and the
// reduce reads rows up to the first empty one.
constexpr int kMaxBalancedSeqs = 2048;
constexpr int kMinShareTiles = 64;
#ifndef DK_ATTN_STREAM_COST
#define DK_ATTN_STREAM_COST 8  // per-stream overhead, in tiles, of the share balance
#endif
#ifndef DK_ATTN_STREAM_COST_FP8
#define DK_ATTN_STREAM_COST_FP8 12  // the same with an fp8 cache (its tiles take about half the time)
#endif
template <bool KV8>
constexpr int stream_cost() {
  return KV8 ? DK_ATTN_STREAM_COST_FP8 : DK_ATTN_STREAM_COST;
}
#ifndef DK_ATTN_PAIR_RATIO
#define DK_ATTN_PAIR_RATIO 200  // with two workgroups per CU: first-half share / second-half share, x100
#endif

template <typename E, int D, bool BS16, int ALIGN, int NW, bool KV8>
__global__ __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(attn_occupancy<D, KV8>(),
                                                                            attn_occupancy<D, KV8>())))
void paged_attention_balanced_kernel(const KParams p) {
  constexpr int NT = NW * kWave;
  __shared__ UnitSmem<D, NW, row_load<BS16, KV8>()> sm;
  __shared__ int pre[kMaxBalancedSeqs + 1];  // cost per KV head of sequences 0 .. s-1
  __shared__ int len[kMaxBalancedSeqs];      // lengths, clamped to the workspace
  // The query strides, read from here once per stream: kept in scalar
  // registers across the piece loop, they were what spilled at head_dim 96.
  __shared__ int32_t q_str[2];
  // The stream walk's KV-head step: [0] heads per sequence on the line (hl
  // below), [1] this workgroup's first KV head (kv0). Read from LDS in the
  // walk for the same reason (two more scalar registers spilled at head_dim 96).
  __shared__ int32_t walk[2];
  // Wave totals of the set-up scan, in wave 0's region (no tile is processed before the set-up's last barrier).
  static_assert(sizeof(sm.w[0]) >= NW * sizeof(int), "scan space");
  int* scan = reinterpret_cast<int*>(&sm.w[0]);
  const int tid = threadIdx.x;
  const int S = p.num_seqs;
  const int P = p.max_partitions;
  const int max_tokens = P * kPart;  // tokens past the workspace are ignored
  auto tiles_of = [&](int s) { return (len[s] + kTile - 1) / kTile; };
  constexpr int kStreamCost = stream_cost<KV8>();
  auto cost_of_len = [](int l) { return l > 0 ? (l + kTile - 1) / kTile + kStreamCost : 0; };

  // Per-thread chunk of sequences -> workgroup-wide inclusive scan of stream costs.
  const int per = (S + NT - 1) / NT;
  const int s0 = min(tid * per, S);
  const int s1 = min(s0 + per, S);
  int cnt = 0;
  for (int s = s0; s < s1; ++s) {
    const int l = min(max(p.seq_lens[s], 0), max_tokens);
    len[s] = l;
    cnt += cost_of_len(l);
  }
  // Inclusive scan: within each wave by shuffles, then the wave totals
  // through LDS (two barriers instead of two per doubling step).
  const int lane = tid % kWave;
  const int wv = tid / kWave;
  int incl = cnt;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(incl, off, kWave);
    if (lane >= off) incl += y;
  }
  if (lane == kWave - 1) scan[wv] = incl;
  __syncthreads();
  for (int w = 0; w < wv; ++w) incl += scan[w];
  int run = incl - cnt;
  for (int s = s0; s < s1; ++s) {
    pre[s] = run;
    run += cost_of_len(len[s]);
  }
  if (tid == NT - 1) pre[S] = incl;
  if (tid == 0) {
    q_str[0] = p.q_ss;
    q_str[1] = p.q_sh;
    walk[0] = p.lockstep ? 1 : p.num_kv_heads;
    walk[1] = p.lockstep ? static_cast<int>(blockIdx.x) % p.num_kv_heads : 0;
  }
  __syncthreads();

  const int hkv = p.num_kv_heads;
  // Lockstep: the line holds sequences only (one position per tile of every
  // KV head at once) and its shares go to groups of hkv consecutive
  // workgroups, workgroup kv0 of a group taking KV head kv0 of the group's
  // share. Otherwise every workgroup is a group of one and the line holds
  // the (sequence, KV head) streams. The host sets lockstep only when hkv
  // divides the grid into at least two groups.
  const bool lock = p.lockstep != 0;
  const int R = lock ? hkv : 1;   // workgroups per group
  const int hl = lock ? 1 : hkv;  // KV heads laid on the line per sequence
  const int total = pre[S] * hl;  // < 2^31 (checked by the host)
  const int G = static_cast<int>(gridDim.x) / R;  // groups
  // Shares: groups [0, H) take share_a each, [H, G) share_b.
  const int H = G / 2;
  int share_a, share_b;
  {
    const int64_t r = p.pair_ratio;
    const int64_t denom = static_cast<int64_t>(H) * r + static_cast<int64_t>(G - H) * 100;
    share_b = static_cast<int>((static_cast<int64_t>(total) * 100 + denom - 1) / denom);
    if (share_b >= kMinShareTiles) {
      share_a = max(kMinShareTiles, static_cast<int>((static_cast<int64_t>(share_b) * r + 99) / 100));
    } else {
      // Too little work for the full ratio above the minimum share: the second
      // half keeps the minimum and the first half takes the rest, so the
      // ratio shrinks towards 1. (Raising the second half to the minimum
      // while keeping the ratio let the first half's shares swallow nearly
      // all the work and left half the grid idle: Llama b8 x 8192 tokens
      // 60.5 -> 54.4 us, b32 x 2048 60.3 -> 55.2, Qwen2.5-7B b64 65.3 -> 60.0
      // with this rule, cold.)
      share_b = kMinShareTiles;
      share_a = max(kMinShareTiles,
                    static_cast<int>((static_cast<int64_t>(total) - static_cast<int64_t>(G - H) * kMinShareTiles + H - 1) /
                                     max(H, 1)));
    }
  }
  // Share boundaries stay below 2^31: total < 2^30 + 2^17 (the host bounds
  // the tiles by 2^30) and the rounding of the shares adds at most a few
  // positions per workgroup.
  const int split_at = H * share_a;
  auto first_pos = [&](int wg) -> int { return wg < H ? wg * share_a : split_at + (wg - H) * share_b; };
  auto owner = [&](int x) -> int {  // group whose share holds cost position x
    return x < split_at ? x / share_a : H + (x - split_at) / share_b;
  };
  const int w = static_cast<int>(blockIdx.x) / R;  // group
  const int kv0 = static_cast<int>(blockIdx.x) - w * R;  // lockstep: this workgroup's KV head; else 0
  if (w >= G || first_pos(w) >= total) return;
  const int a = first_pos(w);
  const int b = min(first_pos(w + 1), total);
  auto cost_of = [&](int s) { return pre[s + 1] - pre[s]; };

  // Stream holding cost position a: the last sequence whose first position
  // is <= a (it has tiles, since pre[S] * hl > a), then the KV head.
  int seq = 0;
  {
    int lo = 0, hi = S;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (pre[mid] * hl <= a) lo = mid;
      else hi = mid;
    }
    seq = lo;
  }
  int kv = kv0 + (a - pre[seq] * hl) / cost_of(seq);
  // Row of this share's piece of that stream: the number of shares before
  // this one that hold its tiles. Every later stream starts inside this share
  // (its first tile lies at or past a), so its row is 0; the share layout
  // (and its scalar registers) is not needed past this point.
  const int first_row = [&]() {
    const int first = pre[seq] * hl + (kv - kv0) * cost_of(seq) + kStreamCost;
    return first < a ? w - owner(first) : 0;
  }();

  // Walk the streams that meet [a, b): each contributes the tiles
  // [lo, hi) of its own (local) numbering that lie inside the share.
  int u = 0, hi = 0, row = 0;
  bool last_tile_here = false;  // this share holds the stream's last tile
  auto advance = [&]() {        // to the next stream with tiles; false if none
    if (++kv < walk[1] + walk[0]) return true;
    kv = walk[1];
    for (;;) {
      if (++seq >= S) return false;
      if (cost_of(seq) > 0) return true;
    }
  };
  auto enter_stream = [&]() {  // false once the streams start past the share
    for (;;) {
      const int first = pre[seq] * walk[0] + (kv - walk[1]) * cost_of(seq) + kStreamCost;  // position of tile 0
      const int n = tiles_of(seq);
      if (first >= b) return false;
      const int lo = max(a, first) - first;
      hi = min(b, first + n) - first;
      if (lo < hi) {
        u = lo;
        row = first < a ? first_row : 0;
        last_tile_here = hi == n;
        return true;
      }
      if (!advance()) return false;  // the share covers only this stream's overhead
    }
  };
  auto next_stream = [&]() { return advance() && enter_stream(); };

  struct Sub {
    Unit unit;
    int tiles;
    bool piece_end, stream_end;
  };
  auto make_sub = [&]() {
    const int m = min(kMinShareTiles, hi - u);
    Sub r;
    r.unit = Unit{kv, seq, u * kTile, min((u + m) * kTile, len[seq]), row, false};
    r.tiles = m;
    r.piece_end = u + m == hi;
    r.stream_end = r.piece_end && last_tile_here;
    return r;
  };

  if (!enter_stream()) return;
  UnitEngine<E, D, true, BS16, ALIGN, NW, KV8> eng(p, sm);
  Sub cur = make_sub();
  int cur_bt = eng.load_bt(cur.unit);
  eng.load_q(cur.unit, q_str[0], q_str[1]);
  eng.prologue(cur.unit, cur_bt);
  for (;;) {
    u += cur.tiles;
    bool more = true;
    bool new_stream = false;
    if (cur.piece_end) {
      more = next_stream();
      new_stream = true;
    }
    Sub nxt{};
    int nxt_bt = 0;
    if (more) {
      nxt = make_sub();
      nxt_bt = eng.load_bt(nxt.unit);  // in flight while this sub-unit runs
    }
    eng.run_tiles(cur.unit, cur_bt);
    if (more) {
      if (new_stream) eng.load_q(nxt.unit, q_str[0], q_str[1]);
      eng.prologue(nxt.unit, nxt_bt);
    }
    if (cur.piece_end) {
      eng.merge(cur.unit);
      eng.reset();
      const int next_row = cur.unit.slot + 1;
      if (cur.stream_end && next_row < P && fresh_vgpr(tid) < p.group) {
        const int64_t r =
            (static_cast<int64_t>(cur.unit.seq) * p.num_q_heads + cur.unit.kv_head * p.group + tid) * P + next_row;
        p.max_logits[r] = -__builtin_huge_valf();
        p.exp_sums[r] = 0.0f;
      }
    }
    if (!more) break;
    cur = nxt;
    cur_bt = nxt_bt;
  }
}

// Log-sum-exp merge of the partial results of one (query head, sequence):
//   M = max_p m_p,  w_p = s_p * exp(m_p - M),  out = sum_p w_p o_p / sum_p w_p
// (reference: csrc/paged_attention.cuh:227-269). Two row layouts:
//   PIECES = false (grid schedule): row p = tokens [512 p, 512 p + 512);
//     results in rows 0, 1 and the even rows >= 2 (1024-token units), odd rows
//     >= 3 hold no result. Rows are walked by index so no load waits on another.
//   PIECES = true (balanced schedule): rows 0 .. n-1 hold the stream's pieces,
//     row n (if < max_partitions) is marked empty (exp-sum 0); n is found with
//     one lane-parallel pass over the exp-sums.
// WPH waves per query head, max(4, WPH) waves per workgroup. The (m_p, s_p)
// pairs are uniform across a wave and each lane accumulates D/64 output
// columns; with WPH > 1 the waves of a head take every WPH-th row and merge
// through LDS. The op is latency-bound: WPH grows with the number of rows a
// head merges (1 wave up to 8, 4 up to 63, 16 beyond; measured).
template <int WPH>
constexpr int reduce_waves() {
  return WPH > 4 ? WPH : 4;
}

template <typename E, int D, int WPH, bool PIECES>
__global__ __launch_bounds__(reduce_waves<WPH>() * kWave) void paged_attention_reduce_kernel(const KParams p) {
  constexpr int kReduceWaves = reduce_waves<WPH>();
  constexpr int C = (D + kWave - 1) / kWave;  // columns per lane (1-4); lanes past D / C idle
  constexpr int HPW = kReduceWaves / WPH;  // heads per workgroup
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
  const int q_head = blockIdx.x * HPW + wave / WPH;
  const int sub = wave % WPH;
  const int seq = blockIdx.y;
  const int lane = threadIdx.x % kWave;
  __shared__ float red[WPH > 1 ? kReduceWaves : 1][D + 1];
  const bool active = q_head < p.num_q_heads;
  const bool cols = C * lane < D;  // this lane owns output columns
  uint16_t* out = p.out + static_cast<int64_t>(seq) * p.o_ss + static_cast<int64_t>(active ? q_head : 0) * p.o_sh +
                  (cols ? C * lane : 0);
  const int64_t row0 = (static_cast<int64_t>(seq) * p.num_q_heads + (active ? q_head : 0)) * p.max_partitions;
  const float* ml = p.max_logits + row0;
  const float* es = p.exp_sums + row0;
  const float* tmp = p.tmp_out + row0 * D + (cols ? C * lane : 0);
  const int P = p.max_partitions;

  float acc[C];
#pragma unroll
  for (int c = 0; c < C; ++c) acc[c] = 0.0f;
  auto load_row = [&](int i, float (&v)[C]) {
    const float* t = tmp + static_cast<int64_t>(i) * D;
    if constexpr (C == 4) {
      const f32x4 x = *reinterpret_cast<const f32x4*>(t);
#pragma unroll
      for (int c = 0; c < 4; ++c) v[c] = x[c];
    } else {
#pragma unroll
      for (int c = 0; c < C; ++c) v[c] = cols ? t[c] : 0.0f;
    }
  };
  auto add_row = [&](float w, const float (&v)[C]) {
#pragma unroll
    for (int c = 0; c < C; ++c) acc[c] = fmaf(w, v[c], acc[c]);
  };

  float W = 0.0f;
  if constexpr (PIECES) {
    // Rows 0 .. n-1 hold the stream's pieces, row n (if < P) is marked
    // empty. Everything that does not depend on n loads at once: the length,
    // the first 64 (exp-sum, max-logit) pairs (lane j holds row j's) and the
    // first kPre rows this wave merges (rows are in the workspace whatever n
    // is; values past n are never used).
    constexpr int kPre = DK_REDUCE_PRE;
    const int seq_len = p.seq_lens[seq];
    const bool in0 = lane < P;
    const float e_l = in0 ? es[lane] : 0.0f;
    const float m_l = in0 ? ml[lane] : -__builtin_huge_valf();
    float pre[kPre][C];
#pragma unroll
    for (int r = 0; r < kPre; ++r) {
      if (sub + r * WPH < P) load_row(sub + r * WPH, pre[r]);
    }
    if (seq_len <= 0) {
      if (active && sub == 0 && cols) {
#pragma unroll
        for (int c = 0; c < C; ++c) out[c] = 0;
      }
      return;
    }
    int entries = P;
    float M = -__builtin_huge_valf();
    {
      const unsigned long long z = __ballot(e_l == 0.0f);  // lanes past P count as empty
      const int t = z != 0 ? __ffsll(static_cast<long long>(z)) - 1 : kWave;
      if (lane < t) M = m_l;
      if (z != 0) entries = t;
    }
    for (int base = kWave; entries == P && base < P; base += kWave) {  // more than 64 rows
      const int j = base + lane;
      const bool in = j < P;
      const float e = in ? es[j] : 0.0f;
      const float m = in ? ml[j] : -__builtin_huge_valf();
      const unsigned long long z = __ballot(e == 0.0f);
      const int t = z != 0 ? __ffsll(static_cast<long long>(z)) - 1 : kWave;
      if (lane < t) M = fmaxf(M, m);
      if (z != 0) entries = base + t;
    }
    M = wave_max(M);
#pragma unroll
    for (int r = 0; r < kPre; ++r) {
      const int j = sub + r * WPH;  // wave-uniform; rows < 64 come from the lanes that loaded them
      if (j < entries) {
        float e, m;
        if (j < kWave) {
          e = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, e_l), j));
          m = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, m_l), j));
        } else {
          e = es[j];
          m = ml[j];
        }
        const float w = e * __builtin_amdgcn_exp2f((m - M) * kLog2e);
        W += w;
        add_row(w, pre[r]);
      }
    }
    // The rest: plain loads (a cross-lane read in this runtime-count loop
    // would keep it from unrolling, and the unrolled loads overlap).
#pragma unroll 4
    for (int j = sub + kPre * WPH; j < entries; j += WPH) {
      const float w = es[j] * __builtin_amdgcn_exp2f((ml[j] - M) * kLog2e);
      W += w;
      float v[C];
      load_row(j, v);
      add_row(w, v);
    }
  } else {
    // Rows p = tokens [512 p, 512 p + 512): results in rows 0, 1 and the
    // even rows >= 2, walked by index.
    const int seq_len = p.seq_lens[seq];
    if (seq_len <= 0) {
      if (active && sub == 0 && cols) {
#pragma unroll
        for (int c = 0; c < C; ++c) out[c] = 0;
      }
      return;
    }
    const int n = min((seq_len + kPart - 1) / kPart, P);
    const int entries = 2 + (n - 1) / 2;  // slot 0, slot 1, then slot 2 (j - 1)
    const bool slot1 = n > 1 && es[1] != 0.0f;
    float M = -__builtin_huge_valf();
    for (int j = lane; j < entries; j += kWave) {
      if (j != 1 || slot1) M = fmaxf(M, ml[j < 2 ? j : 2 * (j - 1)]);
    }
    M = wave_max(M);
#pragma unroll 4
    for (int j = sub; j < entries; j += WPH) {
      if (j == 1 && !slot1) continue;
      const int i = j < 2 ? j : 2 * (j - 1);
      const float w = es[i] * __builtin_amdgcn_exp2f((ml[i] - M) * kLog2e);
      W += w;
      float v[C];
      load_row(i, v);
      add_row(w, v);
    }
  }
  if constexpr (WPH > 1) {
    if (cols) {
#pragma unroll
      for (int c = 0; c < C; ++c) red[wave][C * lane + c] = acc[c];
    }
    if (lane == 0) red[wave][D] = W;
    __syncthreads();
    if (sub != 0 || !active) return;
    W = 0.0f;
#pragma unroll
    for (int c = 0; c < C; ++c) acc[c] = 0.0f;
#pragma unroll
    for (int w = 0; w < WPH; ++w) {
      W += red[wave + w][D];
      if (cols) {
#pragma unroll
        for (int c = 0; c < C; ++c) acc[c] += red[wave + w][C * lane + c];
      }
    }
  }
  if (!active || !cols) return;
  const float inv = 1.0f / W;
#pragma unroll
  for (int c = 0; c < C; ++c) out[c] = E::from_float(acc[c] * inv);
}

constexpr int kMaxDevices = 64;

template <int D>
constexpr int waves_per_group() {
  return D > 128 ? DK_ATTN_WAVES_D256 : kWaves;
}

// Launches the grid kernel (BALANCED = false, one workgroup per unit slot) or
// the balanced kernel for KV pointers aligned to ALIGN bytes. With
// `resident`, only reports how many balanced-kernel workgroups fit on the
// current device at once (0 if unknown), cached per device.
template <typename E, int D, int ALIGN, bool SPLIT, bool BS16, bool BALANCED, bool KV8>
hipError_t launch_kernel(const KParams& kp, unsigned grid, hipStream_t stream, int* resident = nullptr,
                         int* per_cu_out = nullptr) {
  constexpr int NW = waves_per_group<D>();
  if constexpr (BALANCED) {
    const auto kernel = paged_attention_balanced_kernel<E, D, BS16, ALIGN, NW, KV8>;
    if (resident != nullptr) {
      static std::atomic<int> cache[kMaxDevices];
      *resident = 0;
      int dev = 0;
      if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return hipSuccess;
      // Packed (workgroups per CU) << 20 | CUs.
      int v = cache[dev].load(std::memory_order_relaxed);
      if (v <= 0) {
        int per_cu = 0;
        int cus = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kernel), NW * kWave, 0) !=
                hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            per_cu <= 0 || per_cu > 1023 || cus <= 0 || cus >= (1 << 20))
          return hipSuccess;
        v = (per_cu << 20) | cus;
        cache[dev].store(v, std::memory_order_relaxed);
      }
      *resident = (v >> 20) * (v & 0xfffff);
      if (per_cu_out != nullptr) *per_cu_out = v >> 20;
      return hipSuccess;
    }
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(NW * kWave), 0, stream, kp);
  } else {
    hipLaunchKernelGGL((paged_attention_kernel<E, D, SPLIT, BS16, ALIGN, NW, KV8>), dim3(grid), dim3(NW * kWave), 0, stream,
                       kp);
  }
  return hipGetLastError();
}

template <typename E, int D, bool SPLIT, bool BS16, bool BALANCED, bool KV8>
hipError_t launch_aligned(const KParams& kp, unsigned grid, int align, hipStream_t stream, int* resident = nullptr,
                          int* per_cu = nullptr) {
  if constexpr (KV8) {
    // fp8 rows: 16-byte loads when 16-byte aligned, else pairs of 8-byte loads
    // (8-byte alignment is checked by the host).
    if (align >= 16) return launch_kernel<E, D, 16, SPLIT, BS16, BALANCED, true>(kp, grid, stream, resident, per_cu);
    return launch_kernel<E, D, 8, SPLIT, BS16, BALANCED, true>(kp, grid, stream, resident, per_cu);
  } else {
    switch (align) {
      case 16:
        return launch_kernel<E, D, 16, SPLIT, BS16, BALANCED, false>(kp, grid, stream, resident, per_cu);
      case 8:
        if constexpr (D <= 128)
          return launch_kernel<E, D, 8, SPLIT, BS16, BALANCED, false>(kp, grid, stream, resident, per_cu);
        return hipErrorInvalidValue;
      case 4:
        if constexpr (D == 64) return launch_kernel<E, D, 4, SPLIT, BS16, BALANCED, false>(kp, grid, stream, resident, per_cu);
        return hipErrorInvalidValue;
      default:
        return hipErrorInvalidValue;
    }
  }
}

// DK_ATTN_SCHEDULE=grid|balanced|partitions forces the split-K schedule
// (tests and tuning compare them on one input): the grid of 1024-token units,
// the balanced schedule, or the grid of 512-token units (one per workspace
// row); unset or anything else: automatic.
enum class Schedule { kAuto, kGrid, kBalanced, kPartitions };
inline Schedule forced_schedule() {
  const char* v = std::getenv("DK_ATTN_SCHEDULE");
  if (v == nullptr) return Schedule::kAuto;
  if (std::strcmp(v, "grid") == 0) return Schedule::kGrid;
  if (std::strcmp(v, "balanced") == 0) return Schedule::kBalanced;
  if (std::strcmp(v, "partitions") == 0) return Schedule::kPartitions;
  return Schedule::kAuto;
}

// DK_ATTN_LOCKSTEP=0 / 1 overrides the balanced schedule's default grouping
// (read on every call, for tests and measurements).
inline bool lockstep_wanted(bool by_default) {
  const char* v = std::getenv("DK_ATTN_LOCKSTEP");
  if (v != nullptr && std::strcmp(v, "0") == 0) return false;
  if (v != nullptr && std::strcmp(v, "1") == 0) return true;
  return by_default;
}

template <int D, int WPH, bool PIECES, typename E>
void launch_reduce(const KParams& kp, int num_seqs, hipStream_t stream) {
  constexpr int HPW = reduce_waves<WPH>() / WPH;
  const dim3 grid((kp.num_q_heads + HPW - 1) / HPW, num_seqs);
  hipLaunchKernelGGL((paged_attention_reduce_kernel<E, D, WPH, PIECES>), grid, dim3(reduce_waves<WPH>() * kWave), 0,
                     stream, kp);
}

template <typename E, int D, bool PIECES>
void launch_reduce_sized(const KParams& kp, int num_seqs, hipStream_t stream) {
  // Rows a head merges at most.
  const int entries = PIECES ? kp.max_partitions : 2 + (kp.max_partitions - 1) / 2;
  if (entries <= 8) launch_reduce<D, 1, PIECES, E>(kp, num_seqs, stream);
  else if (entries < 64) launch_reduce<D, 4, PIECES, E>(kp, num_seqs, stream);
  else launch_reduce<D, 16, PIECES, E>(kp, num_seqs, stream);
}

template <typename E, int D, bool BS16, bool KV8>
hipError_t launch_split(KParams kp, int num_kv_heads, int num_seqs, int align, hipStream_t stream) {
  const int64_t per_plane = static_cast<int64_t>(num_kv_heads) * num_seqs;
  const int64_t grid_units = per_plane * (kp.num_units + 1);  // 1024-token planes + two 512-token planes
  // The balanced kernel needs the whole length list in LDS and tile counts
  // below 2^31; it pays a short set-up (a scan of the lengths) and wins once
  // the grid would be more than one round of resident workgroups.
  const Schedule forced = forced_schedule();
  const int64_t tile_bound = per_plane * kp.max_partitions * (kPart / kTile);
  // One 512-token unit per workspace row (the reference's partitioning).
  const int64_t partition_units = per_plane * kp.max_partitions;
  int resident = 0;
  int per_cu = 0;
  if (forced != Schedule::kGrid && forced != Schedule::kPartitions &&
      ((num_seqs <= kMaxBalancedSeqs && tile_bound < (int64_t{1} << 30)) || forced == Schedule::kAuto)) {
    const hipError_t e = launch_aligned<E, D, true, BS16, true, KV8>(kp, 0, align, stream, &resident, &per_cu);
    if (e != hipSuccess) return e;
  }
  const bool balanced_ok = num_seqs <= kMaxBalancedSeqs && tile_bound < (int64_t{1} << 30);
  // Two workgroups per CU sharing its SIMDs (4 waves each): the one
  // dispatched first (blockIdx < grid / 2; the second round of dispatch fills
  // each CU's second slot) streams faster, so the first half of the grid
  // takes the larger shares. (2-wave workgroups at 1 wave/SIMD do not share.)
  kp.pair_ratio = per_cu == 2 && waves_per_group<D>() == 4 ? DK_ATTN_PAIR_RATIO : 100;
  // Lockstep groups (a sequence's KV heads over the same tokens at once) for
  // 16-bit caches: 0.5-3% faster over most measured shapes (128K batch 1
  // 2.6%, Llama-3-8B 8 x 32K 3.3%), one 2.5% slower (64 x 8K). With an fp8
  // cache they were up to 23% slower on an NHD cache, so fp8 keeps one
  // workgroup per share.
  kp.lockstep = lockstep_wanted(!KV8) && resident > 0 && resident % num_kv_heads == 0 && resident / num_kv_heads >= 2;
  // Automatic choice: a grid of 512-token units while it needs at most
  // kPartThirds / 3 rounds of resident workgroups (a small call: twice the
  // workgroups of 1024-token units, each with half the tokens, so the call's
  // critical path halves, and no set-up scan); else the balanced schedule
  // when the 1024-token grid would exceed a round; else that grid. The
  // limit per kernel class, measured against the balanced schedule on
  // uniform and ragged batches, vLLM and NHD caches (cold calls):
  //   head_dim <= 64 (4 workgroups per CU): up to 2 rounds (2.5-3 rounds: within +-5%, 4-5: 2-9% slower);
  //   head_dim 96/128, 16-bit cache: 2 rounds (1-2: 0-11% faster; 2-3: vLLM 1-4% slower);
  //   head_dim 96/128, fp8 cache (3 per CU): 4/3 of a round (to 1024 units:
  //     5-15% faster; 1.7-2 rounds: ragged vLLM batches up to 11% slower);
  //   head_dim > 128 (2-wave workgroups): 1 round (1.5-2 rounds: 3-12% slower).
  constexpr int64_t kPartThirds = D > 128 ? 3 : (KV8 && D > 64 ? 4 : 6);
  const bool partitions =
      forced == Schedule::kPartitions ||
      (forced == Schedule::kAuto && resident > 0 && 3 * partition_units <= kPartThirds * resident);
  // An fp8 cache whose KV heads sit side by side within a token (NHD: token
  // stride > head stride), at head_dim 96/128 and contexts up to 4096 tokens,
  // keeps the 1024-token grid: it ran 4-17% faster than the balanced schedule
  // on every such batch measured (Llama-3-8B b64 mixed 69.7 against 83.5 us,
  // b48 x 2048 49.9 / 57.5, Qwen2.5-7B b48 x 4096 47.2 / 52.5), with the same
  // HBM read bytes; at 8K-32K contexts the balanced schedule won as often as
  // it lost, and vLLM / HND caches show no such gap.
  const bool nhd_fp8_grid = KV8 && D > 64 && D <= 128 && kp.k_st > kp.k_sh && kp.max_partitions <= 8;
  const bool balanced =
      !partitions && balanced_ok && resident > 0 &&
      (forced == Schedule::kBalanced || (forced == Schedule::kAuto && grid_units > resident && !nhd_fp8_grid));
  hipError_t e;
  if (partitions) {
    if (partition_units >= (int64_t{1} << 31)) return hipErrorInvalidValue;  // bounded by the host's checks
    kp.unit512 = 1;
    e = launch_aligned<E, D, true, BS16, false, KV8>(kp, static_cast<unsigned>(partition_units), align, stream);
  } else if (balanced) {
    e = launch_aligned<E, D, true, BS16, true, KV8>(kp, static_cast<unsigned>(resident), align, stream);
  } else {
    e = launch_aligned<E, D, true, BS16, false, KV8>(kp, static_cast<unsigned>(grid_units), align, stream);
  }
  if (e != hipSuccess) return e;
  if (balanced || partitions) launch_reduce_sized<E, D, true>(kp, num_seqs, stream);
  else launch_reduce_sized<E, D, false>(kp, num_seqs, stream);
  return hipGetLastError();
}

template <typename E, int D, bool KV8>
hipError_t launch(const KParams& kp, int num_kv_heads, int num_seqs, bool split, bool bs16, int align,
                  hipStream_t stream) {
  if (!split) {
    const unsigned grid = static_cast<unsigned>(num_kv_heads * num_seqs);
    return bs16 ? launch_aligned<E, D, false, true, false, KV8>(kp, grid, align, stream)
                : launch_aligned<E, D, false, false, false, KV8>(kp, grid, align, stream);
  }
  return bs16 ? launch_split<E, D, true, KV8>(kp, num_kv_heads, num_seqs, align, stream)
              : launch_split<E, D, false, KV8>(kp, num_kv_heads, num_seqs, align, stream);
}

template <typename E, int D>
hipError_t launch_kv(const KParams& kp, int num_kv_heads, int num_seqs, bool split, bool bs16, int align, bool kv8,
                     hipStream_t stream) {
  return kv8 ? launch<E, D, true>(kp, num_kv_heads, num_seqs, split, bs16, align, stream)
             : launch<E, D, false>(kp, num_kv_heads, num_seqs, split, bs16, align, stream);
}

// Largest of 16/8/4 bytes that every K/V row start is aligned to, for
// elements of `elt` bytes.
int kv_alignment(const dk_paged_attn_params& a, int elt) {
  const int64_t strides[6] = {a.k_stride_block, a.k_stride_token, a.k_stride_head,
                              a.v_stride_block, a.v_stride_token, a.v_stride_head};
  for (int align : {16, 8, 4}) {
    bool ok = aligned_to(a.k_cache, align) && aligned_to(a.v_cache, align);
    for (int64_t s : strides) ok = ok && ((s * elt) % align == 0);
    if (ok) return align;
  }
  return 1;
}

// Both entry points: 16-bit caches (kv8 = false, scales 1) or e4m3fn caches.
int paged_attention_entry(const dk_paged_attn_params* a, int dtype, int head_dim, int max_seq_len, bool kv8,
                          float k_scale, float v_scale, void* stream) {
  clear_error();
  if (a == nullptr) return fail("paged_attention_decode: params must not be NULL");
  if (dtype != DK_FLOAT16 && dtype != DK_BFLOAT16)
    return fail("paged_attention_decode: expected float16 or bfloat16, got dtype code %d", dtype);
  if (a->num_seqs < 0) return fail("paged_attention_decode: num_seqs must be non-negative");
  if (a->num_seqs == 0) return hipSuccess;
  if (a->num_kv_heads <= 0 || a->num_q_heads <= 0 || a->num_q_heads % a->num_kv_heads != 0)
    return fail("num_q_heads must be a multiple of num_kv_heads");
  const int group = a->num_q_heads / a->num_kv_heads;
  if (group > kMaxGroup) return fail("GQA group size above %d is not supported", kMaxGroup);
  if (head_dim != 64 && head_dim != 96 && head_dim != 128 && head_dim != 192 && head_dim != 256)
    return fail("head_dim must be 64, 96, 128, 192 or 256, got %d", head_dim);
  if (kv8 && head_dim % 64 != 0) return fail("paged_attention_decode_fp8: head_dim must be 64, 128, 192 or 256");
  if (a->block_size <= 0) return fail("paged_attention_decode: block_size must be positive");
  if (max_seq_len < 0) return fail("max_seq_len must be non-negative");
  if (a->q == nullptr || a->out == nullptr || a->k_cache == nullptr || a->v_cache == nullptr ||
      a->block_tables == nullptr || a->seq_lens == nullptr)
    return fail("paged_attention_decode: tensor pointers must not be NULL");
  const int align = kv_alignment(*a, kv8 ? 1 : 2);
  if (kv8) {
    if (align < 8) return fail("fp8 KV-cache pointers and strides must be multiples of 8 bytes");
    if (!(k_scale == k_scale && v_scale == v_scale) || __builtin_isinf(k_scale) || __builtin_isinf(v_scale))
      return fail("paged_attention_decode_fp8: k_scale and v_scale must be finite");
  } else if (align < 4 || (head_dim > 64 && head_dim <= 128 && align < 8) || (head_dim > 128 && align < 16)) {
    return fail("KV-cache pointers must be aligned to head_dim / 16 bytes");
  }
  if (a->num_seqs > 65535 || a->num_kv_heads > 65535 || a->num_q_heads > 65535)
    return fail("paged_attention_decode: num_seqs and head counts must be at most 65535");
  {
    // The kernels take element strides as 32-bit arguments and form every
    // address from them in 64 bits, so any cache size works; only a single
    // stride of 2^31 elements or more (or a negative one) is refused.
    const int64_t st[11] = {a->q_stride_seq,   a->q_stride_head,  a->out_stride_seq, a->out_stride_head,
                            a->k_stride_block, a->k_stride_token, a->k_stride_head,  a->v_stride_block,
                            a->v_stride_token, a->v_stride_head,  a->bt_stride};
    for (int64_t v : st)
      if (v < 0 || v > INT32_MAX)
        return fail("paged_attention_decode: strides must be in [0, 2^31) elements, got %lld",
                    static_cast<long long>(v));
  }

  const bool split = max_seq_len > kPart;
  if (split) {
    if (a->tmp_out == nullptr || a->max_logits == nullptr || a->exp_sums == nullptr)
      return fail("split-K workspace tensors must be provided when max_seq_len > %d", kPart);
    if (a->max_partitions < ceil_div64(max_seq_len, kPart))
      return fail("tmp_out must be [num_seqs, num_q_heads, >= ceil(max_seq_len / 512), head_dim]");
    if (a->max_partitions > 65535) return fail("paged_attention_decode: at most 65535 partitions are supported");
  }

  KParams kp{};
  kp.out = static_cast<uint16_t*>(a->out);
  kp.q = static_cast<const uint16_t*>(a->q);
  kp.k = static_cast<const uint16_t*>(a->k_cache);
  kp.v = static_cast<const uint16_t*>(a->v_cache);
  kp.block_tables = a->block_tables;
  kp.seq_lens = a->seq_lens;
  kp.tmp_out = a->tmp_out;
  kp.max_logits = a->max_logits;
  kp.exp_sums = a->exp_sums;
  kp.q_ss = a->q_stride_seq;
  kp.q_sh = a->q_stride_head;
  kp.o_ss = a->out_stride_seq;
  kp.o_sh = a->out_stride_head;
  kp.k_sb = a->k_stride_block;
  kp.k_st = a->k_stride_token;
  kp.k_sh = a->k_stride_head;
  kp.v_sb = a->v_stride_block;
  kp.v_st = a->v_stride_token;
  kp.v_sh = a->v_stride_head;
  kp.bt_stride = a->bt_stride;
  kp.num_q_heads = a->num_q_heads;
  kp.group = group;
  kp.block_size = a->block_size;
  kp.max_partitions = split ? a->max_partitions : 1;
  // Split-K: the workspace has the reference's shape; its rows hold partial
  // results either per 512-token slot (grid schedule, as the reference's
  // partitions) or per piece (balanced schedule). Like the reference, only
  // max_partitions x 512 tokens are read, so a too-small max_seq_len still
  // bounds every access.
  kp.num_units = split ? static_cast<int>(ceil_div64(a->max_partitions, 2)) : 1;
  kp.scale_log2 = a->scale * k_scale * kLog2e;
  kp.v_scale = v_scale;
  if (static_cast<int64_t>(a->num_seqs) * a->num_kv_heads * (std::max(kp.num_units, kp.max_partitions) + 1) >=
      (int64_t{1} << 31))
    return fail("paged_attention_decode: num_seqs x num_kv_heads x partitions is too large");
  kp.num_seqs = a->num_seqs;
  kp.num_kv_heads = a->num_kv_heads;

  // Whole-tile loads address a tile's 16 rows with 32-bit buffer offsets from
  // the tile's first row; a token stride too large for that takes the per-row
  // path, whose addresses are 64-bit.
  const int64_t elt = kv8 ? 1 : 2;
  const bool rows_fit = static_cast<int64_t>(kTile) * std::max(a->k_stride_token, a->v_stride_token) * elt +
                            2 * head_dim * elt <= INT32_MAX;
  const bool bs16 = a->block_size % kTile == 0 && rows_fit;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (dtype == DK_BFLOAT16) {
    switch (head_dim) {
      case 64: e = launch_kv<Bf16, 64>(kp, a->num_kv_heads, a->num_seqs, split, bs16, align, kv8, s); break;
      case 96: e = launch<Bf16, 96, false>(kp, a->num_kv_heads, a->num_seqs, split, bs16, align, s); break;
      case 128: e = launch_kv<Bf16, 128>(kp, a->num_kv_heads, a->num_seqs, split, bs16, align, kv8, s); break;
      case 192: e = launch_kv<Bf16, 192>(kp, a->num_kv_heads, a->num_seqs, split, bs16, align, kv8, s); break;
      default: e = launch_kv<Bf16, 256>(kp, a->num_kv_heads, a->num_seqs, split, bs16, align, kv8, s); break;
    }
  } else {
    switch (head_dim) {
      case 64: e = launch_kv<F16, 64>(kp, a->num_kv_heads, a->num_seqs, split, bs16, align, kv8, s); break;
      case 96: e = launch<F16, 96, false>(kp, a->num_kv_heads, a->num_seqs, split, bs16, align, s); break;
      case 128: e = launch_kv<F16, 128>(kp, a->num_kv_heads, a->num_seqs, split, bs16, align, kv8, s); break;
      case 192: e = launch_kv<F16, 192>(kp, a->num_kv_heads, a->num_seqs, split, bs16, align, kv8, s); break;
      default: e = launch_kv<F16, 256>(kp, a->num_kv_heads, a->num_seqs, split, bs16, align, kv8, s); break;
    }
  }
  return static_cast<int>(e);
}

int paged_attention_noalloc(const dk_paged_attn_params* a, int dtype, int head_dim, int max_seq_len, void* stream) {
  clear_error();
  if (a == nullptr) return fail("paged_attention_decode_noalloc: params must not be NULL");
  if (a->num_seqs <= 0 || max_seq_len <= kPart) {
    // No split-K: nothing goes through the workspace.
    dk_paged_attn_params b = *a;
    b.tmp_out = b.max_logits = b.exp_sums = nullptr;
    b.max_partitions = 0;
    return paged_attention_entry(&b, dtype, head_dim, max_seq_len, false, 1.0f, 1.0f, stream);
  }
  if (a->num_q_heads <= 0 || head_dim <= 0) return paged_attention_entry(a, dtype, head_dim, max_seq_len, false, 1.0f, 1.0f, stream);
  // Workspace of the reference's shape in the scratch array, each part 256-byte aligned:
  // tmp_out [S, Hq, P, D], then max_logits and exp_sums [S, Hq, P], all fp32.
  const int64_t parts = ceil_div64(max_seq_len, kPart);
  const int64_t rows = static_cast<int64_t>(a->num_seqs) * a->num_q_heads * parts;
  auto up256 = [](int64_t b) { return (b + 255) / 256 * 256; };
  const int64_t tmp_bytes = up256(rows * head_dim * 4);
  const int64_t vec_bytes = up256(rows * 4);
  const int64_t need = tmp_bytes + 2 * vec_bytes;
  if (need > static_cast<int64_t>(DK_NOALLOC_SCRATCH_BYTES))
    return fail("paged_attention_decode_noalloc: the split-K workspace needs %lld bytes (num_seqs x num_q_heads x "
                "ceil(max_seq_len / 512) x (head_dim + 2) x 4), more than the %lld-byte scratch",
                static_cast<long long>(need), static_cast<long long>(DK_NOALLOC_SCRATCH_BYTES));
  int err = 0;
  unsigned char* base = static_cast<unsigned char*>(noalloc_scratch_address(&err));
  if (base == nullptr) return err;
  dk_paged_attn_params b = *a;
  b.tmp_out = reinterpret_cast<float*>(base);
  b.max_logits = reinterpret_cast<float*>(base + tmp_bytes);
  b.exp_sums = reinterpret_cast<float*>(base + tmp_bytes + vec_bytes);
  b.max_partitions = static_cast<int32_t>(parts);
  return paged_attention_entry(&b, dtype, head_dim, max_seq_len, false, 1.0f, 1.0f, stream);
}

}  // namespace attn
}  // namespace dk

extern "C" int dk_paged_attention_decode(const dk_paged_attn_params* a, int dtype, int head_dim, int max_seq_len,
                                         void* stream) {
  return dk::attn::paged_attention_entry(a, dtype, head_dim, max_seq_len, false, 1.0f, 1.0f, stream);
}

extern "C" int dk_paged_attention_decode_noalloc(const dk_paged_attn_params* a, int dtype, int head_dim,
                                                 int max_seq_len, void* stream) {
  return dk::attn::paged_attention_noalloc(a, dtype, head_dim, max_seq_len, stream);
}

extern "C" int dk_paged_attention_decode_fp8(const dk_paged_attn_params* a, int dtype, int head_dim, int max_seq_len,
                                             float k_scale, float v_scale, void* stream) {
  return dk::attn::paged_attention_entry(a, dtype, head_dim, max_seq_len, true, k_scale, v_scale, stream);
}
