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
// * Workgroup = 4 waves of 64 lanes for one (kv_head, seq, partition). The
//   partition's tokens are cut into 16-token tiles; wave w takes tiles
//   w, w+4, ... and keeps its own online-softmax state; the 4 waves merge
//   through LDS at the end (the same log-sum-exp rule as split-K).
// * Q·Kᵀ for a tile is 16 tokens x 16 (padded) query heads x head_dim on
//   v_mfma_f32_16x16x32_{bf16,f16}. Lane l feeds K row (l % 16) with one
//   16-byte load per 32-column step, and the query fragment of head (l % 16)
//   in the model dtype (exact); the fp32 logits come out as
//   S[token 4*(l/16)+r][head l%16], r = 0..3.
// * P·V uses v_mfma_f32_16x16x4_f32, whose A operand (lane l: row l%16,
//   k = l/16) is exactly register r of the Q·Kᵀ result when the 4-token step
//   r takes tokens {4q + r}. Its B operand is a V row per lane group read
//   with one 16-byte load, one MFMA per loaded column, so V never needs a
//   transpose and P stays in fp32. Accumulators: lane l holds
//   O[head 4*(l/16)+i][d(r, l%16)].
// * Logits are kept in log2 units (scale * log2 e folded into one multiply)
//   and exponentiated with v_exp_f32; max_logits are stored in natural-log
//   units so the workspace means what the reference's does.
// * K/V tiles are double-buffered in registers: the loads for tile n+1 are
//   in flight while tile n is multiplied.
#include "../../include/decodekernels_amd.h"
#include "dk_device.h"
#include "dk_host.h"

namespace dk {
namespace attn {

constexpr int kPart = DK_PARTITION_SIZE;  // workspace granularity (tokens)
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
#ifndef DK_ATTN_LOAD_AUX
#define DK_ATTN_LOAD_AUX 0  // cache-policy bits of the K/V buffer loads
#endif
#ifndef DK_ATTN_OCC_D128
#define DK_ATTN_OCC_D128 2  // waves per SIMD targeted at head_dim 128
#endif
#ifndef DK_ATTN_OCC_D64
#define DK_ATTN_OCC_D64 4  // waves per SIMD targeted at head_dim 64
#endif
#ifndef DK_ATTN_UNIT_SLOTS
#define DK_ATTN_UNIT_SLOTS 2  // 512-token workspace slots per split-K work unit (1 or 2)
#endif
static_assert(DK_ATTN_UNIT_SLOTS == 1 || DK_ATTN_UNIT_SLOTS == 2,
              "a work unit's block-table entries must fit one register per lane");
constexpr int kWaves = DK_ATTN_WAVES;
constexpr int kTile = 16;
constexpr int kMaxGroup = DK_MAX_GQA_GROUP;
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
  int64_t q_ss, q_sh, o_ss, o_sh;
  int64_t k_sb, k_st, k_sh, v_sb, v_st, v_sh;
  int64_t bt_stride;
  int num_q_heads, group, block_size, max_partitions;
  int part_tokens;  // tokens per work unit (single pass: 512; split: a multiple of 512)
  float scale_log2;
};


// Word 3 of a gfx9-family buffer resource for raw (untyped) loads.
constexpr int kRsrcWord3 = 0x00020000;

// Raw buffer loads of 8 / 4 consecutive 16-bit elements at byte offset `off`
// of the resource; the resource's num_records bounds the access (0 = none).
template <int ALIGN>
__device__ __forceinline__ u32x4 bload8(__amdgpu_buffer_rsrc_t r, int off) {
  constexpr int A = DK_ATTN_LOAD_AUX;
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
template <int CHUNKS>
struct TileRegs {
  u32x4 k[CHUNKS];
  u32x4 v[CHUNKS];
};

// Log2-units headroom of the lazy running max: exponentials are taken
// against a reference max that only moves when a tile exceeds it by more
// than this, so accumulators are rescaled rarely (weights stay <= 2^8).
constexpr float kLazyMax = 8.0f;

// Waves per SIMD the register allocation targets: head_dim 64 fits four and
// head_dim 128 three without spilling; head_dim 256 keeps its natural
// allocation (one wave, no spills).
template <int D>
constexpr int attn_occupancy() {
  return D >= 256 ? 1 : (D == 128 ? DK_ATTN_OCC_D128 : DK_ATTN_OCC_D64);
}

// NW waves per workgroup; each wave keeps DEPTH tiles of loads in flight.
template <typename E, int D, bool SPLIT, bool BS16, int ALIGN, int NW>
__global__ __launch_bounds__(NW * kWave) __attribute__((amdgpu_waves_per_eu(attn_occupancy<D>(), attn_occupancy<D>())))
void paged_attention_kernel(const KParams p) {
  constexpr int CH = D / 32;  // 32-column chunks per row
  constexpr int NB = D / 16;  // 16-column output blocks
  constexpr int DEPTH = D >= 256 ? 2 : DK_ATTN_DEPTH;
  constexpr int NT = NW * kWave;
  using Tile = TileRegs<CH>;

  const int kv_head = blockIdx.x;
  const int seq = blockIdx.y;
  const int part = blockIdx.z;
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int l16 = lane % 16;  // K/V row of the tile, head of the logits, output column
  const int lg = lane / 16;   // lane group 0..3
  const int group = p.group;

  const int seq_len = p.seq_lens[seq];
  const int start = SPLIT ? part * p.part_tokens : 0;
  if (start >= seq_len) {
    if (!SPLIT) {
      for (int idx = tid; idx < group * D; idx += NT) {
        const int h = idx / D;
        const int d = idx - h * D;
        p.out[seq * p.o_ss + (kv_head * group + h) * p.o_sh + d] = 0;
      }
    }
    return;
  }
  const int end = min(start + p.part_tokens, seq_len);
  const int n_tiles = (end - start + kTile - 1) / kTile;

  __shared__ float sm_m[NW][16];   // reference max per head (log2 units)
  __shared__ float sm_t[NW][16];   // true max per head
  __shared__ float sm_l[NW][16];   // exp-sum against the reference max
  __shared__ float sm_o[NW][kMaxGroup][D];

  // Block-table entries of this work unit (lane e holds entry lb0 + e) when
  // every 16-token tile lies inside one cache block.
  const int32_t* bt_row = p.block_tables + seq * p.bt_stride;
  int lb0 = 0;
  int bt_lane = 0;
  if constexpr (BS16) {
    lb0 = start / p.block_size;
    const int lb_last = (end - 1) / p.block_size;
    if (lb0 + lane <= lb_last) bt_lane = bt_row[lb0 + lane];
  }

  const uint16_t* kbase = p.k + kv_head * p.k_sh;
  const uint16_t* vbase = p.v + kv_head * p.v_sh;

  // Issues the loads of one tile. Tiles past the end are still "loaded" so
  // every wave runs the same load sequence (the compiler then waits for
  // exactly the oldest tile): with whole-tile blocks their buffer resource
  // has num_records = 0 and nothing is read; otherwise the last tile is
  // re-read (an L2 hit). Rows past the sequence end are clamped to its last
  // row, so V never contributes uninitialised cache contents.
  auto load_tile = [&](int tile, Tile& r) {
    const bool live = tile < n_tiles;
    const int tt = live ? tile : n_tiles - 1;
    const int t0 = start + tt * kTile;
    const int row = min(l16, end - 1 - t0);
    if constexpr (BS16) {
      const int lb = t0 / p.block_size;
      const int phys = __builtin_amdgcn_readlane(bt_lane, lb - lb0);
      const int off = t0 - lb * p.block_size;
      const uint16_t* kt = kbase + static_cast<int64_t>(phys) * p.k_sb + static_cast<int64_t>(off) * p.k_st;
      const uint16_t* vt = vbase + static_cast<int64_t>(phys) * p.v_sb + static_cast<int64_t>(off) * p.v_st;
      const int nrec = live ? 0x7fffffff : 0;
      const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(kt), 0, nrec, kRsrcWord3);
      const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(vt), 0, nrec, kRsrcWord3);
      const int koff = 2 * (row * static_cast<int>(p.k_st) + 8 * lg);
      const int voff = 2 * (row * static_cast<int>(p.v_st) + 8 * lg);
#pragma unroll
      for (int c = 0; c < CH; ++c) r.k[c] = bload8<ALIGN>(rk, koff + 64 * c);
#pragma unroll
      for (int c = 0; c < CH; ++c) r.v[c] = bload8<ALIGN>(rv, voff + 64 * c);
    } else {
      const int t = t0 + row;
      const int lb = t / p.block_size;
      const int64_t phys = bt_row[lb];
      const int64_t off = t - lb * p.block_size;
      const uint16_t* kp = kbase + phys * p.k_sb + off * p.k_st + 8 * lg;
      const uint16_t* vp = vbase + phys * p.v_sb + off * p.v_st + 8 * lg;
#pragma unroll
      for (int c = 0; c < CH; ++c) r.k[c] = load8<ALIGN>(kp + 32 * c);
#pragma unroll
      for (int c = 0; c < CH; ++c) r.v[c] = load8<ALIGN>(vp + 32 * c);
    }
  };

  // Query fragments (B operand of Q·Kᵀ): head l16, columns 8*lg + 32*c ... +7,
  // in the model dtype; heads past the group are zero. Loaded before the
  // tiles so that waiting for them never waits for a tile prefetch.
  u32x4 qf[CH];
  {
    const uint16_t* qrow = p.q + seq * p.q_ss + (kv_head * group + l16) * p.q_sh;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (l16 < group) {
        const uint16_t* src = qrow + 8 * lg + 32 * c;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = static_cast<uint32_t>(src[2 * e]) | (static_cast<uint32_t>(src[2 * e + 1]) << 16);
      }
      qf[c] = w;
    }
  }

  // The scheduling barriers keep the tiles' load groups in program order, so
  // the oldest outstanding loads are always those of the next tile consumed.
  Tile buf[DEPTH];
#pragma unroll
  for (int i = 0; i < DEPTH; ++i) {
    load_tile(wave + i * NW, buf[i]);
    __builtin_amdgcn_sched_barrier(0);
  }

  // Identity fragments (B operand of a 16x16x32 MFMA): with them, an MFMA
  // whose A operand is a V chunk returns V transposed into the B-operand
  // layout of v_mfma_f32_16x16x16 -- lane l: V[token 4*lg + r][column l16 (+16)].
  u32x4 eye0, eye1;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int k0 = 8 * lg + 2 * e;
    eye0[e] = (k0 == l16 ? E::kOne : 0u) | ((k0 + 1 == l16 ? E::kOne : 0u) << 16);
    eye1[e] = (k0 == l16 + 16 ? E::kOne : 0u) | ((k0 + 1 == l16 + 16 ? E::kOne : 0u) << 16);
  }

  f32x4 acc[NB];
#pragma unroll
  for (int n = 0; n < NB; ++n) acc[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_ref = -__builtin_huge_valf();   // reference max (log2 units) of head l16
  float m_true = -__builtin_huge_valf();  // exact running max of head l16
  float l_run = 0.0f;                     // this lane's share of the exp-sum against m_ref

  // Online softmax + P·V for one live tile held in `r`.
  auto process = [&](int tile, const Tile& r) {
    // Q·Kᵀ: S[token 4*lg + i][head l16].
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < CH; ++c) s = E::mfma_16x16x32(r.k[c], qf[c], s);

    const int t0 = start + tile * kTile;
    float x[4];
    float tmax = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool valid = t0 + 4 * lg + i < end;
      x[i] = valid ? s[i] * p.scale_log2 : -__builtin_huge_valf();
      tmax = fmaxf(tmax, x[i]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, kWave));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
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
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const f32x4 z = {0.f, 0.f, 0.f, 0.f};
      const f32x4 t_lo = E::mfma_16x16x32(r.v[c], eye0, z);  // columns 32c + l16
      const f32x4 t_hi = E::mfma_16x16x32(r.v[c], eye1, z);  // columns 32c + 16 + l16
      const u32x2 v_lo = {pack2<E>(t_lo[0], t_lo[1]), pack2<E>(t_lo[2], t_lo[3])};
      const u32x2 v_hi = {pack2<E>(t_hi[0], t_hi[1]), pack2<E>(t_hi[2], t_hi[3])};
      acc[2 * c] = E::mfma_16x16x16(p_hi, v_lo, acc[2 * c]);
      acc[2 * c] = E::mfma_16x16x16(p_lo, v_lo, acc[2 * c]);
      acc[2 * c + 1] = E::mfma_16x16x16(p_hi, v_hi, acc[2 * c + 1]);
      acc[2 * c + 1] = E::mfma_16x16x16(p_lo, v_hi, acc[2 * c + 1]);
    }
  };

  // Steady state: consume the oldest tile, refill its registers DEPTH tiles
  // ahead. Loads are issued on every path, so the wait before each tile is
  // for exactly that tile's loads.
  for (int base = wave; base < n_tiles; base += DEPTH * NW) {
#pragma unroll
    for (int i = 0; i < DEPTH; ++i) {
      const int t = base + i * NW;
      if (t < n_tiles) process(t, buf[i]);
      load_tile(t + DEPTH * NW, buf[i]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // Exp-sum of head l16 over all four lane groups.
  float l_tot = l_run + __shfl_xor(l_run, 16, kWave);
  l_tot += __shfl_xor(l_tot, 32, kWave);

  if (lane < 16) {
    sm_m[wave][lane] = m_ref;
    sm_t[wave][lane] = m_true;
    sm_l[wave][lane] = l_tot;
  }
  // acc[n] lane l: O[head 4*lg + i][column 16n + l16].
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = 4 * lg + i;
    if (h < group) {
#pragma unroll
      for (int n = 0; n < NB; ++n) sm_o[wave][h][16 * n + l16] = acc[n][i];
    }
  }
  __syncthreads();

  for (int idx = tid; idx < group * D; idx += NT) {
    const int h = idx / D;
    const int d = idx - h * D;
    float M = sm_m[0][h];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = fmaxf(M, sm_m[w][h]);
    float L = 0.0f;
    float O = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = __builtin_amdgcn_exp2f(sm_m[w][h] - M);
      L += f * sm_l[w][h];
      O += f * sm_o[w][h][d];
    }
    const float res = O / L;
    const int q_head = kv_head * group + h;
    if constexpr (SPLIT) {
      const int64_t row = (static_cast<int64_t>(seq) * p.num_q_heads + q_head) * p.max_partitions + part;
      p.tmp_out[row * D + d] = res;
      if (d == 0) {
        // Report (max logit, exp-sum) against the partition's true max.
        float T = sm_t[0][h];
#pragma unroll
        for (int w = 1; w < NW; ++w) T = fmaxf(T, sm_t[w][h]);
        p.max_logits[row] = T * kLn2;
        p.exp_sums[row] = L * __builtin_amdgcn_exp2f(M - T);
      }
    } else {
      p.out[seq * p.o_ss + q_head * p.o_sh + d] = E::from_float(res);
    }
  }
}

// Log-sum-exp merge of the work units of one (query head, sequence):
//   M = max_p m_p,  w_p = s_p * exp(m_p - M),  out = sum_p w_p o_p / sum_p w_p
// (reference: csrc/paged_attention.cuh:227-269). WPH waves per query head,
// kReduceWaves waves per workgroup. The (m_p, s_p) pairs are uniform across a
// wave (scalar loads) and each lane accumulates D/64 output columns; with
// WPH > 1 the waves of a head take every WPH-th unit and merge through LDS.
constexpr int kReduceWaves = 4;

template <typename E, int D, int WPH>
__global__ __launch_bounds__(kReduceWaves * kWave) void paged_attention_reduce_kernel(const KParams p, int num_slots) {
  constexpr int C = D / kWave;  // columns per lane (1, 2 or 4)
  constexpr int HPW = kReduceWaves / WPH;  // heads per workgroup
  const int wave = static_cast<int>(threadIdx.x) / kWave;
  const int q_head = blockIdx.x * HPW + wave / WPH;
  const int sub = wave % WPH;
  const int seq = blockIdx.y;
  const int lane = threadIdx.x % kWave;
  __shared__ float red[WPH > 1 ? kReduceWaves : 1][D + 1];
  const bool active = q_head < p.num_q_heads;
  uint16_t* out = p.out + seq * p.o_ss + (active ? q_head : 0) * p.o_sh + C * lane;
  const int seq_len = p.seq_lens[seq];
  if (seq_len <= 0) {
    if (active && sub == 0) {
#pragma unroll
      for (int c = 0; c < C; ++c) out[c] = 0;
    }
    return;
  }
  const int n = min((seq_len + p.part_tokens - 1) / p.part_tokens, num_slots);
  const int64_t row0 = (static_cast<int64_t>(seq) * p.num_q_heads + (active ? q_head : 0)) * p.max_partitions;
  const float* ml = p.max_logits + row0;
  const float* es = p.exp_sums + row0;
  const float* tmp = p.tmp_out + row0 * D + C * lane;

  float M = -__builtin_huge_valf();
  for (int i = 0; i < n; ++i) M = fmaxf(M, ml[i]);
  float W = 0.0f;
  float acc[C];
#pragma unroll
  for (int c = 0; c < C; ++c) acc[c] = 0.0f;
#pragma unroll 4
  for (int i = sub; i < n; i += WPH) {
    const float w = es[i] * __builtin_amdgcn_exp2f((ml[i] - M) * kLog2e);
    W += w;
    const float* t = tmp + static_cast<int64_t>(i) * D;
    if constexpr (C == 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(t);
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[c] = fmaf(w, v[c], acc[c]);
    } else {
#pragma unroll
      for (int c = 0; c < C; ++c) acc[c] = fmaf(w, t[c], acc[c]);
    }
  }
  if constexpr (WPH > 1) {
#pragma unroll
    for (int c = 0; c < C; ++c) red[wave][C * lane + c] = acc[c];
    if (lane == 0) red[wave][D] = W;
    __syncthreads();
    if (sub != 0 || !active) return;
    W = 0.0f;
#pragma unroll
    for (int c = 0; c < C; ++c) acc[c] = 0.0f;
#pragma unroll
    for (int w = 0; w < WPH; ++w) {
      W += red[wave + w][D];
#pragma unroll
      for (int c = 0; c < C; ++c) acc[c] += red[wave + w][C * lane + c];
    }
  }
  if (!active) return;
  const float inv = 1.0f / W;
#pragma unroll
  for (int c = 0; c < C; ++c) out[c] = E::from_float(acc[c] * inv);
}

template <typename E, int D, bool SPLIT, bool BS16>
hipError_t launch_main_aligned(const KParams& kp, dim3 grid, int align, hipStream_t stream) {
  constexpr int NW = D >= 256 ? DK_ATTN_WAVES_D256 : kWaves;
  const dim3 block(NW * kWave);
  switch (align) {
    case 16:
      hipLaunchKernelGGL((paged_attention_kernel<E, D, SPLIT, BS16, 16, NW>), grid, block, 0, stream, kp);
      break;
    case 8:
      if constexpr (D <= 128) {
        hipLaunchKernelGGL((paged_attention_kernel<E, D, SPLIT, BS16, 8, NW>), grid, block, 0, stream, kp);
        break;
      }
      return hipErrorInvalidValue;
    case 4:
      if constexpr (D == 64) {
        hipLaunchKernelGGL((paged_attention_kernel<E, D, SPLIT, BS16, 4, NW>), grid, block, 0, stream, kp);
        break;
      }
      return hipErrorInvalidValue;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename E, int D>
hipError_t launch(const KParams& kp, int num_kv_heads, int num_seqs, bool split, int num_slots, bool bs16, int align,
                  hipStream_t stream) {
  if (!split) {
    const dim3 grid(num_kv_heads, num_seqs, 1);
    return bs16 ? launch_main_aligned<E, D, false, true>(kp, grid, align, stream)
                : launch_main_aligned<E, D, false, false>(kp, grid, align, stream);
  }
  const dim3 grid(num_kv_heads, num_seqs, num_slots);
  hipError_t e = bs16 ? launch_main_aligned<E, D, true, true>(kp, grid, align, stream)
                      : launch_main_aligned<E, D, true, false>(kp, grid, align, stream);
  if (e != hipSuccess) return e;
  const dim3 rblock(kReduceWaves * kWave);
  if (num_slots <= 16) {
    const dim3 rgrid((kp.num_q_heads + kReduceWaves - 1) / kReduceWaves, num_seqs);
    hipLaunchKernelGGL((paged_attention_reduce_kernel<E, D, 1>), rgrid, rblock, 0, stream, kp, num_slots);
  } else {
    const dim3 rgrid(kp.num_q_heads, num_seqs);
    hipLaunchKernelGGL((paged_attention_reduce_kernel<E, D, kReduceWaves>), rgrid, rblock, 0, stream, kp, num_slots);
  }
  return hipGetLastError();
}

// Largest of 16/8/4 bytes that every K/V row start is aligned to.
int kv_alignment(const dk_paged_attn_params& a) {
  const int64_t strides[6] = {a.k_stride_block, a.k_stride_token, a.k_stride_head,
                              a.v_stride_block, a.v_stride_token, a.v_stride_head};
  for (int align : {16, 8, 4}) {
    bool ok = aligned_to(a.k_cache, align) && aligned_to(a.v_cache, align);
    for (int64_t s : strides) ok = ok && ((s * 2) % align == 0);
    if (ok) return align;
  }
  return 2;
}

}  // namespace attn
}  // namespace dk

extern "C" int dk_paged_attention_decode(const dk_paged_attn_params* a, int dtype, int head_dim, int max_seq_len,
                                         void* stream) {
  using namespace dk;
  using namespace dk::attn;
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
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail("head_dim must be 64, 128 or 256, got %d", head_dim);
  if (a->block_size <= 0) return fail("paged_attention_decode: block_size must be positive");
  if (max_seq_len < 0) return fail("max_seq_len must be non-negative");
  if (a->q == nullptr || a->out == nullptr || a->k_cache == nullptr || a->v_cache == nullptr ||
      a->block_tables == nullptr || a->seq_lens == nullptr)
    return fail("paged_attention_decode: tensor pointers must not be NULL");
  const int align = kv_alignment(*a);
  if (align < 4 || (head_dim == 128 && align < 8) || (head_dim == 256 && align < 16))
    return fail("KV-cache pointers must be aligned to head_dim / 16 bytes");
  if (a->num_seqs > 65535 || a->num_kv_heads > 65535 || a->num_q_heads > 65535)
    return fail("paged_attention_decode: num_seqs and head counts must be at most 65535");

  const bool split = max_seq_len > kPart;
  int num_slots = 1;
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
  // Split-K work units of DK_ATTN_UNIT_SLOTS x 512 tokens; unit z writes
  // workspace slot z. Like the reference, the grid covers max_partitions x 512
  // tokens, so a too-small max_seq_len still bounds every access.
  kp.part_tokens = split ? kPart * DK_ATTN_UNIT_SLOTS : kPart;
  if (split) num_slots = static_cast<int>(ceil_div64(static_cast<int64_t>(a->max_partitions) * kPart, kp.part_tokens));
  kp.scale_log2 = a->scale * kLog2e;

  const bool bs16 = a->block_size % kTile == 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (dtype == DK_BFLOAT16) {
    switch (head_dim) {
      case 64: e = launch<Bf16, 64>(kp, a->num_kv_heads, a->num_seqs, split, num_slots, bs16, align, s); break;
      case 128: e = launch<Bf16, 128>(kp, a->num_kv_heads, a->num_seqs, split, num_slots, bs16, align, s); break;
      default: e = launch<Bf16, 256>(kp, a->num_kv_heads, a->num_seqs, split, num_slots, bs16, align, s); break;
    }
  } else {
    switch (head_dim) {
      case 64: e = launch<F16, 64>(kp, a->num_kv_heads, a->num_seqs, split, num_slots, bs16, align, s); break;
      case 128: e = launch<F16, 128>(kp, a->num_kv_heads, a->num_seqs, split, num_slots, bs16, align, s); break;
      default: e = launch<F16, 256>(kp, a->num_kv_heads, a->num_seqs, split, num_slots, bs16, align, s); break;
    }
  }
  return static_cast<int>(e);
}
