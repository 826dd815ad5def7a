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
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * kWave;
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

// Column of the V element that MFMA column-step r of lane j (= l % 16) holds.
template <int D>
__device__ __forceinline__ int v_col(int r, int j) {
  if constexpr (D == 64) {
    return 4 * j + r;
  } else {
    return (r / 8) * 128 + 8 * j + (r % 8);
  }
}

template <typename E, int D, bool SPLIT, bool BS16, int ALIGN>
__global__ __launch_bounds__(kThreads) void paged_attention_kernel(const KParams p) {
  constexpr int KSTEPS = D / 32;  // MFMA k-steps of Q·Kᵀ
  constexpr int VPL = D / 16;     // V values per lane per token row
  constexpr int VW = VPL / 2;     // 32-bit words per lane per V row

  const int kv_head = blockIdx.x;
  const int seq = blockIdx.y;
  const int part = blockIdx.z;
  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int l16 = lane % 16;  // token row (K) / head (logits) / column group (V)
  const int lg = lane / 16;   // lane group 0..3
  const int group = p.group;

  const int seq_len = p.seq_lens[seq];
  const int start = SPLIT ? part * p.part_tokens : 0;
  if (start >= seq_len) {
    if (!SPLIT) {
      for (int idx = tid; idx < group * D; idx += kThreads) {
        const int h = idx / D;
        const int d = idx - h * D;
        p.out[seq * p.o_ss + (kv_head * group + h) * p.o_sh + d] = 0;
      }
    }
    return;
  }
  const int end = min(start + p.part_tokens, seq_len);
  const int n_tiles = (end - start + kTile - 1) / kTile;

  __shared__ float sm_m[kWaves][16];
  __shared__ float sm_l[kWaves][16];
  __shared__ float sm_o[kWaves][kMaxGroup][D];

  // Query fragments (B operand of Q·Kᵀ): head l16, columns 8*lg + 32*k ... +7.
  u32x4 qf[KSTEPS];
  {
    const uint16_t* qrow = p.q + seq * p.q_ss + (kv_head * group + l16) * p.q_sh;
#pragma unroll
    for (int k = 0; k < KSTEPS; ++k) {
      u32x4 w = {0u, 0u, 0u, 0u};
      if (l16 < group) {
        const uint16_t* src = qrow + 8 * lg + 32 * k;
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = static_cast<uint32_t>(src[2 * e]) | (static_cast<uint32_t>(src[2 * e + 1]) << 16);
      }
      qf[k] = w;
    }
  }

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

  // Loads one tile's K fragments and V rows into registers.
  auto load_tile = [&](int tile, u32x4 (&kr)[KSTEPS], uint32_t (&vr)[4][VW]) {
    const int t0 = start + tile * kTile;
    const int lim = end - 1 - t0;  // last valid row offset inside the tile
    const int krow = min(l16, lim);
    if constexpr (BS16) {
      const int lb = t0 / p.block_size;
      const int phys = __builtin_amdgcn_readlane(bt_lane, lb - lb0);
      const int off = t0 - lb * p.block_size;
      const uint16_t* kt = kbase + static_cast<int64_t>(phys) * p.k_sb + static_cast<int64_t>(off) * p.k_st;
      const uint16_t* vt = vbase + static_cast<int64_t>(phys) * p.v_sb + static_cast<int64_t>(off) * p.v_st;
      const uint16_t* kp = kt + krow * p.k_st + 8 * lg;
#pragma unroll
      for (int k = 0; k < KSTEPS; ++k) kr[k] = load8<ALIGN>(kp + 32 * k);
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int vrow = min(4 * lg + s, lim);
        const uint16_t* vp = vt + vrow * p.v_st;
        if constexpr (D == 64) {
          const u32x2 w = load4<ALIGN>(vp + 4 * l16);
          vr[s][0] = w[0];
          vr[s][1] = w[1];
        } else {
#pragma unroll
          for (int c = 0; c < VPL / 8; ++c) {
            const u32x4 w = load8<ALIGN>(vp + c * 128 + 8 * l16);
#pragma unroll
            for (int e = 0; e < 4; ++e) vr[s][4 * c + e] = w[e];
          }
        }
      }
    } else {
      {
        const int t = t0 + krow;
        const int lb = t / p.block_size;
        const int phys = bt_row[lb];
        const uint16_t* kp = kbase + static_cast<int64_t>(phys) * p.k_sb +
                             static_cast<int64_t>(t - lb * p.block_size) * p.k_st + 8 * lg;
#pragma unroll
        for (int k = 0; k < KSTEPS; ++k) kr[k] = load8<ALIGN>(kp + 32 * k);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int t = t0 + min(4 * lg + s, lim);
        const int lb = t / p.block_size;
        const int phys = bt_row[lb];
        const uint16_t* vp = vbase + static_cast<int64_t>(phys) * p.v_sb +
                             static_cast<int64_t>(t - lb * p.block_size) * p.v_st;
        if constexpr (D == 64) {
          const u32x2 w = load4<ALIGN>(vp + 4 * l16);
          vr[s][0] = w[0];
          vr[s][1] = w[1];
        } else {
#pragma unroll
          for (int c = 0; c < VPL / 8; ++c) {
            const u32x4 w = load8<ALIGN>(vp + c * 128 + 8 * l16);
#pragma unroll
            for (int e = 0; e < 4; ++e) vr[s][4 * c + e] = w[e];
          }
        }
      }
    }
  };

  f32x4 acc[VPL];
#pragma unroll
  for (int r = 0; r < VPL; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -__builtin_huge_valf();  // running max (log2 units) of head l16
  float l_run = 0.0f;                    // this lane's share of the running exp-sum

  // Online softmax + P·V for one tile whose K/V sit in (kr, vr).
  auto process = [&](int tile, const u32x4 (&kr)[KSTEPS], const uint32_t (&vr)[4][VW]) {
    // Q·Kᵀ for 16 tokens.
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < KSTEPS; ++k) s = E::mfma_16x16x32(kr[k], qf[k], s);

    const int t0 = start + tile * kTile;
    float x[4];
    float tmax = -__builtin_huge_valf();
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const bool valid = t0 + 4 * lg + r < end;
      x[r] = valid ? s[r] * p.scale_log2 : -__builtin_huge_valf();
      tmax = fmaxf(tmax, x[r]);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16, kWave));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32, kWave));
    const float m_new = fmaxf(m_run, tmax);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
    float pr[4];
    float psum = 0.0f;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pr[r] = __builtin_amdgcn_exp2f(x[r] - m_new);
      psum += pr[r];
    }
    l_run = l_run * alpha + psum;

    // Rescale the accumulators of heads 4*lg + i by their alpha.
    if (__any(alpha != 1.0f)) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = __shfl(alpha, 4 * lg + i, kWave);
#pragma unroll
        for (int r = 0; r < VPL; ++r) acc[r][i] *= a;
      }
    }

    // P·V: step st covers tokens {4q + st}; column-step r is one V element per lane.
#pragma unroll
    for (int st = 0; st < 4; ++st) {
#pragma unroll
      for (int w = 0; w < VW; ++w) {
        const uint32_t word = vr[st][w];
        acc[2 * w] = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[st], E::lo(word), acc[2 * w], 0, 0, 0);
        acc[2 * w + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(pr[st], E::hi(word), acc[2 * w + 1], 0, 0, 0);
      }
    }
  };

  // Two statically named register buffers: the next tile loads into one
  // while the other is consumed.
  u32x4 ka[KSTEPS], kb[KSTEPS];
  uint32_t va[4][VW], vb[4][VW];
  int tile = wave;
  if (tile < n_tiles) load_tile(tile, ka, va);
  while (tile < n_tiles) {
    int next = tile + kWaves;
    if (next < n_tiles) load_tile(next, kb, vb);
    process(tile, ka, va);
    tile = next;
    if (tile >= n_tiles) break;
    next = tile + kWaves;
    if (next < n_tiles) load_tile(next, ka, va);
    process(tile, kb, vb);
    tile = next;
  }

  // Exp-sum of head l16 over all four lane groups.
  float l_tot = l_run + __shfl_xor(l_run, 16, kWave);
  l_tot += __shfl_xor(l_tot, 32, kWave);

  if (lane < 16) {
    sm_m[wave][lane] = m_run;
    sm_l[wave][lane] = l_tot;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = 4 * lg + i;
    if (h < group) {
#pragma unroll
      for (int r = 0; r < VPL; ++r) sm_o[wave][h][v_col<D>(r, l16)] = acc[r][i];
    }
  }
  __syncthreads();

  for (int idx = tid; idx < group * D; idx += kThreads) {
    const int h = idx / D;
    const int d = idx - h * D;
    float M = sm_m[0][h];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M = fmaxf(M, sm_m[w][h]);
    float L = 0.0f;
    float O = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
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
        p.max_logits[row] = M * kLn2;
        p.exp_sums[row] = L;
      }
    } else {
      p.out[seq * p.o_ss + q_head * p.o_sh + d] = E::from_float(res);
    }
  }
}

// Log-sum-exp merge of the partitions of one (query head, sequence):
//   M = max_p m_p,  w_p = s_p * exp(m_p - M),  out = sum_p w_p o_p / sum_p w_p
// (reference: csrc/paged_attention.cuh:227-269). Thread groups of D/4 lanes
// take every G-th partition with float4 loads, then merge through LDS.
template <typename E, int D>
__global__ __launch_bounds__(256) void paged_attention_reduce_kernel(const KParams p, int num_slots) {
  constexpr int C4 = D / 4;       // float4 columns
  constexpr int G = 256 / C4;     // partition groups
  extern __shared__ float weights[];  // [num_slots]
  __shared__ float slots[256 / kWave];
  __shared__ f32x4 red[G][C4];

  const int q_head = blockIdx.x;
  const int seq = blockIdx.y;
  const int tid = threadIdx.x;
  uint16_t* out = p.out + seq * p.o_ss + q_head * p.o_sh;
  const int seq_len = p.seq_lens[seq];
  if (seq_len <= 0) {
    for (int d = tid; d < D; d += 256) out[d] = 0;
    return;
  }
  const int n = min((seq_len + p.part_tokens - 1) / p.part_tokens, num_slots);
  const int64_t row0 = (static_cast<int64_t>(seq) * p.num_q_heads + q_head) * p.max_partitions;
  const float* ml = p.max_logits + row0;
  const float* es = p.exp_sums + row0;

  float m = -__builtin_huge_valf();
  for (int i = tid; i < n; i += 256) m = fmaxf(m, ml[i]);
  const float M = block_max(m, slots);
  float tot = 0.0f;
  for (int i = tid; i < n; i += 256) {
    const float w = es[i] * __builtin_amdgcn_exp2f((ml[i] - M) * kLog2e);
    weights[i] = w;
    tot += w;
  }
  tot = block_sum(tot, slots);  // its barriers also publish `weights`
  const float inv = 1.0f / tot;

  const int c = tid % C4;
  const int g = tid / C4;
  const float* tmp = p.tmp_out + row0 * D;
  f32x4 a = {0.f, 0.f, 0.f, 0.f};
  for (int i = g; i < n; i += G) {
    const f32x4 v = reinterpret_cast<const f32x4*>(tmp + static_cast<int64_t>(i) * D)[c];
    const float w = weights[i];
    a[0] = fmaf(w, v[0], a[0]);
    a[1] = fmaf(w, v[1], a[1]);
    a[2] = fmaf(w, v[2], a[2]);
    a[3] = fmaf(w, v[3], a[3]);
  }
  red[g][c] = a;
  __syncthreads();
  if (tid < C4) {
    f32x4 s = red[0][tid];
#pragma unroll
    for (int j = 1; j < G; ++j) {
      const f32x4 t = red[j][tid];
      s[0] += t[0];
      s[1] += t[1];
      s[2] += t[2];
      s[3] += t[3];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) out[4 * tid + e] = E::from_float(s[e] * inv);
  }
}

template <typename E, int D, bool SPLIT, bool BS16>
hipError_t launch_main_aligned(const KParams& kp, dim3 grid, int align, hipStream_t stream) {
  switch (align) {
    case 16:
      hipLaunchKernelGGL((paged_attention_kernel<E, D, SPLIT, BS16, 16>), grid, dim3(kThreads), 0, stream, kp);
      break;
    case 8:
      if constexpr (D <= 128) {
        hipLaunchKernelGGL((paged_attention_kernel<E, D, SPLIT, BS16, 8>), grid, dim3(kThreads), 0, stream, kp);
        break;
      }
      return hipErrorInvalidValue;
    case 4:
      if constexpr (D == 64) {
        hipLaunchKernelGGL((paged_attention_kernel<E, D, SPLIT, BS16, 4>), grid, dim3(kThreads), 0, stream, kp);
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
  const size_t lds = static_cast<size_t>(num_slots) * sizeof(float);
  hipLaunchKernelGGL((paged_attention_reduce_kernel<E, D>), dim3(kp.num_q_heads, num_seqs), dim3(256), lds, stream, kp,
                     num_slots);
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
    if (a->max_partitions > 16384) return fail("paged_attention_decode: at most 16384 partitions are supported");
    // One work unit per 512-token workspace slot, as many as the workspace holds.
    num_slots = a->max_partitions;
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
  kp.part_tokens = kPart;
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
