// The two steps of a decode layer on either side of paged attention that
// DecodeKernels leaves to the serving engine (vLLM runs them as its own ops):
//
//   rotary_embedding: rotates q and k in place by the token's position,
//     pairs (x, y) -> (x cos - y sin, y cos + x sin) with cos / sin from a
//     [max_position, rot_dim] table (cos in the first rot_dim / 2 columns);
//     NeoX pairing takes x = v[i], y = v[i + rot_dim / 2], GPT-J pairing
//     x = v[2i], y = v[2i + 1]; columns past rot_dim are left as they are.
//     fp32 arithmetic with every product and sum rounded on its own (no
//     fused multiply-add), one rounding to the model dtype per output.
//   reshape_and_cache: writes each new token's K and V rows into its paged
//     cache slot (slot_mapping[t] = block * block_size + offset; negative
//     slots are padding and skipped). The caches are addressed by (block,
//     token, head) strides exactly as paged_attention_decode reads them, so
//     NHD, HND and vLLM's interleaved K|V buffers all work.
//
// Both are HBM-bound copies with a little arithmetic: one workgroup per
// token, 16-byte (or 8-byte) vectors where the layout allows, a scalar path
// otherwise. Positions outside the table and slots outside the cache are
// skipped rather than read or written out of bounds. The cache write also
// fills fp8 (e4m3fn) caches (x / scale, saturated, nearest even), and
// rotary_embedding_and_cache runs both steps in one launch with the results
// of the two in sequence, into 16-bit or fp8 caches.
#include <cmath>
#include <type_traits>

#include "../../include/decodekernels_amd.h"
#include "dk_device.h"
#include "dk_host.h"

namespace dk {
namespace rope {

constexpr int kThreads = 256;

struct KParams {
  const int64_t* positions;
  uint16_t* q;
  uint16_t* k;
  const void* cache;
  int64_t q_st, q_sh, k_st, k_sh, cache_stride;
  int num_tokens, hq, hkv, rot_dim, max_position;
};

// Element loader for a cache stored in the model dtype E.
template <typename E, typename CT>
__device__ __forceinline__ float table(const void* base, int64_t idx) {
  if constexpr (sizeof(CT) == 4) {
    return static_cast<const float*>(base)[idx];
  } else {
    return E::to_float(static_cast<const uint16_t*>(base)[idx]);
  }
}

// One rotated pair with each product and the sum rounded to fp32 on its own
// (no fused multiply-add): the same roundings as evaluating the two formulas
// term by term, so the result does not depend on what the compiler fuses.
__device__ __forceinline__ void rotate(float x, float y, float c, float s, float& ox, float& oy) {
#pragma clang fp contract(off)
  ox = x * c - y * s;
  oy = y * c + x * s;
}

// VW pairs per thread step: 4 with vector loads (8 bytes per half for NeoX,
// 16 bytes for GPT-J), 1 on the scalar path.
template <typename E, typename CT, bool NEOX, int VW>
__global__ __launch_bounds__(kThreads) void rotary_kernel(const KParams p) {
  const int t = blockIdx.x;
  const int64_t pos = p.positions[t];
  if (pos < 0 || pos >= p.max_position) return;
  const int half = p.rot_dim / 2;
  const int64_t crow = pos * p.cache_stride;
  const int steps = half / VW;  // per head
  const int total = (p.hq + p.hkv) * steps;
  for (int c = threadIdx.x; c < total; c += kThreads) {
    const int h = c / steps;
    const int i0 = (c - h * steps) * VW;
    uint16_t* v = h < p.hq ? p.q + t * p.q_st + h * p.q_sh : p.k + t * p.k_st + (h - p.hq) * p.k_sh;
    float x[VW], y[VW], cs[VW], sn[VW];
#pragma unroll
    for (int j = 0; j < VW; ++j) {
      cs[j] = table<E, CT>(p.cache, crow + i0 + j);
      sn[j] = table<E, CT>(p.cache, crow + half + i0 + j);
    }
    if constexpr (NEOX) {
      if constexpr (VW == 4) {
        const u32x2 a = *reinterpret_cast<const u32x2*>(v + i0);
        const u32x2 b = *reinterpret_cast<const u32x2*>(v + half + i0);
        x[0] = E::lo(a[0]), x[1] = E::hi(a[0]), x[2] = E::lo(a[1]), x[3] = E::hi(a[1]);
        y[0] = E::lo(b[0]), y[1] = E::hi(b[0]), y[2] = E::lo(b[1]), y[3] = E::hi(b[1]);
      } else {
        x[0] = E::to_float(v[i0]);
        y[0] = E::to_float(v[half + i0]);
      }
    } else {
      if constexpr (VW == 4) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(v + 2 * i0);
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = E::lo(a[j]), y[j] = E::hi(a[j]);
      } else {
        x[0] = E::to_float(v[2 * i0]);
        y[0] = E::to_float(v[2 * i0 + 1]);
      }
    }
    float ox[VW], oy[VW];
#pragma unroll
    for (int j = 0; j < VW; ++j) rotate(x[j], y[j], cs[j], sn[j], ox[j], oy[j]);
    if constexpr (NEOX) {
      if constexpr (VW == 4) {
        *reinterpret_cast<u32x2*>(v + i0) = u32x2{pack2<E>(ox[0], ox[1]), pack2<E>(ox[2], ox[3])};
        *reinterpret_cast<u32x2*>(v + half + i0) = u32x2{pack2<E>(oy[0], oy[1]), pack2<E>(oy[2], oy[3])};
      } else {
        v[i0] = E::from_float(ox[0]);
        v[half + i0] = E::from_float(oy[0]);
      }
    } else {
      if constexpr (VW == 4) {
        u32x4 o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = pack2<E>(ox[j], oy[j]);
        *reinterpret_cast<u32x4*>(v + 2 * i0) = o;
      } else {
        v[2 * i0] = E::from_float(ox[0]);
        v[2 * i0 + 1] = E::from_float(oy[0]);
      }
    }
  }
}

template <typename E, typename CT>
hipError_t launch_rotary(const KParams& kp, bool neox, bool vec, hipStream_t s) {
  const dim3 grid(kp.num_tokens), block(kThreads);
  if (neox) {
    if (vec) hipLaunchKernelGGL((rotary_kernel<E, CT, true, 4>), grid, block, 0, s, kp);
    else hipLaunchKernelGGL((rotary_kernel<E, CT, true, 1>), grid, block, 0, s, kp);
  } else {
    if (vec) hipLaunchKernelGGL((rotary_kernel<E, CT, false, 4>), grid, block, 0, s, kp);
    else hipLaunchKernelGGL((rotary_kernel<E, CT, false, 1>), grid, block, 0, s, kp);
  }
  return hipGetLastError();
}

}  // namespace rope

namespace cache {

constexpr int kThreads = 256;

struct KParams {
  const uint16_t* key;
  const uint16_t* value;
  uint16_t* kc;
  uint16_t* vc;
  const int64_t* slots;
  int64_t k_st, k_sh, v_st, v_sh;
  int64_t kc_sb, kc_st, kc_sh, vc_sb, vc_st, vc_sh;
  int num_tokens, hkv, d, block_size, num_blocks;
};

// VEC elements per copy: 8 (16-byte vectors) or 1.
template <int VEC>
__global__ __launch_bounds__(kThreads) void reshape_and_cache_kernel(const KParams p) {
  const int t = blockIdx.x;
  const int64_t slot = p.slots[t];
  if (slot < 0) return;
  const int64_t blk = slot / p.block_size;
  const int64_t off = slot - blk * p.block_size;
  if (blk >= p.num_blocks) return;
  const int per_head = p.d / VEC;
  const int n = p.hkv * per_head;
  for (int c = threadIdx.x; c < 2 * n; c += kThreads) {
    const bool is_v = c >= n;
    const int cc = is_v ? c - n : c;
    const int h = cc / per_head;
    const int d0 = (cc - h * per_head) * VEC;
    const uint16_t* src = is_v ? p.value + t * p.v_st + h * p.v_sh + d0 : p.key + t * p.k_st + h * p.k_sh + d0;
    uint16_t* dst = is_v ? p.vc + blk * p.vc_sb + off * p.vc_st + h * p.vc_sh + d0
                         : p.kc + blk * p.kc_sb + off * p.kc_st + h * p.kc_sh + d0;
    if constexpr (VEC == 8) {
      *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(src);
    } else {
      *dst = *src;
    }
  }
}

// Into an fp8 (e4m3fn) cache, as vLLM's reshape_and_cache_flash does for an
// "fp8" cache: x / scale in fp32, saturated to the largest finite value
// (+-448; NaN stays NaN), rounded to nearest even by v_cvt_pk_fp8_f32, which
// gives torch's float -> float8_e4m3fn cast on every input (checked on the
// device over all values, midpoints and their neighbours). The caches hold
// one byte per element; strides are in elements.
__device__ __forceinline__ float sat_e4m3(float y) { return y != y ? y : fminf(fmaxf(y, -448.0f), 448.0f); }

// a, b, c, d quantized into the bytes of one word, a in the lowest.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d, float scale) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(sat_e4m3(a / scale), sat_e4m3(b / scale), 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(sat_e4m3(c / scale), sat_e4m3(d / scale), w, true);
  return static_cast<uint32_t>(w);
}

__device__ __forceinline__ uint8_t e4m3(float a, float scale) {
  return static_cast<uint8_t>(__builtin_amdgcn_cvt_pk_fp8_f32(sat_e4m3(a / scale), 0.0f, 0, false) & 0xff);
}

template <typename E, int VEC>
__global__ __launch_bounds__(kThreads) void reshape_and_cache_fp8_kernel(const KParams p, float k_scale, float v_scale) {
  const int t = blockIdx.x;
  const int64_t slot = p.slots[t];
  if (slot < 0) return;
  const int64_t blk = slot / p.block_size;
  const int64_t off = slot - blk * p.block_size;
  if (blk >= p.num_blocks) return;
  uint8_t* kc = reinterpret_cast<uint8_t*>(p.kc);
  uint8_t* vc = reinterpret_cast<uint8_t*>(p.vc);
  const int per_head = p.d / VEC;
  const int n = p.hkv * per_head;
  for (int c = threadIdx.x; c < 2 * n; c += kThreads) {
    const bool is_v = c >= n;
    const int cc = is_v ? c - n : c;
    const int h = cc / per_head;
    const int d0 = (cc - h * per_head) * VEC;
    const uint16_t* src = is_v ? p.value + t * p.v_st + h * p.v_sh + d0 : p.key + t * p.k_st + h * p.k_sh + d0;
    uint8_t* dst = is_v ? vc + blk * p.vc_sb + off * p.vc_st + h * p.vc_sh + d0
                        : kc + blk * p.kc_sb + off * p.kc_st + h * p.kc_sh + d0;
    const float scale = is_v ? v_scale : k_scale;
    if constexpr (VEC == 8) {
      const u32x4 x = *reinterpret_cast<const u32x4*>(src);
      *reinterpret_cast<u32x2*>(dst) = u32x2{e4m3x4(E::lo(x[0]), E::hi(x[0]), E::lo(x[1]), E::hi(x[1]), scale),
                                             e4m3x4(E::lo(x[2]), E::hi(x[2]), E::lo(x[3]), E::hi(x[3]), scale)};
    } else {
      *dst = e4m3(E::to_float(*src), scale);
    }
  }
}

}  // namespace cache

namespace rope_cache {

// 1024 threads per token: with a GEMM's split-K partials to sum first (a
// [tokens, N] row each, 64 tokens at decode batch 64, so only 64 workgroups),
// the row's loads are spread over four times the threads of the rotary /
// cache work alone; 256 threads took 10.9 us for the qkv row of Llama-3-8B at
// batch 64, more than the separate reduce and rotary kernels together.
constexpr int kThreads = 1024;

struct KParams {
  rope::KParams r;   // positions, q, k (rotated in place), cos | sin table
  cache::KParams c;  // key (== r.k), value, caches, slots
  // Split-K input (part != nullptr): q, k and v are views of the rows of a
  // GEMM output C [num_tokens, N] whose K splits left fp32 partial planes
  // [splits][num_tokens][N]; each token's row of C is first formed from them.
  const float* part;
  const uint16_t* bias;
  uint16_t* C;
  int64_t ldc, plane;
  int N, splits, vec_c;
};

// Row t of C = round(sum of the partial planes in split order, starting from
// 0, plus the bias or 0): gemm_splitk_reduce_kernel's arithmetic and store
// path (8-byte packed stores where it uses them, elementwise otherwise), so C
// ends bit for bit as the GEMM's own reduce leaves it.
constexpr int kMaxSplits = 8;  // the GEMM plans split K at most 8 ways (checked by the host)

template <typename E>
__device__ __forceinline__ void reduce_row(const KParams& p, int t) {
  const float* prow = p.part + static_cast<int64_t>(t) * p.N;
  uint16_t* crow = p.C + static_cast<int64_t>(t) * p.ldc;
  for (int n = 4 * static_cast<int>(threadIdx.x); n < p.N; n += 4 * kThreads) {
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (p.N % 4 == 0) {
      // Every split's 16 bytes are loaded before the in-order sum, so one
      // round trip serves them all (a load per split in turn took one each).
      f32x4 x[kMaxSplits];
#pragma unroll
      for (int sp = 0; sp < kMaxSplits; ++sp)
        if (sp < p.splits) x[sp] = *reinterpret_cast<const f32x4*>(prow + sp * p.plane + n);
#pragma unroll
      for (int sp = 0; sp < kMaxSplits; ++sp)
        if (sp < p.splits) {
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] += x[sp][r];
        }
    } else {
      for (int sp = 0; sp < p.splits; ++sp) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < p.N) v[r] += prow[sp * p.plane + n + r];
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] += p.bias != nullptr ? E::to_float(p.bias[min(n + r, p.N - 1)]) : 0.0f;
    if (p.vec_c && n + 3 < p.N) {
      *reinterpret_cast<u32x2*>(crow + n) = u32x2{pack2<E>(v[0], v[1]), pack2<E>(v[2], v[3])};
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (n + r < p.N) crow[n + r] = E::from_float(v[r]);
    }
  }
}

// rotary_embedding followed by reshape_and_cache in one launch, one
// workgroup per token. The thread that rotates a pair of k also writes it to
// the cache slot (nothing is read back after it is written), the k columns
// past rot_dim and the v row are copied. Identical results to the two ops in
// sequence: same per-pair arithmetic, and a skipped position (outside the
// table) caches the unrotated k, a skipped slot rotates without caching.
// VEC: 4 pairs per rotation step and 16-byte copies; else one element.
// FP8: the caches hold e4m3fn bytes and every value is written as the fp8
// cache write quantizes it, after the rounding to E that the two-op sequence
// stores in k first.
template <typename E, typename CT, bool NEOX, bool VEC, bool FP8>
__global__ __launch_bounds__(kThreads) void rotary_and_cache_kernel(const KParams p, float k_scale, float v_scale) {
  constexpr int VW = VEC ? 4 : 1;
  constexpr int VC = VEC ? 8 : 1;
  const int t = blockIdx.x;
  const rope::KParams& r = p.r;
  const cache::KParams& c = p.c;
  if (p.part != nullptr) {  // the token's q | k | v row from the GEMM's partials, before anything reads it
    reduce_row<E>(p, t);
    __syncthreads();
  }
  const int64_t pos = r.positions[t];
  const bool rot = pos >= 0 && pos < r.max_position;
  const int64_t slot = c.slots[t];
  const int64_t blk = slot >= 0 ? slot / c.block_size : 0;
  const bool put = slot >= 0 && blk < c.num_blocks;
  const int64_t off = put ? slot - blk * c.block_size : 0;  // a skipped slot never forms a cache address
  if (!rot && !put) return;
  const int half = r.rot_dim / 2;
  const int64_t crow = pos * r.cache_stride;
  const int steps = half / VW;         // rotation steps per head
  const int rot_items = (r.hq + r.hkv) * steps;
  const int tail = (c.d - r.rot_dim) / VC;  // k copy chunks past rot_dim, per head
  const int vrow = c.d / VC;               // v copy chunks per head
  const int copy_items = put ? c.hkv * (tail + vrow) : 0;
  // Cache rows as element pointers of the cache's own width (fp8: bytes).
  using CE = std::conditional_t<FP8, uint8_t, uint16_t>;
  CE* const kcb = reinterpret_cast<CE*>(c.kc) + blk * c.kc_sb + off * c.kc_st;
  CE* const vcb = reinterpret_cast<CE*>(c.vc) + blk * c.vc_sb + off * c.vc_st;
  for (int it = threadIdx.x; it < rot_items + copy_items; it += kThreads) {
    if (it < rot_items) {
      const int h = it / steps;
      const int i0 = (it - h * steps) * VW;
      const bool is_k = h >= r.hq;
      if (!is_k && !rot) continue;
      if (is_k && !rot && !put) continue;
      const int hk = h - r.hq;
      uint16_t* v = is_k ? r.k + t * r.k_st + hk * r.k_sh : r.q + t * r.q_st + h * r.q_sh;
      // Element offsets of the VW x / y values: NeoX x at i0.., y at half + i0..; GPT-J interleaved at 2 i0.
      float x[VW], y[VW], ox[VW], oy[VW];
      if constexpr (NEOX) {
        if constexpr (VEC) {
          const u32x2 a = *reinterpret_cast<const u32x2*>(v + i0);
          const u32x2 b = *reinterpret_cast<const u32x2*>(v + half + i0);
          x[0] = E::lo(a[0]), x[1] = E::hi(a[0]), x[2] = E::lo(a[1]), x[3] = E::hi(a[1]);
          y[0] = E::lo(b[0]), y[1] = E::hi(b[0]), y[2] = E::lo(b[1]), y[3] = E::hi(b[1]);
        } else {
          x[0] = E::to_float(v[i0]);
          y[0] = E::to_float(v[half + i0]);
        }
      } else {
        if constexpr (VEC) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(v + 2 * i0);
#pragma unroll
          for (int j = 0; j < 4; ++j) x[j] = E::lo(a[j]), y[j] = E::hi(a[j]);
        } else {
          x[0] = E::to_float(v[2 * i0]);
          y[0] = E::to_float(v[2 * i0 + 1]);
        }
      }
      if (rot) {
#pragma unroll
        for (int j = 0; j < VW; ++j) {
          const float cs = rope::table<E, CT>(r.cache, crow + i0 + j);
          const float sn = rope::table<E, CT>(r.cache, crow + half + i0 + j);
          rope::rotate(x[j], y[j], cs, sn, ox[j], oy[j]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < VW; ++j) ox[j] = x[j], oy[j] = y[j];
      }
      // The rotated row itself, in E.
      auto store16 = [&](uint16_t* o) {
        if constexpr (NEOX) {
          if constexpr (VEC) {
            *reinterpret_cast<u32x2*>(o + i0) = u32x2{pack2<E>(ox[0], ox[1]), pack2<E>(ox[2], ox[3])};
            *reinterpret_cast<u32x2*>(o + half + i0) = u32x2{pack2<E>(oy[0], oy[1]), pack2<E>(oy[2], oy[3])};
          } else {
            o[i0] = E::from_float(ox[0]);
            o[half + i0] = E::from_float(oy[0]);
          }
        } else {
          if constexpr (VEC) {
            u32x4 w;
#pragma unroll
            for (int j = 0; j < 4; ++j) w[j] = pack2<E>(ox[j], oy[j]);
            *reinterpret_cast<u32x4*>(o + 2 * i0) = w;
          } else {
            o[2 * i0] = E::from_float(ox[0]);
            o[2 * i0 + 1] = E::from_float(oy[0]);
          }
        }
      };
      if (rot) store16(v);
      if (!(is_k && put)) continue;
      if constexpr (FP8) {
        // The value k holds after the rotation (rounded to E), quantized.
#pragma unroll
        for (int j = 0; j < VW; ++j) ox[j] = E::to_float(E::from_float(ox[j])), oy[j] = E::to_float(E::from_float(oy[j]));
        uint8_t* o = kcb + hk * c.kc_sh;
        if constexpr (NEOX) {
          if constexpr (VEC) {
            *reinterpret_cast<uint32_t*>(o + i0) = cache::e4m3x4(ox[0], ox[1], ox[2], ox[3], k_scale);
            *reinterpret_cast<uint32_t*>(o + half + i0) = cache::e4m3x4(oy[0], oy[1], oy[2], oy[3], k_scale);
          } else {
            o[i0] = cache::e4m3(ox[0], k_scale);
            o[half + i0] = cache::e4m3(oy[0], k_scale);
          }
        } else {
          if constexpr (VEC) {
            *reinterpret_cast<u32x2*>(o + 2 * i0) = u32x2{cache::e4m3x4(ox[0], oy[0], ox[1], oy[1], k_scale),
                                                          cache::e4m3x4(ox[2], oy[2], ox[3], oy[3], k_scale)};
          } else {
            o[2 * i0] = cache::e4m3(ox[0], k_scale);
            o[2 * i0 + 1] = cache::e4m3(oy[0], k_scale);
          }
        }
      } else {
        store16(kcb + hk * c.kc_sh);
      }
    } else {
      // Copies: k columns past rot_dim, then the v row.
      const int cc = it - rot_items;
      const bool is_v = cc >= c.hkv * tail;
      const int ci = is_v ? cc - c.hkv * tail : cc;
      const int per = is_v ? vrow : tail;
      const int h = ci / per;
      const int d0 = (is_v ? 0 : r.rot_dim) + (ci - h * per) * VC;
      const uint16_t* src = is_v ? c.value + t * c.v_st + h * c.v_sh + d0 : c.key + t * c.k_st + h * c.k_sh + d0;
      CE* dst = is_v ? vcb + h * c.vc_sh + d0 : kcb + h * c.kc_sh + d0;
      if constexpr (FP8) {
        const float scale = is_v ? v_scale : k_scale;
        if constexpr (VEC) {
          const u32x4 a = *reinterpret_cast<const u32x4*>(src);
          *reinterpret_cast<u32x2*>(dst) = u32x2{cache::e4m3x4(E::lo(a[0]), E::hi(a[0]), E::lo(a[1]), E::hi(a[1]), scale),
                                                 cache::e4m3x4(E::lo(a[2]), E::hi(a[2]), E::lo(a[3]), E::hi(a[3]), scale)};
        } else {
          *dst = cache::e4m3(E::to_float(*src), scale);
        }
      } else if constexpr (VEC) {
        *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(src);
      } else {
        *dst = *src;
      }
    }
  }
}

template <typename E, typename CT, bool FP8>
hipError_t launch(const KParams& kp, bool neox, bool vec, float k_scale, float v_scale, hipStream_t s) {
  const dim3 grid(kp.r.num_tokens), block(kThreads);
  if (neox) {
    if (vec) hipLaunchKernelGGL((rotary_and_cache_kernel<E, CT, true, true, FP8>), grid, block, 0, s, kp, k_scale, v_scale);
    else hipLaunchKernelGGL((rotary_and_cache_kernel<E, CT, true, false, FP8>), grid, block, 0, s, kp, k_scale, v_scale);
  } else {
    if (vec) hipLaunchKernelGGL((rotary_and_cache_kernel<E, CT, false, true, FP8>), grid, block, 0, s, kp, k_scale, v_scale);
    else hipLaunchKernelGGL((rotary_and_cache_kernel<E, CT, false, false, FP8>), grid, block, 0, s, kp, k_scale, v_scale);
  }
  return hipGetLastError();
}

template <bool FP8>
hipError_t launch_any(const KParams& kp, int dtype, int table_dtype, bool neox, bool vec, float k_scale, float v_scale,
                      hipStream_t s) {
  if (table_dtype == DK_FLOAT32)
    return dtype == DK_BFLOAT16 ? launch<Bf16, float, FP8>(kp, neox, vec, k_scale, v_scale, s)
                                : launch<F16, float, FP8>(kp, neox, vec, k_scale, v_scale, s);
  return dtype == DK_BFLOAT16 ? launch<Bf16, uint16_t, FP8>(kp, neox, vec, k_scale, v_scale, s)
                              : launch<F16, uint16_t, FP8>(kp, neox, vec, k_scale, v_scale, s);
}

}  // namespace rope_cache
}  // namespace dk

namespace dk {
namespace {

// Argument checks and kernel parameters of rotary_embedding; returns a
// dk error code (0: launchable, with *empty set when there is nothing to do).
int rotary_params(const char* op, const dk_rotary_params* a, int dtype, rope::KParams& kp, bool& neox, bool& vec,
                  bool& empty) {
  empty = false;
  if (a == nullptr) return fail("%s: params must not be NULL", op);
  if (dtype != DK_FLOAT16 && dtype != DK_BFLOAT16) return fail("%s: expected float16 or bfloat16, got dtype code %d", op, dtype);
  if (a->cache_dtype != dtype && a->cache_dtype != DK_FLOAT32)
    return fail("%s: cos_sin_cache must be float32 or the query dtype", op);
  if (a->num_tokens < 0 || a->num_q_heads < 0 || a->num_kv_heads < 0) return fail("%s: sizes must be non-negative", op);
  if (a->num_tokens == 0) {
    empty = true;
    return 0;
  }
  if (a->rot_dim <= 0 || a->rot_dim % 2 != 0 || a->rot_dim > a->head_size)
    return fail("%s: rot_dim must be even and at most head_size", op);
  if (a->positions == nullptr || a->query == nullptr || a->cos_sin_cache == nullptr)
    return fail("%s: positions, query and cos_sin_cache must not be NULL", op);
  if (a->num_tokens > 0x7fffffff / 2) return fail("%s: too many tokens", op);
  kp = rope::KParams{};
  kp.positions = a->positions;
  kp.q = static_cast<uint16_t*>(a->query);
  kp.k = static_cast<uint16_t*>(a->key);
  kp.cache = a->cos_sin_cache;
  kp.q_st = a->q_stride_token;
  kp.q_sh = a->q_stride_head;
  kp.k_st = a->k_stride_token;
  kp.k_sh = a->k_stride_head;
  kp.cache_stride = a->cache_stride;
  kp.num_tokens = a->num_tokens;
  kp.hq = a->num_q_heads;
  kp.hkv = a->key != nullptr ? a->num_kv_heads : 0;
  kp.rot_dim = a->rot_dim;
  kp.max_position = a->max_position;
  neox = a->is_neox != 0;
  // Vector path: 4 pairs per step, every row start aligned to the vector.
  const int half = a->rot_dim / 2;
  const int vbytes = neox ? 8 : 16;
  const int velems = vbytes / 2;
  vec = half % 4 == 0 && aligned_to(a->query, vbytes) && a->q_stride_token % velems == 0 &&
        a->q_stride_head % velems == 0 && (!neox || half % velems == 0);
  if (kp.hkv > 0)
    vec = vec && aligned_to(a->key, vbytes) && a->k_stride_token % velems == 0 && a->k_stride_head % velems == 0;
  return 0;
}

// Argument checks and kernel parameters of reshape_and_cache (as above).
int cache_params(const char* op, const dk_cache_write_params* a, int dtype, cache::KParams& kp, bool& vec, bool& empty) {
  empty = false;
  if (a == nullptr) return fail("%s: params must not be NULL", op);
  if (dtype != DK_FLOAT16 && dtype != DK_BFLOAT16) return fail("%s: expected float16 or bfloat16, got dtype code %d", op, dtype);
  if (a->num_tokens < 0 || a->num_kv_heads <= 0 || a->head_size <= 0 || a->block_size <= 0 || a->num_blocks < 0)
    return fail("%s: sizes must be positive", op);
  if (a->num_tokens == 0) {
    empty = true;
    return 0;
  }
  if (a->key == nullptr || a->value == nullptr || a->key_cache == nullptr || a->value_cache == nullptr ||
      a->slot_mapping == nullptr)
    return fail("%s: pointers must not be NULL", op);
  kp = cache::KParams{};
  kp.key = static_cast<const uint16_t*>(a->key);
  kp.value = static_cast<const uint16_t*>(a->value);
  kp.kc = static_cast<uint16_t*>(a->key_cache);
  kp.vc = static_cast<uint16_t*>(a->value_cache);
  kp.slots = a->slot_mapping;
  kp.k_st = a->k_stride_token;
  kp.k_sh = a->k_stride_head;
  kp.v_st = a->v_stride_token;
  kp.v_sh = a->v_stride_head;
  kp.kc_sb = a->kc_stride_block;
  kp.kc_st = a->kc_stride_token;
  kp.kc_sh = a->kc_stride_head;
  kp.vc_sb = a->vc_stride_block;
  kp.vc_st = a->vc_stride_token;
  kp.vc_sh = a->vc_stride_head;
  kp.num_tokens = a->num_tokens;
  kp.hkv = a->num_kv_heads;
  kp.d = a->head_size;
  kp.block_size = a->block_size;
  kp.num_blocks = a->num_blocks;
  vec = a->head_size % 8 == 0 && aligned_to(a->key, 16) && aligned_to(a->value, 16) && aligned_to(a->key_cache, 16) &&
        aligned_to(a->value_cache, 16) && a->k_stride_token % 8 == 0 && a->k_stride_head % 8 == 0 &&
        a->v_stride_token % 8 == 0 && a->v_stride_head % 8 == 0 && a->kc_stride_block % 8 == 0 &&
        a->kc_stride_token % 8 == 0 && a->kc_stride_head % 8 == 0 && a->vc_stride_block % 8 == 0 &&
        a->vc_stride_token % 8 == 0 && a->vc_stride_head % 8 == 0;
  return 0;
}

// Vector path of a cache write into fp8 caches: 16-byte reads of key /
// value, 8-byte writes of e4m3 bytes.
bool fp8_cache_vec(const dk_cache_write_params* a) {
  return a->head_size % 8 == 0 && aligned_to(a->key, 16) && aligned_to(a->value, 16) && aligned_to(a->key_cache, 8) &&
         aligned_to(a->value_cache, 8) && a->k_stride_token % 8 == 0 && a->k_stride_head % 8 == 0 &&
         a->v_stride_token % 8 == 0 && a->v_stride_head % 8 == 0 && a->kc_stride_block % 8 == 0 &&
         a->kc_stride_token % 8 == 0 && a->kc_stride_head % 8 == 0 && a->vc_stride_block % 8 == 0 &&
         a->vc_stride_token % 8 == 0 && a->vc_stride_head % 8 == 0;
}

int check_scales(const char* op, float k_scale, float v_scale) {
  if (!(k_scale > 0.0f && v_scale > 0.0f && k_scale < INFINITY && v_scale < INFINITY))
    return fail("%s: k_scale and v_scale must be positive and finite", op);
  return 0;
}

// Argument checks of the fused rotary + cache write: both halves as above,
// then the agreement between them. *vec: the vector path is usable (with
// 16-bit caches, or with fp8 caches when fp8 is set).
int fused_params(const char* op, const dk_rotary_params* r, const dk_cache_write_params* c, int dtype, bool fp8,
                 rope_cache::KParams& kp, bool& neox, bool& vec, bool& empty) {
  kp = rope_cache::KParams{};  // no split-K input unless the caller sets one
  bool rvec = false, cvec = false, cempty = false;
  if (const int rc = rotary_params(op, r, dtype, kp.r, neox, rvec, empty)) return rc;
  if (const int rc = cache_params(op, c, dtype, kp.c, cvec, cempty)) return rc;
  if (r->num_tokens != c->num_tokens) return fail("%s: the rotary and cache token counts differ", op);
  if (empty) return 0;
  if (r->key == nullptr || r->key != c->key || r->k_stride_token != c->k_stride_token ||
      r->k_stride_head != c->k_stride_head)
    return fail("%s: the rotated key and the cached key must be the same tensor", op);
  if (r->num_kv_heads != c->num_kv_heads || r->head_size != c->head_size)
    return fail("%s: the rotary and cache head counts / sizes differ", op);
  // The vector copies also need rot_dim on an 8-element boundary (the k
  // columns past it are copied in 8-element chunks).
  vec = rvec && (fp8 ? fp8_cache_vec(c) : cvec) && r->rot_dim % 8 == 0;
  return 0;
}

}  // namespace

// rotary_embedding_and_cache (fp8: into e4m3fn caches) whose q, k and v are
// views of the rows of C [M, N]: row strides ldc, every head inside the row.
// With part != nullptr, C's rows are first formed from a GEMM's split-K
// partial planes (and bias), in the same launch. check_only: validate only.
int rotary_and_cache_on_rows(const char* op, const dk_rotary_params* r, const dk_cache_write_params* c, int dtype,
                             bool fp8, float k_scale, float v_scale, const float* part, int splits, const void* bias,
                             void* C, int64_t ldc, int M, int N, bool check_only, hipStream_t s) {
  rope_cache::KParams kp;
  bool neox = false, vec = false, empty = false;
  if (const int rc = fused_params(op, r, c, dtype, fp8, kp, neox, vec, empty)) return rc;
  if (fp8) {
    if (const int rc = check_scales(op, k_scale, v_scale)) return rc;
  }
  if (r->num_tokens != M) return fail("%s: one token per GEMM output row expected (%d tokens, %d rows)", op,
                                      static_cast<int>(r->num_tokens), M);
  auto inside = [&](const void* v, int64_t st, int64_t sh, int heads) {
    const auto* b = static_cast<const uint16_t*>(C);
    const auto* x = static_cast<const uint16_t*>(v);
    return st == ldc && x >= b && sh >= 0 && (x - b) + (heads - 1) * sh + r->head_size <= N;
  };
  if (!inside(r->query, r->q_stride_token, r->q_stride_head, r->num_q_heads) ||
      !inside(r->key, r->k_stride_token, r->k_stride_head, r->num_kv_heads) ||
      !inside(c->value, c->v_stride_token, c->v_stride_head, c->num_kv_heads))
    return fail("%s: query, key and value must be views of the GEMM output's rows", op);
  if (check_only || empty) return 0;
  if (part != nullptr && (splits < 1 || splits > rope_cache::kMaxSplits))
    return fail("%s: %d K splits (at most %d)", op, splits, rope_cache::kMaxSplits);
  if (part != nullptr) {
    kp.part = part;
    kp.bias = static_cast<const uint16_t*>(bias);
    kp.C = static_cast<uint16_t*>(C);
    kp.ldc = ldc;
    kp.plane = static_cast<int64_t>(M) * N;
    kp.N = N;
    kp.splits = splits;
    kp.vec_c = (ldc % 4 == 0 && aligned_to(C, 8)) ? 1 : 0;  // gemm_splitk_reduce_kernel's store choice
  }
  return static_cast<int>(fp8 ? rope_cache::launch_any<true>(kp, dtype, r->cache_dtype, neox, vec, k_scale, v_scale, s)
                              : rope_cache::launch_any<false>(kp, dtype, r->cache_dtype, neox, vec, 1.0f, 1.0f, s));
}

}  // namespace dk

extern "C" int dk_rotary_embedding(const dk_rotary_params* a, int dtype, void* stream) {
  using namespace dk;
  clear_error();
  rope::KParams kp;
  bool neox = false, vec = false, empty = false;
  if (const int rc = rotary_params("rotary_embedding", a, dtype, kp, neox, vec, empty)) return rc;
  if (empty) return hipSuccess;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if (a->cache_dtype == DK_FLOAT32) {
    e = dtype == DK_BFLOAT16 ? rope::launch_rotary<Bf16, float>(kp, neox, vec, s)
                             : rope::launch_rotary<F16, float>(kp, neox, vec, s);
  } else {
    e = dtype == DK_BFLOAT16 ? rope::launch_rotary<Bf16, uint16_t>(kp, neox, vec, s)
                             : rope::launch_rotary<F16, uint16_t>(kp, neox, vec, s);
  }
  return static_cast<int>(e);
}

extern "C" int dk_reshape_and_cache(const dk_cache_write_params* a, int dtype, void* stream) {
  using namespace dk;
  clear_error();
  cache::KParams kp;
  bool vec = false, empty = false;
  if (const int rc = cache_params("reshape_and_cache", a, dtype, kp, vec, empty)) return rc;
  if (empty) return hipSuccess;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(a->num_tokens), block(cache::kThreads);
  if (vec) hipLaunchKernelGGL((cache::reshape_and_cache_kernel<8>), grid, block, 0, s, kp);
  else hipLaunchKernelGGL((cache::reshape_and_cache_kernel<1>), grid, block, 0, s, kp);
  return static_cast<int>(hipGetLastError());
}

extern "C" int dk_reshape_and_cache_fp8(const dk_cache_write_params* a, int dtype, float k_scale, float v_scale,
                                        void* stream) {
  using namespace dk;
  clear_error();
  const char* op = "reshape_and_cache_fp8";
  cache::KParams kp;
  bool vec16 = false, empty = false;
  if (const int rc = cache_params(op, a, dtype, kp, vec16, empty)) return rc;
  if (const int rc = check_scales(op, k_scale, v_scale)) return rc;
  if (empty) return hipSuccess;
  const bool vec = fp8_cache_vec(a);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(a->num_tokens), block(cache::kThreads);
  if (dtype == DK_BFLOAT16) {
    if (vec) hipLaunchKernelGGL((cache::reshape_and_cache_fp8_kernel<Bf16, 8>), grid, block, 0, s, kp, k_scale, v_scale);
    else hipLaunchKernelGGL((cache::reshape_and_cache_fp8_kernel<Bf16, 1>), grid, block, 0, s, kp, k_scale, v_scale);
  } else {
    if (vec) hipLaunchKernelGGL((cache::reshape_and_cache_fp8_kernel<F16, 8>), grid, block, 0, s, kp, k_scale, v_scale);
    else hipLaunchKernelGGL((cache::reshape_and_cache_fp8_kernel<F16, 1>), grid, block, 0, s, kp, k_scale, v_scale);
  }
  return static_cast<int>(hipGetLastError());
}

extern "C" int dk_rotary_embedding_and_cache(const dk_rotary_params* r, const dk_cache_write_params* c, int dtype,
                                             void* stream) {
  using namespace dk;
  clear_error();
  rope_cache::KParams kp;
  bool neox = false, vec = false, empty = false;
  if (const int rc = fused_params("rotary_embedding_and_cache", r, c, dtype, false, kp, neox, vec, empty)) return rc;
  if (empty) return hipSuccess;
  return static_cast<int>(rope_cache::launch_any<false>(kp, dtype, r->cache_dtype, neox, vec, 1.0f, 1.0f,
                                                        static_cast<hipStream_t>(stream)));
}

extern "C" int dk_rotary_embedding_and_cache_fp8(const dk_rotary_params* r, const dk_cache_write_params* c, int dtype,
                                                 float k_scale, float v_scale, void* stream) {
  using namespace dk;
  clear_error();
  const char* op = "rotary_embedding_and_cache_fp8";
  rope_cache::KParams kp;
  bool neox = false, vec = false, empty = false;
  if (const int rc = fused_params(op, r, c, dtype, true, kp, neox, vec, empty)) return rc;
  if (const int rc = check_scales(op, k_scale, v_scale)) return rc;
  if (empty) return hipSuccess;
  return static_cast<int>(rope_cache::launch_any<true>(kp, dtype, r->cache_dtype, neox, vec, k_scale, v_scale,
                                                       static_cast<hipStream_t>(stream)));
}
