// Device-side building blocks shared by every decode kernel (gfx950 only).
//
// * Element types are the compiler's native 16-bit floats (`__bf16`,
//   `_Float16`); memory is always moved as raw 16-bit words and converted in
//   registers, so one kernel template serves both model dtypes.
// * Conversions to the model dtype round to nearest even, like the reference
//   (`csrc/common.cuh:23,29` of DecodeKernels).
// * Reductions are written for 64-lane wavefronts: a full wave reduction is
//   six butterfly steps, and a block reduction needs one LDS slot per wave.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace dk {

constexpr int kWave = 64;

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// 16-bit element types
// ---------------------------------------------------------------------------
struct Bf16 {
  using mfma_vec = bf16x8;
  using vec2 = bf16x2;
  static __device__ __forceinline__ float lo(uint32_t w) { return __uint_as_float(w << 16); }
  static __device__ __forceinline__ float hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
  static __device__ __forceinline__ float to_float(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }
  static __device__ __forceinline__ uint16_t from_float(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
  }
  // 8 elements (one 16-byte fragment) times an 8-element fragment, fp32 accumulate.
  static __device__ __forceinline__ f32x4 mfma_16x16x32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
  // 4 elements x 4 elements: lane l holds A[l%16][4*(l/16)+e] and B[4*(l/16)+e][l%16].
  static __device__ __forceinline__ f32x4 mfma_16x16x16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c, 0,
                                                     0, 0);
  }
  static constexpr uint16_t kOne = 0x3F80;
};

struct F16 {
  using mfma_vec = f16x8;
  using vec2 = f16x2;
  static __device__ __forceinline__ float lo(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xffffu)));
  }
  static __device__ __forceinline__ float hi(uint32_t w) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
  }
  static __device__ __forceinline__ float to_float(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
  }
  static __device__ __forceinline__ uint16_t from_float(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
  static __device__ __forceinline__ f32x4 mfma_16x16x32(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
  static __device__ __forceinline__ f32x4 mfma_16x16x16(u32x2 a, u32x2 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0, 0,
                                                 0);
  }
  static constexpr uint16_t kOne = 0x3C00;
};

// (a, b) rounded to nearest even into one word, a in the low half: one
// two-source v_cvt_pk_{bf16,f16}_f32, the same rounding as from_float on
// each (converting the halves one by one costs a shift and an or on top).
template <typename E>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, typename E::vec2));
}

// ---------------------------------------------------------------------------
// Loads of 8 consecutive 16-bit elements with the alignment the caller can
// guarantee (16, 8 or 4 bytes); the wider forms become single dwordx4/x2 loads.
// ---------------------------------------------------------------------------
template <int ALIGN>
__device__ __forceinline__ u32x4 load8(const uint16_t* p) {
  if constexpr (ALIGN >= 16) {
    return *reinterpret_cast<const u32x4*>(p);
  } else if constexpr (ALIGN == 8) {
    const u32x2 a = reinterpret_cast<const u32x2*>(p)[0];
    const u32x2 b = reinterpret_cast<const u32x2*>(p)[1];
    return u32x4{a[0], a[1], b[0], b[1]};
  } else {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(p);
    return u32x4{w[0], w[1], w[2], w[3]};
  }
}

template <int ALIGN>
__device__ __forceinline__ u32x2 load4(const uint16_t* p) {
  if constexpr (ALIGN >= 8) {
    return *reinterpret_cast<const u32x2*>(p);
  } else {
    const uint32_t* w = reinterpret_cast<const uint32_t*>(p);
    return u32x2{w[0], w[1]};
  }
}

// A per-lane value the compiler must treat as produced here (an empty volatile
// asm on a VGPR): comparisons against it are made where they are written
// instead of being hoisted out of a loop, whose 64-bit lane masks would
// otherwise stay live in scalar registers across it. Costs nothing.
__device__ __forceinline__ int fresh_vgpr(int v) {
  __asm__ volatile("" : "+v"(v));
  return v;
}

// ---------------------------------------------------------------------------
// Wave and block reductions (64 lanes).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// v combined over lanes l, l ^ 16, l ^ 32, l ^ 48 (the four 16-lane rows),
// without an LDS round trip: gfx950's v_permlane16_swap / v_permlane32_swap
// hand each lane its own value and its partner's (lane l ^ 16, then l ^ 32).
// The sum is (v[l] + v[l^16]) + (v[l^32] + v[l^48]) for every lane, the same
// association as two xor-shuffles by 16 and 32.
__device__ __forceinline__ float rows_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float rows_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Sum over the whole workgroup; `slots` holds one float per wave. Every
// thread gets the total. Safe to call repeatedly with the same slots.
__device__ __forceinline__ float block_sum(float v, float* slots) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int waves = (blockDim.x + kWave - 1) / kWave;
  v = wave_sum(v);
  __syncthreads();  // previous users of `slots` are done
  if (lane == 0) slots[wave] = v;
  __syncthreads();
  float t = 0.0f;
  for (int w = 0; w < waves; ++w) t += slots[w];
  return t;
}

__device__ __forceinline__ float block_max(float v, float* slots) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int waves = (blockDim.x + kWave - 1) / kWave;
  v = wave_max(v);
  __syncthreads();
  if (lane == 0) slots[wave] = v;
  __syncthreads();
  float t = -__builtin_huge_valf();
  for (int w = 0; w < waves; ++w) t = fmaxf(t, slots[w]);
  return t;
}

}  // namespace dk
