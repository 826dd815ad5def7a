// Bandwidth-bound decoder-layer ops for gfx950, with vLLM / DecodeKernels
// semantics (reference: csrc/norm_act.cuh:1-200, decode_kernels/reference.py:89-104):
//
//   rms_norm(out, x, w, eps):           out = round(x * inv_rms * w)
//   fused_add_rms_norm(x, res, w, eps): res = round(x + res); x = round(res * inv_rms * w)
//   silu_and_mul(out, x):               out = round(silu(x[:, :d]) * x[:, d:])
//
// All arithmetic is fp32; rounding to the model dtype is to nearest even. The
// sum of squares of fused_add_rms_norm is taken over the *rounded* residual.
// inv_rms = 1 / sqrt(mean + eps) with a correctly rounded square root and
// division, which is how torch's CPU rsqrt evaluates it.
//
// Layout on CDNA4: one workgroup per row for the norms, with the row held in
// registers between the reduction and the write (each element of x, residual
// and weight is read from HBM exactly once). A row of H elements is split
// into 16-byte vectors, NV per thread; NV is a template parameter so the
// vectors stay in VGPRs. silu_and_mul has no reduction, so it runs a 2-D grid
// (row, 2048-column chunk) of 16-byte vector lanes for more parallelism than
// one workgroup per row. Rows that are not 16-byte vectorisable take a scalar
// path that re-reads the row.
#include <cmath>

#include "../../include/decodekernels_amd.h"
#include "dk_device.h"
#include "dk_host.h"

namespace dk {
namespace normact {

constexpr int kVec = 8;  // 16-bit elements per 16-byte vector

#ifndef DK_SILU_NT_LOADS
// silu_and_mul's gate / up loads with the non-temporal bit: 12-14% faster at
// 16384 tokens, 4% at 4096, the same at decode sizes. The norms' row loads
// measured 3-5% slower with it at 4096-16384 rows and keep the default policy.
#define DK_SILU_NT_LOADS 1
#endif

__device__ __forceinline__ float inv_rms(float ss, int H, float eps) {
  return 1.0f / __fsqrt_rn(ss / static_cast<float>(H) + eps);
}

template <typename E>
__device__ __forceinline__ float sumsq8(u32x4 v, float ss) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float a = E::lo(v[e]);
    const float b = E::hi(v[e]);
    ss = fmaf(a, a, ss);
    ss = fmaf(b, b, ss);
  }
  return ss;
}

template <typename E>
__device__ __forceinline__ u32x4 scale8(u32x4 x, u32x4 w, float inv) {
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = pack2<E>(E::lo(x[e]) * inv * E::lo(w[e]), E::hi(x[e]) * inv * E::hi(w[e]));
  return o;
}

// ---------------------------------------------------------------------------
// rms_norm
// ---------------------------------------------------------------------------
template <typename E, int NV>
__global__ __launch_bounds__(1024) void rms_norm_vec_kernel(uint16_t* __restrict__ out, const uint16_t* __restrict__ in,
                                                            const uint16_t* __restrict__ weight, int H,
                                                            int64_t in_stride, int64_t out_stride, float eps) {
  __shared__ float slots[1024 / kWave];
  const u32x4* x = reinterpret_cast<const u32x4*>(in + blockIdx.x * in_stride);
  u32x4* y = reinterpret_cast<u32x4*>(out + blockIdx.x * out_stride);
  const u32x4* w = reinterpret_cast<const u32x4*>(weight);
  const int nvec = H / kVec;
  u32x4 xv[NV];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int i = threadIdx.x + j * blockDim.x;
    xv[j] = i < nvec ? x[i] : u32x4{0u, 0u, 0u, 0u};
    ss = sumsq8<E>(xv[j], ss);
  }
  const float inv = inv_rms(block_sum(ss, slots), H, eps);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int i = threadIdx.x + j * blockDim.x;
    if (i < nvec) y[i] = scale8<E>(xv[j], w[i], inv);
  }
}

template <typename E>
__global__ __launch_bounds__(1024) void rms_norm_scalar_kernel(uint16_t* __restrict__ out,
                                                               const uint16_t* __restrict__ in,
                                                               const uint16_t* __restrict__ weight, int H,
                                                               int64_t in_stride, int64_t out_stride, float eps) {
  __shared__ float slots[1024 / kWave];
  const uint16_t* x = in + blockIdx.x * in_stride;
  uint16_t* y = out + blockIdx.x * out_stride;
  float ss = 0.0f;
  for (int i = threadIdx.x; i < H; i += blockDim.x) {
    const float f = E::to_float(x[i]);
    ss = fmaf(f, f, ss);
  }
  const float inv = inv_rms(block_sum(ss, slots), H, eps);
  for (int i = threadIdx.x; i < H; i += blockDim.x) y[i] = E::from_float(E::to_float(x[i]) * inv * E::to_float(weight[i]));
}

// ---------------------------------------------------------------------------
// fused_add_rms_norm
// ---------------------------------------------------------------------------
// One row of fused_add_rms_norm: x vector i comes from load_x(i), the
// normalised row goes to y. Thread t takes vectors t, t + blockDim.x, ...; the
// sum of squares follows that mapping, so every caller with the same block
// size gets the same bits.
template <typename E, int NV, typename LoadX>
__device__ __forceinline__ void add_rms_norm_row(u32x4* __restrict__ y, u32x4* __restrict__ r,
                                                 const u32x4* __restrict__ w, int H, float eps, float* slots,
                                                 LoadX load_x) {
  const int nvec = H / kVec;
  u32x4 rv[NV];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int i = threadIdx.x + j * blockDim.x;
    u32x4 s = {0u, 0u, 0u, 0u};
    if (i < nvec) {
      const u32x4 a = load_x(i);
      const u32x4 b = r[i];
#pragma unroll
      for (int e = 0; e < 4; ++e) s[e] = pack2<E>(E::lo(a[e]) + E::lo(b[e]), E::hi(a[e]) + E::hi(b[e]));
      r[i] = s;
    }
    rv[j] = s;
    ss = sumsq8<E>(s, ss);
  }
  const float inv = inv_rms(block_sum(ss, slots), H, eps);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int i = threadIdx.x + j * blockDim.x;
    if (i < nvec) y[i] = scale8<E>(rv[j], w[i], inv);
  }
}

template <typename E, int NV>
__global__ __launch_bounds__(1024) void fused_add_rms_norm_vec_kernel(uint16_t* __restrict__ input,
                                                                      uint16_t* __restrict__ residual,
                                                                      const uint16_t* __restrict__ weight, int H,
                                                                      int64_t in_stride, int64_t res_stride,
                                                                      float eps) {
  __shared__ float slots[1024 / kWave];
  u32x4* x = reinterpret_cast<u32x4*>(input + blockIdx.x * in_stride);
  u32x4* r = reinterpret_cast<u32x4*>(residual + blockIdx.x * res_stride);
  add_rms_norm_row<E, NV>(x, r, reinterpret_cast<const u32x4*>(weight), H, eps, slots,
                          [&](int i) { return x[i]; });
}

// fused_add_rms_norm whose input rows are a GEMM's split-K partial tiles:
// x = round(sum of the `splits` fp32 planes [splits][rows][H] in split order,
// starting from 0, plus the bias or 0), exactly as gemm_splitk_reduce_kernel
// rounds them into C, then the residual add and the norm as
// fused_add_rms_norm_vec_kernel. The result equals gemm_tn (split) followed by
// fused_add_rms_norm bit for bit; x itself is never stored, only the
// normalised row (into `out`) and the new residual. S > 0: a compile-time
// split count (all partial loads issued together); S = 0: `splits` at run time.
template <typename E, int NV, int S>
__global__ __launch_bounds__(1024) void splitk_add_rms_norm_kernel(uint16_t* __restrict__ out,
                                                                   uint16_t* __restrict__ residual,
                                                                   const uint16_t* __restrict__ weight, int H,
                                                                   int64_t out_stride, int64_t res_stride, float eps,
                                                                   const float* __restrict__ part, int splits,
                                                                   int64_t plane, const uint16_t* __restrict__ bias) {
  __shared__ float slots[1024 / kWave];
  u32x4* y = reinterpret_cast<u32x4*>(out + blockIdx.x * out_stride);
  u32x4* r = reinterpret_cast<u32x4*>(residual + blockIdx.x * res_stride);
  const float* prow = part + static_cast<int64_t>(blockIdx.x) * H;
  auto load_x = [&](int i) {
    const float* p = prow + kVec * i;
    float v[kVec];
#pragma unroll
    for (int e = 0; e < kVec; ++e) v[e] = 0.0f;
    if constexpr (S > 0) {
      f32x4 lo[S], hi[S];
#pragma unroll
      for (int sp = 0; sp < S; ++sp) {
        lo[sp] = *reinterpret_cast<const f32x4*>(p + sp * plane);
        hi[sp] = *reinterpret_cast<const f32x4*>(p + sp * plane + 4);
      }
#pragma unroll
      for (int sp = 0; sp < S; ++sp)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += lo[sp][e], v[4 + e] += hi[sp][e];
    } else {
      for (int sp = 0; sp < splits; ++sp) {
        const f32x4 lo = *reinterpret_cast<const f32x4*>(p + sp * plane);
        const f32x4 hi = *reinterpret_cast<const f32x4*>(p + sp * plane + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += lo[e], v[4 + e] += hi[e];
      }
    }
#pragma unroll
    for (int e = 0; e < kVec; ++e) v[e] += bias != nullptr ? E::to_float(bias[kVec * i + e]) : 0.0f;
    u32x4 a;
#pragma unroll
    for (int e = 0; e < 4; ++e) a[e] = pack2<E>(v[2 * e], v[2 * e + 1]);
    return a;
  };
  add_rms_norm_row<E, NV>(y, r, reinterpret_cast<const u32x4*>(weight), H, eps, slots, load_x);
}

template <typename E>
__global__ __launch_bounds__(1024) void fused_add_rms_norm_scalar_kernel(uint16_t* __restrict__ input,
                                                                         uint16_t* __restrict__ residual,
                                                                         const uint16_t* __restrict__ weight, int H,
                                                                         int64_t in_stride, int64_t res_stride,
                                                                         float eps) {
  __shared__ float slots[1024 / kWave];
  uint16_t* x = input + blockIdx.x * in_stride;
  uint16_t* r = residual + blockIdx.x * res_stride;
  float ss = 0.0f;
  for (int i = threadIdx.x; i < H; i += blockDim.x) {
    const uint16_t z = E::from_float(E::to_float(x[i]) + E::to_float(r[i]));
    r[i] = z;
    const float f = E::to_float(z);
    ss = fmaf(f, f, ss);
  }
  const float inv = inv_rms(block_sum(ss, slots), H, eps);
  // Each thread re-reads only the residual elements it wrote itself.
  for (int i = threadIdx.x; i < H; i += blockDim.x) x[i] = E::from_float(E::to_float(r[i]) * inv * E::to_float(weight[i]));
}

// ---------------------------------------------------------------------------
// silu_and_mul
// ---------------------------------------------------------------------------
__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

constexpr int kSiluThreads = 256;

template <typename E>
__global__ __launch_bounds__(kSiluThreads) void silu_and_mul_vec_kernel(uint16_t* __restrict__ out,
                                                                        const uint16_t* __restrict__ in, int d,
                                                                        int64_t in_stride, int64_t out_stride) {
  const int i = blockIdx.y * kSiluThreads + threadIdx.x;  // vector index in the row
  if (i >= d / kVec) return;
  const uint16_t* row = in + blockIdx.x * in_stride;
  const u32x4* gp = reinterpret_cast<const u32x4*>(row) + i;
  const u32x4* up = reinterpret_cast<const u32x4*>(row + d) + i;
  const u32x4 g = DK_SILU_NT_LOADS ? __builtin_nontemporal_load(gp) : *gp;
  const u32x4 u = DK_SILU_NT_LOADS ? __builtin_nontemporal_load(up) : *up;
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = pack2<E>(silu(E::lo(g[e])) * E::lo(u[e]), silu(E::hi(g[e])) * E::hi(u[e]));
  reinterpret_cast<u32x4*>(out + blockIdx.x * out_stride)[i] = o;
}

template <typename E>
__global__ __launch_bounds__(kSiluThreads) void silu_and_mul_scalar_kernel(uint16_t* __restrict__ out,
                                                                           const uint16_t* __restrict__ in, int d,
                                                                           int64_t in_stride, int64_t out_stride) {
  const int i = blockIdx.y * kSiluThreads + threadIdx.x;
  if (i >= d) return;
  const uint16_t* row = in + blockIdx.x * in_stride;
  out[blockIdx.x * out_stride + i] = E::from_float(silu(E::to_float(row[i])) * E::to_float(row[d + i]));
}

// ---------------------------------------------------------------------------
// Host-side shape selection
// ---------------------------------------------------------------------------
struct RowShape {
  int threads;
  int nv;  // vectors per thread (1, 2, 4, 8); 0 = scalar path
};

// Vector path: about 256 threads per row, each holding NV 16-byte vectors.
RowShape row_shape(int H, bool vec) {
  if (vec) {
    const int nvec = H / kVec;
    for (int nv : {1, 2, 4, 8}) {
      const int t = static_cast<int>(ceil_div64(nvec, nv));
      if (t <= 256 || (nv == 8 && t <= 1024)) {
        const int threads = static_cast<int>(ceil_div64(t, kWave) * kWave);
        return {threads < kWave ? kWave : threads, nv};
      }
    }
  }
  int threads = static_cast<int>(ceil_div64(H, kWave) * kWave);
  threads = threads < kWave ? kWave : (threads > 1024 ? 1024 : threads);
  return {threads, 0};
}

template <typename E>
hipError_t launch_rms_norm(uint16_t* out, const uint16_t* in, const uint16_t* w, int rows, int H, int64_t is,
                           int64_t os, float eps, bool vec, hipStream_t s) {
  const RowShape rs = row_shape(H, vec);
  const dim3 grid(rows), block(rs.threads);
  switch (rs.nv) {
    case 1: hipLaunchKernelGGL((rms_norm_vec_kernel<E, 1>), grid, block, 0, s, out, in, w, H, is, os, eps); break;
    case 2: hipLaunchKernelGGL((rms_norm_vec_kernel<E, 2>), grid, block, 0, s, out, in, w, H, is, os, eps); break;
    case 4: hipLaunchKernelGGL((rms_norm_vec_kernel<E, 4>), grid, block, 0, s, out, in, w, H, is, os, eps); break;
    case 8: hipLaunchKernelGGL((rms_norm_vec_kernel<E, 8>), grid, block, 0, s, out, in, w, H, is, os, eps); break;
    default: hipLaunchKernelGGL((rms_norm_scalar_kernel<E>), grid, block, 0, s, out, in, w, H, is, os, eps); break;
  }
  return hipGetLastError();
}

template <typename E>
hipError_t launch_fused_add(uint16_t* x, uint16_t* r, const uint16_t* w, int rows, int H, int64_t is, int64_t rs_,
                            float eps, bool vec, hipStream_t s) {
  const RowShape rs = row_shape(H, vec);
  const dim3 grid(rows), block(rs.threads);
  switch (rs.nv) {
    case 1: hipLaunchKernelGGL((fused_add_rms_norm_vec_kernel<E, 1>), grid, block, 0, s, x, r, w, H, is, rs_, eps); break;
    case 2: hipLaunchKernelGGL((fused_add_rms_norm_vec_kernel<E, 2>), grid, block, 0, s, x, r, w, H, is, rs_, eps); break;
    case 4: hipLaunchKernelGGL((fused_add_rms_norm_vec_kernel<E, 4>), grid, block, 0, s, x, r, w, H, is, rs_, eps); break;
    case 8: hipLaunchKernelGGL((fused_add_rms_norm_vec_kernel<E, 8>), grid, block, 0, s, x, r, w, H, is, rs_, eps); break;
    default: hipLaunchKernelGGL((fused_add_rms_norm_scalar_kernel<E>), grid, block, 0, s, x, r, w, H, is, rs_, eps); break;
  }
  return hipGetLastError();
}

template <typename E, int NV>
void launch_splitk_add_nv(uint16_t* out, uint16_t* r, const uint16_t* w, int rows, int H, int64_t os, int64_t rs_,
                          float eps, const float* part, int splits, const uint16_t* bias, dim3 block, hipStream_t s) {
  const int64_t plane = static_cast<int64_t>(rows) * H;
#define DK_SPLIT_CASE(S_)                                                                                     \
  case S_:                                                                                                    \
    hipLaunchKernelGGL((splitk_add_rms_norm_kernel<E, NV, S_>), dim3(rows), block, 0, s, out, r, w, H, os, rs_, \
                       eps, part, splits, plane, bias);                                                       \
    return;
  switch (splits) {
    DK_SPLIT_CASE(2)
    DK_SPLIT_CASE(4)
    DK_SPLIT_CASE(8)
    default:
      hipLaunchKernelGGL((splitk_add_rms_norm_kernel<E, NV, 0>), dim3(rows), block, 0, s, out, r, w, H, os, rs_, eps,
                         part, splits, plane, bias);
  }
#undef DK_SPLIT_CASE
}

template <typename E>
hipError_t launch_splitk_add(uint16_t* out, uint16_t* r, const uint16_t* w, int rows, int H, int64_t os, int64_t rs_,
                             float eps, const float* part, int splits, const uint16_t* bias, hipStream_t s) {
  const RowShape rs = row_shape(H, true);
  const dim3 block(rs.threads);
  switch (rs.nv) {
    case 1: launch_splitk_add_nv<E, 1>(out, r, w, rows, H, os, rs_, eps, part, splits, bias, block, s); break;
    case 2: launch_splitk_add_nv<E, 2>(out, r, w, rows, H, os, rs_, eps, part, splits, bias, block, s); break;
    case 4: launch_splitk_add_nv<E, 4>(out, r, w, rows, H, os, rs_, eps, part, splits, bias, block, s); break;
    case 8: launch_splitk_add_nv<E, 8>(out, r, w, rows, H, os, rs_, eps, part, splits, bias, block, s); break;
    default: return hipErrorInvalidValue;  // the caller checked the vector path applies
  }
  return hipGetLastError();
}

template <typename E>
hipError_t launch_silu(uint16_t* out, const uint16_t* in, int rows, int d, int64_t is, int64_t os, bool vec,
                       hipStream_t s) {
  const int per_row = vec ? d / kVec : d;
  const dim3 grid(rows, static_cast<unsigned>(ceil_div64(per_row, kSiluThreads)));
  if (vec) {
    hipLaunchKernelGGL((silu_and_mul_vec_kernel<E>), grid, dim3(kSiluThreads), 0, s, out, in, d, is, os);
  } else {
    hipLaunchKernelGGL((silu_and_mul_scalar_kernel<E>), grid, dim3(kSiluThreads), 0, s, out, in, d, is, os);
  }
  return hipGetLastError();
}

bool dtype_ok(int dtype) { return dtype == DK_FLOAT16 || dtype == DK_BFLOAT16; }

}  // namespace normact
}  // namespace dk

using namespace dk;
using namespace dk::normact;

extern "C" int dk_rms_norm(int dtype, void* out, const void* input, const void* weight, int rows, int H,
                           int64_t in_stride, int64_t out_stride, float eps, void* stream) {
  clear_error();
  if (!dtype_ok(dtype)) return fail("rms_norm: expected float16 or bfloat16, got dtype code %d", dtype);
  if (rows < 0 || H < 0) return fail("rms_norm: rows and H must be non-negative");
  if (rows == 0 || H == 0) return hipSuccess;
  if (out == nullptr || input == nullptr || weight == nullptr) return fail("rms_norm: pointers must not be NULL");
  // Rows read may repeat (stride 0 broadcasts one row); rows written may not overlap.
  if (in_stride < 0 || (rows > 1 && out_stride < H))
    return fail("rms_norm: strides must be non-negative and out_stride >= H (written rows must not overlap)");
  const bool vec = H % kVec == 0 && in_stride % kVec == 0 && out_stride % kVec == 0 && aligned_to(input, 16) &&
                   aligned_to(out, 16) && aligned_to(weight, 16);
  auto* o = static_cast<uint16_t*>(out);
  auto* x = static_cast<const uint16_t*>(input);
  auto* w = static_cast<const uint16_t*>(weight);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return static_cast<int>(dtype == DK_BFLOAT16 ? launch_rms_norm<Bf16>(o, x, w, rows, H, in_stride, out_stride, eps, vec, s)
                                               : launch_rms_norm<F16>(o, x, w, rows, H, in_stride, out_stride, eps, vec, s));
}

extern "C" int dk_fused_add_rms_norm(int dtype, void* input, void* residual, const void* weight, int rows, int H,
                                     int64_t in_stride, int64_t res_stride, float eps, void* stream) {
  clear_error();
  if (!dtype_ok(dtype)) return fail("fused_add_rms_norm: expected float16 or bfloat16, got dtype code %d", dtype);
  if (rows < 0 || H < 0) return fail("fused_add_rms_norm: rows and H must be non-negative");
  if (rows == 0 || H == 0) return hipSuccess;
  if (input == nullptr || residual == nullptr || weight == nullptr)
    return fail("fused_add_rms_norm: pointers must not be NULL");
  if (rows > 1 && (in_stride < H || res_stride < H))
    return fail("fused_add_rms_norm: in_stride and res_stride must be >= H (both are written; rows must not overlap)");
  const bool vec = H % kVec == 0 && in_stride % kVec == 0 && res_stride % kVec == 0 && aligned_to(input, 16) &&
                   aligned_to(residual, 16) && aligned_to(weight, 16);
  auto* x = static_cast<uint16_t*>(input);
  auto* r = static_cast<uint16_t*>(residual);
  auto* w = static_cast<const uint16_t*>(weight);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return static_cast<int>(dtype == DK_BFLOAT16 ? launch_fused_add<Bf16>(x, r, w, rows, H, in_stride, res_stride, eps, vec, s)
                                               : launch_fused_add<F16>(x, r, w, rows, H, in_stride, res_stride, eps, vec, s));
}

namespace dk {

bool fused_add_rms_norm_vectorizable(int H, int64_t in_stride, int64_t res_stride, const void* input,
                                     const void* residual, const void* weight) {
  return H % normact::kVec == 0 && in_stride % normact::kVec == 0 && res_stride % normact::kVec == 0 &&
         aligned_to(input, 16) && aligned_to(residual, 16) && aligned_to(weight, 16) &&
         normact::row_shape(H, true).nv > 0;
}

int launch_splitk_fused_add_rms_norm(int dtype, const float* part, int splits, const void* bias, void* out,
                                     int64_t out_stride, void* residual, int64_t res_stride, const void* weight,
                                     int rows, int H, float eps, hipStream_t s) {
  auto* o = static_cast<uint16_t*>(out);
  auto* r = static_cast<uint16_t*>(residual);
  auto* w = static_cast<const uint16_t*>(weight);
  auto* b = static_cast<const uint16_t*>(bias);
  return static_cast<int>(dtype == DK_BFLOAT16
                              ? launch_splitk_add<Bf16>(o, r, w, rows, H, out_stride, res_stride, eps, part, splits, b, s)
                              : launch_splitk_add<F16>(o, r, w, rows, H, out_stride, res_stride, eps, part, splits, b, s));
}

}  // namespace dk

extern "C" int dk_silu_and_mul(int dtype, void* out, const void* input, int rows, int d, int64_t in_stride,
                               int64_t out_stride, void* stream) {
  clear_error();
  if (!dtype_ok(dtype)) return fail("silu_and_mul: expected float16 or bfloat16, got dtype code %d", dtype);
  if (rows < 0 || d < 0) return fail("silu_and_mul: rows and d must be non-negative");
  if (rows == 0 || d == 0) return hipSuccess;
  if (out == nullptr || input == nullptr) return fail("silu_and_mul: pointers must not be NULL");
  if (in_stride < 0 || (rows > 1 && out_stride < d))
    return fail("silu_and_mul: strides must be non-negative and out_stride >= d (written rows must not overlap)");
  if (ceil_div64(d, kSiluThreads) > 65535) return fail("silu_and_mul: d is too large");
  const bool vec =
      d % kVec == 0 && in_stride % kVec == 0 && out_stride % kVec == 0 && aligned_to(input, 16) && aligned_to(out, 16);
  auto* o = static_cast<uint16_t*>(out);
  auto* x = static_cast<const uint16_t*>(input);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return static_cast<int>(dtype == DK_BFLOAT16 ? launch_silu<Bf16>(o, x, rows, d, in_stride, out_stride, vec, s)
                                               : launch_silu<F16>(o, x, rows, d, in_stride, out_stride, vec, s));
}
