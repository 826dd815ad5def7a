// Host-side helpers shared by the C-ABI entry points: argument-error
// reporting and small integer utilities.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>

namespace dk {

// Records a description of an argument error for dk_last_error() and returns
// hipErrorInvalidValue, so a validation branch reads `return fail("...")`.
int fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
// Clears the thread's last error message.
void clear_error();

inline int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool aligned_to(const void* p, int bytes) {
  return (reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(bytes)) == 0;
}

// Consumers of a GEMM's split-K partial tiles (fp32 planes [splits][rows][N],
// no bias), used by the fused entry points (norm_act.hip, rope_cache.hip):

// Whether fused_add_rms_norm takes its 16-byte vector path for these rows
// (the split-K form exists only for that path).
bool fused_add_rms_norm_vectorizable(int H, int64_t in_stride, int64_t res_stride, const void* input,
                                     const void* residual, const void* weight);
// fused_add_rms_norm on x = round(sum of the partial planes in split order +
// bias), bit for bit the reduce into `out` followed by fused_add_rms_norm.
int launch_splitk_fused_add_rms_norm(int dtype, const float* part, int splits, const void* bias, void* out,
                                     int64_t out_stride, void* residual, int64_t res_stride, const void* weight,
                                     int rows, int H, float eps, hipStream_t s);
}  // namespace dk

struct dk_rotary_params;
struct dk_cache_write_params;

namespace dk {
// rotary_embedding_and_cache (fp8: into e4m3fn caches) on q / k / v views of
// the rows of C [M, N] (row stride ldc); with part != nullptr C's rows are
// first formed from the partial planes, bit for bit as the GEMM's reduce
// writes them. check_only validates the arguments without launching.
int rotary_and_cache_on_rows(const char* op, const dk_rotary_params* r, const dk_cache_write_params* c, int dtype,
                             bool fp8, float k_scale, float v_scale, const float* part, int splits, const void* bias,
                             void* C, int64_t ldc, int M, int N, bool check_only, hipStream_t s);

namespace attn {
// Device address of the current device's DK_NOALLOC_SCRATCH_BYTES-byte
// workspace of the allocation-free attention entry point (noalloc_scratch.hip);
// nullptr with *err set on failure.
void* noalloc_scratch_address(int* err);
}  // namespace attn

}  // namespace dk
