// PyTorch binding of the decode kernels: `torch.ops.decode_kernels.*`.
//
// The five schemas, the dispatch key (CUDA, which is where PyTorch-ROCm puts
// HIP tensors) and the argument-check messages are DecodeKernels' interface
// (csrc/ops.cu:44-286), kept identical so callers and tests written against
// the reference see the same ops and the same errors. Two more ops,
// rotary_embedding and reshape_and_cache, cover the steps around attention
// that the reference leaves to vLLM, with vLLM's schemas. Each impl checks tensor
// metadata, fills the C-ABI arguments and enqueues the HIP kernels on the
// current stream of the input's device. One op allocates, unlike the
// reference's (csrc/ops.cu:149-182, which allocates nothing): gemm_tn takes
// its split-K workspace (splits * M * N fp32, at most 8.4 MB at the
// Llama-3-8B decode projections) from PyTorch's caching allocator on the shapes
// whose plan splits K. That allocation is stream-ordered and served from the
// graph's private pool under capture, so every op can be captured in a graph;
// callers that must not allocate at all use the C ABI's dk_gemm_tn_ws with a
// workspace of their own (or dk_gemm_tn, which runs those shapes unsplit).
//
// Importing the Python module `decodekernels_amd._C` (this library) runs the
// static op registration.
#include <Python.h>

#include <ATen/ATen.h>
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <torch/library.h>

#include <algorithm>
#include <optional>
#include <string>
#include <tuple>
#include <utility>

#include "decodekernels_amd.h"

namespace {

int dtype_code(at::ScalarType t, const char* name) {
  if (t == at::ScalarType::Half) return DK_FLOAT16;
  if (t == at::ScalarType::BFloat16) return DK_BFLOAT16;
  TORCH_CHECK(false, name, ": expected float16 or bfloat16, got ", t);
}

void check_status(int err, const char* name) {
  if (err == 0) return;
  const char* detail = dk_last_error();
  TORCH_CHECK(false, name, " failed: ", dk_error_string(err), (detail[0] != '\0' ? " (" : ""), detail,
              (detail[0] != '\0' ? ")" : ""));
}

void check_same(const at::Tensor& a, const at::Tensor& b, const char* what) {
  TORCH_CHECK(a.scalar_type() == b.scalar_type(), what, ": dtype mismatch (", a.scalar_type(), " vs ",
              b.scalar_type(), ")");
  TORCH_CHECK(a.device() == b.device(), what, ": tensors must be on the same device");
}

// PyTorch-ROCm reports HIP devices as DeviceType::CUDA, so its "masquerading"
// guard and stream accessors are the ones that accept these tensors.
using DeviceGuard = c10::hip::OptionalHIPGuardMasqueradingAsCUDA;

void* stream_of(const at::Tensor& t) {
  return static_cast<void*>(c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream());
}

bool aligned(const void* p, int64_t bytes) { return reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(bytes) == 0; }

// Row stride of a [..., H] tensor whose leading dims collapse into one
// uniformly strided row index (csrc/ops.cu:189-197).
int64_t row_stride(const at::Tensor& t, const char* name) {
  TORCH_CHECK(t.stride(-1) == 1, name, ": last dimension must be contiguous");
  if (t.dim() == 1) return t.size(0);
  for (int64_t d = 1; d + 1 < t.dim(); ++d) {
    TORCH_CHECK(t.stride(d - 1) == t.stride(d) * t.size(d), name, ": leading dimensions must be collapsible");
  }
  return t.stride(-2);
}

}  // namespace

// ---------------------------------------------------------------------------
// paged_attention_decode (csrc/ops.cu:44-144)
// ---------------------------------------------------------------------------
namespace {

// Shared by the 16-bit-cache op (the reference's) and the fp8-cache op.
void attention_impl(at::Tensor& out, const at::Tensor& q, const at::Tensor& k_cache, const at::Tensor& v_cache,
                    const at::Tensor& block_tables, const at::Tensor& seq_lens, double scale, int64_t max_seq_len,
                    at::Tensor& tmp_out, at::Tensor& max_logits, at::Tensor& exp_sums, bool fp8, double k_scale,
                    double v_scale) {
  TORCH_CHECK(q.is_cuda(), "paged_attention_decode: q must be a CUDA tensor");
  TORCH_CHECK(q.dim() == 3 && out.dim() == 3, "q and out must be [num_seqs, num_q_heads, head_dim]");
  TORCH_CHECK(k_cache.dim() == 4 && v_cache.dim() == 4,
              "k_cache and v_cache must be [num_blocks, block_size, num_kv_heads, head_dim]");
  check_same(q, out, "q/out");
  if (fp8) {
    TORCH_CHECK(k_cache.scalar_type() == at::ScalarType::Float8_e4m3fn &&
                    v_cache.scalar_type() == at::ScalarType::Float8_e4m3fn,
                "paged_attention_decode_fp8: k_cache and v_cache must be float8_e4m3fn");
    TORCH_CHECK(k_cache.device() == q.device() && v_cache.device() == q.device(),
                "paged_attention_decode_fp8: tensors must be on the same device");
  } else {
    check_same(q, k_cache, "q/k_cache");
    check_same(q, v_cache, "q/v_cache");
  }
  TORCH_CHECK(out.sizes() == q.sizes(), "out must have the same shape as q");
  TORCH_CHECK(k_cache.sizes() == v_cache.sizes(), "k_cache and v_cache shapes differ");

  const int64_t num_seqs = q.size(0);
  const int64_t num_q_heads = q.size(1);
  const int64_t head_dim = q.size(2);
  const int64_t num_kv_heads = k_cache.size(2);
  TORCH_CHECK(k_cache.size(3) == head_dim, "cache head_dim does not match q");
  TORCH_CHECK(head_dim == 64 || head_dim == 96 || head_dim == 128 || head_dim == 192 || head_dim == 256,
              "head_dim must be 64, 96, 128, 192 or 256, got ", head_dim);
  TORCH_CHECK(num_kv_heads > 0 && num_q_heads % num_kv_heads == 0, "num_q_heads must be a multiple of num_kv_heads");
  TORCH_CHECK(num_q_heads / num_kv_heads <= DK_MAX_GQA_GROUP, "GQA group size above ", DK_MAX_GQA_GROUP,
              " is not supported");
  TORCH_CHECK(q.stride(2) == 1 && out.stride(2) == 1 && k_cache.stride(3) == 1 && v_cache.stride(3) == 1,
              "head_dim must be the contiguous (innermost) dimension");
  if (fp8) {
    for (int d = 0; d < 3; ++d) {
      TORCH_CHECK(k_cache.stride(d) % 8 == 0 && v_cache.stride(d) % 8 == 0,
                  "fp8 KV-cache pointers and strides must be multiples of 8 bytes");
    }
    TORCH_CHECK(aligned(k_cache.data_ptr(), 8) && aligned(v_cache.data_ptr(), 8),
                "fp8 KV-cache pointers and strides must be multiples of 8 bytes");
  } else {
    // Row starts aligned to 4 / 8 / 16 bytes for head_dim <= 64 / <= 128 / above.
    const int64_t align = head_dim <= 64 ? 4 : (head_dim <= 128 ? 8 : 16);
    for (int d = 0; d < 3; ++d) {
      TORCH_CHECK((k_cache.stride(d) * 2) % align == 0 && (v_cache.stride(d) * 2) % align == 0,
                  "KV-cache strides must be multiples of head_dim / 32 for vectorised loads");
    }
    TORCH_CHECK(aligned(k_cache.data_ptr(), align) && aligned(v_cache.data_ptr(), align),
                "KV-cache pointers must be aligned to head_dim / 16 bytes");
  }
  TORCH_CHECK(block_tables.scalar_type() == at::kInt && block_tables.dim() == 2 && block_tables.stride(1) == 1,
              "block_tables must be a 2-D int32 tensor with a contiguous last dimension");
  TORCH_CHECK(seq_lens.scalar_type() == at::kInt && seq_lens.dim() == 1 && seq_lens.is_contiguous(),
              "seq_lens must be a contiguous 1-D int32 tensor");
  TORCH_CHECK(block_tables.size(0) >= num_seqs && seq_lens.size(0) >= num_seqs,
              "block_tables and seq_lens must have at least num_seqs rows");
  TORCH_CHECK(max_seq_len >= 0, "max_seq_len must be non-negative");

  const bool split = max_seq_len > DK_PARTITION_SIZE;
  const int64_t needed_parts = (max_seq_len + DK_PARTITION_SIZE - 1) / DK_PARTITION_SIZE;
  int64_t max_partitions = 1;
  if (split) {
    TORCH_CHECK(tmp_out.scalar_type() == at::kFloat && max_logits.scalar_type() == at::kFloat &&
                    exp_sums.scalar_type() == at::kFloat,
                "split-K workspace tensors must be float32");
    TORCH_CHECK(tmp_out.is_contiguous() && max_logits.is_contiguous() && exp_sums.is_contiguous(),
                "split-K workspace tensors must be contiguous");
    TORCH_CHECK(tmp_out.dim() == 4 && tmp_out.size(0) == num_seqs && tmp_out.size(1) == num_q_heads &&
                    tmp_out.size(2) >= needed_parts && tmp_out.size(3) == head_dim,
                "tmp_out must be [num_seqs, num_q_heads, >= ceil(max_seq_len / 512), head_dim]");
    TORCH_CHECK(max_logits.sizes() == exp_sums.sizes() && max_logits.dim() == 3 && max_logits.size(0) == num_seqs &&
                    max_logits.size(1) == num_q_heads && max_logits.size(2) == tmp_out.size(2),
                "max_logits / exp_sums must be [num_seqs, num_q_heads, max_partitions]");
    max_partitions = tmp_out.size(2);
  }
  if (num_seqs == 0) return;

  dk_paged_attn_params p{};
  p.out = out.data_ptr();
  p.q = q.data_ptr();
  p.k_cache = k_cache.data_ptr();
  p.v_cache = v_cache.data_ptr();
  p.block_tables = block_tables.data_ptr<int32_t>();
  p.seq_lens = seq_lens.data_ptr<int32_t>();
  p.tmp_out = split ? tmp_out.data_ptr<float>() : nullptr;
  p.max_logits = split ? max_logits.data_ptr<float>() : nullptr;
  p.exp_sums = split ? exp_sums.data_ptr<float>() : nullptr;
  p.q_stride_seq = q.stride(0);
  p.q_stride_head = q.stride(1);
  p.out_stride_seq = out.stride(0);
  p.out_stride_head = out.stride(1);
  p.k_stride_block = k_cache.stride(0);
  p.k_stride_token = k_cache.stride(1);
  p.k_stride_head = k_cache.stride(2);
  p.v_stride_block = v_cache.stride(0);
  p.v_stride_token = v_cache.stride(1);
  p.v_stride_head = v_cache.stride(2);
  p.bt_stride = block_tables.stride(0);
  p.num_seqs = static_cast<int32_t>(num_seqs);
  p.num_q_heads = static_cast<int32_t>(num_q_heads);
  p.num_kv_heads = static_cast<int32_t>(num_kv_heads);
  p.block_size = static_cast<int32_t>(k_cache.size(1));
  p.max_partitions = static_cast<int32_t>(max_partitions);
  p.scale = static_cast<float>(scale);

  const int dt = dtype_code(q.scalar_type(), "paged_attention_decode");
  const DeviceGuard guard(q.device());
  if (fp8) {
    check_status(dk_paged_attention_decode_fp8(&p, dt, static_cast<int>(head_dim), static_cast<int>(max_seq_len),
                                               static_cast<float>(k_scale), static_cast<float>(v_scale), stream_of(q)),
                 "paged_attention_decode_fp8");
  } else {
    check_status(dk_paged_attention_decode(&p, dt, static_cast<int>(head_dim), static_cast<int>(max_seq_len),
                                           stream_of(q)),
                 "paged_attention_decode");
  }
}

}  // namespace

void paged_attention_decode(at::Tensor& out, const at::Tensor& q, const at::Tensor& k_cache,
                            const at::Tensor& v_cache, const at::Tensor& block_tables, const at::Tensor& seq_lens,
                            double scale, int64_t max_seq_len, at::Tensor& tmp_out, at::Tensor& max_logits,
                            at::Tensor& exp_sums) {
  attention_impl(out, q, k_cache, v_cache, block_tables, seq_lens, scale, max_seq_len, tmp_out, max_logits, exp_sums,
                 false, 1.0, 1.0);
}

// The same op over an fp8 (e4m3fn) KV cache with per-tensor scales; no
// counterpart in the reference (README.md:185 lists FP8 KV as unsupported).
void paged_attention_decode_fp8(at::Tensor& out, const at::Tensor& q, const at::Tensor& k_cache,
                                const at::Tensor& v_cache, const at::Tensor& block_tables, const at::Tensor& seq_lens,
                                double scale, int64_t max_seq_len, at::Tensor& tmp_out, at::Tensor& max_logits,
                                at::Tensor& exp_sums, double k_scale, double v_scale) {
  attention_impl(out, q, k_cache, v_cache, block_tables, seq_lens, scale, max_seq_len, tmp_out, max_logits, exp_sums,
                 true, k_scale, v_scale);
}

// ---------------------------------------------------------------------------
// gemm_tn (csrc/ops.cu:149-182)
// ---------------------------------------------------------------------------
namespace {

// Checked arguments of a gemm_tn call, with its split-K workspace (decode
// shapes that split K take it from the caching allocator; freed back to it
// when the op returns, the stream order keeps it alive for the kernels).
struct GemmArgs {
  int dt, M, N, K, lda, ldb, ldc;
  const void* bias;
  at::Tensor ws;
  int64_t ws_bytes;
};

GemmArgs gemm_args(at::Tensor& c, const at::Tensor& a, const at::Tensor& b, const std::optional<at::Tensor>& bias) {
  TORCH_CHECK(a.is_cuda(), "gemm_tn: tensors must be on CUDA");
  TORCH_CHECK(a.dim() == 2 && b.dim() == 2 && c.dim() == 2, "gemm_tn: a [M,K], b [N,K], c [M,N]");
  check_same(a, b, "a/b");
  check_same(a, c, "a/c");
  const int64_t M = a.size(0), K = a.size(1), N = b.size(0);
  TORCH_CHECK(b.size(1) == K, "gemm_tn: K mismatch");
  TORCH_CHECK(c.size(0) == M && c.size(1) == N, "gemm_tn: c must be [M, N]");
  TORCH_CHECK(M < (int64_t{1} << 31) && N < (int64_t{1} << 31) && K < (int64_t{1} << 31) &&
                  a.stride(0) < (int64_t{1} << 31) && b.stride(0) < (int64_t{1} << 31) &&
                  c.stride(0) < (int64_t{1} << 31),
              "gemm_tn: sizes and row strides must fit in 32 bits");
  TORCH_CHECK(a.stride(1) == 1 && b.stride(1) == 1 && c.stride(1) == 1, "gemm_tn: last dims must be contiguous");
  TORCH_CHECK(K % 8 == 0 && a.stride(0) % 8 == 0 && b.stride(0) % 8 == 0,
              "gemm_tn: K and row strides of a/b must be multiples of 8");
  TORCH_CHECK(aligned(a.data_ptr(), 16) && aligned(b.data_ptr(), 16), "gemm_tn: a and b must be 16-byte aligned");
  const void* bias_ptr = nullptr;
  if (bias.has_value()) {
    check_same(a, *bias, "a/bias");
    TORCH_CHECK(bias->dim() == 1 && bias->size(0) == N && bias->is_contiguous(), "gemm_tn: bias must be [N]");
    bias_ptr = bias->data_ptr();
  }
  GemmArgs g{};
  g.dt = dtype_code(a.scalar_type(), "gemm_tn");
  g.M = static_cast<int>(M);
  g.N = static_cast<int>(N);
  g.K = static_cast<int>(K);
  g.lda = static_cast<int>(a.stride(0));
  g.ldb = static_cast<int>(b.stride(0));
  g.ldc = static_cast<int>(c.stride(0));
  g.bias = bias_ptr;
  g.ws_bytes = dk_gemm_tn_workspace_bytes(g.M, g.N, g.K);
  if (g.ws_bytes > 0) g.ws = at::empty({g.ws_bytes / 4}, a.options().dtype(at::kFloat));
  return g;
}

}  // namespace

void gemm_tn(at::Tensor& c, const at::Tensor& a, const at::Tensor& b, const std::optional<at::Tensor>& bias) {
  GemmArgs g = gemm_args(c, a, b, bias);
  const DeviceGuard guard(a.device());
  check_status(dk_gemm_tn_ws(g.dt, a.data_ptr(), b.data_ptr(), g.bias, c.data_ptr(), g.M, g.N, g.K, g.lda, g.ldb, g.ldc,
                             g.ws_bytes > 0 ? g.ws.data_ptr() : nullptr, g.ws_bytes, stream_of(a)),
               "gemm_tn");
}

// gemm_tn into `out`, then fused_add_rms_norm(out, residual, weight, eps); the
// split-K sum of decode shapes happens inside the norm's kernel (same bits as
// the two ops).
void gemm_tn_add_rms_norm(at::Tensor& out, const at::Tensor& a, const at::Tensor& b,
                          const std::optional<at::Tensor>& bias, at::Tensor& residual, const at::Tensor& weight,
                          double eps) {
  GemmArgs g = gemm_args(out, a, b, bias);
  const DeviceGuard guard(a.device());
  check_same(out, residual, "out/residual");
  check_same(out, weight, "out/weight");
  TORCH_CHECK(residual.dim() == 2 && residual.size(0) == g.M && residual.size(1) == g.N && residual.stride(1) == 1,
              "gemm_tn_add_rms_norm: residual must be [M, N] with contiguous rows");
  TORCH_CHECK(residual.stride(0) < (int64_t{1} << 31), "gemm_tn_add_rms_norm: residual row stride must fit in 32 bits");
  TORCH_CHECK(weight.dim() == 1 && weight.size(0) == g.N && weight.is_contiguous(),
              "gemm_tn_add_rms_norm: weight must be [N]");
  check_status(dk_gemm_tn_add_rms_norm(g.dt, a.data_ptr(), b.data_ptr(), g.bias, out.data_ptr(), residual.data_ptr(),
                                       weight.data_ptr(), static_cast<float>(eps), g.M, g.N, g.K, g.lda, g.ldb, g.ldc,
                                       static_cast<int>(residual.stride(0)),
                                       g.ws_bytes > 0 ? g.ws.data_ptr() : nullptr, g.ws_bytes, stream_of(a)),
               "gemm_tn_add_rms_norm");
}

// ---------------------------------------------------------------------------
// rms_norm / fused_add_rms_norm / silu_and_mul (csrc/ops.cu:200-265)
// ---------------------------------------------------------------------------
void rms_norm(at::Tensor& out, const at::Tensor& input, const at::Tensor& weight, double eps) {
  TORCH_CHECK(input.is_cuda(), "rms_norm: input must be on CUDA");
  check_same(input, out, "input/out");
  check_same(input, weight, "input/weight");
  TORCH_CHECK(out.sizes() == input.sizes(), "rms_norm: out must match input shape");
  const int64_t H = input.size(-1);
  TORCH_CHECK(weight.dim() == 1 && weight.size(0) == H && weight.is_contiguous(), "rms_norm: weight must be [H]");
  const int64_t rows = input.numel() / std::max<int64_t>(H, 1);
  const int64_t in_stride = row_stride(input, "rms_norm(input)");
  const int64_t out_stride = row_stride(out, "rms_norm(out)");
  const int dt = dtype_code(input.scalar_type(), "rms_norm");
  const DeviceGuard guard(input.device());
  check_status(dk_rms_norm(dt, out.data_ptr(), input.data_ptr(), weight.data_ptr(), static_cast<int>(rows),
                           static_cast<int>(H), in_stride, out_stride, static_cast<float>(eps), stream_of(input)),
               "rms_norm");
}

void fused_add_rms_norm(at::Tensor& input, at::Tensor& residual, const at::Tensor& weight, double eps) {
  TORCH_CHECK(input.is_cuda(), "fused_add_rms_norm: input must be on CUDA");
  check_same(input, residual, "input/residual");
  check_same(input, weight, "input/weight");
  TORCH_CHECK(residual.sizes() == input.sizes(), "fused_add_rms_norm: residual must match input shape");
  const int64_t H = input.size(-1);
  TORCH_CHECK(weight.dim() == 1 && weight.size(0) == H && weight.is_contiguous(),
              "fused_add_rms_norm: weight must be [H]");
  const int64_t rows = input.numel() / std::max<int64_t>(H, 1);
  const int64_t in_stride = row_stride(input, "fused_add_rms_norm(input)");
  const int64_t res_stride = row_stride(residual, "fused_add_rms_norm(residual)");
  const int dt = dtype_code(input.scalar_type(), "fused_add_rms_norm");
  const DeviceGuard guard(input.device());
  check_status(dk_fused_add_rms_norm(dt, input.data_ptr(), residual.data_ptr(), weight.data_ptr(),
                                     static_cast<int>(rows), static_cast<int>(H), in_stride, res_stride,
                                     static_cast<float>(eps), stream_of(input)),
               "fused_add_rms_norm");
}

void silu_and_mul(at::Tensor& out, const at::Tensor& input) {
  TORCH_CHECK(input.is_cuda(), "silu_and_mul: input must be on CUDA");
  check_same(input, out, "input/out");
  const int64_t d = input.size(-1) / 2;
  TORCH_CHECK(input.size(-1) == 2 * d, "silu_and_mul: last dimension must be even");
  TORCH_CHECK(out.size(-1) == d && out.numel() * 2 == input.numel(), "silu_and_mul: out must be [..., d]");
  const int64_t rows = d == 0 ? 0 : input.numel() / (2 * d);
  const int64_t in_stride = row_stride(input, "silu_and_mul(input)");
  const int64_t out_stride = row_stride(out, "silu_and_mul(out)");
  const int dt = dtype_code(input.scalar_type(), "silu_and_mul");
  const DeviceGuard guard(input.device());
  check_status(dk_silu_and_mul(dt, out.data_ptr(), input.data_ptr(), static_cast<int>(rows), static_cast<int>(d),
                               in_stride, out_stride, stream_of(input)),
               "silu_and_mul");
}

// ---------------------------------------------------------------------------
// rotary_embedding / reshape_and_cache: the steps either side of attention
// that DecodeKernels leaves to the serving engine; the schemas are vLLM's ops
// of the same names (query / key as [tokens, heads * head_size] or
// [tokens, heads, head_size]; caches as the [blocks, block_size, kv_heads,
// head_size] views paged_attention_decode takes).
// ---------------------------------------------------------------------------
namespace {

// (token stride, head stride) of a [T, H * D] or [T, H, D] tensor.
std::pair<int64_t, int64_t> token_head_strides(const at::Tensor& t, int64_t head_size, const char* name) {
  TORCH_CHECK(t.stride(-1) == 1, name, ": last dimension must be contiguous");
  if (t.dim() == 2) {
    TORCH_CHECK(t.size(1) % head_size == 0, name, ": last dimension must be a multiple of head_size");
    return {t.stride(0), head_size};
  }
  TORCH_CHECK(t.dim() == 3 && t.size(2) == head_size, name, ": expected [tokens, heads * head_size] or [tokens, heads, head_size]");
  return {t.stride(0), t.stride(1)};
}

int64_t heads_of(const at::Tensor& t, int64_t head_size) { return t.dim() == 2 ? t.size(1) / head_size : t.size(1); }

}  // namespace

namespace {

// Checked dk_rotary_params of a rotary_embedding call (and its dtype code).
dk_rotary_params rotary_params(const at::Tensor& positions, at::Tensor& query, const std::optional<at::Tensor>& key,
                               int64_t head_size, const at::Tensor& cos_sin_cache, bool is_neox, int& dt) {
  TORCH_CHECK(query.is_cuda(), "rotary_embedding: query must be on CUDA");
  TORCH_CHECK(positions.scalar_type() == at::ScalarType::Long && positions.is_contiguous(),
              "rotary_embedding: positions must be contiguous int64");
  TORCH_CHECK(head_size > 0, "rotary_embedding: head_size must be positive");
  const int64_t T = positions.numel();
  TORCH_CHECK(query.size(0) == T, "rotary_embedding: query must have one row per position");
  TORCH_CHECK(cos_sin_cache.dim() == 2 && cos_sin_cache.stride(1) == 1,
              "rotary_embedding: cos_sin_cache must be [max_position, rot_dim] with contiguous rows");
  TORCH_CHECK(cos_sin_cache.device() == query.device() && positions.device() == query.device(),
              "rotary_embedding: tensors must be on the same device");
  dt = dtype_code(query.scalar_type(), "rotary_embedding");
  int cache_dt;
  if (cos_sin_cache.scalar_type() == at::ScalarType::Float) {
    cache_dt = DK_FLOAT32;
  } else {
    TORCH_CHECK(cos_sin_cache.scalar_type() == query.scalar_type(),
                "rotary_embedding: cos_sin_cache must be float32 or the query dtype");
    cache_dt = dt;
  }
  dk_rotary_params p{};
  p.positions = positions.data_ptr<int64_t>();
  p.query = query.data_ptr();
  std::tie(p.q_stride_token, p.q_stride_head) = token_head_strides(query, head_size, "rotary_embedding(query)");
  p.num_q_heads = static_cast<int32_t>(heads_of(query, head_size));
  if (key.has_value()) {
    check_same(query, *key, "query/key");
    TORCH_CHECK(key->size(0) == T, "rotary_embedding: key must have one row per position");
    p.key = key->data_ptr();
    std::tie(p.k_stride_token, p.k_stride_head) = token_head_strides(*key, head_size, "rotary_embedding(key)");
    p.num_kv_heads = static_cast<int32_t>(heads_of(*key, head_size));
  }
  p.cos_sin_cache = cos_sin_cache.data_ptr();
  p.cache_stride = cos_sin_cache.stride(0);
  p.num_tokens = static_cast<int32_t>(T);
  p.head_size = static_cast<int32_t>(head_size);
  p.rot_dim = static_cast<int32_t>(cos_sin_cache.size(1));
  p.max_position = static_cast<int32_t>(cos_sin_cache.size(0));
  p.is_neox = is_neox ? 1 : 0;
  p.cache_dtype = cache_dt;
  return p;
}

// Checked dk_cache_write_params of a reshape_and_cache call (and its dtype
// code); fp8: the caches are float8_e4m3fn instead of the key's dtype.
dk_cache_write_params cache_params(const at::Tensor& key, const at::Tensor& value, at::Tensor& key_cache,
                                   at::Tensor& value_cache, const at::Tensor& slot_mapping, int& dt, bool fp8 = false) {
  const std::string op = fp8 ? "reshape_and_cache_fp8" : "reshape_and_cache";
  TORCH_CHECK(key.is_cuda(), op, ": key must be on CUDA");
  check_same(key, value, "key/value");
  if (fp8) {
    TORCH_CHECK(key_cache.scalar_type() == at::ScalarType::Float8_e4m3fn &&
                    value_cache.scalar_type() == at::ScalarType::Float8_e4m3fn,
                op, ": caches must be float8_e4m3fn");
    TORCH_CHECK(key_cache.device() == key.device() && value_cache.device() == key.device(), op,
                ": tensors must be on the same device");
  } else {
    check_same(key, key_cache, "key/key_cache");
    check_same(key, value_cache, "key/value_cache");
  }
  TORCH_CHECK(slot_mapping.scalar_type() == at::ScalarType::Long && slot_mapping.is_contiguous() &&
                  slot_mapping.device() == key.device(),
              op, ": slot_mapping must be contiguous int64 on the key's device");
  TORCH_CHECK(key_cache.dim() == 4 && value_cache.dim() == 4 && key_cache.sizes() == value_cache.sizes() &&
                  key_cache.stride(3) == 1 && value_cache.stride(3) == 1,
              op, ": caches must be [num_blocks, block_size, num_kv_heads, head_size] views with contiguous head_size");
  const int64_t D = key_cache.size(3);
  const int64_t T = slot_mapping.numel();
  TORCH_CHECK(key.size(0) == T && value.size(0) == T, op, ": one key / value row per slot");
  TORCH_CHECK(heads_of(key, D) == key_cache.size(2) && heads_of(value, D) == key_cache.size(2),
              op, ": key / value heads must match the cache");
  dk_cache_write_params p{};
  p.key = key.data_ptr();
  p.value = value.data_ptr();
  p.key_cache = key_cache.data_ptr();
  p.value_cache = value_cache.data_ptr();
  p.slot_mapping = slot_mapping.data_ptr<int64_t>();
  std::tie(p.k_stride_token, p.k_stride_head) = token_head_strides(key, D, (op + "(key)").c_str());
  std::tie(p.v_stride_token, p.v_stride_head) = token_head_strides(value, D, (op + "(value)").c_str());
  p.kc_stride_block = key_cache.stride(0);
  p.kc_stride_token = key_cache.stride(1);
  p.kc_stride_head = key_cache.stride(2);
  p.vc_stride_block = value_cache.stride(0);
  p.vc_stride_token = value_cache.stride(1);
  p.vc_stride_head = value_cache.stride(2);
  p.num_tokens = static_cast<int32_t>(T);
  p.num_kv_heads = static_cast<int32_t>(key_cache.size(2));
  p.head_size = static_cast<int32_t>(D);
  p.block_size = static_cast<int32_t>(key_cache.size(1));
  p.num_blocks = static_cast<int32_t>(key_cache.size(0));
  dt = dtype_code(key.scalar_type(), op.c_str());
  return p;
}

}  // namespace

void rotary_embedding(const at::Tensor& positions, at::Tensor& query, const std::optional<at::Tensor>& key,
                      int64_t head_size, const at::Tensor& cos_sin_cache, bool is_neox) {
  int dt = 0;
  const dk_rotary_params p = rotary_params(positions, query, key, head_size, cos_sin_cache, is_neox, dt);
  const DeviceGuard guard(query.device());
  check_status(dk_rotary_embedding(&p, dt, stream_of(query)), "rotary_embedding");
}

void reshape_and_cache(const at::Tensor& key, const at::Tensor& value, at::Tensor& key_cache, at::Tensor& value_cache,
                       const at::Tensor& slot_mapping) {
  int dt = 0;
  const dk_cache_write_params p = cache_params(key, value, key_cache, value_cache, slot_mapping, dt);
  const DeviceGuard guard(key.device());
  check_status(dk_reshape_and_cache(&p, dt, stream_of(key)), "reshape_and_cache");
}

// reshape_and_cache into fp8 (e4m3fn) caches with per-tensor scales.
void reshape_and_cache_fp8(const at::Tensor& key, const at::Tensor& value, at::Tensor& key_cache,
                           at::Tensor& value_cache, const at::Tensor& slot_mapping, double k_scale, double v_scale) {
  int dt = 0;
  const dk_cache_write_params p = cache_params(key, value, key_cache, value_cache, slot_mapping, dt, true);
  const DeviceGuard guard(key.device());
  check_status(dk_reshape_and_cache_fp8(&p, dt, static_cast<float>(k_scale), static_cast<float>(v_scale), stream_of(key)),
               "reshape_and_cache_fp8");
}

// rotary_embedding then reshape_and_cache of the rotated key, in one launch.
void rotary_embedding_and_cache(const at::Tensor& positions, at::Tensor& query, at::Tensor& key,
                                const at::Tensor& value, int64_t head_size, const at::Tensor& cos_sin_cache,
                                bool is_neox, at::Tensor& key_cache, at::Tensor& value_cache,
                                const at::Tensor& slot_mapping) {
  int dt = 0, dt2 = 0;
  const dk_rotary_params r = rotary_params(positions, query, key, head_size, cos_sin_cache, is_neox, dt);
  const dk_cache_write_params c = cache_params(key, value, key_cache, value_cache, slot_mapping, dt2);
  TORCH_CHECK(key_cache.size(3) == head_size, "rotary_embedding_and_cache: cache head_size must equal head_size");
  const DeviceGuard guard(query.device());
  check_status(dk_rotary_embedding_and_cache(&r, &c, dt, stream_of(query)), "rotary_embedding_and_cache");
}

// The same into fp8 (e4m3fn) caches with per-tensor scales.
void rotary_embedding_and_cache_fp8(const at::Tensor& positions, at::Tensor& query, at::Tensor& key,
                                    const at::Tensor& value, int64_t head_size, const at::Tensor& cos_sin_cache,
                                    bool is_neox, at::Tensor& key_cache, at::Tensor& value_cache,
                                    const at::Tensor& slot_mapping, double k_scale, double v_scale) {
  int dt = 0, dt2 = 0;
  const dk_rotary_params r = rotary_params(positions, query, key, head_size, cos_sin_cache, is_neox, dt);
  const dk_cache_write_params c = cache_params(key, value, key_cache, value_cache, slot_mapping, dt2, true);
  TORCH_CHECK(key_cache.size(3) == head_size, "rotary_embedding_and_cache_fp8: cache head_size must equal head_size");
  const DeviceGuard guard(query.device());
  check_status(dk_rotary_embedding_and_cache_fp8(&r, &c, dt, static_cast<float>(k_scale), static_cast<float>(v_scale),
                                                 stream_of(query)),
               "rotary_embedding_and_cache_fp8");
}

// gemm_tn into qkv, then rotary_embedding_and_cache on the query / key / value
// views of qkv's rows; the split-K sum of decode shapes happens inside the
// rotary / cache kernel (same bits as the two ops).
void gemm_tn_rotary_embedding_and_cache(at::Tensor& qkv, const at::Tensor& a, const at::Tensor& b,
                                        const std::optional<at::Tensor>& bias, const at::Tensor& positions,
                                        at::Tensor& query, at::Tensor& key, const at::Tensor& value,
                                        int64_t head_size, const at::Tensor& cos_sin_cache, bool is_neox,
                                        at::Tensor& key_cache, at::Tensor& value_cache,
                                        const at::Tensor& slot_mapping) {
  GemmArgs g = gemm_args(qkv, a, b, bias);
  const DeviceGuard guard(a.device());
  int dt = 0, dt2 = 0;
  const dk_rotary_params r = rotary_params(positions, query, key, head_size, cos_sin_cache, is_neox, dt);
  const dk_cache_write_params c = cache_params(key, value, key_cache, value_cache, slot_mapping, dt2);
  TORCH_CHECK(key_cache.size(3) == head_size, "gemm_tn_rotary_embedding_and_cache: cache head_size must equal head_size");
  check_status(dk_gemm_tn_rotary_embedding_and_cache(g.dt, a.data_ptr(), b.data_ptr(), g.bias, qkv.data_ptr(), g.M,
                                                     g.N, g.K, g.lda, g.ldb, g.ldc, &r, &c,
                                                     g.ws_bytes > 0 ? g.ws.data_ptr() : nullptr, g.ws_bytes,
                                                     stream_of(a)),
               "gemm_tn_rotary_embedding_and_cache");
}

// The same into fp8 (e4m3fn) caches with per-tensor scales.
void gemm_tn_rotary_embedding_and_cache_fp8(at::Tensor& qkv, const at::Tensor& a, const at::Tensor& b,
                                            const std::optional<at::Tensor>& bias, const at::Tensor& positions,
                                            at::Tensor& query, at::Tensor& key, const at::Tensor& value,
                                            int64_t head_size, const at::Tensor& cos_sin_cache, bool is_neox,
                                            at::Tensor& key_cache, at::Tensor& value_cache,
                                            const at::Tensor& slot_mapping, double k_scale, double v_scale) {
  GemmArgs g = gemm_args(qkv, a, b, bias);
  const DeviceGuard guard(a.device());
  int dt = 0, dt2 = 0;
  const dk_rotary_params r = rotary_params(positions, query, key, head_size, cos_sin_cache, is_neox, dt);
  const dk_cache_write_params c = cache_params(key, value, key_cache, value_cache, slot_mapping, dt2, true);
  TORCH_CHECK(key_cache.size(3) == head_size,
              "gemm_tn_rotary_embedding_and_cache_fp8: cache head_size must equal head_size");
  check_status(dk_gemm_tn_rotary_embedding_and_cache_fp8(
                   g.dt, a.data_ptr(), b.data_ptr(), g.bias, qkv.data_ptr(), g.M, g.N, g.K, g.lda, g.ldb, g.ldc, &r,
                   &c, static_cast<float>(k_scale), static_cast<float>(v_scale),
                   g.ws_bytes > 0 ? g.ws.data_ptr() : nullptr, g.ws_bytes, stream_of(a)),
               "gemm_tn_rotary_embedding_and_cache_fp8");
}

// ---------------------------------------------------------------------------
// Registration (csrc/ops.cu:270-286)
// ---------------------------------------------------------------------------
TORCH_LIBRARY(decode_kernels, m) {
  m.def(
      "paged_attention_decode(Tensor! out, Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, "
      "Tensor seq_lens, float scale, int max_seq_len, Tensor! tmp_out, Tensor! max_logits, Tensor! exp_sums) -> ()");
  m.def(
      "paged_attention_decode_fp8(Tensor! out, Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_tables, "
      "Tensor seq_lens, float scale, int max_seq_len, Tensor! tmp_out, Tensor! max_logits, Tensor! exp_sums, "
      "float k_scale, float v_scale) -> ()");
  m.def("gemm_tn(Tensor! c, Tensor a, Tensor b, Tensor? bias) -> ()");
  m.def("rms_norm(Tensor! out, Tensor input, Tensor weight, float eps) -> ()");
  m.def("fused_add_rms_norm(Tensor! input, Tensor! residual, Tensor weight, float eps) -> ()");
  m.def("silu_and_mul(Tensor! out, Tensor input) -> ()");
  m.def(
      "rotary_embedding(Tensor positions, Tensor! query, Tensor!? key, int head_size, Tensor cos_sin_cache, "
      "bool is_neox) -> ()");
  m.def("reshape_and_cache(Tensor key, Tensor value, Tensor! key_cache, Tensor! value_cache, Tensor slot_mapping) -> ()");
  m.def(
      "reshape_and_cache_fp8(Tensor key, Tensor value, Tensor! key_cache, Tensor! value_cache, Tensor slot_mapping, "
      "float k_scale, float v_scale) -> ()");
  m.def(
      "rotary_embedding_and_cache(Tensor positions, Tensor! query, Tensor! key, Tensor value, int head_size, "
      "Tensor cos_sin_cache, bool is_neox, Tensor! key_cache, Tensor! value_cache, Tensor slot_mapping) -> ()");
  m.def(
      "rotary_embedding_and_cache_fp8(Tensor positions, Tensor! query, Tensor! key, Tensor value, int head_size, "
      "Tensor cos_sin_cache, bool is_neox, Tensor! key_cache, Tensor! value_cache, Tensor slot_mapping, "
      "float k_scale, float v_scale) -> ()");
  m.def(
      "gemm_tn_add_rms_norm(Tensor! out, Tensor a, Tensor b, Tensor? bias, Tensor! residual, Tensor weight, "
      "float eps) -> ()");
  m.def(
      "gemm_tn_rotary_embedding_and_cache(Tensor! qkv, Tensor a, Tensor b, Tensor? bias, Tensor positions, "
      "Tensor! query, Tensor! key, Tensor value, int head_size, Tensor cos_sin_cache, bool is_neox, "
      "Tensor! key_cache, Tensor! value_cache, Tensor slot_mapping) -> ()");
  m.def(
      "gemm_tn_rotary_embedding_and_cache_fp8(Tensor! qkv, Tensor a, Tensor b, Tensor? bias, Tensor positions, "
      "Tensor! query, Tensor! key, Tensor value, int head_size, Tensor cos_sin_cache, bool is_neox, "
      "Tensor! key_cache, Tensor! value_cache, Tensor slot_mapping, float k_scale, float v_scale) -> ()");
}

TORCH_LIBRARY_IMPL(decode_kernels, CUDA, m) {
  m.impl("paged_attention_decode", &paged_attention_decode);
  m.impl("paged_attention_decode_fp8", &paged_attention_decode_fp8);
  m.impl("gemm_tn", &gemm_tn);
  m.impl("rms_norm", &rms_norm);
  m.impl("fused_add_rms_norm", &fused_add_rms_norm);
  m.impl("silu_and_mul", &silu_and_mul);
  m.impl("rotary_embedding", &rotary_embedding);
  m.impl("reshape_and_cache", &reshape_and_cache);
  m.impl("rotary_embedding_and_cache", &rotary_embedding_and_cache);
  m.impl("reshape_and_cache_fp8", &reshape_and_cache_fp8);
  m.impl("rotary_embedding_and_cache_fp8", &rotary_embedding_and_cache_fp8);
  m.impl("gemm_tn_add_rms_norm", &gemm_tn_add_rms_norm);
  m.impl("gemm_tn_rotary_embedding_and_cache", &gemm_tn_rotary_embedding_and_cache);
  m.impl("gemm_tn_rotary_embedding_and_cache_fp8", &gemm_tn_rotary_embedding_and_cache_fp8);
}

// Python module entry point: an empty module; importing it loads this
// library and runs the registrations above.
static struct PyModuleDef dk_module = {PyModuleDef_HEAD_INIT, "_C",
                                       "decodekernels_amd._C: registers torch.ops.decode_kernels.* (gfx950 HIP kernels)",
                                       -1, nullptr};

PyMODINIT_FUNC PyInit__C(void) { return PyModule_Create(&dk_module); }
