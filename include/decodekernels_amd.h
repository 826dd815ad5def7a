/*
 * decodekernels_amd — C ABI of the MI355X (gfx950) decode kernels.
 *
 * This is the torch-free boundary of the library: plain pointers, element
 * strides and sizes, a dtype code and a HIP stream passed as `void*`.
 * Every entry point validates its arguments on the host first, then enqueues
 * work on `stream` and returns without synchronising. The return value is a
 * hipError_t code (0 = success); for argument errors the code is
 * hipErrorInvalidValue (1) and dk_last_error() describes the failure.
 * No entry point allocates device memory, so all of them can be recorded
 * into a HIP graph.
 *
 * The five compute entry points of the reference's hot path each replace one
 * launcher of DecodeKernels (the reference), whose `dk::launch_*<T>`
 * templates take the same argument lists for one element type T in
 * {__half, __nv_bfloat16}; here the type is the `dtype` argument. The other
 * compute entry points (fp8 KV cache, RoPE, the KV-cache write) have no
 * counterpart in the reference; each says so and names what it follows.
 */
#ifndef DECODEKERNELS_AMD_H_
#define DECODEKERNELS_AMD_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element type of every 16-bit tensor argument (DK_FLOAT32: the rotary
 * cos / sin table only). */
enum dk_dtype {
  DK_FLOAT16 = 0,
  DK_BFLOAT16 = 1,
  DK_FLOAT32 = 2,
};

/* Tokens per split-K partition of the workspace contract (reference:
 * csrc/paged_attention.cuh:34, decode_kernels/ops.py:14). */
#define DK_PARTITION_SIZE 512
/* Largest GQA group (query heads per KV head); the reference's is 8
 * (csrc/paged_attention.cuh:37), this library's 16. */
#define DK_MAX_GQA_GROUP 16

/*
 * Launch descriptor of paged decode attention. Same fields and meaning as
 * the reference's `dk::PagedAttnParams` (csrc/paged_attention.cuh:39-58):
 *   out          [num_seqs, num_q_heads, head_dim]              (dtype)
 *   q            [num_seqs, num_q_heads, head_dim]              (dtype)
 *   k/v_cache    [num_blocks, block_size, num_kv_heads, head_dim] (dtype),
 *                any strides on the first three dims, head_dim contiguous
 *   block_tables [num_seqs, >= max blocks per seq] int32, row stride bt_stride
 *   seq_lens     [num_seqs] int32, read on the device
 *   tmp_out      [num_seqs, num_q_heads, max_partitions, head_dim] fp32  } only when
 *   max_logits   [num_seqs, num_q_heads, max_partitions] fp32           } max_seq_len
 *   exp_sums     [num_seqs, num_q_heads, max_partitions] fp32           } > 512
 * Strides are in elements.
 */
typedef struct dk_paged_attn_params {
  void* out;
  const void* q;
  const void* k_cache;
  const void* v_cache;
  const int32_t* block_tables;
  const int32_t* seq_lens;
  float* tmp_out;
  float* max_logits;
  float* exp_sums;
  int64_t q_stride_seq, q_stride_head;
  int64_t out_stride_seq, out_stride_head;
  int64_t k_stride_block, k_stride_token, k_stride_head;
  int64_t v_stride_block, v_stride_token, v_stride_head;
  int64_t bt_stride;
  int32_t num_seqs, num_q_heads, num_kv_heads, block_size, max_partitions;
  float scale;
} dk_paged_attn_params;

/*
 * Single-token decode attention over a paged KV cache, with flash-decoding
 * split-K when max_seq_len > DK_PARTITION_SIZE.
 * Replaces dk::launch_paged_attention_decode<T> (csrc/paged_attention.cuh:312-333).
 * head_dim in {64, 96, 128, 192, 256} (the reference: 64, 128, 256);
 * num_q_heads / num_kv_heads <= DK_MAX_GQA_GROUP.
 * max_seq_len is an upper bound on seq_lens that selects the single-pass or
 * split-K path; with split-K, p->max_partitions must be >= ceil(max_seq_len / 512).
 */
int dk_paged_attention_decode(const dk_paged_attn_params* p, int dtype, int head_dim, int max_seq_len, void* stream);

/*
 * The same op over an fp8 KV cache: k_cache / v_cache hold OCP e4m3fn bytes
 * (torch.float8_e4m3fn) with per-tensor dequantisation scales, K = k_scale * k8
 * and V = v_scale * v8; q and out stay in `dtype` (fp16 / bf16). Strides are
 * in elements (bytes); pointers and strides must be multiples of 8 bytes.
 * Same workspace contract as dk_paged_attention_decode.
 * No counterpart in DecodeKernels, whose README lists FP8 KV as unsupported
 * (README.md:185); the signature follows vLLM's fp8 KV cache (e4m3 values,
 * per-tensor k_scale / v_scale).
 */
int dk_paged_attention_decode_fp8(const dk_paged_attn_params* p, int dtype, int head_dim, int max_seq_len,
                                  float k_scale, float v_scale, void* stream);

/* Size of the device array that dk_paged_attention_decode_noalloc uses as its
 * split-K workspace: 64 MiB on each GPU where a no-alloc call has run (the
 * array is in a code object of its own, loaded on a device at its first use
 * there), held until the process ends. */
#define DK_NOALLOC_SCRATCH_BYTES 67108864

/*
 * dk_paged_attention_decode without a caller-provided workspace: the split-K
 * partial results go to a library-owned, statically allocated device array of
 * DK_NOALLOC_SCRATCH_BYTES per GPU instead of p->tmp_out / max_logits /
 * exp_sums (those fields and p->max_partitions are ignored). Same kernels, so
 * the same results bit for bit. It allocates nothing (no hipMalloc, no
 * allocating library call); the array's address is looked up once per device
 * on the first call there. The workspace needs
 * num_seqs * num_q_heads * ceil(max_seq_len / 512) * (head_dim + 2) * 4 bytes
 * (each of its three parts rounded up to 256); larger calls fail with
 * hipErrorInvalidValue and a dk_last_error() message. Every call on one GPU
 * shares that GPU's array: calls that overlap in time on one GPU (different
 * streams, concurrent graph replays) race and must not be issued.
 * No counterpart in DecodeKernels: it is for callers that cannot allocate
 * device memory at all -- code under HIP-graph capture, tight serving loops,
 * harnesses that forbid allocation.
 */
int dk_paged_attention_decode_noalloc(const dk_paged_attn_params* p, int dtype, int head_dim, int max_seq_len,
                                      void* stream);

/*
 * C[M,N] = A[M,K] * B[N,K]^T (+ bias[N]), fp32 accumulation, one rounding.
 * Replaces dk::launch_gemm_tn<T> (csrc/gemm_wmma.cuh:209-219).
 * K, lda and ldb must be multiples of 8, lda and ldb >= K, ldc >= N (the
 * stride of a single row, M = 1 or N = 1, is ignored); A and B 16-byte
 * aligned; bias may be NULL.
 * Takes no workspace: shapes whose fastest plan splits K (see dk_gemm_tn_ws)
 * run unsplit.
 */
int dk_gemm_tn(int dtype, const void* A, const void* B, const void* bias, void* C, int M, int N, int K, int lda,
               int ldb, int ldc, void* stream);

/*
 * Bytes of fp32 workspace with which dk_gemm_tn_ws splits the K reduction of
 * this shape over workgroups; 0 when the shape is not split.
 */
int64_t dk_gemm_tn_workspace_bytes(int M, int N, int K);

/*
 * Launch plan of dk_gemm_tn_ws (with_workspace != 0, workspace large enough)
 * or dk_gemm_tn. Skinny kernel (M <= 64): plan[0..3] = waves along N per
 * workgroup (16 columns each), waves along K, K splits, columns per split;
 * tiled kernel (M > 64, and M <= 64 where 64-row tiles fill the CUs better:
 * plan[0] = 64) = tile rows, tile columns, K splits, columns per split. For
 * tests and tuning; launches nothing.
 * No counterpart in DecodeKernels.
 */
int dk_gemm_tn_plan(int M, int N, int K, int with_workspace, int* plan);

/*
 * dk_gemm_tn with a caller-provided workspace (16-byte aligned). Decode
 * shapes (M <= 64) run one workgroup per CU with wide column tiles, which
 * cuts the activation rows each workgroup re-reads; where that leaves too few
 * column tiles (the MLP down projection, the attention output and qkv
 * projections), and for tiled shapes (M > 64) whose tiles leave CUs idle
 * (batched decode, M of a few hundred), the K reduction is split over
 * workgroups that write fp32 partial tiles to the workspace (at most 64 MiB),
 * and a second kernel sums them in a fixed order, adds the bias in fp32 and
 * rounds once: deterministic, and equal to the unsplit result up to the
 * order of the fp32 additions. A NULL workspace, or one smaller than
 * dk_gemm_tn_workspace_bytes(M, N, K), runs exactly dk_gemm_tn.
 * No counterpart in DecodeKernels, whose dk::launch_gemm_tn<T>
 * (csrc/gemm_wmma.cuh:209-219) takes no workspace; the torch op gemm_tn
 * (csrc/ops.cu:149-182 there) calls this with a workspace from PyTorch's
 * caching allocator.
 */
int dk_gemm_tn_ws(int dtype, const void* A, const void* B, const void* bias, void* C, int M, int N, int K, int lda,
                  int ldb, int ldc, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * out = x * rsqrt(mean(x^2) + eps) * weight, per row of H elements.
 * Replaces dk::launch_rms_norm<T> (csrc/norm_act.cuh:153-166).
 * Strides in elements, non-negative; out_stride >= H when rows > 1 (rows
 * written must not overlap; in_stride 0 repeats one input row).
 */
int dk_rms_norm(int dtype, void* out, const void* input, const void* weight, int rows, int H, int64_t in_stride,
                int64_t out_stride, float eps, void* stream);

/*
 * In place: residual = round(input + residual); input = rms_norm(residual) * weight.
 * Replaces dk::launch_fused_add_rms_norm<T> (csrc/norm_act.cuh:168-183).
 * Both buffers are written: in_stride, res_stride >= H when rows > 1.
 */
int dk_fused_add_rms_norm(int dtype, void* input, void* residual, const void* weight, int rows, int H,
                          int64_t in_stride, int64_t res_stride, float eps, void* stream);

/*
 * out[r, :d] = silu(input[r, :d]) * input[r, d:2d].
 * Replaces dk::launch_silu_and_mul<T> (csrc/norm_act.cuh:185-198).
 * Strides in elements, non-negative; out_stride >= d when rows > 1.
 */
int dk_silu_and_mul(int dtype, void* out, const void* input, int rows, int d, int64_t in_stride, int64_t out_stride,
                    void* stream);

/*
 * Rotary position embedding, in place on q and k: for the first rot_dim
 * columns of every head, pairs (x, y) <- (x cos - y sin, y cos + x sin) with
 * cos = cos_sin_cache[position][i], sin = cos_sin_cache[position][rot_dim/2 + i];
 * NeoX pairing x = v[i], y = v[i + rot_dim/2]; GPT-J pairing x = v[2i],
 * y = v[2i + 1]. fp32 arithmetic, one rounding per output.
 *   positions      [num_tokens] int64; a position outside [0, max_position)
 *                  leaves its token unchanged
 *   query          [num_tokens, num_q_heads, head_size], strides in elements
 *   key            [num_tokens, num_kv_heads, head_size] or NULL
 *   cos_sin_cache  [max_position, rot_dim], row stride cache_stride, float32
 *                  (cache_dtype DK_FLOAT32) or the query dtype
 * No counterpart in DecodeKernels, which leaves this step to the serving
 * engine: it is vLLM's rotary_embedding op (positions, query, key, head_size,
 * cos_sin_cache, is_neox), run before paged attention in every decode step.
 */
typedef struct dk_rotary_params {
  const int64_t* positions;
  void* query;
  void* key;
  const void* cos_sin_cache;
  int64_t q_stride_token, q_stride_head;
  int64_t k_stride_token, k_stride_head;
  int64_t cache_stride;
  int32_t num_tokens, num_q_heads, num_kv_heads, head_size, rot_dim, max_position, is_neox, cache_dtype;
} dk_rotary_params;

int dk_rotary_embedding(const dk_rotary_params* p, int dtype, void* stream);

/*
 * Writes new tokens' K and V rows into the paged cache:
 *   key_cache[slot / block_size, slot % block_size, h, :] = key[t, h, :],
 *   value_cache likewise, with slot = slot_mapping[t] (int64). Negative slots
 *   (padding) and slots at or past num_blocks * block_size are skipped.
 * key / value [num_tokens, num_kv_heads, head_size]; the caches use the
 * (block, token, head) strides of dk_paged_attn_params, so NHD, HND and
 * vLLM's interleaved K|V buffer all work. A bit-exact copy.
 * No counterpart in DecodeKernels, which leaves this step to the serving
 * engine: it is vLLM's reshape_and_cache_flash op, which fills the cache that
 * paged attention then reads.
 */
typedef struct dk_cache_write_params {
  const void* key;
  const void* value;
  void* key_cache;
  void* value_cache;
  const int64_t* slot_mapping;
  int64_t k_stride_token, k_stride_head;
  int64_t v_stride_token, v_stride_head;
  int64_t kc_stride_block, kc_stride_token, kc_stride_head;
  int64_t vc_stride_block, vc_stride_token, vc_stride_head;
  int32_t num_tokens, num_kv_heads, head_size, block_size, num_blocks;
} dk_cache_write_params;

int dk_reshape_and_cache(const dk_cache_write_params* p, int dtype, void* stream);

/*
 * dk_reshape_and_cache into an fp8 (e4m3fn) cache: key / value (dtype
 * DK_FLOAT16 or DK_BFLOAT16) are quantized as x / scale in fp32, saturated to
 * +-448 (NaN stays NaN) and rounded to nearest even, then written to the
 * one-byte-per-element caches (strides in elements, as for the 16-bit caches).
 * k_scale / v_scale must be positive and finite: the per-tensor scales that
 * dk_paged_attention_decode_fp8 then applies when it reads the cache.
 * No counterpart in DecodeKernels: vLLM's reshape_and_cache_flash with
 * kv_cache_dtype "fp8".
 */
int dk_reshape_and_cache_fp8(const dk_cache_write_params* p, int dtype, float k_scale, float v_scale, void* stream);

/*
 * dk_rotary_embedding followed by dk_reshape_and_cache in one launch: q and
 * k rotated in place as by dk_rotary_embedding(r), then the rotated k and v
 * written to the cache as by dk_reshape_and_cache(c). Results are identical
 * to the two calls in sequence (a position outside the table caches the
 * unrotated k; a skipped slot still rotates). r->key must be c->key with the
 * same strides, and the token, KV-head and head-size counts must agree.
 * No counterpart in DecodeKernels or as one op in vLLM: it saves a launch
 * per decoder layer for engines that run both steps back to back.
 */
int dk_rotary_embedding_and_cache(const dk_rotary_params* r, const dk_cache_write_params* c, int dtype,
                                  void* stream);

/*
 * dk_rotary_embedding_and_cache into fp8 (e4m3fn) caches: q and k rotated in
 * place as above, the rotated k (after its rounding to dtype) and v quantized
 * into the caches as by dk_reshape_and_cache_fp8(c, dtype, k_scale, v_scale).
 * Results are identical to dk_rotary_embedding then dk_reshape_and_cache_fp8.
 * No counterpart in DecodeKernels (see dk_reshape_and_cache_fp8).
 */
int dk_rotary_embedding_and_cache_fp8(const dk_rotary_params* r, const dk_cache_write_params* c, int dtype,
                                      float k_scale, float v_scale, void* stream);

/*
 * Decode-layer fusions of a GEMM with the op that consumes its output. The
 * GEMM's plan splits K at decode sizes (see dk_gemm_tn_ws); the consumer's
 * kernel then sums the fp32 partial tiles itself, in split order, and rounds
 * them exactly as the GEMM's own reduce kernel would, so each call equals the
 * two calls in sequence bit for bit while launching one kernel fewer. Plans
 * that do not split run the two ops in sequence. workspace / workspace_bytes
 * as for dk_gemm_tn_ws (dk_gemm_tn_workspace_bytes(M, N, K); NULL: no split).
 * No counterpart in DecodeKernels, whose decode step runs gemm_tn and the
 * norm (csrc/ops.cu:149-182, 200-265) as separate launches and leaves the
 * rotary embedding and cache write to the serving engine.
 *
 * dk_gemm_tn_add_rms_norm: out = A B^T (+ bias) as dk_gemm_tn_ws [M, N] (row
 * stride ld_out), then dk_fused_add_rms_norm(out, residual, weight, eps)
 * over its M rows of N: residual = round(out + residual), out =
 * rms_norm(residual) * weight. The o projection into the post-attention
 * norm, or the down projection into the next layer's input norm.
 */
int dk_gemm_tn_add_rms_norm(int dtype, const void* A, const void* B, const void* bias, void* out, void* residual,
                            const void* weight, float eps, int M, int N, int K, int lda, int ldb, int ld_out,
                            int ld_res, void* workspace, int64_t workspace_bytes, void* stream);

/*
 * dk_gemm_tn_rotary_embedding_and_cache: C = A B^T (+ bias) as dk_gemm_tn_ws
 * (a fused q | k | v projection), then dk_rotary_embedding_and_cache(r, c).
 * r->query, r->key (== c->key) and c->value must be views of C's rows (token
 * stride ldc, every head inside the row) and r->num_tokens == M. _fp8: the
 * caches are e4m3fn, as dk_rotary_embedding_and_cache_fp8.
 */
int dk_gemm_tn_rotary_embedding_and_cache(int dtype, const void* A, const void* B, const void* bias, void* C, int M,
                                          int N, int K, int lda, int ldb, int ldc, const dk_rotary_params* r,
                                          const dk_cache_write_params* c, void* workspace, int64_t workspace_bytes,
                                          void* stream);
int dk_gemm_tn_rotary_embedding_and_cache_fp8(int dtype, const void* A, const void* B, const void* bias, void* C,
                                              int M, int N, int K, int lda, int ldb, int ldc,
                                              const dk_rotary_params* r, const dk_cache_write_params* c,
                                              float k_scale, float v_scale, void* workspace, int64_t workspace_bytes,
                                              void* stream);

/* Description of the last argument error raised on this thread ("" if none).
 * The reference reports these through TORCH_CHECK messages (csrc/ops.cu). */
const char* dk_last_error(void);

/* hipGetErrorString for a code returned above. */
const char* dk_error_string(int code);

/* Library version string. */
const char* dk_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DECODEKERNELS_AMD_H_ */
