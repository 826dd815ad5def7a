/*
 * A torch-free caller of the C ABI (include/decodekernels_amd.h), as an FFI
 * user of the library would write it: device memory from the HIP runtime,
 * plain C everywhere else. It runs, on device 0:
 *   1. dk_gemm_tn (a ragged decode shape with a bias) and dk_gemm_tn_ws (a
 *      shape whose plan splits K, with a workspace of
 *      dk_gemm_tn_workspace_bytes), each against a double-precision GEMM of the
 *      same bf16 inputs;
 *   2. dk_paged_attention_decode over a bf16 NHD cache (block 16), one
 *      sequence past 512 tokens (split-K, caller workspace), one short, one
 *      empty, against a double-precision softmax attention of the same inputs
 *      (an empty sequence gives zeros);
 *   3. two argument errors, which must return hipErrorInvalidValue (1) with
 *      the message the torch ops raise.
 * Tolerance: 2e-2 absolute (the bf16 parity bar of the library's tests; the
 * outputs here are O(1), where half a bf16 ulp is below it). Prints one line
 * per check and exits 0 only if all pass. Built next to this file by
 * build_example.py (from __graft_entry__.build()); run by
 * tests/test_c_abi_example.py.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "decodekernels_amd.h"

static int failures = 0;

#define HIP_OK(x)                                                               \
  do {                                                                          \
    hipError_t e_ = (x);                                                        \
    if (e_ != hipSuccess) {                                                     \
      fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
      exit(2);                                                                  \
    }                                                                           \
  } while (0)

/* fp32 -> bf16, round to nearest even (inputs are finite). */
static uint16_t to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static float from_bf16(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Uniform in [-1, 1) from a 64-bit LCG (deterministic across platforms). */
static uint64_t rng_state = 0x9e3779b97f4a7c15ull;
static float uniform(void) {
  rng_state = rng_state * 6364136223846793005ull + 1442695040888963407ull;
  return (float)((double)(rng_state >> 11) / 9007199254740992.0 * 2.0 - 1.0);
}

static uint16_t* random_bf16(size_t n, float scale) {
  uint16_t* h = (uint16_t*)malloc(n * sizeof(uint16_t));
  for (size_t i = 0; i < n; ++i) h[i] = to_bf16(uniform() * scale);
  return h;
}

static void* to_device(const void* host, size_t bytes) {
  void* d = NULL;
  HIP_OK(hipMalloc(&d, bytes > 0 ? bytes : 16));
  if (host != NULL && bytes > 0) HIP_OK(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice));
  return d;
}

static void report(const char* what, double err, double bar) {
  const int ok = err <= bar;
  printf("%s %s: max abs err %.3e (bar %.1e)\n", ok ? "ok  " : "FAIL", what, err, bar);
  if (!ok) ++failures;
}

/* C = A B^T + bias through dk_gemm_tn (workspace == 0) or dk_gemm_tn_ws. */
static void check_gemm(int M, int N, int K, int with_bias, int with_workspace) {
  uint16_t* a = random_bf16((size_t)M * K, 1.0f);
  uint16_t* b = random_bf16((size_t)N * K, 1.0f / sqrtf((float)K));
  uint16_t* bias = random_bf16((size_t)N, 0.5f);
  void* da = to_device(a, (size_t)M * K * 2);
  void* db = to_device(b, (size_t)N * K * 2);
  void* dbias = with_bias ? to_device(bias, (size_t)N * 2) : NULL;
  void* dc = to_device(NULL, (size_t)M * N * 2);
  int plan[4] = {0, 0, 0, 0};
  int rc = dk_gemm_tn_plan(M, N, K, with_workspace, plan);
  if (rc != 0) {
    printf("FAIL gemm plan: %s\n", dk_last_error());
    ++failures;
  }
  if (with_workspace) {
    const int64_t nbytes = dk_gemm_tn_workspace_bytes(M, N, K);
    void* ws = to_device(NULL, (size_t)nbytes);
    rc = dk_gemm_tn_ws(DK_BFLOAT16, da, db, dbias, dc, M, N, K, K, K, N, ws, nbytes, NULL);
    HIP_OK(hipDeviceSynchronize());
    HIP_OK(hipFree(ws));
  } else {
    rc = dk_gemm_tn(DK_BFLOAT16, da, db, dbias, dc, M, N, K, K, K, N, NULL);
  }
  if (rc != 0) {
    printf("FAIL gemm %dx%dx%d: rc %d: %s\n", M, N, K, rc, dk_last_error());
    ++failures;
    return;
  }
  uint16_t* c = (uint16_t*)malloc((size_t)M * N * 2);
  HIP_OK(hipMemcpy(c, dc, (size_t)M * N * 2, hipMemcpyDeviceToHost));
  double err = 0.0;
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n) {
      double ref = with_bias ? from_bf16(bias[n]) : 0.0;
      for (int k = 0; k < K; ++k) ref += (double)from_bf16(a[(size_t)m * K + k]) * from_bf16(b[(size_t)n * K + k]);
      const double d = fabs((double)from_bf16(c[(size_t)m * N + n]) - ref);
      if (d > err) err = d;
    }
  char what[160];
  snprintf(what, sizeof what, "%s M=%d N=%d K=%d%s, plan (%d, %d, %d splits)", with_workspace ? "dk_gemm_tn_ws" : "dk_gemm_tn",
           M, N, K, with_bias ? " + bias" : "", plan[0], plan[1], plan[2]);
  report(what, err, 2e-2);
  free(a); free(b); free(bias); free(c);
  HIP_OK(hipFree(da)); HIP_OK(hipFree(db)); HIP_OK(hipFree(dc));
  if (dbias) HIP_OK(hipFree(dbias));
}

static void check_attention(void) {
  enum { S = 3, HKV = 2, G = 4, HQ = HKV * G, D = 128, BS = 16 };
  const int lens[S] = {700, 33, 0};
  const int max_len = 700;
  const int max_blocks = (max_len + BS - 1) / BS;
  int num_blocks = 0;
  for (int s = 0; s < S; ++s) num_blocks += (lens[s] + BS - 1) / BS;
  /* Block table: each sequence's blocks in a scattered (reversed) order. */
  int32_t bt[S * ((700 + BS - 1) / BS)];
  int next = num_blocks - 1;
  for (int s = 0; s < S; ++s)
    for (int j = 0; j < max_blocks; ++j) bt[s * max_blocks + j] = j < (lens[s] + BS - 1) / BS ? next-- : 0;
  const size_t kv_elems = (size_t)(num_blocks > 0 ? num_blocks : 1) * BS * HKV * D; /* NHD [blocks, BS, HKV, D] */
  uint16_t* k = random_bf16(kv_elems, 1.0f);
  uint16_t* v = random_bf16(kv_elems, 1.0f);
  uint16_t* q = random_bf16((size_t)S * HQ * D, 1.0f);
  const float scale = 1.0f / sqrtf((float)D);
  const int parts = (max_len + DK_PARTITION_SIZE - 1) / DK_PARTITION_SIZE;

  dk_paged_attn_params p;
  memset(&p, 0, sizeof p);
  p.q = to_device(q, (size_t)S * HQ * D * 2);
  p.k_cache = to_device(k, kv_elems * 2);
  p.v_cache = to_device(v, kv_elems * 2);
  p.block_tables = (const int32_t*)to_device(bt, sizeof bt);
  p.seq_lens = (const int32_t*)to_device(lens, sizeof lens);
  p.out = to_device(NULL, (size_t)S * HQ * D * 2);
  p.tmp_out = (float*)to_device(NULL, (size_t)S * HQ * parts * D * 4);
  p.max_logits = (float*)to_device(NULL, (size_t)S * HQ * parts * 4);
  p.exp_sums = (float*)to_device(NULL, (size_t)S * HQ * parts * 4);
  p.q_stride_seq = HQ * D;
  p.q_stride_head = D;
  p.out_stride_seq = HQ * D;
  p.out_stride_head = D;
  p.k_stride_block = p.v_stride_block = (int64_t)BS * HKV * D;
  p.k_stride_token = p.v_stride_token = HKV * D;
  p.k_stride_head = p.v_stride_head = D;
  p.bt_stride = max_blocks;
  p.num_seqs = S;
  p.num_q_heads = HQ;
  p.num_kv_heads = HKV;
  p.block_size = BS;
  p.max_partitions = parts;
  p.scale = scale;
  int rc = dk_paged_attention_decode(&p, DK_BFLOAT16, D, max_len, NULL);
  if (rc != 0) {
    printf("FAIL dk_paged_attention_decode: rc %d: %s\n", rc, dk_last_error());
    ++failures;
    return;
  }
  uint16_t* out = (uint16_t*)malloc((size_t)S * HQ * D * 2);
  HIP_OK(hipMemcpy(out, p.out, (size_t)S * HQ * D * 2, hipMemcpyDeviceToHost));

  double err = 0.0;
  double* logit = (double*)malloc(sizeof(double) * max_len);
  for (int s = 0; s < S; ++s)
    for (int h = 0; h < HQ; ++h) {
      const int kvh = h / G;
      const uint16_t* qrow = q + ((size_t)s * HQ + h) * D;
      double mx = -INFINITY, sum = 0.0;
      for (int t = 0; t < lens[s]; ++t) {
        const size_t row = (((size_t)bt[s * max_blocks + t / BS] * BS + t % BS) * HKV + kvh) * D;
        double dot = 0.0;
        for (int d = 0; d < D; ++d) dot += (double)from_bf16(qrow[d]) * from_bf16(k[row + d]);
        logit[t] = dot * scale;
        if (logit[t] > mx) mx = logit[t];
      }
      for (int t = 0; t < lens[s]; ++t) sum += exp(logit[t] - mx);
      for (int d = 0; d < D; ++d) {
        double o = 0.0;
        for (int t = 0; t < lens[s]; ++t) {
          const size_t row = (((size_t)bt[s * max_blocks + t / BS] * BS + t % BS) * HKV + kvh) * D;
          o += exp(logit[t] - mx) * from_bf16(v[row + d]);
        }
        const double ref = lens[s] > 0 ? o / sum : 0.0;
        const double e = fabs((double)from_bf16(out[((size_t)s * HQ + h) * D + d]) - ref);
        if (e > err) err = e;
      }
    }
  report("dk_paged_attention_decode bf16 NHD, lens {700, 33, 0}, group 4, head_dim 128 (split-K)", err, 2e-2);
  free(logit); free(out); free(k); free(v); free(q);
  HIP_OK(hipFree((void*)p.q)); HIP_OK(hipFree((void*)p.k_cache)); HIP_OK(hipFree((void*)p.v_cache));
  HIP_OK(hipFree((void*)p.block_tables)); HIP_OK(hipFree((void*)p.seq_lens)); HIP_OK(hipFree(p.out));
  HIP_OK(hipFree(p.tmp_out)); HIP_OK(hipFree(p.max_logits)); HIP_OK(hipFree(p.exp_sums));
}

static void check_error(const char* what, int rc, const char* needle) {
  const char* msg = dk_last_error();
  const int ok = rc == 1 && msg != NULL && strstr(msg, needle) != NULL;
  printf("%s %s: rc %d, \"%s\"\n", ok ? "ok  " : "FAIL", what, rc, msg ? msg : "(null)");
  if (!ok) ++failures;
}

int main(void) {
  HIP_OK(hipSetDevice(0));
  printf("%s\n", dk_version());
  check_gemm(5, 300, 512, 1, 0);
  check_gemm(40, 4100, 1536, 1, 1);
  check_attention();
  /* K not a multiple of 8; a GQA group above DK_MAX_GQA_GROUP. */
  void* d = to_device(NULL, 4096);
  check_error("dk_gemm_tn K = 100", dk_gemm_tn(DK_BFLOAT16, d, d, NULL, d, 4, 8, 100, 100, 100, 8, NULL),
              "multiples of 8");
  dk_paged_attn_params p;
  memset(&p, 0, sizeof p);
  p.q = p.k_cache = p.v_cache = d;
  p.out = d;
  p.num_seqs = 1;
  p.num_q_heads = DK_MAX_GQA_GROUP + 1;
  p.num_kv_heads = 1;
  p.block_size = 16;
  check_error("dk_paged_attention_decode group 17", dk_paged_attention_decode(&p, DK_BFLOAT16, 128, 16, NULL),
              "GQA group");
  HIP_OK(hipFree(d));
  printf("%s\n", failures == 0 ? "c abi example ok" : "c abi example FAILED");
  return failures == 0 ? 0 : 1;
}
