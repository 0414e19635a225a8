/*
 * A C11 caller of libnlearn_hip.so through include/nlearn_hip.h alone: device
 * memory from the HIP runtime API, no torch, no Python. Checks:
 *   - nl_gemm in the four layouts on small-integer bf16 operands with M, N, K
 *     tails: fp32 results must be exact (every partial sum < 2^24);
 *   - nl_flash_attention_fwd (causal, d = 64): the first query sees one key, so
 *     O[0] == V[0] exactly and L[0] == scale * q0 . k0; every row against a
 *     double-precision softmax within bf16 tolerance;
 *   - nl_ce_fwd_bwd: loss, lse and dlogits = (softmax - onehot) * scale against
 *     double precision.
 * Exit status 0 when every check passes; the last line printed says so.
 */
#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "nlearn_hip.h"

#define CHECK_HIP(x)                                                      \
  do {                                                                    \
    hipError_t e_ = (x);                                                  \
    if (e_ != hipSuccess) {                                               \
      fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));      \
      exit(2);                                                            \
    }                                                                     \
  } while (0)
#define CHECK_NL(x)                                                       \
  do {                                                                    \
    int r_ = (x);                                                         \
    if (r_ != NL_OK) {                                                    \
      fprintf(stderr, "%s failed: %d %s\n", #x, r_, nl_last_error());     \
      exit(3);                                                            \
    }                                                                     \
  } while (0)

/* round-to-nearest-even float -> bf16 bits (finite inputs) */
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
static uint32_t rng_state = 12345u;
static int small_int(void) { /* -2 .. 2 */
  rng_state = rng_state * 1664525u + 1013904223u;
  return (int)((rng_state >> 24) % 5u) - 2;
}
static float uniform(float lo, float hi) {
  rng_state = rng_state * 1664525u + 1013904223u;
  return lo + (hi - lo) * (float)(rng_state >> 8) / 16777216.0f;
}
static void* dev_copy(const void* h, size_t bytes) {
  void* d = NULL;
  CHECK_HIP(hipMalloc(&d, bytes));
  CHECK_HIP(hipMemcpy(d, h, bytes, hipMemcpyHostToDevice));
  return d;
}

static int check_gemm(void) {
  const int M = 70, N = 45, K = 130;
  const int64_t ld = 136; /* a multiple of 8 covering every stored row */
  int failures = 0;
  for (int opA = 0; opA < 2; ++opA)
    for (int opB = 0; opB < 2; ++opB) {
      /* logical A[M][K], B[K][N] with small integers */
      int* a = malloc(sizeof(int) * M * K);
      int* b = malloc(sizeof(int) * K * N);
      for (int i = 0; i < M * K; ++i) a[i] = small_int();
      for (int i = 0; i < K * N; ++i) b[i] = small_int();
      const int a_rows = opA ? K : M, b_rows = opB ? N : K;
      uint16_t* ha = calloc((size_t)a_rows * ld, 2);
      uint16_t* hb = calloc((size_t)b_rows * ld, 2);
      for (int m = 0; m < M; ++m)
        for (int k = 0; k < K; ++k)
          ha[opA ? (int64_t)k * ld + m : (int64_t)m * ld + k] = to_bf16((float)a[m * K + k]);
      for (int k = 0; k < K; ++k)
        for (int n = 0; n < N; ++n)
          hb[opB ? (int64_t)n * ld + k : (int64_t)k * ld + n] = to_bf16((float)b[k * N + n]);
      void* da = dev_copy(ha, (size_t)a_rows * ld * 2);
      void* db = dev_copy(hb, (size_t)b_rows * ld * 2);
      float* dc = NULL;
      CHECK_HIP(hipMalloc((void**)&dc, (size_t)M * ld * 4));
      CHECK_NL(nl_gemm(NULL, opA, opB, M, N, K, 1.0f, da, ld, db, ld, 0.0f, dc, NL_DTYPE_F32, ld, NULL));
      CHECK_HIP(hipDeviceSynchronize());
      float* hc = malloc((size_t)M * ld * 4);
      CHECK_HIP(hipMemcpy(hc, dc, (size_t)M * ld * 4, hipMemcpyDeviceToHost));
      int bad = 0;
      for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
          long ref = 0;
          for (int k = 0; k < K; ++k) ref += (long)a[m * K + k] * b[k * N + n];
          if (hc[(int64_t)m * ld + n] != (float)ref) ++bad;
        }
      printf("gemm op%c%c %dx%dx%d: %s (%d mismatches)\n", "NT"[opA], "NT"[opB], M, N, K, bad ? "FAIL" : "exact",
             bad);
      failures += bad != 0;
      free(a); free(b); free(ha); free(hb); free(hc);
      CHECK_HIP(hipFree(da)); CHECK_HIP(hipFree(db)); CHECK_HIP(hipFree(dc));
    }
  return failures;
}

static int check_flash(void) {
  const int B = 1, H = 2, S = 100, D = 64;
  const float scale = 0.125f;
  const size_t n = (size_t)B * H * S * D;
  uint16_t *hq = malloc(n * 2), *hk = malloc(n * 2), *hv = malloc(n * 2), *ho = malloc(n * 2);
  for (size_t i = 0; i < n; ++i) {
    hq[i] = to_bf16(uniform(-1.f, 1.f));
    hk[i] = to_bf16(uniform(-1.f, 1.f));
    hv[i] = to_bf16(uniform(-1.f, 1.f));
  }
  const nl_attn_stride st = {(int64_t)H * S * D, (int64_t)S * D, D};
  void *dq = dev_copy(hq, n * 2), *dk = dev_copy(hk, n * 2), *dv = dev_copy(hv, n * 2), *dout = NULL;
  float* dl = NULL;
  CHECK_HIP(hipMalloc(&dout, n * 2));
  CHECK_HIP(hipMalloc((void**)&dl, (size_t)B * H * S * 4));
  CHECK_NL(nl_flash_attention_fwd(NULL, B, H, S, D, scale, 1, dq, st, dk, st, dv, st, dout, st, dl));
  CHECK_HIP(hipDeviceSynchronize());
  float* hl = malloc((size_t)B * H * S * 4);
  CHECK_HIP(hipMemcpy(ho, dout, n * 2, hipMemcpyDeviceToHost));
  CHECK_HIP(hipMemcpy(hl, dl, (size_t)B * H * S * 4, hipMemcpyDeviceToHost));
  int row0_mismatch = 0;
  double max_err = 0.0, max_l_err = 0.0;
  double* p = malloc(sizeof(double) * S);
  for (int h = 0; h < H; ++h) {
    const uint16_t *q = hq + (size_t)h * S * D, *k = hk + (size_t)h * S * D, *v = hv + (size_t)h * S * D;
    const uint16_t* o = ho + (size_t)h * S * D;
    /* row 0 sees only key 0: O[0] == V[0] bit for bit, L[0] == scale * q0 . k0 */
    for (int c = 0; c < D; ++c) row0_mismatch += o[c] != v[c];
    for (int i = 0; i < S; ++i) {
      double mx = -INFINITY, sum = 0.0;
      for (int j = 0; j <= i; ++j) {
        double s = 0.0;
        for (int c = 0; c < D; ++c) s += (double)from_bf16(q[i * D + c]) * from_bf16(k[j * D + c]);
        p[j] = s * scale;
        if (p[j] > mx) mx = p[j];
      }
      for (int j = 0; j <= i; ++j) sum += (p[j] = exp(p[j] - mx));
      const double lse = mx + log(sum);
      const double le = fabs(lse - hl[(size_t)h * S + i]);
      if (le > max_l_err) max_l_err = le;
      for (int c = 0; c < D; ++c) {
        double ref = 0.0;
        for (int j = 0; j <= i; ++j) ref += p[j] * from_bf16(v[j * D + c]);
        const double e = fabs(ref / sum - from_bf16(o[i * D + c]));
        if (e > max_err) max_err = e;
      }
    }
  }
  const int failures = row0_mismatch != 0 || max_err > 1e-2 || max_l_err > 1e-4;
  printf("flash fwd (1,2,100,64) causal: %d row-0 elements differ from V[0], max |O - ref| %.2e, "
         "max |L - ref| %.2e: %s\n", row0_mismatch, max_err, max_l_err, failures ? "FAIL" : "ok");
  free(hq); free(hk); free(hv); free(ho); free(hl); free(p);
  CHECK_HIP(hipFree(dq)); CHECK_HIP(hipFree(dk)); CHECK_HIP(hipFree(dv)); CHECK_HIP(hipFree(dout));
  CHECK_HIP(hipFree(dl));
  return failures;
}

static int check_ce(void) {
  const int M = 3, V = 1000;
  const int64_t ld = 1000;
  const float scale = 1.0f / M;
  uint16_t* hx = malloc((size_t)M * ld * 2);
  for (int i = 0; i < M * V; ++i) hx[i] = to_bf16(uniform(-4.f, 4.f));
  const int32_t ht[3] = {0, 999, 500};
  void *dx = dev_copy(hx, (size_t)M * ld * 2), *dt = dev_copy(ht, sizeof(ht)), *dd = NULL;
  float *dloss = NULL, *dlse = NULL;
  CHECK_HIP(hipMalloc(&dd, (size_t)M * ld * 2));
  CHECK_HIP(hipMalloc((void**)&dloss, M * 4));
  CHECK_HIP(hipMalloc((void**)&dlse, M * 4));
  CHECK_NL(nl_ce_fwd_bwd(NULL, M, V, dx, ld, dt, dloss, dlse, scale, dd, ld));
  CHECK_HIP(hipDeviceSynchronize());
  float hloss[3], hlse[3];
  uint16_t* hd = malloc((size_t)M * ld * 2);
  CHECK_HIP(hipMemcpy(hloss, dloss, sizeof(hloss), hipMemcpyDeviceToHost));
  CHECK_HIP(hipMemcpy(hlse, dlse, sizeof(hlse), hipMemcpyDeviceToHost));
  CHECK_HIP(hipMemcpy(hd, dd, (size_t)M * ld * 2, hipMemcpyDeviceToHost));
  double max_loss = 0.0, max_d = 0.0;
  for (int m = 0; m < M; ++m) {
    double mx = -INFINITY, sum = 0.0;
    for (int v = 0; v < V; ++v)
      if (from_bf16(hx[m * ld + v]) > mx) mx = from_bf16(hx[m * ld + v]);
    for (int v = 0; v < V; ++v) sum += exp(from_bf16(hx[m * ld + v]) - mx);
    const double lse = mx + log(sum), loss = lse - from_bf16(hx[m * ld + ht[m]]);
    if (fabs(loss - hloss[m]) > max_loss) max_loss = fabs(loss - hloss[m]);
    if (fabs(lse - hlse[m]) > max_loss) max_loss = fabs(lse - hlse[m]);
    for (int v = 0; v < V; ++v) {
      const double ref = (exp(from_bf16(hx[m * ld + v]) - lse) - (v == ht[m])) * scale;
      const double e = fabs(ref - from_bf16(hd[m * ld + v])) / (fabs(ref) + 1e-6);
      if (e > max_d) max_d = e;
    }
  }
  const int failures = max_loss > 1e-4 || max_d > 8e-3;
  printf("ce fwd+bwd (3,1000): max |loss, lse - ref| %.2e, max rel |dlogits - ref| %.2e: %s\n", max_loss, max_d,
         failures ? "FAIL" : "ok");
  free(hx); free(hd);
  CHECK_HIP(hipFree(dx)); CHECK_HIP(hipFree(dt)); CHECK_HIP(hipFree(dd));
  CHECK_HIP(hipFree(dloss)); CHECK_HIP(hipFree(dlse));
  return failures;
}

int main(void) {
  printf("%s\n", nl_version());
  const int failures = check_gemm() + check_flash() + check_ce();
  if (failures) {
    printf("C ABI check: %d FAILED\n", failures);
    return 1;
  }
  printf("C ABI check: all passed\n");
  return 0;
}
