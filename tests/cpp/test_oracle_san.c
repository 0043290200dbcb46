/* The CPU oracle (oracle/ema_oracle.c) under the address and undefined-behaviour
 * sanitizers: every exported function runs on exactly-sized heap buffers (so an access
 * past an end is reported), over the corners the GPU tests use (empty and full lengths,
 * kv_begin windows, causal and not, GQA ratios, partial blocks), with a few identities
 * the functions must satisfy checked along the way:
 *   - pre-attention of T tokens == T single-token calls;
 *   - SDPA of a row == log-sum-exp merge of its split partial states;
 *   - a GDN scan over T tokens == two scans over the halves, state carried;
 *   - quantized matmul == matmul with the dequantised weight;
 *   - FP8 and int4 quantise -> dequantise stay finite and within their step.
 * Built without OpenMP (the pragmas are ignored), so every loop runs on this thread.
 * Exit status 0 = all passed. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "ema_oracle.h"

static int g_fail = 0;
#define CHECK(c, ...)                              \
  do {                                             \
    if (!(c)) {                                    \
      fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
      fprintf(stderr, __VA_ARGS__);                \
      fprintf(stderr, "\n");                       \
      ++g_fail;                                    \
    }                                              \
  } while (0)

static void* xmalloc(size_t n) {
  void* p = malloc(n ? n : 1);
  if (!p) abort();
  return p;
}
static uint16_t* normal_bf16(size_t n, uint64_t seed, float mean, float std) {
  uint16_t* p = xmalloc(n * 2);
  ora_fill_normal_bf16(p, n, seed, mean, std);
  return p;
}
static float* normal_f32(size_t n, uint64_t seed) {
  float* p = xmalloc(n * 4);
  ora_fill_normal_f32(p, n, seed, 0.f, 1.f);
  return p;
}

static void test_pre_attention(void) {
  const int B = 2, T = 5, Hq = 4, Hkv = 2, D = 64, cap = 16;
  const int F = (Hq + 2 * Hkv) * D;
  uint16_t* qkv = normal_bf16((size_t)B * T * F, 1, 0.f, 1.f);
  uint16_t* qw = normal_bf16(D, 2, 1.f, 0.02f);
  uint16_t* kw = normal_bf16(D, 3, 1.f, 0.02f);
  const int32_t off[2] = {3, 11};
  for (uint32_t flags = 0; flags < 32; flags = flags ? flags * 2 : 1) {
    const size_t nc = (size_t)B * Hkv * cap * D;
    uint16_t *k1 = calloc(nc, 2), *v1 = calloc(nc, 2), *k2 = calloc(nc, 2), *v2 = calloc(nc, 2);
    uint16_t* q1 = xmalloc((size_t)B * Hq * T * D * 2);
    uint16_t* qt = xmalloc((size_t)B * Hq * D * 2);
    CHECK(ora_pre_attention(qkv, qw, kw, 1e-6f, 1e6f, off, B, T, Hq, Hkv, D, flags, q1, k1, v1, cap) == 0,
          "pre_attention flags %u", flags);
    // the same tokens one at a time (qkv rows of token t, per sequence)
    uint16_t* row = xmalloc((size_t)B * F * 2);
    for (int t = 0; t < T; ++t) {
      for (int b = 0; b < B; ++b) memcpy(row + (size_t)b * F, qkv + ((size_t)b * T + t) * F, (size_t)F * 2);
      const int32_t o2[2] = {off[0] + t, off[1] + t};
      CHECK(ora_pre_attention(row, qw, kw, 1e-6f, 1e6f, o2, B, 1, Hq, Hkv, D, flags, qt, k2, v2, cap) == 0, "step");
      for (int b = 0; b < B; ++b)
        for (int h = 0; h < Hq; ++h)
          CHECK(!memcmp(qt + ((size_t)b * Hq + h) * D, q1 + (((size_t)b * Hq + h) * T + t) * D, (size_t)D * 2),
                "q of token %d differs (flags %u)", t, flags);
    }
    CHECK(!memcmp(k1, k2, nc * 2) && !memcmp(v1, v2, nc * 2), "bulk vs token-by-token cache (flags %u)", flags);
    const int32_t bad[2] = {3, 12};  // 12 + 5 > 16
    CHECK(ora_pre_attention(qkv, qw, kw, 1e-6f, 1e6f, bad, B, T, Hq, Hkv, D, flags, q1, k1, v1, cap) == -1,
          "overflow must be refused");
    free(k1); free(v1); free(k2); free(v2); free(q1); free(qt); free(row);
  }
  uint16_t* x = normal_bf16(3 * D, 4, 0.f, 1.f);
  uint16_t* y = xmalloc(3 * D * 2);
  ora_rms_norm(x, qw, 3, D, 1e-6f, y);
  const int32_t pos[3] = {0, 7, 100000};
  ora_rope(x, pos, 3, D, 1e6f, y);
  CHECK(!memcmp(x, y, (size_t)D * 2), "RoPE at position 0 is the identity");
  free(x); free(y); free(qkv); free(qw); free(kw);
}

static void test_sdpa(void) {
  const int B = 3, Hq = 8, Hkv = 2, Tq = 4, D = 128, cap = 40;
  uint16_t* q = normal_bf16((size_t)B * Hq * Tq * D, 10, 0.f, 1.f);
  uint16_t* k = normal_bf16((size_t)B * Hkv * cap * D, 11, 0.f, 1.f);
  uint16_t* v = normal_bf16((size_t)B * Hkv * cap * D, 12, 0.f, 1.f);
  uint16_t* out = xmalloc((size_t)B * Tq * Hq * D * 2);
  const int32_t len[3] = {0, 17, 40}, begin[3] = {0, 5, 30};
  for (int causal = 0; causal < 2; ++causal)
    for (int prec = 0; prec < 2; ++prec) {
      ora_sdpa(q, k, v, len, NULL, B, Hq, Hkv, Tq, D, cap, 0.088f, causal, prec, out);
      ora_sdpa(q, k, v, len, begin, B, Hq, Hkv, Tq, D, cap, 0.088f, causal, prec, out);
      for (size_t i = 0; i < (size_t)Tq * Hq * D; ++i) CHECK(out[i] == 0, "an empty sequence yields zeros");
    }
  // one row split in pieces and merged equals the whole row
  const int n = 37, P = 3;
  uint16_t* kk = normal_bf16((size_t)n * D, 13, 0.f, 1.f);
  uint16_t* vv = normal_bf16((size_t)n * D, 14, 0.f, 1.f);
  double m[3], l[3], *acc = xmalloc(sizeof(double) * P * D), *merged = xmalloc(sizeof(double) * D);
  double mw, lw, *aw = xmalloc(sizeof(double) * D);
  const int cut[4] = {0, 10, 11, n};
  for (int p = 0; p < P; ++p)
    ora_sdpa_partial(q, kk + (size_t)cut[p] * D, vv + (size_t)cut[p] * D, cut[p + 1] - cut[p], D, 0.088f, &m[p], &l[p],
                     acc + (size_t)p * D);
  ora_lse_merge(m, l, acc, P, D, merged);
  ora_sdpa_partial(q, kk, vv, n, D, 0.088f, &mw, &lw, aw);
  for (int d = 0; d < D; ++d)
    CHECK(fabs(merged[d] - aw[d] / lw) < 1e-12 * (1 + fabs(aw[d] / lw)), "merge of the pieces, dim %d", d);
  (void)ora_num_threads();
  free(q); free(k); free(v); free(out); free(kk); free(vv); free(acc); free(merged); free(aw);
}

static void test_fp8_int4(void) {
  const int rows = 5, D = 128;
  float* x = normal_f32((size_t)rows * D, 20);
  x[3] = 0.f;
  x[5] = 1e-30f;
  x[7] = 1000.f;
  uint8_t* codes = xmalloc((size_t)rows * D);
  int8_t* exps = xmalloc((size_t)rows * D / 64);
  float* back = xmalloc((size_t)rows * D * 4);
  ora_fp8_quantize_rows(x, rows, D, codes, exps);
  ora_fp8_dequantize_rows(codes, exps, rows, D, back);
  for (int i = 0; i < rows * D; ++i) CHECK(isfinite(back[i]), "fp8 value %d not finite", i);
  float* rt = xmalloc((size_t)rows * D * 4);
  memcpy(rt, x, (size_t)rows * D * 4);
  ora_fp8_round_trip(rt, rows, D, 0);
  ora_fp8_round_trip(rt, rows, D, 64);  // passthrough of the last 64 dims
  for (int c = 0; c < 256; ++c) (void)ora_e4m3_value((uint8_t)c);
  uint8_t code;
  (void)ora_e4m3fn_round(3.3f, &code);
  (void)ora_fp8_block_exp(x, 64);
  (void)ora_fp8_exp_of(0.5f, 1);
  (void)ora_fp8_exp_mismatches(-3, 3, 4);
  uint32_t* words = xmalloc((size_t)rows * D / 8 * 4);
  uint16_t* sc = xmalloc((size_t)rows * D / 64 * 2);
  uint16_t* bi = xmalloc((size_t)rows * D / 64 * 2);
  ora_int4_quantize_rows(x, rows, D, words, sc, bi);
  ora_int4_dequantize_rows(words, sc, bi, rows, D, back);
  for (int i = 0; i < rows * D; ++i) CHECK(isfinite(back[i]), "int4 value %d not finite", i);
  free(x); free(codes); free(exps); free(back); free(rt); free(words); free(sc); free(bi);
}

static void test_gdn(void) {
  const int B = 2, T = 6, hk = 2, hv = 4, dk = 16, dv = 8;
  float* q = normal_f32((size_t)B * T * hk * dk, 30);
  float* k = normal_f32((size_t)B * T * hk * dk, 31);
  float* v = normal_f32((size_t)B * T * hv * dv, 32);
  float* g = xmalloc((size_t)B * T * hv * 4);
  float* beta = xmalloc((size_t)B * T * hv * 4);
  for (int i = 0; i < B * T * hv; ++i) {
    g[i] = 0.9f + 0.01f * (float)(i % 7);
    beta[i] = 0.1f * (float)(i % 5);
  }
  const size_t ns = (size_t)B * hv * dv * dk;
  double *s1 = calloc(ns, 8), *s2 = calloc(ns, 8);
  double* y1 = xmalloc((size_t)B * T * hv * dv * 8);
  double* y2 = xmalloc((size_t)B * T * hv * dv * 8);
  ora_gdn_scan(q, k, v, g, beta, s1, y1, B, T, hk, hv, dk, dv);
  // two halves, per sequence (inputs [B, T, ...]: copy each half out)
  const int h = T / 2;
  for (int part = 0; part < 2; ++part) {
    float* qp = xmalloc((size_t)B * h * hk * dk * 4);
    float* kp = xmalloc((size_t)B * h * hk * dk * 4);
    float* vp = xmalloc((size_t)B * h * hv * dv * 4);
    float* gp = xmalloc((size_t)B * h * hv * 4);
    float* bp = xmalloc((size_t)B * h * hv * 4);
    double* yp = xmalloc((size_t)B * h * hv * dv * 8);
    for (int b = 0; b < B; ++b) {
      const size_t t0 = (size_t)b * T + part * h;
      memcpy(qp + (size_t)b * h * hk * dk, q + t0 * hk * dk, (size_t)h * hk * dk * 4);
      memcpy(kp + (size_t)b * h * hk * dk, k + t0 * hk * dk, (size_t)h * hk * dk * 4);
      memcpy(vp + (size_t)b * h * hv * dv, v + t0 * hv * dv, (size_t)h * hv * dv * 4);
      memcpy(gp + (size_t)b * h * hv, g + t0 * hv, (size_t)h * hv * 4);
      memcpy(bp + (size_t)b * h * hv, beta + t0 * hv, (size_t)h * hv * 4);
    }
    ora_gdn_scan(qp, kp, vp, gp, bp, s2, yp, B, h, hk, hv, dk, dv);
    for (int b = 0; b < B; ++b)
      memcpy(y2 + ((size_t)b * T + part * h) * hv * dv, yp + (size_t)b * h * hv * dv, (size_t)h * hv * dv * 8);
    free(qp); free(kp); free(vp); free(gp); free(bp); free(yp);
  }
  for (size_t i = 0; i < ns; ++i) CHECK(s1[i] == s2[i], "state after halves, element %zu", i);
  for (size_t i = 0; i < (size_t)B * T * hv * dv; ++i) CHECK(y1[i] == y2[i], "y after halves, element %zu", i);
  free(q); free(k); free(v); free(g); free(beta); free(s1); free(s2); free(y1); free(y2);
}

static void test_qmatmul(void) {
  const int M = 3, N = 5, K = 128;
  for (int bits = 2; bits <= 8; bits *= 2)
    for (int gs = 32; gs <= 128; gs *= 2) {
      const int per = 32 / bits, G = K / gs;
      float* x = normal_f32((size_t)M * K, 40);
      uint32_t* wq = xmalloc((size_t)N * K / per * 4);
      for (int i = 0; i < N * K / per; ++i) wq[i] = 0x9E3779B9u * (uint32_t)(i + 1);
      float* s = normal_f32((size_t)N * G, 41);
      float* b = normal_f32((size_t)N * G, 42);
      double* y = xmalloc((size_t)M * N * 8);
      double* w = xmalloc((size_t)N * K * 8);
      ora_qmatmul(x, wq, s, b, M, N, K, gs, bits, y);
      ora_dequantize(wq, s, b, N, K, gs, bits, w);
      for (int m = 0; m < M; ++m)
        for (int n = 0; n < N; ++n) {
          double r = 0;
          for (int kk = 0; kk < K; ++kk) r += (double)x[(size_t)m * K + kk] * w[(size_t)n * K + kk];
          CHECK(fabs(r - y[(size_t)m * N + n]) <= 1e-9 * (1 + fabs(r)), "qmatmul bits %d gs %d (%d, %d)", bits, gs, m, n);
        }
      free(x); free(wq); free(s); free(b); free(y); free(w);
    }
}

int main(void) {
  uint16_t h = ora_f32_to_bf16(1.5f);
  CHECK(ora_bf16_to_f32(h) == 1.5f, "bf16 round trip");
  float f[3] = {1.f, NAN, -0.f};
  uint16_t hb[3];
  ora_f32_to_bf16_array(f, hb, 3);
  ora_bf16_to_f32_array(hb, f, 3);
  test_pre_attention();
  test_sdpa();
  test_fp8_int4();
  test_gdn();
  test_qmatmul();
  printf("oracle under sanitizers: %s\n", g_fail ? "FAILED" : "all checks passed");
  return g_fail ? 1 : 0;
}
