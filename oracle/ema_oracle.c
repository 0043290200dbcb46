/*
 * CPU oracle for the Qwen3 attention hot path (TEST INFRASTRUCTURE ONLY).
 * See ema_oracle.h for the contract and the reference citations. Only tests,
 * the smoke entry and the bench's CPU-baseline leg load this library.
 */
#include "ema_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- bf16 */

uint16_t ora_f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline float bf(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

float ora_bf16_to_f32(uint16_t h) { return bf(h); }

void ora_f32_to_bf16_array(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = ora_f32_to_bf16(in[i]);
}

void ora_bf16_to_f32_array(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = bf(in[i]);
}

/* ----------------------------------------------------------- generator */

static inline uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

/* Standard normal for element i: Box-Muller on the pair (i/2), branch i%2. */
static inline double normal_at(uint64_t seed, size_t i) {
  uint64_t base = splitmix64(seed ^ splitmix64((uint64_t)(i >> 1)));
  uint64_t a = splitmix64(base), b = splitmix64(base + 1);
  double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0); /* (0,1] */
  double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);         /* [0,1) */
  double r = sqrt(-2.0 * log(u1));
  double t = 6.283185307179586476925 * u2;
  return (i & 1) ? r * sin(t) : r * cos(t);
}

void ora_fill_normal_bf16(uint16_t* out, size_t n, uint64_t seed, float mean, float std) {
#pragma omp parallel for schedule(static) if (n > 65536)
  for (long long i = 0; i < (long long)n; ++i)
    out[i] = ora_f32_to_bf16((float)(mean + std * normal_at(seed, (size_t)i)));
}

void ora_fill_normal_f32(float* out, size_t n, uint64_t seed, float mean, float std) {
#pragma omp parallel for schedule(static) if (n > 65536)
  for (long long i = 0; i < (long long)n; ++i)
    out[i] = (float)(mean + std * normal_at(seed, (size_t)i));
}

/* ------------------------------------------------------------- RMSNorm */

/* MLX fast::rms_norm (crates/mlx-ffi/src/ops/real/blas.rs:5-9, called for the
 * Qwen3 q/k norm at crates/serve/src/forward_qwen3.rs:62-63): the normalised
 * value is cast to the input dtype before the weight multiply. */
static void rms_norm_row(const uint16_t* x, const uint16_t* w, int D, float eps, uint16_t* y) {
  double ss = 0.0;
  for (int d = 0; d < D; ++d) ss += (double)bf(x[d]) * (double)bf(x[d]);
  double inv = 1.0 / sqrt(ss / (double)D + (double)eps);
  for (int d = 0; d < D; ++d) {
    uint16_t n = ora_f32_to_bf16((float)((double)bf(x[d]) * inv));
    y[d] = ora_f32_to_bf16(bf(n) * bf(w[d])); /* exact product of two bf16 in f32 */
  }
}

void ora_rms_norm(const uint16_t* x, const uint16_t* w, int64_t rows, int D, float eps,
                  uint16_t* out) {
  for (int64_t r = 0; r < rows; ++r) rms_norm_row(x + r * D, w, D, eps, out + r * D);
}

/* ---------------------------------------------------------------- RoPE */

/* MLX fast::rope, traditional=false, scale=1.0, dims=D
 * (crates/mlx-ffi/src/ops/real/blas.rs:67-80; callers
 * crates/serve/src/forward_qwen3.rs:67-68, crates/serve/src/compiled.rs:146-147).
 * inv_freq_i = 2^(-(i/(D/2)) * log2(theta)) and angle = pos * inv_freq_i are
 * formed in f32 as MLX does; cos/sin of that f32 angle are taken in f64. */
static void rope_row(const uint16_t* x, int pos, int D, float theta, uint16_t* y) {
  int half = D / 2;
  float lt = log2f(theta);
  for (int i = 0; i < half; ++i) {
    float inv_freq = exp2f(-((float)i / (float)half) * lt);
    float ang = (float)pos * inv_freq;
    double c = cos((double)ang), s = sin((double)ang);
    double x1 = bf(x[i]), x2 = bf(x[i + half]);
    y[i] = ora_f32_to_bf16((float)(x1 * c - x2 * s));
    y[i + half] = ora_f32_to_bf16((float)(x1 * s + x2 * c));
  }
}

void ora_rope(const uint16_t* x, const int32_t* pos, int64_t rows, int D, float theta,
              uint16_t* out) {
  for (int64_t r = 0; r < rows; ++r) rope_row(x + r * D, pos[r], D, theta, out + r * D);
}

/* ------------------------------------------------------- pre-attention */

/* Op order of crates/serve/src/forward_qwen3.rs:56-68 and :124-142 (prefill,
 * bulk slice_update at [off, off+T)) and crates/serve/src/compiled.rs:134-161
 * (decode, scatter_single at off): split q|k|v, RMSNorm q and k over D,
 * RoPE at position off+t, write k and v into the cache rows. */
int ora_pre_attention(const uint16_t* qkv, const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                      float eps, float theta, const int32_t* off, int B, int T, int Hq, int Hkv,
                      int D, uint32_t flags, uint16_t* q_out, uint16_t* kcache, uint16_t* vcache,
                      int cap) {
  for (int b = 0; b < B; ++b)
    if (off[b] < 0 || (int64_t)off[b] + T > cap) return -1;
  const int64_t row = (int64_t)(Hq + 2 * Hkv) * D;
  uint16_t* tmp = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)D);
  uint16_t* tmp2 = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)D);
  for (int b = 0; b < B; ++b) {
    for (int t = 0; t < T; ++t) {
      const uint16_t* src = qkv + ((int64_t)b * T + t) * row;
      const int pos = off[b] + t;
      for (int h = 0; h < Hq + 2 * Hkv; ++h) {
        const uint16_t* x = src + (int64_t)h * D;
        uint16_t* dst;
        if (h < Hq) {
          dst = q_out + (((int64_t)b * Hq + h) * T + t) * D;
        } else if (h < Hq + Hkv) {
          dst = kcache + (((int64_t)b * Hkv + (h - Hq)) * cap + pos) * D;
        } else {
          dst = vcache + (((int64_t)b * Hkv + (h - Hq - Hkv)) * cap + pos) * D;
          memcpy(dst, x, sizeof(uint16_t) * (size_t)D); /* v: bit copy */
          continue;
        }
        const uint16_t* cur = x;
        /* optional_qk_norm (crates/ops/src/attention.rs:57-76) applies each norm
         * independently of the other */
        const uint32_t skip = ORA_FLAG_NO_NORM | (h < Hq ? ORA_FLAG_NO_Q_NORM : ORA_FLAG_NO_K_NORM);
        if (!(flags & skip)) {
          rms_norm_row(cur, h < Hq ? q_norm_w : k_norm_w, D, eps, tmp);
          cur = tmp;
        }
        if (!(flags & ORA_FLAG_NO_ROPE)) {
          rope_row(cur, pos, D, theta, tmp2);
          cur = tmp2;
        }
        memcpy(dst, cur, sizeof(uint16_t) * (size_t)D);
      }
    }
  }
  free(tmp);
  free(tmp2);
  return 0;
}

/* ---------------------------------------------------------------- SDPA */

/* f64 reference for one (b, h, i) row. Masking is by exclusion: the additive
 * -1e9 bf16 mask of crates/serve/src/engine_ext.rs:237-260 makes
 * exp(s - 1e9 - m) exactly 0 in f32, so excluded keys contribute nothing. */
static void sdpa_row_f64(const uint16_t* q, const uint16_t* K, const uint16_t* V, int j0, int j1,
                         int D, double scale, double* sc, uint16_t* out) {
  if (j1 <= j0) {
    memset(out, 0, sizeof(uint16_t) * (size_t)D);
    return;
  }
  double m = -INFINITY;
  for (int j = j0; j < j1; ++j) {
    const uint16_t* k = K + (int64_t)j * D;
    double s = 0.0;
    for (int d = 0; d < D; ++d) s += (double)bf(q[d]) * (double)bf(k[d]);
    s *= scale;
    sc[j - j0] = s;
    if (s > m) m = s;
  }
  double l = 0.0;
  for (int j = j0; j < j1; ++j) {
    sc[j - j0] = exp(sc[j - j0] - m);
    l += sc[j - j0];
  }
  double* acc = sc + (j1 - j0);
  for (int d = 0; d < D; ++d) acc[d] = 0.0;
  for (int j = j0; j < j1; ++j) {
    const uint16_t* v = V + (int64_t)j * D;
    double p = sc[j - j0];
    for (int d = 0; d < D; ++d) acc[d] += p * (double)bf(v[d]);
  }
  for (int d = 0; d < D; ++d) out[d] = ora_f32_to_bf16((float)(acc[d] / l));
}

/* f32 arithmetic, G query heads of one kv head at once (shares each K/V row
 * read across the group). */
static void sdpa_group_f32(const float* qf, int G, const uint16_t* K, const uint16_t* V, int j0,
                           int j1, int D, float scale, float* sc, float* acc, uint16_t** outs) {
  int n = j1 - j0;
  if (n <= 0) {
    for (int g = 0; g < G; ++g) memset(outs[g], 0, sizeof(uint16_t) * (size_t)D);
    return;
  }
  float kf[512];
  for (int g = 0; g < G; ++g) sc[(int64_t)g * n] = 0.f;
  for (int j = j0; j < j1; ++j) {
    const uint16_t* k = K + (int64_t)j * D;
    for (int d = 0; d < D; ++d) kf[d] = bf(k[d]);
    for (int g = 0; g < G; ++g) {
      const float* qg = qf + (int64_t)g * D;
      float s = 0.f;
      for (int d = 0; d < D; ++d) s += qg[d] * kf[d];
      sc[(int64_t)g * n + (j - j0)] = s * scale;
    }
  }
  for (int g = 0; g < G; ++g) {
    float* sg = sc + (int64_t)g * n;
    float m = -INFINITY;
    for (int j = 0; j < n; ++j) m = sg[j] > m ? sg[j] : m;
    float l = 0.f;
    for (int j = 0; j < n; ++j) {
      sg[j] = expf(sg[j] - m);
      l += sg[j];
    }
    acc[(int64_t)g * (D + 1) + D] = l;
    for (int d = 0; d < D; ++d) acc[(int64_t)g * (D + 1) + d] = 0.f;
  }
  for (int j = j0; j < j1; ++j) {
    const uint16_t* v = V + (int64_t)j * D;
    for (int d = 0; d < D; ++d) kf[d] = bf(v[d]);
    for (int g = 0; g < G; ++g) {
      float p = sc[(int64_t)g * n + (j - j0)];
      float* a = acc + (int64_t)g * (D + 1);
      for (int d = 0; d < D; ++d) a[d] += p * kf[d];
    }
  }
  for (int g = 0; g < G; ++g) {
    float* a = acc + (int64_t)g * (D + 1);
    float inv = 1.f / a[D];
    for (int d = 0; d < D; ++d) outs[g][d] = ora_f32_to_bf16(a[d] * inv);
  }
}

static inline void key_window(const int32_t* kv_len, const int32_t* kv_begin, int b, int Tq, int i,
                              int causal, int cap, int* j0, int* j1) {
  int len = kv_len[b] < cap ? kv_len[b] : cap;
  int beg = kv_begin ? kv_begin[b] : 0;
  if (beg < 0) beg = 0;
  int end = len;
  if (causal) {
    int lim = len - Tq + i + 1;
    if (lim < end) end = lim;
  }
  *j0 = beg;
  *j1 = end;
}

void ora_sdpa(const uint16_t* q, const uint16_t* kcache, const uint16_t* vcache,
              const int32_t* kv_len, const int32_t* kv_begin, int B, int Hq, int Hkv, int Tq,
              int D, int cap, float scale, int causal, int precision, uint16_t* out) {
  const int G = Hq / Hkv;
  if (D > 512 || G < 1 || Hq % Hkv != 0) return;
  if (precision == 0) {
#pragma omp parallel
    {
      double* sc = (double*)malloc(sizeof(double) * ((size_t)cap + (size_t)D));
#pragma omp for schedule(dynamic) collapse(2)
      for (int b = 0; b < B; ++b)
        for (int h = 0; h < Hq; ++h) {
          const uint16_t* K = kcache + ((int64_t)b * Hkv + h / G) * cap * D;
          const uint16_t* V = vcache + ((int64_t)b * Hkv + h / G) * cap * D;
          for (int i = 0; i < Tq; ++i) {
            int j0, j1;
            key_window(kv_len, kv_begin, b, Tq, i, causal, cap, &j0, &j1);
            const uint16_t* qr = q + (((int64_t)b * Hq + h) * Tq + i) * D;
            uint16_t* o = out + (((int64_t)b * Tq + i) * Hq + h) * D;
            sdpa_row_f64(qr, K, V, j0, j1, D, (double)scale, sc, o);
          }
        }
      free(sc);
    }
    return;
  }
#pragma omp parallel
  {
    float* sc = (float*)malloc(sizeof(float) * (size_t)G * (size_t)cap);
    float* acc = (float*)malloc(sizeof(float) * (size_t)G * ((size_t)D + 1));
    float* qf = (float*)malloc(sizeof(float) * (size_t)G * (size_t)D);
    uint16_t** outs = (uint16_t**)malloc(sizeof(uint16_t*) * (size_t)G);
#pragma omp for schedule(dynamic) collapse(3)
    for (int b = 0; b < B; ++b)
      for (int kh = 0; kh < Hkv; ++kh)
        for (int i = 0; i < Tq; ++i) {
          const uint16_t* K = kcache + ((int64_t)b * Hkv + kh) * cap * D;
          const uint16_t* V = vcache + ((int64_t)b * Hkv + kh) * cap * D;
          int j0, j1;
          key_window(kv_len, kv_begin, b, Tq, i, causal, cap, &j0, &j1);
          for (int g = 0; g < G; ++g) {
            int h = kh * G + g;
            const uint16_t* qr = q + (((int64_t)b * Hq + h) * Tq + i) * D;
            for (int d = 0; d < D; ++d) qf[(int64_t)g * D + d] = bf(qr[d]);
            outs[g] = out + (((int64_t)b * Tq + i) * Hq + h) * D;
          }
          sdpa_group_f32(qf, G, K, V, j0, j1, D, scale, sc, acc, outs);
        }
    free(sc);
    free(acc);
    free(qf);
    free(outs);
  }
}

/* ------------------------------------------------------------- split-K */

void ora_sdpa_partial(const uint16_t* q, const uint16_t* k, const uint16_t* v, int n, int D,
                      float scale, double* m, double* l, double* acc) {
  double mm = -INFINITY;
  double* s = (double*)malloc(sizeof(double) * (size_t)(n > 0 ? n : 1));
  for (int j = 0; j < n; ++j) {
    double t = 0.0;
    for (int d = 0; d < D; ++d) t += (double)bf(q[d]) * (double)bf(k[(int64_t)j * D + d]);
    s[j] = t * (double)scale;
    if (s[j] > mm) mm = s[j];
  }
  double ll = 0.0;
  for (int d = 0; d < D; ++d) acc[d] = 0.0;
  for (int j = 0; j < n; ++j) {
    double p = exp(s[j] - mm);
    ll += p;
    for (int d = 0; d < D; ++d) acc[d] += p * (double)bf(v[(int64_t)j * D + d]);
  }
  free(s);
  *m = mm;
  *l = ll;
}

void ora_lse_merge(const double* m, const double* l, const double* acc, int P, int D,
                   double* out) {
  double M = -INFINITY;
  for (int p = 0; p < P; ++p)
    if (m[p] > M) M = m[p];
  double L = 0.0;
  for (int d = 0; d < D; ++d) out[d] = 0.0;
  for (int p = 0; p < P; ++p) {
    if (m[p] == -INFINITY) continue;
    double w = exp(m[p] - M);
    L += w * l[p];
    for (int d = 0; d < D; ++d) out[d] += w * acc[(int64_t)p * D + d];
  }
  for (int d = 0; d < D; ++d) out[d] = L > 0.0 ? out[d] / L : 0.0;
}

int ora_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* ---------------------------------------------------------------- FP8 E4M3FN
 * Restatement of crates/ops/src/fp8.rs (the FP8 cache of crates/kvcache/src/fp8.rs
 * quantises through it). Magnitude codes 0..126 enumerate the finite non-negative
 * E4M3FN values in increasing order, so "even code" is "even mantissa". */

/* fp8.rs:20-29: exponent field e = code >> 3, mantissa m = code & 7 */
static float e4m3_mag(unsigned i) {
  const unsigned e = (i >> 3) & 15u, m = i & 7u;
  if (e == 0) return (float)m * 0.001953125f; /* m * 2^-9 */
  return (1.0f + (float)m * 0.125f) * ldexpf(1.0f, (int)e - 7);
}

float ora_e4m3_value(uint8_t code) {
  const unsigned mag = code & 0x7Fu;
  if (mag == 0x7Fu) return NAN;
  const float v = e4m3_mag(mag);
  return (code & 0x80u) ? -v : v;
}

/* fp8.rs:36-64 */
float ora_e4m3fn_round(float x, uint8_t* code) {
  const int neg = x < 0.0f;
  const float ax = fminf(fabsf(x), 448.0f); /* NaN -> 448, as f32::min */
  int lo = 0, hi = 126; /* largest code with value <= ax */
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (e4m3_mag((unsigned)mid) <= ax) lo = mid;
    else hi = mid - 1;
  }
  unsigned best = (unsigned)lo;
  if (best < 126) {
    const float d0 = fabsf(ax - e4m3_mag(best)), d1 = fabsf(ax - e4m3_mag(best + 1));
    if (d1 < d0 || (d1 == d0 && ((best + 1) & 1u) == 0 && (best & 1u) != 0)) best += 1;
  }
  if (code) *code = (uint8_t)((neg ? 0x80u : 0u) | best);
  const float v = e4m3_mag(best);
  return neg ? -v : v;
}

int ora_fp8_exp_of(float r, int ref) {
  if (ref) return (int)ceilf(log2f(r));
  return (int)ceilf((float)log2((double)r));
}

/* fp8.rs:80-84: amax folds from 1e-4 with f32::max (NaN operands ignored) */
static float fp8_amax(const float* x, int n) {
  float amax = 1.0e-4f;
  for (int i = 0; i < n; ++i) amax = fmaxf(amax, fabsf(x[i]));
  return amax;
}

int ora_fp8_block_exp(const float* x, int n) { return ora_fp8_exp_of(fp8_amax(x, n) / 448.0f, 1); }

int64_t ora_fp8_exp_mismatches(int kmin, int kmax, int nulps) {
  int64_t bad = 0;
  for (int k = kmin; k <= kmax; ++k) {
    const float p = ldexpf(1.0f, k);
    float up = p, down = p;
    for (int n = 0; n < nulps; ++n) {
      bad += ora_fp8_exp_of(up, 1) != ora_fp8_exp_of(up, 0);
      bad += ora_fp8_exp_of(down, 1) != ora_fp8_exp_of(down, 0);
      up = nextafterf(up, INFINITY);
      down = nextafterf(down, 0.0f);
    }
  }
  return bad;
}

/* one 64-value block: fp8.rs:80-89 */
static void fp8_block(float* v, int n, uint8_t* codes, int8_t* exp_out) {
  const int e = ora_fp8_block_exp(v, n);
  const float scale = powf(2.0f, (float)e);
  const float inv_scale = 1.0f / scale;
  for (int i = 0; i < n; ++i) {
    float y = v[i] * inv_scale;
    if (!isnan(y)) y = y < -448.0f ? -448.0f : (y > 448.0f ? 448.0f : y); /* f32::clamp keeps NaN */
    uint8_t c;
    const float q = ora_e4m3fn_round(y, &c);
    if (codes) codes[i] = c;
    v[i] = q * scale;
  }
  if (exp_out) *exp_out = (int8_t)e;
}

void ora_fp8_round_trip(float* x, int64_t rows, int D, int n_rot) {
  const int n_nope = D - n_rot;
  for (int64_t r = 0; r < rows; ++r)
    for (int off = 0; off < n_nope; off += 64) {
      const int end = off + 64 < n_nope ? off + 64 : n_nope;
      fp8_block(x + r * D + off, end - off, NULL, NULL);
    }
}

void ora_fp8_quantize_rows(const float* x, int64_t rows, int D, uint8_t* codes, int8_t* exps) {
  float blk[64];
  for (int64_t r = 0; r < rows; ++r)
    for (int b = 0; b < D / 64; ++b) {
      memcpy(blk, x + r * D + 64 * b, sizeof(blk));
      fp8_block(blk, 64, codes + r * D + 64 * b, exps + r * (D / 64) + b);
    }
}

void ora_fp8_dequantize_rows(const uint8_t* codes, const int8_t* exps, int64_t rows, int D, float* out) {
  for (int64_t r = 0; r < rows; ++r)
    for (int i = 0; i < D; ++i)
      out[r * D + i] = ldexpf(ora_e4m3_value(codes[r * D + i]), exps[r * (D / 64) + i / 64]);
}

/* ------------------------------------------------------ int4 affine KV */

static void int4_params(float mn, float mx, float* scale, float* bias) {
  float sc = fmaxf((mx - mn) / 15.0f, 1e-7f);
  const int side = fabsf(mn) > fabsf(mx);
  sc = side ? sc : -sc;
  const float edge = side ? mn : mx;
  const float q0 = roundf(edge / sc);
  if (q0 != 0.0f) {
    *scale = edge / q0;
    *bias = edge;
  } else {
    *scale = sc;
    *bias = 0.0f;
  }
}

void ora_int4_quantize_rows(const float* x, int64_t rows, int D, uint32_t* words, uint16_t* scales,
                            uint16_t* biases) {
  const int G = D / 64;
  for (int64_t r = 0; r < rows; ++r)
    for (int g = 0; g < G; ++g) {
      const float* v = x + r * D + 64 * g;
      float mn = v[0], mx = v[0];
      for (int i = 1; i < 64; ++i) {
        mn = fminf(mn, v[i]);
        mx = fmaxf(mx, v[i]);
      }
      float scale, bias;
      int4_params(mn, mx, &scale, &bias);
      scales[r * G + g] = ora_f32_to_bf16(scale);
      biases[r * G + g] = ora_f32_to_bf16(bias);
      uint32_t* w = words + r * (D / 8) + 8 * g;
      for (int i = 0; i < 8; ++i) w[i] = 0u;
      for (int i = 0; i < 64; ++i) {
        float t = fminf(roundf((v[i] - bias) / scale), 15.0f);
        const uint32_t code = t > 0.0f ? (uint32_t)t : 0u;
        w[i / 8] |= code << (4 * (i % 8));
      }
    }
}

void ora_int4_dequantize_rows(const uint32_t* words, const uint16_t* scales, const uint16_t* biases, int64_t rows,
                              int D, float* out) {
  const int G = D / 64;
  for (int64_t r = 0; r < rows; ++r)
    for (int i = 0; i < D; ++i) {
      const uint32_t code = (words[r * (D / 8) + i / 8] >> (4 * (i % 8))) & 15u;
      const float s = bf(scales[r * G + i / 64]), b = bf(biases[r * G + i / 64]);
      out[r * D + i] = bf(ora_f32_to_bf16((float)code * s + b)); /* code * s exact in f32 */
    }
}

/* ------------------------------------------------------ gated deltanet */

void ora_gdn_scan(const float* q, const float* k, const float* v, const float* g, const float* beta,
                  double* state, double* y, int B, int T, int hk, int hv, int dk, int dv) {
  const int rep = hv / hk;
  for (int b = 0; b < B; ++b)
    for (int t = 0; t < T; ++t)
      for (int h = 0; h < hv; ++h) {
        const int kh = h / rep;
        const float* kt = k + (((int64_t)b * T + t) * hk + kh) * dk;
        const float* qt = q + (((int64_t)b * T + t) * hk + kh) * dk;
        const float* vt = v + (((int64_t)b * T + t) * hv + h) * dv;
        const double gg = g[((int64_t)b * T + t) * hv + h];
        const double bb = beta[((int64_t)b * T + t) * hv + h];
        double* S = state + ((int64_t)b * hv + h) * dv * dk;
        double* yt = y + (((int64_t)b * T + t) * hv + h) * dv;
        for (int r = 0; r < dv; ++r) {
          double* Sr = S + (int64_t)r * dk;
          double kv = 0.0;
          for (int d = 0; d < dk; ++d) {
            Sr[d] *= gg;
            kv += Sr[d] * kt[d];
          }
          const double delta = (vt[r] - kv) * bb;
          double acc = 0.0;
          for (int d = 0; d < dk; ++d) {
            Sr[d] += kt[d] * delta;
            acc += Sr[d] * qt[d];
          }
          yt[r] = acc;
        }
      }
}


/* ------------------------------------------------------------ affine quantized matmul */

static inline uint32_t qfield(const uint32_t* row, int k, int bits) {
  const int per = 32 / bits;
  return (row[k / per] >> ((k % per) * bits)) & ((1u << bits) - 1u);
}

void ora_dequantize(const uint32_t* wq, const float* scales, const float* biases, int N, int K,
                    int gs, int bits, double* w) {
  const int G = K / gs;
  const int64_t words = (int64_t)K * bits / 32;
  for (int n = 0; n < N; ++n)
    for (int k = 0; k < K; ++k)
      w[(int64_t)n * K + k] = (double)scales[(int64_t)n * G + k / gs] * qfield(wq + n * words, k, bits) +
                              (double)biases[(int64_t)n * G + k / gs];
}

void ora_qmatmul(const float* x, const uint32_t* wq, const float* scales, const float* biases,
                 int M, int N, int K, int gs, int bits, double* y) {
  const int G = K / gs;
  const int64_t words = (int64_t)K * bits / 32;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    const uint32_t* row = wq + n * words;
    for (int m = 0; m < M; ++m) {
      const float* xm = x + (int64_t)m * K;
      double acc = 0.0;
      for (int g = 0; g < G; ++g) {
        const double s = scales[(int64_t)n * G + g], b = biases[(int64_t)n * G + g];
        for (int k = g * gs; k < (g + 1) * gs; ++k) acc += (double)xm[k] * (s * qfield(row, k, bits) + b);
      }
      y[(int64_t)m * N + n] = acc;
    }
  }
}
