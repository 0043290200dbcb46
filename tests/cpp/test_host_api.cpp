// Tests of the C++ host API (engine-mlx_amd/host/ema_host.hpp), in the shape of
// the reference's own unit tests for the same surface:
//   crates/kvcache/tests/lib.rs     (KvCache trait contract, InMemoryCache)
//   crates/kvcache/tests/concat.rs  (new_is_empty, reset, get bails when empty)
//   crates/attention/tests/gqa.rs   (GqaConfig constructible, gqa_attention errors)
// plus GPU checks of StaticCache, RotatingCache, Fp8Cache, gqa_attention (projections, norms, RoPE,
// cache write, attention, o_proj), sliding_window_attention and qkv_attention against
// the CPU oracle chain ora_qmatmul -> ora_pre_attention -> ora_sdpa -> ora_qmatmul.
//
// usage: test_host_api cpu|gpu   (exit status 0 = all passed)
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "ema_host.hpp"
#include "ema_oracle.h"

using namespace ema;

static int g_failed = 0;

#define EXPECT(cond)                                                             \
  do {                                                                           \
    if (!(cond)) {                                                               \
      std::fprintf(stderr, "  EXPECT failed %s:%d: %s\n", __FILE__, __LINE__, #cond); \
      throw std::runtime_error("expectation failed");                           \
    }                                                                            \
  } while (0)

static void run(const char* name, const std::function<void()>& fn) {
  try {
    fn();
    std::printf("ok   %s\n", name);
  } catch (const std::exception& e) {
    std::printf("FAIL %s: %s\n", name, e.what());
    ++g_failed;
  }
  std::fflush(stdout);
}

template <class F>
static std::string error_of(F&& f) {
  try {
    f();
  } catch (const Error& e) {
    return e.what();
  }
  return "";
}

// ------------------------------------------------------------------ CPU
struct InMemoryCache : KvCache {
  size_t seq_len = 0;
  void append(const Ctx&, const Array&, const Array&) override { seq_len += 1; }
  std::pair<Array, Array> get(const Ctx&) const override { return {Array{}, Array{}}; }
  size_t len() const override { return seq_len; }
  void reset() override { seq_len = 0; }
  size_t memory_bytes() const override { return seq_len * 16; }
};

static void cpu_tests() {
  run("kvcache_is_empty_default_uses_len", [] {
    InMemoryCache c;
    EXPECT(c.is_empty());
    EXPECT(c.memory_bytes() == 0);
  });
  run("kvcache_append_updates_len_and_not_empty", [] {
    InMemoryCache c;
    c.append(Ctx{}, Array{}, Array{});
    EXPECT(c.len() == 1 && !c.is_empty());
    c.reset();
    EXPECT(c.is_empty());
  });
  run("gqa_config_is_constructible", [] {
    GqaConfig cfg{32, 8, 128, 10000.0f, 1e-6f, true};
    EXPECT(cfg.n_heads == 32 && cfg.n_kv_heads == 8);
    SlidingWindowConfig sw{cfg, 4096};
    EXPECT(sw.gqa.head_dim == 128 && sw.window_size == 4096);
  });
  run("error_carries_status_code", [] {
    Error e(EMA_ERR_CAPACITY, "static KV overflow offset=4096 cap=4096");
    EXPECT(e.code() == EMA_ERR_CAPACITY);
    EXPECT(std::string(e.what()).find("overflow") != std::string::npos);
  });
}

// ------------------------------------------------------------------ GPU
static void* upload(const std::vector<uint16_t>& h) {
  void* d = nullptr;
  if (hipMalloc(&d, h.size() * 2) != hipSuccess) throw std::runtime_error("hipMalloc");
  if (hipMemcpy(d, h.data(), h.size() * 2, hipMemcpyHostToDevice) != hipSuccess) throw std::runtime_error("H2D");
  return d;
}
static std::vector<uint16_t> download(const void* d, size_t n) {
  std::vector<uint16_t> h(n);
  if (hipMemcpy(h.data(), d, n * 2, hipMemcpyDeviceToHost) != hipSuccess) throw std::runtime_error("D2H");
  return h;
}
static std::vector<uint16_t> normal(size_t n, uint64_t seed, float mean = 0.f, float std = 1.f) {
  std::vector<uint16_t> h(n);
  ora_fill_normal_bf16(h.data(), n, seed, mean, std);
  return h;
}
static void expect_close(const std::vector<uint16_t>& got, const std::vector<uint16_t>& ref, const char* what) {
  double mx = 0, sum = 0;
  for (size_t i = 0; i < got.size(); ++i) {
    double d = std::fabs((double)ora_bf16_to_f32(got[i]) - (double)ora_bf16_to_f32(ref[i]));
    if (!(d == d)) d = 1e9;
    mx = d > mx ? d : mx;
    sum += d;
  }
  const double mean = sum / (double)got.size();
  std::printf("     %s: max_abs=%.3e mean_abs=%.3e\n", what, mx, mean);
  EXPECT(mx <= 2e-2 && mean <= 2e-3);
}
// The layer output after o_proj: the same bar, with the max-abs bound widened by one bf16
// rounding step of the value itself (2^-7 relative) for outputs above 1.
static void expect_close_out(const std::vector<uint16_t>& got, const std::vector<uint16_t>& ref, const char* what) {
  double worst = 0, sum = 0;
  for (size_t i = 0; i < got.size(); ++i) {
    const double r = ora_bf16_to_f32(ref[i]);
    double d = std::fabs((double)ora_bf16_to_f32(got[i]) - r);
    if (!(d == d)) d = 1e9;
    worst = std::max(worst, d / (2e-2 + std::fabs(r) / 128.0));
    sum += d;
  }
  const double mean = sum / (double)got.size();
  std::printf("     %s: worst/bound=%.3f mean_abs=%.3e\n", what, worst, mean);
  EXPECT(worst <= 1.0 && mean <= 2e-3);
}

// MLX affine 4-bit weights, group 64, for y = x W^T with W [N, K]: random codes,
// scales `scale` * (1 + N(0, 0.1)) and biases -7.5 * scale (centred codes).
struct HostQW {
  std::vector<uint32_t> w;
  std::vector<uint16_t> s, b;
  int N = 0, K = 0;
};
static HostQW random_qw(int N, int K, uint64_t seed, float scale) {
  HostQW q;
  q.N = N;
  q.K = K;
  q.w.resize((size_t)N * K / 8);
  q.s.resize((size_t)N * K / 64);
  q.b.resize(q.s.size());
  uint64_t st = seed * 0x9E3779B97F4A7C15ull + 12345;
  for (auto& x : q.w) {
    st ^= st << 13;
    st ^= st >> 7;
    st ^= st << 17;
    x = (uint32_t)(st >> 16);
  }
  auto noise = normal(q.s.size(), seed + 7, 1.f, 0.1f);
  for (size_t i = 0; i < q.s.size(); ++i) {
    const float sc = scale * ora_bf16_to_f32(noise[i]);
    q.s[i] = ora_f32_to_bf16(sc);
    q.b[i] = ora_f32_to_bf16(-7.5f * ora_bf16_to_f32(q.s[i]));
  }
  return q;
}
// y [M, N] bf16 = x [M, K] W^T through the oracle (f64 sums, one rounding to bf16).
static std::vector<uint16_t> ora_project(const std::vector<uint16_t>& x, int M, const HostQW& q) {
  std::vector<float> xf(x.size()), sf(q.s.size()), bf(q.b.size());
  ora_bf16_to_f32_array(x.data(), xf.data(), x.size());
  ora_bf16_to_f32_array(q.s.data(), sf.data(), q.s.size());
  ora_bf16_to_f32_array(q.b.data(), bf.data(), q.b.size());
  std::vector<double> y((size_t)M * q.N);
  ora_qmatmul(xf.data(), q.w.data(), sf.data(), bf.data(), M, q.N, q.K, 64, 4, y.data());
  std::vector<uint16_t> out(y.size());
  for (size_t i = 0; i < y.size(); ++i) out[i] = ora_f32_to_bf16((float)y[i]);
  return out;
}
static void* upload_bytes(const void* h, size_t n) {
  void* d = nullptr;
  if (hipMalloc(&d, n) != hipSuccess) throw std::runtime_error("hipMalloc");
  if (hipMemcpy(d, h, n, hipMemcpyHostToDevice) != hipSuccess) throw std::runtime_error("H2D");
  return d;
}
struct DevQW {
  QuantWeights qw;
  explicit DevQW(const HostQW& h) {
    qw.weight = Array{upload_bytes(h.w.data(), h.w.size() * 4), {h.N, h.K / 8}, {}};
    qw.scales = Array{upload(h.s), {h.N, h.K / 64}, {}};
    qw.biases = Array{upload(h.b), {h.N, h.K / 64}, {}};
  }
  ~DevQW() {
    for (void* p : {qw.weight.data, qw.scales.data, qw.biases.data}) (void)hipFree(p);
  }
};

// Equal as values (+0 and -0 alike), element by element.
static bool same_values(const std::vector<uint16_t>& a, const std::vector<uint16_t>& b) {
  if (a.size() != b.size()) return false;
  for (size_t i = 0; i < a.size(); ++i)
    if (ora_bf16_to_f32(a[i]) != ora_bf16_to_f32(b[i])) return false;
  return true;
}

// Rows [r0, r0 + n) of each head of a [H, cap, D] bf16 cache replaced by their FP8 round
// trip (exact in bf16: a 4-bit significand times a power of two), the last n_rot dims of
// each row passing through (fp8.rs:69-92).
static void fp8_round_trip_rows(std::vector<uint16_t>& c, int H, int cap, int D, int r0, int n, int n_rot = 0) {
  std::vector<float> f((size_t)n * D);
  for (int h = 0; h < H; ++h) {
    uint16_t* rows = &c[((size_t)h * cap + r0) * D];
    ora_bf16_to_f32_array(rows, f.data(), f.size());
    ora_fp8_round_trip(f.data(), n, D, n_rot);
    for (size_t i = 0; i < f.size(); ++i) rows[i] = ora_f32_to_bf16(f[i]);
  }
}

// Checks that `held` ([H, n, D] decoded FP8 rows) is the oracle's round-tripped cache `ref`
// ([H, cap, D], rows [0, n)) to within one FP8 step: |held - ref| <= |ref| / 4 + 2^-7 s,
// with s = the block scale 2^ceil(log2(amax / 448)) of the oracle's 64-value block (a
// neighbouring code, or the block's scale one step up), on at most `max_frac` of the
// values. Then copies `held` into `ref`.
static void adopt_fp8_rows(std::vector<uint16_t>& ref, const std::vector<uint16_t>& held, int H, int cap, int n, int D,
                           const char* what, double max_frac) {
  size_t differ = 0, total = (size_t)H * n * D;
  double worst = 0;
  for (int h = 0; h < H; ++h)
    for (int r = 0; r < n; ++r)
      for (int b = 0; b < D; b += 64) {
        const uint16_t* want = &ref[((size_t)h * cap + r) * D + b];
        const uint16_t* got = &held[((size_t)h * n + r) * D + b];
        float amax = 1e-4f;
        for (int i = 0; i < 64; ++i) amax = std::max(amax, std::fabs(ora_bf16_to_f32(want[i])));
        const float s = std::ldexp(1.0f, (int)std::ceil(std::log2(amax / 448.0f)));
        for (int i = 0; i < 64; ++i) {
          const float w = ora_bf16_to_f32(want[i]), g = ora_bf16_to_f32(got[i]);
          if (g == w) continue;
          ++differ;
          worst = std::max(worst, (double)std::fabs(g - w) / (std::fabs(w) / 4 + s / 128));
        }
      }
  std::printf("     %s: %zu of %zu values on another FP8 code, worst/bound=%.3f\n", what, differ, total, worst);
  EXPECT(worst <= 1.0 && (double)differ <= max_frac * (double)total);
  for (int h = 0; h < H; ++h) std::copy_n(&held[(size_t)h * n * D], (size_t)n * D, &ref[(size_t)h * cap * D]);
}

// The reference layer on the host (gqa.rs:62-107 with the oracle's ops): q|k|v
// projections, norms (null = absent), RoPE and the cache write at `off`, SDPA over
// [begin, off + T) (causal for T > 1), o_proj. kref/vref are the chronological caches.
struct OracleLayer {
  HostQW q, k, v, o;
  int Hq, Hkv, D, cap;
  std::vector<uint16_t> kref, vref;
  bool fp8 = false;  // the cache keeps the FP8 round trip of each written row (fp8.rs:71-92)
  int n_rot = 0;     // ... with this unquantised RoPE tail
  // FP8 caches: the rows the device cache holds after the call ([Hkv, off + T, D], decoded),
  // which replace the oracle's rows. The device's projected k/v differ from the oracle's
  // within the projection's bf16 tolerance, and one FP8 step is 2^5 bf16 steps, so the
  // caller pins these rows otherwise (as the FP8 round trip of the rows a bf16 cache gets).
  const std::vector<uint16_t>* k_held = nullptr;
  const std::vector<uint16_t>* v_held = nullptr;
  OracleLayer(int hidden, int Hq_, int Hkv_, int D_, int cap_, uint64_t seed)
      : q(random_qw(Hq_ * D_, hidden, seed, 0.0068f)), k(random_qw(Hkv_ * D_, hidden, seed + 1, 0.0068f)),
        v(random_qw(Hkv_ * D_, hidden, seed + 2, 0.0068f)), o(random_qw(hidden, Hq_ * D_, seed + 3, 0.0034f)),
        Hq(Hq_), Hkv(Hkv_), D(D_), cap(cap_), kref((size_t)Hkv_ * cap_ * D_, 0), vref((size_t)Hkv_ * cap_ * D_, 0) {}
  std::vector<uint16_t> run(const std::vector<uint16_t>& x, int T, int off, int begin, const uint16_t* qw,
                            const uint16_t* kw) {
    const int F = (Hq + 2 * Hkv) * D;
    auto pq = ora_project(x, T, q), pk = ora_project(x, T, k), pv = ora_project(x, T, v);
    std::vector<uint16_t> qkv((size_t)T * F);
    for (int t = 0; t < T; ++t) {
      std::copy_n(&pq[(size_t)t * Hq * D], Hq * D, &qkv[(size_t)t * F]);
      std::copy_n(&pk[(size_t)t * Hkv * D], Hkv * D, &qkv[(size_t)t * F + Hq * D]);
      std::copy_n(&pv[(size_t)t * Hkv * D], Hkv * D, &qkv[(size_t)t * F + (Hq + Hkv) * D]);
    }
    const uint32_t flags = (qw ? 0u : (uint32_t)ORA_FLAG_NO_Q_NORM) | (kw ? 0u : (uint32_t)ORA_FLAG_NO_K_NORM);
    std::vector<uint16_t> qh((size_t)Hq * T * D), attn((size_t)T * Hq * D);
    int32_t o32 = off, len = off + T, b32 = begin;
    if (ora_pre_attention(qkv.data(), qw, kw, 1e-6f, 1e6f, &o32, 1, T, Hq, Hkv, D, flags, qh.data(), kref.data(),
                          vref.data(), cap) != 0)
      throw std::runtime_error("oracle overflow");
    if (fp8) {
      fp8_round_trip_rows(kref, Hkv, cap, D, off, T, n_rot);
      fp8_round_trip_rows(vref, Hkv, cap, D, off, T, n_rot);
      for (auto [held, c] : {std::pair{k_held, &kref}, std::pair{v_held, &vref}})
        if (held)
          for (int h = 0; h < Hkv; ++h)
            std::copy_n(&(*held)[(size_t)h * (off + T) * D], (size_t)(off + T) * D, &(*c)[(size_t)h * cap * D]);
    }
    ora_sdpa(qh.data(), kref.data(), vref.data(), &len, &b32, 1, Hq, Hkv, T, D, cap, 1.0f / std::sqrt((float)D),
             T > 1 ? 1 : 0, 0, attn.data());
    return ora_project(attn, T, o);
  }
};

static void gpu_tests() {
  const int Hkv = 2, D = 128, cap = 256, Hq = 8, hidden = 1024;
  const int F = (Hq + 2 * Hkv) * D;
  const GqaConfig cfg{Hq, Hkv, D, 1e6f, 1e-6f, true};
  // one arena for every layer call below (gqa_workspace_bytes covers the largest)
  Ctx ctx;
  ctx.workspace_bytes = gqa_workspace_bytes(cfg, hidden, 64, cap);
  if (hipMalloc(&ctx.workspace, ctx.workspace_bytes) != hipSuccess ||
      hipMemset(ctx.workspace, 0, ctx.workspace_bytes) != hipSuccess)
    throw std::runtime_error("hipMalloc arena");

  run("static_cache_new_is_empty", [&] {
    StaticCache c(Hkv, cap, D);
    EXPECT(c.len() == 0 && c.is_empty());
    EXPECT(c.memory_bytes() == (size_t)2 * Hkv * cap * D * 2);
    EXPECT(error_of([&] { c.get(Ctx{}); }).find("KV cache is empty") != std::string::npos);
  });
  run("static_cache_append_then_get", [&] {
    StaticCache c(Hkv, cap, D);
    const int T1 = 5, T2 = 3;
    auto k1 = normal((size_t)Hkv * T1 * D, 1), v1 = normal((size_t)Hkv * T1 * D, 2);
    auto k2 = normal((size_t)Hkv * T2 * D, 3), v2 = normal((size_t)Hkv * T2 * D, 4);
    void *dk1 = upload(k1), *dv1 = upload(v1), *dk2 = upload(k2), *dv2 = upload(v2);
    c.append(Ctx{}, Array{dk1, {1, Hkv, T1, D}, {}}, Array{dv1, {1, Hkv, T1, D}, {}});
    c.append(Ctx{}, Array{dk2, {1, Hkv, T2, D}, {}}, Array{dv2, {1, Hkv, T2, D}, {}});
    (void)hipDeviceSynchronize();
    EXPECT(c.len() == T1 + T2);
    auto kv = c.get(Ctx{});
    EXPECT(kv.first.shape[2] == T1 + T2 && kv.first.strides[1] == (int64_t)cap * D);
    auto all = download(kv.first.data, (size_t)Hkv * cap * D);
    for (int h = 0; h < Hkv; ++h)
      for (int t = 0; t < T1 + T2; ++t)
        for (int d = 0; d < D; ++d) {
          uint16_t want = t < T1 ? k1[((size_t)h * T1 + t) * D + d] : k2[((size_t)h * T2 + t - T1) * D + d];
          EXPECT(all[((size_t)h * cap + t) * D + d] == want);
        }
    for (void* p : {dk1, dv1, dk2, dv2}) (void)hipFree(p);
  });
  run("static_cache_overflow_bails", [&] {
    StaticCache c(1, 4, D);
    auto k = normal((size_t)5 * D, 5);
    void* dk = upload(k);
    std::string e = error_of([&] { c.append(Ctx{}, Array{dk, {1, 1, 5, D}, {}}, Array{dk, {1, 1, 5, D}, {}}); });
    EXPECT(e.find("static KV overflow") != std::string::npos);
    EXPECT(c.len() == 0);
    (void)hipFree(dk);
  });
  run("gqa_attention_rejects_bad_arguments", [&] {
    // every case throws before any launch (fake device pointers are never read)
    StaticCache c(Hkv, cap, D);
    void* fake = (void*)0x1000;
    auto qw_of = [&](int N, int K) {
      QuantWeights w;
      w.weight = Array{fake, {N, K / 8}, {}};
      w.scales = w.biases = Array{fake, {N, K / 64}, {}};
      return w;
    };
    GqaWeights w{qw_of(Hq * D, hidden), qw_of(Hkv * D, hidden), qw_of(Hkv * D, hidden), qw_of(hidden, Hq * D),
                 std::nullopt, std::nullopt};
    Array x{fake, {1, 4, hidden}, {}};
    EXPECT(error_of([&] { gqa_attention(ctx, Array{fake, {4, hidden}, {}}, w, c, cfg, 0); }).find("x must be") !=
           std::string::npos);
    GqaConfig bad{12, 8, D, 1e6f, 1e-6f, true};
    EXPECT(!error_of([&] { gqa_attention(ctx, x, w, c, bad, 0); }).empty());
    EXPECT(error_of([&] { gqa_attention(ctx, x, w, c, cfg, cap - 2); }).find("static KV overflow") !=
           std::string::npos);
    GqaWeights plain = w;
    plain.k_proj.group_size = 0;
    EXPECT(error_of([&] { gqa_attention(ctx, x, plain, c, cfg, 0); }).find("plain") != std::string::npos);
    GqaWeights mx = w;
    mx.v_proj.mode = "mxfp4";
    EXPECT(error_of([&] { gqa_attention(ctx, x, mx, c, cfg, 0); }).find("affine only") != std::string::npos);
    GqaWeights wrong = w;
    wrong.o_proj = qw_of(hidden, hidden * 2);
    EXPECT(error_of([&] { gqa_attention(ctx, x, wrong, c, cfg, 0); }).find("o_proj: expected weight") !=
           std::string::npos);
    Ctx small = ctx;
    small.workspace_bytes = 4096;
    try {
      gqa_attention(small, x, w, c, cfg, 0);
      EXPECT(false);
    } catch (const Error& e) {
      EXPECT(e.code() == EMA_ERR_WORKSPACE && std::string(e.what()).find("ctx workspace") != std::string::npos);
    }
    EXPECT(c.is_empty());
  });
  // gqa.rs:62-107 end to end: prefill 37 tokens, then 4 decode steps
  auto layer_case = [&](const char* name, bool q_norm, bool k_norm, uint64_t seed) {
    run(name, [&] {
      StaticCache c(Hkv, cap, D);
      OracleLayer ref(hidden, Hq, Hkv, D, cap, seed);
      DevQW dq(ref.q), dk(ref.k), dv(ref.v), dout(ref.o);
      auto qw = normal(D, seed + 10, 1.f, 0.02f), kw = normal(D, seed + 11, 1.f, 0.02f);
      void *dqw = upload(qw), *dkw = upload(kw);
      GqaWeights w{dq.qw, dk.qw, dv.qw, dout.qw, std::nullopt, std::nullopt};
      if (q_norm) w.q_norm = Array{dqw, {D}, {}};
      if (k_norm) w.k_norm = Array{dkw, {D}, {}};
      const int T = 37, steps = 4;
      for (int step = 0; step <= steps; ++step) {
        const int t = step == 0 ? T : 1, off = step == 0 ? 0 : T + step - 1;
        auto x = normal((size_t)t * hidden, seed + 100 + step);
        void* dx = upload(x);
        Array y = gqa_attention(ctx, Array{dx, {1, t, hidden}, {}}, w, c, cfg, off);
        (void)hipDeviceSynchronize();
        EXPECT(c.len() == (size_t)(off + t) && y.shape == std::vector<int64_t>({1, t, hidden}));
        auto want = ref.run(x, t, off, 0, q_norm ? qw.data() : nullptr, k_norm ? kw.data() : nullptr);
        expect_close_out(download(y.data, want.size()), want, step == 0 ? "layer prefill" : "layer decode");
        (void)hipFree(dx);
      }
      // V rows hold the v projection's output: within its rounding of the oracle's (the
      // bit copy of the projected row into the cache is pinned by the pre-attention tests)
      expect_close_out(download(c.desc().v, ref.vref.size()), ref.vref, "V cache");
      c.reset();
      EXPECT(c.is_empty() && c.memory_bytes() == (size_t)2 * Hkv * cap * D * 2);
      (void)hipFree(dqw);
      (void)hipFree(dkw);
    });
  };
  layer_case("gqa_attention_projections_prefill_then_decode_matches_oracle", true, true, 1000);
  layer_case("gqa_attention_k_norm_only_matches_oracle", false, true, 2000);
  layer_case("gqa_attention_without_norms_matches_oracle", false, false, 3000);
  run("qkv_attention_prefill_then_decode_matches_oracle", [&] {
    StaticCache c(Hkv, cap, D);
    auto qw = normal(D, 10, 1.f, 0.02f), kw = normal(D, 11, 1.f, 0.02f);
    void *dqw = upload(qw), *dkw = upload(kw);
    std::vector<uint16_t> kref((size_t)Hkv * cap * D, 0), vref((size_t)Hkv * cap * D, 0);
    const float scale = 1.0f / std::sqrt((float)D);
    const int T = 37, steps = 4;
    for (int step = 0; step <= steps; ++step) {
      const int t = step == 0 ? T : 1, off = step == 0 ? 0 : T + step - 1;
      auto qkv = normal((size_t)t * F, 100 + step);
      void* dqkv = upload(qkv);
      Array out = qkv_attention(ctx, Array{dqkv, {1, t, F}, {}}, Array{dqw, {D}, {}}, Array{dkw, {D}, {}}, c, cfg, off);
      (void)hipDeviceSynchronize();
      EXPECT(c.len() == (size_t)(off + t));
      std::vector<uint16_t> q((size_t)Hq * t * D), ref((size_t)t * Hq * D);
      int32_t o32 = off, len = off + t;
      EXPECT(ora_pre_attention(qkv.data(), qw.data(), kw.data(), 1e-6f, 1e6f, &o32, 1, t, Hq, Hkv, D, 0, q.data(),
                               kref.data(), vref.data(), cap) == 0);
      ora_sdpa(q.data(), kref.data(), vref.data(), &len, nullptr, 1, Hq, Hkv, t, D, cap, scale, 1, 0, ref.data());
      expect_close(download(out.data, ref.size()), ref, step == 0 ? "prefill" : "decode");
      (void)hipFree(dqkv);
    }
    EXPECT(download(c.desc().v, vref.size()) == vref);
    Array ok{(void*)0x1000, {1, 4, (int64_t)F}, {}};
    EXPECT(error_of([&] { qkv_attention(ctx, Array{(void*)0x1000, {1, 4, 100}, {}}, std::nullopt, std::nullopt, c,
                                        cfg, 0); })
               .find("qkv must be") != std::string::npos);
    EXPECT(error_of([&] { qkv_attention(ctx, ok, std::nullopt, std::nullopt, c, cfg, cap - 2); })
               .find("static KV overflow") != std::string::npos);
    (void)hipFree(dqw);
    (void)hipFree(dkw);
  });
  // ---- RotatingCache (crates/kvcache/src/rotating.rs; tests in crates/kvcache/tests/rotating.rs)
  run("rotating_cache_new_is_empty", [&] {
    RotatingCache c(128, 2, 64);
    EXPECT(c.len() == 0 && c.is_empty());
    EXPECT(c.memory_bytes() == (size_t)2 * 2 * 128 * 64 * 2);
    EXPECT(error_of([&] { c.get(Ctx{}); }).find("empty") != std::string::npos);
    c.reset();
    EXPECT(c.is_empty());
  });
  run("rotating_cache_keeps_the_last_window_in_order", [&] {
    const int W = 8, H = 2;
    RotatingCache c(W, H, D);
    std::vector<std::vector<uint16_t>> seq;  // token t of the whole sequence: [H][D]
    auto push = [&](int T, uint64_t seed) {
      auto k = normal((size_t)H * T * D, seed);
      void* dk = upload(k);
      c.append(ctx, Array{dk, {1, H, T, D}, {}}, Array{dk, {1, H, T, D}, {}});
      (void)hipDeviceSynchronize();
      for (int t = 0; t < T; ++t) {
        std::vector<uint16_t> tok((size_t)H * D);
        for (int h = 0; h < H; ++h)
          for (int d = 0; d < D; ++d) tok[(size_t)h * D + d] = k[((size_t)h * T + t) * D + d];
        seq.push_back(tok);
      }
      (void)hipFree(dk);
    };
    for (auto [T, seed] : std::vector<std::pair<int, uint64_t>>{{5, 1}, {6, 2}, {1, 3}, {20, 4}, {3, 5}}) {
      push(T, seed);
      const size_t n = std::min<size_t>(seq.size(), W);
      EXPECT(c.len() == n);
      auto kv = c.get(ctx);
      (void)hipDeviceSynchronize();
      EXPECT(kv.first.shape[2] == (int64_t)n);
      const int64_t sh = kv.first.strides.empty() ? (int64_t)n * D : kv.first.strides[1];
      const int64_t sp = kv.first.strides.empty() ? D : kv.first.strides[2];
      auto all = download(kv.first.data, (size_t)H * (size_t)sh);
      bool ok = true;
      for (size_t i = 0; i < n; ++i)  // i-th held token = position seq.size() - n + i
        for (int h = 0; h < H; ++h)
          for (int d = 0; d < D; ++d)
            ok &= all[(size_t)h * sh + i * sp + d] == seq[seq.size() - n + i][(size_t)h * D + d];
      EXPECT(ok);
    }
    // a wrapped get() needs the arena for its ordered copy
    EXPECT(error_of([&] { c.get(Ctx{}); }).find("ctx workspace") != std::string::npos);
  });
  run("sliding_window_attention_matches_oracle", [&] {
    const int W = 48, cap_ref = 256;
    RotatingCache c(W, Hkv, D);
    SlidingWindowConfig sw{cfg, (size_t)W};
    OracleLayer ref(hidden, Hq, Hkv, D, cap_ref, 4000);
    DevQW dq(ref.q), dk(ref.k), dv(ref.v), dout(ref.o);
    auto qw = normal(D, 20, 1.f, 0.02f), kw = normal(D, 21, 1.f, 0.02f);
    void *dqw = upload(qw), *dkw = upload(kw);
    GqaWeights w{dq.qw, dk.qw, dv.qw, dout.qw, Array{dqw, {D}, {}}, Array{dkw, {D}, {}}};
    // prefill 40, 20 decode steps (the ring wraps), then a 30-token chunk that wraps within it
    std::vector<std::pair<int, int>> calls{{0, 40}};
    for (int i = 0; i < 20; ++i) calls.push_back({40 + i, 1});
    calls.push_back({60, 30});
    int step = 0;
    for (auto [off, t] : calls) {
      auto x = normal((size_t)t * hidden, 300 + step);
      void* dx = upload(x);
      Array y = sliding_window_attention(ctx, Array{dx, {1, t, hidden}, {}}, w, c, sw, off);
      (void)hipDeviceSynchronize();
      EXPECT(c.len() == (size_t)std::min(off + t, W) && c.total_len() == off + t);
      auto want = ref.run(x, t, off, std::max(0, off + t - W), qw.data(), kw.data());
      expect_close_out(download(y.data, want.size()), want, t > 1 ? "window prefill" : "window decode");
      (void)hipFree(dx);
      ++step;
    }
    SlidingWindowConfig bad{cfg, (size_t)W + 1};
    Array ok{(void*)0x1000, {1, 1, (int64_t)hidden}, {}};
    EXPECT(error_of([&] { sliding_window_attention(ctx, ok, w, c, bad, 90); }).find("window_size") !=
           std::string::npos);
    (void)hipFree(dqw);
    (void)hipFree(dkw);
  });
  run("qkv_attention_over_the_ring_matches_oracle", [&] {
    const int W = 48, cap_ref = 128;
    RotatingCache c(W, Hkv, D);
    std::vector<uint16_t> kref((size_t)Hkv * cap_ref * D, 0), vref((size_t)Hkv * cap_ref * D, 0);
    const float scale = 1.0f / std::sqrt((float)D);
    int step = 0;
    for (auto [off, t] : std::vector<std::pair<int, int>>{{0, 40}, {40, 1}, {41, 30}, {71, 1}}) {
      auto qkv = normal((size_t)t * F, 500 + step++);
      void* dqkv = upload(qkv);
      Array out = qkv_attention(ctx, Array{dqkv, {1, t, F}, {}}, std::nullopt, std::nullopt, c, cfg, off);
      (void)hipDeviceSynchronize();
      std::vector<uint16_t> q((size_t)Hq * t * D), ref((size_t)t * Hq * D);
      int32_t o32 = off, len = off + t, begin = std::max(0, off + t - W);
      EXPECT(ora_pre_attention(qkv.data(), nullptr, nullptr, 1e-6f, 1e6f, &o32, 1, t, Hq, Hkv, D, ORA_FLAG_NO_NORM,
                               q.data(), kref.data(), vref.data(), cap_ref) == 0);
      ora_sdpa(q.data(), kref.data(), vref.data(), &len, &begin, 1, Hq, Hkv, t, D, cap_ref, scale, t > 1 ? 1 : 0, 0,
               ref.data());
      expect_close(download(out.data, ref.size()), ref, t > 1 ? "ring prefill" : "ring decode");
      (void)hipFree(dqkv);
    }
  });
  // ---- Fp8Cache (crates/kvcache/src/fp8.rs:27-91; the layer over it, crates/attention/src/lib.rs:22-27)
  run("fp8_cache_new_is_empty", [&] {
    Fp8Cache c(Hkv, 64, D);
    EXPECT(c.len() == 0 && c.is_empty() && c.n_rot() == 0);
    EXPECT(c.memory_bytes() == (size_t)2 * Hkv * 64 * (D + D / 64));
    EXPECT(error_of([&] { c.get(ctx); }).find("empty") != std::string::npos);
    Fp8Cache rot(Hkv, 64, D, 64);  // Fp8Cache::new(128, 64): dims 64..127 kept as bf16
    EXPECT(rot.n_rot() == 64 && rot.memory_bytes() == (size_t)2 * Hkv * 64 * (D + 64 + D / 64));
    try {
      Fp8Cache bad(Hkv, 64, D, 32);
      EXPECT(false);
    } catch (const Error& e) {
      EXPECT(e.code() == EMA_ERR_UNSUPPORTED);
    }
  });
  for (const int nr : {0, 64})
  run(nr ? "fp8_cache_append_then_get_is_the_round_trip_rope_tail_64" : "fp8_cache_append_then_get_is_the_round_trip", [&] {
    const int cap8 = 64, T1 = 5, T2 = 3;
    Fp8Cache c(Hkv, cap8, D, nr);
    // values spread over several binades, so the block exponents differ between blocks
    auto k1 = normal((size_t)Hkv * T1 * D, 31, 0.f, 3.f), v1 = normal((size_t)Hkv * T1 * D, 32, 0.f, 0.01f);
    auto k2 = normal((size_t)Hkv * T2 * D, 33, 0.f, 200.f), v2 = normal((size_t)Hkv * T2 * D, 34);
    void *dk1 = upload(k1), *dv1 = upload(v1), *dk2 = upload(k2), *dv2 = upload(v2);
    c.append(ctx, Array{dk1, {1, Hkv, T1, D}, {}}, Array{dv1, {1, Hkv, T1, D}, {}});
    c.append(ctx, Array{dk2, {1, Hkv, T2, D}, {}}, Array{dv2, {1, Hkv, T2, D}, {}});
    EXPECT(c.len() == T1 + T2);
    auto kv = c.get(ctx);
    (void)hipDeviceSynchronize();
    EXPECT(kv.first.shape == std::vector<int64_t>({1, Hkv, T1 + T2, D}));
    auto gk = download(kv.first.data, (size_t)Hkv * (T1 + T2) * D);
    auto gv = download(kv.second.data, gk.size());
    // the expected cache: the chronological rows, round-tripped per row as the oracle does
    auto expect = [&](const std::vector<uint16_t>& a, const std::vector<uint16_t>& b) {
      std::vector<uint16_t> e((size_t)Hkv * (T1 + T2) * D);
      for (int h = 0; h < Hkv; ++h)
        for (int t = 0; t < T1 + T2; ++t)
          for (int d = 0; d < D; ++d)
            e[((size_t)h * (T1 + T2) + t) * D + d] =
                t < T1 ? a[((size_t)h * T1 + t) * D + d] : b[((size_t)h * T2 + t - T1) * D + d];
      fp8_round_trip_rows(e, 1, Hkv * (T1 + T2), D, 0, Hkv * (T1 + T2), nr);
      return e;
    };
    EXPECT(same_values(gk, expect(k1, k2)));
    EXPECT(same_values(gv, expect(v1, v2)));
    // the stored codes and exponents are the oracle's quantisation of the same rows (head
    // 0, rows [0, T1)); with the tail, a row is 64 codes then the 64 tail values as bf16
    const int R = D + nr, nq = D - nr;  // bytes per stored row, quantised dims
    std::vector<float> f((size_t)T1 * D), fq((size_t)T1 * nq);
    std::vector<uint8_t> codes((size_t)T1 * nq), got_rows((size_t)T1 * R), got_codes;
    std::vector<int8_t> exps((size_t)T1 * nq / 64), got_exps((size_t)T1 * D / 64), want_exps;
    ora_bf16_to_f32_array(k1.data(), f.data(), f.size());
    for (int t = 0; t < T1; ++t) std::copy_n(&f[(size_t)t * D], nq, &fq[(size_t)t * nq]);
    ora_fp8_quantize_rows(fq.data(), T1, nq, codes.data(), exps.data());
    EXPECT(hipMemcpy(got_rows.data(), c.desc().k, got_rows.size(), hipMemcpyDeviceToHost) == hipSuccess);
    EXPECT(hipMemcpy(got_exps.data(), c.desc().k_exp, got_exps.size(), hipMemcpyDeviceToHost) == hipSuccess);
    for (int t = 0; t < T1; ++t) {
      got_codes.insert(got_codes.end(), &got_rows[(size_t)t * R], &got_rows[(size_t)t * R + nq]);
      for (int b = 0; b < D / 64; ++b) want_exps.push_back(b < nq / 64 ? exps[(size_t)t * (nq / 64) + b] : 0);
      // the tail: the bf16 bytes of the appended values
      EXPECT(std::memcmp(&got_rows[(size_t)t * R + nq], &k1[(size_t)t * D + nq], (size_t)nr * 2) == 0);
    }
    for (auto* c : {&codes, &got_codes})  // -0 (0x80) and +0 (0x00) are the same value
      for (auto& b : *c) b = b == 0x80 ? 0 : b;
    EXPECT(got_codes == codes && got_exps == want_exps);
    std::string e = error_of([&] {
      auto big = normal((size_t)Hkv * 60 * D, 35);
      void* db = upload(big);
      try {
        c.append(ctx, Array{db, {1, Hkv, 60, D}, {}}, Array{db, {1, Hkv, 60, D}, {}});
      } catch (...) {
        (void)hipFree(db);
        throw;
      }
      (void)hipFree(db);
    });
    EXPECT(e.find("static KV overflow") != std::string::npos && c.len() == T1 + T2);
    c.reset();
    EXPECT(c.is_empty());
    for (void* p : {dk1, dv1, dk2, dv2}) (void)hipFree(p);
  });
  for (const int nr : {0, 64})
  run(nr ? "gqa_attention_over_fp8_cache_rope_tail_64_matches_oracle" : "gqa_attention_over_fp8_cache_matches_oracle", [&] {
    Fp8Cache c(Hkv, cap, D, nr);
    Ctx fctx;
    fctx.workspace_bytes = gqa_workspace_bytes(cfg, hidden, 64, c);
    EXPECT(fctx.workspace_bytes > gqa_workspace_bytes(cfg, hidden, 64, cap));  // + the prefill's bf16 copy
    EXPECT(hipMalloc(&fctx.workspace, fctx.workspace_bytes) == hipSuccess &&
           hipMemset(fctx.workspace, 0, fctx.workspace_bytes) == hipSuccess);
    OracleLayer ref(hidden, Hq, Hkv, D, cap, 6000 + nr);
    ref.fp8 = true;
    ref.n_rot = nr;
    DevQW dq(ref.q), dk(ref.k), dv(ref.v), dout(ref.o);
    auto qw = normal(D, 60, 1.f, 0.02f), kw = normal(D, 61, 1.f, 0.02f);
    void *dqw = upload(qw), *dkw = upload(kw);
    GqaWeights w{dq.qw, dk.qw, dv.qw, dout.qw, Array{dqw, {D}, {}}, Array{dkw, {D}, {}}};
    int step = 0;
    std::vector<uint16_t> kh, vh;
    ref.k_held = &kh;
    ref.v_held = &vh;
    // The same layer over a bf16 cache: its rows (held to the oracle by the bf16 layer tests)
    // are what the FP8 layer quantises, so the FP8 rows must be their round trip exactly.
    StaticCache c16(Hkv, cap, D);
    auto layer = [&](const Ctx& cx, const Array& x, HipKvCache& cache, int off, bool window) {
      SlidingWindowConfig sw{cfg, 8};
      return window ? sliding_window_attention(cx, x, w, cache, sw, off) : gqa_attention(cx, x, w, cache, cfg, off);
    };
    auto rows_of = [&](const void* base, int n) {  // rows [0, n) of a [Hkv, cap, D] cache
      auto all = download(base, (size_t)Hkv * cap * D);
      std::vector<uint16_t> r((size_t)Hkv * n * D);
      for (int h = 0; h < Hkv; ++h) std::copy_n(&all[(size_t)h * cap * D], (size_t)n * D, &r[(size_t)h * n * D]);
      return r;
    };
    // one layer call; then the output, and the held rows (get() reuses the arena after it)
    auto call = [&](int off, int t, uint64_t seed, bool window) {
      auto x = normal((size_t)t * hidden, seed);
      void* dx = upload(x);
      Array y = layer(fctx, Array{dx, {1, t, hidden}, {}}, c, off, window);
      (void)hipDeviceSynchronize();
      EXPECT(c.len() == (size_t)(off + t));
      auto got = download(y.data, (size_t)t * hidden);
      (void)layer(ctx, Array{dx, {1, t, hidden}, {}}, c16, off, window);
      auto kv = c.get(fctx);
      (void)hipDeviceSynchronize();
      kh = download(kv.first.data, (size_t)Hkv * (off + t) * D);
      vh = download(kv.second.data, kh.size());
      auto k16 = rows_of(c16.desc().k, off + t), v16 = rows_of(c16.desc().v, off + t);
      fp8_round_trip_rows(k16, 1, Hkv * (off + t), D, 0, Hkv * (off + t), nr);
      fp8_round_trip_rows(v16, 1, Hkv * (off + t), D, 0, Hkv * (off + t), nr);
      EXPECT(same_values(kh, k16) && same_values(vh, v16));
      auto want = ref.run(x, t, off, 0, qw.data(), kw.data());
      expect_close_out(got, want, window ? "fp8 window step (whole cache)"
                                         : t > 1 ? "fp8 layer prefill" : "fp8 layer decode");
      (void)hipFree(dx);
    };
    // prefill 37, 3 decode steps, a 20-token chunk over the cache, one more step
    for (auto [off, t] : std::vector<std::pair<int, int>>{{0, 37}, {37, 1}, {38, 1}, {39, 1}, {40, 20}, {60, 1}})
      call(off, t, 700 + step++, false);
    // a window layer over a non-rotating cache attends the whole cache (sliding_window.rs:40-50)
    call(61, 1, 799, true);
    (void)hipFree(dqw);
    (void)hipFree(dkw);
    (void)hipFree(fctx.workspace);
  });
  for (const int nr : {0, 64})
  run(nr ? "qkv_attention_over_fp8_cache_rope_tail_64_matches_oracle" : "qkv_attention_over_fp8_cache_matches_oracle", [&] {
    Fp8Cache c(Hkv, 128, D, nr);
    Ctx fctx;
    fctx.workspace_bytes = qkv_attention_workspace_bytes(cfg, 64, c);
    EXPECT(hipMalloc(&fctx.workspace, fctx.workspace_bytes) == hipSuccess &&
           hipMemset(fctx.workspace, 0, fctx.workspace_bytes) == hipSuccess);
    std::vector<uint16_t> kref((size_t)Hkv * 128 * D, 0), vref((size_t)Hkv * 128 * D, 0);
    const float scale = 1.0f / std::sqrt((float)D);
    int step = 0;
    for (auto [off, t] : std::vector<std::pair<int, int>>{{0, 50}, {50, 1}, {51, 64}, {115, 1}}) {
      auto qkv = normal((size_t)t * F, 900 + step++);
      void* dqkv = upload(qkv);
      Array out = qkv_attention(fctx, Array{dqkv, {1, t, F}, {}}, std::nullopt, std::nullopt, c, cfg, off);
      (void)hipDeviceSynchronize();
      std::vector<uint16_t> q((size_t)Hq * t * D), ref((size_t)t * Hq * D);
      int32_t o32 = off, len = off + t;
      EXPECT(ora_pre_attention(qkv.data(), nullptr, nullptr, 1e-6f, 1e6f, &o32, 1, t, Hq, Hkv, D, ORA_FLAG_NO_NORM,
                               q.data(), kref.data(), vref.data(), 128) == 0);
      fp8_round_trip_rows(kref, Hkv, 128, D, off, t, nr);
      fp8_round_trip_rows(vref, Hkv, 128, D, off, t, nr);
      ora_sdpa(q.data(), kref.data(), vref.data(), &len, nullptr, 1, Hq, Hkv, t, D, 128, scale, t > 1 ? 1 : 0, 0,
               ref.data());
      expect_close(download(out.data, ref.size()), ref, t > 1 ? "fp8 prefill" : "fp8 decode");
      (void)hipFree(dqkv);
    }
    // V rows (written as given) decode to the oracle's round trip exactly; K rows (after
    // RoPE, whose bf16 rounding may differ by one step) to within one FP8 step
    auto kv = c.get(fctx);
    (void)hipDeviceSynchronize();
    std::vector<uint16_t> vwant((size_t)Hkv * 116 * D);
    for (int h = 0; h < Hkv; ++h) std::copy_n(&vref[(size_t)h * 128 * D], (size_t)116 * D, &vwant[(size_t)h * 116 * D]);
    EXPECT(same_values(download(kv.second.data, vwant.size()), vwant));
    adopt_fp8_rows(kref, download(kv.first.data, vwant.size()), Hkv, 128, 116, D, "K rows", 0.01);
    (void)hipFree(fctx.workspace);
  });
  (void)hipFree(ctx.workspace);
}

int main(int argc, char** argv) {
  const std::string mode = argc > 1 ? argv[1] : "cpu";
  if (mode == "cpu") cpu_tests();
  else if (mode == "gpu") gpu_tests();
  else {
    std::fprintf(stderr, "usage: %s cpu|gpu\n", argv[0]);
    return 2;
  }
  std::printf("%s: %d failed\n", mode.c_str(), g_failed);
  return g_failed ? 1 : 0;
}
