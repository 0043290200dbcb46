// Tests of the C++ host API (engine-mlx_amd/host/ema_host.hpp), in the shape of
// the reference's own unit tests for the same surface:
//   crates/kvcache/tests/lib.rs     (KvCache trait contract, InMemoryCache)
//   crates/kvcache/tests/concat.rs  (new_is_empty, reset, get bails when empty)
//   crates/attention/tests/gqa.rs   (GqaConfig constructible, gqa_attention errors)
// plus GPU checks of StaticCache, RotatingCache, gqa_attention (projections, norms, RoPE,
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

// The reference layer on the host (gqa.rs:62-107 with the oracle's ops): q|k|v
// projections, norms (null = absent), RoPE and the cache write at `off`, SDPA over
// [begin, off + T) (causal for T > 1), o_proj. kref/vref are the chronological caches.
struct OracleLayer {
  HostQW q, k, v, o;
  int Hq, Hkv, D, cap;
  std::vector<uint16_t> kref, vref;
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
