// Tests of the C++ host API (engine-mlx_amd/host/ema_host.hpp), in the shape of
// the reference's own unit tests for the same surface:
//   crates/kvcache/tests/lib.rs     (KvCache trait contract, InMemoryCache)
//   crates/kvcache/tests/concat.rs  (new_is_empty, reset, get bails when empty)
//   crates/attention/tests/gqa.rs   (GqaConfig constructible, gqa_attention errors)
// plus GPU checks of StaticCache and gqa_attention against the CPU oracle.
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

static void gpu_tests() {
  const int Hkv = 2, D = 128, cap = 256, Hq = 8;
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
  run("gqa_attention_rejects_bad_shapes", [&] {
    StaticCache c(Hkv, cap, D);
    GqaConfig cfg{Hq, Hkv, D, 1e6f, 1e-6f, true};
    Array qkv{(void*)0x1000, {1, 4, 100}, {}};
    EXPECT(error_of([&] { gqa_attention(Ctx{}, qkv, GqaWeights{}, c, cfg, 0); }).find("qkv must be") !=
           std::string::npos);
    GqaConfig bad{12, 8, D, 1e6f, 1e-6f, true};
    EXPECT(!error_of([&] { gqa_attention(Ctx{}, qkv, GqaWeights{}, c, bad, 0); }).empty());
    Array ok{(void*)0x1000, {1, 4, (int64_t)(Hq + 2 * Hkv) * D}, {}};
    EXPECT(error_of([&] { gqa_attention(Ctx{}, ok, GqaWeights{}, c, cfg, cap - 2); }).find("static KV overflow") !=
           std::string::npos);
  });
  run("gqa_attention_prefill_then_decode_matches_oracle", [&] {
    StaticCache c(Hkv, cap, D);
    GqaConfig cfg{Hq, Hkv, D, 1e6f, 1e-6f, true};
    const int F = (Hq + 2 * Hkv) * D, T = 37, steps = 4;
    auto qw = normal(D, 10, 1.f, 0.02f), kw = normal(D, 11, 1.f, 0.02f);
    void *dqw = upload(qw), *dkw = upload(kw);
    GqaWeights w{Array{dqw, {D}, {}}, Array{dkw, {D}, {}}};
    std::vector<uint16_t> kref((size_t)Hkv * cap * D, 0), vref((size_t)Hkv * cap * D, 0);
    const float scale = 1.0f / std::sqrt((float)D);
    for (int step = 0; step <= steps; ++step) {
      const int t = step == 0 ? T : 1, off = step == 0 ? 0 : T + step - 1;
      auto qkv = normal((size_t)t * F, 100 + step);
      void* dqkv = upload(qkv);
      Array out = gqa_attention(Ctx{}, Array{dqkv, {1, t, F}, {}}, w, c, cfg, off);
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
    // reset keeps the buffers, rewinds the length (crates/serve/src/engine_ext.rs:10-36)
    c.reset();
    EXPECT(c.is_empty() && c.memory_bytes() == (size_t)2 * Hkv * cap * D * 2);
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
      c.append(Ctx{}, Array{dk, {1, H, T, D}, {}}, Array{dk, {1, H, T, D}, {}});
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
      auto kv = c.get(Ctx{});
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
  });
  run("sliding_window_attention_matches_oracle", [&] {
    const int W = 48, cap_ref = 256;
    RotatingCache c(W, Hkv, D);
    GqaConfig cfg{Hq, Hkv, D, 1e6f, 1e-6f, true};
    SlidingWindowConfig sw{cfg, (size_t)W};
    const int F = (Hq + 2 * Hkv) * D;
    auto qw = normal(D, 20, 1.f, 0.02f), kw = normal(D, 21, 1.f, 0.02f);
    void *dqw = upload(qw), *dkw = upload(kw);
    GqaWeights w{Array{dqw, {D}, {}}, Array{dkw, {D}, {}}};
    std::vector<uint16_t> kref((size_t)Hkv * cap_ref * D, 0), vref((size_t)Hkv * cap_ref * D, 0);
    const float scale = 1.0f / std::sqrt((float)D);
    // prefill 40, 20 decode steps (the ring wraps), then a 30-token chunk that wraps within it
    std::vector<std::pair<int, int>> calls{{0, 40}};
    for (int i = 0; i < 20; ++i) calls.push_back({40 + i, 1});
    calls.push_back({60, 30});
    int step = 0;
    for (auto [off, t] : calls) {
      auto qkv = normal((size_t)t * F, 300 + step);
      void* dqkv = upload(qkv);
      Array out = sliding_window_attention(Ctx{}, Array{dqkv, {1, t, F}, {}}, w, c, sw, off);
      (void)hipDeviceSynchronize();
      EXPECT(c.len() == (size_t)std::min(off + t, W) && c.total_len() == off + t);
      std::vector<uint16_t> q((size_t)Hq * t * D), ref((size_t)t * Hq * D);
      int32_t o32 = off, len = off + t, begin = std::max(0, off + t - W);
      EXPECT(ora_pre_attention(qkv.data(), qw.data(), kw.data(), 1e-6f, 1e6f, &o32, 1, t, Hq, Hkv, D, 0, q.data(),
                               kref.data(), vref.data(), cap_ref) == 0);
      ora_sdpa(q.data(), kref.data(), vref.data(), &len, &begin, 1, Hq, Hkv, t, D, cap_ref, scale, t > 1 ? 1 : 0, 0,
               ref.data());
      if (step == 0 || step == 20 || step == 21)
        expect_close(download(out.data, ref.size()), ref, t > 1 ? "window prefill" : "window decode");
      else {
        double mx = 0;
        auto got = download(out.data, ref.size());
        for (size_t i = 0; i < got.size(); ++i)
          mx = std::max(mx, std::fabs((double)ora_bf16_to_f32(got[i]) - (double)ora_bf16_to_f32(ref[i])));
        EXPECT(mx <= 2e-2);
      }
      (void)hipFree(dqkv);
      ++step;
    }
    SlidingWindowConfig bad{cfg, (size_t)W + 1};
    Array ok{(void*)0x1000, {1, 1, (int64_t)F}, {}};
    EXPECT(error_of([&] { sliding_window_attention(Ctx{}, ok, w, c, bad, 90); }).find("window_size") !=
           std::string::npos);
    (void)hipFree(dqw);
    (void)hipFree(dkw);
  });
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
