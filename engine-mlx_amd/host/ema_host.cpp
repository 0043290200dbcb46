// C++ host API over the ema_attn C ABI; see ema_host.hpp for the mapping to
// the reference's KvCache / gqa_attention.
#include "ema_host.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <numeric>

namespace ema {

namespace {

// The reference turns a failing mlx-c status into
// "MLX op '<op>' failed with code <n>" (crates/mlx-ffi/src/ops/real/mod.rs:35-40).
void check(int32_t rc, const char* op) {
  if (rc != EMA_OK) throw Error(rc, std::string("ema op '") + op + "' failed with code " + std::to_string(rc) +
                                        ": " + ema_last_error());
}

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) throw Error(EMA_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

void* grow(void*& buf, size_t& have, size_t need, const char* what) {
  if (need > have) {
    if (buf) check_hip(hipFree(buf), what);
    buf = nullptr;
    have = 0;
    check_hip(hipMalloc(&buf, need), what);
    have = need;
  }
  return buf;
}

std::string shape_str(const std::vector<int64_t>& s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
  return r + "]";
}

}  // namespace

int64_t Array::numel() const {
  return std::accumulate(shape.begin(), shape.end(), (int64_t)1, [](int64_t a, int64_t b) { return a * b; });
}

StaticCache::StaticCache(int32_t n_kv_heads, int32_t capacity, int32_t head_dim) {
  check(ema_kvcache_alloc(&desc_, 1, n_kv_heads, capacity, head_dim), "kvcache_alloc");
  std::vector<int32_t> pos((size_t)capacity + 1);
  std::iota(pos.begin(), pos.end(), 0);
  try {
    check_hip(hipMalloc((void**)&positions_, pos.size() * sizeof(int32_t)), "StaticCache: positions");
    check_hip(hipMemcpy(positions_, pos.data(), pos.size() * sizeof(int32_t), hipMemcpyHostToDevice),
              "StaticCache: positions upload");
  } catch (...) {
    if (positions_) (void)hipFree(positions_);
    ema_kvcache_free(&desc_);
    throw;
  }
}

StaticCache::~StaticCache() {
  ema_kvcache_free(&desc_);
  if (positions_) (void)hipFree(positions_);
  if (q_buf_) (void)hipFree(q_buf_);
  if (o_buf_) (void)hipFree(o_buf_);
  if (ws_) (void)hipFree(ws_);
}

size_t StaticCache::memory_bytes() const {
  uint64_t b = 0;
  check(ema_kvcache_memory_bytes(&desc_, &b), "kvcache_memory_bytes");
  return (size_t)b;
}

const int32_t* StaticCache::device_position(int32_t p) const {
  if (p < 0 || p > desc_.capacity)
    throw Error(EMA_ERR_CAPACITY, "static KV overflow offset=" + std::to_string(p) + " cap=" +
                                      std::to_string(desc_.capacity));
  return positions_ + p;
}

void StaticCache::advance(int32_t n) {
  if (n < 0 || offset_ + n > desc_.capacity)
    throw Error(EMA_ERR_CAPACITY, "static KV overflow offset=" + std::to_string(offset_ + n) + " cap=" +
                                      std::to_string(desc_.capacity));
  offset_ += n;
}

void StaticCache::append(const Ctx& ctx, const Array& k, const Array& v) {
  const int64_t Hkv = desc_.n_kv_heads, D = desc_.head_dim;
  for (const Array* a : {&k, &v}) {
    if (!a->data) throw Error(EMA_ERR_INVALID_ARG, "StaticCache::append: null k/v");
    if (a->shape.size() != 4 || a->shape[0] != 1 || a->shape[1] != Hkv || a->shape[3] != D ||
        (!a->strides.empty()))
      throw Error(EMA_ERR_SHAPE, "StaticCache::append: expected contiguous [1, " + std::to_string(Hkv) +
                                     ", seq, " + std::to_string(D) + "], got " + shape_str(a->shape));
  }
  if (k.shape[2] != v.shape[2]) throw Error(EMA_ERR_SHAPE, "StaticCache::append: k/v lengths differ");
  const int64_t T = k.shape[2];
  if (offset_ + T > desc_.capacity)
    throw Error(EMA_ERR_CAPACITY, "static KV overflow offset=" + std::to_string(offset_ + T) + " cap=" +
                                      std::to_string(desc_.capacity));
  // one strided copy per tensor: Hkv rows of T*D elements into rows [offset, offset+T)
  const size_t width = (size_t)T * D * 2;
  hipStream_t s = (hipStream_t)ctx.stream;
  for (int i = 0; i < 2; ++i) {
    char* dst = (char*)(i == 0 ? desc_.k : desc_.v) + (size_t)offset_ * desc_.stride_pos * 2;
    const void* src = (i == 0 ? k : v).data;
    check_hip(hipMemcpy2DAsync(dst, (size_t)desc_.stride_head * 2, src, width, width, (size_t)Hkv,
                               hipMemcpyDeviceToDevice, s),
              "StaticCache::append copy");
  }
  offset_ += (int32_t)T;
}

std::pair<Array, Array> StaticCache::get(const Ctx&) const {
  if (offset_ == 0) throw Error(EMA_ERR_INVALID_ARG, "KV cache is empty");
  Array k, v;
  k.data = desc_.k;
  v.data = desc_.v;
  k.shape = v.shape = {1, desc_.n_kv_heads, offset_, desc_.head_dim};
  k.strides = v.strides = {desc_.stride_batch, desc_.stride_head, desc_.stride_pos, 1};
  return {k, v};
}

void* StaticCache::q_scratch(size_t bytes) { return grow(q_buf_, q_bytes_, bytes, "StaticCache: q scratch"); }
void* StaticCache::out_scratch(size_t bytes) { return grow(o_buf_, o_bytes_, bytes, "StaticCache: out scratch"); }

void* StaticCache::decode_workspace(int32_t n_heads, uint64_t* bytes) {
  uint64_t need = 0;
  check(ema_decode_workspace_size(1, n_heads, desc_.n_kv_heads, desc_.head_dim, desc_.capacity, &need),
        "decode_workspace_size");
  size_t have = (size_t)ws_bytes_;
  grow(ws_, have, (size_t)need, "StaticCache: decode workspace");
  ws_bytes_ = have;
  *bytes = ws_bytes_;
  return ws_;
}

RotatingCache::RotatingCache(int32_t window_size, int32_t n_kv_heads, int32_t head_dim) {
  check(ema_kvcache_alloc(&desc_, 1, n_kv_heads, window_size, head_dim), "kvcache_alloc");
  desc_.flags = EMA_KV_ROTATING;
}

RotatingCache::~RotatingCache() {
  ema_kvcache_free(&desc_);
  for (void* p : {(void*)positions_, q_buf_, o_buf_, ws_, get_buf_})
    if (p) (void)hipFree(p);
}

size_t RotatingCache::memory_bytes() const {
  uint64_t b = 0;
  check(ema_kvcache_memory_bytes(&desc_, &b), "kvcache_memory_bytes");
  return (size_t)b;
}

const int32_t* RotatingCache::device_position(int64_t p) {
  if (p < 0 || p >= ((int64_t)1 << 31)) throw Error(EMA_ERR_CAPACITY, "rotating KV position " + std::to_string(p));
  if (p >= n_positions_) {
    int64_t n = n_positions_ ? n_positions_ : 4096;
    while (n <= p) n *= 2;
    std::vector<int32_t> pos((size_t)n);
    std::iota(pos.begin(), pos.end(), 0);
    int32_t* fresh = nullptr;
    check_hip(hipMalloc((void**)&fresh, pos.size() * sizeof(int32_t)), "RotatingCache: positions");
    if (hipMemcpy(fresh, pos.data(), pos.size() * sizeof(int32_t), hipMemcpyHostToDevice) != hipSuccess) {
      (void)hipFree(fresh);
      throw Error(EMA_ERR_HIP, "RotatingCache: positions upload");
    }
    if (positions_) {
      // earlier pointers may still be read by queued work
      check_hip(hipDeviceSynchronize(), "RotatingCache: positions");
      (void)hipFree(positions_);
    }
    positions_ = fresh;
    n_positions_ = n;
  }
  return positions_ + p;
}

void RotatingCache::append(const Ctx& ctx, const Array& k, const Array& v) {
  const int64_t Hkv = desc_.n_kv_heads, D = desc_.head_dim, W = desc_.capacity;
  for (const Array* a : {&k, &v}) {
    if (!a->data) throw Error(EMA_ERR_INVALID_ARG, "RotatingCache::append: null k/v");
    if (a->shape.size() != 4 || a->shape[0] != 1 || a->shape[1] != Hkv || a->shape[3] != D || !a->strides.empty())
      throw Error(EMA_ERR_SHAPE, "RotatingCache::append: expected contiguous [1, " + std::to_string(Hkv) + ", seq, " +
                                     std::to_string(D) + "], got " + shape_str(a->shape));
  }
  if (k.shape[2] != v.shape[2]) throw Error(EMA_ERR_SHAPE, "RotatingCache::append: k/v lengths differ");
  const int64_t T = k.shape[2];
  const int64_t skip = T > W ? T - W : 0;  // tokens the window drops within this append
  hipStream_t s = (hipStream_t)ctx.stream;
  // tokens [skip, T) at positions total + t: one or two runs of consecutive ring rows
  for (int64_t t = skip; t < T;) {
    const int64_t row = (total_ + t) % W;
    const int64_t n = std::min<int64_t>(T - t, W - row);
    const size_t width = (size_t)n * D * 2;
    for (int i = 0; i < 2; ++i) {
      char* dst = (char*)(i == 0 ? desc_.k : desc_.v) + (size_t)row * desc_.stride_pos * 2;
      const char* src = (const char*)(i == 0 ? k : v).data + (size_t)t * D * 2;
      check_hip(hipMemcpy2DAsync(dst, (size_t)desc_.stride_head * 2, src, (size_t)T * D * 2, width, (size_t)Hkv,
                                 hipMemcpyDeviceToDevice, s),
                "RotatingCache::append copy");
    }
    t += n;
  }
  total_ += T;
}

std::pair<Array, Array> RotatingCache::get(const Ctx& ctx) const {
  if (total_ == 0) throw Error(EMA_ERR_INVALID_ARG, "Rotating KV cache is empty");
  const int64_t Hkv = desc_.n_kv_heads, D = desc_.head_dim, W = desc_.capacity, n = (int64_t)len();
  Array k, v;
  k.shape = v.shape = {1, Hkv, n, D};
  if (total_ <= W) {  // not wrapped: rows [0, total) are in order
    k.data = desc_.k;
    v.data = desc_.v;
    k.strides = v.strides = {desc_.stride_batch, desc_.stride_head, desc_.stride_pos, 1};
    return {k, v};
  }
  // wrapped: oldest token in row total % W; copy rows [start, W) then [0, start)
  const size_t bytes = (size_t)2 * Hkv * W * D * 2;
  if (bytes > get_bytes_) {
    if (get_buf_) check_hip(hipFree(get_buf_), "RotatingCache: get scratch");
    get_buf_ = nullptr;
    get_bytes_ = 0;
    check_hip(hipMalloc(&get_buf_, bytes), "RotatingCache: get scratch");
    get_bytes_ = bytes;
  }
  const int64_t start = total_ % W;
  hipStream_t s = (hipStream_t)ctx.stream;
  for (int i = 0; i < 2; ++i) {
    const char* src = (const char*)(i == 0 ? desc_.k : desc_.v);
    char* dst = (char*)get_buf_ + (size_t)i * Hkv * W * D * 2;
    const size_t pitch_src = (size_t)desc_.stride_head * 2, pitch_dst = (size_t)W * D * 2;
    check_hip(hipMemcpy2DAsync(dst, pitch_dst, src + (size_t)start * desc_.stride_pos * 2, pitch_src,
                               (size_t)(W - start) * D * 2, (size_t)Hkv, hipMemcpyDeviceToDevice, s),
              "RotatingCache::get copy");
    if (start)
      check_hip(hipMemcpy2DAsync(dst + (size_t)(W - start) * D * 2, pitch_dst, src, pitch_src, (size_t)start * D * 2,
                                 (size_t)Hkv, hipMemcpyDeviceToDevice, s),
                "RotatingCache::get copy");
  }
  k.data = get_buf_;
  v.data = (char*)get_buf_ + (size_t)Hkv * W * D * 2;
  return {k, v};
}

void* RotatingCache::q_scratch(size_t bytes) { return grow(q_buf_, q_bytes_, bytes, "RotatingCache: q scratch"); }
void* RotatingCache::out_scratch(size_t bytes) { return grow(o_buf_, o_bytes_, bytes, "RotatingCache: out scratch"); }

void* RotatingCache::decode_workspace(int32_t n_heads, uint64_t* bytes) {
  uint64_t need = 0;
  check(ema_decode_workspace_size(1, n_heads, desc_.n_kv_heads, desc_.head_dim, desc_.capacity, &need),
        "decode_workspace_size");
  size_t have = (size_t)ws_bytes_;
  grow(ws_, have, (size_t)need, "RotatingCache: decode workspace");
  ws_bytes_ = have;
  *bytes = ws_bytes_;
  return ws_;
}

namespace {

// The attention layer over either cache: pre-attention writes the chunk's K/V (ring rows
// for a rotating cache), then causal prefill (T > 1, gqa.rs:78) or decode (T == 1).
template <class Cache>
Array attend(const Ctx& ctx, const Array& qkv, const GqaWeights& weights, Cache& cache, const GqaConfig& config,
             int32_t offset, bool rotating, const char* op) {
  const int32_t Hq = config.n_heads, Hkv = config.n_kv_heads, D = config.head_dim;
  const std::string name(op);
  if (Hq <= 0 || Hkv <= 0 || D <= 0 || Hq % Hkv)
    throw Error(EMA_ERR_SHAPE, name + ": bad head config n_heads=" + std::to_string(Hq) +
                                   " n_kv_heads=" + std::to_string(Hkv) + " head_dim=" + std::to_string(D));
  if (Hkv != cache.n_kv_heads() || D != cache.head_dim())
    throw Error(EMA_ERR_SHAPE, name + ": config does not match the cache");
  if (!qkv.data || qkv.shape.size() != 3 || qkv.shape[0] != 1 || qkv.shape[2] != (int64_t)(Hq + 2 * Hkv) * D ||
      !qkv.strides.empty())
    throw Error(EMA_ERR_SHAPE, name + ": qkv must be contiguous [1, seq, " + std::to_string((Hq + 2 * Hkv) * D) +
                                   "], got " + shape_str(qkv.shape));
  const int32_t T = (int32_t)qkv.shape[1];
  const int32_t cap = cache.desc().capacity;
  if (T <= 0) throw Error(EMA_ERR_SHAPE, name + ": empty sequence");
  if (!rotating && (offset < 0 || (int64_t)offset + T > cap))
    throw Error(EMA_ERR_CAPACITY, "static KV overflow offset=" + std::to_string((int64_t)offset + T - 1) +
                                      " cap=" + std::to_string(cap));
  if (rotating && (offset < 0 || T > cap))
    throw Error(EMA_ERR_CAPACITY, name + ": " + std::to_string(T) + " tokens exceed the window " + std::to_string(cap));
  if (weights.q_norm.has_value() != weights.k_norm.has_value())
    throw Error(EMA_ERR_UNSUPPORTED, name + ": q_norm and k_norm must be both present or both absent");
  uint32_t flags = 0;
  if (!weights.q_norm) flags |= EMA_PRE_NO_NORM;
  if (!config.use_rope) flags |= EMA_PRE_NO_ROPE;
  const float scale = 1.0f / std::sqrt((float)D);  // crates/attention/src/gqa.rs:73

  void* q = cache.q_scratch((size_t)Hq * T * D * 2);
  void* out = cache.out_scratch((size_t)T * Hq * D * 2);
  check(ema_pre_attention(ctx.stream, qkv.data, weights.q_norm ? weights.q_norm->data : nullptr,
                          weights.k_norm ? weights.k_norm->data : nullptr, config.norm_eps, config.rope_theta,
                          cache.device_position(offset), 1, T, Hq, Hkv, D, flags, q, &cache.desc()),
        "pre_attention");
  if (T > 1) {  // is_prefill (gqa.rs:78): causal over the cache
    check(ema_prefill_attention(ctx.stream, q, &cache.desc(), cache.device_position(offset), T, Hq, scale,
                                EMA_PREFILL_CAUSAL, out),
          "prefill_attention");
  } else {
    uint64_t ws_bytes = 0;
    void* ws = cache.decode_workspace(Hq, &ws_bytes);
    const int32_t max_len = offset + 1 < cap ? offset + 1 : cap;
    check(ema_decode_attention(ctx.stream, q, &cache.desc(), cache.device_position(offset + 1), max_len, Hq, scale,
                               out, ws, ws_bytes),
          "decode_attention");
  }
  cache.reset();
  cache.advance(offset + T);
  Array r;
  r.data = out;
  r.shape = {1, T, (int64_t)Hq * D};
  return r;
}

}  // namespace

Array gqa_attention(const Ctx& ctx, const Array& qkv, const GqaWeights& weights, StaticCache& cache,
                    const GqaConfig& config, int32_t offset) {
  return attend(ctx, qkv, weights, cache, config, offset, false, "gqa_attention");
}

Array sliding_window_attention(const Ctx& ctx, const Array& qkv, const GqaWeights& weights, StaticCache& cache,
                               const SlidingWindowConfig& config, int32_t offset) {
  // The reference delegates to gqa_attention and leaves the window to the
  // cache backend (crates/attention/src/sliding_window.rs:40-50).
  return gqa_attention(ctx, qkv, weights, cache, config.gqa, offset);
}

Array sliding_window_attention(const Ctx& ctx, const Array& qkv, const GqaWeights& weights, RotatingCache& cache,
                               const SlidingWindowConfig& config, int32_t offset) {
  if (config.window_size != (size_t)cache.window_size())
    throw Error(EMA_ERR_SHAPE, "sliding_window_attention: window_size " + std::to_string(config.window_size) +
                                   " differs from the cache's " + std::to_string(cache.window_size()));
  return attend(ctx, qkv, weights, cache, config.gqa, offset, true, "sliding_window_attention");
}

}  // namespace ema
