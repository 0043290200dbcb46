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

constexpr size_t kAlign = 256;
size_t aligned(size_t n) { return (n + kAlign - 1) & ~(kAlign - 1); }

// Carves a call's temporaries out of ctx's arena, in order; throws EMA_ERR_WORKSPACE
// with the total the call needs when the arena is smaller. The decode split's arrival
// counters (EMA_DECODE_COUNTER_BYTES) stay at the start of the arena in every layout:
// a decode workspace starts there, and nothing else is carved over them.
class Arena {
 public:
  Arena(const Ctx& ctx, const char* op)
      : base_((char*)ctx.workspace), have_(ctx.workspace ? ctx.workspace_bytes : 0), used_(EMA_DECODE_COUNTER_BYTES),
        op_(op) {}
  void* take(size_t bytes) {
    const size_t at = used_;
    used_ += aligned(bytes);
    return base_ + at;
  }
  // The decode workspace of `bytes` (counters first): call before any take().
  void* take_decode_workspace(size_t bytes) {
    if (used_ != EMA_DECODE_COUNTER_BYTES || bytes < EMA_DECODE_COUNTER_BYTES)
      throw Error(EMA_ERR_INVALID_ARG, std::string(op_) + ": decode workspace carved out of order");
    used_ += aligned(bytes - EMA_DECODE_COUNTER_BYTES);
    return base_;
  }
  // Call after the last take(): the pointers are valid only if this does not throw.
  void check() const {
    if (used_ > have_ || ((uintptr_t)base_ & (kAlign - 1)))
      throw Error(EMA_ERR_WORKSPACE, std::string(op_) + ": a 256-byte aligned ctx workspace of " +
                                         std::to_string(used_) + " bytes is needed, " + std::to_string(have_) +
                                         " given");
  }

 private:
  char* base_;
  size_t have_;
  size_t used_;
  const char* op_;
};

std::string shape_str(const std::vector<int64_t>& s) {
  std::string r = "[";
  for (size_t i = 0; i < s.size(); ++i) r += (i ? ", " : "") + std::to_string(s[i]);
  return r + "]";
}

}  // namespace

int64_t Array::numel() const {
  return std::accumulate(shape.begin(), shape.end(), (int64_t)1, [](int64_t a, int64_t b) { return a * b; });
}

PositionTable::PositionTable(int32_t n) {
  if (n < 0) throw Error(EMA_ERR_SHAPE, "PositionTable: negative size");
  std::vector<int32_t> pos((size_t)n + 1);
  std::iota(pos.begin(), pos.end(), 0);
  check_hip(hipMalloc((void**)&table_, pos.size() * sizeof(int32_t)), "position table");
  const hipError_t e = hipMemcpy(table_, pos.data(), pos.size() * sizeof(int32_t), hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    (void)hipFree(table_);
    table_ = nullptr;
    check_hip(e, "position table upload");
  }
}

PositionTable::~PositionTable() {
  if (table_) (void)hipFree(table_);
}

StaticCache::StaticCache(int32_t n_kv_heads, int32_t capacity, int32_t head_dim)
    : positions_(capacity > 0 ? capacity : 0) {
  check(ema_kvcache_alloc(&desc_, 1, n_kv_heads, capacity, head_dim), "kvcache_alloc");
}

StaticCache::~StaticCache() { ema_kvcache_free(&desc_); }

size_t StaticCache::memory_bytes() const {
  uint64_t b = 0;
  check(ema_kvcache_memory_bytes(&desc_, &b), "kvcache_memory_bytes");
  return (size_t)b;
}

const int32_t* StaticCache::device_position(int32_t p) const {
  if (p < 0 || p > desc_.capacity)
    throw Error(EMA_ERR_CAPACITY, "static KV overflow offset=" + std::to_string(p) + " cap=" +
                                      std::to_string(desc_.capacity));
  return positions_.at(p);
}

const int32_t* StaticCache::position(const Ctx&, int64_t p) const {
  if (p < 0 || p > desc_.capacity)
    throw Error(EMA_ERR_CAPACITY, "static KV overflow offset=" + std::to_string(p) + " cap=" +
                                      std::to_string(desc_.capacity));
  return positions_.at((int32_t)p);
}

void StaticCache::advance(int32_t n) {
  if (n < 0 || offset_ + n > desc_.capacity)
    throw Error(EMA_ERR_CAPACITY, "static KV overflow offset=" + std::to_string(offset_ + n) + " cap=" +
                                      std::to_string(desc_.capacity));
  offset_ += n;
}

void StaticCache::set_len(int64_t n) {
  if (n < 0 || n > desc_.capacity)
    throw Error(EMA_ERR_CAPACITY, "static KV overflow offset=" + std::to_string(n) + " cap=" +
                                      std::to_string(desc_.capacity));
  offset_ = (int32_t)n;
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

RotatingCache::RotatingCache(int32_t window_size, int32_t n_kv_heads, int32_t head_dim) {
  check(ema_kvcache_alloc(&desc_, 1, n_kv_heads, window_size, head_dim), "kvcache_alloc");
  desc_.flags = EMA_KV_ROTATING;
  if (hipMalloc((void**)&slot_, sizeof(int32_t)) != hipSuccess) {
    ema_kvcache_free(&desc_);
    throw Error(EMA_ERR_HIP, "RotatingCache: position slot");
  }
}

RotatingCache::~RotatingCache() {
  ema_kvcache_free(&desc_);
  if (slot_) (void)hipFree(slot_);
}

size_t RotatingCache::memory_bytes() const {
  uint64_t b = 0;
  check(ema_kvcache_memory_bytes(&desc_, &b), "kvcache_memory_bytes");
  return (size_t)b;
}

const int32_t* RotatingCache::position(const Ctx& ctx, int64_t p) const {
  if (p < 0 || p >= ((int64_t)1 << 31)) throw Error(EMA_ERR_CAPACITY, "rotating KV position " + std::to_string(p));
  check(ema_position_write(ctx.stream, slot_, (int32_t)p), "position_write");
  return slot_;
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
  Arena arena(ctx, "RotatingCache::get");
  char* buf = (char*)arena.take((size_t)2 * Hkv * W * D * 2);
  arena.check();
  const int64_t start = total_ % W;
  hipStream_t s = (hipStream_t)ctx.stream;
  for (int i = 0; i < 2; ++i) {
    const char* src = (const char*)(i == 0 ? desc_.k : desc_.v);
    char* dst = buf + (size_t)i * Hkv * W * D * 2;
    const size_t pitch_src = (size_t)desc_.stride_head * 2, pitch_dst = (size_t)W * D * 2;
    check_hip(hipMemcpy2DAsync(dst, pitch_dst, src + (size_t)start * desc_.stride_pos * 2, pitch_src,
                               (size_t)(W - start) * D * 2, (size_t)Hkv, hipMemcpyDeviceToDevice, s),
              "RotatingCache::get copy");
    if (start)
      check_hip(hipMemcpy2DAsync(dst + (size_t)(W - start) * D * 2, pitch_dst, src, pitch_src, (size_t)start * D * 2,
                                 (size_t)Hkv, hipMemcpyDeviceToDevice, s),
                "RotatingCache::get copy");
  }
  k.data = buf;
  v.data = buf + (size_t)Hkv * W * D * 2;
  return {k, v};
}

Fp8Cache::Fp8Cache(int32_t n_kv_heads, int32_t capacity, int32_t head_dim, int32_t n_rot)
    : positions_(capacity > 0 ? capacity : 0) {
  check(ema_kvcache_alloc_fp8(&desc_, 1, n_kv_heads, capacity, head_dim, n_rot), "kvcache_alloc_fp8");
}

Fp8Cache::~Fp8Cache() { ema_kvcache_free(&desc_); }

size_t Fp8Cache::memory_bytes() const {
  uint64_t b = 0;
  check(ema_kvcache_memory_bytes(&desc_, &b), "kvcache_memory_bytes");
  return (size_t)b;
}

const int32_t* Fp8Cache::position(const Ctx&, int64_t p) const {
  if (p < 0 || p > desc_.capacity)
    throw Error(EMA_ERR_CAPACITY, "static KV overflow offset=" + std::to_string(p) + " cap=" +
                                      std::to_string(desc_.capacity));
  return positions_.at((int32_t)p);
}

void Fp8Cache::set_len(int64_t n) {
  if (n < 0 || n > desc_.capacity)
    throw Error(EMA_ERR_CAPACITY, "static KV overflow offset=" + std::to_string(n) + " cap=" +
                                      std::to_string(desc_.capacity));
  offset_ = (int32_t)n;
}

void Fp8Cache::append(const Ctx& ctx, const Array& k, const Array& v) {
  const int64_t Hkv = desc_.n_kv_heads, D = desc_.head_dim;
  for (const Array* a : {&k, &v}) {
    if (!a->data) throw Error(EMA_ERR_INVALID_ARG, "Fp8Cache::append: null k/v");
    if (a->shape.size() != 4 || a->shape[0] != 1 || a->shape[1] != Hkv || a->shape[3] != D || !a->strides.empty())
      throw Error(EMA_ERR_SHAPE, "Fp8Cache::append: expected contiguous [1, " + std::to_string(Hkv) + ", seq, " +
                                     std::to_string(D) + "], got " + shape_str(a->shape));
  }
  if (k.shape[2] != v.shape[2]) throw Error(EMA_ERR_SHAPE, "Fp8Cache::append: k/v lengths differ");
  const int64_t T = k.shape[2];
  if (offset_ + T > desc_.capacity)
    throw Error(EMA_ERR_CAPACITY, "static KV overflow offset=" + std::to_string(offset_ + T) + " cap=" +
                                      std::to_string(desc_.capacity));
  if (T == 0) return;
  // the new rows as a bf16 cache of T rows, quantised into rows [offset, offset + T)
  ema_kvcache_desc src{};
  check(ema_kvcache_init(&src, k.data, v.data, 1, (int32_t)Hkv, (int32_t)T, (int32_t)D), "kvcache_init");
  check(ema_kvcache_convert(ctx.stream, &src, 0, &desc_, offset_, (int32_t)T), "kvcache_convert");
  offset_ += (int32_t)T;
}

std::pair<Array, Array> Fp8Cache::get(const Ctx& ctx) const {
  if (offset_ == 0) throw Error(EMA_ERR_INVALID_ARG, "FP8 KV cache is empty");
  const int64_t Hkv = desc_.n_kv_heads, D = desc_.head_dim, n = offset_;
  Arena arena(ctx, "Fp8Cache::get");
  char* kb = (char*)arena.take((size_t)Hkv * n * D * 2);
  char* vb = (char*)arena.take((size_t)Hkv * n * D * 2);
  arena.check();
  ema_kvcache_desc dst{};
  check(ema_kvcache_init(&dst, kb, vb, 1, (int32_t)Hkv, (int32_t)n, (int32_t)D), "kvcache_init");
  check(ema_kvcache_convert(ctx.stream, &desc_, 0, &dst, 0, (int32_t)n), "kvcache_convert");
  Array k, v;
  k.data = kb;
  v.data = vb;
  k.shape = v.shape = {1, Hkv, n, D};
  return {k, v};
}

namespace {

void check_config(const GqaConfig& c, const std::string& op) {
  if (c.n_heads <= 0 || c.n_kv_heads <= 0 || c.head_dim <= 0 || c.n_heads % c.n_kv_heads)
    throw Error(EMA_ERR_SHAPE, op + ": bad head config n_heads=" + std::to_string(c.n_heads) +
                                   " n_kv_heads=" + std::to_string(c.n_kv_heads) +
                                   " head_dim=" + std::to_string(c.head_dim));
}

uint64_t decode_ws_bytes(const GqaConfig& c, int32_t capacity) {
  uint64_t need = 0;
  check(ema_decode_workspace_size(1, c.n_heads, c.n_kv_heads, c.head_dim, capacity, &need), "decode_workspace_size");
  return need;
}

// Temporaries of the attention core, carved in this order: the decode split state (decode
// only, at the start of the arena), q (prefill only), the attention output, and an FP8
// cache's prefill workspace (the bf16 copy of the attended rows).
struct CoreBuffers {
  void* q = nullptr;
  void* attn = nullptr;
  void* ws = nullptr;
  uint64_t ws_bytes = 0;
  void* pws = nullptr;
  uint64_t pws_bytes = 0;
};

// Rows the prefill of a call attends to: the ring for a rotating cache, else [0, offset + T).
int32_t prefill_rows(const ema_kvcache_desc& d, int64_t offset, int32_t T) {
  if (d.flags & EMA_KV_ROTATING) return d.capacity;
  const int64_t n = offset + T;
  return (int32_t)(n < d.capacity ? n : d.capacity);
}

uint64_t prefill_ws_bytes(const ema_kvcache_desc& d, int32_t rows) {
  uint64_t need = 0;
  check(ema_prefill_workspace_size(&d, rows, &need), "prefill_workspace_size");
  return need;
}

// Carved first (the decode workspace must start the arena).
CoreBuffers take_core(Arena& arena, const GqaConfig& c, int32_t T, const ema_kvcache_desc& d, int32_t offset) {
  CoreBuffers b;
  const size_t HD = (size_t)c.n_heads * c.head_dim;
  if (T == 1) {
    b.ws_bytes = decode_ws_bytes(c, d.capacity);
    b.ws = arena.take_decode_workspace((size_t)b.ws_bytes);
  }
  if (T > 1) b.q = arena.take(HD * T * 2);
  b.attn = arena.take((size_t)T * HD * 2);
  if (T > 1 && d.dtype != EMA_DTYPE_BF16) {
    b.pws_bytes = prefill_ws_bytes(d, prefill_rows(d, offset, T));
    b.pws = arena.take((size_t)b.pws_bytes);
  }
  return b;
}

// The attention layer over any cache, on q|k|v rows already in device memory:
// pre-attention writes the chunk's K/V (quantised for an FP8 cache, ring rows for a
// rotating one) and causal prefill attends (T > 1, gqa.rs:78), or the fused decode step
// does both (T == 1).
void check_range(const HipKvCache& cache, int32_t offset, int32_t T, const std::string& name) {
  const int32_t cap = cache.capacity();
  if (!cache.rotating() && (offset < 0 || (int64_t)offset + T > cap))
    throw Error(EMA_ERR_CAPACITY, "static KV overflow offset=" + std::to_string((int64_t)offset + T - 1) +
                                      " cap=" + std::to_string(cap));
  if (cache.rotating() && (offset < 0 || T > cap))
    throw Error(EMA_ERR_CAPACITY, name + ": " + std::to_string(T) + " tokens exceed the window " + std::to_string(cap));
}

void attend(const Ctx& ctx, const void* qkv, int32_t T, const std::optional<Array>& q_norm,
            const std::optional<Array>& k_norm, HipKvCache& cache, const GqaConfig& config, int32_t offset,
            const CoreBuffers& buf) {
  const int32_t Hq = config.n_heads, Hkv = config.n_kv_heads, D = config.head_dim;
  const ema_kvcache_desc& d = cache.desc();
  const int32_t cap = d.capacity;
  // optional_qk_norm (crates/ops/src/attention.rs:57-76): each norm on its own
  uint32_t flags = 0;
  if (!q_norm) flags |= EMA_PRE_NO_Q_NORM;
  if (!k_norm) flags |= EMA_PRE_NO_K_NORM;
  if (!config.use_rope) flags |= EMA_PRE_NO_ROPE;
  const void* qw = q_norm ? q_norm->data : nullptr;
  const void* kw = k_norm ? k_norm->data : nullptr;
  const float scale = 1.0f / std::sqrt((float)D);  // crates/attention/src/gqa.rs:73
  const int32_t* pos = cache.position(ctx, offset);
  if (T > 1) {  // is_prefill (gqa.rs:78): causal over the cache
    if (d.dtype == EMA_DTYPE_BF16) {
      check(ema_pre_attention(ctx.stream, qkv, qw, kw, config.norm_eps, config.rope_theta, pos, 1, T, Hq, Hkv, D,
                              flags, buf.q, &d),
            "pre_attention");
      check(ema_prefill_attention(ctx.stream, buf.q, &d, pos, T, Hq, scale, EMA_PREFILL_CAUSAL, buf.attn),
            "prefill_attention");
    } else {
      // FP8: pre-attention also puts the chunk's decoded rows into the prefill's bf16 copy,
      // so the prefill decodes only earlier rows (none for a static cache's first chunk,
      // whose keys are the chunk's own)
      const int32_t rows = prefill_rows(d, offset, T);
      check(ema_pre_attention_ws(ctx.stream, qkv, qw, kw, config.norm_eps, config.rope_theta, pos, 1, T, Hq, Hkv, D,
                                 flags, buf.q, &d, rows, buf.pws, buf.pws_bytes),
            "pre_attention_ws");
      uint32_t pf = EMA_PREFILL_CAUSAL | EMA_PREFILL_ROWS_DECODED;
      if (offset == 0 && !cache.rotating()) pf |= EMA_PREFILL_CHUNK_ONLY;
      check(ema_prefill_attention_ws(ctx.stream, buf.q, &d, pos, T, Hq, scale, pf, buf.attn, rows, buf.pws,
                                     buf.pws_bytes),
            "prefill_attention_ws");
    }
  } else {  // the decode step writes the row at the offset and attends offset + 1 rows
    const int32_t max_len = offset + 1 < cap ? offset + 1 : cap;
    check(ema_decode_step(ctx.stream, qkv, qw, kw, config.norm_eps, config.rope_theta, const_cast<int32_t*>(pos),
                          max_len, Hq, flags, scale, &d, buf.attn, buf.ws, buf.ws_bytes),
          "decode_step");
  }
  cache.set_len((int64_t)offset + T);
}

void check_cache_config(const HipKvCache& cache, const GqaConfig& config, const std::string& name) {
  check_config(config, name);
  if (config.n_kv_heads != cache.n_kv_heads() || config.head_dim != cache.head_dim())
    throw Error(EMA_ERR_SHAPE, name + ": config does not match the cache");
}

int32_t seq_len_of(const Array& a, int64_t width, const std::string& name, const char* what) {
  if (!a.data || a.shape.size() != 3 || a.shape[0] != 1 || a.shape[2] != width || !a.strides.empty() ||
      a.shape[1] <= 0 || a.shape[1] > INT32_MAX)
    throw Error(EMA_ERR_SHAPE, name + ": " + what + " must be contiguous [1, seq, " + std::to_string(width) +
                                   "], got " + shape_str(a.shape));
  return (int32_t)a.shape[1];
}

Array qkv_layer(const Ctx& ctx, const Array& qkv, const std::optional<Array>& q_norm,
                const std::optional<Array>& k_norm, HipKvCache& cache, const GqaConfig& config, int32_t offset,
                const std::string& name) {
  check_cache_config(cache, config, name);
  const int32_t T = seq_len_of(qkv, (int64_t)(config.n_heads + 2 * config.n_kv_heads) * config.head_dim, name, "qkv");
  check_range(cache, offset, T, name);
  Arena arena(ctx, name.c_str());
  const CoreBuffers buf = take_core(arena, config, T, cache.desc(), offset);
  arena.check();
  attend(ctx, qkv.data, T, q_norm, k_norm, cache, config, offset, buf);
  Array r;
  r.data = buf.attn;
  r.shape = {1, T, (int64_t)config.n_heads * config.head_dim};
  return r;
}

// A projection's weights for y = x W^T with W [N, K].
void check_proj(const QuantWeights& w, int32_t N, int32_t K, const std::string& name, const char* which) {
  const std::string what = name + ": " + which;
  if (!w.is_quantized())
    throw Error(EMA_ERR_UNSUPPORTED, what + " holds plain (dequantized) weights; only MLX affine-quantised ones "
                                            "are supported");
  if (!w.mode || std::string(w.mode) != "affine")
    throw Error(EMA_ERR_UNSUPPORTED, what + ": quantisation mode '" + (w.mode ? w.mode : "") + "' (affine only)");
  if (w.bits <= 0 || 32 % w.bits || K % w.group_size)
    throw Error(EMA_ERR_SHAPE, what + ": bits " + std::to_string(w.bits) + " / group_size " +
                                   std::to_string(w.group_size) + " do not fit K=" + std::to_string(K));
  const std::vector<int64_t> ws = {N, (int64_t)K * w.bits / 32}, ss = {N, K / w.group_size};
  if (w.weight.shape != ws || w.scales.shape != ss || w.biases.shape != ss || !w.weight.data || !w.scales.data ||
      !w.biases.data)
    throw Error(EMA_ERR_SHAPE, what + ": expected weight " + shape_str(ws) + " and scales/biases " + shape_str(ss) +
                                   ", got " + shape_str(w.weight.shape) + " / " + shape_str(w.scales.shape) + " / " +
                                   shape_str(w.biases.shape));
}

// One projection y[:, col:col+N] = x W^T (ldy = the row width of y), weights checked.
void project(const Ctx& ctx, const void* x, int64_t ldx, const QuantWeights& w, int32_t M, int32_t N, int32_t K,
             void* y, int64_t ldy) {
  check(ema_quantized_matmul(ctx.stream, x, ldx, (const uint32_t*)w.weight.data, w.scales.data, w.biases.data, y, ldy,
                             M, N, K, w.group_size, w.bits, EMA_DTYPE_BF16),
        "quantized_matmul");
}

// gqa.rs:62-107: project q, k, v into one q|k|v row (run_qkv's separate pieces without
// the concatenation, crates/serve/src/forward/projection.rs:105-128), attend, o_proj
// (attend_and_project, crates/ops/src/attention.rs:162-177).
Array gqa_layer(const Ctx& ctx, const Array& x, const GqaWeights& w, HipKvCache& cache, const GqaConfig& config,
                int32_t offset, const std::string& name) {
  check_cache_config(cache, config, name);
  if (!x.data || x.shape.size() != 3 || x.shape[2] <= 0)
    throw Error(EMA_ERR_SHAPE, name + ": x must be contiguous [1, seq, hidden], got " + shape_str(x.shape));
  const int64_t hidden = x.shape[2];
  if (hidden > INT32_MAX) throw Error(EMA_ERR_SHAPE, name + ": hidden size too large");
  const int32_t T = seq_len_of(x, hidden, name, "x");
  const int32_t Hq = config.n_heads, Hkv = config.n_kv_heads, D = config.head_dim;
  const int64_t F = (int64_t)(Hq + 2 * Hkv) * D;
  check_range(cache, offset, T, name);
  const int32_t K = (int32_t)hidden;
  check_proj(w.q_proj, Hq * D, K, name, "q_proj");
  check_proj(w.k_proj, Hkv * D, K, name, "k_proj");
  check_proj(w.v_proj, Hkv * D, K, name, "v_proj");
  check_proj(w.o_proj, K, Hq * D, name, "o_proj");
  Arena arena(ctx, name.c_str());
  const CoreBuffers buf = take_core(arena, config, T, cache.desc(), offset);
  void* qkv = arena.take((size_t)T * F * 2);
  void* y = arena.take((size_t)T * hidden * 2);
  arena.check();
  project(ctx, x.data, hidden, w.q_proj, T, Hq * D, K, qkv, F);
  project(ctx, x.data, hidden, w.k_proj, T, Hkv * D, K, (char*)qkv + (size_t)Hq * D * 2, F);
  project(ctx, x.data, hidden, w.v_proj, T, Hkv * D, K, (char*)qkv + (size_t)(Hq + Hkv) * D * 2, F);
  attend(ctx, qkv, T, w.q_norm, w.k_norm, cache, config, offset, buf);
  project(ctx, buf.attn, (int64_t)Hq * D, w.o_proj, T, K, Hq * D, y, hidden);
  Array r;
  r.data = y;
  r.shape = {1, T, hidden};
  return r;
}

}  // namespace

size_t qkv_attention_workspace_bytes(const GqaConfig& config, int32_t max_seq_len, int32_t capacity) {
  check_config(config, "qkv_attention_workspace_bytes");
  const size_t HD = (size_t)config.n_heads * config.head_dim, T = (size_t)(max_seq_len > 1 ? max_seq_len : 1);
  return aligned(HD * T * 2) + aligned(T * HD * 2) + aligned((size_t)decode_ws_bytes(config, capacity));
}

size_t qkv_attention_workspace_bytes(const GqaConfig& config, int32_t max_seq_len, const HipKvCache& cache) {
  const ema_kvcache_desc& d = cache.desc();
  size_t bytes = qkv_attention_workspace_bytes(config, max_seq_len, d.capacity);
  if (max_seq_len > 1 && d.dtype != EMA_DTYPE_BF16) bytes += aligned((size_t)prefill_ws_bytes(d, d.capacity));
  return bytes;
}

size_t gqa_workspace_bytes(const GqaConfig& config, int64_t hidden_size, int32_t max_seq_len, int32_t capacity) {
  const size_t T = (size_t)(max_seq_len > 1 ? max_seq_len : 1);
  const size_t F = (size_t)(config.n_heads + 2 * config.n_kv_heads) * config.head_dim;
  return aligned(T * F * 2) + aligned(T * (size_t)hidden_size * 2) +
         qkv_attention_workspace_bytes(config, max_seq_len, capacity);
}

size_t gqa_workspace_bytes(const GqaConfig& config, int64_t hidden_size, int32_t max_seq_len,
                           const HipKvCache& cache) {
  const size_t T = (size_t)(max_seq_len > 1 ? max_seq_len : 1);
  const size_t F = (size_t)(config.n_heads + 2 * config.n_kv_heads) * config.head_dim;
  return aligned(T * F * 2) + aligned(T * (size_t)hidden_size * 2) +
         qkv_attention_workspace_bytes(config, max_seq_len, cache);
}

Array gqa_attention(const Ctx& ctx, const Array& x, const GqaWeights& weights, HipKvCache& cache,
                    const GqaConfig& config, int32_t offset) {
  return gqa_layer(ctx, x, weights, cache, config, offset, "gqa_attention");
}

Array sliding_window_attention(const Ctx& ctx, const Array& x, const GqaWeights& weights, HipKvCache& cache,
                               const SlidingWindowConfig& config, int32_t offset) {
  // The reference delegates to gqa_attention and leaves the window to the cache backend
  // (crates/attention/src/sliding_window.rs:40-50): a ring enforces it.
  if (cache.rotating() && config.window_size != (size_t)cache.capacity())
    throw Error(EMA_ERR_SHAPE, "sliding_window_attention: window_size " + std::to_string(config.window_size) +
                                   " differs from the cache's " + std::to_string(cache.capacity()));
  return gqa_layer(ctx, x, weights, cache, config.gqa, offset, "sliding_window_attention");
}

Array qkv_attention(const Ctx& ctx, const Array& qkv, const std::optional<Array>& q_norm,
                    const std::optional<Array>& k_norm, HipKvCache& cache, const GqaConfig& config, int32_t offset) {
  return qkv_layer(ctx, qkv, q_norm, k_norm, cache, config, offset, "qkv_attention");
}

}  // namespace ema
