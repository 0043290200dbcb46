// C++ host API of the attention hot path: the reference's KvCache trait and
// gqa_attention, restated over the ema_attn C ABI.
//
//   reference (dangranaz/engine-mlx 0.1.18)                  here
//   -------------------------------------------------------  ----------------------------
//   trait KvCache            crates/kvcache/src/lib.rs:52-76  class KvCache
//   static KV state + alloc  crates/serve/src/engine.rs:31-42,
//                            crates/serve/src/engine_ext.rs:266-306
//                                                            class StaticCache
//   struct RotatingCache     crates/kvcache/src/rotating.rs:22-122  class RotatingCache (a ring)
//   struct Fp8Cache          crates/kvcache/src/fp8.rs:27-91    class Fp8Cache (codes + exponents)
//   C: KvCache (the generic parameter of gqa_attention, gqa.rs:62-69)
//                                                            class HipKvCache
//   struct GqaConfig         crates/attention/src/gqa.rs:27-42  struct GqaConfig
//   struct QuantWeights      crates/ops/src/quant.rs:16-40      struct QuantWeights (affine)
//   struct GqaWeights        crates/attention/src/gqa.rs:45-53  struct GqaWeights
//   fn gqa_attention         crates/attention/src/gqa.rs:62-107 gqa_attention
//   fn sliding_window_attention crates/attention/src/sliding_window.rs:40-50
//                                                            sliding_window_attention
//   MlxCtx (stream + allocator)                              struct Ctx (stream + arena)
//
// The layer functions take any HipKvCache (the reference's gqa_attention<C: KvCache>,
// crates/attention/src/gqa.rs:62-69, whose documented use passes an Fp8Cache or a
// RotatingCache, crates/attention/src/lib.rs:22-27): a KvCache that can also hand the
// kernels its descriptor and a device position.
// gqa_attention takes the hidden state x [1, T, hidden] and returns [1, T, hidden]: the
// q, k and v projections (ema_quantized_matmul into one q|k|v row), the q/k norms, RoPE
// and the cache write (ema_pre_attention, or the fused ema_decode_step for T == 1), the
// attention (ema_prefill_attention for T > 1), then o_proj (ema_quantized_matmul).
// qkv_attention is the same layer without the projections.
// Errors are thrown as ema::Error with the reference's message texts
// ("KV cache is empty", "static KV overflow offset=.. cap=..").
#pragma once

#include <cstddef>
#include <cstdint>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "ema_attn.h"

#define EMA_HOST_API __attribute__((visibility("default")))

namespace ema {

class EMA_HOST_API Error : public std::runtime_error {
 public:
  Error(int32_t code, const std::string& msg) : std::runtime_error(msg), code_(code) {}
  int32_t code() const { return code_; }

 private:
  int32_t code_;
};

// Analogue of MlxCtx for this path: the HIP stream work is enqueued on, and the device
// arena the layer calls take their temporaries from (the role of MLX's allocator): q|k|v
// rows, q, the attention output, the o_proj output and the decode split's state. The
// caller sizes it once (gqa_workspace_bytes / qkv_attention_workspace_bytes), zero-fills
// it once (its first EMA_DECODE_COUNTER_BYTES hold the decode split's arrival counters,
// which every call leaves at zero) and no call allocates device memory. An Array a call
// returns that points into the arena stays valid until the next call that uses the same
// arena.
struct Ctx {
  ema_stream_t stream = nullptr;
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
};

// Analogue of mlx_array for this path: a non-owning view of a bf16 device
// tensor. `strides` are in elements; empty means contiguous.
struct Array {
  void* data = nullptr;
  std::vector<int64_t> shape;
  std::vector<int64_t> strides;
  int64_t numel() const;
};

class EMA_HOST_API KvCache {
 public:
  virtual ~KvCache() = default;
  // Append new K and V, shape [1, n_kv_heads, seq_len, head_dim] (attention order).
  virtual void append(const Ctx& ctx, const Array& k, const Array& v) = 0;
  // The full accumulated K and V, [1, n_kv_heads, total_seq, head_dim].
  virtual std::pair<Array, Array> get(const Ctx& ctx) const = 0;
  virtual size_t len() const = 0;
  bool is_empty() const { return len() == 0; }
  virtual void reset() = 0;
  virtual size_t memory_bytes() const = 0;
};

// A cache the attention layer runs over: the KvCache methods, plus the descriptor the
// kernels read (buffers, format, ring flag), a device int32 holding a call's position, and
// the length bookkeeping of a call that wrote its rows in place.
class EMA_HOST_API HipKvCache : public KvCache {
 public:
  virtual const ema_kvcache_desc& desc() const = 0;
  // Device pointer to an int32 holding p (0 <= p < 2^31; a static cache: p <= capacity),
  // valid for work enqueued on ctx's stream after this call.
  virtual const int32_t* position(const Ctx& ctx, int64_t p) const = 0;
  // The cache holds the tokens [0, n) (a ring: the last `capacity` of them).
  virtual void set_len(int64_t n) = 0;
  bool rotating() const { return (desc().flags & EMA_KV_ROTATING) != 0; }
  int32_t capacity() const { return desc().capacity; }
  int32_t n_kv_heads() const { return desc().n_kv_heads; }
  int32_t head_dim() const { return desc().head_dim; }
};

// Device table of the int32 values 0, 1, ..., n (the analogue of the pre-built
// static_offsets scalars, crates/serve/src/engine_ext.rs:293-299), so a step passes its
// offset without a host-to-device copy.
class EMA_HOST_API PositionTable {
 public:
  explicit PositionTable(int32_t n);
  ~PositionTable();
  PositionTable(const PositionTable&) = delete;
  PositionTable& operator=(const PositionTable&) = delete;
  const int32_t* at(int32_t p) const { return table_ + p; }

 private:
  int32_t* table_ = nullptr;
};

// Static pre-allocated bf16 cache of one layer, [1, Hkv, capacity, head_dim],
// allocated zeroed once (alloc_kv_static) and reused: reset() rewinds the
// offset only, stale rows stay and are excluded by the valid length.
class EMA_HOST_API StaticCache final : public HipKvCache {
 public:
  StaticCache(int32_t n_kv_heads, int32_t capacity, int32_t head_dim);
  ~StaticCache() override;
  StaticCache(const StaticCache&) = delete;
  StaticCache& operator=(const StaticCache&) = delete;

  void append(const Ctx& ctx, const Array& k, const Array& v) override;
  std::pair<Array, Array> get(const Ctx& ctx) const override;
  size_t len() const override { return (size_t)offset_; }
  void reset() override { offset_ = 0; }
  size_t memory_bytes() const override;

  const ema_kvcache_desc& desc() const override { return desc_; }
  // Device pointer to the int32 value p, 0 <= p <= capacity (the static_offsets analogue).
  const int32_t* device_position(int32_t p) const;
  const int32_t* position(const Ctx&, int64_t p) const override;
  // Record that rows [offset, offset + n) were written in place.
  void advance(int32_t n);
  void set_len(int64_t n) override;

 private:
  ema_kvcache_desc desc_{};
  int32_t offset_ = 0;
  PositionTable positions_;  // 0, 1, ..., capacity
};

// Rotating (sliding-window) bf16 cache of one layer: the reference's RotatingCache
// (crates/kvcache/src/rotating.rs:22-122), which keeps the last window_size tokens, held
// as a ring [1, Hkv, window_size, head_dim] (EMA_KV_ROTATING): the token at position p
// lives in row p % window_size, so an append writes rows in place instead of
// concatenating and slicing. len() = min(tokens seen, window_size) (rotating.rs:108-110).
class EMA_HOST_API RotatingCache final : public HipKvCache {
 public:
  RotatingCache(int32_t window_size, int32_t n_kv_heads, int32_t head_dim);
  ~RotatingCache() override;
  RotatingCache(const RotatingCache&) = delete;
  RotatingCache& operator=(const RotatingCache&) = delete;

  // Appends at positions [total, total + T); with T > window_size only the last
  // window_size tokens are kept (rotating.rs:81-92).
  void append(const Ctx& ctx, const Array& k, const Array& v) override;
  // The held tokens in order, [1, Hkv, len, head_dim]: the ring itself until it wraps,
  // then a rotated copy in ctx's arena (2 * Hkv * window * head_dim * 2 bytes; valid
  // until the next call that uses the arena).
  std::pair<Array, Array> get(const Ctx& ctx) const override;
  size_t len() const override { return total_ < (int64_t)desc_.capacity ? (size_t)total_ : (size_t)desc_.capacity; }
  void reset() override { total_ = 0; }
  size_t memory_bytes() const override;

  int32_t window_size() const { return desc_.capacity; }
  int64_t total_len() const { return total_; }
  const ema_kvcache_desc& desc() const override { return desc_; }
  // Device pointer to an int32 slot holding p (0 <= p < 2^31), written on ctx's stream
  // by ema_position_write (stream-ordered: a later call rewrites it after the work that
  // read it).
  const int32_t* position(const Ctx& ctx, int64_t p) const override;
  // Record that the tokens [total, total + n) were written in place.
  void advance(int32_t n) { total_ += n; }
  void set_len(int64_t n) override { total_ = n; }

 private:
  ema_kvcache_desc desc_{};
  int64_t total_ = 0;
  int32_t* slot_ = nullptr;  // device int32 [1], allocated with the cache
};

// FP8 E4M3FN cache of one layer: the reference's Fp8Cache (crates/kvcache/src/fp8.rs:27-91,
// which keeps the E4M3FN round trip of every 64-value block of each K/V row), stored as
// one code byte per value plus one exponent byte per block ([1, Hkv, capacity, head_dim]
// codes, [1, Hkv, capacity, head_dim / 64] exponents, ema_kvcache_alloc_fp8), allocated
// zeroed once with a static capacity; reset() rewinds the length only. The layer calls
// quantise the rows they write (ema_pre_attention / ema_decode_step) and attend the
// decoded values. n_rot is the reference's unquantised RoPE tail of each head
// (Fp8Cache::new(head_dim, n_rot), fp8.rs:38-54): 0, or 64, whose dims 64..127 are stored
// as bf16 (other values: EMA_ERR_UNSUPPORTED). head_dim 128.
class EMA_HOST_API Fp8Cache final : public HipKvCache {
 public:
  Fp8Cache(int32_t n_kv_heads, int32_t capacity, int32_t head_dim, int32_t n_rot = 0);
  ~Fp8Cache() override;
  Fp8Cache(const Fp8Cache&) = delete;
  Fp8Cache& operator=(const Fp8Cache&) = delete;

  // Quantises K and V [1, Hkv, T, head_dim] bf16 into rows [len, len + T).
  void append(const Ctx& ctx, const Array& k, const Array& v) override;
  // The held rows decoded to bf16 (exactly the values the reference keeps), [1, Hkv, len,
  // head_dim] each, in ctx's arena (2 * Hkv * len * head_dim * 2 bytes; valid until the
  // next call that uses the arena).
  std::pair<Array, Array> get(const Ctx& ctx) const override;
  size_t len() const override { return (size_t)offset_; }
  void reset() override { offset_ = 0; }
  size_t memory_bytes() const override;
  const ema_kvcache_desc& desc() const override { return desc_; }
  const int32_t* position(const Ctx&, int64_t p) const override;
  void set_len(int64_t n) override;
  int32_t n_rot() const { return desc_.n_rot; }

 private:
  ema_kvcache_desc desc_{};
  int32_t offset_ = 0;
  PositionTable positions_;
};

struct GqaConfig {
  int32_t n_heads = 0;
  int32_t n_kv_heads = 0;
  int32_t head_dim = 0;
  float rope_theta = 1e6f;
  float norm_eps = 1e-6f;
  bool use_rope = true;
};

// A quantised linear layer, MLX affine format (crates/ops/src/quant.rs:16-40):
// weight [N, K * bits / 32] uint32 (lowest bits first), scales and biases
// [N, K / group_size] bf16; y = x W^T. group_size 0 (plain weights) and the mxfp4 mode
// are refused with EMA_ERR_UNSUPPORTED.
struct QuantWeights {
  Array weight;
  Array scales;
  Array biases;
  int32_t bits = 4;
  int32_t group_size = 64;
  const char* mode = "affine";
  bool is_quantized() const { return group_size > 0; }
};

// crates/attention/src/gqa.rs:45-53: the four projections and the optional per-head
// q/k RMSNorm weights ([head_dim] bf16), each norm optional on its own.
struct GqaWeights {
  QuantWeights q_proj, k_proj, v_proj, o_proj;
  std::optional<Array> q_norm;
  std::optional<Array> k_norm;
};

struct SlidingWindowConfig {
  GqaConfig gqa;
  size_t window_size = 0;
};

// Arena bytes gqa_attention needs for up to max_seq_len tokens of hidden size
// `hidden_size` over `cache` (an FP8 cache's prefill adds its bf16 copy of the attended
// rows), or over a bf16 cache of `capacity` rows (the window for a rotating cache).
EMA_HOST_API size_t gqa_workspace_bytes(const GqaConfig& config, int64_t hidden_size, int32_t max_seq_len,
                                        const HipKvCache& cache);
EMA_HOST_API size_t gqa_workspace_bytes(const GqaConfig& config, int64_t hidden_size, int32_t max_seq_len,
                                        int32_t capacity);
// Arena bytes qkv_attention needs.
EMA_HOST_API size_t qkv_attention_workspace_bytes(const GqaConfig& config, int32_t max_seq_len,
                                                  const HipKvCache& cache);
EMA_HOST_API size_t qkv_attention_workspace_bytes(const GqaConfig& config, int32_t max_seq_len, int32_t capacity);

// x [1, T, hidden] bf16 -> [1, T, hidden] bf16 (in ctx's arena), over any HipKvCache (the
// reference's gqa_attention<C: KvCache>). K/V of positions [offset, offset + T) are written
// (quantised for an FP8 cache, to ring rows for a rotating one) and the cache length
// becomes offset + T. T > 1: causal attention over the cache rows [0, offset + T)
// (gqa.rs:78, is_prefill; a ring: the window the cache holds after the append, keys
// [max(0, offset + T - window), p] for query position p, and T must not exceed the
// window); T == 1: decode over offset + 1 rows (a ring: the last window of them).
EMA_HOST_API Array gqa_attention(const Ctx& ctx, const Array& x, const GqaWeights& weights, HipKvCache& cache,
                                 const GqaConfig& config, int32_t offset);

// crates/attention/src/sliding_window.rs:40-50: gqa_attention with the window left to the
// cache. Over a RotatingCache the window is enforced, and config.window_size must equal
// the cache's; any other cache attends as gqa_attention does (the reference's comment:
// "Any KvCache implementation can be passed, but RotatingCache gives the intended sliding
// window behavior").
EMA_HOST_API Array sliding_window_attention(const Ctx& ctx, const Array& x, const GqaWeights& weights,
                                            HipKvCache& cache, const SlidingWindowConfig& config, int32_t offset);

// The layer without its projections: qkv [1, T, (Hq + 2*Hkv) * head_dim] (the q|k|v
// rows) -> the o_proj input [1, T, Hq * head_dim] (in ctx's arena). Same cache
// semantics as gqa_attention.
EMA_HOST_API Array qkv_attention(const Ctx& ctx, const Array& qkv, const std::optional<Array>& q_norm,
                                 const std::optional<Array>& k_norm, HipKvCache& cache, const GqaConfig& config,
                                 int32_t offset);

}  // namespace ema
