// C ABI of the attention hot path: argument validation and dispatch.
//
// Error behaviour follows the reference's FFI wrapper: every call returns a
// status, 0 = OK (crates/mlx-ffi/src/ops/real/mod.rs:35-40 turns a non-zero
// mlx-c status into "MLX op '<op>' failed with code <n>"); here the message
// is kept in a thread-local string readable through ema_last_error().
// Validation runs on the host before any HIP call, so every argument error is
// reported without touching the GPU.
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "ema_common.hpp"

namespace ema {

static thread_local char g_err[512] = "";

int32_t set_error(int32_t code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int32_t check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return EMA_OK;
  return set_error(EMA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

namespace {
constexpr int kMaxDevices = 64;
int current_device() {
  int dev = 0;
  return hipGetDevice(&dev) == hipSuccess && dev >= 0 && dev < kMaxDevices ? dev : 0;
}
}  // namespace

int device_cus() {
  static std::atomic<int> cached[kMaxDevices];
  const int dev = current_device();
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int32_t allow_lds_once(const void* fn, int bytes, std::atomic<uint64_t>* done, const char* what) {
  const uint64_t bit = 1ull << current_device();
  if (done->load(std::memory_order_acquire) & bit) return EMA_OK;
  const int32_t rc = check_hip(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes), what);
  if (rc == EMA_OK) done->fetch_or(bit, std::memory_order_release);
  return rc;
}

}  // namespace ema

using namespace ema;

namespace {

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// ema_position_write: one lane stores the value (a vector store; the address depends on
// the lane index, so the compiler does not turn it into a scalar store).
__global__ void position_write_kernel(int32_t* dst, int32_t v) {
  if (threadIdx.x < 1) dst[threadIdx.x] = v;
}

int32_t check_cache(const char* op, const ema_kvcache_desc* c) {
  if (!c) return set_error(EMA_ERR_INVALID_ARG, "%s: cache descriptor is null", op);
  if (!c->k || !c->v) return set_error(EMA_ERR_INVALID_ARG, "%s: KV cache is empty (null K/V buffer)", op);
  if (c->dtype != EMA_DTYPE_BF16 && c->dtype != EMA_DTYPE_FP8_E4M3 && c->dtype != EMA_DTYPE_INT4_AFFINE)
    return set_error(EMA_ERR_INVALID_ARG, "%s: cache dtype %d is not bf16, fp8 e4m3 or int4 affine", op, c->dtype);
  if (c->dtype == EMA_DTYPE_FP8_E4M3) {
    if (!c->k_exp || !c->v_exp) return set_error(EMA_ERR_INVALID_ARG, "%s: fp8 cache without block exponents", op);
    if (c->head_dim != 128)
      return set_error(EMA_ERR_UNSUPPORTED, "%s: fp8 cache with head_dim %d not supported (128)", op, c->head_dim);
    if (c->stride_pos % 16 || c->stride_head % 16 || c->stride_batch % 16)
      return set_error(EMA_ERR_SHAPE, "%s: fp8 cache strides must be multiples of 16 bytes", op);
    if (c->n_rot != 0 && c->n_rot != 64)
      return set_error(EMA_ERR_UNSUPPORTED, "%s: fp8 cache n_rot %d not supported (0 or 64)", op, c->n_rot);
    if (c->stride_pos < (int64_t)c->head_dim + c->n_rot)
      return set_error(EMA_ERR_SHAPE, "%s: fp8 cache rows with n_rot %d need stride_pos >= %d bytes", op, c->n_rot,
                       c->head_dim + c->n_rot);
  } else if (c->n_rot != 0) {
    return set_error(EMA_ERR_INVALID_ARG, "%s: n_rot %d is an fp8 cache field (0 for other dtypes)", op, c->n_rot);
  }
  if (c->dtype == EMA_DTYPE_INT4_AFFINE) {
    if (!c->k_scales || !c->k_biases || !c->v_scales || !c->v_biases)
      return set_error(EMA_ERR_INVALID_ARG, "%s: int4 cache without scales/biases", op);
    if (!aligned16(c->k_scales) || !aligned16(c->k_biases) || !aligned16(c->v_scales) || !aligned16(c->v_biases))
      return set_error(EMA_ERR_INVALID_ARG, "%s: int4 scales/biases must be 16-byte aligned", op);
    if (c->head_dim != 128)
      return set_error(EMA_ERR_UNSUPPORTED, "%s: int4 cache with head_dim %d not supported (128)", op, c->head_dim);
    if (c->capacity % 32)
      return set_error(EMA_ERR_UNSUPPORTED, "%s: int4 cache capacity %d is not a multiple of 32", op, c->capacity);
    if (c->stride_pos % 32 || c->stride_head % 32 || c->stride_batch % 32)
      return set_error(EMA_ERR_SHAPE, "%s: int4 cache strides must be multiples of 32 elements (16 bytes)", op);
  }
  if (c->flags & ~EMA_KV_ROTATING) return set_error(EMA_ERR_INVALID_ARG, "%s: unknown cache flags 0x%x", op, c->flags);
  if (c->batch <= 0 || c->n_kv_heads <= 0 || c->capacity <= 0 || c->head_dim <= 0)
    return set_error(EMA_ERR_SHAPE, "%s: cache dims must be positive (batch=%d n_kv_heads=%d capacity=%d head_dim=%d)",
                     op, c->batch, c->n_kv_heads, c->capacity, c->head_dim);
  if (c->head_dim % 8 != 0) return set_error(EMA_ERR_SHAPE, "%s: head_dim %d is not a multiple of 8", op, c->head_dim);
  if (c->stride_pos < c->head_dim || c->stride_pos % 8 || c->stride_head % 8 || c->stride_batch % 8 ||
      c->stride_head < 0 || c->stride_batch < 0)
    return set_error(EMA_ERR_SHAPE, "%s: cache strides must be >= head_dim and multiples of 8 elements", op);
  if (!aligned16(c->k) || !aligned16(c->v)) return set_error(EMA_ERR_INVALID_ARG, "%s: cache buffers must be 16-byte aligned", op);
  return EMA_OK;
}

// Static scratch of ema_decode_step_noalloc (the split's header and partial softmax
// states), one copy per device, held until the process ends. In host code `scratch` is only
// a stand-in for the symbol: its device address comes from hipGetSymbolAddress, looked up
// once per device with that device current, and only that address is passed to kernels.
// Its first EMA_DECODE_COUNTER_BYTES hold the split's arrival counters, which must read
// zero when a call starts: a __device__ array is zero when the library is loaded, and every
// call returns each counter it uses to zero before it ends (the last workgroup to arrive at
// a counter resets it). The rest (the tile prefix and the partial states) is written before
// it is read within each call, so it needs no clearing. Calls that overlap on one device
// share the array and race.
__device__ __align__(256) unsigned char scratch[EMA_NOALLOC_SCRATCH_BYTES];
std::atomic<void*> g_scratch_addr[kMaxDevices];
std::mutex g_scratch_mu;

int32_t noalloc_scratch(const char* op, void** addr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(EMA_ERR_HIP, "%s: no usable current device (%d)", op, dev);
  void* p = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (!p) {
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p)
        return set_error(EMA_ERR_HIP, "%s: static scratch address on device %d: %s", op, dev, hipGetErrorString(e));
      g_scratch_addr[dev].store(p, std::memory_order_release);
    }
  }
  *addr = p;
  return EMA_OK;
}

int32_t check_heads(const char* op, int32_t Hq, int32_t Hkv) {
  if (Hq <= 0 || Hkv <= 0) return set_error(EMA_ERR_SHAPE, "%s: head counts must be positive (n_heads=%d n_kv_heads=%d)", op, Hq, Hkv);
  if (Hq % Hkv) return set_error(EMA_ERR_SHAPE, "%s: n_heads %d is not a multiple of n_kv_heads %d", op, Hq, Hkv);
  return EMA_OK;
}

}  // namespace

extern "C" {

const char* ema_last_error(void) { return g_err; }

const char* ema_version(void) { return "ema_attn 0.1.0 (gfx950)"; }

int32_t ema_kvcache_init(ema_kvcache_desc* d, void* k, void* v, int32_t batch, int32_t n_kv_heads,
                         int32_t capacity, int32_t head_dim) {
  if (!d) return set_error(EMA_ERR_INVALID_ARG, "ema_kvcache_init: descriptor is null");
  memset(d, 0, sizeof(*d));
  d->k = k;
  d->v = v;
  d->batch = batch;
  d->n_kv_heads = n_kv_heads;
  d->capacity = capacity;
  d->head_dim = head_dim;
  d->stride_pos = head_dim;
  d->stride_head = (int64_t)capacity * head_dim;
  d->stride_batch = (int64_t)n_kv_heads * capacity * head_dim;
  d->dtype = EMA_DTYPE_BF16;
  return check_cache("ema_kvcache_init", d);
}

int32_t ema_kvcache_alloc(ema_kvcache_desc* out, int32_t batch, int32_t n_kv_heads, int32_t capacity,
                          int32_t head_dim) {
  if (!out) return set_error(EMA_ERR_INVALID_ARG, "ema_kvcache_alloc: descriptor is null");
  memset(out, 0, sizeof(*out));
  if (batch <= 0 || n_kv_heads <= 0 || capacity <= 0 || head_dim <= 0 || head_dim % 8)
    return set_error(EMA_ERR_SHAPE, "ema_kvcache_alloc: bad dims (batch=%d n_kv_heads=%d capacity=%d head_dim=%d)",
                     batch, n_kv_heads, capacity, head_dim);
  const size_t bytes = (size_t)batch * n_kv_heads * capacity * head_dim * 2;
  void *k = nullptr, *v = nullptr;
  int32_t rc = check_hip(hipMalloc(&k, bytes), "ema_kvcache_alloc: hipMalloc K");
  if (rc) return rc;
  rc = check_hip(hipMalloc(&v, bytes), "ema_kvcache_alloc: hipMalloc V");
  if (rc) {
    (void)hipFree(k);
    return rc;
  }
  rc = check_hip(hipMemset(k, 0, bytes), "ema_kvcache_alloc: zero K");
  if (!rc) rc = check_hip(hipMemset(v, 0, bytes), "ema_kvcache_alloc: zero V");
  if (rc) {
    (void)hipFree(k);
    (void)hipFree(v);
    return rc;
  }
  return ema_kvcache_init(out, k, v, batch, n_kv_heads, capacity, head_dim);
}

int32_t ema_kvcache_init_fp8(ema_kvcache_desc* d, void* k, void* v, void* k_exp, void* v_exp, int32_t batch,
                             int32_t n_kv_heads, int32_t capacity, int32_t head_dim, int32_t n_rot) {
  if (!d) return set_error(EMA_ERR_INVALID_ARG, "ema_kvcache_init_fp8: descriptor is null");
  memset(d, 0, sizeof(*d));
  d->k = k;
  d->v = v;
  d->k_exp = k_exp;
  d->v_exp = v_exp;
  d->batch = batch;
  d->n_kv_heads = n_kv_heads;
  d->capacity = capacity;
  d->head_dim = head_dim;
  d->n_rot = n_rot;
  // a row: head_dim - n_rot code bytes, then n_rot bf16 values
  const int64_t row = (int64_t)head_dim + n_rot;
  d->stride_pos = row;
  d->stride_head = (int64_t)capacity * row;
  d->stride_batch = (int64_t)n_kv_heads * capacity * row;
  d->dtype = EMA_DTYPE_FP8_E4M3;
  return check_cache("ema_kvcache_init_fp8", d);
}

int32_t ema_kvcache_alloc_fp8(ema_kvcache_desc* out, int32_t batch, int32_t n_kv_heads, int32_t capacity,
                              int32_t head_dim, int32_t n_rot) {
  const char* op = "ema_kvcache_alloc_fp8";
  if (!out) return set_error(EMA_ERR_INVALID_ARG, "%s: descriptor is null", op);
  memset(out, 0, sizeof(*out));
  if (batch <= 0 || n_kv_heads <= 0 || capacity <= 0 || head_dim != 128)
    return set_error(head_dim != 128 && head_dim > 0 ? EMA_ERR_UNSUPPORTED : EMA_ERR_SHAPE,
                     "%s: bad dims (batch=%d n_kv_heads=%d capacity=%d head_dim=%d; fp8 needs head_dim 128)", op,
                     batch, n_kv_heads, capacity, head_dim);
  if (n_rot != 0 && n_rot != 64)
    return set_error(EMA_ERR_UNSUPPORTED, "%s: n_rot %d not supported (0 or 64)", op, n_rot);
  const size_t rows = (size_t)batch * n_kv_heads * capacity;
  const size_t code_bytes = rows * (head_dim + n_rot), exp_bytes = rows * (head_dim / 64);
  void* p[4] = {nullptr, nullptr, nullptr, nullptr};
  const size_t sz[4] = {code_bytes, code_bytes, exp_bytes, exp_bytes};
  int32_t rc = EMA_OK;
  for (int i = 0; i < 4 && !rc; ++i) {
    rc = check_hip(hipMalloc(&p[i], sz[i]), "ema_kvcache_alloc_fp8: hipMalloc");
    if (!rc) rc = check_hip(hipMemset(p[i], 0, sz[i]), "ema_kvcache_alloc_fp8: zero");
  }
  if (rc) {
    for (int i = 0; i < 4; ++i)
      if (p[i]) (void)hipFree(p[i]);
    return rc;
  }
  return ema_kvcache_init_fp8(out, p[0], p[1], p[2], p[3], batch, n_kv_heads, capacity, head_dim, n_rot);
}

int32_t ema_kvcache_init_int4(ema_kvcache_desc* d, void* k, void* v, void* k_scales, void* k_biases,
                              void* v_scales, void* v_biases, int32_t batch, int32_t n_kv_heads, int32_t capacity,
                              int32_t head_dim) {
  if (!d) return set_error(EMA_ERR_INVALID_ARG, "ema_kvcache_init_int4: descriptor is null");
  memset(d, 0, sizeof(*d));
  d->k = k;
  d->v = v;
  d->k_scales = k_scales;
  d->k_biases = k_biases;
  d->v_scales = v_scales;
  d->v_biases = v_biases;
  d->batch = batch;
  d->n_kv_heads = n_kv_heads;
  d->capacity = capacity;
  d->head_dim = head_dim;
  d->stride_pos = head_dim;  // in 4-bit elements
  d->stride_head = (int64_t)capacity * head_dim;
  d->stride_batch = (int64_t)n_kv_heads * capacity * head_dim;
  d->dtype = EMA_DTYPE_INT4_AFFINE;
  return check_cache("ema_kvcache_init_int4", d);
}

int32_t ema_kvcache_alloc_int4(ema_kvcache_desc* out, int32_t batch, int32_t n_kv_heads, int32_t capacity,
                               int32_t head_dim) {
  const char* op = "ema_kvcache_alloc_int4";
  if (!out) return set_error(EMA_ERR_INVALID_ARG, "%s: descriptor is null", op);
  memset(out, 0, sizeof(*out));
  if (batch <= 0 || n_kv_heads <= 0 || capacity <= 0 || head_dim != 128 || capacity % 32)
    return set_error(head_dim > 0 && capacity > 0 ? EMA_ERR_UNSUPPORTED : EMA_ERR_SHAPE,
                     "%s: bad dims (batch=%d n_kv_heads=%d capacity=%d head_dim=%d; int4 needs head_dim 128 and "
                     "a capacity that is a multiple of 32)", op, batch, n_kv_heads, capacity, head_dim);
  const size_t rows = (size_t)batch * n_kv_heads * capacity;
  const size_t word_bytes = rows * head_dim / 2, meta_bytes = rows * (head_dim / 64) * 2;
  void* p[6] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
  const size_t sz[6] = {word_bytes, word_bytes, meta_bytes, meta_bytes, meta_bytes, meta_bytes};
  int32_t rc = EMA_OK;
  for (int i = 0; i < 6 && !rc; ++i) {
    rc = check_hip(hipMalloc(&p[i], sz[i]), "ema_kvcache_alloc_int4: hipMalloc");
    if (!rc) rc = check_hip(hipMemset(p[i], 0, sz[i]), "ema_kvcache_alloc_int4: zero");
  }
  if (rc) {
    for (int i = 0; i < 6; ++i)
      if (p[i]) (void)hipFree(p[i]);
    return rc;
  }
  return ema_kvcache_init_int4(out, p[0], p[1], p[2], p[3], p[4], p[5], batch, n_kv_heads, capacity, head_dim);
}

int32_t ema_kvcache_quantize_int4(ema_stream_t stream, const ema_kvcache_desc* src, int32_t src_row,
                                  const ema_kvcache_desc* dst, int32_t dst_row, int32_t n_rows) {
  const char* op = "ema_kvcache_quantize_int4";
  int32_t rc = check_cache(op, src);
  if (rc) return rc;
  if ((rc = check_cache(op, dst))) return rc;
  if (src->dtype != EMA_DTYPE_BF16 || dst->dtype != EMA_DTYPE_INT4_AFFINE)
    return set_error(EMA_ERR_INVALID_ARG, "%s: needs a bf16 source and an int4 destination (dtypes %d, %d)", op,
                     src->dtype, dst->dtype);
  if (src->batch != dst->batch || src->n_kv_heads != dst->n_kv_heads || src->head_dim != dst->head_dim)
    return set_error(EMA_ERR_SHAPE, "%s: source (%d, %d, %d) and destination (%d, %d, %d) shapes differ", op,
                     src->batch, src->n_kv_heads, src->head_dim, dst->batch, dst->n_kv_heads, dst->head_dim);
  if (n_rows < 0 || src_row < 0 || dst_row < 0 || (int64_t)src_row + n_rows > src->capacity ||
      (int64_t)dst_row + n_rows > dst->capacity)
    return set_error(EMA_ERR_CAPACITY, "%s: rows [%d, +%d) of the source (capacity %d) or [%d, +%d) of the "
                     "destination (capacity %d) out of range", op, src_row, n_rows, src->capacity, dst_row, n_rows,
                     dst->capacity);
  if (n_rows == 0) return EMA_OK;
  return launch_quantize_int4((hipStream_t)stream, *src, src_row, *dst, dst_row, n_rows);
}

int32_t ema_kvcache_convert(ema_stream_t stream, const ema_kvcache_desc* src, int32_t src_row,
                            const ema_kvcache_desc* dst, int32_t dst_row, int32_t n_rows) {
  const char* op = "ema_kvcache_convert";
  int32_t rc = check_cache(op, src);
  if (rc) return rc;
  if ((rc = check_cache(op, dst))) return rc;
  const bool to_int4 = src->dtype == EMA_DTYPE_BF16 && dst->dtype == EMA_DTYPE_INT4_AFFINE;
  const bool to_fp8 = src->dtype == EMA_DTYPE_BF16 && dst->dtype == EMA_DTYPE_FP8_E4M3;
  const bool from_fp8 = src->dtype == EMA_DTYPE_FP8_E4M3 && dst->dtype == EMA_DTYPE_BF16;
  if (!to_int4 && !to_fp8 && !from_fp8)
    return set_error(EMA_ERR_UNSUPPORTED, "%s: converts bf16 -> fp8, fp8 -> bf16 and bf16 -> int4 rows (dtypes %d -> %d)",
                     op, src->dtype, dst->dtype);
  if (src->batch != dst->batch || src->n_kv_heads != dst->n_kv_heads || src->head_dim != dst->head_dim)
    return set_error(EMA_ERR_SHAPE, "%s: source (%d, %d, %d) and destination (%d, %d, %d) shapes differ", op,
                     src->batch, src->n_kv_heads, src->head_dim, dst->batch, dst->n_kv_heads, dst->head_dim);
  if (n_rows < 0 || src_row < 0 || dst_row < 0 || (int64_t)src_row + n_rows > src->capacity ||
      (int64_t)dst_row + n_rows > dst->capacity)
    return set_error(EMA_ERR_CAPACITY, "%s: rows [%d, +%d) of the source (capacity %d) or [%d, +%d) of the "
                     "destination (capacity %d) out of range", op, src_row, n_rows, src->capacity, dst_row, n_rows,
                     dst->capacity);
  if ((src->dtype == EMA_DTYPE_BF16 && (src->stride_pos % 8 || src->stride_head % 8 || src->stride_batch % 8)) ||
      (dst->dtype == EMA_DTYPE_BF16 && (dst->stride_pos % 8 || dst->stride_head % 8 || dst->stride_batch % 8)))
    return set_error(EMA_ERR_SHAPE, "%s: bf16 strides must be multiples of 8 elements", op);
  if (n_rows == 0) return EMA_OK;
  if (to_int4) return launch_quantize_int4((hipStream_t)stream, *src, src_row, *dst, dst_row, n_rows);
  return launch_fp8_convert((hipStream_t)stream, *src, src_row, *dst, dst_row, n_rows);
}

int32_t ema_position_write(ema_stream_t stream, int32_t* slot, int32_t value) {
  if (!slot) return set_error(EMA_ERR_INVALID_ARG, "ema_position_write: slot is null");
  if (((uintptr_t)slot & 3u) != 0) return set_error(EMA_ERR_INVALID_ARG, "ema_position_write: slot is not 4-byte aligned");
  hipLaunchKernelGGL(position_write_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, slot, value);
  return check_hip(hipGetLastError(), "ema_position_write launch");
}

int32_t ema_kvcache_free(ema_kvcache_desc* d) {
  if (!d) return set_error(EMA_ERR_INVALID_ARG, "ema_kvcache_free: descriptor is null");
  int32_t rc = EMA_OK;
  void* const bufs[8] = {d->k, d->v, d->k_exp, d->v_exp, d->k_scales, d->k_biases, d->v_scales, d->v_biases};
  for (int i = 0; i < 8; ++i)
    if (bufs[i]) {
      const int32_t r2 = check_hip(hipFree(bufs[i]), "ema_kvcache_free");
      rc = rc ? rc : r2;
    }
  memset(d, 0, sizeof(*d));
  return rc;
}

int32_t ema_kvcache_memory_bytes(const ema_kvcache_desc* d, uint64_t* bytes) {
  if (!bytes) return set_error(EMA_ERR_INVALID_ARG, "ema_kvcache_memory_bytes: output is null");
  int32_t rc = check_cache("ema_kvcache_memory_bytes", d);
  if (rc) return rc;
  const uint64_t rows = 2ull * d->batch * d->n_kv_heads * d->capacity;  // K and V
  if (d->dtype == EMA_DTYPE_FP8_E4M3) *bytes = rows * (d->head_dim + d->n_rot + d->head_dim / 64);
  else if (d->dtype == EMA_DTYPE_INT4_AFFINE) *bytes = rows * (d->head_dim / 2 + 4ull * (d->head_dim / 64));
  else *bytes = rows * d->head_dim * 2ull;
  return EMA_OK;
}

// A norm weight may be null only when its norm is switched off.
static int32_t check_norm_weights(const char* op, const void* q_norm_w, const void* k_norm_w, uint32_t flags) {
  const bool q_norm = !(flags & (EMA_PRE_NO_NORM | EMA_PRE_NO_Q_NORM));
  const bool k_norm = !(flags & (EMA_PRE_NO_NORM | EMA_PRE_NO_K_NORM));
  if ((q_norm && !q_norm_w) || (k_norm && !k_norm_w))
    return set_error(EMA_ERR_INVALID_ARG,
                     "%s: norm weights are null (pass EMA_PRE_NO_NORM for models without q/k norm, "
                     "EMA_PRE_NO_Q_NORM / EMA_PRE_NO_K_NORM for one of them)", op);
  return EMA_OK;
}

static int32_t check_pre_attention(const char* op, const void* qkv, const void* q_norm_w, const void* k_norm_w,
                                   float eps, float theta, const int32_t* offsets, int32_t batch, int32_t n_tokens,
                                   int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, uint32_t flags,
                                   void* q_out, const ema_kvcache_desc* cache) {
  int32_t rc = check_cache(op, cache);
  if (rc) return rc;
  if (!qkv || !q_out || !offsets) return set_error(EMA_ERR_INVALID_ARG, "%s: null qkv/q_out/offsets", op);
  if (flags & ~(EMA_PRE_NO_NORM | EMA_PRE_NO_ROPE | EMA_PRE_NO_Q_NORM | EMA_PRE_NO_K_NORM))
    return set_error(EMA_ERR_INVALID_ARG, "%s: unknown flags 0x%x", op, flags);
  if ((rc = check_norm_weights(op, q_norm_w, k_norm_w, flags))) return rc;
  if ((rc = check_heads(op, n_heads, n_kv_heads))) return rc;
  if (batch <= 0 || n_tokens <= 0) return set_error(EMA_ERR_SHAPE, "%s: batch=%d n_tokens=%d must be positive", op, batch, n_tokens);
  if (batch != cache->batch || n_kv_heads != cache->n_kv_heads || head_dim != cache->head_dim)
    return set_error(EMA_ERR_SHAPE, "%s: shape (batch=%d n_kv_heads=%d head_dim=%d) does not match the cache (%d, %d, %d)",
                     op, batch, n_kv_heads, head_dim, cache->batch, cache->n_kv_heads, cache->head_dim);
  if (n_tokens > cache->capacity && !(cache->flags & EMA_KV_ROTATING))  // a ring keeps the last capacity
    return set_error(EMA_ERR_CAPACITY, "%s: static KV overflow: %d tokens exceed capacity %d", op, n_tokens, cache->capacity);
  if (!(eps >= 0.f) || !(theta > 0.f)) return set_error(EMA_ERR_INVALID_ARG, "%s: eps must be >= 0 and theta > 0", op);
  if (!aligned16(qkv) || !aligned16(q_out)) return set_error(EMA_ERR_INVALID_ARG, "%s: qkv/q_out must be 16-byte aligned", op);
  return EMA_OK;
}

int32_t ema_pre_attention(ema_stream_t stream, const void* qkv, const void* q_norm_w, const void* k_norm_w,
                          float eps, float theta, const int32_t* offsets, int32_t batch, int32_t n_tokens,
                          int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, uint32_t flags, void* q_out,
                          const ema_kvcache_desc* cache) {
  int32_t rc = check_pre_attention("ema_pre_attention", qkv, q_norm_w, k_norm_w, eps, theta, offsets, batch,
                                   n_tokens, n_heads, n_kv_heads, head_dim, flags, q_out, cache);
  if (rc) return rc;
  return launch_pre_attention((hipStream_t)stream, qkv, q_norm_w, k_norm_w, eps, theta, offsets, batch, n_tokens,
                              n_heads, n_kv_heads, head_dim, flags, q_out, *cache);
}

// declared below, with the prefill entry points
static int32_t prefill_copy_rows(const ema_kvcache_desc* c, int32_t max_kv_len);
static uint64_t prefill_ws_bytes(const ema_kvcache_desc* c, int32_t max_kv_len);

int32_t ema_pre_attention_ws(ema_stream_t stream, const void* qkv, const void* q_norm_w, const void* k_norm_w,
                             float eps, float theta, const int32_t* offsets, int32_t batch, int32_t n_tokens,
                             int32_t n_heads, int32_t n_kv_heads, int32_t head_dim, uint32_t flags, void* q_out,
                             const ema_kvcache_desc* cache, int32_t max_kv_len, void* workspace,
                             uint64_t workspace_bytes) {
  const char* op = "ema_pre_attention_ws";
  int32_t rc = check_pre_attention(op, qkv, q_norm_w, k_norm_w, eps, theta, offsets, batch, n_tokens, n_heads,
                                   n_kv_heads, head_dim, flags, q_out, cache);
  if (rc) return rc;
  if (cache->dtype != EMA_DTYPE_FP8_E4M3)
    return set_error(EMA_ERR_UNSUPPORTED, "%s: the prefill copy exists for FP8 caches only", op);
  if (max_kv_len < n_tokens || max_kv_len > cache->capacity)
    return set_error(EMA_ERR_CAPACITY, "%s: max_kv_len %d outside [n_tokens %d, capacity %d]", op, max_kv_len,
                     n_tokens, cache->capacity);
  const uint64_t need = prefill_ws_bytes(cache, max_kv_len);
  if (!workspace || workspace_bytes < need)
    return set_error(EMA_ERR_WORKSPACE, "%s: workspace of %llu bytes needed, %llu given", op,
                     (unsigned long long)need, (unsigned long long)(workspace ? workspace_bytes : 0));
  if (!aligned16(workspace)) return set_error(EMA_ERR_INVALID_ARG, "%s: workspace must be 16-byte aligned", op);
  return launch_pre_attention((hipStream_t)stream, qkv, q_norm_w, k_norm_w, eps, theta, offsets, batch, n_tokens,
                              n_heads, n_kv_heads, head_dim, flags, q_out, *cache, workspace,
                              prefill_copy_rows(cache, max_kv_len));
}

int32_t ema_decode_workspace_size(int32_t batch, int32_t n_heads, int32_t n_kv_heads, int32_t head_dim,
                                  int32_t max_len, uint64_t* bytes) {
  const char* op = "ema_decode_workspace_size";
  if (!bytes) return set_error(EMA_ERR_INVALID_ARG, "%s: output is null", op);
  int32_t rc = check_heads(op, n_heads, n_kv_heads);
  if (rc) return rc;
  if (batch <= 0 || head_dim <= 0 || max_len < 0) return set_error(EMA_ERR_SHAPE, "%s: bad dims", op);
  DecodePlan p = plan_decode(batch, n_heads, n_kv_heads, head_dim, max_len);
  *bytes = decode_workspace_bytes(p);
  return EMA_OK;
}

int32_t ema_decode_attention(ema_stream_t stream, const void* q, const ema_kvcache_desc* cache,
                             const int32_t* lengths, int32_t max_len, int32_t n_heads, float scale, void* out,
                             void* workspace, uint64_t workspace_bytes) {
  const char* op = "ema_decode_attention";
  int32_t rc = check_cache(op, cache);
  if (rc) return rc;
  if (!q || !out || !lengths) return set_error(EMA_ERR_INVALID_ARG, "%s: null q/out/lengths", op);
  if ((rc = check_heads(op, n_heads, cache->n_kv_heads))) return rc;
  if (max_len < 0 || max_len > cache->capacity)
    return set_error(EMA_ERR_CAPACITY, "%s: max_len %d outside [0, capacity %d]", op, max_len, cache->capacity);
  if (!(scale > 0.f)) return set_error(EMA_ERR_INVALID_ARG, "%s: scale must be > 0", op);
  if (!aligned16(q) || !aligned16(out)) return set_error(EMA_ERR_INVALID_ARG, "%s: q/out must be 16-byte aligned", op);
  DecodePlan p = plan_decode(cache->batch, n_heads, cache->n_kv_heads, cache->head_dim, max_len);
  const uint64_t need = decode_workspace_bytes(p);
  if (!workspace || workspace_bytes < need)
    return set_error(EMA_ERR_WORKSPACE, "%s: workspace of %llu bytes needed, %llu given", op,
                     (unsigned long long)need, (unsigned long long)(workspace ? workspace_bytes : 0));
  if (!aligned16(workspace)) return set_error(EMA_ERR_INVALID_ARG, "%s: workspace must be 16-byte aligned", op);
  return launch_decode((hipStream_t)stream, q, *cache, lengths, n_heads, scale, out, workspace, p);
}

static int32_t check_decode_step(const char* op, const void* qkv, const void* q_norm_w, const void* k_norm_w,
                                 float eps, float theta, const int32_t* offsets, int32_t max_len, int32_t n_heads,
                                 uint32_t flags, float scale, const ema_kvcache_desc* cache, void* out) {
  int32_t rc = check_cache(op, cache);
  if (rc) return rc;
  if (!qkv || !out || !offsets) return set_error(EMA_ERR_INVALID_ARG, "%s: null qkv/out/offsets", op);
  if (flags & ~(EMA_PRE_NO_NORM | EMA_PRE_NO_ROPE | EMA_PRE_NO_Q_NORM | EMA_PRE_NO_K_NORM | EMA_STEP_ADVANCE))
    return set_error(EMA_ERR_INVALID_ARG, "%s: unknown flags 0x%x", op, flags);
  if ((rc = check_norm_weights(op, q_norm_w, k_norm_w, flags))) return rc;
  if ((rc = check_heads(op, n_heads, cache->n_kv_heads))) return rc;
  if (max_len < 0 || max_len > cache->capacity)
    return set_error(EMA_ERR_CAPACITY, "%s: max_len %d outside [0, capacity %d]", op, max_len, cache->capacity);
  if (!(eps >= 0.f) || !(theta > 0.f) || !(scale > 0.f))
    return set_error(EMA_ERR_INVALID_ARG, "%s: eps must be >= 0, theta and scale > 0", op);
  if (!aligned16(qkv) || !aligned16(out)) return set_error(EMA_ERR_INVALID_ARG, "%s: qkv/out must be 16-byte aligned", op);
  return EMA_OK;
}

int32_t ema_decode_step(ema_stream_t stream, const void* qkv, const void* q_norm_w, const void* k_norm_w,
                        float eps, float theta, int32_t* offsets, int32_t max_len, int32_t n_heads,
                        uint32_t flags, float scale, const ema_kvcache_desc* cache, void* out, void* workspace,
                        uint64_t workspace_bytes) {
  const char* op = "ema_decode_step";
  int32_t rc = check_decode_step(op, qkv, q_norm_w, k_norm_w, eps, theta, offsets, max_len, n_heads, flags, scale,
                                 cache, out);
  if (rc) return rc;
  DecodePlan p = plan_decode(cache->batch, n_heads, cache->n_kv_heads, cache->head_dim, max_len);
  const uint64_t need = decode_workspace_bytes(p);
  if (!workspace || workspace_bytes < need)
    return set_error(EMA_ERR_WORKSPACE, "%s: workspace of %llu bytes needed, %llu given", op,
                     (unsigned long long)need, (unsigned long long)(workspace ? workspace_bytes : 0));
  if (!aligned16(workspace)) return set_error(EMA_ERR_INVALID_ARG, "%s: workspace must be 16-byte aligned", op);
  FusedPre f{qkv, q_norm_w, k_norm_w, offsets, eps, theta, flags};
  return launch_decode((hipStream_t)stream, nullptr, *cache, nullptr, n_heads, scale, out, workspace, p, &f);
}

int32_t ema_decode_step_noalloc(ema_stream_t stream, const void* qkv, const void* q_norm_w, const void* k_norm_w,
                                float eps, float theta, int32_t* offsets, int32_t max_len, int32_t n_heads,
                                uint32_t flags, float scale, const ema_kvcache_desc* cache, void* out) {
  const char* op = "ema_decode_step_noalloc";
  int32_t rc = check_decode_step(op, qkv, q_norm_w, k_norm_w, eps, theta, offsets, max_len, n_heads, flags, scale,
                                 cache, out);
  if (rc) return rc;
  DecodePlan p = plan_decode(cache->batch, n_heads, cache->n_kv_heads, cache->head_dim, max_len);
  const uint64_t need = decode_workspace_bytes(p);
  if (need > EMA_NOALLOC_SCRATCH_BYTES)
    return set_error(EMA_ERR_WORKSPACE,
                     "%s: this shape needs %llu bytes of scratch, more than the %llu-byte static scratch; "
                     "use ema_decode_step with a workspace",
                     op, (unsigned long long)need, (unsigned long long)EMA_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if ((rc = noalloc_scratch(op, &ws))) return rc;
  FusedPre f{qkv, q_norm_w, k_norm_w, offsets, eps, theta, flags};
  return launch_decode((hipStream_t)stream, nullptr, *cache, nullptr, n_heads, scale, out, ws, p, &f);
}

static int32_t check_prefill(const char* op, const void* q, const ema_kvcache_desc* cache,
                             const int32_t* q_offsets, int32_t n_tokens, int32_t n_heads, float scale,
                             uint32_t flags, void* out) {
  int32_t rc = check_cache(op, cache);
  if (rc) return rc;
  if (!q || !out || !q_offsets) return set_error(EMA_ERR_INVALID_ARG, "%s: null q/out/q_offsets", op);
  if (flags & ~(EMA_PREFILL_CAUSAL | EMA_PREFILL_CHUNK_ONLY | EMA_PREFILL_ROWS_DECODED))
    return set_error(EMA_ERR_INVALID_ARG, "%s: unknown flags 0x%x", op, flags);
  if ((flags & EMA_PREFILL_ROWS_DECODED) && cache->dtype != EMA_DTYPE_FP8_E4M3)
    return set_error(EMA_ERR_INVALID_ARG, "%s: EMA_PREFILL_ROWS_DECODED applies to FP8 caches only", op);
  if ((rc = check_heads(op, n_heads, cache->n_kv_heads))) return rc;
  if (n_tokens <= 0) return set_error(EMA_ERR_SHAPE, "%s: n_tokens %d must be positive", op, n_tokens);
  if (n_tokens > cache->capacity)
    return set_error(EMA_ERR_CAPACITY, "%s: %d tokens exceed capacity %d", op, n_tokens, cache->capacity);
  if (!(scale > 0.f)) return set_error(EMA_ERR_INVALID_ARG, "%s: scale must be > 0", op);
  if (!aligned16(q) || !aligned16(out)) return set_error(EMA_ERR_INVALID_ARG, "%s: q/out must be 16-byte aligned", op);
  return EMA_OK;
}

// Rows of the bf16 copy an FP8 prefill decodes into: max_kv_len for a static cache (rows at
// or past it are not attended); the whole ring for a rotating cache, whose positions sit at
// row p % capacity once they wrap, so a copy with fewer rows would put them elsewhere.
static int32_t prefill_copy_rows(const ema_kvcache_desc* c, int32_t max_kv_len) {
  return (c->flags & EMA_KV_ROTATING) ? c->capacity : max_kv_len;
}

static uint64_t prefill_ws_bytes(const ema_kvcache_desc* c, int32_t max_kv_len) {
  if (c->dtype != EMA_DTYPE_FP8_E4M3) return 0;
  return 2ull * (uint64_t)c->batch * c->n_kv_heads * (uint64_t)prefill_copy_rows(c, max_kv_len) * c->head_dim * 2ull;
}

int32_t ema_prefill_workspace_size(const ema_kvcache_desc* cache, int32_t max_kv_len, uint64_t* bytes) {
  const char* op = "ema_prefill_workspace_size";
  if (!bytes) return set_error(EMA_ERR_INVALID_ARG, "%s: output is null", op);
  int32_t rc = check_cache(op, cache);
  if (rc) return rc;
  if (max_kv_len <= 0 || max_kv_len > cache->capacity)
    return set_error(EMA_ERR_CAPACITY, "%s: max_kv_len %d outside (0, capacity %d]", op, max_kv_len, cache->capacity);
  *bytes = prefill_ws_bytes(cache, max_kv_len);
  return EMA_OK;
}

int32_t ema_prefill_attention_ws(ema_stream_t stream, const void* q, const ema_kvcache_desc* cache,
                                 const int32_t* q_offsets, int32_t n_tokens, int32_t n_heads, float scale,
                                 uint32_t flags, void* out, int32_t max_kv_len, void* workspace,
                                 uint64_t workspace_bytes) {
  const char* op = "ema_prefill_attention_ws";
  int32_t rc = check_prefill(op, q, cache, q_offsets, n_tokens, n_heads, scale, flags, out);
  if (rc) return rc;
  if (max_kv_len < n_tokens || max_kv_len > cache->capacity)
    return set_error(EMA_ERR_CAPACITY, "%s: max_kv_len %d outside [n_tokens %d, capacity %d]", op, max_kv_len,
                     n_tokens, cache->capacity);
  if (cache->dtype == EMA_DTYPE_BF16)
    return launch_prefill((hipStream_t)stream, q, *cache, q_offsets, n_tokens, n_heads, scale, flags, out);
  if (cache->dtype == EMA_DTYPE_INT4_AFFINE)
    return set_error(EMA_ERR_UNSUPPORTED, "%s: prefill over an int4 cache is not supported (attend a bf16 cache and "
                     "store the rows with ema_kvcache_quantize_int4)", op);
  const uint64_t need = prefill_ws_bytes(cache, max_kv_len);
  if (!workspace || workspace_bytes < need)
    return set_error(EMA_ERR_WORKSPACE, "%s: workspace of %llu bytes needed, %llu given", op,
                     (unsigned long long)need, (unsigned long long)(workspace ? workspace_bytes : 0));
  if (!aligned16(workspace)) return set_error(EMA_ERR_INVALID_ARG, "%s: workspace must be 16-byte aligned", op);
  if ((int64_t)cache->batch * cache->n_kv_heads > 65535)
    return set_error(EMA_ERR_UNSUPPORTED, "%s: batch * n_kv_heads exceeds 65535", op);
  const int32_t rows = prefill_copy_rows(cache, max_kv_len);
  rc = launch_fp8_to_bf16((hipStream_t)stream, *cache, q_offsets, n_tokens, flags, rows, workspace);
  if (rc) return rc;
  // the bf16 copy: [B, Hkv, rows, D] K then V
  ema_kvcache_desc w{};
  const int64_t per = (int64_t)cache->batch * cache->n_kv_heads * rows * cache->head_dim;
  w.k = workspace;
  w.v = (uint16_t*)workspace + per;
  w.batch = cache->batch;
  w.n_kv_heads = cache->n_kv_heads;
  w.capacity = rows;
  w.head_dim = cache->head_dim;
  w.stride_pos = cache->head_dim;
  w.stride_head = (int64_t)rows * cache->head_dim;
  w.stride_batch = (int64_t)cache->n_kv_heads * rows * cache->head_dim;
  w.dtype = EMA_DTYPE_BF16;
  // a ring stays a ring: the copy holds the cache's rows at the same row indices (the
  // whole ring, so wrapped positions land where the cache holds them)
  w.flags = cache->flags & EMA_KV_ROTATING;
  return launch_prefill((hipStream_t)stream, q, w, q_offsets, n_tokens, n_heads, scale,
                        flags & ~(uint32_t)EMA_PREFILL_ROWS_DECODED, out);
}

int32_t ema_prefill_attention(ema_stream_t stream, const void* q, const ema_kvcache_desc* cache,
                              const int32_t* q_offsets, int32_t n_tokens, int32_t n_heads, float scale,
                              uint32_t flags, void* out) {
  const char* op = "ema_prefill_attention";
  int32_t rc = check_cache(op, cache);
  if (rc) return rc;
  if (!q || !out || !q_offsets) return set_error(EMA_ERR_INVALID_ARG, "%s: null q/out/q_offsets", op);
  if (flags & ~(EMA_PREFILL_CAUSAL | EMA_PREFILL_CHUNK_ONLY))
    return set_error(EMA_ERR_INVALID_ARG, "%s: unknown flags 0x%x", op, flags);
  if ((rc = check_heads(op, n_heads, cache->n_kv_heads))) return rc;
  if (n_tokens <= 0) return set_error(EMA_ERR_SHAPE, "%s: n_tokens %d must be positive", op, n_tokens);
  if (n_tokens > cache->capacity)
    return set_error(EMA_ERR_CAPACITY, "%s: %d tokens exceed capacity %d", op, n_tokens, cache->capacity);
  if (!(scale > 0.f)) return set_error(EMA_ERR_INVALID_ARG, "%s: scale must be > 0", op);
  if (!aligned16(q) || !aligned16(out)) return set_error(EMA_ERR_INVALID_ARG, "%s: q/out must be 16-byte aligned", op);
  if (cache->dtype != EMA_DTYPE_BF16)
    return set_error(EMA_ERR_UNSUPPORTED, "%s: prefill over an %s cache is not supported (bf16 only)", op,
                     cache->dtype == EMA_DTYPE_FP8_E4M3 ? "fp8" : "int4");
  return launch_prefill((hipStream_t)stream, q, *cache, q_offsets, n_tokens, n_heads, scale, flags, out);
}

}  // extern "C"

static int32_t check_gdn_args(const char* op, const void* q, const void* k, const void* v, const float* g,
                              const float* beta, const float* state, const void* y, int32_t batch, int32_t n_tokens,
                              int32_t hk, int32_t hv, int32_t dk, int32_t dv, int32_t dtype) {
  if (!q || !k || !v || !g || !beta || !state || !y)
    return set_error(EMA_ERR_INVALID_ARG, "%s: null q/k/v/g/beta/state/y", op);
  if (dtype != EMA_DTYPE_BF16 && dtype != EMA_DTYPE_F16 && dtype != EMA_DTYPE_F32)
    return set_error(EMA_ERR_INVALID_ARG, "%s: dtype %d is not bf16, f16 or f32", op, dtype);
  if (batch <= 0 || n_tokens <= 0 || hk <= 0 || hv <= 0 || dk <= 0 || dv <= 0)
    return set_error(EMA_ERR_SHAPE, "%s: dims must be positive (batch=%d n_tokens=%d hk=%d hv=%d dk=%d dv=%d)", op,
                     batch, n_tokens, hk, hv, dk, dv);
  if (hv % hk) return set_error(EMA_ERR_SHAPE, "%s: hv %d is not a multiple of hk %d", op, hv, hk);
  if (dk != 64 && dk != 128) return set_error(EMA_ERR_UNSUPPORTED, "%s: dk %d not supported (64, 128)", op, dk);
  if (dv % 16) return set_error(EMA_ERR_SHAPE, "%s: dv %d is not a multiple of 16", op, dv);
  const uintptr_t el_align = dtype == EMA_DTYPE_F32 ? 3u : 1u;
  if (!aligned16(q) || !aligned16(k) || !aligned16(state) || ((uintptr_t)v | (uintptr_t)y) & el_align ||
      ((uintptr_t)g | (uintptr_t)beta) & 3u)
    return set_error(EMA_ERR_INVALID_ARG, "%s: misaligned buffer (q, k and state 16-byte aligned)", op);
  if ((int64_t)batch * n_tokens * hv * dv >= ((int64_t)1 << 31) || (int64_t)batch * hv * dv * dk >= ((int64_t)1 << 40))
    return set_error(EMA_ERR_SHAPE, "%s: tensors too large", op);
  return EMA_OK;
}

int32_t ema_gdn_scan(ema_stream_t stream, const void* q, const void* k, const void* v, const float* g,
                     const float* beta, float* state, void* y, int32_t batch, int32_t n_tokens, int32_t hk,
                     int32_t hv, int32_t dk, int32_t dv, int32_t dtype) {
  const int32_t rc = check_gdn_args("ema_gdn_scan", q, k, v, g, beta, state, y, batch, n_tokens, hk, hv, dk, dv, dtype);
  if (rc) return rc;
  return launch_gdn_scan((hipStream_t)stream, q, k, v, g, beta, state, y, batch, n_tokens, hk, hv, dk, dv, dtype);
}

int32_t ema_gdn_scan_workspace_size(int32_t batch, int32_t n_tokens, int32_t hk, int32_t hv, int32_t dk,
                                    int32_t dv, uint64_t* bytes) {
  const char* op = "ema_gdn_scan_workspace_size";
  if (!bytes) return set_error(EMA_ERR_INVALID_ARG, "%s: null bytes", op);
  *bytes = 0;
  if (batch <= 0 || n_tokens <= 0 || hk <= 0 || hv <= 0 || dv <= 0)
    return set_error(EMA_ERR_SHAPE, "%s: dims must be positive", op);
  if (hv % hk) return set_error(EMA_ERR_SHAPE, "%s: hv %d is not a multiple of hk %d", op, hv, hk);
  if (dk != 64 && dk != 128) return set_error(EMA_ERR_UNSUPPORTED, "%s: dk %d not supported (64, 128)", op, dk);
  if (dv % 16) return set_error(EMA_ERR_SHAPE, "%s: dv %d is not a multiple of 16", op, dv);
  const uint64_t chunks = (uint64_t)(n_tokens + kGdnChunkTokens - 1) / kGdnChunkTokens;
  *bytes = chunks * gdn_wy_chunk_bytes(batch, hk, hv, dk, dv);
  return EMA_OK;
}

int32_t ema_gdn_scan_ws(ema_stream_t stream, const void* q, const void* k, const void* v, const float* g,
                        const float* beta, float* state, void* y, int32_t batch, int32_t n_tokens, int32_t hk,
                        int32_t hv, int32_t dk, int32_t dv, int32_t dtype, void* workspace,
                        uint64_t workspace_bytes) {
  const char* op = "ema_gdn_scan_ws";
  const int32_t rc = check_gdn_args(op, q, k, v, g, beta, state, y, batch, n_tokens, hk, hv, dk, dv, dtype);
  if (rc) return rc;
  if (dtype != EMA_DTYPE_BF16 || n_tokens < kGdnChunkMinTokens || dv > kGdnWyMaxDv || !aligned16(v))
    return launch_gdn_scan((hipStream_t)stream, q, k, v, g, beta, state, y, batch, n_tokens, hk, hv, dk, dv, dtype);
  if (!workspace || !aligned16(workspace))
    return set_error(EMA_ERR_WORKSPACE, "%s: workspace missing or not 16-byte aligned", op);
  if (workspace_bytes < gdn_wy_chunk_bytes(batch, hk, hv, dk, dv))
    return set_error(EMA_ERR_WORKSPACE, "%s: workspace of %llu bytes is below one chunk's %llu", op,
                     (unsigned long long)workspace_bytes,
                     (unsigned long long)gdn_wy_chunk_bytes(batch, hk, hv, dk, dv));
  return launch_gdn_wy((hipStream_t)stream, q, k, v, g, beta, state, y, batch, n_tokens, hk, hv, dk, dv, workspace,
                       workspace_bytes);
}

int32_t ema_quantized_matmul(ema_stream_t stream, const void* x, int64_t ldx, const uint32_t* w, const void* scales,
                             const void* biases, void* y, int64_t ldy, int32_t M, int32_t N, int32_t K,
                             int32_t group_size, int32_t bits, int32_t dtype) {
  const char* op = "ema_quantized_matmul";
  if (M < 0 || N <= 0 || K <= 0)
    return set_error(EMA_ERR_SHAPE, "%s: need M >= 0 and positive N, K (M=%d N=%d K=%d)", op, M, N, K);
  if (M == 0) return EMA_OK;
  if (!x || !w || !scales || !biases || !y) return set_error(EMA_ERR_INVALID_ARG, "%s: null x/w/scales/biases/y", op);
  if (dtype != EMA_DTYPE_BF16 && dtype != EMA_DTYPE_F16)
    return set_error(EMA_ERR_INVALID_ARG, "%s: dtype %d is not bf16 or f16", op, dtype);
  if (bits != 4 && bits != 8) return set_error(EMA_ERR_UNSUPPORTED, "%s: bits %d not supported (4, 8)", op, bits);
  if (group_size != 32 && group_size != 64 && group_size != 128)
    return set_error(EMA_ERR_UNSUPPORTED, "%s: group_size %d not supported (32, 64, 128)", op, group_size);
  if (K % group_size) return set_error(EMA_ERR_SHAPE, "%s: K %d is not a multiple of group_size %d", op, K, group_size);
  if (ldx < K || ldy < N) return set_error(EMA_ERR_SHAPE, "%s: ldx %lld < K %d or ldy %lld < N %d", op, (long long)ldx, K,
                                           (long long)ldy, N);
  if (!aligned16(x) || !aligned16(w) || (ldx & 7) || ((uintptr_t)scales | (uintptr_t)biases | (uintptr_t)y) & 1u)
    return set_error(EMA_ERR_INVALID_ARG,
                     "%s: misaligned buffer (x and w 16-byte aligned, ldx a multiple of 8, scales/biases/y 2-byte)",
                     op);
  // 32-bit buffer offsets inside one 32 x 32 tile
  if (K > (1 << 20) || 31 * ldx + K >= ((int64_t)1 << 30) ||
      ((int64_t)(N + 31) / 32) * ((M + 31) / 32) >= ((int64_t)1 << 31))
    return set_error(EMA_ERR_SHAPE, "%s: tensors too large (K <= 2^20, 31 * ldx + K < 2^30)", op);
  return launch_qmatmul((hipStream_t)stream, x, ldx, w, scales, biases, y, ldy, M, N, K, group_size, bits, dtype);
}
