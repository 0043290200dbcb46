// Shared device/host helpers for the gfx950 attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "ema_attn.h"

namespace ema {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

// bf16 bits -> f32 (exact).
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// f32 -> bf16, round to nearest even (gfx950 v_cvt_pk_bf16_f32; the same
// rounding rule as the oracle for every finite value).
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// c + a.lo*b.lo + a.hi*b.hi over bf16 pairs, f32 accumulate (v_dot2_f32_bf16). Takes the
// pairs by value: clang's __builtin_bit_cast of a vector-element lvalue reads element 0.
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c, false);
}

// 16x16x32 bf16 MFMA, f32 accumulate. Lane layout (checked on gfx950):
//   A[16 x 32]: lane l holds row l%16, k = 8*(l/16) .. +7
//   B[32 x 16]: lane l holds col l%16, k = 8*(l/16) .. +7
//   C[16 x 16]: lane l holds col l%16, rows 4*(l/16) .. +3
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
// 32x32x16 bf16 MFMA. Lane layout (checked on gfx950):
//   A[32 x 16]: lane l holds row l%32, k = 8*(l/32) .. +7
//   B[16 x 32]: lane l holds col l%32, k = 8*(l/32) .. +7
//   C[32 x 32]: lane l holds col l%32, rows (i%4) + 8*(i/4) + 4*(l/32), i = 0..15
__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// s_waitcnt vmcnt(0) (gfx9 encoding: expcnt and lgkmcnt left at their maxima).
// Issued once after loads that stay live across a pipelined loop, so the
// compiler's conservative loop-header wait does not make every iteration wait
// for the loop's own prefetch.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

__device__ __forceinline__ float wave_max_xor(float v, int mask) {
  return fmaxf(v, __shfl_xor(v, mask, 64));
}

// ---- FP8 E4M3FN KV rows (the quantisation of crates/ops/src/fp8.rs:71-92) ----
// Scale exponent of one 64-element block from this lane's share (amax over the 8 lanes
// of the head): ceil(log2(amax / 448)) with amax = max(1e-4, max |x|). The logarithm is
// taken in double and rounded to f32 before the ceiling, which reproduces an f32 log2
// rounded to nearest (the reference's f32::log2) also just above powers of two.
__device__ __forceinline__ int fp8_block_exp(float amax_lane) {
  float amax = fmaxf(amax_lane, 1.0e-4f);
  amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
  amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
  amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
  return (int)ceilf((float)log2((double)(amax / 448.0f)));
}

// 8 values (bf16 bits) -> 8 E4M3FN codes of v * 2^-e: clamp to +-448 (NaN -> +448, as
// the reference's f32::min does), round to nearest even; -0 is stored as +0.
__device__ __forceinline__ u32x2 fp8_encode8(const uint16_t* x, int e) {
  const float inv = ldexpf(1.0f, -e);
  float y[8];
  for (int i = 0; i < 8; ++i) {
    float t = bf16_to_f32(x[i]) * inv;
    t = t != t ? 448.0f : fminf(fmaxf(t, -448.0f), 448.0f);
    y[i] = t + 0.0f;
  }
  u32x2 w;
  for (int h = 0; h < 2; ++h) {
    int d = __builtin_amdgcn_cvt_pk_fp8_f32(y[4 * h], y[4 * h + 1], 0, false);
    d = __builtin_amdgcn_cvt_pk_fp8_f32(y[4 * h + 2], y[4 * h + 3], d, true);
    w[h] = (uint32_t)d;
  }
  return w;
}
// 8 E4M3FN codes -> 8 bf16 values code * 2^e (exact), value i from byte i
__device__ __forceinline__ u32x4 fp8_decode8(u32x2 w, int e) {
  const float sc = __uint_as_float((uint32_t)(e + 127) << 23);
  u32x4 o;
  o[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w[0], sc, false));
  o[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w[0], sc, true));
  o[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w[1], sc, false));
  o[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w[1], sc, true));
  return o;
}

// ---- 4-bit affine KV rows (MLX "affine" quantisation, group 64) ----
// Parameters of one group with minimum mn and maximum mx, as MLX's affine quantiser forms
// them: scale = max((mx - mn) / 15, 1e-7), negated unless |mn| > |mx|; the end of larger
// magnitude (the edge) is moved onto the grid, scale = edge / round(edge / scale), and is
// the bias (bias 0 and the unadjusted scale when round(edge / scale) is 0). f32 with
// correctly rounded division; round() is half away from zero.
__device__ __forceinline__ void i4_params(float mn, float mx, float& scale, float& bias) {
  float sc = fmaxf(__fdiv_rn(mx - mn, 15.0f), 1.0e-7f);
  const bool side = fabsf(mn) > fabsf(mx);
  sc = side ? sc : -sc;
  const float edge = side ? mn : mx;
  const float q0 = roundf(__fdiv_rn(edge, sc));
  const bool at_zero = q0 == 0.0f;
  scale = at_zero ? sc : __fdiv_rn(edge, q0);
  bias = at_zero ? 0.0f : edge;
}
// Code of x in its group: round((x - bias) / scale), at most 15 (and at least 0).
__device__ __forceinline__ uint32_t i4_code(float x, float scale, float bias) {
  const float t = fminf(roundf(__fdiv_rn(x - bias, scale)), 15.0f);
  return t > 0.0f ? (uint32_t)t : 0u;
}
// Quantise and store one 128-value row held by 8 consecutive lanes, lane j (= lane8) with
// values 8j .. 8j+7 in x[0..8) and 64+8j .. 64+8j+7 in x[8..16): words[j] and words[8 + j]
// get the codes (value i at bits 4(i % 8)), *scale_pair / *bias_pair the two groups' bf16
// parameters (group 0 in the low half), written by lane j = 0.
__device__ __forceinline__ void i4_store_row8(const float (&x)[16], uint32_t* words, uint32_t* scale_pair,
                                              uint32_t* bias_pair, int lane8) {
  float mn0 = x[0], mx0 = x[0], mn1 = x[8], mx1 = x[8];
  for (int e = 1; e < 8; ++e) {
    mn0 = fminf(mn0, x[e]);
    mx0 = fmaxf(mx0, x[e]);
    mn1 = fminf(mn1, x[8 + e]);
    mx1 = fmaxf(mx1, x[8 + e]);
  }
  for (int o = 4; o >= 1; o >>= 1) {
    mn0 = fminf(mn0, __shfl_xor(mn0, o, 8));
    mx0 = fmaxf(mx0, __shfl_xor(mx0, o, 8));
    mn1 = fminf(mn1, __shfl_xor(mn1, o, 8));
    mx1 = fmaxf(mx1, __shfl_xor(mx1, o, 8));
  }
  float s0, b0, s1, b1;
  i4_params(mn0, mx0, s0, b0);
  i4_params(mn1, mx1, s1, b1);
  uint32_t w0 = 0u, w1 = 0u;
  for (int e = 0; e < 8; ++e) {
    w0 |= i4_code(x[e], s0, b0) << (4 * e);
    w1 |= i4_code(x[8 + e], s1, b1) << (4 * e);
  }
  words[lane8] = w0;
  words[8 + lane8] = w1;
  if (lane8 == 0) {
    *scale_pair = f32_to_bf16_bits(s0) | (f32_to_bf16_bits(s1) << 16);
    *bias_pair = f32_to_bf16_bits(b0) | (f32_to_bf16_bits(b1) << 16);
  }
}

}  // namespace ema

// ---------------------------------------------------------------- host side
namespace ema {

// Sets the thread-local error message and returns `code`.
int32_t set_error(int32_t code, const char* fmt, ...);
// Compute units of the current device (queried once per device).
int device_cus();
// Raises `fn`'s dynamic LDS limit to `bytes` once per device; bit d of *done records
// device d (thread-safe).
int32_t allow_lds_once(const void* fn, int bytes, std::atomic<uint64_t>* done, const char* what);
// Maps a HIP error to EMA_ERR_HIP with context, or returns EMA_OK.
int32_t check_hip(hipError_t e, const char* what);

// copy (fp8 cache only, else null): also write each stored K and V row, decoded to bf16,
// into row `row` of the prefill's bf16 copy [2][B, Hkv, copy_rows, D] (rows past copy_rows
// are not written)
int32_t launch_pre_attention(hipStream_t s, const void* qkv, const void* qw, const void* kw,
                             float eps, float theta, const int32_t* off, int B, int T, int Hq,
                             int Hkv, int D, uint32_t flags, void* q_out,
                             const ema_kvcache_desc& c, void* copy = nullptr, int copy_rows = 0);

// Arrival counters at the start of every decode workspace: one per (sequence, kv head)
// segment, then one for the grid. The region has a fixed size, so that a workspace reused
// across shapes never holds partial states where a later call keeps counters. Every call
// returns the counters it uses to zero; the region must be zero before the first call.
constexpr int kDecodeCounterSlots = 32768;
constexpr uint64_t kDecodeCounterBytes = (uint64_t)kDecodeCounterSlots * sizeof(int32_t);
static_assert(kDecodeCounterBytes == EMA_DECODE_COUNTER_BYTES, "counter region of the public header");

struct DecodePlan {
  int workers;        // independent wave workers over the flattened (b, kv-head, tile) space
  int segments;       // B * Hkv
  uint64_t part_bytes;  // partial (m, l, o) slots: (workers + segments) pieces
};
DecodePlan plan_decode(int B, int Hq, int Hkv, int D, int max_len);
uint64_t decode_workspace_bytes(const DecodePlan& plan);
// Pre-attention inputs of the fused decode step (ema_decode_step).
struct FusedPre {
  const void* qkv;
  const void* q_norm_w;
  const void* k_norm_w;
  int32_t* offsets;  // advanced in place with EMA_STEP_ADVANCE
  float eps;
  float theta;
  uint32_t flags;
};
int32_t launch_decode(hipStream_t s, const void* q, const ema_kvcache_desc& c, const int32_t* len,
                      int Hq, float scale, void* out, void* ws, const DecodePlan& plan,
                      const FusedPre* fused = nullptr);

int32_t launch_prefill(hipStream_t s, const void* q, const ema_kvcache_desc& c,
                       const int32_t* q_off, int T, int Hq, float scale, uint32_t flags,
                       void* out);
// Gated DeltaNet recurrent scan (arguments validated by the caller).
int32_t launch_gdn_scan(hipStream_t s, const void* q, const void* k, const void* v, const float* g,
                        const float* beta, float* state, void* y, int B, int T, int hk, int hv, int dk,
                        int dv, int dtype);
// Chunkwise scan on the matrix cores (bf16 activations, n_tokens >= kGdnChunkMinTokens).
constexpr int kGdnChunkTokens = 32;  // tokens per chunk
constexpr int kGdnChunkMinTokens = 32;
int32_t launch_gdn_chunked(hipStream_t s, const void* q, const void* k, const void* v, const float* g,
                           const float* beta, float* state, void* y, int B, int T, int hk, int hv, int dk,
                           int dv);
// WY-form scan over a workspace (bf16, n_tokens >= kGdnChunkMinTokens, dv <= 512): bytes of
// one chunk's records, and the launcher (segments the sequence to the workspace).
constexpr int kGdnWyMaxDv = 512;
uint64_t gdn_wy_chunk_bytes(int B, int hk, int hv, int dk, int dv);
int32_t launch_gdn_wy(hipStream_t s, const void* q, const void* k, const void* v, const float* g, const float* beta,
                      float* state, void* y, int B, int T, int hk, int hv, int dk, int dv, void* ws,
                      uint64_t ws_bytes);
// Affine-quantised matmul y = x W^T over MLX-packed W (arguments validated by the caller).
int32_t launch_qmatmul(hipStream_t s, const void* x, int64_t ldx, const void* w, const void* scales,
                       const void* biases, void* y, int64_t ldy, int M, int N, int K, int gs, int bits,
                       int dtype);
// Quantise bf16 cache rows into an int4 affine cache (arguments validated by the caller).
int32_t launch_quantize_int4(hipStream_t s, const ema_kvcache_desc& src, int src_row, const ema_kvcache_desc& dst,
                             int dst_row, int n_rows);
// Decode the fp8 rows a prefill call attends to into bf16 [B, Hkv, R, D] K then V at ws.
int32_t launch_fp8_convert(hipStream_t s, const ema_kvcache_desc& src, int src_row, const ema_kvcache_desc& dst,
                           int dst_row, int n_rows);
int32_t launch_fp8_to_bf16(hipStream_t s, const ema_kvcache_desc& c, const int32_t* q_off, int T,
                           uint32_t flags, int R, void* ws);

}  // namespace ema
