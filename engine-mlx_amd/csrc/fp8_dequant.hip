// FP8 E4M3FN cache rows -> bf16, for prefill over an FP8 cache (ema_prefill_attention_ws).
//
// The reference's FP8 cache hands SDPA its round-tripped values
// (crates/kvcache/src/fp8.rs:60-68, values of crates/ops/src/fp8.rs:71-92). Here the rows
// a prefill call attends to are decoded into a bf16 copy in the caller's workspace and the
// bf16 prefill kernel runs over that copy: code * 2^exp is exact in bf16, so the result is
// that of a bf16 cache holding the decoded values. HBM-bound: 130 bytes read and 256 bytes
// written per row of K or V, small next to the prefill's matrix work.
//
// Mapping: 8 threads per 128-dim row, 16 codes (one 16-byte load) each, 32 rows per
// 256-thread workgroup pass; blockIdx.y = (batch, kv head). Rows [lo, hi) of a sequence
// are decoded, hi = min(q_off + T, rows), lo = q_off with EMA_PREFILL_CHUNK_ONLY (0
// otherwise) -- exactly the rows the prefill kernel reads. A rotating cache (position p in
// row p % cap) has every held row decoded, lo = 0 (a chunk's rows may wrap the ring).
#include "ema_common.hpp"

namespace ema {
namespace {

constexpr int kD = 128;

struct DequantArgs {
  const uint8_t* k;
  const uint8_t* v;
  const uint16_t* kexp;  // [B, Hkv, cap] pairs of int8 block exponents
  const uint16_t* vexp;
  const int32_t* q_off;
  uint16_t* wk;  // [B, Hkv, R, D] bf16
  uint16_t* wv;
  int64_t sb, sh, sp;  // code strides (bytes)
  int Hkv, cap, R, T;
  uint32_t flags;
  int rot;
};

__global__ __launch_bounds__(256) void fp8_to_bf16_kernel(DequantArgs a) {
  const int bh = blockIdx.y;  // b * Hkv + kh
  const int b = bh / a.Hkv, kh = bh % a.Hkv;
  int q_off = a.q_off[b];
  q_off = q_off < 0 ? 0 : q_off;
  int hi = q_off + a.T;
  hi = hi < a.cap ? hi : a.cap;
  hi = hi < a.R ? hi : a.R;
  int lo = (a.flags & EMA_PREFILL_CHUNK_ONLY) && !a.rot ? q_off : 0;
  lo = lo < hi ? lo : hi;
  const int t8 = threadIdx.x & 7;  // 16-code piece of the row: dims 16 t8 .. +15
  const int row = blockIdx.x * 32 + (threadIdx.x >> 3);
  if (row < lo || row >= hi) return;
  const int64_t src = (int64_t)b * a.sb + (int64_t)kh * a.sh + (int64_t)row * a.sp + 16 * t8;
  const int64_t erow = (int64_t)bh * a.cap + row;
  const int64_t dst = ((int64_t)bh * a.R + row) * kD + 16 * t8;
  for (int kv = 0; kv < 2; ++kv) {
    const u32x4 codes = *(const u32x4*)((kv ? a.v : a.k) + src);
    const uint32_t ex = (kv ? a.vexp : a.kexp)[erow];
    const int e = (int)(int8_t)(ex >> (t8 >= 4 ? 8 : 0));  // dims < 64: block 0
    const float sc = __uint_as_float((uint32_t)(e + 127) << 23);
    u32x4 lo4, hi4;
    for (int i = 0; i < 2; ++i) {
      lo4[2 * i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)codes[i], sc, false));
      lo4[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)codes[i], sc, true));
      hi4[2 * i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)codes[2 + i], sc, false));
      hi4[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)codes[2 + i], sc, true));
    }
    uint16_t* const out = (kv ? a.wv : a.wk) + dst;
    *(u32x4*)out = lo4;
    *(u32x4*)(out + 8) = hi4;
  }
}

}  // namespace

int32_t launch_fp8_to_bf16(hipStream_t s, const ema_kvcache_desc& c, const int32_t* q_off, int T,
                           uint32_t flags, int R, void* ws) {
  DequantArgs a;
  a.k = (const uint8_t*)c.k;
  a.v = (const uint8_t*)c.v;
  a.kexp = (const uint16_t*)c.k_exp;
  a.vexp = (const uint16_t*)c.v_exp;
  a.q_off = q_off;
  a.wk = (uint16_t*)ws;
  a.wv = a.wk + (int64_t)c.batch * c.n_kv_heads * R * kD;
  a.sb = c.stride_batch;
  a.sh = c.stride_head;
  a.sp = c.stride_pos;
  a.Hkv = c.n_kv_heads;
  a.cap = c.capacity;
  a.R = R;
  a.T = T;
  a.flags = flags;
  a.rot = (c.flags & EMA_KV_ROTATING) != 0;
  const dim3 grid((unsigned)((R + 31) / 32), (unsigned)(c.batch * c.n_kv_heads));
  hipLaunchKernelGGL(fp8_to_bf16_kernel, grid, dim3(256), 0, s, a);
  return check_hip(hipGetLastError(), "ema_prefill_attention_ws: fp8 decode launch");
}

}  // namespace ema
