// FP8 E4M3FN cache rows: -> bf16 for prefill over an FP8 cache (ema_prefill_attention_ws),
// and the row conversions of ema_kvcache_convert (bf16 <-> FP8).
//
// The reference's FP8 cache hands SDPA its round-tripped values
// (crates/kvcache/src/fp8.rs:60-68, values of crates/ops/src/fp8.rs:71-92). Here the rows
// a prefill call attends to are decoded into a bf16 copy in the caller's workspace and the
// bf16 prefill kernel runs over that copy: code * 2^exp is exact in bf16, so the result is
// that of a bf16 cache holding the decoded values. HBM-bound: 130 bytes read and 256 bytes
// written per row of K or V, small next to the prefill's matrix work.
//
// Mapping: 8 threads per 128-dim row, 16 codes (one 16-byte load) each, 32 rows per
// 256-thread workgroup pass; blockIdx.y = (batch, kv head). With an unquantised RoPE
// tail (n_rot = 64) the threads of dims 64..127 copy their 16 bf16 values. Rows [lo, hi) of a sequence
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
  int nrot;  // dims 64..127 stored as bf16 after the 64 codes of a row
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
  // EMA_PREFILL_ROWS_DECODED: the chunk's rows (positions q_off .. q_off + T - 1: rows
  // (q_off + t) % cap of a ring, rows q_off + t of a static cache) are in the copy already
  if (a.flags & EMA_PREFILL_ROWS_DECODED) {
    const bool chunk = a.rot ? ((row - q_off) % a.cap + a.cap) % a.cap < a.T : row >= q_off && row - q_off < a.T;
    if (chunk) return;
  }
  const int64_t src = (int64_t)b * a.sb + (int64_t)kh * a.sh + (int64_t)row * a.sp + 16 * t8;
  const int64_t erow = (int64_t)bh * a.cap + row;
  const int64_t dst = ((int64_t)bh * a.R + row) * kD + 16 * t8;
  for (int kv = 0; kv < 2; ++kv) {
    if (a.nrot && t8 >= 4) {  // dims 16 t8 .. +15: bf16 at bytes 64 + 2 (16 t8 - 64)
      const uint8_t* tail = (kv ? a.v : a.k) + (src - 16 * t8) + 32 * t8 - 64;
      uint16_t* const out = (kv ? a.wv : a.wk) + dst;
      *(u32x4*)out = *(const u32x4*)tail;
      *(u32x4*)(out + 8) = *(const u32x4*)(tail + 16);
      continue;
    }
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

// Rows [src_row, src_row + n) of every (sequence, kv head) of one cache into rows
// [dst_row, dst_row + n) of another: bf16 -> FP8 (the quantisation of Fp8Cache::append,
// crates/kvcache/src/fp8.rs:47-68, as ema_pre_attention writes it) or FP8 -> bf16 (the
// exact decoded values, what Fp8Cache::get hands SDPA: fp8.rs:60-68). 8 lanes per 128-value
// row, lane j with values 8j .. 8j+7 and 64+8j .. 64+8j+7 (one 64-value block each), 32
// rows per 256-thread workgroup. HBM-bound. With an unquantised RoPE tail (the FP8
// side's n_rot = 64) the second block is copied as bf16 and its exponent written as 0.
struct ConvArgs {
  const uint8_t* sk;  // source K / V (bytes; element strides below)
  const uint8_t* sv;
  const uint16_t* skexp;  // FP8 source: exponent pairs [B, Hkv, cap]
  const uint16_t* svexp;
  uint8_t* dk;
  uint8_t* dv;
  uint16_t* dkexp;  // FP8 destination: exponent pairs
  uint16_t* dvexp;
  int64_t ssb, ssh, ssp;  // source strides (elements)
  int64_t dsb, dsh, dsp;  // destination strides (elements)
  int Hkv, scap, dcap, src_row, dst_row, n;
  int64_t total;  // B * Hkv * n rows
  int nrot;       // the FP8 side keeps dims 64..127 as bf16
};

template <bool kToFp8>
__global__ __launch_bounds__(256) void fp8_convert_kernel(ConvArgs a) {
  const int64_t row = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  if (row >= a.total) return;  // whole 8-lane groups leave together
  const int lane8 = threadIdx.x & 7;
  const int r = (int)(row % a.n);
  const int64_t bh = row / a.n;  // b * Hkv + kh
  const int b = (int)(bh / a.Hkv), kh = (int)(bh % a.Hkv);
  const int64_t srow = (int64_t)b * a.ssb + (int64_t)kh * a.ssh + (int64_t)(a.src_row + r) * a.ssp;
  const int64_t drow = (int64_t)b * a.dsb + (int64_t)kh * a.dsh + (int64_t)(a.dst_row + r) * a.dsp;
  for (int kv = 0; kv < 2; ++kv) {
    if (kToFp8) {
      const uint16_t* src = (const uint16_t*)(kv ? a.sv : a.sk) + srow;
      uint16_t x[16];
      const u32x4 lo = *(const u32x4*)(src + 8 * lane8), hi = *(const u32x4*)(src + 64 + 8 * lane8);
      for (int e = 0; e < 4; ++e) {
        x[2 * e] = (uint16_t)lo[e];
        x[2 * e + 1] = (uint16_t)(lo[e] >> 16);
        x[8 + 2 * e] = (uint16_t)hi[e];
        x[8 + 2 * e + 1] = (uint16_t)(hi[e] >> 16);
      }
      float m0 = 0.f, m1 = 0.f;
      for (int e = 0; e < 8; ++e) {
        m0 = fmaxf(m0, fabsf(bf16_to_f32(x[e])));
        m1 = fmaxf(m1, fabsf(bf16_to_f32(x[8 + e])));
      }
      const int e0 = fp8_block_exp(m0);
      const int e1 = a.nrot ? 0 : fp8_block_exp(m1);  // (uniform over the 8 lanes)
      uint8_t* codes = (kv ? a.dv : a.dk) + drow;
      *(u32x2*)(codes + 8 * lane8) = fp8_encode8(x, e0);
      if (a.nrot) *(u32x4*)(codes + 64 + 16 * lane8) = hi;
      else *(u32x2*)(codes + 64 + 8 * lane8) = fp8_encode8(x + 8, e1);
      if (lane8 == 0)
        (kv ? a.dvexp : a.dkexp)[bh * a.dcap + a.dst_row + r] = (uint16_t)((uint8_t)e0 | ((uint32_t)(uint8_t)e1 << 8));
    } else {
      const uint8_t* codes = (kv ? a.sv : a.sk) + srow;
      const uint32_t ex = (kv ? a.svexp : a.skexp)[bh * a.scap + a.src_row + r];
      uint16_t* dst = (uint16_t*)(kv ? a.dv : a.dk) + drow;
      if (a.nrot) *(u32x4*)(dst + 64 + 8 * lane8) = *(const u32x4*)(codes + 64 + 16 * lane8);
      for (int h = 0; h < (a.nrot ? 1 : 2); ++h) {
        const u32x2 w = *(const u32x2*)(codes + 64 * h + 8 * lane8);
        const float sc = __uint_as_float((uint32_t)((int)(int8_t)(ex >> (8 * h)) + 127) << 23);
        u32x4 o4;
        o4[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w[0], sc, false));
        o4[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w[0], sc, true));
        o4[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w[1], sc, false));
        o4[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)w[1], sc, true));
        *(u32x4*)(dst + 64 * h + 8 * lane8) = o4;
      }
    }
  }
}

}  // namespace

int32_t launch_fp8_convert(hipStream_t s, const ema_kvcache_desc& src, int src_row, const ema_kvcache_desc& dst,
                           int dst_row, int n_rows) {
  ConvArgs a;
  a.sk = (const uint8_t*)src.k;
  a.sv = (const uint8_t*)src.v;
  a.skexp = (const uint16_t*)src.k_exp;
  a.svexp = (const uint16_t*)src.v_exp;
  a.dk = (uint8_t*)dst.k;
  a.dv = (uint8_t*)dst.v;
  a.dkexp = (uint16_t*)dst.k_exp;
  a.dvexp = (uint16_t*)dst.v_exp;
  a.ssb = src.stride_batch;
  a.ssh = src.stride_head;
  a.ssp = src.stride_pos;
  a.dsb = dst.stride_batch;
  a.dsh = dst.stride_head;
  a.dsp = dst.stride_pos;
  a.Hkv = dst.n_kv_heads;
  a.scap = src.capacity;
  a.dcap = dst.capacity;
  a.src_row = src_row;
  a.dst_row = dst_row;
  a.n = n_rows;
  a.total = (int64_t)dst.batch * dst.n_kv_heads * n_rows;
  a.nrot = (dst.dtype == EMA_DTYPE_FP8_E4M3 ? dst.n_rot : src.n_rot) != 0;
  const int64_t blocks = (a.total + 31) / 32;
  if (blocks > 0x7fffffff) return set_error(EMA_ERR_SHAPE, "ema_kvcache_convert: too many rows");
  const bool to_fp8 = dst.dtype == EMA_DTYPE_FP8_E4M3;
  if (to_fp8) hipLaunchKernelGGL(fp8_convert_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  else hipLaunchKernelGGL(fp8_convert_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, a);
  return check_hip(hipGetLastError(), "ema_kvcache_convert launch");
}

int32_t launch_fp8_to_bf16(hipStream_t s, const ema_kvcache_desc& c, const int32_t* q_off, int T,
                           uint32_t flags, int R, void* ws) {
  // the chunk's rows are decoded already and no other row is attended: nothing to do
  if ((flags & EMA_PREFILL_ROWS_DECODED) && (flags & EMA_PREFILL_CHUNK_ONLY) && !(c.flags & EMA_KV_ROTATING))
    return EMA_OK;
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
  a.nrot = c.n_rot != 0;
  const dim3 grid((unsigned)((R + 31) / 32), (unsigned)(c.batch * c.n_kv_heads));
  hipLaunchKernelGGL(fp8_to_bf16_kernel, grid, dim3(256), 0, s, a);
  return check_hip(hipGetLastError(), "ema_prefill_attention_ws: fp8 decode launch");
}

}  // namespace ema
