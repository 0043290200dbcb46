// bf16 cache rows -> 4-bit affine cache rows (ema_kvcache_quantize_int4).
//
// The reference fills its int4 KV buffers one position at a time: quantize_kv_native of the
// [1, nkv, 1, hd] slice, then slice_update of data, scales and biases
// (convert_kv_to_int4, crates/serve/src/engine_ext.rs:158-210, and the int4 store of the
// prefill, crates/serve/src/forward_qwen3.rs:69-120). Here one launch quantises every row of
// the range for all sequences and kv heads, K and V: 8 lanes per 128-value row (16 values,
// two 16-byte loads each), 32 rows per 256-thread workgroup. HBM-bound: 512 bytes read and
// 144 written per row pair (K and V).
#include "ema_common.hpp"

namespace ema {
namespace {

struct QuantArgs {
  const uint16_t* sk;  // bf16 source cache
  const uint16_t* sv;
  int64_t ssb, ssh, ssp;  // source strides (elements)
  uint16_t* dk;           // int4 destination words
  uint16_t* dv;
  uint32_t* ks;  // destination (group 0, group 1) scale / bias pairs [B, Hkv, cap]
  uint32_t* kb;
  uint32_t* vs;
  uint32_t* vb;
  int64_t dsb, dsh, dsp;  // destination strides (4-bit elements)
  int Hkv, cap, src_row, dst_row, n;
  int64_t total;  // B * Hkv * n rows
};

__global__ __launch_bounds__(256) void quantize_int4_kernel(QuantArgs a) {
  const int64_t row = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  if (row >= a.total) return;  // whole 8-lane groups leave together
  const int lane8 = threadIdx.x & 7;
  const int r = (int)(row % a.n);
  const int64_t bh = row / a.n;  // b * Hkv + kh
  const int b = (int)(bh / a.Hkv), kh = (int)(bh % a.Hkv);
  for (int kv = 0; kv < 2; ++kv) {
    const uint16_t* src = (kv ? a.sv : a.sk) + (int64_t)b * a.ssb + (int64_t)kh * a.ssh + (int64_t)(a.src_row + r) * a.ssp;
    const u32x4 lo = *(const u32x4*)(src + 8 * lane8);
    const u32x4 hi = *(const u32x4*)(src + 64 + 8 * lane8);
    float f[16];
    for (int e = 0; e < 4; ++e) {
      f[2 * e] = bf16_lo(lo[e]);
      f[2 * e + 1] = bf16_hi(lo[e]);
      f[8 + 2 * e] = bf16_lo(hi[e]);
      f[8 + 2 * e + 1] = bf16_hi(hi[e]);
    }
    uint32_t* words = (uint32_t*)((uint8_t*)(kv ? a.dv : a.dk) +
                                  ((int64_t)b * a.dsb + (int64_t)kh * a.dsh + (int64_t)(a.dst_row + r) * a.dsp) / 2);
    const int64_t m = bh * a.cap + a.dst_row + r;
    i4_store_row8(f, words, (kv ? a.vs : a.ks) + m, (kv ? a.vb : a.kb) + m, lane8);
  }
}

}  // namespace

int32_t launch_quantize_int4(hipStream_t s, const ema_kvcache_desc& src, int src_row, const ema_kvcache_desc& dst,
                             int dst_row, int n_rows) {
  QuantArgs a;
  a.sk = (const uint16_t*)src.k;
  a.sv = (const uint16_t*)src.v;
  a.ssb = src.stride_batch;
  a.ssh = src.stride_head;
  a.ssp = src.stride_pos;
  a.dk = (uint16_t*)dst.k;
  a.dv = (uint16_t*)dst.v;
  a.ks = (uint32_t*)dst.k_scales;
  a.kb = (uint32_t*)dst.k_biases;
  a.vs = (uint32_t*)dst.v_scales;
  a.vb = (uint32_t*)dst.v_biases;
  a.dsb = dst.stride_batch;
  a.dsh = dst.stride_head;
  a.dsp = dst.stride_pos;
  a.Hkv = dst.n_kv_heads;
  a.cap = dst.capacity;
  a.src_row = src_row;
  a.dst_row = dst_row;
  a.n = n_rows;
  a.total = (int64_t)dst.batch * dst.n_kv_heads * n_rows;
  const int64_t blocks = (a.total + 31) / 32;
  if (blocks > 0x7fffffff) return set_error(EMA_ERR_SHAPE, "ema_kvcache_quantize_int4: too many rows");
  hipLaunchKernelGGL(quantize_int4_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a);
  return check_hip(hipGetLastError(), "ema_kvcache_quantize_int4 launch");
}

}  // namespace ema
