// Fused Qwen3 pre-attention for gfx950: q/k RMSNorm, split-half RoPE and the
// in-place K/V write at the sequence offset, one pass over the fused qkv
// activation.
//
// Replaces the op chain of crates/serve/src/forward_qwen3.rs:56-68 + :124-142
// (prefill: slice, reshape, rms_norm, transpose, rope_dynamic, slice_update)
// and crates/serve/src/compiled.rs:134-161 (decode: dsplit, rms_norm, rope,
// scatter_single). Arithmetic follows MLX fast::rms_norm / fast::rope
// (crates/mlx-ffi/src/ops/real/blas.rs:5-9, :67-80): f32 statistics, the
// normalised value rounded to bf16 before the weight multiply, RoPE angle
// pos * 2^(-(i/(D/2)) * log2(theta)) formed in f32.
//
// Mapping: one workgroup per token (b, t). Its first D/2 threads form the
// token's RoPE table (cos, sin of each frequency) in LDS once; then each group
// of 8 lanes takes head vectors h of the fused row (h over the Hq + 2*Hkv
// heads, stride 32). Lane j holds elements [j*E, j*E+E) and
// [D/2 + j*E, D/2 + j*E + E) with E = D/16 (16-byte accesses at D = 128), so
// each RoPE pair sits in one lane and each half of the row is one contiguous
// D-byte access per group.
// HBM-bound: every byte of qkv is read once, q/k/v written once.
//
// FP8 E4M3FN cache (D = 128): the two halves of a row that the 8 lanes of a head hold
// are exactly its two 64-element blocks; each block's scale exponent comes from an
// 8-lane max, and the lane writes its 2 x 8 codes (the quantisation of
// crates/ops/src/fp8.rs:71-92, applied to the bf16 row as Fp8Cache::append does). With
// an unquantised RoPE tail (n_rot = 64) the second half is written as bf16 after the 64
// codes of the first, and block 1's exponent as 0.
#include "ema_common.hpp"

namespace ema {
namespace {

template <int E>
struct Vec;
template <>
struct Vec<2> {
  typedef uint32_t T;
  static __device__ __forceinline__ void load(const uint16_t* p, uint16_t* x) {
    uint32_t w = *(const uint32_t*)p;
    x[0] = (uint16_t)w;
    x[1] = (uint16_t)(w >> 16);
  }
  static __device__ __forceinline__ void store(uint16_t* p, const uint16_t* x) {
    *(uint32_t*)p = (uint32_t)x[0] | ((uint32_t)x[1] << 16);
  }
};
template <>
struct Vec<4> {
  static __device__ __forceinline__ void load(const uint16_t* p, uint16_t* x) {
    u32x2 w = *(const u32x2*)p;
    for (int i = 0; i < 2; ++i) {
      x[2 * i] = (uint16_t)w[i];
      x[2 * i + 1] = (uint16_t)(w[i] >> 16);
    }
  }
  static __device__ __forceinline__ void store(uint16_t* p, const uint16_t* x) {
    u32x2 w;
    for (int i = 0; i < 2; ++i) w[i] = (uint32_t)x[2 * i] | ((uint32_t)x[2 * i + 1] << 16);
    *(u32x2*)p = w;
  }
};
template <>
struct Vec<8> {
  static __device__ __forceinline__ void load(const uint16_t* p, uint16_t* x) {
    u32x4 w = *(const u32x4*)p;
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = (uint16_t)w[i];
      x[2 * i + 1] = (uint16_t)(w[i] >> 16);
    }
  }
  static __device__ __forceinline__ void store(uint16_t* p, const uint16_t* x) {
    u32x4 w;
    for (int i = 0; i < 4; ++i) w[i] = (uint32_t)x[2 * i] | ((uint32_t)x[2 * i + 1] << 16);
    *(u32x4*)p = w;
  }
};

template <>
struct Vec<16> {
  static __device__ __forceinline__ void load(const uint16_t* p, uint16_t* x) {
    Vec<8>::load(p, x);
    Vec<8>::load(p + 8, x + 8);
  }
  static __device__ __forceinline__ void store(uint16_t* p, const uint16_t* x) {
    Vec<8>::store(p, x);
    Vec<8>::store(p + 8, x + 8);
  }
};

struct PreArgs {
  const uint16_t* qkv;
  const uint16_t* qw;
  const uint16_t* kw;
  const int32_t* off;
  uint16_t* q_out;
  uint16_t* kc;
  uint16_t* vc;
  int8_t* kexp;  // fp8 cache: block exponents [B, Hkv, cap, D/64]
  int8_t* vexp;
  uint32_t* ks;  // int4 cache: (group 0, group 1) bf16 scale and bias pairs [B, Hkv, cap]
  uint32_t* kb;
  uint32_t* vs;
  uint32_t* vb;
  int64_t sb, sh, sp;
  float eps;
  float log2_theta;
  int B, T, Hq, Hkv, cap;
  uint32_t flags;
  int rot;  // rotating cache: position p lives in row p % cap
  int nrot;  // fp8 cache: dims 64..127 kept as bf16 (n_rot = 64)
  // fp8 cache, optional: the prefill's bf16 copy [B, Hkv, R, D] of K (dk) and V (dv); each
  // stored row below R is also written there, decoded (code * 2^e, exact)
  uint16_t* dk;
  uint16_t* dv;
  int R;
};

template <int D, bool kFp8, bool kI4 = false>
__global__ __launch_bounds__(256) void pre_attention_kernel(PreArgs a) {
  constexpr int HALF = D / 2;
  constexpr int E = D / 16;  // elements per lane in each half of the row
  // one workgroup per token (b, t); its 32 groups of 8 lanes walk the token's head vectors
  __shared__ float rope_cs[HALF], rope_sn[HALF];
  const int64_t bt = blockIdx.x;
  const int t = (int)(bt % a.T);
  const int b = (int)(bt / a.T);
  const int off = a.off[b];
  const int pos = off + t;
  // the cache row of this token, and whether it is written: a static cache takes the
  // call's rows only when all fit; a rotating one keeps the last cap tokens of the call
  // (earlier ones would be overwritten within it)
  const int row = a.rot ? pos % a.cap : pos;
  const bool in_cap = a.rot ? off >= 0 && a.T - t <= a.cap : off >= 0 && (int64_t)off + a.T <= a.cap;
  const bool rope = !(a.flags & EMA_PRE_NO_ROPE);
  // RoPE angles of this position, shared by every q and k head of the token
  if (rope && (int)threadIdx.x < HALF) {
    const int i = threadIdx.x;
    const float inv_freq = exp2f(-((float)i / (float)HALF) * a.log2_theta);
    const float ang = (float)pos * inv_freq;
    float sn, cs;
    sincosf(ang, &sn, &cs);
    rope_cs[i] = cs;
    rope_sn[i] = sn;
  }
  __syncthreads();

  const int lane8 = threadIdx.x & 7;
  const int H = a.Hq + 2 * a.Hkv;
  // fp8 cache row (b, kh, pos) from the bf16 values x[0..2E) of this lane (E = 8)
  auto store_fp8 = [&](const uint16_t* x, uint16_t* codes16, int8_t* exps, uint16_t* copy, int b_, int kh, int p_) {
    float m0 = 0.f, m1 = 0.f;
    for (int e = 0; e < E; ++e) {
      m0 = fmaxf(m0, fabsf(bf16_to_f32(x[e])));
      m1 = fmaxf(m1, fabsf(bf16_to_f32(x[E + e])));
    }
    const int e0 = fp8_block_exp(m0);
    const int e1 = a.nrot ? 0 : fp8_block_exp(m1);  // (uniform: all 8 lanes shuffle or none)
    uint8_t* row = (uint8_t*)codes16 + (int64_t)b_ * a.sb + (int64_t)kh * a.sh + (int64_t)p_ * a.sp;
    const u32x2 c0 = fp8_encode8(x, e0);
    *(u32x2*)(row + lane8 * E) = c0;
    u32x2 c1 = {0u, 0u};
    if (a.nrot) Vec<E>::store((uint16_t*)(row + HALF) + lane8 * E, x + E);
    else *(u32x2*)(row + HALF + lane8 * E) = c1 = fp8_encode8(x + E, e1);
    if (copy && p_ < a.R) {  // the decoded row, as the prefill's decode pass would write it
      uint16_t* const d = copy + (((int64_t)b_ * a.Hkv + kh) * a.R + p_) * D;
      *(u32x4*)(d + lane8 * E) = fp8_decode8(c0, e0);
      if (a.nrot) Vec<E>::store(d + HALF + lane8 * E, x + E);
      else *(u32x4*)(d + HALF + lane8 * E) = fp8_decode8(c1, e1);
    }
    if (lane8 == 0) {
      const int64_t r = ((int64_t)b_ * a.Hkv + kh) * a.cap + p_;
      *(uint16_t*)(exps + 2 * r) = (uint16_t)((uint8_t)e0 | ((uint32_t)(uint8_t)e1 << 8));
    }
  };
  // int4 cache row (b, kh, pos) from the bf16 values x[0..2E) of this lane (E = 8); the
  // strides count 4-bit elements
  auto store_i4 = [&](const uint16_t* x, uint16_t* words16, uint32_t* sc, uint32_t* bi, int b_, int kh, int p_) {
    float f[16];
    for (int e = 0; e < 16; ++e) f[e] = bf16_to_f32(x[e]);
    uint32_t* words =
        (uint32_t*)((uint8_t*)words16 + ((int64_t)b_ * a.sb + (int64_t)kh * a.sh + (int64_t)p_ * a.sp) / 2);
    const int64_t r = ((int64_t)b_ * a.Hkv + kh) * a.cap + p_;
    i4_store_row8(f, words, sc + r, bi + r, lane8);
  };
  for (int h = threadIdx.x >> 3; h < H; h += 32) {
    const uint16_t* src = a.qkv + (bt * H + h) * D;
    uint16_t x[2 * E];
    Vec<E>::load(src + lane8 * E, x);
    Vec<E>::load(src + HALF + lane8 * E, x + E);

    if (h >= a.Hq + a.Hkv) {  // v: bit copy into the cache row
      if (!in_cap) continue;
      const int kh = h - a.Hq - a.Hkv;
      if (kFp8) {
        store_fp8(x, a.vc, a.vexp, a.dv, b, kh, row);
        continue;
      }
      if (kI4) {
        store_i4(x, a.vc, a.vs, a.vb, b, kh, row);
        continue;
      }
      uint16_t* dst = a.vc + (int64_t)b * a.sb + (int64_t)kh * a.sh + (int64_t)row * a.sp;
      Vec<E>::store(dst + lane8 * E, x);
      Vec<E>::store(dst + HALF + lane8 * E, x + E);
      continue;
    }
    const bool is_q = h < a.Hq;
    if (!is_q && !in_cap) continue;
    float y[2 * E];
    if (!(a.flags & (EMA_PRE_NO_NORM | (is_q ? EMA_PRE_NO_Q_NORM : EMA_PRE_NO_K_NORM)))) {
      float ss = 0.f;
      for (int e = 0; e < 2 * E; ++e) {
        const float f = bf16_to_f32(x[e]);
        ss += f * f;
      }
      ss += __shfl_xor(ss, 4, 8);
      ss += __shfl_xor(ss, 2, 8);
      ss += __shfl_xor(ss, 1, 8);
      const float inv = 1.0f / sqrtf(ss / (float)D + a.eps);
      const uint16_t* w = is_q ? a.qw : a.kw;
      uint16_t wv[2 * E];
      Vec<E>::load(w + lane8 * E, wv);
      Vec<E>::load(w + HALF + lane8 * E, wv + E);
      for (int e = 0; e < 2 * E; ++e) {
        const float n = bf16_to_f32((uint16_t)f32_to_bf16_bits(bf16_to_f32(x[e]) * inv));
        y[e] = bf16_to_f32((uint16_t)f32_to_bf16_bits(n * bf16_to_f32(wv[e])));
      }
    } else {
      for (int e = 0; e < 2 * E; ++e) y[e] = bf16_to_f32(x[e]);
    }
    uint16_t o[2 * E];
    if (rope) {
      for (int e = 0; e < E; ++e) {
        const int i = lane8 * E + e;
        const float cs = rope_cs[i], sn = rope_sn[i];
        const float x1 = y[e], x2 = y[E + e];
        o[e] = (uint16_t)f32_to_bf16_bits(x1 * cs - x2 * sn);
        o[E + e] = (uint16_t)f32_to_bf16_bits(x1 * sn + x2 * cs);
      }
    } else {
      for (int e = 0; e < 2 * E; ++e) o[e] = (uint16_t)f32_to_bf16_bits(y[e]);
    }
    if (kFp8 && !is_q) {
      store_fp8(o, a.kc, a.kexp, a.dk, b, h - a.Hq, row);
      continue;
    }
    if (kI4 && !is_q) {
      store_i4(o, a.kc, a.ks, a.kb, b, h - a.Hq, row);
      continue;
    }
    uint16_t* dst;
    if (is_q) dst = a.q_out + (((int64_t)b * a.Hq + h) * a.T + t) * D;
    else dst = a.kc + (int64_t)b * a.sb + (int64_t)(h - a.Hq) * a.sh + (int64_t)row * a.sp;
    Vec<E>::store(dst + lane8 * E, o);
    Vec<E>::store(dst + HALF + lane8 * E, o + E);
  }
}

}  // namespace

int32_t launch_pre_attention(hipStream_t s, const void* qkv, const void* qw, const void* kw,
                             float eps, float theta, const int32_t* off, int B, int T, int Hq,
                             int Hkv, int D, uint32_t flags, void* q_out,
                             const ema_kvcache_desc& c, void* copy, int copy_rows) {
  PreArgs a;
  a.qkv = (const uint16_t*)qkv;
  a.qw = (const uint16_t*)qw;
  a.kw = (const uint16_t*)kw;
  a.off = off;
  a.q_out = (uint16_t*)q_out;
  a.kc = (uint16_t*)c.k;
  a.vc = (uint16_t*)c.v;
  a.kexp = (int8_t*)c.k_exp;
  a.vexp = (int8_t*)c.v_exp;
  a.ks = (uint32_t*)c.k_scales;
  a.kb = (uint32_t*)c.k_biases;
  a.vs = (uint32_t*)c.v_scales;
  a.vb = (uint32_t*)c.v_biases;
  a.sb = c.stride_batch;
  a.sh = c.stride_head;
  a.sp = c.stride_pos;
  a.eps = eps;
  a.log2_theta = log2f(theta);
  a.B = B;
  a.T = T;
  a.Hq = Hq;
  a.Hkv = Hkv;
  a.cap = c.capacity;
  a.flags = flags;
  a.rot = (c.flags & EMA_KV_ROTATING) != 0;
  a.nrot = c.dtype == EMA_DTYPE_FP8_E4M3 && c.n_rot != 0;
  a.dk = copy ? (uint16_t*)copy : nullptr;
  a.dv = copy ? (uint16_t*)copy + (int64_t)B * Hkv * copy_rows * D : nullptr;
  a.R = copy ? copy_rows : 0;
  const int threads = 256;
  const int64_t blocks = (int64_t)B * T;  // one workgroup per token
  if (blocks > 0x7fffffff) return set_error(EMA_ERR_SHAPE, "ema_pre_attention: too many tokens");
  if (c.dtype == EMA_DTYPE_FP8_E4M3) {  // head_dim 128 (checked with the descriptor)
    hipLaunchKernelGGL((pre_attention_kernel<128, true>), dim3((unsigned)blocks), dim3(threads), 0, s, a);
    return check_hip(hipGetLastError(), "ema_pre_attention launch");
  }
  if (c.dtype == EMA_DTYPE_INT4_AFFINE) {  // head_dim 128 (checked with the descriptor)
    hipLaunchKernelGGL((pre_attention_kernel<128, false, true>), dim3((unsigned)blocks), dim3(threads), 0, s, a);
    return check_hip(hipGetLastError(), "ema_pre_attention launch");
  }
  switch (D) {
    case 64:
      hipLaunchKernelGGL((pre_attention_kernel<64, false>), dim3((unsigned)blocks), dim3(threads), 0, s, a);
      break;
    case 128:
      hipLaunchKernelGGL((pre_attention_kernel<128, false>), dim3((unsigned)blocks), dim3(threads), 0, s, a);
      break;
    case 256:
      hipLaunchKernelGGL((pre_attention_kernel<256, false>), dim3((unsigned)blocks), dim3(threads), 0, s, a);
      break;
    default:
      return set_error(EMA_ERR_UNSUPPORTED, "ema_pre_attention: head_dim %d not supported (64/128/256)", D);
  }
  return check_hip(hipGetLastError(), "ema_pre_attention launch");
}

}  // namespace ema
