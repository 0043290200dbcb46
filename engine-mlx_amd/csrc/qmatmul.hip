// Affine-quantised matmul over MLX-packed weights on bf16/f16 MFMA (gfx950): MLX
// quantized_matmul(x, w, scales, biases, transpose = true, group_size, bits, "affine")
// (crates/mlx-ffi/src/ops/real/transform.rs:77-88), which the reference's qmatmul
// (crates/ops/src/quant.rs:57-76) and the fused / separate q|k|v and o projections
// (crates/serve/src/forward/projection.rs:105-152, crates/ops/src/attention.rs:31-51,162-177)
// call:
//
//   y[m, n] = sum_k x[m, k] * (s[n, g] * q[n, k] + b[n, g]),   g = k / GS
//
// with q[n, k] the BITS-wide field (k % (32 / BITS)) * BITS of word k / (32 / BITS) of
// weight row n (lowest bits first), s and b the per-group scale and bias, all of x, s,
// b and y in one activation type (bf16 or f16).
//
// Exact products. The MFMA's B operand is not the dequantised weight (which would have to
// be rounded to bf16) but C + q, with the field's bits dropped into the mantissa of the
// constant C (bf16 2^7 or f16 2^10: one and-or per pair of weights), which is exact; an
// 8-bit field in bf16 is converted exactly instead (v_cvt_f32_ubyte, top half), C = 0.
// Per group of GS k, one MFMA chain accumulates a_q = sum x (C + q) and a second, with
// B = 1, a_1 = sum x, both in f32 from exact bf16 x bf16 products; then
//   y += s * a_q + (b - C s) * a_1,
// so no weight is rounded and y carries only f32 accumulation error before its one
// rounding to the output type. The bit pairing of a 32-bit B register (fields r and
// r + 4 of a 4-bit word, or bytes 0 and 2 of an 8-bit word) is matched by permuting
// the x pairs of the A register the same way (v_perm_b32); the order of k within an MFMA
// step is free since the step sums over it.
//
// Work split: one workgroup per 16 weight rows (16 columns of y) and 16 * MR rows of x,
// its waves splitting the K groups, partial tiles summed in LDS. 16x16x32 MFMA tiles give
// N / 16 workgroups, so a decode-sized projection (M <= 32) spreads over the whole chip
// and streams every weight once; each lane keeps up to 8 groups of loads in flight,
// issued in the order they are consumed (vmcnt counts in order), and a wave's groups
// past its range read zeros out of bounds instead of branching. For larger M the row
// tiles of one weight tile are dispatched together on one XCD, so its L2 serves the
// re-reads.
#include "ema_common.hpp"

namespace ema {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kMaxWaves = 8;
constexpr uint32_t kOffRow = 0xF0000000u;  // a buffer offset past every range: loads return 0

struct QmmArgs {
  const uint8_t* x;  // [M, ldx] activations
  const uint8_t* w;  // [N, K * BITS / 8] packed fields
  const uint8_t* s;  // [N, G] scales
  const uint8_t* b;  // [N, G] biases
  uint8_t* y;        // [M, ldy]
  int64_t ldx, ldy;  // row strides in elements
  int M, N, K, G;    // G = K / GS
  int mtiles;        // row tiles of x (16 * MR rows each)
  int remap;         // grid size divisible by 8: give each XCD a contiguous range of tiles
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

template <bool F16>
__device__ __forceinline__ f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                  0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

template <bool F16>
__device__ __forceinline__ float act_to_f32(uint32_t bits16) {
  if constexpr (F16)
    return (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
  else
    return __uint_as_float(bits16 << 16);
}
template <bool F16>
__device__ __forceinline__ uint16_t f32_to_act(float v) {
  if constexpr (F16)
    return __builtin_bit_cast(uint16_t, (_Float16)v);
  else
    return (uint16_t)f32_to_bf16_bits(v);
}

// v_perm_b32 selectors: {lo16(lo), lo16(hi)} and {hi16(lo), hi16(hi)} of two dwords.
constexpr uint32_t kSelLo = 0x05040100u, kSelHi = 0x07060302u;
__device__ __forceinline__ uint32_t pair(uint32_t lo, uint32_t hi, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}

template <int BITS, bool F16>
struct Fields {
  // the weight bits take the mantissa of this constant: value kOff + q, exact
  static constexpr bool kMagic = F16 || BITS == 4;
  static constexpr uint32_t kMagicBits = F16 ? 0x64006400u : 0x43004300u;  // 1024 (f16), 128 (bf16)
  static constexpr float kOff = !kMagic ? 0.0f : (F16 ? 1024.0f : 128.0f);
  static constexpr uint32_t kOnes = F16 ? 0x3C003C00u : 0x3F803F80u;

  // B operand of MFMA step `st`: 8 fields of this lane's weight dwords.
  static __device__ __forceinline__ u32x4 weights(const uint32_t* wd, int st) {
    u32x4 r;
    if constexpr (BITS == 4) {
      const uint32_t w = wd[st];  // fields 0..7; register i holds fields i and i + 4
      r[0] = (w & 0x000F000Fu) | kMagicBits;
      r[1] = ((w >> 4) & 0x000F000Fu) | kMagicBits;
      r[2] = ((w >> 8) & 0x000F000Fu) | kMagicBits;
      r[3] = ((w >> 12) & 0x000F000Fu) | kMagicBits;
    } else if constexpr (F16) {
      const uint32_t w0 = wd[2 * st], w1 = wd[2 * st + 1];  // bytes 0..3, 4..7
      r[0] = (w0 & 0x00FF00FFu) | kMagicBits;               // bytes 0, 2
      r[1] = ((w0 >> 8) & 0x00FF00FFu) | kMagicBits;        // bytes 1, 3
      r[2] = (w1 & 0x00FF00FFu) | kMagicBits;
      r[3] = ((w1 >> 8) & 0x00FF00FFu) | kMagicBits;
    } else {
      const uint32_t w0 = wd[2 * st], w1 = wd[2 * st + 1];
      // an integer below 256 is exact in the top half of its f32
      const uint32_t f0 = __float_as_uint((float)(w0 & 0xFFu)), f1 = __float_as_uint((float)((w0 >> 8) & 0xFFu));
      const uint32_t f2 = __float_as_uint((float)((w0 >> 16) & 0xFFu)), f3 = __float_as_uint((float)(w0 >> 24));
      const uint32_t f4 = __float_as_uint((float)(w1 & 0xFFu)), f5 = __float_as_uint((float)((w1 >> 8) & 0xFFu));
      const uint32_t f6 = __float_as_uint((float)((w1 >> 16) & 0xFFu)), f7 = __float_as_uint((float)(w1 >> 24));
      r[0] = pair(f0, f1, kSelHi);
      r[1] = pair(f2, f3, kSelHi);
      r[2] = pair(f4, f5, kSelHi);
      r[3] = pair(f6, f7, kSelHi);
    }
    return r;
  }
  // A operand of the same step: 8 consecutive activations (4 dwords) paired as the
  // fields above are.
  static __device__ __forceinline__ u32x4 acts(const uint32_t* d) {
    u32x4 r;
    if constexpr (BITS == 4) {  // {x_i, x_i+4}
      r[0] = pair(d[0], d[2], kSelLo);
      r[1] = pair(d[0], d[2], kSelHi);
      r[2] = pair(d[1], d[3], kSelLo);
      r[3] = pair(d[1], d[3], kSelHi);
    } else if constexpr (F16) {  // {x_0, x_2}, {x_1, x_3}, {x_4, x_6}, {x_5, x_7}
      r[0] = pair(d[0], d[1], kSelLo);
      r[1] = pair(d[0], d[1], kSelHi);
      r[2] = pair(d[2], d[3], kSelLo);
      r[3] = pair(d[2], d[3], kSelHi);
    } else {
      r = u32x4{d[0], d[1], d[2], d[3]};
    }
    return r;
  }
};

// Loads N dwords (1, 2 or a multiple of 4) at byte offset `off` of buffer `r`.
template <int N>
__device__ __forceinline__ void load_dw(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t* out) {
  if constexpr (N == 1) {
    out[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
  } else if constexpr (N == 2) {
    const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
    out[0] = v[0];
    out[1] = v[1];
  } else {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16 * i, 0, 0);
      out[4 * i] = v[0];
      out[4 * i + 1] = v[1];
      out[4 * i + 2] = v[2];
      out[4 * i + 3] = v[3];
    }
  }
}

template <int BITS, int GS, bool F16, int MR>
__global__ __launch_bounds__(64 * kMaxWaves) void qmm_kernel(QmmArgs a) {
  using F = Fields<BITS, F16>;
  constexpr int kSteps = GS / 32;          // 16x16x32 MFMA steps per group
  constexpr int kWDw = GS * BITS / 128;    // weight dwords per lane per group: a quarter group of a row
  constexpr int kXDw = GS / 8;             // activation dwords per lane, group and row tile: GS / 4 values
  constexpr uint32_t kWBytes = GS * BITS / 8;  // bytes of one group of one weight row
  constexpr int kRegs = kWDw + MR * kXDw + 2;
  constexpr int D = kRegs <= 12 ? 8 : kRegs <= 24 ? 4 : 2;  // groups in flight per lane
  __shared__ float red[kMaxWaves][MR][16 * 16];

  int tile = blockIdx.x;
  if (a.remap) tile = (tile % 8) * (gridDim.x / 8) + tile / 8;
  const int n0 = (tile / a.mtiles) * 16, m0 = (tile % a.mtiles) * (16 * MR);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int c = lane & 15, j = lane >> 4;  // column (and x row) c of the tile; quarter j of each group
  const int rows_n = min(16, a.N - n0), rows_m = min(16 * MR, a.M - m0);

  const uint32_t wrow = (uint32_t)a.K * BITS / 8;
  const uint32_t xrow = (uint32_t)a.ldx * 2;
  const auto W = rsrc(a.w + (int64_t)n0 * wrow, rows_n * wrow);
  const auto X = rsrc(a.x + (int64_t)m0 * xrow, (rows_m - 1) * xrow + (uint32_t)a.K * 2);
  const auto S = rsrc(a.s + (int64_t)n0 * a.G * 2, (uint32_t)rows_n * a.G * 2);
  const auto Bi = rsrc(a.b + (int64_t)n0 * a.G * 2, (uint32_t)rows_n * a.G * 2);
  const bool wv = c < rows_n;
  const uint32_t woff = c * wrow + j * (kWBytes / 4);
  const uint32_t soff = (uint32_t)c * a.G * 2;
  uint32_t xoff[MR];
#pragma unroll
  for (int t = 0; t < MR; ++t) xoff[t] = 16 * t + c < rows_m ? (16 * t + c) * xrow + j * (GS / 2) : kOffRow;

  // this wave's groups [g0, g1); every wave runs the same number of ring turns
  const int g0 = (wave * a.G) / nw, g1 = ((wave + 1) * a.G) / nw;
  const int span = (a.G + nw - 1) / nw;
  const int turns = (span + D - 1) / D;

  uint32_t wd[D][kWDw], xd[D][MR][kXDw];
  uint32_t sd[D], bd[D];
  auto issue = [&](int i, int g) {  // group g into ring slot i; past g1 every load reads zeros
    const bool in = g < g1;
    load_dw<kWDw>(W, in && wv ? woff + g * kWBytes : kOffRow, wd[i]);
#pragma unroll
    for (int t = 0; t < MR; ++t) load_dw<kXDw>(X, in ? xoff[t] + g * (GS * 2) : kOffRow, xd[i][t]);
    sd[i] = __builtin_amdgcn_raw_buffer_load_b16(S, in && wv ? soff + 2 * g : kOffRow, 0, 0);
    bd[i] = __builtin_amdgcn_raw_buffer_load_b16(Bi, in && wv ? soff + 2 * g : kOffRow, 0, 0);
  };

  f32x4 tot[MR];
#pragma unroll
  for (int t = 0; t < MR; ++t) tot[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  const u32x4 ones = {F::kOnes, F::kOnes, F::kOnes, F::kOnes};
#pragma unroll
  for (int i = 0; i < D; ++i) {
    issue(i, g0 + i);
    __builtin_amdgcn_sched_barrier(0);  // slot order = issue order, as the loop expects
  }
  for (int turn = 0; turn < turns; ++turn) {
#pragma unroll
    for (int i = 0; i < D; ++i) {
      // consume ring slot i, then refill it with group g + D (the slot's registers are
      // dead once the MFMAs have read them, so the refill needs no copies)
      const int g = g0 + turn * D + i;
      const float sc = act_to_f32<F16>(sd[i]);
      const float bc = act_to_f32<F16>(bd[i]) - F::kOff * sc;
      f32x4 aq[MR], a1[MR];
#pragma unroll
      for (int t = 0; t < MR; ++t) aq[t] = a1[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < kSteps; ++st) {
        const u32x4 B = F::weights(wd[i], st);
#pragma unroll
        for (int t = 0; t < MR; ++t) {
          const u32x4 A = F::acts(xd[i][t] + 4 * st);
          aq[t] = mma<F16>(A, B, aq[t]);
          a1[t] = mma<F16>(A, ones, a1[t]);
        }
      }
#pragma unroll
      for (int t = 0; t < MR; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) tot[t][q] = fmaf(sc, aq[t][q], fmaf(bc, a1[t][q], tot[t][q]));
      issue(i, g + D);
      // keep the groups in order: work of a later slot hoisted above this point would wait
      // for that slot's loads here
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // tot[t][q] is y[row 16 t + 4 j + q][col c] of this wave's groups
#pragma unroll
  for (int t = 0; t < MR; ++t)
#pragma unroll
    for (int q = 0; q < 4; ++q) red[wave][t][(4 * j + q) * 16 + c] = tot[t][q];
  __syncthreads();
  for (int e = threadIdx.x; e < MR * 256; e += blockDim.x) {
    const int t = e >> 8, r = (e >> 4) & 15, col = e & 15;
    float v = 0.0f;
    for (int w = 0; w < nw; ++w) v += red[w][t][(r << 4) | col];
    if (16 * t + r < rows_m && col < rows_n)
      reinterpret_cast<uint16_t*>(a.y)[(int64_t)(m0 + 16 * t + r) * a.ldy + n0 + col] = f32_to_act<F16>(v);
  }
}

// One 16-byte LDS-DMA copy per lane (buffer_load_dwordx4 ... lds): lane l's 16 bytes from
// buffer offset voff land at LDS address lds_addr + 16 l. Issued as asm so the compiler
// does not track it; the caller waits with s_waitcnt vmcnt(0) before the barrier that
// publishes the staged data.
__device__ __forceinline__ void dma16(u32x4 rsrc, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(lds_addr)
               : "memory", "m0");
}
__device__ __forceinline__ u32x4 rsrc4(const void* base, uint32_t bytes) {
  const uint64_t addr = (uint64_t)base;
  return u32x4{(uint32_t)addr, (uint32_t)(addr >> 32) & 0xffffu, bytes, 0x00020000u};
}
typedef __attribute__((address_space(3))) void lds_void;

// Staged layout of one workgroup (16 weight rows, the MX rows of x, all of K), in 16-byte
// units, chosen so both the DMA (64 consecutive units per instruction, whole 128-byte
// lines of the source) and the MFMA-layout reads (consecutive lanes on consecutive
// units) run without bank conflicts:
//   weights  row block rb = c / 8 (two, 128 bytes of padding apart), then unit u of the
//            row, then row c % 8:   unit (rb, u, c % 8) <- row c, bytes [16 u, 16 u + 16)
//   x        unit u, then row r:   unit (u, r) <- x row r, bytes [16 u, 16 u + 16)
//   scales   8 groups, then row c: unit (g / 8, c) <- scales row c, groups [g, g + 8)
//   biases   likewise
struct QmvLayout {
  uint32_t U;        // 16-byte units per weight row
  uint32_t rb_bytes; // one row block plus padding
  uint32_t x_off, s_off, b_off, bytes;
  uint32_t nW, nX, nS;  // DMA instructions per region
  __host__ __device__ QmvLayout(int K, int bits, int gs, int mx) {
    const uint32_t G = K / gs;
    U = (uint32_t)K * bits / 128;
    rb_bytes = U * 128 + 128;
    nW = U / 4;  // 16 U units, 64 per instruction
    nX = ((uint32_t)mx * K / 8 + 63) / 64;
    nS = (16 * ((G + 7) / 8) + 63) / 64;
    x_off = (2 * rb_bytes + 1023) & ~1023u;
    s_off = x_off + 1024 * nX;
    b_off = s_off + 1024 * nS;
    bytes = b_off + 1024 * nS;
  }
};

template <int BITS, int GS, bool F16, int MX>
__global__ __launch_bounds__(64 * kMaxWaves) void qmv_kernel(QmmArgs a) {
  using F = Fields<BITS, F16>;
  constexpr int kSteps = GS / 32;
  constexpr int kWDw = GS * BITS / 128;
  constexpr uint32_t kWBytes = GS * BITS / 8;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const QmvLayout L(a.K, BITS, GS, MX);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)smem;

  const int n0 = blockIdx.x * 16;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = blockDim.x >> 6;
  const int rows_n = min(16, a.N - n0), rows_m = min(MX, a.M);
  const uint32_t wrow = (uint32_t)a.K * BITS / 8;
  const uint32_t G2 = (uint32_t)a.G * 2;

  // ---- stage: every DMA instruction of the three regions, spread over the waves
  {
    const u32x4 W = rsrc4(a.w + (int64_t)n0 * wrow, rows_n * wrow);
    const u32x4 X = rsrc4(a.x, (rows_m - 1) * (uint32_t)a.ldx * 2 + (uint32_t)a.K * 2);
    const u32x4 S = rsrc4(a.s + (int64_t)n0 * G2, rows_n * G2);
    const u32x4 B = rsrc4(a.b + (int64_t)n0 * G2, rows_n * G2);
    const uint32_t total = L.nW + L.nX + 2 * L.nS;
    for (uint32_t i = wave; i < total; i += nw) {
      if (i < L.nW) {
        // the instruction's 64 units lie in one row block (8 U is a multiple of 64)
        const uint32_t rb = (64 * i) / (8 * L.U), rem = 64 * i - rb * 8 * L.U + lane;
        const uint32_t c = rb * 8 + (rem & 7), u = rem >> 3;
        const uint32_t dst = __builtin_amdgcn_readfirstlane(lds0 + rb * L.rb_bytes + 16 * (64 * i - rb * 8 * L.U));
        dma16(W, c < (uint32_t)rows_n ? c * wrow + 16 * u : kOffRow, dst);
      } else if (i < L.nW + L.nX) {
        const uint32_t j = i - L.nW, q = 64 * j + lane, u = q / MX, r = q % MX;
        const bool ok = r < (uint32_t)rows_m && u < (uint32_t)a.K / 8;
        dma16(X, ok ? r * (uint32_t)a.ldx * 2 + 16 * u : kOffRow,
              __builtin_amdgcn_readfirstlane(lds0 + L.x_off + 1024 * j));
      } else {
        const uint32_t j = i - L.nW - L.nX, jj = j % L.nS, q = 64 * jj + lane, g8 = q >> 4, c = q & 15;
        const bool ok = c < (uint32_t)rows_n && 8 * g8 < (uint32_t)a.G;
        dma16(j < L.nS ? S : B, ok ? c * G2 + 16 * g8 : kOffRow,
              __builtin_amdgcn_readfirstlane(lds0 + (j < L.nS ? L.s_off : L.b_off) + 1024 * jj));
      }
    }
  }
  wait_vmem();
  __syncthreads();

  // ---- compute: wave w takes groups [g0, g1)
  const int c = lane & 15, j = lane >> 4;
  const int g0 = (wave * a.G) / nw, g1 = ((wave + 1) * a.G) / nw;
  const uint8_t* wbase = smem + (c >> 3) * L.rb_bytes + 16 * (c & 7);
  const uint8_t* xbase = smem + L.x_off + 16 * (c < MX ? c : 0);
  const uint8_t* sbase = smem + L.s_off + 16 * c;
  const uint8_t* bbase = smem + L.b_off + 16 * c;
  const u32x4 ones = {F::kOnes, F::kOnes, F::kOnes, F::kOnes};
  f32x4 tot = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
  for (int g = g0; g < g1; ++g) {
    uint32_t wd[kWDw];
    {
      const uint32_t bo = g * kWBytes + j * (kWBytes / 4);  // byte of row c this lane reads
      if constexpr (kWDw <= 4) {
        const uint8_t* p = wbase + 128 * (bo >> 4) + (bo & 15);
#pragma unroll
        for (int e = 0; e < kWDw; ++e) wd[e] = reinterpret_cast<const uint32_t*>(p)[e];
      } else {
        const uint8_t* p = wbase + 128 * (bo >> 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) wd[e] = reinterpret_cast<const uint32_t*>(p)[e];
#pragma unroll
        for (int e = 0; e < kWDw - 4; ++e) wd[4 + e] = reinterpret_cast<const uint32_t*>(p + 128)[e];
      }
    }
    const uint32_t sb = *reinterpret_cast<const uint16_t*>(sbase + 256 * (g >> 3) + 2 * (g & 7));
    const uint32_t bb = *reinterpret_cast<const uint16_t*>(bbase + 256 * (g >> 3) + 2 * (g & 7));
    const float sc = act_to_f32<F16>(sb);
    const float bc = act_to_f32<F16>(bb) - F::kOff * sc;
    f32x4 aq = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
      const uint32_t u = (g * GS + j * (GS / 4) + 8 * st) >> 3;  // x unit of this step
      u32x4 xv = {0u, 0u, 0u, 0u};
      if (c < MX) xv = *reinterpret_cast<const u32x4*>(xbase + 16 * MX * u);
      uint32_t xd[4] = {xv[0], xv[1], xv[2], xv[3]};
      const u32x4 A = F::acts(xd);
      aq = mma<F16>(A, F::weights(wd, st), aq);
      a1 = mma<F16>(A, ones, a1);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) tot[q] = fmaf(sc, aq[q], fmaf(bc, a1[q], tot[q]));
  }

  // ---- sum the waves' partial tiles (the staging area is free again after the barrier)
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int q = 0; q < 4; ++q) red[wave * 256 + (4 * j + q) * 16 + c] = tot[q];
  __syncthreads();
  for (int e = threadIdx.x; e < 256; e += blockDim.x) {  // a workgroup may have one wave only
    const int r = e >> 4, col = e & 15;
    float v = 0.0f;
    for (int w = 0; w < nw; ++w) v += red[w * 256 + e];
    if (r < rows_m && col < rows_n)
      reinterpret_cast<uint16_t*>(a.y)[(int64_t)r * a.ldy + n0 + col] = f32_to_act<F16>(v);
  }
}

// The staged kernel for up to 8 rows of x when the workgroup's tile fits in LDS: K in
// multiples of 256 (4-bit) / 128 (8-bit), so each weight row block is whole DMA blocks,
// and K / gs a multiple of 8, so each 16-byte scale load ends inside its row.
constexpr uint32_t kQmvMaxLds = 96 * 1024;

template <int BITS, int GS, bool F16, int MX>
int32_t launch_qmv(hipStream_t st, const QmmArgs& a, int nw) {
  const QmvLayout L(a.K, BITS, GS, MX);
  static bool attr_set = false;  // every instantiation needs the LDS above 64 KB allowed once
  if (!attr_set) {
    const int32_t rc = check_hip(hipFuncSetAttribute((const void*)qmv_kernel<BITS, GS, F16, MX>,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, kQmvMaxLds),
                                 "quantized_matmul: LDS attribute");
    if (rc) return rc;
    attr_set = true;
  }
  const uint32_t lds = L.bytes > (uint32_t)nw * 1024 ? L.bytes : (uint32_t)nw * 1024;
  hipLaunchKernelGGL((qmv_kernel<BITS, GS, F16, MX>), dim3((a.N + 15) / 16), dim3(64 * nw), lds, st, a);
  return check_hip(hipGetLastError(), "quantized_matmul launch");
}

// Whether the staged kernel takes this call (and with how many rows of x).
int qmv_rows(int M, int K, int gs, int bits) {
  if (M > 8 || (K * bits / 128) % 8 != 0 || (K / gs) % 8 != 0) return 0;
  const int mx = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
  return QmvLayout(K, bits, gs, mx).bytes <= kQmvMaxLds ? mx : 0;
}

template <int BITS, int GS, bool F16>
int32_t launch_qmv_rows(hipStream_t st, const QmmArgs& a, int mx, int nw) {
  if (mx == 1) return launch_qmv<BITS, GS, F16, 1>(st, a, nw);
  if (mx == 2) return launch_qmv<BITS, GS, F16, 2>(st, a, nw);
  if (mx == 4) return launch_qmv<BITS, GS, F16, 4>(st, a, nw);
  return launch_qmv<BITS, GS, F16, 8>(st, a, nw);
}

template <int BITS, int GS, bool F16>
int32_t launch_t(hipStream_t st, QmmArgs a) {
  int nw = a.G / 8;  // waves per workgroup: about 8 groups each, at most 8 waves
  nw = nw < 1 ? 1 : nw > kMaxWaves ? kMaxWaves : nw;
  if (const int mx = qmv_rows(a.M, a.K, GS, BITS)) return launch_qmv_rows<BITS, GS, F16>(st, a, mx, nw);
  const int mr = a.M <= 16 ? 1 : 2;
  a.mtiles = (a.M + 16 * mr - 1) / (16 * mr);
  const int64_t tiles = (int64_t)a.mtiles * ((a.N + 15) / 16);
  a.remap = a.mtiles > 1 && tiles % 8 == 0;
  if (mr == 1)
    hipLaunchKernelGGL((qmm_kernel<BITS, GS, F16, 1>), dim3((unsigned)tiles), dim3(64 * nw), 0, st, a);
  else
    hipLaunchKernelGGL((qmm_kernel<BITS, GS, F16, 2>), dim3((unsigned)tiles), dim3(64 * nw), 0, st, a);
  return check_hip(hipGetLastError(), "quantized_matmul launch");
}

template <bool F16>
int32_t launch_d(hipStream_t st, const QmmArgs& a, int gs, int bits) {
  if (bits == 4) {
    if (gs == 32) return launch_t<4, 32, F16>(st, a);
    if (gs == 64) return launch_t<4, 64, F16>(st, a);
    return launch_t<4, 128, F16>(st, a);
  }
  if (gs == 32) return launch_t<8, 32, F16>(st, a);
  if (gs == 64) return launch_t<8, 64, F16>(st, a);
  return launch_t<8, 128, F16>(st, a);
}

}  // namespace

int32_t launch_qmatmul(hipStream_t st, const void* x, int64_t ldx, const void* w, const void* scales,
                       const void* biases, void* y, int64_t ldy, int M, int N, int K, int gs, int bits,
                       int dtype) {
  if (M == 0) return EMA_OK;
  QmmArgs a;
  a.x = static_cast<const uint8_t*>(x);
  a.w = static_cast<const uint8_t*>(w);
  a.s = static_cast<const uint8_t*>(scales);
  a.b = static_cast<const uint8_t*>(biases);
  a.y = static_cast<uint8_t*>(y);
  a.ldx = ldx;
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.G = K / gs;
  a.mtiles = 1;
  a.remap = 0;
  return dtype == EMA_DTYPE_F16 ? launch_d<true>(st, a, gs, bits) : launch_d<false>(st, a, gs, bits);
}

}  // namespace ema
