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
// Two regimes, as in MLX, whose quantized matmul takes vector kernels for a few rows of x
// and, for many, kernels that dequantise weight tiles into the activation type first:
// - up to 32 rows (and the streaming fallback): exact products, below;
// - more than 32 rows with K a multiple of 64: qgemm_dq_kernel, on weights dequantised
//   into bf16 / f16 (one rounding each) in LDS.
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
// past its range read zeros out of bounds instead of branching. For larger M (when the
// dequantising GEMM does not apply) the row tiles of one weight tile are dispatched
// together on one XCD, so its L2 serves the re-reads.
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

// (x & m) | c in one v_and_or_b32. gfx950's VOP3 encoding takes no 32-bit literal, so with
// literal masks the compiler splits it into v_and + v_or; the empty asm statements hand the
// constants over as VGPR values (set once per kernel) and the compiler selects the fused
// instruction. The instruction itself is left to the compiler: its result feeds MFMA
// operands, and the hazard recognizer inserts the wait states a VALU write needs before an
// MFMA reads it only for instructions it emits itself, not for an inline-asm VALU
// instruction.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t c) {
  asm("" : "+v"(m));
  asm("" : "+v"(c));
  return (x & m) | c;
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
      r[0] = and_or(w, 0x000F000Fu, kMagicBits);
      r[1] = and_or(w >> 4, 0x000F000Fu, kMagicBits);
      r[2] = and_or(w >> 8, 0x000F000Fu, kMagicBits);
      r[3] = and_or(w >> 12, 0x000F000Fu, kMagicBits);
    } else if constexpr (F16) {
      const uint32_t w0 = wd[2 * st], w1 = wd[2 * st + 1];  // bytes 0..3, 4..7
      r[0] = and_or(w0, 0x00FF00FFu, kMagicBits);           // bytes 0, 2
      r[1] = and_or(w0 >> 8, 0x00FF00FFu, kMagicBits);      // bytes 1, 3
      r[2] = and_or(w1, 0x00FF00FFu, kMagicBits);
      r[3] = and_or(w1 >> 8, 0x00FF00FFu, kMagicBits);
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
  // s_nop 0: the DMA reads M0 no earlier than one wait state after the SALU write, a wait
  // the compiler inserts only for the LDS-DMAs it emits itself. (Its SGPR operands need five
  // after a VALU write; check_hazards.py fails the build if the compiler places one closer.)
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(lds_addr)
               : "memory", "m0");
}
__device__ __forceinline__ u32x4 rsrc4(const void* base, uint32_t bytes) {
  const uint64_t addr = (uint64_t)base;
  return u32x4{(uint32_t)addr, (uint32_t)(addr >> 32) & 0xffffu, bytes, 0x00020000u};
}
typedef __attribute__((address_space(3))) void lds_void;

// Staged kernel for up to 32 rows of x. A workgroup owns 16 NT weight rows (NT column
// tiles of 16) and all of K, walked in NC chunks of KCH. All of its weights, scales and
// biases are staged in LDS by DMA issued up front in chunk order (the HBM stream that
// bounds the call, kept in flight from the start); the rows of x, read from L2, pass
// through a ring of NB slots, the DMA of chunk c + NB issued once chunk c is multiplied
// (NB = NC when x fits, so then everything is in flight at once). LDS layout, in 16-byte
// units, chosen so both the DMA (64 consecutive units per instruction, whole 128-byte
// lines of the source) and the MFMA-layout reads (consecutive lanes on consecutive units)
// run without bank conflicts:
//   weights  row block rb = row / 8 (2 NT of them, 128 bytes of padding apart), then
//            unit u of the row, then row % 8:  unit (rb, u, row % 8) <- row, bytes [16 u, +16)
//   x slot   unit u of the chunk, then row r:  unit (u, r) <- x row r, chunk bytes [16 u, +16)
//   scales   unit (g / 8, row) <- row, groups [g, g + 8); biases likewise
constexpr uint32_t kQmvMaxLds = 160 * 1024;  // all of a gfx950 CU's LDS

struct QmvPlan {
  int NT, KCH, NC, NB;
  uint32_t U;         // weight units per row (all of K)
  uint32_t Uc;        // weight units per row per chunk
  uint32_t rb_bytes;  // one row block plus padding
  uint32_t x_off;     // first x slot
  uint32_t x_slot;    // bytes per x slot
  uint32_t nW, nX;    // DMA instructions per chunk (weights, x)
  uint32_t nS;        // DMA instructions for all scales (and again for the biases)
  uint32_t s_off, b_off, z_off, bytes;
};

// 0..31 outstanding vector-memory operations; larger counts wait for 31 (a longer wait).
__device__ __forceinline__ void wait_vmcnt(uint32_t n) {
  switch (n) {
#define EMA_VM(i) case i: __builtin_amdgcn_s_waitcnt(0x0F70 | ((i) & 15) | (((i) >> 4) << 14)); break;
    EMA_VM(0) EMA_VM(1) EMA_VM(2) EMA_VM(3) EMA_VM(4) EMA_VM(5) EMA_VM(6) EMA_VM(7)
    EMA_VM(8) EMA_VM(9) EMA_VM(10) EMA_VM(11) EMA_VM(12) EMA_VM(13) EMA_VM(14) EMA_VM(15)
    EMA_VM(16) EMA_VM(17) EMA_VM(18) EMA_VM(19) EMA_VM(20) EMA_VM(21) EMA_VM(22) EMA_VM(23)
    EMA_VM(24) EMA_VM(25) EMA_VM(26) EMA_VM(27) EMA_VM(28) EMA_VM(29) EMA_VM(30)
#undef EMA_VM
    default: __builtin_amdgcn_s_waitcnt(0x0F70 | 15 | (1 << 14)); break;
  }
}

template <int BITS, int GS, bool F16, int MX, int NT>
__global__ __launch_bounds__(64 * kMaxWaves) void qmv_kernel(QmmArgs a, QmvPlan p) {
  using F = Fields<BITS, F16>;
  constexpr int MR = MX > 16 ? 2 : 1;       // row tiles of 16
  constexpr int kSteps = GS / 32;
  constexpr int kWDw = GS * BITS / 128;
  constexpr uint32_t kWBytes = GS * BITS / 8;
  constexpr int kRows = 16 * NT;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)smem;

  const int n0 = blockIdx.x * kRows;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = kMaxWaves;
  const int rows_n = min(kRows, a.N - n0), rows_m = min(MX, a.M);
  const uint32_t wrow = (uint32_t)a.K * BITS / 8;
  const uint32_t G2 = (uint32_t)a.G * 2;
  const u32x4 W = rsrc4(a.w + (int64_t)n0 * wrow, rows_n * wrow);
  const u32x4 X = rsrc4(a.x, (rows_m - 1) * (uint32_t)a.ldx * 2 + (uint32_t)a.K * 2);
  const u32x4 S = rsrc4(a.s + (int64_t)n0 * G2, rows_n * G2);
  const u32x4 B = rsrc4(a.b + (int64_t)n0 * G2, rows_n * G2);

  // Each wave issues instructions wave, wave + nw, ... of every list, so it issues the
  // same number of each kind per chunk (cw weights, cx x).
  auto mine = [&](uint32_t n) -> uint32_t { return n > (uint32_t)wave ? (n - wave + nw - 1) / nw : 0; };
  const uint32_t cw = mine(p.nW), cx = mine(p.nX);
  auto issue_w = [&](int c) {
    for (uint32_t i = wave; i < p.nW; i += nw) {
      // 64 units of chunk c's part of one row block (8 Uc is a multiple of 64)
      const uint32_t per_rb = 8 * p.Uc, rb = (64 * i) / per_rb, first = 64 * i - rb * per_rb, rem = first + lane;
      const uint32_t row = rb * 8 + (rem & 7), u = (uint32_t)c * p.Uc + (rem >> 3);
      dma16(W, row < (uint32_t)rows_n ? row * wrow + 16 * u : kOffRow,
            __builtin_amdgcn_readfirstlane(lds0 + rb * p.rb_bytes + 16 * (8 * (uint32_t)c * p.Uc + first)));
    }
  };
  auto issue_x = [&](int c) {
    const uint32_t kb = (uint32_t)c * p.KCH;
    for (uint32_t i = wave; i < p.nX; i += nw) {
      const uint32_t q = 64 * i + lane, u = q / MX, r = q % MX;
      const bool ok = r < (uint32_t)rows_m && u < (uint32_t)p.KCH / 8;
      dma16(X, ok ? r * (uint32_t)a.ldx * 2 + 2 * kb + 16 * u : kOffRow,
            __builtin_amdgcn_readfirstlane(lds0 + p.x_off + (uint32_t)(c % p.NB) * p.x_slot + 1024 * i));
    }
  };
  if (threadIdx.x < 4) reinterpret_cast<uint32_t*>(smem + p.z_off)[threadIdx.x] = 0u;
  // scales and biases first (needed from chunk 0 on), then weights and x chunk by chunk
  for (uint32_t i = wave; i < 2 * p.nS; i += nw) {
    const uint32_t jj = i % p.nS, q = 64 * jj + lane, g8 = q / kRows, row = q % kRows;
    const bool ok = row < (uint32_t)rows_n && 8 * g8 < (uint32_t)a.G;
    dma16(i < p.nS ? S : B, ok ? row * G2 + 16 * g8 : kOffRow,
          __builtin_amdgcn_readfirstlane(lds0 + (i < p.nS ? p.s_off : p.b_off) + 1024 * jj));
  }
  for (int c = 0; c < p.NC; ++c) {
    issue_w(c);
    if (c < p.NB) issue_x(c);
  }

  // wave -> column tile t, and its share of each chunk's groups
  const int per_t = nw / NT, t = wave / per_t, wt = wave % per_t;
  const int GC = p.KCH / GS;
  const int gb = (wt * GC) / per_t, ge = ((wt + 1) * GC) / per_t;
  const int c16 = lane & 15, j = lane >> 4;
  const int row = 16 * t + c16;  // weight row (output column) of this lane
  const uint8_t* wbase = smem + (row >> 3) * p.rb_bytes + 16 * (row & 7);
  const u32x4 ones = {F::kOnes, F::kOnes, F::kOnes, F::kOnes};
  f32x4 tot[MR];
#pragma unroll
  for (int r = 0; r < MR; ++r) tot[r] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int c = 0; c < p.NC; ++c) {
    // loads issued after chunk c's weights and x may stay in flight
    const int later = p.NC - 1 - c;
    const int x_later = p.NB - 1 < later ? p.NB - 1 : later;
    wait_vmcnt((c < p.NB ? (uint32_t)later * cw : 0u) + (uint32_t)x_later * cx);
    __syncthreads();
    const uint8_t* xbase = smem + p.x_off + (uint32_t)(c % p.NB) * p.x_slot;
#pragma unroll 2
    for (int g = gb; g < ge; ++g) {
      const int gg = c * GC + g;  // group index within K
      uint32_t wd[kWDw];
      {
        const uint32_t bo = gg * kWBytes + j * (kWBytes / 4);
        if constexpr (kWDw <= 4) {
          const uint8_t* q = wbase + 128 * (bo >> 4) + (bo & 15);
#pragma unroll
          for (int e = 0; e < kWDw; ++e) wd[e] = reinterpret_cast<const uint32_t*>(q)[e];
        } else {
          const uint8_t* q = wbase + 128 * (bo >> 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) wd[e] = reinterpret_cast<const uint32_t*>(q)[e];
#pragma unroll
          for (int e = 0; e < kWDw - 4; ++e) wd[4 + e] = reinterpret_cast<const uint32_t*>(q + 128)[e];
        }
      }
      const uint32_t so = 16 * ((gg >> 3) * kRows + row) + 2 * (gg & 7);
      const float sc = act_to_f32<F16>(*reinterpret_cast<const uint16_t*>(smem + p.s_off + so));
      const float bc = act_to_f32<F16>(*reinterpret_cast<const uint16_t*>(smem + p.b_off + so)) - F::kOff * sc;
      f32x4 aq[MR], a1[MR];
#pragma unroll
      for (int r = 0; r < MR; ++r) aq[r] = a1[r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < kSteps; ++st) {
        const uint32_t u = (g * GS + j * (GS / 4) + 8 * st) >> 3;  // x unit of this step
        const u32x4 Bw = F::weights(wd, st);
#pragma unroll
        for (int r = 0; r < MR; ++r) {
          const int xr = 16 * r + c16;
          // rows past MX read the zero block (one address select instead of four value selects)
          const u32x4 xv = *reinterpret_cast<const u32x4*>(xr < MX ? xbase + 16 * (u * MX + xr) : smem + p.z_off);
          const uint32_t xd[4] = {xv[0], xv[1], xv[2], xv[3]};
          const u32x4 A = F::acts(xd);
          aq[r] = mma<F16>(A, Bw, aq[r]);
          a1[r] = mma<F16>(A, ones, a1[r]);
        }
      }
#pragma unroll
      for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int q = 0; q < 4; ++q) tot[r][q] = fmaf(sc, aq[r][q], fmaf(bc, a1[r][q], tot[r][q]));
    }
    if (c + p.NB < p.NC) {
      __syncthreads();  // every wave is done with the slot before it is refilled
      issue_x(c + p.NB);
    }
  }

  // ---- sum the partial tiles of each column tile's waves (no DMA is in flight now)
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int q = 0; q < 4; ++q) red[(wave * MR + r) * 256 + (4 * j + q) * 16 + c16] = tot[r][q];
  __syncthreads();
  for (int e = threadIdx.x; e < NT * MR * 256; e += 64 * nw) {
    const int tt = e / (MR * 256), r = (e / 256) % MR, rr = (e >> 4) & 15, col = e & 15;
    float v = 0.0f;
    for (int w = 0; w < per_t; ++w) v += red[((tt * per_t + w) * MR + r) * 256 + (e & 255)];
    const int m = 16 * r + rr, n = 16 * tt + col;
    if (m < rows_m && n < rows_n)
      reinterpret_cast<uint16_t*>(a.y)[(int64_t)m * a.ldy + n0 + n] = f32_to_act<F16>(v);
  }
}


// Plan of the staged kernel for M <= 32 rows, or NC = 0 when it does not apply: a chunk
// is whole DMA blocks per weight row block (KCH * bits / 128 a multiple of 8) and whole
// groups, K is a multiple of it, and K / gs is a multiple of 8 (each 16-byte scale load
// ends inside its row).
QmvPlan plan_qmv(int N, int K, int gs, int bits, int mx, int cus) {
  QmvPlan none{};
  none.NC = 0;
  if ((K / gs) % 8 != 0) return none;
  const int G = K / gs;
  // two column tiles per workgroup only when 16-column tiles would outnumber the CUs (a
  // second round of workgroups costs more than doubling each one's columns)
  const int nt0 = mx >= 8 && (N + 15) / 16 > cus ? 2 : 1;
  for (int nt = nt0; nt >= 1; --nt) {
    const int rows = 16 * nt;
    for (int kch = 1024; kch >= 128; kch /= 2) {
      if (K % kch || kch % gs || (kch * bits / 128) % 8) continue;
      if (nt == 2 && kch < 256) continue;  // measured: more chunks cost more than a second round
      QmvPlan q{};
      q.NT = nt;
      q.KCH = kch;
      q.NC = K / kch;
      q.U = (uint32_t)K * bits / 128;
      q.Uc = (uint32_t)kch * bits / 128;
      q.rb_bytes = q.U * 128 + 128;
      q.nW = (uint32_t)rows * q.Uc / 64;
      q.nX = ((uint32_t)mx * kch / 8 + 63) / 64;
      q.x_slot = 1024 * q.nX;
      q.nS = ((uint32_t)rows * (G / 8) + 63) / 64;
      q.x_off = ((2 * nt) * q.rb_bytes + 1023) & ~1023u;
      const uint32_t fixed = q.x_off + 2 * 1024 * q.nS;
      // all of x if it fits (then everything is in flight from the start), else the
      // deepest ring that fits beside the weights
      int nb = q.NC;
      while (nb > 2 && fixed + 16 + nb * q.x_slot > kQmvMaxLds) --nb;
      q.NB = nb;
      q.s_off = q.x_off + nb * q.x_slot;
      q.b_off = q.s_off + 1024 * q.nS;
      q.z_off = q.b_off + 1024 * q.nS;  // 16 zero bytes read by rows of x past M
      q.bytes = q.z_off + 16;
      const uint32_t red = (uint32_t)kMaxWaves * (mx > 16 ? 2 : 1) * 1024;
      if (q.bytes < red) q.bytes = red;
      // the largest chunk that fits: fewer chunks, fewer barriers (measured faster at
      // 32 rows than deeper rings of smaller chunks)
      if (q.bytes <= kQmvMaxLds) return q;
    }
  }
  return none;
}

// Variant for 16 or 32 rows of x: the weights, scales and biases are staged in LDS as in
// qmv_kernel (all of K, one round of DMA and one barrier), but x does not pass through LDS:
// each wave loads its own x straight into registers in MFMA layout, kXD groups ahead and
// in the order it consumes them, so no chunk barrier stalls the waves on an L2 round trip.
constexpr int kXD = 4;

template <int BITS, int GS, bool F16, int MX, int NT>
__global__ __launch_bounds__(64 * kMaxWaves) void qmvx_kernel(QmmArgs a, QmvPlan p) {
  using F = Fields<BITS, F16>;
  constexpr int MR = MX > 16 ? 2 : 1;
  constexpr int kSteps = GS / 32;
  constexpr int kWDw = GS * BITS / 128;
  constexpr uint32_t kWBytes = GS * BITS / 8;
  constexpr int kRows = 16 * NT;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)smem;

  const int n0 = blockIdx.x * kRows;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = kMaxWaves;
  const int rows_n = min(kRows, a.N - n0), rows_m = min(MX, a.M);
  const uint32_t wrow = (uint32_t)a.K * BITS / 8;
  const uint32_t G2 = (uint32_t)a.G * 2;
  const u32x4 W = rsrc4(a.w + (int64_t)n0 * wrow, rows_n * wrow);
  const u32x4 S = rsrc4(a.s + (int64_t)n0 * G2, rows_n * G2);
  const u32x4 B = rsrc4(a.b + (int64_t)n0 * G2, rows_n * G2);
  const auto X = rsrc(a.x, (rows_m - 1) * (uint32_t)a.ldx * 2 + (uint32_t)a.K * 2);

  // ---- stage all weights (the plan's chunks back to back: Uc = U) and scales
  for (uint32_t i = wave; i < p.nW + 2 * p.nS; i += nw) {
    if (i < p.nW) {
      const uint32_t per_rb = 8 * p.U, rb = (64 * i) / per_rb, first = 64 * i - rb * per_rb, rem = first + lane;
      const uint32_t row = rb * 8 + (rem & 7), u = rem >> 3;
      dma16(W, row < (uint32_t)rows_n ? row * wrow + 16 * u : kOffRow,
            __builtin_amdgcn_readfirstlane(lds0 + rb * p.rb_bytes + 16 * first));
    } else {
      const uint32_t j = i - p.nW, jj = j % p.nS, q = 64 * jj + lane, g8 = q / kRows, row = q % kRows;
      const bool ok = row < (uint32_t)rows_n && 8 * g8 < (uint32_t)a.G;
      dma16(j < p.nS ? S : B, ok ? row * G2 + 16 * g8 : kOffRow,
            __builtin_amdgcn_readfirstlane(lds0 + (j < p.nS ? p.s_off : p.b_off) + 1024 * jj));
    }
  }

  // ---- wave -> column tile t and a contiguous range of groups
  const int per_t = nw / NT, t = wave / per_t, wt = wave % per_t;
  const int g0 = (wt * a.G) / per_t, g1 = ((wt + 1) * a.G) / per_t;
  const int c16 = lane & 15, j = lane >> 4;
  const int row = 16 * t + c16;
  uint32_t xoff[MR];
#pragma unroll
  for (int r = 0; r < MR; ++r) {
    const int xr = 16 * r + c16;
    xoff[r] = xr < rows_m ? xr * (uint32_t)a.ldx * 2 + j * (GS / 2) : kOffRow;
  }
  uint32_t xd[kXD][MR][kSteps][4];
  auto issue_x = [&](int slot, int g) {  // groups past g1 read zeros (and are not used)
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
      for (int st = 0; st < kSteps; ++st) {
        const uint32_t off = g < g1 && xoff[r] != kOffRow ? xoff[r] + g * (GS * 2) + 16 * st : kOffRow;
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(X, off, 0, 0);
        xd[slot][r][st][0] = v[0];
        xd[slot][r][st][1] = v[1];
        xd[slot][r][st][2] = v[2];
        xd[slot][r][st][3] = v[3];
      }
  };
#pragma unroll
  for (int i = 0; i < kXD; ++i) {
    issue_x(i, g0 + i);
    __builtin_amdgcn_sched_barrier(0);
  }
  // the DMA came before those loads: wait for it alone, then publish the weights
  wait_vmcnt((uint32_t)(kXD * MR * kSteps));
  __syncthreads();

  const uint8_t* wbase = smem + (row >> 3) * p.rb_bytes + 16 * (row & 7);
  const u32x4 ones = {F::kOnes, F::kOnes, F::kOnes, F::kOnes};
  f32x4 tot[MR];
#pragma unroll
  for (int r = 0; r < MR; ++r) tot[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int turns = (g1 - g0 + kXD - 1) / kXD;
  for (int turn = 0; turn < turns; ++turn) {
#pragma unroll
    for (int i = 0; i < kXD; ++i) {
      const int g = g0 + turn * kXD + i;
      if (g < g1) {
        uint32_t wd[kWDw];
        const uint32_t bo = g * kWBytes + j * (kWBytes / 4);
        if constexpr (kWDw <= 4) {
          const uint8_t* q = wbase + 128 * (bo >> 4) + (bo & 15);
#pragma unroll
          for (int e = 0; e < kWDw; ++e) wd[e] = reinterpret_cast<const uint32_t*>(q)[e];
        } else {
          const uint8_t* q = wbase + 128 * (bo >> 4);
#pragma unroll
          for (int e = 0; e < 4; ++e) wd[e] = reinterpret_cast<const uint32_t*>(q)[e];
#pragma unroll
          for (int e = 0; e < kWDw - 4; ++e) wd[4 + e] = reinterpret_cast<const uint32_t*>(q + 128)[e];
        }
        const uint32_t so = 16 * ((g >> 3) * kRows + row) + 2 * (g & 7);
        const float sc = act_to_f32<F16>(*reinterpret_cast<const uint16_t*>(smem + p.s_off + so));
        const float bc = act_to_f32<F16>(*reinterpret_cast<const uint16_t*>(smem + p.b_off + so)) - F::kOff * sc;
        f32x4 aq[MR], a1[MR];
#pragma unroll
        for (int r = 0; r < MR; ++r) aq[r] = a1[r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < kSteps; ++st) {
          const u32x4 Bw = F::weights(wd, st);
#pragma unroll
          for (int r = 0; r < MR; ++r) {
            const u32x4 A = F::acts(xd[i][r][st]);
            aq[r] = mma<F16>(A, Bw, aq[r]);
            a1[r] = mma<F16>(A, ones, a1[r]);
          }
        }
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
          for (int q = 0; q < 4; ++q) tot[r][q] = fmaf(sc, aq[r][q], fmaf(bc, a1[r][q], tot[r][q]));
      }
      issue_x(i, g + kXD);  // the slot's registers are dead once the MFMAs have read them
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- sum the partial tiles of each column tile's waves
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int q = 0; q < 4; ++q) red[(wave * MR + r) * 256 + (4 * j + q) * 16 + c16] = tot[r][q];
  __syncthreads();
  for (int e = threadIdx.x; e < NT * MR * 256; e += 64 * nw) {
    const int tt = e / (MR * 256), r = (e / 256) % MR, rr = (e >> 4) & 15, col = e & 15;
    float v = 0.0f;
    for (int w = 0; w < per_t; ++w) v += red[((tt * per_t + w) * MR + r) * 256 + (e & 255)];
    const int m = 16 * r + rr, n = 16 * tt + col;
    if (m < rows_m && n < rows_n)
      reinterpret_cast<uint16_t*>(a.y)[(int64_t)m * a.ldy + n0 + n] = f32_to_act<F16>(v);
  }
}

// Plan of qmvx_kernel: all weights and scales of 16 NT rows in LDS (x not staged).
QmvPlan plan_qmvx(int N, int K, int gs, int bits, int cus) {
  QmvPlan none{};
  none.NC = 0;
  if ((K / gs) % 8 != 0 || (K * bits / 128) % 8 != 0) return none;
  const int G = K / gs;
  const int nt0 = (N + 15) / 16 > cus ? 2 : 1;
  for (int nt = nt0; nt >= 1; --nt) {
    const int rows = 16 * nt;
    QmvPlan q{};
    q.NT = nt;
    q.KCH = K;
    q.NC = 1;
    q.NB = 1;
    q.U = (uint32_t)K * bits / 128;
    q.Uc = q.U;
    q.rb_bytes = q.U * 128 + 128;
    q.nW = (uint32_t)rows * q.U / 64;
    q.nX = 0;
    q.x_slot = 0;
    q.nS = ((uint32_t)rows * (G / 8) + 63) / 64;
    q.x_off = ((2 * nt) * q.rb_bytes + 1023) & ~1023u;
    q.s_off = q.x_off;
    q.b_off = q.s_off + 1024 * q.nS;
    q.z_off = q.b_off + 1024 * q.nS;
    q.bytes = q.z_off + 16;
    const uint32_t red = (uint32_t)kMaxWaves * 2 * 1024;
    if (q.bytes < red) q.bytes = red;
    if (q.bytes <= kQmvMaxLds) return q;
  }
  return none;
}

template <int BITS, int GS, bool F16, int MX, int NT>
int32_t launch_qmvx(hipStream_t st, const QmmArgs& a, const QmvPlan& p) {
  static std::atomic<uint64_t> lds_set{0};  // this instantiation's LDS above 64 KB, per device
  const int32_t rc = allow_lds_once((const void*)qmvx_kernel<BITS, GS, F16, MX, NT>, kQmvMaxLds, &lds_set,
                                    "quantized_matmul: LDS attribute");
  if (rc) return rc;
  hipLaunchKernelGGL((qmvx_kernel<BITS, GS, F16, MX, NT>), dim3((a.N + 16 * NT - 1) / (16 * NT)),
                     dim3(64 * kMaxWaves), p.bytes, st, a, p);
  return check_hip(hipGetLastError(), "quantized_matmul launch");
}

template <int BITS, int GS, bool F16, int MX, int NT>
int32_t launch_qmv(hipStream_t st, const QmmArgs& a, const QmvPlan& p) {
  static std::atomic<uint64_t> lds_set{0};  // this instantiation's LDS above 64 KB, per device
  const int32_t rc = allow_lds_once((const void*)qmv_kernel<BITS, GS, F16, MX, NT>, kQmvMaxLds, &lds_set,
                                    "quantized_matmul: LDS attribute");
  if (rc) return rc;
  hipLaunchKernelGGL((qmv_kernel<BITS, GS, F16, MX, NT>), dim3((a.N + 16 * NT - 1) / (16 * NT)),
                     dim3(64 * kMaxWaves), p.bytes, st, a, p);
  return check_hip(hipGetLastError(), "quantized_matmul launch");
}

int qmv_rows(int M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : M <= 16 ? 16 : 32; }

template <int BITS, int GS, bool F16>
int32_t launch_qmv_rows(hipStream_t st, const QmmArgs& a, int mx, const QmvPlan& p) {
  switch (mx) {
    case 1: return launch_qmv<BITS, GS, F16, 1, 1>(st, a, p);
    case 2: return launch_qmv<BITS, GS, F16, 2, 1>(st, a, p);
    case 4: return launch_qmv<BITS, GS, F16, 4, 1>(st, a, p);
    case 8: return p.NT == 2 ? launch_qmv<BITS, GS, F16, 8, 2>(st, a, p) : launch_qmv<BITS, GS, F16, 8, 1>(st, a, p);
    case 16: return p.NT == 2 ? launch_qmv<BITS, GS, F16, 16, 2>(st, a, p) : launch_qmv<BITS, GS, F16, 16, 1>(st, a, p);
    default: return p.NT == 2 ? launch_qmv<BITS, GS, F16, 32, 2>(st, a, p) : launch_qmv<BITS, GS, F16, 32, 1>(st, a, p);
  }
}

// ---------------------------------------------------------------- dequantising GEMM (M > 32)
// MLX's quantized matmul for many rows (its qmm kernels) dequantises each weight tile into
// the activation type in threadgroup memory and multiplies that. Here likewise: a workgroup
// owns a 256 x 128 tile of y (256 rows of x, 128 weight rows) and walks K in chunks of 64,
// with two roles:
// - eight compute waves, wave (wm, wn) = (wave % 4, wave / 4) multiplying its 64 x 64 block
//   as 4 x 4 16x16x32 MFMA tiles, two k-steps per chunk, from LDS only;
// - eight loader waves, which load each chunk's x, packed weights, scales and biases three
//   chunks ahead into registers (three sets in turn), then write x into LDS and dequantise
//   the weights into it, w = round(fma(s, q, b)) in f32 then to bf16 / f16 (the rounding
//   of MLX's dequantise, parity unpinned as to one rounding or two).
// Two LDS buffers: the loaders fill chunk c + 1's while the compute waves multiply chunk
// c's, one barrier per chunk. The loaders issue every load on every path (a chunk past the
// end loads at offsets past the ranges: zeros, no memory access), so the compiler's waits
// count exactly the chunk they need.
// LDS per buffer: x rows (128 bytes of a chunk each), then weight rows; the 16-byte units of
// a row are swizzled, unit u at u ^ ((row >> 1) & 7), so that the 16 rows an MFMA operand
// read touches at one unit land on 16 different bank groups (rows are 128 bytes: two per
// 256-byte bank cycle).
// Workgroup order: with the tile grid split into eight regions of whole rows and columns
// of tiles, consecutive workgroups (which the dispatcher spreads over the eight XCDs) take
// the same place in different regions, so each XCD works through one region and its L2
// holds that region's x rows and weight rows.
constexpr int kDqBM = 256, kDqBN = 128, kDqKC = 64, kDqCompute = 8, kDqLoaders = 8;
constexpr uint32_t kDqXBytes = kDqBM * 128, kDqBuf = kDqXBytes + kDqBN * 128;
constexpr uint32_t kDqLds = 2 * kDqBuf;  // 96 KB: one workgroup per CU

struct DqPlan {
  int mtiles, ntiles;
  int rm, rn;  // tile rows / columns per region (regions: mtiles / rm x ntiles / rn = 8), or 0
};

// byte I of x as f32 (v_cvt_f32_ubyteI)
template <int I>
__device__ __forceinline__ float ubyte_f32(uint32_t x) { return (float)((x >> (8 * I)) & 0xFFu); }
__device__ __forceinline__ uint32_t dq_unit(uint32_t row, uint32_t u) { return row * 8 + (u ^ ((row >> 1) & 7)); }
// Buffer loads issued as asm, untracked by the compiler: the loader waits for them with
// explicit vmcnt counts (a wait that takes the loaded registers as operands, so that no use
// of them moves above it). With compiler-tracked loads, register reuse across the rotating
// register sets made it wait for the loads just issued.
__device__ __forceinline__ u32x4 ld128(u32x4 rs, uint32_t off) {
  u32x4 v;
  asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(v) : "v"(off), "s"(rs));
  return v;
}
__device__ __forceinline__ u32x2 ld64(u32x4 rs, uint32_t off) {
  u32x2 v;
  asm volatile("buffer_load_dwordx2 %0, %1, %2, 0 offen" : "=v"(v) : "v"(off), "s"(rs));
  return v;
}
__device__ __forceinline__ uint32_t ld16u(u32x4 rs, uint32_t off) {
  uint32_t v;
  asm volatile("buffer_load_ushort %0, %1, %2, 0 offen" : "=v"(v) : "v"(off), "s"(rs));
  return v;
}

template <int BITS, int GS, bool F16>
__global__ __launch_bounds__(64 * (kDqCompute + kDqLoaders)) void qgemm_dq_kernel(QmmArgs a, DqPlan p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  int mt, nt;
  if (p.rm > 0) {
    const int x8 = blockIdx.x % 8, l = blockIdx.x / 8;
    const int rgm = p.mtiles / p.rm;  // regions along M
    mt = (x8 % rgm) * p.rm + l % p.rm;
    nt = (x8 / rgm) * p.rn + l / p.rm;
  } else {
    mt = blockIdx.x / p.ntiles;
    nt = blockIdx.x % p.ntiles;
  }
  const int m0 = mt * kDqBM, n0 = nt * kDqBN;
  const int rows_m = min(kDqBM, a.M - m0), rows_n = min(kDqBN, a.N - n0);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int NC = a.K / kDqKC;

  if (wave >= kDqCompute) {
    // ---- loader: lane ll of the eight loader waves
    const uint32_t ll = (uint32_t)(tid - 64 * kDqCompute);
    const uint32_t xrow = (uint32_t)a.ldx * 2, wrow = (uint32_t)a.K * BITS / 8, G2 = (uint32_t)a.G * 2;
    const u32x4 Xr = rsrc4(a.x + (int64_t)m0 * xrow, (rows_m - 1) * xrow + (uint32_t)a.K * 2);
    const u32x4 W = rsrc4(a.w + (int64_t)n0 * wrow, rows_n * wrow);
    const u32x4 S = rsrc4(a.s + (int64_t)n0 * G2, rows_n * G2);
    const u32x4 Bi = rsrc4(a.b + (int64_t)n0 * G2, rows_n * G2);
    // x: unit u = ll % 8 of rows ll / 8 + 64 i (one load instruction covers 8 whole rows)
    const uint32_t xu = ll & 7, xr0 = ll >> 3;
    uint32_t x_off[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t row = xr0 + 64 * i;
      x_off[i] = row < (uint32_t)rows_m ? row * xrow + 16 * xu : kOffRow;
    }
    // weights: k 16 h .. 16 h + 15 of the chunk (h = ll % 4, LDS units 2 h, 2 h + 1) for
    // weight row ll / 4
    constexpr int kWq = BITS / 2;  // words of 16 fields
    const uint32_t wr_row = ll >> 2, wh = ll & 3;
    const bool w_in = wr_row < (uint32_t)rows_n;
    typedef uint32_t wv_t __attribute__((ext_vector_type(kWq)));
    struct Regs {
      u32x4 x[4];
      wv_t w;
      uint32_t s, b;
    };
    auto load = [&](int c, Regs& r) __attribute__((always_inline)) {
      const bool real = c < NC;
      const uint32_t cc = real ? (uint32_t)c : 0u, no = real ? 0u : kOffRow;
#pragma unroll
      for (int i = 0; i < 4; ++i) r.x[i] = ld128(Xr, (x_off[i] | no) + cc * (2 * kDqKC));
      const uint32_t k0 = cc * kDqKC + 16 * wh;
      const uint32_t wo = (w_in ? wr_row * wrow + k0 * BITS / 8 : kOffRow) | no;
      if constexpr (kWq == 2) r.w = ld64(W, wo);
      else r.w = ld128(W, wo);
      const uint32_t so = (w_in ? wr_row * G2 + 2 * (k0 / GS) : kOffRow) | no;
      r.s = ld16u(S, so);
      r.b = ld16u(Bi, so);
    };
    // loads per chunk: 4 of x, 1 of weights, 2 of scales and biases; staging a set waits
    // for it with the two later sets' loads still in flight
    auto wait_set = [&](Regs& r) __attribute__((always_inline)) {
      asm volatile("s_waitcnt vmcnt(14)"
                   : "+v"(r.x[0]), "+v"(r.x[1]), "+v"(r.x[2]), "+v"(r.x[3]), "+v"(r.w), "+v"(r.s), "+v"(r.b)
                   :
                   : "memory");
    };
    auto stage = [&](Regs& r, int buf) __attribute__((always_inline)) {
      wait_set(r);
      uint8_t* const xb = smem + (uint32_t)buf * kDqBuf;
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(xb + 16 * dq_unit(xr0 + 64 * i, xu)) = r.x[i];
      const float sc = act_to_f32<F16>(r.s), bc = act_to_f32<F16>(r.b);
      uint8_t* const wb = xb + kDqXBytes;
#pragma unroll
      for (int u = 0; u < 2; ++u) {  // unit 2 wh + u: k 8 u .. 8 u + 7 of the quarter
        float q[8];
        if constexpr (BITS == 4) {
          const uint32_t wd = r.w[u], lo = wd & 0x0F0F0F0Fu, hi = (wd >> 4) & 0x0F0F0F0Fu;  // fields 2i, 2i + 1
          q[0] = ubyte_f32<0>(lo);
          q[1] = ubyte_f32<0>(hi);
          q[2] = ubyte_f32<1>(lo);
          q[3] = ubyte_f32<1>(hi);
          q[4] = ubyte_f32<2>(lo);
          q[5] = ubyte_f32<2>(hi);
          q[6] = ubyte_f32<3>(lo);
          q[7] = ubyte_f32<3>(hi);
        } else {
          q[0] = ubyte_f32<0>(r.w[2 * u]);
          q[1] = ubyte_f32<1>(r.w[2 * u]);
          q[2] = ubyte_f32<2>(r.w[2 * u]);
          q[3] = ubyte_f32<3>(r.w[2 * u]);
          q[4] = ubyte_f32<0>(r.w[2 * u + 1]);
          q[5] = ubyte_f32<1>(r.w[2 * u + 1]);
          q[6] = ubyte_f32<2>(r.w[2 * u + 1]);
          q[7] = ubyte_f32<3>(r.w[2 * u + 1]);
        }
        u32x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = (uint32_t)f32_to_act<F16>(__builtin_fmaf(sc, q[2 * e], bc)) |
                 ((uint32_t)f32_to_act<F16>(__builtin_fmaf(sc, q[2 * e + 1], bc)) << 16);
        *reinterpret_cast<u32x4*>(wb + 16 * dq_unit(wr_row, 2 * wh + u)) = o;
      }
    };
    // chunk k in register set k % 3: at iteration c, chunk c + 3 is loaded into the set
    // chunk c left (staged at iteration c - 1) and chunk c + 1 is staged
    Regs r0, r1, r2;
    load(0, r0);
    load(1, r1);
    load(2, r2);
    stage(r0, 0);
    __syncthreads();
    for (int c = 0; c < NC;) {
      load(c + 3, r0);
      if (c + 1 < NC) stage(r1, (c + 1) & 1);
      __syncthreads();
      if (++c >= NC) break;
      load(c + 3, r1);
      if (c + 1 < NC) stage(r2, (c + 1) & 1);
      __syncthreads();
      if (++c >= NC) break;
      load(c + 3, r2);
      if (c + 1 < NC) stage(r0, (c + 1) & 1);
      __syncthreads();
      ++c;
    }
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");  // the loads past the end (zeros)
    return;
  }

  // ---- compute
  const int wm = wave & 3, wn = wave >> 2;
  const uint32_t r16 = (uint32_t)lane & 15, j = (uint32_t)lane >> 4;
  f32x4 acc[4][4];
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) acc[rt][ct] = f32x4{0.f, 0.f, 0.f, 0.f};
  __syncthreads();  // chunk 0 staged
  for (int c = 0; c < NC; ++c) {
    const uint8_t* const xb = smem + (uint32_t)(c & 1) * kDqBuf;
    const uint8_t* const wb = xb + kDqXBytes;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const uint32_t u = 4 * ks + j;
      u32x4 A[4], B[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        A[t] = *reinterpret_cast<const u32x4*>(xb + 16 * dq_unit(64 * wm + 16 * t + r16, u));
        B[t] = *reinterpret_cast<const u32x4*>(wb + 16 * dq_unit(64 * wn + 16 * t + r16, u));
      }
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) acc[rt][ct] = mma<F16>(A[rt], B[ct], acc[rt][ct]);
    }
    __syncthreads();
  }

  // lane (r16, j) of tile (rt, ct) holds rows 4j .. 4j + 3 of column r16
#pragma unroll
  for (int rt = 0; rt < 4; ++rt)
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int m = 64 * wm + 16 * rt + 4 * (int)j + q, n = 64 * wn + 16 * ct + (int)r16;
        if (m < rows_m && n < rows_n)
          reinterpret_cast<uint16_t*>(a.y)[(int64_t)(m0 + m) * a.ldy + n0 + n] = f32_to_act<F16>(acc[rt][ct][q]);
      }
}

// Plan of the dequantising GEMM: K a multiple of the chunk and of the group, x within one
// buffer range per tile. Regions: 2 x 4, 4 x 2, 1 x 8 or 8 x 1 whole tile rows and columns,
// the one with the least bytes per region, when the grid divides into them.
bool plan_dq(int M, int N, int K, int gs, int bits, int64_t ldx, DqPlan* p) {
  if (K % kDqKC || K % gs || (int64_t)kDqBM * ldx * 2 + (int64_t)K * 2 >= ((int64_t)1 << 31)) return false;
  p->mtiles = (M + kDqBM - 1) / kDqBM;
  p->ntiles = (N + kDqBN - 1) / kDqBN;
  p->rm = p->rn = 0;
  const double xb = (double)kDqBM * K * 2, wb = (double)kDqBN * K * (bits / 8.0 + 4.0 / gs);
  double best = 0;
  for (int gm = 1; gm <= 8; gm *= 2) {  // regions along M
    const int gn = 8 / gm;
    if (p->mtiles % gm || p->ntiles % gn) continue;
    const int rm = p->mtiles / gm, rn = p->ntiles / gn;
    const double bytes = rm * xb + rn * wb;
    if (p->rm == 0 || bytes < best) {
      best = bytes;
      p->rm = rm;
      p->rn = rn;
    }
  }
  return true;
}

template <int BITS, int GS, bool F16>
int32_t launch_dq(hipStream_t st, const QmmArgs& a, const DqPlan& p) {
  static std::atomic<uint64_t> lds_set{0};  // this instantiation's LDS above 64 KB, per device
  const int32_t rc = allow_lds_once((const void*)qgemm_dq_kernel<BITS, GS, F16>, kDqLds, &lds_set,
                                    "quantized_matmul: LDS attribute");
  if (rc) return rc;
  hipLaunchKernelGGL((qgemm_dq_kernel<BITS, GS, F16>), dim3((unsigned)(p.mtiles * p.ntiles)),
                     dim3(64 * (kDqCompute + kDqLoaders)),
                     kDqLds, st, a, p);
  return check_hip(hipGetLastError(), "quantized_matmul launch");
}

// ---------------------------------------------------------------- one row of x (M = 1)
// VALU dot products instead of MFMA (which would spend 15 of its 16 rows on nothing): lane
// gl of a slot of L lanes takes group gl (+ L i) of a weight row, so a wave reads whole
// rows coalesced; 64 / L slots cover 64 / L rows at once, and a wave walks R rows. The
// same exact pairs as the MFMA kernels (C + q against x, v_dot2_f32_bf16 / _f16: exact
// products, f32 sums) and the same per-group combination y += s a_q + (b - C s) a_1, with
// a_1 = sum of the group's x. The row sums are reduced across the slot's lanes with xor
// shuffles. R is chosen so the grid is about one workgroup of eight waves per CU.
constexpr int kGemvRows = 4;  // most rows per lane
// rows per lane for one format: two where a group of one row holds 32 dwords (8 bits,
// group 128), whose four rows would not fit the register file beside x
constexpr int gemv_rows(int bits, int gs) { return bits * gs / 32 >= 32 ? 2 : kGemvRows; }

template <bool F16>
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  if constexpr (F16) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a), __builtin_bit_cast(h2, b), c, false);
  } else {
    return dot2_bf16(a, b, c);
  }
}

template <int BITS, int GS, bool F16>
__global__ __launch_bounds__(512) void qgemv1_kernel(QmmArgs a, int np, int L, int gpl) {
  using F = Fields<BITS, F16>;
  constexpr int kRows = gemv_rows(BITS, GS);
  constexpr int kWDw = GS * BITS / 32;  // dwords of one group of one weight row
  constexpr int kXDw = GS / 2;          // dwords of one group of x
  constexpr int kBlk = GS / 8;          // blocks of 8 weights per group
  constexpr uint32_t kWBytes = GS * BITS / 8;
  const int lane = threadIdx.x & 63;
  const int slots = 64 / L, slot = lane / L, gl = lane % L;
  const int R = slots * np;  // rows per wave
  // wave-uniform (an SGPR): the buffer resources below must be uniform, or every load
  // becomes a loop over the lanes' distinct resources
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row0 = ((int64_t)blockIdx.x * 8 + wave) * R;
  // waves past the last row still take part in the x staging and its barrier
  const int rows = (int)max((int64_t)0, min((int64_t)R, (int64_t)a.N - row0));
  const uint32_t wrow = (uint32_t)a.K * BITS / 8;
  const uint32_t G2 = (uint32_t)a.G * 2;
  const auto W = rsrc(a.w + row0 * wrow, rows * wrow);
  const auto S = rsrc(a.s + row0 * G2, rows * G2);
  const auto Bi = rsrc(a.b + row0 * G2, rows * G2);
  const u32x4 ones = {F::kOnes, F::kOnes, F::kOnes, F::kOnes};
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];

  // x once per workgroup into LDS (LDS-DMA, 1 KB per instruction), issued before the
  // weights; every wave then reads its x from LDS instead of from L2
  {
    const u32x4 X = rsrc4(a.x, (uint32_t)a.K * 2);
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)smem;
    const uint32_t nxd = ((uint32_t)a.K * 2 + 1023) / 1024;
    for (uint32_t i = wave; i < nxd; i += 8)
      dma16(X, 1024 * i + 16 * lane, __builtin_amdgcn_readfirstlane(lds0 + 1024 * i));
  }

  float y[kRows];
#pragma unroll
  for (int p = 0; p < kRows; ++p) y[p] = 0.0f;
  for (int i = 0; i < gpl; ++i) {
    const uint32_t g = gl + L * i;
    // weights, scale and bias of every row, in the order they are used
    uint32_t wd[kRows][kWDw], sb[kRows], bb[kRows];
#pragma unroll
    for (int p = 0; p < kRows; ++p) {
      const int r = slot + slots * p;  // row within the wave's rows
      const bool ok = p < np && r < rows;
      load_dw<kWDw>(W, ok ? r * wrow + g * kWBytes : kOffRow, wd[p]);
      sb[p] = __builtin_amdgcn_raw_buffer_load_b16(S, ok ? r * G2 + 2 * g : kOffRow, 0, 0);
      bb[p] = __builtin_amdgcn_raw_buffer_load_b16(Bi, ok ? r * G2 + 2 * g : kOffRow, 0, 0);
    }
    if (i == 0) {
      // the x DMA came before these loads: wait for it alone, then publish it
      constexpr uint32_t kPerRow = (kWDw <= 2 ? 1 : kWDw / 4) + 2;
      wait_vmcnt(kRows * kPerRow);
      __syncthreads();
    }
    uint32_t xd[kXDw];
#pragma unroll
    for (int e = 0; e < kXDw / 4; ++e) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(smem + g * (GS * 2) + 16 * e);
      xd[4 * e] = v[0];
      xd[4 * e + 1] = v[1];
      xd[4 * e + 2] = v[2];
      xd[4 * e + 3] = v[3];
    }
    // x paired as the fields are, and its group sum (exact pairs, f32 sums)
    u32x4 xa[kBlk];
    float a1 = 0.0f;
#pragma unroll
    for (int blk = 0; blk < kBlk; ++blk) {
      xa[blk] = F::acts(xd + 4 * blk);
#pragma unroll
      for (int e = 0; e < 4; ++e) a1 = dot2<F16>(xa[blk][e], ones[e], a1);
    }
#pragma unroll
    for (int p = 0; p < kRows; ++p) {
      if (p >= np) break;
      float aq = 0.0f;
#pragma unroll
      for (int blk = 0; blk < kBlk; ++blk) {
        const u32x4 B = F::weights(wd[p], blk);
#pragma unroll
        for (int e = 0; e < 4; ++e) aq = dot2<F16>(xa[blk][e], B[e], aq);
      }
      const float sc = act_to_f32<F16>(sb[p]);
      const float bc = act_to_f32<F16>(bb[p]) - F::kOff * sc;
      y[p] = fmaf(sc, aq, fmaf(bc, a1, y[p]));
    }
  }
  // sum over the slot's L lanes (xor partners stay inside the slot)
#pragma unroll
  for (int p = 0; p < kRows; ++p) {
    if (p >= np) break;
    float v = y[p];
    for (int m = 1; m < L; m <<= 1) v += __shfl_xor(v, m, 64);
    const int r = slot + slots * p;
    if (gl == 0 && r < rows)
      reinterpret_cast<uint16_t*>(a.y)[row0 + r] = f32_to_act<F16>(v);
  }
}

// Whether the one-row kernel takes this call: K / gs a power of two up to 64, or a
// multiple of 64, and x (2 K bytes) within 64 KB of LDS.
bool gemv1_fits(int G, int K) { return (G % 64 == 0 || (G <= 64 && (G & (G - 1)) == 0)) && K <= 32768; }

template <int BITS, int GS, bool F16>
int32_t launch_gemv1(hipStream_t st, const QmmArgs& a, int cus) {
  const int L = a.G < 64 ? a.G : 64, slots = 64 / L, gpl = a.G / L;
  // rows per lane: about one workgroup of eight waves per CU, at most the format's limit
  const int64_t want = ((int64_t)a.N + 8LL * cus * slots - 1) / (8LL * cus * slots);
  constexpr int kRows = gemv_rows(BITS, GS);
  const int np = (int)(want < 1 ? 1 : want > kRows ? kRows : want);
  const int64_t waves = ((int64_t)a.N + slots * np - 1) / (slots * np);
  const uint32_t lds = ((uint32_t)a.K * 2 + 1023) & ~1023u;  // x, in whole DMA blocks
  hipLaunchKernelGGL((qgemv1_kernel<BITS, GS, F16>), dim3((unsigned)((waves + 7) / 8)), dim3(512), lds, st, a, np,
                     L, gpl);
  return check_hip(hipGetLastError(), "quantized_matmul launch");
}

template <int BITS, int GS, bool F16>
int32_t launch_t(hipStream_t st, QmmArgs a) {
  int nw = a.G / 8;  // waves per workgroup: about 8 groups each, at most 8 waves
  nw = nw < 1 ? 1 : nw > kMaxWaves ? kMaxWaves : nw;
  const int cus = device_cus();
  if (a.M == 1 && gemv1_fits(a.G, a.K)) return launch_gemv1<BITS, GS, F16>(st, a, cus);
  if (a.M <= 32) {
    const int mx = qmv_rows(a.M);
    const QmvPlan p = plan_qmv(a.N, a.K, GS, BITS, mx, cus);
    if (mx >= 16) {
      // x through an LDS ring shared by the column tiles (qmv_kernel) when it reaches the
      // wanted tile count, else x through registers (qmvx_kernel), whose LDS holds only
      // the weights (measured: 4-bit q|k|v at 32 rows 14.9 us against 19.9; 8-bit, where
      // only qmvx_kernel fits two tiles, 21.9 against 23.7)
      const int want = (a.N + 15) / 16 > cus ? 2 : 1;
      const QmvPlan px = p.NC > 0 && p.NT == want ? QmvPlan{} : plan_qmvx(a.N, a.K, GS, BITS, cus);
      if (px.NC > 0 && (p.NC == 0 || px.NT == want)) {
        if (mx == 16)
          return px.NT == 2 ? launch_qmvx<BITS, GS, F16, 16, 2>(st, a, px) : launch_qmvx<BITS, GS, F16, 16, 1>(st, a, px);
        return px.NT == 2 ? launch_qmvx<BITS, GS, F16, 32, 2>(st, a, px) : launch_qmvx<BITS, GS, F16, 32, 1>(st, a, px);
      }
    }
    if (p.NC > 0) return launch_qmv_rows<BITS, GS, F16>(st, a, mx, p);
  } else {
    DqPlan dp;
    if (plan_dq(a.M, a.N, a.K, GS, BITS, a.ldx, &dp)) return launch_dq<BITS, GS, F16>(st, a, dp);
  }
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
