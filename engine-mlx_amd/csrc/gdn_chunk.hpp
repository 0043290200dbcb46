// Pieces shared by the chunkwise Gated DeltaNet kernels (gdn_chunk.hip, gdn_wy.hip), gfx950.
//
// Chunks of C = 32 tokens. With gamma_t = g_0 g_1 ... g_t over a chunk that starts from the
// state S_0 (S is [Dv, Dk], f32), the recurrence of crates/ops/src/gdn.rs:83-150 unrolls to
//   (I + A) Delta = W,   A[t][s] = beta_t (gamma_t / gamma_s) (k_t . k_s)  for s < t,
//                        W_t = beta_t (v_t - gamma_t S_0 k_t),
//   y_t = gamma_t S_0 q_t + sum_{s <= t} (gamma_t / gamma_s) (q_t . k_s) delta_s,
//   S_C = gamma_{C-1} S_0 + sum_s (gamma_{C-1} / gamma_s) delta_s k_s^T.
// Gate ratios are exp2 of differences of log2 cumulative sums, never quotients.
//
// MFMA operand order: the k slots of a 16x16x32 product may be any permutation shared by
// both operands. Slot j (0..7) of lane group c (0..3) stands for token (or dk) p(c, j) =
// 4c + j for j < 4 and 16 + 4c + (j - 4) for j >= 4 of the 32-wide k step: where an
// accumulator tile pair holds its values, so accumulators feed later products as B
// operands without a transpose. Staged A operands follow that order:
//   KA / QA [mt 2][k step DK/32][lane (m, c)]: row 16 mt + m, dk 32 s + p(c, 0..7);
//   KTA [dk tile DK/16][lane (m, c)]: dk 16 t + m of tokens p(c, 0..7);
//   an f32 32-wide operand (L0, L1, M10, the decayed Q K^T) as [hi | lo][lane], lane (m, c)
//   holding row m, columns p(c, 0..7) (16-wide blocks: columns 4c..4c+3 in slots 0..3,
//   zeros in slots 4..7).
// f32 operands are split into bf16 hi + lo, x - hi - lo = O(2^-16 |x|); products keep
// hi*hi, hi*lo and lo*hi. q and k are bf16 inputs, exact as operands.
#pragma once

#include "ema_common.hpp"

namespace ema {
namespace gdnc {

constexpr int kC = 32;       // tokens per chunk
constexpr int kPad = 36;     // row stride (floats) of 32-wide scratch matrices
constexpr int kPad16 = 20;   // row stride (floats) of 16-wide ones
constexpr int kMatWaves = 4; // waves that form one chunk's matrices

// Staged K / Q of one chunk (bytes): KA, QA, KTA.
template <int DK>
struct In {
  static constexpr int kKa = 2 * (DK / 32) * 64;  // u32x4 units of KA (= QA)
  static constexpr int kKta = (DK / 16) * 64;     // u32x4 units of KTA
  static constexpr int kBytes = (2 * kKa + kKta) * 16;
};

// One chunk's matrices (bytes): operand tiles (u32x4 units, each [hi|lo][lane]) then the
// token vectors (floats): gamma[32], beta[32], rho[32] = gamma_31 / gamma_t, gamma_31 at 96.
struct Out {
  static constexpr int kL0 = 0, kL1 = 128, kM10 = 256, kQM = 384;  // QM: [mt][hi|lo][lane]
  static constexpr int kVec = 640 * 16;
  static constexpr int kBytes = kVec + 128 * 4;
};

// Scratch of the matrix waves (floats).
struct Scr {
  static constexpr int kW = 0;                   // per wave: log2 g_t, log2 gamma_t, beta_t (96)
  static constexpr int kAmT = 96 * kMatWaves;    // A, column-major: AmT[s * kPad + t] = A[t][s]
  static constexpr int kQkT = kAmT + 32 * kPad;  // decayed Q K^T, column-major
  static constexpr int kLcT = kQkT + 32 * kPad;  // LcT[(16 b + j) * kPad16 + t] = L_b[t][j]
  static constexpr int kFloats = kLcT + 32 * kPad16;
};

// Orders this wave's LDS writes before its later reads by other lanes.
__device__ __forceinline__ void lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

__device__ __forceinline__ float exp2_(float x) { return __builtin_amdgcn_exp2f(x); }

// a[0..3], b[0..3] -> the bf16 slots 0..7 of hi and lo, x = hi + lo + O(2^-16 |x|).
__device__ __forceinline__ void split8(const f32x4 a, const f32x4 b, bf16x8& hi, bf16x8& lo) {
  u32x4 h, l;
  #pragma unroll
  for (int e = 0; e < 2; ++e) {
    const uint32_t ha = pack_bf16x2(a[2 * e], a[2 * e + 1]);
    const uint32_t hb = pack_bf16x2(b[2 * e], b[2 * e + 1]);
    h[e] = ha;
    h[2 + e] = hb;
    l[e] = pack_bf16x2(a[2 * e] - bf16_lo(ha), a[2 * e + 1] - bf16_hi(ha));
    l[2 + e] = pack_bf16x2(b[2 * e] - bf16_lo(hb), b[2 * e + 1] - bf16_hi(hb));
  }
  hi = as_bf16x8(h);
  lo = as_bf16x8(l);
}

// K / Q staging by 2 DK lanes (li = 0 .. 2 DK - 1): lane li < DK takes 4 tokens x 8 dk of K,
// the others of Q. fetch() loads into registers (tokens past the end read the last token,
// in bounds and without a branch); stage() zeroes those and writes KA / QA / KTA.
template <int DK>
struct KqStager {
  const uint16_t* src;
  int64_t tok_stride;
  int quad, eg, T;
  bool ld_q;
  u32x4 pc[4];

  __device__ __forceinline__ void init(int li, const uint16_t* q, const uint16_t* k, int64_t b, int kh, int hk,
                                       int T_) {
    ld_q = li >= DK;
    const int gi = ld_q ? li - DK : li;
    quad = gi / (DK / 8);
    eg = gi % (DK / 8);
    T = T_;
    src = (ld_q ? q : k) + (b * T * hk + kh) * DK + eg * 8;
    tok_stride = (int64_t)hk * DK;
  }
  __device__ __forceinline__ void fetch(int ch) {
    #pragma unroll
    for (int kq = 0; kq < 4; ++kq) {
      const int t = ch * kC + 4 * quad + kq;
      pc[kq] = *(const u32x4*)(src + (t < T ? t : T - 1) * tok_stride);
    }
  }
  __device__ __forceinline__ void stage(int ch, uint8_t* in) {
    constexpr int S = DK / 32;
    #pragma unroll
    for (int kq = 0; kq < 4; ++kq)
      if (ch * kC + 4 * quad + kq >= T) pc[kq] = u32x4{0u, 0u, 0u, 0u};
    u32x2* const dst = (u32x2*)(in + (ld_q ? In<DK>::kKa * 16 : 0));
    #pragma unroll
    for (int kq = 0; kq < 4; ++kq) {
      const int tok = 4 * quad + kq, mt = tok >> 4, m = tok & 15;
      #pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int d0 = 8 * eg + 4 * hf, s = d0 >> 5, c = (d0 & 15) >> 2, up = (d0 >> 4) & 1;
        dst[((mt * S + s) * 64 + m + 16 * c) * 2 + up] = u32x2{pc[kq][2 * hf], pc[kq][2 * hf + 1]};
      }
    }
    if (!ld_q) {  // the 4 tokens of this quad are 4 consecutive KTA slots
      u32x2* const kt = (u32x2*)(in + 2 * In<DK>::kKa * 16);
      const int c = quad & 3, up = quad >> 2;
      #pragma unroll
      for (int x = 0; x < 8; ++x) {
        const int d = 8 * eg + x, t = d >> 4, m = d & 15, w = x >> 1, sh = 16 * (x & 1);
        const uint32_t e0 = (pc[0][w] >> sh) & 0xffffu, e1 = (pc[1][w] >> sh) & 0xffffu;
        const uint32_t e2 = (pc[2][w] >> sh) & 0xffffu, e3 = (pc[3][w] >> sh) & 0xffffu;
        kt[(t * 64 + m + 16 * c) * 2 + up] = u32x2{e0 | (e1 << 16), e2 | (e3 << 16)};
      }
    }
  }
};

// Matrix wave mw (0..3) forms its share of one chunk's matrices from the staged K / Q at
// `in` into `out`: 0: L0 = (I + N_0)^-1, 1: L1, 2: M10 = A[16.., ..16] and the first row
// tile of the decayed Q K^T, 3: its second row tile; wave 0 also writes the token
// vectors. gv / bv: g_t and beta_t in lane t < n_valid (the chunk's real tokens); padding
// tokens take g = 1, beta = 0. The shares touch disjoint scratch, so no wave waits for
// another.
template <int DK>
__device__ __forceinline__ void chunk_matrices(int mw, int lane, int n_valid, float gv, float bv, const uint8_t* in,
                                               uint8_t* out, float* scr) {
  constexpr int S = DK / 32;
  const int g16 = lane & 15, c4 = lane >> 4;
  if (!(lane < n_valid)) {
    gv = 1.f;
    bv = 0.f;
  }
  float* const vec = (float*)(out + Out::kVec);
  float* const ws = scr + Scr::kW + 96 * mw;
  float* const AmT = scr + Scr::kAmT;
  float* const QkT = scr + Scr::kQkT;
  const u32x4* const KA = (const u32x4*)in;
  const u32x4* const QA = KA + In<DK>::kKa;
  // this wave's product tiles (K K^T into A, or Q K^T), operands read up front
  const int n_tiles = mw >= 2 ? 2 : 1;
  const bool qk0 = mw == 3, qk1 = mw >= 2;
  const int mt0 = mw == 0 ? 0 : 1, nt0 = mw == 1 ? 1 : 0;
  const int mt1 = mw == 2 ? 0 : 1, nt1 = mw == 2 ? 0 : 1;
  u32x4 a4[2][S], b4[2][S];
  #pragma unroll
  for (int s = 0; s < S; ++s) {
    a4[0][s] = (qk0 ? QA : KA)[(mt0 * S + s) * 64 + lane];
    b4[0][s] = KA[(nt0 * S + s) * 64 + lane];
    if (n_tiles == 2) {
      a4[1][s] = (qk1 ? QA : KA)[(mt1 * S + s) * 64 + lane];
      b4[1][s] = KA[(nt1 * S + s) * 64 + lane];
    }
  }
  // log2 gamma_t = sum of log2 g over tokens 0..t, summed in token order by every lane;
  // log2 0 = -inf is clamped so that differences stay finite
  float lv = __builtin_amdgcn_logf(gv);
  lv = lv < -150.f ? -150.f : lv;
  if (lane < kC) {
    ws[lane] = lv;
    ws[64 + lane] = bv;
  }
  lds_fence();
  float x = 0.f, xc = 0.f;
  #pragma unroll
  for (int q = 0; q < 8; ++q) {
    const f32x4 l4 = *(const f32x4*)&ws[4 * q];
    #pragma unroll
    for (int e = 0; e < 4; ++e) {
      xc += l4[e];
      x += 4 * q + e <= lane ? l4[e] : 0.f;
    }
  }
  if (lane < kC) ws[32 + lane] = x;
  if (mw == 0) {
    if (lane < kC) {
      vec[lane] = exp2_(x);
      vec[32 + lane] = bv;
      vec[64 + lane] = exp2_(xc - x);
    }
    if (lane == 0) vec[96] = exp2_(xc);
  }
  f32x4 acc[2];
  #pragma unroll
  for (int k = 0; k < 2; ++k) {
    acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (k < n_tiles)
      #pragma unroll
      for (int s = 0; s < S; ++s) acc[k] = mfma16(as_bf16x8(a4[k][s]), as_bf16x8(b4[k][s]), acc[k]);
  }
  lds_fence();
  // decay and mask; lane (g, c) of tile (mt, nt) holds rows t = 16 mt + 4 c + i, column
  // s = 16 nt + g; written column-major
  #pragma unroll
  for (int k = 0; k < 2; ++k) {
    if (k < n_tiles) {
      const bool qk = k == 0 ? qk0 : qk1;
      const int mt = k == 0 ? mt0 : mt1, nt = k == 0 ? nt0 : nt1;
      const int sc = 16 * nt + g16, t0 = 16 * mt + 4 * c4;
      const f32x4 lt = *(const f32x4*)&ws[32 + t0];
      const f32x4 bt = *(const f32x4*)&ws[64 + t0];
      const float ls = ws[32 + sc];
      f32x4 v;
      #pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float r = sc <= t0 + i ? exp2_(lt[i] - ls) : 0.f;
        v[i] = qk ? r * acc[k][i] : (sc < t0 + i ? bt[i] * r * acc[k][i] : 0.f);
      }
      *(f32x4*)&(qk ? QkT : AmT)[sc * kPad + t0] = v;
    }
  }
  lds_fence();
  const int m = g16, c = c4;
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  u32x4* const op = (u32x4*)out;
  bf16x8 hi, lo;
  if (mw < 2) {
    // L_b = (I + N_b)^-1, N_b = A[16 b.., 16 b..], by forward substitution with N_b in
    // registers; lane j (and its copies in the other lane groups) owns column j
    const int bk = mw, j = g16;
    const float* const N = AmT + 16 * bk * kPad + 16 * bk;  // N[s * kPad + t] = N_b[t][s]
    f32x4 nq[15][4];
    #pragma unroll
    for (int s = 0; s < 15; ++s)
      #pragma unroll
      for (int q = (s + 1) >> 2; q < 4; ++q) nq[s][q] = *(const f32x4*)&N[s * kPad + 4 * q];
    float xv[16];
    #pragma unroll
    for (int t = 0; t < 16; ++t) xv[t] = t == j ? 1.f : 0.f;
    #pragma unroll
    for (int s = 0; s < 15; ++s)
      #pragma unroll
      for (int q = (s + 1) >> 2; q < 4; ++q)
        #pragma unroll
        for (int e = 0; e < 4; ++e)
          if (4 * q + e > s) xv[4 * q + e] = fmaf(-nq[s][q][e], xv[s], xv[4 * q + e]);
    float* const lc = scr + Scr::kLcT + 16 * bk * kPad16;  // lc[j * kPad16 + t] = L_b[t][j]
    if (lane < 16)
      #pragma unroll
      for (int q = 0; q < 4; ++q)
        *(f32x4*)&lc[j * kPad16 + 4 * q] = f32x4{xv[4 * q], xv[4 * q + 1], xv[4 * q + 2], xv[4 * q + 3]};
    lds_fence();
    f32x4 lv4;  // A operand: lane (m, c) holds L_b[m][4 c .. 4 c + 3] in slots 0..3
    #pragma unroll
    for (int e = 0; e < 4; ++e) lv4[e] = lc[(4 * c + e) * kPad16 + m];
    split8(lv4, z, hi, lo);
    const int base = bk ? Out::kL1 : Out::kL0;
    op[base + lane] = __builtin_bit_cast(u32x4, hi);
    op[base + 64 + lane] = __builtin_bit_cast(u32x4, lo);
  } else if (mw == 2) {
    f32x4 mv, q0;  // M10[m][4 c + e] and QKm[m][4 c + e]
    #pragma unroll
    for (int e = 0; e < 4; ++e) {
      mv[e] = AmT[(4 * c + e) * kPad + 16 + m];
      q0[e] = QkT[(4 * c + e) * kPad + m];
    }
    split8(mv, z, hi, lo);
    op[Out::kM10 + lane] = __builtin_bit_cast(u32x4, hi);
    op[Out::kM10 + 64 + lane] = __builtin_bit_cast(u32x4, lo);
    split8(q0, z, hi, lo);
    op[Out::kQM + lane] = __builtin_bit_cast(u32x4, hi);
    op[Out::kQM + 64 + lane] = __builtin_bit_cast(u32x4, lo);
  } else {
    f32x4 q1a, q1b;  // QKm[16 + m][4 c + e] and QKm[16 + m][16 + 4 c + e]
    #pragma unroll
    for (int e = 0; e < 4; ++e) {
      q1a[e] = QkT[(4 * c + e) * kPad + 16 + m];
      q1b[e] = QkT[(16 + 4 * c + e) * kPad + 16 + m];
    }
    split8(q1a, q1b, hi, lo);
    op[Out::kQM + 128 + lane] = __builtin_bit_cast(u32x4, hi);
    op[Out::kQM + 192 + lane] = __builtin_bit_cast(u32x4, lo);
  }
}

// Blocked solve with the chunk's L0 / L1 / M10 operands at `out`: given X as a B operand
// (lane (n, c), slot j: X[p(c, j)][n], split into xh / xl) and X's second half in
// accumulator layout (x1[i] = X[16 + 4 c + i][n]), returns (I + A)^-1 X as two
// accumulator tiles: r[mt][i] = ((I + A)^-1 X)[16 mt + 4 c + i][n].
__device__ __forceinline__ void blocked_solve(const uint8_t* out, int lane, bf16x8 xh, bf16x8 xl, f32x4 x1,
                                              f32x4 (&r)[2]) {
  const u32x4* const op = (const u32x4*)out;
  const bf16x8 l0h = as_bf16x8(op[Out::kL0 + lane]), l0l = as_bf16x8(op[Out::kL0 + 64 + lane]);
  const bf16x8 l1h = as_bf16x8(op[Out::kL1 + lane]), l1l = as_bf16x8(op[Out::kL1 + 64 + lane]);
  const bf16x8 mh = as_bf16x8(op[Out::kM10 + lane]), ml = as_bf16x8(op[Out::kM10 + 64 + lane]);
  const f32x4 z = {0.f, 0.f, 0.f, 0.f};
  r[0] = mfma16(l0l, xh, z);
  r[0] = mfma16(l0h, xl, r[0]);
  r[0] = mfma16(l0h, xh, r[0]);
  bf16x8 h, l;
  split8(r[0], z, h, l);
  f32x4 mu = mfma16(ml, h, z);
  mu = mfma16(mh, l, mu);
  mu = mfma16(mh, h, mu);
  split8(x1 - mu, z, h, l);
  r[1] = mfma16(l1l, h, z);
  r[1] = mfma16(l1h, l, r[1]);
  r[1] = mfma16(l1h, h, r[1]);
}

}  // namespace gdnc
}  // namespace ema
