// Gated DeltaNet scan in chunkwise form on the bf16 matrix cores, gfx950.
//
// Replaces, for bf16 activations and at least kGdnChunkMinTokens tokens, the sequential
// scan of crates/ops/src/gdn_forward.rs:173-192, which applies gdn_step
// (crates/ops/src/gdn.rs:83-150) once per token. Per token t and value head h, with the
// f32 state S of shape [Dv, Dk]:
//   S_t = g_t S_{t-1} + delta_t k_t^T,  delta_t = beta_t (v_t - g_t S_{t-1} k_t),  y_t = S_t q_t.
// Over a chunk of C = 32 tokens that starts from the state S_0, with gamma_t = g_0 g_1 ... g_t,
// the recurrence unrolls (the UT / WY form of the delta rule) to
//   (I + A) Delta = W,   A[t][s] = beta_t (gamma_t / gamma_s) (k_t . k_s)  for s < t,
//                        W_t = beta_t (v_t - gamma_t S_0 k_t),
//   y_t = gamma_t S_0 q_t + sum_{s <= t} (gamma_t / gamma_s) (q_t . k_s) delta_s,
//   S_C = gamma_{C-1} S_0 + sum_s (gamma_{C-1} / gamma_s) delta_s k_s^T,
// so a chunk is a handful of small matrix products and one 32 x 32 unit-lower-triangular
// inverse, and the serial chain is one step per chunk instead of one per token. Gate ratios
// are exp2 of differences of log2 cumulative sums (never quotients, which underflow).
//
// Precision: q and k are bf16 inputs, exact as MFMA operands. Every f32 operand (state,
// W, Delta, the inverse, the decayed q.k matrix) is split into bf16 hi + lo with
// x - hi - lo = O(2^-16 |x|), and a product keeps hi*hi, hi*lo and lo*hi (f32 accumulate);
// the inverse is formed in f32. The state stays f32 in registers across the scan.
//
// Work split: one workgroup per (batch, value head, 64 state rows), eight waves:
//   - four row waves own 16 state rows each (the state, transposed, in MFMA accumulator
//     layout: lane (g, c) holds S[row g][16 t + 4 c + i] in tile t) and run the chunk's
//     products;
//   - four matrix waves form the chunk-shared quantities one chunk ahead, one share each
//     (the diagonal blocks L0, L1 of (I + A)^-1 by forward substitution; the off-diagonal
//     block M10 of A; the decayed Q K^T), written to LDS in MFMA operand layout, and stage
//     the K and Q tiles of the chunk two ahead from HBM into LDS. The row waves finish the
//     inverse as a blocked solve: Delta_0 = L0 W_0, Delta_1 = L1 (W_1 - M10 Delta_0).
// K, Q inputs are triple-buffered in LDS and the chunk matrices double-buffered, so one
// workgroup barrier per chunk orders everything.
//
// Operand permutation: an MFMA sums over k in any order, so the k slots of a 16x16x32
// product may be any permutation shared by both operands. Slot j (0..7) of lane group
// c (0..3) stands for token (or dk) p(c, j) = 4c + j for j < 4 and 16 + 4c + (j - 4) for
// j >= 4 within the 32-wide k step, which is exactly where an accumulator tile pair holds
// its values. Accumulators (the state, W, Delta) then feed the next product as B operands
// with no transpose; the A operands (K, Q, K^T, the chunk matrices) are staged in LDS in
// that order.
#include "ema_common.hpp"

namespace ema {
namespace {

constexpr int kC = 32;                            // tokens per chunk
constexpr int kRowWaves = 4;                      // 16 state rows each
constexpr int kMatWaves = 4;                      // chunk matrices and K / Q staging
constexpr int kThreadsC = 64 * (kRowWaves + kMatWaves);
constexpr int kPad = 36;                          // row stride (floats) of 32-wide scratch matrices
constexpr int kPad16 = 20;                        // row stride (floats) of 16-wide ones

// LDS layout. Operand tiles are lane-major: 16 bytes per lane, 64 lanes per tile.
template <int DK>
struct ChunkLds {
  static constexpr int kKa = 2 * (DK / 32) * 64;  // u32x4 units of KA (= QA): [mt 2][k step][lane]
  static constexpr int kKta = (DK / 16) * 64;     // K^T tiles: [dk tile][lane]
  static constexpr int kInBytes = (2 * kKa + kKta) * 16;
  // chunk matrices as A operands (u32x4 units), each [hi|lo][lane]: the diagonal blocks of
  // (I + A)^-1, L0 and L1, and the off-diagonal block M10 = A[16.., ..16] (16 x 16, in slots
  // 0..3 of every lane group, zero in slots 4..7); the decayed Q K^T as [mt][hi|lo][lane]
  static constexpr int kL0 = 0, kL1 = 128, kM10 = 256, kQM = 384;
  static constexpr int kVec = 640 * 16;           // byte offset of the token vectors in an out buffer
  // token vectors (floats): gamma[32], beta[32], rho[32] = gamma_31 / gamma_t, gamma_31
  static constexpr int kOutBytes = kVec + 128 * 4;
  static constexpr int kOut0 = 3 * kInBytes;
  static constexpr int kScr0 = kOut0 + 2 * kOutBytes;
  // matrix-wave scratch (floats)
  static constexpr int kW = 0;                    // per matrix wave: log2 g_t, log2 gamma_t, beta_t (96)
  static constexpr int kAmT = 96 * kMatWaves;     // A, column-major: AmT[s * kPad + t] = A[t][s]
  static constexpr int kQkT = kAmT + 32 * kPad;   // decayed Q K^T, column-major
  static constexpr int kLcT = kQkT + 32 * kPad;   // LcT[(16 b + j) * kPad16 + t] = L_b[t][j]
  static constexpr int kBytes = kScr0 + (kLcT + 32 * kPad16) * 4;
};

struct ChunkArgs {
  const uint16_t* q;  // [B, T, Hk, DK] bf16
  const uint16_t* k;
  const uint16_t* v;  // [B, T, Hv, Dv] bf16
  const float* g;     // [B, T, Hv]
  const float* beta;  // [B, T, Hv]
  float* state;       // [B, Hv, Dv, DK]
  uint16_t* y;        // [B, T, Hv, Dv] bf16
  int T, hk, hv, dv;
  int groups;         // workgroups per (batch, value head): ceil(Dv / 64)
};

// Orders this wave's LDS writes before its later reads by other lanes.
__device__ __forceinline__ void lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

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

__device__ __forceinline__ float exp2_(float x) { return __builtin_amdgcn_exp2f(x); }

template <int DK>
__global__ __launch_bounds__(kThreadsC) void gdn_chunk_kernel(ChunkArgs a) {
  typedef ChunkLds<DK> L;
  constexpr int S = DK / 32;   // 32-wide k steps over dk
  constexpr int NT = DK / 16;  // 16-wide dk tiles of the state
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  float* const scr = (float*)(lds + L::kScr0);

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g16 = lane & 15, c4 = lane >> 4;
  int64_t id = blockIdx.x;
  const int rg = (int)(id % a.groups);
  id /= a.groups;
  const int h = (int)(id % a.hv);
  const int64_t b = id / a.hv;
  const int kh = h / (a.hv / a.hk);
  const int T = a.T;
  const int nch = (T + kC - 1) / kC;

  // ---- K / Q staging: matrix-wave lanes 0 .. 2 DK - 1, 4 tokens x 8 dk each ----
  const int mw = wave - kRowWaves;  // matrix wave index (negative on row waves)
  const int ltid = tid - 64 * kRowWaves;
  const bool loader = mw >= 0 && ltid < 2 * DK;  // 2 DK <= 64 kMatWaves
  const bool ld_q = ltid >= DK;
  const int gi = ld_q ? ltid - DK : ltid;
  const int quad = gi / (DK / 8), eg = gi % (DK / 8);
  const uint16_t* const src = (ld_q ? a.q : a.k) + (b * T * a.hk + kh) * DK + eg * 8;
  const int64_t tok_stride = (int64_t)a.hk * DK;
  u32x4 pc[4];
  auto fetch = [&](int ch) __attribute__((always_inline)) {
    // tokens past the end read the last token (in bounds, no branch); stage() zeroes them,
    // so the loads stay in flight until then
    #pragma unroll
    for (int kq = 0; kq < 4; ++kq) {
      const int t = ch * kC + 4 * quad + kq;
      pc[kq] = *(const u32x4*)(src + (t < T ? t : T - 1) * tok_stride);
    }
  };
  auto stage = [&](int ch) __attribute__((always_inline)) {
    uint8_t* const in = lds + (ch % 3) * L::kInBytes;
    // KA / QA: lane (m, c) of tile (mt, s) holds row 16 mt + m, dk 32 s + p(c, 0..7)
    u32x2* const dst = (u32x2*)(in + (ld_q ? L::kKa * 16 : 0));
    #pragma unroll
    for (int kq = 0; kq < 4; ++kq)
      if (ch * kC + 4 * quad + kq >= T) pc[kq] = u32x4{0u, 0u, 0u, 0u};
    #pragma unroll
    for (int kq = 0; kq < 4; ++kq) {
      const int tok = 4 * quad + kq, mt = tok >> 4, m = tok & 15;
      #pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int d0 = 8 * eg + 4 * hf, s = d0 >> 5, c = (d0 & 15) >> 2, up = (d0 >> 4) & 1;
        dst[((mt * S + s) * 64 + m + 16 * c) * 2 + up] = u32x2{pc[kq][2 * hf], pc[kq][2 * hf + 1]};
      }
    }
    if (!ld_q) {
      // K^T tiles: lane (m, c) of dk tile t holds dk 16 t + m of tokens p(c, 0..7); the
      // 4 tokens of this quad are 4 consecutive slots
      u32x2* const kt = (u32x2*)(in + 2 * L::kKa * 16);
      const int c = quad & 3, up = quad >> 2;
      #pragma unroll
      for (int x = 0; x < 8; ++x) {
        const int d = 8 * eg + x, t = d >> 4, m = d & 15, w = x >> 1, sh = 16 * (x & 1);
        const uint32_t e0 = (pc[0][w] >> sh) & 0xffffu, e1 = (pc[1][w] >> sh) & 0xffffu;
        const uint32_t e2 = (pc[2][w] >> sh) & 0xffffu, e3 = (pc[3][w] >> sh) & 0xffffu;
        kt[(t * 64 + m + 16 * c) * 2 + up] = u32x2{e0 | (e1 << 16), e2 | (e3 << 16)};
      }
    }
  };

  // ---- chunk-matrix wave ----
  const int64_t gb_base = b * T * a.hv + h;  // g / beta of token t at gb_base + t * hv
  auto load_gb = [&](int ch, float& gv, float& bv) __attribute__((always_inline)) {
    const int t = ch * kC + lane;
    const int64_t at = gb_base + (int64_t)(lane < kC && t < T ? t : T - 1) * a.hv;
    gv = a.g[at];
    bv = a.beta[at];
  };
  // Matrix wave mw forms its share of the chunk matrices: 0: L0 = (I + N_0)^-1, 1: L1, 2: M10
  // and the first row tile of the decayed Q K^T, 3: its second row tile; wave 0 also writes
  // the token vectors. The shares touch disjoint scratch, so no wave waits for another.
  auto chunk_matrices = [&](int ch, float gv, float bv) __attribute__((always_inline)) {
    if (!(lane < kC && ch * kC + lane < T)) {  // padding tokens: g = 1, beta = 0
      gv = 1.f;
      bv = 0.f;
    }
    const uint8_t* const in = lds + (ch % 3) * L::kInBytes;
    uint8_t* const out = lds + L::kOut0 + (ch & 1) * L::kOutBytes;
    float* const vec = (float*)(out + L::kVec);
    float* const ws = scr + L::kW + 96 * mw;
    float* const AmT = scr + L::kAmT;
    float* const QkT = scr + L::kQkT;
    const u32x4* const KA = (const u32x4*)in;
    const u32x4* const QA = KA + L::kKa;
    // this wave's product tiles (kind 0: K K^T into A, 1: Q K^T), operands read up front
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
      float* const lc = scr + L::kLcT + 16 * bk * kPad16;  // lc[j * kPad16 + t] = L_b[t][j]
      if (lane < 16)
        #pragma unroll
        for (int q = 0; q < 4; ++q)
          *(f32x4*)&lc[j * kPad16 + 4 * q] = f32x4{xv[4 * q], xv[4 * q + 1], xv[4 * q + 2], xv[4 * q + 3]};
      lds_fence();
      // A operand: lane (m, c) holds L_b[m][4 c .. 4 c + 3] in slots 0..3
      f32x4 lv4;
      #pragma unroll
      for (int e = 0; e < 4; ++e) lv4[e] = lc[(4 * c + e) * kPad16 + m];
      split8(lv4, z, hi, lo);
      const int base = bk ? L::kL1 : L::kL0;
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
      op[L::kM10 + lane] = __builtin_bit_cast(u32x4, hi);
      op[L::kM10 + 64 + lane] = __builtin_bit_cast(u32x4, lo);
      split8(q0, z, hi, lo);
      op[L::kQM + lane] = __builtin_bit_cast(u32x4, hi);
      op[L::kQM + 64 + lane] = __builtin_bit_cast(u32x4, lo);
    } else {
      f32x4 q1a, q1b;  // QKm[16 + m][4 c + e] and QKm[16 + m][16 + 4 c + e]
      #pragma unroll
      for (int e = 0; e < 4; ++e) {
        q1a[e] = QkT[(4 * c + e) * kPad + 16 + m];
        q1b[e] = QkT[(16 + 4 * c + e) * kPad + 16 + m];
      }
      split8(q1a, q1b, hi, lo);
      op[L::kQM + 128 + lane] = __builtin_bit_cast(u32x4, hi);
      op[L::kQM + 192 + lane] = __builtin_bit_cast(u32x4, lo);
    }
  };

  // ---- row waves ----
  const int row0 = (rg * kRowWaves + wave) * 16;
  const bool rows = wave < kRowWaves && row0 < a.dv;
  float* const st_ptr = a.state + ((b * a.hv + h) * a.dv + row0 + g16) * DK + 4 * c4;  // + 16 t
  const int64_t vy_base = (b * T * a.hv + h) * a.dv + row0 + g16;  // + token * hv * dv
  const int64_t vy_tok = (int64_t)a.hv * a.dv;
  // v of tokens 16 mt + 4 c + i as raw bf16 (converted, and zeroed past the end, at use)
  auto load_v = [&](int ch, uint32_t (&vv)[8]) __attribute__((always_inline)) {
    #pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int t = ch * kC + 16 * (e >> 2) + 4 * c4 + (e & 3);
      vv[e] = a.v[vy_base + (t < T ? t : T - 1) * vy_tok];
    }
  };
  f32x4 st[NT];
  auto row_chunk = [&](int ch, const uint32_t (&vraw)[8]) __attribute__((always_inline)) {
    const uint8_t* const in = lds + (ch % 3) * L::kInBytes;
    const uint8_t* const out = lds + L::kOut0 + (ch & 1) * L::kOutBytes;
    const u32x4* const KA = (const u32x4*)in;
    const u32x4* const QA = KA + L::kKa;
    const u32x4* const KT = KA + 2 * L::kKa;
    const u32x4* const OP = (const u32x4*)out;
    const float* const vec = (const float*)(out + L::kVec);
    // S_0 k_t and S_0 q_t: A = K / Q tiles, B = the state (hi + lo)
    f32x4 ks[2], qs[2];
    u32x4 ka4[2][S], qa4[2][S];  // every K / Q operand read up front
    #pragma unroll
    for (int mt = 0; mt < 2; ++mt)
      #pragma unroll
      for (int s = 0; s < S; ++s) {
        ka4[mt][s] = KA[(mt * S + s) * 64 + lane];
        qa4[mt][s] = QA[(mt * S + s) * 64 + lane];
      }
    #pragma unroll
    for (int mt = 0; mt < 2; ++mt) ks[mt] = qs[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    #pragma unroll
    for (int s = 0; s < S; ++s) {
      bf16x8 sh, sl;
      split8(st[2 * s], st[2 * s + 1], sh, sl);
      #pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const bf16x8 ka = as_bf16x8(ka4[mt][s]);
        const bf16x8 qa = as_bf16x8(qa4[mt][s]);
        ks[mt] = mfma16(ka, sl, ks[mt]);
        ks[mt] = mfma16(ka, sh, ks[mt]);
        qs[mt] = mfma16(qa, sl, qs[mt]);
        qs[mt] = mfma16(qa, sh, qs[mt]);
      }
    }
    // the rest of the chunk's operands
    const bf16x8 l0h = as_bf16x8(OP[L::kL0 + lane]), l0l = as_bf16x8(OP[L::kL0 + 64 + lane]);
    const bf16x8 l1h = as_bf16x8(OP[L::kL1 + lane]), l1l = as_bf16x8(OP[L::kL1 + 64 + lane]);
    const bf16x8 mh = as_bf16x8(OP[L::kM10 + lane]), ml = as_bf16x8(OP[L::kM10 + 64 + lane]);
    f32x4 gam[2], bet[2], rho[2];
    #pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      gam[mt] = *(const f32x4*)&vec[16 * mt + 4 * c4];
      bet[mt] = *(const f32x4*)&vec[32 + 16 * mt + 4 * c4];
      rho[mt] = *(const f32x4*)&vec[64 + 16 * mt + 4 * c4];
    }
    const float gc = vec[96];
    // W = beta (V - gamma S_0 k)
    f32x4 vv[2];
    #pragma unroll
    for (int e = 0; e < 8; ++e)
      vv[e >> 2][e & 3] = ch * kC + 16 * (e >> 2) + 4 * c4 + (e & 3) < T ? __uint_as_float(vraw[e] << 16) : 0.f;
    f32x4 w[2];
    #pragma unroll
    for (int mt = 0; mt < 2; ++mt) w[mt] = bet[mt] * (vv[mt] - gam[mt] * ks[mt]);
    // Delta = (I + A)^-1 W by blocks: Delta_0 = L0 W_0, Delta_1 = L1 (W_1 - M10 Delta_0)
    const f32x4 z = {0.f, 0.f, 0.f, 0.f};
    bf16x8 xh, xl;
    split8(w[0], z, xh, xl);
    f32x4 u[2];
    u[0] = mfma16(l0l, xh, z);
    u[0] = mfma16(l0h, xl, u[0]);
    u[0] = mfma16(l0h, xh, u[0]);
    split8(u[0], z, xh, xl);
    f32x4 mu = mfma16(ml, xh, z);
    mu = mfma16(mh, xl, mu);
    mu = mfma16(mh, xh, mu);
    split8(w[1] - mu, z, xh, xl);
    u[1] = mfma16(l1l, xh, z);
    u[1] = mfma16(l1h, xl, u[1]);
    u[1] = mfma16(l1h, xh, u[1]);
    // y = gamma S_0 q + (decayed Q K^T) Delta
    bf16x8 uh, ul;
    split8(u[0], u[1], uh, ul);
    #pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const bf16x8 qh = as_bf16x8(OP[L::kQM + (2 * mt) * 64 + lane]), ql = as_bf16x8(OP[L::kQM + (2 * mt + 1) * 64 + lane]);
      f32x4 yv = gam[mt] * qs[mt];
      yv = mfma16(ql, uh, yv);
      yv = mfma16(qh, ul, yv);
      yv = mfma16(qh, uh, yv);
      #pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = ch * kC + 16 * mt + 4 * c4 + i;
        if (t < T) a.y[vy_base + t * vy_tok] = (uint16_t)f32_to_bf16_bits(yv[i]);
      }
    }
    // S = gamma_31 S_0 + (rho Delta)^T K: A = K^T tiles, B = rho Delta (hi + lo)
    bf16x8 th, tl;
    split8(rho[0] * u[0], rho[1] * u[1], th, tl);
    #pragma unroll
    for (int t = 0; t < NT; ++t) {
      const bf16x8 kt = as_bf16x8(KT[t * 64 + lane]);
      st[t] = st[t] * gc;
      st[t] = mfma16(kt, tl, st[t]);
      st[t] = mfma16(kt, th, st[t]);
    }
  };

  // ---- prologue: chunk 0 staged, state and chunk 0's v / g / beta in registers ----
  uint32_t vcur[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
  float gcur = 1.f, bcur = 0.f;
  if (loader) {
    fetch(0);
    stage(0);
  }
  if (rows) {
    #pragma unroll
    for (int t = 0; t < NT; ++t) st[t] = *(const f32x4*)(st_ptr + 16 * t);
    load_v(0, vcur);
  }
  if (mw >= 0) load_gb(0, gcur, bcur);
  // settle the loads made before the loop, so that the compiler's loop-entry wait count
  // does not make every iteration wait for the iteration's own prefetches
  wait_vmem();
  __syncthreads();

  // iteration i: row waves run chunk i, the matrix waves chunk i + 1 and stage
  // chunk i + 2 into the buffer chunk i - 1 used
  for (int i = -1; i < nch; ++i) {
    const bool ahead = loader && i + 2 < nch;
    if (ahead) fetch(i + 2);
    if (mw >= 0) {
      if (i + 1 < nch) {
        float gn = 1.f, bn = 0.f;
        if (i + 2 < nch) load_gb(i + 2, gn, bn);
        chunk_matrices(i + 1, gcur, bcur);
        gcur = gn;
        bcur = bn;
      }
    } else if (rows && i >= 0) {
      uint32_t vn[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
      if (i + 1 < nch) load_v(i + 1, vn);
      row_chunk(i, vcur);
      #pragma unroll
      for (int e = 0; e < 8; ++e) vcur[e] = vn[e];
    }
    if (ahead) stage(i + 2);
    __syncthreads();
  }
  if (rows)
    #pragma unroll
    for (int t = 0; t < NT; ++t) *(f32x4*)(st_ptr + 16 * t) = st[t];
}

template <int DK>
int32_t launch_dk(hipStream_t s, const ChunkArgs& a, int64_t blocks) {
  static std::atomic<uint64_t> lds_set;
  const int32_t rc = allow_lds_once((const void*)gdn_chunk_kernel<DK>, ChunkLds<DK>::kBytes, &lds_set,
                                    "ema_gdn_scan: LDS attribute");
  if (rc) return rc;
  hipLaunchKernelGGL(gdn_chunk_kernel<DK>, dim3((unsigned)blocks), dim3(kThreadsC), ChunkLds<DK>::kBytes, s, a);
  return check_hip(hipGetLastError(), "ema_gdn_scan chunked launch");
}

}  // namespace

int32_t launch_gdn_chunked(hipStream_t s, const void* q, const void* k, const void* v, const float* g,
                           const float* beta, float* state, void* y, int B, int T, int hk, int hv, int dk,
                           int dv) {
  ChunkArgs a;
  a.q = (const uint16_t*)q;
  a.k = (const uint16_t*)k;
  a.v = (const uint16_t*)v;
  a.g = g;
  a.beta = beta;
  a.state = state;
  a.y = (uint16_t*)y;
  a.T = T;
  a.hk = hk;
  a.hv = hv;
  a.dv = dv;
  a.groups = (dv + 16 * kRowWaves - 1) / (16 * kRowWaves);
  const int64_t blocks = (int64_t)B * hv * a.groups;
  if (blocks > 0x7fffffff) return set_error(EMA_ERR_SHAPE, "ema_gdn_scan: grid too large");
  return dk == 64 ? launch_dk<64>(s, a, blocks) : launch_dk<128>(s, a, blocks);
}

}  // namespace ema
