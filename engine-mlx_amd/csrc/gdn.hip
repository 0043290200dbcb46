// Gated DeltaNet recurrent scan, gfx950.
//
// Replaces gdn_step (crates/ops/src/gdn.rs:83-150), the fused step kernel
// gdn_step_metal (crates/ops/src/gdn_metal.rs:16-50 body, :56-88 head expansion) and the
// sequential scan that calls them once per token (crates/ops/src/gdn_forward.rs:173-192).
// Per token t and value head h, with key head h / (Hv / Hk) (the tile-based expansion of
// gdn.rs:100-110 and gdn_metal.rs:70-81) and the f32 state S[h] of shape [Dv, Dk]:
//   S = g S;  kv = S k;  delta = (v - kv) beta;  S = S + delta k^T;  y = S q
// (gdn.rs:97-140, in that order). g and beta arrive precomputed, as in both reference
// paths (compute_gate and sigmoid in gdn_forward.rs:160-164).
//
// Work split: one wave per (batch, value head, R rows of S). L = 64 / R lanes share a row;
// lane part p holds the Dk / L elements dk = 4 p + 4 L i + j (j < 4), so a 16-byte state
// load of a wave covers 16 L contiguous bytes of each of its rows, and the row sums kv and
// y are four-way partial sums plus log2(L) DPP exchanges that leave the same value in all
// lanes of the row. The state stays in registers over the n_tokens steps: it is read and
// written once per call.
// R = 4 (16 lanes and 256 contiguous bytes per row per load):
//   - n_tokens = 1 (the decode step): HBM-bound, 8 Dk Dv bytes of state traffic per
//     (batch, value head); k, q, v, g and beta are loaded straight into registers.
//   - n_tokens > 1: the per-token dependency chain and the wave's issue of the per-token
//     work bound the scan; a wave owns only 4 rows, so it issues a quarter of what 16
//     rows would need per token, on 4x the waves. The inputs of 16 tokens at a
//     time are staged in LDS (loaded into registers one chunk ahead, converted to f32 and
//     written to the other LDS buffer when the chunk is done), and each token's operands
//     are read from LDS one token ahead, so no global load latency sits on the chain.
#include "ema_common.hpp"

namespace ema {
namespace {

// State rows per wave. The decode step and the scan share the layout, so a scan over T
// tokens gives bit for bit the results of T single-token calls.
constexpr int kStepRows = 4;
constexpr int kScanRows = 4;
constexpr int kChunk = 16;     // tokens per LDS-staged chunk (n_tokens > 1)

struct GdnArgs {
  const void* q;  // [B, T, Hk, Dk]
  const void* k;  // [B, T, Hk, Dk]
  const void* v;  // [B, T, Hv, Dv]
  const float* g;     // [B, T, Hv]
  const float* beta;  // [B, T, Hv]
  float* state;       // [B, Hv, Dv, Dk]
  void* y;            // [B, T, Hv, Dv]
  int T, hk, hv, dv;
};

// Activation element types: 0 bf16, 1 f16, 2 f32.
template <int A>
struct Act;
template <>
struct Act<0> {
  // 4 consecutive elements from p (8-byte aligned)
  static __device__ __forceinline__ f32x4 load4(const void* p) {
    const u32x2 w = *(const u32x2*)p;
    return f32x4{bf16_lo(w[0]), bf16_hi(w[0]), bf16_lo(w[1]), bf16_hi(w[1])};
  }
  static __device__ __forceinline__ float load1(const void* p) { return bf16_to_f32(*(const uint16_t*)p); }
  static __device__ __forceinline__ void store1(void* p, float x) { *(__bf16*)p = (__bf16)x; }
  static constexpr int kSize = 2;
};
template <>
struct Act<1> {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  static __device__ __forceinline__ f32x4 load4(const void* p) {
    const h4 w = *(const h4*)p;
    return f32x4{(float)w[0], (float)w[1], (float)w[2], (float)w[3]};
  }
  static __device__ __forceinline__ float load1(const void* p) { return (float)*(const _Float16*)p; }
  static __device__ __forceinline__ void store1(void* p, float x) { *(_Float16*)p = (_Float16)x; }
  static constexpr int kSize = 2;
};
template <>
struct Act<2> {
  static __device__ __forceinline__ f32x4 load4(const void* p) { return *(const f32x4*)p; }
  static __device__ __forceinline__ float load1(const void* p) { return *(const float*)p; }
  static __device__ __forceinline__ void store1(void* p, float x) { *(float*)p = x; }
  static constexpr int kSize = 4;
};

// Sum over the L lanes that share a row (L = 4 or 16, aligned groups); every lane of the
// group gets the same bits (each stage adds two partial sums in either order, and float
// addition is commutative). DPP: quad_perm [1,0,3,2], quad_perm [2,3,0,1], then for 16
// lanes row_half_mirror and row_mirror.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
template <int L>
__device__ __forceinline__ float row_sum(float x) {
  x += dpp<0xB1>(x);
  x += dpp<0x4E>(x);
  if (L == 16) {
    x += dpp<0x141>(x);
    x += dpp<0x140>(x);
  }
  return x;
}

// One token of the recurrence on this lane's NI x 4 state elements; returns y of the row.
template <int NI, int L>
__device__ __forceinline__ float gdn_token(f32x4 (&s)[NI], const f32x4 (&kk)[NI], const f32x4 (&qq)[NI], float vv,
                                           float gg, float be) {
  // decay and recall: S = g S, kv = S k (four partial sums, one per j)
  f32x4 kv4 = {0.f, 0.f, 0.f, 0.f};
  for (int i = 0; i < NI; ++i)
    for (int j = 0; j < 4; ++j) {
      s[i][j] *= gg;
      kv4[j] = fmaf(s[i][j], kk[i][j], kv4[j]);
    }
  const float kv = row_sum<L>((kv4[0] + kv4[1]) + (kv4[2] + kv4[3]));
  const float delta = (vv - kv) * be;
  // write and read: S += delta k^T, y = S q
  f32x4 y4 = {0.f, 0.f, 0.f, 0.f};
  for (int i = 0; i < NI; ++i)
    for (int j = 0; j < 4; ++j) {
      s[i][j] = fmaf(kk[i][j], delta, s[i][j]);
      y4[j] = fmaf(s[i][j], qq[i][j], y4[j]);
    }
  return row_sum<L>((y4[0] + y4[1]) + (y4[2] + y4[3]));
}

// Lane layout for R state rows per wave: L = 64 / R lanes per row; lane part p holds the
// NI = DK / (4 L) groups of 4 elements dk = 4 p + 4 L i + j, so a 16-byte state load of a
// wave covers 16 L contiguous bytes of each of its R rows.
template <int DK, int R>
struct Layout {
  static constexpr int L = 64 / R;
  static constexpr int NI = DK / (4 * L);
  static __device__ __forceinline__ int elem(int p, int i) { return 4 * p + 4 * L * i; }
};

// n_tokens = 1: everything from global memory.
template <int DK, int A, int R>
__global__ __launch_bounds__(64) void gdn_step_kernel(GdnArgs a) {
  typedef Act<A> AT;
  typedef Layout<DK, R> LY;
  constexpr int NI = LY::NI;
  const int lane = threadIdx.x;
  const int r = lane / LY::L, p = lane % LY::L;
  const int chunks = a.dv / R;
  int64_t id = blockIdx.x;
  const int c = (int)(id % chunks);
  id /= chunks;
  const int h = (int)(id % a.hv);
  const int64_t b = id / a.hv;
  const int kh = h / (a.hv / a.hk);
  const int row = c * R + r;

  float* const st = a.state + ((b * a.hv + h) * a.dv + row) * DK;
  f32x4 s[NI];
  for (int i = 0; i < NI; ++i) s[i] = *(const f32x4*)(st + LY::elem(p, i));
  const char* const qb = (const char*)a.q + (b * a.hk + kh) * DK * AT::kSize;
  const char* const kb = (const char*)a.k + (b * a.hk + kh) * DK * AT::kSize;
  f32x4 kk[NI], qq[NI];
  for (int i = 0; i < NI; ++i) {
    kk[i] = AT::load4(kb + LY::elem(p, i) * AT::kSize);
    qq[i] = AT::load4(qb + LY::elem(p, i) * AT::kSize);
  }
  const float vv = AT::load1((const char*)a.v + ((b * a.hv + h) * a.dv + row) * AT::kSize);
  const float gg = a.g[b * a.hv + h], be = a.beta[b * a.hv + h];
  const float yv = gdn_token<NI, LY::L>(s, kk, qq, vv, gg, be);
  if (p == 0) AT::store1((char*)a.y + ((b * a.hv + h) * a.dv + row) * AT::kSize, yv);
  for (int i = 0; i < NI; ++i) *(f32x4*)(st + LY::elem(p, i)) = s[i];
}

// n_tokens > 1: inputs staged through LDS (k and q converted to f32 once), 16 tokens at a time.
template <int DK, int A, int R>
__global__ __launch_bounds__(64) void gdn_scan_kernel(GdnArgs a) {
  typedef Act<A> AT;
  typedef Layout<DK, R> LY;
  constexpr int NI = LY::NI;
  constexpr int kVecBytes = DK * AT::kSize;             // one token's k (or q) in memory
  constexpr int kPieces = kChunk * kVecBytes / 16 / 64;  // 16-byte pieces per lane per chunk
  constexpr int kElemsPerPiece = 16 / AT::kSize;
  __shared__ __attribute__((aligned(16))) float kq_lds[2][2][kChunk][DK];  // [buf][k|q][token], f32
  __shared__ float vgb_lds[2][kChunk][R + 2];                               // v rows, g, beta

  const int lane = threadIdx.x;
  const int r = lane / LY::L, p = lane % LY::L;
  const int chunks = a.dv / R;
  int64_t id = blockIdx.x;
  const int c = (int)(id % chunks);
  id /= chunks;
  const int h = (int)(id % a.hv);
  const int64_t b = id / a.hv;
  const int kh = h / (a.hv / a.hk);
  const int row = c * R + r;

  float* const st = a.state + ((b * a.hv + h) * a.dv + row) * DK;
  f32x4 s[NI];
  for (int i = 0; i < NI; ++i) s[i] = *(const f32x4*)(st + LY::elem(p, i));

  const char* const qb = (const char*)a.q + (b * a.T * a.hk + kh) * kVecBytes;
  const char* const kb = (const char*)a.k + (b * a.T * a.hk + kh) * kVecBytes;
  const int64_t qk_step = (int64_t)a.hk * kVecBytes;  // bytes between tokens
  const char* const vb = (const char*)a.v + ((b * a.T * a.hv + h) * a.dv + c * R) * AT::kSize;
  const int64_t v_step = (int64_t)a.hv * a.dv * AT::kSize;
  char* const yb = (char*)a.y + ((b * a.T * a.hv + h) * a.dv + row) * AT::kSize;
  const float* const gb = a.g + b * a.T * a.hv + h;
  const float* const bb = a.beta + b * a.T * a.hv + h;

  // chunk staging: registers first (one chunk ahead), then the idle LDS buffer
  constexpr int kVPer = (kChunk * R + 63) / 64;  // v elements per lane per chunk
  u32x4 pk[kPieces], pq[kPieces];
  float pv[kVPer], pgb = 0.f;
  auto fetch = [&](int t0) __attribute__((always_inline)) {
    for (int m = 0; m < kPieces; ++m) {
      const int pid = lane + 64 * m;
      const int tok = pid / (kVecBytes / 16), off = pid % (kVecBytes / 16);
      const bool ok = t0 + tok < a.T;
      pk[m] = ok ? *(const u32x4*)(kb + (t0 + tok) * qk_step + 16 * off) : u32x4{0u, 0u, 0u, 0u};
      pq[m] = ok ? *(const u32x4*)(qb + (t0 + tok) * qk_step + 16 * off) : u32x4{0u, 0u, 0u, 0u};
    }
    for (int m = 0; m < kVPer; ++m) {  // v: 16 tokens x R rows
      const int e = lane + 64 * m, tok = e / R, rr = e % R;
      pv[m] = e < kChunk * R && t0 + tok < a.T ? AT::load1(vb + (t0 + tok) * v_step + rr * AT::kSize) : 0.f;
    }
    const int tok = lane & 15;  // lanes 0-15: g, 16-31: beta
    pgb = lane < 32 && t0 + tok < a.T ? (lane < 16 ? gb : bb)[(int64_t)(t0 + tok) * a.hv] : 0.f;
  };
  auto stage = [&](int buf) __attribute__((always_inline)) {
    for (int m = 0; m < kPieces; ++m) {
      const int pid = lane + 64 * m;
      const int tok = pid / (kVecBytes / 16), off = pid % (kVecBytes / 16);
      float* const kd = &kq_lds[buf][0][tok][kElemsPerPiece * off];
      float* const qd = &kq_lds[buf][1][tok][kElemsPerPiece * off];
      if (AT::kSize == 4) {
        *(u32x4*)kd = pk[m];
        *(u32x4*)qd = pq[m];
      } else {
        for (int e = 0; e < 2; ++e) {
          const u32x2 kw = {pk[m][2 * e], pk[m][2 * e + 1]}, qw = {pq[m][2 * e], pq[m][2 * e + 1]};
          *(f32x4*)(kd + 4 * e) = AT::load4(&kw);
          *(f32x4*)(qd + 4 * e) = AT::load4(&qw);
        }
      }
    }
    for (int m = 0; m < kVPer; ++m) {
      const int e = lane + 64 * m;
      if (e < kChunk * R) vgb_lds[buf][e / R][e % R] = pv[m];
    }
    if (lane < 32) vgb_lds[buf][lane & 15][R + (lane >> 4)] = pgb;
  };
  // this lane's operands of token `tok` of LDS buffer `buf`
  auto operands = [&](int buf, int tok, f32x4* kk, f32x4* qq, float& vv, float& gg, float& be)
      __attribute__((always_inline)) {
    for (int i = 0; i < NI; ++i) {
      kk[i] = *(const f32x4*)&kq_lds[buf][0][tok][LY::elem(p, i)];
      qq[i] = *(const f32x4*)&kq_lds[buf][1][tok][LY::elem(p, i)];
    }
    vv = vgb_lds[buf][tok][r];
    gg = vgb_lds[buf][tok][R];
    be = vgb_lds[buf][tok][R + 1];
  };

  fetch(0);
  stage(0);
  __syncthreads();
  const int nchunks = (a.T + kChunk - 1) / kChunk;
  for (int ch = 0; ch < nchunks; ++ch) {
    const int buf = ch & 1, t0 = ch * kChunk;
    if (ch + 1 < nchunks) fetch(t0 + kChunk);
    const int n = a.T - t0 < kChunk ? a.T - t0 : kChunk;
    f32x4 kk[NI], qq[NI];
    float vv, gg, be;
    operands(buf, 0, kk, qq, vv, gg, be);
    for (int tok = 0; tok < n; ++tok) {
      f32x4 kn[NI], qn[NI];
      float vn = 0.f, gn = 0.f, bn = 0.f;
      if (tok + 1 < n) operands(buf, tok + 1, kn, qn, vn, gn, bn);
      const float yv = gdn_token<NI, LY::L>(s, kk, qq, vv, gg, be);
      if (p == 0) AT::store1(yb + (t0 + tok) * v_step, yv);
      if (tok + 1 < n) {
        for (int i = 0; i < NI; ++i) {
          kk[i] = kn[i];
          qq[i] = qn[i];
        }
        vv = vn;
        gg = gn;
        be = bn;
      }
    }
    if (ch + 1 < nchunks) {
      stage(buf ^ 1);  // the other buffer was last read in the previous chunk
      __syncthreads();
    }
  }
  for (int i = 0; i < NI; ++i) *(f32x4*)(st + LY::elem(p, i)) = s[i];
}

template <int DK, int A>
hipError_t launch_typed(hipStream_t s, const GdnArgs& a, int64_t bh) {
  if (a.T == 1)
    hipLaunchKernelGGL((gdn_step_kernel<DK, A, kStepRows>), dim3((unsigned)(bh * (a.dv / kStepRows))), dim3(64), 0, s, a);
  else
    hipLaunchKernelGGL((gdn_scan_kernel<DK, A, kScanRows>), dim3((unsigned)(bh * (a.dv / kScanRows))), dim3(64), 0, s, a);
  return hipGetLastError();
}

template <int DK>
hipError_t launch_dk(hipStream_t s, int dtype, const GdnArgs& a, int64_t bh) {
  switch (dtype) {
    case EMA_DTYPE_BF16: return launch_typed<DK, 0>(s, a, bh);
    case EMA_DTYPE_F16: return launch_typed<DK, 1>(s, a, bh);
    default: return launch_typed<DK, 2>(s, a, bh);
  }
}

}  // namespace

int32_t launch_gdn_scan(hipStream_t s, const void* q, const void* k, const void* v, const float* g,
                        const float* beta, float* state, void* y, int B, int T, int hk, int hv, int dk,
                        int dv, int dtype) {
  GdnArgs a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.g = g;
  a.beta = beta;
  a.state = state;
  a.y = y;
  a.T = T;
  a.hk = hk;
  a.hv = hv;
  a.dv = dv;
  const int64_t bh = (int64_t)B * hv;
  if (bh * (dv / 4) > 0x7fffffff) return set_error(EMA_ERR_SHAPE, "ema_gdn_scan: grid too large");
  if (dtype == EMA_DTYPE_BF16 && T >= kGdnChunkMinTokens)
    return launch_gdn_chunked(s, q, k, v, g, beta, state, y, B, T, hk, hv, dk, dv);
  const hipError_t e = dk == 64 ? launch_dk<64>(s, dtype, a, bh) : launch_dk<128>(s, dtype, a, bh);
  return check_hip(e, "ema_gdn_scan launch");
}

}  // namespace ema
