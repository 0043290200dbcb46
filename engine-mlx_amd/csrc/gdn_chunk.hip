// Gated DeltaNet scan in chunkwise form on the bf16 matrix cores, one kernel, gfx950.
//
// Replaces, for bf16 activations and at least kGdnChunkMinTokens tokens, the sequential
// scan of crates/ops/src/gdn_forward.rs:173-192, which applies gdn_step
// (crates/ops/src/gdn.rs:83-150) once per token. The chunk algebra, operand layouts and
// precision scheme are in gdn_chunk.hpp. This kernel needs no workspace; with one,
// gdn_wy.hip forms every chunk's matrices in parallel first and is faster.
//
// Work split: one workgroup per (batch, value head, 64 state rows), eight waves:
//   - four row waves own 16 state rows each (the state, transposed, in MFMA accumulator
//     layout: lane (g, c) holds S[row g][16 t + 4 c + i] in tile t) and run the chunk's
//     products;
//   - four matrix waves form the chunk-shared quantities one chunk ahead
//     (gdnc::chunk_matrices) and stage the K and Q tiles of the chunk two ahead from HBM
//     into LDS. The row waves finish the inverse as a blocked solve
//     (gdnc::blocked_solve).
// K, Q inputs are triple-buffered in LDS and the chunk matrices double-buffered, so one
// workgroup barrier per chunk orders everything.
#include "gdn_chunk.hpp"

namespace ema {
namespace {

using gdnc::kC;
using gdnc::kMatWaves;
constexpr int kRowWaves = 4;  // 16 state rows each
constexpr int kThreadsC = 64 * (kRowWaves + kMatWaves);

template <int DK>
struct ChunkLds {
  static constexpr int kInBytes = gdnc::In<DK>::kBytes;
  static constexpr int kOutBytes = gdnc::Out::kBytes;
  static constexpr int kOut0 = 3 * kInBytes;
  static constexpr int kScr0 = kOut0 + 2 * kOutBytes;
  static constexpr int kBytes = kScr0 + gdnc::Scr::kFloats * 4;
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

  // ---- K / Q staging by the matrix waves' lanes 0 .. 2 DK - 1 ----
  const int mw = wave - kRowWaves;  // matrix wave index (negative on row waves)
  const int ltid = tid - 64 * kRowWaves;
  const bool loader = mw >= 0 && ltid < 2 * DK;  // 2 DK <= 64 kMatWaves
  gdnc::KqStager<DK> kq;
  kq.init(loader ? ltid : 0, a.q, a.k, b, kh, a.hk, T);

  // ---- chunk-matrix wave ----
  const int64_t gb_base = b * T * a.hv + h;  // g / beta of token t at gb_base + t * hv
  auto load_gb = [&](int ch, float& gv, float& bv) __attribute__((always_inline)) {
    const int t = ch * kC + lane;
    const int64_t at = gb_base + (int64_t)(lane < kC && t < T ? t : T - 1) * a.hv;
    gv = a.g[at];
    bv = a.beta[at];
  };
  auto chunk_matrices = [&](int ch, float gv, float bv) __attribute__((always_inline)) {
    const int n_valid = T - ch * kC < kC ? T - ch * kC : kC;
    gdnc::chunk_matrices<DK>(mw, lane, n_valid, gv, bv, lds + (ch % 3) * L::kInBytes,
                             lds + L::kOut0 + (ch & 1) * L::kOutBytes, scr);
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
    const u32x4* const QA = KA + gdnc::In<DK>::kKa;
    const u32x4* const KT = KA + 2 * gdnc::In<DK>::kKa;
    const u32x4* const OP = (const u32x4*)out;
    const float* const vec = (const float*)(out + gdnc::Out::kVec);
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
      gdnc::split8(st[2 * s], st[2 * s + 1], sh, sl);
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
    // Delta = (I + A)^-1 W
    bf16x8 xh, xl;
    gdnc::split8(w[0], w[1], xh, xl);
    f32x4 u[2];
    gdnc::blocked_solve(out, lane, xh, xl, w[1], u);
    // y = gamma S_0 q + (decayed Q K^T) Delta
    bf16x8 uh, ul;
    gdnc::split8(u[0], u[1], uh, ul);
    #pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const bf16x8 qh = as_bf16x8(OP[gdnc::Out::kQM + (2 * mt) * 64 + lane]);
      const bf16x8 ql = as_bf16x8(OP[gdnc::Out::kQM + (2 * mt + 1) * 64 + lane]);
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
    gdnc::split8(rho[0] * u[0], rho[1] * u[1], th, tl);
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
    kq.fetch(0);
    kq.stage(0, lds);
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
    if (ahead) kq.fetch(i + 2);
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
    if (ahead) kq.stage(i + 2, lds + ((i + 2) % 3) * L::kInBytes);
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
