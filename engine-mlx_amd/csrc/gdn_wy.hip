// Gated DeltaNet scan in WY form over a workspace, gfx950: a parallel pass forms every
// chunk's matrices, then a sequential pass carries the state through the chunks.
//
// Replaces, for bf16 activations and at least kGdnChunkMinTokens tokens, the sequential
// scan of crates/ops/src/gdn_forward.rs:173-192 (gdn_step, crates/ops/src/gdn.rs:83-150,
// once per token). With the chunk algebra of gdn_chunk.hpp, Delta = (I + A)^-1 W splits
// into a part that does not depend on the state and one that does:
//   Delta = u - w S_0^T,   u = (I + A)^-1 diag(beta) V,   w = (I + A)^-1 diag(beta gamma) K,
// so the state pass per chunk is only
//   v = u - w S^T;   y = gamma (Q S^T) + (decayed Q K^T) v;   S = gamma_31 S + (rho v)^T K
// (rho_t = gamma_31 / gamma_t), and everything else runs in parallel over all chunks.
//
// gdn_wy_prep_kernel: one workgroup (four waves) per (batch, value head, chunk). It stages
// the chunk's K, Q and V, forms the chunk matrices (gdnc::chunk_matrices), solves for w and
// u a 16-column block at a time (gdnc::blocked_solve), and writes the chunk's records:
//   value-head record: -w as A operands of the state pass ([mt][dk step][hi|lo][lane]), the
//     decayed Q K^T operand, the token vectors, then u in accumulator layout
//     ([row block][mt][lane] f32x4);
//   key-head record (written by the first value head of each group): the Q and K^T
//     operand tiles.
// gdn_wy_scan_kernel: one workgroup per (batch, value head, 64 state rows): four waves own
// 16 state rows each, a fifth copies each chunk's records HBM -> LDS by LDS-DMA two chunks
// ahead (three buffers). The state stays f32 in registers across the scan.
//
// A workspace smaller than the whole sequence is used in segments of as many chunks as
// fit: one prep and one state pass per segment, the state passing through HBM between.
#include "gdn_chunk.hpp"

namespace ema {
namespace {

using gdnc::kC;
using gdnc::kPad;
typedef __attribute__((address_space(3))) void lds_void;

// Workspace record layout (bytes).
template <int DK>
struct Rec {
  static constexpr int kW = 0;                           // -w: [mt 2][DK/32][hi|lo][lane] u32x4
  static constexpr int kQM = 2 * (DK / 32) * 2 * 1024;   // decayed Q K^T: [mt][hi|lo][lane]
  static constexpr int kVec = kQM + 4 * 1024;            // gdnc::Out token vectors (1 KB)
  static constexpr int kU = kVec + 1024;                 // u: [Dv/16][mt][lane] f32x4
  static constexpr int kKey = 128 * DK;                  // key-head record: QA then KTA
  static uint64_t value_bytes(int dv) { return (uint64_t)kU + (uint64_t)dv * 128; }
};

struct WyArgs {
  const uint16_t* q;  // [B, T, Hk, DK] bf16
  const uint16_t* k;
  const uint16_t* v;  // [B, T, Hv, Dv] bf16
  const float* g;     // [B, T, Hv]
  const float* beta;  // [B, T, Hv]
  float* state;       // [B, Hv, Dv, DK]
  uint16_t* y;        // [B, T, Hv, Dv] bf16
  uint8_t* ws;        // the segment's records
  uint64_t v_rec;     // bytes of a value-head record
  uint64_t k_base;    // byte offset of the key-head records
  int T, hk, hv, dv;
  int groups;         // state-pass workgroups per (batch, value head): ceil(Dv / 64)
  int c0, nc;         // first chunk of the segment, chunks in it
};

__device__ __forceinline__ uint8_t* value_rec(const WyArgs& a, int64_t b, int h, int c) {
  return a.ws + ((uint64_t)((b * a.hv + h) * a.nc + c)) * a.v_rec;
}
template <int DK>
__device__ __forceinline__ uint8_t* key_rec(const WyArgs& a, int64_t b, int kh, int c) {
  return a.ws + a.k_base + ((uint64_t)((b * a.hk + kh) * a.nc + c)) * Rec<DK>::kKey;
}

// ---------------------------------------------------------------- prep (parallel) pass
template <int DK>
struct PrepLds {
  static constexpr int kScr = 0;                                  // gdnc::Scr
  static constexpr int kIn = gdnc::Scr::kFloats * 4;              // gdnc::In: KA, QA, KTA
  static constexpr int kOut = kIn + gdnc::In<DK>::kBytes;         // gdnc::Out
  static constexpr int kEnd = kOut + gdnc::Out::kBytes;
  // After the chunk matrices, the scratch, KA and QA are dead: that region holds the waves'
  // w transposes (32 tokens x 32 dk each) and, when it fits, the V^T tiles ([Dv/16][lane]).
  static constexpr int kFree = kIn + 2 * gdnc::In<DK>::kKa * 16;
  static constexpr int kWb = 0;
  static constexpr int kWbBytes = 4 * 32 * kPad * 4;
  static __host__ __device__ int vt(int dv) { return kWbBytes + dv * 64 <= kFree ? kWbBytes : kEnd; }
  static __host__ __device__ int bytes(int dv) { return vt(dv) + dv * 64 > kEnd ? vt(dv) + dv * 64 : kEnd; }
};

template <int DK>
__global__ __launch_bounds__(256) void gdn_wy_prep_kernel(WyArgs a) {
  typedef PrepLds<DK> L;
  constexpr int S = DK / 32;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  uint8_t* const in = lds + L::kIn;
  uint8_t* const out = lds + L::kOut;
  float* const scr = (float*)(lds + L::kScr);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g16 = lane & 15, c4 = lane >> 4;
  int64_t id = blockIdx.x;
  const int c = (int)(id % a.nc);
  id /= a.nc;
  const int h = (int)(id % a.hv);
  const int64_t b = id / a.hv;
  const int kh = h / (a.hv / a.hk);
  const int T = a.T, cg = a.c0 + c;
  const int n_valid = T - cg * kC < kC ? T - cg * kC : kC;

  // stage K / Q (lanes 0 .. 2 DK - 1); V (4 tokens x 8 rows per lane and pass) waits in
  // registers until its LDS region is free; g / beta
  gdnc::KqStager<DK> kq;
  if (tid < 2 * DK) {
    kq.init(tid, a.q, a.k, b, kh, a.hk, T);
    kq.fetch(cg);
  }
  constexpr int kVPasses = kGdnWyMaxDv * 8 / 8 / 256;  // 8-row groups x token quads / lanes
  const int vg = a.dv / 8;
  const int64_t v_tok = (int64_t)a.hv * a.dv;
  const uint16_t* const vsrc = a.v + (b * T * a.hv + h) * a.dv;
  u32x4 pv[kVPasses][4];
  #pragma unroll
  for (int p = 0; p < kVPasses; ++p) {
    const int gi = tid + 256 * p, qd = gi / vg, e8 = gi % vg;
    if (gi < 8 * vg)
      #pragma unroll
      for (int kq4 = 0; kq4 < 4; ++kq4) {
        const int t = cg * kC + 4 * qd + kq4;
        pv[p][kq4] = *(const u32x4*)(vsrc + (t < T ? t : T - 1) * v_tok + 8 * e8);
      }
  }
  float gv = 1.f, bv = 0.f;
  {
    const int t = cg * kC + lane;
    const int64_t at = (b * T + (lane < n_valid ? t : T - 1)) * a.hv + h;
    gv = a.g[at];
    bv = a.beta[at];
  }
  if (tid < 2 * DK) kq.stage(cg, in);
  __syncthreads();
  // the key-head record (Q and K^T tiles) from the first value head of each group, before
  // QA's region is reused
  uint8_t* const vrec = value_rec(a, b, h, c);
  if (h % (a.hv / a.hk) == 0) {
    const u32x4* const ks = (const u32x4*)(in + gdnc::In<DK>::kKa * 16);  // QA, then KTA
    u32x4* const kd = (u32x4*)key_rec<DK>(a, b, kh, c);
    for (int e = tid; e < Rec<DK>::kKey / 16; e += 256) kd[e] = ks[e];
  }

  gdnc::chunk_matrices<DK>(wave, lane, n_valid, gv, bv, in, out, scr);
  __syncthreads();
  // V^T tiles: lane (n, c) of row block rb holds rows 16 rb + n of tokens p(c, 0..7)
  u32x2* const vtile = (u32x2*)(lds + L::vt(a.dv));
  #pragma unroll
  for (int p = 0; p < kVPasses; ++p) {
    const int gi = tid + 256 * p, qd = gi / vg, e8 = gi % vg;
    if (gi < 8 * vg) {
      #pragma unroll
      for (int kq4 = 0; kq4 < 4; ++kq4)
        if (cg * kC + 4 * qd + kq4 >= T) pv[p][kq4] = u32x4{0u, 0u, 0u, 0u};
      const int cc = qd & 3, up = qd >> 2;
      #pragma unroll
      for (int x = 0; x < 8; ++x) {
        const int r = 8 * e8 + x, rb = r >> 4, n = r & 15, w = x >> 1, sh = 16 * (x & 1);
        const uint32_t e0 = (pv[p][0][w] >> sh) & 0xffffu, e1 = (pv[p][1][w] >> sh) & 0xffffu;
        const uint32_t e2 = (pv[p][2][w] >> sh) & 0xffffu, e3 = (pv[p][3][w] >> sh) & 0xffffu;
        vtile[(rb * 64 + n + 16 * cc) * 2 + up] = u32x2{e0 | (e1 << 16), e2 | (e3 << 16)};
      }
    }
  }
  __syncthreads();

  // token scales of this lane's B-operand slots: tokens 4c .. 4c+3 and 16 + 4c .. +3
  const float* const vec = (const float*)(out + gdnc::Out::kVec);
  const f32x4 gam0 = *(const f32x4*)&vec[4 * c4], gam1 = *(const f32x4*)&vec[16 + 4 * c4];
  const f32x4 bet0 = *(const f32x4*)&vec[32 + 4 * c4], bet1 = *(const f32x4*)&vec[48 + 4 * c4];
  // X (bf16 tile in B-operand order) scaled per token -> B operand (hi, lo) and the second
  // half in accumulator order
  auto scaled = [&](u32x4 t4, f32x4 s0, f32x4 s1, bf16x8& xh, bf16x8& xl, f32x4& x1) __attribute__((always_inline)) {
    f32x4 x0;
    x0[0] = bf16_lo(t4[0]) * s0[0];
    x0[1] = bf16_hi(t4[0]) * s0[1];
    x0[2] = bf16_lo(t4[1]) * s0[2];
    x0[3] = bf16_hi(t4[1]) * s0[3];
    x1[0] = bf16_lo(t4[2]) * s1[0];
    x1[1] = bf16_hi(t4[2]) * s1[1];
    x1[2] = bf16_lo(t4[3]) * s1[2];
    x1[3] = bf16_hi(t4[3]) * s1[3];
    gdnc::split8(x0, x1, xh, xl);
  };

  // w: dk tiles 2s and 2s+1 per k step s, in the wave that owns s; transposed through the
  // wave's LDS block into A-operand order and stored negated
  const u32x4* const kta = (const u32x4*)(in + 2 * gdnc::In<DK>::kKa * 16);
  float* const wb = (float*)(lds + L::kWb) + wave * 32 * kPad;
  const f32x4 bg0 = bet0 * gam0, bg1 = bet1 * gam1;
  for (int s = wave; s < S; s += 4) {
    #pragma unroll
    for (int half = 0; half < 2; ++half) {
      bf16x8 xh, xl;
      f32x4 x1, r[2];
      scaled(kta[(2 * s + half) * 64 + lane], bg0, bg1, xh, xl, x1);
      gdnc::blocked_solve(out, lane, xh, xl, x1, r);
      #pragma unroll
      for (int mt = 0; mt < 2; ++mt)
        #pragma unroll
        for (int i = 0; i < 4; ++i) wb[(16 * mt + 4 * c4 + i) * kPad + 16 * half + g16] = r[mt][i];
    }
    gdnc::lds_fence();
    u32x4* const wrec = (u32x4*)(vrec + Rec<DK>::kW);
    #pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const float* const row = wb + (16 * mt + g16) * kPad;  // lane (m, c): w[16 mt + m][32 s + p(c, .)]
      const f32x4 lo4 = *(const f32x4*)&row[4 * c4], hi4 = *(const f32x4*)&row[16 + 4 * c4];
      bf16x8 wh, wl;
      gdnc::split8(-lo4, -hi4, wh, wl);
      wrec[((mt * S + s) * 2 + 0) * 64 + lane] = __builtin_bit_cast(u32x4, wh);
      wrec[((mt * S + s) * 2 + 1) * 64 + lane] = __builtin_bit_cast(u32x4, wl);
    }
    gdnc::lds_fence();  // the next step rewrites the block
  }
  // u: one 16-row block per wave and pass, stored in accumulator order
  {
    const u32x4* const vt = (const u32x4*)(lds + L::vt(a.dv));
    f32x4* const urec = (f32x4*)(vrec + Rec<DK>::kU);
    for (int rb = wave; rb < a.dv / 16; rb += 4) {
      bf16x8 xh, xl;
      f32x4 x1, r[2];
      scaled(vt[rb * 64 + lane], bet0, bet1, xh, xl, x1);
      gdnc::blocked_solve(out, lane, xh, xl, x1, r);
      urec[(rb * 2 + 0) * 64 + lane] = r[0];
      urec[(rb * 2 + 1) * 64 + lane] = r[1];
    }
  }
  // decayed Q K^T operand and token vectors
  {
    const u32x4* const src = (const u32x4*)(out + gdnc::Out::kQM * 16);  // QM, then the vectors
    u32x4* const dst = (u32x4*)(vrec + Rec<DK>::kQM);
    for (int e = tid; e < 256 + 32; e += 256) dst[e] = src[e];
  }
}

// ---------------------------------------------------------------- state (sequential) pass
// 16 bytes per lane from buffer offset voff straight into LDS at lds_addr + 16 lane
// (buffer_load_dwordx4 ... lds, LDS base through M0). Issued as asm, untracked by the
// compiler: the loop waits for it with an explicit vmcnt(0) before the barrier.
__device__ __forceinline__ void dma16(u32x4 rsrc, uint32_t voff, uint32_t lds_addr) {
  // s_nop 0: the DMA reads M0 no earlier than one wait state after the SALU write, a wait
  // the compiler inserts only for the LDS-DMAs it emits itself. (Its SGPR operands need five
  // after a VALU write; check_hazards.py fails the build if the compiler places one closer.)
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory", "m0");
}
__device__ __forceinline__ u32x4 rsrc_of(const void* base, uint32_t bytes) {
  const uint64_t addr = (uint64_t)base;
  return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)addr),
               (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(addr >> 32) & 0xffffu),
               (uint32_t)__builtin_amdgcn_readfirstlane(bytes), 0x00020000u};
}

// s_waitcnt vmcnt(N), expcnt and lgkmcnt left at their maxima (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0xF70);
}

constexpr int kScanWaves = 4;  // 16 state rows each, plus one loader wave
template <int DK>
struct ScanLds {
  static constexpr int kV = Rec<DK>::kU;        // the value-head record up to u
  static constexpr int kK = kV;                 // then the key-head record
  static constexpr int kU = kK + Rec<DK>::kKey; // then u of the workgroup's four row blocks
  static constexpr int kBuf = kU + kScanWaves * 2048;
  static constexpr int kBytes = 3 * kBuf;
  static constexpr int kDma = (kBuf) / 1024;    // 1 KB steps per chunk
};

template <int DK>
__global__ __launch_bounds__(64 * (kScanWaves + 1)) void gdn_wy_scan_kernel(WyArgs a) {
  typedef ScanLds<DK> L;
  constexpr int S = DK / 32, NT = DK / 16;
  static_assert(L::kV % 1024 == 0 && Rec<DK>::kKey % 1024 == 0, "records move in 1 KB DMA steps");
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g16 = lane & 15, c4 = lane >> 4;
  int64_t id = blockIdx.x;
  const int rg = (int)(id % a.groups);
  id /= a.groups;
  const int h = (int)(id % a.hv);
  const int64_t b = id / a.hv;
  const int kh = h / (a.hv / a.hk);
  const int T = a.T;
  const int row0 = (rg * kScanWaves + wave) * 16;
  const bool rows = wave < kScanWaves && row0 < a.dv;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_void*)lds;

  // The loader wave copies chunk c's records HBM -> LDS buffer c % 3 (kDma 1 KB steps: the
  // value-head record up to u, the key-head record, u of this workgroup's row blocks; row
  // blocks past Dv read zeros). It is the only wave that issues these loads, so its vmcnt
  // counts them alone and it can wait for one chunk while the next is in flight.
  auto dma_chunk = [&](int c) __attribute__((always_inline)) {
    const uint32_t buf = lds0 + (uint32_t)((c % 3) * L::kBuf);
    const uint8_t* const vr = value_rec(a, b, h, c);
    const u32x4 rv = rsrc_of(vr, (uint32_t)L::kV);
    const u32x4 rk = rsrc_of(key_rec<DK>(a, b, kh, c), (uint32_t)Rec<DK>::kKey);
    const int blocks = a.dv / 16 - rg * kScanWaves;
    const u32x4 ru = rsrc_of(vr + Rec<DK>::kU + (uint64_t)rg * kScanWaves * 2048,
                             (uint32_t)(blocks < kScanWaves ? blocks : kScanWaves) * 2048u);
    #pragma unroll
    for (int i = 0; i < L::kV / 1024; ++i) dma16(rv, 1024u * i + 16u * lane, buf + 1024u * i);
    #pragma unroll
    for (int i = 0; i < Rec<DK>::kKey / 1024; ++i) dma16(rk, 1024u * i + 16u * lane, buf + L::kK + 1024u * i);
    #pragma unroll
    for (int i = 0; i < 2 * kScanWaves; ++i) dma16(ru, 1024u * i + 16u * lane, buf + L::kU + 1024u * i);
  };

  // The roles run separate loops with the same barriers (one before the first chunk, one
  // after each), so that no register of one role is carried through the other's path.
  if (wave == kScanWaves) {
    dma_chunk(0);
    if (a.nc > 1) {
      dma_chunk(1);
      wait_vmcnt<L::kDma>();
    } else {
      wait_vmcnt<0>();
    }
    __syncthreads();
    for (int c = 0; c < a.nc; ++c) {
      // chunk c + 2 goes in flight; chunk c + 1 has landed before the barrier
      if (c + 2 < a.nc) {
        dma_chunk(c + 2);
        wait_vmcnt<L::kDma>();
      } else {
        wait_vmcnt<0>();
      }
      __syncthreads();
    }
    return;
  }

  float* const st_ptr = a.state + ((b * a.hv + h) * a.dv + row0 + g16) * DK + 4 * c4;  // + 16 t
  // y of token t0 + j at y_wave + (t0 + j) hv dv (32-bit offsets within a chunk: hv dv T < 2^31)
  uint16_t* const y_wave = a.y + (b * T * a.hv + h) * a.dv + row0;
  const int y_tok = a.hv * a.dv;
  f32x4 st[NT];
  if (rows)
    #pragma unroll
    for (int t = 0; t < NT; ++t) st[t] = *(const f32x4*)(st_ptr + 16 * t);
  wait_vmem();
  __syncthreads();
  for (int c = 0; c < a.nc; ++c) {
    if (rows) {
      const uint8_t* const buf = lds + (c % 3) * L::kBuf;
      const u32x4* const W = (const u32x4*)(buf + Rec<DK>::kW);
      const u32x4* const QM = (const u32x4*)(buf + Rec<DK>::kQM);
      const float* const vec = (const float*)(buf + Rec<DK>::kVec);
      const u32x4* const QA = (const u32x4*)(buf + L::kK);
      const u32x4* const KT = QA + gdnc::In<DK>::kKa;
      const f32x4* const U = (const f32x4*)(buf + L::kU) + wave * 128;
      // v = u - w S^T and Q S^T; A = -w / Q tiles, B = the state (hi + lo)
      u32x4 w4[2][S][2], qa4[2][S];
      #pragma unroll
      for (int mt = 0; mt < 2; ++mt)
        #pragma unroll
        for (int s = 0; s < S; ++s) {
          w4[mt][s][0] = W[((mt * S + s) * 2 + 0) * 64 + lane];
          w4[mt][s][1] = W[((mt * S + s) * 2 + 1) * 64 + lane];
          qa4[mt][s] = QA[(mt * S + s) * 64 + lane];
        }
      f32x4 v[2] = {U[lane], U[64 + lane]}, qs[2];
      #pragma unroll
      for (int mt = 0; mt < 2; ++mt) qs[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
      #pragma unroll
      for (int s = 0; s < S; ++s) {
        bf16x8 sh, sl;
        gdnc::split8(st[2 * s], st[2 * s + 1], sh, sl);
        #pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const bf16x8 wh = as_bf16x8(w4[mt][s][0]), wl = as_bf16x8(w4[mt][s][1]);
          const bf16x8 qa = as_bf16x8(qa4[mt][s]);
          v[mt] = mfma16(wl, sh, v[mt]);
          v[mt] = mfma16(wh, sl, v[mt]);
          v[mt] = mfma16(wh, sh, v[mt]);
          qs[mt] = mfma16(qa, sl, qs[mt]);
          qs[mt] = mfma16(qa, sh, qs[mt]);
        }
      }
      f32x4 gam[2], rho[2];
      #pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        gam[mt] = *(const f32x4*)&vec[16 * mt + 4 * c4];
        rho[mt] = *(const f32x4*)&vec[64 + 16 * mt + 4 * c4];
      }
      const float gc = vec[96];
      // S = gamma_31 S + (rho v)^T K: A = K^T tiles, B = rho v (hi + lo)
      bf16x8 th, tl;
      gdnc::split8(rho[0] * v[0], rho[1] * v[1], th, tl);
      #pragma unroll
      for (int t = 0; t < NT; ++t) {
        const bf16x8 kt = as_bf16x8(KT[t * 64 + lane]);
        st[t] = st[t] * gc;
        st[t] = mfma16(kt, tl, st[t]);
        st[t] = mfma16(kt, th, st[t]);
      }
      // y = gamma S q + (decayed Q K^T) v, off the state's chain
      bf16x8 vh, vl;
      gdnc::split8(v[0], v[1], vh, vl);
      const int t0 = (a.c0 + c) * kC;
      // buffer over this chunk's real tokens: stores to padding tokens fall outside and are dropped
      const int n_tok = T - t0 < kC ? T - t0 : kC;
      const __amdgpu_buffer_rsrc_t y_rsrc = __builtin_amdgcn_make_buffer_rsrc(
          y_wave + (int64_t)t0 * y_tok, (short)0, n_tok * y_tok * 2, 0x00020000);
      #pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const bf16x8 qh = as_bf16x8(QM[(2 * mt) * 64 + lane]), ql = as_bf16x8(QM[(2 * mt + 1) * 64 + lane]);
        f32x4 yv = gam[mt] * qs[mt];
        yv = mfma16(ql, vh, yv);
        yv = mfma16(qh, vl, yv);
        yv = mfma16(qh, vh, yv);
        const int j0 = 16 * mt + 4 * c4;
        #pragma unroll
        for (int i = 0; i < 4; ++i)
          __builtin_amdgcn_raw_buffer_store_b16((unsigned short)f32_to_bf16_bits(yv[i]), y_rsrc,
                                                ((j0 + i) * y_tok + g16) * 2, 0, 0);
      }
        }
    __syncthreads();
  }
  if (rows)
    #pragma unroll
    for (int t = 0; t < NT; ++t) *(f32x4*)(st_ptr + 16 * t) = st[t];
}

template <int DK>
int32_t launch_wy_dk(hipStream_t s, WyArgs a, int nch, int nc_max, int B) {
  static std::atomic<uint64_t> lds_set[2];
  const int prep_lds = PrepLds<DK>::bytes(a.dv);
  int32_t rc = allow_lds_once((const void*)gdn_wy_prep_kernel<DK>, PrepLds<DK>::bytes(512), &lds_set[0],
                              "ema_gdn_scan_ws: LDS attribute");
  if (rc) return rc;
  rc = allow_lds_once((const void*)gdn_wy_scan_kernel<DK>, ScanLds<DK>::kBytes, &lds_set[1],
                      "ema_gdn_scan_ws: LDS attribute");
  if (rc) return rc;
  for (int c0 = 0; c0 < nch; c0 += nc_max) {
    a.c0 = c0;
    a.nc = nch - c0 < nc_max ? nch - c0 : nc_max;
    a.k_base = (uint64_t)B * a.hv * a.nc * a.v_rec;
    hipLaunchKernelGGL(gdn_wy_prep_kernel<DK>, dim3((unsigned)((int64_t)B * a.hv * a.nc)), dim3(256), prep_lds, s, a);
    rc = check_hip(hipGetLastError(), "ema_gdn_scan_ws prep launch");
    if (rc) return rc;
    hipLaunchKernelGGL(gdn_wy_scan_kernel<DK>, dim3((unsigned)((int64_t)B * a.hv * a.groups)),
                       dim3(64 * (kScanWaves + 1)), ScanLds<DK>::kBytes, s, a);
    rc = check_hip(hipGetLastError(), "ema_gdn_scan_ws state launch");
    if (rc) return rc;
  }
  return EMA_OK;
}

}  // namespace

uint64_t gdn_wy_chunk_bytes(int B, int hk, int hv, int dk, int dv) {
  const uint64_t v_rec = dk == 64 ? Rec<64>::value_bytes(dv) : Rec<128>::value_bytes(dv);
  const uint64_t k_rec = dk == 64 ? Rec<64>::kKey : Rec<128>::kKey;
  return (uint64_t)B * ((uint64_t)hv * v_rec + (uint64_t)hk * k_rec);
}

int32_t launch_gdn_wy(hipStream_t s, const void* q, const void* k, const void* v, const float* g, const float* beta,
                      float* state, void* y, int B, int T, int hk, int hv, int dk, int dv, void* ws,
                      uint64_t ws_bytes) {
  const int nch = (T + kC - 1) / kC;
  const uint64_t per_chunk = gdn_wy_chunk_bytes(B, hk, hv, dk, dv);
  const uint64_t fit = ws_bytes / per_chunk;
  if (fit < 1)
    return set_error(EMA_ERR_INVALID_ARG, "ema_gdn_scan_ws: workspace of %llu bytes holds no chunk (%llu per chunk)",
                     (unsigned long long)ws_bytes, (unsigned long long)per_chunk);
  const int64_t grid_prep = (int64_t)B * hv * (fit < (uint64_t)nch ? (int64_t)fit : nch);
  if (grid_prep > 0x7fffffff) return set_error(EMA_ERR_SHAPE, "ema_gdn_scan_ws: grid too large");
  WyArgs a;
  a.q = (const uint16_t*)q;
  a.k = (const uint16_t*)k;
  a.v = (const uint16_t*)v;
  a.g = g;
  a.beta = beta;
  a.state = state;
  a.y = (uint16_t*)y;
  a.ws = (uint8_t*)ws;
  a.v_rec = dk == 64 ? Rec<64>::value_bytes(dv) : Rec<128>::value_bytes(dv);
  a.k_base = 0;
  a.T = T;
  a.hk = hk;
  a.hv = hv;
  a.dv = dv;
  a.groups = (dv + 63) / 64;
  a.c0 = 0;
  a.nc = 0;
  const int nc_max = fit < (uint64_t)nch ? (int)fit : nch;
  return dk == 64 ? launch_wy_dk<64>(s, a, nch, nc_max, B) : launch_wy_dk<128>(s, a, nch, nc_max, B);
}

}  // namespace ema
