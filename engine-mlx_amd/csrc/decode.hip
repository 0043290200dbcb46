// GQA split-K decode attention (flash-decoding) over the static KV cache, gfx950.
//
// Replaces MlxCtx::sdpa_masked (crates/mlx-ffi/src/ops/real/transform.rs:8-29)
// as called by the static decode step (crates/serve/src/compiled.rs:163,
// crates/serve/src/decode_eager.rs:140): softmax(scale * q K^T + mask) V with
// the additive static mask of crates/serve/src/engine_ext.rs:237-260 expressed
// as a valid length per sequence. Unlike the reference, which reads the whole
// capacity (docs/benchmarks.md:24-28), only the valid rows are read.
//
// Work split. The valid rows of every (sequence b, kv head kh) pair form a
// "segment" of ceil(len_b / 32) tiles of 32 positions. All segments are laid
// end to end and the flattened tile range is cut into W equal slices, one per
// wave ("worker"), so ragged lengths cost no load imbalance. A worker walks its
// slice; each maximal run inside one segment is a "piece" whose online-softmax
// state (m, l, unnormalised o) goes to partial slot (w + segment index), which
// is unique because w and the segment index never both stay constant from one
// piece to the next. A segment covered by a single worker is normalised and
// written directly; the others are combined by decode_merge_kernel
// (log-sum-exp merge).
//
// Per 32-position tile a wave issues 16 MFMA 16x16x32 (bf16 in, f32 acc):
//   S^T[pos, g] = K[pos, :] . Q^T[:, g]    A = K rows (straight from HBM),
//                                           B = the G query heads of the kv head
//                                           (zero-padded to 16 columns)
//   O^T[d, g] += V^T[d, pos] P^T[pos, g]    A = V^T (8x8 bf16 transpose in
//                                           registers), B = P^T (the S^T
//                                           accumulators after exp, unmoved)
// The row order inside the tile is chosen so that the lane that holds a score
// also holds it in the B-operand slot of P^T, so P never crosses lanes; the
// only cross-lane traffic per tile is the max over the four 16-lane groups.
// All softmax state is f32; P is rounded to bf16 for the PV MFMA.
#include <cstdlib>

#include "ema_common.hpp"

namespace ema {
namespace {

constexpr int kD = 128;
constexpr int kTile = 32;
constexpr int kWaves = 4;       // waves per workgroup, each an independent worker
constexpr int kMaxB = 1024;     // batch rows held in the LDS prefix table
constexpr int kPieceStride = kD + 4;  // floats per (piece, head): m, l, pad, pad, o[D]
constexpr int kHeaderInts = kMaxB + 8;

struct DecodeArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* len;
  uint16_t* out;
  int32_t* hdr;  // workspace header: tile prefix per batch row, then total
  float* part;   // partial slots
  int64_t sb, sh, sp;
  float qk_scale;  // scale * log2(e): scores live in the log2 domain
  int B, Hq, Hkv, G, cap, W;
};

__device__ __forceinline__ int64_t worker_of(int64_t t, int64_t total, int W) {
  return ((t + 1) * (int64_t)W - 1) / total;
}
__device__ __forceinline__ int64_t worker_begin(int64_t w, int64_t total, int W) {
  return w * total / W;
}

__device__ __forceinline__ int clamp_len(int L, int cap) { return L < 0 ? 0 : (L > cap ? cap : L); }

// Tile prefix over batch rows (tiles of all kv heads of rows < b), computed by
// the whole workgroup. pre[B] is the total tile count.
__device__ void build_prefix(const DecodeArgs& a, int32_t* pre) {
  __shared__ int32_t part[256];
  const int tid = threadIdx.x;
  const int chunk = (a.B + 255) / 256;
  const int b0 = tid * chunk;
  int32_t local = 0;
  for (int i = 0; i < chunk; ++i) {
    const int b = b0 + i;
    if (b < a.B) local += ((clamp_len(a.len[b], a.cap) + kTile - 1) / kTile) * a.Hkv;
  }
  part[tid] = local;
  __syncthreads();
  for (int d = 1; d < 256; d <<= 1) {
    int32_t v = tid >= d ? part[tid - d] : 0;
    __syncthreads();
    part[tid] += v;
    __syncthreads();
  }
  int32_t run = part[tid] - local;  // exclusive
  for (int i = 0; i < chunk; ++i) {
    const int b = b0 + i;
    if (b < a.B) {
      pre[b] = run;
      run += ((clamp_len(a.len[b], a.cap) + kTile - 1) / kTile) * a.Hkv;
    }
  }
  if (tid == 255) pre[a.B] = part[255];
  __syncthreads();
}

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *(const u32x4*)p; }

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_kernel(DecodeArgs a) {
  __shared__ int32_t pre[kMaxB + 1];
  build_prefix(a, pre);
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i <= a.B; i += blockDim.x) a.hdr[i] = pre[i];

  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (w >= a.W) return;
  const int64_t total = pre[a.B];
  if (total == 0) return;
  int64_t t = worker_begin(w, total, a.W);
  const int64_t t_end = worker_begin(w + 1, total, a.W);

  const int g = lane & 15;  // query head inside the kv group (B-operand column)
  const int c = lane >> 4;  // 16-lane group
  const int m = lane & 15;  // A-operand row
  // K row feeding A-operand row m of MFMA set r: position 8*(m/4) + 4r + m%4,
  // so that S^T rows 4c..4c+3 of set r are positions 8c + 4r + i.
  const int krow0 = 8 * (m >> 2) + (m & 3);

  while (t < t_end) {
    // locate the segment containing tile t (uniform across the wave)
    int lo = 0, hi = a.B;  // largest b with pre[b] <= t
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (pre[mid] <= t) lo = mid; else hi = mid;
    }
    const int b = lo;
    const int L = clamp_len(a.len[b], a.cap);
    const int nb = (L + kTile - 1) / kTile;
    const int64_t rel = t - pre[b];
    const int kh = (int)(rel / nb);
    const int tile0 = (int)(rel % nb);
    const int64_t seg_first = pre[b] + (int64_t)kh * nb;
    const int64_t seg_end = seg_first + nb;
    const int64_t piece_end = t_end < seg_end ? t_end : seg_end;
    const int tile1 = tile0 + (int)(piece_end - t);

    const uint16_t* Kb = a.k + (int64_t)b * a.sb + (int64_t)kh * a.sh;
    const uint16_t* Vb = a.v + (int64_t)b * a.sb + (int64_t)kh * a.sh;

    // B operand: Q^T, k index of step s <-> dims 8*(4s + c) .. +7
    bf16x8 qop[4];
    {
      // columns g >= G are zero padding; their (clamped, in-bounds) loads are discarded
      const int gc = g < a.G ? g : 0;
      const uint16_t* qh = a.q + ((int64_t)b * a.Hq + (int64_t)kh * a.G + gc) * kD;
      for (int s = 0; s < 4; ++s) {
        const u32x4 z = {0u, 0u, 0u, 0u};
        const u32x4 v = ld16(qh + 8 * (4 * s + c));
        qop[s] = as_bf16x8(g < a.G ? v : z);
      }
    }

    float m_run = -INFINITY, l_run = 0.f;
    f32x4 o[8];
    for (int j = 0; j < 8; ++j) o[j] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 kc[2][4], vc[8], kn[2][4], vn[8];
    auto load_tile = [&](int tile, u32x4 (&kr)[2][4], u32x4 (&vr)[8]) {
      const int p0 = tile * kTile;
      for (int r = 0; r < 2; ++r) {
        int p = p0 + krow0 + 4 * r;
        p = p < L ? p : L - 1;
        const uint16_t* row = Kb + (int64_t)p * a.sp;
        for (int s = 0; s < 4; ++s) kr[r][s] = ld16(row + 8 * (4 * s + c));
      }
      for (int kk = 0; kk < 8; ++kk) {
        int p = p0 + 8 * c + kk;
        p = p < L ? p : L - 1;
        vr[kk] = ld16(Vb + (int64_t)p * a.sp + 8 * m);
      }
    };

    load_tile(tile0, kc, vc);
    for (int tile = tile0; tile < tile1; ++tile) {
      if (tile + 1 < tile1) load_tile(tile + 1, kn, vn);
      const int p0 = tile * kTile;

      f32x4 sc[2];
      for (int r = 0; r < 2; ++r) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s < 4; ++s) acc = mfma16(as_bf16x8(kc[r][s]), qop[s], acc);
        sc[r] = acc;
      }
      float x[8];
      float mx = -INFINITY;
      for (int r = 0; r < 2; ++r)
        for (int i = 0; i < 4; ++i) {
          const int pos = p0 + 8 * c + 4 * r + i;
          const float v = pos < L ? sc[r][i] * a.qk_scale : -INFINITY;
          x[4 * r + i] = v;
          mx = fmaxf(mx, v);
        }
      mx = wave_max_xor(mx, 16);
      mx = wave_max_xor(mx, 32);
      const float m_new = fmaxf(m_run, mx);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      float psum = 0.f;
      for (int e = 0; e < 8; ++e) {
        x[e] = __builtin_amdgcn_exp2f(x[e] - m_new);
        psum += x[e];
      }
      l_run = l_run * alpha + psum;
      m_run = m_new;
      for (int j = 0; j < 8; ++j) o[j] *= alpha;

      // P^T B operand: k = 4r + i <-> position p0 + 8c + k
      u32x4 pw;
      pw[0] = pack_bf16x2(x[0], x[1]);
      pw[1] = pack_bf16x2(x[2], x[3]);
      pw[2] = pack_bf16x2(x[4], x[5]);
      pw[3] = pack_bf16x2(x[6], x[7]);
      const bf16x8 pop = as_bf16x8(pw);
      // V^T A operand for dim residue j: row m <-> dim 8m + j, k <-> position p0 + 8c + k
      for (int j = 0; j < 8; ++j) {
        u32x4 av;
        for (int tt = 0; tt < 4; ++tt) {
          const uint32_t lo = vc[2 * tt][j >> 1];
          const uint32_t hi = vc[2 * tt + 1][j >> 1];
          av[tt] = (j & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
        }
        o[j] = mfma16(as_bf16x8(av), pop, o[j]);
      }
      if (tile + 1 < tile1) {
        for (int r = 0; r < 2; ++r)
          for (int s = 0; s < 4; ++s) kc[r][s] = kn[r][s];
        for (int kk = 0; kk < 8; ++kk) vc[kk] = vn[kk];
      }
    }

    float l_tot = l_run + __shfl_xor(l_run, 16, 64);
    l_tot += __shfl_xor(l_tot, 32, 64);

    // lane (g, c) holds O[g][32c + 8i + j] = o[j][i]
    const bool single = worker_of(seg_first, total, a.W) == worker_of(seg_end - 1, total, a.W);
    if (g < a.G) {
      if (single) {
        const float inv = 1.0f / l_tot;
        uint16_t* dst = a.out + ((int64_t)b * a.Hq + (int64_t)kh * a.G + g) * kD + 32 * c;
        for (int i = 0; i < 4; ++i) {
          u32x4 wv;
          for (int jj = 0; jj < 4; ++jj) wv[jj] = pack_bf16x2(o[2 * jj][i] * inv, o[2 * jj + 1][i] * inv);
          *(u32x4*)(dst + 8 * i) = wv;
        }
      } else {
        const int64_t piece = (int64_t)w + (int64_t)b * a.Hkv + kh;
        float* P = a.part + (piece * a.G + g) * kPieceStride;
        if (c == 0) {
          P[0] = m_run;
          P[1] = l_tot;
        }
        for (int i = 0; i < 4; ++i) {
          float* dst = P + 4 + 32 * c + 8 * i;
          *(f32x4*)dst = f32x4{o[0][i], o[1][i], o[2][i], o[3][i]};
          *(f32x4*)(dst + 4) = f32x4{o[4][i], o[5][i], o[6][i], o[7][i]};
        }
      }
    }
    t = piece_end;
  }
}

// One wave per (segment, query head): log-sum-exp merge of the pieces of
// segments that span several workers; zero output for empty segments.
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t sg = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  const int S = a.B * a.Hkv;
  if (sg >= (int64_t)S * a.G) return;
  const int s = (int)(sg / a.G);
  const int g = (int)(sg % a.G);
  const int b = s / a.Hkv;
  const int kh = s % a.Hkv;
  uint32_t* dst = (uint32_t*)(a.out + ((int64_t)b * a.Hq + (int64_t)kh * a.G + g) * kD) + lane;
  const int L = clamp_len(a.len[b], a.cap);
  if (L == 0) {
    *dst = 0u;
    return;
  }
  const int nb = (L + kTile - 1) / kTile;
  const int64_t total = a.hdr[a.B];
  const int64_t seg_first = a.hdr[b] + (int64_t)kh * nb;
  const int64_t seg_end = seg_first + nb;
  const int64_t w0 = worker_of(seg_first, total, a.W);
  const int64_t w1 = worker_of(seg_end - 1, total, a.W);
  if (w0 == w1) return;  // written by the decode kernel
  float M = -INFINITY;
  for (int64_t w = w0; w <= w1; ++w) {
    if (worker_begin(w, total, a.W) == worker_begin(w + 1, total, a.W)) continue;
    const float* P = a.part + ((w + s) * a.G + g) * kPieceStride;
    M = fmaxf(M, P[0]);
  }
  float lsum = 0.f, o0 = 0.f, o1 = 0.f;
  for (int64_t w = w0; w <= w1; ++w) {
    if (worker_begin(w, total, a.W) == worker_begin(w + 1, total, a.W)) continue;
    const float* P = a.part + ((w + s) * a.G + g) * kPieceStride;
    const float sc = __builtin_amdgcn_exp2f(P[0] - M);
    lsum += sc * P[1];
    o0 += sc * P[4 + 2 * lane];
    o1 += sc * P[5 + 2 * lane];
  }
  const float inv = 1.0f / lsum;
  *dst = pack_bf16x2(o0 * inv, o1 * inv);
}

int max_workers() {
  static int w = [] {
    const char* e = getenv("EMA_DECODE_WORKERS");
    int v = e ? atoi(e) : 0;
    return v > 0 ? v : 2048;
  }();
  return w;
}

}  // namespace

DecodePlan plan_decode(int B, int Hq, int Hkv, int D, int max_len) {
  DecodePlan p;
  const int64_t tiles = (int64_t)B * Hkv * ((max_len + kTile - 1) / kTile);
  int64_t w = tiles < max_workers() ? tiles : max_workers();
  if (w < 1) w = 1;
  p.workers = (int)w;
  p.segments = B * Hkv;
  const int G = Hkv > 0 ? Hq / Hkv : 1;
  p.part_bytes = (uint64_t)(p.workers + p.segments) * G * kPieceStride * sizeof(float);
  return p;
}

uint64_t decode_header_bytes() { return (uint64_t)kHeaderInts * sizeof(int32_t); }

int32_t launch_decode(hipStream_t s, const void* q, const ema_kvcache_desc& c, const int32_t* len,
                      int Hq, float scale, void* out, void* ws, const DecodePlan& plan) {
  if (c.head_dim != kD)
    return set_error(EMA_ERR_UNSUPPORTED, "ema_decode_attention: head_dim %d not supported (128)", c.head_dim);
  if (c.batch > kMaxB)
    return set_error(EMA_ERR_UNSUPPORTED, "ema_decode_attention: batch %d exceeds %d", c.batch, kMaxB);
  const int G = Hq / c.n_kv_heads;
  if (G > 16)
    return set_error(EMA_ERR_UNSUPPORTED, "ema_decode_attention: %d query heads per kv head exceeds 16", G);
  DecodeArgs a;
  a.q = (const uint16_t*)q;
  a.k = (const uint16_t*)c.k;
  a.v = (const uint16_t*)c.v;
  a.len = len;
  a.out = (uint16_t*)out;
  a.hdr = (int32_t*)ws;
  a.part = (float*)((char*)ws + decode_header_bytes());
  a.sb = c.stride_batch;
  a.sh = c.stride_head;
  a.sp = c.stride_pos;
  a.qk_scale = scale * kLog2e;
  a.B = c.batch;
  a.Hq = Hq;
  a.Hkv = c.n_kv_heads;
  a.G = G;
  a.cap = c.capacity;
  a.W = plan.workers;
  const int blocks = (plan.workers + kWaves - 1) / kWaves;
  hipLaunchKernelGGL(decode_kernel, dim3(blocks), dim3(kWaves * 64), 0, s, a);
  int32_t rc = check_hip(hipGetLastError(), "ema_decode_attention launch");
  if (rc) return rc;
  const int64_t merge_waves = (int64_t)plan.segments * G;
  hipLaunchKernelGGL(decode_merge_kernel, dim3((unsigned)((merge_waves + kWaves - 1) / kWaves)),
                     dim3(kWaves * 64), 0, s, a);
  return check_hip(hipGetLastError(), "ema_decode_attention merge launch");
}

}  // namespace ema
