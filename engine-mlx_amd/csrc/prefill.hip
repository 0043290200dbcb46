// Causal / chunked-prefill flash attention over the static KV cache, gfx950.
//
// Replaces MlxCtx::sdpa(..., causal=true) (crates/mlx-ffi/src/ops/real/blas.rs:82-101)
// as called by the prefill (crates/serve/src/forward_qwen3.rs:150) and by
// attend_and_project (crates/ops/src/attention.rs:162-177, via
// crates/attention/src/gqa.rs:100-106). MLX "causal" aligns the query block
// to the end of the key range: query i of a chunk that starts at cache
// position q_off sees keys j <= q_off + i.
//
// Tiling: a workgroup of 4 waves owns 128 query rows of one head (32 per
// wave) and streams 64-key blocks of K and V through double-buffered LDS.
// Both contractions run on MFMA 32x32x16 (bf16 in, f32 accumulate), in the
// transposed form that keeps the softmax lane-local:
//   S^T[key, q] = K[key, :] . Q^T[:, q]   A = K rows (ds_read_b128), B = Q^T in registers
//   O^T[d, q]  += V^T[d, key] P^T[key, q] A = V^T via ds_read_b64_tr_b16 (transposing
//                                          LDS read), B = P^T (the S^T accumulators
//                                          after exp, unmoved)
// Each lane therefore owns one query row's scores, running max, row sum and
// 64 output accumulators; the row max needs one xor-32 exchange per block.
//
// Two workgroups share a CU (2 waves per SIMD). The MFMA sections run at raised
// wave priority (s_setprio 1) and the softmax at normal priority, so when both
// waves of a SIMD are ready the arbiter issues the matrix work first and the
// other wave's softmax VALU fills the gaps (ping-pong between the two waves).
#include "ema_common.hpp"

namespace ema {
namespace {

constexpr int kD = 128;
constexpr int kBM = 128;          // query rows per workgroup
constexpr int kBN = 64;           // keys per block
constexpr int kKStride = kD + 8;  // LDS row stride (elements) of the K tile: conflict-free b128 reads
constexpr int kVStride = kD + 32; // LDS row stride of the V tile: conflict-free transposed reads
constexpr int kKTile = kBN * kKStride;
constexpr int kVTile = kBN * kVStride;
constexpr int kLdsBytes = 2 * (kKTile + kVTile) * 2;
constexpr int kXcds = 8;          // MI355X: 8 XCDs, workgroups dispatched round-robin

struct PrefillArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* q_off;
  uint16_t* out;
  int64_t sb, sh, sp;
  float qk_scale;  // scale * log2(e)
  int B, Hq, Hkv, G, T, cap, nqb;
  uint32_t flags;
};

typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *(const u32x4*)p; }

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_kernel(PrefillArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  uint16_t* const Ks = lds;               // K tiles: buffer i at Ks + i * kKTile
  uint16_t* const Vs = lds + 2 * kKTile;  // V tiles: buffer i at Vs + i * kVTile

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  // Grid mapping. Workgroups are dispatched round-robin over the 8 XCDs (x % 8), each
  // with its own L2. When the (batch, kv head) groups divide evenly over the XCDs, all
  // query heads of a group run on the group's XCD, so its K/V stream is read from HBM
  // once and served from that L2 to every workgroup that attends over it. Inside an XCD
  // (or over the whole grid otherwise) work items are ranked heaviest first (a later
  // query block sees more keys) and the second half of the local index range takes the
  // ranks in reverse, so the two workgroups that share a CU (local indices i and
  // i + n/2 when they are resident together) carry complementary causal work.
  const int groups = a.B * a.Hkv;
  const bool by_xcd = groups % kXcds == 0 && gridDim.x % kXcds == 0;
  const int64_t x = blockIdx.x;
  const int64_t n_local = by_xcd ? gridDim.x / kXcds : gridDim.x;
  const int64_t li = by_xcd ? x / kXcds : x;
  const int64_t half = (n_local + 1) / 2;
  const int64_t rank = li < half ? li : n_local - 1 - (li - half);
  const int groups_local = by_xcd ? groups / kXcds : groups;
  const int per_qb = groups_local * a.G;
  const int qb = a.nqb - 1 - (int)(rank / per_qb);
  const int rest = (int)(rank % per_qb);
  const int grp_id = by_xcd ? (rest / a.G) * kXcds + (int)(x % kXcds) : rest / a.G;
  const int b = grp_id / a.Hkv;
  const int h = (grp_id % a.Hkv) * a.G + rest % a.G;
  const int kh = grp_id % a.Hkv;

  int q_off = a.q_off[b];
  q_off = q_off < 0 ? 0 : q_off;
  int kv_len = q_off + a.T;
  kv_len = kv_len > a.cap ? a.cap : kv_len;
  const bool causal = a.flags & EMA_PREFILL_CAUSAL;
  int kv_begin = (a.flags & EMA_PREFILL_CHUNK_ONLY) ? q_off : 0;
  kv_begin = kv_begin > kv_len ? kv_len : kv_begin;

  const int row0 = qb * kBM;                      // first query row of the workgroup
  int wg_end = kv_len;
  if (causal) {
    const int lim = q_off + row0 + kBM;           // last row sees keys < lim
    wg_end = lim < wg_end ? lim : wg_end;
  }
  const int blk_begin = kv_begin / kBN;
  const int blk_end = (wg_end + kBN - 1) / kBN;

  // this lane's query row
  const int qr = row0 + 32 * wave + (lane & 31);
  const int qr_c = qr < a.T ? qr : a.T - 1;
  const int q_abs = q_off + qr;                   // causal limit: key <= q_abs
  const int wave_first_abs = q_off + row0 + 32 * wave;
  const int wave_last_abs = wave_first_abs + 31;
  const int hh = lane >> 5;                       // which half of the k slots

  // Q^T as B operand: step s covers dims 16s + 8*hh .. +7
  bf16x8 qop[8];
  {
    const uint16_t* qp = a.q + (((int64_t)b * a.Hq + h) * a.T + qr_c) * kD + 8 * hh;
    for (int s = 0; s < 8; ++s) qop[s] = as_bf16x8(ld16(qp + 16 * s));
    wait_vmem();
  }

  const char* Kg = (const char*)(a.k + (int64_t)b * a.sb + (int64_t)kh * a.sh);
  const char* Vg = (const char*)(a.v + (int64_t)b * a.sb + (int64_t)kh * a.sh);
  const int64_t blk_bytes = (int64_t)kBN * a.sp * 2;

  // global -> register staging: the thread owns rows rr + 16i (i < 4) of a block at
  // 16-byte column cc, for K and for V
  const int rr = tid >> 4, cc = (tid & 15) * 8;
  uint32_t toff[4];
  for (int i = 0; i < 4; ++i) toff[i] = (uint32_t)(((int64_t)(rr + 16 * i) * a.sp + cc) * 2);
  u32x4 kst[4], vst[4];
  auto gload = [&](int blk) {
    const int base = blk * kBN;
    if (base + kBN <= kv_len) {  // whole block valid: uniform block base + 32-bit offsets
      const char* kp = Kg + (int64_t)blk * blk_bytes;
      const char* vp = Vg + (int64_t)blk * blk_bytes;
      for (int i = 0; i < 4; ++i) {
        kst[i] = *(const u32x4*)(kp + toff[i]);
        vst[i] = *(const u32x4*)(vp + toff[i]);
      }
    } else {  // tail block: clamp rows to the last valid one (masked later)
      for (int i = 0; i < 4; ++i) {
        int r = base + rr + 16 * i;
        r = r < kv_len ? r : kv_len - 1;
        kst[i] = *(const u32x4*)(Kg + ((int64_t)r * a.sp + cc) * 2);
        vst[i] = *(const u32x4*)(Vg + ((int64_t)r * a.sp + cc) * 2);
      }
    }
  };
  auto sstore = [&](int buf) {
    for (int i = 0; i < 4; ++i) {
      *(u32x4*)(Ks + buf * kKTile + (rr + 16 * i) * kKStride + cc) = kst[i];
      *(u32x4*)(Vs + buf * kVTile + (rr + 16 * i) * kVStride + cc) = vst[i];
    }
  };

  float m_run = -INFINITY, l_run = 0.f;
  f32x16 o[4];
  for (int dt = 0; dt < 4; ++dt)
    for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;

  if (blk_begin < blk_end) {
    gload(blk_begin);
    sstore(0);
  }
  __syncthreads();

  // transposed-read addressing (per 16-lane group)
  const int grp = lane >> 4, s16 = lane & 15;
  const int tr_row = 4 * (grp >> 1) + (s16 >> 2);     // + 16*st_half + 8u + 32*kt
  const int tr_col = 16 * (grp & 1) + 4 * (s16 & 3);  // + 32*dt

  for (int blk = blk_begin; blk < blk_end; ++blk) {
    const int buf = (blk - blk_begin) & 1;
    const bool more = blk + 1 < blk_end;
    if (more) gload(blk + 1);
    const int kbase = blk * kBN;
    const bool active = kbase <= wave_last_abs || !causal;
    if (active) {
      const uint16_t* Kt = Ks + buf * kKTile;
      const uint16_t* Vt = Vs + buf * kVTile;
      // two independent accumulation chains (sub-tiles kt = 0, 1), interleaved
      f32x16 sc[2];
      for (int kt = 0; kt < 2; ++kt)
        for (int i = 0; i < 16; ++i) sc[kt][i] = 0.f;
      const uint16_t* kp = Kt + (lane & 31) * kKStride + 8 * hh;
      __builtin_amdgcn_s_setprio(1);
      for (int s = 0; s < 8; ++s)
        for (int kt = 0; kt < 2; ++kt)
          sc[kt] = mfma32(as_bf16x8(*(const u32x4*)(kp + kt * 32 * kKStride + 16 * s)), qop[s], sc[kt]);
      __builtin_amdgcn_s_setprio(0);
      // mask on raw scores; key of slot i in sub-tile kt: kbase + 32kt + (i%4) + 8(i/4) + 4hh
      const bool need_mask = kbase < kv_begin || kbase + kBN > kv_len ||
                             (causal && kbase + kBN - 1 > wave_first_abs);
      if (need_mask) {
        for (int kt = 0; kt < 2; ++kt)
          for (int i = 0; i < 16; ++i) {
            const int key = kbase + 32 * kt + (i & 3) + 8 * (i >> 2) + 4 * hh;
            const bool ok = key >= kv_begin && key < kv_len && (!causal || key <= q_abs);
            sc[kt][i] = ok ? sc[kt][i] : -INFINITY;
          }
      }
      float mx = -INFINITY;
      for (int kt = 0; kt < 2; ++kt)
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sc[kt][i]);
      mx = wave_max_xor(mx, 32) * a.qk_scale;  // scale > 0: max commutes with it
      // Lazy rescale: the running max (log2 domain) moves only when a row's max
      // grows by more than 8, so p = 2^(s - m) stays <= 256 and the O/l rescale
      // is skipped for most blocks. Any m gives the same normalised result.
      if (__any(mx > m_run + 8.f)) {
        const float m_new = mx > m_run + 8.f ? mx : m_run;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // m_run = -inf -> 0
        l_run *= alpha;
        for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
        m_run = m_new;
      }
      // rows with nothing visible yet keep m = -inf: use 0 as the base (all p = 0)
      const float m_use = m_run == -INFINITY ? 0.f : m_run;
      float psum = 0.f;
      for (int kt = 0; kt < 2; ++kt)
        for (int i = 0; i < 16; ++i) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[kt][i], a.qk_scale, -m_use));
          sc[kt][i] = p;
          psum += p;
        }
      l_run += psum;

      // PV: step st covers S^T slots 8*(st&1) .. +7 of sub-tile st>>1
      __builtin_amdgcn_s_setprio(1);
      for (int st = 0; st < 4; ++st) {
        const int kt = st >> 1, q2 = st & 1;
        u32x4 pw;
        for (int e = 0; e < 4; ++e)
          pw[e] = pack_bf16x2(sc[kt][8 * q2 + 2 * e], sc[kt][8 * q2 + 2 * e + 1]);
        const bf16x8 pop = as_bf16x8(pw);
        const int rbase = 32 * kt + 16 * q2 + tr_row;
        for (int dt = 0; dt < 4; ++dt) {
          const uint16_t* p0 = Vt + rbase * kVStride + 32 * dt + tr_col;
          const uint16_t* p1 = p0 + 8 * kVStride;
          const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p0);
          const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p1);
          typedef short s16x8 __attribute__((ext_vector_type(8)));
          const s16x8 av = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          o[dt] = mfma32(__builtin_bit_cast(bf16x8, av), pop, o[dt]);
        }
      }
    }
    __builtin_amdgcn_s_setprio(0);
    if (more) sstore(buf ^ 1);
    __syncthreads();
  }

  float l_tot = l_run + __shfl_xor(l_run, 32, 64);
  if (qr >= a.T) return;
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  // lane holds O[q][32dt + (i%4) + 8(i/4) + 4hh]
  uint16_t* dst = a.out + (((int64_t)b * a.T + qr) * a.Hq + h) * kD + 4 * hh;
  for (int dt = 0; dt < 4; ++dt)
    for (int qq = 0; qq < 4; ++qq) {
      u32x2 wv;
      wv[0] = pack_bf16x2(o[dt][4 * qq] * inv, o[dt][4 * qq + 1] * inv);
      wv[1] = pack_bf16x2(o[dt][4 * qq + 2] * inv, o[dt][4 * qq + 3] * inv);
      *(u32x2*)(dst + 32 * dt + 8 * qq) = wv;
    }
}

}  // namespace

int32_t launch_prefill(hipStream_t s, const void* q, const ema_kvcache_desc& c,
                       const int32_t* q_off, int T, int Hq, float scale, uint32_t flags,
                       void* out) {
  if (c.head_dim != kD)
    return set_error(EMA_ERR_UNSUPPORTED, "ema_prefill_attention: head_dim %d not supported (128)", c.head_dim);
  static bool attr_set = false;
  if (!attr_set) {
    int32_t rc = check_hip(hipFuncSetAttribute((const void*)prefill_kernel,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes),
                           "ema_prefill_attention: LDS attribute");
    if (rc) return rc;
    attr_set = true;
  }
  PrefillArgs a;
  a.q = (const uint16_t*)q;
  a.k = (const uint16_t*)c.k;
  a.v = (const uint16_t*)c.v;
  a.q_off = q_off;
  a.out = (uint16_t*)out;
  a.sb = c.stride_batch;
  a.sh = c.stride_head;
  a.sp = c.stride_pos;
  a.qk_scale = scale * kLog2e;
  a.B = c.batch;
  a.Hq = Hq;
  a.Hkv = c.n_kv_heads;
  a.G = Hq / c.n_kv_heads;
  a.T = T;
  a.cap = c.capacity;
  a.nqb = (T + kBM - 1) / kBM;
  a.flags = flags;
  const int64_t blocks = (int64_t)a.nqb * Hq * c.batch;
  if (blocks > 0x7fffffff) return set_error(EMA_ERR_SHAPE, "ema_prefill_attention: grid too large");
  hipLaunchKernelGGL(prefill_kernel, dim3((unsigned)blocks), dim3(256), kLdsBytes, s, a);
  return check_hip(hipGetLastError(), "ema_prefill_attention launch");
}

}  // namespace ema
