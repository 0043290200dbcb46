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
// workgroup, so ragged lengths cost no load imbalance. W is taken on the device
// from the actual tile count (one tile per wave at least, at most the host plan's
// workers, which size the workspace for the upper bound of the lengths), so short
// sequences in a long cache are not cut into more pieces than they have waves. A workgroup walks its
// slice; each maximal run inside one segment is a "piece". The four waves of
// the workgroup take the piece's tiles in turn, each keeping its own
// online-softmax state, and combine the four states through LDS at the end of
// the piece. A segment covered by a single workgroup is normalised and written
// directly; otherwise the combined state (m, l, unnormalised o) goes to
// partial slot (w + segment index) -- unique because w and the segment index
// never both stay constant from one piece to the next -- and the workgroup
// counts itself in at the segment's arrival counter in the workspace. The last of
// the segment's workgroups to arrive folds its slots by log-sum-exp and writes the
// output, so one launch does the whole call. The partials cross XCDs (each with its
// own L2) as device-coherent stores and loads (see part_store); the merger returns the
// counter to zero for the next call.
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
//
// FP8 E4M3FN cache: a lane loads the same row pieces as 8 codes (8 bytes) instead of
// 8 bf16 values, plus the row's two block exponents, and turns them into the same bf16
// operands just before use (code value times 2^exp is exact in bf16). Half the bytes,
// identical arithmetic after the decode step. With an unquantised RoPE tail (n_rot = 64:
// a row is 64 codes, then dims 64..127 as bf16) the pieces of dims >= 64 are loaded as
// bf16 and used as they are.
#include "ema_common.hpp"
#include "ema_schedule.hpp"

namespace ema {
namespace {

constexpr int kD = 128;
constexpr int kTile = kSplitTile;
constexpr int kWaves = kSplitWaves;  // waves per workgroup, each an independent worker
constexpr int kMaxB = 1024;     // batch rows held in the LDS prefix table
constexpr int kPieceStride = kD + 4;  // floats per (piece, head): m, l, pad, pad, o[D]

struct DecodeArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* len;
  uint16_t* out;
  int32_t* cnt;  // workspace counters: arrivals per (sequence, kv head) segment, then the grid's
  int32_t* hdr;  // workspace: tile prefix per batch row (pre[0..B]), for decode_merge_kernel
  float* part;   // partial slots
  int64_t sb, sh, sp;
  float qk_scale;  // scale * log2(e): scores live in the log2 domain
  int B, Hq, Hkv, G, cap, W;
  // fused decode step only: the pre-attention inputs; lengths are off[b] + 1
  const uint16_t* qkv;  // [B, (Hq + 2*Hkv) * D]
  const uint16_t* qw;
  const uint16_t* kw;
  const int32_t* off;
  int32_t* adv;  // EMA_STEP_ADVANCE: the offsets, advanced by the grid's last workgroup (else null)
  float eps, log2_theta;
  uint32_t flags;
  int fused;
  int rot;  // rotating cache: the fused step's new row is row off % cap
  int inline_merge;  // merge split segments in this kernel (else decode_merge_kernel does)
  int narrow;        // the split's products w * total stay below 2^31: 32-bit arithmetic
  // fp8 cache: block exponents [B, Hkv, cap, 2] (k, v then hold E4M3FN codes)
  const int8_t* kexp;
  const int8_t* vexp;
  // int4 cache: (group 0, group 1) bf16 scale and bias pairs [B, Hkv, cap] (k, v then hold
  // the packed codes; strides count 4-bit elements)
  uint32_t* ks;
  uint32_t* kb;
  uint32_t* vs;
  uint32_t* vb;
};

// The split's slice bounds, in 32-bit arithmetic when the host has bounded every product
// w * total below 2^31 (a.narrow)
__device__ __forceinline__ int64_t worker_of(const DecodeArgs& a, int64_t t, int64_t total, int W) {
  return a.narrow ? split_worker_of32(t, total, W) : split_worker_of(t, total, W);
}
__device__ __forceinline__ int active_workers(int64_t total, int W) { return split_active_workers(total, W, kWaves); }
__device__ __forceinline__ int64_t worker_begin(const DecodeArgs& a, int64_t w, int64_t total, int W) {
  return a.narrow ? split_begin32(w, total, W) : split_begin(w, total, W);
}

__device__ __forceinline__ int clamp_len(int L, int cap) { return L < 0 ? 0 : (L > cap ? cap : L); }

// Valid positions of sequence b: the given length, or offset + 1 in the fused step
// (the new token is written at the offset before attention reads it).
__device__ __forceinline__ int seq_len(const DecodeArgs& a, int b) {
  return clamp_len(a.fused ? a.off[b] + 1 : a.len[b], a.cap);
}

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
    if (b < a.B) local += ((seq_len(a, b) + kTile - 1) / kTile) * a.Hkv;
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
      run += ((seq_len(a, b) + kTile - 1) / kTile) * a.Hkv;
    }
  }
  if (tid == 255) pre[a.B] = part[255];
  __syncthreads();
}

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) { return *(const u32x4*)p; }
// K/V rows are read exactly once per call: non-temporal (streaming) loads keep them
// from displacing reusable lines (measured: ~10% faster on the batch-32 and 32k shapes).
__device__ __forceinline__ u32x4 ld16_stream(const uint16_t* p) {
  return __builtin_nontemporal_load((const u32x4*)p);
}
__device__ __forceinline__ u32x2 ld8_stream(const uint8_t* p) { return __builtin_nontemporal_load((const u32x2*)p); }


// Quantisation of one 64-value block held one value per lane (the fused step's new row):
// exponent ceil(log2(amax / 448)), amax = max(1e-4, max |x|) over the wave (logarithm in
// double, rounded to f32: an f32 log2 rounded to nearest), code = E4M3FN(x * 2^-e) with
// +-448 saturation (NaN -> +448) and -0 stored as +0. Returns the code; *xq gets the
// decoded bf16 bits.
__device__ __forceinline__ uint32_t fp8_quant_lane(float x, int* e_out, uint16_t* xq) {
  float amax = fmaxf(fabsf(x), 1.0e-4f);
  for (int mm = 32; mm >= 1; mm >>= 1) amax = fmaxf(amax, __shfl_xor(amax, mm, 64));
  const int e = (int)ceilf((float)log2((double)(amax / 448.0f)));
  float y = x * ldexpf(1.0f, -e);
  y = y != y ? 448.0f : fminf(fmaxf(y, -448.0f), 448.0f);
  const uint32_t code = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(y + 0.0f, 0.0f, 0, false) & 0xffu;
  const float sc = __uint_as_float((uint32_t)(e + 127) << 23);
  *xq = (uint16_t)__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)code, sc, false));
  *e_out = e;
  return code;
}

// ---- int4 cache ----
// The codes enter the MFMAs exactly as bf16 values 128 + code (0x4300 | code), and the
// affine parameters are applied around them:
//   scores: S[p, g] = sum_grp s_grp[p] acc_grp[p, g] + (b_grp[p] - 128 s_grp[p]) Qsum_grp[g]
//     with acc_grp the MFMA sum over the group's 64 dims of (128 + code) q and Qsum_grp the
//     sum of the (bf16) q over those dims;
//   output: O[d, g] = sum_p (128 + code[p, d]) P'_grp[p, g] + sum_p (P[p, g] b_grp[p] - 128
//     P'_grp[p, g]) with P'_grp = bf16(P s_grp) as the B operand.
// Both use the exact affine values s * code + b (no bf16 rounding of K and V).
//
// (x & m) | c in one v_and_or_b32. gfx950's VOP3 takes no literal, so the empty asm
// statements hand the constants over as VGPR values (set once per kernel) and the
// compiler selects the fused instruction. The instruction itself is left to the compiler:
// its result feeds MFMA operands, and the hazard recognizer inserts the wait states a VALU
// write needs before an MFMA reads it only for instructions it emits itself, not for an
// inline-asm VALU instruction.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t c) {
  asm("" : "+v"(m));
  asm("" : "+v"(c));
  return (x & m) | c;
}
// The 8 codes of a word (value i at bits 4i) as the bf16 A-operand registers of one MFMA
// step, k-slot order (0, 4), (1, 5), (2, 6), (3, 7).
__device__ __forceinline__ bf16x8 i4_kop(uint32_t w) {
  u32x4 r;
  r[0] = and_or(w, 0x000F000Fu, 0x43004300u);
  r[1] = and_or(w >> 4, 0x000F000Fu, 0x43004300u);
  r[2] = and_or(w >> 8, 0x000F000Fu, 0x43004300u);
  r[3] = and_or(w >> 12, 0x000F000Fu, 0x43004300u);
  return as_bf16x8(r);
}
// bf16 pairs (0, 1), (2, 3), (4, 5), (6, 7) -> (0, 4), (1, 5), (2, 6), (3, 7): the q operand in
// the k-slot order of i4_kop
__device__ __forceinline__ u32x4 i4_qperm(u32x4 w) {
  u32x4 r;
  r[0] = (w[0] & 0xffffu) | (w[2] << 16);
  r[1] = (w[0] >> 16) | (w[2] & 0xffff0000u);
  r[2] = (w[1] & 0xffffu) | (w[3] << 16);
  r[3] = (w[1] >> 16) | (w[3] & 0xffff0000u);
  return r;
}

// One int4 tile of a wave in registers: the K words of the lane's two rows krow0 + 4r
// (steps 2i, 2i+1), the V words (dims 8m .. 8m+7) of its 8 positions 8c + kk, and the
// parameter words it uses. Positions are relative to the tile's first.
struct I4Tile {
  u32x2 k[2][2];   // [r][i]: row krow0 + 4r, dims 64i + 16c .. +15
  uint32_t v[8];   // position 8c + kk
  u32x4 ks[2];     // K (scale 0, scale 1) pairs of positions 8c + 4r + i
  uint32_t kb[2];  // K (bias 0, bias 1) pair of row krow0 + 4r
  u32x4 vs[2];     // V scale pairs of positions 8c + 4h + e
  u32x4 vb[2];     // V bias pairs of positions 8c + 4h + e
};

__device__ __forceinline__ float fmax_asm(float x, float y) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(x), "v"(y));
  return r;
}
// Maximum over the lanes l, l ^ 16, l ^ 32, l ^ 48 (the four 16-lane rows), by the row
// swaps of v_permlane16_swap / v_permlane32_swap instead of LDS permutes: after a swap of
// a value with itself, one result holds the even rows' values in both rows of each pair
// and the other the odd rows'.
__device__ __forceinline__ float max_over_rows(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = fmax_asm(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmax_asm(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

typedef __attribute__((address_space(3))) void lds_void;

// Raw buffer resource over `bytes` bytes at `base` (loads past them return zero), as four
// scalar words for the asm of the LDS loads.
__device__ __forceinline__ u32x4 rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t addr = (uint64_t)base;
  return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)addr),
               (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(addr >> 32) & 0xffffu),
               (uint32_t)__builtin_amdgcn_readfirstlane(bytes), 0x00020000u};
}
// 16 bytes per lane from buffer offset voff + soff straight into LDS at lds + 16 lane
// (buffer_load_dwordx4 ... lds, non-temporal; the LDS base goes through M0). Issued as asm,
// untracked by the compiler: the int4 tile loop orders it with explicit vmcnt waits.
__device__ __forceinline__ void dma16(u32x4 rs, uint32_t voff, uint32_t soff, uint32_t lds) {
  // s_nop 0: the DMA reads M0 no earlier than one wait state after the SALU write, a wait
  // the compiler inserts only for the LDS-DMAs it emits itself. (Its SGPR operands need five
  // after a VALU write; check_hazards.py fails the build if the compiler places one closer.)
  asm volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen nt lds"
               :
               : "v"(voff), "s"(rs), "s"(__builtin_amdgcn_readfirstlane(soff)), "s"(__builtin_amdgcn_readfirstlane(lds))
               : "memory", "m0");
}
// s_waitcnt vmcnt(N), also a compiler memory barrier (the LDS reads after it stay after it)
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// LDS used to combine the four waves' states at the end of a piece.
struct Combine {
  float m[kWaves][16];
  float l[kWaves][16];
  int last;  // this workgroup arrived last (at a segment's counter or the grid's)
};
// Each wave's share of the workgroup's LDS: its [16][kD] f32 output state at the end of a
// piece; for the int4 cache, before that, the ring of tile slots its loads stream into.
// int4 slot: K rows (32 x 64 B), V rows (32 x 64 B), then the K scale, K bias, V scale and
// V bias words of the tile's 32 positions (128 B each).
constexpr int kI4Slot = 2 * kTile * 64 + 4 * kTile * 4;
constexpr int kI4Slots = 3;  // the tile in use and two in flight
constexpr int kI4SlotK = 0, kI4SlotV = kTile * 64, kI4SlotKs = 2 * kTile * 64, kI4SlotKb = kI4SlotKs + 4 * kTile,
              kI4SlotVs = kI4SlotKb + 4 * kTile, kI4SlotVb = kI4SlotVs + 4 * kTile;
constexpr int kStateLds = 16 * kD * 4;
// bf16 slot: the tile's K rows (32 x 256 B) and V rows (32 x 256 B)
constexpr int kBfSlot = 2 * kTile * kD * 2;
// fp8 slot: K codes (32 x 128 B), V codes (32 x 128 B), then the K and V exponent pairs of
// the tile's 32 rows (64 B each); two slots per wave (the tile in use and the next)
constexpr int kF8SlotV = kTile * kD, kF8SlotKe = 2 * kTile * kD, kF8SlotVe = kF8SlotKe + 2 * kTile;
constexpr int kF8Slot = kF8SlotVe + 2 * kTile;
template <bool kFp8, bool kI4, bool kDma>
constexpr int wave_lds_bytes() {
  return kI4 ? (kI4Slots * kI4Slot > kStateLds ? kI4Slots * kI4Slot : kStateLds)
             : kDma ? (kFp8 ? 2 * kF8Slot : kBfSlot) : kStateLds;
}
// The slots' layouts (dec_krow, bf_swz, f8_swz, f8_vrow) are in ema_schedule.hpp, with the
// CPU checks of their gathers and reads.

// Partial states cross XCDs, each with its own L2, without cache maintenance: they are
// written and read with device-coherent (agent-scope) stores and loads, which go past the
// XCD's L2 (sc1), and a writer's stores have completed before its workgroup counts in.
__device__ __forceinline__ void part_store(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float part_load(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Arrival at counter i: every wave waits for its stores to complete (vmcnt(0): the
// partial states have reached the device-coherent level), then thread 0 counts the
// workgroup in. The workgroup that brings the count to n is the last of the n and
// returns the counter to zero for the next call. Returns (to every thread) whether this
// workgroup was last. The counter's index goes through a VGPR so that the atomic is a
// vector one.
__device__ bool arrive_last(const DecodeArgs& a, int64_t i, int n, Combine& cmb) {
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();
  if (threadIdx.x == 0) {
    int idx = (int)i;
    asm volatile("" : "+v"(idx));
    int32_t* c = a.cnt + idx;
    const int old = __hip_atomic_fetch_add(c, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = old == n - 1;
    if (last) __hip_atomic_store(c, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    cmb.last = last;
  }
  __syncthreads();
  return cmb.last != 0;
}

// Head dims lane group c feeds to the QK MFMA of step s (8 of them, d .. d+7). bf16
// cache: d = 8(4s + c), so that the four lanes of a K row read 64 contiguous bytes per
// step. fp8 cache: d = 64(s/2) + 16c + 8(s%2), so that a lane's two steps s = 2i, 2i+1
// are one 16-byte load and the four lanes of a row read 64 contiguous bytes per load.
// Any order works as long as q uses the same one; in both, dims d and d + 64 (a RoPE
// pair) sit in one lane as steps s and s + 2.
template <bool kFp8>
__device__ __forceinline__ int kdim(int s, int c) {
  return kFp8 ? 64 * (s >> 1) + 16 * c + 8 * (s & 1) : 8 * (4 * s + c);
}

// RMSNorm + split-half RoPE of the head vector whose dims kdim(s, c) + j (s < 4, j < 8)
// this lane holds in x[8s + j] (c = lane / 16; the four lanes of one head together
// hold all 128 dims).
// wv[s] holds the norm weights of the same dims. Same arithmetic as the pre-attention
// kernel: f32 statistics, normalised value rounded to bf16 before the weight multiply;
// cs_tab[i] = (cos, sin) of the angle pos * 2^(-(i/64) log2 theta) formed in f32.
template <bool kFp8>
__device__ __forceinline__ void norm_rope(const DecodeArgs& a, float (&x)[32], const u32x4 (&wv)[4],
                                          const float2* cs_tab) {
  const int c = (threadIdx.x & 63) >> 4;
  if (!(a.flags & (EMA_PRE_NO_NORM | EMA_PRE_NO_Q_NORM))) {
    float ss = 0.f;
    for (int e = 0; e < 32; ++e) ss += x[e] * x[e];
    ss += __shfl_xor(ss, 16, 64);
    ss += __shfl_xor(ss, 32, 64);
    const float inv = 1.0f / sqrtf(ss / (float)kD + a.eps);
    for (int s2 = 0; s2 < 4; ++s2) {
      for (int j = 0; j < 8; ++j) {
        const float n = bf16_to_f32((uint16_t)f32_to_bf16_bits(x[8 * s2 + j] * inv));
        const float wj = (j & 1) ? bf16_hi(wv[s2][j >> 1]) : bf16_lo(wv[s2][j >> 1]);
        x[8 * s2 + j] = bf16_to_f32((uint16_t)f32_to_bf16_bits(n * wj));
      }
    }
  }
  if (!(a.flags & EMA_PRE_NO_ROPE)) {
    for (int s2 = 0; s2 < 2; ++s2)
      for (int j = 0; j < 8; ++j) {
        const int i = kdim<kFp8>(s2, c) + j;  // < 64; partner i + 64 is slot s2 + 2
        const float cs = cs_tab[i].x, sn = cs_tab[i].y;
        const float x1 = x[8 * s2 + j], x2 = x[8 * (s2 + 2) + j];
        x[8 * s2 + j] = x1 * cs - x2 * sn;
        x[8 * (s2 + 2) + j] = x1 * sn + x2 * cs;
      }
  }
}

// bf16 pairs of the 4 chunks a lane holds -> f32 x[8s + j]
__device__ __forceinline__ void unpack32(const u32x4 (&r)[4], float (&x)[32]) {
  for (int s = 0; s < 4; ++s)
    for (int j = 0; j < 8; ++j) x[8 * s + j] = (j & 1) ? bf16_hi(r[s][j >> 1]) : bf16_lo(r[s][j >> 1]);
}

// Log-sum-exp merge of segment s = (b, kh), whose pieces are the partial states of
// workers w0..w1, one thread per (head, dim). Every piece's (m, l, o[dim]) is loaded
// independently, so a thread's loads are in flight together: one memory round trip per
// kChunk pieces (the merge kernel takes 16 for segments of more than 8 pieces, as a
// 32k-row segment has, and 8 otherwise, whose loads past the last piece would be wasted).
// kCoherent: the partial states come from workgroups of the same launch (device-coherent
// loads); else from a finished launch (plain loads).
template <bool kCoherent, int kChunk = 8>
__device__ __forceinline__ void merge_element(const DecodeArgs& a, int b, int kh, int64_t s, int64_t w0, int64_t w1,
                                              int gg, int d) {
    float M = -INFINITY, Lsum = 0.f, acc = 0.f;
    for (int64_t c0 = w0; c0 <= w1; c0 += kChunk) {
      float m[kChunk], l[kChunk], v[kChunk];
#pragma unroll
      for (int i = 0; i < kChunk; ++i) {
        const int64_t w = c0 + i <= w1 ? c0 + i : w1;  // clamped: duplicates get weight 0 below
        const float* P = a.part + ((w + s) * a.G + gg) * kPieceStride;
        m[i] = kCoherent ? part_load(P) : P[0];
        l[i] = kCoherent ? part_load(P + 1) : P[1];
        v[i] = kCoherent ? part_load(P + 4 + d) : P[4 + d];
      }
      float Mc = M;
#pragma unroll
      for (int i = 0; i < kChunk; ++i)
        if (c0 + i <= w1) Mc = fmaxf(Mc, m[i]);
      const float r = __builtin_amdgcn_exp2f(M - Mc);
      Lsum *= r;
      acc *= r;
#pragma unroll
      for (int i = 0; i < kChunk; ++i)
        if (c0 + i <= w1) {
          const float sc = __builtin_amdgcn_exp2f(m[i] - Mc);
          Lsum += sc * l[i];
          acc += sc * v[i];
        }
      M = Mc;
    }
    a.out[((int64_t)b * a.Hq + (int64_t)kh * a.G + gg) * kD + d] = (uint16_t)f32_to_bf16_bits(acc / Lsum);
}

__device__ void merge_segment(const DecodeArgs& a, int b, int kh, int64_t s, int64_t w0, int64_t w1) {
  for (int e = threadIdx.x; e < a.G * kD; e += blockDim.x) merge_element<true>(a, b, kh, s, w0, w1, e / kD, e % kD);
}

template <bool kFused, bool kFp8, bool kI4 = false, bool kRot = false, bool kDma = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void decode_kernel(DecodeArgs a) {
  // kRot: FP8 rows with the RoPE tail, read only (the fused step over them is the
  // pre-attention kernel followed by this kernel, see launch_decode)
  static_assert(!kRot || (kFp8 && !kFused), "the RoPE-tail reader is the unfused FP8 decode");
  // kDma: tiles through the wave's LDS slots by LDS-DMA (bf16: small grids; fp8: capacities
  // that are a multiple of 8; see launch_decode)
  static_assert(!kDma || (!kI4 && !kRot), "the LDS-DMA tiles are the bf16 and plain fp8 caches'");
  constexpr bool kNarrow = kFp8 || kI4;  // the fp8 head-dim order (kdim)
  __shared__ int32_t pre[kMaxB + 1];
  __shared__ Combine cmb;
  __shared__ __attribute__((aligned(16))) uint8_t wave_lds[kWaves][wave_lds_bytes<kFp8, kI4, kDma>()];
  __shared__ float2 rope_cs[kWaves][kD / 2];  // fused: each wave's RoPE (cos, sin) table at the offset
  __shared__ __attribute__((aligned(16))) uint16_t new_kv[2][kD];  // fused: the new row, for its owner wave
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)

  // Lengths and tile prefix. Up to 64 sequences, each wave forms them in its lanes (lane
  // b: sequence b, scanned across lanes) into its own slice of the LDS table (lengths at
  // 128 wave, prefix at 128 wave + 64), so no workgroup barrier stands before the first
  // loads; larger batches scan into the workgroup's table (pre[0..B]).
  const bool wtab = a.B <= 64;
  int32_t* const tl = pre + 128 * wave;
  int64_t total;
  if (wtab) {
    const int len_l = lane < a.B ? seq_len(a, lane) : 0;
    const int tb = ((len_l + kTile - 1) / kTile) * a.Hkv;
    int incl = tb;
    for (int d = 1; d < 64; d <<= 1) {
      const int v = __shfl_up(incl, d, 64);
      if (lane >= d) incl += v;
    }
    total = __builtin_amdgcn_readlane(incl, 63);
    tl[lane] = len_l;
    tl[64 + lane] = incl - tb;
    if (!a.inline_merge && blockIdx.x == 0 && wave == 0) {
      if (lane < a.B) a.hdr[lane] = incl - tb;
      if (lane == 0) a.hdr[a.B] = (int32_t)total;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  } else {
    build_prefix(a, pre);
    total = pre[a.B];
    if (!a.inline_merge && blockIdx.x == 0)
      for (int i = threadIdx.x; i <= a.B; i += blockDim.x) a.hdr[i] = pre[i];
  }
  auto len_of = [&](int b) __attribute__((always_inline)) { return wtab ? tl[b] : seq_len(a, b); };

  // sequences with no valid position produce zeros (nothing else visits them)
  if (blockIdx.x == 0) {
    const int row_words = a.Hq * kD / 2;
    for (int b = 0; b < a.B; ++b)
      if (len_of(b) == 0)
        for (int i = threadIdx.x; i < row_words; i += blockDim.x) ((uint32_t*)(a.out + (int64_t)b * a.Hq * kD))[i] = 0u;
  }

  const int w = blockIdx.x;
  const int W = active_workers(total, a.W);
  // workgroups past the active workers have no tiles (they still arrive at the grid's
  // counter below when the offsets advance)
  int64_t t = w < W ? worker_begin(a, w, total, W) : 0;
  const int64_t t_end = w < W ? worker_begin(a, w + 1, total, W) : 0;

  const int g = lane & 15;  // query head inside the kv group (B-operand column)
  const int c = lane >> 4;  // 16-lane group
  const int m = lane & 15;  // A-operand row
  // K row feeding A-operand row m of MFMA set r: position 8*(m/4) + 4r + m%4,
  // so that S^T rows 4c..4c+3 of set r are positions 8c + 4r + i.
  const int krow0 = dec_krow(m, 0);

  while (t < t_end) {
    // locate the segment containing tile t (uniform across the workgroup): the largest b
    // with pre[b] <= t
    int b;
    int64_t pre_b;
    if (wtab) {
      const uint64_t le = __ballot(lane < a.B && tl[64 + lane] <= t);  // lane 0 always (pre 0)
      b = 63 - __builtin_clzll(le);
      pre_b = tl[64 + b];
    } else {
      int lo = 0, hi = a.B;
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (pre[mid] <= t) lo = mid; else hi = mid;
      }
      b = lo;
      pre_b = pre[b];
    }
    const int L = len_of(b);
    const int nb = (L + kTile - 1) / kTile;
    const uint32_t rel = (uint32_t)(t - pre_b);  // the prefix is 32-bit
    const int kh = (int)(rel / (uint32_t)nb);
    const int tile0 = (int)(rel % (uint32_t)nb);
    const int64_t seg_first = pre_b + (int64_t)kh * nb;
    const int64_t seg_end = seg_first + nb;
    const int64_t piece_end = t_end < seg_end ? t_end : seg_end;
    const int tile1 = tile0 + (int)(piece_end - t);

    const uint16_t* Kb = a.k + (int64_t)b * a.sb + (int64_t)kh * a.sh;
    const uint16_t* Vb = a.v + (int64_t)b * a.sb + (int64_t)kh * a.sh;

    float m_run = -INFINITY, l_run = 0.f;
    f32x4 o[8];
    for (int j = 0; j < 8; ++j) o[j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // fp8: codes and exponents of the tile in flight, decoded into kc/vc before use
    const uint8_t* const Kb8 = (const uint8_t*)a.k + (int64_t)b * a.sb + (int64_t)kh * a.sh;
    const uint8_t* const Vb8 = (const uint8_t*)a.v + (int64_t)b * a.sb + (int64_t)kh * a.sh;
    const int64_t erow = ((int64_t)b * a.Hkv + kh) * a.cap;  // fp8 exponent / int4 parameter row of position 0
    const uint16_t* const Ke = kFp8 ? (const uint16_t*)a.kexp + erow : nullptr;
    const uint16_t* const Ve = kFp8 ? (const uint16_t*)a.vexp + erow : nullptr;
    // fp8 exponents. The pairs of 8 consecutive rows are 16 contiguous bytes: the plain FP8
    // reader takes one load per lane for K (rows 8 (m / 4) .. +7 of the tile hold both of
    // its rows) and one for V (rows 8c .. +7) instead of one per row, when the capacity is a
    // multiple of 8 (a group lies wholly inside the plane, or wholly past its end, where the
    // range-checked buffer load returns zeros); otherwise it loads its rows one by one
    // (clamped to L - 1) into the same layout. Rows past L get exponent 0 when the tile is
    // decoded: their codes are row L - 1's (clamped loads), finite at scale 1, and their
    // scores and probabilities are masked and zero. The RoPE-tail reader keeps one exponent
    // pair per row (clamped loads): unpacking the groups costs VALU that its loop, and
    // registers that it, cannot spare (5 % slower at the batch-32 step).
    const bool ex16 = kFp8 && !kRot && (a.cap & 7) == 0;
    const __amdgpu_buffer_rsrc_t ke_rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(Ke), (short)0, kFp8 ? a.cap * 2 : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t ve_rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(Ve), (short)0, kFp8 ? a.cap * 2 : 0, 0x00020000);
    u32x2 k8[2][4], v8[8], k8n[2][4], v8n[8];
    // exponents of the tile in use and of the next: the 8-row groups (g) or, in the RoPE-tail
    // reader, one pair per row (r)
    struct ExK {
      u32x4 g;
      uint32_t r[2];
    };
    struct ExV {
      u32x4 g;
      uint32_t r[8];
    };
    ExK ke, ken;
    ExV ve, ven;
    // RoPE tail (kRot): the bf16 K pieces of steps 2, 3 and one aligned 16-byte V load per
    // position: for lanes m < 8 the codes of dims 8(m & ~1) .. +15 (its own 8 are words
    // 2(m & 1), +1), for m >= 8 the bf16 dims 8m .. 8m+7
    u32x4 kt[2][2], ktn[2][2], vw[8], vwn[8];
    auto load_k8 = [&](int tile, u32x2 (&kr)[2][4], ExK& kx, u32x4 (&ktr)[2][2]) {
      const int p0 = tile * kTile;
      for (int r = 0; r < 2; ++r) {
        int p = p0 + krow0 + 4 * r;
        p = p < L ? p : L - 1;
        const uint8_t* row = Kb8 + (int64_t)p * a.sp;
        for (int i = 0; i < (kRot ? 1 : 2); ++i) {  // steps 2i, 2i+1: one 16-byte load
          const u32x4 w = __builtin_nontemporal_load((const u32x4*)(row + kdim<true>(2 * i, c)));
          kr[r][2 * i] = u32x2{w[0], w[1]};
          kr[r][2 * i + 1] = u32x2{w[2], w[3]};
        }
        if (kRot) {  // dims 64 + 16c .. +15 as bf16: bytes 64 + 32c .. +31 of the row
          ktr[r][0] = __builtin_nontemporal_load((const u32x4*)(row + 64 + 32 * c));
          ktr[r][1] = __builtin_nontemporal_load((const u32x4*)(row + 64 + 32 * c + 16));
          kx.r[r] = Ke[p];
        }
      }
      if (kRot) return;
      if (ex16) {
        kx.g = __builtin_amdgcn_raw_buffer_load_b128(ke_rs, 2u * (uint32_t)(p0 + 8 * (m >> 2)), 0, 0);
      } else {  // row 8 (m / 4) + (m % 4) + 4r of the tile at half (m % 4 + 4r) of the group
        kx.g = u32x4{0u, 0u, 0u, 0u};
        for (int r = 0; r < 2; ++r) {
          int p = p0 + krow0 + 4 * r;
          p = p < L ? p : L - 1;
          const uint32_t e = (uint32_t)Ke[p] << (16 * (m & 1));
          if (m & 2) kx.g[2 * r + 1] = e;
          else kx.g[2 * r] = e;
        }
      }
    };
    auto load_v8 = [&](int tile, u32x2 (&vr)[8], ExV& vx, u32x4 (&vwr)[8]) {
      const int p0 = tile * kTile;
      for (int kk = 0; kk < 8; ++kk) {
        int p = p0 + 8 * c + kk;
        p = p < L ? p : L - 1;
        if (kRot) {
          vwr[kk] = __builtin_nontemporal_load(
              (const u32x4*)(Vb8 + (int64_t)p * a.sp + (m < 8 ? 16 * (m >> 1) : 16 * m - 64)));
          vx.r[kk] = Ve[p];
        } else {
          vr[kk] = ld8_stream(Vb8 + (int64_t)p * a.sp + 8 * m);
        }
      }
      if (kRot) return;
      if (ex16) {
        vx.g = __builtin_amdgcn_raw_buffer_load_b128(ve_rs, 2u * (uint32_t)(p0 + 8 * c), 0, 0);
      } else {
        for (int w = 0; w < 4; ++w) {
          int p = p0 + 8 * c + 2 * w;
          p = p < L ? p : L - 1;
          const int p1 = p + 1 < L ? p + 1 : L - 1;
          vx.g[w] = (uint32_t)Ve[p] | ((uint32_t)Ve[p1] << 16);
        }
      }
    };
    auto load_tile8 = [&](int tile, u32x2 (&kr)[2][4], u32x2 (&vr)[8], ExK& kx, ExV& vx,
                          u32x4 (&ktr)[2][2], u32x4 (&vwr)[8]) {
      load_k8(tile, kr, kx, ktr);
      load_v8(tile, vr, vx, vwr);
    };
    // fp8 with kDma: the tile's codes and exponents by LDS-DMA into slot sl (10 instructions:
    // four of 8 whole K rows, four of 8 whole V rows, two of the 32 exponent pairs on 4
    // lanes), code rows past L clamped to row L - 1; the exponents of rows past L are zeroed
    // when the tile is decoded (rows past the capacity read as zeros: the capacity is a
    // multiple of 8, so no 16-byte piece straddles it).
    uint8_t* const f8base = &wave_lds[wave][0];
    const uint32_t f8lds = (uint32_t)(uintptr_t)(lds_void*)f8base;
    const uint32_t f8plane = (uint32_t)a.cap * (uint32_t)a.sp;  // bounded by the host
    const u32x4 k8_rs = rsrc_words(Kb8, f8plane), v8_rs = rsrc_words(Vb8, f8plane);
    const u32x4 ke8_rs = rsrc_words(Ke, (uint32_t)a.cap * 2u), ve8_rs = rsrc_words(Ve, (uint32_t)a.cap * 2u);
    constexpr int kF8Dma = 10;  // DMA instructions per tile
    auto f8_dma = [&](int tile, int sl) __attribute__((always_inline)) {
      const int p0 = tile * kTile;
      const uint32_t dst = f8lds + (uint32_t)sl * kF8Slot;
      for (int i = 0; i < 4; ++i) {
        const int S = 8 * i + (lane >> 3), u = lane & 7;
        const int pk = p0 + S < L ? p0 + S : L - 1;  // K: slot row S is row S
        const int R = f8_vrow(S);                     // V: slot row S holds row R
        const int pv = p0 + R < L ? p0 + R : L - 1;
        dma16(k8_rs, (uint32_t)pk * (uint32_t)a.sp + 16u * (uint32_t)(u ^ f8_swz(S)), 0u, dst + 1024u * i);
        dma16(v8_rs, (uint32_t)pv * (uint32_t)a.sp + 16u * (uint32_t)u, 0u, dst + kF8SlotV + 1024u * i);
      }
      if (lane < 4) {
        dma16(ke8_rs, 2u * (uint32_t)p0 + 16u * lane, 0u, dst + kF8SlotKe);
        dma16(ve8_rs, 2u * (uint32_t)p0 + 16u * lane, 0u, dst + kF8SlotVe);
      }
    };
    auto f8_read = [&](int sl) __attribute__((always_inline)) {
      const uint8_t* const sp8 = f8base + sl * kF8Slot;
      for (int r = 0; r < 2; ++r) {
        const int R = krow0 + 4 * r;
        for (int i = 0; i < 2; ++i) {  // steps 2i, 2i + 1: chunk 4i + c of the row
          const u32x4 w = *(const u32x4*)(sp8 + 128 * R + 16 * ((4 * i + c) ^ f8_swz(R)));
          k8[r][2 * i] = u32x2{w[0], w[1]};
          k8[r][2 * i + 1] = u32x2{w[2], w[3]};
        }
      }
      for (int kk = 0; kk < 8; ++kk) {
        const int R = 8 * c + kk;
        v8[kk] = *(const u32x2*)(sp8 + kF8SlotV + 128 * f8_vrow(R) + 8 * m);
      }
      ke.g = *(const u32x4*)(sp8 + kF8SlotKe + 16 * (m >> 2));
      ve.g = *(const u32x4*)(sp8 + kF8SlotVe + 16 * c);
    };
    u32x4 kc[2][4], vc[8], kn[2][4], vn[8];
    auto decode_tile8 = [&](int tile) {
      const int p0 = tile * kTile;
      const bool tail = p0 + kTile > L;  // the segment's last tile: rows past L get exponent 0
      for (int r = 0; r < 2; ++r) {
        const int row = p0 + 8 * (m >> 2) + (m & 3) + 4 * r;
        uint32_t kx = kRot ? ke.r[r] : (((m & 2) ? ke.g[2 * r + 1] : ke.g[2 * r]) >> (16 * (m & 1))) & 0xFFFFu;
        if (!kRot && tail && row >= L) kx = 0u;
        for (int s = 0; s < 4; ++s)
          kc[r][s] = kRot && s >= 2 ? kt[r][s - 2] : fp8_decode8(k8[r][s], (int)(int8_t)(kx >> (s >= 2 ? 8 : 0)));
      }
      for (int kk = 0; kk < 8; ++kk) {
        uint32_t vx = kRot ? ve.r[kk] : (ve.g[kk >> 1] >> (16 * (kk & 1))) & 0xFFFFu;
        if (!kRot && tail && p0 + 8 * c + kk >= L) vx = 0u;
        if (kRot) {
          const u32x2 w = (m & 1) ? u32x2{vw[kk][2], vw[kk][3]} : u32x2{vw[kk][0], vw[kk][1]};
          const u32x4 d = fp8_decode8(w, (int)(int8_t)vx);
          vc[kk] = m < 8 ? d : vw[kk];
        } else {
          vc[kk] = fp8_decode8(v8[kk], (int)(int8_t)(vx >> (m >= 8 ? 8 : 0)));
        }
      }
    };
    // bf16 tiles, two ways (positions past L clamped to row L - 1 in both, so every row read
    // is a valid one):
    // - straight into registers in the operands' layout, the next tile's loads in flight
    //   during this one's work (full grids: the loads of many workgroups cover each other);
    // - kDma (small grids): by LDS-DMA of whole rows into the wave's slot, 1 KB (four rows)
    //   per instruction, then read out in the operands' layout. The operand layout takes 64
    //   bytes of each of 16 K rows per load, and a CU issues those loads about 2.5 times
    //   slower than whole rows, which a latency-bound grid pays in full (one tile's loads
    //   per wave: 1.27 against 0.51 us in isolation). Its next tile's DMA can only refill
    //   the slot after this one is read out, which costs full grids their overlap.
    auto load_tile = [&](int tile, u32x4 (&kr)[2][4], u32x4 (&vr)[8]) {
      const int p0 = tile * kTile;
      for (int r = 0; r < 2; ++r) {
        int p = p0 + krow0 + 4 * r;
        p = p < L ? p : L - 1;
        const uint16_t* row = Kb + (int64_t)p * a.sp;
        for (int s = 0; s < 4; ++s) kr[r][s] = ld16_stream(row + 8 * (4 * s + c));
      }
      for (int kk = 0; kk < 8; ++kk) {
        int p = p0 + 8 * c + kk;
        p = p < L ? p : L - 1;
        vr[kk] = ld16_stream(Vb + (int64_t)p * a.sp + 8 * m);
      }
    };
    uint8_t* const bslot = &wave_lds[wave][0];
    const uint32_t bslot_lds = (uint32_t)(uintptr_t)(lds_void*)bslot;
    const uint32_t plane_bytes = (uint32_t)a.cap * (uint32_t)a.sp * 2u;  // bounded by the host
    const u32x4 kbf_rs = rsrc_words(Kb, plane_bytes), vbf_rs = rsrc_words(Vb, plane_bytes);
    auto bf_dma = [&](int tile) __attribute__((always_inline)) {
      const int p0 = tile * kTile;
      for (int i = 0; i < 8; ++i) {
        const int R = 4 * i + (lane >> 4);
        const int p = p0 + R < L ? p0 + R : L - 1;
        const uint32_t roff = (uint32_t)p * (uint32_t)a.sp * 2u;
        dma16(kbf_rs, roff + 16u * (uint32_t)((lane & 15) ^ bf_swz(R)), 0u, bslot_lds + 1024u * i);
        dma16(vbf_rs, roff + 16u * (uint32_t)(lane & 15), 0u, bslot_lds + 8192u + 1024u * i);
      }
    };
    auto bf_read = [&]() __attribute__((always_inline)) {
      for (int r = 0; r < 2; ++r) {
        const int R = krow0 + 4 * r;
        for (int s = 0; s < 4; ++s)
          kc[r][s] = *(const u32x4*)(bslot + 1024 * (R >> 2) + 256 * (R & 3) + 16 * ((4 * s + c) ^ bf_swz(R)));
      }
      for (int kk = 0; kk < 8; ++kk) {
        const int R = 8 * c + kk;
        vc[kk] = *(const u32x4*)(bslot + 8192 + 1024 * (R >> 2) + 256 * (R & 3) + 16 * m);
      }
    };
    // int4: the wave streams its tiles into a ring of kI4Slots LDS slots, two tiles ahead
    // of the one in use, by LDS loads from buffer resources over this segment's code and
    // parameter planes (the tile moves the scalar offset only). Every tile lies inside the
    // capacity (a multiple of 32), so positions past L load stale rows: their codes are
    // finite, their scores are masked and their V parameters zeroed before use.
    const uint32_t rb4 = (uint32_t)(a.sp / 2);  // bytes per cache row of codes
    const int64_t plane4 = ((int64_t)b * a.sb + (int64_t)kh * a.sh) / 2;
    const u32x4 k_rs = rsrc_words((const uint8_t*)a.k + plane4, (uint32_t)a.cap * rb4);
    const u32x4 v_rs = rsrc_words((const uint8_t*)a.v + plane4, (uint32_t)a.cap * rb4);
    const uint32_t pbytes = (uint32_t)a.cap * 4u;
    const u32x4 ks_rs = rsrc_words(a.ks + erow, pbytes);
    const u32x4 kb_rs = rsrc_words(a.kb + erow, pbytes);
    const u32x4 vs_rs = rsrc_words(a.vs + erow, pbytes);
    const u32x4 vb_rs = rsrc_words(a.vb + erow, pbytes);
    // K and V rows: load j, lane l moves bytes 16 (l % 4) .. +15 of row 16 j + l / 4
    const uint32_t row_off = (uint32_t)(lane >> 2) * rb4 + 16u * (lane & 3);
    uint8_t* const ring = &wave_lds[wave][0];
    const uint32_t ring_lds = (uint32_t)(uintptr_t)(lds_void*)ring;
    auto i4_dma = [&](int tile, int slot) __attribute__((always_inline)) {
      const uint32_t p0 = (uint32_t)tile * kTile;
      const uint32_t dst = ring_lds + (uint32_t)slot * kI4Slot;
      for (int j = 0; j < 2; ++j) {
        dma16(k_rs, row_off, (p0 + 16 * j) * rb4, dst + kI4SlotK + 1024 * j);
        dma16(v_rs, row_off, (p0 + 16 * j) * rb4, dst + kI4SlotV + 1024 * j);
      }
      if (lane < 8) {  // 8 lanes x 16 bytes: the words of the tile's 32 positions
        dma16(ks_rs, 16u * lane, 4 * p0, dst + kI4SlotKs);
        dma16(kb_rs, 16u * lane, 4 * p0, dst + kI4SlotKb);
        dma16(vs_rs, 16u * lane, 4 * p0, dst + kI4SlotVs);
        dma16(vb_rs, 16u * lane, 4 * p0, dst + kI4SlotVb);
      }
    };
    auto i4_read = [&](int slot, I4Tile& t) __attribute__((always_inline)) {
      const uint8_t* const sp = ring + slot * kI4Slot;
      for (int r = 0; r < 2; ++r)
        for (int i = 0; i < 2; ++i) t.k[r][i] = *(const u32x2*)(sp + kI4SlotK + 64 * (krow0 + 4 * r) + 32 * i + 8 * c);
      for (int kk = 0; kk < 8; ++kk) t.v[kk] = *(const uint32_t*)(sp + kI4SlotV + 64 * (8 * c + kk) + 4 * m);
      for (int h = 0; h < 2; ++h) {
        t.ks[h] = *(const u32x4*)(sp + kI4SlotKs + 4 * (8 * c + 4 * h));
        t.kb[h] = *(const uint32_t*)(sp + kI4SlotKb + 4 * (krow0 + 4 * h));
        t.vs[h] = *(const u32x4*)(sp + kI4SlotVs + 4 * (8 * c + 4 * h));
        t.vb[h] = *(const u32x4*)(sp + kI4SlotVb + 4 * (8 * c + 4 * h));
      }
    };

    // q loads, then this wave's first tile loads, then the q work: the work below runs
    // while the tiles are in flight. B operand Q^T: step s <-> dims kdim(s, c) .. +7;
    // columns g >= G are zero padding (their clamped, in-bounds loads are discarded).
    const int first = tile0 + wave;
    const int gc = g < a.G ? g : 0;
    const int F = (a.Hq + 2 * a.Hkv) * kD;
    const uint16_t* qh = kFused ? a.qkv + (int64_t)b * F + ((int64_t)kh * a.G + gc) * kD
                                : a.q + ((int64_t)b * a.Hq + (int64_t)kh * a.G + gc) * kD;
    u32x4 qraw[4], qwv[4];
    uint16_t kr1 = 0, kr2 = 0, kw1 = 0, kw2 = 0, vr1 = 0, vr2 = 0;
    for (int s = 0; s < 4; ++s) qraw[s] = ld16(qh + kdim<kNarrow>(s, c));
    // fused: the new k, v row goes to row w of the cache (the offset; offset % cap for a
    // rotating cache) when it is written at all (a static cache skips an offset past the
    // capacity). The wave that will run the tile holding row w forms the row; its inputs
    // are loaded now, with the q row and the norm weights.
    int w_row = -1;
    if (kFused) {
      const int off_b = a.off[b];
      if (a.rot) w_row = off_b >= 0 ? off_b % a.cap : -1;
      else w_row = off_b == L - 1 ? off_b : -1;
    }
    const int w_tile = w_row >= 0 ? w_row / kTile : -1;
    const bool owner = kFused && w_row >= 0 && tile0 <= w_tile && w_tile < tile1 && wave == (w_tile - tile0) % kWaves;
    if (kFused) {
      // unconditional loads: without norm weights (EMA_PRE_NO_NORM) the launcher points
      // qw / kw at the qkv rows, and the values are not used (with a branch here the
      // fused fp8 step spilled 11 VGPRs to scratch and ran 82 us instead of 68.7)
      for (int s = 0; s < 4; ++s) qwv[s] = ld16(a.qw + kdim<kNarrow>(s, c));
      if (owner) {  // lane i: dims i and i + 64 (a RoPE pair)
        const uint16_t* kr = a.qkv + (int64_t)b * F + ((int64_t)a.Hq + kh) * kD;
        const uint16_t* vr = kr + (int64_t)a.Hkv * kD;
        kr1 = kr[lane];
        kr2 = kr[lane + 64];
        kw1 = a.kw[lane];
        kw2 = a.kw[lane + 64];
        vr1 = vr[lane];
        vr2 = vr[lane + 64];
      }
    }
    if (first < tile1) {
      if (kI4) {
        // untracked by the compiler: its waits for the q loads above also wait for these,
        // which are in flight alongside them (the fused step, whose q work waits on more
        // loads, issues them after that work instead)
        if (!kFused) {
          i4_dma(first, 0);
          if (first + kWaves < tile1) i4_dma(first + kWaves, 1);
        }
      } else if (kFp8 && kDma) {
        f8_dma(first, 0);
      } else if (kFp8) {
        load_tile8(first, k8, v8, ke, ve, kt, vw);
      } else {
        if (kDma) bf_dma(first);
        else load_tile(first, kc, vc);
      }
    }
    bf16x8 qop[4];
    const float2* const cs_tab = rope_cs[wave];
    if (!kFused) {
      const u32x4 z = {0u, 0u, 0u, 0u};
      for (int s = 0; s < 4; ++s) qop[s] = as_bf16x8(g < a.G ? (kI4 ? i4_qperm(qraw[s]) : qraw[s]) : z);
    } else {
      // q = rope(norm(q_raw)) of this head, from the fused qkv row. Each wave forms the 64
      // RoPE angles of this sequence's offset into its own table (lane i: angle i), so no
      // workgroup barrier is needed.
      const int off = a.off[b];
      if (!(a.flags & EMA_PRE_NO_ROPE)) {
        const float inv_freq = exp2f(-((float)lane / (float)(kD / 2)) * a.log2_theta);
        float sn, cs;
        sincosf((float)off * inv_freq, &sn, &cs);
        rope_cs[wave][lane] = make_float2(cs, sn);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      float x[32];
      unpack32(qraw, x);
      norm_rope<kNarrow>(a, x, qwv, cs_tab);
      for (int s = 0; s < 4; ++s) {
        u32x4 v;
        for (int e = 0; e < 4; ++e) v[e] = g < a.G ? pack_bf16x2(x[8 * s + 2 * e], x[8 * s + 2 * e + 1]) : 0u;
        qop[s] = as_bf16x8(kI4 ? i4_qperm(v) : v);
      }
      if (owner) {
        // the new row (lane i: dims i, i + 64): k = rope(norm(k_raw)), v a bit copy; it
        // goes to cache row w and to LDS, from where this same wave patches the rows of its
        // tile that load row w (with a static cache, also the rows past L - 1 = w, which
        // the loads clamp to it)
        float k1 = bf16_to_f32(kr1), k2 = bf16_to_f32(kr2);
        if (!(a.flags & (EMA_PRE_NO_NORM | EMA_PRE_NO_K_NORM))) {
          float ss = k1 * k1 + k2 * k2;
          for (int mm = 32; mm >= 1; mm >>= 1) ss += __shfl_xor(ss, mm, 64);
          const float inv = 1.0f / sqrtf(ss / (float)kD + a.eps);
          k1 = bf16_to_f32((uint16_t)f32_to_bf16_bits(bf16_to_f32((uint16_t)f32_to_bf16_bits(k1 * inv)) * bf16_to_f32(kw1)));
          k2 = bf16_to_f32((uint16_t)f32_to_bf16_bits(bf16_to_f32((uint16_t)f32_to_bf16_bits(k2 * inv)) * bf16_to_f32(kw2)));
        }
        if (!(a.flags & EMA_PRE_NO_ROPE)) {
          const float cs = cs_tab[lane].x, sn = cs_tab[lane].y;
          const float r1 = k1 * cs - k2 * sn, r2 = k1 * sn + k2 * cs;
          k1 = r1;
          k2 = r2;
        }
        const uint16_t kb1 = (uint16_t)f32_to_bf16_bits(k1), kb2 = (uint16_t)f32_to_bf16_bits(k2);
        if (kI4) {
          // the row is quantised per 64-dim group (lane i holds dims i and i + 64) and kept
          // in LDS in its stored form: K words 0..15, V words 16..31, then the K scale, K
          // bias, V scale and V bias pairs
          const float nv[4] = {bf16_to_f32(kb1), bf16_to_f32(kb2), bf16_to_f32(vr1), bf16_to_f32(vr2)};
          uint32_t* const nw = (uint32_t*)&new_kv[0][0];
          float sq[4], bq[4];
          uint32_t cw4[4];
          for (int q = 0; q < 4; ++q) {
            float mn = nv[q], mx = nv[q];
            for (int mm = 32; mm >= 1; mm >>= 1) {
              mn = fminf(mn, __shfl_xor(mn, mm, 64));
              mx = fmaxf(mx, __shfl_xor(mx, mm, 64));
            }
            i4_params(mn, mx, sq[q], bq[q]);
            uint32_t t = i4_code(nv[q], sq[q], bq[q]) << (4 * (lane & 7));
            t |= __shfl_xor(t, 1, 64);
            t |= __shfl_xor(t, 2, 64);
            t |= __shfl_xor(t, 4, 64);
            cw4[q] = t;  // word lane / 8 of the group: dims 64 (q % 2) + 8 (lane / 8) .. +7
          }
          const int64_t roff = ((int64_t)b * a.sb + (int64_t)kh * a.sh + (int64_t)w_row * a.sp) / 2;
          uint32_t* const kd = (uint32_t*)((uint8_t*)a.k + roff);
          uint32_t* const vd = (uint32_t*)((uint8_t*)a.v + roff);
          if ((lane & 7) == 0) {
            const int wi = lane >> 3;
            nw[wi] = cw4[0];
            nw[8 + wi] = cw4[1];
            nw[16 + wi] = cw4[2];
            nw[24 + wi] = cw4[3];
            kd[wi] = cw4[0];
            kd[8 + wi] = cw4[1];
            vd[wi] = cw4[2];
            vd[8 + wi] = cw4[3];
          }
          if (lane == 0) {
            const uint32_t ksw = f32_to_bf16_bits(sq[0]) | (f32_to_bf16_bits(sq[1]) << 16);
            const uint32_t kbw = f32_to_bf16_bits(bq[0]) | (f32_to_bf16_bits(bq[1]) << 16);
            const uint32_t vsw = f32_to_bf16_bits(sq[2]) | (f32_to_bf16_bits(sq[3]) << 16);
            const uint32_t vbw = f32_to_bf16_bits(bq[2]) | (f32_to_bf16_bits(bq[3]) << 16);
            nw[32] = ksw;
            nw[33] = kbw;
            nw[34] = vsw;
            nw[35] = vbw;
            a.ks[erow + w_row] = ksw;
            a.kb[erow + w_row] = kbw;
            a.vs[erow + w_row] = vsw;
            a.vb[erow + w_row] = vbw;
          }
        } else if (kFp8) {
          // the row is stored as E4M3FN codes and attended in its decoded form
          uint16_t d[4];
          int e[4];
          const uint32_t c0 = fp8_quant_lane(bf16_to_f32(kb1), &e[0], &d[0]);
          const uint32_t c1 = fp8_quant_lane(bf16_to_f32(kb2), &e[1], &d[1]);
          const uint32_t c2 = fp8_quant_lane(bf16_to_f32(vr1), &e[2], &d[2]);
          const uint32_t c3 = fp8_quant_lane(bf16_to_f32(vr2), &e[3], &d[3]);
          new_kv[0][lane] = d[0];
          new_kv[0][lane + 64] = d[1];
          new_kv[1][lane] = d[2];
          new_kv[1][lane + 64] = d[3];
          uint8_t* const kd = (uint8_t*)a.k + (int64_t)b * a.sb + (int64_t)kh * a.sh + (int64_t)w_row * a.sp;
          uint8_t* const vd = (uint8_t*)a.v + (int64_t)b * a.sb + (int64_t)kh * a.sh + (int64_t)w_row * a.sp;
          kd[lane] = (uint8_t)c0;
          kd[lane + 64] = (uint8_t)c1;
          vd[lane] = (uint8_t)c2;
          vd[lane + 64] = (uint8_t)c3;
          if (lane == 0) {
            ((uint16_t*)a.kexp)[erow + w_row] = (uint16_t)((uint8_t)e[0] | ((uint32_t)(uint8_t)e[1] << 8));
            ((uint16_t*)a.vexp)[erow + w_row] = (uint16_t)((uint8_t)e[2] | ((uint32_t)(uint8_t)e[3] << 8));
          }
        } else {
          new_kv[0][lane] = kb1;
          new_kv[0][lane + 64] = kb2;
          new_kv[1][lane] = vr1;
          new_kv[1][lane + 64] = vr2;
          uint16_t* const kd = (uint16_t*)a.k + (int64_t)b * a.sb + (int64_t)kh * a.sh + (int64_t)w_row * a.sp;
          uint16_t* const vd = (uint16_t*)a.v + (int64_t)b * a.sb + (int64_t)kh * a.sh + (int64_t)w_row * a.sp;
          kd[lane] = kb1;
          kd[lane + 64] = kb2;
          vd[lane] = vr1;
          vd[lane + 64] = vr2;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    }

    if (kI4 && kFused && first < tile1) {
      i4_dma(first, 0);
      if (first + kWaves < tile1) i4_dma(first + kWaves, 1);
    }
    // int4: sums Qs of the (bf16) q over each 64-dim group, per column g. The score MFMAs
    // of a group start from -128 Qs (the offset of the 128 + code operands), and one more
    // MFMA per row set adds b0 Qs0 + b1 Qs1 (k-slots 0..3 of lane group 0: Qs split into
    // bf16 hi and lo parts times the row's bias pair). The output corrections
    // sum_p (P b_grp - 128 P'_grp) accumulate in cb[grp] by two MFMAs per group and tile;
    // every row of cb[grp] holds the column's value.
    float qs0 = 0.f, qs1 = 0.f;
    f32x4 cb[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    u32x4 qbias = {0u, 0u, 0u, 0u};
    if (kI4) {
      for (int s = 0; s < 4; ++s) {
        const u32x4 w = __builtin_bit_cast(u32x4, qop[s]);
        float t = 0.f;
        for (int e = 0; e < 4; ++e) t += bf16_lo(w[e]) + bf16_hi(w[e]);
        if (s < 2) qs0 += t;
        else qs1 += t;
      }
      qs0 += __shfl_xor(qs0, 16, 64);
      qs0 += __shfl_xor(qs0, 32, 64);
      qs1 += __shfl_xor(qs1, 16, 64);
      qs1 += __shfl_xor(qs1, 32, 64);
      if (c == 0) {
        const uint32_t h0 = f32_to_bf16_bits(qs0), h1 = f32_to_bf16_bits(qs1);
        qbias[0] = h0 | (f32_to_bf16_bits(qs0 - bf16_lo(h0)) << 16);
        qbias[1] = h1 | (f32_to_bf16_bits(qs1 - bf16_lo(h1)) << 16);
      }
    }
    const f32x4 ainit0 = {-128.f * qs0, -128.f * qs0, -128.f * qs0, -128.f * qs0};
    const f32x4 ainit1 = {-128.f * qs1, -128.f * qs1, -128.f * qs1, -128.f * qs1};
    const u32x4 neg128 = {0xC300C300u, 0xC300C300u, 0xC300C300u, 0xC300C300u};  // bf16 -128
    // int4 V: lane m and lane m ^ 8 swap half words, so that nibble j of a lane's word is
    // dim 64 (j / 4) + 8 (m % 8) + 4 (m / 8) + j % 4 and the first four nibbles are group 0
    const uint32_t vsel = m < 8 ? 0x05040100u : 0x03020706u;

    // int4 scores of tile `tile` from registers t into x (position p0 + 8c + k <-> x[k]);
    // in a segment's last tile, positions past L (stale rows) are masked and their V
    // parameters (possibly not finite) zeroed.
    auto i4_scores = [&](I4Tile& t, int tile, float* x) __attribute__((always_inline)) {
      const int p0 = tile * kTile;
      if (kFused && owner && tile == w_tile) {
        // the stored form of row w (LDS), into the registers that loaded it
        const uint32_t* nw = (const uint32_t*)&new_kv[0][0];
        for (int r = 0; r < 2; ++r)
          if (p0 + krow0 + 4 * r == w_row) {
            for (int i = 0; i < 2; ++i) t.k[r][i] = u32x2{nw[8 * i + 2 * c], nw[8 * i + 2 * c + 1]};
            t.kb[r] = nw[33];
          }
        for (int kk = 0; kk < 8; ++kk)
          if (p0 + 8 * c + kk == w_row) t.v[kk] = nw[16 + m];
        for (int h = 0; h < 2; ++h)
          for (int e = 0; e < 4; ++e)
            if (p0 + 8 * c + 4 * h + e == w_row) {
              t.ks[h][e] = nw[32];
              t.vs[h][e] = nw[34];
              t.vb[h][e] = nw[35];
            }
      }
      // C row 4c + i of set r is position p0 + 8c + 4r + i
      for (int r = 0; r < 2; ++r) {
        f32x4 acc0 = ainit0, acc1 = ainit1;
        acc0 = mfma16(i4_kop(t.k[r][0][0]), qop[0], acc0);
        acc0 = mfma16(i4_kop(t.k[r][0][1]), qop[1], acc0);
        acc1 = mfma16(i4_kop(t.k[r][1][0]), qop[2], acc1);
        acc1 = mfma16(i4_kop(t.k[r][1][1]), qop[3], acc1);
        u32x4 ab;
        ab[0] = __builtin_amdgcn_perm(t.kb[r], t.kb[r], 0x01000100u);  // (b0, b0)
        ab[1] = __builtin_amdgcn_perm(t.kb[r], t.kb[r], 0x03020302u);  // (b1, b1)
        ab[2] = ab[0];
        ab[3] = ab[1];
        const f32x4 accb = mfma16(as_bf16x8(ab), as_bf16x8(qbias), f32x4{0.f, 0.f, 0.f, 0.f});
        for (int i = 0; i < 4; ++i)
          x[4 * r + i] = __builtin_fmaf(bf16_lo(t.ks[r][i]), acc0[i], __builtin_fmaf(bf16_hi(t.ks[r][i]), acc1[i], accb[i]));
      }
      if (p0 + kTile > L)
        for (int k = 0; k < 8; ++k)
          if (p0 + 8 * c + k >= L) {
            x[k] = -INFINITY;
            t.vs[k >> 2][k & 3] = 0u;
            t.vb[k >> 2][k & 3] = 0u;
          }
    };
    // int4 PV of one tile: probabilities x (position p0 + 8c + k <-> x[k]) against the
    // codes and parameters in t
    auto i4_pv = [&](const I4Tile& t, const float* x) __attribute__((always_inline)) {
      uint32_t cw[8];
      for (int kk = 0; kk < 8; ++kk) {
        const uint32_t pw = (uint32_t)__builtin_amdgcn_mov_dpp((int)t.v[kk], 0x128, 0xF, 0xF, false);  // row_ror:8
        cw[kk] = __builtin_amdgcn_perm(pw, t.v[kk], vsel);
      }
      // B operands P'_grp = bf16(P s_grp) and bf16(P), A operands of the bias rows; k = 2e,
      // 2e + 1 <-> positions p0 + 8c + 2e, +1
      u32x4 pw0, pw1, pb, ab0, ab1;
      for (int e = 0; e < 4; ++e) {
        const uint32_t s_lo = t.vs[e >> 1][2 * (e & 1)], s_hi = t.vs[e >> 1][2 * (e & 1) + 1];
        const uint32_t b_lo = t.vb[e >> 1][2 * (e & 1)], b_hi = t.vb[e >> 1][2 * (e & 1) + 1];
        pw0[e] = pack_bf16x2(x[2 * e] * bf16_lo(s_lo), x[2 * e + 1] * bf16_lo(s_hi));
        pw1[e] = pack_bf16x2(x[2 * e] * bf16_hi(s_lo), x[2 * e + 1] * bf16_hi(s_hi));
        pb[e] = pack_bf16x2(x[2 * e], x[2 * e + 1]);
        ab0[e] = __builtin_amdgcn_perm(b_hi, b_lo, 0x05040100u);  // (b0 of 2e, b0 of 2e + 1)
        ab1[e] = __builtin_amdgcn_perm(b_hi, b_lo, 0x07060302u);  // (b1 of 2e, b1 of 2e + 1)
      }
      const bf16x8 pop0 = as_bf16x8(pw0), pop1 = as_bf16x8(pw1);
      cb[0] = mfma16(as_bf16x8(ab0), as_bf16x8(pb), cb[0]);
      cb[0] = mfma16(as_bf16x8(neg128), pop0, cb[0]);
      cb[1] = mfma16(as_bf16x8(ab1), as_bf16x8(pb), cb[1]);
      cb[1] = mfma16(as_bf16x8(neg128), pop1, cb[1]);
      // A operand of dim slot j: row m, k-slots (2tt, 2tt + 1) = nibble j of the words of
      // positions p0 + 8c + 2tt, +1 (byte j / 2 of both gathered by one v_perm)
      for (int bb = 0; bb < 4; ++bb) {
        u32x4 a0, a1;
        for (int tt = 0; tt < 4; ++tt) {
          const uint32_t w2 = __builtin_amdgcn_perm(cw[2 * tt + 1], cw[2 * tt], 0x0C000C00u | (uint32_t)bb | ((4u + bb) << 16));
          a0[tt] = and_or(w2, 0x000F000Fu, 0x43004300u);
          a1[tt] = and_or(w2 >> 4, 0x000F000Fu, 0x43004300u);
        }
        o[2 * bb] = mfma16(as_bf16x8(a0), bb < 2 ? pop0 : pop1, o[2 * bb]);
        o[2 * bb + 1] = mfma16(as_bf16x8(a1), bb < 2 ? pop0 : pop1, o[2 * bb + 1]);
      }
    };

    if constexpr (kI4) {
      // slot si holds this tile; the tile two ahead goes into the slot read last
      int si = 0;
      for (int tile = first; tile < tile1; tile += kWaves) {
        if (tile + 2 * kWaves < tile1) {
          i4_dma(tile + 2 * kWaves, si == 0 ? 2 : si - 1);
          wait_vm<16>();  // this tile's 8 loads have landed, the 16 after them may not
        } else if (tile + kWaves < tile1) {
          wait_vm<8>();
        } else {
          wait_vm<0>();
        }
        I4Tile t;
        i4_read(si, t);
        float x[8];
        i4_scores(t, tile, x);
        float mx = fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])), fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7])));
        mx = max_over_rows(mx);
        const float m_new = fmaxf(m_run, mx * a.qk_scale);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        const bool grew = __any(m_new > m_run);
        float psum = 0.f;
        for (int e = 0; e < 8; ++e) {
          x[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[e], a.qk_scale, -m_new));
          psum += x[e];
        }
        l_run = l_run * alpha + psum;
        m_run = m_new;
        if (grew) {
          // rescale only when some column's maximum grew (alpha is exactly 1 elsewhere)
          for (int j = 0; j < 8; ++j) o[j] *= alpha;
          cb[0] *= alpha;
          cb[1] *= alpha;
        }
        i4_pv(t, x);
        si = si == 2 ? 0 : si + 1;
      }
    }
    if constexpr (!kI4)
    for (int tile = first; tile < tile1; tile += kWaves) {
      const bool more = tile + kWaves < tile1;
      if (kFp8 && kRot) {
        // decoded first, so that the raw tile dies before the next one's registers are
        // claimed; the next V rows are requested after the score MFMAs, once kc is dead
        decode_tile8(tile);
        if (more) load_k8(tile + kWaves, k8n, ken, ktn);
      } else if (kFp8 && kDma) {
        // two slots: the next tile's DMA goes to the other slot (read out in the previous
        // iteration) before this tile's is waited for
        const int sl = ((tile - first) / kWaves) & 1;
        if (more) {
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          f8_dma(tile + kWaves, sl ^ 1);
          wait_vm<kF8Dma>();
        } else {
          wait_vm<0>();
        }
        f8_read(sl);
        decode_tile8(tile);
      } else if (kFp8) {
        if (more) load_tile8(tile + kWaves, k8n, v8n, ken, ven, ktn, vwn);
        decode_tile8(tile);
      } else if (kDma) {
        wait_vm<0>();  // this tile's DMA has landed (and every load before it)
        bf_read();
        if (more) {
          // the slot's reads are done before the next tile's DMA refills it
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          bf_dma(tile + kWaves);
        }
      } else if (more) {
        load_tile(tile + kWaves, kn, vn);
      }
      const int p0 = tile * kTile;
      if (kFused && owner && tile == w_tile) {
        // rows whose (clamped) load position is w
        for (int r = 0; r < 2; ++r) {
          const int p = p0 + krow0 + 4 * r;
          if ((p < L ? p : L - 1) == w_row)
            for (int s = 0; s < 4; ++s) kc[r][s] = *(const u32x4*)&new_kv[0][kdim<kNarrow>(s, c)];
        }
        for (int kk = 0; kk < 8; ++kk) {
          const int p = p0 + 8 * c + kk;
          if ((p < L ? p : L - 1) == w_row) vc[kk] = *(const u32x4*)&new_kv[1][8 * m];
        }
      }

      f32x4 sc[2];
      for (int r = 0; r < 2; ++r) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s < 4; ++s) acc = mfma16(as_bf16x8(kc[r][s]), qop[s], acc);
        sc[r] = acc;
      }
      if (kFp8 && kRot && more) load_v8(tile + kWaves, v8n, ven, vwn);
      // running max on raw scores (scale > 0), exponent as one fma
      float x[8];
      float mx = -INFINITY;
      for (int r = 0; r < 2; ++r)
        for (int i = 0; i < 4; ++i) {
          const int pos = p0 + 8 * c + 4 * r + i;
          const float v = pos < L ? sc[r][i] : -INFINITY;
          x[4 * r + i] = v;
          mx = fmaxf(mx, v);
        }
      mx = max_over_rows(mx);
      const float m_new = fmaxf(m_run, mx * a.qk_scale);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      float psum = 0.f;
      for (int e = 0; e < 8; ++e) {
        x[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(x[e], a.qk_scale, -m_new));
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
          const uint32_t lo2 = vc[2 * tt][j >> 1];
          const uint32_t hi2 = vc[2 * tt + 1][j >> 1];
          av[tt] = (j & 1) ? ((lo2 >> 16) | (hi2 & 0xffff0000u)) : ((lo2 & 0xffffu) | (hi2 << 16));
        }
        o[j] = mfma16(as_bf16x8(av), pop, o[j]);
      }
      if (!kFp8 && !kDma && more) {
        for (int r = 0; r < 2; ++r)
          for (int s = 0; s < 4; ++s) kc[r][s] = kn[r][s];
        for (int kk = 0; kk < 8; ++kk) vc[kk] = vn[kk];
      }
      if (kFp8 && !kDma && more) {
        for (int r = 0; r < 2; ++r) {
          for (int s = 0; s < 4; ++s) k8[r][s] = k8n[r][s];
          if (kRot) kt[r][0] = ktn[r][0], kt[r][1] = ktn[r][1];
        }
        ke = ken;
        ve = ven;
        for (int kk = 0; kk < 8; ++kk) {
          v8[kk] = v8n[kk];
          if (kRot) vw[kk] = vwn[kk];
        }
      }
    }

    float l_tot = l_run + __shfl_xor(l_run, 16, 64);
    l_tot += __shfl_xor(l_tot, 32, 64);

    // publish this wave's state: lane (g, c) holds O[g][32c + 8i + j] = o[j][i]
    if (c == 0) {
      cmb.m[wave][g] = m_run;
      cmb.l[wave][g] = l_tot;
    }
    if (kI4) {
      // add the corrections of the column; row 4c + i of slot j is dim
      // 64 (j / 4) + 32 (c % 2) + 8i + 4 (c / 2) + j % 4
      const float cor0 = cb[0][0], cor1 = cb[1][0];
      for (int i = 0; i < 4; ++i) {
        float* dst = (float*)&wave_lds[wave][0] + g * kD + 32 * (c & 1) + 8 * i + 4 * (c >> 1);
        *(f32x4*)dst = f32x4{o[0][i] + cor0, o[1][i] + cor0, o[2][i] + cor0, o[3][i] + cor0};
        *(f32x4*)(dst + 64) = f32x4{o[4][i] + cor1, o[5][i] + cor1, o[6][i] + cor1, o[7][i] + cor1};
      }
    } else {
      for (int i = 0; i < 4; ++i) {
        float* dst = (float*)&wave_lds[wave][0] + g * kD + 32 * c + 8 * i;
        *(f32x4*)dst = f32x4{o[0][i], o[1][i], o[2][i], o[3][i]};
        *(f32x4*)(dst + 4) = f32x4{o[4][i], o[5][i], o[6][i], o[7][i]};
      }
    }
    __syncthreads();

    // combine the four waves; thread e covers (head e / 128, dim e % 128)
    const int64_t w0 = worker_of(a, seg_first, total, W), w1 = worker_of(a, seg_end - 1, total, W);
    const bool single = w0 == w1;
    const int64_t s = (int64_t)b * a.Hkv + kh;
    for (int e = tid; e < a.G * kD; e += blockDim.x) {
      const int gg = e / kD, d = e % kD;
      float M = -INFINITY;
      for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, cmb.m[ww][gg]);
      float Lsum = 0.f, acc = 0.f;
      for (int ww = 0; ww < kWaves; ++ww) {
        const float sc = __builtin_amdgcn_exp2f(cmb.m[ww][gg] - M);  // idle waves: m = -inf -> 0
        Lsum += sc * cmb.l[ww][gg];
        acc += sc * ((const float*)&wave_lds[ww][0])[gg * kD + d];
      }
      if (single) {
        a.out[((int64_t)b * a.Hq + (int64_t)kh * a.G + gg) * kD + d] = (uint16_t)f32_to_bf16_bits(acc / Lsum);
      } else {
        float* P = a.part + (((int64_t)w + s) * a.G + gg) * kPieceStride;
        if (a.inline_merge) {  // read by a workgroup of this launch
          if (d == 0) {
            part_store(P, M);
            part_store(P + 1, Lsum);
          }
          part_store(P + 4 + d, acc);
        } else {  // read by decode_merge_kernel
          if (d == 0) {
            P[0] = M;
            P[1] = Lsum;
          }
          P[4 + d] = acc;
        }
      }
    }
    // a segment over several workgroups: the last of them to finish merges the pieces
    if (!single && a.inline_merge && arrive_last(a, s, (int)(w1 - w0 + 1), cmb)) merge_segment(a, b, kh, s, w0, w1);
    __syncthreads();  // cmb is reused by the next piece
    t = piece_end;
  }

  // EMA_STEP_ADVANCE with the merge in this kernel: the grid's last workgroup moves each
  // sequence's offset past the row the step wrote; every other workgroup has finished
  // reading the offsets by then.
  if (a.adv && a.inline_merge && arrive_last(a, (int64_t)a.B * a.Hkv, (int)gridDim.x, cmb)) {
    for (int i = threadIdx.x; i < a.B; i += blockDim.x) {
      const int o = a.adv[i];
      if (o >= 0 && o < INT32_MAX && (a.rot || o < a.cap)) a.adv[i] = o + 1;
    }
  }
}

// The merge of full grids, after the kernel boundary: one thread per (segment, head, dim)
// runs merge_segment's fold for its element. With EMA_STEP_ADVANCE it also moves each
// sequence's offset past the row the step wrote (thread b for sequence b): decode_kernel,
// which reads the offsets, has finished, and no thread here reads them (segment sizes come
// from the tile prefix).
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
  // 32-bit index arithmetic (per-lane 64-bit divisions are long emulations): the grid is
  // segments * G * kD < 2^31 threads (at most 32767 segments, G <= 16)
  const uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
  if (a.adv && e < (uint32_t)a.B) {
    const int o = a.adv[e];
    if (o >= 0 && o < INT32_MAX && (a.rot || o < a.cap)) a.adv[e] = o + 1;
  }
  const uint32_t per_seg = (uint32_t)a.G * kD;
  const uint32_t s = e / per_seg;
  if (s >= (uint32_t)(a.B * a.Hkv)) return;
  const uint32_t r = e - s * per_seg;
  const int gg = (int)(r / kD), d = (int)(r % kD);
  const int b = (int)(s / (uint32_t)a.Hkv), kh = (int)(s - (uint32_t)b * a.Hkv);
  const int64_t total = a.hdr[a.B];  // tile prefix published by decode_kernel
  const int nb = (a.hdr[b + 1] - a.hdr[b]) / a.Hkv;  // tiles per kv head of sequence b
  if (nb == 0 || total == 0) return;
  const int W = active_workers(total, a.W);
  const int64_t seg_first = a.hdr[b] + (int64_t)kh * nb;
  const int64_t w0 = worker_of(a, seg_first, total, W);
  const int64_t w1 = worker_of(a, seg_first + nb - 1, total, W);
  if (w0 == w1) return;  // written directly by decode_kernel
  // (uniform across a workgroup when a segment has at least 256 threads, G >= 2)
  if (w1 - w0 >= 8) merge_element<false, 16>(a, b, kh, s, w0, w1, gg, d);
  else merge_element<false, 8>(a, b, kh, s, w0, w1, gg, d);
}

}  // namespace

DecodePlan plan_decode(int B, int Hq, int Hkv, int D, int max_len) {
  DecodePlan p;
  p.workers = split_plan_workers(B, Hkv, max_len);
  p.segments = B * Hkv;
  const int G = Hkv > 0 ? Hq / Hkv : 1;
  p.part_bytes = (uint64_t)(p.workers + p.segments) * G * kPieceStride * sizeof(float);
  return p;
}

constexpr uint64_t kHeaderBytes = ((kMaxB + 1) * sizeof(int32_t) + 255) & ~(uint64_t)255;

uint64_t decode_workspace_bytes(const DecodePlan& p) { return kDecodeCounterBytes + kHeaderBytes + p.part_bytes; }

// Grids of at most one workgroup per CU are latency-bound: the merge of their split
// segments runs inside the kernel (one launch per call), and a bf16 cache's tiles come by
// LDS-DMA of whole rows (kDma). Fuller grids merge in decode_merge_kernel, whose launch is
// small beside theirs and which keeps the arrival round trips out of their workgroups'
// slices, and load their tiles straight into registers.
constexpr int kInlineMergeMaxWorkers = 256;

int32_t launch_decode(hipStream_t s, const void* q, const ema_kvcache_desc& c, const int32_t* len,
                      int Hq, float scale, void* out, void* ws, const DecodePlan& plan, const FusedPre* fused) {
  if (c.head_dim != kD)
    return set_error(EMA_ERR_UNSUPPORTED, "ema_decode_attention: head_dim %d not supported (128)", c.head_dim);
  if (c.batch > kMaxB)
    return set_error(EMA_ERR_UNSUPPORTED, "ema_decode_attention: batch %d exceeds %d", c.batch, kMaxB);
  if ((int64_t)c.batch * c.n_kv_heads + 1 > kDecodeCounterSlots)
    return set_error(EMA_ERR_UNSUPPORTED, "ema_decode_attention: batch x kv heads %lld exceeds %d",
                     (long long)c.batch * c.n_kv_heads, kDecodeCounterSlots - 1);
  const int G = Hq / c.n_kv_heads;
  if (G > 16)
    return set_error(EMA_ERR_UNSUPPORTED, "ema_decode_attention: %d query heads per kv head exceeds 16", G);
  DecodeArgs a;
  a.q = (const uint16_t*)q;
  a.k = (const uint16_t*)c.k;
  a.v = (const uint16_t*)c.v;
  a.len = len;
  a.out = (uint16_t*)out;
  a.cnt = (int32_t*)ws;
  a.hdr = (int32_t*)((char*)ws + kDecodeCounterBytes);
  a.part = (float*)((char*)ws + kDecodeCounterBytes + kHeaderBytes);
  a.inline_merge = plan.workers <= kInlineMergeMaxWorkers;
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
  // lengths are clamped to the capacity, so the tile count is at most max_tiles: the
  // kernels keep their tile prefix in 32 bits, and the split's products w * total too when
  // they fit
  const int64_t max_tiles = (int64_t)c.batch * c.n_kv_heads * ((c.capacity + kTile - 1) / kTile);
  if (max_tiles >= INT32_MAX)
    return set_error(EMA_ERR_UNSUPPORTED, "ema_decode_attention: %lld tiles of %d positions exceed 2^31 - 1",
                     (long long)max_tiles, kTile);
  a.narrow = split_narrow(max_tiles, plan.workers);
  a.fused = fused != nullptr;
  a.rot = (c.flags & EMA_KV_ROTATING) != 0;
  a.qkv = fused ? (const uint16_t*)fused->qkv : nullptr;
  // null norm weights (EMA_PRE_NO_NORM): the kernel still reads 128 values, from the qkv rows
  a.qw = fused ? (const uint16_t*)(fused->q_norm_w ? fused->q_norm_w : fused->qkv) : nullptr;
  a.kw = fused ? (const uint16_t*)(fused->k_norm_w ? fused->k_norm_w : fused->qkv) : nullptr;
  a.off = fused ? fused->offsets : nullptr;
  a.adv = fused && (fused->flags & EMA_STEP_ADVANCE) ? fused->offsets : nullptr;
  a.eps = fused ? fused->eps : 0.f;
  a.log2_theta = fused ? log2f(fused->theta) : 0.f;
  a.flags = fused ? fused->flags : 0u;
  a.kexp = (const int8_t*)c.k_exp;
  a.vexp = (const int8_t*)c.v_exp;
  a.ks = (uint32_t*)c.k_scales;
  a.kb = (uint32_t*)c.k_biases;
  a.vs = (uint32_t*)c.v_scales;
  a.vb = (uint32_t*)c.v_biases;
  const bool fp8 = c.dtype == EMA_DTYPE_FP8_E4M3;
  const bool i4 = c.dtype == EMA_DTYPE_INT4_AFFINE;
  const bool tail = fp8 && c.n_rot != 0;
  // the bf16 and int4 kernels address a (sequence, kv head) plane of the cache through a
  // 32-bit buffer range
  const int64_t plane = i4 ? (int64_t)c.capacity * (c.stride_pos / 2) : fp8 ? 0 : (int64_t)c.capacity * c.stride_pos * 2;
  if (plane > (int64_t)UINT32_MAX)
    return set_error(EMA_ERR_UNSUPPORTED, "ema_decode_attention: %lld bytes per (sequence, kv head) exceed 2^32",
                     (long long)plane);
  // plain fp8 rows through LDS-DMA slots: whole 16-byte exponent pieces (a capacity that is
  // a multiple of 8) and a plane within a 32-bit buffer range; otherwise straight loads
  const bool f8dma = fp8 && !tail && c.capacity % 8 == 0 && (int64_t)c.capacity * c.stride_pos <= (int64_t)UINT32_MAX;
  const dim3 grid(plan.workers), block(kWaves * 64);
  if (a.fused && tail) {
    // The fused step over FP8 rows with a RoPE tail runs as two kernels: the fused kernel
    // has no registers to spare for the tail's wider rows (it spilled and ran at 155 us
    // against 69 us at the batch-32 shape). The pre-attention kernel writes the new row and
    // puts q in `out` (q [B, Hq, 1, D] and out [B, Hq * D] share one layout); the decode
    // kernel then reads q there and takes its lengths from the offsets (a.fused). Every
    // workgroup reads the q of a (sequence, kv head) segment before it arrives, and out of
    // that segment is written only after the last arrival (or by decode_merge_kernel), so
    // no q is overwritten before it is read.
    int32_t rc = launch_pre_attention(s, fused->qkv, fused->q_norm_w, fused->k_norm_w, fused->eps, fused->theta,
                                      fused->offsets, c.batch, 1, Hq, c.n_kv_heads, kD,
                                      fused->flags & ~(uint32_t)EMA_STEP_ADVANCE, out, c);
    if (rc) return rc;
    a.q = (const uint16_t*)out;
    hipLaunchKernelGGL((decode_kernel<false, true, false, true>), grid, block, 0, s, a);
  } else if (a.fused && i4) hipLaunchKernelGGL((decode_kernel<true, false, true>), grid, block, 0, s, a);
  else if (i4) hipLaunchKernelGGL((decode_kernel<false, false, true>), grid, block, 0, s, a);
  else if (a.fused && f8dma) hipLaunchKernelGGL((decode_kernel<true, true, false, false, true>), grid, block, 0, s, a);
  else if (a.fused && fp8) hipLaunchKernelGGL((decode_kernel<true, true>), grid, block, 0, s, a);
  else if (a.fused && a.inline_merge) hipLaunchKernelGGL((decode_kernel<true, false, false, false, true>), grid, block, 0, s, a);
  else if (a.fused) hipLaunchKernelGGL((decode_kernel<true, false>), grid, block, 0, s, a);
  else if (tail) hipLaunchKernelGGL((decode_kernel<false, true, false, true>), grid, block, 0, s, a);
  else if (f8dma) hipLaunchKernelGGL((decode_kernel<false, true, false, false, true>), grid, block, 0, s, a);
  else if (fp8) hipLaunchKernelGGL((decode_kernel<false, true>), grid, block, 0, s, a);
  else if (a.inline_merge) hipLaunchKernelGGL((decode_kernel<false, false, false, false, true>), grid, block, 0, s, a);
  else hipLaunchKernelGGL((decode_kernel<false, false>), grid, block, 0, s, a);
  int32_t rc = check_hip(hipGetLastError(), "ema_decode_attention launch");
  if (rc || a.inline_merge || (plan.workers == 1 && !a.adv)) return rc;
  const int64_t threads = (int64_t)plan.segments * G * kD;
  // 64-thread workgroups: the same threads over more CUs (8 x 32k rows: 0.2-0.3 us faster
  // per call than 256-thread workgroups; the batch-32 step is unchanged)
  hipLaunchKernelGGL(decode_merge_kernel, dim3((unsigned)((threads + 63) / 64)), dim3(64), 0, s, a);
  return check_hip(hipGetLastError(), "ema_decode_attention merge launch");
}

}  // namespace ema
