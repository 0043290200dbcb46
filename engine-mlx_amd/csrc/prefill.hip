// Causal / chunked-prefill flash attention over the static KV cache, gfx950.
//
// Replaces MlxCtx::sdpa(..., causal=true) (crates/mlx-ffi/src/ops/real/blas.rs:82-101)
// as called by the prefill (crates/serve/src/forward_qwen3.rs:150) and by
// attend_and_project (crates/ops/src/attention.rs:162-177, via
// crates/attention/src/gqa.rs:100-106). MLX "causal" aligns the query block
// to the end of the key range: query i of a chunk that starts at cache
// position q_off sees keys j <= q_off + i.
//
// Work split: one workgroup of 8 waves per CU owns 128 query rows of one head. Its key
// range is cut in two halves at a 64-key block boundary; wave group 0 (waves 0-3)
// attends over the first half and group 1 (waves 4-7) over the second, each wave over
// 32 rows, each group streaming its own 64-key K/V blocks through its own
// double-buffered LDS. The two partial (o, m, l) states of a row meet in LDS at the end.
// Halving the key range halves the longest causal work item, and workgroups are
// dispatched heaviest first, so the short ones fill in behind the long ones. With two or
// more query blocks per CU, each workgroup owns a heavy and a light block of one head and
// runs them as one block stream per group (prefill_kernel<*, true>, described there).
//
// Both contractions run on MFMA 32x32x16 (bf16 in, f32 accumulate), in the transposed
// form that keeps the softmax lane-local:
//   S^T[key, q] = K[key, :] . Q^T[:, q]   A = K rows (ds_read_b128), B = Q^T in registers
//   O^T[d, q]  += V^T[d, key] P^T[key, q] A = V^T via ds_read_b64_tr_b16 (transposing
//                                          LDS read), B = P^T (the S^T accumulators
//                                          after exp, unmoved)
// Each lane owns one query row's scores, row-sum share and 64 output accumulators.
//
// Ping-pong: the two waves on each SIMD belong to different groups, and the groups run
// half a block out of phase, separated by workgroup barriers. In one phase group 0 issues
// its matrix step (PV of block j-1 and QK of block j, 32 MFMAs) while group 1 runs the
// softmax of its block (VALU, exp) and issues the global-to-LDS loads of its next tiles;
// in the next phase the roles swap. The matrix pipe and the vector pipe of a SIMD are fed
// by different waves throughout.
#include "ema_common.hpp"
#include "ema_schedule.hpp"

namespace ema {
namespace {

constexpr int kD = 128;
constexpr int kBM = 128;          // query rows per workgroup
constexpr int kBN = 64;           // keys per block
constexpr int kGroupThreads = 256;  // 4 waves per key-range group
constexpr int kThreads = 2 * kGroupThreads;
// LDS tiles hold 64 unpadded 256-byte rows. The 16-byte chunks of a row are XOR-swizzled
// so that the MFMA operand reads hit distinct banks: chunk p of K row r holds column
// chunk p ^ (r & 15) (the b128 reads of 16 rows at one chunk spread over all banks), and
// chunk p of V row r holds column chunk p ^ 4(r & 3) (the 4 rows of a transposed read
// land in 4 different 64-byte bank groups).
constexpr int kTile = kBN * kD;                    // elements of one K or V tile (16 KB)
constexpr int kGroupElems = 4 * kTile;              // one group: K0 K1 V0 V1
constexpr int kQElems = kBM * kD;                   // the workgroup's Q rows (32 KB)
constexpr int kLdsBytes = (2 * kGroupElems + kQElems) * 2;  // 163840 B: one workgroup per CU

struct PrefillArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const int32_t* q_off;
  uint16_t* out;
  int64_t sb, sh, sp;
  float qk_scale;  // scale * log2(e), applied to Q
  int B, Hq, Hkv, G, T, cap, nqb;
  int paired;  // each workgroup runs query blocks qb and nqb-1-qb of one head, in turn
  uint32_t flags;
};

typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
// compile-time choice of the softmax step's masking code
struct MaskOn { static constexpr bool value = true; };
struct MaskOff { static constexpr bool value = false; };
// the segment of a block stream that a step's block lies in, when the caller knows it
// (paired workgroups: segment A, the light rows, then segment B, the heavy rows)
struct SegAny { static constexpr int value = 0; };
struct SegA { static constexpr int value = 1; };
struct SegB { static constexpr int value = 2; };
typedef __attribute__((address_space(3))) void lds_void;

// Raw buffer resource (V#) over `bytes` bytes from `base`: stride 0, gfx9 dword3 with a
// 32-bit data format. Loads at offsets at or past `bytes` return zeros.
// Every argument is wave-uniform; readfirstlane keeps the words in scalar registers for the
// asm operands that take them.
__device__ __forceinline__ u32x4 buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t addr = (uint64_t)base;
  return u32x4{(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)addr),
               (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(addr >> 32) & 0xffffu),
               (uint32_t)__builtin_amdgcn_readfirstlane(bytes), 0x00020000u};
}

// 16 bytes per lane from buffer offset `voff` + 1024 * I straight into LDS at lds_addr +
// 1024 * I + 16 * lane (buffer_load_dwordx4 ... lds; the LDS base goes through M0, and the
// instruction offset moves the memory and the LDS address alike). Issued as asm so the
// compiler does not track it: the caller orders it with explicit vmcnt waits before the
// barrier that publishes the tile, instead of the compiler draining every load in flight
// at each barrier and before each LDS read.
template <int I>
__device__ __forceinline__ void dma16(u32x4 rsrc, uint32_t voff, uint32_t lds_addr) {
  // lds_addr is wave-uniform; readfirstlane keeps it in a scalar register for M0
  // s_nop 0: the DMA reads M0 no earlier than one wait state after the SALU write, a wait
  // the compiler inserts only for the LDS-DMAs it emits itself. (Its SGPR operands need five
  // after a VALU write; check_hazards.py fails the build if the compiler places one closer.)
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen offset:%3 lds"
               :
               : "v"(voff), "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(lds_addr)), "i"(1024 * I)
               : "memory", "m0");
}
// Block offset that no buffer range reaches (ranges stay below 2^31 bytes, and a per-lane
// offset added to it stays below 2^32): the load returns zeros and touches no memory.
constexpr uint32_t kNoRow = 0xF0000000u;

// Elementwise maximum of three f16 pairs (v_pk_maximum3_f16, NaN-propagating).
__device__ __forceinline__ uint32_t pk_max3_f16(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t r;
  asm("v_pk_maximum3_f16 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// kRot: rotating cache (EMA_KV_ROTATING). The keys of a sequence are the positions
// [base, q_off + T) with base = max(0, q_off + T - cap), position p in row p % cap; the
// kernel works on key indices c = p - base (q_off is taken relative to base), so all its
// causal and range logic is that of a static cache, and only the loads map c to its row.
//
// kPair: the workgroup owns a heavy query block and a light one of the same head (the
// light block's key range is a prefix of the heavy block's). Group 0 streams the light
// rows over all their key blocks and then the heavy rows over the first key blocks of
// the heavy range; group 1 streams the heavy rows over the rest, so both groups take
// half of the pair's key blocks in one pipeline each: one prologue and one merge per
// workgroup instead of two, and no refill of the pipeline between the blocks. The light
// rows are complete when group 0 leaves them; group 0 stores them on its own. A middle
// block paired with itself (odd block count) runs as a heavy block with no light rows.
template <bool kRot, bool kPair>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_kernel(PrefillArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int g = wave >> 2;         // key-range group
  const int wq = wave & 3;         // row tile of the wave inside the workgroup
  // Grid mapping (prefill_item): XCD-local (batch, kv head) groups, heaviest query
  // blocks first, and with two workgroups' worth of query blocks or more per CU a pair
  // per workgroup -- the heavy block nqb-1-p, then the light one p of the same head --
  // which balances the causal work per workgroup and pays one launch per pair.
  const PrefillItem item = prefill_item(blockIdx.x, gridDim.x, a.B, a.Hkv, a.G, a.nqb, kPair ? 1 : 0);
  const int b = item.b;
  const int h = item.h;
  const int kh = item.kh;
  const int q_off_arg = a.q_off[b];  // (a scalar load, waited for after the Q loads are issued)
  const int qb_h = item.qb_first;
  const bool has_light = kPair && item.qb_second != qb_h;
  const int qb_l = has_light ? item.qb_second : qb_h;
  const int row0 = qb_h * kBM;                    // first query row of the heavy block
  const int row0A = qb_l * kBM;                   // and of the light block

  // Prologue, part 1: the workgroup's Q rows go to LDS before anything depends on q_off.
  // Global -> LDS without registers (buffer_load_dwordx4 ... lds): one instruction moves
  // 1 KB, lane l's 16 bytes landing at byte 16l of the destination, i.e. 4 rows of 256 B;
  // wave w moves rows 16w .. 16w+15, chunk p of row r from chunk p ^ (r & 15). Rows past
  // T arrive as zeros.
  const int r4 = lane >> 4, p16 = lane & 15;  // row within the 4, chunk position in the row
  auto load_q = [&](int qrow0, uint32_t dst) __attribute__((always_inline)) {
    const int qrows = a.T - qrow0 < kBM ? a.T - qrow0 : kBM;
    const u32x4 r = buffer_rsrc(a.q + (((int64_t)b * a.Hq + h) * a.T + qrow0) * kD, (uint32_t)qrows * kD * 2);
    for (int i = 0; i < 4; ++i) {
      const uint32_t row = (uint32_t)(16 * wave + 4 * i + r4);
      dma16<0>(r, row * kD * 2 + (uint32_t)((p16 ^ (4 * i + r4)) * 16), dst + 4 * i * kD * 2);
    }
  };
  // The heavy rows in the Q area for the whole stream. The light rows' Q (pairs): rows
  // 0-63 in group 0's second V tile, rows 64-127 in group 1's; those tiles are first
  // loaded by the groups' first softmax steps, after group 0 has read its Q^T operand
  // from them.
  uint16_t* const Qs = lds + 2 * kGroupElems;
  auto light_q = [&](int r) __attribute__((always_inline)) { return lds + (r >> 6) * kGroupElems + 3 * kTile + (r & 63) * kD; };
  load_q(row0, (uint32_t)(uintptr_t)(lds_void*)(Qs + 16 * wave * kD));
  if (has_light) load_q(row0A, (uint32_t)(uintptr_t)(lds_void*)light_q(16 * wave));

  int q_off = q_off_arg < 0 ? 0 : q_off_arg;
  int key_base = 0;  // absolute position of key index 0 (rotating cache; n_tokens <= cap)
  if (kRot) {
    key_base = q_off + a.T - a.cap;
    key_base = key_base < 0 ? 0 : key_base;
    q_off -= key_base;
  }
  int kv_len = q_off + a.T;
  kv_len = kv_len > a.cap ? a.cap : kv_len;
  const bool causal = a.flags & EMA_PREFILL_CAUSAL;
  int kv_begin = (a.flags & EMA_PREFILL_CHUNK_ONLY) ? q_off : 0;
  kv_begin = kv_begin > kv_len ? kv_len : kv_begin;
  const int blk_begin = kv_begin / kBN;
  // 64-key blocks attended by query block qb: [blk_begin, blk_begin + blocks_of(qb))
  auto blocks_of = [&](int qb) __attribute__((always_inline)) {
    int wg_end = kv_len;
    if (causal) {
      const int lim = q_off + qb * kBM + kBM;     // its last row sees keys < lim
      wg_end = lim < wg_end ? lim : wg_end;
    }
    const int blk_end = (wg_end + kBN - 1) / kBN;
    return blk_end > blk_begin ? blk_end - blk_begin : 0;
  };

  // The wave's block stream: segment A (group 0 of a pair: the light rows over all their
  // blocks), then segment B (the heavy rows: the first n0 - n1 of their blocks in group 0,
  // the rest in group 1). Without a light block group 0 takes the first half.
  const int nblk_h = blocks_of(qb_h);
  const int nblk_l = has_light ? blocks_of(qb_l) : 0;   // <= nblk_h
  const int n0 = prefill_group0_blocks(nblk_h, nblk_l);   // blocks of group 0
  const PrefillStream ps = prefill_stream(g, nblk_h, nblk_l);
  const int n1 = kPair ? ps.n1 : 0;                       // segment A
  const int gbA = blk_begin;
  const int gbB = blk_begin + ps.gbB;                     // first block of segment B
  const int nB = ps.nB;
  const int ng = n1 + nB;                                 // blocks of this wave's stream
  // stream block j: in segment A (tag SegAny: decided from j), and its absolute block index
  auto in_a = [&](int j, auto seg) __attribute__((always_inline)) {
    constexpr int kSeg = decltype(seg)::value;
    return kSeg == 1 || (kSeg == 0 && kPair && j < n1);
  };
  const int offB = gbB - n1;
  auto blk_of = [&](int j) __attribute__((always_inline)) { return j + (in_a(j, SegAny{}) ? gbA : offB); };

  const int hh = lane >> 5;                       // which half of the k slots
  // the wave's first query row in either segment; lane row: + (lane & 31), causal limit
  // key <= that
  const int wfaB = q_off + row0 + 32 * wq, wfaA = q_off + row0A + 32 * wq;
  auto wfa_of = [&](int j, auto seg) __attribute__((always_inline)) { return in_a(j, seg) ? wfaA : wfaB; };

  uint16_t* const Ks = lds + g * kGroupElems;     // this group's K tiles: buffer i at Ks + i * kTile
  uint16_t* const Vs = Ks + 2 * kTile;            // and V tiles

  // K/V of this (batch, kv head) through buffer loads. A resource covers the rows below
  // kv_len, so rows past the valid length read as zeros (finite, and masked out) without
  // per-lane clamping. Static cache: each tile load gets a resource of its own whose base
  // is the tile's first row (scalar arithmetic), so the per-lane offsets never change.
  // Rotating cache: one resource per tensor, the block's offset added to the per-lane
  // offsets (rows may wrap around the ring).
  const char* Kg = (const char*)(a.k + (int64_t)b * a.sb + (int64_t)kh * a.sh);
  const char* Vg = (const char*)(a.v + (int64_t)b * a.sb + (int64_t)kh * a.sh);
  const uint32_t row_bytes = (uint32_t)a.sp * 2;
  const uint32_t kv_bytes = (uint32_t)kv_len * row_bytes;
  const u32x4 k_rsrc = buffer_rsrc(Kg, kv_bytes);
  const u32x4 v_rsrc = buffer_rsrc(Vg, kv_bytes);
  // resource of the tile at byte offset ob of `base` (blk_off: below kv_bytes, or kNoRow
  // for an empty range that reads all zeros)
  auto tile_rsrc = [&](const char* base, uint32_t ob) __attribute__((always_inline)) {
    const bool none = ob == kNoRow;
    return buffer_rsrc(base + (none ? 0u : ob), none ? 0u : kv_bytes - ob);
  };

  // Global -> LDS without registers (buffer_load_dwordx4 ... lds): one instruction moves
  // 1 KB, lane l's 16 bytes landing at byte 16l of the destination, i.e. 4 tile rows.
  // Wave wq of the group moves rows 16wq .. 16wq+15 (4 instructions per tile, the i-th
  // at instruction offset 1024 i); the per-lane source offsets below apply the swizzle,
  // have that instruction offset taken out (row >= 4i and row_bytes >= 256 keep them
  // non-negative) and stay the same for every block.
  uint32_t koff[4], voff[4];
  for (int i = 0; i < 4; ++i) {
    const uint32_t row = (uint32_t)(16 * wq + 4 * i + r4);
    koff[i] = row * row_bytes + (uint32_t)((p16 ^ (4 * i + r4)) * 16) - 1024u * i;
    voff[i] = row * row_bytes + (uint32_t)((p16 ^ (4 * r4)) * 16) - 1024u * i;
  }
  // byte offset of block j of this group, or kNoRow past the group's range (its loads
  // then fill the tile with zeros that nothing reads, which keeps the issue count of a
  // step fixed). Rotating cache: the row of the block's first key, and wrap_rows, the
  // number of its rows before the ring's end (rows past it are cap rows back).
  auto blk_off = [&](int j) __attribute__((always_inline)) {
    if (j >= ng) return kNoRow;
    if (kRot) return (uint32_t)((key_base + blk_of(j) * kBN) % a.cap) * row_bytes;
    return (uint32_t)(blk_of(j) * kBN) * row_bytes;
  };
  auto wrap_rows = [&](int j) __attribute__((always_inline)) {
    return kRot && j < ng ? a.cap - (key_base + blk_of(j) * kBN) % a.cap : kBN;
  };
  const uint32_t ring_bytes = (uint32_t)a.cap * row_bytes;
  auto tile_dst = [&](const uint16_t* tile) __attribute__((always_inline)) {
    return (uint32_t)(uintptr_t)(lds_void*)(tile + 16 * wq * kD);
  };
  // one of the 4 instructions of a tile load (spread over the softmax step so the four
  // waves of a group do not queue 32 KB at the address unit at once)
  // r: the tensor's resource (rotating cache) or the tile's (static cache: off_blk is used
  // only to empty this lane's row when it is kNoRow and `lane_rows` is set)
  auto dma_part = [&](const u32x4 r, uint32_t off_blk, const uint32_t* off, uint32_t dst, int i, int wrap,
                      bool lane_rows = false) __attribute__((always_inline)) {
    if (kRot) {
      // true offsets (the instruction offset unused, the LDS address moved through M0), so
      // a row past the ring's end, moved cap rows back, never goes below zero
      uint32_t o = off[i] + 1024u * i + off_blk;
      if (16 * wq + 4 * i + r4 >= wrap) o -= ring_bytes;
      dma16<0>(r, o, dst + 1024u * i);
      return;
    }
    const uint32_t o = lane_rows && off_blk == kNoRow ? kNoRow : off[i];
    switch (i) {
      case 0: dma16<0>(r, o, dst); break;
      case 1: dma16<1>(r, o, dst); break;
      case 2: dma16<2>(r, o, dst); break;
      default: dma16<3>(r, o, dst); break;
    }
  };
  auto dma = [&](const char* tensor, const u32x4 tensor_r, int j, const uint32_t* off, const uint16_t* tile)
      __attribute__((always_inline)) {
    const uint32_t ob = blk_off(j), dst = tile_dst(tile);
    const u32x4 r = kRot ? tensor_r : tile_rsrc(tensor, ob);
    const int wrap = wrap_rows(j);
    const int base = blk_of(j) * kBN;
    if (j < ng && base < kv_begin) {
      // first block of a chunk-only window: rows before kv_begin are outside the
      // attended range; an out-of-range offset makes them arrive as zeros, so whatever
      // the cache holds there (even NaN) cannot reach the masked products
      for (int i = 0; i < 4; ++i) {
        const int row = base + 16 * wq + 4 * i + r4;
        dma_part(r, row < kv_begin ? kNoRow : ob, off, dst, i, row < kv_begin ? kBN : wrap, true);
      }
    } else {
      for (int i = 0; i < 4; ++i) dma_part(r, ob, off, dst, i, wrap);
    }
  };
  auto load_k = [&](int j) __attribute__((always_inline)) { dma(Kg, k_rsrc, j, koff, Ks + (j & 1) * kTile); };
  auto load_v = [&](int j) __attribute__((always_inline)) { dma(Vg, v_rsrc, j, voff, Vs + (j & 1) * kTile); };

  // Online softmax state of this lane's row, in the log2 domain. The accumulators hold
  // o and l relative to the base m_use (p = 2^(s - m_use)); the score MFMA chains start
  // from -m_use (each softmax step leaves it in the score registers once it has read the
  // scores), so they yield s - m_use directly. m_use only changes on the slow path of the
  // softmax step.
  float m_use = 0.f;
  bool seen = false;      // m_use is this row's running max (some score was finite)
  bool all_seen = false;  // wave-uniform: every row of the wave is seen
  bool rescale = false;   // wave-uniform: o and the row sums are to be scaled before the next PV
  float o_scale = 1.f;    // factor of this lane's row
  f32x16 o[4], sc[2];
  // Row sums of P, accumulated on the matrix pipe by a 16x16x32 MFMA whose A operand selects
  // (B = the P^T chunk of a PV step: lane l holds row l % 32, so column n of the 16-wide view
  // holds rows n (lanes n, n+32: k 0-7, 16-23) and n+16 (lanes n+16, n+48: k 8-15, 24-31)).
  // A row 0 is one over k 0-7 and 16-23, row 1 over k 8-15 and 24-31, the rest zero, so
  // lane n < 16 accumulates row n's sum in lsum[0] and row n+16's in lsum[1]. These sums are
  // taken over the bf16-rounded P that PV multiplies, and VALU dot products would cost about
  // 40 cycles each beside the other wave's MFMAs.
  f32x4 lsum = {0.f, 0.f, 0.f, 0.f};
  const bool sel = ((lane & 15) == 0 && ((lane >> 4) & 1) == 0) || ((lane & 15) == 1 && ((lane >> 4) & 1) == 1);
  const uint32_t sel_w = sel ? 0x3F803F80u : 0u;
  const bf16x8 sum_sel = as_bf16x8(u32x4{sel_w, sel_w, sel_w, sel_w});
  for (int dt = 0; dt < 4; ++dt)
    for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
  for (int kt = 0; kt < 2; ++kt)
    for (int i = 0; i < 16; ++i) sc[kt][i] = 0.f;
  u32x4 pw[4] = {};  // P^T of the last softmax step as bf16 pairs, for the next PV
  bf16x8 qop[8];     // Q^T operand (set after the prologue)

  // K operand reads: row (lane & 31) (+32 for sub-tile 1), column chunk 2s + hh, stored
  // at chunk (2s + hh) ^ (lane & 15)
  const int k_lane = (lane & 31) * kD + 8 * (hh ^ (lane & 1));
  const int k_x = 16 * ((lane & 15) >> 1);            // element offset, xored with 16s
  // V^T operand reads (per 16-lane group): rows tr_row + 16*st_half + 8u + 32*kt,
  // columns 4(s16 & 3) + 16(grp & 1) + 32dt, stored at column chunk ^ 4(s16 >> 2)
  const int grp = lane >> 4, s16 = lane & 15;
  const int tr_row = 4 * (grp >> 1) + (s16 >> 2);
  int v_col[4];
  for (int dt = 0; dt < 4; ++dt) v_col[dt] = tr_row * kD + 16 * (grp & 1) + 4 * (s16 & 3) + 32 * (dt ^ (s16 >> 2));

  // Some row of the wave attends to a key of block j (the last row's limit is the first's + 31).
  auto active = [&](int j, auto seg) __attribute__((always_inline)) {
    return !causal || (j + (in_a(j, seg) ? gbA : offB)) * kBN <= wfa_of(j, seg) + 31;
  };
  // Block j holds keys outside [kv_begin, kv_len) or above the causal limit of some row
  // of this wave. Inside a segment, for its blocks after the first, this holds exactly
  // from the segment's block j_mask on.
  auto need_mask = [&](int j, auto seg) __attribute__((always_inline)) {
    const int kbase = (j + (in_a(j, seg) ? gbA : offB)) * kBN;
    return kbase < kv_begin || kbase + kBN > kv_len || (causal && kbase + kBN - 1 > wfa_of(j, seg));
  };
  // first block of a segment (starting at absolute block gb, rows from wave_first) that
  // needs a mask, at least 1; and the blocks of its n that the wave attends to
  auto seg_mask = [&](int gb, int wave_first) __attribute__((always_inline)) {
    int jm = kv_len / kBN - gb;  // first block reaching past kv_len
    if (causal) {
      const int jc = (wave_first + 1) / kBN - gb;  // first block reaching past row 0's limit
      jm = jc < jm ? jc : jm;
    }
    return jm < 1 ? 1 : jm;
  };
  auto seg_act = [&](int gb, int wave_first, int n) __attribute__((always_inline)) {
    if (!causal) return n;
    const int last = (wave_first + 31) / kBN - gb + 1;
    return last < 0 ? 0 : (last < n ? last : n);
  };

  // Matrix step j: O += V^T P^T for block j-1, then S^T = K Q^T - m_use for block j. A base
  // change of the softmax step before is applied to o first.
  auto pv = [&](int jb) __attribute__((always_inline)) {
    const uint16_t* Vt = Vs + (jb & 1) * kTile;
    for (int st = 0; st < 4; ++st) {
      const int kt = st >> 1, q2 = st & 1;
      const bf16x8 pop = as_bf16x8(pw[st]);
      const int rbase = (32 * kt + 16 * q2) * kD;
      for (int dt = 0; dt < 4; ++dt) {
        const uint16_t* p0 = Vt + rbase + v_col[dt];
        const uint16_t* p1 = p0 + 8 * kD;
        const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p0);
        const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p1);
        typedef short s16x8 __attribute__((ext_vector_type(8)));
        const s16x8 av = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        o[dt] = mfma32(__builtin_bit_cast(bf16x8, av), pop, o[dt]);
      }
      lsum = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sum_sel, pop, lsum, 0, 0, 0);
    }
  };
  auto qk = [&](int jb) __attribute__((always_inline)) {
    const uint16_t* kp = Ks + (jb & 1) * kTile + k_lane;
    // two independent accumulation chains (sub-tiles kt = 0, 1), interleaved
    for (int s = 0; s < 8; ++s) {
      const uint16_t* ks = kp + (k_x ^ (16 * s));
      for (int kt = 0; kt < 2; ++kt)
        sc[kt] = mfma32(as_bf16x8(*(const u32x4*)(ks + kt * 32 * kD)), qop[s], sc[kt]);
    }
  };
  // Issue order of the steady-state matrix step (one wave runs it alone on its SIMD, so
  // it must hide its own LDS latency): operands stay kRA MFMAs ahead of their use, and
  // the first K reads are issued under the last PV MFMAs.
  constexpr int kRA = 4;
  auto pv_qk_schedule = [&]() __attribute__((always_inline)) {
    // 20 MFMAs: per PV step st, its 4 PV MFMAs and the row-sum MFMA of its P chunk
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * kRA, 0);  // V^T reads of the first kRA PV MFMAs
    for (int i = 0; i < 16 - kRA; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // PV MFMA i
      if ((i & 3) == 3) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // row sum of step i / 4
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);       // V^T reads of PV MFMA i + kRA
    }
    for (int i = 0; i < kRA; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // PV MFMA 16 - kRA + i
      if (i == kRA - 1) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // row sum of the last step
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);       // K read of QK MFMA i
    }
    for (int i = 0; i < 16 - kRA; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);       // QK MFMA i
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);       // K read of QK MFMA i + kRA
    }
    for (int i = 0; i < kRA; ++i) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  };
  auto apply_rescale = [&]() __attribute__((always_inline)) {
    if (rescale) {
      for (int dt = 0; dt < 4; ++dt) o[dt] *= o_scale;
      lsum[0] *= o_scale;
      lsum[1] *= __shfl(o_scale, (lane & 15) + 16, 64);  // lanes 0-15 hold row (lane & 15) + 16's sum
      rescale = false;
    }
  };
  // general matrix step (first and last steps, causal-inactive blocks)
  auto mstep = [&](int j, auto seg) __attribute__((always_inline)) {
    apply_rescale();
    const bool do_pv = j >= 1 && j - 1 < ng && active(j - 1, seg);
    const bool do_qk = j < ng && active(j, seg);
    __builtin_amdgcn_s_setprio(1);
    if (do_pv) pv(j - 1);
    if (do_qk) qk(j);
    __builtin_amdgcn_s_setprio(0);
  };
  // steady-state matrix step: both halves run, as one scheduled region
  auto mstep_full = [&](int j) __attribute__((always_inline)) {
    apply_rescale();
    __builtin_amdgcn_s_setprio(1);
    pv(j - 1);
    qk(j);
    pv_qk_schedule();
    __builtin_amdgcn_s_setprio(0);
  };

  // Softmax step j: P for block j (into pw), then the loads of K for block j+2 (its
  // buffer held K of block j, last read by the matrix step just before) and of V for
  // block j+1 (its buffer held V of block j-1, last read by that same matrix step).
  // With kMask false the block is known to need no mask (the steady-state loop).
  auto vstep = [&](int j, auto mask_tag, auto seg) __attribute__((always_inline)) {
    constexpr bool kMask = decltype(mask_tag)::value;
    if (j < 0 || j >= ng) return;
    if (active(j, seg)) {
      const int kbase = blk_of(j) * kBN;
      // key of slot i in sub-tile kt: kbase + 32kt + (i%4) + 8(i/4) + 4hh
      if (kMask && need_mask(j, seg)) {
        const int q_abs = wfa_of(j, seg) + (lane & 31);
        int hi = causal && q_abs < kv_len - 1 ? q_abs : kv_len - 1;
        hi -= kbase + 4 * hh;
        const int lo = kv_begin - kbase - 4 * hh;
        for (int kt = 0; kt < 2; ++kt)
          for (int i = 0; i < 16; ++i) {
            const int koff = 32 * kt + (i & 3) + 8 * (i >> 2);
            sc[kt][i] = koff <= hi && koff >= lo ? sc[kt][i] : -INFINITY;
          }
      }
      // P^T as bf16 pairs for the PV steps (step st: slots 8*(st&1) .. +7 of sub-tile st>>1).
      // Fast path: p = 2^(s - m_use) with the running base m_use as is, kept when every p
      // of the wave is at most 256 (a lazy rescale with threshold 8 in the log2 domain), so
      // no row max is formed and nothing is rescaled. The check takes the maximum of the
      // packed bf16 words read as f16 pairs: for p >= 0 the bit patterns below 0x7C00 are
      // ordered alike in both formats, and larger ones (p >= 2^121, inf, NaN) read as f16
      // inf or NaN, which the maximum keeps.
      bool fast = all_seen;
      if (fast) {
        const uint32_t kob = blk_off(j + 2), vob = blk_off(j + 1);
        const int kwrap = wrap_rows(j + 2), vwrap = wrap_rows(j + 1);
        const u32x4 kr = kRot ? k_rsrc : tile_rsrc(Kg, kob), vr = kRot ? v_rsrc : tile_rsrc(Vg, vob);
        const uint32_t kdst = tile_dst(Ks + (j & 1) * kTile), vdst = tile_dst(Vs + ((j + 1) & 1) * kTile);
        for (int st = 0; st < 4; ++st) {
          dma_part(kr, kob, koff, kdst, st, kwrap);
          dma_part(vr, vob, voff, vdst, st, vwrap);
          for (int e = 0; e < 4; ++e) {
            const int kt = st >> 1, i = 8 * (st & 1) + 2 * e;
            pw[st][e] = pack_bf16x2(__builtin_amdgcn_exp2f(sc[kt][i]), __builtin_amdgcn_exp2f(sc[kt][i + 1]));
          }
        }
        uint32_t pm = pk_max3_f16(pw[0][0], pw[0][1], pw[0][2]);
        pm = pk_max3_f16(pm, pw[0][3], pw[1][0]);
        pm = pk_max3_f16(pm, pw[1][1], pw[1][2]);
        pm = pk_max3_f16(pm, pw[1][3], pw[2][0]);
        pm = pk_max3_f16(pm, pw[2][1], pw[2][2]);
        pm = pk_max3_f16(pm, pw[2][3], pw[3][0]);
        pm = pk_max3_f16(pm, pw[3][1], pw[3][2]);
        pm = pk_max3_f16(pm, pw[3][3], pw[3][3]);
        fast = !__any((pm & 0xffffu) > 0x4380u || pm > 0x4380ffffu);  // some p > 256
      } else {
        load_k(j + 2);
        load_v(j + 1);
      }
      if (!fast) {
        // Slow path (first block of a row, or a row max that grew): move the base to
        // the row's running max and rescale what was accumulated.
        float mx = sc[0][0];
        for (int kt = 0; kt < 2; ++kt)
          for (int i = kt ? 0 : 1; i < 16; ++i) mx = fmaxf(mx, sc[kt][i]);
        const float bm = wave_max_xor(mx, 32);
        const float delta = seen ? fmaxf(bm, 0.f) : (bm == -INFINITY ? 0.f : bm);
        seen = seen || bm != -INFINITY;
        const float alpha = __builtin_amdgcn_exp2f(-delta);
        o_scale = alpha;
        rescale = true;
        m_use += delta;
        for (int st = 0; st < 4; ++st)
          for (int e = 0; e < 4; ++e) {
            const int kt = st >> 1, i = 8 * (st & 1) + 2 * e;
            pw[st][e] = pack_bf16x2(__builtin_amdgcn_exp2f(sc[kt][i] - delta),
                                    __builtin_amdgcn_exp2f(sc[kt][i + 1] - delta));
          }
        all_seen = __all(seen);
      }
    } else {
      load_k(j + 2);
      load_v(j + 1);
    }
    // the score chains of the next matrix step start from -m_use
    for (int kt = 0; kt < 2; ++kt)
      for (int i = 0; i < 16; ++i) sc[kt][i] = -m_use;
    // the loads of the previous softmax step (K of block j+1, V of block j) are read by
    // the next matrix step: wait for them, leaving this step's own 8 loads in flight
    // (loads complete in issue order); step 0's predecessors were waited for up front
    __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8)
  };

  // Prologue, part 2: this group's first tiles (K of blocks 0 and 1, V of block 0; zero
  // fills past the stream, so the count is fixed). The first matrix step reads Q and K of
  // block 0 only: the wait leaves the last 8 loads in flight, and the first softmax step's
  // wait (before the barrier that precedes the second matrix step) covers them.
  load_k(0);
  load_v(0);
  load_k(1);
  __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8)
  __syncthreads();

  // Q^T as B operand: step s covers dims 16s + 8*hh .. +7 of row 32wq + (lane & 31). Q is
  // scaled by scale*log2(e) and rounded to bf16 here, so the scores come out of the
  // MFMA in the log2 domain and the softmax needs no multiply per score.
  auto scale_q = [&](const u32x4 raw) __attribute__((always_inline)) {
    u32x4 w;
    for (int e = 0; e < 4; ++e) w[e] = pack_bf16x2(bf16_lo(raw[e]) * a.qk_scale, bf16_hi(raw[e]) * a.qk_scale);
    return as_bf16x8(w);
  };
  // Segment B's rows: Q^T of the heavy rows from LDS, and a fresh softmax state (o and
  // the row sums are cleared where segment A's output leaves).
  auto start_b = [&]() __attribute__((always_inline)) {
    const uint16_t* qp = Qs + 32 * wq * kD + k_lane;
    for (int s = 0; s < 8; ++s) qop[s] = scale_q(*(const u32x4*)(qp + (k_x ^ (16 * s))));
    m_use = 0.f;
    seen = false;
    all_seen = false;
    for (int kt = 0; kt < 2; ++kt)
      for (int i = 0; i < 16; ++i) sc[kt][i] = 0.f;
  };
  // Segment A's rows are complete (the PV of their last block ran in the matrix step
  // before): normalise, stage the wave's 32 rows in its own rows of the Q area (whose heavy
  // Q^T it has read), store them as whole 256-byte rows, and clear o and the row sums.
  auto finish_a = [&]() __attribute__((always_inline)) {
    const float l_lo = __shfl(lsum[0], lane & 15, 64), l_hi = __shfl(lsum[1], lane & 15, 64);
    const float l_run = (lane & 16) ? l_hi : l_lo;
    const float inv = l_run > 0.f ? 1.0f / l_run : 0.f;
    const int rr = 32 * wq + (lane & 31);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    for (int dt = 0; dt < 4; ++dt)
      for (int i4 = 0; i4 < 4; ++i4) {
        // lane holds O[rr][32dt + (i%4) + 8(i/4) + 4hh]: chunk 4dt + i4, half hh
        u32x2 wv;
        wv[0] = pack_bf16x2(o[dt][4 * i4] * inv, o[dt][4 * i4 + 1] * inv);
        wv[1] = pack_bf16x2(o[dt][4 * i4 + 2] * inv, o[dt][4 * i4 + 3] * inv);
        const int c = 4 * dt + i4;
        *(u32x2*)(Qs + rr * kD + 8 * (c ^ (rr & 15)) + 4 * hh) = wv;
      }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the wave reads what its lanes wrote
    for (int it = 0; it < 8; ++it) {
      const int n = it * 64 + lane;
      const int r = 32 * wq + (n >> 4), c = n & 15;
      const u32x4 v = *(const u32x4*)(Qs + r * kD + 8 * (c ^ (r & 15)));
      if (row0A + r < a.T) *(u32x4*)(a.out + (((int64_t)b * a.T + row0A + r) * a.Hq + h) * kD + 8 * c) = v;
    }
    for (int dt = 0; dt < 4; ++dt)
      for (int i = 0; i < 16; ++i) o[dt][i] = 0.f;
    lsum = f32x4{0.f, 0.f, 0.f, 0.f};
  };

  // Phase 2t + half: group 0 runs matrix step t then softmax step t; group 1 runs
  // softmax step t-1 then matrix step t, so the groups always sit in opposite halves.
  // Every wave passes the same number of barriers (n0 + 1 phase pairs). Matrix steps whose
  // two halves are both active and inside one segment run in loops of their own with the
  // scheduled full step; those loops also run only over softmax steps of blocks that need
  // no mask, so their softmax step carries no masking code.
  const MaskOn mask_on;
  const MaskOff mask_off;
  const int actB = seg_act(gbB, wfaB, nB), maskB = seg_mask(gbB, wfaB);
  if (g == 0) {
    auto half0 = [&](int t, bool full, auto mask_tag, auto seg, bool switch_rows) __attribute__((always_inline)) {
      if (full) mstep_full(t);
      else mstep(t, seg);
      __syncthreads();
      vstep(t, mask_tag, seg);
      if (switch_rows) start_b();
      __syncthreads();
    };
    int t = 0;
    if (kPair && n1 > 0) {
      // segment A: blocks 0 .. n1-1, the last one followed by the switch of the Q operand
      const uint16_t* qp = light_q(32 * wq) + k_lane;
      for (int s = 0; s < 8; ++s) qop[s] = scale_q(*(const u32x4*)(qp + (k_x ^ (16 * s))));
      const int actA = seg_act(gbA, wfaA, n1), maskA = seg_mask(gbA, wfaA);
      const int tfA = actA < maskA ? actA : maskA;
      for (; t < n1 - 1 && t < 1; ++t) half0(t, false, mask_on, SegA{}, false);
      for (; t < n1 - 1 && t < tfA; ++t) half0(t, true, mask_off, SegA{}, false);
      for (; t < n1 - 1; ++t) half0(t, false, mask_on, SegA{}, false);
      half0(t, false, mask_on, SegA{}, true);
      ++t;
    } else {
      start_b();
    }
    // step n1: the PV of segment A's last block beside the QK of segment B's first; segment
    // A's rows leave in the softmax half
    mstep(t, SegAny{});
    __syncthreads();
    vstep(t, mask_on, SegB{});
    if (has_light) finish_a();
    __syncthreads();
    ++t;
    const int tfB = n1 + (actB < maskB ? actB : maskB);
    for (; t < tfB; ++t) half0(t, true, mask_off, SegB{}, false);
    for (; t <= n0; ++t) half0(t, false, mask_on, SegB{}, false);
  } else {
    start_b();
    auto half1 = [&](int t, bool full, auto mask_tag) __attribute__((always_inline)) {
      vstep(t - 1, mask_tag, SegB{});
      __syncthreads();
      if (full) mstep_full(t);
      else mstep(t, SegB{});
      __syncthreads();
    };
    const int t_full = actB < maskB + 1 ? actB : maskB + 1;
    int t = 0;
    for (; t <= n0 && t < 2; ++t) half1(t, false, mask_on);
    for (; t < t_full; ++t) half1(t, true, mask_off);
    for (; t <= n0; ++t) half1(t, false, mask_on);
  }

  // the last softmax steps' loads (zero fills past the range) land before the merge
  // reuses the tiles
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();

  // Merge. Each group finishes half of the head dims: group g keeps dims 64g .. 64g+63
  // (accumulators dt = 2g, 2g+1) and hands the other half to the other group through LDS
  // (the tiles are dead now), together with its (m, l). The normalised bf16 rows go to a
  // staging tile in the Q area (Q is in registers since the prologue), from which all
  // eight waves store whole 256-byte rows with 16-byte stores.
  //   xo[g]: [d][i4][wq][lane] f32x4, the dims of group g that the other group finishes
  //   xm[g], xl[g]: [wq][lane] this group's m (or -inf) and row sum l
  float* const xo = (float*)lds;
  float* const xm = xo + 2 * 2 * 4 * 4 * 64 * 4;
  float* const xl = xm + 2 * 4 * 64;
  const int rr = 32 * wq + (lane & 31);  // row inside the workgroup
  // this lane's row sum (the whole row: both key halves of the wave are in it)
  const float l_lo = __shfl(lsum[0], lane & 15, 64), l_hi = __shfl(lsum[1], lane & 15, 64);
  const float l_run = (lane & 16) ? l_hi : l_lo;
  {
    float* const mx = xo + g * (2 * 4 * 4 * 64 * 4);
    auto publish = [&](const int dt0) __attribute__((always_inline)) {
      for (int d = 0; d < 2; ++d)
        for (int i4 = 0; i4 < 4; ++i4) {
          const f32x16& od = o[dt0 + d];
          const f32x4 v = {od[4 * i4], od[4 * i4 + 1], od[4 * i4 + 2], od[4 * i4 + 3]};
          *(f32x4*)(mx + (((d * 4 + i4) * 4 + wq) * 64 + lane) * 4) = v;
        }
    };
    if (g == 0) publish(2);
    else publish(0);
    xm[(g * 4 + wq) * 64 + lane] = seen ? m_use : -INFINITY;
    xl[(g * 4 + wq) * 64 + lane] = l_run;
  }
  __syncthreads();
  {
    const float m0 = xm[wq * 64 + lane], m1 = xm[(4 + wq) * 64 + lane];
    const float l0 = xl[wq * 64 + lane], l1 = xl[(4 + wq) * 64 + lane];
    const float m = fmaxf(m0, m1);
    const float a0 = m0 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m0 - m);
    const float a1 = m1 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - m);
    const float l_tot = l0 * a0 + l1 * a1;
    const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    const float a_mine = g ? a1 : a0, a_other = g ? a0 : a1;
    const float* const ox = xo + (1 - g) * (2 * 4 * 4 * 64 * 4);
    uint16_t* const St = Qs;  // bf16 [128 rows][128 dims], 16-byte chunk c of row r at c ^ (r & 15)
    auto finish = [&](const int dt0) __attribute__((always_inline)) {
      for (int d = 0; d < 2; ++d)
        for (int i4 = 0; i4 < 4; ++i4) {
          const f32x4 v = *(const f32x4*)(ox + (((d * 4 + i4) * 4 + wq) * 64 + lane) * 4);
          float r[4];
          for (int e = 0; e < 4; ++e) r[e] = (o[dt0 + d][4 * i4 + e] * a_mine + v[e] * a_other) * inv;
          // lane holds O[rr][32dt + (i%4) + 8(i/4) + 4hh]: chunk 4dt + i4, half hh
          u32x2 wv;
          wv[0] = pack_bf16x2(r[0], r[1]);
          wv[1] = pack_bf16x2(r[2], r[3]);
          const int c = 4 * (dt0 + d) + i4;
          *(u32x2*)(St + rr * kD + 8 * (c ^ (rr & 15)) + 4 * hh) = wv;
        }
    };
    if (g == 0) finish(0);
    else finish(2);
  }
  __syncthreads();
  {
    // 128 rows x 16 chunks over 512 threads: a wave stores 4 whole rows per instruction
    for (int it = 0; it < 4; ++it) {
      const int n = it * kThreads + tid;
      const int r = n >> 4, c = n & 15;
      const u32x4 v = *(const u32x4*)(Qs + r * kD + 8 * (c ^ (r & 15)));
      if (row0 + r < a.T) *(u32x4*)(a.out + (((int64_t)b * a.T + row0 + r) * a.Hq + h) * kD + 8 * c) = v;
    }
  }
}

}  // namespace

int32_t launch_prefill(hipStream_t s, const void* q, const ema_kvcache_desc& c,
                       const int32_t* q_off, int T, int Hq, float scale, uint32_t flags,
                       void* out) {
  if (c.head_dim != kD)
    return set_error(EMA_ERR_UNSUPPORTED, "ema_prefill_attention: head_dim %d not supported (128)", c.head_dim);
  // K/V rows are addressed through buffer resources with 32-bit byte ranges
  if ((int64_t)c.capacity * c.stride_pos * 2 >= ((int64_t)1 << 31))
    return set_error(EMA_ERR_UNSUPPORTED,
                     "ema_prefill_attention: capacity %d x stride_pos %lld exceeds the 2 GiB per-head range",
                     c.capacity, (long long)c.stride_pos);
  static std::atomic<uint64_t> lds_set[4];  // per instantiation, one bit per device
  const void* kernels[4] = {(const void*)prefill_kernel<false, false>, (const void*)prefill_kernel<true, false>,
                            (const void*)prefill_kernel<false, true>, (const void*)prefill_kernel<true, true>};
  for (int i = 0; i < 4; ++i) {
    const int32_t rc = allow_lds_once(kernels[i], kLdsBytes, &lds_set[i], "ema_prefill_attention: LDS attribute");
    if (rc) return rc;
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
  // pair the query blocks when there are at least two workgroups' worth per CU
  const int cus = device_cus();
  const int64_t items = (int64_t)a.nqb * Hq * c.batch;
  a.paired = a.nqb >= 2 && items >= 2 * (int64_t)cus;
  const int64_t blocks = prefill_grid(c.batch, Hq, a.nqb, a.paired);
  if (blocks > 0x7fffffff) return set_error(EMA_ERR_SHAPE, "ema_prefill_attention: grid too large");
  const bool rot = c.flags & EMA_KV_ROTATING;
  if (rot && a.paired)
    hipLaunchKernelGGL((prefill_kernel<true, true>), dim3((unsigned)blocks), dim3(kThreads), kLdsBytes, s, a);
  else if (rot)
    hipLaunchKernelGGL((prefill_kernel<true, false>), dim3((unsigned)blocks), dim3(kThreads), kLdsBytes, s, a);
  else if (a.paired)
    hipLaunchKernelGGL((prefill_kernel<false, true>), dim3((unsigned)blocks), dim3(kThreads), kLdsBytes, s, a);
  else
    hipLaunchKernelGGL((prefill_kernel<false, false>), dim3((unsigned)blocks), dim3(kThreads), kLdsBytes, s, a);
  return check_hip(hipGetLastError(), "ema_prefill_attention launch");
}

}  // namespace ema
