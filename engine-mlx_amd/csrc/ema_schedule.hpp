// Integer work schedules of the attention kernels: which (sequence, head, query block) a
// prefill workgroup runs, and how the decode split cuts the tile range of all
// (sequence, kv head) segments into worker slices. The kernels call these functions on
// the device; the CPU tests (tests/cpp/test_schedule.cpp, built with a host compiler)
// call the same definitions to check that every work item is covered exactly once.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define EMA_HD __host__ __device__ __forceinline__
#else
#define EMA_HD inline
#endif

namespace ema {

// ------------------------------------------------------------------ prefill
// MI355X dispatches consecutive workgroups round-robin over its 8 XCDs (workgroup x
// runs on XCD x % 8), each XCD with its own L2.
constexpr int kSchedXcds = 8;

struct PrefillItem {
  int b;          // sequence
  int kh;         // kv head
  int h;          // query head
  int qb_first;   // query block run first
  int qb_second;  // query block run second (== qb_first: none)
};

// Work item of prefill workgroup x out of `grid`, for B sequences, Hkv kv heads with G
// query heads each, and nqb query blocks per head.
//
// When the (sequence, kv head) groups divide evenly over the XCDs (and so does the grid),
// all query heads of a group run on the group's XCD, so its K/V stream is read from HBM
// once and served from that L2 to every workgroup attending over it. Inside an XCD (or
// over the whole grid otherwise) work items are ranked heaviest first, because a later
// query block sees more keys under the causal mask. With `paired`, a workgroup takes the
// heavy query block nqb-1-p and then the light block p of the same head (grid =
// ceil(nqb/2) * B * Hkv * G); with odd nqb the middle block is paired with itself and run
// once.
EMA_HD PrefillItem prefill_item(int64_t x, int64_t grid, int B, int Hkv, int G, int nqb, int paired) {
  const int groups = B * Hkv;
  const bool by_xcd = groups % kSchedXcds == 0 && grid % kSchedXcds == 0;
  const int64_t rank = by_xcd ? x / kSchedXcds : x;
  const int groups_local = by_xcd ? groups / kSchedXcds : groups;
  const int64_t per_qb = (int64_t)groups_local * G;
  PrefillItem it;
  it.qb_first = nqb - 1 - (int)(rank / per_qb);
  it.qb_second = paired ? nqb - 1 - it.qb_first : it.qb_first;
  const int rest = (int)(rank % per_qb);
  const int grp = by_xcd ? (rest / G) * kSchedXcds + (int)(x % kSchedXcds) : rest / G;
  it.b = grp / Hkv;
  it.kh = grp % Hkv;
  it.h = it.kh * G + rest % G;
  return it;
}

// Grid size for prefill_item: nqb * B * Hq items, or ceil(nqb/2) * B * Hq pairs.
EMA_HD int64_t prefill_grid(int B, int Hq, int nqb, int paired) {
  return (int64_t)(paired ? (nqb + 1) / 2 : nqb) * B * Hq;
}

// Block streams of a prefill workgroup's two wave groups. A query block attends the
// 64-key blocks [blk_begin, blk_begin + n) of its key range; the heavy block has nblk_h
// of them, the light block of a pair nblk_l <= nblk_h (0 without a light block: a single
// block, or an empty range). Group 0 streams segment A, the light rows over all their
// blocks [0, n1), then segment B, the heavy rows over [gbB, gbB + nB) = [0, nh0); group 1
// streams segment B only, the heavy rows over the rest [nh0, nblk_h). Group 0 thus takes
// prefill_group0_blocks of the pair's blocks and group 1 the others (as many, or one
// fewer), and the heavy rows' two partial states meet in the merge. Block indices are
// relative to blk_begin.
struct PrefillStream {
  int n1;   // segment A's blocks (group 0 of a pair only)
  int gbB;  // segment B's first block
  int nB;   // segment B's blocks
};

EMA_HD int prefill_group0_blocks(int nblk_h, int nblk_l) { return (nblk_l + nblk_h + 1) / 2; }

EMA_HD PrefillStream prefill_stream(int g, int nblk_h, int nblk_l) {
  const int n0 = prefill_group0_blocks(nblk_h, nblk_l);
  const int nh0 = n0 - nblk_l;  // heavy blocks of group 0
  PrefillStream s;
  s.n1 = g == 0 ? nblk_l : 0;
  s.gbB = g == 0 ? 0 : nh0;
  s.nB = g == 0 ? nh0 : nblk_h - nh0;
  return s;
}

// ------------------------------------------------------------------ decode split
// The valid rows of every (sequence b, kv head kh) pair form a segment of ceil(len/32)
// tiles; segments are laid end to end (sequence-major, then kv head) and the flattened
// range of `total` tiles is cut into W slices, slice w = [split_begin(w), split_begin(w+1)).

constexpr int kSplitTile = 32;         // positions per tile
constexpr int kSplitWaves = 4;         // waves per decode workgroup, each an independent worker
constexpr int kSplitMaxWorkers = 512;  // workgroups of the split (and staging rows of the merge)

// Workgroups the plan sizes the workspace for, from the host's upper bound of the lengths:
// at least one tile per wave, at most kSplitMaxWorkers.
EMA_HD int split_plan_workers(int B, int Hkv, int max_len) {
  const int64_t tiles = (int64_t)B * Hkv * ((max_len + kSplitTile - 1) / kSplitTile);
  const int64_t want = (tiles + kSplitWaves - 1) / kSplitWaves;
  const int64_t w = want < kSplitMaxWorkers ? want : kSplitMaxWorkers;
  return (int)(w < 1 ? 1 : w);
}

// Workers used for `total` tiles: at least one tile per wave (`waves` per workgroup), at
// most the plan's W, which sizes the workspace from the host's upper bound of the lengths.
EMA_HD int split_active_workers(int64_t total, int W, int waves) {
  const int64_t want = (total + waves - 1) / waves;
  return (int)(want < W ? want : W);
}
// First tile of slice w.
EMA_HD int64_t split_begin(int64_t w, int64_t total, int W) { return w * total / W; }
// Slice holding tile t (the inverse of split_begin).
EMA_HD int64_t split_worker_of(int64_t t, int64_t total, int W) { return ((t + 1) * (int64_t)W - 1) / total; }

// The same two functions in 32-bit arithmetic, equal to them whenever every product
// w * total (w <= W) stays below 2^31, which split_narrow checks for the largest tile count
// the lengths allow. The decode kernels take these on the latency path of small grids,
// where a 64-bit division is a long scalar emulation.
EMA_HD bool split_narrow(int64_t max_total, int W) { return max_total * W < ((int64_t)1 << 31); }
EMA_HD int64_t split_begin32(int64_t w, int64_t total, int W) {
  return (int64_t)((uint32_t)w * (uint32_t)total / (uint32_t)W);
}
EMA_HD int64_t split_worker_of32(int64_t t, int64_t total, int W) {
  return (int64_t)((((uint32_t)t + 1u) * (uint32_t)W - 1u) / (uint32_t)total);
}

// ------------------------------------------------------------------ decode tile slots
// LDS layouts of the decode kernels' tiles when they arrive by LDS-DMA: instruction i, lane l
// writes the 16 bytes at slot byte 1024 i + 16 l, gathered from any source address; the
// operands are then read in the MFMA layouts. The QK operand's lane (m, c) of row set r
// reads row dec_krow(m, r) of the 32-row tile, chunk 4s + c (bf16: 16 bytes of step s) or
// 4i + c (fp8: 16 bytes of steps 2i, 2i + 1).
EMA_HD int dec_krow(int m, int r) { return 8 * (m >> 2) + (m & 3) + 4 * r; }
// bf16: 256-byte rows, four per instruction (row R at byte 256 R); unit u of K row R holds
// chunk u ^ bf_swz(R), so the 16 rows of one operand read land on 16 distinct 16-byte bank
// groups of a 256-byte bank window (bf_swz(dec_krow(m, r)) = m).
EMA_HD int bf_swz(int R) { return (R & 3) + 4 * ((R >> 3) & 3); }
// fp8: 128-byte rows, eight per instruction. Unit u of K row R holds chunk u ^ f8_swz(R): the
// row's parity picks the 128-byte half of the window and the swizzle the unit within it, so
// again the 16 rows of a read use 16 distinct bank groups. V row R sits at slot row
// f8_vrow(R) (an involution), so the rows 8c + kk of one read (16 lanes per row, c = 0..3)
// alternate between the window's halves.
EMA_HD int f8_swz(int R) { return ((R >> 1) & 1) | (((R >> 3) & 3) << 1); }
EMA_HD int f8_vrow(int R) { return R ^ ((R >> 3) & 1); }

}  // namespace ema
