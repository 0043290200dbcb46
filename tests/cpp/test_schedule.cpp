// CPU checks of the attention kernels' integer work schedules (engine-mlx_amd/csrc/
// ema_schedule.hpp, the same definitions the kernels call on the device):
//  - prefill: every (sequence, query head, query block) is run by exactly one workgroup,
//    paired or not, with and without the XCD grouping; the heavy block of a pair runs
//    first; with the XCD grouping every item of a (sequence, kv head) group lands on the
//    group's XCD; ranks run heaviest first; inside a workgroup the two wave groups' block
//    streams see each (row set, key block) once and stay balanced;
//  - decode split: the worker slices tile [0, total) exactly once, split_worker_of
//    inverts split_begin, the merge's slot range [w0, w1] of every segment is exactly the
//    set of slices that intersect it, and the partial-state slots (w + segment) of split
//    segments are distinct and inside the workspace the plan sizes; the 32-bit forms of
//    split_begin / split_worker_of equal the 64-bit ones wherever split_narrow holds, up
//    to its edge;
//  - decode tile slots: the LDS-DMA gathers and the operand reads of the bf16 and fp8 slot
//    layouts agree byte for byte, and each read spreads over distinct bank groups.
// Built with g++ (no HIP), also under -fsanitize=address,undefined. Prints one line per
// group of checks and exits non-zero on the first failure.
#include <cstdio>
#include <cstdlib>
#include <set>
#include <vector>

#include "ema_schedule.hpp"

using namespace ema;

static int g_checks = 0;
#define CHECK(cond, ...)                                   \
  do {                                                     \
    ++g_checks;                                            \
    if (!(cond)) {                                         \
      std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
      std::fprintf(stderr, __VA_ARGS__);                   \
      std::fprintf(stderr, "\n");                          \
      std::exit(1);                                        \
    }                                                      \
  } while (0)

static void prefill_case(int B, int Hkv, int G, int nqb, int paired) {
  const int Hq = Hkv * G;
  const int64_t grid = prefill_grid(B, Hq, nqb, paired);
  std::vector<int> seen((size_t)B * Hq * nqb, 0);
  const bool by_xcd = (B * Hkv) % kSchedXcds == 0 && grid % kSchedXcds == 0;
  std::vector<int> last_qb(kSchedXcds, 1 << 30);
  for (int64_t x = 0; x < grid; ++x) {
    const PrefillItem it = prefill_item(x, grid, B, Hkv, G, nqb, paired);
    CHECK(it.b >= 0 && it.b < B && it.kh >= 0 && it.kh < Hkv, "x=%lld b=%d kh=%d", (long long)x, it.b, it.kh);
    CHECK(it.h / G == it.kh && it.h >= 0 && it.h < Hq, "x=%lld h=%d kh=%d G=%d", (long long)x, it.h, it.kh, G);
    CHECK(it.qb_first >= 0 && it.qb_first < nqb && it.qb_second >= 0 && it.qb_second < nqb,
          "x=%lld qb %d/%d of %d", (long long)x, it.qb_first, it.qb_second, nqb);
    CHECK(it.qb_first >= it.qb_second, "pair must run its heavy block first (x=%lld)", (long long)x);
    if (!paired) CHECK(it.qb_first == it.qb_second, "unpaired grid ran two blocks (x=%lld)", (long long)x);
    const size_t base = ((size_t)it.b * Hq + it.h) * nqb;
    ++seen[base + it.qb_first];
    if (it.qb_second != it.qb_first) ++seen[base + it.qb_second];
    const int lane = by_xcd ? (int)(x % kSchedXcds) : 0;
    if (by_xcd)
      CHECK((it.b * Hkv + it.kh) % kSchedXcds == lane, "group %d off its XCD %d (x=%lld)", it.b * Hkv + it.kh, lane,
            (long long)x);
    CHECK(it.qb_first <= last_qb[lane], "ranks must run heaviest first (x=%lld)", (long long)x);
    last_qb[lane] = it.qb_first;
  }
  for (size_t i = 0; i < seen.size(); ++i)
    CHECK(seen[i] == 1, "B=%d Hkv=%d G=%d nqb=%d paired=%d: item (b=%zu h=%zu qb=%zu) run %d times", B, Hkv, G, nqb,
          paired, i / ((size_t)Hq * nqb), i / nqb % Hq, i % nqb, seen[i]);
}

static void test_prefill() {
  const int shapes[][4] = {
      // B, Hkv, G, nqb
      {1, 8, 4, 16},   // 8B shape, T 2048 (XCD-grouped, paired on MI355X)
      {1, 8, 2, 16},   // 1.7B shape
      {4, 4, 4, 8},    // B 4, 16q/4kv, T 1000
      {4, 4, 4, 9},    // odd block count: the middle block pairs with itself
      {3, 3, 8, 7},    // groups not a multiple of the XCD count
      {1, 8, 8, 1},    // one query block
      {2, 1, 1, 5},    // MHA-like, tiny
      {16, 8, 8, 33},  // chunk shape, long
      {5, 2, 3, 4},    // grid not divisible by 8
      {8, 1, 3, 3},    // groups == XCDs, odd nqb
  };
  for (const auto& s : shapes)
    for (int paired = 0; paired < 2; ++paired) prefill_case(s[0], s[1], s[2], s[3], paired);
  std::printf("prefill schedule: %zu shapes x {unpaired, paired}: every (b, h, qb) exactly once\n",
              sizeof(shapes) / sizeof(shapes[0]));
}

// Decode split for tile counts nb[s] per segment s (segments in sequence-major order).
static void decode_case(const std::vector<int>& nb, int plan_workers, int waves) {
  std::vector<int64_t> first(nb.size() + 1, 0);
  for (size_t s = 0; s < nb.size(); ++s) first[s + 1] = first[s] + nb[s];
  const int64_t total = first.back();
  if (total == 0) return;
  const int W = split_active_workers(total, plan_workers, waves);
  CHECK(W >= 1 && W <= plan_workers, "active workers %d of %d", W, plan_workers);
  // slices tile the range exactly once; worker_of inverts begin
  CHECK(split_begin(0, total, W) == 0 && split_begin(W, total, W) == total, "slice ends");
  for (int w = 0; w < W; ++w) {
    const int64_t a = split_begin(w, total, W), b = split_begin(w + 1, total, W);
    CHECK(a < b, "empty slice %d of %d (total %lld)", w, W, (long long)total);
    for (int64_t t = a; t < b; ++t)
      CHECK(split_worker_of(t, total, W) == w, "worker_of(%lld) = %lld, not %d", (long long)t,
            (long long)split_worker_of(t, total, W), w);
  }
  // the 32-bit forms agree wherever the kernels take them
  if (split_narrow(total, plan_workers)) {
    for (int w = 0; w <= W; ++w)
      CHECK(split_begin32(w, total, W) == split_begin(w, total, W), "begin32(%d) of %lld", w, (long long)total);
    for (int64_t t = 0; t < total; ++t)
      CHECK(split_worker_of32(t, total, W) == split_worker_of(t, total, W), "worker_of32(%lld)", (long long)t);
  }
  // merge ranges and partial slots
  std::set<int64_t> slots;
  for (size_t s = 0; s < nb.size(); ++s) {
    if (nb[s] == 0) continue;
    const int64_t w0 = split_worker_of(first[s], total, W), w1 = split_worker_of(first[s + 1] - 1, total, W);
    for (int w = 0; w < W; ++w) {
      const bool meets = split_begin(w, total, W) < first[s + 1] && split_begin(w + 1, total, W) > first[s];
      CHECK(meets == (w >= w0 && w <= w1), "segment %zu, worker %d: merge range [%lld, %lld]", s, w, (long long)w0,
            (long long)w1);
    }
    if (w0 == w1) continue;  // written directly, no partial state
    for (int64_t w = w0; w <= w1; ++w) {
      const int64_t slot = w + (int64_t)s;
      CHECK(slot < (int64_t)plan_workers + (int64_t)nb.size(), "slot %lld outside the workspace", (long long)slot);
      CHECK(slots.insert(slot).second, "slot %lld written twice", (long long)slot);
    }
  }
}

static void test_decode() {
  unsigned rng = 12345u;
  auto next = [&rng]() {
    rng = rng * 1664525u + 1013904223u;
    return rng >> 8;
  };
  int cases = 0;
  for (int rep = 0; rep < 400; ++rep) {
    const int B = 1 + (int)(next() % 40), Hkv = 1 + (int)(next() % 8);
    const int cap = 1 + (int)(next() % 9000);
    std::vector<int> len(B);
    int max_len = 0;
    for (int b = 0; b < B; ++b) {
      const unsigned r = next() % 10;
      len[b] = r == 0 ? 0 : (r == 1 ? cap : (int)(next() % (unsigned)(cap + 1)));
      if (len[b] > max_len) max_len = len[b];
    }
    // the plan sizes the split from the host's upper bound (here: the capacity or the
    // true maximum), the kernel splits the actual tile count
    const int plan_workers = split_plan_workers(B, Hkv, (rep & 1) ? cap : max_len);
    std::vector<int> nb;
    for (int b = 0; b < B; ++b)
      for (int kh = 0; kh < Hkv; ++kh) nb.push_back((len[b] + kSplitTile - 1) / kSplitTile);
    decode_case(nb, plan_workers, kSplitWaves);
    ++cases;
  }
  // edges: one segment, one tile, more workers than tiles, the worker cap
  decode_case({1}, 1, kSplitWaves);
  decode_case({3}, kSplitMaxWorkers, kSplitWaves);
  decode_case({256}, 64, kSplitWaves);
  decode_case(std::vector<int>(32 * 8, 256), split_plan_workers(32, 8, 8192), kSplitWaves);
  decode_case({0, 0, 5, 0, 7}, 2, kSplitWaves);
  // the 32-bit forms at the edge of split_narrow: total * W just below 2^31, and just above
  for (const int W : {1, 7, 64, 511, kSplitMaxWorkers}) {
    const int64_t edge = (((int64_t)1 << 31) - 1) / W;
    CHECK(split_narrow(edge, W) && !split_narrow(edge + 1, W), "split_narrow edge at W = %d", W);
    for (int64_t w = 0; w <= W; ++w)
      CHECK(split_begin32(w, edge, W) == split_begin(w, edge, W), "begin32 at the edge, W = %d", W);
    for (int64_t t = 0; t < edge; t += 1 + edge / 200003)
      CHECK(split_worker_of32(t, edge, W) == split_worker_of(t, edge, W), "worker_of32 at the edge");
    CHECK(split_worker_of32(edge - 1, edge, W) == split_worker_of(edge - 1, edge, W), "worker_of32 of the last tile");
  }
  std::printf("decode split: %d random batches + 5 edge cases: tiles covered once, merge ranges and slots exact; "
              "32-bit forms equal wherever split_narrow holds\n",
              cases);
}

// The two wave groups' block streams of a prefill workgroup (prefill_stream): the light
// rows see each of their blocks once (group 0), the heavy rows each of theirs once (group
// 0's head, group 1's tail, no block twice or missed), group 0 runs
// prefill_group0_blocks of them and group 1 as many or one fewer, so both groups run the
// same number of matrix steps.
static void test_prefill_streams() {
  int cases = 0;
  for (int nh = 0; nh <= 80; ++nh)
    for (int nl = 0; nl <= nh; ++nl) {
      const int n0 = prefill_group0_blocks(nh, nl);
      const PrefillStream s0 = prefill_stream(0, nh, nl), s1 = prefill_stream(1, nh, nl);
      CHECK(s0.n1 == nl && s1.n1 == 0, "nh=%d nl=%d: segment A (%d, %d)", nh, nl, s0.n1, s1.n1);
      CHECK(s0.n1 + s0.nB == n0, "nh=%d nl=%d: group 0 runs %d blocks, not %d", nh, nl, s0.n1 + s0.nB, n0);
      CHECK(s1.nB >= 0 && s0.nB >= 0, "nh=%d nl=%d: negative segment", nh, nl);
      CHECK(s1.nB == n0 || s1.nB == n0 - 1 || (nh + nl == 0 && s1.nB == 0),
            "nh=%d nl=%d: group 1 runs %d blocks against %d", nh, nl, s1.nB, n0);
      std::vector<int> heavy(nh, 0);
      for (int j = 0; j < s0.nB; ++j) ++heavy[s0.gbB + j];
      for (int j = 0; j < s1.nB; ++j) {
        CHECK(s1.gbB + j < nh, "nh=%d nl=%d: group 1 block %d past the range", nh, nl, s1.gbB + j);
        ++heavy[s1.gbB + j];
      }
      for (int j = 0; j < nh; ++j) CHECK(heavy[j] == 1, "nh=%d nl=%d: heavy block %d seen %d times", nh, nl, j, heavy[j]);
      CHECK(s0.gbB == 0 && s1.gbB == s0.nB, "nh=%d nl=%d: segment B bounds", nh, nl);
      ++cases;
    }
  std::printf("prefill streams: %d (heavy, light) block counts: each block of each row set once, groups balanced\n",
              cases);
}

// Decode tile slots: an LDS-DMA instruction i writes lane l's 16 bytes at slot byte
// 1024 i + 16 l from the source the gather chose for that lane. Simulated per byte as
// (row, byte of the row) pairs: every operand read must find the row and chunk it wants,
// and the 16 lanes of one K read (one V row per 16 lanes) must spread over the bank
// groups of a 256-byte window.
static void test_decode_slots() {
  // bf16: K rows of 256 bytes, four per instruction; the gather puts chunk u ^ bf_swz(R) in unit u
  {
    std::vector<int> src(8192, -1);  // slot byte -> row * 256 + byte of the row
    for (int i = 0; i < 8; ++i)
      for (int l = 0; l < 64; ++l) {
        const int R = 4 * i + (l >> 4), ch = (l & 15) ^ bf_swz(R);
        for (int b = 0; b < 16; ++b) src[1024 * i + 16 * l + b] = R * 256 + 16 * ch + b;
      }
    for (int r = 0; r < 2; ++r)
      for (int s = 0; s < 4; ++s)
        for (int c = 0; c < 4; ++c) {
          std::set<int> units;
          for (int m = 0; m < 16; ++m) {
            const int R = dec_krow(m, r), ch = 4 * s + c;
            const int at = 1024 * (R >> 2) + 256 * (R & 3) + 16 * (ch ^ bf_swz(R));
            for (int b = 0; b < 16; ++b)
              CHECK(src[at + b] == R * 256 + 16 * ch + b, "bf16 slot: K row %d chunk %d byte %d", R, ch, b);
            units.insert((at / 16) % 16);
          }
          CHECK(units.size() == 16, "bf16 slot: K read r=%d s=%d c=%d on %zu bank groups", r, s, c, units.size());
        }
  }
  // fp8: K and V rows of 128 bytes, eight per instruction
  {
    std::vector<int> ksrc(4096, -1), vsrc(4096, -1);
    for (int i = 0; i < 4; ++i)
      for (int l = 0; l < 64; ++l) {
        const int S = 8 * i + (l >> 3), u = l & 7;
        for (int b = 0; b < 16; ++b) {
          ksrc[1024 * i + 16 * l + b] = S * 128 + 16 * (u ^ f8_swz(S)) + b;
          vsrc[1024 * i + 16 * l + b] = f8_vrow(S) * 128 + 16 * u + b;
        }
      }
    for (int R = 0; R < 32; ++R) CHECK(f8_vrow(f8_vrow(R)) == R && f8_vrow(R) < 32, "f8_vrow(%d)", R);
    for (int r = 0; r < 2; ++r)
      for (int i = 0; i < 2; ++i)
        for (int c = 0; c < 4; ++c) {
          std::set<int> units;
          for (int m = 0; m < 16; ++m) {
            const int R = dec_krow(m, r), ch = 4 * i + c;
            const int at = 128 * R + 16 * (ch ^ f8_swz(R));
            for (int b = 0; b < 16; ++b)
              CHECK(ksrc[at + b] == R * 128 + 16 * ch + b, "fp8 slot: K row %d chunk %d byte %d", R, ch, b);
            units.insert((at / 16) % 16);
          }
          CHECK(units.size() == 16, "fp8 slot: K read r=%d i=%d c=%d on %zu bank groups", r, i, c, units.size());
        }
    for (int kk = 0; kk < 8; ++kk)
      for (int c0 = 0; c0 < 4; c0 += 2) {
        std::set<int> words;  // the 32 lanes of two adjacent c read 8 bytes each
        for (int c = c0; c < c0 + 2; ++c)
          for (int m = 0; m < 16; ++m) {
            const int R = 8 * c + kk, at = 128 * f8_vrow(R) + 8 * m;
            for (int b = 0; b < 8; ++b) CHECK(vsrc[at + b] == R * 128 + 8 * m + b, "fp8 slot: V row %d byte %d", R, 8 * m + b);
            words.insert((at / 8) % 32);
          }
        CHECK(words.size() == 32, "fp8 slot: V read kk=%d c=%d..%d on %zu bank pairs", kk, c0, c0 + 1, words.size());
      }
  }
  std::printf("decode slots: bf16 and fp8 gathers give every operand read its row and chunk; reads spread over the "
              "bank groups\n");
}

int main() {
  test_prefill();
  test_prefill_streams();
  test_decode();
  test_decode_slots();
  std::printf("%d checks passed\n", g_checks);
  return 0;
}
