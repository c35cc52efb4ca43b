// Host checker for tpu-cake_amd/csrc/rpa_schedule.h (the work decomposition the attention and
// combine kernels share).  For many random batches it builds the unit list the way the kernels
// walk it (sequence-major, kv head, row block, chunk) and checks:
//   * the balanced partition covers units [0, W) exactly once, ranges contiguous, sizes q or q+1;
//   * owner_of(u) is the workgroup whose range holds u;
//   * every row block split across workgroups has exactly one describer (the owner of its last
//     unit, so no two split row blocks share a descriptor), its contributors are the consecutive
//     workgroups owner(first)..owner(last), each workgroup contributes to at most one split row
//     block that began before its range and one that runs past its end, and the partial slots
//     they write (2*b0+1, then 2*b) are distinct across the whole call;
//   * a row block's units visit keys up to the causal limit of its last row and no further, and
//     with a sliding window start at the chunk of the lowest key its first row sees (every key
//     below is masked for every row of the block) and no later;
//   * the heavy split row blocks of a call (kHeavyContrib or more contributors) have distinct
//     helper slots heavy_slot(describer), all below heavy_slots(grid).
// Prints "OK <cases>" or the first violation.
#include <cstdio>
#include <cstdlib>
#include <random>
#include <set>
#include <vector>

#include "rpa_schedule.h"

using namespace rpa;

struct Unit { int seq, h, rb, c, nch; };

static int fail(const char* what, long long a, long long b) {
  std::printf("FAIL %s (%lld, %lld)\n", what, a, b);
  return 1;
}

int main() {
  std::mt19937_64 rng(1234);
  int cases = 0;
  long long heavy_blocks = 0;
  for (int it = 0; it < 400; ++it) {
    const int Hkv = 1 + (int)(rng() % 8);
    const int G = 1 + (int)(rng() % 16);
    const int N = 1 + (int)(rng() % 40);
    const bool skip = rng() % 4 != 0;
    const int window = rng() % 3 == 0 ? 1 + (int)(rng() % 700) : 0;
    std::vector<int> kv(N), ql(N);
    for (int i = 0; i < N; ++i) {
      const int mode = (int)(rng() % 4);
      kv[i] = mode == 0 ? 1 + (int)(rng() % 40) : mode == 1 ? 1 + (int)(rng() % 3000) : 1 + (int)(rng() % 200);
      ql[i] = rng() % 3 == 0 ? 1 + (int)(rng() % kv[i]) : 1;
      if (rng() % 17 == 0) ql[i] = 0;  // an empty sequence
    }
    std::vector<Unit> units;
    for (int i = 0; i < N; ++i) {
      const int per_head = seq_units_per_head(kv[i], ql[i], G, skip, window);
      int sum = 0;
      for (int h = 0; h < Hkv; ++h)
        for (int rb = 0; rb < num_row_blocks(ql[i], G); ++rb) {
          const int n = rb_units(kv[i], ql[i], G, rb, skip, window);
          const int c0 = rb_first_chunk(kv[i], ql[i], G, rb, skip, window);
          const int vis = rb_visible_keys(kv[i], ql[i], G, rb, skip);
          if (vis > 0 && ((c0 + n) * KV_CHUNK < vis || (c0 + n - 1) * KV_CHUNK >= vis))
            return fail("chunks vs visible keys", c0 + n, vis);
          if (vis <= 0 && n != 0) return fail("units of an invisible block", n, vis);
          // the window: no visible key of any row lies below chunk c0, and (a tight start) the
          // first row sees a key of chunk c0
          const int first_row_pos = kv[i] - ql[i] + rb * ROW_BLOCK / G;
          if (window > 0 && skip) {
            const int lowest = first_row_pos - window + 1;  // keys <= pos - window are masked
            if (c0 * KV_CHUNK > (lowest > 0 ? lowest : 0)) return fail("window start past a visible key", c0, lowest);
            if (lowest > 0 && (c0 + 1) * KV_CHUNK <= lowest) return fail("window start not tight", c0, lowest);
          } else if (c0 != 0) {
            return fail("chunk start without a window", c0, window);
          }
          if (skip) {  // causal limit of the block's last existing row
            const int last_row = std::min(ql[i] * G - 1, rb * ROW_BLOCK + ROW_BLOCK - 1);
            const int limit = kv[i] - ql[i] + last_row / G + 1;
            if (vis != std::min(limit, kv[i])) return fail("visible keys", vis, limit);
          } else if (vis != kv[i]) {
            return fail("visible keys (finite mask)", vis, kv[i]);
          }
          for (int c = 0; c < n; ++c) units.push_back({i, h, rb, c, n});
          if (h == 0) sum += n;
        }
      if (sum != per_head) return fail("seq_units_per_head", sum, per_head);
    }
    const long long W = (long long)units.size();
    for (long long grid : {1LL, 7LL, 64LL, 2048LL, W + 3}) {
      if (W == 0) break;
      const Partition pt = make_partition(W, grid);
      std::vector<long long> owner(W, -1);
      for (long long b = 0; b < grid; ++b) {
        const long long u0 = range_start(b, pt), u1 = range_start(b + 1, pt);
        const long long sz = u1 - u0;
        if (sz != pt.q && sz != pt.q + 1) return fail("range size", sz, pt.q);
        if (b > 0 && range_start(b, pt) < range_start(b - 1, pt)) return fail("ranges not monotone", b, 0);
        for (long long u = u0; u < u1; ++u) {
          if (owner[u] != -1) return fail("unit owned twice", u, b);
          owner[u] = b;
        }
      }
      if (range_start(grid, pt) != W) return fail("partition end", range_start(grid, pt), W);
      for (long long u = 0; u < W; ++u) {
        if (owner[u] < 0) return fail("unit unowned", u, 0);
        if (owner_of(u, pt) != owner[u]) return fail("owner_of", owner_of(u, pt), owner[u]);
      }
      // split row blocks: describer, contributors, slots
      std::set<long long> slots, counters, heavy;  // counters: descriptor indices
      std::vector<int> heads(grid, 0), tails(grid, 0);
      long long start = 0;
      while (start < W) {
        const Unit& f = units[start];
        const long long end = start + f.nch;  // units of one row block are consecutive
        for (long long u = start; u < end; ++u)
          if (units[u].seq != f.seq || units[u].h != f.h || units[u].rb != f.rb || units[u].c != u - start)
            return fail("row block not contiguous", start, u);
        const long long b0 = owner_of(start, pt), b1 = owner_of(end - 1, pt);
        if (b0 != b1) {
          // the kernel's view: b0 processes c == 0 (started_here) and runs past its range end;
          // every later contributor starts inside the block; b1 ends it and describes it.
          if (!counters.insert(b1).second) return fail("descriptor reused", b1, b0);
          if (b1 - b0 + 1 >= kHeavyContrib) {
            const int hs = heavy_slot(b1);
            if (hs < 0 || hs >= heavy_slots((int)grid)) return fail("heavy slot out of range", hs, grid);
            if (!heavy.insert(hs).second) return fail("heavy slot shared", hs, b1);
            ++heavy_blocks;
          }
          for (long long b = b0; b <= b1; ++b) {
            if (++(b == b0 ? tails : heads)[b] > 1) return fail("two pieces of one kind", b, b0);
            const long long u0 = range_start(b, pt), u1 = range_start(b + 1, pt);
            if (u1 <= u0) return fail("empty workgroup inside a split row block", b, 0);
            const bool started_here = u0 <= start;
            if (started_here != (b == b0)) return fail("started_here", b, b0);
            const long long slot = partial_slot(b, b == b0);
            if (!slots.insert(slot).second) return fail("partial slot reused", slot, b);
            if (slot < 0 || slot >= 2 * grid) return fail("slot out of range", slot, grid);
          }
        }
        start = end;
      }
    }
    ++cases;
  }
  if (heavy_blocks == 0) return fail("no heavy split row block exercised", 0, 0);
  std::printf("OK %d (%lld heavy split row blocks)\n", cases, heavy_blocks);
  return 0;
}
