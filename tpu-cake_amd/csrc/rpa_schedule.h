// Work decomposition shared by the device kernels and the host-side checker.
//
// A call's work is linearised into UNITS.  One unit is KV_CHUNK consecutive
// keys of one (sequence i, kv head h, row block rb):
//   * a row block is ROW_BLOCK consecutive query rows of sequence i, where
//     query row r <-> (query token r / G, query head h*G + r % G), G = Hq/Hkv
//     (the GQA mapping of ragged_paged_attention.py:130-131);
//   * a row block only visits keys up to the causal limit of its last row,
//     kv_len - q_len + last_token (ragged_paged_attention.py:134-138), so
//     fully masked chunks are never loaded -- exact when the mask value makes
//     masked weights vanish in fp32 (skip_masked); with a finite mask value
//     the reference gives masked keys weight exp(s + mask - m), so every key
//     below kv_len is visited instead;
//   * with a sliding window w (and masked weights that vanish), a row block also
//     starts at the first chunk that holds a key inside the window of its FIRST
//     row (rb_first_chunk): keys at or below pos_first - w are masked for every
//     row of the block (ragged_paged_attention.py:532-534), so their chunks are
//     never loaded either (the reference starts each sequence's KV walk at
//     max(kv_q_gap - window, 0) // bkv, src/tpu_cake/rpa_owned_kernel.py:185-193,
//     :705-712, :748-749).
// Units are ordered sequence-major, then kv head, then row block, then chunk.
// Workgroup b of a grid of `grid` owns units [start(b), start(b+1)): with q = W / grid and
// r = W % grid, the first r workgroups own q + 1 units and the rest q, so every workgroup gets
// the same number of
// KV chunks (+-1) whatever the length distribution ("stream-K").
//
// Everything here is plain integer arithmetic usable on host and device.
#ifndef RPA_SCHEDULE_H_
#define RPA_SCHEDULE_H_

#include <stdint.h>

#ifndef RPA_HD
#if defined(__HIPCC__)
#define RPA_HD __host__ __device__ __forceinline__
#else
#define RPA_HD inline
#endif
#endif

namespace rpa {

constexpr int KV_CHUNK = 32;   // keys per unit (the K extent of one PV MFMA)
constexpr int ROW_BLOCK = 16;  // query rows per row block (the N extent of the MFMAs)

// Keys visible to row block rb (causal limit of its last valid row), or 0.
RPA_HD int rb_visible_keys(int kv_len, int q_len, int group, int rb, bool skip_masked) {
  if (!skip_masked) return kv_len;
  // A block that holds the sequence's last row (row q_len*group - 1) ends at its last token:
  // every decode row block, with no division.
  const bool last_block = (long long)(rb + 1) * ROW_BLOCK >= (long long)q_len * group;
  const int last_tok = last_block ? q_len - 1 : (rb * ROW_BLOCK + ROW_BLOCK - 1) / group;
  int vis = kv_len - q_len + last_tok + 1;
  return vis < kv_len ? vis : kv_len;
}

// First chunk visited by row block rb: 0 without a window (or when masked keys keep a nonzero
// weight), else the chunk of key pos_first - window + 1, the lowest key any row of the block sees.
RPA_HD int rb_first_chunk(int kv_len, int q_len, int group, int rb, bool skip_masked, int window) {
  if (!skip_masked || window <= 0) return 0;
  const int first_tok = rb == 0 ? 0 : rb * ROW_BLOCK / group;
  const long long lo = (long long)kv_len - q_len + first_tok - window + 1;
  return lo > 0 ? (int)(lo / KV_CHUNK) : 0;
}

// Units (chunks) of row block rb: from rb_first_chunk to the chunk of its last visible key.
RPA_HD int rb_units(int kv_len, int q_len, int group, int rb, bool skip_masked, int window) {
  int vis = rb_visible_keys(kv_len, q_len, group, rb, skip_masked);
  if (vis <= 0) return 0;
  const int hi = (vis + KV_CHUNK - 1) / KV_CHUNK;
  const int lo = rb_first_chunk(kv_len, q_len, group, rb, skip_masked, window);
  return hi > lo ? hi - lo : 0;
}

RPA_HD int num_row_blocks(int q_len, int group) {
  return q_len > 0 ? (q_len * group + ROW_BLOCK - 1) / ROW_BLOCK : 0;
}

// Units of one kv head of a sequence (sum over its row blocks).
RPA_HD int seq_units_per_head(int kv_len, int q_len, int group, bool skip_masked, int window) {
  if (q_len <= 0 || kv_len <= 0) return 0;
  if (q_len <= ROW_BLOCK && q_len * group <= ROW_BLOCK)  // one row block (decode): no loop
    return rb_units(kv_len, q_len, group, 0, skip_masked, window);
  int nrb = num_row_blocks(q_len, group);
  int u = 0;
  for (int rb = 0; rb < nrb; ++rb) u += rb_units(kv_len, q_len, group, rb, skip_masked, window);
  return u;
}

// Balanced partition of W units over `grid` workgroups (q = W / grid, r = W % grid): the first
// r workgroups own q + 1 units, the rest q.  Workgroups that own nothing (b >= W when W < grid)
// all come last, so the owners of any unit range are consecutive non-empty workgroups.
struct Partition {
  int64_t q, r;
};

RPA_HD Partition make_partition(int64_t total, int64_t grid) {
  Partition pt;
  pt.q = total / grid;
  pt.r = total - pt.q * grid;
  return pt;
}

// First unit of workgroup b.
RPA_HD int64_t range_start(int64_t b, const Partition& pt) {
  return b * pt.q + (b < pt.r ? b : pt.r);
}

// The workgroup whose range holds unit u.
RPA_HD int64_t owner_of(int64_t u, const Partition& pt) {
  const int64_t big = pt.r * (pt.q + 1);  // units owned by the first r workgroups
  return u < big ? u / (pt.q + 1) : pt.r + (u - big) / pt.q;
}

// Split-K partial slots: each workgroup writes at most two partial segments,
// slot 2b for the segment its range starts inside of (the triple began in an
// earlier workgroup), slot 2b+1 for the segment that begins in b and runs past
// its range end.
RPA_HD int64_t partial_slot(int64_t b, bool started_here) {
  return 2 * b + (started_here ? 1 : 0);
}

// Heavy merges: a split row block with at least kHeavyContrib contributors (a long sequence spread
// over many workgroups) is merged by kHeavySlices helper workgroups per head, each over 32 of the
// 128 dims, instead of one.  Its contributors b0..b span at least kHeavyContrib - 1 workgroup
// boundaries and the next heavy descriptor's first contributor is >= b, so b / (kHeavyContrib - 1)
// differs between any two heavy descriptors of a call: that is its helper slot.
constexpr int kHeavyContrib = 32;
constexpr int kHeavySlices = 4;
RPA_HD constexpr int heavy_slot(int64_t b) { return (int)(b / (kHeavyContrib - 1)); }
RPA_HD constexpr int heavy_slots(int grid) { return (grid - 1) / (kHeavyContrib - 1) + 1; }

}  // namespace rpa

#endif  // RPA_SCHEDULE_H_
