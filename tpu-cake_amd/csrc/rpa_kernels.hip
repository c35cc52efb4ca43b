// Ragged paged attention for MI355X (gfx950): kernels and the C ABI of include/rpa.h.
//
// Semantics: ref_ragged_paged_attention, ecosystem/source/jax/ragged_paged_attention.py:73-148
// (causal offset kv_len - q_len, GQA kv_head = q_head / G, K at combined head 2h and V at
// 2h+1, fp32 scores and softmax, optional sliding window / soft cap / mask value / K,V scales).
//
// Structure (one call = two launches on the caller's stream):
//   rpa_attn_kernel     persistent grid with two roles, split by a cost model every workgroup
//                       evaluates identically from the metadata:
//                       * prefill tiles (sequences with many query tokens): 256-row tiles of one
//                         kv head, K/V chunks staged once per workgroup in LDS (see the prefill
//                         section below);
//                       * stream-K over (sequence, kv-head group, row block, 32-key chunk) units
//                         (see rpa_schedule.h) for the other sequences.  A workgroup is one wave
//                         per kv head of a group of HG heads (HG = the largest divisor of Hkv that
//                         is <= 8): its waves walk the same units in step, wave w computing kv
//                         head group*HG + w, so the HG heads' slices of each key's 2*Hkv*D row are
//                         fetched together (full rows reach HBM far better than isolated per-head
//                         slices); QK^T and PV on v_mfma_f32_16x16x32_bf16; online softmax in fp32
//                         (exp2 domain).  A row block finished inside one workgroup is written
//                         directly; a row block split across workgroups leaves one partial
//                         (m, l, acc) per workgroup, and the workgroup owning its last unit leaves
//                         a descriptor of it.
//   rpa_combine_kernel  one 2- or 4-wave workgroup per (descriptor, head): the partials' (m, l, acc)
//                       folded in one pass with coalesced loads (waves take every 2nd or 4th
//                       contributor, running states merged through LDS); writes the rows,
//                       clears the descriptor; blocks split over 32+ workgroups go to helper
//                       workgroups, four per head, each over 32 dims; resets the prefill tile
//                       queue for the next call.
//
// MFMA operand layouts (16x16x32 bf16, wave64): A[i][k] and B[k][j] place row i / column j
// at lane%16 and the 32 k-slots at (lane/16, element 0..7); D[i][j] sits at lane
// j + 16*(i/4), element i%4.  Only the A/B k-slot correspondence matters for a contraction,
// so k-slots are assigned freely:
//   QK^T  A = K chunk  [16 keys  x 32 dims]  lane%16 = key, slot (j,e) = dim 32s+8j+e
//         B = Q^T      [32 dims  x 16 rows]  lane%16 = query row
//         D = S        lane l holds keys 4j+r (+16 for the second 16-key block), row l%16
//   PV    A = V^T      [16 dims  x 32 keys]  lane%16 = dim, slot (j,e) = key tau(j,e)
//         B = P^T      [32 keys  x 16 rows]  lane%16 = row, slots straight from S's registers
//         D = O^T      lane l holds dims 4j+r (+16 per block), row l%16
//   with tau(j,e) = 16*(e/4) + 4j + e%4: the keys lane (row, j) already holds after QK^T, so
//   P needs no cross-lane movement.  V is stored to LDS as key rows and its A fragments are read
//   with gfx950's transposing LDS read (ds_read_b64_tr_b16), four keys of one dim per read.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <string>
#include <vector>

#include "rpa.h"
#include "rpa_schedule.h"

namespace rpa {
namespace {

constexpr int kD = 128;          // head_dim built
constexpr int kVRow = kD * 2 + 32;            // a 32-key V chunk as key rows of 288 bytes (conflict-free transposing reads)
constexpr int kVtBytes_ = KV_CHUNK * kVRow;  // one wave's V region (prefill tiles lay their buffers over these)
constexpr int kKtRow = kD * 2 + 16;            // the full-line path's K tile: key rows of 272 bytes
constexpr int kKtBytes = KV_CHUNK * kKtRow;
constexpr int kWaveLds = kVtBytes_ + kKtBytes;  // LDS per decode wave: V region + K tile
constexpr int kMaxWavesPerCU = 8;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleLog2 = 8.f;  // lazy softmax rescale threshold (log2 units)
constexpr float kDefaultMask = -0.7f * 3.4028234663852886e38f;  // ragged_paged_attention.py:32

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short short4_t __attribute__((ext_vector_type(4)));

// KV_BF16_BIAS: bf16 KV plus an additive relative-position bias table (the fused Inkling decode).
// KV_BF16_FUSED: the fused Inkling decode step in one attention launch (Params::fused).
enum KvMode { KV_BF16 = 0, KV_BF16_SCALED = 1, KV_FP8 = 2, KV_BF16_BIAS = 3, KV_BF16_FUSED = 4 };

// Per-workgroup timeline of the attention kernel, compiled in only with -DRPA_TIMELINE (the
// library variant tpu_cake_amd.timeline builds; the product library records nothing).  Thread 0
// of workgroup b writes row b: stamps of the 100 MHz constant clock (s_memrealtime) at the
// kernel's phases, the role, work counts, per-tile phase sums of the prefill tiles, and where
// the workgroup ran.  Only the workgroup's own thread 0 reads or writes its row.
enum TlField {
  TL_START = 0,   // kernel entry
  TL_SCHED,       // work split and roles known
  TL_FIRST,       // stream-K: first unit's loads issued (0: no stream-K range)
  TL_DEC,         // stream-K range done
  TL_TILES0,      // prefill-tile role entered (0: none)
  TL_RANKED,      // tile order ready (first queue fetch next)
  TL_END,         // kernel exit
  TL_ROLE,        // bit 0 prefill-first workgroup, bit 1 stream-K range, bit 2 tiles joined after it
  TL_UNITS,       // stream-K units of the range
  TL_NTILES,      // prefill tiles (or tile parts) taken
  TL_NSTEPS,      // 32-key chunk steps of those tiles
  TL_QUEUE,       // clock ticks in queue fetches
  TL_SETUP,       // ticks from a tile's start to its first chunk step (tables, prologue DMAs)
  TL_LOOP,        // ticks in the chunk-step loops
  TL_WRITE,       // ticks from the last step to the tile's rows written
  TL_WHERE,       // XCC_ID << 32 | HW_ID (CU, shader array, shader engine)
  TL_FIELDS
};
#ifdef RPA_TIMELINE
constexpr int kTlRows = 8192;
__device__ long long g_timeline[kTlRows * TL_FIELDS];
__device__ __forceinline__ long long tl_clock() { return (long long)__builtin_amdgcn_s_memrealtime(); }
__device__ __forceinline__ void tl_set(int f, long long v) {
  if (threadIdx.x == 0 && blockIdx.x < kTlRows) g_timeline[blockIdx.x * TL_FIELDS + f] = v;
}
__device__ __forceinline__ void tl_add(int f, long long v) {
  if (threadIdx.x == 0 && blockIdx.x < kTlRows) g_timeline[blockIdx.x * TL_FIELDS + f] += v;
}
__device__ __forceinline__ void tl_begin() {
  if (threadIdx.x == 0 && blockIdx.x < kTlRows) {
    long long* row = g_timeline + blockIdx.x * TL_FIELDS;
    for (int f = 1; f < TL_FIELDS; ++f) row[f] = 0;
    const unsigned xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20);  // XCC_ID[3:0]
    const unsigned hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);   // HW_ID
    row[TL_WHERE] = (long long)xcc << 32 | hw;
  }
}
#define RPA_TL(...) __VA_ARGS__
#else
#define RPA_TL(...)
#endif
// Per-workgroup sums of the prefill tiles' phases, kept in registers (empty without RPA_TIMELINE).
struct TlAcc {
#ifdef RPA_TIMELINE
  long long queue = 0, setup = 0, loop = 0, write = 0, tiles = 0, steps = 0;
#endif
};

// Modes that add a relative-position bias to the scores.
template <int MODE>
constexpr bool has_bias() {
  return MODE == KV_BF16_BIAS || MODE == KV_BF16_FUSED;
}
constexpr int kModes = 5;

enum ErrBits { ERR_PAGE = 1, ERR_QROW = 2, ERR_KVLEN = 4, ERR_QLEN = 8 };

// A row block split across workgroups b0..b (b = the owner of its last unit).
struct SplitDesc {
  int valid[8];  // one flag per wave (kv head of the group); the combine clears its own
  int nch, q_start, q_len, h, rb, pad;  // h = kv-head group
  long long b0;
};


struct Params {
  const uint16_t* q;
  const uint8_t* kv;
  const float* kv_scales;
  const int32_t* kv_lens;
  const int32_t* page_indices;
  const int32_t* cu_q_lens;
  const int32_t* num_seqs;
  uint16_t* out;
  float* part_acc;  // [2*grid][16][kD]
  float* part_ml;   // [2*grid][16][2]  (m in log2 units, l)
  struct SplitDesc* desc;  // [grid] split row block ending in workgroup b (valid = 0 otherwise)
  int32_t* heavy;          // [heavy_slots(grid)][8 heads][kHeavySlices] b + 1 of a heavy descriptor (0 = none)
  struct SplitDesc* heavy_desc;  // [heavy_slots(grid)] copy of the slot's heavy descriptor (read with the flag)
  int32_t* err;
  int T, Hq, Hkv, G, P, S, log2S, Nmax, PPS;
  int HG, NG;  // kv heads per workgroup (one wave each) and kv-head groups (Hkv / HG)
  float sm_scale;
  float scale_log2;  // sm_scale * log2(e)
  float mask_log2;   // mask_value * log2(e)
  float soft_cap;    // 0 = off
  int sliding_window;
  float k_scale, v_scale;
  int grid;
  bool skip_masked;  // mask value so negative that masked keys get weight exactly 0
  const float* rel_bias;  // KV_BF16_BIAS: fp32 table by KEY position (bias_chunk_lo): the bias of each
                          // key, 0 outside the window of the rel_extent keys nearest the (single)
                          // query row, added to its scaled score
  int rel_extent;
  // KV_BF16_FUSED, the fused decode step in one attention launch (src/tpu_cake/rpa_owned_kernel.py:473-522,
  // :811-813 fuse the cache write the same way): the kernel reads the step's own metadata -- one
  // query token per sequence (q row i), num_seqs = fused_nseq, sequence i's pages at
  // page_indices[cu_kv[i] / S + j] -- takes key kv_len-1 of every sequence from new_k / new_v
  // ([B, Hkv, kD] bf16: the token this step writes; the combine kernel stores it into the cache),
  // and forms the relative bias of each score in the kernel (rel_states [B, Hq, 16] @
  // rel_proj[:, kv_len-1-key] for distances below rel_extent, rel_proj [16, E]; rel_states NULL:
  // no bias, rel_proj then 8 zero columns).  fused is set for the combine launch's token stores.
  int fused;
  int fused_nseq;
  int fused_entries;  // length of page_indices in the fused layout
  const int32_t* cu_kv;
  const uint16_t* new_k;
  const uint16_t* new_v;
  const uint16_t* rel_states;
  const uint16_t* rel_proj;
  int pf_tq;         // tokens per prefill tile (0 = prefill tiles off)
  int pf_min;        // sequences with at least this many query tokens take prefill tiles
  float pf_cost;     // cost of one prefill tile chunk in stream-K units (work split model)
  // the prefill kernel (rpa_prefill_kernel): when pf_kernel is set, sequences with at least pf_min
  // query tokens are its tiles of pf_tq tokens (256 rows), the attention kernel skips them and
  // runs no prefill role of its own
  bool pf_kernel;
  // co-resident layout (mixed batches): 4-wave workgroups, two per CU (workgroups b and b + grid/2
  // share a CU); the prefill tiles are 128 rows, one prefill workgroup beside one stream-K
  // workgroup on a CU, and stream-K workgroups join the tile queue when their range is done
  int co;
  int co_split_max;            // split co tiles the workspace holds
  struct CoDesc* co_desc;      // [co_split_max]
  int pk_grid;                 // prefill-kernel workgroups
  float* pk_acc;               // [2 * pk_grid][256][kD] split-tile partials
  float* pk_ml;                // [2 * pk_grid][256][2]
  struct PkDesc* pk_desc;      // [pk_grid] split tile ending in prefill workgroup b
  int D;  // head_dim of q, kv_pages and out rows: kD, or a narrower one (rpa_attn_kernel NW)
};

// A co-resident prefill tile split into nparts chunk ranges: its partials are in slots slot0 ..
// slot0 + nparts - 1 of [slot][128 rows][kD] (acc) and [slot][128 rows][2] (m, l) over the
// prefill-kernel partial areas (unused in that layout); the combine merges them.  Descriptors live
// in an area of their own: fields left by one layout must never read as another's flags.
struct CoDesc {
  int valid[4];  // one per 32-row group; the combine workgroup of that group clears it
  int q_row0;    // first query token of the tile
  int ntok, h, nparts, slot0, pad[3];
};

// A prefill tile split across prefill-kernel workgroups b0..b (b = the owner of its last chunk).
struct PkDesc {
  int valid[16];  // one per 16-row group of the tile; the combine workgroup of that group clears it
  int q_start;    // first query token of the tile (the sequence's first token + tok0)
  int ntok, h, pad;
  long long b0;
};

// ---------------------------------------------------------------------------------------------
// wave helpers
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ int rl(int v, int lane) { return __builtin_amdgcn_readlane(v, lane); }

__device__ __forceinline__ long long rl64(long long v, int lane) {
  int lo = __builtin_amdgcn_readlane((int)(v & 0xffffffffll), lane);
  int hi = __builtin_amdgcn_readlane((int)(v >> 32), lane);
  return ((long long)hi << 32) | (unsigned int)lo;
}

// Wave-uniform value -> SGPR (the compiler cannot prove shuffle results uniform by itself).
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

__device__ __forceinline__ long long uni64(long long v) {
  int lo = __builtin_amdgcn_readfirstlane((int)(v & 0xffffffffll));
  int hi = __builtin_amdgcn_readfirstlane((int)(v >> 32));
  return ((long long)hi << 32) | (unsigned int)lo;
}

__device__ __forceinline__ long long wave_sum64(long long x) {
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return uni64(x);
}

__device__ __forceinline__ long long wave_incl_scan64(long long x, int lane) {
  for (int o = 1; o < 64; o <<= 1) {
    long long y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  return x;
}

// 32-bit wave sum and inclusive scan with DPP moves inside 16-lane rows (VALU, a few cycles a
// step, where a shuffle is an LDS round trip) and the row totals read out with readlane.
// Every lane of the wave must be active.
template <int CTRL, bool BOUND_ZERO>
__device__ __forceinline__ int dpp(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, BOUND_ZERO);
}

__device__ __forceinline__ int wave_sum32(int x) {
  x += dpp<0xB1, false>(x);   // quad_perm [1,0,3,2]
  x += dpp<0x4E, false>(x);   // quad_perm [2,3,0,1]
  x += dpp<0x124, false>(x);  // row_ror:4
  x += dpp<0x128, false>(x);  // row_ror:8: every lane holds its row's total
  return rl(x, 0) + rl(x, 16) + rl(x, 32) + rl(x, 48);
}

__device__ __forceinline__ float wave_sumf(float v) {
  int x = __builtin_bit_cast(int, v);
  v += __builtin_bit_cast(float, dpp<0xB1, false>(x));
  x = __builtin_bit_cast(int, v);
  v += __builtin_bit_cast(float, dpp<0x4E, false>(x));
  x = __builtin_bit_cast(int, v);
  v += __builtin_bit_cast(float, dpp<0x124, false>(x));
  x = __builtin_bit_cast(int, v);
  v += __builtin_bit_cast(float, dpp<0x128, false>(x));
  x = __builtin_bit_cast(int, v);
  return (__builtin_bit_cast(float, rl(x, 0)) + __builtin_bit_cast(float, rl(x, 16))) +
         (__builtin_bit_cast(float, rl(x, 32)) + __builtin_bit_cast(float, rl(x, 48)));
}

__device__ __forceinline__ int wave_incl_scan32(int x, int lane) {
  x += dpp<0x111, true>(x);  // row_shr:1 (lanes shifted in from outside the row read 0)
  x += dpp<0x112, true>(x);  // row_shr:2
  x += dpp<0x114, true>(x);  // row_shr:4
  x += dpp<0x118, true>(x);  // row_shr:8: inclusive scan inside each row
  const int r0 = rl(x, 15), r1 = rl(x, 31), r2 = rl(x, 47), row = lane >> 4;
  return x + (row > 0 ? r0 : 0) + (row > 1 ? r1 : 0) + (row > 2 ? r2 : 0);
}

// The balanced partition (rpa_schedule.h) with a 32-bit division when the total fits.
__device__ __forceinline__ Partition make_partition_fast(long long total, int grid) {
  if (total < (1ll << 31)) {
    Partition pt;
    pt.q = (int)total / grid;
    pt.r = total - pt.q * grid;
    return pt;
  }
  return make_partition(total, grid);
}

// Per-lane unit counts below 2^24 (every realistic batch) take the 32-bit DPP paths.
constexpr long long kSmallUnits = 1ll << 24;

__device__ __forceinline__ long long wave_sum_units(long long x) {
  if (__ballot(x >= kSmallUnits) == 0) return (long long)wave_sum32((int)x);
  return wave_sum64(x);
}

__device__ __forceinline__ long long wave_incl_scan_units(long long x, int lane) {
  if (__ballot(x >= kSmallUnits) == 0) return (long long)wave_incl_scan32((int)x, lane);
  return wave_incl_scan64(x, lane);
}

// Reduce a per-lane value over lanes {l, l^16, l^32, l^48} -- the four 16-lane rows that hold
// one query row's keys -- with gfx950's v_permlane16_swap / v_permlane32_swap (VALU, no LDS).
// permlane16_swap(x, x) returns rows (0,0,2,2) and (1,1,3,3); permlane32_swap returns
// halves (lo,lo) and (hi,hi): combining each pair reduces over all four rows in every lane.
__device__ __forceinline__ float rows4_max(float v) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  v = fmaxf(__builtin_bit_cast(float, (unsigned)a[0]), __builtin_bit_cast(float, (unsigned)a[1]));
  const unsigned w = __builtin_bit_cast(unsigned, v);
  const auto c = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)c[0]), __builtin_bit_cast(float, (unsigned)c[1]));
}

// rows4_max of two values at once, in three swaps: permlane16_swap(a, b) gives rows (a0, b0, a2,
// b2) and (a1, b1, a3, b3), whose maximum w holds a's and b's pairs; permlane32_swap(w, w) and a
// maximum leave (A, B, A, B); permlane16_swap of that gives A in every lane of one result and B in
// every lane of the other.
__device__ __forceinline__ void rows4_max2(float& a, float& b) {
  const auto s1 = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, a), __builtin_bit_cast(unsigned, b),
                                                   false, false);
  const float w = fmaxf(__builtin_bit_cast(float, (unsigned)s1[0]), __builtin_bit_cast(float, (unsigned)s1[1]));
  const unsigned wu = __builtin_bit_cast(unsigned, w);
  const auto s2 = __builtin_amdgcn_permlane32_swap(wu, wu, false, false);
  const float x = fmaxf(__builtin_bit_cast(float, (unsigned)s2[0]), __builtin_bit_cast(float, (unsigned)s2[1]));
  const unsigned xu = __builtin_bit_cast(unsigned, x);
  const auto s3 = __builtin_amdgcn_permlane16_swap(xu, xu, false, false);
  a = __builtin_bit_cast(float, (unsigned)s3[0]);
  b = __builtin_bit_cast(float, (unsigned)s3[1]);
}

__device__ __forceinline__ float rows4_sum(float v) {
  const unsigned u = __builtin_bit_cast(unsigned, v);
  const auto a = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  v = __builtin_bit_cast(float, (unsigned)a[0]) + __builtin_bit_cast(float, (unsigned)a[1]);
  const unsigned w = __builtin_bit_cast(unsigned, v);
  const auto c = __builtin_amdgcn_permlane32_swap(w, w, false, false);
  return __builtin_bit_cast(float, (unsigned)c[0]) + __builtin_bit_cast(float, (unsigned)c[1]);
}

// Orders this wave's accesses to its private LDS tile across lanes.  A wave's LDS instructions
// execute in issue order, so keeping the compiler from moving LDS accesses across this point
// (wavefront-scope fences; no instruction is emitted) is all that is needed.
__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// A zero the compiler cannot see through.  Added to a wave-uniform load index it keeps the loaded
// value in a VGPR: a value the compiler proves uniform is copied to an SGPR right after its load,
// and that copy waits (in-order vmcnt) for every load in flight, including the prefetches.
__device__ __forceinline__ int opaque_zero() {
  int z;
  asm volatile("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}

// A non-temporal (streaming) load: for lines read once, and only where one load instruction covers
// whole 128-byte lines (with half-line loads the second half misses a line already dropped).
template <typename T>
__device__ __forceinline__ T ld_stream(const T* ptr) {
  return __builtin_nontemporal_load(ptr);
}

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int page_of(int kt, const Params& p) {
  return p.log2S >= 0 ? (kt >> p.log2S) : (kt / p.S);
}

__device__ __forceinline__ int slot_of(int kt, const Params& p) {
  return p.log2S >= 0 ? (kt & (p.S - 1)) : (kt % p.S);
}

// Element index of combined head `comb` of key `kt` stored in page `pg`.
// D: the pool's head dim (kD everywhere but the narrow decode instantiation).
__device__ __forceinline__ size_t kv_elem(const Params& p, int pg, int kt, int comb, int D = kD) {
  return (((size_t)pg * (size_t)p.S + (size_t)slot_of(kt, p)) * (size_t)(2 * p.Hkv) + (size_t)comb) *
         (size_t)D;
}

// Head geometry of the decode role: wave wv of kv-head group h computes virtual head v = h * HG +
// wv.  With 256-dim heads (D = 2 kD) every kv head r is two 128-dim virtual heads v = 2r + half,
// paired in one workgroup (HG even): half `half` reads dims 128 half .. +127 of the head's K, V,
// query and output rows and the pair adds its two halves' scores (wide_scores).
__device__ __forceinline__ int real_head(int v, int D) { return D > kD ? v >> 1 : v; }
__device__ __forceinline__ int half_offset(int v, int D) { return D > kD ? kD * (v & 1) : 0; }

// Two floats to bf16 (round to nearest even), lo in the low half: one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// ---------------------------------------------------------------------------------------------
// sequence metadata (range-checked) and the unit -> position walk
// ---------------------------------------------------------------------------------------------
struct SeqInfo {
  int kv_len, q_start, q_len, units;  // units: per kv head
};

// Sequence metadata from raw kv_lens[i], cu_q_lens[i], cu_q_lens[i + 1] (valid = i < num_seqs).
// A sequence with at least pf_min query tokens (pf_min > 0) belongs to the prefill tiles and
// contributes no stream-K units.  Straight-line selects per lane; the row-block loop of
// seq_units_per_head runs only when some lane holds a sequence of more than one row block.
__device__ __forceinline__ SeqInfo make_seq(const Params& p, int kv, int c0, int c1, bool valid, int pf_min,
                                            int& err) {
  const long long cap = (long long)p.PPS * p.S;
  int e = kv > cap ? ERR_KVLEN : 0;
  kv = kv > cap ? (int)cap : (kv < 0 ? 0 : kv);
  int ql = c1 - c0;
  const bool bad_rows = c0 < 0 || ql < 0 || c1 > p.T;
  e |= bad_rows ? ERR_QROW : 0;
  ql = bad_rows ? 0 : ql;
  e |= ql > kv ? ERR_QLEN : 0;
  const bool one_block = ql <= ROW_BLOCK && ql * p.G <= ROW_BLOCK;
  const bool prefill = pf_min > 0 && ql >= pf_min;  // a prefill tile sequence: no units to count
  const bool loop = !one_block && !prefill;
  int units = 0;
  if (ql > 0 && kv > 0) units = rb_units(kv, ql, p.G, 0, p.skip_masked, p.sliding_window);
  if (__ballot(valid && loop) != 0 && loop) units = seq_units_per_head(kv, ql, p.G, p.skip_masked, p.sliding_window);
  if (prefill) units = 0;
  err |= valid ? e : 0;
  SeqInfo s;
  s.kv_len = valid ? kv : 0;
  s.q_start = valid ? c0 : 0;
  s.q_len = valid ? ql : 0;
  s.units = valid ? units : 0;
  return s;
}

// Field-wise conditional copy (value selects keep the windows in registers).
__device__ __forceinline__ void select_seq(SeqInfo& d, const SeqInfo& s, bool c) {
  d.kv_len = c ? s.kv_len : d.kv_len;
  d.q_start = c ? s.q_start : d.q_start;
  d.q_len = c ? s.q_len : d.q_len;
  d.units = c ? s.units : d.units;
}

// Fused decode step (Params::fused): sequence i owns q row i and the page entries from
// cu_kv[i] / S.  Its q_start field carries that first page entry (the q row is i itself); a
// sequence whose cu_kv is negative, not page-aligned, or whose pages run past the page table is
// dropped (no units) and flagged.
__device__ __forceinline__ SeqInfo make_fused_seq(const Params& p, int kv, int cu, int i, bool valid, int& err) {
  SeqInfo s = make_seq(p, kv, i, i + 1, valid, 0, err);
  const int pb = p.log2S >= 0 ? (cu >> p.log2S) : (cu / p.S);
  const int npg = p.log2S >= 0 ? ((s.kv_len + p.S - 1) >> p.log2S) : ((s.kv_len + p.S - 1) / p.S);
  const bool bad = cu < 0 || pb * p.S != cu || (long long)pb + npg > (long long)p.fused_entries;
  err |= valid && bad ? ERR_PAGE : 0;
  s.units = bad ? 0 : s.units;
  s.q_start = bad ? 0 : pb;
  return s;
}

// The fused decode step's metadata is read only by the mode that runs it.
template <int MODE>
__device__ __forceinline__ constexpr bool fused_on(const Params&) {
  return MODE == KV_BF16_FUSED;
}

template <int MODE>
__device__ __forceinline__ SeqInfo load_seq(const Params& p, int i, int nseq, int pf_min, int& err) {
  if (i >= nseq) return SeqInfo{0, 0, 0, 0};
  if (fused_on<MODE>(p)) return make_fused_seq(p, p.kv_lens[i], p.cu_kv[i], i, true, err);
  return make_seq(p, p.kv_lens[i], p.cu_q_lens[i], p.cu_q_lens[i + 1], true, pf_min, err);
}

template <int MODE>
__device__ __forceinline__ long long total_units(const Params& p, int nseq, int lane, int& err) {
  long long w = 0;
  for (int base = 0; base < nseq; base += 64) {
    SeqInfo s = load_seq<MODE>(p, base + lane, nseq, 0, err);
    w += wave_sum_units((long long)s.units * p.NG);
  }
  return w;
}

// Sequence holding unit u and the first unit of that sequence (wave-uniform results).
template <int MODE>
__device__ __forceinline__ void locate_seq(const Params& p, int nseq, int lane, long long u, int& seq,
                                           long long& seq_start, int& err) {
  long long off = 0;
  for (int base = 0; base < nseq; base += 64) {
    SeqInfo s = load_seq<MODE>(p, base + lane, nseq, 0, err);
    long long cnt = (long long)s.units * p.NG;
    long long incl = wave_incl_scan_units(cnt, lane);
    long long tile = rl64(incl, 63);
    if (u < off + tile) {
      unsigned long long below = __ballot(off + incl <= u);
      int idx = __popcll(below);
      seq = uni(base + idx);
      seq_start = uni64(off + rl64(incl - cnt, idx));
      return;
    }
    off += tile;
  }
  seq = nseq;
  seq_start = off;
}

// Per-lane metadata of sequences [base, base + 64); pf_min as in make_seq.
struct Window {
  int base;
  int pf_min;
  SeqInfo s;
};

template <int MODE>
__device__ __forceinline__ void load_window(const Params& p, int nseq, int base, int lane, Window& w, int& err) {
  w.base = base;
  w.s = load_seq<MODE>(p, base + lane, nseq, w.pf_min, err);
}

struct Cursor {
  int i, h, rb, c;  // sequence, kv-head group, row block, chunk (0 .. nch-1 from the block's first)
  int nch;          // chunks of (i, h, rb); 0 = past the end
  int c0;           // first chunk of the row block (rb_first_chunk: > 0 only with a sliding window)
  int nrb;
  int kv_len, q_len, q_start;
  int pbase;  // fused step: the sequence's first page entry
  // first key of the cursor's chunk
  __device__ __forceinline__ int key0() const { return (c0 + c) * KV_CHUNK; }
};

// Chunk range of row block x.rb.
__device__ __forceinline__ void set_row_block(const Params& p, Cursor& x) {
  x.nch = rb_units(x.kv_len, x.q_len, p.G, x.rb, p.skip_masked, p.sliding_window);
  x.c0 = rb_first_chunk(x.kv_len, x.q_len, p.G, x.rb, p.skip_masked, p.sliding_window);
}

template <int MODE>
__device__ __forceinline__ void cursor_load_seq(const Params& p, const Window& w, int i, Cursor& x) {
  int k = i - w.base;
  x.i = i;
  x.kv_len = rl(w.s.kv_len, k);
  x.q_len = rl(w.s.q_len, k);
  const int qs = rl(w.s.q_start, k);
  const bool fz = fused_on<MODE>(p);
  x.q_start = fz ? i : qs;  // fused step: q row i; the field held the first page entry
  x.pbase = fz ? qs : 0;
  x.nrb = num_row_blocks(x.q_len, p.G);
}

template <int MODE>
__device__ __forceinline__ Cursor cursor_at(const Params& p, const Window& w, int seq, long long ul) {
  Cursor x;
  cursor_load_seq<MODE>(p, w, seq, x);
  int per_head = rl(w.s.units, seq - w.base);
  // one kv-head group: no division; else a 32-bit division when it fits
  x.h = p.NG == 1 ? 0 : (ul < (1ll << 31) ? (int)ul / per_head : (int)(ul / per_head));
  int rem = (int)(ul - (long long)x.h * per_head);
  x.rb = 0;
  for (;;) {
    set_row_block(p, x);
    if (rem < x.nch) {
      x.c = rem;
      break;
    }
    rem -= x.nch;
    x.rb++;
  }
  return x;
}

template <int MODE>
__device__ __forceinline__ void advance(const Params& p, int nseq, int lane, Window& w, Cursor& x, int& err) {
  if (x.c + 1 < x.nch) {
    x.c++;
    return;
  }
  x.c = 0;
  for (;;) {
    if (x.rb + 1 < x.nrb) {
      x.rb++;
    } else if (x.h + 1 < p.NG) {
      x.h++;
      x.rb = 0;
    } else {
      int i = x.i;
      for (;;) {
        ++i;
        if (i >= nseq) {
          x.nch = 0;
          return;
        }
        if (i >= w.base + 64) load_window<MODE>(p, nseq, i, lane, w, err);
        if (rl(w.s.units, i - w.base) > 0) break;
      }
      cursor_load_seq<MODE>(p, w, i, x);
      x.h = 0;
      x.rb = 0;
    }
    set_row_block(p, x);
    if (x.nch > 0) return;
  }
}

// ---------------------------------------------------------------------------------------------
// per-unit loads
// ---------------------------------------------------------------------------------------------
// Lane (n = lane%16, j = lane/16) loads keys c*32 + 16*blk + n, dims 32*s + 8*j .. +8.
struct Pages {
  int pg[2];
};

// Loads in the streaming loop are never predicated: lanes past kv_len (and cursors past the
// end of the range, nch == 0) read clamped, always-valid addresses -- key kv_len-1, or row 0 --
// whose values the -inf scores then exclude.  Straight-line loads let the compiler count
// outstanding loads exactly (s_waitcnt vmcnt(N)) so the next unit's loads stay in flight.
// UPG: page_size is a multiple of KV_CHUNK, so a chunk lies in one page and its page id is
// wave-uniform: one scalar load instead of two vector loads per lane.
template <int MODE>
__device__ __forceinline__ size_t page_row(const Params& p, const Cursor& x) {
  if (fused_on<MODE>(p)) return (size_t)x.pbase;
  return (size_t)x.i * p.PPS;
}

template <int MODE, bool UPG>
__device__ __forceinline__ Pages load_pages(const Params& p, const Cursor& x, int n) {
  Pages r;
  if constexpr (UPG) {
    // one load at a wave-uniform address, kept per lane until it is used (a step later)
    const size_t idx = x.nch > 0 ? page_row<MODE>(p, x) + page_of(x.key0(), p) : 0;
    const int pg = p.page_indices[idx + opaque_zero()];
    r.pg[0] = r.pg[1] = pg;
    return r;
  }
  const bool live = x.nch > 0;
  const int last = x.kv_len > 0 ? x.kv_len - 1 : 0;
  const size_t row = live ? page_row<MODE>(p, x) : 0;
  if constexpr (MODE == KV_BF16_FUSED) {
    // the full-line path with pages smaller than a unit: lane L's key key0 + L % 32 -- its page id
    // and its slot in the page (line_addr)
    int kt = x.key0() + (n + 16 * ((threadIdx.x >> 4) & 1));
    kt = live ? (kt < last ? kt : last) : 0;
    r.pg[0] = p.page_indices[row + page_of(kt, p)];
    r.pg[1] = slot_of(kt, p);
    return r;
  }
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    int kt = x.key0() + 16 * blk + n;
    kt = live ? (kt < last ? kt : last) : 0;
    r.pg[blk] = p.page_indices[row + page_of(kt, p)];
  }
  return r;
}

// K and V of one unit for one lane: keys c*32 + 16*blk + n, dims 32*s + 8*j .. +8.
template <int MODE>
struct HalfRegs;

template <>
struct HalfRegs<KV_BF16> {
  u32x4 w[2][4];
};
template <>
struct HalfRegs<KV_BF16_SCALED> {
  u32x4 w[2][4];
};
template <>
struct HalfRegs<KV_BF16_BIAS> {
  u32x4 w[2][4];
  f32x4 bias[2];  // K half only: bias of keys 16*blk + 4j + rr (0 outside the window)
};

// Relative-bias table layout (decode rows: one query position pos = kv_len - 1 per sequence):
// kBiasHead zeros, then one row of bias_row_len(E) entries per (sequence s, q head h).  Entry t of
// a row is the bias of key 32 * bias_chunk_lo(kv_len, E) + t: the first 32-key chunk that holds a
// key of the window [kv_len - E, kv_len - 1], so every chunk from there to the end of the sequence
// lies inside the row, and entries of keys outside the window are 0.  A lane's 4 consecutive keys
// (a multiple-of-4 start) are one aligned 16-byte load; chunks before the window read the zero head.
constexpr int kBiasHead = 32;
constexpr int kRelRows = 16;  // relative-bias width of the fused step's in-kernel bias (rel_states [.., 16])
__host__ __device__ __forceinline__ int bias_row_len(int E) { return ((E + 31) / 32 + 1) * 32; }
__host__ __device__ __forceinline__ int bias_chunk_lo(int kv_len, int E) { return kv_len > E ? (kv_len - E) / 32 : 0; }
template <>
struct HalfRegs<KV_FP8> {
  u32x4 w[2][2];  // 16 codes per load: dims kdim(j, 2i) .. +7 and kdim(j, 2i+1) .. +7 (see kdim)
  float sc[2];    // per-(page, kv head) scale of each of the lane's two keys (k_scale/v_scale not
                  // applied); UPG: the K registers hold the unit's page's (K, V) scales, V's none
};

// The 8 dims lane group j holds in MFMA k-step s (QK^T; the same for K, Q and V rows).  bf16:
// 8j + 32s.  fp8: one 16-byte load covers two k-steps, so lane group j reads bytes 16j .. 16j+15 of
// each 64-byte half of a row -- 64 bytes per row per load instruction, half the requests per byte
// of 8-byte loads.
template <int MODE>
__device__ __forceinline__ int kdim(int j, int s) {
  if constexpr (MODE == KV_FP8) return 16 * j + 64 * (s >> 1) + 8 * (s & 1);
  return 8 * j + 32 * s;
}

// Where this lane's two keys of unit x live (element index of their K row) and their pages.
struct UnitAddr {
  size_t e[2];  // + 8j: dims 8j of the 8-dims-per-lane layout
  int pg[2];
  int h;
  int j8;       // 8j (fp8 adds it again: 16 dims per lane)
  int bias_at;  // KV_BF16_BIAS: table index of this lane's keys c*32 + 4j .. +3 (+16 for the second block)
};

__device__ __forceinline__ UnitAddr unit_addr(const Params& p, const Cursor& x, const Pages& pages, int n, int j,
                                              int wv, int& err, int D = kD) {
  UnitAddr a;
  const bool live = x.nch > 0;
  const int last = x.kv_len > 0 ? x.kv_len - 1 : 0;
  const int v = live ? x.h * p.HG + wv : 0;
  a.h = real_head(v, D);
  a.j8 = 8 * j;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    int kt = x.key0() + 16 * blk + n;
    const bool in_seq = live && kt < x.kv_len;
    kt = live ? (kt < last ? kt : last) : 0;
    int pg = pages.pg[blk];
    const bool pg_ok = pg >= 0 && pg < p.P;
    if (in_seq && !pg_ok) err |= ERR_PAGE;
    pg = pg_ok ? pg : 0;
    a.pg[blk] = pg;
    a.e[blk] = kv_elem(p, pg, kt, 2 * a.h, D) + half_offset(v, D) + 8 * j;
  }
  // relative-bias table position of the scores this lane holds: row n, keys c*32 + 4j .. +3 (the
  // host keeps every index below 2^31); chunks before the window read the zero head
  const int row = x.rb * ROW_BLOCK + n;
  const int lo = bias_chunk_lo(x.kv_len, p.rel_extent);
  const int at = kBiasHead + (x.i * p.Hq + (x.h * p.HG + wv) * p.G + row % p.G) * bias_row_len(p.rel_extent) +
                 (x.c0 + x.c - lo) * KV_CHUNK + 4 * j;
  a.bias_at = live && x.c0 + x.c >= lo ? at : 0;
  return a;
}

// which = 0 loads K (combined head 2h), 1 loads V (2h+1, one row of kD further).
// A narrow pool (D < kD) is read as rows of kD elements from each row's start: the elements past
// D belong to the next row of the key (zero in Q, so they add nothing to a score; in V they only
// reach output dims >= D, which are not stored); pieces wholly past D read the row's first piece
// instead, so no load leaves the key's rows.
template <int MODE, bool UPG>
__device__ __forceinline__ void load_half(const Params& p, const UnitAddr& a, int which, HalfRegs<MODE>& r,
                                          int D = kD) {
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const size_t e = a.e[blk] + (size_t)which * D;
    if constexpr (MODE == KV_BF16_BIAS) {
      if (which == 0) r.bias[blk] = *(const f32x4*)(p.rel_bias + a.bias_at + 16 * blk);  // aligned
    }
    if constexpr (MODE == KV_FP8) {
      const uint8_t* kp = p.kv + e + a.j8;  // bytes 16j (+64) of the row: kdim<KV_FP8>
#pragma unroll
      for (int i = 0; i < 2; ++i) r.w[blk][i] = *(const u32x4*)(kp + (D == kD || 2 * a.j8 + 64 * i < D ? 64 * i : 0));
      // the raw per-(page, head) scale; multiplied in where it is used (to_bf16x8), a step later,
      // so that nothing waits for this load here.  UPG: one page per unit, whose K and V scales
      // (adjacent) come with K in one 8-byte load
      if constexpr (UPG) {
        if (which == 0 && blk == 0) {
          if (p.kv_scales) {
            const f32x2 kvs = *(const f32x2*)(p.kv_scales + ((size_t)a.pg[0] * p.Hkv + a.h) * 2);
            r.sc[0] = kvs[0];
            r.sc[1] = kvs[1];
          } else {
            r.sc[0] = r.sc[1] = 1.f;
          }
        }
      } else {
        r.sc[blk] = p.kv_scales ? p.kv_scales[((size_t)a.pg[blk] * p.Hkv + a.h) * 2 + which] : 1.f;
      }
    } else {
      const uint16_t* kp = (const uint16_t*)p.kv + e;
#pragma unroll
      for (int s = 0; s < 4; ++s) r.w[blk][s] = *(const u32x4*)(kp + (D == kD || a.j8 + 32 * s < D ? 32 * s : 0));
    }
  }
}

// Query rows of cursor x as the B operand of QK^T.  Rows past q_len * G read row 0 of the
// sequence instead: their columns of S and O are never stored, and MFMA columns are independent.
// rst (fused step with a relative bias): components 4j .. 4j+3 of the row's rel_states, loaded
// with its queries (once per row block).
template <int MODE>
__device__ __forceinline__ void load_q(const Params& p, const Cursor& x, int n, int j, int wv, bf16x8 q[4],
                                       uint32_t* rst = nullptr, int D = kD) {
  const bool live = x.nch > 0;
  int row = x.rb * ROW_BLOCK + n;
  if (!(live && row < x.q_len * p.G)) row = 0;
  const int tok = row / p.G;
  const int g = row - tok * p.G;
  const int v = live ? x.h * p.HG + wv : 0;
  const size_t base = live ? (size_t)x.q_start * p.Hq + (size_t)real_head(v, D) * p.G : 0;
  const size_t qrow = (size_t)tok * p.Hq + base + g;
  const uint16_t* qp = p.q + qrow * D + half_offset(v, D);
#pragma unroll
  for (int s = 0; s < 4; ++s) {  // a narrow row's dims past D are zero
    const int d = kdim<MODE>(j, s);
    const bool in = D == kD || d < D;
    const u32x4 w = *(const u32x4*)(qp + (in ? d : 0));
    q[s] = __builtin_bit_cast(bf16x8, in ? w : u32x4{0u, 0u, 0u, 0u});
  }
  if constexpr (MODE == KV_BF16_FUSED) {
    if (rst && p.rel_states) {
      const uint2 sv = *(const uint2*)(p.rel_states + qrow * kRelRows + 4 * j);
      rst[0] = sv.x;
      rst[1] = sv.y;
    }
  }
}

// bf16(float(x) * scale) for 8 packed bf16 values (the reference's k_scale formula, :124-129).
__device__ __forceinline__ u32x4 scale_bf16x8(u32x4 w, float sc) {
  u32x4 o;
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    float lo = __builtin_bit_cast(float, w[t] << 16) * sc;
    float hi = __builtin_bit_cast(float, w[t] & 0xffff0000u) * sc;
    o[t] = pack_bf16x2(lo, hi);
  }
  return o;
}

// 8 OCP e4m3 codes -> bf16(float(x) * scale).
__device__ __forceinline__ u32x4 fp8x8_to_bf16x8(u32x2 w, float sc) {
  u32x4 o;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    auto a = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[t], false);
    auto b = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[t], true);
    o[2 * t] = pack_bf16x2(a[0] * sc, a[1] * sc);
    o[2 * t + 1] = pack_bf16x2(b[0] * sc, b[1] * sc);
  }
  return o;
}

// 8 OCP e4m3 codes -> bf16, exactly (every finite e4m3 value is a bf16 value): gfx950's scaled
// conversion with scale 1 (it applies only the scale's power of two), two codes per instruction.
__device__ __forceinline__ u32x4 fp8x8_to_bf16x8_exact(u32x2 w) {
  u32x4 o;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    o[2 * t] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[t], 1.f, false));
    o[2 * t + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[t], 1.f, true));
  }
  return o;
}

// UPG fp8: a unit's 32 keys share one page, hence one K and one V scale per head, both loaded with
// K (HalfRegs::sc).  K codes convert exactly (e4m3 values are bf16 values) and the K scale
// multiplies the unit's fp32 scores (compute_unit); V keeps the reference's bf16(v * scale) per
// element, with the V scale passed in (vs).  Per-key pages (not UPG) apply bf16(x * scale) to K
// and V elements with each key's own scale.
template <int MODE, bool UPG>
__device__ __forceinline__ u32x4 to_bf16x8(const HalfRegs<MODE>& r, const Params& p, int blk, int s, int which,
                                           float vs = 1.f) {
  if constexpr (MODE == KV_FP8) {
    const u32x4 w4 = r.w[blk][s >> 1];
    const u32x2 c8 = (s & 1) ? u32x2{w4[2], w4[3]} : u32x2{w4[0], w4[1]};  // the codes of k-step s
    if constexpr (UPG) {
      if (which) return fp8x8_to_bf16x8(c8, vs);
      return fp8x8_to_bf16x8_exact(c8);
    } else {
      return fp8x8_to_bf16x8(c8, (which ? p.v_scale : p.k_scale) * r.sc[blk]);
    }
  } else if constexpr (MODE == KV_BF16_SCALED) {
    return scale_bf16x8(r.w[blk][s], which ? p.v_scale : p.k_scale);
  } else {
    return r.w[blk][s];
  }
}

// ---------------------------------------------------------------------------------------------
// the attention kernel
// ---------------------------------------------------------------------------------------------
struct RowState {
  f32x4 acc[8];  // O^T: dims 16*blk + 4j + r, row n
  float m, l;    // running max (log2 units) and this lane's partial sum
  int pos;       // causal limit of this lane's row (last visible key)
  bool started_here;
};

// The unit's scores s0, s1 (keys 16*blk + 4j + rr of row n) -> online-softmax update of st and
// P^T packed for the PV MFMA.  bias (KV_BF16_BIAS): the relative bias of those scores.
template <int MODE>
__device__ __forceinline__ bf16x8 unit_softmax(const Params& p, const Cursor& x, f32x4 s0, f32x4 s1,
                                               const f32x4* bias, RowState& st, int j) {
  // scores in log2 units; this lane holds keys 16*blk + 4j + rr of row n.  A chunk every row
  // of the block sees in full (no window, no soft cap) needs no per-score masking.
  float xs[2][4];
  const int first_row_limit = x.kv_len - x.q_len + (x.rb * ROW_BLOCK) / p.G + 1;  // keys seen by row 0
  bool plain = !(p.soft_cap > 0.f) && p.sliding_window <= 0 &&
               x.key0() + KV_CHUNK <= (first_row_limit < x.kv_len ? first_row_limit : x.kv_len);
  if (!has_bias<MODE>() && plain && p.scale_log2 > 0.f) {
    // the raw scores' maximum, scaled once (a positive scale commutes with each score's rounding),
    // and each probability as exp2(fma(s, scale, -m))
    const float mr = fmaxf(fmaxf(fmaxf(s0[0], s0[1]), fmaxf(s0[2], s0[3])), fmaxf(fmaxf(s1[0], s1[1]), fmaxf(s1[2], s1[3])));
    const float mc = rows4_max(mr) * p.scale_log2;
    const bool grow = mc > st.m + kRescaleLog2;
    if (__ballot(grow)) {
      const float mn = grow ? mc : st.m;
      const float alpha = __builtin_amdgcn_exp2f(st.m - (mn == -INFINITY ? 0.f : mn));
      st.l *= alpha;
#pragma unroll
      for (int d = 0; d < 8; ++d) st.acc[d] *= alpha;
      st.m = mn;
    }
    const float nmu = st.m == -INFINITY ? 0.f : -st.m;
    float pr[2][4];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      pr[0][rr] = __builtin_amdgcn_exp2f(__builtin_fmaf(s0[rr], p.scale_log2, nmu));
      pr[1][rr] = __builtin_amdgcn_exp2f(__builtin_fmaf(s1[rr], p.scale_log2, nmu));
    }
    st.l += ((pr[0][0] + pr[0][1]) + (pr[0][2] + pr[0][3])) + ((pr[1][0] + pr[1][1]) + (pr[1][2] + pr[1][3]));
    u32x4 pw;
    pw[0] = pack_bf16x2(pr[0][0], pr[0][1]);
    pw[1] = pack_bf16x2(pr[0][2], pr[0][3]);
    pw[2] = pack_bf16x2(pr[1][0], pr[1][1]);
    pw[3] = pack_bf16x2(pr[1][2], pr[1][3]);
    return __builtin_bit_cast(bf16x8, pw);
  }
  if (plain) {
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      xs[0][rr] = s0[rr] * p.scale_log2;
      xs[1][rr] = s1[rr] * p.scale_log2;
      if constexpr (has_bias<MODE>()) {  // the bias is 0 for keys outside the window
        xs[0][rr] += bias[0][rr] * kLog2e;
        xs[1][rr] += bias[1][rr] * kLog2e;
      }
    }
  } else {
    const int key0 = x.key0() + 4 * j;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        float sv = blk ? s1[rr] : s0[rr];
        float xv;
        if (p.soft_cap > 0.f) {
          float t = sv * p.sm_scale;
          xv = p.soft_cap * tanhf(t / p.soft_cap) * kLog2e;
        } else {
          xv = sv * p.scale_log2;
        }
        int kt = key0 + 16 * blk + rr;
        if constexpr (has_bias<MODE>()) xv += bias[blk][rr] * kLog2e;
        bool masked = kt > st.pos || (p.sliding_window > 0 && kt <= st.pos - p.sliding_window);
        if (masked) xv += p.mask_log2;
        if (kt >= x.kv_len) xv = -INFINITY;
        xs[blk][rr] = xv;
      }
  }

  // Online softmax with a lazily moved reference: st.m only moves when a row's chunk maximum
  // exceeds it by more than kRescaleLog2 (probabilities then stay <= 2^kRescaleLog2), so most
  // chunks skip the rescale of l and acc.  Any reference gives the same normalised result.
  float mc = fmaxf(fmaxf(fmaxf(xs[0][0], xs[0][1]), fmaxf(xs[0][2], xs[0][3])),
                   fmaxf(fmaxf(xs[1][0], xs[1][1]), fmaxf(xs[1][2], xs[1][3])));
  mc = rows4_max(mc);
  const bool grow = mc > st.m + kRescaleLog2;
  if (__ballot(grow)) {
    const float mn = grow ? mc : st.m;
    const float alpha = __builtin_amdgcn_exp2f(st.m - (mn == -INFINITY ? 0.f : mn));
    st.l *= alpha;
#pragma unroll
    for (int d = 0; d < 8; ++d) st.acc[d] *= alpha;
    st.m = mn;
  }
  const float mu = st.m == -INFINITY ? 0.f : st.m;
  float pr[2][4];
  float lsum = 0.f;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      pr[blk][rr] = __builtin_amdgcn_exp2f(xs[blk][rr] - mu);
      lsum += pr[blk][rr];
    }
  st.l += lsum;

  u32x4 pw;
  pw[0] = pack_bf16x2(pr[0][0], pr[0][1]);
  pw[1] = pack_bf16x2(pr[0][2], pr[0][3]);
  pw[2] = pack_bf16x2(pr[1][0], pr[1][1]);
  pw[3] = pack_bf16x2(pr[1][2], pr[1][3]);
  const bf16x8 pb = __builtin_bit_cast(bf16x8, pw);
  return pb;
}

// The eight A fragments of O^T += V^T P^T from a wave's V chunk stored as key rows (kVRow
// stride): fragment d covers dims 16d .. 16d+15 in the PV key order (k = 8j + 4h + e <-> key
// 16h + 4j + e, the order the QK^T output holds).  ds_read_b64_tr_b16 transposes within each
// 16-lane group: lane n of group j reads dims 16d + 4(n%4) .. +3 of key 16h + 4j + n/4, and lane n
// receives dim 16d + n of keys 16h + 4j .. +3.
template <int ND = 8>  // the first ND 16-dim blocks (narrow heads fill fewer than 8)
__device__ __forceinline__ void read_vt_fragments(const uint8_t* vt, int n, int j, bf16x8 va[8]) {
  typedef __attribute__((address_space(3))) short4_t* lds_s4;
  const uint8_t* vb = vt + (4 * j + (n >> 2)) * kVRow + 8 * (n & 3);
#pragma unroll
  for (int d = 0; d < ND; ++d) {
    const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(vb + 32 * d));
    const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(vb + 16 * kVRow + 32 * d));
    va[d] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
}

// The two halves of a 256-dim head add their scores: each wave of the pair stores its 16 x 32
// tile past the workgroup's wave regions and reads its partner's after a workgroup barrier (every
// wave is at the same unit; the barrier waits for LDS only, the unit's prefetches stay in flight).
// fp32 a + b is commutative, so both halves hold the same scores.  The previous unit's reads of
// these slots finished before the step's opening barrier.
constexpr int kWideSlot = 64 * 2 * 16;  // bytes per wave: 64 lanes x two f32x4
__device__ __forceinline__ void wide_scores(uint8_t* vt, int wv, int lane, int hg, f32x4& s0, f32x4& s1) {
  uint8_t* base = vt - wv * kWaveLds + hg * kWaveLds;
  f32x4* mine = (f32x4*)(base + wv * kWideSlot) + 2 * lane;
  mine[0] = s0;
  mine[1] = s1;
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  const f32x4* other = (const f32x4*)(base + (wv ^ 1) * kWideSlot) + 2 * lane;
  s0 += other[0];
  s1 += other[1];
}

template <int MODE>
__device__ __forceinline__ const f32x4* bias_of(const HalfRegs<MODE>& r) {
  if constexpr (MODE == KV_BF16_BIAS) return r.bias;
  return nullptr;
}

// One unit.  S = K Q^T; V goes to LDS as key rows; then, if the next unit starts a new row block,
// its queries are loaded into q (their registers are free once QK^T has issued), after which the
// next unit's V is loaded into the registers just released; then softmax and O^T += V^T P^T.
template <int MODE, bool UPG>
__device__ __forceinline__ void compute_unit(const Params& p, const Cursor& x, const HalfRegs<MODE>& kr,
                                             const HalfRegs<MODE>& vr, bf16x8 q[4], const Cursor& nx,
                                             const UnitAddr& nx_addr, HalfRegs<MODE>& v_next, RowState& st,
                                             uint8_t* vt, int n, int j, int wv, int D = kD) {
  // S = K Q^T for the two 16-key blocks
  f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    s0 = mfma(__builtin_bit_cast(bf16x8, to_bf16x8<MODE, UPG>(kr, p, 0, s, 0)), q[s], s0);
    s1 = mfma(__builtin_bit_cast(bf16x8, to_bf16x8<MODE, UPG>(kr, p, 1, s, 0)), q[s], s1);
  }
  if constexpr (MODE == KV_FP8 && UPG) {  // the unit's K scale (one page), on the fp32 scores
    const float ks = p.k_scale * kr.sc[0];
    s0 *= ks;
    s1 *= ks;
  }
  if (D > kD) wide_scores(vt, wv, n + 16 * j, p.HG, s0, s1);
  float vs = 1.f;
  if constexpr (MODE == KV_FP8 && UPG) vs = p.v_scale * kr.sc[1];  // the unit's V scale (one page)

  // V into LDS as key rows (key 16*blk + n, kVRow stride), one 16-byte store per 8 dims; the PV
  // A fragments are read back transposed (ds_read_b64_tr_b16)
  wave_lds_fence();
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int s = 0; s < 4; ++s)
      *(u32x4*)(vt + (16 * blk + n) * kVRow + 2 * kdim<MODE>(j, s)) = to_bf16x8<MODE, UPG>(vr, p, blk, s, 1, vs);
  if (nx.c == 0) load_q<MODE>(p, nx, n, j, wv, q, nullptr, D);  // a new row block's queries (as in compute_unit_line)
  load_half<MODE, UPG>(p, nx_addr, 1, v_next, D);

  const bf16x8 pb = unit_softmax<MODE>(p, x, s0, s1, bias_of(kr), st, j);

  wave_lds_fence();
  bf16x8 va[8];
  read_vt_fragments(vt, n, j, va);
#pragma unroll
  for (int d = 0; d < 8; ++d) st.acc[d] = mfma(va[d], pb, st.acc[d]);
  __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);
  __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
}

__device__ __forceinline__ void begin_row_block(const Params& p, const Cursor& x, RowState& st, int n) {
#pragma unroll
  for (int d = 0; d < 8; ++d) st.acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.l = 0.f;
  const int row = x.rb * ROW_BLOCK + n;
  st.pos = x.kv_len - x.q_len + row / p.G;
  st.started_here = x.c == 0;
}

__device__ __forceinline__ void finish_row_block(const Params& p, const Cursor& x, RowState& st, int b,
                                                 bool complete, int n, int j, int wv, int D = kD) {
  const float lt = rows4_sum(st.l);
  if (complete) {
    const int row = x.rb * ROW_BLOCK + n;
    if (row < x.q_len * p.G) {
      const int tok = row / p.G;
      const int v = x.h * p.HG + wv;
      const int head = real_head(v, D) * p.G + (row - tok * p.G);
      const float inv = 1.f / lt;
      uint16_t* op = p.out + ((size_t)(x.q_start + tok) * p.Hq + head) * D + half_offset(v, D) + 4 * j;
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        u32x2 w;
        w[0] = pack_bf16x2(st.acc[d][0] * inv, st.acc[d][1] * inv);
        w[1] = pack_bf16x2(st.acc[d][2] * inv, st.acc[d][3] * inv);
        if (D == kD || 16 * d + 4 * j < D) *(u32x2*)(op + 16 * d) = w;  // a narrow row stores dims < D
      }
    }
  } else {
    // split row block: this workgroup's share, rows that exist only (read by rpa_combine_kernel)
    const int row = x.rb * ROW_BLOCK + n;
    if (row < x.q_len * p.G) {
      const size_t slot = (size_t)partial_slot(b, st.started_here) * p.HG + wv;
      float* ap = p.part_acc + (slot * ROW_BLOCK + n) * kD + 4 * j;
#pragma unroll
      for (int d = 0; d < 8; ++d) *(f32x4*)(ap + 16 * d) = st.acc[d];
      if (j == 0) {
        float* mp = p.part_ml + (slot * ROW_BLOCK + n) * 2;
        mp[0] = st.m;
        mp[1] = lt;
      }
    }
  }
}

// Workgroup b owns the split row block's last unit u: describe the block for the combine (every
// wave writes the same fields, its own valid flag and, for a heavy block, its head's helper flags).
__device__ __forceinline__ void write_split_desc(const Params& p, const Cursor& cur, long long u, const Partition& pt,
                                                 int b, int wv) {
  SplitDesc* d = p.desc + b;
  const long long b0 = owner_of(u - cur.c, pt);
  d->nch = cur.nch;
  d->q_start = cur.q_start;
  d->q_len = cur.q_len;
  d->h = cur.h;
  d->rb = cur.rb;
  d->b0 = b0;
  d->valid[wv] = 1;
  if (b - b0 + 1 >= kHeavyContrib) {
    SplitDesc* hd = p.heavy_desc + heavy_slot(b);
    hd->q_start = cur.q_start;
    hd->q_len = cur.q_len;
    hd->h = cur.h;
    hd->rb = cur.rb;
    hd->b0 = b0;
    int32_t* f = p.heavy + ((size_t)heavy_slot(b) * 8 + wv) * kHeavySlices;
#pragma unroll
    for (int sl = 0; sl < kHeavySlices; ++sl) f[sl] = b + 1;
  }
}

template <int MODE, bool UPG>
__device__ __forceinline__ void step(const Params& p, int nseq, int lane, int n, int j, int b, long long u,
                                     long long u0, long long u1, Window& win, Cursor& cur, Cursor& nxt,
                                     Pages& pg_nxt, const HalfRegs<MODE>& k_cur, const HalfRegs<MODE>& v_cur,
                                     HalfRegs<MODE>& k_nxt, HalfRegs<MODE>& v_nxt, bf16x8 q[4], RowState& st,
                                     uint8_t* vt, int& err, const Partition& pt, int wv, int D = kD) {
  // Prefetch, oldest-needed first: page ids two units ahead, then the next unit's K (its page
  // ids arrived a step ago); its queries and V follow inside compute_unit as registers free up.
  // Every buffer is redefined each step.
  Cursor ahead = nxt;
  if (u + 2 < u1)
    advance<MODE>(p, nseq, lane, win, ahead, err);
  else
    ahead.nch = 0;
  const Pages pg_ahead = load_pages<MODE, UPG>(p, ahead, n);
  const UnitAddr nx_addr = unit_addr(p, nxt, pg_nxt, n, j, wv, err, D);
  // keep the workgroup's waves (the kv heads of one group) in step, so the heads' slices of the
  // same keys reach the memory system together
  __syncthreads();
  load_half<MODE, UPG>(p, nx_addr, 0, k_nxt, D);

  if (u == u0 || cur.c == 0) begin_row_block(p, cur, st, n);
  compute_unit<MODE, UPG>(p, cur, k_cur, v_cur, q, nxt, nx_addr, v_nxt, st, vt, n, j, wv, D);
  const bool last_of_rb = cur.c == cur.nch - 1;
  if (last_of_rb || u == u1 - 1) {
    const bool complete = st.started_here && last_of_rb;
    finish_row_block(p, cur, st, b, complete, n, j, wv, D);
    if (!complete && !st.started_here && last_of_rb && lane == 0) write_split_desc(p, cur, u, pt, b, wv);
  }

  pg_nxt = pg_ahead;
  cur = nxt;
  nxt = ahead;
}


// ---------------------------------------------------------------------------------------------
// full-line decode path (bf16 KV, page size a multiple of 32)
// ---------------------------------------------------------------------------------------------
// The path above loads K and V straight into the MFMA operand layout: 16 keys x 64 bytes per load
// instruction, half of every 128-byte line.  Here a wave loads its kv head's K (then V) rows of a
// unit as whole lines -- load i covers keys 4i .. 4i+3, lane L holding key 4i + L/16, dims
// 8*(L%16) .. +7 -- with non-temporal loads, since every line is read once.  K goes to a
// wave-private LDS tile (key rows, 272-byte stride), written at the end of the step that loaded
// it and read by the next step's QK^T; V goes to the wave's V region (288-byte key rows, one 16-byte
// store per load) and is read back transposed (read_vt_fragments).  Measured on C2's pool (a loads
// + LDS probe of both patterns): 104 vs 111 us per 638 MB.  One K and one V register set suffice:
// K of the next unit lands while this unit's K is read from the tile, V of the next unit is loaded
// once this unit's V is stored.

template <int MODE, bool UPG>
struct LinePath {
  static constexpr bool on =
      MODE == KV_BF16_FUSED || (UPG && (MODE == KV_BF16 || MODE == KV_BF16_SCALED || MODE == KV_BF16_BIAS));
};

struct LineRegs {
  u32x4 w[8];  // load i: key 4i + lane/16, dims 8*(lane%16) .. +7 of the K (or V) row
};

// DN = 32 or 64 (instantiations for those head dims; 0 = rows of kD elements): rows of DN
// elements, load i (i < DN/16) covering keys (512/DN) i .. +512/DN-1, lane L holding key
// (512/DN) i + L/(DN/8), dims 8*(L % (DN/8)) .. +7 -- DN/16 loads per unit half instead of 8,
// each reading whole rows -- and QK^T / PV over the DN/32 k-steps and DN/16 dim blocks those rows
// fill (the K tile's and V region's columns past DN are neither written nor read).
template <int DN>
struct Lines {
  static constexpr int loads = DN ? DN / 16 : 8;      // per unit half
  static constexpr int keys = 32 / loads;             // keys per load
  static constexpr int lanes = 64 / keys;             // lanes per key
  static constexpr int ksteps = DN ? DN / 32 : 4;     // QK^T k-steps of 32 dims
  static constexpr int dblocks = DN ? DN / 16 : 8;    // PV dim blocks of 16
};

struct LineAddr {
  size_t e0;    // element index of this lane's dims of the unit's first key, K row
  int kmax;     // the unit's last key with data (keys past it read it instead)
  int bias_at;  // as UnitAddr
  int knew;       // fused step: the unit's key (0..31) read from new_k / new_v instead, -1 = none
  size_t newoff;  // fused step: element index of this lane's dims of that key's row in new_k / new_v
  int row;        // fused step, pages smaller than a unit: pool row (page * S + slot) of key lane % 32
};

template <int MODE, bool UPG = true, int DN = 0>
__device__ __forceinline__ LineAddr line_addr(const Params& p, const Cursor& x, const Pages& pages, int lane, int n,
                                              int j, int wv, int& err, int D = kD) {
  LineAddr a;
  const bool live = x.nch > 0;
  if constexpr (!UPG) {
    // (the fused step only: D = kD, head v = h * HG + wv) pages smaller than a unit: the keys of
    // one load instruction may lie in different pages; lane L checks the page of key L % 32 and
    // keeps its pool row, which load_lines hands to the lanes that read that key
    static_assert(MODE == KV_BF16_FUSED, "per-key pages on the full-line path: the fused step only");
    const int v = live ? x.h * p.HG + wv : 0;
    const bool in_seq = live && x.key0() + (lane & 31) < x.kv_len;
    const bool pg_ok = pages.pg[0] >= 0 && pages.pg[0] < p.P;
    if (in_seq && !pg_ok) err |= ERR_PAGE;
    a.row = (pg_ok ? pages.pg[0] : 0) * p.S + pages.pg[1];
    a.e0 = (size_t)(2 * v) * kD + 8 * (lane & 15);
    const int k = live ? x.kv_len - 1 - x.key0() : 0;
    a.kmax = k < KV_CHUNK - 1 ? k : KV_CHUNK - 1;
    a.bias_at = 0;
    a.knew = -1;
    a.newoff = 0;
    if (live && k < KV_CHUNK) {
      a.knew = k;
      a.newoff = ((size_t)x.i * p.Hkv + v) * p.D + (8 * (lane & 15) < p.D ? 8 * (lane & 15) : 0);
    }
    return a;
  }
  const UnitAddr u = unit_addr(p, x, pages, n, j, wv, err, D);  // page checks, head, bias position
  a.row = 0;
  // (a narrow pool's pieces wholly past D read the row's first piece, as in load_half)
  const int piece = 8 * (lane & (Lines<DN>::lanes - 1));
  a.e0 = kv_elem(p, u.pg[0], live ? x.key0() : 0, 2 * u.h, D) + half_offset(live ? x.h * p.HG + wv : 0, D) +
         (D == kD || piece < D ? piece : 0);
  const int k = live ? x.kv_len - 1 - x.key0() : 0;
  a.kmax = k < KV_CHUNK - 1 ? k : KV_CHUNK - 1;
  a.bias_at = u.bias_at;
  a.knew = -1;
  a.newoff = 0;
  if constexpr (MODE == KV_BF16_FUSED) {
    // the step's new token (key kv_len-1) is not in the cache yet: its rows come from new_k/new_v
    if (live && k < KV_CHUNK) {  // (rows of p.D elements; pieces past them read the first piece)
      a.knew = k;
      a.newoff = ((size_t)x.i * p.Hkv + u.h) * p.D + (8 * (lane & 15) < p.D ? 8 * (lane & 15) : 0);
    }
  }
  return a;
}

// which = 0: K rows (combined head 2h), 1: V rows (2h+1).
template <int MODE, bool UPG = true, int DN = 0>
__device__ __forceinline__ void load_lines(const Params& p, const LineAddr& a, int lane, int which, LineRegs& r,
                                           int D = kD) {
  const uint16_t* kv = (const uint16_t*)p.kv + a.e0 + (size_t)which * D;
  const size_t row = (size_t)(2 * p.Hkv) * D;
  if constexpr (DN != 0) {
    static_assert(UPG && MODE != KV_BF16_FUSED, "narrow rows: whole-page units, cache rows of D");
    using L = Lines<DN>;
#pragma unroll
    for (int i = 0; i < L::loads; ++i) {
      int key = L::keys * i + lane / L::lanes;
      key = key < a.kmax ? key : a.kmax;
      r.w[i] = ld_stream((const u32x4*)(kv + (size_t)key * row));
    }
    return;
  }
  const uint16_t* nw = nullptr;
  if constexpr (MODE == KV_BF16_FUSED) nw = (which ? p.new_v : p.new_k) + a.newoff;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    int key = 4 * i + (lane >> 4);
    key = key < a.kmax ? key : a.kmax;
    const uint16_t* src;
    if constexpr (UPG)
      src = kv + (size_t)key * row;
    else  // the key's pool row, from lane key (line_addr)
      src = kv + (size_t)__builtin_amdgcn_ds_bpermute(4 * key, a.row) * row;
    if constexpr (MODE == KV_BF16_FUSED) src = key == a.knew ? nw : src;  // the step's new token
    r.w[i] = ld_stream((const u32x4*)src);
  }
}

// The bias inputs of one unit, loaded with its K.  KV_BF16_BIAS: the two f32x4 table entries of
// the lane's keys (as bits).  KV_BF16_FUSED: two 8-element groups of rel_proj rows over the unit's
// distance window (row lane/4, groups lane%4 and 4); the row's rel_states come with its queries
// (load_q).
struct LineBias {
  u32x4 w[2];
};

// Relative bias staging per wave (after the HG wave regions): 16 rel_proj rows x 40 distances
// (bf16), row stride 80 bytes.  A unit's 32 keys have distances dlo .. dlo+31 (dlo = kv_len - 1 -
// key0 - 31); the window holds the five aligned 8-element groups from dlo & ~7.
constexpr int kRelRowBytes = 80;
constexpr int kRelStage = kRelRows * kRelRowBytes;

__device__ __forceinline__ int rel_dlo(const Cursor& x) { return x.kv_len - 1 - x.key0() - (KV_CHUNK - 1); }

template <int MODE>
__device__ __forceinline__ void load_line_bias(const Params& p, const Cursor& x, const LineAddr& a, int lane, int n,
                                               int j, int wv, LineBias& b) {
  if constexpr (MODE == KV_BF16_FUSED) {
    // groups gbase + (lane & 3) and gbase + 4 of rel_proj row lane >> 2 (clamped into the table:
    // groups outside [0, E/8) are zeroed when staged).  A unit with no key in the window reads
    // one 16-byte group at one address (one cache line per instruction).
    const int dlo = rel_dlo(x), gbase = dlo >> 3, ng = p.rel_extent >> 3;
    const bool inw = x.nch > 0 && dlo < p.rel_extent && dlo + KV_CHUNK - 1 >= 0;
    const int r = inw ? lane >> 2 : 0;
    int g0 = gbase + (lane & 3), g1 = gbase + 4;
    g0 = !inw || g0 < 0 ? 0 : (g0 >= ng ? ng - 1 : g0);
    g1 = !inw || g1 < 0 ? 0 : (g1 >= ng ? ng - 1 : g1);
    b.w[0] = *(const u32x4*)(p.rel_proj + (size_t)r * p.rel_extent + 8 * g0);
    b.w[1] = *(const u32x4*)(p.rel_proj + (size_t)r * p.rel_extent + 8 * g1);
  }
  if constexpr (MODE == KV_BF16_BIAS) {
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
      b.w[blk] = *(const u32x4*)(p.rel_bias + a.bias_at + 16 * blk);  // aligned
  }
}


// The bias of the lane's 8 scores (keys 16*blk + 4j + rr of row n) from the unit's LineBias.
// KV_BF16_FUSED: the five groups are staged in the wave's rows, then bias[blk] = P_blk @ S with
// P_blk[key][r] = rel_proj[r][distance of key] (16 x 16, zero outside [0, E)) and S[r][row] =
// rel_states[q head of row][r]: one 16x16x16 bf16 MFMA per 16 keys, fp32 sums of exact products.
template <int MODE>
__device__ __forceinline__ void line_bias_values(const Params& p, const Cursor& x, const LineBias& b,
                                                 const uint32_t rst[2], uint8_t* rs, int lane, int n, int j,
                                                 f32x4 bias[2]) {
  if constexpr (MODE == KV_BF16_FUSED) {
    const int dlo = rel_dlo(x), gbase = dlo >> 3, ng = p.rel_extent >> 3;
    bias[0] = bias[1] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (x.nch <= 0 || dlo >= p.rel_extent || dlo + KV_CHUNK - 1 < 0) return;  // no key in the window
    const int r = lane >> 2, g0 = gbase + (lane & 3), g1 = gbase + 4;
    const u32x4 z = {0u, 0u, 0u, 0u};
    wave_lds_fence();  // the previous unit's fragments have been read
    *(u32x4*)(rs + r * kRelRowBytes + 16 * (lane & 3)) = g0 >= 0 && g0 < ng ? b.w[0] : z;
    if ((lane & 3) == 0) *(u32x4*)(rs + r * kRelRowBytes + 64) = g1 >= 0 && g1 < ng ? b.w[1] : z;
    wave_lds_fence();
    short4_t sb;
    sb[0] = (short)(rst[0] & 0xffffu);
    sb[1] = (short)(rst[0] >> 16);
    sb[2] = (short)(rst[1] & 0xffffu);
    sb[3] = (short)(rst[1] >> 16);
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      const int col = dlo + (KV_CHUNK - 1) - (16 * blk + n) - 8 * gbase;  // 0 .. 38
      short4_t af;
#pragma unroll
      for (int t = 0; t < 4; ++t) af[t] = *(const short*)(rs + (4 * j + t) * kRelRowBytes + 2 * col);
      bias[blk] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(af, sb, f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    }
  }
  if constexpr (MODE == KV_BF16_BIAS) {
    bias[0] = __builtin_bit_cast(f32x4, b.w[0]);
    bias[1] = __builtin_bit_cast(f32x4, b.w[1]);
  }
}

template <int MODE>
__device__ __forceinline__ u32x4 line_word(const LineRegs& r, int i, const Params& p, int which) {
  if constexpr (MODE == KV_BF16_SCALED) return scale_bf16x8(r.w[i], which ? p.v_scale : p.k_scale);
  return r.w[i];
}

// K of a unit into the wave's K tile.
template <int MODE, int DN = 0>
__device__ __forceinline__ void store_k_tile(const Params& p, const LineRegs& k, uint8_t* kt, int lane) {
  wave_lds_fence();  // the tile's previous unit has been read
  using L = Lines<DN>;
#pragma unroll
  for (int i = 0; i < L::loads; ++i)
    *(u32x4*)(kt + (L::keys * i + lane / L::lanes) * kKtRow + (lane % L::lanes) * 16) = line_word<MODE>(k, i, p, 0);
}

// compute_unit with K read from the K tile, V stored as key rows from the line layout and the
// next unit's V loaded into v (after that store).
template <int MODE, bool UPG = true, int DN = 0>
__device__ __forceinline__ void compute_unit_line(const Params& p, const Cursor& x, LineRegs& v, const f32x4* bias,
                                                  bf16x8 q[4], uint32_t rst[2], const Cursor& nx,
                                                  const LineAddr& nx_addr,
                                                  RowState& st, uint8_t* vt, const uint8_t* kt, int lane, int n,
                                                  int j, int wv, int D = kD, int Dq = kD) {
  using L = Lines<DN>;
  f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < L::ksteps; ++s) {
    const bf16x8 a0 = *(const bf16x8*)(kt + n * kKtRow + (32 * s + 8 * j) * 2);
    const bf16x8 a1 = *(const bf16x8*)(kt + (16 + n) * kKtRow + (32 * s + 8 * j) * 2);
    s0 = mfma(a0, q[s], s0);
    s1 = mfma(a1, q[s], s1);
  }
  if (D > kD) wide_scores(vt, wv, lane, p.HG, s0, s1);

  // V as key rows (key 4i + lane/16, kVRow stride), as the K tile; read back transposed below
  wave_lds_fence();
#pragma unroll
  for (int i = 0; i < L::loads; ++i)
    *(u32x4*)(vt + (L::keys * i + lane / L::lanes) * kVRow + (lane % L::lanes) * 16) = line_word<MODE>(v, i, p, 1);
  // a new row block's queries (else q already holds its rows), issued after the wait for this
  // unit's V: vmcnt retires in order and the compiler counts the path without these loads, so
  // issued before it they would make that wait also retire the next unit's K
  if (nx.c == 0) load_q<MODE>(p, nx, n, j, wv, q, rst, Dq);
  load_lines<MODE, UPG, DN>(p, nx_addr, lane, 1, v, D);

  const bf16x8 pb = unit_softmax<MODE>(p, x, s0, s1, bias, st, j);

  wave_lds_fence();
  bf16x8 va[8];
  read_vt_fragments<L::dblocks>(vt, n, j, va);
#pragma unroll
  for (int d = 0; d < L::dblocks; ++d) st.acc[d] = mfma(va[d], pb, st.acc[d]);
  __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);
  __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);
}

template <int MODE, bool UPG, int DN = 0>
__device__ __forceinline__ void step_line(const Params& p, int nseq, int lane, int n, int j, int b, long long u,
                                          long long u0, long long u1, Window& win, Cursor& cur, Cursor& nxt,
                                          Pages& pg_nxt, LineRegs& k, LineRegs& v, f32x4 bias[2], bf16x8 q[4],
                                          uint32_t rst[2], RowState& st, uint8_t* vt, uint8_t* kt, uint8_t* rs,
                                          int& err,
                                          const Partition& pt, int wv, int D = kD) {
  Cursor ahead = nxt;
  if (u + 2 < u1)
    advance<MODE>(p, nseq, lane, win, ahead, err);
  else
    ahead.nch = 0;
  const Pages pg_ahead = load_pages<MODE, UPG>(p, ahead, n);
  const LineAddr nx_addr = line_addr<MODE, UPG, DN>(p, nxt, pg_nxt, lane, n, j, wv, err, D);
  __syncthreads();
  load_lines<MODE, UPG, DN>(p, nx_addr, lane, 0, k, D);  // the next unit's K (this unit's K is in the tile)
  LineBias bias_nx;
  load_line_bias<MODE>(p, nxt, nx_addr, lane, n, j, wv, bias_nx);

  if (u == u0 || cur.c == 0) begin_row_block(p, cur, st, n);
  // the fused step's queries and output rows are p.D wide (its cache rows kD)
  const int Dq = MODE == KV_BF16_FUSED ? p.D : D;
  compute_unit_line<MODE, UPG, DN>(p, cur, v, bias, q, rst, nxt, nx_addr, st, vt, kt, lane, n, j, wv, D, Dq);
  // The next unit's K goes to the tile before a row block's finish stores: its wait then counts
  // the same younger operations (the next unit's V) on every path.  Issued before it, the stores
  // made that wait also retire most of the V just loaded on the steps that end a row block.
  store_k_tile<MODE, DN>(p, k, kt, lane);
  const bool last_of_rb = cur.c == cur.nch - 1;
  if (last_of_rb || u == u1 - 1) {
    const bool complete = st.started_here && last_of_rb;
    finish_row_block(p, cur, st, b, complete, n, j, wv, Dq);
    if (!complete && !st.started_here && last_of_rb && lane == 0) write_split_desc(p, cur, u, pt, b, wv);
  }
  line_bias_values<MODE>(p, nxt, bias_nx, rst, rs, lane, n, j, bias);

  pg_nxt = pg_ahead;
  cur = nxt;
  nxt = ahead;
}

// ---------------------------------------------------------------------------------------------
// prefill tiles (sequences with many query tokens)
// ---------------------------------------------------------------------------------------------
// A tile is (sequence, kv head h, pf_tq consecutive query tokens): rows r = token*G + g (q head
// h*G + g) over the 32*HG rows of a workgroup, wave w owning rows 32w .. 32w+31 as two 16-row
// MFMA blocks.  Each 32-key chunk of kv head h is fetched from HBM once per tile by the whole
// workgroup (a four-deep register ring, three chunks ahead) into double-buffered LDS: K as
// 256-byte key rows whose 16-byte column groups are XOR-swizzled by key % 16 (the A fragment reads
// measured conflict-free; a 272-byte stride reads at half that rate), V as 288-byte key rows read
// back transposed (read_vt_fragments).  Every wave reads its A fragments from LDS and uses each
// for both of its row blocks; softmax as in compute_unit.  Tiles come from a queue (an atomic
// counter in the workspace header, reset by the combine kernel), the last tile of each
// sequence first.
constexpr int kPfKRow = kD * 2;  // K key rows, column groups swizzled (pf_store_chunk, pf_compute)
constexpr int kPfKBytes = KV_CHUNK * kPfKRow;
constexpr int kPfBufBytes = kPfKBytes + KV_CHUNK * kVRow;
constexpr int kPfQWave = 2 * 4 * 64 * 16;  // one wave's Q^T fragments: 2 row blocks x 4 k-steps x 64 lanes x 16 B
constexpr int kPfQBase = 2 * kPfBufBytes;    // the tile's Q fragments follow the two chunk buffers
// prefill tiles run in workgroups of eight waves, whose dynamic LDS is eight decode-wave regions
static_assert(kPfQBase + 8 * kPfQWave <= 8 * kWaveLds, "prefill tile LDS exceeds the workgroup's allocation");
constexpr int kQueueWord = 16;  // int index of the tile counter in the workspace header
constexpr int kXcds = 8;        // the co-resident layout's tile queues: one per XCD, words kQueueWord ..+7
constexpr float kPfCost = 0.45f;  // prefill chunk-step cost in stream-K units (Latin-square search on C3)

struct PfPages {
  int pg[2];  // page ids of this thread's keys (pieces 0 and 1) for one chunk
};

// One ring slot: a chunk's K and V pieces of this thread, and the page ids of a later chunk
// (loaded two steps before they address that chunk's data).
template <int NP>  // 16-byte pieces of K (and of V) per thread per chunk: 512 / threads
struct PfRegs {
  u32x4 k[NP], v[NP];
  PfPages pg;
};

struct PfTile {
  int seq, h;
  int kv_len, q_len, q_start;
  int tok0, ntok;  // first token (sequence-relative) and tokens of the tile
  int c_lo, c_hi;  // chunks visited
};

// Prefill-tile count of a sequence per kv head (0 if it is not a prefill sequence).
__device__ __forceinline__ int pf_tiles_of(const Params& p, const SeqInfo& si, int pf_min) {
  if (pf_min <= 0 || si.q_len < pf_min || si.kv_len <= 0) return 0;
  return (si.q_len + p.pf_tq - 1) / p.pf_tq;
}

// Which K/V piece of a chunk thread tid (of 512) carries: wave w, lane l: key 16*(e/4) + 4*(w/2)
// + e%4 with e = l/8, dims 64*(w%2) + 8*(l%8) .. +8 -- one 16-byte load and one 16-byte LDS store
// each of K and V per thread and chunk.
struct PfPiece {
  int key, d0;
};

__device__ __forceinline__ PfPiece pf_piece(int tid) {
  const int w = tid >> 6, l = tid & 63, e = l >> 3;
  PfPiece pc;
  pc.key = 16 * (e >> 2) + 4 * (w >> 1) + (e & 3);
  pc.d0 = 64 * (w & 1) + 8 * (l & 7);
  return pc;
}

// Raw page ids of this thread's key in chunk c; checked and (UPG) made wave-uniform where they
// are used (pf_load_chunk), two steps later, so that nothing waits for them here.  UPG
// (page_size a multiple of 32): the chunk lies in one page, loaded at one uniform address.
template <int NP, bool UPG>
__device__ __forceinline__ PfPages pf_load_pages(const Params& p, const PfTile& tl, int c, int tid, int nthreads) {
  static_assert(NP == 1, "prefill tiles use 512-thread workgroups");
  PfPages r;
  if constexpr (UPG) {
    r.pg[0] = r.pg[1] = p.page_indices[(size_t)tl.seq * p.PPS + page_of(c * KV_CHUNK, p) + opaque_zero()];
    return r;
  }
  int kt = c * KV_CHUNK + pf_piece(tid).key;
  kt = kt < tl.kv_len ? kt : tl.kv_len - 1;
  r.pg[0] = r.pg[1] = p.page_indices[(size_t)tl.seq * p.PPS + page_of(kt, p)];
  return r;
}

// This thread's K and V pieces of chunk c.  Keys past kv_len read key kv_len - 1 (always written
// data: the scores of such keys are -inf, but their V still meets P = 0 in the PV product).
template <int NP, bool UPG>
__device__ __forceinline__ void pf_load_chunk(const Params& p, const PfTile& tl, int c, const PfPages& pages, int tid,
                                              int nthreads, PfRegs<NP>& r, int& err) {
  const uint16_t* kv = (const uint16_t*)p.kv;
  const PfPiece pc = pf_piece(tid);
  if constexpr (UPG) {
    int pg = uni(pages.pg[0]);
    if (pg < 0 || pg >= p.P) {  // out-of-range page id: never dereferenced
      err |= ERR_PAGE;
      pg = 0;
    }
    const uint16_t* base = kv + kv_elem(p, pg, c * KV_CHUNK, 2 * tl.h);
    const int kmax = tl.kv_len - 1 - c * KV_CHUNK;
    const int off = (pc.key < kmax ? pc.key : kmax) * (2 * p.Hkv * kD) + pc.d0;
    r.k[0] = *(const u32x4*)(base + off);
    r.v[0] = *(const u32x4*)(base + off + kD);
    return;
  }
  int kt = c * KV_CHUNK + pc.key;
  kt = kt < tl.kv_len ? kt : tl.kv_len - 1;
  int pg = pages.pg[0];
  if (pg < 0 || pg >= p.P) {  // out-of-range page id: never dereferenced
    err |= ERR_PAGE;
    pg = 0;
  }
  const size_t e = kv_elem(p, pg, kt, 2 * tl.h) + pc.d0;
  r.k[0] = *(const u32x4*)(kv + e);
  r.v[0] = *(const u32x4*)(kv + e + kD);
}

template <int NP>
__device__ __forceinline__ void pf_store_chunk(uint8_t* buf, const PfRegs<NP>& r, int tid, int nthreads) {
  const PfPiece pc = pf_piece(tid);
  *(u32x4*)(buf + pc.key * kPfKRow + 16 * ((pc.d0 >> 3) ^ (pc.key & 15))) = r.k[0];
  *(u32x4*)(buf + kPfKBytes + pc.key * kVRow + pc.d0 * 2) = r.v[0];  // V as key rows (read_vt_fragments)
}

struct PfRow {
  f32x4 acc[8];
  float m, l;
  int pos;   // last visible key of this lane's row
  bool ok;   // the row exists (token in the tile, pos >= 0)
};

// The lane's maximum of one 16-row block's raw scores of a chunk (keys 16kb + 4j + rr of row n).
__device__ __forceinline__ float pf_lane_max(const f32x4 sc[2]) {
  return fmaxf(fmaxf(fmaxf(sc[0][0], sc[0][1]), fmaxf(sc[0][2], sc[0][3])),
               fmaxf(fmaxf(sc[1][0], sc[1][1]), fmaxf(sc[1][2], sc[1][3])));
}

// One chunk for one 16-row block that every row sees in full (no masking, scale_log2 > 0), given
// the row's maximum raw score of the chunk mraw (rows4_max of pf_lane_max).
__device__ __forceinline__ bf16x8 pf_softmax_plain_m(const Params& p, const f32x4 sc[2], PfRow& st, float mraw) {
  // no masking: the raw scores' maximum, scaled once (scale_log2 > 0, so it commutes with the
  // rounding of each scaled score), and each probability as exp2(fma(s, scale, -m))
  const float mc = mraw * p.scale_log2;
  const bool grow = mc > st.m + kRescaleLog2;
  if (__ballot(grow)) {
    const float mn = grow ? mc : st.m;
    const float alpha = __builtin_amdgcn_exp2f(st.m - (mn == -INFINITY ? 0.f : mn));
    st.l *= alpha;
#pragma unroll
    for (int d = 0; d < 8; ++d) st.acc[d] *= alpha;
    st.m = mn;
  }
  const float nmu = st.m == -INFINITY ? 0.f : -st.m;
  float pr[2][4];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) pr[kb][rr] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[kb][rr], p.scale_log2, nmu));
  st.l += ((pr[0][0] + pr[0][1]) + (pr[0][2] + pr[0][3])) + ((pr[1][0] + pr[1][1]) + (pr[1][2] + pr[1][3]));
  u32x4 pw;
  pw[0] = pack_bf16x2(pr[0][0], pr[0][1]);
  pw[1] = pack_bf16x2(pr[0][2], pr[0][3]);
  pw[2] = pack_bf16x2(pr[1][0], pr[1][1]);
  pw[3] = pack_bf16x2(pr[1][2], pr[1][3]);
  return __builtin_bit_cast(bf16x8, pw);
}

__device__ __forceinline__ bf16x8 pf_softmax_plain(const Params& p, const f32x4 sc[2], PfRow& st) {
  return pf_softmax_plain_m(p, sc, st, rows4_max(pf_lane_max(sc)));
}

// One chunk for one 16-row block: scores sc[kb] (keys 16kb + 4j + rr of row n), softmax update,
// P^T packed for the PV MFMA.
__device__ __forceinline__ bf16x8 pf_softmax(const Params& p, const PfTile& tl, int c, const f32x4 sc[2], PfRow& st,
                                             int j) {
  float xs[2][4];
  {
    const int key0 = c * KV_CHUNK + 4 * j;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const float sv = sc[kb][rr];
        float xv;
        if (p.soft_cap > 0.f) {
          const float t = sv * p.sm_scale;
          xv = p.soft_cap * tanhf(t / p.soft_cap) * kLog2e;
        } else {
          xv = sv * p.scale_log2;
        }
        const int kt = key0 + 16 * kb + rr;
        const bool masked = kt > st.pos || (p.sliding_window > 0 && kt <= st.pos - p.sliding_window);
        if (masked) xv += p.mask_log2;
        if (kt >= tl.kv_len) xv = -INFINITY;
        xs[kb][rr] = xv;
      }
  }
  float mc = fmaxf(fmaxf(fmaxf(xs[0][0], xs[0][1]), fmaxf(xs[0][2], xs[0][3])),
                   fmaxf(fmaxf(xs[1][0], xs[1][1]), fmaxf(xs[1][2], xs[1][3])));
  mc = rows4_max(mc);
  const bool grow = mc > st.m + kRescaleLog2;
  if (__ballot(grow)) {
    const float mn = grow ? mc : st.m;
    const float alpha = __builtin_amdgcn_exp2f(st.m - (mn == -INFINITY ? 0.f : mn));
    st.l *= alpha;
#pragma unroll
    for (int d = 0; d < 8; ++d) st.acc[d] *= alpha;
    st.m = mn;
  }
  const float mu = st.m == -INFINITY ? 0.f : st.m;
  float pr[2][4];
  float lsum = 0.f;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      pr[kb][rr] = __builtin_amdgcn_exp2f(xs[kb][rr] - mu);
      lsum += pr[kb][rr];
    }
  st.l += lsum;
  u32x4 pw;
  pw[0] = pack_bf16x2(pr[0][0], pr[0][1]);
  pw[1] = pack_bf16x2(pr[0][2], pr[0][3]);
  pw[2] = pack_bf16x2(pr[1][0], pr[1][1]);
  pw[3] = pack_bf16x2(pr[1][2], pr[1][3]);
  return __builtin_bit_cast(bf16x8, pw);
}

// One chunk from LDS buffer buf for the wave's two row blocks.
// One chunk from LDS buffer buf for the wave's two row blocks.  The wave's Q^T fragments (B
// operands) come from its LDS copy qs, lane-contiguous per (row block, k-step): registers are the
// prefill role's limit, LDS is not.  PLAIN: every row of the tile sees the chunk in full (no soft
// cap, window or masking; scale_log2 > 0), so the softmax needs no per-score work beyond the
// exponent (pf_softmax_plain); the tile loop runs such chunks in a loop of their own, so neither
// path carries the other's registers.
template <bool PLAIN>
__device__ __forceinline__ void pf_compute(const Params& p, const PfTile& tl, int c, const uint8_t* buf,
                                           const uint8_t* qs, PfRow st[2], int n, int j) {
  const int lane = 16 * j + n;
  f32x4 sc[2][2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) sc[rb][0] = sc[rb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const bf16x8 q0 = *(const bf16x8*)(qs + ((0 * 4 + s) * 64 + lane) * 16);
    const bf16x8 q1 = *(const bf16x8*)(qs + ((1 * 4 + s) * 64 + lane) * 16);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const bf16x8 a = *(const bf16x8*)(buf + (16 * kb + n) * kPfKRow + 16 * ((4 * s + j) ^ n));
      sc[0][kb] = mfma(a, q0, sc[0][kb]);
      sc[1][kb] = mfma(a, q1, sc[1][kb]);
    }
  }
  const uint8_t* vt = buf + kPfKBytes;
  bf16x8 pb0, pb1;
  if constexpr (PLAIN) {
    float m0 = pf_lane_max(sc[0]), m1 = pf_lane_max(sc[1]);
    rows4_max2(m0, m1);  // both row blocks' row maxima in three swaps
    pb0 = pf_softmax_plain_m(p, sc[0], st[0], m0);
    pb1 = pf_softmax_plain_m(p, sc[1], st[1], m1);
  } else {
    pb0 = pf_softmax(p, tl, c, sc[0], st[0], j);
    pb1 = pf_softmax(p, tl, c, sc[1], st[1], j);
  }
  bf16x8 va[8];
  read_vt_fragments(vt, n, j, va);
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    st[0].acc[d] = mfma(va[d], pb0, st[0].acc[d]);
    st[1].acc[d] = mfma(va[d], pb1, st[1].acc[d]);
  }
  // the sixteen fragment reads go out together, then the sixteen MFMAs (not read, wait, MFMA x 8)
  __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);
  __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
}

// Step on chunk c (in LDS buffer c & 1).  Ring slot x % 4 holds chunk x's data and, from two
// steps before that data is fetched, its page ids.  Order matters with in-order vmcnt: page ids
// of chunk c + 5 (into `nx`, whose data, chunk c + 1, is still to be stored), then chunk c + 3's
// data (into `ld`, with the page ids it received two steps ago); compute chunk c; store chunk
// c + 1 (`nx`) to the other LDS buffer.  No wait here needs a load younger than the chunk it
// waits for.
template <int NP, bool UPG, bool PLAIN>
__device__ __forceinline__ void pf_step(const Params& p, const PfTile& tl, int c, uint8_t* lds, const uint8_t* qs,
                                        PfRow st[2], PfRegs<NP>& ld, PfRegs<NP>& nx, int tid, int nthreads, int n,
                                        int j, int& err) {
  const int last = tl.c_hi - 1;
  nx.pg = pf_load_pages<NP, UPG>(p, tl, c + 5 < last ? c + 5 : last, tid, nthreads);
  pf_load_chunk<NP, UPG>(p, tl, c + 3 < last ? c + 3 : last, ld.pg, tid, nthreads, ld, err);
  pf_compute<PLAIN>(p, tl, c, lds + (c & 1) * kPfBufBytes, qs, st, n, j);
  if (c + 1 < tl.c_hi) pf_store_chunk<NP>(lds + ((c + 1) & 1) * kPfBufBytes, nx, tid, nthreads);
  __syncthreads();
}

template <int NP, bool UPG>
__device__ __forceinline__ void pf_tile(const Params& p, const PfTile& tl, uint8_t* lds, int wv, int n, int j,
                                        int& err) {
  const int tid = threadIdx.x, nthreads = 64 * p.HG;
  // queries: row r = 32*wv + 16*rb + n of the tile; B operand dims 32s + 8j .. +8, kept in the
  // wave's LDS region (written before the prologue's barriers, read by this wave only)
  uint8_t* qs = lds + kPfQBase + wv * kPfQWave;
  PfRow st[2];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int r = 32 * wv + 16 * rb + n;
    const int tok = r / p.G, g = r - tok * p.G;
    st[rb].ok = tok < tl.ntok;
    st[rb].pos = tl.kv_len - tl.q_len + tl.tok0 + tok;
    st[rb].ok = st[rb].ok && st[rb].pos >= 0;
    const int qtok = st[rb].ok ? tl.q_start + tl.tok0 + tok : tl.q_start;
    const uint16_t* qp = p.q + ((size_t)qtok * p.Hq + tl.h * p.G + (st[rb].ok ? g : 0)) * kD + 8 * j;
#pragma unroll
    for (int s = 0; s < 4; ++s) *(u32x4*)(qs + ((rb * 4 + s) * 64 + 16 * j + n) * 16) = *(const u32x4*)(qp + 32 * s);
#pragma unroll
    for (int d = 0; d < 8; ++d) st[rb].acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    st[rb].m = -INFINITY;
    st[rb].l = 0.f;
  }

  // ring prologue: page ids of chunks c_lo .. c_lo+4, data of c_lo .. c_lo+2 in flight; c_lo goes
  // to LDS buffer (c_lo & 1)
  const int c0 = tl.c_lo, last = tl.c_hi - 1;
  auto cl = [&](int c) { return c < last ? c : last; };
  PfRegs<NP> r0, r1, r2, r3;
  r0.pg = pf_load_pages<NP, UPG>(p, tl, c0, tid, nthreads);
  r1.pg = pf_load_pages<NP, UPG>(p, tl, cl(c0 + 1), tid, nthreads);
  r2.pg = pf_load_pages<NP, UPG>(p, tl, cl(c0 + 2), tid, nthreads);
  r3.pg = pf_load_pages<NP, UPG>(p, tl, cl(c0 + 3), tid, nthreads);
  pf_load_chunk<NP, UPG>(p, tl, c0, r0.pg, tid, nthreads, r0, err);
  pf_load_chunk<NP, UPG>(p, tl, cl(c0 + 1), r1.pg, tid, nthreads, r1, err);
  pf_load_chunk<NP, UPG>(p, tl, cl(c0 + 2), r2.pg, tid, nthreads, r2, err);
  r0.pg = pf_load_pages<NP, UPG>(p, tl, cl(c0 + 4), tid, nthreads);
  __syncthreads();  // the previous tile's last chunk is no longer read
  pf_store_chunk<NP>(lds + (c0 & 1) * kPfBufBytes, r0, tid, nthreads);
  __syncthreads();

  // chunk c lives in ring slot (c - c0) % 4.  Chunks below cp are seen in full by every row of the
  // tile: they run four at a time in the plain loop; the rest (the diagonal, a window, a soft cap,
  // and up to three plain chunks left over) in the general one, entered at the same ring phase.
  int cp = c0;
  if (!(p.soft_cap > 0.f) && p.sliding_window <= 0 && p.scale_log2 > 0.f) {
    const int pos_min = tl.kv_len - tl.q_len + tl.tok0;  // last key the tile's first row sees
    cp = (pos_min + 1) / KV_CHUNK;
    cp = cp < tl.kv_len / KV_CHUNK ? cp : tl.kv_len / KV_CHUNK;
  }
  int c = c0;
  while (c + 4 <= cp) {
    pf_step<NP, UPG, true>(p, tl, c, lds, qs, st, r3, r1, tid, nthreads, n, j, err);
    pf_step<NP, UPG, true>(p, tl, c + 1, lds, qs, st, r0, r2, tid, nthreads, n, j, err);
    pf_step<NP, UPG, true>(p, tl, c + 2, lds, qs, st, r1, r3, tid, nthreads, n, j, err);
    pf_step<NP, UPG, true>(p, tl, c + 3, lds, qs, st, r2, r0, tid, nthreads, n, j, err);
    c += 4;
  }
  if (c < tl.c_hi)
    for (;;) {
      pf_step<NP, UPG, false>(p, tl, c, lds, qs, st, r3, r1, tid, nthreads, n, j, err);
      if (++c >= tl.c_hi) break;
      pf_step<NP, UPG, false>(p, tl, c, lds, qs, st, r0, r2, tid, nthreads, n, j, err);
      if (++c >= tl.c_hi) break;
      pf_step<NP, UPG, false>(p, tl, c, lds, qs, st, r1, r3, tid, nthreads, n, j, err);
      if (++c >= tl.c_hi) break;
      pf_step<NP, UPG, false>(p, tl, c, lds, qs, st, r2, r0, tid, nthreads, n, j, err);
      if (++c >= tl.c_hi) break;
    }

#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const float lt = rows4_sum(st[rb].l);
    if (!st[rb].ok) continue;
    const int r = 32 * wv + 16 * rb + n;
    const int tok = r / p.G, g = r - tok * p.G;
    const float inv = 1.f / lt;
    uint16_t* op = p.out + ((size_t)(tl.q_start + tl.tok0 + tok) * p.Hq + tl.h * p.G + g) * kD + 4 * j;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      u32x2 w;
      w[0] = pack_bf16x2(st[rb].acc[d][0] * inv, st[rb].acc[d][1] * inv);
      w[1] = pack_bf16x2(st[rb].acc[d][2] * inv, st[rb].acc[d][3] * inv);
      *(u32x2*)(op + 16 * d) = w;
    }
  }
}

// The prefill role of a workgroup: take tiles from the queue until it runs dry.  wsi: the four
// metadata windows (nseq <= 256), total: the call's tile count.
// The chunks a tile visits, from its sequence's kv_len / q_len and its tokens tok0 .. tok0+ntok-1:
// up to the causal limit of its last row, from the sliding-window start of its first row (with a
// finite mask value, where masked keys keep a weight: all of them).
// c_hi <= c_lo: no key to visit (q_len > kv_len: rows left unwritten).
__device__ __forceinline__ void pf_tile_chunks(const Params& p, PfTile& tl) {
  tl.c_lo = tl.c_hi = 0;
  const int prior = tl.kv_len - tl.q_len;
  const int pos_hi = prior + tl.tok0 + tl.ntok - 1;  // last key any row of the tile sees
  if (pos_hi < 0) return;
  if (!p.skip_masked) {  // a finite mask value: masked keys keep a weight, so every key is visited
    tl.c_hi = (tl.kv_len + KV_CHUNK - 1) / KV_CHUNK;
    return;
  }
  int lo = 0;
  if (p.sliding_window > 0) {
    lo = prior + tl.tok0 - p.sliding_window + 1;  // keys below are masked for every row
    lo = lo < 0 ? 0 : lo;
  }
  tl.c_lo = lo / KV_CHUNK;
  tl.c_hi = ((pos_hi < tl.kv_len - 1 ? pos_hi : tl.kv_len - 1) + KV_CHUNK) / KV_CHUNK;
}

// Tile ti of the call's queue order (sequences in window order, each sequence's tiles last token
// block first, kv heads innermost): its sequence, kv head, token block and chunk range.  seq < 0:
// no tile (not reached for ti < total); c_hi <= c_lo: no key to visit.  Wave-collective.
__device__ __forceinline__ PfTile pf_lookup(const Params& p, const SeqInfo wsi[4], int pf_min, int ti, int lane) {
  PfTile tl;
  tl.seq = -1;
  tl.c_lo = tl.c_hi = 0;
  int off = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const int cnt = pf_tiles_of(p, wsi[w], pf_min) * p.Hkv;
    int tot = cnt;
    for (int o = 32; o > 0; o >>= 1) tot += __shfl_xor(tot, o, 64);
    tot = uni(tot);
    if (tl.seq < 0 && ti < off + tot) {
      int incl = cnt;
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o, 64);
        if (lane >= o) incl += y;
      }
      const int idx = __popcll(__ballot(off + incl <= ti));
      const int li = ti - off - rl(incl - cnt, idx);  // tile index inside the sequence
      tl.seq = 64 * w + idx;
      tl.kv_len = rl(wsi[w].kv_len, idx);
      tl.q_len = rl(wsi[w].q_len, idx);
      tl.q_start = rl(wsi[w].q_start, idx);
      const int nt = (tl.q_len + p.pf_tq - 1) / p.pf_tq;
      tl.h = li % p.Hkv;
      const int t = nt - 1 - li / p.Hkv;  // last tile of the sequence first
      tl.tok0 = t * p.pf_tq;
      tl.ntok = tl.q_len - tl.tok0 < p.pf_tq ? tl.q_len - tl.tok0 : p.pf_tq;
    }
    off += tot;
  }
  if (tl.seq < 0) return tl;
  pf_tile_chunks(p, tl);
  return tl;
}

// The queue hands out tiles longest first (longest-processing-time order over the prefill
// workgroups): every workgroup ranks the call's (sequence, token block) pairs by chunk count in
// LDS (ties: queue order, so a sequence's last token block still comes first) and maps queue
// position r to the pair of rank r / Hkv, kv head r % Hkv.  Calls with more pairs than
// kPfOrderMax keep the queue order.
constexpr int kPfOrderMax = 512;
constexpr int kPfOrderBase = kPfQBase + 8 * kPfQWave;  // after the Q fragments
static_assert(kPfOrderBase + 2 * kPfOrderMax * 4 <= 8 * kWaveLds, "prefill tile order exceeds the LDS allocation");

template <int NP, bool UPG>
__device__ __forceinline__ void pf_role(const Params& p, const SeqInfo wsi[4], int pf_min, int total, uint8_t* lds,
                                        int* s_tile, int lane, int wv, int n, int j, int& err) {
  const int npairs = total / p.Hkv;
  const bool ranked = npairs <= kPfOrderMax;
  int* psz = (int*)(lds + kPfOrderBase);  // chunk count of pair i
  int* pord = psz + kPfOrderMax;          // pair of rank r
  if (ranked) {
    for (int i = wv; i < npairs; i += 8) {
      const PfTile t = pf_lookup(p, wsi, pf_min, i * p.Hkv, lane);
      if (lane == 0) psz[i] = t.c_hi > t.c_lo ? t.c_hi - t.c_lo : 0;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < npairs; i += blockDim.x) {
      const int si = psz[i];
      int r = 0;
      for (int k = 0; k < npairs; ++k) {
        const int sk = psz[k];
        r += sk > si || (sk == si && k < i);
      }
      pord[r] = i;
    }
    __syncthreads();
  }
  for (;;) {
    if (threadIdx.x == 0) *s_tile = atomicAdd(p.err + kQueueWord, 1);
    __syncthreads();
    const int tq = uni(*s_tile);
    __syncthreads();
    if (tq >= total) break;
    const int ti = ranked ? uni(pord[tq / p.Hkv]) * p.Hkv + tq % p.Hkv : tq;
    const PfTile tl = pf_lookup(p, wsi, pf_min, ti, lane);
    if (tl.seq < 0 || tl.c_hi <= tl.c_lo) continue;
    pf_tile<NP, UPG>(p, tl, lds, wv, n, j, err);
  }
}

// ---------------------------------------------------------------------------------------------
// prefill tiles of the co-resident layout (Params::co): 4-wave workgroups, 128-row tiles
// ---------------------------------------------------------------------------------------------
// A tile is (sequence, kv head, 128 / G tokens); wave w owns rows 32w .. 32w+31 as two 16-row MFMA
// blocks, its queries in registers.  K/V chunks (32 keys) go from HBM straight into LDS with
// gfx950's global_load_lds_dwordx4 (no registers held for data in flight), into a ring of four
// 16 KiB slots, three chunks ahead of the compute.  Slot layout: K as 256-byte key rows whose
// 16-byte column groups sit at group ^ (key % 16) (conflict-free A fragment reads), then V as
// 256-byte key rows whose 32-byte dim blocks sit at block ^ (key % 8) (conflict-free transposing
// reads, read_vt_fragments_x).  Each DMA instruction writes one contiguous KiB (64 lanes x 16 B);
// the lane's source address picks which piece lands where.  The chunks' page ids come from a
// table the workgroup copies into LDS per segment of up to kCoPages pages.
//
// Waits: the DMA is issued from inline asm, so the compiler neither sees nor counts it, and the
// only loads in the step loop are those DMAs (kCoDmas per wave per chunk).  The step's barrier
// (co_barrier) therefore waits with an exact vmcnt for this wave's share of the chunk it is about
// to read, and the barrier makes every wave's share visible.  (Issued as the compiler's builtin,
// the DMA makes it wait for every DMA in flight before each LDS read it cannot tell apart,
// draining the ring every step.)  No load in asm writes a register: a register the compiler
// believed loaded could be reused before the load lands.
//
// Scaled bf16 and fp8 pools (the reference dequantises K and V as bf16(float(x) * scale),
// ragged_paged_attention.py:124-129) add one pass per chunk, one step ahead of its compute, so the
// step keeps one barrier: scaled bf16 chunks are scaled in place in their ring slot; fp8 chunks
// (half the bytes) land in a ring of four 8 KiB code slots and are converted into a double buffer
// of bf16 slots of the layout above, with the page's K and V scales (per (page, kv head), from a
// table loaded with the page ids).
constexpr int kCoWaves = 4;
constexpr int kCoSlot = 16384;                    // one chunk: K (8 KiB) + V (8 KiB)
constexpr int kCoSlots = 4;
constexpr int kCoCodeSlot = 8192;                 // one fp8 chunk: K codes (4 KiB) + V codes (4 KiB)
constexpr int kCoOrderBase = kCoSlots * kCoSlot;  // tile order tables (2 x kPfOrderMax ints)
constexpr int kCoPages = 128;                     // page-id table entries (and fp8 scale pairs)
constexpr int kCoPageBase = kCoOrderBase + 2 * kPfOrderMax * 4;
constexpr int kCoScaleBase = kCoPageBase + kCoPages * 4;
static_assert(kCoScaleBase + kCoPages * 8 <= kCoWaves * kWaveLds,
              "co-resident prefill LDS exceeds the workgroup's allocation");
static_assert(kCoSlots * kCoCodeSlot + 2 * kCoSlot <= kCoOrderBase, "fp8 code ring and bf16 buffers");

// Modes with co-resident prefill tiles.
template <int MODE>
constexpr bool co_tiles() {
  return MODE == KV_BF16 || MODE == KV_BF16_SCALED || MODE == KV_FP8;
}
template <int MODE>
constexpr int co_dmas() {  // DMA instructions per wave and chunk
  return MODE == KV_FP8 ? 2 : 4;
}
template <int MODE>
constexpr bool co_converts() {  // a pass per chunk one step ahead (scaled or fp8)
  return MODE != KV_BF16;
}

// The step's barrier: this wave's DMAs of the chunk the step reads first (chunk c, or c + 1 for the
// modes that convert one step ahead) have landed -- N younger DMAs may still be in flight -- and
// its LDS reads are done, then s_barrier.  A workgroup-scope release fence (__syncthreads) would
// wait for every DMA in flight.
template <int N>
__device__ __forceinline__ void co_barrier() {
  static_assert(N >= 0 && N < 16, "co_barrier's vmcnt");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(N) : "memory");
}

// Every DMA of this wave has landed.
__device__ __forceinline__ void co_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Byte address in LDS of a pointer into the workgroup's LDS.
__device__ __forceinline__ uint32_t lds_addr_of(const void* ptr) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)ptr;
}

// One 16-byte-per-lane DMA into the 1 KiB of LDS at lds_addr (wave-uniform); m0 is saved and
// restored around it, so the compiler's use of m0 is untouched.
__device__ __forceinline__ void co_dma(const void* src, uint32_t lds_addr) {
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "v"(src), "s"(lds_addr)
      : "memory");
}

// The same DMA with the address split into a wave-uniform base (SGPRs) and a per-lane 32-bit byte
// offset: the form for chunks whose every key exists, whose per-lane offsets are fixed for a tile.
__device__ __forceinline__ void co_dma_s(const void* base, uint32_t off, uint32_t lds_addr) {
  uint32_t save;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(save)
      : "v"(off), "s"(base), "s"(lds_addr)
      : "memory");
}

// Per-lane parts of the DMA addresses, the same for every chunk.  bf16: lane l of wave wv carries,
// for t = 0, 1, key 4i + l/16 of block i = wv + 4t, and 16-byte LDS position l % 16 of that key's K
// row (column group pos ^ (key % 16)) and V row (dims of 32-byte block (pos/2) ^ (key % 8), half
// pos % 2).  fp8 (key[0], colk[0]): key 8 wv + l/8, bytes 16 (l % 8) .. +15 of its 128-byte row.
struct CoLane {
  int key[2];   // key within the chunk
  int colk[2];  // element offset of the K piece within the key's row of kv head h
  int colv[2];  // element offset of the V piece
  uint32_t off[4];  // byte offsets from the chunk's first key row of kv head h: K pieces t = 0, 1, then V
};

template <int MODE>
__device__ __forceinline__ CoLane co_lane(const Params& p, int wv, int lane) {
  CoLane c;
  const uint32_t stride = 2 * p.Hkv * kD;  // elements per key row of the pool
  if constexpr (MODE == KV_FP8) {
    c.key[0] = c.key[1] = 8 * wv + (lane >> 3);
    c.colk[0] = c.colk[1] = 16 * (lane & 7);
    c.colv[0] = c.colv[1] = kD + 16 * (lane & 7);
    c.off[0] = c.off[1] = (uint32_t)c.key[0] * stride + c.colk[0];  // (1-byte elements)
    c.off[2] = c.off[3] = (uint32_t)c.key[0] * stride + c.colv[0];
    return c;
  }
  const int pos = lane & 15;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int k = 4 * (wv + kCoWaves * t) + (lane >> 4);
    c.key[t] = k;
    c.colk[t] = 8 * (pos ^ (k & 15));
    c.colv[t] = kD + 16 * ((pos >> 1) ^ (k & 7)) + 8 * (pos & 1);
    c.off[t] = 2 * ((uint32_t)k * stride + c.colk[t]);
    c.off[2 + t] = 2 * ((uint32_t)k * stride + c.colv[t]);
  }
  return c;
}

// A segment of a tile's chunks whose pages fit the page-id table.
struct CoSeg {
  int c_lo, c_hi;  // chunks
  int p_lo;        // page of chunk c_lo (table entry 0)
  int cps;         // chunks per page (page_size / 32)
};

// This wave's share of chunk c into LDS at dst (wave-uniform LDS address).  bf16: K blocks wv and
// wv + 4 (keys 4i .. 4i+3 each, 1 KiB per DMA) and the same V blocks into a 16 KiB slot; fp8: K
// codes of keys 8 wv .. 8 wv + 7 (1 KiB) and their V codes into an 8 KiB code slot.  Keys past
// kv_len read key kv_len - 1 (scores -inf; V meets P = 0).
template <int MODE>
__device__ __forceinline__ void co_issue(const Params& p, const PfTile& tl, const CoLane& cl, const CoSeg& sg,
                                         const int* ptab, int c, uint32_t dst, int wv, int& err) {
  int pg = uni(ptab[c / sg.cps - sg.p_lo]);
  if (pg < 0 || pg >= p.P) {  // out-of-range page id: never dereferenced
    err |= ERR_PAGE;
    pg = 0;
  }
  const int kmax = tl.kv_len - 1 - c * KV_CHUNK, stride = 2 * p.Hkv * kD;
  if (kmax >= KV_CHUNK - 1) {  // every key of the chunk exists: a uniform base and the lane's fixed offsets
    const uint8_t* base = p.kv + kv_elem(p, pg, c * KV_CHUNK, 2 * tl.h) * (MODE == KV_FP8 ? 1 : 2);
    if constexpr (MODE == KV_FP8) {
      co_dma_s(base, cl.off[0], dst + 1024u * wv);
      co_dma_s(base, cl.off[2], dst + 4096u + 1024u * wv);
    } else {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const uint32_t i = (uint32_t)(wv + kCoWaves * t);
        co_dma_s(base, cl.off[t], dst + 1024u * i);
        co_dma_s(base, cl.off[2 + t], dst + 8192u + 1024u * i);
      }
    }
    return;
  }
  if constexpr (MODE == KV_FP8) {
    const uint8_t* base = p.kv + kv_elem(p, pg, c * KV_CHUNK, 2 * tl.h);
    const uint8_t* row = base + (unsigned)((cl.key[0] < kmax ? cl.key[0] : kmax) * stride);
    co_dma(row + cl.colk[0], dst + 1024u * wv);
    co_dma(row + cl.colv[0], dst + 4096u + 1024u * wv);
    return;
  }
  const uint16_t* base = (const uint16_t*)p.kv + kv_elem(p, pg, c * KV_CHUNK, 2 * tl.h);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const uint32_t i = (uint32_t)(wv + kCoWaves * t);
    const uint16_t* row = base + (unsigned)((cl.key[t] < kmax ? cl.key[t] : kmax) * stride);
    co_dma(row + cl.colk[t], dst + 1024u * i);
    co_dma(row + cl.colv[t], dst + 8192u + 1024u * i);
  }
}

// The pass one step ahead: chunk c's data at src becomes the bf16 slot dst.  Scaled bf16: in place
// (src == dst), every element times its scale, rounded to bf16 (the layout does not matter);
// fp8: thread t converts key t / 8, dims 16 (t % 8) .. +15 of K and V with the page's scales into
// the slot layout (K groups at group ^ (key % 16), V blocks at block ^ (key % 8)).
template <int MODE>
__device__ __forceinline__ void co_convert(const Params& p, const CoSeg& sg, const float* scl, int c, const uint8_t* src,
                                           uint8_t* dst) {
  const int t = threadIdx.x;
  if constexpr (MODE == KV_BF16_SCALED) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      u32x4* w = (u32x4*)(dst + 8192 * h + 32 * t);
      const float sc = h ? p.v_scale : p.k_scale;
      const u32x4 a = w[0], b = w[1];
      w[0] = scale_bf16x8(a, sc);
      w[1] = scale_bf16x8(b, sc);
    }
  } else if constexpr (MODE == KV_FP8) {
    const int key = t >> 3, g = t & 7, e = 2 * (c / sg.cps - sg.p_lo);
    const float ks = scl[e], vs = scl[e + 1];
    const u32x4 kc = *(const u32x4*)(src + key * 128 + 16 * g);
    const u32x4 vc = *(const u32x4*)(src + 4096 + key * 128 + 16 * g);
    uint8_t* krow = dst + key * 256;
    *(u32x4*)(krow + 16 * ((2 * g) ^ (key & 15))) = fp8x8_to_bf16x8(u32x2{kc[0], kc[1]}, ks);
    *(u32x4*)(krow + 16 * ((2 * g + 1) ^ (key & 15))) = fp8x8_to_bf16x8(u32x2{kc[2], kc[3]}, ks);
    uint8_t* vblk = dst + 8192 + key * 256 + 32 * (g ^ (key & 7));
    *(u32x4*)vblk = fp8x8_to_bf16x8(u32x2{vc[0], vc[1]}, vs);
    *(u32x4*)(vblk + 16) = fp8x8_to_bf16x8(u32x2{vc[2], vc[3]}, vs);
  }
}

// Where chunk x's data lands (DMA) and where its bf16 slot is read from (compute).
template <int MODE>
__device__ __forceinline__ uint8_t* co_land(uint8_t* lds, int x) {
  return MODE == KV_FP8 ? lds + (x & (kCoSlots - 1)) * kCoCodeSlot : lds + (x & (kCoSlots - 1)) * kCoSlot;
}
template <int MODE>
__device__ __forceinline__ uint8_t* co_slot(uint8_t* lds, int x) {
  return MODE == KV_FP8 ? lds + kCoSlots * kCoCodeSlot + (x & 1) * kCoSlot : lds + (x & (kCoSlots - 1)) * kCoSlot;
}

// read_vt_fragments for a slot's V rows (256 bytes at slot + 8192, 32-byte blocks at block ^
// (key % 8)).
__device__ __forceinline__ void read_vt_fragments_x(const uint8_t* slot, int n, int j, bf16x8 va[8]) {
  typedef __attribute__((address_space(3))) short4_t* lds_s4;
  const int k = 4 * j + (n >> 2), x = k & 7;  // key of the low half; the high half (k + 16) has the same k % 8
  const uint8_t* vb = slot + 8192 + k * 256 + 8 * (n & 3);
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    const int off = 32 * (d ^ x);
    const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(vb + off));
    const short4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(vb + 16 * 256 + off));
    va[d] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
  }
}

// S = K Q^T of chunk slot buf for the wave's two row blocks: the eight K fragment reads go out
// together, then the sixteen MFMAs.
__device__ __forceinline__ void co_qk(const uint8_t* buf, const bf16x8 q[2][4], f32x4 sc[2][2], int n, int j) {
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) sc[rb][0] = sc[rb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  bf16x8 a[4][2];
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) a[s][kb] = *(const bf16x8*)(buf + (16 * kb + n) * 256 + 16 * ((4 * s + j) ^ n));
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      sc[0][kb] = mfma(a[s][kb], q[0][s], sc[0][kb]);
      sc[1][kb] = mfma(a[s][kb], q[1][s], sc[1][kb]);
    }
  __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);
  __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
}

// Softmax and O += P V of chunk slot buf, the V^T fragments read before the softmax.
template <bool PLAIN>
__device__ __forceinline__ void co_pv(const Params& p, const PfTile& tl, int c, const uint8_t* buf, const f32x4 sc[2][2],
                                      PfRow st[2], int n, int j) {
  bf16x8 va[8];
  read_vt_fragments_x(buf, n, j, va);
  bf16x8 pb0, pb1;
  if constexpr (PLAIN) {
    float m0 = pf_lane_max(sc[0]), m1 = pf_lane_max(sc[1]);
    rows4_max2(m0, m1);  // both row blocks' row maxima in three swaps
    pb0 = pf_softmax_plain_m(p, sc[0], st[0], m0);
    pb1 = pf_softmax_plain_m(p, sc[1], st[1], m1);
  } else {
    pb0 = pf_softmax(p, tl, c, sc[0], st[0], j);
    pb1 = pf_softmax(p, tl, c, sc[1], st[1], j);
  }
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    st[0].acc[d] = mfma(va[d], pb0, st[0].acc[d]);
    st[1].acc[d] = mfma(va[d], pb1, st[1].acc[d]);
  }
}

// Step on chunk c of segment sg.  In flight on entry: the DMAs of c, c + 1, c + 2.  Wait (bf16: for
// this wave's DMAs of c; converting modes: of c + 1, c having been converted by the previous step),
// barrier (every wave's share is in LDS, the previous step's conversion visible, and every wave done
// with chunk c - 1's slot); converting modes: chunk c + 1's pass; S = K Q^T of c; the DMAs of c + 3
// into the freed ring slot (issued while the MFMAs run); the softmax and P V of c.
template <int MODE, bool PLAIN>
__device__ __forceinline__ void co_step(const Params& p, const PfTile& tl, const CoLane& cl, const CoSeg& sg,
                                        const int* ptab, const float* scl, int c, uint8_t* lds, const bf16x8 q[2][4],
                                        PfRow st[2], int wv, int n, int j, int& err) {
  const int last = sg.c_hi - 1;
  co_barrier<(co_converts<MODE>() ? 1 : 2) * co_dmas<MODE>()>();
  if constexpr (co_converts<MODE>()) {
    const int cn = c + 1 < last ? c + 1 : last;
    co_convert<MODE>(p, sg, scl, cn, co_land<MODE>(lds, c + 1), co_slot<MODE>(lds, c + 1));
  }
  const uint8_t* buf = co_slot<MODE>(lds, c);
  f32x4 sc[2][2];
  co_qk(buf, q, sc, n, j);
  const int cn = c + 3 < last ? c + 3 : last;
  co_issue<MODE>(p, tl, cl, sg, ptab, cn, lds_addr_of(co_land<MODE>(lds, c + 3)), wv, err);
  co_pv<PLAIN>(p, tl, c, buf, sc, st, n, j);
}

// slot >= 0: the tile is one part of a split tile, its (m, l, acc) go to that partial slot
template <int MODE>
__device__ __forceinline__ void co_tile(const Params& p, const PfTile& tl, const CoLane& cln, uint8_t* lds, int wv,
                                        int lane, int n, int j, int& err, int slot, TlAcc& ta) {
  RPA_TL(const long long tl_a = tl_clock(); long long tl_b = 0;)
  PfRow st[2];
  bf16x8 q[2][4];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const int r = 32 * wv + 16 * rb + n;
    const int tok = r / p.G, g = r - tok * p.G;
    st[rb].ok = tok < tl.ntok;
    st[rb].pos = tl.kv_len - tl.q_len + tl.tok0 + tok;
    st[rb].ok = st[rb].ok && st[rb].pos >= 0;
    const int qtok = st[rb].ok ? tl.q_start + tl.tok0 + tok : tl.q_start;
    const uint16_t* qp = p.q + ((size_t)qtok * p.Hq + tl.h * p.G + (st[rb].ok ? g : 0)) * kD + 8 * j;
#pragma unroll
    for (int s = 0; s < 4; ++s) q[rb][s] = *(const bf16x8*)(qp + 32 * s);
#pragma unroll
    for (int d = 0; d < 8; ++d) st[rb].acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    st[rb].m = -INFINITY;
    st[rb].l = 0.f;
  }
  // chunks below cp are seen in full by every row (the plain softmax); the rest (the diagonal, a
  // window, a soft cap, masked keys of a finite mask value) take the general one
  int cp = tl.c_lo;
  if (!(p.soft_cap > 0.f) && p.sliding_window <= 0 && p.scale_log2 > 0.f) {
    const int pos_min = tl.kv_len - tl.q_len + tl.tok0;
    cp = (pos_min + 1) / KV_CHUNK;
    cp = cp < tl.kv_len / KV_CHUNK ? cp : tl.kv_len / KV_CHUNK;
  }
  int* ptab = (int*)(lds + kCoPageBase);
  float* scl = (float*)(lds + kCoScaleBase);
  CoSeg sg;
  sg.cps = p.S / KV_CHUNK;
  for (sg.c_lo = tl.c_lo; sg.c_lo < tl.c_hi; sg.c_lo = sg.c_hi) {
    sg.p_lo = sg.c_lo / sg.cps;
    sg.c_hi = (sg.p_lo + kCoPages) * sg.cps;
    sg.c_hi = sg.c_hi < tl.c_hi ? sg.c_hi : tl.c_hi;
    const int npg = (sg.c_hi - 1) / sg.cps - sg.p_lo + 1;
    __syncthreads();  // the previous segment's or tile's tables and slots are no longer read
    for (int t = threadIdx.x; t < npg; t += kCoWaves * 64) {
      const int pg = p.page_indices[(size_t)tl.seq * p.PPS + sg.p_lo + t];
      ptab[t] = pg;
      if constexpr (MODE == KV_FP8) {  // the page's K and V scales of kv head h (page 0's for a bad id)
        f32x2 sv = f32x2{1.f, 1.f};  // times the scalar k_scale / v_scale, as the decode role applies them
        if (p.kv_scales) sv = *(const f32x2*)(p.kv_scales + ((size_t)(pg >= 0 && pg < p.P ? pg : 0) * p.Hkv + tl.h) * 2);
        *(f32x2*)(scl + 2 * t) = f32x2{sv[0] * p.k_scale, sv[1] * p.v_scale};
      }
    }
    // the tables and (first segment) the queries have landed, on every path: the compiler then has
    // no load of its own left to wait for inside the step loop
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    __syncthreads();
    const int c0 = sg.c_lo, last = sg.c_hi - 1;
    auto cl = [&](int c) { return c < last ? c : last; };
#pragma unroll
    for (int k = 0; k < 3; ++k)
      co_issue<MODE>(p, tl, cln, sg, ptab, cl(c0 + k), lds_addr_of(co_land<MODE>(lds, c0 + k)), wv, err);
    if constexpr (co_converts<MODE>()) {  // chunk c0's pass before the loop takes over
      co_barrier<2 * co_dmas<MODE>()>();
      co_convert<MODE>(p, sg, scl, c0, co_land<MODE>(lds, c0), co_slot<MODE>(lds, c0));
    }
    int c = c0;
    RPA_TL(if (tl_b == 0) tl_b = tl_clock();)
    const int cpe = cp < sg.c_hi ? cp : sg.c_hi;
    for (; c < cpe; ++c) co_step<MODE, true>(p, tl, cln, sg, ptab, scl, c, lds, q, st, wv, n, j, err);
    for (; c < sg.c_hi; ++c) co_step<MODE, false>(p, tl, cln, sg, ptab, scl, c, lds, q, st, wv, n, j, err);
    co_drain();  // the clamped DMAs past the segment land before the slots are reused
  }
  RPA_TL(const long long tl_c = tl_clock(); ta.setup += tl_b - tl_a; ta.loop += tl_c - tl_b; ta.tiles += 1;
         ta.steps += tl.c_hi - tl.c_lo;)

  if (slot >= 0) {  // a part of a split tile: its unnormalised state, (m, l) in log2 units
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const float lt = rows4_sum(st[rb].l);
      if (!st[rb].ok) continue;
      const int r = 32 * wv + 16 * rb + n;
      float* ml = p.pk_ml + ((size_t)slot * 128 + r) * 2;
      if (j == 0) *(f32x2*)ml = f32x2{st[rb].m, lt};
      float* acc = p.pk_acc + ((size_t)slot * 128 + r) * kD + 4 * j;
#pragma unroll
      for (int d = 0; d < 8; ++d) *(f32x4*)(acc + 16 * d) = st[rb].acc[d];
    }
    RPA_TL(ta.write += tl_clock() - tl_c;)
    return;
  }
#pragma unroll
  for (int rb = 0; rb < 2; ++rb) {
    const float lt = rows4_sum(st[rb].l);
    if (!st[rb].ok) continue;
    const int r = 32 * wv + 16 * rb + n;
    const int tok = r / p.G, g = r - tok * p.G;
    const float inv = 1.f / lt;
    uint16_t* op = p.out + ((size_t)(tl.q_start + tl.tok0 + tok) * p.Hq + tl.h * p.G + g) * kD + 4 * j;
#pragma unroll
    for (int d = 0; d < 8; ++d) {
      u32x2 w;
      w[0] = pack_bf16x2(st[rb].acc[d][0] * inv, st[rb].acc[d][1] * inv);
      w[1] = pack_bf16x2(st[rb].acc[d][2] * inv, st[rb].acc[d][3] * inv);
      *(u32x2*)(op + 16 * d) = w;
    }
  }
  RPA_TL(ta.write += tl_clock() - tl_c;)
}

// The (sequence, token block) pairs of the call's prefill tiles in queue order (sequences in window
// order, each sequence's token blocks last first), held per lane: lane l's sequence of window w
// owns pairs base[w] + off[w] .. + nt[w] - 1.  One DPP scan per window; a pair's tile then costs
// a ballot and a few readlanes (co_tile_of), not a scan.
struct CoPairs {
  int off[4], nt[4];  // per lane
  int base[5];        // uniform; base[4] = pairs in all
};

__device__ __forceinline__ CoPairs co_pairs(const Params& p, const SeqInfo wsi[4], int pf_min, int lane) {
  CoPairs cp;
  int base = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const int nt = pf_tiles_of(p, wsi[w], pf_min);
    const int incl = wave_incl_scan32(nt, lane);
    cp.nt[w] = nt;
    cp.off[w] = incl - nt;
    cp.base[w] = base;
    base += rl(incl, 63);
  }
  cp.base[4] = base;
  return cp;
}

// The tile of pair pi (< base[4]) and kv head h.  Wave-collective.
__device__ __forceinline__ PfTile co_tile_of(const Params& p, const SeqInfo wsi[4], const CoPairs& cp, int pi, int h) {
  PfTile tl;
  tl.seq = -1;
  tl.c_lo = tl.c_hi = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    if (pi >= cp.base[w] && pi < cp.base[w + 1]) {
      const int r = pi - cp.base[w];
      // the last lane whose first pair is <= r holds pair r (offsets never decrease, and a later lane
      // with no pairs has an offset above r)
      const int idx = __popcll(__ballot(cp.off[w] <= r)) - 1;
      const int k = r - rl(cp.off[w], idx), nt = rl(cp.nt[w], idx);
      tl.seq = 64 * w + idx;
      tl.kv_len = rl(wsi[w].kv_len, idx);
      tl.q_len = rl(wsi[w].q_len, idx);
      tl.q_start = rl(wsi[w].q_start, idx);
      tl.h = h;
      tl.tok0 = (nt - 1 - k) * p.pf_tq;  // last token block first
      tl.ntok = tl.q_len - tl.tok0 < p.pf_tq ? tl.q_len - tl.tok0 : p.pf_tq;
    }
  }
  if (tl.seq >= 0) pf_tile_chunks(p, tl);
  return tl;
}

// Splitting: a call whose tiles are fewer than the grid's workgroups (the queue cannot keep them
// all busy) cuts every tile longer than kCoMinSplit chunks into up to np equal chunk ranges
// (units), np = min(kCoMaxParts, grid / tiles), each unit's partial merged by the combine kernel.
// Unit u = pair * np + part; parts past a short tile's own count are empty.  Units are ranked
// longest first by a 32-bit key: chunk count (15 bits) over the unit index (16 bits).
constexpr int kCoMaxParts = 4;
constexpr int kCoMinSplit = 16;  // tiles of up to this many chunks (512 keys) are never split

// Chunk count of pair k (0 = the last token block) of a sequence with nt token blocks.
__device__ __forceinline__ int co_pair_size(const Params& p, int kv_len, int q_len, int nt, int k) {
  PfTile t;
  t.kv_len = kv_len;
  t.q_len = q_len;
  t.tok0 = (nt - 1 - k) * p.pf_tq;
  t.ntok = q_len - t.tok0 < p.pf_tq ? q_len - t.tok0 : p.pf_tq;
  pf_tile_chunks(p, t);
  return t.c_hi > t.c_lo ? t.c_hi - t.c_lo : 0;
}

// Parts of a tile of sz chunks when the call splits into np.
__device__ __forceinline__ int co_tile_parts(int sz, int np) {
  if (np <= 1 || sz <= kCoMinSplit) return 1;
  const int k = (sz + kCoMinSplit - 1) / kCoMinSplit;  // parts of at least kCoMinSplit chunks
  return k < np ? k : np;
}

// The co-resident layout's prefill role: take units from the queue until it runs dry.  The
// workgroup writes every unit's key (one thread per unit: a binary search over the sequences'
// first pairs finds its sequence), ranks them in LDS and maps queue position r to the unit of rank
// r / Hkv, kv head r % Hkv.  Calls with more units than kPfOrderMax keep the pair order unsplit.
template <int MODE>
__device__ __forceinline__ void co_role(const Params& p, const SeqInfo wsi[4], int pf_min, uint8_t* lds, int* s_tile,
                                        int lane, int wv, int n, int j, int& err, int gpre, bool pf_first) {
  RPA_TL(tl_set(TL_TILES0, tl_clock());)
  // fixed first positions when every CU holds a prefill-first workgroup (below): b and b + grid/2
  // share a CU and an XCD (b mod 8), so the pair's positions in that XCD's queue are k and
  // sn - 1 - k, with k the CU's rank on its XCD
  int sq = -1, sn = 0;
  {
    const int half = p.grid >> 1, b = blockIdx.x;
    if (gpre == half && (half & (kXcds - 1)) == 0) {
      const int per = half / kXcds;  // CUs per XCD
      sn = 2 * per;
      sq = pf_first ? (b - half) / kXcds : 2 * per - 1 - b / kXcds;
    }
  }
  TlAcc ta;
  const CoPairs cp = co_pairs(p, wsi, pf_min, lane);
  const int npairs = cp.base[4];
  int np = 1;
  if (npairs * p.Hkv < p.grid && npairs * p.Hkv <= p.co_split_max) {
    np = p.grid / (npairs * p.Hkv);
    np = np < kCoMaxParts ? np : kCoMaxParts;
    if (npairs * np > kPfOrderMax) np = kPfOrderMax / npairs;
    np = np < 1 ? 1 : np;
  }
  const int nunits = npairs * np;
  const bool ranked = nunits <= kPfOrderMax;
  int nvalid = nunits;
  int* pkey = (int*)(lds + kCoOrderBase);
  int* pord = pkey + kPfOrderMax;
  const CoLane cln = co_lane<MODE>(p, wv, lane);
  if (ranked) {
    // per sequence (256 entries each, over pord's area and the page table until they are
    // written): its first pair (the exclusive scan of the pair counts: never decreasing, and a
    // sequence with no pairs shares its successor's), kv_len, q_len
    int* sq_off = pord;
    int* sq_kv = pord + 256;
    int* sq_ql = (int*)(lds + kCoPageBase);
    static_assert(kCoPages * 12 >= 256 * 4, "sequence table over the page-id and scale tables");
    if (wv == 0) {
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int i = 64 * w + lane;
        sq_off[i] = cp.base[w] + cp.off[w];
        sq_kv[i] = wsi[w].kv_len;
        sq_ql[i] = wsi[w].q_len;
      }
    }
    __syncthreads();
    for (int u = threadIdx.x; u < nunits; u += blockDim.x) {
      const int pair = u / np, part = u - pair * np;
      int seq = 0;  // the last sequence whose first pair is <= pair (sq_off[0] = 0)
#pragma unroll
      for (int step = 128; step > 0; step >>= 1)
        if (sq_off[seq + step] <= pair) seq += step;
      const int k = pair - sq_off[seq], q_len = sq_ql[seq];
      const int nt = (q_len + p.pf_tq - 1) / p.pf_tq;
      const int sz = co_pair_size(p, sq_kv[seq], q_len, nt, k);
      const int parts = co_tile_parts(sz, np);
      int psz = part < parts ? (sz * (part + 1)) / parts - (sz * part) / parts : -1;
      psz = psz < 0x7fff ? psz : 0x7fff;  // keys stay positive
      pkey[u] = psz < 0 ? -1 : (psz << 16) | u;
    }
    __syncthreads();
    const int n4 = (nunits + 3) / 4;
    if (wv == 0) {
      for (int i = nunits + lane; i < n4 * 4; i += 64) pkey[i] = -1;  // pad to whole int4s
      int cnt = 0;  // units with a key (empty parts have none)
      for (int i = lane; i < nunits; i += 64) cnt += pkey[i] >= 0;
      cnt = wave_sum32(cnt);
      if (lane == 0) *s_tile = cnt;
    }
    __syncthreads();
    nvalid = uni(*s_tile);
    // the ranks of the units with a key are 0 .. nvalid-1 (keys are distinct)
    for (int i = threadIdx.x; i < nunits; i += blockDim.x) {
      const int ki = pkey[i];
      if (ki < 0) continue;
      int r = 0;
      for (int k4 = 0; k4 < n4; ++k4) {
        const int4 v = ((const int4*)pkey)[k4];
        r += (v.x > ki) + (v.y > ki) + (v.z > ki) + (v.w > ki);
      }
      pord[r] = i;
    }
    __syncthreads();
  }
  const int total = (ranked ? nvalid : npairs) * p.Hkv;
  RPA_TL(tl_set(TL_RANKED, tl_clock());)
  // Tile t (queue order t = rank * Hkv + head) is queued on XCD t % 8, so with Hkv a multiple of 8
  // every token block of one (sequence, kv head) runs on one XCD and re-reads the causal prefix
  // its neighbours just fetched from that XCD's L2.  A workgroup takes tiles from its own XCD's
  // queue; once that is empty, wave 0 reads all eight counters at once (agent-scope loads) and
  // takes from the queue with the most tiles left, until none has any.
  //
  // sq >= 0 (every CU with one prefill-first and one stream-K workgroup): the first sn positions of
  // each XCD's queue are handed out statically -- the prefill-first workgroup of a CU takes position
  // k (its rank among its XCD's prefill-first workgroups, longest tiles first), the CU's stream-K
  // workgroup, joining later, position sn - 1 - k: each CU pairs a long first tile with a short
  // late one, and neither pays a queue round trip for it.  The counters then hand out positions
  // sn, sn + 1, ...
  const int x0 = (int)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & (kXcds - 1));  // XCC_ID
  bool own_left = true;  // wave 0's view of its own queue
  for (int first = 1;; first = 0) {
    RPA_TL(const long long tl_q = tl_clock();)
    if (wv == 0) {
      int t = total;
      if (first && sq >= 0) {
        const int ts = sq * kXcds + ((int)blockIdx.x & (kXcds - 1));  // the static position's tile
        t = ts < total ? ts : total;
      }
      if (sn * kXcds >= total) own_left = false;  // the fixed positions cover every queue
      if (t >= total && own_left) {
        int q = 0;
        if (lane == 0) q = atomicAdd(p.err + kQueueWord + x0, 1);
        q = uni(q) + sn;
        if (q < (total - x0 + kXcds - 1) / kXcds)
          t = q * kXcds + x0;
        else
          own_left = false;
      }
      while (t >= total && sn * kXcds < total) {
        const int x = (x0 + lane) & (kXcds - 1);
        int left = 0;
        if (lane < kXcds)
          left = (total - x + kXcds - 1) / kXcds - sn -
                 __hip_atomic_load(p.err + kQueueWord + x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int key = left > 0 ? (left << 3) | (kXcds - 1 - lane) : -1;  // most left, then nearest
        int best = -1;
#pragma unroll
        for (int i = 0; i < kXcds; ++i) best = max(best, rl(key, i));
        if (best < 0) break;  // every queue is empty
        const int bl = kXcds - 1 - (best & (kXcds - 1)), bx = (x0 + bl) & (kXcds - 1);
        int q = 0;
        if (lane == 0) q = atomicAdd(p.err + kQueueWord + bx, 1);
        q = uni(q) + sn;
        if (q < (total - bx + kXcds - 1) / kXcds) t = q * kXcds + bx;
      }
      if (lane == 0) *s_tile = t;
    }
    __syncthreads();
    const int tq = uni(*s_tile);
    __syncthreads();
    RPA_TL(ta.queue += tl_clock() - tl_q;)
    if (tq >= total) break;
    const int h = tq % p.Hkv;
    int pair = tq / p.Hkv, part = 0, unit_np = 1;
    if (ranked) {
      const int u = uni(pord[tq / p.Hkv]);
      pair = u / np;
      part = u - pair * np;
      unit_np = np;
    }
    PfTile tl = co_tile_of(p, wsi, cp, pair, h);
    if (tl.seq < 0 || tl.c_hi <= tl.c_lo) continue;
    int slot = -1;
    const int parts = co_tile_parts(tl.c_hi - tl.c_lo, unit_np);
    if (parts > 1) {
      const int sz = tl.c_hi - tl.c_lo, c0 = tl.c_lo;
      tl.c_lo = c0 + (sz * part) / parts;
      tl.c_hi = c0 + (sz * (part + 1)) / parts;
      const int st = pair * p.Hkv + h;  // split tile (npairs * Hkv <= co_split_max)
      slot = st * kCoMaxParts + part;
      if (part == 0 && threadIdx.x < 4) {  // its merge descriptor (read by the combine launch)
        CoDesc* d = p.co_desc + st;
        if (threadIdx.x == 0) {
          d->q_row0 = tl.q_start + tl.tok0;
          d->ntok = tl.ntok;
          d->h = h;
          d->nparts = parts;
          d->slot0 = st * kCoMaxParts;
        }
        d->valid[threadIdx.x] = 1;
      }
    }
    co_tile<MODE>(p, tl, cln, lds, wv, lane, n, j, err, slot, ta);
  }
  RPA_TL(tl_set(TL_NTILES, ta.tiles); tl_set(TL_NSTEPS, ta.steps); tl_set(TL_QUEUE, ta.queue);
         tl_set(TL_SETUP, ta.setup); tl_set(TL_LOOP, ta.loop); tl_set(TL_WRITE, ta.write);)
}

// CO: the co-resident layout's instantiation (p.co set), with the co-resident prefill role; the
// other instantiations carry the 8-wave prefill role (plain bf16 KV) or none, so the decode-only
// launches keep the registers of a kernel without the co-resident role.
// NW: a narrow head dim (p.D < kD; decode role only, every row through stream-K).  DN: a narrow
// head dim of 32 or 64 fixed at compile time, whose full-line loads read whole DN-element rows
// (Lines<DN>).
template <int MODE, bool UPG, bool CO = false, bool NW = false, int DN = 0>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void rpa_attn_kernel(Params p) {
  static_assert(DN == 0 || (NW && UPG && (DN == 32 || DN == 64)), "DN: a narrow instantiation of 32 or 64");
  constexpr bool kTiles = NW ? false : CO ? co_tiles<MODE>() : MODE == KV_BF16;  // a prefill-tile role exists
  const int D = DN ? DN : NW ? p.D : kD;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];  // HG x (V region, K tile)
  const int lane = threadIdx.x & 63;
  const int wv = uni(threadIdx.x >> 6);
  uint8_t* vt = smem + wv * kWaveLds;  // this wave's V region, then its K tile (full-line path)
  uint8_t* kt = vt + kVtBytes_;
  const int n = lane & 15, j = lane >> 4;
  const int b = blockIdx.x;
  int err = 0;
  RPA_TL(const long long tl_t0 = tl_clock(); tl_begin(); tl_set(TL_START, tl_t0);)

  // Schedule: total work W, this workgroup's range [u0, u1), the sequence holding u0 and a
  // window of per-lane sequence metadata.  num_seqs and the metadata of the first 256 sequences
  // (four 64-sequence windows) are fetched in one round trip; lanes past max_num_seqs load
  // nothing.  More sequences than that take one further round trip per window.
  constexpr int kWin = 4;
  Window win;
  SeqInfo wsi[kWin];
  int nseq, tv, pf_min;
  {
    int kv[kWin], c0[kWin], c1[kWin];
    // fused decode step: q rows 0..B-1 one per sequence, cu_kv in place of the second q bound
    constexpr bool fz = MODE == KV_BF16_FUSED;
    const int ns_raw = fz ? p.fused_nseq : p.num_seqs[0];
#pragma unroll
    for (int w = 0; w < kWin; ++w) {
      kv[w] = c0[w] = c1[w] = 0;
      const int i = 64 * w + lane;
      if (i < p.Nmax) {
        kv[w] = p.kv_lens[i];
        if (fz) {
          c0[w] = i;
          c1[w] = p.cu_kv[i];
        } else {
          c0[w] = p.cu_q_lens[i];
          c1[w] = p.cu_q_lens[i + 1];
        }
      }
    }
    nseq = uni(ns_raw);
    nseq = nseq < 0 ? 0 : (nseq > p.Nmax ? p.Nmax : nseq);
    // cu_q_lens[num_seqs]: rows from here on belong to no sequence
    tv = rl(c0[0], 0);
#pragma unroll
    for (int w = 0; w < kWin; ++w)
      if (nseq > 64 * w && nseq <= 64 * (w + 1)) tv = rl(c1[w], nseq - 1 - 64 * w);
    if (nseq > 64 * kWin) tv = fz ? 0 : uni(p.cu_q_lens[nseq]);
    if (fz) tv = nseq;
    // prefill tiles need the whole metadata in the four windows
    pf_min = (kTiles && p.pf_tq > 0 && nseq <= 64 * kWin) ? p.pf_min : 0;
#pragma unroll
    for (int w = 0; w < kWin; ++w) {
      wsi[w] = SeqInfo{0, 0, 0, 0};
      if (nseq > 64 * w) {  // windows past num_seqs hold no sequence (a uniform branch)
        if (fz)
          wsi[w] = make_fused_seq(p, kv[w], c1[w], c0[w], 64 * w + lane < nseq, err);
        else
          wsi[w] = make_seq(p, kv[w], c0[w], c1[w], 64 * w + lane < nseq, pf_min, err);
      }
    }
  }
  win.pf_min = pf_min;
  long long W = 0, tile[kWin];
  if (nseq <= 64 * kWin) {
#pragma unroll
    for (int w = 0; w < kWin; ++w) {
      tile[w] = nseq > 64 * w ? wave_sum_units((long long)wsi[w].units * p.NG) : 0;
      W += tile[w];
    }
  } else {
    W = total_units<MODE>(p, nseq, lane, err);
  }

  // Work split: the first gpre workgroups take prefill tiles, the rest run stream-K over the
  // other sequences.  Every workgroup computes the same split from the same metadata.
  int gpre = 0, pf_total = 0;
  bool any_pf = false;
#pragma unroll
  for (int w = 0; w < kWin; ++w) any_pf = any_pf || wsi[w].q_len >= pf_min;
  if (kTiles && pf_min > 0 && !p.pf_kernel && __ballot(any_pf) != 0) {
    // per lane over the four windows, then one wave sum each (skipped when no sequence is a
    // prefill sequence)
    float st = 0.f;
    int cnt = 0;
#pragma unroll
    for (int w = 0; w < kWin; ++w) {
      const int nt = pf_tiles_of(p, wsi[w], pf_min);
      const float prior = (float)(wsi[w].kv_len - wsi[w].q_len);
      // chunks of key positions the tiles visit (causal), summed over the sequence's tiles
      st += nt > 0 ? (float)p.Hkv * ((float)nt * prior + (float)p.pf_tq * 0.5f * (float)nt * (float)(nt + 1)) /
                         (float)KV_CHUNK
                   : 0.f;
      cnt += nt * p.Hkv;
    }
    float steps = 0.f;
    if (__ballot(cnt > 0) != 0) {
      steps = wave_sumf(st);
      pf_total = wave_sum32(cnt);
    }
    if (pf_total > 0) {
      const float pw = p.pf_cost * steps, dw = (float)W;
      gpre = (int)((float)p.grid * pw / (pw + dw) + 0.5f);
      gpre = gpre < 1 ? 1 : gpre;
      if (W > 0 && gpre > p.grid - 1) gpre = p.grid - 1;
      if (CO && gpre > p.grid / 2) gpre = p.grid / 2;  // at most one prefill workgroup per CU
      if (gpre > pf_total) gpre = pf_total;
    }
  }
  // Roles.  One workgroup per CU (8 waves): workgroups 0 .. gpre-1 take prefill tiles, the rest
  // run stream-K.  Co-resident layout (two 4-wave workgroups per CU, b and b + grid/2 on one CU):
  // workgroups grid/2 .. grid/2 + gpre - 1 take prefill tiles, so each sits beside a stream-K
  // workgroup, and every stream-K workgroup takes tiles too once its range is done.
  __shared__ int s_tile;
  bool pf_first;
  int bd;
  if constexpr (CO) {
    const int half = p.grid >> 1;
    pf_first = b >= half && b < half + gpre;
    bd = pf_first ? -1 : (b < half ? b : b - gpre);
  } else {
    pf_first = b < gpre;
    bd = b - gpre;
  }
  const int gd = p.grid - gpre;  // stream-K workgroup count
  RPA_TL(tl_set(TL_SCHED, tl_clock()); int tl_role = pf_first ? 1 : 0;)
  if (kTiles && pf_first) {
    if constexpr (CO)
      co_role<MODE>(p, wsi, pf_min, smem, &s_tile, lane, wv, n, j, err, gpre, pf_first);
    else if constexpr (MODE == KV_BF16)  // (HG == 8: one K and one V piece per thread per chunk)
      pf_role<1, UPG>(p, wsi, pf_min, pf_total, smem, &s_tile, lane, wv, n, j, err);
  }
  const Partition pt = make_partition_fast(W, gd > 0 ? gd : 1);
  const long long u0 = uni64(range_start(bd, pt)), u1 = uni64(range_start(bd + 1, pt));
  if (bd >= 0 && W > 0 && u0 < u1) {
    int seq;
    long long seq_start;
    if (nseq <= 64 * kWin) {
      // the window holding u0 (u0 < W, so one does), then the sequence inside it
      int wsel = -1;
      long long off = 0, off_sel = 0;
#pragma unroll
      for (int w = 0; w < kWin; ++w) {
        if (wsel < 0 && u0 < off + tile[w]) {
          wsel = w;
          off_sel = off;
        }
        off += tile[w];
      }
      if (wsel < 0) {  // not reached: u0 < W
        seq = nseq;
        seq_start = W;
      } else {
        win.base = 64 * wsel;
        win.s = wsi[0];
#pragma unroll
        for (int w = 1; w < kWin; ++w) select_seq(win.s, wsi[w], wsel == w);
        const long long cnt = (long long)win.s.units * p.NG;
        const long long incl = wave_incl_scan_units(cnt, lane);
        const int idx = __popcll(__ballot(off_sel + incl <= u0));
        seq = uni(win.base + idx);
        seq_start = uni64(off_sel + rl64(incl - cnt, idx));
      }
    } else {
      locate_seq<MODE>(p, nseq, lane, u0, seq, seq_start, err);
      load_window<MODE>(p, nseq, seq, lane, win, err);
    }
    if (seq < nseq) {
      Cursor cur = cursor_at<MODE>(p, win, seq, u0 - seq_start);
      Cursor nxt = cur;
      if (u0 + 1 < u1)
        advance<MODE>(p, nseq, lane, win, nxt, err);
      else
        nxt.nch = 0;
      const Pages pg_cur = load_pages<MODE, UPG>(p, cur, n);
      Pages pg_nxt = load_pages<MODE, UPG>(p, nxt, n);
      if constexpr (LinePath<MODE, UPG>::on) {
        LineRegs k, v;
        f32x4 bias[2];
        LineBias bias_in;
        bf16x8 q[4];
        uint32_t rst[2] = {0u, 0u};
        uint8_t* rs = smem + p.HG * kWaveLds + wv * kRelStage;  // relative-bias staging (fused step)
        // K, bias, queries, V: the loop's order (vmcnt retires in order, and the compiler
        // counts each wait for the least favourable path into it, this prologue included)
        {
          const LineAddr a0 = line_addr<MODE, UPG, DN>(p, cur, pg_cur, lane, n, j, wv, err, D);
          load_lines<MODE, UPG, DN>(p, a0, lane, 0, k, D);
          load_line_bias<MODE>(p, cur, a0, lane, n, j, wv, bias_in);
          load_q<MODE>(p, cur, n, j, wv, q, rst, MODE == KV_BF16_FUSED ? p.D : D);
          load_lines<MODE, UPG, DN>(p, a0, lane, 1, v, D);
        }
        RPA_TL(tl_set(TL_FIRST, tl_clock()); tl_set(TL_UNITS, u1 - u0); tl_role |= 2;)
        store_k_tile<MODE, DN>(p, k, kt, lane);
        line_bias_values<MODE>(p, cur, bias_in, rst, rs, lane, n, j, bias);
        RowState st;
        long long u = u0;
        for (;;) {
          step_line<MODE, UPG, DN>(p, nseq, lane, n, j, bd, u, u0, u1, win, cur, nxt, pg_nxt, k, v, bias, q, rst, st, vt,
                               kt, rs, err, pt, wv, D);
          if (++u >= u1) break;
        }
      } else {
        HalfRegs<MODE> ka, va, kb, vb;
        bf16x8 q[4];
        {  // K, queries, V: the loop's order (as above)
          const UnitAddr a0 = unit_addr(p, cur, pg_cur, n, j, wv, err, D);
          load_half<MODE, UPG>(p, a0, 0, ka, D);
          load_q<MODE>(p, cur, n, j, wv, q, nullptr, D);
          load_half<MODE, UPG>(p, a0, 1, va, D);
        }
        RPA_TL(tl_set(TL_FIRST, tl_clock()); tl_set(TL_UNITS, u1 - u0); tl_role |= 2;)
        RowState st;

        long long u = u0;
        for (;;) {
          step<MODE, UPG>(p, nseq, lane, n, j, bd, u, u0, u1, win, cur, nxt, pg_nxt, ka, va, kb, vb, q, st, vt, err, pt,
                          wv, D);
          if (++u >= u1) break;
          step<MODE, UPG>(p, nseq, lane, n, j, bd, u, u0, u1, win, cur, nxt, pg_nxt, kb, vb, ka, va, q, st, vt, err, pt,
                          wv, D);
          if (++u >= u1) break;
        }
      }
    }
  }
  RPA_TL(tl_set(TL_DEC, tl_clock());)
  if (CO && !pf_first && pf_total > 0) {
    __syncthreads();  // every wave is done with its stream-K LDS regions
    RPA_TL(tl_role |= 4;)
    co_role<MODE>(p, wsi, pf_min, smem, &s_tile, lane, wv, n, j, err, gpre, pf_first);
  }

  {  // rows at or past cu_q_lens[num_seqs] belong to no sequence: zero them
    tv = tv < 0 ? 0 : (tv > p.T ? p.T : tv);
    const size_t first = (size_t)tv * p.Hq * D / 8, last = (size_t)p.T * p.Hq * D / 8;
    u32x4* o = (u32x4*)p.out;
    for (size_t k = first + (size_t)b * blockDim.x + threadIdx.x; k < last; k += (size_t)p.grid * blockDim.x)
      o[k] = u32x4{0u, 0u, 0u, 0u};
  }
  RPA_TL(tl_set(TL_END, tl_clock()); tl_set(TL_ROLE, tl_role);)
  if (err) atomicOr(p.err, err);
}

// ---------------------------------------------------------------------------------------------
// prefill kernel: the MFMA-dense rows
// ---------------------------------------------------------------------------------------------
// Sequences with at least pf_min query tokens are cut into TILES: (sequence, kv head h, pf_tq =
// 256 / G consecutive tokens), 256 rows r = token * G + g (q head h*G + g).  A tile's work is its
// 64-key CHUNK STEPS over the keys its rows see (causal limit of its last row, sliding window of
// its first).  Chunk steps are ordered tile by tile (sequence, head, token block) and split evenly
// over the grid (the balanced partition of rpa_schedule.h, one workgroup per CU), so a long causal
// prefix is shared by several workgroups; a tile split across workgroups leaves one (m, l, acc)
// partial per workgroup, merged by rpa_combine_kernel.
//
// Workgroup = 4 waves, one per SIMD, wave w owning rows 64w .. 64w+63 as four 16-row MFMA blocks
// (the whole register file of a SIMD: 64 rows of fp32 accumulators, the queries and a chunk's
// scores stay in registers).  Per chunk the workgroup stages K and V (key rows, 272 and 288-byte
// strides; V read back transposed, read_vt_fragments) in one of two LDS buffers.  Every K and V^T fragment
// feeds the wave's four row blocks: 64 + 64 MFMAs per chunk per wave.  Loads run two chunk steps
// ahead (page ids three), stores of the next chunk follow the compute, one barrier per step.
constexpr int kPkRows = 256;
constexpr int kPkChunk = 64;
constexpr int kPkKRow = kD * 2 + 16;            // 272 B per K row
constexpr int kPkKTile = kPkChunk * kPkKRow;    // 17408 B
constexpr int kPkVtTile = kPkChunk * kVRow;     // 18432 B: V as key rows (read_vt_fragments per 32 keys)
constexpr int kPkStage = kPkKTile + kPkVtTile;  // 35840 B
constexpr int kPkLds = 2 * kPkStage;

struct PkTile {
  int seq, h, t, nt;       // sequence, kv head, token block, token blocks of the sequence
  int kv_len, q_len, q_start;
  int tok0, ntok;          // first token (sequence-relative) and tokens of the tile
  int c_lo, c_hi;          // chunks visited
};

// Chunk range of token block t (0 units when its rows see no key).
__device__ __forceinline__ void pk_range(const Params& p, PkTile& tl) {
  tl.tok0 = tl.t * p.pf_tq;
  tl.ntok = tl.q_len - tl.tok0 < p.pf_tq ? tl.q_len - tl.tok0 : p.pf_tq;
  const int prior = tl.kv_len - tl.q_len;
  int hi = prior + tl.tok0 + tl.ntok - 1;  // last key any row of the tile sees
  hi = hi < tl.kv_len - 1 ? hi : tl.kv_len - 1;
  int lo = 0;
  if (p.sliding_window > 0) {  // keys below are masked for every row of the tile
    lo = prior + tl.tok0 - p.sliding_window + 1;
    lo = lo < 0 ? 0 : lo;
  }
  tl.c_lo = lo / kPkChunk;
  tl.c_hi = hi >= lo ? hi / kPkChunk + 1 : tl.c_lo;
}

// Chunk steps of one kv head of a sequence (a prefill sequence: q_len >= pf_min).
__device__ __forceinline__ int pk_units_per_head(const Params& p, int kv_len, int q_len) {
  if (q_len < p.pf_min || kv_len <= 0) return 0;
  PkTile tl;
  tl.kv_len = kv_len;
  tl.q_len = q_len;
  const int nt = (q_len + p.pf_tq - 1) / p.pf_tq;
  int u = 0;
  for (int t = 0; t < nt; ++t) {
    tl.t = t;
    pk_range(p, tl);
    u += tl.c_hi - tl.c_lo;
  }
  return u;
}

// A sequence's metadata out of the four per-lane windows (s wave-uniform, < 256).
__device__ __forceinline__ void pk_seq(const SeqInfo wsi[4], const int units[4], int s, PkTile& tl, int& u) {
  const int w = s >> 6, k = s & 63;
  int kv = 0, ql = 0, qs = 0, un = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {  // value selects keep the windows in registers
    kv = w == i ? wsi[i].kv_len : kv;
    ql = w == i ? wsi[i].q_len : ql;
    qs = w == i ? wsi[i].q_start : qs;
    un = w == i ? units[i] : un;
  }
  tl.seq = s;
  tl.kv_len = rl(kv, k);
  tl.q_len = rl(ql, k);
  tl.q_start = rl(qs, k);
  u = rl(un, k);
}

struct PkCur {
  PkTile tl;
  int c;      // chunk
  int units;  // chunk steps per kv head of tl.seq
  bool live;  // false past the workgroup's range
};

// The next chunk step (tile by tile: token block, then kv head, then sequence).
__device__ __forceinline__ void pk_advance(const Params& p, const SeqInfo wsi[4], const int units[4], int nseq,
                                           PkCur& x) {
  if (!x.live) return;
  if (x.c + 1 < x.tl.c_hi) {
    x.c++;
    return;
  }
  for (;;) {
    if (x.tl.t + 1 < x.tl.nt) {
      x.tl.t++;
    } else if (x.tl.h + 1 < p.Hkv) {
      x.tl.h++;
      x.tl.t = 0;
    } else {
      int s = x.tl.seq;
      int un = 0;
      do {
        if (++s >= nseq) {
          x.live = false;
          return;
        }
        pk_seq(wsi, units, s, x.tl, un);
      } while (un == 0);
      x.units = un;
      x.tl.nt = (x.tl.q_len + p.pf_tq - 1) / p.pf_tq;
      x.tl.h = 0;
      x.tl.t = 0;
    }
    pk_range(p, x.tl);
    if (x.tl.c_hi > x.tl.c_lo) {
      x.c = x.tl.c_lo;
      return;
    }
  }
}

// The chunk steps' K and V pieces of one thread (4 + 4 x 16 bytes).
struct PkRegs {
  u32x4 k[4], v[4];
};

// Issue the loads of chunk step x (page id pg, read a step earlier).  K and V piece i: key
// (tid / 16) + 16 i, dims 8 (tid % 16) .. (whole 128-byte lines, non-temporal).  Keys past kv_len
// read key kv_len - 1 (masked by their scores).  The chunk's base address is wave-uniform; each
// piece is a 32-bit byte offset from it.
__device__ __forceinline__ void pk_load(const Params& p, const PkCur& x, int pg, int tid, PkRegs& r, int& err) {
  pg = uni(pg);
  if (pg < 0 || pg >= p.P) {  // out-of-range page id: never dereferenced
    if (x.live) err |= ERR_PAGE;
    pg = 0;
  }
  const int key0 = x.live ? x.c * kPkChunk : 0;
  const int kmax = x.live ? x.tl.kv_len - 1 - key0 : 0;
  const uint8_t* base = p.kv + 2 * kv_elem(p, pg, key0, 2 * (x.live ? x.tl.h : 0));
  const uint32_t row = (uint32_t)(2 * p.Hkv) * kD * 2;  // bytes between consecutive keys of a page
  const uint32_t kcol = 16u * (tid & 15);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int kk = (tid >> 4) + 16 * i;
    kk = kk < kmax ? kk : kmax;
    r.k[i] = ld_stream((const u32x4*)(base + ((uint32_t)kk * row + kcol)));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    int kk = (tid >> 4) + 16 * i;
    kk = kk < kmax ? kk : kmax;
    r.v[i] = ld_stream((const u32x4*)(base + ((uint32_t)kk * row + 2u * kD + kcol)));
  }
}

__device__ __forceinline__ int pk_page_id(const Params& p, const PkCur& x) {
  const size_t idx = x.live ? (size_t)x.tl.seq * p.PPS + page_of(x.c * kPkChunk, p) : 0;
  return p.page_indices[idx + opaque_zero()];
}

__device__ __forceinline__ void pk_store(uint8_t* stage, const PkRegs& r, int tid) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
    *(u32x4*)(stage + ((tid >> 4) + 16 * i) * kPkKRow + 16 * (tid & 15)) = r.k[i];
  uint8_t* vt = stage + kPkKTile;
#pragma unroll
  for (int i = 0; i < 4; ++i) *(u32x4*)(vt + ((tid >> 4) + 16 * i) * kVRow + 16 * (tid & 15)) = r.v[i];
}

struct PkRow {
  f32x4 acc[8];  // O^T: dims 16 db + 4 j + r, row n
  float m, l;
  int pos;       // last visible key of this lane's row
  bool ok;       // the row exists
};

// One 16-row block's softmax over 32 keys k0 ..: scores sc[kb] (keys k0 + 16 kb + 4 j + r of row n)
// -> P^T for the PV step (k-slots in the tau order of the scores).
__device__ __forceinline__ bf16x8 pk_softmax(const Params& p, const PkTile& tl, int k0, bool plain, const f32x4 sc[2],
                                             PkRow& st, int j) {
  float xs[2][4];
  if (plain) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) xs[kb][r] = sc[kb][r] * p.scale_log2;
  } else {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float sv = sc[kb][r];
        float xv;
        if (p.soft_cap > 0.f) {
          const float t = sv * p.sm_scale;
          xv = p.soft_cap * tanhf(t / p.soft_cap) * kLog2e;
        } else {
          xv = sv * p.scale_log2;
        }
        const int kt = k0 + 4 * j + 16 * kb + r;
        const bool masked = kt > st.pos || (p.sliding_window > 0 && kt <= st.pos - p.sliding_window);
        if (masked) xv += p.mask_log2;
        if (kt >= tl.kv_len) xv = -INFINITY;
        xs[kb][r] = xv;
      }
  }
  float mc = fmaxf(fmaxf(fmaxf(xs[0][0], xs[0][1]), fmaxf(xs[0][2], xs[0][3])),
                   fmaxf(fmaxf(xs[1][0], xs[1][1]), fmaxf(xs[1][2], xs[1][3])));
  mc = rows4_max(mc);
  const bool grow = mc > st.m + kRescaleLog2;
  if (__ballot(grow)) {
    const float mn = grow ? mc : st.m;
    const float alpha = __builtin_amdgcn_exp2f(st.m - (mn == -INFINITY ? 0.f : mn));
    st.l *= alpha;
#pragma unroll
    for (int d = 0; d < 8; ++d) st.acc[d] *= alpha;
    st.m = mn;
  }
  const float mu = st.m == -INFINITY ? 0.f : st.m;
  float pr[2][4];
  float lsum = 0.f;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      pr[kb][r] = __builtin_amdgcn_exp2f(xs[kb][r] - mu);
      lsum += pr[kb][r];
    }
  st.l += lsum;
  u32x4 pw;
  pw[0] = pack_bf16x2(pr[0][0], pr[0][1]);
  pw[1] = pack_bf16x2(pr[0][2], pr[0][3]);
  pw[2] = pack_bf16x2(pr[1][0], pr[1][1]);
  pw[3] = pack_bf16x2(pr[1][2], pr[1][3]);
  return __builtin_bit_cast(bf16x8, pw);
}

// Row r = 64 wv + 16 rb + n of tile tl: its token (tile-relative) and whether it exists.
__device__ __forceinline__ bool pk_row(const Params& p, const PkTile& tl, int r, int& tok, int& g, int& pos) {
  tok = r / p.G;
  g = r - tok * p.G;
  pos = tl.kv_len - tl.q_len + tl.tok0 + tok;
  return tok < tl.ntok && pos >= 0;
}

// Queries of the wave's four row blocks for tile tl (rows past the tile read its first row).
__device__ __forceinline__ void pk_load_q(const Params& p, const PkTile& tl, int wv, int n, int j, bf16x8 q[4][4]) {
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    int tok, g, pos;
    const bool ok = pk_row(p, tl, 64 * wv + 16 * rb + n, tok, g, pos);
    const int qtok = ok ? tl.q_start + tl.tok0 + tok : tl.q_start;
    const uint16_t* qp = p.q + ((size_t)qtok * p.Hq + tl.h * p.G + (ok ? g : 0)) * kD + 8 * j;
#pragma unroll
    for (int s = 0; s < 4; ++s) q[rb][s] = __builtin_bit_cast(bf16x8, *(const u32x4*)(qp + 32 * s));
  }
}

// Row states at the start of tile tl.
__device__ __forceinline__ void pk_begin(const Params& p, const PkTile& tl, PkRow st[4], int wv, int n) {
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    int tok, g, pos;
    st[rb].ok = pk_row(p, tl, 64 * wv + 16 * rb + n, tok, g, pos);
    st[rb].pos = pos;
#pragma unroll
    for (int d = 0; d < 8; ++d) st[rb].acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    st[rb].m = -INFINITY;
    st[rb].l = 0.f;
  }
}

// One chunk step from LDS stage `stage` for the wave's four row blocks, as two 32-key halves (QK^T,
// softmax, PV each); when the next chunk step starts a new tile (next_q), its queries are loaded
// into q once the last QK^T products have read them.
__device__ __forceinline__ void pk_compute(const Params& p, const PkTile& tl, int c, const uint8_t* stage,
                                           bf16x8 q[4][4], PkRow st[4], int wv, int n, int j, bool next_q,
                                           const PkTile& ntl) {
  const uint8_t* vt = stage + kPkKTile;
  const int pos_min = tl.kv_len - tl.q_len + tl.tok0 + (64 * wv) / p.G;
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    f32x4 sc[4][2];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) sc[rb][0] = sc[rb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    bf16x8 ka[4][2];  // the half's K fragments, all read before its MFMAs
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
        ka[s][kb] = *(const bf16x8*)(stage + (32 * hf + 16 * kb + n) * kPkKRow + (32 * s + 8 * j) * 2);
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) sc[rb][kb] = mfma(ka[s][kb], q[rb][s], sc[rb][kb]);
    if (hf == 1 && next_q) pk_load_q(p, ntl, wv, n, j, q);
    const int k0 = c * kPkChunk + 32 * hf;
    const bool plain = !(p.soft_cap > 0.f) && p.sliding_window <= 0 && k0 + 31 <= pos_min && k0 + 32 <= tl.kv_len;
    bf16x8 pb[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) pb[rb] = pk_softmax(p, tl, k0, plain, sc[rb], st[rb], j);
    bf16x8 va[8];  // the half's V^T fragments
    read_vt_fragments(vt + 32 * hf * kVRow, n, j, va);
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) st[rb].acc[db] = mfma(va[db], pb[rb], st[rb].acc[db]);
  }
}

// The tile's rows of this workgroup: written out (complete) or left as a partial (split).
__device__ __forceinline__ void pk_finish(const Params& p, const PkTile& tl, PkRow st[4], bool complete, int b,
                                          bool started_here, int wv, int n, int j) {
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const float lt = rows4_sum(st[rb].l);
    const int r = 64 * wv + 16 * rb + n;
    if (complete) {
      if (!st[rb].ok) continue;
      const int tok = r / p.G, g = r - tok * p.G;
      const float inv = 1.f / lt;
      uint16_t* op = p.out + ((size_t)(tl.q_start + tl.tok0 + tok) * p.Hq + tl.h * p.G + g) * kD + 4 * j;
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        u32x2 w2;
        w2[0] = pack_bf16x2(st[rb].acc[d][0] * inv, st[rb].acc[d][1] * inv);
        w2[1] = pack_bf16x2(st[rb].acc[d][2] * inv, st[rb].acc[d][3] * inv);
        *(u32x2*)(op + 16 * d) = w2;
      }
    } else {
      const size_t slot = (size_t)partial_slot(b, started_here);
      float* ap = p.pk_acc + (slot * kPkRows + r) * kD + 4 * j;
#pragma unroll
      for (int d = 0; d < 8; ++d) *(f32x4*)(ap + 16 * d) = st[rb].acc[d];
      if (j == 0) {
        float* mp = p.pk_ml + (slot * kPkRows + r) * 2;
        mp[0] = st[rb].m;
        mp[1] = lt;
      }
    }
  }
}

// Workgroup b describes the split tile whose last chunk step u it owns (thread 0).
__device__ __forceinline__ void pk_describe(const Params& p, const PkTile& tl, long long first_unit, const Partition& pt,
                                            int b) {
  PkDesc* d = p.pk_desc + b;
  d->q_start = tl.q_start + tl.tok0;
  d->ntok = tl.ntok;
  d->h = tl.h;
  d->b0 = owner_of(first_unit, pt);
#pragma unroll
  for (int g = 0; g < 16; ++g) d->valid[g] = 1;
}

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void rpa_prefill_kernel(Params p) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63, wv = uni(tid >> 6);
  const int n = lane & 15, j = lane >> 4;
  const int b = blockIdx.x;
  int err = 0;

  // metadata of the first 256 sequences in one round trip (the attention kernel leaves prefill
  // sequences to this kernel only when num_seqs <= 256)
  constexpr int kWin = 4;
  SeqInfo wsi[kWin];
  int units[kWin];
  const int ns_raw = p.num_seqs[0];
  int kvv[kWin], c0[kWin], c1[kWin];
#pragma unroll
  for (int w = 0; w < kWin; ++w) {
    kvv[w] = c0[w] = c1[w] = 0;
    const int i = 64 * w + lane;
    if (i < p.Nmax) {
      kvv[w] = p.kv_lens[i];
      c0[w] = p.cu_q_lens[i];
      c1[w] = p.cu_q_lens[i + 1];
    }
  }
  int nseq = uni(ns_raw);
  nseq = nseq < 0 ? 0 : (nseq > p.Nmax ? p.Nmax : nseq);
  if (nseq > 64 * kWin) return;
  long long W = 0, tile_units[kWin];
#pragma unroll
  for (int w = 0; w < kWin; ++w) {
    wsi[w] = SeqInfo{0, 0, 0, 0};
    units[w] = 0;
    if (nseq > 64 * w) {
      wsi[w] = make_seq(p, kvv[w], c0[w], c1[w], 64 * w + lane < nseq, 0, err);
      units[w] = pk_units_per_head(p, wsi[w].kv_len, wsi[w].q_len);
    }
    tile_units[w] = nseq > 64 * w ? (long long)wave_sum32(units[w] * p.Hkv) : 0;
    W += tile_units[w];
  }
  const Partition pt = make_partition_fast(W, p.pk_grid);
  const long long u0 = uni64(range_start(b, pt)), u1 = uni64(range_start(b + 1, pt));
  if (W == 0 || u0 >= u1) return;

  // the chunk step u0: its sequence (window scan), kv head, token block
  PkCur cur;
  {
    long long off = 0;
    int s = -1;
    long long s_start = 0;
#pragma unroll
    for (int w = 0; w < kWin; ++w) {
      if (s < 0 && u0 < off + tile_units[w]) {
        const int cnt = units[w] * p.Hkv;
        const int incl = wave_incl_scan32(cnt, lane);
        const int idx = __popcll(__ballot(off + incl <= u0));
        s = 64 * w + idx;
        s_start = off + rl(incl - cnt, idx);
      }
      off += tile_units[w];
    }
    int un = 0;
    pk_seq(wsi, units, s, cur.tl, un);
    cur.units = un;
    cur.live = true;
    const int ul = (int)(u0 - s_start);
    cur.tl.h = ul / un;
    int rem = ul - cur.tl.h * un;
    cur.tl.nt = (cur.tl.q_len + p.pf_tq - 1) / p.pf_tq;
    cur.tl.t = 0;
    for (;;) {
      pk_range(p, cur.tl);
      const int cnt = cur.tl.c_hi - cur.tl.c_lo;
      if (rem < cnt) {
        cur.c = cur.tl.c_lo + rem;
        break;
      }
      rem -= cnt;
      cur.tl.t++;
    }
  }
  // first unit of cur's tile (for its split descriptor)
  long long tile_first = u0 - (cur.c - cur.tl.c_lo);

  auto ahead = [&](const PkCur& x, long long ux) {  // the cursor of chunk step ux + 1
    PkCur y = x;
    if (ux + 1 < u1)
      pk_advance(p, wsi, units, nseq, y);
    else
      y.live = false;
    return y;
  };
  // Pipeline invariant at the start of step u: LDS stage u & 1 holds chunk step u and pg_n1 is the
  // page id of step u+1.  Step u loads the page id of u+2 and the data of u+1 (into registers),
  // computes u, finishes u's tile if it ends there, stores u+1 to the other stage, barrier.
  PkCur n1 = ahead(cur, u0);
  int pg_n1;
  PkRegs r;
  {
    const int pg_cur = pk_page_id(p, cur);
    pg_n1 = pk_page_id(p, n1);
    pk_load(p, cur, pg_cur, tid, r, err);
  }
  bf16x8 q[4][4];
  PkRow st[4];
  pk_load_q(p, cur.tl, wv, n, j, q);
  pk_begin(p, cur.tl, st, wv, n);
  bool started_here = cur.c == cur.tl.c_lo;
  pk_store(smem + (u0 & 1) * kPkStage, r, tid);
  __syncthreads();

  for (long long u = u0;; ++u) {
    const PkCur n2 = ahead(n1, u + 1);
    const int pg_n2 = pk_page_id(p, n2);
    pk_load(p, n1, pg_n1, tid, r, err);
    const bool tile_end = cur.c + 1 >= cur.tl.c_hi;
    const bool range_end = u + 1 >= u1;
    pk_compute(p, cur.tl, cur.c, smem + (u & 1) * kPkStage, q, st, wv, n, j, tile_end && !range_end, n1.tl);
    if (tile_end || range_end) {
      const bool complete = started_here && tile_end;
      pk_finish(p, cur.tl, st, complete, b, started_here, wv, n, j);
      if (!complete && !started_here && tile_end && tid == 0) pk_describe(p, cur.tl, tile_first, pt, b);
      if (range_end) break;
      pk_begin(p, n1.tl, st, wv, n);  // the next tile starts here (its queries are loading)
      started_here = true;
      tile_first = u + 1;
    }
    pk_store(smem + ((u + 1) & 1) * kPkStage, r, tid);
    __syncthreads();
    cur = n1;
    n1 = n2;
    pg_n1 = pg_n2;
  }
  if (err) atomicOr(p.err, err);
}

// ---------------------------------------------------------------------------------------------
// split-K combine
// ---------------------------------------------------------------------------------------------
// Partial of contributor k (0-based) of descriptor d for head hw: (m, l) pairs [16 rows][2] and
// acc [16 rows][kD], row-major.
__device__ __forceinline__ size_t combine_slot(const Params& p, const SplitDesc& d, int hw, int k) {
  return (size_t)partial_slot(d.b0 + k, k == 0) * p.HG + hw;
}

// One-pass merge of a split row block's partials by a workgroup of CW waves.  A lane holds NP row
// slots: row RS*i + lane/(64/RS) of the block, dims dim0 + 4*(lane % (64/RS)) .. +3 (RS = 2: two
// whole 512-byte rows per load instruction; RS = 8: a 32-dim slice of eight rows).  Wave wv takes
// contributors wv, wv+CW, ..., U at a time with all their (m, l, acc) loads issued before any is
// used (sched_barrier), and folds each into a running (m, l, o) with the online log-sum-exp update
// -- in contributor order, so the result is deterministic.
template <int NP>
struct MergeAcc {
  f32x4 o[NP];
  float m[NP], l[NP];
};

template <int CW, int NP, int U, int RS>
__device__ __forceinline__ void merge_rows(const Params& p, const SplitDesc& d, int hw, int ncontrib, int wv, int lane,
                                           int row0, int dim0, MergeAcc<NP>& a) {
  constexpr int kLanesPerRow = 64 / RS;
  const int r0 = row0 + lane / kLanesPerRow, c4 = dim0 + 4 * (lane % kLanesPerRow);
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    a.o[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    a.m[i] = -INFINITY;
    a.l[i] = 0.f;
  }
#pragma unroll 1
  for (int k = wv; k < ncontrib; k += CW * U) {
    f32x4 x[U][NP];
    float mc[U][NP], lc[U][NP];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int kk = k + CW * u < ncontrib ? k + CW * u : k;  // past the end: a valid slot, skipped below
      const size_t sc = combine_slot(p, d, hw, kk);
      const float* ml = p.part_ml + sc * ROW_BLOCK * 2;
      const float* acc = p.part_acc + sc * ROW_BLOCK * kD + c4;
#pragma unroll
      for (int i = 0; i < NP; ++i) {
        const int row = RS * i + r0;
        mc[u][i] = ml[2 * row];
        lc[u][i] = ml[2 * row + 1];
        x[u][i] = *(const f32x4*)(acc + row * kD);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (k + CW * u < ncontrib)
#pragma unroll
        for (int i = 0; i < NP; ++i) {
          const float mn = fmaxf(a.m[i], mc[u][i]), mu = mn == -INFINITY ? 0.f : mn;
          const float sa = __builtin_amdgcn_exp2f(a.m[i] - mu), sb = __builtin_amdgcn_exp2f(mc[u][i] - mu);
          a.o[i] = a.o[i] * sa + x[u][i] * sb;
          a.l[i] = a.l[i] * sa + lc[u][i] * sb;
          a.m[i] = mn;
        }
  }
}

// The CW waves' running states merged through LDS (waves 1..CW-1 into wave 0, in that order),
// divided by the denominator and written as bf16: rows below nrows of descriptor d, head hw.
// red / redml rows hold a lane's 4 NP (<= 16) o values and 2 NP (m, l) values, at odd strides.
template <int CW, int NP, int RS>
__device__ __forceinline__ void merge_waves_store(const Params& p, const SplitDesc& d, int hw, int nrows, int wv,
                                                  int lane, int row0, int dim0, const MergeAcc<NP>& a,
                                                  float (*red)[64][17], float (*redml)[64][9]) {
  constexpr int kLanesPerRow = 64 / RS;
  if (wv > 0) {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) red[wv - 1][lane][4 * i + e] = a.o[i][e];
      redml[wv - 1][lane][2 * i] = a.m[i];
      redml[wv - 1][lane][2 * i + 1] = a.l[i];
    }
  }
  __syncthreads();
  if (wv == 0) {
    const int r0 = row0 + lane / kLanesPerRow, c4 = dim0 + 4 * (lane % kLanesPerRow);
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const int row = RS * i + r0;
      if (row >= nrows) continue;
      float M = a.m[i];
      for (int w = 0; w < CW - 1; ++w) M = fmaxf(M, redml[w][lane][2 * i]);
      const float mu = M == -INFINITY ? 0.f : M;
      float sw = __builtin_amdgcn_exp2f(a.m[i] - mu);
      f32x4 v = a.o[i] * sw;
      float L = a.l[i] * sw;
      for (int w = 0; w < CW - 1; ++w) {
        sw = __builtin_amdgcn_exp2f(redml[w][lane][2 * i] - mu);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += red[w][lane][4 * i + e] * sw;
        L += redml[w][lane][2 * i + 1] * sw;
      }
      const float inv = 1.f / L;
      const int grow = d.rb * ROW_BLOCK + row;  // row of the sequence's (token, head) rows
      const int tok = grow / p.G;
      const int vh = d.h * p.HG + hw;  // virtual head (finish_row_block)
      const int head = real_head(vh, p.D) * p.G + (grow - tok * p.G);
      // a partial's row n holds O^T column n: dim d at index d (see finish_row_block)
      u32x2 w2;
      w2[0] = pack_bf16x2(v[0] * inv, v[1] * inv);
      w2[1] = pack_bf16x2(v[2] * inv, v[3] * inv);
      if (c4 < p.D)  // dims < D
        *(u32x2*)(p.out + ((size_t)(d.q_start + tok) * p.Hq + head) * p.D + half_offset(vh, p.D) + c4) = w2;
    }
  }
  __syncthreads();  // red / redml free for a next merge
}

__device__ __forceinline__ int rows_of(const Params& p, const SplitDesc& d) {
  const int nrows = d.q_len * p.G - d.rb * ROW_BLOCK;
  return nrows < ROW_BLOCK ? nrows : ROW_BLOCK;
}

// Helper workgroup hb (the first workgroups of the launch): heavy slot hb / (HG * kHeavySlices),
// head and dim slice from the rest.  Its flag (set by the attention kernel) says whether the slot
// holds a heavy descriptor this call; the flag and the slot's copy of the descriptor come in one
// round trip.  The workgroup merges those 32 dims of the block's rows and clears its flag.
template <int CW>
__device__ __forceinline__ void combine_heavy(const Params& p, int hb, float (*red)[64][17], float (*redml)[64][9]) {
  const int slot = hb / (p.HG * kHeavySlices), rem = hb - slot * (p.HG * kHeavySlices);
  const int hw = rem / kHeavySlices, slice = rem - hw * kHeavySlices;
  int32_t* flag = p.heavy + ((size_t)slot * 8 + hw) * kHeavySlices + slice;
  int f = *flag;
  SplitDesc d = p.heavy_desc[slot];
  asm volatile("" : "+v"(f), "+v"(d.q_start), "+v"(d.q_len), "+v"(d.h), "+v"(d.rb), "+v"(d.b0));
  f = __builtin_amdgcn_readfirstlane(f);
  if (f <= 0 || f > p.grid) return;
  const int b = f - 1;
  const int t = threadIdx.x, wv = t >> 6, lane = t & 63;
  const int ncontrib = (int)(b - d.b0 + 1), nrows = rows_of(p, d);
  if (nrows <= 8) {
    MergeAcc<1> a;
    // two waves keep 32 contributors in flight as four do, each taking twice as many
    merge_rows<CW, 1, CW == 2 ? 16 : 8, 8>(p, d, hw, ncontrib, wv, lane, 0, 32 * slice, a);
    merge_waves_store<CW, 1, 8>(p, d, hw, nrows, wv, lane, 0, 32 * slice, a, red, redml);
  } else {
    MergeAcc<2> a;
    merge_rows<CW, 2, 4, 8>(p, d, hw, ncontrib, wv, lane, 0, 32 * slice, a);
    merge_waves_store<CW, 2, 8>(p, d, hw, nrows, wv, lane, 0, 32 * slice, a, red, redml);
  }
  if (t == 0) *flag = 0;
}

// Prefill merge workgroup idx: split tile pk_desc[b] (b = pk_grid - 1 - idx / 16), rows
// 16 g .. 16 g + 15 (g = idx % 16).  The tile's partials [slot][256][kD] are sixteen 16-row
// blocks, so the decode merge reads them as slots of 16 rows (slot * 16 + g); its rows map to
// (token, q head) as the tile's rows do: row 16 g + i -> token tok0 + (16 g + i) / G, head
// h G + (16 g + i) % G.
template <int CW>
__device__ __forceinline__ void combine_prefill(const Params& p, int idx, float (*red)[64][17], float (*redml)[64][9]) {
  const int b = p.pk_grid - 1 - idx / 16, g = idx % 16;
  int valid = p.pk_desc[b].valid[g];
  PkDesc pd = p.pk_desc[b];
  asm volatile("" : "+v"(valid), "+v"(pd.q_start), "+v"(pd.ntok), "+v"(pd.h), "+v"(pd.b0));
  if (!__builtin_amdgcn_readfirstlane(valid)) return;
  const int t = threadIdx.x, wv = t >> 6, lane = t & 63;
  SplitDesc d;
  d.q_start = pd.q_start;
  d.q_len = pd.ntok;
  d.h = pd.h;
  d.rb = g;
  d.b0 = pd.b0;
  Params pm = p;  // partial slots of 16 rows: slot * 16 + g
  pm.part_acc = p.pk_acc;
  pm.part_ml = p.pk_ml;
  pm.HG = 16;
  Params ps = p;  // output rows: head h * G + row % G
  ps.HG = 1;
  const int ncontrib = (int)(b - d.b0 + 1), nrows = rows_of(p, d);
  if (nrows > 0 && nrows <= 4) {
    MergeAcc<2> a;
    merge_rows<CW, 2, 4, 2>(pm, d, g, ncontrib, wv, lane, 0, 0, a);
    merge_waves_store<CW, 2, 2>(ps, d, 0, nrows, wv, lane, 0, 0, a, red, redml);
  } else if (nrows > 0) {
#pragma unroll 1
    for (int row0 = 0; row0 < nrows; row0 += 8) {
      MergeAcc<4> a;
      merge_rows<CW, 4, 1, 2>(pm, d, g, ncontrib, wv, lane, row0, 0, a);
      merge_waves_store<CW, 4, 2>(ps, d, 0, nrows, wv, lane, row0, 0, a, red, redml);
    }
  }
  if (t == 0) p.pk_desc[b].valid[g] = 0;
}

// Workgroup b merges the row block described by desc[b] for head hw: contributors b0..b, b0's
// share in slot 2*b0+1 and every later one's in slot 2*bb (merge_rows, merge_waves_store), unless
// the block is heavy (its slot's helper workgroups merge it).  The heavy-merge helpers come
// first in the launch, then the (descriptor, head) workgroups, then (with the prefill kernel) 16
// per prefill workgroup for its split tiles.
// Fused decode step: block s stores sequence s's new token (key kv_len-1, K of kv head h at combined
// row 2h, V at 2h+1) into the cache, at slot (kv_len-1) % S of page page_indices[cu_kv[s] / S +
// (kv_len-1) / S] (src/tpu_cake/workloads/inkling_rpa.py:518-534).  The attention kernel read
// that key from new_k / new_v, so the store may follow it.  Anything out of range is skipped and
// flagged.
__device__ __forceinline__ void fused_store_token(const Params& p, int s) {
  if (s >= p.fused_nseq) return;
  const int len = p.kv_lens[s], cu = p.cu_kv[s];
  const int pos = len - 1;
  const long long entry = (long long)(cu >= 0 ? cu / p.S : 0) + (pos >= 0 ? pos / p.S : 0);
  bool ok = len >= 1 && (long long)len <= (long long)p.PPS * p.S && cu >= 0 && cu % p.S == 0 &&
            entry < p.fused_entries;
  const int page = ok ? p.page_indices[entry] : 0;
  ok = ok && page >= 0 && page < p.P;
  if (!ok) {
    if (threadIdx.x == 0) atomicOr(p.err, ERR_PAGE);
    return;
  }
  uint16_t* rows = (uint16_t*)p.kv + ((size_t)page * p.S + pos % p.S) * (size_t)(2 * p.Hkv) * kD;
  const int n = 2 * p.Hkv * kD;
  for (int i = 8 * threadIdx.x; i < n; i += 8 * blockDim.x) {  // new rows of p.D elements, zeros past them
    const int r = i / kD, d = i - r * kD;
    const uint16_t* src = ((r & 1) ? p.new_v : p.new_k) + ((size_t)s * p.Hkv + (r >> 1)) * p.D + d;
    *(u32x4*)(rows + i) = d < p.D ? *(const u32x4*)src : u32x4{0u, 0u, 0u, 0u};
  }
}

// Co-resident split tile merge: workgroup idx merges rows 32 g .. 32 g + 31 (g = idx % 4) of split
// tile idx / 4 from its nparts partial slots: thread t takes rows 32 g + t / 8 (+ blockDim / 8 ...),
// dims 16 (t % 8) .. +15, folds the parts in order with the online log-sum-exp update and writes
// bf16.
__device__ __forceinline__ void combine_co_split(const Params& p, int idx) {
  const int st = idx >> 2, g = idx & 3;
  if (st >= p.co_split_max) return;
  CoDesc* dp = p.co_desc + st;
  int valid = dp->valid[g];
  CoDesc d = *dp;
  asm volatile("" : "+v"(valid), "+v"(d.q_row0), "+v"(d.ntok), "+v"(d.h), "+v"(d.nparts), "+v"(d.slot0));
  if (!__builtin_amdgcn_readfirstlane(valid)) return;
  const int t = threadIdx.x, c16 = 16 * (t & 7);
  const int nparts = __builtin_amdgcn_readfirstlane(d.nparts);
#pragma unroll 1
  for (int row = 32 * g + (t >> 3); row < 32 * g + 32; row += (int)(blockDim.x >> 3)) {
    if (row >= d.ntok * p.G) break;
    f32x4 o[4];
    float m = -INFINITY, l = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < nparts && k < kCoMaxParts; ++k) {
      const size_t slot = (size_t)d.slot0 + k;
      const f32x2 ml = *(const f32x2*)(p.pk_ml + (slot * 128 + row) * 2);
      const float* acc = p.pk_acc + (slot * 128 + row) * kD + c16;
      const float mn = fmaxf(m, ml[0]), mu = mn == -INFINITY ? 0.f : mn;
      const float sa = __builtin_amdgcn_exp2f(m - mu), sb = __builtin_amdgcn_exp2f(ml[0] - mu);
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = o[e] * sa + *(const f32x4*)(acc + 4 * e) * sb;
      l = l * sa + ml[1] * sb;
      m = mn;
    }
    const float inv = 1.f / l;
    const int tok = row / p.G, head = d.h * p.G + (row - tok * p.G);
    uint16_t* op = p.out + ((size_t)(d.q_row0 + tok) * p.Hq + head) * kD + c16;
    u32x4 w0, w1;
    w0[0] = pack_bf16x2(o[0][0] * inv, o[0][1] * inv);
    w0[1] = pack_bf16x2(o[0][2] * inv, o[0][3] * inv);
    w0[2] = pack_bf16x2(o[1][0] * inv, o[1][1] * inv);
    w0[3] = pack_bf16x2(o[1][2] * inv, o[1][3] * inv);
    w1[0] = pack_bf16x2(o[2][0] * inv, o[2][1] * inv);
    w1[1] = pack_bf16x2(o[2][2] * inv, o[2][3] * inv);
    w1[2] = pack_bf16x2(o[3][0] * inv, o[3][1] * inv);
    w1[3] = pack_bf16x2(o[3][2] * inv, o[3][3] * inv);
    *(u32x4*)op = w0;
    *(u32x4*)(op + 8) = w1;
  }
  if (t == 0) dp->valid[g] = 0;
}

// The merge launch, in workgroups of CW waves.  CW = 2 (G <= 4: a decode row block's merge covers
// at most 4 rows; no prefill-kernel split tiles; the host chooses): two-wave workgroups, eight per
// CU, so a call's workgroups run in half the rounds of four-wave ones.
template <int CW>
__global__ __launch_bounds__(64 * CW) __attribute__((amdgpu_waves_per_eu(4))) void rpa_combine_kernel(Params p) {
  static_assert(CW == 2 || CW == 4, "combine workgroups of 2 or 4 waves");
  __shared__ float red[CW - 1][64][17];   // waves 1..CW-1's o (odd stride: conflict-free)
  __shared__ float redml[CW - 1][64][9];  // waves 1..CW-1's (m, l) per row slot
  if (blockIdx.x == 0 && threadIdx.x < kXcds) p.err[kQueueWord + threadIdx.x] = 0;  // tile queues, for the next call
  // the heavy-merge helpers first (a heavy merge is the longest, so it starts with the launch),
  // then the (descriptor, head) merges, then the rest
  const int nheavy = heavy_slots(p.grid) * p.HG * kHeavySlices;
  if ((int)blockIdx.x < nheavy) {
    combine_heavy<CW>(p, blockIdx.x, red, redml);
    return;
  }
  const int mb = (int)blockIdx.x - nheavy;
  if (mb >= p.grid * p.HG) {
    const int hb = mb - p.grid * p.HG;
    if (p.fused)
      fused_store_token(p, hb);
    else if (p.co)
      combine_co_split(p, hb);
    else
      combine_prefill<CW>(p, hb, red, redml);
    return;
  }
  // descriptor (last first: long splits end in late workgroups), wave (head) of its group
  const int bi = mb / p.HG, hw = mb - bi * p.HG, b = p.grid - 1 - bi;
  // the flag and the fields in one round trip (the empty asm keeps the compiler from moving the
  // field loads behind the flag test)
  int valid = p.desc[b].valid[hw];
  SplitDesc d = p.desc[b];
  asm volatile("" : "+v"(valid), "+v"(d.nch), "+v"(d.q_start), "+v"(d.q_len), "+v"(d.h), "+v"(d.rb), "+v"(d.b0));
  if (!__builtin_amdgcn_readfirstlane(valid)) return;
  const int t = threadIdx.x, wv = t >> 6, lane = t & 63;
  const int ncontrib = (int)(b - d.b0 + 1);
  if (ncontrib < kHeavyContrib) {
    const int nrows = rows_of(p, d);
    if (nrows <= 4) {
      MergeAcc<2> a;
      merge_rows<CW, 2, 4, 2>(p, d, hw, ncontrib, wv, lane, 0, 0, a);
      merge_waves_store<CW, 2, 2>(p, d, hw, nrows, wv, lane, 0, 0, a, red, redml);
    } else {
      // rows 0..7, then (16-row blocks) rows 8..15
#pragma unroll 1
      for (int row0 = 0; row0 < nrows; row0 += 8) {
        MergeAcc<4> a;
        merge_rows<CW, 4, 1, 2>(p, d, hw, ncontrib, wv, lane, row0, 0, a);
        merge_waves_store<CW, 4, 2>(p, d, hw, nrows, wv, lane, row0, 0, a, red, redml);
      }
    }
  }
  if (t == 0) p.desc[b].valid[hw] = 0;
}

// ---------------------------------------------------------------------------------------------
// gather probe
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rpa_gather_kernel(Params p, uint8_t* dense, long long dense_rows, int elem) {
  const int i = blockIdx.x;
  int nseq = p.num_seqs[0];
  nseq = nseq < 0 ? 0 : (nseq > p.Nmax ? p.Nmax : nseq);
  if (i >= nseq) return;
  long long row0 = 0;
  const long long cap = (long long)p.PPS * p.S;
  for (int k = 0; k < i; ++k) {
    long long L = p.kv_lens[k];
    row0 += L < 0 ? 0 : (L > cap ? cap : L);
  }
  long long L = p.kv_lens[i];
  L = L < 0 ? 0 : (L > cap ? cap : L);
  if (row0 + L > dense_rows) {
    if (threadIdx.x == 0) atomicOr(p.err, ERR_KVLEN);
    return;
  }
  const int row_bytes = 2 * p.Hkv * p.D * elem;
  const int vec = row_bytes / 16;
  for (long long t = 0; t < L; ++t) {
    int kt = (int)t;
    int pg = p.page_indices[(size_t)i * p.PPS + page_of(kt, p)];
    if (pg < 0 || pg >= p.P) {
      if (threadIdx.x == 0) atomicOr(p.err, ERR_PAGE);
      continue;
    }
    const u32x4* src = (const u32x4*)(p.kv + kv_elem(p, pg, kt, 0, p.D) * elem);
    u32x4* dst = (u32x4*)(dense + (size_t)(row0 + t) * row_bytes);
    for (int v = threadIdx.x; v < vec; v += blockDim.x) dst[v] = src[v];
  }
}

// ---------------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------------
thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

constexpr size_t kHeaderBytes = 256;

// Zeros standing in for rel_proj ([16, 8]) when the fused step has no relative bias.
__device__ uint16_t g_zero_proj[kRelRows * 8];

struct DeviceInfo {
  int cus = 0;
  const uint16_t* zero_proj = nullptr;  // this device's g_zero_proj
  int grid[kModes][9] = {};  // workgroups per launch, by kv mode and heads per workgroup (1..8)
};

std::mutex g_mu;
DeviceInfo g_dev[64];

// Heads per workgroup: the largest divisor of Hkv that is <= 8 (one wave each).
int heads_per_group(int hkv) {
  for (int g = hkv < 8 ? hkv : 8; g > 1; --g)
    if (hkv % g == 0) return g;
  return 1;
}

constexpr int kVtBytes = kWaveLds;  // LDS per wave: V region + K tile

// Workgroups for the persistent grid: the kernel's occupancy (2 waves per SIMD) in workgroups
// of hg waves, capped so no CU holds more than kMaxWavesPerCU waves.
template <int MODE>
int occupancy_grid(int cus, int hg) {
  int per_cu = 0;
  // the fused step runs only on the full-line path (whole-page units or per-key pages), with its
  // relative-bias staging: the smaller occupancy of its two instantiations
  constexpr bool kFused = MODE == KV_BF16_FUSED;
  const size_t lds = hg * (kVtBytes + (kFused ? kRelStage : 0));
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, rpa_attn_kernel<MODE, kFused>, 64 * hg, lds) !=
          hipSuccess ||
      per_cu <= 0)
    per_cu = 1;
  if constexpr (kFused) {
    int pl = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&pl, rpa_attn_kernel<MODE, false>, 64 * hg, lds) !=
            hipSuccess ||
        pl <= 0)
      pl = 1;
    per_cu = pl < per_cu ? pl : per_cu;
  }
  int max_groups = kMaxWavesPerCU / hg;
  if (max_groups < 1) max_groups = 1;
  if (per_cu > max_groups) per_cu = max_groups;
  return cus * per_cu;
}

// The attention grid: the occupancy grid (occ workgroups of hg waves on `cus` CUs), and with
// waves_per_cu in 1 .. kMaxWavesPerCU - 1 (rpa_options_t, a per-call tuning knob like the
// reference's block-size parameters) at most cus * waves_per_cu waves in all: floor(cus *
// waves_per_cu / hg) workgroups, at least one.  With 8 waves per workgroup, waves_per_cu = 4 is
// one workgroup per two CUs.
// Waves per combine workgroup: 2 when a decode row block's merge covers at most 4 rows (G <= 4)
// and no prefill-kernel split tile needs the 256-thread merges; 4 otherwise (rows of 8 and more
// merge faster over four waves).
int combine_waves(const Params& p) { return p.G <= 4 && !p.pf_kernel ? 2 : 4; }

int grid_rule(int occ, int cus, int hg, int waves_per_cu) {
  int grid = occ;
  if (waves_per_cu >= 1 && waves_per_cu < kMaxWavesPerCU) {
    long long cap = (long long)cus * waves_per_cu / hg;
    cap = cap < 1 ? 1 : cap;
    if (grid > cap) grid = (int)cap;
  }
  return grid;
}

int grid_for_call(const DeviceInfo& d, int mode, int hg, int waves_per_cu) {
  return grid_rule(d.grid[mode][hg], d.cus, hg, waves_per_cu);
}

int device_info(DeviceInfo& out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail(RPA_E_HIP, "hipGetDevice failed");
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceInfo& d = g_dev[dev];
  if (d.cus == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      return fail(RPA_E_HIP, "hipDeviceGetAttribute(MultiprocessorCount) failed");
    for (int hg = 1; hg <= 8; ++hg) {
      d.grid[KV_BF16][hg] = occupancy_grid<KV_BF16>(cus, hg);
      d.grid[KV_BF16_SCALED][hg] = occupancy_grid<KV_BF16_SCALED>(cus, hg);
      d.grid[KV_FP8][hg] = occupancy_grid<KV_FP8>(cus, hg);
      d.grid[KV_BF16_BIAS][hg] = occupancy_grid<KV_BF16_BIAS>(cus, hg);
      d.grid[KV_BF16_FUSED][hg] = occupancy_grid<KV_BF16_FUSED>(cus, hg);
    }
    // 8 zero columns of a 16-wide relative projection: the fused step without a relative bias
    if (hipGetSymbolAddress((void**)&d.zero_proj, HIP_SYMBOL(g_zero_proj)) != hipSuccess || !d.zero_proj)
      return fail(RPA_E_HIP, "hipGetSymbolAddress(zero projection) failed");
    d.cus = cus;
  }
  out = d;
  return RPA_OK;
}

// Workspace: [error word | pad to 256] [split descriptors, one per workgroup] [heavy-merge helper
// flags and descriptors] [prefill split descriptors] [split co tile descriptors] [partial m,l]
// [partial acc] [prefill partial m,l] [prefill partial acc] (the last two also hold the partials of
// split co tiles, whose layout never runs the prefill kernel).  Header, descriptors and flags are zeroed once (rpa_workspace_init);
// every call leaves each descriptor invalid and each flag clear again when its combine has run.
struct WsLayout {
  size_t desc, heavy, heavy_desc, pk_desc, co_desc, ml, acc, pk_ml, pk_acc, total;
};

size_t round256(size_t x) { return (x + 255) / 256 * 256; }

WsLayout ws_layout(const DeviceInfo& d) {
  const size_t gmax = (size_t)d.cus * kMaxWavesPerCU;
  WsLayout w;
  w.desc = kHeaderBytes;
  w.heavy = w.desc + round256(gmax * sizeof(SplitDesc));
  w.heavy_desc = w.heavy + round256((size_t)heavy_slots((int)gmax) * 8 * kHeavySlices * sizeof(int32_t));
  w.pk_desc = w.heavy_desc + round256((size_t)heavy_slots((int)gmax) * sizeof(SplitDesc));
  const size_t pk = (size_t)d.cus;  // prefill-kernel workgroups: one per CU
  w.co_desc = w.pk_desc + round256(pk * sizeof(PkDesc));  // split co tiles: one per CU
  w.ml = w.co_desc + round256((size_t)d.cus * sizeof(CoDesc));
  w.acc = w.ml + round256(2 * gmax * ROW_BLOCK * 2 * sizeof(float));
  w.pk_ml = w.acc + round256(2 * gmax * ROW_BLOCK * kD * sizeof(float));
  w.pk_acc = w.pk_ml + round256(2 * pk * kPkRows * 2 * sizeof(float));
  w.total = w.pk_acc + 2 * pk * kPkRows * kD * sizeof(float);
  return w;
}

size_t workspace_bytes_for(const DeviceInfo& d) { return ws_layout(d).total; }

int check_shape(const rpa_shape_t* s) {
  if (!s) return fail(RPA_E_INVALID, "shape is NULL");
  // head dims: 128; narrower ones read as 128-element rows, and 256 as two 128-dim halves (the
  // decode role's NW instantiation); a 16-byte piece of a narrow row is wholly inside or past it
  if (s->head_dim > kD && s->head_dim != 2 * kD)
    return fail(RPA_E_UNSUPPORTED, "head_dim " + std::to_string(s->head_dim) + " is not built (at most 128, or 256)");
  if (s->head_dim < kD && (s->kv_dtype == RPA_KV_FP8_E4M3 ? s->head_dim < 64 || s->head_dim % 16
                                                            : s->head_dim < 32 || s->head_dim % 8))
    return fail(RPA_E_UNSUPPORTED, "head_dim " + std::to_string(s->head_dim) +
                                       " is not built (a multiple of 8 in [32, 128]; fp8: of 16 in [64, 128]; or 256)");
  if (s->num_tokens < 0 || s->num_q_heads <= 0 || s->num_kv_heads <= 0 || s->total_pages <= 0 ||
      s->page_size <= 0 || s->max_num_seqs < 0 || s->pages_per_seq <= 0)
    return fail(RPA_E_INVALID, "non-positive dimension in shape");
  if (s->num_q_heads % s->num_kv_heads)
    return fail(RPA_E_INVALID, "num_q_heads=" + std::to_string(s->num_q_heads) +
                                   " must be divisible by num_kv_heads=" + std::to_string(s->num_kv_heads));
  if (s->kv_dtype != RPA_KV_BF16 && s->kv_dtype != RPA_KV_FP8_E4M3)
    return fail(RPA_E_INVALID, "kv_dtype must be RPA_KV_BF16 or RPA_KV_FP8_E4M3");
  if ((long long)s->pages_per_seq * s->page_size > 0x7fffffffll)
    return fail(RPA_E_INVALID, "pages_per_seq * page_size overflows int32");
  return RPA_OK;
}

// ---------------------------------------------------------------------------------------------
// fused Inkling decode: cache write, metadata expansion, bias table (small launches around the
// attention kernel; src/tpu_cake/workloads/inkling_rpa.py:471-589)
// ---------------------------------------------------------------------------------------------
constexpr int kMaxRelDim = 256;
constexpr int kBiasHeads = 4;    // q heads per bias-table block
constexpr int kBiasSlab = 256;   // table entries per bias-table block (one per thread)

struct FusedArgs {
  const uint16_t* q;        // [B, Hq, D]
  const uint16_t* keys;     // [B, Hkv, D]
  const uint16_t* values;   // [B, Hkv, D]
  uint16_t* cache;          // [P, S, 2*Hkv, W]
  const int32_t* kv_lens;   // [B]
  const int32_t* pages;     // [page_entries]
  const int32_t* cu_kv;     // [B+1]
  const uint16_t* rel_states;  // [B, Hq, R]
  const uint16_t* rel_proj;    // [R, E]
  int32_t* table;           // [B, PPS]
  int32_t* cu_q;            // [B+1]
  int32_t* nseq;            // [1]
  float* bias;              // kBiasHead zeros + [B, Hq, bias_row_len(E)]
  uint16_t* qpad;           // [B, Hq, W] (when D < W)
  int32_t* err;
  int B, Hq, Hkv, D, P, S, W, entries, pps, R, E;
  int vec;  // cache, keys and values 16-byte aligned and D % 8 == 0: rows written 8 elements at a time
};

__device__ __forceinline__ float bf16f(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// Block s: the new token's 2*Hkv rows (K of kv head h at combined row 2h, V at 2h+1), zero-padded
// to W, at slot (kv_len-1) % S of page pages[cu_kv[s]/S + (kv_len-1)/S].  Anything out of range is
// skipped and flagged (the host preflight rejects such metadata before the launch).
__device__ __forceinline__ void fused_write_rows(const FusedArgs& a, int s) {
  const int len = a.kv_lens[s], base = a.cu_kv[s];
  const int pos = len - 1;
  const long long entry = (long long)(base / a.S) + pos / a.S;
  bool ok = len >= 1 && len <= a.pps * a.S && base >= 0 && base % a.S == 0 && entry < a.entries;
  const int page = ok ? a.pages[entry] : 0;
  ok = ok && page >= 0 && page < a.P;
  if (!ok) {
    if (threadIdx.x == 0) atomicOr(a.err, ERR_PAGE);
    return;
  }
  uint16_t* rows = a.cache + ((size_t)page * a.S + pos % a.S) * (2 * a.Hkv) * a.W;
  const int n = 2 * a.Hkv * a.W;
  if (a.vec) {
    for (int i = 8 * threadIdx.x; i < n; i += 8 * blockDim.x) {
      const int r = i / a.W, d = i - r * a.W;
      u32x4 v = {0u, 0u, 0u, 0u};
      if (d < a.D) v = *(const u32x4*)(((r & 1) ? a.values : a.keys) + ((size_t)s * a.Hkv + (r >> 1)) * a.D + d);
      *(u32x4*)(rows + i) = v;
    }
  } else {
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      const int r = i / a.W, d = i - r * a.W;
      rows[i] = d < a.D ? ((r & 1) ? a.values : a.keys)[((size_t)s * a.Hkv + (r >> 1)) * a.D + d] : (uint16_t)0;
    }
  }
}

// One launch before the attention kernel (256 threads a block): blocks [0, B) write the new
// tokens' rows; the next B * ceil(Hq/kBiasHeads) * ceil(len/kBiasSlab) blocks the bias table
// (entry t of rows (s, h0..h0+3): the bias of the key at distance d = sum_r states[s, h, r] *
// proj[r, d] in fp32, 0 outside the window); the rest, grid-stride, the zero head, the
// [B, pages_per_seq] page table, cu_q = 0..B, num_seqs = B and the padded queries.
__global__ __launch_bounds__(256) void rpa_fused_prep_kernel(FusedArgs a, int write_blocks, int bias_blocks) {
  __shared__ float states[kBiasHeads * kMaxRelDim];
  if ((int)blockIdx.x < write_blocks) {
    fused_write_rows(a, blockIdx.x);
    return;
  }
  if ((int)blockIdx.x < write_blocks + bias_blocks) {
    const int len = bias_row_len(a.E), slabs = (len + kBiasSlab - 1) / kBiasSlab;
    const int hgroups = (a.Hq + kBiasHeads - 1) / kBiasHeads;
    const int nb = blockIdx.x - write_blocks, s = nb / (hgroups * slabs), rem = nb - s * hgroups * slabs;
    const int h0 = (rem / slabs) * kBiasHeads, t = (rem - (rem / slabs) * slabs) * kBiasSlab + threadIdx.x;
    for (int i = threadIdx.x; i < kBiasHeads * a.R; i += blockDim.x)
      states[i] = h0 + i / a.R < a.Hq ? bf16f(a.rel_states[((size_t)s * a.Hq + h0) * a.R + i]) : 0.f;
    __syncthreads();
    const int kv_len = a.kv_lens[s], d = (kv_len - 1) - (32 * bias_chunk_lo(kv_len, a.E) + t);
    float acc[kBiasHeads] = {};
    if (t < len && d >= 0 && d < a.E) {
#pragma unroll 16
      for (int r = 0; r < a.R; ++r) {
        const float pv = bf16f(a.rel_proj[(size_t)r * a.E + d]);
#pragma unroll
        for (int h = 0; h < kBiasHeads; ++h) acc[h] += states[h * a.R + r] * pv;
      }
    }
    if (t < len)
#pragma unroll
      for (int h = 0; h < kBiasHeads; ++h)
        if (h0 + h < a.Hq) a.bias[kBiasHead + ((size_t)s * a.Hq + h0 + h) * len + t] = acc[h];
    return;
  }
  const int first = write_blocks + bias_blocks;
  const long long tid = (long long)(blockIdx.x - first) * blockDim.x + threadIdx.x,
                  stride = (long long)(gridDim.x - first) * blockDim.x;
  for (long long i = tid; i < (long long)a.B * a.pps; i += stride) {
    const int s = (int)(i / a.pps), pg = (int)(i - (long long)s * a.pps);
    const int len = a.kv_lens[s];
    const long long e = (long long)(a.cu_kv[s] / a.S) + pg;
    a.table[i] = (pg < (len + a.S - 1) / a.S && e >= 0 && e < a.entries) ? a.pages[e] : 0;
  }
  for (long long i = tid; i <= a.B; i += stride) a.cu_q[i] = (int32_t)i;
  if (a.bias)
    for (long long i = tid; i < kBiasHead; i += stride) a.bias[i] = 0.f;
  if (tid == 0) a.nseq[0] = a.B;
  if (a.qpad)
    for (long long i = tid; i < (long long)a.B * a.Hq * a.W; i += stride) {
      const long long row = i / a.W;
      const int d = (int)(i - row * a.W);
      a.qpad[i] = d < a.D ? a.q[row * a.D + d] : (uint16_t)0;
    }
}

// out[s, h, :D] = padded[s, h, :D]
__global__ __launch_bounds__(256) void rpa_fused_unpad_kernel(const uint16_t* padded, uint16_t* out, long long rows,
                                                             int D, int W) {
  const long long tid = (long long)blockIdx.x * blockDim.x + threadIdx.x, stride = (long long)gridDim.x * blockDim.x;
  for (long long i = tid; i < rows * D; i += stride) {
    const long long row = i / D;
    out[i] = padded[row * W + (i - row * D)];
  }
}

// ---------------------------------------------------------------------------------------------
// Inkling decode, v1 contract (src/tpu_cake/workloads/inkling_rpa.py:37-73): separate K and V
// caches [P, S, Hkv, D], a [B, MP] page table, a bias [H, L] indexed by key position, scale 1/D.
// One prep launch packs the caches into the operator's combined layout and builds the metadata
// and the bias table; then the operator's kernels in bias mode.
// ---------------------------------------------------------------------------------------------
struct V1Args {
  const uint16_t* q;       // [B, H, D]
  const uint16_t* kc;      // [P, S, Hkv, D]
  const uint16_t* vc;      // [P, S, Hkv, D]
  const uint16_t* bias;    // [H, L]
  uint16_t* cache;         // [P, S, 2*Hkv, kD]
  float* table;            // kBiasHead zeros + [B, H, bias_row_len(L)]
  int32_t* cu_q;           // [B+1]
  int32_t* nseq;           // [1]
  uint16_t* qpad;          // [B, H, kD] when D < kD
  int B, H, Hkv, D, P, S, L;
  int vec;                 // caches 16-byte aligned and D % 8 == 0
};

// Grid-stride roles: the combined cache rows (8 elements a thread), the bias table, the
// metadata and the padded queries.
__global__ __launch_bounds__(256) void rpa_inkling_v1_prep_kernel(V1Args a) {
  const long long tid = (long long)blockIdx.x * blockDim.x + threadIdx.x, stride = (long long)gridDim.x * blockDim.x;
  const long long rows = (long long)a.P * a.S * 2 * a.Hkv;
  for (long long i = tid; i < rows * (kD / 8); i += stride) {
    const long long row = i / (kD / 8);
    const int d8 = (int)(i - row * (kD / 8)) * 8;
    const int comb = (int)(row % (2 * a.Hkv));
    const long long ps = row / (2 * a.Hkv);  // page * S + slot
    const uint16_t* src = ((comb & 1) ? a.vc : a.kc) + (ps * a.Hkv + (comb >> 1)) * a.D;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (a.vec) {
      if (d8 < a.D) v = *(const u32x4*)(src + d8);
    } else {
      uint16_t e[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) e[k] = d8 + k < a.D ? src[d8 + k] : (uint16_t)0;
#pragma unroll
      for (int k = 0; k < 4; ++k) v[k] = (uint32_t)e[2 * k] | ((uint32_t)e[2 * k + 1] << 16);
    }
    *(u32x4*)(a.cache + row * kD + d8) = v;
  }
  const int len = bias_row_len(a.L);
  for (long long i = tid; i < kBiasHead + (long long)a.B * a.H * len; i += stride) {
    float v = 0.f;
    if (i >= kBiasHead) {
      const long long k = i - kBiasHead, r = k / len;
      const int t = (int)(k - r * len), h = (int)(r % a.H);
      if (t < a.L) v = bf16f(a.bias[(size_t)h * a.L + t]);  // entry t = key t (the window starts at key 0)
    }
    a.table[i] = v;
  }
  for (long long i = tid; i <= a.B; i += stride) a.cu_q[i] = (int32_t)i;
  if (tid == 0) a.nseq[0] = a.B;
  if (a.qpad)
    for (long long i = tid; i < (long long)a.B * a.H * kD; i += stride) {
      const long long row = i / kD;
      const int d = (int)(i - row * kD);
      a.qpad[i] = d < a.D ? a.q[row * a.D + d] : (uint16_t)0;
    }
}

struct V1Layout {
  size_t cache, table, cu_q, nseq, qpad, opad, total;
};

struct FusedLayout {
  size_t table, cu_q, nseq, bias, qpad, opad, total;
};

Params base_params(const rpa_shape_t* s) {
  Params p;
  memset(&p, 0, sizeof(p));
  p.T = s->num_tokens;
  p.Hq = s->num_q_heads;
  p.Hkv = s->num_kv_heads;
  p.G = s->num_q_heads / s->num_kv_heads;
  p.P = s->total_pages;
  p.S = s->page_size;
  p.log2S = -1;
  if ((s->page_size & (s->page_size - 1)) == 0) p.log2S = __builtin_ctz((unsigned)s->page_size);
  p.Nmax = s->max_num_seqs;
  p.PPS = s->pages_per_seq;
  p.HG = heads_per_group(p.Hkv);
  p.D = s->head_dim;
  if (p.D == 2 * kD) {  // two 128-dim halves per kv head, both in one workgroup
    int g = p.Hkv < 4 ? p.Hkv : 4;
    while (p.Hkv % g) --g;
    p.HG = 2 * g;
  }
  p.NG = (p.D == 2 * kD ? 2 * p.Hkv : p.Hkv) / p.HG;
  return p;
}

// hipGetLastError reports the last failure of ANY runtime call on this thread (a caller's, or
// the framework's); clear it before launching so a launch check reports this library's own.
void clear_stale_error() { (void)hipGetLastError(); }

int check_fused(const rpa_fused_shape_t* f) {
  if (!f) return fail(RPA_E_INVALID, "fused shape is NULL");
  if (f->num_seqs < 1 || f->num_q_heads < 1 || f->num_kv_heads < 1 || f->num_q_heads % f->num_kv_heads)
    return fail(RPA_E_INVALID, "fused: bad sequence or head counts");
  if (f->cache_width != kD) return fail(RPA_E_UNSUPPORTED, "fused: cache_width must be 128");
  if (f->head_dim < 1 || f->head_dim > f->cache_width) return fail(RPA_E_INVALID, "fused: head_dim must be in [1, cache_width]");
  if (f->total_pages < 1 || f->page_size < 1 || f->page_entries < 1 || f->pages_per_seq < 1)
    return fail(RPA_E_INVALID, "fused: bad page counts");
  if (f->relative_dim < 0 || f->relative_dim > kMaxRelDim ||
      (f->relative_dim > 0 && (f->relative_extent < 1 || f->relative_extent > (1 << 24))))
    return fail(RPA_E_INVALID, "fused: relative_dim must be in [0, 256] with an extent in [1, 2^24]");
  if (f->relative_dim > 0 &&
      kBiasHead + (long long)f->num_seqs * f->num_q_heads * bias_row_len(f->relative_extent) >= (1LL << 31))
    return fail(RPA_E_INVALID, "fused: relative bias table exceeds 2^31 entries");
  if ((long long)f->pages_per_seq * f->page_size > INT32_MAX ||
      (long long)f->num_seqs * f->pages_per_seq > INT32_MAX ||
      (long long)f->num_seqs * f->num_q_heads * (f->relative_dim > 0 ? f->relative_extent : 1) > INT32_MAX)
    return fail(RPA_E_INVALID, "fused: sizes overflow int32");
  return RPA_OK;
}

rpa_shape_t fused_rpa_shape(const rpa_fused_shape_t* f) {
  rpa_shape_t r;
  r.num_tokens = f->num_seqs;
  r.num_q_heads = f->num_q_heads;
  r.num_kv_heads = f->num_kv_heads;
  r.head_dim = kD;
  r.total_pages = f->total_pages;
  r.page_size = f->page_size;
  r.max_num_seqs = f->num_seqs;
  r.pages_per_seq = f->pages_per_seq;
  r.kv_dtype = RPA_KV_BF16;
  return r;
}

// [operator workspace][page table][cu_q][num_seqs][bias table][padded q][padded out]
FusedLayout fused_layout(const DeviceInfo& d, const rpa_fused_shape_t* f) {
  FusedLayout l;
  const size_t B = (size_t)f->num_seqs, rows = B * f->num_q_heads;
  const size_t pad = f->head_dim < kD ? rows * kD * 2 : 0;
  l.table = round256(ws_layout(d).total);
  l.cu_q = l.table + round256(B * f->pages_per_seq * 4);
  l.nseq = l.cu_q + round256((B + 1) * 4);
  l.bias = l.nseq + 256;
  l.qpad = l.bias + round256(f->relative_dim > 0 ? (kBiasHead + rows * bias_row_len(f->relative_extent)) * 4 : 0);
  l.opad = l.qpad + round256(pad);
  l.total = l.opad + pad;
  return l;
}

int check_v1(const rpa_inkling_shape_t* f) {
  if (!f) return fail(RPA_E_INVALID, "inkling shape is NULL");
  if (f->num_seqs < 1 || f->num_q_heads < 1 || f->num_kv_heads < 1 || f->num_q_heads % f->num_kv_heads)
    return fail(RPA_E_INVALID, "inkling: query heads must divide evenly across key and value heads");
  if (f->head_dim < 1 || f->head_dim > kD) return fail(RPA_E_UNSUPPORTED, "inkling: head_dim must be in [1, 128]");
  if (f->total_pages < 1 || f->page_size < 1 || f->pages_per_seq < 1)
    return fail(RPA_E_INVALID, "inkling: bad page counts");
  if (f->bias_len < 1 || f->bias_len > (1 << 24)) return fail(RPA_E_INVALID, "inkling: bias_len must be in [1, 2^24]");
  if (kBiasHead + (long long)f->num_seqs * f->num_q_heads * bias_row_len(f->bias_len) >= (1LL << 31) ||
      (long long)f->pages_per_seq * f->page_size > INT32_MAX || (long long)f->num_seqs * f->pages_per_seq > INT32_MAX)
    return fail(RPA_E_INVALID, "inkling: sizes overflow int32");
  return RPA_OK;
}

rpa_shape_t v1_rpa_shape(const rpa_inkling_shape_t* f) {
  rpa_shape_t r;
  r.num_tokens = f->num_seqs;
  r.num_q_heads = f->num_q_heads;
  r.num_kv_heads = f->num_kv_heads;
  r.head_dim = kD;
  r.total_pages = f->total_pages;
  r.page_size = f->page_size;
  r.max_num_seqs = f->num_seqs;
  r.pages_per_seq = f->pages_per_seq;
  r.kv_dtype = RPA_KV_BF16;
  return r;
}

// [operator workspace][combined cache][bias table][cu_q][num_seqs][padded q][padded out]
V1Layout v1_layout(const DeviceInfo& d, const rpa_inkling_shape_t* f) {
  V1Layout l;
  const size_t B = (size_t)f->num_seqs, rows = B * f->num_q_heads;
  const size_t pad = f->head_dim < kD ? rows * kD * 2 : 0;
  l.cache = round256(ws_layout(d).total);
  l.table = l.cache + round256((size_t)f->total_pages * f->page_size * 2 * f->num_kv_heads * kD * 2);
  l.cu_q = l.table + round256((kBiasHead + rows * bias_row_len(f->bias_len)) * 4);
  l.nseq = l.cu_q + round256((B + 1) * 4);
  l.qpad = l.nseq + 256;
  l.opad = l.qpad + round256(pad);
  l.total = l.opad + pad;
  return l;
}

// ---------------------------------------------------------------------------------------------
// allocation-free entry (rpa_ragged_paged_attention_noalloc): the operator's workspace lives in a
// file-scope device array, one copy per GPU, found with hipGetSymbolAddress once per device
// ---------------------------------------------------------------------------------------------
// Bytes of the array: the workspace of a device with up to 320 CUs (about 400 KiB per CU: split
// descriptors, heavy-merge flags and split-K partials for a persistent grid of 8 waves per CU, and
// the prefill kernel's 256-row tile partials for one workgroup per CU).
constexpr size_t kScratchBytes = 128ull << 20;

__global__ __launch_bounds__(256) void rpa_scratch_clear_kernel(u32x4* p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
    p[i] = u32x4{0u, 0u, 0u, 0u};
}

struct ScratchState {
  void* ptr = nullptr;   // the device address of `scratch` on this device (never its host name)
  bool cleared = false;  // its header, descriptors and flags zeroed (every call leaves them so)
};
std::mutex g_scratch_mu;
ScratchState g_scratch[64];

}  // namespace
}  // namespace rpa

// The allocation-free entry point's workspace.  Host code never passes this name to a kernel or a
// copy: it is a host-side stand-in; the device address comes from hipGetSymbolAddress.
static __device__ __align__(256) uint8_t scratch[rpa::kScratchBytes];

using namespace rpa;

namespace rpa {
namespace {
// This device's scratch address; on first use on a device, its zero-initialised region (header,
// descriptors, heavy-merge flags) is cleared with a fill kernel on `stream` (a kernel, not a
// memset node, so the call stays capturable).
int scratch_for_device(const WsLayout& w, hipStream_t stream, void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail(RPA_E_HIP, "hipGetDevice failed");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchState& s = g_scratch[dev];
  if (!s.ptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(RPA_E_HIP, std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
    s.ptr = ptr;
  }
  if (!s.cleared) {
    // the clear must run before any call uses the array, so it cannot be left to a captured graph
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess)
      return fail(RPA_E_HIP, "hipStreamIsCapturing failed");
    if (cap != hipStreamCaptureStatusNone)
      return fail(RPA_E_INVALID, "the first allocation-free call on a device must run outside graph capture "
                                 "(it clears the device's scratch)");
    const size_t n16 = w.ml / 16;  // header .. heavy descriptors: a multiple of 256 bytes
    hipLaunchKernelGGL(rpa_scratch_clear_kernel, dim3(64), dim3(256), 0, stream, (u32x4*)s.ptr, n16);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(RPA_E_HIP, std::string("scratch clear launch failed: ") + hipGetErrorString(e));
    s.cleared = true;
  }
  *out = s.ptr;
  return RPA_OK;
}
}  // namespace
}  // namespace rpa

extern "C" {

int rpa_abi_version(void) { return RPA_ABI_VERSION; }

const char* rpa_last_error(void) { return g_last_error.c_str(); }

size_t rpa_workspace_size(const rpa_shape_t* shape) {
  if (check_shape(shape) != RPA_OK) return 0;
  DeviceInfo d;
  if (device_info(d) != RPA_OK) return 0;
  return workspace_bytes_for(d);
}

int rpa_workspace_init(void* workspace, size_t workspace_bytes, void* stream) {
  DeviceInfo d;
  int rc = device_info(d);
  if (rc) return rc;
  const WsLayout w = ws_layout(d);
  if (!workspace || workspace_bytes < w.total) return fail(RPA_E_WORKSPACE, "workspace too small");
  if (hipMemsetAsync(workspace, 0, w.ml, (hipStream_t)stream) != hipSuccess)
    return fail(RPA_E_HIP, "hipMemsetAsync failed");
  return RPA_OK;
}

int rpa_read_error_word(const void* workspace, size_t workspace_bytes, int32_t* host_word, void* stream) {
  if (!workspace || workspace_bytes < kHeaderBytes || !host_word) return fail(RPA_E_INVALID, "bad arguments");
  if (hipMemcpyAsync(host_word, workspace, sizeof(int32_t), hipMemcpyDeviceToHost, (hipStream_t)stream) !=
          hipSuccess ||
      hipStreamSynchronize((hipStream_t)stream) != hipSuccess)
    return fail(RPA_E_HIP, "reading the error word failed");
  return RPA_OK;
}

int rpa_timeline_read(int64_t* host_rows, int32_t rows, void* stream) {
#ifdef RPA_TIMELINE
  if (!host_rows || rows <= 0 || rows > kTlRows) return fail(RPA_E_INVALID, "bad timeline arguments");
  if (hipStreamSynchronize((hipStream_t)stream) != hipSuccess ||
      hipMemcpyFromSymbol(host_rows, HIP_SYMBOL(g_timeline), (size_t)rows * TL_FIELDS * sizeof(long long)) !=
          hipSuccess)
    return fail(RPA_E_HIP, "reading the timeline failed");
  return RPA_OK;
#else
  (void)host_rows, (void)rows, (void)stream;
  return fail(RPA_E_UNSUPPORTED, "this library was built without RPA_TIMELINE");
#endif
}

// Workspaces whose last call could not launch its combine kernel (descriptors, flags and the tile
// counter left set): cleared by the next call on them before it launches.
std::mutex g_dirty_mu;
std::vector<const void*> g_dirty_ws;

void mark_workspace_dirty(const void* ws) {
  std::lock_guard<std::mutex> lock(g_dirty_mu);
  for (const void* w : g_dirty_ws)
    if (w == ws) return;
  g_dirty_ws.push_back(ws);
}

bool take_workspace_dirty(const void* ws) {
  std::lock_guard<std::mutex> lock(g_dirty_mu);
  if (g_dirty_ws.empty()) return false;
  for (size_t i = 0; i < g_dirty_ws.size(); ++i)
    if (g_dirty_ws[i] == ws) {
      g_dirty_ws.erase(g_dirty_ws.begin() + i);
      return true;
    }
  return false;
}

// The fused decode step's own inputs when it runs in the attention launch (Params::fused).
struct FusedInline {
  int nseq, entries;
  const int32_t* cu_kv;
  const uint16_t* new_k;
  const uint16_t* new_v;
  const uint16_t* rel_states;  // nullptr: no relative bias
  const uint16_t* rel_proj;
  int rel_extent;
  int head_dim;  // of queries, new K/V rows and the output (the cache rows are kD wide)
};

int check_options(const rpa_options_t* opt) {
  if (opt->sliding_window < 0) return fail(RPA_E_INVALID, "sliding_window must be positive");
  if (opt->waves_per_cu < 0 || opt->waves_per_cu > kMaxWavesPerCU)
    return fail(RPA_E_INVALID, "waves_per_cu must be in [0, 8]");
  if (opt->prefill_tiles < -1 || opt->prefill_tiles > 3)
    return fail(RPA_E_INVALID, "prefill_tiles must be -1, 0, 1, 2 or 3");
  if (!(opt->prefill_cost >= 0.f && opt->prefill_cost <= 64.f))
    return fail(RPA_E_INVALID, "prefill_cost must be in [0, 64]");
  return RPA_OK;
}

// Workgroups per CU of the attention kernel at its occupancy (2 waves per SIMD, kMaxWavesPerCU
// waves) within the CU's LDS, for hg waves per workgroup and lds bytes of dynamic LDS each: what
// hipOccupancyMaxActiveBlocksPerMultiprocessor reports on gfx950.
constexpr int kLdsPerCu = 160 * 1024;
int nominal_per_cu(int hg, size_t lds) {
  int per_cu = kMaxWavesPerCU / hg;
  const int by_lds = (int)(kLdsPerCu / (lds + 256));  // 256: the kernel's static LDS, rounded up
  per_cu = per_cu < by_lds ? per_cu : by_lds;
  return per_cu < 1 ? 1 : per_cu;
}

// Where the rows of sequences with >= 16 query tokens go, and the workgroup shape that follows:
//   prefill_tiles 2 or 0, bf16 KV (plain or with scalar k/v scales) or fp8 KV, any mask value,
//     page size a multiple of 32, Hkv a multiple of 4, and num_tokens >= max_num_seqs + 15 (the
//     batch can hold such a sequence; a batch of one token per sequence keeps the decode layout):
//     the attention kernel's tiles in the co-resident layout (4-wave workgroups, two per CU, one
//     prefill and one stream-K workgroup side by side);
//   prefill_tiles 3, or 2 / 0 otherwise, for plain bf16 KV whose masked keys get weight 0 and
//     eight kv heads per workgroup: the attention kernel's tiles in 8-wave workgroups, one per
//     CU, roles split by CU;
//   prefill_tiles 1, or 0 when none of these applies: the prefill kernel (plain bf16 KV, masked
//     keys at weight 0, chunks in one page: page size a multiple of 64);
//   otherwise, and with -1: causal row blocks of the stream-K role.
void resolve_layout(Params& p, int mode, const rpa_shape_t* shape, const rpa_options_t* opt) {
  if (p.D != kD) return;  // a narrow head dim: every row through stream-K
  const int pt = opt->prefill_tiles;
  const bool bf = mode == KV_BF16 && p.skip_masked;
  const bool co_mode = mode == KV_BF16 || mode == KV_BF16_SCALED || mode == KV_FP8;  // any mask value
  const bool co_ok = co_mode && (pt == 0 || pt == 2) && p.S % KV_CHUNK == 0 && p.Hkv % kCoWaves == 0 &&
                     p.G <= 32 * kCoWaves && (long long)shape->num_tokens >= (long long)shape->max_num_seqs + 15;
  const bool tiles_ok = bf && p.HG == 8 && p.G <= 32 * p.HG;
  const bool pk_ok = bf && p.G <= kPkRows && p.S % kPkChunk == 0;
  const float cost = opt->prefill_cost > 0.f ? opt->prefill_cost : kPfCost;
  if (co_ok) {
    p.co = 1;
    p.HG = kCoWaves;
    p.NG = p.Hkv / kCoWaves;
    p.pf_tq = 32 * kCoWaves / p.G;
    p.pf_min = 16;
    p.pf_cost = cost;
  } else if (pk_ok && (pt == 1 || (pt == 0 && !tiles_ok))) {
    p.pf_kernel = true;
    p.pf_tq = kPkRows / p.G;
    p.pf_min = 16;
  } else if (tiles_ok && pt >= 0) {
    p.pf_tq = 32 * p.HG / p.G;
    p.pf_min = 16;
    p.pf_cost = cost;
  }
}

static int launch_rpa(const rpa_shape_t* shape, const rpa_options_t* opt, const void* q, const void* kv_pages,
                      const float* kv_scales, const int32_t* kv_lens, const int32_t* page_indices,
                      const int32_t* cu_q_lens, const int32_t* num_seqs, void* out, void* workspace,
                      size_t workspace_bytes, void* stream, void* ev_begin, void* ev_end,
                      const float* rel_bias = nullptr, int rel_extent = 0, const FusedInline* fz = nullptr) {
  int rc = check_shape(shape);
  if (rc) return rc;
  if (!opt) return fail(RPA_E_INVALID, "options is NULL");
  if (!kv_lens || !page_indices || (!fz && (!cu_q_lens || !num_seqs)) || !kv_pages)
    return fail(RPA_E_INVALID, "NULL metadata or kv_pages pointer");
  if (shape->num_tokens > 0 && (!q || !out)) return fail(RPA_E_INVALID, "NULL q or out pointer");
  if (q == out && q) return fail(RPA_E_INVALID, "out must not alias q");
  rc = check_options(opt);
  if (rc) return rc;
  if (shape->num_tokens == 0 || shape->max_num_seqs == 0) return RPA_OK;
  DeviceInfo d;
  rc = device_info(d);
  if (rc) return rc;
  const size_t need = workspace_bytes_for(d);
  if (!workspace || workspace_bytes < need)
    return fail(RPA_E_WORKSPACE, "workspace of " + std::to_string(workspace_bytes) + " bytes, need " +
                                     std::to_string(need));

  clear_stale_error();
  if (take_workspace_dirty(workspace)) {  // a previous call on it could not launch its combine
    const size_t n16 = ws_layout(d).ml / 16;
    hipLaunchKernelGGL(rpa_scratch_clear_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, (u32x4*)workspace, n16);
    const hipError_t ce = hipGetLastError();
    if (ce != hipSuccess) {
      mark_workspace_dirty(workspace);
      return fail(RPA_E_HIP, std::string("workspace clear failed: ") + hipGetErrorString(ce));
    }
  }
  Params p = base_params(shape);
  p.q = (const uint16_t*)q;
  p.kv = (const uint8_t*)kv_pages;
  p.kv_lens = kv_lens;
  p.page_indices = page_indices;
  p.cu_q_lens = cu_q_lens;
  p.num_seqs = num_seqs;
  p.out = (uint16_t*)out;
  p.err = (int32_t*)workspace;
  const WsLayout w = ws_layout(d);
  p.desc = (SplitDesc*)((uint8_t*)workspace + w.desc);
  p.heavy = (int32_t*)((uint8_t*)workspace + w.heavy);
  p.heavy_desc = (SplitDesc*)((uint8_t*)workspace + w.heavy_desc);
  p.part_ml = (float*)((uint8_t*)workspace + w.ml);
  p.part_acc = (float*)((uint8_t*)workspace + w.acc);
  p.pk_desc = (PkDesc*)((uint8_t*)workspace + w.pk_desc);
  p.pk_ml = (float*)((uint8_t*)workspace + w.pk_ml);
  p.pk_acc = (float*)((uint8_t*)workspace + w.pk_acc);
  p.sm_scale = opt->sm_scale;
  p.scale_log2 = opt->sm_scale * kLog2e;
  const float mask = opt->has_mask_value ? opt->mask_value : kDefaultMask;
  p.mask_log2 = mask * kLog2e;
  p.skip_masked = mask <= -1e30f;
  p.soft_cap = fabsf(opt->soft_cap);  // c * tanh(s / c) == |c| * tanh(s / |c|)
  p.sliding_window = opt->sliding_window;
  p.k_scale = opt->has_k_scale ? opt->k_scale : 1.f;
  p.v_scale = opt->has_v_scale ? opt->v_scale : 1.f;

  int mode = KV_BF16;
  if (fz) {  // the fused decode step in the attention launch (bias, if any, formed in the kernel)
    if ((long long)p.P * p.S > INT32_MAX)  // the per-key path's pool rows are 32-bit
      return fail(RPA_E_INVALID, "fused step in one launch needs total_pages * page_size < 2^31");
    mode = KV_BF16_FUSED;
    p.fused = 1;
    p.fused_nseq = fz->nseq;
    p.fused_entries = fz->entries;
    p.cu_kv = fz->cu_kv;
    p.new_k = fz->new_k;
    p.new_v = fz->new_v;
    p.rel_states = fz->rel_states;
    p.rel_proj = fz->rel_states ? fz->rel_proj : d.zero_proj;
    p.rel_extent = fz->rel_states ? fz->rel_extent : 8;
    p.D = fz->head_dim;  // (the cache rows keep kD: the kernel's row strides stay kD)
  } else if (rel_bias) {
    if (shape->kv_dtype != RPA_KV_BF16 || kv_scales || opt->has_k_scale || opt->has_v_scale || rel_extent <= 0)
      return fail(RPA_E_INVALID, "a relative bias needs bf16 kv_pages without scales and a positive extent");
    mode = KV_BF16_BIAS;
    p.rel_bias = rel_bias;
    p.rel_extent = rel_extent;
  } else if (shape->kv_dtype == RPA_KV_FP8_E4M3) {
    mode = KV_FP8;
    p.kv_scales = kv_scales;
  } else {
    if (kv_scales) return fail(RPA_E_INVALID, "kv_scales is only used with fp8 kv_pages");
    if (opt->has_k_scale || opt->has_v_scale) mode = KV_BF16_SCALED;
  }
  resolve_layout(p, mode, shape, opt);
  p.grid = grid_for_call(d, mode, p.HG, opt->waves_per_cu);
  if (p.pf_kernel) p.pk_grid = d.cus;
  // split co tiles: descriptors over the prefill-kernel descriptor area (one PkDesc per CU), partial
  // slots of 128 rows over its partial areas (2 x 256 rows per CU)
  static_assert(kCoMaxParts * 128 <= 2 * kPkRows, "co split tiles exceed the prefill-kernel partial areas");
  if (p.co) {
    p.co_split_max = d.cus;
    p.co_desc = (CoDesc*)((uint8_t*)workspace + w.co_desc);
  }
  hipStream_t st = (hipStream_t)stream;
  if (ev_begin && hipEventRecord((hipEvent_t)ev_begin, st) != hipSuccess)
    return fail(RPA_E_HIP, "hipEventRecord(begin) failed");
  const bool upg = p.S % KV_CHUNK == 0;
  const dim3 grid(p.grid), block(64 * p.HG);
  const size_t lds = (size_t)p.HG * (kVtBytes + (mode == KV_BF16_FUSED ? kRelStage : 0) +
                                     (p.D > kD ? kWideSlot : 0));
  if (mode == KV_BF16_FUSED) {
    if (upg) hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16_FUSED, true>), grid, block, lds, st, p);
    else hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16_FUSED, false>), grid, block, lds, st, p);
  } else if (mode == KV_BF16_BIAS) {
    if (upg) hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16_BIAS, true>), grid, block, lds, st, p);
    else hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16_BIAS, false>), grid, block, lds, st, p);
  } else if (p.D != kD) {  // a narrow head dim (decode role only)
    if (mode == KV_FP8) {
      if (upg) hipLaunchKernelGGL((rpa_attn_kernel<KV_FP8, true, false, true>), grid, block, lds, st, p);
      else hipLaunchKernelGGL((rpa_attn_kernel<KV_FP8, false, false, true>), grid, block, lds, st, p);
    } else if (mode == KV_BF16_SCALED) {
      // (32- and 64-element rows on the full-line path: their own instantiations, Lines<DN>)
      if (upg && p.D == 64) hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16_SCALED, true, false, true, 64>), grid, block, lds, st, p);
      else if (upg && p.D == 32) hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16_SCALED, true, false, true, 32>), grid, block, lds, st, p);
      else if (upg) hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16_SCALED, true, false, true>), grid, block, lds, st, p);
      else hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16_SCALED, false, false, true>), grid, block, lds, st, p);
    } else {
      if (upg && p.D == 64) hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16, true, false, true, 64>), grid, block, lds, st, p);
      else if (upg && p.D == 32) hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16, true, false, true, 32>), grid, block, lds, st, p);
      else if (upg) hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16, true, false, true>), grid, block, lds, st, p);
      else hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16, false, false, true>), grid, block, lds, st, p);
    }
  } else if (mode == KV_FP8) {
    if (p.co) hipLaunchKernelGGL((rpa_attn_kernel<KV_FP8, true, true>), grid, block, lds, st, p);
    else if (upg) hipLaunchKernelGGL((rpa_attn_kernel<KV_FP8, true>), grid, block, lds, st, p);
    else hipLaunchKernelGGL((rpa_attn_kernel<KV_FP8, false>), grid, block, lds, st, p);
  } else if (mode == KV_BF16_SCALED) {
    if (p.co) hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16_SCALED, true, true>), grid, block, lds, st, p);
    else if (upg) hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16_SCALED, true>), grid, block, lds, st, p);
    else hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16_SCALED, false>), grid, block, lds, st, p);
  } else {
    if (p.co) hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16, true, true>), grid, block, lds, st, p);
    else if (upg) hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16, true>), grid, block, lds, st, p);
    else hipLaunchKernelGGL((rpa_attn_kernel<KV_BF16, false>), grid, block, lds, st, p);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(RPA_E_HIP, std::string("attention launch failed: ") + hipGetErrorString(e));
  // From here the attention kernel has run, and its descriptors and tile counter wait in the
  // workspace for the combine kernel, which returns them to zero: the combine is launched whatever
  // else fails, and if it cannot be, the workspace is cleared before its next use.
  int err_rc = RPA_OK;
  if (p.pf_kernel) {
    hipLaunchKernelGGL(rpa_prefill_kernel, dim3(p.pk_grid), dim3(256), kPkLds, st, p);
    e = hipGetLastError();
    if (e != hipSuccess) err_rc = fail(RPA_E_HIP, std::string("prefill launch failed: ") + hipGetErrorString(e));
  }
  if (ev_end && hipEventRecord((hipEvent_t)ev_end, st) != hipSuccess && err_rc == RPA_OK)
    err_rc = fail(RPA_E_HIP, "hipEventRecord(end) failed");
  // the heavy-merge helpers of every slot, then one workgroup per (descriptor, head), then 16 per
  // prefill workgroup; two-wave workgroups when a decode row block has at most 4 rows (G <= 4,
  // no prefill-kernel split tiles), four-wave ones otherwise
  const dim3 cgrid(p.grid * p.HG + heavy_slots(p.grid) * p.HG * kHeavySlices + (p.pf_kernel ? 16 * p.pk_grid : 0) +
                   (p.fused ? p.fused_nseq : 0) + (p.co ? 4 * p.co_split_max : 0));
  if (combine_waves(p) == 2)
    hipLaunchKernelGGL(rpa_combine_kernel<2>, cgrid, dim3(128), 0, st, p);
  else
    hipLaunchKernelGGL(rpa_combine_kernel<4>, cgrid, dim3(256), 0, st, p);
  e = hipGetLastError();
  if (e != hipSuccess) {
    mark_workspace_dirty(workspace);
    return fail(RPA_E_HIP, std::string("combine launch failed: ") + hipGetErrorString(e));
  }
  return err_rc;
}

int rpa_attention_grid(const rpa_shape_t* shape, const rpa_options_t* opt, int32_t cus, int32_t* grid,
                       int32_t* waves_per_workgroup) {
  int rc = check_shape(shape);
  if (rc) return rc;
  if (!opt || !grid || !waves_per_workgroup) return fail(RPA_E_INVALID, "NULL options or output pointer");
  rc = check_options(opt);
  if (rc) return rc;
  if (cus < 0) return fail(RPA_E_INVALID, "cus must be >= 0");
  Params p = base_params(shape);
  const float mask = opt->has_mask_value ? opt->mask_value : kDefaultMask;
  p.skip_masked = mask <= -1e30f;
  int mode = KV_BF16;
  if (shape->kv_dtype == RPA_KV_FP8_E4M3)
    mode = KV_FP8;
  else if (opt->has_k_scale || opt->has_v_scale)
    mode = KV_BF16_SCALED;
  resolve_layout(p, mode, shape, opt);
  int occ;
  if (cus > 0) {
    occ = cus * nominal_per_cu(p.HG, (size_t)p.HG * kVtBytes);
  } else {
    DeviceInfo d;
    rc = device_info(d);
    if (rc) return rc;
    cus = d.cus;
    occ = d.grid[mode][p.HG];
  }
  *grid = grid_rule(occ, cus, p.HG, opt->waves_per_cu);
  *waves_per_workgroup = p.HG;
  return RPA_OK;
}

int rpa_ragged_paged_attention(const rpa_shape_t* shape, const rpa_options_t* opt, const void* q,
                               const void* kv_pages, const float* kv_scales, const int32_t* kv_lens,
                               const int32_t* page_indices, const int32_t* cu_q_lens, const int32_t* num_seqs,
                               void* out, void* workspace, size_t workspace_bytes, void* stream) {
  return launch_rpa(shape, opt, q, kv_pages, kv_scales, kv_lens, page_indices, cu_q_lens, num_seqs, out, workspace,
                    workspace_bytes, stream, nullptr, nullptr);
}

int rpa_ragged_paged_attention_timed(const rpa_shape_t* shape, const rpa_options_t* opt, const void* q,
                                     const void* kv_pages, const float* kv_scales, const int32_t* kv_lens,
                                     const int32_t* page_indices, const int32_t* cu_q_lens,
                                     const int32_t* num_seqs, void* out, void* workspace, size_t workspace_bytes,
                                     void* stream, void* event_begin, void* event_end) {
  return launch_rpa(shape, opt, q, kv_pages, kv_scales, kv_lens, page_indices, cu_q_lens, num_seqs, out, workspace,
                    workspace_bytes, stream, event_begin, event_end);
}

int rpa_ragged_paged_attention_noalloc(const rpa_shape_t* shape, const rpa_options_t* opt, const void* q,
                                       const void* kv_pages, const float* kv_scales, const int32_t* kv_lens,
                                       const int32_t* page_indices, const int32_t* cu_q_lens,
                                       const int32_t* num_seqs, void* out, void* stream) {
  int rc = check_shape(shape);
  if (rc) return rc;
  if (!opt) return fail(RPA_E_INVALID, "options is NULL");
  DeviceInfo d;
  rc = device_info(d);
  if (rc) return rc;
  const WsLayout w = ws_layout(d);
  if (w.total > kScratchBytes)
    return fail(RPA_E_WORKSPACE, "this device needs " + std::to_string(w.total) +
                                     " bytes of workspace; the allocation-free entry's scratch holds " +
                                     std::to_string(kScratchBytes) + " (use rpa_ragged_paged_attention)");
  void* ws = nullptr;
  rc = scratch_for_device(w, (hipStream_t)stream, &ws);
  if (rc) return rc;
  return launch_rpa(shape, opt, q, kv_pages, kv_scales, kv_lens, page_indices, cu_q_lens, num_seqs, out, ws,
                    kScratchBytes, stream, nullptr, nullptr);
}

int rpa_gather_kv(const rpa_shape_t* shape, const void* kv_pages, const int32_t* kv_lens,
                  const int32_t* page_indices, const int32_t* num_seqs, void* dense_out, int64_t dense_rows,
                  void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_shape(shape);
  if (rc) return rc;
  if (!kv_pages || !kv_lens || !page_indices || !num_seqs || (!dense_out && dense_rows > 0))
    return fail(RPA_E_INVALID, "NULL pointer");
  if (!workspace || workspace_bytes < kHeaderBytes) return fail(RPA_E_WORKSPACE, "workspace too small");
  if (shape->max_num_seqs == 0) return RPA_OK;
  Params p = base_params(shape);
  p.kv = (const uint8_t*)kv_pages;
  p.kv_lens = kv_lens;
  p.page_indices = page_indices;
  p.num_seqs = num_seqs;
  p.err = (int32_t*)workspace;
  const int elem = shape->kv_dtype == RPA_KV_FP8_E4M3 ? 1 : 2;
  hipLaunchKernelGGL(rpa_gather_kernel, dim3(shape->max_num_seqs), dim3(256), 0, (hipStream_t)stream, p,
                     (uint8_t*)dense_out, (long long)dense_rows, elem);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(RPA_E_HIP, std::string("gather launch failed: ") + hipGetErrorString(e));
  return RPA_OK;
}

size_t rpa_fused_workspace_size(const rpa_fused_shape_t* shape) {
  if (check_fused(shape) != RPA_OK) return 0;
  DeviceInfo d;
  if (device_info(d) != RPA_OK) return 0;
  return fused_layout(d, shape).total;
}

size_t rpa_inkling_workspace_size(const rpa_inkling_shape_t* shape) {
  if (check_v1(shape) != RPA_OK) return 0;
  DeviceInfo d;
  if (device_info(d) != RPA_OK) return 0;
  return v1_layout(d, shape).total;
}

int rpa_inkling_decode(const rpa_inkling_shape_t* f, float sm_scale, const void* query, const void* key_cache,
                       const void* value_cache, const int32_t* page_table, const int32_t* sequence_lengths,
                       const void* bias, void* out, void* workspace, size_t workspace_bytes, void* stream) {
  clear_stale_error();
  int rc = check_v1(f);
  if (rc) return rc;
  if (!query || !key_cache || !value_cache || !page_table || !sequence_lengths || !bias || !out)
    return fail(RPA_E_INVALID, "inkling: NULL pointer");
  DeviceInfo d;
  rc = device_info(d);
  if (rc) return rc;
  const V1Layout l = v1_layout(d, f);
  if (!workspace || workspace_bytes < l.total)
    return fail(RPA_E_WORKSPACE, "inkling workspace of " + std::to_string(workspace_bytes) + " bytes, need " +
                                     std::to_string(l.total));
  uint8_t* ws = (uint8_t*)workspace;
  V1Args a;
  a.q = (const uint16_t*)query;
  a.kc = (const uint16_t*)key_cache;
  a.vc = (const uint16_t*)value_cache;
  a.bias = (const uint16_t*)bias;
  a.cache = (uint16_t*)(ws + l.cache);
  a.table = (float*)(ws + l.table);
  a.cu_q = (int32_t*)(ws + l.cu_q);
  a.nseq = (int32_t*)(ws + l.nseq);
  a.qpad = f->head_dim < kD ? (uint16_t*)(ws + l.qpad) : nullptr;
  a.B = f->num_seqs;
  a.H = f->num_q_heads;
  a.Hkv = f->num_kv_heads;
  a.D = f->head_dim;
  a.P = f->total_pages;
  a.S = f->page_size;
  a.L = f->bias_len;
  a.vec = ((uintptr_t)key_cache | (uintptr_t)value_cache) % 16 == 0 && a.D % 8 == 0;
  hipStream_t st = (hipStream_t)stream;
  const long long work = (long long)a.P * a.S * 2 * a.Hkv * (kD / 8);
  long long blocks = (work + 255) / 256;
  blocks = blocks < 1 ? 1 : (blocks > 4096 ? 4096 : blocks);
  hipLaunchKernelGGL(rpa_inkling_v1_prep_kernel, dim3((unsigned)blocks), dim3(256), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(RPA_E_HIP, std::string("inkling prep launch failed: ") + hipGetErrorString(e));

  const rpa_shape_t rs = v1_rpa_shape(f);
  rpa_options_t o;
  memset(&o, 0, sizeof(o));
  o.sm_scale = sm_scale;
  void* attn_out = a.qpad ? (void*)(ws + l.opad) : out;
  rc = launch_rpa(&rs, &o, a.qpad ? (const void*)a.qpad : query, a.cache, nullptr, sequence_lengths, page_table,
                  a.cu_q, a.nseq, attn_out, workspace, workspace_bytes, stream, nullptr, nullptr, a.table, a.L);
  if (rc) return rc;
  if (a.qpad) {
    const long long rows = (long long)a.B * a.H;
    long long ub = (rows * a.D + 255) / 256;
    ub = ub < 1 ? 1 : (ub > 2048 ? 2048 : ub);
    hipLaunchKernelGGL(rpa_fused_unpad_kernel, dim3((unsigned)ub), dim3(256), 0, st, (const uint16_t*)attn_out,
                       (uint16_t*)out, rows, a.D, kD);
    e = hipGetLastError();
    if (e != hipSuccess) return fail(RPA_E_HIP, std::string("inkling unpad launch failed: ") + hipGetErrorString(e));
  }
  return RPA_OK;
}

int rpa_inkling_fused_decode(const rpa_fused_shape_t* f, float sm_scale, const void* queries, const void* keys,
                             const void* values, void* cache, const int32_t* kv_lens, const int32_t* page_indices,
                             const int32_t* cu_q_lens, const int32_t* cu_kv_lens, const int32_t* distribution,
                             const void* relative_states, const void* relative_projection, void* out,
                             void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_fused(f);
  if (rc) return rc;
  clear_stale_error();
  (void)cu_q_lens;     // decode-only contract: validated by the host preflight
  (void)distribution;
  if (!queries || !keys || !values || !cache || !kv_lens || !page_indices || !cu_kv_lens || !out)
    return fail(RPA_E_INVALID, "fused: NULL pointer");
  if (f->relative_dim > 0 && (!relative_states || !relative_projection))
    return fail(RPA_E_INVALID, "fused: NULL relative bias tensors");
  DeviceInfo d;
  rc = device_info(d);
  if (rc) return rc;
  const FusedLayout l = fused_layout(d, f);
  if (!workspace || workspace_bytes < l.total)
    return fail(RPA_E_WORKSPACE, "fused workspace of " + std::to_string(workspace_bytes) + " bytes, need " +
                                     std::to_string(l.total));
  uint8_t* ws = (uint8_t*)workspace;
  hipStream_t st = (hipStream_t)stream;
  // One attention launch (metadata, new token and relative bias handled in the kernel, the token
  // stored by the combine launch) on the full-line path -- whole-page units when the page size is
  // a multiple of 32, per-key pages otherwise -- with aligned tensors, head dims that are
  // multiples of 8 in [32, 128] (queries, new rows and the output of that width, the cache rows
  // 128) and no or a 16-wide relative projection; the prep launch below otherwise.
  const bool aligned = ((uintptr_t)queries | (uintptr_t)keys | (uintptr_t)values | (uintptr_t)cache |
                        (uintptr_t)relative_states | (uintptr_t)relative_projection) % 16 == 0;
  if (f->head_dim >= 32 && f->head_dim % 8 == 0 && (long long)f->total_pages * f->page_size <= INT32_MAX && aligned &&
      (f->relative_dim == 0 || (f->relative_dim == kRelRows && f->relative_extent % 8 == 0))) {
    const rpa_shape_t rs = fused_rpa_shape(f);
    rpa_options_t o;
    memset(&o, 0, sizeof(o));
    o.sm_scale = sm_scale;
    FusedInline fi;
    fi.nseq = f->num_seqs;
    fi.entries = f->page_entries;
    fi.cu_kv = cu_kv_lens;
    fi.new_k = (const uint16_t*)keys;
    fi.new_v = (const uint16_t*)values;
    fi.rel_states = f->relative_dim > 0 ? (const uint16_t*)relative_states : nullptr;
    fi.rel_proj = f->relative_dim > 0 ? (const uint16_t*)relative_projection : nullptr;
    fi.rel_extent = f->relative_dim > 0 ? f->relative_extent : 0;
    fi.head_dim = f->head_dim;
    return launch_rpa(&rs, &o, queries, cache, nullptr, kv_lens, page_indices, nullptr, nullptr, out, workspace,
                      workspace_bytes, stream, nullptr, nullptr, nullptr, 0, &fi);
  }
  FusedArgs a;
  a.q = (const uint16_t*)queries;
  a.keys = (const uint16_t*)keys;
  a.values = (const uint16_t*)values;
  a.cache = (uint16_t*)cache;
  a.kv_lens = kv_lens;
  a.pages = page_indices;
  a.cu_kv = cu_kv_lens;
  a.rel_states = (const uint16_t*)relative_states;
  a.rel_proj = (const uint16_t*)relative_projection;
  a.table = (int32_t*)(ws + l.table);
  a.cu_q = (int32_t*)(ws + l.cu_q);
  a.nseq = (int32_t*)(ws + l.nseq);
  a.bias = f->relative_dim > 0 ? (float*)(ws + l.bias) : nullptr;
  a.qpad = f->head_dim < kD ? (uint16_t*)(ws + l.qpad) : nullptr;
  a.err = (int32_t*)workspace;
  a.B = f->num_seqs;
  a.Hq = f->num_q_heads;
  a.Hkv = f->num_kv_heads;
  a.D = f->head_dim;
  a.P = f->total_pages;
  a.S = f->page_size;
  a.W = f->cache_width;
  a.entries = f->page_entries;
  a.pps = f->pages_per_seq;
  a.R = f->relative_dim;
  a.E = f->relative_dim > 0 ? f->relative_extent : 0;
  a.vec = ((uintptr_t)cache | (uintptr_t)keys | (uintptr_t)values) % 16 == 0 && a.D % 8 == 0 && a.W % 8 == 0;
  const int write_blocks = a.B,
            bias_blocks = a.bias ? a.B * ((a.Hq + kBiasHeads - 1) / kBiasHeads) *
                                       ((bias_row_len(a.E) + kBiasSlab - 1) / kBiasSlab)
                                 : 0;
  long long work = (long long)a.B * a.pps;
  if (a.qpad) work = work > (long long)a.B * a.Hq * a.W ? work : (long long)a.B * a.Hq * a.W;
  long long blocks = (work + 255) / 256;
  blocks = blocks < 1 ? 1 : (blocks > 2048 ? 2048 : blocks);
  hipLaunchKernelGGL(rpa_fused_prep_kernel, dim3((unsigned)(write_blocks + bias_blocks + blocks)), dim3(256), 0, st, a,
                     write_blocks, bias_blocks);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(RPA_E_HIP, std::string("fused prep launch failed: ") + hipGetErrorString(e));

  const rpa_shape_t rs = fused_rpa_shape(f);
  rpa_options_t o;
  memset(&o, 0, sizeof(o));
  o.sm_scale = sm_scale;
  void* attn_out = a.qpad ? (void*)(ws + l.opad) : out;
  rc = launch_rpa(&rs, &o, a.qpad ? (const void*)a.qpad : queries, cache, nullptr, kv_lens, a.table, a.cu_q, a.nseq,
                  attn_out, workspace, workspace_bytes, stream, nullptr, nullptr, a.bias, a.E);
  if (rc) return rc;
  if (a.qpad) {
    const long long rows = (long long)a.B * a.Hq;
    long long ub = (rows * a.D + 255) / 256;
    ub = ub < 1 ? 1 : (ub > 2048 ? 2048 : ub);
    hipLaunchKernelGGL(rpa_fused_unpad_kernel, dim3((unsigned)ub), dim3(256), 0, st, (const uint16_t*)attn_out,
                       (uint16_t*)out, rows, a.D, kD);
    e = hipGetLastError();
    if (e != hipSuccess) return fail(RPA_E_HIP, std::string("fused unpad launch failed: ") + hipGetErrorString(e));
  }
  return RPA_OK;
}

}  // extern "C"
