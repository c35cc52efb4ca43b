// Ragged paged attention for MI355X (gfx950): kernels and the C ABI of include/rpa.h.
//
// Semantics: ref_ragged_paged_attention, ecosystem/source/jax/ragged_paged_attention.py:73-148
// (causal offset kv_len - q_len, GQA kv_head = q_head / G, K at combined head 2h and V at
// 2h+1, fp32 scores and softmax, optional sliding window / soft cap / mask value / K,V scales).
//
// Structure (one call = two launches on the caller's stream):
//   rpa_attn_kernel     stream-K over (sequence, kv head, row block, 32-key chunk) units
//                       (see rpa_schedule.h); one 64-lane wave per workgroup; QK^T and PV
//                       on v_mfma_f32_16x16x32_bf16; online softmax in fp32 (exp2 domain);
//                       writes finished rows, or a split-K partial (m, l, acc).
//   rpa_combine_kernel  log-sum-exp merge of the partials of rows split across workgroups,
//                       and zeroes output rows at or past cu_q_lens[num_seqs].
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
//   P needs no cross-lane movement; V is transposed through LDS to match.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>
#include <string.h>

#include <mutex>
#include <string>

#include "rpa.h"
#include "rpa_schedule.h"

namespace rpa {
namespace {

constexpr int kD = 128;          // head_dim built
constexpr int kVTRow = 80;       // bytes per LDS row (one dim) of the transposed V chunk: 64 + 16 pad
constexpr int kMaxWavesPerCU = 8;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kDefaultMask = -0.7f * 3.4028234663852886e38f;  // ragged_paged_attention.py:32

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

enum KvMode { KV_BF16 = 0, KV_BF16_SCALED = 1, KV_FP8 = 2 };

enum ErrBits { ERR_PAGE = 1, ERR_QROW = 2, ERR_KVLEN = 4, ERR_QLEN = 8 };

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
  int32_t* err;
  int T, Hq, Hkv, G, P, S, log2S, Nmax, PPS;
  float sm_scale;
  float scale_log2;  // sm_scale * log2(e)
  float mask_log2;   // mask_value * log2(e)
  float soft_cap;    // 0 = off
  int sliding_window;
  float k_scale, v_scale;
  int grid;
  bool skip_masked;  // mask value so negative that masked keys get weight exactly 0
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
__device__ __forceinline__ size_t kv_elem(const Params& p, int pg, int kt, int comb) {
  return (((size_t)pg * (size_t)p.S + (size_t)slot_of(kt, p)) * (size_t)(2 * p.Hkv) + (size_t)comb) *
         (size_t)kD;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  __bf16 a = (__bf16)lo, b = (__bf16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// ---------------------------------------------------------------------------------------------
// sequence metadata (range-checked) and the unit -> position walk
// ---------------------------------------------------------------------------------------------
struct SeqInfo {
  int kv_len, q_start, q_len, units;  // units: per kv head
};

__device__ __forceinline__ SeqInfo load_seq(const Params& p, int i, int nseq) {
  SeqInfo s{0, 0, 0, 0};
  if (i < nseq) {
    int kv = p.kv_lens[i];
    int c0 = p.cu_q_lens[i];
    int c1 = p.cu_q_lens[i + 1];
    int err = 0;
    long long cap = (long long)p.PPS * p.S;
    if (kv > cap) { kv = (int)cap; err |= ERR_KVLEN; }
    if (kv < 0) kv = 0;
    int ql = c1 - c0;
    if (c0 < 0 || ql < 0 || c1 > p.T) { ql = 0; err |= ERR_QROW; }
    if (ql > kv) err |= ERR_QLEN;
    if (err) atomicOr(p.err, err);
    s.kv_len = kv;
    s.q_start = c0;
    s.q_len = ql;
    s.units = seq_units_per_head(kv, ql, p.G, p.skip_masked);
  }
  return s;
}

__device__ __forceinline__ long long total_units(const Params& p, int nseq, int lane) {
  long long w = 0;
  for (int base = 0; base < nseq; base += 64) {
    SeqInfo s = load_seq(p, base + lane, nseq);
    w += wave_sum64((long long)s.units * p.Hkv);
  }
  return w;
}

// Sequence holding unit u and the first unit of that sequence (wave-uniform results).
__device__ __forceinline__ void locate_seq(const Params& p, int nseq, int lane, long long u, int& seq,
                                           long long& seq_start) {
  long long off = 0;
  for (int base = 0; base < nseq; base += 64) {
    SeqInfo s = load_seq(p, base + lane, nseq);
    long long cnt = (long long)s.units * p.Hkv;
    long long incl = wave_incl_scan64(cnt, lane);
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

// Per-lane metadata of sequences [base, base + 64).
struct Window {
  int base;
  SeqInfo s;
};

__device__ __forceinline__ void load_window(const Params& p, int nseq, int base, int lane, Window& w) {
  w.base = base;
  w.s = load_seq(p, base + lane, nseq);
}

struct Cursor {
  int i, h, rb, c;  // sequence, kv head, row block, chunk
  int nch;          // chunks of (i, h, rb); 0 = past the end
  int nrb;
  int kv_len, q_len, q_start;
};

__device__ __forceinline__ void cursor_load_seq(const Params& p, const Window& w, int i, Cursor& x) {
  int k = i - w.base;
  x.i = i;
  x.kv_len = rl(w.s.kv_len, k);
  x.q_len = rl(w.s.q_len, k);
  x.q_start = rl(w.s.q_start, k);
  x.nrb = num_row_blocks(x.q_len, p.G);
}

__device__ __forceinline__ Cursor cursor_at(const Params& p, const Window& w, int seq, long long ul) {
  Cursor x;
  cursor_load_seq(p, w, seq, x);
  int per_head = rl(w.s.units, seq - w.base);
  x.h = (int)(ul / per_head);
  int rem = (int)(ul - (long long)x.h * per_head);
  x.rb = 0;
  for (;;) {
    int n = rb_units(x.kv_len, x.q_len, p.G, x.rb, p.skip_masked);
    if (rem < n) {
      x.c = rem;
      x.nch = n;
      break;
    }
    rem -= n;
    x.rb++;
  }
  return x;
}

__device__ __forceinline__ void advance(const Params& p, int nseq, int lane, Window& w, Cursor& x) {
  if (x.c + 1 < x.nch) {
    x.c++;
    return;
  }
  x.c = 0;
  for (;;) {
    if (x.rb + 1 < x.nrb) {
      x.rb++;
    } else if (x.h + 1 < p.Hkv) {
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
        if (i >= w.base + 64) load_window(p, nseq, i, lane, w);
        if (rl(w.s.units, i - w.base) > 0) break;
      }
      cursor_load_seq(p, w, i, x);
      x.h = 0;
      x.rb = 0;
    }
    x.nch = rb_units(x.kv_len, x.q_len, p.G, x.rb, p.skip_masked);
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

__device__ __forceinline__ Pages load_pages(const Params& p, const Cursor& x, int n) {
  Pages r;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    int kt = x.c * KV_CHUNK + 16 * blk + n;
    r.pg[blk] = 0;
    if (x.nch > 0 && kt < x.kv_len) r.pg[blk] = p.page_indices[(size_t)x.i * p.PPS + page_of(kt, p)];
  }
  return r;
}

template <int MODE>
struct KvRegs;

template <>
struct KvRegs<KV_BF16> {
  u32x4 k[2][4], v[2][4];
};
template <>
struct KvRegs<KV_BF16_SCALED> {
  u32x4 k[2][4], v[2][4];
};
template <>
struct KvRegs<KV_FP8> {
  u32x2 k[2][4], v[2][4];
  float ks[2], vs[2];
};

template <int MODE>
__device__ __forceinline__ void load_kv(const Params& p, const Cursor& x, const Pages& pages, int n, int j,
                                        KvRegs<MODE>& r) {
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    int kt = x.c * KV_CHUNK + 16 * blk + n;
    int pg = pages.pg[blk];
    bool in_seq = x.nch > 0 && kt < x.kv_len;
    bool ok = in_seq && pg >= 0 && pg < p.P;
    if (in_seq && !ok) atomicOr(p.err, ERR_PAGE);
    if constexpr (MODE == KV_FP8) {
      r.ks[blk] = p.k_scale;
      r.vs[blk] = p.v_scale;
#pragma unroll
      for (int s = 0; s < 4; ++s) r.k[blk][s] = r.v[blk][s] = u32x2{0u, 0u};
      if (ok) {
        size_t e = kv_elem(p, pg, kt, 2 * x.h) + 8 * j;
        const uint8_t* kp = p.kv + e;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          r.k[blk][s] = *(const u32x2*)(kp + 32 * s);
          r.v[blk][s] = *(const u32x2*)(kp + kD + 32 * s);
        }
        if (p.kv_scales) {
          const float* sc = p.kv_scales + ((size_t)pg * p.Hkv + x.h) * 2;
          r.ks[blk] *= sc[0];
          r.vs[blk] *= sc[1];
        }
      }
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) r.k[blk][s] = r.v[blk][s] = u32x4{0u, 0u, 0u, 0u};
      if (ok) {
        size_t e = kv_elem(p, pg, kt, 2 * x.h) + 8 * j;
        const uint16_t* kp = (const uint16_t*)p.kv + e;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          r.k[blk][s] = *(const u32x4*)(kp + 32 * s);
          r.v[blk][s] = *(const u32x4*)(kp + kD + 32 * s);
        }
      }
    }
  }
}

// Query rows of cursor x as the B operand of QK^T (zero for rows past q_len * G).
__device__ __forceinline__ void load_q(const Params& p, const Cursor& x, int n, int j, bf16x8 q[4]) {
  int row = x.rb * ROW_BLOCK + n;
  bool ok = x.nch > 0 && row < x.q_len * p.G;
  int tok = row / p.G;
  int g = row - tok * p.G;
#pragma unroll
  for (int s = 0; s < 4; ++s) q[s] = bf16x8{};
  if (ok) {
    const uint16_t* qp = p.q + ((size_t)(x.q_start + tok) * p.Hq + (size_t)x.h * p.G + g) * kD + 8 * j;
#pragma unroll
    for (int s = 0; s < 4; ++s) q[s] = __builtin_bit_cast(bf16x8, *(const u32x4*)(qp + 32 * s));
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

template <int MODE>
__device__ __forceinline__ void kv_to_bf16(const KvRegs<MODE>& r, const Params& p, u32x4 k[2][4],
                                           u32x4 v[2][4]) {
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if constexpr (MODE == KV_FP8) {
        k[blk][s] = fp8x8_to_bf16x8(r.k[blk][s], r.ks[blk]);
        v[blk][s] = fp8x8_to_bf16x8(r.v[blk][s], r.vs[blk]);
      } else if constexpr (MODE == KV_BF16_SCALED) {
        k[blk][s] = scale_bf16x8(r.k[blk][s], p.k_scale);
        v[blk][s] = scale_bf16x8(r.v[blk][s], p.v_scale);
      } else {
        k[blk][s] = r.k[blk][s];
        v[blk][s] = r.v[blk][s];
      }
    }
}

// ---------------------------------------------------------------------------------------------
// the attention kernel
// ---------------------------------------------------------------------------------------------
struct RowState {
  f32x4 acc[8];  // O^T: dims 16*blk + 4j + r, row n
  float m, l;    // running max (log2 units) and this lane's partial sum
  int pos;       // causal limit of this lane's row (last visible key)
  int row_ok;    // row < q_len * G
  int tok, head; // query token and query head of this lane's row
  bool started_here;
};

template <int MODE>
__device__ __forceinline__ void compute_unit(const Params& p, const Cursor& x, const KvRegs<MODE>& r,
                                             const bf16x8 q[4], RowState& st, uint8_t* vt, int n, int j) {
  u32x4 kb[2][4], vb[2][4];
  kv_to_bf16<MODE>(r, p, kb, vb);

  // S = K Q^T for the two 16-key blocks
  f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    s0 = mfma(__builtin_bit_cast(bf16x8, kb[0][s]), q[s], s0);
    s1 = mfma(__builtin_bit_cast(bf16x8, kb[1][s]), q[s], s1);
  }

  // V^T into LDS: key t = 16*blk + n goes to slot pos = 8*(n/4) + 4*blk + n%4 of each dim row
  __syncthreads();
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
    const int slot_b = 2 * (8 * (n >> 2) + 4 * blk + (n & 3));
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        uint32_t w = vb[blk][s][t];
        int d = 32 * s + 8 * j + 2 * t;
        *(uint16_t*)(vt + d * kVTRow + slot_b) = (uint16_t)(w & 0xffffu);
        *(uint16_t*)(vt + (d + 1) * kVTRow + slot_b) = (uint16_t)(w >> 16);
      }
  }

  // scores in log2 units with masks; this lane holds keys 16*blk + 4j + rr of row n
  float xs[2][4];
  const int key0 = x.c * KV_CHUNK + 4 * j;
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
      bool masked = kt > st.pos || (p.sliding_window > 0 && kt <= st.pos - p.sliding_window);
      if (masked) xv += p.mask_log2;
      if (kt >= x.kv_len) xv = -INFINITY;
      xs[blk][rr] = xv;
    }

  float mc = xs[0][0];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) mc = fmaxf(mc, xs[blk][rr]);
  mc = fmaxf(mc, __shfl_xor(mc, 16, 64));
  mc = fmaxf(mc, __shfl_xor(mc, 32, 64));
  const float mn = fmaxf(st.m, mc);
  const float mu = (mn == -INFINITY) ? 0.f : mn;
  const float alpha = __builtin_amdgcn_exp2f(st.m - mu);
  float pr[2][4];
  float lsum = 0.f;
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      pr[blk][rr] = __builtin_amdgcn_exp2f(xs[blk][rr] - mu);
      lsum += pr[blk][rr];
    }
  st.l = st.l * alpha + lsum;
  st.m = mn;
#pragma unroll
  for (int d = 0; d < 8; ++d) st.acc[d] *= alpha;

  u32x4 pw;
  pw[0] = pack_bf16x2(pr[0][0], pr[0][1]);
  pw[1] = pack_bf16x2(pr[0][2], pr[0][3]);
  pw[2] = pack_bf16x2(pr[1][0], pr[1][1]);
  pw[3] = pack_bf16x2(pr[1][2], pr[1][3]);
  const bf16x8 pb = __builtin_bit_cast(bf16x8, pw);

  __syncthreads();
#pragma unroll
  for (int d = 0; d < 8; ++d) {
    bf16x8 a = *(const bf16x8*)(vt + (16 * d + n) * kVTRow + 16 * j);
    st.acc[d] = mfma(a, pb, st.acc[d]);
  }
}

__device__ __forceinline__ void begin_row_block(const Params& p, const Cursor& x, RowState& st, int n) {
#pragma unroll
  for (int d = 0; d < 8; ++d) st.acc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  st.m = -INFINITY;
  st.l = 0.f;
  int row = x.rb * ROW_BLOCK + n;
  st.row_ok = row < x.q_len * p.G;
  st.tok = row / p.G;
  st.head = x.h * p.G + (row - st.tok * p.G);
  st.pos = x.kv_len - x.q_len + st.tok;
  st.started_here = x.c == 0;
}

__device__ __forceinline__ void finish_row_block(const Params& p, const Cursor& x, RowState& st, int b,
                                                 bool complete, int n, int j) {
  float lt = st.l;
  lt += __shfl_xor(lt, 16, 64);
  lt += __shfl_xor(lt, 32, 64);
  if (complete) {
    if (st.row_ok) {
      const float inv = 1.f / lt;
      uint16_t* op = p.out + ((size_t)(x.q_start + st.tok) * p.Hq + st.head) * kD + 4 * j;
#pragma unroll
      for (int d = 0; d < 8; ++d) {
        u32x2 w;
        w[0] = pack_bf16x2(st.acc[d][0] * inv, st.acc[d][1] * inv);
        w[1] = pack_bf16x2(st.acc[d][2] * inv, st.acc[d][3] * inv);
        *(u32x2*)(op + 16 * d) = w;
      }
    }
  } else {
    const size_t slot = (size_t)partial_slot(b, st.started_here);
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

template <int MODE>
__device__ __forceinline__ void step(const Params& p, int nseq, int lane, int n, int j, int b, long long u,
                                     long long u0, long long u1, Window& win, Cursor& cur, Cursor& nxt,
                                     Pages& pg_nxt, const KvRegs<MODE>& kv_cur, KvRegs<MODE>& kv_nxt,
                                     bf16x8 q[4], RowState& st, uint8_t* vt) {
  // Prefetch.  Every buffer is redefined on every path (zeros when there is no next unit) so a
  // buffer's previous contents are never kept alive across a step.
  //   K/V of the next unit: its page ids arrived during the previous step.
  load_kv<MODE>(p, nxt, pg_nxt, n, j, kv_nxt);
  //   queries of the next unit: new rows only when it starts a row block.
  bf16x8 qn[4];
  if (nxt.nch > 0 && nxt.c == 0) {
    load_q(p, nxt, n, j, qn);
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) qn[s] = q[s];
  }
  //   page ids two units ahead.
  Cursor ahead = nxt;
  if (u + 2 < u1)
    advance(p, nseq, lane, win, ahead);
  else
    ahead.nch = 0;
  pg_nxt = load_pages(p, ahead, n);

  if (u == u0 || cur.c == 0) begin_row_block(p, cur, st, n);
  compute_unit<MODE>(p, cur, kv_cur, q, st, vt, n, j);
  const bool last_of_rb = cur.c == cur.nch - 1;
  if (last_of_rb || u == u1 - 1) finish_row_block(p, cur, st, b, st.started_here && last_of_rb, n, j);

#pragma unroll
  for (int s = 0; s < 4; ++s) q[s] = qn[s];
  cur = nxt;
  nxt = ahead;
}

template <int MODE>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2, 2))) void rpa_attn_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) uint8_t vt[kD * kVTRow];
  const int lane = threadIdx.x;
  const int n = lane & 15, j = lane >> 4;
  const int b = blockIdx.x;
  int nseq = uni(p.num_seqs[0]);
  nseq = nseq < 0 ? 0 : (nseq > p.Nmax ? p.Nmax : nseq);

  const long long W = total_units(p, nseq, lane);
  if (W == 0) return;
  const long long u0 = uni64(range_start(b, W, p.grid)), u1 = uni64(range_start(b + 1, W, p.grid));
  if (u0 >= u1) return;

  int seq;
  long long seq_start;
  locate_seq(p, nseq, lane, u0, seq, seq_start);
  if (seq >= nseq) return;
  Window win;
  load_window(p, nseq, seq, lane, win);

  Cursor cur = cursor_at(p, win, seq, u0 - seq_start);
  Cursor nxt = cur;
  if (u0 + 1 < u1)
    advance(p, nseq, lane, win, nxt);
  else
    nxt.nch = 0;
  const Pages pg_cur = load_pages(p, cur, n);
  Pages pg_nxt = load_pages(p, nxt, n);
  KvRegs<MODE> kva, kvb;
  bf16x8 q[4];
  load_kv<MODE>(p, cur, pg_cur, n, j, kva);
  load_q(p, cur, n, j, q);
  RowState st;

  long long u = u0;
  for (;;) {
    step<MODE>(p, nseq, lane, n, j, b, u, u0, u1, win, cur, nxt, pg_nxt, kva, kvb, q, st, vt);
    if (++u >= u1) break;
    step<MODE>(p, nseq, lane, n, j, b, u, u0, u1, win, cur, nxt, pg_nxt, kvb, kva, q, st, vt);
    if (++u >= u1) break;
  }
}

// ---------------------------------------------------------------------------------------------
// split-K combine (+ zero fill of rows past the last sequence)
// ---------------------------------------------------------------------------------------------
__global__ __launch_bounds__(64) void rpa_combine_kernel(Params p) {
  const int lane = threadIdx.x;
  const int b = blockIdx.x;
  int nseq = p.num_seqs[0];
  nseq = nseq < 0 ? 0 : (nseq > p.Nmax ? p.Nmax : nseq);

  if (b == 0) {
    int tv = p.cu_q_lens[nseq];
    tv = tv < 0 ? 0 : (tv > p.T ? p.T : tv);
    const size_t first = (size_t)tv * p.Hq * kD / 8, last = (size_t)p.T * p.Hq * kD / 8;
    u32x4* o = (u32x4*)p.out;
    for (size_t k = first + lane; k < last; k += 64) o[k] = u32x4{0u, 0u, 0u, 0u};
  }

  const long long W = total_units(p, nseq, lane);
  if (W == 0) return;
  const long long u0 = range_start(b, W, p.grid), u1 = range_start(b + 1, W, p.grid);
  if (u0 >= u1) return;
  int seq;
  long long seq_start;
  locate_seq(p, nseq, lane, u0, seq, seq_start);
  if (seq >= nseq) return;
  Window win;
  load_window(p, nseq, seq, lane, win);
  const Cursor x = cursor_at(p, win, seq, u0 - seq_start);
  if (x.c == 0) return;                         // the row block began in this workgroup
  const long long tstart = u0 - x.c, tend = tstart + x.nch;
  if (tend > u1) return;                        // a later workgroup holds its end
  const long long b0 = owner_of(tstart, W, p.grid);

  const int n = lane & 15, quarter = lane >> 4;  // row n, dims 32*quarter .. +32
  float mstar = -INFINITY;
  for (long long bb = b0; bb <= b; ++bb) {
    if (range_start(bb, W, p.grid) == range_start(bb + 1, W, p.grid)) continue;
    const size_t slot = (size_t)partial_slot(bb, bb == b0);
    mstar = fmaxf(mstar, p.part_ml[(slot * ROW_BLOCK + n) * 2]);
  }
  const float mu = mstar == -INFINITY ? 0.f : mstar;
  float o[32];
#pragma unroll
  for (int k = 0; k < 32; ++k) o[k] = 0.f;
  float lsum = 0.f;
  for (long long bb = b0; bb <= b; ++bb) {
    if (range_start(bb, W, p.grid) == range_start(bb + 1, W, p.grid)) continue;
    const size_t slot = (size_t)partial_slot(bb, bb == b0);
    const float* ml = p.part_ml + (slot * ROW_BLOCK + n) * 2;
    const float w = __builtin_amdgcn_exp2f(ml[0] - mu);
    lsum += w * ml[1];
    const f32x4* ap = (const f32x4*)(p.part_acc + (slot * ROW_BLOCK + n) * kD + 32 * quarter);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      f32x4 a = ap[k];
      o[4 * k + 0] += w * a[0];
      o[4 * k + 1] += w * a[1];
      o[4 * k + 2] += w * a[2];
      o[4 * k + 3] += w * a[3];
    }
  }
  const int row = x.rb * ROW_BLOCK + n;
  if (row < x.q_len * p.G) {
    const int tok = row / p.G;
    const int head = x.h * p.G + (row - tok * p.G);
    const float inv = 1.f / lsum;
    // partial acc rows are stored as O^T column n: dim d at index d (see finish_row_block)
    uint16_t* op = p.out + ((size_t)(x.q_start + tok) * p.Hq + head) * kD + 32 * quarter;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      u32x2 w;
      w[0] = pack_bf16x2(o[4 * k + 0] * inv, o[4 * k + 1] * inv);
      w[1] = pack_bf16x2(o[4 * k + 2] * inv, o[4 * k + 3] * inv);
      *(u32x2*)(op + 4 * k) = w;
    }
  }
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
  const int row_bytes = 2 * p.Hkv * kD * elem;
  const int vec = row_bytes / 16;
  for (long long t = 0; t < L; ++t) {
    int kt = (int)t;
    int pg = p.page_indices[(size_t)i * p.PPS + page_of(kt, p)];
    if (pg < 0 || pg >= p.P) {
      if (threadIdx.x == 0) atomicOr(p.err, ERR_PAGE);
      continue;
    }
    const u32x4* src = (const u32x4*)(p.kv + kv_elem(p, pg, kt, 0) * elem);
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

struct DeviceInfo {
  int cus = 0;
  int grid[3] = {0, 0, 0};
};

std::mutex g_mu;
DeviceInfo g_dev[64];

template <int MODE>
int occupancy_grid(int cus) {
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, rpa_attn_kernel<MODE>, 64, 0) != hipSuccess ||
      per_cu <= 0)
    per_cu = 2;
  if (per_cu > kMaxWavesPerCU) per_cu = kMaxWavesPerCU;
  return cus * per_cu;
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
    d.grid[KV_BF16] = occupancy_grid<KV_BF16>(cus);
    d.grid[KV_BF16_SCALED] = occupancy_grid<KV_BF16_SCALED>(cus);
    d.grid[KV_FP8] = occupancy_grid<KV_FP8>(cus);
    d.cus = cus;
  }
  out = d;
  return RPA_OK;
}

size_t workspace_bytes_for(const DeviceInfo& d) {
  int gmax = d.cus * kMaxWavesPerCU;
  size_t ml = (size_t)2 * gmax * ROW_BLOCK * 2 * sizeof(float);
  size_t acc = (size_t)2 * gmax * ROW_BLOCK * kD * sizeof(float);
  return kHeaderBytes + ((ml + 255) / 256) * 256 + acc;
}

int check_shape(const rpa_shape_t* s) {
  if (!s) return fail(RPA_E_INVALID, "shape is NULL");
  if (s->head_dim != kD)
    return fail(RPA_E_UNSUPPORTED, "head_dim " + std::to_string(s->head_dim) + " is not built (only 128)");
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
  return p;
}

}  // namespace
}  // namespace rpa

using namespace rpa;

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
  if (!workspace || workspace_bytes < kHeaderBytes) return fail(RPA_E_WORKSPACE, "workspace too small");
  if (hipMemsetAsync(workspace, 0, kHeaderBytes, (hipStream_t)stream) != hipSuccess)
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

static int launch_rpa(const rpa_shape_t* shape, const rpa_options_t* opt, const void* q, const void* kv_pages,
                      const float* kv_scales, const int32_t* kv_lens, const int32_t* page_indices,
                      const int32_t* cu_q_lens, const int32_t* num_seqs, void* out, void* workspace,
                      size_t workspace_bytes, void* stream, void* ev_begin, void* ev_end) {
  int rc = check_shape(shape);
  if (rc) return rc;
  if (!opt) return fail(RPA_E_INVALID, "options is NULL");
  if (!kv_lens || !page_indices || !cu_q_lens || !num_seqs || !kv_pages)
    return fail(RPA_E_INVALID, "NULL metadata or kv_pages pointer");
  if (shape->num_tokens > 0 && (!q || !out)) return fail(RPA_E_INVALID, "NULL q or out pointer");
  if (q == out && q) return fail(RPA_E_INVALID, "out must not alias q");
  if (opt->sliding_window < 0) return fail(RPA_E_INVALID, "sliding_window must be positive");
  if (shape->num_tokens == 0 || shape->max_num_seqs == 0) return RPA_OK;
  DeviceInfo d;
  rc = device_info(d);
  if (rc) return rc;
  const size_t need = workspace_bytes_for(d);
  if (!workspace || workspace_bytes < need)
    return fail(RPA_E_WORKSPACE, "workspace of " + std::to_string(workspace_bytes) + " bytes, need " +
                                     std::to_string(need));

  Params p = base_params(shape);
  p.q = (const uint16_t*)q;
  p.kv = (const uint8_t*)kv_pages;
  p.kv_lens = kv_lens;
  p.page_indices = page_indices;
  p.cu_q_lens = cu_q_lens;
  p.num_seqs = num_seqs;
  p.out = (uint16_t*)out;
  p.err = (int32_t*)workspace;
  const int gmax = d.cus * kMaxWavesPerCU;
  const size_t ml_bytes = (((size_t)2 * gmax * ROW_BLOCK * 2 * sizeof(float)) + 255) / 256 * 256;
  p.part_ml = (float*)((uint8_t*)workspace + kHeaderBytes);
  p.part_acc = (float*)((uint8_t*)workspace + kHeaderBytes + ml_bytes);
  p.sm_scale = opt->sm_scale;
  p.scale_log2 = opt->sm_scale * kLog2e;
  const float mask = opt->has_mask_value ? opt->mask_value : kDefaultMask;
  p.mask_log2 = mask * kLog2e;
  p.skip_masked = mask <= -1e30f;
  p.soft_cap = opt->soft_cap;
  p.sliding_window = opt->sliding_window;
  p.k_scale = opt->has_k_scale ? opt->k_scale : 1.f;
  p.v_scale = opt->has_v_scale ? opt->v_scale : 1.f;

  int mode = KV_BF16;
  if (shape->kv_dtype == RPA_KV_FP8_E4M3) {
    mode = KV_FP8;
    p.kv_scales = kv_scales;
  } else {
    if (kv_scales) return fail(RPA_E_INVALID, "kv_scales is only used with fp8 kv_pages");
    if (opt->has_k_scale || opt->has_v_scale) mode = KV_BF16_SCALED;
  }
  p.grid = d.grid[mode];
  hipStream_t st = (hipStream_t)stream;
  if (ev_begin && hipEventRecord((hipEvent_t)ev_begin, st) != hipSuccess)
    return fail(RPA_E_HIP, "hipEventRecord(begin) failed");
  if (mode == KV_FP8)
    hipLaunchKernelGGL(rpa_attn_kernel<KV_FP8>, dim3(p.grid), dim3(64), 0, st, p);
  else if (mode == KV_BF16_SCALED)
    hipLaunchKernelGGL(rpa_attn_kernel<KV_BF16_SCALED>, dim3(p.grid), dim3(64), 0, st, p);
  else
    hipLaunchKernelGGL(rpa_attn_kernel<KV_BF16>, dim3(p.grid), dim3(64), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(RPA_E_HIP, std::string("attention launch failed: ") + hipGetErrorString(e));
  if (ev_end && hipEventRecord((hipEvent_t)ev_end, st) != hipSuccess)
    return fail(RPA_E_HIP, "hipEventRecord(end) failed");
  hipLaunchKernelGGL(rpa_combine_kernel, dim3(p.grid), dim3(64), 0, st, p);
  e = hipGetLastError();
  if (e != hipSuccess) return fail(RPA_E_HIP, std::string("combine launch failed: ") + hipGetErrorString(e));
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

}  // extern "C"
