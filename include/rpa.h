/*
 * librpa -- ragged paged attention (RPA) for AMD Instinct MI355X (gfx950).
 *
 * C ABI: plain pointers and sizes, no C++ or torch types.  All tensor
 * pointers are DEVICE pointers owned by the caller; the library never
 * allocates or frees on the call path.  Every entry point returns 0 on
 * success or a negative RPA_E* code; rpa_last_error() then describes it
 * (thread-local string).
 *
 * Tensor layouts are the reference operator's
 * (ecosystem/source/jax/ragged_paged_attention.py:718-750):
 *   q            bf16  [num_tokens, num_q_heads, head_dim]
 *   kv_pages     bf16 | fp8-e4m3 (OCP E4M3FN)  [total_pages, page_size, 2*num_kv_heads, head_dim]
 *                K of kv head h is combined head 2h, V is 2h+1 (:116-121, :361-393)
 *   kv_lens      int32 [max_num_seqs]
 *   page_indices int32 [max_num_seqs, pages_per_seq] (row-major)
 *   cu_q_lens    int32 [max_num_seqs + 1]
 *   num_seqs     int32 [1]
 *   out          bf16  [num_tokens, num_q_heads, head_dim]
 */
#ifndef RPA_H_
#define RPA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RPA_ABI_VERSION 2

enum {
  RPA_OK = 0,
  RPA_E_INVALID = -1,    /* bad shape / option / pointer */
  RPA_E_UNSUPPORTED = -2,/* valid for the reference but not built here (e.g. head_dim) */
  RPA_E_WORKSPACE = -3,  /* workspace missing or too small */
  RPA_E_HIP = -4         /* a HIP runtime call failed */
};

enum { RPA_KV_BF16 = 0, RPA_KV_FP8_E4M3 = 1 };

/* Static description of one call (shapes are the reference's, :73-80). */
typedef struct rpa_shape {
  int32_t num_tokens;    /* T = q.shape[0] (max_num_batched_tokens) */
  int32_t num_q_heads;   /* Hq */
  int32_t num_kv_heads;  /* Hkv; kv_pages.shape[2] == 2*Hkv */
  int32_t head_dim;      /* D: 128; a multiple of 8 in [32, 128) (fp8: of 16 in [64, 128)); or
                            256 -- the last two run every row through the decode role */
  int32_t total_pages;   /* P = kv_pages.shape[0] */
  int32_t page_size;     /* S = kv_pages.shape[1] */
  int32_t max_num_seqs;  /* N_max = page_indices.shape[0] */
  int32_t pages_per_seq; /* PPS = page_indices.shape[1] */
  int32_t kv_dtype;      /* RPA_KV_BF16 | RPA_KV_FP8_E4M3 */
} rpa_shape_t;

/* Scalar knobs of the reference signature (:718-731).  Zero-initialise and
 * set what is used: sliding_window 0 = none, soft_cap 0 = none (any nonzero
 * value caps as the reference's soft_cap * tanh(s / soft_cap), which equals
 * |soft_cap| * tanh(s / |soft_cap|)), has_mask_value 0 = DEFAULT_MASK_VALUE
 * (-0.7 * FLT_MAX, :32), has_k_scale / has_v_scale 0 = no scalar K/V scale.
 *
 * Tuning knobs (ABI 2), per call, zero = the library default; they change the
 * schedule, never the result beyond fp32 summation order.  They take the place
 * of the reference's per-call block sizes num_kv_pages_per_block /
 * num_queries_per_block (ragged_paged_attention.py:726-728, :801-816):
 *   waves_per_cu   1..7 caps the persistent attention grid at cus * waves_per_cu
 *                  waves: floor(cus * waves_per_cu / waves_per_workgroup)
 *                  workgroups, at least one (with 8-wave workgroups, 4 is one
 *                  workgroup per two CUs); 0 or 8: the kernel's occupancy, 8
 *                  waves per CU (rpa_attention_grid reports the result);
 *   prefill_tiles  sequences with at least 16 query tokens (bf16 KV without
 *                  scales, the default mask value): 2 = the attention kernel's
 *                  own MFMA prefill tiles, in two 4-wave workgroups per CU (one
 *                  prefill, one stream-K) when the page size is a multiple of
 *                  32, Hkv a multiple of 4 and num_tokens >= max_num_seqs + 15,
 *                  else in one 8-wave workgroup per CU (8 kv heads per
 *                  workgroup); 3 = those tiles in one 8-wave workgroup per CU;
 *                  1 = the standalone prefill kernel (page size a multiple of
 *                  64); 0 = 2, else 1, whichever applies first; -1 = causal row
 *                  blocks of the stream-K role (also whenever none applies);
 *   prefill_cost   > 0: the cost of one prefill-tile chunk step in stream-K
 *                  units, which sets the work split between the two roles
 *                  (0 = 0.45). */
typedef struct rpa_options {
  float sm_scale;
  int32_t sliding_window;
  float soft_cap;
  int32_t has_mask_value;
  float mask_value;
  int32_t has_k_scale;
  float k_scale;
  int32_t has_v_scale;
  float v_scale;
  int32_t waves_per_cu;
  int32_t prefill_tiles;
  float prefill_cost;
} rpa_options_t;

/* The attention launch a call of this shape and these options makes: *grid workgroups of
 * *waves_per_workgroup waves, on a device of `cus` compute units at the kernel's nominal
 * occupancy (8 waves per CU within 160 KiB of LDS; no device is touched), or on the current
 * device when cus is 0.  No counterpart in the reference (its grid is (Hq/Hq_blk, cdiv(T,
 * q_per_blk)), ragged_paged_attention.py:822-823); it lets a tuner tell the waves_per_cu knob's
 * values apart. */
int rpa_attention_grid(const rpa_shape_t* shape, const rpa_options_t* options, int32_t cus, int32_t* grid,
                       int32_t* waves_per_workgroup);

/* ABI version of the loaded library (RPA_ABI_VERSION). */
int rpa_abi_version(void);

/* Message for the last nonzero return on this thread ("" if none). */
const char* rpa_last_error(void);

/* Bytes of device workspace rpa_ragged_paged_attention needs for this shape
 * on the CURRENT device (split-K partials, error word).  0 on error.
 * Replaces the scratch the reference's pallas_call allocates itself
 * (ragged_paged_attention.py:837-863). */
size_t rpa_workspace_size(const rpa_shape_t* shape);

/* One-time initialisation of a freshly allocated workspace (zeroes the error
 * word, the split-K descriptors and the heavy-merge flags, which every call
 * leaves cleared again),
 * stream-ordered.  Call once per workspace buffer.  Calls sharing one
 * workspace must not overlap in time (same stream, or ordered by events). */
int rpa_workspace_init(void* workspace, size_t workspace_bytes, void* stream);

/* Ragged paged attention forward.  Replaces
 *   ragged_paged_attention(q, kv_pages, kv_lens, page_indices, cu_q_lens, num_seqs, *,
 *       sm_scale, sliding_window, soft_cap, mask_value, k_scale, v_scale, ...)
 *   ecosystem/source/jax/ragged_paged_attention.py:718-899
 * with the semantics of its oracle ref_ragged_paged_attention (:73-148):
 * causal (query j of a sequence sits at kv position kv_len - q_len + j),
 * GQA kv_head = q_head / (Hq / Hkv), fp32 softmax and accumulation.
 *
 * kv_scales: NULL, or fp32 [total_pages, num_kv_heads, 2] per-(page, kv head)
 *   K and V dequantisation scales (an extension of the reference's scalar
 *   k_scale / v_scale, :124-129); dequantised K = bf16(float(k) * scale).
 * Rows of `out` at or past cu_q_lens[num_seqs] are written as zeros.
 * Stream-ordered and asynchronous; no host synchronisation inside.
 * Metadata is range-checked on the device, and an out-of-range value is never
 * dereferenced: a page id outside [0, total_pages) is replaced by page 0 (the
 * rows that read it hold values computed from page 0's keys, i.e. garbage), a
 * query range outside [0, num_tokens) makes its sequence contribute no rows
 * (left unwritten), kv_len is clamped to pages_per_seq * page_size, and a bit
 * of the error word is set (rpa_read_error_word).  A caller that cannot rule
 * out bad metadata must read the error word and discard the output when it is
 * nonzero; the reference instead rejects such metadata on the host before any
 * launch (ragged_paged_attention.py:152-212, rpa_lowering.py:71-128), which is
 * what the Python wrapper does. */
int rpa_ragged_paged_attention(const rpa_shape_t* shape, const rpa_options_t* options,
                               const void* q, const void* kv_pages, const float* kv_scales,
                               const int32_t* kv_lens, const int32_t* page_indices,
                               const int32_t* cu_q_lens, const int32_t* num_seqs,
                               void* out, void* workspace, size_t workspace_bytes,
                               void* stream);

/* Measurement hook: rpa_ragged_paged_attention, additionally recording the
 * caller's hipEvent_t event_begin / event_end on `stream` immediately before
 * and after the attention kernel (not the split-K combine that follows it),
 * so a caller can time the dominant kernel alone.  No counterpart in the reference (its runner
 * reads per-kernel device time from XProf, src/tpu_cake/rpa_bundle.py:114-139). */
int rpa_ragged_paged_attention_timed(const rpa_shape_t* shape, const rpa_options_t* options,
                                     const void* q, const void* kv_pages, const float* kv_scales,
                                     const int32_t* kv_lens, const int32_t* page_indices,
                                     const int32_t* cu_q_lens, const int32_t* num_seqs, void* out,
                                     void* workspace, size_t workspace_bytes, void* stream,
                                     void* event_begin, void* event_end);

/* Allocation-free variant of rpa_ragged_paged_attention.  No counterpart in the reference: it is
 * for callers that cannot allocate or pass device memory -- code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  Same arguments, kernels and results (bitwise)
 * as rpa_ragged_paged_attention, minus the workspace: that lives in a file-scope device array of
 * 128 MiB which each GPU the library is loaded on holds until the process ends.  The call allocates
 * nothing (no hipMalloc / hipFree); on its first call on a device it resolves that device's copy
 * of the array and clears its header with a fill kernel on `stream`, so that first call must not
 * be under graph capture (RPA_E_INVALID; later calls may be).  Returns RPA_E_WORKSPACE if
 * the device needs more workspace than the array holds (more than 320 compute units).  Every call
 * on a GPU shares that GPU's array: calls that overlap in time on one GPU (other streams, other
 * threads) race and must be ordered by the caller.  The device error word of these calls lives in
 * the array and is not readable; callers validate metadata on the host. */
int rpa_ragged_paged_attention_noalloc(const rpa_shape_t* shape, const rpa_options_t* options,
                                       const void* q, const void* kv_pages, const float* kv_scales,
                                       const int32_t* kv_lens, const int32_t* page_indices,
                                       const int32_t* cu_q_lens, const int32_t* num_seqs, void* out,
                                       void* stream);

/* Gather probe: copies every (sequence, token < kv_len) K/V row the attention
 * kernel reads, in logical order, into dense [sum(kv_lens), 2*Hkv, head_dim]
 * (same element type as kv_pages).  Uses the attention kernel's page-address
 * function; restates the gather of MultiPageAsyncCopyDescriptor
 * (ragged_paged_attention.py:35-70).  Row offsets are the exclusive prefix
 * sum of kv_lens over the first num_seqs sequences. */
int rpa_gather_kv(const rpa_shape_t* shape, const void* kv_pages, const int32_t* kv_lens,
                  const int32_t* page_indices, const int32_t* num_seqs, void* dense_out,
                  int64_t dense_rows, void* workspace, size_t workspace_bytes, void* stream);

/* Copies the workspace error word to *host_word (synchronous on `stream`).
 * Bit 0: page id out of [0, total_pages); bit 1: query row out of
 * [0, num_tokens); bit 2: kv_len clamped to pages_per_seq * page_size;
 * bit 3: a sequence with q_len > kv_len (its uncovered rows are left unwritten). */
int rpa_read_error_word(const void* workspace, size_t workspace_bytes, int32_t* host_word,
                        void* stream);

/* Diagnostic, with no counterpart in the reference: the attention kernel's per-workgroup
 * timeline of the last launch, for a library built with -DRPA_TIMELINE (the variant
 * `python -m tpu_cake_amd.timeline` builds); the product library returns RPA_E_UNSUPPORTED.
 * Synchronises `stream`, then copies rows 0 .. rows-1 (workgroup b = row b, rows <= 8192),
 * 16 int64 fields each: stamps of the 100 MHz constant clock at kernel entry, work split known,
 * first stream-K loads issued, stream-K range done, prefill-tile role entered, tile order ready,
 * kernel exit; the role bits (1 prefill-first, 2 stream-K range, 4 tiles joined after it);
 * stream-K units; prefill tiles and their 32-key chunk steps; clock ticks summed over the tiles
 * in queue fetches, tile set-up, chunk-step loops and row writes; XCC_ID << 32 | HW_ID. */
int rpa_timeline_read(int64_t* host_rows, int32_t rows, void* stream);

/* ---------------------------------------------------------------------------------------
 * Fused Inkling decode (v3 semantics): write each sequence's new K/V token into the paged
 * cache, then attend over the updated cache with an additive relative-position bias.
 * Replaces FusedRpaPlan.invoke / run_preflighted (src/tpu_cake/rpa_lowering.py:232-288) over
 * the fused kernel whose semantics the reference pins in inkling_fused_rpa_reference
 * (src/tpu_cake/workloads/inkling_rpa.py:471-589):
 *   * decode only: one query token per sequence (cu_q_lens = 0..B, distribution = (B, B, B));
 *   * sequence s's pages are page_indices[cu_kv_lens[s] / S ...] (cu_kv_lens page-aligned);
 *   * K of kv head h goes to combined row 2h, V to 2h+1, at slot (kv_len-1) % S of page
 *     page_indices[cu_kv_lens[s]/S + (kv_len-1)/S]; rows are zero-padded to cache_width;
 *   * score = (q . k) * sm_scale + relative_states[s,h,:] . relative_projection[:, d]
 *     for distances d = kv_len-1-key < relative_extent (else no bias); fp32 softmax.
 * The cache is updated in place (the reference aliases it to an output).  Metadata must have
 * passed the reference's preflight (rpa_lowering.py:71-128; the Python wrapper runs it);
 * the device still range-checks what it dereferences (error word).  cu_q_lens and
 * distribution are part of the reference's input list and are validated by that preflight;
 * the device does not read them.  head_dim <= cache_width = 128.
 * With head_dim a multiple of 8 in [32, 128], 16-byte aligned tensors, P * S < 2^31 and R in
 * {0, 16} with E a multiple of 8 -- any page size -- the step is one attention launch (new token
 * read from keys/values, bias formed in the kernel) plus the merge launch, which also stores the
 * token; other shapes take a preparation launch first (cache write, page table, bias table).
 * --------------------------------------------------------------------------------------- */
typedef struct rpa_fused_shape {
  int32_t num_seqs;          /* B */
  int32_t num_q_heads;       /* Hq */
  int32_t num_kv_heads;      /* Hkv */
  int32_t head_dim;          /* D: width of queries, new K/V and the output (<= cache_width) */
  int32_t total_pages;       /* P */
  int32_t page_size;         /* S */
  int32_t cache_width;       /* padded row width of the cache (128) */
  int32_t page_entries;      /* length of the flat page_indices list */
  int32_t pages_per_seq;     /* max over sequences of ceil(kv_len / S) */
  int32_t relative_dim;      /* R in [0, 256] (0: no relative bias) */
  int32_t relative_extent;   /* E in [1, 2^24] when R > 0; B * Hq * (E + 63) must stay below 2^31 */
} rpa_fused_shape_t;

/* Workspace bytes for rpa_inkling_fused_decode on the current device (0 on a bad shape). */
size_t rpa_fused_workspace_size(const rpa_fused_shape_t* shape);

/* queries bf16 [B, Hq, D]; keys, values bf16 [B, Hkv, D] (the new token); cache bf16
 * [P, S, 2*Hkv, cache_width] (the reference's [P, S, 2*Hkv/packing, packing, width]);
 * kv_lens int32 [B] (including the new token); page_indices int32 [page_entries];
 * cu_q_lens int32 [B+1]; cu_kv_lens int32 [B+1]; distribution int32 [3];
 * relative_states bf16 [B, Hq, R]; relative_projection bf16 [R, E] (both NULL when R = 0);
 * out bf16 [B, Hq, D].  The workspace is initialised with rpa_workspace_init like the
 * operator's. */
int rpa_inkling_fused_decode(const rpa_fused_shape_t* shape, float sm_scale, const void* queries,
                             const void* keys, const void* values, void* cache, const int32_t* kv_lens,
                             const int32_t* page_indices, const int32_t* cu_q_lens, const int32_t* cu_kv_lens,
                             const int32_t* distribution, const void* relative_states,
                             const void* relative_projection, void* out, void* workspace,
                             size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------
 * Inkling decode, v1 contract: the workload the reference renders as `experiment inkling-rpa`
 * (src/tpu_cake/workloads/inkling_rpa.py:87-143, contract :693-723) with the semantics of its
 * numpy oracle inkling_rpa_reference (:37-73), executed here:
 *   out[b, h] = softmax_l( q[b, h] . k[l, h/G] * sm_scale + bias[h, l] ) @ v[l, h/G]
 * over the keys l < sequence_lengths[b] of pages page_table[b, :]; the oracle's scale is 1/D.
 * Separate key and value caches; bias indexed by key position (bias_len >= every length).
 * The reference's `experiment inkling-rpa` renders the experiment artifact for this workload
 * (cli.py:667-676); this entry executes it.  The caches are packed into the operator's
 * combined layout in the workspace on every call (a copy of the whole cache: this entry serves
 * the contract's shapes; a serving cache belongs in the combined layout of
 * rpa_ragged_paged_attention).
 * --------------------------------------------------------------------------------------- */
typedef struct rpa_inkling_shape {
  int32_t num_seqs;       /* B */
  int32_t num_q_heads;    /* H */
  int32_t num_kv_heads;   /* Hkv: key and value heads (H % Hkv == 0) */
  int32_t head_dim;       /* D <= 128 (queries, keys, values, output) */
  int32_t total_pages;    /* P */
  int32_t page_size;      /* S */
  int32_t pages_per_seq;  /* MP: page_table row length */
  int32_t bias_len;       /* L: bias columns, in [1, 2^24] */
} rpa_inkling_shape_t;

/* Workspace bytes for rpa_inkling_decode on the current device (0 on a bad shape). */
size_t rpa_inkling_workspace_size(const rpa_inkling_shape_t* shape);

/* query bf16 [B, H, D]; key_cache, value_cache bf16 [P, S, Hkv, D]; page_table int32 [B, MP];
 * sequence_lengths int32 [B] (each in [1, min(MP * S, L)]); bias bf16 [H, L]; out bf16 [B, H, D].
 * The workspace is initialised with rpa_workspace_init like the operator's. */
int rpa_inkling_decode(const rpa_inkling_shape_t* shape, float sm_scale, const void* query, const void* key_cache,
                       const void* value_cache, const int32_t* page_table, const int32_t* sequence_lengths,
                       const void* bias, void* out, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RPA_H_ */
