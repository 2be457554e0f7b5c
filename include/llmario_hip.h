/*
 * llmario_hip.h — C ABI of the MI355X-native paged-KV attention backend.
 *
 * The drop-in boundary for the attention / KV-cache part of LLMario's `ModelBackend`
 * (crates/engine/model/src/backend.rs:17-106). A Rust `HipBackend` binds these symbols with an
 * `extern "C"` block. Plain C types only: fixed-width
 * integers, plain pointers and sizes, opaque handles. Device pointers are HIP device addresses;
 * `stream` is a `hipStream_t` passed as `void*` (NULL = the default stream).
 *
 * Status codes: every entry point returns int32_t LMH_* below. LMH_KV_FULL leaves all state as
 * it was and reports `needed`/`free` blocks through out-parameters. No C++ exception crosses this
 * boundary. A handle is single-threaded (the reference's `ModelBackend: Send`, not `Sync`), and
 * the device work of one handle must be stream-ordered: issue it on one stream, or order the
 * streams yourself.
 *
 * Page layout: blocks of `block_tokens` positions (any power of two, kv.rs:402-406), each holding
 * every layer's K then V for those positions, as the reference's block does (kv.rs:286-324,
 * 402-497), with the same bytes per block; inside a block each (layer, KV head) owns a contiguous
 * region. For the geometries with a matrix-core decode instance (f16 / bf16 head widths 32, 64, 96,
 * 128, 192, 256 and 192 / 128; q8_0 64, 128, 192, 256; f32 64, 128, 256) on blocks of at least 16
 * positions, its bytes are in the order the kernels' operands want them (one 16-byte load per lane
 * per operand chunk reads 1 KiB contiguous per wave); every other geometry the reference accepts
 * (any widths up to 512, q8_0 multiples of 32, hd != hdv, blocks under 16 positions) keeps
 * row-major rows in the reference's row encoding, read by a VALU kernel (as Metal's
 * attn_vec_generic covers widths off its instances). Block ids, reference counts and the LRU free
 * queue follow BlockPool (kv/src/lib.rs:36-176), so block tables and page indices match the
 * reference bit for bit.
 */
#ifndef LLMARIO_HIP_H
#define LLMARIO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LMH_ABI_VERSION 3u

/* status codes */
#define LMH_OK 0
#define LMH_INVALID_ARGUMENT 1
#define LMH_KV_FULL 2
#define LMH_UNSUPPORTED 3
#define LMH_DEVICE_ERROR 4
#define LMH_OUT_OF_MEMORY 5

/* KvType (kv.rs:56-63) plus two declared extensions (F32, BF16) the configurations need. */
#define LMH_KV_F16 0u
#define LMH_KV_Q8_0 1u
#define LMH_KV_F32 2u
#define LMH_KV_BF16 3u

typedef struct lmh_kv lmh_kv; /* opaque: the device page pool + host block bookkeeping */

/* Per attention layer geometry: AttnGeom (model/src/arch.rs:73-95) restricted to what the cache
 * and the kernels read. A sliding-window layer (`window` > 0, the reference's `AttnGeom::window`)
 * keeps its rows in the window pool (metal/src/kv.rs:13-17, 37-47): blocks addressed by absolute
 * block number, each released once every position in it is at least `window` behind the
 * sequence's next token. All window layers share one width; at least one layer is not windowed. */
typedef struct lmh_layer_desc {
  uint32_t n_head;
  uint32_t n_kv;
  uint32_t hd;
  uint32_t hdv;
  uint32_t window;      /* sliding-window width (0 = full attention, in the paged blocks) */
  uint32_t reserved0;
} lmh_layer_desc;

/* KvOptions (kv.rs:328-375). */
typedef struct lmh_kv_options {
  uint32_t abi_version; /* LMH_ABI_VERSION */
  uint32_t kv_type;     /* LMH_KV_* */
  uint32_t block_tokens;
  uint32_t n_layers;
  const lmh_layer_desc* layers;
  uint64_t max_ctx;
  uint64_t n_seqs;
  uint64_t pool_tokens; /* 0 = None: every sequence can hold max_ctx at once */
  int32_t device;       /* HIP device ordinal */
  uint32_t n_batch;     /* most positions one call appends to one sequence: sizes the window pool
                           (metal/src/kv.rs:130-133); 0 = 512, the plan's default n_batch */
} lmh_kv_options;

/* KvLayout (kv.rs:377-400): sizes are the reference's for the same options. */
typedef struct lmh_layout_info {
  uint64_t block_bytes;
  uint64_t blocks_per_seq;
  uint64_t n_seqs;
  uint64_t pool_blocks;
  uint64_t max_ctx;
  uint32_t block_tokens;
  uint32_t kv_type;
} lmh_layout_info;

/* SeqTokens (forward.rs:31-35): the attention level needs the count, not the token ids. */
typedef struct lmh_seq_tokens {
  uint64_t seq;
  uint64_t n_tokens;
} lmh_seq_tokens;

/* Seg (forward.rs:37-47): rows start..start+n of the stacked batch belong to `seq` and sit at
 * positions pos0..pos0+n. */
typedef struct lmh_seg {
  uint64_t seq;
  uint64_t start;
  uint64_t n;
  uint64_t pos0;
} lmh_seg;

/* ---- handle lifetime (KvCache::with_options, kv.rs:577-603; MetalKv::new, metal/src/kv.rs:66-100) */
int32_t lmh_kv_create(const lmh_kv_options* opt, lmh_kv** out);
void lmh_kv_destroy(lmh_kv* kv);
/* Message of the last failed call on this handle ("" if none). */
const char* lmh_kv_last_error(const lmh_kv* kv);
/* Message of the last lmh_kv_create failure on this thread. */
const char* lmh_create_error(void);
int32_t lmh_kv_layout(const lmh_kv* kv, lmh_layout_info* out);
/* Layout hash for snapshots, tagged "hip" (KvCache::fingerprint, kv.rs:983-999). */
uint64_t lmh_kv_fingerprint(const lmh_kv* kv);

/* ---- sequence bookkeeping (KvCache, kv.rs:640-827; ModelBackend, backend.rs:24-48) ---- */
int32_t lmh_kv_seq_len(const lmh_kv* kv, uint64_t seq, uint64_t* len);
/* Set a sequence's cached length directly (the reference tests write `seq_mut(s).len`). */
int32_t lmh_kv_set_seq_len(lmh_kv* kv, uint64_t seq, uint64_t len);
int32_t lmh_kv_free_blocks(const lmh_kv* kv, uint64_t* free_blocks);
int32_t lmh_kv_resident_blocks(const lmh_kv* kv, uint64_t* n);
int32_t lmh_kv_blocks_needed(const lmh_kv* kv, uint64_t seq, uint64_t new_len, uint64_t* needed);
int32_t lmh_kv_reserve(lmh_kv* kv, uint64_t seq, uint64_t new_len, uint64_t* needed, uint64_t* free_blocks);
int32_t lmh_kv_truncate(lmh_kv* kv, uint64_t seq, uint64_t n);
int32_t lmh_kv_clear(lmh_kv* kv, uint64_t seq);
/* The sequence's block table (BlockTable::locate, kv/src/lib.rs:243-253): writes up to `cap`
 * ids, returns the count in *n. */
int32_t lmh_kv_block_table(const lmh_kv* kv, uint64_t seq, uint32_t* out, uint64_t cap, uint64_t* n);
/* The window pool (present when a layer has a window): its width, block bytes, blocks and free
 * blocks; and a sequence's window blocks by absolute block number (-1: released or never taken). */
typedef struct lmh_window_info {
  uint64_t window;
  uint64_t block_bytes;
  uint64_t pool_blocks;
  uint64_t free_blocks;
} lmh_window_info;
int32_t lmh_kv_window_info(const lmh_kv* kv, lmh_window_info* out);
int32_t lmh_kv_window_table(const lmh_kv* kv, uint64_t seq, int32_t* out, uint64_t cap, uint64_t* n);
/* Test and benchmark hook: give an empty sequence exactly these free blocks, in order (e.g. a
 * seeded permutation of the pool), as if reserve had handed them out. */
int32_t lmh_kv_adopt_blocks(lmh_kv* kv, uint64_t seq, const uint32_t* blocks, uint64_t n);
/* ---- snapshots (KvCache::snapshot_bytes / write_seq / read_seq, kv.rs:1009-1130; the disk tier,
 * server/src/kvtier.rs) ----
 * A sequence's state is its first ceil(len / block_tokens) blocks in the reference's block format
 * (per layer K rows then V rows, each in the reference's row encoding), so a snapshot is
 * byte-identical to the one the reference's CPU cache writes for the same contents (stale slots
 * past len included). Pair snapshots with lmh_kv_fingerprint, as the reference does. */
int32_t lmh_kv_snapshot_bytes(const lmh_kv* kv, uint64_t len, uint64_t* bytes);
/* ModelBackend::snapshot_trimmable (backend.rs:64; CPU kv.rs:1003-1007, Metal
 * metal/src/backend.rs:2141-2143): whether a restored snapshot can be cut back to a shorter prefix
 * (*trimmable = 1): true for a cache of plain paged layers, false when it has window layers (their
 * blocks behind the window are released, so a shorter prefix may need rows that are gone). */
int32_t lmh_kv_snapshot_trimmable(const lmh_kv* kv, int32_t* trimmable);
/* Writes snapshot_bytes(len(seq)) bytes to `dst` (device memory, `cap` bytes); *written = size. */
int32_t lmh_kv_write_seq(lmh_kv* kv, uint64_t seq, void* dst, uint64_t cap, uint64_t* written, void* stream);
/* Replaces the sequence with `len` tokens of snapshot `src` (device memory, n_bytes ==
 * snapshot_bytes(len)). The sequence's own unshared blocks count as free; without room it fails
 * with LMH_KV_FULL (needed / free reported) and nothing changes. */
int32_t lmh_kv_read_seq(lmh_kv* kv, uint64_t seq, uint64_t len, const void* src, uint64_t n_bytes,
                        uint64_t* needed, uint64_t* free_blocks, void* stream);
/* BlockPool per-block state (kv/src/lib.rs:146-167) and prefix-cache hooks (lib.rs:112-143). */
int32_t lmh_pool_refs(const lmh_kv* kv, uint32_t block, uint32_t* refs);
int32_t lmh_pool_set_hash(lmh_kv* kv, uint32_t block, const uint8_t hash[32]);
int32_t lmh_pool_clear_hash(lmh_kv* kv, uint32_t block);
int32_t lmh_pool_is_cached(const lmh_kv* kv, uint32_t block, int32_t* cached);

/* ---- batch hand-off (Model::forward_batch, forward.rs:207-291) ----
 * Validates the batch (non-empty, at most n_seqs entries, no sequence twice, no empty entry, no
 * context overflow), reserves every entry's room all-or-nothing (LMH_KV_FULL changes nothing),
 * and writes one lmh_seg per entry in batch order (the stacked row order the caller's q/out
 * arrays use). `segs_out` holds n entries. Lengths do not move until lmh_batch_commit. */
int32_t lmh_batch_prepare(lmh_kv* kv, const lmh_seq_tokens* batch, uint64_t n, lmh_seg* segs_out,
                          uint64_t* n_rows, uint64_t* needed, uint64_t* free_blocks);
/* run_layers' tail (forward.rs:363-366): every segment's sequence grows by its row count. */
int32_t lmh_batch_commit(lmh_kv* kv, const lmh_seg* segs, uint64_t n_segs);

/* ---- device work (all enqueued on `stream`) ---- */
/* KvCache::store_k/store_v (kv.rs:870-889) for every row of the segments: k is
 * [n_rows][n_kv*hd] f32, v is [n_rows][n_kv*hdv] f32 (device), encoded to the cache type
 * (f16/bf16 round to nearest even; q8_0 as quantize_q8_0, kv.rs:156-171). */
int32_t lmh_kv_store(lmh_kv* kv, uint32_t layer, const lmh_seg* segs, uint64_t n_segs, const float* k,
                     const float* v, void* stream);
/* The same rows given already encoded, in the reference's row format (KvType::store output:
 * f16/bf16 bits, f32, or q8_0 34-byte blocks): k is [n_rows][k_row] bytes, v [n_rows][v_row]. */
int32_t lmh_kv_store_encoded(lmh_kv* kv, uint32_t layer, const lmh_seg* segs, uint64_t n_segs,
                             const void* k_rows, const void* v_rows, void* stream);
/* Parity hooks: read rows back (LayerReader::row, kv.rs:1166-1179), decoded to f32 ... */
int32_t lmh_kv_gather(lmh_kv* kv, uint32_t layer, const lmh_seg* segs, uint64_t n_segs, float* k_out,
                      float* v_out, void* stream);
/* ... or in the reference's row encoding, byte for byte. */
int32_t lmh_kv_gather_encoded(lmh_kv* kv, uint32_t layer, const lmh_seg* segs, uint64_t n_segs,
                              void* k_rows, void* v_rows, void* stream);

/* The producer side of the cache, fused: attention_block's per-row tail (forward.rs:427-453;
 * the Metal sibling is qk_rope_kv_t, misc.metal:195-273). For every row t (sequence, position pos)
 * of the segments, per head:
 *   Q heads: optional per-head RMS norm with weight q_norm (per_head_norm, forward.rs:832-838 over
 *            rms_norm, cpu/src/ops.rs:18-29), then RoPE at pos (rope, ops.rs:46-66), written to
 *            q_out [n_rows][n_head][hd] f32;
 *   K heads: the same with k_norm, then stored into the cache at (seq, pos) like lmh_kv_store;
 *   V heads: optionally a weightless RMS norm (Metal's v_norm, misc.metal:218-226), then stored.
 * q_in is [n_rows][n_head][q_stride] f32 (q_stride >= hd; the first hd values of each head are
 * used), k_in [n_rows][n_kv][hd], v_in [n_rows][n_kv][hdv] (device). RoPE: pairs i < rot_dim/2,
 * (2i, 2i+1) (Normal) or (i, i + rot_dim/2) (Neox), freq = theta^(-2i/rot_dim) in f32 as the
 * reference computes it, angle = pos * freq_scale * freq (/ freq_div[i] when given: Metal's
 * per-pair divisors), rotation scaled by attn_factor. q_out may not alias the inputs. The layer
 * must have hd == hdv <= 512 (LMH_UNSUPPORTED otherwise); q_stride is a multiple of 4 and the
 * four arrays are 16-byte aligned (LMH_INVALID_ARGUMENT otherwise). */
#define LMH_ROPE_Q_NORM 1u   /* q_norm weights given: RMS-norm each Q head */
#define LMH_ROPE_K_NORM 2u   /* k_norm weights given: RMS-norm each K head */
#define LMH_ROPE_V_NORM 4u   /* weightless RMS norm of each V head */
#define LMH_ROPE_APPLY 8u    /* rotate (clear on NoPE layers) */
#define LMH_ROPE_NEOX 16u    /* pair (i, i + rot_dim/2) instead of (2i, 2i+1) */
typedef struct lmh_rope_params {
  uint32_t abi_version;   /* LMH_ABI_VERSION */
  uint32_t flags;         /* LMH_ROPE_* */
  uint32_t rot_dim;       /* rotated dimensions: even, <= hd */
  uint32_t q_stride;      /* floats between consecutive Q heads of a row in q_in (0 = hd) */
  float eps;              /* RMS-norm epsilon */
  float theta;
  float freq_scale;       /* linear position scale (1 = none) */
  float attn_factor;      /* scale of the rotated values (1 = none) */
  const float* q_norm;    /* device [hd] (LMH_ROPE_Q_NORM) */
  const float* k_norm;    /* device [hd] (LMH_ROPE_K_NORM) */
  const float* freq_div;  /* device [rot_dim/2] per-pair angle divisors, or NULL */
} lmh_rope_params;
int32_t lmh_qk_rope_store(lmh_kv* kv, uint32_t layer, const lmh_seg* segs, uint64_t n_segs,
                          const float* q_in, const float* k_in, const float* v_in, float* q_out,
                          const lmh_rope_params* params, void* stream);

/* attend (forward.rs:585-678) + attend_split (forward.rs:688-807) in one call: every row t of
 * the segments (sequence segs[i].seq, position pos0+j) attends causally to positions
 * p_lo..=pos of its own sequence (p_lo = pos+1-window when window > 0 and pos+1 > window, else 0),
 * softmax(scale * q.K) V per query head with GQA head kvh = h / (n_head / n_kv); fp32
 * accumulation. q is [n_rows][n_head][hd] f32, out is [n_rows][n_head][hdv] f32 (device).
 * Decode rows, split-K over pages and prefill tiles are packed into one work list: segments of at
 * least prefill_min_rows rows on f16, bf16 or q8_0 pages of head width 64 or 128 (hd = hdv) run on
 * the matrix-core prefill kernel (Metal's attn_prefill_hd{64,128}[_q8_0], backend.rs:563-569); the
 * other rows on the decode kernels. A stream under graph capture is refused with LMH_UNSUPPORTED
 * before anything is enqueued: the call's work list sits in a staging slot that later calls reuse,
 * which a replayed graph would read. */
int32_t lmh_attend(lmh_kv* kv, uint32_t layer, const lmh_seg* segs, uint64_t n_segs, const float* q,
                   float* out, float scale, uint64_t window, void* stream);

/* lmh_attend for callers that cannot allocate (tight serving loops, harnesses that forbid
 * allocation); no counterpart in the reference. Same arguments, results and errors as lmh_attend
 * (graph capture refused likewise), and it allocates nothing: no device, pinned or event
 * allocation (the staging slots and their events are made at lmh_kv_create). It may wait for an
 * earlier call's kernels before reusing the staging slot they read. Split-K
 * partials and the merge list live in a file-scope device array of 32 MiB per GPU, held until the
 * process ends (its address is resolved once per device when a handle is created there): the
 * split count is capped to what it holds, and a call that still needs more split-K scratch, or
 * whose work list exceeds the staging capacity reserved at lmh_kv_create (1 MiB per slot: ~32 K
 * decode items), fails with LMH_INVALID_ARGUMENT and a message naming both sizes. Nothing in the
 * scratch must start at zero (every partial is written before it is read). Every call on one GPU
 * shares its array, which keeps the last call's contents: calls that overlap on one GPU (other
 * streams or other handles on the same device) race; issue them in order on one stream. The
 * timing hook records nothing for these calls. */
int32_t lmh_attend_noalloc(lmh_kv* kv, uint32_t layer, const lmh_seg* segs, uint64_t n_segs,
                           const float* q, float* out, float scale, uint64_t window, void* stream);

/* Handle options of lmh_attend's planning and precision (no counterpart in the reference, whose
 * CPU path has no such choices; its thread-count split rule is forward.rs:613-633). Set once or
 * between calls; a zero field selects the default (lmh_kv_get_tuning returns the fields as set, so
 * reading the options and writing them back changes nothing).
 *   prefill_p_f16: 1 = the prefill products take P rounded to f16, the precision of Metal's
 *     attn_prefill (attn_prefill.metal: half P); 0 (default) = P as f16 hi + lo parts (~22 bits,
 *     the CPU path's f32 weights to within the 2e-3 bound even on rows whose output cancels).
 *     Applies to f16 / bf16 pages: q8_0 prompts always carry their scaled weights as bf16 hi + lo.
 *   prefill_min_rows: segments of at least this many rows go to the matrix-core prefill kernel
 *     (default 8, as Metal routes prompts of 8 tokens or more to its flash prefill; 1 .. 2^32).
 *   decode_target_items: split-K target of decode work items (default: half the items the device
 *     holds at once, from the occupancy query, for the matrix-core decode kernel; all of them for
 *     f32 and row-layout layers).
 *   decode_min_tiles: smallest split-K chunk in 16-key tiles (default 8; 2 for f32 pages; 4 for
 *     row-layout layers; 1 .. 64).
 *   prefill_whole_units: 1 = prefill units always run whole; 0 (default) = when whole units would
 *     leave the device unbalanced (few, long units), their key ranges are cut into pieces spread over
 *     the workgroups, whose partial results a merge launch combines (heads per KV group <= 16).
 *   prefill_q_split: how the f16 / bf16 prefill launch takes a Q with bits below the page type
 *     (Q as f16 hi + lo parts either way, results within the same bound): 1 = the launch for
 *     exact Q, whose units with such bits run two passes of half their columns; 2 = the launch
 *     whose every unit runs one pass with the hi + lo products (a Q exact in the page type runs
 *     slower there); 0 (default) = the second when the handle's previous prefill launch found
 *     such bits (each launch records it), else the first. q8_0 pages always take the first.
 * Out-of-range values fail with LMH_INVALID_ARGUMENT and change nothing. */
typedef struct lmh_attend_tuning {
  uint32_t abi_version;        /* LMH_ABI_VERSION */
  uint32_t prefill_p_f16;
  uint64_t prefill_min_rows;
  uint64_t decode_target_items;
  uint64_t decode_min_tiles;
  uint64_t prefill_workgroups;  /* cap on the prefill kernel's workgroups (0: every slot of the device);
                                   fewer workgroups run more units each */
  uint32_t prefill_whole_units;
  uint32_t prefill_q_split;     /* 0 (default), 1 or 2 */
} lmh_attend_tuning;
int32_t lmh_kv_set_tuning(lmh_kv* kv, const lmh_attend_tuning* t);
/* The options as set (0 = the default, which each call resolves). */
int32_t lmh_kv_get_tuning(const lmh_kv* kv, lmh_attend_tuning* t);

/* Timing hook for benchmarks: when enabled, lmh_attend and lmh_qk_rope_store time each kernel
 * they launch with a HIP event pair that the kernel's own dispatch records (hipExtLaunchKernel: the
 * kernel alone), and the snapshot calls bracket their kernels with HIP events on `stream`;
 * lmh_kv_kernel_time returns the accumulated milliseconds and launch count of one kernel kind
 * since its last read, and resets them (it waits for the recorded events). */
#define LMH_KERNEL_DECODE 0u
#define LMH_KERNEL_PREFILL 1u
#define LMH_KERNEL_MERGE 2u
#define LMH_KERNEL_ROPE_STORE 3u /* lmh_qk_rope_store's kernel */
#define LMH_KERNEL_SNAPSHOT 4u   /* lmh_kv_write_seq / lmh_kv_read_seq kernels */
#define LMH_KERNEL_MIXED 5u      /* lmh_attend's one launch for a call with both prefill units and decode rows */
int32_t lmh_kv_set_timing(lmh_kv* kv, int32_t enable);
int32_t lmh_kv_kernel_time(lmh_kv* kv, uint32_t kernel, double* ms, uint64_t* launches);

/* Benchmark hook (no counterpart in the reference; for benchmark drivers that report how far the
 * attention kernels are from what the device can stream): allocates `bytes` (rounded down to 16)
 * on `device`, reads them `iters` times with a plain streaming-read kernel, and returns the read
 * rate in GB/s over the launches' summed durations (events recorded by each dispatch, as
 * lmh_attend's kernels are timed). Synchronous; frees what it allocated. */
int32_t lmh_bench_read_ceiling(int32_t device, uint64_t bytes, uint32_t iters, double* gbps);

/* Test hook (no counterpart in the reference; for CPU tests of the planner, which run under the
 * sanitizers): lmh_attend's work-list planner on host data alone, no device touched. `d` gives a
 * layer geometry as lmh_kv_create takes it, the device facts the planner uses (n_cu; the decode
 * items the device holds at once, 0 = 8 per CU) and a block table [n_seqs][bps] (-1: no block);
 * the segments are validated as lmh_attend validates them (every block a row's key range
 * starts or ends in must be in the table). The plan lmh_attend would run is copied out as its
 * internal records: decode items, split-K merges and prefill units (pf_wg lists of pf_per_wg
 * units, an empty unit ending a list), `counts` giving the number of records and the uint32
 * words per record. Lists too small for the plan: LMH_INVALID_ARGUMENT with `counts` filled. */
typedef struct lmh_plan_desc {
  uint32_t abi_version;   /* LMH_ABI_VERSION */
  uint32_t kv_type;
  uint32_t n_head, n_kv, hd, hdv;
  uint32_t block_tokens;
  uint32_t n_cu;
  uint64_t decode_capacity;
  uint64_t n_seqs, bps;
  const int32_t* table;
  uint64_t window;
  float scale;
  uint32_t noalloc;       /* 1: plan as lmh_attend_noalloc does */
  lmh_attend_tuning tuning;
} lmh_plan_desc;
typedef struct lmh_plan_counts {
  uint64_t n_items, n_merges, n_units;
  uint32_t item_words, merge_words, unit_words;
  uint32_t ng, slots, pf_wg, pf_per_wg, max_pages;
  uint32_t local;   /* 0, or the waves per workgroup inside which split decode rows merge (8 for f32
                       pages and beside prefill units, 4 for the matrix-core decode launch) */
  uint32_t layout;
  uint32_t chunk;   /* decode split chunk in 16-key tiles */
} lmh_plan_counts;
int32_t lmh_plan_attend(const lmh_plan_desc* d, const lmh_seg* segs, uint64_t n_segs, uint32_t* items,
                        uint64_t items_cap, uint32_t* merges, uint64_t merges_cap, uint32_t* units,
                        uint64_t units_cap, lmh_plan_counts* counts);

/* ---- request scheduler: the host side of the batch hand-off ----
 * Scheduler (crates/engine/sched/src/lib.rs:75-282) over the block pool, with Sequence
 * (kv/src/lib.rs:262-335) for admission. Each step takes every decoding slot's next token, then
 * prompt chunks of the prefilling slots, both in (priority descending, arrival) order, up to
 * token_budget tokens. Admission reserves blocks for the prompt plus ceil(max_new *
 * conservativeness) tokens, reclaiming cached prefix blocks by their SHA-256 chain hash; when the
 * pool is short a request retracts the lowest-priority, youngest running slot of strictly lower
 * priority, which goes back to the queue head; with nothing to retract the request is queued.
 *
 * Standalone (kv NULL at creation): the scheduler owns BlockPool::new(n_blocks, block_tokens).
 * Bound (kv given): it shares the handle's pool (n_blocks and block_tokens are the handle's);
 * every admitted slot holds one empty sequence slot of the handle, whose block table becomes the
 * slot's reserved blocks and whose length starts at the slot's cached tokens, and a reservation
 * is capped at max_ctx positions. lmh_sched_prepare turns a step into lmh_batch_prepare's batch.
 * A scheduler is single-threaded and, when bound, used from the handle's thread. */
#define LMH_PRIORITY_BATCH 0u       /* Priority (sched/src/lib.rs:19-24) */
#define LMH_PRIORITY_API 1u
#define LMH_PRIORITY_INTERACTIVE 2u

typedef struct lmh_sched lmh_sched;

/* Scheduler::new (sched/src/lib.rs:89-101) plus the CacheKey (kv/src/lib.rs:189-197) every block
 * hash covers. Strings are NUL-terminated (NULL = empty); byte fields are pointer + length. */
typedef struct lmh_sched_options {
  uint32_t abi_version;      /* LMH_ABI_VERSION */
  uint32_t max_slots;        /* clamped to >= 1; bound: at most the handle's n_seqs */
  uint64_t token_budget;     /* clamped to >= 1 */
  double conservativeness;   /* multiplier on max_new when reserving (the reference starts at 1.0) */
  uint64_t n_blocks;         /* standalone pool size */
  uint32_t block_tokens;     /* standalone pool block size (> 0) */
  uint32_t reserved0;
  const uint8_t* model_digest;
  uint64_t model_digest_len;
  const char* kv_types;
  const char* rope_params;
  const char* template_hash;
  const uint8_t* salt;       /* per-client salt: different salts never share blocks */
  uint64_t salt_len;
} lmh_sched_options;

/* Request (sched/src/lib.rs:58-62). The prompt is copied. */
typedef struct lmh_request {
  const uint32_t* prompt;
  uint64_t n_prompt;
  uint64_t max_new;
  uint32_t priority;         /* LMH_PRIORITY_* */
  uint32_t reserved0;
} lmh_request;

/* Admission (sched/src/lib.rs:65-73): Admitted { slot, cached_tokens, retracted } or Queued. */
typedef struct lmh_admission {
  uint32_t admitted;         /* 1 = admitted, 0 = queued */
  uint32_t slot;
  uint64_t cached_tokens;    /* prompt tokens already in the cache (< the prompt length) */
  uint64_t n_retracted;      /* slots retracted, in order; the first `cap` ids are written */
} lmh_admission;

/* Step (sched/src/lib.rs:48-55). The caller owns both arrays; lmh_sched_next_step fills at most
 * max_slots entries of each. */
typedef struct lmh_prefill_range {
  uint32_t slot;
  uint32_t reserved0;
  uint64_t start;            /* prompt[start..end] is prefilled this step */
  uint64_t end;
} lmh_prefill_range;
typedef struct lmh_step {
  uint32_t* decodes;
  uint64_t n_decodes;
  lmh_prefill_range* prefills;
  uint64_t n_prefills;
  uint64_t tokens;
} lmh_step;

/* Slot (sched/src/lib.rs:34-45). */
typedef struct lmh_slot_info {
  uint32_t id;
  uint32_t priority;
  uint32_t decoding;         /* SlotState::Decoding (1) or Prefilling { done } (0) */
  uint32_t reserved0;
  uint64_t done;             /* prompt tokens prefilled */
  uint64_t n_prompt;
  uint64_t max_new;
  uint64_t generated;
  uint64_t seq_no;           /* arrival order */
  uint64_t kv_seq;           /* bound: the handle's sequence slot; standalone: UINT64_MAX */
  uint64_t n_blocks;         /* blocks in the slot's table */
} lmh_slot_info;

/* A queued request: (seq_no, Request) of the queue (sched/src/lib.rs:82). */
typedef struct lmh_queued_info {
  uint64_t seq_no;
  uint64_t n_prompt;
  uint64_t max_new;
  uint32_t priority;
  uint32_t reserved0;
} lmh_queued_info;

/* Scheduler counters plus PoolStats (kv/src/lib.rs:178-186) of the pool it admits from. */
typedef struct lmh_sched_stats {
  uint64_t slots, queued, retractions;
  uint64_t n_blocks, free, cached_free, hits, misses, evictions;
} lmh_sched_stats;

int32_t lmh_sched_create(const lmh_sched_options* opt, lmh_kv* kv, lmh_sched** out);
/* Bound: releases the blocks of every slot it still holds. A bound scheduler whose handle was
 * destroyed first fails every call with LMH_INVALID_ARGUMENT and can only be destroyed. */
void lmh_sched_destroy(lmh_sched* s);
const char* lmh_sched_last_error(const lmh_sched* s);
/* Scheduler::admit (sched/src/lib.rs:118-183). `retracted` holds `cap` ids (NULL when cap = 0);
 * max_slots entries always suffice. Bound: a prompt longer than max_ctx is LMH_INVALID_ARGUMENT. */
int32_t lmh_sched_admit(lmh_sched* s, const lmh_request* r, lmh_admission* out, uint32_t* retracted,
                        uint64_t cap);
/* Scheduler::drain_queue (sched/src/lib.rs:186-217): admits queued requests oldest first while
 * they fit; the first `cap` admitted slot ids are written, *n is the count. */
int32_t lmh_sched_drain_queue(lmh_sched* s, uint32_t* admitted, uint64_t cap, uint64_t* n);
/* Scheduler::next_step (sched/src/lib.rs:220-249). */
int32_t lmh_sched_next_step(const lmh_sched* s, lmh_step* step);
/* Scheduler::complete (sched/src/lib.rs:253-268): prefill cursors advance (a slot whose end
 * reaches its prompt length decodes from then on), each decode slot counts one generated token.
 * Unknown slot ids are skipped. */
int32_t lmh_sched_complete(lmh_sched* s, const lmh_step* step);
/* Scheduler::finish (sched/src/lib.rs:277-281): the slot leaves and its blocks return to the
 * pool (published blocks stay cached in the free queue). Unknown ids are a no-op. */
int32_t lmh_sched_finish(lmh_sched* s, uint32_t slot);
/* Sequence::publish (kv/src/lib.rs:320-328) for a slot: tokens[0..n] are the positions written so
 * far (tokens NULL: the slot's own prompt[0..n], n <= its length); every full block among them
 * gets its chain hash, so later admissions can reclaim it.
 * Bound: the full blocks must already be written (n / block_tokens * block_tokens <= the
 * sequence length), LMH_INVALID_ARGUMENT otherwise. */
int32_t lmh_sched_publish(lmh_sched* s, uint32_t slot, const uint32_t* tokens, uint64_t n);
/* Bound only: the step as a batch for lmh_batch_prepare, decodes first (one row each, so the
 * decode rows are one contiguous range at the top) then the prefill chunks, in step order; the
 * segments come back in that order with the handle's sequence ids. A prefill range must start at
 * its sequence's length. LMH_KV_FULL (a slot outgrew its reservation) changes nothing. After the
 * step's device work: lmh_batch_commit(kv, segs), then lmh_sched_complete. */
int32_t lmh_sched_prepare(lmh_sched* s, const lmh_step* step, lmh_seg* segs_out, uint64_t* n_rows,
                          uint64_t* needed, uint64_t* free_blocks);
int32_t lmh_sched_get_stats(const lmh_sched* s, lmh_sched_stats* out);
/* Running slot ids in admission order (the order next_step breaks ties by is seq_no). */
int32_t lmh_sched_slots(const lmh_sched* s, uint32_t* ids, uint64_t cap, uint64_t* n);
int32_t lmh_sched_slot(const lmh_sched* s, uint32_t slot, lmh_slot_info* out);
int32_t lmh_sched_slot_blocks(const lmh_sched* s, uint32_t slot, uint32_t* out, uint64_t cap, uint64_t* n);
int32_t lmh_sched_queued_at(const lmh_sched* s, uint64_t i, lmh_queued_info* out);
/* chain_hashes (kv/src/lib.rs:216-239): one 32-byte SHA-256 per full block of tokens, under the
 * CacheKey fields of `key` (other fields unused); `out` holds cap hashes, *n_hashes is the count. */
/* Test hook: SHA-256 of msg[0..n] (path -1: the path the library uses, 0: portable code, 1: the
 * x86 SHA extensions, LMH_UNSUPPORTED where the host lacks them). */
int32_t lmh_sha256(const uint8_t* msg, uint64_t n, int32_t path, uint8_t out[32]);
int32_t lmh_chain_hashes(const uint32_t* tokens, uint64_t n, uint32_t block_tokens, const lmh_sched_options* key,
                         uint8_t* out, uint64_t cap, uint64_t* n_hashes);

#ifdef __cplusplus
}
#endif
#endif /* LLMARIO_HIP_H */
