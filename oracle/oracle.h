/*
 * oracle.h — CPU restatement of LLMario's paged-KV attention path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker for the HIP path in
 * llmario_amd/. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it. The product never links, loads or calls it, and it is never the thing being measured
 * on the GPU.
 *
 * The reference is Rust (the crates/engine tree). No Rust toolchain exists in this image, so the
 * reference itself cannot be built (no oracle/_ref). Every function below restates one
 * reference function and cites it as path:line relative to the reference root.
 *
 * Parity pinning (how each part is checked independently of this restatement):
 *   codecs        — IEEE-754 binary16 / bfloat16 round-to-nearest-even closed forms, exhaustive
 *                   over all 65536 encodings (tests/test_oracle_codecs.py);
 *                   q8_0 known answers of kv.rs:1195-1247.
 *   layout, pool  — the reference unit tests' expectations, restated as known answers
 *                   (kv/src/lib.rs:351-460, forward.rs:1156-1221).
 *   attend        — naive float64 attention on the same decoded cache values, plus the reference
 *                   tests' invariants and the window known answer (gemma4.rs:925-1003).
 */
#ifndef LLMARIO_ORACLE_H
#define LLMARIO_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* KvType (kv.rs:56-63) with two declared extensions the configs need (F32, BF16). */
#define ORC_KV_F16 0
#define ORC_KV_Q8_0 1
#define ORC_KV_F32 2
#define ORC_KV_BF16 3

#define ORC_OK 0
#define ORC_KV_FULL 2
#define ORC_INVALID 1

/* ---- element codecs (kv.rs:104-184, core/src/dequant.rs:15-22) ---- */
uint16_t orc_f16_from_f32(float x);
float orc_f16_to_f32(uint16_t h);
uint16_t orc_bf16_from_f32(float x);
float orc_bf16_to_f32(uint16_t h);
void orc_f16_from_f32_n(const float* x, size_t n, uint16_t* out);
void orc_bf16_from_f32_n(const float* x, size_t n, uint16_t* out);
size_t orc_row_bytes(int kv_type, size_t n);
void orc_quantize_q8_0(const float* src, size_t n, uint8_t* dst);
void orc_dequantize_q8_0(const uint8_t* src, size_t n, float* out);
void orc_store_row(int kv_type, const float* src, size_t n, uint8_t* dst);
void orc_load_row(int kv_type, const uint8_t* src, size_t start, size_t len, float* out);

/* ---- layout (kv.rs:286-497), paged attention layers only ---- */
typedef struct orc_layer_geom {
  uint64_t n_head, n_kv, hd, hdv;
} orc_layer_geom;

typedef struct orc_options {
  uint64_t max_ctx;
  uint64_t n_seqs;
  uint64_t block_tokens;
  uint64_t pool_tokens; /* 0 = None */
  int32_t kv_type;
} orc_options;

typedef struct orc_layout_info {
  uint64_t block_bytes, blocks_per_seq, n_seqs, pool_blocks, max_ctx, block_tokens;
} orc_layout_info;

typedef struct orc_layer_info {
  uint64_t kv_dim, v_dim, k_row, v_row, k_base, v_base;
} orc_layer_info;

/* ---- BlockPool (kv/src/lib.rs:36-176) ---- */
typedef struct orc_pool orc_pool;
orc_pool* orc_pool_new(uint64_t n_blocks, uint64_t block_tokens, uint64_t block_bytes);
void orc_pool_free(orc_pool* p);
uint64_t orc_pool_free_blocks(const orc_pool* p);
int orc_pool_alloc(orc_pool* p, uint64_t n, uint32_t* out); /* 0 ok, ORC_KV_FULL if short */
void orc_pool_release(orc_pool* p, uint32_t b);
void orc_pool_set_hash(orc_pool* p, uint32_t b, const uint8_t* h32);
int orc_pool_reclaim(orc_pool* p, const uint8_t* h32, uint32_t* out); /* 1 hit, 0 miss */
uint32_t orc_pool_refs(const orc_pool* p, uint32_t b);
int orc_pool_is_cached(const orc_pool* p, uint32_t b);
void orc_pool_clear_hash(orc_pool* p, uint32_t b);
void orc_pool_note_miss(orc_pool* p);
uint64_t orc_pool_block_tokens(const orc_pool* p);
void orc_pool_stats(const orc_pool* p, uint64_t* out6); /* n_blocks free cached_free hits misses evictions */

/* ---- KvCache (kv.rs:562-939) ---- */
typedef struct orc_cache orc_cache;
orc_cache* orc_cache_new(const orc_options* o, const orc_layer_geom* layers, uint64_t n_layers);
void orc_cache_free(orc_cache* c);
void orc_cache_layout(const orc_cache* c, orc_layout_info* out);
void orc_cache_layer(const orc_cache* c, uint64_t l, orc_layer_info* out);
orc_pool* orc_cache_pool(orc_cache* c);
uint64_t orc_cache_len(const orc_cache* c, uint64_t s);
void orc_cache_set_len(orc_cache* c, uint64_t s, uint64_t len);
uint64_t orc_cache_blocks_needed(const orc_cache* c, uint64_t s, uint64_t new_len);
int orc_cache_reserve(orc_cache* c, uint64_t s, uint64_t new_len, uint64_t* needed, uint64_t* free_);
void orc_cache_truncate(orc_cache* c, uint64_t s, uint64_t n);
void orc_cache_clear(orc_cache* c, uint64_t s);
uint64_t orc_cache_resident_blocks(const orc_cache* c);
uint64_t orc_cache_seq_blocks(const orc_cache* c, uint64_t s, uint32_t* out, uint64_t cap);
/* Test hook: impose a block table (e.g. a seeded permutation). Takes the listed free blocks out of
 * the pool in that order; fails (ORC_INVALID) if any is not free or the sequence holds blocks. */
int orc_cache_adopt_blocks(orc_cache* c, uint64_t s, const uint32_t* blocks, uint64_t n);
int orc_cache_bind_seq(orc_cache* c, uint64_t s, const uint32_t* blocks, uint64_t n, uint64_t len);
void orc_cache_store_k(orc_cache* c, uint64_t s, uint64_t l, uint64_t pos, const float* k);
void orc_cache_store_v(orc_cache* c, uint64_t s, uint64_t l, uint64_t pos, const float* v);
/* Write one row already in the cache's row encoding (row_bytes(kv_dim) bytes). */
void orc_cache_store_k_raw(orc_cache* c, uint64_t s, uint64_t l, uint64_t pos, const uint8_t* row);
void orc_cache_store_v_raw(orc_cache* c, uint64_t s, uint64_t l, uint64_t pos, const uint8_t* row);
/* Bulk forms: rows pos0..pos0+n of sequence s (k: [n][kv_dim] f32 or [n][k_row] bytes). */
void orc_cache_store_rows(orc_cache* c, uint64_t s, uint64_t l, uint64_t pos0, uint64_t n, const float* k,
                          const float* v);
void orc_cache_store_rows_raw(orc_cache* c, uint64_t s, uint64_t l, uint64_t pos0, uint64_t n, const uint8_t* k,
                              const uint8_t* v);
/* Encoded rows back (reference row encoding), for byte-exact comparisons. */
void orc_cache_load_rows_raw(const orc_cache* c, uint64_t s, uint64_t l, uint64_t pos0, uint64_t n, uint8_t* k,
                             uint8_t* v);
void orc_cache_load_k(const orc_cache* c, uint64_t s, uint64_t l, uint64_t pos, uint64_t start,
                      uint64_t len, float* out);
void orc_cache_load_v(const orc_cache* c, uint64_t s, uint64_t l, uint64_t pos, uint64_t start,
                      uint64_t len, float* out);

/* ---- batch hand-off (forward.rs:29-86, 207-291) ---- */
typedef struct orc_seg {
  uint64_t seq, start, n, pos0;
} orc_seg;

/* Validate + reserve all-or-nothing + stack rows. Returns ORC_OK, ORC_KV_FULL (nothing changed,
 * needed/free filled) or ORC_INVALID (a batch the reference would reject with a panic). */
int orc_prepare_batch(orc_cache* c, const uint64_t* seqs, const uint64_t* n_tokens, uint64_t m,
                      orc_seg* segs_out, uint64_t* n_rows, uint64_t* needed, uint64_t* free_);
/* run_layers' tail (forward.rs:363-366): every segment's sequence grows by its row count. */
void orc_commit_batch(orc_cache* c, const orc_seg* segs, uint64_t n_segs);

/* ---- attention (forward.rs:566-807, cpu/src/ops.rs:69-80, 127-151) ---- */
uint64_t orc_attend_splits(uint64_t n_rows, uint64_t n_kv, uint64_t threads, uint64_t span);
/* window 0 = None. q: [n][n_head][hd] f32, out: [n][n_head][hdv] f32. */
void orc_attend(const orc_cache* c, uint64_t l, const orc_seg* segs, uint64_t n_segs,
                const float* q, uint64_t n_head, float scale, uint64_t window, uint64_t threads,
                float* out);
/* Independent float64 softmax attention over the same decoded cache values (pinning only). */
void orc_attend_naive_f64(const orc_cache* c, uint64_t l, const orc_seg* segs, uint64_t n_segs,
                          const float* q, uint64_t n_head, double scale, uint64_t window,
                          double* out);

/* ops restated for direct tests */
float orc_dot(const float* a, const float* b, uint64_t n);
void orc_softmax(float* x, uint64_t n);

/* ---- snapshots (KvCache::snapshot_bytes / write_seq / read_seq, kv.rs:1009-1130) ---- */
uint64_t orc_cache_snapshot_bytes(const orc_cache* c, uint64_t len);
void orc_cache_write_seq(const orc_cache* c, uint64_t s, uint8_t* out);
int orc_cache_read_seq(orc_cache* c, uint64_t s, uint64_t len, const uint8_t* bytes, uint64_t n, uint64_t* needed,
                       uint64_t* free_);

/* ---- QK-norm + RoPE (cpu/src/ops.rs:18-66, model/src/forward.rs:427-453, 832-838) ---- */
typedef struct orc_rope_params {
  int32_t apply;        /* rotate (0 on NoPE layers) */
  int32_t neox;         /* pair (i, i + rot_dim/2) instead of (2i, 2i+1) */
  int32_t v_norm;       /* weightless RMS norm of each V head (Metal misc.metal:218-226) */
  uint32_t rot_dim;
  float eps, theta, freq_scale, attn_factor;
  const float* q_norm;  /* [hd] or NULL */
  const float* k_norm;  /* [hd] or NULL */
  const float* freq_div; /* [rot_dim/2] or NULL */
} orc_rope_params;
void orc_rms_norm(const float* x, const float* w, float eps, float* y, size_t n);
void orc_rope_apply(float* x, size_t n_heads, size_t hd, uint32_t pos, const orc_rope_params* p);
void orc_qk_rope(const float* q_in, const float* k_in, const float* v_in, const uint32_t* pos, size_t n_rows,
                 size_t n_head, size_t n_kv, size_t hd, size_t hdv, size_t q_stride, const orc_rope_params* p,
                 float* q_out, float* k_out, float* v_out);

#ifdef __cplusplus
}
#endif
#endif
