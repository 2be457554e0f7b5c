// work.h — the per-call work lists lmh_attend's planner (plan.cpp, host only) builds and the
// attention kernels read: plain structures, no device headers.
#pragma once

#include <stdint.h>

namespace lmh {

enum : uint32_t { KV_F16 = 0, KV_Q8 = 1, KV_F32 = 2, KV_BF16 = 3 };
constexpr uint32_t LAYOUT_TILES = 0, LAYOUT_ROWS = 1;

// One decode work item: row `row` (its sequence and position come from the row arrays), KV head
// `kvh`, query heads kvh*group + h0 .. + n_heads, keys [p0, p1). `slot` is the partial-result slot
// (split-K) or NO_SLOT when the item covers the row's whole key range and writes the output.
struct DecodeItem {
  uint32_t row;
  uint32_t kvh;
  uint32_t h0;
  uint32_t p0, p1;
  uint32_t slot;
  uint32_t seq;   // the row's sequence (saves a dependent read of the row arrays)
  uint32_t blk0;  // block id of the first tile p0 >> 4 (the first fetch skips the block-table read)
};
constexpr uint32_t NO_SLOT = 0xffffffffu;
// Tiles per decode item: the matrix-core kernel keeps two block ids per lane (the planner uses the
// second for f16 / bf16 pages), the f32 and row-layout kernels one.
constexpr uint32_t MFMA_ITEM_TILES = 128;
constexpr uint32_t ITEM_TILES = 64;
// A split item merged inside its workgroup (f32 decode of short rows; matrix-core decode whose rows
// split at most MFMA_LOCAL_WAVES ways): LOCAL_SLOT | (its index in the row's group << 8) | the
// group's size; the group's items are consecutive waves of one workgroup, which merges their
// partials from LDS, so the call needs no merge launch.
constexpr uint32_t LOCAL_SLOT = 0x80000000u;
constexpr uint32_t LOCAL_MERGE_MAX = 1024;   // heads x hdv of an item whose partials a wave keeps in LDS
constexpr int LOCAL_WAVES = 8;               // waves per workgroup of an f32 local-merge call (its largest group)
// The same for the matrix-core decode kernel (its own 4-wave workgroups). Not 8-wave ones for rows
// of up to 8 splits: c2 (rows of 512-4,096 keys) ran its 1,328 items on 166 such workgroups, the
// CUs left idle slowed the kernel from 50.0 to 62.8 us, more than the merge launch costs.
constexpr int MFMA_LOCAL_WAVES = 4;
// The decode workgroups of a mixed launch (prefill units beside decode rows) have 8 waves.
constexpr int MIXED_LOCAL_WAVES = 8;

// Merge of `n_split` consecutive partial slots starting at `slot0` for (row, kvh, heads h0 ..
// h0 + nh - 1). nh = 0 (a decode row's merge): up to the item's head count ng, head h0 + i at
// position i of a slot. nh != 0 (a prompt token's merge over the key pieces of its unit): head h
// at position h of a slot (the slot holds the whole KV group: group <= 16 = ng).
struct MergeItem {
  uint32_t row;
  uint32_t kvh;
  uint32_t h0;
  uint32_t slot0;
  uint32_t n_split;
  uint32_t nh;
};
// A prompt token's merge (nh != 0) combines at most this many key pieces, and nh * n_split <=
// PF_MERGE_ROWS unless nh = 1 (the merge folds an item's partial rows within one wave, loading up
// to PF_MERGE_ROWS rows at once); such merges precede the decode merges in a call's list.
constexpr uint32_t PF_MAX_PIECES = 64;
constexpr uint32_t PF_MERGE_ROWS = 32;

// One prefill work unit: KV head `kvh` of sequence `seq`. Its columns are the (token, query head)
// pairs of the stacked rows row0, row0 + 1, .. (positions pos0, pos0 + 1, ..) flattened
// token-major from head c_off of the first token: column c < n_col is token (c + c_off) / group,
// head (c + c_off) % group (n_col <= prefill_cols_per_unit(); n_tok = the tokens the columns
// touch). Its keys are pages page0 .. page0 + n_pages - 1 of the sequence (16 positions each),
// within each column's own range (causal, window). slot = NO_SLOT: those pages are the columns'
// whole ranges and the unit writes the output. Otherwise the unit is one key piece of a longer
// range: column (t, h)'s partial (o, m, l) goes to slot `slot + t * slot_stride`, at position h,
// and a merge launch combines the pieces.
// blk: the block ids of pages page0 .. page0 + 7 (clamped to the last page), so the first K/V
// tiles are fetched without waiting for the block table.
struct PrefillItem {
  uint32_t seq;
  uint32_t kvh;
  uint32_t row0;
  uint32_t pos0;
  uint32_t n_tok;
  uint32_t c_off, n_col;
  uint32_t page0, n_pages;
  uint32_t slot, slot_stride;
  uint32_t pad;
  uint32_t blk[8];
};

}  // namespace lmh
