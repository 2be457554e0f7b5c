// plan.h — lmh_attend's work-list planner: from a call's segments (forward.rs:31-86) to the
// decode items, split-K merges and prefill units the kernels run. Host code only (no device
// calls), so the CPU tests drive it directly (lmh_plan_attend) and the sanitizer build covers it.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <vector>

#include "../../include/llmario_hip.h"
#include "work.h"

namespace lmh {

struct PlanIn {
  // the call's stacked rows (sequence and position of each) and its segments
  const int32_t* row_seq = nullptr;
  const int32_t* row_pos = nullptr;
  uint64_t n_rows = 0;
  const lmh_seg* segs = nullptr;
  uint64_t n_segs = 0;
  // the layer's block table (host copy, [n_seqs][bps]) and block size
  const int32_t* table = nullptr;
  uint64_t bps = 0;
  uint32_t bt_shift = 4;
  // the layer
  uint32_t n_head = 0, n_kv = 0, hd = 0, hdv = 0;
  uint32_t layout = LAYOUT_TILES;   // LAYOUT_TILES / LAYOUT_ROWS
  uint32_t kv_type = 0;             // LMH_KV_*
  uint64_t window = 0;              // the call's attention window (0: none)
  float scale = 0.f;
  // the device
  uint32_t n_cu = 1;
  uint64_t decode_capacity = 1;     // decode items the layer's decode kernel holds at once
  // lmh_attend_tuning (0: the default)
  uint64_t prefill_min_rows = 0, decode_target_items = 0, decode_min_tiles = 0, prefill_workgroups = 0;
  bool prefill_no_split = false;    // units are never cut into key pieces
  // lmh_attend_noalloc: split slots and merges bounded by the scratch
  bool noalloc = false;
  size_t noalloc_bytes = 0;
  // facts of the kernel modules
  bool prefill_supported = false;   // a prefill instance takes (type, hd, hdv, group)
  uint32_t unit_cols = 256;         // columns (token x query head) per prefill unit
  uint32_t prefill_wg_per_cu = 1;
  size_t prefill_lds_fixed = 0;     // prefill LDS besides the unit list and the block ids
  size_t lds_limit = 160 * 1024;
  uint32_t rows_max_heads = 4;      // query heads per item of the row-layout kernel
  bool local_merge_ok = false;      // f32 decode: split rows may merge inside their workgroup
  bool mfma_local_ok = false;       // matrix-core decode: the same, for rows split at most 4 ways
};

struct PlanOut {
  std::vector<uint8_t> decode_row;    // per row: 1 = a decode row, 0 = in a prefill unit
  std::vector<DecodeItem> items;
  std::vector<MergeItem> merges;
  std::vector<PrefillItem> pitems;    // pf_wg lists of pf_per_wg units (an empty unit ends a list)
  uint32_t ng = 0;                    // query heads per decode item
  uint32_t slots = 0;                 // split-K partial slots
  uint32_t pf_wg = 0, pf_per_wg = 0, max_pages = 0;
  uint32_t chunk = 0;                 // decode split chunk (16-key tiles)
  uint32_t local = 0;                 // decode items merge inside workgroups of this many waves (0: no)
};

// Segments of at least this many rows run on the matrix-core prefill kernel by default (Metal's
// FA_MIN_TOKENS, metal/src/backend.rs:181). Measured on 8-row segments at contexts of 512..4096,
// 32/8 heads, hd 128: the prefill kernel takes 89 us for 8 sequences (86 us as decode rows, each
// re-reading its prefix) and 105 us for 32 (354 us as decode rows); at 4 rows the decode rows win
// for 8 sequences (41 against 89 us).
constexpr uint64_t DEFAULT_PREFILL_MIN_ROWS = 8;

void plan_attend(const PlanIn& in, PlanOut& out);

}  // namespace lmh
