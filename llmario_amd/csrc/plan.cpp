// plan.cpp — lmh_attend's work-list planner (host only). What is computed per row is attend /
// attend_split's (forward.rs:585-807): each row attends to keys [lo, pos] of its sequence; rows
// of long ranges are cut into split-K items whose partials merge with the log-sum-exp merge
// (forward.rs:772-806). How the rows are cut and packed is this backend's own.
#include "plan.h"

#include <algorithm>
#include <queue>
#include <utility>

namespace lmh {
namespace {

uint64_t key_lo(uint64_t pos, uint64_t window) { return (window > 0 && pos + 1 > window) ? pos + 1 - window : 0; }

// Prefill units grouped per workgroup: prefill_wg_per_cu workgroups per CU, each running a list
// of units. Longest-processing-time-first: units by decreasing key pages (plus a fixed cost for
// the unit's Q load and output), each to the currently least loaded workgroup. Lists are padded
// to the longest with empty units (n_tok = 0) at a fixed stride.
void assign_prefill_units(std::vector<PrefillItem>& items, uint64_t window, uint32_t slots, uint32_t& n_wg,
                          uint32_t& per_wg) {
  n_wg = (uint32_t)std::min<uint64_t>(items.size(), std::max<uint32_t>(slots, 1));
  per_wg = 0;
  if (n_wg == 0) return;
  auto work = [&](const PrefillItem& it) -> uint64_t {
    const uint64_t last = (uint64_t)it.pos0 + it.n_tok - 1;
    return last / 16 - key_lo(it.pos0, window) / 16 + 1 + 8;
  };
  std::stable_sort(items.begin(), items.end(),
                   [&](const PrefillItem& a, const PrefillItem& b) { return work(a) > work(b); });
  std::vector<std::vector<uint32_t>> lists(n_wg);
  std::priority_queue<std::pair<uint64_t, uint32_t>, std::vector<std::pair<uint64_t, uint32_t>>,
                      std::greater<std::pair<uint64_t, uint32_t>>> load;
  for (uint32_t b = 0; b < n_wg; b++) load.push({0, b});
  for (uint32_t i = 0; i < items.size(); i++) {
    auto [l, b] = load.top();
    load.pop();
    lists[b].push_back(i);
    load.push({l + work(items[i]), b});
  }
  for (const auto& li : lists) per_wg = std::max<uint32_t>(per_wg, (uint32_t)li.size());
  std::vector<PrefillItem> out((size_t)n_wg * per_wg, PrefillItem{});
  for (uint32_t b = 0; b < n_wg; b++)
    for (size_t j = 0; j < lists[b].size(); j++) out[(size_t)b * per_wg + j] = items[lists[b][j]];
  items.swap(out);
}

}  // namespace

void plan_attend(const PlanIn& in, PlanOut& o) {
  const uint64_t n_rows = in.n_rows, window = in.window;
  const uint32_t group = in.n_head / in.n_kv;
  // heads per decode item: up to 16 (the matrix-core tile's columns), fewer on the row-layout kernel
  o.ng = std::min<uint32_t>(group, in.layout == LAYOUT_ROWS ? in.rows_max_heads : 16);
  const uint32_t ng = o.ng;
  const uint32_t head_blocks = (group + ng - 1) / ng;
  o.decode_row.assign(n_rows, 1);
  o.items.clear();
  o.merges.clear();
  o.pitems.clear();
  o.slots = o.pf_wg = o.pf_per_wg = o.max_pages = 0;
  o.local = false;
  auto blk_at = [&](uint64_t seq, uint64_t p) {   // block id of the tile holding key p
    return (uint32_t)in.table[seq * in.bps + (((p >> 4) << 4) >> in.bt_shift)];
  };

  // ---- prefill units: segments of at least `pf_min` rows go to the matrix-core prefill kernel
  // in units of up to unit_cols / group tokens per KV head, balanced over prefill_wg_per_cu
  // workgroups per CU.
  const uint64_t pf_min = in.prefill_min_rows ? in.prefill_min_rows : DEFAULT_PREFILL_MIN_ROWS;
  const bool pf_ok = in.scale > 0.f && in.layout == LAYOUT_TILES && in.prefill_supported;
  if (pf_ok) {
    const uint32_t unit_tok = std::max<uint32_t>(in.unit_cols / group, 1);
    for (uint64_t i = 0; i < in.n_segs; i++) {
      const lmh_seg& sg = in.segs[i];
      if (sg.n < pf_min) continue;
      for (uint64_t u = 0; u < sg.n; u += unit_tok) {
        const uint32_t n_tok = (uint32_t)std::min<uint64_t>(unit_tok, sg.n - u);
        const uint64_t pos0 = sg.pos0 + u, last = pos0 + n_tok - 1;
        const uint64_t lo = key_lo(pos0, window);
        o.max_pages = std::max<uint32_t>(o.max_pages, (uint32_t)(last / 16 - lo / 16 + 1));
        PrefillItem it{(uint32_t)sg.seq, 0, (uint32_t)(sg.start + u), (uint32_t)pos0, n_tok, 0, 0, 0, {}};
        const uint64_t page0 = lo / 16, n_pages = last / 16 - lo / 16 + 1;
        for (uint64_t b = 0; b < 8; b++) it.blk[b] = blk_at(sg.seq, (page0 + std::min<uint64_t>(b, n_pages - 1)) << 4);
        for (uint32_t kvh = 0; kvh < in.n_kv; kvh++) {
          it.kvh = kvh;
          o.pitems.push_back(it);
        }
      }
      for (uint64_t j = 0; j < sg.n; j++) o.decode_row[sg.start + j] = 0;
    }
    const uint32_t slots = in.n_cu * in.prefill_wg_per_cu;
    assign_prefill_units(o.pitems, window,
                         in.prefill_workgroups ? (uint32_t)std::min<uint64_t>(in.prefill_workgroups, slots) : slots,
                         o.pf_wg, o.pf_per_wg);
    if (in.prefill_lds_fixed + (size_t)o.pf_per_wg * sizeof(PrefillItem) + (size_t)o.max_pages * 4 > in.lds_limit) {
      // key ranges too long to list in LDS: those segments go through the decode kernel
      o.pitems.clear();
      std::fill(o.decode_row.begin(), o.decode_row.end(), 1);
      o.max_pages = 0;
      o.pf_wg = o.pf_per_wg = 0;
    }
  }

  // ---- decode work list: per (row, KV head, head block), the key range [lo, pos] cut into
  // chunks of whole 16-token tiles, spread evenly; rows whose range fits one chunk write the output.
  auto row_tiles = [&](uint64_t t) {
    const uint64_t pos = (uint64_t)in.row_pos[t];
    return pos / 16 - key_lo(pos, window) / 16 + 1;
  };
  uint64_t total_tiles = 0;
  for (uint64_t t = 0; t < n_rows; t++)
    if (o.decode_row[t]) total_tiles += row_tiles(t);
  total_tiles *= (uint64_t)in.n_kv * head_blocks;
  // Items the GPU holds at once: with at most that many, every item starts in the first round and
  // none waits for a slot to free up (a second, mostly empty round would double the kernel time).
  // The matrix-core decode kernel targets half of them: one item per SIMD streams each key range
  // with its two-deep prefetch as fast as two do, and half the items halve the per-item start-up,
  // the partials and the merge (often to none: 128 rows of 512 keys become one item per row and
  // KV head, 56.4 -> 42.6 us; c2 cold 51.2 -> 49.6 us; 4 rows of 16 K keys 54.0 -> 48.9 us; c4 and
  // rows of a group of 8 unchanged). The f32 and row-layout kernels, latency-bound, keep all of them.
  const bool mfma_decode = in.layout == LAYOUT_TILES && in.kv_type != LMH_KV_F32;
  const uint64_t cap_target = mfma_decode ? std::max<uint64_t>(in.decode_capacity / 2, in.n_cu) : in.decode_capacity;
  uint64_t target = std::max<uint64_t>(in.decode_target_items ? in.decode_target_items : cap_target, 1);
  // no-allocation calls: at most as many split slots (and merges) as the scratch holds
  const size_t slot_bytes = (size_t)ng * (in.hdv + 4) * 4;
  if (in.noalloc)
    target = std::max<uint64_t>(1, std::min<uint64_t>(target, in.noalloc_bytes / (slot_bytes + sizeof(MergeItem))));
  // Smallest chunk: 8 tiles for the matrix-core kernels (enough work per wave to stream at full
  // rate); 2 tiles for f32 rows, whose VALU kernel walks keys with dependent loads (latency-bound:
  // more, shorter items hide it better); 4 for the row layout.
  const uint64_t min_chunk = in.decode_min_tiles ? in.decode_min_tiles
                                                 : (in.layout == LAYOUT_ROWS ? 4 : in.kv_type == LMH_KV_F32 ? 2 : 8);
  // chunks of whole tiles; at most 64 per item (the decode kernel keeps one block id per lane);
  // grown until the rows' rounded-up split counts fit the target
  auto n_items_for = [&](uint64_t c) {
    uint64_t n = 0;
    for (uint64_t t = 0; t < n_rows; t++)
      if (o.decode_row[t]) n += (row_tiles(t) + c - 1) / c;
    return n * in.n_kv * head_blocks;
  };
  uint64_t chunk = std::min<uint64_t>(64, std::max<uint64_t>(min_chunk, (total_tiles + target - 1) / target));
  while (chunk < 64 && n_items_for(chunk) > target) chunk++;
  o.chunk = (uint32_t)chunk;
  // f32 pages, short rows (at most 16 tiles): a row's split items are consecutive waves of one
  // 8-wave workgroup and merge there (no merge launch). A row splits into 1, 2, 4 or 8 items of
  // at most 2 tiles (the f32 kernel's smallest chunk); groups of 8 go first, then 4, 2 and single
  // items, so no group crosses a workgroup. Not with explicit split settings.
  if (in.layout == LAYOUT_TILES && in.kv_type == LMH_KV_F32 && in.local_merge_ok && !in.decode_target_items &&
      !in.decode_min_tiles) {
    uint64_t max_nt = 0;
    for (uint64_t t = 0; t < n_rows; t++)
      if (o.decode_row[t]) max_nt = std::max<uint64_t>(max_nt, row_tiles(t));
    o.local = max_nt > 2 && max_nt <= 16;
  }
  if (o.local) {
    std::vector<DecodeItem> by_size[4];   // groups of 8, 4, 2, single items
    for (uint64_t t = 0; t < n_rows; t++) {
      if (!o.decode_row[t]) continue;
      const uint64_t pos = (uint64_t)in.row_pos[t];
      const uint64_t lo = key_lo(pos, window), hi = pos + 1;
      const uint64_t tlo = lo / 16, n_t = pos / 16 - tlo + 1;
      const uint32_t n = n_t <= 2 ? 1 : n_t <= 4 ? 2 : n_t <= 8 ? 4 : 8;
      std::vector<DecodeItem>& dst = by_size[n == 8 ? 0 : n == 4 ? 1 : n == 2 ? 2 : 3];
      const uint32_t seq = (uint32_t)in.row_seq[t];
      for (uint32_t kvh = 0; kvh < in.n_kv; kvh++) {
        for (uint32_t hb = 0; hb < head_blocks; hb++) {
          for (uint32_t s = 0; s < n; s++) {
            const uint64_t a = tlo + s * n_t / n, b = tlo + (s + 1) * n_t / n;
            const uint64_t p0 = std::max(lo, a * 16), p1 = std::min(hi, b * 16);
            const uint32_t slot = n == 1 ? NO_SLOT : LOCAL_SLOT | (s << 8) | n;
            dst.push_back(DecodeItem{(uint32_t)t, kvh, hb * ng, (uint32_t)p0, (uint32_t)p1, slot, seq, blk_at(seq, p0)});
          }
        }
      }
    }
    for (auto& v : by_size) o.items.insert(o.items.end(), v.begin(), v.end());
    return;
  }
  for (uint64_t t = 0; t < n_rows; t++) {
    if (!o.decode_row[t]) continue;
    const uint64_t pos = (uint64_t)in.row_pos[t];
    const uint64_t lo = key_lo(pos, window), hi = pos + 1;
    const uint64_t tlo = lo / 16, n_t = pos / 16 - tlo + 1;
    const uint64_t n_split = (n_t + chunk - 1) / chunk;
    const uint32_t seq = (uint32_t)in.row_seq[t];
    for (uint32_t kvh = 0; kvh < in.n_kv; kvh++) {
      for (uint32_t hb = 0; hb < head_blocks; hb++) {
        if (n_split == 1) {
          o.items.push_back(DecodeItem{(uint32_t)t, kvh, hb * ng, (uint32_t)lo, (uint32_t)hi, NO_SLOT, seq, blk_at(seq, lo)});
          continue;
        }
        o.merges.push_back(MergeItem{(uint32_t)t, kvh, hb * ng, o.slots, (uint32_t)n_split, 0});
        for (uint64_t s = 0; s < n_split; s++) {
          const uint64_t a = tlo + s * n_t / n_split, b = tlo + (s + 1) * n_t / n_split;
          const uint64_t p0 = std::max(lo, a * 16), p1 = std::min(hi, b * 16);
          o.items.push_back(DecodeItem{(uint32_t)t, kvh, hb * ng, (uint32_t)p0, (uint32_t)p1, o.slots++, seq, blk_at(seq, p0)});
        }
      }
    }
  }
}

}  // namespace lmh
