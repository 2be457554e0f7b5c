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

// Prefill cost model, in units of one 64-key tile of a unit with all 256 columns: a tile of a unit
// with fewer columns costs less (waves without columns only stage tiles), and every unit (or key
// piece of one) pays a fixed cost for its Q loads and its output (measured on c3 / c5: a full tile
// 2.2-2.4 us, the per-unit Q load, barrier and stores ~8 us).
constexpr double PF_UNIT_COST = 3.5;
double tile_cost(uint32_t n_col) { return 0.35 + 0.65 * std::min(8u, (n_col + 31) / 32) / 8.0; }
// Key pieces are at least this many 64-key tiles (a unit is cut only when it has twice as many).
#ifndef LMH_PF_MIN_PIECE
#define LMH_PF_MIN_PIECE 8
#endif
constexpr uint32_t PF_MIN_PIECE = LMH_PF_MIN_PIECE;
// A decode row's 16-key tile for one KV head, in the same units (c2's decode kernel streams 36,864
// such tiles in ~50 us on 256 CUs, 0.34 CU-us each, at a 2.2-us tile: 0.16; CUs that share HBM
// with prefill work stream faster each).
constexpr double DECODE_TILE_COST = 0.1;
// A decode item's own time per 16-key tile, in the same units: a wave streams a tile in ~1.2 us
// (8 KiB per 16-key tile at the ~7 GB/s one wave's two-deep prefetch sustains).
constexpr double DECODE_WAVE_TILE = 0.5;
// A mixed launch's decode chunk may grow (so split rows merge inside their workgroups) while its
// longest item stays within this fraction of the prefill part's largest workgroup load.
constexpr double MIXED_DECODE_SLACK = 0.75;

struct PfUnit {
  PrefillItem it;   // page0 / n_pages: the whole unit's key pages
  uint32_t tiles;
  double cpt;
  double cost() const { return tiles * cpt + PF_UNIT_COST; }
};

// The merge of cut units' pieces, in the same units per (token, query head, piece) partial read
// (c5's 76,960 such partials of hdv 128 merge in 10.6 us more than its decode rows' merges alone,
// at a 2.5-us tile), and the merge launch's own cost when no decode rows need one.
constexpr double PF_MERGE_PARTIAL = 5.6e-5;
constexpr double PF_MERGE_LAUNCH = 1.5;
// Cut units only when that is estimated to finish at most this fraction of the whole units' time
// (the walk's estimate was measured optimistic on c5: 7 tiles gained, 4.7 measured).
#ifndef LMH_PF_CUT_GAIN
#define LMH_PF_CUT_GAIN 0.9
#endif
constexpr double PF_CUT_GAIN = LMH_PF_CUT_GAIN;

// Prefill items per workgroup in the order they were added, as (workgroup, item) pairs appended to
// two flat arrays: a call lists ~1,000 units over ~256 workgroups, and one vector per workgroup
// cost more host time in allocations than the planning itself.
struct WgLists {
  uint32_t n_wg = 0;
  std::vector<uint32_t> wg;
  std::vector<PrefillItem> it;
  void reset(uint32_t n, size_t cap) {
    n_wg = n;
    wg.clear();
    it.clear();
    wg.reserve(cap);
    it.reserve(cap);
  }
  void push(uint32_t b, const PrefillItem& x) {
    wg.push_back(b);
    it.push_back(x);
  }
};

// Whole units grouped per workgroup, longest-processing-time-first: units by decreasing cost (ties
// in list order), each to the currently least loaded workgroup (ties to the lower index). Returns
// the largest workgroup load. The loads live in a binary min-heap of (load, workgroup) whose top
// is updated in place; the pairs are distinct, so the least one, and with it the plan, does not
// depend on how the heap orders equal loads.
double assign_whole_units(const std::vector<PfUnit>& units, uint32_t slots, WgLists& lists) {
  const uint32_t n_wg = (uint32_t)std::min<uint64_t>(units.size(), std::max<uint32_t>(slots, 1));
  lists.reset(n_wg, units.size());
  std::vector<std::pair<double, uint32_t>> order(units.size());
  for (uint32_t i = 0; i < order.size(); i++) order[i] = {-units[i].cost(), i};
  std::sort(order.begin(), order.end());
  std::vector<std::pair<double, uint32_t>> heap(n_wg);
  for (uint32_t b = 0; b < n_wg; b++) heap[b] = {0.0, b};   // ascending: already a heap
  for (const auto& oi : order) {
    const PfUnit& u = units[oi.second];
    lists.push(heap[0].second, u.it);
    heap[0].first += u.cost();
    for (size_t j = 0;;) {   // sift the grown top down
      const size_t c = 2 * j + 1;
      if (c >= heap.size()) break;
      const size_t m = c + 1 < heap.size() && heap[c + 1] < heap[c] ? c + 1 : c;
      if (!(heap[m] < heap[j])) break;
      std::swap(heap[m], heap[j]);
      j = m;
    }
  }
  double mx = 0.0;
  for (const auto& h : heap) mx = std::max(mx, h.first);
  return mx;
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
  o.local = 0;
  auto blk_at = [&](uint64_t seq, uint64_t p) {   // block id of the tile holding key p
    return (uint32_t)in.table[seq * in.bps + (((p >> 4) << 4) >> in.bt_shift)];
  };

  // ---- prefill units: segments of at least `pf_min` rows go to the matrix-core prefill kernel.
  // Per segment and KV head, the (token, query head) columns are packed token-major in units of
  // unit_cols (a unit may start mid-token, so no unit is a remnant of a few columns); a unit's keys
  // are the pages from its first token's range start to its last token.
  double pf_load = 0.0;   // the prefill part's largest workgroup load (estimate)
  const uint64_t pf_min = in.prefill_min_rows ? in.prefill_min_rows : DEFAULT_PREFILL_MIN_ROWS;
  const bool pf_ok = in.scale > 0.f && in.layout == LAYOUT_TILES && in.prefill_supported;
  if (pf_ok) {
    std::vector<PfUnit> units;
    uint64_t n_units = 0;
    for (uint64_t i = 0; i < in.n_segs; i++)
      if (in.segs[i].n >= pf_min) n_units += (in.segs[i].n * group + in.unit_cols - 1) / in.unit_cols * in.n_kv;
    units.reserve(n_units);
    for (uint64_t i = 0; i < in.n_segs; i++) {
      const lmh_seg& sg = in.segs[i];
      if (sg.n < pf_min) continue;
      const uint64_t total = sg.n * group;
      for (uint64_t c0 = 0; c0 < total; c0 += in.unit_cols) {
        const uint32_t n_col = (uint32_t)std::min<uint64_t>(in.unit_cols, total - c0);
        const uint64_t t0 = c0 / group, t1 = (c0 + n_col - 1) / group;
        const uint64_t pos0 = sg.pos0 + t0, last = sg.pos0 + t1;
        const uint64_t page_lo = key_lo(pos0, window) / 16, n_pages = last / 16 - page_lo + 1;
        PfUnit u{};
        u.it.seq = (uint32_t)sg.seq;
        u.it.row0 = (uint32_t)(sg.start + t0);
        u.it.pos0 = (uint32_t)pos0;
        u.it.n_tok = (uint32_t)(t1 - t0 + 1);
        u.it.c_off = (uint32_t)(c0 % group);
        u.it.n_col = n_col;
        u.it.page0 = (uint32_t)page_lo;
        u.it.n_pages = (uint32_t)n_pages;
        u.it.slot = NO_SLOT;
        u.tiles = (uint32_t)((n_pages + 3) / 4);
        u.cpt = tile_cost(n_col);
        for (uint32_t kvh = 0; kvh < in.n_kv; kvh++) {
          u.it.kvh = kvh;
          units.push_back(u);
        }
      }
      for (uint64_t j = 0; j < sg.n; j++) o.decode_row[sg.start + j] = 0;
    }
    // Workgroups for the prefill units. With decode rows in the same launch, the CUs are shared in
    // proportion to the two kinds' estimated cost (the decode workgroups take the others).
    uint32_t slots = in.n_cu * in.prefill_wg_per_cu;
    double w_pf = 0.0;
    uint32_t max_tiles = 0;
    double max_cost = 0.0;
    for (const PfUnit& u : units) {
      w_pf += u.cost();
      max_tiles = std::max(max_tiles, u.tiles);
      max_cost = std::max(max_cost, u.cost());
    }
    uint64_t decode_tiles = 0;
    for (uint64_t t = 0; t < n_rows; t++) {
      if (!o.decode_row[t]) continue;
      const uint64_t pos = (uint64_t)in.row_pos[t];
      decode_tiles += pos / 16 - key_lo(pos, window) / 16 + 1;
    }
    if (decode_tiles > 0 && !units.empty() && slots > 1) {
      const double w_dec = (double)decode_tiles * in.n_kv * head_blocks * DECODE_TILE_COST;
      const double share = w_pf / (w_pf + w_dec);
      slots = std::min<uint32_t>(slots - 1, std::max<uint32_t>(1, (uint32_t)(slots * share + 0.5)));
    }
    if (in.prefill_workgroups) slots = (uint32_t)std::min<uint64_t>(in.prefill_workgroups, slots);
    WgLists lists;
    // Whole units (longest first, each to the least loaded workgroup), unless cutting is estimated
    // to finish well ahead: then the concatenated tiles of all units are cut into one stretch per
    // workgroup (stream-K), a unit spanning several workgroups running as key pieces that each leave
    // partials (O, m, l) per column for the merge launch (attend_split's merge,
    // forward.rs:772-806). A piece's partial slot per token holds the unit's heads of that token:
    // groups of up to 16 heads, as the decode items'. The cut plan is kept when its largest load
    // plus the merge's estimate is below PF_CUT_GAIN of the whole units' largest load; a first
    // bound on its load is the tiles shared evenly with about one more piece per workgroup.
    const double whole = assign_whole_units(units, slots, lists);
    pf_load = whole;
    double w_cut = 0.0;
    for (const PfUnit& u : units) w_cut += u.tiles * u.cpt;
    const double cap = (w_cut + PF_UNIT_COST * ((double)units.size() + slots)) / std::max<uint32_t>(slots, 1);
    const bool try_cut = !in.prefill_no_split && group <= 16 && !units.empty() && max_tiles >= 2 * PF_MIN_PIECE &&
                         cap < PF_CUT_GAIN * whole;
    // A cut unit's merges: per token over the unit's heads of that token, in groups of heads whose
    // partial rows (heads x pieces) one merge wave loads at once. for_each_merge(u, k, f) calls
    // f(token, first head, heads) for each.
    auto for_each_merge = [&](const PfUnit& u, uint32_t k, auto&& f) {
      const uint32_t hpm = std::max<uint32_t>(1, PF_MERGE_ROWS / k);
      const uint64_t c_abs = u.it.c_off;   // the unit's first column, counted from its first token
      for (uint32_t i = 0; i < u.it.n_tok; i++) {
        const uint64_t h_lo = i == 0 ? c_abs : 0;
        const uint64_t h_hi = std::min<uint64_t>(group, c_abs + u.it.n_col - (uint64_t)i * group);
        for (uint64_t h = h_lo; h < h_hi; h += hpm) f(i, (uint32_t)h, (uint32_t)std::min<uint64_t>(hpm, h_hi - h));
      }
    };
    auto piece_merges = [&](const PfUnit& u, uint32_t k) {
      uint64_t n = 0;
      for_each_merge(u, k, [&](uint32_t, uint32_t, uint32_t) { n++; });
      return n;
    };
    const size_t pf_slot_bytes = (size_t)ng * (in.hdv + 4) * 4;   // a slot holds the group's heads (ng = group)
    // a unit's pieces (workgroup, first tile) into the lists; a unit of several pieces gets a
    // partial slot per (token, piece) and its merges
    auto emit_pieces = [&](const PfUnit& u, const std::vector<std::pair<uint32_t, uint32_t>>& pieces) {
      const uint32_t k = (uint32_t)pieces.size();
      const uint32_t base = o.slots;
      if (k > 1) {
        for_each_merge(u, k, [&](uint32_t i, uint32_t h, uint32_t nh) {
          o.merges.push_back(MergeItem{u.it.row0 + i, u.it.kvh, h, base + i * k, k, nh});
        });
        o.slots += u.it.n_tok * k;
      }
      for (uint32_t s = 0; s < k; s++) {
        const uint32_t a = pieces[s].second, b = s + 1 < k ? pieces[s + 1].second : u.tiles;
        PrefillItem it = u.it;
        it.page0 = u.it.page0 + 4 * a;
        it.n_pages = std::min(u.it.n_pages, 4 * b) - 4 * a;
        it.slot = k > 1 ? base + s : NO_SLOT;
        it.slot_stride = k > 1 ? k : 0;
        lists.push(pieces[s].first, it);
      }
    };
    if (try_cut) {
      // Walk the units' tiles with a capacity per workgroup: a piece fills the current workgroup
      // (at least PF_MIN_PIECE tiles, and no remainder under PF_MIN_PIECE left behind), the next
      // piece starts on the next workgroup. The capacity is the smallest (to 1%) whose walk fits
      // the workgroups with at most PF_MAX_PIECES pieces per unit.
      std::vector<std::vector<std::pair<uint32_t, uint32_t>>> cuts(units.size());   // (workgroup, first tile)
      auto walk = [&](double c) -> uint32_t {   // workgroups used (UINT32_MAX: a unit over PF_MAX_PIECES)
        uint32_t wg = 0;
        double load = 0.0;
        for (size_t ui = 0; ui < units.size(); ui++) {
          const PfUnit& u = units[ui];
          cuts[ui].clear();
          uint32_t t = 0;
          while (t < u.tiles) {
            if (cuts[ui].size() == PF_MAX_PIECES) return UINT32_MAX;
            const double avail = c - load - PF_UNIT_COST;
            if (avail < PF_MIN_PIECE * u.cpt && load > 0.0) {
              wg++;
              load = 0.0;
              continue;
            }
            uint32_t take = (uint32_t)std::max<double>(PF_MIN_PIECE, avail / u.cpt);
            if (take >= u.tiles - t || u.tiles - t - take < PF_MIN_PIECE) take = u.tiles - t;
            cuts[ui].push_back({wg, t});
            t += take;
            load += PF_UNIT_COST + take * u.cpt;
            if (load >= c - PF_MIN_PIECE * u.cpt) {
              wg++;
              load = 0.0;
            }
          }
        }
        return load > 0.0 ? wg + 1 : wg;
      };
      // the walk over at most n workgroups: the workgroups it uses
      auto walk_fit = [&](uint32_t n) -> uint32_t {
        const double lo0 = (w_cut + PF_UNIT_COST * ((double)units.size() + n)) / n;
        double lo_c = lo0, hi_c = std::max(lo0, max_cost) * 2.0;
        while (walk(hi_c) > n) hi_c *= 2.0;
        for (int i = 0; i < 30 && hi_c > lo_c * 1.01; i++) {
          const double mid = 0.5 * (lo_c + hi_c);
          if (walk(mid) <= n) hi_c = mid;
          else lo_c = mid;
        }
        return walk(hi_c);
      };
      // No-allocation calls: the pieces' partial slots and merges must fit their share of the
      // scratch (half of it beside decode rows, whose splits take the rest; all of it otherwise),
      // so the walk takes half the workgroups until they do.
      auto pf_scratch = [&]() -> size_t {
        uint64_t n_slots = 0, n_merges = 0;
        for (size_t ui = 0; ui < units.size(); ui++) {
          const uint64_t k = cuts[ui].size();
          if (k > 1) {
            n_slots += units[ui].it.n_tok * k;
            n_merges += piece_merges(units[ui], (uint32_t)k);
          }
        }
        return (n_slots * pf_slot_bytes + 255) / 256 * 256 + n_merges * sizeof(MergeItem);
      };
      const size_t pf_budget = decode_tiles > 0 ? in.noalloc_bytes / 2 : in.noalloc_bytes - 256;
      uint32_t n_cap = slots;
      uint32_t n_wg = walk_fit(n_cap);
      bool fits = !in.noalloc || pf_scratch() <= pf_budget;
      while (!fits && n_cap > 1) {
        n_cap /= 2;
        n_wg = walk_fit(n_cap);
        fits = pf_scratch() <= pf_budget;
      }
      // the cut plan's largest load and its merge estimate
      std::vector<double> load(n_wg, 0.0);
      double partials = 0.0;
      for (size_t ui = 0; ui < units.size(); ui++) {
        const PfUnit& u = units[ui];
        const auto& pieces = cuts[ui];
        for (size_t s = 0; s < pieces.size(); s++) {
          const uint32_t b = s + 1 < pieces.size() ? pieces[s + 1].second : u.tiles;
          load[pieces[s].first] += PF_UNIT_COST + (b - pieces[s].second) * u.cpt;
        }
        if (pieces.size() > 1) partials += (double)u.it.n_col * pieces.size();
      }
      const double merge = partials * PF_MERGE_PARTIAL * (in.hdv + 4) / 132.0 +
                           (decode_tiles == 0 && partials > 0 ? PF_MERGE_LAUNCH : 0.0);
      const double cut_load = *std::max_element(load.begin(), load.end()) + merge;
      if (fits && cut_load < PF_CUT_GAIN * whole) {
        pf_load = cut_load;
        lists.reset(n_wg, units.size() + n_wg);
        for (size_t ui = 0; ui < units.size(); ui++) emit_pieces(units[ui], cuts[ui]);
        lists.n_wg = 0;   // workgroups past the last one given a piece stay unlaunched
        for (uint32_t b : lists.wg) lists.n_wg = std::max(lists.n_wg, b + 1);
      }
    }
    // pf_wg lists of pf_per_wg items, each workgroup's items in the order they were added
    o.pf_wg = lists.n_wg;
    std::vector<uint32_t> fill(o.pf_wg, 0);
    for (uint32_t b : lists.wg) o.pf_per_wg = std::max(o.pf_per_wg, ++fill[b]);
    o.pitems.assign((size_t)o.pf_wg * o.pf_per_wg, PrefillItem{});
    std::fill(fill.begin(), fill.end(), 0u);
    for (size_t k = 0; k < lists.wg.size(); k++) {
      const uint32_t b = lists.wg[k];
      PrefillItem it = lists.it[k];
      for (uint32_t i = 0; i < 8; i++) it.blk[i] = blk_at(it.seq, (uint64_t)(it.page0 + std::min(i, it.n_pages - 1)) << 4);
      o.max_pages = std::max(o.max_pages, it.n_pages);
      o.pitems[(size_t)b * o.pf_per_wg + fill[b]++] = it;
    }
    if (in.prefill_lds_fixed + (size_t)o.pf_per_wg * sizeof(PrefillItem) + (size_t)o.max_pages * 4 > in.lds_limit) {
      // key ranges too long to list in LDS: those segments go through the decode kernel
      o.pitems.clear();
      o.merges.clear();
      o.slots = 0;
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
  if (in.noalloc) {
    // what the prompt pieces' partials and merges left of the scratch (each region 256-aligned)
    const size_t used = ((size_t)o.slots * slot_bytes + 255) / 256 * 256 + o.merges.size() * sizeof(MergeItem) + 256;
    const size_t left = in.noalloc_bytes > used ? in.noalloc_bytes - used : 0;
    target = std::max<uint64_t>(1, std::min<uint64_t>(target, left / (slot_bytes + sizeof(MergeItem))));
  }
  // Smallest chunk: 8 tiles for the matrix-core kernels (enough work per wave to stream at full
  // rate); 2 tiles for f32 rows, whose VALU kernel walks keys with dependent loads (latency-bound:
  // more, shorter items hide it better); 4 for the row layout.
  const uint64_t min_chunk = in.decode_min_tiles ? in.decode_min_tiles
                                                 : (in.layout == LAYOUT_ROWS ? 4 : in.kv_type == LMH_KV_F32 ? 2 : 8);
  // chunks of whole tiles, grown until the rows' rounded-up split counts fit the target; at most
  // 128 per item on the matrix-core kernel for f16 / bf16 pages (two block ids per lane), 64 on the
  // others (one). Long rows reach the cap: at 128 their items halve to one wave per SIMD (8 rows x
  // 32 K keys, f16: step 172.5 -> 164.6 us; bf16 170.9 -> 165.3; 16 x 16 K 169.5 -> 163.1), while
  // q8_0, whose tiles carry ~4x the VALU work, needs two waves per SIMD to hide its loads (c4 97.3
  // -> 103.3 us at 128).
  const uint64_t max_chunk = mfma_decode && in.kv_type != LMH_KV_Q8_0 ? MFMA_ITEM_TILES : ITEM_TILES;
  auto n_items_for = [&](uint64_t c) {
    uint64_t n = 0;
    for (uint64_t t = 0; t < n_rows; t++)
      if (o.decode_row[t]) n += (row_tiles(t) + c - 1) / c;
    return n * in.n_kv * head_blocks;
  };
  uint64_t chunk = std::min<uint64_t>(max_chunk, std::max<uint64_t>(min_chunk, (total_tiles + target - 1) / target));
  while (chunk < max_chunk && n_items_for(chunk) > target) chunk++;
  o.chunk = (uint32_t)chunk;
  // Split rows that merge inside their workgroup (no partials in HBM, no merge launch). A row's
  // split count n is 1, 2, 4 or 8 and its items are consecutive waves of one workgroup: groups of
  // 8 go first, then 4, 2 and single items, so no group crosses a workgroup. Not with explicit
  // split settings.
  //  - f32 pages, short rows (at most 16 tiles): 8-wave workgroups; a row splits into items of at
  //    most 2 tiles (the f32 kernel's smallest chunk).
  //  - matrix-core pages, a call of decode rows alone whose rows split at most 4 ways at the
  //    chunk above: the kernel's 4-wave workgroups; a row's split count rounded up to 1, 2 or 4
  //    (items of (chunk/2, chunk] tiles; every item still resident in one round: at most 4/3 of
  //    the target of half the capacity).
  //  - matrix-core pages beside prefill units (one mixed launch): its 8-wave decode workgroups,
  //    split counts rounded up to 1, 2, 4 or 8, the chunk grown (within the item cap) until no row
  //    splits more than 8 ways, as long as the longest item's estimate stays well within the
  //    prefill part's (c5: 992 items of up to 36 tiles and 128 merges in a merge launch become
  //    items of up to 64 tiles merged in place; the decode part finishes long before the prefill).
  uint64_t (*split_of)(uint64_t n_t, uint64_t chunk) = nullptr;
  if (in.layout == LAYOUT_TILES && !in.decode_target_items && !in.decode_min_tiles) {
    uint64_t max_nt = 0;
    for (uint64_t t = 0; t < n_rows; t++)
      if (o.decode_row[t]) max_nt = std::max<uint64_t>(max_nt, row_tiles(t));
    if (in.kv_type == LMH_KV_F32 && in.local_merge_ok && max_nt > 2 && max_nt <= 16) {
      o.local = LOCAL_WAVES;
      split_of = [](uint64_t n_t, uint64_t) -> uint64_t { return n_t <= 2 ? 1 : n_t <= 4 ? 2 : n_t <= 8 ? 4 : 8; };
    } else if (mfma_decode && in.mfma_local_ok && o.pitems.empty() && max_nt > chunk &&
               (max_nt + chunk - 1) / chunk <= (uint64_t)MFMA_LOCAL_WAVES) {
      o.local = MFMA_LOCAL_WAVES;
      split_of = [](uint64_t n_t, uint64_t c) -> uint64_t {
        const uint64_t k = (n_t + c - 1) / c;
        return k <= 1 ? 1 : k <= 2 ? 2 : 4;
      };
    } else if (mfma_decode && in.mfma_local_ok && !o.pitems.empty() && max_nt > chunk) {
      const uint64_t c8 = std::max<uint64_t>(chunk, (max_nt + MIXED_LOCAL_WAVES - 1) / MIXED_LOCAL_WAVES);
      if (c8 <= max_chunk && (double)c8 * DECODE_WAVE_TILE <= MIXED_DECODE_SLACK * pf_load) {
        chunk = c8;
        o.chunk = (uint32_t)c8;
        o.local = MIXED_LOCAL_WAVES;
        split_of = [](uint64_t n_t, uint64_t c) -> uint64_t {
          const uint64_t k = (n_t + c - 1) / c;
          return k <= 1 ? 1 : k <= 2 ? 2 : k <= 4 ? 4 : 8;
        };
      }
    }
  }
  // A row's key range cut into k pieces of whole tiles, [tlo + floor(s n_t / k), tlo +
  // floor((s + 1) n_t / k)) clipped to [lo, pos], with the block id of each piece's first tile:
  // computed once per row (its KV heads and head blocks share them), the floors by increments
  // (q = n_t / k whole tiles each, the remainders carried) instead of two divisions per item.
  struct Piece {
    uint32_t p0, p1, blk0;
  };
  std::vector<Piece> pieces;
  auto cut_row = [&](uint64_t t, uint64_t k) {
    const uint64_t pos = (uint64_t)in.row_pos[t];
    const uint64_t lo = key_lo(pos, window), hi = pos + 1;
    const uint64_t tlo = lo / 16, n_t = pos / 16 - tlo + 1;
    const uint64_t seq = (uint64_t)in.row_seq[t];
    const uint64_t q = n_t / k, r = n_t % k;
    pieces.clear();
    uint64_t a = tlo, carry = 0;
    for (uint64_t s = 0; s < k; s++) {
      uint64_t b = a + q;
      carry += r;
      if (carry >= k) {
        carry -= k;
        b++;
      }
      const uint64_t p0 = std::max(lo, a * 16), p1 = std::min(hi, b * 16);
      pieces.push_back(Piece{(uint32_t)p0, (uint32_t)p1, blk_at(seq, p0)});
      a = b;
    }
  };
  if (o.local) {
    std::vector<DecodeItem> by_size[4];   // groups of 8, 4, 2, single items
    for (uint64_t t = 0; t < n_rows; t++) {
      if (!o.decode_row[t]) continue;
      const uint32_t n = (uint32_t)split_of(row_tiles(t), chunk);
      cut_row(t, n);
      std::vector<DecodeItem>& dst = by_size[n == 8 ? 0 : n == 4 ? 1 : n == 2 ? 2 : 3];
      const uint32_t seq = (uint32_t)in.row_seq[t];
      for (uint32_t kvh = 0; kvh < in.n_kv; kvh++) {
        for (uint32_t hb = 0; hb < head_blocks; hb++) {
          for (uint32_t s = 0; s < n; s++) {
            const uint32_t slot = n == 1 ? NO_SLOT : LOCAL_SLOT | (s << 8) | n;
            dst.push_back(DecodeItem{(uint32_t)t, kvh, hb * ng, pieces[s].p0, pieces[s].p1, slot, seq, pieces[s].blk0});
          }
        }
      }
    }
    for (auto& v : by_size) o.items.insert(o.items.end(), v.begin(), v.end());
    return;
  }
  for (uint64_t t = 0; t < n_rows; t++) {
    if (!o.decode_row[t]) continue;
    const uint64_t n_split = (row_tiles(t) + chunk - 1) / chunk;
    cut_row(t, n_split);
    const uint32_t seq = (uint32_t)in.row_seq[t];
    for (uint32_t kvh = 0; kvh < in.n_kv; kvh++) {
      for (uint32_t hb = 0; hb < head_blocks; hb++) {
        if (n_split == 1) {
          o.items.push_back(DecodeItem{(uint32_t)t, kvh, hb * ng, pieces[0].p0, pieces[0].p1, NO_SLOT, seq, pieces[0].blk0});
          continue;
        }
        o.merges.push_back(MergeItem{(uint32_t)t, kvh, hb * ng, o.slots, (uint32_t)n_split, 0});   // nh 0: ng heads
        for (uint64_t s = 0; s < n_split; s++)
          o.items.push_back(DecodeItem{(uint32_t)t, kvh, hb * ng, pieces[s].p0, pieces[s].p1, o.slots++, seq, pieces[s].blk0});
      }
    }
  }
}

}  // namespace lmh
