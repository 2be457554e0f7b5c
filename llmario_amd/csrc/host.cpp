// host.cpp — the C ABI (include/llmario_hip.h): device page pool, block bookkeeping and the
// attention hand-off for MI355X.
//
// Host-side semantics follow the reference engine exactly where block ids and lengths are
// concerned (they must match bit for bit):
//   BlockPool            crates/engine/kv/src/lib.rs:36-176   (FIFO/LRU free queue, refcounts,
//                                                              content hashes)
//   KvLayout sizes       crates/engine/model/src/kv.rs:402-497 (block_bytes, pool_blocks, ...)
//   KvCache reserve/COW  kv.rs:715-827
//   forward_batch checks crates/engine/model/src/forward.rs:207-291
// The device side is this backend's own: one hipMalloc'd pool of pool_blocks x block_bytes,
// an int32 block table [n_seqs][blocks_per_seq] mirrored to the device when it changes, and a
// per-call packed work list (decode items, split-K slots, merges) that the kernels read straight
// from pinned, device-mapped host memory (no copy on the stream ahead of them).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <queue>
#include <string>
#include <vector>

#include "../../include/llmario_hip.h"
#include "device.h"
#include "kv_hooks.h"
#include "plan.h"
#include "pool.h"

using namespace lmh;

namespace {

thread_local std::string g_create_error;

struct LayerLayout {
  uint32_t n_head, n_kv, hd, hdv;
  uint32_t layout;        // LAYOUT_TILES (matrix-core operand order) or LAYOUT_ROWS (row-major rows)
  bool win;               // sliding-window layer: offsets are inside a window-pool block
  uint64_t k_row, v_row;  // the reference's row bytes (encoded I/O)
  uint32_t k_off, v_off, k_head, v_head, k_tile, v_tile, k_scale, v_scale, k_tile_s, v_tile_s;
};

uint64_t ref_row_bytes(uint32_t t, uint64_t n) {  // kv.rs:94-99 (+ F32/BF16)
  switch (t) {
    case LMH_KV_F16: return 2 * n;
    case LMH_KV_Q8_0: return (n + 31) / 32 * 34;
    case LMH_KV_F32: return 4 * n;
    case LMH_KV_BF16: return 2 * n;
  }
  return 0;
}

// Bytes of one tile of `rows` positions (16, or the whole block when it is smaller) of values
// (codes for q8_0) for `dim` dims, and of its q8_0 scales.
uint32_t tile_bytes(uint32_t t, uint32_t dim, uint32_t rows) {
  switch (t) {
    case LMH_KV_F16:
    case LMH_KV_BF16: return rows * dim * 2;
    case LMH_KV_Q8_0: return rows * dim;
    default: return rows * dim * 4;
  }
}
uint32_t tile_scale_bytes(uint32_t t, uint32_t dim, uint32_t rows) { return t == LMH_KV_Q8_0 ? rows * (dim / 32) * 2 : 0; }
constexpr uint32_t MAX_HEAD_DIM = 512;  // the widest head any kernel takes (Metal's ATTN_MAX_HD)

struct DirtyRows {  // the rows [lo, hi) of a host-side table that differ from the device copy
  uint64_t lo = ~0ull, hi = 0;
  void mark(uint64_t r) {
    lo = std::min(lo, r);
    hi = std::max(hi, r + 1);
  }
  void all(uint64_t n) {
    lo = 0;
    hi = n;
  }
  bool any() const { return lo < hi; }
  void clear() {
    lo = ~0ull;
    hi = 0;
  }
};

// Ring of pinned, device-mapped staging slots (a call's work list, table rows, zero lists), each
// reused only once the work that read it has completed. Work on one stream completes in order, so
// one event covers every use enqueued before it: an event is recorded every EVERY uses (and when
// the stream changes) instead of after each call, since each event record on the stream costs the
// GPU ~3 us between a call's last kernel and the next call's first (c2's step 59.4 -> 57.0 us,
// c1's 14.0 -> 10.9 us, one event per 4 uses; per 8 uses, c2 54.8-55.4 -> 54.4-54.7 us and c4
// 99.5-100.4 -> 98.2-98.5 us on one box).
struct Uploader {
  static constexpr int N = 16;      // slots (N > EVERY: a slot comes round after its use is covered)
  static constexpr int EVERY = 8;   // uses per completion event
  uint8_t* host[N] = {};
  uint8_t* dev[N] = {};  // the device address of host[i]
  size_t cap[N] = {};
  uint64_t use[N] = {};  // the use number of the slot's last use (0: free)
  hipEvent_t ev[N] = {};
  uint64_t ev_use[N] = {};  // ev[k] completes after all work enqueued up to use number ev_use[k] (0: unused)
  int ev_next = 0;
  uint64_t uses = 0, covered = 0;  // uses so far; uses covered by a recorded event
  hipStream_t last = nullptr;      // the stream of the latest use (null is the default stream)
  bool has_last = false;
  int next = 0;
  ~Uploader() {
    for (int i = 0; i < N; i++) {
      if (ev[i]) {
        if (ev_use[i]) (void)hipEventSynchronize(ev[i]);
        (void)hipEventDestroy(ev[i]);
      }
    }
    if (covered < uses) (void)hipDeviceSynchronize();   // uses no event covers (the stream may be gone)
    for (int i = 0; i < N; i++)
      if (host[i]) (void)hipHostFree(host[i]);
  }
  // Every slot allocated up front with at least `bytes`, and every completion event created, so
  // calls on the hot path do not pay for a pinned allocation or an event the first time a slot
  // comes round (and calls that may not allocate never make one).
  hipError_t reserve(size_t bytes) {
    for (int i = 0; i < N; i++) {
      int idx;
      uint8_t* p;
      hipError_t e = acquire(bytes, idx, p);
      if (e == hipSuccess && !ev[i]) e = hipEventCreateWithFlags(&ev[i], hipEventDisableTiming);
      if (e != hipSuccess) return e;
    }
    reserved = bytes;
    return hipSuccess;
  }
  size_t reserved = 0;  // every slot holds at least this many bytes (set at creation)
  // An event after everything enqueued on the latest use's stream so far.
  hipError_t cover() {
    if (covered == uses || !has_last) return hipSuccess;
    const int k = ev_next;
    ev_next = (ev_next + 1) % N;
    hipError_t e;
    if (!ev[k] && (e = hipEventCreateWithFlags(&ev[k], hipEventDisableTiming)) != hipSuccess) return e;
    if (ev_use[k] && (e = hipEventSynchronize(ev[k])) != hipSuccess) return e;  // covers older uses only
    if ((e = hipEventRecord(ev[k], last)) != hipSuccess) return e;
    ev_use[k] = uses;
    covered = uses;
    return hipSuccess;
  }
  // A host buffer of at least `bytes` that no enqueued work still reads. may_grow = false: a slot
  // too small is not reallocated (hipErrorOutOfMemory, nothing allocated): calls that may not
  // allocate stay within the capacity reserved at creation.
  hipError_t acquire(size_t bytes, int& idx, uint8_t*& ptr, bool may_grow = true) {
    if (!may_grow && bytes > reserved) return hipErrorOutOfMemory;
    idx = next;
    next = (next + 1) % N;
    hipError_t e;
    if (use[idx]) {
      if (covered < use[idx] && (e = cover()) != hipSuccess) return e;
      int best = -1;  // the earliest event covering the slot's last use
      for (int k = 0; k < N; k++)
        if (ev_use[k] >= use[idx] && (best < 0 || ev_use[k] < ev_use[best])) best = k;
      if (best >= 0) {
        if ((e = hipEventSynchronize(ev[best])) != hipSuccess) return e;
      } else if ((e = hipDeviceSynchronize()) != hipSuccess) {  // not reached: cover() recorded one
        return e;
      }
      use[idx] = 0;
    }
    if (cap[idx] < bytes) {
      if (host[idx]) (void)hipHostFree(host[idx]);
      host[idx] = nullptr;
      size_t c = std::max<size_t>(bytes, 1 << 16);
      if ((e = hipHostMalloc((void**)&host[idx], c, hipHostMallocMapped | hipHostMallocCoherent)) != hipSuccess) {
        cap[idx] = 0;
        return e;
      }
      if ((e = hipHostGetDevicePointer((void**)&dev[idx], host[idx], 0)) != hipSuccess) return e;
      cap[idx] = c;
    }
    ptr = host[idx];
    return hipSuccess;
  }
  // The slot's contents are in use by work enqueued on `s` so far.
  hipError_t mark(int idx, hipStream_t s) {
    hipError_t e;
    if (has_last && s != last && (e = cover()) != hipSuccess) return e;  // close the previous stream's uses
    last = s;
    has_last = true;
    use[idx] = ++uses;
    if (uses % EVERY == 0) return cover();
    return hipSuccess;
  }
  // The slot's first `bytes` (a multiple of 4) to device memory, copied by a kernel on `s` that
  // reads the mapped slot (a host-to-device copy would run on the copy engine, and the stream's
  // next kernel would wait for its completion signal).
  hipError_t send(int idx, void* dst, size_t bytes, hipStream_t s) {
    hipError_t e = launch_copy_words((uint32_t*)dst, (const uint32_t*)dev[idx], bytes / 4, s);
    if (e != hipSuccess) return e;
    return mark(idx, s);
  }
};

struct DevBuf {  // grow-only device scratch
  void* p = nullptr;
  size_t cap = 0;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
  hipError_t ensure(size_t bytes) {
    if (cap >= bytes) return hipSuccess;
    if (p) {
      (void)hipDeviceSynchronize();  // in-flight work of earlier calls may still read it
      (void)hipFree(p);
      p = nullptr;
      cap = 0;
    }
    size_t c = std::max<size_t>(bytes + bytes / 4, 1 << 16);
    hipError_t e = hipMalloc(&p, c);
    if (e == hipSuccess) cap = c;
    return e;
  }
};

struct Seq {
  std::vector<uint32_t> blocks;
  std::vector<int32_t> wblocks;  // window-pool block by absolute block number (-1: released / none)
  uint64_t len = 0;
};

// Pending device-side page operations queued by host bookkeeping (reserve), run in order at the
// start of the next device call, on that call's stream: zero a freshly backed block (src < 0)
// or copy a shared block for copy-on-write.
struct PageOp {
  int32_t src, dst;
  int32_t win = 0;  // 1: a block of the window pool (zeroing only)
};

}  // namespace

struct lmh_kv {
  // ---- layout
  uint32_t kv_type = 0, bt = 16, bt_shift = 4;
  uint64_t max_ctx = 0, n_seqs = 0, bps = 0, pool_blocks = 0, block_bytes = 0;
  std::vector<LayerLayout> layers;
  // ---- BlockPool (kv/src/lib.rs:36-176)
  BlockPool pool;
  std::vector<uint8_t> backed;
  // ---- window pool (metal/src/kv.rs:37-47): window layers' rows, blocks released behind the window
  uint64_t window = 0;           // width shared by the window layers (0: none)
  uint64_t wblock_bytes = 0, wpool_blocks = 0;
  BlockPool wpool;
  uint8_t* d_wpool = nullptr;
  int32_t* d_wtable = nullptr;
  std::vector<int32_t> h_wtable;
  DirtyRows wtable_rows;
  // ---- sequences
  std::vector<Seq> seqs;
  // ---- device
  int device = 0;
  uint32_t n_cu = 0;                        // compute units of the device
  std::vector<uint32_t> decode_capacity;    // per layer: decode items resident at once (0 = not yet asked)
  uint8_t* d_pool = nullptr;
  int32_t* d_table = nullptr;
  std::vector<int32_t> h_table;
  DirtyRows table_rows;
  std::vector<PageOp> pending;
  Uploader up;
  DevBuf part_buf, merge_buf;
  uint8_t* scratch = nullptr;               // this device's copy of the no-allocation scratch
  // ---- per-call host scratch
  std::vector<int32_t> row_seq, row_pos;
  PlanOut plan;   // the latest lmh_attend call's work lists
  // ---- timing
  bool timing = false;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> evs;
  std::vector<uint32_t> ev_kind;
  size_t ev_used = 0;
  double acc_ms[6] = {0, 0, 0, 0, 0, 0};
  uint64_t launches[6] = {0, 0, 0, 0, 0, 0};
  std::vector<uint8_t> payload;
  std::vector<lmh_sched*> scheds;           // schedulers bound to this handle
  // ---- lmh_attend planning / precision options (lmh_kv_set_tuning)
  bool prefill_p_f16 = false;
  uint64_t prefill_min_rows = 0, decode_target_items = 0, decode_min_tiles = 0;  // 0: defaults
  uint64_t prefill_workgroups = 0;                                                  // 0: every slot
  bool prefill_whole_units = false;   // prefill units never cut into key pieces
  uint32_t prefill_q_split = 0;       // 0: from q_flag; 1: exact-Q launch; 2: hi + lo launch
  // Written by each prefill launch (workgroup 0): whether its first unit's Q has bits below the
  // page type. Pinned and device-mapped, read without waiting: the next call's launch choice.
  volatile uint32_t* q_flag = nullptr;
  uint32_t* q_flag_dev = nullptr;
  std::string err;

  ~lmh_kv() {
    if (d_pool || d_table || d_wpool) (void)hipDeviceSynchronize();
    if (d_pool) (void)hipFree(d_pool);
    if (d_table) (void)hipFree(d_table);
    if (d_wpool) (void)hipFree(d_wpool);
    if (d_wtable) (void)hipFree(d_wtable);
    if (q_flag) (void)hipHostFree((void*)q_flag);
    for (auto& p : evs) {
      (void)hipEventDestroy(p.first);
      (void)hipEventDestroy(p.second);
    }
  }

  int32_t fail(int32_t code, const std::string& m) {
    err = m;
    return code;
  }
  int32_t hip_fail(hipError_t e, const char* what) {
    err = std::string(what) + ": " + hipGetErrorString(e);
    return e == hipErrorOutOfMemory ? LMH_OUT_OF_MEMORY : LMH_DEVICE_ERROR;
  }

  // ---- BlockPool operations --------------------------------------------------------------
  bool pool_alloc(uint64_t n, std::vector<uint32_t>& out) { return pool.alloc(n, out); }  // lib.rs:93-109
  void pool_release(uint32_t b) { pool.release(b); }                                      // lib.rs:121-128
  void pool_clear_hash(uint32_t b) { pool.clear_hash(b); }                                // lib.rs:161-167
  // ---- backing (kv.rs:690-712): a block is resident while referenced or cached
  void back(uint32_t b, bool zero) {
    if (!backed[b]) {
      backed[b] = 1;
      if (zero) pending.push_back({-1, (int32_t)b});
    }
  }
  void maybe_unback(uint32_t b) {
    if (pool.meta[b].refs == 0 && !pool.meta[b].has_hash) backed[b] = 0;
  }
  void release_block(uint32_t b) {
    pool_release(b);
    maybe_unback(b);
  }
  void set_table(uint64_t s) {
    int32_t* row = h_table.data() + s * bps;
    const auto& bl = seqs[s].blocks;
    for (uint64_t i = 0; i < bps; i++) row[i] = i < bl.size() ? (int32_t)bl[i] : -1;
    table_rows.mark(s);
  }

  // ---- window pool (metal/src/kv.rs:304-372) ---------------------------------------------
  // The query at position len sees keys p > len - window: window blocks before this one are dead.
  uint64_t first_live(uint64_t len) const { return (len + 1 > window ? len + 1 - window : 0) / bt; }
  void set_wtable(uint64_t s) {
    int32_t* row = h_wtable.data() + s * bps;
    const auto& wb = seqs[s].wblocks;
    for (uint64_t i = 0; i < bps; i++) row[i] = i < wb.size() ? wb[i] : -1;
    wtable_rows.mark(s);
  }
  // Window blocks reserve_window(s, len, new_len) releases and takes (whole calls are checked
  // before any change, so a short window pool fails like a short paged pool: nothing changes).
  void window_delta(uint64_t s, uint64_t len, uint64_t new_len, uint64_t& take, uint64_t& give) const {
    take = give = 0;
    if (!window) return;
    const auto& wb = seqs[s].wblocks;
    const uint64_t first = first_live(len), need = (new_len + bt - 1) / bt;
    for (uint64_t i = 0; i < std::min<uint64_t>(first, wb.size()); i++) give += wb[i] >= 0 ? 1 : 0;
    for (uint64_t i = std::max<uint64_t>(wb.size(), first); i < need; i++) take++;
  }
  void release_wblock(int32_t& slot) {
    if (slot >= 0) wpool.release((uint32_t)slot);
    slot = -1;
  }
  // Release the window blocks no query from position len on can see, then take blocks (zeroed
  // before the next device call) for every block up to new_len. Checked by window_delta first.
  void reserve_window(uint64_t s, uint64_t len, uint64_t new_len) {
    if (!window) return;
    auto& wb = seqs[s].wblocks;
    const uint64_t first = first_live(len), need = (new_len + bt - 1) / bt;
    for (uint64_t i = 0; i < std::min<uint64_t>(first, wb.size()); i++) release_wblock(wb[i]);
    if (wb.size() < first && wb.size() < need) wb.resize(std::min(first, need), -1);
    while (wb.size() < need) {
      std::vector<uint32_t> nb;
      wpool.alloc(1, nb);
      pending.push_back({-1, (int32_t)nb[0], 1});
      wb.push_back((int32_t)nb[0]);
    }
    set_wtable(s);
  }
  void release_window_from(uint64_t s, uint64_t from) {
    auto& wb = seqs[s].wblocks;
    while (wb.size() > from) {
      release_wblock(wb.back());
      wb.pop_back();
    }
    set_wtable(s);
  }
  // every window block a row at position pos of sequence s touches is live: its own (lo = pos)
  // or those of its attention range [lo, pos]
  bool window_live(uint64_t s, uint64_t lo, uint64_t hi) const {
    const auto& wb = seqs[s].wblocks;
    for (uint64_t b = lo / bt; b <= hi / bt; b++)
      if (b >= wb.size() || wb[b] < 0) return false;
    return true;
  }

  // kv.rs:715-725
  uint64_t blocks_needed(uint64_t s, uint64_t new_len) const {
    const Seq& q = seqs[s];
    const uint64_t want = (new_len + bt - 1) / bt;
    const uint64_t missing = want > q.blocks.size() ? want - q.blocks.size() : 0;
    const bool cow = q.len % bt != 0 && q.len < new_len && pool.meta[q.blocks[q.len / bt]].refs > 1;
    return missing + (cow ? 1 : 0);
  }

  // kv.rs:730-785
  int32_t reserve(uint64_t s, uint64_t new_len, uint64_t* needed, uint64_t* free_blocks, bool with_window = true) {
    if (new_len > max_ctx) return fail(LMH_INVALID_ARGUMENT, "context overflow");
    const uint64_t len = seqs[s].len;
    const uint64_t want = (new_len + bt - 1) / bt;
    const uint64_t missing = want > seqs[s].blocks.size() ? want - seqs[s].blocks.size() : 0;
    const uint64_t wanted = blocks_needed(s, new_len);
    const bool cow = wanted > missing;
    if (pool.free_blocks() < wanted) {
      if (needed) *needed = wanted;
      if (free_blocks) *free_blocks = pool.free_blocks();
      return fail(LMH_KV_FULL, "KV cache full: " + std::to_string(wanted) + " more blocks needed, " +
                                   std::to_string(pool.free_blocks()) + " free");
    }
    uint64_t w_take = 0, w_give = 0;
    if (with_window) window_delta(s, len, new_len, w_take, w_give);
    if (w_take > wpool.free_blocks() + w_give) {
      if (needed) *needed = w_take;
      if (free_blocks) *free_blocks = wpool.free_blocks() + w_give;
      return fail(LMH_KV_FULL, "window pool full: " + std::to_string(w_take) + " window blocks needed, " +
                                   std::to_string(wpool.free_blocks() + w_give) + " free");
    }
    if (with_window) reserve_window(s, len, new_len);
    if (len % bt != 0 && len < new_len) {
      const uint64_t bi = len / bt;
      const uint32_t old = seqs[s].blocks[bi];
      if (cow) {
        std::vector<uint32_t> nb;
        pool_alloc(1, nb);
        back(nb[0], false);  // fully overwritten by the copy below
        pending.push_back({(int32_t)old, (int32_t)nb[0]});
        seqs[s].blocks[bi] = nb[0];
        release_block(old);
      } else {
        pool_clear_hash(old);
      }
    }
    if (missing > 0) {
      std::vector<uint32_t> fresh;
      pool_alloc(missing, fresh);
      for (uint32_t b : fresh) {
        back(b, true);
        seqs[s].blocks.push_back(b);
      }
    }
    set_table(s);
    return LMH_OK;
  }

  // kv.rs:792-816 (paged layers: no rings, no recurrent state)
  void truncate(uint64_t s, uint64_t n) {
    n = std::min(n, seqs[s].len);
    // metal/src/kv.rs:393-405: when a window block the next query needs is already released,
    // the whole sequence is cleared instead
    if (window && n > 0) {
      const uint64_t last = (n + bt - 1) / bt;
      for (uint64_t i = first_live(n); i < last; i++)
        if (i >= seqs[s].wblocks.size() || seqs[s].wblocks[i] < 0) {
          n = 0;
          break;
        }
    }
    seqs[s].len = n;
    const uint64_t keep = (n + bt - 1) / bt;
    while (seqs[s].blocks.size() > keep) {
      const uint32_t b = seqs[s].blocks.back();
      seqs[s].blocks.pop_back();
      release_block(b);
    }
    set_table(s);
    if (window) release_window_from(s, keep);
  }
  void clear(uint64_t s) {  // kv.rs:820-827
    seqs[s].len = 0;
    while (!seqs[s].blocks.empty()) {
      const uint32_t b = seqs[s].blocks.back();
      seqs[s].blocks.pop_back();
      release_block(b);
    }
    set_table(s);
    if (window) release_window_from(s, 0);
  }

  // ---- device helpers --------------------------------------------------------------------
  int32_t flush(hipStream_t st) {
    hipError_t e;
    if (hipSetDevice(device) != hipSuccess) return fail(LMH_DEVICE_ERROR, "hipSetDevice failed");
    size_t i = 0;
    while (i < pending.size()) {
      if (pending[i].src < 0) {
        // block ids in pieces no larger than a staging slot's reserved bytes, so flushing never
        // grows the staging ring
        size_t j = i;
        std::vector<int32_t> zb;
        const int32_t w = pending[i].win;
        const size_t max_ids = std::max<size_t>(up.reserved / 4, 1);
        while (j < pending.size() && pending[j].src < 0 && pending[j].win == w && zb.size() < max_ids)
          zb.push_back(pending[j++].dst);
        int idx;
        uint8_t* h;
        if ((e = up.acquire(zb.size() * 4, idx, h)) != hipSuccess) return hip_fail(e, "staging");
        std::memcpy(h, zb.data(), zb.size() * 4);
        // the zero kernel reads the block ids from the mapped staging slot
        if ((e = launch_zero_blocks(w ? d_wpool : d_pool, w ? wblock_bytes : block_bytes, (const int32_t*)up.dev[idx],
                                    (uint32_t)zb.size(), st)) != hipSuccess)
          return hip_fail(e, "zero kernel");
        if ((e = up.mark(idx, st)) != hipSuccess) return hip_fail(e, "event");
        i = j;
      } else {
        e = hipMemcpyAsync(d_pool + (size_t)pending[i].dst * block_bytes,
                           d_pool + (size_t)pending[i].src * block_bytes, block_bytes, hipMemcpyDeviceToDevice, st);
        if (e != hipSuccess) return hip_fail(e, "copy-on-write");
        i++;
      }
    }
    pending.clear();
    // the block-table rows changed since the last upload (one copy spanning them)
    // (in pieces of at most a staging slot's reserved bytes)
    auto upload = [&](DirtyRows& d, const std::vector<int32_t>& h_tab, int32_t* d_tab) -> int32_t {
      if (!d.any()) return LMH_OK;
      const size_t off = d.lo * bps, bytes = (d.hi - d.lo) * bps * 4;
      const size_t piece = std::max<size_t>(up.reserved / 4 * 4, 4);
      for (size_t done = 0; done < bytes; done += piece) {
        const size_t n = std::min(piece, bytes - done);
        int idx;
        uint8_t* h;
        if ((e = up.acquire(n, idx, h)) != hipSuccess) return hip_fail(e, "staging");
        std::memcpy(h, (const uint8_t*)(h_tab.data() + off) + done, n);
        if ((e = up.send(idx, (uint8_t*)(d_tab + off) + done, n, st)) != hipSuccess) return hip_fail(e, "table upload");
      }
      d.clear();
      return LMH_OK;
    };
    int32_t rc = upload(table_rows, h_table, d_table);
    if (rc == LMH_OK && window) rc = upload(wtable_rows, h_wtable, d_wtable);
    return rc;
  }

  PageGeom geom(uint32_t l) const {
    const LayerLayout& y = layers[l];
    PageGeom g{};
    g.pool = y.win ? d_wpool : d_pool;
    g.block_bytes = y.win ? wblock_bytes : block_bytes;
    g.k_off = y.k_off;
    g.v_off = y.v_off;
    g.k_head = y.k_head;
    g.v_head = y.v_head;
    g.k_tile = y.k_tile;
    g.v_tile = y.v_tile;
    g.k_scale = y.k_scale;
    g.v_scale = y.v_scale;
    g.k_tile_s = y.k_tile_s;
    g.v_tile_s = y.v_tile_s;
    g.bt_shift = bt_shift;
    g.bps = (uint32_t)bps;
    g.table = y.win ? d_wtable : d_table;
    g.kv_type = kv_type;
    g.n_kv = y.n_kv;
    g.hd = y.hd;
    g.hdv = y.hdv;
    g.layout = y.layout;
    return g;
  }

  // A window layer's rows exist only while their window blocks are live: every row of the segments
  // must have its own block live (store / gather), or, with attn_window > 0, every block of its
  // attention range [pos + 1 - attn_window, pos] (attend).
  int32_t check_window_rows(uint32_t layer, const lmh_seg* segs, uint64_t n_segs, uint64_t attn_window) {
    if (!layers[layer].win) return LMH_OK;
    for (uint64_t i = 0; i < n_segs; i++) {
      const lmh_seg& sg = segs[i];
      if (sg.n == 0) continue;
      const uint64_t first = sg.pos0, last = sg.pos0 + sg.n - 1;
      const uint64_t lo = attn_window == 0 ? first : (first + 1 > attn_window ? first + 1 - attn_window : 0);
      if (!window_live(sg.seq, lo, last))
        return fail(LMH_INVALID_ARGUMENT, "window layer rows outside the sequence's live window blocks");
    }
    return LMH_OK;
  }

  // Validate segments against the tables; fill row_seq/row_pos. Rows must be stacked in segment
  // order (start = running row count), as Rows::push builds them (forward.rs:63-77).
  int32_t rows_from(const lmh_seg* segs, uint64_t n_segs, uint64_t& n_rows) {
    row_seq.clear();
    row_pos.clear();
    n_rows = 0;
    if (n_segs > 0 && !segs) return fail(LMH_INVALID_ARGUMENT, "null segments");
    for (uint64_t i = 0; i < n_segs; i++) {
      const lmh_seg& sg = segs[i];
      if (sg.seq >= n_seqs) return fail(LMH_INVALID_ARGUMENT, "segment sequence out of range");
      if (sg.start != n_rows) return fail(LMH_INVALID_ARGUMENT, "segments must stack rows in order");
      if (sg.pos0 + sg.n > seqs[sg.seq].blocks.size() * bt)
        return fail(LMH_INVALID_ARGUMENT, "segment positions beyond the sequence's reserved blocks");
      if (sg.pos0 + sg.n > 0x7fffffffull) return fail(LMH_INVALID_ARGUMENT, "position too large");
      for (uint64_t j = 0; j < sg.n; j++) {
        row_seq.push_back((int32_t)sg.seq);
        row_pos.push_back((int32_t)(sg.pos0 + j));
      }
      n_rows += sg.n;
    }
    if (n_rows > 0x7fffffffull) return fail(LMH_INVALID_ARGUMENT, "too many rows");
    return LMH_OK;
  }

  // Stage row arrays plus up to two payloads (each 256-byte aligned, back to back) in a pinned,
  // device-mapped staging slot: the kernels read this per-call metadata straight from host memory
  // (a few dozen bytes per wave), so no copy has to run on the stream before them. The caller
  // enqueues every kernel that reads the slot, then calls release_rows(slot, stream).
  int32_t stage_rows(const void* extra, size_t extra_bytes, const void* extra2, size_t extra2_bytes,
                     const int32_t*& d_rs, const int32_t*& d_rp, const uint8_t*& d_extra, int& slot,
                     bool may_grow = true) {
    const size_t nr = row_seq.size();
    const size_t rows_bytes = (nr * 8 + 255) / 256 * 256;
    const size_t extra_pad = (extra_bytes + 255) / 256 * 256;
    const size_t total = rows_bytes + extra_pad + extra2_bytes;
    hipError_t e;
    uint8_t* h;
    if (!may_grow && total > up.reserved)
      return fail(LMH_INVALID_ARGUMENT, "the call's work list (" + std::to_string(total) +
                                            " bytes) exceeds the staging capacity reserved at creation (" +
                                            std::to_string(up.reserved) + " bytes)");
    if ((e = up.acquire(total, slot, h, may_grow)) != hipSuccess) return hip_fail(e, "staging");
    std::memcpy(h, row_seq.data(), nr * 4);
    std::memcpy(h + nr * 4, row_pos.data(), nr * 4);
    if (extra_bytes) std::memcpy(h + rows_bytes, extra, extra_bytes);
    if (extra2_bytes) std::memcpy(h + rows_bytes + extra_pad, extra2, extra2_bytes);
    uint8_t* d = up.dev[slot];
    d_rs = (const int32_t*)d;
    d_rp = d_rs + nr;
    d_extra = d + rows_bytes;
    return LMH_OK;
  }
  int32_t release_rows(int slot, hipStream_t st) {
    hipError_t e = up.mark(slot, st);
    return e == hipSuccess ? LMH_OK : hip_fail(e, "event");
  }

  // Event pairs around one kernel launch of kind LMH_KERNEL_* (timing hook for benchmarks).
  hipError_t time_begin(hipStream_t st, uint32_t kind) {
    if (!timing) return hipSuccess;
    if (ev_used == evs.size()) {
      hipEvent_t a, b;
      hipError_t e = hipEventCreate(&a);
      if (e == hipSuccess) e = hipEventCreate(&b);
      if (e != hipSuccess) return e;
      evs.push_back({a, b});
      ev_kind.push_back(0);
    }
    ev_kind[ev_used] = kind;
    return hipEventRecord(evs[ev_used].first, st);
  }
  // The same pair for a launch that records it itself (LaunchEv: start and stop are stamped by the
  // kernel's dispatch), so the interval is the kernel alone. Empty when timing is off.
  hipError_t time_launch(uint32_t kind, LaunchEv& ev) {
    ev = LaunchEv{};
    if (!timing) return hipSuccess;
    if (ev_used == evs.size()) {
      hipEvent_t a, b;
      hipError_t e = hipEventCreate(&a);
      if (e == hipSuccess) e = hipEventCreate(&b);
      if (e != hipSuccess) return e;
      evs.push_back({a, b});
      ev_kind.push_back(0);
    }
    ev_kind[ev_used] = kind;
    ev.start = evs[ev_used].first;
    ev.stop = evs[ev_used].second;
    ev_used++;
    return hipSuccess;
  }
  hipError_t time_end(hipStream_t st) {
    if (!timing) return hipSuccess;
    hipError_t e = hipEventRecord(evs[ev_used].second, st);
    ev_used++;
    return e;
  }
  // Fold recorded pairs into the per-kind totals.
  hipError_t collect_times() {
    for (size_t i = 0; i < ev_used; i++) {
      float t = 0;
      hipError_t e = hipEventSynchronize(evs[i].second);
      if (e == hipSuccess) e = hipEventElapsedTime(&t, evs[i].first, evs[i].second);
      if (e != hipSuccess) return e;
      acc_ms[ev_kind[i]] += t;
      launches[ev_kind[i]]++;
    }
    ev_used = 0;
    return hipSuccess;
  }
};

namespace {

// FNV-1a (kv.rs:944-960 StableHasher)
struct Fnv {
  uint64_t h = 0xcbf29ce484222325ull;
  void bytes(const void* p, size_t n) {
    const uint8_t* b = (const uint8_t*)p;
    for (size_t i = 0; i < n; i++) h = (h ^ b[i]) * 0x00000100000001b3ull;
  }
  void u64(uint64_t v) { bytes(&v, 8); }
};

}  // namespace

// =============================================================================================
// C ABI
// =============================================================================================

// ---- hooks for the scheduler (kv_hooks.h) ----
namespace lmh {
BlockPool& kv_pool(lmh_kv* kv) { return kv->pool; }
uint64_t kv_n_seqs(const lmh_kv* kv) { return kv->n_seqs; }
uint64_t kv_max_ctx(const lmh_kv* kv) { return kv->max_ctx; }
bool kv_has_window(const lmh_kv* kv) { return kv->window > 0; }
uint64_t kv_seq_len(const lmh_kv* kv, uint64_t seq) { return kv->seqs[seq].len; }
bool kv_seq_empty(const lmh_kv* kv, uint64_t seq) { return kv->seqs[seq].blocks.empty() && kv->seqs[seq].len == 0; }
const std::vector<uint32_t>& kv_seq_blocks(const lmh_kv* kv, uint64_t seq) { return kv->seqs[seq].blocks; }
void kv_bind_seq(lmh_kv* kv, uint64_t seq, const std::vector<uint32_t>& blocks, uint64_t len) {
  for (uint32_t b : blocks) kv->back(b, true);
  kv->seqs[seq].blocks = blocks;
  kv->seqs[seq].len = len;
  kv->set_table(seq);
}
void kv_clear_seq(lmh_kv* kv, uint64_t seq) { kv->clear(seq); }
void kv_set_error(lmh_kv* kv, const char* msg) { kv->err = msg; }
void kv_attach(lmh_kv* kv, lmh_sched* s) { kv->scheds.push_back(s); }
void kv_detach(lmh_kv* kv, lmh_sched* s) {
  kv->scheds.erase(std::remove(kv->scheds.begin(), kv->scheds.end(), s), kv->scheds.end());
}
}  // namespace lmh

extern "C" {

const char* lmh_create_error(void) { return g_create_error.c_str(); }

int32_t lmh_kv_create(const lmh_kv_options* o, lmh_kv** out) {
  g_create_error.clear();
  if (!o || !out) {
    g_create_error = "null argument";
    return LMH_INVALID_ARGUMENT;
  }
  *out = nullptr;
  if (o->abi_version != LMH_ABI_VERSION) {
    g_create_error = "ABI version mismatch";
    return LMH_INVALID_ARGUMENT;
  }
  if (o->kv_type > LMH_KV_BF16) {
    g_create_error = "unknown KV type";
    return LMH_INVALID_ARGUMENT;
  }
  const uint32_t bt = o->block_tokens;
  if (bt == 0 || (bt & (bt - 1)) != 0) {  // kv.rs:403-406
    g_create_error = "block size must be a power of two";
    return LMH_INVALID_ARGUMENT;
  }
  if (o->n_layers == 0 || !o->layers) {
    g_create_error = "no attention layers";
    return LMH_INVALID_ARGUMENT;
  }
  lmh_kv* kv = new (std::nothrow) lmh_kv();
  if (!kv) return LMH_OUT_OF_MEMORY;
  kv->kv_type = o->kv_type;
  kv->bt = bt;
  kv->bt_shift = 0;
  while ((1u << kv->bt_shift) < bt) kv->bt_shift++;
  kv->max_ctx = std::max<uint64_t>(o->max_ctx, 1);
  kv->n_seqs = std::max<uint64_t>(o->n_seqs, 1);
  // KvLayout::new (kv.rs:402-497): per layer K rows then V rows of bt positions; same byte totals.
  // Window layers (which the reference keeps in rings, outside the block) go to the window pool's
  // blocks, laid out the same way (metal/src/kv.rs:111-126).
  uint64_t off = 0, woff = 0;
  for (uint32_t l = 0; l < o->n_layers; l++) {
    const lmh_layer_desc& d = o->layers[l];
    if (d.window > 0 && kv->window > 0 && d.window != kv->window) {
      delete kv;
      g_create_error = "sliding-window layers with different widths";
      return LMH_UNSUPPORTED;
    }
    if (d.window > 0) kv->window = d.window;
    if (d.n_kv == 0 || d.n_head == 0 || d.n_head % d.n_kv != 0 || d.hd == 0 || d.hdv == 0) {
      delete kv;
      g_create_error = "bad layer geometry";
      return LMH_INVALID_ARGUMENT;
    }
    if (o->kv_type == LMH_KV_Q8_0 && (d.hd % 32 != 0 || d.hdv % 32 != 0)) {  // kv.rs:103-109
      delete kv;
      g_create_error = "q8_0 cannot hold heads that are not a multiple of 32 wide";
      return LMH_INVALID_ARGUMENT;
    }
    if (d.hd > MAX_HEAD_DIM || d.hdv > MAX_HEAD_DIM) {  // Metal refuses the same (backend.rs:574-580)
      delete kv;
      g_create_error = "head widths above 512 are not supported";
      return LMH_UNSUPPORTED;
    }
    LayerLayout y{};
    y.n_head = d.n_head;
    y.n_kv = d.n_kv;
    y.hd = d.hd;
    y.hdv = d.hdv;
    // tiles in matrix-core operand order where a decode instance takes the geometry; otherwise
    // (other widths, hd != hdv without an instance, blocks under 16 positions) row-major rows
    y.layout = (bt >= 16 && decode_tiles_supported(o->kv_type, d.hd, d.hdv)) ? LAYOUT_TILES : LAYOUT_ROWS;
    y.k_row = ref_row_bytes(o->kv_type, (uint64_t)d.n_kv * d.hd);
    y.v_row = ref_row_bytes(o->kv_type, (uint64_t)d.n_kv * d.hdv);
    const uint32_t rows = std::min<uint32_t>(bt, 16), tiles = bt / rows;
    y.k_tile = tile_bytes(o->kv_type, d.hd, rows);
    y.v_tile = tile_bytes(o->kv_type, d.hdv, rows);
    y.k_tile_s = tile_scale_bytes(o->kv_type, d.hd, rows);
    y.v_tile_s = tile_scale_bytes(o->kv_type, d.hdv, rows);
    y.k_scale = tiles * y.k_tile;
    y.v_scale = tiles * y.v_tile;
    y.k_head = tiles * (y.k_tile + y.k_tile_s);
    y.v_head = tiles * (y.v_tile + y.v_tile_s);
    y.win = d.window > 0;
    uint64_t& o_ = y.win ? woff : off;
    y.k_off = (uint32_t)o_;
    o_ += (uint64_t)d.n_kv * y.k_head;
    y.v_off = (uint32_t)o_;
    o_ += (uint64_t)d.n_kv * y.v_head;
    kv->layers.push_back(y);
  }
  if (off == 0) {
    delete kv;
    g_create_error = "every layer is a window layer (at least one full-attention layer is needed)";
    return LMH_UNSUPPORTED;
  }
  kv->block_bytes = off;
  kv->wblock_bytes = woff;
  kv->bps = (kv->max_ctx + bt - 1) / bt;
  if (o->pool_tokens > 0) {
    const uint64_t t = o->pool_tokens;
    kv->pool_blocks = std::min((t + bt - 1) / bt, kv->n_seqs * kv->bps) + kv->n_seqs;
  } else {
    kv->pool_blocks = kv->n_seqs * (kv->bps + 1);
  }
  if (kv->pool_blocks > 0x7fffffffull) {
    delete kv;
    g_create_error = "pool too large";
    return LMH_INVALID_ARGUMENT;
  }
  kv->pool.init(kv->pool_blocks, bt);
  kv->backed.assign(kv->pool_blocks, 0);
  kv->seqs.assign(kv->n_seqs, Seq{});
  kv->h_table.assign(kv->n_seqs * kv->bps, -1);
  kv->table_rows.all(kv->n_seqs);
  if (kv->window) {
    // metal/src/kv.rs:130-133: a sequence's live window blocks are the window behind its first new
    // token plus one call's tokens, and a partial block at each end
    const uint64_t n_batch = o->n_batch ? o->n_batch : 512;
    kv->wpool_blocks = kv->n_seqs * std::min<uint64_t>((kv->window + n_batch + bt - 1) / bt + 1, kv->bps);
    kv->wpool.init(kv->wpool_blocks, bt);
    kv->h_wtable.assign(kv->n_seqs * kv->bps, -1);
    kv->wtable_rows.all(kv->n_seqs);
  }
  kv->device = o->device;
  hipError_t e = hipSetDevice(o->device);
  int n_cu = 0;
  if (e == hipSuccess) e = hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, o->device);
  kv->n_cu = (uint32_t)std::max(n_cu, 1);
  kv->decode_capacity.assign(kv->layers.size(), 0);
  if (e == hipSuccess) e = hipMalloc((void**)&kv->d_pool, kv->pool_blocks * kv->block_bytes);
  if (e == hipSuccess) e = hipMalloc((void**)&kv->d_table, std::max<uint64_t>(kv->h_table.size(), 1) * 4);
  if (e == hipSuccess && kv->window) e = hipMalloc((void**)&kv->d_wpool, kv->wpool_blocks * kv->wblock_bytes);
  if (e == hipSuccess && kv->window) e = hipMalloc((void**)&kv->d_wtable, kv->h_wtable.size() * 4);
  // staging slots sized for a call's work list (decode items, merges, prefill units: 1 MiB holds
  // ~32 K decode items) and 16 block-table rows, so calls do not grow them
  if (e == hipSuccess) e = kv->up.reserve(std::max<size_t>(1 << 20, kv->bps * 4 * 16));
  // this device's copy of lmh_attend_noalloc's scratch (resolved once per device)
  if (e == hipSuccess) e = noalloc_scratch(o->device, &kv->scratch);
  if (e == hipSuccess) {
    void* f = nullptr;
    e = hipHostMalloc(&f, 256, hipHostMallocMapped | hipHostMallocCoherent);
    if (e == hipSuccess) {
      kv->q_flag = (volatile uint32_t*)f;
      *kv->q_flag = 0;
      e = hipHostGetDevicePointer((void**)&kv->q_flag_dev, f, 0);
    }
  }
  if (e != hipSuccess) {
    g_create_error = std::string("device allocation failed: ") + hipGetErrorString(e);
    delete kv;
    return e == hipErrorOutOfMemory ? LMH_OUT_OF_MEMORY : LMH_DEVICE_ERROR;
  }
  *out = kv;
  return LMH_OK;
}

void lmh_kv_destroy(lmh_kv* kv) {
  if (!kv) return;
  for (lmh_sched* s : kv->scheds) sched_kv_destroyed(s);
  delete kv;
}

const char* lmh_kv_last_error(const lmh_kv* kv) { return kv ? kv->err.c_str() : "null handle"; }

int32_t lmh_kv_layout(const lmh_kv* kv, lmh_layout_info* out) {
  if (!kv || !out) return LMH_INVALID_ARGUMENT;
  out->block_bytes = kv->block_bytes;
  out->blocks_per_seq = kv->bps;
  out->n_seqs = kv->n_seqs;
  out->pool_blocks = kv->pool_blocks;
  out->max_ctx = kv->max_ctx;
  out->block_tokens = kv->bt;
  out->kv_type = kv->kv_type;
  return LMH_OK;
}

uint64_t lmh_kv_fingerprint(const lmh_kv* kv) {
  if (!kv) return 0;
  Fnv h;
  h.bytes("hip", 3);
  const uint32_t one = 1;
  h.bytes(&one, 1);  // little-endian tag
  h.u64(kv->kv_type);
  h.u64(kv->bt);
  h.u64(kv->block_bytes);
  h.u64(kv->max_ctx);
  h.u64(kv->window);
  h.u64(kv->wblock_bytes);
  for (const auto& y : kv->layers) {
    h.u64(y.win ? 1 : 0);
    h.u64(y.n_kv);
    h.u64(y.hd);
    h.u64(y.hdv);
    h.u64(y.k_off);
    h.u64(y.v_off);
    h.u64(y.k_head);
    h.u64(y.v_head);
  }
  return h.h;
}

int32_t lmh_kv_seq_len(const lmh_kv* kv, uint64_t seq, uint64_t* len) {
  if (!kv || !len || seq >= kv->n_seqs) return LMH_INVALID_ARGUMENT;
  *len = kv->seqs[seq].len;
  return LMH_OK;
}

int32_t lmh_kv_set_seq_len(lmh_kv* kv, uint64_t seq, uint64_t len) {
  if (!kv || seq >= kv->n_seqs) return LMH_INVALID_ARGUMENT;
  if (len > kv->seqs[seq].blocks.size() * kv->bt) return kv->fail(LMH_INVALID_ARGUMENT, "length beyond reserved blocks");
  if (kv->window) {  // the window blocks the next query can see: [first_live(len), ceil(len / bt))
    uint64_t take, give;
    kv->window_delta(seq, len, len, take, give);
    if (take > kv->wpool.free_blocks() + give) return kv->fail(LMH_KV_FULL, "window pool full");
    kv->reserve_window(seq, len, len);
  }
  kv->seqs[seq].len = len;
  return LMH_OK;
}

int32_t lmh_kv_free_blocks(const lmh_kv* kv, uint64_t* n) {
  if (!kv || !n) return LMH_INVALID_ARGUMENT;
  *n = kv->pool.free_blocks();
  return LMH_OK;
}

int32_t lmh_kv_resident_blocks(const lmh_kv* kv, uint64_t* n) {
  if (!kv || !n) return LMH_INVALID_ARGUMENT;
  uint64_t c = 0;
  for (uint8_t b : kv->backed) c += b;
  *n = c;
  return LMH_OK;
}

int32_t lmh_kv_blocks_needed(const lmh_kv* kv, uint64_t seq, uint64_t new_len, uint64_t* needed) {
  if (!kv || !needed || seq >= kv->n_seqs) return LMH_INVALID_ARGUMENT;
  *needed = kv->blocks_needed(seq, new_len);
  return LMH_OK;
}

int32_t lmh_kv_reserve(lmh_kv* kv, uint64_t seq, uint64_t new_len, uint64_t* needed, uint64_t* free_blocks) {
  if (!kv || seq >= kv->n_seqs) return LMH_INVALID_ARGUMENT;
  return kv->reserve(seq, new_len, needed, free_blocks);
}

int32_t lmh_kv_truncate(lmh_kv* kv, uint64_t seq, uint64_t n) {
  if (!kv || seq >= kv->n_seqs) return LMH_INVALID_ARGUMENT;
  kv->truncate(seq, n);
  return LMH_OK;
}

int32_t lmh_kv_clear(lmh_kv* kv, uint64_t seq) {
  if (!kv || seq >= kv->n_seqs) return LMH_INVALID_ARGUMENT;
  kv->clear(seq);
  return LMH_OK;
}

// ---- snapshots (kv.rs:1009-1130), paged layers: whole blocks in the reference's block format ----
// With window layers, the paged blocks are followed by the window blocks a query after len can
// still see, [first_live(len), ceil(len / bt)), each in the same block format restricted to the
// window layers (Metal's snapshot, metal/src/kv.rs:455-490).
static void window_span(const lmh_kv* kv, uint64_t len, uint64_t& first, uint64_t& end) {
  first = end = 0;
  if (!kv->window) return;
  first = kv->first_live(len);
  end = std::max<uint64_t>((len + kv->bt - 1) / kv->bt, first);
}

int32_t lmh_kv_snapshot_bytes(const lmh_kv* kv, uint64_t len, uint64_t* bytes) {
  if (!kv || !bytes) return LMH_INVALID_ARGUMENT;
  uint64_t first, end;
  window_span(kv, len, first, end);
  *bytes = len == 0 ? 0 : (len + kv->bt - 1) / kv->bt * kv->block_bytes + (end - first) * kv->wblock_bytes;
  return LMH_OK;
}

// One launch per layer over the positions of the sequence's first n_blocks blocks; the layer's
// region of a reference block starts after the earlier layers' bt*(k_row + v_row) bytes
// (KvLayout::new, kv.rs:402-497).
// Window layers: the same per block, over window blocks first..end of the window table (the
// table row is entered at `first`, so the kernels' block index counts from there) after the paged part.
static int32_t snapshot_layers(lmh_kv* kv, bool write, uint64_t seq, uint64_t n_blocks, uint8_t* bytes,
                               hipStream_t st) {
  uint64_t first, end;
  window_span(kv, kv->seqs[seq].len, first, end);
  uint64_t ref_off = 0, wref_off = 0;
  for (uint32_t l = 0; l < kv->layers.size(); l++) {
    const LayerLayout& y = kv->layers[l];
    PageGeom g = kv->geom(l);
    uint64_t n_pos = n_blocks * kv->bt, bb = kv->block_bytes, off = ref_off;
    uint8_t* at = bytes;
    if (y.win) {
      g.table += first;
      n_pos = (end - first) * kv->bt;
      bb = kv->wblock_bytes;
      off = wref_off;
      at = bytes + n_blocks * kv->block_bytes;
    }
    hipError_t e = kv->time_begin(st, LMH_KERNEL_SNAPSHOT);
    if (e == hipSuccess)
      e = launch_snapshot(write, g, (uint32_t)seq, (uint32_t)n_pos, kv->bt, bb, off, (uint32_t)y.k_row, (uint32_t)y.v_row,
                          at, st);
    if (e == hipSuccess) e = kv->time_end(st);
    if (e != hipSuccess) return kv->hip_fail(e, "snapshot kernel");
    (y.win ? wref_off : ref_off) += kv->bt * (y.k_row + y.v_row);
  }
  return LMH_OK;
}

// backend.rs:64; Metal's rule (metal/src/backend.rs:2141-2143): no window layer (this cache holds
// no recurrent state)
int32_t lmh_kv_snapshot_trimmable(const lmh_kv* kv, int32_t* trimmable) {
  if (!kv || !trimmable) return LMH_INVALID_ARGUMENT;
  *trimmable = kv->window == 0 ? 1 : 0;
  return LMH_OK;
}

int32_t lmh_kv_write_seq(lmh_kv* kv, uint64_t seq, void* dst, uint64_t cap, uint64_t* written, void* stream) {
  if (!kv || seq >= kv->n_seqs) return LMH_INVALID_ARGUMENT;
  const uint64_t len = kv->seqs[seq].len;
  uint64_t bytes;
  lmh_kv_snapshot_bytes(kv, len, &bytes);
  if (written) *written = bytes;
  if (bytes == 0) return LMH_OK;
  if (!dst || cap < bytes) return kv->fail(LMH_INVALID_ARGUMENT, "snapshot destination smaller than snapshot_bytes(len)");
  uint64_t first, end;
  window_span(kv, len, first, end);
  if (end > first && !kv->window_live(seq, first * kv->bt, end * kv->bt - 1))
    return kv->fail(LMH_INVALID_ARGUMENT, "a window block the snapshot needs is not live");
  hipStream_t st = (hipStream_t)stream;
  int32_t rc = kv->flush(st);
  if (rc != LMH_OK) return rc;
  return snapshot_layers(kv, true, seq, (len + kv->bt - 1) / kv->bt, (uint8_t*)dst, st);
}

int32_t lmh_kv_read_seq(lmh_kv* kv, uint64_t seq, uint64_t len, const void* src, uint64_t n_bytes, uint64_t* needed,
                        uint64_t* free_blocks, void* stream) {
  if (!kv || seq >= kv->n_seqs) return LMH_INVALID_ARGUMENT;
  if (len > kv->max_ctx) return kv->fail(LMH_INVALID_ARGUMENT, "snapshot longer than the context");
  uint64_t bytes;
  lmh_kv_snapshot_bytes(kv, len, &bytes);
  if (n_bytes != bytes || (bytes && !src)) return kv->fail(LMH_INVALID_ARGUMENT, "snapshot size");
  // room first: clearing frees this sequence's unshared blocks, so they count as available
  const uint64_t nb = (len + kv->bt - 1) / kv->bt;
  uint64_t own = 0;
  for (uint32_t b : kv->seqs[seq].blocks) own += kv->pool.meta[b].refs == 1 ? 1 : 0;
  if (nb > kv->pool.free_blocks() + own) {
    if (needed) *needed = nb;
    if (free_blocks) *free_blocks = kv->pool.free_blocks() + own;
    return kv->fail(LMH_KV_FULL, "KV cache full: snapshot needs " + std::to_string(nb) + " blocks");
  }
  uint64_t first, end;
  window_span(kv, len, first, end);
  uint64_t wown = 0;
  for (int32_t b : kv->seqs[seq].wblocks) wown += b >= 0 ? 1 : 0;
  if (end - first > kv->wpool.free_blocks() + wown) {
    if (needed) *needed = end - first;
    if (free_blocks) *free_blocks = kv->wpool.free_blocks() + wown;
    return kv->fail(LMH_KV_FULL, "window pool full: snapshot needs " + std::to_string(end - first) + " window blocks");
  }
  kv->clear(seq);
  if (len == 0) return LMH_OK;
  // paged blocks only; the window blocks go at their absolute numbers (metal/src/kv.rs:508-537)
  int32_t rc = kv->reserve(seq, len, needed, free_blocks, false);
  if (rc != LMH_OK) return rc;
  if (kv->window) {
    auto& wb = kv->seqs[seq].wblocks;
    wb.assign(first, -1);
    for (uint64_t i = first; i < end; i++) {
      std::vector<uint32_t> b1;
      kv->wpool.alloc(1, b1);
      wb.push_back((int32_t)b1[0]);
    }
    kv->set_wtable(seq);
  }
  hipStream_t st = (hipStream_t)stream;
  if ((rc = kv->flush(st)) != LMH_OK) return rc;
  kv->seqs[seq].len = len;
  return snapshot_layers(kv, false, seq, nb, (uint8_t*)src, st);
}

int32_t lmh_kv_window_info(const lmh_kv* kv, lmh_window_info* out) {
  if (!kv || !out) return LMH_INVALID_ARGUMENT;
  out->window = kv->window;
  out->block_bytes = kv->wblock_bytes;
  out->pool_blocks = kv->wpool_blocks;
  out->free_blocks = kv->wpool.free_blocks();
  return LMH_OK;
}

int32_t lmh_kv_window_table(const lmh_kv* kv, uint64_t seq, int32_t* out, uint64_t cap, uint64_t* n) {
  if (!kv || !n || seq >= kv->n_seqs) return LMH_INVALID_ARGUMENT;
  const auto& b = kv->seqs[seq].wblocks;
  for (uint64_t i = 0; i < b.size() && i < cap && out; i++) out[i] = b[i];
  *n = b.size();
  return LMH_OK;
}

int32_t lmh_kv_block_table(const lmh_kv* kv, uint64_t seq, uint32_t* out, uint64_t cap, uint64_t* n) {
  if (!kv || !n || seq >= kv->n_seqs) return LMH_INVALID_ARGUMENT;
  const auto& b = kv->seqs[seq].blocks;
  for (uint64_t i = 0; i < b.size() && i < cap && out; i++) out[i] = b[i];
  *n = b.size();
  return LMH_OK;
}

int32_t lmh_kv_adopt_blocks(lmh_kv* kv, uint64_t seq, const uint32_t* blocks, uint64_t n) {
  if (!kv || seq >= kv->n_seqs || (n > 0 && !blocks)) return LMH_INVALID_ARGUMENT;
  if (!kv->seqs[seq].blocks.empty()) return kv->fail(LMH_INVALID_ARGUMENT, "sequence already holds blocks");
  if (n > kv->bps) return kv->fail(LMH_INVALID_ARGUMENT, "more blocks than one sequence can hold");
  std::vector<uint8_t> want(kv->pool_blocks, 0);
  for (uint64_t i = 0; i < n; i++) {
    if (blocks[i] >= kv->pool_blocks || want[blocks[i]])
      return kv->fail(LMH_INVALID_ARGUMENT, "block id out of range or repeated");
    want[blocks[i]] = 1;
  }
  for (uint64_t i = 0; i < n; i++)
    if (!kv->pool.is_free(blocks[i])) return kv->fail(LMH_INVALID_ARGUMENT, "a requested block is not free");
  for (uint64_t i = 0; i < n; i++) {
    kv->pool.unlink_free(blocks[i]);
    BlockMeta& m = kv->pool.meta[blocks[i]];
    if (m.has_hash) {
      kv->pool.by_hash.erase(m.hash);
      m.has_hash = false;
      kv->pool.evictions++;
    }
    m.refs = 1;
    kv->back(blocks[i], true);
    kv->seqs[seq].blocks.push_back(blocks[i]);
  }
  kv->set_table(seq);
  return LMH_OK;
}

int32_t lmh_pool_refs(const lmh_kv* kv, uint32_t block, uint32_t* refs) {
  if (!kv || !refs || block >= kv->pool_blocks) return LMH_INVALID_ARGUMENT;
  *refs = kv->pool.meta[block].refs;
  return LMH_OK;
}

int32_t lmh_pool_set_hash(lmh_kv* kv, uint32_t block, const uint8_t hash[32]) {  // lib.rs:113-118
  if (!kv || !hash || block >= kv->pool_blocks) return LMH_INVALID_ARGUMENT;
  Hash h;
  std::memcpy(h.data(), hash, 32);
  kv->pool.set_hash(block, h);
  return LMH_OK;
}

int32_t lmh_pool_clear_hash(lmh_kv* kv, uint32_t block) {
  if (!kv || block >= kv->pool_blocks) return LMH_INVALID_ARGUMENT;
  kv->pool_clear_hash(block);
  kv->maybe_unback(block);
  return LMH_OK;
}

int32_t lmh_pool_is_cached(const lmh_kv* kv, uint32_t block, int32_t* cached) {
  if (!kv || !cached || block >= kv->pool_blocks) return LMH_INVALID_ARGUMENT;
  *cached = kv->pool.meta[block].has_hash ? 1 : 0;
  return LMH_OK;
}

// forward.rs:207-262: checks, then all-or-nothing reservation, then Rows::push in batch order
// (one pass: paged layers never bound the per-call append, kv.rs:522-531).
int32_t lmh_batch_prepare(lmh_kv* kv, const lmh_seq_tokens* batch, uint64_t n, lmh_seg* segs_out, uint64_t* n_rows,
                          uint64_t* needed, uint64_t* free_blocks) {
  if (!kv) return LMH_INVALID_ARGUMENT;
  if (n == 0 || !batch || !segs_out) return kv->fail(LMH_INVALID_ARGUMENT, "empty batch");
  if (n > kv->n_seqs) return kv->fail(LMH_INVALID_ARGUMENT, "more sequences than slots in one call");
  for (uint64_t i = 0; i < n; i++) {
    if (batch[i].seq >= kv->n_seqs) return kv->fail(LMH_INVALID_ARGUMENT, "sequence out of range");
    if (batch[i].n_tokens == 0) return kv->fail(LMH_INVALID_ARGUMENT, "empty token list");
    for (uint64_t j = 0; j < i; j++)
      if (batch[j].seq == batch[i].seq) return kv->fail(LMH_INVALID_ARGUMENT, "sequence appears twice in one batch");
    if (kv->seqs[batch[i].seq].len + batch[i].n_tokens > kv->max_ctx)
      return kv->fail(LMH_INVALID_ARGUMENT, "context overflow");
  }
  uint64_t need = 0;
  for (uint64_t i = 0; i < n; i++) need += kv->blocks_needed(batch[i].seq, kv->seqs[batch[i].seq].len + batch[i].n_tokens);
  if (need > kv->pool.free_blocks()) {
    if (needed) *needed = need;
    if (free_blocks) *free_blocks = kv->pool.free_blocks();
    return kv->fail(LMH_KV_FULL, "KV cache full: " + std::to_string(need) + " more blocks needed, " +
                                     std::to_string(kv->pool.free_blocks()) + " free");
  }
  if (kv->window) {  // the window pool, entry by entry in batch order (each releases before it takes)
    uint64_t free = kv->wpool.free_blocks(), w_need = 0;
    bool short_ = false;
    for (uint64_t i = 0; i < n; i++) {
      uint64_t take, give;
      const uint64_t len = kv->seqs[batch[i].seq].len;
      kv->window_delta(batch[i].seq, len, len + batch[i].n_tokens, take, give);
      free += give;
      w_need += take;
      if (take > free) short_ = true;
      free -= std::min(take, free);
    }
    if (short_) {
      if (needed) *needed = w_need;
      if (free_blocks) *free_blocks = kv->wpool.free_blocks();
      return kv->fail(LMH_KV_FULL, "window pool full: " + std::to_string(w_need) + " window blocks needed");
    }
  }
  for (uint64_t i = 0; i < n; i++) kv->reserve(batch[i].seq, kv->seqs[batch[i].seq].len + batch[i].n_tokens, nullptr, nullptr);
  uint64_t start = 0;
  for (uint64_t i = 0; i < n; i++) {
    segs_out[i].seq = batch[i].seq;
    segs_out[i].start = start;
    segs_out[i].n = batch[i].n_tokens;
    segs_out[i].pos0 = kv->seqs[batch[i].seq].len;
    start += batch[i].n_tokens;
  }
  if (n_rows) *n_rows = start;
  return LMH_OK;
}

int32_t lmh_batch_commit(lmh_kv* kv, const lmh_seg* segs, uint64_t n_segs) {
  if (!kv || (n_segs > 0 && !segs)) return LMH_INVALID_ARGUMENT;
  for (uint64_t i = 0; i < n_segs; i++) {
    if (segs[i].seq >= kv->n_seqs) return kv->fail(LMH_INVALID_ARGUMENT, "sequence out of range");
    const uint64_t nl = kv->seqs[segs[i].seq].len + segs[i].n;
    if (nl > kv->seqs[segs[i].seq].blocks.size() * kv->bt) return kv->fail(LMH_INVALID_ARGUMENT, "commit beyond reserved blocks");
  }
  for (uint64_t i = 0; i < n_segs; i++) kv->seqs[segs[i].seq].len += segs[i].n;
  return LMH_OK;
}

static int32_t kv_io(lmh_kv* kv, uint32_t layer, const lmh_seg* segs, uint64_t n_segs, const void* a, const void* b,
                     void* stream, int mode) {
  if (!kv) return LMH_INVALID_ARGUMENT;
  if (layer >= kv->layers.size()) return kv->fail(LMH_INVALID_ARGUMENT, "layer out of range");
  uint64_t n_rows;
  int32_t rc = kv->rows_from(segs, n_segs, n_rows);
  if (rc != LMH_OK) return rc;
  if (n_rows == 0) return LMH_OK;
  if ((rc = kv->check_window_rows(layer, segs, n_segs, 0)) != LMH_OK) return rc;
  if (!a || !b) return kv->fail(LMH_INVALID_ARGUMENT, "null data pointer");
  hipStream_t st = (hipStream_t)stream;
  if ((rc = kv->flush(st)) != LMH_OK) return rc;
  const int32_t *rs, *rp;
  const uint8_t* ex;
  int slot;
  if ((rc = kv->stage_rows(nullptr, 0, nullptr, 0, rs, rp, ex, slot)) != LMH_OK) return rc;
  const PageGeom g = kv->geom(layer);
  const LayerLayout& y = kv->layers[layer];
  hipError_t e = hipSuccess;
  switch (mode) {
    case 0: e = launch_store_f32(g, rs, rp, (uint32_t)n_rows, (const float*)a, (const float*)b, st); break;
    case 1:
      e = launch_store_encoded(g, rs, rp, (uint32_t)n_rows, (const uint8_t*)a, (const uint8_t*)b, (uint32_t)y.k_row,
                               (uint32_t)y.v_row, st);
      break;
    case 2: e = launch_gather(g, rs, rp, (uint32_t)n_rows, (float*)a, (float*)b, st); break;
    case 3:
      e = launch_gather_encoded(g, rs, rp, (uint32_t)n_rows, (uint8_t*)a, (uint8_t*)b, (uint32_t)y.k_row,
                                (uint32_t)y.v_row, st);
      break;
  }
  if (e != hipSuccess) return kv->hip_fail(e, "kernel launch");
  return kv->release_rows(slot, st);
}

int32_t lmh_kv_store(lmh_kv* kv, uint32_t layer, const lmh_seg* segs, uint64_t n_segs, const float* k, const float* v,
                     void* stream) {
  return kv_io(kv, layer, segs, n_segs, k, v, stream, 0);
}
int32_t lmh_kv_store_encoded(lmh_kv* kv, uint32_t layer, const lmh_seg* segs, uint64_t n_segs, const void* k,
                             const void* v, void* stream) {
  return kv_io(kv, layer, segs, n_segs, k, v, stream, 1);
}
int32_t lmh_kv_gather(lmh_kv* kv, uint32_t layer, const lmh_seg* segs, uint64_t n_segs, float* k, float* v,
                      void* stream) {
  return kv_io(kv, layer, segs, n_segs, k, v, stream, 2);
}
int32_t lmh_kv_gather_encoded(lmh_kv* kv, uint32_t layer, const lmh_seg* segs, uint64_t n_segs, void* k, void* v,
                              void* stream) {
  return kv_io(kv, layer, segs, n_segs, k, v, stream, 3);
}

int32_t lmh_qk_rope_store(lmh_kv* kv, uint32_t layer, const lmh_seg* segs, uint64_t n_segs, const float* q_in,
                          const float* k_in, const float* v_in, float* q_out, const lmh_rope_params* p,
                          void* stream) {
  if (!kv) return LMH_INVALID_ARGUMENT;
  if (layer >= kv->layers.size()) return kv->fail(LMH_INVALID_ARGUMENT, "layer out of range");
  if (!p || p->abi_version != LMH_ABI_VERSION) return kv->fail(LMH_INVALID_ARGUMENT, "rope params: null or ABI version");
  const LayerLayout& y = kv->layers[layer];
  const bool apply = (p->flags & LMH_ROPE_APPLY) != 0;
  if (p->flags & ~(LMH_ROPE_Q_NORM | LMH_ROPE_K_NORM | LMH_ROPE_V_NORM | LMH_ROPE_APPLY | LMH_ROPE_NEOX))
    return kv->fail(LMH_INVALID_ARGUMENT, "unknown rope flag");
  if (apply && (p->rot_dim == 0 || p->rot_dim % 2 || p->rot_dim > y.hd))
    return kv->fail(LMH_INVALID_ARGUMENT, "rot_dim must be even and in [2, hd]");
  const uint32_t q_stride = p->q_stride ? p->q_stride : y.hd;
  if (q_stride < y.hd) return kv->fail(LMH_INVALID_ARGUMENT, "q_stride < hd");
  if (((p->flags & LMH_ROPE_Q_NORM) && !p->q_norm) || ((p->flags & LMH_ROPE_K_NORM) && !p->k_norm))
    return kv->fail(LMH_INVALID_ARGUMENT, "norm flag without weights");
  if (y.hd > ROPE_MAX_DIM || y.hdv != y.hd)
    return kv->fail(LMH_UNSUPPORTED, "the fused kernel takes hd == hdv <= 512");
  if (q_stride % 4 || ((uintptr_t)q_in | (uintptr_t)k_in | (uintptr_t)v_in | (uintptr_t)q_out) % 16)
    return kv->fail(LMH_INVALID_ARGUMENT, "q_stride must be a multiple of 4 and the arrays 16-byte aligned");
  uint64_t n_rows;
  int32_t rc = kv->rows_from(segs, n_segs, n_rows);
  if (rc == LMH_OK) rc = kv->check_window_rows(layer, segs, n_segs, 0);
  if (rc != LMH_OK) return rc;
  if (n_rows == 0) return LMH_OK;
  if (!q_in || !k_in || !v_in || !q_out) return kv->fail(LMH_INVALID_ARGUMENT, "null data pointer");
  // rope's per-pair frequency, as the reference forms it in f32 (ops.rs:52):
  // theta.powf(-(2i as f32) / rot_dim as f32)
  const uint32_t half_rot = apply ? p->rot_dim / 2 : 0;
  std::vector<float> freq(std::max<uint32_t>(half_rot, 1), 0.f);
  for (uint32_t i = 0; i < half_rot; i++) freq[i] = powf(p->theta, -(2.0f * (float)i) / (float)p->rot_dim);
  hipStream_t st = (hipStream_t)stream;
  if ((rc = kv->flush(st)) != LMH_OK) return rc;
  const int32_t *rs, *rp;
  const uint8_t* ex;
  int slot;
  // rows of f16 / bf16 segments in aligned runs of 4 positions go to the 4-token kernel (whole
  // 8-byte V runs); the others (decode rows, segment edges) to the per-row kernel
  std::vector<int32_t> lists;  // [quads..., rest...]
  uint32_t n_quads = 0;
  if (kv->kv_type == LMH_KV_F16 || kv->kv_type == LMH_KV_BF16) {
    std::vector<int32_t> rest;
    for (uint64_t i = 0; i < n_segs; i++) {
      const lmh_seg& sg = segs[i];
      for (uint64_t j = 0; j < sg.n;) {
        if (((sg.pos0 + j) & 3) == 0 && j + 4 <= sg.n) {
          lists.push_back((int32_t)(sg.start + j));
          j += 4;
        } else {
          rest.push_back((int32_t)(sg.start + j));
          j++;
        }
      }
    }
    n_quads = (uint32_t)lists.size();
    lists.insert(lists.end(), rest.begin(), rest.end());
  }
  const size_t freq_bytes = freq.size() * 4;
  if ((rc = kv->stage_rows(freq.data(), freq_bytes, lists.data(), lists.size() * 4, rs, rp, ex, slot)) != LMH_OK)
    return rc;
  const int32_t* d_lists = (const int32_t*)(ex + (freq_bytes + 255) / 256 * 256);
  RopeGeom r{y.n_head, q_stride, p->flags, half_rot, p->eps, p->freq_scale, p->attn_factor,
             (p->flags & LMH_ROPE_Q_NORM) ? p->q_norm : nullptr, (p->flags & LMH_ROPE_K_NORM) ? p->k_norm : nullptr,
             apply ? p->freq_div : nullptr, (const float*)ex};
  hipError_t e;
  LaunchEv ev;
  if ((e = kv->time_launch(LMH_KERNEL_ROPE_STORE, ev)) != hipSuccess) return kv->hip_fail(e, "event");
  e = launch_qk_rope_store(kv->geom(layer), r, rs, rp, (uint32_t)n_rows, q_in, k_in, v_in, q_out, d_lists, n_quads,
                           d_lists + n_quads, (uint32_t)(lists.size() - n_quads), st, ev);
  if (e != hipSuccess) return kv->hip_fail(e, "kernel launch");
  return kv->release_rows(slot, st);
}

// What the planner needs to know of the kernel modules for a layer's geometry.
static void fill_kernel_facts(PlanIn& in, uint32_t kv_type, uint32_t hd, uint32_t hdv, uint32_t group) {
  in.prefill_supported = prefill_supported(kv_type, hd, hdv, group);
  in.unit_cols = prefill_cols_per_unit();
  in.prefill_wg_per_cu = prefill_wg_per_cu();
  in.prefill_lds_fixed = in.prefill_supported ? prefill_lds_bytes(kv_type, hd, 0, 0) + prefill_static_lds_bytes() : 0;
  in.lds_limit = 160 * 1024;
  in.rows_max_heads = decode_rows_max_heads();
  in.local_merge_ok = decode_local_merge_ok(hd, hdv, group);
  in.mfma_local_ok = decode_mfma_local_ok(kv_type, hd, hdv);
}

// lmh_attend and lmh_attend_noalloc. noalloc: split-K partials and the merge list go to the
// device's no-allocation scratch (the split target capped to what it holds, a call that still
// needs more is refused), the staged work list must fit the staging capacity reserved at
// creation, and no timing events are made or recorded: the call allocates nothing.
static int32_t attend_impl(lmh_kv* kv, uint32_t layer, const lmh_seg* segs, uint64_t n_segs, const float* q,
                           float* out, float scale, uint64_t window, void* stream, bool noalloc) {
  if (!kv) return LMH_INVALID_ARGUMENT;
  if (noalloc && !kv->scratch) return kv->fail(LMH_DEVICE_ERROR, "no-allocation scratch not resolved");
  // A captured graph would replay this call's kernels against a staging slot that later calls
  // overwrite (the work list is read from it when the kernels run), so capture is refused before
  // anything is enqueued.
  {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing((hipStream_t)stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
      return kv->fail(LMH_UNSUPPORTED, "lmh_attend cannot be captured into a graph: its work list lives in a "
                                       "staging slot that later calls reuse");
  }
  if (layer >= kv->layers.size()) return kv->fail(LMH_INVALID_ARGUMENT, "layer out of range");
  if (!std::isfinite(scale)) return kv->fail(LMH_INVALID_ARGUMENT, "scale must be finite");
  uint64_t n_rows;
  int32_t rc = kv->rows_from(segs, n_segs, n_rows);
  if (rc != LMH_OK) return rc;
  if (n_rows == 0) return LMH_OK;
  if (!q || !out) return kv->fail(LMH_INVALID_ARGUMENT, "null q/out");
  const LayerLayout& y = kv->layers[layer];
  // a window layer attends within its width: its pool holds nothing older
  if (y.win && (window == 0 || window > kv->window))
    return kv->fail(LMH_INVALID_ARGUMENT, "a window layer's attention window must be 1..its width");
  if ((rc = kv->check_window_rows(layer, segs, n_segs, window)) != LMH_OK) return rc;
  const uint32_t group = y.n_head / y.n_kv;
  hipStream_t st = (hipStream_t)stream;
  if (kv->decode_capacity[layer] == 0)
    kv->decode_capacity[layer] = decode_waves_per_cu(kv->kv_type, y.hd, y.hdv, group, y.layout) * kv->n_cu;
  PlanIn pin;
  pin.row_seq = kv->row_seq.data();
  pin.row_pos = kv->row_pos.data();
  pin.n_rows = n_rows;
  pin.segs = segs;
  pin.n_segs = n_segs;
  pin.table = y.win ? kv->h_wtable.data() : kv->h_table.data();
  pin.bps = kv->bps;
  pin.bt_shift = kv->bt_shift;
  pin.n_head = y.n_head;
  pin.n_kv = y.n_kv;
  pin.hd = y.hd;
  pin.hdv = y.hdv;
  pin.layout = y.layout;
  pin.kv_type = kv->kv_type;
  pin.window = window;
  pin.scale = scale;
  pin.n_cu = kv->n_cu;
  pin.decode_capacity = kv->decode_capacity[layer];
  pin.prefill_min_rows = kv->prefill_min_rows;
  pin.decode_target_items = kv->decode_target_items;
  pin.decode_min_tiles = kv->decode_min_tiles;
  pin.prefill_workgroups = kv->prefill_workgroups;
  pin.prefill_no_split = kv->prefill_whole_units;
  pin.noalloc = noalloc;
  pin.noalloc_bytes = NOALLOC_SCRATCH_BYTES;
  fill_kernel_facts(pin, kv->kv_type, y.hd, y.hdv, group);
  PlanOut& pl = kv->plan;
  plan_attend(pin, pl);
  const uint32_t ng = pl.ng, slots = pl.slots, pf_wg = pl.pf_wg, pf_per_wg = pl.pf_per_wg, max_pages = pl.max_pages;
  const bool local = pl.local != 0;
  const size_t slot_bytes = (size_t)ng * (y.hdv + 4) * 4;
  if ((rc = kv->flush(st)) != LMH_OK) return rc;
  const size_t items_bytes = kv->plan.items.size() * sizeof(DecodeItem);
  const size_t items_pad = (items_bytes + 255) / 256 * 256;
  const size_t merges_bytes = kv->plan.merges.size() * sizeof(MergeItem);
  const size_t merges_pad = (merges_bytes + 255) / 256 * 256;
  // one staged payload: [decode items | merges | prefill items]
  kv->payload.resize(items_pad + merges_pad + kv->plan.pitems.size() * sizeof(PrefillItem));
  if (items_bytes) std::memcpy(kv->payload.data(), kv->plan.items.data(), items_bytes);
  if (merges_bytes) std::memcpy(kv->payload.data() + items_pad, kv->plan.merges.data(), merges_bytes);
  if (!kv->plan.pitems.empty())
    std::memcpy(kv->payload.data() + items_pad + merges_pad, kv->plan.pitems.data(), kv->plan.pitems.size() * sizeof(PrefillItem));
  const int32_t *rs, *rp;
  const uint8_t* ex;
  int slot;
  hipError_t e;
  // the split partials' buffer first: growing it synchronises the device
  float* part = (float*)kv->part_buf.p;
  uint32_t* merge_dst = (uint32_t*)kv->merge_buf.p;
  if (slots > 0) {
    const size_t part_bytes = (size_t)slots * slot_bytes;
    if (noalloc) {
      const size_t part_pad = (part_bytes + 255) / 256 * 256;
      if (part_pad + merges_bytes > NOALLOC_SCRATCH_BYTES)
        return kv->fail(LMH_INVALID_ARGUMENT, "the call needs " + std::to_string(part_pad + merges_bytes) +
                                                  " bytes of split-K scratch; lmh_attend_noalloc holds " +
                                                  std::to_string(NOALLOC_SCRATCH_BYTES));
      part = (float*)kv->scratch;
      merge_dst = (uint32_t*)(kv->scratch + part_pad);
    } else {
      if ((e = kv->part_buf.ensure(part_bytes)) != hipSuccess) return kv->hip_fail(e, "hipMalloc");
      if ((e = kv->merge_buf.ensure(merges_bytes)) != hipSuccess) return kv->hip_fail(e, "hipMalloc");
      part = (float*)kv->part_buf.p;
      merge_dst = (uint32_t*)kv->merge_buf.p;
    }
  }
  if ((rc = kv->stage_rows(kv->payload.data(), kv->payload.size(), nullptr, 0, rs, rp, ex, slot, !noalloc)) != LMH_OK)
    return rc;
  const PageGeom g = kv->geom(layer);
  RowGeom r{};
  r.row_seq = rs;
  r.row_pos = rp;
  r.n_head = y.n_head;
  r.group = group;
  r.ng = ng;
  r.scale_log2 = scale * 1.4426950408889634f;
  r.window = (uint32_t)std::min<uint64_t>(window, 0xffffffffull);
  r.local_merge = pl.local;   // 0, or the waves per workgroup of a local-merge launch
  PrefillGeom pg{};
  pg.n_head = y.n_head;
  pg.group = group;
  pg.scale_log2 = r.scale_log2;
  pg.window = r.window;
  pg.p_f16 = kv->prefill_p_f16 ? 1u : 0u;
  pg.ng = ng;
  pg.part = part;
  pg.q_flag = kv->q_flag_dev;
  // the launch for a Q with bits below the page type (one pass of hi + lo products), when asked
  // for or when the handle's previous prefill launch found such bits
  pg.q_split = kv->prefill_q_split == 2 || (kv->prefill_q_split == 0 && *kv->q_flag != 0) ? 1u : 0u;
  const MergeCopy mc{(const uint32_t*)(ex + items_pad), merge_dst,
                     kv->plan.merges.empty() ? 0u : (uint32_t)(merges_bytes / 4)};
  // timing events are made on first use: not on the no-allocation path
  auto time_launch = [&](uint32_t kind, LaunchEv& ev) -> hipError_t {
    ev = LaunchEv{};
    return noalloc ? hipSuccess : kv->time_launch(kind, ev);
  };
  // A mixed batch (prefill units and decode items) runs as one launch: the prefill workgroups
  // first (one per CU they reach), then the decode items, a wave each, on the CUs left free.
  const bool overlap = !kv->plan.pitems.empty() && !kv->plan.items.empty();
  LaunchEv ev;
  if (overlap) {
    if ((e = time_launch(LMH_KERNEL_MIXED, ev)) != hipSuccess) return kv->hip_fail(e, "event");
    e = launch_mixed(g, pg, (const PrefillItem*)(ex + items_pad + merges_pad), pf_wg, pf_per_wg, max_pages, r,
                     (const DecodeItem*)ex, (uint32_t)kv->plan.items.size(), q, out, part, mc, st, ev);
    if (e != hipSuccess) return kv->hip_fail(e, "mixed kernel");
  }
  if (!overlap && !kv->plan.pitems.empty()) {
    if ((e = time_launch(LMH_KERNEL_PREFILL, ev)) != hipSuccess) return kv->hip_fail(e, "event");
    e = launch_prefill(g, pg, (const PrefillItem*)(ex + items_pad + merges_pad), pf_wg, pf_per_wg, max_pages, q, out,
                       mc, st, ev);
    if (e != hipSuccess) return kv->hip_fail(e, "prefill kernel");
  }
  if (!overlap && !kv->plan.items.empty()) {
    if ((e = time_launch(LMH_KERNEL_DECODE, ev)) != hipSuccess) return kv->hip_fail(e, "event");
    e = launch_decode(g, r, (const DecodeItem*)ex, (uint32_t)kv->plan.items.size(), q, out, part, mc, st,
                      ev);
    if (e != hipSuccess) return kv->hip_fail(e, "decode kernel");
  }
  if (!kv->plan.merges.empty()) {
    if ((e = time_launch(LMH_KERNEL_MERGE, ev)) != hipSuccess) return kv->hip_fail(e, "event");
    // the planner lists the prompt tokens' merges (nh != 0) before the decode merges
    uint32_t max_split = 0, n_pf = 0, max_pf_rows = 0;
    for (const MergeItem& m : kv->plan.merges) {
      if (m.nh != 0) {
        max_pf_rows = std::max(max_pf_rows, m.nh * m.n_split);
        if (n_pf != (uint32_t)(&m - kv->plan.merges.data()) || m.n_split > PF_MAX_PIECES ||
            (m.nh > 1 && m.nh * m.n_split > PF_MERGE_ROWS) || (y.hdv != 64 && y.hdv != 128))
          return kv->fail(LMH_UNSUPPORTED, "attend: the planner's prompt merges are out of order or too long");
        n_pf++;
      } else {
        max_split = std::max(max_split, m.n_split);
      }
    }
    e = launch_merge(r, y.hdv, (const MergeItem*)merge_dst, (uint32_t)kv->plan.merges.size(), n_pf, max_pf_rows,
                     part, out, max_split, st, ev);
    if (e != hipSuccess) return kv->hip_fail(e, "merge kernel");
  }
  return kv->release_rows(slot, st);
}

int32_t lmh_attend(lmh_kv* kv, uint32_t layer, const lmh_seg* segs, uint64_t n_segs, const float* q, float* out,
                   float scale, uint64_t window, void* stream) {
  return attend_impl(kv, layer, segs, n_segs, q, out, scale, window, stream, false);
}

int32_t lmh_attend_noalloc(lmh_kv* kv, uint32_t layer, const lmh_seg* segs, uint64_t n_segs, const float* q,
                           float* out, float scale, uint64_t window, void* stream) {
  return attend_impl(kv, layer, segs, n_segs, q, out, scale, window, stream, true);
}

// nullptr, or what is wrong with the options
static const char* tuning_error(const lmh_attend_tuning* t) {
  if (!t || t->abi_version != LMH_ABI_VERSION) return "tuning: null or ABI version";
  if (t->prefill_p_f16 > 1) return "tuning: prefill_p_f16 must be 0 or 1";
  if (t->prefill_min_rows > (1ull << 32)) return "tuning: prefill_min_rows out of range";
  if (t->decode_min_tiles > 64) return "tuning: decode_min_tiles must be <= 64";
  if (t->decode_target_items > (1ull << 32)) return "tuning: decode_target_items out of range";
  if (t->prefill_workgroups > (1ull << 32)) return "tuning: prefill_workgroups out of range";
  if (t->prefill_whole_units > 1) return "tuning: prefill_whole_units must be 0 or 1";
  if (t->prefill_q_split > 2) return "tuning: prefill_q_split must be 0, 1 or 2";
  return nullptr;
}

int32_t lmh_kv_set_tuning(lmh_kv* kv, const lmh_attend_tuning* t) {
  if (!kv) return LMH_INVALID_ARGUMENT;
  if (const char* why = tuning_error(t)) return kv->fail(LMH_INVALID_ARGUMENT, why);
  kv->prefill_p_f16 = t->prefill_p_f16 != 0;
  kv->prefill_workgroups = t->prefill_workgroups;
  kv->prefill_min_rows = t->prefill_min_rows;
  kv->decode_target_items = t->decode_target_items;
  kv->decode_min_tiles = t->decode_min_tiles;
  kv->prefill_whole_units = t->prefill_whole_units != 0;
  kv->prefill_q_split = t->prefill_q_split;
  return LMH_OK;
}

int32_t lmh_kv_get_tuning(const lmh_kv* kv, lmh_attend_tuning* t) {
  if (!kv || !t) return LMH_INVALID_ARGUMENT;
  t->abi_version = LMH_ABI_VERSION;
  t->prefill_p_f16 = kv->prefill_p_f16 ? 1u : 0u;
  t->prefill_min_rows = kv->prefill_min_rows;
  t->decode_target_items = kv->decode_target_items;
  t->decode_min_tiles = kv->decode_min_tiles;
  t->prefill_workgroups = kv->prefill_workgroups;
  t->prefill_whole_units = kv->prefill_whole_units ? 1u : 0u;
  t->prefill_q_split = kv->prefill_q_split;
  return LMH_OK;
}

// The planner alone on host data (no device): validates like lmh_kv_create / lmh_attend, plans as
// lmh_attend would for a layer of this geometry, and copies the work lists out.
int32_t lmh_plan_attend(const lmh_plan_desc* d, const lmh_seg* segs, uint64_t n_segs, uint32_t* items,
                        uint64_t items_cap, uint32_t* merges, uint64_t merges_cap, uint32_t* units, uint64_t units_cap,
                        lmh_plan_counts* counts) {
  if (!d || !counts || d->abi_version != LMH_ABI_VERSION || (n_segs > 0 && !segs)) return LMH_INVALID_ARGUMENT;
  const uint32_t bt = d->block_tokens;
  if (d->kv_type > LMH_KV_BF16 || bt == 0 || (bt & (bt - 1)) != 0 || d->n_kv == 0 || d->n_head == 0 ||
      d->n_head % d->n_kv != 0 || d->hd == 0 || d->hdv == 0 || d->hd > MAX_HEAD_DIM || d->hdv > MAX_HEAD_DIM ||
      (d->kv_type == LMH_KV_Q8_0 && (d->hd % 32 != 0 || d->hdv % 32 != 0)) || d->n_cu == 0 || d->n_seqs == 0 ||
      d->bps == 0 || !d->table || !std::isfinite(d->scale) || tuning_error(&d->tuning))
    return LMH_INVALID_ARGUMENT;
  uint32_t bt_shift = 0;
  while ((1u << bt_shift) < bt) bt_shift++;
  std::vector<int32_t> row_seq, row_pos;
  uint64_t n_rows = 0;
  for (uint64_t i = 0; i < n_segs; i++) {
    const lmh_seg& sg = segs[i];
    if (sg.seq >= d->n_seqs || sg.start != n_rows || sg.pos0 + sg.n > d->bps * bt || sg.pos0 + sg.n > 0x7fffffffull)
      return LMH_INVALID_ARGUMENT;
    for (uint64_t j = 0; j < sg.n; j++) {   // every block the row's range touches is in the table
      const uint64_t pos = sg.pos0 + j, lo = (d->window > 0 && pos + 1 > d->window) ? pos + 1 - d->window : 0;
      if (d->table[sg.seq * d->bps + (pos >> bt_shift)] < 0 || d->table[sg.seq * d->bps + (lo >> bt_shift)] < 0)
        return LMH_INVALID_ARGUMENT;
      row_seq.push_back((int32_t)sg.seq);
      row_pos.push_back((int32_t)pos);
    }
    n_rows += sg.n;
  }
  PlanIn in;
  in.row_seq = row_seq.data();
  in.row_pos = row_pos.data();
  in.n_rows = n_rows;
  in.segs = segs;
  in.n_segs = n_segs;
  in.table = d->table;
  in.bps = d->bps;
  in.bt_shift = bt_shift;
  in.n_head = d->n_head;
  in.n_kv = d->n_kv;
  in.hd = d->hd;
  in.hdv = d->hdv;
  in.layout = (bt >= 16 && decode_tiles_supported(d->kv_type, d->hd, d->hdv)) ? LAYOUT_TILES : LAYOUT_ROWS;
  in.kv_type = d->kv_type;
  in.window = d->window;
  in.scale = d->scale;
  in.n_cu = d->n_cu;
  in.decode_capacity = d->decode_capacity ? d->decode_capacity : 8ull * d->n_cu;
  in.prefill_min_rows = d->tuning.prefill_min_rows;
  in.decode_target_items = d->tuning.decode_target_items;
  in.decode_min_tiles = d->tuning.decode_min_tiles;
  in.prefill_workgroups = d->tuning.prefill_workgroups;
  in.prefill_no_split = d->tuning.prefill_whole_units != 0;
  in.noalloc = d->noalloc != 0;
  in.noalloc_bytes = NOALLOC_SCRATCH_BYTES;
  fill_kernel_facts(in, d->kv_type, d->hd, d->hdv, d->n_head / d->n_kv);
  PlanOut o;
  if (n_rows > 0) plan_attend(in, o);
  counts->n_items = o.items.size();
  counts->n_merges = o.merges.size();
  counts->n_units = o.pitems.size();
  counts->item_words = sizeof(DecodeItem) / 4;
  counts->merge_words = sizeof(MergeItem) / 4;
  counts->unit_words = sizeof(PrefillItem) / 4;
  counts->ng = o.ng;
  counts->slots = o.slots;
  counts->pf_wg = o.pf_wg;
  counts->pf_per_wg = o.pf_per_wg;
  counts->max_pages = o.max_pages;
  counts->local = o.local;
  counts->layout = in.layout;
  counts->chunk = o.chunk;
  if (o.items.size() > items_cap || o.merges.size() > merges_cap || o.pitems.size() > units_cap)
    return LMH_INVALID_ARGUMENT;   // the counts say how much room the lists need
  if (!o.items.empty()) std::memcpy(items, o.items.data(), o.items.size() * sizeof(DecodeItem));
  if (!o.merges.empty()) std::memcpy(merges, o.merges.data(), o.merges.size() * sizeof(MergeItem));
  if (!o.pitems.empty()) std::memcpy(units, o.pitems.data(), o.pitems.size() * sizeof(PrefillItem));
  return LMH_OK;
}

int32_t lmh_bench_read_ceiling(int32_t device, uint64_t bytes, uint32_t iters, double* gbps) {
  bytes &= ~15ull;
  if (!gbps || bytes == 0 || iters == 0) return LMH_INVALID_ARGUMENT;
  if (hipSetDevice(device) != hipSuccess) return LMH_DEVICE_ERROR;
  uint8_t* p = nullptr;
  uint32_t* sink = nullptr;
  LaunchEv ev;
  hipError_t e = hipMalloc((void**)&p, bytes);
  if (e == hipSuccess) e = hipMalloc((void**)&sink, 16);
  if (e == hipSuccess) e = hipMemset(p, 1, bytes);
  if (e == hipSuccess) e = hipEventCreate(&ev.start);
  if (e == hipSuccess) e = hipEventCreate(&ev.stop);
  for (uint32_t i = 0; e == hipSuccess && i < 3; i++) e = launch_read_ceiling(p, bytes, sink, nullptr, LaunchEv{});
  // each launch timed by events its own dispatch records, as the attention kernels are timed
  double total_ms = 0.0;
  for (uint32_t i = 0; e == hipSuccess && i < iters; i++) {
    e = launch_read_ceiling(p, bytes, sink, nullptr, ev);
    if (e == hipSuccess) e = hipEventSynchronize(ev.stop);
    float ms = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, ev.start, ev.stop);
    total_ms += ms;
  }
  if (ev.start) (void)hipEventDestroy(ev.start);
  if (ev.stop) (void)hipEventDestroy(ev.stop);
  if (sink) (void)hipFree(sink);
  if (p) (void)hipFree(p);
  if (e != hipSuccess) return e == hipErrorOutOfMemory ? LMH_OUT_OF_MEMORY : LMH_DEVICE_ERROR;
  *gbps = (double)bytes * iters / (total_ms * 1e-3) / 1e9;
  return LMH_OK;
}

int32_t lmh_kv_set_timing(lmh_kv* kv, int32_t enable) {
  if (!kv) return LMH_INVALID_ARGUMENT;
  kv->timing = enable != 0;
  return LMH_OK;
}

int32_t lmh_kv_kernel_time(lmh_kv* kv, uint32_t kernel, double* ms, uint64_t* launches) {
  if (!kv || kernel > LMH_KERNEL_MIXED) return LMH_INVALID_ARGUMENT;
  hipError_t e = kv->collect_times();
  if (e != hipSuccess) return kv->hip_fail(e, "event timing");
  if (ms) *ms = kv->acc_ms[kernel];
  if (launches) *launches = kv->launches[kernel];
  kv->acc_ms[kernel] = 0;
  kv->launches[kernel] = 0;
  return LMH_OK;
}

}  // extern "C"
