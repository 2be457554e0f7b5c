// sched.cpp — the request scheduler behind lmh_sched_*: token-budget steps, admission with
// retraction over the block pool, prefix reuse by chain hash, and the packing of a step into the
// KV handle's batch. Host code only.
//
//   Scheduler   crates/engine/sched/src/lib.rs:75-282
//   Sequence    crates/engine/kv/src/lib.rs:262-335 (acquire / publish / release)
#include <algorithm>
#include <cmath>
#include <cstring>
#include <deque>
#include <string>
#include <vector>

#include "../../include/llmario_hip.h"
#include "kv_hooks.h"
#include "pool.h"

using namespace lmh;

namespace {

struct Slot {
  uint32_t id = 0;
  uint32_t priority = 0;
  std::vector<uint32_t> prompt;
  uint64_t max_new = 0, generated = 0;
  bool decoding = false;
  uint64_t done = 0;
  uint64_t seq_no = 0;
  std::vector<uint32_t> blocks;  // standalone: the Sequence's block table (bound: the handle's)
  uint64_t kv_seq = UINT64_MAX;
  // chain hashes already computed for this slot: chain[i] covers chain_tokens[0 .. (i+1)*bt]
  std::vector<Hash> chain;
  std::vector<uint32_t> chain_tokens;
};

struct Queued {
  uint64_t seq_no;
  std::vector<uint32_t> prompt;
  uint64_t max_new;
  uint32_t priority;
};

std::string c_str_or_empty(const char* s) { return s ? std::string(s) : std::string(); }

std::vector<uint8_t> key_extra(const lmh_sched_options* o) {
  std::vector<uint8_t> digest, salt;
  if (o->model_digest && o->model_digest_len) digest.assign(o->model_digest, o->model_digest + o->model_digest_len);
  if (o->salt && o->salt_len) salt.assign(o->salt, o->salt + o->salt_len);
  return cache_key_extra(digest, c_str_or_empty(o->kv_types), c_str_or_empty(o->rope_params),
                         c_str_or_empty(o->template_hash), salt);
}

}  // namespace

struct lmh_sched {
  uint64_t token_budget = 1, max_slots = 1;
  double conservativeness = 1.0;
  std::vector<uint8_t> extra;
  std::vector<Slot> slots;
  std::deque<Queued> queue;
  uint32_t next_id = 1;
  uint64_t next_seq = 1;
  uint64_t retractions = 0;
  BlockPool own;
  lmh_kv* kv = nullptr;
  bool kv_gone = false;  // bound, and the handle was destroyed first: every call fails
  std::string err;

  BlockPool& pool() { return kv ? kv_pool(kv) : own; }
  const BlockPool& pool() const { return kv ? kv_pool(kv) : own; }

  int32_t fail(int32_t code, const std::string& m) {
    err = m;
    return code;
  }
  Slot* find(uint32_t id) {
    for (Slot& s : slots)
      if (s.id == id) return &s;
    return nullptr;
  }
  const Slot* find(uint32_t id) const {
    for (const Slot& s : slots)
      if (s.id == id) return &s;
    return nullptr;
  }
  const std::vector<uint32_t>& blocks_of(const Slot& s) const { return kv ? kv_seq_blocks(kv, s.kv_seq) : s.blocks; }

  // sched/src/lib.rs:113-115 (bound: no sequence can hold more than max_ctx positions)
  uint64_t reserve_tokens(const std::vector<uint32_t>& prompt, uint64_t max_new) const {
    const uint64_t r = prompt.size() + (uint64_t)ceil((double)max_new * conservativeness);
    return kv ? std::min<uint64_t>(r, kv_max_ctx(kv)) : r;
  }
  // Bound: the lowest-numbered sequence slot of the handle that no slot holds and that is empty.
  int64_t free_kv_seq() const {
    if (!kv) return 0;
    const uint64_t n = kv_n_seqs(kv);
    for (uint64_t q = 0; q < n; q++) {
      bool held = false;
      for (const Slot& s : slots) held = held || s.kv_seq == q;
      if (!held && kv_seq_empty(kv, q)) return (int64_t)q;
    }
    return -1;
  }

  // Sequence::acquire (kv/src/lib.rs:272-316): reclaim the cached prefix blocks by chain hash
  // (stopping at the first miss), then allocate the rest; on failure nothing is held. The hashes
  // are computed block by block up to the first miss (the ones after it are never looked up);
  // `chain` returns those of the reclaimed blocks.
  bool acquire(const std::vector<uint32_t>& tokens, uint64_t reserve, std::vector<uint32_t>& blocks,
               uint64_t& cached, std::vector<Hash>& chain) {
    BlockPool& p = pool();
    const uint32_t bt = p.block_tokens;
    blocks.clear();
    chain.clear();
    cached = 0;
    // a handle with window layers keeps no window rows behind its window, so a cached prefix
    // cannot be resumed: nothing is reclaimed (and no lookup is counted)
    const bool reuse = !(kv && kv_has_window(kv));
    for (size_t i = 0; reuse && i + bt <= tokens.size(); i += bt) {
      const Hash h = block_hash(chain.empty() ? nullptr : &chain.back(), tokens.data() + i, bt, extra);
      uint32_t b;
      if (!p.reclaim(h, b)) {
        p.note_miss();
        break;
      }
      chain.push_back(h);
      blocks.push_back(b);
      cached += bt;
    }
    const uint64_t needed = (std::max<uint64_t>(reserve, tokens.size()) + bt - 1) / bt;
    const uint64_t fresh = needed > blocks.size() ? needed - blocks.size() : 0;
    if (!p.alloc(fresh, blocks)) {
      for (uint32_t b : blocks) p.release(b);
      blocks.clear();
      chain.clear();
      return false;
    }
    return true;
  }

  // Sequence::release (kv/src/lib.rs:330-334)
  void release(Slot& s) {
    if (kv) {
      kv_clear_seq(kv, s.kv_seq);
    } else {
      for (uint32_t b : s.blocks) own.release(b);
      s.blocks.clear();
    }
  }

  // The admission shared by admit and drain_queue (sched/src/lib.rs:121-146, 192-211): a slot
  // and a reservation, or false with nothing held.
  bool try_admit(const std::vector<uint32_t>& prompt, uint64_t max_new, uint32_t priority, uint32_t& id,
                 uint64_t& done) {
    if (slots.size() >= max_slots) return false;
    const int64_t q = free_kv_seq();
    if (q < 0) return false;
    std::vector<uint32_t> blocks;
    std::vector<Hash> chain;
    uint64_t cached = 0;
    if (!acquire(prompt, reserve_tokens(prompt, max_new), blocks, cached, chain)) return false;
    Slot s;
    s.id = id = next_id++;
    s.priority = priority;
    s.prompt = prompt;
    s.max_new = max_new;
    s.seq_no = next_seq++;
    s.done = done = std::min<uint64_t>(cached, prompt.empty() ? 0 : prompt.size() - 1);
    s.chain = std::move(chain);
    s.chain_tokens.assign(prompt.begin(), prompt.begin() + cached);
    if (kv) {
      s.kv_seq = (uint64_t)q;
      kv_bind_seq(kv, s.kv_seq, blocks, s.done);
    } else {
      s.blocks = std::move(blocks);
    }
    slots.push_back(std::move(s));
    return true;
  }
};

extern "C" {

int32_t lmh_sched_create(const lmh_sched_options* o, lmh_kv* kv, lmh_sched** out) {
  if (!o || !out || o->abi_version != LMH_ABI_VERSION) return LMH_INVALID_ARGUMENT;
  if ((o->model_digest_len && !o->model_digest) || (o->salt_len && !o->salt)) return LMH_INVALID_ARGUMENT;
  if (!(o->conservativeness >= 0.0) || !std::isfinite(o->conservativeness)) return LMH_INVALID_ARGUMENT;
  *out = nullptr;
  lmh_sched* s = new lmh_sched;
  s->token_budget = std::max<uint64_t>(o->token_budget, 1);
  s->max_slots = std::max<uint64_t>(o->max_slots, 1);
  s->conservativeness = o->conservativeness;
  s->extra = key_extra(o);
  if (kv) {
    if (s->max_slots > kv_n_seqs(kv)) {
      kv_set_error(kv, "max_slots exceeds the handle's sequence slots");
      delete s;
      return LMH_INVALID_ARGUMENT;
    }
    s->kv = kv;
    kv_attach(kv, s);
  } else {
    if (o->block_tokens == 0 || o->n_blocks > 0x7fffffffull) {
      delete s;
      return LMH_INVALID_ARGUMENT;
    }
    s->own.init(o->n_blocks, o->block_tokens);
  }
  *out = s;
  return LMH_OK;
}

void lmh_sched_destroy(lmh_sched* s) {
  if (!s) return;
  if (s->kv) {
    for (Slot& q : s->slots) s->release(q);
    kv_detach(s->kv, s);
  } else if (!s->kv_gone) {
    for (Slot& q : s->slots) s->release(q);
  }
  delete s;
}

const char* lmh_sched_last_error(const lmh_sched* s) { return s ? s->err.c_str() : "null scheduler"; }

int32_t lmh_sched_admit(lmh_sched* s, const lmh_request* r, lmh_admission* out, uint32_t* retracted, uint64_t cap) {
  if (s && s->kv_gone) return LMH_INVALID_ARGUMENT;
  if (!s || !r || !out || (r->n_prompt > 0 && !r->prompt) || (cap > 0 && !retracted)) return LMH_INVALID_ARGUMENT;
  if (r->priority > LMH_PRIORITY_INTERACTIVE) return s->fail(LMH_INVALID_ARGUMENT, "unknown priority");
  if (s->kv && r->n_prompt > kv_max_ctx(s->kv)) return s->fail(LMH_INVALID_ARGUMENT, "prompt longer than the context");
  std::vector<uint32_t> prompt(r->prompt, r->prompt + r->n_prompt);
  *out = lmh_admission{};
  for (;;) {
    uint32_t id;
    uint64_t done;
    if (s->try_admit(prompt, r->max_new, r->priority, id, done)) {
      out->admitted = 1;
      out->slot = id;
      out->cached_tokens = done;
      return LMH_OK;
    }
    // sched/src/lib.rs:148-154: the lowest-priority, youngest slot below the request's priority
    Slot* victim = nullptr;
    for (Slot& q : s->slots)
      if (q.priority < r->priority &&
          (!victim || q.priority < victim->priority || (q.priority == victim->priority && q.seq_no > victim->seq_no)))
        victim = &q;
    if (!victim) {
      s->queue.push_back(Queued{s->next_seq++, std::move(prompt), r->max_new, r->priority});
      return LMH_OK;
    }
    // lib.rs:156-173: released, counted, and back at the queue head with what it has left to generate
    const uint32_t vid = victim->id;
    Slot v = std::move(*victim);
    s->slots.erase(s->slots.begin() + (victim - s->slots.data()));
    s->release(v);
    s->retractions++;
    s->queue.push_front(
        Queued{v.seq_no, std::move(v.prompt), v.max_new > v.generated ? v.max_new - v.generated : 0, v.priority});
    if (out->n_retracted < cap) retracted[out->n_retracted] = vid;
    out->n_retracted++;
  }
}

int32_t lmh_sched_drain_queue(lmh_sched* s, uint32_t* admitted, uint64_t cap, uint64_t* n) {
  if (s && s->kv_gone) return LMH_INVALID_ARGUMENT;
  if (!s || !n || (cap > 0 && !admitted)) return LMH_INVALID_ARGUMENT;
  *n = 0;
  while (!s->queue.empty()) {
    const Queued& f = s->queue.front();
    uint32_t id;
    uint64_t done;
    if (!s->try_admit(f.prompt, f.max_new, f.priority, id, done)) break;
    s->queue.pop_front();
    if (*n < cap) admitted[*n] = id;
    (*n)++;
  }
  return LMH_OK;
}

int32_t lmh_sched_next_step(const lmh_sched* s, lmh_step* st) {
  if (s && s->kv_gone) return LMH_INVALID_ARGUMENT;
  if (!s || !st || (!s->slots.empty() && (!st->decodes || !st->prefills))) return LMH_INVALID_ARGUMENT;
  std::vector<const Slot*> order;
  order.reserve(s->slots.size());
  for (const Slot& q : s->slots) order.push_back(&q);
  std::stable_sort(order.begin(), order.end(), [](const Slot* a, const Slot* b) {
    return a->priority != b->priority ? a->priority > b->priority : a->seq_no < b->seq_no;
  });
  uint64_t budget = s->token_budget;
  st->n_decodes = st->n_prefills = 0;
  for (const Slot* q : order) {
    if (budget == 0) break;
    if (q->decoding) {
      st->decodes[st->n_decodes++] = q->id;
      budget--;
    }
  }
  for (const Slot* q : order) {
    if (budget == 0) break;
    if (!q->decoding) {
      const uint64_t take = std::min<uint64_t>(q->prompt.size() - q->done, budget);
      if (take > 0) {
        st->prefills[st->n_prefills++] = lmh_prefill_range{q->id, 0, q->done, q->done + take};
        budget -= take;
      }
    }
  }
  st->tokens = s->token_budget - budget;
  return LMH_OK;
}

int32_t lmh_sched_complete(lmh_sched* s, const lmh_step* st) {
  if (s && s->kv_gone) return LMH_INVALID_ARGUMENT;
  if (!s || !st || (st->n_prefills && !st->prefills) || (st->n_decodes && !st->decodes)) return LMH_INVALID_ARGUMENT;
  for (uint64_t i = 0; i < st->n_prefills; i++) {
    Slot* q = s->find(st->prefills[i].slot);
    if (!q) continue;
    if (st->prefills[i].end >= q->prompt.size()) {
      q->decoding = true;
      q->done = q->prompt.size();
    } else {
      q->decoding = false;
      q->done = st->prefills[i].end;
    }
  }
  for (uint64_t i = 0; i < st->n_decodes; i++) {
    Slot* q = s->find(st->decodes[i]);
    if (q) q->generated++;
  }
  return LMH_OK;
}

int32_t lmh_sched_finish(lmh_sched* s, uint32_t slot) {
  if (s && s->kv_gone) return LMH_INVALID_ARGUMENT;
  if (!s) return LMH_INVALID_ARGUMENT;
  for (size_t i = 0; i < s->slots.size(); i++)
    if (s->slots[i].id == slot) {
      Slot v = std::move(s->slots[i]);
      s->slots.erase(s->slots.begin() + i);
      s->release(v);
      break;
    }
  return LMH_OK;
}

int32_t lmh_sched_publish(lmh_sched* s, uint32_t slot, const uint32_t* tokens, uint64_t n) {
  if (s && s->kv_gone) return LMH_INVALID_ARGUMENT;
  if (!s) return LMH_INVALID_ARGUMENT;
  Slot* q = s->find(slot);
  if (!q) return s->fail(LMH_INVALID_ARGUMENT, "no such slot");
  if (!tokens) {  // the slot's own prompt
    if (n > q->prompt.size()) return s->fail(LMH_INVALID_ARGUMENT, "more tokens than the prompt holds");
    tokens = q->prompt.data();
  }
  BlockPool& p = s->pool();
  const uint64_t full = n / p.block_tokens;
  const std::vector<uint32_t>& blocks = s->blocks_of(*q);
  if (full > blocks.size()) return s->fail(LMH_INVALID_ARGUMENT, "more full blocks than the slot holds");
  if (s->kv && full * p.block_tokens > kv_seq_len(s->kv, q->kv_seq))
    return s->fail(LMH_INVALID_ARGUMENT, "publishing positions the sequence has not written");
  // Sequence::publish hashes every full block of tokens[0..n]; the slot's memo of earlier hashes
  // stands in for the blocks whose tokens it covers unchanged.
  const uint32_t bt = p.block_tokens;
  size_t k = 0;
  const size_t have = std::min<size_t>(q->chain.size(), full);
  while (k < have && std::memcmp(q->chain_tokens.data() + k * bt, tokens + k * bt, bt * 4) == 0) k++;
  if (k < have) {  // the tokens differ from the memo's from block k on
    q->chain.resize(k);
    q->chain_tokens.resize(k * bt);
  }
  for (size_t i = q->chain.size(); i < full; i++) {
    q->chain.push_back(block_hash(i ? &q->chain[i - 1] : nullptr, tokens + i * bt, bt, s->extra));
    q->chain_tokens.insert(q->chain_tokens.end(), tokens + i * bt, tokens + (i + 1) * bt);
  }
  for (uint64_t i = 0; i < full; i++) p.set_hash(blocks[i], q->chain[i]);
  return LMH_OK;
}

int32_t lmh_sched_prepare(lmh_sched* s, const lmh_step* st, lmh_seg* segs_out, uint64_t* n_rows, uint64_t* needed,
                          uint64_t* free_blocks) {
  if (s && s->kv_gone) return LMH_INVALID_ARGUMENT;
  if (!s || !st || !segs_out || (st->n_prefills && !st->prefills) || (st->n_decodes && !st->decodes))
    return LMH_INVALID_ARGUMENT;
  if (!s->kv) return s->fail(LMH_INVALID_ARGUMENT, "the scheduler is not bound to a KV handle");
  std::vector<lmh_seq_tokens> batch;
  batch.reserve(st->n_decodes + st->n_prefills);
  for (uint64_t i = 0; i < st->n_decodes; i++) {
    const Slot* q = s->find(st->decodes[i]);
    if (!q || !q->decoding) return s->fail(LMH_INVALID_ARGUMENT, "decode of a slot that is not decoding");
    batch.push_back(lmh_seq_tokens{q->kv_seq, 1});
  }
  for (uint64_t i = 0; i < st->n_prefills; i++) {
    const lmh_prefill_range& r = st->prefills[i];
    const Slot* q = s->find(r.slot);
    if (!q || q->decoding || r.end <= r.start || r.end > q->prompt.size())
      return s->fail(LMH_INVALID_ARGUMENT, "prefill range outside a prefilling slot's prompt");
    if (r.start != kv_seq_len(s->kv, q->kv_seq))
      return s->fail(LMH_INVALID_ARGUMENT, "prefill range does not start at the sequence's length");
    batch.push_back(lmh_seq_tokens{q->kv_seq, r.end - r.start});
  }
  if (batch.empty()) return s->fail(LMH_INVALID_ARGUMENT, "empty step");
  const int32_t rc = lmh_batch_prepare(s->kv, batch.data(), batch.size(), segs_out, n_rows, needed, free_blocks);
  if (rc != LMH_OK) s->err = lmh_kv_last_error(s->kv);
  return rc;
}

int32_t lmh_sched_get_stats(const lmh_sched* s, lmh_sched_stats* o) {
  if (s && s->kv_gone) return LMH_INVALID_ARGUMENT;
  if (!s || !o) return LMH_INVALID_ARGUMENT;
  const BlockPool& p = s->pool();
  o->slots = s->slots.size();
  o->queued = s->queue.size();
  o->retractions = s->retractions;
  o->n_blocks = p.meta.size();
  o->free = p.free_blocks();
  o->cached_free = p.cached_free_blocks();
  o->hits = p.hits;
  o->misses = p.misses;
  o->evictions = p.evictions;
  return LMH_OK;
}

int32_t lmh_sched_slots(const lmh_sched* s, uint32_t* ids, uint64_t cap, uint64_t* n) {
  if (s && s->kv_gone) return LMH_INVALID_ARGUMENT;
  if (!s || !n || (cap > 0 && !ids)) return LMH_INVALID_ARGUMENT;
  *n = s->slots.size();
  for (uint64_t i = 0; i < std::min<uint64_t>(cap, s->slots.size()); i++) ids[i] = s->slots[i].id;
  return LMH_OK;
}

int32_t lmh_sched_slot(const lmh_sched* s, uint32_t slot, lmh_slot_info* o) {
  if (s && s->kv_gone) return LMH_INVALID_ARGUMENT;
  if (!s || !o) return LMH_INVALID_ARGUMENT;
  const Slot* q = s->find(slot);
  if (!q) return LMH_INVALID_ARGUMENT;
  *o = lmh_slot_info{};
  o->id = q->id;
  o->priority = q->priority;
  o->decoding = q->decoding ? 1 : 0;
  o->done = q->done;
  o->n_prompt = q->prompt.size();
  o->max_new = q->max_new;
  o->generated = q->generated;
  o->seq_no = q->seq_no;
  o->kv_seq = q->kv_seq;
  o->n_blocks = s->blocks_of(*q).size();
  return LMH_OK;
}

int32_t lmh_sched_slot_blocks(const lmh_sched* s, uint32_t slot, uint32_t* out, uint64_t cap, uint64_t* n) {
  if (s && s->kv_gone) return LMH_INVALID_ARGUMENT;
  if (!s || !n || (cap > 0 && !out)) return LMH_INVALID_ARGUMENT;
  const Slot* q = s->find(slot);
  if (!q) return LMH_INVALID_ARGUMENT;
  const std::vector<uint32_t>& b = s->blocks_of(*q);
  *n = b.size();
  for (uint64_t i = 0; i < std::min<uint64_t>(cap, b.size()); i++) out[i] = b[i];
  return LMH_OK;
}

int32_t lmh_sched_queued_at(const lmh_sched* s, uint64_t i, lmh_queued_info* o) {
  if (s && s->kv_gone) return LMH_INVALID_ARGUMENT;
  if (!s || !o || i >= s->queue.size()) return LMH_INVALID_ARGUMENT;
  const Queued& q = s->queue[i];
  *o = lmh_queued_info{q.seq_no, q.prompt.size(), q.max_new, q.priority, 0};
  return LMH_OK;
}

int32_t lmh_sha256(const uint8_t* msg, uint64_t n, int32_t path, uint8_t out[32]) {
  if ((n > 0 && !msg) || !out || path < -1 || path > 1) return LMH_INVALID_ARGUMENT;
  if (path < 0) {
    Sha256 h;
    h.update(msg, n);
    const Hash d = h.finish();
    std::memcpy(out, d.data(), 32);
    return LMH_OK;
  }
  // the same padding as Sha256::finish, compressed by the requested path
  std::vector<uint8_t> m(msg, msg + n);
  m.push_back(0x80);
  while (m.size() % 64 != 56) m.push_back(0);
  for (int i = 0; i < 8; i++) m.push_back((uint8_t)((uint64_t)n * 8 >> (56 - 8 * i)));
  uint32_t st[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au, 0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
  if (!sha256_compress_path(path, st, m.data(), m.size() / 64)) return LMH_UNSUPPORTED;
  for (int i = 0; i < 8; i++)
    for (int j = 0; j < 4; j++) out[4 * i + j] = (uint8_t)(st[i] >> (24 - 8 * j));
  return LMH_OK;
}

int32_t lmh_chain_hashes(const uint32_t* tokens, uint64_t n, uint32_t block_tokens, const lmh_sched_options* key,
                         uint8_t* out, uint64_t cap, uint64_t* n_hashes) {
  if (!key || !n_hashes || block_tokens == 0 || (n > 0 && !tokens) || (cap > 0 && !out)) return LMH_INVALID_ARGUMENT;
  if ((key->model_digest_len && !key->model_digest) || (key->salt_len && !key->salt)) return LMH_INVALID_ARGUMENT;
  const std::vector<Hash> h = chain_hashes(tokens, n, block_tokens, key_extra(key));
  *n_hashes = h.size();
  for (uint64_t i = 0; i < std::min<uint64_t>(cap, h.size()); i++) memcpy(out + 32 * i, h[i].data(), 32);
  return LMH_OK;
}

}  // extern "C"

namespace lmh {
// The bound handle is being destroyed: its sequences (and the slots' blocks) go with it.
void sched_kv_destroyed(lmh_sched* s) {
  s->kv = nullptr;
  s->kv_gone = true;
  s->slots.clear();
  s->err = "the KV handle this scheduler was bound to was destroyed";
}
}  // namespace lmh
