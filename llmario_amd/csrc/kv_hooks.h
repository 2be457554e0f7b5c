// kv_hooks.h — what the scheduler (sched.cpp) needs of a KV handle (host.cpp) when it is bound to
// one: the handle's block pool, and binding a sequence slot to a block list the scheduler acquired.
// C++ linkage, library-internal.
#pragma once

#include <stdint.h>

#include <vector>

#include "pool.h"

struct lmh_kv;
struct lmh_sched;

namespace lmh {

BlockPool& kv_pool(lmh_kv* kv);
uint64_t kv_n_seqs(const lmh_kv* kv);
uint64_t kv_max_ctx(const lmh_kv* kv);
// true when the handle has sliding-window layers (their rows are not kept for prefix reuse)
bool kv_has_window(const lmh_kv* kv);
uint64_t kv_seq_len(const lmh_kv* kv, uint64_t seq);
// true when sequence `seq` holds no blocks and no positions (free for binding)
bool kv_seq_empty(const lmh_kv* kv, uint64_t seq);
const std::vector<uint32_t>& kv_seq_blocks(const lmh_kv* kv, uint64_t seq);
// Give the empty sequence `seq` the blocks (already referenced for it in the pool) and length
// `len`; blocks not yet resident are zeroed before the next device call, as reserve does.
void kv_bind_seq(lmh_kv* kv, uint64_t seq, const std::vector<uint32_t>& blocks, uint64_t len);
// Release every block of `seq` and set its length to zero (KvCache::clear_seq).
void kv_clear_seq(lmh_kv* kv, uint64_t seq);
// Set the handle's last error message (returned by lmh_kv_last_error).
void kv_set_error(lmh_kv* kv, const char* msg);
// A scheduler bound to the handle registers itself, so that destroying the handle first leaves
// the scheduler detached (sched_kv_destroyed) instead of pointing at freed memory.
void kv_attach(lmh_kv* kv, lmh_sched* s);
void kv_detach(lmh_kv* kv, lmh_sched* s);
void sched_kv_destroyed(lmh_sched* s);  // defined in sched.cpp

}  // namespace lmh
