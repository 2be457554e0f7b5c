// pool.h — the block pool and the prefix-cache hash chain, shared by the KV handle (host.cpp) and
// the scheduler (sched.cpp). Host-side bookkeeping only.
//
//   BlockPool     kv/src/lib.rs:36-176: refcounted block ids, an LRU free queue whose blocks keep
//                 their content hash until they are handed out again, reclaim by hash.
//   block_hash    kv/src/lib.rs:216-241: SHA-256 over (parent hash or 32 zero bytes, the block's
//                 tokens as little-endian u32, the cache key's extra bytes); one hash per full block.
//   CacheKey      kv/src/lib.rs:188-213: model digest, KV types, RoPE parameters, template hash and
//                 the client salt, NUL-separated.
#pragma once

#include <stdint.h>

#include <algorithm>
#include <array>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

namespace lmh {

using Hash = std::array<uint8_t, 32>;

// A content hash is SHA-256 output, so its first 8 bytes already spread keys evenly.
struct HashKey {
  size_t operator()(const Hash& h) const {
    uint64_t x;
    std::memcpy(&x, h.data(), 8);
    return (size_t)x;
  }
};

struct BlockMeta {
  uint32_t refs = 0;
  bool has_hash = false;
  Hash hash{};
  uint32_t prev = 0xffffffffu, next = 0xffffffffu;  // free-queue links (held while refs == 0)
};

// The block pool of kv/src/lib.rs:75-186. The LRU free queue is a list threaded through the
// blocks' metadata (a block is on it exactly while it has no references), so taking a cached block
// back out of the middle (reclaim) is O(1) where a queue scan would cost O(free blocks); the free
// and cached-free counts are kept as the queue changes.
struct BlockPool {
  static constexpr uint32_t NIL = 0xffffffffu;
  std::vector<BlockMeta> meta;
  uint32_t head = NIL, tail = NIL;
  uint64_t n_free = 0, n_cached_free = 0;
  std::unordered_map<Hash, uint32_t, HashKey> by_hash;
  uint64_t hits = 0, misses = 0, evictions = 0;
  uint32_t block_tokens = 16;

  void init(uint64_t n_blocks, uint32_t bt) {
    block_tokens = bt;
    meta.assign(n_blocks, BlockMeta{});
    head = tail = NIL;
    n_free = n_cached_free = 0;
    by_hash.clear();
    hits = misses = evictions = 0;
    for (uint64_t i = 0; i < n_blocks; i++) push_free((uint32_t)i);
  }
  uint64_t free_blocks() const { return n_free; }
  uint64_t cached_free_blocks() const { return n_cached_free; }
  bool is_free(uint32_t b) const { return meta[b].refs == 0; }
  // append to the back of the free queue / unlink from anywhere in it
  void push_free(uint32_t b) {
    BlockMeta& m = meta[b];
    m.prev = tail;
    m.next = NIL;
    if (tail != NIL) meta[tail].next = b;
    else head = b;
    tail = b;
    n_free++;
    if (m.has_hash) n_cached_free++;
  }
  void unlink_free(uint32_t b) {
    BlockMeta& m = meta[b];
    if (m.prev != NIL) meta[m.prev].next = m.next;
    else head = m.next;
    if (m.next != NIL) meta[m.next].prev = m.prev;
    else tail = m.prev;
    m.prev = m.next = NIL;
    n_free--;
    if (m.has_hash) n_cached_free--;
  }
  // lib.rs:93-109: n blocks LRU-first, evicting cached content; false (nothing taken) if short
  bool alloc(uint64_t n, std::vector<uint32_t>& out) {
    if (n_free < n) return false;
    for (uint64_t i = 0; i < n; i++) {
      const uint32_t b = head;
      unlink_free(b);
      BlockMeta& m = meta[b];
      if (m.has_hash) {
        by_hash.erase(m.hash);
        m.has_hash = false;
        evictions++;
      }
      m.refs = 1;
      out.push_back(b);
    }
    return true;
  }
  // lib.rs:121-128: at zero references the block joins the back of the free queue, hash kept
  void release(uint32_t b) {
    BlockMeta& m = meta[b];
    if (m.refs == 0) return;
    if (--m.refs == 0) push_free(b);
  }
  // lib.rs:113-118 (a call that would change nothing returns early)
  void set_hash(uint32_t b, const Hash& h) {
    BlockMeta& m = meta[b];
    if (m.has_hash && m.hash == h) {
      auto it = by_hash.find(h);
      if (it != by_hash.end() && it->second == b) return;
    }
    if (m.has_hash) by_hash.erase(m.hash);
    else if (m.refs == 0) n_cached_free++;
    m.hash = h;
    m.has_hash = true;
    by_hash[h] = b;
  }
  // lib.rs:161-167
  void clear_hash(uint32_t b) {
    BlockMeta& m = meta[b];
    if (!m.has_hash) return;
    auto it = by_hash.find(m.hash);
    if (it != by_hash.end() && it->second == b) by_hash.erase(it);
    m.has_hash = false;
    if (m.refs == 0) n_cached_free--;
  }
  // lib.rs:132-143: a free cached block leaves the free queue, an in-use one gains a reference
  bool reclaim(const Hash& h, uint32_t& b) {
    auto it = by_hash.find(h);
    if (it == by_hash.end()) return false;
    b = it->second;
    if (meta[b].refs == 0) unlink_free(b);
    meta[b].refs++;
    hits++;
    return true;
  }
  void note_miss() { misses++; }
};

// SHA-256 (FIPS 180-4), streaming. The compression function runs on the x86 SHA extensions when
// the host has them (checked once at run time), else in portable scalar code; both give the same
// digest.
void sha256_compress(uint32_t state[8], const uint8_t* data, size_t blocks);  // sha256.cpp
// Test hook: path 0 = scalar, 1 = SHA extensions (false if this host lacks them).
bool sha256_compress_path(int path, uint32_t state[8], const uint8_t* data, size_t blocks);

class Sha256 {
 public:
  Sha256() {
    static const uint32_t h0[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                                   0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
    for (int i = 0; i < 8; i++) h_[i] = h0[i];
  }
  void update(const uint8_t* p, size_t n) {
    len_ += n;
    if (fill_) {
      const size_t take = std::min<size_t>(64 - fill_, n);
      std::memcpy(buf_ + fill_, p, take);
      fill_ += take;
      p += take;
      n -= take;
      if (fill_ < 64) return;
      sha256_compress(h_, buf_, 1);
      fill_ = 0;
    }
    if (n >= 64) {
      sha256_compress(h_, p, n / 64);
      p += n / 64 * 64;
      n %= 64;
    }
    std::memcpy(buf_, p, n);
    fill_ = n;
  }
  Hash finish() {
    const uint64_t bits = len_ * 8;
    buf_[fill_++] = 0x80;
    if (fill_ > 56) {
      std::memset(buf_ + fill_, 0, 64 - fill_);
      sha256_compress(h_, buf_, 1);
      fill_ = 0;
    }
    std::memset(buf_ + fill_, 0, 56 - fill_);
    for (int i = 0; i < 8; i++) buf_[56 + i] = (uint8_t)(bits >> (56 - 8 * i));
    sha256_compress(h_, buf_, 1);
    Hash out;
    for (int i = 0; i < 8; i++)
      for (int j = 0; j < 4; j++) out[4 * i + j] = (uint8_t)(h_[i] >> (24 - 8 * j));
    return out;
  }

 private:
  uint32_t h_[8];
  uint8_t buf_[64];
  size_t fill_ = 0;
  uint64_t len_ = 0;
};

// CacheKey::extra (lib.rs:200-213): the key fields NUL-separated
inline std::vector<uint8_t> cache_key_extra(const std::vector<uint8_t>& digest, const std::string& kv_types,
                                            const std::string& rope, const std::string& tmpl,
                                            const std::vector<uint8_t>& salt) {
  std::vector<uint8_t> v(digest);
  v.push_back(0);
  v.insert(v.end(), kv_types.begin(), kv_types.end());
  v.push_back(0);
  v.insert(v.end(), rope.begin(), rope.end());
  v.push_back(0);
  v.insert(v.end(), tmpl.begin(), tmpl.end());
  v.push_back(0);
  v.insert(v.end(), salt.begin(), salt.end());
  return v;
}

// block_hash (lib.rs:216-227): SHA-256 of the parent hash (32 zero bytes for the first block), the
// block's tokens as little-endian u32 and the cache key's extra bytes
inline Hash block_hash(const Hash* parent, const uint32_t* tokens, uint32_t bt, const std::vector<uint8_t>& extra) {
  static const Hash zero{};
  Sha256 h;
  h.update((parent ? *parent : zero).data(), 32);
  uint8_t le[64];
  for (uint32_t i = 0; i < bt; i += 16) {
    const uint32_t m = std::min<uint32_t>(16, bt - i);
    for (uint32_t j = 0; j < m; j++) {
      const uint32_t t = tokens[i + j];
      le[4 * j] = (uint8_t)t;
      le[4 * j + 1] = (uint8_t)(t >> 8);
      le[4 * j + 2] = (uint8_t)(t >> 16);
      le[4 * j + 3] = (uint8_t)(t >> 24);
    }
    h.update(le, 4 * m);
  }
  h.update(extra.data(), extra.size());
  return h.finish();
}

// chain_hashes (lib.rs:230-239): one hash per full block of `tokens`
inline std::vector<Hash> chain_hashes(const uint32_t* tokens, size_t n, uint32_t bt, const std::vector<uint8_t>& extra) {
  std::vector<Hash> out;
  out.reserve(n / bt);
  for (size_t b = 0; b + bt <= n; b += bt) out.push_back(block_hash(out.empty() ? nullptr : &out.back(), tokens + b, bt, extra));
  return out;
}

}  // namespace lmh
