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
#include <deque>
#include <map>
#include <string>
#include <vector>

namespace lmh {

using Hash = std::array<uint8_t, 32>;

struct BlockMeta {
  uint32_t refs = 0;
  bool has_hash = false;
  Hash hash{};
};

struct BlockPool {
  std::vector<BlockMeta> meta;
  std::deque<uint32_t> free_q;
  std::map<Hash, uint32_t> by_hash;
  uint64_t hits = 0, misses = 0, evictions = 0;
  uint32_t block_tokens = 16;

  void init(uint64_t n_blocks, uint32_t bt) {
    block_tokens = bt;
    meta.assign(n_blocks, BlockMeta{});
    free_q.clear();
    by_hash.clear();
    hits = misses = evictions = 0;
    for (uint64_t i = 0; i < n_blocks; i++) free_q.push_back((uint32_t)i);
  }
  uint64_t free_blocks() const { return free_q.size(); }
  // lib.rs:93-109: n blocks LRU-first, evicting cached content; false (nothing taken) if short
  bool alloc(uint64_t n, std::vector<uint32_t>& out) {
    if (free_q.size() < n) return false;
    for (uint64_t i = 0; i < n; i++) {
      const uint32_t b = free_q.front();
      free_q.pop_front();
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
    if (--m.refs == 0) free_q.push_back(b);
  }
  // lib.rs:113-118
  void set_hash(uint32_t b, const Hash& h) {
    BlockMeta& m = meta[b];
    if (m.has_hash) by_hash.erase(m.hash);
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
  }
  // lib.rs:132-143: a free cached block leaves the free queue, an in-use one gains a reference
  bool reclaim(const Hash& h, uint32_t& b) {
    auto it = by_hash.find(h);
    if (it == by_hash.end()) return false;
    b = it->second;
    BlockMeta& m = meta[b];
    if (m.refs == 0) {
      for (auto q = free_q.begin(); q != free_q.end(); ++q)
        if (*q == b) {
          free_q.erase(q);
          break;
        }
    }
    m.refs++;
    hits++;
    return true;
  }
  void note_miss() { misses++; }
};

// SHA-256 (FIPS 180-4), streaming.
class Sha256 {
 public:
  Sha256() {
    static const uint32_t h0[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                                   0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
    for (int i = 0; i < 8; i++) h_[i] = h0[i];
  }
  void update(const uint8_t* p, size_t n) {
    len_ += n;
    while (n > 0) {
      const size_t take = std::min<size_t>(64 - fill_, n);
      for (size_t i = 0; i < take; i++) buf_[fill_ + i] = p[i];
      fill_ += take;
      p += take;
      n -= take;
      if (fill_ == 64) {
        block(buf_);
        fill_ = 0;
      }
    }
  }
  Hash finish() {
    const uint64_t bits = len_ * 8;
    const uint8_t one = 0x80, zero = 0;
    update(&one, 1);
    while (fill_ != 56) update(&zero, 1);
    uint8_t lb[8];
    for (int i = 0; i < 8; i++) lb[i] = (uint8_t)(bits >> (56 - 8 * i));
    update(lb, 8);
    Hash out;
    for (int i = 0; i < 8; i++)
      for (int j = 0; j < 4; j++) out[4 * i + j] = (uint8_t)(h_[i] >> (24 - 8 * j));
    return out;
  }

 private:
  static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }
  void block(const uint8_t* p) {
    static const uint32_t k[64] = {
        0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u, 0x923f82a4u, 0xab1c5ed5u,
        0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u, 0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u,
        0xe49b69c1u, 0xefbe4786u, 0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
        0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u, 0x06ca6351u, 0x14292967u,
        0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u, 0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u,
        0xa2bfe8a1u, 0xa81a664bu, 0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
        0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au, 0x5b9cca4fu, 0x682e6ff3u,
        0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u, 0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};
    uint32_t w[64];
    for (int i = 0; i < 16; i++)
      w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 | p[4 * i + 3];
    for (int i = 16; i < 64; i++) {
      const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
      const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
      w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = h_[0], b = h_[1], c = h_[2], d = h_[3], e = h_[4], f = h_[5], g = h_[6], h = h_[7];
    for (int i = 0; i < 64; i++) {
      const uint32_t t1 = h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + k[i] + w[i];
      const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
      h = g;
      g = f;
      f = e;
      e = d + t1;
      d = c;
      c = b;
      b = a;
      a = t1 + t2;
    }
    h_[0] += a;
    h_[1] += b;
    h_[2] += c;
    h_[3] += d;
    h_[4] += e;
    h_[5] += f;
    h_[6] += g;
    h_[7] += h;
  }
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

// block_hash / chain_hashes (lib.rs:216-241): one hash per full block of `tokens`
inline std::vector<Hash> chain_hashes(const uint32_t* tokens, size_t n, uint32_t bt, const std::vector<uint8_t>& extra) {
  std::vector<Hash> out;
  Hash parent{};
  for (size_t b = 0; b + bt <= n; b += bt) {
    Sha256 h;
    h.update(parent.data(), 32);  // the first block hashes 32 zero bytes in place of a parent
    for (size_t i = 0; i < bt; i++) {
      const uint32_t t = tokens[b + i];
      const uint8_t le[4] = {(uint8_t)t, (uint8_t)(t >> 8), (uint8_t)(t >> 16), (uint8_t)(t >> 24)};
      h.update(le, 4);
    }
    h.update(extra.data(), extra.size());
    parent = h.finish();
    out.push_back(parent);
  }
  return out;
}

}  // namespace lmh
