// oracle.cpp — CPU restatement of LLMario's paged-KV attention path.
//
// TEST INFRASTRUCTURE ONLY: the checker for the HIP path, never the product and never the thing
// measured on the GPU. See oracle.h for the pinning plan. Citations are path:line relative to
// the reference root (crates/engine/...).
//
// Floating-point order: every loop keeps the reference's evaluation order. Build with
// -ffp-contract=off (Rust never contracts a*b+c into an FMA) and without -ffast-math.

#include "oracle.h"

#include <algorithm>
#include <array>
#include <atomic>
#include <condition_variable>
#include <cmath>
#include <cstring>
#include <deque>
#include <map>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

namespace {

// ---------------------------------------------------------------------------------------------
// Codecs
// ---------------------------------------------------------------------------------------------

inline uint32_t f32_bits(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  return u;
}
inline float bits_f32(uint32_t u) {
  float x;
  std::memcpy(&x, &u, 4);
  return x;
}

// IEEE-754 binary32 -> binary16, round to nearest, ties to even: what `half` 2.7.1's
// `f16::from_f32` computes (kv.rs:122, 166), in software.
uint16_t f16_from_f32(float f) {
  const uint32_t x = f32_bits(f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exp = (x >> 23) & 0xffu;
  uint32_t man = x & 0x7fffffu;
  if (exp == 0xffu) {
    if (man == 0) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | 0x7e00u | (man >> 13));  // quiet NaN, payload kept
  }
  const int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    man |= 0x800000u;
    const int shift = 14 - e;
    uint32_t hm = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (hm & 1u))) hm++;
    return (uint16_t)(sign | hm);
  }
  uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
  const uint32_t rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;  // a carry rounds up into the exponent
  return (uint16_t)h;
}

float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  if (exp == 0) {
    if (man == 0) return bits_f32(sign);
    // subnormal: value = man * 2^-24, exact in f32
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  if (exp == 31) return bits_f32(sign | 0x7f800000u | (man << 13));
  return bits_f32(sign | ((exp - 15 + 127) << 23) | (man << 13));
}

// bfloat16 extension (the reference has no BF16 cache type; core/src/dequant.rs:20-22 defines
// its decode as `bits << 16`). Encode: round to nearest even on the dropped 16 bits.
uint16_t bf16_from_f32(float f) {
  uint32_t x = f32_bits(f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}
float bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

constexpr size_t Q8_BLOCK = 32;  // kv.rs:66
constexpr size_t Q8_BYTES = 34;  // kv.rs:67

// kv.rs:94-99 (+ F32 / BF16 extensions)
size_t row_bytes(int t, size_t n) {
  switch (t) {
    case ORC_KV_F16: return 2 * n;
    case ORC_KV_Q8_0: return (n + Q8_BLOCK - 1) / Q8_BLOCK * Q8_BYTES;
    case ORC_KV_F32: return 4 * n;
    case ORC_KV_BF16: return 2 * n;
  }
  return 0;
}

// kv.rs:156-171: per 32 values d = amax/127, id = d ? 1/d : 0, q = round_ties_even(x*id).
void quantize_q8_0(const float* src, size_t n, uint8_t* dst) {
  for (size_t b = 0; b < n / Q8_BLOCK; b++) {
    const float* blk = src + b * Q8_BLOCK;
    uint8_t* out = dst + b * Q8_BYTES;
    float amax = 0.0f;
    for (size_t i = 0; i < Q8_BLOCK; i++) amax = std::fmax(amax, std::fabs(blk[i]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = f16_from_f32(d);
    out[0] = (uint8_t)(dh & 0xff);
    out[1] = (uint8_t)(dh >> 8);
    for (size_t i = 0; i < Q8_BLOCK; i++) {
      // round_ties_even; `as i32` saturates in Rust, values here are within ±128
      const float r = std::nearbyint(blk[i] * id);
      int32_t qi = r >= 2147483647.0f ? 2147483647 : (r <= -2147483648.0f ? (int32_t)-2147483647 - 1 : (int32_t)r);
      out[2 + i] = (uint8_t)(int8_t)qi;
    }
  }
}

// kv.rs:174-184
void dequantize_q8_0(const uint8_t* src, size_t n, float* out) {
  for (size_t b = 0; b < n / Q8_BLOCK; b++) {
    const uint8_t* blk = src + b * Q8_BYTES;
    const float d = f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    for (size_t i = 0; i < Q8_BLOCK; i++) out[b * Q8_BLOCK + i] = (float)(int8_t)blk[2 + i] * d;
  }
}

// KvType::store (kv.rs:112-126)
void store_row(int t, const float* src, size_t n, uint8_t* dst) {
  switch (t) {
    case ORC_KV_F16:
      for (size_t i = 0; i < n; i++) {
        uint16_t h = f16_from_f32(src[i]);
        std::memcpy(dst + 2 * i, &h, 2);
      }
      break;
    case ORC_KV_Q8_0: quantize_q8_0(src, n, dst); break;
    case ORC_KV_F32: std::memcpy(dst, src, 4 * n); break;
    case ORC_KV_BF16:
      for (size_t i = 0; i < n; i++) {
        uint16_t h = bf16_from_f32(src[i]);
        std::memcpy(dst + 2 * i, &h, 2);
      }
      break;
  }
}

// KvType::load (kv.rs:131-151): elements start..start+len of a row.
void load_row(int t, const uint8_t* src, size_t start, size_t len, float* out) {
  switch (t) {
    case ORC_KV_F16:
      for (size_t i = 0; i < len; i++) {
        uint16_t h;
        std::memcpy(&h, src + 2 * (start + i), 2);
        out[i] = f16_to_f32(h);
      }
      break;
    case ORC_KV_Q8_0: dequantize_q8_0(src + start / Q8_BLOCK * Q8_BYTES, len, out); break;
    case ORC_KV_F32: std::memcpy(out, src + 4 * start, 4 * len); break;
    case ORC_KV_BF16:
      for (size_t i = 0; i < len; i++) {
        uint16_t h;
        std::memcpy(&h, src + 2 * (start + i), 2);
        out[i] = bf16_to_f32(h);
      }
      break;
  }
}

// ---------------------------------------------------------------------------------------------
// BlockPool (kv/src/lib.rs:36-176)
// ---------------------------------------------------------------------------------------------

using Hash = std::array<uint8_t, 32>;

struct Meta {
  uint32_t refs = 0;
  bool has_hash = false;
  Hash hash{};
};

}  // namespace

struct orc_pool {
  uint64_t block_tokens, block_bytes;
  std::vector<Meta> meta;
  std::deque<uint32_t> free;  // LRU order, front = evict first
  std::map<Hash, uint32_t> by_hash;
  uint64_t hits = 0, misses = 0, evictions = 0;

  orc_pool(uint64_t n, uint64_t bt, uint64_t bb) : block_tokens(bt), block_bytes(bb), meta(n) {
    for (uint64_t i = 0; i < n; i++) free.push_back((uint32_t)i);
  }
  // lib.rs:93-109
  bool alloc(uint64_t n, std::vector<uint32_t>& out) {
    if (free.size() < n) return false;
    for (uint64_t i = 0; i < n; i++) {
      uint32_t b = free.front();
      free.pop_front();
      Meta& m = meta[b];
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
  // lib.rs:113-118
  void set_hash(uint32_t b, const Hash& h) {
    Meta& m = meta[b];
    if (m.has_hash) by_hash.erase(m.hash);
    m.hash = h;
    m.has_hash = true;
    by_hash[h] = b;
  }
  // lib.rs:121-128
  void release(uint32_t b) {
    Meta& m = meta[b];
    if (m.refs == 0) std::abort();  // "double release"
    m.refs--;
    if (m.refs == 0) free.push_back(b);
  }
  // lib.rs:132-143
  bool reclaim(const Hash& h, uint32_t* out) {
    auto it = by_hash.find(h);
    if (it == by_hash.end()) return false;
    uint32_t b = it->second;
    Meta& m = meta[b];
    if (m.refs == 0) {
      auto pos = std::find(free.begin(), free.end(), b);
      if (pos != free.end()) free.erase(pos);
    }
    m.refs++;
    hits++;
    *out = b;
    return true;
  }
  // lib.rs:161-167
  void clear_hash(uint32_t b) {
    Meta& m = meta[b];
    if (!m.has_hash) return;
    auto it = by_hash.find(m.hash);
    if (it != by_hash.end() && it->second == b) by_hash.erase(it);
    m.has_hash = false;
  }
};

namespace {

// ---------------------------------------------------------------------------------------------
// Layout (kv.rs:286-324, 402-497) — paged attention layers only
// ---------------------------------------------------------------------------------------------

struct Layer {
  size_t n_head, n_kv, hd, hdv;
  size_t kv_dim, v_dim, k_row, v_row;
  size_t off, rows;
  size_t k_off(size_t slot) const { return off + slot * k_row; }
  size_t v_off(size_t slot) const { return off + rows * k_row + slot * v_row; }
};

struct Layout {
  int kv_type;
  size_t max_ctx, block_tokens, block_bytes, blocks_per_seq, n_seqs, pool_blocks;
  std::vector<Layer> layers;
};

Layout make_layout(const orc_options& o, const orc_layer_geom* g, size_t n_layers) {
  Layout L{};
  L.kv_type = o.kv_type;
  L.max_ctx = std::max<size_t>(o.max_ctx, 1);
  L.block_tokens = o.block_tokens;
  size_t block_off = 0;
  for (size_t l = 0; l < n_layers; l++) {
    Layer y{};
    y.n_head = g[l].n_head;
    y.n_kv = g[l].n_kv;
    y.hd = g[l].hd;
    y.hdv = g[l].hdv;
    y.kv_dim = y.n_kv * y.hd;
    y.v_dim = y.n_kv * y.hdv;
    y.k_row = row_bytes(o.kv_type, y.kv_dim);
    y.v_row = row_bytes(o.kv_type, y.v_dim);
    y.off = block_off;
    y.rows = o.block_tokens;
    block_off += o.block_tokens * (y.k_row + y.v_row);
    L.layers.push_back(y);
  }
  L.n_seqs = std::max<size_t>(o.n_seqs, 1);
  L.blocks_per_seq = block_off > 0 ? (L.max_ctx + o.block_tokens - 1) / o.block_tokens : 0;
  if (block_off > 0) {
    if (o.pool_tokens > 0) {
      size_t t = std::max<size_t>(o.pool_tokens, 1);
      L.pool_blocks = std::min((t + o.block_tokens - 1) / o.block_tokens, L.n_seqs * L.blocks_per_seq) + L.n_seqs;
    } else {
      L.pool_blocks = L.n_seqs * (L.blocks_per_seq + 1);
    }
  }
  L.block_bytes = block_off;
  return L;
}

struct Seq {
  std::vector<uint32_t> blocks;
  size_t len = 0;
};

}  // namespace

// ---------------------------------------------------------------------------------------------
// KvCache (kv.rs:562-939)
// ---------------------------------------------------------------------------------------------

struct orc_cache {
  Layout lay;
  orc_pool pool;
  std::vector<std::vector<uint8_t>> backing;  // empty = not backed
  std::vector<Seq> seqs;

  orc_cache(const Layout& l)
      : lay(l), pool(l.pool_blocks, l.block_tokens, l.block_bytes), backing(l.pool_blocks), seqs(l.n_seqs) {}

  void back(uint32_t b) {
    if (backing[b].empty()) backing[b].assign(lay.block_bytes, 0);
  }
  void maybe_unback(uint32_t b) {
    if (pool.meta[b].refs == 0 && !pool.meta[b].has_hash) {
      std::vector<uint8_t>().swap(backing[b]);
    }
  }
  void release_block(uint32_t b) {
    pool.release(b);
    maybe_unback(b);
  }
  // kv.rs:715-725
  size_t blocks_needed(size_t s, size_t new_len) const {
    if (lay.block_bytes == 0) return 0;
    const size_t bt = lay.block_tokens;
    const Seq& q = seqs[s];
    size_t want = (new_len + bt - 1) / bt;
    size_t missing = want > q.blocks.size() ? want - q.blocks.size() : 0;
    bool cow = q.len % bt != 0 && q.len < new_len && pool.meta[q.blocks[q.len / bt]].refs > 1;
    return missing + (cow ? 1 : 0);
  }
  // kv.rs:730-785
  int reserve(size_t s, size_t new_len, uint64_t* needed, uint64_t* free_) {
    if (new_len > lay.max_ctx) return ORC_INVALID;
    if (lay.block_bytes == 0) return ORC_OK;
    const size_t bt = lay.block_tokens;
    const size_t len = seqs[s].len;
    size_t want = (new_len + bt - 1) / bt;
    size_t missing = want > seqs[s].blocks.size() ? want - seqs[s].blocks.size() : 0;
    size_t wanted = blocks_needed(s, new_len);
    bool cow = wanted > missing;
    if (pool.free.size() < wanted) {
      if (needed) *needed = wanted;
      if (free_) *free_ = pool.free.size();
      return ORC_KV_FULL;
    }
    if (len % bt != 0 && len < new_len) {
      size_t bi = len / bt;
      uint32_t old = seqs[s].blocks[bi];
      if (cow) {
        std::vector<uint32_t> nb;
        pool.alloc(1, nb);
        back(nb[0]);
        std::memcpy(backing[nb[0]].data(), backing[old].data(), lay.block_bytes);
        seqs[s].blocks[bi] = nb[0];
        release_block(old);
      } else {
        pool.clear_hash(old);
      }
    }
    if (missing > 0) {
      std::vector<uint32_t> fresh;
      pool.alloc(missing, fresh);
      for (uint32_t b : fresh) {
        back(b);
        seqs[s].blocks.push_back(b);
      }
    }
    return ORC_OK;
  }
  // kv.rs:792-816 (paged layers only: no rings, no recurrent state)
  void truncate(size_t s, size_t n) {
    size_t len = seqs[s].len;
    n = std::min(n, len);
    seqs[s].len = n;
    size_t keep = (n + lay.block_tokens - 1) / std::max<size_t>(lay.block_tokens, 1);
    while (seqs[s].blocks.size() > keep) {
      uint32_t b = seqs[s].blocks.back();
      seqs[s].blocks.pop_back();
      release_block(b);
    }
  }
  // kv.rs:820-827
  void clear(size_t s) {
    seqs[s].len = 0;
    while (!seqs[s].blocks.empty()) {
      uint32_t b = seqs[s].blocks.back();
      seqs[s].blocks.pop_back();
      release_block(b);
    }
  }
  // snapshot_bytes (kv.rs:1009-1028), paged layers only: whole blocks covering len tokens
  size_t snapshot_bytes(size_t len) const {
    if (len == 0 || lay.block_bytes == 0) return 0;
    return (len + lay.block_tokens - 1) / lay.block_tokens * lay.block_bytes;
  }
  // write_seq (kv.rs:1030-1056): the sequence's first ceil(len/bt) blocks, byte for byte
  void write_seq(size_t s, uint8_t* out) const {
    const size_t len = seqs[s].len, bt = lay.block_tokens, bb = lay.block_bytes;
    if (len == 0 || bb == 0) return;
    for (size_t i = 0; i < (len + bt - 1) / bt; i++) std::memcpy(out + i * bb, backing[seqs[s].blocks[i]].data(), bb);
  }
  // read_seq (kv.rs:1058-1130): room first (the sequence's own blocks count as available), else
  // KvFull with nothing changed; then clear, reserve and copy the blocks in
  int read_seq(size_t s, size_t len, const uint8_t* bytes, size_t n_bytes, uint64_t* needed, uint64_t* free_) {
    if (len > lay.max_ctx || n_bytes != snapshot_bytes(len)) return ORC_INVALID;
    const size_t bt = lay.block_tokens, bb = lay.block_bytes;
    const size_t nb = bb > 0 ? (len + bt - 1) / bt : 0;
    size_t own = 0;
    for (uint32_t b : seqs[s].blocks) own += pool.meta[b].refs == 1 ? 1 : 0;
    if (nb > pool.free.size() + own) {
      if (needed) *needed = nb;
      if (free_) *free_ = pool.free.size() + own;
      return ORC_KV_FULL;
    }
    clear(s);
    if (len == 0) return ORC_OK;
    reserve(s, len, nullptr, nullptr);
    for (size_t i = 0; i < seqs[s].blocks.size(); i++) std::memcpy(backing[seqs[s].blocks[i]].data(), bytes + i * bb, bb);
    seqs[s].len = len;
    return ORC_OK;
  }
  // kv.rs:839-866 (paged branch)
  uint8_t* row_ptr(size_t s, size_t l, size_t pos, bool v) const {
    const Layer& y = lay.layers[l];
    const size_t bt = lay.block_tokens;
    uint32_t b = seqs[s].blocks[pos / bt];
    const uint8_t* base = backing[b].data();
    size_t off = v ? y.v_off(pos % bt) : y.k_off(pos % bt);
    return const_cast<uint8_t*>(base + off);
  }
};

namespace {

// ---------------------------------------------------------------------------------------------
// LayerReader (kv.rs:1155-1188): block bases resolved once, row = bases[pos >> shift] + off
// ---------------------------------------------------------------------------------------------

struct Reader {
  int kv_type;
  const Layer* y;
  std::vector<const uint8_t*> bases;
  unsigned shift;
  size_t mask;
  const uint8_t* row(size_t pos, bool v) const {
    const uint8_t* base = bases[pos >> shift];
    size_t slot = pos & mask;
    return base + (v ? y->v_off(slot) : y->k_off(slot));
  }
  void load_k(size_t pos, size_t start, float* out, size_t len) const { load_row(kv_type, row(pos, false), start, len, out); }
  void load_v(size_t pos, size_t start, float* out, size_t len) const { load_row(kv_type, row(pos, true), start, len, out); }
};

Reader make_reader(const orc_cache* c, size_t s, size_t l) {
  Reader r;
  r.kv_type = c->lay.kv_type;
  r.y = &c->lay.layers[l];
  for (uint32_t b : c->seqs[s].blocks) r.bases.push_back(c->backing[b].data());
  unsigned sh = 0;
  while ((size_t(1) << sh) < c->lay.block_tokens) sh++;
  r.shift = sh;
  r.mask = c->lay.block_tokens - 1;
  return r;
}

// ---------------------------------------------------------------------------------------------
// ops (cpu/src/ops.rs:69-80, 127-151)
// ---------------------------------------------------------------------------------------------

// 16 independent lane sums, pairwise tree 16->1, then the scalar tail.
float dot(const float* a, const float* b, size_t n) {
  constexpr size_t L = 16;
  float acc[L] = {0};
  size_t full = n / L * L;
  for (size_t c = 0; c < full; c += L)
    for (size_t l = 0; l < L; l++) acc[l] += a[c + l] * b[c + l];
  size_t w = L;
  while (w > 1) {
    w /= 2;
    for (size_t l = 0; l < w; l++) acc[l] += acc[l + w];
  }
  float s = acc[0];
  for (size_t i = full; i < n; i++) s += a[i] * b[i];
  return s;
}

void softmax(float* x, size_t n) {
  float max = -INFINITY;
  for (size_t i = 0; i < n; i++) max = std::fmax(max, x[i]);
  float sum = 0.0f;
  for (size_t i = 0; i < n; i++) {
    x[i] = std::exp(x[i] - max);
    sum += x[i];
  }
  float inv = 1.0f / sum;
  for (size_t i = 0; i < n; i++) x[i] *= inv;
}

// ---------------------------------------------------------------------------------------------
// the cache's producer side: QK-norm and RoPE (cpu/src/ops.rs:18-66, forward.rs:427-453, 832-838)
// ---------------------------------------------------------------------------------------------

// rms_norm (ops.rs:18-29): y = x * (1 / sqrt(sum(x^2) / n + eps)) * w, the sum taken in order.
// w == nullptr: the weightless form (Metal's v_norm, misc.metal:218-226).
void rms_norm(const float* x, const float* w, float eps, float* y, size_t n) {
  float ss = 0.0f;
  for (size_t i = 0; i < n; i++) ss += x[i] * x[i];
  const float scale = 1.0f / std::sqrt(ss / (float)n + eps);
  for (size_t i = 0; i < n; i++) y[i] = w ? x[i] * scale * w[i] : x[i] * scale;
}

// per_head_norm (forward.rs:832-838): rms_norm of each hd-long head in place.
void per_head_norm(float* x, size_t n_heads, size_t hd, const float* w, float eps) {
  std::vector<float> tmp(hd);
  for (size_t h = 0; h < n_heads; h++) {
    rms_norm(x + h * hd, w, eps, tmp.data(), hd);
    std::memcpy(x + h * hd, tmp.data(), hd * 4);
  }
}

// rope (ops.rs:46-66): pairs i < rot_dim/2 rotate by angle = pos * freq_scale * freq with
// freq = theta^(-2i/rot_dim) in f32; (2i, 2i+1) for Normal, (i, i + rot_dim/2) for Neox; the
// rotation is scaled by attn_factor. freq_div (Metal's per-pair divisors, misc.metal:252-256)
// divides the angle when given.
void rope(float* x, size_t n_heads, size_t hd, uint32_t pos, const orc_rope_params* p) {
  const size_t half = p->rot_dim / 2;
  for (size_t h = 0; h < n_heads; h++) {
    float* head = x + h * hd;
    for (size_t i = 0; i < half; i++) {
      const float freq = std::pow(p->theta, -(2.0f * (float)i) / (float)p->rot_dim);
      float angle = (float)pos * p->freq_scale * freq;
      if (p->freq_div) angle = angle / p->freq_div[i];
      const float sn = std::sin(angle) * p->attn_factor, cs = std::cos(angle) * p->attn_factor;
      const size_t a = p->neox ? i : 2 * i, b = p->neox ? i + half : 2 * i + 1;
      const float x0 = head[a], x1 = head[b];
      head[a] = x0 * cs - x1 * sn;
      head[b] = x0 * sn + x1 * cs;
    }
  }
}

// ThreadPool (cpu/src/pool.rs:53-180): a persistent pool per thread count, its workers spinning
// for a bounded time on a new region, then parked on a condition variable; the caller is worker
// 0. parallel_for (pool.rs:115-180): `n_chunks = threads` contiguous chunks of ceil(n / n_chunks),
// claimed from a per-region counter (so a late worker only touches its own region's counters),
// and the caller waits until every chunk is done (spinning briefly, then sleeping).
class Pool {
 public:
  explicit Pool(size_t n) : n_threads_(n) {
    for (size_t i = 1; i < n; i++) workers_.emplace_back([this] { worker(); });
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> g(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    for (auto& t : workers_) t.join();
  }
  template <typename F>
  void run(size_t n, F& f) {
    auto job = std::make_shared<Job>();
    job->n_chunks = std::min(n_threads_, n);
    job->chunk = (n + job->n_chunks - 1) / job->n_chunks;
    job->n = n;
    job->ctx = &f;
    job->fn = [](void* c, size_t s, size_t e) { (*(F*)c)(s, e); };
    bool wake;
    {
      std::lock_guard<std::mutex> g(mu_);
      job_ = job;
      gen_.store(gen_.load(std::memory_order_relaxed) + 1, std::memory_order_release);
      wake = parked_ > 0;
    }
    if (wake) cv_.notify_all();
    run_chunks(*job);
    for (int i = 0; i < DONE_SPIN && job->done.load(std::memory_order_acquire) < job->n_chunks; i++) spin_pause();
    if (job->done.load(std::memory_order_acquire) < job->n_chunks) {
      std::unique_lock<std::mutex> g(done_mu_);
      done_cv_.wait(g, [&] { return job->done.load(std::memory_order_acquire) >= job->n_chunks; });
    }
    std::lock_guard<std::mutex> g(mu_);
    if (job_ == job) job_.reset();
  }

 private:
  struct Job {
    size_t n_chunks = 0, chunk = 0, n = 0;
    void* ctx = nullptr;
    void (*fn)(void*, size_t, size_t) = nullptr;
    std::atomic<size_t> next{0}, done{0};
  };
  static constexpr int SPIN = 40000, DONE_SPIN = 20000;   // pool.rs:60-62
  static void spin_pause() { __builtin_ia32_pause(); }
  void run_chunks(Job& j) {
    for (;;) {
      const size_t c = j.next.fetch_add(1, std::memory_order_acq_rel);
      if (c >= j.n_chunks) return;
      const size_t s = c * j.chunk, e = std::min(j.n, s + j.chunk);
      if (s < e) j.fn(j.ctx, s, e);
      if (j.done.fetch_add(1, std::memory_order_acq_rel) + 1 == j.n_chunks) {
        std::lock_guard<std::mutex> g(done_mu_);   // the caller may be about to sleep
        done_cv_.notify_all();
      }
    }
  }
  void worker() {
    uint64_t seen = 0;
    for (;;) {
      std::shared_ptr<Job> job;
      for (int i = 0; i < SPIN && !job; i++) {
        if (gen_.load(std::memory_order_acquire) != seen) {
          std::lock_guard<std::mutex> g(mu_);
          if (stop_) return;
          seen = gen_.load(std::memory_order_relaxed);
          job = job_;
        } else {
          spin_pause();
        }
      }
      if (!job) {
        std::unique_lock<std::mutex> g(mu_);
        parked_++;
        cv_.wait(g, [&] { return stop_ || gen_.load(std::memory_order_relaxed) != seen; });
        parked_--;
        if (stop_) return;
        seen = gen_.load(std::memory_order_relaxed);
        job = job_;
      }
      if (job) run_chunks(*job);
    }
  }
  size_t n_threads_;
  std::vector<std::thread> workers_;
  std::mutex mu_, done_mu_;
  std::condition_variable cv_, done_cv_;
  std::shared_ptr<Job> job_;
  std::atomic<uint64_t> gen_{0};
  size_t parked_ = 0;
  bool stop_ = false;
};

// One pool per thread count, created on first use and kept (the reference's engine holds one
// pool for its lifetime).
Pool& pool_for(size_t threads) {
  static std::mutex mu;
  static std::map<size_t, std::unique_ptr<Pool>> pools;
  std::lock_guard<std::mutex> g(mu);
  auto& p = pools[threads];
  if (!p) p = std::make_unique<Pool>(threads);
  return *p;
}

template <typename F>
void parallel_for(size_t n, size_t threads, F f) {
  if (n == 0) return;
  const size_t n_chunks = std::min(std::max<size_t>(threads, 1), n);
  if (threads <= 1 || n_chunks == 1) {
    f(0, n);
    return;
  }
  pool_for(threads).run(n, f);
}

constexpr size_t SPLIT_MIN_KEYS = 128;  // forward.rs:681

// forward.rs:624-633
size_t attend_splits(size_t n_rows, size_t n_kv, size_t threads, size_t span) {
  size_t tasks = n_rows * n_kv;
  if (tasks < 2 * threads && span >= 2 * SPLIT_MIN_KEYS) {
    size_t s = (2 * threads + tasks - 1) / tasks;
    s = std::min(s, span / SPLIT_MIN_KEYS);
    return std::max<size_t>(s, 1);
  }
  return 1;
}

struct Rows {
  std::vector<size_t> seq, pos, seg_of;
  std::vector<orc_seg> segs;
};

Rows rows_from_segs(const orc_seg* segs, size_t n_segs) {
  Rows r;
  for (size_t i = 0; i < n_segs; i++) {
    r.segs.push_back(segs[i]);
    for (size_t j = 0; j < segs[i].n; j++) {
      r.seq.push_back(segs[i].seq);
      r.pos.push_back(segs[i].pos0 + j);
      r.seg_of.push_back(i);
    }
  }
  return r;
}

// attend_split (forward.rs:688-807)
void attend_split(const std::vector<Reader>& readers, const Rows& rows, const float* q_all, size_t n_head,
                  size_t n_kv, size_t hd, size_t hdv, float scale, size_t window, size_t splits, size_t span,
                  float* out, size_t threads) {
  const size_t n = rows.pos.size();
  const size_t q_dim = n_head * hd;
  const size_t group = n_head / n_kv;
  const size_t attn_dim = n_head * hdv;
  const size_t stride = group * (hdv + 2);
  std::vector<float> part(n * n_kv * splits * stride, 0.0f);
  const size_t chunk = (span + splits - 1) / splits;
  parallel_for(n * n_kv * splits, threads, [&](size_t start, size_t end) {
    std::vector<float> scores(group * chunk, 0.0f);
    std::vector<float> row(std::max(hd, hdv), 0.0f);
    for (size_t idx = start; idx < end; idx++) {
      size_t sp = idx % splits;
      size_t task = idx / splits;
      size_t t = task / n_kv;
      size_t kvh = task % n_kv;
      const Reader& rd = readers[rows.seg_of[t]];
      size_t t_abs = rows.pos[t];
      size_t p_lo = window ? (t_abs + 1 > window ? t_abs + 1 - window : 0) : 0;
      size_t r0 = p_lo + sp * chunk;
      size_t r1 = std::min(r0 + chunk, t_abs + 1);
      float* o_all = part.data() + idx * stride;
      if (r0 >= r1) {
        for (size_t g = 0; g < group; g++) {
          o_all[g * (hdv + 2) + hdv] = -INFINITY;
          o_all[g * (hdv + 2) + hdv + 1] = 0.0f;
        }
        continue;
      }
      size_t m_pos = r1 - r0;
      for (size_t p = r0, i = 0; p < r1; p++, i++) {
        rd.load_k(p, kvh * hd, row.data(), hd);
        for (size_t g = 0; g < group; g++) {
          size_t h = kvh * group + g;
          const float* q = q_all + t * q_dim + h * hd;
          scores[g * chunk + i] = dot(q, row.data(), hd) * scale;
        }
      }
      for (size_t g = 0; g < group; g++) {
        float* sc = scores.data() + g * chunk;
        float m = -INFINITY;
        for (size_t i = 0; i < m_pos; i++) m = std::fmax(m, sc[i]);
        float l = 0.0f;
        for (size_t i = 0; i < m_pos; i++) {
          sc[i] = std::exp(sc[i] - m);
          l += sc[i];
        }
        float* o = o_all + g * (hdv + 2);
        for (size_t j = 0; j < hdv; j++) o[j] = 0.0f;
        o[hdv] = m;
        o[hdv + 1] = l;
      }
      for (size_t p = r0, i = 0; p < r1; p++, i++) {
        rd.load_v(p, kvh * hdv, row.data(), hdv);
        for (size_t g = 0; g < group; g++) {
          float w = scores[g * chunk + i];
          float* o = o_all + g * (hdv + 2);
          for (size_t j = 0; j < hdv; j++) o[j] += w * row[j];
        }
      }
    }
  });
  std::vector<float> merged(hdv);
  for (size_t task = 0; task < n * n_kv; task++) {
    size_t t = task / n_kv, kvh = task % n_kv;
    for (size_t g = 0; g < group; g++) {
      auto at = [&](size_t sp) { return (task * splits + sp) * stride + g * (hdv + 2); };
      float m_star = -INFINITY;
      for (size_t sp = 0; sp < splits; sp++) m_star = std::fmax(m_star, part[at(sp) + hdv]);
      std::fill(merged.begin(), merged.end(), 0.0f);
      float l_star = 0.0f;
      for (size_t sp = 0; sp < splits; sp++) {
        const float* o = part.data() + at(sp);
        if (o[hdv] == -INFINITY) continue;
        float c = std::exp(o[hdv] - m_star);
        l_star += c * o[hdv + 1];
        for (size_t j = 0; j < hdv; j++) merged[j] += c * o[j];
      }
      float inv = l_star > 0.0f ? 1.0f / l_star : 0.0f;
      float* dst = out + t * attn_dim + (kvh * group + g) * hdv;
      for (size_t j = 0; j < hdv; j++) dst[j] = merged[j] * inv;
    }
  }
}

}  // namespace

// =============================================================================================
// C ABI
// =============================================================================================

extern "C" {

uint16_t orc_f16_from_f32(float x) { return f16_from_f32(x); }
float orc_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t orc_bf16_from_f32(float x) { return bf16_from_f32(x); }
float orc_bf16_to_f32(uint16_t h) { return bf16_to_f32(h); }
void orc_f16_from_f32_n(const float* x, size_t n, uint16_t* out) {
  for (size_t i = 0; i < n; i++) out[i] = f16_from_f32(x[i]);
}
void orc_bf16_from_f32_n(const float* x, size_t n, uint16_t* out) {
  for (size_t i = 0; i < n; i++) out[i] = bf16_from_f32(x[i]);
}
size_t orc_row_bytes(int t, size_t n) { return row_bytes(t, n); }
void orc_quantize_q8_0(const float* src, size_t n, uint8_t* dst) { quantize_q8_0(src, n, dst); }
void orc_dequantize_q8_0(const uint8_t* src, size_t n, float* out) { dequantize_q8_0(src, n, out); }
void orc_store_row(int t, const float* src, size_t n, uint8_t* dst) { store_row(t, src, n, dst); }
void orc_load_row(int t, const uint8_t* src, size_t start, size_t len, float* out) {
  load_row(t, src, start, len, out);
}

orc_pool* orc_pool_new(uint64_t n, uint64_t bt, uint64_t bb) { return new orc_pool(n, bt, bb); }
void orc_pool_free(orc_pool* p) { delete p; }
uint64_t orc_pool_free_blocks(const orc_pool* p) { return p->free.size(); }
int orc_pool_alloc(orc_pool* p, uint64_t n, uint32_t* out) {
  std::vector<uint32_t> v;
  if (!p->alloc(n, v)) return ORC_KV_FULL;
  std::copy(v.begin(), v.end(), out);
  return ORC_OK;
}
void orc_pool_release(orc_pool* p, uint32_t b) { p->release(b); }
void orc_pool_set_hash(orc_pool* p, uint32_t b, const uint8_t* h32) {
  Hash h;
  std::memcpy(h.data(), h32, 32);
  p->set_hash(b, h);
}
int orc_pool_reclaim(orc_pool* p, const uint8_t* h32, uint32_t* out) {
  Hash h;
  std::memcpy(h.data(), h32, 32);
  return p->reclaim(h, out) ? 1 : 0;
}
uint32_t orc_pool_refs(const orc_pool* p, uint32_t b) { return p->meta[b].refs; }
int orc_pool_is_cached(const orc_pool* p, uint32_t b) { return p->meta[b].has_hash ? 1 : 0; }
void orc_pool_clear_hash(orc_pool* p, uint32_t b) { p->clear_hash(b); }
void orc_pool_note_miss(orc_pool* p) { p->misses++; }  // lib.rs:145-147
uint64_t orc_pool_block_tokens(const orc_pool* p) { return p->block_tokens; }
void orc_pool_stats(const orc_pool* p, uint64_t* o) {
  o[0] = p->meta.size();
  o[1] = p->free.size();
  uint64_t cf = 0;
  for (uint32_t b : p->free) cf += p->meta[b].has_hash ? 1 : 0;
  o[2] = cf;
  o[3] = p->hits;
  o[4] = p->misses;
  o[5] = p->evictions;
}

orc_cache* orc_cache_new(const orc_options* o, const orc_layer_geom* layers, uint64_t n_layers) {
  return new orc_cache(make_layout(*o, layers, n_layers));
}
void orc_cache_free(orc_cache* c) { delete c; }
void orc_cache_layout(const orc_cache* c, orc_layout_info* out) {
  out->block_bytes = c->lay.block_bytes;
  out->blocks_per_seq = c->lay.blocks_per_seq;
  out->n_seqs = c->lay.n_seqs;
  out->pool_blocks = c->lay.pool_blocks;
  out->max_ctx = c->lay.max_ctx;
  out->block_tokens = c->lay.block_tokens;
}
void orc_cache_layer(const orc_cache* c, uint64_t l, orc_layer_info* out) {
  const Layer& y = c->lay.layers[l];
  out->kv_dim = y.kv_dim;
  out->v_dim = y.v_dim;
  out->k_row = y.k_row;
  out->v_row = y.v_row;
  out->k_base = y.off;
  out->v_base = y.off + y.rows * y.k_row;
}
orc_pool* orc_cache_pool(orc_cache* c) { return &c->pool; }
uint64_t orc_cache_len(const orc_cache* c, uint64_t s) { return c->seqs[s].len; }
void orc_cache_set_len(orc_cache* c, uint64_t s, uint64_t len) { c->seqs[s].len = len; }
uint64_t orc_cache_blocks_needed(const orc_cache* c, uint64_t s, uint64_t n) { return c->blocks_needed(s, n); }
int orc_cache_reserve(orc_cache* c, uint64_t s, uint64_t n, uint64_t* needed, uint64_t* free_) {
  return c->reserve(s, n, needed, free_);
}
void orc_cache_truncate(orc_cache* c, uint64_t s, uint64_t n) { c->truncate(s, n); }
void orc_cache_clear(orc_cache* c, uint64_t s) { c->clear(s); }
uint64_t orc_cache_snapshot_bytes(const orc_cache* c, uint64_t len) { return c->snapshot_bytes(len); }
void orc_cache_write_seq(const orc_cache* c, uint64_t s, uint8_t* out) { c->write_seq(s, out); }
int orc_cache_read_seq(orc_cache* c, uint64_t s, uint64_t len, const uint8_t* bytes, uint64_t n, uint64_t* needed,
                       uint64_t* free_) {
  return c->read_seq(s, len, bytes, n, needed, free_);
}
uint64_t orc_cache_resident_blocks(const orc_cache* c) {
  uint64_t n = 0;
  for (auto& b : c->backing) n += b.empty() ? 0 : 1;
  return n;
}
uint64_t orc_cache_seq_blocks(const orc_cache* c, uint64_t s, uint32_t* out, uint64_t cap) {
  const auto& b = c->seqs[s].blocks;
  for (size_t i = 0; i < b.size() && i < cap; i++) out[i] = b[i];
  return b.size();
}
int orc_cache_adopt_blocks(orc_cache* c, uint64_t s, const uint32_t* blocks, uint64_t n) {
  if (!c->seqs[s].blocks.empty()) return ORC_INVALID;
  for (uint64_t i = 0; i < n; i++) {
    auto it = std::find(c->pool.free.begin(), c->pool.free.end(), blocks[i]);
    if (it == c->pool.free.end()) return ORC_INVALID;
  }
  for (uint64_t i = 0; i < n; i++) {
    uint32_t b = blocks[i];
    c->pool.free.erase(std::find(c->pool.free.begin(), c->pool.free.end(), b));
    Meta& m = c->pool.meta[b];
    if (m.has_hash) {
      c->pool.by_hash.erase(m.hash);
      m.has_hash = false;
      c->pool.evictions++;
    }
    m.refs = 1;
    c->back(b);
    c->seqs[s].blocks.push_back(b);
  }
  return ORC_OK;
}
// The scheduler driving this cache: sequence slot s takes the blocks Sequence::acquire referenced
// for it (kv/src/lib.rs:272-316) as its table, and starts at len positions.
int orc_cache_bind_seq(orc_cache* c, uint64_t s, const uint32_t* blocks, uint64_t n, uint64_t len) {
  if (!c->seqs[s].blocks.empty() || c->seqs[s].len != 0 || len > n * c->lay.block_tokens) return ORC_INVALID;
  for (uint64_t i = 0; i < n; i++) {
    c->back(blocks[i]);
    c->seqs[s].blocks.push_back(blocks[i]);
  }
  c->seqs[s].len = len;
  return ORC_OK;
}
void orc_cache_store_k(orc_cache* c, uint64_t s, uint64_t l, uint64_t pos, const float* k) {
  store_row(c->lay.kv_type, k, c->lay.layers[l].kv_dim, c->row_ptr(s, l, pos, false));
}
void orc_cache_store_v(orc_cache* c, uint64_t s, uint64_t l, uint64_t pos, const float* v) {
  store_row(c->lay.kv_type, v, c->lay.layers[l].v_dim, c->row_ptr(s, l, pos, true));
}
void orc_cache_store_k_raw(orc_cache* c, uint64_t s, uint64_t l, uint64_t pos, const uint8_t* row) {
  std::memcpy(c->row_ptr(s, l, pos, false), row, c->lay.layers[l].k_row);
}
void orc_cache_store_v_raw(orc_cache* c, uint64_t s, uint64_t l, uint64_t pos, const uint8_t* row) {
  std::memcpy(c->row_ptr(s, l, pos, true), row, c->lay.layers[l].v_row);
}
void orc_cache_store_rows(orc_cache* c, uint64_t s, uint64_t l, uint64_t pos0, uint64_t n, const float* k,
                          const float* v) {
  const Layer& y = c->lay.layers[l];
  for (uint64_t i = 0; i < n; i++) {
    store_row(c->lay.kv_type, k + i * y.kv_dim, y.kv_dim, c->row_ptr(s, l, pos0 + i, false));
    store_row(c->lay.kv_type, v + i * y.v_dim, y.v_dim, c->row_ptr(s, l, pos0 + i, true));
  }
}
void orc_cache_store_rows_raw(orc_cache* c, uint64_t s, uint64_t l, uint64_t pos0, uint64_t n, const uint8_t* k,
                              const uint8_t* v) {
  const Layer& y = c->lay.layers[l];
  for (uint64_t i = 0; i < n; i++) {
    std::memcpy(c->row_ptr(s, l, pos0 + i, false), k + i * y.k_row, y.k_row);
    std::memcpy(c->row_ptr(s, l, pos0 + i, true), v + i * y.v_row, y.v_row);
  }
}
void orc_cache_load_rows_raw(const orc_cache* c, uint64_t s, uint64_t l, uint64_t pos0, uint64_t n, uint8_t* k,
                             uint8_t* v) {
  const Layer& y = c->lay.layers[l];
  for (uint64_t i = 0; i < n; i++) {
    std::memcpy(k + i * y.k_row, c->row_ptr(s, l, pos0 + i, false), y.k_row);
    std::memcpy(v + i * y.v_row, c->row_ptr(s, l, pos0 + i, true), y.v_row);
  }
}
void orc_cache_load_k(const orc_cache* c, uint64_t s, uint64_t l, uint64_t pos, uint64_t start, uint64_t len,
                      float* out) {
  load_row(c->lay.kv_type, c->row_ptr(s, l, pos, false), start, len, out);
}
void orc_cache_load_v(const orc_cache* c, uint64_t s, uint64_t l, uint64_t pos, uint64_t start, uint64_t len,
                      float* out) {
  load_row(c->lay.kv_type, c->row_ptr(s, l, pos, true), start, len, out);
}

// forward.rs:207-291 (validation, all-or-nothing reservation) and Rows::push (forward.rs:63-77).
// The reference's chunk loop (forward.rs:264-291) is one pass for paged layers (max_batch =
// usize::MAX, kv.rs:522-531), so the rows are the batch's in batch order.
int orc_prepare_batch(orc_cache* c, const uint64_t* seqs, const uint64_t* n_tokens, uint64_t m,
                      orc_seg* segs_out, uint64_t* n_rows, uint64_t* needed, uint64_t* free_) {
  if (m == 0 || m > c->seqs.size()) return ORC_INVALID;
  for (uint64_t i = 0; i < m; i++) {
    if (seqs[i] >= c->seqs.size() || n_tokens[i] == 0) return ORC_INVALID;
    for (uint64_t j = 0; j < i; j++)
      if (seqs[j] == seqs[i]) return ORC_INVALID;
    if (c->seqs[seqs[i]].len + n_tokens[i] > c->lay.max_ctx) return ORC_INVALID;
  }
  uint64_t need = 0;
  for (uint64_t i = 0; i < m; i++) need += c->blocks_needed(seqs[i], c->seqs[seqs[i]].len + n_tokens[i]);
  if (need > c->pool.free.size()) {
    if (needed) *needed = need;
    if (free_) *free_ = c->pool.free.size();
    return ORC_KV_FULL;
  }
  for (uint64_t i = 0; i < m; i++) c->reserve(seqs[i], c->seqs[seqs[i]].len + n_tokens[i], nullptr, nullptr);
  uint64_t start = 0;
  for (uint64_t i = 0; i < m; i++) {
    segs_out[i].seq = seqs[i];
    segs_out[i].start = start;
    segs_out[i].n = n_tokens[i];
    segs_out[i].pos0 = c->seqs[seqs[i]].len;
    start += n_tokens[i];
  }
  if (n_rows) *n_rows = start;
  return ORC_OK;
}

void orc_commit_batch(orc_cache* c, const orc_seg* segs, uint64_t n_segs) {
  for (uint64_t i = 0; i < n_segs; i++) c->seqs[segs[i].seq].len += segs[i].n;
}

uint64_t orc_attend_splits(uint64_t n_rows, uint64_t n_kv, uint64_t threads, uint64_t span) {
  return attend_splits(n_rows, n_kv, threads, span);
}

void orc_rms_norm(const float* x, const float* w, float eps, float* y, size_t n) { rms_norm(x, w, eps, y, n); }
void orc_rope_apply(float* x, size_t n_heads, size_t hd, uint32_t pos, const orc_rope_params* p) { rope(x, n_heads, hd, pos, p); }
// attention_block's per-row tail (forward.rs:427-453): QK-norm, RoPE at each row's position; q_out
// [n][n_head][hd], k_out [n][n_kv][hd], v_out [n][n_kv][hdv] (f32, before the cache encoding).
void orc_qk_rope(const float* q_in, const float* k_in, const float* v_in, const uint32_t* pos, size_t n_rows,
                 size_t n_head, size_t n_kv, size_t hd, size_t hdv, size_t q_stride, const orc_rope_params* p,
                 float* q_out, float* k_out, float* v_out) {
  for (size_t t = 0; t < n_rows; t++) {
    float* q = q_out + t * n_head * hd;
    float* k = k_out + t * n_kv * hd;
    float* v = v_out + t * n_kv * hdv;
    for (size_t h = 0; h < n_head; h++) std::memcpy(q + h * hd, q_in + (t * n_head + h) * q_stride, hd * 4);
    std::memcpy(k, k_in + t * n_kv * hd, n_kv * hd * 4);
    std::memcpy(v, v_in + t * n_kv * hdv, n_kv * hdv * 4);
    if (p->q_norm) per_head_norm(q, n_head, hd, p->q_norm, p->eps);
    if (p->k_norm) per_head_norm(k, n_kv, hd, p->k_norm, p->eps);
    if (p->v_norm) per_head_norm(v, n_kv, hdv, nullptr, p->eps);
    if (p->apply) {
      rope(q, n_head, hd, pos[t], p);
      rope(k, n_kv, hd, pos[t], p);
    }
  }
}
float orc_dot(const float* a, const float* b, uint64_t n) { return dot(a, b, n); }
void orc_softmax(float* x, uint64_t n) { softmax(x, n); }

// attend (forward.rs:585-678)
void orc_attend(const orc_cache* c, uint64_t l, const orc_seg* segs, uint64_t n_segs, const float* q_all,
                uint64_t n_head, float scale, uint64_t window, uint64_t threads, float* out) {
  const Layer& y = c->lay.layers[l];
  const size_t n_kv = y.n_kv, hd = y.hd, hdv = y.hdv;
  Rows rows = rows_from_segs(segs, n_segs);
  const size_t n = rows.pos.size();
  if (n == 0) return;
  const size_t q_dim = n_head * hd;
  const size_t group = n_head / n_kv;
  std::vector<Reader> readers;
  for (size_t i = 0; i < n_segs; i++) readers.push_back(make_reader(c, segs[i].seq, l));
  const size_t attn_dim = n_head * hdv;
  size_t n_ctx = 0;
  for (size_t p : rows.pos) n_ctx = std::max(n_ctx, p);
  n_ctx += 1;
  const size_t span = window ? std::min(window, n_ctx) : n_ctx;
  const size_t splits = attend_splits(n, n_kv, threads, span);
  if (splits > 1) {
    attend_split(readers, rows, q_all, n_head, n_kv, hd, hdv, scale, window, splits, span, out, threads);
    return;
  }
  parallel_for(n * n_kv, threads, [&](size_t start, size_t end) {
    std::vector<float> scores(group * span, 0.0f);
    std::vector<float> row(std::max(hd, hdv), 0.0f);
    std::vector<float> acc(group * hdv, 0.0f);
    for (size_t idx = start; idx < end; idx++) {
      size_t t = idx / n_kv;
      size_t kvh = idx % n_kv;
      const Reader& rd = readers[rows.seg_of[t]];
      size_t t_abs = rows.pos[t];
      size_t p_lo = window ? (t_abs + 1 > window ? t_abs + 1 - window : 0) : 0;
      size_t n_pos = t_abs + 1 - p_lo;
      for (size_t p = p_lo, i = 0; p <= t_abs; p++, i++) {
        rd.load_k(p, kvh * hd, row.data(), hd);
        for (size_t g = 0; g < group; g++) {
          size_t h = kvh * group + g;
          const float* q = q_all + t * q_dim + h * hd;
          scores[g * span + i] = dot(q, row.data(), hd) * scale;
        }
      }
      for (size_t g = 0; g < group; g++) softmax(scores.data() + g * span, n_pos);
      std::fill(acc.begin(), acc.end(), 0.0f);
      for (size_t p = p_lo, i = 0; p <= t_abs; p++, i++) {
        rd.load_v(p, kvh * hdv, row.data(), hdv);
        for (size_t g = 0; g < group; g++) {
          float w = scores[g * span + i];
          float* a = acc.data() + g * hdv;
          for (size_t j = 0; j < hdv; j++) a[j] += w * row[j];
        }
      }
      std::memcpy(out + t * attn_dim + kvh * group * hdv, acc.data(), group * hdv * sizeof(float));
    }
  });
}

// Plain float64 attention, written independently of the restatement above (no 16-lane dot, no
// online merge): the pinning reference for orc_attend.
void orc_attend_naive_f64(const orc_cache* c, uint64_t l, const orc_seg* segs, uint64_t n_segs, const float* q,
                          uint64_t n_head, double scale, uint64_t window, double* out) {
  const Layer& y = c->lay.layers[l];
  const size_t group = n_head / y.n_kv;
  std::vector<float> k(y.hd), v(y.hdv);
  size_t t = 0;
  for (size_t si = 0; si < n_segs; si++) {
    for (size_t j = 0; j < segs[si].n; j++, t++) {
      size_t pos = segs[si].pos0 + j;
      size_t lo = (window && pos + 1 > window) ? pos + 1 - window : 0;
      for (size_t h = 0; h < n_head; h++) {
        size_t kvh = h / group;
        std::vector<double> s;
        for (size_t p = lo; p <= pos; p++) {
          orc_cache_load_k(c, segs[si].seq, l, p, kvh * y.hd, y.hd, k.data());
          double acc = 0;
          for (size_t d = 0; d < y.hd; d++) acc += (double)q[(t * n_head + h) * y.hd + d] * (double)k[d];
          s.push_back(acc * scale);
        }
        double mx = -INFINITY;
        for (double x : s) mx = std::max(mx, x);
        double z = 0;
        for (double& x : s) {
          x = std::exp(x - mx);
          z += x;
        }
        double* o = out + (t * n_head + h) * y.hdv;
        for (size_t d = 0; d < y.hdv; d++) o[d] = 0;
        for (size_t p = lo, i = 0; p <= pos; p++, i++) {
          orc_cache_load_v(c, segs[si].seq, l, p, kvh * y.hdv, y.hdv, v.data());
          for (size_t d = 0; d < y.hdv; d++) o[d] += s[i] / z * (double)v[d];
        }
      }
    }
  }
}

}  // extern "C"
