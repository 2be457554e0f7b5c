// decode_tile.h — the matrix-core decode work item (one wave per (row, KV head, key range)),
// shared by the decode kernel (decode.hip) and the mixed-batch kernel (prefill.hip), which runs
// a call's decode items in the same launch as its prefill units.
//
// f16 / bf16 / q8_0 pages: per 16-token tile,
//   S^T[16 keys x 16 heads] = K[16 x hd] . Q^T[hd x 16]     (v_mfma_f32_16x16x32_{f16,bf16})
//   O^T[hdv x 16 heads]    += V^T[hdv x 16] . P^T[16 x 16]    (v_mfma_f32_16x16x16_f16)
// (forward.rs:585-807 for what is computed; the layout and algorithm notes are in decode.hip).
#pragma once

#include "device.h"

#include <type_traits>

namespace lmh {
namespace dtile {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ inline float xmax_groups(float x) {  // max over lanes l, l^16, l^32, l^48
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
__device__ inline float xsum_groups(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

__device__ inline uint16_t bf16_rne(float x) {
  uint32_t u = __float_as_uint(x);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// int8 x4 (packed in a uint32) -> f16 x4, exact.
// Four int8 codes -> four f16, exactly: each byte biased to unsigned (q ^ 0x80 = q + 128) becomes
// the low mantissa byte of f16 1024 (0x64xx = 1024 + u, exact for u < 256), then 1152 is
// subtracted two lanes at a time (packed f16).
__device__ inline h4 i8x4_to_h4(uint32_t w) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const uint32_t u = w ^ 0x80808080u;
  const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // [b0, 0x64, b1, 0x64]
  const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // [b2, 0x64, b3, 0x64]
  const h2 off = {(_Float16)1152.0f, (_Float16)1152.0f};
  const h2 a = __builtin_bit_cast(h2, lo) - off, b = __builtin_bit_cast(h2, hi) - off;
  return h4{a[0], a[1], b[0], b[1]};
}

// bf16 x4 (two uint32) -> f16 x4 (exact for normal f16 range).
__device__ inline h4 bf4_to_h4(uint32_t a, uint32_t b) {
  h4 r;
  r[0] = (_Float16)__uint_as_float(a << 16);
  r[1] = (_Float16)__uint_as_float(a & 0xffff0000u);
  r[2] = (_Float16)__uint_as_float(b << 16);
  r[3] = (_Float16)__uint_as_float(b & 0xffff0000u);
  return r;
}

__device__ inline float h_to_f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }

// Weights (a, b) as packed f16 hi parts and packed f16 lo parts (a - hi, b - hi): each lo part one
// v_fma_mix_f32 that reads the f16 hi part directly (hi * -1 + a), then one conversion per pair.
// The -1 is hidden from constant folding (an empty asm statement, which emits nothing) so the
// compiler keeps the fma form instead of converting hi back to f32 and subtracting; every
// instruction is the compiler's own, so its hazard tracking sees them.
__device__ inline void split_pair(float a, float b, uint32_t& hi, uint32_t& lo) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  float m1 = -1.0f;
  asm("" : "+v"(m1));
  const h2 h = __builtin_convertvector((f2){a, b}, h2);
  const f2 r = {__builtin_fmaf((float)h[0], m1, a), __builtin_fmaf((float)h[1], m1, b)};
  hi = __builtin_bit_cast(uint32_t, h);
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, h2));
}

// (p0 * d0, p1 * d1) as packed f16 hi parts and packed f16 lo parts (p*d - hi from one fma, rounded
// once), for f16 scales d: the compiler forms both from v_fma_mix{lo,hi}_f16, which read the f32
// weight and the f16 scale as they are.
__device__ inline void scaled_split(float p0, _Float16 d0, float p1, _Float16 d1, uint32_t& hi, uint32_t& lo) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 h = {(_Float16)__builtin_fmaf(p0, (float)d0, 0.0f), (_Float16)__builtin_fmaf(p1, (float)d1, 0.0f)};
  const h2 l = {(_Float16)__builtin_fmaf(p0, (float)d0, -(float)h[0]),
                (_Float16)__builtin_fmaf(p1, (float)d1, -(float)h[1])};
  hi = __builtin_bit_cast(uint32_t, h);
  lo = __builtin_bit_cast(uint32_t, l);
}

template <int KVT, int HD, int HDV>
struct TileRegs {
  // f16/bf16: K one uint4 per 32 dims, V one uint4 per 32 dims.
  // q8_0: K codes one uint4 per 64 dims, V codes one uint4 per 64 dims, plus the lane's scales.
  static constexpr int NK = (KVT == KV_Q8) ? HD / 64 : HD / 32;
  static constexpr int NV = (KVT == KV_Q8) ? HDV / 64 : HDV / 32;
  static constexpr int NKS = (KVT == KV_Q8) ? (4 * (HD / 32) * 2 + 15) / 16 : 0;   // scale uint4s
  static constexpr int NVS = (KVT == KV_Q8) ? (4 * (HDV / 32) * 2 + 15) / 16 : 0;
  uint4 k[NK];
  uint4 v[NV];
  uint4 ks[NKS > 0 ? NKS : 1];
  uint4 vs[NVS > 0 ? NVS : 1];
};

// 16 bytes of a page, non-temporal: an engine's step reads each layer's pages once, and a layer's
// pages were last read a whole step (every other layer's pages) earlier, so they come from HBM;
// streaming them past the caches reads a cold 1.5 GB at 7.1 TB/s against 6.4 TB/s for ordinary
// loads. (Re-reading one layer's 297 MB step after step, which fits the last-level cache, ordinary
// loads were 3% faster.)
__device__ inline uint4 load_stream(const uint8_t* p) {
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  const u4 v = __builtin_nontemporal_load((const u4*)p);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

template <int KVT, int HD, int HDV>
__device__ inline void load_tile(TileRegs<KVT, HD, HDV>& t, const uint8_t* kb, const uint8_t* vb,
                                 const uint8_t* ksb, const uint8_t* vsb, uint32_t lane) {
  using T = TileRegs<KVT, HD, HDV>;
#pragma unroll
  for (int c = 0; c < T::NK; c++) t.k[c] = load_stream(kb + c * 1024 + lane * 16);
#pragma unroll
  for (int c = 0; c < T::NV; c++) t.v[c] = load_stream(vb + c * 1024 + lane * 16);
  if constexpr (KVT == KV_Q8) {
    // scales [key m][chunk]: lane group g = lane/16 needs keys 4g..4g+3, all chunks (contiguous)
    const uint32_t g = lane >> 4;
#pragma unroll
    for (int c = 0; c < T::NKS; c++) t.ks[c] = *(const uint4*)(ksb + g * (4 * (HD / 32) * 2) + c * 16);
#pragma unroll
    for (int c = 0; c < T::NVS; c++) t.vs[c] = *(const uint4*)(vsb + g * (4 * (HDV / 32) * 2) + c * 16);
  }
}

// f16 scale of key 4g+r, chunk c, from the lane's scale registers.
template <int NCH>
__device__ inline _Float16 scale_h(const uint4* s, int r, int c) {
  const int idx = r * NCH + c;
  const uint32_t w = ((const uint32_t*)s)[idx >> 1];
  return __builtin_bit_cast(_Float16, (uint16_t)((idx & 1) ? (w >> 16) : (w & 0xffff)));
}

// Scale (as f32) for key 4g+r, chunk c, from the lane's scale registers.
template <int NCH>
__device__ inline float scale_at(const uint4* s, int r, int c) {
  const int idx = r * NCH + c;  // f16 index
  const uint32_t w = ((const uint32_t*)s)[idx >> 1];
  return h_to_f((uint16_t)((idx & 1) ? (w >> 16) : (w & 0xffff)));
}

// The workgroups of a decode, prefill or mixed launch copy the call's merge list from the staged
// (host-mapped) work list into device memory beside their own work, a slice each (a word per
// thread for up to block x grid words): the merge kernel that follows then starts from device
// memory instead of a round trip over the bus, and no workgroup spends more than one bus round
// trip on it (a list of thousands of prompt merges copied by one workgroup held that workgroup
// back by tens of microseconds).
__device__ inline void copy_merges(const MergeCopy& mc, uint32_t block, uint32_t n_blocks) {
  const uint32_t stride = n_blocks * blockDim.x;
  for (uint32_t i = block * blockDim.x + threadIdx.x; i < mc.n_words; i += stride) mc.dst[i] = mc.src[i];
}

// Floats of a wave's partial in LDS when a row's split items merge inside their workgroup: the
// O^T blocks lane-major (a float4 per lane and 16-dim block, as the accumulators hold them), then
// m and l of the 16 heads.
template <int HDV>
constexpr int local_partial_floats() {
  return (HDV / 16) * 256 + 32;
}

// One decode work item, items[wi], computed by the calling wave: the partial (o, m, l) to
// `part` for a split item, else the normalised output row to `out`. LOCAL: an item whose slot is
// LOCAL_SLOT | ... leaves its partial in the wave's share of `lds` (local_partial_floats floats
// per wave) for the workgroup's merge instead.
template <int KVT, int HD, int HDV, bool LOCAL = false>
__device__ __forceinline__ void decode_item(const PageGeom& g, const RowGeom& r, const DecodeItem* items, uint32_t wi,
                                            const float* q, float* out, float* part, float* lds = nullptr) {
  constexpr int NC = HD / 32;    // Q.K chunks of 32 dims
  constexpr int NJ = HDV / 16;   // O^T blocks of 16 dims
  constexpr bool Q8 = KVT == KV_Q8;
  using MT = typename std::conditional<KVT == KV_BF16, b8, h8>::type;
  const uint32_t lane = threadIdx.x & 63u;
  // the item is the same for the whole wave: its fields in scalar registers keep the tile loop's
  // address arithmetic and range tests on the scalar unit
  DecodeItem it = items[wi];
  it.row = __builtin_amdgcn_readfirstlane(it.row);
  it.kvh = __builtin_amdgcn_readfirstlane(it.kvh);
  it.h0 = __builtin_amdgcn_readfirstlane(it.h0);
  it.p0 = __builtin_amdgcn_readfirstlane(it.p0);
  it.p1 = __builtin_amdgcn_readfirstlane(it.p1);
  it.slot = __builtin_amdgcn_readfirstlane(it.slot);
  it.seq = __builtin_amdgcn_readfirstlane(it.seq);
  it.blk0 = __builtin_amdgcn_readfirstlane(it.blk0);
  const int seq = (int)it.seq;
  const int32_t* tab = g.table + (size_t)seq * g.bps;
  const uint32_t hq = lane & 15u, grp = lane >> 4;
  const bool hv = hq < r.ng && it.h0 + hq < r.group;
  const uint32_t head = it.kvh * r.group + it.h0 + hq;

  // Q as the B operand of S^T = K Q^T: chunk c, lane (grp, hq) holds dims 32c + 8grp .. +8.
  MT qh[NC], ql[NC];
  {
    const float* qp = q + ((size_t)it.row * r.n_head + (hv ? head : 0)) * HD;
#pragma unroll
    for (int c = 0; c < NC; c++) {
      float4 a = hv ? *(const float4*)(qp + 32 * c + 8 * grp) : make_float4(0, 0, 0, 0);
      float4 b = hv ? *(const float4*)(qp + 32 * c + 8 * grp + 4) : make_float4(0, 0, 0, 0);
      const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 8; i++) {
        if constexpr (KVT == KV_BF16) {
          const uint16_t hb = bf16_rne(x[i]);
          const float hf = __uint_as_float((uint32_t)hb << 16);
          qh[c][i] = __builtin_bit_cast(__bf16, hb);
          ql[c][i] = __builtin_bit_cast(__bf16, bf16_rne(x[i] - hf));
        } else {
          const _Float16 hh = (_Float16)x[i];
          qh[c][i] = hh;
          ql[c][i] = (_Float16)(x[i] - (float)hh);
        }
      }
    }
  }

  // Weights are p = 2^(s - m + pup): the reference max shifted by pup (the partial's m is written
  // as m - pup). f16 / bf16 pages: pup = 7, so every weight is <= 2^(8 + pup) and the f16 lo
  // parts below stay normal for all weights above 2^(-pup - 2) of the largest. q8_0 pages: the
  // f16 operand is weight x V scale, whose range is the scales' (f16 scales span 2^-24 .. 2^16),
  // so pup follows them: pup = 7 - e with 2^e above the largest V scale seen, which keeps every
  // product <= 2^15 (finite) and the products of the heaviest weights near 2^7 (22 bits through
  // hi + lo, whatever the scales' magnitude). The first tile of the item sets it; a later tile
  // with scales more than twice as large can overflow a product, which leaves O non-finite: the
  // item then runs again with every tile's scales checked, lowering pup (and rescaling O and lsum
  // exactly, by a power of two) before a tile whose scales need it.
  float m, lsum, pup;
  f4 O[NJ];
  bool checked = false;   // q8_0: every tile's V scales checked (the pass after an overflow)

  // The item's tiles t0..t1 (at most MFMA_ITEM_TILES = 128, the host caps chunks): lane i holds
  // the block ids of tiles t0 + i and t0 + 64 + i, so the loop reads ids with readlane instead of
  // a dependent memory load.
  const uint32_t t0 = it.p0 >> 4, t1 = (it.p1 - 1) >> 4;
  const uint32_t bt_mask = (1u << g.bt_shift) - 1u;
  int my_blk = 0, my_blk_hi = 0;
  if (t0 + lane <= t1) my_blk = tab[((t0 + lane) << 4) >> g.bt_shift];
  if (t0 + 64 + lane <= t1) my_blk_hi = tab[((t0 + 64 + lane) << 4) >> g.bt_shift];
  auto ptrs = [&](uint32_t t, const uint8_t*& kb, const uint8_t*& vb, const uint8_t*& ksb, const uint8_t*& vsb,
                  bool first = false) {
    const uint32_t pos = t << 4;
    const uint32_t d = t - t0;   // wave-uniform
    const int blk = first ? (int)it.blk0
                          : d < 64 ? __builtin_amdgcn_readlane(my_blk, (int)d) : __builtin_amdgcn_readlane(my_blk_hi, (int)(d - 64));
    const uint32_t sub = (pos & bt_mask) >> 4;
    const uint8_t* base = g.pool + (size_t)blk * g.block_bytes;
    const uint8_t* kh = base + g.k_off + it.kvh * g.k_head;
    const uint8_t* vh = base + g.v_off + it.kvh * g.v_head;
    kb = kh + sub * g.k_tile;
    vb = vh + sub * g.v_tile;
    ksb = kh + g.k_scale + sub * g.k_tile_s;
    vsb = vh + g.v_scale + sub * g.v_tile_s;
  };
  auto fetch = [&](TileRegs<KVT, HD, HDV>& buf, uint32_t t, bool first = false) {
    const uint8_t *kb, *vb, *ksb, *vsb;
    ptrs(t, kb, vb, ksb, vsb, first);
    load_tile(buf, kb, vb, ksb, vsb, lane);
  };

  auto step = [&](const TileRegs<KVT, HD, HDV>& cur, uint32_t t) {
    // ---- scores S^T for 16 keys x 16 heads
    f4 s = f4{0.f, 0.f, 0.f, 0.f};
    if constexpr (KVT == KV_Q8) {
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const uint32_t* w = (const uint32_t*)&cur.k[c >> 1];
        const int o = (c & 1) * 2;
        const h4 lo4 = i8x4_to_h4(w[o]), hi4 = i8x4_to_h4(w[o + 1]);
        const h8 kc = h8{lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
        f4 sc = f4{0.f, 0.f, 0.f, 0.f};
        sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kc, qh[c], sc, 0, 0, 0);
        sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kc, ql[c], sc, 0, 0, 0);
#pragma unroll
        for (int rr = 0; rr < 4; rr++) s[rr] += sc[rr] * scale_at<NC>(cur.ks, rr, c);
      }
    } else {
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const MT kc = __builtin_bit_cast(MT, cur.k[c]);
        if constexpr (KVT == KV_BF16) {
          s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kc, qh[c], s, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kc, ql[c], s, 0, 0, 0);
        } else {
          s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kc, qh[c], s, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_16x16x32_f16(kc, ql[c], s, 0, 0, 0);
        }
      }
    }
    // ---- online softmax (log2 domain), keys outside [p0, p1) masked
    const uint32_t kbase = (t << 4) + 4u * grp;
    float sc[4];
    if ((t << 4) < it.p0 || (t << 4) + 16u > it.p1) {   // a tile at an end of the range (uniform)
#pragma unroll
      for (int rr = 0; rr < 4; rr++) {
        const uint32_t key = kbase + rr;
        sc[rr] = (key >= it.p0 && key < it.p1) ? s[rr] * r.scale_log2 : -INFINITY;
      }
    } else {
#pragma unroll
      for (int rr = 0; rr < 4; rr++) sc[rr] = s[rr] * r.scale_log2;
    }
    // Lazy reference max: m (per head) moves only when a score exceeds it by more than 8, so
    // p = 2^(s - m) <= 2^8 and O is rescaled on few tiles; each lane checks its own 4 scores and
    // only a triggered tile reduces the head's max across the lane groups.
    const float lm = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    if (__ballot(lm > m + 8.0f)) {
      const float tm = xmax_groups(lm);
      const float mn = tm > m + 8.0f ? tm : m;
      // no key of this head seen yet (m = -inf): O and lsum are still zero
      const float alpha = mn == m ? 1.f : (m == -INFINITY ? 0.f : exp2_fast(m - mn));
      lsum *= alpha;
#pragma unroll
      for (int j = 0; j < NJ; j++) O[j] *= alpha;
      m = mn;
    }
    if constexpr (Q8) {
      if (checked || t == t0) {   // uniform: the item's first tile, or every tile after an overflow
        // the tile's largest |V scale| (a lane group's lanes hold the same 4 keys' scales)
        constexpr int NCH = HDV / 32;
        uint32_t mx = 0;
#pragma unroll
        for (int i = 0; i < 4 * NCH; i++) {
          const uint32_t w = ((const uint32_t*)cur.vs)[i >> 1];
          mx = max(mx, ((i & 1) ? (w >> 16) : w) & 0x7fffu);
        }
        const float dm = xmax_groups(h_to_f((uint16_t)mx));
        const float pc = (float)(7 - __builtin_amdgcn_readfirstlane(__builtin_amdgcn_frexp_expf(dm)));
        if (pc < pup) {   // O and lsum are zero on the first tile; otherwise an exact rescale
          const float alpha = exp2_fast(pc - pup);
          lsum *= alpha;
#pragma unroll
          for (int j = 0; j < NJ; j++) O[j] *= alpha;
          pup = pc;
        }
      }
    }
    const float mref = (m == -INFINITY ? 0.f : m) - pup;  // every score is -inf while m is
    float p[4];
#pragma unroll
    for (int rr = 0; rr < 4; rr++) p[rr] = exp2_fast(sc[rr] - mref);
    lsum += (p[0] + p[1]) + (p[2] + p[3]);
    // ---- O^T += V^T P^T, P carried past f16 as hi + lo halves (two products on the same V
    // operand): the weights keep ~22 bits, as the f32 weights of the CPU path (forward.rs:645-666)
    if constexpr (KVT == KV_Q8) {
      // P times the V scale of each (key, 32-dim block), in f32, then split: the lane's scales
      // sit as [key i][block b] halves.
      constexpr int NCH = HDV / 32;
#pragma unroll
      for (int b = 0; b < HDV / 32; b++) {
        uint32_t hw[2], lw[2];
#pragma unroll
        for (int i = 0; i < 2; i++)
          scaled_split(p[2 * i], scale_h<NCH>(cur.vs, 2 * i, b), p[2 * i + 1], scale_h<NCH>(cur.vs, 2 * i + 1, b),
                       hw[i], lw[i]);
        const h4 ph = __builtin_bit_cast(h4, make_uint2(hw[0], hw[1]));
        const h4 pl = __builtin_bit_cast(h4, make_uint2(lw[0], lw[1]));
#pragma unroll
        for (int jj = 0; jj < 2; jj++) {
          const int j = 2 * b + jj;
          const uint32_t w = ((const uint32_t*)&cur.v[j >> 2])[j & 3];
          const h4 va = i8x4_to_h4(w);
          O[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, ph, O[j], 0, 0, 0);
          O[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pl, O[j], 0, 0, 0);
        }
      }
    } else {
      uint32_t hw[2], lw[2];
#pragma unroll
      for (int i = 0; i < 2; i++) split_pair(p[2 * i], p[2 * i + 1], hw[i], lw[i]);
      const h4 ph = __builtin_bit_cast(h4, make_uint2(hw[0], hw[1]));
      const h4 pl = __builtin_bit_cast(h4, make_uint2(lw[0], lw[1]));
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        const uint32_t* w = (const uint32_t*)&cur.v[j >> 1];
        const int o = (j & 1) * 2;
        h4 va;
        if constexpr (KVT == KV_BF16) {
          va = bf4_to_h4(w[o], w[o + 1]);
        } else {
          va = __builtin_bit_cast(h4, make_uint2(w[o], w[o + 1]));
        }
        O[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, ph, O[j], 0, 0, 0);
        O[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pl, O[j], 0, 0, 0);
      }
    }
  };

  // Two-deep ping-pong: tile t+1 is in flight while tile t is computed. The fetches past the last
  // tile re-read the last tile (in bounds, and unconditional, so the buffers need no copies).
  TileRegs<KVT, HD, HDV> b0, b1;
  for (;;) {
    m = -INFINITY;
    lsum = 0.0f;
    pup = Q8 ? INFINITY : 7.0f;   // q8_0: set by the first tile's scales
#pragma unroll
    for (int j = 0; j < NJ; j++) O[j] = f4{0.f, 0.f, 0.f, 0.f};
    fetch(b0, t0, true);   // block id from the item: in flight beside the Q and block-table reads
    for (uint32_t t = t0; t <= t1; t += 2) {
      fetch(b1, min(t + 1, t1));
      step(b0, t);
      if (t + 1 > t1) break;
      fetch(b0, min(t + 2, t1));
      step(b1, t + 1);
    }
    if constexpr (!Q8) break;
    if (checked) break;
    // a product of weight and V scale that overflowed f16 leaves O non-finite (any sum with an
    // inf or NaN term is); the second pass checks every tile's scales
    float z = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; j++) z += (O[j][0] + O[j][1]) + (O[j][2] + O[j][3]);
    if (!__ballot(hv && !__builtin_isfinite(z))) break;
    checked = true;
  }
  lsum = xsum_groups(lsum);

  if constexpr (LOCAL) {
    if (it.slot != NO_SLOT && (it.slot & LOCAL_SLOT) != 0) {
      float* lw = lds + (threadIdx.x >> 6) * local_partial_floats<HDV>();
#pragma unroll
      for (int j = 0; j < NJ; j++) *(f4*)(lw + (j * 64 + lane) * 4) = O[j];
      if (grp == 0) {
        lw[NJ * 256 + hq] = m - pup;   // the reference the weights were taken against
        lw[NJ * 256 + 16 + hq] = lsum;
      }
      return;
    }
  }
  if (it.slot == NO_SLOT) {
    if (!hv) return;
    const float inv = 1.0f / lsum;
    float* op = out + ((size_t)it.row * r.n_head + head) * HDV;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const f4 o = O[j] * inv;
      *(float4*)(op + 16 * j + 4 * grp) = make_float4(o[0], o[1], o[2], o[3]);
    }
    return;
  }
  if (hv) {
    float* pp = part + ((size_t)it.slot * r.ng + hq) * (HDV + 4);
#pragma unroll
    for (int j = 0; j < NJ; j++) *(float4*)(pp + 16 * j + 4 * grp) = make_float4(O[j][0], O[j][1], O[j][2], O[j][3]);
    if (grp == 0) {
      pp[HDV] = m - pup;  // the reference the weights were taken against
      pp[HDV + 1] = lsum;
    }
  }
}

// The workgroup-local merge (forward.rs:772-806's log-sum-exp merge) after decode_item<.., true>
// and a barrier: a row's split items are consecutive waves of one W-wave workgroup (their slots
// LOCAL_SLOT | index << 8 | count), each of which left its partial in its share of `lds`; wave s of
// a group of n folds the group's partials for the O blocks j = s, s + n, .. and writes them.
template <int HDV, int W>
__device__ __forceinline__ void local_merge(const RowGeom& r, const DecodeItem* items, uint32_t wi, const float* lds,
                                            float* out) {
  constexpr int NJ = HDV / 16, LF = local_partial_floats<HDV>();
  const uint32_t w = threadIdx.x >> 6, lane = threadIdx.x & 63u;
  const uint32_t slot = __builtin_amdgcn_readfirstlane(items[wi].slot);
  if (slot == NO_SLOT || (slot & LOCAL_SLOT) == 0) return;
  const uint32_t row = __builtin_amdgcn_readfirstlane(items[wi].row);
  const uint32_t kvh = __builtin_amdgcn_readfirstlane(items[wi].kvh);
  const uint32_t h0 = __builtin_amdgcn_readfirstlane(items[wi].h0);
  const uint32_t s = (slot >> 8) & 0x7fu, n = slot & 0xffu;
  if (s >= n || s > w || w - s + n > (uint32_t)W) return;   // a group inside the workgroup (the planner's)
  const float* grp0 = lds + (w - s) * LF;   // the group's first wave
  const uint32_t hq = lane & 15u, grp = lane >> 4;
  float M = -INFINITY;
  for (uint32_t k = 0; k < n; k++) M = fmaxf(M, grp0[k * LF + NJ * 256 + hq]);
  float c[W], L = 0.f;
#pragma unroll
  for (int k = 0; k < W; k++) {
    c[k] = 0.f;
    if ((uint32_t)k < n) {
      const float ms = grp0[k * LF + NJ * 256 + hq];
      c[k] = ms == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ms - M);
      L = fmaf(c[k], grp0[k * LF + NJ * 256 + 16 + hq], L);
    }
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  if (hq >= r.ng || h0 + hq >= r.group) return;
  float* op = out + ((size_t)row * r.n_head + kvh * r.group + h0 + hq) * HDV + 4 * grp;
  for (uint32_t j = s; j < (uint32_t)NJ; j += n) {
    f4 acc = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < W; k++)
      if ((uint32_t)k < n) acc += c[k] * *(const f4*)(grp0 + k * LF + (j * 64 + lane) * 4);
    acc *= inv;
    *(float4*)(op + 16 * j) = make_float4(acc[0], acc[1], acc[2], acc[3]);
  }
}

}  // namespace dtile
}  // namespace lmh
