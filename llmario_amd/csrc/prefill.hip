// prefill.hip — causal / chunked-prefill attention on gfx950 matrix cores.
//
// Computes what `attend` computes for the rows of a multi-token segment
// (crates/engine/model/src/forward.rs:585-678): row t at position pos attends to keys
// lo..=pos of its own sequence (lo = pos+1-window with a window, else 0), softmax(scale q.k) v
// per query head, fp32 accumulation. The Metal sibling is attn_prefill_t
// (crates/engine/metal/src/shaders/attn_prefill.metal:17-195); this kernel is designed for CDNA4.
//
// Work unit: one sequence, one KV head, a run of up to 256/G tokens. Its "columns" are the
// (token, query-head) pairs of the run flattened token-major (c = token*G + head), so all G query
// heads of the KV group share every K/V tile. One workgroup of 8 waves (two per SIMD, one
// workgroup per CU) runs a list of units the host balanced across the workgroups; wave w owns
// columns 32w .. 32w+31 as two 16-column MFMA blocks. Per 64-key tile, in two 32-key halves:
//   S^T[32 keys x 32 cols] = K . Q^T     v_mfma_f32_16x16x32_{f16,bf16}, Q resident in VGPRs
//   online softmax per column in the S^T layout (keys along the 4 lane groups and 4 registers)
//   O^T[hd x 32 cols]     += V^T . P^T  v_mfma_f32_16x16x32_f16, P as f16 hi + lo (two products
//                                        on the same V operand; without PLO, P rounded to f16)
// K/V tiles go from HBM straight into LDS (global_load_lds, four stages, two tiles in flight)
// in the page layout, which already holds each 16-token tile in MFMA operand order. bf16 V is
// widened to f16 in LDS once per tile by the thread that loaded it (exact for |x| in
// [2^-14, 65504]); bf16 K too when Q is not exact in bf16 (Q then runs as f16 hi + lo parts), while
// a Q exact in bf16 multiplies bf16 K as it is. A Q with bits below the page type runs, in the
// launch for exact Q, as two passes of 16 columns per wave; the QS launch (chosen per call from
// the previous launch's Q) runs every unit as one pass whose Q.K products are the hi part then the
// lo part into one accumulator. Q stays unscaled; each column's reference max
// enters (negated) as the initial accumulator of Q.K, so a product is s - m and its weight one fma
// and one exp2 away. The reference max moves lazily (a lane's weight sum past a bound sends the
// wave to a rare path that reduces the column max), so the O accumulators are almost never
// rescaled.
//
// q8_0 pages (the Metal sibling's attn_prefill_hd{64,128}_q8_0, attn_prefill.metal:200-203) keep
// the decode kernel's exact scheme rather than dequantising to 16 bits (d*q rounded to f16 misses
// the per-row bound on rows whose output cancels): each wave's DMA brings a page tile's int8 codes
// and its f16 scales into LDS, the thread that loaded the codes rewrites them in place as
// int8-valued f16 (K) or bf16 (V), both exact, and the products apply the scales:
//   S^T = sum over 32-dim chunks c of d_K[key][c] * (K_c . Q_c^T)   (one MFMA per chunk and column
//         block: a Q exact in f16 runs one pass of 32 columns, any other Q the two-pass form with
//         its hi + lo products summed before the scale)
//   O^T += V^T . (P * d_V[.][b])^T per 32-dim V block b, the scaled weights as bf16 hi + lo
//         (v_mfma_f32_16x16x32_bf16; bf16 has f32's range, so no product of a weight and a scale
//         leaves it)
#include "decode_tile.h"

namespace lmh {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int PW = 8;          // waves per workgroup
constexpr int NT = 64 * PW;    // threads per workgroup
static_assert(PW == MIXED_LOCAL_WAVES, "a mixed launch's decode workgroups hold the planner's local groups");
constexpr int COLS = 32;       // columns per wave (two 16-column MFMA blocks)
constexpr int NCB = COLS / 16;
constexpr int BK = 64;         // keys per tile (4 page tiles of 16)
constexpr int NSTAGE = 4;      // K/V tiles in LDS (see the pipeline comment in the kernel)

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// max / sum of a value over the four 16-lane groups of a wave (lanes l, l^16, l^32, l^48), with
// the gfx950 lane-swap instructions instead of LDS permutes
__device__ inline float max_over_groups(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const float y = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ inline float sum_over_groups(float x) {
  const uint32_t u = __float_as_uint(x);
  const auto a = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  const float y = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}


// 16 bytes per lane from global memory straight into LDS (global_load_lds_dwordx4): lane L reads
// sbase + voff(L) and writes LDS address lds_dst + 16*L, where sbase and lds_dst are wave-uniform
// (an SGPR pair and M0). The LDS address is an integer (a generic pointer cast back to the LDS
// address space needs a null test the backend can select illegally). Issued from inline assembly
// so the compiler does not track it: the kernel waits for these loads itself (s_waitcnt vmcnt)
// before the barrier that publishes a stage, and nothing else in the tile loop touches vector
// memory. The compiler cannot see inside the statement, so it carries its own wait states: the
// base's SGPRs often come from v_readfirstlane right before it, and a vector-memory instruction
// may read an SGPR that a VALU instruction wrote only 5 wait states later (s_nop 4); an LDS DMA
// may read M0 one wait state after an SALU write (s_nop 0). The compiler puts the same wait
// states before its own global_load_lds.
__device__ inline void lds_dma16(const uint8_t* sbase, uint32_t voff, uint32_t lds_dst) {
  const uint32_t l = __builtin_amdgcn_readfirstlane(lds_dst);
  asm volatile("s_nop 4\n\ts_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(l), "v"(voff),
               "s"(sbase)
               : "memory", "m0");
}

// bf16 pair (one uint32) -> f16 pair (one uint32), exact in the normal f16 range.
__device__ inline uint32_t bf2_to_h2(uint32_t w) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const f2 x = {__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u)};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, h2));
}

// Weights (a, b) as packed bf16 hi parts and packed bf16 lo parts (a - hi, b - hi), both rounded to
// nearest even: 16 significant bits per weight (|w - hi - lo| <= 2^-18 |w|). Each difference is one
// v_dot2c_f32_bf16 that reads the packed hi parts directly: (-1, 0) . (hi_a, hi_b) + a, exact (the
// product is exact and a - hi is representable). The two constant pairs stay in VGPRs (an empty
// asm statement hides their values): as an inline constant the compiler encodes (-1, 0) as -1.0,
// which this instruction reads as the 32-bit pattern 0xbf800000, i.e. the pair (0, -1) (checked on
// the GPU: every lane's first difference came out as a - hi_b).
__device__ inline void split_pair_bf16(float a, float b, uint32_t& hi, uint32_t& lo) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
  const f2 v = {a, b};
  const bf2 h = __builtin_convertvector(v, bf2);
  uint32_t c0 = 0x0000bf80u, c1 = 0xbf800000u;   // the bf16 pairs (-1, 0) and (0, -1)
  asm("" : "+v"(c0), "+v"(c1));
  const bf2 m0 = __builtin_bit_cast(bf2, c0), m1 = __builtin_bit_cast(bf2, c1);
  const f2 r = {__builtin_amdgcn_fdot2_f32_bf16(h, m0, a, false), __builtin_amdgcn_fdot2_f32_bf16(h, m1, b, false)};
  hi = __builtin_bit_cast(uint32_t, h);
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(r, bf2));
}

// Eight int8 codes (two uint32) -> eight f16 (uint4), exact.
__device__ inline uint4 i8x8_to_h8(uint32_t a, uint32_t b) {
  const dtile::h4 x = dtile::i8x4_to_h4(a), y = dtile::i8x4_to_h4(b);
  const uint2 u = __builtin_bit_cast(uint2, x), v = __builtin_bit_cast(uint2, y);
  return make_uint4(u.x, u.y, v.x, v.y);
}
// Eight int8 codes -> eight bf16, exact (|q| <= 128 has at most 8 significant bits): each code
// converted to f32, whose upper half is then the bf16 value.
__device__ inline uint32_t i8x2_to_bf2(uint32_t w, int sh) {
  const float f0 = (float)(int)(signed char)(w >> sh), f1 = (float)(int)(signed char)(w >> (sh + 8));
  return (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xffff0000u);
}
__device__ inline uint4 i8x8_to_bf8(uint32_t a, uint32_t b) {
  return make_uint4(i8x2_to_bf2(a, 0), i8x2_to_bf2(a, 16), i8x2_to_bf2(b, 0), i8x2_to_bf2(b, 16));
}

// Workgroup `wg` of a prefill launch: its list of units, items[wg * per_wg ..]. PLO: P carried
// past f16 as hi + lo halves (two P.V products on the same V operand); without it P is rounded
// to f16, the precision of the Metal sibling's prefill.
template <int KVT, int HD, bool PLO, bool QS>
__device__ __forceinline__ void prefill_wg(const PageGeom& g, const PrefillGeom& pg, const PrefillItem* items,
                                           uint32_t per_wg, const float* q, float* out, uint32_t wg,
                                           const MergeCopy& mc) {
  constexpr int NC = HD / 32;                 // Q.K chunks of 32 dims
  constexpr int NJ = HD / 16;                 // O^T blocks of 16 dims
  constexpr int TILE = 16 * HD * 2;           // bytes of one 16-token page tile (K or V) in LDS
  constexpr bool Q8 = KVT == KV_Q8;
  // q8_0: each stage also holds the scales of its 8 page tiles (K tiles 0-3, V tiles 0-3), 16 keys x
  // HD/32 f16 per tile (32*NC bytes, NSL lanes of 16 bytes)
  constexpr int NSL = 2 * NC;
  constexpr int STAGE = 8 * TILE + (Q8 ? 8 * 16 * NSL : 0);
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* kv_lds = smem;                                          // [NSTAGE][K 4 tiles | V 4 tiles | scales]
  const uint32_t kv_lds_addr = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
  PrefillItem* units = (PrefillItem*)(smem + NSTAGE * STAGE);      // this workgroup's unit list
  int* blk_lds = (int*)(units + per_wg);                           // block id of each key page in range

  // The workgroups copy the call's merge list, a slice each (units that are key pieces of a longer
  // range leave partials for the merge launch that follows).
  dtile::copy_merges(mc, wg, gridDim.x);
  // The workgroup's units (the host's balanced assignment, per_wg slots, an empty unit ends the
  // list): fetched once, so each unit starts without a memory round trip for its descriptor.
  {
    const uint32_t* src = (const uint32_t*)(items + (size_t)wg * per_wg);
    for (uint32_t i = threadIdx.x; i < per_wg * (sizeof(PrefillItem) / 4); i += NT) ((uint32_t*)units)[i] = src[i];
  }
  __syncthreads();
  // Steps over (unit, pass): one pass per unit, or two when its Q has lo parts (below).
  uint32_t unit = 0, pass = 0;
  bool lo_any = false;
  while (unit < per_wg) {
  const PrefillItem it = units[unit];
  if (it.n_tok == 0) break;
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, kept in a scalar register
  const uint32_t hq = lane & 15u, grp = lane >> 4;
  const uint32_t G = pg.group;
  const uint32_t pos_last = it.pos0 + it.n_tok - 1;
  const uint32_t page0 = it.page0, n_pages = it.n_pages;   // the unit's key pages
  const uint32_t c_off = it.c_off, n_col = it.n_col;

  // ---- K/V staging. Tile i covers keys (page0 + 4i)*16 .. +64: 4 K and 4 V page tiles, each
  // R rows of 1 KiB (one wave-wide DMA per row). Every wave issues 2*CPT DMAs per tile, so its
  // block ids are wave-uniform and the addresses scalar.
  //   f16: wave w copies half (w & 1) of page tile (w >> 1) on both sides (one page).
  //   bf16: K as two consecutive rows of one page tile; V as the same row of page tiles 2h and
  //      2h+1 (the two tiles of half h), so the thread that loaded them can interleave them for
  //      the P.V products (settle, below). hd 128 (R = 4): every wave does two K rows and one V
  //      row pair; hd 64 (R = 2): waves 0-3 a V row pair each, waves 4-7 two K rows each.
  //   q8_0: wave w copies page tile (w >> 1) of side (w & 1): its QR rows of int8 codes (1 KiB
  //      each) into the upper half of the tile's LDS slot, and its scales (NSL lanes).
  // Pages past the range re-read the last page (finite values whose keys are masked), so stale
  // LDS never meets a zero weight.
  constexpr bool PAIR_V = KVT == KV_BF16;
  constexpr int QR = TILE / 2048;             // q8_0: rows of codes per page tile
  constexpr int R = TILE / 1024;
  constexpr int CPT = TILE / 2 / 1024;        // DMAs per wave per side per tile (on average)
  static_assert((R == 4 || R == 2) && CPT * 2048 == TILE, "page tiles of 2 or 4 KiB");
  const uint32_t n_tiles = __builtin_amdgcn_readfirstlane((n_pages + 3) / 4);   // scalar: bounds barrier loops
  const bool do_k = R == 4 || w >= 4, do_v = R == 4 || w < 4;
  const uint32_t kw = R == 4 ? w : w - 4;
  const uint32_t k_tile = 2 * kw / R, k_row = (2 * kw) % R * 1024;   // K rows k_row, k_row + 1 KiB
  const uint32_t v_half = w / R, v_row = w % R * 1024;               // V row of tiles 2h, 2h+1
  const uint32_t my_tile = w >> 1, my_row = (w & 1) * (TILE / 2);   // f16: both sides
  const uint64_t k_head = g.k_off + (uint64_t)it.kvh * g.k_head;
  const uint64_t v_head = g.v_off + (uint64_t)it.kvh * g.v_head;
  // Scalar base address of page tile `tile` of tile ti, K side or V side. Tiles 0 and 1 take
  // their block ids from the unit descriptor (the block-id list is not in LDS yet). Later tiles
  // read lane-held addresses: lane i holds the K and V base of page 64c + i of the unit's range
  // (clamped to its last page) for the current 64-page chunk c, computed from the block-id list
  // once per 16 tiles, so a DMA costs two readlanes instead of an LDS read that waits for every
  // LDS operation in flight (the operand reads of the tile being computed among them).
  // q8_0 keeps one lane-held block id instead of the four address words, the address then formed
  // in scalar registers: its instance has no registers to spare, and the four words spilled to
  // scratch memory were reloaded on every tile.
  const uint32_t bt_mask = (1u << g.bt_shift) - 1u;
  uint32_t pk_lo = 0, pk_hi = 0, pv_lo = 0, pv_hi = 0, chunk = ~0u;
  int blk_lane = 0;
  auto load_chunk = [&](uint32_t c) {
    const uint32_t p = min(c * 64 + lane, n_pages - 1);
    if constexpr (Q8) {
      blk_lane = blk_lds[p];
      chunk = c;
      return;
    }
    const uint64_t b = (uint64_t)(uintptr_t)g.pool + (uint64_t)(uint32_t)blk_lds[p] * g.block_bytes;
    const uint32_t sub = (((page0 + p) << 4) & bt_mask) >> 4;
    const uint64_t kb = b + k_head + (uint64_t)sub * g.k_tile, vb = b + v_head + (uint64_t)sub * g.v_tile;
    pk_lo = (uint32_t)kb;
    pk_hi = (uint32_t)(kb >> 32);
    pv_lo = (uint32_t)vb;
    pv_hi = (uint32_t)(vb >> 32);
    chunk = c;
  };
  auto page_any = [&](uint32_t ti, uint32_t tile, bool v_side) -> const uint8_t* {
    if (ti < 2) {
      const uint32_t p = min(ti * 4 + tile, n_pages - 1);
      const uint64_t blk = (uint32_t)__builtin_amdgcn_readfirstlane(units[unit].blk[ti * 4 + tile]);
      const uint32_t sub = (((page0 + p) << 4) & bt_mask) >> 4;
      return g.pool + blk * g.block_bytes + (v_side ? v_head + (uint64_t)sub * g.v_tile : k_head + (uint64_t)sub * g.k_tile);
    }
    const uint32_t p = ti * 4 + tile;
    if ((p >> 6) != chunk) load_chunk(p >> 6);
    if constexpr (Q8) {   // lane p % 64 holds the block id of page min(p, n_pages - 1)
      const uint64_t blk = (uint32_t)__builtin_amdgcn_readlane(blk_lane, (int)(p & 63u));
      const uint32_t sub = (((page0 + min(p, n_pages - 1)) << 4) & bt_mask) >> 4;
      return g.pool + blk * g.block_bytes + (v_side ? v_head + (uint64_t)sub * g.v_tile : k_head + (uint64_t)sub * g.k_tile);
    }
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane(v_side ? pv_lo : pk_lo, (int)(p & 63u));
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane(v_side ? pv_hi : pk_hi, (int)(p & 63u));
    return (const uint8_t*)(uintptr_t)(((uint64_t)hi << 32) | lo);
  };
  auto page = [&](uint32_t ti, uint32_t tile, bool v_side) -> const uint8_t* {
    const uint8_t* a = page_any(ti, tile, v_side);
    const uint64_t u = (uint64_t)(uintptr_t)a;   // wave-uniform: kept in scalar registers
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)u);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
    return (const uint8_t*)(uintptr_t)(((uint64_t)hi << 32) | lo);
  };
  // q8_0: the scales of the page tile whose codes start at `codes` (the same page, clamped as
  // page_any clamps it): head base + scale offset + sub * scale stride.
  auto page_scales = [&](uint32_t ti, uint32_t tile, bool v_side, const uint8_t* codes) -> const uint8_t* {
    const uint32_t p = min(ti * 4 + tile, n_pages - 1);
    const uint64_t sub = (((page0 + p) << 4) & bt_mask) >> 4;
    const uint64_t off = v_side ? (uint64_t)g.v_scale + sub * g.v_tile_s - sub * g.v_tile
                                : (uint64_t)g.k_scale + sub * g.k_tile_s - sub * g.k_tile;
    const uint64_t u = (uint64_t)(uintptr_t)codes + off;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)u);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
    return (const uint8_t*)(uintptr_t)(((uint64_t)hi << 32) | lo);
  };
  auto issue = [&](uint32_t ti) {
    const uint32_t stage = kv_lds_addr + (ti % NSTAGE) * STAGE;
    if constexpr (Q8) {
      const uint32_t side = w & 1u, pt = w >> 1;
      const uint8_t* cb = page(ti, pt, side != 0);
      const uint32_t slot = stage + side * 4 * TILE + pt * TILE;
#pragma unroll
      for (int r = 0; r < QR; r++) lds_dma16(cb, r * 1024 + lane * 16, slot + (QR + r) * 1024);
      const uint8_t* sb = page_scales(ti, pt, side != 0, cb);
      // the first NSL lanes: their LDS destinations are the slot's first NSL*16 bytes whether the
      // DMA places a lane by its index or by its rank among the active lanes
      if (lane < (uint32_t)NSL) lds_dma16(sb, lane * 16, stage + 8 * TILE + (side * 4 + pt) * (NSL * 16));
      return;
    }
    if constexpr (!PAIR_V) {
      const uint8_t* kb = page(ti, my_tile, false);
      const uint8_t* vb = page(ti, my_tile, true);
#pragma unroll
      for (int k = 0; k < CPT; k++) {
        lds_dma16(kb, my_row + k * 1024 + lane * 16, stage + my_tile * TILE + my_row + k * 1024);
        lds_dma16(vb, my_row + k * 1024 + lane * 16, stage + 4 * TILE + my_tile * TILE + my_row + k * 1024);
      }
      return;
    }
    if (do_k) {
      const uint8_t* kb = page(ti, k_tile, false);
      lds_dma16(kb, k_row + lane * 16, stage + k_tile * TILE + k_row);
      lds_dma16(kb, k_row + 1024 + lane * 16, stage + k_tile * TILE + k_row + 1024);
    }
    if (do_v) {
#pragma unroll
      for (int t2 = 0; t2 < 2; t2++) {
        const uint8_t* vb = page(ti, 2 * v_half + t2, true);
        lds_dma16(vb, v_row + lane * 16, stage + 4 * TILE + (2 * v_half + t2) * TILE + v_row);
      }
    }
  };
  // After this thread's rows of tile ti have landed, bf16 only: K and V are widened to f16 in
  // place (so both products run in f16 and Q keeps 11 bits per part), and the thread's two V
  // chunks A (tile 2h) and B (tile 2h+1), each [4 keys of dim d | 4 keys of dim d+16], are
  // rewritten as A' = [A keys of d | B keys of d] and B' = [A keys of d+16 | B keys of d+16], so
  // one 16-byte read is a whole 32-key operand of the P.V product. f16 tiles are used as loaded
  // (the extra LDS pass would cost more than the operand assembly it saves).
  // q8_0: the thread's rows of codes (row r at LDS row QR + r of its slot, 16 bytes per lane) are
  // rewritten as 16-bit values in place, read first and then written: the first 8 codes of row r
  // (K: dims 64r + 8g .. +8 of key m, lane 16g + m; V: keys 4(lane/16) .. +4 of dims 64r + lane%16
  // and 64r + 16 + lane%16) are the lane's 16 bytes of LDS row 2r in the f16 tile layout, the last
  // 8 those of row 2r + 1. K becomes f16, V bf16 (the type its scaled weights are carried in).
  bool widen_k = true;   // bf16 pages: false while the unit's Q.K products run on bf16 (below)
  auto settle = [&](uint32_t ti) {
    uint8_t* stage = kv_lds + (ti % NSTAGE) * STAGE;
    if constexpr (Q8) {
      const uint32_t side = w & 1u, pt = w >> 1;
      uint8_t* slot = stage + side * 4 * TILE + pt * TILE + lane * 16;
      uint4 c[QR];
#pragma unroll
      for (int r = 0; r < QR; r++) c[r] = *(const uint4*)(slot + (QR + r) * 1024);
#pragma unroll
      for (int r = 0; r < QR; r++) {
        if (side == 0) {
          *(uint4*)(slot + (2 * r) * 1024) = i8x8_to_h8(c[r].x, c[r].y);
          *(uint4*)(slot + (2 * r + 1) * 1024) = i8x8_to_h8(c[r].z, c[r].w);
        } else {
          *(uint4*)(slot + (2 * r) * 1024) = i8x8_to_bf8(c[r].x, c[r].y);
          *(uint4*)(slot + (2 * r + 1) * 1024) = i8x8_to_bf8(c[r].z, c[r].w);
        }
      }
      return;
    }
    if constexpr (KVT == KV_BF16) {
      if (do_k && widen_k) {
#pragma unroll
        for (int r = 0; r < 2; r++) {
          uint4* p = (uint4*)(stage + k_tile * TILE + k_row + r * 1024 + lane * 16);
          uint4 x = *p;
          x.x = bf2_to_h2(x.x);
          x.y = bf2_to_h2(x.y);
          x.z = bf2_to_h2(x.z);
          x.w = bf2_to_h2(x.w);
          *p = x;
        }
      }
    }
    if constexpr (KVT == KV_BF16) {
      if (do_v) {
        uint4* pa = (uint4*)(stage + 4 * TILE + 2 * v_half * TILE + v_row + lane * 16);
        uint4* pb = (uint4*)((uint8_t*)pa + TILE);
        uint4 x = *pa, y = *pb;
        x = make_uint4(bf2_to_h2(x.x), bf2_to_h2(x.y), bf2_to_h2(x.z), bf2_to_h2(x.w));
        y = make_uint4(bf2_to_h2(y.x), bf2_to_h2(y.y), bf2_to_h2(y.z), bf2_to_h2(y.w));
        *pa = make_uint4(x.x, x.y, y.x, y.y);
        *pb = make_uint4(x.z, x.w, y.z, y.w);
      }
    }
  };

  // ---- unit prologue: the first two tiles' loads go out first (block ids from the descriptor),
  // then the Q loads and the block-id list, so their round trips overlap; the barrier that
  // publishes tile 0 also publishes the list.
  issue(0);
  if (n_tiles > 1) issue(1);
  // Q of column c (pair (token c / G, head c % G)) in dims 32ch + 8grp .. +8 as f16. Q stays
  // unscaled: a Q held in f16 or bf16 values (activations already rounded to the cache's 16-bit
  // type) is then exact in f16, and the products are exact against exactly represented K; the
  // scale multiplies the accumulator in the exponent. A Q with bits below f16 splits into
  // hi + lo f16 parts (~22 bits) whose products sum in one accumulator: in the launch for exact Q,
  // when any lane of the workgroup has a nonzero lo part, the unit runs in two passes of 16
  // columns per wave, the second column block's registers holding the first's lo part (same
  // registers, same products per pass, twice the passes); the QS launch holds both blocks' lo
  // parts too (ql) and runs one pass.
  auto load_q = [&](uint32_t c, float4 (&raw)[NC][2]) {
    const uint32_t t = (c + c_off) / G, hh = (c + c_off) % G;
    const bool valid = c < n_col;
    const float* qp = q + ((size_t)(it.row0 + (valid ? t : 0)) * pg.n_head + it.kvh * G + hh) * HD;
#pragma unroll
    for (int ch = 0; ch < NC; ch++) {
      raw[ch][0] = valid ? *(const float4*)(qp + 32 * ch + 8 * grp) : make_float4(0, 0, 0, 0);
      raw[ch][1] = valid ? *(const float4*)(qp + 32 * ch + 8 * grp + 4) : make_float4(0, 0, 0, 0);
    }
  };
  // f16 hi and lo parts of the raw rows; returns whether any lo part of this lane is nonzero
  auto split_q = [&](const float4 (&raw)[NC][2], h8 (&hi)[NC], h8 (&lo)[NC]) {
    bool nz = false;
#pragma unroll
    for (int ch = 0; ch < NC; ch++) {
      const float4 a = raw[ch][0], b = raw[ch][1];
      const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const _Float16 h = (_Float16)x[i];
        const _Float16 l = (_Float16)(x[i] - (float)h);
        hi[ch][i] = h;
        lo[ch][i] = l;
        nz |= l != (_Float16)0.0f;
      }
    }
    return nz;
  };
  // bf16 pages: a Q held in bf16 values multiplies bf16 K exactly on the bf16 matrix cores, so K
  // needs no widening; qf then holds bf16 bits (split_q_bf16). Any other Q takes the f16 hi + lo
  // path with K widened (two passes, or one in the QS launch). q8_0 pages: the codes are widened
  // to f16 either way; a Q exact in f16 runs one pass.
  // A value is exact in bf16 when the low 16 bits of its f32 encoding are zero: the test ORs the
  // encodings and the bf16 values are their upper halves (one byte permute per pair); the values are
  // only used when every one was exact (otherwise the unit takes the two-pass path).
  auto split_q_bf16 = [&](const float4 (&raw)[NC][2], h8 (&hi)[NC]) {
    uint32_t low = 0;
#pragma unroll
    for (int ch = 0; ch < NC; ch++) {
      const float4 a = raw[ch][0], b = raw[ch][1];
      const uint32_t u[8] = {__float_as_uint(a.x), __float_as_uint(a.y), __float_as_uint(a.z), __float_as_uint(a.w),
                             __float_as_uint(b.x), __float_as_uint(b.y), __float_as_uint(b.z), __float_as_uint(b.w)};
      uint32_t wd[4];
#pragma unroll
      for (int i = 0; i < 8; i += 2) {
        low |= u[i] | u[i + 1];
        wd[i / 2] = __builtin_amdgcn_perm(u[i + 1], u[i], 0x07060302u);   // [hi16(u[i]), hi16(u[i+1])]
      }
      hi[ch] = __builtin_bit_cast(h8, make_uint4(wd[0], wd[1], wd[2], wd[3]));
    }
    return (low & 0xffffu) != 0;
  };
  h8 qf[2][NC];
  if (pass == 0) {
    bool lo_need = false;
    {
      float4 raw[2][NC][2];
      load_q(w * COLS + hq, raw[0]);
      load_q(w * COLS + 16 + hq, raw[1]);
      // ---- block ids of every key page this unit reads
      const int32_t* tab = g.table + (size_t)it.seq * g.bps;
      for (uint32_t p = tid; p < n_pages; p += NT) blk_lds[p] = tab[((page0 + p) << 4) >> g.bt_shift];
      if constexpr (KVT == KV_BF16) {
        lo_need |= split_q_bf16(raw[0], qf[0]);
        lo_need |= split_q_bf16(raw[1], qf[1]);
      } else {
        h8 lo_unused[NC];   // the lo parts are only tested here
        lo_need |= split_q(raw[0], qf[0], lo_unused);
        lo_need |= split_q(raw[1], qf[1], lo_unused);
      }
    }
    // workgroup-wide OR of the lo flags: one word per wave (written by its first lane) behind a
    // barrier (which also publishes the block-id list)
    __shared__ uint32_t lo_flags[PW];
    {
      const bool wave_lo = __ballot(lo_need) != 0;
      if (lane == 0) lo_flags[w] = wave_lo ? 1u : 0u;
    }
    __syncthreads();
    uint32_t lo_or = 0;
#pragma unroll
    for (int i = 0; i < PW; i++) lo_or |= lo_flags[i];
    lo_any = lo_or != 0;
    // the handle's record for its next call's launch choice (workgroup 0's first unit)
    if (wg == 0 && unit == 0 && tid == 0 && pg.q_flag) *pg.q_flag = lo_any ? 1u : 0u;
  }
  // QS: every unit of a 16-bit page launch runs one pass with Q as hi + lo parts
  constexpr bool SPLIT_ALL = QS && !Q8;
  widen_k = KVT != KV_BF16 || lo_any || SPLIT_ALL;
  // Q as f16 hi + lo parts: the QS launch of 16-bit pages runs every unit as one pass of both
  // column blocks, Q as hi (qf) + lo (ql); otherwise a Q with bits below the page type runs two
  // passes of one column block, its Q as hi (qf[0]) + lo (qf[1]).
  h8 ql[NCB][NC];
  if constexpr (SPLIT_ALL) {
#pragma unroll
    for (int x = 0; x < NCB; x++) {
      float4 raw[NC][2];
      load_q(w * COLS + x * 16 + hq, raw);
      split_q(raw, qf[x], ql[x]);
    }
  } else if (lo_any) {
    float4 raw[NC][2];
    load_q(w * COLS + pass * 16 + hq, raw);
    split_q(raw, qf[0], qf[1]);
  }

  // One pass over the unit's key tiles for this wave's column blocks: MODE 0, both blocks
  // (columns 32w .. 32w+31) with Q in f16 (or bf16); MODE 2, both blocks with Q as f16 hi (qf) +
  // lo (ql) parts, the two products of each summed in one accumulator; MODE 1 (LO), block `pb`
  // (columns 32w + 16pb ..) with
  // its Q as hi (qf[0]) + lo (qf[1]).
  auto run = [&](auto mode_tag, uint32_t pb) {
  constexpr int MODE = decltype(mode_tag)::value;
  constexpr bool LO = MODE == 1, LO2 = MODE == 2;
  constexpr int NX = LO ? 1 : NCB;            // column blocks of the pass
  const float c2 = pg.scale_log2;             // scale * log2(e): raw score -> log2 domain
  uint32_t cpos[NCB], clo[NCB];
  bool cval[NCB];
#pragma unroll
  for (int x = 0; x < NX; x++) {
    const uint32_t c = w * COLS + (LO ? pb : x) * 16 + hq;
    const uint32_t t = (c + c_off) / G;
    cval[x] = c < n_col;
    cpos[x] = it.pos0 + (cval[x] ? t : 0);
    clo[x] = (pg.window > 0 && cpos[x] + 1 > pg.window) ? cpos[x] + 1 - pg.window : 0;
  }

  // Online-softmax state per column. The accumulator of Q.K starts at nm = -m (m: the column's
  // reference max in raw score units, 0 while it has seen no key), so a product is s - m and the
  // weight is p = 2^(c2 (s - m) + PUP): weights are scaled by 2^PUP so that every weight (<=
  // 2^(12 + PUP), below) keeps a normal f16 lo part down to 2^(-PUP - 2) of the largest. thr: the
  // relative score (log2 domain) above which m must move (8, or -inf while no key is visible).
  // l: row sum; O^T.
  constexpr float PUP = 3.0f;
  float nm[NCB], thr[NCB], l[NCB];
  f4 nmv[NCB];
  f4 O[NJ][NCB];
#pragma unroll
  for (int x = 0; x < NX; x++) {
    nm[x] = 0.f;
    nmv[x] = f4{0.f, 0.f, 0.f, 0.f};
    thr[x] = -INFINITY;
    l[x] = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; j++) O[j][x] = f4{0.f, 0.f, 0.f, 0.f};
  }
  // this wave's lowest/highest column positions in the pass (mask-free tiles)
  const uint32_t c_first = w * COLS + (LO ? pb * 16 : 0), c_span = LO ? 16 : COLS;
  const bool wave_active = c_first < n_col;
  uint32_t wpos_min, wpos_max;
  {
    const uint32_t c_last = min(c_first + c_span, n_col) - 1;   // n_col >= 1
    const uint32_t t1 = (c_last + c_off) / G;
    wpos_min = it.pos0 + min((c_first + c_off) / G, t1);
    wpos_max = it.pos0 + t1;
  }
  const uint32_t wlo_max = (pg.window > 0 && wpos_max + 1 > pg.window) ? wpos_max + 1 - pg.window : 0;

  // Matrix-core operands of one 32-key half, read from LDS ahead of the products that use them
  // (the reads of one phase are in flight while the previous phase computes).
  // q8_0: s[kk] holds the scales of keys 4g .. 4g+3 of page tile kk (all HD/32 chunks, f16, key-major)
  constexpr int NSC = Q8 ? NC / 2 : 1;
  struct KOps { uint4 a[NC][2]; uint4 s[2][NSC]; };   // K: chunk ch of page tile kk
  struct VOps { uint4 a[NJ]; uint4 s[2][NSC]; };      // V^T: dims 16j.. of both page tiles (8 bytes each)
  // the scales of page tile `tile` on side `side` of the stage at `st`, this lane's keys
  auto load_scales = [&](uint4 (&s)[NSC], const uint8_t* st, int side, int tile) {
#pragma unroll
    for (int c = 0; c < NSC; c++)
      s[c] = *(const uint4*)(st + 8 * TILE + (side * 4 + tile) * (NSL * 16) + grp * (8 * NC) + c * 16);
  };
  auto load_k = [&](KOps& o, const uint8_t* kt, int kp) {
#pragma unroll
    for (int ch = 0; ch < NC; ch++)
#pragma unroll
      for (int kk = 0; kk < 2; kk++) o.a[ch][kk] = *(const uint4*)(kt + (2 * kp + kk) * TILE + ch * 1024 + lane * 16);
    if constexpr (Q8) {
#pragma unroll
      for (int kk = 0; kk < 2; kk++) load_scales(o.s[kk], kt, 0, 2 * kp + kk);
    }
  };
  // k index 8g+i of the P.V product is key 4g+i of the half's first 16-key page tile (i < 4) or
  // key 4g+i-4 of its second: 8 bytes from each page tile (f16), or after settle (bf16) one
  // 16-byte chunk (in the first tile's slot for even j, the second's for odd j).
  auto load_v = [&](VOps& o, const uint8_t* vt, int kp) {
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      if constexpr (KVT == KV_BF16) {
        o.a[j] = *(const uint4*)(vt + (2 * kp + (j & 1)) * TILE + (j >> 1) * 1024 + lane * 16);
      } else {
        const uint32_t off = (j >> 1) * 1024 + lane * 16 + (j & 1) * 8;
        const uint2 v0 = *(const uint2*)(vt + (2 * kp) * TILE + off);
        const uint2 v1 = *(const uint2*)(vt + (2 * kp + 1) * TILE + off);
        o.a[j] = make_uint4(v0.x, v0.y, v1.x, v1.y);
      }
    }
    if constexpr (Q8) {
#pragma unroll
      for (int kk = 0; kk < 2; kk++) load_scales(o.s[kk], vt - 4 * TILE, 1, 2 * kp + kk);
    }
  };
  // S^T for the 32 keys of a half (two 16-key page tiles) x the pass's columns (LO: the hi and
  // lo products of one column block, summed)
  auto qk = [&](f4 (&S)[2][NCB], const KOps& ko) {
    if constexpr (Q8 && !LO) {   // per chunk: Q (exact in f16) against the codes, times the key's scale
#pragma unroll
      for (int ch = 0; ch < NC; ch++) {
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
          const h8 a = __builtin_bit_cast(h8, ko.a[ch][kk]);
#pragma unroll
          for (int cb = 0; cb < NCB; cb++) {
            const f4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[cb][ch], f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
            for (int r = 0; r < 4; r++)
              S[kk][cb][r] = fmaf(t[r], (float)dtile::scale_h<NC>(ko.s[kk], r, ch), ch == 0 ? nm[cb] : S[kk][cb][r]);
          }
        }
      }
      return;
    }
    if constexpr (Q8) {   // (two-pass form) per chunk: the hi + lo products, times the key's scale
#pragma unroll
      for (int ch = 0; ch < NC; ch++) {
#pragma unroll
        for (int kk = 0; kk < 2; kk++) {
          const h8 a = __builtin_bit_cast(h8, ko.a[ch][kk]);
          f4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[0][ch], f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
          t = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[1][ch], t, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 4; r++)
            S[kk][0][r] = fmaf(t[r], (float)dtile::scale_h<NC>(ko.s[kk], r, ch), ch == 0 ? nm[0] : S[kk][0][r]);
        }
      }
      return;
    }
#pragma unroll
    for (int ch = 0; ch < NC; ch++) {
#pragma unroll
      for (int kk = 0; kk < 2; kk++) {
        const h8 a = __builtin_bit_cast(h8, ko.a[ch][kk]);
        if constexpr (LO2) {
#pragma unroll
          for (int cb = 0; cb < NCB; cb++) {
            const f4 acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[cb][ch], ch == 0 ? nmv[cb] : S[kk][cb], 0, 0, 0);
            S[kk][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, ql[cb][ch], acc, 0, 0, 0);
          }
        } else if constexpr (LO) {
          S[kk][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[0][ch], ch == 0 ? nmv[0] : S[kk][0], 0, 0, 0);
          S[kk][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[1][ch], ch == 0 ? f4{0.f, 0.f, 0.f, 0.f} : S[kk][1],
                                                            0, 0, 0);
        } else {
#pragma unroll
          for (int cb = 0; cb < NCB; cb++) {
            const f4 acc = ch == 0 ? nmv[cb] : S[kk][cb];
            if constexpr (KVT == KV_BF16)   // bf16 K as loaded, bf16 Q
              S[kk][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(dtile::b8, ko.a[ch][kk]),
                                                                 __builtin_bit_cast(dtile::b8, qf[cb][ch]), acc, 0, 0, 0);
            else
              S[kk][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[cb][ch], acc, 0, 0, 0);
          }
        }
      }
    }
    if constexpr (LO) {
#pragma unroll
      for (int kk = 0; kk < 2; kk++) S[kk][0] += S[kk][1];
    }
  };
  // keys outside a column's [lo, pos] get -inf (keys past the range are past every position)
  auto mask = [&](f4 (&S)[2][NCB], uint32_t kbase) {
#pragma unroll
    for (int x = 0; x < NX; x++) {
#pragma unroll
      for (int kk = 0; kk < 2; kk++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const uint32_t key = kbase + kk * 16 + grp * 4 + r;
          S[kk][x][r] = (key > cpos[x] || key < clo[x]) ? -INFINITY : S[kk][x][r];
        }
      }
    }
  };
  // Lazy reference max: m moves (rescaling O and l) only when the weights of a half grow too
  // large. Each lane sums its own 8 weights per column (the row-sum terms, needed anyway); a sum
  // above 2^(12 + PUP) (some relative score above 9: every score <= 8 gives a sum <= 2^(11 + PUP))
  // or a column with no visible key yet sends the wave to the rare path, where the column max is
  // reduced over the lane groups and m moves to it if it exceeds m + 8 (or is the first finite
  // score). So every weight converted to f16 is <= 2^(12 + PUP), and O is almost never rescaled.
  // The scores of the next half, already computed against the old m, are shifted with it.
  auto expo = [&](const f4 (&S)[2][NCB], float (&pw)[NCB][8], float (&ps)[NCB]) {
#pragma unroll
    for (int x = 0; x < NX; x++) {
#pragma unroll
      for (int kk = 0; kk < 2; kk++) {
#pragma unroll
        for (int r = 0; r < 4; r++) pw[x][kk * 4 + r] = exp2_fast(fmaf(S[kk][x][r], c2, PUP));
      }
      ps[x] = ((pw[x][0] + pw[x][1]) + (pw[x][2] + pw[x][3])) + ((pw[x][4] + pw[x][5]) + (pw[x][6] + pw[x][7]));
    }
  };
  auto rebase = [&](f4 (&S)[2][NCB], f4 (&Sn)[2][NCB]) {
#pragma unroll
    for (int x = 0; x < NX; x++) {
      const float lm = fmaxf(fmaxf(fmaxf(S[0][x][0], S[0][x][1]), fmaxf(S[0][x][2], S[0][x][3])),
                             fmaxf(fmaxf(S[1][x][0], S[1][x][1]), fmaxf(S[1][x][2], S[1][x][3])));
      const float tmax = max_over_groups(lm);   // raw units, relative to m
      const bool mv = tmax * c2 > thr[x];
      const float sh = mv ? tmax : 0.f;
      const float nm_new = nm[x] - sh;
      // no key seen yet (thr = -inf): O and l are zero, and tmax may be any finite value
      const float alpha = !mv ? 1.f : (thr[x] == -INFINITY ? 0.f : exp2_fast((nm_new - nm[x]) * c2));
      l[x] *= alpha;
#pragma unroll
      for (int j = 0; j < NJ; j++) O[j][x] *= alpha;
#pragma unroll
      for (int kk = 0; kk < 2; kk++) {
        S[kk][x] -= sh;
        Sn[kk][x] -= sh;
      }
      nm[x] = nm_new;
      nmv[x] = f4{nm_new, nm_new, nm_new, nm_new};
      thr[x] = mv ? 8.0f : thr[x];
    }
  };
  // P = 2^(c2 (s - m) + PUP) as f16 hi (+ lo) parts, row sums in f32 (Sn: the next half's scores,
  // see rebase)
  // q8_0: the weights stay in f32 (pq) for pv, which scales them per V block
  float pq[NCB][8];
  auto softmax = [&](f4 (&S)[2][NCB], h8 (&Ph)[NCB], h8 (&Pl)[NCB], f4 (&Sn)[2][NCB]) {
    float pw[NCB][8], ps[NCB];
    expo(S, pw, ps);
    bool need = false;
#pragma unroll
    for (int x = 0; x < NX; x++) need |= !(ps[x] <= 4096.f * 8.f) || thr[x] == -INFINITY;
    if (__ballot(need)) {
      rebase(S, Sn);
      expo(S, pw, ps);
    }
    if constexpr (Q8) {
#pragma unroll
      for (int x = 0; x < NX; x++) {
        l[x] += ps[x];
#pragma unroll
        for (int e = 0; e < 8; e++) pq[x][e] = pw[x][e];
      }
      return;
    }
#pragma unroll
    for (int x = 0; x < NX; x++) {
      l[x] += ps[x];
      uint32_t hw[4], lw[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        if constexpr (PLO) {
          dtile::split_pair(pw[x][2 * i], pw[x][2 * i + 1], hw[i], lw[i]);
        } else {
          typedef float f2 __attribute__((ext_vector_type(2)));
          typedef _Float16 h2 __attribute__((ext_vector_type(2)));
          const f2 v = {pw[x][2 * i], pw[x][2 * i + 1]};
          hw[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, h2));
          lw[i] = 0;
        }
      }
      Ph[x] = __builtin_bit_cast(h8, make_uint4(hw[0], hw[1], hw[2], hw[3]));
      Pl[x] = __builtin_bit_cast(h8, make_uint4(lw[0], lw[1], lw[2], lw[3]));
    }
  };
  // O^T += V^T P^T over a half, 32 keys per MFMA
  auto pv = [&](const h8 (&Ph)[NCB], const h8 (&Pl)[NCB], const VOps& vo) {
    if constexpr (Q8) {   // per 32-dim V block b: P * d_V[key][b] as bf16 hi + lo
#pragma unroll
      for (int b = 0; b < NC; b++) {
#pragma unroll
        for (int x = 0; x < NX; x++) {
          uint32_t hw[4], lw[4];
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int e0 = 2 * i, e1 = 2 * i + 1;   // weight e: key 4g + e%4 of page tile e/4
            // weight x scale as v_fma_mix_f32 on the f16 scale in place (weights and scales >= 0)
            split_pair_bf16(__builtin_fmaf(pq[x][e0], (float)dtile::scale_h<NC>(vo.s[e0 / 4], e0 % 4, b), 0.0f),
                            __builtin_fmaf(pq[x][e1], (float)dtile::scale_h<NC>(vo.s[e1 / 4], e1 % 4, b), 0.0f),
                            hw[i], lw[i]);
          }
          const dtile::b8 ph = __builtin_bit_cast(dtile::b8, make_uint4(hw[0], hw[1], hw[2], hw[3]));
          const dtile::b8 pl = __builtin_bit_cast(dtile::b8, make_uint4(lw[0], lw[1], lw[2], lw[3]));
#pragma unroll
          for (int jj = 0; jj < 2; jj++) {
            const dtile::b8 va = __builtin_bit_cast(dtile::b8, vo.a[2 * b + jj]);
            O[2 * b + jj][x] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, ph, O[2 * b + jj][x], 0, 0, 0);
            O[2 * b + jj][x] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pl, O[2 * b + jj][x], 0, 0, 0);
          }
        }
      }
      return;
    }
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const h8 va = __builtin_bit_cast(h8, vo.a[j]);
#pragma unroll
      for (int x = 0; x < NX; x++) {
        O[j][x] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, Ph[x], O[j][x], 0, 0, 0);
        if constexpr (PLO) O[j][x] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, Pl[x], O[j][x], 0, 0, 0);
      }
    }
  };

  // Pipeline. Tile ti's loads are issued at the start of iteration ti-2. In iteration ti-1
  // each thread waits for its own share of them and widens it (bf16) inside the first block, where
  // the conversions overlap that block's matrix products; the barrier in the middle of iteration
  // ti-1 then publishes tile ti, right before the block that finishes tile ti-1 (softmax + P.V of
  // its second half) and starts tile ti (Q.K of its first half), so the matrix products of one
  // half always have the other half's exponentials beside them.
  // Stage reuse: tile ti+2 goes to stage (ti+2) % 4, last read while finishing tile ti-2, which
  // every wave completed before the barrier of iteration ti-1. A thread issues 2*CPT loads per
  // tile, so "at most 2*CPT outstanding" means its share of the older tile has landed. The last
  // iteration widens a stage no later tile uses (harmless), which keeps that block branch-free.
  // Every tile is computed (keys outside a column's range are masked), except by waves that own
  // no column at all.
  auto wait_tile = [&](uint32_t ti) {  // this thread's loads of tile ti have landed
    if (ti + 1 < n_tiles) {   // a thread's loads per tile: 2*CPT, or QR + 1 (q8_0: codes, scales)
      if constexpr (Q8 ? QR + 1 == 2 : CPT == 1)
        asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
      else if constexpr (Q8)
        asm volatile("s_waitcnt vmcnt(3)" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
  };
  auto sync = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
  f4 S0[2][NCB], S1[2][NCB];
  h8 Ph[NCB], Pl[NCB];
  KOps ko;
  VOps vo;
  wait_tile(0);
  settle(0);
  sync();
  if (wave_active) {
    load_k(ko, kv_lds, 0);
    qk(S0, ko);
  }
  for (uint32_t ti = 0; ti < n_tiles; ti++) {
    if (ti + 2 < n_tiles) issue(ti + 2);
    const uint8_t* kt = kv_lds + (ti % NSTAGE) * STAGE;
    const uint8_t* vt = kt + 4 * TILE;
    const uint32_t key0 = (page0 + ti * 4) * 16;
    const bool need_mask = key0 + BK - 1 > wpos_min || key0 < wlo_max || key0 + BK - 1 > pos_last;
    if (wave_active) {
      load_k(ko, kt, 1);
      // MODE 2 (twice the Q registers): V's operands are read once the K operands are consumed,
      // during the exponentials, so the two sets are not held at once
      if constexpr (!LO2) load_v(vo, vt, 0);
      if (need_mask) mask(S0, key0);
      wait_tile(ti + 1);
      settle(ti + 1);
      qk(S1, ko);
      if constexpr (LO2) load_v(vo, vt, 0);
      softmax(S0, Ph, Pl, S1);
      pv(Ph, Pl, vo);
      if (need_mask) mask(S1, key0 + 32);
    } else {
      wait_tile(ti + 1);
      settle(ti + 1);
    }
    if (ti + 1 < n_tiles) sync();
    if (wave_active) {
      if constexpr (!LO2) load_v(vo, vt, 1);
      // first half of the next tile (after the last tile: a stale stage, never used), issued
      // before this half's exponentials so its products overlap them and are complete when the
      // next iteration reads S0
      load_k(ko, kv_lds + ((ti + 1) % NSTAGE) * STAGE, 0);
      qk(S0, ko);
      if constexpr (LO2) load_v(vo, vt, 1);
      softmax(S1, Ph, Pl, S0);
      pv(Ph, Pl, vo);
    }
  }

  // ---- epilogue: per column, out = O / l (l summed over the lane groups); a key piece of a longer
  // range leaves its partial (O, m, l) instead, m as the log2-domain reference its weights were
  // taken against (c2 (s - m_raw) + PUP = c2 s - (c2 m_raw - PUP)), -inf if no key was visible
#pragma unroll
  for (int x = 0; x < NX; x++) {
    const float lt = sum_over_groups(l[x]);
    if (!cval[x]) continue;
    const uint32_t col = w * COLS + (LO ? pb : x) * 16 + hq;
    const uint32_t t = (col + c_off) / G, hh = (col + c_off) % G;
    if (it.slot != NO_SLOT) {
      float* pp = pg.part + ((size_t)(it.slot + t * it.slot_stride) * pg.ng + hh) * (HD + 4);
#pragma unroll
      for (int j = 0; j < NJ; j++) *(float4*)(pp + 16 * j + 4 * grp) = make_float4(O[j][x][0], O[j][x][1], O[j][x][2], O[j][x][3]);
      if (grp == 0) {
        pp[HD] = thr[x] == -INFINITY ? -INFINITY : -nm[x] * c2 - PUP;
        pp[HD + 1] = lt;
      }
      continue;
    }
    // the output is stored non-temporally (nothing here reads it again; lines left dirty in the
    // L2 would be written back at the kernel's end, between it and the next launch: c3's step
    // 217.7 -> 211-212 us); the partials above stay cacheable for the merge that follows
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    float* op = out + ((size_t)(it.row0 + t) * pg.n_head + it.kvh * G + hh) * HD;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const f4 o = O[j][x] * inv;
      __builtin_nontemporal_store(o, (f4*)(op + 16 * j + 4 * grp));
    }
  }
  // every wave is done with the stages and block ids before the next pass or unit refills them
  __syncthreads();
  };

  if constexpr (SPLIT_ALL) {
    run(std::integral_constant<int, 2>{}, 0);
    unit++;
  } else {
    if (!lo_any) {
      run(std::integral_constant<int, 0>{}, 0);
      unit++;
    } else {
      run(std::integral_constant<int, 1>{}, pass);
      pass ^= 1u;
      if (pass == 0) unit++;
    }
  }
  }
}

template <int KVT, int HD, bool PLO, bool QS>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_kernel(PageGeom g, PrefillGeom pg, const PrefillItem* items, uint32_t per_wg, const float* q,
                    float* out, MergeCopy mc) {
  prefill_wg<KVT, HD, PLO, QS>(g, pg, items, per_wg, q, out, blockIdx.x, mc);
}

// A mixed batch (prefill units and decode items) in one launch: workgroups 0 .. pf_wg-1 run the
// prefill units as prefill_kernel does (one per CU it reaches), the others take PW decode items
// each, a wave per item, on the CUs the prefill workgroups leave free and then on those they
// release. The decode waves fit the same register budget (two waves per SIMD) and each
// workgroup carries the prefill LDS allocation, so a CU holds one workgroup of either kind: the
// same eight waves per CU the decode kernel runs at. One launch instead of a decode launch on a
// second stream saves the two cross-stream waits and their idle gaps. r.local_merge (= PW): a
// split row's items are waves of one decode workgroup and merge there, in the workgroup's LDS
// (no merge launch).
template <int KVT, int HD, bool PLO, bool QS>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mixed_kernel(PageGeom g, PrefillGeom pg, const PrefillItem* pitems, uint32_t per_wg, uint32_t pf_wg, RowGeom r,
                  const DecodeItem* items, uint32_t n_items, const float* q, float* out, float* part, MergeCopy mc) {
  dtile::copy_merges(mc, blockIdx.x, gridDim.x);   // every workgroup copies a slice of the merge list
  if (blockIdx.x < pf_wg) {
    prefill_wg<KVT, HD, PLO, QS>(g, pg, pitems, per_wg, q, out, blockIdx.x, MergeCopy{nullptr, nullptr, 0});
    return;
  }
  const uint32_t b = blockIdx.x - pf_wg;
  const uint32_t wi = b * PW + (threadIdx.x >> 6);
  if (r.local_merge) {   // uniform over the launch
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    float* lp = (float*)smem;   // PW partials: within the prefill allocation every workgroup carries
    if (wi < n_items) dtile::decode_item<KVT, HD, HD, true>(g, r, items, wi, q, out, part, lp);
    __syncthreads();   // every wave of the workgroup, with an item or not
    if (wi < n_items) dtile::local_merge<HD, PW>(r, items, wi, lp, out);
    return;
  }
  if (wi < n_items) dtile::decode_item<KVT, HD, HD>(g, r, items, wi, q, out, part);
}

template <int KVT, int HD>
hipError_t launch_t(const PageGeom& g, const PrefillGeom& pg, const PrefillItem* items, uint32_t n_wg,
                    uint32_t per_wg, uint32_t max_pages, const float* q, float* out, const MergeCopy& mc, hipStream_t s,
                    const LaunchEv& ev) {
  const uint32_t lds = (uint32_t)prefill_lds_bytes(KVT, HD, max_pages, per_wg);
  // q8_0 has one instance: its scaled weights are always carried as hi + lo (prefill_p_f16 applies to
  // 16-bit pages) and its Q with lo parts runs two passes; 16-bit pages have an instance per Q form
  if constexpr (KVT != KV_Q8) {
    if (pg.p_f16 && pg.q_split)
      LMH_LAUNCH(ev, (prefill_kernel<KVT, HD, false, true>), dim3(n_wg), dim3(NT), lds, s, g, pg, items, per_wg, q, out, mc);
    else if (pg.p_f16)
      LMH_LAUNCH(ev, (prefill_kernel<KVT, HD, false, false>), dim3(n_wg), dim3(NT), lds, s, g, pg, items, per_wg, q, out, mc);
    else if (pg.q_split)
      LMH_LAUNCH(ev, (prefill_kernel<KVT, HD, true, true>), dim3(n_wg), dim3(NT), lds, s, g, pg, items, per_wg, q, out, mc);
    else
      LMH_LAUNCH(ev, (prefill_kernel<KVT, HD, true, false>), dim3(n_wg), dim3(NT), lds, s, g, pg, items, per_wg, q, out, mc);
    return hipGetLastError();
  }
  LMH_LAUNCH(ev, (prefill_kernel<KVT, HD, true, false>), dim3(n_wg), dim3(NT), lds, s, g, pg, items, per_wg, q, out, mc);
  return hipGetLastError();
}

template <int KVT, int HD>
hipError_t launch_mixed_t(const PageGeom& g, const PrefillGeom& pg, const PrefillItem* pitems, uint32_t pf_wg,
                          uint32_t per_wg, uint32_t max_pages, const RowGeom& r, const DecodeItem* items,
                          uint32_t n_items, const float* q, float* out, float* part, const MergeCopy& mc,
                          hipStream_t s, const LaunchEv& ev) {
  const uint32_t lds = (uint32_t)prefill_lds_bytes(KVT, HD, max_pages, per_wg);
  const uint32_t n_wg = pf_wg + (n_items + PW - 1) / PW;
  if (r.local_merge && (r.local_merge != (uint32_t)PW || lds < PW * dtile::local_partial_floats<HD>() * sizeof(float)))
    return hipErrorInvalidValue;
#define LMH_MIXED_LAUNCH(P, S)                                                                               \
  LMH_LAUNCH(ev, (mixed_kernel<KVT, HD, P, S>), dim3(n_wg), dim3(NT), lds, s, g, pg, pitems, per_wg, pf_wg, r, items, \
             n_items, q, out, part, mc)
  if constexpr (KVT != KV_Q8) {
    if (pg.p_f16 && pg.q_split) LMH_MIXED_LAUNCH(false, true);
    else if (pg.p_f16) LMH_MIXED_LAUNCH(false, false);
    else if (pg.q_split) LMH_MIXED_LAUNCH(true, true);
    else LMH_MIXED_LAUNCH(true, false);
    return hipGetLastError();
  }
  LMH_MIXED_LAUNCH(true, false);
#undef LMH_MIXED_LAUNCH
  return hipGetLastError();
}

}  // namespace

uint32_t prefill_cols_per_unit() { return PW * COLS; }

uint32_t prefill_wg_per_cu() { return 1; }   // the LDS stages fill a CU

size_t prefill_static_lds_bytes() { return 64; }  // lo_flags[PW] rounded up

size_t prefill_lds_bytes(uint32_t kv_type, uint32_t hd, uint32_t max_pages, uint32_t per_wg) {
  const size_t stage = 8 * (16 * (size_t)hd * 2) + (kv_type == KV_Q8 ? 8 * (size_t)hd : 0);   // + q8_0 scales
  return NSTAGE * stage + (size_t)per_wg * sizeof(PrefillItem) + (size_t)max_pages * 4;
}

bool prefill_supported(uint32_t kv_type, uint32_t hd, uint32_t hdv, uint32_t group) {
  return (kv_type == KV_F16 || kv_type == KV_BF16 || kv_type == KV_Q8) && hd == hdv && (hd == 64 || hd == 128) &&
         group >= 1 && group <= PW * COLS;
}

hipError_t launch_mixed(const PageGeom& g, const PrefillGeom& pg, const PrefillItem* pitems, uint32_t pf_wg,
                        uint32_t per_wg, uint32_t max_pages, const RowGeom& r, const DecodeItem* items,
                        uint32_t n_items, const float* q, float* out, float* part, const MergeCopy& mc,
                        hipStream_t s, const LaunchEv& ev) {
  if (pf_wg == 0 || per_wg == 0 || n_items == 0 || g.hd != g.hdv) return hipErrorInvalidValue;
#define LMH_MIXED(T, D)                                                                                          \
  if (g.kv_type == T && g.hd == D)                                                                               \
    return launch_mixed_t<T, D>(g, pg, pitems, pf_wg, per_wg, max_pages, r, items, n_items, q, out, part, mc, s, ev);
  LMH_MIXED(KV_F16, 128) LMH_MIXED(KV_F16, 64) LMH_MIXED(KV_BF16, 128) LMH_MIXED(KV_BF16, 64)
  LMH_MIXED(KV_Q8, 128) LMH_MIXED(KV_Q8, 64)
#undef LMH_MIXED
  return hipErrorInvalidValue;
}

hipError_t launch_prefill(const PageGeom& g, const PrefillGeom& pg, const PrefillItem* items, uint32_t n_wg,
                          uint32_t per_wg, uint32_t max_pages, const float* q, float* out, const MergeCopy& mc,
                          hipStream_t s, const LaunchEv& ev) {
  if (n_wg == 0 || per_wg == 0) return hipSuccess;
  if (g.kv_type == KV_BF16) {
    if (g.hd == 128) return launch_t<KV_BF16, 128>(g, pg, items, n_wg, per_wg, max_pages, q, out, mc, s, ev);
    if (g.hd == 64) return launch_t<KV_BF16, 64>(g, pg, items, n_wg, per_wg, max_pages, q, out, mc, s, ev);
  } else if (g.kv_type == KV_F16) {
    if (g.hd == 128) return launch_t<KV_F16, 128>(g, pg, items, n_wg, per_wg, max_pages, q, out, mc, s, ev);
    if (g.hd == 64) return launch_t<KV_F16, 64>(g, pg, items, n_wg, per_wg, max_pages, q, out, mc, s, ev);
  } else if (g.kv_type == KV_Q8) {
    if (g.hd == 128) return launch_t<KV_Q8, 128>(g, pg, items, n_wg, per_wg, max_pages, q, out, mc, s, ev);
    if (g.hd == 64) return launch_t<KV_Q8, 64>(g, pg, items, n_wg, per_wg, max_pages, q, out, mc, s, ev);
  }
  return hipErrorInvalidValue;
}

}  // namespace lmh
