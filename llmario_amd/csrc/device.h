// device.h — structures shared by the host side (host.cpp) and the HIP kernels.
//
// Page layout (one layer's share of one block; the block holds every layer, K then V, like the
// reference's block, crates/engine/model/src/kv.rs:286-324):
//
//   [K: head 0 .. n_kv-1][V: head 0 .. n_kv-1]
//
// Each (layer, KV head) region covers the block's `block_tokens` positions as 16-token tiles.
// Inside a tile, elements sit in the order the matrix-core operands of the decode/prefill kernels
// read them, so a wave's 16-byte-per-lane load covers 1 KiB of contiguous HBM:
//
//   f16/bf16 K (MFMA 16x16x32 A operand, lane l = 16*g + m holds key m, dims 32c+8g .. +8):
//       byte(m, d) = (d/32)*1024 + (16*((d/8)%4) + m)*16 + (d%8)*2
//   f16/bf16 V (MFMA 16x16x16 A operand of O^T = V^T P^T, lane l = 16*(k/4) + d%16 holds
//       keys 4*(k/4) .. +4 of dim d):
//       byte(k, d) = (d/32)*1024 + (16*(k/4) + d%16)*16 + ((d/16)%2)*8 + (k%4)*2
//   q8_0 K codes: byte(m, d) = (d/64)*1024 + (16*((d/8)%4) + m)*16 + ((d/32)%2)*8 + d%8
//   q8_0 V codes: byte(k, d) = (d/64)*1024 + (16*(k/4) + d%16)*16 + ((d/16)%4)*4 + k%4
//   q8_0 scales (K and V alike), f16, after all code tiles of the head: [tile][key m][d/32]
//   f32 K/V: plain row-major [key m][d] (the VALU decode path reads rows).
//
// Row layout (PageGeom::layout = 1), for the geometries the tile layouts above do not take (head
// widths off the matrix-core instances, hd != hdv pairs without one, blocks under 16 positions):
// each (layer, KV head) region holds min(bt, 16)-row tiles of key rows m in the reference's row
// encoding, row-major [m][d] (f16 / bf16 bits, f32, q8_0 codes), q8_0 scales after the codes as
// above. Same bytes per block; read by the VALU decode kernel (decode_rows_kernel).
//
// The total bytes per block equal the reference's `block_bytes` for the same geometry and type
// (q8_0: 34 bytes per 32 values; f16/bf16: 2 bytes; f32: 4 bytes per value).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "work.h"

namespace lmh {

// Where one layer's pages live. Tile t (16 positions) of KV head h in block b:
//   K values at pool + b*block_bytes + k_off + h*k_head + t*k_tile
//   K scales at pool + b*block_bytes + k_off + h*k_head + k_scale + t*k_tile_s  (q8_0 only)
struct PageGeom {
  uint8_t* pool;
  uint64_t block_bytes;
  uint32_t k_off, v_off;
  uint32_t k_head, v_head;
  uint32_t k_tile, v_tile;
  uint32_t k_scale, v_scale;
  uint32_t k_tile_s, v_tile_s;
  uint32_t bt_shift;  // log2(block_tokens)
  uint32_t bps;       // blocks per sequence (table row length)
  const int32_t* table;  // [n_seqs][bps] block ids
  uint32_t kv_type, n_kv, hd, hdv;
  uint32_t layout;  // 0: tiles in matrix-core operand order; 1: row-major rows (see above)
};

__host__ __device__ inline uint32_t k16_off(uint32_t m, uint32_t d) {
  return (d >> 5) * 1024u + ((((d >> 3) & 3u) << 4) + m) * 16u + (d & 7u) * 2u;
}
__host__ __device__ inline uint32_t v16_off(uint32_t k, uint32_t d) {
  return (d >> 5) * 1024u + (((k >> 2) << 4) + (d & 15u)) * 16u + ((d >> 4) & 1u) * 8u + (k & 3u) * 2u;
}
__host__ __device__ inline uint32_t kq8_off(uint32_t m, uint32_t d) {
  return (d >> 6) * 1024u + ((((d >> 3) & 3u) << 4) + m) * 16u + ((d >> 5) & 1u) * 8u + (d & 7u);
}
__host__ __device__ inline uint32_t vq8_off(uint32_t k, uint32_t d) {
  return (d >> 6) * 1024u + (((k >> 2) << 4) + (d & 15u)) * 16u + ((d >> 4) & 3u) * 4u + (k & 3u);
}

struct RowGeom {
  const int32_t* row_seq;  // [n_rows]
  const int32_t* row_pos;  // [n_rows]
  uint32_t n_head, group;  // group = n_head / n_kv
  uint32_t ng;             // heads per item = min(group, 16)
  float scale_log2;        // scale * log2(e): scores kept in the log2 domain
  uint32_t window;         // 0 = none
  uint32_t local_merge;    // decode: 0, or split rows merge inside workgroups of this many waves (slots LOCAL_SLOT | ...)
};

struct PrefillGeom {
  uint32_t n_head, group;
  float scale_log2;  // scale * log2(e)
  uint32_t window;   // 0 = none
  uint32_t p_f16;    // 1: P rounded to f16 for P.V (Metal's prefill precision); 0: f16 hi + lo (q8_0: always hi + lo)
  uint32_t ng;       // heads per partial slot (units that are key pieces write partials)
  uint32_t q_split;  // 1: f16 / bf16 pages run every unit as one pass of Q hi + lo products
  float* part;       // the call's partial slots
  uint32_t* q_flag;  // workgroup 0 records whether its first unit's Q has bits below the page type
};

// Fused per-row tail of attention_block (see lmh_qk_rope_store): flags as LMH_ROPE_*.
struct RopeGeom {
  uint32_t n_head, q_stride, flags, half_rot;  // half_rot: rotated pairs (0 = no rotation)
  float eps, freq_scale, attn_factor;
  const float* q_norm;    // [hd] or null
  const float* k_norm;    // [hd] or null
  const float* freq_div;  // [half_rot] or null
  const float* freq;      // [half_rot] theta^(-2i/rot_dim), computed on the host
};
constexpr uint32_t ROPE_Q_NORM = 1, ROPE_K_NORM = 2, ROPE_V_NORM = 4, ROPE_APPLY = 8, ROPE_NEOX = 16;
constexpr uint32_t ROPE_MAX_DIM = 512;  // largest hd / hdv the fused kernel stages per wave

// Benchmark timing: a launch may carry a start / stop event pair that its own dispatch records
// (hipExtLaunchKernel), so the measured interval is the kernel alone, without event packets queued
// around it. Null events: an ordinary launch. A pair of launches bracketed by one pair of events
// passes the start to the first launch and the stop to the second (either may be null alone).
struct LaunchEv {
  hipEvent_t start = nullptr, stop = nullptr;
};
#define LMH_LAUNCH(ev, kernel, grid, block, lds, stream, ...)                                             \
  do {                                                                                                    \
    if ((ev).start || (ev).stop)                                                                          \
      hipExtLaunchKernelGGL(kernel, grid, block, lds, stream, (ev).start, (ev).stop, 0u, __VA_ARGS__);     \
    else                                                                                                  \
      hipLaunchKernelGGL(kernel, grid, block, lds, stream, __VA_ARGS__);                                  \
  } while (0)

// Launch wrappers (defined in the .hip files). Return hipSuccess or the launch error.
hipError_t launch_store_f32(const PageGeom& g, const int32_t* row_seq, const int32_t* row_pos, uint32_t n_rows,
                            const float* k, const float* v, hipStream_t s);
hipError_t launch_store_encoded(const PageGeom& g, const int32_t* row_seq, const int32_t* row_pos,
                                uint32_t n_rows, const uint8_t* k, const uint8_t* v, uint32_t k_row,
                                uint32_t v_row, hipStream_t s);
hipError_t launch_gather(const PageGeom& g, const int32_t* row_seq, const int32_t* row_pos, uint32_t n_rows,
                         float* k, float* v, hipStream_t s);
hipError_t launch_gather_encoded(const PageGeom& g, const int32_t* row_seq, const int32_t* row_pos,
                                 uint32_t n_rows, uint8_t* k, uint8_t* v, uint32_t k_row, uint32_t v_row,
                                 hipStream_t s);
hipError_t launch_qk_rope_store(const PageGeom& g, const RopeGeom& r, const int32_t* row_seq, const int32_t* row_pos,
                                uint32_t n_rows, const float* q, const float* k, const float* v, float* q_out,
                                const int32_t* quads, uint32_t n_quads, const int32_t* rest, uint32_t n_rest,
                                hipStream_t s, const LaunchEv& ev = {});
// One layer's share of a sequence's snapshot (write: pages -> reference block format; read: the
// reverse), positions 0 .. n_pos-1.
hipError_t launch_snapshot(bool write, const PageGeom& g, uint32_t seq, uint32_t n_pos, uint32_t bt, uint64_t bb,
                           uint64_t ref_off, uint32_t k_row, uint32_t v_row, uint8_t* bytes, hipStream_t s);
hipError_t launch_zero_blocks(uint8_t* pool, uint64_t block_bytes, const int32_t* blocks, uint32_t n,
                              hipStream_t s);
// n words from src (host-mapped staging memory) to dst (device memory), as a kernel on s
hipError_t launch_copy_words(uint32_t* dst, const uint32_t* src, uint64_t n, hipStream_t s);
// benchmark hook: one streaming read of `bytes` (a multiple of 16) at p
hipError_t launch_read_ceiling(const uint8_t* p, uint64_t bytes, uint32_t* sink, hipStream_t s, const LaunchEv& ev);
// Returns hipErrorInvalidValue for a (type, hd, hdv) with no kernel instance.
// The merge list of the call (src: staged, host-mapped; dst: device memory), copied by the decode
// launch for the merge kernel that follows it (n_words = 0: nothing to copy).
struct MergeCopy {
  const uint32_t* src;
  uint32_t* dst;
  uint32_t n_words;
};
hipError_t launch_decode(const PageGeom& g, const RowGeom& r, const DecodeItem* items, uint32_t n_items,
                         const float* q, float* out, float* part, const MergeCopy& mc, hipStream_t s,
                         const LaunchEv& ev = {});
// items: n_pf prompt-token merges (nh != 0, n_split <= 64) first, then the decode merges;
// max_pf_rows: the largest nh * n_split of the prompt merges; max_split: the largest n_split of the
// decode merges (over 16: rows loaded in groups of 16)
hipError_t launch_merge(const RowGeom& r, uint32_t hdv, const MergeItem* items, uint32_t n_items, uint32_t n_pf,
                        uint32_t max_pf_rows, const float* part, float* out, uint32_t max_split, hipStream_t s,
                        const LaunchEv& ev = {});
// The device scratch of lmh_attend_noalloc (split-K partials, then the merge list): its size, and
// the address of `device`'s copy (call with that device current; resolved once per device).
constexpr size_t NOALLOC_SCRATCH_BYTES = size_t(32) << 20;
hipError_t noalloc_scratch(int device, uint8_t** out);
// Decode work items (waves) one CU holds at once for a layer's decode kernel (occupancy query).
// The instance a launch picks depends on the group for f32 pages and on the layout.
uint32_t decode_waves_per_cu(uint32_t kv_type, uint32_t hd, uint32_t hdv, uint32_t group, uint32_t layout);
// Whether (type, hd, hdv) has a tile-layout decode instance (matrix-core, or f32 VALU); every
// other geometry up to 512 wide takes the row layout and its VALU kernel.
bool decode_tiles_supported(uint32_t kv_type, uint32_t hd, uint32_t hdv);
// Query heads per work item the row-layout kernel takes (its items use ng <= this).
uint32_t decode_rows_max_heads();
// f32 decode: the calls whose split rows may merge inside their workgroup (tile layout instances).
bool decode_local_merge_ok(uint32_t hd, uint32_t hdv, uint32_t group);
// matrix-core decode (f16 / bf16 / q8_0 pages): an instance whose split rows (up to 4 items, the
// waves of one workgroup) merge inside their workgroup
bool decode_mfma_local_ok(uint32_t kv_type, uint32_t hd, uint32_t hdv);

// Prefill (multi-token segments on matrix cores): n_wg workgroups, workgroup b runs the units
// items[b * per_wg ..] up to the first with n_tok == 0. `max_pages` bounds the key pages of any unit.
hipError_t launch_prefill(const PageGeom& g, const PrefillGeom& pg, const PrefillItem* items, uint32_t n_wg,
                          uint32_t per_wg, uint32_t max_pages, const float* q, float* out, const MergeCopy& mc,
                          hipStream_t s, const LaunchEv& ev = {});
bool prefill_supported(uint32_t kv_type, uint32_t hd, uint32_t hdv, uint32_t group);
// A call holding both prefill units and decode items, in one launch (any type and head size
// prefill_supported accepts): pf_wg prefill workgroups, then the decode items eight per workgroup.
hipError_t launch_mixed(const PageGeom& g, const PrefillGeom& pg, const PrefillItem* pitems, uint32_t pf_wg,
                        uint32_t per_wg, uint32_t max_pages, const RowGeom& r, const DecodeItem* items,
                        uint32_t n_items, const float* q, float* out, float* part, const MergeCopy& mc,
                        hipStream_t s, const LaunchEv& ev = {});
uint32_t prefill_wg_per_cu();     // prefill workgroups a CU holds when their LDS fits (160 KiB / this)
uint32_t prefill_cols_per_unit();
// LDS the prefill kernels declare statically, beside prefill_lds_bytes() of dynamic LDS
size_t prefill_static_lds_bytes();
size_t prefill_lds_bytes(uint32_t kv_type, uint32_t hd, uint32_t max_pages, uint32_t per_wg);

}  // namespace lmh
