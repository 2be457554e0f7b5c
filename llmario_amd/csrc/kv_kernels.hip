// kv_kernels.hip — paged KV writes, reads and block zeroing on gfx950.
//
// store:   KvCache::store_k / store_v (crates/engine/model/src/kv.rs:870-889) for a batch of
//          rows: f32 in, encoded as the cache type (KvType::store, kv.rs:112-126), scattered to
//          the row's (block, tile, slot) through the block table (BlockTable::locate,
//          kv/src/lib.rs:243-253).
// encoded: the same rows given in the reference's row encoding (f16/bf16 bits, f32, q8_0
//          34-byte blocks), transcoded into the page layout; the inverse read gives the bytes back.
// gather:  LayerReader::row + KvType::load (kv.rs:1166-1179, 131-151) decoded to f32.
// producer: the per-row tail of attention_block (forward.rs:427-453): QK-norm and RoPE of Q and K
//          in place, then K and V stored as above, in one launch (qk_rope_store_*: per row, or per
//          aligned run of 4 tokens and share of the heads for 16-bit caches).
// snapshot: KvCache::write_seq / read_seq (kv.rs:1030-1130), one sequence's pages to and from the
//          reference's byte format.
// Also: zeroing of newly backed blocks, and two benchmark / staging helpers (a plain streaming
// read, and a word copy on the caller's stream).
//
// store / gather: one workgroup per row; like the rest they move bytes and are HBM-bound.
#include "device.h"

#include <algorithm>

namespace lmh {
namespace {

struct Slot {
  uint8_t* base;  // block base + layer offset handled by callers
  uint32_t tile, m;
};

__device__ inline Slot locate(const PageGeom& g, int seq, uint32_t pos) {
  const int blk = g.table[(size_t)seq * g.bps + (pos >> g.bt_shift)];
  const uint32_t in_blk = pos & ((1u << g.bt_shift) - 1u);
  Slot s;
  s.base = g.pool + (size_t)blk * g.block_bytes;
  s.tile = in_blk >> 4;
  s.m = in_blk & 15u;
  return s;
}

// f32 -> f16, round to nearest even (v_cvt_f16_f32 under the default rounding mode).
__device__ inline uint16_t f16_bits(float x) {
  _Float16 h = (_Float16)x;
  return __builtin_bit_cast(uint16_t, h);
}
__device__ inline float f16_val(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
// f32 -> bf16, round to nearest even on the dropped 16 bits (NaN kept quiet).
__device__ inline uint16_t bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ inline float bf16_val(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// Byte offset of element (m, d) of a tile, for one side (K or V), in the tile layout (layout 0)
// or the row layout (layout 1: row-major codes of the type's width).
__device__ inline uint32_t elem_off(uint32_t type, bool is_v, uint32_t m, uint32_t d, uint32_t dim,
                                    uint32_t layout = LAYOUT_TILES) {
  if (layout == LAYOUT_ROWS) return (m * dim + d) * (type == KV_F32 ? 4u : type == KV_Q8 ? 1u : 2u);
  switch (type) {
    case KV_F16:
    case KV_BF16: return is_v ? v16_off(m, d) : k16_off(m, d);
    case KV_Q8: return is_v ? vq8_off(m, d) : kq8_off(m, d);
    default: return (m * dim + d) * 4u;
  }
}

struct Side {
  uint32_t off, head, tile, scale, tile_s, dim;
};
__device__ inline Side side(const PageGeom& g, bool is_v) {
  Side s;
  s.off = is_v ? g.v_off : g.k_off;
  s.head = is_v ? g.v_head : g.k_head;
  s.tile = is_v ? g.v_tile : g.k_tile;
  s.scale = is_v ? g.v_scale : g.k_scale;
  s.tile_s = is_v ? g.v_tile_s : g.k_tile_s;
  s.dim = is_v ? g.hdv : g.hd;
  return s;
}

// Encode one row side (n_kv*dim values starting at src) into its pages. Threads stride over the
// elements in steps of blockDim.x (a multiple of 32), so a q8_0 block of 32 values is one half
// wave and its amax is a 32-lane reduction.
__device__ void store_side(const PageGeom& g, const Slot& sl, bool is_v, const float* src) {
  const Side sd = side(g, is_v);
  const uint32_t n = g.n_kv * sd.dim;
  for (uint32_t e = threadIdx.x; e < n; e += blockDim.x) {
    const uint32_t h = e / sd.dim, d = e % sd.dim;
    uint8_t* head = sl.base + sd.off + h * sd.head;
    const float x = src[e];
    const uint32_t o = sl.tile * sd.tile + elem_off(g.kv_type, is_v, sl.m, d, sd.dim, g.layout);
    switch (g.kv_type) {
      case KV_F16: *(uint16_t*)(head + o) = f16_bits(x); break;
      case KV_BF16: *(uint16_t*)(head + o) = bf16_bits(x); break;
      case KV_F32: *(float*)(head + o) = x; break;
      case KV_Q8: {
        // quantize_q8_0 (kv.rs:156-171): d = amax/127, id = d ? 1/d : 0, q = round_ties_even(x*id)
        float amax = fabsf(x);
        for (int w = 16; w >= 1; w >>= 1) amax = fmaxf(amax, __shfl_xor(amax, w, 32));
        const float dsc = amax / 127.0f;
        const float id = dsc != 0.0f ? 1.0f / dsc : 0.0f;
        const float r = rintf(x * id);
        head[o] = (uint8_t)(int8_t)(int32_t)r;
        if ((d & 31u) == 0) {
          uint8_t* sp = head + sd.scale + sl.tile * sd.tile_s + (sl.m * (sd.dim >> 5) + (d >> 5)) * 2u;
          *(uint16_t*)sp = f16_bits(dsc);
        }
        break;
      }
    }
  }
}

__global__ void store_f32_kernel(PageGeom g, const int32_t* row_seq, const int32_t* row_pos, const float* k,
                                 const float* v) {
  const uint32_t row = blockIdx.x;
  const Slot sl = locate(g, row_seq[row], (uint32_t)row_pos[row]);
  store_side(g, sl, false, k + (size_t)row * g.n_kv * g.hd);
  store_side(g, sl, true, v + (size_t)row * g.n_kv * g.hdv);
}

// ---- fused per-row tail of attention_block (forward.rs:427-453; Metal qk_rope_kv_t,
// misc.metal:195-273): per-head RMS norm, RoPE, Q written out, K and V stored into the pages.

// Encode head h of one row side from the wave's staged values x[0 .. dim) into its page slot.
// Lane L handles elements L, L+64, ...: a q8_0 block of 32 values is one half wave.
__device__ void store_head_wave(const PageGeom& g, const Slot& sl, bool is_v, uint32_t h, const float* x,
                                uint32_t lane) {
  const Side sd = side(g, is_v);
  uint8_t* head = sl.base + sd.off + h * sd.head;
  for (uint32_t d = lane; d < sd.dim; d += 64) {
    const float v = x[d];
    const uint32_t o = sl.tile * sd.tile + elem_off(g.kv_type, is_v, sl.m, d, sd.dim, g.layout);
    switch (g.kv_type) {
      case KV_F16: *(uint16_t*)(head + o) = f16_bits(v); break;
      case KV_BF16: *(uint16_t*)(head + o) = bf16_bits(v); break;
      case KV_F32: *(float*)(head + o) = v; break;
      case KV_Q8: {
        // quantize_q8_0 (kv.rs:156-171)
        float amax = fabsf(v);
        for (int w = 16; w >= 1; w >>= 1) amax = fmaxf(amax, __shfl_xor(amax, w, 32));
        const float dsc = amax / 127.0f;
        const float id = dsc != 0.0f ? 1.0f / dsc : 0.0f;
        head[o] = (uint8_t)(int8_t)(int32_t)rintf(v * id);
        if ((d & 31u) == 0) {
          uint8_t* sp = head + sd.scale + sl.tile * sd.tile_s + (sl.m * (sd.dim >> 5) + (d >> 5)) * 2u;
          *(uint16_t*)sp = f16_bits(dsc);
        }
        break;
      }
    }
  }
}

// The wave's LDS writes are complete and visible to its other lanes (LDS executes one wave's
// accesses in order; this also keeps the compiler from moving LDS accesses across it).
__device__ inline void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Encode head h from per-lane values: lane L holds elements L*VPL .. L*VPL+VPL-1 (dim = 64*VPL).
// f16/bf16 K: the VPL values are consecutive bytes of one 16-byte operand row (VPL <= 8), one
// store; V and f32: per element. q8_0: a block of 32 values spans 32/VPL lanes (amax over them).
template <int VPL>
__device__ void store_head_lanes(const PageGeom& g, const Slot& sl, bool is_v, uint32_t h, const float (&x)[VPL],
                                 uint32_t lane) {
  const Side sd = side(g, is_v);
  uint8_t* head = sl.base + sd.off + h * sd.head + sl.tile * sd.tile;
  const uint32_t d0 = lane * VPL;
  switch (g.kv_type) {
    case KV_F16:
    case KV_BF16: {
      uint16_t b[VPL];
#pragma unroll
      for (int c = 0; c < VPL; c++) b[c] = g.kv_type == KV_F16 ? f16_bits(x[c]) : bf16_bits(x[c]);
      if (!is_v && VPL >= 2) {
        uint8_t* dst = head + k16_off(sl.m, d0);
        if constexpr (VPL == 2) *(uint32_t*)dst = b[0] | ((uint32_t)b[1] << 16);
        else {
#pragma unroll
          for (int c = 0; c < VPL; c += 2) *(uint32_t*)(dst + 2 * c) = b[c] | ((uint32_t)b[c + 1] << 16);
        }
      } else {
#pragma unroll
        for (int c = 0; c < VPL; c++) *(uint16_t*)(head + elem_off(g.kv_type, is_v, sl.m, d0 + c, sd.dim, g.layout)) = b[c];
      }
      break;
    }
    case KV_F32: {
#pragma unroll
      for (int c = 0; c < VPL; c++) *(float*)(head + elem_off(KV_F32, is_v, sl.m, d0 + c, sd.dim, g.layout)) = x[c];
      break;
    }
    case KV_Q8: {
      // quantize_q8_0 (kv.rs:156-171) over blocks of 32 values = 32/VPL lanes
      float amax = 0.f;
#pragma unroll
      for (int c = 0; c < VPL; c++) amax = fmaxf(amax, fabsf(x[c]));
      for (int m = 16 / VPL; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m));
      const float dsc = amax / 127.0f;
      const float id = dsc != 0.0f ? 1.0f / dsc : 0.0f;
#pragma unroll
      for (int c = 0; c < VPL; c++) head[elem_off(KV_Q8, is_v, sl.m, d0 + c, sd.dim, g.layout)] = (uint8_t)(int8_t)(int32_t)rintf(x[c] * id);
      if ((d0 & 31u) == 0) {
        uint8_t* sp = sl.base + sd.off + h * sd.head + sd.scale + sl.tile * sd.tile_s + (sl.m * (sd.dim >> 5) + (d0 >> 5)) * 2u;
        *(uint16_t*)sp = f16_bits(dsc);
      }
      break;
    }
  }
}

__device__ inline float wave_sum(float x) {
#pragma unroll
  for (int w = 32; w >= 1; w >>= 1) x += __shfl_xor(x, w);
  return x;
}

// One workgroup (4 waves) per row. The row's heads (Q, then K, then V; hd == hdv) are pulled into
// LDS in chunks of up to ROPE_LDS_FLOATS floats with 16-byte loads spread over all threads, so one
// round trip fetches a whole row. Meanwhile the rotation factors are computed once per row: the
// angle in f32 exactly as the reference forms it (pos * freq_scale * freq), its sine and cosine in
// double and rounded (so they match a correctly rounded sinf/cosf), scaled by attn_factor. Each
// wave then takes whole heads from LDS: RMS norm (rms_norm: y = x * (1/sqrt(ss/n + eps)) * w),
// rotation of its pairs (disjoint, so lanes never read what another writes), and the output (Q as
// f32 rows, K and V encoded into their page slot).
constexpr uint32_t ROPE_LDS_FLOATS = 8192;  // 32 KiB of staged head values per workgroup
__global__ __launch_bounds__(256) void qk_rope_store_kernel(PageGeom g, RopeGeom r, const int32_t* row_seq,
                                                            const int32_t* row_pos, const float* q, const float* k,
                                                            const float* v, float* q_out) {
  __shared__ float2 cs[ROPE_MAX_DIM / 2];
  __shared__ float wq[ROPE_MAX_DIM], wk[ROPE_MAX_DIM];
  __shared__ __attribute__((aligned(16))) float buf[ROPE_LDS_FLOATS];
  const uint32_t row = blockIdx.x, tid = threadIdx.x;
  const uint32_t pos = (uint32_t)row_pos[row];
  const uint32_t hd = g.hd, f4 = hd / 4;  // float4s per head
  const uint32_t n_items = r.n_head + 2 * g.n_kv, per_chunk = ROPE_LDS_FLOATS / hd;
  const uint32_t w = tid >> 6, lane = tid & 63u;
  auto src_of = [&](uint32_t it) -> const float* {
    if (it < r.n_head) return q + ((size_t)row * r.n_head + it) * r.q_stride;
    if (it < r.n_head + g.n_kv) return k + ((size_t)row * g.n_kv + it - r.n_head) * hd;
    return v + ((size_t)row * g.n_kv + it - r.n_head - g.n_kv) * hd;
  };
  Slot sl;  // the row's page slot, looked up once the first loads are in flight
  const bool neox = (r.flags & ROPE_NEOX) != 0;
  // A chunk is at most ROPE_LDS_FLOATS / 4 float4s: LPT per thread, all requested before any is
  // written to LDS (one round trip per chunk); the first chunk's loads overlap the set-up.
  constexpr uint32_t LPT = ROPE_LDS_FLOATS / 4 / 256;
  for (uint32_t i0 = 0; i0 < n_items; i0 += per_chunk) {
    const uint32_t n = min(n_items - i0, per_chunk);
    if (i0 > 0) __syncthreads();  // every wave is done with the previous chunk
    float4 tmp[LPT];
#pragma clang loop unroll(full)
    for (uint32_t u = 0; u < LPT; u++) {
      const uint32_t f = tid + u * 256;
      const bool live = f < n * f4;
      const float* p = src_of(i0 + (live ? f / f4 : 0)) + (live ? 4 * (f % f4) : 0);
      tmp[u] = live ? *(const float4*)p : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (i0 == 0) {
      sl = locate(g, row_seq[row], pos);
      for (uint32_t i = tid; i < r.half_rot; i += blockDim.x) {
        float angle = (float)pos * r.freq_scale * r.freq[i];
        if (r.freq_div) angle = angle / r.freq_div[i];
        double sn, cn;
        sincos((double)angle, &sn, &cn);
        cs[i] = make_float2((float)cn * r.attn_factor, (float)sn * r.attn_factor);
      }
      for (uint32_t d = tid; d < hd; d += blockDim.x) {
        wq[d] = r.q_norm ? r.q_norm[d] : 1.0f;
        wk[d] = r.k_norm ? r.k_norm[d] : 1.0f;
      }
    }
#pragma clang loop unroll(full)
    for (uint32_t u = 0; u < LPT; u++) {
      const uint32_t f = tid + u * 256;
      if (f < n * f4) *(float4*)(buf + 4 * f) = tmp[u];
    }
    __syncthreads();
    for (uint32_t j = w; j < n; j += 4) {
      const uint32_t it = i0 + j;
      const bool is_q = it < r.n_head, is_v = it >= r.n_head + g.n_kv;
      const bool norm = is_q ? (r.flags & ROPE_Q_NORM) != 0
                             : is_v ? (r.flags & ROPE_V_NORM) != 0 : (r.flags & ROPE_K_NORM) != 0;
      float* x = buf + (size_t)j * hd;
      if (norm) {
        float ss = 0.f;
        for (uint32_t d = lane; d < hd; d += 64) ss += x[d] * x[d];
        const float scale = 1.0f / sqrtf(wave_sum(ss) / (float)hd + r.eps);
        const float* nw = is_q ? wq : wk;
        for (uint32_t d = lane; d < hd; d += 64) x[d] = is_v ? x[d] * scale : x[d] * scale * nw[d];
        wave_lds_sync();
      }
      if (!is_v && r.half_rot) {
        for (uint32_t i = lane; i < r.half_rot; i += 64) {
          const uint32_t a = neox ? i : 2 * i, b = neox ? i + r.half_rot : 2 * i + 1;
          const float2 c = cs[i];
          const float x0 = x[a], x1 = x[b];
          x[a] = x0 * c.x - x1 * c.y;
          x[b] = x0 * c.y + x1 * c.x;
        }
        wave_lds_sync();
      }
      if (is_q) {
        float4* dst = (float4*)(q_out + ((size_t)row * r.n_head + it) * hd);
        for (uint32_t o = lane; o < f4; o += 64) dst[o] = *(const float4*)(x + 4 * o);
      } else {
        store_head_wave(g, sl, is_v, is_v ? it - r.n_head - g.n_kv : it - r.n_head, x, lane);
      }
    }
  }
}

// Register fast path of the same computation, for hd == hdv = 64*VPL and a rotated fraction that
// keeps pair partners a power-of-two lane distance apart (rot_dim*32/hd a power of two, or no
// rotation): lane L holds elements L*VPL .. L*VPL+VPL-1 of a head, so a head is one vector load
// per lane, the RMS norm a wave reduction, and a pair partner sits in the same lane (Normal, VPL >=
// 2) or in lane L ^ m (Neox: m = rot_dim*32/hd; Normal with VPL == 1: m = 1). Each wave loads all
// its heads of a group before processing any (one round trip per group). The rotation factors are
// computed once per row in f32 (sincosf, correctly range-reduced; within an ulp of the
// reference's sinf/cosf) and read by each lane once.
template <int VPL>
__global__ __launch_bounds__(256) void qk_rope_store_reg_kernel(PageGeom g, RopeGeom r, const int32_t* row_seq,
                                                                const int32_t* row_pos, const float* q, const float* k,
                                                                const float* v, float* q_out) {
  constexpr uint32_t HD = 64 * VPL;
  constexpr int GRP = 16;  // heads a wave requests before processing them
  typedef float fv __attribute__((ext_vector_type(VPL)));
  __shared__ float2 cs[ROPE_MAX_DIM / 2];
  const uint32_t row = blockIdx.x, tid = threadIdx.x, w = tid >> 6, lane = tid & 63u;
  const uint32_t pos = (uint32_t)row_pos[row];
  const uint32_t n_items = r.n_head + 2 * g.n_kv;
  auto src_of = [&](uint32_t it) -> const float* {
    if (it < r.n_head) return q + ((size_t)row * r.n_head + it) * r.q_stride;
    if (it < r.n_head + g.n_kv) return k + ((size_t)row * g.n_kv + it - r.n_head) * HD;
    return v + ((size_t)row * g.n_kv + it - r.n_head - g.n_kv) * HD;
  };
  // first group's heads in flight before anything else
  fv xs[GRP];
#pragma unroll
  for (int j = 0; j < GRP; j++) {
    const uint32_t it = w + 4 * j;
    xs[j] = it < n_items ? *(const fv*)(src_of(it) + lane * VPL) : fv{};
  }
  for (uint32_t i = tid; i < r.half_rot; i += blockDim.x) {
    float angle = (float)pos * r.freq_scale * r.freq[i];
    if (r.freq_div) angle = angle / r.freq_div[i];
    float sn, cn;
    sincosf(angle, &sn, &cn);
    cs[i] = make_float2(cn * r.attn_factor, sn * r.attn_factor);
  }
  const Slot sl = locate(g, row_seq[row], pos);
  fv wq, wk;
#pragma unroll
  for (int c = 0; c < VPL; c++) {
    wq[c] = r.q_norm ? r.q_norm[lane * VPL + c] : 1.0f;
    wk[c] = r.k_norm ? r.k_norm[lane * VPL + c] : 1.0f;
  }
  __syncthreads();
  // this lane's rotation factor per element, and whether the element is the pair's first
  const bool neox = (r.flags & ROPE_NEOX) != 0;
  const uint32_t half = r.half_rot;
  const uint32_t pmask = neox ? half / VPL : 1;  // lane distance to the partner when not in-lane
  float2 cf[VPL];
  bool first[VPL], rot[VPL];
#pragma unroll
  for (int c = 0; c < VPL; c++) {
    const uint32_t e = lane * VPL + c;
    rot[c] = e < 2 * half;
    first[c] = neox ? e < half : (e & 1) == 0;
    const uint32_t i = neox ? (e < half ? e : e - half) : e >> 1;
    cf[c] = rot[c] ? cs[i] : make_float2(1.f, 0.f);
  }
  for (uint32_t g0 = 0; g0 * 4 < n_items; g0 += GRP) {
    if (g0 > 0) {
#pragma unroll
      for (int j = 0; j < GRP; j++) {
        const uint32_t it = w + 4 * (g0 + j);
        xs[j] = it < n_items ? *(const fv*)(src_of(it) + lane * VPL) : fv{};
      }
    }
#pragma unroll
    for (int j = 0; j < GRP; j++) {
      const uint32_t it = w + 4 * (g0 + j);
      if (it >= n_items) continue;
      const bool is_q = it < r.n_head, is_v = it >= r.n_head + g.n_kv;
      const bool norm = is_q ? (r.flags & ROPE_Q_NORM) != 0
                             : is_v ? (r.flags & ROPE_V_NORM) != 0 : (r.flags & ROPE_K_NORM) != 0;
      fv x = xs[j];
      if (norm) {
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < VPL; c++) ss += x[c] * x[c];
        const float scale = 1.0f / sqrtf(wave_sum(ss) / (float)HD + r.eps);
        const fv nw = is_q ? wq : wk;
#pragma unroll
        for (int c = 0; c < VPL; c++) x[c] = is_v ? x[c] * scale : x[c] * scale * nw[c];
      }
      if (!is_v && half) {
        fv p;  // each element's pair partner
#pragma unroll
        for (int c = 0; c < VPL; c++) {
          if (neox || VPL == 1)
            p[c] = __shfl_xor(x[c], (int)pmask);
          else
            p[c] = x[c ^ 1];
        }
#pragma unroll
        for (int c = 0; c < VPL; c++) {
          if (!rot[c]) continue;
          // (x0, x1) = (x[a], x[b]): x[a] = x0 cos - x1 sin, x[b] = x0 sin + x1 cos
          x[c] = first[c] ? x[c] * cf[c].x - p[c] * cf[c].y : p[c] * cf[c].y + x[c] * cf[c].x;
        }
      }
      if (is_q) {
        __builtin_nontemporal_store(x, (fv*)(q_out + ((size_t)row * r.n_head + it) * HD + lane * VPL));
      } else {
        float xa[VPL];
#pragma unroll
        for (int c = 0; c < VPL; c++) xa[c] = x[c];
        store_head_lanes<VPL>(g, sl, is_v, is_v ? it - r.n_head - g.n_kv : it - r.n_head, xa, lane);
      }
    }
  }
}

// Reference row encoding -> page layout (bit copy, no re-rounding).
__device__ void store_enc_side(const PageGeom& g, const Slot& sl, bool is_v, const uint8_t* src) {
  const Side sd = side(g, is_v);
  const uint32_t n = g.n_kv * sd.dim;
  for (uint32_t e = threadIdx.x; e < n; e += blockDim.x) {
    const uint32_t h = e / sd.dim, d = e % sd.dim;
    uint8_t* head = sl.base + sd.off + h * sd.head;
    const uint32_t o = sl.tile * sd.tile + elem_off(g.kv_type, is_v, sl.m, d, sd.dim, g.layout);
    switch (g.kv_type) {
      case KV_F16:
      case KV_BF16: *(uint16_t*)(head + o) = (uint16_t)(src[2 * e] | (src[2 * e + 1] << 8)); break;
      case KV_F32: {
        uint32_t u = src[4 * e] | (src[4 * e + 1] << 8) | (src[4 * e + 2] << 16) | ((uint32_t)src[4 * e + 3] << 24);
        *(uint32_t*)(head + o) = u;
        break;
      }
      case KV_Q8: {
        const uint8_t* blk = src + (e >> 5) * 34u;
        head[o] = blk[2 + (e & 31u)];
        if ((d & 31u) == 0) {
          uint8_t* sp = head + sd.scale + sl.tile * sd.tile_s + (sl.m * (sd.dim >> 5) + (d >> 5)) * 2u;
          *(uint16_t*)sp = (uint16_t)(blk[0] | (blk[1] << 8));
        }
        break;
      }
    }
  }
}

__global__ void store_encoded_kernel(PageGeom g, const int32_t* row_seq, const int32_t* row_pos, const uint8_t* k,
                                     const uint8_t* v, uint32_t k_row, uint32_t v_row) {
  const uint32_t row = blockIdx.x;
  const Slot sl = locate(g, row_seq[row], (uint32_t)row_pos[row]);
  store_enc_side(g, sl, false, k + (size_t)row * k_row);
  store_enc_side(g, sl, true, v + (size_t)row * v_row);
}

__device__ float load_elem(const PageGeom& g, const Slot& sl, bool is_v, uint32_t e) {
  const Side sd = side(g, is_v);
  const uint32_t h = e / sd.dim, d = e % sd.dim;
  const uint8_t* head = sl.base + sd.off + h * sd.head;
  const uint32_t o = sl.tile * sd.tile + elem_off(g.kv_type, is_v, sl.m, d, sd.dim, g.layout);
  switch (g.kv_type) {
    case KV_F16: return f16_val(*(const uint16_t*)(head + o));
    case KV_BF16: return bf16_val(*(const uint16_t*)(head + o));
    case KV_F32: return *(const float*)(head + o);
    default: {
      // dequantize_q8_0 (kv.rs:174-184): (q as i8) as f32 * d, exact in f32
      const uint8_t* sp = head + sd.scale + sl.tile * sd.tile_s + (sl.m * (sd.dim >> 5) + (d >> 5)) * 2u;
      return (float)(int8_t)head[o] * f16_val(*(const uint16_t*)sp);
    }
  }
}

__global__ void gather_kernel(PageGeom g, const int32_t* row_seq, const int32_t* row_pos, float* k, float* v) {
  const uint32_t row = blockIdx.x;
  const Slot sl = locate(g, row_seq[row], (uint32_t)row_pos[row]);
  const uint32_t nk = g.n_kv * g.hd, nv = g.n_kv * g.hdv;
  for (uint32_t e = threadIdx.x; e < nk; e += blockDim.x) k[(size_t)row * nk + e] = load_elem(g, sl, false, e);
  for (uint32_t e = threadIdx.x; e < nv; e += blockDim.x) v[(size_t)row * nv + e] = load_elem(g, sl, true, e);
}

__device__ void gather_enc_side(const PageGeom& g, const Slot& sl, bool is_v, uint8_t* dst) {
  const Side sd = side(g, is_v);
  const uint32_t n = g.n_kv * sd.dim;
  for (uint32_t e = threadIdx.x; e < n; e += blockDim.x) {
    const uint32_t h = e / sd.dim, d = e % sd.dim;
    const uint8_t* head = sl.base + sd.off + h * sd.head;
    const uint32_t o = sl.tile * sd.tile + elem_off(g.kv_type, is_v, sl.m, d, sd.dim, g.layout);
    switch (g.kv_type) {
      case KV_F16:
      case KV_BF16: {
        const uint16_t b = *(const uint16_t*)(head + o);
        dst[2 * e] = (uint8_t)b;
        dst[2 * e + 1] = (uint8_t)(b >> 8);
        break;
      }
      case KV_F32: {
        const uint32_t u = *(const uint32_t*)(head + o);
        for (int i = 0; i < 4; i++) dst[4 * e + i] = (uint8_t)(u >> (8 * i));
        break;
      }
      case KV_Q8: {
        uint8_t* blk = dst + (e >> 5) * 34u;
        blk[2 + (e & 31u)] = head[o];
        if ((d & 31u) == 0) {
          const uint8_t* sp = head + sd.scale + sl.tile * sd.tile_s + (sl.m * (sd.dim >> 5) + (d >> 5)) * 2u;
          blk[0] = sp[0];
          blk[1] = sp[1];
        }
        break;
      }
    }
  }
}

__global__ void gather_encoded_kernel(PageGeom g, const int32_t* row_seq, const int32_t* row_pos, uint8_t* k,
                                      uint8_t* v, uint32_t k_row, uint32_t v_row) {
  const uint32_t row = blockIdx.x;
  const Slot sl = locate(g, row_seq[row], (uint32_t)row_pos[row]);
  gather_enc_side(g, sl, false, k + (size_t)row * k_row);
  gather_enc_side(g, sl, true, v + (size_t)row * v_row);
}

// ---- snapshots (KvCache::write_seq / read_seq, kv.rs:1030-1130): one layer's share of a
// sequence's blocks in the reference's block format. Snapshot block i is the sequence's block i;
// inside it, the layer's K rows then V rows (ref_off + slot*k_row, ref_off + bt*k_row + slot*v_row)
// in the row encoding. One workgroup per position of the covered blocks (every slot, written or
// not, so the bytes equal the reference's block byte for byte).
__global__ void snapshot_write_kernel(PageGeom g, uint32_t seq, uint32_t bt, uint64_t bb, uint64_t ref_off,
                                      uint32_t k_row, uint32_t v_row, uint8_t* out) {
  const uint32_t p = blockIdx.x, bi = p / bt, j = p % bt;
  const Slot sl = locate(g, (int)seq, p);
  uint8_t* blk = out + (size_t)bi * bb + ref_off;
  gather_enc_side(g, sl, false, blk + (size_t)j * k_row);
  gather_enc_side(g, sl, true, blk + (size_t)bt * k_row + (size_t)j * v_row);
}
__global__ void snapshot_read_kernel(PageGeom g, uint32_t seq, uint32_t bt, uint64_t bb, uint64_t ref_off,
                                     uint32_t k_row, uint32_t v_row, const uint8_t* in) {
  const uint32_t p = blockIdx.x, bi = p / bt, j = p % bt;
  const Slot sl = locate(g, (int)seq, p);
  const uint8_t* blk = in + (size_t)bi * bb + ref_off;
  store_enc_side(g, sl, false, blk + (size_t)j * k_row);
  store_enc_side(g, sl, true, blk + (size_t)bt * k_row + (size_t)j * v_row);
}

// Tiled form (used when every head's row segment is a whole number of 4-byte words): one
// workgroup per (snapshot block, 16-token tile, KV head, side). The page tile (and its q8_0
// scales) and the tile's 16 row segments (head h of rows t*16 .. t*16+15, h*seg bytes into each
// row) are staged in LDS; bytes are remapped between the two layouts there, so HBM sees 16-byte
// accesses on the page side and 4-byte accesses running along each row segment.

// Four consecutive tokens of one sequence, aligned to 4 positions (so they share a 16-token tile
// and, in the V tile, one 8-byte run per dimension: v16_off interleaves 4 keys), per workgroup:
// the f16 / bf16 rows of a prefill chunk. Each wave takes whole heads for all four tokens; K goes
// out as in the row kernel (per token), V as one 8-byte store per dimension carrying the four
// tokens' values, where the row kernel writes 2-byte pieces. NT = 1 is the same work for one row
// (a decode row or a chunk's unaligned edge), V written per element as in the row kernel.
// Items it0 .. n_items-1 of [Q heads][K heads][V heads] are the workgroup's share.
template <int VPL, int NT>
__device__ void rope_tokens(const PageGeom& g, const RopeGeom& r, float2 (*cs)[ROPE_MAX_DIM / 2], uint32_t row0,
                            uint32_t it0, uint32_t n_items, const int32_t* row_seq, const int32_t* row_pos,
                            const float* q, const float* k, const float* v, float* q_out) {
  constexpr uint32_t HD = 64 * VPL;
  constexpr int GRP = 2;  // heads (x 4 tokens) a wave requests before processing them (more heads
                          // cost occupancy: 2 keeps the kernel at 4 waves per SIMD)
  typedef float fv __attribute__((ext_vector_type(VPL)));
  const uint32_t tid = threadIdx.x, w = tid >> 6, lane = tid & 63u;
  const uint32_t pos0 = (uint32_t)row_pos[row0];
  auto src_of = [&](uint32_t it, uint32_t t) -> const float* {
    const size_t row = row0 + t;
    if (it < r.n_head) return q + (row * r.n_head + it) * r.q_stride;
    if (it < r.n_head + g.n_kv) return k + (row * g.n_kv + it - r.n_head) * HD;
    return v + (row * g.n_kv + it - r.n_head - g.n_kv) * HD;
  };
  fv xs[GRP][NT];
#pragma unroll
  for (int j = 0; j < GRP; j++) {
    const uint32_t it = it0 + w + 4 * j;
#pragma unroll
    for (int t = 0; t < NT; t++) xs[j][t] = it < n_items ? *(const fv*)(src_of(it, t) + lane * VPL) : fv{};
  }
  const uint32_t half = r.half_rot;
  for (uint32_t i = tid; i < NT * half; i += blockDim.x) {
    const uint32_t t = i / half, ii = i - t * half;
    float angle = (float)(pos0 + t) * r.freq_scale * r.freq[ii];
    if (r.freq_div) angle = angle / r.freq_div[ii];
    float sn, cn;
    sincosf(angle, &sn, &cn);
    cs[t][ii] = make_float2(cn * r.attn_factor, sn * r.attn_factor);
  }
  const Slot sl0 = locate(g, row_seq[row0], pos0);
  fv wq, wk;
#pragma unroll
  for (int c = 0; c < VPL; c++) {
    wq[c] = r.q_norm ? r.q_norm[lane * VPL + c] : 1.0f;
    wk[c] = r.k_norm ? r.k_norm[lane * VPL + c] : 1.0f;
  }
  __syncthreads();
  const bool neox = (r.flags & ROPE_NEOX) != 0;
  const uint32_t pmask = neox ? half / VPL : 1;
  float2 cf[NT][VPL];
  bool first[VPL], rot[VPL];
#pragma unroll
  for (int c = 0; c < VPL; c++) {
    const uint32_t e = lane * VPL + c;
    rot[c] = e < 2 * half;
    first[c] = neox ? e < half : (e & 1) == 0;
    const uint32_t i = neox ? (e < half ? e : e - half) : e >> 1;
#pragma unroll
    for (int t = 0; t < NT; t++) cf[t][c] = rot[c] ? cs[t][i] : make_float2(1.f, 0.f);
  }
  const Side sv = side(g, true);
  for (uint32_t g0 = 0; it0 + g0 * 4 < n_items; g0 += GRP) {
    if (g0 > 0) {
#pragma unroll
      for (int j = 0; j < GRP; j++) {
        const uint32_t it = it0 + w + 4 * (g0 + j);
#pragma unroll
        for (int t = 0; t < NT; t++) xs[j][t] = it < n_items ? *(const fv*)(src_of(it, t) + lane * VPL) : fv{};
      }
    }
#pragma unroll
    for (int j = 0; j < GRP; j++) {
      const uint32_t it = it0 + w + 4 * (g0 + j);
      if (it >= n_items) continue;
      const bool is_q = it < r.n_head, is_v = it >= r.n_head + g.n_kv;
      const bool norm = is_q ? (r.flags & ROPE_Q_NORM) != 0
                             : is_v ? (r.flags & ROPE_V_NORM) != 0 : (r.flags & ROPE_K_NORM) != 0;
      fv x[NT];
#pragma unroll
      for (int t = 0; t < NT; t++) {
        x[t] = xs[j][t];
        if (norm) {
          float ss = 0.f;
#pragma unroll
          for (int c = 0; c < VPL; c++) ss += x[t][c] * x[t][c];
          const float scale = 1.0f / sqrtf(wave_sum(ss) / (float)HD + r.eps);
          const fv nw = is_q ? wq : wk;
#pragma unroll
          for (int c = 0; c < VPL; c++) x[t][c] = is_v ? x[t][c] * scale : x[t][c] * scale * nw[c];
        }
        if (!is_v && half) {
          fv p;
#pragma unroll
          for (int c = 0; c < VPL; c++) {
            if (neox || VPL == 1)
              p[c] = __shfl_xor(x[t][c], (int)pmask);
            else
              p[c] = x[t][c ^ 1];
          }
#pragma unroll
          for (int c = 0; c < VPL; c++) {
            if (!rot[c]) continue;
            x[t][c] = first[c] ? x[t][c] * cf[t][c].x - p[c] * cf[t][c].y : p[c] * cf[t][c].y + x[t][c] * cf[t][c].x;
          }
        }
      }
      if (is_q) {
#pragma unroll
        for (int t = 0; t < NT; t++) __builtin_nontemporal_store(x[t], (fv*)(q_out + ((size_t)(row0 + t) * r.n_head + it) * HD + lane * VPL));
      } else if (!is_v || NT == 1) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
          Slot sl = sl0;
          sl.m += t;
          float xa[VPL];
#pragma unroll
          for (int c = 0; c < VPL; c++) xa[c] = x[t][c];
          store_head_lanes<VPL>(g, sl, is_v, is_v ? it - r.n_head - g.n_kv : it - r.n_head, xa, lane);
        }
      } else {
        uint8_t* head = sl0.base + sv.off + (it - r.n_head - g.n_kv) * sv.head + sl0.tile * sv.tile;
        const bool f16 = g.kv_type == KV_F16;
#pragma unroll
        for (int c = 0; c < VPL; c++) {
          uint32_t b[4];
#pragma unroll
          for (int t = 0; t < 4; t++) b[t] = f16 ? f16_bits(x[t][c]) : bf16_bits(x[t][c]);
          *(uint2*)(head + v16_off(sl0.m, lane * VPL + c)) = make_uint2(b[0] | (b[1] << 16), b[2] | (b[3] << 16));
        }
      }
    }
  }
}

// Workgroups x < n_quads take an aligned run of 4 f16 / bf16 tokens each (quads[x] = its first
// row), the others one of the remaining rows (rest[x - n_quads], or row x - n_quads without a
// list), in one launch. blockIdx.y picks the workgroup's share of the heads, items y*ipw .. y*ipw+ipw-1, so a
// short call still spreads over the chip instead of leaving each workgroup a long chain of round
// trips.
template <int VPL>
__global__ __launch_bounds__(256) void qk_rope_store_quad_kernel(PageGeom g, RopeGeom r, const int32_t* quads,
                                                                 uint32_t n_quads, const int32_t* rest,
                                                                 const int32_t* row_seq, const int32_t* row_pos,
                                                                 const float* q, const float* k, const float* v,
                                                                 float* q_out, uint32_t ipw) {
  __shared__ float2 cs[4][ROPE_MAX_DIM / 2];
  const uint32_t it0 = blockIdx.y * ipw, n_items = min(r.n_head + 2 * g.n_kv, it0 + ipw);
  if (blockIdx.x < n_quads)
    rope_tokens<VPL, 4>(g, r, cs, (uint32_t)quads[blockIdx.x], it0, n_items, row_seq, row_pos, q, k, v, q_out);
  else
    rope_tokens<VPL, 1>(g, r, cs, rest ? (uint32_t)rest[blockIdx.x - n_quads] : blockIdx.x - n_quads, it0, n_items,
                        row_seq, row_pos, q, k, v, q_out);
}

// Sum over each group of 8 lanes, the same bits in all 8 (DPP: lane l + lane 7-l, then the quad
// swaps 1 and 2; every lane adds the same pairs, only in another order of operands).
__device__ inline float lanes8_sum(float s) {
  s += __builtin_amdgcn_update_dpp(0.f, s, 0x141, 0xf, 0xf, false);  // row_half_mirror
  s += __builtin_amdgcn_update_dpp(0.f, s, 0xb1, 0xf, 0xf, false);   // quad_perm [1,0,3,2]
  s += __builtin_amdgcn_update_dpp(0.f, s, 0x4e, 0xf, 0xf, false);   // quad_perm [2,3,0,1]
  return s;
}
// Sum over each half wave (32 lanes), the same bits in all of them.
__device__ inline float lanes32_sum(float s) {
  s = lanes8_sum(s);
  s += __builtin_amdgcn_update_dpp(0.f, s, 0x140, 0xf, 0xf, false);  // row_mirror: + lane 15-l
  return s + __shfl_xor(s, 16);
}
// Two values in the page's 16-bit type (round to nearest even; v_cvt_pk_{bf16,f16}_f32).
template <bool BF>
__device__ inline uint32_t pack16x2(float a, float b) {
  if constexpr (BF) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    const b2 h = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, h);
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 h = {(_Float16)a, (_Float16)b};
    return __builtin_bit_cast(uint32_t, h);
  }
}

// An aligned run of 4 f16 / bf16 tokens when hd == hdv == HD (64, 128, 256) and every rotated
// pair sits in one lane (Normal pairs; Neox over all HD dims): the same results as
// rope_tokens<HD / 64, 4>, with the work counted in slots of two heads of one kind (Q, K or V) for
// the run's four tokens, so every lane of a wave runs the same code, and every access 8 or 16
// bytes wide.
//   Q / K slot: lane L holds row (head 2s + (L >> 3 & 1), token L >> 4), the float4s
//   sub + 8f (sub = L & 7, f < HD/64) of each half row: a row's loads are whole 128-byte runs,
//   Neox partners (e, e + HD/2) share the lane, the sum of squares is an 8-lane DPP reduction,
//   and each float4 of K is half of one 16-byte operand row of the tile (8 dims of one key).
//   V slot: lane L takes head 2s + (L >> 5) and HD/64 consecutive 16-byte tile chunks: dims d and
//   d + 16 of the four keys, loaded from the four rows and written with one store per chunk.
// Slots y*spw .. y*spw+spw-1 of [Q pairs][K pairs][V pairs] are the workgroup's share.
template <int HD, bool BF>
__device__ void rope_quad_slots(const PageGeom& g, const RopeGeom& r, float2 (*cs)[ROPE_MAX_DIM / 2], uint32_t row0,
                                uint32_t s0, uint32_t s1, const int32_t* row_seq, const int32_t* row_pos,
                                const float* q, const float* k, const float* v, float* q_out) {
  constexpr uint32_t NF = HD / 64, H2 = HD / 2;
  typedef float fc __attribute__((ext_vector_type(NF)));
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t qs = (r.n_head + 1) / 2, ks = (g.n_kv + 1) / 2;
  const uint32_t sub = lane & 7u, hsel = (lane >> 3) & 1u, t = lane >> 4;
  const size_t row = row0 + t;
  const uint32_t q0 = (lane & 31u) * NF, d0 = 32u * (q0 >> 4) + (q0 & 15u);  // a V slot's dims
  // the values of slot sn, requested one slot ahead of their use (the first before the
  // workgroup's angles and page slot). Q / K: the lane's float4s of its row; V: dims d0 .. and
  // d0+16 .. of the four tokens, as fc values 0..3 and 4..7 of the same registers
  auto load_slot = [&](uint32_t sn, float4 (&x)[2][NF]) {
    if (sn < qs + ks) {
      const bool isq = sn < qs;
      const uint32_t hh = 2 * (isq ? sn : sn - qs) + hsel;
      const bool on = hh < (isq ? r.n_head : g.n_kv);
      const float* src = isq ? q + (row * r.n_head + hh) * r.q_stride : k + (row * g.n_kv + hh) * HD;
#pragma unroll
      for (uint32_t hb = 0; hb < 2; hb++)
#pragma unroll
        for (uint32_t f = 0; f < NF; f++)
          x[hb][f] = on ? *(const float4*)(src + hb * H2 + 4 * (sub + 8 * f)) : make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
      const uint32_t hv = 2 * (sn - qs - ks) + (lane >> 5);
      const bool on = hv < g.n_kv;
      fc* p = (fc*)&x[0][0];
#pragma unroll
      for (uint32_t tt = 0; tt < 4; tt++) {
        const float* src = v + ((size_t)(row0 + tt) * g.n_kv + hv) * HD;
        p[tt] = on ? *(const fc*)(src + d0) : fc{};
        p[4 + tt] = on ? *(const fc*)(src + d0 + 16) : fc{};
      }
    }
  };
  float4 xn[2][NF];
  if (s0 + w < s1) load_slot(s0 + w, xn);
  const uint32_t pos0 = (uint32_t)row_pos[row0];
  const uint32_t half = r.half_rot;
  for (uint32_t i = tid; i < 4 * half; i += blockDim.x) {
    const uint32_t tk = i / half, ii = i - tk * half;
    float angle = (float)(pos0 + tk) * r.freq_scale * r.freq[ii];
    if (r.freq_div) angle = angle / r.freq_div[ii];
    float sn, cn;
    sincosf(angle, &sn, &cn);
    cs[tk][ii] = make_float2(cn * r.attn_factor, sn * r.attn_factor);
  }
  const Slot sl0 = locate(g, row_seq[row0], pos0);
  __syncthreads();
  const bool neox = (r.flags & ROPE_NEOX) != 0;
  // rotation factors of the lane's elements, the same for every Q / K slot: Neox, element c of
  // float4 f pairs with the same element of the other half (angle 4(sub+8f)+c); Normal, the two
  // pairs of the first half's float4 ([0], [1]) and of the second half's ([2], [3])
  float2 cf[NF][4];
#pragma unroll
  for (uint32_t f = 0; f < NF; f++) {
    const uint32_t e = 4 * (sub + 8 * f);
#pragma unroll
    for (uint32_t c = 0; c < 4; c++) {
      const uint32_t i = neox ? e + c : (c < 2 ? e / 2 + c : H2 / 2 + e / 2 + c - 2);
      cf[f][c] = i < half ? cs[t][i] : make_float2(1.f, 0.f);
    }
  }
  float4 wn[2][NF];   // norm weights of the lane's elements for the kind in hand
  uint32_t wn_kind = 3;
  for (uint32_t s = s0 + w; s < s1; s += 4) {
    const uint32_t kind = s < qs ? 0u : s < qs + ks ? 1u : 2u;
    float4 x[2][NF];
#pragma unroll
    for (uint32_t hb = 0; hb < 2; hb++)
#pragma unroll
      for (uint32_t f = 0; f < NF; f++) x[hb][f] = xn[hb][f];
    if (s + 4 < s1) load_slot(s + 4, xn);
    if (kind < 2) {
      const uint32_t hh = 2 * (kind == 0 ? s : s - qs) + hsel;
      const bool on = hh < (kind == 0 ? r.n_head : g.n_kv);
      if (kind == 0 ? (r.flags & ROPE_Q_NORM) != 0 : (r.flags & ROPE_K_NORM) != 0) {
        if (wn_kind != kind) {
          const float* wsrc = kind == 0 ? r.q_norm : r.k_norm;
#pragma unroll
          for (uint32_t hb = 0; hb < 2; hb++)
#pragma unroll
            for (uint32_t f = 0; f < NF; f++)
              wn[hb][f] = wsrc ? *(const float4*)(wsrc + hb * H2 + 4 * (sub + 8 * f)) : make_float4(1.f, 1.f, 1.f, 1.f);
          wn_kind = kind;
        }
        float ss = 0.f;
#pragma unroll
        for (uint32_t hb = 0; hb < 2; hb++)
#pragma unroll
          for (uint32_t f = 0; f < NF; f++)
            ss += x[hb][f].x * x[hb][f].x + x[hb][f].y * x[hb][f].y + x[hb][f].z * x[hb][f].z + x[hb][f].w * x[hb][f].w;
        const float scale = 1.0f / sqrtf(lanes8_sum(ss) / (float)HD + r.eps);
#pragma unroll
        for (uint32_t hb = 0; hb < 2; hb++)
#pragma unroll
          for (uint32_t f = 0; f < NF; f++) {
            x[hb][f].x = x[hb][f].x * scale * wn[hb][f].x;
            x[hb][f].y = x[hb][f].y * scale * wn[hb][f].y;
            x[hb][f].z = x[hb][f].z * scale * wn[hb][f].z;
            x[hb][f].w = x[hb][f].w * scale * wn[hb][f].w;
          }
      }
      if (half) {
#pragma unroll
        for (uint32_t f = 0; f < NF; f++) {
          if (neox) {
            float* a = (float*)&x[0][f];
            float* b = (float*)&x[1][f];
#pragma unroll
            for (uint32_t c = 0; c < 4; c++) {
              const float xa = a[c], xb = b[c];
              a[c] = xa * cf[f][c].x - xb * cf[f][c].y;
              b[c] = xa * cf[f][c].y + xb * cf[f][c].x;
            }
          } else {
#pragma unroll
            for (uint32_t hb = 0; hb < 2; hb++) {
              float* a = (float*)&x[hb][f];
#pragma unroll
              for (uint32_t p = 0; p < 2; p++) {
                // pairs past the rotated dims keep their values as they are (no x*1 - y*0)
                const bool rp = hb * (H2 / 2) + 2 * (sub + 8 * f) + p < half;
                const float2 c = cf[f][2 * hb + p];
                const float x0 = a[2 * p], x1 = a[2 * p + 1];
                a[2 * p] = rp ? x0 * c.x - x1 * c.y : x0;
                a[2 * p + 1] = rp ? x0 * c.y + x1 * c.x : x1;
              }
            }
          }
        }
      }
      if (!on) continue;
      if (kind == 0) {
        float* dst = q_out + (row * r.n_head + hh) * HD;
#pragma unroll
        for (uint32_t hb = 0; hb < 2; hb++)
#pragma unroll
          for (uint32_t f = 0; f < NF; f++) {
            // Q is stored non-temporally (rope_c3: kernel 75 -> 60 us); the K/V pages stay
            // cacheable for the attention call that reads them next (non-temporal there: no gain)
            typedef float f4 __attribute__((ext_vector_type(4)));
            const f4 v = {x[hb][f].x, x[hb][f].y, x[hb][f].z, x[hb][f].w};
            __builtin_nontemporal_store(v, (f4*)(dst + hb * H2 + 4 * (sub + 8 * f)));
          }
      } else {
        uint8_t* head = sl0.base + g.k_off + hh * g.k_head + sl0.tile * g.k_tile;
#pragma unroll
        for (uint32_t hb = 0; hb < 2; hb++)
#pragma unroll
          for (uint32_t f = 0; f < NF; f++)
            *(uint2*)(head + k16_off(sl0.m + t, hb * H2 + 4 * (sub + 8 * f))) =
                make_uint2(pack16x2<BF>(x[hb][f].x, x[hb][f].y), pack16x2<BF>(x[hb][f].z, x[hb][f].w));
      }
    } else {
      const uint32_t hv = 2 * (s - qs - ks) + (lane >> 5);
      const bool on = hv < g.n_kv;
      const fc* p = (const fc*)&x[0][0];
      fc a[4], b[4];  // dims d0 .. d0+NF-1 and d0+16 .. of the four tokens
#pragma unroll
      for (uint32_t tt = 0; tt < 4; tt++) {
        a[tt] = p[tt];
        b[tt] = p[4 + tt];
      }
      if (r.flags & ROPE_V_NORM) {
#pragma unroll
        for (uint32_t tt = 0; tt < 4; tt++) {
          float ss = 0.f;
#pragma unroll
          for (uint32_t c = 0; c < NF; c++) ss += a[tt][c] * a[tt][c] + b[tt][c] * b[tt][c];
          const float scale = 1.0f / sqrtf(lanes32_sum(ss) / (float)HD + r.eps);
#pragma unroll
          for (uint32_t c = 0; c < NF; c++) {
            a[tt][c] = a[tt][c] * scale;
            b[tt][c] = b[tt][c] * scale;
          }
        }
      }
      if (!on) continue;
      uint8_t* head = sl0.base + g.v_off + hv * g.v_head + sl0.tile * g.v_tile;
#pragma unroll
      for (uint32_t c = 0; c < NF; c++)
        *(uint4*)(head + v16_off(sl0.m, d0 + c)) =
            make_uint4(pack16x2<BF>(a[0][c], a[1][c]), pack16x2<BF>(a[2][c], a[3][c]),
                       pack16x2<BF>(b[0][c], b[1][c]), pack16x2<BF>(b[2][c], b[3][c]));
    }
  }
}

// The launch of rope_quad_slots: workgroups x < n_quads take an aligned run of 4 tokens and
// slots y*spw .. ; the others one remaining row and items y*ipw .. (rope_tokens<HD / 64, 1>).
template <int HD, bool BF>
__global__ __launch_bounds__(256) void qk_rope_store_slots_kernel(PageGeom g, RopeGeom r, const int32_t* quads,
                                                                  uint32_t n_quads, const int32_t* rest,
                                                                  const int32_t* row_seq, const int32_t* row_pos,
                                                                  const float* q, const float* k, const float* v,
                                                                  float* q_out, uint32_t ipw, uint32_t spw) {
  __shared__ float2 cs[4][ROPE_MAX_DIM / 2];
  if (blockIdx.x < n_quads) {
    const uint32_t n_slots = (r.n_head + 1) / 2 + 2 * ((g.n_kv + 1) / 2);
    const uint32_t s0 = blockIdx.y * spw, s1 = min(n_slots, s0 + spw);
    if (s0 >= s1) return;
    rope_quad_slots<HD, BF>(g, r, cs, (uint32_t)quads[blockIdx.x], s0, s1, row_seq, row_pos, q, k, v, q_out);
  } else {
    const uint32_t it0 = blockIdx.y * ipw, n_items = min(r.n_head + 2 * g.n_kv, it0 + ipw);
    if (it0 >= n_items) return;
    rope_tokens<HD / 64, 1>(g, r, cs, rest ? (uint32_t)rest[blockIdx.x - n_quads] : blockIdx.x - n_quads, it0,
                            n_items, row_seq, row_pos, q, k, v, q_out);
  }
}

struct SnapGeom {
  uint32_t seq, bt, k_row, v_row;
  uint64_t bb, ref_off;
  uint32_t seg_k, seg_v;  // bytes of one head's values in a K / V row of the reference encoding
};
// byte u of one head's segment of a row (token m) in the reference encoding, as a byte of the
// staged page tile: element bytes for f16/bf16/f32, code or scale bytes for q8_0
__device__ inline uint32_t seg_to_tile(uint32_t type, bool is_v, uint32_t m, uint32_t u, uint32_t dim, uint32_t tile_bytes) {
  switch (type) {
    case KV_F16:
    case KV_BF16: return elem_off(type, is_v, m, u >> 1, dim) + (u & 1u);
    case KV_F32: return elem_off(type, is_v, m, u >> 2, dim) + (u & 3u);
    default: {
      const uint32_t b = u / 34u, r = u % 34u;  // block b: [f16 scale][32 codes]
      if (r < 2) return tile_bytes + (m * (dim >> 5) + b) * 2u + r;
      return elem_off(KV_Q8, is_v, m, 32u * b + r - 2u, dim);
    }
  }
}

template <bool WRITE>
__global__ __launch_bounds__(256) void snapshot_tiles_kernel(PageGeom g, SnapGeom sg, uint8_t* snap) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const uint32_t tid = threadIdx.x;
  uint32_t id = blockIdx.x;
  const bool is_v = id & 1u;
  id >>= 1;
  const uint32_t h = id % g.n_kv;
  id /= g.n_kv;
  const uint32_t tpb = sg.bt >> 4, t = id % tpb, bi = id / tpb;
  const Side sd = side(g, is_v);
  const uint32_t tb = sd.tile, ts = g.kv_type == KV_Q8 ? sd.tile_s : 0, seg = is_v ? sg.seg_v : sg.seg_k;
  const uint32_t row = is_v ? sg.v_row : sg.k_row;
  const int blk = g.table[(size_t)sg.seq * g.bps + bi];
  uint8_t* head = g.pool + (size_t)blk * g.block_bytes + sd.off + h * sd.head;
  uint8_t* tile = head + t * tb;
  uint8_t* scales = head + sd.scale + t * ts;
  uint8_t* rows = snap + (size_t)bi * sg.bb + sg.ref_off + (is_v ? (size_t)sg.bt * sg.k_row : 0) +
                  (size_t)(t * 16) * row + (size_t)h * seg;
  uint8_t* lt = smem;                        // page tile [tb] + scales [ts]
  uint8_t* ls = smem + ((tb + ts + 15) & ~15u);  // row segments [16][seg]
  const uint32_t sw = seg >> 2;              // 4-byte words per segment
  if (WRITE) {
    for (uint32_t o = tid * 16; o < tb; o += 256 * 16) *(uint4*)(lt + o) = *(const uint4*)(tile + o);
    for (uint32_t o = tid * 4; o < ts; o += 256 * 4) *(uint32_t*)(lt + tb + o) = *(const uint32_t*)(scales + o);
    __syncthreads();
    for (uint32_t i = tid; i < 16 * seg; i += 256) {
      const uint32_t m = i / seg, u = i % seg;
      ls[i] = lt[seg_to_tile(g.kv_type, is_v, m, u, sd.dim, tb)];
    }
    __syncthreads();
    for (uint32_t i = tid; i < 16 * sw; i += 256) {
      const uint32_t m = i / sw, wd = i % sw;
      *(uint32_t*)(rows + (size_t)m * row + 4 * wd) = *(const uint32_t*)(ls + m * seg + 4 * wd);
    }
  } else {
    for (uint32_t i = tid; i < 16 * sw; i += 256) {
      const uint32_t m = i / sw, wd = i % sw;
      *(uint32_t*)(ls + m * seg + 4 * wd) = *(const uint32_t*)(rows + (size_t)m * row + 4 * wd);
    }
    __syncthreads();
    for (uint32_t i = tid; i < 16 * seg; i += 256) {
      const uint32_t m = i / seg, u = i % seg;
      lt[seg_to_tile(g.kv_type, is_v, m, u, sd.dim, tb)] = ls[i];
    }
    __syncthreads();
    for (uint32_t o = tid * 16; o < tb; o += 256 * 16) *(uint4*)(tile + o) = *(const uint4*)(lt + o);
    for (uint32_t o = tid * 4; o < ts; o += 256 * 4) *(uint32_t*)(scales + o) = *(const uint32_t*)(lt + tb + o);
  }
}


// n16 16-byte chunks into LDS, chunk i from src(i) to dst(i), with up to 8 loads in flight per
// thread: every load of a batch is issued before the first LDS store, so a workgroup pays one
// memory round trip per batch instead of one per head.
template <typename SrcF, typename DstF>
__device__ __forceinline__ void stage16(uint32_t n16, SrcF src, DstF dst) {
  const uint32_t tid = threadIdx.x;
  for (uint32_t base = 0; base < n16; base += 8 * 256) {
    uint4 v0, v1, v2, v3, v4, v5, v6, v7;
    // chunks past the end re-read the last one (in bounds); only real chunks are stored
    auto ld = [&](int k) { return *(const uint4*)src(min(base + k * 256 + tid, n16 - 1)); };
    v0 = ld(0); v1 = ld(1); v2 = ld(2); v3 = ld(3); v4 = ld(4); v5 = ld(5); v6 = ld(6); v7 = ld(7);
    auto st = [&](int k, const uint4& v) {
      const uint32_t i = base + k * 256 + tid;
      if (i < n16) *(uint4*)dst(i) = v;
    };
    st(0, v0); st(1, v1); st(2, v2); st(3, v3); st(4, v4); st(5, v5); st(6, v6); st(7, v7);
  }
}

// One workgroup per (block, 16-token tile, side) covering every KV head: the page side of that
// unit (each head's codes, then each head's q8_0 scales) and its reference side (16 rows of
// n_kv * seg bytes, one contiguous run) are both staged whole, so HBM sees only 16-byte
// accesses; the byte permutation between them runs in LDS with the geometry known at compile
// time. WRITE: page -> rows (gathered from the staged page bytes); read: rows -> page (scattered
// into a staged page image, then copied out).
template <bool WRITE, int TYPE, int DIM, bool IS_V>
__device__ inline void snapshot_side(const PageGeom& g, const SnapGeom& sg, uint8_t* snap, uint8_t* smem) {
  constexpr uint32_t TB = TYPE == KV_Q8 ? 16 * DIM : TYPE == KV_F32 ? 64 * DIM : 32 * DIM;  // a tile's codes
  constexpr uint32_t TS = TYPE == KV_Q8 ? 16 * (DIM / 32) * 2 : 0;                         // its q8_0 scales
  constexpr uint32_t SEG = TYPE == KV_Q8 ? DIM / 32 * 34 : TYPE == KV_F32 ? 4 * DIM : 2 * DIM;  // a head's row bytes
  constexpr uint32_t PH = TB + TS;  // staged page bytes per head
  const uint32_t tid = threadIdx.x;
  constexpr bool is_v = IS_V;
  const uint32_t id = blockIdx.x >> 1, tpb = sg.bt >> 4, t = id % tpb, bi = id / tpb;
  const Side sd = side(g, is_v);
  const uint32_t nkv = g.n_kv, row = nkv * SEG, span = 16 * row;
  const int blk = g.table[(size_t)sg.seq * g.bps + bi];
  uint8_t* head0 = g.pool + (size_t)blk * g.block_bytes + sd.off;
  uint8_t* rows = snap + (size_t)bi * sg.bb + sg.ref_off + (is_v ? (size_t)sg.bt * sg.k_row : 0) + (size_t)(t * 16) * row;
  uint8_t* pg_l = smem;                                  // [nkv][PH] page image
  uint8_t* rw_l = smem + ((nkv * PH + 15) & ~15u);       // [16 rows][row] (read direction)
  // the page side (each head's codes, then its q8_0 scales) staged into pg_l, and the rows staged
  // into rw_l, each with its loads batched
  auto stage_page = [&]() {
    constexpr uint32_t C16 = PH / 16, T16 = TB / 16;
    stage16(
        nkv * C16,
        [&](uint32_t i) -> const uint8_t* {
          const uint32_t h = i / C16, r = i - h * C16;
          const uint8_t* src = head0 + (size_t)h * sd.head;
          return r < T16 ? src + t * TB + r * 16 : src + sd.scale + t * TS + (r - T16) * 16;
        },
        [&](uint32_t i) -> uint8_t* { return pg_l + (size_t)i * 16; });
  };
  auto stage_rows = [&]() {
    stage16(span / 16, [&](uint32_t i) -> const uint8_t* { return rows + (size_t)i * 16; },
            [&](uint32_t i) -> uint8_t* { return rw_l + (size_t)i * 16; });
  };
  // page byte of (token m, byte u of a head's row segment), relative to the head's staged bytes
  auto page_byte = [&](uint32_t m, uint32_t u) -> uint32_t {
    if constexpr (TYPE == KV_Q8) {
      const uint32_t b = u / 34u, r = u % 34u;
      if (r < 2) return TB + (m * (DIM / 32) + b) * 2u + r;
      return elem_off(KV_Q8, is_v, m, 32u * b + r - 2u, DIM);
    } else if constexpr (TYPE == KV_F32) {
      return elem_off(KV_F32, is_v, m, u >> 2, DIM) + (u & 3u);
    } else {
      return elem_off(TYPE, is_v, m, u >> 1, DIM) + (u & 1u);
    }
  };
  if constexpr (TYPE == KV_Q8) {
    // whole q8_0 row blocks ([f16 scale][32 codes], 34 bytes, 2-byte aligned in the row run):
    // K codes of a block are 4 runs of 8 bytes in the tile; V codes hold 4 tokens per 4-byte
    // word (one word per dimension), so V moves in groups of 4 tokens
    constexpr uint32_t NB = DIM / 32;
    auto scale_at = [&](uint32_t h, uint32_t m, uint32_t b) { return (uint16_t*)(pg_l + h * PH + TB + (m * NB + b) * 2u); };
    auto row_at = [&](uint32_t h, uint32_t m, uint32_t b) { return (uint16_t*)(rw_l + m * row + h * SEG + b * 34u); };
    if (WRITE)
      stage_page();
    else
      stage_rows();
    __syncthreads();
    if constexpr (!IS_V) {
      for (uint32_t un = tid; un < 16 * nkv * NB; un += 256) {
        const uint32_t m = un / (nkv * NB), rem = un - m * (nkv * NB), h = rem / NB, b = rem - h * NB;
        uint8_t* pb = pg_l + h * PH;
        uint16_t* rb = row_at(h, m, b);
        if (WRITE) {
          uint32_t w[8];
#pragma unroll
          for (int r = 0; r < 4; r++) {
            const uint2 x = *(const uint2*)(pb + kq8_off(m, 32 * b + 8 * r));
            w[2 * r] = x.x;
            w[2 * r + 1] = x.y;
          }
          rb[0] = *scale_at(h, m, b);
#pragma unroll
          for (int j = 0; j < 16; j++) rb[1 + j] = (uint16_t)(w[j >> 1] >> (16 * (j & 1)));
        } else {
          uint32_t w[8];
#pragma unroll
          for (int j = 0; j < 8; j++) w[j] = (uint32_t)rb[1 + 2 * j] | ((uint32_t)rb[2 + 2 * j] << 16);
          *scale_at(h, m, b) = rb[0];
#pragma unroll
          for (int r = 0; r < 4; r++) *(uint2*)(pb + kq8_off(m, 32 * b + 8 * r)) = make_uint2(w[2 * r], w[2 * r + 1]);
        }
      }
    } else {
      for (uint32_t un = tid; un < 4 * nkv * NB; un += 256) {
        const uint32_t qg = un / (nkv * NB), rem = un - qg * (nkv * NB), h = rem / NB, b = rem - h * NB;
        uint8_t* pb = pg_l + h * PH;
        uint32_t w[32];  // w[d]: the 4 tokens' codes of dimension 32b + d
        if (WRITE) {
#pragma unroll
          for (int d = 0; d < 32; d++) w[d] = *(const uint32_t*)(pb + vq8_off(4 * qg, 32 * b + d));
#pragma unroll
          for (int k = 0; k < 4; k++) {
            const uint32_t m = 4 * qg + k;
            uint16_t* rb = row_at(h, m, b);
            rb[0] = *scale_at(h, m, b);
#pragma unroll
            for (int j = 0; j < 16; j++)
              rb[1 + j] = (uint16_t)(((w[2 * j] >> (8 * k)) & 0xffu) | (((w[2 * j + 1] >> (8 * k)) & 0xffu) << 8));
          }
        } else {
#pragma unroll
          for (int d = 0; d < 32; d++) w[d] = 0;
#pragma unroll
          for (int k = 0; k < 4; k++) {
            const uint32_t m = 4 * qg + k;
            const uint16_t* rb = row_at(h, m, b);
            *scale_at(h, m, b) = rb[0];
#pragma unroll
            for (int j = 0; j < 16; j++) {
              const uint32_t v2 = rb[1 + j];
              w[2 * j] |= (v2 & 0xffu) << (8 * k);
              w[2 * j + 1] |= (v2 >> 8) << (8 * k);
            }
          }
#pragma unroll
          for (int d = 0; d < 32; d++) *(uint32_t*)(pb + vq8_off(4 * qg, 32 * b + d)) = w[d];
        }
      }
    }
    __syncthreads();
    if (WRITE) {
      for (uint32_t o = tid * 16; o < span; o += 256 * 16) *(uint4*)(rows + o) = *(const uint4*)(rw_l + o);
    } else {
      for (uint32_t h = 0; h < nkv; h++) {
        uint8_t* dst = head0 + (size_t)h * sd.head;
        for (uint32_t o = tid * 16; o < TB; o += 256 * 16) *(uint4*)(dst + t * TB + o) = *(const uint4*)(pg_l + h * PH + o);
        for (uint32_t o = tid * 4; o < TS; o += 256 * 4)
          *(uint32_t*)(dst + sd.scale + t * TS + o) = *(const uint32_t*)(pg_l + h * PH + TB + o);
      }
    }
    return;
  }
  if (WRITE) {
    stage_page();
    __syncthreads();
    for (uint32_t c = tid; c < span / 16; c += 256) {
      const uint32_t x0 = c * 16;
      uint32_t m = x0 / row, rem = x0 - m * row, h = rem / SEG, u = rem - h * SEG;
      uint32_t w4[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        uint32_t acc = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
          acc |= (uint32_t)pg_l[h * PH + page_byte(m, u)] << (8 * j);
          if (++u == SEG) {
            u = 0;
            if (++h == nkv) {
              h = 0;
              m++;
            }
          }
        }
        w4[k] = acc;
      }
      *(uint4*)(rows + x0) = make_uint4(w4[0], w4[1], w4[2], w4[3]);
    }
  } else {
    stage_rows();
    __syncthreads();
    for (uint32_t c = tid; c < span / 16; c += 256) {
      const uint32_t x0 = c * 16;
      uint32_t m = x0 / row, rem = x0 - m * row, h = rem / SEG, u = rem - h * SEG;
#pragma unroll
      for (int j = 0; j < 16; j++) {
        pg_l[h * PH + page_byte(m, u)] = rw_l[x0 + j];
        if (++u == SEG) {
          u = 0;
          if (++h == nkv) {
            h = 0;
            m++;
          }
        }
      }
    }
    __syncthreads();
    for (uint32_t h = 0; h < nkv; h++) {
      uint8_t* dst = head0 + (size_t)h * sd.head;
      for (uint32_t o = tid * 16; o < TB; o += 256 * 16) *(uint4*)(dst + t * TB + o) = *(const uint4*)(pg_l + h * PH + o);
      if constexpr (TS > 0)
        for (uint32_t o = tid * 4; o < TS; o += 256 * 4)
          *(uint32_t*)(dst + sd.scale + t * TS + o) = *(const uint32_t*)(pg_l + h * PH + TB + o);
    }
  }
}
template <bool WRITE, int TYPE, int DIM>
__global__ __launch_bounds__(256) void snapshot_side_kernel(PageGeom g, SnapGeom sg, uint8_t* snap) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  if (blockIdx.x & 1u)
    snapshot_side<WRITE, TYPE, DIM, true>(g, sg, snap, smem);
  else
    snapshot_side<WRITE, TYPE, DIM, false>(g, sg, snap, smem);
}

// Zero whole blocks (a newly backed block reads as zeros, like the reference's anonymous
// mappings, kv.rs:29-37). block_bytes is a multiple of 16.
__global__ void zero_blocks_kernel(uint8_t* pool, uint64_t block_bytes, const int32_t* blocks, uint32_t n) {
  const uint64_t per = block_bytes / 16u;
  const uint32_t b = blockIdx.y;
  if (b >= n) return;
  uint4* base = (uint4*)(pool + (size_t)blocks[b] * block_bytes);
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < per; i += (uint64_t)gridDim.x * blockDim.x)
    base[i] = make_uint4(0, 0, 0, 0);
}

}  // namespace

hipError_t launch_store_f32(const PageGeom& g, const int32_t* row_seq, const int32_t* row_pos, uint32_t n_rows,
                            const float* k, const float* v, hipStream_t s) {
  if (n_rows == 0) return hipSuccess;
  hipLaunchKernelGGL(store_f32_kernel, dim3(n_rows), dim3(256), 0, s, g, row_seq, row_pos, k, v);
  return hipGetLastError();
}

hipError_t launch_store_encoded(const PageGeom& g, const int32_t* row_seq, const int32_t* row_pos,
                                uint32_t n_rows, const uint8_t* k, const uint8_t* v, uint32_t k_row,
                                uint32_t v_row, hipStream_t s) {
  if (n_rows == 0) return hipSuccess;
  hipLaunchKernelGGL(store_encoded_kernel, dim3(n_rows), dim3(256), 0, s, g, row_seq, row_pos, k, v, k_row, v_row);
  return hipGetLastError();
}

hipError_t launch_gather(const PageGeom& g, const int32_t* row_seq, const int32_t* row_pos, uint32_t n_rows,
                         float* k, float* v, hipStream_t s) {
  if (n_rows == 0) return hipSuccess;
  hipLaunchKernelGGL(gather_kernel, dim3(n_rows), dim3(256), 0, s, g, row_seq, row_pos, k, v);
  return hipGetLastError();
}

hipError_t launch_gather_encoded(const PageGeom& g, const int32_t* row_seq, const int32_t* row_pos,
                                 uint32_t n_rows, uint8_t* k, uint8_t* v, uint32_t k_row, uint32_t v_row,
                                 hipStream_t s) {
  if (n_rows == 0) return hipSuccess;
  hipLaunchKernelGGL(gather_encoded_kernel, dim3(n_rows), dim3(256), 0, s, g, row_seq, row_pos, k, v, k_row,
                     v_row);
  return hipGetLastError();
}

hipError_t launch_qk_rope_store(const PageGeom& g, const RopeGeom& r, const int32_t* row_seq, const int32_t* row_pos,
                                uint32_t n_rows, const float* q, const float* k, const float* v, float* q_out,
                                const int32_t* quads, uint32_t n_quads, const int32_t* rest, uint32_t n_rest,
                                hipStream_t s, const LaunchEv& ev) {
  if (n_rows == 0) return hipSuccess;
  // register path: hd == hdv = 64*VPL; Normal pairs are always in-lane (VPL >= 2) or one lane
  // apart; Neox partners are half_rot/VPL lanes apart, which must be a whole power of two. The
  // tile layout's widths stop at 256, so VPL is 1, 2 or 4.
  const uint32_t vpl = g.hd / 64, half = r.half_rot;
  const bool neox = (r.flags & ROPE_NEOX) != 0;
  const bool pairs_ok = half == 0 || !neox || (half % vpl == 0 && ((half / vpl) & (half / vpl - 1)) == 0);
  const bool reg = g.layout == LAYOUT_TILES && g.hd == g.hdv && g.hd % 64 == 0 &&
                   (vpl == 1 || vpl == 2 || vpl == 4) && pairs_ok;
  if (reg) {
    // aligned runs of 4 f16 / bf16 rows (when the caller found any) with the other rows, or a
    // short call of any type (decode rows), go to the split kernel: one launch, each row's heads
    // split over workgroups (8 items = one round of 2 heads per wave at the least) until the grid
    // holds about 1024 workgroups, the 4 per CU its registers allow (measured on 256 .. 8192 rows:
    // a target of 512 or 2048 is slower at 2048 and 4096 rows). Long calls without runs go to the
    // row kernel, which keeps 16 heads per wave in flight.
    const bool quad_ok = n_quads > 0 && (g.kv_type == KV_F16 || g.kv_type == KV_BF16);
    if (!quad_ok) {
      n_quads = 0;
      rest = nullptr;
      n_rest = n_rows;
    }
    // the slot kernel: hd == hdv in {64, 128, 256}, rotated pairs inside a lane (Normal, or Neox
    // over all dims), every row and weight vector 16-byte aligned
    const auto al16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
    const bool slots = quad_ok && g.hd == g.hdv && (g.hd == 64 || g.hd == 128 || g.hd == 256) &&
                       (!neox || half == 0 || half == g.hd / 2) && r.q_stride % 4 == 0 && al16(q) && al16(k) &&
                       al16(v) && al16(q_out) && al16(r.q_norm) && al16(r.k_norm);
    if (slots) {
      // slots (two heads of one kind for a run's 4 tokens) split over workgroups until the grid
      // holds about 1024 of them, at least one slot per wave; the remaining rows take items
      // (heads) in as many shares
      const uint32_t n_wg = n_quads + n_rest, n_items = r.n_head + 2 * g.n_kv;
      const uint32_t n_slots = (r.n_head + 1) / 2 + 2 * ((g.n_kv + 1) / 2), max_split = (n_slots + 3) / 4;
      const uint32_t split = std::min(max_split, std::max(1u, (1024u + n_wg - 1) / n_wg));
      const uint32_t spw = (n_slots + split - 1) / split, ipw = ((n_items + split - 1) / split + 3) & ~3u;
      const dim3 grid(n_wg, std::max((n_slots + spw - 1) / spw, (n_items + ipw - 1) / ipw));
#define LMH_SLOTS(H, B)                                                                                            \
  LMH_LAUNCH(ev, (qk_rope_store_slots_kernel<H, B>), grid, dim3(256), 0, s, g, r, quads, n_quads, rest, row_seq, \
             row_pos, q, k, v, q_out, ipw, spw)
      const bool bf = g.kv_type == KV_BF16;
      switch (g.hd) {
        case 64: if (bf) LMH_SLOTS(64, true); else LMH_SLOTS(64, false); break;
        case 128: if (bf) LMH_SLOTS(128, true); else LMH_SLOTS(128, false); break;
        default: if (bf) LMH_SLOTS(256, true); else LMH_SLOTS(256, false); break;
      }
#undef LMH_SLOTS
      return hipGetLastError();
    }
    if (quad_ok || n_rows < 1024) {
      const uint32_t n_wg = n_quads + n_rest, n_items = r.n_head + 2 * g.n_kv, max_split = (n_items + 7) / 8;
      const uint32_t split = std::min(max_split, std::max(1u, (1024u + n_wg - 1) / n_wg));
      const uint32_t ipw = ((n_items + split - 1) / split + 3) & ~3u;
      const dim3 grid(n_wg, (n_items + ipw - 1) / ipw);
#define LMH_QUAD(V)                                                                                            \
  LMH_LAUNCH(ev, qk_rope_store_quad_kernel<V>, grid, dim3(256), 0, s, g, r, quads, n_quads, rest, row_seq, row_pos, \
             q, k, v, q_out, ipw)
      switch (vpl) {
        case 1: LMH_QUAD(1); break;
        case 2: LMH_QUAD(2); break;
        default: LMH_QUAD(4); break;
      }
#undef LMH_QUAD
      return hipGetLastError();
    }
    switch (vpl) {
      case 1: LMH_LAUNCH(ev, qk_rope_store_reg_kernel<1>, dim3(n_rows), dim3(256), 0, s, g, r, row_seq, row_pos, q, k, v, q_out); break;
      case 2: LMH_LAUNCH(ev, qk_rope_store_reg_kernel<2>, dim3(n_rows), dim3(256), 0, s, g, r, row_seq, row_pos, q, k, v, q_out); break;
      default: LMH_LAUNCH(ev, qk_rope_store_reg_kernel<4>, dim3(n_rows), dim3(256), 0, s, g, r, row_seq, row_pos, q, k, v, q_out); break;
    }
  } else {
    LMH_LAUNCH(ev, qk_rope_store_kernel, dim3(n_rows), dim3(256), 0, s, g, r, row_seq, row_pos, q, k, v, q_out);
  }
  return hipGetLastError();
}

hipError_t launch_snapshot(bool write, const PageGeom& g, uint32_t seq, uint32_t n_pos, uint32_t bt, uint64_t bb,
                           uint64_t ref_off, uint32_t k_row, uint32_t v_row, uint8_t* bytes, hipStream_t s) {
  if (n_pos == 0) return hipSuccess;
  const uint32_t seg_k = k_row / g.n_kv, seg_v = v_row / g.n_kv;
  const bool tiles = g.layout == LAYOUT_TILES;
  if (tiles && g.hd == g.hdv && bt % 16 == 0 && (g.kv_type == KV_F16 || g.kv_type == KV_BF16 || g.kv_type == KV_Q8) &&
      (g.hd == 64 || g.hd == 128 || g.hd == 256)) {
    const SnapGeom sg{seq, bt, k_row, v_row, bb, ref_off, seg_k, seg_v};
    const uint32_t ph = g.k_tile + (g.kv_type == KV_Q8 ? g.k_tile_s : 0);
    const size_t lds = ((g.n_kv * ph + 15) & ~15u) + (write && g.kv_type != KV_Q8 ? 0 : 16 * (size_t)k_row);
    if (lds <= 64 * 1024) {
      const uint32_t n_wg = n_pos / 16 * 2;
#define LMH_SNAP(T, D)                                                                                       \
  if (g.kv_type == T && g.hd == D) {                                                                          \
    if (write)                                                                                                \
      hipLaunchKernelGGL((snapshot_side_kernel<true, T, D>), dim3(n_wg), dim3(256), lds, s, g, sg, bytes);    \
    else                                                                                                      \
      hipLaunchKernelGGL((snapshot_side_kernel<false, T, D>), dim3(n_wg), dim3(256), lds, s, g, sg, bytes);   \
    return hipGetLastError();                                                                                 \
  }
      LMH_SNAP(KV_F16, 64) LMH_SNAP(KV_F16, 128) LMH_SNAP(KV_F16, 256)
      LMH_SNAP(KV_BF16, 64) LMH_SNAP(KV_BF16, 128) LMH_SNAP(KV_BF16, 256)
      LMH_SNAP(KV_Q8, 64) LMH_SNAP(KV_Q8, 128) LMH_SNAP(KV_Q8, 256)
#undef LMH_SNAP
    }
  }
  if (tiles && seg_k % 4 == 0 && seg_v % 4 == 0 && bt % 16 == 0) {
    const SnapGeom sg{seq, bt, k_row, v_row, bb, ref_off, seg_k, seg_v};
    const uint32_t tb = std::max(g.k_tile + (g.kv_type == KV_Q8 ? g.k_tile_s : 0),
                                 g.v_tile + (g.kv_type == KV_Q8 ? g.v_tile_s : 0));
    const size_t lds = ((tb + 15) & ~15u) + 16 * (size_t)std::max(seg_k, seg_v);
    const uint32_t n_wg = n_pos / 16 * g.n_kv * 2;
    if (write)
      hipLaunchKernelGGL(snapshot_tiles_kernel<true>, dim3(n_wg), dim3(256), lds, s, g, sg, bytes);
    else
      hipLaunchKernelGGL(snapshot_tiles_kernel<false>, dim3(n_wg), dim3(256), lds, s, g, sg, bytes);
    return hipGetLastError();
  }
  if (write)
    hipLaunchKernelGGL(snapshot_write_kernel, dim3(n_pos), dim3(256), 0, s, g, seq, bt, bb, ref_off, k_row, v_row, bytes);
  else
    hipLaunchKernelGGL(snapshot_read_kernel, dim3(n_pos), dim3(256), 0, s, g, seq, bt, bb, ref_off, k_row, v_row,
                       (const uint8_t*)bytes);
  return hipGetLastError();
}

// Benchmark hook: every 16-byte word of a buffer read once (grid-stride, folded so the loads are
// kept), the plain streaming read the decode kernel's bandwidth is compared with.
// Non-temporal 16-byte loads, four per thread per step: the fastest plain stream measured on
// MI355X (a cold 1.5 GB at 7.1 TB/s, ordinary loads 6.4 TB/s).
__global__ __launch_bounds__(256) void read_ceiling_kernel(const uint4* __restrict__ p, uint64_t n, uint32_t* sink) {
  typedef unsigned int u4 __attribute__((ext_vector_type(4)));
  uint32_t acc = 0;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x * 4;
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x * 4 + threadIdx.x; i < n; i += stride) {
    u4 x[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const uint64_t j = i + (uint64_t)k * blockDim.x;
      x[k] = j < n ? __builtin_nontemporal_load((const u4*)(p + j)) : u4{0, 0, 0, 0};
    }
#pragma unroll
    for (int k = 0; k < 4; k++) acc ^= x[k][0] ^ x[k][1] ^ x[k][2] ^ x[k][3];
  }
  if (acc == 0x9e3779b9u) sink[0] = acc;  // practically never: the loads are not dead code
}

hipError_t launch_read_ceiling(const uint8_t* p, uint64_t bytes, uint32_t* sink, hipStream_t s, const LaunchEv& ev) {
  LMH_LAUNCH(ev, read_ceiling_kernel, dim3(4096), dim3(256), 0, s, (const uint4*)p, bytes / 16, sink);
  return hipGetLastError();
}

// Words from host-mapped staging memory into device memory (block-table rows): a kernel on the
// caller's stream, where a host-to-device copy would go to the copy engine and make the stream's
// next kernel wait for its completion signal.
__global__ __launch_bounds__(256) void copy_words_kernel(uint32_t* __restrict__ dst, const uint32_t* __restrict__ src,
                                                         uint64_t n) {
  for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

hipError_t launch_copy_words(uint32_t* dst, const uint32_t* src, uint64_t n, hipStream_t s) {
  if (n == 0) return hipSuccess;
  const uint64_t wg = (n + 255) / 256;
  hipLaunchKernelGGL(copy_words_kernel, dim3((uint32_t)(wg < 1024 ? wg : 1024)), dim3(256), 0, s, dst, src, n);
  return hipGetLastError();
}

hipError_t launch_zero_blocks(uint8_t* pool, uint64_t block_bytes, const int32_t* blocks, uint32_t n,
                              hipStream_t s) {
  if (n == 0) return hipSuccess;
  const uint64_t per = block_bytes / 16u;
  uint32_t gx = (uint32_t)((per + 255) / 256);
  if (gx > 64) gx = 64;
  for (uint32_t b0 = 0; b0 < n; b0 += 65535u) {
    const uint32_t nb = (n - b0) < 65535u ? (n - b0) : 65535u;
    hipLaunchKernelGGL(zero_blocks_kernel, dim3(gx, nb), dim3(256), 0, s, pool, block_bytes, blocks + b0, nb);
  }
  return hipGetLastError();
}

}  // namespace lmh
