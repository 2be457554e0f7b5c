// prefill.hip — causal / chunked-prefill attention on gfx950 matrix cores.
//
// Computes what `attend` computes for the rows of a multi-token segment
// (crates/engine/model/src/forward.rs:585-678): row t at position pos attends to keys
// lo..=pos of its own sequence (lo = pos+1-window with a window, else 0), softmax(scale q.k) v
// per query head, fp32 accumulation. The Metal sibling is attn_prefill_t
// (crates/engine/metal/src/shaders/attn_prefill.metal:17-195); this kernel is designed for CDNA4.
//
// Work unit (one workgroup, 4 waves): one sequence, one KV head, a run of up to 256/G tokens.
// Its "columns" are the (token, query-head) pairs of the run flattened token-major
// (c = token*G + head), so all G query heads of the KV group share every K/V tile; wave w owns
// columns 64w .. 64w+63 as four 16-column MFMA blocks. Per 64-key tile:
//   S^T[64 keys x 64 cols] = K . Q^T     v_mfma_f32_16x16x32_{bf16,f16}, Q resident in VGPRs
//   online softmax per column in the S^T layout (keys along the 4 lane groups and 4 registers)
//   O^T[hd x 64 cols]     += V^T . P^T  v_mfma_f32_16x16x16_f16, P rounded to f16
// K/V tiles are staged through LDS (double buffered, all 256 threads load 16 B each per 4 KiB
// page tile), straight from the page layout, which already holds each 16-token tile in operand
// order; bf16 V is widened to f16 on the way in (exact for |v| in [2^-14, 65504]). Scores are
// scaled in fp32 (log2 domain) rather than pre-scaling Q in the 16-bit type.
#include "device.h"

namespace lmh {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int PW = 4;          // waves per workgroup
constexpr int COLS = 64;       // columns per wave
constexpr int BK = 64;         // keys per tile (4 page tiles of 16)

__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ inline uint16_t bf16_rne(float x) {
  uint32_t u = __float_as_uint(x);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// bf16 pair (one uint32) -> f16 pair (one uint32), exact in the normal f16 range.
__device__ inline uint32_t bf2_to_h2(uint32_t w) {
  const _Float16 a = (_Float16)__uint_as_float(w << 16);
  const _Float16 b = (_Float16)__uint_as_float(w & 0xffff0000u);
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

template <int KVT, int HD>
__global__ __launch_bounds__(64 * PW) __attribute__((amdgpu_waves_per_eu(1, 1)))
void prefill_kernel(PageGeom g, PrefillGeom pg, const PrefillItem* items, const float* q, float* out) {
  constexpr int NC = HD / 32;   // Q.K chunks of 32 dims
  constexpr int NJ = HD / 16;   // O^T blocks of 16 dims
  constexpr int TILE = 16 * HD * 2;     // bytes of one 16-token page tile (K or V)
  using MT = typename std::conditional<KVT == KV_BF16, b8, h8>::type;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* kv_lds = smem;                                 // [2 stages][K 4 tiles | V 4 tiles]
  int* blk_lds = (int*)(smem + 2 * 8 * TILE);             // block id of each key page in range

  const PrefillItem it = items[blockIdx.x];
  const uint32_t tid = threadIdx.x, lane = tid & 63u, w = tid >> 6;
  const uint32_t hq = lane & 15u, grp = lane >> 4;
  const uint32_t G = pg.group;
  const uint32_t pos_last = it.pos0 + it.n_tok - 1;
  const uint32_t lo_first = (pg.window > 0 && it.pos0 + 1 > pg.window) ? it.pos0 + 1 - pg.window : 0;
  const uint32_t page0 = lo_first >> 4, page1 = pos_last >> 4;
  const uint32_t n_pages = page1 - page0 + 1;

  // ---- block ids of every key page this unit reads
  {
    const int32_t* tab = g.table + (size_t)it.seq * g.bps;
    for (uint32_t p = tid; p < n_pages; p += 64 * PW) blk_lds[p] = tab[((page0 + p) << 4) >> g.bt_shift];
  }

  // ---- this lane's four columns (one per 16-column block) and their Q fragments
  uint32_t cpos[4], clo[4];
  bool cval[4];
  MT qf[4][NC];
#pragma unroll
  for (int cb = 0; cb < 4; cb++) {
    const uint32_t c = w * COLS + cb * 16 + hq;
    const uint32_t t = c / G, hh = c % G;
    cval[cb] = t < it.n_tok;
    cpos[cb] = it.pos0 + (cval[cb] ? t : 0);
    clo[cb] = (pg.window > 0 && cpos[cb] + 1 > pg.window) ? cpos[cb] + 1 - pg.window : 0;
    const float* qp = q + ((size_t)(it.row0 + (cval[cb] ? t : 0)) * pg.n_head + it.kvh * G + hh) * HD;
#pragma unroll
    for (int ch = 0; ch < NC; ch++) {
      float4 a = cval[cb] ? *(const float4*)(qp + 32 * ch + 8 * grp) : make_float4(0, 0, 0, 0);
      float4 b = cval[cb] ? *(const float4*)(qp + 32 * ch + 8 * grp + 4) : make_float4(0, 0, 0, 0);
      const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int i = 0; i < 8; i++) {
        if constexpr (KVT == KV_BF16) {
          qf[cb][ch][i] = __builtin_bit_cast(__bf16, bf16_rne(x[i]));
        } else {
          qf[cb][ch][i] = (_Float16)x[i];
        }
      }
    }
  }
  __syncthreads();

  // ---- K/V tile staging: tile i covers keys (page0 + 4i)*16 .. +64; each thread moves 16 B of
  // each of the 4 K and 4 V page tiles of a stage (a page tile is 16*HD*2 bytes: 4 KiB at hd 128
  // = 256 threads x 16 B; at hd 64 half the threads carry it).
  constexpr bool PART = TILE < 64 * PW * 16;
  const bool carrier = !PART || tid * 16 < (uint32_t)TILE;
  const uint32_t n_tiles = (n_pages + 3) / 4;
  uint4 stk[4], stv[4];
  auto fetch = [&](uint32_t ti) {
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const uint32_t p = ti * 4 + s;
      if (p < n_pages && carrier) {
        const int blk = blk_lds[p];
        const uint32_t sub = (((page0 + p) << 4) & ((1u << g.bt_shift) - 1u)) >> 4;
        const uint8_t* base = g.pool + (size_t)blk * g.block_bytes;
        stk[s] = *(const uint4*)(base + g.k_off + it.kvh * g.k_head + sub * g.k_tile + tid * 16);
        stv[s] = *(const uint4*)(base + g.v_off + it.kvh * g.v_head + sub * g.v_tile + tid * 16);
      } else {
        stk[s] = make_uint4(0, 0, 0, 0);
        stv[s] = make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto commit = [&](uint32_t stage) {
    if (!carrier) return;
    uint8_t* dst = kv_lds + stage * 8 * TILE;
#pragma unroll
    for (int s = 0; s < 4; s++) {
      *(uint4*)(dst + s * TILE + tid * 16) = stk[s];
      uint4 v = stv[s];
      if constexpr (KVT == KV_BF16) {
        v.x = bf2_to_h2(v.x);
        v.y = bf2_to_h2(v.y);
        v.z = bf2_to_h2(v.z);
        v.w = bf2_to_h2(v.w);
      }
      *(uint4*)(dst + (4 + s) * TILE + tid * 16) = v;
    }
  };

  float m[4], l[4];
  f4 O[NJ][4];
#pragma unroll
  for (int cb = 0; cb < 4; cb++) {
    m[cb] = -INFINITY;
    l[cb] = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; j++) O[j][cb] = f4{0.f, 0.f, 0.f, 0.f};
  }
  // lowest/highest column positions of this wave (for whole-tile skips and mask-free tiles)
  uint32_t wpos_min = 0xffffffffu, wpos_max = 0, wlo_max = 0;
  {
    const uint32_t c0 = w * COLS, c1 = w * COLS + COLS - 1;
    const uint32_t t0 = c0 / G, t1 = c1 / G < it.n_tok ? c1 / G : (it.n_tok ? it.n_tok - 1 : 0);
    wpos_min = it.pos0 + (t0 < it.n_tok ? t0 : t1);
    wpos_max = it.pos0 + t1;
    wlo_max = (pg.window > 0 && wpos_max + 1 > pg.window) ? wpos_max + 1 - pg.window : 0;
  }
  const bool wave_active = w * COLS / G < it.n_tok;
  const uint32_t wlo_min = (pg.window > 0 && wpos_min + 1 > pg.window) ? wpos_min + 1 - pg.window : 0;

  fetch(0);
  commit(0);
  __syncthreads();
  for (uint32_t ti = 0; ti < n_tiles; ti++) {
    if (ti + 1 < n_tiles) fetch(ti + 1);
    const uint8_t* kt = kv_lds + (ti & 1) * 8 * TILE;
    const uint8_t* vt = kt + 4 * TILE;
    const uint32_t key0 = (page0 + ti * 4) * 16;
    // Tiles entirely after this wave's last position or before its window are skipped.
    const bool skip = !wave_active || key0 > wpos_max || key0 + BK <= wlo_min;
    if (!skip) {
      const bool need_mask = key0 + BK - 1 > wpos_min || key0 < wlo_max || key0 + BK - 1 > pos_last;
      f4 S[4][4];
#pragma unroll
      for (int kb = 0; kb < 4; kb++) {
#pragma unroll
        for (int cb = 0; cb < 4; cb++) S[kb][cb] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ch = 0; ch < NC; ch++) {
          const MT a = __builtin_bit_cast(MT, *(const uint4*)(kt + kb * TILE + ch * 1024 + lane * 16));
#pragma unroll
          for (int cb = 0; cb < 4; cb++) {
            if constexpr (KVT == KV_BF16)
              S[kb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[cb][ch], S[kb][cb], 0, 0, 0);
            else
              S[kb][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[cb][ch], S[kb][cb], 0, 0, 0);
          }
        }
      }
      // ---- online softmax per column (log2 domain)
      h4 P[4][4];
#pragma unroll
      for (int cb = 0; cb < 4; cb++) {
        float tm = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
#pragma unroll
          for (int r = 0; r < 4; r++) {
            float s = S[kb][cb][r] * pg.scale_log2;
            if (need_mask) {
              const uint32_t key = key0 + kb * 16 + grp * 4 + r;
              if (key > cpos[cb] || key < clo[cb]) s = -INFINITY;
            }
            S[kb][cb][r] = s;
            tm = fmaxf(tm, s);
          }
        }
        tm = fmaxf(tm, __shfl_xor(tm, 16));
        tm = fmaxf(tm, __shfl_xor(tm, 32));
        const float mn = fmaxf(m[cb], tm);
        // a column with no visible key yet keeps m = -inf and contributes nothing
        const float mref = mn == -INFINITY ? 0.f : mn;
        const float alpha = exp2_fast(m[cb] - mref);
        float ls = 0.f;
#pragma unroll
        for (int kb = 0; kb < 4; kb++) {
          float p[4];
#pragma unroll
          for (int r = 0; r < 4; r++) {
            p[r] = exp2_fast(S[kb][cb][r] - mref);
            ls += p[r];
          }
          P[kb][cb] = h4{(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3]};
        }
        l[cb] = l[cb] * alpha + ls;
        m[cb] = mn;
#pragma unroll
        for (int j = 0; j < NJ; j++) O[j][cb] *= alpha;
      }
      // ---- O^T += V^T P^T
#pragma unroll
      for (int kb = 0; kb < 4; kb++) {
#pragma unroll
        for (int j = 0; j < NJ; j++) {
          const h4 va = __builtin_bit_cast(h4, *(const uint2*)(vt + kb * TILE + (j >> 1) * 1024 + lane * 16 + (j & 1) * 8));
#pragma unroll
          for (int cb = 0; cb < 4; cb++) O[j][cb] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, P[kb][cb], O[j][cb], 0, 0, 0);
        }
      }
    }
    if (ti + 1 < n_tiles) {
      __syncthreads();  // everyone is done reading the stage about to be overwritten
      commit((ti + 1) & 1);
      __syncthreads();
    }
  }

  // ---- epilogue: per column, out = O / l (l summed over the lane groups)
#pragma unroll
  for (int cb = 0; cb < 4; cb++) {
    float lt = l[cb];
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
    if (!cval[cb]) continue;
    const uint32_t c = w * COLS + cb * 16 + hq;
    const uint32_t t = c / G, hh = c % G;
    const float inv = lt > 0.f ? 1.0f / lt : 0.f;
    float* op = out + ((size_t)(it.row0 + t) * pg.n_head + it.kvh * G + hh) * HD;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const f4 o = O[j][cb] * inv;
      *(float4*)(op + 16 * j + 4 * grp) = make_float4(o[0], o[1], o[2], o[3]);
    }
  }
}

template <int KVT, int HD>
hipError_t launch_t(const PageGeom& g, const PrefillGeom& pg, const PrefillItem* items, uint32_t n_items,
                    uint32_t max_pages, const float* q, float* out, hipStream_t s) {
  const size_t lds = 2 * 8 * (16 * HD * 2) + (size_t)max_pages * 4;
  hipLaunchKernelGGL((prefill_kernel<KVT, HD>), dim3(n_items), dim3(64 * PW), lds, s, g, pg, items, q, out);
  return hipGetLastError();
}

}  // namespace

uint32_t prefill_cols_per_unit() { return PW * COLS; }

size_t prefill_lds_bytes(uint32_t hd, uint32_t max_pages) { return 2 * 8 * (16 * (size_t)hd * 2) + (size_t)max_pages * 4; }

bool prefill_supported(uint32_t kv_type, uint32_t hd, uint32_t hdv, uint32_t group) {
  return (kv_type == KV_F16 || kv_type == KV_BF16) && hd == hdv && (hd == 64 || hd == 128) && group >= 1 &&
         group <= PW * COLS;
}

hipError_t launch_prefill(const PageGeom& g, const PrefillGeom& pg, const PrefillItem* items, uint32_t n_items,
                          uint32_t max_pages, const float* q, float* out, hipStream_t s) {
  if (n_items == 0) return hipSuccess;
  if (g.kv_type == KV_BF16) {
    if (g.hd == 128) return launch_t<KV_BF16, 128>(g, pg, items, n_items, max_pages, q, out, s);
    if (g.hd == 64) return launch_t<KV_BF16, 64>(g, pg, items, n_items, max_pages, q, out, s);
  } else if (g.kv_type == KV_F16) {
    if (g.hd == 128) return launch_t<KV_F16, 128>(g, pg, items, n_items, max_pages, q, out, s);
    if (g.hd == 64) return launch_t<KV_F16, 64>(g, pg, items, n_items, max_pages, q, out, s);
  }
  return hipErrorInvalidValue;
}

}  // namespace lmh
