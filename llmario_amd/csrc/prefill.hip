// prefill.hip — causal / chunked-prefill attention on gfx950 matrix cores.
//
// Computes what `attend` computes for the rows of a multi-token segment
// (crates/engine/model/src/forward.rs:585-678): row t at position pos attends to keys
// lo..=pos of its own sequence (lo = pos+1-window with a window, else 0), softmax(scale q.k) v
// per query head, fp32 accumulation. The Metal sibling is attn_prefill_t
// (crates/engine/metal/src/shaders/attn_prefill.metal:17-195); this kernel is designed for CDNA4.
//
// Work unit (one workgroup of 8 waves, two per SIMD): one sequence, one KV head, a run of up to
// 256/G tokens. Its "columns" are the (token, query-head) pairs of the run flattened token-major
// (c = token*G + head), so all G query heads of the KV group share every K/V tile; wave w owns
// columns 32w .. 32w+31 as two 16-column MFMA blocks. Per 64-key tile, in two 32-key halves:
//   S^T[32 keys x 32 cols] = K . Q^T     v_mfma_f32_16x16x32_{bf16,f16}, Q resident in VGPRs
//   online softmax per column in the S^T layout (keys along the 4 lane groups and 4 registers)
//   O^T[hd x 32 cols]     += V^T . P^T  v_mfma_f32_16x16x32_f16, P rounded to f16
// K/V tiles go from HBM straight into LDS (global_load_lds, three stages, two tiles in flight)
// in the page layout, which already holds each 16-token tile in MFMA operand order; bf16 V is
// widened to f16 in LDS once per tile by the thread that loaded it (exact for |v| in
// [2^-14, 65504]). Scores are scaled in fp32 (log2 domain) rather than pre-scaling Q in the
// 16-bit type. The reference max of a column moves lazily (only when a block's max exceeds it
// by more than 2^8), so the O accumulators are almost never rescaled.
#include "device.h"

namespace lmh {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int PW = 8;          // waves per workgroup
constexpr int NT = 64 * PW;    // threads per workgroup
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

__device__ inline uint16_t bf16_rne(float x) {
  uint32_t u = __float_as_uint(x);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// 16 bytes per lane from global memory straight into LDS (global_load_lds_dwordx4): lane L reads
// sbase + voff(L) and writes lds_dst + 16*L, where sbase and lds_dst are wave-uniform (an SGPR pair
// and M0). Issued from inline assembly so the compiler does not track it: the kernel waits for
// these loads itself (s_waitcnt vmcnt) before the barrier that publishes a stage, and nothing else
// in the tile loop touches vector memory.
__device__ inline void lds_dma16(const uint8_t* sbase, uint32_t voff, uint8_t* lds_dst) {
  const uint32_t l = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(void __attribute__((address_space(3)))*)lds_dst);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(l), "v"(voff), "s"(sbase) : "memory", "m0");
}

// bf16 pair (one uint32) -> f16 pair (one uint32), exact in the normal f16 range.
__device__ inline uint32_t bf2_to_h2(uint32_t w) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const f2 x = {__uint_as_float(w << 16), __uint_as_float(w & 0xffff0000u)};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(x, h2));
}

template <int KVT, int HD>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
void prefill_kernel(PageGeom g, PrefillGeom pg, const PrefillItem* items, const float* q, float* out) {
  constexpr int NC = HD / 32;                 // Q.K chunks of 32 dims
  constexpr int NJ = HD / 16;                 // O^T blocks of 16 dims
  constexpr int TILE = 16 * HD * 2;           // bytes of one 16-token page tile (K or V)
  using MT = typename std::conditional<KVT == KV_BF16, b8, h8>::type;
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* kv_lds = smem;                                 // [NSTAGE][K 4 tiles | V 4 tiles]
  int* blk_lds = (int*)(smem + NSTAGE * 8 * TILE);        // block id of each key page in range

  const PrefillItem it = items[blockIdx.x];
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  const uint32_t w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, kept in a scalar register
  const uint32_t hq = lane & 15u, grp = lane >> 4;
  const uint32_t G = pg.group;
  const uint32_t pos_last = it.pos0 + it.n_tok - 1;
  const uint32_t lo_first = (pg.window > 0 && it.pos0 + 1 > pg.window) ? it.pos0 + 1 - pg.window : 0;
  const uint32_t page0 = lo_first >> 4, page1 = pos_last >> 4;
  const uint32_t n_pages = page1 - page0 + 1;

  // ---- block ids of every key page this unit reads
  {
    const int32_t* tab = g.table + (size_t)it.seq * g.bps;
    for (uint32_t p = tid; p < n_pages; p += NT) blk_lds[p] = tab[((page0 + p) << 4) >> g.bt_shift];
  }

  // ---- this lane's columns (one per 16-column block) and their Q fragments
  uint32_t cpos[NCB], clo[NCB];
  bool cval[NCB];
  MT qf[NCB][NC];
#pragma unroll
  for (int cb = 0; cb < NCB; cb++) {
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

  // ---- K/V staging. Tile i covers keys (page0 + 4i)*16 .. +64: 4 K and 4 V page tiles. Wave w
  // copies half (w & 1) of page tile (w >> 1) on each side, CPT rows of 1024 bytes, so its page
  // (and the block id behind it) is wave-uniform and the addresses are scalar. Pages past the
  // range re-read the last page (finite values whose keys are masked), so stale LDS never meets a
  // zero weight.
  constexpr int CPT = TILE / 2 / 1024;        // DMA rows per wave per side per tile
  static_assert(CPT >= 1 && 8 * CPT * 1024 == 4 * TILE, "8 waves cover the 4 page tiles of a side");
  const uint32_t n_tiles = (n_pages + 3) / 4;
  const uint32_t my_tile = w >> 1, my_off = my_tile * TILE + (w & 1) * (TILE / 2);
  const uint32_t voff = (w & 1) * (TILE / 2) + lane * 16;
  const uint64_t k_head = g.k_off + (uint64_t)it.kvh * g.k_head;
  const uint64_t v_head = g.v_off + (uint64_t)it.kvh * g.v_head;
  auto issue = [&](uint32_t ti) {
    uint8_t* stage = kv_lds + (ti % NSTAGE) * 8 * TILE;
    const uint32_t p = min(ti * 4 + my_tile, n_pages - 1);
    const uint64_t blk = (uint32_t)__builtin_amdgcn_readfirstlane(blk_lds[p]);
    const uint32_t sub = (((page0 + p) << 4) & ((1u << g.bt_shift) - 1u)) >> 4;
    const uint8_t* pb = g.pool + blk * g.block_bytes;
    const uint8_t* kb = pb + k_head + sub * g.k_tile;
    const uint8_t* vb = pb + v_head + sub * g.v_tile;
#pragma unroll
    for (int k = 0; k < CPT; k++) {
      lds_dma16(kb, voff + k * 1024, stage + my_off + k * 1024);
      lds_dma16(vb, voff + k * 1024, stage + 4 * TILE + my_off + k * 1024);
    }
  };
  // After this wave's share of tile ti has landed: widen its V rows from bf16 to f16 in place.
  auto widen = [&](uint32_t ti) {
    if constexpr (KVT == KV_BF16) {
      uint8_t* v = kv_lds + (ti % NSTAGE) * 8 * TILE + 4 * TILE + my_off + lane * 16;
#pragma unroll
      for (int k = 0; k < CPT; k++) {
        uint4* p = (uint4*)(v + k * 1024);
        uint4 x = *p;
        x.x = bf2_to_h2(x.x);
        x.y = bf2_to_h2(x.y);
        x.z = bf2_to_h2(x.z);
        x.w = bf2_to_h2(x.w);
        *p = x;
      }
    }
  };

  // Online-softmax state per column: reference max m (log2 domain), -m (0 while no key is
  // visible), the threshold on raw scores above which m must move, row sum l, and O^T.
  float m[NCB], nm[NCB], thr[NCB], l[NCB];
  f4 O[NJ][NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; cb++) {
    m[cb] = -INFINITY;
    nm[cb] = 0.f;
    thr[cb] = -INFINITY;
    l[cb] = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; j++) O[j][cb] = f4{0.f, 0.f, 0.f, 0.f};
  }
  // this wave's lowest/highest column positions (mask-free tiles)
  const bool wave_active = w * COLS / G < it.n_tok;
  uint32_t wpos_min, wpos_max;
  {
    const uint32_t t0 = w * COLS / G, tl = (w * COLS + COLS - 1) / G;
    const uint32_t t1 = tl < it.n_tok ? tl : it.n_tok - 1;
    wpos_min = it.pos0 + (t0 < it.n_tok ? t0 : t1);
    wpos_max = it.pos0 + t1;
  }
  const uint32_t wlo_max = (pg.window > 0 && wpos_max + 1 > pg.window) ? wpos_max + 1 - pg.window : 0;
  const float c = pg.scale_log2;  // > 0 (the host routes other scales to the decode kernel)

  // S^T for the 32 keys of half kp of a tile (two 16-key page tiles) x this wave's 32 columns
  auto qk = [&](f4 (&S)[2][NCB], const uint8_t* kt, int kp) {
#pragma unroll
    for (int kk = 0; kk < 2; kk++) {
#pragma unroll
      for (int cb = 0; cb < NCB; cb++) S[kk][cb] = f4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int ch = 0; ch < NC; ch++) {
#pragma unroll
      for (int kk = 0; kk < 2; kk++) {
        const MT a = __builtin_bit_cast(MT, *(const uint4*)(kt + (2 * kp + kk) * TILE + ch * 1024 + lane * 16));
#pragma unroll
        for (int cb = 0; cb < NCB; cb++) {
          if constexpr (KVT == KV_BF16)
            S[kk][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[cb][ch], S[kk][cb], 0, 0, 0);
          else
            S[kk][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[cb][ch], S[kk][cb], 0, 0, 0);
        }
      }
    }
  };
  // keys outside a column's [lo, pos] get -inf (keys past the range are past every position)
  auto mask = [&](f4 (&S)[2][NCB], uint32_t kbase) {
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
#pragma unroll
      for (int kk = 0; kk < 2; kk++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const uint32_t key = kbase + kk * 16 + grp * 4 + r;
          S[kk][cb][r] = (key > cpos[cb] || key < clo[cb]) ? -INFINITY : S[kk][cb][r];
        }
      }
    }
  };
  // Lazy reference max: m moves (rescaling O and l) only when a score exceeds it by more than 8 in
  // the log2 domain, so p = 2^(s*c - m) <= 2^8 and O is rarely touched. Each lane checks its own 8
  // scores per column; only when some lane needs a move is the column max reduced over the lane
  // groups (the decision is then the same on every lane of a column).
  auto rebase = [&](const f4 (&S)[2][NCB]) {
    float lm[NCB];
    bool need = false;
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
      lm[cb] = fmaxf(fmaxf(fmaxf(S[0][cb][0], S[0][cb][1]), fmaxf(S[0][cb][2], S[0][cb][3])),
                     fmaxf(fmaxf(S[1][cb][0], S[1][cb][1]), fmaxf(S[1][cb][2], S[1][cb][3])));
      need |= lm[cb] > thr[cb];
    }
    if (__ballot(need)) {
#pragma unroll
      for (int cb = 0; cb < NCB; cb++) {
        const float tmax = max_over_groups(lm[cb]) * c;
        const bool mv = tmax > m[cb] + 8.0f;
        // m = -inf (first visible key of this column): O and l are still zero
        const float alpha = !mv ? 1.f : (m[cb] == -INFINITY ? 0.f : exp2_fast(m[cb] - tmax));
        l[cb] *= alpha;
#pragma unroll
        for (int j = 0; j < NJ; j++) O[j][cb] *= alpha;
        m[cb] = mv ? tmax : m[cb];
        nm[cb] = m[cb] == -INFINITY ? 0.f : -m[cb];
        thr[cb] = (m[cb] + 8.0f) / c;
      }
    }
  };
  // P = 2^(s*c - m) rounded to f16 (<= 2^8), row sums in f32
  auto softmax = [&](const f4 (&S)[2][NCB], h8 (&P)[NCB]) {
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
      float pv[8];
#pragma unroll
      for (int kk = 0; kk < 2; kk++) {
#pragma unroll
        for (int r = 0; r < 4; r++) pv[kk * 4 + r] = exp2_fast(__builtin_fmaf(S[kk][cb][r], c, nm[cb]));
      }
      l[cb] += ((pv[0] + pv[1]) + (pv[2] + pv[3])) + ((pv[4] + pv[5]) + (pv[6] + pv[7]));
      P[cb] = h8{(_Float16)pv[0], (_Float16)pv[1], (_Float16)pv[2], (_Float16)pv[3],
                 (_Float16)pv[4], (_Float16)pv[5], (_Float16)pv[6], (_Float16)pv[7]};
    }
  };
  // O^T += V^T P^T over half kp, 32 keys per MFMA: k index 8g+i is key 4g+i of the half's first
  // 16-key page tile (i < 4) or key 4g+i-4 of its second; the V^T operand reads the same keys
  // (8 bytes from each of the two page tiles).
  auto pv = [&](const h8 (&P)[NCB], const uint8_t* vt, int kp) {
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const uint32_t off = (j >> 1) * 1024 + lane * 16 + (j & 1) * 8;
      const uint2 v0 = *(const uint2*)(vt + (2 * kp) * TILE + off);
      const uint2 v1 = *(const uint2*)(vt + (2 * kp + 1) * TILE + off);
      const h8 va = __builtin_bit_cast(h8, make_uint4(v0.x, v0.y, v1.x, v1.y));
#pragma unroll
      for (int cb = 0; cb < NCB; cb++) O[j][cb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, P[cb], O[j][cb], 0, 0, 0);
    }
  };

  // Pipeline. Tile ti's loads are issued at the start of iteration ti-2 and published (waited
  // for, widened, barrier) in the middle of iteration ti-1, right before the block that finishes
  // tile ti-1 (softmax + P.V of its second half) and starts tile ti (Q.K of its first half), so
  // the matrix products of one half always have the other half's exponentials beside them.
  // Stage reuse: tile ti+2 goes to stage (ti+2) % 4, last read while finishing tile ti-2, which
  // every wave completed before the barrier of iteration ti-1. A thread issues 2*CPT loads per
  // tile, so "at most 2*CPT outstanding" means its share of the older tile has landed.
  // Every tile is computed (keys outside a column's range are masked), except by waves that own
  // no column at all.
  auto publish = [&](uint32_t ti) {  // tile ti has landed for everyone after this
    if (ti + 1 < n_tiles) {
      if constexpr (CPT == 1)
        asm volatile("s_waitcnt vmcnt(2)" ::: "memory");
      else
        asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    widen(ti);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };
  f4 S0[2][NCB], S1[2][NCB];
  h8 P[NCB];
  issue(0);
  if (n_tiles > 1) issue(1);
  publish(0);
  if (wave_active) qk(S0, kv_lds, 0);
  for (uint32_t ti = 0; ti < n_tiles; ti++) {
    if (ti + 2 < n_tiles) issue(ti + 2);
    const uint8_t* kt = kv_lds + (ti % NSTAGE) * 8 * TILE;
    const uint8_t* vt = kt + 4 * TILE;
    const uint32_t key0 = (page0 + ti * 4) * 16;
    const bool need_mask = key0 + BK - 1 > wpos_min || key0 < wlo_max || key0 + BK - 1 > pos_last;
    if (wave_active) {
      if (need_mask) mask(S0, key0);
      rebase(S0);
      qk(S1, kt, 1);
      softmax(S0, P);
      pv(P, vt, 0);
      if (need_mask) mask(S1, key0 + 32);
      rebase(S1);
    }
    if (ti + 1 < n_tiles) publish(ti + 1);
    if (wave_active) {
      softmax(S1, P);
      pv(P, vt, 1);
      // first half of the next tile (after the last tile: a stale stage, never used)
      qk(S0, kv_lds + ((ti + 1) % NSTAGE) * 8 * TILE, 0);
    }
  }

  // ---- epilogue: per column, out = O / l (l summed over the lane groups)
#pragma unroll
  for (int cb = 0; cb < NCB; cb++) {
    const float lt = sum_over_groups(l[cb]);
    if (!cval[cb]) continue;
    const uint32_t col = w * COLS + cb * 16 + hq;
    const uint32_t t = col / G, hh = col % G;
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
  const size_t lds = prefill_lds_bytes(HD, max_pages);
  hipLaunchKernelGGL((prefill_kernel<KVT, HD>), dim3(n_items), dim3(NT), lds, s, g, pg, items, q, out);
  return hipGetLastError();
}

}  // namespace

uint32_t prefill_cols_per_unit() { return PW * COLS; }

size_t prefill_lds_bytes(uint32_t hd, uint32_t max_pages) {
  return NSTAGE * 8 * (16 * (size_t)hd * 2) + (size_t)max_pages * 4;
}

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
