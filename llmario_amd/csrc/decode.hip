// decode.hip — paged-attention decode on gfx950 (CDNA4).
//
// Computes what `attend` / `attend_split` compute for decode-style rows
// (crates/engine/model/src/forward.rs:585-807): for a row at position `pos` of sequence `seq`
// and KV head `kvh`, every query head of the GQA group attends to keys p_lo..=pos through the
// block table, softmax(scale * q.k) v with fp32 accumulation.
//
// Work decomposition (built on the host from the batch's segments): one wave64 per work item
// (row, KV head, contiguous key range aligned to 16-token tiles). The key range of a long row is
// cut into several items (split-K, as attend_split does for long contexts, forward.rs:688-807);
// their partial (o, m, l) go to `part`, and `merge_kernel` combines them with the exact
// log-sum-exp merge of forward.rs:772-806 (f32 pages with rows of at most 16 tiles: the row's
// split items are waves of one workgroup and merge there, in LDS; see decode_f32_kernel).
//
// f16 / bf16 / q8_0 pages (matrix cores): per 16-token tile,
//   S^T[16 keys x 16 heads] = K[16 x hd] . Q^T[hd x 16]     (v_mfma_f32_16x16x32_{f16,bf16})
//   O^T[hdv x 16 heads]    += V^T[hdv x 16] . P^T[16 x 16]    (v_mfma_f32_16x16x16_f16)
// The C layout of S^T (lane l: keys 4*(l/16)+r, head l%16) is exactly the B layout P^T needs,
// and O^T's C layout keeps each head in the lanes that own its softmax state, so the online
// softmax needs no data movement besides two cross-lane max/sum steps. The page bytes are
// stored in operand order, so each operand is one 16-byte load per lane (1 KiB per wave).
// Q is split into hi + lo halves of the MFMA input type, so scores keep ~22 bits of Q precision
// (f16) or ~16 bits (bf16) against exactly represented K. P is carried past f16 as hi + lo halves
// (two P.V products on the same V operand); bf16 V is widened to f16 (exact for |v| in
// [2^-14, 65504]). q8_0: each 32-dim chunk of Q.K is one MFMA whose result is scaled by that
// chunk's per-key scale; V scales fold into P (and its hi + lo split) per 32-dim block.
//
// f32 pages (VALU): lane per key for Q.K, lane per dim for P.V, fp32 throughout.
#include "decode_tile.h"

#include <mutex>
#include <unordered_map>

namespace lmh {
namespace {

using namespace dtile;

constexpr int WAVES = 4;  // waves (work items) per workgroup

// Waves per SIMD the register allocator must allow: two tile buffers in flight per wave fit in
// 256 VGPRs up to hd 128 (and 192 / 128) (2 waves/SIMD); hd 256 and 192 / 192 need the whole
// file (1 wave/SIMD).
#ifndef LMH_DECODE_WPE
#define LMH_DECODE_WPE 2
#endif
template <int HD, int HDV>
constexpr int waves_per_eu() {
  return (HD >= 256 || (HD >= 192 && HDV >= 192)) ? 1 : LMH_DECODE_WPE;
}

// A prompt token's merge (MergeItem.nh != 0: the key pieces of a cut prefill unit), one wave per
// item: heads h0 .. h0 + nh - 1 of its KV group, each the merge of the n_split = k piece partials
// in slots slot0 .. slot0 + k - 1 (head h at position h of a slot). Lane h * K + s (K: k rounded up
// to a power of two) holds (m, l) of head h's piece s and turns them into 2^(m - M_h) and 1 / L_h,
// the max and sum taken by butterflies within each aligned group of K lanes (log2 K exchange
// steps, not k dependent ones); every lane then folds the item's nh * k partial rows, up to
// PF_MERGE_ROWS loads in flight (the planner keeps nh * k within that, or nh = 1; nh * K
// <= 64 follows), into its NP dims, storing a head after its last piece, RB rows at a time (16
// when no item has more: the lighter kernel runs more waves per SIMD). Prompt merges exist only
// for hdv = 64 or 128 (the prefill's widths), i.e. hdv = 64 * NP.
template <int NP, int RB>
__device__ void merge_heads(const RowGeom& r, uint32_t hdv, const MergeItem& mi, const float* part, float* out,
                            uint32_t lane) {
  {
    const uint32_t k = mi.n_split, nrow = mi.nh * k;
    const uint32_t lk = k > 1 ? 32u - (uint32_t)__builtin_clz(k - 1) : 0u;   // K = 2^lk >= k
    const size_t hstride = hdv + 4, stride = (size_t)r.ng * hstride;
    const float* base = part + (size_t)mi.slot0 * stride + (size_t)mi.h0 * hstride;
    const uint32_t jh = lane >> lk, js = lane & ((1u << lk) - 1u);
    float m = -INFINITY, l = 0.f;
    if (jh < mi.nh && js < k) {
      const float* pr = base + (size_t)js * stride + (size_t)jh * hstride + hdv;
      m = pr[0];   // separate loads: (m, l) are 8-byte aligned only for even hdv
      l = pr[1];
    }
    float M = m;
    for (uint32_t x = 1; x < (1u << lk); x <<= 1) M = fmaxf(M, __shfl_xor(M, (int)x));
    const float c = m == -INFINITY ? 0.f : exp2_fast(m - M);
    float L = c * l;
    for (uint32_t x = 1; x < (1u << lk); x <<= 1) L += __shfl_xor(L, (int)x);
    const float inv = L > 0.f ? 1.0f / L : 0.f;
    float acc[NP];
#pragma unroll
    for (int i = 0; i < NP; i++) acc[i] = 0.f;
    // (head, piece) of row j0 + t, advanced row by row (scalar: no division in the loops). hdv is
    // 64 * NP here, so every lane loads its NP dims of a row as one vector; rows past the item's
    // last re-read that row (in bounds, no branch between the loads) and are not folded.
    typedef float fv __attribute__((ext_vector_type(NP)));
    uint32_t h_at = 0, s_at = 0;
    for (uint32_t j0 = 0; j0 < nrow; j0 += RB) {
      fv pre[RB];
      uint32_t h = h_at, sp = s_at;
#pragma unroll
      for (int t = 0; t < RB; t++) {
        pre[t] = *(const fv*)(base + (size_t)sp * stride + (size_t)h * hstride + lane * NP);
        if (j0 + t + 1 < nrow && ++sp == k) {
          sp = 0;
          h++;
        }
      }
#pragma unroll
      for (int t = 0; t < RB; t++) {
        const uint32_t j = j0 + t;
        if (j < nrow) {
          const float cj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(c), (int)((h_at << lk) + s_at)));
#pragma unroll
          for (int i = 0; i < NP; i++) acc[i] += cj * pre[t][i];
          if (++s_at == k) {
            const float iv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(inv), (int)(h_at << lk)));
            fv o;
#pragma unroll
            for (int i = 0; i < NP; i++) {
              o[i] = acc[i] * iv;
              acc[i] = 0.f;
            }
            *(fv*)(out + ((size_t)mi.row * r.n_head + mi.kvh * r.group + mi.h0 + h_at) * hdv + lane * NP) = o;
            s_at = 0;
            h_at++;
          }
        }
      }
    }
  }
}

// Split-K merge (forward.rs:772-806): merge_prompt_kernel runs the prompt tokens' merges (one wave
// each, merge_heads), merge_kernel the decode rows' merges, one wave per (item, query head), lanes
// over dims:
// m* = max m_s, out = sum 2^(m_s - m*) o_s / sum 2^(m_s - m*) l_s, with m in the log2 domain.
// A separate launch: the kernel boundary makes every split's partials visible across XCDs.
// GROUPS: some decode item has more than 16 splits (rows past the first 16 are loaded in groups of
// 16; without it the kernel keeps the lighter code that a call with at most 16 splits per item
// runs).
template <int NP, int RB>
__global__ __launch_bounds__(256) void merge_prompt_kernel(RowGeom r, uint32_t hdv, const MergeItem* items,
                                                           uint32_t n_items, const float* part, float* out) {
  const uint32_t wv = __builtin_amdgcn_readfirstlane(blockIdx.x * 4 + (threadIdx.x >> 6));
  if (wv < n_items) merge_heads<NP, RB>(r, hdv, items[wv], part, out, threadIdx.x & 63u);
}

template <int NP, bool GROUPS>
__global__ __launch_bounds__(256) void merge_kernel(RowGeom r, uint32_t hdv, const MergeItem* items, uint32_t n_items,
                                                    const float* part, float* out) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wi = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wi >= n_items * r.ng) return;
  const MergeItem mi = items[wi / r.ng];
  const uint32_t h = wi % r.ng;
  if (mi.h0 + h >= r.group) return;
  // lane L folds dims L*NP .. L*NP+NP-1 (NP = ceil(hdv / 64); lanes past hdv idle)
  const bool lane_on = lane * NP < hdv;
  const size_t stride = (size_t)r.ng * (hdv + 4);
  const float* base = part + (size_t)mi.slot0 * stride + (size_t)h * (hdv + 4);
  float acc[NP];
#pragma unroll
  for (int i = 0; i < NP; i++) acc[i] = 0.f;
  float M = -INFINITY, L = 0.f;
  // Up to 64 splits per round: lane s holds split s's (m, l); every lane then folds all of the
  // round's partial rows into its NP dims. The round's first 16 rows (only those that exist: the
  // row count is wave-uniform, so a merge of 4 splits issues 4 loads per lane, not 16) are loaded
  // together with (m, l), so a merge of up to 16 splits costs one memory round trip; later rows
  // follow in groups of 16.
  for (uint32_t s0 = 0; s0 < mi.n_split; s0 += 64) {
    const uint32_t s = s0 + lane;
    const uint32_t n = (mi.n_split - s0) < 64u ? (mi.n_split - s0) : 64u;
    float ms = -INFINITY, ls = 0.f;
    if (s < mi.n_split) {
      ms = base[s * stride + hdv];   // separate loads: (m, l) are 8-byte aligned only for even hdv
      ls = base[s * stride + hdv + 1];
    }
    float pre[16][NP];
#pragma unroll
    for (int k = 0; k < 16; k++) {
      const float* pp = base + (s0 + k) * stride + lane * NP;   // loaded only for live rows (k < n)
#pragma unroll
      for (int i = 0; i < NP; i++) pre[k][i] = (uint32_t)k < n && lane_on && lane * NP + i < hdv ? pp[i] : 0.f;
    }
    float Mr = ms;
    for (int x = 32; x >= 1; x >>= 1) Mr = fmaxf(Mr, __shfl_xor(Mr, x));
    const float Mn = fmaxf(M, Mr);
    const float rescale = M == -INFINITY ? 0.f : exp2_fast(M - Mn);
    const float c = ms == -INFINITY ? 0.f : exp2_fast(ms - Mn);
    float Ls = c * ls;
    for (int x = 32; x >= 1; x >>= 1) Ls += __shfl_xor(Ls, x);
    L = L * rescale + Ls;
#pragma unroll
    for (int i = 0; i < NP; i++) acc[i] *= rescale;
    M = Mn;
    if constexpr (!GROUPS) {
#pragma unroll
      for (int k = 0; k < 16; k++) {
        const float ck = (uint32_t)k < n ? __shfl(c, k) : 0.f;
#pragma unroll
        for (int i = 0; i < NP; i++) acc[i] += ck * pre[k][i];
      }
      continue;
    }
    // rows in groups of 16, each group's loads issued together and one group ahead of its sums
    // (a split count of 17..64 costs one round trip per group, not one per row)
    for (uint32_t k0 = 0; k0 < n; k0 += 16) {
      float nxt[16][NP];
      if (k0 + 16 < n) {
#pragma unroll
        for (int k = 0; k < 16; k++) {
          const uint32_t row = k0 + 16 + k < n ? k0 + 16 + k : k0 + 16;
          const float* pp = base + (s0 + row) * stride + lane * NP;
#pragma unroll
          for (int i = 0; i < NP; i++) nxt[k][i] = lane_on && lane * NP + i < hdv ? pp[i] : 0.f;
        }
      }
#pragma unroll
      for (int k = 0; k < 16; k++) {
        const float ck = k0 + k < n ? __shfl(c, (int)(k0 + k)) : 0.f;
#pragma unroll
        for (int i = 0; i < NP; i++) acc[i] += ck * pre[k][i];
      }
      if (k0 + 16 < n) {
#pragma unroll
        for (int k = 0; k < 16; k++)
#pragma unroll
          for (int i = 0; i < NP; i++) pre[k][i] = nxt[k][i];
      }
    }
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  float* op = out + ((size_t)mi.row * r.n_head + mi.kvh * r.group + mi.h0 + h) * hdv + lane * NP;
#pragma unroll
  for (int i = 0; i < NP; i++)
    if (lane_on && lane * NP + i < hdv) op[i] = acc[i] * inv;
}

template <int KVT, int HD, int HDV>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(waves_per_eu<HD, HDV>(), waves_per_eu<HD, HDV>())))
void decode_mfma_kernel(PageGeom g, RowGeom r, const DecodeItem* items, uint32_t n_items, const float* q, float* out,
                        float* part, MergeCopy mc) {
  const uint32_t wi = blockIdx.x * WAVES + (threadIdx.x >> 6);
  copy_merges(mc, blockIdx.x, gridDim.x);
  if (wi < n_items) decode_item<KVT, HD, HDV>(g, r, items, wi, q, out, part);
}

// Matrix-core decode whose split rows merge inside their workgroup: a row's items (1, 2 or 4) are
// consecutive waves of one workgroup (the planner never lets a group cross one). Each split wave
// leaves its partial in LDS; after the barrier, wave s of a group of n folds the group's partials
// (forward.rs:772-806's log-sum-exp merge) for the O blocks j = s, s + n, .. and writes them. No
// partials go to HBM and the call needs no merge launch. Instances: decode_mfma_local_ok.
static_assert(WAVES == MFMA_LOCAL_WAVES, "the planner's local groups fill the decode kernel's workgroups");
template <int KVT, int HD, int HDV>
constexpr bool mfma_local_ok() {
  return KVT != KV_F32 && HD == HDV && (HD == 64 || HD == 128);
}

template <int KVT, int HD, int HDV>
__global__ __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(waves_per_eu<HD, HDV>(), waves_per_eu<HD, HDV>())))
void decode_mfma_local_kernel(PageGeom g, RowGeom r, const DecodeItem* items, uint32_t n_items, const float* q,
                              float* out, float* part, MergeCopy mc) {
  __shared__ __align__(16) float lp[WAVES * local_partial_floats<HDV>()];
  const uint32_t wi = blockIdx.x * WAVES + (threadIdx.x >> 6);
  copy_merges(mc, blockIdx.x, gridDim.x);
  if (wi < n_items) decode_item<KVT, HD, HDV, true>(g, r, items, wi, q, out, part, lp);
  __syncthreads();   // every wave of the workgroup, with an item or not
  if (wi < n_items) local_merge<HDV, WAVES>(r, items, wi, lp, out);
}

// ---- f32 pages: VALU path ----------------------------------------------------------------------
// NG: query heads per item (the launch's ng when the group is 1, 2, 4 or 8; 16 otherwise, with a
// run-time guard for a last head block shorter than 16), so the per-head loops carry no guards
// for the common group sizes.
// Instances that run a workgroup-local merge: the item's partials fit a wave's LDS share and the
// 8-wave instance keeps its registers without spilling.
template <int HD, int HDV, int N>
constexpr bool f32_local_ok() {
  return HD == HDV && N * HDV <= (int)LOCAL_MERGE_MAX && (HD == 64 || (HD == 128 && N <= 2) || (HD == 256 && N <= 4));
}

template <int HD, int HDV, int NG, int W = WAVES>
__global__ __launch_bounds__(64 * W) void decode_f32_kernel(PageGeom g, RowGeom r, const DecodeItem* items,
                                                                uint32_t n_items, const float* q, float* out,
                                                                float* part, MergeCopy mc) {
  constexpr int ND = HDV / 64 > 0 ? HDV / 64 : 1;  // dims per lane in P.V
  constexpr int LPH = HDV + 2;                             // a head's partial in LDS: o, m, l
  constexpr int LPN = NG * HDV <= LOCAL_MERGE_MAX ? NG * LPH : 1;
  __shared__ float qs[W][NG][HD];
  __shared__ float ps[W][NG][64];
  __shared__ float lp[W][LPN];   // local merge: each wave's partials
  const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
  const uint32_t wi = blockIdx.x * W + w;
  copy_merges(mc, blockIdx.x, gridDim.x);
  const bool active = wi < n_items;
  // local merge: every wave reaches the workgroup barrier before the merge, active or not
  const bool local = LPN > 1 && r.local_merge != 0;
  DecodeItem it = active ? items[wi] : DecodeItem{0, 0, 0, 0, 0, NO_SLOT, 0, 0};
  const uint32_t ng = r.ng;
  // heads of this item; NG < 16 only when it equals the group size, so every item has NG heads
  const uint32_t nh = NG < 16 ? (uint32_t)NG : (it.h0 + ng <= r.group) ? ng : r.group - it.h0;
  if (active) {
    for (uint32_t e = lane; e < nh * HD; e += 64) {
      const uint32_t h = e / HD, d = e % HD;
      qs[w][h][d] = q[((size_t)it.row * r.n_head + it.kvh * r.group + it.h0 + h) * HD + d];
    }
  }
  __syncthreads();
  if (!active && !local) return;
  const int seq = (int)it.seq;
  const int32_t* tab = g.table + (size_t)seq * g.bps;
  const uint32_t bt_mask = (1u << g.bt_shift) - 1u;
  float m[NG], l[NG], o[NG][ND];
#pragma unroll
  for (int h = 0; h < NG; h++) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int i = 0; i < ND; i++) o[h][i] = 0.f;
  }
  // Per 64-key chunk: lane = key for Q.K, lane = dim for P.V. The memory round trips overlap: the
  // chunk's block ids come from the previous chunk's prefetch, its first 16 V rows are requested
  // with its K rows (before any score), and each later group of 16 V rows is requested while the
  // previous one is being accumulated. Keys past the range re-read a valid key's row with
  // weight 0.
  auto blk_of = [&](uint32_t c0) {
    const uint32_t key = c0 + lane;
    return tab[(key < it.p1 ? key : it.p0) >> g.bt_shift];
  };
  int blk = active ? blk_of(it.p0) : 0;
  auto load_v16 = [&](float (&vv)[16][ND], uint32_t c0, uint32_t k0, uint32_t nk) {
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const uint32_t kq = (k0 + j < nk) ? k0 + j : nk - 1;
      const int b2 = __builtin_amdgcn_readlane(blk, (int)kq);  // lane kq resolved key c0 + kq's block
      const uint32_t ib = (c0 + kq) & bt_mask;
      const float* vrow = (const float*)(g.pool + (size_t)b2 * g.block_bytes + g.v_off + it.kvh * g.v_head +
                                         (ib >> 4) * g.v_tile) + (ib & 15u) * HDV;
#pragma unroll
      for (int i = 0; i < ND; i++) vv[j][i] = (lane + 64 * i < (uint32_t)HDV) ? vrow[lane + 64 * i] : 0.f;
    }
  };
  for (uint32_t c0 = it.p0; c0 < it.p1; c0 += 64) {
    const uint32_t key = c0 + lane;
    const bool valid = key < it.p1;
    const uint32_t kk = valid ? key : it.p0;
    const uint32_t in_blk = kk & bt_mask;
    const uint8_t* base = g.pool + (size_t)blk * g.block_bytes;
    const float* krow = (const float*)(base + g.k_off + it.kvh * g.k_head + (in_blk >> 4) * g.k_tile) + (in_blk & 15u) * HD;
    const uint32_t nk = (it.p1 - c0) < 64u ? (it.p1 - c0) : 64u;
    // hd <= 128: K row and two groups of V rows in registers; hd 256 streams K and single-buffers V
    constexpr bool PRE = HD <= 128;
    float4 kr[PRE ? HD / 4 : 1];
    if constexpr (PRE) {
#pragma unroll
      for (int d = 0; d < HD / 4; d++) kr[d] = *(const float4*)(krow + 4 * d);
    }
    float vv[PRE ? 2 : 1][16][ND];
    load_v16(vv[0], c0, 0, nk);
    const int blk_next = (c0 + 64 < it.p1) ? blk_of(c0 + 64) : blk;
    float s[NG];
#pragma unroll
    for (int h = 0; h < NG; h++) s[h] = 0.f;
#pragma unroll
    for (int d = 0; d < HD / 4; d++) {
      const float4 kv = PRE ? kr[PRE ? d : 0] : *(const float4*)(krow + 4 * d);
#pragma unroll
      for (int h = 0; h < NG; h++) {
        if (h < (int)nh) {
          s[h] = fmaf(qs[w][h][4 * d], kv.x, s[h]);
          s[h] = fmaf(qs[w][h][4 * d + 1], kv.y, s[h]);
          s[h] = fmaf(qs[w][h][4 * d + 2], kv.z, s[h]);
          s[h] = fmaf(qs[w][h][4 * d + 3], kv.w, s[h]);
        }
      }
    }
#pragma unroll
    for (int h = 0; h < NG; h++) {
      if (h < (int)nh) {
        const float sc = valid ? s[h] * r.scale_log2 : -INFINITY;
        float cm = sc;
        for (int x = 32; x >= 1; x >>= 1) cm = fmaxf(cm, __shfl_xor(cm, x));
        const float mn = fmaxf(m[h], cm);
        const float alpha = exp2_fast(m[h] - mn);
        const float p = exp2_fast(sc - mn);
        float ssum = p;
        for (int x = 32; x >= 1; x >>= 1) ssum += __shfl_xor(ssum, x);
        l[h] = l[h] * alpha + ssum;
        m[h] = mn;
#pragma unroll
        for (int i = 0; i < ND; i++) o[h][i] *= alpha;
        ps[w][h][lane] = p;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int bq = 0; bq < 4; bq++) {
      const uint32_t k0 = 16 * bq;
      if (k0 >= nk) break;
      if (PRE && bq < 3 && k0 + 16 < nk) load_v16(vv[PRE ? (bq + 1) & 1 : 0], c0, k0 + 16, nk);
      if (!PRE && bq > 0) load_v16(vv[0], c0, k0, nk);
#pragma unroll
      for (int j = 0; j < 16; j++) {
#pragma unroll
        for (int h = 0; h < NG; h++) {
          if (h < (int)nh) {
            const float pw = (k0 + j < nk) ? ps[w][h][k0 + j] : 0.f;
#pragma unroll
            for (int i = 0; i < ND; i++) o[h][i] = fmaf(pw, vv[PRE ? bq & 1 : 0][j][i], o[h][i]);
          }
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    blk = blk_next;
  }
  if (active && it.slot == NO_SLOT) {
#pragma unroll
    for (int h = 0; h < NG; h++) {
      if (h < (int)nh) {
        float* op = out + ((size_t)it.row * r.n_head + it.kvh * r.group + it.h0 + h) * HDV;
        const float inv = 1.0f / l[h];
#pragma unroll
        for (int i = 0; i < ND; i++)
          if (lane + 64 * i < (uint32_t)HDV) op[lane + 64 * i] = o[h][i] * inv;
      }
    }
  }
  const bool in_wg = active && it.slot != NO_SLOT && (it.slot & LOCAL_SLOT) != 0;
  if (active && it.slot != NO_SLOT && !in_wg) {
#pragma unroll
    for (int h = 0; h < NG; h++) {
      if (h < (int)nh) {
        float* pp = part + ((size_t)it.slot * r.ng + h) * (HDV + 4);
#pragma unroll
        for (int i = 0; i < ND; i++)
          if (lane + 64 * i < (uint32_t)HDV) pp[lane + 64 * i] = o[h][i];
        if (lane == 0) {
          pp[HDV] = m[h];
          pp[HDV + 1] = l[h];
        }
      }
    }
  }
  if (!local) return;
  // Local merge (forward.rs:772-806's log-sum-exp merge, in LDS): each split wave leaves its
  // partial in lp; after the barrier the row's first wave folds its group's partials.
  if (in_wg) {
#pragma unroll
    for (int h = 0; h < NG; h++) {
      if (h < (int)nh) {
#pragma unroll
        for (int i = 0; i < ND; i++)
          if (lane + 64 * i < (uint32_t)HDV) lp[w][h * LPH + lane + 64 * i] = o[h][i];
        if (lane == 0) {
          lp[w][h * LPH + HDV] = m[h];
          lp[w][h * LPH + HDV + 1] = l[h];
        }
      }
    }
  }
  __syncthreads();
  if (!in_wg || ((it.slot >> 8) & 0xffu) != 0) return;
  const uint32_t n_split = it.slot & 0xffu;
#pragma unroll
  for (int h = 0; h < NG; h++) {
    if (h >= (int)nh) break;
    float M = -INFINITY;
    for (uint32_t s = 0; s < n_split; s++) M = fmaxf(M, lp[w + s][h * LPH + HDV]);
    float L = 0.f, acc[ND];
#pragma unroll
    for (int i = 0; i < ND; i++) acc[i] = 0.f;
    for (uint32_t s = 0; s < n_split; s++) {
      const float ms = lp[w + s][h * LPH + HDV];
      const float c = ms == -INFINITY ? 0.f : exp2_fast(ms - M);
      L = fmaf(c, lp[w + s][h * LPH + HDV + 1], L);
#pragma unroll
      for (int i = 0; i < ND; i++)
        if (lane + 64 * i < (uint32_t)HDV) acc[i] = fmaf(c, lp[w + s][h * LPH + lane + 64 * i], acc[i]);
    }
    const float inv = L > 0.f ? 1.0f / L : 0.f;
    float* op = out + ((size_t)it.row * r.n_head + it.kvh * r.group + it.h0 + h) * HDV;
#pragma unroll
    for (int i = 0; i < ND; i++)
      if (lane + 64 * i < (uint32_t)HDV) op[lane + 64 * i] = acc[i] * inv;
  }
}

// ---- row layout (any head widths up to 512, hd != hdv, blocks under 16 positions): VALU ------
// One wave per item (row, KV head, up to RNG heads of the group, key range), the reference's
// row encoding read directly: per 64-key chunk, lane = key for Q.K (each lane walks its key's row,
// Q broadcast from LDS), lane = dim for P.V (each key's V row read across the lanes), fp32
// throughout, online softmax in the log2 domain as the other decode kernels.
constexpr int RNG = 4;                 // heads per item
constexpr uint32_t ROWS_MAX_DIM = 512;

template <int KVT>
__device__ inline float row_elem(const uint8_t* row, uint32_t d) {
  if constexpr (KVT == KV_F16) return h_to_f(((const uint16_t*)row)[d]);
  else if constexpr (KVT == KV_BF16) return __uint_as_float((uint32_t)((const uint16_t*)row)[d] << 16);
  else if constexpr (KVT == KV_F32) return ((const float*)row)[d];
  else return (float)(int8_t)row[d];   // q8_0 code (the caller applies the block scale)
}

template <int KVT>
__global__ __launch_bounds__(64 * WAVES) void decode_rows_kernel(PageGeom g, RowGeom r, const DecodeItem* items,
                                                                 uint32_t n_items, const float* q, float* out,
                                                                 float* part, MergeCopy mc) {
  constexpr uint32_t ES = KVT == KV_F32 ? 4 : KVT == KV_Q8 ? 1 : 2;   // bytes per value (q8_0: code)
  __shared__ float qs[WAVES][RNG][ROWS_MAX_DIM];
  __shared__ float ps[WAVES][RNG][64];
  const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
  const uint32_t wi = blockIdx.x * WAVES + w;
  copy_merges(mc, blockIdx.x, gridDim.x);
  if (wi >= n_items) return;   // no block-wide barrier below: each wave works alone
  const DecodeItem it = items[wi];
  const uint32_t hd = g.hd, hdv = g.hdv;
  const uint32_t nh = (it.h0 + r.ng <= r.group) ? r.ng : r.group - it.h0;   // heads of this item (<= RNG)
  for (uint32_t e = lane; e < nh * hd; e += 64) {
    const uint32_t h = e / hd, d = e % hd;
    qs[w][h][d] = q[((size_t)it.row * r.n_head + it.kvh * r.group + it.h0 + h) * hd + d];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int32_t* tab = g.table + (size_t)it.seq * g.bps;
  const uint32_t bt_mask = (1u << g.bt_shift) - 1u;
  const uint32_t nd = (hdv + 63) / 64;   // V dims per lane in P.V (<= 8)
  float m[RNG], l[RNG], o[RNG][ROWS_MAX_DIM / 64];
#pragma unroll
  for (int h = 0; h < RNG; h++) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int i = 0; i < (int)(ROWS_MAX_DIM / 64); i++) o[h][i] = 0.f;
  }
  // byte offsets of a key's K / V row (codes) and q8_0 scale rows inside its block
  auto k_at = [&](int blk, uint32_t key, const uint8_t*& row, const uint8_t*& sc) {
    const uint32_t ib = key & bt_mask;
    const uint8_t* head = g.pool + (size_t)blk * g.block_bytes + g.k_off + it.kvh * g.k_head;
    row = head + (ib >> 4) * g.k_tile + (ib & 15u) * hd * ES;
    sc = head + g.k_scale + (ib >> 4) * g.k_tile_s + (ib & 15u) * (hd / 32) * 2;
  };
  auto v_at = [&](int blk, uint32_t key, const uint8_t*& row, const uint8_t*& sc) {
    const uint32_t ib = key & bt_mask;
    const uint8_t* head = g.pool + (size_t)blk * g.block_bytes + g.v_off + it.kvh * g.v_head;
    row = head + (ib >> 4) * g.v_tile + (ib & 15u) * hdv * ES;
    sc = head + g.v_scale + (ib >> 4) * g.v_tile_s + (ib & 15u) * (hdv / 32) * 2;
  };
  for (uint32_t c0 = it.p0; c0 < it.p1; c0 += 64) {
    const uint32_t key = c0 + lane;
    const bool valid = key < it.p1;
    const uint32_t kk = valid ? key : it.p0;
    const int blk = tab[kk >> g.bt_shift];
    const uint32_t nk = (it.p1 - c0) < 64u ? (it.p1 - c0) : 64u;
    const uint8_t *krow, *ksc;
    k_at(blk, kk, krow, ksc);
    float s[RNG] = {0.f, 0.f, 0.f, 0.f};
    // Q.K over 32-dim blocks (q8_0: one scale per block) and a tail of hd % 32 dims
    for (uint32_t d0 = 0; d0 < hd; d0 += 32) {
      const uint32_t dn = hd - d0 < 32u ? hd - d0 : 32u;
      float b[RNG] = {0.f, 0.f, 0.f, 0.f};
      for (uint32_t d = 0; d < dn; d++) {
        const float kx = row_elem<KVT>(krow, d0 + d);
#pragma unroll
        for (int h = 0; h < RNG; h++) b[h] = fmaf(qs[w][h][d0 + d], kx, b[h]);
      }
      const float ksc_b = KVT == KV_Q8 ? h_to_f(((const uint16_t*)ksc)[d0 / 32]) : 1.0f;
#pragma unroll
      for (int h = 0; h < RNG; h++) s[h] = fmaf(b[h], ksc_b, s[h]);
    }
#pragma unroll
    for (int h = 0; h < RNG; h++) {
      if (h >= (int)nh) break;
      const float sc = valid ? s[h] * r.scale_log2 : -INFINITY;
      float cm = sc;
      for (int x = 32; x >= 1; x >>= 1) cm = fmaxf(cm, __shfl_xor(cm, x));
      const float mn = fmaxf(m[h], cm);
      const float alpha = exp2_fast(m[h] - mn);
      const float p = exp2_fast(sc - mn);
      float ssum = p;
      for (int x = 32; x >= 1; x >>= 1) ssum += __shfl_xor(ssum, x);
      l[h] = l[h] * alpha + ssum;
      m[h] = mn;
#pragma unroll
      for (int i = 0; i < (int)(ROWS_MAX_DIM / 64); i++) o[h][i] *= alpha;
      ps[w][h][lane] = p;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    for (uint32_t j = 0; j < nk; j++) {
      const int bj = __builtin_amdgcn_readlane(blk, (int)j);   // lane j resolved key c0 + j's block
      const uint8_t *vrow, *vsc;
      v_at(bj, c0 + j, vrow, vsc);
#pragma unroll
      for (int i = 0; i < (int)(ROWS_MAX_DIM / 64); i++) {
        const uint32_t d = lane + 64 * i;
        if ((uint32_t)i < nd && d < hdv) {
          float vx = row_elem<KVT>(vrow, d);
          if constexpr (KVT == KV_Q8) vx *= h_to_f(((const uint16_t*)vsc)[d / 32]);
#pragma unroll
          for (int h = 0; h < RNG; h++)
            if (h < (int)nh) o[h][i] = fmaf(ps[w][h][j], vx, o[h][i]);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
#pragma unroll
  for (int h = 0; h < RNG; h++) {
    if (h >= (int)nh) break;
    if (it.slot == NO_SLOT) {
      float* op = out + ((size_t)it.row * r.n_head + it.kvh * r.group + it.h0 + h) * hdv;
      const float inv = 1.0f / l[h];
#pragma unroll
      for (int i = 0; i < (int)(ROWS_MAX_DIM / 64); i++)
        if (lane + 64 * i < hdv) op[lane + 64 * i] = o[h][i] * inv;
    } else {
      float* pp = part + ((size_t)it.slot * r.ng + h) * (hdv + 4);
#pragma unroll
      for (int i = 0; i < (int)(ROWS_MAX_DIM / 64); i++)
        if (lane + 64 * i < hdv) pp[lane + 64 * i] = o[h][i];
      if (lane == 0) {
        pp[hdv] = m[h];
        pp[hdv + 1] = l[h];
      }
    }
  }
}

template <int KVT, int HD, int HDV>
hipError_t launch_one(const PageGeom& g, const RowGeom& r, const DecodeItem* items, uint32_t n_items,
                      const float* q, float* out, float* part, const MergeCopy& mc, hipStream_t s, const LaunchEv& ev) {
  const dim3 grid((n_items + WAVES - 1) / WAVES), block(64 * WAVES);
  if constexpr (KVT == KV_F32) {
    if (r.local_merge) {   // a row's split items (up to 8) are waves of one 8-wave workgroup
      const dim3 grid8((n_items + LOCAL_WAVES - 1) / LOCAL_WAVES), block8(64 * LOCAL_WAVES);
#define LMH_F32L(N)                                                                                        \
  if constexpr (f32_local_ok<HD, HDV, N>())                                                                \
    LMH_LAUNCH(ev, (decode_f32_kernel<HD, HDV, N, LOCAL_WAVES>), grid8, block8, 0, s, g, r, items, n_items, q, out, \
               part, mc);                                                                                  \
  else                                                                                                     \
    return hipErrorInvalidValue
      switch (r.group) {
        case 1: LMH_F32L(1); break;
        case 2: LMH_F32L(2); break;
        case 4: LMH_F32L(4); break;
        case 8: LMH_F32L(8); break;
        default: LMH_F32L(16); break;
      }
#undef LMH_F32L
      return hipGetLastError();
    }
    switch (r.group) {
      case 1: LMH_LAUNCH(ev, (decode_f32_kernel<HD, HDV, 1>), grid, block, 0, s, g, r, items, n_items, q, out, part, mc); break;
      case 2: LMH_LAUNCH(ev, (decode_f32_kernel<HD, HDV, 2>), grid, block, 0, s, g, r, items, n_items, q, out, part, mc); break;
      case 4: LMH_LAUNCH(ev, (decode_f32_kernel<HD, HDV, 4>), grid, block, 0, s, g, r, items, n_items, q, out, part, mc); break;
      case 8: LMH_LAUNCH(ev, (decode_f32_kernel<HD, HDV, 8>), grid, block, 0, s, g, r, items, n_items, q, out, part, mc); break;
      default: LMH_LAUNCH(ev, (decode_f32_kernel<HD, HDV, 16>), grid, block, 0, s, g, r, items, n_items, q, out, part, mc); break;
    }
  } else if (r.local_merge) {   // the planner's groups of at most MFMA_LOCAL_WAVES (= WAVES) items
    if constexpr (mfma_local_ok<KVT, HD, HDV>()) {
      if (r.local_merge != (uint32_t)WAVES) return hipErrorInvalidValue;
      LMH_LAUNCH(ev, (decode_mfma_local_kernel<KVT, HD, HDV>), grid, block, 0, s, g, r, items, n_items, q, out, part,
                 mc);
    } else {
      return hipErrorInvalidValue;
    }
  } else {
    LMH_LAUNCH(ev, (decode_mfma_kernel<KVT, HD, HDV>), grid, block, 0, s, g, r, items, n_items, q, out, part, mc);
  }
  return hipGetLastError();
}

// The matrix-core (and f32) decode instances; any other geometry reads the row layout.
#define LMH_TILE_GEOMS_MFMA(X) X(32, 32) X(64, 64) X(96, 96) X(128, 128) X(192, 192) X(256, 256) X(192, 128)
#define LMH_TILE_GEOMS_Q8(X) X(64, 64) X(128, 128) X(192, 192) X(256, 256)
#define LMH_TILE_GEOMS_F32(X) X(64, 64) X(128, 128) X(256, 256)

template <int KVT>
hipError_t dispatch_hd(const PageGeom& g, const RowGeom& r, const DecodeItem* items, uint32_t n_items,
                       const float* q, float* out, float* part, const MergeCopy& mc, hipStream_t s, const LaunchEv& ev) {
#define LMH_HD(H, V) \
  if (g.hd == H && g.hdv == V) return launch_one<KVT, H, V>(g, r, items, n_items, q, out, part, mc, s, ev);
  if constexpr (KVT == KV_F32) {
    LMH_TILE_GEOMS_F32(LMH_HD)
  } else if constexpr (KVT == KV_Q8) {
    LMH_TILE_GEOMS_Q8(LMH_HD)
  } else {
    LMH_TILE_GEOMS_MFMA(LMH_HD)
  }
#undef LMH_HD
  return hipErrorInvalidValue;
}

template <int KVT>
hipError_t launch_rows(const PageGeom& g, const RowGeom& r, const DecodeItem* items, uint32_t n_items,
                       const float* q, float* out, float* part, const MergeCopy& mc, hipStream_t s, const LaunchEv& ev) {
  if (g.hd > ROWS_MAX_DIM || g.hdv > ROWS_MAX_DIM || r.ng > (uint32_t)RNG) return hipErrorInvalidValue;
  const dim3 grid((n_items + WAVES - 1) / WAVES), block(64 * WAVES);
  LMH_LAUNCH(ev, (decode_rows_kernel<KVT>), grid, block, 0, s, g, r, items, n_items, q, out, part, mc);
  return hipGetLastError();
}

// Work items (waves) one CU holds at once, from the occupancy of the instance a launch picks.
template <int KVT, int HD, int HDV>
uint32_t resident_t(uint32_t group) {
  int blocks = 0;
  hipError_t e;
  if constexpr (KVT == KV_F32) {
    switch (group) {   // the instance launch_one picks for this group
      case 1: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, decode_f32_kernel<HD, HDV, 1>, 64 * WAVES, 0); break;
      case 2: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, decode_f32_kernel<HD, HDV, 2>, 64 * WAVES, 0); break;
      case 4: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, decode_f32_kernel<HD, HDV, 4>, 64 * WAVES, 0); break;
      case 8: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, decode_f32_kernel<HD, HDV, 8>, 64 * WAVES, 0); break;
      default: e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, decode_f32_kernel<HD, HDV, 16>, 64 * WAVES, 0); break;
    }
  } else {
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, decode_mfma_kernel<KVT, HD, HDV>, 64 * WAVES, 0);
  }
  return (e == hipSuccess && blocks > 0) ? (uint32_t)blocks * WAVES : WAVES;
}

template <int KVT>
uint32_t resident_rows() {
  int blocks = 0;
  const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, decode_rows_kernel<KVT>, 64 * WAVES, 0);
  return (e == hipSuccess && blocks > 0) ? (uint32_t)blocks * WAVES : WAVES;
}

template <int KVT>
uint32_t resident_geom(uint32_t hd, uint32_t hdv, uint32_t group, uint32_t layout) {
  if (layout == LAYOUT_ROWS) return resident_rows<KVT>();
#define LMH_RES(H, V) \
  if (hd == H && hdv == V) return resident_t<KVT, H, V>(group);
  if constexpr (KVT == KV_F32) {
    LMH_TILE_GEOMS_F32(LMH_RES)
  } else if constexpr (KVT == KV_Q8) {
    LMH_TILE_GEOMS_Q8(LMH_RES)
  } else {
    LMH_TILE_GEOMS_MFMA(LMH_RES)
  }
#undef LMH_RES
  return resident_rows<KVT>();
}

template <int KVT>
bool tiles_geom(uint32_t hd, uint32_t hdv) {
#define LMH_HAS(H, V) \
  if (hd == H && hdv == V) return true;
  if constexpr (KVT == KV_F32) {
    LMH_TILE_GEOMS_F32(LMH_HAS)
  } else if constexpr (KVT == KV_Q8) {
    LMH_TILE_GEOMS_Q8(LMH_HAS)
  } else {
    LMH_TILE_GEOMS_MFMA(LMH_HAS)
  }
#undef LMH_HAS
  return false;
}

}  // namespace

// ---- scratch of lmh_attend_noalloc --------------------------------------------------------------
// Split-K partials and the merge list of calls that may not allocate: a file-scope device array,
// one copy per GPU, held until the process ends. Host code never names `scratch` as an address
// (in host code the name is a stand-in, not the device address): noalloc_scratch() resolves each
// device's copy once with hipGetSymbolAddress, with that device current, and the launches take the
// resolved pointer like any other buffer.
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

hipError_t noalloc_scratch(int device, uint8_t** out) {
  static std::mutex mu;
  static std::unordered_map<int, uint8_t*> addr;  // device ordinal -> address of its copy
  std::lock_guard<std::mutex> lock(mu);
  auto it = addr.find(device);
  if (it != addr.end()) {
    *out = it->second;
    return hipSuccess;
  }
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return e;
  if (cur != device) return hipErrorInvalidDevice;   // the caller makes `device` current first
  void* p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  if (!p) return hipErrorInvalidSymbol;
  addr[device] = (uint8_t*)p;
  *out = (uint8_t*)p;
  return hipSuccess;
}

uint32_t decode_waves_per_cu(uint32_t kv_type, uint32_t hd, uint32_t hdv, uint32_t group, uint32_t layout) {
  switch (kv_type) {
    case KV_F16: return resident_geom<KV_F16>(hd, hdv, group, layout);
    case KV_BF16: return resident_geom<KV_BF16>(hd, hdv, group, layout);
    case KV_Q8: return resident_geom<KV_Q8>(hd, hdv, group, layout);
    default: return resident_geom<KV_F32>(hd, hdv, group, layout);
  }
}

bool decode_tiles_supported(uint32_t kv_type, uint32_t hd, uint32_t hdv) {
  switch (kv_type) {
    case KV_F16: return tiles_geom<KV_F16>(hd, hdv);
    case KV_BF16: return tiles_geom<KV_BF16>(hd, hdv);
    case KV_Q8: return tiles_geom<KV_Q8>(hd, hdv);
    case KV_F32: return tiles_geom<KV_F32>(hd, hdv);
  }
  return false;
}

uint32_t decode_rows_max_heads() { return RNG; }

bool decode_local_merge_ok(uint32_t hd, uint32_t hdv, uint32_t group) {
  const uint32_t n = group == 1 || group == 2 || group == 4 || group == 8 ? group : 16;
#define LMH_LOK(H)                                                                                         \
  if (hd == H && hdv == H)                                                                                 \
    return n == 1 ? f32_local_ok<H, H, 1>() : n == 2 ? f32_local_ok<H, H, 2>() : n == 4 ? f32_local_ok<H, H, 4>() \
           : n == 8 ? f32_local_ok<H, H, 8>() : f32_local_ok<H, H, 16>();
  LMH_LOK(64) LMH_LOK(128) LMH_LOK(256)
#undef LMH_LOK
  return false;
}

bool decode_mfma_local_ok(uint32_t kv_type, uint32_t hd, uint32_t hdv) {
#define LMH_MLOK(T)                                                                                       \
  if (kv_type == T) return (hd == 64 && hdv == 64) ? mfma_local_ok<T, 64, 64>() : (hd == 128 && hdv == 128) ? mfma_local_ok<T, 128, 128>() : false;
  LMH_MLOK(KV_F16) LMH_MLOK(KV_BF16) LMH_MLOK(KV_Q8)
#undef LMH_MLOK
  return false;
}

hipError_t launch_decode(const PageGeom& g, const RowGeom& r, const DecodeItem* items, uint32_t n_items,
                         const float* q, float* out, float* part, const MergeCopy& mc, hipStream_t s,
                         const LaunchEv& ev) {
  if (n_items == 0) return hipSuccess;
  if (g.layout == LAYOUT_ROWS) {
    switch (g.kv_type) {
      case KV_F16: return launch_rows<KV_F16>(g, r, items, n_items, q, out, part, mc, s, ev);
      case KV_BF16: return launch_rows<KV_BF16>(g, r, items, n_items, q, out, part, mc, s, ev);
      case KV_Q8: return launch_rows<KV_Q8>(g, r, items, n_items, q, out, part, mc, s, ev);
      case KV_F32: return launch_rows<KV_F32>(g, r, items, n_items, q, out, part, mc, s, ev);
    }
    return hipErrorInvalidValue;
  }
  switch (g.kv_type) {
    case KV_F16: return dispatch_hd<KV_F16>(g, r, items, n_items, q, out, part, mc, s, ev);
    case KV_BF16: return dispatch_hd<KV_BF16>(g, r, items, n_items, q, out, part, mc, s, ev);
    case KV_Q8: return dispatch_hd<KV_Q8>(g, r, items, n_items, q, out, part, mc, s, ev);
    case KV_F32: return dispatch_hd<KV_F32>(g, r, items, n_items, q, out, part, mc, s, ev);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_merge(const RowGeom& r, uint32_t hdv, const MergeItem* items, uint32_t n_items, uint32_t n_pf,
                        uint32_t max_pf_rows, const float* part, float* out, uint32_t max_split, hipStream_t s,
                        const LaunchEv& ev) {
  if (n_items == 0) return hipSuccess;
  if (hdv == 0 || hdv > ROWS_MAX_DIM || n_pf > n_items || (n_pf > 0 && hdv != 64 && hdv != 128))
    return hipErrorInvalidValue;
  // the prompt tokens' merges and the decode merges as two launches when the call has both (the
  // timing events then bracket the pair)
  const uint32_t n_dec = n_items - n_pf;
  const LaunchEv ev_pf{ev.start, n_dec ? nullptr : ev.stop}, ev_dec{n_pf ? nullptr : ev.start, ev.stop};
  if (n_pf > 0) {
    const dim3 grid((n_pf + 3) / 4), block(256);
    if (max_pf_rows > 64) return hipErrorInvalidValue;   // nh * k <= PF_MERGE_ROWS, or nh = 1 and k <= 64
    const bool light = max_pf_rows <= 16;
    if (hdv == 64 && light) LMH_LAUNCH(ev_pf, (merge_prompt_kernel<1, 16>), grid, block, 0, s, r, hdv, items, n_pf, part, out);
    else if (hdv == 64) LMH_LAUNCH(ev_pf, (merge_prompt_kernel<1, PF_MERGE_ROWS>), grid, block, 0, s, r, hdv, items, n_pf, part, out);
    else if (light) LMH_LAUNCH(ev_pf, (merge_prompt_kernel<2, 16>), grid, block, 0, s, r, hdv, items, n_pf, part, out);
    else LMH_LAUNCH(ev_pf, (merge_prompt_kernel<2, PF_MERGE_ROWS>), grid, block, 0, s, r, hdv, items, n_pf, part, out);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || n_dec == 0) return e;
  }
  items += n_pf;
  const uint64_t waves = (uint64_t)n_dec * r.ng;
  const dim3 grid((uint32_t)((waves + 3) / 4)), block(256);
  // dims per lane: ceil(hdv / 64) rounded up to a power of two
  const uint32_t np = hdv <= 64 ? 1 : hdv <= 128 ? 2 : hdv <= 256 ? 4 : 8;
#define LMH_MERGE(NP)                                                                                              \
  if (np == NP) {                                                                                                  \
    if (max_split > 16)                                                                                            \
      LMH_LAUNCH(ev_dec, (merge_kernel<NP, true>), grid, block, 0, s, r, hdv, items, n_dec, part, out);           \
    else LMH_LAUNCH(ev_dec, (merge_kernel<NP, false>), grid, block, 0, s, r, hdv, items, n_dec, part, out);       \
    return hipGetLastError();                                                                                      \
  }
  LMH_MERGE(1) LMH_MERGE(2) LMH_MERGE(4) LMH_MERGE(8)
#undef LMH_MERGE
  return hipErrorInvalidValue;
}

}  // namespace lmh
