// Block selectors: the decode steps of the reference's qbb modes
// (Quest-style per-block channel bounds, EV:5508-5617), brep modes (block
// representatives, EV:5361-5505, with their BlockRepState, EV:1853-1918) and
// qboracle modes (block maxima of the partial scores, EV:5008-5097), on
// GQA-shaped bf16 or fp16 K/V (D = 128; query, K and the dim-major copy
// share the dtype).
//
// Rows are (sequence, query head) r = b * Hq + h, reading K head h / (Hq/Hkv).
// Per step:
//   qbb_meta_kernel / brep_meta_kernel  per-KV-head block metadata, kept
//       across steps and refreshed only for the blocks new tokens touch:
//       per-channel min and max (qbb), or the R tokens of largest squared
//       norm (brep);
//   block_scores_kernel  per (row, block): the bound sum_s q_s * (q_s >= 0 ?
//       max : min) over the row's top-|q| dims, or the best representative's
//       partial score;
//   block_max_partial_kernel  (qboracle, no metadata) per (row, block): the
//       largest partial score of the block's tokens, from the dim-major copy;
//   (qkv_topk)           the best blocks;
//   scan_partial_kernel  partial scores of the chosen blocks' tokens from the
//       dim-major K copy (the blocks' tokens are contiguous there);
//   rerank_kernel        one 1024-thread workgroup per row: the best
//       candidates by partial score, their full-D scores, the best of those,
//       the final mask and the final token list (sink / recent / current).
// Arithmetic follows the reference's fp32 formulas with separately rounded
// products and sums in dim order (built with -ffp-contract=off); selections
// keep the lower index on ties.  EV = ymluo/projects/qwen3_top2_head_limit3_ppl/
// src/evaluate_qwen3_top2_head_limit3_ppl.py.
#include <math.h>

#include <type_traits>

#include "common.h"
#include "ref_common.h"
#include "select.h"

namespace qkv {
namespace {

constexpr int kBT = 256;
constexpr int kHD = 128;             // head size
constexpr int kMaxCand = 4096;       // candidates per row (rerank LDS list)
constexpr int kRerankNT = 1024;
constexpr int kMaxScan = kRerankNT * 40;   // scanned tokens per row in one workgroup

// The row's top-|q| dims in selection order (descending |q|, lower dim on
// ties; QK:123-145), from an LDS copy of q (published by the barrier this
// begins with).  Ends with a barrier.
__device__ void rank_dims(const float* q_s, int count, int* sel_idx, float* sel_q) {
  __shared__ __attribute__((aligned(16))) uint64_t key_s[kHD];
  __syncthreads();
  rank_dims128(q_s, key_s, kHD, count, sel_idx, sel_q);
}

// The 16-bit pattern of v, a value of the dtype (exact).
template <bool F16>
__device__ __forceinline__ uint16_t half_bits(float v) {
  if constexpr (F16) return __builtin_bit_cast(uint16_t, static_cast<_Float16>(v));
  else return static_cast<uint16_t>(__float_as_uint(v) >> 16);
}

// scaling * sum_d q[d] * K[d] over d ascending, separately rounded (the
// reference's fp32 order), for one bf16 (fp16) K row of kHD values (16-byte
// aligned) and q in LDS (16-byte aligned).  The row's loads go out first;
// q is read eight values per 16-byte word where it is used (the empty asm
// keeps those reads from being hoisted all at once next to the row loads).
template <bool F16>
__device__ __forceinline__ float full_score(const uint16_t* __restrict__ krow, const float* q_s, float scaling) {
  const uint4* kr = reinterpret_cast<const uint4*>(krow);
  uint4 x[kHD / 8];
#pragma unroll
  for (int c = 0; c < kHD / 8; ++c) x[c] = kr[c];
  const float4* q4 = reinterpret_cast<const float4*>(q_s);
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < kHD / 8; ++c) {
    asm volatile("" ::: "memory");
    const float4 qa = q4[2 * c], qb = q4[2 * c + 1];
    const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    const uint32_t w[4] = {x[c].x, x[c].y, x[c].z, x[c].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc = acc + qv[2 * e] * half_lo<F16>(w[e]);
      acc = acc + qv[2 * e + 1] * half_hi<F16>(w[e]);
    }
  }
  return acc * scaling;
}

// ---------------------------------------------------------------------------
// Metadata.  qbb: per block a 512-byte record [min(128) | max(128)] in K's
// dtype (exact: they are elements of K).  brep: per block R int32 token
// indices, descending squared norm, lower index on ties, -1 where the block
// has fewer tokens.  Blocks [j0, j0 + grid.x) over tokens below t_end are
// rebuilt.
// ---------------------------------------------------------------------------

// Squared norm of one K row of kHD values (16-byte aligned), an fp32 sum in
// channel order (BlockRepState's norm, EV:1899-1913).
template <bool F16>
__device__ __forceinline__ float sq_norm(const uint16_t* __restrict__ krow) {
  const uint4* kr = reinterpret_cast<const uint4*>(krow);
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < kHD / 8; ++c) {
    const uint4 x = kr[c];
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = half_lo<F16>(w[e]), hi = half_hi<F16>(w[e]);
      acc = acc + lo * lo;
      acc = acc + hi * hi;
    }
  }
  return acc;
}

// (norm, token) of the better representative: larger norm, then lower token.
__device__ __forceinline__ void rep_better(float& bn, int& bt, float on, int ot) {
  if (on > bn || (on == bn && ot < bt)) {
    bn = on;
    bt = ot;
  }
}
template <bool F16>
__global__ __launch_bounds__(kBT) void qbb_meta_kernel(const uint16_t* __restrict__ key, int kv_heads, int64_t sb,
                                                       int64_t sh, int64_t st, int block, int t_end, int j0,
                                                       uint16_t* __restrict__ meta, int64_t meta_blocks) {
  const int j = j0 + blockIdx.x, row = blockIdx.y, tid = threadIdx.x;
  const int b = row / kv_heads, h = row - b * kv_heads;
  const int t_lo = j * block, t_hi = min(t_end, t_lo + block);
  const uint16_t* kb = key + b * sb + h * sh;
  uint16_t* rec = meta + (static_cast<int64_t>(row) * meta_blocks + j) * 2 * kHD;
  for (int c = tid; c < kHD; c += kBT) {
    float mn = __builtin_huge_valf(), mx = -__builtin_huge_valf();
    for (int t = t_lo; t < t_hi; ++t) {
      const float v = half_to_f32<F16>(kb[static_cast<int64_t>(t) * st + c]);
      mn = fminf(mn, v);
      mx = fmaxf(mx, v);
    }
    rec[c] = half_bits<F16>(mn);
    rec[kHD + c] = half_bits<F16>(mx);
  }
}

// One wave per block (block <= 64): lane l scores token j*block + l.
template <bool F16>
__global__ __launch_bounds__(kBT) void brep_meta_kernel(const uint16_t* __restrict__ key, int kv_heads, int64_t sb,
                                                        int64_t sh, int64_t st, int block, int reps, int t_end,
                                                        int j0, int j_end, int32_t* __restrict__ meta,
                                                        int64_t meta_blocks) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, row = blockIdx.y;
  const int j = j0 + blockIdx.x * (kBT / 64) + wave;
  if (j >= j_end) return;   // whole waves leave; no workgroup barrier below
  const int b = row / kv_heads, h = row - b * kv_heads;
  const int t = j * block + lane;
  const bool ok = lane < block && t < t_end;
  float norm = -1.0f;   // below every real norm
  if (ok) norm = sq_norm<F16>(key + b * sb + h * sh + static_cast<int64_t>(t) * st);
  int32_t* rec = meta + (static_cast<int64_t>(row) * meta_blocks + j) * reps;
  for (int r = 0; r < reps; ++r) {
    // the lane with the largest (norm, -lane)
    float bn = norm;
    int bl = lane;
    for (int off = 32; off > 0; off >>= 1) {
      const float on = __shfl_xor(bn, off);
      const int ol = __shfl_xor(bl, off);
      if (on > bn || (on == bn && ol < bl)) {
        bn = on;
        bl = ol;
      }
    }
    if (lane == 0) rec[r] = bn >= 0.0f ? j * block + bl : -1;
    if (lane == bl) norm = -1.0f;   // taken
  }
}

// Blocks longer than a wave: one workgroup per block.  Thread i holds the
// norms of its first kRepCache tokens (t_lo + i + kRepNT*c) in registers and
// recomputes any further ones every round (blocks above kRepNT*kRepCache
// tokens); each of the R rounds is a workgroup argmax, and the taken tokens
// are listed in LDS.
constexpr int kRepNT = 1024;
constexpr int kRepCache = 16;

template <bool F16>
__global__ __launch_bounds__(kRepNT) void brep_meta_wide_kernel(const uint16_t* __restrict__ key, int kv_heads,
                                                                int64_t sb, int64_t sh, int64_t st, int block,
                                                                int reps, int t_end, int j0,
                                                                int32_t* __restrict__ meta, int64_t meta_blocks) {
  constexpr int NW = kRepNT / 64;
  __shared__ float red_n[NW];
  __shared__ int red_t[NW];
  __shared__ int taken[64];
  const int j = j0 + blockIdx.x, row = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = row / kv_heads, h = row - b * kv_heads;
  const int t_lo = j * block, t_hi = min(t_end, t_lo + block);
  const uint16_t* kb = key + b * sb + h * sh;
  float cache[kRepCache];
#pragma unroll
  for (int c = 0; c < kRepCache; ++c) {
    const int t = t_lo + tid + c * kRepNT;
    cache[c] = t < t_hi ? sq_norm<F16>(kb + static_cast<int64_t>(t) * st) : -1.0f;
  }
  int32_t* rec = meta + (static_cast<int64_t>(row) * meta_blocks + j) * reps;
  for (int r = 0; r < reps; ++r) {
    float bn = -1.0f;
    int bt = 0x7FFFFFFF;
#pragma unroll
    for (int c = 0; c < kRepCache; ++c) rep_better(bn, bt, cache[c], t_lo + tid + c * kRepNT);
    for (int t = t_lo + tid + kRepCache * kRepNT; t < t_hi; t += kRepNT) {
      bool was = false;
      for (int i = 0; i < r; ++i) was |= taken[i] == t;
      if (!was) rep_better(bn, bt, sq_norm<F16>(kb + static_cast<int64_t>(t) * st), t);
    }
    for (int off = 32; off > 0; off >>= 1) {
      const float on = __shfl_xor(bn, off);
      const int ot = __shfl_xor(bt, off);
      rep_better(bn, bt, on, ot);
    }
    if (lane == 0) {
      red_n[wave] = bn;
      red_t[wave] = bt;
    }
    __syncthreads();
    bn = red_n[0];
    bt = red_t[0];
    for (int w = 1; w < NW; ++w) rep_better(bn, bt, red_n[w], red_t[w]);
    const int win = bn >= 0.0f ? bt : -1;   // every thread holds the winner
    if (tid == 0) {
      rec[r] = win;
      taken[r] = win;
    }
#pragma unroll
    for (int c = 0; c < kRepCache; ++c)
      if (win == t_lo + tid + c * kRepNT) cache[c] = -1.0f;
    __syncthreads();   // red_n / red_t are rewritten next round; taken[r] is visible
  }
}

// ---------------------------------------------------------------------------
// Block scores of one row: qbb bound (EV:5554) or best representative
// (EV:5431-5435; no valid representative -> finfo(float32).min).
// ---------------------------------------------------------------------------
template <int KIND, bool F16>   // KIND 0: qbb, 1: brep
__global__ __launch_bounds__(kBT) void block_scores_kernel(
    const uint16_t* __restrict__ query, const uint16_t* __restrict__ key, int q_heads, int group, int kv_heads,
    int64_t sb, int64_t sh, int64_t st, const void* __restrict__ meta, int64_t meta_blocks, int reps, int nb,
    int count, float* __restrict__ out, int64_t out_ld) {
  __shared__ float q_s[kHD];
  __shared__ int sel_idx[kHD];
  __shared__ float sel_q[kHD];
  const int row = blockIdx.y, tid = threadIdx.x;
  const int b = row / q_heads, h = row - b * q_heads;
  const int kvrow = b * kv_heads + h / group;
  for (int d = tid; d < kHD; d += kBT) q_s[d] = half_to_f32<F16>(query[static_cast<int64_t>(row) * kHD + d]);
  __syncthreads();
  rank_dims(q_s, count, sel_idx, sel_q);
  const int j = blockIdx.x * kBT + tid;
  if (j >= nb) return;
  float acc;
  if constexpr (KIND == 0) {
    const uint16_t* rec = static_cast<const uint16_t*>(meta) + (static_cast<int64_t>(kvrow) * meta_blocks + j) * 2 * kHD;
    acc = 0.0f;
    for (int s = 0; s < count; ++s) {
      const float qs = sel_q[s];
      const int d = sel_idx[s];
      const float e = half_to_f32<F16>(qs >= 0.0f ? rec[kHD + d] : rec[d]);
      acc = acc + qs * e;
    }
  } else {
    const int32_t* rec = static_cast<const int32_t*>(meta) + (static_cast<int64_t>(kvrow) * meta_blocks + j) * reps;
    const uint16_t* kb = key + b * sb + (h / group) * sh;
    acc = -3.40282347e38f;   // finfo(float32).min
    for (int r = 0; r < reps; ++r) {
      const int tok = rec[r];
      if (tok < 0) continue;
      const uint16_t* kr = kb + static_cast<int64_t>(tok) * st;
      float sc = 0.0f;
      for (int s = 0; s < count; ++s) sc = sc + sel_q[s] * half_to_f32<F16>(kr[sel_idx[s]]);
      acc = fmaxf(acc, sc);
    }
  }
  out[static_cast<int64_t>(row) * out_ld + j] = acc;
}

// ---------------------------------------------------------------------------
// Partial scores of the chosen blocks' tokens (EV:5576-5581) from the
// dim-major copy: position p of a row is token blocks[p / block] * block +
// p % block; positions at or past the history score -inf.
// ---------------------------------------------------------------------------
template <bool F16>
__global__ __launch_bounds__(kBT) void scan_partial_kernel(
    const uint16_t* __restrict__ query, const uint16_t* __restrict__ kdm, int q_heads, int group, int64_t db,
    int64_t dh, int64_t dd, const int32_t* __restrict__ blocks, int n_scan, int block, int history, int count,
    float* __restrict__ out, int64_t out_ld, const uint16_t* __restrict__ key, int64_t sb, int64_t sh, int64_t st,
    float scaling, float* __restrict__ full) {
  __shared__ __attribute__((aligned(16))) float q_s[kHD];
  __shared__ int sel_idx[kHD];
  __shared__ float sel_q[kHD];
  const int row = blockIdx.y, tid = threadIdx.x;
  const int b = row / q_heads, h = row - b * q_heads;
  for (int d = tid; d < kHD; d += kBT) q_s[d] = half_to_f32<F16>(query[static_cast<int64_t>(row) * kHD + d]);
  __syncthreads();
  rank_dims(q_s, count, sel_idx, sel_q);
  const int p = blockIdx.x * kBT + tid;
  if (p >= n_scan * block) return;
  const int jb = p / block;
  const int tok = blocks[static_cast<int64_t>(row) * n_scan + jb] * block + (p - jb * block);
  float acc = -__builtin_huge_valf();
  if (tok >= 0 && tok < history) {
    const uint16_t* base = kdm + b * db + (h / group) * dh + tok;
    acc = 0.0f;
    for (int s0 = 0; s0 < count; s0 += 8) {   // eight dims' loads in flight, added in order
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = half_to_f32<F16>(base[sel_idx[min(s0 + j, count - 1)] * dd]);
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (s0 + j < count) acc = acc + sel_q[s0 + j] * v[j];
    }
  }
  out[static_cast<int64_t>(row) * out_ld + p] = acc;
  if (full) {   // the full-D score the rerank ranks its candidates by (every scanned position)
    const bool in = tok >= 0 && tok < history;
    const float f = in ? full_score<F16>(key + b * sb + (h / group) * sh + static_cast<int64_t>(tok) * st, q_s, scaling)
                       : -__builtin_huge_valf();
    full[static_cast<int64_t>(row) * out_ld + p] = f;
  }
}

// ---------------------------------------------------------------------------
// qboracle block scores (EV:5030-5044): per block, the maximum over its
// history tokens of the partial score on the row's top-|q| dims, from the
// dim-major copy (consecutive lanes read consecutive tokens of a dim).  A
// workgroup owns whole blocks, at most kQboTokens tokens, whose scores go
// through LDS to the block maxima -- or, for blocks longer than that, one
// block, each thread keeping the maximum of its tokens and the workgroup
// reducing those.
// ---------------------------------------------------------------------------
constexpr int kQboTokens = kBT * 8;

template <bool F16>
__global__ __launch_bounds__(kBT) void block_max_partial_kernel(
    const uint16_t* __restrict__ query, const uint16_t* __restrict__ kdm, int q_heads, int group, int64_t db,
    int64_t dh, int64_t dd, int history, int block, int nb, int blocks_per_wg, int count, float* __restrict__ out,
    int64_t out_ld) {
  __shared__ float q_s[kHD];
  __shared__ int sel_idx[kHD];
  __shared__ float sel_q[kHD];
  __shared__ float sc[kQboTokens];
  const int row = blockIdx.y, tid = threadIdx.x;
  const int b = row / q_heads, h = row - b * q_heads;
  for (int d = tid; d < kHD; d += kBT) q_s[d] = half_to_f32<F16>(query[static_cast<int64_t>(row) * kHD + d]);
  __syncthreads();
  rank_dims(q_s, count, sel_idx, sel_q);
  const int j0 = blockIdx.x * blocks_per_wg, j1 = min(nb, j0 + blocks_per_wg);
  const int t0 = j0 * block, t1 = min(history, j1 * block);
  const uint16_t* base = kdm + b * db + (h / group) * dh;
  auto score = [&](int t) -> float {
    const uint16_t* kt = base + t;
    float acc = 0.0f;
    for (int s0 = 0; s0 < count; s0 += 8) {   // eight dims' loads in flight, added in order
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = half_to_f32<F16>(kt[sel_idx[min(s0 + e, count - 1)] * dd]);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (s0 + e < count) acc = acc + sel_q[s0 + e] * v[e];
    }
    return acc;
  };
  if (block > kQboTokens) {   // one long block (blocks_per_wg = 1)
    float m = -__builtin_huge_valf();
    for (int t = t0 + tid; t < t1; t += kBT) m = fmaxf(m, score(t));
    sc[tid] = m;
    __syncthreads();
    if (tid == 0) {
      for (int i = 1; i < kBT; ++i) m = fmaxf(m, sc[i]);
      out[static_cast<int64_t>(row) * out_ld + j0] = m;
    }
    return;
  }
  for (int i = tid; i < t1 - t0; i += kBT) sc[i] = score(t0 + i);
  __syncthreads();
  for (int j = j0 + tid; j < j1; j += kBT) {
    const int a = j * block - t0, e = min(t1, (j + 1) * block) - t0;
    float m = -__builtin_huge_valf();
    for (int i = a; i < e; ++i) m = fmaxf(m, sc[i]);
    out[static_cast<int64_t>(row) * out_ld + j] = m;
  }
}

// ---------------------------------------------------------------------------
// Rerank of one row (EV:5583-5605): the n_cand best scanned tokens by partial
// score (-inf positions never taken), their full-D scores * scaling, the
// n_keep best of those, then the final mask over [0, key_count) (the kept
// tokens, the first sink_end and the recent history positions, the current
// token) and the token list for attention: kept tokens (ascending; -1 where
// a kept token lies in a protected range or past the kept count), then the
// sink range, the recent range and the current token.
// ---------------------------------------------------------------------------
template <int VPL1, int VPL2, bool F16>
__global__ __launch_bounds__(kRerankNT) void rerank_kernel(
    const uint16_t* __restrict__ query, const uint16_t* __restrict__ key, int q_heads, int group, int64_t sb,
    int64_t sh, int64_t st, const float* __restrict__ partial, const float* __restrict__ full, int64_t partial_ld,
    const int32_t* __restrict__ blocks, int n_scan, int block, int history, int key_count, int n_cand, int n_keep,
    int sink_end, int recent_start,
    int rec_begin, int n_rec, int keep_self, float scaling, uint8_t* __restrict__ keep_mask, int64_t keep_ld,
    int32_t* __restrict__ attn_ids, int n_out) {
  using WS1 = WideSelect<VPL1, true>;
  using WS2 = WideSelect<VPL2, false>;
  __shared__ union {
    typename WS1::Shared a;
    typename WS2::Shared b;
  } lds;
  __shared__ __attribute__((aligned(16))) float q_s[kHD];
  __shared__ int32_t cand[kMaxCand], cand_pos[kMaxCand];
  const int row = blockIdx.x, tid = threadIdx.x;
  const int b = row / q_heads, h = row - b * q_heads;
  for (int d = tid; d < kHD; d += kRerankNT) q_s[d] = half_to_f32<F16>(query[static_cast<int64_t>(row) * kHD + d]);
  uint8_t* mrow = keep_mask + static_cast<int64_t>(row) * keep_ld;
  // the protected mask, 16 bytes per store where the row is 16-byte aligned
  auto prot = [&](int t) -> uint32_t {
    return (t < sink_end) || (t >= recent_start && t < history) || (keep_self && t == history);
  };
  const int body = (reinterpret_cast<uintptr_t>(mrow) & 15) ? 0 : (key_count & ~15);
  for (int t0 = 16 * tid; t0 < body; t0 += 16 * kRerankNT) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t x = 0;
#pragma unroll
      for (int bb = 0; bb < 4; ++bb) x |= prot(t0 + 4 * j + bb) << (8 * bb);
      w[j] = x;
    }
    *reinterpret_cast<uint4*>(mrow + t0) = make_uint4(w[0], w[1], w[2], w[3]);
  }
  for (int t = body + tid; t < key_count; t += kRerankNT) mrow[t] = prot(t);

  // 1. candidates (the first radix digit counted as the scores arrive)
  WS1 ws1;
  ws1.load_count(partial + static_cast<int64_t>(row) * partial_ld, n_scan * block, lds.a);
  const int kk1 = ws1.run_counted(n_cand, lds.a);
  const int32_t* brow = blocks + static_cast<int64_t>(row) * n_scan;
  auto emit1 = [&](int pos, int o, int) {
    const int jb = pos / block;
    cand[o] = brow[jb] * block + (pos - jb * block);
    cand_pos[o] = pos;
  };
  if constexpr (VPL1 <= 8) ws1.place_uniform(lds.a, emit1);
  else ws1.place(lds.a, emit1);

  // 2. full scores of the candidates (computed by the scan launch when full
  // is given: then only read back here), 3. the kept ones
  WS2 ws2;
  const uint16_t* kb = key + b * sb + (h / group) * sh;
  const float* frow = full ? full + static_cast<int64_t>(row) * partial_ld : nullptr;
  // (place ended with a barrier: lds.b's histogram is cleared for the count)
#pragma unroll
  for (int j = 0; j < WS2::NB / kRerankNT; ++j) lds.b.hist[0][tid + kRerankNT * j] = 0;
  __syncthreads();
  int ninf = 0;
#pragma unroll
  for (int i = 0; i < VPL2; ++i) {
    const int ci = WS2::pos(i);
    const bool ok = ci < kk1;
    float acc = 0.0f;
    if (ok) acc = frow ? frow[cand_pos[ci]] : full_score<F16>(kb + static_cast<int64_t>(cand[ci]) * st, q_s, scaling);
    ws2.set(i, acc, ok);
    ws2.count(i, lds.b, ninf);
  }
  ws2.count_done(lds.b, ninf);
  const int kk2 = ws2.run_counted(n_keep, lds.b);
  int32_t* ids = attn_ids + static_cast<int64_t>(row) * n_out;
  auto emit2 = [&](int ci, int o, int) {
    const int tok = cand[ci];
    mrow[tok] = 1;
    const bool fv = tok >= sink_end && !(tok >= recent_start && tok < history);
    ids[o] = fv ? tok : -1;
  };
  if constexpr (VPL2 <= 8) ws2.place_uniform(lds.b, emit2);
  else ws2.place(lds.b, emit2);
  for (int o = kk2 + tid; o < n_keep; o += kRerankNT) ids[o] = -1;
  const int extra = sink_end + n_rec + keep_self;
  for (int i = tid; i < extra; i += kRerankNT)
    ids[n_keep + i] = i < sink_end ? i : (i < sink_end + n_rec ? rec_begin + (i - sink_end) : key_count - 1);
}

// ---------------------------------------------------------------------------
// The rerank of rows past rerank_kernel's one-workgroup limits (more than
// kMaxScan scanned tokens or kMaxCand candidates), and qboracle rows whose
// candidates run past their scanned tokens, in five launches over a
// workspace:
//   dense_partial_kernel  per history token its candidate score: the partial
//       score where its block was scanned, else `fill` -- finfo(float32).min
//       for qboracle, which ranks every history token and so reaches unscanned
//       ones once the scanned run out (EV:5055-5058), -inf (never a
//       candidate) for qbb / brep;
//   (qkv_topk_ws)         the n_cand best tokens, ascending;
//   cand_full_kernel      their full-D scores * scaling, -inf for -inf picks;
//   (qkv_topk_ws)         the n_keep best candidates;
//   rerank_finish_kernel  mask and token list as rerank_kernel writes them.
// Ties go to the lower token at both selections, as in rerank_kernel
// (ascending positions there are ascending tokens).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kBT) void dense_partial_kernel(const float* __restrict__ partial, int64_t partial_ld,
                                                            const int32_t* __restrict__ blocks, int n_scan,
                                                            int block, int history, float fill,
                                                            float* __restrict__ dense, int64_t dense_ld) {
  const int row = blockIdx.y;
  const int t = blockIdx.x * kBT + threadIdx.x;
  if (t >= history) return;
  const int32_t* br = blocks + static_cast<int64_t>(row) * n_scan;
  const int j = t / block;
  int lo = 0, hi = n_scan;   // the first slot whose block id is >= j (ids ascending)
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (br[mid] < j) lo = mid + 1;
    else hi = mid;
  }
  const bool in = lo < n_scan && br[lo] == j;
  dense[static_cast<int64_t>(row) * dense_ld + t] =
      in ? partial[static_cast<int64_t>(row) * partial_ld + static_cast<int64_t>(lo) * block + (t - j * block)]
         : fill;
}

template <bool F16>
__global__ __launch_bounds__(kBT) void cand_full_kernel(const uint16_t* __restrict__ query,
                                                        const uint16_t* __restrict__ key, int q_heads, int group,
                                                        int64_t sb, int64_t sh, int64_t st,
                                                        const float* __restrict__ dense, int64_t dense_ld,
                                                        const int32_t* __restrict__ cand, int n_cand, float scaling,
                                                        float* __restrict__ cf) {
  __shared__ __attribute__((aligned(16))) float q_s[kHD];
  const int row = blockIdx.y, tid = threadIdx.x;
  const int b = row / q_heads, h = row - b * q_heads;
  for (int d = tid; d < kHD; d += kBT) q_s[d] = half_to_f32<F16>(query[static_cast<int64_t>(row) * kHD + d]);
  __syncthreads();
  const int i = blockIdx.x * kBT + tid;
  if (i >= n_cand) return;
  const int tok = cand[static_cast<int64_t>(row) * n_cand + i];
  const bool ok = dense[static_cast<int64_t>(row) * dense_ld + tok] != -__builtin_huge_valf();
  cf[static_cast<int64_t>(row) * n_cand + i] =
      ok ? full_score<F16>(key + b * sb + (h / group) * sh + static_cast<int64_t>(tok) * st, q_s, scaling)
         : -__builtin_huge_valf();
}

// One workgroup per row: the protected mask, then the kept candidates (kept
// holds ascending indices into the row's ascending candidate tokens) in
// order with the -inf picks dropped, -1 padding, and the protected tail.
__global__ __launch_bounds__(kRerankNT) void rerank_finish_kernel(
    const int32_t* __restrict__ cand, const float* __restrict__ cf, int n_cand, const int32_t* __restrict__ kept,
    int n_kept, int n_keep, int history, int key_count, int sink_end, int recent_start, int rec_begin, int n_rec,
    int keep_self, uint8_t* __restrict__ keep_mask, int64_t keep_ld, int32_t* __restrict__ attn_ids, int n_out) {
  constexpr int NW = kRerankNT / 64;
  __shared__ int wave_cnt[NW];
  __shared__ int base_s;
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint8_t* mrow = keep_mask + static_cast<int64_t>(row) * keep_ld;
  for (int t = tid; t < key_count; t += kRerankNT)
    mrow[t] = (t < sink_end) || (t >= recent_start && t < history) || (keep_self && t == history);
  if (tid == 0) base_s = 0;
  __syncthreads();
  int32_t* ids = attn_ids + static_cast<int64_t>(row) * n_out;
  const int32_t* krow = kept + static_cast<int64_t>(row) * n_kept;
  const int32_t* crow = cand + static_cast<int64_t>(row) * n_cand;
  const float* frow = cf + static_cast<int64_t>(row) * n_cand;
  for (int o0 = 0; o0 < n_kept; o0 += kRerankNT) {
    const int o = o0 + tid;
    int tok = -1;
    bool ok = false;
    if (o < n_kept) {
      const int ci = krow[o];
      ok = frow[ci] != -__builtin_huge_valf();
      tok = crow[ci];
    }
    const uint64_t m = __ballot(ok);
    if (lane == 0) wave_cnt[wave] = __popcll(m);
    __syncthreads();
    int at = base_s + __popcll(m & ((uint64_t(1) << lane) - 1));
    for (int w = 0; w < wave; ++w) at += wave_cnt[w];
    if (ok) {
      mrow[tok] = 1;
      ids[at] = (tok >= sink_end && !(tok >= recent_start && tok < history)) ? tok : -1;
    }
    __syncthreads();
    if (tid == 0) {
      int sum = 0;
      for (int w = 0; w < NW; ++w) sum += wave_cnt[w];
      base_s += sum;
    }
    __syncthreads();
  }
  for (int o = base_s + tid; o < n_keep; o += kRerankNT) ids[o] = -1;
  const int extra = sink_end + n_rec + keep_self;
  for (int i = tid; i < extra; i += kRerankNT)
    ids[n_keep + i] = i < sink_end ? i : (i < sink_end + n_rec ? rec_begin + (i - sink_end) : key_count - 1);
}

// ---------------------------------------------------------------------------
// brep_partial_scores, the kernel the reference imports but never shipped
// (wrapper EV:3847-3877, used at EV:5419-5431): the partial score of every
// history token on the row's top-|q| dims (fp32 query, K in its own dtype,
// products and sums in selection order), then -inf on every token outside
// the scanned blocks -- the n_scan blocks whose best valid representative
// scores highest (ties to the lower block), as the reference's fallback
// ranks them (EV:5431-5443).
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(kBT) void brep_token_scores_kernel(
    const float* __restrict__ query, const typename Elem<DT>::T* __restrict__ key, float* __restrict__ out,
    int heads, int tokens, int head_dim, int count, int64_t ksb, int64_t ksh, int64_t kst) {
  __shared__ int sel_idx[kMaxDims];
  __shared__ float sel_q[kMaxDims];
  const int row = blockIdx.y;
  const int b = row / heads, h = row - b * heads;
  select_dims<QKV_DTYPE_FP32>(query + static_cast<int64_t>(row) * head_dim, head_dim, count, sel_idx, sel_q);
  __syncthreads();
  const int t = blockIdx.x * kBT + threadIdx.x;
  if (t >= tokens) return;
  const typename Elem<DT>::T* k_row = key + b * ksb + h * ksh + t * kst;
  float acc = 0.0f;
  for (int s = 0; s < count; ++s) acc = acc + sel_q[s] * Elem<DT>::load(k_row + sel_idx[s]);
  out[static_cast<int64_t>(row) * tokens + t] = acc;
}

constexpr int kBrepMaxBlocks = kRerankNT * 40;

// One 1024-thread workgroup per row: block scores from the token scores of
// the representatives (finfo(float32).min without a valid one), the n_scan
// best blocks into an LDS bitmap, then -inf on the tokens of every other
// block.  Every read of the row's scores happens before the selection's
// first barrier, every write after its last one.
template <int VPL>
__global__ __launch_bounds__(kRerankNT) void brep_scan_mask_kernel(float* __restrict__ scores, int tokens,
                                                                   const int64_t* __restrict__ rep_idx,
                                                                   const uint8_t* __restrict__ rep_valid,
                                                                   int reps, int block, int nb, int n_scan) {
  using WS = WideSelect<VPL, false>;
  __shared__ typename WS::Shared lds;
  __shared__ uint32_t scanned[kBrepMaxBlocks / 32];
  const int row = blockIdx.x, tid = threadIdx.x;
  float* srow = scores + static_cast<int64_t>(row) * tokens;
  const int64_t* irow = rep_idx + static_cast<int64_t>(row) * nb * reps;
  const uint8_t* vrow = rep_valid + static_cast<int64_t>(row) * nb * reps;
  for (int w = tid; w < (nb + 31) / 32; w += kRerankNT) scanned[w] = 0u;
  WS ws;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int j = WS::pos(i);
    float best = -3.40282347e38f;   // finfo(float32).min
    if (j < nb) {
      for (int r = 0; r < reps; ++r) {
        const int64_t e = static_cast<int64_t>(j) * reps + r;
        const int64_t tok = irow[e];
        if (vrow[e] && tok >= 0 && tok < tokens) best = fmaxf(best, srow[tok]);
      }
    }
    ws.set(i, best, j < nb);
  }
  ws.run(n_scan, lds);
  ws.place(lds, [&](int pos, int, int) { atomicOr(&scanned[pos >> 5], 1u << (pos & 31)); });
  __syncthreads();
  for (int t = tid; t < tokens; t += kRerankNT) {
    const int j = t / block;
    if (!((scanned[j >> 5] >> (j & 31)) & 1u)) srow[t] = -__builtin_huge_valf();
  }
}

template <int DT> struct RunBrepTokens {
  static int run(const float* q, const void* k, float* out, int64_t B, int64_t H, int64_t T, int64_t D,
                 const int64_t* ks, int count, hipStream_t st) {
    dim3 grid(static_cast<unsigned>(cdiv(T, kBT)), static_cast<unsigned>(B * H));
    brep_token_scores_kernel<DT><<<grid, kBT, 0, st>>>(q, static_cast<const typename Elem<DT>::T*>(k), out,
                                                       static_cast<int>(H), static_cast<int>(T),
                                                       static_cast<int>(D), count, ks[0], ks[1], ks[2]);
    return check_launch("qkv_brep_partial_scores");
  }
};

// Keys per thread for rows of n scanned tokens / n candidates: the fewest
// that hold the row, so short rows run short loops.
template <typename F>
int with_scan_vpl(int64_t n, F&& f) {
  if (n <= kRerankNT) return f(std::integral_constant<int, 1>{});
  if (n <= 2 * kRerankNT) return f(std::integral_constant<int, 2>{});
  if (n <= 4 * kRerankNT) return f(std::integral_constant<int, 4>{});
  if (n <= 8 * kRerankNT) return f(std::integral_constant<int, 8>{});
  if (n <= 16 * kRerankNT) return f(std::integral_constant<int, 16>{});
  if (n <= 32 * kRerankNT) return f(std::integral_constant<int, 32>{});
  return f(std::integral_constant<int, 40>{});
}

template <typename F>
int with_cand_vpl(int64_t n, F&& f) {
  if (n <= kRerankNT) return f(std::integral_constant<int, 1>{});
  if (n <= 2 * kRerankNT) return f(std::integral_constant<int, 2>{});
  return f(std::integral_constant<int, 4>{});
}

int check_rows(const char* what, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim) {
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads)
    return fail(QKV_ERR_INVALID, "%s: need batch > 0 and q_heads a positive multiple of kv_heads", what);
  if (batch * q_heads > 65535) return fail(QKV_ERR_INVALID, "%s: batch * q_heads must be <= 65535", what);
  if (head_dim != kHD) return fail(QKV_ERR_UNSUPPORTED, "%s: head_dim must be 128", what);
  return QKV_OK;
}

bool kv_aligned(const void* p, const int64_t* s) { return aligned(p, 16) && (s[0] | s[1] | s[2]) % 8 == 0; }

// Whether every row's rerank fits rerank_kernel: at most kMaxScan scanned
// positions and kMaxCand candidates, and (qboracle, whose candidates may be
// unscanned tokens) no more candidates than the fewest scanned history
// tokens a row can have -- then every row's candidates are scanned tokens.
bool rerank_fits(int64_t history, int64_t n_scan, int64_t block, int64_t n_cand, bool unscanned) {
  if (n_scan * block > kMaxScan || n_cand > kMaxCand) return false;
  if (!unscanned) return true;
  const int64_t fewest = n_scan * block - (cdiv(history, block) * block - history);
  return n_cand <= fewest;
}

// Workspace of the general rerank: dense scores [rows, dense_ld], candidate
// tokens and their full scores [rows, n1], kept indices [rows, n2], then the
// top-k workspace shared by both selections; 256-byte aligned parts.
struct WideRerank {
  int64_t dense_ld, n1, n2, off_cand, off_cf, off_kept, off_topk, topk_bytes, total;
};

WideRerank wide_rerank_layout(int64_t rows, int64_t history, int64_t n_cand, int64_t n_keep) {
  auto al = [](int64_t x) { return cdiv(x, 256) * 256; };
  WideRerank w;
  w.dense_ld = cdiv(history, 64) * 64;
  w.n1 = std::min(n_cand, history);
  w.n2 = std::min(n_keep, w.n1);
  int64_t off = al(rows * w.dense_ld * 4);
  w.off_cand = off;
  off += al(rows * w.n1 * 4);
  w.off_cf = off;
  off += al(rows * w.n1 * 4);
  w.off_kept = off;
  off += al(rows * w.n2 * 4);
  w.off_topk = off;
  w.topk_bytes = std::max(qkv_topk_workspace_bytes(rows, history, w.n1), qkv_topk_workspace_bytes(rows, w.n1, w.n2));
  w.total = off + al(std::max<int64_t>(w.topk_bytes, 0));
  return w;
}

}  // namespace
}  // namespace qkv

using namespace qkv;

QKV_EXPORT int64_t qkv_block_meta_bytes(int kind, int64_t batch, int64_t kv_heads, int64_t meta_blocks,
                                        int64_t reps) {
  if (batch <= 0 || kv_heads <= 0 || meta_blocks <= 0) return -1;
  if (kind == QKV_BLOCK_QBB) return batch * kv_heads * meta_blocks * 2 * kHD * 2;
  if (kind == QKV_BLOCK_BREP && reps >= 1 && reps <= 64) return batch * kv_heads * meta_blocks * reps * 4;
  return -1;
}

QKV_EXPORT int qkv_block_meta_update(int kind, const void* key, const int64_t* k_strides, int64_t batch,
                                     int64_t kv_heads, int64_t head_dim, int64_t block, int64_t reps, int64_t t_begin,
                                     int64_t t_end, void* meta, int64_t meta_blocks, int dtype, void* stream) {
  const char* what = "qkv_block_meta_update";
  if (!key || !k_strides || !meta) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  bool f16;
  if (int rc = half_dtype(dtype, what, &f16)) return rc;
  if (batch <= 0 || kv_heads <= 0 || batch * kv_heads > 65535 || head_dim != kHD)
    return fail(QKV_ERR_INVALID, "%s: need batch, kv_heads > 0 and head_dim 128", what);
  if (block <= 0 || t_begin < 0 || t_end < t_begin || cdiv(t_end, block) > meta_blocks || t_end >= (int64_t(1) << 31))
    return fail(QKV_ERR_INVALID, "%s: need block > 0, 0 <= t_begin <= t_end, ceil(t_end/block) <= meta_blocks", what);
  if (k_strides[3] != 1 || !kv_aligned(key, k_strides))
    return fail(QKV_ERR_INVALID, "%s: K rows must be contiguous and 16-byte aligned", what);
  if (t_end == t_begin) return QKV_OK;
  const int64_t j0 = t_begin / block, j1 = cdiv(t_end, block);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* k = static_cast<const uint16_t*>(key);
  if (kind != QKV_BLOCK_QBB && kind != QKV_BLOCK_BREP)
    return fail(QKV_ERR_INVALID, "%s: unknown selector kind %d", what, kind);
  if (kind == QKV_BLOCK_BREP && (reps < 1 || reps > 64 || reps > block))
    return fail(QKV_ERR_INVALID, "%s: brep needs 1 <= reps <= min(block, 64)", what);
  return with_half(f16, [&](auto ff) {
    constexpr bool F = decltype(ff)::value;
    if (kind == QKV_BLOCK_QBB) {
      dim3 grid(static_cast<unsigned>(j1 - j0), static_cast<unsigned>(batch * kv_heads));
      qbb_meta_kernel<F><<<grid, kBT, 0, st>>>(k, static_cast<int>(kv_heads), k_strides[0], k_strides[1],
                                               k_strides[2], static_cast<int>(block), static_cast<int>(t_end),
                                               static_cast<int>(j0), static_cast<uint16_t*>(meta), meta_blocks);
    } else if (block <= 64) {
      dim3 grid(static_cast<unsigned>(cdiv(j1 - j0, kBT / 64)), static_cast<unsigned>(batch * kv_heads));
      brep_meta_kernel<F><<<grid, kBT, 0, st>>>(k, static_cast<int>(kv_heads), k_strides[0], k_strides[1],
                                                k_strides[2], static_cast<int>(block), static_cast<int>(reps),
                                                static_cast<int>(t_end), static_cast<int>(j0), static_cast<int>(j1),
                                                static_cast<int32_t*>(meta), meta_blocks);
    } else {
      dim3 grid(static_cast<unsigned>(j1 - j0), static_cast<unsigned>(batch * kv_heads));
      brep_meta_wide_kernel<F><<<grid, kRepNT, 0, st>>>(k, static_cast<int>(kv_heads), k_strides[0], k_strides[1],
                                                        k_strides[2], static_cast<int>(block), static_cast<int>(reps),
                                                        static_cast<int>(t_end), static_cast<int>(j0),
                                                        static_cast<int32_t*>(meta), meta_blocks);
    }
    return check_launch(what);
  });
}

QKV_EXPORT int qkv_block_scores(int kind, const void* query, const void* key, const int64_t* k_strides,
                                const void* meta, int64_t meta_blocks, int64_t batch, int64_t q_heads,
                                int64_t kv_heads, int64_t history, int64_t head_dim, int64_t block, int64_t reps,
                                int64_t dim_count, float* out, int64_t out_ld, int dtype, void* stream) {
  const char* what = "qkv_block_scores";
  int rc = check_rows(what, batch, q_heads, kv_heads, head_dim);
  if (rc) return rc;
  bool f16;
  if ((rc = half_dtype(dtype, what, &f16))) return rc;
  if (!query || !key || !k_strides || !meta || !out) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  const int64_t nb = block > 0 ? cdiv(history, block) : 0;
  if (history <= 0 || block <= 0 || nb > meta_blocks || out_ld < nb || history >= (int64_t(1) << 31))
    return fail(QKV_ERR_INVALID, "%s: need history, block > 0, ceil(history/block) <= meta_blocks and out_ld", what);
  if (kind == QKV_BLOCK_BREP && (reps < 1 || reps > 64)) return fail(QKV_ERR_INVALID, "%s: reps in [1, 64]", what);
  if (k_strides[3] != 1) return fail(QKV_ERR_UNSUPPORTED, "%s: K channels must be contiguous", what);
  const int count = static_cast<int>(std::min<int64_t>(std::max<int64_t>(dim_count, 1), kHD));
  dim3 grid(static_cast<unsigned>(cdiv(nb, kBT)), static_cast<unsigned>(batch * q_heads));
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (kind != QKV_BLOCK_QBB && kind != QKV_BLOCK_BREP)
    return fail(QKV_ERR_INVALID, "%s: unknown selector kind %d", what, kind);
#define QKV_BLOCK_SCORES(K, F)                                                                                 \
  block_scores_kernel<K, F><<<grid, kBT, 0, st>>>(                                                             \
      static_cast<const uint16_t*>(query), static_cast<const uint16_t*>(key), static_cast<int>(q_heads),       \
      static_cast<int>(q_heads / kv_heads), static_cast<int>(kv_heads), k_strides[0], k_strides[1], k_strides[2], \
      meta, meta_blocks, static_cast<int>(reps), static_cast<int>(nb), count, out, out_ld)
  return with_half(f16, [&](auto ff) {
    constexpr bool F = decltype(ff)::value;
    if (kind == QKV_BLOCK_QBB) QKV_BLOCK_SCORES(0, F);
    else QKV_BLOCK_SCORES(1, F);
    return check_launch(what);
  });
#undef QKV_BLOCK_SCORES
}

QKV_EXPORT int qkv_block_scan_scores(const void* query, const void* key_dim_major, const int64_t* kdm_strides,
                                     const void* key, const int64_t* k_strides, int64_t batch, int64_t q_heads,
                                     int64_t kv_heads, int64_t history, int64_t head_dim, const int32_t* blocks,
                                     int64_t n_scan, int64_t block, int64_t dim_count, float scaling, float* out,
                                     float* full, int64_t out_ld, int dtype, void* stream) {
  const char* what = "qkv_block_scan_scores";
  int rc = check_rows(what, batch, q_heads, kv_heads, head_dim);
  if (rc) return rc;
  bool f16;
  if ((rc = half_dtype(dtype, what, &f16))) return rc;
  if (!query || !key_dim_major || !kdm_strides || !blocks || !out) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  if (history <= 0 || block <= 0 || n_scan <= 0 || n_scan * block >= (int64_t(1) << 30) || out_ld < n_scan * block)
    return fail(QKV_ERR_INVALID, "%s: need history, block, n_scan > 0 and out_ld >= n_scan * block", what);
  if (kdm_strides[3] != 1) return fail(QKV_ERR_UNSUPPORTED, "%s: the copy's token axis must be contiguous", what);
  if (full && (!key || !k_strides)) return fail(QKV_ERR_INVALID, "%s: full scores need key and k_strides", what);
  if (full && (k_strides[3] != 1 || !kv_aligned(key, k_strides)))
    return fail(QKV_ERR_INVALID, "%s: K rows must be contiguous and 16-byte aligned", what);
  const int count = static_cast<int>(std::min<int64_t>(std::max<int64_t>(dim_count, 1), kHD));
  dim3 grid(static_cast<unsigned>(cdiv(n_scan * block, kBT)), static_cast<unsigned>(batch * q_heads));
  return with_half(f16, [&](auto ff) {
    scan_partial_kernel<decltype(ff)::value><<<grid, kBT, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint16_t*>(query), static_cast<const uint16_t*>(key_dim_major), static_cast<int>(q_heads),
        static_cast<int>(q_heads / kv_heads), kdm_strides[0], kdm_strides[1], kdm_strides[2], blocks,
        static_cast<int>(n_scan), static_cast<int>(block), static_cast<int>(history), count, out, out_ld,
        static_cast<const uint16_t*>(key), full ? k_strides[0] : 0, full ? k_strides[1] : 0,
        full ? k_strides[2] : 0, scaling, full);
    return check_launch(what);
  });
}

QKV_EXPORT int qkv_block_max_partial_scores(const void* query, const void* key_dim_major, const int64_t* kdm_strides,
                                            int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t history,
                                            int64_t head_dim, int64_t block, int64_t dim_count, float* out,
                                            int64_t out_ld, int dtype, void* stream) {
  const char* what = "qkv_block_max_partial_scores";
  int rc = check_rows(what, batch, q_heads, kv_heads, head_dim);
  if (rc) return rc;
  bool f16;
  if ((rc = half_dtype(dtype, what, &f16))) return rc;
  if (!query || !key_dim_major || !kdm_strides || !out) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  const int64_t nb = block > 0 ? cdiv(history, block) : 0;
  if (history <= 0 || history >= (int64_t(1) << 31) || block <= 0 || out_ld < nb)
    return fail(QKV_ERR_INVALID, "%s: need history, block > 0 and out_ld >= ceil(history/block)", what);
  if (kdm_strides[3] != 1) return fail(QKV_ERR_UNSUPPORTED, "%s: the copy's token axis must be contiguous", what);
  const int count = static_cast<int>(std::min<int64_t>(std::max<int64_t>(dim_count, 1), kHD));
  const int64_t per_wg = std::max<int64_t>(1, kQboTokens / block);
  dim3 grid(static_cast<unsigned>(cdiv(nb, per_wg)), static_cast<unsigned>(batch * q_heads));
  return with_half(f16, [&](auto ff) {
    block_max_partial_kernel<decltype(ff)::value><<<grid, kBT, 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint16_t*>(query), static_cast<const uint16_t*>(key_dim_major), static_cast<int>(q_heads),
        static_cast<int>(q_heads / kv_heads), kdm_strides[0], kdm_strides[1], kdm_strides[2],
        static_cast<int>(history), static_cast<int>(block), static_cast<int>(nb), static_cast<int>(per_wg), count,
        out, out_ld);
    return check_launch(what);
  });
}

QKV_EXPORT int qkv_brep_partial_scores(const float* query, const void* key_history, const int64_t* rep_indices,
                                       const uint8_t* rep_valid, float* out, int key_dtype, int64_t batch,
                                       int64_t heads, int64_t history, int64_t head_dim, const int64_t* k_strides,
                                       int64_t reps, int64_t block_size, int64_t dim_count, double scan_fraction,
                                       void* stream) {
  const char* what = "qkv_brep_partial_scores";
  if (!query || !key_history || !rep_indices || !rep_valid || !out || !k_strides)
    return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  if (batch <= 0 || heads <= 0 || batch * heads > 65535)
    return fail(QKV_ERR_INVALID, "%s: need batch, heads > 0 and batch * heads <= 65535", what);
  if (head_dim <= 0 || head_dim > 1024) return fail(QKV_ERR_INVALID, "%s: need 0 < head_dim <= 1024", what);
  if (history <= 0 || history >= (int64_t(1) << 31) || block_size <= 0 || reps <= 0)
    return fail(QKV_ERR_INVALID, "%s: need history, block_size, reps > 0", what);
  if (scan_fraction != scan_fraction) return fail(QKV_ERR_INVALID, "%s: scan_fraction is NaN", what);
  const int64_t nb = cdiv(history, block_size);
  if (nb > kBrepMaxBlocks)
    return fail(QKV_ERR_UNSUPPORTED, "%s: at most %d blocks per row (got %lld)", what, kBrepMaxBlocks, (long long)nb);
  if (k_strides[3] != 1) return fail(QKV_ERR_UNSUPPORTED, "%s: K channels must be contiguous", what);
  // min(blocks, max(1, ceil(scan_fraction * history / block_size))) in double, as EV:5442 computes it
  const double want = std::ceil(scan_fraction * static_cast<double>(history) / static_cast<double>(block_size));
  const int64_t n_scan = want >= static_cast<double>(nb) ? nb : want < 1.0 ? 1 : static_cast<int64_t>(want);
  const int count = static_cast<int>(std::min<int64_t>(std::max<int64_t>(dim_count, 1), std::min<int64_t>(head_dim, kMaxDims)));
  hipStream_t st = static_cast<hipStream_t>(stream);
  int rc = dispatch_dtype<RunBrepTokens>(key_dtype, query, key_history, out, batch, heads, history, head_dim,
                                         k_strides, count, st);
  if (rc != QKV_OK) return rc;
  return with_scan_vpl(nb, [&](auto vpl) {
    brep_scan_mask_kernel<decltype(vpl)::value><<<static_cast<unsigned>(batch * heads), kRerankNT, 0, st>>>(
        out, static_cast<int>(history), rep_indices, rep_valid, static_cast<int>(reps), static_cast<int>(block_size),
        static_cast<int>(nb), static_cast<int>(n_scan));
    return check_launch(what);
  });
}

QKV_EXPORT int64_t qkv_final_list_count(int64_t history, int64_t n_keep, int64_t protect_sink, int64_t protect_recent,
                                        int keep_self) {
  if (history <= 0 || n_keep < 0) return -1;
  const int64_t sink_end = protect_sink > 0 ? std::min(protect_sink, history) : 0;
  const int64_t recent_start = protect_recent > 0 ? std::max<int64_t>(0, history - protect_recent) : history;
  const int64_t rec_begin = std::max(recent_start, sink_end);
  const int64_t n_rec = (protect_recent > 0 && rec_begin < history) ? history - rec_begin : 0;
  return n_keep + sink_end + n_rec + (keep_self ? 1 : 0);
}

QKV_EXPORT int64_t qkv_block_rerank_workspace_bytes(int64_t rows, int64_t history, int64_t n_scan, int64_t block,
                                                    int64_t n_cand, int64_t n_keep, int unscanned) {
  if (rows <= 0 || rows > 65535 || history <= 0 || history >= (int64_t(1) << 31) || n_scan <= 0 || block <= 0 ||
      n_cand < 1 || n_keep < 1 || n_keep > n_cand)
    return -1;
  if (rerank_fits(history, n_scan, block, n_cand, unscanned != 0)) return 0;
  return wide_rerank_layout(rows, history, n_cand, n_keep).total;
}

QKV_EXPORT int qkv_block_rerank(const void* query, const void* key, const int64_t* k_strides, int64_t batch,
                                int64_t q_heads, int64_t kv_heads, int64_t key_count, int64_t head_dim,
                                const float* partial, const float* full, int64_t partial_ld, const int32_t* blocks,
                                int64_t n_scan, int64_t block, int64_t n_cand, int64_t n_keep, int64_t protect_sink,
                                int64_t protect_recent, int keep_self, float scaling, uint8_t* keep_mask,
                                int64_t keep_ld, int32_t* attn_ids, int64_t n_out, int unscanned, void* workspace,
                                int64_t workspace_bytes, int dtype, void* stream) {
  const char* what = "qkv_block_rerank";
  int rc = check_rows(what, batch, q_heads, kv_heads, head_dim);
  if (rc) return rc;
  bool f16;
  if ((rc = half_dtype(dtype, what, &f16))) return rc;
  if (!query || !key || !k_strides || !partial || !blocks || !keep_mask || !attn_ids)
    return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  const int64_t history = key_count - 1;
  if (history <= 0 || key_count >= (int64_t(1) << 31) || keep_ld < key_count)
    return fail(QKV_ERR_INVALID, "%s: need 2 <= key_count < 2^31 and keep_ld >= key_count", what);
  if (block <= 0 || n_scan <= 0 || n_scan * block >= (int64_t(1) << 30) || partial_ld < n_scan * block)
    return fail(QKV_ERR_INVALID, "%s: need block, n_scan > 0 and partial_ld >= n_scan * block < 2^30", what);
  if (n_cand < 1 || n_keep < 1 || n_keep > n_cand)
    return fail(QKV_ERR_INVALID, "%s: need 1 <= n_keep <= n_cand", what);
  if (k_strides[3] != 1 || !kv_aligned(key, k_strides))
    return fail(QKV_ERR_INVALID, "%s: K rows must be contiguous and 16-byte aligned", what);
  const int64_t sink_end = protect_sink > 0 ? std::min(protect_sink, history) : 0;
  const int64_t recent_start = protect_recent > 0 ? std::max<int64_t>(0, history - protect_recent) : history;
  const int64_t rec_begin = std::max(recent_start, sink_end);
  const int64_t n_rec = (protect_recent > 0 && rec_begin < history) ? history - rec_begin : 0;
  if (n_out != n_keep + sink_end + n_rec + (keep_self ? 1 : 0))
    return fail(QKV_ERR_INVALID, "%s: token lists hold %lld entries, the selection needs %lld", what,
                (long long)n_out, (long long)(n_keep + sink_end + n_rec + (keep_self ? 1 : 0)));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int rows = static_cast<int>(batch * q_heads);
  if (!rerank_fits(history, n_scan, block, n_cand, unscanned != 0)) {
    const WideRerank w = wide_rerank_layout(rows, history, n_cand, n_keep);
    if (!workspace || !aligned(workspace, 256) || workspace_bytes < w.total)
      return fail(QKV_ERR_INVALID, "%s: this rerank needs a 256-byte aligned workspace of %lld bytes, got %lld",
                  what, (long long)w.total, (long long)workspace_bytes);
    char* ws = static_cast<char*>(workspace);
    float* dense = reinterpret_cast<float*>(ws);
    int32_t* cand = reinterpret_cast<int32_t*>(ws + w.off_cand);
    float* cf = reinterpret_cast<float*>(ws + w.off_cf);
    int32_t* kept = reinterpret_cast<int32_t*>(ws + w.off_kept);
    void* tws = ws + w.off_topk;
    const float fill = unscanned ? -3.40282347e38f : -__builtin_huge_valf();   // finfo(float32).min / -inf
    dense_partial_kernel<<<dim3(static_cast<unsigned>(cdiv(history, kBT)), rows), kBT, 0, st>>>(
        partial, partial_ld, blocks, static_cast<int>(n_scan), static_cast<int>(block), static_cast<int>(history),
        fill, dense, w.dense_ld);
    if ((rc = check_launch(what))) return rc;
    if ((rc = qkv_topk_ws(dense, rows, history, w.dense_ld, w.n1, cand, tws, w.topk_bytes, stream))) return rc;
    rc = with_half(f16, [&](auto ff) {
      cand_full_kernel<decltype(ff)::value><<<dim3(static_cast<unsigned>(cdiv(w.n1, kBT)), rows), kBT, 0, st>>>(
          static_cast<const uint16_t*>(query), static_cast<const uint16_t*>(key), static_cast<int>(q_heads),
          static_cast<int>(q_heads / kv_heads), k_strides[0], k_strides[1], k_strides[2], dense, w.dense_ld, cand,
          static_cast<int>(w.n1), scaling, cf);
      return check_launch(what);
    });
    if (rc) return rc;
    if ((rc = qkv_topk_ws(cf, rows, w.n1, w.n1, w.n2, kept, tws, w.topk_bytes, stream))) return rc;
    rerank_finish_kernel<<<static_cast<unsigned>(rows), kRerankNT, 0, st>>>(
        cand, cf, static_cast<int>(w.n1), kept, static_cast<int>(w.n2), static_cast<int>(n_keep),
        static_cast<int>(history), static_cast<int>(key_count), static_cast<int>(sink_end),
        static_cast<int>(recent_start), static_cast<int>(rec_begin), static_cast<int>(n_rec), keep_self ? 1 : 0,
        keep_mask, keep_ld, attn_ids, static_cast<int>(n_out));
    return check_launch(what);
  }
  return with_scan_vpl(n_scan * block, [&](auto vpl) {
   return with_cand_vpl(n_cand, [&](auto vpl2) {
    return with_half(f16, [&](auto ff) {
    rerank_kernel<decltype(vpl)::value, decltype(vpl2)::value, decltype(ff)::value>
        <<<static_cast<unsigned>(batch * q_heads), kRerankNT, 0, st>>>(
        static_cast<const uint16_t*>(query), static_cast<const uint16_t*>(key), static_cast<int>(q_heads),
        static_cast<int>(q_heads / kv_heads), k_strides[0], k_strides[1], k_strides[2], partial, full, partial_ld,
        blocks,
        static_cast<int>(n_scan), static_cast<int>(block), static_cast<int>(history), static_cast<int>(key_count),
        static_cast<int>(n_cand), static_cast<int>(n_keep), static_cast<int>(sink_end),
        static_cast<int>(recent_start), static_cast<int>(rec_begin), static_cast<int>(n_rec), keep_self ? 1 : 0,
        scaling, keep_mask, keep_ld, attn_ids, static_cast<int>(n_out));
    return check_launch(what);
    });
   });
  });
}
