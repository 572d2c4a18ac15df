// Lagged candidate reuse: the refresh tests and the candidate union of the
// reference's lagtop2 / lagrefresh{N} / qdrift[maj|head|share|cos|coshead] /
// pconf{T} modes (EV:4020-4198), ahead of the exact rerank of the union
// (qkv_reuse_select).  A row is one (sequence, query head) r = b * Hq + h.
//
//   lag_flags_kernel      one workgroup per row: the row's top-|q| dims and
//                         their q values (the state the next step compares
//                         with), then the row's refresh test: top-dim overlap,
//                         or overlap or cosine;
//   lag_ess_kernel        the pconf test, a row's positions split over several
//   lag_ess_merge_kernel  workgroups, then merged: the effective sample size of
//                         the attention weights over the previous final
//                         selection;
//   lag_union_kernel      16 positions of one row per thread (a workgroup per
//                         4096 positions of a row): keeps the current
//                         candidates of the rows that refresh (zeroes the
//                         others) and writes the union with the previous final
//                         mask, the candidates shared across heads
//                         (qdriftshare) and the sink / recent ranges.
// The step-wide decisions (any / majority of the flags) are taken inside the
// union kernel, so a step needs no host round trip.  EV = ymluo/projects/
// qwen3_top2_head_limit3_ppl/src/evaluate_qwen3_top2_head_limit3_ppl.py.
#include <math.h>

#include "ref_common.h"

namespace qkv {
namespace {

constexpr int kLagNT = 256;                    // threads per workgroup (4 waves)
constexpr int kLagWaves = kLagNT / 64;
constexpr int kLagPass = kLagNT * 16;          // ESS: mask positions per pass (16 per thread)
constexpr int kLagWGs = 1024;                  // ESS: target workgroups (rows x splits)
constexpr int kUnionChunk = 16;                // union: positions per thread

// Bit j set when byte j of the 16 bytes is nonzero.
__device__ __forceinline__ uint32_t nonzero_bytes(uint4 w) {
  const uint32_t v[4] = {w.x, w.y, w.z, w.w};
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) m |= ((v[i] >> (8 * j)) & 0xFFu ? 1u : 0u) << (4 * i + j);
  return m;
}

template <int DT>
__global__ __launch_bounds__(kLagNT) void lag_flags_kernel(
    const typename Elem<DT>::T* __restrict__ query, int head_dim, int count, int test,
    const int32_t* __restrict__ prev_dims, const float* __restrict__ prev_vals, int32_t* __restrict__ dims_out,
    float* __restrict__ vals_out, uint8_t* __restrict__ flags) {
  using E = typename Elem<DT>::T;
  __shared__ float q_s[128];
  __shared__ __attribute__((aligned(16))) uint64_t key_s[128];
  __shared__ int sel_idx[128];
  __shared__ float sel_q[128];
  __shared__ int pd_s[128];
  __shared__ int cnt_s[kLagWaves];
  __shared__ float red_s[3][kLagWaves];
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const E* q_row = query + static_cast<int64_t>(row) * head_dim;
  for (int d = tid; d < 128; d += kLagNT) q_s[d] = d < head_dim ? Elem<DT>::load(q_row + d) : 0.f;
  if (test != QKV_LAG_DIMS)   // the previous dims load beside q (published by the ranking's barriers)
    for (int s = tid; s < count; s += kLagNT)
      pd_s[s] = min(max(prev_dims[static_cast<int64_t>(row) * count + s], 0), head_dim - 1);
  __syncthreads();
  // the step's top-|q| dims, descending |q| with ties to the lower dim, and
  // q at them (EV:4026-4027, recorded at EV:4384-4393)
  rank_dims128(q_s, key_s, head_dim, count, sel_idx, sel_q);
  for (int s = tid; s < count; s += kLagNT) {
    dims_out[static_cast<int64_t>(row) * count + s] = sel_idx[s];
    vals_out[static_cast<int64_t>(row) * count + s] = sel_q[s];
  }
  if (test == QKV_LAG_DIMS) return;
  {
    // current dims found among the previous ones (EV:4047-4048)
    int hit = 0;
    for (int s = tid; s < count; s += kLagNT) {
      const int d = sel_idx[s];
      bool found = false;
      for (int j = 0; j < count; ++j) found |= pd_s[j] == d;
      hit += found ? 1 : 0;
    }
    // q on the previous dims against the previous values (EV:4049-4056)
    float num = 0.f, na = 0.f, nb = 0.f;
    if (test == QKV_LAG_COS)
      for (int s = tid; s < count; s += kLagNT) {
        const float a = q_s[pd_s[s]], b = prev_vals[static_cast<int64_t>(row) * count + s];
        num += a * b;
        na += a * a;
        nb += b * b;
      }
    hit = wave_sum_i(hit);
    num = wave_sum(num);
    na = wave_sum(na);
    nb = wave_sum(nb);
    if (lane == 0) {
      cnt_s[wave] = hit;
      red_s[0][wave] = num;
      red_s[1][wave] = na;
      red_s[2][wave] = nb;
    }
    __syncthreads();
    if (tid == 0) {
      int h = 0;
      float n = 0.f, a = 0.f, b = 0.f;
      for (int w = 0; w < kLagWaves; ++w) {
        h += cnt_s[w];
        n += red_s[0][w];
        a += red_s[1][w];
        b += red_s[2][w];
      }
      bool flagged = h < max(1, (count + 1) / 2);
      if (test == QKV_LAG_COS) flagged |= n / fmaxf(sqrtf(a) * sqrtf(b), 1e-6f) < 0.5f;
      flags[row] = flagged ? 1 : 0;
    }
    return;
  }

}

// QKV_LAG_ESS (EV:4068-4087): softmax weights of q over the tokens of the
// previous final mask (full-D dot rounded to the input dtype, times scaling
// rounded again, as the reference's matmul and multiply in that dtype leave
// them), e = exp(s - max), ESS = 1 / max(sum (e / sum e)^2, 1e-12), flagged
// when ESS / max(count, 1) > the threshold (always, for an empty mask).  A row's positions are
// cut into `splits` spans of `span` positions, one workgroup each (the first
// also records the row's top-|q| dims); a pass gathers the set positions of
// kLagPass mask bytes in LDS and spreads their dot products over the
// workgroup.  Each workgroup leaves (max, sum e, sum e^2, count) of its span
// in part[row * splits + split]; lag_ess_merge_kernel combines them.
// BITS: prev_final is a bitset (mask_ld words per row).
template <int DT, bool BITS = false>
__global__ __launch_bounds__(kLagNT) void lag_ess_kernel(
    const typename Elem<DT>::T* __restrict__ query, int q_heads, int group, int head_dim, int count,
    int32_t* __restrict__ dims_out, float* __restrict__ vals_out, const typename Elem<DT>::T* __restrict__ key,
    int64_t sb, int64_t sh, int64_t st, bool kvec, int history, int span, const uint8_t* __restrict__ prev_final,
    int64_t mask_ld, bool mvec, float scaling, float4* __restrict__ part) {
  using E = typename Elem<DT>::T;
  __shared__ float q_s[128];
  __shared__ __attribute__((aligned(16))) uint64_t key_s[128];
  __shared__ int sel_idx[128];
  __shared__ float sel_q[128];
  __shared__ int cnt_s[kLagWaves];
  __shared__ float red_s[3][kLagWaves];
  __shared__ int list[kLagPass];
  const int split = blockIdx.x, row = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const E* q_row = query + static_cast<int64_t>(row) * head_dim;
  for (int d = tid; d < 128; d += kLagNT) q_s[d] = d < head_dim ? Elem<DT>::load(q_row + d) : 0.f;
  __syncthreads();
  if (split == 0) {   // uniform: the row's top-|q| dims, as lag_flags_kernel records them
    rank_dims128(q_s, key_s, head_dim, count, sel_idx, sel_q);
    for (int s = tid; s < count; s += kLagNT) {
      dims_out[static_cast<int64_t>(row) * count + s] = sel_idx[s];
      vals_out[static_cast<int64_t>(row) * count + s] = sel_q[s];
    }
  }
  const int bq = row / q_heads, kvh = (row - bq * q_heads) / group;
  const E* krow = key + bq * sb + kvh * sh;
  const uint8_t* mrow = prev_final + static_cast<int64_t>(row) * mask_ld * (BITS ? 8 : 1);
  float m_t = -INFINITY, z_t = 0.f, z2_t = 0.f;
  int total = 0;
  const int p_begin = split * span, p_end = min(history, p_begin + span);
  for (int p0 = p_begin; p0 < p_end; p0 += kLagPass) {
    const int p = p0 + tid * 16;
    const int n = min(16, p_end - p);
    uint32_t bm = 0;
    if constexpr (BITS) {   // positions p .. p + 15 lie in one word (p is a multiple of 16)
      if (n > 0) {
        const uint64_t w = reinterpret_cast<const uint64_t*>(mrow)[p >> 6];
        bm = static_cast<uint32_t>(w >> (p & 63)) & (n >= 16 ? 0xFFFFu : ((1u << n) - 1u));
      }
    } else if (mvec && n == 16) {
      bm = nonzero_bytes(*reinterpret_cast<const uint4*>(mrow + p));
    } else {
      for (int j = 0; j < n; ++j)
        if (mrow[p + j]) bm |= 1u << j;
    }
    const int c = __builtin_popcount(bm);
    const int inc = wave_incl_scan(c);
    if (lane == 63) cnt_s[wave] = inc;
    __syncthreads();
    int off = inc - c, pass = 0;
    for (int w = 0; w < kLagWaves; ++w) {
      off += w < wave ? cnt_s[w] : 0;
      pass += cnt_s[w];
    }
    while (bm) {
      const int j = __builtin_ctz(bm);
      bm &= bm - 1;
      list[off++] = p + j;
    }
    __syncthreads();
    for (int e = tid; e < pass; e += kLagNT) {
      const E* kp = krow + static_cast<int64_t>(list[e]) * st;
      float acc = 0.f;
      if (kvec && head_dim == 128) {   // every load of the row in flight before the arithmetic
        constexpr int kWords = DT == QKV_DTYPE_FP32 ? 32 : 16;   // 16-byte words of a 128-dim row
        constexpr int kPer = 128 / kWords;
        uint4 raw[kWords];
#pragma unroll
        for (int i = 0; i < kWords; ++i) raw[i] = reinterpret_cast<const uint4*>(kp)[i];
#pragma unroll
        for (int i = 0; i < kWords; ++i) {
          const uint32_t w[4] = {raw[i].x, raw[i].y, raw[i].z, raw[i].w};
#pragma unroll
          for (int j = 0; j < kPer; ++j) {
            float x;
            if constexpr (DT == QKV_DTYPE_FP32) {
              x = __uint_as_float(w[j]);
            } else {
              const uint16_t h = static_cast<uint16_t>(w[j >> 1] >> (16 * (j & 1)));
              x = Elem<DT>::load(&h);
            }
            acc += q_s[i * kPer + j] * x;
          }
        }
      } else if (kvec) {
        for (int d = 0; d < head_dim; d += 8) {
          float kv[8];
          load8<DT>(kp + d, kv);
#pragma unroll
          for (int j = 0; j < 8; ++j) acc += q_s[d + j] * kv[j];
        }
      } else {
        for (int d = 0; d < head_dim; ++d) acc += q_s[d] * Elem<DT>::load(kp + d);
      }
      E rr = Elem<DT>::store(acc);
      float sc = Elem<DT>::load(&rr) * scaling;
      rr = Elem<DT>::store(sc);
      sc = Elem<DT>::load(&rr);
      const float m = fmaxf(m_t, sc);
      const float a = expf(m_t - m), ex = expf(sc - m);
      z_t = z_t * a + ex;
      z2_t = z2_t * a * a + ex * ex;
      m_t = m;
    }
    total += pass;
    __syncthreads();   // list and cnt_s are rewritten by the next pass
  }
  // the workgroup's (max, sum e, sum e^2)
  const float mw = wave_max(m_t);
  if (lane == 0) red_s[0][wave] = mw;
  __syncthreads();
  float mx = red_s[0][0];
  for (int w = 1; w < kLagWaves; ++w) mx = fmaxf(mx, red_s[0][w]);
  const float f = m_t == -INFINITY ? 0.f : expf(m_t - mx);
  const float z = wave_sum(z_t * f), z2 = wave_sum(z2_t * f * f);
  if (lane == 0) {
    red_s[1][wave] = z;
    red_s[2][wave] = z2;
  }
  __syncthreads();
  if (tid == 0) {
    float zs = 0.f, z2s = 0.f;
    for (int w = 0; w < kLagWaves; ++w) {
      zs += red_s[1][w];
      z2s += red_s[2][w];
    }
    part[static_cast<int64_t>(row) * gridDim.x + split] = make_float4(mx, zs, z2s, __int_as_float(total));
  }
}

__global__ __launch_bounds__(kLagNT) void lag_ess_merge_kernel(const float4* __restrict__ part, int rows, int splits,
                                                            float ess_threshold, uint8_t* __restrict__ flags) {
  const int row = blockIdx.x * kLagNT + threadIdx.x;
  if (row >= rows) return;
  const float4* pr = part + static_cast<int64_t>(row) * splits;
  float mx = -INFINITY;
  int total = 0;
  for (int i = 0; i < splits; ++i) {
    const float4 v = pr[i];
    mx = fmaxf(mx, v.x);
    total += __float_as_int(v.w);
  }
  float z = 0.f, z2 = 0.f;
  for (int i = 0; i < splits; ++i) {
    const float4 v = pr[i];
    if (v.x == -INFINITY) continue;   // an empty span
    const float f = expf(v.x - mx);
    z += v.y * f;
    z2 += v.z * f * f;
  }
  // the reference's expression: sum w^2 over the normalised weights w = e / z,
  // ESS = 1 / max(sum w^2, 1e-12), over max(count, 1) (EV:4079-4083)
  const float sum_w2 = total == 0 ? 0.f : z2 / (z * z);
  const float frac = (1.0f / fmaxf(sum_w2, 1.0e-12f)) / static_cast<float>(max(total, 1));
  flags[row] = frac > ess_threshold ? 1 : 0;
}

// 16 mask bytes at p, bytes at or past `n` read as 0.
__device__ __forceinline__ uint4 load16(const uint8_t* row, int p, int n, bool vec) {
  if (vec && n == 16) return *reinterpret_cast<const uint4*>(row + p);
  uint32_t w[4] = {0, 0, 0, 0};
  for (int j = 0; j < n; ++j) w[j >> 2] |= static_cast<uint32_t>(row[p + j]) << (8 * (j & 3));
  return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ void store16(uint8_t* row, int p, int n, bool vec, uint4 v) {
  if (vec && n == 16) {
    *reinterpret_cast<uint4*>(row + p) = v;
    return;
  }
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  for (int j = 0; j < n; ++j) row[p + j] = static_cast<uint8_t>(w[j >> 2] >> (8 * (j & 3)));
}

__device__ __forceinline__ uint4 or4(uint4 a, uint4 b) { return make_uint4(a.x | b.x, a.y | b.y, a.z | b.z, a.w | b.w); }

__global__ __launch_bounds__(kLagNT) void lag_union_kernel(
    uint8_t* __restrict__ cur, const uint8_t* __restrict__ prev_final, int64_t mask_ld,
    const uint8_t* __restrict__ flags, int rows, int q_heads, int history, int refresh, int share, int sink_end,
    int recent_start, uint8_t* __restrict__ uni, int64_t uni_ld, bool vec) {
  __shared__ int cnt_s[kLagWaves];
  const int r = blockIdx.y, tid = threadIdx.x;
  const int b = r / q_heads;
  // which rows keep their current candidates (EV:4024-4115)
  bool all = refresh == QKV_REFRESH_ALL;
  if (refresh == QKV_REFRESH_ANY || refresh == QKV_REFRESH_MAJORITY) {
    int c = 0;
    for (int i = tid; i < rows; i += kLagNT) c += flags[i] ? 1 : 0;
    c = wave_sum_i(c);
    if ((tid & 63) == 0) cnt_s[tid >> 6] = c;
    __syncthreads();
    int t = 0;
    for (int w = 0; w < kLagWaves; ++w) t += cnt_s[w];
    all = refresh == QKV_REFRESH_ANY ? t > 0 : 2 * t > rows;   // EV:4057-4066
  }
  const bool per_row = refresh == QKV_REFRESH_PER_ROW;
  const int p = (blockIdx.x * kLagNT + tid) * kUnionChunk;
  if (p >= history) return;
  const int n = min(kUnionChunk, history - p);
  uint32_t pw[4] = {0, 0, 0, 0};   // the sink and recent ranges (EV:4166-4171)
  for (int j = 0; j < n; ++j)
    if (p + j < sink_end || p + j >= recent_start) pw[j >> 2] |= 1u << (8 * (j & 3));
  uint4 u = make_uint4(pw[0], pw[1], pw[2], pw[3]);
  if (share) {   // the candidates of every refreshed row of the sequence (EV:4107-4109)
    for (int h = 0; h < q_heads; ++h) {
      const int i = b * q_heads + h;
      if (per_row ? flags[i] != 0 : all) u = or4(u, load16(cur + static_cast<int64_t>(i) * mask_ld, p, n, vec));
    }
  }
  uint8_t* crow = cur + static_cast<int64_t>(r) * mask_ld;
  if (per_row ? flags[r] != 0 : all) u = or4(u, load16(crow, p, n, vec));
  else store16(crow, p, n, vec, make_uint4(0, 0, 0, 0));   // a row that does not refresh has no candidates
  if (prev_final) u = or4(u, load16(prev_final + static_cast<int64_t>(r) * mask_ld, p, n, vec));
  store16(uni + static_cast<int64_t>(r) * uni_ld, p, n, vec, u);
}

// lag_union_kernel on bitsets: one thread per 64-position word.
__global__ __launch_bounds__(kLagNT) void lag_union_bits_kernel(
    uint64_t* __restrict__ cur, const uint64_t* __restrict__ prev_final, int64_t words_ld,
    const uint8_t* __restrict__ flags, int rows, int q_heads, int history, int refresh, int share, int sink_end,
    int recent_start, uint64_t* __restrict__ uni, int64_t uni_ld) {
  __shared__ int cnt_s[kLagWaves];
  const int r = blockIdx.y, tid = threadIdx.x;
  const int b = r / q_heads;
  bool all = refresh == QKV_REFRESH_ALL;
  if (refresh == QKV_REFRESH_ANY || refresh == QKV_REFRESH_MAJORITY) {
    int c = 0;
    for (int i = tid; i < rows; i += kLagNT) c += flags[i] ? 1 : 0;
    c = wave_sum_i(c);
    if ((tid & 63) == 0) cnt_s[tid >> 6] = c;
    __syncthreads();
    int t = 0;
    for (int w = 0; w < kLagWaves; ++w) t += cnt_s[w];
    all = refresh == QKV_REFRESH_ANY ? t > 0 : 2 * t > rows;   // EV:4057-4066
  }
  const bool per_row = refresh == QKV_REFRESH_PER_ROW;
  const int w = blockIdx.x * kLagNT + tid;
  if (w >= (history + 63) / 64) return;
  // the sink and recent ranges (EV:4166-4171)
  auto range = [&](int a, int e) -> uint64_t {
    const int lo = max(a, 64 * w) - 64 * w, hi = min(e, 64 * w + 64) - 64 * w;
    if (hi <= lo) return 0ull;
    const uint64_t upto = hi >= 64 ? ~0ull : ((1ull << hi) - 1ull);
    return upto & ~((1ull << lo) - 1ull);
  };
  uint64_t u = range(0, sink_end) | range(recent_start, history);
  if (share) {   // the candidates of every refreshed row of the sequence (EV:4107-4109)
    for (int h = 0; h < q_heads; ++h) {
      const int i = b * q_heads + h;
      if (per_row ? flags[i] != 0 : all) u |= cur[static_cast<int64_t>(i) * words_ld + w];
    }
  }
  uint64_t* crow = cur + static_cast<int64_t>(r) * words_ld;
  if (per_row ? flags[r] != 0 : all) u |= crow[w];
  else crow[w] = 0;   // a row that does not refresh has no candidates
  if (prev_final) u |= prev_final[static_cast<int64_t>(r) * words_ld + w];
  uni[static_cast<int64_t>(r) * uni_ld + w] = u;
}

// Spans of the ESS test: about kLagWGs workgroups over the rows, each span a
// whole number of passes.
struct EssSplit {
  int splits, span;
};
EssSplit ess_split(int64_t rows, int64_t history) {
  const int64_t passes = cdiv(history, kLagPass);
  const int64_t want = std::min<int64_t>(std::max<int64_t>(cdiv(kLagWGs, rows), 1), passes);
  const int64_t span = cdiv(passes, want) * kLagPass;
  return {static_cast<int>(cdiv(history, span)), static_cast<int>(span)};
}

template <int DT> struct RunLagFlags {
  static int run(const void* q, int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int count, int test,
                 const int32_t* pd, const float* pv, int32_t* dims_out, float* vals_out, const void* key,
                 const int64_t* ks, int64_t history, const uint8_t* prev_final, int64_t mask_ld, float scaling,
                 float ess_threshold, uint8_t* flags, void* workspace, hipStream_t st, bool bits = false) {
    using E = typename Elem<DT>::T;
    const char* what = "qkv_reuse_lag_flags";
    if (test != QKV_LAG_ESS) {
      lag_flags_kernel<DT><<<static_cast<unsigned>(B * Hq), kLagNT, 0, st>>>(
          static_cast<const E*>(q), static_cast<int>(D), count, test, pd, pv, dims_out, vals_out, flags);
      return check_launch(what);
    }
    const int64_t ev = DT == QKV_DTYPE_FP32 ? 4 : 8;   // elements per 16 bytes
    const bool kvec = D % 8 == 0 && aligned(key, 16) && ks[0] % ev == 0 && ks[1] % ev == 0 && ks[2] % ev == 0;
    const bool mvec = aligned(prev_final, 16) && mask_ld % 16 == 0;
    const EssSplit sp = ess_split(B * Hq, history);
    float4* part = static_cast<float4*>(workspace);
    const dim3 grid(static_cast<unsigned>(sp.splits), static_cast<unsigned>(B * Hq));
    if (bits)
      lag_ess_kernel<DT, true><<<grid, kLagNT, 0, st>>>(
          static_cast<const E*>(q), static_cast<int>(Hq), static_cast<int>(Hq / Hkv), static_cast<int>(D), count,
          dims_out, vals_out, static_cast<const E*>(key), ks[0], ks[1], ks[2], kvec, static_cast<int>(history),
          sp.span, prev_final, mask_ld, false, scaling, part);
    else
      lag_ess_kernel<DT><<<grid, kLagNT, 0, st>>>(
          static_cast<const E*>(q), static_cast<int>(Hq), static_cast<int>(Hq / Hkv), static_cast<int>(D), count,
          dims_out, vals_out, static_cast<const E*>(key), ks[0], ks[1], ks[2], kvec, static_cast<int>(history),
          sp.span, prev_final, mask_ld, mvec, scaling, part);
    int rc = check_launch(what);
    if (rc) return rc;
    lag_ess_merge_kernel<<<static_cast<unsigned>(cdiv(B * Hq, kLagNT)), kLagNT, 0, st>>>(
        part, static_cast<int>(B * Hq), sp.splits, ess_threshold, flags);
    return check_launch(what);
  }
};

}  // namespace
}  // namespace qkv

using namespace qkv;

QKV_EXPORT int64_t qkv_reuse_lag_flags_workspace_bytes(int64_t rows, int64_t history) {
  if (rows <= 0 || history <= 0 || history >= (int64_t(1) << 30)) return -1;
  return rows * ess_split(rows, history).splits * static_cast<int64_t>(sizeof(float4));
}

QKV_EXPORT int qkv_reuse_lag_flags(const void* query, int dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
                                   int64_t head_dim, int64_t dim_count, int test, const int32_t* previous_dims,
                                   const float* previous_values, int32_t* dims_out, float* values_out,
                                   const void* key, const int64_t* k_strides, int64_t history,
                                   const uint8_t* previous_final, int64_t mask_ld, float scaling,
                                   float ess_threshold, uint8_t* flags, void* workspace, int64_t workspace_bytes,
                                   void* stream) {
  const char* what = "qkv_reuse_lag_flags";
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads || batch * q_heads > 65535)
    return fail(QKV_ERR_INVALID, "%s: need batch * q_heads <= 65535, q_heads a positive multiple of kv_heads", what);
  if (head_dim <= 0 || head_dim > 128) return fail(QKV_ERR_UNSUPPORTED, "%s: head_dim must be in [1, 128]", what);
  if (!query || !dims_out || !values_out) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  if (test < QKV_LAG_DIMS || test > QKV_LAG_ESS) return fail(QKV_ERR_INVALID, "%s: unknown test %d", what, test);
  if (test != QKV_LAG_DIMS && !flags) return fail(QKV_ERR_INVALID, "%s: null flags", what);
  if ((test == QKV_LAG_OVERLAP || test == QKV_LAG_COS) && !previous_dims)
    return fail(QKV_ERR_INVALID, "%s: the overlap and cosine tests need the previous dims", what);
  if (test == QKV_LAG_COS && !previous_values)
    return fail(QKV_ERR_INVALID, "%s: the cosine test needs the previous values", what);
  if (test == QKV_LAG_ESS) {
    if (!key || !k_strides || !previous_final) return fail(QKV_ERR_INVALID, "%s: the ESS test needs K and the previous final mask", what);
    if (k_strides[3] != 1) return fail(QKV_ERR_UNSUPPORTED, "%s: K channels must be contiguous", what);
    if (history <= 0 || history >= (int64_t(1) << 30) || mask_ld < history)
      return fail(QKV_ERR_INVALID, "%s: need 0 < history < 2^30 and mask_ld >= history", what);
    const int64_t need = qkv_reuse_lag_flags_workspace_bytes(batch * q_heads, history);
    if (!workspace || workspace_bytes < need)
      return fail(QKV_ERR_INVALID, "%s: workspace needs %lld bytes, got %lld", what, (long long)need,
                  (long long)workspace_bytes);
  }
  const int count = static_cast<int>(std::min<int64_t>(std::max<int64_t>(dim_count, 1), head_dim));
  return dispatch_dtype<RunLagFlags>(dtype, query, batch, q_heads, kv_heads, head_dim, count, test, previous_dims,
                                     previous_values, dims_out, values_out, test == QKV_LAG_ESS ? key : nullptr,
                                     k_strides, history, test == QKV_LAG_ESS ? previous_final : nullptr, mask_ld,
                                     scaling, ess_threshold, flags, workspace, static_cast<hipStream_t>(stream));
}

QKV_EXPORT int qkv_reuse_lag_union(uint8_t* current, const uint8_t* previous_final, int64_t mask_ld,
                                   const uint8_t* flags, int64_t batch, int64_t q_heads, int64_t history,
                                   int refresh, int share, int64_t protect_sink, int64_t protect_recent,
                                   uint8_t* union_out, int64_t union_ld, void* stream) {
  const char* what = "qkv_reuse_lag_union";
  if (!current || !union_out) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  if (batch <= 0 || q_heads <= 0 || batch * q_heads > 65535)
    return fail(QKV_ERR_INVALID, "%s: need batch, q_heads > 0 and batch * q_heads <= 65535", what);
  if (history <= 0 || history >= (int64_t(1) << 31) || mask_ld < history || union_ld < history)
    return fail(QKV_ERR_INVALID, "%s: need 0 < history < 2^31, mask_ld and union_ld >= history", what);
  if (refresh < QKV_REFRESH_NONE || refresh > QKV_REFRESH_MAJORITY)
    return fail(QKV_ERR_INVALID, "%s: unknown refresh %d", what, refresh);
  if (refresh >= QKV_REFRESH_PER_ROW && !flags) return fail(QKV_ERR_INVALID, "%s: null flags", what);
  if (protect_sink < 0 || protect_recent < 0) return fail(QKV_ERR_INVALID, "%s: negative protection", what);
  const int sink_end = static_cast<int>(std::min(protect_sink, history));
  const int recent_start = static_cast<int>(std::max<int64_t>(0, history - protect_recent));
  const bool vec = mask_ld % 16 == 0 && union_ld % 16 == 0 && aligned(current, 16) && aligned(union_out, 16) &&
                   (!previous_final || aligned(previous_final, 16));
  dim3 grid(static_cast<unsigned>(cdiv(history, kLagNT * kUnionChunk)), static_cast<unsigned>(batch * q_heads));
  lag_union_kernel<<<grid, kLagNT, 0, static_cast<hipStream_t>(stream)>>>(
      current, previous_final, mask_ld, flags, static_cast<int>(batch * q_heads), static_cast<int>(q_heads),
      static_cast<int>(history), refresh, share ? 1 : 0, sink_end, recent_start, union_out, union_ld, vec);
  return check_launch(what);
}

QKV_EXPORT int qkv_reuse_lag_flags_bits(const void* query, int dtype, int64_t batch, int64_t q_heads,
                                        int64_t kv_heads, int64_t head_dim, int64_t dim_count, int test,
                                        const int32_t* previous_dims, const float* previous_values, int32_t* dims_out,
                                        float* values_out, const void* key, const int64_t* k_strides,
                                        int64_t history, const uint64_t* previous_final, int64_t words_ld,
                                        float scaling, float ess_threshold, uint8_t* flags, void* workspace,
                                        int64_t workspace_bytes, void* stream) {
  const char* what = "qkv_reuse_lag_flags_bits";
  if (test == QKV_LAG_ESS) {
    if (!previous_final || !aligned(previous_final, 8))
      return fail(QKV_ERR_INVALID, "%s: the ESS test needs the previous final bitset (8-byte aligned)", what);
    if (history <= 0 || history >= (int64_t(1) << 30) || words_ld < (history + 63) / 64)
      return fail(QKV_ERR_INVALID, "%s: need 0 < history < 2^30 and words_ld covering the history", what);
  }
  if (test != QKV_LAG_ESS)   // the other tests read no mask
    return qkv_reuse_lag_flags(query, dtype, batch, q_heads, kv_heads, head_dim, dim_count, test, previous_dims,
                               previous_values, dims_out, values_out, key, k_strides, history, nullptr, 0, scaling,
                               ess_threshold, flags, workspace, workspace_bytes, stream);
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads || batch * q_heads > 65535)
    return fail(QKV_ERR_INVALID, "%s: need batch * q_heads <= 65535, q_heads a positive multiple of kv_heads", what);
  if (head_dim <= 0 || head_dim > 128) return fail(QKV_ERR_UNSUPPORTED, "%s: head_dim must be in [1, 128]", what);
  if (!query || !dims_out || !values_out || !flags || !key || !k_strides)
    return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  if (k_strides[3] != 1) return fail(QKV_ERR_UNSUPPORTED, "%s: K channels must be contiguous", what);
  const int64_t need = qkv_reuse_lag_flags_workspace_bytes(batch * q_heads, history);
  if (!workspace || workspace_bytes < need)
    return fail(QKV_ERR_INVALID, "%s: workspace needs %lld bytes, got %lld", what, (long long)need,
                (long long)workspace_bytes);
  const int count = static_cast<int>(std::min<int64_t>(std::max<int64_t>(dim_count, 1), head_dim));
  return dispatch_dtype<RunLagFlags>(dtype, query, batch, q_heads, kv_heads, head_dim, count, test, previous_dims,
                                     previous_values, dims_out, values_out, key, k_strides, history,
                                     reinterpret_cast<const uint8_t*>(previous_final), words_ld, scaling,
                                     ess_threshold, flags, workspace, static_cast<hipStream_t>(stream), true);
}

QKV_EXPORT int qkv_reuse_lag_union_bits(uint64_t* current, const uint64_t* previous_final, int64_t words_ld,
                                        const uint8_t* flags, int64_t batch, int64_t q_heads, int64_t history,
                                        int refresh, int share, int64_t protect_sink, int64_t protect_recent,
                                        uint64_t* union_out, int64_t union_ld, void* stream) {
  const char* what = "qkv_reuse_lag_union_bits";
  if (!current || !union_out) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  if (batch <= 0 || q_heads <= 0 || batch * q_heads > 65535)
    return fail(QKV_ERR_INVALID, "%s: need batch, q_heads > 0 and batch * q_heads <= 65535", what);
  const int64_t words = (history + 63) / 64;
  if (history <= 0 || history >= (int64_t(1) << 31) || words_ld < words || union_ld < words)
    return fail(QKV_ERR_INVALID, "%s: need 0 < history < 2^31, words_ld and union_ld covering the history", what);
  if (!aligned(current, 8) || !aligned(union_out, 8) || !aligned(previous_final, 8))
    return fail(QKV_ERR_INVALID, "%s: bitsets must be 8-byte aligned", what);
  if (refresh < QKV_REFRESH_NONE || refresh > QKV_REFRESH_MAJORITY)
    return fail(QKV_ERR_INVALID, "%s: unknown refresh %d", what, refresh);
  if (refresh >= QKV_REFRESH_PER_ROW && !flags) return fail(QKV_ERR_INVALID, "%s: null flags", what);
  if (protect_sink < 0 || protect_recent < 0) return fail(QKV_ERR_INVALID, "%s: negative protection", what);
  const int sink_end = static_cast<int>(std::min(protect_sink, history));
  const int recent_start = static_cast<int>(std::max<int64_t>(0, history - protect_recent));
  dim3 grid(static_cast<unsigned>(cdiv(words, kLagNT)), static_cast<unsigned>(batch * q_heads));
  lag_union_bits_kernel<<<grid, kLagNT, 0, static_cast<hipStream_t>(stream)>>>(
      current, previous_final, words_ld, flags, static_cast<int>(batch * q_heads), static_cast<int>(q_heads),
      static_cast<int>(history), refresh, share ? 1 : 0, sink_end, recent_start, union_out, union_ld);
  return check_launch(what);
}
