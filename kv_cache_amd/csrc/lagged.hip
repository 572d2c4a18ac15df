// Lagged candidate reuse: the refresh tests and the candidate union of the
// reference's lagtop2 / lagrefresh{N} / qdrift[maj|head|share|cos|coshead] /
// pconf{T} modes (EV:4020-4198), ahead of the exact rerank of the union
// (qkv_reuse_select).  A row is one (sequence, query head) r = b * Hq + h.
//
//   lag_flags_kernel   one workgroup per row: the row's top-|q| dims and their
//                      q values (the state the next step compares with), then
//                      the row's refresh test: top-dim overlap, overlap or
//                      cosine, or the effective sample size of the previous
//                      final selection's attention weights;
//   lag_union_kernel   16 positions per thread, every head of a sequence:
//                      keeps the current candidates of the rows that refresh
//                      (zeroes the others), and writes the union with the
//                      previous final mask, the candidates shared across heads
//                      (qdriftshare) and the sink / recent ranges.
// The step-wide decisions (any / majority of the flags) are taken inside the
// union kernel, so a step needs no host round trip.  EV = ymluo/projects/
// qwen3_top2_head_limit3_ppl/src/evaluate_qwen3_top2_head_limit3_ppl.py.
#include <math.h>

#include "ref_common.h"

namespace qkv {
namespace {

constexpr int kLagNT = 256;                    // threads per workgroup (4 waves)
constexpr int kLagWaves = kLagNT / 64;
constexpr int kLagChunks = 8;                  // ESS: 16-position mask chunks per thread and pass
constexpr int kLagSpan = kLagNT * 16 * kLagChunks;   // ESS: positions per pass
constexpr int kLagList = 8192;                 // ESS: positions gathered in LDS per pass
constexpr int kUnionChunk = 16;                // union: positions per thread
constexpr int kMaxLagHeads = 1024;             // union: query heads per sequence

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
    const typename Elem<DT>::T* __restrict__ query, int q_heads, int group, int head_dim, int count, int test,
    const int32_t* __restrict__ prev_dims, const float* __restrict__ prev_vals, int32_t* __restrict__ dims_out,
    float* __restrict__ vals_out, const typename Elem<DT>::T* __restrict__ key, int64_t sb, int64_t sh, int64_t st,
    bool kvec, int history, const uint8_t* __restrict__ prev_final, int64_t mask_ld, bool mvec, float scaling,
    float ess_threshold, uint8_t* __restrict__ flags) {
  using E = typename Elem<DT>::T;
  __shared__ float q_s[128];
  __shared__ __attribute__((aligned(16))) uint64_t key_s[128];
  __shared__ int sel_idx[128];
  __shared__ float sel_q[128];
  __shared__ int pd_s[128];
  __shared__ int cnt_s[kLagWaves];
  __shared__ float red_s[3][kLagWaves];
  __shared__ int list[kLagList];
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const E* q_row = query + static_cast<int64_t>(row) * head_dim;
  for (int d = tid; d < 128; d += kLagNT) q_s[d] = d < head_dim ? Elem<DT>::load(q_row + d) : 0.f;
  __syncthreads();
  // the step's top-|q| dims, descending |q| with ties to the lower dim, and
  // q at them (EV:4026-4027, recorded at EV:4384-4393)
  rank_dims128(q_s, key_s, head_dim, count, sel_idx, sel_q);
  for (int s = tid; s < count; s += kLagNT) {
    dims_out[static_cast<int64_t>(row) * count + s] = sel_idx[s];
    vals_out[static_cast<int64_t>(row) * count + s] = sel_q[s];
  }
  if (test == QKV_LAG_DIMS) return;

  if (test == QKV_LAG_OVERLAP || test == QKV_LAG_COS) {
    for (int s = tid; s < count; s += kLagNT)
      pd_s[s] = min(max(prev_dims[static_cast<int64_t>(row) * count + s], 0), head_dim - 1);
    __syncthreads();
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

  // QKV_LAG_ESS (EV:4068-4087): softmax weights of q over the tokens of the
  // previous final mask (full-D dot rounded to the input dtype, times
  // scaling rounded again, as the reference's matmul and multiply in that
  // dtype leave them), ESS = (sum e)^2 / sum e^2 with e = exp(s - max),
  // flagged when ESS / count > the threshold or the mask is empty.  Each
  // pass gathers up to kLagList set positions of kLagSpan mask bytes in LDS
  // and spreads their dot products over the workgroup; positions past the
  // list are scored by the thread that found them.
  const int bq = row / q_heads, kvh = (row - bq * q_heads) / group;
  const E* krow = key + bq * sb + kvh * sh;
  const uint8_t* mrow = prev_final + static_cast<int64_t>(row) * mask_ld;
  float m_t = -INFINITY, z_t = 0.f, z2_t = 0.f;
  auto add = [&](int p) {
    const E* kp = krow + static_cast<int64_t>(p) * st;
    float acc = 0.f;
    if (kvec) {
      for (int d = 0; d < head_dim; d += 8) {
        float kv[8];
        load8<DT>(kp + d, kv);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc += q_s[d + j] * kv[j];
      }
    } else {
      for (int d = 0; d < head_dim; ++d) acc += q_s[d] * Elem<DT>::load(kp + d);
    }
    E r = Elem<DT>::store(acc);
    float s = Elem<DT>::load(&r) * scaling;
    r = Elem<DT>::store(s);
    s = Elem<DT>::load(&r);
    const float m = fmaxf(m_t, s);
    const float c = __expf(m_t - m), e = __expf(s - m);
    z_t = z_t * c + e;
    z2_t = z2_t * c * c + e * e;
    m_t = m;
  };
  int total = 0;
  for (int p0 = 0; p0 < history; p0 += kLagSpan) {
    uint32_t set[kLagChunks];
    int c = 0;
#pragma unroll
    for (int i = 0; i < kLagChunks; ++i) {
      const int p = p0 + (i * kLagNT + tid) * 16;
      uint32_t bm = 0;
      if (mvec && p + 16 <= history) {
        bm = nonzero_bytes(*reinterpret_cast<const uint4*>(mrow + p));
      } else {
        for (int j = 0; j < 16; ++j)
          if (p + j < history && mrow[p + j]) bm |= 1u << j;
      }
      set[i] = bm;
      c += __builtin_popcount(bm);
    }
    const int inc = wave_incl_scan(c);
    if (lane == 63) cnt_s[wave] = inc;
    __syncthreads();
    int off = inc - c, pass = 0;
    for (int w = 0; w < kLagWaves; ++w) {
      off += w < wave ? cnt_s[w] : 0;
      pass += cnt_s[w];
    }
#pragma unroll
    for (int i = 0; i < kLagChunks; ++i) {
      uint32_t bm = set[i];
      const int p = p0 + (i * kLagNT + tid) * 16;
      while (bm) {
        const int j = __builtin_ctz(bm);
        bm &= bm - 1;
        if (off < kLagList) list[off] = p + j;
        else add(p + j);
        ++off;
      }
    }
    __syncthreads();
    const int n = min(pass, kLagList);
    for (int e = tid; e < n; e += kLagNT) add(list[e]);
    total += pass;
    __syncthreads();   // list and cnt_s are rewritten by the next pass
  }
  // merge the threads' (max, sum e, sum e^2)
  float mw = wave_max(m_t);
  if (lane == 0) red_s[0][wave] = mw;
  __syncthreads();
  float mx = red_s[0][0];
  for (int w = 1; w < kLagWaves; ++w) mx = fmaxf(mx, red_s[0][w]);
  const float sc = m_t == -INFINITY ? 0.f : __expf(m_t - mx);
  const float z = wave_sum(z_t * sc), z2 = wave_sum(z2_t * sc * sc);
  __syncthreads();
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
    const bool flagged = total == 0 || (zs * zs / z2s) / static_cast<float>(total) > ess_threshold;
    flags[row] = flagged ? 1 : 0;
  }
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
  __shared__ uint8_t fresh[kMaxLagHeads];
  __shared__ int cnt_s[kLagWaves];
  const int b = blockIdx.y, tid = threadIdx.x;
  // which heads of sequence b keep their current candidates (EV:4024-4115)
  bool all = refresh == QKV_REFRESH_ALL;
  if (refresh == QKV_REFRESH_ANY || refresh == QKV_REFRESH_MAJORITY) {
    int c = 0;
    for (int r = tid; r < rows; r += kLagNT) c += flags[r] ? 1 : 0;
    c = wave_sum_i(c);
    if ((tid & 63) == 0) cnt_s[tid >> 6] = c;
    __syncthreads();
    int t = 0;
    for (int w = 0; w < kLagWaves; ++w) t += cnt_s[w];
    all = refresh == QKV_REFRESH_ANY ? t > 0 : 2 * t > rows;   // EV:4057-4066
  }
  for (int h = tid; h < q_heads; h += kLagNT)
    fresh[h] = (refresh == QKV_REFRESH_PER_ROW ? flags[b * q_heads + h] != 0 : all) ? 1 : 0;
  __syncthreads();
  const int p = (blockIdx.x * kLagNT + tid) * kUnionChunk;
  if (p >= history) return;
  const int n = min(kUnionChunk, history - p);
  uint32_t pw[4] = {0, 0, 0, 0};   // the sink and recent ranges (EV:4166-4171)
  for (int j = 0; j < n; ++j)
    if (p + j < sink_end || p + j >= recent_start) pw[j >> 2] |= 1u << (8 * (j & 3));
  uint4 base = make_uint4(pw[0], pw[1], pw[2], pw[3]);
  if (share) {   // the candidates of every refreshed head of the sequence (EV:4107-4109)
    for (int h = 0; h < q_heads; ++h)
      if (fresh[h]) base = or4(base, load16(cur + static_cast<int64_t>(b * q_heads + h) * mask_ld, p, n, vec));
  }
  const uint4 zero = make_uint4(0, 0, 0, 0);
  for (int h = 0; h < q_heads; ++h) {
    const int64_t r = b * q_heads + h;
    uint8_t* crow = cur + r * mask_ld;
    uint4 u = base;
    if (fresh[h]) u = or4(u, load16(crow, p, n, vec));
    else store16(crow, p, n, vec, zero);   // a row that does not refresh has no current candidates
    if (prev_final) u = or4(u, load16(prev_final + r * mask_ld, p, n, vec));
    store16(uni + r * uni_ld, p, n, vec, u);
  }
}

template <int DT> struct RunLagFlags {
  static int run(const void* q, int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int count, int test,
                 const int32_t* pd, const float* pv, int32_t* dims_out, float* vals_out, const void* key,
                 const int64_t* ks, int64_t history, const uint8_t* prev_final, int64_t mask_ld, float scaling,
                 float ess_threshold, uint8_t* flags, hipStream_t st) {
    using E = typename Elem<DT>::T;
    const int64_t ev = DT == QKV_DTYPE_FP32 ? 4 : 8;   // elements per 16 bytes
    const bool kvec = key && D % 8 == 0 && aligned(key, 16) && ks[0] % ev == 0 && ks[1] % ev == 0 &&
                      ks[2] % ev == 0;
    const bool mvec = prev_final && aligned(prev_final, 16) && mask_ld % 16 == 0;
    lag_flags_kernel<DT><<<static_cast<unsigned>(B * Hq), kLagNT, 0, st>>>(
        static_cast<const E*>(q), static_cast<int>(Hq), static_cast<int>(Hq / Hkv), static_cast<int>(D), count,
        test, pd, pv, dims_out, vals_out, static_cast<const E*>(key), key ? ks[0] : 0, key ? ks[1] : 0,
        key ? ks[2] : 0, kvec, static_cast<int>(history), prev_final, mask_ld, mvec, scaling, ess_threshold, flags);
    return check_launch("qkv_reuse_lag_flags");
  }
};

}  // namespace
}  // namespace qkv

using namespace qkv;

QKV_EXPORT int qkv_reuse_lag_flags(const void* query, int dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
                                   int64_t head_dim, int64_t dim_count, int test, const int32_t* previous_dims,
                                   const float* previous_values, int32_t* dims_out, float* values_out,
                                   const void* key, const int64_t* k_strides, int64_t history,
                                   const uint8_t* previous_final, int64_t mask_ld, float scaling,
                                   float ess_threshold, uint8_t* flags, void* stream) {
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
  }
  const int count = static_cast<int>(std::min<int64_t>(std::max<int64_t>(dim_count, 1), head_dim));
  return dispatch_dtype<RunLagFlags>(dtype, query, batch, q_heads, kv_heads, head_dim, count, test, previous_dims,
                                     previous_values, dims_out, values_out, test == QKV_LAG_ESS ? key : nullptr,
                                     k_strides, history, test == QKV_LAG_ESS ? previous_final : nullptr, mask_ld,
                                     scaling, ess_threshold, flags, static_cast<hipStream_t>(stream));
}

QKV_EXPORT int qkv_reuse_lag_union(uint8_t* current, const uint8_t* previous_final, int64_t mask_ld,
                                   const uint8_t* flags, int64_t batch, int64_t q_heads, int64_t history,
                                   int refresh, int share, int64_t protect_sink, int64_t protect_recent,
                                   uint8_t* union_out, int64_t union_ld, void* stream) {
  const char* what = "qkv_reuse_lag_union";
  if (!current || !union_out) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  if (batch <= 0 || q_heads <= 0 || q_heads > kMaxLagHeads || batch * q_heads > 65535)
    return fail(QKV_ERR_INVALID, "%s: need 0 < q_heads <= %d and batch * q_heads <= 65535", what, kMaxLagHeads);
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
  dim3 grid(static_cast<unsigned>(cdiv(history, kLagNT * kUnionChunk)), static_cast<unsigned>(batch));
  lag_union_kernel<<<grid, kLagNT, 0, static_cast<hipStream_t>(stream)>>>(
      current, previous_final, mask_ld, flags, static_cast<int>(batch * q_heads), static_cast<int>(q_heads),
      static_cast<int>(history), refresh, share ? 1 : 0, sink_end, recent_start, union_out, union_ld, vec);
  return check_launch(what);
}
