// Row-wise top-k with the lowest-index tie-break: one workgroup per row, or,
// for long rows, a staged reduction over 4096-key chunks (topk_stage_kernel).
//
// The reference calls torch.topk over partial scores or block maxima
// (evaluate_qwen3_top2_head_limit3_ppl.py:4448, 5046), whose tie order is
// unspecified.  Here: keys map to order-preserving uint32; a 3-pass radix
// select (11/11/10-bit digits, LDS histograms) finds the k-th largest key
// theta and how many keys equal to theta are kept; a stable compaction in
// index order then writes every key > theta plus the lowest-index keys equal
// to theta, so the output is already in ascending index order.
#include <atomic>
#include <mutex>
#include <vector>

#include "common.h"
#include "select.h"
#include "window.h"

namespace qkv {
namespace {

constexpr int kBins = 2048;
constexpr int kLdsKeys = 12288;   // rows up to this many keys are staged in LDS (48 KB)
#ifndef QKV_TOPK_WAVE_MAX_VPL
#define QKV_TOPK_WAVE_MAX_VPL 16
#endif
// Rows up to 64 * kWaveMaxVPL keys take the one-wave-per-row kernel when
// there are at least kWaveMinRows of them.
constexpr int kWaveMaxVPL = QKV_TOPK_WAVE_MAX_VPL;
constexpr int64_t kWaveMinRows = 1024;

template <int NT>
__device__ int block_excl_scan(int v, int* buf) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  constexpr int NW = NT / 64;
  int inc = wave_incl_scan(v);
  if (lane == 63) buf[wave] = inc;
  __syncthreads();
  if (wave == 0) {
    int w = lane < NW ? buf[lane] : 0;
    int wi = wave_incl_scan(w);
    if (lane < NW) buf[NW + lane] = wi - w;
  }
  __syncthreads();
  int res = buf[NW + wave] + inc - v;
  __syncthreads();
  return res;
}

template <int NT, bool IN_LDS>
__global__ __launch_bounds__(NT) void topk_kernel(const float* __restrict__ values, int n, int64_t ld,
                                                  int k, int32_t* __restrict__ out) {
  extern __shared__ uint32_t keys_lds[];
  __shared__ int hist[kBins];
  __shared__ int scan_buf[2 * (NT / 64)];
  __shared__ int sh_bin, sh_kr;
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const float* vals = values + static_cast<int64_t>(row) * ld;

  if (IN_LDS) {
    for (int i = tid; i < n; i += NT) keys_lds[i] = f32_sortable(vals[i]);
    __syncthreads();
  }
  auto get = [&](int i) -> uint32_t { return IN_LDS ? keys_lds[i] : f32_sortable(vals[i]); };

  uint32_t prefix = 0, mask = 0;
  int kr = k;
  const int shifts[3] = {21, 10, 0};
  const int widths[3] = {11, 11, 10};
#pragma unroll
  for (int p = 0; p < 3; ++p) {
    const int shift = shifts[p];
    const int nbins = 1 << widths[p];
    for (int i = tid; i < nbins; i += NT) hist[i] = 0;
    __syncthreads();
    for (int i = tid; i < n; i += NT) {
      uint32_t u = get(i);
      if ((u & mask) == prefix) atomicAdd(&hist[(u >> shift) & (nbins - 1)], 1);
    }
    __syncthreads();
    // Thread t owns bins [nbins - (t+1)*bpt, nbins - t*bpt): thread order is
    // descending bin order, so an exclusive scan gives the count above.
    const int bpt = (nbins + NT - 1) / NT;
    const int hi = nbins - tid * bpt;
    int local = 0;
    for (int bb = hi - 1; bb >= hi - bpt && bb >= 0; --bb) local += hist[bb];
    int above = block_excl_scan<NT>(local, scan_buf);
    for (int bb = hi - 1; bb >= hi - bpt && bb >= 0; --bb) {
      const int c = hist[bb];
      if (above < kr && kr <= above + c) {
        sh_bin = bb;
        sh_kr = kr - above;
      }
      above += c;
    }
    __syncthreads();
    prefix |= static_cast<uint32_t>(sh_bin) << shift;
    mask |= static_cast<uint32_t>(nbins - 1) << shift;
    kr = sh_kr;
    __syncthreads();
  }
  const uint32_t theta = prefix;

  // Stable compaction over contiguous per-thread ranges.
  const int ipt = (n + NT - 1) / NT;
  const int i0 = min(n, tid * ipt), i1 = min(n, i0 + ipt);
  int gt = 0, eq = 0;
  for (int i = i0; i < i1; ++i) {
    uint32_t u = get(i);
    gt += u > theta;
    eq += u == theta;
  }
  const int eq_before = block_excl_scan<NT>(eq, scan_buf);
  int take = min(max(kr - eq_before, 0), eq);
  int pos = block_excl_scan<NT>(gt + take, scan_buf);
  int32_t* orow = out + static_cast<int64_t>(row) * k;
  for (int i = i0; i < i1; ++i) {
    uint32_t u = get(i);
    if (u > theta) {
      orow[pos++] = i;
    } else if (u == theta && take > 0) {
      orow[pos++] = i;
      --take;
    }
  }
}

// Rows of at most 64*VPL keys: one wave per row, four rows per workgroup,
// no workgroup barrier.  Lane l holds the VPL consecutive keys from l*VPL
// (16-byte loads where the row allows), so the output, in index order, is
// lane order: a lane's taken keys go after those of the lanes before it (one
// DPP scan of per-lane counts) instead of a ballot round per slot.  The
// radix select uses a wave-private 256-bin LDS histogram (a wave's LDS
// operations complete in order) and a DPP scan.  With many rows the kernel
// is bound by VALU issue (about 1000 instructions a row of 1024 keys), not
// latency.  Same contract as select_row.
//
// wave_select_row is the selection once the lane's keys are in registers as
// order-preserving uint32 (valid[i]: key first + i is selectable); wh is the
// wave's 256-int LDS histogram, orow the row's k output slots.
template <int VPL>
__device__ __forceinline__ void wave_select_row(uint32_t (&u)[VPL], const bool (&valid)[VPL], int first, int k,
                                                int* wh, int32_t* orow) {
  const int lane = threadIdx.x & 63;
  uint32_t umax = 0, umin = 0xFFFFFFFFu;
  int nval = 0;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    if (valid[i]) {
      umax = max(umax, u[i]);
      umin = min(umin, u[i]);
    }
    nval += __popcll(__ballot(valid[i]));
  }
  const uint32_t lane_max = umax;   // 0 when the lane holds no valid key
  umax = wave_minmax_u32<true>(umax);
  umin = wave_minmax_u32<false>(umin);
  const int kk = min(k, nval);
  // A lower bound of the k-th largest key (k <= 64: at least k lanes' maxima
  // are >= it); the radix passes start from the bits it shares with the
  // largest key, and keys under it stay out of the histograms.
  const uint32_t lo = max(umin, wave_lower_bound(lane_max, kk, umax, umin));

  int kr = kk;
  uint32_t prefix = umax, mask = 0xFFFFFFFFu;
  int remaining = (umax == lo || kk == 0) ? 0 : 32 - __builtin_clz(umax ^ lo);
  if (remaining) {
    mask = remaining == 32 ? 0u : ~((1u << remaining) - 1u);
    prefix = umax & mask;
  }
  if (kk == nval) {
    prefix = umin;
    kr = 0x7FFFFFFF;
    remaining = 0;
  }
  while (remaining > 0) {   // wave-uniform
    const int shift = remaining > 8 ? remaining - 8 : 0;
    const uint32_t dmask = (1u << (remaining - shift)) - 1u;
#pragma unroll
    for (int b = 0; b < 4; ++b) wh[4 * lane + b] = 0;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      if (valid[i] && u[i] >= lo && (u[i] & mask) == prefix) atomicAdd(&wh[(u[i] >> shift) & dmask], 1);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // Lane l owns bins 255-4l .. 252-4l (descending order of keys).
    int c[4], tot = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      c[b] = wh[255 - 4 * lane - b];
      tot += c[b];
    }
    int above = wave_incl_scan_dpp(tot) - tot;
    int my_bin = -1, my_kr = 0, my_whole = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (above < kr && kr <= above + c[b]) {
        my_bin = 255 - 4 * lane - b;
        my_kr = kr - above;
        my_whole = (kr - above) == c[b];
      }
      above += c[b];
    }
    const uint64_t who = __ballot(my_bin >= 0);
    const int src = __builtin_ctzll(who);   // exactly one lane holds the kr-th key's bin
    const int bin = __builtin_amdgcn_readlane(my_bin, src);
    kr = __builtin_amdgcn_readlane(my_kr, src);
    prefix |= static_cast<uint32_t>(bin) << shift;
    mask |= dmask << shift;
    remaining = shift;
    if (__builtin_amdgcn_readlane(my_whole, src)) {
      kr = 0x7FFFFFFF;
      break;
    }
  }
  const uint32_t theta = prefix;

  // Keys > theta and == theta of this lane, then of the lanes before it; the
  // lane takes its first min(ce, kr - eq_before) keys equal to theta.
  uint32_t gtm = 0, eqm = 0;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    gtm |= static_cast<uint32_t>(valid[i] && u[i] > theta) << i;
    eqm |= static_cast<uint32_t>(valid[i] && u[i] == theta) << i;
  }
  const int cg = __popc(gtm), ce = __popc(eqm);
  const int gt_before = wave_incl_scan_dpp(cg) - cg;
  const int eq_before = wave_incl_scan_dpp(ce) - ce;
  const int eq_take = min(ce, max(kr - eq_before, 0));
  int o = gt_before + min(eq_before, kr);
  int eq_seen = 0;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const bool gt = (gtm >> i) & 1u, eq = (eqm >> i) & 1u;
    const bool take = gt || (eq && eq_seen < eq_take);
    if (take) orow[o] = first + i;
    o += take ? 1 : 0;
    eq_seen += eq ? 1 : 0;
  }
  for (int j = kk + lane; j < k; j += 64) orow[j] = -1;
}

template <int VPL, bool FINITE>
__global__ __launch_bounds__(256) void topk_wave_kernel(const float* __restrict__ values, int64_t rows, int n,
                                                        int64_t ld, int k, int32_t* __restrict__ out) {
  __shared__ int hist[4][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  if (row >= rows) return;   // wave-uniform
  const float* vals = values + row * ld;

  uint32_t u[VPL];
  bool valid[VPL];
  const int first = lane * VPL;
  if (VPL % 4 == 0 && n == 64 * VPL && (reinterpret_cast<uintptr_t>(vals) & 15) == 0) {   // wave-uniform
#pragma unroll
    for (int i = 0; i < VPL; i += 4) {
      const uint4 w = *reinterpret_cast<const uint4*>(vals + first + i);
      u[i] = w.x;
      u[i + 1] = w.y;
      u[i + 2] = w.z;
      u[i + 3] = w.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < VPL; ++i) u[i] = __float_as_uint(vals[min(first + i, n - 1)]);
  }
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    u[i] = f32_sortable(__uint_as_float(u[i]));
    valid[i] = first + i < n && (!FINITE || u[i] != kNegInfKey);
  }
  wave_select_row<VPL>(u, valid, first, k, hist[wave], out + row * k);
}

// Many rows of finite or -inf keys (block maxima of a prefill chunk), k <= 64,
// -inf never selected: one wave per row as in topk_wave_kernel, but only the
// keys that can be selected enter the radix passes and the placement.  The k-th
// largest key of any subset of the row bounds the row's k-th largest from
// below; the subset here is every lane's two largest keys (128 keys, so a few
// lanes left empty by a causal -inf tail still leave k of them), and its k-th
// largest is resolved to 10 bits by ballot counts.  For i.i.d. keys about 72
// of a 1024-key row reach that bound (sampled: at most 91 in 20000 rows, with
// or without a 32-key -inf tail).  Those candidates are compacted, in index
// order, into a wave-private LDS list, and each lane then works on list
// entries lane, lane + 64, ... (one or two, where the full row puts 16 keys on
// a lane).  The list being in index order, a taken entry's output position is
// the count of taken entries in the slots before plus mbcnt of the slot's
// ballot.  Candidates are found with a float compare against the bound's
// float, which keeps every key whose order-preserving form is at or above the
// bound (the map folds -0 onto +0 as the compare does); a row with more than
// kCandCap candidates (heavy ties) takes the full-row selection.
constexpr int kCandCap = 256;

// A lower bound of the j-th largest of the wave's values v1, v2 (two per
// lane, 0 = none), given the largest value vmax and a value vmin <= every
// nonzero one: the largest x with at least j values at or above it, resolved
// to BITS bits below the bits vmax and vmin share; 0 when fewer than j values
// exist.  Wave-uniform.
template <int BITS>
__device__ __forceinline__ uint32_t wave_lower_bound2(uint32_t v1, uint32_t v2, int j, uint32_t vmax,
                                                      uint32_t vmin) {
  if (__popcll(__ballot(v1 != 0)) + __popcll(__ballot(v2 != 0)) < j) return 0;
  if (vmax == vmin) return vmax;   // every value is vmax
  const int top = 31 - __builtin_clz(vmax ^ vmin);
  uint32_t x = top == 31 ? 0u : vmax & ~((2u << top) - 1u);
#pragma unroll
  for (int b = 0; b < BITS; ++b) {
    if (top - b < 0) break;
    const uint32_t c = x | (1u << (top - b));
    if (__popcll(__ballot(v1 >= c)) + __popcll(__ballot(v2 >= c)) >= j) x = c;
  }
  return x;
}

// Keys of one row into registers, positions past n as -inf.
template <int VPL>
__device__ __forceinline__ void load_row_keys(const float* vals, int n, int first, uint32_t (&w)[VPL]) {
  if (VPL % 4 == 0 && n == 64 * VPL && (reinterpret_cast<uintptr_t>(vals) & 15) == 0) {   // wave-uniform
#pragma unroll
    for (int i = 0; i < VPL; i += 4) {
      const uint4 q = *reinterpret_cast<const uint4*>(vals + first + i);
      w[i] = q.x;
      w[i + 1] = q.y;
      w[i + 2] = q.z;
      w[i + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const uint32_t x = __float_as_uint(vals[min(first + i, n - 1)]);
      w[i] = first + i < n ? x : 0xFF800000u;
    }
  }
}

template <int VPL>
__device__ __forceinline__ void cand_select_row(const uint32_t (&w)[VPL], int first, int k, int32_t* orow,
                                                uint2* cl, int* wh) {
  constexpr int kSlots = kCandCap / 64;
  const int lane = threadIdx.x & 63;
  // the lane's largest (m1) and second largest (m2) key: the median of
  // {m1, m2, x} is the new second largest
  float m1 = __uint_as_float(w[0]), m2 = -INFINITY;
#pragma unroll
  for (int i = 1; i < VPL; ++i) {
    const float x = __uint_as_float(w[i]);
    m2 = __builtin_amdgcn_fmed3f(m1, m2, x);
    m1 = fmaxf(m1, x);
  }
  const uint32_t k1 = m1 > -INFINITY ? f32_sortable(m1) : 0u;   // 0: none
  const uint32_t k2 = m2 > -INFINITY ? f32_sortable(m2) : 0u;
  const uint32_t umax = wave_minmax_u32<true>(k1);
  if (umax == 0) {   // nothing selectable
    for (int j = lane; j < k; j += 64) orow[j] = -1;
    return;
  }
  const uint32_t vmin = wave_minmax_u32<false>(k2 ? k2 : (k1 ? k1 : 0xFFFFFFFFu));
  // 0 when fewer than k of the 128 hold a key: then every finite key is a candidate
  const uint32_t lo = max(wave_lower_bound2<10>(k1, k2, k, umax, vmin), kNegInfKey + 1);
  const float lo_f = sortable_f32(lo);   // -FLT_MAX at the floor

  int c = 0;
#pragma unroll
  for (int i = 0; i < VPL; ++i) c += __uint_as_float(w[i]) >= lo_f ? 1 : 0;
  const int incl = wave_incl_scan_dpp(c);
  const int total = __builtin_amdgcn_readlane(incl, 63);
  if (total > kCandCap) {   // wave-uniform: the full-row selection
    uint32_t u[VPL];
    bool valid[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      u[i] = f32_sortable(__uint_as_float(w[i]));
      valid[i] = u[i] != kNegInfKey;
    }
    wave_select_row<VPL>(u, valid, first, k, wh, orow);
    return;
  }
  int pos = incl - c;
  // total <= k: every candidate is selected (a bound above the floor has at
  // least k keys at or above it, so total == k; at the floor the candidates
  // are all the selectable keys)
  if (total <= k) {
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      if (__uint_as_float(w[i]) >= lo_f) orow[pos++] = first + i;
    for (int j = total + lane; j < k; j += 64) orow[j] = -1;
    return;
  }
#pragma unroll
  for (int i = 0; i < VPL; ++i)
    if (__uint_as_float(w[i]) >= lo_f) cl[pos++] = make_uint2(w[i], static_cast<uint32_t>(first + i));
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int ns = (total + 63) >> 6;   // wave-uniform
  uint32_t cu[kSlots];
  int32_t ci[kSlots];
#pragma unroll
  for (int s = 0; s < kSlots; ++s) {
    cu[s] = 0u;   // below every bound: never counted or taken
    ci[s] = -1;
    if (s < ns) {
      const int j = s * 64 + lane;
      const uint2 e = cl[j];
      if (j < total) {
        cu[s] = f32_sortable(__uint_as_float(e.x));
        ci[s] = static_cast<int32_t>(e.y);
      }
    }
  }

  // Radix select of the k-th largest candidate at or above lo, 8 bits a pass
  // below the bits it shares with the row's largest key.
  int kr = k;
  uint32_t prefix = umax, mask = 0xFFFFFFFFu;
  int remaining = umax == lo ? 0 : 32 - __builtin_clz(umax ^ lo);
  if (remaining) {
    mask = remaining == 32 ? 0u : ~((1u << remaining) - 1u);
    prefix = umax & mask;
  }
  while (remaining > 0) {   // wave-uniform
    const int shift = remaining > 8 ? remaining - 8 : 0;
    const uint32_t dmask = (1u << (remaining - shift)) - 1u;
#pragma unroll
    for (int b = 0; b < 4; ++b) wh[4 * lane + b] = 0;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int s = 0; s < kSlots; ++s)
      if (s < ns && cu[s] >= lo && (cu[s] & mask) == prefix) atomicAdd(&wh[(cu[s] >> shift) & dmask], 1);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    int cb[4], tot = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      cb[b] = wh[255 - 4 * lane - b];
      tot += cb[b];
    }
    int above = wave_incl_scan_dpp(tot) - tot;
    int my_bin = -1, my_kr = 0, my_whole = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (above < kr && kr <= above + cb[b]) {
        my_bin = 255 - 4 * lane - b;
        my_kr = kr - above;
        my_whole = (kr - above) == cb[b];
      }
      above += cb[b];
    }
    const uint64_t who = __ballot(my_bin >= 0);
    const int src = __builtin_ctzll(who);   // exactly one lane holds the kr-th key's bin
    const int bin = __builtin_amdgcn_readlane(my_bin, src);
    kr = __builtin_amdgcn_readlane(my_kr, src);
    prefix |= static_cast<uint32_t>(bin) << shift;
    mask |= dmask << shift;
    remaining = shift;
    if (__builtin_amdgcn_readlane(my_whole, src)) {
      kr = 0x7FFFFFFF;
      break;
    }
  }
  const uint32_t theta = prefix;

  // Entries > theta, and the first kr entries == theta, in list (= index) order.
  int before = 0, eq_seen = 0;
#pragma unroll
  for (int s = 0; s < kSlots; ++s) {
    if (s < ns) {
      const bool eq = cu[s] == theta;
      const uint64_t em = __ballot(eq);
      const int erank = eq_seen + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                      static_cast<uint32_t>(em >> 32),
                                      __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(em), 0u)));
      const bool take = cu[s] > theta || (eq && erank < kr);
      const uint64_t tm = __ballot(take);
      const int o = before + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                 static_cast<uint32_t>(tm >> 32),
                                 __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(tm), 0u)));
      if (take) orow[o] = ci[s];
      before += __popcll(tm);
      eq_seen += __popcll(em);
    }
  }
}

template <int VPL>
__global__ __launch_bounds__(256) void topk_cand_wave_kernel(const float* __restrict__ values, int64_t rows,
                                                             int n, int64_t ld, int k, int32_t* __restrict__ out) {
  __shared__ uint2 cand[4][kCandCap];   // (key bits, index)
  __shared__ int hist[4][256];
  const int wave = threadIdx.x >> 6;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  if (row >= rows) return;   // wave-uniform
  const int first = (threadIdx.x & 63) * VPL;
  uint32_t w[VPL];
  load_row_keys<VPL>(values + row * ld, n, first, w);
  cand_select_row<VPL>(w, first, k, out + row * k, cand[wave], hist[wave]);
}

template <int VPL, bool FINITE>
__global__ __launch_bounds__(256) void topk_rows_kernel(const float* __restrict__ values, int n, int64_t ld,
                                                        int k, int32_t* __restrict__ out) {
  __shared__ int32_t sel[256 * VPL];
  const int row = blockIdx.x;
  const int kk = select_row<VPL, FINITE>(values + static_cast<int64_t>(row) * ld, n, k, sel);
  int32_t* orow = out + static_cast<int64_t>(row) * k;
  for (int j = threadIdx.x; j < k; j += 256) orow[j] = j < kk ? sel[j] : -1;
}

// ---------------------------------------------------------------------------
// Staged top-k for long rows (n > kStageChunk, k <= kStageMaxK).  Stage s
// splits each row of candidates into chunks of kStageChunk; a workgroup keeps
// its chunk's local top-k (value and original index), so every key of the
// row's top-k survives: a key beaten by fewer than k keys of the row is beaten
// by fewer than k keys of its chunk (ties broken by position, and positions
// follow the original index order).  Chunk c of a full stage writes its k
// candidates at c*k, in ascending position order, so the candidate rows stay
// in ascending original index order.  The last stage (one chunk) writes the
// original indices of its top-k to out.
//
// The first stage also bounds the row's k-th key from below: chunk c writes
// x_c, a lower bound of its ceil(k/C)-th largest key (C chunks; the waves'
// lane-maximum bound of select_row), so at least k keys of the row are >=
// min_c x_c.  Later stages treat keys under that minimum as unselectable:
// their chunks hold few selectable candidates and end in select_row's
// take-all path, and a chunk with fewer than k writes -inf after them (below
// the floor whenever a chunk can run short).
// ---------------------------------------------------------------------------
constexpr int kStageMaxK = 1024;

__global__ __launch_bounds__(256) void topk_stage_kernel(const float* __restrict__ in_val,
                                                         const int32_t* __restrict__ in_idx, int64_t in_ld,
                                                         int n, int k, float* __restrict__ out_val,
                                                         int32_t* __restrict__ out_idx, int64_t out_ld,
                                                         int32_t* __restrict__ out, uint32_t* __restrict__ bounds,
                                                         int n_bounds, int bound_j) {
  constexpr int VPL = kStageChunk / 256;
  __shared__ int32_t sel[kStageChunk];
  __shared__ uint32_t wave_bound[4];
  const int row = blockIdx.y, c = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int base = c * kStageChunk;
  const int len = min(kStageChunk, n - base);
  const int kc = min(k, len);
  const float* vals = in_val + static_cast<int64_t>(row) * in_ld + base;
  const int32_t* idx = in_idx ? in_idx + static_cast<int64_t>(row) * in_ld + base : nullptr;
  const bool first = in_idx == nullptr;
  uint32_t floor = 0;
  if (!first) {   // the smallest of the first stage's chunk bounds
    floor = 0xFFFFFFFFu;
    for (int b = 0; b < n_bounds; ++b) floor = min(floor, bounds[static_cast<int64_t>(row) * n_bounds + b]);
  }
  uint32_t lane_max = 0;
  const int kk = select_row<VPL, false>(vals, len, kc, sel, floor, &lane_max);
  if (first && bounds) {
    const uint32_t x = wave_lower_bound(lane_max, bound_j, wave_minmax_u32<true>(lane_max),
                                        wave_minmax_u32<false>(lane_max != 0 ? lane_max : 0xFFFFFFFFu));
    if (lane == 0) wave_bound[wave] = x;
    __syncthreads();
    if (threadIdx.x == 0)
      bounds[static_cast<int64_t>(row) * n_bounds + c] =
          min(min(wave_bound[0], wave_bound[1]), min(wave_bound[2], wave_bound[3]));
  }
  if (out) {   // last stage: original indices, ascending (kk = k: at least k keys reach it)
    int32_t* orow = out + static_cast<int64_t>(row) * k;
    for (int j = threadIdx.x; j < kc; j += 256) orow[j] = j >= kk ? -1 : idx ? idx[sel[j]] : base + sel[j];
    return;
  }
  const int64_t o = static_cast<int64_t>(row) * out_ld + static_cast<int64_t>(c) * k;
  for (int j = threadIdx.x; j < kc; j += 256) {
    const int pos = j < kk ? sel[j] : 0;
    out_val[o + j] = j < kk ? vals[pos] : -__builtin_huge_valf();
    out_idx[o + j] = idx ? idx[pos] : base + pos;
  }
}

// The last stage of rows whose candidates outgrow one 4096-key chunk but fit
// one 1024-thread workgroup (at most kWideFinal): WideSelect over the whole
// candidate row, keys under the first stage's floor left out, in place of
// further 4096-key stages (cfg4: one launch instead of three).
constexpr int kWideFinal = 1024 * 40;

template <int VPL>
__global__ __launch_bounds__(1024) void topk_wide_final_kernel(const float* __restrict__ in_val,
                                                               const int32_t* __restrict__ in_idx, int64_t in_ld,
                                                               int n, int k, const uint32_t* __restrict__ bounds,
                                                               int n_bounds, int32_t* __restrict__ out) {
  using WS = WideSelect<VPL, false>;
  __shared__ typename WS::Shared sh;
  const int row = blockIdx.x;
  uint32_t floor = 0xFFFFFFFFu;
  for (int b = 0; b < n_bounds; ++b) floor = min(floor, bounds[static_cast<int64_t>(row) * n_bounds + b]);
  WS ws;
  ws.load(in_val + static_cast<int64_t>(row) * in_ld, n, floor);
  const int kk = ws.run(k, sh);
  int32_t* orow = out + static_cast<int64_t>(row) * k;
  const int32_t* irow = in_idx + static_cast<int64_t>(row) * in_ld;
  ws.place(sh, [&](int pos, int o, int) { orow[o] = irow[pos]; });
  for (int o = kk + static_cast<int>(threadIdx.x); o < k; o += 1024) orow[o] = -1;   // not reached: k keys pass the floor
}

// ---------------------------------------------------------------------------
// Histogram-and-filter top-k for long rows of at most kFilterMaxChunks chunks
// of kStageChunk keys whose candidate lists fit one WideSelect (chunks * k <=
// kFilterMaxLists): three light launches instead of exact per-chunk
// selections.
//  1. topk_hist_kernel: each chunk histograms its keys over the top
//     kHistBits bits of the order-preserving key (sign, exponent, 3 mantissa
//     bits: bins 1/8 of an octave wide) and writes the part that can hold the
//     row's k-th key: t_c, the bin where its own count from the top reaches
//     k (its lowest bin if it holds fewer keys), the kWin bins from t_c up,
//     and how many of its keys lie above them.  The row's k-th key x is never
//     below a chunk's own k-th key (else that chunk alone would hold k keys
//     above x), so x lies in a bin >= t_c for every full chunk.
//  2. topk_filter_kernel: the row's floor is the lower edge of the highest
//     bin b whose count from the top reaches k, with every chunk's count
//     taken from its window: exact for b in [max t_c, min t_c + kWin], never
//     more than the true count elsewhere (a chunk's keys below t_c, or above
//     a bin past its window, are left out), so at least k keys are >= floor
//     and, with b in the exact range, fewer than k + (b's count) pass.  Each
//     chunk keeps its keys >= floor, in position order, in its own list of k
//     slots (value, original index) with a count; a chunk where more than k
//     pass keeps its exact top-k among them (only those can be in the row's
//     top-k).
//  3. topk_lists_final_kernel: one 1024-thread WideSelect per row over the
//     concatenated lists (chunk offsets from one wave scan of the counts),
//     which are in ascending original index order, so the output is too.
// A minimum of per-chunk lower bounds (the staged path's floor) let 5k-31k of
// cfg4's 131072 scores per row through.
// ---------------------------------------------------------------------------
constexpr int kFilterMaxChunks = 64;
constexpr int kFilterMaxLists = 32 * 1024;   // list slots per row (chunks * k): 32 keys per thread
constexpr int kFilterVPL = kStageChunk / 256;   // keys per thread of a chunk

__global__ __launch_bounds__(256) void topk_hist_kernel(const float* __restrict__ values, int64_t ld, int n, int k,
                                                        int n_chunks, int32_t* __restrict__ win) {
  __shared__ uint32_t h[kHistBins];
  __shared__ int wave_sum[4];
  __shared__ int t_sh;
  const int row = blockIdx.y, c = blockIdx.x, tid = threadIdx.x;
  for (int i = tid; i < kHistBins; i += 256) h[i] = 0;
  if (tid == 0) t_sh = 0;
  __syncthreads();
  const int base = c * kStageChunk;
  const int len = min(kStageChunk, n - base);
  const float* vals = values + static_cast<int64_t>(row) * ld + base;
  uint32_t key[kFilterVPL];   // every load in flight before the first atomic
#pragma unroll
  for (int i = 0; i < kFilterVPL; ++i) key[i] = f32_sortable(vals[min(tid * kFilterVPL + i, len - 1)]);
#pragma unroll
  for (int i = 0; i < kFilterVPL; ++i)
    if (tid * kFilterVPL + i < len) atomicAdd(&h[key[i] >> (32 - kHistBits)], 1u);
  __syncthreads();
  chunk_window<256, false>(h, min(k, len), win + (static_cast<int64_t>(row) * n_chunks + c) * kWinWords, wave_sum,
                           &t_sh);
}

__global__ __launch_bounds__(256) void topk_filter_kernel(const float* __restrict__ values, int64_t ld, int n, int k,
                                                          const int32_t* __restrict__ win, int n_chunks,
                                                          float* __restrict__ lval, int32_t* __restrict__ lidx,
                                                          int32_t* __restrict__ lcnt) {
  __shared__ int32_t sel[kStageChunk];
  __shared__ int wave_sum[4];
  __shared__ int wl[kFilterMaxChunks * kWinWords];   // the row's windows, then their suffix sums in place
  __shared__ int best_sh;
  const int row = blockIdx.y, c = blockIdx.x, tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int base = c * kStageChunk;
  const int len = min(kStageChunk, n - base);
  const float* vals = values + static_cast<int64_t>(row) * ld + base;
  // this thread's keys [tid * VPL, tid * VPL + VPL) of the chunk, and the
  // row's windows, all loads in flight before the floor is worked out
  float v[kFilterVPL];
#pragma unroll
  for (int i = 0; i < kFilterVPL; ++i) v[i] = vals[min(tid * kFilterVPL + i, len - 1)];
  const int32_t* wr = win + static_cast<int64_t>(row) * n_chunks * kWinWords;
  {
    constexpr int U = (kFilterMaxChunks * kWinWords + 255) / 256;
    const int nw = n_chunks * kWinWords;
    int x[U];   // every load issued before the first LDS store
#pragma unroll
    for (int u = 0; u < U; ++u) x[u] = wr[min(tid + 256 * u, nw - 1)];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (tid + 256 * u < nw) wl[tid + 256 * u] = x[u];
  }
  if (tid == 0) best_sh = 0x7FFFFFFF;
  __syncthreads();
  // window j: wl[j*W] = t_j, wl[j*W + 1] = keys above it, wl[j*W + 2 + i] = bin t_j + i;
  // in place: wl[j*W + 1 + d] = keys of chunk j in bins >= t_j + d (d = 0..64)
  int top = 0;
  for (int j0 = wave; j0 < n_chunks; j0 += 8) {   // windows j0 and j0 + 4 of this wave at a time
    const bool two = j0 + 4 < n_chunks;            // wave-uniform
    int* w0 = wl + j0 * kWinWords;
    int* w1 = wl + (two ? j0 + 4 : j0) * kWinWords;
    const int t0 = w0[0], t1 = w1[0], over0 = w0[1], over1 = w1[1];
    const int b0 = w0[2 + kWin - 1 - lane], b1 = w1[2 + kWin - 1 - lane];   // bins 63 - lane
    const int x0 = wave_incl_scan_dpp(b0), x1 = wave_incl_scan_dpp(b1);   // bins 63 - lane .. 63
    __builtin_amdgcn_wave_barrier();   // (a wave's LDS reads complete before its writes)
    w0[kWin - lane] = x0 + over0;      // d = 63 - lane, at 1 + d
    if (lane == 0) w0[1 + kWin] = over0;   // d = 64
    if (two) {
      w1[kWin - lane] = x1 + over1;
      if (lane == 0) w1[1 + kWin] = over1;
    }
    top = max(top, max(t0, t1) + kWin - 1);
  }
  if (lane == 0) wave_sum[wave] = top;
  __syncthreads();
  const int top_bin = min(max(max(wave_sum[0], wave_sum[1]), max(wave_sum[2], wave_sum[3])), kHistBins - 1);
  {
    const int b = top_bin - tid;   // thread j evaluates bin top - j
    bool hit = false;
    if (b >= 0) {
      int cum = 0;   // never above the row's true count of keys in bins >= b
      for (int j0 = 0; j0 < n_chunks; j0 += 8) {   // eight windows' reads in flight at a time
        int t8[8], v8[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) t8[u] = wl[min(j0 + u, n_chunks - 1) * kWinWords];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int d = b - t8[u];
          v8[u] = wl[min(j0 + u, n_chunks - 1) * kWinWords + 1 + min(max(d, 0), kWin)];
          v8[u] = d > kWin || j0 + u >= n_chunks ? 0 : v8[u];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) cum += v8[u];
      }
      hit = cum >= k;
    }
    // The count only grows with the thread index (lower bins): a wave's first
    // hit is its candidate for the highest such bin, one LDS atomic per wave.
    const uint64_t hits = __ballot(hit);
    if (hits != 0 && lane == 0) atomicMin(&best_sh, wave * 64 + static_cast<int>(__builtin_ctzll(hits)));
  }
  __syncthreads();
  const uint32_t floor = best_sh == 0x7FFFFFFF ? 0u : static_cast<uint32_t>(top_bin - best_sh) << (32 - kHistBits);
  uint32_t pass = 0;
#pragma unroll
  for (int i = 0; i < kFilterVPL; ++i) {
    const int p = tid * kFilterVPL + i;
    pass |= static_cast<uint32_t>(p < len && f32_sortable(v[i]) >= floor) << i;
  }
  const int cnt = __popc(pass);
  const int incl = wave_incl_scan_dpp(cnt);
  if (lane == 63) wave_sum[wave] = incl;
  __syncthreads();
  int before = incl - cnt, total = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    before += w < wave ? wave_sum[w] : 0;
    total += wave_sum[w];
  }
  const int64_t o = (static_cast<int64_t>(row) * n_chunks + c) * k;
  if (total <= k) {   // uniform: every passing key, in position order
#pragma unroll
    for (int i = 0; i < kFilterVPL; ++i) {
      if ((pass >> i) & 1u) {
        lval[o + before] = v[i];
        lidx[o + before] = base + tid * kFilterVPL + i;
        ++before;
      }
    }
    if (tid == 0) lcnt[static_cast<int64_t>(row) * n_chunks + c] = total;
    return;
  }
  // more than k pass: the chunk's exact top-k among them
  const int kk = select_row<kFilterVPL, false>(vals, len, k, sel, floor);
  for (int j = tid; j < kk; j += 256) {
    lval[o + j] = vals[sel[j]];
    lidx[o + j] = base + sel[j];
  }
  if (tid == 0) lcnt[static_cast<int64_t>(row) * n_chunks + c] = kk;
}

// Rows whose lists hold at most kFinalLds keys: gathered into LDS in list
// order and selected by WideSelect with kFinalLds / 1024 keys per thread;
// longer lists: WideSelect with VPLB keys per thread (covering chunks * k),
// read from the lists directly.
constexpr int kFinalLds = 4096, kFinalLdsLog2 = 12;

template <int VPLB>
__global__ __launch_bounds__(1024) void topk_lists_final_kernel(const float* __restrict__ lval,
                                                                const int32_t* __restrict__ lidx,
                                                                const int32_t* __restrict__ lcnt, int n_chunks,
                                                                int k, int32_t* __restrict__ out) {
  using WB = WideSelect<VPLB, false>;
  using WC = WideSelect<kFinalLds / 1024, false>;
  __shared__ union {
    typename WB::Shared b;
    typename WC::Shared c;
  } sh;
  __shared__ float cval[kFinalLds];
  __shared__ int32_t cidx[kFinalLds];
  __shared__ int off[kFilterMaxChunks + 1];
  const int row = blockIdx.x, tid = threadIdx.x;
  if (tid < 64) {   // list offsets: one load per chunk, a wave scan
    const int len = tid < n_chunks ? lcnt[static_cast<int64_t>(row) * n_chunks + tid] : 0;
    const int incl = wave_incl_scan_dpp(len);
    if (tid < n_chunks) off[tid] = incl - len;
    if (tid == 63) off[n_chunks] = incl;   // the total
  }
  __syncthreads();
  const int total = off[n_chunks];
  const int64_t rbase = static_cast<int64_t>(row) * n_chunks * k;
  int32_t* orow = out + static_cast<int64_t>(row) * k;
  auto entry = [&](int p) -> int64_t {   // list slot of concatenated position p < total
    int lo = 0, hi = n_chunks - 1;        // the last chunk whose list starts at or before p
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (off[mid] <= p) lo = mid;
      else hi = mid - 1;
    }
    return rbase + static_cast<int64_t>(lo) * k + (p - off[lo]);
  };
  if (total <= kFinalLds) {   // uniform across the workgroup
    constexpr int U = kFinalLds / 1024;
    float xv[U];
    int32_t xi[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {   // every load issued before the first LDS store
      const int p = tid + 1024 * u;
      const int64_t e = p < total ? entry(p) : 0;
      xv[u] = lval[e];
      xi[u] = lidx[e];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int p = tid + 1024 * u;
      if (p < total) {
        cval[p] = xv[u];
        cidx[p] = xi[u];
      }
    }
#pragma unroll
    for (int j = 0; j < WC::NB / 1024; ++j) sh.c.hist[0][tid + 1024 * j] = 0;   // (counted below)
    __syncthreads();
    WC wc;
    int ninf = 0;
#pragma unroll
    for (int i = 0; i < kFinalLds / 1024; ++i) {
      const int p = WC::pos(i);
      wc.set(i, p < total ? cval[p] : 0.0f, p < total);
      wc.count(i, sh.c, ninf);
    }
    wc.count_done(sh.c, ninf);
    const int kk = wc.run_counted(k, sh.c);
    wc.place_uniform(sh.c, [&](int p, int o, int) { orow[o] = cidx[p]; });
    for (int o = kk + tid; o < k; o += 1024) orow[o] = -1;   // not reached: k keys pass the floor
    return;
  }
  // (the original index of a taken key is looked up again from its position:
  // a register array indexed by the taken slot would live in scratch)
  WB wb;
#pragma unroll
  for (int i = 0; i < VPLB; ++i) {
    const int p = wb.pos(i);
    const bool ok = p < total;
    wb.set(i, ok ? lval[ok ? entry(p) : 0] : 0.0f, ok);
  }
  const int kk = wb.run(k, sh.b);
  wb.place(sh.b, [&](int p, int o, int) { orow[o] = lidx[entry(p)]; });
  for (int o = kk + tid; o < k; o += 1024) orow[o] = -1;   // not reached: k keys pass the floor
}

// ---------------------------------------------------------------------------
// The three steps above in one launch, for grids whose workgroups are all
// resident at once (rows * chunks <= kFusedMaxWGs; one 1024-thread workgroup
// per chunk, 4 keys per thread held in registers throughout):
//  a. the chunk's histogram and window, published with device-coherent
//     stores, then the row's first ticket;
//  b. the workgroup waits until every chunk of its row has published (a
//     bounded wait: past g_spin_ticks of the real-time clock it takes floor 0,
//     i.e. keeps its exact top-k, which is always a valid list, so the launch
//     ends whatever the residency);
//  c. the row's floor exactly as topk_filter_kernel computes it, and the
//     chunk's list;
//  d. the row's second ticket: the last chunk to arrive selects from the lists
//     as topk_lists_final_kernel does and returns both tickets to zero.
// ---------------------------------------------------------------------------
constexpr int kFusedMaxWGs = 256;
constexpr int kFusedVPL = kStageChunk / 1024;   // keys per thread
constexpr int kTicketSlotWords = kFusedMaxWGs;  // (windows published, lists written) per row; rows <= 128
constexpr int kTicketSlots = 4096;
constexpr int64_t kSpinTicks = 1 << 17;           // ~1.3 ms of the 100 MHz real-time clock
int64_t g_spin_ticks = kSpinTicks;                // qkv_topk_set_wait_limit

// given: the windows are in win already (written by an earlier launch, such
// as the decode scoring of qkv_int4_decode_topk): a and b are skipped.
__global__ __launch_bounds__(1024) void topk_fused_kernel(const float* __restrict__ values, int64_t ld, int n,
                                                          int k, int n_chunks, uint64_t spin_ticks,
                                                          uint32_t* __restrict__ tickets, int32_t* __restrict__ win,
                                                          float* __restrict__ lval, int32_t* __restrict__ lidx,
                                                          int32_t* __restrict__ lcnt, int32_t* __restrict__ out,
                                                          int given) {
  using WS = WideSelect<kFusedVPL, false>;
  using WB = WideSelect<kFilterMaxLists / 1024, false>;
  constexpr int NW = 16, BPT = kHistBins / 1024;
  __shared__ union {
    uint32_t h[kHistBins];                  // a: the chunk's histogram
    int wl[kFilterMaxChunks * kWinWords];   // c: the row's windows, then their suffix sums
    struct {
      typename WS::Shared s;
      float cval[kFinalLds];
      int32_t cidx[kFinalLds];
    } fin;                                  // c (more than k pass) and d
    typename WB::Shared b;                  // d, lists longer than kFinalLds
  } sh;
  __shared__ int wave_a[NW], wave_b[NW];
  __shared__ int t_sh, best_sh, flag_sh;
  __shared__ int off[kFilterMaxChunks + 1], lens[kFilterMaxChunks];
  const int row = blockIdx.y, c = blockIdx.x, tid = threadIdx.x;
  const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int base = c * kStageChunk;
  const int len = min(kStageChunk, n - base);
  const float* vals = values + static_cast<int64_t>(row) * ld + base;
  uint32_t* tk = tickets + 2 * static_cast<int64_t>(row);

  // a. histogram of the keys' top kHistBits bits
  if (tid == 0) {
    t_sh = 0;
    best_sh = 0x7FFFFFFF;
    flag_sh = 1;
  }
  WS ws;
  ws.load(vals, len);   // key i of this thread: chunk position WS::pos(i)
  if (!given) {   // uniform
#pragma unroll
    for (int i = 0; i < BPT; ++i) sh.h[tid + 1024 * i] = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kFusedVPL; ++i)
      if (ws.on(i)) atomicAdd(&sh.h[ws.u[i] >> (32 - kHistBits)], 1u);
    __syncthreads();
    chunk_window<1024, true>(sh.h, min(k, len), win + (static_cast<int64_t>(row) * n_chunks + c) * kWinWords,
                             wave_a, &t_sh);
    // Every window store of this workgroup has completed before the ticket.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    // b. wait for the row's other chunks
    if (tid == 0) {
      // The windows went out as coherent (sc1) stores and have completed
      // (s_waitcnt above) before the ticket; the compiler-only fences keep the
      // compiler from moving memory operations across the ticket and the wait.
      // Release/acquire orderings here would add a whole-L2 write-back and
      // invalidate per workgroup (2.7 us at 8 rows x 32 chunks).
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      __hip_atomic_fetch_add(tk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
      int ok = 1;
      while (__hip_atomic_load(tk, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < static_cast<uint32_t>(n_chunks)) {
        __builtin_amdgcn_s_sleep(2);
        if (__builtin_amdgcn_s_memrealtime() - t0 >= spin_ticks) {
          ok = 0;
          break;
        }
      }
      __atomic_signal_fence(__ATOMIC_SEQ_CST);
      flag_sh = ok;
    }
  }
  __syncthreads();

  // c. the row's floor (as in topk_filter_kernel), then this chunk's list
  uint32_t floor = 0;
  if (flag_sh) {   // uniform
    const int32_t* wr = win + static_cast<int64_t>(row) * n_chunks * kWinWords;
    {
      constexpr int U = (kFilterMaxChunks * kWinWords + 1023) / 1024;
      const int nw = n_chunks * kWinWords;
      int x[U];
#pragma unroll
      for (int u = 0; u < U; ++u) x[u] = ld_coherent(wr + min(tid + 1024 * u, nw - 1));
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (tid + 1024 * u < nw) sh.wl[tid + 1024 * u] = x[u];
    }
    __syncthreads();
    int top = 0;
    for (int j = wave; j < n_chunks; j += NW) {   // window j: suffix sums in place
      int* wj = sh.wl + j * kWinWords;
      const int tj = wj[0], overj = wj[1];
      const int x = wave_incl_scan_dpp(wj[2 + kWin - 1 - lane]);   // bins 63 - lane .. 63
      __builtin_amdgcn_wave_barrier();   // (a wave's LDS reads complete before its writes)
      wj[kWin - lane] = x + overj;
      if (lane == 0) wj[1 + kWin] = overj;
      top = max(top, tj + kWin - 1);
    }
    if (lane == 0) wave_a[wave] = top;
    __syncthreads();
    int top_bin = 0;
#pragma unroll
    for (int v = 0; v < NW; ++v) top_bin = max(top_bin, wave_a[v]);
    top_bin = min(top_bin, kHistBins - 1);
    const int b = top_bin - tid;   // thread j evaluates bin top - j
    bool hit = false;
    if (b >= 0) {
      int cum = 0;   // never above the row's true count of keys in bins >= b
      for (int j0 = 0; j0 < n_chunks; j0 += 8) {
        int t8[8], v8[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) t8[u] = sh.wl[min(j0 + u, n_chunks - 1) * kWinWords];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int d = b - t8[u];
          v8[u] = sh.wl[min(j0 + u, n_chunks - 1) * kWinWords + 1 + min(max(d, 0), kWin)];
          v8[u] = d > kWin || j0 + u >= n_chunks ? 0 : v8[u];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) cum += v8[u];
      }
      hit = cum >= k;
    }
    const uint64_t hits = __ballot(hit);   // one LDS atomic per wave, as in topk_filter_kernel
    if (hits != 0 && lane == 0) atomicMin(&best_sh, wave * 64 + static_cast<int>(__builtin_ctzll(hits)));
    __syncthreads();
    floor = best_sh == 0x7FFFFFFF ? 0u : static_cast<uint32_t>(top_bin - best_sh) << (32 - kHistBits);
  }
  uint64_t bl[kFusedVPL];
  int wtot = 0;
#pragma unroll
  for (int i = 0; i < kFusedVPL; ++i) {
    bl[i] = __ballot(ws.on(i) && ws.u[i] >= floor);
    wtot += __popcll(bl[i]);
  }
  if (lane == 0) wave_b[wave] = wtot;   // wave_b's last reads were before two barriers
  __syncthreads();
  int before = 0, total = 0;
#pragma unroll
  for (int v = 0; v < NW; ++v) {
    before += v < wave ? wave_b[v] : 0;
    total += wave_b[v];
  }
  const int64_t o = (static_cast<int64_t>(row) * n_chunks + c) * k;
  if (total <= k) {   // uniform: every passing key, in position order
    const uint64_t below = (1ull << lane) - 1ull;
#pragma unroll
    for (int i = 0; i < kFusedVPL; ++i) {
      if ((bl[i] >> lane) & 1ull) {
        const int at = before + __popcll(bl[i] & below);
        st_coherent(lval + o + at, sortable_f32(ws.u[i]));
        st_coherent(lidx + o + at, base + WS::pos(i));
      }
      before += __popcll(bl[i]);
    }
    if (tid == 0) st_coherent(lcnt + static_cast<int64_t>(row) * n_chunks + c, total);
  } else {   // more than k pass: the chunk's exact top-k among them
#pragma unroll
    for (int i = 0; i < kFusedVPL; ++i)
      if (ws.on(i) && ws.u[i] < floor) ws.valid &= ~(1ull << i);
    const int kk = ws.run(k, sh.fin.s);
    ws.place(sh.fin.s, [&](int p, int at, int) {
      st_coherent(lval + o + at, vals[p]);
      st_coherent(lidx + o + at, base + p);
    });
    if (tid == 0) st_coherent(lcnt + static_cast<int64_t>(row) * n_chunks + c, kk);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // d. the row's last chunk selects from the lists
  if (tid == 0) {
    // the lists, coherent stores completed above, stay before this ticket
    // and the last chunk's list reads after it (compiler-only fences)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const uint32_t a = __hip_atomic_fetch_add(tk + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const bool last = a == static_cast<uint32_t>(n_chunks - 1);
    if (last) {   // every chunk of the row has left its wait
      __hip_atomic_store(tk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(tk + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    flag_sh = last;
  }
  __syncthreads();
  if (!flag_sh) return;
  // The lists' counts and the first S entries of every list in one batch of
  // loads (S = kFinalLds / chunks rounded up to a power of two); a list
  // longer than S sends the row through a second round of loads.
  const int64_t rbase = static_cast<int64_t>(row) * n_chunks * k;
  const int sh_s = kFinalLdsLog2 - (n_chunks <= 1 ? 0 : 32 - __builtin_clz(n_chunks - 1));
  constexpr int U = kFinalLds / 1024;
  float xv[U];
  int32_t xi[U];
  int l = 0;
  if (tid < 64)   // (clamped: a count outside [0, k] cannot send a load outside the lists)
    l = tid < n_chunks ? min(max(ld_coherent(lcnt + static_cast<int64_t>(row) * n_chunks + tid), 0), k) : 0;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int f = tid + 1024 * u, j = f >> sh_s, slot = f & ((1 << sh_s) - 1);
    const int64_t e = j < n_chunks && slot < k ? rbase + static_cast<int64_t>(j) * k + slot : rbase;
    xv[u] = ld_coherent(lval + e);
    xi[u] = ld_coherent(lidx + e);
  }
  if (tid < 64) {   // list offsets: a wave scan of the counts
    const int x = wave_incl_scan_dpp(l);
    if (tid < n_chunks) {
      off[tid] = x - l;
      lens[tid] = l;
    }
    if (tid == 63) off[n_chunks] = x;
    const bool longer = __ballot(l > (1 << sh_s)) != 0;
    if (tid == 0) flag_sh = longer;
  }
  __syncthreads();
  const int all = off[n_chunks];
  int32_t* orow = out + static_cast<int64_t>(row) * k;
  auto entry = [&](int p) -> int64_t {   // list slot of concatenated position p < all
    int lo = 0, hi = n_chunks - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (off[mid] <= p) lo = mid;
      else hi = mid - 1;
    }
    return rbase + static_cast<int64_t>(lo) * k + (p - off[lo]);
  };
  if (all <= kFinalLds) {   // uniform
    if (!flag_sh) {   // every entry is among those loaded
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int f = tid + 1024 * u, j = f >> sh_s, slot = f & ((1 << sh_s) - 1);
        if (j < n_chunks && slot < lens[j]) {
          sh.fin.cval[off[j] + slot] = xv[u];
          sh.fin.cidx[off[j] + slot] = xi[u];
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int p = tid + 1024 * u;
        const int64_t e = p < all ? entry(p) : rbase;
        xv[u] = ld_coherent(lval + e);
        xi[u] = ld_coherent(lidx + e);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int p = tid + 1024 * u;
        if (p < all) {
          sh.fin.cval[p] = xv[u];
          sh.fin.cidx[p] = xi[u];
        }
      }
    }
#pragma unroll
    for (int j = 0; j < WS::NB / 1024; ++j) sh.fin.s.hist[0][tid + 1024 * j] = 0;   // (counted below)
    __syncthreads();
    WS wc;
    int ninf = 0;
#pragma unroll
    for (int i = 0; i < kFusedVPL; ++i) {
      const int p = WS::pos(i);
      wc.set(i, p < all ? sh.fin.cval[p] : 0.0f, p < all);
      wc.count(i, sh.fin.s, ninf);
    }
    wc.count_done(sh.fin.s, ninf);
    const int kk = wc.run_counted(k, sh.fin.s);
    wc.place_uniform(sh.fin.s, [&](int p, int at, int) { orow[at] = sh.fin.cidx[p]; });
    for (int at = kk + tid; at < k; at += 1024) orow[at] = -1;   // not reached: k keys pass the floor
    return;
  }
  WB wb;
#pragma unroll
  for (int i = 0; i < kFilterMaxLists / 1024; ++i) {
    const int p = wb.pos(i);
    const bool ok = p < all;
    wb.set(i, ok ? ld_coherent(lval + (ok ? entry(p) : rbase)) : 0.0f, ok);
  }
  const int kk = wb.run(k, sh.b);
  wb.place(sh.b, [&](int p, int at, int) { orow[at] = ld_coherent(lidx + entry(p)); });
  for (int at = kk + tid; at < k; at += 1024) orow[at] = -1;   // not reached: k keys pass the floor
}

// Candidates left after a stage over n keys: k from every full chunk, and
// min(k, rest) from the last.
int64_t stage_out(int64_t n, int64_t k) {
  const int64_t c = cdiv(n, kStageChunk);
  return (c - 1) * k + std::min<int64_t>(k, n - (c - 1) * kStageChunk);
}

bool staged(int64_t n, int64_t k) { return n > kStageChunk && k <= kStageMaxK; }

// Staged rows that take the histogram-and-filter path.
bool filtered(int64_t n, int64_t k) {
  const int64_t chunks = cdiv(n, kStageChunk);
  return staged(n, k) && chunks <= kFilterMaxChunks && chunks * k <= kFilterMaxLists;
}

template <bool FINITE>
int launch_rows(const float* values, int64_t rows, int64_t n, int64_t ld, int64_t k, int32_t* out,
                hipStream_t st) {
  const int nn = static_cast<int>(n), kk = static_cast<int>(k);
  // One wave per row pays off when rows are many and short (measured: 65536
  // rows of 1024 keys 181 -> 110 us; 64 rows of 2048 keys 6.7 -> 11.3 us).
  if (n <= 64 * kWaveMaxVPL && rows >= kWaveMinRows) {
    const unsigned wg4 = static_cast<unsigned>(cdiv(rows, 4));
    if (FINITE && k <= 64 && n > 512) {   // candidate lists (prefill block maxima)
      if (n <= 1024) topk_cand_wave_kernel<16><<<wg4, 256, 0, st>>>(values, rows, nn, ld, kk, out);
      else topk_cand_wave_kernel<32><<<wg4, 256, 0, st>>>(values, rows, nn, ld, kk, out);
      return check_launch("qkv_topk");
    }
    if (n <= 256) topk_wave_kernel<4, FINITE><<<wg4, 256, 0, st>>>(values, rows, nn, ld, kk, out);
    else if (n <= 512) topk_wave_kernel<8, FINITE><<<wg4, 256, 0, st>>>(values, rows, nn, ld, kk, out);
    else if (n <= 1024) topk_wave_kernel<16, FINITE><<<wg4, 256, 0, st>>>(values, rows, nn, ld, kk, out);
    else topk_wave_kernel<32, FINITE><<<wg4, 256, 0, st>>>(values, rows, nn, ld, kk, out);
    return check_launch("qkv_topk");
  }
  const unsigned wg = static_cast<unsigned>(rows);
  if (n <= 256) topk_rows_kernel<1, FINITE><<<wg, 256, 0, st>>>(values, nn, ld, kk, out);
  else if (n <= 512) topk_rows_kernel<2, FINITE><<<wg, 256, 0, st>>>(values, nn, ld, kk, out);
  else if (n <= 1024) topk_rows_kernel<4, FINITE><<<wg, 256, 0, st>>>(values, nn, ld, kk, out);
  else if (n <= 2048) topk_rows_kernel<8, FINITE><<<wg, 256, 0, st>>>(values, nn, ld, kk, out);
  else topk_rows_kernel<16, FINITE><<<wg, 256, 0, st>>>(values, nn, ld, kk, out);
  return check_launch("qkv_topk");
}

}  // namespace
}  // namespace qkv

// Row tickets of topk_fused_kernel: a file-scope device array, one copy per
// GPU, held until the process ends, zero when the code object loads.  Host
// code never passes the array's name to a kernel (it is a host-side stand-in);
// each GPU's copy is found with hipGetSymbolAddress once, with that GPU
// current.  Calls take its slots in turn, so calls in flight together on one
// GPU (on different streams) count in different words unless kTicketSlots
// calls were issued between them; every completed call leaves its words zero.
// A call made while its stream is being captured into a graph keeps its slot
// for every replay of that graph, so such a slot is reserved: no later call is
// given it (at most kTicketSlots - 1 captured calls per GPU and process).
static __device__ __align__(256) uint32_t topk_tickets[qkv::kTicketSlots * qkv::kTicketSlotWords];

namespace qkv {
namespace {

constexpr int kTicketDevices = 64;
std::mutex g_ticket_mu;
uint32_t* g_ticket_pool[kTicketDevices];
std::atomic<uint32_t> g_ticket_next[kTicketDevices];
std::vector<bool> g_ticket_reserved[kTicketDevices];   // slots held by captured graphs (under g_ticket_mu)
uint32_t g_ticket_n_reserved[kTicketDevices];

// This call's ticket words on the current device.
int ticket_slot(hipStream_t stream, uint32_t** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kTicketDevices)
    return fail(QKV_ERR_LAUNCH, "qkv_topk_ws: no current device below %d", kTicketDevices);
  uint32_t* pool = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_ticket_mu);
    if (!g_ticket_pool[dev]) {
      void* p = nullptr;
      const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(topk_tickets));
      if (e != hipSuccess || !p)
        return fail(QKV_ERR_LAUNCH, "qkv_topk_ws: hipGetSymbolAddress(topk_tickets) on device %d: %s", dev,
                    hipGetErrorString(e));
      g_ticket_pool[dev] = static_cast<uint32_t*>(p);
    }
    pool = g_ticket_pool[dev];
  }
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cap) != hipSuccess)
    return fail(QKV_ERR_LAUNCH, "qkv_topk_ws: hipStreamIsCapturing failed");
  const bool captured = cap == hipStreamCaptureStatusActive;
  uint32_t slot = 0;
  {
    std::lock_guard<std::mutex> lock(g_ticket_mu);
    std::vector<bool>& reserved = g_ticket_reserved[dev];
    if (reserved.empty()) reserved.assign(kTicketSlots, false);
    if (g_ticket_n_reserved[dev] + 1 >= static_cast<uint32_t>(kTicketSlots))
      return fail(QKV_ERR_UNSUPPORTED, "qkv_topk_ws: %d graph-captured calls hold every ticket slot of device %d",
                  kTicketSlots - 1, dev);
    do {
      slot = g_ticket_next[dev].fetch_add(1u, std::memory_order_relaxed) % kTicketSlots;
    } while (reserved[slot]);
    if (captured) {
      reserved[slot] = true;
      ++g_ticket_n_reserved[dev];
    }
  }
  *out = pool + static_cast<int64_t>(slot) * kTicketSlotWords;
  return QKV_OK;
}

}  // namespace

// The histogram-and-filter path of qkv_topk_ws (filtered(n, k)): the chunk
// windows at the workspace's start, then the per-chunk lists and counts.
// given: the windows are there already (chunk_window layout, written by an
// earlier launch on the stream), so the histogram pass is skipped.
int topk_filtered(const float* values, int64_t rows, int64_t n, int64_t ld, int64_t k, int32_t* out,
                  void* workspace, hipStream_t st, bool given) {
  const int n_bounds = static_cast<int>(cdiv(n, kStageChunk));
  int32_t* win = static_cast<int32_t*>(workspace);
  float* lval = reinterpret_cast<float*>(win + rows * n_bounds * kWinWords);
  int32_t* lidx = reinterpret_cast<int32_t*>(lval + rows * n_bounds * k);
  int32_t* lcnt = lidx + rows * n_bounds * k;
  dim3 grid(static_cast<unsigned>(n_bounds), static_cast<unsigned>(rows));
  if (rows * n_bounds <= kFusedMaxWGs) {
    uint32_t* tickets = nullptr;
    if (int rc = ticket_slot(st, &tickets)) return rc;
    topk_fused_kernel<<<grid, 1024, 0, st>>>(values, ld, static_cast<int>(n), static_cast<int>(k), n_bounds,
                                             static_cast<uint64_t>(g_spin_ticks), tickets, win, lval, lidx, lcnt,
                                             out, given ? 1 : 0);
    return check_launch("qkv_topk_ws");
  }
  if (!given) {
    topk_hist_kernel<<<grid, 256, 0, st>>>(values, ld, static_cast<int>(n), static_cast<int>(k), n_bounds, win);
    if (int rc = check_launch("qkv_topk_ws")) return rc;
  }
  topk_filter_kernel<<<grid, 256, 0, st>>>(values, ld, static_cast<int>(n), static_cast<int>(k), win, n_bounds,
                                           lval, lidx, lcnt);
  if (int rc = check_launch("qkv_topk_ws")) return rc;
  topk_lists_final_kernel<kFilterMaxLists / 1024><<<static_cast<unsigned>(rows), 1024, 0, st>>>(
      lval, lidx, lcnt, n_bounds, static_cast<int>(k), out);
  return check_launch("qkv_topk_ws");
}

// Whether qkv_topk_ws takes the histogram-and-filter path for (n, k).
bool topk_takes_windows(int64_t n, int64_t k) { return filtered(n, k); }

}  // namespace qkv

using namespace qkv;

QKV_EXPORT int qkv_topk(const float* values, int64_t rows, int64_t n, int64_t ld, int64_t k,
                        int32_t* out, void* stream) {
  if (!values || !out) return fail(QKV_ERR_INVALID, "qkv_topk: null pointer");
  if (rows <= 0 || n <= 0 || ld < n || n >= (int64_t(1) << 31))
    return fail(QKV_ERR_INVALID, "qkv_topk: bad sizes rows=%lld n=%lld ld=%lld", (long long)rows,
                (long long)n, (long long)ld);
  if (k < 1 || k > n) return fail(QKV_ERR_INVALID, "qkv_topk: need 1 <= k <= n (k=%lld, n=%lld)",
                                  (long long)k, (long long)n);
  if (rows > 0x7FFFFFFF) return fail(QKV_ERR_INVALID, "qkv_topk: too many rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (n <= 4096) return launch_rows<false>(values, rows, n, ld, k, out, st);
  const unsigned grid = static_cast<unsigned>(rows);
  if (n <= kLdsKeys) {
    topk_kernel<1024, true><<<grid, 1024, n * sizeof(uint32_t), st>>>(values, static_cast<int>(n), ld,
                                                                       static_cast<int>(k), out);
  } else {
    topk_kernel<1024, false><<<grid, 1024, 0, st>>>(values, static_cast<int>(n), ld,
                                                    static_cast<int>(k), out);
  }
  return check_launch("qkv_topk");
}

QKV_EXPORT int64_t qkv_topk_workspace_bytes(int64_t rows, int64_t n, int64_t k) {
  if (rows <= 0 || n <= 0 || k < 1 || k > n) return -1;
  if (!staged(n, k)) return 0;
  const int64_t chunks = cdiv(n, kStageChunk);
  if (filtered(n, k))   // chunk windows, then per-chunk lists of k (value, index) and their counts
    return rows * chunks * (kWinWords + k * 2 + 1) * 4;
  // two candidate buffers (value + index) sized for the first stage's output,
  // then the first stage's chunk bounds
  return 2 * rows * stage_out(n, k) * static_cast<int64_t>(sizeof(float) + sizeof(int32_t)) +
         rows * chunks * static_cast<int64_t>(sizeof(uint32_t));
}

QKV_EXPORT int qkv_topk_ws(const float* values, int64_t rows, int64_t n, int64_t ld, int64_t k, int32_t* out,
                           void* workspace, int64_t workspace_bytes, void* stream) {
  if (!staged(n, k)) return qkv_topk(values, rows, n, ld, k, out, stream);
  if (!values || !out || !workspace) return fail(QKV_ERR_INVALID, "qkv_topk_ws: null pointer");
  if (rows <= 0 || rows > 65535 || ld < n || n >= (int64_t(1) << 31))
    return fail(QKV_ERR_INVALID, "qkv_topk_ws: bad sizes rows=%lld n=%lld ld=%lld", (long long)rows,
                (long long)n, (long long)ld);
  const int64_t need = qkv_topk_workspace_bytes(rows, n, k);
  if (workspace_bytes < need)
    return fail(QKV_ERR_INVALID, "qkv_topk_ws: workspace needs %lld bytes, got %lld", (long long)need,
                (long long)workspace_bytes);
  if (!aligned(workspace, 16)) return fail(QKV_ERR_INVALID, "qkv_topk_ws: workspace must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t n1 = stage_out(n, k);
  float* val_buf[2];
  int32_t* idx_buf[2];
  val_buf[0] = static_cast<float*>(workspace);
  idx_buf[0] = reinterpret_cast<int32_t*>(val_buf[0] + rows * n1);
  val_buf[1] = reinterpret_cast<float*>(idx_buf[0] + rows * n1);
  idx_buf[1] = reinterpret_cast<int32_t*>(val_buf[1] + rows * n1);
  uint32_t* bounds = reinterpret_cast<uint32_t*>(idx_buf[1] + rows * n1);
  const int n_bounds = static_cast<int>(cdiv(n, kStageChunk));
  const int bound_j = static_cast<int>(cdiv(cdiv(k, n_bounds), 4));   // per wave; above 64: no bound
  if (filtered(n, k)) return topk_filtered(values, rows, n, ld, k, out, workspace, st, false);
  const float* cur_val = values;
  const int32_t* cur_idx = nullptr;
  int64_t cur_ld = ld, cur_n = n;
  int buf = 0;
  while (true) {
    const int64_t chunks = cdiv(cur_n, kStageChunk);
    if (cur_idx && chunks > 1 && cur_n <= kWideFinal) {   // the rest in one 1024-thread workgroup per row
      const unsigned wg = static_cast<unsigned>(rows);
      const int nn = static_cast<int>(cur_n), kk = static_cast<int>(k);
      if (cur_n <= 16 * 1024)
        topk_wide_final_kernel<16><<<wg, 1024, 0, st>>>(cur_val, cur_idx, cur_ld, nn, kk, bounds, n_bounds, out);
      else if (cur_n <= 32 * 1024)
        topk_wide_final_kernel<32><<<wg, 1024, 0, st>>>(cur_val, cur_idx, cur_ld, nn, kk, bounds, n_bounds, out);
      else
        topk_wide_final_kernel<40><<<wg, 1024, 0, st>>>(cur_val, cur_idx, cur_ld, nn, kk, bounds, n_bounds, out);
      return check_launch("qkv_topk_ws");
    }
    const bool last = chunks == 1;
    dim3 grid(static_cast<unsigned>(chunks), static_cast<unsigned>(rows));
    topk_stage_kernel<<<grid, 256, 0, st>>>(cur_val, cur_idx, cur_ld, static_cast<int>(cur_n), static_cast<int>(k),
                                            last ? nullptr : val_buf[buf], last ? nullptr : idx_buf[buf], n1,
                                            last ? out : nullptr, bounds, n_bounds, bound_j);
    if (int rc = check_launch("qkv_topk_ws")) return rc;
    if (last) return QKV_OK;
    cur_val = val_buf[buf];
    cur_idx = idx_buf[buf];
    cur_ld = n1;
    cur_n = stage_out(cur_n, k);
    buf ^= 1;
  }
}

QKV_EXPORT int qkv_topk_set_wait_limit(int64_t ticks) {
  g_spin_ticks = ticks < 0 ? kSpinTicks : ticks;
  return QKV_OK;
}

QKV_EXPORT int qkv_prefill_block_topk(const float* bmax, int64_t rows, int64_t n, int64_t ld, int64_t k,
                                      int32_t* out, void* stream) {
  if (!bmax || !out) return fail(QKV_ERR_INVALID, "qkv_prefill_block_topk: null pointer");
  if (rows <= 0 || rows > 0x7FFFFFFF || n <= 0 || ld < n)
    return fail(QKV_ERR_INVALID, "qkv_prefill_block_topk: bad sizes rows=%lld n=%lld ld=%lld", (long long)rows,
                (long long)n, (long long)ld);
  if (n > 4096) return fail(QKV_ERR_UNSUPPORTED, "qkv_prefill_block_topk: at most 4096 blocks per row");
  if (k < 1 || k > n) return fail(QKV_ERR_INVALID, "qkv_prefill_block_topk: need 1 <= k <= n");
  return launch_rows<true>(bmax, rows, n, ld, k, out, static_cast<hipStream_t>(stream));
}
