// Exact top-k selection of one row inside one workgroup, shared by
// the top-k kernels and the fused selection in sparse attention.  Keys map to
// order-preserving uint32 (-0 folded onto +0); the k largest are kept, ties to
// the lower position.
#pragma once

#include "common.h"

namespace qkv {
namespace {

constexpr uint32_t kNegInfKey = 0x007FFFFFu;   // f32_sortable(-inf)


// ---------------------------------------------------------------------------
// Wave-level helpers.  Reductions and scans use DPP (a few cycles a step,
// where an LDS permute round trip costs ~100).
// ---------------------------------------------------------------------------
template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t old, uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(old), static_cast<int>(v), CTRL,
                                                           ROW_MASK, BANK_MASK, false));
}

// Max (IS_MAX) or min over the wave, via the row reduction (quad_perm,
// row_half_mirror, row_mirror) and then row_bcast:15 / row_bcast:31, which
// leave the wave's result in lane 63.
template <bool IS_MAX>
__device__ __forceinline__ uint32_t wave_minmax_u32(uint32_t v) {
  auto op = [](uint32_t a, uint32_t b) { return IS_MAX ? max(a, b) : min(a, b); };
  v = op(v, dpp_u32<0xB1>(v, v));
  v = op(v, dpp_u32<0x4E>(v, v));
  v = op(v, dpp_u32<0x141>(v, v));
  v = op(v, dpp_u32<0x140>(v, v));
  v = op(v, dpp_u32<0x142, 0xA>(v, v));
  v = op(v, dpp_u32<0x143, 0xC>(v, v));
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63));
}

// Inclusive prefix sum over the 64 lanes (row_shr 1,2,3 then 4 and 8 within
// each row of 16, then row_bcast:15 / row_bcast:31 across rows).
__device__ __forceinline__ int wave_incl_scan_dpp(int v) {
  uint32_t x = static_cast<uint32_t>(v);
  uint32_t r = x + dpp_u32<0x111>(0u, x);
  r += dpp_u32<0x112>(0u, x);
  r += dpp_u32<0x113>(0u, x);
  r += dpp_u32<0x114, 0xF, 0xE>(0u, r);
  r += dpp_u32<0x118, 0xF, 0xC>(0u, r);
  r += dpp_u32<0x142, 0xA>(0u, r);
  r += dpp_u32<0x143, 0xC>(0u, r);
  return static_cast<int>(r);
}

// A lower bound of the wave's j-th largest lane value v (0: the lane has
// none), given the wave's largest value vmax and a value vmin <= every
// nonzero v: the largest x with at least j lanes at or above it, resolved to
// 8 bits below the bits vmax and vmin share (the lower bits left zero keep it
// a lower bound); 0 when fewer than j lanes hold a value.  Wave-uniform.
__device__ __forceinline__ uint32_t wave_lower_bound(uint32_t v, int j, uint32_t vmax, uint32_t vmin) {
  if (j > 64 || __popcll(__ballot(v != 0)) < j) return 0;
  if (vmax == vmin) return vmax;   // every value is vmax
  const int top = 31 - __builtin_clz(vmax ^ vmin);
  uint32_t x = top == 31 ? 0u : vmax & ~((2u << top) - 1u);
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    if (top - b < 0) break;
    const uint32_t c = x | (1u << (top - b));
    if (__popcll(__ballot(v >= c)) >= j) x = c;
  }
  return x;
}

// Rows of at most 64*NW*VPL keys: one workgroup of NW waves per row.  Thread t
// holds the VPL consecutive keys from t*VPL as order-preserving uint32
// (16-byte loads where the row allows), loaded without branches so that
// every load is in flight at once.  The bits shared by the
// row's largest and smallest key are skipped; the rest are resolved 8 bits
// at a time with per-wave 256-bin histograms that wave 0 sums, scans with
// DPP and clears again for the next digit (two barriers per digit).
// Output positions follow index order, which is thread order: the keys taken
// before thread t's are the keys > theta of threads before it plus min(kr,
// keys == theta of threads before it), one workgroup scan of per-thread
// counts, and each thread writes its own taken keys in turn.
// A row is one workgroup and so runs on few waves: the code keeps the wave
// index scalar and avoids per-slot branches, since every dependent
// instruction's latency is exposed.
// FINITE: keys equal to -inf are not selectable; a row with fewer than k
// other keys selects them all and pads its output with -1.
//
// floor: keys whose order-preserving value is below it are not selectable
// either (0: none excluded), and kk counts only the others.  lane_max_out,
// when given, receives the largest selectable key of this thread (0: none).
//
// select_row runs the selection for one row inside a workgroup of NW waves
// (64*NW threads): it writes the positions of the kk selected keys,
// ascending, to sel (LDS, 64*NW*VPL entries) and returns kk (k, or with
// FINITE or a floor possibly fewer).  Every thread of the workgroup must
// call it; it ends with a barrier.
//
// Rows of at most 64*NW keys (when lane_max_out is not asked for) take
// select_small instead: one key per thread, each selectable key's rank (the
// keys above it plus the equal keys at lower positions) counted against
// every key of the row in LDS, read back by broadcast 16-byte loads; a key is
// taken when its rank is under kk, which is exactly the lowest-position tie
// rule, and positions follow from one scan of the taken flags.  Three
// barriers instead of a radix pass's two per 8 bits.  A key that is not
// selectable is kept as 0, under every selectable key (only a -NaN maps to
// 0, and NaN is outside the contract).
template <bool FINITE, int NW>
__device__ __forceinline__ int select_small(const float* __restrict__ vals, int n, int k, int32_t* sel,
                                            uint32_t floor) {
  constexpr int NT = 64 * NW;
  __shared__ __attribute__((aligned(16))) uint32_t keys[NT];
  __shared__ int small_cnt[NW][2];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t u = f32_sortable(vals[min(tid, n - 1)]);
  const bool ok = tid < n && (!FINITE || u != kNegInfKey) && u >= floor && u != 0u;
  const uint32_t key = ok ? u : 0u;
  keys[tid] = key;
  const int nw_ok = static_cast<int>(__popcll(__ballot(ok)));
  if (lane == 0) small_cnt[wave][0] = nw_ok;
  __syncthreads();
  int nval = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) nval += small_cnt[w][0];
  const int kk = min(k, nval);
  int rank = 0;   // keys above this one, then equal keys at lower positions
  const int nr = (n + 3) & ~3;   // (keys at or past n are 0)
#pragma unroll 4
  for (int i = 0; i < nr; i += 4) {
    const uint4 c = *reinterpret_cast<const uint4*>(keys + i);
    rank += (c.x > key || (c.x == key && i < tid)) ? 1 : 0;
    rank += (c.y > key || (c.y == key && i + 1 < tid)) ? 1 : 0;
    rank += (c.z > key || (c.z == key && i + 2 < tid)) ? 1 : 0;
    rank += (c.w > key || (c.w == key && i + 3 < tid)) ? 1 : 0;
  }
  const bool take = ok && rank < kk;
  const uint64_t tb = __ballot(take);
  if (lane == 0) small_cnt[wave][1] = static_cast<int>(__popcll(tb));
  __syncthreads();
  int pos = static_cast<int>(__popcll(tb & ((1ull << lane) - 1ull)));
#pragma unroll
  for (int w = 0; w < NW - 1; ++w) pos += w < wave ? small_cnt[w][1] : 0;
  if (take) sel[pos] = tid;
  __syncthreads();
  return kk;
}

template <int VPL, bool FINITE, int NW = 4>
__device__ __forceinline__ int select_row(const float* __restrict__ vals, int n, int k, int32_t* sel, uint32_t floor = 0,
                          uint32_t* lane_max_out = nullptr) {
  static_assert(VPL <= 32, "one mask bit per key of a thread");
  static_assert(NW >= 4 && NW <= 16, "4 to 16 waves");
  constexpr int NT = 64 * NW;
  if (n <= NT && !lane_max_out) return select_small<FINITE, NW>(vals, n, k, sel, floor);   // uniform
  __shared__ __attribute__((aligned(16))) int hist[NW][260];   // one copy per wave, padded across banks
  __shared__ int wave_cnt[NW][2];
  __shared__ uint32_t red[NW][4];
  __shared__ int sh_bin, sh_kr, sh_whole;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  uint32_t u[VPL];
  bool valid[VPL];
  const int first = tid * VPL;
  if (VPL % 4 == 0 && n == NT * VPL && (reinterpret_cast<uintptr_t>(vals) & 15) == 0) {   // uniform
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
    valid[i] = first + i < n && (!FINITE || u[i] != kNegInfKey) && u[i] >= floor;
  }
  if (tid < 256) {
#pragma unroll
    for (int w = 0; w < NW; ++w) hist[w][tid] = 0;
  }
  uint32_t umax = 0, umin = 0xFFFFFFFFu;
  int nval = 0;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    umax = max(umax, valid[i] ? u[i] : 0u);
    umin = min(umin, valid[i] ? u[i] : 0xFFFFFFFFu);
    nval += __popcll(__ballot(valid[i]));
  }
  const uint32_t lane_max = umax;   // 0 when the lane holds no valid key
  if (lane_max_out) *lane_max_out = lane_max;
  umax = wave_minmax_u32<true>(umax);
  umin = wave_minmax_u32<false>(umin);
  // A lower bound of the k-th largest key: when j = ceil(k/NW) lanes of every
  // wave hold a key >= x_w, at least k keys are >= min_w x_w.  Keys under the
  // bound cannot be selected and stay out of the histograms.
  const uint32_t lbound = wave_lower_bound(lane_max, (k + NW - 1) / NW, umax, umin);
  if (lane == 0) {
    red[wave][0] = umax;
    red[wave][1] = umin;
    red[wave][2] = nval;
    red[wave][3] = lbound;
  }
  __syncthreads();
  uint32_t lb_min = red[0][3];
  umax = red[0][0];
  umin = red[0][1];
  nval = red[0][2];
#pragma unroll
  for (int w = 1; w < NW; ++w) {
    umax = max(umax, red[w][0]);
    umin = min(umin, red[w][1]);
    nval += red[w][2];
    lb_min = min(lb_min, red[w][3]);
  }
  const int kk = min(k, nval);   // keys selected; k unless FINITE drops some
  const uint32_t lo = max(umin, lb_min);

  // Radix select over the bits below the common prefix of umax and lo.
  int kr = kk;
  uint32_t prefix = umax, mask = 0xFFFFFFFFu;
  int remaining = (umax == lo || kk == 0) ? 0 : 32 - __builtin_clz(umax ^ lo);
  if (remaining) {
    mask = remaining == 32 ? 0u : ~((1u << remaining) - 1u);
    prefix = umax & mask;
  }
  if (kk == nval) {   // every valid key is taken: no select needed
    prefix = umin;
    kr = 0x7FFFFFFF;
    remaining = 0;
  }
  while (remaining > 0) {   // uniform across the workgroup
    const int shift = remaining > 8 ? remaining - 8 : 0;
    const uint32_t dmask = (1u << (remaining - shift)) - 1u;
    // Only keys >= lo on the prefix count: they are few, and sending the
    // rest to a dummy bin would serialize on one LDS address.
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      if (valid[i] && u[i] >= lo && (u[i] & mask) == prefix) atomicAdd(&hist[wave][(u[i] >> shift) & dmask], 1);
    }
    __syncthreads();
    if (wave == 0) {
      // Lane l owns bins 252-4l .. 255-4l, read and cleared as one 16-byte
      // word per histogram; the exclusive scan of the lane totals (highest
      // bins first) counts the keys in higher bins.  Exactly one bin holds
      // the kr-th key, since kr never exceeds the keys on the prefix.
      const int b0 = 252 - 4 * lane;
      int4 h = *reinterpret_cast<const int4*>(&hist[0][b0]);
#pragma unroll
      for (int w = 1; w < NW; ++w) {
        const int4 x = *reinterpret_cast<const int4*>(&hist[w][b0]);
        h.x += x.x;
        h.y += x.y;
        h.z += x.z;
        h.w += x.w;
      }
#pragma unroll
      for (int w = 0; w < NW; ++w) *reinterpret_cast<int4*>(&hist[w][b0]) = int4{0, 0, 0, 0};
      const int c[4] = {h.w, h.z, h.y, h.x};   // bins 255-4l, 254-4l, 253-4l, 252-4l
      const int tot = c[0] + c[1] + c[2] + c[3];
      int above = wave_incl_scan_dpp(tot) - tot;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        if (above < kr && kr <= above + c[i]) {
          sh_bin = 255 - 4 * lane - i;
          sh_kr = kr - above;
          sh_whole = (kr - above) == c[i];
        }
        above += c[i];
      }
    }
    __syncthreads();
    prefix |= static_cast<uint32_t>(sh_bin) << shift;
    mask |= dmask << shift;
    kr = sh_kr;
    remaining = shift;
    // The boundary bin is taken whole: every key on the new prefix is
    // >= prefix (low bits zero), so theta = prefix with all ties taken
    // selects exactly the same keys.
    if (sh_whole) {
      kr = 0x7FFFFFFF;
      break;
    }
  }
  const uint32_t theta = prefix;

  // Keys > theta and == theta of this thread, then of the threads before
  // it; the thread takes its first min(ce, kr - eq_before) keys equal to theta.
  uint32_t gtm = 0, eqm = 0;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    gtm |= static_cast<uint32_t>(valid[i] && u[i] > theta) << i;
    eqm |= static_cast<uint32_t>(valid[i] && u[i] == theta) << i;
  }
  const int cg = __popc(gtm), ce = __popc(eqm);
  const int ig = wave_incl_scan_dpp(cg), ie = wave_incl_scan_dpp(ce);
  if (lane == 63) {
    wave_cnt[wave][0] = ig;
    wave_cnt[wave][1] = ie;
  }
  __syncthreads();
  int gt_before = ig - cg, eq_before = ie - ce;
#pragma unroll
  for (int w = 0; w < NW - 1; ++w) {
    gt_before += w < wave ? wave_cnt[w][0] : 0;
    eq_before += w < wave ? wave_cnt[w][1] : 0;
  }
  const int eq_take = min(ce, max(kr - eq_before, 0));
  int o = gt_before + min(eq_before, kr), eq_seen = 0;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const bool gt = (gtm >> i) & 1u, eq = (eqm >> i) & 1u;
    const bool take = gt || (eq && eq_seen < eq_take);
    if (take) sel[o] = first + i;
    o += take ? 1 : 0;
    eq_seen += eq ? 1 : 0;
  }
  __syncthreads();
  return kk;
}

// ---------------------------------------------------------------------------
// Rows of up to 1024 * VPL keys in one 1024-thread workgroup (16 waves).
// Wave w owns positions [w*64*VPL, (w+1)*64*VPL); its lane l holds the keys
// at w*64*VPL + 64*i + l (i < VPL) in registers, so every load and every
// mask store is one contiguous 256-byte run per wave, the row is read once,
// and position order is (wave, slot, lane) order.  The radix resolution is
// select_row's, with one histogram per wave.  run() finds theta (the
// smallest taken key) and kr (how many keys equal to theta are taken, the
// lowest positions first); place() then hands every taken position, in
// ascending order, to a callback with its output slot.  Positions at or past
// n are never taken.
// ---------------------------------------------------------------------------
template <int VPL, bool FINITE>
struct WideSelect {
  static constexpr int NW = 16, NT = 64 * NW;
  static_assert(VPL <= 64, "one validity bit per key");
  uint32_t u[VPL];
  uint64_t valid = 0;   // bit i: key i of this thread takes part
  uint32_t theta = 0;
  int kr = 0, kk = 0;
  uint32_t lane_max = 0, lane_min = 0xFFFFFFFFu;   // load_count(): this thread's valid keys

  // LDS of the selection (the caller declares one and passes it in).
  static constexpr int RB = 12, NB = 1 << RB;   // radix digit: 12 bits, 4096 bins
  static constexpr int RECW = 6;                // dwords per slot record (place)
  static_assert(NW * VPL * RECW <= NB, "slot records fit in the histogram's place");
  struct Shared {
    union {
      int hist[2][NB];                // run(): the radix histograms of even and odd passes
      uint32_t rec[NW * VPL * RECW];  // place(): per (wave, slot) prefix counts and lane masks
    };
    int wave_sum[NW];
    int wave_gt[NW], wave_eq[NW];
    uint32_t red[NW][3];
  };

  // Position of key i of this thread.
  __device__ __forceinline__ static int pos(int i) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    return wave * 64 * VPL + 64 * i + lane;
  }

  // A raw buffer of exactly the row's n * 4 bytes: positions past the row
  // read 0 from the range check instead of touching memory.  Keys whose
  // order-preserving value is below floor never take part.
  __device__ __forceinline__ void load(const float* __restrict__ vals, int n, uint32_t floor = 0) {
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(vals), 0, n * 4, 0x00020000);
    const int base = pos(0);
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      u[i] = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rsrc, (base + 64 * i) * 4, 0, 0));
    // key i is inside the row while 64 i < n - base
    const int nv = min(max((n - base + 63) / 64, 0), VPL);
    valid = nv >= 64 ? ~0ull : ((1ull << nv) - 1ull);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      u[i] = f32_sortable(__uint_as_float(u[i]));
      if ((FINITE && u[i] == kNegInfKey) || u[i] < floor) valid &= ~(1ull << i);
    }
  }

  // Key i from a value computed in place (ok = false: never taken).
  __device__ __forceinline__ void set(int i, float v, bool ok) {
    u[i] = f32_sortable(v);
    valid = ok ? (valid | (1ull << i)) : (valid & ~(1ull << i));
  }

  __device__ __forceinline__ bool on(int i) const { return (valid >> i) & 1ull; }

  // Marks the validity bits as changed here, so each phase derives its
  // per-slot lane masks anew instead of keeping VPL scalar-register pairs
  // alive across the whole kernel.
  __device__ __forceinline__ void refresh() { asm volatile("" : "+v"(valid)); }

  // The row's largest and smallest valid key and the count of valid keys,
  // reduced over the workgroup through sh.red (one barrier); LANE: this
  // thread's extremes are lane_max / lane_min already (load_count).
  template <bool LANE = false>
  __device__ __forceinline__ void reduce_row(Shared& sh, uint32_t& umax, uint32_t& umin, int& nval) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    umax = lane_max;
    umin = lane_min;
    if (!LANE) {
      umax = 0;
      umin = 0xFFFFFFFFu;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        if (on(i)) {
          umax = max(umax, u[i]);
          umin = min(umin, u[i]);
        }
      }
    }
    nval = wave_incl_scan_dpp(__popcll(valid));
    umax = wave_minmax_u32<true>(umax);
    umin = wave_minmax_u32<false>(umin);
    if (lane == 63) {
      sh.red[wave][0] = umax;
      sh.red[wave][1] = umin;
      sh.red[wave][2] = nval;
    }
    __syncthreads();
    umax = 0;
    umin = 0xFFFFFFFFu;
    nval = 0;
#pragma unroll 4
    for (int w = 0; w < NW; ++w) {
      umax = max(umax, sh.red[w][0]);
      umin = min(umin, sh.red[w][1]);
      nval += static_cast<int>(sh.red[w][2]);
    }
  }

  // The bin of a complete 4096-bin histogram that holds the kr-th key from
  // the top, the rank kr within it, and whether the bin is taken whole.
  // Every thread reads its 4 bins (clearing other's in the same step, the
  // next pass's histogram) and publishes its wave's sum; after that one
  // barrier every wave finds the boundary itself -- the wave of bins holding
  // the kr-th key, then the bin among its 256 -- instead of waiting for one
  // thread to publish it.
  __device__ __forceinline__ void boundary(Shared& sh, const int* hist, int* other, int& bin, int& krl, int& whole) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // (the other histogram was last read before this pass's atomics)
#pragma unroll
    for (int j = 0; j < NB / NT; ++j) other[tid + NT * j] = 0;
    // Thread t owns bins NB-1-4t .. NB-4-4t (descending), so the keys in
    // higher bins are those of lower threads and of its own earlier bins.
    int tot = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) tot += hist[NB - 1 - 4 * tid - j];
    const int incl = wave_incl_scan_dpp(tot);
    if (lane == 63) sh.wave_sum[wave] = incl;
    __syncthreads();
    const int wsum = lane < NW ? sh.wave_sum[lane] : 0;
    const int wcum = wave_incl_scan_dpp(wsum);
    const int bw = __builtin_ctzll(__ballot(lane < NW && wcum >= kr));   // the boundary's wave of bins
    const int t2 = bw * 64 + lane;
    int c[4], tot2 = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      c[j] = hist[NB - 1 - 4 * t2 - j];
      tot2 += c[j];
    }
    int above = __builtin_amdgcn_readlane(wcum - wsum, bw) + wave_incl_scan_dpp(tot2) - tot2;
    const int bl = __builtin_ctzll(__ballot(above < kr && kr <= above + tot2));   // its lane
    bin = 0;
    krl = 0;
    whole = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (above < kr && kr <= above + c[j]) {
        bin = NB - 1 - 4 * t2 - j;
        krl = kr - above;
        whole = krl == c[j];
      }
      above += c[j];
    }
    bin = __builtin_amdgcn_readlane(bin, bl);
    krl = __builtin_amdgcn_readlane(krl, bl);
    whole = __builtin_amdgcn_readlane(whole, bl);
  }

  // Radix passes over the bits below the resolved prefix: one shared
  // histogram of 4096 bins per pass (a 12-bit digit of sign, exponent and
  // top mantissa bits spreads typical scores over enough bins that a wave's
  // atomics rarely collide; an 8-bit digit of such floats holds a handful of
  // exponents and serializes on them), alternating between sh.hist[buf] and
  // the other, two barriers per digit.  Ends with a barrier when it counted.
  __device__ __forceinline__ void passes(Shared& sh, uint32_t prefix, uint32_t mask, int remaining, int buf, uint32_t umin,
                         bool counted) {
    const int lane = threadIdx.x & 63;
    const bool any = counted || remaining > 0;
    while (remaining > 0) {   // uniform across the workgroup
      refresh();
      const int shift = remaining > RB ? remaining - RB : 0;
      const uint32_t dmask = (1u << (remaining - shift)) - 1u;
      int* hist = sh.hist[buf];
      // Keys equal to the row minimum are counted per wave instead: a flood
      // of equal keys (the -inf of unscored positions) would serialize on
      // one LDS address.
      int at_min = 0;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        if (on(i) && (u[i] & mask) == prefix) {
          if (u[i] == umin) ++at_min;
          else atomicAdd(&hist[(u[i] >> shift) & dmask], 1);
        }
      }
      at_min = wave_incl_scan_dpp(at_min);
      if (lane == 63 && at_min) atomicAdd(&hist[(umin >> shift) & dmask], at_min);
      __syncthreads();
      int bin, krl, whole;
      boundary(sh, hist, sh.hist[buf ^ 1], bin, krl, whole);
      prefix |= static_cast<uint32_t>(bin) << shift;
      mask |= dmask << shift;
      kr = krl;
      remaining = shift;
      buf ^= 1;
      if (whole) {   // the boundary bin is taken whole: theta = its lower bound
        kr = 0x7FFFFFFF;
        break;
      }
    }
    if (any) __syncthreads();   // the last histogram reads are done before sh is reused
    theta = prefix;
  }

  // theta and kr for the k largest valid keys; returns kk = min(k, valid keys).
  // Every thread calls it; the caller's earlier uses of sh have completed
  // (a barrier since).  The bits the row's largest and smallest keys share
  // are skipped.
  __device__ __forceinline__ int run(int k, Shared& sh) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < NB / NT; ++j) sh.hist[0][tid + NT * j] = 0;
    uint32_t umax, umin;
    int nval;
    reduce_row(sh, umax, umin, nval);
    kk = min(k, nval);
    kr = kk;
    uint32_t prefix = umax, mask = 0xFFFFFFFFu;
    int remaining = (umax == umin || kk == 0) ? 0 : 32 - __builtin_clz(umax ^ umin);
    if (remaining) {
      mask = remaining == 32 ? 0u : ~((1u << remaining) - 1u);
      prefix = umax & mask;
    }
    if (kk == nval) {   // every valid key is taken
      prefix = umin;
      kr = 0x7FFFFFFF;
      remaining = 0;
    }
    passes(sh, prefix, mask, remaining, 0, umin, false);
    return kk;
  }

  // load() with run()'s first digit counted on the way: every load is
  // issued first, then each key's top 12 bits go into sh.hist[0] as the key
  // arrives, so the LDS atomics overlap the row's transfer instead of
  // following it.  run_counted() then resolves that digit and continues
  // with run()'s passes.  -inf keys (a flood of unscored positions) are
  // counted by ballot.  Every thread calls both; the caller's earlier uses
  // of sh have completed (a barrier since).
  __device__ __forceinline__ void load_count(const float* __restrict__ vals, int n, Shared& sh) {
    const int tid = threadIdx.x;
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(vals), 0, n * 4, 0x00020000);
    const int base = pos(0);
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      u[i] = static_cast<uint32_t>(__builtin_amdgcn_raw_buffer_load_b32(rsrc, (base + 64 * i) * 4, 0, 0));
#pragma unroll
    for (int j = 0; j < NB / NT; ++j) sh.hist[0][tid + NT * j] = 0;
    const int nv = min(max((n - base + 63) / 64, 0), VPL);
    valid = nv >= 64 ? ~0ull : ((1ull << nv) - 1ull);
    __syncthreads();   // the histogram is clear (the loads are in flight meanwhile)
    int ninf = 0;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      u[i] = f32_sortable(__uint_as_float(u[i]));
      if (FINITE && u[i] == kNegInfKey) valid &= ~(1ull << i);
      count(i, sh, ninf);
    }
    count_done(sh, ninf);
  }

  // The counting of load_count() for keys given one by one with set(): the
  // caller clears sh.hist[0] before a barrier, then calls count(i) after
  // each set(i) (so the atomics follow the keys' loads as they arrive) and
  // count_done() once; run_counted() follows.
  __device__ __forceinline__ void count(int i, Shared& sh, int& ninf) {
    if (on(i)) {
      lane_max = max(lane_max, u[i]);
      lane_min = min(lane_min, u[i]);
      if (u[i] == kNegInfKey) ++ninf;
      else atomicAdd(&sh.hist[0][u[i] >> (32 - RB)], 1);
    }
  }
  __device__ __forceinline__ void count_done(Shared& sh, int ninf) {
    ninf = wave_incl_scan_dpp(ninf);
    if ((threadIdx.x & 63) == 63 && ninf) atomicAdd(&sh.hist[0][kNegInfKey >> (32 - RB)], ninf);
  }

  __device__ __forceinline__ int run_counted(int k, Shared& sh) {
    uint32_t umax, umin;
    int nval;
    reduce_row<true>(sh, umax, umin, nval);   // (its barrier also completes load_count's atomics)
    kk = min(k, nval);
    kr = kk;
    if (kk == nval) {   // every valid key is taken
      kr = 0x7FFFFFFF;
      passes(sh, umin, 0xFFFFFFFFu, 0, 0, umin, true);
      return kk;
    }
    int bin, krl, whole;
    boundary(sh, sh.hist[0], sh.hist[1], bin, krl, whole);
    kr = krl;
    const uint32_t prefix = static_cast<uint32_t>(bin) << (32 - RB);
    if (whole) {
      kr = 0x7FFFFFFF;
      passes(sh, prefix, 0xFFFFFFFFu, 0, 1, umin, true);
    } else {
      passes(sh, prefix, ~((1u << (32 - RB)) - 1u), 32 - RB, 1, umin, true);
    }
    return kk;
  }

  // place() for few keys per thread: one uniform pass over the slots with a
  // ballot per slot instead of each thread walking its own candidates
  // through LDS records (the walk is a chain of dependent LDS reads per
  // candidate; a slot's taken keys here cost two ballots and two bit
  // counts).  The same output indices.  Ends with a barrier.
  template <typename Emit>
  __device__ __forceinline__ void place_uniform(Shared& sh, Emit&& emit) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    refresh();
    uint64_t bg[VPL], be[VPL];
    int cg = 0, ce = 0;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      bg[i] = __ballot(on(i) && u[i] > theta);
      be[i] = __ballot(on(i) && u[i] == theta);
      cg += __popcll(bg[i]);
      ce += __popcll(be[i]);
    }
    if (lane == 0) {
      sh.wave_gt[wave] = cg;
      sh.wave_eq[wave] = ce;
    }
    __syncthreads();
    int g = 0, e = 0;   // keys of the earlier waves
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      g += w < wave ? sh.wave_gt[w] : 0;
      e += w < wave ? sh.wave_eq[w] : 0;
    }
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const int gl = g + static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bg[i] >> 32),
                                                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bg[i]), 0)));
      const int el = e + static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(be[i] >> 32),
                                                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(be[i]), 0)));
      const bool gt = (bg[i] >> lane) & 1ull, eq = (be[i] >> lane) & 1ull;
      if (gt || (eq && el < kr)) emit(pos(i), gl + min(el, kr), i);
      g += __popcll(bg[i]);
      e += __popcll(be[i]);
    }
    __syncthreads();
  }

  // Calls emit(position, output index, slot) for every taken key, output
  // indices 0..kk-1 in ascending position order: a taken key's index is the
  // number of keys above theta before it plus min(keys equal to theta before
  // it, kr).  Lane i of each wave first gathers slot i's lane masks and
  // within-wave prefix counts into an LDS record; then every thread visits
  // only its own taken keys (a few), instead of the wave stepping through
  // all VPL slots.  Ends with a barrier.
  template <typename Emit>
  __device__ __forceinline__ void place(Shared& sh, Emit&& emit) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t below = (1ull << lane) - 1ull;
    refresh();
    uint64_t gtm = 0, eqm = 0;   // bit i: key i above / equal to theta
    uint32_t g_lo = 0, g_hi = 0, e_lo = 0, e_hi = 0;   // lane i: slot i's lane masks
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const bool gt = on(i) && u[i] > theta, eq = on(i) && u[i] == theta;
      gtm |= static_cast<uint64_t>(gt) << i;
      eqm |= static_cast<uint64_t>(eq) << i;
      const uint64_t bg = __ballot(gt), be = __ballot(eq);
      g_lo = lane == i ? static_cast<uint32_t>(bg) : g_lo;
      g_hi = lane == i ? static_cast<uint32_t>(bg >> 32) : g_hi;
      e_lo = lane == i ? static_cast<uint32_t>(be) : e_lo;
      e_hi = lane == i ? static_cast<uint32_t>(be >> 32) : e_hi;
    }
    asm volatile("" : "+v"(gtm), "+v"(eqm));
    const int cg = __popc(g_lo) + __popc(g_hi), ce = __popc(e_lo) + __popc(e_hi);   // 0 past VPL
    const int ig = wave_incl_scan_dpp(cg), ie = wave_incl_scan_dpp(ce);
    if (lane < VPL) {
      uint32_t* rp = sh.rec + (wave * VPL + lane) * RECW;
      *reinterpret_cast<uint2*>(rp) = make_uint2(static_cast<uint32_t>(ig - cg), static_cast<uint32_t>(ie - ce));
      *reinterpret_cast<uint2*>(rp + 2) = make_uint2(g_lo, g_hi);
      *reinterpret_cast<uint2*>(rp + 4) = make_uint2(e_lo, e_hi);
    }
    if (lane == 63) {
      sh.wave_gt[wave] = ig;
      sh.wave_eq[wave] = ie;
    }
    __syncthreads();
    int g = 0, e = 0;   // keys of the earlier waves
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      g += w < wave ? sh.wave_gt[w] : 0;
      e += w < wave ? sh.wave_eq[w] : 0;
    }
    uint64_t cand = gtm | eqm;
    while (cand) {   // a thread's candidates in slot (position) order
      const int i = __builtin_ctzll(cand);
      cand &= cand - 1;
      const uint32_t* rp = sh.rec + (wave * VPL + i) * RECW;
      const uint2 pc = *reinterpret_cast<const uint2*>(rp);
      const uint2 mg = *reinterpret_cast<const uint2*>(rp + 2);
      const uint2 me = *reinterpret_cast<const uint2*>(rp + 4);
      const uint64_t bgt = (static_cast<uint64_t>(mg.y) << 32) | mg.x;
      const uint64_t beq = (static_cast<uint64_t>(me.y) << 32) | me.x;
      const int el = e + static_cast<int>(pc.y) + __popcll(beq & below);
      if (!((gtm >> i) & 1ull) && el >= kr) {   // equal keys after it are not taken either
        cand &= gtm;
        continue;
      }
      const int gl = g + static_cast<int>(pc.x) + __popcll(bgt & below);
      emit(pos(i), gl + min(el, kr), i);
    }
    __syncthreads();
  }
};

}  // namespace
}  // namespace qkv
