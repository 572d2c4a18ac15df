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
#include "common.h"
#include "select.h"

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
// is bound by instruction issue, not latency.  Same contract as select_row.
template <int VPL, bool FINITE>
__global__ __launch_bounds__(256) void topk_wave_kernel(const float* __restrict__ values, int64_t rows, int n,
                                                        int64_t ld, int k, int32_t* __restrict__ out) {
  __shared__ int hist[4][256];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  if (row >= rows) return;   // wave-uniform
  const float* vals = values + row * ld;
  int* wh = hist[wave];

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
  umax = wave_minmax_u32<true>(umax);
  umin = wave_minmax_u32<false>(umin);
  const int kk = min(k, nval);

  int kr = kk;
  uint32_t prefix = umax, mask = 0xFFFFFFFFu;
  int remaining = (umax == umin || kk == 0) ? 0 : 32 - __builtin_clz(umax ^ umin);
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
      if (valid[i] && (u[i] & mask) == prefix) atomicAdd(&wh[(u[i] >> shift) & dmask], 1);
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

  int32_t* orow = out + row * k;
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
constexpr int kStageChunk = 4096;
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

// Candidates left after a stage over n keys: k from every full chunk, and
// min(k, rest) from the last.
int64_t stage_out(int64_t n, int64_t k) {
  const int64_t c = cdiv(n, kStageChunk);
  return (c - 1) * k + std::min<int64_t>(k, n - (c - 1) * kStageChunk);
}

bool staged(int64_t n, int64_t k) { return n > kStageChunk && k <= kStageMaxK; }

template <bool FINITE>
int launch_rows(const float* values, int64_t rows, int64_t n, int64_t ld, int64_t k, int32_t* out,
                hipStream_t st) {
  const int nn = static_cast<int>(n), kk = static_cast<int>(k);
  // One wave per row pays off when rows are many and short (measured: 65536
  // rows of 1024 keys 181 -> 110 us; 64 rows of 2048 keys 6.7 -> 11.3 us).
  if (n <= 64 * kWaveMaxVPL && rows >= kWaveMinRows) {
    const unsigned wg4 = static_cast<unsigned>(cdiv(rows, 4));
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
  // two candidate buffers (value + index) sized for the first stage's output,
  // then the first stage's chunk bounds
  return 2 * rows * stage_out(n, k) * static_cast<int64_t>(sizeof(float) + sizeof(int32_t)) +
         rows * cdiv(n, kStageChunk) * static_cast<int64_t>(sizeof(uint32_t));
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
