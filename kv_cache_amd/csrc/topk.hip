// Row-wise top-k with the lowest-index tie-break, one workgroup per row.
//
// The reference calls torch.topk over partial scores or block maxima
// (evaluate_qwen3_top2_head_limit3_ppl.py:4448, 5046), whose tie order is
// unspecified.  Here: keys map to order-preserving uint32; a 3-pass radix
// select (11/11/10-bit digits, LDS histograms) finds the k-th largest key
// theta and how many keys equal to theta are kept; a stable compaction in
// index order then writes every key > theta plus the lowest-index keys equal
// to theta, so the output is already in ascending index order.
#include "common.h"

namespace qkv {
namespace {

constexpr int kBins = 2048;
constexpr int kLdsKeys = 12288;   // rows up to this many keys are staged in LDS (48 KB)

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
  const unsigned grid = static_cast<unsigned>(rows);
  if (n <= 4096) {
    topk_kernel<256, true><<<grid, 256, n * sizeof(uint32_t), st>>>(values, static_cast<int>(n), ld,
                                                                     static_cast<int>(k), out);
  } else if (n <= kLdsKeys) {
    topk_kernel<1024, true><<<grid, 1024, n * sizeof(uint32_t), st>>>(values, static_cast<int>(n), ld,
                                                                       static_cast<int>(k), out);
  } else {
    topk_kernel<1024, false><<<grid, 1024, 0, st>>>(values, static_cast<int>(n), ld,
                                                    static_cast<int>(k), out);
  }
  return check_launch("qkv_topk");
}
