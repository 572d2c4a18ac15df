// Chunk windows of the long-row top-k (qkv_topk_ws's histogram-and-filter
// path), shared by the top-k kernels and the decode scoring launch that can
// produce them while it scores.
//
// A row is cut into chunks of kStageChunk keys.  A chunk's window, from the
// 4096-bin histogram of its keys' top kHistBits order-preserving bits:
//   w[0]            t_c, the bin at which the chunk's count from the top
//                   reaches min(k, chunk length);
//   w[1]            the chunk's keys in bins >= t_c + kWin;
//   w[2 .. 2+kWin)  the counts of bins t_c .. t_c + kWin - 1 (0 past 4095).
// The row's floor is worked out from every chunk's window (topk.hip).
#pragma once

#include "common.h"
#include "select.h"

namespace qkv {
namespace {

constexpr int kStageChunk = 4096;
constexpr int kHistBits = 12, kHistBins = 1 << kHistBits;
constexpr int kWin = 64;               // window bins per chunk
constexpr int kWinWords = kWin + 2;    // t_c, the count above the window, the window

// The window of a chunk whose histogram is complete in LDS (h, kHistBins
// counts) into w, computed by a workgroup of NT threads (thread t holds bins
// [4096 - BPT(t+1), 4096 - BPT t)).  wsum: NT / 64 ints of LDS; t_sh: an LDS
// int the caller set to 0 before a barrier.  COH: device-coherent stores
// (for a reader in the same launch).  Every thread calls it; it starts and
// ends with the workgroup in step (no barrier needed after the histogram's
// last atomics beyond the caller's).
template <int NT, bool COH>
__device__ void chunk_window(const uint32_t* h, int target, int32_t* __restrict__ w, int* wsum, int* t_sh) {
  constexpr int BPT = kHistBins / NT, NW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b0 = kHistBins - BPT * (tid + 1);
  int hb[BPT], cnt = 0;
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    hb[i] = static_cast<int>(h[b0 + i]);
    cnt += hb[i];
  }
  const int incl = wave_incl_scan_dpp(cnt);
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int above = incl - cnt;
#pragma unroll
  for (int v = 0; v < NW; ++v) above += v < wave ? wsum[v] : 0;
  if (above < target && above + cnt >= target) {   // one thread
    int t = b0;
#pragma unroll
    for (int i = BPT - 1; i >= 0; --i) {
      if (above < target && above + hb[i] >= target) t = b0 + i;
      above += hb[i];
    }
    *t_sh = t;
  }
  __syncthreads();
  const int t = *t_sh;
  if (tid < kWin) {
    const int32_t c = t + tid < kHistBins ? static_cast<int32_t>(h[t + tid]) : 0;
    if (COH) st_coherent(w + 2 + tid, c);
    else w[2 + tid] = c;
  }
  int over = 0;   // keys above the window: this thread's bins from t + kWin up
#pragma unroll
  for (int i = 0; i < BPT; ++i) over += b0 + i >= t + kWin ? hb[i] : 0;
  over = wave_incl_scan_dpp(over);
  __syncthreads();   // (wsum is reused)
  if (lane == 63) wsum[wave] = over;
  __syncthreads();
  if (tid == 0) {
    int sum = 0;
#pragma unroll
    for (int v = 0; v < NW; ++v) sum += wsum[v];
    if (COH) {
      st_coherent(w, t);
      st_coherent(w + 1, sum);
    } else {
      w[0] = t;
      w[1] = sum;
    }
  }
}

}  // namespace
}  // namespace qkv
