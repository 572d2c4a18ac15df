// Candidate reuse and exact rerank: the decode step of the reference's
// qabs{S}cand{pct}reuse[final|2set] modes (EV:3991-4397) and the selector it
// asks of its absent reuse_select kernel (EV:3881-3919), on GQA-shaped K/V.
//
// A row is one (sequence, query head) r = b * Hq + h; it reads K/V head
// h / (Hq / Hkv).  Per step:
//   reuse_partial_kernel    fp32 partial scores over the row's top-|q| dims,
//                           read from the dim-major K copy (one coalesced
//                           stream of S * 2 bytes per token);
//   (top-k) + reuse_mask_kernel   candidates = scores >= the k-th largest;
//   reuse_scores_kernel     union of the current / previous candidate and
//                           previous final masks, compacted per 1024-token
//                           tile in LDS; full-D fp32 scores of the union only;
//   (top-k) + reuse_finalize_kernel  the final selection, its validity, the
//                           final mask with the protected ranges, and the
//                           final index list (EV:2938-2982).
// The fp32 dot products add separately rounded products in dim order
// (built with -ffp-contract=off), as the reference's kernels do (QK:91-94,
// 210-213), so scores, masks and indices match the CPU restatement bit for
// bit.  EV = ymluo/projects/qwen3_top2_head_limit3_ppl/src/
// evaluate_qwen3_top2_head_limit3_ppl.py, QK = .../qabs_cuda_kernels.py.
#include <math.h>

#include <type_traits>

#include "ref_common.h"
#include "select.h"

namespace qkv {
namespace {

constexpr int kRT = 256;          // threads per workgroup
// Measured at 32 rows x 32792 tokens (graph step, us/layer): tiles of 512
// 50.7, 1024 50.8, 2048 51.7, 4096 58.0 (one thread per union token).
#ifndef QKV_SCORE_TILE
#define QKV_SCORE_TILE 1024
#endif
constexpr int kScoreTile = QKV_SCORE_TILE;   // tokens per workgroup in reuse_scores_kernel
constexpr int kScoreNT = kScoreTile / 4;     // its threads (four positions each)
constexpr int kMaskTile = 4096;   // tokens per workgroup in reuse_mask_kernel

// ---------------------------------------------------------------------------
// Partial scores: out[r, t] = sum_s q[d_s] * K[d_s, t] over the row's
// top-|q| dims d_s in selection order (QK:63-96 on the dim-major copy of
// EV:2018-2042; dims chosen as QK:120-145).  Eight tokens per thread.
// HIST: each score's top 12 order-preserving bits (the first radix digit of
// the candidate selection, kCandBins bins) are also counted into
// hist[row * kCandBins + digit], through a workgroup histogram in LDS and
// one global atomic per non-empty bin.
// ---------------------------------------------------------------------------
constexpr int kCandBits = 12, kCandBins = 1 << kCandBits;
// (256, 512 and 1024 threads measured within 0.3 us/layer of each other.)
#ifndef QKV_PARTIAL_NT
#define QKV_PARTIAL_NT 256
#endif
constexpr int kPartNT = QKV_PARTIAL_NT;   // threads per workgroup (8 tokens each)

template <int DT, bool HIST = false>
__global__ __launch_bounds__(kPartNT) void reuse_partial_kernel(
    const typename Elem<DT>::T* __restrict__ query, const typename Elem<DT>::T* __restrict__ kdm,
    int q_heads, int group, int history, int head_dim, int count, int64_t sb, int64_t sh, int64_t sd,
    bool vec, float* __restrict__ out, int64_t out_ld, const uint8_t* __restrict__ gate, int gate_refresh,
    int gate_rows, int* __restrict__ hist = nullptr) {
  using E = typename Elem<DT>::T;
  __shared__ int hist_s[HIST ? kCandBins : 1];
  if constexpr (HIST) {
#pragma unroll
    for (int j = 0; j < kCandBins / kPartNT; ++j) hist_s[threadIdx.x + kPartNT * j] = 0;   // (a barrier follows)
  }
  __shared__ float q_s[512];
  __shared__ __attribute__((aligned(16))) uint64_t key_s[128];
  __shared__ int sel_idx[kMaxDims];
  __shared__ float sel_q[kMaxDims];
  const int row = blockIdx.y, tid = threadIdx.x;
  if (gate) {   // a lagged step: rows that keep no new candidates are skipped (uniform)
    __shared__ int gate_cnt[kPartNT / 64];
    if (!lag_refreshes(gate, gate_refresh, gate_rows, row, gate_cnt)) return;
  }
  const int b = row / q_heads, h = row - b * q_heads;
  const typename Elem<DT>::T* q_row = query + static_cast<int64_t>(row) * head_dim;
  for (int d = tid; d < head_dim; d += kPartNT) q_s[d] = Elem<DT>::load(q_row + d);
  __syncthreads();
  if (head_dim <= 128) {   // uniform
    rank_dims128(q_s, key_s, head_dim, count, sel_idx, sel_q);
  } else {
    for (int s = tid; s < count; s += kPartNT) {   // valid even for a NaN query
      sel_idx[s] = 0;
      sel_q[s] = q_s[0];
    }
    __syncthreads();
    // rank(d) = #{e : |q_e| > |q_d| or (|q_e| == |q_d| and e < d)} (QK:123-145)
    for (int d = tid; d < head_dim; d += kPartNT) {
      const float a = fabsf(q_s[d]);
      int rank = 0;
      for (int e = 0; e < head_dim; ++e) {
        const float c = fabsf(q_s[e]);
        rank += (c > a) || (c == a && e < d);
      }
      if (rank < count) {
        sel_idx[rank] = d;
        sel_q[rank] = q_s[d];
      }
    }
    __syncthreads();
  }
  const int t0 = (blockIdx.x * kPartNT + tid) * 8;
  if (!HIST && t0 >= history) return;
  const int nt = max(min(8, history - t0), 0);   // this thread's tokens
  const E* base = kdm + b * sb + (h / group) * sh + min(t0, history - 1);
  float* o = out + static_cast<int64_t>(row) * out_ld + t0;
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  if (nt == 0) {
    // (HIST: a thread past the row still takes part in the barriers below)
  } else if (vec && nt == 8) {
    // eight dims' loads in flight at once (clamped, in bounds), then the
    // products added in selection order
    for (int s0 = 0; s0 < count; s0 += 8) {
      float v[8][8];
#pragma unroll
      for (int j = 0; j < 8; ++j) load8<DT>(base + sel_idx[min(s0 + j, count - 1)] * sd, v[j]);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (s0 + j < count) {
          const float qs = sel_q[s0 + j];
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[i] = acc[i] + qs * v[j][i];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = acc[i];
  } else {
    // the row's last n < 8 tokens (or an unaligned copy): the same order,
    // every load in flight at once at clamped in-row addresses, then only
    // the n tokens stored (a load-then-add loop over runtime n waits for
    // each load in turn)
    const int n = min(8, history - t0);
    for (int s0 = 0; s0 < count; s0 += 8) {
      float v[8][8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const E* p = base + sel_idx[min(s0 + j, count - 1)] * sd;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[j][i] = Elem<DT>::load(p + min(i, n - 1));
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (s0 + j < count) {
          const float qs = sel_q[s0 + j];
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[i] = acc[i] + qs * v[j][i];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (i < n) o[i] = acc[i];
  }
  if constexpr (HIST) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (i < nt) atomicAdd(&hist_s[f32_sortable(acc[i]) >> (32 - kCandBits)], 1);
    __syncthreads();
    int* hrow = hist + static_cast<int64_t>(row) * kCandBins;
#pragma unroll
    for (int j = 0; j < kCandBins / kPartNT; ++j) {
      const int c = hist_s[tid + kPartNT * j];
      if (c) __hip_atomic_fetch_add(hrow + tid + kPartNT * j, c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---------------------------------------------------------------------------
// Candidate mask: mask[r, t] = values[r, t] >= the smallest of the row's k
// selected values, i.e. the k-th largest (EV:3988-3989; ties at the
// threshold are all kept).  Sixteen tokens per thread.
// ---------------------------------------------------------------------------
// The threshold is the smallest of the k values at sel's indices, or, with
// sel null, thr_in[row] (a given threshold, EV:3967-3971).  thr_out
// (optional) receives it.
__global__ __launch_bounds__(kRT) void reuse_mask_kernel(const float* __restrict__ values, int64_t ld, int n,
                                                         const int32_t* __restrict__ sel, int k,
                                                         const float* __restrict__ thr_in,
                                                         uint8_t* __restrict__ mask, int64_t mask_ld,
                                                         bool vec, float* __restrict__ thr_out) {
  __shared__ float red[kRT / 64];
  const int row = blockIdx.y, tid = threadIdx.x;
  const float* vrow = values + static_cast<int64_t>(row) * ld;
  float thr;
  if (sel) {
    const int32_t* srow = sel + static_cast<int64_t>(row) * k;
    thr = __builtin_huge_valf();
    for (int i = tid; i < k; i += kRT) thr = fminf(thr, vrow[srow[i]]);
    for (int off = 32; off > 0; off >>= 1) thr = fminf(thr, __shfl_xor(thr, off));
    if ((tid & 63) == 0) red[tid >> 6] = thr;
    __syncthreads();
    thr = fminf(fminf(red[0], red[1]), fminf(red[2], red[3]));
  } else {
    thr = thr_in[row];
  }
  if (thr_out && blockIdx.x == 0 && tid == 0) thr_out[row] = thr;
  uint8_t* mrow = mask + static_cast<int64_t>(row) * mask_ld;
  const int t0 = blockIdx.x * kMaskTile + tid * 16;
  if (t0 >= n) return;
  if (vec && t0 + 16 <= n) {
    const float4* v4 = reinterpret_cast<const float4*>(vrow + t0);
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 x = v4[i];
      w[i] = static_cast<uint32_t>(x.x >= thr) | static_cast<uint32_t>(x.y >= thr) << 8 |
             static_cast<uint32_t>(x.z >= thr) << 16 | static_cast<uint32_t>(x.w >= thr) << 24;
    }
    *reinterpret_cast<uint4*>(mrow + t0) = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    for (int t = t0; t < min(n, t0 + 16); ++t) mrow[t] = vrow[t] >= thr;
  }
}

// reuse_mask_kernel's mask as a bitset (64 positions per word): each wave
// writes the ballots of its 64-position words, NW words per wave.
__global__ __launch_bounds__(kRT) void reuse_mask_bits_kernel(const float* __restrict__ values, int64_t ld, int n,
                                                              const int32_t* __restrict__ sel, int k,
                                                              const float* __restrict__ thr_in,
                                                              uint64_t* __restrict__ bits, int64_t bits_ld,
                                                              float* __restrict__ thr_out) {
  constexpr int NW = 4;   // words per wave
  __shared__ float red[kRT / 64];
  const int row = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const float* vrow = values + static_cast<int64_t>(row) * ld;
  float thr;
  if (sel) {
    const int32_t* srow = sel + static_cast<int64_t>(row) * k;
    thr = __builtin_huge_valf();
    for (int i = tid; i < k; i += kRT) thr = fminf(thr, vrow[srow[i]]);
    for (int off = 32; off > 0; off >>= 1) thr = fminf(thr, __shfl_xor(thr, off));
    if (lane == 0) red[wave] = thr;
    __syncthreads();
    thr = fminf(fminf(red[0], red[1]), fminf(red[2], red[3]));
  } else {
    thr = thr_in[row];
  }
  if (thr_out && blockIdx.x == 0 && tid == 0) thr_out[row] = thr;
  uint64_t* brow = bits + static_cast<int64_t>(row) * bits_ld;
  const int w0 = (blockIdx.x * (kRT / 64) + wave) * NW;
  float v[NW];
#pragma unroll
  for (int j = 0; j < NW; ++j) {
    const int t = (w0 + j) * 64 + lane;
    v[j] = t < n ? vrow[t] : -__builtin_huge_valf();
  }
#pragma unroll
  for (int j = 0; j < NW; ++j) {
    const int t = (w0 + j) * 64 + lane;
    const uint64_t m = __ballot(t < n && v[j] >= thr);
    if (lane == 0 && (w0 + j) * 64 < n) brow[w0 + j] = m;
  }
}

// The sample_quantile candidate mask (EV:3972-3987) of rows with at most kRT
// sampled columns, in one launch: every workgroup of a row gathers the row's
// samples (one per thread, its own tile's values already in flight), counts
// for each sample the samples above it and at or above it in LDS (the k-th
// largest value, which torch.topk(...).values[-1] returns, is the one with
// fewer than k above and at least k at or above), and compares its tile
// with it.  The row's first workgroup writes the threshold.  Columns
// lie in [0, n) (the caller's contract).
__global__ __launch_bounds__(kRT) void sample_mask_kernel(const float* __restrict__ values, int64_t ld, int n,
                                                          const int32_t* __restrict__ cols, int n_sample, int k,
                                                          uint8_t* __restrict__ mask, int64_t mask_ld, bool vec,
                                                          float* __restrict__ thr_out) {
  __shared__ __attribute__((aligned(16))) uint32_t keys[kRT];
  __shared__ float thr_s;
  const int row = blockIdx.y, tid = threadIdx.x;
  const float* vrow = values + static_cast<int64_t>(row) * ld;
  const int t0 = blockIdx.x * kMaskTile + tid * 16;
  const bool full = vec && t0 + 16 <= n;
  float4 x[4];
  if (full) {
    const float4* v4 = reinterpret_cast<const float4*>(vrow + t0);
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = v4[i];
  }
  const bool sampled = tid < n_sample;
  const float sv = vrow[sampled ? cols[tid] : 0];
  keys[tid] = sampled ? f32_sortable(sv) : 0u;   // below every finite key
  __syncthreads();
  if (sampled) {   // own is the k-th largest when fewer than k samples lie above it and k at or above
    const uint32_t own = keys[tid];
    int gt = 0, ge = 0;
#pragma unroll 8
    for (int j = 0; j < kRT; j += 4) {
      const uint4 c = *reinterpret_cast<const uint4*>(keys + j);
      gt += (c.x > own) + (c.y > own) + (c.z > own) + (c.w > own);
      ge += (c.x >= own) + (c.y >= own) + (c.z >= own) + (c.w >= own);
    }
    if (gt < k && ge >= k) thr_s = sv;   // equal keys hold equal values (signed zeros compare equal)
  }
  __syncthreads();
  const float thr = thr_s;
  if (thr_out && blockIdx.x == 0 && tid == 0) thr_out[row] = thr;
  if (t0 >= n || !mask) return;   // (mask null: the threshold only)
  uint8_t* mrow = mask + static_cast<int64_t>(row) * mask_ld;
  if (full) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = static_cast<uint32_t>(x[i].x >= thr) | static_cast<uint32_t>(x[i].y >= thr) << 8 |
             static_cast<uint32_t>(x[i].z >= thr) << 16 | static_cast<uint32_t>(x[i].w >= thr) << 24;
    *reinterpret_cast<uint4*>(mrow + t0) = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
    for (int t = t0; t < min(n, t0 + 16); ++t) mrow[t] = vrow[t] >= thr;
  }
}

// ---------------------------------------------------------------------------
// Union scores: out[r, t] = scaling * sum_d q[d] * K[t, d] (d ascending)
// where current | previous | previous_final is set at t, else -inf
// (QK:160-216 without sink/recent protection, as EV:4257-4267 calls it).
// The tile's union tokens are compacted in LDS so that every lane scores one.
// DFIX = 128 fixes the head size so that a token's 16 row loads issue at once;
// registers are held to five waves per SIMD so that a row's 33 workgroups
// times 32 rows are resident together (at three, a second batch waited).
// BITS: the three masks are bitsets (64 positions per uint64 word, mask_ld
// in words) instead of byte masks.
// ---------------------------------------------------------------------------
template <int DT, int DFIX, bool BITS>
__global__ __launch_bounds__(kScoreNT) __attribute__((amdgpu_waves_per_eu(5))) void reuse_scores_kernel(
    const typename Elem<DT>::T* __restrict__ query, const typename Elem<DT>::T* __restrict__ key,
    int q_heads, int group, int history, int head_dim, int64_t sb, int64_t sh, int64_t st, bool kvec,
    const uint8_t* __restrict__ cur, const uint8_t* __restrict__ prev, const uint8_t* __restrict__ fin,
    int64_t mask_ld, bool mvec, float scaling, float* __restrict__ out, int64_t out_ld,
    float* __restrict__ cscore, int32_t* __restrict__ ctok, int32_t* __restrict__ ccnt, int64_t c_ld) {
  using E = typename Elem<DT>::T;
  __shared__ __attribute__((aligned(16))) float q_s[512];
  __shared__ uint16_t list[kScoreTile];
  __shared__ int wave_tot[kScoreNT / 64];
  __shared__ int n_finite;
  const int row = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = row / q_heads, h = row - b * q_heads;
  // the query's first kScoreNT values and this thread's mask words are all in
  // flight before any is used (a load stored to LDS at once, or a load under
  // a branch, would wait for each in turn)
  const E* q_row = query + static_cast<int64_t>(row) * head_dim;
  const float q0 = Elem<DT>::load(q_row + min(tid, head_dim - 1));

  const int tile0 = blockIdx.x * kScoreTile;
  const int t0 = tile0 + tid * 4;
  const int64_t moff = static_cast<int64_t>(row) * mask_ld + t0;
  uint32_t bits = 0;
  if (BITS) {   // positions t0..t0+3 lie in one word; bits past the history are clear
    const int64_t w = static_cast<int64_t>(row) * mask_ld + (min(t0, history - 1) >> 6);
    const uint64_t* c64 = reinterpret_cast<const uint64_t*>(cur);
    const uint64_t a = c64[w];
    const uint64_t p = reinterpret_cast<const uint64_t*>(prev ? prev : cur)[w];
    const uint64_t f = reinterpret_cast<const uint64_t*>(fin ? fin : cur)[w];
    if (t0 < history) {
      const uint64_t u = a | (prev ? p : 0ull) | (fin ? f : 0ull);
      const int n = min(4, history - t0);
      bits = static_cast<uint32_t>(u >> (t0 & 63)) & ((1u << n) - 1u);
    }
  } else if (mvec && t0 + 4 <= history) {
    uint32_t u = *reinterpret_cast<const uint32_t*>(cur + moff);
    if (prev) u |= *reinterpret_cast<const uint32_t*>(prev + moff);
    if (fin) u |= *reinterpret_cast<const uint32_t*>(fin + moff);
#pragma unroll
    for (int i = 0; i < 4; ++i) bits |= static_cast<uint32_t>(((u >> (8 * i)) & 0xFFu) != 0) << i;
  } else if (t0 < history) {
    // the row's last few positions (or unaligned masks): every byte load in
    // flight at once at clamped in-row positions, then the positions past
    // the row dropped (short-circuit loads would wait for one another)
    const int n = min(4, history - t0);
    uint8_t c[4], p[4], f[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t at = moff + min(i, n - 1);
      c[i] = cur[at];
      p[i] = prev ? prev[at] : 0;
      f[i] = fin ? fin[at] : 0;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) bits |= static_cast<uint32_t>(i < n && (c[i] | p[i] | f[i]) != 0) << i;
  }
  if (tid < head_dim) q_s[tid] = q0;
  for (int d = tid + kScoreNT; d < head_dim; d += kScoreNT) q_s[d] = Elem<DT>::load(q_row + d);
  float* orow = out + static_cast<int64_t>(row) * out_ld;
  const float ninf = -__builtin_huge_valf();
  if (bits == 0 && t0 + 4 <= history && ((reinterpret_cast<uintptr_t>(orow + t0) & 15) == 0)) {
    *reinterpret_cast<float4*>(orow + t0) = make_float4(ninf, ninf, ninf, ninf);
  } else {
    for (int i = 0; i < 4 && t0 + i < history; ++i)
      if (!((bits >> i) & 1u)) orow[t0 + i] = ninf;
  }

  // Compaction: the tile's union tokens in index order.
  const int cnt = __popc(bits);
  const int incl = wave_incl_scan_dpp(cnt);
  if (lane == 63) wave_tot[wave] = incl;
  __syncthreads();
  int base = incl - cnt;
  for (int w = 0; w < wave; ++w) base += wave_tot[w];
  for (int i = 0; i < 4; ++i)
    if ((bits >> i) & 1u) list[base++] = static_cast<uint16_t>(tid * 4 + i);
  if (tid == 0) n_finite = 0;
  __syncthreads();
  int total = 0;
#pragma unroll
  for (int w = 0; w < kScoreNT / 64; ++w) total += wave_tot[w];

  // cscore (optional): the tile's union scores again, compacted at the
  // tile's offset, with their tokens and (list length, finite scores) per
  // tile, so that the final selection can rank the union alone
  float* crow = cscore ? cscore + static_cast<int64_t>(row) * c_ld + tile0 : nullptr;
  int32_t* trow = cscore ? ctok + static_cast<int64_t>(row) * c_ld + tile0 : nullptr;
  int n_fin_own = 0;
  const E* kbase = key + b * sb + (h / group) * sh;
  for (int i = tid; i < total; i += kScoreNT) {
    const int t = tile0 + list[i];
    const E* kr = kbase + static_cast<int64_t>(t) * st;
    float acc = 0.0f;
    if (DFIX && kvec) {
      // the row's 16-byte loads first, 16 at a time (the whole row for
      // 16-bit types), kept packed; q comes from LDS four values at a time
      // where it is used (the empty asm keeps those reads from being
      // hoisted next to the loads, which held 128 q values in registers)
      constexpr int EPL = DT == QKV_DTYPE_FP32 ? 4 : 8;   // elements per 16 bytes
      constexpr int NL = DFIX ? DFIX / EPL : 1, NB = NL < 16 ? NL : 16;   // (DFIX = 0 never gets here)
      const float4* q4 = reinterpret_cast<const float4*>(q_s);
#pragma unroll
      for (int c0 = 0; c0 < NL; c0 += NB) {
        uint4 w[NB];
#pragma unroll
        for (int c = 0; c < NB; ++c) w[c] = *reinterpret_cast<const uint4*>(kr + (c0 + c) * EPL);
#pragma unroll
        for (int c = 0; c < NB; ++c) {
          asm volatile("" ::: "memory");
          const uint32_t ww[4] = {w[c].x, w[c].y, w[c].z, w[c].w};
#pragma unroll
          for (int h2 = 0; h2 < EPL / 4; ++h2) {
            const float4 qv = q4[((c0 + c) * EPL) / 4 + h2];
            const float qa[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float kv;
              if constexpr (DT == QKV_DTYPE_FP32) {
                kv = __uint_as_float(ww[e]);
              } else {
                const uint32_t half = (ww[(h2 * 4 + e) >> 1] >> (16 * ((h2 * 4 + e) & 1))) & 0xFFFFu;
                kv = DT == QKV_DTYPE_BF16 ? bf16_to_f32(half) : f16bits_to_f32(half);
              }
              acc = acc + qa[e] * kv;
            }
          }
        }
      }
    } else if (kvec) {
#pragma unroll
      for (int d = 0; d < head_dim; d += 8) {
        float v[8];
        load8<DT>(kr + d, v);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = acc + q_s[d + e] * v[e];
      }
    } else {
      for (int d = 0; d < head_dim; ++d) acc = acc + q_s[d] * Elem<DT>::load(kr + d);
    }
    const float sc = acc * scaling;
    orow[t] = sc;
    if (crow) {
      crow[i] = sc;
      trow[i] = t;
      n_fin_own += isfinite(sc) ? 1 : 0;
    }
  }
  if (crow) {
    if (n_fin_own) atomicAdd(&n_finite, n_fin_own);
    __syncthreads();
    if (tid == 0) {
      int32_t* cn = ccnt + (static_cast<int64_t>(row) * gridDim.x + blockIdx.x) * 2;
      cn[0] = total;
      cn[1] = n_finite;
    }
  }
}

// ---------------------------------------------------------------------------
// Final selection of one row (EV:4270-4307, 4365, 2938-2982): the final
// mask is the protected ranges plus every selected index whose score is
// finite; the index list is the selection (sink and recent entries marked
// invalid), then the sink range, the recent range and the current token.
// attn_ids (optional) repeats the list with -1 for invalid entries.
// ---------------------------------------------------------------------------
// BITS: hf is a bitset (64 positions per uint64 word, hf_ld in words).
template <bool BITS = false>
__global__ __launch_bounds__(kRT) void reuse_finalize_kernel(
    const float* __restrict__ scores, int64_t scores_ld, const int32_t* __restrict__ sel, int keep,
    int history, int key_count, int sink_end, int recent_start, int rec_begin, int n_rec, int keep_self,
    int64_t* __restrict__ final_idx, uint8_t* __restrict__ final_valid, int32_t* __restrict__ attn_ids,
    int n_out, uint8_t* __restrict__ hf, int64_t hf_ld, int append = 0) {
  const int row = blockIdx.x, tid = threadIdx.x;
  uint8_t* hrow = hf + static_cast<int64_t>(row) * hf_ld * (BITS ? 8 : 1);
  uint64_t* hw = reinterpret_cast<uint64_t*>(hrow);
  if constexpr (BITS) {
    for (int j = tid; j < (history + 63) / 64; j += kRT) {
      uint64_t w = 0;
      for (int b = 0; b < 64; ++b) {
        const int t = 64 * j + b;
        w |= static_cast<uint64_t>(t < history && ((t < sink_end) || (t >= recent_start))) << b;
      }
      hw[j] = w;
    }
  } else {
    for (int t = tid; t < history; t += kRT) hrow[t] = (t < sink_end) || (t >= recent_start);
  }
  __syncthreads();
  const int32_t* srow = sel + static_cast<int64_t>(row) * keep;
  const float* sc = scores + static_cast<int64_t>(row) * scores_ld;
  const int64_t o = static_cast<int64_t>(row) * n_out;
  for (int i = tid; i < keep; i += kRT) {
    const int idx = srow[i];
    const float s = sc[idx];
    const bool valid = isfinite(s);
    if (valid) {
      if constexpr (BITS) atomicOr(reinterpret_cast<unsigned long long*>(hw + (idx >> 6)), 1ull << (idx & 63));
      else hrow[idx] = 1;
    }
    const bool fv = valid && (append || (idx >= sink_end && !(idx >= recent_start && idx < history)));
    final_idx[o + i] = idx;
    final_valid[o + i] = fv;
    if (attn_ids) attn_ids[o + i] = fv ? idx : -1;
  }
  const int extra = sink_end + n_rec + keep_self;
  for (int i = tid; i < extra; i += kRT) {
    const int idx = i < sink_end ? i : (i < sink_end + n_rec ? rec_begin + (i - sink_end) : key_count - 1);
    final_idx[o + keep + i] = idx;
    final_valid[o + keep + i] = 1;
    if (attn_ids) attn_ids[o + keep + i] = idx;
  }
}

// The final list of a given selection (EV:2938-2982, as the periodic
// candidate mode rebuilds it from the indices a previous step kept,
// EV:4535-4548 and 4592-4600): entry i < n_sel is selected index i, valid
// where it lies in [0, history) outside the sink and recent ranges; then the
// sink range, the recent range and the current token.  One thread per entry.
__global__ __launch_bounds__(kRT) void final_from_selected_kernel(
    const int64_t* __restrict__ sel, int64_t sel_ld, int n_sel, int history, int key_count, int sink_end,
    int recent_start, int rec_begin, int n_rec, int64_t* __restrict__ final_idx, uint8_t* __restrict__ final_valid,
    int32_t* __restrict__ attn_ids, int n_out) {
  const int row = blockIdx.y, i = blockIdx.x * kRT + threadIdx.x;
  if (i >= n_out) return;
  int64_t idx;
  bool fv = true;
  if (i < n_sel) {
    idx = sel[static_cast<int64_t>(row) * sel_ld + i];
    fv = idx >= sink_end && idx < history && !(idx >= recent_start);
  } else {
    const int e = i - n_sel;
    idx = e < sink_end ? e : (e < sink_end + n_rec ? rec_begin + (e - sink_end) : key_count - 1);
  }
  const int64_t o = static_cast<int64_t>(row) * n_out + i;
  final_idx[o] = idx;
  final_valid[o] = fv ? 1 : 0;
  if (attn_ids) attn_ids[o] = fv ? static_cast<int32_t>(idx) : -1;
}

// ---------------------------------------------------------------------------
// Rows of at most kWideMax values: one 1024-thread workgroup per row holds
// the row in registers (WideSelect) and does the whole selection in one
// launch.  Longer rows take the staged top-k and the kernels above.
// ---------------------------------------------------------------------------
constexpr int kWideNT = 1024;
constexpr int kWideMax = kWideNT * 40;

// mask[r, t] = values[r, t] >= the row's k-th largest value.
// thr_out (optional) receives the k-th largest value; with mask null only
// the threshold is written.  bits (optional, with mask null): the mask as a
// bitset instead, 64 positions per word (bit t % 64 of word t / 64; row
// stride bits_ld words), the words of [0, ceil(n / 64)) written.
template <int VPL>
__global__ __launch_bounds__(kWideNT) void reuse_mask_wide_kernel(const float* __restrict__ values, int64_t ld, int n,
                                                                  int k, uint8_t* __restrict__ mask, int64_t mask_ld,
                                                                  float* __restrict__ thr_out,
                                                                  const uint8_t* __restrict__ gate = nullptr,
                                                                  int gate_refresh = 0, int gate_rows = 0,
                                                                  uint64_t* __restrict__ bits = nullptr,
                                                                  int64_t bits_ld = 0) {
  using WS = WideSelect<VPL, false>;
  __shared__ typename WS::Shared sh;
  WS ws;
  const int row = blockIdx.x, tid = threadIdx.x;
  if (gate) {   // a lagged step: rows that keep no new candidates are skipped (uniform)
    __shared__ int gate_cnt[kWideNT / 64];
    if (!lag_refreshes(gate, gate_refresh, gate_rows, row, gate_cnt)) return;
  }
  ws.load_count(values + static_cast<int64_t>(row) * ld, n, sh);   // the first digit counted as keys arrive
  ws.run_counted(k, sh);
  if (thr_out) {
    // theta may be the lower bound of a boundary bin taken whole: the k-th
    // largest is the smallest key at or above it
    __shared__ uint32_t wave_min[kWideNT / 64];
    uint32_t m = 0xFFFFFFFFu;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      if (WS::pos(i) < n && ws.u[i] >= ws.theta) m = min(m, ws.u[i]);
    m = wave_minmax_u32<false>(m);
    if ((tid & 63) == 0) wave_min[tid >> 6] = m;
    __syncthreads();
    if (tid == 0) {
      for (int w = 1; w < kWideNT / 64; ++w) m = min(m, wave_min[w]);
      thr_out[row] = sortable_f32(min(m, wave_min[0]));
    }
  }
  if (bits) {   // slot i of wave w covers the 64 positions of word w * VPL + i: one ballot each
    const int lane = tid & 63, wave = tid >> 6;
    uint64_t* brow = bits + static_cast<int64_t>(row) * bits_ld;
    const int n_words = (n + 63) / 64;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const uint64_t m = __ballot(ws.on(i) && ws.u[i] >= ws.theta);
      if (lane == 0 && wave * VPL + i < n_words) brow[wave * VPL + i] = m;
    }
    return;
  }
  if (!mask) return;
  // A slot of a wave covers 64 consecutive positions: its flags are one
  // ballot.  The wave's VPL ballots go to LDS; lane l then writes the 16
  // flags of positions 16q..16q+15 of the wave's range (q = l, l + 64, ...)
  // as one 16-byte store (bytes one by one past the row end or when the row
  // is not 16-byte aligned).
  __shared__ uint64_t bal[kWideNT / 64][VPL];
  uint8_t* mrow = mask + static_cast<int64_t>(row) * mask_ld;
  const int lane = tid & 63, wave = tid >> 6;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const uint64_t m = __ballot(ws.u[i] >= ws.theta);
    if (lane == 0) bal[wave][i] = m;
  }
  __builtin_amdgcn_wave_barrier();   // (a wave's LDS writes complete before its reads)
  const bool vec = (reinterpret_cast<uintptr_t>(mrow) & 15) == 0;
  const int wbase = wave * 64 * VPL;
  for (int q = lane; q < 4 * VPL; q += 64) {
    const uint32_t bits = static_cast<uint32_t>(bal[wave][q >> 2] >> (16 * (q & 3))) & 0xFFFFu;
    const int t0 = wbase + 16 * q;
    if (vec && t0 + 16 <= n) {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) w[j] = (((bits >> (4 * j)) & 0xFu) * 0x00204081u) & 0x01010101u;   // 4 bits -> 4 bytes
      *reinterpret_cast<uint4*>(mrow + t0) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
      for (int j = 0; j < 16 && t0 + j < n; ++j) mrow[t0 + j] = (bits >> j) & 1u;
    }
  }
}

// The candidate bitset across several workgroups per row (rows of at most
// kWideMax scores), in one launch after reuse_partial_kernel<DT, true> has
// counted every row's first digit into hist.  Slice s of a row (kWideNT * J
// scores; slot i of wave w covers bitset word s * 16 * J + w * J + i) finds
// the row's boundary bin from the histogram -- the bin holding the k-th
// largest score, as WideSelect resolves its first digit -- and writes its
// words with the scores above that bin set.  Its scores inside the bin go,
// compacted, to its part of the row's list (list_val / list_pos from
// s * kWideNT * J), their count to state[row * kCandState + s].  The row's
// last slice to finish (ticket state[row * kCandState + kCandSlices]) then
// selects the rank-th largest of the list (the k-th largest of the row),
// sets the bits of the list's scores at or above it, writes it to thr_out
// (optional), and returns the row's histogram and ticket to zero for the
// next call.  Slices store coherently and complete their stores before the
// ticket; the last slice reads coherently.  The ticket is the only atomic
// that workgroups share (a chain of same-address atomics from many
// workgroups costs about 0.2 us a link).
// ---------------------------------------------------------------------------
constexpr int kCandSlices = kWideMax / kWideNT;   // slices of at least kWideNT scores
constexpr int kCandState = kCandSlices + 8;       // state ints per row

// Offset in the row's list of its p-th bin score: slice s's scores start at
// s * slice_len, pre[s] of them before it (pre: slices + 1 prefix counts).
__device__ __forceinline__ int cand_list_at(const int* pre, int slices, int slice_len, int p) {
  int lo = 0, hi = slices - 1;   // the last slice with pre[s] <= p
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (pre[mid] <= p) lo = mid;
    else hi = mid - 1;
  }
  return lo * slice_len + (p - pre[lo]);
}

// The smallest of the taken scores' keys over the workgroup, as the row's
// threshold (theta may be the lower bound of a boundary bin taken whole).
__device__ void cand_write_threshold(uint32_t mn, float* __restrict__ thr) {
  __shared__ uint32_t wave_min[kWideNT / 64];
  mn = wave_minmax_u32<false>(mn);
  if ((threadIdx.x & 63) == 0) wave_min[threadIdx.x >> 6] = mn;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kWideNT / 64; ++w) mn = min(mn, wave_min[w]);
    *thr = sortable_f32(mn);
  }
}

// The rank-th largest of the m list scores held in registers (m <= kWideNT *
// VPL), its bits set in brow.
// The list's scores share the boundary bin's digit: the radix passes start
// below it, in sh.hist[1] (clear: boundary() cleared it).
template <int VPL, typename At>
__device__ void cand_list_finish(void* raw, const float* __restrict__ lv, const int* __restrict__ lp, int m,
                                 int rank, int bin, int n, uint64_t* __restrict__ brow, float* __restrict__ thr,
                                 At&& at) {
  using WS = WideSelect<VPL, false>;
  auto& sh = *static_cast<typename WS::Shared*>(raw);
  WS ws;
  int off[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int p = WS::pos(i);
    off[i] = p < m ? at(p) : 0;
    ws.set(i, p < m ? ld_coherent(lv + off[i]) : 0.0f, p < m);
  }
  ws.kr = rank;
  ws.kk = rank;
  const uint32_t prefix = static_cast<uint32_t>(bin) << (32 - kCandBits);
  ws.passes(sh, prefix, ~((1u << (32 - kCandBits)) - 1u), 32 - kCandBits, 1, prefix, false);
  uint32_t mn = 0xFFFFFFFFu;
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    if (ws.on(i) && ws.u[i] >= ws.theta) {
      const int pos = ld_coherent(lp + off[i]);
      if (static_cast<unsigned>(pos) < static_cast<unsigned>(n))   // (a position of this row's scores)
        atomicOr(reinterpret_cast<unsigned long long*>(brow + (pos >> 6)), 1ull << (pos & 63));
      mn = min(mn, ws.u[i]);
    }
  }
  if (thr) cand_write_threshold(mn, thr);
}

// The same for a list too long for registers: radix passes over the bits
// below the boundary bin's digit, the list read from memory on every pass.
template <typename At>
__device__ void cand_list_finish_stream(void* raw, const float* __restrict__ lv, const int* __restrict__ lp, int m,
                                        int rank, int bin, int n, uint64_t* __restrict__ brow,
                                        float* __restrict__ thr, At&& at) {
  using WS = WideSelect<1, false>;
  auto& sh = *static_cast<typename WS::Shared*>(raw);
  const int tid = threadIdx.x;
  WS ws;
  ws.kr = rank;
  uint32_t prefix = static_cast<uint32_t>(bin) << (32 - kCandBits), mask = ~((1u << (32 - kCandBits)) - 1u);
  int remaining = 32 - kCandBits, buf = 0;
#pragma unroll
  for (int j = 0; j < WS::NB / kWideNT; ++j) sh.hist[0][tid + kWideNT * j] = 0;
  __syncthreads();
  while (remaining > 0) {   // uniform
    const int shift = remaining > WS::RB ? remaining - WS::RB : 0;
    const uint32_t dmask = (1u << (remaining - shift)) - 1u;
    for (int p = tid; p < m; p += kWideNT) {
      const uint32_t u = f32_sortable(ld_coherent(lv + at(p)));
      if ((u & mask) == prefix) atomicAdd(&sh.hist[buf][(u >> shift) & dmask], 1);
    }
    __syncthreads();
    int b, krl, whole;
    ws.boundary(sh, sh.hist[buf], sh.hist[buf ^ 1], b, krl, whole);
    prefix |= static_cast<uint32_t>(b) << shift;
    mask |= dmask << shift;
    ws.kr = krl;
    remaining = whole ? 0 : shift;
    buf ^= 1;
    __syncthreads();   // (the histogram's reads are done before the next pass)
  }
  // prefix: the smallest taken key or the lower bound of a bin taken whole
  uint32_t mn = 0xFFFFFFFFu;
  for (int p = tid; p < m; p += kWideNT) {
    const int o = at(p);
    const uint32_t u = f32_sortable(ld_coherent(lv + o));
    if (u >= prefix) {
      const int pos = ld_coherent(lp + o);
      if (static_cast<unsigned>(pos) < static_cast<unsigned>(n))
        atomicOr(reinterpret_cast<unsigned long long*>(brow + (pos >> 6)), 1ull << (pos & 63));
      mn = min(mn, u);
    }
  }
  if (thr) cand_write_threshold(mn, thr);
}

// The exact-candidate attention's final list (reuse_final_wide_kernel's
// outputs for its scores path): where the list, flags and mask go, and the
// row's protected ranges.
struct QabsListOut {
  uint64_t* nf;             // workspace: non-finite scores, one bit per position (row stride bits_ld)
  int64_t* final_idx;
  uint8_t* final_valid;
  int32_t* attn_ids;        // optional
  int n_out;
  uint8_t* hf;              // byte mask [rows, hf_ld]
  int64_t hf_ld;
  int key_count, sink_end, recent_start, rec_begin, n_rec, keep_self, append;
};

// The bin's taken scores (above theta, or equal to it among the first kr in
// position order: WideSelect's rule) as bits of fw, from the list in
// registers (m <= kWideNT * VPL).  The radix passes start below the bin's
// digit in sh.hist[1] (clear: boundary() cleared it).
template <int VPL, typename At>
__device__ void qabs_bin_taken(void* raw, const float* __restrict__ lv, const int* __restrict__ lp, int m, int rank,
                               int bin, int n, uint64_t* fw, At&& at) {
  using WS = WideSelect<VPL, false>;
  auto& sh = *static_cast<typename WS::Shared*>(raw);
  WS ws;
  int off[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int p = WS::pos(i);
    off[i] = p < m ? at(p) : 0;
    ws.set(i, p < m ? ld_coherent(lv + off[i]) : 0.0f, p < m);
  }
  ws.kr = rank;
  ws.kk = rank;
  const uint32_t prefix = static_cast<uint32_t>(bin) << (32 - kCandBits);
  ws.passes(sh, prefix, ~((1u << (32 - kCandBits)) - 1u), 32 - kCandBits, 1, prefix, false);
  ws.place_uniform(sh, [&](int, int, int slot) {
    const int pos = ld_coherent(lp + off[slot]);
    if (static_cast<unsigned>(pos) < static_cast<unsigned>(n)) atomicOr(&fw[pos >> 6], 1ull << (pos & 63));
  });
}

// The same for a list too long for registers: radix passes over the list in
// memory, then the equal scores ranked in position order 1024 at a time.
template <typename At>
__device__ void qabs_bin_taken_stream(void* raw, const float* __restrict__ lv, const int* __restrict__ lp, int m,
                                      int rank, int bin, int n, uint64_t* fw, At&& at) {
  using WS = WideSelect<1, false>;
  auto& sh = *static_cast<typename WS::Shared*>(raw);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  WS ws;
  ws.kr = rank;
  uint32_t prefix = static_cast<uint32_t>(bin) << (32 - kCandBits), mask = ~((1u << (32 - kCandBits)) - 1u);
  int remaining = 32 - kCandBits, buf = 0;
#pragma unroll
  for (int j = 0; j < WS::NB / kWideNT; ++j) sh.hist[0][tid + kWideNT * j] = 0;
  __syncthreads();
  while (remaining > 0) {   // uniform
    const int shift = remaining > WS::RB ? remaining - WS::RB : 0;
    const uint32_t dmask = (1u << (remaining - shift)) - 1u;
    for (int p = tid; p < m; p += kWideNT) {
      const uint32_t u = f32_sortable(ld_coherent(lv + at(p)));
      if ((u & mask) == prefix) atomicAdd(&sh.hist[buf][(u >> shift) & dmask], 1);
    }
    __syncthreads();
    int b, krl, whole;
    ws.boundary(sh, sh.hist[buf], sh.hist[buf ^ 1], b, krl, whole);
    prefix |= static_cast<uint32_t>(b) << shift;
    mask |= dmask << shift;
    ws.kr = whole ? 0x7FFFFFFF : krl;
    remaining = whole ? 0 : shift;
    buf ^= 1;
    __syncthreads();   // (the histogram's reads are done before the next pass)
  }
  // prefix: theta; equal keys are taken while fewer than kr came before
  const int kr = ws.kr;
  int eq_seen = 0;   // equal keys in the earlier rounds (uniform)
  for (int p0 = 0; p0 < m; p0 += kWideNT) {   // uniform
    const int p = p0 + tid;
    const int o = p < m ? at(p) : 0;
    const uint32_t u = p < m ? f32_sortable(ld_coherent(lv + o)) : 0u;
    const bool gt = p < m && u > prefix, eq = p < m && u == prefix;
    const uint64_t be = __ballot(eq);
    if (lane == 0) sh.wave_eq[wave] = __popcll(be);
    __syncthreads();
    int before = eq_seen, round = 0;
#pragma unroll
    for (int w = 0; w < WS::NW; ++w) {
      before += w < wave ? sh.wave_eq[w] : 0;
      round += sh.wave_eq[w];
    }
    before += static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(be >> 32),
                                                         __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(be), 0)));
    if (gt || (eq && before < kr)) {
      const int pos = ld_coherent(lp + o);
      if (static_cast<unsigned>(pos) < static_cast<unsigned>(n)) atomicOr(&fw[pos >> 6], 1ull << (pos & 63));
    }
    eq_seen += round;
    __syncthreads();   // (wave_eq is rewritten next round)
  }
}

// The row's final list from its taken positions (fw, LDS, one word per
// thread): ascending positions, an entry valid when its score is finite and
// (append or) it lies outside the protected ranges; then the sink range,
// the recent range and the current token; the byte mask = the protected
// ranges plus the taken positions with finite scores
// (reuse_final_wide_kernel's emit, EV:2938-2982).  wsum: kWideNT / 64 ints
// of LDS.
__device__ void qabs_emit_list(const uint64_t* fw, const uint64_t* __restrict__ nf_row, int history, int keep,
                               int row, const QabsListOut& qs, int* wsum) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n_words = (history + 63) / 64;
  const uint64_t w = tid < n_words ? fw[tid] : 0ull;
  const uint64_t nf = tid < n_words ? __hip_atomic_load(nf_row + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                    : 0ull;
  const int c = __popcll(w), incl = wave_incl_scan_dpp(c);
  __syncthreads();   // (wsum's last readers are done)
  if (lane == 63) wsum[wave] = incl;
  __syncthreads();
  int p = incl - c;
#pragma unroll
  for (int v = 0; v < kWideNT / 64; ++v) p += v < wave ? wsum[v] : 0;
  const int64_t o = static_cast<int64_t>(row) * qs.n_out;
  for (uint64_t x = w; x; x &= x - 1) {   // this word's taken positions, ascending
    const int idx = 64 * tid + __builtin_ctzll(x);
    if (p < keep) {
      const bool finite = !((nf >> (idx & 63)) & 1ull);
      const bool fv = finite && (qs.append || (idx >= qs.sink_end && !(idx >= qs.recent_start && idx < history)));
      qs.final_idx[o + p] = idx;
      qs.final_valid[o + p] = fv;
      if (qs.attn_ids) qs.attn_ids[o + p] = fv ? idx : -1;
    }
    ++p;
  }
  // the byte mask, 64 positions per thread
  if (tid < n_words) {
    auto range = [](int j, int a, int b) -> uint64_t {   // bits of [a, b) in word j
      const int lo = max(a, 64 * j) - 64 * j, hi = min(b, 64 * j + 64) - 64 * j;
      if (hi <= lo) return 0ull;
      const uint64_t upto = hi >= 64 ? ~0ull : ((1ull << hi) - 1ull);
      return upto & ~((1ull << lo) - 1ull);
    };
    const uint64_t bitsm = (w & ~nf) | range(tid, 0, qs.sink_end) | range(tid, qs.recent_start, history);
    uint8_t* hrow = qs.hf + static_cast<int64_t>(row) * qs.hf_ld + 64 * tid;
    if (64 * tid + 64 <= history && (reinterpret_cast<uintptr_t>(hrow) & 15) == 0) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t b16 = static_cast<uint32_t>(bitsm >> (16 * q)) & 0xFFFFu;
        uint32_t x4[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) x4[j] = (((b16 >> (4 * j)) & 0xFu) * 0x00204081u) & 0x01010101u;
        *reinterpret_cast<uint4*>(hrow + 16 * q) = make_uint4(x4[0], x4[1], x4[2], x4[3]);
      }
    } else {
      for (int j = 0; j < 64 && 64 * tid + j < history; ++j) hrow[j] = (bitsm >> j) & 1ull;
    }
  }
  const int extra = qs.sink_end + qs.n_rec + qs.keep_self;
  for (int i = tid; i < extra; i += kWideNT) {
    const int idx = i < qs.sink_end ? i : (i < qs.sink_end + qs.n_rec ? qs.rec_begin + (i - qs.sink_end)
                                                                      : qs.key_count - 1);
    qs.final_idx[o + keep + i] = idx;
    qs.final_valid[o + keep + i] = 1;
    if (qs.attn_ids) qs.attn_ids[o + keep + i] = idx;
  }
}

// LIST: the row's final selection of the exact-candidate attention instead
// (reuse_final_wide_kernel's output from the row's scores, qs): k = keep,
// equal scores at the threshold taken lowest positions first; bits are the
// workspace's above-bin words, qs.nf its non-finite-score words, and the
// last slice writes the final list, flags and mask (qabs_emit_list).
template <int J, bool LIST = false>
__global__ __launch_bounds__(kWideNT) void reuse_cand_slices_kernel(
    const float* __restrict__ values, int64_t ld, int n, int k, int slices, int* __restrict__ hist,
    int* __restrict__ state, float* __restrict__ list_val, int* __restrict__ list_pos, int64_t list_ld,
    uint64_t* __restrict__ bits, int64_t bits_ld, float* __restrict__ thr_out, QabsListOut qs = {},
    const uint8_t* __restrict__ gate = nullptr, int gate_refresh = 0, int gate_rows = 0) {
  using WS = WideSelect<1, false>;
  static_assert(sizeof(typename WideSelect<1, false>::Shared) == sizeof(typename WideSelect<8, false>::Shared),
                "one shared layout for every list length");
  __shared__ typename WS::Shared sh;
  __shared__ int wave_cnt[kWideNT / 64];
  __shared__ int pre[kCandSlices + 1];
  __shared__ int last_sh;
  __shared__ uint64_t fw[LIST ? kWideMax / 64 : 1];   // LIST: the row's taken positions
  const int row = blockIdx.x / slices, s = blockIdx.x - row * slices;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (gate) {   // a lagged step: rows that keep no new candidates are skipped (uniform; the
                // partial scores skipped them too, so their histogram and ticket stay zero)
    if (!lag_refreshes(gate, gate_refresh, gate_rows, row, wave_cnt)) return;
    __syncthreads();   // (wave_cnt is reused)
  }
  int* hrow = hist + static_cast<int64_t>(row) * kCandBins;
  const float* vrow = values + static_cast<int64_t>(row) * ld;
  // the histogram (4 bins per thread) and the slice's scores, all loads in flight
  const int4 hv = *reinterpret_cast<const int4*>(hrow + 4 * tid);
  const int w0 = s * 16 * J + wave * J;   // the wave's first word
  float v[J];
#pragma unroll
  for (int i = 0; i < J; ++i) v[i] = vrow[min(64 * (w0 + i) + lane, n - 1)];
  *reinterpret_cast<int4*>(sh.hist[0] + 4 * tid) = hv;
  __syncthreads();
  WS ws;
  ws.kr = k;
  int bin, rank, whole;
  ws.boundary(sh, sh.hist[0], sh.hist[1], bin, rank, whole);
  int* srow = state + static_cast<int64_t>(row) * kCandState;
  uint64_t* brow = bits + static_cast<int64_t>(row) * bits_ld;
  const int n_words = (n + 63) / 64;
  uint32_t inbin = 0;   // bit i: slot i's score is in the boundary bin
#pragma unroll
  for (int i = 0; i < J; ++i) {
    const int p = 64 * (w0 + i) + lane;
    const uint32_t d = f32_sortable(v[i]) >> (32 - kCandBits);
    const uint64_t w = __ballot(p < n && d > static_cast<uint32_t>(bin));
    if (lane == 0 && w0 + i < n_words)
      __hip_atomic_store(brow + w0 + i, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if constexpr (LIST) {
      const uint64_t f = __ballot(p < n && !isfinite(v[i]));
      if (lane == 0 && w0 + i < n_words)
        __hip_atomic_store(qs.nf + static_cast<int64_t>(row) * bits_ld + w0 + i, f, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    inbin |= static_cast<uint32_t>(p < n && d == static_cast<uint32_t>(bin)) << i;
  }
  // the slice's bin scores compacted in (wave, slot, lane) = position order
  // (one ballot per slot: a thread's own slots are 64 positions apart)
  uint64_t bal[J];
  int wtot = 0;
#pragma unroll
  for (int i = 0; i < J; ++i) {
    bal[i] = __ballot((inbin >> i) & 1u);
    wtot += __popcll(bal[i]);
  }
  if (lane == 0) wave_cnt[wave] = wtot;
  __syncthreads();
  int at = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kWideNT / 64; ++w) {
    at += w < wave ? wave_cnt[w] : 0;
    total += wave_cnt[w];
  }
  if (tid == 0) st_coherent(srow + s, total);
  if (wtot) {   // uniform per wave
    const int64_t base = static_cast<int64_t>(row) * list_ld + static_cast<int64_t>(s) * kWideNT * J;
#pragma unroll
    for (int i = 0; i < J; ++i) {
      if ((inbin >> i) & 1u) {
        const int e = at + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                               static_cast<uint32_t>(bal[i] >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal[i]), 0)));
        st_coherent(list_val + base + e, v[i]);
        st_coherent(list_pos + base + e, 64 * (w0 + i) + lane);
      }
      at += __popcll(bal[i]);
    }
  }
  // Every word, count and list store of this workgroup has completed before its ticket.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    // compiler-only fences keep memory operations on their side of the ticket
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const int t = __hip_atomic_fetch_add(srow + kCandSlices, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    const bool last = t == slices - 1;
    if (last) __hip_atomic_store(srow + kCandSlices, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_sh = last;
  }
  __syncthreads();
  if (!last_sh) return;
  // The row's last slice: every slice has read the histogram and stored its list.
  if (tid < 64) {   // prefix counts of the slices' lists (slices <= 40)
    const int c = tid < slices ? ld_coherent(srow + tid) : 0;
    const int inc = wave_incl_scan_dpp(c);
    if (tid <= slices) pre[tid] = inc - c;
  }
  *reinterpret_cast<int4*>(hrow + 4 * tid) = make_int4(0, 0, 0, 0);
  __syncthreads();
  const int m = min(pre[slices], n);
  const float* lv = list_val + static_cast<int64_t>(row) * list_ld;
  const int* lp = list_pos + static_cast<int64_t>(row) * list_ld;
  float* thr = thr_out ? thr_out + row : nullptr;
  const int slice_len = kWideNT * J;
  auto at_fn = [&](int p) { return cand_list_at(pre, slices, slice_len, p); };
  if constexpr (LIST) {
    for (int j = tid; j < n_words; j += kWideNT)
      fw[j] = __hip_atomic_load(brow + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (m <= kWideNT) qabs_bin_taken<1>(&sh, lv, lp, m, rank, bin, n, fw, at_fn);
    else if (m <= 8 * kWideNT) qabs_bin_taken<8>(&sh, lv, lp, m, rank, bin, n, fw, at_fn);
    else qabs_bin_taken_stream(&sh, lv, lp, m, rank, bin, n, fw, at_fn);
    __syncthreads();
    qabs_emit_list(fw, qs.nf + static_cast<int64_t>(row) * bits_ld, n, k, row, qs, wave_cnt);
  } else {
    if (m <= kWideNT) cand_list_finish<1>(&sh, lv, lp, m, rank, bin, n, brow, thr, at_fn);
    else if (m <= 8 * kWideNT) cand_list_finish<8>(&sh, lv, lp, m, rank, bin, n, brow, thr, at_fn);
    else cand_list_finish_stream(&sh, lv, lp, m, rank, bin, n, brow, thr, at_fn);
  }
}

// The step's candidates in one launch (rows of at most kWideMax history
// tokens, head_dim <= 128, a 16-byte aligned dim-major copy): one 1024-thread
// workgroup per row forms the row's partial scores as reuse_partial_kernel
// does (eight consecutive tokens per thread and chunk, NCH chunks, the same
// loads and summation order), writes them, counts their first radix digit
// as they are formed, selects the k-th largest in registers (WideSelect)
// and writes mask = score >= it; thr_out (optional) receives it.  The row's
// scores never make the round trip through memory that the two-launch form
// (partial scores, then reuse_mask_wide_kernel) takes.  With rows a multiple
// of 8 the rows are spread so that each XCD (blockIdx.x % 8 on gfx950) runs
// rows/8 consecutive ones -- the query heads of one KV head, which read the
// same copy rows, share that XCD's L2.  gate: as reuse_mask_wide_kernel.
template <int DT, int NCH>
__global__ __launch_bounds__(kWideNT) void reuse_candidates_kernel(
    const typename Elem<DT>::T* __restrict__ query, const typename Elem<DT>::T* __restrict__ kdm, int q_heads,
    int group, int history, int head_dim, int count, int64_t sb, int64_t sh, int64_t sd, float* __restrict__ out,
    int64_t out_ld, int k, uint8_t* __restrict__ mask, int64_t mask_ld, float* __restrict__ thr_out,
    const uint8_t* __restrict__ gate, int gate_refresh, int rows, uint64_t* __restrict__ bits, int64_t bits_ld) {
  using E = typename Elem<DT>::T;
  constexpr int VPL = 8 * NCH;
  using WS = WideSelect<VPL, false>;
  __shared__ typename WS::Shared wsh;
  __shared__ float q_s[128];
  __shared__ __attribute__((aligned(16))) uint64_t key_s[128];
  __shared__ int sel_idx[kMaxDims];
  __shared__ float sel_q[kMaxDims];
  const int tid = threadIdx.x;
  const int row = rows % 8 == 0 ? (blockIdx.x % 8) * (rows / 8) + blockIdx.x / 8 : blockIdx.x;
  if (gate) {   // a lagged step: rows that keep no new candidates are skipped (uniform)
    __shared__ int gate_cnt[kWideNT / 64];
    if (!lag_refreshes(gate, gate_refresh, rows, row, gate_cnt)) return;
  }
  const int b = row / q_heads, h = row - b * q_heads;
  if (tid < head_dim) q_s[tid] = Elem<DT>::load(query + static_cast<int64_t>(row) * head_dim + tid);
#pragma unroll
  for (int j = 0; j < WS::NB / kWideNT; ++j) wsh.hist[0][tid + kWideNT * j] = 0;
  __syncthreads();
  rank_dims128(q_s, key_s, head_dim, count, sel_idx, sel_q);   // (ends with a barrier)

  WS ws;
  int ninf = 0;
  const E* base = kdm + b * sb + (h / group) * sh;
  float* orow = out + static_cast<int64_t>(row) * out_ld;
  const bool ovec = (reinterpret_cast<uintptr_t>(orow) & 15) == 0;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int t0 = (c * kWideNT + tid) * 8;
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    if (t0 + 8 <= history) {
      for (int s0 = 0; s0 < count; s0 += 8) {   // eight dims' loads in flight, added in selection order
        float v[8][8];
#pragma unroll
        for (int j = 0; j < 8; ++j) load8<DT>(base + sel_idx[min(s0 + j, count - 1)] * sd + t0, v[j]);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (s0 + j < count) {
            const float qs = sel_q[s0 + j];
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = acc[i] + qs * v[j][i];
          }
        }
      }
      if (ovec) {
        *reinterpret_cast<float4*>(orow + t0) = make_float4(acc[0], acc[1], acc[2], acc[3]);
        *reinterpret_cast<float4*>(orow + t0 + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) orow[t0 + i] = acc[i];
      }
    } else if (t0 < history) {   // the row's last n < 8 tokens: clamped in-row loads, n stored
      const int n = history - t0;
      for (int s0 = 0; s0 < count; s0 += 8) {
        float v[8][8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const E* p = base + sel_idx[min(s0 + j, count - 1)] * sd + t0;
#pragma unroll
          for (int i = 0; i < 8; ++i) v[j][i] = Elem<DT>::load(p + min(i, n - 1));
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          if (s0 + j < count) {
            const float qs = sel_q[s0 + j];
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = acc[i] + qs * v[j][i];
          }
        }
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (i < n) orow[t0 + i] = acc[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      ws.set(8 * c + i, acc[i], t0 + i < history);
      ws.count(8 * c + i, wsh, ninf);
    }
  }
  ws.count_done(wsh, ninf);
  ws.run_counted(k, wsh);
  if (thr_out) {   // the k-th largest: the smallest key at or above theta
    __shared__ uint32_t wave_min[kWideNT / 64];
    uint32_t m = 0xFFFFFFFFu;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      if (ws.on(i) && ws.u[i] >= ws.theta) m = min(m, ws.u[i]);
    m = wave_minmax_u32<false>(m);
    if ((tid & 63) == 0) wave_min[tid >> 6] = m;
    __syncthreads();
    if (tid == 0) {
      for (int w = 1; w < kWideNT / 64; ++w) m = min(m, wave_min[w]);
      thr_out[row] = sortable_f32(min(m, wave_min[0]));
    }
  }
  if (bits) {   // the 8 flags of a thread's 8 tokens are one byte of the bitset
    uint8_t* brow = reinterpret_cast<uint8_t*>(bits + static_cast<int64_t>(row) * bits_ld);
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int t0 = (c * kWideNT + tid) * 8;
      uint32_t f = 0;
#pragma unroll
      for (int i = 0; i < 8; ++i) f |= static_cast<uint32_t>(ws.on(8 * c + i) && ws.u[8 * c + i] >= ws.theta) << i;
      if (t0 < history) brow[t0 / 8] = static_cast<uint8_t>(f);
    }
    if (tid < 7) {   // the rest of the last word
      const int t = ((history + 7) / 8 + tid) * 8;
      if (t < (history + 63) / 64 * 64) brow[t / 8] = 0;
    }
    return;
  }
  uint8_t* mrow = mask + static_cast<int64_t>(row) * mask_ld;
  const bool mvec = (reinterpret_cast<uintptr_t>(mrow) & 7) == 0;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int t0 = (c * kWideNT + tid) * 8;
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      lo |= static_cast<uint32_t>(ws.on(8 * c + i) && ws.u[8 * c + i] >= ws.theta) << (8 * i);
      hi |= static_cast<uint32_t>(ws.on(8 * c + 4 + i) && ws.u[8 * c + 4 + i] >= ws.theta) << (8 * i);
    }
    if (mvec && t0 + 8 <= history) {
      *reinterpret_cast<uint2*>(mrow + t0) = make_uint2(lo, hi);
    } else {
      for (int i = 0; i < 8 && t0 + i < history; ++i) mrow[t0 + i] = ((i < 4 ? lo >> (8 * i) : hi >> (8 * (i - 4))) & 1u);
    }
  }
}

// out[r, i] = values[r, cols[i]] for i < n_cols (the sampled partial scores
// of the sample_quantile candidate selection, EV:3972-3984).
__global__ __launch_bounds__(kRT) void gather_cols_kernel(const float* __restrict__ values, int64_t ld,
                                                          const int32_t* __restrict__ cols, int n_cols,
                                                          float* __restrict__ out) {
  const int row = blockIdx.y;
  const int i = blockIdx.x * kRT + threadIdx.x;
  if (i < n_cols) out[static_cast<int64_t>(row) * n_cols + i] = values[static_cast<int64_t>(row) * ld + cols[i]];
}

// The final selection of reuse_finalize_kernel, with the keep largest scores
// selected in the same launch.  When the row's union holds at least keep
// finite scores and at most VPLC * 1024 entries (the usual case: the union
// is a few percent of the history), the selection ranks the compacted union
// lists of reuse_scores_kernel (VPLC keys per thread) instead of the whole
// row (VPL keys per thread); up to 2 VPLC * 1024 entries (the block modes,
// whose previous final covers whole blocks) in a wider form of the same.  The keep largest are then finite union scores
// either way, and the lists keep token order, so both paths select and
// place the same entries (ties to the lower token).
constexpr int kMaxTiles = kWideMax / kScoreTile;
constexpr int kTilesPL = (kMaxTiles + 1 + 63) / 64;   // tiles per lane in the offset scan (and the end)
constexpr int kTileStep0 = kMaxTiles >= 64 ? 64 : 32;   // the tile search's first step
static_assert(kMaxTiles < 128, "the final selection's tile search takes seven steps");

// The token attention of one row (a query head) over its final list, by the
// workgroup that selected it (reuse_final_wide_kernel with ATTN): softmax(
// scaling * q.K[t]) . V[t] over the list's valid entries (-1 skipped), in
// fp32, the output rounded once to the K/V dtype; a row with no valid entry
// gives zeros (QK:388, 404).  Lane 16g + c of a wave holds channels
// 8c..8c+7 of the list entry e = 64 s + 4 w + g at step s (wave w), the
// dot product a 16-lane sum; the K/V rows of four steps are in flight ahead
// of the one computed.  Each (wave, lane group) keeps a running maximum and
// sum; the 64 partials meet in LDS.
struct ReuseAttn {
  const uint16_t *q, *k, *v;   // q [rows, 128]; K/V [B, Hkv, T, 128] at (sb, sh, st), channels contiguous
  int64_t sb, sh, st;
  int q_heads, group;
  float scale_log2;            // scaling * log2(e)
  uint16_t* out;               // [rows, 128]
};
constexpr int kAttnList = 4096;   // the longest final list the fused attention holds in LDS
struct AttnPartials {
  float acc[64][128];
  float m[64], l[64];
};

template <int DT>
__device__ __forceinline__ void unpack8_16(const uint4& w, float (&x)[8]) {
  const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t lo = static_cast<uint16_t>(u[i] & 0xFFFFu), hi = static_cast<uint16_t>(u[i] >> 16);
    x[2 * i] = Elem<DT>::load(&lo);
    x[2 * i + 1] = Elem<DT>::load(&hi);
  }
}

template <int DT>
__device__ __forceinline__ void reuse_attend(const int32_t* ids_s, int n, const ReuseAttn& a, int row,
                                             AttnPartials& part) {
  constexpr int DEPTH = 4;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 4, c = lane & 15;
  const int b = row / a.q_heads, h = row - b * a.q_heads;
  const int64_t kv_off = b * a.sb + (h / a.group) * a.sh + 8 * c;
  const uint16_t* kb = a.k + kv_off;
  const uint16_t* vb = a.v + kv_off;
  float qf[8];
  unpack8_16<DT>(*reinterpret_cast<const uint4*>(a.q + static_cast<int64_t>(row) * 128 + 8 * c), qf);
  const float ninf = -__builtin_huge_valf();
  float m = ninf, l = 0.0f, acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
  const int steps = (n + 63) / 64;
  auto tok_of = [&](int s) -> int {
    const int e = s * 64 + wave * 4 + g;
    return (s < steps && e < n) ? ids_s[e] : -1;
  };
  int tk[DEPTH];
  uint4 kx[DEPTH], vx[DEPTH];
#pragma unroll
  for (int u = 0; u < DEPTH; ++u) {   // invalid entries read token 0 (in bounds) and are skipped
    tk[u] = tok_of(u);
    const int64_t at = static_cast<int64_t>(max(tk[u], 0)) * a.st;
    kx[u] = *reinterpret_cast<const uint4*>(kb + at);
    vx[u] = *reinterpret_cast<const uint4*>(vb + at);
  }
  for (int s0 = 0; s0 < steps; s0 += DEPTH) {
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) {
      float kf[8], vf[8];
      unpack8_16<DT>(kx[u], kf);
      unpack8_16<DT>(vx[u], vf);
      const int t = tk[u];
      // the step DEPTH ahead goes out before this one is computed
      tk[u] = tok_of(s0 + u + DEPTH);
      if (s0 + u + DEPTH < steps) {
        const int64_t at = static_cast<int64_t>(max(tk[u], 0)) * a.st;
        kx[u] = *reinterpret_cast<const uint4*>(kb + at);
        vx[u] = *reinterpret_cast<const uint4*>(vb + at);
      }
      float d = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) d = __builtin_fmaf(qf[j], kf[j], d);
      d += dpp_f<0xB1>(d);    // quad_perm [1,0,3,2]
      d += dpp_f<0x4E>(d);    // quad_perm [2,3,0,1]
      d += dpp_f<0x141>(d);   // row_half_mirror
      d += dpp_f<0x140>(d);   // row_mirror: every lane of the 16 holds the sum
      if (t >= 0) {           // uniform in the 16 lanes of the entry
        const float sc = d * a.scale_log2;
        const float mn = fmaxf(m, sc);
        const float al = exp2f(m - mn);   // 0 while m = -inf
        const float p = exp2f(sc - mn);
        l = __builtin_fmaf(l, al, p);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = __builtin_fmaf(acc[j], al, p * vf[j]);
        m = mn;
      }
    }
  }
  const int pi = wave * 4 + g;
#pragma unroll
  for (int j = 0; j < 8; ++j) part.acc[pi][8 * c + j] = acc[j];
  if (c == 0) {
    part.m[pi] = m;
    part.l[pi] = l;
  }
  __syncthreads();
  if (tid < 128) {
    float mx = ninf;
    for (int i = 0; i < 64; ++i) mx = fmaxf(mx, part.m[i]);
    float num = 0.0f, den = 0.0f;
    if (mx != ninf) {
      for (int i = 0; i < 64; ++i) {
        if (part.m[i] == ninf) continue;
        const float w = exp2f(part.m[i] - mx);
        num = __builtin_fmaf(part.acc[i][tid], w, num);
        den = __builtin_fmaf(part.l[i], w, den);
      }
    }
    a.out[static_cast<int64_t>(row) * 128 + tid] = Elem<DT>::store(mx == ninf ? 0.0f : num / den);
  }
}

// The bits of positions [a, b) in 64-position word j.
__device__ __forceinline__ uint64_t word_range_bits(int j, int a, int b) {
  const int lo = max(a, 64 * j) - 64 * j, hi = min(b, 64 * j + 64) - 64 * j;
  if (hi <= lo) return 0ull;
  const uint64_t upto = hi >= 64 ? ~0ull : ((1ull << hi) - 1ull);
  return upto & ~((1ull << lo) - 1ull);
}

// ATTN: the workgroup then attends over the row's final list (reuse_attend;
// DT the K/V dtype, n_out <= kAttnList, head size 128).
// BITS: hf is a bitset (64 positions per uint64 word, hf_ld in words),
// assembled in LDS and stored once.
// xblock > 0 (BITS only): the block modes' expansion in the same launch --
// every aligned block of xblock positions holding a final bit is filled in
// the LDS bitset before it is stored, and the index list is the expanded
// one of reuse_expand_kernel (body_cap body entries, then the sink range,
// the recent range and the current token; n_out = body_cap + those).
template <int VPL, int VPLC, bool BITS = false, int DT = QKV_DTYPE_BF16, bool ATTN = false>
__global__ __launch_bounds__(kWideNT) void reuse_final_wide_kernel(
    const float* __restrict__ scores, int64_t scores_ld, const float* __restrict__ cscore,
    const int32_t* __restrict__ ctok, const int32_t* __restrict__ ccnt, int n_tiles, int64_t c_ld, int keep,
    int history, int key_count, int sink_end, int recent_start, int rec_begin, int n_rec, int keep_self,
    int64_t* __restrict__ final_idx, uint8_t* __restrict__ final_valid, int32_t* __restrict__ attn_ids, int n_out,
    uint8_t* __restrict__ hf, int64_t hf_ld, int append = 0, ReuseAttn at = {}, int xblock = 0, int body_cap = 0) {
  using WS = WideSelect<VPL, false>;
  using WC = WideSelect<2 * VPLC, false>;   // (the LDS of both compacted forms)
  __shared__ union {
    typename WS::Shared d;
    typename WC::Shared c;
    AttnPartials a;
  } sh;
  // the final list staged in LDS (n_out <= kAttnList): entry p holds the
  // index, bitwise negated when the entry is invalid; written out coalesced
  // after the selection instead of three scattered stores per entry
  __shared__ int32_t ids_s[kAttnList];
  __shared__ int tile_off[kMaxTiles + 1];
  __shared__ int n_fin;
  __shared__ uint64_t fin_s[BITS ? kWideMax / 64 : 1];
  const int row = blockIdx.x, tid = threadIdx.x;
  uint8_t* hrow = hf + static_cast<int64_t>(row) * hf_ld * (BITS ? 8 : 1);
  const int n_words = (history + 63) / 64;
  // the tile lists' lengths first (kTilesPL consecutive tiles per lane of
  // wave 0), in flight while the protected ranges are written
  int len[kTilesPL] = {}, nf = 0;
  if (tid < 64 && cscore) {
    const int32_t* cn = ccnt + static_cast<int64_t>(row) * n_tiles * 2;
#pragma unroll
    for (int j = 0; j < kTilesPL; ++j) {
      const int t = tid * kTilesPL + j;
      if (t < n_tiles) {
        len[j] = cn[2 * t];
        nf += cn[2 * t + 1];
      }
    }
  }
  // the protected ranges, 16 bytes per store where the row is 16-byte aligned;
  // written after the selection's loads are out, and ordered before the
  // scatter below by the barriers of the selection (run) or of place
  auto write_protected = [&]() {
    if constexpr (BITS) {   // the protected ranges' bits of every word
      for (int j = tid; j < n_words; j += kWideNT)
        fin_s[j] = word_range_bits(j, 0, sink_end) | word_range_bits(j, recent_start, history);
      return;
    }
    const int body = (reinterpret_cast<uintptr_t>(hrow) & 15) ? 0 : (history & ~15);   // bytes in 16-byte stores
    for (int t0 = 16 * tid; t0 < body; t0 += 16 * kWideNT) {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t x = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int t = t0 + 4 * j + b;
          x |= static_cast<uint32_t>((t < sink_end) || (t >= recent_start)) << (8 * b);
        }
        w[j] = x;
      }
      *reinterpret_cast<uint4*>(hrow + t0) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    for (int t = body + tid; t < history; t += kWideNT) hrow[t] = (t < sink_end) || (t >= recent_start);
  };
  if (tid < 64) {   // tile list offsets: a wave scan of the lengths
    int own = 0;
#pragma unroll
    for (int j = 0; j < kTilesPL; ++j) own += len[j];
    const int incl = wave_incl_scan_dpp(own), fin_all = wave_incl_scan_dpp(nf);
    int at = incl - own;
#pragma unroll
    for (int j = 0; j < kTilesPL; ++j) {
      const int t = tid * kTilesPL + j;
      if (t <= n_tiles) tile_off[t] = at;   // tile_off[n_tiles] = the total
      at += len[j];
    }
    if (tid == 63) n_fin = fin_all;
  }
  if (cscore) {   // the candidates' first digit is counted as they arrive (cleared before the barrier)
#pragma unroll
    for (int j = 0; j < WC::NB / kWideNT; ++j) sh.c.hist[0][tid + kWideNT * j] = 0;
  }
  __syncthreads();
  const int64_t o = static_cast<int64_t>(row) * n_out;
  const bool expand = BITS && xblock > 0;                    // uniform
  const bool staged = !expand && (ATTN || n_out <= kAttnList);   // uniform
  auto emit = [&](int idx, int p, bool valid) {
    if (valid) {
      if constexpr (BITS) atomicOr(&fin_s[idx >> 6], 1ull << (idx & 63));
      else hrow[idx] = 1;
    }
    if (expand) return;   // the list is the expanded one, written below
    const bool fv = valid && (append || (idx >= sink_end && !(idx >= recent_start && idx < history)));
    if (staged) {
      ids_s[p] = fv ? idx : ~idx;
    } else {
      final_idx[o + p] = idx;
      final_valid[o + p] = fv;
      if (attn_ids) attn_ids[o + p] = fv ? idx : -1;
    }
  };
  const int total = tile_off[n_tiles];
  // the compacted union in registers, C keys per thread
  auto compacted = [&](auto c) {
    constexpr int C = decltype(c)::value;
    using WU = WideSelect<C, false>;
    auto& shc = *reinterpret_cast<typename WU::Shared*>(&sh.c);
    WU wc;
    int tok[C];
    const float* crow = cscore + static_cast<int64_t>(row) * c_ld;
    const int32_t* trow = ctok + static_cast<int64_t>(row) * c_ld;
#pragma unroll
    for (int i = 0; i < C; ++i) {
      const int p = WU::pos(i);
      const bool ok = p < total;
      // the last tile whose list starts at or before p, in fixed steps
      // (so the C searches interleave instead of running one by one)
      int lo = 0;
#pragma unroll
      for (int step = kTileStep0; step > 0; step >>= 1) {
        const int mid = lo + step;
        lo = (mid < n_tiles && tile_off[min(mid, n_tiles)] <= p) ? mid : lo;
      }
      const int64_t e = static_cast<int64_t>(lo) * kScoreTile + (p - tile_off[lo]);
      tok[i] = ok ? trow[e] : 0;
      wc.set(i, ok ? crow[e] : 0.0f, ok);
    }
    int ninf = 0;
#pragma unroll
    for (int i = 0; i < C; ++i) wc.count(i, shc, ninf);
    wc.count_done(shc, ninf);
    write_protected();
    wc.run_counted(keep, shc);
    uint64_t fin = 0;
#pragma unroll
    for (int i = 0; i < C; ++i) fin |= static_cast<uint64_t>(isfinite(sortable_f32(wc.u[i]))) << i;
    wc.place_uniform(shc, [&](int, int p, int slot) { emit(tok[slot], p, (fin >> slot) & 1ull); });
  };
  // (uniform across the workgroup) a union of up to VPLC keys per thread, or
  // up to twice that (the block modes' unions) in the wider form
  if (cscore && n_fin >= keep && total <= VPLC * kWideNT) {
    compacted(std::integral_constant<int, VPLC>{});
  } else if (cscore && n_fin >= keep && total <= 2 * VPLC * kWideNT) {
    compacted(std::integral_constant<int, 2 * VPLC>{});
  } else {
    WS ws;
    ws.load_count(scores + static_cast<int64_t>(row) * scores_ld, history, sh.d);   // first digit counted on load
    ws.run_counted(keep, sh.d);
    write_protected();
    uint64_t fin = 0;   // bit i: key i is a finite score
#pragma unroll
    for (int i = 0; i < VPL; ++i) fin |= static_cast<uint64_t>(isfinite(sortable_f32(ws.u[i]))) << i;
    ws.place(sh.d, [&](int idx, int p, int slot) { emit(idx, p, (fin >> slot) & 1ull); });
  }
  const int extra = sink_end + n_rec + keep_self;
  const int list_at = expand ? body_cap : keep;   // where the protected entries go
  for (int i = tid; i < extra; i += kWideNT) {
    const int idx = i < sink_end ? i : (i < sink_end + n_rec ? rec_begin + (i - sink_end) : key_count - 1);
    if (staged) {
      ids_s[keep + i] = idx;
    } else {
      final_idx[o + list_at + i] = idx;
      final_valid[o + list_at + i] = 1;
      if (attn_ids) attn_ids[o + list_at + i] = idx;
    }
  }
  if (BITS || staged) __syncthreads();   // every emit is done (the selection's LDS is free)
  if constexpr (BITS) {
    if (expand) {
      // thread j of a round owns block j0 + j: tests the block's bits, fills
      // a hit block (LDS atomics: several blocks share a word, and a block's
      // bits are changed only by its own thread), and lists its positions
      // outside the protected ranges in ascending order (as reuse_expand_kernel)
      int* run_off = reinterpret_cast<int*>(&sh);
      int* run_lo = run_off + kWideNT;
      int* wave_tot = run_lo + kWideNT;
      const int lane = tid & 63, wave = tid >> 6;
      const int nblk = (history + xblock - 1) / xblock;
      int base = 0;
      for (int j0 = 0; j0 < nblk; j0 += kWideNT) {
        const int j = j0 + tid;
        int lo = 0, hi = 0;
        if (j < nblk) {
          const int b_lo = j * xblock, b_hi = min(b_lo + xblock, history);
          const int w_lo = b_lo >> 6, w_hi = (b_hi - 1) >> 6;
          uint64_t any = 0;
          for (int w = w_lo; w <= w_hi; ++w) any |= fin_s[w] & word_range_bits(w, b_lo, b_hi);
          if (any) {
            for (int w = w_lo; w <= w_hi; ++w) atomicOr(&fin_s[w], word_range_bits(w, b_lo, b_hi));
            lo = max(b_lo, sink_end);
            hi = min(b_hi, recent_start);
          }
        }
        const int cnt = hi > lo ? hi - lo : 0;
        const int incl = wave_incl_scan_dpp(cnt);
        run_off[tid] = incl - cnt;
        run_lo[tid] = lo;
        if (lane == 63) wave_tot[wave] = incl;
        __syncthreads();
        int wave_base = base, total = 0;
#pragma unroll
        for (int w = 0; w < kWideNT / 64; ++w) {
          const int x = wave_tot[w];
          wave_base += w < wave ? x : 0;
          total += x;
        }
        const int w64 = wave * 64, wave_cnt = wave_tot[wave];
        for (int q = lane; q < wave_cnt && wave_base + q < body_cap; q += 64) {
          int k = 0;   // the last lane whose run starts at or before q
#pragma unroll
          for (int step = 32; step > 0; step >>= 1) k += run_off[w64 + k + step] <= q ? step : 0;
          const int t = run_lo[w64 + k] + (q - run_off[w64 + k]);
          const int64_t e = o + wave_base + q;
          final_idx[e] = t;
          final_valid[e] = 1;
          if (attn_ids) attn_ids[e] = t;
        }
        base += total;
        __syncthreads();   // (run_off, wave_tot and the filled words before the next round and the store)
      }
      for (int p = min(base, body_cap) + tid; p < body_cap; p += kWideNT) {
        final_idx[o + p] = 0;
        final_valid[o + p] = 0;
        if (attn_ids) attn_ids[o + p] = -1;
      }
    }
  }
  if (staged) {
    for (int p = tid; p < n_out; p += kWideNT) {
      const int v = ids_s[p];
      final_idx[o + p] = v >= 0 ? v : ~v;
      final_valid[o + p] = v >= 0;
      if (attn_ids) attn_ids[o + p] = v >= 0 ? v : -1;
    }
  }
  if constexpr (BITS) {
    uint64_t* hw = reinterpret_cast<uint64_t*>(hrow);
    for (int j = tid; j < n_words; j += kWideNT) hw[j] = fin_s[j];
  }
  if constexpr (ATTN) reuse_attend<DT>(ids_s, n_out, at, row, sh.a);
}

// ---------------------------------------------------------------------------
// Block expansion of the final selection (the reuse...blk{bs} modes,
// EV:4314-4316 with EV:2914-2922) and the final index list re-read from the
// expanded mask (EV:2896-2911, 2938-2982).  One 1024-thread workgroup per
// row; thread j of a round owns block j0 + j: it ORs the block's flags
// (16-byte loads when the block is a multiple of 16 bytes and the row is
// aligned), fills a hit block with ones in place (a block without a set flag
// is already all zero), and counts the block's positions outside the
// protected ranges [0, sink_end) and [recent_start, history) from its span.
// A workgroup scan of the counts numbers the entries, so the body lists the
// expanded positions in ascending order; each wave then writes its share of
// the list with consecutive lanes on consecutive entries (an entry's owning
// thread found by a binary search over the wave's 64 run offsets in LDS).
// At most body_cap entries, padded with (0, invalid, -1); the sink range,
// the recent range and the current token follow.
// ---------------------------------------------------------------------------
constexpr int kExpandNT = 1024;
constexpr int kMaxExpandBlock = 4096;   // one thread scans a block

__global__ __launch_bounds__(kExpandNT) void reuse_expand_kernel(
    uint8_t* __restrict__ hf, int64_t hf_ld, int history, int block, int body_cap, int key_count, int sink_end,
    int recent_start, int rec_begin, int n_rec, int keep_self, int64_t* __restrict__ final_idx,
    uint8_t* __restrict__ final_valid, int32_t* __restrict__ attn_ids, int n_out) {
  __shared__ int wave_tot[kExpandNT / 64];
  __shared__ int run_off[kExpandNT], run_lo[kExpandNT];   // a thread's first entry within its wave, position
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  uint8_t* hrow = hf + static_cast<int64_t>(row) * hf_ld;
  const int64_t o = static_cast<int64_t>(row) * n_out;
  const bool vec = (block & 15) == 0 && (reinterpret_cast<uintptr_t>(hrow) & 15) == 0;
  const int nblk = static_cast<int>((static_cast<int64_t>(history) + block - 1) / block);
  int base = 0;   // body entries listed so far
  for (int j0 = 0; j0 < nblk; j0 += kExpandNT) {
    const int j = j0 + tid;
    int64_t lo = 0, hi = 0;   // the block's body positions [lo, hi) when it is hit
    if (j < nblk) {
      const int64_t b_lo = static_cast<int64_t>(j) * block;
      const int64_t b_hi = std::min<int64_t>(b_lo + block, history);
      bool any = false;
      if (vec && b_hi - b_lo == block) {
        uint32_t acc = 0;
        for (int64_t t = b_lo; t < b_hi; t += 16) {
          const uint4 w = *reinterpret_cast<const uint4*>(hrow + t);
          acc |= w.x | w.y | w.z | w.w;
        }
        any = acc != 0;
        if (any)
          for (int64_t t = b_lo; t < b_hi; t += 16)
            *reinterpret_cast<uint4*>(hrow + t) = make_uint4(0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u);
      } else {
        for (int64_t t = b_lo; t < b_hi; ++t) any |= hrow[t] != 0;
        if (any)
          for (int64_t t = b_lo; t < b_hi; ++t) hrow[t] = 1;
      }
      if (any) {
        lo = std::max<int64_t>(b_lo, sink_end);
        hi = std::min<int64_t>(b_hi, recent_start);
      }
    }
    const int cnt = hi > lo ? static_cast<int>(hi - lo) : 0;
    const int incl = wave_incl_scan_dpp(cnt);
    run_off[tid] = incl - cnt;
    run_lo[tid] = static_cast<int>(lo);
    if (lane == 63) wave_tot[wave] = incl;
    __syncthreads();
    int wave_base = base, total = 0;
#pragma unroll
    for (int w = 0; w < kExpandNT / 64; ++w) {
      const int x = wave_tot[w];
      wave_base += w < wave ? x : 0;
      total += x;
    }
    const int w64 = wave * 64, wave_cnt = wave_tot[wave];
    for (int q = lane; q < wave_cnt && wave_base + q < body_cap; q += 64) {
      int k = 0;   // the last lane whose run starts at or before q
#pragma unroll
      for (int step = 32; step > 0; step >>= 1) k += run_off[w64 + k + step] <= q ? step : 0;
      const int t = run_lo[w64 + k] + (q - run_off[w64 + k]);
      const int64_t e = o + wave_base + q;
      final_idx[e] = t;
      final_valid[e] = 1;
      if (attn_ids) attn_ids[e] = t;
    }
    base += total;
    __syncthreads();   // wave_tot is rewritten by the next round
  }
  for (int p = min(base, body_cap) + tid; p < body_cap; p += kExpandNT) {
    final_idx[o + p] = 0;
    final_valid[o + p] = 0;
    if (attn_ids) attn_ids[o + p] = -1;
  }
  const int extra = sink_end + n_rec + keep_self;
  for (int i = tid; i < extra; i += kExpandNT) {
    const int idx = i < sink_end ? i : (i < sink_end + n_rec ? rec_begin + (i - sink_end) : key_count - 1);
    final_idx[o + body_cap + i] = idx;
    final_valid[o + body_cap + i] = 1;
    if (attn_ids) attn_ids[o + body_cap + i] = idx;
  }
}

// reuse_expand_kernel on a bitset final selection (hf_ld words per row): a
// block's test reads its own bits, a hit block's bits are set by atomic OR
// (blocks of fewer than 64 positions, or not a multiple of 64, share words);
// the list is written as there.
__global__ __launch_bounds__(kExpandNT) void reuse_expand_bits_kernel(
    uint64_t* __restrict__ hf, int64_t hf_ld, int history, int block, int body_cap, int key_count, int sink_end,
    int recent_start, int rec_begin, int n_rec, int keep_self, int64_t* __restrict__ final_idx,
    uint8_t* __restrict__ final_valid, int32_t* __restrict__ attn_ids, int n_out) {
  __shared__ int wave_tot[kExpandNT / 64];
  __shared__ int run_off[kExpandNT], run_lo[kExpandNT];
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  uint64_t* hrow = hf + static_cast<int64_t>(row) * hf_ld;
  const int64_t o = static_cast<int64_t>(row) * n_out;
  const int nblk = static_cast<int>((static_cast<int64_t>(history) + block - 1) / block);
  int base = 0;
  for (int j0 = 0; j0 < nblk; j0 += kExpandNT) {
    const int j = j0 + tid;
    int lo = 0, hi = 0;
    if (j < nblk) {
      const int b_lo = j * block, b_hi = min(b_lo + block, history);
      const int w_lo = b_lo >> 6, w_hi = (b_hi - 1) >> 6;
      uint64_t any = 0;
      for (int w = w_lo; w <= w_hi; ++w) any |= hrow[w] & word_range_bits(w, b_lo, b_hi);
      if (any) {
        for (int w = w_lo; w <= w_hi; ++w) {
          const uint64_t m = word_range_bits(w, b_lo, b_hi);
          if (m == ~0ull) hrow[w] = m;   // a word of this block alone
          else atomicOr(reinterpret_cast<unsigned long long*>(hrow + w), m);
        }
        lo = max(b_lo, sink_end);
        hi = min(b_hi, recent_start);
      }
    }
    const int cnt = hi > lo ? hi - lo : 0;
    const int incl = wave_incl_scan_dpp(cnt);
    run_off[tid] = incl - cnt;
    run_lo[tid] = lo;
    if (lane == 63) wave_tot[wave] = incl;
    __syncthreads();
    int wave_base = base, total = 0;
#pragma unroll
    for (int w = 0; w < kExpandNT / 64; ++w) {
      const int x = wave_tot[w];
      wave_base += w < wave ? x : 0;
      total += x;
    }
    const int w64 = wave * 64, wave_cnt = wave_tot[wave];
    for (int q = lane; q < wave_cnt && wave_base + q < body_cap; q += 64) {
      int k = 0;   // the last lane whose run starts at or before q
#pragma unroll
      for (int step = 32; step > 0; step >>= 1) k += run_off[w64 + k + step] <= q ? step : 0;
      const int t = run_lo[w64 + k] + (q - run_off[w64 + k]);
      const int64_t e = o + wave_base + q;
      final_idx[e] = t;
      final_valid[e] = 1;
      if (attn_ids) attn_ids[e] = t;
    }
    base += total;
    __syncthreads();   // wave_tot is rewritten by the next round
  }
  for (int p = min(base, body_cap) + tid; p < body_cap; p += kExpandNT) {
    final_idx[o + p] = 0;
    final_valid[o + p] = 0;
    if (attn_ids) attn_ids[o + p] = -1;
  }
  const int extra = sink_end + n_rec + keep_self;
  for (int i = tid; i < extra; i += kExpandNT) {
    const int idx = i < sink_end ? i : (i < sink_end + n_rec ? rec_begin + (i - sink_end) : key_count - 1);
    final_idx[o + body_cap + i] = idx;
    final_valid[o + body_cap + i] = 1;
    if (attn_ids) attn_ids[o + body_cap + i] = idx;
  }
}

// VPL for a row of n values: 16, 32 or 40 (n <= kWideMax).
template <typename F>
int with_wide_vpl(int64_t n, F&& f) {
  if (n <= 16 * kWideNT) return f(std::integral_constant<int, 16>{});
  if (n <= 32 * kWideNT) return f(std::integral_constant<int, 32>{});
  return f(std::integral_constant<int, 40>{});
}

// ---------------------------------------------------------------------------
// Dim-major copy of K: kdm[b, j, d, t] = K[b, j, t, d] for t in [t0, t1),
// through a 32-token LDS tile (coalesced on both sides).
// ---------------------------------------------------------------------------
constexpr int kDmTile = 32;

template <int DT>
__global__ __launch_bounds__(kRT) void dim_major_kernel(const typename Elem<DT>::T* __restrict__ key, int kv_heads,
                                                         int head_dim, int t0, int t1, int64_t sb, int64_t sh,
                                                         int64_t st, typename Elem<DT>::T* __restrict__ kdm,
                                                         int64_t db, int64_t dh, int64_t dd) {
  using E = typename Elem<DT>::T;
  __shared__ E tile[kDmTile][DT == QKV_DTYPE_FP32 ? 257 : 513];   // head_dim <= 256 (fp32) / 512
  const int row = blockIdx.y, tid = threadIdx.x;
  const int b = row / kv_heads, j = row - b * kv_heads;
  const int tb = t0 + blockIdx.x * kDmTile;
  const int n = min(kDmTile, t1 - tb);
  const E* src = key + b * sb + j * sh;
  for (int e = tid; e < n * head_dim; e += kRT) {
    const int t = e / head_dim, d = e - t * head_dim;
    tile[t][d] = src[static_cast<int64_t>(tb + t) * st + d];
  }
  __syncthreads();
  E* dst = kdm + b * db + j * dh + tb;
  for (int e = tid; e < n * head_dim; e += kRT) {
    const int d = e / n, t = e - d * n;
    dst[d * dd + t] = tile[t][d];
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
struct ReuseCounts {
  int64_t keep, sink_end, recent_start, rec_begin, n_rec, n_out;
};

ReuseCounts reuse_counts(int64_t history, int64_t sink, int64_t recent, double top_fraction, int keep_self) {
  ReuseCounts c;
  c.keep = std::min<int64_t>(history, std::max<int64_t>(1, static_cast<int64_t>(ceil(top_fraction * history))));
  c.sink_end = sink > 0 ? std::min(sink, history) : 0;
  c.recent_start = recent > 0 ? std::max<int64_t>(0, history - recent) : history;
  c.rec_begin = std::max(c.recent_start, c.sink_end);
  c.n_rec = (recent > 0 && c.rec_begin < history) ? history - c.rec_begin : 0;
  c.n_out = c.keep + c.sink_end + c.n_rec + (keep_self ? 1 : 0);
  return c;
}

// Entries of the body of a block-expanded final list: the expanded
// selection outside the protected ranges [0, sink_end) and
// [recent_start, history).  Each of the keep selections adds at most one
// block, and the blocks that hold the ends of the two protected ranges add at
// most block - 1 positions each.
int64_t block_body_cap(const ReuseCounts& c, int64_t block) {
  const int64_t open = std::max<int64_t>(0, c.recent_start - c.sink_end);
  return std::min(open, c.keep * block + 2 * (block - 1));
}

constexpr int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

// Scores, selection, staged top-k workspace, then (rows the wide kernel
// selects in one workgroup) the compacted union lists and their counts.
int64_t reuse_compact_bytes(int64_t rows, int64_t history) {
  if (history > kWideMax) return 0;
  const int64_t slots = cdiv(history, kScoreTile) * kScoreTile;
  return 2 * align256(rows * slots * 4) + align256(rows * cdiv(history, kScoreTile) * 2 * 4);
}

int64_t reuse_ws_bytes(int64_t rows, int64_t history, int64_t keep) {
  const int64_t tk = qkv_topk_workspace_bytes(rows, history, keep);
  if (tk < 0) return -1;
  return align256(rows * history * 4) + align256(rows * keep * 4) + align256(tk) + reuse_compact_bytes(rows, history);
}

int64_t mask_ws_bytes(int64_t rows, int64_t n, int64_t k) {
  const int64_t tk = qkv_topk_workspace_bytes(rows, n, k);
  if (tk < 0) return -1;
  return align256(rows * k * 4) + align256(tk);
}

// hist (optional, [B * Hq, kCandBins] int, zero): every row's first-digit
// counts (reuse_partial_kernel's HIST).
template <int DT> struct RunReusePartial {
  static int run(const void* q, const void* kdm, const int64_t* ks, int64_t B, int64_t Hq, int64_t Hkv,
                 int64_t T, int64_t D, int count, float* out, int64_t out_ld, hipStream_t st,
                 const uint8_t* gate = nullptr, int gate_refresh = 0, int* hist = nullptr) {
    using E = typename Elem<DT>::T;
    const int64_t ev = DT == QKV_DTYPE_FP32 ? 4 : 8;   // elements per 16 bytes
    const bool vec = aligned(kdm, 16) && ks[0] % ev == 0 && ks[1] % ev == 0 && ks[2] % ev == 0;
    dim3 grid(static_cast<unsigned>(cdiv(T, 8 * kPartNT)), static_cast<unsigned>(B * Hq));
#define QKV_REUSE_PARTIAL(HH)                                                                                  \
  reuse_partial_kernel<DT, HH><<<grid, kPartNT, 0, st>>>(static_cast<const E*>(q), static_cast<const E*>(kdm),     \
                                                     static_cast<int>(Hq), static_cast<int>(Hq / Hkv),         \
                                                     static_cast<int>(T), static_cast<int>(D), count, ks[0],   \
                                                     ks[1], ks[2], vec, out, out_ld, gate, gate_refresh,       \
                                                     static_cast<int>(B * Hq), hist)
    if (hist) QKV_REUSE_PARTIAL(true);
    else QKV_REUSE_PARTIAL(false);
#undef QKV_REUSE_PARTIAL
    return check_launch("qkv_reuse_partial_scores");
  }
};

template <int DT> struct RunReuseScores {
  static int run(const void* q, const void* k, const int64_t* ks, int64_t B, int64_t Hq, int64_t Hkv, int64_t T,
                 int64_t D, const uint8_t* cur, const uint8_t* prev, const uint8_t* fin, int64_t mask_ld,
                 float scaling, float* out, int64_t out_ld, float* cscore, int32_t* ctok, int32_t* ccnt,
                 int64_t c_ld, hipStream_t st, bool bitsets = false) {
    using E = typename Elem<DT>::T;
    const int64_t ev = DT == QKV_DTYPE_FP32 ? 4 : 8;
    const bool kvec = ks[3] == 1 && D % 8 == 0 && aligned(k, 16) && ks[0] % ev == 0 && ks[1] % ev == 0 &&
                      ks[2] % ev == 0;
    const bool mvec = mask_ld % 4 == 0 && aligned(cur, 4) && (!prev || aligned(prev, 4)) && (!fin || aligned(fin, 4));
    dim3 grid(static_cast<unsigned>(cdiv(T, kScoreTile)), static_cast<unsigned>(B * Hq));
    if (ks[3] != 1) return fail(QKV_ERR_UNSUPPORTED, "qkv_reuse_select: K channels must be contiguous");
#define QKV_REUSE_SCORES(DF, BB)                                                                               \
  reuse_scores_kernel<DT, DF, BB><<<grid, kScoreNT, 0, st>>>(static_cast<const E*>(q), static_cast<const E*>(k),    \
                                                        static_cast<int>(Hq), static_cast<int>(Hq / Hkv),      \
                                                        static_cast<int>(T), static_cast<int>(D), ks[0], ks[1], \
                                                        ks[2], kvec, cur, prev, fin, mask_ld, mvec, scaling, out, \
                                                        out_ld, cscore, ctok, ccnt, c_ld)
    if (bitsets) {
      if (kvec && D == 128) QKV_REUSE_SCORES(128, true);
      else QKV_REUSE_SCORES(0, true);
    } else {
      if (kvec && D == 128) QKV_REUSE_SCORES(128, false);
      else QKV_REUSE_SCORES(0, false);
    }
#undef QKV_REUSE_SCORES
    return check_launch("qkv_reuse_select");
  }
};

template <int DT> struct RunDimMajor2 {
  static int run(const void* k, const int64_t* ks, int64_t B, int64_t Hkv, int64_t D, int64_t t0, int64_t t1,
                 void* kdm, const int64_t* ds, hipStream_t st) {
    using E = typename Elem<DT>::T;
    dim3 grid(static_cast<unsigned>(cdiv(t1 - t0, kDmTile)), static_cast<unsigned>(B * Hkv));
    dim_major_kernel<DT><<<grid, kRT, 0, st>>>(static_cast<const E*>(k), static_cast<int>(Hkv), static_cast<int>(D),
                                               static_cast<int>(t0), static_cast<int>(t1), ks[0], ks[1], ks[2],
                                               static_cast<E*>(kdm), ds[0], ds[1], ds[2]);
    return check_launch("qkv_dim_major_append");
  }
};

int check_heads(const char* what, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim) {
  if (batch <= 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads)
    return fail(QKV_ERR_INVALID, "%s: need batch > 0 and q_heads a positive multiple of kv_heads", what);
  if (batch * q_heads > 65535) return fail(QKV_ERR_INVALID, "%s: batch * q_heads must be <= 65535", what);
  if (head_dim <= 0 || head_dim > 512) return fail(QKV_ERR_UNSUPPORTED, "%s: head_dim must be in [1, 512]", what);
  return QKV_OK;
}

// mask = values >= the row's k-th largest (threshold to thr_out when given);
// with bits (mask null) the mask is written as a bitset instead.
int threshold_mask_impl(const char* what, const float* values, int64_t rows, int64_t n, int64_t ld, int64_t k,
                        uint8_t* mask, int64_t mask_ld, float* thr_out, void* workspace, int64_t workspace_bytes,
                        hipStream_t st, const uint8_t* gate = nullptr, int gate_refresh = 0,
                        uint64_t* bits = nullptr, int64_t bits_ld = 0) {
  if (n <= kWideMax) {   // (rows past the one-workgroup length are selected whatever the gate says)
    return with_wide_vpl(n, [&](auto vpl) {
      reuse_mask_wide_kernel<decltype(vpl)::value><<<static_cast<unsigned>(rows), kWideNT, 0, st>>>(
          values, ld, static_cast<int>(n), static_cast<int>(k), mask, mask_ld, thr_out, gate, gate_refresh,
          static_cast<int>(rows), bits, bits_ld);
      return check_launch(what);
    });
  }
  int32_t* sel = static_cast<int32_t*>(workspace);
  void* tk_ws = static_cast<char*>(workspace) + align256(rows * k * 4);
  int rc = qkv_topk_ws(values, rows, n, ld, k, sel, tk_ws, workspace_bytes - align256(rows * k * 4), st);
  if (rc) return rc;
  if (bits) {
    dim3 grid(static_cast<unsigned>(cdiv(n, kRT * 4)), static_cast<unsigned>(rows));
    reuse_mask_bits_kernel<<<grid, kRT, 0, st>>>(values, ld, static_cast<int>(n), sel, static_cast<int>(k), nullptr,
                                                 bits, bits_ld, thr_out);
    return check_launch(what);
  }
  const bool vec = ld % 4 == 0 && aligned(values, 16) && mask_ld % 16 == 0 && aligned(mask, 16);
  dim3 grid(static_cast<unsigned>(cdiv(n, kMaskTile)), static_cast<unsigned>(rows));
  reuse_mask_kernel<<<grid, kRT, 0, st>>>(values, ld, static_cast<int>(n), sel, static_cast<int>(k), nullptr, mask,
                                          mask_ld, vec, thr_out);
  return check_launch(what);
}

constexpr int64_t kFusedCandRows = 128;

// The state of the cross-workgroup candidate selection at the start of a
// candidates workspace: per row the first-digit histogram (kCandBins ints),
// then per row the slices' list counts and the ticket (kCandState ints);
// the histograms and tickets are zero between calls.
int64_t cand_state_bytes(int64_t rows) { return align256(rows * kCandBins * 4) + align256(rows * kCandState * 4); }

// The rest of the workspace: the boundary-bin lists (a score and a position
// per history token and row) or, on the other paths, qkv_threshold_mask's.
int64_t cand_scratch_bytes(int64_t rows, int64_t n, int64_t k) {
  const int64_t m = mask_ws_bytes(rows, n, k);
  return m < 0 ? -1 : std::max(m, 2 * align256(rows * n * 4));
}

struct CandSplit {
  int* hist = nullptr;   // null: the selection runs one workgroup per row
  int* state = nullptr;
  float* list_val = nullptr;
  int* list_pos = nullptr;
};

// reuse_cand_slices_kernel over rows x slices workgroups: J scores per
// thread, the smallest J that keeps the grid within QKV_CAND_TARGET_WGS
// workgroups.  Measured at 32 rows x 32792 scores (graph step, us/layer):
// 288 workgroups of J = 4 51.6, 160 of J = 8 50.3-50.8, 96 of J = 16 52.0,
// 64 of J = 32 56.0.
#ifndef QKV_CAND_TARGET_WGS
#define QKV_CAND_TARGET_WGS 256
#endif
int launch_cand_slices(const char* what, const float* values, int64_t ld, int64_t rows, int64_t n, int64_t k,
                       const CandSplit& cs, uint64_t* bits, int64_t bits_ld, float* thr_out, hipStream_t st,
                       const uint8_t* gate = nullptr, int refresh = 0) {
  auto launch = [&](auto jc) {
    constexpr int J = decltype(jc)::value;
    const int64_t slices = cdiv(n, int64_t(kWideNT) * J);
    reuse_cand_slices_kernel<J><<<static_cast<unsigned>(rows * slices), kWideNT, 0, st>>>(
        values, ld, static_cast<int>(n), static_cast<int>(k), static_cast<int>(slices), cs.hist, cs.state,
        cs.list_val, cs.list_pos, n, bits, bits_ld, thr_out, QabsListOut{}, gate, refresh, static_cast<int>(rows));
    return check_launch(what);
  };
  auto wgs = [&](int64_t j) { return rows * cdiv(n, int64_t(kWideNT) * j); };
  if (wgs(1) <= QKV_CAND_TARGET_WGS) return launch(std::integral_constant<int, 1>{});
  if (wgs(2) <= QKV_CAND_TARGET_WGS) return launch(std::integral_constant<int, 2>{});
  if (wgs(4) <= QKV_CAND_TARGET_WGS) return launch(std::integral_constant<int, 4>{});
  if (wgs(8) <= QKV_CAND_TARGET_WGS) return launch(std::integral_constant<int, 8>{});
  if (wgs(16) <= QKV_CAND_TARGET_WGS) return launch(std::integral_constant<int, 16>{});
  return launch(std::integral_constant<int, 32>{});
}

// reuse_cand_slices_kernel<J, true>: the exact-candidate attention's final
// list across slices (J as launch_cand_slices picks it); bits / nf: the
// above-bin and non-finite words, bits_ld words per row.
int launch_qabs_slices(const char* what, const float* values, int64_t ld, int64_t rows, int64_t n, int64_t keep,
                       const CandSplit& cs, uint64_t* bits, int64_t bits_ld, const QabsListOut& qs, hipStream_t st) {
  auto launch = [&](auto jc) {
    constexpr int J = decltype(jc)::value;
    const int64_t slices = cdiv(n, int64_t(kWideNT) * J);
    reuse_cand_slices_kernel<J, true><<<static_cast<unsigned>(rows * slices), kWideNT, 0, st>>>(
        values, ld, static_cast<int>(n), static_cast<int>(keep), static_cast<int>(slices), cs.hist, cs.state,
        cs.list_val, cs.list_pos, n, bits, bits_ld, nullptr, qs);
    return check_launch(what);
  };
  auto wgs = [&](int64_t j) { return rows * cdiv(n, int64_t(kWideNT) * j); };
  if (wgs(1) <= QKV_CAND_TARGET_WGS) return launch(std::integral_constant<int, 1>{});
  if (wgs(2) <= QKV_CAND_TARGET_WGS) return launch(std::integral_constant<int, 2>{});
  if (wgs(4) <= QKV_CAND_TARGET_WGS) return launch(std::integral_constant<int, 4>{});
  if (wgs(8) <= QKV_CAND_TARGET_WGS) return launch(std::integral_constant<int, 8>{});
  if (wgs(16) <= QKV_CAND_TARGET_WGS) return launch(std::integral_constant<int, 16>{});
  return launch(std::integral_constant<int, 32>{});
}

// The split selection's part of a qkv_qabs_candidates workspace after its
// state: the boundary-bin lists, then the above-bin and non-finite words.
int64_t qabs_split_bytes(int64_t rows, int64_t history) {
  return 2 * align256(rows * history * 4) + 2 * align256(rows * cdiv(history, 64) * 8);
}

template <int DT> struct RunCandidates {
  static int run(const char* what, const void* q, const void* kdm, const int64_t* ks, int64_t B, int64_t Hq,
                 int64_t Hkv, int64_t T, int64_t D, int count, int64_t k, float* partial, int64_t partial_ld,
                 uint8_t* mask, int64_t mask_ld, float* thr_out, void* workspace, int64_t workspace_bytes,
                 hipStream_t st, const uint8_t* gate, int refresh, uint64_t* bits = nullptr,
                 int64_t bits_ld = 0, const CandSplit& split = CandSplit{}) {
    using E = typename Elem<DT>::T;
    const int64_t ev = DT == QKV_DTYPE_FP32 ? 4 : 8;   // elements per 16 bytes
    const bool vec = aligned(kdm, 16) && ks[0] % ev == 0 && ks[1] % ev == 0 && ks[2] % ev == 0;
    const int64_t rows = B * Hq;
    // One launch pays off once the rows fill the GPU: measured at 32768 tokens,
    // 32 rows took 27.1 us fused against 26.3 us for the two launches (and more
    // inside a decode step, where the copy's rows come from HBM), 128 rows 31.1
    // against 41.1 us, 256 rows 40.4 against 58.1 us.
    if (vec && T <= kWideMax && D <= 128 && rows >= kFusedCandRows) {
      auto launch = [&](auto nch) {
        reuse_candidates_kernel<DT, decltype(nch)::value><<<static_cast<unsigned>(rows), kWideNT, 0, st>>>(
            static_cast<const E*>(q), static_cast<const E*>(kdm), static_cast<int>(Hq), static_cast<int>(Hq / Hkv),
            static_cast<int>(T), static_cast<int>(D), count, ks[0], ks[1], ks[2], partial, partial_ld,
            static_cast<int>(k), mask, mask_ld, thr_out, gate, refresh, static_cast<int>(rows), bits, bits_ld);
        return check_launch(what);
      };
      const int64_t per = 8 * kWideNT;   // tokens per chunk
      if (T <= per) return launch(std::integral_constant<int, 1>{});
      if (T <= 2 * per) return launch(std::integral_constant<int, 2>{});
      if (T <= 3 * per) return launch(std::integral_constant<int, 3>{});
      if (T <= 4 * per) return launch(std::integral_constant<int, 4>{});
      return launch(std::integral_constant<int, 5>{});
    }
    if (split.hist && bits && T <= kWideMax) {
      // the partial scores count the first digit; several workgroups per row select
      // (gate: the rows that keep no new candidates skip both launches)
      int rc = RunReusePartial<DT>::run(q, kdm, ks, B, Hq, Hkv, T, D, count, partial, partial_ld, st, gate, refresh,
                                        split.hist);
      if (rc) return rc;
      return launch_cand_slices(what, partial, partial_ld, rows, T, k, split, bits, bits_ld, thr_out, st, gate,
                                refresh);
    }
    int rc = RunReusePartial<DT>::run(q, kdm, ks, B, Hq, Hkv, T, D, count, partial, partial_ld, st, gate, refresh);
    if (rc) return rc;
    return threshold_mask_impl(what, partial, rows, T, partial_ld, k, mask, mask_ld, thr_out, workspace,
                               workspace_bytes, st, gate, refresh, bits, bits_ld);
  }
};

}  // namespace
}  // namespace qkv

using namespace qkv;

QKV_EXPORT int64_t qkv_reuse_final_count(int64_t history, int64_t protect_sink, int64_t protect_recent,
                                         double top_fraction, int keep_self) {
  if (history <= 0) return -1;
  return reuse_counts(history, protect_sink, protect_recent, top_fraction, keep_self).n_out;
}

QKV_EXPORT int64_t qkv_reuse_select_workspace_bytes(int64_t rows, int64_t history, double top_fraction) {
  if (rows <= 0 || history <= 0 || history >= (int64_t(1) << 31)) return -1;
  return reuse_ws_bytes(rows, history, reuse_counts(history, 0, 0, top_fraction, 0).keep);
}

namespace {

int reuse_select_impl(const char* what, bool bits, const void* query, const void* key, const int64_t* k_strides,
                      int dtype, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t key_count,
                      int64_t head_dim, const uint8_t* current, const uint8_t* previous,
                      const uint8_t* previous_final, int64_t mask_ld, int64_t protect_sink, int64_t protect_recent,
                      double top_fraction, int keep_self, float scaling, void* workspace, int64_t workspace_bytes,
                      int64_t* final_indices, uint8_t* final_valid, int32_t* attn_ids, int64_t n_out,
                      uint8_t* history_final, int64_t history_final_ld, void* stream, const void* value = nullptr,
                      void* out = nullptr, int* attended = nullptr, int64_t xblock = 0) {
  int rc = check_heads(what, batch, q_heads, kv_heads, head_dim);
  if (rc) return rc;
  if (!query || !key || !k_strides || !current || !workspace || !final_indices || !final_valid || !history_final)
    return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  const int64_t history = key_count - 1;
  if (history <= 0 || key_count >= (int64_t(1) << 31))
    return fail(QKV_ERR_INVALID, "%s: need 2 <= key_count < 2^31 (history excludes the current token)", what);
  const int64_t cover = bits ? cdiv(history, 64) : history;   // words or bytes per row
  if (mask_ld < cover || history_final_ld < cover)
    return fail(QKV_ERR_INVALID, "%s: mask row strides must cover the history", what);
  if (bits && (!aligned(current, 8) || !aligned(previous, 8) || !aligned(previous_final, 8) ||
               !aligned(history_final, 8)))
    return fail(QKV_ERR_INVALID, "%s: bitsets must be 8-byte aligned", what);
  if (!(top_fraction >= 0.0)) return fail(QKV_ERR_INVALID, "%s: top_fraction must be >= 0", what);
  const ReuseCounts c = reuse_counts(history, protect_sink, protect_recent, top_fraction, keep_self);
  int64_t body_cap = 0;
  if (xblock) {   // the block expansion in the final selection's launch (bitsets of rows up to kWideMax)
    if (xblock < 1 || xblock > kMaxExpandBlock)
      return fail(QKV_ERR_INVALID, "%s: block must be in [1, %d]", what, kMaxExpandBlock);
    if (!bits || history > kWideMax)
      return fail(QKV_ERR_UNSUPPORTED, "%s: the expansion runs on bitsets of at most %d history tokens", what,
                  kWideMax);
    body_cap = block_body_cap(c, xblock);
    const int64_t need_out = body_cap + c.sink_end + c.n_rec + (keep_self ? 1 : 0);
    if (n_out != need_out)
      return fail(QKV_ERR_INVALID, "%s: index rows hold %lld entries, the expanded selection needs %lld", what,
                  (long long)n_out, (long long)need_out);
  } else if (n_out != c.n_out) {
    return fail(QKV_ERR_INVALID, "%s: index rows hold %lld entries, the selection needs %lld", what,
                (long long)n_out, (long long)c.n_out);
  }
  const int64_t rows = batch * q_heads;
  const int64_t need = reuse_ws_bytes(rows, history, c.keep);
  if (need < 0 || workspace_bytes < need)
    return fail(QKV_ERR_INVALID, "%s: workspace needs %lld bytes, got %lld", what, (long long)need,
                (long long)workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  float* scores = reinterpret_cast<float*>(ws);
  int64_t off = align256(rows * history * 4);
  int32_t* sel = reinterpret_cast<int32_t*>(ws + off);
  off += align256(rows * c.keep * 4);
  void* tk_ws = ws + off;
  const int64_t tk_bytes = align256(qkv_topk_workspace_bytes(rows, history, c.keep));
  off += tk_bytes;
  const bool wide = history <= kWideMax;
  const int64_t n_tiles = cdiv(history, kScoreTile), c_ld = n_tiles * kScoreTile;
  float* cscore = wide ? reinterpret_cast<float*>(ws + off) : nullptr;
  int32_t* ctok = wide ? reinterpret_cast<int32_t*>(ws + off + align256(rows * c_ld * 4)) : nullptr;
  int32_t* ccnt = wide ? reinterpret_cast<int32_t*>(ws + off + 2 * align256(rows * c_ld * 4)) : nullptr;

  rc = dispatch_dtype<RunReuseScores>(dtype, query, key, k_strides, batch, q_heads, kv_heads, history, head_dim,
                                      current, previous, previous_final, mask_ld, scaling, scores, history, cscore,
                                      ctok, ccnt, c_ld, st, bits);
  if (rc) return rc;
  // the final selection's workgroup also attends over the row's list (one launch less) where it
  // holds the list: 16-bit K/V rows of 128 channels, 16-byte aligned, V laid out as K
  const bool fuse = !xblock && out && value && bits && wide && n_out <= kAttnList && head_dim == 128 &&
                    (dtype == QKV_DTYPE_BF16 || dtype == QKV_DTYPE_FP16) && k_strides[3] == 1 &&
                    aligned(key, 16) && aligned(value, 16) && aligned(query, 16) && aligned(out, 16) &&
                    (k_strides[0] | k_strides[1] | k_strides[2]) % 8 == 0;
  if (attended) *attended = fuse ? 1 : 0;
  if (wide) {
    // compacted unions of up to 1/8 of the row's width (at least 2048 entries), or twice that
    return with_wide_vpl(history, [&](auto vpl) {
      constexpr int VPL = decltype(vpl)::value;
      constexpr int VPLC = VPL / 8 > 2 ? VPL / 8 : 2;
      const ReuseAttn at{static_cast<const uint16_t*>(query), static_cast<const uint16_t*>(key),
                         static_cast<const uint16_t*>(value), k_strides[0], k_strides[1], k_strides[2],
                         static_cast<int>(q_heads), static_cast<int>(q_heads / kv_heads),
                         scaling * 1.4426950408889634f, static_cast<uint16_t*>(out)};
      auto launch = [&](auto bb, auto dt, auto attn) {
        reuse_final_wide_kernel<VPL, VPLC, decltype(bb)::value, decltype(dt)::value, decltype(attn)::value>
            <<<static_cast<unsigned>(rows), kWideNT, 0, st>>>(
                scores, history, cscore, ctok, ccnt, static_cast<int>(n_tiles), c_ld, static_cast<int>(c.keep),
                static_cast<int>(history), static_cast<int>(key_count),
                static_cast<int>(c.sink_end), static_cast<int>(c.recent_start), static_cast<int>(c.rec_begin),
                static_cast<int>(c.n_rec), keep_self ? 1 : 0, final_indices, final_valid, attn_ids,
                static_cast<int>(n_out), history_final, history_final_ld, 0, at, static_cast<int>(xblock),
                static_cast<int>(body_cap));
        return check_launch(what);
      };
      using BF = std::integral_constant<int, QKV_DTYPE_BF16>;
      using FH = std::integral_constant<int, QKV_DTYPE_FP16>;
      if (fuse) {
        if (dtype == QKV_DTYPE_FP16) return launch(std::true_type{}, FH{}, std::true_type{});
        return launch(std::true_type{}, BF{}, std::true_type{});
      }
      return bits ? launch(std::true_type{}, BF{}, std::false_type{})
                  : launch(std::false_type{}, BF{}, std::false_type{});
    });
  }
  rc = qkv_topk_ws(scores, rows, history, history, c.keep, sel, tk_ws, tk_bytes, stream);
  if (rc) return rc;
  auto fin = [&](auto bb) {
    reuse_finalize_kernel<decltype(bb)::value><<<static_cast<unsigned>(rows), kRT, 0, st>>>(
        scores, history, sel, static_cast<int>(c.keep), static_cast<int>(history), static_cast<int>(key_count),
        static_cast<int>(c.sink_end), static_cast<int>(c.recent_start), static_cast<int>(c.rec_begin),
        static_cast<int>(c.n_rec), keep_self ? 1 : 0, final_indices, final_valid, attn_ids, static_cast<int>(n_out),
        history_final, history_final_ld);
    return check_launch(what);
  };
  return bits ? fin(std::true_type{}) : fin(std::false_type{});
}

}  // namespace

QKV_EXPORT int qkv_reuse_select(const void* query, const void* key, const int64_t* k_strides, int dtype,
                                int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t key_count,
                                int64_t head_dim, const uint8_t* current, const uint8_t* previous,
                                const uint8_t* previous_final, int64_t mask_ld, int64_t protect_sink,
                                int64_t protect_recent, double top_fraction, int keep_self, float scaling,
                                void* workspace, int64_t workspace_bytes, int64_t* final_indices,
                                uint8_t* final_valid, int32_t* attn_ids, int64_t n_out, uint8_t* history_final,
                                int64_t history_final_ld, void* stream) {
  return reuse_select_impl("qkv_reuse_select", false, query, key, k_strides, dtype, batch, q_heads, kv_heads,
                           key_count, head_dim, current, previous, previous_final, mask_ld, protect_sink,
                           protect_recent, top_fraction, keep_self, scaling, workspace, workspace_bytes,
                           final_indices, final_valid, attn_ids, n_out, history_final, history_final_ld, stream);
}

QKV_EXPORT int qkv_reuse_select_bits(const void* query, const void* key, const int64_t* k_strides, int dtype,
                                     int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t key_count,
                                     int64_t head_dim, const uint64_t* current, const uint64_t* previous,
                                     const uint64_t* previous_final, int64_t words_ld, int64_t protect_sink,
                                     int64_t protect_recent, double top_fraction, int keep_self, float scaling,
                                     void* workspace, int64_t workspace_bytes, int64_t* final_indices,
                                     uint8_t* final_valid, int32_t* attn_ids, int64_t n_out,
                                     uint64_t* history_final, int64_t history_final_ld, const void* value, void* out,
                                     int* attended, void* stream) {
  if (attended) *attended = 0;
  return reuse_select_impl("qkv_reuse_select_bits", true, query, key, k_strides, dtype, batch, q_heads, kv_heads,
                           key_count, head_dim, reinterpret_cast<const uint8_t*>(current),
                           reinterpret_cast<const uint8_t*>(previous), reinterpret_cast<const uint8_t*>(previous_final),
                           words_ld, protect_sink, protect_recent, top_fraction, keep_self, scaling, workspace,
                           workspace_bytes, final_indices, final_valid, attn_ids, n_out,
                           reinterpret_cast<uint8_t*>(history_final), history_final_ld, stream, value, out, attended);
}

QKV_EXPORT int qkv_reuse_select_bits_blocks(const void* query, const void* key, const int64_t* k_strides, int dtype,
                                            int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t key_count,
                                            int64_t head_dim, const uint64_t* current, const uint64_t* previous,
                                            const uint64_t* previous_final, int64_t words_ld, int64_t protect_sink,
                                            int64_t protect_recent, double top_fraction, int keep_self,
                                            float scaling, int64_t block, void* workspace, int64_t workspace_bytes,
                                            int64_t* final_indices, uint8_t* final_valid, int32_t* attn_ids,
                                            int64_t n_out, uint64_t* history_final, int64_t history_final_ld,
                                            void* stream) {
  if (block < 1) return fail(QKV_ERR_INVALID, "qkv_reuse_select_bits_blocks: block must be >= 1");
  return reuse_select_impl("qkv_reuse_select_bits_blocks", true, query, key, k_strides, dtype, batch, q_heads,
                           kv_heads, key_count, head_dim, reinterpret_cast<const uint8_t*>(current),
                           reinterpret_cast<const uint8_t*>(previous), reinterpret_cast<const uint8_t*>(previous_final),
                           words_ld, protect_sink, protect_recent, top_fraction, keep_self, scaling, workspace,
                           workspace_bytes, final_indices, final_valid, attn_ids, n_out,
                           reinterpret_cast<uint8_t*>(history_final), history_final_ld, stream, nullptr, nullptr,
                           nullptr, block);
}

QKV_EXPORT int64_t qkv_qabs_candidate_select_workspace_bytes(int64_t rows, int64_t history,
                                                            double candidate_fraction) {
  if (rows <= 0 || history <= 0 || history >= (int64_t(1) << 31) || !(candidate_fraction >= 0.0)) return -1;
  if (history <= kWideMax) return 0;   // one workgroup per row: no workspace
  return mask_ws_bytes(rows, history, reuse_counts(history, 0, 0, candidate_fraction, 0).keep);
}

QKV_EXPORT int qkv_qabs_candidate_select(const float* scores, int64_t rows, int64_t key_count, int64_t scores_ld,
                                         double candidate_fraction, int64_t protect_sink, int64_t protect_recent,
                                         int keep_self, int append, void* workspace, int64_t workspace_bytes,
                                         int64_t* final_indices, uint8_t* final_valid, int32_t* attn_ids,
                                         int64_t n_out, uint8_t* history_final, int64_t history_final_ld,
                                         void* stream) {
  const char* what = "qkv_qabs_candidate_select";
  if (!scores || !final_indices || !final_valid || !history_final) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  const int64_t history = key_count - 1;
  if (rows <= 0 || rows > 65535 || history <= 0 || key_count >= (int64_t(1) << 31))
    return fail(QKV_ERR_INVALID, "%s: need 0 < rows <= 65535 and 2 <= key_count < 2^31", what);
  if (scores_ld < history || history_final_ld < history)
    return fail(QKV_ERR_INVALID, "%s: row strides must cover the history", what);
  if (!(candidate_fraction >= 0.0)) return fail(QKV_ERR_INVALID, "%s: candidate_fraction must be >= 0", what);
  const ReuseCounts c = reuse_counts(history, protect_sink, protect_recent, candidate_fraction, keep_self);
  if (n_out != c.n_out)
    return fail(QKV_ERR_INVALID, "%s: index rows hold %lld entries, the selection needs %lld", what,
                (long long)n_out, (long long)c.n_out);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (history <= kWideMax) {   // the whole row in one workgroup
    return with_wide_vpl(history, [&](auto vpl) {
      constexpr int VPL = decltype(vpl)::value;
      reuse_final_wide_kernel<VPL, 2><<<static_cast<unsigned>(rows), kWideNT, 0, st>>>(
          scores, scores_ld, nullptr, nullptr, nullptr, 0, 0, static_cast<int>(c.keep), static_cast<int>(history),
          static_cast<int>(key_count), static_cast<int>(c.sink_end), static_cast<int>(c.recent_start),
          static_cast<int>(c.rec_begin), static_cast<int>(c.n_rec), keep_self ? 1 : 0, final_indices, final_valid,
          attn_ids, static_cast<int>(n_out), history_final, history_final_ld, append ? 1 : 0);
      return check_launch(what);
    });
  }
  const int64_t need = mask_ws_bytes(rows, history, c.keep);
  if (!workspace || need < 0 || workspace_bytes < need)
    return fail(QKV_ERR_INVALID, "%s: workspace needs %lld bytes, got %lld", what, (long long)need,
                (long long)workspace_bytes);
  int32_t* sel = static_cast<int32_t*>(workspace);
  void* tk_ws = static_cast<char*>(workspace) + align256(rows * c.keep * 4);
  int rc = qkv_topk_ws(scores, rows, history, scores_ld, c.keep, sel, tk_ws,
                       workspace_bytes - align256(rows * c.keep * 4), stream);
  if (rc) return rc;
  reuse_finalize_kernel<<<static_cast<unsigned>(rows), kRT, 0, st>>>(
      scores, scores_ld, sel, static_cast<int>(c.keep), static_cast<int>(history), static_cast<int>(key_count),
      static_cast<int>(c.sink_end), static_cast<int>(c.recent_start), static_cast<int>(c.rec_begin),
      static_cast<int>(c.n_rec), keep_self ? 1 : 0, final_indices, final_valid, attn_ids, static_cast<int>(n_out),
      history_final, history_final_ld, append ? 1 : 0);
  return check_launch(what);
}

QKV_EXPORT int64_t qkv_qabs_candidates_workspace_bytes(int64_t rows, int64_t history, double candidate_fraction) {
  const int64_t old = qkv_qabs_candidate_select_workspace_bytes(rows, history, candidate_fraction);
  if (old < 0) return -1;
  const int64_t split = history <= kWideMax ? qabs_split_bytes(rows, history) : 0;
  return cand_state_bytes(rows) + std::max(old, split);
}

QKV_EXPORT int qkv_qabs_candidates(const void* query, const void* key_dim_major, const int64_t* kdm_strides, int dtype,
                                   int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t key_count,
                                   int64_t head_dim, int64_t dim_count, double candidate_fraction,
                                   int64_t protect_sink, int64_t protect_recent, int keep_self, int append,
                                   float* partial, int64_t partial_ld, void* workspace, int64_t workspace_bytes,
                                   int64_t* final_indices, uint8_t* final_valid, int32_t* attn_ids, int64_t n_out,
                                   uint8_t* history_final, int64_t history_final_ld, void* stream) {
  const char* what = "qkv_qabs_candidates";
  int rc = check_heads(what, batch, q_heads, kv_heads, head_dim);
  if (rc) return rc;
  if (!query || !key_dim_major || !kdm_strides || !partial || !workspace || !final_indices || !final_valid ||
      !history_final)
    return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  const int64_t history = key_count - 1;
  if (history <= 0 || key_count >= (int64_t(1) << 31) || partial_ld < history || history_final_ld < history)
    return fail(QKV_ERR_INVALID, "%s: need 2 <= key_count < 2^31 and row strides covering the history", what);
  if (kdm_strides[3] != 1) return fail(QKV_ERR_UNSUPPORTED, "%s: the token axis of K must be contiguous", what);
  if (!(candidate_fraction >= 0.0)) return fail(QKV_ERR_INVALID, "%s: candidate_fraction must be >= 0", what);
  if (protect_sink < 0 || protect_recent < 0) return fail(QKV_ERR_INVALID, "%s: negative protection", what);
  const int64_t rows = batch * q_heads;
  const ReuseCounts c = reuse_counts(history, protect_sink, protect_recent, candidate_fraction, keep_self);
  if (n_out != c.n_out)
    return fail(QKV_ERR_INVALID, "%s: index rows hold %lld entries, the selection needs %lld", what,
                (long long)n_out, (long long)c.n_out);
  const int64_t need = qkv_qabs_candidates_workspace_bytes(rows, history, candidate_fraction);
  if (need < 0 || workspace_bytes < need)
    return fail(QKV_ERR_INVALID, "%s: workspace needs %lld bytes, got %lld", what, (long long)need,
                (long long)workspace_bytes);
  if (!aligned(workspace, 16)) return fail(QKV_ERR_INVALID, "%s: the workspace must be 16-byte aligned", what);
  const int count = static_cast<int>(std::min<int64_t>(std::max<int64_t>(dim_count, 1),
                                                       std::min<int64_t>(head_dim, kMaxDims)));
  hipStream_t st = static_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  const int64_t state = cand_state_bytes(rows);
  if (history > kWideMax || rows >= kFusedCandRows) {   // the partial scores, then qkv_qabs_candidate_select
    rc = dispatch_dtype<RunReusePartial>(dtype, query, key_dim_major, kdm_strides, batch, q_heads, kv_heads, history,
                                         head_dim, count, partial, partial_ld, st);
    if (rc) return rc;
    return qkv_qabs_candidate_select(partial, rows, key_count, partial_ld, candidate_fraction, protect_sink,
                                     protect_recent, keep_self, append, ws + state, workspace_bytes - state,
                                     final_indices, final_valid, attn_ids, n_out, history_final, history_final_ld,
                                     stream);
  }
  CandSplit split;
  split.hist = reinterpret_cast<int*>(ws);
  split.state = reinterpret_cast<int*>(ws + align256(rows * kCandBins * 4));
  split.list_val = reinterpret_cast<float*>(ws + state);
  split.list_pos = reinterpret_cast<int*>(ws + state + align256(rows * history * 4));
  const int64_t n_words = cdiv(history, 64);
  uint64_t* words = reinterpret_cast<uint64_t*>(ws + state + 2 * align256(rows * history * 4));
  uint64_t* nf = reinterpret_cast<uint64_t*>(reinterpret_cast<char*>(words) + align256(rows * n_words * 8));
  rc = dispatch_dtype<RunReusePartial>(dtype, query, key_dim_major, kdm_strides, batch, q_heads, kv_heads, history,
                                       head_dim, count, partial, partial_ld, st, nullptr, 0, split.hist);
  if (rc) return rc;
  QabsListOut qs;
  qs.nf = nf;
  qs.final_idx = final_indices;
  qs.final_valid = final_valid;
  qs.attn_ids = attn_ids;
  qs.n_out = static_cast<int>(n_out);
  qs.hf = history_final;
  qs.hf_ld = history_final_ld;
  qs.key_count = static_cast<int>(key_count);
  qs.sink_end = static_cast<int>(c.sink_end);
  qs.recent_start = static_cast<int>(c.recent_start);
  qs.rec_begin = static_cast<int>(c.rec_begin);
  qs.n_rec = static_cast<int>(c.n_rec);
  qs.keep_self = keep_self ? 1 : 0;
  qs.append = append ? 1 : 0;
  return launch_qabs_slices(what, partial, partial_ld, rows, history, c.keep, split, words, n_words, qs, st);
}

QKV_EXPORT int qkv_final_indices_from_selected(const int64_t* selected, int64_t selected_ld, int64_t n_sel,
                                              int64_t rows, int64_t key_count, int64_t protect_sink,
                                              int64_t protect_recent, int keep_self, int64_t* final_indices,
                                              uint8_t* final_valid, int32_t* attn_ids, int64_t n_out,
                                              void* stream) {
  const char* what = "qkv_final_indices_from_selected";
  if (!final_indices || !final_valid || (n_sel > 0 && !selected)) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  const int64_t history = key_count - 1;
  if (rows <= 0 || rows > 65535 || history <= 0 || key_count >= (int64_t(1) << 31) || n_sel < 0 ||
      (n_sel > 0 && selected_ld < n_sel))
    return fail(QKV_ERR_INVALID, "%s: need 0 < rows <= 65535, 2 <= key_count < 2^31, selected_ld >= n_sel >= 0", what);
  if (protect_sink < 0 || protect_recent < 0) return fail(QKV_ERR_INVALID, "%s: negative protection", what);
  const ReuseCounts c = reuse_counts(history, protect_sink, protect_recent, 0.0, keep_self);
  const int64_t need = n_sel + c.sink_end + c.n_rec + (keep_self ? 1 : 0);
  if (n_out != need)
    return fail(QKV_ERR_INVALID, "%s: index rows hold %lld entries, the list needs %lld", what, (long long)n_out,
                (long long)need);
  final_from_selected_kernel<<<dim3(static_cast<unsigned>(cdiv(n_out, kRT)), static_cast<unsigned>(rows)), kRT, 0,
                               static_cast<hipStream_t>(stream)>>>(
      selected, selected_ld, static_cast<int>(n_sel), static_cast<int>(history), static_cast<int>(key_count),
      static_cast<int>(c.sink_end), static_cast<int>(c.recent_start), static_cast<int>(c.rec_begin),
      static_cast<int>(c.n_rec), final_indices, final_valid, attn_ids, static_cast<int>(n_out));
  return check_launch(what);
}

QKV_EXPORT int64_t qkv_reuse_block_final_count(int64_t history, int64_t block, int64_t protect_sink,
                                               int64_t protect_recent, double top_fraction, int keep_self) {
  if (history <= 0 || block < 1) return -1;
  const ReuseCounts c = reuse_counts(history, protect_sink, protect_recent, top_fraction, keep_self);
  return block_body_cap(c, block) + c.sink_end + c.n_rec + (keep_self ? 1 : 0);
}

QKV_EXPORT int qkv_reuse_expand_blocks(uint8_t* history_final, int64_t history_final_ld, int64_t rows,
                                       int64_t key_count, int64_t block, int64_t protect_sink,
                                       int64_t protect_recent, double top_fraction, int keep_self,
                                       int64_t* final_indices, uint8_t* final_valid, int32_t* attn_ids,
                                       int64_t n_out, void* stream) {
  const char* what = "qkv_reuse_expand_blocks";
  if (!history_final || !final_indices || !final_valid) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  if (rows <= 0 || rows > 65535) return fail(QKV_ERR_INVALID, "%s: need 1 <= rows <= 65535", what);
  const int64_t history = key_count - 1;
  if (history <= 0 || key_count >= (int64_t(1) << 31))
    return fail(QKV_ERR_INVALID, "%s: need 2 <= key_count < 2^31 (history excludes the current token)", what);
  if (history_final_ld < history) return fail(QKV_ERR_INVALID, "%s: mask row stride must cover the history", what);
  if (block < 1 || block > kMaxExpandBlock)
    return fail(QKV_ERR_INVALID, "%s: block must be in [1, %d]", what, kMaxExpandBlock);
  if (!(top_fraction >= 0.0)) return fail(QKV_ERR_INVALID, "%s: top_fraction must be >= 0", what);
  const ReuseCounts c = reuse_counts(history, protect_sink, protect_recent, top_fraction, keep_self);
  const int64_t body = block_body_cap(c, block);
  const int64_t need = body + c.sink_end + c.n_rec + (keep_self ? 1 : 0);
  if (n_out != need)
    return fail(QKV_ERR_INVALID, "%s: index rows hold %lld entries, the expanded selection needs %lld", what,
                (long long)n_out, (long long)need);
  reuse_expand_kernel<<<static_cast<unsigned>(rows), kExpandNT, 0, static_cast<hipStream_t>(stream)>>>(
      history_final, history_final_ld, static_cast<int>(history), static_cast<int>(block),
      static_cast<int>(body), static_cast<int>(key_count), static_cast<int>(c.sink_end),
      static_cast<int>(c.recent_start), static_cast<int>(c.rec_begin), static_cast<int>(c.n_rec), keep_self ? 1 : 0,
      final_indices, final_valid, attn_ids, static_cast<int>(n_out));
  return check_launch(what);
}

QKV_EXPORT int qkv_reuse_expand_blocks_bits(uint64_t* history_final, int64_t history_final_ld, int64_t rows,
                                            int64_t key_count, int64_t block, int64_t protect_sink,
                                            int64_t protect_recent, double top_fraction, int keep_self,
                                            int64_t* final_indices, uint8_t* final_valid, int32_t* attn_ids,
                                            int64_t n_out, void* stream) {
  const char* what = "qkv_reuse_expand_blocks_bits";
  if (!history_final || !final_indices || !final_valid) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  if (rows <= 0 || rows > 65535) return fail(QKV_ERR_INVALID, "%s: need 1 <= rows <= 65535", what);
  const int64_t history = key_count - 1;
  if (history <= 0 || key_count >= (int64_t(1) << 31))
    return fail(QKV_ERR_INVALID, "%s: need 2 <= key_count < 2^31 (history excludes the current token)", what);
  if (history_final_ld < cdiv(history, 64) || !aligned(history_final, 8))
    return fail(QKV_ERR_INVALID, "%s: the bitset's row stride must cover the history (8-byte aligned)", what);
  if (block < 1 || block > kMaxExpandBlock)
    return fail(QKV_ERR_INVALID, "%s: block must be in [1, %d]", what, kMaxExpandBlock);
  if (!(top_fraction >= 0.0)) return fail(QKV_ERR_INVALID, "%s: top_fraction must be >= 0", what);
  const ReuseCounts c = reuse_counts(history, protect_sink, protect_recent, top_fraction, keep_self);
  const int64_t body = block_body_cap(c, block);
  const int64_t need = body + c.sink_end + c.n_rec + (keep_self ? 1 : 0);
  if (n_out != need)
    return fail(QKV_ERR_INVALID, "%s: index rows hold %lld entries, the expanded selection needs %lld", what,
                (long long)n_out, (long long)need);
  reuse_expand_bits_kernel<<<static_cast<unsigned>(rows), kExpandNT, 0, static_cast<hipStream_t>(stream)>>>(
      history_final, history_final_ld, static_cast<int>(history), static_cast<int>(block),
      static_cast<int>(body), static_cast<int>(key_count), static_cast<int>(c.sink_end),
      static_cast<int>(c.recent_start), static_cast<int>(c.rec_begin), static_cast<int>(c.n_rec), keep_self ? 1 : 0,
      final_indices, final_valid, attn_ids, static_cast<int>(n_out));
  return check_launch(what);
}

QKV_EXPORT int qkv_reuse_partial_scores(const void* query, const void* key_dim_major, const int64_t* kdm_strides,
                                        int dtype, int64_t batch, int64_t q_heads, int64_t kv_heads,
                                        int64_t history, int64_t head_dim, int64_t dim_count, float* out,
                                        int64_t out_ld, void* stream) {
  const char* what = "qkv_reuse_partial_scores";
  int rc = check_heads(what, batch, q_heads, kv_heads, head_dim);
  if (rc) return rc;
  if (!query || !key_dim_major || !kdm_strides || !out) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  if (history <= 0 || history >= (int64_t(1) << 31) || out_ld < history)
    return fail(QKV_ERR_INVALID, "%s: need 0 < history < 2^31 and out_ld >= history", what);
  if (kdm_strides[3] != 1) return fail(QKV_ERR_UNSUPPORTED, "%s: the token axis of K must be contiguous", what);
  const int count = static_cast<int>(std::min<int64_t>(std::max<int64_t>(dim_count, 1),
                                                       std::min<int64_t>(head_dim, kMaxDims)));
  return dispatch_dtype<RunReusePartial>(dtype, query, key_dim_major, kdm_strides, batch, q_heads, kv_heads,
                                         history, head_dim, count, out, out_ld, static_cast<hipStream_t>(stream));
}

QKV_EXPORT int64_t qkv_threshold_mask_workspace_bytes(int64_t rows, int64_t n, int64_t k) {
  if (rows <= 0 || n <= 0 || k < 1 || k > n) return -1;
  return mask_ws_bytes(rows, n, k);
}

QKV_EXPORT int qkv_threshold_mask(const float* values, int64_t rows, int64_t n, int64_t ld, int64_t k,
                                  uint8_t* mask, int64_t mask_ld, void* workspace, int64_t workspace_bytes,
                                  void* stream) {
  const char* what = "qkv_threshold_mask";
  if (!values || !mask || !workspace) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  if (rows <= 0 || rows > 65535 || n <= 0 || n >= (int64_t(1) << 31) || k < 1 || k > n || ld < n || mask_ld < n)
    return fail(QKV_ERR_INVALID, "%s: need 0 < rows <= 65535, 1 <= k <= n, ld and mask_ld >= n", what);
  const int64_t need = mask_ws_bytes(rows, n, k);
  if (need < 0 || workspace_bytes < need)
    return fail(QKV_ERR_INVALID, "%s: workspace needs %lld bytes, got %lld", what, (long long)need,
                (long long)workspace_bytes);
  return threshold_mask_impl(what, values, rows, n, ld, k, mask, mask_ld, nullptr, workspace, workspace_bytes,
                             static_cast<hipStream_t>(stream));
}

QKV_EXPORT int qkv_reuse_lag_candidates(const void* query, const void* key_dim_major, const int64_t* kdm_strides,
                                        int dtype, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t history,
                                        int64_t head_dim, int64_t dim_count, int64_t k, const uint8_t* flags,
                                        int refresh, float* partial, int64_t partial_ld, uint8_t* mask,
                                        int64_t mask_ld, void* workspace, int64_t workspace_bytes, void* stream) {
  const char* what = "qkv_reuse_lag_candidates";
  int rc = check_heads(what, batch, q_heads, kv_heads, head_dim);
  if (rc) return rc;
  if (!query || !key_dim_major || !kdm_strides || !partial || !mask || !workspace)
    return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  if (history <= 0 || history >= (int64_t(1) << 31) || partial_ld < history || mask_ld < history || k < 1 ||
      k > history)
    return fail(QKV_ERR_INVALID, "%s: need 0 < history < 2^31, 1 <= k <= history, partial_ld and mask_ld >= history",
                what);
  if (kdm_strides[3] != 1) return fail(QKV_ERR_UNSUPPORTED, "%s: the token axis of K must be contiguous", what);
  if (refresh < QKV_REFRESH_NONE || refresh > QKV_REFRESH_MAJORITY)
    return fail(QKV_ERR_INVALID, "%s: unknown refresh %d", what, refresh);
  if (refresh >= QKV_REFRESH_PER_ROW && !flags) return fail(QKV_ERR_INVALID, "%s: null flags", what);
  const int64_t rows = batch * q_heads;
  const int64_t need = mask_ws_bytes(rows, history, k);
  if (need < 0 || workspace_bytes < need)
    return fail(QKV_ERR_INVALID, "%s: workspace needs %lld bytes, got %lld", what, (long long)need,
                (long long)workspace_bytes);
  if (refresh == QKV_REFRESH_NONE) return QKV_OK;   // no row takes new candidates
  const uint8_t* gate = refresh == QKV_REFRESH_ALL ? nullptr : flags;
  const int count = static_cast<int>(std::min<int64_t>(std::max<int64_t>(dim_count, 1),
                                                       std::min<int64_t>(head_dim, kMaxDims)));
  return dispatch_dtype<RunCandidates>(dtype, what, query, key_dim_major, kdm_strides, batch, q_heads, kv_heads,
                                       history, head_dim, count, k, partial, partial_ld, mask, mask_ld, nullptr,
                                       workspace, workspace_bytes, static_cast<hipStream_t>(stream), gate, refresh);
}

QKV_EXPORT int qkv_reuse_lag_candidates_bits(const void* query, const void* key_dim_major,
                                             const int64_t* kdm_strides, int dtype, int64_t batch, int64_t q_heads,
                                             int64_t kv_heads, int64_t history, int64_t head_dim, int64_t dim_count,
                                             int64_t k, const uint8_t* flags, int refresh, float* partial,
                                             int64_t partial_ld, uint64_t* bits, int64_t bits_ld, void* workspace,
                                             int64_t workspace_bytes, void* stream) {
  const char* what = "qkv_reuse_lag_candidates_bits";
  int rc = check_heads(what, batch, q_heads, kv_heads, head_dim);
  if (rc) return rc;
  if (!query || !key_dim_major || !kdm_strides || !partial || !bits || !workspace)
    return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  if (history <= 0 || history >= (int64_t(1) << 31) || partial_ld < history || bits_ld < cdiv(history, 64) ||
      !aligned(bits, 8) || k < 1 || k > history)
    return fail(QKV_ERR_INVALID, "%s: need 0 < history < 2^31, 1 <= k <= history, row strides covering the history",
                what);
  if (kdm_strides[3] != 1) return fail(QKV_ERR_UNSUPPORTED, "%s: the token axis of K must be contiguous", what);
  if (refresh < QKV_REFRESH_NONE || refresh > QKV_REFRESH_MAJORITY)
    return fail(QKV_ERR_INVALID, "%s: unknown refresh %d", what, refresh);
  if (refresh >= QKV_REFRESH_PER_ROW && !flags) return fail(QKV_ERR_INVALID, "%s: null flags", what);
  const int64_t rows = batch * q_heads;
  const int64_t need = qkv_reuse_candidates_workspace_bytes(rows, history, k);
  if (need < 0 || workspace_bytes < need)
    return fail(QKV_ERR_INVALID, "%s: workspace needs %lld bytes, got %lld", what, (long long)need,
                (long long)workspace_bytes);
  if (!aligned(workspace, 16)) return fail(QKV_ERR_INVALID, "%s: the workspace must be 16-byte aligned", what);
  if (refresh == QKV_REFRESH_NONE) return QKV_OK;   // no row takes new candidates
  const uint8_t* gate = refresh == QKV_REFRESH_ALL ? nullptr : flags;
  const int count = static_cast<int>(std::min<int64_t>(std::max<int64_t>(dim_count, 1),
                                                       std::min<int64_t>(head_dim, kMaxDims)));
  char* ws = static_cast<char*>(workspace);
  const int64_t state = cand_state_bytes(rows);
  CandSplit split;
  split.hist = reinterpret_cast<int*>(ws);
  split.state = reinterpret_cast<int*>(ws + align256(rows * kCandBins * 4));
  split.list_val = reinterpret_cast<float*>(ws + state);
  split.list_pos = reinterpret_cast<int*>(ws + state + align256(rows * history * 4));
  return dispatch_dtype<RunCandidates>(dtype, what, query, key_dim_major, kdm_strides, batch, q_heads, kv_heads,
                                       history, head_dim, count, k, partial, partial_ld, nullptr, 0, nullptr,
                                       ws + state, workspace_bytes - state, static_cast<hipStream_t>(stream), gate,
                                       refresh, bits, bits_ld, split);
}

QKV_EXPORT int qkv_reuse_candidates(const void* query, const void* key_dim_major, const int64_t* kdm_strides,
                                    int dtype, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t history,
                                    int64_t head_dim, int64_t dim_count, int64_t k, float* partial,
                                    int64_t partial_ld, uint8_t* mask, int64_t mask_ld, uint64_t* bits,
                                    int64_t bits_ld, float* thr_out, void* workspace, int64_t workspace_bytes,
                                    void* stream) {
  const char* what = "qkv_reuse_candidates";
  int rc = check_heads(what, batch, q_heads, kv_heads, head_dim);
  if (rc) return rc;
  if (!query || !key_dim_major || !kdm_strides || !partial || !workspace || !mask == !bits)
    return fail(QKV_ERR_INVALID, "%s: null pointer (or not exactly one of mask and bits)", what);
  if (history <= 0 || history >= (int64_t(1) << 31) || partial_ld < history || k < 1 || k > history ||
      (mask && mask_ld < history) || (bits && (bits_ld < cdiv(history, 64) || !aligned(bits, 8))))
    return fail(QKV_ERR_INVALID, "%s: need 0 < history < 2^31, 1 <= k <= history, row strides covering the history",
                what);
  if (kdm_strides[3] != 1) return fail(QKV_ERR_UNSUPPORTED, "%s: the token axis of K must be contiguous", what);
  const int64_t rows = batch * q_heads;
  const int64_t need = qkv_reuse_candidates_workspace_bytes(rows, history, k);
  if (need < 0 || workspace_bytes < need)
    return fail(QKV_ERR_INVALID, "%s: workspace needs %lld bytes, got %lld", what, (long long)need,
                (long long)workspace_bytes);
  if (!aligned(workspace, 16)) return fail(QKV_ERR_INVALID, "%s: the workspace must be 16-byte aligned", what);
  const int count = static_cast<int>(std::min<int64_t>(std::max<int64_t>(dim_count, 1),
                                                       std::min<int64_t>(head_dim, kMaxDims)));
  char* ws = static_cast<char*>(workspace);
  const int64_t state = cand_state_bytes(rows);
  CandSplit split;
  split.hist = reinterpret_cast<int*>(ws);
  split.state = reinterpret_cast<int*>(ws + align256(rows * kCandBins * 4));   // (kCandState ints per row)
  split.list_val = reinterpret_cast<float*>(ws + state);
  split.list_pos = reinterpret_cast<int*>(ws + state + align256(rows * history * 4));
  return dispatch_dtype<RunCandidates>(dtype, what, query, key_dim_major, kdm_strides, batch, q_heads, kv_heads,
                                       history, head_dim, count, k, partial, partial_ld, mask, mask_ld, thr_out,
                                       ws + state, workspace_bytes - state, static_cast<hipStream_t>(stream), nullptr,
                                       QKV_REFRESH_ALL, bits, bits_ld, split);
}

QKV_EXPORT int64_t qkv_reuse_candidates_workspace_bytes(int64_t rows, int64_t history, int64_t k) {
  if (rows <= 0 || history <= 0 || history >= (int64_t(1) << 31) || k < 1 || k > history) return -1;
  const int64_t scratch = cand_scratch_bytes(rows, history, k);
  return scratch < 0 ? -1 : cand_state_bytes(rows) + scratch;
}

QKV_EXPORT int64_t qkv_candidate_mask_workspace_bytes(int64_t rows, int64_t n, int selection, int64_t k,
                                                      int64_t n_sample) {
  if (rows <= 0 || n <= 0) return -1;
  if (selection == QKV_CAND_TOPK) return qkv_threshold_mask_workspace_bytes(rows, n, k);
  if (selection == QKV_CAND_PREVIOUS_THRESHOLD) return 0;
  if (selection != QKV_CAND_SAMPLE_QUANTILE || n_sample < 1 || n_sample > n || k < 1 || k > n_sample) return -1;
  const int64_t kth = n_sample <= kWideMax ? 0 : mask_ws_bytes(rows, n_sample, k);
  return kth < 0 ? -1 : align256(rows * n_sample * 4) + kth;
}

QKV_EXPORT int qkv_candidate_mask(const float* values, int64_t rows, int64_t n, int64_t ld, int selection,
                                  int64_t k, const int32_t* sample_cols, int64_t n_sample, float* thresholds,
                                  uint8_t* mask, int64_t mask_ld, uint64_t* bits, int64_t bits_ld, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
  const char* what = "qkv_candidate_mask";
  if (!values || !mask == !bits) return fail(QKV_ERR_INVALID, "%s: null pointer (or not exactly one of mask and bits)", what);
  if (rows <= 0 || rows > 65535 || n <= 0 || n >= (int64_t(1) << 31) || ld < n || (mask && mask_ld < n) ||
      (bits && (bits_ld < cdiv(n, 64) || !aligned(bits, 8))))
    return fail(QKV_ERR_INVALID, "%s: need 0 < rows <= 65535, ld and the mask's row stride covering n", what);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 bgrid(static_cast<unsigned>(cdiv(n, kRT * 4)), static_cast<unsigned>(rows));   // bitset launches
  if (selection == QKV_CAND_TOPK) {
    if (k < 1 || k > n) return fail(QKV_ERR_INVALID, "%s: need 1 <= k <= n", what);
    if (!workspace) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
    const int64_t need = mask_ws_bytes(rows, n, k);
    if (need < 0 || workspace_bytes < need)
      return fail(QKV_ERR_INVALID, "%s: workspace needs %lld bytes, got %lld", what, (long long)need,
                  (long long)workspace_bytes);
    return threshold_mask_impl(what, values, rows, n, ld, k, mask, mask_ld, thresholds, workspace, workspace_bytes,
                               st, nullptr, 0, bits, bits_ld);
  }
  if (!thresholds) return fail(QKV_ERR_INVALID, "%s: this selection needs the thresholds array", what);
  const bool vec = ld % 4 == 0 && aligned(values, 16) && mask_ld % 16 == 0 && aligned(mask, 16);
  dim3 grid(static_cast<unsigned>(cdiv(n, kMaskTile)), static_cast<unsigned>(rows));
  if (selection == QKV_CAND_PREVIOUS_THRESHOLD) {
    if (bits)
      reuse_mask_bits_kernel<<<bgrid, kRT, 0, st>>>(values, ld, static_cast<int>(n), nullptr, 0, thresholds, bits,
                                                    bits_ld, nullptr);
    else
      reuse_mask_kernel<<<grid, kRT, 0, st>>>(values, ld, static_cast<int>(n), nullptr, 0, thresholds, mask, mask_ld,
                                              vec, nullptr);
    return check_launch(what);
  }
  if (selection != QKV_CAND_SAMPLE_QUANTILE) return fail(QKV_ERR_INVALID, "%s: unknown selection %d", what, selection);
  if (!sample_cols || !workspace) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  if (n_sample < 1 || n_sample > n || k < 1 || k > n_sample)
    return fail(QKV_ERR_INVALID, "%s: need 1 <= k <= n_sample <= n", what);
  const int64_t need = qkv_candidate_mask_workspace_bytes(rows, n, selection, k, n_sample);
  if (need < 0 || workspace_bytes < need)
    return fail(QKV_ERR_INVALID, "%s: workspace needs %lld bytes, got %lld", what, (long long)need,
                (long long)workspace_bytes);
  if (n_sample <= kRT) {   // gather, k-th of the sample and compare in one launch
    if (!bits) {
      sample_mask_kernel<<<grid, kRT, 0, st>>>(values, ld, static_cast<int>(n), sample_cols,
                                               static_cast<int>(n_sample), static_cast<int>(k), mask, mask_ld, vec,
                                               thresholds);
      return check_launch(what);
    }
    // the threshold from one tile's launch, then the bitset
    sample_mask_kernel<<<dim3(1, static_cast<unsigned>(rows)), kRT, 0, st>>>(
        values, ld, static_cast<int>(n), sample_cols, static_cast<int>(n_sample), static_cast<int>(k), nullptr, 0,
        false, thresholds);
    int rc = check_launch(what);
    if (rc) return rc;
    reuse_mask_bits_kernel<<<bgrid, kRT, 0, st>>>(values, ld, static_cast<int>(n), nullptr, 0, thresholds, bits,
                                                  bits_ld, nullptr);
    return check_launch(what);
  }
  float* sampled = static_cast<float*>(workspace);
  gather_cols_kernel<<<dim3(static_cast<unsigned>(cdiv(n_sample, kRT)), static_cast<unsigned>(rows)), kRT, 0, st>>>(
      values, ld, sample_cols, static_cast<int>(n_sample), sampled);
  int rc = check_launch(what);
  if (rc) return rc;
  // the k-th largest sampled value, then the mask over the whole row
  if (n_sample <= kWideMax) {
    rc = with_wide_vpl(n_sample, [&](auto vpl) {
      reuse_mask_wide_kernel<decltype(vpl)::value><<<static_cast<unsigned>(rows), kWideNT, 0, st>>>(
          sampled, n_sample, static_cast<int>(n_sample), static_cast<int>(k), nullptr, 0, thresholds);
      return check_launch(what);
    });
  } else {
    char* rest = static_cast<char*>(workspace) + align256(rows * n_sample * 4);
    int32_t* sel = reinterpret_cast<int32_t*>(rest);
    rc = qkv_topk_ws(sampled, rows, n_sample, n_sample, k, sel, rest + align256(rows * k * 4),
                     workspace_bytes - align256(rows * n_sample * 4) - align256(rows * k * 4), stream);
    if (rc) return rc;
    // a one-token-tile launch of the mask kernel writes the threshold only
    reuse_mask_kernel<<<dim3(1, static_cast<unsigned>(rows)), kRT, 0, st>>>(
        sampled, n_sample, 0, sel, static_cast<int>(k), nullptr, mask, mask_ld, false, thresholds);
    rc = check_launch(what);
  }
  if (rc) return rc;
  if (bits)
    reuse_mask_bits_kernel<<<bgrid, kRT, 0, st>>>(values, ld, static_cast<int>(n), nullptr, 0, thresholds, bits,
                                                  bits_ld, nullptr);
  else
    reuse_mask_kernel<<<grid, kRT, 0, st>>>(values, ld, static_cast<int>(n), nullptr, 0, thresholds, mask, mask_ld,
                                            vec, nullptr);
  return check_launch(what);
}

QKV_EXPORT int qkv_dim_major_append(const void* key, const int64_t* k_strides, int dtype, int64_t batch,
                                    int64_t kv_heads, int64_t head_dim, int64_t t_begin, int64_t t_end,
                                    void* key_dim_major, const int64_t* kdm_strides, void* stream) {
  const char* what = "qkv_dim_major_append";
  if (!key || !k_strides || !key_dim_major || !kdm_strides) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  if (batch <= 0 || kv_heads <= 0 || batch * kv_heads > 65535 || head_dim <= 0 || head_dim > 512)
    return fail(QKV_ERR_INVALID, "%s: bad sizes", what);
  if (t_begin < 0 || t_end < t_begin || t_end >= (int64_t(1) << 31))
    return fail(QKV_ERR_INVALID, "%s: need 0 <= t_begin <= t_end < 2^31", what);
  if (k_strides[3] != 1 || kdm_strides[3] != 1)
    return fail(QKV_ERR_UNSUPPORTED, "%s: K channels and the copy's token axis must be contiguous", what);
  if (dtype == QKV_DTYPE_FP32 && head_dim > 256)
    return fail(QKV_ERR_UNSUPPORTED, "%s: fp32 K needs head_dim <= 256", what);
  if (t_end == t_begin) return QKV_OK;
  return dispatch_dtype<RunDimMajor2>(dtype, key, k_strides, batch, kv_heads, head_dim, t_begin, t_end,
                                      key_dim_major, kdm_strides, static_cast<hipStream_t>(stream));
}
