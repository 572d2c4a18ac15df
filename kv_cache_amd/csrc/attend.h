// Sparse gather attention: the launch-shape knobs, the slot map, the
// workgroup epilogue (wave combine, split publish / merge) and the
// matrix-core attention body shared by attention.hip's kernels.  The design
// is described in attention.hip.
#pragma once

#include "common.h"
#include "select.h"

#ifndef QKV_ATTN_TARGET_WGS
#define QKV_ATTN_TARGET_WGS 256
#endif
// Workgroups per CU the register budget is sized for (at 4 waves each; an
// 8-wave workgroup counts as two).
#ifndef QKV_ATTN_WG_PER_CU
#define QKV_ATTN_WG_PER_CU 2
#endif
// Waves per workgroup (4 or 8).
#ifndef QKV_ATTN_WAVES
#define QKV_ATTN_WAVES 4
#endif
// Chunks of K/V a wave holds in registers: the one it computes and
// QKV_ATTN_DEPTH - 1 in flight.
#ifndef QKV_ATTN_DEPTH
#define QKV_ATTN_DEPTH 2
#endif

namespace qkv {
namespace {

constexpr int kD = 128;     // head dim
constexpr int kWaves = QKV_ATTN_WAVES;
static_assert(kWaves == 4 || kWaves == 8, "4 or 8 waves per workgroup");
constexpr int kDepth = QKV_ATTN_DEPTH;
static_assert(kDepth == 2 || kDepth == 3, "2 or 3 chunks of K/V in registers");
// Ticket words at the start of the workspace, one per possible row, so calls
// of any shape that share a workspace find their tickets at the same place.
constexpr int64_t kTicketWords = 65536;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u) return static_cast<uint16_t>((u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u));
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// 16-byte load with the non-temporal hint: K/V rows are read once per step.
__device__ __forceinline__ uint4 ld_nt(const uint16_t* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// Output element of the 16-bit dtype (bf16, or fp16 with F16), rounded to nearest even.
template <bool F16>
__device__ __forceinline__ uint16_t f32_to_half(float f) {
  if constexpr (F16) return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  else return f32_to_bf16_rne(f);
}

// c + a.lo * b.lo + a.hi * b.hi over packed pairs of the 16-bit dtype, in fp32
// (v_dot2_f32_bf16 / v_dot2_f32_f16).
template <bool F16>
__device__ __forceinline__ float dot2_half(uint32_t a, uint32_t b, float c) {
  if constexpr (F16)
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c, false);
  else
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                           false);
}

// Sum over each row of 16 lanes; every lane of the row receives the sum.
// quad_perm [1,0,3,2] and [2,3,0,1] reduce each quad, then row_half_mirror
// and row_mirror pair every lane with the other quad / other half.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  v += dpp_f<0x140>(v);
  return v;
}

// Rows of at most kSelMaxBlocks block maxima can select in the kernel.
constexpr int kSelMaxVPL = 16;
constexpr int kSelMaxBlocks = 256 * kSelMaxVPL;

// Slot -> token map of one row.  Slot s < n_blk_slots is token
// ids[s / block] * block + s % block, masked (-1) where that lies past the
// history or inside the sink or recent range; protected slot n_blk_slots + i
// is sink token i, then recent token rec_begin + (i - sink_end), then the
// current token (EV:2938-2982).
struct RowSlots {
  const int32_t* ids;   // the row's block ids (global memory, or the LDS selection)
  int n_blk_slots, n_slots, block, nb, tokens, sink_end, recent_start, rec_begin, n_rec, self_tok;

  // Block id of `slot` for a lane that has one (ok), -2 - i for protected
  // slot i, else -1.  The id load always happens, from a clamped index.
  __device__ __forceinline__ int id_of(int slot, bool ok) const {
    const bool blk = ok && slot < n_blk_slots;
    const int v = ids[blk ? slot / block : 0];
    return blk ? v : (ok && slot < n_slots ? n_blk_slots - 2 - slot : -1);
  }
  // Token of `slot` given its id_of, or -1.
  __device__ __forceinline__ int token_of(int slot, int id) const {
    if (id <= -2) {
      const int i = -2 - id;
      return i < sink_end ? i : i < sink_end + n_rec ? rec_begin + (i - sink_end) : self_tok;
    }
    if (id < 0 || id >= nb) return -1;
    const int t = id * block + (slot - (slot / block) * block);
    return (t < tokens && t >= sink_end && t < recent_start) ? t : -1;
  }
};

// Workgroup epilogue of both attention kernels, entered by every thread once
// red_m / red_l / red_acc hold each wave's (max, sum, weighted V) per head
// and a barrier has passed.  A row that fits one workgroup writes its output
// (bf16, or fp16 with F16); otherwise the workgroup publishes its partial, takes a ticket, and
// the row's last workgroup merges all partials.
template <int G, int NW, bool F16>
__device__ __forceinline__ void finish_workgroup(const float (&red_acc)[NW][G][kD], const float (&red_m)[NW][G],
                                                 const float (&red_l)[NW][G], int& last_flag, int r, int split,
                                                 int nsplit, uint16_t* __restrict__ out_row,
                                                 float* __restrict__ ws_acc, float* __restrict__ ws_ml,
                                                 uint32_t* __restrict__ tickets) {
  constexpr int NT = 64 * NW;
  const int tid = threadIdx.x;
  const float ninf = -__builtin_huge_valf();
  // Workgroup max per head and the rescale factor of each wave.
  float wg_m[G], wg_l[G], fs[G][NW];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float mx = red_m[0][h];
#pragma unroll
    for (int w = 1; w < NW; ++w) mx = fmaxf(mx, red_m[w][h]);
    wg_m[h] = mx;
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      fs[h][w] = (red_m[w][h] == ninf) ? 0.0f : exp2f(red_m[w][h] - mx);
      sum = __builtin_fmaf(red_l[w][h], fs[h][w], sum);
    }
    wg_l[h] = sum;
  }
  auto wg_acc = [&](int h, int d) -> float {
    float o = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) o = __builtin_fmaf(red_acc[w][h][d], fs[h][w], o);
    return o;
  };

  if (nsplit == 1) {
    for (int idx = tid; idx < G * kD; idx += NT) {
      const int h = idx / kD, d = idx - h * kD;
      const float o = (wg_m[h] == ninf) ? 0.0f : wg_acc(h, d) / wg_l[h];
      out_row[h * kD + d] = f32_to_half<F16>(o);
    }
    return;
  }

  const int64_t part = static_cast<int64_t>(r) * nsplit + split;
  for (int idx = tid; idx < G * kD; idx += NT) {
    const int h = idx / kD, d = idx - h * kD;
    st_coherent(ws_acc + part * G * kD + idx, wg_acc(h, d));
  }
  if (tid < G) {
    st_coherent(ws_ml + (part * G + tid) * 2 + 0, wg_m[tid]);
    st_coherent(ws_ml + (part * G + tid) * 2 + 1, wg_l[tid]);
  }
  // Every store of this workgroup has completed before the ticket is taken.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const uint32_t t = __hip_atomic_fetch_add(tickets + r, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = t == static_cast<uint32_t>(nsplit - 1);
    if (last) __hip_atomic_store(tickets + r, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = last;
  }
  __syncthreads();
  if (!last_flag) return;

  // Last workgroup of the row: merge the splits.  Thread t owns outputs
  // t + NT*k; the (max, sum, weighted V) loads of MS splits of every owned
  // output are all issued before any arithmetic.
  constexpr int OPT = (G * kD + NT - 1) / NT;
  constexpr int MS = OPT >= 4 ? 4 : 16 / OPT;   // splits per batch of loads
  float mx[OPT], den[OPT], o[OPT];
#pragma unroll
  for (int k = 0; k < OPT; ++k) {
    mx[k] = ninf;
    den[k] = 0.0f;
    o[k] = 0.0f;
  }
  const float* ml_row = ws_ml + static_cast<int64_t>(r) * nsplit * G * 2;
  const float* acc_row = ws_acc + static_cast<int64_t>(r) * nsplit * G * kD;
  for (int i0 = 0; i0 < nsplit; i0 += MS) {
    float mi[OPT][MS], li[OPT][MS], ai[OPT][MS];
#pragma unroll
    for (int k = 0; k < OPT; ++k) {
      const int idx = min(tid + k * NT, G * kD - 1);
      const int h = idx / kD;
#pragma unroll
      for (int u = 0; u < MS; ++u) {
        const int i = min(i0 + u, nsplit - 1);
        ai[k][u] = ld_coherent(acc_row + static_cast<int64_t>(i) * G * kD + idx);
        mi[k][u] = ld_coherent(ml_row + (i * G + h) * 2);
        li[k][u] = ld_coherent(ml_row + (i * G + h) * 2 + 1);
      }
    }
#pragma unroll
    for (int k = 0; k < OPT; ++k) {
      float m2 = mx[k];
#pragma unroll
      for (int u = 0; u < MS; ++u)
        if (i0 + u < nsplit) m2 = fmaxf(m2, mi[k][u]);
      if (m2 == ninf) continue;
      const float c = (mx[k] == ninf) ? 0.0f : exp2f(mx[k] - m2);
      den[k] *= c;
      o[k] *= c;
#pragma unroll
      for (int u = 0; u < MS; ++u) {
        if (i0 + u < nsplit && mi[k][u] != ninf) {
          const float w = exp2f(mi[k][u] - m2);
          den[k] = __builtin_fmaf(li[k][u], w, den[k]);
          o[k] = __builtin_fmaf(ai[k][u], w, o[k]);
        }
      }
      mx[k] = m2;
    }
  }
#pragma unroll
  for (int k = 0; k < OPT; ++k) {
    const int idx = tid + k * NT;
    if (idx < G * kD) {
      const float v = (mx[k] == ninf) ? 0.0f : o[k] / den[k];
      out_row[idx] = f32_to_half<F16>(v);
    }
  }
}

// Chunks per wave: doubled (up to max_iters) while the grid keeps `target`
// workgroups (QKV_ATTN_TARGET_WGS), so long selections take few splits per
// row; doubling stops once one workgroup covers the whole row (further
// chunks would only walk empty slots).  per_iter = slots a workgroup covers
// per chunk round.
inline int chunk_rounds(int64_t rows, int64_t n_slots, int64_t per_iter, int max_iters,
                        int64_t target = QKV_ATTN_TARGET_WGS) {
  int it = 1;
  while (it < max_iters && per_iter * it < n_slots && rows * cdiv(n_slots, per_iter * it * 2) >= target) it *= 2;
  return it;
}

// Words of split partials a workspace needs for calls of up to n_slots slots
// per row.  The split count is not monotonic in the slot count, but below
// the chunk cap a doubling that failed bounds it: splits <= 2 *
// (ceil(target/rows) - 1); at the cap it grows with the slots.  The larger of
// that bound and this size's own count covers every call with fewer slots,
// so one workspace serves all smaller selections.  Per split: weighted V per
// head, then (max, sum) per head.
inline int64_t attention_partial_words(int64_t rows, int64_t n_slots, int64_t g, int64_t per_iter, int max_iters,
                                       int64_t target = QKV_ATTN_TARGET_WGS) {
  const int64_t own = cdiv(n_slots, per_iter * chunk_rounds(rows, n_slots, per_iter, max_iters, target));
  const int64_t below_cap = std::min(cdiv(n_slots, per_iter), 2 * (cdiv(target, rows) - 1));
  return rows * std::max(own, below_cap) * g * (kD + 2);
}

// Arguments of both attention kernels.
struct AttnArgs {
  const uint16_t *q, *k, *v;
  int64_t sb, sh, st;
  int q_heads, kv_heads, tokens;
  const int32_t* block_ids;
  int n_sel, block, nb;
  float scale_log2;
  int nsplit;
  float *ws_acc, *ws_ml;
  uint32_t* tickets;
  uint16_t* out;
  const float* bmax;
  int64_t bmax_ld;
  int32_t* sel_out;
  int kv_div, n_prot, sink_end, recent_start, rec_begin, n_rec, self_tok;
};

// Where a row's block ids come from (attend_mfma).
enum { kIdsGiven = 0, kIdsSelect = 1 };

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// c + A.B on a 16x16x32 tile, eight 16-bit elements per lane in a and b
// (v_mfma_f32_16x16x32_bf16 / _f16).
template <bool F16>
__device__ __forceinline__ f32x4_t mfma_16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                  0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
}

// c + A.B on a 16x16x16 tile, four 16-bit elements per lane in a and b
// (v_mfma_f32_16x16x16_bf16 / _f16).
template <bool F16>
__device__ __forceinline__ f32x4_t mfma_16x16x16(u32x2_t a, u32x2_t b, f32x4_t c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4_t, a), __builtin_bit_cast(f16x4_t, b), c,
                                                 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4_t, a), __builtin_bit_cast(s16x4_t, b),
                                                     c, 0, 0, 0);
}

// Four fp32 values rounded (nearest even) to the 16-bit dtype and packed.
template <bool F16>
__device__ __forceinline__ u32x2_t pack4_half(const float (&p)[4]) {
  if constexpr (F16)
    return __builtin_bit_cast(u32x2_t, f16x4_t{static_cast<_Float16>(p[0]), static_cast<_Float16>(p[1]),
                                               static_cast<_Float16>(p[2]), static_cast<_Float16>(p[3])});
  else
    return __builtin_bit_cast(u32x2_t, bf16x4_t{static_cast<__bf16>(p[0]), static_cast<__bf16>(p[1]),
                                                static_cast<__bf16>(p[2]), static_cast<__bf16>(p[3])});
}

__device__ __forceinline__ u32x4_t ld_nt4(const uint16_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
}

// Lazy rescaling in the MFMA kernel: the maximum a wave exponentiates against
// is raised only when some head's chunk maximum exceeds it by more than this
// (log2 units).  P then stays below 2^8, and the accumulators are rescaled on
// the few chunks that raise it instead of on every chunk; O / l is unchanged.
constexpr float kLazyLog2 = 8.0f;
// A wave's V tile in LDS, channel-major: 16 slots (32 bytes) per channel plus
// 4 bytes of padding, so the transposing 16-bit stores and the 8-byte reads
// of one instruction spread over the banks.
constexpr int kVtStride = 18;   // uint16 per channel

// Sparse attention on the matrix cores for row r, split `split`, any G <= 16
// (the body of sparse_attn_mfma_kernel).  Work split, selection, protected
// slots and the workgroup epilogue are those of sparse_attn_kernel; a wave's
// chunk is 16 slots, ITERS chunks per wave.  IDS: the row's block ids are
// given (kIdsGiven) or selected from the row's block maxima in the
// workgroup (kIdsSelect, SELV keys per thread).
//   QK: S^T[slot][head] = sum_k K[slot][k] Q[head][k], four
//   v_mfma_f32_16x16x32_bf16 (_f16 with F16) over k = 32s..32s+31 with A = K (lane 16g+c
//   reads 16 bytes of slot c's row: channels 32s+8g..32s+8g+7) and B = Q^T
//   (heads past G are zero columns).  Lane 16g+c then holds head c for slots
//   4g..4g+3.
//   P.V: O[head][ch] += sum_slot P[head][slot] V[slot][ch], eight
//   v_mfma_f32_16x16x16_bf16 (_f16) of 16 channels each.  P (rounded to the
//   K/V dtype, as the reference's attention does) is already in the A layout; V is loaded
//   as in sparse_attn_kernel (lane 16g+c: slot 4i+g, channels 8c..8c+7),
//   stored channel-major into the wave's LDS tile, and read back as B, four
//   slots of one channel per lane.
// Softmax is per head over the lanes of its column (in-lane over 4 slots, then
// the lane swaps), in the log2 domain with lazy rescaling.
template <int G, int ITERS, int SELV, int IDS, bool F16>
__device__ __forceinline__ void attend_mfma(const AttnArgs& a, int r, int split) {
  constexpr int NW = 4, NT = 256, CH = 16;
  static_assert(G <= 16, "the heads are the 16 columns of the QK tile");
  static_assert(IDS != kIdsSelect || SELV > 0, "the in-kernel selection needs keys per thread");
  constexpr int n_it = ITERS;   // chunks per wave

  __shared__ float red_acc[NW][G][kD];
  __shared__ float red_m[NW][G], red_l[NW][G];
  __shared__ int last_flag;
  constexpr bool SEL = IDS == kIdsSelect;   // ids come from LDS
  __shared__ int32_t sel_lds[IDS == kIdsSelect ? NT * SELV : 1];
  __shared__ __attribute__((aligned(16))) uint16_t vt[NW][kD * kVtStride];

  const int b = r / a.kv_heads, j = r - b * a.kv_heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g4 = lane >> 4, c16 = lane & 15;
  const float ninf = -__builtin_huge_valf();
  if constexpr (IDS == kIdsSelect) {
    select_row<SELV, false, NW>(a.bmax + static_cast<int64_t>(r) * a.bmax_ld, a.nb, a.n_sel, sel_lds);
    if (a.sel_out && split == 0)
      for (int i = tid; i < a.n_sel; i += NT) a.sel_out[static_cast<int64_t>(r) * a.n_sel + i] = sel_lds[i];
  }
  const int n_blk_slots = a.n_sel * a.block;
  const RowSlots rs{SEL ? sel_lds : a.block_ids + static_cast<int64_t>(r) * a.n_sel, n_blk_slots,
                    n_blk_slots + a.n_prot, a.block, a.nb, a.tokens, a.sink_end, a.recent_start, a.rec_begin,
                    a.n_rec, a.self_tok};
  const int wg_base = split * (NW * CH * n_it);
  auto slot_of = [&](int c) -> int { return wg_base + (NW * c + wave) * CH + lane; };
  auto load_id = [&](int c) -> int { return rs.id_of(slot_of(c), lane < CH); };
  auto token_of = [&](int c, int id) -> int { return rs.token_of(slot_of(c), id); };

  const int jk = j / a.kv_div;   // the K/V head this row reads
  const uint16_t* kb = a.k + b * a.sb + jk * a.sh + 8 * g4;
  const uint16_t* vb = a.v + b * a.sb + jk * a.sh + 8 * c16;
  const int64_t st = a.st;
  const float scale_log2 = a.scale_log2;

  u32x4_t qb[4];   // B operand of QK: Q[head c16][32s + 8g4 ..], zero for heads >= G
  {
    const uint16_t* qrow = a.q + (static_cast<int64_t>(b) * a.q_heads + j * G + min(c16, G - 1)) * kD + 8 * g4;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4_t w = *reinterpret_cast<const u32x4_t*>(qrow + 32 * s);
      if (c16 >= G) w = u32x4_t{0u, 0u, 0u, 0u};
      qb[s] = w;
    }
  }

  // Loads of one chunk from the tokens its 16 lanes resolved (-1 elsewhere):
  // K rows of slot c16, V rows of slot 4i + g4 (invalid slots read token 0 of
  // the row and are masked), and the chunk's valid-slot mask.
  auto gather = [&](int my_tok, u32x4_t (&kx)[4], u32x4_t (&vx)[4], uint32_t& vm) {
    const int ta = __builtin_amdgcn_ds_bpermute(c16 << 2, my_tok);
    vm = static_cast<uint32_t>(__ballot(my_tok >= 0));
#pragma unroll
    for (int s = 0; s < 4; ++s) kx[s] = ld_nt4(kb + static_cast<int64_t>(max(ta, 0)) * st + 32 * s);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tv = __builtin_amdgcn_ds_bpermute((4 * i + g4) << 2, my_tok);
      vx[i] = ld_nt4(vb + static_cast<int64_t>(max(tv, 0)) * st);
    }
  };

  f32x4_t o[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) o[q] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float m = ninf, lsum = 0.0f;   // head c16: running maximum (log2) and this lane's share of the sum
  uint16_t* vtw = vt[wave];
  const uint32_t* vt32 = reinterpret_cast<const uint32_t*>(vt[wave]);

  auto compute = [&](const u32x4_t (&kx)[4], const u32x4_t (&vx)[4], uint32_t vm) {
    // V tile, channel-major (the stores run while the QK tile computes).
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = vx[i][e];
        const int at = (8 * c16 + 2 * e) * kVtStride + 4 * i + g4;
        vtw[at] = static_cast<uint16_t>(w);
        vtw[at + kVtStride] = static_cast<uint16_t>(w >> 16);
      }
    }
    f32x4_t sacc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < 4; ++s)
      sacc = mfma_16x16x32<F16>(kx[s], qb[s], sacc);
    float sv[4], cm = ninf;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sv[i] = ((vm >> (4 * g4 + i)) & 1u) ? sacc[i] * scale_log2 : ninf;
      cm = fmaxf(cm, sv[i]);
    }
    cm = max_x32(max_x16(cm));   // the chunk maximum of head c16, in all four of its lanes
    const float mn = fmaxf(m, cm);
    if (__ballot(c16 < G && mn > m + kLazyLog2)) {   // wave-uniform
      const float al = (mn == ninf) ? 1.0f : exp2f(m - mn);   // 0 while m = -inf
      lsum *= al;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // accumulator row i of this lane is head 4*g4 + i, whose factor lane 4*g4 + i holds
        const float a = __int_as_float(__builtin_amdgcn_ds_bpermute((4 * g4 + i) << 2, __float_as_int(al)));
#pragma unroll
        for (int q = 0; q < 8; ++q) o[q][i] *= a;
      }
      m = mn;
    }
    const float ms = (m == ninf) ? 0.0f : m;
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = exp2f(sv[i] - ms);   // 0 for masked slots
      lsum += p[i];
    }
    const u32x2_t pa = pack4_half<F16>(p);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int at = ((16 * q + c16) * kVtStride + 4 * g4) >> 1;
      const u32x2_t w = {vt32[at], vt32[at + 1]};
      o[q] = mfma_16x16x16<F16>(pa, w, o[q]);
    }
    pin(lsum);
  };

  // Chunk pipeline as in sparse_attn_kernel.
  constexpr int P = kDepth - 1;
  u32x4_t kx[kDepth][4], vx[kDepth][4];
  uint32_t vm[kDepth];
  int id_next = -1;
  {
    int id = load_id(0);
#pragma unroll
    for (int c = 0; c < P && c < n_it; ++c) {
      const int idn = c + 1 < n_it ? load_id(c + 1) : -1;
      gather(token_of(c, id), kx[c], vx[c], vm[c]);
      id = idn;
    }
    id_next = id;
  }
#pragma unroll
  for (int c0 = 0; c0 < n_it; c0 += kDepth) {
#pragma unroll
    for (int u = 0; u < kDepth; ++u) {
      const int c = c0 + u;
      if (c >= n_it) break;
      const int nxt = (u + P) % kDepth;
      __builtin_amdgcn_sched_barrier(0);
      if (c + P < n_it) {
        const int dz = c > 0 ? zero_after(lsum) : 0;
        const int tn = token_of(c + P, id_next + dz);
        if (c + P + 1 < n_it) id_next = load_id(c + P + 1 + dz);
        gather(tn, kx[nxt], vx[nxt], vm[nxt]);
      }
      __builtin_amdgcn_sched_barrier(0);
      compute(kx[u], vx[u], vm[u]);
    }
  }

  // The four lanes of a head hold the same maximum; their sums add up.
  const float lw = sum_x32(sum_x16(lsum));
  if (lane < G) {
    red_m[wave][lane] = m;
    red_l[wave][lane] = lw;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int h = 4 * g4 + i;
    if (h < G) {
#pragma unroll
      for (int q = 0; q < 8; ++q) red_acc[wave][h][16 * q + c16] = o[q][i];
    }
  }
  __syncthreads();
  finish_workgroup<G, NW, F16>(red_acc, red_m, red_l, last_flag, r, split, a.nsplit,
                          a.out + (static_cast<int64_t>(b) * a.q_heads + j * G) * kD, a.ws_acc, a.ws_ml, a.tickets);
}

}  // namespace
}  // namespace qkv
