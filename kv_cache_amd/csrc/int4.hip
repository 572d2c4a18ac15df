// int4 K cache: quantize/pack, static channel subset, subset slab, and the
// decode scoring kernel fused with block max-pooling.
//
// The reference scores fp32 over GQA-expanded bf16 K (qabs_cuda_kernels.py:
// 63-158) and keeps a transposed bf16 K copy for it (evaluate_qwen3_top2_
// head_limit3_ppl.py:2018-2042).  Here the scored stream is an int4 slab of
// S channels per token (S/2 bytes + one fp16 scale), read once with 128-bit
// loads; the dot is v_dot4_i32_i8 on nibbles shifted into the high half of
// each byte, so no sign-extension or bias pass is needed.
//
// Built with -ffp-contract=off: the ranking key fp32(scale) * fp32(I) is a
// single IEEE multiply, identical to the CPU oracle.
#include <algorithm>

#include "common.h"

#ifndef QKV_SCORE_TARGET_WGS
#define QKV_SCORE_TARGET_WGS 4096
#endif
// Waves per decode-scoring workgroup (the kernel has no workgroup barrier:
// the waves only share the workgroup's chunk of the row).
#ifndef QKV_SCORE_WAVES
#define QKV_SCORE_WAVES 4
#endif

namespace qkv {
namespace {

constexpr int kThreads = 256;
constexpr int kScoreWaves = QKV_SCORE_WAVES;
constexpr int kScoreThreads = 64 * kScoreWaves;

// Exact fp16 value times 2^24 (every finite fp16 is a multiple of 2^-24).
__device__ __forceinline__ uint64_t fp16_fixed24(uint32_t bits) {
  uint32_t e = (bits >> 10) & 0x1Fu;
  uint32_t m = bits & 0x3FFu;
  if (e == 0) return m;
  return static_cast<uint64_t>(1024u + m) << (e - 1);
}

__device__ __forceinline__ void bf16x8(const uint4& raw, float* x) {
  x[0] = bf16lo(raw.x); x[1] = bf16hi(raw.x);
  x[2] = bf16lo(raw.y); x[3] = bf16hi(raw.y);
  x[4] = bf16lo(raw.z); x[5] = bf16hi(raw.z);
  x[6] = bf16lo(raw.w); x[7] = bf16hi(raw.w);
}

// Quantizes 8 values against the group amax `a` (already reduced) and packs
// them into one little-endian word of nibbles (channel i at bits 4i..4i+3).
__device__ __forceinline__ uint32_t quantize8(const float* x, float a, uint32_t* sbits_out) {
  uint32_t sbits = f32_to_f16bits_sat(a / 7.0f);
  float s = f16bits_to_f32(sbits);
  uint32_t word = 0;
  if (s != 0.0f) {
#pragma unroll
    for (int i = 0; i < 8; ++i) word |= (static_cast<uint32_t>(int4_code(x[i], s)) & 0xFu) << (4 * i);
  }
  *sbits_out = sbits;
  return word;
}

// ---------------------------------------------------------------------------
// Pack: one thread per 8 channels of a token; GROUP/8 lanes share a scale.
// ---------------------------------------------------------------------------
template <int GROUP>
__global__ __launch_bounds__(kThreads) void pack_kernel(
    const uint16_t* __restrict__ key, int64_t ksb, int64_t ksh, int64_t kst, int kv_heads,
    int t_begin, int ntok, int head_dim, uint8_t* __restrict__ packed,
    uint16_t* __restrict__ scales, int64_t capacity, int64_t total) {
  constexpr int TPG = GROUP / 8;
  const int tpt = head_dim / 8;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const bool active = gid < total;
  const int64_t g = active ? gid : 0;
  const int64_t tok_lin = g / tpt;
  const int c8 = static_cast<int>(g - tok_lin * tpt);
  const int64_t r = tok_lin / ntok;
  const int t = t_begin + static_cast<int>(tok_lin - r * ntok);
  const int b = static_cast<int>(r / kv_heads), h = static_cast<int>(r % kv_heads);
  uint4 raw = make_uint4(0, 0, 0, 0);
  if (active) raw = *reinterpret_cast<const uint4*>(key + b * ksb + h * ksh + t * kst + c8 * 8);
  float x[8];
  bf16x8(raw, x);
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) a = fmaxf(a, fabsf(x[i]));
#pragma unroll
  for (int m = 1; m < TPG; m <<= 1) a = fmaxf(a, shfl_xor(a, m));
  uint32_t sbits;
  uint32_t word = quantize8(x, a, &sbits);
  if (active) {
    const int64_t tok = r * capacity + t;
    reinterpret_cast<uint32_t*>(packed)[tok * tpt + c8] = word;
    if (c8 % TPG == 0) scales[tok * (head_dim / GROUP) + c8 / TPG] = static_cast<uint16_t>(sbits);
  }
}

// ---------------------------------------------------------------------------
// Channel statistic: sum_t |code| * F(scale), exact in uint64 (atomics are
// order-free on integers, so the result is deterministic).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void zero_u64_kernel(uint64_t* p, int64_t n) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  if (i < n) p[i] = 0;
}

__global__ __launch_bounds__(kThreads) void channel_stats_kernel(
    const uint8_t* __restrict__ packed, const uint16_t* __restrict__ scales, int tokens,
    int64_t capacity, int head_dim, int group, int chunk, uint64_t* __restrict__ stats) {
  __shared__ uint64_t part[kThreads * 8];
  const int r = blockIdx.y;
  const int tpt = head_dim / 8;          // threads per token
  const int rows_per_iter = kThreads / tpt;
  const int c8 = threadIdx.x % tpt, tl = threadIdx.x / tpt;
  const int t0 = blockIdx.x * chunk, t1 = min(tokens, t0 + chunk);
  const int spt = head_dim / group;
  uint64_t acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const uint32_t* words = reinterpret_cast<const uint32_t*>(packed);
  for (int t = t0 + tl; t < t1; t += rows_per_iter) {
    const int64_t tok = static_cast<int64_t>(r) * capacity + t;
    uint32_t w = words[tok * tpt + c8];
    uint64_t f = fp16_fixed24(scales[tok * spt + (c8 * 8) / group]);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      int c = static_cast<int>(w << (28 - 4 * i)) >> 28;   // sign-extend nibble i
      acc[i] += f * static_cast<uint64_t>(c < 0 ? -c : c);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) part[tl * head_dim + c8 * 8 + i] = acc[i];
  __syncthreads();
  for (int c = threadIdx.x; c < head_dim; c += kThreads) {
    uint64_t s = 0;
    for (int row = 0; row < rows_per_iter; ++row) s += part[row * head_dim + c];
    if (s) atomicAdd(reinterpret_cast<unsigned long long*>(stats + static_cast<int64_t>(r) * head_dim + c),
                     static_cast<unsigned long long>(s));
  }
}

// One wave per row: rank(c) = #{e : st[e] > st[c] or (st[e] == st[c] and e < c)};
// the channels of rank < S are written in ascending channel order.
__global__ __launch_bounds__(64) void select_channels_kernel(const uint64_t* __restrict__ stats,
                                                             int head_dim, int selected,
                                                             int32_t* __restrict__ chan_idx) {
  __shared__ uint64_t st[256];
  const int r = blockIdx.x, lane = threadIdx.x;
  for (int c = lane; c < head_dim; c += 64) st[c] = stats[static_cast<int64_t>(r) * head_dim + c];
  __syncthreads();
  int base = 0;
  for (int c0 = 0; c0 < head_dim; c0 += 64) {
    const int c = c0 + lane;
    bool sel = false;
    if (c < head_dim) {
      const uint64_t v = st[c];
      int rank = 0;
      for (int e = 0; e < head_dim; ++e) rank += (st[e] > v) || (st[e] == v && e < c);
      sel = rank < selected;
    }
    const uint64_t mask = __ballot(sel);
    if (sel) {
      int pos = base + __popcll(mask & ((1ull << lane) - 1ull));
      chan_idx[static_cast<int64_t>(r) * selected + pos] = c;
    }
    base += __popcll(mask);
  }
}

// ---------------------------------------------------------------------------
// Subset slab: S/8 lanes per token, each gathers 8 selected channels.
//
// The slab's codes are stored in tiles of 4096 bytes = 64 lanes x 4 chunks of
// 16 bytes, one tile per 8192/S keys.  Lane l of a tile owns the 128/S
// consecutive keys [l * 128/S, (l+1) * 128/S), i.e. 64 logical bytes; its
// logical byte b sits at tile offset (64 * (b / 16) + l) * 16 + b % 16.  A
// wave reading chunk 64j + l in load j therefore issues fully coalesced
// 16-byte loads and still ends with whole, consecutive keys in each lane.
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int64_t slab_tile_keys(int s) { return 8192 / s; }

// Byte offset, within a row's slab, of logical code byte x of key t.
template <int S>
__device__ __forceinline__ int64_t slab_offset(int64_t t, int x) {
  constexpr int KPLN = 128 / S;            // keys per lane
  const int64_t tile = t / slab_tile_keys(S);
  const int k = static_cast<int>(t - tile * slab_tile_keys(S));
  const int lane = k / KPLN;
  const int b = (k - lane * KPLN) * (S / 2) + x;
  return tile * 4096 + (64 * (b >> 4) + lane) * 16 + (b & 15);
}
template <int S>
__global__ __launch_bounds__(kThreads) void build_slab_kernel(
    const uint16_t* __restrict__ key, int64_t ksb, int64_t ksh, int64_t kst, int kv_heads,
    int t_begin, int ntok, int head_dim, const int32_t* __restrict__ chan_idx,
    uint8_t* __restrict__ slab, uint16_t* __restrict__ slab_scales, int64_t capacity, int64_t total) {
  constexpr int TPT = S / 8;
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  const bool active = gid < total;
  const int64_t g = active ? gid : 0;
  const int64_t tok_lin = g / TPT;
  const int jj = static_cast<int>(g - tok_lin * TPT);
  const int64_t r = tok_lin / ntok;
  const int t = t_begin + static_cast<int>(tok_lin - r * ntok);
  const int b = static_cast<int>(r / kv_heads), h = static_cast<int>(r % kv_heads);
  float x[8];
  const uint16_t* row = key + b * ksb + h * ksh + static_cast<int64_t>(t) * kst;
  const int32_t* idx = chan_idx + r * S + jj * 8;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    // channel ids come from qkv_int4_select_channels; clamping keeps a bad id in the row
    const int c = min(max(active ? idx[i] : 0, 0), head_dim - 1);
    x[i] = active ? bf16_to_f32(row[c]) : 0.0f;
  }
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) a = fmaxf(a, fabsf(x[i]));
#pragma unroll
  for (int m = 1; m < TPT; m <<= 1) a = fmaxf(a, shfl_xor(a, m));
  uint32_t sbits;
  uint32_t word = quantize8(x, a, &sbits);
  if (active) {
    const int64_t tok = r * capacity + t;
    *reinterpret_cast<uint32_t*>(slab + r * capacity * (S / 2) + slab_offset<S>(t, 4 * jj)) = word;
    if (jj == 0) slab_scales[tok] = static_cast<uint16_t>(sbits);
  }
}

// ---------------------------------------------------------------------------
// Decode scoring fused with block max-pooling.
//
// One wave stage is one slab tile: lane l issues four coalesced 16-byte
// non-temporal loads (chunks 64j + l) and one coalesced load of its KPLN
// scales, and then holds whole keys [l*KPLN, (l+1)*KPLN) of the tile.  The
// dot is v_dot4_i32_i8 on nibbles moved to the high half of each byte --
// (w << 4) & 0xF0F0F0F0 for even channels, w & 0xF0F0F0F0 for odd ones -- so
// each byte is 16 * code as a signed int8 and the int32 sum is 16 * I.
// Block maxima are an in-lane max and a DPP reduction over block/KPLN lanes;
// a stage's maxima leave in one store.
// ---------------------------------------------------------------------------
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 ld_nt(const uint4* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

template <int DPP>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP, 0xF, 0xF, false));
}

// Max over aligned groups of n lanes (n a power of two <= 64); every lane of
// a group receives it.  quad_perm xor 1 / xor 2, then row_half_mirror and
// row_mirror pair each quad / half-row with its partner, then 32 and 64.
__device__ __forceinline__ float lanes_max(float v, int n) {
  if (n >= 2) v = fmaxf(v, dpp_f<0xB1>(v));
  if (n >= 4) v = fmaxf(v, dpp_f<0x4E>(v));
  if (n >= 8) v = fmaxf(v, dpp_f<0x141>(v));
  if (n >= 16) v = fmaxf(v, dpp_f<0x140>(v));
  if (n >= 32) v = fmaxf(v, swz_xor<16>(v));
  if (n >= 64) v = fmaxf(v, shfl_xor(v, 32));
  return v;
}

// The KPLN fp16 scales of one lane, loaded with one coalesced load.
template <int KPLN> struct LaneScales;
template <> struct LaneScales<1> {
  uint32_t w[1];
  __device__ void load(const uint16_t* p) { w[0] = __builtin_nontemporal_load(p); }
  __device__ uint32_t get(int) const { return w[0] & 0xFFFFu; }
};
template <> struct LaneScales<2> {
  uint32_t w[1];
  __device__ void load(const uint16_t* p) { w[0] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(p)); }
  __device__ uint32_t get(int i) const { return (w[0] >> (16 * i)) & 0xFFFFu; }
};
template <> struct LaneScales<4> {
  uint32_t w[2];
  __device__ void load(const uint16_t* p) {
    typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
    const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
    w[0] = v.x;
    w[1] = v.y;
  }
  __device__ uint32_t get(int i) const { return (w[i >> 1] >> (16 * (i & 1))) & 0xFFFFu; }
};
template <> struct LaneScales<8> {
  uint32_t w[4];
  __device__ void load(const uint16_t* p) {
    const uint4 v = ld_nt(reinterpret_cast<const uint4*>(p));
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  }
  __device__ uint32_t get(int i) const { return (w[i >> 1] >> (16 * (i & 1))) & 0xFFFFu; }
};

// Per-row int8 query of decode scoring, computed by one wave: q8[s] =
// rint(qg[s] / (amax/127)), qg the fp32 sum of the row's G query heads over
// its channels in head order, amax = max |qg|.  Code dword d of a key holds
// channels 8d..8d+7 (channel 8d+i in nibble i), so qlo[d] packs the int8
// query of its even channels and qhi[d] the odd ones; both arrays and *qs
// come back wave-uniform.
//
// Split in two so that a caller can put other loads between them: the load
// phase issues every global load the query needs (the channel ids and the
// first kQPre head rows, lane l holding channels 2l, 2l+1), the finish phase
// does the arithmetic.  Loads return in issue order, so loads issued after
// the load phase stay in flight while the finish phase waits for its own.
constexpr int kQPre = 8;   // head rows loaded ahead; rows beyond are loaded in the finish phase

template <int S>
struct RowQueryLoads {
  uint32_t w[kQPre];
  int c0, c1;
};

template <int S>
__device__ __forceinline__ RowQueryLoads<S> row_query_load(const uint16_t* __restrict__ query, int q_heads,
                                                           int kv_heads, int head_dim,
                                                           const int32_t* __restrict__ chan_idx, int r) {
  const int lane = threadIdx.x & 63;
  const int G = q_heads / kv_heads;
  const int b = r / kv_heads, j = r - b * kv_heads;
  const int32_t* cidx = chan_idx + static_cast<int64_t>(r) * S;
  const uint32_t* qrow = reinterpret_cast<const uint32_t*>(
      query + (static_cast<int64_t>(b) * q_heads + j * G) * head_dim);
  const int hd2 = head_dim / 2;   // channel pairs per head row
  // Unconditional loads from clamped indices (redundant ones hit in cache);
  // the finish phase ignores the lanes and rows they stand in for.
  RowQueryLoads<S> L;
  L.c0 = cidx[min(lane, S - 1)];
  L.c1 = S > 64 ? cidx[lane + 64] : 0;
  const int lw = min(lane, hd2 - 1);
#pragma unroll
  for (int i = 0; i < kQPre; ++i) L.w[i] = qrow[min(i, G - 1) * hd2 + lw];
  return L;
}

template <int S>
__device__ __forceinline__ void row_query_finish(const RowQueryLoads<S>& L, const uint16_t* __restrict__ query,
                                                 int q_heads, int kv_heads, int head_dim, int r,
                                                 uint32_t (&qlo)[S / 8], uint32_t (&qhi)[S / 8],
                                                 float* qs_out) {
  const int lane = threadIdx.x & 63;
  const int G = q_heads / kv_heads;
  const int hd2 = head_dim / 2;
  // The empty asm keeps every use of the loaded ids here, after whatever
  // loads the caller issued since the load phase.
  int c0 = L.c0, c1 = L.c1;
  asm volatile("" : "+v"(c0), "+v"(c1));
  float lo = 0.0f, hi = 0.0f;     // fp32 head sums of channels 2*lane, 2*lane+1, in head order
#pragma unroll
  for (int i = 0; i < kQPre; ++i) {
    if (i < G) {
      lo = lo + bf16lo(L.w[i]);
      hi = hi + bf16hi(L.w[i]);
    }
  }
  if (lane >= hd2) lo = hi = 0.0f;   // no channel pair: never picked
  if (G > kQPre && lane < hd2) {
    const int b = r / kv_heads, j = r - b * kv_heads;
    const uint32_t* qrow = reinterpret_cast<const uint32_t*>(
        query + (static_cast<int64_t>(b) * q_heads + j * G) * head_dim);
    for (int i = kQPre; i < G; ++i) {
      const uint32_t w = qrow[i * hd2 + lane];
      lo = lo + bf16lo(w);
      hi = hi + bf16hi(w);
    }
  }
  // qg of channel c, read from lane c/2 (ds_bpermute reads only lanes that
  // execute it, so every lane runs it; it takes the lane index modulo 64, so
  // an id outside the row cannot fault).
  auto pick = [&](int c) -> float {
    const float vl = __int_as_float(__builtin_amdgcn_ds_bpermute((c >> 1) << 2, __float_as_int(lo)));
    const float vh = __int_as_float(__builtin_amdgcn_ds_bpermute((c >> 1) << 2, __float_as_int(hi)));
    return (c & 1) ? vh : vl;
  };
  const float p0 = pick(c0);
  const float qg0 = lane < S ? p0 : 0.0f;
  const float qg1 = S > 64 ? pick(c1) : 0.0f;
  const float amax = wave_max_nonneg(fmaxf(fabsf(qg0), fabsf(qg1)));
  const float qs = amax / 127.0f;
  auto q8 = [&](float v) -> uint32_t {
    if (qs == 0.0f) return 0u;
    float t = __builtin_rintf(v / qs);
    return static_cast<uint32_t>(static_cast<int>(fminf(fmaxf(t, -127.0f), 127.0f))) & 0xFFu;
  };
  // Lane s holds the int8 query of subset channel s (s + 64 in the second
  // word).  Three DPP row shifts gather channels s, s+2, s+4, s+6 into lane
  // s's bytes 0..3, so lane 8d holds qlo[d] and lane 8d+1 holds qhi[d]
  // (8d+7 stays inside the lane's row of 16).
  auto gather4 = [](uint32_t b) -> uint32_t {
    return b | (dpp_mov<0x102>(0u, b) << 8) | (dpp_mov<0x104>(0u, b) << 16) | (dpp_mov<0x106>(0u, b) << 24);
  };
  const uint32_t w0 = gather4(q8(qg0));
  const uint32_t w1 = S > 64 ? gather4(q8(qg1)) : 0u;
#pragma unroll
  for (int d = 0; d < S / 8; ++d) {
    const uint32_t w = d < 8 ? w0 : w1;
    const int l = (8 * d) & 63;
    qlo[d] = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(w), l));
    qhi[d] = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(w), l + 1));
  }
  *qs_out = qs;
}

// The row's query words as a table: qwords[2d] = qlo[d], qwords[2d+1] = qhi[d].
template <int S>
__global__ __launch_bounds__(64) void query_words_kernel(
    const uint16_t* __restrict__ query, int q_heads, int kv_heads, int head_dim,
    const int32_t* __restrict__ chan_idx, uint32_t* __restrict__ qwords, float* __restrict__ qscale_out) {
  const int r = blockIdx.x, lane = threadIdx.x;
  uint32_t qlo[S / 8], qhi[S / 8];
  float qs;
  const RowQueryLoads<S> ql = row_query_load<S>(query, q_heads, kv_heads, head_dim, chan_idx, r);
  row_query_finish<S>(ql, query, q_heads, kv_heads, head_dim, r, qlo, qhi, &qs);
  uint32_t* out = qwords + static_cast<int64_t>(r) * (S / 4);
#pragma unroll
  for (int d = 0; d < S / 8; ++d) {
    if (lane == 2 * d) out[2 * d] = qlo[d];
    if (lane == 2 * d + 1) out[2 * d + 1] = qhi[d];
  }
  if (qscale_out && lane == 0) qscale_out[r] = qs;
}

template <int S, bool DEBUG>
__global__ __launch_bounds__(kScoreThreads) void decode_scores_kernel(
    const uint16_t* __restrict__ query, int q_heads, int kv_heads, int head_dim,
    const int32_t* __restrict__ chan_idx, const uint8_t* __restrict__ slab,
    const uint16_t* __restrict__ slab_scales, int64_t capacity, int tokens, int block,
    int chunk, float* __restrict__ bmax, int nb, int32_t* __restrict__ isum,
    float* __restrict__ keys_out, float* __restrict__ qscale_out) {
  constexpr int KPLN = 128 / S;                        // keys per lane per stage
  constexpr int STAGE = static_cast<int>(slab_tile_keys(S));   // keys per wave stage = 64 * KPLN
  constexpr int DW = S / 8;                            // code dwords per key
  using LS = LaneScales<KPLN>;

  const int r = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

  // Every wave builds the row's int8 query itself (a separate per-row kernel
  // costs a launch; sharing one wave's result through LDS puts its latency in
  // front of every wave, measured slower).  Its few loads go out first, the
  // first slab stage's loads right behind them; the query arithmetic then
  // waits only for its own loads and overlaps the slab loads in flight.
  const RowQueryLoads<S> ql = row_query_load<S>(query, q_heads, kv_heads, head_dim, chan_idx, r);
  __builtin_amdgcn_sched_barrier(0);

  const int64_t row_tok = static_cast<int64_t>(r) * capacity;
  const uint4* codes = reinterpret_cast<const uint4*>(slab + row_tok * (S / 2));
  const uint16_t* scl = slab_scales + row_tok;
  const int t_lo = blockIdx.x * chunk;
  const int t_hi = min(tokens, t_lo + chunk);

  // A wave's stages start at t_lo + wave*STAGE and step by kScoreWaves*STAGE;
  // t_lo is a multiple of kScoreWaves*STAGE, so every stage is one whole tile.  A stage with
  // tb < t_hi <= tokens <= capacity lies inside the row's slab and scales
  // (capacity is a multiple of STAGE), so its loads need no per-lane guard:
  // lanes past t_hi read padding that score_stage masks to -inf.  Loads
  // issued without branches let the compiler count them exactly, so a wait
  // for older loads never waits for the stage loads behind them.
  auto load_stage = [&](int tb, uint4 (&cw)[4], LS& sv) {
    const uint4* tile = codes + (static_cast<int64_t>(tb) / STAGE) * 256;
#pragma unroll
    for (int i = 0; i < 4; ++i) cw[i] = ld_nt(tile + i * 64 + lane);
    sv.load(scl + tb + lane * KPLN);
  };

  int tb = t_lo + wave * STAGE;
  if (tb >= t_hi) return;   // wave-uniform; the kernel has no workgroup barrier
  const int nst = (t_hi - tb + kScoreWaves * STAGE - 1) / (kScoreWaves * STAGE);   // stages of this wave
  uint4 cw[4];
  LS sv;
  load_stage(tb, cw, sv);
  __builtin_amdgcn_sched_barrier(0);

  uint32_t qlo[DW], qhi[DW];
  float qs;
  row_query_finish<S>(ql, query, q_heads, kv_heads, head_dim, r, qlo, qhi, &qs);
  if (qscale_out && blockIdx.x == 0 && wave == 0 && lane == 0) qscale_out[r] = qs;

  const float ninf = -__builtin_huge_valf();
  // block <= KPLN: each lane writes KPLN / block maxima; else lanes in groups
  // of blk_lanes share a block and the group's first lane writes it.
  const int blk_lanes = block > KPLN ? block / KPLN : 1;

  auto score_stage = [&](int tbase, const uint4 (&cwr)[4], const LS& svr) {
    const uint32_t w[16] = {cwr[0].x, cwr[0].y, cwr[0].z, cwr[0].w, cwr[1].x, cwr[1].y, cwr[1].z, cwr[1].w,
                            cwr[2].x, cwr[2].y, cwr[2].z, cwr[2].w, cwr[3].x, cwr[3].y, cwr[3].z, cwr[3].w};
    const int k0 = tbase + lane * KPLN;
    float key[KPLN];
#pragma unroll
    for (int e = 0; e < KPLN; ++e) {
      int acc = 0;
#pragma unroll
      for (int d = 0; d < DW; ++d) {
        const uint32_t x = w[e * DW + d];
        acc = __builtin_amdgcn_sdot4(static_cast<int>(qlo[d]), static_cast<int>((x << 4) & 0xF0F0F0F0u), acc, false);
        acc = __builtin_amdgcn_sdot4(static_cast<int>(qhi[d]), static_cast<int>(x & 0xF0F0F0F0u), acc, false);
      }
      const int isc = acc >> 4;   // exact: every term is a multiple of 16
      float kf = f16bits_to_f32(svr.get(e)) * static_cast<float>(isc);
      kf = (kf == 0.0f) ? 0.0f : kf;
      // Keys past this workgroup's range (the row end or the next chunk)
      // take no part: blocks never straddle chunks, which are whole stages.
      const int t = k0 + e;
      if (t >= t_hi) kf = ninf;
      key[e] = kf;
      if (DEBUG && t < t_hi) {
        isum[static_cast<int64_t>(r) * tokens + t] = isc;
        keys_out[static_cast<int64_t>(r) * tokens + t] = kf;
      }
    }
    if (bmax) {
      float* brow = bmax + static_cast<int64_t>(r) * nb;
      if (block <= KPLN) {
#pragma unroll
        for (int e0 = 0; e0 < KPLN; e0 += 1) {
          if (e0 % block) continue;
          float m = key[e0];
          for (int e = 1; e < block; ++e) m = fmaxf(m, key[e0 + e]);
          if (k0 + e0 < t_hi) brow[(k0 + e0) / block] = m;
        }
      } else {
        float m = key[0];
#pragma unroll
        for (int e = 1; e < KPLN; ++e) m = fmaxf(m, key[e]);
        m = lanes_max(m, blk_lanes);
        if ((lane % blk_lanes) == 0 && k0 < t_hi) brow[k0 / block] = m;
      }
    }
  };

  // Each wave walks its stages with the next stage's loads in flight.
  for (int i = 1; i < nst; ++i) {
    const int tn = tb + kScoreWaves * STAGE;
    uint4 nw[4];
    LS nsv;
    load_stage(tn, nw, nsv);
    score_stage(tb, cw, sv);
#pragma unroll
    for (int u = 0; u < 4; ++u) cw[u] = nw[u];
    sv = nsv;
    tb = tn;
  }
  score_stage(tb, cw, sv);
}

template <bool DEBUG>
int launch_scores(int S, dim3 grid, hipStream_t st, const uint16_t* q, int hq, int hkv, int d,
                  const int32_t* ci, const uint8_t* slab, const uint16_t* ss, int64_t cap, int T,
                  int block, int chunk, float* bmax, int nb, int32_t* isum, float* keys, float* qs) {
  switch (S) {
#define QKV_CASE(SS)                                                                               \
  case SS:                                                                                         \
    decode_scores_kernel<SS, DEBUG><<<grid, kScoreThreads, 0, st>>>(q, hq, hkv, d, ci, slab, ss, cap, T, \
                                                               block, chunk, bmax, nb, isum, keys, \
                                                               qs);                                \
    break;
    QKV_CASE(16) QKV_CASE(32) QKV_CASE(64) QKV_CASE(128)
#undef QKV_CASE
    default: return fail(QKV_ERR_UNSUPPORTED, "selected channel count %d not built", S);
  }
  return check_launch("qkv_int4_decode_scores");
}

bool pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

}  // namespace
}  // namespace qkv

using namespace qkv;

QKV_EXPORT int qkv_int4_pack_k(const void* key, const int64_t* k_strides, int64_t batch,
                               int64_t kv_heads, int64_t t_begin, int64_t t_end, int64_t head_dim,
                               int64_t group, uint8_t* packed, uint16_t* scales, int64_t capacity,
                               void* stream) {
  if (!key || !k_strides || !packed || !scales) return fail(QKV_ERR_INVALID, "qkv_int4_pack_k: null pointer");
  if (batch <= 0 || kv_heads <= 0 || t_begin < 0 || t_end < t_begin || t_end > capacity)
    return fail(QKV_ERR_INVALID, "qkv_int4_pack_k: bad token range [%lld, %lld) for capacity %lld",
                (long long)t_begin, (long long)t_end, (long long)capacity);
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(QKV_ERR_UNSUPPORTED, "qkv_int4_pack_k: head_dim must be 64, 128 or 256");
  if ((group != 32 && group != 64 && group != 128) || head_dim % group)
    return fail(QKV_ERR_INVALID, "qkv_int4_pack_k: group must be 32, 64 or 128 and divide head_dim");
  if (!aligned(key, 16) || (k_strides[0] | k_strides[1] | k_strides[2]) % 8)
    return fail(QKV_ERR_INVALID, "qkv_int4_pack_k: K rows must be 16-byte aligned");
  if (capacity % 64 || !aligned(packed, 16) || !aligned(scales, 16))
    return fail(QKV_ERR_INVALID, "qkv_int4_pack_k: capacity must be a multiple of 64 and outputs 16-byte aligned");
  const int64_t ntok = t_end - t_begin;
  if (ntok == 0) return QKV_OK;
  const int64_t total = batch * kv_heads * ntok * (head_dim / 8);
  dim3 grid(static_cast<unsigned>(cdiv(total, kThreads)));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* k = static_cast<const uint16_t*>(key);
#define QKV_PACK(GG)                                                                                  \
  pack_kernel<GG><<<grid, kThreads, 0, st>>>(k, k_strides[0], k_strides[1], k_strides[2],            \
                                             static_cast<int>(kv_heads), static_cast<int>(t_begin),  \
                                             static_cast<int>(ntok), static_cast<int>(head_dim),     \
                                             packed, scales, capacity, total)
  if (group == 32) QKV_PACK(32);
  else if (group == 64) QKV_PACK(64);
  else QKV_PACK(128);
#undef QKV_PACK
  return check_launch("qkv_int4_pack_k");
}

QKV_EXPORT int qkv_int4_select_channels(const uint8_t* packed, const uint16_t* scales, int64_t rows,
                                        int64_t tokens, int64_t capacity, int64_t head_dim,
                                        int64_t group, int64_t selected, uint64_t* stats,
                                        int32_t* chan_idx, void* stream) {
  if (!packed || !scales || !stats || !chan_idx)
    return fail(QKV_ERR_INVALID, "qkv_int4_select_channels: null pointer");
  if (rows <= 0 || rows > 65535 || tokens <= 0 || tokens > capacity || tokens > (int64_t(1) << 20))
    return fail(QKV_ERR_INVALID, "qkv_int4_select_channels: need 1 <= tokens <= min(capacity, 2^20), rows <= 65535");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(QKV_ERR_UNSUPPORTED, "qkv_int4_select_channels: head_dim must be 64, 128 or 256");
  if ((group != 32 && group != 64 && group != 128) || head_dim % group)
    return fail(QKV_ERR_INVALID, "qkv_int4_select_channels: bad group");
  if (selected < 1 || selected > head_dim)
    return fail(QKV_ERR_INVALID, "qkv_int4_select_channels: selected must be in [1, head_dim]");
  if (capacity % 64) return fail(QKV_ERR_INVALID, "qkv_int4_select_channels: capacity must be a multiple of 64");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t n = rows * head_dim;
  zero_u64_kernel<<<static_cast<unsigned>(cdiv(n, kThreads)), kThreads, 0, st>>>(stats, n);
  int rc = check_launch("qkv_int4_select_channels(zero)");
  if (rc) return rc;
  const int chunk = 4096;
  dim3 grid(static_cast<unsigned>(cdiv(tokens, chunk)), static_cast<unsigned>(rows));
  channel_stats_kernel<<<grid, kThreads, 0, st>>>(packed, scales, static_cast<int>(tokens), capacity,
                                                  static_cast<int>(head_dim), static_cast<int>(group),
                                                  chunk, stats);
  rc = check_launch("qkv_int4_select_channels(stats)");
  if (rc) return rc;
  select_channels_kernel<<<static_cast<unsigned>(rows), 64, 0, st>>>(stats, static_cast<int>(head_dim),
                                                                     static_cast<int>(selected), chan_idx);
  return check_launch("qkv_int4_select_channels(select)");
}

QKV_EXPORT int qkv_int4_build_slab(const void* key, const int64_t* k_strides, int64_t batch,
                                   int64_t kv_heads, int64_t t_begin, int64_t t_end,
                                   int64_t head_dim, const int32_t* chan_idx, int64_t selected,
                                   uint8_t* slab, uint16_t* slab_scales, int64_t capacity,
                                   void* stream) {
  if (!key || !k_strides || !chan_idx || !slab || !slab_scales)
    return fail(QKV_ERR_INVALID, "qkv_int4_build_slab: null pointer");
  if (batch <= 0 || kv_heads <= 0 || t_begin < 0 || t_end < t_begin || t_end > capacity)
    return fail(QKV_ERR_INVALID, "qkv_int4_build_slab: bad token range");
  if (selected != 16 && selected != 32 && selected != 64 && selected != 128)
    return fail(QKV_ERR_UNSUPPORTED, "qkv_int4_build_slab: selected must be 16, 32, 64 or 128");
  if (selected > head_dim) return fail(QKV_ERR_INVALID, "qkv_int4_build_slab: selected > head_dim");
  if (capacity % slab_tile_keys(static_cast<int>(selected)) || !aligned(slab, 16) || !aligned(slab_scales, 16))
    return fail(QKV_ERR_INVALID, "qkv_int4_build_slab: capacity must be a multiple of %lld and outputs 16-byte aligned",
                (long long)slab_tile_keys(static_cast<int>(selected)));
  const int64_t ntok = t_end - t_begin;
  if (ntok == 0) return QKV_OK;
  const int64_t total = batch * kv_heads * ntok * (selected / 8);
  dim3 grid(static_cast<unsigned>(cdiv(total, kThreads)));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* k = static_cast<const uint16_t*>(key);
#define QKV_SLAB(SS)                                                                                 \
  build_slab_kernel<SS><<<grid, kThreads, 0, st>>>(k, k_strides[0], k_strides[1], k_strides[2],     \
                                                   static_cast<int>(kv_heads), static_cast<int>(t_begin), \
                                                   static_cast<int>(ntok), static_cast<int>(head_dim),   \
                                                   chan_idx, slab, slab_scales,                        \
                                                   capacity, total)
  switch (selected) {
    case 16: QKV_SLAB(16); break;
    case 32: QKV_SLAB(32); break;
    case 64: QKV_SLAB(64); break;
    default: QKV_SLAB(128); break;
  }
#undef QKV_SLAB
  return check_launch("qkv_int4_build_slab");
}

// Shared argument checks of the query side (scoring and query words).
static int check_query(const void* query, int64_t batch, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                const int32_t* chan_idx, int64_t selected, const char* what) {
  if (!query || !chan_idx) return fail(QKV_ERR_INVALID, "%s: null query pointer", what);
  if (batch <= 0 || kv_heads <= 0 || q_heads % kv_heads)
    return fail(QKV_ERR_INVALID, "%s: q_heads must be a multiple of kv_heads", what);
  if (batch * kv_heads > 65535) return fail(QKV_ERR_INVALID, "%s: too many rows", what);
  if (head_dim != 64 && head_dim != 128) return fail(QKV_ERR_UNSUPPORTED, "%s: head_dim must be 64 or 128", what);
  if (selected != 16 && selected != 32 && selected != 64 && selected != 128)
    return fail(QKV_ERR_UNSUPPORTED, "%s: selected must be 16, 32, 64 or 128", what);
  if (selected > head_dim) return fail(QKV_ERR_INVALID, "%s: selected > head_dim", what);
  if (!aligned(query, 4)) return fail(QKV_ERR_INVALID, "%s: query must be 4-byte aligned", what);
  return QKV_OK;
}

QKV_EXPORT int qkv_int4_query_words(const void* query, int64_t batch, int64_t q_heads,
                                    int64_t kv_heads, int64_t head_dim, const int32_t* chan_idx,
                                    int64_t selected, uint32_t* qwords, float* qscale, void* stream) {
  if (int rc = check_query(query, batch, q_heads, kv_heads, head_dim, chan_idx, selected, "qkv_int4_query_words"))
    return rc;
  if (!qwords) return fail(QKV_ERR_INVALID, "qkv_int4_query_words: null qwords pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned grid = static_cast<unsigned>(batch * kv_heads);
  const uint16_t* q = static_cast<const uint16_t*>(query);
  const int hq = static_cast<int>(q_heads), hkv = static_cast<int>(kv_heads), hd = static_cast<int>(head_dim);
  switch (selected) {
    case 16: query_words_kernel<16><<<grid, 64, 0, st>>>(q, hq, hkv, hd, chan_idx, qwords, qscale); break;
    case 32: query_words_kernel<32><<<grid, 64, 0, st>>>(q, hq, hkv, hd, chan_idx, qwords, qscale); break;
    case 64: query_words_kernel<64><<<grid, 64, 0, st>>>(q, hq, hkv, hd, chan_idx, qwords, qscale); break;
    default: query_words_kernel<128><<<grid, 64, 0, st>>>(q, hq, hkv, hd, chan_idx, qwords, qscale); break;
  }
  return check_launch("qkv_int4_query_words");
}

QKV_EXPORT int qkv_int4_decode_scores(const void* query, int64_t batch, int64_t q_heads,
                                      int64_t kv_heads, int64_t head_dim, const int32_t* chan_idx,
                                      int64_t selected, const uint8_t* slab,
                                      const uint16_t* slab_scales, int64_t capacity, int64_t tokens,
                                      int64_t block, float* bmax, int32_t* isum, float* keys,
                                      float* qscale, void* stream) {
  if (int rc = check_query(query, batch, q_heads, kv_heads, head_dim, chan_idx, selected,
                           "qkv_int4_decode_scores"))
    return rc;
  if (!slab || !slab_scales) return fail(QKV_ERR_INVALID, "qkv_int4_decode_scores: null slab pointer");
  if (!bmax && !(isum && keys))
    return fail(QKV_ERR_INVALID, "qkv_int4_decode_scores: need bmax or both isum and keys");
  if ((isum == nullptr) != (keys == nullptr))
    return fail(QKV_ERR_INVALID, "qkv_int4_decode_scores: isum and keys go together");
  if (tokens <= 0 || tokens > capacity || tokens >= (int64_t(1) << 30))
    return fail(QKV_ERR_INVALID, "qkv_int4_decode_scores: need 1 <= tokens <= capacity");
  if (!aligned(slab, 16) || !aligned(slab_scales, 16))
    return fail(QKV_ERR_INVALID, "qkv_int4_decode_scores: slab and scales must be 16-byte aligned");
  if (capacity % slab_tile_keys(static_cast<int>(selected)))
    return fail(QKV_ERR_INVALID, "qkv_int4_decode_scores: capacity must be a multiple of %lld for %lld channels",
                (long long)slab_tile_keys(static_cast<int>(selected)), (long long)selected);
  const int stage = static_cast<int>(slab_tile_keys(static_cast<int>(selected)));   // keys per wave stage
  if (!pow2(block) || block > stage)
    return fail(QKV_ERR_INVALID, "qkv_int4_decode_scores: block must be a power of two <= %d", stage);
  const int64_t rows = batch * kv_heads;
  const int stage_wg = kScoreWaves * stage;   // keys one workgroup stage covers
  int64_t chunk = cdiv(rows * tokens, QKV_SCORE_TARGET_WGS);
  chunk = std::max<int64_t>(stage_wg, cdiv(chunk, stage_wg) * stage_wg);
  dim3 grid(static_cast<unsigned>(cdiv(tokens, chunk)), static_cast<unsigned>(rows));
  const int nb = static_cast<int>(cdiv(tokens, block));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* q = static_cast<const uint16_t*>(query);
  const int hq = static_cast<int>(q_heads), hkv = static_cast<int>(kv_heads), hd = static_cast<int>(head_dim);
  if (isum)
    return launch_scores<true>(static_cast<int>(selected), grid, st, q, hq, hkv, hd, chan_idx, slab, slab_scales,
                               capacity, static_cast<int>(tokens), static_cast<int>(block),
                               static_cast<int>(chunk), bmax, nb, isum, keys, qscale);
  return launch_scores<false>(static_cast<int>(selected), grid, st, q, hq, hkv, hd, chan_idx, slab, slab_scales,
                              capacity, static_cast<int>(tokens), static_cast<int>(block),
                              static_cast<int>(chunk), bmax, nb, nullptr, nullptr, qscale);
}
