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

#include "score.h"
#include "window.h"

#ifndef QKV_SCORE_TARGET_WGS
#define QKV_SCORE_TARGET_WGS 4096
#endif

namespace qkv {
namespace {

constexpr int kThreads = 256;

// Exact fp16 value times 2^24 (every finite fp16 is a multiple of 2^-24).
__device__ __forceinline__ uint64_t fp16_fixed24(uint32_t bits) {
  uint32_t e = (bits >> 10) & 0x1Fu;
  uint32_t m = bits & 0x3FFu;
  if (e == 0) return m;
  return static_cast<uint64_t>(1024u + m) << (e - 1);
}

// Eight bf16 (or, with F16, fp16) channels of a 16-byte load, widened exactly.
template <bool F16>
__device__ __forceinline__ void halfx8(const uint4& raw, float* x) {
  x[0] = half_lo<F16>(raw.x); x[1] = half_hi<F16>(raw.x);
  x[2] = half_lo<F16>(raw.y); x[3] = half_hi<F16>(raw.y);
  x[4] = half_lo<F16>(raw.z); x[5] = half_hi<F16>(raw.z);
  x[6] = half_lo<F16>(raw.w); x[7] = half_hi<F16>(raw.w);
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
template <int GROUP, bool F16>
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
  halfx8<F16>(raw, x);
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
template <int S, bool F16>
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
    x[i] = active ? half_to_f32<F16>(row[c]) : 0.0f;
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

// The row's query words as a table: qwords[2d] = qlo[d], qwords[2d+1] = qhi[d].
template <int S, bool F16>
__global__ __launch_bounds__(64) void query_words_kernel(
    const uint16_t* __restrict__ query, int q_heads, int kv_heads, int head_dim,
    const int32_t* __restrict__ chan_idx, uint32_t* __restrict__ qwords, float* __restrict__ qscale_out) {
  const int r = blockIdx.x, lane = threadIdx.x;
  uint32_t qlo[S / 8], qhi[S / 8];
  float qs;
  const RowQueryLoads<S> ql = row_query_load<S>(query, q_heads, kv_heads, head_dim, chan_idx, r);
  row_query_finish<S, F16>(ql, query, q_heads, kv_heads, head_dim, r, qlo, qhi, &qs);
  uint32_t* out = qwords + static_cast<int64_t>(r) * (S / 4);
#pragma unroll
  for (int d = 0; d < S / 8; ++d) {
    if (lane == 2 * d) out[2 * d] = qlo[d];
    if (lane == 2 * d + 1) out[2 * d + 1] = qhi[d];
  }
  if (qscale_out && lane == 0) qscale_out[r] = qs;
}

template <int S, bool DEBUG, bool F16>
__global__ __launch_bounds__(kScoreThreads) void decode_scores_kernel(
    const uint16_t* __restrict__ query, int q_heads, int kv_heads, int head_dim,
    const int32_t* __restrict__ chan_idx, const uint8_t* __restrict__ slab,
    const uint16_t* __restrict__ slab_scales, int64_t capacity, int tokens, int block,
    int chunk, float* __restrict__ bmax, int nb, int32_t* __restrict__ isum,
    float* __restrict__ keys_out, float* __restrict__ qscale_out) {
  score_chunk<S, DEBUG, F16>(query, q_heads, kv_heads, head_dim, chan_idx, slab, slab_scales, capacity, tokens,
                               block, chunk, bmax, nb, isum, keys_out, qscale_out, blockIdx.y, blockIdx.x);
}

template <bool DEBUG, bool F16>
int launch_scores(int S, dim3 grid, hipStream_t st, const uint16_t* q, int hq, int hkv, int d,
                  const int32_t* ci, const uint8_t* slab, const uint16_t* ss, int64_t cap, int T,
                  int block, int chunk, float* bmax, int nb, int32_t* isum, float* keys, float* qs) {
  switch (S) {
#define QKV_CASE(SS)                                                                               \
  case SS:                                                                                         \
    decode_scores_kernel<SS, DEBUG, F16><<<grid, kScoreThreads, 0, st>>>(q, hq, hkv, d, ci, slab, ss, cap, T, \
                                                               block, chunk, bmax, nb, isum, keys, \
                                                               qs);                                \
    break;
    QKV_CASE(16) QKV_CASE(32) QKV_CASE(64) QKV_CASE(128)
#undef QKV_CASE
    default: return fail(QKV_ERR_UNSUPPORTED, "selected channel count %d not built", S);
  }
  return check_launch("qkv_int4_decode_scores");
}

// Decode scoring of qkv_int4_decode_topk: token scores (block 1), one
// workgroup per 4096-key chunk of the long-row top-k, each key also counted
// in the chunk's 12-bit histogram in LDS, and the chunk's top-k window
// (chunk_window) written where qkv_topk_ws's histogram pass would write it.
// win_waves: the chunk's waves, every wave stage one whole slab tile.
constexpr int win_waves(int s) {
  return kStageChunk / slab_tile_keys(s) >= 16 ? 16 : static_cast<int>(kStageChunk / slab_tile_keys(s));
}

template <int S, bool F16>
__global__ __launch_bounds__(64 * win_waves(S)) void decode_scores_win_kernel(
    const uint16_t* __restrict__ query, int q_heads, int kv_heads, int head_dim,
    const int32_t* __restrict__ chan_idx, const uint8_t* __restrict__ slab,
    const uint16_t* __restrict__ slab_scales, int64_t capacity, int tokens, int k, float* __restrict__ scores,
    int n_chunks, int32_t* __restrict__ win, float* __restrict__ qscale_out) {
  constexpr int NWV = win_waves(S), NT = 64 * NWV;
  static_assert(kStageChunk % (NWV * slab_tile_keys(S)) == 0, "a chunk is whole workgroup stages");
  __shared__ uint32_t h[kHistBins];
  __shared__ int wsum[NWV];
  __shared__ int t_sh;
#pragma unroll
  for (int i = 0; i < kHistBins / NT; ++i) h[threadIdx.x + NT * i] = 0;
  if (threadIdx.x == 0) t_sh = 0;
  __syncthreads();
  score_chunk<S, false, F16, NWV>(query, q_heads, kv_heads, head_dim, chan_idx, slab, slab_scales, capacity, tokens,
                                  1, kStageChunk, scores, tokens, nullptr, nullptr, qscale_out, blockIdx.y,
                                  blockIdx.x, h);
  __syncthreads();
  const int len = min(kStageChunk, tokens - static_cast<int>(blockIdx.x) * kStageChunk);
  chunk_window<NT, false>(h, min(k, len), win + (static_cast<int64_t>(blockIdx.y) * n_chunks + blockIdx.x) * kWinWords,
                          wsum, &t_sh);
}

bool pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }

}  // namespace
}  // namespace qkv

using namespace qkv;

QKV_EXPORT int qkv_int4_pack_k(const void* key, const int64_t* k_strides, int64_t batch,
                               int64_t kv_heads, int64_t t_begin, int64_t t_end, int64_t head_dim,
                               int64_t group, uint8_t* packed, uint16_t* scales, int64_t capacity,
                               int dtype, void* stream) {
  if (!key || !k_strides || !packed || !scales) return fail(QKV_ERR_INVALID, "qkv_int4_pack_k: null pointer");
  bool f16;
  if (int rc = half_dtype(dtype, "qkv_int4_pack_k", &f16)) return rc;
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
#define QKV_PACK(GG, FF)                                                                              \
  pack_kernel<GG, FF><<<grid, kThreads, 0, st>>>(k, k_strides[0], k_strides[1], k_strides[2],        \
                                                 static_cast<int>(kv_heads), static_cast<int>(t_begin), \
                                                 static_cast<int>(ntok), static_cast<int>(head_dim),  \
                                                 packed, scales, capacity, total)
  if (f16) {
    if (group == 32) QKV_PACK(32, true);
    else if (group == 64) QKV_PACK(64, true);
    else QKV_PACK(128, true);
  } else {
    if (group == 32) QKV_PACK(32, false);
    else if (group == 64) QKV_PACK(64, false);
    else QKV_PACK(128, false);
  }
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
                                   int dtype, void* stream) {
  if (!key || !k_strides || !chan_idx || !slab || !slab_scales)
    return fail(QKV_ERR_INVALID, "qkv_int4_build_slab: null pointer");
  bool f16;
  if (int rc = half_dtype(dtype, "qkv_int4_build_slab", &f16)) return rc;
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
#define QKV_SLAB(SS, FF)                                                                             \
  build_slab_kernel<SS, FF><<<grid, kThreads, 0, st>>>(k, k_strides[0], k_strides[1], k_strides[2], \
                                                       static_cast<int>(kv_heads), static_cast<int>(t_begin), \
                                                       static_cast<int>(ntok), static_cast<int>(head_dim), \
                                                       chan_idx, slab, slab_scales, capacity, total)
#define QKV_SLAB_ALL(FF)                  \
  switch (selected) {                     \
    case 16: QKV_SLAB(16, FF); break;     \
    case 32: QKV_SLAB(32, FF); break;     \
    case 64: QKV_SLAB(64, FF); break;     \
    default: QKV_SLAB(128, FF); break;    \
  }
  if (f16) QKV_SLAB_ALL(true) else QKV_SLAB_ALL(false)
#undef QKV_SLAB_ALL
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
                                    int64_t selected, uint32_t* qwords, float* qscale, int dtype,
                                    void* stream) {
  if (int rc = check_query(query, batch, q_heads, kv_heads, head_dim, chan_idx, selected, "qkv_int4_query_words"))
    return rc;
  bool f16;
  if (int rc = half_dtype(dtype, "qkv_int4_query_words", &f16)) return rc;
  if (!qwords) return fail(QKV_ERR_INVALID, "qkv_int4_query_words: null qwords pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const unsigned grid = static_cast<unsigned>(batch * kv_heads);
  const uint16_t* q = static_cast<const uint16_t*>(query);
  const int hq = static_cast<int>(q_heads), hkv = static_cast<int>(kv_heads), hd = static_cast<int>(head_dim);
#define QKV_QW(SS, FF) query_words_kernel<SS, FF><<<grid, 64, 0, st>>>(q, hq, hkv, hd, chan_idx, qwords, qscale)
#define QKV_QW_ALL(FF)                \
  switch (selected) {                 \
    case 16: QKV_QW(16, FF); break;   \
    case 32: QKV_QW(32, FF); break;   \
    case 64: QKV_QW(64, FF); break;   \
    default: QKV_QW(128, FF); break;  \
  }
  if (f16) QKV_QW_ALL(true) else QKV_QW_ALL(false)
#undef QKV_QW_ALL
#undef QKV_QW
  return check_launch("qkv_int4_query_words");
}

QKV_EXPORT int qkv_int4_decode_scores(const void* query, int64_t batch, int64_t q_heads,
                                      int64_t kv_heads, int64_t head_dim, const int32_t* chan_idx,
                                      int64_t selected, const uint8_t* slab,
                                      const uint16_t* slab_scales, int64_t capacity, int64_t tokens,
                                      int64_t block, float* bmax, int32_t* isum, float* keys,
                                      float* qscale, int dtype, void* stream) {
  if (int rc = check_query(query, batch, q_heads, kv_heads, head_dim, chan_idx, selected,
                           "qkv_int4_decode_scores"))
    return rc;
  bool f16;
  if (int rc = half_dtype(dtype, "qkv_int4_decode_scores", &f16)) return rc;
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
#define QKV_SC(DBG, FF, IS, KS)                                                                      \
  return launch_scores<DBG, FF>(static_cast<int>(selected), grid, st, q, hq, hkv, hd, chan_idx, slab,  \
                                slab_scales, capacity, static_cast<int>(tokens), static_cast<int>(block), \
                                static_cast<int>(chunk), bmax, nb, IS, KS, qscale)
  if (isum) {
    if (f16) QKV_SC(true, true, isum, keys);
    QKV_SC(true, false, isum, keys);
  }
  if (f16) QKV_SC(false, true, nullptr, nullptr);
  QKV_SC(false, false, nullptr, nullptr);
#undef QKV_SC
}

namespace qkv {
int topk_filtered(const float* values, int64_t rows, int64_t n, int64_t ld, int64_t k, int32_t* out,
                  void* workspace, hipStream_t st, bool given);
bool topk_takes_windows(int64_t n, int64_t k);
}  // namespace qkv

QKV_EXPORT int qkv_int4_decode_topk(const void* query, int64_t batch, int64_t q_heads, int64_t kv_heads,
                                    int64_t head_dim, const int32_t* chan_idx, int64_t selected,
                                    const uint8_t* slab, const uint16_t* slab_scales, int64_t capacity,
                                    int64_t tokens, int64_t k, float* scores, int32_t* out, void* workspace,
                                    int64_t workspace_bytes, int dtype, void* stream) {
  static const char* what = "qkv_int4_decode_topk";
  if (int rc = check_query(query, batch, q_heads, kv_heads, head_dim, chan_idx, selected, what)) return rc;
  bool f16;
  if (int rc = half_dtype(dtype, what, &f16)) return rc;
  if (!slab || !slab_scales || !scores || !out) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  if (tokens <= 0 || tokens > capacity || tokens >= (int64_t(1) << 30))
    return fail(QKV_ERR_INVALID, "%s: need 1 <= tokens <= capacity", what);
  if (k < 1 || k > tokens) return fail(QKV_ERR_INVALID, "%s: need 1 <= k <= tokens", what);
  if (!aligned(slab, 16) || !aligned(slab_scales, 16))
    return fail(QKV_ERR_INVALID, "%s: slab and scales must be 16-byte aligned", what);
  if (capacity % slab_tile_keys(static_cast<int>(selected)))
    return fail(QKV_ERR_INVALID, "%s: capacity must be a multiple of %lld for %lld channels", what,
                (long long)slab_tile_keys(static_cast<int>(selected)), (long long)selected);
  const int64_t rows = batch * kv_heads;
  const int64_t need = qkv_topk_workspace_bytes(rows, tokens, k);
  if (need < 0 || workspace_bytes < need || (need > 0 && !workspace))
    return fail(QKV_ERR_INVALID, "%s: workspace needs %lld bytes, got %lld", what, (long long)need,
                (long long)workspace_bytes);
  if (need > 0 && !aligned(workspace, 16)) return fail(QKV_ERR_INVALID, "%s: workspace must be 16-byte aligned", what);
  if (!topk_takes_windows(tokens, k) || rows > 65535) {   // the scores, then qkv_topk_ws as it stands
    if (int rc = qkv_int4_decode_scores(query, batch, q_heads, kv_heads, head_dim, chan_idx, selected, slab,
                                        slab_scales, capacity, tokens, 1, scores, nullptr, nullptr, nullptr, dtype,
                                        stream))
      return rc;
    return qkv_topk_ws(scores, rows, tokens, tokens, k, out, workspace, workspace_bytes, stream);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int n_chunks = static_cast<int>(cdiv(tokens, kStageChunk));
  dim3 grid(static_cast<unsigned>(n_chunks), static_cast<unsigned>(rows));
  const uint16_t* q = static_cast<const uint16_t*>(query);
  int32_t* win = static_cast<int32_t*>(workspace);   // qkv_topk_ws's window region
  auto launch = [&](auto sc, auto fc) {
    constexpr int SS = decltype(sc)::value;
    constexpr bool FF = decltype(fc)::value;
    decode_scores_win_kernel<SS, FF><<<grid, 64 * win_waves(SS), 0, st>>>(
        q, static_cast<int>(q_heads), static_cast<int>(kv_heads), static_cast<int>(head_dim), chan_idx, slab,
        slab_scales, capacity, static_cast<int>(tokens), static_cast<int>(k), scores, n_chunks, win, nullptr);
    return check_launch(what);
  };
  auto with_f = [&](auto sc) {
    return f16 ? launch(sc, std::true_type{}) : launch(sc, std::false_type{});
  };
  int rc;
  switch (selected) {
    case 16: rc = with_f(std::integral_constant<int, 16>{}); break;
    case 32: rc = with_f(std::integral_constant<int, 32>{}); break;
    case 64: rc = with_f(std::integral_constant<int, 64>{}); break;
    case 128: rc = with_f(std::integral_constant<int, 128>{}); break;
    default: return fail(QKV_ERR_UNSUPPORTED, "%s: selected channel count %lld not built", what, (long long)selected);
  }
  if (rc) return rc;
  return topk_filtered(scores, rows, tokens, tokens, k, out, workspace, st, true);
}
