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
#define QKV_SCORE_TARGET_WGS 2048
#endif
#ifndef QKV_SCORE_UNROLL
#define QKV_SCORE_UNROLL 2
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
// ---------------------------------------------------------------------------
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
    reinterpret_cast<uint32_t*>(slab)[tok * TPT + jj] = word;
    if (jj == 0) slab_scales[tok] = static_cast<uint16_t>(sbits);
  }
}

// ---------------------------------------------------------------------------
// Decode scoring fused with block max-pooling.
//
// Each lane owns KPL = 128/S consecutive keys of a wave tile (64 bytes of
// codes = four 128-bit loads, plus KPL fp16 scales in one load).  Nibble
// pairs are moved to the high half of each byte -- (w << 4) & 0xF0F0F0F0 for
// even channels, w & 0xF0F0F0F0 for odd ones -- so each byte is 16 * code as
// a signed int8, and two v_dot4_i32_i8 per code dword give 16 * I exactly.
// ---------------------------------------------------------------------------
template <int KPL> struct ScaleVec;
template <> struct ScaleVec<1> { using T = uint16_t; static __device__ uint32_t get(T v, int) { return v; } };
template <> struct ScaleVec<2> { using T = uint32_t; static __device__ uint32_t get(T v, int i) { return (v >> (16 * i)) & 0xFFFFu; } };
template <> struct ScaleVec<4> {
  using T = uint2;
  static __device__ uint32_t get(T v, int i) { uint32_t w = (i < 2) ? v.x : v.y; return (w >> (16 * (i & 1))) & 0xFFFFu; }
};
template <> struct ScaleVec<8> {
  using T = uint4;
  static __device__ uint32_t get(T v, int i) {
    uint32_t w = (i < 2) ? v.x : (i < 4) ? v.y : (i < 6) ? v.z : v.w;
    return (w >> (16 * (i & 1))) & 0xFFFFu;
  }
};

template <int S, bool DEBUG>
__global__ __launch_bounds__(kThreads) void decode_scores_kernel(
    const uint16_t* __restrict__ query, int q_heads, int kv_heads, int head_dim,
    const int32_t* __restrict__ chan_idx, const uint8_t* __restrict__ slab,
    const uint16_t* __restrict__ slab_scales, int64_t capacity, int tokens, int block,
    int chunk, float* __restrict__ bmax, int nb, int32_t* __restrict__ isum,
    float* __restrict__ keys_out, float* __restrict__ qscale_out) {
  constexpr int KPL = 128 / S;          // keys per lane
  constexpr int DW = S / 8;             // code dwords per key
  constexpr int TILE = 64 * KPL;        // keys per wave tile
  constexpr int U = QKV_SCORE_UNROLL;   // tiles in flight per wave
  using SV = ScaleVec<KPL>;

  __shared__ uint32_t q_lds[2 * DW];   // per code dword: {even-channel bytes, odd-channel bytes}
  const int r = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = q_heads / kv_heads;
  const int b = r / kv_heads, j = r - b * kv_heads;

  // Prologue (wave 0): q8[s] = rint(qg[s] / (amax/127)), qg = sum of the G heads.
  if (wave == 0) {
    float qg0 = 0.0f, qg1 = 0.0f;
    const int32_t* cidx = chan_idx + static_cast<int64_t>(r) * S;
    const uint16_t* qrow = query + (static_cast<int64_t>(b) * q_heads + j * G) * head_dim;
    if (lane < S) {
      const int c = min(max(cidx[lane], 0), head_dim - 1);
      for (int i = 0; i < G; ++i) qg0 = qg0 + bf16_to_f32(qrow[i * head_dim + c]);
    }
    if (S > 64) {
      const int c = min(max(cidx[lane + 64], 0), head_dim - 1);
      for (int i = 0; i < G; ++i) qg1 = qg1 + bf16_to_f32(qrow[i * head_dim + c]);
    }
    const float amax = wave_max(fmaxf(fabsf(qg0), fabsf(qg1)));
    const float qs = amax / 127.0f;
    auto q8 = [&](float v) -> int {
      if (qs == 0.0f) return 0;
      float t = __builtin_rintf(v / qs);
      return static_cast<int>(fminf(fmaxf(t, -127.0f), 127.0f));
    };
    // byte position of channel s: dword 2*(s/8) + (s&1), byte (s%8)/2
    uint8_t* qb = reinterpret_cast<uint8_t*>(q_lds);
    if (lane < S) qb[8 * (lane >> 3) + 4 * (lane & 1) + ((lane & 7) >> 1)] = static_cast<uint8_t>(q8(qg0));
    if (S > 64) {
      const int s = lane + 64;
      qb[8 * (s >> 3) + 4 * (s & 1) + ((s & 7) >> 1)] = static_cast<uint8_t>(q8(qg1));
    }
    if (qscale_out && blockIdx.x == 0 && lane == 0) qscale_out[r] = qs;
  }
  __syncthreads();
  uint32_t qlo[DW], qhi[DW];
#pragma unroll
  for (int d = 0; d < DW; ++d) {
    qlo[d] = __builtin_amdgcn_readfirstlane(q_lds[2 * d]);
    qhi[d] = __builtin_amdgcn_readfirstlane(q_lds[2 * d + 1]);
  }

  const int64_t row_tok = static_cast<int64_t>(r) * capacity;
  const uint4* codes = reinterpret_cast<const uint4*>(slab) + row_tok * S / 32;
  const typename SV::T* scl = reinterpret_cast<const typename SV::T*>(slab_scales + row_tok);
  const int t_lo = blockIdx.x * chunk;
  const int t_hi = min(tokens, t_lo + chunk);
  const float ninf = -__builtin_huge_valf();
  const int lanes_per_block = block >= KPL ? block / KPL : 1;

  for (int tb = t_lo + wave * TILE * U; tb < t_hi; tb += 4 * TILE * U) {
    uint4 cw[U][4];
    typename SV::T sv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k0 = tb + u * TILE + lane * KPL;
      if (k0 < t_hi) {
#pragma unroll
        for (int i = 0; i < 4; ++i) cw[u][i] = codes[(static_cast<int64_t>(k0) * S) / 32 + i];
        sv[u] = scl[k0 / KPL];
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) cw[u][i] = make_uint4(0, 0, 0, 0);
        sv[u] = typename SV::T{};
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k0 = tb + u * TILE + lane * KPL;
      const uint32_t* w = reinterpret_cast<const uint32_t*>(&cw[u][0]);
      float key[KPL];
#pragma unroll
      for (int q = 0; q < KPL; ++q) {
        int acc = 0;
#pragma unroll
        for (int d = 0; d < DW; ++d) {
          const uint32_t x = w[q * DW + d];
          acc = __builtin_amdgcn_sdot4(static_cast<int>(qlo[d]), static_cast<int>((x << 4) & 0xF0F0F0F0u), acc, false);
          acc = __builtin_amdgcn_sdot4(static_cast<int>(qhi[d]), static_cast<int>(x & 0xF0F0F0F0u), acc, false);
        }
        const int isc = acc >> 4;   // exact: every term is a multiple of 16
        float kf = f16bits_to_f32(SV::get(sv[u], q)) * static_cast<float>(isc);
        kf = (kf == 0.0f) ? 0.0f : kf;
        // Keys past this workgroup's range (the row end or the next chunk)
        // take no part: blocks never straddle chunks, which are whole tiles.
        const int t = k0 + q;
        if (t >= t_hi) kf = ninf;
        key[q] = kf;
        if (DEBUG && t < t_hi) {
          isum[static_cast<int64_t>(r) * tokens + t] = isc;
          keys_out[static_cast<int64_t>(r) * tokens + t] = kf;
        }
      }
      if (bmax) {
        if (block >= KPL) {
          float m = key[0];
#pragma unroll
          for (int q = 1; q < KPL; ++q) m = fmaxf(m, key[q]);
          for (int msk = 1; msk < lanes_per_block; msk <<= 1) m = fmaxf(m, shfl_xor(m, msk));
          if ((lane % lanes_per_block) == 0 && k0 < t_hi) bmax[static_cast<int64_t>(r) * nb + k0 / block] = m;
        } else {
          for (int q0 = 0; q0 < KPL; q0 += block) {
            float m = key[q0];
            for (int q = 1; q < block; ++q) m = fmaxf(m, key[q0 + q]);
            if (k0 + q0 < t_hi) bmax[static_cast<int64_t>(r) * nb + (k0 + q0) / block] = m;
          }
        }
      }
    }
  }
}

template <bool DEBUG>
int launch_scores(int S, dim3 grid, hipStream_t st, const uint16_t* q, int hq, int hkv, int d,
                  const int32_t* ci, const uint8_t* slab, const uint16_t* ss, int64_t cap, int T,
                  int block, int chunk, float* bmax, int nb, int32_t* isum, float* keys, float* qs) {
  switch (S) {
#define QKV_CASE(SS)                                                                         \
  case SS:                                                                                   \
    decode_scores_kernel<SS, DEBUG><<<grid, kThreads, 0, st>>>(q, hq, hkv, d, ci, slab, ss, \
                                                               cap, T, block, chunk, bmax, nb, \
                                                               isum, keys, qs);              \
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
  if (capacity % 64 || !aligned(slab, 16) || !aligned(slab_scales, 16))
    return fail(QKV_ERR_INVALID, "qkv_int4_build_slab: capacity must be a multiple of 64 and outputs 16-byte aligned");
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

QKV_EXPORT int qkv_int4_decode_scores(const void* query, int64_t batch, int64_t q_heads,
                                      int64_t kv_heads, int64_t head_dim, const int32_t* chan_idx,
                                      int64_t selected, const uint8_t* slab,
                                      const uint16_t* slab_scales, int64_t capacity, int64_t tokens,
                                      int64_t block, float* bmax, int32_t* isum, float* keys,
                                      float* qscale, void* stream) {
  if (!query || !chan_idx || !slab || !slab_scales)
    return fail(QKV_ERR_INVALID, "qkv_int4_decode_scores: null input pointer");
  if (!bmax && !(isum && keys))
    return fail(QKV_ERR_INVALID, "qkv_int4_decode_scores: need bmax or both isum and keys");
  if ((isum == nullptr) != (keys == nullptr))
    return fail(QKV_ERR_INVALID, "qkv_int4_decode_scores: isum and keys go together");
  if (batch <= 0 || kv_heads <= 0 || q_heads % kv_heads || q_heads / kv_heads > 64)
    return fail(QKV_ERR_INVALID, "qkv_int4_decode_scores: q_heads must be a multiple of kv_heads");
  if (batch * kv_heads > 65535) return fail(QKV_ERR_INVALID, "qkv_int4_decode_scores: too many rows");
  if (selected != 16 && selected != 32 && selected != 64 && selected != 128)
    return fail(QKV_ERR_UNSUPPORTED, "qkv_int4_decode_scores: selected must be 16, 32, 64 or 128");
  if (selected > head_dim) return fail(QKV_ERR_INVALID, "qkv_int4_decode_scores: selected > head_dim");
  if (tokens <= 0 || tokens > capacity || tokens >= (int64_t(1) << 30))
    return fail(QKV_ERR_INVALID, "qkv_int4_decode_scores: need 1 <= tokens <= capacity");
  if (capacity % 64 || !aligned(slab, 16) || !aligned(slab_scales, 16))
    return fail(QKV_ERR_INVALID, "qkv_int4_decode_scores: capacity must be a multiple of 64 and slab 16-byte aligned");
  const int kpl = static_cast<int>(128 / selected);
  if (!pow2(block) || block > 64 * kpl)
    return fail(QKV_ERR_INVALID, "qkv_int4_decode_scores: block must be a power of two <= %d", 64 * kpl);
  const int64_t rows = batch * kv_heads;
  const int tile_wg = 4 * 64 * kpl * QKV_SCORE_UNROLL;   // keys one workgroup pass covers
  int64_t chunk = cdiv(rows * tokens, QKV_SCORE_TARGET_WGS);
  chunk = std::max<int64_t>(tile_wg, cdiv(chunk, tile_wg) * tile_wg);
  dim3 grid(static_cast<unsigned>(cdiv(tokens, chunk)), static_cast<unsigned>(rows));
  const int nb = static_cast<int>(cdiv(tokens, block));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint16_t* q = static_cast<const uint16_t*>(query);
  if (isum)
    return launch_scores<true>(static_cast<int>(selected), grid, st, q, static_cast<int>(q_heads),
                               static_cast<int>(kv_heads), static_cast<int>(head_dim), chan_idx, slab,
                               slab_scales, capacity, static_cast<int>(tokens), static_cast<int>(block),
                               static_cast<int>(chunk), bmax, nb, isum, keys, qscale);
  return launch_scores<false>(static_cast<int>(selected), grid, st, q, static_cast<int>(q_heads),
                              static_cast<int>(kv_heads), static_cast<int>(head_dim), chan_idx, slab,
                              slab_scales, capacity, static_cast<int>(tokens), static_cast<int>(block),
                              static_cast<int>(chunk), bmax, nb, nullptr, nullptr, qscale);
}
