// Decode scoring of the int4 subset slab fused with block max-pooling, as a
// device function (the decode_scores kernel in int4.hip runs one chunk per
// workgroup).
#pragma once

#include "common.h"

// Waves per decode-scoring workgroup (the chunk's waves share no barrier,
// only the workgroup's chunk of the row).
#ifndef QKV_SCORE_WAVES
#define QKV_SCORE_WAVES 4
#endif

namespace qkv {
namespace {

constexpr int kScoreWaves = QKV_SCORE_WAVES;
constexpr int kScoreThreads = 64 * kScoreWaves;

// Keys per 4096-byte slab tile (the layout is described in int4.hip).
__host__ __device__ constexpr int64_t slab_tile_keys(int s) { return 8192 / s; }

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
__device__ __forceinline__ uint4 ld_nt(const uint4* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
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

// Per-row int8 query of decode scoring (q bf16, or fp16 with F16), computed by one wave: q8[s] =
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

template <int S, bool F16>
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
      lo = lo + half_lo<F16>(L.w[i]);
      hi = hi + half_hi<F16>(L.w[i]);
    }
  }
  if (lane >= hd2) lo = hi = 0.0f;   // no channel pair: never picked
  if (G > kQPre && lane < hd2) {
    const int b = r / kv_heads, j = r - b * kv_heads;
    const uint32_t* qrow = reinterpret_cast<const uint32_t*>(
        query + (static_cast<int64_t>(b) * q_heads + j * G) * head_dim);
    for (int i = kQPre; i < G; ++i) {
      const uint32_t w = qrow[i * hd2 + lane];
      lo = lo + half_lo<F16>(w);
      hi = hi + half_hi<F16>(w);
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

// Scores chunk `bx` of row r (keys [bx*chunk, min(tokens, (bx+1)*chunk)))
// in one workgroup of kScoreWaves waves, writing its block maxima to bmax
// and, with DEBUG, every key's int32 sum and fp32 key.
// NWV: the workgroup's waves.  hist (optional, LDS, 4096 bins): every key of
// the chunk is also counted at its top 12 order-preserving bits.
template <int S, bool DEBUG, bool F16, int NWV = kScoreWaves>
__device__ __forceinline__ void score_chunk(
    const uint16_t* __restrict__ query, int q_heads, int kv_heads, int head_dim,
    const int32_t* __restrict__ chan_idx, const uint8_t* __restrict__ slab,
    const uint16_t* __restrict__ slab_scales, int64_t capacity, int tokens, int block,
    int chunk, float* __restrict__ bmax, int nb, int32_t* __restrict__ isum,
    float* __restrict__ keys_out, float* __restrict__ qscale_out, int r, int bx, uint32_t* hist = nullptr) {
  constexpr int KPLN = 128 / S;                        // keys per lane per stage
  constexpr int STAGE = static_cast<int>(slab_tile_keys(S));   // keys per wave stage = 64 * KPLN
  constexpr int DW = S / 8;                            // code dwords per key
  using LS = LaneScales<KPLN>;

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
  const int t_lo = bx * chunk;
  const int t_hi = min(tokens, t_lo + chunk);

  // A wave's stages start at t_lo + wave*STAGE and step by NWV*STAGE;
  // t_lo is a multiple of NWV*STAGE, so every stage is one whole tile.  A stage with
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
  if (tb >= t_hi) return;   // wave-uniform; the chunk's waves share no barrier
  const int nst = (t_hi - tb + NWV * STAGE - 1) / (NWV * STAGE);   // stages of this wave
  uint4 cw[4];
  LS sv;
  load_stage(tb, cw, sv);
  __builtin_amdgcn_sched_barrier(0);

  uint32_t qlo[DW], qhi[DW];
  float qs;
  row_query_finish<S, F16>(ql, query, q_heads, kv_heads, head_dim, r, qlo, qhi, &qs);
  if (qscale_out && bx == 0 && wave == 0 && lane == 0) qscale_out[r] = qs;

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
      else if (hist) atomicAdd(&hist[f32_sortable(kf) >> 20], 1u);
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
    const int tn = tb + NWV * STAGE;
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

}  // namespace
}  // namespace qkv
