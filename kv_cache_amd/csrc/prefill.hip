// Chunked-prefill scoring as a dense contraction on int8 MFMA.
//
// The reference prefills with dense bf16 attention (evaluate_qwen3_top2_head_
// limit3_ppl.py:7079-7111, dense QK at EV:6602-6604) and has no block
// selection for a query chunk.  Here every query row of a chunk scores every
// cached key of its KV head exactly, I = sum_c q8[c] * code[t,c] over all
// 128 channels (int32), ranks key t by fp32(scale[t]) * fp32(I), max-pools
// the keys of each 64-key block under the causal mask, and keeps the top-k
// blocks per query row.
//
// MFMA mapping (v_mfma_i32_16x16x64_i8, two per 16x16 tile over 128
// channels): A = 16 keys, B = 16 queries.  Lane l of the A operand loads the
// 16 packed bytes of key l%16 at byte 16*(l/16) -- channels 32g..32g+31 of
// the key, g = l/16 -- so a wave's A load is one coalesced kilobyte.  Those
// nibbles become bytes holding 16*code ((w << 4) & 0xF0F0F0F0 for even
// channels, w & 0xF0F0F0F0 for odd ones); the query rows are stored
// pre-permuted (prefill_query_kernel) so that B byte slot s of lane group g
// holds the same channel as A byte slot s.  The result is 16*I, and
// fp32(scale) * fp32(16*I), rounded once, is exactly 16 times
// fp32(scale) * fp32(I), so block maxima are taken on 16*key and scaled
// back by 1/16 (exact).
// The output tile has lane l hold keys 4*(l/16)+i of query l%16: a block max
// is an in-lane max plus two cross-row shuffles.
#include "common.h"

namespace qkv {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kD = 128;
constexpr int kBlock = 64;          // keys per selection block
constexpr int kNT = 8;              // 16-query column tiles per wave
constexpr int kQTile = 16 * kNT;    // queries per wave
constexpr int kChunkBlocks = 16;    // blocks per workgroup key chunk
static_assert(kNT % 4 == 0, "the block-end reduction takes four query tiles at a time");

// Byte position, within a permuted query row, of channel c.
__host__ __device__ constexpr int perm_slot(int c) {
  const int g = c >> 5, half = (c >> 4) & 1, c16 = c & 15;
  return g * 32 + half * 16 + (c16 >> 3) * 8 + (c16 & 1) * 4 + ((c16 & 7) >> 1);
}

// Channel held by byte slot s: perm_slot maps the low channel bits (b3 b2 b1
// b0) to slot bits (b3 b0 b2 b1), so slot bits (t3 t2 t1 t0) come from
// channel bits (t3 t1 t0 t2).
__host__ __device__ constexpr int perm_channel(int s) {
  return (s & ~15) | (s & 8) | ((s & 2) << 1) | ((s & 1) << 1) | ((s >> 2) & 1);
}

constexpr bool perm_inverts() {
  for (int c = 0; c < kD; ++c)
    if (perm_channel(perm_slot(c)) != c) return false;
  return true;
}
static_assert(perm_inverts(), "perm_channel inverts perm_slot");

// ---------------------------------------------------------------------------
// Query quantization: q8 = clamp(rint(q / (amax/127)), +-127) over each row's
// 128 channels, written in the permuted MFMA order.  A wave takes kQRows rows
// and issues all their loads before the first row is quantized (one row per
// wave ran 65536 waves in eight rounds of load latency: 15 us at cfg5); lane l
// loads the two channels of output slots 2l and 2l+1 and writes them as one
// 2-byte store, so a row's 128 bytes leave in one coalesced store.  The row
// maximum of |q| is a DPP reduction on the bit patterns (exact for
// non-negative floats).
// ---------------------------------------------------------------------------
constexpr int kQRows = 8;

template <bool F16>
__global__ __launch_bounds__(256) void prefill_query_kernel(const uint16_t* __restrict__ q, int64_t q_row_stride,
                                                            int64_t rows, int8_t* __restrict__ q8,
                                                            float* __restrict__ qscale) {
  const int lane = threadIdx.x & 63;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * kQRows;
  if (row0 >= rows) return;   // wave-uniform
  const int ca = perm_channel(2 * lane), cb = perm_channel(2 * lane + 1);
  float x0[kQRows], x1[kQRows];
#pragma unroll
  for (int r = 0; r < kQRows; ++r) {
    const uint16_t* qr = q + min(row0 + r, rows - 1) * q_row_stride;
    x0[r] = half_to_f32<F16>(qr[ca]);
    x1[r] = half_to_f32<F16>(qr[cb]);
  }
#pragma unroll
  for (int r = 0; r < kQRows; ++r) {
    if (row0 + r >= rows) break;   // wave-uniform
    const float qs = wave_max_nonneg(fmaxf(fabsf(x0[r]), fabsf(x1[r]))) / 127.0f;
    auto quant = [&](float v) -> uint32_t {
      if (qs == 0.0f) return 0u;
      const float t = __builtin_rintf(v / qs);
      return static_cast<uint8_t>(static_cast<int8_t>(static_cast<int>(fminf(fmaxf(t, -127.0f), 127.0f))));
    };
    const int64_t row = row0 + r;
    reinterpret_cast<uint16_t*>(q8 + row * kD)[lane] = static_cast<uint16_t>(quant(x0[r]) | (quant(x1[r]) << 8));
    if (qscale && lane == 0) qscale[row] = qs;
  }
}

// The same quantization for rows 16-byte aligned (row stride a multiple of 8
// channels): channels 8m..8m+7 land in output bytes 8m..8m+7 (perm_slot keeps
// each aligned group of 8, reordered inside it: channel 8m+e to byte 8m +
// 4*(e%2) + e/2), so lane l of a 16-lane row group loads channels 8m..8m+7 (m
// = l%16) of row l/16 in one 16-byte load and writes its 8 bytes in one
// 8-byte store; a load instruction covers 4 rows, and the row maximum is a
// DPP reduction within the row of 16 lanes.  kQVRows rows per wave.
constexpr int kQVRows = 4;

template <bool F16>
__global__ __launch_bounds__(256) void prefill_query_vec_kernel(const uint16_t* __restrict__ q,
                                                                int64_t q_row_stride, int64_t rows,
                                                                int8_t* __restrict__ q8,
                                                                float* __restrict__ qscale) {
  constexpr int kLoads = kQVRows / 4;
  const int lane = threadIdx.x & 63, m = lane & 15;
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6)) * kQVRows + (lane >> 4);
  if (row0 - (lane >> 4) >= rows) return;   // wave-uniform
  uint4 w[kLoads];
#pragma unroll
  for (int it = 0; it < kLoads; ++it)
    w[it] = *reinterpret_cast<const uint4*>(q + min(row0 + 4 * it, rows - 1) * q_row_stride + 8 * m);
#pragma unroll
  for (int it = 0; it < kLoads; ++it) {
    const int64_t row = row0 + 4 * it;
    float x[8];
    const uint32_t ws[4] = {w[it].x, w[it].y, w[it].z, w[it].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = half_lo<F16>(ws[e]);
      x[2 * e + 1] = half_hi<F16>(ws[e]);
    }
    float a = fabsf(x[0]);
#pragma unroll
    for (int e = 1; e < 8; ++e) a = fmaxf(a, fabsf(x[e]));
    // max over the row's 16 lanes, on the bit patterns of non-negative floats
    uint32_t v = __float_as_uint(a);
    v = max(v, dpp_mov<0xB1>(v, v));
    v = max(v, dpp_mov<0x4E>(v, v));
    v = max(v, dpp_mov<0x141>(v, v));
    v = max(v, dpp_mov<0x140>(v, v));
    const float qs = __uint_as_float(v) / 127.0f;
    uint32_t b[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float t = qs == 0.0f ? 0.0f : __builtin_rintf(x[e] / qs);
      b[e] = static_cast<uint8_t>(static_cast<int8_t>(static_cast<int>(fminf(fmaxf(t, -127.0f), 127.0f))));
    }
    if (row < rows) {
      // byte 4*(e%2) + e/2 holds channel 8m + e
      const uint2 o = make_uint2(b[0] | (b[2] << 8) | (b[4] << 16) | (b[6] << 24),
                                 b[1] | (b[3] << 8) | (b[5] << 16) | (b[7] << 24));
      *reinterpret_cast<uint2*>(q8 + row * kD + 8 * m) = o;
      if (qscale && m == 0) qscale[row] = qs;
    }
  }
}

__device__ __forceinline__ v4i unpack_half(uint32_t w0, uint32_t w1) {
  v4i a;
  a.x = static_cast<int>((w0 << 4) & 0xF0F0F0F0u);
  a.y = static_cast<int>(w0 & 0xF0F0F0F0u);
  a.z = static_cast<int>((w1 << 4) & 0xF0F0F0F0u);
  a.w = static_cast<int>(w1 & 0xF0F0F0F0u);
  return a;
}

// ---------------------------------------------------------------------------
// Block scores.  A workgroup holds W waves: W query heads of one KV head that
// share one tile of kQTile query rows (W = 4 when the GQA group size G is a
// multiple of 4, else 2 or 1), so all its waves see the same keys under the
// same causal mask.  Grid: x = key chunk (kChunkBlocks blocks of 64 keys),
// y = (query tile, group of W heads), z = (batch, KV head).
//
// Per 64-key block the workgroup stages the block once in LDS: wave w loads
// the packed codes of key tiles w, w+W, .. (one coalesced kilobyte each) and
// writes them unpacked (bytes holding 16*code, the MFMA A layout), and wave
// 0 converts the block's 64 fp16 scales to fp32 s and -12582912*s.  Each wave
// then issues per 16-key tile 16 MFMAs against its 128 resident query rows
// and the epilogue: 16*key = fma(s, acc, -12582912*s) per accumulator (the
// biased accumulator, below), maximum over the keys a lane holds with
// v_max3, and at the block end over the 4 row groups with lane swaps.  The
// LDS copy is double-buffered: block kb+1 is staged while block kb is
// scored, one workgroup barrier per block.  Only blocks on the causal
// diagonal or past the last token take the masked epilogue (uniform over
// the workgroup).
//
// Every accumulator starts at the bit pattern of 1.5 * 2^23, so the int32
// result 0x4B400000 + 16*I read as fp32 is exactly 12582912 + 16*I (|16*I| <
// 2^22).  Then fma(s, f, -12582912 * s) = round(s * 16*I): one rounding of
// the exact product, i.e. 16 times fp32(s) * fp32(I), with no integer
// conversion (-12582912 * s is exact: s has 11 significant bits).  Block
// maxima are taken on 16*key and scaled back by 1/16 (exact).
// ---------------------------------------------------------------------------
// Issue order of one pipelined step: each MFMA followed by three vector
// instructions (the previous tile's epilogue: 48 per tile), and nothing moved
// across steps.
__device__ __forceinline__ void interleave_step() {
#pragma unroll
  for (int i = 0; i < 2 * kNT; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);   // three VALU
  }
  __builtin_amdgcn_sched_barrier(0);
}

template <int W>
__global__ __launch_bounds__(64 * W, 8 / W) void prefill_scores_kernel(
    const int8_t* __restrict__ q8, const uint8_t* __restrict__ kpacked, const uint16_t* __restrict__ kscales,
    int q_heads, int kv_heads, int nq, int tokens, int64_t capacity, int q_pos0, int nb,
    float* __restrict__ bmax) {
  static_assert(W == 1 || W == 2 || W == 4, "1, 2 or 4 waves per workgroup");
  constexpr int kTiles = 4 / W;                       // key tiles a wave stages per block
  __shared__ v4i abuf[2][4][2][64];                    // [slot][key tile][channel half][lane]
  __shared__ float sbuf[2][4][4][8];                   // [slot][key tile][row group][s x4, -12582912*s x4]
  __shared__ float tile[W][kQTile][kChunkBlocks + 1];
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = q_heads / kv_heads;
  const int hgroups = G / W;
  const int qt = blockIdx.y / hgroups, hg = blockIdx.y - qt * hgroups;
  const int bj = blockIdx.z;                         // b * kv_heads + j
  const int b = bj / kv_heads, j = bj - b * kv_heads;
  const int head = j * G + hg * W + wave;
  const int64_t qrow0 = (static_cast<int64_t>(b) * q_heads + head) * nq;
  const int q0 = qt * kQTile;
  const int g = lane >> 4, col = lane & 15;

  // B fragments: query q0 + 16n + col, channel group g, both halves.
  v4i bq[kNT][2];
#pragma unroll
  for (int n = 0; n < kNT; ++n) {
    const int qi = q0 + 16 * n + col;
    if (qi < nq) {
      const v4i* p = reinterpret_cast<const v4i*>(q8 + (qrow0 + qi) * kD + g * 32);
      bq[n][0] = p[0];
      bq[n][1] = p[1];
    } else {
      bq[n][0] = v4i{0, 0, 0, 0};
      bq[n][1] = v4i{0, 0, 0, 0};
    }
  }
  const int qlast = min(nq, q0 + kQTile) - 1;
  const int pos_lo = q_pos0 + q0, pos_hi = q_pos0 + qlast;   // positions of the tile's first/last query

  const int blk0 = blockIdx.x * kChunkBlocks;
  const int nblk = min(kChunkBlocks, nb - blk0);
  // Blocks [0, nvis) of the chunk hold a key some query of the tile sees;
  // blocks [0, nfull) need no mask: every key is at or before the first
  // query's position and below `tokens`.
  const int nvis = pos_hi < blk0 * kBlock ? 0 : min(nblk, (pos_hi - blk0 * kBlock) / kBlock + 1);
  const int lim_pos = pos_lo >= kBlock - 1 ? (pos_lo - (kBlock - 1)) / kBlock + 1 : 0;
  const int nfull = max(0, min(min(lim_pos, tokens / kBlock) - blk0, nvis));
  const uint8_t* krow = kpacked + static_cast<int64_t>(bj) * capacity * (kD / 2);
  const uint16_t* srow = kscales + static_cast<int64_t>(bj) * capacity;
  const float ninf = -__builtin_huge_valf();

  // Buffer loads over the chunk (every block below nb lies inside the
  // capacity, a multiple of 64): lane l of a key tile loads key l%16,
  // channels 32g..32g+31; lane l of wave 0 loads the scale of key l.
  const int64_t key0 = static_cast<int64_t>(blk0) * kBlock;
  const auto krsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(krow + key0 * (kD / 2)), 0,
                                                       nblk * kBlock * (kD / 2), 0x00020000);
  const auto srsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(srow + key0), 0, nblk * kBlock * 2,
                                                       0x00020000);
  const int kvoff = col * (kD / 2) + g * 16;
  uint4 raw[kTiles];
  uint32_t sraw = 0;
  auto gload = [&](int kb) {
#pragma unroll
    for (int r = 0; r < kTiles; ++r) {
      const int kt = wave + W * r;
      const auto a = __builtin_amdgcn_raw_buffer_load_b128(krsrc, kvoff + kt * 16 * (kD / 2), kb * kBlock * (kD / 2), 0);
      raw[r] = uint4{a[0], a[1], a[2], a[3]};
    }
    if (wave == 0) sraw = __builtin_amdgcn_raw_buffer_load_b16(srsrc, 2 * lane, kb * kBlock * 2, 0);
  };
  auto stage = [&](int slot) {
#pragma unroll
    for (int r = 0; r < kTiles; ++r) {
      const int kt = wave + W * r;
      abuf[slot][kt][0][lane] = unpack_half(raw[r].x, raw[r].y);
      abuf[slot][kt][1][lane] = unpack_half(raw[r].z, raw[r].w);
    }
    if (wave == 0) {
      const float s = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(sraw)));
      float* e = &sbuf[slot][lane >> 4][(lane >> 2) & 3][lane & 3];
      e[0] = s;
      e[4] = __builtin_fmaf(s, -12582912.0f, 0.0f);
    }
  };

  const v4i kBias = v4i{0x4B400000, 0x4B400000, 0x4B400000, 0x4B400000};
  // Fragments of key tile kt from LDS slot `slot`: the A operands of both
  // channel halves, and s / -12582912*s of the 4 keys the lane's rows hold.
  auto frag = [&](int slot, int kt, v4i& a0, v4i& a1, float4& s, float4& c) {
    a0 = abuf[slot][kt][0][lane];
    a1 = abuf[slot][kt][1][lane];
    s = *reinterpret_cast<const float4*>(&sbuf[slot][kt][g][0]);
    c = *reinterpret_cast<const float4*>(&sbuf[slot][kt][g][4]);
  };
  auto mfma_tile = [&](const v4i& a0, const v4i& a1, v4i (&acc)[kNT]) {
#pragma unroll
    for (int n = 0; n < kNT; ++n) acc[n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, bq[n][0], kBias, 0, 0, 0);
#pragma unroll
    for (int n = 0; n < kNT; ++n) acc[n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bq[n][1], acc[n], 0, 0, 0);
  };
  float run[kNT];
  // Unmasked epilogue of one key tile into the running block maxima (the
  // block's first tile starts them).
  auto epi = [&](const v4i (&acc)[kNT], const float4 s, const float4 c, bool first) {
#pragma unroll
    for (int n = 0; n < kNT; ++n) {
      const float k0 = __builtin_fmaf(s.x, __int_as_float(acc[n].x), c.x);
      const float k1 = __builtin_fmaf(s.y, __int_as_float(acc[n].y), c.y);
      const float k2 = __builtin_fmaf(s.z, __int_as_float(acc[n].z), c.z);
      const float k3 = __builtin_fmaf(s.w, __int_as_float(acc[n].w), c.w);
      if (first) {
        run[n] = fmaxf(fmaxf(fmaxf(k0, k1), k2), k3);
      } else {
        run[n] = fmaxf(fmaxf(run[n], k0), k1);
        run[n] = fmaxf(fmaxf(run[n], k2), k3);
      }
    }
    // Keep the epilogue in its step (next to the MFMAs it overlaps) rather
    // than sunk to where the block maxima are consumed.
#pragma unroll
    for (int n = 0; n < kNT; ++n) pin(run[n]);
  };
  // Masked epilogue: key t of the lane's rows is visible to query q when t <=
  // pos(q) and t < tokens; lim = min(pos(q), tokens - 1) - (first key of the
  // row group) compares once per key.
  auto epi_masked = [&](const v4i (&acc)[kNT], const float4 s, const float4 c, int kt, int base) {
#pragma unroll
    for (int n = 0; n < kNT; ++n) {
      const int lim = min(q_pos0 + q0 + 16 * n + col, tokens - 1) - (base + 4 * g);
      const float ks[4] = {__builtin_fmaf(s.x, __int_as_float(acc[n].x), c.x),
                           __builtin_fmaf(s.y, __int_as_float(acc[n].y), c.y),
                           __builtin_fmaf(s.z, __int_as_float(acc[n].z), c.z),
                           __builtin_fmaf(s.w, __int_as_float(acc[n].w), c.w)};
      float m = kt == 0 ? ninf : run[n];
#pragma unroll
      for (int i = 0; i < 4; ++i) m = fmaxf(m, (kt * 16 + i <= lim) ? ks[i] : ninf);
      run[n] = m;
    }
  };
  auto block_end = [&](int kb) {
#pragma unroll
    for (int n0 = 0; n0 + 4 <= kNT; n0 += 4) {
      const float m = max_rows4(run[n0], run[n0 + 1], run[n0 + 2], run[n0 + 3]);
      tile[wave][16 * (n0 + g) + col][kb] = __builtin_fmaf(m, 0.0625f, 0.0f);
    }
  };
  // Stages block kb+1 (its codes were loaded one block earlier) and loads
  // block kb+2.  Slot (kb+1) % 2 was last read for block kb-1, before the
  // barrier that ended it.
  auto stage_next = [&](int kb) {
    if (kb + 1 < nvis) {
      stage((kb + 1) & 1);
      if (kb + 2 < nvis) gload(kb + 2);
    }
  };

  if (nvis > 0) {
    gload(0);
    stage(0);
    if (nvis > 1) gload(1);
    __syncthreads();
  }
  // Unmasked blocks [0, nfull), pipelined by key tile: the MFMAs of tile kt
  // are issued ahead of the epilogue of tile kt-1 (the other accumulator
  // set); the last tile's epilogue runs after the block's barrier, behind
  // the next block's first MFMAs.
  v4i acc0[kNT], acc1[kNT];
  v4i a0, a1, n0, n1;
  float4 s0, c0, s1, c1;
  if (nfull > 0) {
    frag(0, 0, a0, a1, s0, c0);
    frag(0, 1, n0, n1, s1, c1);
    mfma_tile(a0, a1, acc0);
  }
  for (int kb = 0; kb < nfull; ++kb) {
    const int slot = kb & 1;
    float4 s2, c2;
    frag(slot, 2, a0, a1, s2, c2);          // prefetch tile 2
    mfma_tile(n0, n1, acc1);                // tile 1
    epi(acc0, s0, c0, true);                // tile 0
    interleave_step();
    frag(slot, 3, n0, n1, s0, c0);          // prefetch tile 3 (s0/c0 now tile 3's)
    mfma_tile(a0, a1, acc0);                // tile 2
    epi(acc1, s1, c1, false);               // tile 1
    interleave_step();
    mfma_tile(n0, n1, acc1);                // tile 3
    epi(acc0, s2, c2, false);               // tile 2
    interleave_step();
    stage_next(kb);
    __syncthreads();
    if (kb + 1 < nfull) {
      frag(slot ^ 1, 0, a0, a1, s2, c2);
      frag(slot ^ 1, 1, n0, n1, s1, c1);
      mfma_tile(a0, a1, acc0);              // next block's tile 0
      epi(acc1, s0, c0, false);             // tile 3
      interleave_step();
      block_end(kb);
      s0 = s2;
      c0 = c2;
    } else {
      epi(acc1, s0, c0, false);
      block_end(kb);
    }
  }
  // Blocks [nfull, nvis) hold keys past some query of the tile (the causal
  // diagonal) or past the last token: masked, one tile at a time.
  for (int kb = nfull; kb < nvis; ++kb) {
    const int slot = kb & 1, base = (blk0 + kb) * kBlock;
    v4i a0, a1;
    float4 s0, c0;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      frag(slot, kt, a0, a1, s0, c0);
      mfma_tile(a0, a1, acc0);
      epi_masked(acc0, s0, c0, kt, base);
    }
    block_end(kb);
    stage_next(kb);
    __syncthreads();
  }
  for (int kb = nvis; kb < nblk; ++kb) {
    if (lane < 16) {
#pragma unroll
      for (int n = 0; n < kNT; ++n) tile[wave][16 * n + col][kb] = ninf;
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // Coalesced write: consecutive lanes take consecutive blocks of one row.
  for (int idx = lane; idx < kQTile * kChunkBlocks; idx += 64) {
    const int r = idx / kChunkBlocks, kb = idx - r * kChunkBlocks;
    if (kb < nblk && q0 + r < nq) bmax[(qrow0 + q0 + r) * nb + blk0 + kb] = tile[wave][r][kb];
  }
}

}  // namespace
}  // namespace qkv

using namespace qkv;

QKV_EXPORT int qkv_prefill_quantize_query(const void* query, int64_t rows, int64_t head_dim,
                                          int64_t row_stride, int8_t* q8, float* qscale, int dtype, void* stream) {
  if (!query || !q8) return fail(QKV_ERR_INVALID, "qkv_prefill_quantize_query: null pointer");
  bool f16;
  if (int rc = half_dtype(dtype, "qkv_prefill_quantize_query", &f16)) return rc;
  if (head_dim != kD) return fail(QKV_ERR_UNSUPPORTED, "qkv_prefill_quantize_query: head_dim must be 128");
  if (rows <= 0 || row_stride < head_dim || row_stride % 2 || !aligned(query, 4))
    return fail(QKV_ERR_INVALID, "qkv_prefill_quantize_query: bad rows or row stride");
  if (!aligned(q8, 2)) return fail(QKV_ERR_INVALID, "qkv_prefill_quantize_query: q8 must be 2-byte aligned");
  if (cdiv(rows, 4 * kQRows) > 0x7FFFFFFF) return fail(QKV_ERR_INVALID, "qkv_prefill_quantize_query: too many rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const bool vec = row_stride % 8 == 0 && aligned(query, 16) && aligned(q8, 8);
  return with_half(f16, [&](auto ff) {
    constexpr bool F = decltype(ff)::value;
    if (vec)
      prefill_query_vec_kernel<F><<<static_cast<unsigned>(cdiv(rows, 4 * kQVRows)), 256, 0, st>>>(
          static_cast<const uint16_t*>(query), row_stride, rows, q8, qscale);
    else
      prefill_query_kernel<F><<<static_cast<unsigned>(cdiv(rows, 4 * kQRows)), 256, 0, st>>>(
          static_cast<const uint16_t*>(query), row_stride, rows, q8, qscale);
    return check_launch("qkv_prefill_quantize_query");
  });
}

QKV_EXPORT int qkv_prefill_block_scores(const int8_t* q8, int64_t batch, int64_t q_heads,
                                        int64_t kv_heads, int64_t queries, const uint8_t* packed,
                                        const uint16_t* scales, int64_t capacity, int64_t tokens,
                                        int64_t q_pos0, int64_t head_dim, int64_t block,
                                        float* bmax, void* stream) {
  if (!q8 || !packed || !scales || !bmax) return fail(QKV_ERR_INVALID, "qkv_prefill_block_scores: null pointer");
  if (head_dim != kD) return fail(QKV_ERR_UNSUPPORTED, "qkv_prefill_block_scores: head_dim must be 128");
  if (block != kBlock) return fail(QKV_ERR_UNSUPPORTED, "qkv_prefill_block_scores: block must be 64");
  if (batch <= 0 || kv_heads <= 0 || q_heads % kv_heads)
    return fail(QKV_ERR_INVALID, "qkv_prefill_block_scores: q_heads must be a multiple of kv_heads");
  if (queries <= 0 || tokens <= 0 || tokens > capacity || capacity % 64 || q_pos0 < 0 ||
      tokens >= (int64_t(1) << 30) || q_pos0 + queries >= (int64_t(1) << 30))
    return fail(QKV_ERR_INVALID, "qkv_prefill_block_scores: need 1 <= tokens <= capacity (a multiple of 64), q_pos0 >= 0");
  if (!aligned(q8, 16) || !aligned(packed, 16) || !aligned(scales, 8))
    return fail(QKV_ERR_INVALID, "qkv_prefill_block_scores: q8 and packed K must be 16-byte aligned");
  const int64_t nb = cdiv(tokens, kBlock);
  const int64_t g = q_heads / kv_heads;
  const int w = g % 4 == 0 ? 4 : (g % 2 == 0 ? 2 : 1);
  const int64_t ytiles = cdiv(queries, kQTile) * (g / w);
  if (batch * kv_heads > 65535 || ytiles > 65535 || cdiv(nb, kChunkBlocks) > 0x7FFFFFFF)
    return fail(QKV_ERR_INVALID, "qkv_prefill_block_scores: grid too large");
  dim3 grid(static_cast<unsigned>(cdiv(nb, kChunkBlocks)), static_cast<unsigned>(ytiles),
            static_cast<unsigned>(batch * kv_heads));
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int hq = static_cast<int>(q_heads), hkv = static_cast<int>(kv_heads), nq = static_cast<int>(queries);
  const int t = static_cast<int>(tokens), p0 = static_cast<int>(q_pos0), nbi = static_cast<int>(nb);
  if (w == 4)
    prefill_scores_kernel<4><<<grid, 256, 0, st>>>(q8, packed, scales, hq, hkv, nq, t, capacity, p0, nbi, bmax);
  else if (w == 2)
    prefill_scores_kernel<2><<<grid, 128, 0, st>>>(q8, packed, scales, hq, hkv, nq, t, capacity, p0, nbi, bmax);
  else
    prefill_scores_kernel<1><<<grid, 64, 0, st>>>(q8, packed, scales, hq, hkv, nq, t, capacity, p0, nbi, bmax);
  return check_launch("qkv_prefill_block_scores");
}
