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
#ifndef QKV_PF_NT
#define QKV_PF_NT 6
#endif
#ifndef QKV_PF_CHUNK
#define QKV_PF_CHUNK 32
#endif
#ifndef QKV_PF_WG_PER_CU
#define QKV_PF_WG_PER_CU 2
#endif
constexpr int kNT = QKV_PF_NT;              // 16-query column tiles per wave
constexpr int kQTile = 16 * kNT;            // queries per wave
constexpr int kChunkBlocks = QKV_PF_CHUNK;  // blocks per workgroup key chunk
static_assert(kNT % 2 == 0, "the block-end reduction pairs the query tiles");

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
    x0[r] = __uint_as_float(static_cast<uint32_t>(qr[ca]) << 16);
    x1[r] = __uint_as_float(static_cast<uint32_t>(qr[cb]) << 16);
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
      x[2 * e] = bf16lo(ws[e]);
      x[2 * e + 1] = bf16hi(ws[e]);
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
// Block scores.  Grid: x = key chunk (kChunkBlocks blocks), y = group of 4
// (query tile, head) pairs of one KV head, z = (batch, KV head).  Each wave
// owns one pair: kQTile query rows of one head, resident as B fragments, and
// streams the chunk's blocks that its queries can see.  No workgroup barrier:
// the 4 waves of a group read the same keys (the other waves' loads hit in
// cache) and stage their block maxima in their own LDS region before a
// coalesced write.
//
// Per block a wave loads the next block's codes and scales while it issues
// the current block's 32 MFMAs back to back (the first half of every tile's
// channels, then the second half, so dependent MFMAs are 4 apart) and then
// runs the epilogue: 16*key = fp32(scale) * fp32(16*I) as one v_fma_f32 per
// key on the biased int32 accumulator (below), maximum over the 16 keys a
// lane holds with v_max3, then over the 4 row groups with VALU lane swaps,
// times 1/16.  Only blocks on the causal diagonal or past the last token take the
// masked epilogue (a wave-uniform branch).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256, QKV_PF_WG_PER_CU) void prefill_scores_kernel(
    const int8_t* __restrict__ q8, const uint8_t* __restrict__ kpacked, const uint16_t* __restrict__ kscales,
    int q_heads, int kv_heads, int nq, int tokens, int64_t capacity, int q_pos0, int nb,
    float* __restrict__ bmax) {
  __shared__ float tile[4][kQTile][kChunkBlocks + 1];
  // The wave index is uniform: read it into a scalar register, so that the
  // query tile, the visible block count and the block offsets are scalar too.
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int G = q_heads / kv_heads;
  const int n_qtiles = (nq + kQTile - 1) / kQTile;
  const int combo = blockIdx.y * 4 + wave;
  if (combo >= n_qtiles * G) return;
  const int qt = combo / G, h = combo - qt * G;
  const int bj = blockIdx.z;                         // b * kv_heads + j
  const int b = bj / kv_heads, j = bj - b * kv_heads;
  const int head = j * G + h;
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
  const int pos_lo = q_pos0 + q0, pos_hi = q_pos0 + qlast;   // positions of the wave's first/last query

  const int blk0 = blockIdx.x * kChunkBlocks;
  const int nblk = min(kChunkBlocks, nb - blk0);
  // Blocks [0, nvis) of the chunk hold a key some query of the wave sees.
  const int nvis = pos_hi < blk0 * kBlock ? 0 : min(nblk, (pos_hi - blk0 * kBlock) / kBlock + 1);
  const uint8_t* krow = kpacked + static_cast<int64_t>(bj) * capacity * (kD / 2);
  const uint16_t* srow = kscales + static_cast<int64_t>(bj) * capacity;
  const float ninf = -__builtin_huge_valf();

  // Lane l loads key (base + 16kt + l%16), channels 32g..32g+31, and the
  // scales of the 4 keys its output rows hold (base + 16kt + 4g + i).  Every
  // block below nb lies inside the capacity (a multiple of 64).  Buffer
  // loads over the chunk: a per-lane constant offset plus the block's scalar
  // offset, so no per-load address arithmetic on the VALU.
  const int64_t key0 = static_cast<int64_t>(blk0) * kBlock;
  const auto krsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(krow + key0 * (kD / 2)), 0,
                                                       nblk * kBlock * (kD / 2), 0x00020000);
  const auto srsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(srow + key0), 0, nblk * kBlock * 2,
                                                       0x00020000);
  const int kvoff = col * (kD / 2) + g * 16, svoff = 8 * g;
  auto load_block = [&](int kb, uint4 (&ka)[4], uint2 (&ks)[4]) {
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      const auto a = __builtin_amdgcn_raw_buffer_load_b128(krsrc, kvoff + kt * 16 * (kD / 2), kb * kBlock * (kD / 2), 0);
      const auto s = __builtin_amdgcn_raw_buffer_load_b64(srsrc, svoff + kt * 32, kb * kBlock * 2, 0);
      ka[kt] = uint4{a[0], a[1], a[2], a[3]};
      ks[kt] = uint2{s[0], s[1]};
    }
  };

  // One block: two halves of 2 key tiles each (16 MFMAs, then their
  // epilogue), which keeps the accumulators at 32 registers.
  //
  // Every accumulator starts at the bit pattern of 1.5 * 2^23, so the int32
  // result 0x4B400000 + 16*I read as fp32 is exactly 12582912 + 16*I (|16*I|
  // < 2^22).  Then fma(s, f, -12582912 * s) = round(s * 16*I): one rounding
  // of the exact product, i.e. 16 times fp32(s) * fp32(I), with no integer
  // conversion (-12582912 * s is exact: s has 11 significant bits).
  const v4i kBias = v4i{0x4B400000, 0x4B400000, 0x4B400000, 0x4B400000};
  // MFMAs of one half block (key tiles 2h, 2h+1) into acc.
  auto mfma_half = [&](int half, const uint4 (&ka)[4], v4i (&acc)[2][kNT]) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int kt = 2 * half + u;
      const v4i a0 = unpack_half(ka[kt].x, ka[kt].y);
      const v4i a1 = unpack_half(ka[kt].z, ka[kt].w);
#pragma unroll
      for (int n = 0; n < kNT; ++n) acc[u][n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, bq[n][0], kBias, 0, 0, 0);
#pragma unroll
      for (int n = 0; n < kNT; ++n) acc[u][n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bq[n][1], acc[u][n], 0, 0, 0);
    }
  };
  // Epilogue of one half block: 16*key per accumulator, running block max.
  auto epi_half = [&](int half, const uint2 (&ks)[4], const v4i (&acc)[2][kNT], bool masked, int base,
                      float (&run)[kNT]) {
    // The fp16 scales feed v_fma_mix_f32 straight from their packed words.
    _Float16 sc[2][4];
    float cb[2][4];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const uint2 sr = ks[2 * half + u];
      sc[u][0] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(sr.x & 0xFFFFu));
      sc[u][1] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(sr.x >> 16));
      sc[u][2] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(sr.y & 0xFFFFu));
      sc[u][3] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(sr.y >> 16));
#pragma unroll
      for (int i = 0; i < 4; ++i) cb[u][i] = __builtin_fmaf(static_cast<float>(sc[u][i]), -12582912.0f, 0.0f);
    }
    auto key16 = [&](int u, int i, int a) -> float {
      return __builtin_fmaf(static_cast<float>(sc[u][i]), __int_as_float(a), cb[u][i]);
    };
    if (!masked) {
#pragma unroll
      for (int n = 0; n < kNT; ++n) {
        float m = run[n];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          m = fmaxf(fmaxf(m, key16(u, 0, acc[u][n].x)), key16(u, 1, acc[u][n].y));
          m = fmaxf(fmaxf(m, key16(u, 2, acc[u][n].z)), key16(u, 3, acc[u][n].w));
        }
        run[n] = m;
      }
    } else {
      // Key t of the lane's rows is visible to query q when t <= pos(q) and
      // t < tokens; lim = min(pos(q), tokens - 1) - (first key of the row
      // group) compares once per key.
#pragma unroll
      for (int n = 0; n < kNT; ++n) {
        const int lim = min(q_pos0 + q0 + 16 * n + col, tokens - 1) - (base + 4 * g);
        float m = run[n];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int accs[4] = {acc[u][n].x, acc[u][n].y, acc[u][n].z, acc[u][n].w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float v = key16(u, i, accs[i]);
            m = fmaxf(m, ((2 * half + u) * 16 + i <= lim) ? v : ninf);
          }
        }
        run[n] = m;
      }
    }
  };
  auto process = [&](int kb, const uint4 (&ka)[4], const uint2 (&ks)[4]) {
    const int base = (blk0 + kb) * kBlock;
    const bool need_mask = base + kBlock - 1 > pos_lo || base + kBlock > tokens;
    float run[kNT];
#pragma unroll
    for (int n = 0; n < kNT; ++n) run[n] = ninf;
    v4i acc0[2][kNT], acc1[2][kNT];
    mfma_half(0, ka, acc0);
    if (!need_mask) {
      mfma_half(1, ka, acc1);
      epi_half(0, ks, acc0, false, base, run);
      epi_half(1, ks, acc1, false, base, run);
    } else {
      mfma_half(1, ka, acc1);
      epi_half(0, ks, acc0, true, base, run);
      epi_half(1, ks, acc1, true, base, run);
    }
    // Max over the 4 row groups, four (then two) tiles per round of lane
    // swaps, after which row group g holds tile n0 + g; back to key scale
    // (exact), where adding +0 turns a -0 into +0 and leaves every other
    // value alone.
#pragma unroll
    for (int n0 = 0; n0 + 4 <= kNT; n0 += 4) {
      const float m = max_rows4(run[n0], run[n0 + 1], run[n0 + 2], run[n0 + 3]);
      tile[wave][16 * (n0 + g) + col][kb] = __builtin_fmaf(m, 0.0625f, 0.0f);
    }
    if constexpr (kNT % 4 == 2) {
      const float m = max_rows2(run[kNT - 2], run[kNT - 1]);
      if (lane < 32) tile[wave][16 * (kNT - 2 + g) + col][kb] = __builtin_fmaf(m, 0.0625f, 0.0f);
    }
  };

  // Two register buffers, the block loop unrolled by two; an odd count ends
  // by processing its last block twice (same result, same LDS slot).
  uint4 ka[2][4];
  uint2 ks[2][4];
  if (nvis > 0) load_block(0, ka[0], ks[0]);
  for (int kb = 0; kb < nvis; kb += 2) {
    const int k1 = min(kb + 1, nvis - 1), k2 = min(kb + 2, nvis - 1);
    load_block(k1, ka[1], ks[1]);
    process(kb, ka[0], ks[0]);
    load_block(k2, ka[0], ks[0]);
    process(k1, ka[1], ks[1]);
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
                                          int64_t row_stride, int8_t* q8, float* qscale, void* stream) {
  if (!query || !q8) return fail(QKV_ERR_INVALID, "qkv_prefill_quantize_query: null pointer");
  if (head_dim != kD) return fail(QKV_ERR_UNSUPPORTED, "qkv_prefill_quantize_query: head_dim must be 128");
  if (rows <= 0 || row_stride < head_dim || row_stride % 2 || !aligned(query, 4))
    return fail(QKV_ERR_INVALID, "qkv_prefill_quantize_query: bad rows or row stride");
  if (!aligned(q8, 2)) return fail(QKV_ERR_INVALID, "qkv_prefill_quantize_query: q8 must be 2-byte aligned");
  if (cdiv(rows, 4 * kQRows) > 0x7FFFFFFF) return fail(QKV_ERR_INVALID, "qkv_prefill_quantize_query: too many rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (row_stride % 8 == 0 && aligned(query, 16) && aligned(q8, 8)) {
    prefill_query_vec_kernel<<<static_cast<unsigned>(cdiv(rows, 4 * kQVRows)), 256, 0, st>>>(
        static_cast<const uint16_t*>(query), row_stride, rows, q8, qscale);
    return check_launch("qkv_prefill_quantize_query");
  }
  prefill_query_kernel<<<static_cast<unsigned>(cdiv(rows, 4 * kQRows)), 256, 0, st>>>(
      static_cast<const uint16_t*>(query), row_stride, rows, q8, qscale);
  return check_launch("qkv_prefill_quantize_query");
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
  const int64_t groups = cdiv(cdiv(queries, kQTile) * g, 4);
  if (batch * kv_heads > 65535 || groups > 65535 || cdiv(nb, kChunkBlocks) > 0x7FFFFFFF)
    return fail(QKV_ERR_INVALID, "qkv_prefill_block_scores: grid too large");
  dim3 grid(static_cast<unsigned>(cdiv(nb, kChunkBlocks)), static_cast<unsigned>(groups),
            static_cast<unsigned>(batch * kv_heads));
  hipStream_t st = static_cast<hipStream_t>(stream);
  prefill_scores_kernel<<<grid, 256, 0, st>>>(q8, packed, scales, static_cast<int>(q_heads),
                                              static_cast<int>(kv_heads), static_cast<int>(queries),
                                              static_cast<int>(tokens), capacity, static_cast<int>(q_pos0),
                                              static_cast<int>(nb), bmax);
  return check_launch("qkv_prefill_block_scores");
}
