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
// fp32(scale/16) * fp32(16*I) equals fp32(scale) * fp32(I) exactly.
// The output tile has lane l hold keys 4*(l/16)+i of query l%16: a block max
// is an in-lane max plus two cross-row shuffles.
#include "common.h"

namespace qkv {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kD = 128;
constexpr int kBlock = 64;          // keys per selection block
constexpr int kChunkBlocks = 32;    // blocks per workgroup key chunk
constexpr int kQTile = 64;          // queries per wave (4 MFMA column tiles)
constexpr int kNT = 4;              // 16-query column tiles per wave

// Byte position, within a permuted query row, of channel c.
__host__ __device__ constexpr int perm_slot(int c) {
  const int g = c >> 5, half = (c >> 4) & 1, c16 = c & 15;
  return g * 32 + half * 16 + (c16 >> 3) * 8 + (c16 & 1) * 4 + ((c16 & 7) >> 1);
}

// ---------------------------------------------------------------------------
// Query quantization: one wave per query row.  q8 = clamp(rint(q / (amax/127)),
// +-127) over the row's 128 channels, written in the permuted MFMA order.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prefill_query_kernel(const uint16_t* __restrict__ q, int64_t q_row_stride,
                                                            int64_t rows, int8_t* __restrict__ q8,
                                                            float* __restrict__ qscale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint32_t w = reinterpret_cast<const uint32_t*>(q + row * q_row_stride)[lane];   // channels 2l, 2l+1
  const float x0 = bf16lo(w), x1 = bf16hi(w);
  const float amax = wave_max(fmaxf(fabsf(x0), fabsf(x1)));
  const float qs = amax / 127.0f;
  auto quant = [&](float v) -> int {
    if (qs == 0.0f) return 0;
    const float t = __builtin_rintf(v / qs);
    return static_cast<int>(fminf(fmaxf(t, -127.0f), 127.0f));
  };
  int8_t* out = q8 + row * kD;
  out[perm_slot(2 * lane)] = static_cast<int8_t>(quant(x0));
  out[perm_slot(2 * lane + 1)] = static_cast<int8_t>(quant(x1));
  if (qscale && lane == 0) qscale[row] = qs;
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
// streams the chunk's keys.  No workgroup barrier: the 4 waves of a group
// read the same keys (the other waves' loads hit in cache) and stage their
// block maxima in their own LDS region before a coalesced write.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void prefill_scores_kernel(
    const int8_t* __restrict__ q8, const uint8_t* __restrict__ kpacked, const uint16_t* __restrict__ kscales,
    int q_heads, int kv_heads, int nq, int tokens, int64_t capacity, int q_pos0, int nb,
    float* __restrict__ bmax) {
  __shared__ float tile[4][kQTile][kChunkBlocks + 1];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
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
  const uint8_t* krow = kpacked + static_cast<int64_t>(bj) * capacity * (kD / 2);
  const uint16_t* srow = kscales + static_cast<int64_t>(bj) * capacity;
  const float ninf = -__builtin_huge_valf();

  for (int kb = 0; kb < nblk; ++kb) {
    const int base = (blk0 + kb) * kBlock;
    float run[kNT];
#pragma unroll
    for (int n = 0; n < kNT; ++n) run[n] = ninf;
    if (base <= pos_hi) {   // some key of the block is visible to some query
      const bool need_mask = base + kBlock - 1 > pos_lo || base + kBlock > tokens;
#pragma unroll
      for (int kt = 0; kt < 4; ++kt) {
        const int key = base + kt * 16 + col;
        const uint4 raw = *reinterpret_cast<const uint4*>(krow + static_cast<int64_t>(key) * (kD / 2) + g * 16);
        const v4i a0 = unpack_half(raw.x, raw.y);
        const v4i a1 = unpack_half(raw.z, raw.w);
        // scales of the 4 keys this lane's output rows hold: base + 16kt + 4g + i
        const uint2 sraw = *reinterpret_cast<const uint2*>(srow + base + kt * 16 + 4 * g);
        float s16[4];
        s16[0] = f16bits_to_f32(sraw.x & 0xFFFFu) * 0.0625f;
        s16[1] = f16bits_to_f32(sraw.x >> 16) * 0.0625f;
        s16[2] = f16bits_to_f32(sraw.y & 0xFFFFu) * 0.0625f;
        s16[3] = f16bits_to_f32(sraw.y >> 16) * 0.0625f;
#pragma unroll
        for (int n = 0; n < kNT; ++n) {
          v4i acc = v4i{0, 0, 0, 0};
          acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, bq[n][0], acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, bq[n][1], acc, 0, 0, 0);
          const int accs[4] = {acc.x, acc.y, acc.z, acc.w};
          if (!need_mask) {
#pragma unroll
            for (int i = 0; i < 4; ++i) run[n] = fmaxf(run[n], s16[i] * static_cast<float>(accs[i]));
          } else {
            const int qpos = q_pos0 + q0 + 16 * n + col;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int t = base + kt * 16 + 4 * g + i;
              const float v = s16[i] * static_cast<float>(accs[i]);
              run[n] = fmaxf(run[n], (t <= qpos && t < tokens) ? v : ninf);
            }
          }
        }
      }
    }
    // Max over the 4 row groups; -0 (only from a zero scale) reads as +0.
#pragma unroll
    for (int n = 0; n < kNT; ++n) {
      float m = run[n];
      m = fmaxf(m, swz_xor<16>(m));
      m = fmaxf(m, shfl_xor(m, 32));
      m = (m == 0.0f) ? 0.0f : m;
      if (lane < 16) tile[wave][16 * n + col][kb] = m;
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
  if (cdiv(rows, 4) > 0x7FFFFFFF) return fail(QKV_ERR_INVALID, "qkv_prefill_quantize_query: too many rows");
  hipStream_t st = static_cast<hipStream_t>(stream);
  prefill_query_kernel<<<static_cast<unsigned>(cdiv(rows, 4)), 256, 0, st>>>(
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
