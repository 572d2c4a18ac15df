// GQA-native sparse gather attention over selected KV blocks (bf16 K/V,
// fp32 accumulation), split over the selected tokens with a log-sum-exp merge.
//
// The reference expands K/V to every query head (evaluate_qwen3_top2_head_
// limit3_ppl.py:6248-6251) and then gathers per head (EV:4490-4502, kernel
// qabs_cuda_kernels.py:335-419).  Here the G query heads of a KV head share
// one pass over the selected rows: each 256-token split is read once from
// HBM (512 bytes per token), scored for all G heads, and its partial
// (max, sum, weighted V) goes to a workspace that a second kernel merges.
#include "common.h"

namespace qkv {
namespace {

constexpr int kD = 128;     // head dim
constexpr int kCT = 256;    // tokens per split workgroup
constexpr int kNT = 256;    // threads per workgroup

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u) return static_cast<uint16_t>((u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u));
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ void bf16x8(const uint4& raw, float* x) {
  x[0] = bf16lo(raw.x); x[1] = bf16hi(raw.x);
  x[2] = bf16lo(raw.y); x[3] = bf16hi(raw.y);
  x[4] = bf16lo(raw.z); x[5] = bf16hi(raw.z);
  x[6] = bf16lo(raw.w); x[7] = bf16hi(raw.w);
}

template <int G>
__global__ __launch_bounds__(kNT) void attn_partial_kernel(
    const uint16_t* __restrict__ query, const uint16_t* __restrict__ key,
    const uint16_t* __restrict__ value, int64_t sb, int64_t sh, int64_t st, int q_heads,
    int kv_heads, int tokens, const int32_t* __restrict__ block_ids, int n_sel, int block,
    int bps, float scale_log2, int nsplit, float* __restrict__ ws_acc, float* __restrict__ ws_ml) {
  __shared__ float q_s[G][kD];
  __shared__ int tok_s[kCT];
  __shared__ float p_s[G][kCT];
  __shared__ float red[kNT / 64][G];
  __shared__ float red_acc[kNT / 64][G][kD];
  __shared__ float ml_s[G][2];

  const int r = blockIdx.y, split = blockIdx.x;
  const int b = r / kv_heads, j = r - b * kv_heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nb = (tokens + block - 1) / block;
  const float ninf = -__builtin_huge_valf();

  const uint16_t* qrow = query + (static_cast<int64_t>(b) * q_heads + j * G) * kD;
  for (int i = tid; i < G * kD; i += kNT) q_s[i / kD][i % kD] = bf16_to_f32(qrow[i]);
  {
    int tok = -1;
    if (tid < bps * block) {
      const int slot = split * bps + tid / block;
      if (slot < n_sel) {
        const int id = block_ids[static_cast<int64_t>(r) * n_sel + slot];
        if (id >= 0 && id < nb) {
          const int tt = id * block + tid % block;
          if (tt < tokens) tok = tt;
        }
      }
    }
    tok_s[tid] = tok;
  }
  __syncthreads();

  const uint16_t* kbase = key + b * sb + j * sh;
  const uint16_t* vbase = value + b * sb + j * sh;

  // Phase 1: one token per thread, scores for all G heads (log2 domain).
  float s[G];
  {
    const int tok = tok_s[tid];
    if (tok >= 0) {
      const uint4* krow = reinterpret_cast<const uint4*>(kbase + static_cast<int64_t>(tok) * st);
      float acc[G];
#pragma unroll
      for (int h = 0; h < G; ++h) acc[h] = 0.0f;
#pragma unroll 4
      for (int c = 0; c < kD / 8; ++c) {
        float kx[8];
        bf16x8(krow[c], kx);
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[h] = __builtin_fmaf(q_s[h][c * 8 + i], kx[i], acc[h]);
      }
#pragma unroll
      for (int h = 0; h < G; ++h) s[h] = acc[h] * scale_log2;
    } else {
#pragma unroll
      for (int h = 0; h < G; ++h) s[h] = ninf;
    }
  }

  // Phase 2: split-local softmax statistics.
  float m[G], l[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float v = wave_max(s[h]);
    if (lane == 0) red[wave][h] = v;
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float v = red[0][h];
    for (int w = 1; w < kNT / 64; ++w) v = fmaxf(v, red[w][h]);
    m[h] = v;
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const float p = (s[h] == ninf) ? 0.0f : exp2f(s[h] - m[h]);
    p_s[h][tid] = p;
    const float v = wave_sum(p);
    if (lane == 0) red[wave][h] = v;
  }
  __syncthreads();
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float v = 0.0f;
    for (int w = 0; w < kNT / 64; ++w) v += red[w][h];
    l[h] = v;
  }

  // Phase 3: P.V with 16 dim groups (8 channels, one 128-bit load) x 16 token lanes.
  const int dg = tid & 15, tl = tid >> 4;
  float acc[G][8];
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[h][i] = 0.0f;
  for (int tt = tl; tt < kCT; tt += 16) {
    const int tk = tok_s[tt];
    if (tk < 0) continue;
    float vx[8];
    bf16x8(reinterpret_cast<const uint4*>(vbase + static_cast<int64_t>(tk) * st)[dg], vx);
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float p = p_s[h][tt];
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[h][i] = __builtin_fmaf(p, vx[i], acc[h][i]);
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float v = acc[h][i];
      v += shfl_xor(v, 16);
      v += shfl_xor(v, 32);
      acc[h][i] = v;
    }
  if (lane < 16) {
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int i = 0; i < 8; ++i) red_acc[wave][h][dg * 8 + i] = acc[h][i];
  }
  if (tid == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      ml_s[h][0] = m[h];
      ml_s[h][1] = l[h];
    }
  }
  __syncthreads();
  const int64_t part = static_cast<int64_t>(r) * nsplit + split;
  float* pacc = ws_acc + part * G * kD;
  for (int idx = tid; idx < G * kD; idx += kNT) {
    const int h = idx / kD, d = idx - h * kD;
    float v = red_acc[0][h][d];
    for (int w = 1; w < kNT / 64; ++w) v += red_acc[w][h][d];
    pacc[idx] = v;
  }
  if (tid < G) {
    ws_ml[(part * G + tid) * 2 + 0] = ml_s[tid][0];
    ws_ml[(part * G + tid) * 2 + 1] = ml_s[tid][1];
  }
}

template <int G>
__global__ __launch_bounds__(kD) void attn_merge_kernel(const float* __restrict__ ws_acc,
                                                        const float* __restrict__ ws_ml, int nsplit,
                                                        int q_heads, int kv_heads,
                                                        uint16_t* __restrict__ out) {
  const int r = blockIdx.x, d = threadIdx.x;
  const int b = r / kv_heads, j = r - b * kv_heads;
  const float ninf = -__builtin_huge_valf();
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float mx = ninf;
    for (int i = 0; i < nsplit; ++i) mx = fmaxf(mx, ws_ml[((static_cast<int64_t>(r) * nsplit + i) * G + h) * 2]);
    float o = 0.0f;
    if (mx != ninf) {
      float den = 0.0f;
      for (int i = 0; i < nsplit; ++i) {
        const int64_t part = static_cast<int64_t>(r) * nsplit + i;
        const float mi = ws_ml[(part * G + h) * 2];
        const float w = (mi == ninf) ? 0.0f : exp2f(mi - mx);
        den = __builtin_fmaf(ws_ml[(part * G + h) * 2 + 1], w, den);
        o = __builtin_fmaf(ws_acc[(part * G + h) * kD + d], w, o);
      }
      o = o / den;
    }
    out[(static_cast<int64_t>(b) * q_heads + j * G + h) * kD + d] = f32_to_bf16_rne(o);
  }
}

int64_t splits_for(int64_t n_sel, int64_t block) {
  const int64_t bps = std::max<int64_t>(1, kCT / block);
  return cdiv(n_sel, bps);
}

}  // namespace
}  // namespace qkv

using namespace qkv;

QKV_EXPORT int64_t qkv_sparse_attention_workspace_bytes(int64_t batch, int64_t q_heads,
                                                        int64_t kv_heads, int64_t head_dim,
                                                        int64_t n_sel, int64_t block) {
  if (batch <= 0 || kv_heads <= 0 || q_heads % kv_heads || head_dim != kD || n_sel <= 0 ||
      block <= 0 || block > kCT)
    return -1;
  const int64_t g = q_heads / kv_heads;
  return 4 * batch * kv_heads * splits_for(n_sel, block) * g * (kD + 2);
}

QKV_EXPORT int qkv_sparse_attention(const void* query, const void* key, const void* value,
                                    const int64_t* kv_strides, int64_t batch, int64_t q_heads,
                                    int64_t kv_heads, int64_t tokens, int64_t head_dim,
                                    const int32_t* block_ids, int64_t n_sel, int64_t block,
                                    float scaling, float* workspace, int64_t workspace_bytes,
                                    void* out, void* stream) {
  if (!query || !key || !value || !kv_strides || !block_ids || !workspace || !out)
    return fail(QKV_ERR_INVALID, "qkv_sparse_attention: null pointer");
  if (head_dim != kD) return fail(QKV_ERR_UNSUPPORTED, "qkv_sparse_attention: head_dim must be 128");
  if (batch <= 0 || kv_heads <= 0 || q_heads % kv_heads)
    return fail(QKV_ERR_INVALID, "qkv_sparse_attention: q_heads must be a multiple of kv_heads");
  const int64_t g = q_heads / kv_heads;
  if (g != 1 && g != 2 && g != 4 && g != 8)
    return fail(QKV_ERR_UNSUPPORTED, "qkv_sparse_attention: group size %lld not built", (long long)g);
  if (batch * kv_heads > 65535) return fail(QKV_ERR_INVALID, "qkv_sparse_attention: too many rows");
  if (tokens <= 0 || tokens >= (int64_t(1) << 30) || n_sel <= 0 || block <= 0 || block > kCT)
    return fail(QKV_ERR_INVALID, "qkv_sparse_attention: need tokens > 0, n_sel > 0, 1 <= block <= %d", kCT);
  if (!aligned(key, 16) || !aligned(value, 16) || (kv_strides[0] | kv_strides[1] | kv_strides[2]) % 8)
    return fail(QKV_ERR_INVALID, "qkv_sparse_attention: K/V rows must be 16-byte aligned");
  const int64_t need = qkv_sparse_attention_workspace_bytes(batch, q_heads, kv_heads, head_dim, n_sel, block);
  if (workspace_bytes < need)
    return fail(QKV_ERR_INVALID, "qkv_sparse_attention: workspace needs %lld bytes, got %lld",
                (long long)need, (long long)workspace_bytes);
  const int64_t rows = batch * kv_heads;
  const int64_t nsplit = splits_for(n_sel, block);
  if (nsplit > 65535) return fail(QKV_ERR_INVALID, "qkv_sparse_attention: too many selected blocks");
  const int bps = static_cast<int>(std::max<int64_t>(1, kCT / block));
  float* ws_acc = workspace;
  float* ws_ml = workspace + rows * nsplit * g * kD;
  const float scale_log2 = scaling * 1.4426950408889634f;
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<unsigned>(nsplit), static_cast<unsigned>(rows));
  const uint16_t* q = static_cast<const uint16_t*>(query);
  const uint16_t* k = static_cast<const uint16_t*>(key);
  const uint16_t* v = static_cast<const uint16_t*>(value);
  uint16_t* o = static_cast<uint16_t*>(out);
#define QKV_ATTN(GG)                                                                                    \
  attn_partial_kernel<GG><<<grid, kNT, 0, st>>>(q, k, v, kv_strides[0], kv_strides[1], kv_strides[2],   \
                                                static_cast<int>(q_heads), static_cast<int>(kv_heads),  \
                                                static_cast<int>(tokens), block_ids,                    \
                                                static_cast<int>(n_sel), static_cast<int>(block), bps,  \
                                                scale_log2, static_cast<int>(nsplit), ws_acc, ws_ml);   \
  if (int rc = check_launch("qkv_sparse_attention(partial)")) return rc;                              \
  attn_merge_kernel<GG><<<static_cast<unsigned>(rows), kD, 0, st>>>(ws_acc, ws_ml, static_cast<int>(nsplit), \
                                                                    static_cast<int>(q_heads),          \
                                                                    static_cast<int>(kv_heads), o);
  switch (g) {
    case 1: QKV_ATTN(1); break;
    case 2: QKV_ATTN(2); break;
    case 4: QKV_ATTN(4); break;
    default: QKV_ATTN(8); break;
  }
#undef QKV_ATTN
  return check_launch("qkv_sparse_attention(merge)");
}
