// GQA-native sparse gather attention over selected KV blocks (bf16 K/V,
// fp32 softmax and accumulation), one launch per call.
//
// The reference expands K/V to every query head (evaluate_qwen3_top2_head_
// limit3_ppl.py:6248-6251) and then gathers per head (EV:4490-4502, kernel
// qabs_cuda_kernels.py:335-419).  Here the G query heads of a KV head share
// one pass over the selected rows, so every selected K/V row is read from HBM
// once (512 bytes per token at D = 128).
//
// Work split: a workgroup (4 waves) owns 16*NI consecutive token slots of one
// (sequence, KV head) row, where slot s is token (block_ids[s / block] * block
// + s % block).  Inside a wave, 16 lanes share a token: lane (16*g + c) holds
// channels 8c..8c+7 of the token of slot 4i + g in iteration i, so each load
// instruction reads four whole 256-byte K (or V) rows.  All K and V loads of a
// wave are issued before any arithmetic.  QK is v_dot2_f32_bf16 on the packed
// channel pairs followed by a 16-lane DPP reduction; softmax runs in the log2
// domain; P.V accumulates in fp32.  Each workgroup reduces its waves through
// LDS into (max, sum, weighted V) per head.  A row that fits one workgroup
// writes its bf16 output directly.  Otherwise every workgroup publishes its
// partial with device-coherent stores (relaxed agent-scope atomic stores:
// global_store sc1, written through the XCD's L2), waits for them to
// complete, and takes a ticket; the row's last workgroup reads the partials
// back with device-coherent loads (sc1) and writes the output.  No release /
// acquire fence is used: on gfx950 those write back and invalidate the whole
// L2 of the XCD (buffer_wbl2 / buffer_inv), which measured 3x slower here.
#include "common.h"

namespace qkv {
namespace {

constexpr int kD = 128;     // head dim
constexpr int kNT = 256;    // threads per workgroup
// Ticket words at the start of the workspace, one per possible row, so calls
// of any shape that share a workspace find their tickets at the same place.
constexpr int64_t kTicketWords = 65536;

__device__ __forceinline__ void st_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u) return static_cast<uint16_t>((u >> 16) | ((u & 0xFFFFu) ? 0x40u : 0u));
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte load with the non-temporal hint: K/V rows are read once per step.
__device__ __forceinline__ uint4 ld_nt(const uint16_t* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c,
                                         false);
}

template <int DPP>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP, 0xF, 0xF, false));
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

template <int G, int NI>
__global__ __launch_bounds__(kNT) void sparse_attn_kernel(
    const uint16_t* __restrict__ query, const uint16_t* __restrict__ key,
    const uint16_t* __restrict__ value, int64_t sb, int64_t sh, int64_t st, int q_heads,
    int kv_heads, int64_t tokens, const int32_t* __restrict__ block_ids, int n_sel, int block,
    int nb, float scale_log2, int nsplit, float* __restrict__ ws_acc, float* __restrict__ ws_ml,
    uint32_t* __restrict__ tickets, uint16_t* __restrict__ out) {
  constexpr int SLOTS_W = 4 * NI;          // token slots per wave
  constexpr int SLOTS_WG = 4 * SLOTS_W;    // token slots per workgroup
  static_assert(SLOTS_W <= 64, "one slot per lane when resolving token ids");

  __shared__ float red_acc[4][G][kD];   // per wave weighted V
  __shared__ float red_m[4][G], red_l[4][G];
  __shared__ int last_flag;

  const int r = blockIdx.y, split = blockIdx.x;
  const int b = r / kv_heads, j = r - b * kv_heads;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = lane >> 4, cc = lane & 15;
  const float ninf = -__builtin_huge_valf();

  // Token id of slot (wave base + lane), then of this lane's slot 4i + grp.
  int my_tok = -1;
  if (lane < SLOTS_W) {
    const int64_t slot = static_cast<int64_t>(split) * SLOTS_WG + wave * SLOTS_W + lane;
    const int64_t bs = slot / block;
    if (bs < n_sel) {
      const int id = block_ids[static_cast<int64_t>(r) * n_sel + bs];
      if (id >= 0 && id < nb) {
        const int64_t t = static_cast<int64_t>(id) * block + (slot - bs * block);
        if (t < tokens) my_tok = static_cast<int>(t);
      }
    }
  }
  int tok[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) tok[i] = __builtin_amdgcn_ds_bpermute((4 * i + grp) << 2, my_tok);

  const uint16_t* kb = key + b * sb + j * sh + cc * 8;
  const uint16_t* vb = value + b * sb + j * sh + cc * 8;
  uint4 kx[NI], vx[NI];
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    kx[i] = make_uint4(0, 0, 0, 0);
    if (tok[i] >= 0) kx[i] = ld_nt(kb + static_cast<int64_t>(tok[i]) * st);
  }
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    vx[i] = make_uint4(0, 0, 0, 0);
    if (tok[i] >= 0) vx[i] = ld_nt(vb + static_cast<int64_t>(tok[i]) * st);
  }
  uint4 qx[G];
  const uint16_t* qrow = query + (static_cast<int64_t>(b) * q_heads + j * G) * kD + cc * 8;
#pragma unroll
  for (int h = 0; h < G; ++h) qx[h] = *reinterpret_cast<const uint4*>(qrow + h * kD);

  // Scores (log2 domain) and the wave max per head.
  float s[G][NI];
  float m[G];
#pragma unroll
  for (int h = 0; h < G; ++h) m[h] = ninf;
#pragma unroll
  for (int i = 0; i < NI; ++i) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      float a = dot2_bf16(qx[h].x, kx[i].x, 0.0f);
      a = dot2_bf16(qx[h].y, kx[i].y, a);
      a = dot2_bf16(qx[h].z, kx[i].z, a);
      a = dot2_bf16(qx[h].w, kx[i].w, a);
      a = row16_sum(a) * scale_log2;
      s[h][i] = tok[i] >= 0 ? a : ninf;
      m[h] = fmaxf(m[h], s[h][i]);
    }
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
    m[h] = fmaxf(m[h], shfl_xor(m[h], 16));
    m[h] = fmaxf(m[h], shfl_xor(m[h], 32));
  }

  // p = 2^(s - m); per-group sums and P.V over this lane's 8 channels.
  float acc[G][8];
  float l[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    l[h] = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) acc[h][c] = 0.0f;
  }
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    float v[8];
    v[0] = bf16lo(vx[i].x); v[1] = bf16hi(vx[i].x);
    v[2] = bf16lo(vx[i].y); v[3] = bf16hi(vx[i].y);
    v[4] = bf16lo(vx[i].z); v[5] = bf16hi(vx[i].z);
    v[6] = bf16lo(vx[i].w); v[7] = bf16hi(vx[i].w);
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float p = (s[h][i] == ninf) ? 0.0f : exp2f(s[h][i] - m[h]);
      l[h] += p;
#pragma unroll
      for (int c = 0; c < 8; ++c) acc[h][c] = __builtin_fmaf(p, v[c], acc[h][c]);
    }
  }

  // The four token groups of a wave share the wave max: sum them in
  // registers, then combine the four waves through LDS.
#pragma unroll
  for (int h = 0; h < G; ++h) {
    l[h] += shfl_xor(l[h], 16);
    l[h] += shfl_xor(l[h], 32);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      acc[h][c] += shfl_xor(acc[h][c], 16);
      acc[h][c] += shfl_xor(acc[h][c], 32);
    }
  }
  if (grp == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int c = 0; c < 8; ++c) red_acc[wave][h][cc * 8 + c] = acc[h][c];
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      red_m[wave][h] = m[h];
      red_l[wave][h] = l[h];
    }
  }
  __syncthreads();

  // Workgroup max per head and the rescale factor of each wave.
  float wg_m[G], wg_l[G], fs[G][4];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float mx = fmaxf(fmaxf(red_m[0][h], red_m[1][h]), fmaxf(red_m[2][h], red_m[3][h]));
    wg_m[h] = mx;
    float sum = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      fs[h][w] = (red_m[w][h] == ninf) ? 0.0f : exp2f(red_m[w][h] - mx);
      sum = __builtin_fmaf(red_l[w][h], fs[h][w], sum);
    }
    wg_l[h] = sum;
  }
  auto wg_acc = [&](int h, int d) -> float {
    float o = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) o = __builtin_fmaf(red_acc[w][h][d], fs[h][w], o);
    return o;
  };

  if (nsplit == 1) {
    for (int idx = tid; idx < G * kD; idx += kNT) {
      const int h = idx / kD, d = idx - h * kD;
      const float o = (wg_m[h] == ninf) ? 0.0f : wg_acc(h, d) / wg_l[h];
      out[(static_cast<int64_t>(b) * q_heads + j * G + h) * kD + d] = f32_to_bf16_rne(o);
    }
    return;
  }

  const int64_t part = static_cast<int64_t>(r) * nsplit + split;
  for (int idx = tid; idx < G * kD; idx += kNT) {
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

  // Last workgroup of the row: merge the splits, MS at a time with every load
  // in flight before any arithmetic.
  constexpr int MS = 8;
  for (int idx = tid; idx < G * kD; idx += kNT) {
    const int h = idx / kD;
    const float* ml = ws_ml + static_cast<int64_t>(r) * nsplit * G * 2 + h * 2;
    const float* pa = ws_acc + static_cast<int64_t>(r) * nsplit * G * kD + idx;
    float mx = ninf, den = 0.0f, o = 0.0f;
    for (int i0 = 0; i0 < nsplit; i0 += MS) {
      float mi[MS], li[MS], ai[MS];
#pragma unroll
      for (int u = 0; u < MS; ++u) {
        const int i = min(i0 + u, nsplit - 1);
        mi[u] = ld_coherent(ml + i * G * 2);
        li[u] = ld_coherent(ml + i * G * 2 + 1);
        ai[u] = ld_coherent(pa + static_cast<int64_t>(i) * G * kD);
      }
      float m2 = mx;
#pragma unroll
      for (int u = 0; u < MS; ++u)
        if (i0 + u < nsplit) m2 = fmaxf(m2, mi[u]);
      if (m2 == ninf) continue;
      const float c = (mx == ninf) ? 0.0f : exp2f(mx - m2);
      den *= c;
      o *= c;
#pragma unroll
      for (int u = 0; u < MS; ++u) {
        if (i0 + u < nsplit && mi[u] != ninf) {
          const float w = exp2f(mi[u] - m2);
          den = __builtin_fmaf(li[u], w, den);
          o = __builtin_fmaf(ai[u], w, o);
        }
      }
      mx = m2;
    }
    o = (mx == ninf) ? 0.0f : o / den;
    out[(static_cast<int64_t>(b) * q_heads + j * G) * kD + idx] = f32_to_bf16_rne(o);
  }
}

// Token slots per wave / 4 (128 slots per workgroup: measured faster than 256 at cfg2).
constexpr int ni_for(int64_t g) { return 8; }

int64_t splits_for(int64_t n_sel, int64_t block, int64_t g) {
  return cdiv(n_sel * block, 16 * ni_for(g));
}

}  // namespace
}  // namespace qkv

using namespace qkv;

QKV_EXPORT int64_t qkv_sparse_attention_workspace_bytes(int64_t batch, int64_t q_heads,
                                                        int64_t kv_heads, int64_t head_dim,
                                                        int64_t n_sel, int64_t block) {
  if (batch <= 0 || kv_heads <= 0 || q_heads % kv_heads || head_dim != kD || n_sel <= 0 ||
      block <= 0 || n_sel * block >= (int64_t(1) << 31))
    return -1;
  const int64_t g = q_heads / kv_heads;
  const int64_t rows = batch * kv_heads;
  // tickets, then per split: weighted V per head, then (max, sum) per head
  return 4 * (kTicketWords + rows * splits_for(n_sel, block, g) * g * (kD + 2));
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
  if (tokens <= 0 || tokens >= (int64_t(1) << 31) || n_sel <= 0 || block <= 0 ||
      n_sel * block >= (int64_t(1) << 31))
    return fail(QKV_ERR_INVALID, "qkv_sparse_attention: need tokens > 0, n_sel > 0, block > 0");
  if (!aligned(query, 16) || !aligned(key, 16) || !aligned(value, 16) ||
      (kv_strides[0] | kv_strides[1] | kv_strides[2]) % 8)
    return fail(QKV_ERR_INVALID, "qkv_sparse_attention: q/K/V rows must be 16-byte aligned");
  const int64_t need = qkv_sparse_attention_workspace_bytes(batch, q_heads, kv_heads, head_dim, n_sel, block);
  if (workspace_bytes < need)
    return fail(QKV_ERR_INVALID, "qkv_sparse_attention: workspace needs %lld bytes, got %lld",
                (long long)need, (long long)workspace_bytes);
  const int64_t rows = batch * kv_heads;
  const int64_t nsplit = splits_for(n_sel, block, g);
  if (nsplit > 65535) return fail(QKV_ERR_INVALID, "qkv_sparse_attention: too many selected blocks");
  uint32_t* tickets = reinterpret_cast<uint32_t*>(workspace);
  float* ws_acc = workspace + kTicketWords;
  float* ws_ml = ws_acc + rows * nsplit * g * kD;
  const int nb = static_cast<int>(cdiv(tokens, block));
  const float scale_log2 = scaling * 1.4426950408889634f;
  hipStream_t st = static_cast<hipStream_t>(stream);
  dim3 grid(static_cast<unsigned>(nsplit), static_cast<unsigned>(rows));
  const uint16_t* q = static_cast<const uint16_t*>(query);
  const uint16_t* k = static_cast<const uint16_t*>(key);
  const uint16_t* v = static_cast<const uint16_t*>(value);
  uint16_t* o = static_cast<uint16_t*>(out);
#define QKV_ATTN(GG)                                                                                   \
  sparse_attn_kernel<GG, ni_for(GG)><<<grid, kNT, 0, st>>>(                                            \
      q, k, v, kv_strides[0], kv_strides[1], kv_strides[2], static_cast<int>(q_heads),                 \
      static_cast<int>(kv_heads), tokens, block_ids, static_cast<int>(n_sel), static_cast<int>(block), \
      nb, scale_log2, static_cast<int>(nsplit), ws_acc, ws_ml, tickets, o)
  switch (g) {
    case 1: QKV_ATTN(1); break;
    case 2: QKV_ATTN(2); break;
    case 4: QKV_ATTN(4); break;
    default: QKV_ATTN(8); break;
  }
#undef QKV_ATTN
  return check_launch("qkv_sparse_attention");
}
