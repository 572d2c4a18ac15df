// The four kernels behind the reference's Python API, with the reference's
// numerics (fp32 accumulation in the reference's order), written for gfx950:
// the channel selector is a wave-parallel stable rank instead of a serial
// scan, and the attention kernel spreads the selected rows over the whole
// workgroup.  Citations: QK = ymluo/projects/qwen3_top2_head_limit3_ppl/src/
// qabs_cuda_kernels.py.
//
// Built with -ffp-contract=off: every `acc + a * b` below is a separately
// rounded multiply and add, so results equal a sequential fp32 loop.
#include "ref_common.h"

namespace qkv {
namespace {

constexpr int kTile = 256;      // tokens per workgroup (QK:61)

template <int DT>
__global__ __launch_bounds__(kTile) void partial_scores_kernel(
    const typename Elem<DT>::T* __restrict__ query, const typename Elem<DT>::T* __restrict__ key,
    float* __restrict__ out, int heads, int keys, int head_dim, int count, int64_t ksb,
    int64_t ksh, int64_t kst, int64_t ksd) {
  __shared__ int sel_idx[kMaxDims];
  __shared__ float sel_q[kMaxDims];
  const int row = blockIdx.y;
  const int b = row / heads, h = row - b * heads;
  select_dims<DT>(query + static_cast<int64_t>(row) * head_dim, head_dim, count, sel_idx, sel_q);
  __syncthreads();
  const int t = blockIdx.x * kTile + threadIdx.x;
  if (t >= keys) return;
  const typename Elem<DT>::T* k_row = key + b * ksb + h * ksh + t * kst;
  float acc = 0.0f;
  for (int s = 0; s < count; ++s) acc = acc + sel_q[s] * Elem<DT>::load(k_row + sel_idx[s] * ksd);
  out[static_cast<int64_t>(row) * keys + t] = acc;
}

template <int DT>
__global__ __launch_bounds__(kTile) void partial_scores_dim_major_kernel(
    const typename Elem<DT>::T* __restrict__ query, const typename Elem<DT>::T* __restrict__ kdm,
    const int64_t* __restrict__ dim_indices, float* __restrict__ out, int heads, int keys,
    int head_dim, int count, int64_t ksb, int64_t ksh, int64_t ksd, int64_t kst) {
  __shared__ int sel_idx[kMaxDims];
  __shared__ float sel_q[kMaxDims];
  const int row = blockIdx.y;
  const int b = row / heads, h = row - b * heads;
  const typename Elem<DT>::T* q_row = query + static_cast<int64_t>(row) * head_dim;
  const int64_t* dims = dim_indices + static_cast<int64_t>(row) * count;
  for (int s = threadIdx.x; s < count; s += blockDim.x) {
    // an index outside [0, D) is clamped rather than read out of bounds
    int d = static_cast<int>(min(max(dims[s], int64_t(0)), int64_t(head_dim - 1)));
    sel_idx[s] = d;
    sel_q[s] = Elem<DT>::load(q_row + d);
  }
  __syncthreads();
  const int t = blockIdx.x * kTile + threadIdx.x;
  if (t >= keys) return;
  const typename Elem<DT>::T* k_base = kdm + b * ksb + h * ksh + t * kst;
  float acc = 0.0f;
  for (int s = 0; s < count; ++s) acc = acc + sel_q[s] * Elem<DT>::load(k_base + sel_idx[s] * ksd);
  out[static_cast<int64_t>(row) * keys + t] = acc;
}

template <int DT>
__global__ __launch_bounds__(kTile) void candidate_full_scores_kernel(
    const typename Elem<DT>::T* __restrict__ query, const typename Elem<DT>::T* __restrict__ key,
    const uint8_t* __restrict__ current, const uint8_t* __restrict__ previous,
    const uint8_t* __restrict__ previous_final, float* __restrict__ out, int heads, int keys,
    int head_dim, int sink, int recent, float scaling, int64_t ksb, int64_t ksh, int64_t kst,
    int64_t ksd) {
  __shared__ float q_s[512];
  const int row = blockIdx.y;
  const int b = row / heads, h = row - b * heads;
  const typename Elem<DT>::T* q_row = query + static_cast<int64_t>(row) * head_dim;
  for (int d = threadIdx.x; d < head_dim; d += blockDim.x) q_s[d] = Elem<DT>::load(q_row + d);
  __syncthreads();
  const int t = blockIdx.x * kTile + threadIdx.x;
  if (t >= keys) return;
  const int64_t off = static_cast<int64_t>(row) * keys + t;
  bool sel = current[off] != 0;
  if (previous) sel = sel || previous[off] != 0;
  if (previous_final) sel = sel || previous_final[off] != 0;
  if (sink > 0 && t < sink) sel = true;
  if (recent > 0 && t >= max(0, keys - recent)) sel = true;
  if (!sel) {
    out[off] = -__builtin_huge_valf();
    return;
  }
  const typename Elem<DT>::T* k_row = key + b * ksb + h * ksh + t * kst;
  float acc = 0.0f;
  for (int d = 0; d < head_dim; ++d) acc = acc + q_s[d] * Elem<DT>::load(k_row + d * ksd);
  out[off] = acc * scaling;
}

// Sparse attention with the reference kernel's semantics (QK:335-419): one
// workgroup per (b,h); selected rows are scored across all threads, then
// every thread owns output channels.  Scores live in dynamic LDS.
template <int DT>
__global__ __launch_bounds__(256) void final_attention_kernel(
    const typename Elem<DT>::T* __restrict__ query, const typename Elem<DT>::T* __restrict__ key,
    const typename Elem<DT>::T* __restrict__ value, const int64_t* __restrict__ indices,
    const uint8_t* __restrict__ valid, typename Elem<DT>::T* __restrict__ out, int keys,
    int selected, int head_dim, float scaling) {
  extern __shared__ float smem[];
  float* w = smem;                 // [selected]
  float* q_s = smem + selected;    // [head_dim]
  __shared__ float red[256 / 64];
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6, nwaves = blockDim.x >> 6;
  const typename Elem<DT>::T* q_row = query + static_cast<int64_t>(row) * head_dim;
  const typename Elem<DT>::T* k_base = key + static_cast<int64_t>(row) * keys * head_dim;
  const typename Elem<DT>::T* v_base = value + static_cast<int64_t>(row) * keys * head_dim;
  const int64_t* idx_row = indices + static_cast<int64_t>(row) * selected;
  const uint8_t* valid_row = valid + static_cast<int64_t>(row) * selected;
  for (int d = tid; d < head_dim; d += blockDim.x) q_s[d] = Elem<DT>::load(q_row + d);
  __syncthreads();

  const float ninf = -__builtin_huge_valf();
  float local_max = ninf;
  for (int s = tid; s < selected; s += blockDim.x) {
    int64_t idx = idx_row[s];
    float score = ninf;
    if (valid_row[s] != 0 && idx >= 0 && idx < keys) {
      const typename Elem<DT>::T* k_vec = k_base + idx * head_dim;
      float acc = 0.0f;
      for (int d = 0; d < head_dim; ++d) acc = acc + q_s[d] * Elem<DT>::load(k_vec + d);
      score = acc * scaling;
      local_max = fmaxf(local_max, score);
    }
    w[s] = score;
  }
  local_max = wave_max(local_max);
  if (lane == 0) red[wave] = local_max;
  __syncthreads();
  float m = red[0];
  for (int i = 1; i < nwaves; ++i) m = fmaxf(m, red[i]);
  if (!(m > ninf && m < __builtin_huge_valf())) m = 0.0f;   // QK:388
  __syncthreads();

  float local_den = 0.0f;
  for (int s = tid; s < selected; s += blockDim.x) {
    float sc = w[s];
    float e = (sc > ninf) ? __expf(sc - m) : 0.0f;
    w[s] = e;
    local_den += e;
  }
  local_den = wave_sum(local_den);
  if (lane == 0) red[wave] = local_den;
  __syncthreads();
  float den = 0.0f;
  for (int i = 0; i < nwaves; ++i) den += red[i];
  den = fmaxf(den, 1.0e-20f);   // QK:404
  const float inv = 1.0f / den;

  for (int d = tid; d < head_dim; d += blockDim.x) {
    float acc = 0.0f;
    for (int s = 0; s < selected; ++s) {
      float ws = w[s];
      if (ws != 0.0f) {
        int64_t idx = idx_row[s];
        if (idx >= 0 && idx < keys) acc += (ws * inv) * Elem<DT>::load(v_base + idx * head_dim + d);
      }
    }
    out[static_cast<int64_t>(row) * head_dim + d] = Elem<DT>::store(acc);
  }
}

template <int DT> struct RunPartial {
  static int run(const void* q, const void* k, float* out, int64_t B, int64_t H, int64_t T,
                 int64_t D, const int64_t* ks, int count, hipStream_t st) {
    using E = typename Elem<DT>::T;
    dim3 grid(static_cast<unsigned>(cdiv(T, kTile)), static_cast<unsigned>(B * H));
    partial_scores_kernel<DT><<<grid, kTile, 0, st>>>(
        static_cast<const E*>(q), static_cast<const E*>(k), out, static_cast<int>(H),
        static_cast<int>(T), static_cast<int>(D), count, ks[0], ks[1], ks[2], ks[3]);
    return check_launch("qkv_partial_scores");
  }
};
template <int DT> struct RunDimMajor {
  static int run(const void* q, const void* kdm, const int64_t* idx, float* out, int64_t B,
                 int64_t H, int64_t T, int64_t D, int64_t S, const int64_t* ks, hipStream_t st) {
    using E = typename Elem<DT>::T;
    dim3 grid(static_cast<unsigned>(cdiv(T, kTile)), static_cast<unsigned>(B * H));
    partial_scores_dim_major_kernel<DT><<<grid, kTile, 0, st>>>(
        static_cast<const E*>(q), static_cast<const E*>(kdm), idx, out, static_cast<int>(H),
        static_cast<int>(T), static_cast<int>(D), static_cast<int>(S), ks[0], ks[1], ks[2], ks[3]);
    return check_launch("qkv_partial_scores_dim_major");
  }
};
template <int DT> struct RunCandidate {
  static int run(const void* q, const void* k, const uint8_t* cur, const uint8_t* prev,
                 const uint8_t* pfin, float* out, int64_t B, int64_t H, int64_t T, int64_t D,
                 const int64_t* ks, int sink, int recent, float scaling, hipStream_t st) {
    using E = typename Elem<DT>::T;
    dim3 grid(static_cast<unsigned>(cdiv(T, kTile)), static_cast<unsigned>(B * H));
    candidate_full_scores_kernel<DT><<<grid, kTile, 0, st>>>(
        static_cast<const E*>(q), static_cast<const E*>(k), cur, prev, pfin, out,
        static_cast<int>(H), static_cast<int>(T), static_cast<int>(D), sink, recent, scaling,
        ks[0], ks[1], ks[2], ks[3]);
    return check_launch("qkv_candidate_full_scores");
  }
};
template <int DT> struct RunFinal {
  static int run(const void* q, const void* k, const void* v, const int64_t* idx,
                 const uint8_t* valid, void* out, int64_t B, int64_t H, int64_t T, int64_t N,
                 int64_t D, float scaling, hipStream_t st) {
    using E = typename Elem<DT>::T;
    size_t lds = static_cast<size_t>(N + D) * sizeof(float);
    final_attention_kernel<DT><<<static_cast<unsigned>(B * H), 256, lds, st>>>(
        static_cast<const E*>(q), static_cast<const E*>(k), static_cast<const E*>(v), idx, valid,
        static_cast<E*>(out), static_cast<int>(T), static_cast<int>(N), static_cast<int>(D),
        scaling);
    return check_launch("qkv_final_attention");
  }
};

int check_common(const void* q, const void* k, int64_t B, int64_t H, int64_t T, int64_t D,
                 const char* what) {
  if (!q || !k) return fail(QKV_ERR_INVALID, "%s: null input pointer", what);
  if (B <= 0 || H <= 0 || T < 0 || D <= 0)
    return fail(QKV_ERR_INVALID, "%s: bad sizes B=%lld H=%lld T=%lld D=%lld", what,
                (long long)B, (long long)H, (long long)T, (long long)D);
  if (B * H > 65535) return fail(QKV_ERR_INVALID, "%s: batch*heads must be <= 65535", what);
  if (T >= (int64_t(1) << 31)) return fail(QKV_ERR_INVALID, "%s: too many keys", what);
  return QKV_OK;
}

}  // namespace
}  // namespace qkv

using namespace qkv;

QKV_EXPORT int qkv_partial_scores(const void* query, const void* key, float* out, int dtype,
                                  int64_t batch, int64_t heads, int64_t keys, int64_t head_dim,
                                  const int64_t* k_strides, int64_t dim_count, void* stream) {
  int rc = check_common(query, key, batch, heads, keys, head_dim, "qkv_partial_scores");
  if (rc) return rc;
  if (!out || !k_strides) return fail(QKV_ERR_INVALID, "qkv_partial_scores: null pointer");
  if (keys == 0) return QKV_OK;
  int count = static_cast<int>(std::min<int64_t>(std::max<int64_t>(dim_count, 1),
                                                 std::min<int64_t>(head_dim, kMaxDims)));
  return dispatch_dtype<RunPartial>(dtype, query, key, out, batch, heads, keys, head_dim, k_strides,
                                    count, static_cast<hipStream_t>(stream));
}

QKV_EXPORT int qkv_partial_scores_dim_major(const void* query, const void* key_dim_major,
                                            const int64_t* dim_indices, float* out, int dtype,
                                            int64_t batch, int64_t heads, int64_t keys,
                                            int64_t head_dim, int64_t selected,
                                            const int64_t* kdm_strides, void* stream) {
  int rc = check_common(query, key_dim_major, batch, heads, keys, head_dim,
                        "qkv_partial_scores_dim_major");
  if (rc) return rc;
  if (!out || !dim_indices || !kdm_strides)
    return fail(QKV_ERR_INVALID, "qkv_partial_scores_dim_major: null pointer");
  if (selected < 1 || selected > kMaxDims)
    return fail(QKV_ERR_INVALID, "qkv_partial_scores_dim_major: selected dims must be in [1, %d]",
                kMaxDims);
  if (keys == 0) return QKV_OK;
  return dispatch_dtype<RunDimMajor>(dtype, query, key_dim_major, dim_indices, out, batch, heads,
                                     keys, head_dim, selected, kdm_strides,
                                     static_cast<hipStream_t>(stream));
}

QKV_EXPORT int qkv_candidate_full_scores(const void* query, const void* key, const uint8_t* current,
                                         const uint8_t* previous, const uint8_t* previous_final,
                                         float* out, int dtype, int64_t batch, int64_t heads,
                                         int64_t keys, int64_t head_dim, const int64_t* k_strides,
                                         int64_t protect_sink, int64_t protect_recent,
                                         float scaling, void* stream) {
  int rc = check_common(query, key, batch, heads, keys, head_dim, "qkv_candidate_full_scores");
  if (rc) return rc;
  if (!out || !current || !k_strides)
    return fail(QKV_ERR_INVALID, "qkv_candidate_full_scores: null pointer");
  if (head_dim > 512) return fail(QKV_ERR_UNSUPPORTED, "qkv_candidate_full_scores: head_dim > 512");
  if (keys == 0) return QKV_OK;
  int sink = static_cast<int>(std::min<int64_t>(std::max<int64_t>(protect_sink, 0), keys));
  int recent = static_cast<int>(std::min<int64_t>(std::max<int64_t>(protect_recent, 0), keys));
  return dispatch_dtype<RunCandidate>(dtype, query, key, current, previous, previous_final, out,
                                      batch, heads, keys, head_dim, k_strides, sink, recent,
                                      scaling, static_cast<hipStream_t>(stream));
}

QKV_EXPORT int qkv_final_attention(const void* query, const void* key, const void* value,
                                   const int64_t* indices, const uint8_t* valid, void* out,
                                   int dtype, int64_t batch, int64_t heads, int64_t keys,
                                   int64_t selected, int64_t head_dim, float scaling,
                                   void* stream) {
  int rc = check_common(query, key, batch, heads, keys, head_dim, "qkv_final_attention");
  if (rc) return rc;
  if (!value || !indices || !valid || !out)
    return fail(QKV_ERR_INVALID, "qkv_final_attention: null pointer");
  if (selected <= 0) return fail(QKV_ERR_INVALID, "select_count must be positive");   // QK:609
  if (selected + head_dim > 16384 + 512)
    return fail(QKV_ERR_UNSUPPORTED, "qkv_final_attention: at most 16384 selected rows");
  return dispatch_dtype<RunFinal>(dtype, query, key, value, indices, valid, out, batch, heads, keys,
                                  selected, head_dim, scaling, static_cast<hipStream_t>(stream));
}
