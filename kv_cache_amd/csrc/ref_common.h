// Element access for the reference's three dtypes, the reference's
// top-|q| dimension selector, and dtype dispatch: shared by the
// reference-semantics kernels and the candidate-reuse kernels.
#pragma once
#include "common.h"

namespace qkv {
namespace {

constexpr int kMaxDims = 128;   // QK:60

template <int DT> struct Elem;
template <> struct Elem<QKV_DTYPE_BF16> {
  using T = uint16_t;
  static __device__ __forceinline__ float load(const T* p) { return bf16_to_f32(*p); }
  static __device__ __forceinline__ T store(float f) {
    // round-to-nearest-even fp32 -> bf16 (finite inputs)
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7F800000u) == 0x7F800000u) return static_cast<T>(u >> 16);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return static_cast<T>(u >> 16);
  }
};
template <> struct Elem<QKV_DTYPE_FP16> {
  using T = uint16_t;
  static __device__ __forceinline__ float load(const T* p) { return f16bits_to_f32(*p); }
  static __device__ __forceinline__ T store(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  }
};
template <> struct Elem<QKV_DTYPE_FP32> {
  using T = float;
  static __device__ __forceinline__ float load(const T* p) { return *p; }
  static __device__ __forceinline__ T store(float f) { return f; }
};

// Selects the top-|q| dims of one query row into LDS in the reference's order:
// descending |q|, equal magnitudes by ascending dim (QK:123-145 uses a strict
// '>' over ascending d).  rank(d) = #{d' : |q_d'| > |q_d| or (== and d' < d)}.
template <int DT>
__device__ void select_dims(const typename Elem<DT>::T* q_row, int head_dim, int count,
                            int* sel_idx, float* sel_q) {
  int tid = threadIdx.x;
  // Every slot starts valid, so a NaN query (whose rank is ill-defined)
  // cannot leave a slot holding an out-of-range dim.
  for (int s = tid; s < count; s += blockDim.x) {
    sel_idx[s] = 0;
    sel_q[s] = Elem<DT>::load(q_row);
  }
  __syncthreads();
  for (int d = tid; d < head_dim; d += blockDim.x) {
    float a = fabsf(Elem<DT>::load(q_row + d));
    int rank = 0;
    for (int e = 0; e < head_dim; ++e) {
      float b = fabsf(Elem<DT>::load(q_row + e));
      rank += (b > a) || (b == a && e < d);
    }
    if (rank < count) {
      sel_idx[rank] = d;
      sel_q[rank] = Elem<DT>::load(q_row + d);
    }
  }
}

// The same order for head_dim <= 128 dims whose query values sit in LDS
// (q_s), with one 64-bit key per dim: the bits of |q_d| (for non-negative
// floats the integer order is the numeric order) above 255 - d, so that
// "larger |q|, or equal |q| and lower dim" is one unsigned compare and
// rank(d) is the number of keys above d's.  The 128 keys (dims past head_dim
// pad with 0, under every real key) are read back by broadcast 16-byte LDS
// loads.  key_s: 128 LDS words of 8 bytes.  Every thread calls it; it begins
// after a barrier that published q_s and ends with one.
__device__ inline void rank_dims128(const float* q_s, uint64_t* key_s, int head_dim, int count, int* sel_idx,
                                    float* sel_q) {
  const int tid = threadIdx.x;
  for (int s = tid; s < count; s += blockDim.x) {   // valid even for a NaN query
    sel_idx[s] = 0;
    sel_q[s] = q_s[0];
  }
  for (int d = tid; d < 128; d += blockDim.x)
    key_s[d] = d < head_dim ? (static_cast<uint64_t>(__float_as_uint(q_s[d]) & 0x7FFFFFFFu) << 8) |
                                  static_cast<uint64_t>(255 - d)
                            : 0ull;
  __syncthreads();
  for (int d = tid; d < head_dim; d += blockDim.x) {
    const uint64_t own = key_s[d];
    int rank = 0;
#pragma unroll 8   // (eight 16-byte reads in flight; a full unroll holds all 128 keys in registers)
    for (int e = 0; e < 128; e += 2) {
      const ulonglong2 c = *reinterpret_cast<const ulonglong2*>(key_s + e);
      rank += (c.x > own ? 1 : 0) + (c.y > own ? 1 : 0);
    }
    if (rank < count) {
      sel_idx[rank] = d;
      sel_q[rank] = q_s[d];
    }
  }
  __syncthreads();
}

// Eight consecutive elements at p as fp32 (p 16-byte aligned).
template <int DT>
__device__ __forceinline__ void load8(const typename Elem<DT>::T* p, float (&v)[8]) {
  if constexpr (DT == QKV_DTYPE_FP32) {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint4 c = *reinterpret_cast<const uint4*>(p + 4);
    v[0] = __uint_as_float(a.x); v[1] = __uint_as_float(a.y);
    v[2] = __uint_as_float(a.z); v[3] = __uint_as_float(a.w);
    v[4] = __uint_as_float(c.x); v[5] = __uint_as_float(c.y);
    v[6] = __uint_as_float(c.z); v[7] = __uint_as_float(c.w);
  } else {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t lo = static_cast<uint16_t>(w[i] & 0xFFFFu), hi = static_cast<uint16_t>(w[i] >> 16);
      v[2 * i] = Elem<DT>::load(&lo);
      v[2 * i + 1] = Elem<DT>::load(&hi);
    }
  }
}

// Whether row `row` takes new candidates in a lagged reuse step (QKV_REFRESH_*
// over the per-row flags, EV:4024-4115).  Every thread of the workgroup
// calls it at the same point (the step-wide kinds synchronize); cnt_s holds
// one int per wave.
__device__ __forceinline__ bool lag_refreshes(const uint8_t* flags, int refresh, int rows, int row, int* cnt_s) {
  if (refresh == QKV_REFRESH_ALL) return true;
  if (refresh == QKV_REFRESH_NONE) return false;
  if (refresh == QKV_REFRESH_PER_ROW) return flags[row] != 0;
  int c = 0;
  for (int i = threadIdx.x; i < rows; i += blockDim.x) c += flags[i] ? 1 : 0;
  c = wave_sum_i(c);
  if ((threadIdx.x & 63) == 0) cnt_s[threadIdx.x >> 6] = c;
  __syncthreads();
  int t = 0;
  for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) t += cnt_s[w];
  return refresh == QKV_REFRESH_ANY ? t > 0 : 2 * t > rows;
}

template <template <int> class F, typename... A>
int dispatch_dtype(int dtype, A&&... args) {
  switch (dtype) {
    case QKV_DTYPE_BF16: return F<QKV_DTYPE_BF16>::run(args...);
    case QKV_DTYPE_FP16: return F<QKV_DTYPE_FP16>::run(args...);
    case QKV_DTYPE_FP32: return F<QKV_DTYPE_FP32>::run(args...);
    default: return fail(QKV_ERR_INVALID, "unsupported dtype %d", dtype);
  }
}

}  // namespace
}  // namespace qkv
