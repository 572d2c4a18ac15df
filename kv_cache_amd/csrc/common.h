// Shared device helpers and C-ABI error plumbing for libqkv (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <type_traits>

#include "../../include/qkv.h"

#define QKV_EXPORT extern "C" __attribute__((visibility("default")))

namespace qkv {

// Records a printf-style message as this thread's last error and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Checks hipGetLastError() after a launch; returns QKV_OK or QKV_ERR_LAUNCH.
int check_launch(const char* what);

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Resolves the dtype of a 16-bit operand (query, K, V): sets *f16 (false for
// bf16, true for fp16) and returns QKV_OK, or fails for fp32 and unknown codes.
inline int half_dtype(int dtype, const char* what, bool* f16) {
  if (dtype == QKV_DTYPE_BF16 || dtype == QKV_DTYPE_FP16) {
    *f16 = dtype == QKV_DTYPE_FP16;
    return QKV_OK;
  }
  return fail(dtype == QKV_DTYPE_FP32 ? QKV_ERR_UNSUPPORTED : QKV_ERR_INVALID,
              "%s: dtype %d is not bf16 (%d) or fp16 (%d)", what, dtype, QKV_DTYPE_BF16, QKV_DTYPE_FP16);
}

// Calls f(std::integral_constant<bool, f16>{}) and returns its result: one
// template instantiation per 16-bit dtype.
template <typename F>
int with_half(bool f16, F&& f) {
  return f16 ? f(std::integral_constant<bool, true>{}) : f(std::integral_constant<bool, false>{});
}

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

__device__ __forceinline__ float f16bits_to_f32(uint32_t bits16) {
  _Float16 h = __builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16));
  return static_cast<float>(h);
}

// The 16-bit floats of q, K and V: bf16 (F16 = false) or fp16 (F16 = true),
// widened to fp32 exactly -- one value, or the low / high half of a word.
template <bool F16>
__device__ __forceinline__ float half_to_f32(uint32_t bits16) {
  if constexpr (F16) return f16bits_to_f32(bits16 & 0xFFFFu);
  else return bf16_to_f32(bits16 & 0xFFFFu);
}
template <bool F16>
__device__ __forceinline__ float half_lo(uint32_t w) {
  if constexpr (F16) return f16bits_to_f32(w & 0xFFFFu);
  else return bf16lo(w);
}
template <bool F16>
__device__ __forceinline__ float half_hi(uint32_t w) {
  if constexpr (F16) return f16bits_to_f32(w >> 16);
  else return bf16hi(w);
}

// fp32 -> fp16 round-to-nearest-even (v_cvt_f16_f32 in the default mode), with
// +inf saturated to 65504.  The argument is a non-negative magnitude.
__device__ __forceinline__ uint32_t f32_to_f16bits_sat(float x) {
  _Float16 h = static_cast<_Float16>(x);
  uint32_t bits = __builtin_bit_cast(uint16_t, h);
  return bits == 0x7C00u ? 0x7BFFu : bits;
}

// Symmetric int4 code of x for an fp16-representable scale s (s > 0):
// clamp(rint_even(x / s), -8, 7).  The division is the IEEE-correct one
// (hipcc's default for fp32 '/').
__device__ __forceinline__ int int4_code(float x, float s) {
  float r = __builtin_rintf(x / s);
  r = fminf(fmaxf(r, -8.0f), 7.0f);
  return static_cast<int>(r);
}

// Order-preserving map of an fp32 key onto uint32 (larger float -> larger
// integer), with -0 folded onto +0.  NaN inputs are outside the contract.
__device__ __forceinline__ uint32_t f32_sortable(float f) {
  uint32_t u = __float_as_uint(f);
  if (u == 0x80000000u) u = 0;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float sortable_f32(uint32_t u) {
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u);
}

// ds_swizzle in bit-mask mode: lane i reads lane (i ^ m) within groups of 32.
template <int M>
__device__ __forceinline__ float swz_xor(float v) {
  static_assert(M > 0 && M < 32, "xor mask must stay inside 32 lanes");
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x1F | (M << 10)));
}
template <int M>
__device__ __forceinline__ int swz_xor_i(int v) {
  static_assert(M > 0 && M < 32, "xor mask must stay inside 32 lanes");
  return __builtin_amdgcn_ds_swizzle(v, 0x1F | (M << 10));
}

// Lane i reads lane i ^ m for any m < 64 (ds_bpermute).
__device__ __forceinline__ float shfl_xor(float v, int m) {
  int lane = __lane_id();
  return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ m) << 2, __float_as_int(v)));
}
__device__ __forceinline__ int shfl_xor_i(int v, int m) {
  int lane = __lane_id();
  return __builtin_amdgcn_ds_bpermute((lane ^ m) << 2, v);
}

__device__ __forceinline__ float wave_max(float v) {
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, shfl_xor(v, m));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  for (int m = 32; m >= 1; m >>= 1) v += shfl_xor(v, m);
  return v;
}
__device__ __forceinline__ int wave_sum_i(int v) {
  for (int m = 32; m >= 1; m >>= 1) v += shfl_xor_i(v, m);
  return v;
}

// DPP move: lane i receives `v` of the lane CTRL selects (row_shl:n = lane
// i + n of the same row of 16, quad_perm, row mirrors, row_bcast ...).
template <int CTRL, int ROW_MASK = 0xF, int BANK_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t old, uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(static_cast<int>(old), static_cast<int>(v), CTRL,
                                                           ROW_MASK, BANK_MASK, false));
}

// Max of a non-negative float over the 64 lanes, wave-uniform: row
// reductions (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror),
// then row_bcast:15 and row_bcast:31 leave the wave's maximum in lane 63.
// Non-negative floats order like their bit patterns, so the max is exact.
__device__ __forceinline__ float wave_max_nonneg(float x) {
  uint32_t v = __float_as_uint(x);
  v = max(v, dpp_mov<0xB1>(v, v));
  v = max(v, dpp_mov<0x4E>(v, v));
  v = max(v, dpp_mov<0x141>(v, v));
  v = max(v, dpp_mov<0x140>(v, v));
  v = max(v, dpp_mov<0x142, 0xA>(v, v));
  v = max(v, dpp_mov<0x143, 0xC>(v, v));
  return __uint_as_float(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), 63)));
}

// Pairs of lanes 16 and 32 apart, exchanged on the VALU.  v_permlane16_swap
// swaps the odd rows of its first operand with the even rows of its second;
// with both operands x, the two results hold x of the even and of the odd
// row of each pair of rows, in every lane of the pair.  v_permlane32_swap
// does the same for the two halves of the wave.  Both orders of the two
// values are the same in every lane, so sums come out identical.
__device__ __forceinline__ float sum_x16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_x32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_x16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_x32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Maximum of two lane-swap results that are never NaN, as one v_med3_f32
// against +inf: fmaxf would first quiet each operand (the compiler cannot
// tell that a swapped value is no signalling NaN), two more instructions.
// The +inf comes from a scalar move the compiler cannot see through;
// against a visible constant it rewrites the median back into fmaxf.
__device__ __forceinline__ float max_swapped(uint32_t a, uint32_t b) {
  float pinf;
  asm("s_mov_b32 %0, 0x7f800000" : "=s"(pinf));
  return __builtin_amdgcn_fmed3f(__uint_as_float(a), __uint_as_float(b), pinf);
}
// Four maxima over the wave's 4 rows (lanes 16r..16r+15) at once: row r of
// the result holds, lane by lane, the maximum of x_r over the 4 rows.
// v_permlane16_swap(x0, x1) leaves (x0.0, x1.0, x0.2, x1.2) and
// (x0.1, x1.1, x0.3, x1.3), whose maximum is (x0.01, x1.01, x0.23, x1.23);
// v_permlane32_swap of that and the same for x2, x3 pairs the halves.
__device__ __forceinline__ float max_rows4(float x0, float x1, float x2, float x3) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x0), __float_as_uint(x1), false, false);
  const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x2), __float_as_uint(x3), false, false);
  const float ma = max_swapped(a[0], a[1]), mb = max_swapped(b[0], b[1]);
  const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(ma), __float_as_uint(mb), false, false);
  return max_swapped(c[0], c[1]);
}
// Two maxima over the 4 rows: rows 0 and 2 of the result hold x0's, rows 1
// and 3 x1's.
__device__ __forceinline__ float max_rows2(float x0, float x1) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x0), __float_as_uint(x1), false, false);
  const float ma = max_swapped(a[0], a[1]);
  const auto c = __builtin_amdgcn_permlane32_swap(__float_as_uint(ma), __float_as_uint(ma), false, false);
  return max_swapped(c[0], c[1]);
}

// Inclusive prefix sum across the 64 lanes of a wave.
__device__ __forceinline__ int wave_incl_scan(int v) {
  int lane = __lane_id();
  for (int d = 1; d < 64; d <<= 1) {
    int o = __builtin_amdgcn_ds_bpermute(((lane - d) & 63) << 2, v);
    if (lane >= d) v += o;
  }
  return v;
}

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// DPP move within rows of 16 lanes (quad_perm, row_shl/shr, row mirrors ...),
// every row and bank enabled.
template <int DPP>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), DPP, 0xF, 0xF, false));
}

// Device-coherent stores and loads (relaxed agent-scope atomics: sc1, written
// through / read past the XCD's L2), for data one workgroup hands another
// inside a launch (the attention's split partials).
__device__ __forceinline__ void st_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float* p) {
  return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_coherent(int32_t* p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t ld_coherent(const int32_t* p) {
  return __hip_atomic_load(const_cast<int32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Zero that the compiler cannot see through, available only once `dep` is:
// adding it to an address keeps a load after the code that produced `dep`.
__device__ __forceinline__ int zero_after(float dep) {
  int z = 0;
  asm volatile("" : "+v"(z) : "v"(dep));
  return z;
}
// Marks x as final at this point: the volatile asm statements keep their
// order, so whatever comes after a later one cannot move above the code
// that computed x.
__device__ __forceinline__ void pin(float& x) { asm volatile("" : "+v"(x)); }

}  // namespace qkv
