// Streaming HBM read probe: the read ceiling a single launch of a given size
// reaches on this GPU, with the access shape of the decode scoring kernel
// (int4.hip): each wave reads whole 4 KiB tiles, one 16-byte non-temporal
// load per lane per 1 KiB, the next tile's loads in flight while the
// current one is consumed.  Not part of the reference; the benchmark reports
// it next to the scoring kernel's rate.
#include "common.h"

#ifndef QKV_PROBE_TARGET_WGS
#define QKV_PROBE_TARGET_WGS 4096
#endif

namespace qkv {
namespace {

constexpr int kProbeThreads = 256;
constexpr int64_t kTile = 4096;                  // bytes per wave stage
constexpr int64_t kWgStage = 4 * kTile;          // bytes per workgroup stage

__device__ __forceinline__ uint4 ld_stream(const uint4* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Workgroup w reads bytes [w * chunk, min(bytes, (w + 1) * chunk)); its wave
// v reads the tiles v, v + 4, v + 8, ... of that range.  Every lane folds
// what it read into one word; lane 0 of each wave stores the wave's fold.
__global__ __launch_bounds__(kProbeThreads) void read_probe_kernel(const uint4* __restrict__ src, int64_t bytes,
                                                                  int64_t chunk, uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t lo = static_cast<int64_t>(blockIdx.x) * chunk;
  const int64_t hi = min(bytes, lo + chunk);
  uint32_t acc = 0;
  int64_t t = lo + wave * kTile;
  if (t < hi) {
    uint4 cur[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) cur[i] = ld_stream(src + t / 16 + i * 64 + lane);
    for (int64_t n = t + kWgStage; n < hi; n += kWgStage) {
      uint4 nxt[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) nxt[i] = ld_stream(src + n / 16 + i * 64 + lane);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc ^= cur[i].x ^ cur[i].y ^ cur[i].z ^ cur[i].w;
#pragma unroll
      for (int i = 0; i < 4; ++i) cur[i] = nxt[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) acc ^= cur[i].x ^ cur[i].y ^ cur[i].z ^ cur[i].w;
  }
  for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off);
  if (lane == 0) sink[static_cast<int64_t>(blockIdx.x) * 4 + wave] = acc;
}

}  // namespace
}  // namespace qkv

using namespace qkv;

QKV_EXPORT int64_t qkv_hbm_read_probe_sink_words(int64_t bytes) {
  if (bytes <= 0 || bytes % kWgStage) return -1;
  int64_t chunk = std::max<int64_t>(kWgStage, cdiv(cdiv(bytes, QKV_PROBE_TARGET_WGS), kWgStage) * kWgStage);
  return 4 * cdiv(bytes, chunk);
}

QKV_EXPORT int qkv_hbm_read_probe(const void* src, int64_t bytes, uint32_t* sink, int64_t sink_words, void* stream) {
  const char* what = "qkv_hbm_read_probe";
  if (!src || !sink) return fail(QKV_ERR_INVALID, "%s: null pointer", what);
  if (bytes <= 0 || bytes % kWgStage || !aligned(src, 16))
    return fail(QKV_ERR_INVALID, "%s: need a 16-byte aligned source of a positive multiple of %lld bytes", what,
                (long long)kWgStage);
  const int64_t chunk = std::max<int64_t>(kWgStage, cdiv(cdiv(bytes, QKV_PROBE_TARGET_WGS), kWgStage) * kWgStage);
  const int64_t wgs = cdiv(bytes, chunk);
  if (sink_words < 4 * wgs) return fail(QKV_ERR_INVALID, "%s: the sink needs %lld words", what, (long long)(4 * wgs));
  if (wgs > 0x7FFFFFFF) return fail(QKV_ERR_INVALID, "%s: source too large", what);
  read_probe_kernel<<<static_cast<unsigned>(wgs), kProbeThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint4*>(src), bytes, chunk, sink);
  return check_launch(what);
}
