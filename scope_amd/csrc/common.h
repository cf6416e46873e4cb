// Shared device/host helpers of the SCOPE gfx950 library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/scope_amd.h"

namespace scope {

// ---- error reporting (defined in api.hip) ---------------------------------
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int check_launch(const char* what);

#define SCOPE_REQUIRE(cond, ...)                        \
  do {                                                  \
    if (!(cond)) return ::scope::set_error(SCOPE_EINVAL, __VA_ARGS__); \
  } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

constexpr int kWave = 64;

// ---- bf16 ------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
// round-to-nearest-even fp32 -> bf16 bits (NaN kept quiet)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

// ---- wave helpers ------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return __lane_id(); }

template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int mask) {
  return __shfl_xor(v, mask, kWave);
}

__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

__device__ __forceinline__ float wave_max_f32(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
  return v;
}

__host__ __device__ __forceinline__ int ceil_div(int64_t a, int64_t b) {
  return static_cast<int>((a + b - 1) / b);
}
__host__ __device__ __forceinline__ int next_pow2(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

// lowbias32 integer hash and the counter-based uniform of the block-scoring
// Gumbel draw: u = (hash(seed, h, qb, kb) >> 8) * 2^-24 in [0, 1).
__host__ __device__ __forceinline__ uint32_t mix32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}
__host__ __device__ __forceinline__ float counter_uniform(uint64_t seed, uint32_t h, uint32_t qb,
                                                          uint32_t kb) {
  uint32_t x = mix32(static_cast<uint32_t>(seed) ^ mix32(static_cast<uint32_t>(seed >> 32)));
  x = mix32(x ^ (h + 0x9e3779b9u));
  x = mix32(x ^ (qb + 0x3c6ef372u));
  x = mix32(x ^ (kb + 0xdaa66d2bu));
  return static_cast<float>(x >> 8) * (1.0f / 16777216.0f);
}

}  // namespace scope
