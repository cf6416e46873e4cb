// Peak microbenchmarks used to report measured ceilings next to the vendor
// figures (bf16 dense MFMA, HBM copy bandwidth).  Not part of the SCOPE path
// itself; no reference counterpart.
#include "attn_common.h"

namespace scope {

// Four independent v_mfma_f32_32x32x16_bf16 accumulator chains per wavefront,
// iters steps each; the accumulators are written out so nothing is removed.
__global__ __launch_bounds__(256) void probe_mfma_kernel(float* __restrict__ out, int iters) {
  const int lane = threadIdx.x & 63;
  const uint32_t w = 0x3f803f80u ^ static_cast<uint32_t>(lane);  // bf16 pairs near 1.0
  const uint4 av = make_uint4(w, w + 1, w + 2, w + 3), bv = make_uint4(w + 4, w + 5, w + 6, w + 7);
  f32x16_t c0 = zero16(), c1 = zero16(), c2 = zero16(), c3 = zero16();
  for (int i = 0; i < iters; ++i) {
    c0 = mfma32(av, bv, c0);
    c1 = mfma32(bv, av, c1);
    c2 = mfma32(av, av, c2);
    c3 = mfma32(bv, bv, c3);
  }
  float s = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) s += c0[r] + c1[r] + c2[r] + c3[r];
  out[static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x] = s;
}

// The same four chains on data: each lane's A and B operands cycle through 8
// register sets each, loaded from `ops` (16 uint4 per thread), so the MFMA
// inputs toggle as attention operands do.  With random bf16 data the chip
// draws more power per MFMA than with the constant operands above, and its
// power limit lowers the clock.  iters is a multiple of 8.
__global__ __launch_bounds__(256) void probe_mfma_data_kernel(const uint4* __restrict__ ops, float* __restrict__ out,
                                                              int iters) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  uint4 a[8], b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = ops[t * 16 + i];
    b[i] = ops[t * 16 + 8 + i];
  }
  f32x16_t c0 = zero16(), c1 = zero16(), c2 = zero16(), c3 = zero16();
  for (int i = 0; i < iters; i += 8) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const uint4 bb = b[(s + 3) & 7];
      c0 = mfma32(a[s], bb, c0);
      c1 = mfma32(a[(s + 1) & 7], bb, c1);
      c2 = mfma32(a[(s + 2) & 7], bb, c2);
      c3 = mfma32(a[(s + 5) & 7], bb, c3);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) s += c0[r] + c1[r] + c2[r] + c3[r];
  out[t] = s;
}

// Streaming copy, 16 bytes per lane per step, grid-stride.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void probe_copy_kernel(const u32x4_t* __restrict__ src, u32x4_t* __restrict__ dst,
                                                         int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

}  // namespace scope

using namespace scope;

extern "C" int64_t scope_probe_mfma_flops(int blocks, int iters) {
  // 4 MFMAs of 32·32·16·2 FLOP per step per wavefront, 4 wavefronts per block
  return static_cast<int64_t>(blocks) * 4 * iters * 4 * 32768;
}

extern "C" int scope_probe_mfma(float* out, int blocks, int iters, void* stream) {
  SCOPE_REQUIRE(out && blocks > 0 && iters > 0, "scope_probe_mfma: bad arguments");
  hipLaunchKernelGGL(probe_mfma_kernel, dim3(blocks), dim3(256), 0, as_stream(stream), out, iters);
  return check_launch("probe_mfma_kernel");
}

extern "C" int scope_probe_mfma_data(const void* operands, float* out, int blocks, int iters, void* stream) {
  SCOPE_REQUIRE(operands && out && blocks > 0 && iters > 0 && iters % 8 == 0,
                "scope_probe_mfma_data: bad arguments (iters must be a positive multiple of 8)");
  SCOPE_REQUIRE((reinterpret_cast<uintptr_t>(operands) & 15) == 0, "scope_probe_mfma_data: 16-byte aligned operands");
  hipLaunchKernelGGL(probe_mfma_data_kernel, dim3(blocks), dim3(256), 0, as_stream(stream),
                     static_cast<const uint4*>(operands), out, iters);
  return check_launch("probe_mfma_data_kernel");
}

extern "C" int scope_probe_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  SCOPE_REQUIRE(src && dst && bytes > 0 && bytes % 16 == 0, "scope_probe_copy: bytes must be a positive multiple of 16");
  SCOPE_REQUIRE(((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0,
                "scope_probe_copy: 16-byte aligned buffers");
  const int64_t n = bytes / 16;
  hipLaunchKernelGGL(probe_copy_kernel, dim3(256 * 8), dim3(256), 0, as_stream(stream),
                     static_cast<const u32x4_t*>(src), static_cast<u32x4_t*>(dst), n);
  return check_launch("probe_copy_kernel");
}
