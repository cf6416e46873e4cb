// Error state, version and the spectral tables of the SCOPE gfx950 library.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <string>

#include "common.h"

namespace scope {

static thread_local std::string g_last_error;

int set_error(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SCOPE_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  return SCOPE_OK;
}

// Block mode: row r of [NB][16] fp32 holds cos(ω_k r) for k < 8, then sin(ω_k r).
// Token mode: row j of [T][32] bf16 holds cos(ω_k j) and sin(ω_k j) as bf16
// hi parts, then the bf16 lo parts (x - hi).
// Phases are reduced in double precision so that large offsets keep full
// fp32 accuracy; unused bands (k >= K) are zero.
__global__ void spectral_table_kernel(const float* __restrict__ omegas, int K, int64_t rows,
                                      int bf16_out, void* __restrict__ table) {
  int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  float c[8], s[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    if (k < K) {
      double ph = static_cast<double>(omegas[k]) * static_cast<double>(r);
      ph = fmod(ph, 6.283185307179586476925286766559);
      c[k] = static_cast<float>(cos(ph));
      s[k] = static_cast<float>(sin(ph));
    } else {
      c[k] = 0.f;
      s[k] = 0.f;
    }
  }
  if (bf16_out) {
    // hi = bf16(x), lo = bf16(x - hi): [cos hi, sin hi, cos lo, sin lo]
    uint32_t* o = reinterpret_cast<uint32_t*>(table) + r * 16;
    float cl[8], sl[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      cl[k] = c[k] - bf16_to_f32(f32_to_bf16(c[k]));
      sl[k] = s[k] - bf16_to_f32(f32_to_bf16(s[k]));
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      o[k] = pack_bf16x2(c[2 * k], c[2 * k + 1]);
      o[4 + k] = pack_bf16x2(s[2 * k], s[2 * k + 1]);
      o[8 + k] = pack_bf16x2(cl[2 * k], cl[2 * k + 1]);
      o[12 + k] = pack_bf16x2(sl[2 * k], sl[2 * k + 1]);
    }
  } else {
    float* o = reinterpret_cast<float*>(table) + r * 16;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      o[k] = c[k];
      o[8 + k] = s[k];
    }
  }
}

}  // namespace scope

using namespace scope;

extern "C" {

int scope_abi_version(void) { return SCOPE_ABI_VERSION; }

const char* scope_last_error(void) { return g_last_error.c_str(); }

int64_t scope_spectral_table_bytes(int bias_mode, int64_t T, int bs) {
  if (bias_mode == SCOPE_BIAS_BLOCK) return (T / bs) * 16 * 4;
  if (bias_mode == SCOPE_BIAS_TOKEN) return T * 32 * 2;
  return 0;
}

int scope_spectral_table(int bias_mode, const float* omegas, int K, int64_t T, int bs, void* table,
                         void* stream) {
  SCOPE_REQUIRE(bias_mode == SCOPE_BIAS_BLOCK || bias_mode == SCOPE_BIAS_TOKEN,
                "scope_spectral_table: bias_mode must be block (1) or token (2), got %d", bias_mode);
  SCOPE_REQUIRE(K >= 1 && K <= 8, "scope_spectral_table: K must be in [1, 8], got %d", K);
  SCOPE_REQUIRE(bs > 0 && T > 0 && T % bs == 0, "scope_spectral_table: T=%lld must be a positive multiple of bs=%d",
                (long long)T, bs);
  SCOPE_REQUIRE(omegas && table, "scope_spectral_table: null pointer");
  int64_t rows = bias_mode == SCOPE_BIAS_BLOCK ? T / bs : T;
  int threads = 256;
  int blocks = ceil_div(rows, threads);
  hipLaunchKernelGGL(spectral_table_kernel, dim3(blocks), dim3(threads), 0, as_stream(stream), omegas, K,
                     rows, bias_mode == SCOPE_BIAS_TOKEN ? 1 : 0, table);
  return check_launch("spectral_table_kernel");
}

}  // extern "C"
