// Transposed block lists for the dK/dV pass: for every (head, kv block) the
// q-blocks that list it, ascending.  Compact CSR replacement of
// torch:nn/attention/flex_attention.py:399-441 (_transpose_ordered), which
// builds a dense [H, NB, NB+1] matrix and argsorts it.
//
//   count  : q_off[h][kb+1] += 1 per listed (h, qb, kb)      (integer atomics)
//   scan   : exclusive prefix sum per head (one workgroup per head)
//   fill   : q_list[h][q_off[h][kb] + cursor++] = qb          (integer atomics)
//   sort   : each bucket sorted ascending (bitonic in LDS)
// The atomics only fix the set of each bucket; the sort fixes its order, so
// the result is deterministic.
#include <limits.h>

#include "common.h"

namespace scope {

__global__ void fill_i32_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__global__ void tr_count_kernel(const int32_t* __restrict__ kv_num, const int32_t* __restrict__ kv_idx, int H,
                                int QB, int NB, int maxkv, int32_t* __restrict__ q_off) {
  int64_t row = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (row >= static_cast<int64_t>(H) * QB) return;
  const int h = static_cast<int>(row / QB);
  const int n = kv_num[row];
  for (int i = 0; i < n; ++i) {
    const int kb = kv_idx[row * maxkv + i];
    atomicAdd(&q_off[static_cast<int64_t>(h) * (NB + 1) + kb + 1], 1);
  }
}

__global__ __launch_bounds__(1024) void tr_scan_kernel(int NB, int32_t* __restrict__ q_off) {
  const int h = blockIdx.x;
  int32_t* row = q_off + static_cast<int64_t>(h) * (NB + 1);
  __shared__ int tsum[1024];
  __shared__ int carry_s;
  if (threadIdx.x == 0) carry_s = 0;
  __syncthreads();
  // inclusive scan of row[1..NB] in chunks of 1024; row[0] stays 0
  for (int base = 1; base <= NB; base += 1024) {
    const int i = base + threadIdx.x;
    int v = i <= NB ? row[i] : 0;
    tsum[threadIdx.x] = v;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {
      int add = threadIdx.x >= o ? tsum[threadIdx.x - o] : 0;
      __syncthreads();
      tsum[threadIdx.x] += add;
      __syncthreads();
    }
    const int carry = carry_s;
    if (i <= NB) row[i] = tsum[threadIdx.x] + carry;
    __syncthreads();
    if (threadIdx.x == 1023) carry_s = carry + tsum[1023];
    __syncthreads();
  }
  if (threadIdx.x == 0) row[0] = 0;
}

__global__ void tr_fill_kernel(const int32_t* __restrict__ kv_num, const int32_t* __restrict__ kv_idx, int H,
                               int QB, int NB, int maxkv, const int32_t* __restrict__ q_off,
                               int32_t* __restrict__ cursor, int32_t* __restrict__ q_list) {
  int64_t row = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (row >= static_cast<int64_t>(H) * QB) return;
  const int h = static_cast<int>(row / QB);
  const int qb = static_cast<int>(row % QB);
  const int n = kv_num[row];
  const int64_t list_stride = static_cast<int64_t>(QB) * maxkv;
  for (int i = 0; i < n; ++i) {
    const int kb = kv_idx[row * maxkv + i];
    const int pos = atomicAdd(&cursor[static_cast<int64_t>(h) * NB + kb], 1);
    q_list[h * list_stride + q_off[static_cast<int64_t>(h) * (NB + 1) + kb] + pos] = qb;
  }
}

// One workgroup of 256 threads per bucket: a list of up to 64 entries is sorted
// in registers by the first wavefront (bitonic over the lanes); a longer one
// (a global block listed by every q-block of a long document) by the whole
// workgroup, bitonic in LDS.
__global__ __launch_bounds__(256) void tr_sort_kernel(int NB, int QB, int maxkv, const int32_t* __restrict__ q_off,
                                                     int32_t* __restrict__ q_list, int cap) {
  extern __shared__ int s[];
  const int h = blockIdx.y;
  const int kb = blockIdx.x;
  const int64_t o0 = q_off[static_cast<int64_t>(h) * (NB + 1) + kb];
  const int n = q_off[static_cast<int64_t>(h) * (NB + 1) + kb + 1] - static_cast<int>(o0);
  if (n <= 1) return;
  int32_t* b = q_list + static_cast<int64_t>(h) * QB * maxkv + o0;
  const int lane = threadIdx.x;
  const int nt = blockDim.x;
  if (n <= kWave) {
    if (lane >= kWave) return;
    // register bitonic over 64 lanes
    int v = lane < n ? b[lane] : INT_MAX;
#pragma unroll
    for (int k = 2; k <= kWave; k <<= 1) {
#pragma unroll
      for (int j = k >> 1; j > 0; j >>= 1) {
        int o = __shfl_xor(v, j, kWave);
        bool lower = (lane & j) == 0;
        bool up = (lane & k) == 0;
        int mn = min(v, o), mx = max(v, o);
        v = (lower == up) ? mn : mx;
      }
    }
    if (lane < n) b[lane] = v;
    return;
  }
  const int N = next_pow2(n);
  if (N > cap) return;  // guarded on the host: cap >= next_pow2(QB)
  for (int i = lane; i < N; i += nt) s[i] = i < n ? b[i] : INT_MAX;
  __syncthreads();
  for (int k = 2; k <= N; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = lane; i < (N >> 1); i += nt) {
        int lo = 2 * j * (i / j) + (i % j);
        int hi = lo + j;
        bool up = (lo & k) == 0;
        int a = s[lo], c = s[hi];
        if ((a > c) == up) {
          s[lo] = c;
          s[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  for (int i = lane; i < n; i += nt) b[i] = s[i];
}

}  // namespace scope

using namespace scope;

extern "C" {

int64_t scope_transpose_workspace_bytes(int H, int NB) { return static_cast<int64_t>(H) * NB * 4; }

int scope_transpose_blocks(const int32_t* kv_num, const int32_t* kv_idx, int H, int QB, int NB, int maxkv,
                           int32_t* q_off, int32_t* q_list, void* workspace, void* stream) {
  SCOPE_REQUIRE(kv_num && kv_idx && q_off && q_list && workspace, "scope_transpose_blocks: null pointer");
  SCOPE_REQUIRE(H >= 1 && QB >= 1 && NB >= 1 && maxkv >= 1, "scope_transpose_blocks: bad sizes");
  const int cap = next_pow2(QB);
  SCOPE_REQUIRE(cap * 4 <= 64 * 1024, "scope_transpose_blocks: QB=%d exceeds the LDS sort capacity", QB);
  hipStream_t s = as_stream(stream);
  int32_t* cursor = static_cast<int32_t*>(workspace);
  const int64_t n_off = static_cast<int64_t>(H) * (NB + 1);
  const int64_t n_cur = static_cast<int64_t>(H) * NB;
  hipLaunchKernelGGL(fill_i32_kernel, dim3(ceil_div(n_off, 256)), dim3(256), 0, s, q_off, n_off, 0);
  hipLaunchKernelGGL(fill_i32_kernel, dim3(ceil_div(n_cur, 256)), dim3(256), 0, s, cursor, n_cur, 0);
  const int64_t rows = static_cast<int64_t>(H) * QB;
  hipLaunchKernelGGL(tr_count_kernel, dim3(ceil_div(rows, 256)), dim3(256), 0, s, kv_num, kv_idx, H, QB, NB, maxkv,
                     q_off);
  hipLaunchKernelGGL(tr_scan_kernel, dim3(H), dim3(1024), 0, s, NB, q_off);
  hipLaunchKernelGGL(tr_fill_kernel, dim3(ceil_div(rows, 256)), dim3(256), 0, s, kv_num, kv_idx, H, QB, NB, maxkv,
                     q_off, cursor, q_list);
  hipLaunchKernelGGL(tr_sort_kernel, dim3(NB, H), dim3(256), cap * sizeof(int), s, NB, QB, maxkv, q_off, q_list, cap);
  return check_launch("transpose kernels");
}

}  // extern "C"
