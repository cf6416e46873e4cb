// Transposed block lists for the dK/dV pass: for every (head, kv block) the
// q-blocks that list it, ascending.  Compact CSR replacement of
// torch:nn/attention/flex_attention.py:399-441 (_transpose_ordered), which
// builds a dense [H, NB, NB+1] matrix and argsorts it.
//
//   count  : q_off[h][kb+1] += 1 per listed (h, qb, kb)      (integer atomics, a thread per list slot)
//   scan   : exclusive prefix sum per head (one workgroup per head); the
//            head's list entries past its total set to -1
//   fill   : q_list[h][q_off[h][kb] + cursor++] = qb          (integer atomics)
//   sort   : each bucket sorted ascending (bitonic over a wavefront's lanes,
//            or a counting sort in LDS for a bucket longer than 64)
// The atomics only fix the set of each bucket; the sort fixes its order, so
// the result is deterministic.
#include <limits.h>

#include <mutex>

#include "common.h"

// Scratch of scope_transpose_blocks_noalloc: the per-(head, key block) fill
// cursors, in device memory the library owns, so that entry point allocates
// nothing.  Each device holds its own copy until the process ends; host code
// uses the device address hipGetSymbolAddress reports for the current device,
// never this name.
static __device__ __align__(256) int32_t scratch[SCOPE_NOALLOC_MAX_HNB];

namespace scope {

__global__ void fill_i32_kernel(int32_t* __restrict__ p, int64_t n, int32_t v) {
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// count and fill take a thread per list slot, in the order (h, i, qb): the
// lanes of a wavefront hold position i of 64 consecutive rows.  A key block
// listed at the same position by many rows (a document's global block, first
// in every row's ascending list) then falls on whole wavefronts, which add
// to its counter with one atomic: the lanes whose bucket equals the first
// active lane's are counted by a ballot.
struct SlotEntry {
  int64_t bucket;  // h·NB + kb, or -1 for an empty or out-of-range slot
  int qb;
};

__device__ __forceinline__ SlotEntry slot_entry(const int32_t* __restrict__ kv_num,
                                                const int32_t* __restrict__ kv_idx, int QB, int NB, int maxkv,
                                                int64_t e) {
  const int64_t per_head = static_cast<int64_t>(maxkv) * QB;
  const int h = static_cast<int>(e / per_head);
  const int64_t r = e % per_head;
  const int i = static_cast<int>(r / QB);
  const int qb = static_cast<int>(r % QB);
  const int64_t row = static_cast<int64_t>(h) * QB + qb;
  SlotEntry s{-1, qb};
  if (i >= kv_num[row]) return s;
  const int kb = kv_idx[row * maxkv + i];
  if (kb < 0 || kb >= NB) return s;  // an entry outside the key blocks is no block (scope_check_lists reports it)
  s.bucket = static_cast<int64_t>(h) * NB + kb;
  return s;
}

// The lanes of the calling (active) lanes whose bucket equals the first
// active lane's, and whether this lane is one of them.
__device__ __forceinline__ uint64_t same_bucket_lanes(int64_t bucket, bool* mine) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(bucket));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(bucket) >> 32));
  const int64_t first = static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
  *mine = bucket == first;
  return __ballot(*mine);
}

__global__ void tr_count_kernel(const int32_t* __restrict__ kv_num, const int32_t* __restrict__ kv_idx, int H,
                                int QB, int NB, int maxkv, int32_t* __restrict__ q_off) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= static_cast<int64_t>(H) * QB * maxkv) return;
  const SlotEntry s = slot_entry(kv_num, kv_idx, QB, NB, maxkv, e);
  if (s.bucket < 0) return;
  // q_off[h][kb + 1] sits at bucket + h + 1
  const int64_t at = s.bucket + s.bucket / NB + 1;
  bool mine = false;
  const uint64_t grp = same_bucket_lanes(s.bucket, &mine);
  if (mine) {
    if (lane_id() == __ffsll(static_cast<unsigned long long>(grp)) - 1) atomicAdd(&q_off[at], __popcll(grp));
  } else {
    atomicAdd(&q_off[at], 1);
  }
}

// also sets the head's list entries past its total to -1 (the fill kernel
// writes only below it) and clears the head's fill cursors (the count kernel
// before it does not read them, the fill kernel after it does)
__global__ __launch_bounds__(1024) void tr_scan_kernel(int NB, int32_t* __restrict__ q_off, int64_t list_len,
                                                       int32_t* __restrict__ q_list, int32_t* __restrict__ cursor) {
  const int h = blockIdx.x;
  for (int i = threadIdx.x; i < NB; i += 1024) cursor[static_cast<int64_t>(h) * NB + i] = 0;
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
  const int64_t total = carry_s;  // the head's entry count (carry after the last chunk)
  int32_t* lst = q_list + static_cast<int64_t>(h) * list_len;
  for (int64_t i = total + threadIdx.x; i < list_len; i += 1024) lst[i] = -1;
}

__global__ void tr_fill_kernel(const int32_t* __restrict__ kv_num, const int32_t* __restrict__ kv_idx, int H,
                               int QB, int NB, int maxkv, const int32_t* __restrict__ q_off,
                               int32_t* __restrict__ cursor, int32_t* __restrict__ q_list) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= static_cast<int64_t>(H) * QB * maxkv) return;
  const SlotEntry s = slot_entry(kv_num, kv_idx, QB, NB, maxkv, e);
  if (s.bucket < 0) return;  // skipped by the count kernel too
  const int h = static_cast<int>(s.bucket / NB);
  const int kb = static_cast<int>(s.bucket % NB);
  bool mine = false;
  const uint64_t grp = same_bucket_lanes(s.bucket, &mine);
  int pos;
  if (mine) {
    const int leader = __ffsll(static_cast<unsigned long long>(grp)) - 1;
    int base = 0;
    if (lane_id() == leader) base = atomicAdd(&cursor[s.bucket], __popcll(grp));
    base = __shfl(base, leader, kWave);
    pos = base + __popcll(grp & ((1ull << lane_id()) - 1));
  } else {
    pos = atomicAdd(&cursor[s.bucket], 1);
  }
  q_list[static_cast<int64_t>(h) * QB * maxkv + q_off[static_cast<int64_t>(h) * (NB + 1) + kb] + pos] = s.qb;
}

// Four buckets per workgroup of 256 threads.  A bucket of up to 64 entries
// is sorted in registers by its own wavefront (bitonic over the lanes).  A
// longer one (a global block listed by every q-block of a long document) is
// sorted by the whole workgroup by counting: its entries are q-blocks in
// [0, QB), so per-value counts in LDS, their exclusive prefix sum and a
// write of each value count times give the ascending list, repeats kept.
constexpr int kSortBuckets = 4;

__global__ __launch_bounds__(256) void tr_sort_kernel(int NB, int QB, int maxkv, const int32_t* __restrict__ q_off,
                                                     int32_t* __restrict__ q_list) {
  extern __shared__ int cnt[];  // [QB]
  __shared__ int wtot[kSortBuckets];
  const int h = blockIdx.y;
  const int kb0 = blockIdx.x * kSortBuckets;
  const int32_t* off = q_off + static_cast<int64_t>(h) * (NB + 1);
  int32_t* lst = q_list + static_cast<int64_t>(h) * QB * maxkv;
  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid / kWave;
  {
    const int kb = kb0 + wave;
    const int o0 = kb < NB ? off[kb] : 0;
    const int n = kb < NB ? off[kb + 1] - o0 : 0;
    if (n > 1 && n <= kWave) {
      int32_t* b = lst + o0;
      int v = lane < n ? b[lane] : INT_MAX;
#pragma unroll
      for (int k = 2; k <= kWave; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
          const int o = __shfl_xor(v, j, kWave);
          const bool lower = (lane & j) == 0;
          const bool up = (lane & k) == 0;
          const int mn = min(v, o), mx = max(v, o);
          v = (lower == up) ? mn : mx;
        }
      }
      if (lane < n) b[lane] = v;
    }
  }
  // the long buckets, one after another (the bounds are the same for every
  // thread, so every barrier below is reached by the whole workgroup)
  const int per = (QB + 255) / 256;  // values per thread in the prefix sum
  for (int w = 0; w < kSortBuckets; ++w) {
    const int kb = kb0 + w;
    if (kb >= NB) break;
    const int o0 = off[kb];
    const int n = off[kb + 1] - o0;
    if (n <= kWave) continue;
    int32_t* b = lst + o0;
    for (int v = tid; v < QB; v += 256) cnt[v] = 0;
    __syncthreads();
    for (int i = tid; i < n; i += 256) {
      const int v = b[i];
      if (v >= 0 && v < QB) atomicAdd(&cnt[v], 1);  // the fill writes q-blocks only
    }
    __syncthreads();
    // exclusive prefix sum over the values: thread t takes [t·per, t·per + per)
    const int v0 = min(tid * per, QB), v1 = min(v0 + per, QB);
    int mine = 0;
    for (int v = v0; v < v1; ++v) mine += cnt[v];
    int incl = mine;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int t = __shfl_up(incl, o, kWave);
      if (lane >= o) incl += t;
    }
    if (lane == kWave - 1) wtot[wave] = incl;
    __syncthreads();
    int base = incl - mine;
    for (int ww = 0; ww < wave; ++ww) base += wtot[ww];
    for (int v = v0; v < v1; ++v) {
      const int c = cnt[v];
      for (int r = 0; r < c; ++r) b[base + r] = v;
      base += c;
    }
    __syncthreads();  // cnt and wtot are reused by the next long bucket
  }
}

// List validation: one wavefront per row (h, qb) of the compact lists, a
// bitmap of the row's key blocks in LDS (NB bits per wavefront) to find
// repeated entries.  res: [0] rows whose kv_num is outside [0, maxkv],
// [1] entries outside [0, NB), [2] entries after their q-block (causal
// lists), [3] repeated entries, [4] the first offending row h·QB + qb
// (INT_MAX when there is none).  res is set to {0, 0, 0, 0, INT_MAX} by
// chk_init_kernel first.
__global__ void chk_init_kernel(int32_t* __restrict__ res) {
  if (threadIdx.x < 4) res[threadIdx.x] = 0;
  if (threadIdx.x == 4) res[4] = INT_MAX;
}

__global__ __launch_bounds__(256) void chk_lists_kernel(const int32_t* __restrict__ kv_num,
                                                       const int32_t* __restrict__ kv_idx, int H, int QB, int NB,
                                                       int maxkv, int causal, int32_t* __restrict__ res) {
  extern __shared__ uint32_t bm_all[];
  const int words = (NB + 31) >> 5;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  if (row >= static_cast<int64_t>(H) * QB) return;  // uniform per wavefront; no barrier follows
  uint32_t* bm = bm_all + static_cast<int64_t>(wave) * words;
  for (int w = lane; w < words; w += kWave) bm[w] = 0u;
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wavefront's clears have landed
  __builtin_amdgcn_wave_barrier();
  const int qb = static_cast<int>(row % QB);
  const int n = kv_num[row];
  int bad[4] = {0, 0, 0, 0};
  if (n < 0 || n > maxkv) {
    bad[0] = lane == 0;
  } else {
    for (int e = lane; e < n; e += kWave) {
      const int kb = kv_idx[row * maxkv + e];
      if (kb < 0 || kb >= NB) {
        ++bad[1];
      } else if (causal && kb > qb) {
        ++bad[2];
      } else {
        const uint32_t bit = 1u << (kb & 31);
        if (atomicOr(&bm[kb >> 5], bit) & bit) ++bad[3];
      }
    }
  }
  int any = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = wave_sum_i32(bad[i]);
    if (t && lane == 0) atomicAdd(&res[i], t);
    any |= t;
  }
  if (any && lane == 0) atomicMin(&res[4], static_cast<int32_t>(row));
}

// Address of `scratch` on each device, looked up once per device with that
// device current.
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static int32_t* g_scratch_ptr[kMaxDevices] = {};

static int noalloc_scratch(void* stream, int32_t** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return set_error(SCOPE_ELAUNCH, "scope_transpose_blocks_noalloc: hipGetDevice: %s",
                                        hipGetErrorString(e));
  if (stream) {
    hipDevice_t sdev = -1;
    e = hipStreamGetDevice(as_stream(stream), &sdev);
    if (e != hipSuccess)
      return set_error(SCOPE_ELAUNCH, "scope_transpose_blocks_noalloc: hipStreamGetDevice: %s", hipGetErrorString(e));
    if (sdev != dev)
      return set_error(SCOPE_EINVAL, "scope_transpose_blocks_noalloc: the stream belongs to device %d, the current "
                       "device is %d", static_cast<int>(sdev), dev);
  }
  if (dev < 0 || dev >= kMaxDevices)
    return set_error(SCOPE_ERANGE, "scope_transpose_blocks_noalloc: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return set_error(SCOPE_ELAUNCH, "scope_transpose_blocks_noalloc: hipGetSymbolAddress(scratch) on device %d: %s",
                       dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<int32_t*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return SCOPE_OK;
}

static int transpose_checks(const int32_t* kv_num, const int32_t* kv_idx, int H, int QB, int NB, int maxkv,
                            const int32_t* q_off, const int32_t* q_list, const char* fn) {
  SCOPE_REQUIRE(kv_num && kv_idx && q_off && q_list, "%s: null pointer", fn);
  SCOPE_REQUIRE(H >= 1 && QB >= 1 && NB >= 1 && maxkv >= 1, "%s: bad sizes", fn);
  SCOPE_REQUIRE(static_cast<int64_t>(QB) * 4 <= 64 * 1024, "%s: QB=%d exceeds the LDS sort capacity", fn, QB);
  return SCOPE_OK;
}

// count -> scan -> fill -> sort with `cursor` [H·NB] as the fill cursors
// (cleared by the scan kernel, not by a memset, so the launches can be
// captured in a graph).
static int transpose_launch(const int32_t* kv_num, const int32_t* kv_idx, int H, int QB, int NB, int maxkv,
                            int32_t* q_off, int32_t* q_list, int32_t* cursor, hipStream_t s) {
  const int64_t n_off = static_cast<int64_t>(H) * (NB + 1);
  hipLaunchKernelGGL(fill_i32_kernel, dim3(ceil_div(n_off, 256)), dim3(256), 0, s, q_off, n_off, 0);
  const int64_t slots = static_cast<int64_t>(H) * QB * maxkv;
  hipLaunchKernelGGL(tr_count_kernel, dim3(ceil_div(slots, 256)), dim3(256), 0, s, kv_num, kv_idx, H, QB, NB, maxkv,
                     q_off);
  hipLaunchKernelGGL(tr_scan_kernel, dim3(H), dim3(1024), 0, s, NB, q_off, static_cast<int64_t>(QB) * maxkv, q_list,
                     cursor);
  hipLaunchKernelGGL(tr_fill_kernel, dim3(ceil_div(slots, 256)), dim3(256), 0, s, kv_num, kv_idx, H, QB, NB, maxkv,
                     q_off, cursor, q_list);
  hipLaunchKernelGGL(tr_sort_kernel, dim3(ceil_div(NB, kSortBuckets), H), dim3(256), QB * sizeof(int), s, NB, QB,
                     maxkv, q_off, q_list);
  return check_launch("transpose kernels");
}

}  // namespace scope

using namespace scope;

extern "C" {

int64_t scope_transpose_workspace_bytes(int H, int NB) { return static_cast<int64_t>(H) * NB * 4; }

int scope_transpose_blocks(const int32_t* kv_num, const int32_t* kv_idx, int H, int QB, int NB, int maxkv,
                           int32_t* q_off, int32_t* q_list, void* workspace, void* stream) {
  int rc = transpose_checks(kv_num, kv_idx, H, QB, NB, maxkv, q_off, q_list, "scope_transpose_blocks");
  if (rc) return rc;
  SCOPE_REQUIRE(workspace, "scope_transpose_blocks: null workspace");
  return transpose_launch(kv_num, kv_idx, H, QB, NB, maxkv, q_off, q_list, static_cast<int32_t*>(workspace),
                          as_stream(stream));
}

int scope_transpose_blocks_noalloc(const int32_t* kv_num, const int32_t* kv_idx, int H, int QB, int NB, int maxkv,
                                   int32_t* q_off, int32_t* q_list, void* stream) {
  int rc = transpose_checks(kv_num, kv_idx, H, QB, NB, maxkv, q_off, q_list, "scope_transpose_blocks_noalloc");
  if (rc) return rc;
  if (static_cast<int64_t>(H) * NB > SCOPE_NOALLOC_MAX_HNB)
    return set_error(SCOPE_ERANGE, "scope_transpose_blocks_noalloc: H*NB = %lld exceeds the static scratch of %d "
                     "cursors (use scope_transpose_blocks with a workspace)",
                     static_cast<long long>(H) * NB, SCOPE_NOALLOC_MAX_HNB);
  int32_t* cursor = nullptr;
  rc = noalloc_scratch(stream, &cursor);
  if (rc) return rc;
  return transpose_launch(kv_num, kv_idx, H, QB, NB, maxkv, q_off, q_list, cursor, as_stream(stream));
}

int scope_check_lists(const int32_t* kv_num, const int32_t* kv_idx, int H, int QB, int NB, int maxkv, int causal,
                      int32_t* res, void* stream) {
  SCOPE_REQUIRE(kv_num && kv_idx && res, "scope_check_lists: null pointer");
  SCOPE_REQUIRE(H >= 1 && QB >= 1 && NB >= 1 && maxkv >= 1, "scope_check_lists: bad sizes");
  SCOPE_REQUIRE(NB <= 65536, "scope_check_lists: NB=%d above 65536", NB);
  const hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(chk_init_kernel, dim3(1), dim3(64), 0, s, res);
  const int64_t rows = static_cast<int64_t>(H) * QB;
  const size_t lds = static_cast<size_t>(4) * ((NB + 31) / 32) * sizeof(uint32_t);
  hipLaunchKernelGGL(chk_lists_kernel, dim3(ceil_div(rows, 4)), dim3(256), lds, s, kv_num, kv_idx, H, QB, NB, maxkv,
                     causal ? 1 : 0, res);
  return check_launch("scope_check_lists");
}

}  // extern "C"
