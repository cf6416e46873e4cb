// Kernel 3: fused mask statistics for gfx950.
//
// One thread per (head, q-block) computes, in one pass, whichever groups the
// caller enabled:
//   A  forward debug statistics        model/attn_bias.py:510-600
//   B  mask debug statistics           model/attn_bias.py:839-849
//   C  block-scoring pick statistics   (same histograms over the picks)
// Histograms and counts are exact integers (LDS atomics, then one global
// atomic per bin and workgroup).  Fractions are count/n in fp32, as
// bool.float().mean() gives for exact counts.  The π-entropy mean is summed
// in a fixed order (deterministic).  Compiled with -ffp-contract=off.
#include <math.h>

#include "common.h"

namespace scope {

__constant__ int64_t kTokenEdges[15] = {0,     127,   255,    511,    1023,   2047,   4095,   8191,
                                        16383, 32767, 65535, 131071, 262143, 524287, 1048575};
__constant__ int64_t kBlockEdges[14] = {0, 1, 3, 7, 15, 31, 63, 127, 255, 511, 1023, 2047, 4095, 8191};

// torch.bucketize(right=False): number of edges strictly below x
__device__ __forceinline__ int bucket_tok(int64_t x) {
  int i = 0;
#pragma unroll
  for (int e = 0; e < 15; ++e) i += kTokenEdges[e] < x ? 1 : 0;
  return i;
}
__device__ __forceinline__ int bucket_blk(int64_t x) {
  int i = 0;
#pragma unroll
  for (int e = 0; e < 14; ++e) i += kBlockEdges[e] < x ? 1 : 0;
  return i;
}
__device__ __forceinline__ int64_t floor_div(int64_t a, int64_t b) {
  int64_t q = a / b;
  return (a % b != 0 && ((a < 0) != (b < 0))) ? q - 1 : q;
}

struct StatsLaunch {
  scope_stats_params p;
  int n_counts;  // total length of the counts array
};

__global__ void stats_zero_kernel(int32_t* __restrict__ counts, int n) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) counts[i] = 0;
}

__global__ __launch_bounds__(256) void stats_kernel(StatsLaunch A, const float* __restrict__ delta_star,
                                                     const float* __restrict__ pi,
                                                     const int32_t* __restrict__ ds_ptr_fwd,
                                                     const int32_t* __restrict__ ds_local_fwd,
                                                     const int32_t* __restrict__ kv_num,
                                                     const int32_t* __restrict__ radius,
                                                     const int32_t* __restrict__ picks,
                                                     const int32_t* __restrict__ ds_ptr,
                                                     const int32_t* __restrict__ ds_local,
                                                     int32_t* __restrict__ counts, float* __restrict__ entropy) {
  extern __shared__ int sh[];
  const scope_stats_params& P = A.p;
  for (int i = threadIdx.x; i < A.n_counts; i += blockDim.x) sh[i] = 0;
  __syncthreads();
  const int64_t row = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int QB = P.QB;
  if (row < static_cast<int64_t>(P.H) * QB) {
    const int h = static_cast<int>(row / QB);
    const int qb = static_cast<int>(row % QB);
    const int NB = QB;
    const int64_t t_rep = static_cast<int64_t>(qb + 1) * P.bs - 1;
    const int kv_off = SCOPE_ST_FIXED;
    const int r_off = kv_off + P.maxkv_bins;
    const int e_off = r_off + P.radius_bins;

    // ---- A: forward statistics
    if (delta_star && pi) {
      const int local = min(P.local_blocks_cfg, NB);
      int64_t local_start = max(static_cast<int64_t>(qb) - (local - 1), static_cast<int64_t>(0));
      if (P.docstart_enabled) local_start = max(local_start, static_cast<int64_t>(ds_local_fwd[qb]));
      float ent = 0.f;
      for (int m = 0; m < P.M; ++m) {
        const int64_t base = h * P.stride_h + m;
        float d, pr;
        if (!P.rep_mean) {
          d = delta_star[base + t_rep * P.stride_t];
          pr = pi[base + t_rep * P.stride_t];
        } else {
          float sd = 0.f, sp = 0.f;
          const int64_t t0 = static_cast<int64_t>(qb) * P.bs;
          for (int i = 0; i < P.bs; ++i) {
            sd += delta_star[base + (t0 + i) * P.stride_t];
            sp += pi[base + (t0 + i) * P.stride_t];
          }
          d = sd / static_cast<float>(P.bs);
          pr = sp / static_cast<float>(P.bs);
        }
        const int64_t dtok = static_cast<int64_t>(d);
        atomicAdd(&sh[SCOPE_ST_DELTA_TOKENS + bucket_tok(dtok)], 1);
        atomicAdd(&sh[SCOPE_ST_DELTA_BLOCKS + bucket_blk(floor_div(dtok, P.bs))], 1);
        float key = fmaxf(static_cast<float>(t_rep) - d, 0.0f);
        int64_t c = min(static_cast<int64_t>(key) / P.bs, static_cast<int64_t>(qb));
        if (P.has_docs) {
          c = max(c, static_cast<int64_t>(ds_ptr_fwd[qb]));
          if (P.docstart_enabled && c == ds_ptr_fwd[qb]) atomicAdd(&sh[SCOPE_ST_DOCSTART], 1);
        }
        atomicAdd(&sh[SCOPE_ST_CENTER + bucket_blk(c)], 1);
        if (c < local_start) atomicAdd(&sh[SCOPE_ST_OUTSIDE], 1);
        if (c == 0) atomicAdd(&sh[SCOPE_ST_BLOCK0], 1);
        if (qb >= 4 && c == 0) atomicAdd(&sh[SCOPE_ST_BLOCK0_EXCL], 1);
        const float lg = logf(pr + P.eps);
        ent = ent - pr * lg;
      }
      entropy[row] = ent;
    }
    // ---- B: mask statistics (reference mode)
    if (radius) {
      atomicAdd(&sh[kv_off + kv_num[row]], 1);
      int sum = 0;
      for (int m = 0; m < P.M; ++m) {
        const int r = radius[row * P.M + m];
        atomicAdd(&sh[r_off + r], 1);
        if (r == 0) atomicAdd(&sh[SCOPE_ST_RADIUS0], 1);
        sum += r;
      }
      atomicAdd(&sh[e_off + min(sum, P.extra_bins - 1)], 1);
    }
    // ---- C: block-scoring picks
    if (picks) {
      if (!radius) atomicAdd(&sh[kv_off + kv_num[row]], 1);
      const int loc = max(max(qb - (P.bs_local_blocks - 1), 0), ds_local[qb]);
      for (int i = 0; i < P.budget; ++i) {
        const int pk = picks[row * P.budget + i];
        if (pk < 0) continue;
        atomicAdd(&sh[SCOPE_ST_BS_N], 1);
        atomicAdd(&sh[SCOPE_ST_PTR_DIST + bucket_blk(qb - pk)], 1);
        if (pk < loc) atomicAdd(&sh[SCOPE_ST_BS_OUTSIDE], 1);
        if (pk == 0) atomicAdd(&sh[SCOPE_ST_BS_BLOCK0], 1);
        if (qb >= 4) {
          atomicAdd(&sh[SCOPE_ST_BS_N_EXCL], 1);
          if (pk == 0) atomicAdd(&sh[SCOPE_ST_BS_BLOCK0_EXCL], 1);
        }
        if (pk == ds_ptr[qb]) atomicAdd(&sh[SCOPE_ST_BS_DOCSTART], 1);
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < A.n_counts; i += blockDim.x)
    if (sh[i]) atomicAdd(&counts[i], sh[i]);
}

__device__ __forceinline__ float ratio(int c, int n) {
  return n > 0 ? static_cast<float>(c) / static_cast<float>(n) : 0.0f;
}

__global__ __launch_bounds__(256) void stats_finalize_kernel(StatsLaunch A, int has_fwd, int has_radius,
                                                              int has_picks, const float* __restrict__ entropy,
                                                              int32_t* __restrict__ counts,
                                                              float* __restrict__ values) {
  const scope_stats_params& P = A.p;
  __shared__ float red[256];
  const int64_t n = static_cast<int64_t>(P.H) * P.QB;
  float s = 0.f;
  if (has_fwd)
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) s += entropy[i];
  red[threadIdx.x] = s;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (threadIdx.x < o) red[threadIdx.x] += red[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x != 0) return;
  const int NB = P.QB;
  const int nc = P.H * P.QB * P.M;
  const int nx = NB > 4 ? P.H * (P.QB - 4) * P.M : 0;
  if (has_fwd) {
    counts[SCOPE_ST_N_CENTRES] = nc;
    counts[SCOPE_ST_N_CENTRES_EXCL] = nx;
    values[SCOPE_SV_PI_ENTROPY_MEAN] = red[0] / static_cast<float>(n);
    values[SCOPE_SV_DOCSTART_FRAC] = P.docstart_enabled ? ratio(counts[SCOPE_ST_DOCSTART], nc) : 0.0f;
    values[SCOPE_SV_OUTSIDE_LOCAL_FRAC] = ratio(counts[SCOPE_ST_OUTSIDE], nc);
    values[SCOPE_SV_BLOCK0_FRAC] = ratio(counts[SCOPE_ST_BLOCK0], nc);
    values[SCOPE_SV_BLOCK0_FRAC_EXCL] = NB > 4 ? ratio(counts[SCOPE_ST_BLOCK0_EXCL], nx) : 0.0f;
  }
  if (has_radius) {
    counts[SCOPE_ST_N_RADIUS] = P.H * P.QB * P.M;
    values[SCOPE_SV_RADIUS0_FRAC] = ratio(counts[SCOPE_ST_RADIUS0], P.H * P.QB * P.M);
  }
  if (has_picks) {
    const int nb = counts[SCOPE_ST_BS_N];
    values[SCOPE_SV_BS_OUTSIDE_LOCAL_FRAC] = ratio(counts[SCOPE_ST_BS_OUTSIDE], nb);
    values[SCOPE_SV_BS_BLOCK0_FRAC] = ratio(counts[SCOPE_ST_BS_BLOCK0], nb);
    values[SCOPE_SV_BS_BLOCK0_FRAC_EXCL] = ratio(counts[SCOPE_ST_BS_BLOCK0_EXCL], counts[SCOPE_ST_BS_N_EXCL]);
    values[SCOPE_SV_BS_DOCSTART_FRAC] = ratio(counts[SCOPE_ST_BS_DOCSTART], nb);
  }
}

}  // namespace scope

using namespace scope;

extern "C" {

int64_t scope_stats_counts_len(const scope_stats_params* p) {
  if (!p) return 0;
  return SCOPE_ST_FIXED + p->maxkv_bins + p->radius_bins + p->extra_bins;
}

int64_t scope_stats_workspace_bytes(const scope_stats_params* p) {
  if (!p) return 0;
  return static_cast<int64_t>(p->H) * p->QB * 4;
}

int scope_mask_stats(const scope_stats_params* p, const float* delta_star, const float* pi,
                     const int32_t* ds_ptr_fwd, const int32_t* ds_local_fwd, const int32_t* kv_num,
                     const int32_t* radius, const int32_t* picks, const int32_t* ds_ptr, const int32_t* ds_local,
                     int32_t* counts, float* values, void* workspace, void* stream) {
  SCOPE_REQUIRE(p && counts && values, "scope_mask_stats: null pointer");
  SCOPE_REQUIRE(p->H >= 1 && p->QB >= 1 && p->bs >= 1, "scope_mask_stats: bad sizes");
  const bool has_fwd = delta_star && pi;
  SCOPE_REQUIRE(!has_fwd || (workspace && p->M >= 1 && p->T == static_cast<int64_t>(p->QB) * p->bs),
                "scope_mask_stats: forward statistics need workspace, M >= 1 and T == QB*bs");
  SCOPE_REQUIRE(!has_fwd || !p->has_docs || (ds_ptr_fwd && ds_local_fwd),
                "scope_mask_stats: forward statistics with docs need ds_ptr_fwd/ds_local_fwd");
  SCOPE_REQUIRE(!(radius && picks), "scope_mask_stats: radius and picks statistics are exclusive");
  SCOPE_REQUIRE(!(radius || picks) || kv_num, "scope_mask_stats: kv_num required");
  SCOPE_REQUIRE(!radius || (p->M >= 1 && p->radius_bins >= 1 && p->extra_bins >= 1 && p->maxkv_bins >= 1),
                "scope_mask_stats: bad histogram sizes");
  SCOPE_REQUIRE(!picks || (ds_ptr && ds_local && p->maxkv_bins >= 1 && p->budget >= 0),
                "scope_mask_stats: pick statistics need ds_ptr/ds_local and kv bins");
  StatsLaunch A;
  A.p = *p;
  A.n_counts = static_cast<int>(scope_stats_counts_len(p));
  SCOPE_REQUIRE(A.n_counts * 4 <= 48 * 1024, "scope_mask_stats: %d counters exceed LDS", A.n_counts);
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(stats_zero_kernel, dim3(ceil_div(A.n_counts, 256)), dim3(256), 0, s, counts, A.n_counts);
  const int64_t rows = static_cast<int64_t>(p->H) * p->QB;
  hipLaunchKernelGGL(stats_kernel, dim3(ceil_div(rows, 256)), dim3(256), A.n_counts * sizeof(int), s, A,
                     has_fwd ? delta_star : nullptr, has_fwd ? pi : nullptr, ds_ptr_fwd, ds_local_fwd, kv_num, radius,
                     picks, ds_ptr, ds_local, counts, static_cast<float*>(workspace));
  int rc = check_launch("stats_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(stats_finalize_kernel, dim3(1), dim3(256), 0, s, A, has_fwd ? 1 : 0, radius ? 1 : 0,
                     picks ? 1 : 0, static_cast<const float*>(workspace), counts, values);
  return check_launch("stats_finalize_kernel");
}

}  // extern "C"
