// Fused coefficient head of SpectralBias.forward (model/attn_bias.py:419-506):
// the [rows, M, K] mixture that turns the MLP output y into the band
// coefficients and the per-row pointer terms, its regularisers, and its
// backward.  The MLP that produces y runs before it (mlp.hip); everything
// between y and the outputs is one pass over y with eight lanes per (b, h, t)
// row, lane m taking mixture peak m.
//
// Per row, with y = [delta_raw | mu_raw | sigma_raw | pi_logits |
// budget_logits | c_raw] (M columns each, c_raw only with use_slope):
//   Δ*_m = σ(delta_raw_m)·cap                       (:436-438)
//   μ_m  = logw_min + (logw_max - logw_min)·σ(mu_raw_m)   (:441-443)
//   s_m  = 0.25 + 1.75·σ(sigma_raw_m)                (:445)
//   π    = softmax(pi_logits)                          (:446)
//   slope = c_scale·tanh(c_raw)                         (:448-451)
//   a_mk = e_mk / (Σ_k e_mk + eps),  e_mk = exp(-(log ω_k - μ_m)² / (2 s_m²))   (:453-459)
//   coeff_cos_k = Σ_m π_m a_mk cos(ω_k Δ*_m), coeff_sin_k likewise with sin (:461-468)
//   b0 = Σ_k coeff_cos_k                                (:470-473)
//   delta_main = Δ*_{argmax π} (first maximum), width = w_min + (w_max - w_min)·σ(mean_m μ_m) (:476-478)
// Regularisers (training, :480-506), per row and then averaged:
//   omega     λ_ω · mean_{rows,m} Σ_k ω_k² a_mk²
//   entropy   λ_H · mean_rows relu(h_floor - H(π)),  H = -Σ π log(π + eps)
//   delta_edge λ_e · mean_{rows,m} relu(ε - u) + relu(u - (1 - ε)),  u = clamp(Δ*/max(cap, 1), 0, 1)
//   zero_mean λ_0 · (mean_rows b̄)²,  b̄ = Σ_k cc_k c̄_k + Σ_k cs_k s̄_k + slope·(L-1)/2 - b0
// The per-row partial sums are reduced in a fixed order (per workgroup in
// double precision, then the workgroups in index order), so the result does
// not depend on scheduling.
#include <math.h>

#include "common.h"

namespace scope {

namespace {

constexpr int kMaxM = 8, kMaxK = 16;
constexpr int kCoeffThreads = 256;

__device__ __forceinline__ float sigm(float x) { return 1.f / (1.f + expf(-x)); }

__device__ __forceinline__ float load_y(const void* y, bool bf16, int64_t i) {
  return bf16 ? bf16_to_f32(static_cast<const uint16_t*>(y)[i]) : static_cast<const float*>(y)[i];
}

// Lanes per row: lane m of a group of eight takes peak m (m < M <= 8); the
// sums over the peaks are 8-lane reductions inside the group.  With a thread
// per row the kernels would run two wavefronts per SIMD, each working through
// M·K exp and sincos calls one after another.
constexpr int kCoeffGroup = 8;
constexpr int kCoeffRows = kCoeffThreads / kCoeffGroup;  // rows per workgroup pass
constexpr int kCoeffPasses = 4;                           // forward: passes per workgroup (one partial per 128 rows)

template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
// op over the 8 lanes of the group, the same value in every lane (op is
// commutative): quad xor 1, quad xor 2, then the mirrored quad of the eight
template <typename Op>
__device__ __forceinline__ float grp_reduce(float x, Op op) {
  x = op(x, dpp_f<0xB1>(x));
  x = op(x, dpp_f<0x4E>(x));
  x = op(x, dpp_f<0x141>(x));
  return x;
}
__device__ __forceinline__ float grp_sum(float x) {
  return grp_reduce(x, [](float u, float v) { return u + v; });
}
__device__ __forceinline__ float grp_max(float x) {
  return grp_reduce(x, [](float u, float v) { return fmaxf(u, v); });
}
__device__ __forceinline__ float grp_min(float x) {
  return grp_reduce(x, [](float u, float v) { return fminf(u, v); });
}

// One lane's peak m of a row, and the row terms every lane of the group holds.
// Lanes m >= M read column 0 for the sigmoids (finite, unused) and carry π = 0.
struct CoeffPeak {
  float sd, ds;  // σ(delta_raw_m), Δ*_m
  float sm, mu;  // σ(mu_raw_m), μ_m
  float ss, sg;  // σ(sigma_raw_m), s_m
  float pi;      // π_m
  float th;      // tanh(c_raw) of the row
  int amax;      // first maximum of π over the row
};

// Every lane of the group must call this (group reductions inside).
__device__ __forceinline__ void coeff_peak(const scope_coeff_params& p, const void* y, int64_t row, int m, bool act,
                                           CoeffPeak& R) {
  const int M = p.M;
  const bool bf = p.y_bf16 != 0;
  const int64_t base = row * p.y_stride;
  const int mm = act ? m : 0;
  R.sd = sigm(load_y(y, bf, base + mm));
  R.ds = R.sd * p.delta_cap;
  R.sm = sigm(load_y(y, bf, base + M + mm));
  R.mu = p.logw_min + (p.logw_max - p.logw_min) * R.sm;
  R.ss = sigm(load_y(y, bf, base + 2 * M + mm));
  R.sg = 0.25f + 1.75f * R.ss;
  const float lg = act ? load_y(y, bf, base + 3 * M + mm) : -INFINITY;
  const float mx = grp_max(lg);
  const float ex = act ? expf(lg - mx) : 0.f;
  R.pi = ex / grp_sum(ex);
  const float best = grp_max(R.pi);
  R.amax = static_cast<int>(grp_min(act && R.pi == best ? static_cast<float>(m) : static_cast<float>(kCoeffGroup)));
  R.th = p.use_slope ? tanhf(load_y(y, bf, base + 5 * M)) : 0.f;
}

// e_mk for one peak (the caller normalises)
__device__ __forceinline__ float coeff_e(const float* logw, int k, float mu, float sg) {
  const float d = logw[k] - mu;
  return expf(-(d * d) / (2.f * (sg * sg)));
}

}  // namespace

template <int KK>
__global__ __launch_bounds__(kCoeffThreads) void coeff_fwd_kernel(
    scope_coeff_params p, const void* __restrict__ y, const float* __restrict__ omegas,
    const float* __restrict__ logw, const float* __restrict__ cmean, const float* __restrict__ smean,
    float* __restrict__ cc_out, float* __restrict__ cs_out, float* __restrict__ slope_out, float* __restrict__ b0_out,
    float* __restrict__ ds_out, float* __restrict__ pi_out, float* __restrict__ bl_out, float* __restrict__ dm_out,
    float* __restrict__ w_out, double* __restrict__ partial) {
  const int m = threadIdx.x % kCoeffGroup;
  double r_omega = 0.0, r_ent = 0.0, r_edge = 0.0, r_b = 0.0;  // this lane's regulariser terms
  for (int pass = 0; pass < kCoeffPasses; ++pass) {
    const int64_t row_id = (static_cast<int64_t>(blockIdx.x) * kCoeffPasses + pass) * kCoeffRows +
                           threadIdx.x / kCoeffGroup;
    const bool valid = row_id < p.rows;
    const int64_t row = valid ? row_id : p.rows - 1;  // every lane takes part in the group reductions
    const int M = p.M, K = p.K;
    const bool act = m < M;
    CoeffPeak R;
    coeff_peak(p, y, row, m, act, R);
    // cc_k = Σ_m π_m a_mk cos(ω_k Δ*_m): this lane's term, summed over the group
    float cc[KK], cs[KK];
    float om = 0.f;  // Σ_k ω_k² a_mk² of this peak
    {
      float e[KK], S = 0.f;
  #pragma unroll
      for (int k = 0; k < KK; ++k) {
        if (k >= K) break;
        e[k] = coeff_e(logw, k, R.mu, R.sg);
        S += e[k];
      }
      const float inv = 1.f / (S + p.eps);
  #pragma unroll
      for (int k = 0; k < KK; ++k) {
        if (k >= K) break;
        const float a = e[k] * inv;
        float sn, cn;
        sincosf(omegas[k] * R.ds, &sn, &cn);
        const float w = act ? R.pi * a : 0.f;
        cc[k] = grp_sum(w * cn);
        cs[k] = grp_sum(w * sn);
        if (act) om += omegas[k] * omegas[k] * a * a;
      }
    }
    float b0 = 0.f;
  #pragma unroll
    for (int k = 0; k < KK; ++k)
      if (k < K) b0 += cc[k];
    if (!p.subtract_b0) b0 = 0.f;
    const float slope = p.use_slope ? p.c_scale * R.th : 0.f;
    const float mus = grp_sum(act ? R.mu : 0.f);
    const float dmain = grp_sum(m == R.amax ? R.ds : 0.f);  // one nonzero term
    if (valid) {
      const int64_t rk = row * K, rm = row * M;
  #pragma unroll
      for (int k = 0; k < KK; ++k) {
        if (k >= K) break;
        if (k % kCoeffGroup == m) {
          cc_out[rk + k] = cc[k];
          cs_out[rk + k] = cs[k];
        }
      }
      if (act) {
        ds_out[rm + m] = R.ds;
        pi_out[rm + m] = R.pi;
        bl_out[rm + m] = load_y(y, p.y_bf16 != 0, row * p.y_stride + 4 * M + m);
      }
      if (m == 0) {
        slope_out[row] = slope;
        b0_out[row] = b0;
        dm_out[row] = dmain;
        w_out[row] = p.width_min + (p.width_max - p.width_min) * sigm(mus / static_cast<float>(M));
      }
    }
    if (p.training) {
      // per-lane terms: ω (per peak), entropy and zero-mean (per row, lane 0), edge (per peak)
      const float H = -grp_sum(act ? R.pi * logf(R.pi + p.eps) : 0.f);
      const float denom = fmaxf(p.delta_cap, 1.f);
      const float u = fminf(fmaxf(R.ds / denom, 0.f), 1.f);
      const float edge = fmaxf(p.delta_edge_eps - u, 0.f) + fmaxf(u - (1.f - p.delta_edge_eps), 0.f);
      float bb = slope * (0.5f * static_cast<float>(p.L - 1)) - b0;
  #pragma unroll
      for (int k = 0; k < KK; ++k)
        if (k < K) bb += cc[k] * cmean[k] + cs[k] * smean[k];
      if (valid && act) {
        r_omega += om;
        r_edge += edge;
      }
      if (valid && m == 0) {
        r_ent += fmaxf(p.entropy_floor - H, 0.f);
        r_b += bb;
      }
    }
  }
  if (!p.training) return;
  // workgroup partial sums, fixed order: lanes by xor-butterfly, wavefronts in index order
  double v[4] = {r_omega, r_ent, r_edge, r_b};
  for (int i = 0; i < 4; ++i)
    for (int o = 32; o > 0; o >>= 1) v[i] += __shfl_xor(v[i], o, kWave);
  __shared__ double red[kCoeffThreads / kWave][4];
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0)
    for (int i = 0; i < 4; ++i) red[wave][i] = v[i];
  __syncthreads();
  if (threadIdx.x < 4) {
    double s = 0.0;
    for (int w = 0; w < kCoeffThreads / kWave; ++w) s += red[w][threadIdx.x];
    partial[static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x] = s;
  }
}

// reg = [total, omega, entropy, delta_edge, zero_mean, mean_b]; one workgroup:
// thread t sums the workgroup partials t, t + 1024, ... into four interleaved
// accumulators (loads in flight), added in a fixed order, then a fixed tree
// over the threads
constexpr int kRegThreads = 1024;
__global__ __launch_bounds__(kRegThreads) void coeff_reg_kernel(scope_coeff_params p, int nblk,
                                                                const double* __restrict__ partial,
                                                                float* __restrict__ reg) {
  __shared__ double red[4][kRegThreads];
  const int t = threadIdx.x;
  double v[4][4] = {};
  int b = t;
  for (; b + 3 * kRegThreads < nblk; b += 4 * kRegThreads)
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) v[u][i] += partial[static_cast<int64_t>(b + u * kRegThreads) * 4 + i];
  for (; b < nblk; b += kRegThreads)
#pragma unroll
    for (int i = 0; i < 4; ++i) v[0][i] += partial[static_cast<int64_t>(b) * 4 + i];
#pragma unroll
  for (int i = 0; i < 4; ++i) red[i][t] = (v[0][i] + v[1][i]) + (v[2][i] + v[3][i]);
  __syncthreads();
  for (int o = kRegThreads / 2; o > 0; o >>= 1) {
    if (t < o)
      for (int i = 0; i < 4; ++i) red[i][t] += red[i][t + o];
    __syncthreads();
  }
  if (t != 0) return;
  const double tot[4] = {red[0][0], red[1][0], red[2][0], red[3][0]};
  const double N = static_cast<double>(p.rows), NM = N * p.M;
  const float omega = p.lambda_omega > 0.f ? static_cast<float>(p.lambda_omega * (tot[0] / NM)) : 0.f;
  const float ent = p.lambda_entropy > 0.f && p.entropy_floor > 0.f ? static_cast<float>(p.lambda_entropy * (tot[1] / N)) : 0.f;
  const float edge = p.lambda_delta_edge > 0.f ? static_cast<float>(p.lambda_delta_edge * (tot[2] / NM)) : 0.f;
  const float mb = static_cast<float>(tot[3] / N);
  const float zm = p.lambda_zero_mean > 0.f ? p.lambda_zero_mean * mb * mb : 0.f;
  reg[0] = omega + ent + edge + zm;  // the reference's order of the sum (:508)
  reg[1] = omega;
  reg[2] = ent;
  reg[3] = edge;
  reg[4] = zm;
  reg[5] = mb;
}

template <int KK>
__global__ __launch_bounds__(kCoeffThreads) void coeff_bwd_kernel(
    scope_coeff_params p, const void* __restrict__ y, const float* __restrict__ omegas,
    const float* __restrict__ logw, const float* __restrict__ cmean, const float* __restrict__ smean,
    const float* __restrict__ g_cc, const float* __restrict__ g_cs, const float* __restrict__ g_slope,
    const float* __restrict__ g_b0, const float* __restrict__ g_ds, const float* __restrict__ g_pi,
    const float* __restrict__ g_bl, const float* __restrict__ g_dm, const float* __restrict__ g_w,
    const float* __restrict__ g_reg, const float* __restrict__ reg, void* __restrict__ dy) {
  const int m = threadIdx.x % kCoeffGroup;
  const int64_t row_id = static_cast<int64_t>(blockIdx.x) * kCoeffRows + threadIdx.x / kCoeffGroup;
  const bool valid = row_id < p.rows;
  const int64_t row = valid ? row_id : p.rows - 1;  // every lane takes part in the group reductions
  const int M = p.M, K = p.K;
  const bool act = m < M;
  const int64_t rk = row * K, rm = row * M;
  CoeffPeak R;
  coeff_peak(p, y, row, m, act, R);
  float gcc[KK], gcs[KK];
#pragma unroll
  for (int k = 0; k < KK; ++k) {
    if (k >= K) break;
    gcc[k] = g_cc ? g_cc[rk + k] : 0.f;
    gcs[k] = g_cs ? g_cs[rk + k] : 0.f;
  }
  float gsl = g_slope ? g_slope[row] : 0.f;
  float gb0 = g_b0 ? g_b0[row] : 0.f;
  float gds = g_ds && act ? g_ds[rm + m] : 0.f;
  float gpi = g_pi && act ? g_pi[rm + m] : 0.f;
  float gmu = 0.f, gsg = 0.f;
  const float gr = (p.training && g_reg) ? g_reg[0] : 0.f;  // the same in every lane
  const float N = static_cast<float>(p.rows), NM = N * static_cast<float>(M);
  float c_om = 0.f;
  if (gr != 0.f) {
    if (p.lambda_zero_mean > 0.f) {
      const float gb = gr * p.lambda_zero_mean * 2.f * reg[5] / N;
#pragma unroll
      for (int k = 0; k < KK; ++k) {
        if (k >= K) break;
        gcc[k] += gb * cmean[k];
        gcs[k] += gb * smean[k];
      }
      gsl += gb * (0.5f * static_cast<float>(p.L - 1));
      gb0 -= gb;
    }
    if (p.lambda_entropy > 0.f && p.entropy_floor > 0.f) {
      const float H = -grp_sum(act ? R.pi * logf(R.pi + p.eps) : 0.f);
      if (p.entropy_floor - H > 0.f && act) {
        const float ge = gr * p.lambda_entropy / N;
        gpi += ge * (logf(R.pi + p.eps) + R.pi / (R.pi + p.eps));
      }
    }
    if (p.lambda_delta_edge > 0.f && act) {
      const float denom = fmaxf(p.delta_cap, 1.f), ge = gr * p.lambda_delta_edge / NM;
      const float x = R.ds / denom;
      const float u = fminf(fmaxf(x, 0.f), 1.f);
      const float de = (p.delta_edge_eps - u > 0.f ? -1.f : 0.f) + (u - (1.f - p.delta_edge_eps) > 0.f ? 1.f : 0.f);
      if (x >= 0.f && x <= 1.f) gds += ge * de / denom;
    }
    if (p.lambda_omega > 0.f) c_om = gr * p.lambda_omega / NM * 2.f;
  }
  if (p.subtract_b0) {
#pragma unroll
    for (int k = 0; k < KK; ++k)
      if (k < K) gcc[k] += gb0;
  }
  if (g_dm && m == R.amax) gds += g_dm[row];
  {
    float e[KK], a[KK], ga[KK], S = 0.f;
#pragma unroll
    for (int k = 0; k < KK; ++k) {
      if (k >= K) break;
      e[k] = coeff_e(logw, k, R.mu, R.sg);
      S += e[k];
    }
    const float inv = 1.f / (S + p.eps);
    float gdsm = 0.f, gpim = 0.f;
#pragma unroll
    for (int k = 0; k < KK; ++k) {
      if (k >= K) break;
      a[k] = e[k] * inv;
      float sn, cn;
      sincosf(omegas[k] * R.ds, &sn, &cn);
      const float G = gcc[k] * cn + gcs[k] * sn;
      gpim += a[k] * G;
      ga[k] = R.pi * G + c_om * omegas[k] * omegas[k] * a[k];
      gdsm += R.pi * a[k] * omegas[k] * (gcs[k] * cn - gcc[k] * sn);
    }
    gpi += gpim;
    gds += gdsm;
    // a = e / (S + eps)
    float dot = 0.f;
#pragma unroll
    for (int k = 0; k < KK; ++k)
      if (k < K) dot += ga[k] * a[k];
    const float is2 = 1.f / (R.sg * R.sg);
#pragma unroll
    for (int k = 0; k < KK; ++k) {
      if (k >= K) break;
      const float ge = (ga[k] - dot) * inv * e[k];
      const float d = logw[k] - R.mu;
      gmu += ge * d * is2;
      gsg += ge * d * d * is2 / R.sg;
    }
  }
  if (g_w) {
    const float mus = grp_sum(act ? R.mu : 0.f);
    const float sw = sigm(mus / static_cast<float>(M));
    gmu += g_w[row] * (p.width_max - p.width_min) * sw * (1.f - sw) / static_cast<float>(M);
  }
  const float gsum = grp_sum(act ? R.pi * gpi : 0.f);
  if (!valid) return;
  const bool bf = p.y_bf16 != 0;
  const int64_t base = row * p.y_stride;
  auto put = [&](int c, float v) {
    if (bf) static_cast<uint16_t*>(dy)[base + c] = f32_to_bf16(v);
    else static_cast<float*>(dy)[base + c] = v;
  };
  if (act) {
    put(m, gds * p.delta_cap * R.sd * (1.f - R.sd));
    put(M + m, gmu * (p.logw_max - p.logw_min) * R.sm * (1.f - R.sm));
    put(2 * M + m, gsg * 1.75f * R.ss * (1.f - R.ss));
    put(3 * M + m, R.pi * (gpi - gsum));
    put(4 * M + m, g_bl ? g_bl[rm + m] : 0.f);
  }
  int c0 = 5 * M;
  if (p.use_slope) {
    if (m == 0) put(c0, gsl * p.c_scale * (1.f - R.th * R.th));
    ++c0;
  }
  for (int c = c0 + m; c < p.y_cols; c += kCoeffGroup) put(c, 0.f);
}

}  // namespace scope

using namespace scope;

static int coeff_check(const scope_coeff_params* p, const char* who) {
  SCOPE_REQUIRE(p, "%s: null params", who);
  SCOPE_REQUIRE(p->M >= 1 && p->M <= kMaxM, "%s: M=%d outside [1, %d]", who, p->M, kMaxM);
  SCOPE_REQUIRE(p->K >= 1 && p->K <= kMaxK, "%s: K=%d outside [1, %d]", who, p->K, kMaxK);
  SCOPE_REQUIRE(p->rows >= 1 && p->L >= 1, "%s: rows=%lld L=%lld", who, (long long)p->rows, (long long)p->L);
  SCOPE_REQUIRE(p->y_cols >= 5 * p->M + (p->use_slope ? 1 : 0) && p->y_stride >= p->y_cols,
                "%s: y has %d columns (stride %d), needs %d", who, p->y_cols, p->y_stride,
                5 * p->M + (p->use_slope ? 1 : 0));
  return SCOPE_OK;
}

extern "C" int64_t scope_coeff_head_workspace_bytes(const scope_coeff_params* p) {
  if (!p || p->rows <= 0) return 0;
  return static_cast<int64_t>(ceil_div(p->rows, kCoeffPasses * kCoeffRows)) * 4 * static_cast<int64_t>(sizeof(double));
}

extern "C" int scope_coeff_head_fwd(const scope_coeff_params* p, const void* y, const float* omegas,
                                    const float* log_omegas, const float* cos_mean, const float* sin_mean,
                                    float* coeff_cos, float* coeff_sin, float* slope, float* b0, float* delta_star,
                                    float* pi, float* budget_logits, float* delta_main, float* width, float* reg,
                                    void* workspace, void* stream) {
  int rc = coeff_check(p, "scope_coeff_head_fwd");
  if (rc) return rc;
  SCOPE_REQUIRE(y && omegas && log_omegas && coeff_cos && coeff_sin && slope && b0 && delta_star && pi &&
                    budget_logits && delta_main && width,
                "scope_coeff_head_fwd: null pointer");
  SCOPE_REQUIRE(!p->training || (reg && workspace && cos_mean && sin_mean),
                "scope_coeff_head_fwd: training needs reg, workspace, cos_mean and sin_mean");
  const int nblk = ceil_div(p->rows, kCoeffPasses * kCoeffRows);
  hipStream_t s = as_stream(stream);
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(nblk), dim3(kCoeffThreads), 0, s, *p, y, omegas, log_omegas, cos_mean, sin_mean,
                       coeff_cos, coeff_sin, slope, b0, delta_star, pi, budget_logits, delta_main, width,
                       static_cast<double*>(workspace));
  };
  if (p->K <= 8) go(coeff_fwd_kernel<8>);
  else go(coeff_fwd_kernel<kMaxK>);
  rc = check_launch("coeff_fwd_kernel");
  if (rc || !p->training) return rc;
  hipLaunchKernelGGL(coeff_reg_kernel, dim3(1), dim3(kRegThreads), 0, s, *p, nblk, static_cast<const double*>(workspace),
                     reg);
  return check_launch("coeff_reg_kernel");
}

extern "C" int scope_coeff_head_bwd(const scope_coeff_params* p, const void* y, const float* omegas,
                                    const float* log_omegas, const float* cos_mean, const float* sin_mean,
                                    const float* g_coeff_cos, const float* g_coeff_sin, const float* g_slope,
                                    const float* g_b0, const float* g_delta_star, const float* g_pi,
                                    const float* g_budget_logits, const float* g_delta_main, const float* g_width,
                                    const float* g_reg, const float* reg, void* dy, void* stream) {
  int rc = coeff_check(p, "scope_coeff_head_bwd");
  if (rc) return rc;
  SCOPE_REQUIRE(y && omegas && log_omegas && dy, "scope_coeff_head_bwd: null pointer");
  SCOPE_REQUIRE(!(p->training && g_reg) || (reg && cos_mean && sin_mean),
                "scope_coeff_head_bwd: a regulariser gradient needs reg, cos_mean and sin_mean");
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(ceil_div(p->rows, kCoeffRows)), dim3(kCoeffThreads), 0, as_stream(stream), *p,
                       y, omegas, log_omegas, cos_mean, sin_mean, g_coeff_cos, g_coeff_sin, g_slope, g_b0,
                       g_delta_star, g_pi, g_budget_logits, g_delta_main, g_width, g_reg, reg, dy);
  };
  if (p->K <= 8) go(coeff_bwd_kernel<8>);
  else go(coeff_bwd_kernel<kMaxK>);
  return check_launch("coeff_bwd_kernel");
}
