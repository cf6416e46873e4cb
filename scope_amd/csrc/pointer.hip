// Kernel 1: pointer-driven block selection for gfx950.
//
//  * doc starts         model/attn_bias.py:688-709
//  * reference mode     model/attn_bias.py:711-837  (build_pointer_blockmask body)
//  * block means        q̄, k̄ per block (block-scoring mode)
//  * block-scoring mode block-mean q·k logits + distance prior + Gumbel top-k
//                       under a budget, union with window and global blocks
//
// One wavefront per (head, q-block).  Lists are sorted with a bitonic network
// in LDS and packed like the reference (unique ascending, then duplicates
// ascending).  Compiled with -ffp-contract=off: the radius allocation and the
// Gumbel scores must round exactly like the reference's fp32 tensor ops.
#include <limits.h>
#include <math.h>

#include "attn_common.h"

namespace scope {

constexpr int kMaxPeaks = 32;   // M limit of the reference mode (one lane per peak)
constexpr int kMaxBudget = 16;  // pointer slots of the block-scoring mode
constexpr int kMaxList = 1024;  // MAXKV limit (LDS sort network)

// ---------------------------------------------------------------------------
// shared wave-level utilities
// ---------------------------------------------------------------------------
// Bitonic sort of s[0..N) ascending (N a power of two) by one wavefront.
// Every wave of the workgroup must call it with the same N (it uses
// workgroup barriers between the network stages).
__device__ void wave_bitonic_sort(int* s, int N) {
  const int lane = lane_id();
  for (int k = 2; k <= N; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = lane; i < (N >> 1); i += kWave) {
        int lo = 2 * j * (i / j) + (i % j);
        int hi = lo + j;
        bool up = (lo & k) == 0;
        int a = s[lo], b = s[hi];
        if ((a > b) == up) {
          s[lo] = b;
          s[hi] = a;
        }
      }
      __syncthreads();
    }
  }
}

// Pack the sorted s[0..n): unique values ascending first, then duplicates
// ascending (model/attn_bias.py:829-837).  Returns the unique count.
__device__ int wave_pack_sorted(const int* s, int n, int* __restrict__ out, bool write) {
  const int lane = lane_id();
  const uint64_t below = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
  int nkeep = 0;
  for (int base = 0; base < n; base += kWave) {
    int e = base + lane;
    bool keep = e < n && (e == 0 || s[e] != s[e - 1]);
    nkeep += __popcll(__ballot(keep));
  }
  int kc = 0, dc = 0;
  for (int base = 0; base < n; base += kWave) {
    int e = base + lane;
    bool valid = e < n;
    bool keep = valid && (e == 0 || s[e] != s[e - 1]);
    bool dup = valid && !keep;
    uint64_t mk = __ballot(keep), md = __ballot(dup);
    if (write && keep) out[kc + __popcll(mk & below)] = s[e];
    if (write && dup) out[nkeep + dc + __popcll(md & below)] = s[e];
    kc += __popcll(mk);
    dc += __popcll(md);
  }
  return nkeep;
}

__device__ __forceinline__ float sigmoid_ref(float x) {
  // torch.sigmoid on fp32: 1 / (1 + exp(-x))
  float e = expf(-x);
  return 1.0f / (1.0f + e);
}

__device__ __forceinline__ float gumbel_of(float u, float eps) {
  // g = -log(-log(u + eps) + eps)   (model/attn_bias.py:771)
  float a = u + eps;
  float b = -logf(a);
  float c = b + eps;
  return -logf(c);
}

// ---------------------------------------------------------------------------
// doc starts
// ---------------------------------------------------------------------------
// Phase 1: per block, the last change point inside it (or -1) and whether the
// block's first token is a change point.
__global__ __launch_bounds__(256) void doc_blocks_kernel(const int32_t* __restrict__ docs, int64_t T,
                                                          int bs, int32_t* __restrict__ last_change,
                                                          int32_t* __restrict__ first_change) {
  const int b = blockIdx.x;
  const int64_t t0 = static_cast<int64_t>(b) * bs;
  int best = -1;
  for (int i = threadIdx.x; i < bs; i += blockDim.x) {
    int64_t t = t0 + i;
    bool ch = (t == 0) || (docs[t] != docs[t - 1]);
    if (ch) best = max(best, static_cast<int>(t));
  }
  __shared__ int red[256];
  red[threadIdx.x] = best;
  __syncthreads();
  for (int s = blockDim.x / 2; s > 0; s >>= 1) {
    if (threadIdx.x < s) red[threadIdx.x] = max(red[threadIdx.x], red[threadIdx.x + s]);
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    last_change[b] = red[0];
    first_change[b] = (t0 == 0 || docs[t0] != docs[t0 - 1]) ? 1 : 0;
  }
}

// Phase 2 (one workgroup): prefix max over blocks, then the three outputs.
// last_change aliases ds_tok_end and first_change aliases ds_local.
__global__ __launch_bounds__(1024) void doc_scan_kernel(int NB, int bs, int doc_clamp, int reset_len,
                                                         int32_t* __restrict__ ds_ptr,
                                                         int32_t* __restrict__ ds_local,
                                                         int32_t* __restrict__ ds_tok_end) {
  __shared__ int carry_s;
  __shared__ int wmax[16];
  if (threadIdx.x == 0) carry_s = -1;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  for (int base = 0; base < NB; base += 1024) {
    int b = base + threadIdx.x;
    int lc = b < NB ? ds_tok_end[b] : -1;
    int fc = b < NB ? ds_local[b] : 0;
    // inclusive prefix max of lc within the chunk: within each wavefront by
    // shuffles, then over the wavefronts' maxima
    int v = lc;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int u = __shfl_up(v, o, 64);
      if (lane >= o) v = max(v, u);
    }
    if (lane == 63) wmax[wv] = v;
    __syncthreads();  // wmax complete; carry_s of the previous chunk visible
    int before = carry_s;  // maximum of everything before this wavefront
    for (int w = 0; w < wv; ++w) before = max(before, wmax[w]);
    const int incl = max(v, before);
    const int prev = __shfl_up(incl, 1, 64);
    const int excl = lane > 0 ? prev : before;
    __syncthreads();  // everyone has read wmax and carry_s
    if (threadIdx.x == 1023) carry_s = incl;
    if (b < NB) {
      int64_t first_tok = static_cast<int64_t>(b) * bs;
      int64_t last_tok = first_tok + bs - 1;
      int dst_end = incl;                                     // doc start of the last token
      int dst_first = fc ? static_cast<int>(first_tok) : excl;  // doc start of the first token
      int p = doc_clamp ? dst_end / bs : 0;
      int l = doc_clamp ? dst_first / bs : 0;
      if (reset_len > 0) {
        int sp = static_cast<int>(((last_tok / reset_len) * reset_len) / bs);
        int sl = static_cast<int>(((first_tok / reset_len) * reset_len) / bs);
        p = max(p, sp);
        l = max(l, sl);
      }
      ds_ptr[b] = p;
      ds_local[b] = l;
      ds_tok_end[b] = dst_end;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// reference mode
// ---------------------------------------------------------------------------
struct RefLaunch {
  scope_ptr_ref_params p;
  int NB, L, N, NP, gmax;
};

__global__ __launch_bounds__(256) void ptr_ref_kernel(RefLaunch A, const float* __restrict__ delta_star,
                                                       const float* __restrict__ budget_logits,
                                                       const float* __restrict__ gumbel_u,
                                                       const int32_t* __restrict__ ds_ptr_a,
                                                       const int32_t* __restrict__ ds_local_a,
                                                       int32_t* __restrict__ kv_num, int32_t* __restrict__ kv_idx,
                                                       int32_t* __restrict__ radius, int32_t* __restrict__ centre) {
  extern __shared__ int smem[];
  const scope_ptr_ref_params& P = A.p;
  const int wave = threadIdx.x / kWave;
  const int lane = lane_id();
  const int NB = A.NB;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  const bool active = row < static_cast<int64_t>(P.H) * NB;
  const int h = active ? static_cast<int>(row / NB) : 0;
  const int qb = active ? static_cast<int>(row % NB) : 0;
  const int M = P.M;
  int* list = smem + wave * A.N;
  float* fs = reinterpret_cast<float*>(smem + 4 * A.N) + wave * 5 * kMaxPeaks;
  float* s_d = fs;                   // Δ* representatives
  float* s_b = fs + kMaxPeaks;       // budget representatives
  float* s_f = fs + 2 * kMaxPeaks;   // fractional parts / Gumbel scores
  int* s_r = reinterpret_cast<int*>(fs + 3 * kMaxPeaks);  // radius
  int* s_c = reinterpret_cast<int*>(fs + 4 * kMaxPeaks);  // centres
  const int ds_p = ds_ptr_a[qb];
  const int ds_l = ds_local_a[qb];
  const int64_t t_rep = static_cast<int64_t>(qb + 1) * P.bs - 1;

  // 1. representatives (model/attn_bias.py:713-719)
  if (active && lane < M) {
    const int64_t base = h * P.stride_h + lane;
    float d, b;
    if (!P.rep_mean) {
      d = delta_star[base + t_rep * P.stride_t];
      b = budget_logits[base + t_rep * P.stride_t];
    } else {
      float sd = 0.f, sb = 0.f;
      const int64_t t0 = static_cast<int64_t>(qb) * P.bs;
      for (int i = 0; i < P.bs; ++i) {
        sd += delta_star[base + (t0 + i) * P.stride_t];
        sb += budget_logits[base + (t0 + i) * P.stride_t];
      }
      d = sd / static_cast<float>(P.bs);
      b = sb / static_cast<float>(P.bs);
    }
    s_d[lane] = d;
    s_b[lane] = b;
  }
  __syncthreads();

  // 2. radius allocation (model/attn_bias.py:721-758)
  int r = 0;
  float fr = 0.f;
  int fl = 0, rem_int = 0;
  if (active && lane < M && P.radius_mode_pi && P.budget_rem > 0) {
    float rem = static_cast<float>(P.budget_rem);
    float a = 0.f;
    int floor_sum = 0;
    for (int mm = 0; mm < M - 1; ++mm) {
      float u = s_b[mm] / P.budget_temp;
      float v = sigmoid_ref(u);
      float bb = v * rem;
      if (mm == lane) a = bb;
      floor_sum += static_cast<int>(floorf(bb));
      rem = rem - bb;
    }
    if (lane == M - 1) a = rem;
    floor_sum += static_cast<int>(floorf(rem));
    float fa = floorf(a);
    fl = static_cast<int>(fa);
    fr = a - fa;
    rem_int = min(max(P.budget_rem - floor_sum, 0), M);
  }
  if (active && lane < M) s_f[lane] = fr;
  __syncthreads();
  if (active && lane < M) {
    if (P.radius_mode_pi) {
      if (P.budget_rem > 0) {
        int rank = 0;
        for (int mm = 0; mm < M; ++mm) {
          float o = s_f[mm];
          rank += (o > fr || (o == fr && mm < lane)) ? 1 : 0;
        }
        r = min(max(fl + (rank < rem_int ? 1 : 0), 0), P.ptr_half_blocks);
      } else {
        r = 0;
      }
    } else {
      r = P.half_active;
    }
    r = min(r, P.half_active);
    if (!P.mask_active) r = 0;
  }
  __syncthreads();
  // Gumbel top-k over peaks (model/attn_bias.py:763-777)
  if (P.gumbel_k > 0) {
    float sc = 0.f;
    if (active && lane < M) {
      float u = gumbel_u[(static_cast<int64_t>(h) * NB + qb) * M + lane];
      float b = s_b[lane] / P.gumbel_tau;
      sc = b + gumbel_of(u, P.eps);
      s_f[lane] = sc;
    }
    __syncthreads();
    if (active && lane < M) {
      int rank = 0;
      for (int mm = 0; mm < M; ++mm) {
        float o = s_f[mm];
        rank += (o > sc || (o == sc && mm < lane)) ? 1 : 0;
      }
      if (rank >= P.gumbel_k) r = 0;
    }
  }
  // centres (model/attn_bias.py:779-784)
  if (active && lane < M) {
    float key = static_cast<float>(t_rep) - s_d[lane];
    key = fmaxf(key, 0.0f);
    int64_t c = static_cast<int64_t>(key) / P.bs;
    c = min(c, static_cast<int64_t>(qb));
    if (!P.mask_active) c = qb;
    c = max(c, static_cast<int64_t>(ds_p));
    s_r[lane] = r;
    s_c[lane] = static_cast<int>(c);
    radius[(static_cast<int64_t>(h) * NB + qb) * M + lane] = r;
    centre[(static_cast<int64_t>(h) * NB + qb) * M + lane] = static_cast<int>(c);
  }
  __syncthreads();

  // 3. pieces: local | pointer | global (model/attn_bias.py:786-823)
  const int local = P.local_blocks;
  const int p = P.ptr_half_blocks;
  for (int e = lane; e < A.N; e += kWave) {
    int v = INT_MAX;
    if (active && e < A.L) {
      if (e < local) {
        v = max(max(qb - e, 0), ds_l);
      } else if (e < local + A.NP) {
        int idx = e - local;
        if (p > 0) {
          int m = idx / (2 * p + 1);
          int o = idx % (2 * p + 1) - p;
          int c = s_c[m];
          if (abs(o) <= s_r[m]) {
            v = min(max(c + o, 0), NB - 1);
            v = min(v, qb);
            v = max(v, ds_p);
          } else {
            v = c;
          }
        } else {
          v = s_c[idx];
        }
      } else {
        int g = e - local - A.NP;
        int ga = min(max(P.global_active, 0), A.gmax);
        v = g < ga ? min(ds_p + g, qb) : qb;
      }
    }
    list[e] = v;
  }
  __syncthreads();

  // 4. sort, dedupe, pack (model/attn_bias.py:825-837)
  wave_bitonic_sort(list, A.N);
  int n = wave_pack_sorted(list, A.L, kv_idx + row * A.L, active);
  if (active && lane == 0) kv_num[row] = n;
}

// ---------------------------------------------------------------------------
// block means
// ---------------------------------------------------------------------------
// With docs (scope_block_means_docs), the workgroups of head 0 also do the
// first phase of the document starts for their block (doc_blocks_kernel's
// work): the last change point inside it into last_change[b], whether its
// first token is one into first_change[b].
template <int D>
__global__ __launch_bounds__(256) void block_means_kernel(const uint16_t* __restrict__ q,
                                                           const uint16_t* __restrict__ k, int bs,
                                                           int64_t q_sh, int64_t q_st, int64_t k_sh,
                                                           int64_t k_st, int NB, float* __restrict__ qbar,
                                                           float* __restrict__ kbar,
                                                           const int32_t* __restrict__ docs = nullptr,
                                                           int32_t* __restrict__ last_change = nullptr,
                                                           int32_t* __restrict__ first_change = nullptr) {
  constexpr int kChunks = D / 8;        // 16-byte chunks per row
  constexpr int kGroups = 256 / kChunks;  // row groups
  __shared__ float red[2][kGroups][D + 4];
  const int b = blockIdx.x;
  const int h = blockIdx.y;
  const int c = threadIdx.x % kChunks;
  const int g = threadIdx.x / kChunks;
  float sq[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  float sk[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const int64_t t0 = static_cast<int64_t>(b) * bs;
  // up to four rows' loads in flight per thread.  Every byte of q and k is
  // read once here, so the loads are nontemporal (no cache retention): the
  // pass runs at 6.3-6.6 TB/s at T=131072 against 5.1-5.4 with plain loads.
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
#pragma unroll 4
  for (int r = g; r < bs; r += kGroups) {
    const u32x4 vq = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(q + h * q_sh + (t0 + r) * q_st + c * 8));
    const u32x4 vk = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(k + h * k_sh + (t0 + r) * k_st + c * 8));
    const uint32_t wq[4] = {vq.x, vq.y, vq.z, vq.w};
    const uint32_t wk[4] = {vk.x, vk.y, vk.z, vk.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sq[2 * i] += __uint_as_float(wq[i] << 16);
      sq[2 * i + 1] += __uint_as_float(wq[i] & 0xffff0000u);
      sk[2 * i] += __uint_as_float(wk[i] << 16);
      sk[2 * i + 1] += __uint_as_float(wk[i] & 0xffff0000u);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    red[0][g][c * 8 + i] = sq[i];
    red[1][g][c * 8 + i] = sk[i];
  }
  __syncthreads();
  if (threadIdx.x < 2 * D) {
    const int which = threadIdx.x / D;
    const int d = threadIdx.x % D;
    float s = 0.f;
    for (int gg = 0; gg < kGroups; ++gg) s += red[which][gg][d];
    float* out = which ? kbar : qbar;
    out[(static_cast<int64_t>(h) * NB + b) * D + d] = s / static_cast<float>(bs);
  }
  if (docs && h == 0) {
    // the block's last change point: the maximum over the tokens, per
    // wavefront by shuffles, then over the four wavefronts
    __shared__ int wbest[4];
    int best = -1;
    for (int i = threadIdx.x; i < bs; i += 256) {
      const int64_t t = t0 + i;
      if (t == 0 || docs[t] != docs[t - 1]) best = max(best, static_cast<int>(t));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) best = max(best, __shfl_xor(best, o, 64));
    if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
      last_change[b] = max(max(wbest[0], wbest[1]), max(wbest[2], wbest[3]));
      first_change[b] = (t0 == 0 || docs[t0] != docs[t0 - 1]) ? 1 : 0;
    }
  }
}

// ---------------------------------------------------------------------------
// block-scoring selection
// ---------------------------------------------------------------------------
struct ScoreLaunch {
  scope_ptr_score_params p;
  int L, N;
};

// better(a, b): higher score first, lower block index on ties
__device__ __forceinline__ bool better(float za, int ka, float zb, int kb) {
  return za > zb || (za == zb && ka < kb);
}

// One wavefront per q-block, kScoreQ q-blocks per workgroup.  The workgroup
// walks the key blocks of its range in chunks of 64 (one candidate per lane):
// each chunk's k̄ rows are staged in LDS once for all kScoreQ wavefronts, the
// next chunk's rows load into registers while the current one is scored, and
// the workgroups are issued last q-blocks first (they have the most
// candidates).
constexpr int kScoreQ = 8;

// KB: slots of the per-lane top list (the budget rounded up to 2, 4, 8 or 16).
// LG: the logits are given (logits_in): each wavefront walks its own
// candidates, the logits of four chunks loaded ahead, no k̄ staging.
template <int D, int KB, bool LG = false>
__global__ __launch_bounds__(kScoreQ * 64) void ptr_score_kernel(ScoreLaunch A, const float* __restrict__ qbar,
                                                                 const float* __restrict__ kbar,
                                                                 const float* __restrict__ logits_in,
                                                                 const float* __restrict__ prior,
                                                                 const float* __restrict__ gumbel_u,
                                                                 const int32_t* __restrict__ ds_ptr_a,
                                                                 const int32_t* __restrict__ ds_local_a,
                                                                 int32_t* __restrict__ kv_num,
                                                                 int32_t* __restrict__ kv_idx,
                                                                 int32_t* __restrict__ picks,
                                                                 float* __restrict__ logits_out) {
  constexpr int kStride = D + 4;  // padded k̄ row in LDS (16-byte aligned, conflict-free float4 reads)
  constexpr int NT = kScoreQ * kWave;
  constexpr int PF = (kWave * D / 4 + NT - 1) / NT;  // float4 of a chunk per thread
  __shared__ float ks[LG ? 1 : 2][LG ? 4 : kWave * kStride];  // k̄ chunks (not with given logits)
  __shared__ int lists[kScoreQ * 64];
  const scope_ptr_score_params& P = A.p;
  const int NB = P.NB;
  const int wave = threadIdx.x / kWave;
  const int lane = lane_id();
  const int h = blockIdx.y;
  const int qb0 = (gridDim.x - 1 - blockIdx.x) * kScoreQ;
  const int qb = __builtin_amdgcn_readfirstlane(qb0 + wave);
  const bool active = qb < NB;
  const int qbc = active ? qb : NB - 1;
  const int ds_p = ds_ptr_a[qbc];
  const int ds_l = ds_local_a[qbc];
  const int W = min(P.window, NB);
  const int G = min(P.n_global, NB);
  const int B = P.budget;
  const int wlo = max(qbc - W + 1, ds_l);        // window = [wlo, qb]
  const int ghi = min(ds_p + G - 1, qbc);         // global = [ds_p, ghi] (G > 0)
  const int64_t rowq = static_cast<int64_t>(h) * NB + qbc;

  // per-lane top-KB list (KB >= B), sorted best first; an empty slot holds
  // z = NaN (and kb = INT_MAX) until the merge, which sees -inf there
  float tz[KB];
  int tk[KB];
#pragma unroll
  for (int i = 0; i < KB; ++i) {
    tz[i] = __builtin_nanf("");
    tk[i] = INT_MAX;
  }
  const bool unit_temp = P.temp == 1.f;  // z = logit / 1 is the logit itself
  // candidate kb with its logit: the noise and the insertion into the list.
  // A lane meets its candidates in increasing kb (both loops below), so a new
  // candidate loses every tie on z to the entries already listed: it goes
  // into the first slot whose z it exceeds (!(z <= tz) is also true on an
  // empty slot, so a -inf z still takes the first empty one, as the lower
  // index wins its tie with an empty slot's -inf), and the slots below shift
  // down.  The compares all read the list before the insertion.
  auto consider = [&](int kb, float logit) __attribute__((always_inline)) {
    float z = unit_temp ? logit : logit / P.temp;
    if (P.noise_mode != 0) {
      float u = P.noise_mode == 1 ? gumbel_u[rowq * NB + kb]
                                  : counter_uniform(P.seed, static_cast<uint32_t>(h), static_cast<uint32_t>(qbc),
                                                    static_cast<uint32_t>(kb));
      z = z + gumbel_of(u, P.eps);
    }
    if (z != z) return;  // a NaN z (from NaN logits) never enters, as in the general comparison
    bool c[KB];
#pragma unroll
    for (int i = 0; i < KB; ++i) c[i] = !(z <= tz[i]);
#pragma unroll
    for (int i = KB - 1; i > 0; --i) {
      tz[i] = c[i - 1] ? tz[i - 1] : (c[i] ? z : tz[i]);
      tk[i] = c[i - 1] ? tk[i - 1] : (c[i] ? kb : tk[i]);
    }
    tz[0] = c[0] ? z : tz[0];
    tk[0] = c[0] ? kb : tk[0];
  };
  if constexpr (LG) {
    // this wavefront's candidates lie in [ds_p, qb]; chunks of 64, one per lane
    constexpr int PFN = 4;
    float lq[PFN];
    const int lo = ds_p;
    const bool copy_out = logits_out && logits_out != logits_in;
    auto load = [&](int kb0) __attribute__((always_inline)) {
      const int kb = kb0 + lane;
      return active && kb <= qbc ? logits_in[rowq * NB + kb] : 0.f;
    };
#pragma unroll
    for (int i = 0; i < PFN; ++i) lq[i] = load(lo + i * kWave);
    for (int kb0 = lo; kb0 <= qbc; kb0 += PFN * kWave) {
#pragma unroll
      for (int i = 0; i < PFN; ++i) {
        const int kb = kb0 + i * kWave + lane;
        const float logit = lq[i];
        lq[i] = load(kb0 + (i + PFN) * kWave);  // the chunk PFN ahead (0 past the row)
        if (copy_out && active && kb <= qbc) logits_out[rowq * NB + kb] = logit;
        const bool cand = active && kb <= qbc && !(kb >= wlo) && !(G > 0 && kb <= ghi);
        if (cand) consider(kb, logit);
      }
    }
  }

  if constexpr (!LG) {
  float qv[D];
  if (!logits_in) {
#pragma unroll
    for (int d = 0; d < D; ++d) qv[d] = qbar[rowq * D + d];
  }
  // kb range of the workgroup: [ds_ptr of its first q-block, its last q-block]
  const int lo_wg = ds_ptr_a[qb0];
  const int hi_wg = min(qb0 + kScoreQ - 1, NB - 1);
  float4 pf[PF];
  // rows kb0 .. min(kb0 + 63, hi_wg) of k̄ into registers, then into buffer b
  auto fetch = [&](int kb0) __attribute__((always_inline)) {
    const int nrow = min(kWave, hi_wg - kb0 + 1);
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int i = threadIdx.x + j * NT, rr = i / (D / 4), cc = i % (D / 4);
      pf[j] = i < kWave * D / 4 && rr < nrow
                  ? *reinterpret_cast<const float4*>(kbar + (static_cast<int64_t>(h) * NB + kb0 + rr) * D + cc * 4)
                  : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto stash = [&](int b) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < PF; ++j) {
      const int i = threadIdx.x + j * NT, rr = i / (D / 4), cc = i % (D / 4);
      if (i < kWave * D / 4) *reinterpret_cast<float4*>(&ks[b][rr * kStride + cc * 4]) = pf[j];
    }
  };
  if (!logits_in) {
    fetch(lo_wg);
    stash(0);
  }
  int buf = 0;
  for (int kb0 = lo_wg; kb0 <= hi_wg; kb0 += kWave) {
    const bool more = kb0 + kWave <= hi_wg;
    if (!logits_in) {
      __syncthreads();  // ks[buf] is complete; every wavefront is done with ks[buf ^ 1]
      if (more) fetch(kb0 + kWave);
    }
    const int kb = kb0 + lane;
    const bool cand = active && kb >= ds_p && kb <= qbc && !(kb >= wlo) && !(G > 0 && kb <= ghi);
    float logit = 0.f;
    bool causal = active && kb >= ds_p && kb <= qbc;
    if (causal) {
      if (logits_in) {
        logit = logits_in[rowq * NB + kb];
      } else {
        float acc = 0.f;
        const float* kr = &ks[buf][lane * kStride];
#pragma unroll
        for (int d = 0; d < D; d += 4) {
          const float4 kv4 = *reinterpret_cast<const float4*>(kr + d);
          acc = fmaf(qv[d], kv4.x, acc);
          acc = fmaf(qv[d + 1], kv4.y, acc);
          acc = fmaf(qv[d + 2], kv4.z, acc);
          acc = fmaf(qv[d + 3], kv4.w, acc);
        }
        logit = P.logit_scale * acc;
        if (prior) logit = logit + prior[h * P.prior_head_stride + (qbc - kb)];
      }
      if (logits_out) logits_out[rowq * NB + kb] = logit;
    }
    if (cand) consider(kb, logit);
    if (!logits_in && more) {
      stash(buf ^ 1);
      buf ^= 1;
    }
  }
  }  // !LG
  if (logits_out && active && !(P.flags & SCOPE_PTR_LOGITS_SCRATCH)) {
    // entries outside [ds_ptr, qb] are not candidates: -inf
    for (int kb = lane; kb < NB; kb += kWave)
      if (kb < ds_p || kb > qbc) logits_out[rowq * NB + kb] = -INFINITY;
  }

  // wave merge: B rounds of arg-best over the lanes' list heads
#pragma unroll
  for (int i = 0; i < KB; ++i) tz[i] = tk[i] == INT_MAX ? -INFINITY : tz[i];
  int* list = lists + wave * 64;
  for (int i = 0; i < B; ++i) {
    float bz = tz[0];
    int bk = tk[0];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      float oz = __shfl_xor(bz, o, kWave);
      int ok = __shfl_xor(bk, o, kWave);
      if (better(oz, ok, bz, bk)) {
        bz = oz;
        bk = ok;
      }
    }
    const bool valid = bk != INT_MAX;
    if (valid && tk[0] == bk) {
#pragma unroll
      for (int j = 0; j < KB - 1; ++j) {
        tz[j] = tz[j + 1];
        tk[j] = tk[j + 1];
      }
      tz[KB - 1] = -INFINITY;
      tk[KB - 1] = INT_MAX;
    }
    if (active && lane == 0) picks[rowq * B + i] = valid ? bk : -1;
    if (lane == 0) list[W + i] = valid ? bk : qbc;
  }
  // window and global entries
  if (lane < W) list[lane] = max(max(qbc - lane, 0), ds_l);
  if (lane < G) list[W + B + lane] = min(ds_p + lane, qbc);
  if (lane >= A.L && lane < A.N) list[lane] = INT_MAX;
  __syncthreads();
  wave_bitonic_sort(list, A.N);
  int n = wave_pack_sorted(list, A.L, kv_idx + rowq * A.L, active);
  if (active && lane == 0) kv_num[rowq] = n;
}


// ---------------------------------------------------------------------------
// block-scoring logits on bf16 MFMA with split operands (long sequences)
// ---------------------------------------------------------------------------
// logit[h, qb, kb] = logit_scale·q̄[qb]·k̄[kb] + prior[qb - kb] for kb <= qb.
// Each fp32 mean x is split into bf16 parts x = hi + lo + e with
// hi = bf16(x), lo = bf16(x - hi) and |e| <= 2^-18·|x|, and the product takes
// hi·hi + hi·lo + lo·hi on v_mfma_f32_32x32x16_bf16 (exact bf16 products,
// fp32 accumulation); the dropped lo·lo and the e terms are at most
// 3·2^-18 of |q̄_d·k̄_d| per term, far below the 1e-4 the selection's logits
// are held to.  The selection then reads the logits (ptr_score_kernel with
// logits_in).  With thousands of candidates per q-block the
// wavefront-per-row dot products of ptr_score_kernel (a fmaf chain per
// candidate) would take several times longer; the sum order differs, within
// fp32 rounding.
//
// One workgroup of sixteen wavefronts per CU (the split tiles' 139 KB of
// LDS leave room for one) loops over the 128x128 tiles of the lower
// triangle (all heads).  A tile's 128 q̄ rows and 128 k̄ rows are loaded into
// registers while the previous tile's MFMAs run, then split once into hi and
// lo bf16 tiles in LDS (rows padded by 16 bytes, so the 16-byte operand reads
// of 32 rows spread over the banks); each wavefront computes a 32x32
// sixteenth (3 MFMAs per step of 16 over D).  The tile loop is latency
// bound: at T=1M with four wavefronts of 64x64 it took 195 us, with eight
// of 32x64 147 us, with sixteen 131 us (the stores of the logits alone are
// about 50 us of HBM time).
constexpr int kLgTile = 128;
constexpr int kLgRow = 128 + 8;  // padded bf16 row of a split tile

__global__ __launch_bounds__(1024) void ptr_logits_kernel(int H, int NB, float logit_scale,
                                                         const float* __restrict__ qbar,
                                                         const float* __restrict__ kbar,
                                                         const float* __restrict__ prior, int64_t prior_stride,
                                                         float* __restrict__ logits) {
  constexpr int D = 128;
  constexpr int NT = 1024;
  constexpr int NF = kLgTile * D / 4 / NT;  // float4 per thread and operand
  // [operand: q̄ hi, q̄ lo, k̄ hi, k̄ lo][row][d]
  __shared__ __attribute__((aligned(16))) uint16_t sp[4][kLgTile * kLgRow];
  // the tile's prior values: prior[d] for d = qb - kb in dbase .. dbase + 255,
  // one per thread
  static_assert(2 * kLgTile == 256, "one prior value per thread of the first 256");
  __shared__ float spr[2 * kLgTile];
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, m = lane % 32, g = lane / 32;
  const int wr = wave / 4, wc = wave % 4;  // this wavefront's 32x32 sixteenth of the tile
  const int nt = (NB + kLgTile - 1) / kLgTile;
  const int per_h = nt * (nt + 1) / 2;
  const int total = H * per_h;
  // tile index -> (h, row tile rt, column tile ct <= rt)
  auto coords = [&](int t, int& h, int& rt, int& ct) __attribute__((always_inline)) {
    h = t / per_h;
    const int rem = t % per_h;
    rt = static_cast<int>((sqrtf(8.f * static_cast<float>(rem) + 1.f) - 1.f) * 0.5f);
    while (rt * (rt + 1) / 2 > rem) --rt;
    while ((rt + 1) * (rt + 2) / 2 <= rem) ++rt;
    ct = rem - rt * (rt + 1) / 2;
  };
  // raw operands of a tile: float4 f = tid + 256·i of the 128x128 q̄ (a) and
  // k̄ (b) row blocks, row f / 32, d = 4·(f % 32)
  float4 ra[NF], rb[NF];
  float rp = 0.f;  // this thread's prior value of the tile (index tid of its window)
  auto load = [&](int t) __attribute__((always_inline)) {
    int h, rt, ct;
    coords(t, h, rt, ct);
    if (prior && tid < 2 * kLgTile) {
      const int d = (rt - ct) * kLgTile - (kLgTile - 1) + tid;
      rp = d >= 0 && d < NB ? prior[h * prior_stride + d] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < NF; ++i) {
      const int f = tid + NT * i, r = f / (D / 4), d4 = f % (D / 4);
      const int qr = min(rt * kLgTile + r, NB - 1), kr = min(ct * kLgTile + r, NB - 1);
      ra[i] = *reinterpret_cast<const float4*>(qbar + (static_cast<int64_t>(h) * NB + qr) * D + 4 * d4);
      rb[i] = *reinterpret_cast<const float4*>(kbar + (static_cast<int64_t>(h) * NB + kr) * D + 4 * d4);
    }
  };
  auto stash = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NF; ++i) {
      const int f = tid + NT * i, r = f / (D / 4), d4 = f % (D / 4);
      const float4 v[2] = {ra[i], rb[i]};
#pragma unroll
      for (int o = 0; o < 2; ++o) {
        const uint32_t h01 = cvt_pk_bf16(v[o].x, v[o].y), h23 = cvt_pk_bf16(v[o].z, v[o].w);
        const uint32_t l01 = cvt_pk_bf16(v[o].x - bf16_lo(h01), v[o].y - bf16_hi(h01));
        const uint32_t l23 = cvt_pk_bf16(v[o].z - bf16_lo(h23), v[o].w - bf16_hi(h23));
        *reinterpret_cast<uint2*>(&sp[2 * o][r * kLgRow + 4 * d4]) = make_uint2(h01, h23);
        *reinterpret_cast<uint2*>(&sp[2 * o + 1][r * kLgRow + 4 * d4]) = make_uint2(l01, l23);
      }
    }
  };
  // XCD-contiguous tile ranges: workgroup b runs on XCD b % 8 and takes every
  // (grid/8)-th tile of that XCD's eighth of the (head, row tile, column
  // tile) sequence, so an XCD's L2 serves the q̄ and k̄ rows of its own
  // heads (one head per XCD at H = 8).  The grid is a multiple of 8.
  const int xcd = blockIdx.x % 8, per_x = gridDim.x / 8;
  const int t_hi = static_cast<int>(static_cast<int64_t>(total) * (xcd + 1) / 8);
  int t = static_cast<int>(static_cast<int64_t>(total) * xcd / 8) + static_cast<int>(blockIdx.x / 8);
  if (t < t_hi) load(t);
  for (; t < t_hi; t += per_x) {
    int h, rt, ct;
    coords(t, h, rt, ct);
    __syncthreads();  // every wavefront is done reading the previous tile
    stash();
    if (tid < 2 * kLgTile) spr[tid] = rp;
    const int dbase = (rt - ct) * kLgTile - (kLgTile - 1);
    __syncthreads();  // the split tile is complete
    if (t + per_x < t_hi) load(t + per_x);  // under this tile's MFMAs
    f32x16_t acc = zero16();
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
      // A: q̄ row 32·wr + m, d = 16ks + 8g .. +7; B: the same for k̄ row 32·wc + m
      const int ar = (32 * wr + m) * kLgRow + 16 * ks + 8 * g;
      const int br = (32 * wc + m) * kLgRow + 16 * ks + 8 * g;
      const uint4 ah = *reinterpret_cast<const uint4*>(&sp[0][ar]);
      const uint4 al = *reinterpret_cast<const uint4*>(&sp[1][ar]);
      const uint4 bh = *reinterpret_cast<const uint4*>(&sp[2][br]);
      const uint4 bl = *reinterpret_cast<const uint4*>(&sp[3][br]);
      acc = mfma32(ah, bh, acc);
      acc = mfma32(ah, bl, acc);
      acc = mfma32(al, bh, acc);
    }
    // C layout: column m (key block), register r -> row 8(r/4) + 4g + r%4
    const int kb = ct * kLgTile + 32 * wc + m;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qb = rt * kLgTile + 32 * wr + 8 * (r / 4) + 4 * g + (r % 4);
      if (qb < NB && kb <= qb) {
        float lg = logit_scale * acc[r];
        if (prior) lg = lg + spr[qb - kb - dbase];
        logits[(static_cast<int64_t>(h) * NB + qb) * NB + kb] = lg;
      }
    }
  }
}

// two floats -> packed bf16 pair (round to nearest even; lo in the low half)
__device__ __forceinline__ uint32_t bf16_pack(float lo, float hi) {
  typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
  bf16x2_v v;
  v[0] = static_cast<__bf16>(lo);
  v[1] = static_cast<__bf16>(hi);
  return __builtin_bit_cast(uint32_t, v);
}

// ---------------------------------------------------------------------------
// soft pointer weights (no reference counterpart: model/attn_bias.py:623
// selects under torch.no_grad)
// ---------------------------------------------------------------------------
// b[h,qb,e] = log σ(z/τ_w) for the pick entries of the packed list (e <
// kv_num and kv_idx[e] one of the picks), 0 otherwise; z is the noise-free
// selection logit, computed exactly as ptr_score_kernel computes it (the
// same fmaf chain over d, then the prior), so b follows the ranked value.
// One wavefront per (h, qb), one lane per list entry.
template <int D>
__global__ __launch_bounds__(256) void pair_bias_kernel(ScoreLaunch A, float soft_temp, const float* __restrict__ qbar,
                                                         const float* __restrict__ kbar,
                                                         const float* __restrict__ logits_in,
                                                         const float* __restrict__ prior,
                                                         const int32_t* __restrict__ kv_num,
                                                         const int32_t* __restrict__ kv_idx,
                                                         const int32_t* __restrict__ picks, float* __restrict__ out) {
  const scope_ptr_score_params& P = A.p;
  const int NB = P.NB, B = P.budget, L = A.L;
  const int lane = lane_id();
  const int qb = blockIdx.x * 4 + threadIdx.x / kWave;
  const int h = blockIdx.y;
  if (qb >= NB || lane >= L) return;
  const int64_t row = static_cast<int64_t>(h) * NB + qb;
  const int n = kv_num[row];
  const int kb = kv_idx[row * L + lane];
  bool pick = false;
  for (int i = 0; i < B; ++i) pick = pick || (picks[row * B + i] == kb);
  float b = 0.f;
  if (lane < n && pick) {
    float logit;
    if (logits_in) {
      logit = logits_in[row * NB + kb];
    } else {
      const float* qr = qbar + row * D;
      const float* kr = kbar + (static_cast<int64_t>(h) * NB + kb) * D;
      float acc = 0.f;
#pragma unroll 8
      for (int d = 0; d < D; ++d) acc = fmaf(qr[d], kr[d], acc);
      logit = P.logit_scale * acc;
      if (prior) logit = logit + prior[h * P.prior_head_stride + (qb - kb)];
    }
    const float x = logit / soft_temp;
    b = fminf(x, 0.f) - log1pf(expf(-fabsf(x)));  // log σ(x)
  }
  out[row * L + lane] = b;
}

// Pointer backward, q side: per (h, qb), dz_e = db_e·(1 - e^b_e)/τ_w for the
// listed entries (0 where b = 0), stored for the k side; dq̄ = ls·Σ_e dz_e·k̄_kb
// (entries in list order), and every row of the q-block gets dq̄/bs.
__global__ __launch_bounds__(256) void ptr_bwd_q_kernel(scope_ptr_bwd_params P, const float* __restrict__ kbar,
                                                        const int32_t* __restrict__ kv_num,
                                                        const int32_t* __restrict__ kv_idx,
                                                        const float* __restrict__ pair_bias,
                                                        const float* __restrict__ dpair, float* __restrict__ dz,
                                                        uint16_t* __restrict__ dq) {
  __shared__ float dzs[64];
  __shared__ int kbs[64];
  __shared__ float dqb[128];
  const int qb = blockIdx.x, h = blockIdx.y;
  const int64_t row = static_cast<int64_t>(h) * P.NB + qb;
  const int L = P.maxkv;
  const int n = min(kv_num[row], L);
  for (int e = threadIdx.x; e < L; e += blockDim.x) {
    float v = 0.f;
    if (e < n) {
      const float b = pair_bias[row * L + e];
      v = b != 0.f ? dpair[row * L + e] * (1.f - expf(b)) / P.soft_temp : 0.f;
    }
    dz[row * L + e] = v;
    if (e < 64) {
      dzs[e] = v;
      kbs[e] = e < n ? kv_idx[row * L + e] : 0;
    }
  }
  __syncthreads();
  if (threadIdx.x < P.D) {
    const int d = threadIdx.x;
    float acc = 0.f;
    for (int e = 0; e < n; ++e)
      if (dzs[e] != 0.f) acc += dzs[e] * kbar[(static_cast<int64_t>(h) * P.NB + kbs[e]) * P.D + d];
    dqb[d] = P.logit_scale * acc / static_cast<float>(P.bs);
  }
  __syncthreads();
  // rows of the q-block: 8 bf16 per thread step
  const int chunks = P.bs * P.D / 8;
  for (int c = threadIdx.x; c < chunks; c += blockDim.x) {
    const int r = c / (P.D / 8), d0 = (c % (P.D / 8)) * 8;
    uint16_t* ptr = dq + h * P.q_sh + (static_cast<int64_t>(qb) * P.bs + r) * P.q_st + d0;
    uint4 v = *reinterpret_cast<const uint4*>(ptr);
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = __uint_as_float(w[i] << 16) + dqb[d0 + 2 * i];
      const float hi = __uint_as_float(w[i] & 0xffff0000u) + dqb[d0 + 2 * i + 1];
      w[i] = bf16_pack(lo, hi);
    }
    *reinterpret_cast<uint4*>(ptr) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

// Pointer backward, k side: per (h, kb), dk̄ = ls·Σ dz·q̄_qb over the q-blocks
// that list kb (the transposed list, ascending), and every row of the key
// block gets dk̄/bs.  The list is taken in chunks of 256 entries: first each
// thread finds its entry's dz (kb's position in that q-block's list, a scan
// of at most 64 contiguous entries), then the columns are summed over the
// chunk in list order.
__global__ __launch_bounds__(256) void ptr_bwd_k_kernel(scope_ptr_bwd_params P, const float* __restrict__ qbar,
                                                        const int32_t* __restrict__ kv_num,
                                                        const int32_t* __restrict__ kv_idx,
                                                        const int32_t* __restrict__ q_off,
                                                        const int32_t* __restrict__ q_list,
                                                        const float* __restrict__ dz, uint16_t* __restrict__ dk) {
  __shared__ float wz[256];
  __shared__ int wq[256];
  __shared__ float dks[128];
  __shared__ float part[2][128];
  const int kb = blockIdx.x, h = blockIdx.y;
  const int NB = P.NB, L = P.maxkv;
  const int32_t* qo = q_off + static_cast<int64_t>(h) * (NB + 1);
  const int32_t* ql = q_list + static_cast<int64_t>(h) * NB * L + qo[kb];
  const int nq = qo[kb + 1] - qo[kb];
  const int d = threadIdx.x & 127, half = threadIdx.x >> 7;
  float acc = 0.f;
  for (int c0 = 0; c0 < nq; c0 += 256) {
    const int cn = min(256, nq - c0);
    __syncthreads();  // the previous chunk's wz / wq are consumed
    if (threadIdx.x < cn) {
      const int qb = ql[c0 + threadIdx.x];
      const int64_t row = static_cast<int64_t>(h) * NB + qb;
      const int n = min(kv_num[row], L);
      float z = 0.f;
      for (int e = 0; e < n; ++e)
        if (kv_idx[row * L + e] == kb) z = dz[row * L + e];
      wz[threadIdx.x] = z;
      wq[threadIdx.x] = qb;
    }
    __syncthreads();
    if (d < P.D) {
      // the two halves of the chunk, each in list order
      const int mid = (cn + 1) / 2;
      const int i0 = half == 0 ? 0 : mid, i1 = half == 0 ? mid : cn;
      for (int i = i0; i < i1; ++i) {
        const float z = wz[i];
        if (z != 0.f) acc += z * qbar[(static_cast<int64_t>(h) * NB + wq[i]) * P.D + d];
      }
    }
  }
  if (d < P.D) part[half][d] = acc;
  __syncthreads();
  if (threadIdx.x < P.D) dks[threadIdx.x] = P.logit_scale * (part[0][threadIdx.x] + part[1][threadIdx.x]) /
                                           static_cast<float>(P.bs);
  __syncthreads();
  const int chunks = P.bs * P.D / 8;
  for (int c = threadIdx.x; c < chunks; c += blockDim.x) {
    const int r = c / (P.D / 8), d0 = (c % (P.D / 8)) * 8;
    uint16_t* ptr = dk + h * P.k_sh + (static_cast<int64_t>(kb) * P.bs + r) * P.k_st + d0;
    uint4 v = *reinterpret_cast<const uint4*>(ptr);
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float lo = __uint_as_float(w[i] << 16) + dks[d0 + 2 * i];
      const float hi = __uint_as_float(w[i] & 0xffff0000u) + dks[d0 + 2 * i + 1];
      w[i] = bf16_pack(lo, hi);
    }
    *reinterpret_cast<uint4*>(ptr) = make_uint4(w[0], w[1], w[2], w[3]);
  }
}

}  // namespace scope

using namespace scope;

extern "C" {

int scope_doc_starts(const int32_t* docs, int64_t T, int bs, int doc_clamp, int reset_len, int32_t* ds_ptr,
                     int32_t* ds_local, int32_t* ds_tok_end, void* stream) {
  SCOPE_REQUIRE(docs && ds_ptr && ds_local && ds_tok_end, "scope_doc_starts: null pointer");
  SCOPE_REQUIRE(bs > 0 && T > 0 && T % bs == 0, "scope_doc_starts: T=%lld must be a positive multiple of bs=%d",
                (long long)T, bs);
  SCOPE_REQUIRE(T < (1ll << 31), "scope_doc_starts: T=%lld exceeds int32 token indices", (long long)T);
  const int NB = static_cast<int>(T / bs);
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(doc_blocks_kernel, dim3(NB), dim3(256), 0, s, docs, T, bs, ds_tok_end, ds_local);
  int rc = check_launch("doc_blocks_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(doc_scan_kernel, dim3(1), dim3(1024), 0, s, NB, bs, doc_clamp, reset_len, ds_ptr, ds_local,
                     ds_tok_end);
  return check_launch("doc_scan_kernel");
}

int scope_ptr_ref_maxkv(const scope_ptr_ref_params* p) {
  if (!p || p->bs <= 0) return 0;
  const int NB = static_cast<int>(p->T / p->bs);
  const int local = min(max(1, p->local_blocks), NB);
  const int np = p->ptr_half_blocks > 0 ? p->M * (2 * p->ptr_half_blocks + 1) : p->M;
  const int gmax = min(max(p->global_blocks_cfg, 0), NB);
  return local + np + gmax;
}

int scope_pointer_mask_ref(const scope_ptr_ref_params* p, const float* delta_star, const float* budget_logits,
                           const float* gumbel_u, const int32_t* ds_ptr, const int32_t* ds_local, int32_t* kv_num,
                           int32_t* kv_idx, int32_t* radius, int32_t* centre, void* stream) {
  SCOPE_REQUIRE(p && delta_star && budget_logits && ds_ptr && ds_local && kv_num && kv_idx && radius && centre,
                "scope_pointer_mask_ref: null pointer");
  SCOPE_REQUIRE(p->bs > 0 && p->T > 0 && p->T % p->bs == 0, "scope_pointer_mask_ref: T=%lld not a multiple of bs=%d",
                (long long)p->T, p->bs);
  SCOPE_REQUIRE(p->M >= 1 && p->M <= kMaxPeaks, "scope_pointer_mask_ref: M=%d outside [1, %d]", p->M, kMaxPeaks);
  SCOPE_REQUIRE(p->H >= 1, "scope_pointer_mask_ref: H=%d", p->H);
  SCOPE_REQUIRE(p->ptr_half_blocks >= 0 && p->local_blocks >= 1, "scope_pointer_mask_ref: bad local/half blocks");
  SCOPE_REQUIRE(p->gumbel_k == 0 || gumbel_u, "scope_pointer_mask_ref: Gumbel active but no uniforms given");
  SCOPE_REQUIRE(p->T < (1ll << 24), "scope_pointer_mask_ref: T=%lld: token indices must stay exact in fp32",
                (long long)p->T);
  RefLaunch A;
  A.p = *p;
  A.NB = static_cast<int>(p->T / p->bs);
  A.p.local_blocks = min(max(1, p->local_blocks), A.NB);
  A.NP = p->ptr_half_blocks > 0 ? p->M * (2 * p->ptr_half_blocks + 1) : p->M;
  A.gmax = min(max(p->global_blocks_cfg, 0), A.NB);
  A.L = A.p.local_blocks + A.NP + A.gmax;
  A.N = next_pow2(A.L);
  SCOPE_REQUIRE(A.N <= kMaxList, "scope_pointer_mask_ref: list length %d exceeds %d", A.L, kMaxList);
  const int64_t rows = static_cast<int64_t>(p->H) * A.NB;
  const size_t shm = 4 * A.N * sizeof(int) + 4 * 5 * kMaxPeaks * sizeof(float);
  hipLaunchKernelGGL(ptr_ref_kernel, dim3(ceil_div(rows, 4)), dim3(256), shm, as_stream(stream), A, delta_star,
                     budget_logits, gumbel_u, ds_ptr, ds_local, kv_num, kv_idx, radius, centre);
  return check_launch("ptr_ref_kernel");
}

static int block_means_launch(const char* who, const uint16_t* q, const uint16_t* k, int H, int64_t T, int D, int bs,
                              int64_t q_sh, int64_t q_st, int64_t k_sh, int64_t k_st, float* qbar, float* kbar,
                              const int32_t* docs, int32_t* last_change, int32_t* first_change, hipStream_t st) {
  SCOPE_REQUIRE(q && k && qbar && kbar, "%s: null pointer", who);
  SCOPE_REQUIRE(D == 64 || D == 128, "%s: D=%d (supported: 64, 128)", who, D);
  SCOPE_REQUIRE(bs > 0 && T > 0 && T % bs == 0, "%s: T=%lld not a positive multiple of bs=%d", who, (long long)T, bs);
  SCOPE_REQUIRE(q_st % 8 == 0 && k_st % 8 == 0 && q_sh % 8 == 0 && k_sh % 8 == 0,
                "%s: strides must keep 16-byte row alignment", who);
  const int NB = static_cast<int>(T / bs);
  dim3 grid(NB, H);
  if (D == 128)
    hipLaunchKernelGGL(block_means_kernel<128>, grid, dim3(256), 0, st, q, k, bs, q_sh, q_st, k_sh, k_st, NB, qbar,
                       kbar, docs, last_change, first_change);
  else
    hipLaunchKernelGGL(block_means_kernel<64>, grid, dim3(256), 0, st, q, k, bs, q_sh, q_st, k_sh, k_st, NB, qbar,
                       kbar, docs, last_change, first_change);
  return check_launch("block_means_kernel");
}

int scope_block_means(const uint16_t* q, const uint16_t* k, int H, int64_t T, int D, int bs, int64_t q_sh,
                      int64_t q_st, int64_t k_sh, int64_t k_st, float* qbar, float* kbar, void* stream) {
  return block_means_launch("scope_block_means", q, k, H, T, D, bs, q_sh, q_st, k_sh, k_st, qbar, kbar, nullptr,
                            nullptr, nullptr, as_stream(stream));
}

int scope_block_means_docs(const uint16_t* q, const uint16_t* k, const int32_t* docs, int H, int64_t T, int D, int bs,
                           int64_t q_sh, int64_t q_st, int64_t k_sh, int64_t k_st, int doc_clamp, int reset_len,
                           float* qbar, float* kbar, int32_t* ds_ptr, int32_t* ds_local, int32_t* ds_tok_end,
                           void* stream) {
  SCOPE_REQUIRE(docs && ds_ptr && ds_local && ds_tok_end, "scope_block_means_docs: null pointer");
  SCOPE_REQUIRE(T < (1ll << 31), "scope_block_means_docs: T=%lld exceeds int32 token indices", (long long)T);
  hipStream_t st = as_stream(stream);
  // the document-block phase rides on head 0's workgroups; its outputs go
  // where doc_scan_kernel reads them (ds_tok_end, ds_local)
  int rc = block_means_launch("scope_block_means_docs", q, k, H, T, D, bs, q_sh, q_st, k_sh, k_st, qbar, kbar, docs,
                              ds_tok_end, ds_local, st);
  if (rc) return rc;
  hipLaunchKernelGGL(doc_scan_kernel, dim3(1), dim3(1024), 0, st, static_cast<int>(T / bs), bs, doc_clamp, reset_len,
                     ds_ptr, ds_local, ds_tok_end);
  return check_launch("doc_scan_kernel");
}

// compute units of the current device (one persistent workgroup each), per device
static int num_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// number of blocks from which scope_pointer_select computes the logits on MFMA
// (when it has a logits_out buffer to hold them)
constexpr int kLogitsGemmNB = 1024;

int scope_pointer_select(const scope_ptr_score_params* p, const float* qbar, const float* kbar,
                         const float* logits_in, const float* prior, const float* gumbel_u, const int32_t* ds_ptr,
                         const int32_t* ds_local, int32_t* kv_num, int32_t* kv_idx, int32_t* picks,
                         float* logits_out, void* stream) {
  SCOPE_REQUIRE(p && ds_ptr && ds_local && kv_num && kv_idx && picks, "scope_pointer_select: null pointer");
  SCOPE_REQUIRE(logits_in || (qbar && kbar), "scope_pointer_select: need logits_in or qbar/kbar");
  SCOPE_REQUIRE(p->D == 64 || p->D == 128, "scope_pointer_select: D=%d (supported: 64, 128)", p->D);
  SCOPE_REQUIRE(p->budget >= 0 && p->budget <= kMaxBudget, "scope_pointer_select: budget=%d outside [0, %d]",
                p->budget, kMaxBudget);
  SCOPE_REQUIRE(p->window >= 1 && p->n_global >= 0, "scope_pointer_select: window >= 1 and n_global >= 0 required");
  SCOPE_REQUIRE(p->NB >= 1 && p->H >= 1, "scope_pointer_select: bad NB/H");
  SCOPE_REQUIRE(p->noise_mode >= 0 && p->noise_mode <= 2, "scope_pointer_select: noise_mode %d", p->noise_mode);
  SCOPE_REQUIRE(p->noise_mode != 1 || gumbel_u, "scope_pointer_select: noise_mode 1 needs gumbel_u");
  SCOPE_REQUIRE(p->temp > 0.f, "scope_pointer_select: temp must be > 0");
  ScoreLaunch A;
  A.p = *p;
  A.L = min(p->window, p->NB) + p->budget + min(p->n_global, p->NB);
  A.N = next_pow2(A.L);
  SCOPE_REQUIRE(A.N <= 64, "scope_pointer_select: list length %d exceeds 64", A.L);
  dim3 grid(ceil_div(p->NB, kScoreQ), p->H);
  hipStream_t st = as_stream(stream);
  if (!logits_in && logits_out && p->D == 128 && p->NB >= kLogitsGemmNB) {
    // long sequences: the logits on bf16 MFMA (split operands) into logits_out, then the selection reads them
    // one workgroup per CU looping over the tiles
    const int nt = ceil_div(p->NB, kLgTile);
    const int lg_grid = std::max(8, std::min(p->H * (nt * (nt + 1) / 2), num_cus()) / 8 * 8);
    hipLaunchKernelGGL(ptr_logits_kernel, dim3(lg_grid), dim3(1024), 0, st, p->H, p->NB,
                       p->logit_scale, qbar, kbar, prior, prior ? p->prior_head_stride : 0, logits_out);
    logits_in = logits_out;
    qbar = kbar = nullptr;
    prior = nullptr;  // already in the logits
  }
  auto go = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, dim3(kScoreQ * 64), 0, st, A, qbar, kbar, logits_in, prior, gumbel_u, ds_ptr,
                       ds_local, kv_num, kv_idx, picks, logits_out);
  };
  const int kb = p->budget <= 2 ? 2 : p->budget <= 4 ? 4 : p->budget <= 8 ? 8 : 16;
  if (logits_in) {
    if (kb == 2) go(ptr_score_kernel<128, 2, true>);
    else if (kb == 4) go(ptr_score_kernel<128, 4, true>);
    else if (kb == 8) go(ptr_score_kernel<128, 8, true>);
    else go(ptr_score_kernel<128, 16, true>);
  } else if (p->D == 128) {
    if (kb == 2) go(ptr_score_kernel<128, 2>);
    else if (kb == 4) go(ptr_score_kernel<128, 4>);
    else if (kb == 8) go(ptr_score_kernel<128, 8>);
    else go(ptr_score_kernel<128, 16>);
  } else {
    if (kb == 2) go(ptr_score_kernel<64, 2>);
    else if (kb == 4) go(ptr_score_kernel<64, 4>);
    else if (kb == 8) go(ptr_score_kernel<64, 8>);
    else go(ptr_score_kernel<64, 16>);
  }
  return check_launch("ptr_score_kernel");
}


int scope_pointer_pair_bias(const scope_ptr_score_params* p, float soft_temp, const float* qbar, const float* kbar,
                            const float* logits_in, const float* prior, const int32_t* kv_num, const int32_t* kv_idx,
                            const int32_t* picks, float* pair_bias, void* stream) {
  SCOPE_REQUIRE(p && kv_num && kv_idx && picks && pair_bias, "scope_pointer_pair_bias: null pointer");
  SCOPE_REQUIRE(logits_in || (qbar && kbar), "scope_pointer_pair_bias: need logits_in or qbar/kbar");
  SCOPE_REQUIRE(p->D == 64 || p->D == 128, "scope_pointer_pair_bias: D=%d (supported: 64, 128)", p->D);
  SCOPE_REQUIRE(p->budget >= 1 && p->budget <= kMaxBudget, "scope_pointer_pair_bias: budget=%d outside [1, %d]",
                p->budget, kMaxBudget);
  SCOPE_REQUIRE(soft_temp > 0.f, "scope_pointer_pair_bias: soft_temp must be > 0");
  ScoreLaunch A;
  A.p = *p;
  A.L = min(p->window, p->NB) + p->budget + min(p->n_global, p->NB);
  A.N = next_pow2(A.L);
  SCOPE_REQUIRE(A.L <= 64, "scope_pointer_pair_bias: list length %d exceeds 64", A.L);
  dim3 grid(ceil_div(p->NB, 4), p->H);
  if (p->D == 128)
    hipLaunchKernelGGL(pair_bias_kernel<128>, grid, dim3(256), 0, as_stream(stream), A, soft_temp, qbar, kbar,
                       logits_in, prior, kv_num, kv_idx, picks, pair_bias);
  else
    hipLaunchKernelGGL(pair_bias_kernel<64>, grid, dim3(256), 0, as_stream(stream), A, soft_temp, qbar, kbar,
                       logits_in, prior, kv_num, kv_idx, picks, pair_bias);
  return check_launch("pair_bias_kernel");
}

int64_t scope_pointer_bwd_workspace_bytes(const scope_ptr_bwd_params* p) {
  if (!p) return 0;
  return static_cast<int64_t>(p->H) * p->NB * p->maxkv * 4;
}

int scope_pointer_bwd(const scope_ptr_bwd_params* p, const float* qbar, const float* kbar, const int32_t* kv_num,
                      const int32_t* kv_idx, const int32_t* q_off, const int32_t* q_list, const float* pair_bias,
                      const float* dpair_bias, uint16_t* dq, uint16_t* dk, void* workspace, void* stream) {
  SCOPE_REQUIRE(p && qbar && kbar && kv_num && kv_idx && q_off && q_list && pair_bias && dpair_bias && dq && dk &&
                    workspace,
                "scope_pointer_bwd: null pointer");
  SCOPE_REQUIRE(p->D == 64 || p->D == 128, "scope_pointer_bwd: D=%d (supported: 64, 128)", p->D);
  SCOPE_REQUIRE(p->maxkv >= 1 && p->maxkv <= 64, "scope_pointer_bwd: maxkv=%d outside [1, 64]", p->maxkv);
  SCOPE_REQUIRE(p->soft_temp > 0.f && p->bs > 0 && p->NB >= 1 && p->H >= 1, "scope_pointer_bwd: bad parameters");
  SCOPE_REQUIRE(p->bs * p->D % 8 == 0 && p->q_st % 8 == 0 && p->k_st % 8 == 0 && p->q_sh % 8 == 0 && p->k_sh % 8 == 0,
                "scope_pointer_bwd: dq/dk rows must stay 16-byte aligned");
  SCOPE_REQUIRE(((reinterpret_cast<uintptr_t>(dq) | reinterpret_cast<uintptr_t>(dk)) & 15) == 0,
                "scope_pointer_bwd: dq and dk must start on a 16-byte boundary");
  float* dz = static_cast<float*>(workspace);
  hipStream_t s = as_stream(stream);
  dim3 grid(p->NB, p->H);
  hipLaunchKernelGGL(ptr_bwd_q_kernel, grid, dim3(256), 0, s, *p, kbar, kv_num, kv_idx, pair_bias, dpair_bias, dz, dq);
  int rc = check_launch("ptr_bwd_q_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(ptr_bwd_k_kernel, grid, dim3(256), 0, s, *p, qbar, kv_num, kv_idx, q_off, q_list, dz, dk);
  return check_launch("ptr_bwd_k_kernel");
}

}  // extern "C"
