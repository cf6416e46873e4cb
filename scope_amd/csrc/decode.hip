// Single-token attention of the decode loop: the query of position t against
// the KV cache, restricted to the current q-block's listed key blocks, with
// the document-causal mask (keys j <= t of the same document).
//
// Split over the listed blocks: one wavefront per (head, list entry) scores
// the entry's bs keys against the query (q staged in LDS, one key per lane
// and step, fp32 dot products), keeps the entry's running max m, sum l and
// unnormalised P·V row o[D] in a workspace; a second kernel merges the
// entries of each head (max-rescaled sums) into the output row and its LSE.
// Decode work is a few blocks of keys per head and layer: the kernels are
// latency bound, so they favour many small workgroups over MFMA tiles.
#include <math.h>

#include "common.h"

namespace scope {

namespace {
constexpr int kDecD = 128;
constexpr float kDecLog2e = 1.4426950408889634f;
constexpr float kDecLn2 = 0.6931471805599453f;
}  // namespace

// work: [H][maxkv][D + 2] fp32 = o[0..D), m (log2 units), l
__global__ __launch_bounds__(64) void decode_part_kernel(scope_decode_params p, const uint16_t* __restrict__ q,
                                                         const uint16_t* __restrict__ kc,
                                                         const uint16_t* __restrict__ vc,
                                                         const int32_t* __restrict__ kv_num,
                                                         const int32_t* __restrict__ kv_idx,
                                                         const int32_t* __restrict__ docs, float* __restrict__ work,
                                                         const int64_t* __restrict__ t_dev) {
  const int e = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  float* w = work + (static_cast<int64_t>(h) * p.maxkv + e) * (kDecD + 2);
  const int n = kv_num[h];
  // the position: from the parameters, or from device memory (checked here:
  // a position outside the cache gives no mass and an all-zero output)
  const int64_t t = t_dev ? *t_dev : p.t;
  const int64_t k0 = e < n ? static_cast<int64_t>(kv_idx[static_cast<int64_t>(h) * p.maxkv + e]) * p.bs : -1;
  if (k0 < 0 || k0 > t || t < 0 || t >= p.T_cap) {  // unused slot, a block after the query, or no valid position
    if (lane == 0) {
      w[kDecD] = -INFINITY;
      w[kDecD + 1] = 0.f;
    }
    return;
  }
  __shared__ float qs[kDecD];
  __shared__ float ps[256];  // P of the entry's keys (bs <= 256)
  const uint16_t* qh = q + static_cast<int64_t>(h) * p.q_sh;
  qs[2 * lane] = bf16_to_f32(qh[2 * lane]) * p.scale * kDecLog2e;
  qs[2 * lane + 1] = bf16_to_f32(qh[2 * lane + 1]) * p.scale * kDecLog2e;
  __syncthreads();
  const int doc_t = docs[t];
  // scores (log2 units), one key per lane per step
  float m = -INFINITY;
  for (int j0 = 0; j0 < p.bs; j0 += 64) {
    const int64_t j = k0 + j0 + lane;
    float s = -INFINITY;
    if (j <= t && docs[j] == doc_t) {
      const uint4* kr = reinterpret_cast<const uint4*>(kc + static_cast<int64_t>(h) * p.k_sh + j * p.k_st);
      float acc = 0.f;
#pragma unroll 4
      for (int c = 0; c < kDecD / 8; ++c) {
        const uint4 u = kr[c];
        const uint32_t wv[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc = fmaf(__uint_as_float(wv[i] << 16), qs[8 * c + 2 * i], acc);
          acc = fmaf(__uint_as_float(wv[i] & 0xffff0000u), qs[8 * c + 2 * i + 1], acc);
        }
      }
      s = acc;
    }
    ps[j0 + lane] = s;
    m = fmaxf(m, s);
  }
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, kWave));
  float l = 0.f;
  for (int j0 = 0; j0 < p.bs; j0 += 64) {
    const float pv = m == -INFINITY ? 0.f : exp2f(ps[j0 + lane] - m);
    ps[j0 + lane] = pv;
    l += pv;
  }
  for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, kWave);
  __syncthreads();
  // o[d] for d = 2·lane, 2·lane + 1: Σ_j P_j v_j[d] (rows read whole by the wavefront)
  float o0 = 0.f, o1 = 0.f;
  const uint32_t* vr = reinterpret_cast<const uint32_t*>(vc + static_cast<int64_t>(h) * p.v_sh + k0 * p.v_st) + lane;
  const int64_t vst = p.v_st / 2;  // in 32-bit words
  for (int j = 0; j < p.bs; ++j) {
    const float pj = ps[j];
    if (pj != 0.f) {
      const uint32_t u = vr[j * vst];
      o0 = fmaf(pj, __uint_as_float(u << 16), o0);
      o1 = fmaf(pj, __uint_as_float(u & 0xffff0000u), o1);
    }
  }
  w[2 * lane] = o0;
  w[2 * lane + 1] = o1;
  if (lane == 0) {
    w[kDecD] = m;
    w[kDecD + 1] = l;
  }
}

__global__ __launch_bounds__(kDecD) void decode_merge_kernel(scope_decode_params p, const float* __restrict__ work,
                                                             uint16_t* __restrict__ out, float* __restrict__ lse) {
  const int h = blockIdx.x, d = threadIdx.x;
  const float* w = work + static_cast<int64_t>(h) * p.maxkv * (kDecD + 2);
  float M = -INFINITY;
  for (int e = 0; e < p.maxkv; ++e) M = fmaxf(M, w[e * (kDecD + 2) + kDecD]);
  float L = 0.f, O = 0.f;
  if (M != -INFINITY) {
    for (int e = 0; e < p.maxkv; ++e) {
      const float me = w[e * (kDecD + 2) + kDecD];
      if (me == -INFINITY) continue;
      const float sc = exp2f(me - M);
      L += sc * w[e * (kDecD + 2) + kDecD + 1];
      O += sc * w[e * (kDecD + 2) + d];
    }
  }
  out[static_cast<int64_t>(h) * p.o_sh + d] = f32_to_bf16(L > 0.f ? O / L : 0.f);
  if (d == 0 && lse) lse[h] = L > 0.f ? (M + log2f(L)) * kDecLn2 : -INFINITY;
}

}  // namespace scope

using namespace scope;

extern "C" int64_t scope_decode_workspace_bytes(const scope_decode_params* p) {
  if (!p || p->H <= 0 || p->maxkv <= 0) return 0;
  return static_cast<int64_t>(p->H) * p->maxkv * (kDecD + 2) * static_cast<int64_t>(sizeof(float));
}

static int decode_launch(const scope_decode_params* p, const int64_t* t_dev, const uint16_t* q,
                         const uint16_t* k_cache, const uint16_t* v_cache, const int32_t* kv_num,
                         const int32_t* kv_idx, const int32_t* docs, void* workspace, uint16_t* out, float* lse,
                         void* stream, const char* fn) {
  SCOPE_REQUIRE(p && q && k_cache && v_cache && kv_num && kv_idx && docs && workspace && out, "%s: null pointer", fn);
  SCOPE_REQUIRE(p->D == kDecD, "%s: head dim D=%d (supported: 128)", fn, p->D);
  SCOPE_REQUIRE(p->bs == 64 || p->bs == 128 || p->bs == 256, "%s: block size %d (64, 128, 256)", fn, p->bs);
  SCOPE_REQUIRE(p->H >= 1 && p->maxkv >= 1 && p->maxkv <= 65535, "%s: bad H=%d / maxkv=%d", fn, p->H, p->maxkv);
  SCOPE_REQUIRE(t_dev || (p->t >= 0 && p->t < p->T_cap), "%s: position t=%lld outside the cache (%lld tokens)", fn,
                (long long)p->t, (long long)p->T_cap);
  SCOPE_REQUIRE(p->T_cap % p->bs == 0, "%s: cache length %lld not a multiple of bs=%d", fn, (long long)p->T_cap,
                p->bs);
  SCOPE_REQUIRE(p->k_st % 8 == 0 && p->k_sh % 8 == 0 && p->v_st % 2 == 0 && p->v_sh % 2 == 0 &&
                    (reinterpret_cast<uintptr_t>(k_cache) & 15) == 0 && (reinterpret_cast<uintptr_t>(v_cache) & 3) == 0,
                "%s: k rows must be 16-byte aligned and v rows 4-byte aligned", fn);
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(decode_part_kernel, dim3(p->maxkv, p->H), dim3(64), 0, s, *p, q, k_cache, v_cache, kv_num,
                     kv_idx, docs, static_cast<float*>(workspace), t_dev);
  int rc = check_launch("decode_part_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(decode_merge_kernel, dim3(p->H), dim3(kDecD), 0, s, *p, static_cast<const float*>(workspace),
                     out, lse);
  return check_launch("decode_merge_kernel");
}

extern "C" int scope_decode_attn(const scope_decode_params* p, const uint16_t* q, const uint16_t* k_cache,
                                 const uint16_t* v_cache, const int32_t* kv_num, const int32_t* kv_idx,
                                 const int32_t* docs, void* workspace, uint16_t* out, float* lse, void* stream) {
  return decode_launch(p, nullptr, q, k_cache, v_cache, kv_num, kv_idx, docs, workspace, out, lse, stream,
                       "scope_decode_attn");
}

extern "C" int scope_decode_attn_at(const scope_decode_params* p, const int64_t* t_dev, const uint16_t* q,
                                    const uint16_t* k_cache, const uint16_t* v_cache, const int32_t* kv_num,
                                    const int32_t* kv_idx, const int32_t* docs, void* workspace, uint16_t* out,
                                    float* lse, void* stream) {
  SCOPE_REQUIRE(t_dev, "scope_decode_attn_at: null position pointer");
  return decode_launch(p, t_dev, q, k_cache, v_cache, kv_num, kv_idx, docs, workspace, out, lse, stream,
                       "scope_decode_attn_at");
}
