// Single-token attention of the decode loop: the query of position t against
// the KV cache, restricted to the current q-block's listed key blocks, with
// the document-causal mask (keys j <= t of the same document).
//
// Split over the listed blocks: one workgroup per (head, list entry) scores
// the entry's bs keys against the query (fp32 dot products, sixteen lanes per
// key row), keeps the entry's max m, sum l and unnormalised P·V row o[D] in a
// workspace; a second kernel merges the entries of each head (max-rescaled
// sums) into the output row and its LSE.  Decode work is a few blocks of
// keys per head and layer: the kernels are bound by the latency of their
// loads, so each workgroup issues all of its rows' loads at once.
#include <math.h>

#include "common.h"

namespace scope {

namespace {
constexpr int kDecD = 128;
constexpr float kDecLog2e = 1.4426950408889634f;
constexpr float kDecLn2 = 0.6931471805599453f;
}  // namespace

// work: [H][maxkv][D + 2] fp32 = o[0..D), m (log2 units), l
// One 256-thread workgroup per (list entry, head): wavefront w takes keys
// w·BS/4 .. +BS/4 of the entry's block, sixteen lanes per key row (lane l
// holds the 16-byte chunk l % 16, features 8·(l % 16) .. +7, of row l / 16
// of each group of four), so that every load of the wavefront reads four
// whole 256-byte rows.  The K and V chunks of all its rows are loaded first;
// every row read lies in the entry's block, which the cache holds whole
// (k0 <= t < T_cap, T_cap a multiple of BS).
constexpr int kDecWaves = 4;

// The attention layer's glue fused into the decode attention (one token):
// q, k, v of the token from its qkv row [3H, D] (the qkv projection), q and
// k RMS-normed and rotated at position t, v mixed with ve, exactly as
// qkv_glue_kernel forms them; k and v go to cache row t.
struct DecGlue {
  const uint16_t* qkv;
  const uint16_t* ve;  // [H·D] or null
  float va, vb, eps;
  const float* cos_t;
  const float* sin_t;
  int64_t rot_rows, rot_st;
  uint16_t* q_out;  // [H, D] or null
  uint16_t* k_cache;
  uint16_t* v_cache;
};

template <int BS, bool GLUE>
__global__ __launch_bounds__(64 * kDecWaves) void decode_part_kernel(
    scope_decode_params p, const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
    const uint16_t* __restrict__ vc, const int32_t* __restrict__ kv_num, const int32_t* __restrict__ kv_idx,
    const int32_t* __restrict__ docs, float* __restrict__ work, const int64_t* __restrict__ t_dev, DecGlue gl) {
  constexpr int PER = BS / kDecWaves, NIT = PER / 4;  // keys per wavefront, row groups per wavefront
  const int e = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int sub = lane >> 4, ch = lane & 15;
  float* w = work + (static_cast<int64_t>(h) * p.maxkv + e) * (kDecD + 2);
  const int n = kv_num[h];
  // the position: from the parameters, or from device memory (checked here:
  // a position outside the cache gives no mass and an all-zero output)
  const int64_t t = t_dev ? *t_dev : p.t;
  const int64_t k0 = e < n ? static_cast<int64_t>(kv_idx[static_cast<int64_t>(h) * p.maxkv + e]) * BS : -1;
  // GLUE: the token's rotated q (as fp32 of its bf16 values) and its k, v rows
  __shared__ float gq[GLUE ? kDecD : 1], gx[GLUE ? 2 * kDecD : 1], gpart[kDecWaves];
  __shared__ __attribute__((aligned(16))) uint16_t gk[GLUE ? kDecD : 8], gv[GLUE ? kDecD : 8];
  if constexpr (GLUE) {
    const bool pos_ok = t >= 0 && t < p.T_cap && t < gl.rot_rows;  // uniform over the workgroup
    if (pos_ok) {
      const int d = tid & (kDecD - 1), isk = tid >= kDecD;  // threads 0-127: q, 128-255: k
      const float x = bf16_to_f32(gl.qkv[(isk ? p.H + h : h) * kDecD + d]);
      float sq = x * x;
      for (int o = 32; o > 0; o >>= 1) sq += __shfl_xor(sq, o, kWave);
      if (lane == 0) gpart[wave] = sq;
      __syncthreads();
      const float r = 1.f / sqrtf((gpart[2 * isk] + gpart[2 * isk + 1]) / kDecD + gl.eps);
      const float xn = bf16_to_f32(f32_to_bf16(__fmul_rn(x, r)));
      gx[isk * kDecD + d] = xn;
      __syncthreads();
      constexpr int HD = kDecD / 2;
      const float c = gl.cos_t[t * gl.rot_st + (d % HD)], sn = gl.sin_t[t * gl.rot_st + (d % HD)];
      const float y = d < HD ? __fadd_rn(__fmul_rn(xn, c), __fmul_rn(gx[isk * kDecD + d + HD], sn))
                             : __fadd_rn(__fmul_rn(gx[isk * kDecD + d - HD], -sn), __fmul_rn(xn, c));
      const uint16_t yb = f32_to_bf16(y);
      if (isk) {
        gk[d] = yb;
      } else {
        gq[d] = bf16_to_f32(yb);
        if (gl.q_out && e == 0) gl.q_out[static_cast<int64_t>(h) * kDecD + d] = yb;
        const float v = bf16_to_f32(gl.qkv[(2 * p.H + h) * kDecD + d]);
        float vv = bf16_to_f32(f32_to_bf16(__fmul_rn(gl.va, v)));
        if (gl.ve) {
          const float ev = bf16_to_f32(gl.ve[static_cast<int64_t>(h) * kDecD + d]);
          vv = bf16_to_f32(f32_to_bf16(__fadd_rn(vv, bf16_to_f32(f32_to_bf16(__fmul_rn(gl.vb, ev))))));
        }
        gv[d] = f32_to_bf16(vv);
      }
      __syncthreads();
      // cache row t, written once per head (the workgroup whose block holds
      // t takes the new row from LDS, not from the cache)
      if (e == 0 && tid < kDecD) {
        gl.k_cache[h * p.k_sh + t * p.k_st + tid] = gk[tid];
        gl.v_cache[h * p.v_sh + t * p.v_st + tid] = gv[tid];
      }
    } else if (gl.q_out && e == 0 && tid < kDecD) {
      gl.q_out[static_cast<int64_t>(h) * kDecD + tid] = 0;
    }
  }
  if (k0 < 0 || k0 > t || t < 0 || t >= p.T_cap || (GLUE && t >= gl.rot_rows)) {
    // an unused slot, a block after the query, or no valid position
    if (tid == 0) {
      w[kDecD] = -INFINITY;
      w[kDecD + 1] = 0.f;
    }
    return;
  }
  __shared__ float ps[BS];  // scores, then P, of the entry's keys
  __shared__ float red[2][kDecWaves];
  __shared__ float opart[kDecWaves][kDecD];
  const int64_t jw = k0 + wave * PER;  // this wavefront's first key
  const uint16_t* kr = kc + static_cast<int64_t>(h) * p.k_sh + 8 * ch;
  const uint16_t* vr = vc + static_cast<int64_t>(h) * p.v_sh + 8 * ch;
  uint4 ku[NIT], vu[NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int64_t j = jw + 4 * it + sub;
    ku[it] = *reinterpret_cast<const uint4*>(kr + j * p.k_st);
    vu[it] = *reinterpret_cast<const uint4*>(vr + j * p.v_st);
    if (GLUE && j == t) {  // the token's own row: the new k, v
      ku[it] = *reinterpret_cast<const uint4*>(&gk[8 * ch]);
      vu[it] = *reinterpret_cast<const uint4*>(&gv[8 * ch]);
    }
  }
  float qv[8];
  if constexpr (GLUE) {
#pragma unroll
    for (int i = 0; i < 8; ++i) qv[i] = gq[8 * ch + i] * p.scale * kDecLog2e;
  } else {
    const uint4 u = *reinterpret_cast<const uint4*>(q + static_cast<int64_t>(h) * p.q_sh + 8 * ch);
    const uint32_t wq[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qv[2 * i] = __uint_as_float(wq[i] << 16) * p.scale * kDecLog2e;
      qv[2 * i + 1] = __uint_as_float(wq[i] & 0xffff0000u) * p.scale * kDecLog2e;
    }
  }
  const int doc_t = docs[t];
  // scores (log2 units) of the wavefront's keys: partial dot products over
  // each lane's 8 features, summed over the row's sixteen lanes
  float m = -INFINITY;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const int64_t j = jw + 4 * it + sub;
    const uint32_t wk[4] = {ku[it].x, ku[it].y, ku[it].z, ku[it].w};
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      acc = fmaf(__uint_as_float(wk[i] << 16), qv[2 * i], acc);
      acc = fmaf(__uint_as_float(wk[i] & 0xffff0000u), qv[2 * i + 1], acc);
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) acc += __shfl_xor(acc, o, kWave);
    const float sc = (j <= t && docs[min(j, t)] == doc_t) ? acc : -INFINITY;  // docs read up to t only
    if (ch == 0) ps[j - k0] = sc;
    m = fmaxf(m, sc);
  }
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, kWave));
  if (lane == 0) red[0][wave] = m;
  __syncthreads();  // scores and the wavefronts' maxima
  float M = red[0][0];
#pragma unroll
  for (int i = 1; i < kDecWaves; ++i) M = fmaxf(M, red[0][i]);
  float pl = 0.f;
  if (tid < BS) {
    const float pv = M == -INFINITY ? 0.f : exp2f(ps[tid] - M);
    ps[tid] = pv;
    pl = pv;
  }
  for (int o = 32; o > 0; o >>= 1) pl += __shfl_xor(pl, o, kWave);
  if (lane == 0) red[1][wave] = pl;
  __syncthreads();  // P and the wavefronts' sums
  float L = 0.f;
#pragma unroll
  for (int i = 0; i < kDecWaves; ++i) L += red[1][i];
  // o[8·ch .. +7] over the wavefront's keys (a masked key, P = 0, adds nothing
  // whatever its cache row holds), summed over the four rows of each group
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    const float pj = ps[wave * PER + 4 * it + sub];
    const uint32_t wv[4] = {vu[it].x, vu[it].y, vu[it].z, vu[it].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = pj != 0.f ? fmaf(pj, __uint_as_float(wv[i] << 16), o[2 * i]) : o[2 * i];
      o[2 * i + 1] = pj != 0.f ? fmaf(pj, __uint_as_float(wv[i] & 0xffff0000u), o[2 * i + 1]) : o[2 * i + 1];
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    o[i] += __shfl_xor(o[i], 16, kWave);
    o[i] += __shfl_xor(o[i], 32, kWave);
  }
  if (sub == 0)
#pragma unroll
    for (int i = 0; i < 8; ++i) opart[wave][8 * ch + i] = o[i];
  __syncthreads();  // every wavefront's P·V share
  if (tid < kDecD) {
    float acc = opart[0][tid];
#pragma unroll
    for (int i = 1; i < kDecWaves; ++i) acc += opart[i][tid];
    w[tid] = acc;
  }
  if (tid == 0) {
    w[kDecD] = M;
    w[kDecD + 1] = L;
  }
}

// Feature d of one head's merged output from its maxkv partials w
// ([maxkv][D + 2]): (o_d, M, L) with o_d = Σ_e 2^(m_e - M) o_e[d] / L.  The
// entries go in groups of 16 whose loads are all issued before any is used
// (one memory latency per group, not one per entry); a later group rescales
// the running sums to its larger maximum.
__device__ __forceinline__ float3 merge_entries(const float* __restrict__ w, int maxkv, int d) {
  constexpr int U = 16;
  float M = -INFINITY, L = 0.f, O = 0.f;
  for (int e0 = 0; e0 < maxkv; e0 += U) {
    float me[U], le[U], oe[U];
#pragma unroll
    for (int i = 0; i < U; ++i) {
      const int e = min(e0 + i, maxkv - 1);  // in bounds; entries past maxkv are dropped below
      me[i] = e0 + i < maxkv ? w[e * (kDecD + 2) + kDecD] : -INFINITY;
      le[i] = w[e * (kDecD + 2) + kDecD + 1];
      oe[i] = w[e * (kDecD + 2) + d];
    }
    float Mg = M;
#pragma unroll
    for (int i = 0; i < U; ++i) Mg = fmaxf(Mg, me[i]);
    if (Mg == -INFINITY) continue;
    if (M != -INFINITY && Mg != M) {
      const float r = exp2f(M - Mg);
      L *= r;
      O *= r;
    }
    M = Mg;
#pragma unroll
    for (int i = 0; i < U; ++i) {
      if (me[i] == -INFINITY) continue;  // an unused slot (its o is not written)
      const float sc = exp2f(me[i] - M);
      L += sc * le[i];
      O += sc * oe[i];
    }
  }
  return make_float3(L > 0.f ? O / L : 0.f, M, L);
}

__global__ __launch_bounds__(kDecD) void decode_merge_kernel(scope_decode_params p, const float* __restrict__ work,
                                                             uint16_t* __restrict__ out, float* __restrict__ lse) {
  const int h = blockIdx.x, d = threadIdx.x;
  const float3 r = merge_entries(work + static_cast<int64_t>(h) * p.maxkv * (kDecD + 2), p.maxkv, d);
  out[static_cast<int64_t>(h) * p.o_sh + d] = f32_to_bf16(r.x);
  if (d == 0 && lse) lse[h] = r.z > 0.f ? (r.y + log2f(r.z)) * kDecLn2 : -INFINITY;
}

// The attention layer's glue of the decoder for T tokens
// (scoped_medium.py:339-345 with norm :266-267 and Rotary :291-310): q and k
// RMS-normalised over D (fp32, eps given: F.rms_norm's default for bf16
// inputs is the fp32 epsilon of its compute type; rounded to bf16), rotated by the half-truncated rotary tables at
// their positions (y1 = x1·cos + x2·sin, y2 = x1·(-sin) + x2·cos, each
// product and sum rounded to fp32 as separate tensor ops round them, the
// result to bf16), v = a·v + b·ve (each product and the sum rounded to bf16,
// as bf16 tensor arithmetic does; b·ve dropped without ve).  q goes to
// q_out [T, H, D]; k and v go to row pos[t] of the caches (cache_at_pos) or
// to row t.  One 128-thread workgroup per (token, head).
__global__ __launch_bounds__(kDecD) void qkv_glue_kernel(int H, int64_t rows, float eps, float va, float vb,
                                                          const uint16_t* __restrict__ qkv,
                                                          const uint16_t* __restrict__ ve,
                                                          const int64_t* __restrict__ pos,
                                                          const float* __restrict__ cos_t,
                                                          const float* __restrict__ sin_t, int64_t rot_rows,
                                                          int64_t rot_st, uint16_t* __restrict__ q_out,
                                                          uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                          int64_t k_sh, int64_t k_st, int64_t v_sh, int64_t v_st,
                                                          int cache_at_pos) {
  constexpr int D = kDecD, HD = kDecD / 2;
  const int t = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  const int64_t p = pos[t];
  const int64_t w = cache_at_pos ? p : t;  // the k/v row written
  uint16_t* qo = q_out + (static_cast<int64_t>(t) * H + h) * D + d;
  if (p < 0 || p >= rot_rows || w < 0 || w >= rows) {  // uniform over the workgroup: no rotary row / no cache row
    *qo = 0;
    return;
  }
  const uint16_t* row = qkv + static_cast<int64_t>(t) * 3 * H * D;
  const float q = bf16_to_f32(row[h * D + d]);
  const float k = bf16_to_f32(row[(H + h) * D + d]);
  const float v = bf16_to_f32(row[(2 * H + h) * D + d]);
  __shared__ float part[2][2];
  __shared__ float xs[2][D];
  float sq = q * q, sk = k * k;
  for (int o = 32; o > 0; o >>= 1) {
    sq += __shfl_xor(sq, o, kWave);
    sk += __shfl_xor(sk, o, kWave);
  }
  if ((d & 63) == 0) {
    part[d >> 6][0] = sq;
    part[d >> 6][1] = sk;
  }
  __syncthreads();
  const float rq = 1.f / sqrtf((part[0][0] + part[1][0]) / D + eps);
  const float rk = 1.f / sqrtf((part[0][1] + part[1][1]) / D + eps);
  const float qn = bf16_to_f32(f32_to_bf16(__fmul_rn(q, rq)));
  const float kn = bf16_to_f32(f32_to_bf16(__fmul_rn(k, rk)));
  xs[0][d] = qn;
  xs[1][d] = kn;
  __syncthreads();
  const float c = cos_t[p * rot_st + (d % HD)], sn = sin_t[p * rot_st + (d % HD)];
  float yq, yk;
  if (d < HD) {
    yq = __fadd_rn(__fmul_rn(qn, c), __fmul_rn(xs[0][d + HD], sn));
    yk = __fadd_rn(__fmul_rn(kn, c), __fmul_rn(xs[1][d + HD], sn));
  } else {
    yq = __fadd_rn(__fmul_rn(xs[0][d - HD], -sn), __fmul_rn(qn, c));
    yk = __fadd_rn(__fmul_rn(xs[1][d - HD], -sn), __fmul_rn(kn, c));
  }
  *qo = f32_to_bf16(yq);
  kc[h * k_sh + w * k_st + d] = f32_to_bf16(yk);
  float vv = bf16_to_f32(f32_to_bf16(__fmul_rn(va, v)));
  if (ve) {
    const float e = bf16_to_f32(ve[static_cast<int64_t>(t) * H * D + h * D + d]);
    vv = bf16_to_f32(f32_to_bf16(__fadd_rn(vv, bf16_to_f32(f32_to_bf16(__fmul_rn(vb, e))))));
  }
  vc[h * v_sh + w * v_st + d] = f32_to_bf16(vv);
}


// ---------------------------------------------------------------------------
// Row-vector products of the decoder's token step, fused with the ops around
// them (one token: every weight row is read once, the step is bound by the
// weights' bytes and by launches, so each kernel replaces a chain of torch
// ops).  y = epi(W · pre(x)), x [K] bf16, W [N, K] bf16 (row stride ldw):
//   pre: x := bf16(x + addx) when addx is given (the U-net skip, w = 1), that
//        x written to xout by workgroup 0, then with norm bf16(x·r), r =
//        1/sqrt(mean(x²) + eps) (F.rms_norm of a bf16 row);
//   epi: the linear's bf16 output z = bf16(Σ W·x), then
//        kGemvPlain z | kGemvRelu2 bf16(relu(z)²) | kGemvResid bf16(res + z) |
//        kGemvLogit 30·σ(float(z) / 7.5) in fp32.
// Each wavefront takes R rows (1; 2 for N >= 16384, the logit head); lane l holds the input elements
// 8·(l + 64c) .. +7 (c < K/512; at K = 256 lanes 32-63 hold none) and the
// rows' chunks at the same columns.
// ---------------------------------------------------------------------------
constexpr int kGemvWaves = 4;
enum { kGemvPlain = 0, kGemvRelu2 = 1, kGemvResid = 2, kGemvLogit = 3 };

__device__ __forceinline__ void unpack8(const uint4& u, float (&f)[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

template <int K, int EPI, int R>
__global__ __launch_bounds__(64 * kGemvWaves) void gemv_kernel(int N, int64_t ldw, int norm, float eps,
                                                               const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ addx,
                                                               uint16_t* __restrict__ xout,
                                                               const uint16_t* __restrict__ w,
                                                               const uint16_t* __restrict__ res,
                                                               void* __restrict__ out) {
  constexpr int NCH = K / 8, KC = (NCH + 63) / 64;  // 16-byte chunks per row and per lane
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool part = NCH % 64 != 0 && lane >= NCH % 64;  // K = 256: this lane holds no chunk
  // chunk c of this lane in a row starting at p (zero for a lane without
  // one, which reads chunk 0 so that every address stays inside the row)
  auto chunk = [&](const uint16_t* p, int c) __attribute__((always_inline)) {
    const uint4 u = *reinterpret_cast<const uint4*>(p + 8 * (part ? 0 : lane + 64 * c));
    return part ? make_uint4(0, 0, 0, 0) : u;
  };
  const int row0 = (blockIdx.x * kGemvWaves + wave) * R;
  // the weight chunks first, so that their loads are in flight during the prologue
  uint4 wv[R][KC];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = min(row0 + r, N - 1);  // rows past N load row N-1 and write nothing
#pragma unroll
    for (int c = 0; c < KC; ++c)
      wv[r][c] = chunk(w + static_cast<int64_t>(row) * ldw, c);
  }
  float xv[KC][8];
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < KC; ++c) {
    unpack8(chunk(x, c), xv[c]);
    if (addx) {
      float av[8];
      unpack8(chunk(addx, c), av);
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[c][i] = bf16_to_f32(f32_to_bf16(__fadd_rn(xv[c][i], av[i])));
    }
    if (xout && blockIdx.x == 0 && wave == 0 && !part) {
      uint4 o;
      o.x = pack_bf16x2(xv[c][0], xv[c][1]);
      o.y = pack_bf16x2(xv[c][2], xv[c][3]);
      o.z = pack_bf16x2(xv[c][4], xv[c][5]);
      o.w = pack_bf16x2(xv[c][6], xv[c][7]);
      *reinterpret_cast<uint4*>(xout + 8 * (lane + 64 * c)) = o;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) ss = fmaf(xv[c][i], xv[c][i], ss);
  }
  if (norm) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, kWave);
    const float r = 1.f / sqrtf(ss / K + eps);
#pragma unroll
    for (int c = 0; c < KC; ++c)
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[c][i] = bf16_to_f32(f32_to_bf16(__fmul_rn(xv[c][i], r)));
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < KC; ++c) {
      float wf[8];
      unpack8(wv[r][c], wf);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc = fmaf(wf[i], xv[c][i], acc);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, kWave);
    const int row = row0 + r;
    if (lane != 0 || row >= N) continue;
    const float z = bf16_to_f32(f32_to_bf16(acc));
    if constexpr (EPI == kGemvPlain) {
      static_cast<uint16_t*>(out)[row] = f32_to_bf16(z);
    } else if constexpr (EPI == kGemvRelu2) {
      const float hz = fmaxf(z, 0.f);
      static_cast<uint16_t*>(out)[row] = f32_to_bf16(__fmul_rn(hz, hz));
    } else if constexpr (EPI == kGemvResid) {
      static_cast<uint16_t*>(out)[row] = f32_to_bf16(__fadd_rn(bf16_to_f32(res[row]), z));
    } else {
      const float v = __fdiv_rn(z, 7.5f);
      static_cast<float*>(out)[row] = 30.f * (1.f / (1.f + expf(-v)));
    }
  }
}


// The start of a decoder token step at the position *t_dev = t (one
// 256-thread workgroup): tokens[t] = tok, docs[t] = docs[t-1] (0 at t = 0)
// + (tok == eot); x0 = F.rms_norm(embed[tok]) (fp32 with eps, rounded to
// bf16); ve_out[i] = value_embed_i[tok] for the nve tables given.  A token
// outside [0, vocab) or a position outside [0, T_cap) leaves tokens and docs
// as they are and writes zero rows.
constexpr int kPrologueThreads = 256;

__global__ __launch_bounds__(kPrologueThreads) void step_prologue_kernel(
    const int64_t* __restrict__ tok_p, const int64_t* __restrict__ t_dev, int64_t T_cap, int64_t vocab, int dm,
    float eps, int64_t eot, int64_t* __restrict__ tokens, int32_t* __restrict__ docs,
    const uint16_t* __restrict__ embed, const uint16_t* __restrict__ ve0, const uint16_t* __restrict__ ve1,
    const uint16_t* __restrict__ ve2, uint16_t* __restrict__ x0, uint16_t* __restrict__ ve_out) {
  const int tid = threadIdx.x;
  const int64_t tok = *tok_p, t = *t_dev;
  if (tok < 0 || tok >= vocab || t < 0 || t >= T_cap) {  // uniform over the workgroup
    const bool given[3] = {ve0 != nullptr, ve1 != nullptr, ve2 != nullptr};  // rows exist for given tables only
    for (int c = tid; c < dm / 8; c += kPrologueThreads) {
      *reinterpret_cast<uint4*>(x0 + 8 * c) = make_uint4(0, 0, 0, 0);
      for (int i = 0; i < 3; ++i)
        if (given[i]) *reinterpret_cast<uint4*>(ve_out + static_cast<int64_t>(i) * dm + 8 * c) = make_uint4(0, 0, 0, 0);
    }
    return;
  }
  if (tid == 0) {
    tokens[t] = tok;
    docs[t] = (t > 0 ? docs[t - 1] : 0) + (tok == eot ? 1 : 0);
  }
  // dm / 8 chunks of 8 features; thread i takes chunks i, i + 256, ...
  __shared__ float part[kPrologueThreads / kWave];
  const uint16_t* er = embed + tok * dm;
  float ss = 0.f;
  for (int c = tid; c < dm / 8; c += kPrologueThreads) {
    const uint4 u = *reinterpret_cast<const uint4*>(er + 8 * c);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = __uint_as_float(w[i] << 16), b = __uint_as_float(w[i] & 0xffff0000u);
      ss = fmaf(a, a, ss);
      ss = fmaf(b, b, ss);
    }
  }
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, kWave);
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kPrologueThreads / kWave; ++i) tot += part[i];
  const float r = 1.f / sqrtf(tot / dm + eps);
  for (int c = tid; c < dm / 8; c += kPrologueThreads) {
    const uint4 u = *reinterpret_cast<const uint4*>(er + 8 * c);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
    uint4 o;
    uint32_t* ow = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      ow[i] = pack_bf16x2(__fmul_rn(__uint_as_float(w[i] << 16), r), __fmul_rn(__uint_as_float(w[i] & 0xffff0000u), r));
    *reinterpret_cast<uint4*>(x0 + 8 * c) = o;
  }
  const uint16_t* ves[3] = {ve0, ve1, ve2};
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    if (!ves[i]) continue;
    for (int c = tid; c < dm / 8; c += kPrologueThreads)
      *reinterpret_cast<uint4*>(ve_out + static_cast<int64_t>(i) * dm + 8 * c) =
          *reinterpret_cast<const uint4*>(ves[i] + tok * dm + 8 * c);
  }
}


// Greedy choice of the decode loop: the index of the largest of n fp32
// values (the first one on ties, as torch.argmax; NaN values are never
// chosen), one 1024-thread workgroup.
constexpr int kArgmaxThreads = 1024;

__global__ __launch_bounds__(kArgmaxThreads) void argmax_kernel(const float* __restrict__ x, int64_t n,
                                                                int64_t* __restrict__ out) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float best = -INFINITY;
  int64_t bi = n;  // n: none yet
  // sixteen loads in flight per thread, then compared in index order
  constexpr int U = 16;
  for (int64_t i0 = tid; i0 < n; i0 += static_cast<int64_t>(U) * kArgmaxThreads) {
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + static_cast<int64_t>(u) * kArgmaxThreads;
      v[u] = i < n ? x[i] : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + static_cast<int64_t>(u) * kArgmaxThreads;
      if (i < n && (v[u] > best || (bi == n && v[u] == best))) {  // strictly larger; the first of a -inf run
        best = v[u];
        bi = i;
      }
    }
  }
  auto better = [](float v, int64_t i, float bv, int64_t b) { return v > bv || (v == bv && i < b); };
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, kWave);
    const int64_t oi = __shfl_xor(bi, o, kWave);
    if (better(ov, oi, best, bi)) best = ov, bi = oi;
  }
  __shared__ float sv[kArgmaxThreads / kWave];
  __shared__ int64_t si[kArgmaxThreads / kWave];
  if (lane == 0) sv[wave] = best, si[wave] = bi;
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < kArgmaxThreads / kWave; ++w)
      if (better(sv[w], si[w], best, bi)) best = sv[w], bi = si[w];
    *out = bi < n ? bi : 0;  // all NaN: index 0
  }
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
                         void* stream, const char* fn, const DecGlue* glue = nullptr) {
  SCOPE_REQUIRE(p && (q || glue) && k_cache && v_cache && kv_num && kv_idx && docs && workspace && out, "%s: null pointer", fn);
  SCOPE_REQUIRE(p->D == kDecD, "%s: head dim D=%d (supported: 128)", fn, p->D);
  SCOPE_REQUIRE(p->bs == 64 || p->bs == 128 || p->bs == 256, "%s: block size %d (64, 128, 256)", fn, p->bs);
  SCOPE_REQUIRE(p->H >= 1 && p->maxkv >= 1 && p->maxkv <= 65535, "%s: bad H=%d / maxkv=%d", fn, p->H, p->maxkv);
  SCOPE_REQUIRE(t_dev || (p->t >= 0 && p->t < p->T_cap), "%s: position t=%lld outside the cache (%lld tokens)", fn,
                (long long)p->t, (long long)p->T_cap);
  SCOPE_REQUIRE(p->T_cap % p->bs == 0, "%s: cache length %lld not a multiple of bs=%d", fn, (long long)p->T_cap,
                p->bs);
  const auto a16 = [](const void* x) { return (reinterpret_cast<uintptr_t>(x) & 15) == 0; };
  SCOPE_REQUIRE(p->k_st % 8 == 0 && p->k_sh % 8 == 0 && p->v_st % 8 == 0 && p->v_sh % 8 == 0 && p->q_sh % 8 == 0 &&
                    a16(k_cache) && a16(v_cache) && (glue || a16(q)),
                "%s: the rows of q, k and v must be 16-byte aligned", fn);
  hipStream_t s = as_stream(stream);
  const dim3 grid(p->maxkv, p->H), blk(64 * kDecWaves);
  float* ws = static_cast<float*>(workspace);
  if (glue) {
    if (p->bs == 64)
      hipLaunchKernelGGL((decode_part_kernel<64, true>), grid, blk, 0, s, *p, q, k_cache, v_cache, kv_num, kv_idx, docs,
                         ws, t_dev, *glue);
    else if (p->bs == 128)
      hipLaunchKernelGGL((decode_part_kernel<128, true>), grid, blk, 0, s, *p, q, k_cache, v_cache, kv_num, kv_idx,
                         docs, ws, t_dev, *glue);
    else
      hipLaunchKernelGGL((decode_part_kernel<256, true>), grid, blk, 0, s, *p, q, k_cache, v_cache, kv_num, kv_idx,
                         docs, ws, t_dev, *glue);
  } else {
    const DecGlue none{};
    if (p->bs == 64)
      hipLaunchKernelGGL((decode_part_kernel<64, false>), grid, blk, 0, s, *p, q, k_cache, v_cache, kv_num, kv_idx,
                         docs, ws, t_dev, none);
    else if (p->bs == 128)
      hipLaunchKernelGGL((decode_part_kernel<128, false>), grid, blk, 0, s, *p, q, k_cache, v_cache, kv_num, kv_idx,
                         docs, ws, t_dev, none);
    else
      hipLaunchKernelGGL((decode_part_kernel<256, false>), grid, blk, 0, s, *p, q, k_cache, v_cache, kv_num, kv_idx,
                         docs, ws, t_dev, none);
  }
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

extern "C" int scope_decoder_qkv_glue(int T, int H, int D, int64_t rows, float eps, float va, float vb,
                                      const uint16_t* qkv, const uint16_t* ve, const int64_t* pos, const float* cos_t,
                                      const float* sin_t, int64_t rot_rows, int64_t rot_st, uint16_t* q_out,
                                      uint16_t* k_out, uint16_t* v_out, int64_t k_sh, int64_t k_st, int64_t v_sh,
                                      int64_t v_st, int cache_at_pos, void* stream) {
  SCOPE_REQUIRE(qkv && pos && cos_t && sin_t && q_out && k_out && v_out, "scope_decoder_qkv_glue: null pointer");
  SCOPE_REQUIRE(D == kDecD, "scope_decoder_qkv_glue: head dim D=%d (supported: 128)", D);
  SCOPE_REQUIRE(T >= 1 && T <= 2147483647 && H >= 1 && H <= 65535 && rows >= 1 && rot_rows >= 1 && rot_st >= D / 2,
                "scope_decoder_qkv_glue: bad T=%d / H=%d / rows=%lld / rotary table", T, H, (long long)rows);
  hipLaunchKernelGGL(qkv_glue_kernel, dim3(T, H), dim3(kDecD), 0, as_stream(stream), H, rows, eps, va, vb, qkv, ve,
                     pos, cos_t, sin_t, rot_rows, rot_st, q_out, k_out, v_out, k_sh, k_st, v_sh, v_st, cache_at_pos);
  return check_launch("qkv_glue_kernel");
}

template <int K, int R>
static void gemv_launch_r(int epi, dim3 grid, hipStream_t st, int N, int64_t ldw, int norm, float eps,
                          const uint16_t* x, const uint16_t* addx, uint16_t* xout, const uint16_t* w,
                          const uint16_t* res, void* out) {
  const dim3 blk(64 * kGemvWaves);
  if (epi == kGemvPlain)
    hipLaunchKernelGGL((gemv_kernel<K, kGemvPlain, R>), grid, blk, 0, st, N, ldw, norm, eps, x, addx, xout, w, res,
                       out);
  else if (epi == kGemvRelu2)
    hipLaunchKernelGGL((gemv_kernel<K, kGemvRelu2, R>), grid, blk, 0, st, N, ldw, norm, eps, x, addx, xout, w, res,
                       out);
  else if (epi == kGemvResid)
    hipLaunchKernelGGL((gemv_kernel<K, kGemvResid, R>), grid, blk, 0, st, N, ldw, norm, eps, x, addx, xout, w, res,
                       out);
  else
    hipLaunchKernelGGL((gemv_kernel<K, kGemvLogit, R>), grid, blk, 0, st, N, ldw, norm, eps, x, addx, xout, w, res,
                       out);
}

// one row per wavefront (more workgroups in flight), two for the logit head's
// N >= 16384 rows, where the extra workgroups cost more than they hide
template <int K>
static void gemv_launch(int epi, hipStream_t st, int N, int64_t ldw, int norm, float eps, const uint16_t* x,
                        const uint16_t* addx, uint16_t* xout, const uint16_t* w, const uint16_t* res, void* out) {
  if (N >= 16384)
    gemv_launch_r<K, 2>(epi, dim3(ceil_div(N, kGemvWaves * 2)), st, N, ldw, norm, eps, x, addx, xout, w, res, out);
  else
    gemv_launch_r<K, 1>(epi, dim3(ceil_div(N, kGemvWaves)), st, N, ldw, norm, eps, x, addx, xout, w, res, out);
}

extern "C" int scope_decoder_gemv(int N, int K, int64_t ldw, int norm, float eps, int epi, const uint16_t* x,
                                  const uint16_t* addx, uint16_t* xout, const uint16_t* w, const uint16_t* res,
                                  void* out, void* stream) {
  SCOPE_REQUIRE(x && w && out, "scope_decoder_gemv: null pointer");
  SCOPE_REQUIRE(N >= 1 && (K == 256 || K == 512 || K == 1024 || K == 2048 || K == 4096),
                "scope_decoder_gemv: N=%d >= 1 and K in {256, 512, 1024, 2048, 4096} required (K=%d)", N, K);
  SCOPE_REQUIRE(ldw >= K && ldw % 8 == 0, "scope_decoder_gemv: row stride %lld must be >= K and a multiple of 8",
                (long long)ldw);
  SCOPE_REQUIRE(epi >= SCOPE_GEMV_PLAIN && epi <= SCOPE_GEMV_LOGIT, "scope_decoder_gemv: unknown epilogue %d", epi);
  SCOPE_REQUIRE((epi == SCOPE_GEMV_RESID) == (res != nullptr),
                "scope_decoder_gemv: the residual is given exactly with SCOPE_GEMV_RESID");
  SCOPE_REQUIRE(!xout || addx, "scope_decoder_gemv: xout needs addx");
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  SCOPE_REQUIRE(a16(x) && a16(w) && (!addx || a16(addx)) && (!xout || a16(xout)),
                "scope_decoder_gemv: x, w, addx and xout must be 16-byte aligned");
  static_assert(SCOPE_GEMV_PLAIN == kGemvPlain && SCOPE_GEMV_RELU2 == kGemvRelu2 &&
                    SCOPE_GEMV_RESID == kGemvResid && SCOPE_GEMV_LOGIT == kGemvLogit,
                "epilogue codes");
  hipStream_t st = as_stream(stream);
  if (K == 256) gemv_launch<256>(epi, st, N, ldw, norm, eps, x, addx, xout, w, res, out);
  else if (K == 512) gemv_launch<512>(epi, st, N, ldw, norm, eps, x, addx, xout, w, res, out);
  else if (K == 1024) gemv_launch<1024>(epi, st, N, ldw, norm, eps, x, addx, xout, w, res, out);
  else if (K == 2048) gemv_launch<2048>(epi, st, N, ldw, norm, eps, x, addx, xout, w, res, out);
  else gemv_launch<4096>(epi, st, N, ldw, norm, eps, x, addx, xout, w, res, out);
  return check_launch("gemv_kernel");
}

extern "C" int scope_decoder_step_prologue(const int64_t* tok, const int64_t* t_dev, int64_t T_cap, int64_t vocab,
                                           int dm, float eps, int64_t eot, int64_t* tokens, int32_t* docs,
                                           const uint16_t* embed, const uint16_t* ve0, const uint16_t* ve1,
                                           const uint16_t* ve2, uint16_t* x0, uint16_t* ve_out, void* stream) {
  SCOPE_REQUIRE(tok && t_dev && tokens && docs && embed && x0, "scope_decoder_step_prologue: null pointer");
  SCOPE_REQUIRE(!(ve0 || ve1 || ve2) || ve_out, "scope_decoder_step_prologue: value embeddings need ve_out");
  SCOPE_REQUIRE(T_cap >= 1 && vocab >= 1 && dm >= 8 && dm % 8 == 0 && dm <= 65536,
                "scope_decoder_step_prologue: T_cap=%lld, vocab=%lld >= 1 and dm=%d a multiple of 8 required",
                (long long)T_cap, (long long)vocab, dm);
  const auto a16 = [](const void* x) { return (reinterpret_cast<uintptr_t>(x) & 15) == 0; };
  SCOPE_REQUIRE(a16(embed) && a16(x0) && (!ve0 || a16(ve0)) && (!ve1 || a16(ve1)) && (!ve2 || a16(ve2)) &&
                    (!ve_out || a16(ve_out)),
                "scope_decoder_step_prologue: the embedding tables and outputs must be 16-byte aligned");
  hipLaunchKernelGGL(step_prologue_kernel, dim3(1), dim3(kPrologueThreads), 0, as_stream(stream), tok, t_dev, T_cap,
                     vocab, dm, eps, eot, tokens, docs, embed, ve0, ve1, ve2, x0, ve_out);
  return check_launch("step_prologue_kernel");
}

extern "C" int scope_decode_attn_glue_at(const scope_decode_params* p, const int64_t* t_dev, const uint16_t* qkv,
                                         const uint16_t* ve, float va, float vb, float eps, const float* cos_t,
                                         const float* sin_t, int64_t rot_rows, int64_t rot_st, uint16_t* k_cache,
                                         uint16_t* v_cache, const int32_t* kv_num, const int32_t* kv_idx,
                                         const int32_t* docs, void* workspace, uint16_t* out, float* lse,
                                         uint16_t* q_out, void* stream) {
  SCOPE_REQUIRE(t_dev && qkv && cos_t && sin_t, "scope_decode_attn_glue_at: null pointer");
  SCOPE_REQUIRE(p && p->H >= 1 && p->H <= 65535 && rot_rows >= 1 && rot_st >= kDecD / 2,
                "scope_decode_attn_glue_at: bad H or rotary tables");
  DecGlue g{qkv, ve, va, vb, eps, cos_t, sin_t, rot_rows, rot_st, q_out, k_cache, v_cache};
  return decode_launch(p, t_dev, nullptr, k_cache, v_cache, kv_num, kv_idx, docs, workspace, out, lse, stream,
                       "scope_decode_attn_glue_at", &g);
}

extern "C" int scope_argmax_f32(const float* x, int64_t n, int64_t* out, void* stream) {
  SCOPE_REQUIRE(x && out, "scope_argmax_f32: null pointer");
  SCOPE_REQUIRE(n >= 1, "scope_argmax_f32: n=%lld >= 1 required", (long long)n);
  hipLaunchKernelGGL(argmax_kernel, dim3(1), dim3(kArgmaxThreads), 0, as_stream(stream), x, n, out);
  return check_launch("argmax_kernel");
}
