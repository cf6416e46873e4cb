// Kernel 2 (forward): block-sparse flash attention with the SCOPE spectral
// bias, bf16 MFMA on gfx950.  Replaces the FlexAttention forward
// (torch:_inductor/kernel/flex/templates/flex_attention.py.jinja) for the
// pointer BlockMask with mask_mod document_causal (model/attn_bias.py:674-679)
// and the spectral score_mod (scoped_medium.py:425-457).
//
// One workgroup per (head, q-block) of BS rows (BS = block size, 128 or 256),
// one wavefront per 32 query rows.  The workgroup walks only the key blocks of
// its list, staging each BN-row sub-tile of K (row-major) and V (transposed)
// in LDS; the next sub-tile's global loads are in flight while the current
// one is computed.  Scores are kept in the log2 domain (exp2).
//
// Bias modes:
//   0 none
//   1 block offsets: β Σ_k A_k(i) cos(ω_k r) + B_k(i) sin(ω_k r), r = qb - kb,
//     a per-(row, key block) constant folded into the softmax offset
//   2 token offsets (the reference's score_mod): the band term enters as
//     extra MFMA k-steps over 16 features (cos/sin(ω_k j) on the key side,
//     the angle-addition coefficients on the query side), each split into
//     bf16 hi + lo; -b0 is a row constant; slope·Δ and the softplus/relu gate
//     are evaluated per element.
//
// Masking: a sub-tile is unmasked when it ends at or before the wave's first
// row and no document starts between its first key and the block's last
// token; sub-tiles entirely after the wave's rows are skipped; the rest apply
// kv <= q && docs[kv] == docs[q] per element.
#include <math.h>
#include <stdlib.h>

#include "attn_common.h"

namespace scope {

template <int BS, int BN, int MODE>
__global__ __launch_bounds__(2 * BS) void attn_fwd_kernel(AttnArgs a) {
  constexpr int NT = 2 * BS;
  constexpr int D = 128;
  constexpr int KSTR = D + 8;   // bf16 per K row in LDS   (68 dwords: conflict-free b128 reads)
  constexpr int VSTR = BN + 4;  // bf16 per V^T row in LDS (conflict-free b64 reads)
  constexpr int FSTR = 40;      // bf16 per feature row    (20 dwords: conflict-free b128 reads)
  constexpr int NSUB = BS / BN;
  constexpr int MB = BN / 32;
  constexpr int KCH = BN * 16;             // 16-byte K chunks per sub-tile
  constexpr int VBL = BN * 4;              // 4x8 V blocks per sub-tile
  constexpr int KL = (KCH + NT - 1) / NT;  // per thread
  constexpr int VL = (VBL + NT - 1) / NT;
  constexpr int FCH = BN * 4;              // 16-byte feature chunks per sub-tile (token mode)
  constexpr int FL = (FCH + NT - 1) / NT;

  __shared__ __attribute__((aligned(16))) uint16_t Ks[BN * KSTR];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[D * VSTR];
  __shared__ __attribute__((aligned(16))) uint16_t Fs[MODE == 2 ? BN * FSTR : 8];
  __shared__ __attribute__((aligned(16))) int docs_s[BN];

  const int tid = threadIdx.x;
  const int wave = tid / 64, lane = tid % 64, g = lane / 32, lr = lane % 32;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int h = tile / a.QB, qb = tile % a.QB;
  const int64_t q0 = static_cast<int64_t>(qb) * BS;
  const int64_t wrow_lo = q0 + wave * 32;
  const int64_t row = wrow_lo + lr;
  const int64_t hT = static_cast<int64_t>(h) * a.T;

  uint4 qreg[8];
  {
    const uint16_t* qp = a.q + h * a.q_sh + row * a.q_st + g * 8;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qreg[ks] = *reinterpret_cast<const uint4*>(qp + ks * 16);
  }

  // ---- bias set-up (per row)
  float ca[8], sa[8];
  uint4 qf = make_uint4(0, 0, 0, 0), qfl = make_uint4(0, 0, 0, 0);
  float rowc = 0.f, slp = 0.f, dm = 0.f, wd = 0.f, glam = 0.f;
  if (MODE == 1) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      ca[k] = k < a.K ? a.coeff_cos[(hT + row) * a.K + k] * a.beta_log2 : 0.f;
      sa[k] = k < a.K ? a.coeff_sin[(hT + row) * a.K + k] * a.beta_log2 : 0.f;
    }
  }
  if (MODE == 2) {
    token_qfeat(a, hT, row, g, qf, qfl, nullptr, nullptr);
    if (a.subtract_b0) rowc = -a.beta_log2 * a.b0[hT + row];
    if (a.use_slope) slp = a.beta_log2 * a.slope[hT + row];
    if (a.gate_kind != SCOPE_GATE_NONE) {
      dm = a.delta_main[hT + row];
      wd = a.width[hT + row];
      glam = a.beta_log2 * a.ramp_lambda;
    }
  }
  const bool extra = MODE == 2 && (a.use_slope || (a.gate_kind != SCOPE_GATE_NONE && a.ramp_lambda > 0.f));

  const int64_t lrow = static_cast<int64_t>(h) * a.QB + qb;
  const int n = a.kv_num[lrow];
  const int32_t* lst = a.kv_idx + lrow * a.maxkv;
  const int total = n * NSUB;
  const int ds_end = a.ds_tok_end[qb];
  const int doc_row = a.docs[row];

  // ---- global -> register prefetch of one sub-tile
  uint4 kpre[KL];
  uint4 vpre[VL][4];
  int dpre = 0;
  uint4 fpre[FL];
  auto load = [&](int it) {
    const int kb = lst[it / NSUB];
    const int64_t kv0 = static_cast<int64_t>(kb) * BS + (it % NSUB) * BN;
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      const int idx = tid + i * NT;
      const int r = idx / 16, c = idx % 16;
      if (KCH % NT == 0 || idx < KCH)
        kpre[i] = *reinterpret_cast<const uint4*>(a.k + h * a.k_sh + (kv0 + r) * a.k_st + c * 8);
    }
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      const int idx = tid + i * NT;
      const int c = idx % 16, kvg = idx / 16;
      if (VBL % NT == 0 || idx < VBL) {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          vpre[i][rr] = *reinterpret_cast<const uint4*>(a.v + h * a.v_sh + (kv0 + kvg * 4 + rr) * a.v_st + c * 8);
      }
    }
    if (tid < BN) dpre = a.docs[kv0 + tid];
    if (MODE == 2) {
#pragma unroll
      for (int i = 0; i < FL; ++i) {
        const int idx = tid + i * NT;
        if (FCH % NT == 0 || idx < FCH)
          fpre[i] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.table) + (kv0 + idx / 4) * kTokRow +
                                                    (idx % 4) * 8);
      }
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int i = 0; i < KL; ++i) {
      const int idx = tid + i * NT;
      const int r = idx / 16, c = idx % 16;
      if (KCH % NT == 0 || idx < KCH) *reinterpret_cast<uint4*>(&Ks[r * KSTR + c * 8]) = kpre[i];
    }
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      const int idx = tid + i * NT;
      const int c = idx % 16, kvg = idx / 16;
      if (!(VBL % NT == 0 || idx < VBL)) continue;
      const uint32_t w0[4] = {vpre[i][0].x, vpre[i][0].y, vpre[i][0].z, vpre[i][0].w};
      const uint32_t w1[4] = {vpre[i][1].x, vpre[i][1].y, vpre[i][1].z, vpre[i][1].w};
      const uint32_t w2[4] = {vpre[i][2].x, vpre[i][2].y, vpre[i][2].z, vpre[i][2].w};
      const uint32_t w3[4] = {vpre[i][3].x, vpre[i][3].y, vpre[i][3].z, vpre[i][3].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int w = e / 2;
        uint2 val;
        if (e & 1) {
          val.x = pack_hi16(w0[w], w1[w]);
          val.y = pack_hi16(w2[w], w3[w]);
        } else {
          val.x = pack_lo16(w0[w], w1[w]);
          val.y = pack_lo16(w2[w], w3[w]);
        }
        *reinterpret_cast<uint2*>(&Vt[(c * 8 + e) * VSTR + kvg * 4]) = val;
      }
    }
    if (tid < BN) docs_s[tid] = dpre;
    if (MODE == 2) {
#pragma unroll
      for (int i = 0; i < FL; ++i) {
        const int idx = tid + i * NT;
        if (FCH % NT == 0 || idx < FCH) *reinterpret_cast<uint4*>(&Fs[(idx / 4) * FSTR + (idx % 4) * 8]) = fpre[i];
      }
    }
  };

  f32x16_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = zero16();
  float m_run = -INFINITY, l_run = 0.f;
  float bt = 0.f;
  const float cs = a.scale_log2;

  if (total > 0) load(0);
  for (int it = 0; it < total; ++it) {
    __syncthreads();
    store();
    __syncthreads();
    if (it + 1 < total) load(it + 1);

    const int t = it / NSUB, st = it % NSUB;
    const int kb = lst[t];
    const int64_t kv0 = static_cast<int64_t>(kb) * BS + st * BN;
    if (kv0 > wrow_lo + 31) continue;  // every key after every row of this wave
    const bool full = (kv0 + BN - 1 <= wrow_lo) && (ds_end <= kv0);

    if (MODE == 1 && st == 0) {
      const float* tr = static_cast<const float*>(a.table) + static_cast<int64_t>(qb - kb) * 16;
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) acc += ca[k] * tr[k] + sa[k] * tr[8 + k];
      bt = acc;
    }
    const float tconst = MODE == 1 ? bt : rowc;

    // S^T = K Q^T  (+ token features)
    f32x16_t s[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      s[mb] = zero16();
      const uint16_t* kr = &Ks[(mb * 32 + lr) * KSTR + g * 8];
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) s[mb] = mfma32(*reinterpret_cast<const uint4*>(kr + ks * 16), qreg[ks], s[mb]);
      if (MODE == 2) {
        const uint4 fh = *reinterpret_cast<const uint4*>(&Fs[(mb * 32 + lr) * FSTR + g * 8]);
        const uint4 fl = *reinterpret_cast<const uint4*>(&Fs[(mb * 32 + lr) * FSTR + 16 + g * 8]);
        s[mb] = mfma32(fh, qf, s[mb]);
        s[mb] = mfma32(fh, qfl, s[mb]);
        s[mb] = mfma32(fl, qf, s[mb]);
      }
    }

    if (!full) {
      // branch-free: per-element control flow around accumulator updates
      // is both slow and fragile, so read the documents unconditionally and
      // select
      const int lim = static_cast<int>(row - kv0);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
          const int j0 = mb * 32 + 8 * rq + 4 * g;
          const int4 d4 = *reinterpret_cast<const int4*>(&docs_s[j0]);
          const int dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const bool ok = (j0 + i <= lim) & (dv[i] == doc_row);
            s[mb][4 * rq + i] = ok ? s[mb][4 * rq + i] : -INFINITY;
          }
        }
    }
    if (extra) {
      const int dbase = static_cast<int>(row - kv0);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = mb * 32 + 8 * (r / 4) + 4 * g + (r % 4);
          const float df = static_cast<float>(dbase - j);
          float e = slp * df;
          if (a.gate_kind != SCOPE_GATE_NONE) {
            const float x = (fabsf(df - dm) - wd) * a.inv_tau;
            const float gt = a.gate_kind == SCOPE_GATE_SOFTPLUS ? fmaxf(x, 0.f) + log1pf(__expf(-fabsf(x)))
                                                                : fmaxf(x, 0.f);
            e -= glam * gt;
          }
          s[mb][r] = fmaf(s[mb][r], cs, e);
        }
    }

    float mx = -INFINITY;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[mb][r]);
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_t = (extra ? mx : mx * cs) + tconst;
    const float m_new = fmaxf(m_run, m_t);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m_run - m_use);
    const float off = tconst - m_use;

    uint4 pb[2 * MB];
    float psum = 0.f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        float p[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float x = s[mb][hf * 8 + j];
          p[j] = exp2f(extra ? x + off : fmaf(x, cs, off));
          psum += p[j];
        }
        pb[mb * 2 + hf] = make_uint4(cvt_pk_bf16(p[0], p[1]), cvt_pk_bf16(p[2], p[3]), cvt_pk_bf16(p[4], p[5]),
                                     cvt_pk_bf16(p[6], p[7]));
      }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    if (__ballot(alpha != 1.f)) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
    }

    // O^T += V^T P^T
#pragma unroll
    for (int md = 0; md < 4; ++md) {
      const uint16_t* vr = &Vt[(md * 32 + lr) * VSTR + 4 * g];
#pragma unroll
      for (int s2 = 0; s2 < 2 * MB; ++s2) {
        const uint2 lo = *reinterpret_cast<const uint2*>(vr + 16 * s2);
        const uint2 hi = *reinterpret_cast<const uint2*>(vr + 16 * s2 + 8);
        o[md] = mfma32(make_uint4(lo.x, lo.y, hi.x, hi.y), pb[s2], o[md]);
      }
    }
  }

  // ---- epilogue
  const float l_row = l_run + __shfl_xor(l_run, 32, 64);
  const float inv = l_row > 0.f ? 1.f / l_row : 0.f;
  uint16_t* op = a.out + h * a.o_sh + row * a.o_st + 4 * g;
#pragma unroll
  for (int md = 0; md < 4; ++md)
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      uint2 val;
      val.x = cvt_pk_bf16(o[md][4 * rq] * inv, o[md][4 * rq + 1] * inv);
      val.y = cvt_pk_bf16(o[md][4 * rq + 2] * inv, o[md][4 * rq + 3] * inv);
      *reinterpret_cast<uint2*>(op + md * 32 + 8 * rq) = val;
    }
  if (g == 0) a.lse_out[hT + row] = l_row > 0.f ? (m_run + log2f(l_row)) * kLn2 : -INFINITY;
}

template <int BS, int BN>
static void launch_fwd_bn(const AttnArgs& a, int mode, int grid, hipStream_t s) {
  if (mode == SCOPE_BIAS_BLOCK)
    hipLaunchKernelGGL((attn_fwd_kernel<BS, BN, 1>), dim3(grid), dim3(2 * BS), 0, s, a);
  else if (mode == SCOPE_BIAS_TOKEN)
    hipLaunchKernelGGL((attn_fwd_kernel<BS, BN, 2>), dim3(grid), dim3(2 * BS), 0, s, a);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<BS, BN, 0>), dim3(grid), dim3(2 * BS), 0, s, a);
}

// Key sub-tile rows staged per LDS round (64 or 128); SCOPE_FWD_BN overrides
// the default for tuning sweeps.
static int fwd_tile_bn(int bs) {
  static int env = -1;
  if (env < 0) {
    const char* e = getenv("SCOPE_FWD_BN");
    env = e ? atoi(e) : 0;
  }
  if (env == 64 || env == 128) return env;
  return bs == 256 ? 128 : 64;
}

int validate_attn(const scope_attn_params* p, const void* q, const void* k, const void* v, const int32_t* kv_num,
                  const int32_t* kv_idx, const int32_t* docs, const int32_t* ds_tok_end, const void* table,
                  const float* cc, const float* cs, const float* b0, const float* slope, const float* dm,
                  const float* wd, const char* who) {
  SCOPE_REQUIRE(p && q && k && v && kv_num && kv_idx && docs && ds_tok_end, "%s: null pointer", who);
  SCOPE_REQUIRE(p->D == 128, "%s: head dim D=%d (supported: 128)", who, p->D);
  SCOPE_REQUIRE(p->bs == 128 || p->bs == 256, "%s: block size %d (supported: 128, 256)", who, p->bs);
  SCOPE_REQUIRE(p->T > 0 && p->T % p->bs == 0, "%s: T=%lld must be a positive multiple of bs=%d", who,
                (long long)p->T, p->bs);
  SCOPE_REQUIRE(p->T < (1ll << 31), "%s: T=%lld exceeds int32 token indices", who, (long long)p->T);
  SCOPE_REQUIRE(p->H >= 1 && p->maxkv >= 1, "%s: bad H/maxkv", who);
  SCOPE_REQUIRE(p->q_st % 8 == 0 && p->k_st % 8 == 0 && p->v_st % 8 == 0 && p->o_st % 8 == 0 &&
                    p->q_sh % 8 == 0 && p->k_sh % 8 == 0 && p->v_sh % 8 == 0 && p->o_sh % 8 == 0,
                "%s: strides must be multiples of 8 elements (16-byte rows)", who);
  auto al16 = [](const void* x) { return (reinterpret_cast<uintptr_t>(x) & 15) == 0; };
  SCOPE_REQUIRE(al16(q) && al16(k) && al16(v) && al16(docs) && al16(cc) && al16(cs) && al16(b0) && al16(slope) &&
                    al16(dm) && al16(wd) && al16(table),
                "%s: tensors must start on a 16-byte boundary", who);
  SCOPE_REQUIRE(p->bias_mode >= 0 && p->bias_mode <= 2, "%s: bias_mode %d", who, p->bias_mode);
  if (p->bias_mode != SCOPE_BIAS_NONE) {
    SCOPE_REQUIRE(p->K >= 1 && p->K <= 8, "%s: K=%d outside [1, 8]", who, p->K);
    SCOPE_REQUIRE(table && cc && cs, "%s: spectral bias needs table, coeff_cos and coeff_sin", who);
  }
  if (p->bias_mode == SCOPE_BIAS_TOKEN) {
    SCOPE_REQUIRE(!p->subtract_b0 || b0, "%s: subtract_b0 needs b0", who);
    SCOPE_REQUIRE(!p->use_slope || slope, "%s: use_slope needs slope", who);
    SCOPE_REQUIRE(p->gate_kind >= 0 && p->gate_kind <= 2, "%s: gate_kind %d", who, p->gate_kind);
    SCOPE_REQUIRE(p->gate_kind == SCOPE_GATE_NONE || (dm && wd && p->tau > 0.f), "%s: gate needs delta_main, width and tau > 0",
                  who);
  }
  return SCOPE_OK;
}

AttnArgs make_args(const scope_attn_params* p) {
  AttnArgs a = {};
  a.H = p->H;
  a.T = p->T;
  a.QB = static_cast<int>(p->T / p->bs);
  a.maxkv = p->maxkv;
  a.K = p->K;
  a.q_sh = p->q_sh;
  a.q_st = p->q_st;
  a.k_sh = p->k_sh;
  a.k_st = p->k_st;
  a.v_sh = p->v_sh;
  a.v_st = p->v_st;
  a.o_sh = p->o_sh;
  a.o_st = p->o_st;
  a.scale = p->scale;
  a.scale_log2 = p->scale * kLog2e;
  a.beta = p->beta;
  a.beta_log2 = p->beta * kLog2e;
  a.feat_scale = p->scale != 0.f ? p->beta / p->scale : 0.f;
  a.use_slope = p->use_slope;
  a.subtract_b0 = p->subtract_b0;
  a.gate_kind = p->gate_kind;
  a.ramp_lambda = p->ramp_lambda;
  a.inv_tau = p->tau > 0.f ? 1.f / p->tau : 0.f;
  return a;
}

}  // namespace scope

using namespace scope;

extern "C" int scope_attn_fwd(const scope_attn_params* p, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              const int32_t* kv_num, const int32_t* kv_idx, const int32_t* docs,
                              const int32_t* ds_tok_end, const void* table, const float* coeff_cos,
                              const float* coeff_sin, const float* b0, const float* slope, const float* delta_main,
                              const float* width, uint16_t* out, float* lse, void* stream) {
  int rc = validate_attn(p, q, k, v, kv_num, kv_idx, docs, ds_tok_end, table, coeff_cos, coeff_sin, b0, slope,
                         delta_main, width, "scope_attn_fwd");
  if (rc) return rc;
  SCOPE_REQUIRE(out && lse, "scope_attn_fwd: null output");
  AttnArgs a = make_args(p);
  a.q = q;
  a.k = k;
  a.v = v;
  a.kv_num = kv_num;
  a.kv_idx = kv_idx;
  a.docs = docs;
  a.ds_tok_end = ds_tok_end;
  a.table = table;
  a.coeff_cos = coeff_cos;
  a.coeff_sin = coeff_sin;
  a.b0 = b0;
  a.slope = slope;
  a.delta_main = delta_main;
  a.width = width;
  a.out = out;
  a.lse_out = lse;
  const int grid = p->H * a.QB;
  hipStream_t s = as_stream(stream);
  const int bn = fwd_tile_bn(p->bs);
  if (p->bs == 256) {
    if (bn == 64)
      launch_fwd_bn<256, 64>(a, p->bias_mode, grid, s);
    else
      launch_fwd_bn<256, 128>(a, p->bias_mode, grid, s);
  } else {
    if (bn == 128)
      launch_fwd_bn<128, 128>(a, p->bias_mode, grid, s);
    else
      launch_fwd_bn<128, 64>(a, p->bias_mode, grid, s);
  }
  return check_launch("attn_fwd_kernel");
}
