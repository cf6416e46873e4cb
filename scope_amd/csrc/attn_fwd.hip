// Kernel 2 (forward): block-sparse flash attention with the SCOPE spectral
// bias, bf16 MFMA on gfx950.  Replaces the FlexAttention forward
// (torch:_inductor/kernel/flex/templates/flex_attention.py.jinja) for the
// pointer BlockMask with mask_mod document_causal (model/attn_bias.py:674-679)
// and the spectral score_mod (scoped_medium.py:425-457).
//
// One workgroup per (head, q-block) of BS rows (BS = block size, 128 or 256),
// one wavefront per 32 query rows.  The workgroup walks only the key blocks of
// its list in 64-key tiles.  Each tile (K and V rows, document ids, the block
// table row or the key features) is copied straight into LDS by
// global_load_lds, two buffers alternating so that tile j+1 is in flight while
// tile j is computed.  S^T = K·Q^T reads K rows; O^T += V^T·P^T reads V through
// transpose loads (ds_read_b64_tr_b16), so no tile is ever rearranged.  Scores
// are kept in the log2 domain (exp2) and the running maximum is only raised
// when a row's tile maximum exceeds it by more than 2^kLazy.
//
// Bias modes (template MODE):
//   0 none
//   1 block offsets: β Σ_k A_k(i) cos(ω_k r) + B_k(i) sin(ω_k r), r = qb - kb,
//     a per-(row, key block) constant folded into the softmax offset
//   2 token offsets (the reference's score_mod): the band term enters as
//     extra MFMA k-steps over 16 features (cos/sin(ω_k j) on the key side,
//     the angle-addition coefficients on the query side), each split into
//     bf16 hi + lo; -b0 is a row constant; slope·Δ is evaluated per element
//   3 as 2 with the softplus/relu gate on |Δ - Δmain| - width
//
// Masking: a tile is unmasked when it ends at or before the wave's first row
// and no document starts between its first key and the block's last token;
// tiles entirely after the wave's rows are skipped; the rest apply
// kv <= q && docs[kv] == docs[q] per element.
#include <math.h>
#include <stdlib.h>

#include <type_traits>

#include "attn_common.h"

namespace scope {

constexpr float kLazy = 8.f;  // log2 headroom before the running maximum is raised

// per-row state of the forward (one query row per lane pair l, l^32)
struct FwdRow {
  float rowc, slp, dm, wd;
  int row, doc;
};

// Bias and mask terms of one tile's scores in place.  Token modes: on return
// s holds the log2-domain score without the row offset (x·scale·log2e + the
// per-element terms).  Modes 0 and 1 leave the raw q·k (the scale is applied
// inside the exponent's FMA) and only mask.  Masked entries are -inf.
template <int MODE, bool MASK, typename Tile>
__device__ __forceinline__ void fwd_scores(const AttnArgs& a, const Tile& b, const FwdRow& R, int kv0,
                                           int lane, f32x16_t (&s)[2]) {
  constexpr bool TOK = MODE >= 2, GATE = MODE == 3;
  const int g = lane >> 5;
  const float cs = a.scale_log2;
  const float glam = a.beta_log2 * a.ramp_lambda;
  const float spw = a.gate_kind == SCOPE_GATE_SOFTPLUS ? kLn2 : 0.f;
  const int lim = R.row - kv0;  // keys j <= lim are causal
  // slope term slp·(lim - j), j = jc + 4g with jc a constant of the register:
  // fma(-slp, jc, slp·(lim - 4g)) (the integers are exact in fp32)
  const float sbase = GATE ? 0.f : R.slp * static_cast<float>(lim - 4 * g);
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      const int j0 = mb * 32 + 8 * rq + 4 * g;
      int dcv[4] = {0, 0, 0, 0};
      if (MASK) {
        const int4 d4 = *reinterpret_cast<const int4*>(&b.docs[j0]);
        dcv[0] = d4.x, dcv[1] = d4.y, dcv[2] = d4.z, dcv[3] = d4.w;
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 4 * rq + i, j = j0 + i;
        float x;
        if (TOK) {
          const float df = static_cast<float>(lim - j);
          float e = GATE ? R.slp * df : fmaf(-R.slp, static_cast<float>(mb * 32 + 8 * rq + i), sbase);
          if (GATE) {
            // softplus(x) = max(x,0) + ln2·log2(1 + 2^(-|x|·log2 e)); relu drops the second term
            const float xx = (fabsf(df - R.dm) - R.wd) * a.inv_tau;
            const float sp = __builtin_amdgcn_logf(1.f + __builtin_amdgcn_exp2f(-fabsf(xx) * kLog2e));
            e -= glam * fmaf(spw, sp, fmaxf(xx, 0.f));
          }
          x = fmaf(s[mb][r], cs, e);
        } else {
          x = s[mb][r];
        }
        if (MASK) x = mask_score(x, j, lim, dcv[i], R.doc);
        s[mb][r] = x;
      }
    }
}

// What the forward kernel produces: the attention output and its LSE; the
// LSE alone (no P·V); or, given the LSE, the probability mass of every
// listed key block summed over the q-block's rows (no P·V either).
enum FwdKind { kFwdAttn = 0, kFwdLse = 1, kFwdMass = 2 };

// Every mode runs two wavefronts per SIMD at either block size: for bs=128
// the compiler would otherwise take up to 512 registers and run one (the
// token modes then fit in 249-253 registers without spills; two 80.5 KB
// workgroups share a CU).
template <int BS, int MODE, int KIND = kFwdAttn>
__global__ __launch_bounds__(2 * BS) __attribute__((amdgpu_waves_per_eu(2))) void attn_fwd_kernel(
    AttnArgs a) {
  constexpr int NT = 2 * BS;
  constexpr int NW = NT / 64;  // wavefronts
  constexpr int BN = 64;  // keys per staged tile
  constexpr int NSUB = BS / BN;
  constexpr bool TOK = MODE >= 2, GATE = MODE == 3;
  constexpr bool MASS = KIND == kFwdMass, PV = KIND == kFwdAttn;
  // bs=256 attention: wavefronts 4-7 run half a tile behind wavefronts 0-3
  // (see the loop below), which needs a third tile buffer
  constexpr bool STAGGER = PV && BS == 256;

  using Tile = KvTile<MODE, PV>;  // the LSE and mass kinds stage no V rows
  __shared__ Tile buf0, buf1;
  __shared__ typename std::conditional<STAGGER, Tile, int>::type buf2;
  // key-block indices of the list (< 65536, checked on the host): 16 bits keep the
  // bs=128 workgroup under half of the CU's LDS, two workgroups per CU
  __shared__ uint16_t kbs[kListLds];
  __shared__ float kbias[kListLds];  // pair bias per list entry (log2 units), when given
  // mass: per list entry and wavefront, the wavefront's share (each slot has one writer)
  __shared__ float mslot[MASS ? kListLds * NW : 1];
  // block mode: β·log2e-scaled coefficient rows of the block's queries, [BS][16] (cos 0..7, sin 8..15)
  __shared__ __attribute__((aligned(16))) float coef[MODE == 1 ? BS * 16 : 4];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid % 64, g = lane / 32, lr = lane % 32;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int h = tile / a.QB, qb = tile % a.QB;
  const int64_t q0 = static_cast<int64_t>(qb) * BS;
  const int wrow_lo = static_cast<int>(q0) + wave * 32;
  const int64_t hT = static_cast<int64_t>(h) * a.T;
  FwdRow R;
  R.row = wrow_lo + lr;

  const int64_t lrow = static_cast<int64_t>(h) * a.QB + qb;
  const int n = min(a.kv_num[lrow], a.maxkv);  // maxkv <= kListLds
  const int32_t* lst = a.kv_idx + lrow * a.maxkv;
  for (int t = tid; t < min(n, kListLds); t += NT) kbs[t] = lst[t];
  const bool pbias = a.pair_bias != nullptr;
  if (pbias)
    for (int t = tid; t < min(n, kListLds); t += NT) kbias[t] = a.pair_bias[lrow * a.maxkv + t] * kLog2e;
  if (MASS)
    for (int t = tid; t < n * NW; t += NT) mslot[t] = 0.f;  // n <= kListLds (checked on the host)

  const TileOffs to = tile_offs(lane);
  uint4 qreg[8];
  {
    const uint16_t* qp = a.q + h * a.q_sh + R.row * a.q_st + g * 8;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) qreg[ks] = *reinterpret_cast<const uint4*>(qp + ks * 16);
  }

  // ---- bias set-up (per row)
  uint4 qf = make_uint4(0, 0, 0, 0), qfl = make_uint4(0, 0, 0, 0);
  R.rowc = R.slp = R.dm = R.wd = 0.f;
  if (MODE == 1) {
    // lane pair (l, l^32) fills the cos (g = 0) or sin (g = 1) half of its row
    const float* cf = (g == 0 ? a.coeff_cos : a.coeff_sin) + (hT + R.row) * a.K;
    const int cr = wave * 32 + lr;
#pragma unroll
    for (int k = 0; k < 8; ++k) coef[row16_off(cr, 2 * g + k / 4) + k % 4] = k < a.K ? cf[k] * a.beta_log2 : 0.f;
  }
  if (TOK) {
    token_qfeat(a, hT, R.row, g, qf, qfl, nullptr, nullptr);
    if (a.subtract_b0) R.rowc = -a.beta_log2 * a.b0[hT + R.row];
    if (a.use_slope) R.slp = a.beta_log2 * a.slope[hT + R.row];
    if (GATE) {
      R.dm = a.delta_main[hT + R.row];
      R.wd = a.width[hT + R.row];
    }
  }
  const int ds_end = a.ds_tok_end[qb];
  R.doc = a.docs[R.row];

  f32x16_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = zero16();
  float m_run = -INFINITY, l_run = 0.f;
  // mass: this lane's probability sum over the tiles of list entry pent,
  // folded into the entry's slot (one wavefront reduction) when the entry changes
  float pacc = 0.f;
  int pent = -1;
  auto mass_flush = [&]() __attribute__((always_inline)) {
    if (pent < 0) return;
#pragma unroll
    for (int o2 = 32; o2 > 0; o2 >>= 1) pacc += __shfl_xor(pacc, o2, 64);
    if (lane == 0) mslot[pent * NW + wave] += pacc;
    pacc = 0.f;
  };
  float lse2 = 0.f;  // mass: the row's LSE in log2 units
  if (MASS) lse2 = a.lse[hT + R.row] * kLog2e;
  float bt = 0.f;  // block mode: β·bias of the current key block (log2 units)
  float eb = 0.f;  // pair bias of the current key block (log2 units)

  // flat iteration index it = list entry · NSUB + key tile; tiles that start
  // after the block's last row are skipped
  const int total = n * NSUB;
  const int qmax = static_cast<int>(q0) + BS - 1;
  // the list lives in LDS (width <= kListLds, checked on the host): a read that
  // could also reach global memory would be a flat load, whose wait also waits
  // for the tile copies in flight
  auto kb_at = [&](int t) __attribute__((always_inline)) { return kbs[t]; };
  auto next_valid = [&](int it) __attribute__((always_inline)) {
    while (it < total && kb_at(it / NSUB) * BS + (it % NSUB) * BN > qmax) ++it;
    return it;
  };
  auto issue = [&](int it, Tile& b) __attribute__((always_inline)) {
    const int kb = kb_at(it / NSUB);
    const int rd = min(max(qb - kb, 0), a.QB - 1);
    kv_issue<MODE, NT, PV>(a, h, static_cast<int64_t>(kb) * BS + (it % NSUB) * BN, rd, b, tid);
  };
  // probabilities of one 32-key half mb of a tile's scores into pb[2mb], pb[2mb + 1]
  auto probs_half = [&](const f32x16_t& sm, int mb, float csm, float off, uint4 (&pb)[4], float& psum)
                        __attribute__((always_inline)) {
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      float p[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        p[j] = __builtin_amdgcn_exp2f(fmaf(sm[hf * 8 + j], csm, off));
        psum += p[j];
      }
      pb[mb * 2 + hf] = make_uint4(cvt_pk_bf16(p[0], p[1]), cvt_pk_bf16(p[2], p[3]), cvt_pk_bf16(p[4], p[5]),
                                   cvt_pk_bf16(p[6], p[7]));
    }
  };
  // a tile cut between its two halves of probabilities (run_a with SPLIT):
  // the second half's scores, its exponent offset and the partial row sum
  f32x16_t sp_s1 = zero16();
  float sp_off = 0.f, sp_csm = 0.f, sp_psum = 0.f;
  // one tile in two parts: scores and probabilities (P^T as bf16 B operands
  // in pb; false when the wavefront has nothing to do), then O^T += V^T P^T.
  // With SPLIT the probabilities of the second 32-key half are left to run_a_rest.
  auto run_a = [&](int it, const Tile& b, uint4 (&pb)[4], auto split) __attribute__((always_inline)) -> bool {
    constexpr bool SPLIT = decltype(split)::value;
    const int kv0 = kb_at(it / NSUB) * BS + (it % NSUB) * BN;
    if (kv0 > wrow_lo + 31) return false;  // every key follows this wavefront's rows
    const bool full = (kv0 + BN - 1 <= wrow_lo) && (ds_end <= kv0);
    if (MODE == 1 && it % NSUB == 0) {
      // block term of this key block (a key block's first tile is never skipped)
      const float4* tr = reinterpret_cast<const float4*>(b.tab);
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 c4 = *reinterpret_cast<const float4*>(coef + row16_off(wave * 32 + lr, i)), t4 = tr[i];
        acc += c4.x * t4.x + c4.y * t4.y + c4.z * t4.z + c4.w * t4.w;
      }
      bt = acc;
    }
    if (it % NSUB == 0) eb = pbias ? kbias[it / NSUB] : 0.f;  // per key block (its first tile is never skipped)
    const float tconst = (MODE == 1 ? bt : R.rowc) + eb;
    // S^T = K Q^T (+ token features): keys in two 32-row blocks, this lane's row as the column
    f32x16_t s[2];
    s[0] = zero16();
    s[1] = zero16();
    {
      // operands of step st = 2·ks + mb read RA steps ahead into a ring
      constexpr int RA = 2;
      uint4 ka[RA + 1];
#pragma unroll
      for (int i = 0; i < RA; ++i) ka[i] = lds_row8_o(b.k, to, (i % 2) * 32, i / 2);
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const int ks = st / 2, mb = st % 2;
        if (st + RA < 16) ka[(st + RA) % (RA + 1)] = lds_row8_o(b.k, to, ((st + RA) % 2) * 32, (st + RA) / 2);
        s[mb] = mfma32(ka[st % (RA + 1)], qreg[ks], s[mb]);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (TOK) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        const uint4 fh = lds_row8_32(b.f, mb * 32 + lr, g * 8);
        const uint4 fl = lds_row8_32(b.f, mb * 32 + lr, 16 + g * 8);
        s[mb] = mfma32(fh, qf, s[mb]);
        s[mb] = mfma32(fh, qfl, s[mb]);
        s[mb] = mfma32(fl, qf, s[mb]);
      }
    }
    // token modes add their per-element terms on every tile, the mask only where it is needed
    if (!full) fwd_scores<MODE, true>(a, b, R, kv0, lane, s);
    else if (TOK) fwd_scores<MODE, false>(a, b, R, kv0, lane, s);
    // exponent = s·csm + off: modes 0/1 keep raw scores (csm = scale·log2e > 0)
    const float csm = TOK ? 1.f : a.scale_log2;
    if (MASS) {
      // P = 2^(s·csm + tconst - lse2); a row without visible keys (lse = -inf) has none
      const float off = lse2 == -INFINITY ? -INFINITY : tconst - lse2;
      float ps = 0.f;
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) ps += __builtin_amdgcn_exp2f(fmaf(s[mb][r], csm, off));
      if (it / NSUB != pent) {  // the tiles of a list entry come in a row (it / NSUB is uniform)
        mass_flush();
        pent = it / NSUB;
      }
      pacc += ps;
      return false;
    }

    // online softmax (log2 domain); the running maximum moves only by more than kLazy
    float mx = -INFINITY;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[mb][r]);
    mx = fmaxf(mx, xor32(mx));
    const float m_t = mx * csm + tconst;
    const bool raise = m_t > m_run + kLazy;
    if (__ballot(raise)) {
      // rows that do not raise keep alpha = 1 (their m_run may still be -inf,
      // where exp2(m_run - m_run) would be NaN); raised rows from -inf get 0
      const float alpha = raise ? __builtin_amdgcn_exp2f(m_run - m_t) : 1.f;
      l_run *= alpha;
      if (PV) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[i][r] *= alpha;
      }
      m_run = raise ? m_t : m_run;
    }
    const float off = m_run == -INFINITY ? -INFINITY : tconst - m_run;

    float psum = 0.f;
    probs_half(s[0], 0, csm, off, pb, psum);
    if constexpr (SPLIT) {
      sp_s1 = s[1];
      sp_off = off;
      sp_csm = csm;
      sp_psum = psum;
      return PV;
    }
    probs_half(s[1], 1, csm, off, pb, psum);
    l_run += psum;
    return PV;
  };
  // the second half of a tile that run_a left with SPLIT
  auto run_a_rest = [&](uint4 (&pb)[4]) __attribute__((always_inline)) {
    float psum = sp_psum;
    probs_half(sp_s1, 1, sp_csm, sp_off, pb, psum);
    l_run += psum;
  };
  using NoSplit = std::integral_constant<bool, false>;
  using Split = std::integral_constant<bool, true>;
  auto run_b = [&](const Tile& b, const uint4 (&pb)[4]) __attribute__((always_inline)) {
#pragma unroll
    for (int s2 = 0; s2 < 4; ++s2)
#pragma unroll
      for (int md = 0; md < 4; ++md) o[md] = mfma32(lds_kmajor_o(b.v, to, 16 * s2, md), pb[s2], o[md]);
  };
  auto run = [&](int it, const Tile& b) __attribute__((always_inline)) {
    uint4 pb[4];
    if (run_a(it, b, pb, NoSplit{})) run_b(b, pb);
  };

  __syncthreads();  // kbs
  if constexpr (STAGGER) {
    // Wavefronts 0-3 (one per SIMD) process whole tiles; wavefronts 4-7 run
    // half a tile behind them: their k-th barrier falls between the scores
    // and the P·V of tile k-1.  Each SIMD then holds one wavefront in its
    // score/softmax phase while the other runs MFMAs, instead of both in
    // the same phase.  The leading group alone copies the tiles (256
    // threads), into three rotating buffers: at its k-th barrier the lagging
    // group is done with tile k-2, whose buffer then takes tile k+1.  Both
    // groups pass n+1 barriers for n tiles.
    const int tid4 = tid & 255;
    auto issue4 = [&](int it, Tile& b) __attribute__((always_inline)) {
      const int kb = kb_at(it / NSUB);
      const int rd = min(max(qb - kb, 0), a.QB - 1);
      kv_issue<MODE, 256, PV>(a, h, static_cast<int64_t>(kb) * BS + (it % NSUB) * BN, rd, b, tid4);
    };
    if (wave < 4) {
      int cur = next_valid(0);
      if (cur < total) issue4(cur, buf0);
      auto lead = [&](Tile& bc, Tile& bn) __attribute__((always_inline)) {
        wait_vm0();
        __syncthreads();  // tile cur is in bc for everyone; the lagging group is done with bn
        const int nxt = next_valid(cur + 1);
        if (nxt < total) issue4(nxt, bn);
        run(cur, bc);
        cur = nxt;
      };
      while (cur < total) {
        lead(buf0, buf1);
        if (cur >= total) break;
        lead(buf1, buf2);
        if (cur >= total) break;
        lead(buf2, buf0);
      }
      __syncthreads();  // matches the lagging group's last barrier
    } else {
      // The lagging group's barrier falls between the two halves of a tile's
      // probabilities: after the leading group's k-th barrier it finishes the
      // probabilities of tile k-1 (VALU) while the leading group runs the
      // scores of tile k (MFMA), runs P·V of tile k-1 and the scores of tile
      // k (MFMA) under the leading group's probabilities, and starts the
      // probabilities of tile k (VALU) under the leading group's P·V.
      __syncthreads();  // tile 0 is in buf0
      int cur = next_valid(0);
      uint4 pb[4];
      bool act = cur < total && run_a(cur, buf0, pb, Split{});
      auto lag = [&](const Tile& bc, const Tile& bn) __attribute__((always_inline)) {
        __syncthreads();  // the leading group starts the tile after cur
        if (act) {
          run_a_rest(pb);
          run_b(bc, pb);
        }
        cur = next_valid(cur + 1);
        act = cur < total && run_a(cur, bn, pb, Split{});
      };
      while (cur < total) {
        lag(buf0, buf1);
        if (cur >= total) break;
        lag(buf1, buf2);
        if (cur >= total) break;
        lag(buf2, buf0);
      }
    }
  } else {
    int cur = next_valid(0);
    if (cur < total) issue(cur, buf0);
    while (cur < total) {
      wait_vm0();
      __syncthreads();  // tile cur is in buf0; every wavefront is done with buf1
      int nxt = next_valid(cur + 1);
      if (nxt < total) issue(nxt, buf1);
      run(cur, buf0);
      cur = nxt;
      if (cur >= total) break;
      wait_vm0();
      __syncthreads();
      nxt = next_valid(cur + 1);
      if (nxt < total) issue(nxt, buf0);
      run(cur, buf1);
      cur = nxt;
    }
  }

  // ---- epilogue
  if (MASS) {
    mass_flush();
    __syncthreads();  // every wavefront's shares are in mslot
    float* mrow = a.mass + lrow * a.QB;
    for (int e = tid; e < n; e += NT) {
      float m = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) m += mslot[e * NW + w];
      mrow[kbs[e]] = m;
    }
    return;
  }
  const float l_row = l_run + xor32(l_run);
  const float inv = l_row > 0.f ? 1.f / l_row : 0.f;
  if (PV) {
    uint16_t* op = a.out + h * a.o_sh + R.row * a.o_st + 4 * g;
#pragma unroll
    for (int md = 0; md < 4; ++md)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        uint2 val;
        val.x = cvt_pk_bf16(o[md][4 * rq] * inv, o[md][4 * rq + 1] * inv);
        val.y = cvt_pk_bf16(o[md][4 * rq + 2] * inv, o[md][4 * rq + 3] * inv);
        *reinterpret_cast<uint2*>(op + md * 32 + 8 * rq) = val;
      }
  }
  if (g == 0) a.lse_out[hT + R.row] = l_row > 0.f ? (m_run + log2f(l_row)) * kLn2 : -INFINITY;
}

template <int BS, int KIND = kFwdAttn>
static void launch_fwd(const AttnArgs& a, int mode, int grid, hipStream_t s) {
  const bool gate = a.gate_kind != SCOPE_GATE_NONE && a.ramp_lambda > 0.f;
  if (mode == SCOPE_BIAS_BLOCK)
    hipLaunchKernelGGL((attn_fwd_kernel<BS, 1, KIND>), dim3(grid), dim3(2 * BS), 0, s, a);
  else if (mode == SCOPE_BIAS_TOKEN && gate)
    hipLaunchKernelGGL((attn_fwd_kernel<BS, 3, KIND>), dim3(grid), dim3(2 * BS), 0, s, a);
  else if (mode == SCOPE_BIAS_TOKEN)
    hipLaunchKernelGGL((attn_fwd_kernel<BS, 2, KIND>), dim3(grid), dim3(2 * BS), 0, s, a);
  else
    hipLaunchKernelGGL((attn_fwd_kernel<BS, 0, KIND>), dim3(grid), dim3(2 * BS), 0, s, a);
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
  SCOPE_REQUIRE(p->maxkv <= kListLds, "%s: MAXKV=%d above %d listed blocks per q-block", who, p->maxkv, kListLds);
  SCOPE_REQUIRE(p->q_st % 8 == 0 && p->k_st % 8 == 0 && p->v_st % 8 == 0 && p->o_st % 8 == 0 &&
                    p->q_sh % 8 == 0 && p->k_sh % 8 == 0 && p->v_sh % 8 == 0 && p->o_sh % 8 == 0,
                "%s: strides must be multiples of 8 elements (16-byte rows)", who);
  // tile copies address a 64-row tile with 32-bit byte offsets from its first row
  SCOPE_REQUIRE(p->q_st < (1 << 24) && p->k_st < (1 << 24) && p->v_st < (1 << 24) && p->o_st < (1 << 24),
                "%s: token strides must be below 2^24 elements", who);
  auto al16 = [](const void* x) { return (reinterpret_cast<uintptr_t>(x) & 15) == 0; };
  SCOPE_REQUIRE(al16(q) && al16(k) && al16(v) && al16(docs) && al16(cc) && al16(cs) && al16(b0) && al16(slope) &&
                    al16(dm) && al16(wd) && al16(table),
                "%s: tensors must start on a 16-byte boundary", who);
  SCOPE_REQUIRE(p->scale > 0.f && p->scale < 1e30f, "%s: scale must be positive and finite (got %g)", who,
                static_cast<double>(p->scale));
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
  a.pair_bias = p->pair_bias;
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
  SCOPE_REQUIRE(p->T / p->bs <= 65536, "scope_attn_fwd: %lld key blocks (at most 65536)",
                (long long)(p->T / p->bs));
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
  if (p->bs == 256)
    launch_fwd<256>(a, p->bias_mode, grid, s);
  else
    launch_fwd<128>(a, p->bias_mode, grid, s);
  return check_launch("attn_fwd_kernel");
}

extern "C" int scope_attn_block_mass(const scope_attn_params* p, const uint16_t* q, const uint16_t* k,
                                     const int32_t* kv_num, const int32_t* kv_idx, const int32_t* docs,
                                     const int32_t* ds_tok_end, const void* table, const float* coeff_cos,
                                     const float* coeff_sin, const float* b0, const float* slope,
                                     const float* delta_main, const float* width, float* lse, float* mass,
                                     void* stream) {
  int rc = validate_attn(p, q, k, k, kv_num, kv_idx, docs, ds_tok_end, table, coeff_cos, coeff_sin, b0, slope,
                         delta_main, width, "scope_attn_block_mass");
  if (rc) return rc;
  SCOPE_REQUIRE(lse && mass, "scope_attn_block_mass: null output");
  SCOPE_REQUIRE(p->T / p->bs <= 65536, "scope_attn_block_mass: %lld key blocks (at most 65536)",
                (long long)(p->T / p->bs));
  SCOPE_REQUIRE(p->maxkv <= kListLds, "scope_attn_block_mass: MAXKV=%d above %d listed blocks per q-block",
                p->maxkv, kListLds);
  AttnArgs a = make_args(p);
  a.q = q;
  a.k = k;
  a.v = k;  // staged with the keys but never read
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
  a.lse_out = lse;
  a.lse = lse;
  a.mass = mass;
  const int grid = p->H * a.QB;
  hipStream_t s = as_stream(stream);
  // pass 1: the LSE of every row; pass 2: the block masses from it
  if (p->bs == 256)
    launch_fwd<256, kFwdLse>(a, p->bias_mode, grid, s);
  else
    launch_fwd<128, kFwdLse>(a, p->bias_mode, grid, s);
  rc = check_launch("attn_fwd_kernel (lse)");
  if (rc) return rc;
  if (p->bs == 256)
    launch_fwd<256, kFwdMass>(a, p->bias_mode, grid, s);
  else
    launch_fwd<128, kFwdMass>(a, p->bias_mode, grid, s);
  return check_launch("attn_fwd_kernel (mass)");
}
