// Kernel 2 (backward): gradients of the block-sparse attention with the
// SCOPE spectral bias, bf16 MFMA on gfx950.  Replaces the FlexAttention
// backward (torch:_inductor/kernel/flex/templates/flex_backwards.py.jinja;
// eager semantics torch:_higher_order_ops/flex_attention.py:826-975),
// including the gradients of the score_mod's captured coefficient tensors.
//
//   dS = P ∘ (dP - Δ),  P = exp(s - lse),  dP = dO·V^T,  Δ = rowsum(dO ∘ O)
//   dQ = scale·dS·K,  dK = scale·dS^T·Q,  dV = P^T·dO
//
// Pass A (q-major, one workgroup per (head, q-block), like the forward):
//   Δ, dQ, and the bias gradients: block mode dA_k = β Σ_tiles cos(ω_k r)·Σ_j dS,
//   token mode through extra MFMAs over the key features (bf16 hi + lo)
//   (C_k = Σ_j dS cos ω_k j, S_k = Σ_j dS sin ω_k j), slope / b0 / gate per element.
// Pass A also stores, for the modes without token offsets, each row's
// softmax offset for every listed key block (block term + pair bias - lse, log2
// units), and in the token modes each row's offset without the pair bias
// (-β·b0 - lse) and β·slope: pass B copies those of a query tile into LDS
// with the tile instead of recomputing them in every wavefront.
// Plan: per key block, its q-list is cut into chunks of 32 or 64 q-blocks.
// Pass B (kv-major, one workgroup per (head, 128 keys of a key block, chunk)):
//   dK, dV over the q-list; a block with one chunk writes bf16 directly,
//   longer lists write fp32 partials that a reduce kernel sums in chunk order
//   (deterministic, no floating-point atomics).  Every mode but the gated
//   token mode runs 16 keys per wavefront on v_mfma_f32_16x16x32_bf16, eight
//   wavefronts in two staggered groups (attn_bwd_dkv16_kernel); the gated
//   token mode runs 32 keys per wavefront on the 32x32x16 form, four
//   wavefronts (attn_bwd_dkv_kernel).
#include <math.h>

#include <algorithm>

#include "attn_common.h"

namespace scope {

// q-blocks per dK/dV work item: q-lists of up to one chunk (the window, the
// pointer picks and the global blocks of documents up to a chunk of blocks
// long) are one item and write bf16 directly; only longer lists pay for fp32
// partials and their reduce.  32 q-blocks keep the items short where a head
// has few blocks; from 2048 blocks per head, 64 halve the partials and their
// reduce for the global blocks that every q-block of a long document lists.
constexpr int kChunkMax = 64;
__host__ __device__ __forceinline__ int bwd_chunk(int QB) { return QB >= 2048 ? 64 : 32; }

// ---------------------------------------------------------------------------
// pass A
// ---------------------------------------------------------------------------
// per-row state of pass A (one query row per lane pair l, l^32)
struct DqRow {
  float delta, lse2, rowc, slp, dm, wd;
  int row, doc;
};

// ---------------------------------------------------------------------------
// pass A, two wavefronts per SIMD (block size 256, no bias or block bias)
// ---------------------------------------------------------------------------
// Probabilities and dS^T of one 32-key half (mb) of a tile for this lane's
// query row: dsb[hf] is k-step 2·mb + hf of dQ^T = K^T·dS^T.
template <int MODE, bool MASK>
__device__ __forceinline__ void dq2_probs(const KvTile<MODE>& b, const DqRow& R, int kv0, float off, float cs,
                                          int lane, int mb, const f32x16_t& s, const f32x16_t& dp, uint4 (&dsb)[2],
                                          float& rs, float& pm) {
  const int g = lane >> 5;
  const int lim = R.row - kv0;  // keys j <= lim are causal
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    float dsv[8];
    int dcv[8];
    if (MASK) {
      const int4 d0 = *reinterpret_cast<const int4*>(&b.docs[mb * 32 + 16 * hf + 4 * g]);
      const int4 d1 = *reinterpret_cast<const int4*>(&b.docs[mb * 32 + 16 * hf + 8 + 4 * g]);
      dcv[0] = d0.x, dcv[1] = d0.y, dcv[2] = d0.z, dcv[3] = d0.w;
      dcv[4] = d1.x, dcv[5] = d1.y, dcv[6] = d1.z, dcv[7] = d1.w;
    }
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const int r = hf * 8 + jj;
      const int j = mb * 32 + 8 * (r / 4) + 4 * g + (r % 4);  // key within the tile
      float x = fmaf(s[r], cs, off);
      if (MASK) x = mask_score(x, j, lim, dcv[jj], R.doc);
      const float p = __builtin_amdgcn_exp2f(x);
      const float d = p * (dp[r] - R.delta);
      dsv[jj] = d;
      rs += d;
      pm += p;
    }
    dsb[hf] = make_uint4(cvt_pk_bf16(dsv[0], dsv[1]), cvt_pk_bf16(dsv[2], dsv[3]), cvt_pk_bf16(dsv[4], dsv[5]),
                         cvt_pk_bf16(dsv[6], dsv[7]));
  }
}

template <int BS, int MODE>
__global__ __launch_bounds__(2 * BS) void attn_bwd_dq2_kernel(AttnArgs a) {
  static_assert(MODE <= 1, "token modes use attn_bwd_dq16_kernel");
  constexpr int NT = 2 * BS;  // BS/32 wavefronts of 32 query rows: the whole q-block
  constexpr int BN = 64;      // keys per staged tile, processed in two 32-key halves
  constexpr int NSUB = BS / BN;

  __shared__ KvTile<MODE> buf0, buf1, buf2;
  __shared__ int kbs[kListLds];
  __shared__ float kbias[kListLds];  // pair bias per list entry (log2 units), when given
  // block mode: β·log2e-scaled coefficients [BS][cos 8 | sin 8] and the
  // coefficient-gradient sums [BS][Σrs·cos 8 | Σpm·cos 8 | Σrs·sin 8 | Σpm·sin 8]
  __shared__ __attribute__((aligned(16))) float coef[MODE == 1 ? BS * 16 : 4];
  __shared__ __attribute__((aligned(16))) float gacc[MODE == 1 ? BS * 32 : 4];

  const int tid = threadIdx.x;
  const int wave = tid / 64, lane = tid % 64, g = lane / 32, lr = lane % 32;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int h = tile / a.QB, qb = tile % a.QB;
  const int64_t q0 = static_cast<int64_t>(qb) * BS;
  const int wrow_lo = static_cast<int>(q0) + wave * 32;
  const int64_t hT = static_cast<int64_t>(h) * a.T;
  const int lrow_ = wave * 32 + lr;  // row within the block
  DqRow R;
  R.row = wrow_lo + lr;

  const int64_t lrow = static_cast<int64_t>(h) * a.QB + qb;
  const int n = min(a.kv_num[lrow], a.maxkv);  // maxkv <= kListLds
  const int32_t* lst = a.kv_idx + lrow * a.maxkv;
  for (int t = tid; t < min(n, kListLds); t += NT) kbs[t] = lst[t];
  const bool pbias = a.pair_bias != nullptr;
  if (pbias)
    for (int t = tid; t < min(n, kListLds); t += NT) kbias[t] = a.pair_bias[lrow * a.maxkv + t] * kLog2e;

  uint4 qreg[8], doreg[8];
  {
    const uint16_t* qp = a.q + h * a.q_sh + R.row * a.q_st + g * 8;
    const uint16_t* op = a.o + h * a.o_sh + R.row * a.o_st + g * 8;
    const uint16_t* dp = a.dout + h * a.o_sh + R.row * a.o_st + g * 8;
    float dsum = 0.f;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      qreg[ks] = *reinterpret_cast<const uint4*>(qp + ks * 16);
      doreg[ks] = *reinterpret_cast<const uint4*>(dp + ks * 16);
      const uint4 ov = *reinterpret_cast<const uint4*>(op + ks * 16);
      const uint32_t dw[4] = {doreg[ks].x, doreg[ks].y, doreg[ks].z, doreg[ks].w};
      const uint32_t ow[4] = {ov.x, ov.y, ov.z, ov.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dsum += __uint_as_float(dw[i] << 16) * __uint_as_float(ow[i] << 16);
        dsum += __uint_as_float(dw[i] & 0xffff0000u) * __uint_as_float(ow[i] & 0xffff0000u);
      }
    }
    R.delta = dsum + __shfl_xor(dsum, 32, 64);
  }
  const float lse_nat = a.lse[hT + R.row];
  R.lse2 = lse_nat == -INFINITY ? INFINITY : lse_nat * kLog2e;
  R.rowc = R.slp = R.dm = R.wd = 0.f;
  if (MODE == 1) {
    // lane pair (l, l^32): g = 0 fills the cos half of its row, g = 1 the sin half
    const float* cf = (g == 0 ? a.coeff_cos : a.coeff_sin) + (hT + R.row) * a.K;
#pragma unroll
    for (int k = 0; k < 8; ++k) coef[row16_off(lrow_, 2 * g + k / 4) + k % 4] = k < a.K ? cf[k] * a.beta_log2 : 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) gacc[row32_off(lrow_, 4 * g + k / 4) + k % 4] = 0.f;
  }
  const int ds_end = a.ds_tok_end[qb];
  R.doc = a.docs[R.row];
  const float cs = a.scale_log2;
  const TileOffs to = tile_offs(lane);

  f32x16_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = zero16();
  float rs_tot = 0.f;  // per lane (half the keys of the row) until the epilogue
  float bt = 0.f, rs_kb = 0.f, pm_kb = 0.f;
  float eb = 0.f;  // pair bias of the current key block (log2 units)

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
  auto issue = [&](int it, KvTile<MODE>& b) __attribute__((always_inline)) {
    const int kb = kb_at(it / NSUB);
    const int rd = min(max(qb - kb, 0), a.QB - 1);
    kv_issue<MODE, NT>(a, h, static_cast<int64_t>(kb) * BS + (it % NSUB) * BN, rd, b, tid);
  };
  // One tile in two parts.  Part A: scores, probabilities and dQ of the
  // first 32-key half, then scores and probabilities of the second (its dS^T
  // returned in dsb1); part B: the second half's dQ.
  auto dq_half = [&](const KvTile<MODE>& b, int mb, const uint4 (&dsb)[2]) __attribute__((always_inline)) {
    // dQ^T += K^T dS^T over keys mb·32 .. +31 (step st: k-step 2·mb + st/4, columns 32·(st%4))
    uint4 ta[2];
    ta[0] = lds_kmajor_o(b.k, to, 32 * mb, 0);
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      if (st + 1 < 8) ta[(st + 1) % 2] = lds_kmajor_o(b.k, to, 16 * (2 * mb + (st + 1) / 4), (st + 1) % 4);
      o[st % 4] = mfma32(ta[st % 2], dsb[st / 4], o[st % 4]);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  auto compute_a = [&](int kv0, const KvTile<MODE>& b, float eb, uint4 (&dsb1)[2]) __attribute__((always_inline)) {
    const bool full = (kv0 + BN - 1 <= wrow_lo) && (ds_end <= kv0);
    const float off = (MODE == 1 ? bt : 0.f) + eb - R.lse2;
    float rs = 0.f, pm = 0.f;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      // S^T and dP^T of keys mb·32 .. +31 (A operand) against this lane's row (B)
      // (operands one k-step ahead; each step's reads go out before its MFMAs)
      f32x16_t s = zero16(), dp = zero16();
      uint4 ka[2], va[2];
      ka[0] = lds_row8_o(b.k, to, mb * 32, 0);
      va[0] = lds_row8_o(b.v, to, mb * 32, 0);
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        if (ks + 1 < 8) {
          ka[(ks + 1) % 2] = lds_row8_o(b.k, to, mb * 32, ks + 1);
          va[(ks + 1) % 2] = lds_row8_o(b.v, to, mb * 32, ks + 1);
        }
        s = mfma32(ka[ks % 2], qreg[ks], s);
        dp = mfma32(va[ks % 2], doreg[ks], dp);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      uint4 dsb[2];
      if (!full)
        dq2_probs<MODE, true>(b, R, kv0, off, cs, lane, mb, s, dp, dsb, rs, pm);
      else
        dq2_probs<MODE, false>(b, R, kv0, off, cs, lane, mb, s, dp, dsb, rs, pm);
      if (mb == 0) {
        dq_half(b, 0, dsb);
      } else {
        dsb1[0] = dsb[0];
        dsb1[1] = dsb[1];
      }
    }
    rs_kb += rs;
    pm_kb += pm;
    rs_tot += rs;
  };
  // part A of tile it with the block-mode bookkeeping; false when the
  // wavefront has nothing to do for this tile
  auto run_a = [&](int it, int nxt, const KvTile<MODE>& b, uint4 (&dsb1)[2]) __attribute__((always_inline)) -> bool {
    const int kv0 = kb_at(it / NSUB) * BS + (it % NSUB) * BN;
    if (MODE == 1 && it % NSUB == 0) {
      // block term of this key block (its first tile is never skipped)
      const float4* t4 = reinterpret_cast<const float4*>(b.tab);
      float acc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 c4 = *reinterpret_cast<const float4*>(coef + row16_off(lrow_, i)), tt = t4[i];
        acc[i] = c4.x * tt.x + c4.y * tt.y + c4.z * tt.z + c4.w * tt.w;
      }
      bt = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    }
    if (it % NSUB == 0) eb = pbias ? kbias[it / NSUB] : 0.f;  // per key block
    const bool act = kv0 <= wrow_lo + 31;  // else every key follows this wavefront's rows
    if (act) compute_a(kv0, b, eb, dsb1);
    if (MODE == 1 && (nxt >= total || nxt / NSUB != it / NSUB)) {
      // last tile of this key block: fold the row sums (combined over the lane
      // pair) into the gradient sums; g = 0 keeps the cos half, g = 1 the sin half
      const float rsr = rs_kb + __shfl_xor(rs_kb, 32, 64), pmr = pm_kb + __shfl_xor(pm_kb, 32, 64);
      const float4* t4 = reinterpret_cast<const float4*>(b.tab + g * 8);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float4 tt = t4[i];
        float4* gr = reinterpret_cast<float4*>(gacc + row32_off(lrow_, 4 * g + i));
        float4* gp = reinterpret_cast<float4*>(gacc + row32_off(lrow_, 4 * g + 2 + i));
        float4 ar = *gr, ap = *gp;
        ar.x += rsr * tt.x, ar.y += rsr * tt.y, ar.z += rsr * tt.z, ar.w += rsr * tt.w;
        ap.x += pmr * tt.x, ap.y += pmr * tt.y, ap.z += pmr * tt.z, ap.w += pmr * tt.w;
        *gr = ar;
        *gp = ap;
      }
      rs_kb = pm_kb = 0.f;
    }
    return act;
  };

  __syncthreads();  // kbs
  // Wavefronts 0-3 (one per SIMD) process whole tiles and copy them (256
  // threads) into three rotating buffers; wavefronts 4-7 run part of a tile
  // behind: their k-th barrier falls between part A and part B of tile k-1,
  // so the two wavefronts of a SIMD are not in the same phase.  At the
  // leading group's k-th barrier the lagging group is done with tile k-2,
  // whose buffer then takes tile k+1.  Both groups pass n+1 barriers for n
  // tiles.
  const int tid4 = tid & 255;
  auto issue4 = [&](int it, KvTile<MODE>& b) __attribute__((always_inline)) {
    const int kb = kb_at(it / NSUB);
    const int rd = min(max(qb - kb, 0), a.QB - 1);
    kv_issue<MODE, 256>(a, h, static_cast<int64_t>(kb) * BS + (it % NSUB) * BN, rd, b, tid4);
  };
  int cur = next_valid(0);
  if (wave < 4) {
    if (cur < total) issue4(cur, buf0);
    auto lead = [&](const KvTile<MODE>& bc, KvTile<MODE>& bn) __attribute__((always_inline)) {
      wait_vm0();
      __syncthreads();  // tile cur is in bc for everyone; the lagging group is done with bn
      const int nxt = next_valid(cur + 1);
      if (nxt < total) issue4(nxt, bn);
      uint4 dsb1[2];
      if (run_a(cur, nxt, bc, dsb1)) dq_half(bc, 1, dsb1);
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
    __syncthreads();  // tile 0 is in buf0
    auto lag = [&](const KvTile<MODE>& bc) __attribute__((always_inline)) {
      const int nxt = next_valid(cur + 1);
      uint4 dsb1[2];
      const bool act = run_a(cur, nxt, bc, dsb1);
      __syncthreads();  // the leading group starts the next tile
      if (act) dq_half(bc, 1, dsb1);
      cur = nxt;
    };
    while (cur < total) {
      lag(buf0);
      if (cur >= total) break;
      lag(buf1);
      if (cur >= total) break;
      lag(buf2);
    }
  }

  // ---- epilogue: dQ = scale·o, coefficient gradients.  The lane's row and
  // the addresses from it are formed again here from an opaque copy of the
  // lane index, so that none of them is held (or spilled) through the tiles.
  int tid_e = tid;
  asm volatile("" : "+v"(tid_e));
  const int lane_e = tid_e % 64, ge = lane_e / 32, lrow_e = (tid_e / 64) * 32 + lane_e % 32;
  R.row = static_cast<int>(q0) + lrow_e;
  rs_tot += __shfl_xor(rs_tot, 32, 64);
  const float dd_err = rs_tot;  // Δ_true - Δ
  // the kv-major pass reads Δ_true = Δ + (Δ_true - Δ): its dS, dK and the
  // pair-bias sums then do not carry the bf16 rounding of the output
  if (ge == 0) a.delta[hT + R.row] = -(R.delta + dd_err);  // stored negated: the kv-major dP accumulators start from it
  uint16_t* dqp = a.dq + h * a.q_sh + R.row * a.q_st + 4 * ge;
#pragma unroll
  for (int md = 0; md < 4; ++md)
#pragma unroll
    for (int rq = 0; rq < 4; ++rq) {
      uint2 val;
      val.x = cvt_pk_bf16(o[md][4 * rq] * a.scale, o[md][4 * rq + 1] * a.scale);
      val.y = cvt_pk_bf16(o[md][4 * rq + 2] * a.scale, o[md][4 * rq + 3] * a.scale);
      *reinterpret_cast<uint2*>(dqp + md * 32 + 8 * rq) = val;
    }
  if (MODE == 1 && a.dcoeff_cos) {
    // g = 0 writes the cos coefficients of its row, g = 1 the sin ones
    float* dst = (ge == 0 ? a.dcoeff_cos : a.dcoeff_sin) + (hT + R.row) * a.K;
    for (int k = 0; k < a.K; ++k) {
      const float rs = gacc[row32_off(lrow_e, 4 * ge + k / 4) + k % 4];
      const float pm = gacc[row32_off(lrow_e, 4 * ge + 2 + k / 4) + k % 4];
      dst[k] = a.beta * (rs - dd_err * pm);
    }
  }
  // ---- this row's softmax offset for every listed key block (the block term
  // as in the loop, plus the pair bias, minus lse), read per tile by the
  // kv-major pass; after the dQ store, when its accumulators are free
  if (ge == 0) {
    float* rof = a.roff + lrow * a.maxkv * BS + lrow_e;
    for (int e = 0; e < n; ++e) {
      float t = pbias ? kbias[e] : 0.f;
      if (MODE == 1) {
        const int rd = min(max(qb - kb_at(e), 0), a.QB - 1);
        const float4* t4 = reinterpret_cast<const float4*>(static_cast<const float*>(a.table) + rd * 16);
        float acc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 c4 = *reinterpret_cast<const float4*>(coef + row16_off(lrow_e, i)), tt = t4[i];
          acc[i] = c4.x * tt.x + c4.y * tt.y + c4.z * tt.z + c4.w * tt.w;
        }
        t += (acc[0] + acc[1]) + (acc[2] + acc[3]);
      }
      rof[e * BS] = t - R.lse2;
    }
  }
}

// ---------------------------------------------------------------------------
// plan: chunked work items for the kv-major pass
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void bwd_plan_kernel(int NB, int chunk, const int32_t* __restrict__ q_off,
                                                         int32_t* __restrict__ items_start,
                                                         int32_t* __restrict__ slots_start,
                                                         int32_t* __restrict__ multi) {
  const int h = blockIdx.x;
  const int32_t* off = q_off + static_cast<int64_t>(h) * (NB + 1);
  int32_t* it = items_start + static_cast<int64_t>(h) * (NB + 1);
  int32_t* sl = slots_start + static_cast<int64_t>(h) * (NB + 1);
  int32_t* ml = multi + static_cast<int64_t>(h) * (NB + 1);
  __shared__ int s_it[1024], s_sl[1024], s_ml[1024];
  __shared__ int carry_it, carry_sl, carry_ml;
  if (threadIdx.x == 0) carry_it = carry_sl = carry_ml = 0;
  __syncthreads();
  for (int base = 0; base < NB; base += 1024) {
    const int kb = base + threadIdx.x;
    int nit = 0, nsl = 0, nml = 0;
    if (kb < NB) {
      const int n = off[kb + 1] - off[kb];
      const int nch = max(1, (n + chunk - 1) / chunk);
      nit = nch;
      nsl = nch > 1 ? nch : 0;
      nml = nch > 1 ? 1 : 0;
    }
    s_it[threadIdx.x] = nit;
    s_sl[threadIdx.x] = nsl;
    s_ml[threadIdx.x] = nml;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {
      const int ai = threadIdx.x >= o ? s_it[threadIdx.x - o] : 0;
      const int as = threadIdx.x >= o ? s_sl[threadIdx.x - o] : 0;
      const int am = threadIdx.x >= o ? s_ml[threadIdx.x - o] : 0;
      __syncthreads();
      s_it[threadIdx.x] += ai;
      s_sl[threadIdx.x] += as;
      s_ml[threadIdx.x] += am;
      __syncthreads();
    }
    const int ci = carry_it, cl = carry_sl, cm = carry_ml;
    if (kb < NB) {
      it[kb] = ci + s_it[threadIdx.x] - nit;
      sl[kb] = cl + s_sl[threadIdx.x] - nsl;
      if (nml) ml[1 + cm + s_ml[threadIdx.x] - 1] = kb;  // ascending key blocks
    }
    __syncthreads();
    if (threadIdx.x == 1023) {
      carry_it = ci + s_it[1023];
      carry_sl = cl + s_sl[1023];
      carry_ml = cm + s_ml[1023];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    it[NB] = carry_it;
    sl[NB] = carry_sl;
    ml[0] = carry_ml;
  }
}

// ---------------------------------------------------------------------------
// pass B
// ---------------------------------------------------------------------------
struct KvPlan {
  const int32_t* items_start;
  const int32_t* slots_start;
  const int32_t* multi;  // per head [NB+1]: the count, then the key blocks with more than one chunk
  const int32_t* q_pos;  // with a pair bias: for each q-list entry, kb's position in that q-block's kv list
  float* part_dk;
  float* part_dv;
  int64_t max_slots;  // per head
  int max_items;      // work items per head (upper bound)
  int chunk;          // q-blocks per work item (bwd_chunk)
};

// q_pos[h][i] = the position of key block kb in the kv list of q-block
// q_list[h][i], for every entry i of kb's q-list (its first kv_num entries
// are unique; a scan of independent loads).  A thread per q-list entry: the
// entry's key block is the bucket of q_off that holds i (a binary search),
// so a key block listed by every q-block (a long document's global block)
// is spread over as many threads as it has entries.
__global__ __launch_bounds__(256) void qpos_kernel(AttnArgs a, int32_t* __restrict__ q_pos) {
  const int NB = a.QB;
  const int64_t per_head = static_cast<int64_t>(a.QB) * a.maxkv;
  const int64_t n = per_head * a.H;
  for (int64_t s = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; s < n;
       s += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int h = static_cast<int>(s / per_head);
    const int i = static_cast<int>(s % per_head);
    const int32_t* qo = a.q_off + static_cast<int64_t>(h) * (NB + 1);
    if (i >= qo[NB]) continue;  // past the head's entries
    // the largest kb with qo[kb] <= i: qo[kb] <= i < qo[kb + 1]
    int lo = 0, hi = NB - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) / 2;
      if (qo[mid] <= i) lo = mid;
      else hi = mid - 1;
    }
    const int kb = lo;
    const int64_t base = static_cast<int64_t>(h) * per_head;
    const int qb = a.q_list[base + i];
    const int64_t row = static_cast<int64_t>(h) * a.QB + qb;
    const int nl = min(a.kv_num[row], a.maxkv);
    const int32_t* lst = a.kv_idx + row * a.maxkv;
    int pos = -1;
    for (int e = 0; e < nl; ++e)
      if (lst[e] == kb) pos = e;
    q_pos[base + i] = pos;
  }
}

// Sum of x over the 64 lanes of the wavefront.
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

// LDS staging of one 64-row query tile of pass B.  Everything arrives by
// global_load_lds (no registers): two such buffers alternate, so the loads of
// tile j+1 run under the MFMAs of tile j.
template <int MODE>
struct alignas(16) DkvBuf {
  uint16_t q[64 * 128];            // Q rows, swizzled (swz_off)
  uint16_t d[64 * 128];            // dO rows, swizzled
  float ra[256];                   // softmax offset without the pair bias (log2) | -Δ | doc id (int32), 64 rows each
  float rb[MODE <= 1 ? 4 : 1024];  // token: query features [64][32] bf16 (chunk-swizzled)
  float rc[MODE >= 2 ? 256 : 4];   // token: β·slope (log2 units) | delta_main | width
};

// Issue part `part` (0..9) of the copies of the 64-row query tile starting at
// token q0 into b: 0-3 Q rows, 4-7 dO rows, 8 per-row constants, 9 block
// coefficients or token features.  The parts are spread over the MFMAs of the
// current tile, so that no wavefront stalls on a burst of memory instructions.
template <int MODE>
__device__ __forceinline__ void dkv_issue_part(const AttnArgs& a, int h, int64_t hT, int64_t q0v, const float* rof,
                                               DkvBuf<MODE>& b, int tid, int part) {
  // q0 and the wavefront index are the same in every lane: keep them, and
  // every row base below, in scalar registers (global_load_lds with a scalar
  // base and a 32-bit lane byte offset)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int64_t q0 = __builtin_amdgcn_readfirstlane(static_cast<int>(q0v));
  if (part < 8) {
    // chunk jj·256 + tid: row jj·16 + tid/16, physical chunk tid%16 (holds logical chunk p ^ swz(row))
    const int jj = part & 3;
    const int r = (tid >> 4) + jj * 16, c = (tid & 15) ^ swz(r);
    if (part < 4) {
      const char* base = reinterpret_cast<const char*>(a.q + h * a.q_sh + q0 * a.q_st);
      g2lds16(base, static_cast<uint32_t>((r * static_cast<int>(a.q_st) + c * 8) * 2), b.q + (jj * 256 + wave * 64) * 8);
    } else {
      const char* base = reinterpret_cast<const char*>(a.dout + h * a.o_sh + q0 * a.o_st);
      g2lds16(base, static_cast<uint32_t>((r * static_cast<int>(a.o_st) + c * 8) * 2), b.d + (jj * 256 + wave * 64) * 8);
    }
    return;
  }
  const uint32_t lo = static_cast<uint32_t>(lane) * 16;  // 16 lanes x 16 bytes = one 64-row float array
  if (part == 8) {
    // wavefront w copies per-row array w: the softmax offsets (modes 0/1: per
    // list entry; token modes: per row, the pair bias added per tile), -Δ,
    // document ids
    const char* base = wave == 0   ? reinterpret_cast<const char*>(MODE <= 1 ? rof : a.rowoff + hT + q0)
                       : wave == 1 ? reinterpret_cast<const char*>(a.delta + hT + q0)
                                   : reinterpret_cast<const char*>(a.docs + q0);
    if (lane < 16 && wave < 3) g2lds16(base, lo, b.ra + wave * 64);
    if (MODE >= 2) {
      // token terms: β·slope, delta_main, width on wavefronts 0, 1, 2
      const char* tb = wave == 0   ? reinterpret_cast<const char*>(a.rowslope + hT + q0)
                       : wave == 1 ? reinterpret_cast<const char*>(a.delta_main + hT + q0)
                                   : reinterpret_cast<const char*>(a.width + hT + q0);
      const bool need = wave == 0 || (wave < 3 && MODE == 3);
      if (lane < 16 && need) g2lds16(tb, lo, b.rc + wave * 64);
    }
    return;
  }
  if (MODE >= 2) {
    const int r = tid >> 2, c = (tid & 3) ^ swz32(r);
    const char* base = reinterpret_cast<const char*>(a.qfeat + (hT + q0) * kTokRow);
    g2lds16(base, static_cast<uint32_t>((r * kTokRow + c * 8) * 2), reinterpret_cast<uint16_t*>(b.rb) + wave * 64 * 8);
  }
}

template <int MODE>
__device__ __forceinline__ void dkv_issue(const AttnArgs& a, int h, int64_t hT, int64_t q0, const float* rof,
                                          DkvBuf<MODE>& b, int tid) {
#pragma unroll
  for (int part = 0; part < 10; ++part) dkv_issue_part<MODE>(a, h, hT, q0, rof, b, tid, part);
}

// P and dS of register quad (mq, rq) of one tile as bf16 B operands (k index:
// the 64 query rows): the quad is k-step 2·mq + rq/2, slots 4·(rq%2) .. +3.
// MASK applies the causal and document masks.
template <int MODE, bool MASK, bool DP>
__device__ __forceinline__ void dkv_probs_quad(const AttnArgs& a, const DkvBuf<MODE>& b, const float* offw, int q0,
                                               int lane, int wkv, int doc_kv, const f32x16_t (&s)[2],
                                               const f32x16_t (&dp)[2], uint4 (&pb)[4], uint4 (&dsb)[4], int mq,
                                               int rq, float& dsum) {
  constexpr bool TOK = MODE >= 2, GATE = MODE == 3;
  const int g = lane >> 5;
  const int* docq = reinterpret_cast<const int*>(b.ra + 128);
  const float cs = a.scale_log2;
  const float glam = a.beta_log2 * a.ramp_lambda;
  const float slsc = TOK ? 1.f : 0.f;  // b.rc holds β·slope (zero without the slope term)
  const float spw = a.gate_kind == SCOPE_GATE_SOFTPLUS ? kLn2 : 0.f;
  const int qi0 = mq * 32 + 8 * rq + 4 * g;  // 4 consecutive query rows of this register quad
  const float4 of4 = *reinterpret_cast<const float4*>(&offw[qi0]);
  const float4 dl4 = *reinterpret_cast<const float4*>(&b.ra[64 + qi0]);
  const float ofv[4] = {of4.x, of4.y, of4.z, of4.w};
  const float dlv[4] = {dl4.x, dl4.y, dl4.z, dl4.w};
  int dcv[4] = {0, 0, 0, 0};
  if (MASK) {
    const int4 dc4 = *reinterpret_cast<const int4*>(&docq[qi0]);
    dcv[0] = dc4.x;
    dcv[1] = dc4.y;
    dcv[2] = dc4.z;
    dcv[3] = dc4.w;
  }
  float pv[4], dsv[4];
#pragma unroll
  for (int i2 = 0; i2 < 4; ++i2) {
    const int r = 4 * rq + i2;
    const int q = q0 + qi0 + i2;
    float xv;
    if (TOK) {
      // slope and gate terms; softplus(x) = max(x,0) + ln2·log2(1 + 2^(-|x|·log2 e))
      const float df = static_cast<float>(q - wkv);
      float e = slsc * b.rc[qi0 + i2] * df;
      if (GATE) {
        const float xx = (fabsf(df - b.rc[64 + qi0 + i2]) - b.rc[128 + qi0 + i2]) * a.inv_tau;
        const float sp = __builtin_amdgcn_logf(1.f + __builtin_amdgcn_exp2f(-fabsf(xx) * kLog2e));
        e -= glam * fmaf(spw, sp, fmaxf(xx, 0.f));
      }
      xv = fmaf(s[mq][r], cs, e + ofv[i2]);
    } else {
      xv = fmaf(s[mq][r], cs, ofv[i2]);
    }
    if (MASK) xv = mask_score(xv, wkv, q, doc_kv, dcv[i2]);
    const float p = __builtin_amdgcn_exp2f(xv);
    pv[i2] = p;
    dsv[i2] = p * (dp[mq][r] + dlv[i2]);  // dlv holds -Δ
    if (DP) dsum += dsv[i2];
  }
  const int ksx = 2 * mq + rq / 2;
  const uint32_t p01 = cvt_pk_bf16(pv[0], pv[1]), p23 = cvt_pk_bf16(pv[2], pv[3]);
  const uint32_t d01 = cvt_pk_bf16(dsv[0], dsv[1]), d23 = cvt_pk_bf16(dsv[2], dsv[3]);
  if (rq % 2 == 0) {
    pb[ksx].x = p01;
    pb[ksx].y = p23;
    dsb[ksx].x = d01;
    dsb[ksx].y = d23;
  } else {
    pb[ksx].z = p01;
    pb[ksx].w = p23;
    dsb[ksx].z = d01;
    dsb[ksx].w = d23;
  }
}

// Per-row exponent offsets of a tile (lane = row), private to the wavefront.
template <int MODE>
__device__ __forceinline__ void dkv_offsets(const AttnArgs& a, const DkvBuf<MODE>& b, float* offw, const float* tab,
                                            float eb, int lane) {
  static_assert(MODE >= 2, "modes 0/1 read the offsets the q-major pass stored");
  offw[lane] = b.ra[lane] + eb;  // the row's offset (-β·b0 - lse, or -inf) and the pair bias
}

// One 64-row query tile against this wavefront's 32 keys: S, dP, then
// dV^T += dO^T·P and dK^T += Q^T·dS.  The copies of the next tile are issued
// by the caller, before this tile's reads.
template <int BS, int MODE, bool DP>
__device__ __forceinline__ void dkv_tile(const AttnArgs& a, const DkvBuf<MODE>& b, bool masked, float* offw,
                                         const float* tab, float eb,
                                         int64_t q0, int lane, int64_t wkv_lo, int doc_kv,
                                         const uint4 (&kreg)[8], const uint4 (&vreg)[8], const uint4& kf,
                                         const uint4& kfl, f32x16_t (&dvT)[4], f32x16_t (&dkT)[4],
                                         const TileOffs& to, float* slot) {
  const int g = lane >> 5, lr = lane & 31;
  const int wkv = static_cast<int>(wkv_lo) + lr;
  dkv_offsets<MODE>(a, b, offw, tab, eb, lane);
  // S and dP, query rows in two 32-row blocks (A operand), keys as columns (B)
  f32x16_t s[2], dp[2];
#pragma unroll
  for (int mq = 0; mq < 2; ++mq) {
    s[mq] = zero16();
    dp[mq] = zero16();
  }
  // four independent accumulator chains; the A operands of k-step ks+1 are
  // read from LDS while k-step ks runs (the fences stop the compiler from
  // hoisting every read, which would exhaust the registers)
  uint4 qa0 = lds_row8_o(b.q, to, 0, 0), qa1 = lds_row8_o(b.q, to, 32, 0);
  uint4 da0 = lds_row8_o(b.d, to, 0, 0), da1 = lds_row8_o(b.d, to, 32, 0);
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    uint4 qn0 = qa0, qn1 = qa1, dn0 = da0, dn1 = da1;
    if (ks < 7) {
      qn0 = lds_row8_o(b.q, to, 0, ks + 1);
      qn1 = lds_row8_o(b.q, to, 32, ks + 1);
      dn0 = lds_row8_o(b.d, to, 0, ks + 1);
      dn1 = lds_row8_o(b.d, to, 32, ks + 1);
    }
    s[0] = mfma32(qa0, kreg[ks], s[0]);
    dp[0] = mfma32(da0, vreg[ks], dp[0]);
    s[1] = mfma32(qa1, kreg[ks], s[1]);
    dp[1] = mfma32(da1, vreg[ks], dp[1]);
    // the next k-step's reads go out before this k-step's MFMAs
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
    __builtin_amdgcn_sched_barrier(0);
    qa0 = qn0, qa1 = qn1, da0 = dn0, da1 = dn1;
  }
  if (MODE >= 2) {
    const uint16_t* qf = reinterpret_cast<const uint16_t*>(b.rb);
#pragma unroll
    for (int mq = 0; mq < 2; ++mq) {
      const uint4 qh = lds_row8_32(qf, mq * 32 + lr, g * 8);
      const uint4 qlo = lds_row8_32(qf, mq * 32 + lr, 16 + g * 8);
      s[mq] = mfma32(qh, kf, s[mq]);
      s[mq] = mfma32(qlo, kf, s[mq]);
      s[mq] = mfma32(qh, kfl, s[mq]);
    }
  }
  uint4 pb[4], dsb[4];
  float dsum = 0.f;
  if (MODE >= 2 || masked) {  // token modes always take the masked form (one copy of their longer code)
#pragma unroll
    for (int mq = 0; mq < 2; ++mq)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq)
        dkv_probs_quad<MODE, true, DP>(a, b, offw, static_cast<int>(q0), lane, wkv, doc_kv, s, dp, pb, dsb, mq, rq,
                                       dsum);
  } else {
#pragma unroll
    for (int mq = 0; mq < 2; ++mq)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq)
        dkv_probs_quad<MODE, false, DP>(a, b, offw, static_cast<int>(q0), lane, wkv, doc_kv, s, dp, pb, dsb, mq, rq,
                                        dsum);
  }
  if (DP) {
    dsum = wave_sum(dsum);
    if (lane == 0) *slot += dsum;
  }
  // dV^T += dO^T P,  dK^T += Q^T dS  (k index: the 64 query rows); a step is
  // two MFMAs, so the operands are read TPD steps ahead into a ring
  __builtin_amdgcn_sched_barrier(0);
  constexpr int TPD = 3;
  uint4 ta[TPD + 1], tb[TPD + 1];
#pragma unroll
  for (int i = 0; i < TPD; ++i) {
    ta[i] = lds_kmajor_o(b.d, to, 16 * (i / 4), i % 4);
    tb[i] = lds_kmajor_o(b.q, to, 16 * (i / 4), i % 4);
  }
#pragma unroll
  for (int st = 0; st < 16; ++st) {
    const int s4 = st / 4, md = st % 4;
    if (st + TPD < 16) {
      ta[(st + TPD) % (TPD + 1)] = lds_kmajor_o(b.d, to, 16 * ((st + TPD) / 4), (st + TPD) % 4);
      tb[(st + TPD) % (TPD + 1)] = lds_kmajor_o(b.q, to, 16 * ((st + TPD) / 4), (st + TPD) % 4);
    }
    dvT[md] = mfma32(ta[st % (TPD + 1)], pb[s4], dvT[md]);
    dkT[md] = mfma32(tb[st % (TPD + 1)], dsb[s4], dkT[md]);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int BS, int MODE, bool DP>
__global__ __launch_bounds__(256) void attn_bwd_dkv_kernel(AttnArgs a, KvPlan pl) {
  constexpr int D = 128;
  constexpr int BM = 64;  // query rows per staged tile
  constexpr int NS = BS / BM;

  __shared__ DkvBuf<MODE> buf0, buf1;
  __shared__ __attribute__((aligned(16))) float offw[4][BM];
  __shared__ __attribute__((aligned(16))) float tabs[MODE == 1 ? kChunkMax * 16 : 4];
  __shared__ int qbs[kChunkMax], dse[kChunkMax], epos[kChunkMax];
  __shared__ float ebias[kChunkMax];
  __shared__ float pslot[kChunkMax][4];  // pair-bias gradient: per entry and wavefront

  constexpr int P = BS / 128;  // workgroups (128 keys each) per key block
  const int NB = a.QB;
  // 1-D grid, XCD-aware: the hardware deals workgroup ids round-robin over the
  // 8 XCDs, so id L runs on XCD L % 8.  Each XCD takes a contiguous range of
  // (head, item) pairs, and the P parts of one item get consecutive slots on
  // the same XCD: they read the same query tiles, which then come from its L2.
  const int L = blockIdx.x;
  const int per_xcd = gridDim.x / 8 / P;  // items per XCD (the grid is a multiple of 8·P)
  const int pair = (L / 8) / P, zpart = (L / 8) % P;
  const int item = (L % 8) * per_xcd + pair;
  if (item >= a.H * pl.max_items) return;
  const int h = item / pl.max_items;
  const int x = item % pl.max_items;
  const int32_t* its = pl.items_start + static_cast<int64_t>(h) * (NB + 1);
  if (x >= its[NB]) return;
  // key block owning item x: largest kb with its[kb] <= x
  int lo = 0, hi = NB - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (its[mid] <= x) lo = mid;
    else hi = mid - 1;
  }
  const int kb = lo;
  const int chunk = x - its[kb];
  const int32_t* qo = a.q_off + static_cast<int64_t>(h) * (NB + 1);
  const int nq = qo[kb + 1] - qo[kb];
  const int CH = pl.chunk;
  const int nch = max(1, (nq + CH - 1) / CH);
  const int i0 = chunk * CH, i1 = min(nq, i0 + CH);
  const int ne = max(0, i1 - i0);
  const int32_t* ql = a.q_list + static_cast<int64_t>(h) * a.QB * a.maxkv + qo[kb];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid % 64, g = lane / 32, lr = lane % 32;
  const int64_t kv0 = static_cast<int64_t>(kb) * BS + zpart * 128;  // first key row of this workgroup
  const int64_t wkv_lo = kv0 + wave * 32;
  const int64_t wkv = wkv_lo + lr;
  const int krow = zpart * 128 + wave * 32 + lr;  // key row within the block
  const int64_t hT = static_cast<int64_t>(h) * a.T;

  // The q-list is ascending, so only its first entry can be the diagonal
  // block; there the query sub-tiles that end before kv0 are skipped.
  const int qb_first = ne > 0 ? ql[i0] : 0;
  const int skip0 = ne > 0 && qb_first == kb ? (zpart * 128) / BM : 0;
  const int n_it = ne * NS - skip0;

  if (tid < ne) {
    const int qb = ql[i0 + tid];
    qbs[tid] = qb;
    dse[tid] = a.ds_tok_end[qb];
    float eb = 0.f;
    int pos = -1;
    if (pl.q_pos) {
      pos = pl.q_pos[static_cast<int64_t>(h) * a.QB * a.maxkv + qo[kb] + i0 + tid];
      if (a.pair_bias && pos >= 0) eb = a.pair_bias[(static_cast<int64_t>(h) * a.QB + qb) * a.maxkv + pos] * kLog2e;
    }
    ebias[tid] = eb;
    epos[tid] = pos;
  }
  for (int t = tid; DP && t < CH * 4; t += blockDim.x) pslot[t / 4][t % 4] = 0.f;
  // block-mode table row of distance qb - kb (clamped: a later key block is fully masked anyway)
  for (int t = tid; MODE == 1 && t < ne * 16; t += blockDim.x) {
    const int r = min(max(ql[i0 + t / 16] - kb, 0), NB - 1);
    tabs[t] = static_cast<const float*>(a.table)[static_cast<int64_t>(r) * 16 + t % 16];
  }
  if (n_it > 0) {
    const int64_t q0 = static_cast<int64_t>(qb_first) * BS + (skip0 % NS) * BM;
    dkv_issue<MODE>(a, h, hT, q0, nullptr, buf0, tid);
  }

  uint4 kreg[8], vreg[8];
  {
    const uint16_t* kp = a.k + h * a.k_sh + wkv * a.k_st + g * 8;
    const uint16_t* vp = a.v + h * a.v_sh + wkv * a.v_st + g * 8;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      kreg[ks] = *reinterpret_cast<const uint4*>(kp + ks * 16);
      vreg[ks] = *reinterpret_cast<const uint4*>(vp + ks * 16);
    }
  }
  uint4 kf = make_uint4(0, 0, 0, 0), kfl = make_uint4(0, 0, 0, 0);
  if (MODE >= 2) {
    kf = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.table) + wkv * kTokRow + g * 8);
    kfl = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.table) + wkv * kTokRow + 16 + g * 8);
  }
  const int doc_kv = a.docs[wkv];
  const TileOffs to = tile_offs(lane);

  f32x16_t dvT[4], dkT[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    dvT[i] = zero16();
    dkT[i] = zero16();
  }

  // iteration j covers flat index f = j + skip0: list entry f / NS, sub-tile f % NS
  auto tile_q0 = [&](int j, int& e) __attribute__((always_inline)) {
    const int f = j + skip0;
    e = f / NS;
    return static_cast<int64_t>(qbs[e]) * BS + (f % NS) * BM;
  };
  for (int j = 0; j < n_it; j += 2) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int jj = j + half;
      if (jj < n_it) {
        wait_vm0();
        __syncthreads();  // tile jj is in LDS; every wavefront is done with tile jj-1
        int e, en;
        if (jj + 1 < n_it) {
          const int64_t qn = tile_q0(jj + 1, en);
          if (half == 0) dkv_issue<MODE>(a, h, hT, qn, nullptr, buf1, tid);
          else dkv_issue<MODE>(a, h, hT, qn, nullptr, buf0, tid);
        }
        const int64_t q0 = tile_q0(jj, e);
        const float* tab = tabs + (MODE == 1 ? e * 16 : 0);
        if (q0 + BM - 1 >= wkv_lo) {  // else every query row precedes this wavefront's keys
          const bool masked = !((wkv_lo + 31 <= q0) && (dse[e] <= wkv_lo));
          const DkvBuf<MODE>& bc = half == 0 ? buf0 : buf1;
          dkv_tile<BS, MODE, DP>(a, bc, masked, offw[wave], tab, ebias[e], q0, lane, wkv_lo, doc_kv, kreg, vreg, kf,
                                 kfl, dvT, dkT, to, &pslot[e][wave]);
        }
      }
    }
  }

  if (DP) {
    __syncthreads();  // every wavefront's slots are final
    if (tid < ne && epos[tid] >= 0) {
      const float t = (pslot[tid][0] + pslot[tid][1]) + (pslot[tid][2] + pslot[tid][3]);
      const int64_t row = static_cast<int64_t>(h) * a.QB + qbs[tid];
      a.dpair[(static_cast<int64_t>(zpart) * a.H * a.QB + row) * a.maxkv + epos[tid]] = t;
    }
  }

  // ---- write dK = scale·dkT^T, dV = dvT^T
  if (nch == 1) {
    uint16_t* dkp = a.dk + h * a.k_sh + wkv * a.k_st + 4 * g;
    uint16_t* dvp = a.dv + h * a.v_sh + wkv * a.v_st + 4 * g;
#pragma unroll
    for (int md = 0; md < 4; ++md)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        uint2 vk, vv;
        vk.x = cvt_pk_bf16(dkT[md][4 * rq] * a.scale, dkT[md][4 * rq + 1] * a.scale);
        vk.y = cvt_pk_bf16(dkT[md][4 * rq + 2] * a.scale, dkT[md][4 * rq + 3] * a.scale);
        vv.x = cvt_pk_bf16(dvT[md][4 * rq], dvT[md][4 * rq + 1]);
        vv.y = cvt_pk_bf16(dvT[md][4 * rq + 2], dvT[md][4 * rq + 3]);
        *reinterpret_cast<uint2*>(dkp + md * 32 + 8 * rq) = vk;
        *reinterpret_cast<uint2*>(dvp + md * 32 + 8 * rq) = vv;
      }
  } else {
    const int64_t slot = h * pl.max_slots + pl.slots_start[static_cast<int64_t>(h) * (NB + 1) + kb] + chunk;
    float* pk = pl.part_dk + (slot * BS + krow) * D + 4 * g;
    float* pv = pl.part_dv + (slot * BS + krow) * D + 4 * g;
#pragma unroll
    for (int md = 0; md < 4; ++md)
#pragma unroll
      for (int rq = 0; rq < 4; ++rq) {
        *reinterpret_cast<float4*>(pk + md * 32 + 8 * rq) =
            make_float4(dkT[md][4 * rq], dkT[md][4 * rq + 1], dkT[md][4 * rq + 2], dkT[md][4 * rq + 3]);
        *reinterpret_cast<float4*>(pv + md * 32 + 8 * rq) =
            make_float4(dvT[md][4 * rq], dvT[md][4 * rq + 1], dvT[md][4 * rq + 2], dvT[md][4 * rq + 3]);
      }
  }
}

// ---------------------------------------------------------------------------
// pass B, 16 keys per wavefront (modes 0 and 1)
// ---------------------------------------------------------------------------
// Eight wavefronts of 16 keys share a workgroup of 128 keys, two wavefronts
// per SIMD, so that one wavefront's probabilities run under the other's
// matrix products.  Per 64-row query tile a wavefront computes, with
// v_mfma_f32_16x16x32_bf16:
//   S = Q·K^T, dP = dO·V^T   (M = 16 query rows × 4, N = its 16 keys, K and V
//                             of those keys held in registers as B operands)
//   dV^T += dO^T·P, dK^T += Q^T·dS   (M = 16 columns of D × 8, K = 64 rows)
// The S accumulator of row block mb holds rows 16mb + 4g + r (g = lane / 16)
// for key lane % 16, so P and dS are the B operands of the second pair with
// no data movement: k-step kk takes slots 0-3 from row block 2kk and slots
// 4-7 from row block 2kk+1; the transpose reads of dO^T and Q^T use the same
// row order.

// P and dS of one tile for this lane's key as the B operands of the
// transposed products (pb[kk], dsb[kk]: k-step kk, see above).  Modes 0/1:
// the rows' softmax offsets are in b.ra[0..63].  Token modes: the offset
// of a row is -β·b0 + the pair bias eb - lse (log2 units, b.ra: lse | Δ |
// doc | b0), and each score adds the slope term β·slope·(i - j) and, with
// the gate (mode 3), -β·λ·gate(|i - j - δ| - w).
template <int MODE, bool MASK, bool DP>
__device__ __forceinline__ void dkv16_probs(const AttnArgs& a, const DkvBuf<MODE>& b, const float* offw, float eb,
                                            float cs, int q0, int wkv, int doc_kv, int g, const f32x4_t (&s)[4],
                                            const f32x4_t (&dp)[4], uint4 (&pb)[2], uint4 (&dsb)[2], float& dsum) {
  constexpr bool TOK = MODE >= 2, GATE = MODE == 3;
  const int* docq = reinterpret_cast<const int*>(b.ra + 128);
  uint32_t pw[8], dw[8];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    const int qi0 = 16 * mb + 4 * g;  // rows qi0 .. qi0+3 of the tile
    float ofv[4], slv[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (TOK) {
      // the rows' offsets (-β·b0 - lse) and β·slope, stored by the q-major pass
      const float4 o4 = *reinterpret_cast<const float4*>(&b.ra[qi0]);
      const float4 s4 = *reinterpret_cast<const float4*>(&b.rc[qi0]);
      ofv[0] = o4.x + eb, ofv[1] = o4.y + eb, ofv[2] = o4.z + eb, ofv[3] = o4.w + eb;
      slv[0] = s4.x, slv[1] = s4.y, slv[2] = s4.z, slv[3] = s4.w;
    } else {
      const float4 of4 = *reinterpret_cast<const float4*>(&offw[qi0]);
      ofv[0] = of4.x, ofv[1] = of4.y, ofv[2] = of4.z, ofv[3] = of4.w;
    }
    int dcv[4] = {0, 0, 0, 0};
    if (MASK) {
      const int4 dc4 = *reinterpret_cast<const int4*>(&docq[qi0]);
      dcv[0] = dc4.x, dcv[1] = dc4.y, dcv[2] = dc4.z, dcv[3] = dc4.w;
    }
    float pv[4], dv[4];
    const float dfb = static_cast<float>(q0 + qi0 - wkv);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float x;
      if constexpr (TOK) {
        const float df = dfb + static_cast<float>(i);  // q - wkv, exact in fp32
        float e = slv[i] * df;
        if constexpr (GATE) {
          // softplus(x) = max(x,0) + ln2·log2(1 + 2^(-|x|·log2 e)); relu drops the second term
          const float xx = (fabsf(df - b.rc[64 + qi0 + i]) - b.rc[128 + qi0 + i]) * a.inv_tau;
          const float sp = __builtin_amdgcn_logf(1.f + __builtin_amdgcn_exp2f(-fabsf(xx) * kLog2e));
          const float spw = a.gate_kind == SCOPE_GATE_SOFTPLUS ? kLn2 : 0.f;
          e -= a.beta_log2 * a.ramp_lambda * fmaf(spw, sp, fmaxf(xx, 0.f));
        }
        x = fmaf(s[mb][i], cs, e + ofv[i]);
      } else {
        x = fmaf(s[mb][i], cs, ofv[i]);
      }
      if (MASK) x = mask_score(x, wkv, q0 + qi0 + i, doc_kv, dcv[i]);
      const float p = __builtin_amdgcn_exp2f(x);
      pv[i] = p;
      dv[i] = p * dp[mb][i];  // the dP accumulator started from -Δ
      if (DP) dsum += dv[i];
    }
    pw[2 * mb] = cvt_pk_bf16(pv[0], pv[1]);
    pw[2 * mb + 1] = cvt_pk_bf16(pv[2], pv[3]);
    dw[2 * mb] = cvt_pk_bf16(dv[0], dv[1]);
    dw[2 * mb + 1] = cvt_pk_bf16(dv[2], dv[3]);
  }
  pb[0] = make_uint4(pw[0], pw[1], pw[2], pw[3]);
  pb[1] = make_uint4(pw[4], pw[5], pw[6], pw[7]);
  dsb[0] = make_uint4(dw[0], dw[1], dw[2], dw[3]);
  dsb[1] = make_uint4(dw[4], dw[5], dw[6], dw[7]);
}

// Lane byte offsets of the 16x16 operand reads of a swizzled tile.
// Row reads: at k-step ks lane group g takes columns 32g + 8ks .. +7 (the
// k order of the contraction is free as long as both operands follow it; with
// 4ks + g instead, the b128 reads of 64 lanes conflict two ways).
struct TileOffs16 {
  uint32_t row[4];  // row c = lane % 16, columns 32g + 8·ks .. +7 (g = lane / 16)
  uint32_t tr[8];   // transpose read: row 4g + (c / 4), columns 16·md + 4·(c % 4) .. +3
};

__device__ __forceinline__ TileOffs16 tile_offs16(int lane) {
  TileOffs16 o;
  const int g = lane >> 4, c = lane & 15, s = c >> 2, t = c & 3;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) o.row[ks] = 2u * static_cast<uint32_t>(swz_off(c, 32 * g + 8 * ks));
#pragma unroll
  for (int md = 0; md < 8; ++md) o.tr[md] = 2u * static_cast<uint32_t>(swz_off(4 * g + s, 16 * md + 4 * t));
  return o;
}

// A operand of k-step kk whose m index is column 16·md + lane % 16: rows
// 32kk + 4g + 0..3 (slots 0-3) and 32kk + 16 + 4g + 0..3 (slots 4-7).
__device__ __forceinline__ uint4 lds_kmajor16(const uint16_t* tile, const TileOffs16& o, int kk, int md) {
  const char* base = reinterpret_cast<const char*>(tile) + kk * 32 * 256;
  lds_bf16x4_t* plo = (lds_bf16x4_t*)(const_cast<char*>(base + o.tr[md]));
  lds_bf16x4_t* phi = (lds_bf16x4_t*)(const_cast<char*>(base + 16 * 256 + o.tr[md]));
  const uint2 lo = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(plo));
  const uint2 hi = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(phi));
  return make_uint4(lo.x, lo.y, hi.x, hi.y);
}

__device__ __forceinline__ uint4 lds_row16(const uint16_t* tile, const TileOffs16& o, int mb, int ks) {
  return *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(tile) + mb * 16 * 256 + o.row[ks]);
}

// One 64-row query tile against this wavefront's 16 keys, first part:
// per-row offsets, S and dP, then P and dS as bf16 B operands.
// With DP, the tile's dS values are added to this lane's running sum dacc
// (reduced over the wavefront once per list entry by the caller).
// Token modes add the key-feature term: the query features [hi | lo] of a
// row (one k=32 operand, b.rb) against [k_hi | k_hi] (kf[0]) and [k_lo | 0]
// (kf[1]) give q_hi·k_hi + q_lo·k_hi + q_hi·k_lo in two MFMAs; eb is the
// pair bias of the tile's list entry (log2 units).
template <int MODE, bool DP>
__device__ __forceinline__ void dkv16_a(const AttnArgs& a, const DkvBuf<MODE>& b, bool masked, int q0, int lane,
                                        int wkv, int doc_kv, const uint4 (&kreg)[4], const uint4 (&vreg)[4],
                                        const uint4 (&kf)[2], float eb, const TileOffs16& to, uint4 (&pb)[2],
                                        uint4 (&dsb)[2], float& dacc) {
  const int g = lane >> 4;
  f32x4_t s[4], dp[4];
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) {
    s[mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    // dP - Δ: the accumulator of rows 16mb + 4g .. +3 starts from their -Δ (stored negated)
    dp[mb] = *reinterpret_cast<const f32x4_t*>(&b.ra[64 + 16 * mb + 4 * g]);
  }
  // step st = 4·ks + mb; operands read RA steps ahead into a ring
  constexpr int RA = 2;
  uint4 qa[RA + 1], da[RA + 1];
#pragma unroll
  for (int i = 0; i < RA; ++i) {
    qa[i] = lds_row16(b.q, to, i % 4, i / 4);
    da[i] = lds_row16(b.d, to, i % 4, i / 4);
  }
#pragma unroll
  for (int st = 0; st < 16; ++st) {
    const int ks = st / 4, mb = st % 4;
    if (st + RA < 16) {
      qa[(st + RA) % (RA + 1)] = lds_row16(b.q, to, (st + RA) % 4, (st + RA) / 4);
      da[(st + RA) % (RA + 1)] = lds_row16(b.d, to, (st + RA) % 4, (st + RA) / 4);
    }
    s[mb] = mfma16(qa[st % (RA + 1)], kreg[ks], s[mb]);
    dp[mb] = mfma16(da[st % (RA + 1)], vreg[ks], dp[mb]);
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
  if constexpr (MODE >= 2) {
    const uint16_t* qf = reinterpret_cast<const uint16_t*>(b.rb);
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) {
      const uint4 fa = lds_row8_32(qf, 16 * mb + (lane & 15), 8 * g);
      s[mb] = mfma16(fa, kf[0], s[mb]);
      s[mb] = mfma16(fa, kf[1], s[mb]);
    }
  }
  // modes 0/1: the tile's softmax offsets (block term, pair bias and lse per row) are in b.ra[0..63]
  if (masked)
    dkv16_probs<MODE, true, DP>(a, b, b.ra, eb, a.scale_log2, q0, wkv, doc_kv, g, s, dp, pb, dsb, dacc);
  else
    dkv16_probs<MODE, false, DP>(a, b, b.ra, eb, a.scale_log2, q0, wkv, doc_kv, g, s, dp, pb, dsb, dacc);
}

// Second part: dV^T += dO^T P, dK^T += Q^T dS (step st = 8·kk + md).
template <int MODE>
__device__ __forceinline__ void dkv16_b(const DkvBuf<MODE>& b, const TileOffs16& to, const uint4 (&pb)[2],
                                        const uint4 (&dsb)[2], f32x4_t (&dvT)[8], f32x4_t (&dkT)[8]) {
  constexpr int RB = 2;
  uint4 ta[RB + 1], tb[RB + 1];
#pragma unroll
  for (int i = 0; i < RB; ++i) {
    ta[i] = lds_kmajor16(b.d, to, i / 8, i % 8);
    tb[i] = lds_kmajor16(b.q, to, i / 8, i % 8);
  }
#pragma unroll
  for (int st = 0; st < 16; ++st) {
    const int kk = st / 8, md = st % 8;
    if (st + RB < 16) {
      ta[(st + RB) % (RB + 1)] = lds_kmajor16(b.d, to, (st + RB) / 8, (st + RB) % 8);
      tb[(st + RB) % (RB + 1)] = lds_kmajor16(b.q, to, (st + RB) / 8, (st + RB) % 8);
    }
    dvT[md] = mfma16(ta[st % (RB + 1)], pb[kk], dvT[md]);
    dkT[md] = mfma16(tb[st % (RB + 1)], dsb[kk], dkT[md]);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <int BS, int MODE, bool DP>
__global__ __launch_bounds__(512) void attn_bwd_dkv16_kernel(AttnArgs a, KvPlan pl) {
  constexpr int D = 128;
  constexpr int BM = 64;  // query rows per staged tile
  constexpr int NS = BS / BM;

  __shared__ DkvBuf<MODE> buf0, buf1, buf2;
  __shared__ int qbs[kChunkMax], dse[kChunkMax], epos[kChunkMax];
  __shared__ float pslot[kChunkMax][8];  // pair-bias gradient: per entry and wavefront

  constexpr int P = BS / 128;  // workgroups (128 keys each) per key block
  const int NB = a.QB;
  // 1-D grid, XCD-aware, as attn_bwd_dkv_kernel
  const int L = blockIdx.x;
  const int per_xcd = gridDim.x / 8 / P;
  const int pair = (L / 8) / P, zpart = (L / 8) % P;
  const int item = (L % 8) * per_xcd + pair;
  if (item >= a.H * pl.max_items) return;
  const int h = item / pl.max_items;
  const int x = item % pl.max_items;
  const int32_t* its = pl.items_start + static_cast<int64_t>(h) * (NB + 1);
  if (x >= its[NB]) return;
  int lo = 0, hi = NB - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) / 2;
    if (its[mid] <= x) lo = mid;
    else hi = mid - 1;
  }
  const int kb = lo;
  const int chunk = x - its[kb];
  const int32_t* qo = a.q_off + static_cast<int64_t>(h) * (NB + 1);
  const int nq = qo[kb + 1] - qo[kb];
  const int CH = pl.chunk;
  const int nch = max(1, (nq + CH - 1) / CH);
  const int i0 = chunk * CH, i1 = min(nq, i0 + CH);
  const int ne = max(0, i1 - i0);
  const int32_t* ql = a.q_list + static_cast<int64_t>(h) * a.QB * a.maxkv + qo[kb];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid % 64, g = lane / 16, c = lane % 16;
  const int64_t kv0 = static_cast<int64_t>(kb) * BS + zpart * 128;  // first key row of this workgroup
  const int wkv_lo = static_cast<int>(kv0) + wave * 16;
  const int wkv = wkv_lo + c;
  const int krow = zpart * 128 + wave * 16 + c;  // key row within the block
  const int64_t hT = static_cast<int64_t>(h) * a.T;

  const int qb_first = ne > 0 ? ql[i0] : 0;
  const int skip0 = ne > 0 && qb_first == kb ? (zpart * 128) / BM : 0;
  const int n_it = ne * NS - skip0;

  if (tid < ne) {
    const int qb = ql[i0 + tid];
    qbs[tid] = qb;
    dse[tid] = a.ds_tok_end[qb];
    // position of kb in this q-block's list: its offsets rows in roff
    epos[tid] = pl.q_pos[static_cast<int64_t>(h) * a.QB * a.maxkv + qo[kb] + i0 + tid];
  }
  for (int t = tid; DP && t < CH * 8; t += blockDim.x) pslot[t / 8][t % 8] = 0.f;
  __syncthreads();  // qbs, epos
  // the offsets of tile j (q-block qbs[e], rows (f % NS)·64 .. +63 of the list entry)
  auto tile_rof = [&](int j) __attribute__((always_inline)) -> const float* {
    if constexpr (MODE >= 2) return nullptr;  // token modes: per-row constants, no stored offsets
    const int f = j + skip0, e = f / NS;
    return a.roff + ((static_cast<int64_t>(h) * a.QB + qbs[e]) * a.maxkv + epos[e]) * BS + (f % NS) * BM;
  };
  if (n_it > 0 && wave < 4) {
    const int64_t q0 = static_cast<int64_t>(qb_first) * BS + (skip0 % NS) * BM;
    dkv_issue<MODE>(a, h, hT, q0, tile_rof(0), buf0, tid);
  }

  uint4 kreg[4], vreg[4];
  {
    // k-step ks: columns 32g + 8ks .. +7, the order of the row reads
    const uint16_t* kp = a.k + h * a.k_sh + static_cast<int64_t>(wkv) * a.k_st + g * 32;
    const uint16_t* vp = a.v + h * a.v_sh + static_cast<int64_t>(wkv) * a.v_st + g * 32;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      kreg[ks] = *reinterpret_cast<const uint4*>(kp + ks * 8);
      vreg[ks] = *reinterpret_cast<const uint4*>(vp + ks * 8);
    }
  }
  const int doc_kv = a.docs[wkv];
  const TileOffs16 to = tile_offs16(lane);
  // token modes: this lane's key features as B operands (see dkv16_a); the
  // table row of key j is cos hi[8], sin hi[8], cos lo[8], sin lo[8]
  uint4 kf[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
  if constexpr (MODE >= 2) {
    const uint16_t* tr = static_cast<const uint16_t*>(a.table) + static_cast<int64_t>(wkv) * kTokRow;
    kf[0] = *reinterpret_cast<const uint4*>(tr + 8 * (g & 1));
    if (g < 2) kf[1] = *reinterpret_cast<const uint4*>(tr + 16 + 8 * g);
  }
  const bool pbias = MODE >= 2 && a.pair_bias != nullptr;

  f32x4_t dvT[8], dkT[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    dvT[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    dkT[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  auto tile_q0 = [&](int j, int& e) __attribute__((always_inline)) {
    const int f = j + skip0;
    e = f / NS;
    return qbs[e] * BS + (f % NS) * BM;
  };
  // Wavefronts 0-3 (one per SIMD) process whole tiles and copy them into
  // three rotating buffers (256 threads); wavefronts 4-7 run half a tile
  // behind: their k-th barrier falls between the first and the second part
  // of tile k-1, so each SIMD holds one wavefront in its probabilities while
  // the other runs MFMAs.  At the leading group's k-th barrier the lagging
  // group is done with tile k-2, whose buffer then takes tile k+1.  Both
  // groups pass n_it + 1 barriers.
  // pair-bias gradient: this lane's running dS sum of list entry dcur,
  // reduced over the wavefront when the entry changes (a wavefront takes the
  // entries in order, each entry's tiles back to back)
  float dacc = 0.f;
  int dcur = -1;
  auto flush = [&]() __attribute__((always_inline)) {
    if (dcur >= 0) {
      const float t = wave_sum(dacc);
      if (lane == 0) pslot[dcur][wave] += t;
    }
    dacc = 0.f;
  };
  auto part_a = [&](const DkvBuf<MODE>& bc, int j, uint4 (&pb)[2], uint4 (&dsb)[2]) __attribute__((always_inline)) {
    int e;
    const int q0 = tile_q0(j, e);
    if (q0 + BM - 1 < wkv_lo) return false;  // every query row precedes this wavefront's keys
    if (DP && e != dcur) {
      flush();
      dcur = e;
    }
    const bool masked = !((wkv_lo + 15 <= q0) && (dse[e] <= wkv_lo));
    // token modes: the pair bias of the list entry (modes 0/1 have it in the stored offsets)
    const float eb = pbias && epos[e] >= 0
                         ? a.pair_bias[(static_cast<int64_t>(h) * a.QB + qbs[e]) * a.maxkv + epos[e]] * kLog2e
                         : 0.f;
    dkv16_a<MODE, DP>(a, bc, masked, q0, lane, wkv, doc_kv, kreg, vreg, kf, eb, to, pb, dsb, dacc);
    return true;
  };
  if (wave < 4) {
    int j = 0;
    auto lead = [&](const DkvBuf<MODE>& bc, DkvBuf<MODE>& bn) __attribute__((always_inline)) {
      wait_vm0();
      __syncthreads();  // tile j is in bc for everyone; the lagging group is done with bn
      if (j + 1 < n_it) {
        int en;
        dkv_issue<MODE>(a, h, hT, tile_q0(j + 1, en), tile_rof(j + 1), bn, tid);
      }
      uint4 pb[2], dsb[2];
      if (part_a(bc, j, pb, dsb)) dkv16_b<MODE>(bc, to, pb, dsb, dvT, dkT);
      ++j;
    };
    while (j < n_it) {
      lead(buf0, buf1);
      if (j >= n_it) break;
      lead(buf1, buf2);
      if (j >= n_it) break;
      lead(buf2, buf0);
    }
    __syncthreads();  // matches the lagging group's last barrier
  } else {
    __syncthreads();  // tile 0 is in buf0
    int j = 0;
    auto lag = [&](const DkvBuf<MODE>& bc) __attribute__((always_inline)) {
      uint4 pb[2], dsb[2];
      const bool act = part_a(bc, j, pb, dsb);
      __syncthreads();  // the leading group starts the next tile
      if (act) dkv16_b<MODE>(bc, to, pb, dsb, dvT, dkT);
      ++j;
    };
    while (j < n_it) {
      lag(buf0);
      if (j >= n_it) break;
      lag(buf1);
      if (j >= n_it) break;
      lag(buf2);
    }
  }
  wait_vm0();  // no copy may still target LDS when the workgroup exits
  if (DP) {
    flush();
    __syncthreads();  // every wavefront's slots are final
  }
  if (DP && tid < ne && epos[tid] >= 0) {
    float t = 0.f;
#pragma unroll
    for (int w = 0; w < 8; ++w) t += pslot[tid][w];
    const int64_t row = static_cast<int64_t>(h) * a.QB + qbs[tid];
    a.dpair[(static_cast<int64_t>(zpart) * a.H * a.QB + row) * a.maxkv + epos[tid]] = t;
  }

  // ---- write dK = scale·dkT^T, dV = dvT^T: lane holds columns 16md + 4g .. +3 of key wkv
  if (nch == 1) {
    uint16_t* dkp = a.dk + h * a.k_sh + static_cast<int64_t>(wkv) * a.k_st + 4 * g;
    uint16_t* dvp = a.dv + h * a.v_sh + static_cast<int64_t>(wkv) * a.v_st + 4 * g;
#pragma unroll
    for (int md = 0; md < 8; ++md) {
      uint2 vk, vv;
      vk.x = cvt_pk_bf16(dkT[md][0] * a.scale, dkT[md][1] * a.scale);
      vk.y = cvt_pk_bf16(dkT[md][2] * a.scale, dkT[md][3] * a.scale);
      vv.x = cvt_pk_bf16(dvT[md][0], dvT[md][1]);
      vv.y = cvt_pk_bf16(dvT[md][2], dvT[md][3]);
      *reinterpret_cast<uint2*>(dkp + md * 16) = vk;
      *reinterpret_cast<uint2*>(dvp + md * 16) = vv;
    }
  } else {
    const int64_t slot = h * pl.max_slots + pl.slots_start[static_cast<int64_t>(h) * (NB + 1) + kb] + chunk;
    float* pk = pl.part_dk + (slot * BS + krow) * D + 4 * g;
    float* pv = pl.part_dv + (slot * BS + krow) * D + 4 * g;
#pragma unroll
    for (int md = 0; md < 8; ++md) {
      *reinterpret_cast<float4*>(pk + md * 16) = make_float4(dkT[md][0], dkT[md][1], dkT[md][2], dkT[md][3]);
      *reinterpret_cast<float4*>(pv + md * 16) = make_float4(dvT[md][0], dvT[md][1], dvT[md][2], dvT[md][3]);
    }
  }
}

// ---------------------------------------------------------------------------
// pass A, 16 query rows per wavefront (two wavefronts per SIMD, any mode)
// ---------------------------------------------------------------------------
// Transpose read of a 64 x 32 feature tile (swz32_off) as the A operand of a
// 16x16x32 MFMA: m = feature 16·fb + lane % 16, k = the keys of k-step kk in
// the slot order of lds_kmajor16 (rows 32kk + 4g + 0..3, then 32kk + 16 + 4g
// + 0..3).
__device__ __forceinline__ uint4 lds_kmajor16_32(const uint16_t* tile, int kk, int fb, int lane) {
  const int g = lane >> 4, j = lane & 15, s = j >> 2, t = j & 3;
  const int r0 = 32 * kk + 4 * g + s, d = 16 * fb + 4 * t;
  lds_bf16x4_t* plo = (lds_bf16x4_t*)(const_cast<uint16_t*>(tile + swz32_off(r0, d)));
  lds_bf16x4_t* phi = (lds_bf16x4_t*)(const_cast<uint16_t*>(tile + swz32_off(r0 + 16, d)));
  const uint2 lo = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(plo));
  const uint2 hi = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(phi));
  return make_uint4(lo.x, lo.y, hi.x, hi.y);
}

// x summed over the four lane groups of 16 (lanes l, l ^ 16, l ^ 32, l ^ 48)
__device__ __forceinline__ float sum_groups16(float x) {
  x += __shfl_xor(x, 16, 64);
  return x + xor32(x);
}

// The q-major pass with 16 query rows per wavefront on v_mfma_f32_16x16x32_bf16:
// lane l owns query row l % 16 of its wavefront and, in every 16-key block of
// a tile, the keys 4g .. 4g+3 (g = l / 16).  S^T = K·Q^T and dP^T = V·dO^T
// per 16-key block (K, V rows from the tile, Q and dO of the lane's row in
// registers; dP starts from -Δ), the token modes' key features as two k=32
// MFMAs (the table row [k_hi | k_lo] against [q_hi | q_hi] and [q_lo | 0]),
// then dQ^T += K^T·dS^T and, in token modes, the feature gradient
// dF^T += F^T·dS^T (and its P-weighted twin for the Δ correction) from
// transpose reads.  Eight wavefronts (128 rows) per workgroup, two per SIMD;
// every mode, both block sizes (the gated mode takes a tile's four 16-key
// blocks in two halves to fit its registers).  It stores Δ_true (negated) and,
// in modes 0/1, every row's softmax offset per listed key block for the
// kv-major pass, and the token modes' query features.
template <int BS, int MODE>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_bwd_dq16_kernel(AttnArgs a) {
  constexpr int SPLIT = BS / 128;  // workgroups per q-block (8 wavefronts = 128 query rows each)
  constexpr int BN = 64;           // keys per staged tile
  constexpr int NSUB = BS / BN;
  constexpr int NT = 512;
  constexpr bool TOK = MODE >= 2, GATE = MODE == 3;

  // the gated mode runs its wavefronts in step (the staggered loop's second
  // code path would cost it registers it does not have)
  constexpr bool STAGGER = !GATE;
  __shared__ KvTile<MODE> buf0, buf1;
  __shared__ typename std::conditional<STAGGER, KvTile<MODE>, int>::type buf2;
  __shared__ int kbs[kListLds];
  __shared__ float kbias[kListLds];  // pair bias per list entry (log2 units), when given

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid % 64, g = lane / 16, c = lane % 16;
  const int tile = xcd_remap(blockIdx.x, gridDim.x);
  const int h = tile / (a.QB * SPLIT), qb = (tile / SPLIT) % a.QB, part = tile % SPLIT;
  const int64_t q0 = static_cast<int64_t>(qb) * BS + part * 128;
  const int wrow_lo = static_cast<int>(q0) + wave * 16;
  const int64_t hT = static_cast<int64_t>(h) * a.T;
  const int row = wrow_lo + c;

  const int64_t lrow = static_cast<int64_t>(h) * a.QB + qb;
  const int n = min(a.kv_num[lrow], a.maxkv);  // maxkv <= kListLds
  const int32_t* lst = a.kv_idx + lrow * a.maxkv;
  for (int t = tid; t < min(n, kListLds); t += NT) kbs[t] = lst[t];
  const bool pbias = a.pair_bias != nullptr;
  if (pbias)
    for (int t = tid; t < min(n, kListLds); t += NT) kbias[t] = a.pair_bias[lrow * a.maxkv + t] * kLog2e;

  // Q and dO of this lane's row, k-step ks: columns 32g + 8ks .. +7 (the order of the row reads)
  uint4 qreg[4], doreg[4];
  float delta;
  {
    const uint16_t* qp = a.q + h * a.q_sh + static_cast<int64_t>(row) * a.q_st + g * 32;
    const uint16_t* op = a.o + h * a.o_sh + static_cast<int64_t>(row) * a.o_st + g * 32;
    const uint16_t* dp = a.dout + h * a.o_sh + static_cast<int64_t>(row) * a.o_st + g * 32;
    float dsum = 0.f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      qreg[ks] = *reinterpret_cast<const uint4*>(qp + ks * 8);
      doreg[ks] = *reinterpret_cast<const uint4*>(dp + ks * 8);
      const uint4 ov = *reinterpret_cast<const uint4*>(op + ks * 8);
      const uint32_t dw[4] = {doreg[ks].x, doreg[ks].y, doreg[ks].z, doreg[ks].w};
      const uint32_t ow[4] = {ov.x, ov.y, ov.z, ov.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dsum += __uint_as_float(dw[i] << 16) * __uint_as_float(ow[i] << 16);
        dsum += __uint_as_float(dw[i] & 0xffff0000u) * __uint_as_float(ow[i] & 0xffff0000u);
      }
    }
    delta = sum_groups16(dsum);
  }
  const float lse_nat = a.lse[hT + row];
  const float lse2 = lse_nat == -INFINITY ? INFINITY : lse_nat * kLog2e;
  const int doc = a.docs[row];

  // ---- bias set-up (as in the forward)
  float ca[8], sa[8];
  uint4 qf1 = make_uint4(0, 0, 0, 0), qf2 = make_uint4(0, 0, 0, 0);
  float rowc = 0.f, slp = 0.f, dm = 0.f, wd = 0.f;
  // token mode: cos/sin(ω_k row) of the bands k = 4g..4g+3 are read again in the
  // epilogue (keeping them live through the tile loop costs registers)
  if (MODE == 1) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      ca[k] = k < a.K ? a.coeff_cos[(hT + row) * a.K + k] * a.beta_log2 : 0.f;
      sa[k] = k < a.K ? a.coeff_sin[(hT + row) * a.K + k] * a.beta_log2 : 0.f;
    }
  }
  if (TOK) {
    // the row's features: half g % 2 (cos half, sin half), hi and lo bf16 parts
    uint4 hi, lo;
    token_qfeat(a, hT, row, g & 1, hi, lo, nullptr, nullptr);
    qf1 = hi;                                     // [q_hi | q_hi]
    if (g < 2) qf2 = lo;                          // [q_lo | 0]
    if (g < 2) {
      // kept for the kv-major pass, which stages them per query tile
      *reinterpret_cast<uint4*>(a.qfeat + (hT + row) * kTokRow + g * 8) = hi;
      *reinterpret_cast<uint4*>(a.qfeat + (hT + row) * kTokRow + 16 + g * 8) = lo;
    }
    if (a.subtract_b0) rowc = -a.beta_log2 * a.b0[hT + row];
    if (a.use_slope) slp = a.beta_log2 * a.slope[hT + row];
    if (GATE) {
      dm = a.delta_main[hT + row];
      wd = a.width[hT + row];
    }
  }
  const int ds_end = a.ds_tok_end[qb];
  const TileOffs16 to = tile_offs16(lane);

  f32x4_t dqT[8];  // dQ^T: D rows 16·md + 4g + r, this lane's query row
#pragma unroll
  for (int i = 0; i < 8; ++i) dqT[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // Bias gradients use Δ_true = Σ_j P dP rather than the Δ of the bf16
  // output: since Σ_j P = 1, the row total Σ_j dS equals Δ_true - Δ, so each
  // per-tile sum is corrected by subtracting that total times the tile's
  // probability mass (every sum has a P-weighted twin).  All stay per lane
  // (a quarter of the row's keys) until the epilogue.
  f32x4_t facc[2], facc_p[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) facc[i] = facc_p[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  float accA[8], accB[8], accPA[8], accPB[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) accA[k] = accB[k] = accPA[k] = accPB[k] = 0.f;
  float rs_tot = 0.f, pm_tot = 0.f;
  float ex[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};  // Σ dS·df, dS·σ·sgn, dS·σ, then the P-weighted three

  const int total = n * NSUB;
  const int qmax = static_cast<int>(q0) + 127;
  auto kb_at = [&](int t) __attribute__((always_inline)) { return kbs[t]; };
  auto next_valid = [&](int it) __attribute__((always_inline)) {
    while (it < total && kb_at(it / NSUB) * BS + (it % NSUB) * BN > qmax) ++it;
    return it;
  };
  float bt = 0.f, rs_kb = 0.f, pm_kb = 0.f;
  float eb = 0.f;  // pair bias of the current list entry (log2 units)
  const float cs = a.scale_log2;
  // part A of a tile: S, dP, the probabilities and dS (B operands dsb, pb) and the row sums
  auto compute_a = [&](int kv0, const KvTile<MODE>& b, uint4 (&dsb)[2], uint4 (&pb)[2])
                       __attribute__((always_inline)) {
    const bool full = (kv0 + BN - 1 <= wrow_lo) && (ds_end <= kv0);
    const float off = (MODE == 1 ? bt : rowc) + eb - lse2;
    // probabilities and dS^T: key j = 16·kb4 + 4g + r of the tile
    const int lim = row - kv0;  // keys j <= lim are causal
    const float dfl = static_cast<float>(lim - 4 * g);
    const bool softplus = a.gate_kind == SCOPE_GATE_SOFTPLUS;
    const float glam = a.beta_log2 * a.ramp_lambda;
    float rs = 0.f, pm = 0.f;
    uint32_t dw[8], pw[8];
    // The gated mode takes the tile's four 16-key blocks in two halves (the
    // S and dP accumulators of two blocks live at a time); the others at once.
    constexpr int NH = GATE ? 2 : 1, KB = 4 / NH;
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) {
      // S^T and dP^T - Δ per 16-key block kb4 = KB·hh + kl (step st = KB·ks + kl),
      // operands RA steps ahead
      f32x4_t s[KB], dp[KB];
#pragma unroll
      for (int kl = 0; kl < KB; ++kl) {
        s[kl] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        dp[kl] = f32x4_t{-delta, -delta, -delta, -delta};
      }
      constexpr int RA = 2;
      constexpr int NST = 4 * KB;
      uint4 ka[RA + 1], va[RA + 1];
#pragma unroll
      for (int i = 0; i < RA; ++i) {
        ka[i] = lds_row16(b.k, to, KB * hh + i % KB, i / KB);
        va[i] = lds_row16(b.v, to, KB * hh + i % KB, i / KB);
      }
#pragma unroll
      for (int st = 0; st < NST; ++st) {
        const int ks = st / KB, kl = st % KB;
        if (st + RA < NST) {
          ka[(st + RA) % (RA + 1)] = lds_row16(b.k, to, KB * hh + (st + RA) % KB, (st + RA) / KB);
          va[(st + RA) % (RA + 1)] = lds_row16(b.v, to, KB * hh + (st + RA) % KB, (st + RA) / KB);
        }
        s[kl] = mfma16(ka[st % (RA + 1)], qreg[ks], s[kl]);
        dp[kl] = mfma16(va[st % (RA + 1)], doreg[ks], dp[kl]);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (TOK) {
#pragma unroll
        for (int kl = 0; kl < KB; ++kl) {
          const uint4 fa = lds_row8_32(b.f, 16 * (KB * hh + kl) + c, 8 * g);
          s[kl] = mfma16(fa, qf1, s[kl]);
          s[kl] = mfma16(fa, qf2, s[kl]);
        }
      }
      // the causal and document mask only on the tiles that need it (a
      // mask-free copy for the rest, in every mode)
      auto probs = [&](auto mask_tag) __attribute__((always_inline)) {
        constexpr bool MASK = decltype(mask_tag)::value;
#pragma unroll
        for (int kl = 0; kl < KB; ++kl) {
          const int kb4 = KB * hh + kl;
          int dcv[4] = {0, 0, 0, 0};
          if (MASK) {
            const int4 d4 = *reinterpret_cast<const int4*>(&b.docs[16 * kb4 + 4 * g]);
            dcv[0] = d4.x, dcv[1] = d4.y, dcv[2] = d4.z, dcv[3] = d4.w;
          }
          float dv[4], pv[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int j = 16 * kb4 + 4 * g + r;
            float x;
            float sig = 0.f, sgn = 0.f, df = 0.f;
            if (TOK) {
              df = dfl - static_cast<float>(16 * kb4 + r);  // lim - j, exact in fp32
              float e = slp * df;
              if (GATE) {
                const float dd = df - dm;
                const float xx = (fabsf(dd) - wd) * a.inv_tau;
                const float en = __builtin_amdgcn_exp2f(-fabsf(xx) * kLog2e);
                const float inv = __builtin_amdgcn_rcpf(1.f + en);
                const float lp = kLn2 * __builtin_amdgcn_logf(1.f + en);
                const float gt = fmaxf(xx, 0.f) + (softplus ? lp : 0.f);
                sig = softplus ? (xx >= 0.f ? inv : en * inv) : (xx > 0.f ? 1.f : 0.f);
                sgn = dd > 0.f ? 1.f : (dd < 0.f ? -1.f : 0.f);
                e -= glam * gt;
              }
              x = fmaf(s[kl][r], cs, e + off);
            } else {
              x = fmaf(s[kl][r], cs, off);
            }
            if (MASK) x = mask_score(x, j, lim, dcv[r], doc);
            const float p = __builtin_amdgcn_exp2f(x);
            const float d = p * dp[kl][r];  // dP accumulator started from -Δ
            dv[r] = d;
            pv[r] = p;
            rs += d;
            pm += p;
            if (TOK) {
              ex[0] += d * df;
              ex[3] += p * df;
              if (GATE) {
                ex[1] += d * sig * sgn;
                ex[2] += d * sig;
                ex[4] += p * sig * sgn;
                ex[5] += p * sig;
              }
            }
          }
          dw[2 * kb4] = cvt_pk_bf16(dv[0], dv[1]);
          dw[2 * kb4 + 1] = cvt_pk_bf16(dv[2], dv[3]);
          pw[2 * kb4] = cvt_pk_bf16(pv[0], pv[1]);
          pw[2 * kb4 + 1] = cvt_pk_bf16(pv[2], pv[3]);
        }
      };
      if (full) probs(std::false_type{});
      else probs(std::true_type{});
    }
    // B operands of k-step kk: blocks 2kk (slots 0-3) and 2kk+1 (slots 4-7)
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      dsb[kk] = make_uint4(dw[4 * kk], dw[4 * kk + 1], dw[4 * kk + 2], dw[4 * kk + 3]);
      pb[kk] = make_uint4(pw[4 * kk], pw[4 * kk + 1], pw[4 * kk + 2], pw[4 * kk + 3]);
    }
    rs_kb += rs;
    pm_kb += pm;
    rs_tot += rs;
    pm_tot += pm;
  };
  // part B: dQ^T += K^T dS^T and, token modes, the feature gradients
  auto compute_b = [&](const KvTile<MODE>& b, const uint4 (&dsb)[2], const uint4 (&pb)[2])
                       __attribute__((always_inline)) {
    // dQ^T += K^T dS^T (step st = 8·kk + md), operands two steps ahead
    {
      constexpr int RB = 2;
      uint4 ta[RB + 1];
#pragma unroll
      for (int i = 0; i < RB; ++i) ta[i] = lds_kmajor16(b.k, to, i / 8, i % 8);
#pragma unroll
      for (int st = 0; st < 16; ++st) {
        const int kk = st / 8, md = st % 8;
        if (st + RB < 16) ta[(st + RB) % (RB + 1)] = lds_kmajor16(b.k, to, (st + RB) / 8, (st + RB) % 8);
        dqT[md] = mfma16(ta[st % (RB + 1)], dsb[kk], dqT[md]);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (TOK) {
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
#pragma unroll
        for (int fb = 0; fb < 2; ++fb) {
          const uint4 ft = lds_kmajor16_32(b.f, kk, fb, lane);
          facc[fb] = mfma16(ft, dsb[kk], facc[fb]);
          facc_p[fb] = mfma16(ft, pb[kk], facc_p[fb]);
        }
    }
  };
  // part A of tile it with the block-mode bookkeeping; false when the
  // wavefront has nothing to do for this tile
  auto run_a = [&](int it, int nxt, const KvTile<MODE>& b, uint4 (&dsb)[2], uint4 (&pb)[2])
                   __attribute__((always_inline)) -> bool {
    const int kv0 = kb_at(it / NSUB) * BS + (it % NSUB) * BN;
    if (MODE == 1 && it % NSUB == 0) {
      // a key block's first tile is never skipped (it starts at or before every row)
      const float4* t4 = reinterpret_cast<const float4*>(b.tab);
      const float4 c0 = t4[0], c1 = t4[1], s0 = t4[2], s1 = t4[3];
      bt = (ca[0] * c0.x + ca[1] * c0.y + ca[2] * c0.z + ca[3] * c0.w) +
           (ca[4] * c1.x + ca[5] * c1.y + ca[6] * c1.z + ca[7] * c1.w) +
           (sa[0] * s0.x + sa[1] * s0.y + sa[2] * s0.z + sa[3] * s0.w) +
           (sa[4] * s1.x + sa[5] * s1.y + sa[6] * s1.z + sa[7] * s1.w);
    }
    if (it % NSUB == 0) eb = pbias ? kbias[it / NSUB] : 0.f;  // per key block (its first tile is never skipped)
    const bool act = kv0 <= wrow_lo + 15;  // else every key follows this wavefront's rows
    if (act) compute_a(kv0, b, dsb, pb);
    if (MODE == 1 && (nxt >= total || nxt / NSUB != it / NSUB)) {
      // last tile of this key block: fold its sums into the coefficient gradients
      const float4* t4 = reinterpret_cast<const float4*>(b.tab);
      const float tb[16] = {t4[0].x, t4[0].y, t4[0].z, t4[0].w, t4[1].x, t4[1].y, t4[1].z, t4[1].w,
                            t4[2].x, t4[2].y, t4[2].z, t4[2].w, t4[3].x, t4[3].y, t4[3].z, t4[3].w};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        accA[k] += rs_kb * tb[k];
        accB[k] += rs_kb * tb[8 + k];
        accPA[k] += pm_kb * tb[k];
        accPB[k] += pm_kb * tb[8 + k];
      }
      rs_kb = pm_kb = 0.f;
    }
    return act;
  };

  __syncthreads();  // kbs, kbias
  // Wavefronts 0-3 (one per SIMD) process whole tiles and copy them (256
  // threads) into three rotating buffers; wavefronts 4-7 run part of a tile
  // behind: their k-th barrier falls between part A and part B of tile k-1,
  // so the two wavefronts of a SIMD are not in the same phase.  At the
  // leading group's k-th barrier the lagging group is done with tile k-2,
  // whose buffer then takes tile k+1.  Both groups pass n+1 barriers for n
  // tiles.
  const int tid4 = tid & 255;
  auto issue4 = [&](int it, KvTile<MODE>& b) __attribute__((always_inline)) {
    const int kb = kb_at(it / NSUB);
    const int rd = min(max(qb - kb, 0), a.QB - 1);
    kv_issue<MODE, 256>(a, h, static_cast<int64_t>(kb) * BS + (it % NSUB) * BN, rd, b, tid4);
  };
  int cur = next_valid(0);
  if constexpr (!STAGGER) {
    auto issue = [&](int it, KvTile<MODE>& b) __attribute__((always_inline)) {
      const int kb = kb_at(it / NSUB);
      const int rd = min(max(qb - kb, 0), a.QB - 1);
      kv_issue<MODE, NT>(a, h, static_cast<int64_t>(kb) * BS + (it % NSUB) * BN, rd, b, tid);
    };
    auto step = [&](const KvTile<MODE>& bc, KvTile<MODE>& bn) __attribute__((always_inline)) {
      wait_vm0();
      __syncthreads();  // tile cur is in bc; every wavefront is done with bn
      const int nxt = next_valid(cur + 1);
      if (nxt < total) issue(nxt, bn);
      uint4 dsb[2], pb[2];
      if (run_a(cur, nxt, bc, dsb, pb)) compute_b(bc, dsb, pb);
      cur = nxt;
    };
    if (cur < total) issue(cur, buf0);
    while (cur < total) {
      step(buf0, buf1);
      if (cur >= total) break;
      step(buf1, buf0);
    }
  } else if (wave < 4) {
    if (cur < total) issue4(cur, buf0);
    auto lead = [&](const KvTile<MODE>& bc, KvTile<MODE>& bn) __attribute__((always_inline)) {
      wait_vm0();
      __syncthreads();  // tile cur is in bc for everyone; the lagging group is done with bn
      const int nxt = next_valid(cur + 1);
      if (nxt < total) issue4(nxt, bn);
      uint4 dsb[2], pb[2];
      if (run_a(cur, nxt, bc, dsb, pb)) compute_b(bc, dsb, pb);
      cur = nxt;
    };
    if constexpr (STAGGER) {
      while (cur < total) {
        lead(buf0, buf1);
        if (cur >= total) break;
        lead(buf1, buf2);
        if (cur >= total) break;
        lead(buf2, buf0);
      }
    }
    __syncthreads();  // matches the lagging group's last barrier
  } else {
    __syncthreads();  // tile 0 is in buf0
    auto lag = [&](const KvTile<MODE>& bc) __attribute__((always_inline)) {
      const int nxt = next_valid(cur + 1);
      uint4 dsb[2], pb[2];
      const bool act = run_a(cur, nxt, bc, dsb, pb);
      __syncthreads();  // the leading group starts the next tile
      if (act) compute_b(bc, dsb, pb);
      cur = nxt;
    };
    if constexpr (STAGGER) {
      while (cur < total) {
        lag(buf0);
        if (cur >= total) break;
        lag(buf1);
        if (cur >= total) break;
        lag(buf2);
      }
    }
  }
  wait_vm0();  // no copy may still target LDS when the workgroup exits

  // ---- epilogue: sums over the four lane groups of a row, dQ = scale·o
  rs_tot = sum_groups16(rs_tot);
  pm_tot = sum_groups16(pm_tot);
  const float dd_err = rs_tot;  // Δ_true - Δ
  // the kv-major pass reads Δ_true = Δ + (Δ_true - Δ), stored negated (its dP accumulators start from it)
  if (g == 0) a.delta[hT + row] = -(delta + dd_err);
  uint16_t* dqp = a.dq + h * a.q_sh + static_cast<int64_t>(row) * a.q_st + 4 * g;
#pragma unroll
  for (int md = 0; md < 8; ++md) {
    uint2 val;
    val.x = cvt_pk_bf16(dqT[md][0] * a.scale, dqT[md][1] * a.scale);
    val.y = cvt_pk_bf16(dqT[md][2] * a.scale, dqT[md][3] * a.scale);
    *reinterpret_cast<uint2*>(dqp + md * 16) = val;
  }
  const float beta = a.beta;
  if (MODE == 1 && a.dcoeff_cos) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      accA[k] = sum_groups16(accA[k]);
      accB[k] = sum_groups16(accB[k]);
      accPA[k] = sum_groups16(accPA[k]);
      accPB[k] = sum_groups16(accPB[k]);
    }
    if (g == 0)
      for (int k = 0; k < a.K; ++k) {
        a.dcoeff_cos[(hT + row) * a.K + k] = beta * (accA[k] - dd_err * accPA[k]);
        a.dcoeff_sin[(hT + row) * a.K + k] = beta * (accB[k] - dd_err * accPB[k]);
      }
  }
  if (TOK) {
    if (a.dcoeff_cos) {
      // facc[fb] register r: feature 16·fb + 4g + r; features 0-7 cos hi, 8-15 sin hi,
      // 16-23 cos lo, 24-31 sin lo (band k = feature % 8): lane groups 0, 1 hold the
      // cos half of bands 4g .. 4g+3, lane groups 2, 3 the sin half of the same bands
      float C[4], Cp[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        C[i] = facc[0][i] + facc[1][i];
        Cp[i] = facc_p[0][i] + facc_p[1][i];
      }
      float S[4], Sp[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        S[i] = __shfl_xor(C[i], 32, 64);
        Sp[i] = __shfl_xor(Cp[i], 32, 64);
      }
      if (g < 2) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int k = 4 * g + i;
          if (k < a.K) {
            const float Cc = C[i] - dd_err * Cp[i], Sc = S[i] - dd_err * Sp[i];
            float ci, si;
            tok_trig(static_cast<const uint32_t*>(a.table) + static_cast<int64_t>(row) * (kTokRow / 2), k, ci, si);
            a.dcoeff_cos[(hT + row) * a.K + k] = beta * (ci * Cc + si * Sc);
            a.dcoeff_sin[(hT + row) * a.K + k] = beta * (si * Cc - ci * Sc);
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 6; ++i) ex[i] = sum_groups16(ex[i]);
    if (g == 0) {
      // for the kv-major pass: the row's offset without the pair bias (-inf
      // for a row without visible keys: lse2 is +inf there) and β·slope
      a.rowoff[hT + row] = rowc - lse2;
      a.rowslope[hT + row] = slp;
      if (a.db0) a.db0[hT + row] = -beta * (rs_tot - dd_err * pm_tot);
      if (a.dslope) a.dslope[hT + row] = beta * (ex[0] - dd_err * ex[3]);
      const float gsc = beta * a.ramp_lambda * a.inv_tau;
      if (a.ddelta_main) a.ddelta_main[hT + row] = GATE ? gsc * (ex[1] - dd_err * ex[4]) : 0.f;
      if (a.dwidth) a.dwidth[hT + row] = GATE ? gsc * (ex[2] - dd_err * ex[5]) : 0.f;
    }
  }
  // ---- modes 0/1: this row's softmax offset for every listed key block (the
  // block term, plus the pair bias, minus lse), read per tile by the kv-major
  // pass; the four lanes of a row take every fourth entry
  if (MODE <= 1) {
    float* rof = a.roff + lrow * a.maxkv * BS + (row - qb * BS);
    for (int e = g; e < n; e += 4) {
      float t = pbias ? kbias[e] : 0.f;
      if (MODE == 1) {
        const int rd = min(max(qb - kb_at(e), 0), a.QB - 1);
        const float4* t4 = reinterpret_cast<const float4*>(static_cast<const float*>(a.table) + rd * 16);
        const float4 c0 = t4[0], c1 = t4[1], s0 = t4[2], s1 = t4[3];
        t += (ca[0] * c0.x + ca[1] * c0.y + ca[2] * c0.z + ca[3] * c0.w) +
             (ca[4] * c1.x + ca[5] * c1.y + ca[6] * c1.z + ca[7] * c1.w) +
             (sa[0] * s0.x + sa[1] * s0.y + sa[2] * s0.z + sa[3] * s0.w) +
             (sa[4] * s1.x + sa[5] * s1.y + sa[6] * s1.z + sa[7] * s1.w);
      }
      rof[e * BS] = t - lse2;
    }
  }
}

// dK and dV of the key blocks whose q-list spans several chunks: the sum of
// the chunks' fp32 partials in chunk order, dK scaled, rounded to bf16.  A
// fixed grid walks the work units (multi-chunk key block of any head, one of
// kSlices column slices of 256 float4), so no workgroup is launched for a
// single-chunk block and a long q-list (a global block listed by every
// q-block of a long document) is summed by many workgroups: at bs=256 one
// key block is 32 units.  Each thread sums one float4 column of dK and of dV,
// four chunks at a time (eight loads in flight); the partials are read once,
// by nontemporal loads.  Each workgroup first forms the exclusive prefix of
// the heads' multi-chunk counts in LDS (one load per head, all in parallel),
// so a unit finds its head by a search in LDS and its key block, q-list
// length and first slot by one level of loads.
template <int BS>
__global__ __launch_bounds__(256) void bwd_reduce_kernel(AttnArgs a, KvPlan pl) {
  constexpr int D = 128;
  constexpr int64_t per_slot = static_cast<int64_t>(BS) * D / 4;  // float4 per partial
  constexpr int kSlices = static_cast<int>(per_slot / 256);
  constexpr int kAhead = 4;
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  extern __shared__ int hoff[];  // [H]: multi-chunk key blocks of the heads before h
  __shared__ int wsum[4];
  const int NB = a.QB;
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  int total = 0;  // the same in every thread
  for (int h0 = 0; h0 < a.H; h0 += 256) {
    const int h = h0 + static_cast<int>(threadIdx.x);
    const int c = h < a.H ? pl.multi[static_cast<int64_t>(h) * (NB + 1)] : 0;
    int incl = c;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int t = __shfl_up(incl, o, kWave);
      if (lane >= o) incl += t;
    }
    if (lane == kWave - 1) wsum[wave] = incl;
    __syncthreads();
    int base = total;
    for (int w = 0; w < wave; ++w) base += wsum[w];
    if (h < a.H) hoff[h] = base + incl - c;
    total += wsum[0] + wsum[1] + wsum[2] + wsum[3];
    __syncthreads();  // hoff complete; wsum free for the next 256 heads
  }
  const int64_t units = static_cast<int64_t>(total) * kSlices;
  for (int64_t u = blockIdx.x; u < units; u += gridDim.x) {
    int m = static_cast<int>(u / kSlices);
    const int e0 = static_cast<int>(u % kSlices) * 256 + threadIdx.x;
    // the head: the largest h with hoff[h] <= m (heads without multi-chunk
    // blocks share their successor's offset and are passed over)
    int h = 0, hi = a.H - 1;
    while (h < hi) {
      const int mid = (h + hi + 1) / 2;
      if (hoff[mid] <= m) h = mid;
      else hi = mid - 1;
    }
    m -= hoff[h];
    const int kb = pl.multi[static_cast<int64_t>(h) * (NB + 1) + 1 + m];
    const int32_t* qo = a.q_off + static_cast<int64_t>(h) * (NB + 1);
    const int nch = (qo[kb + 1] - qo[kb] + pl.chunk - 1) / pl.chunk;
    const int64_t slot0 = h * pl.max_slots + pl.slots_start[static_cast<int64_t>(h) * (NB + 1) + kb];
    const f32x4* pk = reinterpret_cast<const f32x4*>(pl.part_dk) + slot0 * per_slot + e0;
    const f32x4* pv = reinterpret_cast<const f32x4*>(pl.part_dv) + slot0 * per_slot + e0;
    f32x4 sk = {0.f, 0.f, 0.f, 0.f}, sv = {0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < nch; c += kAhead) {
      f32x4 xk[kAhead], xv[kAhead];
#pragma unroll
      for (int i = 0; i < kAhead; ++i) {
        if (c + i < nch) {
          xk[i] = __builtin_nontemporal_load(pk + (c + i) * per_slot);
          xv[i] = __builtin_nontemporal_load(pv + (c + i) * per_slot);
        }
      }
#pragma unroll
      for (int i = 0; i < kAhead; ++i) {
        if (c + i < nch) {
          sk += xk[i];
          sv += xv[i];
        }
      }
    }
    const int64_t kv0 = static_cast<int64_t>(kb) * BS;
    const int r = (e0 * 4) / D, d = (e0 * 4) % D;
    uint2 vk, vv;
    vk.x = cvt_pk_bf16(sk.x * a.scale, sk.y * a.scale);
    vk.y = cvt_pk_bf16(sk.z * a.scale, sk.w * a.scale);
    vv.x = cvt_pk_bf16(sv.x, sv.y);
    vv.y = cvt_pk_bf16(sv.z, sv.w);
    *reinterpret_cast<uint2*>(a.dk + h * a.k_sh + (kv0 + r) * a.k_st + d) = vk;
    *reinterpret_cast<uint2*>(a.dv + h * a.v_sh + (kv0 + r) * a.v_st + d) = vv;
  }
}

struct BwdLayout {
  int64_t delta, qfeat, items, slots, multi, part_dk, part_dv, q_pos, roff, rowoff, dpair, total, max_slots;
  int max_items;
};

static BwdLayout bwd_layout(const scope_attn_params* p) {
  BwdLayout L = {};
  const int64_t QB = p->T / p->bs, NB = QB;
  const int chunk = bwd_chunk(static_cast<int>(QB));
  const int64_t per_head_items = NB + (QB * p->maxkv + chunk - 1) / chunk;
  L.max_items = static_cast<int>(per_head_items);
  L.max_slots = (2 * QB * p->maxkv + chunk - 1) / chunk + 1;
  auto al = [](int64_t x) { return (x + 255) & ~static_cast<int64_t>(255); };
  int64_t o = 0;
  L.delta = o;
  o += al(static_cast<int64_t>(p->H) * p->T * 4);
  L.qfeat = o;
  if (p->bias_mode == SCOPE_BIAS_TOKEN) o += al(static_cast<int64_t>(p->H) * p->T * 32 * 2);
  L.items = o;
  o += al(static_cast<int64_t>(p->H) * (NB + 1) * 4);
  L.slots = o;
  o += al(static_cast<int64_t>(p->H) * (NB + 1) * 4);
  L.multi = o;
  o += al(static_cast<int64_t>(p->H) * (NB + 1) * 4);
  const int64_t part = static_cast<int64_t>(p->H) * L.max_slots * p->bs * 128 * 4;
  L.part_dk = o;
  o += al(part);
  L.part_dv = o;
  o += al(part);
  L.q_pos = o;
  o += al(static_cast<int64_t>(p->H) * QB * p->maxkv * 4);
  // per-(h, qb, entry, row) softmax offsets of modes 0/1
  L.roff = o;
  if (p->bias_mode != SCOPE_BIAS_TOKEN) o += al(static_cast<int64_t>(p->H) * QB * p->maxkv * p->bs * 4);
  // token modes: per-row offsets and slopes, [2][H][T]
  L.rowoff = o;
  if (p->bias_mode == SCOPE_BIAS_TOKEN) o += al(2 * static_cast<int64_t>(p->H) * p->T * 4);
  // pair-bias gradient partials, one per 128-key part of a key block
  L.dpair = o;
  if (p->dpair_bias) o += al(static_cast<int64_t>(p->bs / 128) * p->H * QB * p->maxkv * 4);
  L.total = o;
  return L;
}

// dpair_bias[h][qb][e] = the sum of the key-block parts' tile sums for the
// listed entries (in part order), 0 for e >= kv_num.
__global__ __launch_bounds__(256) void dpair_sum_kernel(AttnArgs a, int parts, float* __restrict__ out) {
  const int64_t rows = static_cast<int64_t>(a.H) * a.QB;
  const int64_t n = rows * a.maxkv;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t row = i / a.maxkv;
    const int e = static_cast<int>(i % a.maxkv);
    float t = 0.f;
    if (e < min(a.kv_num[row], a.maxkv))
      for (int pp = 0; pp < parts; ++pp) t += a.dpair[pp * n + i];
    out[i] = t;
  }
}

template <int BS>
static void launch_bwd(const AttnArgs& a, const KvPlan& pl, int mode, int phases, int grid_q, int max_items,
                       float* dpair_out, hipStream_t s) {
  constexpr int P = BS / 128;
  const int per_xcd = (a.H * max_items + 7) / 8;
  dim3 gq(grid_q * P), gk(8 * per_xcd * P), gr(4096);
  // token mode with an active gate runs the kernels' MODE 3 variant
  const bool gate = a.gate_kind != SCOPE_GATE_NONE && a.ramp_lambda > 0.f;
  bool dq_done = false;
  if constexpr (BS == 256) {
    if ((phases & SCOPE_BWD_DQ) && mode != SCOPE_BIAS_TOKEN) {
      // one workgroup per q-block, two wavefronts per SIMD
      if (mode == SCOPE_BIAS_BLOCK)
        hipLaunchKernelGGL((attn_bwd_dq2_kernel<BS, 1>), dim3(grid_q), dim3(2 * BS), 0, s, a);
      else
        hipLaunchKernelGGL((attn_bwd_dq2_kernel<BS, 0>), dim3(grid_q), dim3(2 * BS), 0, s, a);
      dq_done = true;
    }
  }
  if ((phases & SCOPE_BWD_DQ) && !dq_done) {
    // 16 query rows per wavefront, eight wavefronts (two per SIMD) per 128 rows
    if (mode == SCOPE_BIAS_BLOCK)
      hipLaunchKernelGGL((attn_bwd_dq16_kernel<BS, 1>), gq, dim3(512), 0, s, a);
    else if (mode == SCOPE_BIAS_TOKEN && gate)
      hipLaunchKernelGGL((attn_bwd_dq16_kernel<BS, 3>), gq, dim3(512), 0, s, a);
    else if (mode == SCOPE_BIAS_TOKEN)
      hipLaunchKernelGGL((attn_bwd_dq16_kernel<BS, 2>), gq, dim3(512), 0, s, a);
    else
      hipLaunchKernelGGL((attn_bwd_dq16_kernel<BS, 0>), gq, dim3(512), 0, s, a);
  }
  if (phases & SCOPE_BWD_DKV) phases |= SCOPE_BWD_DKV_PLAN | SCOPE_BWD_DKV_MAIN | SCOPE_BWD_DKV_REDUCE;
  if (phases & SCOPE_BWD_DKV_PLAN) {
    hipLaunchKernelGGL(bwd_plan_kernel, dim3(a.H), dim3(1024), 0, s, a.QB, pl.chunk, a.q_off,
                       const_cast<int32_t*>(pl.items_start),
                       const_cast<int32_t*>(pl.slots_start), const_cast<int32_t*>(pl.multi));
    if (pl.q_pos) {
      const int64_t n = static_cast<int64_t>(a.H) * a.QB * a.maxkv;
      const int blocks = static_cast<int>(std::min<int64_t>((n + 255) / 256, 65536));
      hipLaunchKernelGGL(qpos_kernel, dim3(blocks), dim3(256), 0, s, a, const_cast<int32_t*>(pl.q_pos));
    }
  }
  const bool dp = a.dpair != nullptr;  // the pair-bias gradient runs in its own instantiation
  if (phases & SCOPE_BWD_DKV_MAIN) {
    // 16 keys per wavefront, 8 wavefronts (two per SIMD) per 128 keys
    // (the gated token mode spills 20-40 registers here: it keeps the
    // 32-keys-per-wavefront kernel, one wavefront per SIMD)
    const int m = mode == SCOPE_BIAS_TOKEN ? (gate ? 3 : 2) : (mode == SCOPE_BIAS_BLOCK ? 1 : 0);
    if (m == 3 && dp) hipLaunchKernelGGL((attn_bwd_dkv_kernel<BS, 3, true>), gk, dim3(256), 0, s, a, pl);
    else if (m == 3) hipLaunchKernelGGL((attn_bwd_dkv_kernel<BS, 3, false>), gk, dim3(256), 0, s, a, pl);
    else if (m == 2 && dp) hipLaunchKernelGGL((attn_bwd_dkv16_kernel<BS, 2, true>), gk, dim3(512), 0, s, a, pl);
    else if (m == 2) hipLaunchKernelGGL((attn_bwd_dkv16_kernel<BS, 2, false>), gk, dim3(512), 0, s, a, pl);
    else if (m == 1 && dp) hipLaunchKernelGGL((attn_bwd_dkv16_kernel<BS, 1, true>), gk, dim3(512), 0, s, a, pl);
    else if (m == 1) hipLaunchKernelGGL((attn_bwd_dkv16_kernel<BS, 1, false>), gk, dim3(512), 0, s, a, pl);
    else if (dp) hipLaunchKernelGGL((attn_bwd_dkv16_kernel<BS, 0, true>), gk, dim3(512), 0, s, a, pl);
    else hipLaunchKernelGGL((attn_bwd_dkv16_kernel<BS, 0, false>), gk, dim3(512), 0, s, a, pl);
  }
  if (phases & SCOPE_BWD_DKV_REDUCE) {
    hipLaunchKernelGGL(bwd_reduce_kernel<BS>, gr, dim3(256), static_cast<size_t>(a.H) * sizeof(int), s, a, pl);
    if (a.dpair && dpair_out) {
      const int64_t n = static_cast<int64_t>(a.H) * a.QB * a.maxkv;
      const int blocks = static_cast<int>(std::min<int64_t>((n + 255) / 256, 4096));
      hipLaunchKernelGGL(dpair_sum_kernel, dim3(blocks), dim3(256), 0, s, a, P, dpair_out);
    }
  }
}

}  // namespace scope

using namespace scope;

extern "C" int64_t scope_attn_bwd_workspace_bytes(const scope_attn_params* p) {
  if (!p || p->bs <= 0 || p->T <= 0) return 0;
  return bwd_layout(p).total;
}

extern "C" int scope_attn_bwd_phase(const scope_attn_params* p, int phases, const uint16_t* q, const uint16_t* k,
                                    const uint16_t* v, const uint16_t* out, const uint16_t* dout, const float* lse,
                                    const int32_t* kv_num, const int32_t* kv_idx, const int32_t* q_off,
                                    const int32_t* q_list, const int32_t* docs, const int32_t* ds_tok_end,
                                    const void* table, const float* coeff_cos, const float* coeff_sin, const float* b0,
                                    const float* slope, const float* delta_main, const float* width, uint16_t* dq,
                                    uint16_t* dk, uint16_t* dv, float* dcoeff_cos, float* dcoeff_sin, float* db0,
                                    float* dslope, float* ddelta_main, float* dwidth, void* workspace, void* stream) {
  SCOPE_REQUIRE(phases >= 1 && phases <= 31, "scope_attn_bwd_phase: phases must be a non-empty set of SCOPE_BWD_* bits (got %d)",
                phases);
  int rc = validate_attn(p, q, k, v, kv_num, kv_idx, docs, ds_tok_end, table, coeff_cos, coeff_sin, b0, slope,
                         delta_main, width, "scope_attn_bwd");
  if (rc) return rc;
  SCOPE_REQUIRE(out && dout && lse && q_off && q_list && dq && dk && dv && workspace,
                "scope_attn_bwd: null pointer");
  SCOPE_REQUIRE(((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(dout) |
                  reinterpret_cast<uintptr_t>(lse) | reinterpret_cast<uintptr_t>(workspace)) &
                 15) == 0,
                "scope_attn_bwd: out, dout, lse and workspace must start on a 16-byte boundary");
  SCOPE_REQUIRE(!dcoeff_cos == !dcoeff_sin, "scope_attn_bwd: dcoeff_cos and dcoeff_sin go together");
  AttnArgs a = make_args(p);
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = out;
  a.dout = dout;
  a.lse = lse;
  a.kv_num = kv_num;
  a.kv_idx = kv_idx;
  a.q_off = q_off;
  a.q_list = q_list;
  a.docs = docs;
  a.ds_tok_end = ds_tok_end;
  a.table = table;
  a.coeff_cos = coeff_cos;
  a.coeff_sin = coeff_sin;
  a.b0 = b0;
  a.slope = slope;
  a.delta_main = delta_main;
  a.width = width;
  a.dq = dq;
  a.dk = dk;
  a.dv = dv;
  a.dcoeff_cos = p->bias_mode != SCOPE_BIAS_NONE ? dcoeff_cos : nullptr;
  a.dcoeff_sin = p->bias_mode != SCOPE_BIAS_NONE ? dcoeff_sin : nullptr;
  const bool tok = p->bias_mode == SCOPE_BIAS_TOKEN;
  a.db0 = tok && p->subtract_b0 ? db0 : nullptr;
  a.dslope = tok && p->use_slope ? dslope : nullptr;
  a.ddelta_main = tok && p->gate_kind != SCOPE_GATE_NONE ? ddelta_main : nullptr;
  a.dwidth = tok && p->gate_kind != SCOPE_GATE_NONE ? dwidth : nullptr;
  const BwdLayout L = bwd_layout(p);
  char* ws = static_cast<char*>(workspace);
  a.delta = reinterpret_cast<float*>(ws + L.delta);
  a.qfeat = reinterpret_cast<uint16_t*>(ws + L.qfeat);
  KvPlan pl;
  pl.items_start = reinterpret_cast<const int32_t*>(ws + L.items);
  pl.slots_start = reinterpret_cast<const int32_t*>(ws + L.slots);
  pl.multi = reinterpret_cast<const int32_t*>(ws + L.multi);
  pl.part_dk = reinterpret_cast<float*>(ws + L.part_dk);
  pl.part_dv = reinterpret_cast<float*>(ws + L.part_dv);
  pl.q_pos = reinterpret_cast<const int32_t*>(ws + L.q_pos);
  a.roff = p->bias_mode != SCOPE_BIAS_TOKEN ? reinterpret_cast<float*>(ws + L.roff) : nullptr;
  a.rowoff = p->bias_mode == SCOPE_BIAS_TOKEN ? reinterpret_cast<float*>(ws + L.rowoff) : nullptr;
  a.rowslope = a.rowoff ? a.rowoff + static_cast<int64_t>(p->H) * p->T : nullptr;
  pl.max_slots = L.max_slots;
  pl.max_items = L.max_items;
  pl.chunk = bwd_chunk(a.QB);
  hipStream_t s = as_stream(stream);
  const int grid_q = p->H * a.QB;
  a.dpair = p->dpair_bias ? reinterpret_cast<float*>(ws + L.dpair) : nullptr;
  if (p->bs == 256)
    launch_bwd<256>(a, pl, p->bias_mode, phases, grid_q, L.max_items, p->dpair_bias, s);
  else
    launch_bwd<128>(a, pl, p->bias_mode, phases, grid_q, L.max_items, p->dpair_bias, s);
  return check_launch("attention backward kernels");
}

extern "C" int scope_attn_bwd(const scope_attn_params* p, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              const uint16_t* out, const uint16_t* dout, const float* lse, const int32_t* kv_num,
                              const int32_t* kv_idx, const int32_t* q_off, const int32_t* q_list, const int32_t* docs,
                              const int32_t* ds_tok_end, const void* table, const float* coeff_cos,
                              const float* coeff_sin, const float* b0, const float* slope, const float* delta_main,
                              const float* width, uint16_t* dq, uint16_t* dk, uint16_t* dv, float* dcoeff_cos,
                              float* dcoeff_sin, float* db0, float* dslope, float* ddelta_main, float* dwidth,
                              void* workspace, void* stream) {
  return scope_attn_bwd_phase(p, SCOPE_BWD_DQ | SCOPE_BWD_DKV, q, k, v, out, dout, lse, kv_num, kv_idx, q_off, q_list,
                              docs, ds_tok_end, table, coeff_cos, coeff_sin, b0, slope, delta_main, width, dq, dk, dv,
                              dcoeff_cos, dcoeff_sin, db0, dslope, ddelta_main, dwidth, workspace, stream);
}
