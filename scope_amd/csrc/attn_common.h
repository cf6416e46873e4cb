// Shared pieces of the block-sparse attention kernels (gfx950, bf16 MFMA).
//
// MFMA operand layouts of v_mfma_f32_32x32x16_bf16 (wave64), lane l,
// g = l / 32, c = l % 32:
//   A (32 x 16, M x K): row c, k = 8g .. 8g+7          (8 bf16, one uint4)
//   B (16 x 32, K x N): col c, k = 8g .. 8g+7          (8 bf16, one uint4)
//   C (32 x 32):        col c, register r -> row 8(r/4) + 4g + (r%4)
//
// The forward computes S^T = K·Q^T (M = keys, N = queries): every lane owns
// one query row (c) and 16 keys per 32-key block, so the softmax statistics
// of a row live in the lane pair (l, l^32).  P^T is then the B operand of
// O^T = V^T·P^T without any data movement: k-step s covers keys
// 16s + 8(j/4) + 4g + (j%4) for slot j, which is exactly where the S^T
// accumulator registers 8(s%2)..8(s%2)+7 of key block s/2 sit.
#pragma once

#include "common.h"

namespace scope {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16_t mfma32(const uint4& a, const uint4& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}

// v_mfma_f32_16x16x32_bf16 (wave64), lane l, g = l / 16, c = l % 16:
//   A (16 x 32, M x K): row c, k = 8g .. 8g+7;  B (32 x 16, K x N): col c,
//   k = 8g .. 8g+7;  C (16 x 16): col c, register r -> row 4g + r.
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma16(const uint4& a, const uint4& b, const f32x4_t& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}

__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  bf16x2_t v;
  v[0] = static_cast<__bf16>(lo);
  v[1] = static_cast<__bf16>(hi);
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ f32x16_t zero16() {
  f32x16_t z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// byte permute: out = {a.half(sel_a), b.half(sel_b)} packed (lo from a, hi from b)
__device__ __forceinline__ uint32_t pack_lo16(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi16(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// ---- swizzled row-major LDS tiles -------------------------------------------
// A tile row holds 128 bf16 (256 bytes = all 64 banks).  The 16-byte chunk c
// of row r is stored at chunk c ^ swz(r), swz(r) = 4·(r%4) + 2·b2 + b3 with
// b2, b3 the bits 2 and 3 of r.  With this mapping these access patterns are
// bank-conflict free:
//   * row reads (16 lanes, 16 consecutive rows, same logical chunk),
//   * transpose reads of the 32x32 operands (32 lanes, 4 rows × 8 eight-byte
//     column groups), and
//   * transpose reads of the 16x16 operands (32 lanes: rows 4g .. 4g+3 of
//     lane group g = 0, 1, the same 4 column groups): bits 1-3 of swz(r)
//     encode r mod 8, so the 8 rows of the two groups land on 8 distinct
//     chunk pairs.
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | (((r >> 2) & 1) << 1) | ((r >> 3) & 1); }
// element offset of (row r, column d) in a swizzled tile
__device__ __forceinline__ int swz_off(int r, int d) { return r * 128 + (((d >> 3) ^ swz(r)) << 3) + (d & 7); }

// Per-row fp32 arrays that each lane reads as float4 chunks of its own row
// (coefficients, gradient sums).  Row strides of 64 or 128 bytes would put
// 4 or 8 of 16 consecutive rows on the same banks; the chunk index is XORed
// with row bits so that 16 consecutive rows reading the same chunk hit
// distinct banks.  Offsets in floats; chunk c covers floats 4c..4c+3.
__device__ __forceinline__ int row16_off(int r, int c) { return r * 16 + ((c ^ ((r >> 2) & 3)) << 2); }
__device__ __forceinline__ int row32_off(int r, int c) { return r * 32 + ((c ^ ((r >> 1) & 7)) << 2); }

__device__ __forceinline__ uint4 lds_row8(const uint16_t* tile, int r, int d) {
  return *reinterpret_cast<const uint4*>(tile + swz_off(r, d));
}

typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_t;

// ds_read_b64_tr_b16: within each group of 16 lanes, lane j supplies an
// 8-byte address A_j and lane i receives slot s = A_{4s + i/4}[i % 4].  With
// lane 4s+t pointing at (row r0+s, column d0+4t), lane i gets the column
// d0+i of rows r0..r0+3, i.e. an MFMA operand whose k index runs along rows.
__device__ __forceinline__ uint2 lds_tr4(const uint16_t* tile, int r0, int d0, int lane16) {
  const int s = lane16 >> 2, t = lane16 & 3;
  const uint16_t* p = tile + swz_off(r0 + s, d0 + 4 * t);
  // address-space cast (generic -> LDS) needs a C-style cast
  lds_bf16x4_t* lp = (lds_bf16x4_t*)(const_cast<uint16_t*>(p));
  return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(lp));
}

// A/B operand of v_mfma_f32_32x32x16_bf16 whose k index runs along the rows
// of a swizzled tile and whose m/n index is the column d = dm0 + (lane % 32):
// k-step covering rows k0..k0+15 in the slot order used throughout
// (slots 0-3: rows k0+4g+0..3, slots 4-7: rows k0+8+4g+0..3).
__device__ __forceinline__ uint4 lds_kmajor(const uint16_t* tile, int k0, int dm0, int lane) {
  const int g = lane >> 5, l16 = lane & 15, d0 = dm0 + ((lane >> 4) & 1) * 16;
  const uint2 lo = lds_tr4(tile, k0 + 4 * g, d0, l16);
  const uint2 hi = lds_tr4(tile, k0 + 8 + 4 * g, d0, l16);
  return make_uint4(lo.x, lo.y, hi.x, hi.y);
}

// Lane byte offsets of the swizzled-tile reads, computed once per kernel.
// swz(r) depends only on r mod 16, so a read at row offset r0 (a multiple of
// 16: a k-step, or the second 32-row block) is the lane's offset for r0 = 0
// plus the constant r0·256 bytes.  The inner loops then issue ds_reads whose
// only per-read term is an immediate: no swizzle arithmetic per read.
struct TileOffs {
  uint32_t row[8];              // lds_row8(tile, lane % 32, 16·ks + 8·(lane / 32)), ks = 0..7
  uint32_t tr_lo[4], tr_hi[4];  // the two transpose reads of lds_kmajor(tile, 0, 32·md, lane), md = 0..3
};

__device__ __forceinline__ TileOffs tile_offs(int lane) {
  TileOffs o;
  const int g = lane >> 5, lr = lane & 31, l16 = lane & 15, s = l16 >> 2, t = l16 & 3, hf = (lane >> 4) & 1;
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) o.row[ks] = 2u * static_cast<uint32_t>(swz_off(lr, ks * 16 + g * 8));
#pragma unroll
  for (int md = 0; md < 4; ++md) {
    const int d = md * 32 + hf * 16 + 4 * t;
    o.tr_lo[md] = 2u * static_cast<uint32_t>(swz_off(4 * g + s, d));
    o.tr_hi[md] = 2u * static_cast<uint32_t>(swz_off(8 + 4 * g + s, d));
  }
  return o;
}

// lds_row8(tile, r0 + lane % 32, 16·ks + 8·(lane / 32)) for r0 a multiple of 16
__device__ __forceinline__ uint4 lds_row8_o(const uint16_t* tile, const TileOffs& o, int r0, int ks) {
  return *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(tile) + r0 * 256 + o.row[ks]);
}

// lds_kmajor(tile, k0, 32·md, lane) for k0 a multiple of 16
__device__ __forceinline__ uint4 lds_kmajor_o(const uint16_t* tile, const TileOffs& o, int k0, int md) {
  const char* base = reinterpret_cast<const char*>(tile) + k0 * 256;
  lds_bf16x4_t* plo = (lds_bf16x4_t*)(const_cast<char*>(base + o.tr_lo[md]));
  lds_bf16x4_t* phi = (lds_bf16x4_t*)(const_cast<char*>(base + o.tr_hi[md]));
  const uint2 lo = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(plo));
  const uint2 hi = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(phi));
  return make_uint4(lo.x, lo.y, hi.x, hi.y);
}

// ---- swizzled 32-column tiles (64-byte rows: token features) ---------------
// The 16-byte chunk c of row r is stored at chunk c ^ swz32(r), swz32(r) the
// two bits of (r/4) % 4 reversed.  Rows r and r + 4 lie 256 bytes apart, on the
// same banks; with the reversed bits the transpose reads of lane groups 0 and
// 1 (rows 0-3 and 4-7, chunks {0, 1} of each) land on chunks {0, 1} and
// {2, 3}.  Row reads of 16 consecutive rows stay conflict free.
__device__ __forceinline__ int swz32(int r) { return ((r >> 3) & 1) | (((r >> 2) & 1) << 1); }
__device__ __forceinline__ int swz32_off(int r, int d) { return r * 32 + (((d >> 3) ^ swz32(r)) << 3) + (d & 7); }

__device__ __forceinline__ uint4 lds_row8_32(const uint16_t* tile, int r, int d) {
  return *reinterpret_cast<const uint4*>(tile + swz32_off(r, d));
}

// A operand (32 columns x 16 rows of k) of a 32-column tile, slot order as lds_kmajor
__device__ __forceinline__ uint4 lds_kmajor_32(const uint16_t* tile, int k0, int lane) {
  const int g = lane >> 5, l16 = lane & 15, d0 = ((lane >> 4) & 1) * 16;
  const int s = l16 >> 2, t = l16 & 3;
  lds_bf16x4_t* plo = (lds_bf16x4_t*)(const_cast<uint16_t*>(tile + swz32_off(k0 + 4 * g + s, d0 + 4 * t)));
  lds_bf16x4_t* phi = (lds_bf16x4_t*)(const_cast<uint16_t*>(tile + swz32_off(k0 + 8 + 4 * g + s, d0 + 4 * t)));
  const uint2 lo = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(plo));
  const uint2 hi = __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(phi));
  return make_uint4(lo.x, lo.y, hi.x, hi.y);
}

// ---- direct global -> LDS copies ----------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;

// 16-byte global -> LDS copy of base + off (off per lane, base the same for
// the whole wavefront) to LDS address dst_wave + 16·lane (dst_wave the same
// for the whole wavefront): global_load_lds_dwordx4 with a scalar base.
//
// Issued as inline assembly rather than through __builtin_amdgcn_global_load_lds:
// while a builtin copy is in flight, the compiler's wait insertion treats the
// LDS counter as out of order and waits with lgkmcnt(0) before every LDS
// operand, so an operand read one step ahead is waited for at once together
// with every younger read.  Hidden from the compiler, the copies leave the
// LDS reads with exact lgkmcnt(N) waits.  The price is that the compiler
// knows nothing of the copies: every reader of a copied buffer is ordered
// after them by wait_vm0() and a barrier (each tile loop does both before it
// touches the tile), and a workgroup waits for its copies before it exits.
// M0 (the LDS base of the copy) is saved and restored around the copy.
__device__ __forceinline__ void g2lds16(const void* base, uint32_t off, void* dst_wave) {
  // (readfirstlane returns int: each half goes through uint32_t before widening,
  // or the low half would be sign-extended into the high one)
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b)));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<uint32_t>(b >> 32)));
  const uint64_t sb = (static_cast<uint64_t>(hi) << 32) | lo;
  const uint32_t m0v =
      __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void_t*)dst_wave)));
  uint32_t keep;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, %2\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(keep)
      : "v"(off), "s"(sb), "s"(m0v)
      : "memory");
}

// vmcnt(0): every global load of this wavefront (including global_load_lds) has landed
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// x where key j is visible from a row (j <= lim and the same document), else
// -inf, with integer sign-bit arithmetic only: comparisons would each take an
// SGPR pair, and a tile's worth of them exhausts the scalar registers.
__device__ __forceinline__ float mask_score(float x, int j, int lim, int doc_key, int doc_row) {
  const uint32_t d = static_cast<uint32_t>(doc_key ^ doc_row);
  const int ne = static_cast<int>(d | (0u - d));  // sign bit set iff the documents differ
  const int bad = ((lim - j) | ne) >> 31;         // all ones when j > lim or the documents differ
  return __int_as_float((__float_as_int(x) & ~bad) | (static_cast<int>(0xff800000u) & bad));
}

// Map a linear workgroup id so that the workgroups one XCD runs (the
// hardware deals ids round-robin over the 8 XCDs) cover consecutive tiles,
// which then share key blocks in that XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int n) {
  constexpr int kXcd = 8;
  if (n % kXcd != 0) return bid;
  return (bid % kXcd) * (n / kXcd) + bid / kXcd;
}

constexpr float kLog2e = 1.4426950408889634f;

// Token-mode table row (one per token j): 32 bf16 = cos(ω_k j) hi[8], sin hi[8],
// cos lo[8], sin lo[8], where hi = bf16(x) and lo = bf16(x - hi).  The band
// term runs as three MFMA k-steps (hi·hi + hi·lo + lo·hi), which carries the
// features at about 16 mantissa bits.
constexpr int kTokRow = 32;

// x of lane l ^ 32: v_permlane32_swap exchanges the halves of two registers
// without the LDS round trip of ds_bpermute (with both operands x, the
// returned first register holds the swapped lanes 32-63, the second 0-31)
__device__ __forceinline__ float xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float((__lane_id() & 32) ? r[0] : r[1]);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// cos/sin(ω_k j) (hi + lo) for band k from a table row
__device__ __forceinline__ void tok_trig(const uint32_t* row32, int k, float& c, float& s) {
  const uint32_t ch = row32[k / 2], sh = row32[4 + k / 2], cl = row32[8 + k / 2], sl = row32[12 + k / 2];
  c = (k & 1) ? bf16_hi(ch) + bf16_hi(cl) : bf16_lo(ch) + bf16_lo(cl);
  s = (k & 1) ? bf16_hi(sh) + bf16_hi(sl) : bf16_lo(sh) + bf16_lo(sl);
}

// 8 fp32 -> (hi, lo) bf16x8 pairs
__device__ __forceinline__ void split8(const float* f, uint4& hi, uint4& lo) {
  float r[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = f[i] - static_cast<float>(static_cast<__bf16>(f[i]));
  hi = make_uint4(cvt_pk_bf16(f[0], f[1]), cvt_pk_bf16(f[2], f[3]), cvt_pk_bf16(f[4], f[5]), cvt_pk_bf16(f[6], f[7]));
  lo = make_uint4(cvt_pk_bf16(r[0], r[1]), cvt_pk_bf16(r[2], r[3]), cvt_pk_bf16(r[4], r[5]), cvt_pk_bf16(r[6], r[7]));
}
constexpr float kLn2 = 0.6931471805599453f;

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dout;
  const float* lse;
  const int32_t* kv_num;
  const int32_t* kv_idx;
  const int32_t* q_off;
  const int32_t* q_list;
  const int32_t* docs;
  const int32_t* ds_tok_end;
  const void* table;
  const float* coeff_cos;
  const float* coeff_sin;
  const float* b0;
  const float* slope;
  const float* delta_main;
  const float* width;
  uint16_t* out;
  float* lse_out;
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  float* dcoeff_cos;
  float* dcoeff_sin;
  float* db0;
  float* dslope;
  float* ddelta_main;
  float* dwidth;
  float* delta;      // rowsum(dO∘O) [H,T]
  uint16_t* qfeat;   // token mode: query-side features [H,T][kTokRow] (hi g0, hi g1, lo g0, lo g1)
  float* mass;       // block mass [H,QB,NB] (forward mass pass)
  const float* pair_bias;  // per-list-entry score bias [H,QB,maxkv] (natural log) or null
  float* dpair;            // backward: tile sums of dS per (key-block part, h, qb, entry) [P][H][QB][maxkv] or null
  // backward, no bias or block bias: the log2-domain softmax offset of every
  // (h, qb, list entry, row), [H][QB][maxkv][bs] = block term + pair bias -
  // lse·log2e, written by the q-major pass and read per tile by the kv-major pass
  float* roff;
  // backward, token modes: each row's softmax offset without the pair bias,
  // -β·b0 - lse (log2 units, -inf for a row without visible keys), and its
  // slope β·slope (log2 units), [H][T] each, written by the q-major pass and
  // copied per tile by the kv-major pass
  float* rowoff;
  float* rowslope;
  int H, QB, maxkv, K;
  int64_t T;
  int64_t q_sh, q_st, k_sh, k_st, v_sh, v_st, o_sh, o_st;
  float scale_log2;   // scale * log2(e)
  float scale;
  float beta;
  float beta_log2;    // beta * log2(e)
  float feat_scale;   // beta / scale (token-mode MFMA features)
  int use_slope, subtract_b0, gate_kind;
  float ramp_lambda, inv_tau;
};

// Query-side token features of one row for lane group g (0: A cos + B sin,
// 1: A sin - B cos, k = 0..7) scaled by feat_scale, split hi/lo; also returns
// cos/sin(ω_k row) for k = 4g..4g+3 (for the coefficient gradients).
struct AttnArgs;
__device__ __forceinline__ void token_qfeat(const AttnArgs& a, int64_t hT, int64_t row, int g, uint4& hi, uint4& lo,
                                            float* cos_g, float* sin_g);

// host helpers shared by the forward and backward entry points (attn_fwd.hip)
int validate_attn(const scope_attn_params* p, const void* q, const void* k, const void* v, const int32_t* kv_num,
                  const int32_t* kv_idx, const int32_t* docs, const int32_t* ds_tok_end, const void* table,
                  const float* cc, const float* cs, const float* b0, const float* slope, const float* dm,
                  const float* wd, const char* who);
AttnArgs make_args(const scope_attn_params* p);

__device__ __forceinline__ void token_qfeat(const AttnArgs& a, int64_t hT, int64_t row, int g, uint4& hi, uint4& lo,
                                            float* cos_g, float* sin_g) {
  const uint32_t* tb = static_cast<const uint32_t*>(a.table) + row * (kTokRow / 2);
  float f[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    float c, s;
    tok_trig(tb, k, c, s);
    const float A = k < a.K ? a.coeff_cos[(hT + row) * a.K + k] : 0.f;
    const float B = k < a.K ? a.coeff_sin[(hT + row) * a.K + k] : 0.f;
    f[k] = (g == 0 ? (A * c + B * s) : (A * s - B * c)) * a.feat_scale;
    if (cos_g && (k >> 2) == g) {
      cos_g[k & 3] = c;
      sin_g[k & 3] = s;
    }
  }
  split8(f, hi, lo);
}


// ---- one 64-key tile staged in LDS (q-major passes: forward, dQ) -----------
// Filled by global_load_lds; two buffers alternate so the copies of tile j+1
// run under the MFMAs of tile j.  WV = false: no V rows (the forward's LSE
// and block-mass kinds, which form no P·V).
template <int MODE, bool WV = true>
struct alignas(16) KvTile {
  uint16_t k[64 * 128];                      // K rows, swizzled (swz_off)
  uint16_t v[WV ? 64 * 128 : 8];             // V rows, swizzled
  int docs[64];                              // document id per key
  float tab[16];                             // block mode: table row of distance qb - kb
  uint16_t f[MODE >= 2 ? 64 * kTokRow : 8];  // token modes: key features [64][32] (swz32_off)
};

constexpr int kListLds = 1024;  // kv-list entries staged in LDS: the widest list the q-major kernels take

// Issue the copies of keys kv0 .. kv0+63 (and the block-table row rdist) into
// b; NT threads (128, 256 or 512) take part.
template <int MODE, int NT, bool WV = true>
__device__ __forceinline__ void kv_issue(const AttnArgs& a, int h, int64_t kv0, int rdist, KvTile<MODE, WV>& b,
                                         int tid) {
  static_assert(NT == 128 || NT == 256 || NT == 512, "kv_issue: 128, 256 or 512 threads");
  // kv0, rdist and the wavefront index are the same in every lane: the row
  // bases live in scalar registers and each lane adds a 32-bit byte offset
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int64_t k0 = __builtin_amdgcn_readfirstlane(static_cast<int>(kv0));
  const char* kbase = reinterpret_cast<const char*>(a.k + h * a.k_sh + k0 * a.k_st);
  const char* vbase = reinterpret_cast<const char*>(a.v + h * a.v_sh + k0 * a.v_st);
#pragma unroll
  for (int jj = 0; jj < 1024 / NT; ++jj) {
    // 16-byte chunk idx sits at LDS byte 16·idx: row idx/16, physical chunk
    // idx%16, which holds the logical chunk (idx%16) ^ swz(row)
    const int idx = jj * NT + tid;
    const int r = idx >> 4, c = (idx & 15) ^ swz(r);
    g2lds16(kbase, static_cast<uint32_t>((r * static_cast<int>(a.k_st) + c * 8) * 2), b.k + (jj * NT + wave * 64) * 8);
    if constexpr (WV)
      g2lds16(vbase, static_cast<uint32_t>((r * static_cast<int>(a.v_st) + c * 8) * 2), b.v + (jj * NT + wave * 64) * 8);
  }
  if (wave == 0 && lane < 16) g2lds16(a.docs + k0, lane * 16, b.docs);
  if (MODE == 1 && wave == 1 && lane < 4) {
    const int rd = __builtin_amdgcn_readfirstlane(rdist);
    g2lds16(static_cast<const float*>(a.table) + static_cast<int64_t>(rd) * 16, lane * 16, b.tab);
  }
  if (MODE >= 2) {
    const char* fbase = reinterpret_cast<const char*>(static_cast<const uint16_t*>(a.table) + k0 * kTokRow);
#pragma unroll
    for (int idx0 = 0; idx0 < 256; idx0 += NT) {
      const int idx = idx0 + tid;
      const int r = idx >> 2, c = (idx & 3) ^ swz32(r);
      if (idx < 256)
        g2lds16(fbase, static_cast<uint32_t>((r * kTokRow + c * 8) * 2), b.f + (idx0 + wave * 64) * 8);
    }
  }
}
}  // namespace scope
