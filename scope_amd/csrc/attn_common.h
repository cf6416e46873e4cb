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

// Map a linear workgroup id so that the workgroups one XCD runs (the
// hardware deals ids round-robin over the 8 XCDs) cover consecutive tiles,
// which then share key blocks in that XCD's L2.
__device__ __forceinline__ int xcd_remap(int bid, int n) {
  constexpr int kXcd = 8;
  if (n % kXcd != 0) return bid;
  return (bid % kXcd) * (n / kXcd) + bid / kXcd;
}

constexpr float kLog2e = 1.4426950408889634f;
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
  float* delta;  // rowsum(dO∘O) [H,T]
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

// host helpers shared by the forward and backward entry points (attn_fwd.hip)
int validate_attn(const scope_attn_params* p, const void* q, const void* k, const void* v, const int32_t* kv_num,
                  const int32_t* kv_idx, const int32_t* docs, const int32_t* ds_tok_end, const void* table,
                  const float* cc, const float* cs, const float* b0, const float* slope, const float* dm,
                  const float* wd, const char* who);
AttnArgs make_args(const scope_attn_params* p);

}  // namespace scope
