// Kernel 2 (backward): not built yet in this revision.
#include "attn_common.h"

using namespace scope;

extern "C" int64_t scope_attn_bwd_workspace_bytes(const scope_attn_params* p) { return 0; }

extern "C" int scope_attn_bwd(const scope_attn_params* p, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                              const uint16_t* out, const uint16_t* dout, const float* lse, const int32_t* kv_num,
                              const int32_t* kv_idx, const int32_t* q_off, const int32_t* q_list, const int32_t* docs,
                              const int32_t* ds_tok_end, const void* table, const float* coeff_cos,
                              const float* coeff_sin, const float* b0, const float* slope, const float* delta_main,
                              const float* width, uint16_t* dq, uint16_t* dk, uint16_t* dv, float* dcoeff_cos,
                              float* dcoeff_sin, float* db0, float* dslope, float* ddelta_main, float* dwidth,
                              void* workspace, void* stream) {
  return set_error(SCOPE_EINVAL, "scope_attn_bwd: backward not available in this build");
}
