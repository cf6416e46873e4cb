/*
 * scope_amd.h — C ABI of the MI355X (gfx950) SCOPE attention hot path.
 *
 * Every entry point takes plain device pointers, sizes and a HIP stream
 * (passed as void*, NULL = the default stream).  No call allocates device
 * memory: callers pass outputs and, where one is needed, a workspace whose
 * size the matching *_workspace_bytes() function reports.  All launches are
 * asynchronous on the given stream; no entry point synchronises the host.
 *
 * Return value: 0 on success, a negative SCOPE_E* code otherwise; the
 * message of the last failure on the calling thread is scope_last_error().
 *
 * Layout conventions (B = 1 throughout, as the reference asserts,
 * scoped_medium.py:336):
 *   q, k, v, out, dout, dq, dk, dv : bf16 bits (uint16_t), logical [H, T, D],
 *                                    element strides (stride_h, stride_t), d stride 1
 *   docs                           : int32 [T] document ids
 *   NB = QB = T / bs               : number of key blocks = number of query blocks
 *   kv_num [H, QB], kv_idx [H, QB, MAXKV] : compact BlockMask rows (int32)
 *   q_off [H, NB + 1], q_list [H, QB * MAXKV] : transposed lists (CSR, int32)
 */
#ifndef SCOPE_AMD_H
#define SCOPE_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SCOPE_ABI_VERSION 3

enum {
  SCOPE_OK = 0,
  SCOPE_EINVAL = -1,  /* bad shape, size or parameter                  */
  SCOPE_ELAUNCH = -2, /* a kernel launch failed (hipGetLastError)       */
  SCOPE_ERANGE = -3   /* a size exceeds a compiled limit                */
};

int scope_abi_version(void);
const char* scope_last_error(void);

/* ------------------------------------------------------------------------
 * Document starts.  Replaces model/attn_bias.py:688-709 (doc_change_tok,
 * cummax, floor_divide, reset segments) of build_pointer_blockmask and the
 * same steps of the forward debug statistics (:543-569).
 *   ds_ptr[qb]     doc start block of token (qb+1)*bs-1, clamped by resets
 *   ds_local[qb]   doc start block of token qb*bs, clamped by resets
 *   ds_tok_end[qb] doc start token of token (qb+1)*bs-1 (no clamp, no reset)
 * doc_clamp = 0 zeroes ds_ptr/ds_local (:698-700); reset_len > 0 applies the
 * reset segments (:703-709).
 * ---------------------------------------------------------------------- */
int scope_doc_starts(const int32_t* docs, int64_t T, int bs, int doc_clamp, int reset_len,
                     int32_t* ds_ptr, int32_t* ds_local, int32_t* ds_tok_end, void* stream);

/* ------------------------------------------------------------------------
 * Reference-mode pointer mask.  Replaces the body of
 * SpectralBias.build_pointer_blockmask, model/attn_bias.py:711-837
 * (representatives, radius allocation, Gumbel top-k over peaks, centres,
 * local/pointer/global pieces, sort + dedupe + pack).
 * ---------------------------------------------------------------------- */
typedef struct {
  int H, M, bs;
  int64_t T;
  int64_t stride_h, stride_t;  /* element strides of delta_star / budget_logits [H,T,M] */
  int rep_mean;                /* 0: token (qb+1)*bs-1 ("last"), 1: block mean        */
  int local_blocks;            /* after call-site override and max(1, .)              */
  int ptr_half_blocks;         /* p, after override and max(0, .)                    */
  int global_blocks_cfg;       /* pointer_global_blocks (constructor)                 */
  int global_active;           /* active global count (argument or schedule buffer)   */
  int radius_mode_pi;          /* 1: "pi", 0: "fixed"                                 */
  int budget_rem;              /* integer half budget, model/attn_bias.py:724-734     */
  float budget_temp;           /* max(pointer_budget_temp, 1e-6)                      */
  int mask_active;             /* _pointer_mask_active                                */
  int half_active;             /* _pointer_half_blocks_active                         */
  int gumbel_k;                /* 0: Gumbel off; else k (< M), training only          */
  float gumbel_tau;            /* max(gumbel_topk_tau, 1e-6)                          */
  float eps;                   /* SpectralBias.eps                                    */
} scope_ptr_ref_params;

/* MAXKV of the reference-mode list: local + (p>0 ? M(2p+1) : M) + min(G, NB). */
int scope_ptr_ref_maxkv(const scope_ptr_ref_params* p);

int scope_pointer_mask_ref(const scope_ptr_ref_params* p, const float* delta_star,
                           const float* budget_logits, const float* gumbel_u /* [H,QB,M] or NULL */,
                           const int32_t* ds_ptr, const int32_t* ds_local, int32_t* kv_num,
                           int32_t* kv_idx /* [H,QB,MAXKV] */, int32_t* radius /* [H,QB,M] */,
                           int32_t* centre /* [H,QB,M] */, void* stream);

/* ------------------------------------------------------------------------
 * Block-scoring pointer selection (block-mean q·k + radius prior + Gumbel
 * top-k under a budget: the block-scoring form of the pointer kernel).  Produces
 * the same (kv_num, kv_idx) layout as build_pointer_blockmask
 * (model/attn_bias.py:825-837) for the union window ∪ pointers ∪ global.
 * ---------------------------------------------------------------------- */
/* Block means q̄, k̄ [H, NB, D] fp32 of bf16 q, k. */
int scope_block_means(const uint16_t* q, const uint16_t* k, int H, int64_t T, int D, int bs,
                      int64_t q_sh, int64_t q_st, int64_t k_sh, int64_t k_st, float* qbar,
                      float* kbar, void* stream);
/* scope_block_means and scope_doc_starts in two launches instead of three:
 * the per-block document phase runs inside the block-means pass (on head
 * 0's workgroups), then the scan.  The same outputs, bit for bit, as the two
 * calls; T < 2^31. */
int scope_block_means_docs(const uint16_t* q, const uint16_t* k, const int32_t* docs, int H, int64_t T,
                           int D, int bs, int64_t q_sh, int64_t q_st, int64_t k_sh, int64_t k_st,
                           int doc_clamp, int reset_len, float* qbar, float* kbar, int32_t* ds_ptr,
                           int32_t* ds_local, int32_t* ds_tok_end, void* stream);

typedef struct {
  int H, NB, D, bs;
  int window, n_global, budget; /* W, G, pointer slots (budget <= 16)                   */
  float temp;                   /* τ of z = logit/τ + g                                  */
  float logit_scale;            /* logit = logit_scale * q̄·k̄ + prior[qb-kb]             */
  int noise_mode;               /* 0: none, 1: explicit uniforms, 2: counter-based draw  */
  uint64_t seed;                /* noise_mode 2                                          */
  float eps;                    /* Gumbel eps (1e-9)                                     */
  int64_t prior_head_stride;    /* 0: prior is [NB] shared; NB: prior is [H, NB]         */
  int flags;                    /* SCOPE_PTR_* bits below (ABI 3)                        */
} scope_ptr_score_params;

/* flags: logits_out is only the work buffer of the MFMA logits below; its
 * entries outside [ds_ptr, qb] are left unset instead of set to -inf. */
#define SCOPE_PTR_LOGITS_SCRATCH 1

int scope_pointer_select(const scope_ptr_score_params* p, const float* qbar, const float* kbar,
                         const float* logits_in /* [H,QB,NB] or NULL */,
                         const float* prior /* or NULL */, const float* gumbel_u /* [H,QB,NB] or NULL */,
                         const int32_t* ds_ptr, const int32_t* ds_local, int32_t* kv_num,
                         int32_t* kv_idx /* [H,QB,W+budget+G] */, int32_t* picks /* [H,QB,budget] */,
                         float* logits_out /* [H,QB,NB] or NULL */, void* stream);
/* With qbar/kbar (D = 128), NB >= 1024 and a logits_out buffer, the logits
 * of the lower triangle are first computed into logits_out as a product of
 * the block-mean matrices on bf16 MFMA, each fp32 mean split into two bf16
 * parts (hi·hi + hi·lo + lo·hi: within about 1e-5 of the fp32 dot product,
 * relative to Σ|q̄_d·k̄_d|, where the per-candidate fmaf chain used otherwise
 * rounds at fp32), and the selection reads them back; give logits_out to get
 * that path at long sequences (with SCOPE_PTR_LOGITS_SCRATCH when the caller
 * does not read the logits).  scope_pointer_pair_bias keeps the fmaf
 * chain. */

/* Soft pointer weights (no reference counterpart: build_pointer_blockmask
 * selects under torch.no_grad, model/attn_bias.py:623; this is the
 * differentiable inclusion weight the block-scoring specification asks for).
 * pair_bias [H,QB,W+budget+G] aligned with kv_idx: log σ(z/soft_temp) for
 * the pick entries (z the noise-free selection logit, computed like
 * scope_pointer_select computes it), 0 for window, global and padding
 * entries.  It is the scope_attn_params.pair_bias input of the attention. */
int scope_pointer_pair_bias(const scope_ptr_score_params* p, float soft_temp, const float* qbar,
                            const float* kbar, const float* logits_in /* [H,QB,NB] or NULL */,
                            const float* prior /* or NULL */, const int32_t* kv_num, const int32_t* kv_idx,
                            const int32_t* picks /* [H,QB,budget] */, float* pair_bias, void* stream);

/* Backward of the soft pointer weights: given dpair_bias (the attention
 * backward's gradient of pair_bias), dz = dpair·(1 - e^pair)/soft_temp and
 * the block-mean chain z = logit_scale·q̄·k̄ + prior add
 *   dq[i] += logit_scale/bs · Σ_e dz[qb(i),e] k̄[kv_idx[qb(i),e]]
 *   dk[j] += logit_scale/bs · Σ_{qb lists kb(j)} dz[qb, pos of kb(j)] q̄[qb]
 * to dq, dk (bf16, in place; fixed summation order).  The prior is treated as
 * a constant schedule (no gradient).  workspace: scope_pointer_bwd_workspace_bytes. */
typedef struct {
  int H, NB, D, bs, maxkv;
  float logit_scale, soft_temp;
  int64_t q_sh, q_st, k_sh, k_st; /* element strides of dq, dk [H, T, D] */
} scope_ptr_bwd_params;

int64_t scope_pointer_bwd_workspace_bytes(const scope_ptr_bwd_params* p);
int scope_pointer_bwd(const scope_ptr_bwd_params* p, const float* qbar, const float* kbar,
                      const int32_t* kv_num, const int32_t* kv_idx, const int32_t* q_off,
                      const int32_t* q_list, const float* pair_bias, const float* dpair_bias, uint16_t* dq,
                      uint16_t* dk, void* workspace, void* stream);

/* ------------------------------------------------------------------------
 * Transposed (q-major) lists.  Replaces BlockMask.from_kv_blocks ->
 * _transpose_ordered (torch:nn/attention/flex_attention.py:399-441, called at
 * model/attn_bias.py:867-873) with a compact CSR: for each kv block the
 * q-blocks that list it, ascending; a head's entries past q_off[h][NB] are
 * set to -1.
 * ---------------------------------------------------------------------- */
int64_t scope_transpose_workspace_bytes(int H, int NB);
int scope_transpose_blocks(const int32_t* kv_num, const int32_t* kv_idx, int H, int QB, int NB,
                           int maxkv, int32_t* q_off, int32_t* q_list, void* workspace,
                           void* stream);

/* scope_transpose_blocks without a workspace: it allocates nothing (no
 * hipMalloc, no allocating library call), for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops,
 * harnesses that forbid it.  No counterpart in the reference.  Same kernels
 * and results; the fill cursors live in a static device array of the library
 * (SCOPE_NOALLOC_MAX_HNB int32 per device, 1 MiB, held until the process
 * ends), so H*NB must not exceed SCOPE_NOALLOC_MAX_HNB (else SCOPE_ERANGE).
 * The array is shared by every call on a device and cleared by each call:
 * calls that overlap on one device (concurrent streams, threads) race.  The
 * stream must belong to the current device. */
#define SCOPE_NOALLOC_MAX_HNB 262144
int scope_transpose_blocks_noalloc(const int32_t* kv_num, const int32_t* kv_idx, int H, int QB, int NB,
                                   int maxkv, int32_t* q_off, int32_t* q_list, void* stream);

/* List validation.  The reference's pack (model/attn_bias.py:825-837)
 * guarantees what every kernel here relies on: for each row (h, qb),
 * 0 <= kv_num <= MAXKV and the first kv_num entries are distinct key blocks
 * in [0, NB), each <= qb for the causal masks.  This checks a list that did
 * not come from the library's own builders.  res (device int32 [5]) receives
 * the number of rows with kv_num outside [0, MAXKV], of entries outside
 * [0, NB), of entries after their q-block (only with causal != 0), of
 * repeated entries, and the first offending row h·QB + qb (INT32_MAX when
 * there is none).  Asynchronous on the stream; NB <= 65536. */
int scope_check_lists(const int32_t* kv_num, const int32_t* kv_idx, int H, int QB, int NB, int maxkv, int causal,
                      int32_t* res, void* stream);

/* ------------------------------------------------------------------------
 * Fused coefficient head.  Replaces the [B,H,L,M,K] mixture of
 * SpectralBias.forward between the MLP output and the returned terms
 * (model/attn_bias.py:419-478), its regularisers (:480-506) and, through
 * autograd, their backward.  The two MLP GEMMs stay with the caller (BLAS).
 *   y [rows, y_stride] (fp32, or bf16 bits with y_bf16): the MLP output,
 *     columns delta_raw | mu_raw | sigma_raw | pi_logits | budget_logits
 *     (M each) | c_raw (with use_slope); rows = B·H·L.
 *   outputs: coeff_cos, coeff_sin [rows, K]; slope, b0, delta_main, width
 *     [rows]; delta_star, pi, budget_logits [rows, M] (all fp32).
 *   reg [6] (training): total, omega, entropy, delta_edge, zero_mean, and
 *     the mean of b̄ that the backward of zero_mean needs.
 * The backward writes dy (same dtype and stride as y) from the upstream
 * gradients of the outputs (each may be NULL = zero) and of reg[0] (g_reg,
 * a device scalar, or NULL).
 * ---------------------------------------------------------------------- */
typedef struct {
  int M, K;                      /* peaks (<= 8), bands (<= 16)                        */
  int64_t rows;                  /* B·H·L                                               */
  int64_t L;                     /* sequence length                                     */
  int y_cols, y_stride;          /* 5M + use_slope; elements between rows of y / dy      */
  int y_bf16;                    /* 1: y and dy are bf16 bits, 0: fp32                  */
  int use_slope, subtract_b0;
  int training;                  /* regularisers on                                     */
  float delta_cap;               /* clamp(_delta_star_max_active, 0, L-1)               */
  float logw_min, logw_max;      /* log ω bounds of μ                                   */
  float c_scale, width_min, width_max, eps;
  float lambda_omega, lambda_entropy, lambda_zero_mean, lambda_delta_edge;
  float entropy_floor;           /* pi_entropy_floor_frac · log M                       */
  float delta_edge_eps;          /* _delta_edge_eps_active                              */
} scope_coeff_params;

int64_t scope_coeff_head_workspace_bytes(const scope_coeff_params* p);
int scope_coeff_head_fwd(const scope_coeff_params* p, const void* y, const float* omegas /* [K] */,
                         const float* log_omegas /* [K] */, const float* cos_mean /* [K] or NULL */,
                         const float* sin_mean /* [K] or NULL */, float* coeff_cos, float* coeff_sin, float* slope,
                         float* b0, float* delta_star, float* pi, float* budget_logits, float* delta_main,
                         float* width, float* reg /* [6] or NULL */, void* workspace, void* stream);
int scope_coeff_head_bwd(const scope_coeff_params* p, const void* y, const float* omegas, const float* log_omegas,
                         const float* cos_mean, const float* sin_mean, const float* g_coeff_cos,
                         const float* g_coeff_sin, const float* g_slope, const float* g_b0,
                         const float* g_delta_star, const float* g_pi, const float* g_budget_logits,
                         const float* g_delta_main, const float* g_width, const float* g_reg, const float* reg,
                         void* dy, void* stream);

/* ------------------------------------------------------------------------
 * Weight and bias gradients of the head's MLP layers.  Replaces autograd's
 * weight-gradient GEMM and bias-gradient reduction of the shared
 * Linear(D, 2D) -> SiLU -> Linear(2D, 5M+1) (model/attn_bias.py:271-276,
 * applied at :380-398 to every (b, h, t) row), whose contraction runs over
 * all rows:  dw[m][n] = Σ_r a[r][m]·b[r][n],  db[m] = Σ_r a[r][m]
 * with a the layer's output gradient and b its input, both bf16.  Row r is
 * row r % seg of segment r / seg: a + (r / seg)·a_ss + (r % seg)·a_rs
 * (elements), likewise b.  rows and seg are multiples of 64; (M, N) is
 * (64, 128), (64, 256), (128, 128), (128, 256), (256, 64) or (256, 128).
 * dw [M][N] and db [M] (db may be NULL) are fp32, each rounded to bf16
 * first when round_bf16 (the gradient of a bf16 copy of an fp32 weight).
 * Sums run in a fixed order (no atomics).  workspace:
 * scope_linear_wgrad_workspace_bytes.
 * ---------------------------------------------------------------------- */
typedef struct {
  int64_t rows, seg;
  int M, N;
  int64_t a_ss, a_rs, b_ss, b_rs;
  int round_bf16;
} scope_wgrad_params;

int64_t scope_linear_wgrad_workspace_bytes(const scope_wgrad_params* p);
int scope_linear_wgrad(const scope_wgrad_params* p, const uint16_t* a, const uint16_t* b, float* dw, float* db,
                       void* workspace, void* stream);

/* ------------------------------------------------------------------------
 * The head's shared MLP, fused.  Replaces the two F.linear and the SiLU of
 * SpectralBias._mlp_forward (model/attn_bias.py:271-276, 380-386) on bf16
 * rows, and the row-wise part of their autograd:
 *   forward   y = W2·SiLU(W1·q + b1) + b2               y [rows][O] bf16
 *   backward  z1 = W1·q + b1, x1 = SiLU(z1), dx1 = gy·W2,
 *             dz1 = SiLU'(z1)·dx1, dq = dz1·W1          dq [rows][128],
 *             x1, dz1 [rows][256], gyp = gy padded to [rows][64] (bf16)
 * with the weights fp32 as in the module (W1 [256][128], b1 [256],
 * W2 [O][256], b2 [O], rounded to bf16 like the reference's .to(q.dtype))
 * and every intermediate rounded to bf16 where the reference's tensors are;
 * D = 128, hidden = 256, 1 <= O <= 64.  Row r of q is row r % seg of
 * segment r / seg: q + (r / seg)·q_ss + (r % seg)·q_rs (elements); rows is
 * a multiple of 32; y, gy, dq, dz1, x1 and gyp are contiguous.  x1 and dz1
 * are optional (both null: not written).  The weight and bias gradients of
 * the bf16 weight copies, rounded to bf16 (autograd of the two F.linear over
 * all rows):
 *   scope_coeff_mlp_wgrad  dW1 = Σ_r dz1^T q [256][128], db1 = Σ_r dz1 [256],
 *                          dW2 = Σ_r gyp^T x1 [64][256], db2 = Σ_r gyp [64]
 * from q and gyp alone (z1, x1 and dz1 recomputed per tile, never stored;
 * seg a multiple of 128; the workspace is
 * scope_coeff_mlp_wgrad_workspace_bytes); rows O.. of dW2 and db2 are zero.
 * ---------------------------------------------------------------------- */
typedef struct {
  int64_t rows, seg, q_ss, q_rs;
  int D, H, O;
} scope_mlp_params;

int scope_coeff_mlp_fwd(const scope_mlp_params* p, const uint16_t* q, const float* w1, const float* b1,
                        const float* w2, const float* b2, uint16_t* y, void* stream);
int scope_coeff_mlp_bwd(const scope_mlp_params* p, const uint16_t* q, const uint16_t* gy, const float* w1,
                        const float* b1, const float* w2, const float* b2, uint16_t* dq, uint16_t* dz1,
                        uint16_t* x1, uint16_t* gyp, void* stream);
int64_t scope_coeff_mlp_wgrad_workspace_bytes(const scope_mlp_params* p);
int scope_coeff_mlp_wgrad(const scope_mlp_params* p, const uint16_t* q, const uint16_t* gyp, const float* w1,
                          const float* b1, const float* w2, float* dw1, float* db1, float* dw2, float* db2,
                          void* workspace, void* stream);

/* ------------------------------------------------------------------------
 * Sliding-window block masks of the layers without the pointer mask.
 * Replaces GPT.create_blockmasks (scoped_medium.py:535-576): the long (W)
 * and short (W // 2) masks of a window of W blocks.
 *   counts [6][NB]: n_partial, n_full (dense_to_ordered counts, :562-563),
 *     then the window-clamped partial / full counts of the long mask
 *     (:568, :570) and of the short mask (the BlockMask's kv_num_blocks and
 *     full_kv_num_blocks; a full count is negative for W = 0, like the
 *     reference's clamp_max(n_full, W - 1)).
 *   partial_idx, full_idx [NB][NB] (or NULL): the ordered rows of
 *     dense_to_ordered (:545-548), shared by both masks.
 *   kv_num_long [NB], kv_idx_long [NB][scope_swa_width(T, bs, W)] and the
 *     short pair [NB][scope_swa_width(T, bs, W / 2)]: the compact lists the
 *     attention kernels read (kept full entries, then kept partial entries,
 *     each descending; the row tail repeats the first entry).
 * ---------------------------------------------------------------------- */
/* row width of a compact list: max(1, min(window_blocks, NB + 1)) */
int scope_swa_width(int64_t T, int bs, int window_blocks);
int scope_swa_blockmask(const int32_t* docs, int64_t T, int bs, int window_blocks, int32_t* counts,
                        int32_t* partial_idx, int32_t* full_idx, int32_t* kv_num_long, int32_t* kv_idx_long,
                        int32_t* kv_num_short, int32_t* kv_idx_short, void* stream);

/* ------------------------------------------------------------------------
 * Fused mask statistics.  Replaces model/attn_bias.py:510-600 (forward debug
 * statistics) and :839-849 (mask debug statistics) and defines the same
 * histograms for the block-scoring mode.  Integer counts go to `counts`
 * (layout SCOPE_ST_*, then the three variable-length histograms), derived
 * fp32 values to `values` (SCOPE_SV_*).
 * ---------------------------------------------------------------------- */
enum {
  SCOPE_ST_DELTA_TOKENS = 0,  /* 16 bins */
  SCOPE_ST_DELTA_BLOCKS = 16, /* 15 bins */
  SCOPE_ST_CENTER = 31,       /* 15 bins */
  SCOPE_ST_DOCSTART = 46,
  SCOPE_ST_OUTSIDE = 47,
  SCOPE_ST_BLOCK0 = 48,
  SCOPE_ST_BLOCK0_EXCL = 49,
  SCOPE_ST_N_CENTRES = 50,
  SCOPE_ST_N_CENTRES_EXCL = 51,
  SCOPE_ST_PTR_DIST = 52,     /* 15 bins, block-scoring picks */
  SCOPE_ST_BS_OUTSIDE = 67,
  SCOPE_ST_BS_BLOCK0 = 68,
  SCOPE_ST_BS_BLOCK0_EXCL = 69,
  SCOPE_ST_BS_DOCSTART = 70,
  SCOPE_ST_BS_N = 71,
  SCOPE_ST_BS_N_EXCL = 72,
  SCOPE_ST_RADIUS0 = 73,
  SCOPE_ST_N_RADIUS = 74,
  SCOPE_ST_FIXED = 75         /* kv_unique[maxkv_bins], radius[radius_bins], extra_sum[extra_bins] follow */
};
enum {
  SCOPE_SV_PI_ENTROPY_MEAN = 0,
  SCOPE_SV_DOCSTART_FRAC = 1,
  SCOPE_SV_OUTSIDE_LOCAL_FRAC = 2,
  SCOPE_SV_BLOCK0_FRAC = 3,
  SCOPE_SV_BLOCK0_FRAC_EXCL = 4,
  SCOPE_SV_RADIUS0_FRAC = 5,
  SCOPE_SV_BS_OUTSIDE_LOCAL_FRAC = 6,
  SCOPE_SV_BS_BLOCK0_FRAC = 7,
  SCOPE_SV_BS_BLOCK0_FRAC_EXCL = 8,
  SCOPE_SV_BS_DOCSTART_FRAC = 9,
  SCOPE_SV_COUNT = 10
};

typedef struct {
  int H, QB, bs, M;
  int64_t T;
  /* forward statistics (model/attn_bias.py:510-600); delta_star / pi non-NULL enables them */
  int64_t stride_h, stride_t;
  int rep_mean;
  int has_docs;           /* docs given to SpectralBias.forward                      */
  int docstart_enabled;   /* docs and (pointer_doc_clamp or reset_active)            */
  int local_blocks_cfg;   /* pointer_local_blocks (constructor)                      */
  float eps;
  /* mask statistics (model/attn_bias.py:839-849); radius non-NULL enables them      */
  int maxkv_bins;         /* _dbg_kv_unique_hist.numel()                             */
  int radius_bins;        /* _dbg_ptr_radius_hist.numel()                            */
  int extra_bins;         /* _dbg_ptr_extra_sum_hist.numel()                         */
  /* block-scoring statistics; picks non-NULL enables them                           */
  int budget;
  int bs_local_blocks;
} scope_stats_params;

int64_t scope_stats_counts_len(const scope_stats_params* p);
int64_t scope_stats_workspace_bytes(const scope_stats_params* p);
int scope_mask_stats(const scope_stats_params* p, const float* delta_star, const float* pi,
                     const int32_t* ds_ptr_fwd, const int32_t* ds_local_fwd, const int32_t* kv_num,
                     const int32_t* radius, const int32_t* picks, const int32_t* ds_ptr,
                     const int32_t* ds_local, int32_t* counts, float* values, void* workspace,
                     void* stream);

/* ------------------------------------------------------------------------
 * Block-sparse flash attention with the SCOPE spectral bias.  Replaces the
 * FlexAttention calls of scoped_medium.py:422, 459-466, 470-476 (Triton
 * templates torch:_inductor/kernel/flex/templates/flex_attention.py.jinja and
 * flex_backwards.py.jinja) for the pointer BlockMask with the
 * document_causal mask_mod (model/attn_bias.py:674-679) and the spectral
 * score_mod (scoped_medium.py:425-457).
 * ---------------------------------------------------------------------- */
enum { SCOPE_BIAS_NONE = 0, SCOPE_BIAS_BLOCK = 1, SCOPE_BIAS_TOKEN = 2 };
enum { SCOPE_GATE_NONE = 0, SCOPE_GATE_SOFTPLUS = 1, SCOPE_GATE_RELU = 2 };

typedef struct {
  int H, D, bs, maxkv;
  int64_t T;
  float scale, beta;
  int bias_mode;           /* SCOPE_BIAS_*                                           */
  int K;                   /* spectral bands, <= 8                                   */
  int use_slope, subtract_b0, gate_kind;
  float ramp_lambda, tau;
  int64_t q_sh, q_st, k_sh, k_st, v_sh, v_st, o_sh, o_st;  /* element strides */
  /* Soft pointer weights (no reference counterpart: the reference selects
   * under torch.no_grad, model/attn_bias.py:623).  pair_bias [H, QB, maxkv]
   * fp32, aligned with kv_idx, is added (natural-log units, not scaled by
   * beta) to every score of the tile (q-block qb, key block kv_idx[h,qb,e]);
   * NULL = none.  The backward writes its gradient, the tile sum of dS, to
   * dpair_bias [H, QB, maxkv] (entries e >= kv_num: 0) when non-NULL. */
  const float* pair_bias;
  float* dpair_bias;
} scope_attn_params;

/* Spectral tables: block mode [NB][16] fp32 (cos ω_k r, sin ω_k r);
 * token mode [T][32] bf16 (cos ω_k j, sin ω_k j as bf16 hi parts, then the
 * bf16 lo parts x - hi).  Replaces
 * SpectralBias._get_trig_tables, model/attn_bias.py:326-340. */
int64_t scope_spectral_table_bytes(int bias_mode, int64_t T, int bs);
int scope_spectral_table(int bias_mode, const float* omegas, int K, int64_t T, int bs, void* table,
                         void* stream);

int scope_attn_fwd(const scope_attn_params* p, const uint16_t* q, const uint16_t* k,
                   const uint16_t* v, const int32_t* kv_num, const int32_t* kv_idx,
                   const int32_t* docs, const int32_t* ds_tok_end, const void* table,
                   const float* coeff_cos, const float* coeff_sin, const float* b0,
                   const float* slope, const float* delta_main, const float* width, uint16_t* out,
                   float* lse, void* stream);

/* Block mass of the attention probabilities: mass[h][qb][kb] = the sum over
 * the q-block's rows i and the key block's keys j of P_ij, for every listed
 * kb (other entries untouched: zero mass first).  Replaces the teacher's
 * per-q-block loop (scoped_medium.py:1799-1819: dense softmax, row sum,
 * scatter_add per key block) for any list — the teacher passes the dense
 * document-causal one.  Two passes over the lists: the LSE of every row
 * (written to lse [H,T]), then the masses; no P·V.  MAXKV <= 1024.
 * mass: fp32 [H, QB, NB]. */
int scope_attn_block_mass(const scope_attn_params* p, const uint16_t* q, const uint16_t* k,
                          const int32_t* kv_num, const int32_t* kv_idx, const int32_t* docs,
                          const int32_t* ds_tok_end, const void* table, const float* coeff_cos,
                          const float* coeff_sin, const float* b0, const float* slope,
                          const float* delta_main, const float* width, float* lse, float* mass,
                          void* stream);

/* ------------------------------------------------------------------------
 * Decode: the attention of one new token (position t) against the KV cache,
 * over its q-block's listed key blocks with the document-causal mask.  No
 * reference counterpart (the reference has no decode path); it serves the
 * token loop of the 16-layer decoder (scoped_medium.py:266-639 forward, one
 * position at a time).  q [H, D] (head stride q_sh); k_cache / v_cache
 * [H, T_cap, D] with (head, token) strides; kv_num [H], kv_idx [H, maxkv];
 * docs [T_cap] (entries up to t are read); out [H, D] bf16 (head stride
 * o_sh); lse [H] natural log (or NULL).  The rows of q, k_cache and v_cache
 * are 16-byte aligned (head and token strides multiples of 8).  The
 * workspace holds one partial (max, sum, P·V row) per (head, list entry).
 * ---------------------------------------------------------------------- */
typedef struct {
  int H, D, bs, maxkv;
  int64_t T_cap;                 /* tokens the cache holds (multiple of bs)  */
  int64_t t;                     /* position of the query                    */
  float scale;
  int64_t q_sh, k_sh, k_st, v_sh, v_st, o_sh;
} scope_decode_params;

int64_t scope_decode_workspace_bytes(const scope_decode_params* p);
int scope_decode_attn(const scope_decode_params* p, const uint16_t* q, const uint16_t* k_cache,
                      const uint16_t* v_cache, const int32_t* kv_num, const int32_t* kv_idx,
                      const int32_t* docs, void* workspace, uint16_t* out, float* lse, void* stream);
/* As scope_decode_attn with the position read from device memory (*t_dev;
 * p->t is ignored; a position outside [0, T_cap) gives an all-zero output and
 * lse = -inf).  No counterpart in the reference, which has no decode loop: for
 * callers that keep the position on the device, such as a decode step
 * captured once in a HIP graph and replayed for every token. */
int scope_decode_attn_at(const scope_decode_params* p, const int64_t* t_dev, const uint16_t* q,
                         const uint16_t* k_cache, const uint16_t* v_cache, const int32_t* kv_num,
                         const int32_t* kv_idx, const int32_t* docs, void* workspace, uint16_t* out,
                         float* lse, void* stream);

/* scope_decode_attn_at with the attention layer's glue fused in, for one
 * token (the decode step inside a block, where the lists are fixed): from
 * qkv [3H, D] bf16 (the qkv projection) it forms q, k and v exactly as
 * scope_decoder_qkv_glue does (eps, va, vb, ve [H·D] or NULL, rotary tables
 * cos_t / sin_t [rot_rows, D/2] with row stride rot_st, at the position
 * *t_dev), writes k and v to row *t_dev of k_cache / v_cache, and attends
 * with the new row; q_out [H, D] (or NULL) receives q.  One launch instead
 * of the glue's and the attention's.  No counterpart in the reference. */
int scope_decode_attn_glue_at(const scope_decode_params* p, const int64_t* t_dev, const uint16_t* qkv,
                              const uint16_t* ve, float va, float vb, float eps, const float* cos_t,
                              const float* sin_t, int64_t rot_rows, int64_t rot_st, uint16_t* k_cache,
                              uint16_t* v_cache, const int32_t* kv_num, const int32_t* kv_idx, const int32_t* docs,
                              void* workspace, uint16_t* out, float* lse, uint16_t* q_out, void* stream);

/* The decoder attention layer's glue for T tokens (replaces, in the token
 * loop and the prefill, scoped_medium.py:339-345 with norm :266-267 and
 * Rotary :291-310): from qkv [T, 3H, D] bf16 (the qkv projection), q and k
 * RMS-normalised (eps: F.rms_norm's default for bf16 inputs is the fp32
 * epsilon) and rotated by the rotary tables cos_t / sin_t
 * [rot_rows, D/2] fp32 (row stride rot_st) at positions pos [T] (int64, on
 * the device), v = va·v + vb·ve (ve [T, H·D] bf16 or NULL).  q -> q_out
 * [T, H, D]; k, v -> row pos[t] (cache_at_pos) or row t of k_out / v_out
 * ([H, rows, D] with the given head and row strides).  A position outside
 * the tables or a row outside [0, rows) writes a zero q and no k/v. */
int scope_decoder_qkv_glue(int T, int H, int D, int64_t rows, float eps, float va, float vb,
                           const uint16_t* qkv, const uint16_t* ve, const int64_t* pos, const float* cos_t,
                           const float* sin_t, int64_t rot_rows, int64_t rot_st, uint16_t* q_out,
                           uint16_t* k_out, uint16_t* v_out, int64_t k_sh, int64_t k_st, int64_t v_sh,
                           int64_t v_st, int cache_at_pos, void* stream);

/* One row-vector product of the decoder's token step, fused with the ops
 * around it (replaces, for one token, the torch chains of scoped_medium.py:
 * the qkv projection of a normed row :339 with norm :266-267, the MLP
 * :318-321, the residual adds :606-613 with the U-net skip :607, and the
 * head :624-626).  x [K] bf16, W [N, K] bf16 with row stride ldw (elements):
 *   x := bf16(x + addx) when addx [K] is given, that row written to xout;
 *   x := F.rms_norm(x) (in fp32 with eps, rounded to bf16) when norm != 0;
 *   z = bf16(W·x) per row, then by epi:
 *     SCOPE_GEMV_PLAIN z -> out bf16 [N]
 *     SCOPE_GEMV_RELU2 bf16(relu(z)²) -> out bf16 [N]
 *     SCOPE_GEMV_RESID bf16(res + z), res [N] bf16 (out may be res) -> out bf16 [N]
 *     SCOPE_GEMV_LOGIT 30·σ(z / 7.5) -> out fp32 [N]
 * K in {256, 512, 1024, 2048, 4096}; x, w, addx and xout 16-byte aligned; out
 * must not overlap x, addx or w.  No counterpart in the reference, whose
 * forward runs these as separate ops on the whole sequence. */
enum { SCOPE_GEMV_PLAIN = 0, SCOPE_GEMV_RELU2 = 1, SCOPE_GEMV_RESID = 2, SCOPE_GEMV_LOGIT = 3 };
int scope_decoder_gemv(int N, int K, int64_t ldw, int norm, float eps, int epi, const uint16_t* x,
                       const uint16_t* addx, uint16_t* xout, const uint16_t* w, const uint16_t* res,
                       void* out, void* stream);

/* The start of a decoder token step (replaces, for one token at the
 * position *t_dev held on the device, the embedding and norm of
 * scoped_medium.py:596-600 with the value embeddings :586-590, and the
 * decoder's token and document bookkeeping): tokens[t] = *tok; docs[t] =
 * docs[t-1] (0 at t = 0) + (*tok == eot); x0 [dm] = F.rms_norm(embed[*tok])
 * (fp32 with eps, rounded to bf16); ve_out [3, dm] row i = table i's row
 * *tok for each of ve0..ve2 given (NULL tables are skipped).  A token
 * outside [0, vocab) or a position outside [0, T_cap) leaves tokens and docs
 * as they are and writes zeros to x0 and the given tables' rows.  dm a
 * multiple of 8; tables and outputs 16-byte aligned.  No counterpart in the
 * reference, which has no decode loop. */
int scope_decoder_step_prologue(const int64_t* tok, const int64_t* t_dev, int64_t T_cap, int64_t vocab, int dm,
                                float eps, int64_t eot, int64_t* tokens, int32_t* docs, const uint16_t* embed,
                                const uint16_t* ve0, const uint16_t* ve1, const uint16_t* ve2, uint16_t* x0,
                                uint16_t* ve_out, void* stream);

/* The greedy choice of the decoder's token loop: *out = the index of the
 * largest of x[0..n) fp32 (the first on ties, as torch.argmax; NaN values
 * are never chosen; all NaN gives 0).  One workgroup.  No counterpart in the
 * reference, which has no decode loop. */
int scope_argmax_f32(const float* x, int64_t n, int64_t* out, void* stream);

int64_t scope_attn_bwd_workspace_bytes(const scope_attn_params* p);
int scope_attn_bwd(const scope_attn_params* p, const uint16_t* q, const uint16_t* k,
                   const uint16_t* v, const uint16_t* out, const uint16_t* dout, const float* lse,
                   const int32_t* kv_num, const int32_t* kv_idx, const int32_t* q_off,
                   const int32_t* q_list, const int32_t* docs, const int32_t* ds_tok_end,
                   const void* table, const float* coeff_cos, const float* coeff_sin,
                   const float* b0, const float* slope, const float* delta_main,
                   const float* width, uint16_t* dq, uint16_t* dk, uint16_t* dv,
                   float* dcoeff_cos, float* dcoeff_sin, float* db0, float* dslope,
                   float* ddelta_main, float* dwidth, void* workspace, void* stream);

/* The backward in stream-ordered phases sharing one workspace:
 * SCOPE_BWD_DQ  (q-major: Δ = rowsum(dO∘O), dQ and the coefficient gradients;
 * it also stores what the kv-major pass reads: the query features in token
 * mode, otherwise the softmax offset of every row and listed key block),
 * then SCOPE_BWD_DKV (kv-major: dK, dV), which is the three steps
 * SCOPE_BWD_DKV_PLAN (work items), SCOPE_BWD_DKV_MAIN (the dK/dV kernel) and
 * SCOPE_BWD_DKV_REDUCE (ordered sum of chunk partials), run in that order.
 * scope_attn_bwd runs everything; the split lets a caller time or overlap the
 * phases.  No reference counterpart beyond the FlexAttention backward that
 * scope_attn_bwd replaces. */
enum {
  SCOPE_BWD_DQ = 1,
  SCOPE_BWD_DKV = 2,
  SCOPE_BWD_DKV_PLAN = 4,
  SCOPE_BWD_DKV_MAIN = 8,
  SCOPE_BWD_DKV_REDUCE = 16
};
int scope_attn_bwd_phase(const scope_attn_params* p, int phases, const uint16_t* q, const uint16_t* k,
                         const uint16_t* v, const uint16_t* out, const uint16_t* dout, const float* lse,
                         const int32_t* kv_num, const int32_t* kv_idx, const int32_t* q_off,
                         const int32_t* q_list, const int32_t* docs, const int32_t* ds_tok_end,
                         const void* table, const float* coeff_cos, const float* coeff_sin,
                         const float* b0, const float* slope, const float* delta_main,
                         const float* width, uint16_t* dq, uint16_t* dk, uint16_t* dv,
                         float* dcoeff_cos, float* dcoeff_sin, float* db0, float* dslope,
                         float* ddelta_main, float* dwidth, void* workspace, void* stream);

/* ---- peak probes (measurement only; no reference counterpart) ------------
 * scope_probe_mfma: blocks x 4 wavefronts each run four independent bf16
 * v_mfma_f32_32x32x16 chains of iters steps, writing one float per thread to
 * out [blocks*256]; scope_probe_mfma_flops gives the FLOP count of one call.
 * scope_probe_mfma_data: the same chains (same FLOP count) on operands from
 * data: operands [blocks*256][16] 16-byte bf16x8 values (8 A and 8 B
 * operands per thread, cycled); iters a multiple of 8.  With random data
 * this is the MFMA rate under the power limit that attention operands see.
 * scope_probe_copy: streaming copy of bytes (multiple of 16, 16-byte aligned
 * buffers); 2·bytes move through HBM. */
int64_t scope_probe_mfma_flops(int blocks, int iters);
int scope_probe_mfma(float* out, int blocks, int iters, void* stream);
int scope_probe_mfma_data(const void* operands, float* out, int blocks, int iters, void* stream);
int scope_probe_copy(const void* src, void* dst, int64_t bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* SCOPE_AMD_H */
