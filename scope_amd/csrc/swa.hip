// Sliding-window block masks of the layers without the pointer mask: the
// long / short pair of GPT.create_blockmasks (scoped_medium.py:535-576).
//
// Block rules (scoped_medium.py:552-563), with lo / hi the document ids of a
// block's first and last token:
//   any(qb, kb) = qb >= kb && lo[qb] <= hi[kb] && hi[qb] >= lo[kb]
//   all(qb, kb) = qb >  kb && lo[qb] == hi[kb] && hi[qb] == lo[kb]
//   partial = any && !all,  full = all.
// Each row is ordered like dense_to_ordered (:545-548), a stable ascending
// argsort flipped: the set's blocks descending, then the other blocks
// descending.  A window of W blocks keeps the leading
//   min(n_full, W - 1)                  full entries    (:570; negative for W = 0)
//   min(n_partial, max(W - n_full, 1))  partial entries (:568)
// and the pair is W (long) and W // 2 (short) (:576).
//
// One workgroup per q-block walks the key blocks from the last one down in
// chunks of 256 (one key block per thread); a ballot per wavefront and an LDS
// carry across the four wavefronts give each key block its position in both
// orderings.  The compact lists the attention kernels read keep the selected
// full entries (descending) followed by the selected partial entries
// (descending); the tail of each row repeats its first entry.
#include <algorithm>

#include "common.h"

namespace scope {

namespace {

struct SwaRow {
  int lo, hi;
};

__device__ __forceinline__ SwaRow swa_row(const int32_t* __restrict__ docs, int bs, int b) {
  return {docs[static_cast<int64_t>(b) * bs], docs[static_cast<int64_t>(b) * bs + bs - 1]};
}

// count of set flags among lanes below this one, and the wavefront total
__device__ __forceinline__ void wave_rank(bool flag, int lane, int& below, int& total) {
  const uint64_t m = __ballot(flag);
  below = __popcll(m & ((uint64_t(1) << lane) - 1));
  total = __popcll(m);
}

}  // namespace

__global__ __launch_bounds__(256) void swa_count_kernel(const int32_t* __restrict__ docs, int bs, int NB,
                                                        int32_t* __restrict__ counts) {
  const int qb = blockIdx.x, tid = threadIdx.x;
  const SwaRow q = swa_row(docs, bs, qb);
  int nf = 0, np = 0;
  for (int kb = tid; kb <= qb; kb += 256) {
    const SwaRow k = swa_row(docs, bs, kb);
    const bool any = q.lo <= k.hi && q.hi >= k.lo;
    const bool all = qb > kb && q.lo == k.hi && q.hi == k.lo;
    nf += all;
    np += any && !all;
  }
  nf = wave_sum_i32(nf);
  np = wave_sum_i32(np);
  __shared__ int red[2][4];
  const int wave = tid >> 6, lane = tid & 63;
  if (lane == 0) {
    red[0][wave] = nf;
    red[1][wave] = np;
  }
  __syncthreads();
  if (tid == 0) {
    counts[qb] = red[1][0] + red[1][1] + red[1][2] + red[1][3];               // n_partial
    counts[NB + qb] = red[0][0] + red[0][1] + red[0][2] + red[0][3];          // n_full
  }
}

// rows: partial_idx / full_idx [NB][NB] (either may be null), compact lists
// [NB][wl] and [NB][ws] with their counts; counts = [6][NB] (n_partial,
// n_full, then the window-clamped partial / full counts of the long and the
// short mask)
__global__ __launch_bounds__(256) void swa_rows_kernel(const int32_t* __restrict__ docs, int bs, int NB, int W, int Ws,
                                                       int32_t* __restrict__ counts, int32_t* __restrict__ partial_idx,
                                                       int32_t* __restrict__ full_idx, int32_t* __restrict__ kv_num_l,
                                                       int32_t* __restrict__ kv_idx_l, int wl,
                                                       int32_t* __restrict__ kv_num_s, int32_t* __restrict__ kv_idx_s,
                                                       int ws) {
  const int qb = blockIdx.x, tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const SwaRow q = swa_row(docs, bs, qb);
  const int np = counts[qb], nf = counts[NB + qb];
  // window clamps (scoped_medium.py:568-570)
  const int cpl = min(np, max(W - nf, 1)), cfl = min(nf, W - 1);
  const int cps = min(np, max(Ws - nf, 1)), cfs = min(nf, Ws - 1);
  const int kfl = max(cfl, 0), kfs = max(cfs, 0);  // full entries the compact lists keep
  if (tid == 0) {
    counts[2 * NB + qb] = cpl;
    counts[3 * NB + qb] = cfl;
    counts[4 * NB + qb] = cps;
    counts[5 * NB + qb] = cfs;
    kv_num_l[qb] = kfl + cpl;
    kv_num_s[qb] = kfs + cps;
  }
  int32_t* rl = kv_idx_l + static_cast<int64_t>(qb) * wl;
  int32_t* rs = kv_idx_s + static_cast<int64_t>(qb) * ws;
  int32_t* pr = partial_idx ? partial_idx + static_cast<int64_t>(qb) * NB : nullptr;
  int32_t* fr = full_idx ? full_idx + static_cast<int64_t>(qb) * NB : nullptr;

  __shared__ int cnt[4][4];  // per wavefront: full, not full, partial, not partial
  // running counts of the chunks above: blocks in / out of each set with larger ids
  int run_f = 0, run_nf = 0, run_p = 0, run_np = 0;
  for (int base = NB - 1; base >= 0; base -= 256) {
    const int kb = base - tid;
    const bool valid = kb >= 0;
    bool all = false, part = false;
    if (valid && kb <= qb) {
      const SwaRow k = swa_row(docs, bs, kb);
      const bool any = q.lo <= k.hi && q.hi >= k.lo;
      all = qb > kb && q.lo == k.hi && q.hi == k.lo;
      part = any && !all;
    }
    int bf, tf, bnf, tnf, bp, tp, bnp, tnp;
    wave_rank(valid && all, lane, bf, tf);
    wave_rank(valid && !all, lane, bnf, tnf);
    wave_rank(valid && part, lane, bp, tp);
    wave_rank(valid && !part, lane, bnp, tnp);
    if (lane == 0) {
      cnt[wave][0] = tf;
      cnt[wave][1] = tnf;
      cnt[wave][2] = tp;
      cnt[wave][3] = tnp;
    }
    __syncthreads();
    int of = run_f, onf = run_nf, op = run_p, onp = run_np;
    for (int w = 0; w < wave; ++w) {
      of += cnt[w][0];
      onf += cnt[w][1];
      op += cnt[w][2];
      onp += cnt[w][3];
    }
    if (valid) {
      // position in the dense_to_ordered row: the set's blocks first, both parts descending
      const int pos_f = all ? of + bf : nf + onf + bnf;
      const int pos_p = part ? op + bp : np + onp + bnp;
      if (fr) fr[pos_f] = kb;
      if (pr) pr[pos_p] = kb;
      if (all) {
        const int i = of + bf;
        if (i < kfl) rl[i] = kb;
        if (i < kfs) rs[i] = kb;
      }
      if (part) {
        const int i = op + bp;
        if (i < cpl) rl[kfl + i] = kb;
        if (i < cps) rs[kfs + i] = kb;
      }
    }
    for (int w = 0; w < 4; ++w) {
      run_f += cnt[w][0];
      run_nf += cnt[w][1];
      run_p += cnt[w][2];
      run_np += cnt[w][3];
    }
    __syncthreads();  // cnt is rewritten by the next chunk
  }
}

// tail of each compact row: its first entry (every row keeps at least the
// diagonal block, a partial entry)
__global__ __launch_bounds__(256) void swa_pad_kernel(int NB, const int32_t* __restrict__ kv_num, int32_t* __restrict__ kv_idx,
                                                      int w) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<int64_t>(NB) * w) return;
  const int qb = static_cast<int>(i / w), j = static_cast<int>(i % w);
  if (j >= kv_num[qb]) kv_idx[i] = kv_idx[static_cast<int64_t>(qb) * w];
}

}  // namespace scope

using namespace scope;

extern "C" int scope_swa_blockmask(const int32_t* docs, int64_t T, int bs, int window_blocks, int32_t* counts,
                                   int32_t* partial_idx, int32_t* full_idx, int32_t* kv_num_long,
                                   int32_t* kv_idx_long, int32_t* kv_num_short, int32_t* kv_idx_short,
                                   void* stream) {
  SCOPE_REQUIRE(docs && counts && kv_num_long && kv_idx_long && kv_num_short && kv_idx_short,
                "scope_swa_blockmask: null pointer");
  SCOPE_REQUIRE(bs > 0 && T > 0 && T % bs == 0, "scope_swa_blockmask: T=%lld must be a positive multiple of bs=%d",
                (long long)T, bs);
  SCOPE_REQUIRE(T < (1ll << 31), "scope_swa_blockmask: T=%lld exceeds int32 token indices", (long long)T);
  SCOPE_REQUIRE(window_blocks >= 0, "scope_swa_blockmask: window_blocks=%d must be >= 0", window_blocks);
  const int NB = static_cast<int>(T / bs);
  // windows beyond NB + 1 blocks keep every entry of both sets, as NB + 1 does
  const int W = min(window_blocks, NB + 1), Ws = min(window_blocks / 2, NB + 1);
  const int wl = max(W, 1), ws = max(Ws, 1);
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(swa_count_kernel, dim3(NB), dim3(256), 0, s, docs, bs, NB, counts);
  int rc = check_launch("swa_count_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(swa_rows_kernel, dim3(NB), dim3(256), 0, s, docs, bs, NB, W, Ws, counts, partial_idx, full_idx,
                     kv_num_long, kv_idx_long, wl, kv_num_short, kv_idx_short, ws);
  rc = check_launch("swa_rows_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(swa_pad_kernel, dim3(ceil_div(static_cast<int64_t>(NB) * wl, 256)), dim3(256), 0, s, NB,
                     kv_num_long, kv_idx_long, wl);
  rc = check_launch("swa_pad_kernel");
  if (rc) return rc;
  hipLaunchKernelGGL(swa_pad_kernel, dim3(ceil_div(static_cast<int64_t>(NB) * ws, 256)), dim3(256), 0, s, NB,
                     kv_num_short, kv_idx_short, ws);
  return check_launch("swa_pad_kernel");
}

extern "C" int scope_swa_width(int64_t T, int bs, int window_blocks) {
  if (bs <= 0 || T <= 0) return 1;
  const int64_t w = std::min<int64_t>(window_blocks, T / bs + 1);
  return w > 1 ? static_cast<int>(w) : 1;
}
