// The MLP of SpectralBias (model/attn_bias.py:271-276, 380-398: Linear(D,
// 2D) -> SiLU -> Linear(2D, 5M+1), shared across heads and applied to every
// (b, h, t) row): the fused forward, the row-wise backward (dq), the fused
// weight and bias gradients that recompute the hidden layer per tile, and
// the general split-row weight gradient of a linear layer below.
//
// Split-row weight gradient: autograd's weight gradient of a linear layer is a GEMM whose
// contraction runs over all B·H·T rows (131072 at T = 16384, H = 8):
//   dW[m][n] = Σ_r A[r][m] B[r][n],   db[m] = Σ_r A[r][m]
// with A the output gradient and B the layer input.  The contraction is
// split over workgroups, each summing a contiguous run of 64-row chunks on
// bf16 MFMAs into fp32 partials, which a second kernel adds in workgroup
// order (no atomics: the result does not depend on scheduling).
//
// Operands: both chunks are copied into swizzled LDS tiles (rows of 128
// columns) by global_load_lds; the MFMA operands of A^T and of B run along
// rows (the contraction index), so both come from transpose reads
// (lds_kmajor_o).  For v_mfma_f32_32x32x16_bf16 with A^T as the A operand
// and B as the B operand, the accumulator of block (mb, nb) holds
// dW[32·mb + 8(r/4) + 4g + r%4][32·nb + lane % 32] in register r.
#include <math.h>

#include <algorithm>

#include "attn_common.h"

namespace scope {

namespace {

constexpr int kWgradThreads = 256;
constexpr int kWgradMaxGroups = 256;
constexpr int kChunkRows = 64;

struct WgradArgs {
  const uint16_t* a;
  const uint16_t* b;
  int64_t rows, seg;  // rows summed over; rows per segment (row r = segment r / seg, row r % seg)
  int64_t a_ss, a_rs, b_ss, b_rs;
  float* part;        // [groups][M·N + M]
  int chunks_per_group;
};

// Copy rows r0 .. r0+63 of an operand with C columns (64, 128 or 256) into
// C/128 swizzled tiles (a 64-column operand fills the left half of one).
template <int C>
__device__ __forceinline__ void wgrad_copy(const uint16_t* x, int64_t ss, int64_t rs, int64_t seg, int64_t r0,
                                           uint16_t* tiles, int tid) {
  constexpr int NTILE = C < 128 ? 1 : C / 128;
  const int64_t s = r0 / seg, t0 = r0 % seg;  // a chunk never spans segments (seg % 64 == 0)
  const uint16_t* base = x + s * ss + t0 * rs;
  const int wave = tid >> 6;
#pragma unroll
  for (int tl = 0; tl < NTILE; ++tl) {
#pragma unroll
    for (int jj = 0; jj < 1024 / kWgradThreads; ++jj) {
      // physical 16-byte slot idx of the tile: row idx/16, holding logical chunk (idx%16) ^ swz(row)
      const int idx = jj * kWgradThreads + tid;
      const int r = idx >> 4, c = (idx & 15) ^ swz(r);
      uint16_t* dst = tiles + tl * (64 * 128) + (jj * kWgradThreads + wave * 64) * 8;
      const uint32_t off = static_cast<uint32_t>((r * rs + tl * 128 + c * 8) * 2);
      if (C >= 128 || c < C / 8) g2lds16(base, off, dst);
    }
  }
}

// Which accumulator blocks a wavefront owns: the four wavefronts split the
// MB x NB grid of 32x32 blocks by m blocks (MB % 4 == 0), else by n blocks
// (NB % 4 == 0), else two by two.
template <int MB, int NB>
struct WgradSplit {
  static constexpr bool BY_M = MB % 4 == 0;
  static constexpr bool BY_N = !BY_M && NB % 4 == 0;
  static constexpr int WM = BY_M ? MB / 4 : (BY_N ? MB : MB / 2);  // m blocks per wavefront
  static constexpr int WN = BY_M ? NB : (BY_N ? NB / 4 : NB / 2);  // n blocks per wavefront
  __device__ static int mb(int wave, int i) { return BY_M ? wave + 4 * i : (BY_N ? i : (wave / 2) * WM + i); }
  __device__ static int nb(int wave, int j) { return BY_M ? j : (BY_N ? wave + 4 * j : (wave % 2) * WN + j); }
  // the column sums of A are taken by the wavefronts that own n block 0
  __device__ static bool colsum(int wave) { return BY_M ? true : (BY_N ? wave == 0 : wave % 2 == 0); }
};

// global_load_lds copies one thread issues per chunk of an operand with C columns
template <int C>
constexpr int kCopiesPerChunk = (C < 128 ? 1 : C / 128) * (1024 / kWgradThreads);

template <int MB, int NB>
__global__ __launch_bounds__(kWgradThreads) void wgrad_kernel(WgradArgs g) {
  constexpr int M = 32 * MB, N = 32 * NB;
  constexpr int TA = M < 128 ? 1 : M / 128, TB = N < 128 ? 1 : N / 128;
  using S = WgradSplit<MB, NB>;
  static_assert(S::WM * S::WN <= 8, "wgrad_kernel: at most 8 accumulator blocks per wavefront");
  // three chunk buffers: chunk c+2 is copied while chunk c is summed
  __shared__ __attribute__((aligned(16))) uint16_t sa[3][TA * 64 * 128];
  __shared__ __attribute__((aligned(16))) uint16_t sb[3][TB * 64 * 128];

  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  const int64_t chunks = g.rows / kChunkRows;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * g.chunks_per_group;
  const int64_t c1 = c0 + g.chunks_per_group < chunks ? c0 + g.chunks_per_group : chunks;
  const TileOffs to = tile_offs(lane);

  f32x16_t acc[S::WM][S::WN];
#pragma unroll
  for (int i = 0; i < S::WM; ++i)
#pragma unroll
    for (int j = 0; j < S::WN; ++j) acc[i][j] = zero16();
  float cs[S::WM];
#pragma unroll
  for (int i = 0; i < S::WM; ++i) cs[i] = 0.f;
  const bool do_cs = S::colsum(wave);
  // vmcnt counts this wavefront's copies in issue order: with chunk c+1's copies
  // issued after chunk c's, "at most one chunk's copies outstanding" means chunk c landed
  constexpr int kPerChunk = kCopiesPerChunk<M> + kCopiesPerChunk<N>;
  static_assert(kPerChunk <= 15, "wgrad_kernel: vmcnt field");
  auto wait_vm_copies_but_one_chunk = []() __attribute__((always_inline)) {
    // s_waitcnt vmcnt(kPerChunk) (expcnt and lgkmcnt at their maximum: not waited for)
    __builtin_amdgcn_s_waitcnt(0x0F70 | kPerChunk);
  };

  auto issue = [&](int64_t c, int buf) __attribute__((always_inline)) {
    wgrad_copy<M>(g.a, g.a_ss, g.a_rs, g.seg, c * kChunkRows, sa[buf], tid);
    wgrad_copy<N>(g.b, g.b_ss, g.b_rs, g.seg, c * kChunkRows, sb[buf], tid);
  };
  if (c0 < c1) issue(c0, 0);
  if (c0 + 1 < c1) issue(c0 + 1, 1);
  for (int64_t c = c0; c < c1; ++c) {
    const int buf = static_cast<int>((c - c0) % 3);
    // chunk c is the older of at most two chunks in flight: wait for it alone
    if (c + 1 < c1)
      wait_vm_copies_but_one_chunk();
    else
      wait_vm0();
    __syncthreads();  // chunk c is in buffer buf; every wavefront is done with the buffer of chunk c-1
    if (c + 2 < c1) issue(c + 2, static_cast<int>((c + 2 - c0) % 3));
#pragma unroll
    for (int ks = 0; ks < kChunkRows / 16; ++ks) {
      uint4 av[S::WM], bv[S::WN];
#pragma unroll
      for (int i = 0; i < S::WM; ++i) {
        const int mb = S::mb(wave, i);
        av[i] = lds_kmajor_o(sa[buf] + (mb / 4) * (64 * 128), to, 16 * ks, mb % 4);
      }
#pragma unroll
      for (int j = 0; j < S::WN; ++j) {
        const int nb = S::nb(wave, j);
        bv[j] = lds_kmajor_o(sb[buf] + (nb / 4) * (64 * 128), to, 16 * ks, nb % 4);
      }
#pragma unroll
      for (int i = 0; i < S::WM; ++i)
#pragma unroll
        for (int j = 0; j < S::WN; ++j) acc[i][j] = mfma32(av[i], bv[j], acc[i][j]);
      if (do_cs) {
#pragma unroll
        for (int i = 0; i < S::WM; ++i) {
          const uint32_t w4[4] = {av[i].x, av[i].y, av[i].z, av[i].w};
#pragma unroll
          for (int q = 0; q < 4; ++q) cs[i] += bf16_lo(w4[q]) + bf16_hi(w4[q]);
        }
      }
    }
  }
  wait_vm0();  // no copy may still target LDS when the workgroup exits

  // partials of this workgroup: dW block rows as above, then the column sums
  float* part = g.part + static_cast<int64_t>(blockIdx.x) * (M * N + M);
  const int gq = lane / 32, c = lane % 32;
#pragma unroll
  for (int i = 0; i < S::WM; ++i) {
    const int mb = S::mb(wave, i);
#pragma unroll
    for (int j = 0; j < S::WN; ++j) {
      const int nb = S::nb(wave, j);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = 32 * mb + 8 * (r / 4) + 4 * gq + (r % 4);
        part[m * N + 32 * nb + c] = acc[i][j][r];
      }
    }
    if (do_cs) {
      // lanes l and l ^ 32 hold different rows of the same column
      const float t = cs[i] + __shfl_xor(cs[i], 32, 64);
      if (gq == 0) part[M * N + 32 * mb + c] = t;
    }
  }
}

__device__ __forceinline__ float round_bf16(float x) { return static_cast<float>(static_cast<__bf16>(x)); }

// dw[m][n] (then db[m]) = the sum over workgroups.  A workgroup takes 64
// consecutive elements; its four wavefronts sum a quarter of the groups each
// with eight interleaved accumulators (eight loads in flight per lane), and
// the quarters are added in order: a fixed association, so the result does
// not depend on scheduling.
__device__ __forceinline__ void wgrad_reduce_block(int blk, const float* __restrict__ part, int groups, int MN, int M,
                                                   int rnd, float* __restrict__ dw, float* __restrict__ db) {
  __shared__ float qsum[4][64];
  const int e = blk * 64 + threadIdx.x % 64, quarter = threadIdx.x / 64;
  const int stride = MN + M;
  const int per_q = (groups + 3) / 4;
  const int w0 = quarter * per_q, w1 = min(groups, w0 + per_q);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if (e < stride) {
    int w = w0;
    for (; w + 8 <= w1; w += 8) {
#pragma unroll
      for (int u = 0; u < 8; ++u) acc[u] += part[static_cast<int64_t>(w + u) * stride + e];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (w + u < w1) acc[u] += part[static_cast<int64_t>(w + u) * stride + e];
  }
  qsum[quarter][threadIdx.x % 64] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  __syncthreads();
  if (quarter != 0 || e >= stride || (e >= MN && !db)) return;
  const int i = threadIdx.x;
  float t = ((qsum[0][i] + qsum[1][i]) + qsum[2][i]) + qsum[3][i];
  if (rnd) t = round_bf16(t);
  if (e < MN)
    dw[e] = t;
  else
    db[e - MN] = t;
}

__global__ __launch_bounds__(256) void wgrad_reduce_kernel(const float* __restrict__ part, int groups, int MN, int M,
                                                           int rnd, float* __restrict__ dw, float* __restrict__ db) {
  wgrad_reduce_block(blockIdx.x, part, groups, MN, M, rnd, dw, db);
}

int wgrad_groups(const scope_wgrad_params* p) {
  const int64_t chunks = p->rows / kChunkRows;
  return static_cast<int>(chunks < kWgradMaxGroups ? chunks : kWgradMaxGroups);
}

template <int MB, int NB>
void launch_wgrad(const WgradArgs& g, int groups, hipStream_t s) {
  hipLaunchKernelGGL((wgrad_kernel<MB, NB>), dim3(groups), dim3(kWgradThreads), 0, s, g);
}


// ---------------------------------------------------------------------------
// The MLP itself, fused: forward y = W2·SiLU(W1·q + b1) + b2 per row and the
// backward's row-wise part (model/attn_bias.py:271-276, 380-386; autograd of
// two F.linear and a SiLU on bf16 rows).
// ---------------------------------------------------------------------------
// One 512-thread workgroup per CU walks tiles of 256 rows, 32 rows per
// wavefront.  W1 [256][128] and W2^T [256][64] (the module's fp32 weights
// rounded to bf16, as the reference's .to(q.dtype)) sit in LDS as swizzled
// 256-byte-row tiles, so the attention kernels' operand reads serve both
// orientations.  Per hidden block of 32 units (v_mfma_f32_32x32x16_bf16):
//   Z^T = W1·X^T (A: W1 rows, B: the wavefront's rows of q in registers),
//   x1 = SiLU(bf16(Z^T + b1)) in the C layout, which is directly the B
//   operand of Y^T += W2·X1^T (A: W2^T through transpose reads).
// The backward recomputes Z^T, takes dX1^T = W2^T·gY^T, dZ1 = SiLU'(z)·dx1
// and dQ^T += W1^T·dZ1^T, and writes dq and the output gradient padded to 64
// columns (for the fused weight-gradient kernel below), and x1 and dz1 when
// asked (for the split-row kernel above).  b1 enters Z^T as one
// more k-step (a row of ones against the bias).  Every intermediate is
// rounded to bf16 where the reference's tensors are (z1, x1, dx1, dz1): the
// head's outputs downstream (the peak positions among them) are not
// continuous in y, so the MLP keeps the reference's rounding points.
constexpr int kMlpD = 128, kMlpH = 256, kMlpOMax = 64;
constexpr int kMlpThreads = 512;
constexpr int kMlpTileRows = 256;  // 8 wavefronts x 32 rows

struct MlpArgs {
  const uint16_t* q;
  int64_t rows, seg, q_ss, q_rs;  // row r of q: q + (r / seg)·q_ss + (r % seg)·q_rs (elements)
  const float* w1;                // [256][128]
  const float* b1;                // [256]
  const float* w2;                // [O][256]
  const float* b2;                // [O]
  int O;
  uint16_t* y;                    // forward: [rows][O]
  const uint16_t* gy;             // backward: [rows][O]
  uint16_t* dq;                   // [rows][128]
  uint16_t* dz1;                  // [rows][256]
  uint16_t* x1;                   // [rows][256]
  uint16_t* gyp;                  // [rows][64], the output gradient padded with zeros
};

struct MlpLds {
  uint16_t w1[kMlpH * 128];   // W1, swizzled rows of 128 (swz_off)
  uint16_t w2t[kMlpH * 128];  // W2^T: row h holds W2[0..O-1][h], zeros up to column 63 (swz_off)
  uint16_t b1[kMlpH];  // bf16 bits: the A operand of the bias k-step
  float b2[kMlpOMax];
};

__device__ __forceinline__ float bf16_round(float x) { return static_cast<float>(static_cast<__bf16>(x)); }

// q's row r0 (a wavefront's first row; its 32 rows lie in one segment, as
// segments are a multiple of 32 rows): the segment split once per
// wavefront, in scalar registers
__device__ __forceinline__ const uint16_t* mlp_wave_rows(const MlpArgs& g, int64_t r0) {
  const int64_t r = static_cast<int64_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(r0 >> 5))) * 32;
  return g.q + (r / g.seg) * g.q_ss + (r % g.seg) * g.q_rs;
}

__device__ __forceinline__ float mlp_sigmoid(float z) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-z * kLog2e));
}

__device__ void mlp_load_weights(const MlpArgs& g, MlpLds& L, int tid) {
  // every load of the thread is issued before the first conversion (a loop
  // of load, convert, store waits one memory latency per step)
  constexpr int N1 = kMlpH * kMlpD / 4 / kMlpThreads;  // float4 of W1 per thread: 16
  constexpr int N2 = kMlpH * kMlpOMax / kMlpThreads;   // elements of W2^T per thread: 32
  float4 w1v[N1];
  float w2v[N2];
#pragma unroll
  for (int j = 0; j < N1; ++j) {
    const int i = tid + j * kMlpThreads, r = i / (kMlpD / 4), d = (i % (kMlpD / 4)) * 4;
    w1v[j] = *reinterpret_cast<const float4*>(g.w1 + r * kMlpD + d);
  }
#pragma unroll
  for (int j = 0; j < N2; ++j) {
    // element (h, o) of W2^T = W2[o][h]: consecutive threads read consecutive h
    const int i = tid + j * kMlpThreads, h = i % kMlpH, o = i / kMlpH;
    w2v[j] = o < g.O ? g.w2[o * kMlpH + h] : 0.f;
  }
  const float b1v = g.b1[tid % kMlpH];
  const float b2v = tid < g.O ? g.b2[tid] : 0.f;
#pragma unroll
  for (int j = 0; j < N1; ++j) {
    const int i = tid + j * kMlpThreads, r = i / (kMlpD / 4), d = (i % (kMlpD / 4)) * 4;
    *reinterpret_cast<uint2*>(&L.w1[swz_off(r, d)]) =
        make_uint2(cvt_pk_bf16(w1v[j].x, w1v[j].y), cvt_pk_bf16(w1v[j].z, w1v[j].w));
  }
#pragma unroll
  for (int j = 0; j < N2; ++j) {
    const int i = tid + j * kMlpThreads, h = i % kMlpH, o = i / kMlpH;
    L.w2t[swz_off(h, o)] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(w2v[j]));
  }
  if (tid < kMlpH) L.b1[tid] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(b1v));
  if (tid < kMlpOMax) L.b2[tid] = bf16_round(b2v);
}

// The bias as one more k-step of Z^T = W1·X^T + b1·1^T: A holds b1 of the
// lane's hidden unit in slot 0 of lane group 0 (k = 0), B a row of ones
// (kOnes: 1.0 in k = 0, lane group 0), every other product zero.
__device__ __forceinline__ uint4 mlp_bias_a(const MlpLds& L, int hb, int lr, int gq) {
  return make_uint4(gq == 0 ? static_cast<uint32_t>(L.b1[32 * hb + lr]) : 0u, 0u, 0u, 0u);
}
__device__ __forceinline__ uint4 mlp_ones_b(int gq) { return make_uint4(gq == 0 ? 0x3F80u : 0u, 0u, 0u, 0u); }

// Z^T + b1 of hidden block hb for this wavefront's 32 rows (xb: the rows' q as B operands)
__device__ __forceinline__ f32x16_t mlp_z(const MlpLds& L, const TileOffs& to, int hb, const uint4 (&xb)[8], int lr,
                                          int gq) {
  f32x16_t z = mfma32(mlp_bias_a(L, hb, lr, gq), mlp_ones_b(gq), zero16());
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) z = mfma32(lds_row8_o(L.w1, to, 32 * hb, ks), xb[ks], z);
  return z;
}

__global__ __launch_bounds__(kMlpThreads) void mlp_fwd_kernel(MlpArgs g) {
  __shared__ MlpLds L;
  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64, gq = lane / 32, lr = lane % 32;
  mlp_load_weights(g, L, tid);
  __syncthreads();
  const TileOffs to = tile_offs(lane);
  const int64_t tiles = (g.rows + kMlpTileRows - 1) / kMlpTileRows;
  for (int64_t t = blockIdx.x; t < tiles; t += gridDim.x) {
    const int64_t row = t * kMlpTileRows + wave * 32 + lr;  // rows is a multiple of 32: whole wavefronts
    if (t * kMlpTileRows + wave * 32 >= g.rows) break;
    const uint16_t* qp = mlp_wave_rows(g, t * kMlpTileRows + wave * 32) + lr * g.q_rs + 8 * gq;
    uint4 xb[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) xb[ks] = *reinterpret_cast<const uint4*>(qp + 16 * ks);
    // software pipeline over the hidden blocks: the Z^T MFMAs of block hb+1
    // (operands read at the top of the step) run under the SiLU of block hb
    f32x16_t y[2] = {zero16(), zero16()};
    f32x16_t z = mlp_z(L, to, 0, xb, lr, gq);
#pragma unroll
    for (int hb = 0; hb < 8; ++hb) {
      uint4 an[8], aw[4];
      if (hb < 7) {
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) an[ks] = lds_row8_o(L.w1, to, 32 * (hb + 1), ks);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) aw[i] = lds_kmajor_o(L.w2t, to, 32 * hb + 16 * (i / 2), i % 2);
      f32x16_t zn = zero16();
      if (hb < 7) {
        zn = mfma32(mlp_bias_a(L, hb + 1, lr, gq), mlp_ones_b(gq), zn);
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) zn = mfma32(an[ks], xb[ks], zn);
      }
      uint32_t w[8];
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        const float z0 = bf16_round(z[r]), z1 = bf16_round(z[r + 1]);  // z1 is a bf16 tensor in the reference
        w[r / 2] = cvt_pk_bf16(z0 * mlp_sigmoid(z0), z1 * mlp_sigmoid(z1));
      }
      const uint4 xp[2] = {make_uint4(w[0], w[1], w[2], w[3]), make_uint4(w[4], w[5], w[6], w[7])};
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i % 2] = mfma32(aw[i], xp[i / 2], y[i % 2]);
      z = zn;
    }
    uint16_t* yp = g.y + row * g.O;
#pragma unroll
    for (int ob = 0; ob < 2; ++ob)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int o = 32 * ob + 8 * (r / 4) + 4 * gq + r % 4;
        if (o < g.O) yp[o] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(y[ob][r] + L.b2[o]));
      }
  }
}

__global__ __launch_bounds__(kMlpThreads) void mlp_bwd_kernel(MlpArgs g) {
  __shared__ MlpLds L;
  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64, gq = lane / 32, lr = lane % 32;
  mlp_load_weights(g, L, tid);
  __syncthreads();
  const TileOffs to = tile_offs(lane);
  const int64_t tiles = (g.rows + kMlpTileRows - 1) / kMlpTileRows;
  for (int64_t t = blockIdx.x; t < tiles; t += gridDim.x) {
    const int64_t row = t * kMlpTileRows + wave * 32 + lr;
    if (t * kMlpTileRows + wave * 32 >= g.rows) break;
    const uint16_t* qp = mlp_wave_rows(g, t * kMlpTileRows + wave * 32) + lr * g.q_rs + 8 * gq;
    uint4 xb[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) xb[ks] = *reinterpret_cast<const uint4*>(qp + 16 * ks);
    // the output gradient as B operands of dX1^T (k = outputs 16ks + 8gq .. +7), zero past O;
    // the same values padded to 64 columns for the weight gradient
    uint4 gb[4];
    const uint16_t* gp = g.gy + row * g.O;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int o = 16 * ks + 8 * gq + 2 * j;
        const uint32_t lo = o < g.O ? gp[o] : 0u, hi = o + 1 < g.O ? gp[o + 1] : 0u;
        w[j] = lo | (hi << 16);
      }
      gb[ks] = make_uint4(w[0], w[1], w[2], w[3]);
      *reinterpret_cast<uint4*>(g.gyp + row * kMlpOMax + 16 * ks + 8 * gq) = gb[ks];
    }
    // per hidden block: Z^T and dX1^T, the VALU work, the dQ^T products (the
    // other wavefront of the SIMD fills the gaps; holding the next block's
    // accumulators as well would spill)
    f32x16_t dq[4] = {zero16(), zero16(), zero16(), zero16()};
    auto zdx = [&](int hb, f32x16_t& z, f32x16_t& dx) __attribute__((always_inline)) {
      uint4 an[8], ag[4];
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) an[ks] = lds_row8_o(L.w1, to, 32 * hb, ks);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) ag[ks] = lds_row8_o(L.w2t, to, 32 * hb, ks);
      z = mfma32(mlp_bias_a(L, hb, lr, gq), mlp_ones_b(gq), zero16());
      dx = zero16();
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        z = mfma32(an[ks], xb[ks], z);
        if (ks < 4) dx = mfma32(ag[ks], gb[ks], dx);
      }
    };
#pragma unroll
    for (int hb = 0; hb < 8; ++hb) {
      f32x16_t z, dx;
      zdx(hb, z, dx);
      uint32_t xw[8], dw[8];
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        float xv[2], dv[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          // z1 and dx1 = gy·W2 are bf16 tensors in the reference
          const float zz = bf16_round(z[r + i]);
          const float sg = mlp_sigmoid(zz);
          xv[i] = zz * sg;
          dv[i] = bf16_round(dx[r + i]) * (sg * fmaf(zz, 1.f - sg, 1.f));  // SiLU'(z1)·dx1
        }
        xw[r / 2] = cvt_pk_bf16(xv[0], xv[1]);
        dw[r / 2] = cvt_pk_bf16(dv[0], dv[1]);
      }
      if (g.x1) {
        // x1 and dz1 rows: hidden 32hb + 8q + 4gq .. +3 in register quad q
        uint16_t* xr = g.x1 + row * kMlpH + 32 * hb + 4 * gq;
        uint16_t* dr = g.dz1 + row * kMlpH + 32 * hb + 4 * gq;
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
          *reinterpret_cast<uint2*>(xr + 8 * qd) = make_uint2(xw[2 * qd], xw[2 * qd + 1]);
          *reinterpret_cast<uint2*>(dr + 8 * qd) = make_uint2(dw[2 * qd], dw[2 * qd + 1]);
        }
      }
      const uint4 dp[2] = {make_uint4(dw[0], dw[1], dw[2], dw[3]), make_uint4(dw[4], dw[5], dw[6], dw[7])};
#pragma unroll
      for (int i = 0; i < 8; ++i) dq[i % 4] = mfma32(lds_kmajor_o(L.w1, to, 32 * hb + 16 * (i / 4), i % 4), dp[i / 4], dq[i % 4]);
    }
    // dq rows: columns 32md + 8q + 4gq .. +3 in register quad q
    uint16_t* dqp = g.dq + row * kMlpD + 4 * gq;
#pragma unroll
    for (int md = 0; md < 4; ++md)
#pragma unroll
      for (int qd = 0; qd < 4; ++qd)
        *reinterpret_cast<uint2*>(dqp + 32 * md + 8 * qd) =
            make_uint2(cvt_pk_bf16(dq[md][4 * qd], dq[md][4 * qd + 1]), cvt_pk_bf16(dq[md][4 * qd + 2], dq[md][4 * qd + 3]));
  }
}

// ---------------------------------------------------------------------------
// The MLP's weight and bias gradients without its intermediates in memory:
//   dW1 = Σ_r dz1[r]^T q[r], db1 = Σ_r dz1[r], dW2 = Σ_r gy[r]^T x1[r],
//   db2 = Σ_r gy[r]
// over all rows, with z1, x1 and dz1 recomputed per tile as in the row-wise
// backward (the same bf16 rounding points).  A workgroup takes four hidden
// blocks of 32 units (4·hq .. 4·hq + 3) over a contiguous run of 64-row tiles;
// wavefront w computes hidden block 4·hq + w/2 for rows 32·(w%2) .. +31:
//   Z = q·W1[hb]^T + b1[hb] and dX1 = gy·W2[:, hb] (v_mfma_f32_32x32x16_bf16:
//   the tile's q and gy rows as A operands through LDS row reads, W1[hb] and
//   W2[:, hb] as B operands in registers, b1 as one more k-step);
//   their C layout (lane: hidden unit, register r: row 8(r/4) + 4g + r%4) is
//   directly the A operand of dW1[hb] += dz1^T·q and dW2^T[hb] += x1^T·gy,
//   whose k runs over rows in the slot order of the transpose reads
//   (lds_kmajor_o) of the same q and gy tiles.
// Four tile buffers: the copies run three tiles ahead of the MFMAs.  The two
// wavefronts of a hidden block add their sums in LDS in a fixed order; each
// workgroup writes one partial per row group, which wgrad_reduce_kernel adds
// in group order (no atomics anywhere).
// ---------------------------------------------------------------------------
constexpr int kMwTileRows = 64;
constexpr int kMwBufs = 4;
constexpr int kMwMaxGroups = 128;
constexpr int kMwPart1 = kMlpH * kMlpD + kMlpH;         // dW1 [256][128], db1 [256]
constexpr int kMwPart2 = kMlpOMax * kMlpH + kMlpOMax;   // dW2 [64][256], db2 [64]
constexpr int kMwCopies = 2 * kMwTileRows * 16 / kMlpThreads;  // global_load_lds per thread and tile (q, gy)

struct MlpWgradLds {
  uint16_t q[kMwBufs][kMwTileRows * 128];   // q rows, swizzled 256-byte rows (swz_off)
  uint16_t gy[kMwBufs][kMwTileRows * 128];  // gy padded to 64 columns, in the same 256-byte-row layout
};
// the two wavefronts' sums of one hidden block, added in LDS at the end
struct MlpWgradSum {
  float dw1[32 * kMlpD];      // [hidden][d]
  float dw2[32 * kMlpOMax];   // [hidden][o]
  float db1[32];
  float db2[kMlpOMax];
};
static_assert(4 * sizeof(MlpWgradSum) <= sizeof(MlpWgradLds), "mlp_wgrad_kernel: the sums reuse the tile buffers");
static_assert(kMwCopies == 4, "mlp_wgrad_kernel: the waits below count four copies per tile");

// both reductions of the MLP's partials in one launch: blocks [0, nb1) sum
// part1 (dW1, db1), the rest part2 (dW2, db2)
__global__ __launch_bounds__(256) void mlp_wgrad_reduce_kernel(const float* __restrict__ part1,
                                                               const float* __restrict__ part2, int groups, int nb1,
                                                               float* __restrict__ dw1, float* __restrict__ db1,
                                                               float* __restrict__ dw2, float* __restrict__ db2) {
  if (static_cast<int>(blockIdx.x) < nb1)
    wgrad_reduce_block(blockIdx.x, part1, groups, kMlpH * kMlpD, kMlpH, 1, dw1, db1);
  else
    wgrad_reduce_block(blockIdx.x - nb1, part2, groups, kMlpOMax * kMlpH, kMlpOMax, 1, dw2, db2);
}

__global__ __launch_bounds__(kMlpThreads) void mlp_wgrad_kernel(MlpArgs g, float* __restrict__ part1,
                                                                float* __restrict__ part2, int groups,
                                                                int tiles_per_group) {
  __shared__ __attribute__((aligned(16))) MlpWgradLds L;
  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64, gq = lane / 32, lr = lane % 32;
  // workgroup -> (hidden quad hq, row group gi); dispatch is round robin over
  // the 8 XCDs, so with groups % 8 == 0 both quads of a row group share one
  // XCD (and its L2 copy of the rows)
  int hq, gi;
  if (groups % 8 == 0) {
    const int x = blockIdx.x % 8, j = blockIdx.x / 8;
    hq = j % 2;
    gi = (j / 2) * 8 + x;
  } else {
    hq = blockIdx.x % 2;
    gi = blockIdx.x / 2;
  }
  const int hl = wave / 2, rsub = wave % 2;
  const int hb = 4 * hq + hl;
  const int h = 32 * hb + lr;  // this lane's hidden unit in the C layout

  // B operands in registers: W1[h][16ks + 8gq .. +7] and W2[16ks + 8gq .. +7][h] (zero past O), bf16
  uint4 wb[8], w2b[4];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    const float4 u = *reinterpret_cast<const float4*>(g.w1 + h * kMlpD + 16 * ks + 8 * gq);
    const float4 v = *reinterpret_cast<const float4*>(g.w1 + h * kMlpD + 16 * ks + 8 * gq + 4);
    wb[ks] = make_uint4(cvt_pk_bf16(u.x, u.y), cvt_pk_bf16(u.z, u.w), cvt_pk_bf16(v.x, v.y), cvt_pk_bf16(v.z, v.w));
  }
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    float w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int o = 16 * ks + 8 * gq + j;
      w[j] = o < g.O ? g.w2[o * kMlpH + h] : 0.f;
    }
    w2b[ks] = make_uint4(cvt_pk_bf16(w[0], w[1]), cvt_pk_bf16(w[2], w[3]), cvt_pk_bf16(w[4], w[5]),
                         cvt_pk_bf16(w[6], w[7]));
  }
  // the bias k-step: a column of ones (A, k = 0 in lane group 0) against b1[h] (B)
  const uint4 ones_a = mlp_ones_b(gq);
  const uint4 bias_b =
      make_uint4(gq == 0 ? static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(g.b1[h]))) : 0u,
                 0u, 0u, 0u);

  const int64_t tiles = g.rows / kMwTileRows;  // rows is a multiple of 128 (checked on the host)
  const int64_t t0 = static_cast<int64_t>(gi) * tiles_per_group;
  const int64_t t1 = t0 + tiles_per_group < tiles ? t0 + tiles_per_group : tiles;
  // tile copies: q rows (16 chunks of 16 bytes) and gy rows (8 chunks; the
  // other half of each 256-byte row stays unused), two of each per thread
  auto issue = [&](int64_t t, int buf) __attribute__((always_inline)) {
    const int64_t r0 = t * kMwTileRows;
    const uint16_t* qb = g.q + (r0 / g.seg) * g.q_ss + (r0 % g.seg) * g.q_rs;  // a tile never spans segments
    const uint16_t* gb = g.gyp + r0 * kMlpOMax;
#pragma unroll
    for (int jj = 0; jj < kMwTileRows * 16 / kMlpThreads; ++jj) {
      const int idx = jj * kMlpThreads + tid;
      const int r = idx >> 4, c = (idx & 15) ^ swz(r);
      g2lds16(qb, static_cast<uint32_t>((r * static_cast<int>(g.q_rs) + c * 8) * 2),
              L.q[buf] + (jj * kMlpThreads + wave * 64) * 8);
    }
#pragma unroll
    for (int jj = 0; jj < kMwTileRows * 16 / kMlpThreads; ++jj) {
      const int idx = jj * kMlpThreads + tid;
      const int r = idx >> 4, c = (idx & 15) ^ swz(r);
      // every wavefront's copy has active lanes: 4 rows of 16 slots, 8 of them holding gy
      if (c < kMlpOMax / 8)
        g2lds16(gb, static_cast<uint32_t>((r * kMlpOMax + c * 8) * 2), L.gy[buf] + (jj * kMlpThreads + wave * 64) * 8);
    }
  };

  const TileOffs to = tile_offs(lane);
  f32x16_t acc1[4], acc2[2];  // dW1[hb] (d blocks), dW2^T[hb] (o blocks)
#pragma unroll
  for (int i = 0; i < 4; ++i) acc1[i] = zero16();
  acc2[0] = acc2[1] = zero16();
  float db1 = 0.f, db2[2] = {0.f, 0.f};
  const bool do_db2 = hb == 0;
  for (int i = 0; i < kMwBufs - 1; ++i)
    if (t0 + i < t1) issue(t0 + i, i);
  for (int64_t t = t0; t < t1; ++t) {
    const int buf = static_cast<int>((t - t0) % kMwBufs);
    // tiles t+1 .. t+ahead were issued after tile t: wait for tile t alone
    const int64_t ahead = (t1 - 1 - t) < kMwBufs - 2 ? (t1 - 1 - t) : kMwBufs - 2;
    if (ahead >= 2)
      __builtin_amdgcn_s_waitcnt(0x0F70 | 8);  // vmcnt(2·kMwCopies)
    else if (ahead == 1)
      __builtin_amdgcn_s_waitcnt(0x0F70 | 4);  // vmcnt(kMwCopies)
    else
      wait_vm0();
    __syncthreads();  // tile t is in buf for everyone; every wavefront is done with tile t-1's buffer
    if (t + kMwBufs - 1 < t1) issue(t + kMwBufs - 1, static_cast<int>((t + kMwBufs - 1 - t0) % kMwBufs));
    const uint16_t* qt = L.q[buf];
    const uint16_t* gt = L.gy[buf];
    f32x16_t z = mfma32(ones_a, bias_b, zero16());
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) z = mfma32(lds_row8_o(qt, to, 32 * rsub, ks), wb[ks], z);
    f32x16_t dx = zero16();
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) dx = mfma32(lds_row8_o(gt, to, 32 * rsub, ks), w2b[ks], dx);
    uint32_t xw[8], dw[8];
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      float xv[2], dv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const float zz = bf16_round(z[r + i]);
        const float sg = mlp_sigmoid(zz);
        xv[i] = zz * sg;
        dv[i] = bf16_round(dx[r + i]) * (sg * fmaf(zz, 1.f - sg, 1.f));  // SiLU'(z1)·dx1
      }
      xw[r / 2] = cvt_pk_bf16(xv[0], xv[1]);
      dw[r / 2] = cvt_pk_bf16(dv[0], dv[1]);
      db1 += bf16_lo(dw[r / 2]) + bf16_hi(dw[r / 2]);
    }
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const uint4 xa = make_uint4(xw[4 * kk], xw[4 * kk + 1], xw[4 * kk + 2], xw[4 * kk + 3]);
      const uint4 da = make_uint4(dw[4 * kk], dw[4 * kk + 1], dw[4 * kk + 2], dw[4 * kk + 3]);
#pragma unroll
      for (int nb = 0; nb < 4; ++nb) acc1[nb] = mfma32(da, lds_kmajor_o(qt, to, 32 * rsub + 16 * kk, nb), acc1[nb]);
#pragma unroll
      for (int ob = 0; ob < 2; ++ob) {
        const uint4 gv = lds_kmajor_o(gt, to, 32 * rsub + 16 * kk, ob);
        acc2[ob] = mfma32(xa, gv, acc2[ob]);
        if (do_db2) {
          const uint32_t w4[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) db2[ob] += bf16_lo(w4[j]) + bf16_hi(w4[j]);
        }
      }
    }
  }
  wait_vm0();       // no copy may still target LDS
  __syncthreads();  // every wavefront is done with the tiles: the sums take their place

  // lanes l and l ^ 32 summed different rows of the same unit / column
  db1 += __shfl_xor(db1, 32, 64);
  db2[0] += __shfl_xor(db2[0], 32, 64);
  db2[1] += __shfl_xor(db2[1], 32, 64);
  MlpWgradSum& S = reinterpret_cast<MlpWgradSum*>(&L)[hl];
  for (int step = 0; step < 2; ++step) {
    if (rsub == step) {
#pragma unroll
      for (int nb = 0; nb < 4; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float& d = S.dw1[(8 * (r / 4) + 4 * gq + r % 4) * kMlpD + 32 * nb + lr];
          d = step == 0 ? acc1[nb][r] : d + acc1[nb][r];
        }
#pragma unroll
      for (int ob = 0; ob < 2; ++ob)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float& d = S.dw2[(8 * (r / 4) + 4 * gq + r % 4) * kMlpOMax + 32 * ob + lr];
          d = step == 0 ? acc2[ob][r] : d + acc2[ob][r];
        }
      if (gq == 0) {
        S.db1[lr] = step == 0 ? db1 : S.db1[lr] + db1;
        S.db2[lr] = step == 0 ? db2[0] : S.db2[lr] + db2[0];
        S.db2[32 + lr] = step == 0 ? db2[1] : S.db2[32 + lr] + db2[1];
      }
    }
    __syncthreads();
  }
  // this workgroup's hidden units 128·hq .. +127 of the row group's partials
  float* p1 = part1 + static_cast<int64_t>(gi) * kMwPart1;
  float* p2 = part2 + static_cast<int64_t>(gi) * kMwPart2;
  const MlpWgradSum* SS = reinterpret_cast<const MlpWgradSum*>(&L);
  for (int e = tid; e < 128 * kMlpD; e += kMlpThreads) {
    const int hh = e / kMlpD;  // 0..127
    p1[(128 * hq + hh) * kMlpD + e % kMlpD] = SS[hh / 32].dw1[(hh % 32) * kMlpD + e % kMlpD];
  }
  for (int e = tid; e < kMlpOMax * 128; e += kMlpThreads) {
    const int o = e / 128, hh = e % 128;
    p2[o * kMlpH + 128 * hq + hh] = SS[hh / 32].dw2[(hh % 32) * kMlpOMax + o];
  }
  if (tid < 128) p1[kMlpH * kMlpD + 128 * hq + tid] = SS[tid / 32].db1[tid % 32];
  if (hq == 0 && tid < kMlpOMax) p2[kMlpOMax * kMlpH + tid] = SS[0].db2[tid];
}

}  // namespace

}  // namespace scope

using namespace scope;

extern "C" int64_t scope_linear_wgrad_workspace_bytes(const scope_wgrad_params* p) {
  if (!p || p->rows <= 0 || p->M <= 0 || p->N <= 0) return 0;
  return static_cast<int64_t>(wgrad_groups(p)) * (static_cast<int64_t>(p->M) * p->N + p->M) * 4;
}

extern "C" int scope_linear_wgrad(const scope_wgrad_params* p, const uint16_t* a, const uint16_t* b, float* dw,
                                  float* db, void* workspace, void* stream) {
  SCOPE_REQUIRE(p && a && b && dw && workspace, "scope_linear_wgrad: null pointer");
  const int M = p->M, N = p->N;
  const bool shape_ok = (M == 64 && (N == 128 || N == 256)) || (M == 128 && (N == 128 || N == 256)) ||
                        (M == 256 && (N == 64 || N == 128));
  SCOPE_REQUIRE(shape_ok, "scope_linear_wgrad: (M, N) = (%d, %d) not supported (64, 128 or 256 with M·N <= 32768)",
                M, N);
  SCOPE_REQUIRE(p->rows > 0 && p->rows % kChunkRows == 0, "scope_linear_wgrad: rows=%lld must be a positive multiple of %d",
                (long long)p->rows, kChunkRows);
  SCOPE_REQUIRE(p->seg > 0 && p->seg % kChunkRows == 0 && p->rows % p->seg == 0,
                "scope_linear_wgrad: seg=%lld must be a multiple of %d dividing rows", (long long)p->seg, kChunkRows);
  SCOPE_REQUIRE(p->a_rs >= M && p->b_rs >= N && p->a_rs % 8 == 0 && p->b_rs % 8 == 0 && p->a_ss % 8 == 0 &&
                    p->b_ss % 8 == 0 && p->a_ss >= 0 && p->b_ss >= 0,
                "scope_linear_wgrad: row strides must cover the row and all strides be multiples of 8 elements");
  // each chunk's lane offsets are 32-bit byte offsets from the chunk's first row
  SCOPE_REQUIRE(p->a_rs < (1 << 24) && p->b_rs < (1 << 24), "scope_linear_wgrad: row strides must be below 2^24");
  SCOPE_REQUIRE(((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                  reinterpret_cast<uintptr_t>(workspace)) & 15) == 0,
                "scope_linear_wgrad: a, b and workspace must start on a 16-byte boundary");
  const int groups = wgrad_groups(p);
  const int64_t chunks = p->rows / kChunkRows;
  WgradArgs g;
  g.a = a;
  g.b = b;
  g.rows = p->rows;
  g.seg = p->seg;
  g.a_ss = p->a_ss;
  g.a_rs = p->a_rs;
  g.b_ss = p->b_ss;
  g.b_rs = p->b_rs;
  g.part = static_cast<float*>(workspace);
  g.chunks_per_group = static_cast<int>((chunks + groups - 1) / groups);
  hipStream_t s = as_stream(stream);
  if (M == 64 && N == 128) launch_wgrad<2, 4>(g, groups, s);
  else if (M == 64) launch_wgrad<2, 8>(g, groups, s);
  else if (M == 128 && N == 128) launch_wgrad<4, 4>(g, groups, s);
  else if (M == 128) launch_wgrad<4, 8>(g, groups, s);
  else if (N == 64) launch_wgrad<8, 2>(g, groups, s);
  else launch_wgrad<8, 4>(g, groups, s);
  const int total = M * N + M;
  hipLaunchKernelGGL(wgrad_reduce_kernel, dim3((total + 63) / 64), dim3(256), 0, s, g.part, groups, M * N, M,
                     p->round_bf16, dw, db);
  return check_launch("linear weight gradient kernels");
}

static int mlp_check(const scope_mlp_params* p, const uint16_t* q, const float* w1, const float* b1, const float* w2,
                     const float* b2, const char* who) {
  SCOPE_REQUIRE(p && q && w1 && b1 && w2 && b2, "%s: null pointer", who);
  SCOPE_REQUIRE(p->D == kMlpD && p->H == kMlpH && p->O >= 1 && p->O <= kMlpOMax,
                "%s: (D, hidden, outputs) = (%d, %d, %d); the kernel takes (128, 256, 1..64)", who, p->D, p->H, p->O);
  SCOPE_REQUIRE(p->rows > 0 && p->rows % 32 == 0, "%s: rows=%lld must be a positive multiple of 32", who,
                (long long)p->rows);
  SCOPE_REQUIRE(p->seg > 0 && p->seg % 32 == 0 && p->rows % p->seg == 0,
                "%s: seg=%lld must be a multiple of 32 dividing rows", who, (long long)p->seg);
  SCOPE_REQUIRE(p->q_rs >= kMlpD && p->q_rs % 8 == 0 && p->q_ss >= 0 && p->q_ss % 8 == 0,
                "%s: q's row stride must cover a row and both strides be multiples of 8 elements", who);
  SCOPE_REQUIRE(((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(w1)) & 15) == 0,
                "%s: q and w1 must start on a 16-byte boundary", who);
  return 0;
}

static MlpArgs mlp_args(const scope_mlp_params* p, const uint16_t* q, const float* w1, const float* b1,
                        const float* w2, const float* b2) {
  MlpArgs g = {};
  g.q = q;
  g.rows = p->rows;
  g.seg = p->seg;
  g.q_ss = p->q_ss;
  g.q_rs = p->q_rs;
  g.w1 = w1;
  g.b1 = b1;
  g.w2 = w2;
  g.b2 = b2;
  g.O = p->O;
  return g;
}

static int mlp_grid(int64_t rows) {
  // one workgroup per CU (129 KB of LDS each), walking the 256-row tiles
  const int64_t tiles = (rows + kMlpTileRows - 1) / kMlpTileRows;
  return static_cast<int>(std::min<int64_t>(tiles, 256));
}

extern "C" int scope_coeff_mlp_fwd(const scope_mlp_params* p, const uint16_t* q, const float* w1, const float* b1,
                                   const float* w2, const float* b2, uint16_t* y, void* stream) {
  if (int rc = mlp_check(p, q, w1, b1, w2, b2, "scope_coeff_mlp_fwd")) return rc;
  SCOPE_REQUIRE(y != nullptr, "scope_coeff_mlp_fwd: null output");
  MlpArgs g = mlp_args(p, q, w1, b1, w2, b2);
  g.y = y;
  hipLaunchKernelGGL(mlp_fwd_kernel, dim3(mlp_grid(p->rows)), dim3(kMlpThreads), 0, as_stream(stream), g);
  return check_launch("MLP forward kernel");
}

extern "C" int scope_coeff_mlp_bwd(const scope_mlp_params* p, const uint16_t* q, const uint16_t* gy, const float* w1,
                                   const float* b1, const float* w2, const float* b2, uint16_t* dq, uint16_t* dz1,
                                   uint16_t* x1, uint16_t* gyp, void* stream) {
  if (int rc = mlp_check(p, q, w1, b1, w2, b2, "scope_coeff_mlp_bwd")) return rc;
  SCOPE_REQUIRE(gy && dq && gyp, "scope_coeff_mlp_bwd: null pointer");
  SCOPE_REQUIRE((dz1 == nullptr) == (x1 == nullptr), "scope_coeff_mlp_bwd: dz1 and x1 are given together or not at all");
  SCOPE_REQUIRE(((reinterpret_cast<uintptr_t>(dq) | reinterpret_cast<uintptr_t>(dz1) | reinterpret_cast<uintptr_t>(x1) |
                  reinterpret_cast<uintptr_t>(gyp)) & 15) == 0,
                "scope_coeff_mlp_bwd: dq, dz1, x1 and gyp must start on a 16-byte boundary");
  MlpArgs g = mlp_args(p, q, w1, b1, w2, b2);
  g.gy = gy;
  g.dq = dq;
  g.dz1 = dz1;
  g.x1 = x1;
  g.gyp = gyp;
  hipLaunchKernelGGL(mlp_bwd_kernel, dim3(mlp_grid(p->rows)), dim3(kMlpThreads), 0, as_stream(stream), g);
  return check_launch("MLP backward kernel");
}

static int mlp_wgrad_groups(int64_t rows) {
  const int64_t tiles = rows / kMwTileRows;
  if (tiles < 8) return static_cast<int>(tiles);
  const int64_t g = tiles < kMwMaxGroups ? tiles - tiles % 8 : kMwMaxGroups;
  return static_cast<int>(g);
}

extern "C" int64_t scope_coeff_mlp_wgrad_workspace_bytes(const scope_mlp_params* p) {
  if (!p || p->rows <= 0) return 0;
  return static_cast<int64_t>(mlp_wgrad_groups(p->rows)) * (kMwPart1 + kMwPart2) * 4;
}

extern "C" int scope_coeff_mlp_wgrad(const scope_mlp_params* p, const uint16_t* q, const uint16_t* gyp,
                                     const float* w1, const float* b1, const float* w2, float* dw1, float* db1,
                                     float* dw2, float* db2, void* workspace, void* stream) {
  // b2 takes no part in the gradients: b1 stands in for it in the shared checks
  if (int rc = mlp_check(p, q, w1, b1, w2, b1, "scope_coeff_mlp_wgrad")) return rc;
  SCOPE_REQUIRE(gyp && dw1 && db1 && dw2 && db2 && workspace, "scope_coeff_mlp_wgrad: null pointer");
  SCOPE_REQUIRE(p->seg % 128 == 0, "scope_coeff_mlp_wgrad: seg=%lld must be a multiple of 128", (long long)p->seg);
  SCOPE_REQUIRE(((reinterpret_cast<uintptr_t>(gyp) | reinterpret_cast<uintptr_t>(workspace)) & 15) == 0,
                "scope_coeff_mlp_wgrad: gyp and workspace must start on a 16-byte boundary");
  SCOPE_REQUIRE(p->q_rs < (1 << 24), "scope_coeff_mlp_wgrad: q's row stride must be below 2^24");
  MlpArgs g = mlp_args(p, q, w1, b1, w2, b1);
  g.gyp = const_cast<uint16_t*>(gyp);
  const int groups = mlp_wgrad_groups(p->rows);
  const int64_t tiles = p->rows / kMwTileRows;
  const int tpg = static_cast<int>((tiles + groups - 1) / groups);
  float* part1 = static_cast<float*>(workspace);
  float* part2 = part1 + static_cast<int64_t>(groups) * kMwPart1;
  hipStream_t s = as_stream(stream);
  hipLaunchKernelGGL(mlp_wgrad_kernel, dim3(2 * groups), dim3(kMlpThreads), 0, s, g, part1, part2, groups, tpg);
  const int nb1 = (kMwPart1 + 63) / 64, nb2 = (kMwPart2 + 63) / 64;
  hipLaunchKernelGGL(mlp_wgrad_reduce_kernel, dim3(nb1 + nb2), dim3(256), 0, s, part1, part2, groups, nb1, dw1, db1,
                     dw2, db2);
  return check_launch("MLP weight gradient kernels");
}
