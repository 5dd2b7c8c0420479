// fp32 MFMA GEMM with fused epilogues: the pointwise (1x1) conv, the rec
// linears (MatMul + Add(bias) [+ GELU] [+ residual]) and the rec head.
//
// C[b][i][j] = sum_k A[b][i][k] * B[b][k][j], A and B row-major.  Each
// output element is one fma chain over k in ascending order starting from 0
// (or from the bias where the reference seeds it), exactly as the reference
// panel kernels compute it (qppocr-kernels/src/gemm.rs:523-596,
// x86.rs:134-444): v_mfma_f32_32x32x2f32 adds its two k terms in order with
// one rounding each, so the MFMA k-loop is that chain.
//
// Tiling: a 256-thread workgroup (2x2 waves) owns a (64*MI) x (64*NI) tile;
// each wave holds MI x NI 32x32 accumulators (16 floats per lane each).
// K advances in slabs of 16 staged through LDS (A transposed to [k][m] so a
// wave's 32 rows at one k are 32 consecutive words), with the next slab's
// global loads issued before the current slab's MFMAs.
#include "qph_internal.h"

namespace qph {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define GEMM_BK 16

// Reference bias placement (gemm.rs:7-16): rule 0 (panel kernel): seeded
// when row is in the M%4 tail and the 32-column panel is partial; rule 1
// (m-rows kernel): seeded for columns j >= n - n%32.
__device__ __forceinline__ bool bias_seeded(int rule, int64_t i, int64_t j, int64_t m, int64_t n) {
  if (rule == 1) return j >= n - n % 32;
  int64_t n0 = (j >> 5) << 5;
  return (n - n0) < 32 && i >= m - m % 4;
}

// Epilogue in two phases: every operand the outputs need (bias, residual)
// is loaded first, then the values are finished and stored.  The stores to C
// may alias those operands as far as the compiler knows, so interleaving
// them would serialise one load round trip per output.
struct EpiIn {
  float add;   // bias term (added when has_add)
  float res;   // residual term
  bool has_add, ok;
};

__device__ __forceinline__ EpiIn epilogue_gather(const GemmArgs& g, const float* R, int64_t i,
                                                 int64_t j) {
  EpiIn e{0.0f, 0.0f, false, i < g.m && j < g.n};
  if (!e.ok) return e;
  if (g.bias_mode == 1) {
    if (!bias_seeded(g.seed_rule, i, j, g.m, g.n)) {
      e.add = g.bias[i];
      e.has_add = true;
    }
  } else if (g.bias_mode == 2) {
    e.add = g.bias[j];
    e.has_add = true;
  }
  if (R) {
    if (g.res_up == 2) {
      int64_t oy = j / g.up_w, ox = j - oy * g.up_w;
      e.res = R[i * g.ldr + (oy >> 1) * g.up_cw + (ox >> 1)];
    } else {
      e.res = R[i * g.ldr + j];
    }
  }
  return e;
}

__device__ __forceinline__ void epilogue_put(const GemmArgs& g, float* C, bool has_res,
                                             const EpiIn& e, int64_t i, int64_t j, float x) {
  if (!e.ok) return;
  if (e.has_add) x = x + e.add;
  x = act_apply(x, g.act);
  if (has_res) x = x + e.res;
  if (g.trans_out)
    C[j * g.ldc + i] = x;
  else
    C[i * g.ldc + j] = x;
}

template <int MI, int NI>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(GemmArgs g) {
  constexpr int BM = 64 * MI, BN = 64 * NI;
  constexpr int PA = BM + 4, PB = BN + 4;  // padded LDS rows
  __shared__ float sA[2][GEMM_BK * PA];
  __shared__ float sB[2][GEMM_BK * PB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave & 1) * (BM / 2);
  const int wn0 = (wave >> 1) * (BN / 2);
  const int64_t bz = blockIdx.z;
  const int64_t i0 = (int64_t)blockIdx.y * BM;
  const int64_t j0 = (int64_t)blockIdx.x * BN;
  const float* A = g.a + bz * g.a_batch;
  const float* B = g.b + bz * g.b_batch;
  const int64_t M = g.m, N = g.n, K = g.k;

  // global -> register staging.  A: thread t covers k = t % 16, rows
  // t / 16 + 16 r (BM / 16 rows).  B: thread t covers column t % BN',
  // k rows (t / BN') + step.
  constexpr int A_PER = BM * GEMM_BK / 256;
  constexpr int B_PER = BN * GEMM_BK / 256;
  float ra[A_PER], rb[B_PER];
  const int ak = tid & 15;
  const int arow = tid >> 4;
  constexpr int BCOLS = BN < 256 ? BN : 256;
  const int bcol = tid % BCOLS;
  const int bk0 = tid / BCOLS;
  constexpr int BKSTEP = 256 / BCOLS;

  auto load_tile = [&](int64_t k0) {
#pragma unroll
    for (int r = 0; r < A_PER; r++) {
      int64_t i = i0 + arow + 16 * r;
      int64_t k = k0 + ak;
      ra[r] = (i < M && k < K) ? A[i * g.lda + k] : 0.0f;
    }
#pragma unroll
    for (int r = 0; r < B_PER; r++) {
      int kr = bk0 + BKSTEP * (r / (BN / BCOLS));
      int cc = bcol + BCOLS * (r % (BN / BCOLS));
      int64_t k = k0 + kr;
      int64_t j = j0 + cc;
      rb[r] = (k < K && j < N) ? B[k * g.ldb + j] : 0.0f;
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int r = 0; r < A_PER; r++) sA[buf][ak * PA + arow + 16 * r] = ra[r];
#pragma unroll
    for (int r = 0; r < B_PER; r++) {
      int kr = bk0 + BKSTEP * (r / (BN / BCOLS));
      int cc = bcol + BCOLS * (r % (BN / BCOLS));
      sB[buf][kr * PB + cc] = rb[r];
    }
  };

  // accumulators, seeded with the bias where the reference seeds it
  f32x16 acc[MI][NI];
  const int lr = lane & 31;
  const int lh = lane >> 5;
#pragma unroll
  for (int mi = 0; mi < MI; mi++)
#pragma unroll
    for (int ni = 0; ni < NI; ni++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        float s = 0.0f;
        if (g.bias_mode == 1) {
          int64_t i = i0 + wm0 + mi * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
          int64_t j = j0 + wn0 + ni * 32 + lr;
          if (i < M && j < N && bias_seeded(g.seed_rule, i, j, M, N)) s = g.bias[i];
        }
        acc[mi][ni][v] = s;
      }

  const int64_t nk = (K + GEMM_BK - 1) / GEMM_BK;
  load_tile(0);
  store_tile(0);
  __syncthreads();
  for (int64_t t = 0; t < nk; t++) {
    const int buf = (int)(t & 1);
    if (t + 1 < nk) load_tile((t + 1) * GEMM_BK);
    const float* a_s = sA[buf];
    const float* b_s = sB[buf];
#pragma unroll
    for (int kk = 0; kk < GEMM_BK; kk += 2) {
      const int kr = kk + lh;
      float av[MI], bv[NI];
#pragma unroll
      for (int mi = 0; mi < MI; mi++) av[mi] = a_s[kr * PA + wm0 + mi * 32 + lr];
#pragma unroll
      for (int ni = 0; ni < NI; ni++) bv[ni] = b_s[kr * PB + wn0 + ni * 32 + lr];
#pragma unroll
      for (int mi = 0; mi < MI; mi++)
#pragma unroll
        for (int ni = 0; ni < NI; ni++)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[mi], bv[ni], acc[mi][ni], 0, 0, 0);
    }
    if (t + 1 < nk) {
      store_tile(buf ^ 1);
    }
    __syncthreads();
  }

  // epilogue: bias (after the chain), act, residual, store
  float* C = g.c + bz * g.c_batch;
  const float* R = g.res ? g.res + bz * g.r_batch : nullptr;
#pragma unroll
  for (int mi = 0; mi < MI; mi++)
#pragma unroll
    for (int ni = 0; ni < NI; ni++) {
      EpiIn e[16];
#pragma unroll
      for (int v = 0; v < 16; v++)
        e[v] = epilogue_gather(g, R, i0 + wm0 + mi * 32 + 8 * (v >> 2) + 4 * lh + (v & 3),
                               j0 + wn0 + ni * 32 + lr);
#pragma unroll
      for (int v = 0; v < 16; v++)
        epilogue_put(g, C, R != nullptr, e[v], i0 + wm0 + mi * 32 + 8 * (v >> 2) + 4 * lh + (v & 3),
                     j0 + wn0 + ni * 32 + lr, acc[mi][ni][v]);
    }
}

// ------------------------------------------------------------ skinny tiles
//
// For GEMMs whose 128x128 tiling leaves most of the chip idle (the rec
// linears, 1280 x {256..1024} x {256, 1024}; the pointwise convs): a
// workgroup owns 32x32 outputs, each wave one 16x16 block accumulated with
// v_mfma_f32_16x16x4f32 (4 k per instruction in order), so a K-deep chain
// takes K/4 dependent MFMAs and the grid has M*N/256 waves.  K advances in
// slabs of 64 through double-buffered LDS; A is staged row-major (stride
// 66: a 16-row x 2-k read hits 32 distinct banks), B row-major (stride 48).

#define SK_BK 64
#define SK_PA (SK_BK + 2)
#define SK_PB 48

template <bool VEC>
__global__ __launch_bounds__(256) void gemm_skinny_kernel(GemmArgs g) {
  __shared__ float sA[2][32 * SK_PA];
  __shared__ float sB[2][SK_BK * SK_PB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lg = lane >> 4, l16 = lane & 15;
  const int wm = wave & 1, wn = wave >> 1;
  const int64_t bz = blockIdx.z;
  const int64_t i0 = (int64_t)blockIdx.y * 32;
  const int64_t j0 = (int64_t)blockIdx.x * 32;
  const float* A = g.a + bz * g.a_batch;
  const float* B = g.b + bz * g.b_batch;
  const int64_t M = g.m, N = g.n, K = g.k;

  // staging: A slab 32 rows x 64 k (thread: row tid/8, k 8*(tid%8) .. +8),
  // B slab 64 k x 32 cols (thread: k row tid/4, cols 8*(tid%4) .. +8)
  const int ar = tid >> 3, ak = (tid & 7) * 8;
  const int br = tid >> 2, bc = (tid & 3) * 8;
  float ra[8], rb[8];
  auto load = [&](int64_t k0) {
    const int64_t ia = i0 + ar, ka = k0 + ak;
    const int64_t kb = k0 + br, jb = j0 + bc;
    if (VEC && ia < M && ka + 8 <= K) {
      const float4* pa = (const float4*)(A + ia * g.lda + ka);
      float4 v0 = pa[0], v1 = pa[1];
      ra[0] = v0.x; ra[1] = v0.y; ra[2] = v0.z; ra[3] = v0.w;
      ra[4] = v1.x; ra[5] = v1.y; ra[6] = v1.z; ra[7] = v1.w;
    } else {
#pragma unroll
      for (int u = 0; u < 8; u++) ra[u] = (ia < M && ka + u < K) ? A[ia * g.lda + ka + u] : 0.0f;
    }
    if (VEC && kb < K && jb + 8 <= N) {
      const float4* pb = (const float4*)(B + kb * g.ldb + jb);
      float4 v0 = pb[0], v1 = pb[1];
      rb[0] = v0.x; rb[1] = v0.y; rb[2] = v0.z; rb[3] = v0.w;
      rb[4] = v1.x; rb[5] = v1.y; rb[6] = v1.z; rb[7] = v1.w;
    } else {
#pragma unroll
      for (int u = 0; u < 8; u++) rb[u] = (kb < K && jb + u < N) ? B[kb * g.ldb + jb + u] : 0.0f;
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int u = 0; u < 8; u++) sA[buf][ar * SK_PA + ak + u] = ra[u];
#pragma unroll
    for (int u = 0; u < 8; u++) sB[buf][br * SK_PB + bc + u] = rb[u];
  };

  const int64_t ii = i0 + wm * 16;     // this wave's 16x16 block
  const int64_t jj = j0 + wn * 16;
  f32x4 acc;
#pragma unroll
  for (int v = 0; v < 4; v++) {
    float s0 = 0.0f;
    if (g.bias_mode == 1) {
      int64_t i = ii + 4 * lg + v, j = jj + l16;
      if (i < M && j < N && bias_seeded(g.seed_rule, i, j, M, N)) s0 = g.bias[i];
    }
    acc[v] = s0;
  }

  const int64_t nk = (K + SK_BK - 1) / SK_BK;
  load(0);
  store(0);
  __syncthreads();
  for (int64_t t = 0; t < nk; t++) {
    const int buf = (int)(t & 1);
    if (t + 1 < nk) load((t + 1) * SK_BK);
    const float* a_s = sA[buf] + (wm * 16 + l16) * SK_PA + lg;
    const float* b_s = sB[buf] + lg * SK_PB + wn * 16 + l16;
#pragma unroll
    for (int kk = 0; kk < SK_BK; kk += 4)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a_s[kk], b_s[kk * SK_PB], acc, 0, 0, 0);
    if (t + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }

  float* C = g.c + bz * g.c_batch;
  const float* R = g.res ? g.res + bz * g.r_batch : nullptr;
  EpiIn e[4];
#pragma unroll
  for (int v = 0; v < 4; v++) e[v] = epilogue_gather(g, R, ii + 4 * lg + v, jj + l16);
#pragma unroll
  for (int v = 0; v < 4; v++) epilogue_put(g, C, R != nullptr, e[v], ii + 4 * lg + v, jj + l16, acc[v]);
}

static int launch_skinny(const GemmArgs& g, hipStream_t s) {
  dim3 grid(ceil_div(g.n, 32), ceil_div(g.m, 32), (unsigned)g.batch);
  const bool vec = (g.lda % 4 == 0) && (g.ldb % 4 == 0) && (g.a_batch % 4 == 0) &&
                   (g.b_batch % 4 == 0) && ((uintptr_t)g.a % 16 == 0) &&
                   ((uintptr_t)g.b % 16 == 0);
  if (vec)
    hipLaunchKernelGGL(gemm_skinny_kernel<true>, grid, dim3(256), 0, s, g);
  else
    hipLaunchKernelGGL(gemm_skinny_kernel<false>, grid, dim3(256), 0, s, g);
  return launch_check("gemm_skinny_kernel");
}

template <int MI, int NI>
static int launch_cfg(const GemmArgs& g, hipStream_t s) {
  constexpr int BM = 64 * MI, BN = 64 * NI;
  dim3 grid(ceil_div(g.n, BN), ceil_div(g.m, BM), (unsigned)g.batch);
  hipLaunchKernelGGL((gemm_mfma_kernel<MI, NI>), grid, dim3(256), 0, s, g);
  return launch_check("gemm_mfma_kernel");
}

// ------------------------------------------------------------- wide tiles
//
// The large GEMMs (the rec head, 1280 x 18709 x 256): 128x128 tiles, 4 waves
// of 64x64 (2x2 v_mfma_f32_32x32x2f32 accumulators each), K slabs of 32
// through double-buffered LDS with 16-byte global loads (needs lda, ldb
// multiples of 4 and 16-byte aligned bases: the session pads the head
// weight rows).  Tile order is XCD-aware: workgroup b runs on XCD b % 8
// (round-robin dispatch), and each XCD gets a contiguous range of tiles in
// column-block-major order, so one B column block stays in that XCD's L2
// while all row blocks pass over it, and A (small) is read once per XCD.

#define WB_BK 32
#define WB_PA (128 + 1)
#define WB_PB (128 + 4)
#define NUM_XCD 8

__global__ __launch_bounds__(256) void gemm_wide_kernel(GemmArgs g, int mb, int nb,
                                                        int tiles_per_xcd) {
  __shared__ float sA[2][WB_BK * WB_PA];
  __shared__ __attribute__((aligned(16))) float sB[2][WB_BK * WB_PB];
  const int b = blockIdx.x;
  const int tile = (b % NUM_XCD) * tiles_per_xcd + b / NUM_XCD;
  if (tile >= mb * nb) return;
  const int nblk = tile / mb, mblk = tile - nblk * mb;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave & 1) * 64, wn0 = (wave >> 1) * 64;
  const int64_t i0 = (int64_t)mblk * 128, j0 = (int64_t)nblk * 128;
  const int64_t bz = blockIdx.z;
  const float* A = g.a + bz * g.a_batch;
  const float* B = g.b + bz * g.b_batch;
  const int64_t M = g.m, N = g.n, K = g.k;

  // A slab 128 x 32: thread -> rows t/8 + 32 r, k 4*(t%8); B slab 32 x 128:
  // thread -> k rows t/32 + 8 r, columns 4*(t%32)
  const int ar = tid >> 3, ak = (tid & 7) * 4;
  const int br = tid >> 5, bc = (tid & 31) * 4;
  float4 ra[4], rb[4];
  auto load = [&](int64_t k0) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int64_t i = i0 + ar + 32 * r, k = k0 + ak;
      if (i < M && k + 4 <= K) {
        ra[r] = *(const float4*)(A + i * g.lda + k);
      } else {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = (i < M && k + u < K) ? A[i * g.lda + k + u] : 0.0f;
        ra[r] = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int64_t k = k0 + br + 8 * r, j = j0 + bc;
      if (k < K && j + 4 <= N) {
        rb[r] = *(const float4*)(B + k * g.ldb + j);
      } else {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = (k < K && j + u < N) ? B[k * g.ldb + j + u] : 0.0f;
        rb[r] = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
  };
  auto store = [&](int buf) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      float* d = sA[buf] + ak * WB_PA + ar + 32 * r;   // transposed: [k][m]
      d[0] = ra[r].x;
      d[WB_PA] = ra[r].y;
      d[2 * WB_PA] = ra[r].z;
      d[3 * WB_PA] = ra[r].w;
    }
#pragma unroll
    for (int r = 0; r < 4; r++) *(float4*)(sB[buf] + (br + 8 * r) * WB_PB + bc) = rb[r];
  };

  const int lr = lane & 31, lh = lane >> 5;
  f32x16 acc[2][2];
#pragma unroll
  for (int mi = 0; mi < 2; mi++)
#pragma unroll
    for (int ni = 0; ni < 2; ni++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        float s0 = 0.0f;
        if (g.bias_mode == 1) {
          int64_t i = i0 + wm0 + mi * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
          int64_t j = j0 + wn0 + ni * 32 + lr;
          if (i < M && j < N && bias_seeded(g.seed_rule, i, j, M, N)) s0 = g.bias[i];
        }
        acc[mi][ni][v] = s0;
      }

  const int64_t nk = (K + WB_BK - 1) / WB_BK;
  load(0);
  store(0);
  __syncthreads();
  for (int64_t t = 0; t < nk; t++) {
    const int buf = (int)(t & 1);
    if (t + 1 < nk) load((t + 1) * WB_BK);
    const float* a_s = sA[buf] + lh * WB_PA + wm0 + lr;
    const float* b_s = sB[buf] + lh * WB_PB + wn0 + lr;
    // operands of k-step kk+2 are read before the MFMAs of k-step kk issue
    float op[2][4];
    op[0][0] = a_s[0];
    op[0][1] = a_s[32];
    op[0][2] = b_s[0];
    op[0][3] = b_s[32];
#pragma unroll
    for (int kk = 0; kk < WB_BK; kk += 2) {
      const int cur = (kk >> 1) & 1, nxt = cur ^ 1;
      if (kk + 2 < WB_BK) {
        op[nxt][0] = a_s[(kk + 2) * WB_PA];
        op[nxt][1] = a_s[(kk + 2) * WB_PA + 32];
        op[nxt][2] = b_s[(kk + 2) * WB_PB];
        op[nxt][3] = b_s[(kk + 2) * WB_PB + 32];
      }
      acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(op[cur][0], op[cur][2], acc[0][0], 0, 0, 0);
      acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(op[cur][0], op[cur][3], acc[0][1], 0, 0, 0);
      acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(op[cur][1], op[cur][2], acc[1][0], 0, 0, 0);
      acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(op[cur][1], op[cur][3], acc[1][1], 0, 0, 0);
    }
    if (t + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }

  float* C = g.c + bz * g.c_batch;
  const float* R = g.res ? g.res + bz * g.r_batch : nullptr;
#pragma unroll
  for (int mi = 0; mi < 2; mi++)
#pragma unroll
    for (int ni = 0; ni < 2; ni++) {
      EpiIn e[16];
#pragma unroll
      for (int v = 0; v < 16; v++)
        e[v] = epilogue_gather(g, R, i0 + wm0 + mi * 32 + 8 * (v >> 2) + 4 * lh + (v & 3),
                               j0 + wn0 + ni * 32 + lr);
#pragma unroll
      for (int v = 0; v < 16; v++)
        epilogue_put(g, C, R != nullptr, e[v], i0 + wm0 + mi * 32 + 8 * (v >> 2) + 4 * lh + (v & 3),
                     j0 + wn0 + ni * 32 + lr, acc[mi][ni][v]);
    }
}

static int launch_wide(const GemmArgs& g, hipStream_t s) {
  const int mb = (int)ceil_div(g.m, 128), nb = (int)ceil_div(g.n, 128);
  const int tiles = mb * nb;
  const int per = (tiles + NUM_XCD - 1) / NUM_XCD;
  dim3 grid((unsigned)(per * NUM_XCD), 1, (unsigned)g.batch);
  hipLaunchKernelGGL(gemm_wide_kernel, grid, dim3(256), 0, s, g, mb, nb, per);
  return launch_check("gemm_wide_kernel");
}

int launch_gemm(const GemmArgs& g, hipStream_t s) {
  if (g.m <= 0 || g.n <= 0 || g.k <= 0 || g.batch <= 0) return QPH_OK;
  if (g.m > (1ll << 31) || g.n > (1ll << 31) || g.batch > 65535)
    return fail(QPH_EUNSUPPORTED, "gemm: dimension too large");
  // Tile choice: the largest tile that still yields about two workgroups
  // per CU (256 CUs) for the whole launch.
  auto tiles = [&](int bm, int bn) {
    return (double)ceil_div(g.m, bm) * (double)ceil_div(g.n, bn) * (double)g.batch;
  };
  if (g.m >= 128 && g.n >= 128 && tiles(128, 128) >= 512) {
    const bool vec = (g.lda % 4 == 0) && (g.ldb % 4 == 0) && (g.a_batch % 4 == 0) &&
                     (g.b_batch % 4 == 0) && ((uintptr_t)g.a % 16 == 0) &&
                     ((uintptr_t)g.b % 16 == 0);
    if (vec && tiles(128, 128) < (1u << 30)) return launch_wide(g, s);
    return launch_cfg<2, 2>(g, s);
  }
  return launch_skinny(g, s);
}

}  // namespace qph
