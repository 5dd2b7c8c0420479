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
    for (int ni = 0; ni < NI; ni++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        int64_t i = i0 + wm0 + mi * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
        int64_t j = j0 + wn0 + ni * 32 + lr;
        if (i >= M || j >= N) continue;
        float x = acc[mi][ni][v];
        if (g.bias_mode == 1) {
          if (!bias_seeded(g.seed_rule, i, j, M, N)) x = x + g.bias[i];
        } else if (g.bias_mode == 2) {
          x = x + g.bias[j];
        }
        x = act_apply(x, g.act);
        if (R) {
          float r;
          if (g.res_up == 2) {
            // nearest 2x upsample of a coarse map: row stride ldr (channel
            // plane), coarse width up_cw, output width up_w.
            int64_t oy = j / g.up_w, ox = j - oy * g.up_w;
            r = R[i * g.ldr + (oy >> 1) * g.up_cw + (ox >> 1)];
          } else {
            r = R[i * g.ldr + j];
          }
          x = x + r;
        }
        if (g.trans_out)
          C[j * g.ldc + i] = x;
        else
          C[i * g.ldc + j] = x;
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

__device__ __forceinline__ void epilogue_store(const GemmArgs& g, float* C, const float* R,
                                               int64_t i, int64_t j, float x) {
  const int64_t M = g.m, N = g.n;
  if (g.bias_mode == 1) {
    if (!bias_seeded(g.seed_rule, i, j, M, N)) x = x + g.bias[i];
  } else if (g.bias_mode == 2) {
    x = x + g.bias[j];
  }
  x = act_apply(x, g.act);
  if (R) {
    float r;
    if (g.res_up == 2) {
      int64_t oy = j / g.up_w, ox = j - oy * g.up_w;
      r = R[i * g.ldr + (oy >> 1) * g.up_cw + (ox >> 1)];
    } else {
      r = R[i * g.ldr + j];
    }
    x = x + r;
  }
  if (g.trans_out)
    C[j * g.ldc + i] = x;
  else
    C[i * g.ldc + j] = x;
}

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
#pragma unroll
  for (int v = 0; v < 4; v++) {
    int64_t i = ii + 4 * lg + v, j = jj + l16;
    if (i < M && j < N) epilogue_store(g, C, R, i, j, acc[v]);
  }
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

int launch_gemm(const GemmArgs& g, hipStream_t s) {
  if (g.m <= 0 || g.n <= 0 || g.k <= 0 || g.batch <= 0) return QPH_OK;
  if (g.m > (1ll << 31) || g.n > (1ll << 31) || g.batch > 65535)
    return fail(QPH_EUNSUPPORTED, "gemm: dimension too large");
  // Tile choice: the largest tile that still yields about two workgroups
  // per CU (256 CUs) for the whole launch.
  auto tiles = [&](int bm, int bn) {
    return (double)ceil_div(g.m, bm) * (double)ceil_div(g.n, bn) * (double)g.batch;
  };
  if (g.m >= 128 && g.n >= 128 && tiles(128, 128) >= 512) return launch_cfg<2, 2>(g, s);
  return launch_skinny(g, s);
}

}  // namespace qph
