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
  if (g.n >= 128 && tiles(64, 128) >= 512) return launch_cfg<1, 2>(g, s);
  return launch_cfg<1, 1>(g, s);
}

}  // namespace qph
