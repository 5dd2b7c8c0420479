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
#include <type_traits>

#include "qph_internal.h"

namespace qph {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int v4u32_t __attribute__((ext_vector_type(4)));

#define GEMM_BK 16

// Epilogue in two phases: every operand the outputs need (bias, residual)
// is loaded first, then the values are finished and stored.  The stores to C
// may alias those operands as far as the compiler knows, so interleaving
// them would serialise one load round trip per output.
struct EpiIn {
  float add;   // bias term (added when has_add)
  float res;   // residual term
  bool has_add, ok;
};

// Residual column of output column j: j itself, or for the upsample-add
// (res_up == 2) the coarse-map offset of pixel j (nearest 2x).  Column
// indices of an upsampled map fit 32 bits (checked by the launcher's
// caller), so the division is a 32-bit one; computed once per column.
__device__ __forceinline__ int64_t res_col(const GemmArgs& g, int64_t j) {
  if (g.res_up != 2) return j;
  const unsigned ju = (unsigned)j, w = (unsigned)g.up_w;
  const unsigned oy = ju / w, ox = ju - oy * w;
  return (int64_t)(oy >> 1) * g.up_cw + (ox >> 1);
}

__device__ __forceinline__ EpiIn epilogue_gather(const GemmArgs& g, const float* R, int64_t i,
                                                 int64_t j, int64_t rcol) {
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
  if (R) e.res = R[i * g.ldr + rcol];
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
      const int64_t rc = R ? res_col(g, j0 + wn0 + ni * 32 + lr) : 0;
#pragma unroll
      for (int v = 0; v < 16; v++)
        e[v] = epilogue_gather(g, R, i0 + wm0 + mi * 32 + 8 * (v >> 2) + 4 * lh + (v & 3),
                               j0 + wn0 + ni * 32 + lr, rc);
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
// slabs of 64 through double-buffered LDS.  A is staged k-deinterleaved,
// [m][g][s] with k = 4s + g (row pitch 68), so a lane's 16 k-steps of a
// slab are four ds_read_b128; B row-major (stride 48).  All of a slab's
// operand reads are issued before its 16 MFMAs.

#define SK_BK 64
#define SK_PA 68
#define SK_PB 48

template <bool VEC>
__global__ __launch_bounds__(256) void gemm_skinny_kernel(GemmArgs g) {
  __shared__ __attribute__((aligned(16))) float sA[2][32 * SK_PA];
  __shared__ float sB[2][SK_BK * SK_PB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lg = lane >> 4, l16 = lane & 15;
  const int wm = wave & 1, wn = wave >> 1;
  const int64_t bz = blockIdx.z;
  if (g.rn && *g.rn != 0 && bz >= (int64_t)*g.rn * g.rn_per) return;   // past the real batch
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
    for (int u = 0; u < 8; u++) {
      const int k = ak + u;
      sA[buf][ar * SK_PA + (k & 3) * 16 + (k >> 2)] = ra[u];
    }
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

  // epilogue operands (bias, residual) fetched now, their latency under the
  // k-loop's
  float* C = g.c + bz * g.c_batch;
  const float* R = g.res ? g.res + bz * g.r_batch : nullptr;
  EpiIn e[4];
  const int64_t rc = R ? res_col(g, jj + l16) : 0;
#pragma unroll
  for (int v = 0; v < 4; v++) e[v] = epilogue_gather(g, R, ii + 4 * lg + v, jj + l16, rc);

  const int64_t nk = (K + SK_BK - 1) / SK_BK;
  load(0);
  store(0);
  __syncthreads();
  for (int64_t t = 0; t < nk; t++) {
    const int buf = (int)(t & 1);
    if (t + 1 < nk) load((t + 1) * SK_BK);
    const float* a_s = sA[buf] + (wm * 16 + l16) * SK_PA + lg * 16;
    const float* b_s = sB[buf] + lg * SK_PB + wn * 16 + l16;
    f32x4 av[4];
    float bv[16];
#pragma unroll
    for (int q = 0; q < 4; q++) av[q] = *(const f32x4*)(a_s + 4 * q);
#pragma unroll
    for (int st = 0; st < 16; st++) bv[st] = b_s[4 * st * SK_PB];
    // only the k-steps that hold real k (the chain takes no padding terms
    // while K is a multiple of 4)
    const int64_t steps = min((int64_t)16, (K - t * SK_BK + 3) / 4);
#pragma unroll
    for (int st = 0; st < 16; st++)
      if (st < steps)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[st >> 2][st & 3], bv[st], acc, 0, 0, 0);
    if (t + 1 < nk) store(buf ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int v = 0; v < 4; v++) epilogue_put(g, C, R != nullptr, e[v], ii + 4 * lg + v, jj + l16, acc[v]);
}

// ------------------------------------------------------- pointwise tiles
//
// 1x1 convs with few output channels over many pixels (the det FPN
// laterals, M = 96, K = 32..256, N = 400..25600): C[M][N] = W[M][K] X[K][N],
// then bias, act and residual (or the nearest-2x upsampled coarse map) as in
// epilogue_gather / epilogue_put.  A workgroup is one wave owning 16 columns
// and MBW 16-row blocks, each a v_mfma_f32_16x16x4f32 chain over k in order
// (from 0, or from the bias where the reference seeds it).  K advances in
// slabs of 16 through an NST-stage LDS ring filled by 16-byte buffer->LDS
// loads: one for the X slab (16 rows x 16 columns) and MBW for the W slab
// (16 k of each row, its four 16-byte chunks rotated by row % 4 so that the
// A reads of one step spread over the banks).  The wave waits only on its own
// loads: no workgroup barrier.  Bias and residual terms are loaded before
// the first slab, so the slab waits, which count loads in issue order, never
// wait for them.  The loads are inline asm, so the compiler adds no waits
// of its own for the stages.
template <int MBW, int NST>
__device__ __forceinline__ void pw_tile(const GemmArgs& g, int mgroups, int blk, int64_t bt,
                                        float* pw_lds) {
  constexpr int STAGE = 256 * (1 + MBW);   // floats: X slab, then W slab
  constexpr int PER = 1 + MBW;             // loads per slab
  if (g.rn && *g.rn != 0 && bt >= (int64_t)*g.rn * g.rn_per) return;   // past the real batch
  const int lane = threadIdx.x;
  const int l16 = lane & 15, lg = lane >> 4;
  const int mg = blk % mgroups, pg = blk / mgroups;
  const int64_t n0 = (int64_t)pg * 16, m0 = (int64_t)mg * (16 * MBW);
  const int64_t M = g.m, N = g.n;
  const unsigned OOB = 0x80000000u;
  const float* Ab = g.a + bt * g.a_batch;
  const float* Bb = g.b + bt * g.b_batch;

  // bias and residual terms first
  const float* R = g.res ? g.res + bt * g.r_batch : nullptr;
  const int64_t j = n0 + l16;
  const int64_t rcol = (R && j < N) ? res_col(g, j) : 0;
  float bld[MBW][4], rld[MBW][4];
#pragma unroll
  for (int mb = 0; mb < MBW; mb++)
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int64_t i = m0 + 16 * mb + 4 * lg + v;
      const bool ok = i < M && j < N;
      bld[mb][v] = (g.bias_mode == 1 && ok) ? g.bias[i] : 0.0f;
      rld[mb][v] = (R && ok) ? R[i * g.ldr + rcol] : 0.0f;
    }
  __asm__ volatile("" ::: "memory");

  // per-lane slab offsets (the k0 part is the scalar offset)
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)Bb, 0, (int)(g.k * g.ldb * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)Ab, 0, (int)(M * g.lda * 4), 0x00020000);
  const int xrow = lane >> 2, xc = lane & 3;
  const unsigned xoff = (n0 + 4 * xc < N) ? (unsigned)((xrow * g.ldb + n0 + 4 * xc) * 4) : OOB;
  unsigned woff[MBW];
#pragma unroll
  for (int q = 0; q < MBW; q++) {
    const int idx = 64 * q + lane, r = idx >> 2, c = (idx & 3) ^ (r & 3);
    woff[q] = (m0 + r < M) ? (unsigned)(((m0 + r) * g.lda + 4 * c) * 4) : OOB;
  }
  const unsigned xstep = __builtin_amdgcn_readfirstlane((unsigned)(16 * g.ldb * 4));
  const int nslab = (int)(g.k / 16);
  auto issue = [&](int q) {
    float* st = pw_lds + (q % NST) * STAGE;
    const unsigned lx = __builtin_amdgcn_readfirstlane(
        (unsigned)(uintptr_t)(__attribute__((address_space(3))) float*)st);
    const unsigned sx = (unsigned)q * xstep, sw = (unsigned)q * 64u;
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"   // m0 is reserved; nothing else uses it here
    __asm__ volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lx),
                     "v"(xoff), "s"(xr), "s"(sx)
                     : "m0");
#pragma unroll
    for (int w = 0; w < MBW; w++)
      __asm__ volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(
                           lx + 1024u * (1 + w)),
                       "v"(woff[w]), "s"(wr), "s"(sw)
                       : "m0");
#pragma clang diagnostic pop
  };
#pragma unroll
  for (int q = 0; q < NST - 1; q++)
    if (q < nslab) issue(q);
  // the bias and residual values are first used after the first loads are out
#pragma unroll
  for (int mb = 0; mb < MBW; mb++)
    __asm__ volatile("" : "+v"(bld[mb][0]), "+v"(bld[mb][1]), "+v"(bld[mb][2]),
                     "+v"(bld[mb][3]), "+v"(rld[mb][0]), "+v"(rld[mb][1]), "+v"(rld[mb][2]),
                     "+v"(rld[mb][3])::"memory");
  f32x4 acc[MBW];
  float bterm[MBW][4];
#pragma unroll
  for (int mb = 0; mb < MBW; mb++)
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int64_t i = m0 + 16 * mb + 4 * lg + v;
      const bool seeded = g.bias_mode == 1 && i < M && j < N && bias_seeded(g.seed_rule, i, j, M, N);
      acc[mb][v] = seeded ? bld[mb][v] : 0.0f;
      bterm[mb][v] = (g.bias_mode == 1 && !seeded) ? bld[mb][v] : -0.0f;
    }
  // operand offsets inside a stage
  const int boff = lg * 16 + l16;   // + 64 s
  int aoff[MBW];
#pragma unroll
  for (int mb = 0; mb < MBW; mb++) {
    const int r = 16 * mb + l16;
    aoff[mb] = 256 + r * 16 + lg;   // + 4 (s ^ (r & 3))
  }
  for (int q = 0; q < nslab; q++) {
    __asm__ volatile("" ::: "memory");
    if (q + NST - 1 < nslab) {
      __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): slab q - 1's reads are done
      issue(q + NST - 1);
    }
    // slab q in: the loads of the slabs after it may still be in flight
    const int after = min(NST - 1, nslab - 1 - q);
    if (NST >= 4 && after >= 3) wait_vmcnt<3 * PER>();
    else if (NST >= 3 && after == 2) wait_vmcnt<2 * PER>();
    else if (after == 1) wait_vmcnt<PER>();
    else wait_vmcnt<0>();
    __asm__ volatile("" ::: "memory");
    const float* st = pw_lds + (q % NST) * STAGE;
    float bv[4], av[4][MBW];
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++) {
      bv[s4] = st[boff + 64 * s4];
#pragma unroll
      for (int mb = 0; mb < MBW; mb++) {
        const int r = 16 * mb + l16;
        av[s4][mb] = st[aoff[mb] + 4 * (s4 ^ (r & 3))];
      }
    }
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++)
#pragma unroll
      for (int mb = 0; mb < MBW; mb++)
        acc[mb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[s4][mb], bv[s4], acc[mb], 0, 0, 0);
  }
  float* Cb = g.c + bt * g.c_batch;
#pragma unroll
  for (int mb = 0; mb < MBW; mb++)
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int64_t i = m0 + 16 * mb + 4 * lg + v;
      if (i >= M || j >= N) continue;
      float x = acc[mb][v] + bterm[mb][v];
      x = act_apply(x, g.act);
      if (R) x = x + rld[mb][v];
      Cb[i * g.ldc + j] = x;
    }
}

template <int MBW, int NST>
__global__ __launch_bounds__(64) void gemm_pw_kernel(GemmArgs g, int mgroups) {
  extern __shared__ float pw_lds[];
  pw_tile<MBW, NST>(g, mgroups, blockIdx.x, blockIdx.z, pw_lds);
}

// Up to three independent pointwise GEMMs in one launch, one 16-row block a
// wave (the FPN laterals of the coarse levels, which no longer wait on one
// another): workgroups [start[i], start[i + 1]) take GEMM i.  The branches
// keep each GEMM's arguments in the kernel-argument segment.
struct PwGroup {
  GemmArgs g[3];
  int mgroups[3];
  int start[3];
};

template <int NST>
__global__ __launch_bounds__(64) void gemm_pw_group_kernel(PwGroup p) {
  extern __shared__ float pw_lds[];
  const int b = blockIdx.x;
  if (b >= p.start[2])
    pw_tile<1, NST>(p.g[2], p.mgroups[2], b - p.start[2], blockIdx.z, pw_lds);
  else if (b >= p.start[1])
    pw_tile<1, NST>(p.g[1], p.mgroups[1], b - p.start[1], blockIdx.z, pw_lds);
  else
    pw_tile<1, NST>(p.g[0], p.mgroups[0], b, blockIdx.z, pw_lds);
}

// The pointwise kernel takes K a multiple of 16, M <= 128, 16-byte aligned
// rows of both operands, N a multiple of 4 and offsets within 31 bits.
static bool pw_eligible(const GemmArgs& g) {
  return !g.trans_out && g.part == nullptr && g.bias_mode != 2 && g.k % 16 == 0 &&
         g.k >= 16 && g.m <= 128 && g.n % 4 == 0 && g.ldb % 4 == 0 && g.lda % 4 == 0 &&
         g.a_batch % 4 == 0 && g.b_batch % 4 == 0 && (uintptr_t)g.a % 16 == 0 &&
         (uintptr_t)g.b % 16 == 0 && g.k * g.ldb * 4 < (1ll << 31) &&
         g.m * g.lda * 4 < (1ll << 31) && g.ldb >= g.n && g.lda >= g.k;
}

bool pw_group_eligible(const GemmArgs& g) {
  return pw_eligible(g) && !g.res && g.batch >= 1 && g.batch <= 65535 &&
         (double)ceil_div(g.n, 16) * (double)ceil_div(g.m, 16) < (double)(1 << 29);
}

int launch_pw_group(const GemmArgs* g, int n, hipStream_t s) {
  if (n < 1 || n > 3) return fail(QPH_EINVAL, "pointwise group: 1 to 3 GEMMs");
  PwGroup p{};
  int64_t total = 0;
  bool deep = false;
  for (int i = 0; i < n; i++) {
    if (!pw_group_eligible(g[i]) || g[i].batch != g[0].batch)
      return fail(QPH_EUNSUPPORTED, "pointwise group: a GEMM the group kernel does not take");
    p.g[i] = g[i];
    p.mgroups[i] = (int)ceil_div(g[i].m, 16);
    p.start[i] = (int)total;
    total += ceil_div(g[i].n, 16) * p.mgroups[i];
    deep = deep || g[i].k > 32;
  }
  for (int i = n; i < 3; i++) p.start[i] = (int)total;
  if (total >= (1ll << 31)) return fail(QPH_EUNSUPPORTED, "pointwise group: grid too large");
  const dim3 grid((unsigned)total, 1, (unsigned)g[0].batch);
  const size_t lds = (size_t)(deep ? 4 : 2) * 256 * 2 * 4;
  if (deep)
    hipLaunchKernelGGL(gemm_pw_group_kernel<4>, grid, dim3(64), lds, s, p);
  else
    hipLaunchKernelGGL(gemm_pw_group_kernel<2>, grid, dim3(64), lds, s, p);
  return launch_check("gemm_pw_group_kernel");
}

// FPN top-down over the level-3 maps of every batch item: in4 = t4 + up2(in5)
// and in3 = t3 + up2(in4), each Add rounded as the laterals' residual
// epilogues round it.  A lane takes four consecutive level-3 elements of
// one row (w3 is a multiple of 4): the level-4 values t4 + in5 of their
// columns, in3 = t3 + that, and in4 stored by the even-position elements.
__global__ __launch_bounds__(256) void fpn_topdown_kernel(const float* __restrict__ t4,
                                                          const float* __restrict__ in5,
                                                          const float* __restrict__ t3,
                                                          float* __restrict__ in4,
                                                          float* __restrict__ in3, int h3, int w3,
                                                          int total) {
  const int e0 = ((int)blockIdx.x * 256 + (int)threadIdx.x) * 4;
  if (e0 >= total) return;
  const int hw3 = h3 * w3, w4 = w3 >> 1, w5 = w3 >> 2, hw4 = hw3 >> 2, hw5 = hw3 >> 4;
  const int plane = e0 / hw3, r = e0 - plane * hw3;
  const int y = r / w3, x = r - y * w3;
  const float* a4 = t4 + (int64_t)plane * hw4 + (y >> 1) * w4;
  const float* a5 = in5 + (int64_t)plane * hw5 + (y >> 2) * w5;
  const f32x4 a3 = *(const f32x4*)(t3 + (int64_t)plane * hw3 + r);
  f32x4 o;
  float v4[4];
#pragma unroll
  for (int u = 0; u < 4; u++) {
    v4[u] = a4[(x + u) >> 1] + a5[(x + u) >> 2];
    o[u] = a3[u] + v4[u];
  }
  *(f32x4*)(in3 + (int64_t)plane * hw3 + r) = o;
  if (!(y & 1)) {
    float* d4 = in4 + (int64_t)plane * hw4 + (y >> 1) * w4 + (x >> 1);
    d4[0] = v4[0];
    d4[1] = v4[2];
  }
}

int launch_fpn_topdown(const float* t4, const float* in5, const float* t3, float* in4, float* in3,
                       int64_t n, int64_t c, int64_t h3, int64_t w3, hipStream_t s) {
  if (h3 % 4 || w3 % 4 || h3 <= 0 || w3 <= 0)
    return fail(QPH_EINVAL, "fpn top-down: level-3 sides must be multiples of 4");
  const int64_t total = n * c * h3 * w3;
  if (total <= 0) return QPH_OK;
  if (total >= (1ll << 31)) return fail(QPH_EUNSUPPORTED, "fpn top-down: maps too large");
  const auto al = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  if (!al(t3) || !al(in3)) return fail(QPH_EUNSUPPORTED, "fpn top-down: level-3 maps not 16-byte aligned");
  hipLaunchKernelGGL(fpn_topdown_kernel, dim3((unsigned)ceil_div(total, 1024)), dim3(256), 0, s,
                     t4, in5, t3, in4, in3, (int)h3, (int)w3, (int)total);
  return launch_check("fpn_topdown_kernel");
}

template <int MBW>
static void launch_pw_m(const GemmArgs& g, int mgroups, dim3 grid, bool deep, hipStream_t s) {
  const size_t lds = (size_t)(deep ? 4 : 2) * 256 * (1 + MBW) * 4;
  if (deep)
    hipLaunchKernelGGL((gemm_pw_kernel<MBW, 4>), grid, dim3(64), lds, s, g, mgroups);
  else
    hipLaunchKernelGGL((gemm_pw_kernel<MBW, 2>), grid, dim3(64), lds, s, g, mgroups);
}

static int launch_pw(const GemmArgs& g, hipStream_t s) {
  const int mb = (int)ceil_div(g.m, 16);
  const int64_t pgroups = ceil_div(g.n, 16);
  // blocks per wave: the largest divisor of mb that still leaves >= 2048
  // waves (else 1): more blocks share one X slab, fewer spread the chains
  int mbw = 1;
  for (int c = mb; c >= 1; c--)
    if (mb % c == 0 && pgroups * (mb / c) * g.batch >= 2048) {
      mbw = c;
      break;
    }
  const int mgroups = mb / mbw;
  if (pgroups * mgroups >= (1ll << 31)) return fail(QPH_EUNSUPPORTED, "gemm: grid too large");
  dim3 grid((unsigned)(pgroups * mgroups), 1, (unsigned)g.batch);
  const bool deep = g.k > 32;
  switch (mbw) {
    case 1: launch_pw_m<1>(g, mgroups, grid, deep, s); break;
    case 2: launch_pw_m<2>(g, mgroups, grid, deep, s); break;
    case 3: launch_pw_m<3>(g, mgroups, grid, deep, s); break;
    case 4: launch_pw_m<4>(g, mgroups, grid, deep, s); break;
    case 5: launch_pw_m<5>(g, mgroups, grid, deep, s); break;
    case 6: launch_pw_m<6>(g, mgroups, grid, deep, s); break;
    case 7: launch_pw_m<7>(g, mgroups, grid, deep, s); break;
    default: launch_pw_m<8>(g, mgroups, grid, deep, s); break;
  }
  return launch_check("gemm_pw_kernel");
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
// of 64x64 (2x2 v_mfma_f32_32x32x2f32 accumulators each), K slabs of 16
// (K must be a multiple of 16).
//
// Slabs go from global memory straight into LDS (buffer loads with the LDS
// bit, one word per lane, no staging registers), double-buffered, the next
// slab in flight while the current one is multiplied.  Every LDS position is
// one lane of one load, so the layout is whatever the per-lane offsets say:
//   A slab: [m][h][s], row pitch 20 words (16 + 4 pad), element k = 2s + h.
//     A lane of the MFMA needs A[m][2s + h] for s = 0..7 (h = lane / 32), so
//     one ds_read_b128 brings four k-steps; 20-word rows keep the eight
//     lanes of one b128 read on distinct banks.
//   B slab: rows r = 8h + s hold B[k0 + 2s + h][j0 .. j0 + 127].
// The buffer resources start at the tile's (row, k0) and (k0, column)
// corner, so the per-lane offsets are the same for every slab and tile.
// Range checks give the edges: A rows past M and B rows past K lie beyond
// the range and read 0; B columns past N read the next row's words, which
// only reach output columns past N (never stored).
//
// Persistent: each workgroup walks its tiles; workgroup b runs on XCD b % 8
// (round-robin dispatch) and every XCD owns a contiguous range of tiles in
// column-block-major order, so a B column block stays in that XCD's L2
// while the row blocks pass over it.  The first slab of a workgroup's next
// tile is loaded while the current tile's epilogue runs.

#define WB_BK 16
#define WB_PA 20
#define WB_A (128 * WB_PA)
#define WB_B (WB_BK * 128)
#define WB_STAGE (WB_A + WB_B)
#define WB_AL 10   // A-slab loads per wave (128 * 20 words / 64 lanes / 4 waves)
#define WB_BL 8    // B-slab loads per wave
#define NUM_XCD 8

// (The plain case -- column bias or none, no activation, residual or
// transposed store, the rec head -- runs on gemm_wave_kernel below.)
__global__ __launch_bounds__(256) void gemm_wide_kernel(GemmArgs g, int mb, int nb,
                                                        int ntiles, int per_xcd, int wg_xcd) {
  __shared__ __attribute__((aligned(16))) float lds[2 * WB_STAGE];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int xcd = (int)(blockIdx.x % NUM_XCD), wl = (int)(blockIdx.x / NUM_XCD);
  const int t_end = min(xcd * per_xcd + per_xcd, ntiles);
  int tile = xcd * per_xcd + wl;
  if (tile >= t_end) return;

  const int lr = lane & 31, lh = lane >> 5;
  const int wm0 = (wave & 1) * 64, wn0 = (wave >> 1) * 64;
  // all word offsets below fit 31 bits (checked by the launcher)
  const int M = (int)g.m, N = (int)g.n, K = (int)g.k;
  const int lda = (int)g.lda, ldb = (int)g.ldb;
  const int nk = K / WB_BK;
  const int a_words = (M - 1) * lda + K, b_words = (K - 1) * ldb + N;

  unsigned aoff[WB_AL], boff[WB_BL];
#pragma unroll
  for (int r = 0; r < WB_AL; r++) {
    const int p = (wave + 4 * r) * 64 + lane;
    const int m = p / WB_PA, q = p - m * WB_PA;
    aoff[r] = q < 16 ? (unsigned)(m * lda + 2 * (q & 7) + (q >> 3)) * 4u : 0x80000000u;
  }
#pragma unroll
  for (int r = 0; r < WB_BL; r++) {
    const int p = (wave + 4 * r) * 64 + lane;
    const int row = p >> 7;
    boff[r] = (unsigned)((2 * (row & 7) + (row >> 3)) * ldb + (p & 127)) * 4u;
  }

  // tile t -> batch, row block, column block
  auto corner = [&](int t, int& bz, int& i0, int& j0) {
    const int per_b = mb * nb;
    bz = t / per_b;
    const int tt = t - bz * per_b;
    const int nblk = tt / mb;
    i0 = (tt - nblk * mb) * 128;
    j0 = nblk * 128;
  };
  // loads of slab kt of the tile at (bz, i0, j0) into LDS stage st
  auto issue = [&](int bz, int i0, int j0, int kt, int st) {
    const int k0 = kt * WB_BK;
    const int ab = i0 * lda + k0, bb = k0 * ldb + j0;
    const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(g.a + bz * g.a_batch + ab), 0, (a_words - ab) * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(g.b + bz * g.b_batch + bb), 0, (b_words - bb) * 4, 0x00020000);
    float* sa = lds + st * WB_STAGE;
    float* sb = sa + WB_A;
#pragma unroll
    for (int r = 0; r < WB_AL; r++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          ar, (__attribute__((address_space(3))) void*)(sa + (wave + 4 * r) * 64), 4, aoff[r],
          0, 0, 0);
#pragma unroll
    for (int r = 0; r < WB_BL; r++)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          br, (__attribute__((address_space(3))) void*)(sb + (wave + 4 * r) * 64), 4, boff[r],
          0, 0, 0);
  };

  int bz, i0, j0;
  corner(tile, bz, i0, j0);
  int st = 0;
  issue(bz, i0, j0, 0, st);
  while (true) {
    // accumulators start at 0, or at the bias where the reference seeds it
    // (row bias only; the seeded region is whole 32-column panels)
    f32x16 acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
      for (int ni = 0; ni < 2; ni++) {
#pragma unroll
        for (int v = 0; v < 16; v++) acc[mi][ni][v] = 0.0f;
        const int n0 = j0 + wn0 + ni * 32;
        if (g.bias_mode == 1 && n0 < N &&
            (g.seed_rule == 1 ? n0 >= N - N % 32 : N - n0 < 32)) {
#pragma unroll
          for (int v = 0; v < 16; v++) {
            const int i = i0 + wm0 + mi * 32 + 8 * (v >> 2) + 4 * lh + (v & 3);
            if (i < M && n0 + lr < N && bias_seeded(g.seed_rule, i, n0 + lr, M, N))
              acc[mi][ni][v] = g.bias[i];
          }
        }
      }

    const int next = tile + wg_xcd;
    int nbz = 0, ni0 = 0, nj0 = 0;
    if (next < t_end) corner(next, nbz, ni0, nj0);
    for (int kt = 0; kt < nk; kt++) {
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      // every wave is past slab kt-1, whose stage now takes slab kt+1 (or
      // the next tile's first slab)
      if (kt + 1 < nk)
        issue(bz, i0, j0, kt + 1, st ^ 1);
      else if (next < t_end)
        issue(nbz, ni0, nj0, 0, st ^ 1);
      const float* sa = lds + st * WB_STAGE + (wm0 + lr) * WB_PA + lh * 8;
      const float* sb = lds + st * WB_STAGE + WB_A + lh * 8 * 128 + wn0 + lr;
      f32x4 ga[2][2];
      float gb[2][2][4];
#pragma unroll
      for (int gp = 0; gp < 2; gp++) {
#pragma unroll
        for (int mi = 0; mi < 2; mi++) ga[gp][mi] = *(const f32x4*)(sa + mi * 32 * WB_PA + gp * 4);
#pragma unroll
        for (int ni = 0; ni < 2; ni++)
#pragma unroll
          for (int u = 0; u < 4; u++) gb[gp][ni][u] = sb[(gp * 4 + u) * 128 + ni * 32];
      }
#pragma unroll
      for (int gp = 0; gp < 2; gp++)
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
          for (int mi = 0; mi < 2; mi++)
#pragma unroll
            for (int ni = 0; ni < 2; ni++)
              acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(ga[gp][mi][u], gb[gp][ni][u],
                                                                 acc[mi][ni], 0, 0, 0);
      // all of the slab's operand reads go out before its 32 MFMAs
      __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 32, 0);
      st ^= 1;
    }

    float* C = g.c + (int64_t)bz * g.c_batch;
    const float* R = g.res ? g.res + (int64_t)bz * g.r_batch : nullptr;
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
      for (int ni = 0; ni < 2; ni++) {
        EpiIn e[16];
        const int64_t rc = R ? res_col(g, j0 + wn0 + ni * 32 + lr) : 0;
#pragma unroll
        for (int v = 0; v < 16; v++)
          e[v] = epilogue_gather(g, R, i0 + wm0 + mi * 32 + 8 * (v >> 2) + 4 * lh + (v & 3),
                                 j0 + wn0 + ni * 32 + lr, rc);
#pragma unroll
        for (int v = 0; v < 16; v++)
          epilogue_put(g, C, R != nullptr, e[v],
                       i0 + wm0 + mi * 32 + 8 * (v >> 2) + 4 * lh + (v & 3),
                       j0 + wn0 + ni * 32 + lr, acc[mi][ni][v]);
      }
    if (next >= t_end) break;
    tile = next;
    bz = nbz;
    i0 = ni0;
    j0 = nj0;
  }
}

// ------------------------------------------------ one-wave 64x64 tiles
//
// The rec head (PLAIN: column bias, no activation / residual / transposed
// store) on workgroups of a single wave, each owning whole 64x64 tiles: the
// wave loads its own A and B slabs (K in slabs of 16, double-buffered), so
// no workgroup barrier ties its progress to other waves.  Two such waves per
// SIMD keep the MFMA pipe fed through each other's slab waits, where the
// four-wave 128x128 tiles stall together at every slab barrier.  Persistent
// and XCD-aware like gemm_wide_kernel; tiles of 64.
//
// Slabs arrive by 16-byte buffer->LDS loads (a slab is 5 + 4 instructions):
// A as its rows, k in order, 20 words a row (the fifth four-word chunk of a
// row is padding and reads 0); B as the rows of gemm_wide_kernel (r = 8h + s
// holds k = 2s + h).  A lane reads its A terms k = 2s + h two words apart
// (ds_read2) and its B terms one word each.

#define WV_PA 20
#define WV_A (64 * WV_PA)
#define WV_B (16 * 64)
#define WV_STAGE (WV_A + WV_B)
#define WV_AL (WV_A / 256)  // A-slab loads (16 bytes a lane)
#define WV_BL (WV_B / 256)  // B-slab loads (16 bytes a lane: four 64-column rows each)

// Epilogue modes: WV_EPI_ELEM each lane stores its own 64 values;
// WV_EPI_ROWS the row-store epilogue (whole 64-row blocks, 16-byte aligned
// output rows); WV_EPI_ARGMAX no C at all: per row of the tile, the
// (max, first index of the max, sum of exp1(v - max)) of its 64 columns goes
// to g.part (one float4 per row and 64-column block), for head_pairs_kernel.
#define WV_EPI_ELEM 0
#define WV_EPI_ROWS 1
#define WV_EPI_ARGMAX 2

template <int EPI>
__global__ __launch_bounds__(64) void gemm_wave_kernel(GemmArgs g, int mb, int nb, int ntiles,
                                                       int per_xcd, int wg_xcd) {
  constexpr bool ROWS = EPI == WV_EPI_ROWS;
  __shared__ __attribute__((aligned(16))) float lds[2 * WV_STAGE];
  const int lane = threadIdx.x;
  const int xcd = (int)(blockIdx.x % NUM_XCD), wl = (int)(blockIdx.x / NUM_XCD);
  const int t_end = min(xcd * per_xcd + per_xcd, ntiles);
  int tile = xcd * per_xcd + wl;
  if (tile >= t_end) return;
  const int lr = lane & 31, lh = lane >> 5;
  // all word offsets fit 31 bits (checked by the launcher)
  const int M = (int)g.m, N = (int)g.n, K = (int)g.k;
  const int lda = (int)g.lda, ldb = (int)g.ldb;
  const int nk = K / WB_BK;
  const int a_words = (M - 1) * lda + K, b_words = (K - 1) * ldb + N;
  unsigned aoff[WV_AL], boff[WV_BL];
#pragma unroll
  for (int u = 0; u < WV_AL; u++) {
    // four-word chunk c = 64u + lane: row c / 5, k 4 (c % 5) .. + 3 (the
    // fifth chunk of a row is its padding: out of range, reads 0)
    const int c = u * 64 + lane;
    const int m = c / 5, q = c - m * 5;
    aoff[u] = q < 4 ? (unsigned)(m * lda + 4 * q) * 4u : 0x80000000u;
  }
#pragma unroll
  for (int u = 0; u < WV_BL; u++) {
    // row r holds B[k0 + 2s + h][j0 .. j0 + 63] for r = 8h + s; load u
    // brings rows 4u .. 4u + 3, lane L four columns of row 4u + L / 16
    const int r = 4 * u + (lane >> 4);
    boff[u] = (unsigned)((2 * (r & 7) + (r >> 3)) * ldb + 4 * (lane & 15)) * 4u;
  }
  auto corner = [&](int t, int& bz, int& i0, int& j0) {
    const int per_b = mb * nb;
    bz = t / per_b;
    const int tt = t - bz * per_b;
    const int nblk = tt / mb;
    i0 = (tt - nblk * mb) * 64;
    j0 = nblk * 64;
  };
  auto issue = [&](int bz, int i0, int j0, int kt, int st) {
    const int k0 = kt * WB_BK;
    const int ab = i0 * lda + k0, bb = k0 * ldb + j0;
    const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(g.a + bz * g.a_batch + ab), 0, (a_words - ab) * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(g.b + bz * g.b_batch + bb), 0, (b_words - bb) * 4, 0x00020000);
    float* sa = lds + st * WV_STAGE;
    float* sb = sa + WV_A;
#pragma unroll
    for (int u = 0; u < WV_AL; u++) lds_load16(ar, sa + u * 256, aoff[u], 0);
#pragma unroll
    for (int u = 0; u < WV_BL; u++) lds_load16(br, sb + u * 256, boff[u], 0);
  };

  int bz, i0, j0;
  corner(tile, bz, i0, j0);
  int st = 0;
  issue(bz, i0, j0, 0, st);
  bool stored = false;   // the previous tile's 16 row stores follow this slab's loads
  while (true) {
    f32x16 acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
      for (int ni = 0; ni < 2; ni++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[mi][ni][v] = 0.0f;
    const int next = tile + wg_xcd;
    int nbz = 0, ni0 = 0, nj0 = 0;
    if (next < t_end) corner(next, nbz, ni0, nj0);
    for (int kt = 0; kt < nk; kt++) {
      // this wave's loads of slab kt are done (the previous tile's row
      // stores, issued after them, may still be draining); its reads of slab
      // kt - 1 are done too, so that stage takes slab kt + 1
      if (ROWS && kt == 0 && stored)
        wait_vmcnt<16>();
      else if (EPI == WV_EPI_ARGMAX && kt == 0 && stored)
        wait_vmcnt<2>();
      else
        wait_vmcnt<0>();
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __asm__ volatile("" ::: "memory");
      if (kt + 1 < nk)
        issue(bz, i0, j0, kt + 1, st ^ 1);
      else if (next < t_end)
        issue(nbz, ni0, nj0, 0, st ^ 1);
      const float* sa = lds + st * WV_STAGE + lr * WV_PA + lh;
      const float* sb = lds + st * WV_STAGE + WV_A + lh * 8 * 64 + lr;
      f32x4 ga[2][2];
      float gb[2][2][4];
#pragma unroll
      for (int gp = 0; gp < 2; gp++) {
#pragma unroll
        for (int mi = 0; mi < 2; mi++)
#pragma unroll
          for (int u = 0; u < 4; u++) ga[gp][mi][u] = sa[mi * 32 * WV_PA + 2 * (4 * gp + u)];
#pragma unroll
        for (int ni = 0; ni < 2; ni++)
#pragma unroll
          for (int u = 0; u < 4; u++) gb[gp][ni][u] = sb[(gp * 4 + u) * 64 + ni * 32];
      }
#pragma unroll
      for (int gp = 0; gp < 2; gp++)
#pragma unroll
        for (int u = 0; u < 4; u++)
#pragma unroll
          for (int mi = 0; mi < 2; mi++)
#pragma unroll
            for (int ni = 0; ni < 2; ni++)
              acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x2f32(ga[gp][mi][u], gb[gp][ni][u],
                                                                 acc[mi][ni], 0, 0, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 32, 0);
      st ^= 1;
    }
    // column bias or none (a term of -0.0 leaves every value unchanged).
    // The tile goes out as rows: each 32-row half through the stage the last
    // slab came from (pitch 72: a write's two row groups and a read's rows
    // fall on distinct banks), then 16-byte stores, four rows of 64 columns
    // per instruction.
    float* C = g.c + (int64_t)bz * g.c_batch;
    float badd[2];
#pragma unroll
    for (int ni = 0; ni < 2; ni++) {
      const int j = j0 + ni * 32 + lr;
      badd[ni] = g.bias_mode == 2 && j < N ? g.bias[j] : -0.0f;
    }
    if constexpr (EPI == WV_EPI_ARGMAX) {
      // each 32-row half through the stage of the last slab (pitch 72), then
      // lane L takes row L % 32, columns 32 (L / 32) .. + 31 of the tile, in
      // order: first strict max, then the exp1 sum against it; lanes L and
      // L + 32 combine; exactly one 16-byte buffer store per half (rows past
      // M and the upper lanes store out of range, which is dropped), so the
      // next tile's first wait can count on two stores in flight
      float* sc = lds + (st ^ 1) * WV_STAGE;
      const int r = lane & 31, ch = lane >> 5;
      const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
          (void*)g.part, 0, (int)((int64_t)M * nb * 16), 0x00020000);
      const int cb = j0 >> 6;
#pragma unroll
      for (int mi = 0; mi < 2; mi++) {
        __builtin_amdgcn_s_waitcnt(0xC07F);
#pragma unroll
        for (int ni = 0; ni < 2; ni++)
#pragma unroll
          for (int v = 0; v < 16; v++)
            sc[(8 * (v >> 2) + 4 * lh + (v & 3)) * 72 + ni * 32 + lr] = acc[mi][ni][v] + badd[ni];
        __builtin_amdgcn_s_waitcnt(0xC07F);
        float vals[32];
#pragma unroll
        for (int q = 0; q < 8; q++) {
          const f32x4 t = *(const f32x4*)(sc + r * 72 + 32 * ch + 4 * q);
          vals[4 * q] = t[0];
          vals[4 * q + 1] = t[1];
          vals[4 * q + 2] = t[2];
          vals[4 * q + 3] = t[3];
        }
        const int jb = j0 + 32 * ch;
        float m = -__builtin_inff();
        int idx = 0x7fffffff;
#pragma unroll
        for (int q = 0; q < 32; q++)
          if (jb + q < N && vals[q] > m) {
            m = vals[q];
            idx = jb + q;
          }
        // exp by the hardware exp2 (the sum only has to agree to float
        // rounding; the polynomial exp1 costs ~7x the instructions here)
        float sum = 0.0f;
#pragma unroll
        for (int q = 0; q < 32; q++)
          if (jb + q < N) sum += __builtin_amdgcn_exp2f((vals[q] - m) * 1.44269504f);
        const float mo = __shfl_xor(m, 32, 64);
        const int io = __shfl_xor(idx, 32, 64);
        const float so = __shfl_xor(sum, 32, 64);
        // lane r (< 32) holds columns 0..31, its partner 32..63
        const float mm = fmaxf(m, mo);
        const int ii = mo > m ? io : idx;
        const float ss = sum * __builtin_amdgcn_exp2f((m - mm) * 1.44269504f) +
                         (so > 0.0f ? so * __builtin_amdgcn_exp2f((mo - mm) * 1.44269504f) : 0.0f);
        const int i = i0 + mi * 32 + r;
        const unsigned off =
            (ch == 0 && i < M) ? (unsigned)(((int64_t)i * nb + cb) * 16) : 0x80000000u;
        f32x4 out;
        out[0] = mm;
        out[1] = __int_as_float(ii);
        out[2] = ss;
        out[3] = 0.0f;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u32_t, out), pr, off, 0, 0);
      }
    } else if constexpr (!ROWS) {
#pragma unroll
      for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < 2; ni++) {
          const int j = j0 + ni * 32 + lr;
          const int ib = i0 + mi * 32 + 4 * lh;
          if (j < N) {
            float* cj = C + j;
#pragma unroll
            for (int v = 0; v < 16; v++) {
              const int i = ib + 8 * (v >> 2) + (v & 3);
              if (i < M) cj[(int64_t)i * g.ldc] = acc[mi][ni][v] + badd[ni];
            }
          }
        }
    } else {
    float* sc = lds + (st ^ 1) * WV_STAGE;   // the stage of slab nk - 1
    const int rr = lane >> 4, c4 = (lane & 15) * 4;
    const int jc = j0 + c4;
#pragma unroll
    for (int mi = 0; mi < 2; mi++) {
      // (the reads of the previous half / slab are back before the writes)
      __builtin_amdgcn_s_waitcnt(0xC07F);
#pragma unroll
      for (int ni = 0; ni < 2; ni++)
#pragma unroll
        for (int v = 0; v < 16; v++)
          sc[(8 * (v >> 2) + 4 * lh + (v & 3)) * 72 + ni * 32 + lr] = acc[mi][ni][v] + badd[ni];
      __builtin_amdgcn_s_waitcnt(0xC07F);
#pragma unroll
      for (int it = 0; it < 8; it++) {
        const int r = 4 * it + rr;
        const int i = i0 + mi * 32 + r;
        const f32x4 val = *(const f32x4*)(sc + r * 72 + c4);
        float* cp = C + (int64_t)i * g.ldc + jc;
        if (i < M) {
          if (jc + 4 <= N) {
            *(f32x4*)cp = val;
          } else {
#pragma unroll
            for (int q = 0; q < 4; q++)
              if (jc + q < N) cp[q] = val[q];
          }
        }
      }
    }
    }
    stored = true;
    if (next >= t_end) break;
    tile = next;
    bz = nbz;
    i0 = ni0;
    j0 = nj0;
  }
}

// Per row: combines the (max, first index, exp1 sum) partials of its nb
// column blocks into the (value, index) pair of the row's softmax argmax.
// One wave per row, one pass over the partials: each lane keeps a running
// (max, index, sum against that max), rescaling the sum when the max rises;
// block t holds columns 64 t .. 64 t + 63, so a lane's first strict max and,
// across lanes, the lower index among equal maxima give the first maximum.
__global__ __launch_bounds__(256) void head_pairs_kernel(const float* __restrict__ part,
                                                         int64_t rows, int nb,
                                                         float* __restrict__ pairs) {
  const float L2E = 1.44269504f;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const f32x4* pr = (const f32x4*)part + row * nb;
  float m = -__builtin_inff(), sum = 0.0f;
  int idx = 0x7fffffff;
  for (int t = lane; t < nb; t += 64) {
    const f32x4 q = pr[t];
    if (q[0] > m) {
      sum = (sum > 0.0f ? sum * __builtin_amdgcn_exp2f((m - q[0]) * L2E) : 0.0f) + q[2];
      m = q[0];
      idx = __float_as_int(q[1]);
    } else {
      sum += q[2] * __builtin_amdgcn_exp2f((q[0] - m) * L2E);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float mo = __shfl_xor(m, off, 64);
    const int io = __shfl_xor(idx, off, 64);
    const float so = __shfl_xor(sum, off, 64);
    const float mm = fmaxf(m, mo);
    // a lane without partials has sum 0 and max -inf: its term is 0
    sum = (sum > 0.0f ? sum * __builtin_amdgcn_exp2f((m - mm) * L2E) : 0.0f) +
          (so > 0.0f ? so * __builtin_amdgcn_exp2f((mo - mm) * L2E) : 0.0f);
    if (mo > m || (mo == m && io < idx)) idx = io;
    m = mm;
  }
  if (lane == 0) {
    pairs[2 * row] = 1.0f / sum;   // the max's exponential is exp1(0) = 1
    pairs[2 * row + 1] = __int_as_float(idx);
  }
}

bool head_argmax_eligible(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb) {
  const int64_t tiles = (int64_t)ceil_div(m, 64) * ceil_div(n, 64);
  return m > 0 && n > 0 && k > 0 && k % WB_BK == 0 && lda % 4 == 0 && tiles < (1ll << 30) &&
         ((m - 1) * lda + k) * 4 < (1ll << 31) && ((k - 1) * ldb + n) * 4 < (1ll << 31) &&
         (k * ldb + 128) * 4 < (1ll << 31) && (64 * lda + k) * 4 < (1ll << 31) &&
         m * ceil_div(n, 64) * 16 < (1ll << 31);
}

int64_t head_argmax_part_floats(int64_t m, int64_t n) { return m * ceil_div(n, 64) * 4; }

// Logits x[M][K] . w[K][N] + bias[N] never stored: the one-wave GEMM's
// argmax epilogue writes per-block partials, head_pairs_kernel the pairs.
int launch_head_argmax(const float* x, int64_t m, int64_t k, const float* w, int64_t ldb,
                       int64_t n, const float* bias, float* part, float* pairs, hipStream_t s) {
  if (!head_argmax_eligible(m, n, k, k, ldb))
    return fail(QPH_EUNSUPPORTED, "fused head: shape outside the one-wave GEMM");
  if ((uintptr_t)x % 16 != 0) return fail(QPH_EUNSUPPORTED, "fused head: A not 16-byte aligned");
  GemmArgs g{};
  g.a = x; g.lda = k; g.b = w; g.ldb = ldb;
  g.m = m; g.n = n; g.k = k; g.batch = 1;
  g.bias = bias; g.bias_mode = bias ? 2 : 0;
  g.act = make_act(nullptr);
  g.part = part;
  const int mb = (int)ceil_div(m, 64), nb = (int)ceil_div(n, 64);
  const int ntiles = mb * nb;
  const int per_xcd = (ntiles + NUM_XCD - 1) / NUM_XCD;
  // one tile a wave (not persistent): with pages in flight the other
  // streams' kernels get CUs between the head's waves (two pages: 3477
  // against 3421 steps/s with the persistent grid); alone on the GPU the
  // persistent grid is ahead (one page in flight: 2877 against 2801)
  const int wg_xcd = std::max(1, per_xcd);
  hipLaunchKernelGGL(gemm_wave_kernel<WV_EPI_ARGMAX>, dim3((unsigned)(wg_xcd * NUM_XCD)), dim3(64),
                     0, s, g, mb, nb, ntiles, per_xcd, wg_xcd);
  QPH_TRY(launch_check("gemm_wave_kernel<argmax>"));
  hipLaunchKernelGGL(head_pairs_kernel, dim3(ceil_div(m, 4)), dim3(256), 0, s, part, m, nb, pairs);
  return launch_check("head_pairs_kernel");
}

static int launch_wave(const GemmArgs& g, hipStream_t s) {
  int occ = 0, cus = 0;
  QPH_TRY(device_cus(nullptr, &cus));
  QPH_TRY(kernel_occupancy((const void*)gemm_wave_kernel<WV_EPI_ROWS>, 64, &occ));
  const int mb = (int)ceil_div(g.m, 64), nb = (int)ceil_div(g.n, 64);
  const int ntiles = mb * nb * (int)g.batch;
  const int per_xcd = (ntiles + NUM_XCD - 1) / NUM_XCD;
  const int wg_xcd = std::max(1, std::min(per_xcd, occ * cus / NUM_XCD));
  // whole 64-row blocks: every tile issues its 16 row stores, which the
  // next tile's first wait counts on; 16-byte aligned output rows
  const bool rows = g.m % 64 == 0 && g.ldc % 4 == 0 && (uintptr_t)g.c % 16 == 0 &&
                    g.c_batch % 4 == 0;
  if (rows)
    hipLaunchKernelGGL(gemm_wave_kernel<WV_EPI_ROWS>, dim3((unsigned)(wg_xcd * NUM_XCD)), dim3(64), 0, s,
                       g, mb, nb, ntiles, per_xcd, wg_xcd);
  else
    hipLaunchKernelGGL(gemm_wave_kernel<WV_EPI_ELEM>, dim3((unsigned)(wg_xcd * NUM_XCD)), dim3(64), 0, s,
                       g, mb, nb, ntiles, per_xcd, wg_xcd);
  return launch_check("gemm_wave_kernel");
}

// K in whole slabs, operands within the 32-bit buffer offsets.
static bool wide_fits(const GemmArgs& g) {
  const int64_t ab = ((g.m - 1) * g.lda + g.k) * 4, bb = ((g.k - 1) * g.ldb + g.n) * 4;
  return g.k % WB_BK == 0 && ab < (1ll << 31) && bb < (1ll << 31) &&
         (g.k * g.ldb + 128) * 4 < (1ll << 31) && (128 * g.lda + g.k) * 4 < (1ll << 31);
}

static int launch_wide(const GemmArgs& g, hipStream_t s) {
  int occ = 0, cus = 0;
  QPH_TRY(device_cus(nullptr, &cus));
  QPH_TRY(kernel_occupancy((const void*)gemm_wide_kernel, 256, &occ));
  const int mb = (int)ceil_div(g.m, 128), nb = (int)ceil_div(g.n, 128);
  const int ntiles = mb * nb * (int)g.batch;
  const int per_xcd = (ntiles + NUM_XCD - 1) / NUM_XCD;
  const int wg_xcd = std::max(1, std::min(per_xcd, occ * cus / NUM_XCD));
  hipLaunchKernelGGL(gemm_wide_kernel, dim3((unsigned)(wg_xcd * NUM_XCD)), dim3(256), 0, s, g, mb,
                     nb, ntiles, per_xcd, wg_xcd);
  return launch_check("gemm_wide_kernel");
}

// Tile choice: 128x128 tiles when they still yield about two workgroups per
// CU (256 CUs) for the whole launch, else the 32x32 kernels.
bool gemm_takes_wide(int64_t m, int64_t n, int64_t batch) {
  const double tiles = (double)ceil_div(m, 128) * (double)ceil_div(n, 128) * (double)batch;
  return m >= 128 && n >= 128 && tiles >= 512;
}

int launch_gemm(const GemmArgs& g, hipStream_t s) {
  if (g.m <= 0 || g.n <= 0 || g.k <= 0 || g.batch <= 0) return QPH_OK;
  if (g.m > (1ll << 31) || g.n > (1ll << 31) || g.batch > 65535)
    return fail(QPH_EUNSUPPORTED, "gemm: dimension too large");
  if (gemm_takes_wide(g.m, g.n, g.batch)) {
    const double tiles = (double)ceil_div(g.m, 128) * (double)ceil_div(g.n, 128) * (double)g.batch;
    const bool plain = g.act.kind == 0 && g.res == nullptr && !g.trans_out && g.bias_mode != 1;
    // (16-byte aligned A rows for the one-wave kernel's slab loads)
    if (plain && wide_fits(g) && g.lda % 4 == 0 && (uintptr_t)g.a % 16 == 0 &&
        g.a_batch % 4 == 0 && tiles < (double)(1u << 28))
      return launch_wave(g, s);
    if (wide_fits(g) && tiles < (double)(1u << 30)) return launch_wide(g, s);
    return launch_cfg<2, 2>(g, s);
  }
  if (pw_eligible(g)) return launch_pw(g, s);
  return launch_skinny(g, s);
}

// ------------------------------------------------- linears, resident W^T
//
// The session's linears below the 128x128 size (the rec QKV, projection and
// MLP, 1280 x {256..1024} x {256, 1024}) keep their weight transposed,
// Wt[N][K], so both operands are k-contiguous rows.  A workgroup owns TM x TN
// outputs (TM, TN in {32, 64}) as 2 x 2 waves; a wave holds
// (TM/32) x (TN/32) 16x16 blocks, each accumulated with v_mfma_f32_16x16x4f32
// (four k per instruction, in order), so a K-deep output is K/4 dependent
// MFMAs and a wave interleaves the chains of its blocks.  On these shapes
// the cost is the MFMA chains plus the operand traffic from L2, which the
// tile shape trades against each other (larger tiles: fewer bytes per
// FLOP, fewer waves to spread the chains over); the launcher picks it.
//
// K advances in slabs of 64 through a ring of NS LDS stages filled by
// 16-byte buffer->LDS loads (no staging registers; one instruction moves
// four 256-byte slab rows); NS - 1 slabs are in flight while one is
// multiplied.  Each stage's A and Wt slabs are __shared__ arrays of their
// own and the loop is unrolled over the ring, so the compiler can tell the
// loads into one slab from the reads of another (and places no wait of its
// own before the operand reads).
// Slab rows are 64 words (16 chunks of 4 k) with the chunks XOR-swizzled by
// the row: chunk c of row r sits at chunk position c ^ (r % 16).  A load lane
// picks its source chunk to match, and the MFMA lane that needs k = 4s + g of
// row r reads word 4 (s ^ (r % 16)) + g: the 64 lanes of one read (16 rows x
// 4 g) then hit 64 distinct banks.  Rows past M or N read 0 through the
// buffer range check (their outputs are not stored).
//
// Workgroup b runs on XCD b % 8; XCD x takes the contiguous tile range
// [x * per_xcd, (x + 1) * per_xcd) in row-block-major order, so its L2 holds
// a few A row blocks and the whole (small) Wt, instead of every A row block
// for a few Wt column blocks.

#define LT_BK 64


// NK > 0: K / 64 fixed at compile time, so the slab loop unrolls completely
// (and each stage's loads and reads stay distinguishable to the compiler's
// wait placement across the whole chain); NK = 0: any K / 64, run-time loop.
template <int TM, int TN, int NS, int NK>
__global__ __launch_bounds__(256) void linear_nt_kernel(LinArgs g, int ntiles, int per_xcd) {
  static_assert((TM == 32 || TM == 64) && (TN == 32 || TN == 64) && (NS >= 2 && NS <= 4), "");
  constexpr int BM = TM / 32, BN = TN / 32;   // 16x16 blocks per wave
  constexpr int LA = TM / 16, LB = TN / 16;   // loads per wave per slab
  constexpr int L = LA + LB;
  // stage s: A slab in sN, Wt slab in tN
  __shared__ __attribute__((aligned(16))) float s0[TM * LT_BK], s1[TM * LT_BK], s2[TM * LT_BK],
      s3[TM * LT_BK];
  __shared__ __attribute__((aligned(16))) float t0[TN * LT_BK], t1[TN * LT_BK], t2[TN * LT_BK],
      t3[TN * LT_BK];
  const int tid = threadIdx.x, lane = tid & 63;
  // "& 3" bounds the wave index for the compiler: with it the LDS offsets of
  // every load and read have known ranges, which is what lets the compiler
  // see that a stage's reads do not touch the stages still loading
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6) & 3;
  const int lg = lane >> 4, l16 = lane & 15;
  const int wm = wave & 1, wn = wave >> 1;
  // all word offsets fit 31 bits (checked by the launcher)
  const int M = (int)g.m, N = (int)g.n, K = (int)g.k, lda = (int)g.lda;
  const int nb = (N + TN - 1) / TN;
  const int tile = (int)(blockIdx.x % NUM_XCD) * per_xcd + (int)(blockIdx.x / NUM_XCD);
  if (tile >= ntiles) return;
  const int i0 = (tile / nb) * TM, j0 = (tile % nb) * TN;
  const int nk = NK > 0 ? NK : K / LT_BK;

  const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
      (void*)g.a, 0, ((M - 1) * lda + K) * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
      (void*)g.wt, 0, N * K * 4, 0x00020000);
  // this wave loads slab rows [wave * TM/4, (wave + 1) * TM/4) of A (and the
  // same for Wt with TN), four rows per instruction: lane L -> row
  // wave * TM/4 + 4u + L/16, chunk position L % 16
  unsigned aoff[LA], boff[LB];
#pragma unroll
  for (int u = 0; u < LA; u++) {
    const int rl = wave * (TM / 4) + 4 * u + (lane >> 4);
    const int r = i0 + rl;
    aoff[u] = r < M ? (unsigned)(r * lda + 4 * ((lane & 15) ^ (rl & 15))) * 4u : 0x80000000u;
  }
#pragma unroll
  for (int u = 0; u < LB; u++) {
    const int rl = wave * (TN / 4) + 4 * u + (lane >> 4);
    const int n = j0 + rl;
    boff[u] = n < N ? (unsigned)(n * K + 4 * ((lane & 15) ^ (rl & 15))) * 4u : 0x80000000u;
  }

  auto stage_a = [&](auto st) -> float* {
    constexpr int S = decltype(st)::value;
    if constexpr (S == 0) return s0;
    else if constexpr (S == 1) return s1;
    else if constexpr (S == 2) return s2;
    else return s3;
  };
  auto stage_b = [&](auto st) -> float* {
    constexpr int S = decltype(st)::value;
    if constexpr (S == 0) return t0;
    else if constexpr (S == 1) return t1;
    else if constexpr (S == 2) return t2;
    else return t3;
  };
  // slab kt -> stage S: L loads per wave (k offset in the scalar offset)
  auto issue = [&](auto st, int kt) {
    float* a = stage_a(st) + wave * (TM / 4) * LT_BK;
    float* b = stage_b(st) + wave * (TN / 4) * LT_BK;
    const int so = kt * LT_BK * 4;
#pragma unroll
    for (int u = 0; u < LA; u++) lds_load16(ar, a + 4 * u * LT_BK, aoff[u], so);
#pragma unroll
    for (int u = 0; u < LB; u++) lds_load16(br, b + 4 * u * LT_BK, boff[u], so);
  };
  // each chain starts at 0, or at its column's bias when the bias seeds it
  // (a lane's four accumulator rows share the column j)
  f32x4 acc[BM][BN];
#pragma unroll
  for (int bn = 0; bn < BN; bn++) {
    const int j = j0 + wn * (TN / 2) + bn * 16 + l16;
    const float b0 = (g.bias_seed && g.bias && j < N) ? g.bias[j] : 0.0f;
#pragma unroll
    for (int bm = 0; bm < BM; bm++) acc[bm][bn] = f32x4{b0, b0, b0, b0};
  }
  float av[BM][16], bv[BN][16];
  // operands of a slab: lane (g, l16) takes k = 4s + g of its rows, s = 0..15
  auto fetch = [&](auto st) {
#pragma unroll
    for (int bm = 0; bm < BM; bm++) {
      const float* a = stage_a(st) + (wm * (TM / 2) + bm * 16 + l16) * LT_BK + lg;
#pragma unroll
      for (int s = 0; s < 16; s++) av[bm][s] = a[4 * (s ^ l16)];
    }
#pragma unroll
    for (int bn = 0; bn < BN; bn++) {
      const float* b = stage_b(st) + (wn * (TN / 2) + bn * 16 + l16) * LT_BK + lg;
#pragma unroll
      for (int s = 0; s < 16; s++) bv[bn][s] = b[4 * (s ^ l16)];
    }
  };
  auto mfmas = [&]() {
#pragma unroll
    for (int s = 0; s < 16; s++)
#pragma unroll
      for (int bm = 0; bm < BM; bm++)
#pragma unroll
        for (int bn = 0; bn < BN; bn++)
          acc[bm][bn] =
              __builtin_amdgcn_mfma_f32_16x16x4f32(av[bm][s], bv[bn][s], acc[bm][bn], 0, 0, 0);
  };
  // workgroup barrier that leaves the loads in flight: only this wave's
  // LDS reads must be back (lgkmcnt 0) before a stage it read is refilled
  auto barrier = [&]() {
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;

  // epilogue operands (bias, residual) loaded now, their latency under the
  // slab loop's
  float badd[BN], rres[BM][BN][4];
#pragma unroll
  for (int bn = 0; bn < BN; bn++) {
    const int j = j0 + wn * (TN / 2) + bn * 16 + l16;
    badd[bn] = (g.bias && !g.bias_seed && j < N) ? g.bias[j] : -0.0f;
#pragma unroll
    for (int bm = 0; bm < BM; bm++) {
      const int ib = i0 + wm * (TM / 2) + bm * 16 + 4 * lg;
#pragma unroll
      for (int v = 0; v < 4; v++)
        rres[bm][bn][v] = (g.res && j < N && ib + v < M) ? g.res[(int64_t)(ib + v) * N + j] : 0.0f;
    }
  }

  issue(S0{}, 0);
  if constexpr (NS > 2)
    if (nk > 1) issue(S1{}, 1);
  if constexpr (NS > 3)
    if (nk > 2) issue(S2{}, 2);
  // slab t: wait until it is in (at most the NS - 2 slabs after it still
  // loading), then refill the stage freed by slab t - 1 with slab t + NS - 1
  auto step = [&](auto st, int t) {
    constexpr int S = decltype(st)::value;
    const int ahead = NS == 2 ? 0 : min(NS - 2, nk - 1 - t);
    if (ahead >= 2) wait_vmcnt<2 * L>();
    else if (ahead == 1) wait_vmcnt<L>();
    else wait_vmcnt<0>();
    barrier();
    // the operand reads go out before the refill, so they wait on no load
    fetch(st);
    if (t + NS - 1 < nk) issue(std::integral_constant<int, (S + NS - 1) % NS>{}, t + NS - 1);
    mfmas();
  };
  auto ring = [&](int t) {
    step(S0{}, t);
    if (t + 1 < nk) step(S1{}, t + 1);
    if constexpr (NS > 2)
      if (t + 2 < nk) step(S2{}, t + 2);
    if constexpr (NS > 3)
      if (t + 3 < nk) step(S3{}, t + 3);
  };
  if constexpr (NK > 0) {
#pragma unroll
    for (int t = 0; t < NK; t += NS) ring(t);
  } else {
    for (int t = 0; t < nk; t += NS) ring(t);
  }

  // epilogue: MatMul, then + bias (a term of -0.0 leaves a value unchanged),
  // activation, then + residual
#pragma unroll
  for (int bn = 0; bn < BN; bn++) {
    const int j = j0 + wn * (TN / 2) + bn * 16 + l16;
    if (j >= N) continue;
#pragma unroll
    for (int bm = 0; bm < BM; bm++) {
      const int ib = i0 + wm * (TM / 2) + bm * 16 + 4 * lg;
#pragma unroll
      for (int v = 0; v < 4; v++) {
        if (ib + v >= M) continue;
        float x = acc[bm][bn][v] + badd[bn];
        x = act_apply(x, g.act);
        if (g.res) x = x + rres[bm][bn][v];
        g.c[(int64_t)(ib + v) * N + j] = x;
      }
    }
  }
}

bool linear_nt_eligible(int64_t m, int64_t n, int64_t k, int64_t lda) {
  if (m <= 0 || n <= 0 || k < LT_BK || k % LT_BK != 0 || lda < k) return false;
  return ((m - 1) * lda + k) * 4 < (1ll << 31) && n * k * 4 < (1ll << 31) &&
         m * n < (1ll << 31) && (double)ceil_div(m, 32) * (double)ceil_div(n, 32) < 1e9;
}

template <int TM, int TN, int NS>
static void launch_lt(const LinArgs& g, hipStream_t s) {
  const int ntiles = (int)(ceil_div(g.n, TN) * ceil_div(g.m, TM));
  const int per_xcd = (ntiles + NUM_XCD - 1) / NUM_XCD;
  const dim3 grid((unsigned)(per_xcd * NUM_XCD));
  const int64_t nk = g.k / LT_BK;
  if (nk == 4)
    hipLaunchKernelGGL((linear_nt_kernel<TM, TN, NS, 4>), grid, dim3(256), 0, s, g, ntiles, per_xcd);
  else if (nk == 16)
    hipLaunchKernelGGL((linear_nt_kernel<TM, TN, NS, 16>), grid, dim3(256), 0, s, g, ntiles,
                       per_xcd);
  else
    hipLaunchKernelGGL((linear_nt_kernel<TM, TN, NS, 0>), grid, dim3(256), 0, s, g, ntiles, per_xcd);
}

// Tile shape and ring depth as measured on the rec linears (1280 rows, K
// 256 / 1024, N 256..1024) and 1x1 convs (K 64..256): 32x32 tiles beat 64x32
// and 64x64 on all of them.  Three stages (48 KB, three workgroups per CU)
// beat four (two per CU) and, where the slabs are many or the tiles fill
// three workgroups per CU, two; two stages (32 KB) win for K <= 128 and when
// the tiles need two rounds at three per CU but one at four (QKV: 960).
int launch_linear_nt(const LinArgs& g, hipStream_t s) {
  if (!linear_nt_eligible(g.m, g.n, g.k, g.lda))
    return fail(QPH_EUNSUPPORTED, "linear: shape outside the resident-weight kernel");
  int cus_i = 0;
  QPH_TRY(device_cus(nullptr, &cus_i));
  const int64_t tiles = (int64_t)ceil_div(g.m, 32) * ceil_div(g.n, 32);
  const int64_t cus = cus_i;
  if (g.k <= 128 || (tiles > 3 * cus && tiles <= 4 * cus))
    launch_lt<32, 32, 2>(g, s);
  else
    launch_lt<32, 32, 3>(g, s);
  return launch_check("linear_nt_kernel");
}

__global__ void transpose_kernel(const float* __restrict__ w, int64_t k, int64_t n,
                                 float* __restrict__ wt) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= k * n) return;
  const int64_t j = e / k, i = e - j * k;
  wt[e] = w[i * n + j];
}

int launch_transpose(const float* w, int64_t k, int64_t n, float* wt, hipStream_t s) {
  if (k <= 0 || n <= 0) return QPH_OK;
  hipLaunchKernelGGL(transpose_kernel, dim3(ceil_div(k * n, 256)), dim3(256), 0, s, w, k, n, wt);
  return launch_check("transpose_kernel");
}

}  // namespace qph
