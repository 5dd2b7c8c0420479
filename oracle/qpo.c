/*
 * qpo.c -- CPU oracle: a plain-C restatement of the qppocr-kernels CPU
 * arithmetic for the det/rec operator set.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP library and
 * the "port" CPU baseline timed next to it.  Nothing in the product
 * (qppocr_amd/, include/) links, loads or calls it.
 *
 * The reference is Rust (crates/qppocr-kernels); its scalar "judge" kernels
 * are bit-identical to its AVX2 kernels (qppocr-kernels/src/x86.rs:1-9), so a
 * scalar C restatement that keeps every fma, every rounding step and every
 * reduction order reproduces the reference's output bits.  Each function
 * cites the reference lines it follows.  FTZ|DAZ is set on every worker
 * thread exactly as the reference executor does (qppocr-kernels/src/par.rs:229-256,
 * qppocr-core/src/executor.rs:215).
 *
 * Threading (OpenMP) only distributes independent output elements; every
 * output element's arithmetic is fixed, so results do not depend on the
 * thread count.  Loops are written so gcc -O3 -mavx2 -mfma vectorises them
 * without changing any element's operation sequence (-ffp-contract=off keeps
 * every non-fma a*b+c as two roundings, as Rust does).  The GEMMs run whole
 * 6 x 16 tiles in the register form of the reference's AVX2 panel kernel
 * (x86.rs:134-444) and the edges in a scalar form; qpo_set_scalar(1) makes
 * every GEMM scalar, and the test suite checks the two give the same bits.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <immintrin.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QPO_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------ basics */

/* FTZ|DAZ on the calling thread: qppocr-kernels/src/par.rs:229-245. */
static inline void qpo_ftz(void) { _mm_setcsr(_mm_getcsr() | 0x8040); }

QPO_API int qpo_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

QPO_API void qpo_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* Forces the scalar form of the GEMMs and the softmax (for the
 * scalar-vs-AVX2 self-check of the test suite; both forms give the same
 * bits). */
static int g_scalar = 0;
QPO_API void qpo_set_scalar(int on) { g_scalar = on != 0; }

static inline float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* exp1: qppocr-kernels/src/activation.rs:28-47 (x86.rs:28-57 exp256_ps).
 * clamp +-88, k = rint(x*inv_ln2) (ties-even), two fnmadd range-reduction
 * steps, degree-6 Horner in fma, scale by 2^k built from exponent bits. */
static inline float exp1(float x) {
  const float LN2_HI = 0.6931472f;
  const float LN2_LO = -2.9802322e-8f;
  const float INV_LN2 = 1.442695f;
  x = fminf(x, 88.0f);
  x = fmaxf(x, -88.0f);
  float kf = rintf(x * INV_LN2);
  float r = fmaf(-kf, LN2_HI, x);
  r = fmaf(-kf, LN2_LO, r);
  float p = 1.0f / 720.0f;
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int32_t ki = (int32_t)kf + 127;
  return bits_f((uint32_t)ki << 23) * p;
}

/* erf1: qppocr-kernels/src/activation.rs:53-66 (x86.rs:63-77), A&S 7.1.26. */
static inline float erf1(float x) {
  float ax = bits_f(f_bits(x) & 0x7fffffffu);
  float t = 1.0f / fmaf(0.3275911f, ax, 1.0f);
  float p = 1.0614054f;
  p = fmaf(p, t, -1.453152027f);
  p = fmaf(p, t, 1.421413741f);
  p = fmaf(p, t, -0.284496736f);
  p = fmaf(p, t, 0.2548296f);
  p *= t;
  float e = exp1(ax * (0.0f - ax));
  float r = fmaf(-p, e, 1.0f);
  return bits_f(f_bits(r) | (f_bits(x) & 0x80000000u));
}

/* exp1 on eight lanes: the reference's exp256_ps (x86.rs:28-57) step for
 * step -- min/max clamp, round-to-nearest-even, two fnmadd steps, the same
 * Horner fmas, 2^k from exponent bits -- so each lane equals exp1. */
static inline __m256 exp1x8(__m256 x) {
  x = _mm256_min_ps(x, _mm256_set1_ps(88.0f));
  x = _mm256_max_ps(x, _mm256_set1_ps(-88.0f));
  const __m256 kf = _mm256_round_ps(_mm256_mul_ps(x, _mm256_set1_ps(1.442695f)),
                                    _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
  __m256 r = _mm256_fnmadd_ps(kf, _mm256_set1_ps(0.6931472f), x);
  r = _mm256_fnmadd_ps(kf, _mm256_set1_ps(-2.9802322e-8f), r);
  __m256 p = _mm256_set1_ps(1.0f / 720.0f);
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 120.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 24.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f / 6.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(0.5f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
  p = _mm256_fmadd_ps(p, r, _mm256_set1_ps(1.0f));
  const __m256i ki = _mm256_add_epi32(_mm256_cvtps_epi32(kf), _mm256_set1_epi32(127));
  return _mm256_mul_ps(_mm256_castsi256_ps(_mm256_slli_epi32(ki, 23)), p);
}

QPO_API float qpo_exp1(float x) { return exp1(x); }
QPO_API void qpo_exp1x8(const float* x, float* y) { _mm256_storeu_ps(y, exp1x8(_mm256_loadu_ps(x))); }
QPO_API float qpo_erf1(float x) { return erf1(x); }

/* ------------------------------------------------------------- activations */

/* act kinds shared with the HIP library's qph_act:
 *   0 none, 1 gelu(c1,c2,c3), 2 relu, 3 hardswish(alpha=c1, beta=c2),
 *   4 sigmoid.
 * The reference's Activation has only None/Gelu/Relu (activation.rs:75-95);
 * hardswish and sigmoid are separate graph nodes there (executor.rs:737-758,
 * 885-951) and are applied here with exactly those nodes' arithmetic. */

/* relu: activation.rs:232-239 (v > 0 ? v : 0, NaN -> 0). */
static inline float relu1(float v) { return v > 0.0f ? v : 0.0f; }

/* hardsigmoid: activation.rs:168-187 / x86.rs:795-824. */
static inline float hsig1(float x, float alpha, float beta) {
  float v = fmaf(x, alpha, beta);
  return v < 0.0f ? 0.0f : (v > 1.0f ? 1.0f : v);
}

/* hardswish as the graph composes it: HardSigmoid node then Mul node
 * (executor.rs:746-758 then elementwise.rs:197-205): y = x * hs(x). */
static inline float hswish1(float x, float alpha, float beta) { return x * hsig1(x, alpha, beta); }

/* sigmoid: activation.rs:196-201 / x86.rs:828-843. */
static inline float sigmoid1(float x) { return 1.0f / (1.0f + exp1(-x)); }

/* gelu: activation.rs:209-215 / x86.rs:82-85: (c3*x) * (erf1(x*inv_c1) + c2). */
static inline float gelu1(float v, float inv_c1, float c2, float c3) {
  return c3 * v * (erf1(v * inv_c1) + c2);
}

static inline float act1(float v, int kind, float c1, float c2, float c3, float inv_c1) {
  switch (kind) {
    case 1: return gelu1(v, inv_c1, c2, c3);
    case 2: return relu1(v);
    case 3: return hswish1(v, c1, c2);
    case 4: return sigmoid1(v);
    case 5: return hsig1(v, c1, c2);
    default: return v;
  }
}

/* Apply act (then optional residual add) to a contiguous range, the order of
 * gemm.rs:478-507 finish_res: act first, then += residual. */
static void act_res_range(float* y, const float* res, size_t n, int kind, float c1, float c2,
                          float c3) {
  float inv_c1 = 1.0f / c1;
  if (kind != 0)
    for (size_t i = 0; i < n; i++) y[i] = act1(y[i], kind, c1, c2, c3, inv_c1);
  if (res)
    for (size_t i = 0; i < n; i++) y[i] = y[i] + res[i];
}

QPO_API void qpo_relu_inplace(float* t, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; i++) t[i] = relu1(t[i]);
}

QPO_API void qpo_hardsigmoid(const float* x, float* y, int64_t n, float alpha, float beta) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; i++) y[i] = hsig1(x[i], alpha, beta);
}

QPO_API void qpo_sigmoid(const float* x, float* y, int64_t n) {
#pragma omp parallel
  {
    qpo_ftz();
#pragma omp for schedule(static)
    for (int64_t i = 0; i < n; i++) y[i] = sigmoid1(x[i]);
  }
}

QPO_API void qpo_gelu_inplace(float* t, int64_t n, float c1, float c2, float c3) {
  float inv_c1 = 1.0f / c1;
#pragma omp parallel
  {
    qpo_ftz();
#pragma omp for schedule(static)
    for (int64_t i = 0; i < n; i++) t[i] = gelu1(t[i], inv_c1, c2, c3);
  }
}

QPO_API void qpo_erf_inplace(float* t, int64_t n) {
  for (int64_t i = 0; i < n; i++) t[i] = erf1(t[i]);
}

/* clip: activation.rs:221-228 (comparison chain, NaN passes through). */
QPO_API void qpo_clip_inplace(float* t, int64_t n, float lo, float hi) {
  for (int64_t i = 0; i < n; i++) {
    float v = t[i];
    float m = v < lo ? lo : v;
    t[i] = hi < m ? hi : m;
  }
}

/* ----------------------------------------------------------------- softmax */

/* hsum8: activation.rs:313-316, the association of x86.rs:91-97. */
static inline float hsum8(const float* v) {
  float t0 = v[0] + v[4], t1 = v[1] + v[5], t2 = v[2] + v[6], t3 = v[3] + v[7];
  return (t0 + t1) + (t2 + t3);
}

/* One row: activation.rs:346-403 (scalar mirror of x86.rs:1091-1134). */
static void softmax_row(float* row, int64_t inner) {
  int64_t i = 0;
  float mx;
  if (inner >= 8) {
    float vmax[8];
    for (int j = 0; j < 8; j++) vmax[j] = row[j];
    while (i + 8 <= inner) {
      for (int j = 0; j < 8; j++)
        if (row[i + j] > vmax[j]) vmax[j] = row[i + j];
      i += 8;
    }
    mx = vmax[0];
    for (int j = 1; j < 8; j++)
      if (vmax[j] > mx) mx = vmax[j];
  } else {
    i = 1;
    mx = row[0];
  }
  for (; i < inner; i++)
    if (row[i] > mx) mx = row[i];
  float sum = 0.0f;
  int64_t i2 = 0;
  if (inner >= 8) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (g_scalar) {
      while (i2 + 8 <= inner) {
        for (int j = 0; j < 8; j++) {
          float ev = exp1(row[i2 + j] - mx);
          row[i2 + j] = ev;
          acc[j] += ev;
        }
        i2 += 8;
      }
    } else {
      /* the same eight lane chains as one vector (x86.rs:1091-1134) */
      const __m256 vm = _mm256_set1_ps(mx);
      __m256 va = _mm256_setzero_ps();
      while (i2 + 8 <= inner) {
        const __m256 ev = exp1x8(_mm256_sub_ps(_mm256_loadu_ps(row + i2), vm));
        _mm256_storeu_ps(row + i2, ev);
        va = _mm256_add_ps(va, ev);
        i2 += 8;
      }
      _mm256_storeu_ps(acc, va);
    }
    sum = hsum8(acc);
  }
  for (; i2 < inner; i2++) {
    row[i2] = exp1(row[i2] - mx);
    sum += row[i2];
  }
  float inv = 1.0f / sum;
  for (int64_t k = 0; k < inner; k++) row[k] *= inv;
}

/* softmax_last_dim: activation.rs:321-334. */
QPO_API void qpo_softmax_last_dim(float* t, int64_t rows, int64_t inner) {
#pragma omp parallel
  {
    qpo_ftz();
#pragma omp for schedule(static)
    for (int64_t r = 0; r < rows; r++) softmax_row(t + r * inner, inner);
  }
}

/* ---------------------------------------------------------------- sgemm */

/* Bias placement of the reference sgemm (gemm.rs:7-16):
 *   path 0 = panel kernel (gemm.rs:523-596, x86.rs:134-444): 32-column
 *     panels; rows in the M%4 tail of a panel narrower than 32 columns start
 *     the fma chain from the bias ("seeded"); everything else adds the bias
 *     after the chain.
 *   path 1 = m-rows kernel (gemm.rs:598-643, x86.rs:717-772), taken by the
 *     parallel sgemm when n <= 32 (np == 1): columns j >= n - n%32 are seeded.
 * Every element's chain is acc = fma(a[i][kk], b[kk][j], acc), kk ascending. */
static inline int bias_seeded(int path, int64_t i, int64_t j, int64_t m, int64_t n) {
  if (path == 1) return j >= n - n % 32;
  int64_t n0 = (j / 32) * 32;
  int64_t nn = n - n0 < 32 ? n - n0 : 32;
  return nn < 32 && i >= m - m % 4;
}

/* Path the reference sgemm/sgemm_res takes for a shape (gemm.rs:249-466):
 * serial (panel) when called from a parallel region or m*n*k < gemm_par_min
 * (2e5, par.rs:41-48); otherwise panel when np >= 2, m-rows when np == 1.
 * The baseline runs with more than one thread (par::threads() > 1). */
QPO_API int qpo_sgemm_path(int64_t m, int64_t n, int64_t k, int serial) {
  if (serial) return 0;
  if ((double)m * (double)n * (double)k < 2e5) return 0;
  return (n + 31) / 32 >= 2 ? 0 : 1;
}

/* C[M,N] (row stride ldc) = A[M,K] * B where B's row kk starts at
 * brow[kk] (implicit GEMM, gemm.rs:75-128) or at b + kk*ldb; bias per row.
 * Scalar form over rows [i0, i1) x columns [j0, j1): 4 rows x 32 columns at
 * a time, fma chains in registers. */
static void gemm_block_scalar(const float* a, int64_t lda, const float* b, int64_t ldb,
                              const float* const* brow, float* c, int64_t ldc, int64_t m,
                              int64_t n, int64_t k, const float* bias, int path, int64_t i0,
                              int64_t i1, int64_t j0, int64_t j1) {
  for (int64_t i = i0; i < i1; i += 4) {
    int64_t ni = i1 - i < 4 ? i1 - i : 4;
    for (int64_t jb = j0; jb < j1; jb += 32) {
      int64_t nj = j1 - jb < 32 ? j1 - jb : 32;
      float acc[4][32];
      for (int r = 0; r < 4; r++)
        for (int j = 0; j < 32; j++) {
          float s = 0.0f;
          if (bias && r < ni && j < nj && bias_seeded(path, i + r, jb + j, m, n)) s = bias[i + r];
          acc[r][j] = s;
        }
      for (int64_t kk = 0; kk < k; kk++) {
        const float* bp = brow ? brow[kk] + jb : b + kk * ldb + jb;
        float bv[32];
        for (int j = 0; j < 32; j++) bv[j] = j < nj ? bp[j] : 0.0f;
        for (int r = 0; r < 4; r++) {
          float av = r < ni ? a[(i + r) * lda + kk] : 0.0f;
          for (int j = 0; j < 32; j++) acc[r][j] = fmaf(av, bv[j], acc[r][j]);
        }
      }
      for (int r = 0; r < ni; r++)
        for (int j = 0; j < nj; j++) {
          float v = acc[r][j];
          if (bias && !bias_seeded(path, i + r, jb + j, m, n)) v = v + bias[i + r];
          c[(i + r) * ldc + jb + j] = v;
        }
    }
  }
}

/* One full 6 x 16 tile at (i, j0) in the register form of the reference's
 * AVX2 panel micro-kernel (x86.rs:134-444): twelve 8-wide accumulators,
 * the row's A term broadcast, k ascending, one fma per term -- each
 * element's chain is exactly the scalar form's. */
static void tile6x16(const float* a, int64_t lda, const float* b, int64_t ldb,
                     const float* const* brow, float* c, int64_t ldc, int64_t m, int64_t n,
                     int64_t k, const float* bias, int path, int64_t i, int64_t j0) {
  float init[6][16];
  for (int r = 0; r < 6; r++)
    for (int j = 0; j < 16; j++)
      init[r][j] = (bias && bias_seeded(path, i + r, j0 + j, m, n)) ? bias[i + r] : 0.0f;
  __m256 c0a = _mm256_loadu_ps(init[0]), c0b = _mm256_loadu_ps(init[0] + 8);
  __m256 c1a = _mm256_loadu_ps(init[1]), c1b = _mm256_loadu_ps(init[1] + 8);
  __m256 c2a = _mm256_loadu_ps(init[2]), c2b = _mm256_loadu_ps(init[2] + 8);
  __m256 c3a = _mm256_loadu_ps(init[3]), c3b = _mm256_loadu_ps(init[3] + 8);
  __m256 c4a = _mm256_loadu_ps(init[4]), c4b = _mm256_loadu_ps(init[4] + 8);
  __m256 c5a = _mm256_loadu_ps(init[5]), c5b = _mm256_loadu_ps(init[5] + 8);
  const float* a0 = a + i * lda;
  for (int64_t kk = 0; kk < k; kk++) {
    const float* bp = brow ? brow[kk] + j0 : b + kk * ldb + j0;
    const __m256 b0 = _mm256_loadu_ps(bp), b1 = _mm256_loadu_ps(bp + 8);
    __m256 av;
    av = _mm256_broadcast_ss(a0 + kk);
    c0a = _mm256_fmadd_ps(av, b0, c0a); c0b = _mm256_fmadd_ps(av, b1, c0b);
    av = _mm256_broadcast_ss(a0 + lda + kk);
    c1a = _mm256_fmadd_ps(av, b0, c1a); c1b = _mm256_fmadd_ps(av, b1, c1b);
    av = _mm256_broadcast_ss(a0 + 2 * lda + kk);
    c2a = _mm256_fmadd_ps(av, b0, c2a); c2b = _mm256_fmadd_ps(av, b1, c2b);
    av = _mm256_broadcast_ss(a0 + 3 * lda + kk);
    c3a = _mm256_fmadd_ps(av, b0, c3a); c3b = _mm256_fmadd_ps(av, b1, c3b);
    av = _mm256_broadcast_ss(a0 + 4 * lda + kk);
    c4a = _mm256_fmadd_ps(av, b0, c4a); c4b = _mm256_fmadd_ps(av, b1, c4b);
    av = _mm256_broadcast_ss(a0 + 5 * lda + kk);
    c5a = _mm256_fmadd_ps(av, b0, c5a); c5b = _mm256_fmadd_ps(av, b1, c5b);
  }
  float out[6][16];
  _mm256_storeu_ps(out[0], c0a); _mm256_storeu_ps(out[0] + 8, c0b);
  _mm256_storeu_ps(out[1], c1a); _mm256_storeu_ps(out[1] + 8, c1b);
  _mm256_storeu_ps(out[2], c2a); _mm256_storeu_ps(out[2] + 8, c2b);
  _mm256_storeu_ps(out[3], c3a); _mm256_storeu_ps(out[3] + 8, c3b);
  _mm256_storeu_ps(out[4], c4a); _mm256_storeu_ps(out[4] + 8, c4b);
  _mm256_storeu_ps(out[5], c5a); _mm256_storeu_ps(out[5] + 8, c5b);
  for (int r = 0; r < 6; r++)
    for (int j = 0; j < 16; j++) {
      float v = out[r][j];
      if (bias && !bias_seeded(path, i + r, j0 + j, m, n)) v = v + bias[i + r];
      c[(i + r) * ldc + j0 + j] = v;
    }
}

/* Rows [i0, i1) x columns [j0, j1) of the GEMM above: whole 6 x 16 tiles in
 * the AVX2 form, the edges in the scalar form (same bits either way). */
static void gemm_block(const float* a, int64_t lda, const float* b, int64_t ldb,
                       const float* const* brow, float* c, int64_t ldc, int64_t m, int64_t n,
                       int64_t k, const float* bias, int path, int64_t i0, int64_t i1,
                       int64_t j0, int64_t j1) {
  if (g_scalar) {
    gemm_block_scalar(a, lda, b, ldb, brow, c, ldc, m, n, k, bias, path, i0, i1, j0, j1);
    return;
  }
  const int64_t i6 = i0 + (i1 - i0) / 6 * 6, j16 = j0 + (j1 - j0) / 16 * 16;
  for (int64_t i = i0; i < i6; i += 6)
    for (int64_t j = j0; j < j16; j += 16)
      tile6x16(a, lda, b, ldb, brow, c, ldc, m, n, k, bias, path, i, j);
  if (j16 < j1 && i6 > i0)
    gemm_block_scalar(a, lda, b, ldb, brow, c, ldc, m, n, k, bias, path, i0, i6, j16, j1);
  if (i6 < i1)
    gemm_block_scalar(a, lda, b, ldb, brow, c, ldc, m, n, k, bias, path, i6, i1, j0, j1);
}

/* sgemm / sgemm_res: gemm.rs:37-70, 223-507.  Result = chain (+bias by the
 * placement rule), then act, then += residual (residual has C's layout). */
QPO_API void qpo_sgemm(const float* a, const float* b, float* c, int64_t m, int64_t n, int64_t k,
                       int64_t ldc, const float* bias, int act, float c1, float c2, float c3,
                       const float* residual, int serial) {
  if (m == 0 || n == 0 || k == 0) return;
  int path = qpo_sgemm_path(m, n, k, serial);
  /* blocks of 48 rows x 128 columns: the B block stays in L2 across the
   * block's eight 6-row tiles */
  int64_t mblocks = (m + 47) / 48;
  int64_t nblocks = (n + 127) / 128;
#pragma omp parallel
  {
    qpo_ftz();
#pragma omp for schedule(dynamic, 1) collapse(2)
    for (int64_t nb = 0; nb < nblocks; nb++)
      for (int64_t mb = 0; mb < mblocks; mb++) {
        int64_t i0 = mb * 48, i1 = i0 + 48 < m ? i0 + 48 : m;
        int64_t j0 = nb * 128, j1 = j0 + 128 < n ? j0 + 128 : n;
        gemm_block(a, k, b, n, NULL, c, ldc, m, n, k, bias, path, i0, i1, j0, j1);
      }
#pragma omp for schedule(static)
    for (int64_t i = 0; i < m; i++)
      act_res_range(c + i * ldc, residual ? residual + i * ldc : NULL, (size_t)n, act, c1, c2, c3);
  }
}

/* ------------------------------------------------------------------ conv2d */

/* conv2d_out_shape: conv.rs:146-156. Returns 0 on success. */
QPO_API int qpo_conv2d_out_shape(const int64_t* xs, const int64_t* ws, const int64_t* p,
                                 int64_t* ys) {
  /* p = {sh, sw, ph, pw, peh, pew, dh, dw, group} (ConvParams, conv.rs:124-143) */
  int64_t n = xs[0], c = xs[1], h = xs[2], w = xs[3];
  int64_t m = ws[0], cg = ws[1], kh = ws[2], kw = ws[3];
  if (p[6] != 1 || p[7] != 1) return -1;
  if (p[8] * cg != c || m % p[8] != 0) return -2;
  int64_t oh = (h + p[2] + p[4] - kh) / p[0] + 1;
  int64_t ow = (w + p[3] + p[5] - kw) / p[1] + 1;
  if (oh <= 0 || ow <= 0) return -3;
  ys[0] = n; ys[1] = m; ys[2] = oh; ys[3] = ow;
  return 0;
}

/* conv2d_res_into: conv.rs:222-715.  Branches:
 *   1x1 s1 g1 -> sgemm (conv.rs:264-460): per batch item W[M,C] x X[C,HW];
 *   depthwise (g > 1, C/g == 1) -> padded-plane direct conv (conv.rs:461-505,
 *     x86.rs:994-1060): acc = fma(w, x, acc) over ky then kx from 0, + bias;
 *   general, x-stride 1 or 2 -> implicit GEMM per output row
 *     (conv.rs:506-637): K order ch -> ky -> kx, N = ow, panel bias
 *     placement, act on each row GEMM;
 *   general, other x-strides -> im2col tiles (conv.rs:639-661): same K order,
 *     N = rows * ow per tile.
 * act then residual (conv.rs:673-713, gemm.rs:478-507). */
QPO_API int qpo_conv2d(const float* x, const int64_t* xs, const float* wt, const int64_t* ws,
                       const float* bias, const int64_t* p, int act, float c1, float c2, float c3,
                       const float* residual, float* y, int64_t* ys_out) {
  int64_t ys[4];
  int rc = qpo_conv2d_out_shape(xs, ws, p, ys);
  if (rc) return rc;
  if (ys_out) memcpy(ys_out, ys, sizeof ys);
  const int64_t n = xs[0], c = xs[1], h = xs[2], wd = xs[3];
  const int64_t m = ws[0], cg = ws[1], kh = ws[2], kw = ws[3];
  const int64_t sh = p[0], sw = p[1], ph = p[2], pw = p[3], peh = p[4], pew = p[5], g = p[8];
  const int64_t oh = ys[2], ow = ys[3], ohw = oh * ow;
  const int depthwise = g > 1 && cg == 1;
  const float inv_c1 = 1.0f / c1;

  /* the reference's 1x1 test (conv.rs:264) does not look at the padding; its
   * GEMM reads X as [C][oh*ow], which is the input only without padding, so a
   * padded 1x1 conv is taken as the ordinary conv it is (general branch) */
  if (g == 1 && kh == 1 && kw == 1 && sh == 1 && sw == 1 && ph == 0 && pw == 0 && peh == 0 &&
      pew == 0) {
    /* 1x1: conv.rs:370-460.  N > 1 with threads > 1 runs sgemm_serial_res
     * per chunk (panel path); N == 1 runs sgemm_res (parallel rules). */
    int serial = n > 1;
    for (int64_t bn = 0; bn < n; bn++)
      qpo_sgemm(wt, x + bn * c * ohw, y + bn * m * ohw, m, ohw, c, ohw, bias, act, c1, c2, c3,
                residual ? residual + bn * m * ohw : NULL, serial);
    return 0;
  }

  /* depthwise with one output per channel (conv.rs:461-505 indexes the
   * weight by input channel); a channel multiplier goes the general way */
  if (depthwise && m == c) {
    const int64_t pheight = ph + h + peh;
    const int64_t pwidth = pw + wd + pew;
#pragma omp parallel
    {
      qpo_ftz();
      float* pad = (float*)malloc(sizeof(float) * (size_t)(pheight * pwidth));
#pragma omp for schedule(dynamic, 1)
      for (int64_t u = 0; u < n * c; u++) {
        int64_t bn = u / c, ch = u % c;
        const float* xch = x + (bn * c + ch) * h * wd;
        const float* wc = wt + ch * kh * kw;
        float bv = bias ? bias[ch] : 0.0f;
        /* pad_channel: conv.rs:78-119 */
        memset(pad, 0, sizeof(float) * (size_t)(pheight * pwidth));
        for (int64_t yy = 0; yy < h; yy++)
          memcpy(pad + (ph + yy) * pwidth + pw, xch + yy * wd, sizeof(float) * (size_t)wd);
        float* yc = y + (bn * m + ch) * ohw;
        for (int64_t oy = 0; oy < oh; oy++) {
          const float* base = pad + oy * sh * pwidth;
          for (int64_t ox = 0; ox < ow; ox++) {
            float acc = 0.0f;
            for (int64_t ky = 0; ky < kh; ky++) {
              const float* row = base + ky * pwidth;
              for (int64_t kx = 0; kx < kw; kx++) acc = fmaf(wc[ky * kw + kx], row[ox * sw + kx], acc);
            }
            yc[oy * ow + ox] = acc + bv;
          }
        }
        /* conv.rs:673-677 act (never fused for group > 1 by the optimizer,
         * applied if asked), then conv.rs:701-713 residual. */
        if (act != 0)
          for (int64_t i = 0; i < ohw; i++) yc[i] = act1(yc[i], act, c1, c2, c3, inv_c1);
        if (residual) {
          const float* rs = residual + (bn * m + ch) * ohw;
          for (int64_t i = 0; i < ohw; i++) yc[i] = yc[i] + rs[i];
        }
      }
      free(pad);
    }
    return 0;
  }

  const int64_t mg = m / g, kk = cg * kh * kw;
  if (sw != 1 && sw != 2) {
    /* im2col branch (conv.rs:639-661, gemm.rs:771-867): tiles of `tile`
     * output rows, each one sgemm_serial_res over the materialised patch
     * matrix [kk][rows * ow] (N = rows * ow, so the panel bias rule runs over
     * the tile's flattened columns).  The tile height is the reference's on
     * one thread (conv.rs:508-524 with par::threads() == 1):
     * min(oh, max(1, 2^19 / (kk * ow))). */
    int64_t tile = ((int64_t)1 << 19) / (kk * ow > 1 ? kk * ow : 1);
    if (tile < 1) tile = 1;
    if (tile > oh) tile = oh;
    const int64_t ntiles = (oh + tile - 1) / tile;
#pragma omp parallel
    {
      qpo_ftz();
      float* cols = (float*)malloc(sizeof(float) * (size_t)(kk * tile * ow));
#pragma omp for schedule(dynamic, 1) collapse(3)
      for (int64_t bn = 0; bn < n; bn++)
        for (int64_t gi = 0; gi < g; gi++)
          for (int64_t t = 0; t < ntiles; t++) {
            const int64_t oy0 = t * tile, rows = oh - oy0 < tile ? oh - oy0 : tile;
            const int64_t nn = rows * ow;
            const float* xg = x + (bn * c + gi * cg) * h * wd;
            /* im2col: row k = (ch, ky, kx), column (r, ox) */
            for (int64_t ch = 0; ch < cg; ch++)
              for (int64_t ky = 0; ky < kh; ky++)
                for (int64_t kx = 0; kx < kw; kx++) {
                  float* dst = cols + ((ch * kh + ky) * kw + kx) * nn;
                  for (int64_t r = 0; r < rows; r++) {
                    const int64_t iy = (oy0 + r) * sh - ph + ky;
                    for (int64_t ox = 0; ox < ow; ox++) {
                      const int64_t ix = ox * sw - pw + kx;
                      dst[r * ow + ox] = (iy >= 0 && iy < h && ix >= 0 && ix < wd)
                                             ? xg[(ch * h + iy) * wd + ix]
                                             : 0.0f;
                    }
                  }
                }
            float* yt = y + (bn * m + gi * mg) * ohw + oy0 * ow;
            const float* bg = bias ? bias + gi * mg : NULL;
            gemm_block(wt + gi * mg * kk, kk, cols, nn, NULL, yt, ohw, mg, nn, kk, bg, 0, 0, mg, 0,
                       nn);
            if (act != 0)
              for (int64_t r = 0; r < mg; r++)
                for (int64_t i = 0; i < nn; i++)
                  yt[r * ohw + i] = act1(yt[r * ohw + i], act, c1, c2, c3, inv_c1);
          }
      free(cols);
    }
    if (residual) {
      int64_t total = n * m * ohw;
#pragma omp parallel for schedule(static)
      for (int64_t i = 0; i < total; i++) y[i] = y[i] + residual[i];
    }
    return 0;
  }

  /* general grouped conv, strides 1 and 2 along x: implicit GEMM, one output
   * row per sgemm call. */
  const int64_t pwidth = (ow - 1) * sw + kw;
#pragma omp parallel
  {
    qpo_ftz();
    float* slab = (float*)malloc(sizeof(float) * (size_t)(cg * kh * pwidth));
    const float** brow = (const float**)malloc(sizeof(float*) * (size_t)kk);
    float* patch = (float*)malloc(sizeof(float) * (size_t)(kk * ow));
#pragma omp for schedule(dynamic, 1) collapse(3)
    for (int64_t bn = 0; bn < n; bn++)
      for (int64_t gi = 0; gi < g; gi++)
        for (int64_t oy = 0; oy < oh; oy++) {
          const float* xg = x + (bn * c + gi * cg) * h * wd;
          /* zero-padded slab of the kh input rows this output row reads */
          for (int64_t ch = 0; ch < cg; ch++)
            for (int64_t ky = 0; ky < kh; ky++) {
              float* dst = slab + (ch * kh + ky) * pwidth;
              int64_t iy = oy * sh - ph + ky;
              for (int64_t xx = 0; xx < pwidth; xx++) {
                int64_t ix = xx - pw;
                dst[xx] = (iy >= 0 && iy < h && ix >= 0 && ix < wd) ? xg[(ch * h + iy) * wd + ix] : 0.0f;
              }
            }
          /* B row k = (ch, ky, kx): element ox = slab[ch][ky][ox*sw + kx] */
          for (int64_t ch = 0; ch < cg; ch++)
            for (int64_t ky = 0; ky < kh; ky++)
              for (int64_t kx = 0; kx < kw; kx++) {
                int64_t kidx = (ch * kh + ky) * kw + kx;
                const float* src = slab + (ch * kh + ky) * pwidth + kx;
                float* dst = patch + kidx * ow;
                for (int64_t ox = 0; ox < ow; ox++) dst[ox] = src[ox * sw];
                brow[kidx] = dst;
              }
          float* yrow = y + (bn * m + gi * mg) * ohw + oy * ow;
          const float* bg = bias ? bias + gi * mg : NULL;
          gemm_block(wt + gi * mg * kk, kk, NULL, 0, brow, yrow, ohw, mg, ow, kk, bg, 0, 0, mg, 0, ow);
          for (int64_t r = 0; r < mg; r++) {
            float* yr = yrow + r * ohw;
            if (act != 0)
              for (int64_t i = 0; i < ow; i++) yr[i] = act1(yr[i], act, c1, c2, c3, inv_c1);
          }
        }
    free(slab);
    free((void*)brow);
    free(patch);
  }
  if (residual) {
    int64_t total = n * m * ohw;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < total; i++) y[i] = y[i] + residual[i];
  }
  return 0;
}

/* --------------------------------------------------------- convtranspose */

/* convtranspose2d, 2x2 s2 p0 only, no bias: conv.rs:730-838 (x86.rs:1065-1085).
 * w is ONNX [Ci, Co, 2, 2]; out(2iy+ky, 2ix+kx) = chain over ci ascending of
 * fma(x, w, acc) from 0. */
QPO_API int qpo_convtranspose2x2(const float* x, const int64_t* xs, const float* w,
                                 const int64_t* ws, float* y) {
  int64_t n = xs[0], c = xs[1], h = xs[2], wd = xs[3];
  int64_t cin = ws[0], m = ws[1];
  if (cin != c || ws[2] != 2 || ws[3] != 2) return -1;
  int64_t oh = 2 * h, ow = 2 * wd;
#pragma omp parallel
  {
    qpo_ftz();
#pragma omp for schedule(static) collapse(3)
    for (int64_t bn = 0; bn < n; bn++)
      for (int64_t co = 0; co < m; co++)
        for (int64_t iy = 0; iy < h; iy++) {
          const float* xn = x + bn * c * h * wd;
          for (int ky = 0; ky < 2; ky++) {
            float* orow = y + ((bn * m + co) * oh + 2 * iy + ky) * ow;
            for (int64_t j = 0; j < wd; j++) {
              float a0 = 0.0f, a1 = 0.0f;
              for (int64_t ch = 0; ch < c; ch++) {
                float xv = xn[(ch * h + iy) * wd + j];
                const float* wc = w + ((ch * m + co) * 4 + ky * 2);
                a0 = fmaf(xv, wc[0], a0);
                a1 = fmaf(xv, wc[1], a1);
              }
              orow[2 * j] = a0;
              orow[2 * j + 1] = a1;
            }
          }
        }
  }
  return 0;
}

/* ------------------------------------------------------------------ resize */

/* resize_nearest: resize.rs:26-57: iy = min((int)((float)oy * H / oh), H-1). */
QPO_API void qpo_resize_nearest(const float* x, int64_t nc, int64_t h, int64_t w, int64_t oh,
                                int64_t ow, float* y) {
#pragma omp parallel for schedule(static)
  for (int64_t p = 0; p < nc; p++) {
    for (int64_t oy = 0; oy < oh; oy++) {
      int64_t iy = (int64_t)((float)oy * (float)h / (float)oh);
      if (iy > h - 1) iy = h - 1;
      for (int64_t ox = 0; ox < ow; ox++) {
        int64_t ix = (int64_t)((float)ox * (float)w / (float)ow);
        if (ix > w - 1) ix = w - 1;
        y[(p * oh + oy) * ow + ox] = x[(p * h + iy) * w + ix];
      }
    }
  }
}

/* ------------------------------------------------------- elementwise, reduce */

/* Binary ops, same-shape flat pass: elementwise.rs:197-205 (x86.rs:867-892).
 * op: 0 add, 1 sub, 2 mul, 3 div, 4 pow (powf, elementwise.rs:48-56). */
static inline float binop(int op, float a, float b) {
  switch (op) {
    case 0: return a + b;
    case 1: return a - b;
    case 2: return a * b;
    case 3: return a / b;
    default: return powf(a, b);
  }
}

QPO_API void qpo_binary_flat(float* a, const float* b, int64_t n, int op) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; i++) a[i] = binop(op, a[i], b[i]);
}

/* y = x op s (scalar_first 0) or s op x: binary_op's one-element fast path
 * (elementwise.rs:350-363; binary_scalar_bcast_scalar elementwise.rs:635-650,
 * x86.rs:1241-1278), one IEEE op an element. */
QPO_API void qpo_binary_scalar(const float* x, int64_t n, float s, int op, int scalar_first,
                               float* y) {
#pragma omp parallel
  {
    qpo_ftz();
#pragma omp for schedule(static)
    for (int64_t i = 0; i < n; i++) y[i] = scalar_first ? binop(op, s, x[i]) : binop(op, x[i], s);
  }
}

/* a[R,C] op= b broadcast: bmode 0 = b[R] per row (a [R,C] op [R,1]),
 * 1 = b[C] per column (a [R,C] op [C]), 2 = scalar b[0].  The run paths of
 * binary_op_inplace (elementwise.rs:207-298, x86.rs:895-942). */
QPO_API void qpo_binary_bcast(float* a, const float* b, int64_t rows, int64_t cols, int op,
                              int bmode) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; r++)
    for (int64_t j = 0; j < cols; j++) {
      float bv = bmode == 0 ? b[r] : (bmode == 1 ? b[j] : b[0]);
      a[r * cols + j] = binop(op, a[r * cols + j], bv);
    }
}

/* reduce_mean over the last axis: shape.rs:510-560 (f64 accumulation,
 * ascending, then (s / mid) rounded to f32). */
QPO_API void qpo_reduce_mean_last(const float* x, int64_t rows, int64_t cols, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; r++) {
    double s = 0.0;
    for (int64_t j = 0; j < cols; j++) s += (double)x[r * cols + j];
    out[r] = (float)(s / (double)cols);
  }
}

QPO_API void qpo_sqrt_inplace(float* t, int64_t n) {
  for (int64_t i = 0; i < n; i++) t[i] = sqrtf(t[i]);
}

/* LayerNorm exactly as the exported graph runs it on the CPU executor
 * (ReduceMean -> Sub -> Pow(2) -> ReduceMean -> Add(eps) -> Sqrt -> Div ->
 * Mul(gamma) -> Add(beta)), each node rounding to f32:
 * shape.rs:510-560, elementwise.rs:185-298, activation.rs:449-459.
 * Pow(d, 2) is the correctly rounded square d*d, as the reference's GPU plan
 * lowers it (qppocr-gpu/src/plan.rs:2319-2330, shaders/n_elem.comp:61); the
 * CPU executor calls the platform libm powf (elementwise.rs:32-34, "ulp-level
 * differences across implementations"), which under glibc 2.35 returns the
 * neighbouring float for about 0.07% of inputs. */
QPO_API void qpo_layernorm_chain(const float* x, const float* gamma, const float* beta, float eps,
                                 int64_t rows, int64_t cols, float* y) {
#pragma omp parallel
  {
    qpo_ftz();
    float* d = (float*)malloc(sizeof(float) * (size_t)cols);
#pragma omp for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
      const float* xr = x + r * cols;
      double s = 0.0;
      for (int64_t j = 0; j < cols; j++) s += (double)xr[j];
      float mu = (float)(s / (double)cols);
      for (int64_t j = 0; j < cols; j++) d[j] = xr[j] - mu;
      double s2 = 0.0;
      for (int64_t j = 0; j < cols; j++) s2 += (double)(d[j] * d[j]);
      float var = (float)(s2 / (double)cols);
      float sd = sqrtf(var + eps);
      float* yr = y + r * cols;
      for (int64_t j = 0; j < cols; j++) {
        float v = d[j] / sd;
        v = v * gamma[j];
        yr[j] = v + beta[j];
      }
    }
    free(d);
  }
}

/* ------------------------------------------------------------------ matmul */

/* Batched matmul without bias: shape.rs:568-698.  Every path (folded sgemm,
 * per-batch sgemm, row outer product) computes each element as the chain
 * c = fma(a[kk], b[kk][j], c) from 0, kk ascending, so one loop serves.
 * a: [batch, m, k] (abatch 1 = shared), b: [batch, k, n] (bbatch 1 = shared). */
QPO_API void qpo_matmul(const float* a, const float* b, float* out, int64_t batch, int64_t m,
                        int64_t k, int64_t n, int a_shared, int b_shared) {
  /* every element: c = 0; c = fma(a_kk, b_kk_j, c) for kk ascending (no
   * bias), in blocks of 48 rows x 128 columns per batch item */
  const int64_t mblocks = (m + 47) / 48, nblocks = (n + 127) / 128;
#pragma omp parallel
  {
    qpo_ftz();
#pragma omp for schedule(dynamic, 1) collapse(3)
    for (int64_t bi = 0; bi < batch; bi++)
      for (int64_t nb = 0; nb < nblocks; nb++)
        for (int64_t mb = 0; mb < mblocks; mb++) {
          const float* ab = a + (a_shared ? 0 : bi * m * k);
          const float* bb = b + (b_shared ? 0 : bi * k * n);
          int64_t i0 = mb * 48, i1 = i0 + 48 < m ? i0 + 48 : m;
          int64_t j0 = nb * 128, j1 = j0 + 128 < n ? j0 + 128 : n;
          gemm_block(ab, k, bb, n, NULL, out + bi * m * n, n, m, n, k, NULL, 0, i0, i1, j0, j1);
        }
  }
}

/* --------------------------------------------------------------------- CTC */

/* Per-row argmax, first strict maximum (ties -> lowest index):
 * qppocr-core/src/pipeline/rec.rs:46-54.  pairs[2t] = value,
 * pairs[2t+1] = index as f32 bits (rec.rs:82-90, device.rs:160-165). */
QPO_API void qpo_ctc_argmax(const float* probs, int64_t rows, int64_t cols, float* pairs) {
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < rows; t++) {
    const float* row = probs + t * cols;
    int64_t best = 0;
    float bestv = row[0];
    for (int64_t c = 1; c < cols; c++)
      if (row[c] > bestv) {
        bestv = row[c];
        best = c;
      }
    uint32_t ib = (uint32_t)best;
    pairs[2 * t] = bestv;
    memcpy(&pairs[2 * t + 1], &ib, 4);
  }
}

/* Greedy CTC collapse over pairs: rec.rs:82-115 (emit when idx != 0 and
 * idx != previous; confidence = f64 mean of emitted values).  Returns the
 * number of emitted ids written to ids (capacity t_len). */
QPO_API int64_t qpo_ctc_collapse(const float* pairs, int64_t t_len, int32_t* ids, float* conf) {
  int64_t prev = -1, cnt = 0;
  double cs = 0.0;
  for (int64_t t = 0; t < t_len; t++) {
    uint32_t ib;
    memcpy(&ib, &pairs[2 * t + 1], 4);
    int64_t b = (int64_t)ib;
    if (b != 0 && b != prev) {
      ids[cnt++] = (int32_t)b;
      cs += (double)pairs[2 * t];
    }
    prev = b;
  }
  if (conf) *conf = cnt > 0 ? (float)(cs / (double)cnt) : 0.0f;
  return cnt;
}

/* ------------------------------------------- pooling, SE gate, bilinear */

/* global_avg_pool: pool2d.rs:10-29 -- per (n, c) plane, f64 sum in
 * ascending order, (sum / plane) as f32: reduce_mean over the plane. */
QPO_API void qpo_global_avg_pool(const float* x, int64_t nc, int64_t plane, float* out) {
  qpo_reduce_mean_last(x, nc, plane, out);
}

/* mul_add_scale: elementwise.rs:134-179 -- out = f * gate[plane % c] + r,
 * the Mul and the Add each rounded (no fma). */
QPO_API void qpo_mul_add_scale(const float* f, const float* gate, const float* r, float* out,
                               int64_t c, int64_t hw, int64_t total) {
  const int64_t planes = total / hw;
#pragma omp parallel for schedule(static)
  for (int64_t p = 0; p < planes; p++) {
    const float g = gate[p % c];
    for (int64_t i = 0; i < hw; i++) out[p * hw + i] = f[p * hw + i] * g + r[p * hw + i];
  }
}

/* Rust's f32::max (IEEE maxNum: a NaN operand yields the other). */
static inline float maxnum(float a, float b) { return fmaxf(a, b); }

/* pool2d_out_hw: pool2d.rs:34-49. */
QPO_API void qpo_pool2d_out_hw(int64_t h, int64_t w, int64_t kh, int64_t kw, int64_t sh,
                               int64_t sw, int64_t ph, int64_t pw, int64_t peh, int64_t pew,
                               int64_t* oh, int64_t* ow) {
  const int64_t hh = h + ph + peh, ww = w + pw + pew;
  *oh = (hh > kh ? hh - kh : 0) / sh + 1;
  *ow = (ww > kw ? ww - kw : 0) / sw + 1;
}

/* pool2d_into: pool2d.rs:94-236.
 *   2x2 s1 SAME_UPPER max (ph = pw = 0, peh = pew = 1, oh = h, ow = w):
 *     vm[j] = max(r0[j], r1[j]) (r1 = next row, absent on the last row),
 *     vm[w] = -f32::MAX, out[j] = max(vm[j], vm[j + 1])
 *     (pool2x2_row_scalar, pool2d.rs:242-259);
 *   otherwise per output: acc = -3.4e38 (max) or 0 (avg), taps ky outer, kx
 *     inner, out-of-range taps skipped; max: v > acc ? v : acc; avg:
 *     acc + v, then acc / (kh * kw) (the divisor counts padding). */
QPO_API void qpo_pool2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w, int64_t kh,
                        int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t peh,
                        int64_t pew, int max_pool, float* y) {
  int64_t oh, ow;
  qpo_pool2d_out_hw(h, w, kh, kw, sh, sw, ph, pw, peh, pew, &oh, &ow);
  const int special = max_pool && kh == 2 && kw == 2 && sh == 1 && sw == 1 && ph == 0 &&
                      pw == 0 && peh == 1 && pew == 1 && oh == h && ow == w;
#pragma omp parallel
  {
    float* vm = (float*)malloc(sizeof(float) * (size_t)(w + 1));
#pragma omp for schedule(static)
    for (int64_t p = 0; p < n * c; p++) {
      const float* xp = x + p * h * w;
      float* yp = y + p * oh * ow;
      if (special) {
        for (int64_t oy = 0; oy < oh; oy++) {
          const float* r0 = xp + oy * w;
          const float* r1 = oy + 1 < h ? r0 + w : NULL;
          for (int64_t j = 0; j < w; j++) vm[j] = r1 ? maxnum(r0[j], r1[j]) : r0[j];
          vm[w] = -3.40282347e38f;
          for (int64_t j = 0; j < w; j++) yp[oy * ow + j] = maxnum(vm[j], vm[j + 1]);
        }
        continue;
      }
      for (int64_t oy = 0; oy < oh; oy++)
        for (int64_t ox = 0; ox < ow; ox++) {
          float acc = max_pool ? -3.4e38f : 0.0f;
          for (int64_t ky = 0; ky < kh; ky++) {
            const int64_t iy = oy * sh - ph + ky;
            if (iy < 0 || iy >= h) continue;
            for (int64_t kx = 0; kx < kw; kx++) {
              const int64_t ix = ox * sw - pw + kx;
              if (ix < 0 || ix >= w) continue;
              const float v = xp[iy * w + ix];
              acc = max_pool ? (v > acc ? v : acc) : acc + v;
            }
          }
          yp[oy * ow + ox] = max_pool ? acc : acc / (float)(kh * kw);
        }
    }
    free(vm);
  }
}

/* resize_bilinear_into: resize.rs:60-142 with bilinear_row_scalar
 * (resize.rs:252-273).  Source coordinate per output index i (f32):
 * align_corners: i * (H - 1) / (oh - 1); else max(0, (i + 0.5) * H / oh - 0.5);
 * base = clamp(floor(v), 0, H - 1), next = min(base + 1, H - 1),
 * frac = v - base.  Value: t = r0[i0] * (1 - lx) * (1 - ly);
 * t = fma(r0[i1] * lx, 1 - ly, t); t = fma(r1[i0] * (1 - lx), ly, t);
 * out = fma(r1[i1] * lx, ly, t). */
static void bilinear_map(int64_t n_out, int64_t n_in, int align, int64_t* i0, int64_t* i1,
                         float* f) {
  for (int64_t i = 0; i < n_out; i++) {
    float v;
    if (align && n_out > 1)
      v = (float)i * (float)(n_in - 1) / (float)(n_out - 1);
    else {
      v = ((float)i + 0.5f) * (float)n_in / (float)n_out - 0.5f;
      v = v > 0.0f ? v : 0.0f;
    }
    int64_t b = (int64_t)floorf(v);
    if (b < 0) b = 0;
    if (b > n_in - 1) b = n_in - 1;
    i0[i] = b;
    i1[i] = b + 1 < n_in - 1 ? b + 1 : n_in - 1;
    f[i] = v - (float)b;
  }
}

QPO_API void qpo_resize_bilinear(const float* x, int64_t nc, int64_t h, int64_t w, int64_t oh,
                                 int64_t ow, int align, float* y) {
  int64_t* iy0 = (int64_t*)malloc(sizeof(int64_t) * (size_t)oh);
  int64_t* iy1 = (int64_t*)malloc(sizeof(int64_t) * (size_t)oh);
  float* fy = (float*)malloc(sizeof(float) * (size_t)oh);
  int64_t* ix0 = (int64_t*)malloc(sizeof(int64_t) * (size_t)ow);
  int64_t* ix1 = (int64_t*)malloc(sizeof(int64_t) * (size_t)ow);
  float* fx = (float*)malloc(sizeof(float) * (size_t)ow);
  bilinear_map(oh, h, align, iy0, iy1, fy);
  bilinear_map(ow, w, align, ix0, ix1, fx);
#pragma omp parallel for schedule(static)
  for (int64_t p = 0; p < nc; p++)
    for (int64_t oy = 0; oy < oh; oy++) {
      const float* r0 = x + (p * h + iy0[oy]) * w;
      const float* r1 = x + (p * h + iy1[oy]) * w;
      const float ly = fy[oy];
      for (int64_t ox = 0; ox < ow; ox++) {
        const float lx = fx[ox];
        const int64_t a = ix0[ox], b = ix1[ox];
        float t = r0[a] * (1.0f - lx) * (1.0f - ly);
        t = fmaf(r0[b] * lx, 1.0f - ly, t);
        t = fmaf(r1[a] * (1.0f - lx), ly, t);
        y[(p * oh + oy) * ow + ox] = fmaf(r1[b] * lx, ly, t);
      }
    }
  free(iy0); free(iy1); free(fy); free(ix0); free(ix1); free(fx);
}

/* Rank-4 transpose: y[i_perm] = x[i] with y's dim d = x's dim perm[d]. */
QPO_API void qpo_transpose4(const float* x, const int64_t* xs, const int64_t* perm, float* y) {
  int64_t ys[4], xst[4];
  xst[3] = 1;
  for (int d = 2; d >= 0; d--) xst[d] = xst[d + 1] * xs[d + 1];
  for (int d = 0; d < 4; d++) ys[d] = xs[perm[d]];
  const int64_t total = xs[0] * xs[1] * xs[2] * xs[3];
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < total; o++) {
    int64_t r = o, src = 0;
    for (int d = 3; d >= 0; d--) {
      const int64_t i = r % ys[d];
      r /= ys[d];
      src += i * xst[perm[d]];
    }
    y[o] = x[src];
  }
}

/* -------------------------------------- steps either side of the path */

/* det input: u8 RGB (h x w x 3, interleaved) -> NCHW f32,
 * v = u8 * (1 / 255) then (v - 0.5) * (1 / 0.5) (engine.rs:959-982). */
QPO_API void qpo_det_normalize(const uint8_t* rgb, int64_t h, int64_t w, float* out) {
  const float scale = 1.0f / 255.0f, mean = 0.5f, istd = 1.0f / 0.5f;
#pragma omp parallel for schedule(static)
  for (int64_t y = 0; y < h; y++)
    for (int64_t c = 0; c < 3; c++)
      for (int64_t x = 0; x < w; x++) {
        const float v = (float)rgb[(y * w + x) * 3 + c] * scale;
        out[(c * h + y) * w + x] = (v - mean) * istd;
      }
}

/* resize_bilinear_rgb_u8: resize.rs:153-209 (= pipeline/image.rs
 * resize_bilinear_img for 3 channels): half-pixel map with (v as usize)
 * truncation, the same two-multiply-then-fma weighting, then
 * (val + 0.5).clamp(0, 255) as u8. */
QPO_API void qpo_resize_bilinear_rgb_u8(const uint8_t* src, int64_t sw, int64_t sh, uint8_t* dst,
                                        int64_t dw, int64_t dh) {
  const float sx = (float)sw / (float)dw, sy = (float)sh / (float)dh;
  int64_t* x0 = (int64_t*)malloc(sizeof(int64_t) * (size_t)dw);
  int64_t* x1 = (int64_t*)malloc(sizeof(int64_t) * (size_t)dw);
  float* fx = (float*)malloc(sizeof(float) * (size_t)dw);
  for (int64_t x = 0; x < dw; x++) {
    float v = ((float)x + 0.5f) * sx - 0.5f;
    v = v > 0.0f ? v : 0.0f;
    int64_t i0 = (int64_t)v;
    if (i0 > sw - 1) i0 = sw - 1;
    x0[x] = i0;
    x1[x] = i0 + 1 < sw - 1 ? i0 + 1 : sw - 1;
    fx[x] = v - (float)i0;
  }
#pragma omp parallel for schedule(static)
  for (int64_t y = 0; y < dh; y++) {
    float v = ((float)y + 0.5f) * sy - 0.5f;
    v = v > 0.0f ? v : 0.0f;
    int64_t j0 = (int64_t)v;
    if (j0 > sh - 1) j0 = sh - 1;
    const int64_t j1 = j0 + 1 < sh - 1 ? j0 + 1 : sh - 1;
    const float fy = v - (float)j0;
    const uint8_t* r0 = src + j0 * sw * 3;
    const uint8_t* r1 = src + j1 * sw * 3;
    for (int64_t x = 0; x < dw; x++) {
      const int64_t a = x0[x] * 3, b = x1[x] * 3;
      const float lx = fx[x];
      for (int ch = 0; ch < 3; ch++) {
        const float p00 = r0[a + ch], p01 = r0[b + ch], p10 = r1[a + ch], p11 = r1[b + ch];
        float t = p00 * (1.0f - lx) * (1.0f - fy);
        t = fmaf(p01 * lx, 1.0f - fy, t);
        t = fmaf(p10 * (1.0f - lx), fy, t);
        float val = fmaf(p11 * lx, fy, t);
        val = val + 0.5f;
        val = val < 0.0f ? 0.0f : (val > 255.0f ? 255.0f : val);
        dst[(y * dw + x) * 3 + ch] = (uint8_t)val;
      }
    }
  }
  free(x0); free(x1); free(fx);
}

/* pack_crop: crop.rs:153-190 -- a text-line crop (u8 RGB, ch x cw) into one
 * [3, img_h, img_w] slot of the zero-filled rec batch: pad_only: centred at
 * original size (rows y0 = (img_h - ch) / 2 on, columns < min(cw, img_w));
 * else resized (resize_bilinear_rgb_u8) to img_h x rw, rw =
 * clamp(ceil(img_h * (cw / ch)), 1, img_w); value (u8 / 255 - 0.5) / 0.5
 * (true divisions).  Positions not written stay 0. */
QPO_API void qpo_pack_crop(const uint8_t* crop, int64_t ch, int64_t cw, int64_t img_h,
                           int64_t img_w, float* dst, int pad_only) {
  const int64_t plane = img_h * img_w;
  if (pad_only) {
    const int64_t y0 = (img_h - ch) / 2;
    const int64_t cols = cw < img_w ? cw : img_w;
    for (int64_t y = 0; y < ch; y++)
      for (int64_t x = 0; x < cols; x++)
        for (int c = 0; c < 3; c++) {
          const float v = (float)crop[(y * cw + x) * 3 + c] / 255.0f;
          dst[c * plane + (y + y0) * img_w + x] = (v - 0.5f) / 0.5f;
        }
    return;
  }
  const float ratio = (float)cw / (float)ch;
  int64_t rw = (int64_t)ceilf((float)img_h * ratio);
  if (rw > img_w) rw = img_w;
  if (rw < 1) rw = 1;
  uint8_t* r = (uint8_t*)malloc((size_t)(rw * img_h * 3));
  qpo_resize_bilinear_rgb_u8(crop, cw, ch, r, rw, img_h);
  for (int64_t y = 0; y < img_h; y++)
    for (int64_t x = 0; x < rw; x++)
      for (int c = 0; c < 3; c++) {
        const float v = (float)r[(y * rw + x) * 3 + c] / 255.0f;
        dst[(c * img_h + y) * img_w + x] = (v - 0.5f) / 0.5f;
      }
  free(r);
}

/* DB post front end (geometry.rs:287-301): mask = pred > thresh ? 1 : 0;
 * with dilation, dilate2x2_max (resize.rs:219-247): out[y][x] = max over
 * the in-range samples of rows y - 1 .. y and columns x - 1 .. x. */
QPO_API void qpo_db_mask(const float* pred, int64_t h, int64_t w, float thresh, int dilate,
                         uint8_t* out) {
  uint8_t* m = (uint8_t*)malloc((size_t)(h * w));
  for (int64_t i = 0; i < h * w; i++) m[i] = pred[i] > thresh ? 1 : 0;
  if (!dilate) {
    memcpy(out, m, (size_t)(h * w));
    free(m);
    return;
  }
  for (int64_t y = 0; y < h; y++)
    for (int64_t x = 0; x < w; x++) {
      uint8_t v = 0;
      for (int64_t dy = -1; dy <= 0; dy++)
        for (int64_t dx = -1; dx <= 0; dx++) {
          const int64_t ny = y + dy, nx = x + dx;
          if (ny < 0 || nx < 0) continue;
          const uint8_t s = m[ny * w + nx];
          v = s > v ? s : v;
        }
      out[y * w + x] = v;
    }
  free(m);
}
