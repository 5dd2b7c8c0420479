// Row kernels of the rec model: LayerNorm, softmax (+ argmax), multi-head
// attention; and the small elementwise / layout kernels.
#include <algorithm>

#include "qph_internal.h"

namespace qph {

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// ---------------------------------------------------------------- LayerNorm
//
// The exported LayerNorm runs on the CPU executor as nine nodes
// (qppocr-core/src/executor.rs:1518-1557 ReduceMean, 885-951 binary ops,
// activation.rs:449-459 Sqrt), each rounding to f32:
//   mu = (float)(sum_f64(x) / C); d = x - mu; sq = d*d (Pow 2);
//   var = (float)(sum_f64(sq) / C); sd = sqrt(var + eps);
//   y = ((d / sd) * gamma) + beta.
// The reference sums each row sequentially in ascending order
// (shape.rs:551-557).  One wave per row; the row (cols <= 64*V) stays in
// registers across the three passes.  Each mean is taken from a shuffle-tree
// f64 sum when that provably gives the sequential sum's f32 mean, else from
// the sequential sum itself (lane 0 walks the row): see f64_mean_order_free.
// Denormal terms count as zero (the CPU path converts with DAZ set,
// par.rs:229-256).

__device__ __forceinline__ double f64_daz(float v) {
  return ((__float_as_uint(v) >> 23) & 0xff) == 0 ? 0.0 : (double)v;
}

// s + the f64 values of v over lanes 0..n-1 in lane order (every lane gets
// the same sum): the terms come through v_readlane as wave-uniform values,
// so the chain of adds runs without memory round trips.
__device__ __forceinline__ double seq_sum_lanes(double s, float v, int n) {
  n = __builtin_amdgcn_readfirstlane(n);
  for (int l = 0; l < n; l++)
    s += f64_daz(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)));
  return s;
}

// Biased f32 exponent of a term as an exactness witness: nonzero finite
// terms give their exponent, zeros (and DAZ-flushed denormals) 255.
__device__ __forceinline__ int term_exp(float v) {
  const int e = (int)((__float_as_uint(v) >> 23) & 0xff);
  return e == 0 ? 255 : e;
}

// s, a: this lane's f64 partial sum of the row's terms and of their
// magnitudes; emin: the smallest term_exp of its terms.  True (wave-uniform)
// with *mean = (float)(sum / n) when the shuffle-tree sum gives the same f32
// mean as the reference's sequential sum:
//  - exact: every term is a multiple of 2^L, L = e_min - 127 - 23, and every
//    partial sum of any order is at most sum|x_i| in magnitude; when that is
//    below 2^(L + 53) every partial sum is exact in f64, so every order gives
//    the exact sum;
//  - else bounded: any order of n terms is within gamma_(n-1) * sum|x_i| of
//    the exact sum (gamma_k = k u / (1 - k u), u = 2^-53), so the two sums
//    are within twice that; division by n and the conversion to f32 are
//    monotone, so when (tree - D) / n and (tree + D) / n round to the same
//    f32 bits, with D twice that bound (the extra covers the rounding of
//    tree +- D), the sequential sum rounds to it as well.
// False for Inf / NaN and for the rare rows that meet neither test, which
// then take the sequential sum.
// f64_mean_check is the test on a row's totals (however they were summed);
// f64_mean_order_free first sums the wave's lane partials.
__device__ __forceinline__ bool f64_mean_check(double s, double a, int emin, int64_t n,
                                               float* mean) {
  if (emin == 255 || a * (1.0 + 0x1p-40) < __builtin_ldexp(1.0, emin - 127 - 23 + 53)) {
    *mean = (float)(s / (double)n);
    return __builtin_isfinite(*mean);
  }
  const double k = (double)(n - 1) * 0x1p-53;
  const double d = 4.0 * (k / (1.0 - k)) * a * (1.0 + 0x1p-30);
  const float lo = (float)((s - d) / (double)n), hi = (float)((s + d) / (double)n);
  *mean = lo;
  return __float_as_uint(lo) == __float_as_uint(hi) && __builtin_isfinite(lo);
}

__device__ __forceinline__ bool f64_mean_order_free(double s, double a, int emin, int64_t n,
                                                    float* mean) {
  s = wave_sum_f64(s);
  a = wave_sum_f64(a);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) emin = min(emin, __shfl_xor(emin, off, 64));
  return f64_mean_check(s, a, emin, n, mean);
}

template <int V>
__global__ __launch_bounds__(256) void layernorm_kernel(const float* __restrict__ x,
                                                        const float* __restrict__ gamma,
                                                        const float* __restrict__ beta, float eps,
                                                        int64_t rows, int64_t cols,
                                                        float* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* xr = x + row * cols;
  float* yr = y + row * cols;
  float xv[V], gv[V], bv[V];
#pragma unroll
  for (int u = 0; u < V; u++) {
    const int64_t j = lane + 64 * u;
    const bool in = j < cols;
    xv[u] = in ? xr[j] : 0.0f;
    gv[u] = in ? gamma[j] : 0.0f;
    bv[u] = in ? beta[j] : 0.0f;
  }
  double s = 0.0, sa = 0.0;
  int emin = 255;
#pragma unroll
  for (int u = 0; u < V; u++)
    if (lane + 64 * u < cols) {
      const double t = f64_daz(xv[u]);
      s += t;
      sa += __builtin_fabs(t);
      emin = min(emin, term_exp(xv[u]));
    }
  float mu;
  if (!f64_mean_order_free(s, sa, emin, cols, &mu)) {
    // the reference's order: element 64 u + l sits in lane l, slot u
    s = 0.0;
    for (int u = 0; u < V; u++)
      s = seq_sum_lanes(s, xv[u], (int)min<int64_t>(64, cols - 64 * u));
    mu = (float)(s / (double)cols);
  }
  float sq[V];
  double s2 = 0.0;
  int emin2 = 255;
#pragma unroll
  for (int u = 0; u < V; u++) {
    const float d = xv[u] - mu;
    sq[u] = d * d;
    if (lane + 64 * u < cols) {
      s2 += f64_daz(sq[u]);
      emin2 = min(emin2, term_exp(sq[u]));
    }
  }
  float var;
  if (!f64_mean_order_free(s2, s2, emin2, cols, &var)) {   // squares: |x| = x
    s2 = 0.0;
    for (int u = 0; u < V; u++)
      s2 = seq_sum_lanes(s2, sq[u], (int)min<int64_t>(64, cols - 64 * u));
    var = (float)(s2 / (double)cols);
  }
  const float sd = __builtin_sqrtf(var + eps);
#pragma unroll
  for (int u = 0; u < V; u++) {
    const int64_t j = lane + 64 * u;
    if (j < cols) {
      float d = xv[u] - mu;
      float v = d / sd;
      v = v * gv[u];
      yr[j] = v + bv[u];
    }
  }
}

int launch_layernorm(const float* x, const float* gamma, const float* beta, float eps,
                     int64_t rows, int64_t cols, float* y, hipStream_t s) {
  dim3 grid(ceil_div(rows, 4));
  if (cols <= 256)
    hipLaunchKernelGGL(layernorm_kernel<4>, grid, dim3(256), 0, s, x, gamma, beta, eps, rows, cols, y);
  else if (cols <= 1024)
    hipLaunchKernelGGL(layernorm_kernel<16>, grid, dim3(256), 0, s, x, gamma, beta, eps, rows, cols, y);
  else
    hipLaunchKernelGGL(layernorm_kernel<64>, grid, dim3(256), 0, s, x, gamma, beta, eps, rows, cols, y);
  return launch_check("layernorm_kernel");
}

// ------------------------------------------------------------------ softmax
//
// softmax_last_dim row semantics (qppocr-kernels/src/activation.rs:346-403,
// x86.rs:1091-1134): mx = row max; e = exp1(x - mx); the sum is eight lane
// partials (lane j takes e[j], e[j+8], ... in order) reduced as
// ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7)), then the cols%8 tail added in
// order; rows narrower than 8 sum sequentially; y = e * (1/sum).
// Workgroup per row.  The max is order-free (no NaN inputs).  The row is
// walked in LDS chunks, double-buffered: waves 1-3 compute e for chunk c+1
// (stored to LDS and to the output) while lanes 0-7 of wave 0 run the eight
// lane chains over chunk c, so the summation order is the reference's.

#define SM_CHUNK 4096  // floats per LDS chunk (16 KB), a multiple of 8

__device__ __forceinline__ float block_max_256(float v, float* red) {
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < 4; i++) r = fmaxf(r, red[i]);
  return r;
}

// probs may alias logits (in-place softmax) or be NULL (pairs only: the
// exponentials are then recomputed from the logits where the probabilities
// would have been read back; exp1 is deterministic, so the values are the
// same).  pairs may be NULL.
// A row past the real batch (rn set and *rn != 0: rows >= *rn * rpb, the
// plan model's word 0) returns at once in every softmax kernel.
__device__ __forceinline__ bool past_real(const unsigned* rn, int64_t rpb, int64_t row) {
  if (!rn) return false;
  const unsigned r = *rn;
  return r != 0 && row >= (int64_t)r * rpb;
}

__global__ __launch_bounds__(256) void softmax_rows_kernel(const float* logits, int64_t cols,
                                                           int64_t ld, float* probs, int64_t ldo,
                                                           float* pairs, const unsigned* rn,
                                                           int64_t rpb) {
  __shared__ float buf[2][SM_CHUNK];
  __shared__ float part[16];
  __shared__ float red[8];
  __shared__ int redi[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  if (past_real(rn, rpb, row)) return;
  const float* xr = logits + row * ld;
  float* pr = probs + row * ldo;

  // max over the row, eight loads in flight per thread
  float mx = -__builtin_inff();
  for (int64_t i0 = tid; i0 < cols; i0 += 256 * 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      int64_t i = i0 + 256 * u;
      v[u] = i < cols ? xr[i] : -__builtin_inff();
    }
#pragma unroll
    for (int u = 0; u < 8; u++) mx = fmaxf(mx, v[u]);
  }
  mx = block_max_256(mx, red);
  __syncthreads();  // every read of the row precedes any in-place write

  const int64_t full = cols >= 8 ? (cols / 8) * 8 : 0;
  const int64_t nch = (cols + SM_CHUNK - 1) / SM_CHUNK;
  // e for chunk c by waves 1-3 (192 threads)
  auto compute = [&](int64_t c) {
    const int64_t base = c * SM_CHUNK;
    const int64_t n = (cols - base) < SM_CHUNK ? (cols - base) : SM_CHUNK;
    float* bb = buf[c & 1];
    for (int64_t j0 = tid - 64; j0 < n; j0 += 192 * 4) {
      float v[4];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        int64_t j = j0 + 192 * u;
        v[u] = j < n ? xr[base + j] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 4; u++) {
        int64_t j = j0 + 192 * u;
        if (j < n) {
          float e = exp1(v[u] - mx);
          bb[j] = e;
          if (probs) pr[base + j] = e;
        }
      }
    }
  };
  if (wave != 0) compute(0);
  __syncthreads();
  float lanesum = 0.0f;  // lanes 0..7 of wave 0
  for (int64_t c = 0; c < nch; c++) {
    if (wave == 0) {
      if (lane < 8) {
        const int64_t base = c * SM_CHUNK;
        const int64_t n = full - base < SM_CHUNK ? full - base : SM_CHUNK;  // full part only
        const float* bb = buf[c & 1];
        float s = lanesum;
        int64_t i = lane;
        for (; i + 8 * 31 < n; i += 8 * 32) {
          float v[32];
#pragma unroll
          for (int u = 0; u < 32; u++) v[u] = bb[i + 8 * u];
#pragma unroll
          for (int u = 0; u < 32; u++) s = s + v[u];
        }
        for (; i < n; i += 8) s = s + bb[i];
        lanesum = s;
      }
    } else if (c + 1 < nch) {
      compute(c + 1);
    }
    __syncthreads();
  }
  if (wave == 0 && lane < 8) part[lane] = lanesum;
  __syncthreads();
  if (tid == 0) {
    float sum;
    if (cols >= 8) {
      float t0 = part[0] + part[4], t1 = part[1] + part[5], t2 = part[2] + part[6],
            t3 = part[3] + part[7];
      sum = (t0 + t1) + (t2 + t3);
    } else {
      sum = 0.0f;
    }
    for (int64_t i = full; i < cols; i++)   // tail, in order
      sum = sum + (probs ? pr[i] : exp1(xr[i] - mx));
    part[8] = sum;
  }
  __syncthreads();
  const float inv = 1.0f / part[8];

  // normalise (+ argmax of the probabilities)
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
  for (int64_t i0 = tid; i0 < cols; i0 += 256 * 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      int64_t i = i0 + 256 * u;
      v[u] = i < cols ? (probs ? pr[i] : exp1(xr[i] - mx)) : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 8; u++) {
      int64_t i = i0 + 256 * u;
      if (i < cols) {
        float p = v[u] * inv;
        if (probs) pr[i] = p;
        if (p > bv) {  // ascending i per thread: keeps the first strict max
          bv = p;
          bi = (int)i;
        }
      }
    }
  }
  if (!pairs) return;
  // argmax reduction: larger value wins, ties -> lower index (rec.rs:46-54)
  for (int off = 32; off >= 1; off >>= 1) {
    float ov = __shfl_xor(bv, off, 64);
    int oi = __shfl_xor(bi, off, 64);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  __syncthreads();
  if (lane == 0) {
    red[wave] = bv;
    redi[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    float v = red[0];
    int ix = redi[0];
    for (int w = 1; w < 4; w++)
      if (red[w] > v || (red[w] == v && redi[w] < ix)) {
        v = red[w];
        ix = redi[w];
      }
    pairs[2 * row] = v;
    pairs[2 * row + 1] = __uint_as_float((unsigned)ix);
  }
}

// Rows of up to 20480 floats (the rec head, 18709): each of the 512 threads
// keeps its elements (i = tid + 512 u) in registers, so the row is read from
// HBM once and the probabilities written once, and a workgroup needs only a
// small LDS window: several rows are resident per CU.  The eight lane chains
// run in lanes 0-7 of wave 0 over windows of 2048 elements that all threads
// write transposed (element j + 8t of the window at j * 264 + t: one
// ds_read_b128 gives a chain lane four of its terms, and a wave's writes hit
// 64 distinct banks), double-buffered so the chains of one window overlap
// the writes of the next.  Same operation sequence as above.
#define SM_REG_MAX_COLS 20480
#define SM_REG_PER_THREAD 40     // SM_REG_MAX_COLS / 512
#define SM_WIN 2048              // elements per chain window (4 per thread)
#define SM_WIN_PITCH 264         // floats per chain lane in a window (8 mod 64)

__device__ __forceinline__ float block_max_512(float v, float* red) {
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < 8; i++) r = fmaxf(r, red[i]);
  return r;
}

__global__ __launch_bounds__(512) void softmax_reg_kernel(const float* logits, int cols, int ld,
                                                          float* probs, int ldo, float* pairs,
                                                          const unsigned* rn, int64_t rpb) {
  __shared__ __attribute__((aligned(16))) float win[2][8 * SM_WIN_PITCH];
  __shared__ float part[16];
  __shared__ float red[8];
  __shared__ int redi[8];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t row = blockIdx.x;
  if (past_real(rn, rpb, row)) return;
  const int nu = (cols - tid + 511) >> 9;   // this thread's elements: u < nu
  // row to registers (out-of-range reads give 0 and are never used)
  float e[SM_REG_PER_THREAD];
  {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(logits + row * ld), 0, cols * 4, 0x00020000);
#pragma unroll
    for (int u = 0; u < SM_REG_PER_THREAD; u++)
      e[u] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(r, (unsigned)(tid + 512 * u) * 4u, 0, 0));
  }
  float mx = -__builtin_inff();
#pragma unroll
  for (int u = 0; u < SM_REG_PER_THREAD; u++) mx = u < nu ? fmaxf(mx, e[u]) : mx;
  mx = block_max_512(mx, red);
#pragma unroll
  for (int u = 0; u < SM_REG_PER_THREAD; u++) e[u] = exp1(e[u] - mx);

  const int full = cols >= 8 ? (cols / 8) * 8 : 0;
  const int t8 = full / 8;
  const int nwin = (full + SM_WIN - 1) / SM_WIN;
  // window w holds elements [w * 2048, w * 2048 + 2048) of the full part:
  // this thread's u = 4w .. 4w + 3
  auto put = [&](int w) {
    float* b = win[w & 1];
#pragma unroll
    for (int q = 0; q < 4; q++) {
#pragma unroll
      for (int u = 0; u < SM_REG_PER_THREAD; u++) {
        if (u != 4 * w + q) continue;
        const int il = tid + 512 * q;      // index inside the window
        if (w * SM_WIN + il < full) b[(il & 7) * SM_WIN_PITCH + (il >> 3)] = e[u];
      }
    }
  };
  float s = 0.0f;   // chain of lane j = lane (lanes 0-7 of wave 0)
  if (nwin > 0) put(0);
  __syncthreads();
  // fully unrolled, so put() picks its registers statically
#pragma unroll
  for (int w = 0; w < SM_REG_MAX_COLS / SM_WIN; w++) {
    if (w >= nwin) continue;   // uniform
    if (w + 1 < nwin) put(w + 1);
    if (wave == 0 && lane < 8) {
      const float* ej = win[w & 1] + lane * SM_WIN_PITCH;
      const int nt = min(t8 - w * (SM_WIN / 8), SM_WIN / 8);   // terms in this window
      int t = 0;
      for (; t + 32 <= nt; t += 32) {
        f32x4 v[8];
#pragma unroll
        for (int q = 0; q < 8; q++) v[q] = *(const f32x4*)(ej + t + 4 * q);
#pragma unroll
        for (int q = 0; q < 8; q++) {
          s = s + v[q][0];
          s = s + v[q][1];
          s = s + v[q][2];
          s = s + v[q][3];
        }
      }
      for (; t < nt; t++) s = s + ej[t];
    }
    __syncthreads();
  }
  // tail elements (full <= i < cols) to LDS for the in-order tail sum
#pragma unroll
  for (int u = 0; u < SM_REG_PER_THREAD; u++) {
    const int i = tid + 512 * u;
    if (i >= full && u < nu) win[0][i - full] = e[u];
  }
  if (wave == 0 && lane < 8) part[lane] = s;
  __syncthreads();
  if (tid == 0) {
    float sum;
    if (cols >= 8) {
      float a0 = part[0] + part[4], a1 = part[1] + part[5], a2 = part[2] + part[6],
            a3 = part[3] + part[7];
      sum = (a0 + a1) + (a2 + a3);
    } else {
      sum = 0.0f;
    }
    for (int i = 0; i < cols - full; i++) sum = sum + win[0][i];   // tail, in order
    part[8] = sum;
  }
  __syncthreads();
  const float inv = 1.0f / part[8];
  float* pr = probs + row * ldo;
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
#pragma unroll
  for (int u = 0; u < SM_REG_PER_THREAD; u++) {
    if (u < nu) {
      const int i = tid + 512 * u;
      const float p = e[u] * inv;
      if (probs) pr[i] = p;
      if (p > bv) {  // ascending i per thread: keeps the first strict max
        bv = p;
        bi = i;
      }
    }
  }
  if (!pairs) return;
  for (int off = 32; off >= 1; off >>= 1) {
    float ov = __shfl_xor(bv, off, 64);
    int oi = __shfl_xor(bi, off, 64);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    red[wave] = bv;
    redi[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    float v = red[0];
    int ix = redi[0];
    for (int w = 1; w < 8; w++)
      if (red[w] > v || (red[w] == v && redi[w] < ix)) {
        v = red[w];
        ix = redi[w];
      }
    pairs[2 * row] = v;
    pairs[2 * row + 1] = __uint_as_float((unsigned)ix);
  }
}

// Rows of up to 19008 floats (the rec head, 18709): registers as in
// softmax_reg_kernel, but all the exponentials of the full part go to LDS at
// once, in the chain layout (element 8t + j at j * SM_TP + t; a wave's
// writes hit 64 distinct banks, a chain lane reads four terms per
// ds_read_b128), so the eight lane chains run in one pass with a single
// barrier before it.  Wave 0 then forms the sum itself (the reference's
// pairwise tree of the chains, then the tail in order).  76 KB of LDS: two
// workgroups per CU.  Same operation sequence as softmax_rows_kernel.
#define SM_TP 2376                      // floats per chain lane (8 mod 64)
#define SM_LDS_MAX_COLS (8 * SM_TP)     // 19008
#define SM_LDS_PER_THREAD 38            // ceil(SM_LDS_MAX_COLS / 512)

__global__ __launch_bounds__(512) void softmax_lds_kernel(const float* logits, int cols, int ld,
                                                          float* probs, int ldo, float* pairs,
                                                          const unsigned* rn, int64_t rpb) {
  __shared__ __attribute__((aligned(16))) float tr[8 * SM_TP];
  __shared__ float tail[8];
  __shared__ float red[8];
  __shared__ int redi[8];
  __shared__ float total;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t row = blockIdx.x;
  if (past_real(rn, rpb, row)) return;
  const int nu = (cols - tid + 511) >> 9;   // this thread's elements: u < nu
  float e[SM_LDS_PER_THREAD];
  {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(logits + row * ld), 0, cols * 4, 0x00020000);
#pragma unroll
    for (int u = 0; u < SM_LDS_PER_THREAD; u++)
      e[u] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(r, (unsigned)(tid + 512 * u) * 4u, 0, 0));
  }
  float mx = -__builtin_inff();
#pragma unroll
  for (int u = 0; u < SM_LDS_PER_THREAD; u++) mx = u < nu ? fmaxf(mx, e[u]) : mx;
  mx = block_max_512(mx, red);
#pragma unroll
  for (int u = 0; u < SM_LDS_PER_THREAD; u++) e[u] = exp1(e[u] - mx);

  const int full = cols >= 8 ? (cols / 8) * 8 : 0;
  const int t8 = full >> 3;
  {
    // element i = tid + 512 u: chain lane i & 7 = tid & 7, term i >> 3
    float* tp = tr + (tid & 7) * SM_TP + (tid >> 3);
#pragma unroll
    for (int u = 0; u < SM_LDS_PER_THREAD; u++) {
      const int i = tid + 512 * u;
      if (i < full)
        tp[64 * u] = e[u];
      else if (u < nu)
        tail[i - full] = e[u];
    }
  }
  __syncthreads();
  if (wave == 0) {
    float s = 0.0f;   // chain of lane j = lane (lanes 0-7)
    if (lane < 8) {
      const float* ej = tr + lane * SM_TP;
      int t = 0;
      for (; t + 32 <= t8; t += 32) {
        f32x4 v[8];
#pragma unroll
        for (int q = 0; q < 8; q++) v[q] = *(const f32x4*)(ej + t + 4 * q);
#pragma unroll
        for (int q = 0; q < 8; q++) {
          s = s + v[q][0];
          s = s + v[q][1];
          s = s + v[q][2];
          s = s + v[q][3];
        }
      }
      for (; t < t8; t++) s = s + ej[t];
    }
    // ((s0 + s4) + (s1 + s5)) + ((s2 + s6) + (s3 + s7)) in lane 0
    const float a = s + __shfl_down(s, 4, 64);   // lane j < 4: s_j + s_(j+4)
    const float b = a + __shfl_down(a, 1, 64);   // lane 0: a0 + a1, lane 2: a2 + a3
    const float c = b + __shfl_down(b, 2, 64);   // lane 0: (a0 + a1) + (a2 + a3)
    if (lane == 0) {
      float sum = cols >= 8 ? c : 0.0f;
      for (int i = 0; i < cols - full; i++) sum = sum + tail[i];   // tail, in order
      total = sum;
    }
  }
  __syncthreads();
  const float inv = 1.0f / total;
  float* pr = probs + row * ldo;
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
#pragma unroll
  for (int u = 0; u < SM_LDS_PER_THREAD; u++) {
    if (u < nu) {
      const int i = tid + 512 * u;
      const float p = e[u] * inv;
      if (probs) pr[i] = p;
      if (p > bv) {  // ascending i per thread: keeps the first strict max
        bv = p;
        bi = i;
      }
    }
  }
  if (!pairs) return;
  for (int off = 32; off >= 1; off >>= 1) {
    float ov = __shfl_xor(bv, off, 64);
    int oi = __shfl_xor(bi, off, 64);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    red[wave] = bv;
    redi[wave] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    float v = red[0];
    int ix = redi[0];
    for (int w = 1; w < 8; w++)
      if (red[w] > v || (red[w] == v && redi[w] < ix)) {
        v = red[w];
        ix = redi[w];
      }
    pairs[2 * row] = v;
    pairs[2 * row + 1] = __uint_as_float((unsigned)ix);
  }
}

// Narrow rows (cols <= SM_SMALL_MAX_COLS, e.g. the attention's T-wide
// rows): eight threads per row, thread j running the reference's lane j
// (activation.rs:346-403 / x86.rs:1091-1134): its max over elements
// 8 g + j of the full groups, its chain of exp1 terms; lane 0 then combines
// the eight maxima in order and takes the tail elements one by one, forms
// the hadd tree ((l0 + l4) + (l1 + l5)) + ((l2 + l6) + (l3 + l7)) and adds
// the tail exponentials in order; every element is multiplied by 1 / sum.
// pairs: the first strict maximum of the probabilities (lane maxima
// combined by value, then lowest index).  In place when probs == logits
// (each element is read before it is written, by the thread that writes it).
#define SM_SMALL_MAX_COLS 128
__global__ __launch_bounds__(256) void softmax_small_kernel(const float* logits, int64_t rows,
                                                            int cols, int64_t ld, float* probs,
                                                            int64_t ldo, float* pairs,
                                                            const unsigned* rn, int64_t rpb) {
  const int j = threadIdx.x & 7;
  const int64_t row = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
  const bool live = row < rows && !past_real(rn, rpb, row);
  const float* xr = logits + (live ? row : 0) * ld;
  float* pr = probs + (live ? row : 0) * ldo;
  const int q = cols >= 8 ? cols / 8 : 0;  // full groups of eight
  float vm = -__builtin_inff();
  if (live && q > 0) {
    vm = xr[j];
    for (int g = 1; g < q; g++) {
      const float v = xr[8 * g + j];
      if (v > vm) vm = v;
    }
  }
  // lane 0 of the row: the reference's combination order
  float mx = 0.0f;
  {
    float lm[8];
#pragma unroll
    for (int t = 0; t < 8; t++) lm[t] = __shfl(vm, t, 8);
    if (j == 0 && live) {
      int i;
      if (q > 0) {
        mx = lm[0];
        for (int t = 1; t < 8; t++)
          if (lm[t] > mx) mx = lm[t];
        i = 8 * q;
      } else {
        mx = xr[0];
        i = 1;
      }
      for (; i < cols; i++)
        if (xr[i] > mx) mx = xr[i];
    }
    mx = __shfl(mx, 0, 8);
  }
  float acc = 0.0f;
  if (live)
    for (int g = 0; g < q; g++) {
      const float e = exp1(xr[8 * g + j] - mx);
      pr[8 * g + j] = e;
      acc = acc + e;
    }
  float inv;
  {
    float la[8];
#pragma unroll
    for (int t = 0; t < 8; t++) la[t] = __shfl(acc, t, 8);
    float sum = 0.0f;
    if (j == 0 && live) {
      if (q > 0) sum = ((la[0] + la[4]) + (la[1] + la[5])) + ((la[2] + la[6]) + (la[3] + la[7]));
      for (int i = 8 * q; i < cols; i++) {
        const float e = exp1(xr[i] - mx);
        pr[i] = e;
        sum = sum + e;
      }
    }
    inv = __shfl(1.0f / sum, 0, 8);
  }
  float bv = -__builtin_inff();
  int bi = 0x7fffffff;
  if (live)
    for (int k = j; k < cols; k += 8) {
      const float p = pr[k] * inv;
      pr[k] = p;
      if (bi == 0x7fffffff || p > bv) {
        bv = p;
        bi = k;
      }
    }
  if (pairs) {
#pragma unroll
    for (int off = 4; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 8);
      const int oi = __shfl_xor(bi, off, 8);
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (j == 0 && live) {
      pairs[2 * row] = bv;
      pairs[2 * row + 1] = __uint_as_float((unsigned)bi);
    }
  }
}

// logits rows ld floats apart (ld >= cols); probs rows ldo floats apart.
int launch_softmax_pitched(const float* logits, int64_t rows, int64_t cols, int64_t ld,
                           float* probs, int64_t ldo, float* pairs, hipStream_t s,
                           const unsigned* rn, int64_t rpb) {
  if (rows > (1ll << 31)) return fail(QPH_EUNSUPPORTED, "softmax: too many rows");
  if (ld < cols || ldo < cols) return fail(QPH_EINVAL, "softmax: row pitch below the row width");
  if (probs == logits && ldo != ld) return fail(QPH_EINVAL, "softmax: in place with two pitches");
  if (cols <= SM_SMALL_MAX_COLS && probs) {
    hipLaunchKernelGGL(softmax_small_kernel, dim3(ceil_div(rows, 32)), dim3(256), 0, s, logits,
                       rows, (int)cols, ld, probs, ldo, pairs, rn, rpb);
    return launch_check("softmax_small_kernel");
  }
  if (cols <= SM_LDS_MAX_COLS && ld < (1ll << 31) && ldo < (1ll << 31)) {
    hipLaunchKernelGGL(softmax_lds_kernel, dim3((unsigned)rows), dim3(512), 0, s, logits,
                       (int)cols, (int)ld, probs, (int)ldo, pairs, rn, rpb);
    return launch_check("softmax_lds_kernel");
  }
  if (cols <= SM_REG_MAX_COLS && ld < (1ll << 31) && ldo < (1ll << 31)) {
    hipLaunchKernelGGL(softmax_reg_kernel, dim3((unsigned)rows), dim3(512), 0, s, logits,
                       (int)cols, (int)ld, probs, (int)ldo, pairs, rn, rpb);
    return launch_check("softmax_reg_kernel");
  }
  hipLaunchKernelGGL(softmax_rows_kernel, dim3((unsigned)rows), dim3(256), 0, s, logits, cols,
                     ld, probs, ldo, pairs, rn, rpb);
  return launch_check("softmax_rows_kernel");
}

static int launch_softmax(const float* logits, int64_t rows, int64_t cols, int64_t ld,
                          float* probs, float* pairs, hipStream_t s) {
  return launch_softmax_pitched(logits, rows, cols, ld, probs, cols, pairs, s);
}

int launch_softmax_rows(float* t, int64_t rows, int64_t cols, hipStream_t s) {
  return launch_softmax(t, rows, cols, cols, t, nullptr, s);
}

int launch_softmax_argmax(const float* logits, int64_t rows, int64_t cols, int64_t ld,
                          float* probs, float* pairs, hipStream_t s) {
  if (!probs && !pairs) return fail(QPH_EINVAL, "softmax_argmax: no output");
  return launch_softmax(logits, rows, cols, ld, probs, pairs, s);
}

// argmax over probabilities: first strict max (rec.rs:46-54).
__global__ __launch_bounds__(256) void argmax_kernel(const float* __restrict__ probs,
                                                     int64_t rows, int64_t cols, int64_t ld,
                                                     float* __restrict__ pairs) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* pr = probs + row * ld;
  float bv = pr[0];
  int bi = 0;
  bool have = false;
  for (int64_t i = lane; i < cols; i += 64) {
    float p = pr[i];
    if (!have || p > bv) {
      bv = p;
      bi = (int)i;
      have = true;
    }
  }
  if (!have) {
    bv = -__builtin_inff();
    bi = 0x7fffffff;
  }
  for (int off = 32; off >= 1; off >>= 1) {
    float ov = __shfl_xor(bv, off, 64);
    int oi = __shfl_xor(bi, off, 64);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    pairs[2 * row] = bv;
    pairs[2 * row + 1] = __uint_as_float((unsigned)bi);
  }
}

int launch_argmax_pitched(const float* probs, int64_t rows, int64_t cols, int64_t ld,
                          float* pairs, hipStream_t s) {
  hipLaunchKernelGGL(argmax_kernel, dim3(ceil_div(rows, 4)), dim3(256), 0, s, probs, rows, cols,
                     ld, pairs);
  return launch_check("argmax_kernel");
}

int launch_argmax(const float* probs, int64_t rows, int64_t cols, float* pairs, hipStream_t s) {
  return launch_argmax_pitched(probs, rows, cols, cols, pairs, s);
}

// Steps t >= t_valid[b] become (0, blank): the padded tail of a bucketed
// line never emits (CTC collapse skips index 0).
__global__ void mask_pairs_kernel(float* pairs, int64_t batch, int64_t t, const int32_t* tv) {
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= batch * t) return;
  int64_t b = idx / t, s = idx - b * t;
  if (s >= tv[b]) {
    pairs[2 * idx] = 0.0f;
    pairs[2 * idx + 1] = __uint_as_float(0u);
  }
}

int launch_mask_pairs(float* pairs, int64_t batch, int64_t t, const int32_t* tv, hipStream_t s) {
  hipLaunchKernelGGL(mask_pairs_kernel, dim3(ceil_div(batch * t, 256)), dim3(256), 0, s, pairs,
                     batch, t, tv);
  return launch_check("mask_pairs_kernel");
}

// ---------------------------------------------------------------- attention
//
// SVTR-style self-attention on the packed QKV MatMul output
// qkv[b][t][3][H][dh]: q = q * scale (Mul node), S = q . k^T and O = P . v
// through the small-matmul path (qppocr-kernels/src/shape.rs:664-697: each
// element is fma(a[kk], b[kk][j], c) from 0, kk ascending), P = softmax over
// the last axis (activation.rs:346-403), out[b][t][h*dh + d].
// One workgroup per (b, h); K and V of that head in LDS; each wave takes
// query rows t1 = wave, wave+4, ... (the loop runs the same number of times
// in every wave so that the block barriers stay uniform).

__global__ __launch_bounds__(256) void attention_kernel(const float* __restrict__ qkv, int64_t T,
                                                        int64_t H, int64_t DH, float scale,
                                                        float* __restrict__ out) {
  extern __shared__ float sm[];
  const int64_t b = blockIdx.x / H, h = blockIdx.x - b * H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t D = H * DH;
  const int ldk = (int)DH + 1;
  float* sk = sm;                        // T x (DH+1)
  float* sv = sk + T * ldk;              // T x (DH+1)
  float* sp = sv + T * ldk;              // 4 waves x (T scores + DH scaled q)
  const float* base = qkv + b * T * 3 * D;
  for (int64_t i = tid; i < T * DH; i += 256) {
    int64_t t = i / DH, d = i - t * DH;
    const float* row = base + t * 3 * D + h * DH + d;
    sk[t * ldk + d] = row[D];
    sv[t * ldk + d] = row[2 * D];
  }
  float* p = sp + wave * (T + DH);
  float* qrow = p + T;
  for (int64_t tb = 0; tb < T; tb += 4) {
    const int64_t t1 = tb + wave;
    const bool active = t1 < T;
    if (active)
      for (int64_t d = lane; d < DH; d += 64) qrow[d] = base[t1 * 3 * D + h * DH + d] * scale;
    __syncthreads();
    // scores: lane j -> S[t1][j] = chain over d of fma(q[t1][d], k[j][d], acc)
    if (active)
      for (int64_t j = lane; j < T; j += 64) {
        float acc = 0.0f;
        for (int64_t d = 0; d < DH; d++) acc = __builtin_fmaf(qrow[d], sk[j * ldk + d], acc);
        p[j] = acc;
      }
    __syncthreads();
    // softmax over p[0..T) in the reference order
    float mx = 0.0f;
    if (active) {
      if (T >= 8) {
        mx = -__builtin_inff();
        for (int64_t j = lane; j < T; j += 64) mx = fmaxf(mx, p[j]);
        for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
      } else {
        mx = p[0];
        for (int64_t j = 1; j < T; j++)
          if (p[j] > mx) mx = p[j];
      }
    }
    __syncthreads();
    if (active)
      for (int64_t j = lane; j < T; j += 64) p[j] = exp1(p[j] - mx);
    __syncthreads();
    float inv = 0.0f;
    if (active) {
      float part = 0.0f;
      const int64_t full = T >= 8 ? (T / 8) * 8 : 0;
      if (lane < 8)
        for (int64_t j = lane; j < full; j += 8) part = part + p[j];
      float l[8];
#pragma unroll
      for (int q = 0; q < 8; q++) l[q] = __shfl(part, q, 64);
      float sum;
      int64_t j0;
      if (T >= 8) {
        float t0 = l[0] + l[4], t1s = l[1] + l[5], t2 = l[2] + l[6], t3 = l[3] + l[7];
        sum = (t0 + t1s) + (t2 + t3);
        j0 = full;
      } else {
        sum = 0.0f;
        j0 = 0;
      }
      for (int64_t j = j0; j < T; j++) sum = sum + p[j];
      inv = 1.0f / sum;
    }
    __syncthreads();
    if (active)
      for (int64_t j = lane; j < T; j += 64) p[j] = p[j] * inv;
    __syncthreads();
    // O[t1][d] = chain over j of fma(P[t1][j], v[j][d], acc)
    if (active)
      for (int64_t d = lane; d < DH; d += 64) {
        float acc = 0.0f;
        for (int64_t j = 0; j < T; j++) acc = __builtin_fmaf(p[j], sv[j * ldk + d], acc);
        out[(b * T + t1) * D + h * DH + d] = acc;
      }
    __syncthreads();
  }
}

// Head dimension known at compile time: one workgroup per (batch, head);
// q (times scale: the Mul node), k and v of all T rows arrive in LDS in one
// burst of loads, then the query rows go in blocks (all rows up to 64).
// Scores: one chain of DH fmas per (row, key).  Softmax: eight threads per
// row, thread j owning elements j, j+8, ... -- its max part, its exp1 values
// and exactly the reference's lane-j chain -- then the
// ((l0+l4)+(l1+l5))+((l2+l6)+(l3+l7)) tree and the tail in order within the
// group of eight (no workgroup barrier).  P.V: one chain of T fmas per
// (row, d).
// MF (T % 4 == 0): both products on v_mfma_f32_16x16x4f32, whose four k
// terms per instruction are added in order, so each 16x16 output block is
// the same fma chains (k = d for the scores, k = j for P.V, each from 0);
// q, k and v rows are zero-filled up to a multiple of 16 and the score /
// probability block to 16-row, 16-column tiles, whose extra outputs are
// never used.

// The attention of one (batch, head) once q (times scale), k and v of its
// rows are in LDS (rows t .. tp - 1 zero): scores, the softmax with the
// reference's lane chains, P.V, written to out[r * D + d] (out at the
// head's first column of the batch's first row).  NT threads.
template <int DH, bool MF, int NT>
__device__ __forceinline__ void attention_rows(const float* sq, const float* sk, const float* sv,
                                               float* sp, int t, int tp, int ldp, int blk,
                                               int64_t D, float* __restrict__ out) {
  constexpr int LD = DH + 1;
  const int full = t >= 8 ? (t / 8) * 8 : 0;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lg = lane >> 4, l16 = lane & 15;
  for (int r0 = 0; r0 < t; r0 += blk) {
    const int rb = (t - r0) < blk ? (t - r0) : blk;
    if (MF) {
      // S block (rb x t) in 16x16 tiles over the waves
      const int nr = (rb + 15) / 16, nc = tp / 16;
      for (int tl = wave; tl < nr * nc; tl += NT / 64) {
        const int br = tl / nc, bc = tl - br * nc;
        const float* a = sq + (r0 + 16 * br + l16) * LD + lg;
        const float* bk = sk + (16 * bc + l16) * LD + lg;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int s4 = 0; s4 < DH / 4; s4++)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[4 * s4], bk[4 * s4], acc, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 4; v++) sp[(16 * br + 4 * lg + v) * ldp + 16 * bc + l16] = acc[v];
      }
    } else {
      // scores S[r][j] = chain over d of fma(q[r][d], k[j][d], acc)
      for (int i = tid; i < rb * t; i += NT) {
        const int r = i / t, j = i - r * t;
        const float* qr = sq + (r0 + r) * LD;
        const float* kj = sk + j * LD;
        float acc = 0.0f;
#pragma unroll
        for (int d = 0; d < DH; d++) acc = __builtin_fmaf(qr[d], kj[d], acc);
        sp[r * ldp + j] = acc;
      }
    }
    __syncthreads();
    // softmax, eight threads per row (groups never straddle a wave)
    for (int g0 = 0; g0 < rb; g0 += NT / 8) {
      const int r = g0 + (tid >> 3), lj = tid & 7;
      const bool rowok = r < rb;
      float* pr = sp + (rowok ? r : 0) * ldp;
      float mx = -__builtin_inff();
      if (rowok)
        for (int j = lj; j < t; j += 8) mx = fmaxf(mx, pr[j]);
      for (int off = 4; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 8));
      if (t < 8 && rowok) {   // narrow rows: sequential max from the first element
        mx = pr[0];
        for (int j = 1; j < t; j++)
          if (pr[j] > mx) mx = pr[j];
      }
      float s = 0.0f;
      if (rowok)
        for (int j = lj; j < t; j += 8) {
          const float e = exp1(pr[j] - mx);
          pr[j] = e;
          if (j < full) s = s + e;   // lane lj's chain, ascending j
        }
      // tree of the eight lane chains, then the tail in order (lane 0)
      const int gb = (threadIdx.x & 63) & ~7;
      const float l0 = __shfl(s, gb + 0, 64), l1 = __shfl(s, gb + 1, 64);
      const float l2 = __shfl(s, gb + 2, 64), l3 = __shfl(s, gb + 3, 64);
      const float l4 = __shfl(s, gb + 4, 64), l5 = __shfl(s, gb + 5, 64);
      const float l6 = __shfl(s, gb + 6, 64), l7 = __shfl(s, gb + 7, 64);
      float sum = 0.0f;
      if (rowok && lj == 0) {
        if (t >= 8) sum = ((l0 + l4) + (l1 + l5)) + ((l2 + l6) + (l3 + l7));
        for (int j = full; j < t; j++) sum = sum + pr[j];
      }
      sum = __shfl(sum, gb, 64);
      const float inv = 1.0f / sum;
      if (rowok)
        for (int j = lj; j < t; j += 8) pr[j] = pr[j] * inv;
    }
    __syncthreads();
    if (MF) {
      // O block (rb x DH) = P . v in 16x16 tiles, k = j over exactly t terms
      const int nr = (rb + 15) / 16;
      for (int tl = wave; tl < nr * (DH / 16); tl += NT / 64) {
        const int br = tl / (DH / 16), bc = tl - br * (DH / 16);
        const float* a = sp + (16 * br + l16) * ldp + lg;
        const float* bv = sv + lg * LD + 16 * bc + l16;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int s4 = 0; s4 < t / 4; s4++)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[4 * s4], bv[4 * s4 * LD], acc, 0, 0, 0);
#pragma unroll
        for (int v = 0; v < 4; v++) {
          const int r = 16 * br + 4 * lg + v;
          if (r < rb) out[(int64_t)(r0 + r) * D + 16 * bc + l16] = acc[v];
        }
      }
    } else {
      // O[r][d] = chain over j of fma(P[r][j], v[j][d], acc); operands read
      // eight j at a time so their LDS reads are in flight together
      for (int i = tid; i < rb * DH; i += NT) {
        const int r = i / DH, d = i - r * DH;
        const float* p = sp + r * ldp;
        const float* vd = sv + d;
        float acc = 0.0f;
        int j = 0;
        for (; j + 8 <= t; j += 8) {
          float pv[8], vv[8];
#pragma unroll
          for (int u = 0; u < 8; u++) {
            pv[u] = p[j + u];
            vv[u] = vd[(j + u) * LD];
          }
#pragma unroll
          for (int u = 0; u < 8; u++) acc = __builtin_fmaf(pv[u], vv[u], acc);
        }
        for (; j < t; j++) acc = __builtin_fmaf(p[j], vd[j * LD], acc);
        out[(int64_t)(r0 + r) * D + d] = acc;
      }
    }
    __syncthreads();
  }
}

template <int DH, bool MF>
__global__ __launch_bounds__(256) void attention_dh_kernel(const float* __restrict__ qkv,
                                                           int64_t T, int64_t H, float scale,
                                                           int blk, float* __restrict__ out) {
  extern __shared__ float sm[];
  constexpr int LD = DH + 1;
  const int64_t b = blockIdx.x / H, h = blockIdx.x - b * H;
  const int tid = threadIdx.x;
  const int64_t D = H * DH;
  const int t = (int)T;
  const int tp = MF ? (t + 15) / 16 * 16 : t;     // rows held (zero past t)
  const int ldp = MF ? tp + 1 : t + 1;
  float* sq = sm;                 // tp x LD (scaled q)
  float* sk = sq + tp * LD;       // tp x LD
  float* sv = sk + tp * LD;       // tp x LD
  float* sp = sv + tp * LD;       // blk (rounded to 16) x ldp scores / probabilities
  const float* base = qkv + b * T * 3 * D + h * DH;
  for (int i0 = tid; i0 < tp * DH; i0 += 256 * 4) {
    float q[4], k[4], v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int i = i0 + 256 * u;
      q[u] = k[u] = v[u] = 0.0f;
      if (i < t * DH) {
        const float* row = base + (int64_t)(i / DH) * 3 * D + (i % DH);
        q[u] = row[0];
        k[u] = row[D];
        v[u] = row[2 * D];
      }
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int i = i0 + 256 * u;
      if (i < tp * DH) {
        const int r = i / DH, d = i - r * DH;
        sq[r * LD + d] = q[u] * scale;   // Mul node
        sk[r * LD + d] = k[u];
        sv[r * LD + d] = v[u];
      }
    }
  }
  __syncthreads();
  attention_rows<DH, MF, 256>(sq, sk, sv, sp, t, tp, ldp, blk, D, out + b * T * D + h * DH);
}

// The rec QKV linear and the attention that reads it, one launch: one
// workgroup of 512 threads per (batch, head) computes its head's q, k and v
// columns of the linear for the batch's T rows (T <= 64, T % 4 == 0, head
// dimension 32, K = 64 NK <= 256), then the attention of those rows; the
// QKV tensor never reaches HBM.  The product is linear_nt_kernel's: 16x16
// output blocks on v_mfma_f32_16x16x4f32, each a chain over k ascending
// from 0 (x rows as A, the resident transposed weight rows as B, the same
// 64-k slabs with 16-byte chunks swizzled by row), then + bias (or -0.0,
// the exact identity), so q, k and v are bit-identical to the stored
// linear output; q is then multiplied by scale and rows T .. tp - 1 are 0,
// as attention_dh_kernel loads them.  K slabs go through two LDS stages
// (x: 64 rows, rows past T read 0; weights: the head's 96 rows), 5 loads
// per wave per slab.  Reference: the MatMul (+ Add) of the QKV projection
// (gemm.rs) and the attention nodes after it (qppocr-core/src/executor.rs).
#define QA_ROWS 64                      // x rows of a slab (T <= 64)
#define QA_STAGE ((QA_ROWS + 96) * 64)  // floats: x slab, then weight slab
template <int NK>
__global__ __launch_bounds__(512) void qkv_attention_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ wt,
                                                            const float* __restrict__ bias,
                                                            int T, int H, float scale, int blk,
                                                            float* __restrict__ out) {
  constexpr int DH = 32, LD = DH + 1, K = NK * 64;
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lg = lane >> 4, l16 = lane & 15;
  const int b = blockIdx.x / H, h = blockIdx.x - b * H;
  const int64_t D = (int64_t)H * DH;
  const int tp = (T + 15) / 16 * 16;
  const int nrb = tp / 16, nblk = nrb * 6;   // 16x16 blocks: row blocks x (q, k, v) x 2
  // this wave's blocks j = wave + 8 i (at most 3: tp <= 64 gives 24 blocks)
  float badd[3];
#pragma unroll
  for (int i = 0; i < 3; i++) {
    const int j = wave + 8 * i, cb = j % 6, n = 16 * cb + l16;
    const int64_t col = (int64_t)(n / 32) * D + h * DH + (n & 31);
    badd[i] = (bias && j < nblk) ? bias[col] : -0.0f;
  }
  const unsigned OOB = 0x80000000u;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(x + (int64_t)b * T * K), 0, T * K * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)wt, 0, (int)(3 * D * K * 4), 0x00020000);
  // load u of a slab (0..4 per wave): 16-byte chunk q = 64 (5 wave + u) +
  // lane of the stage; x rows 0..63 (chunks 0..1023), then weight rows
  // 0..95; chunk position p of row r holds source chunk p ^ (r % 16)
  unsigned off[5];
#pragma unroll
  for (int u = 0; u < 5; u++) {
    const int q = 64 * (5 * wave + u) + lane;
    if (q < QA_ROWS * 16) {
      const int r = q >> 4, c = (q & 15) ^ (r & 15);
      off[u] = r < T ? (unsigned)((r * K + 4 * c) * 4) : OOB;
    } else {
      const int n = (q >> 4) - QA_ROWS, c = (q & 15) ^ (n & 15);
      const int64_t col = (int64_t)(n / 32) * D + h * DH + (n & 31);
      off[u] = (unsigned)((col * K + 4 * c) * 4);
    }
  }
  // the loads as inline asm: the compiler then leaves the waits to the
  // explicit vmcnt counts below (it cannot tell the two stages apart and
  // would wait for both before every slab's reads)
  auto issue = [&](int kt, float* st) {
    const unsigned so = __builtin_amdgcn_readfirstlane((unsigned)(kt * 64 * 4));
#pragma unroll
    for (int u = 0; u < 5; u++) {
      const bool isx = 5 * wave + u < QA_ROWS / 4;   // wave-uniform
      const unsigned m = __builtin_amdgcn_readfirstlane(
          (unsigned)(uintptr_t)(__attribute__((address_space(3))) float*)(st + 256 * (5 * wave + u)));
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"   // m0 is reserved; nothing else uses it here
      __asm__ volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(m),
                       "v"(off[u]), "s"(isx ? xr : wr), "s"(so)
                       : "m0");
#pragma clang diagnostic pop
    }
  };
  float* st0 = sm;
  float* st1 = sm + QA_STAGE;
  issue(0, st0);
  if (NK > 1) issue(1, st1);
  f32x4 acc[3];
#pragma unroll
  for (int i = 0; i < 3; i++) acc[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // a wave's blocks j = wave + 8 i; a wave whose third block is past nblk
  // runs the two-chain form of the slab loop (past nblk, a block index
  // reads block 0: in bounds, never used)
  int arow[3], wrow[3];
#pragma unroll
  for (int i = 0; i < 3; i++) {
    const int j = wave + 8 * i < nblk ? wave + 8 * i : 0, rb = j / 6, cb = j - 6 * rb;
    arow[i] = (16 * rb + l16) * 64 + lg;
    wrow[i] = (QA_ROWS + 16 * cb + l16) * 64 + lg;
  }
  // the slab loop over NB of the wave's chains (every wave reaches every
  // barrier whichever form it runs)
  auto slabs = [&](auto nbc) {
    constexpr int NB = decltype(nbc)::value;
#pragma unroll
    for (int kt = 0; kt < NK; kt++) {
      __asm__ volatile("" ::: "memory");
      if (kt + 1 < NK)
        wait_vmcnt<5>();
      else
        wait_vmcnt<0>();
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_s_barrier();
      __asm__ volatile("" ::: "memory");
      const float* st = (kt & 1) ? st1 : st0;
      float av[NB][16], bv[NB][16];
#pragma unroll
      for (int i = 0; i < NB; i++)
#pragma unroll
        for (int s4 = 0; s4 < 16; s4++) {
          av[i][s4] = st[arow[i] + 4 * (s4 ^ l16)];
          bv[i][s4] = st[wrow[i] + 4 * (s4 ^ l16)];
        }
#pragma unroll
      for (int s4 = 0; s4 < 16; s4++)
#pragma unroll
        for (int i = 0; i < NB; i++)
          acc[i] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i][s4], bv[i][s4], acc[i], 0, 0, 0);
      if (kt + 2 < NK) {
        // every wave's reads of this stage done, then its refill
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_s_barrier();
        __asm__ volatile("" ::: "memory");
        issue(kt + 2, (kt & 1) ? st1 : st0);
      }
    }
  };
  if (wave + 16 < nblk)
    slabs(std::integral_constant<int, 3>{});
  else
    slabs(std::integral_constant<int, 2>{});
  __syncthreads();   // the stages are free: q, k, v go where they were
  float* sq = sm;                       // tp x LD (scaled q)
  float* sk = sq + QA_ROWS * LD;        // tp x LD
  float* sv = sk + QA_ROWS * LD;        // tp x LD
  float* sp = sv + QA_ROWS * LD;        // blk (rounded to 16) x (tp + 1)
#pragma unroll
  for (int i = 0; i < 3; i++) {
    const int j = wave + 8 * i, rb = j / 6, cb = j - 6 * rb;
    if (j < nblk) {
      const int n = 16 * cb + l16, which = n / 32, d = n & 31;
      float* dst = which == 0 ? sq : which == 1 ? sk : sv;
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const int r = 16 * rb + 4 * lg + v;
        const float y = acc[i][v] + badd[i];
        dst[r * LD + d] = r < T ? (which == 0 ? y * scale : y) : 0.0f;   // Mul node on q
      }
    }
  }
  __syncthreads();
  attention_rows<DH, true, 512>(sq, sk, sv, sp, T, tp, tp + 1, blk, D,
                                out + (int64_t)b * T * D + h * DH);
}

bool qkv_attention_eligible(int64_t batch, int64_t t, int64_t heads, int64_t dh, int64_t k) {
  return dh == 32 && t > 0 && t <= QA_ROWS && t % 4 == 0 && k % 64 == 0 && k >= 64 &&
         k <= 256 && batch * heads < (1ll << 31) && 3 * heads * dh * k * 4 < (1ll << 31) &&
         t * k * 4 < (1ll << 31);
}

int launch_qkv_attention(const float* x, const float* wt, const float* bias, int64_t batch,
                         int64_t t, int64_t heads, int64_t dh, int64_t k, float scale, float* out,
                         hipStream_t s) {
  if (!qkv_attention_eligible(batch, t, heads, dh, k))
    return fail(QPH_EUNSUPPORTED, "qkv + attention: shape outside the fused kernel");
  if ((uintptr_t)x % 16 || (uintptr_t)wt % 16)
    return fail(QPH_EUNSUPPORTED, "qkv + attention: operands not 16-byte aligned");
  // the two stages (the attention's q, k, v and scores fit in them after)
  const size_t lds = (size_t)2 * QA_STAGE * 4;
  const int blk = (int)t;   // all query rows in one block
  const dim3 grid((unsigned)(batch * heads));
  switch (k / 64) {
    case 1:
      QPH_TRY(allow_full_lds((const void*)qkv_attention_kernel<1>));
      hipLaunchKernelGGL(qkv_attention_kernel<1>, grid, dim3(512), lds, s, x, wt, bias, (int)t,
                         (int)heads, scale, blk, out);
      break;
    case 2:
      QPH_TRY(allow_full_lds((const void*)qkv_attention_kernel<2>));
      hipLaunchKernelGGL(qkv_attention_kernel<2>, grid, dim3(512), lds, s, x, wt, bias, (int)t,
                         (int)heads, scale, blk, out);
      break;
    case 3:
      QPH_TRY(allow_full_lds((const void*)qkv_attention_kernel<3>));
      hipLaunchKernelGGL(qkv_attention_kernel<3>, grid, dim3(512), lds, s, x, wt, bias, (int)t,
                         (int)heads, scale, blk, out);
      break;
    default:
      QPH_TRY(allow_full_lds((const void*)qkv_attention_kernel<4>));
      hipLaunchKernelGGL(qkv_attention_kernel<4>, grid, dim3(512), lds, s, x, wt, bias, (int)t,
                         (int)heads, scale, blk, out);
      break;
  }
  return launch_check("qkv_attention_kernel");
}

static size_t attention_dh_lds(int64_t t, int64_t dh, int64_t blk, bool mf) {
  const int64_t tp = mf ? (t + 15) / 16 * 16 : t;
  const int64_t bp = mf ? (blk + 15) / 16 * 16 : blk;
  return (size_t)(3 * tp * (dh + 1) + bp * (tp + 1)) * sizeof(float);
}

int launch_attention(const float* qkv, int64_t batch, int64_t t, int64_t heads, int64_t dh,
                     float scale, float* out, hipStream_t s) {
  // query rows per block: all of them up to 64, else 64 or 32 as LDS allows
  const bool mf = t % 4 == 0;
  int64_t blk = t <= 64 ? t : 64;
  if (attention_dh_lds(t, dh, blk, mf) > 160 * 1024) blk = 32;
  if ((dh == 32 || dh == 64) && attention_dh_lds(t, dh, blk, mf) <= 160 * 1024) {
    if (batch * heads > (1ll << 31)) return fail(QPH_EUNSUPPORTED, "attention: grid too large");
    const size_t lds = attention_dh_lds(t, dh, blk, mf);
    const void* fn = dh == 32 ? (mf ? (const void*)attention_dh_kernel<32, true>
                                    : (const void*)attention_dh_kernel<32, false>)
                              : (mf ? (const void*)attention_dh_kernel<64, true>
                                    : (const void*)attention_dh_kernel<64, false>);
    QPH_TRY(allow_full_lds(fn));
    const dim3 grid((unsigned)(batch * heads));
    if (dh == 32 && mf)
      hipLaunchKernelGGL((attention_dh_kernel<32, true>), grid, dim3(256), lds, s, qkv, t, heads,
                         scale, (int)blk, out);
    else if (dh == 32)
      hipLaunchKernelGGL((attention_dh_kernel<32, false>), grid, dim3(256), lds, s, qkv, t, heads,
                         scale, (int)blk, out);
    else if (mf)
      hipLaunchKernelGGL((attention_dh_kernel<64, true>), grid, dim3(256), lds, s, qkv, t, heads,
                         scale, (int)blk, out);
    else
      hipLaunchKernelGGL((attention_dh_kernel<64, false>), grid, dim3(256), lds, s, qkv, t, heads,
                         scale, (int)blk, out);
    return launch_check("attention_dh_kernel");
  }
  return launch_attention_generic(qkv, batch, t, heads, dh, scale, out, s);
}

int launch_attention_generic(const float* qkv, int64_t batch, int64_t t, int64_t heads,
                             int64_t dh, float scale, float* out, hipStream_t s) {
  size_t lds = (size_t)(2 * t * (dh + 1) + 4 * (t + dh)) * sizeof(float);
  if (lds > 64 * 1024) return fail(QPH_EUNSUPPORTED, "attention: T*dh too large for LDS");
  if (batch * heads > (1ll << 31)) return fail(QPH_EUNSUPPORTED, "attention: grid too large");
  hipLaunchKernelGGL(attention_kernel, dim3((unsigned)(batch * heads)), dim3(256), lds, s, qkv,
                     t, heads, dh, scale, out);
  return launch_check("attention_kernel");
}

// ------------------------------------------------------------- elementwise

__global__ void act_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n, Act a) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    float v = x[i];
    y[i] = act_apply(v, a);
  }
}

int launch_elementwise_act(const float* x, float* y, int64_t n, const Act& a, hipStream_t s) {
  int64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(act_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, y, n, a);
  return launch_check("act_kernel");
}

// resize_nearest (qppocr-kernels/src/resize.rs:26-57):
// iy = min((int)((float)oy * (float)H / (float)oh), H-1), likewise ix.
__global__ void resize_nearest_kernel(const float* __restrict__ x, int64_t h, int64_t w,
                                      int64_t oh, int64_t ow, float* __restrict__ y) {
  const int64_t p = blockIdx.y;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= oh * ow) return;
  const int64_t oy = idx / ow, ox = idx - oy * ow;
  int64_t iy = (int64_t)((float)oy * (float)h / (float)oh);
  int64_t ix = (int64_t)((float)ox * (float)w / (float)ow);
  if (iy > h - 1) iy = h - 1;
  if (ix > w - 1) ix = w - 1;
  y[p * oh * ow + idx] = x[(p * h + iy) * w + ix];
}

int launch_resize_nearest(const float* x, int64_t nc, int64_t h, int64_t w, int64_t oh,
                          int64_t ow, float* y, hipStream_t s) {
  if (nc > 65535) return fail(QPH_EUNSUPPORTED, "resize: too many planes");
  hipLaunchKernelGGL(resize_nearest_kernel, dim3(ceil_div(oh * ow, 256), (unsigned)nc), dim3(256),
                     0, s, x, h, w, oh, ow, y);
  return launch_check("resize_nearest_kernel");
}

// Broadcast binary op in place (elementwise.rs:185-298): one IEEE op each.
__global__ void binary_kernel(float* __restrict__ a, const float* __restrict__ b, int64_t rows,
                              int64_t cols, int op, int bmode) {
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; idx < rows * cols; idx += stride) {
    int64_t r = idx / cols, j = idx - r * cols;
    float bv = bmode == 0 ? b[r] : (bmode == 1 ? b[j] : (bmode == 2 ? b[0] : b[idx]));
    float av = a[idx];
    float o;
    switch (op) {
      case 0: o = av + bv; break;
      case 1: o = av - bv; break;
      case 2: o = av * bv; break;
      default: o = av / bv; break;
    }
    a[idx] = o;
  }
}

int launch_binary(float* a, const float* b, int64_t rows, int64_t cols, int op, int bmode,
                  hipStream_t s) {
  int64_t blocks = (rows * cols + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(binary_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a, b, rows, cols, op,
                     bmode);
  return launch_check("binary_kernel");
}

// y = x op b element for element (mode 0), x op scalar (mode 1) or scalar
// op x (mode 2): binary_op's same-shape pass and its one-element fast path
// (elementwise.rs:185-298, 350-363; x86.rs:1241-1278), one IEEE op each.
// Four elements a thread by 16-byte accesses when every pointer allows.
template <int OP, int MODE, bool V4>
__global__ __launch_bounds__(256) void binary_out_kernel(const float* __restrict__ x,
                                                         const float* __restrict__ b, float sv,
                                                         float* __restrict__ y, int64_t n) {
  auto op = [&](float a, float c) {
    if constexpr (OP == 0) return a + c;
    else if constexpr (OP == 1) return a - c;
    else if constexpr (OP == 2) return a * c;
    else return a / c;
  };
  auto one = [&](float xv, float bv) {
    if constexpr (MODE == 0) return op(xv, bv);
    else if constexpr (MODE == 1) return op(xv, sv);
    else return op(sv, xv);
  };
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if constexpr (V4) {
    for (; 4 * i < n; i += stride) {
      const f32x4 xv = *(const f32x4*)(x + 4 * i);
      f32x4 bv = {0.0f, 0.0f, 0.0f, 0.0f};
      if constexpr (MODE == 0) bv = *(const f32x4*)(b + 4 * i);
      f32x4 o;
#pragma unroll
      for (int q = 0; q < 4; q++) o[q] = one(xv[q], bv[q]);
      *(f32x4*)(y + 4 * i) = o;
    }
  } else {
    for (; i < n; i += stride) y[i] = one(x[i], MODE == 0 ? b[i] : 0.0f);
  }
}

template <int OP, int MODE>
static void launch_binary_out_t(const float* x, const float* b, float sv, float* y, int64_t n,
                                bool v4, hipStream_t s) {
  const int64_t items = v4 ? n / 4 : n;
  const unsigned blocks = (unsigned)std::max<int64_t>(1, std::min<int64_t>((items + 255) / 256, 16384));
  if (v4)
    hipLaunchKernelGGL((binary_out_kernel<OP, MODE, true>), dim3(blocks), dim3(256), 0, s, x, b,
                       sv, y, n);
  else
    hipLaunchKernelGGL((binary_out_kernel<OP, MODE, false>), dim3(blocks), dim3(256), 0, s, x, b,
                       sv, y, n);
}

template <int OP>
static void launch_binary_out_m(const float* x, const float* b, float sv, float* y, int64_t n,
                                int mode, bool v4, hipStream_t s) {
  if (mode == 0) launch_binary_out_t<OP, 0>(x, b, sv, y, n, v4, s);
  else if (mode == 1) launch_binary_out_t<OP, 1>(x, b, sv, y, n, v4, s);
  else launch_binary_out_t<OP, 2>(x, b, sv, y, n, v4, s);
}

int launch_binary_out(const float* x, const float* b, float sv, float* y, int64_t n, int op,
                      int mode, hipStream_t s) {
  if (op < 0 || op > 3 || mode < 0 || mode > 2 || (mode == 0 && !b))
    return fail(QPH_EINVAL, "binary: op 0..3 and mode 0..2 (mode 0 needs b)");
  if (n <= 0) return QPH_OK;
  auto al = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  const bool v4 = n % 4 == 0 && al(x) && al(y) && (mode != 0 || al(b));
  switch (op) {
    case 0: launch_binary_out_m<0>(x, b, sv, y, n, mode, v4, s); break;
    case 1: launch_binary_out_m<1>(x, b, sv, y, n, mode, v4, s); break;
    case 2: launch_binary_out_m<2>(x, b, sv, y, n, mode, v4, s); break;
    default: launch_binary_out_m<3>(x, b, sv, y, n, mode, v4, s); break;
  }
  return launch_check("binary_out_kernel");
}

// reduce_mean over the last axis (shape.rs:510-560): f64 sum, / cols, to f32.
// Row r's element j is x[(r / rpg) * gstride + (r % rpg) * rstride + j * estride]
// (contiguous rows: rpg = rows, rstride = cols, estride = 1); its mean goes
// to out[r * ostride], and with ostride == 4 the other three words of the
// row's group of four are set to 0.
struct MeanRows {
  const float* x;
  int64_t rows, cols, rpg, gstride, rstride, estride;
  float* out;
  int64_t ostride;
  const unsigned* rn;   // plan path: rows >= *rn * rpb skipped when *rn != 0
  int64_t rpb;
};

__global__ __launch_bounds__(256) void reduce_mean_kernel(MeanRows p) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= p.rows || past_real(p.rn, p.rpb, row)) return;
  const int64_t cols = p.cols, es = p.estride;
  const float* xr = p.x + (row / p.rpg) * p.gstride + (row % p.rpg) * p.rstride;
  double s = 0.0, sa = 0.0;
  int emin = 255;
  for (int64_t j = lane; j < cols; j += 64) {
    const float v = xr[j * es];
    const double t = f64_daz(v);
    s += t;
    sa += __builtin_fabs(t);
    emin = min(emin, term_exp(v));
  }
  float mean;
  // the reference's ascending sequential sum (shape.rs:551-557) wherever a
  // tree sum could round to another f32 mean (f64_mean_order_free)
  if (!f64_mean_order_free(s, sa, emin, cols, &mean)) {
    s = 0.0;
    for (int64_t j0 = 0; j0 < cols; j0 += 64) {
      const float v = j0 + lane < cols ? xr[(j0 + lane) * es] : 0.0f;
      s = seq_sum_lanes(s, v, (int)min<int64_t>(64, cols - j0));
    }
    mean = (float)(s / (double)cols);
  }
  if (lane == 0) p.out[row * p.ostride] = mean;
  if (p.ostride == 4 && lane >= 1 && lane <= 3) p.out[row * 4 + lane] = 0.0f;
}

// Long rows (a global average pool's planes): one 256-thread workgroup per
// row, every load of a pass issued before its terms are summed (16-byte
// loads when the row is contiguous and aligned: 16 a thread, so a pass covers
// 16384 terms).  The lane partials meet through LDS and f64_mean_check runs
// on the row's totals: it holds for any summation order, and a row that
// fails it takes the same sequential sum as above, on wave 0.
template <bool VEC>
__global__ __launch_bounds__(256) void reduce_mean_wg_kernel(MeanRows p) {
  __shared__ double ls[4], la[4];
  __shared__ int le[4];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  if (past_real(p.rn, p.rpb, row)) return;
  const int64_t cols = p.cols, es = p.estride;
  const float* xr = p.x + (row / p.rpg) * p.gstride + (row % p.rpg) * p.rstride;
  double s = 0.0, sa = 0.0;
  int emin = 255;
  // padding terms are 0.0f: they add 0 and their term_exp (255) is no minimum
  auto term = [&](float v) {
    const double t = f64_daz(v);
    s += t;
    sa += __builtin_fabs(t);
    emin = min(emin, term_exp(v));
  };
  if constexpr (VEC) {
    const int64_t nq = cols >> 2;
    const f32x4* xq = (const f32x4*)xr;
    for (int64_t q0 = 0; q0 < nq; q0 += 256 * 16) {
      f32x4 v[16];
#pragma unroll
      for (int u = 0; u < 16; u++) {
        const int64_t q = q0 + u * 256 + tid;
        v[u] = q < nq ? xq[q] : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
      for (int u = 0; u < 16; u++)
#pragma unroll
        for (int c = 0; c < 4; c++) term(v[u][c]);
    }
    for (int64_t j = (nq << 2) + tid; j < cols; j += 256) term(xr[j]);
  } else {
    for (int64_t j0 = 0; j0 < cols; j0 += 256 * 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int64_t j = j0 + u * 256 + tid;
        v[u] = j < cols ? xr[j * es] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 8; u++) term(v[u]);
    }
  }
  s = wave_sum_f64(s);
  sa = wave_sum_f64(sa);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) emin = min(emin, __shfl_xor(emin, off, 64));
  if (lane == 0) {
    ls[wave] = s;
    la[wave] = sa;
    le[wave] = emin;
  }
  __syncthreads();
  s = ((ls[0] + ls[1]) + ls[2]) + ls[3];
  sa = ((la[0] + la[1]) + la[2]) + la[3];
  emin = min(min(le[0], le[1]), min(le[2], le[3]));
  float mean;
  if (!f64_mean_check(s, sa, emin, cols, &mean)) {   // the same outcome in every thread
    if (wave != 0) return;
    s = 0.0;
    for (int64_t j0 = 0; j0 < cols; j0 += 64) {
      const float v = j0 + lane < cols ? xr[(j0 + lane) * es] : 0.0f;
      s = seq_sum_lanes(s, v, (int)min<int64_t>(64, cols - j0));
    }
    mean = (float)(s / (double)cols);
  }
  if (tid == 0) p.out[row * p.ostride] = mean;
  if (p.ostride == 4 && tid >= 1 && tid <= 3) p.out[row * 4 + tid] = 0.0f;
}

int launch_reduce_mean_rows(const float* x, int64_t rows, int64_t cols, int64_t rpg,
                            int64_t gstride, int64_t rstride, int64_t estride, float* out,
                            int64_t ostride, hipStream_t s, const unsigned* rn, int64_t rpb) {
  if (rows >= (1ll << 33)) return fail(QPH_EUNSUPPORTED, "reduce_mean: too many rows");
  if (rows <= 0 || cols <= 0 || rpg <= 0) return fail(QPH_EINVAL, "reduce_mean: empty rows");
  MeanRows p{x, rows, cols, rpg, gstride, rstride, estride, out, ostride, rn, rpb};
  if (cols >= 1024 && rows < (1ll << 31)) {
    const bool vec = estride == 1 && (uintptr_t)x % 16 == 0 && gstride % 4 == 0 &&
                     rstride % 4 == 0;
    if (vec)
      hipLaunchKernelGGL(reduce_mean_wg_kernel<true>, dim3((unsigned)rows), dim3(256), 0, s, p);
    else
      hipLaunchKernelGGL(reduce_mean_wg_kernel<false>, dim3((unsigned)rows), dim3(256), 0, s, p);
    return launch_check("reduce_mean_wg_kernel");
  }
  hipLaunchKernelGGL(reduce_mean_kernel, dim3(ceil_div(rows, 4)), dim3(256), 0, s, p);
  return launch_check("reduce_mean_kernel");
}

int launch_reduce_mean(const float* x, int64_t rows, int64_t cols, float* out, hipStream_t s) {
  return launch_reduce_mean_rows(x, rows, cols, rows, 0, cols, 1, out, 1, s);
}

}  // namespace qph

using namespace qph;

extern "C" QPH_API int qph_reduce_mean_last(qph_ctx* ctx, const float* x, int64_t rows,
                                            int64_t cols, float* out) {
  if (!ctx) return fail(QPH_EINVAL, "null context");
  if (rows <= 0 || cols <= 0 || !x || !out) return fail(QPH_EINVAL, "reduce_mean: bad argument");
  return launch_reduce_mean(x, rows, cols, out, ctx->stream);
}
