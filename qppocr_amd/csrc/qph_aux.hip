// The rest of the det / cls / rec operator set around the hot path:
// pooling (global average, max / average), the SE gate's MulAddScale,
// bilinear resize, rank-4 transpose, and the steps either side of the
// networks (det input normalisation, rec line packing, the DB threshold and
// dilation).  All are bandwidth-bound: one thread per output element (or per
// four), coalesced along the fastest output axis, each output written once.
#include <algorithm>

#include "qph_internal.h"

namespace qph {

// Output plane p (batch item p / c, channel p % c) of an op whose output may
// be a channel slice [coff, coff + c) of a tensor with ctot channels (the
// zero-copy Concat slot, executor.rs:1889-1916).
__device__ __forceinline__ int64_t out_plane(int64_t p, int64_t c, int64_t ctot, int64_t coff) {
  const int64_t bn = p / c;
  return bn * ctot + coff + (p - bn * c);
}

// ---------------------------------------------------------- MulAddScale
//
// mul_add_scale (qppocr-kernels/src/elementwise.rs:134-179):
// out = f * gate[plane % gmod] + r, the Mul and the Add each rounded; gmod =
// c for a per-channel gate, n * c for one gate per batch item and channel
// (the reference's Mul-then-Add fallback, the same two roundings).  With r
// NULL, out = f * gate alone: the gate Mul of an SE block without a
// residual (binary_op's inner-run path, elementwise.rs:366-420).
__global__ __launch_bounds__(256) void mul_add_scale_kernel(const float* __restrict__ f,
                                                            const float* __restrict__ gate,
                                                            const float* __restrict__ r,
                                                            float* __restrict__ out, int64_t c,
                                                            int64_t gmod, int64_t hw,
                                                            int64_t planes, int64_t ctot,
                                                            int64_t coff) {
  // a workgroup: 1024 elements of a plane (four coalesced passes); planes
  // by blockIdx.y, so no thread divides its index
  const int64_t e0 = (int64_t)blockIdx.x * 1024 + threadIdx.x;
  for (int64_t p = blockIdx.y; p < planes; p += gridDim.y) {
    const float g = gate[p % gmod];
    const float* fp = f + p * hw;
    const float* rp = r ? r + p * hw : nullptr;
    float* op = out + out_plane(p, c, ctot, coff) * hw;
    float fv[4], rv[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int64_t e = e0 + u * 256;
      fv[u] = e < hw ? fp[e] : 0.0f;
      rv[u] = (r && e < hw) ? rp[e] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const int64_t e = e0 + u * 256;
      const float v = fv[u] * g;
      if (e < hw) op[e] = r ? v + rv[u] : v;
    }
  }
}

int launch_mul_add_scale(const float* f, const float* gate, const float* r, float* out, int64_t c,
                         int64_t gmod, int64_t hw, int64_t planes, int64_t ctot, int64_t coff,
                         hipStream_t s) {
  if (planes <= 0 || hw <= 0) return QPH_OK;
  if (ceil_div(hw, 1024) >= (1ll << 31))
    return fail(QPH_EUNSUPPORTED, "mul_add_scale: plane too large");
  hipLaunchKernelGGL(mul_add_scale_kernel,
                     dim3((unsigned)ceil_div(hw, 1024), (unsigned)std::min<int64_t>(planes, 65535)),
                     dim3(256), 0, s, f, gate, r, out, c, gmod, hw, planes, ctot, coff);
  return launch_check("mul_add_scale_kernel");
}

// Division of n < 2^31 by a divisor d >= 1 fixed per launch: with l =
// ceil(log2 d) and M = ceil(2^(32 + l) / d) (at most 33 bits), floor(n / d)
// = (n * M) >> (32 + l), since M d - 2^(32 + l) < d keeps the product's
// excess over n / d below n / 2^(32 + l) < 1 / (2d) (Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994).
static void invariant_divisor(int64_t d, uint64_t* m, int* sh) {
  int l = 0;
  while ((1ll << l) < d) l++;
  const unsigned __int128 num = (unsigned __int128)1 << (32 + l);
  *m = (uint64_t)((num + (unsigned __int128)(d - 1)) / (unsigned __int128)d);
  *sh = 32 + l;
}

// ---------------------------------------------------------------- pool2d
//
// pool2d_into (qppocr-kernels/src/pool2d.rs:94-236):
//  - 2x2 stride 1 SAME_UPPER max (pads 0 / 1, output the input's size):
//    vm[j] = max(r0[j], r1[j]) (no r1 on the last row), vm[w] = -f32::MAX,
//    out[j] = max(vm[j], vm[j + 1]) (pool2x2_row_scalar, pool2d.rs:242-259);
//  - otherwise acc = -3.4e38 (max) or 0 (average), taps ky outer, kx inner,
//    out-of-range taps skipped; max keeps v > acc ? v : acc, average adds,
//    then divides by kh * kw (padding counted).
// Rust's f32::max is IEEE maxNum (fmaxf); the sign of a max of +0 and -0
// is unspecified there as here.
struct PoolK {
  const float* x;
  float* y;
  int64_t c, h, w, oh, ow, kh, kw, sh, sw, ph, pw;
  int64_t ctot, coff;
  int special, max_pool;
  uint64_t mag;   // oy = (idx * mag) >> shift: idx / ow for idx < oh * ow < 2^31
  int shift;
  int pair;       // 2x2 window, sw 2, pw 0, even w, 8-byte aligned x: float2 rows
};

// One thread per output of a plane (planes by blockIdx.y); K = the window's
// side when it is K x K (taps unrolled), 0 for any window.
template <int K>
__global__ __launch_bounds__(256) void pool2d_kernel(PoolK p) {
  const int64_t plane = blockIdx.y;
  const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
  if (idx >= (uint32_t)(p.oh * p.ow)) return;
  const uint32_t oyu = (uint32_t)(((uint64_t)idx * p.mag) >> p.shift);
  const int64_t oy = oyu, ox = idx - oyu * (uint32_t)p.ow;
  const float* xp = p.x + plane * p.h * p.w;
  float v;
  if (p.special) {
    const float* r0 = xp + oy * p.w;
    const bool has_r1 = oy + 1 < p.h;
    const float a = has_r1 ? fmaxf(r0[ox], r0[ox + p.w]) : r0[ox];
    float b = -3.40282347e38f;
    if (ox + 1 < p.w) b = has_r1 ? fmaxf(r0[ox + 1], r0[ox + 1 + p.w]) : r0[ox + 1];
    v = fmaxf(a, b);
  } else if (K == 2 && p.pair) {
    // 2x2, column stride 2, no column padding, even width: each window row is
    // one 8-byte load; taps still in the order (0,0), (0,1), (1,0), (1,1)
    float acc = p.max_pool ? -3.4e38f : 0.0f;
#pragma unroll
    for (int ky = 0; ky < 2; ky++) {
      const int64_t iy = oy * p.sh - p.ph + ky;
      if (iy < 0 || iy >= p.h) continue;
      const float2 t = *(const float2*)(xp + iy * p.w + 2 * ox);
      acc = p.max_pool ? (t.x > acc ? t.x : acc) : acc + t.x;
      acc = p.max_pool ? (t.y > acc ? t.y : acc) : acc + t.y;
    }
    v = p.max_pool ? acc : acc / 4.0f;
  } else {
    const int64_t kh = K ? K : p.kh, kw = K ? K : p.kw;
    float acc = p.max_pool ? -3.4e38f : 0.0f;
#pragma unroll(K > 0 ? K : 1)
    for (int64_t ky = 0; ky < kh; ky++) {
      const int64_t iy = oy * p.sh - p.ph + ky;
      if (iy < 0 || iy >= p.h) continue;
#pragma unroll(K > 0 ? K : 1)
      for (int64_t kx = 0; kx < kw; kx++) {
        const int64_t ix = ox * p.sw - p.pw + kx;
        if (ix < 0 || ix >= p.w) continue;
        const float t = xp[iy * p.w + ix];
        acc = p.max_pool ? (t > acc ? t : acc) : acc + t;
      }
    }
    v = p.max_pool ? acc : acc / (float)(kh * kw);
  }
  p.y[out_plane(plane, p.c, p.ctot, p.coff) * p.oh * p.ow + idx] = v;
}

void pool2d_out_hw(int64_t h, int64_t w, int64_t kh, int64_t kw, int64_t sh, int64_t sw,
                   int64_t ph, int64_t pw, int64_t peh, int64_t pew, int64_t* oh, int64_t* ow) {
  const int64_t hh = h + ph + peh, ww = w + pw + pew;
  *oh = (hh > kh ? hh - kh : 0) / sh + 1;
  *ow = (ww > kw ? ww - kw : 0) / sw + 1;
}

int launch_pool2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w, int64_t kh,
                  int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t peh,
                  int64_t pew, int max_pool, float* y, int64_t ctot, int64_t coff,
                  hipStream_t s) {
  PoolK p{};
  p.x = x; p.y = y; p.c = c; p.h = h; p.w = w;
  pool2d_out_hw(h, w, kh, kw, sh, sw, ph, pw, peh, pew, &p.oh, &p.ow);
  p.kh = kh; p.kw = kw; p.sh = sh; p.sw = sw; p.ph = ph; p.pw = pw;
  p.ctot = ctot; p.coff = coff;
  p.max_pool = max_pool;
  p.special = max_pool && kh == 2 && kw == 2 && sh == 1 && sw == 1 && ph == 0 && pw == 0 &&
              peh == 1 && pew == 1 && p.oh == h && p.ow == w;
  if (n * c > 65535 || p.oh * p.ow >= (1ll << 31))
    return fail(QPH_EUNSUPPORTED, "pool2d: grid too large");
  invariant_divisor(p.ow, &p.mag, &p.shift);
  // every window's two columns 2 ox, 2 ox + 1 lie inside the row (2 (ow - 1) + 1
  // <= w - 1 with pw = 0) and start 8-byte aligned when w is even
  p.pair = kh == 2 && kw == 2 && sw == 2 && pw == 0 && w % 2 == 0 &&
           (uintptr_t)x % 8 == 0 && 2 * (p.ow - 1) + 1 <= w - 1;
  const dim3 grid((unsigned)ceil_div(p.oh * p.ow, 256), (unsigned)(n * c));
  if (!p.special && kh == 2 && kw == 2)
    hipLaunchKernelGGL(pool2d_kernel<2>, grid, dim3(256), 0, s, p);
  else if (!p.special && kh == 3 && kw == 3)
    hipLaunchKernelGGL(pool2d_kernel<3>, grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(pool2d_kernel<0>, grid, dim3(256), 0, s, p);
  return launch_check("pool2d_kernel");
}

// ------------------------------------------------------ bilinear resize
//
// resize_bilinear_into (qppocr-kernels/src/resize.rs:60-142) with
// bilinear_row_scalar (resize.rs:252-273).  Source coordinate of output
// index i (f32): align_corners: i * (H - 1) / (oh - 1); otherwise
// max(0, (i + 0.5) * H / oh - 0.5); base = clamp(floor(v), 0, H - 1), next
// = min(base + 1, H - 1), frac = v - base.  Value:
// t = r0[i0] * (1 - lx) * (1 - ly); t = fma(r0[i1] * lx, 1 - ly, t);
// t = fma(r1[i0] * (1 - lx), ly, t); out = fma(r1[i1] * lx, ly, t).
__device__ __forceinline__ void bilinear_coord(int64_t i, int64_t n_out, int64_t n_in, int align,
                                               int64_t& i0, int64_t& i1, float& f) {
  float v;
  if (align && n_out > 1) {
    v = (float)i * (float)(n_in - 1) / (float)(n_out - 1);
  } else {
    v = ((float)i + 0.5f) * (float)n_in / (float)n_out - 0.5f;
    v = v > 0.0f ? v : 0.0f;
  }
  int64_t b = (int64_t)__builtin_floorf(v);
  b = b < 0 ? 0 : (b > n_in - 1 ? n_in - 1 : b);
  i0 = b;
  i1 = b + 1 < n_in - 1 ? b + 1 : n_in - 1;
  f = v - (float)b;
}

struct BilinearK {
  const float* x;
  float* y;
  int64_t c, h, w, oh, ow, ctot, coff;
  int align;
};

#define AUX_RY 8   // output rows per thread of the 2-D resize and mask kernels

// A workgroup: 256 output columns x AUX_RY output rows of one plane.  The
// rows' source coordinates are computed once (into LDS), each thread's
// column coordinate once for its AUX_RY outputs; row groups by blockIdx.y
// (strided past 65535 groups), planes by blockIdx.z.
__global__ __launch_bounds__(256) void resize_bilinear_kernel(BilinearK p) {
  __shared__ int64_t ry0[AUX_RY], ry1[AUX_RY];
  __shared__ float rly[AUX_RY];
  const int64_t plane = blockIdx.z;
  const int64_t ox = (int64_t)blockIdx.x * 256 + threadIdx.x;
  int64_t x0, x1;
  float lx;
  bilinear_coord(ox, p.ow, p.w, p.align, x0, x1, lx);
  const float* xp = p.x + plane * p.h * p.w;
  float* yp = p.y + out_plane(plane, p.c, p.ctot, p.coff) * p.oh * p.ow;
  for (int64_t oy0 = (int64_t)blockIdx.y * AUX_RY; oy0 < p.oh;
       oy0 += (int64_t)gridDim.y * AUX_RY) {
    __syncthreads();   // the previous group's reads of the row table are done
    if (threadIdx.x < AUX_RY) {
      int64_t a, b;
      float f;
      bilinear_coord(oy0 + threadIdx.x, p.oh, p.h, p.align, a, b, f);
      ry0[threadIdx.x] = a;
      ry1[threadIdx.x] = b;
      rly[threadIdx.x] = f;
    }
    __syncthreads();
    if (ox < p.ow) {
      const int nr = (int)std::min<int64_t>(p.oh - oy0, AUX_RY);
      for (int r = 0; r < nr; r++) {
        const float ly = rly[r];
        const float* r0 = xp + ry0[r] * p.w;
        const float* r1 = xp + ry1[r] * p.w;
        float t = r0[x0] * (1.0f - lx) * (1.0f - ly);
        t = __builtin_fmaf(r0[x1] * lx, 1.0f - ly, t);
        t = __builtin_fmaf(r1[x0] * (1.0f - lx), ly, t);
        yp[(oy0 + r) * p.ow + ox] = __builtin_fmaf(r1[x1] * lx, ly, t);
      }
    }
  }
}

int launch_resize_bilinear(const float* x, int64_t n, int64_t c, int64_t h, int64_t w,
                           int64_t oh, int64_t ow, int align, float* y, int64_t ctot,
                           int64_t coff, hipStream_t s) {
  if (n * c > 65535 || ceil_div(ow, 256) >= (1ll << 31))
    return fail(QPH_EUNSUPPORTED, "resize_bilinear: grid too large");
  BilinearK p{x, y, c, h, w, oh, ow, ctot, coff, align};
  hipLaunchKernelGGL(resize_bilinear_kernel,
                     dim3((unsigned)ceil_div(ow, 256),
                          (unsigned)std::min<int64_t>(ceil_div(oh, AUX_RY), 65535),
                          (unsigned)(n * c)),
                     dim3(256), 0, s, p);
  return launch_check("resize_bilinear_kernel");
}

// ------------------------------------------------------------- transpose
//
// Rank-4 Transpose (qppocr-core/src/executor.rs Transpose node): output
// dimension d is input dimension perm[d]; one thread per output element,
// writes coalesced.
struct TransposeK {
  const float* x;
  float* y;
  int64_t ys[4];
  int64_t xst[4];   // input stride of output dimension d's source dimension
  int64_t total;
  uint64_t mag[4];  // n / ys[d] = (n * mag[d]) >> sh[d] for n < 2^31 (32-bit form)
  int sh[4];
};

template <bool I32>
__global__ __launch_bounds__(256) void transpose4_kernel(TransposeK p) {
  for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < p.total;
       o += (int64_t)gridDim.x * blockDim.x) {
    int64_t src = 0;
    if constexpr (I32) {
      uint32_t r = (uint32_t)o;
#pragma unroll
      for (int d = 3; d >= 0; d--) {
        const uint32_t q = (uint32_t)(((uint64_t)r * p.mag[d]) >> p.sh[d]);
        src += (int64_t)(r - q * (uint32_t)p.ys[d]) * p.xst[d];
        r = q;
      }
    } else {
      int64_t r = o;
#pragma unroll
      for (int d = 3; d >= 0; d--) {
        const int64_t i = r % p.ys[d];
        r /= p.ys[d];
        src += i * p.xst[d];
      }
    }
    p.y[o] = p.x[src];
  }
}

// Tiled form, for a permutation that moves the input's contiguous axis:
// output axis 3 reads input axis A = perm[3] != 3.  A workgroup copies a
// 64 (axis A) x 64 (input axis 3) tile at one index of the two other input
// axes through LDS: its loads run along input axis 3, its stores along
// output axis 3 (input axis A), both contiguous.  The tile's rows are 65
// floats apart, so the column reads of the store phase fall on distinct
// banks.
struct TransposeTileK {
  const float* x;
  float* y;
  int64_t na, n3;         // sizes of input axes A and 3
  int64_t ia;             // input stride of axis A
  int64_t o3;             // output stride of the output axis input axis 3 lands on
  int64_t nc;             // size of the inner batch axis C
  int64_t ib, ic, ob, oc; // input / output strides of the batch axes B (outer), C
  int64_t tiles_a;        // tiles along axis A
};

// V4: n3 and every row start a multiple of 4 floats (16-byte aligned), so a
// thread loads 4 consecutive elements of a tile row at once.
template <bool V4>
__global__ __launch_bounds__(256) void transpose4_tile_kernel(TransposeTileK p) {
  __shared__ float t[64 * 65];
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const int64_t a0 = (int64_t)(blockIdx.x % p.tiles_a) * 64;
  const int64_t c0 = (int64_t)(blockIdx.x / p.tiles_a) * 64;
  const int64_t bb = blockIdx.y / p.nc, bc = blockIdx.y - bb * p.nc;
  const float* xb = p.x + bb * p.ib + bc * p.ic;
  float* yb = p.y + bb * p.ob + bc * p.oc;
  if constexpr (V4) {
    // 16 threads a tile row (4 columns each), 16 rows a pass
    const int cq = (threadIdx.x & 15) * 4, rq = threadIdx.x >> 4;
#pragma unroll
    for (int r = rq; r < 64; r += 16) {
      const int64_t a = a0 + r, c = c0 + cq;
      if (a < p.na && c < p.n3) {   // n3 % 4 == 0: the quad is whole
        const float4 v = *(const float4*)(xb + a * p.ia + c);
        t[r * 65 + cq] = v.x;
        t[r * 65 + cq + 1] = v.y;
        t[r * 65 + cq + 2] = v.z;
        t[r * 65 + cq + 3] = v.w;
      }
    }
  } else {
#pragma unroll 4
    for (int r = ty; r < 64; r += 4) {
      const int64_t a = a0 + r, c = c0 + tx;
      if (a < p.na && c < p.n3) t[r * 65 + tx] = xb[a * p.ia + c];
    }
  }
  __syncthreads();
#pragma unroll 4
  for (int r = ty; r < 64; r += 4) {
    const int64_t c = c0 + r, a = a0 + tx;
    if (a < p.na && c < p.n3) yb[c * p.o3 + a] = t[tx * 65 + r];
  }
}

int launch_transpose4(const float* x, const int64_t xs[4], const int32_t perm[4], float* y,
                      hipStream_t s) {
  if (perm[3] != 3) {
    // output strides, and the output stride of each input axis
    int64_t ost[4], o_in[4];
    ost[3] = 1;
    for (int d = 2; d >= 0; d--) ost[d] = ost[d + 1] * xs[perm[d + 1]];
    for (int d = 0; d < 4; d++) o_in[perm[d]] = ost[d];
    int64_t ist[4];
    ist[3] = 1;
    for (int d = 2; d >= 0; d--) ist[d] = ist[d + 1] * xs[d + 1];
    const int A = perm[3];
    int bax[2], nb = 0;
    for (int k = 0; k < 3; k++)
      if (k != A) bax[nb++] = k;
    TransposeTileK p{};
    p.x = x;
    p.y = y;
    p.na = xs[A];
    p.n3 = xs[3];
    p.ia = ist[A];
    p.o3 = o_in[3];
    p.nc = xs[bax[1]];
    p.ib = ist[bax[0]];
    p.ic = ist[bax[1]];
    p.ob = o_in[bax[0]];
    p.oc = o_in[bax[1]];
    p.tiles_a = ceil_div(p.na, 64);
    const int64_t tiles = p.tiles_a * ceil_div(p.n3, 64);
    const int64_t batch = xs[bax[0]] * xs[bax[1]];
    if (p.na * p.n3 >= 256 && batch <= 65535 && tiles < (1ll << 31)) {
      const dim3 grid((unsigned)tiles, (unsigned)batch);
      // row starts b * ib + c * ic + a * ia: 16-byte aligned when x is and
      // every input stride of axes 0..2 is a multiple of 4 (n3 % 4 == 0)
      if (p.n3 % 4 == 0 && (uintptr_t)x % 16 == 0)
        hipLaunchKernelGGL(transpose4_tile_kernel<true>, grid, dim3(256), 0, s, p);
      else
        hipLaunchKernelGGL(transpose4_tile_kernel<false>, grid, dim3(256), 0, s, p);
      return launch_check("transpose4_tile_kernel");
    }
  }
  TransposeK p{};
  p.x = x;
  p.y = y;
  int64_t st[4];
  st[3] = 1;
  for (int d = 2; d >= 0; d--) st[d] = st[d + 1] * xs[d + 1];
  for (int d = 0; d < 4; d++) {
    p.ys[d] = xs[perm[d]];
    p.xst[d] = st[perm[d]];
    invariant_divisor(p.ys[d], &p.mag[d], &p.sh[d]);
  }
  p.total = xs[0] * xs[1] * xs[2] * xs[3];
  if (p.total <= 0) return QPH_OK;
  int64_t blocks = (p.total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  // the 32-bit form: every index and grid-stride step stays below 2^31 + 2^24
  if (p.total < (1ll << 31))
    hipLaunchKernelGGL(transpose4_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(transpose4_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, s, p);
  return launch_check("transpose4_kernel");
}

// ----------------------------------------------- channel-slice copy
//
// Concat of a tensor that no producer can write in place (the graph input,
// a tensor with other readers): its planes copied into [coff, coff + c) of
// the concat output (executor.rs:1889-1916, the unaliased slots).
__global__ __launch_bounds__(256) void copy_slot_kernel(const float* __restrict__ x,
                                                        float* __restrict__ y, int64_t c,
                                                        int64_t hw, int64_t planes, int64_t ctot,
                                                        int64_t coff) {
  const int64_t total = planes * hw;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t p = i / hw, e = i - p * hw;
    y[out_plane(p, c, ctot, coff) * hw + e] = x[i];
  }
}

int launch_copy_slot(const float* x, float* y, int64_t c, int64_t hw, int64_t planes,
                     int64_t ctot, int64_t coff, hipStream_t s) {
  const int64_t total = planes * hw;
  if (total <= 0) return QPH_OK;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(copy_slot_kernel, dim3((unsigned)blocks), dim3(256), 0, s, x, y, c, hw,
                     planes, ctot, coff);
  return launch_check("copy_slot_kernel");
}

// ------------------------------------------- det input normalisation
//
// qppocr-core/src/pipeline/engine.rs:959-982: the det input from u8 RGB
// (interleaved, h x w x 3) to NCHW f32: v = u8 * (1 / 255) then
// (v - 0.5) * (1 / 0.5).  A thread takes four consecutive pixels of one row:
// twelve bytes in (three dwords when the rows allow), four floats out per
// channel plane.  Quads by blockIdx.x, rows by blockIdx.y (strided).
__global__ __launch_bounds__(256) void det_normalize_kernel(const uint8_t* __restrict__ rgb,
                                                            int64_t h, int64_t w,
                                                            float* __restrict__ out, int vec) {
  const int64_t qx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t wq = (w + 3) / 4;
  if (qx >= wq) return;
  const int64_t x0 = qx * 4;
  const float scale = 1.0f / 255.0f, mean = 0.5f, istd = 1.0f / 0.5f;
  const int n = (int)(w - x0 < 4 ? w - x0 : 4);
  for (int64_t y = blockIdx.y; y < h; y += gridDim.y) {
    const uint8_t* src = rgb + (y * w + x0) * 3;
    uint8_t b[12];
    if (vec) {   // w % 4 == 0: the quad's twelve bytes start 4-byte aligned
      const uint32_t* s32 = (const uint32_t*)src;
#pragma unroll
      for (int q = 0; q < 3; q++) {
        const uint32_t t = s32[q];
#pragma unroll
        for (int k = 0; k < 4; k++) b[4 * q + k] = (uint8_t)(t >> (8 * k));
      }
    } else {
#pragma unroll
      for (int i = 0; i < 12; i++) b[i] = i < 3 * n ? src[i] : 0;
    }
    float v[3][4];
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int c = 0; c < 3; c++) {
        const float u = k < n ? (float)b[k * 3 + c] : 0.0f;
        v[c][k] = (u * scale - mean) * istd;
      }
#pragma unroll
    for (int c = 0; c < 3; c++) {
      float* d = out + (c * h + y) * w + x0;
      if (vec) {
        *(float4*)d = make_float4(v[c][0], v[c][1], v[c][2], v[c][3]);
      } else {
        for (int k = 0; k < n; k++) d[k] = v[c][k];
      }
    }
  }
}

int launch_det_normalize(const uint8_t* rgb, int64_t h, int64_t w, float* out, hipStream_t s) {
  const int64_t wq = (w + 3) / 4;
  if (ceil_div(wq, 256) >= (1ll << 31))
    return fail(QPH_EUNSUPPORTED, "det_normalize: image too wide");
  // whole quads, 16-byte aligned output rows, 4-byte aligned input quads
  const int vec = (w & 3) == 0 && (uintptr_t)out % 16 == 0 && (uintptr_t)rgb % 4 == 0;
  hipLaunchKernelGGL(det_normalize_kernel,
                     dim3((unsigned)ceil_div(wq, 256), (unsigned)std::min<int64_t>(h, 65535)),
                     dim3(256), 0, s, rgb, h, w, out, vec);
  return launch_check("det_normalize_kernel");
}

// -------------------------------------------- u8 RGB bilinear resize
//
// resize_bilinear_rgb_u8 (qppocr-kernels/src/resize.rs:153-209; the same
// values as pipeline/image.rs resize_bilinear_img): half-pixel map with
// truncation, sx = sw / dw; the two-multiplies-then-fma weighting;
// (val + 0.5).clamp(0, 255) as u8.
__device__ __forceinline__ void u8_axis(int64_t i, float scale, int64_t n_in, int64_t& i0,
                                        int64_t& i1, float& f) {
  float v = ((float)i + 0.5f) * scale - 0.5f;
  v = v > 0.0f ? v : 0.0f;
  int64_t b = (int64_t)v;
  b = b > n_in - 1 ? n_in - 1 : b;
  i0 = b;
  i1 = b + 1 < n_in - 1 ? b + 1 : n_in - 1;
  f = v - (float)b;
}

__device__ __forceinline__ uint8_t u8_mix(float p00, float p01, float p10, float p11, float lx,
                                          float fy) {
  float t = p00 * (1.0f - lx) * (1.0f - fy);
  t = __builtin_fmaf(p01 * lx, 1.0f - fy, t);
  t = __builtin_fmaf(p10 * (1.0f - lx), fy, t);
  float val = __builtin_fmaf(p11 * lx, fy, t) + 0.5f;
  val = val < 0.0f ? 0.0f : (val > 255.0f ? 255.0f : val);
  return (uint8_t)val;
}

__device__ __forceinline__ uint8_t u8_sample(const uint8_t* r0, const uint8_t* r1, int64_t a,
                                             int64_t b, float lx, float fy, int ch) {
  const float p00 = r0[a + ch], p01 = r0[b + ch], p10 = r1[a + ch], p11 = r1[b + ch];
  float t = p00 * (1.0f - lx) * (1.0f - fy);
  t = __builtin_fmaf(p01 * lx, 1.0f - fy, t);
  t = __builtin_fmaf(p10 * (1.0f - lx), fy, t);
  float val = __builtin_fmaf(p11 * lx, fy, t) + 0.5f;
  val = val < 0.0f ? 0.0f : (val > 255.0f ? 255.0f : val);
  return (uint8_t)val;
}

struct RgbResizeK {
  const uint8_t* src;
  int64_t sw, sh, dw, dh;
  float sx, sy;
  int64_t total;   // source bytes
  int words;       // src 4-byte aligned: tap pairs by dword loads
};

// One thread per output pixel: columns by blockIdx.x, rows by blockIdx.y
// (strided past 65535 rows), so no thread divides its index.  (With one
// column of several rows a thread, its 12 byte gathers a pixel leave too few
// waves in flight.)
__global__ __launch_bounds__(256) void resize_rgb_u8_kernel(RgbResizeK p, uint8_t* __restrict__ dst) {
  const int64_t x = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (x >= p.dw) return;
  int64_t x0, x1;
  float lx;
  u8_axis(x, p.sx, p.sw, x0, x1, lx);
  for (int64_t y = blockIdx.y; y < p.dh; y += gridDim.y) {
    int64_t j0, j1;
    float fy;
    u8_axis(y, p.sy, p.sh, j0, j1, fy);
    const uint8_t* r0 = p.src + j0 * p.sw * 3;
    const uint8_t* r1 = p.src + j1 * p.sw * 3;
    uint8_t* d = dst + (y * p.dw + x) * 3;
    const int64_t o0 = (j0 * p.sw + x0) * 3, o1 = (j1 * p.sw + x0) * 3;
    const int64_t b0 = o0 & ~(int64_t)3, b1 = o1 & ~(int64_t)3;
    if (p.words && x1 == x0 + 1 && b0 + 12 <= p.total && b1 + 12 <= p.total) {
      // both taps of a row are the 6 bytes from o: three aligned dwords hold
      // them (o - base <= 3, so bytes up to base + 8)
      uint8_t q0[6], q1[6];
      const uint32_t* w0 = (const uint32_t*)(p.src + b0);
      const uint32_t* w1 = (const uint32_t*)(p.src + b1);
      const uint32_t a0 = w0[0], a1 = w0[1], a2 = w0[2];
      const uint32_t c0 = w1[0], c1 = w1[1], c2 = w1[2];
      const int s0 = (int)(o0 - b0) * 8, s1 = (int)(o1 - b1) * 8;
      const uint64_t lo0 = (uint64_t)a0 | ((uint64_t)a1 << 32);
      const uint64_t lo1 = (uint64_t)c0 | ((uint64_t)c1 << 32);
      const uint64_t v0 = s0 ? (lo0 >> s0) | ((uint64_t)a2 << (64 - s0)) : lo0;
      const uint64_t v1 = s1 ? (lo1 >> s1) | ((uint64_t)c2 << (64 - s1)) : lo1;
#pragma unroll
      for (int k = 0; k < 6; k++) {
        q0[k] = (uint8_t)(v0 >> (8 * k));
        q1[k] = (uint8_t)(v1 >> (8 * k));
      }
#pragma unroll
      for (int ch = 0; ch < 3; ch++)
        d[ch] = u8_mix(q0[ch], q0[3 + ch], q1[ch], q1[3 + ch], lx, fy);
    } else {
#pragma unroll
      for (int ch = 0; ch < 3; ch++) d[ch] = u8_sample(r0, r1, x0 * 3, x1 * 3, lx, fy, ch);
    }
  }
}

int launch_resize_rgb_u8(const uint8_t* src, int64_t sw, int64_t sh, uint8_t* dst, int64_t dw,
                         int64_t dh, hipStream_t s) {
  if (ceil_div(dw, 256) >= (1ll << 31)) return fail(QPH_EUNSUPPORTED, "resize_rgb_u8: too wide");
  RgbResizeK p{src, sw, sh, dw, dh, (float)sw / (float)dw, (float)sh / (float)dh,
               sw * sh * 3, (uintptr_t)src % 4 == 0};
  hipLaunchKernelGGL(resize_rgb_u8_kernel,
                     dim3((unsigned)ceil_div(dw, 256), (unsigned)std::min<int64_t>(dh, 65535)),
                     dim3(256), 0, s, p, dst);
  return launch_check("resize_rgb_u8_kernel");
}

// ----------------------------------------------------------- pack_crop
//
// qppocr-core/src/pipeline/crop.rs:153-190: a text-line crop (u8 RGB,
// ch x cw) into one [3, img_h, img_w] slot of the rec batch, in one pass
// (the resized u8 image never reaches memory): without pad_only the crop is
// resized to img_h x rw, rw = clamp(ceil(img_h * (cw / ch)), 1, img_w), with
// the u8 resize above; with pad_only it is centred at its own size (rows
// from (img_h - ch) / 2, columns < min(cw, img_w)).  Value
// (u8 / 255 - 0.5) / 0.5 (true divisions); every other position of the slot
// is 0 (the reference packs into a zero-filled batch).
struct PackCropK {
  const uint8_t* crop;
  float* dst;
  int64_t ch, cw, img_h, img_w, rw, y0;
  float sx, sy;
  int pad_only;
};

// The value of slot pixel (y, x) for one crop, channels in v (0 outside the
// crop's placed / resized area).
__device__ __forceinline__ void pack_pixel(const uint8_t* crop, int64_t ch, int64_t cw, int64_t rw,
                                           int64_t y0, float sx, float sy, int pad_only,
                                           int64_t y, int64_t x, float v[3]) {
  v[0] = v[1] = v[2] = 0.0f;
  bool in = false;
  uint8_t u[3];
  if (pad_only) {
    const int64_t cy = y - y0;
    if (cy >= 0 && cy < ch && x < cw) {
      in = true;
#pragma unroll
      for (int c = 0; c < 3; c++) u[c] = crop[(cy * cw + x) * 3 + c];
    }
  } else if (x < rw) {
    in = true;
    int64_t j0, j1, x0, x1;
    float fy, lx;
    u8_axis(y, sy, ch, j0, j1, fy);
    u8_axis(x, sx, cw, x0, x1, lx);
    const uint8_t* r0 = crop + j0 * cw * 3;
    const uint8_t* r1 = crop + j1 * cw * 3;
#pragma unroll
    for (int c = 0; c < 3; c++) u[c] = u8_sample(r0, r1, x0 * 3, x1 * 3, lx, fy, c);
  }
  if (in) {
#pragma unroll
    for (int c = 0; c < 3; c++) v[c] = ((float)u[c] / 255.0f - 0.5f) / 0.5f;
  }
}

__global__ __launch_bounds__(256) void pack_crop_kernel(PackCropK p) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= p.img_h * p.img_w) return;
  const int64_t y = idx / p.img_w, x = idx - y * p.img_w;
  const int64_t plane = p.img_h * p.img_w;
  float v[3];
  pack_pixel(p.crop, p.ch, p.cw, p.rw, p.y0, p.sx, p.sy, p.pad_only, y, x, v);
#pragma unroll
  for (int c = 0; c < 3; c++) p.dst[c * plane + idx] = v[c];
}

// A whole rec batch in one launch: up to PACK_LINES crops, their descriptors
// in the kernel arguments; line blockIdx.y fills slot blockIdx.y.
#define PACK_LINES 64
struct PackLine {
  const uint8_t* crop;
  int32_t ch, cw, rw, y0;
  float sx, sy;
  int32_t pad_only, pad;
};
struct PackCropsK {
  float* dst;
  int64_t img_h, img_w;
  uint64_t mag;   // idx / img_w = (idx * mag) >> shift (slot size < 2^31)
  int32_t shift;
  PackLine line[PACK_LINES];
};

__global__ __launch_bounds__(256) void pack_crops_kernel(PackCropsK p) {
  const PackLine& L = p.line[blockIdx.y];
  const int64_t plane = p.img_h * p.img_w;
  const uint32_t idx = blockIdx.x * 256u + threadIdx.x;
  if (idx >= (uint32_t)plane) return;
  const int64_t y = (int64_t)(((uint64_t)idx * p.mag) >> p.shift), x = idx - y * p.img_w;
  float v[3];
  pack_pixel(L.crop, L.ch, L.cw, L.rw, L.y0, L.sx, L.sy, L.pad_only, y, x, v);
  float* d = p.dst + (int64_t)blockIdx.y * 3 * plane;
#pragma unroll
  for (int c = 0; c < 3; c++) d[c * plane + idx] = v[c];
}

// The resized width and the axis scales of one crop (crop.rs:153-190).
static void pack_geometry(int64_t ch, int64_t cw, int64_t img_h, int64_t img_w, int pad_only,
                          int64_t* rw, int64_t* y0, float* sx, float* sy) {
  *y0 = (img_h - ch) / 2;
  *rw = 0;
  *sx = *sy = 0.0f;
  if (!pad_only) {
    const float ratio = (float)cw / (float)ch;
    int64_t r = (int64_t)__builtin_ceilf((float)img_h * ratio);
    r = r > img_w ? img_w : r;
    *rw = r < 1 ? 1 : r;
    *sx = (float)cw / (float)*rw;
    *sy = (float)ch / (float)img_h;
  }
}

int launch_pack_crops(int n, const uint8_t* const* crops, const int64_t* ch, const int64_t* cw,
                      const int32_t* pad_only, int64_t img_h, int64_t img_w, float* dst,
                      hipStream_t s) {
  if (img_h * img_w >= (1ll << 31)) return fail(QPH_EUNSUPPORTED, "pack_crops: slot too large");
  for (int i = 0; i < n; i++)
    if (ch[i] >= (1ll << 31) || cw[i] >= (1ll << 31))
      return fail(QPH_EUNSUPPORTED, "pack_crops: crop too large");
  PackCropsK p{};
  p.img_h = img_h;
  p.img_w = img_w;
  invariant_divisor(img_w, &p.mag, &p.shift);
  for (int b = 0; b < n; b += PACK_LINES) {
    const int m = std::min(PACK_LINES, n - b);
    p.dst = dst + (int64_t)b * 3 * img_h * img_w;
    for (int i = 0; i < m; i++) {
      PackLine& L = p.line[i];
      int64_t rw, y0;
      pack_geometry(ch[b + i], cw[b + i], img_h, img_w, pad_only[b + i], &rw, &y0, &L.sx, &L.sy);
      L.crop = crops[b + i];
      L.ch = (int32_t)ch[b + i];
      L.cw = (int32_t)cw[b + i];
      L.rw = (int32_t)rw;
      L.y0 = (int32_t)y0;
      L.pad_only = pad_only[b + i] != 0;
    }
    hipLaunchKernelGGL(pack_crops_kernel, dim3((unsigned)ceil_div(img_h * img_w, 256), (unsigned)m),
                       dim3(256), 0, s, p);
    QPH_TRY(launch_check("pack_crops_kernel"));
  }
  return QPH_OK;
}

int launch_pack_crop(const uint8_t* crop, int64_t ch, int64_t cw, int64_t img_h, int64_t img_w,
                     float* dst, int pad_only, hipStream_t s) {
  PackCropK p{};
  p.crop = crop; p.dst = dst; p.ch = ch; p.cw = cw; p.img_h = img_h; p.img_w = img_w;
  p.pad_only = pad_only;
  pack_geometry(ch, cw, img_h, img_w, pad_only, &p.rw, &p.y0, &p.sx, &p.sy);
  hipLaunchKernelGGL(pack_crop_kernel, dim3(ceil_div(img_h * img_w, 256)), dim3(256), 0, s, p);
  return launch_check("pack_crop_kernel");
}

// ------------------------------------------- DB threshold + dilation
//
// qppocr-core/src/pipeline/geometry.rs:287-301 and dilate2x2_max
// (qppocr-kernels/src/resize.rs:219-247): mask = pred > thresh; with
// dilation out[y][x] = max of the in-range masks of rows y - 1, y and
// columns x - 1, x.  One pass: each thread thresholds its own window.
// A thread: one column of AUX_RY rows (row groups by blockIdx.y, strided),
// carrying the masks of the row above (columns x - 1 and x) down the column.
__global__ __launch_bounds__(256) void db_mask_kernel(const float* __restrict__ pred, int64_t h,
                                                      int64_t w, float thresh, int dilate,
                                                      uint8_t* __restrict__ out) {
  const int64_t x = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (x >= w) return;
  for (int64_t y0 = (int64_t)blockIdx.y * AUX_RY; y0 < h; y0 += (int64_t)gridDim.y * AUX_RY) {
    bool up = false, upl = false;   // masks at (y - 1, x) and (y - 1, x - 1)
    if (dilate && y0 > 0) {
      const float* pr = pred + (y0 - 1) * w;
      up = pr[x] > thresh;
      upl = x > 0 && pr[x - 1] > thresh;
    }
    const int nr = (int)std::min<int64_t>(h - y0, AUX_RY);
    for (int r = 0; r < nr; r++) {
      const float* pr = pred + (y0 + r) * w;
      const bool m = pr[x] > thresh;
      const bool ml = dilate && x > 0 && pr[x - 1] > thresh;
      out[(y0 + r) * w + x] = (m || (dilate && (ml || up || upl))) ? 1 : 0;
      up = m;
      upl = ml;
    }
  }
}

int launch_db_mask(const float* pred, int64_t h, int64_t w, float thresh, int dilate,
                   uint8_t* out, hipStream_t s) {
  if (ceil_div(w, 256) >= (1ll << 31)) return fail(QPH_EUNSUPPORTED, "db_mask: map too wide");
  hipLaunchKernelGGL(db_mask_kernel,
                     dim3((unsigned)ceil_div(w, 256),
                          (unsigned)std::min<int64_t>(ceil_div(h, AUX_RY), 65535)),
                     dim3(256), 0, s, pred, h, w, thresh, dilate, out);
  return launch_check("db_mask_kernel");
}

}  // namespace qph

using namespace qph;

#define CTX_CHECK(ctx) \
  if (!(ctx)) return fail(QPH_EINVAL, "null context")

extern "C" {

QPH_API int qph_global_avg_pool(qph_ctx* ctx, const float* x, int64_t n, int64_t c, int64_t hw,
                                float* out) {
  CTX_CHECK(ctx);
  if (n <= 0 || c <= 0 || hw <= 0 || !x || !out)
    return fail(QPH_EINVAL, "global_avg_pool: bad argument");
  return launch_reduce_mean(x, n * c, hw, out, ctx->stream);
}

QPH_API int qph_mul_add_scale(qph_ctx* ctx, const float* feature, const float* gate,
                              const float* residual, int64_t n, int64_t c, int64_t hw,
                              float* out) {
  CTX_CHECK(ctx);
  if (n <= 0 || c <= 0 || hw <= 0 || !feature || !gate || !residual || !out)
    return fail(QPH_EINVAL, "mul_add_scale: bad argument");
  return launch_mul_add_scale(feature, gate, residual, out, c, c, hw, n * c, c, 0, ctx->stream);
}

QPH_API int qph_pool2d(qph_ctx* ctx, const float* x, const int64_t xs[4], int64_t kh, int64_t kw,
                       int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t peh, int64_t pew,
                       int32_t max_pool, float* y, int64_t ys_out[4]) {
  CTX_CHECK(ctx);
  if (!x || !y || !xs) return fail(QPH_EINVAL, "pool2d: NULL argument");
  for (int d = 0; d < 4; d++)
    if (xs[d] <= 0) return fail(QPH_EINVAL, "pool2d: empty input");
  if (kh <= 0 || kw <= 0 || sh <= 0 || sw <= 0 || ph < 0 || pw < 0 || peh < 0 || pew < 0)
    return fail(QPH_EINVAL, "pool2d: bad window");
  int64_t oh, ow;
  pool2d_out_hw(xs[2], xs[3], kh, kw, sh, sw, ph, pw, peh, pew, &oh, &ow);
  if (ys_out) {
    ys_out[0] = xs[0]; ys_out[1] = xs[1]; ys_out[2] = oh; ys_out[3] = ow;
  }
  return launch_pool2d(x, xs[0], xs[1], xs[2], xs[3], kh, kw, sh, sw, ph, pw, peh, pew,
                       max_pool != 0, y, xs[1], 0, ctx->stream);
}

QPH_API int qph_resize_bilinear(qph_ctx* ctx, const float* x, int64_t nc, int64_t h, int64_t w,
                                int64_t oh, int64_t ow, int32_t align_corners, float* y) {
  CTX_CHECK(ctx);
  if (nc <= 0 || h <= 0 || w <= 0 || oh <= 0 || ow <= 0 || !x || !y)
    return fail(QPH_EINVAL, "resize_bilinear: bad argument");
  return launch_resize_bilinear(x, 1, nc, h, w, oh, ow, align_corners != 0, y, nc, 0,
                                ctx->stream);
}

QPH_API int qph_transpose(qph_ctx* ctx, const float* x, const int64_t xs[4],
                          const int32_t perm[4], float* y) {
  CTX_CHECK(ctx);
  if (!x || !y || !xs || !perm) return fail(QPH_EINVAL, "transpose: NULL argument");
  int seen = 0;
  for (int d = 0; d < 4; d++) {
    if (xs[d] <= 0) return fail(QPH_EINVAL, "transpose: empty input");
    if (perm[d] < 0 || perm[d] > 3 || (seen >> perm[d]) & 1)
      return fail(QPH_EINVAL, "transpose: perm is not a permutation of 0..3");
    seen |= 1 << perm[d];
  }
  return launch_transpose4(x, xs, perm, y, ctx->stream);
}

QPH_API int qph_det_normalize_u8(qph_ctx* ctx, const uint8_t* rgb, int64_t h, int64_t w,
                                 float* out) {
  CTX_CHECK(ctx);
  if (h <= 0 || w <= 0 || !rgb || !out) return fail(QPH_EINVAL, "det_normalize: bad argument");
  return launch_det_normalize(rgb, h, w, out, ctx->stream);
}

QPH_API int qph_resize_bilinear_rgb_u8(qph_ctx* ctx, const uint8_t* src, int64_t sw, int64_t sh,
                                       uint8_t* dst, int64_t dw, int64_t dh) {
  CTX_CHECK(ctx);
  if (sw <= 0 || sh <= 0 || dw <= 0 || dh <= 0 || !src || !dst)
    return fail(QPH_EINVAL, "resize_rgb_u8: bad argument");
  return launch_resize_rgb_u8(src, sw, sh, dst, dw, dh, ctx->stream);
}

QPH_API int qph_pack_crop(qph_ctx* ctx, const uint8_t* crop, int64_t ch, int64_t cw,
                          int64_t img_h, int64_t img_w, int32_t pad_only, float* dst) {
  CTX_CHECK(ctx);
  if (ch <= 0 || cw <= 0 || img_h <= 0 || img_w <= 0 || !crop || !dst)
    return fail(QPH_EINVAL, "pack_crop: bad argument");
  if (pad_only && ch > img_h) return fail(QPH_EINVAL, "pack_crop: pad_only crop taller than img_h");
  return launch_pack_crop(crop, ch, cw, img_h, img_w, dst, pad_only != 0, ctx->stream);
}

QPH_API int qph_pack_crops(qph_ctx* ctx, int32_t n, const uint8_t* const* crops,
                           const int64_t* ch, const int64_t* cw, const int32_t* pad_only,
                           int64_t img_h, int64_t img_w, float* dst) {
  CTX_CHECK(ctx);
  if (n <= 0 || !crops || !ch || !cw || !pad_only || img_h <= 0 || img_w <= 0 || !dst)
    return fail(QPH_EINVAL, "pack_crops: bad argument");
  for (int32_t i = 0; i < n; i++) {
    if (!crops[i] || ch[i] <= 0 || cw[i] <= 0)
      return fail(QPH_EINVAL, "pack_crops: bad crop " + std::to_string(i));
    if (pad_only[i] && ch[i] > img_h)
      return fail(QPH_EINVAL, "pack_crops: pad_only crop " + std::to_string(i) +
                                  " taller than img_h");
  }
  return launch_pack_crops(n, crops, ch, cw, pad_only, img_h, img_w, dst, ctx->stream);
}

QPH_API int qph_db_mask(qph_ctx* ctx, const float* pred, int64_t h, int64_t w, float thresh,
                        int32_t dilate, uint8_t* mask) {
  CTX_CHECK(ctx);
  if (h <= 0 || w <= 0 || !pred || !mask) return fail(QPH_EINVAL, "db_mask: bad argument");
  return launch_db_mask(pred, h, w, thresh, dilate != 0, mask, ctx->stream);
}

}  // extern "C"
