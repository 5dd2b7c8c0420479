// Convolution kernels: implicit-GEMM dense conv on fp32 MFMA, depthwise
// direct conv, 2x2 s2 ConvTranspose (single and the fused det-head pair).
#include "qph_internal.h"

namespace qph {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------ dense conv
//
// Reference: the implicit-GEMM branch of conv2d_res_into
// (qppocr-kernels/src/conv.rs:506-637 -> gemm.rs:75-128 -> x86.rs:134-444):
// per output row, C[co][ox] = sum_k W[co][k] * patch[k][ox] with
// k = (ci, ky, kx) ascending, zero-padded taps contributing fma(w, 0, acc),
// bias added after the chain (seeded in the M%4 tail of partial 32-column
// panels), then the activation.
//
// Kernel: a 256-thread workgroup owns WM*16 output channels x a TH x TW
// block of output pixels.  The input halo of the block (all or a chunk of
// the input channels) sits in LDS, zero-filled outside the image, so every
// tap is a plain LDS read.  Waves issue v_mfma_f32_16x16x4f32 (16 channels x
// 16 pixels, 4 k per instruction, each k its own fma in order).  Weights
// come from a k-major repack wk[Kpad][Mpad] (zero rows past K), so a lane
// reads W[co][k] as one coalesced word.

#define CONV_LDS_FLOATS 12288  // 48 KB halo budget per workgroup
#define CONV_KOFF_MAX 4096

// wk[k][mo] = w[mo][k] for k < kk, mo < m; zero elsewhere (Kpad x Mpad).
__global__ void repack_conv_w_kernel(const float* __restrict__ w, int64_t m, int64_t kk,
                                     int64_t kpad, int64_t mpad, float* __restrict__ wk) {
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= kpad * mpad) return;
  int64_t k = idx / mpad, mo = idx - k * mpad;
  wk[idx] = (k < kk && mo < m) ? w[mo * kk + k] : 0.0f;
}

static inline int64_t kpad_of(int64_t kk) { return (kk + 3) / 4 * 4; }
static inline int64_t mpad_of(int64_t m) { return (m + 31) / 32 * 32; }

int64_t dense_conv_wk_floats(int64_t m, int64_t cg, int64_t kh, int64_t kw) {
  return kpad_of(cg * kh * kw) * mpad_of(m);
}

int launch_repack_conv_w(const float* wt, int64_t m, int64_t kk, float* wk, hipStream_t s) {
  int64_t kpad = kpad_of(kk), mpad = mpad_of(m);
  int64_t total = kpad * mpad;
  hipLaunchKernelGGL(repack_conv_w_kernel, dim3(ceil_div(total, 256)), dim3(256), 0, s, wt, m,
                     kk, kpad, mpad, wk);
  return launch_check("repack_conv_w_kernel");
}

struct DenseConvK {
  const float* x;
  const float* wk;
  const float* bias;
  const float* res;
  float* y;
  int64_t c, h, w, m, mpad, kh, kw, sh, sw, ph, pw, oh, ow;
  int64_t y_ctotal, y_coff, y_up;
  int tw, th;          // pixel block: th rows x tw cols (th * tw = pixels per workgroup)
  int cchunk;          // input channels per LDS fill
  int rt, ct;          // halo rows / cols
  int tiles_x;         // pixel blocks along ow
  Act act;
};

// WM: waves along M (1: 16 channels, 4 waves along pixels; 2: 32 channels,
// 2 waves along pixels).  NT: 16-pixel MFMA tiles per wave.
template <int WM, int NT>
__global__ __launch_bounds__(256) void dense_conv_kernel(DenseConvK p) {
  constexpr int WP = 4 / WM;             // waves along pixels
  constexpr int PIX = WP * NT * 16;      // pixels per workgroup
  __shared__ float tile[CONV_LDS_FLOATS];
  __shared__ int koff[CONV_KOFF_MAX];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wp = wave / WM;
  const int64_t bn = blockIdx.z;
  const int64_t m0 = (int64_t)blockIdx.y * (16 * WM) + 16 * wm;
  const int tyb = blockIdx.x / p.tiles_x, txb = blockIdx.x - tyb * p.tiles_x;
  const int64_t oy0 = (int64_t)tyb * p.th, ox0 = (int64_t)txb * p.tw;
  const int64_t iy0 = oy0 * p.sh - p.ph, ix0 = ox0 * p.sw - p.pw;
  const int khkw = (int)(p.kh * p.kw);
  const int kk_total = (int)(p.c * khkw);
  const int plane = p.rt * p.ct;

  // per-lane pixel offsets into the halo tile for each of this wave's tiles
  int poff[NT];
  bool pval[NT];
  int64_t poy[NT], pox[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    int pix = (wp * NT + t) * 16 + (lane & 15);
    int py = pix / p.tw, px = pix - py * p.tw;
    poy[t] = oy0 + py;
    pox[t] = ox0 + px;
    pval[t] = pix < PIX && py < p.th && poy[t] < p.oh && pox[t] < p.ow;
    poff[t] = pval[t] ? (int)(py * p.sh * p.ct + px * p.sw) : 0;
  }

  // accumulators (bias-seeded where the reference seeds)
  f32x4 acc[NT];
  const int lg = lane >> 4;
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int v = 0; v < 4; v++) {
      float s0 = 0.0f;
      int64_t co = m0 + 4 * lg + v;
      if (p.bias && co < p.m && pval[t]) {
        int64_t n0 = (pox[t] >> 5) << 5;
        if ((p.ow - n0) < 32 && co >= p.m - p.m % 4) s0 = p.bias[co];
      }
      acc[t][v] = s0;
    }

  const float* xn = p.x + bn * p.c * p.h * p.w;
  for (int c0 = 0; c0 < p.c; c0 += p.cchunk) {
    const int cc = (int)((p.c - c0) < p.cchunk ? (p.c - c0) : p.cchunk);
    const int kloc = cc * khkw;
    __syncthreads();
    // halo fill: cc channels x rt rows x ct cols, zero outside the image
    for (int idx = tid; idx < cc * plane; idx += 256) {
      int ci = idx / plane, r = idx - ci * plane;
      int ry = r / p.ct, rx = r - ry * p.ct;
      int64_t iy = iy0 + ry, ix = ix0 + rx;
      float v = 0.0f;
      if (iy >= 0 && iy < p.h && ix >= 0 && ix < p.w) v = xn[((c0 + ci) * p.h + iy) * p.w + ix];
      tile[idx] = v;
    }
    for (int k = tid; k < ((kloc + 3) & ~3); k += 256) {
      int off = 0;
      if (k < kloc) {
        int ci = k / khkw, r = k - ci * khkw;
        int ky = r / (int)p.kw, kx = r - ky * (int)p.kw;
        off = ci * plane + ky * p.ct + kx;
      }
      koff[k] = off;
    }
    __syncthreads();
    const int kbase = c0 * khkw;
    const float* wkp = p.wk + (int64_t)kbase * p.mpad + m0 + (lane & 15);
    for (int k0 = 0; k0 < kloc; k0 += 4) {
      const int kl = k0 + lg;
      const float a = wkp[(int64_t)kl * p.mpad];  // zero past K (repack)
      const int ko = koff[kl];
#pragma unroll
      for (int t = 0; t < NT; t++) {
        float b = tile[ko + poff[t]];
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[t], 0, 0, 0);
      }
    }
  }
  (void)kk_total;

  // epilogue
  const int64_t yoh = p.oh * p.y_up, yow = p.ow * p.y_up;
#pragma unroll
  for (int t = 0; t < NT; t++) {
    if (!pval[t]) continue;
#pragma unroll
    for (int v = 0; v < 4; v++) {
      int64_t co = m0 + 4 * lg + v;
      if (co >= p.m) continue;
      float xv = acc[t][v];
      if (p.bias) {
        int64_t n0 = (pox[t] >> 5) << 5;
        bool seeded = (p.ow - n0) < 32 && co >= p.m - p.m % 4;
        if (!seeded) xv = xv + p.bias[co];
      }
      xv = act_apply(xv, p.act);
      if (p.res) xv = xv + p.res[((bn * p.m + co) * p.oh + poy[t]) * p.ow + pox[t]];
      float* yb = p.y + ((bn * p.y_ctotal + p.y_coff + co) * yoh) * yow;
      for (int dy = 0; dy < p.y_up; dy++)
        for (int dx = 0; dx < p.y_up; dx++)
          yb[(poy[t] * p.y_up + dy) * yow + pox[t] * p.y_up + dx] = xv;
    }
  }
}

int launch_dense_conv(const ConvArgs& a, hipStream_t s, float* scratch_wk) {
  const int64_t kk = a.c * a.kh * a.kw;
  const float* wk = a.wk;
  if (!wk) {
    if (!scratch_wk) return fail(QPH_EINVAL, "dense conv: no repacked weights");
    QPH_TRY(launch_repack_conv_w(a.wt, a.m, kk, scratch_wk, s));
    wk = scratch_wk;
  }
  DenseConvK p{};
  p.x = a.x; p.wk = wk; p.bias = a.bias; p.res = a.res; p.y = a.y;
  p.c = a.c; p.h = a.h; p.w = a.w; p.m = a.m; p.mpad = mpad_of(a.m);
  p.kh = a.kh; p.kw = a.kw; p.sh = a.sh; p.sw = a.sw; p.ph = a.ph; p.pw = a.pw;
  p.oh = a.oh; p.ow = a.ow;
  p.y_ctotal = a.y_ctotal; p.y_coff = a.y_coff; p.y_up = a.y_up;
  p.act = a.act;
  const bool wide_m = a.m > 16;
  // 2 MFMA tiles per wave; pixels per workgroup: 64 (WM=2) or 128 (WM=1)
  const int pix = wide_m ? 64 : 128;
  p.tw = a.ow >= 32 ? 32 : 16;
  p.th = pix / p.tw;
  p.rt = (int)((p.th - 1) * a.sh + a.kh);
  p.ct = (int)((p.tw - 1) * a.sw + a.kw);
  const int plane = p.rt * p.ct;
  // channel chunk: fits the halo budget, and each chunk's K is a multiple
  // of 4 so that MFMA k-groups never straddle two fills
  int khkw = (int)(a.kh * a.kw);
  int cch = CONV_LDS_FLOATS / plane;
  if (cch > CONV_KOFF_MAX / khkw) cch = CONV_KOFF_MAX / khkw;
  if (cch >= a.c) {
    cch = (int)a.c;
  } else {
    while (cch > 0 && (cch * khkw) % 4 != 0) cch--;
  }
  if (cch <= 0) return fail(QPH_EUNSUPPORTED, "dense conv: kernel too large for the LDS tile");
  p.cchunk = cch;
  p.tiles_x = (int)ceil_div(a.ow, p.tw);
  const int tiles_y = (int)ceil_div(a.oh, p.th);
  const int64_t mblk = wide_m ? 32 : 16;
  dim3 grid((unsigned)(p.tiles_x * tiles_y), ceil_div(a.m, mblk), (unsigned)a.n);
  if (a.n > 65535 || (int64_t)p.tiles_x * tiles_y > (1ll << 31))
    return fail(QPH_EUNSUPPORTED, "dense conv: grid too large");
  if (wide_m)
    hipLaunchKernelGGL((dense_conv_kernel<2, 2>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((dense_conv_kernel<1, 2>), grid, dim3(256), 0, s, p);
  return launch_check("dense_conv_kernel");
}

// --------------------------------------------------------------- depthwise
//
// Reference: conv.rs:461-505 + depthwise_plane_padded_avx2 (x86.rs:994-1060):
// acc = 0; for ky: for kx: acc = fma(w[ky][kx], xpad[oy*sh+ky][ox*sw+kx], acc);
// y = acc + bias; then act (hardswish = HardSigmoid + Mul nodes) and residual.
// Kernel: one workgroup per (plane, block of th x tw outputs); the input
// halo of the block is staged in LDS with the zero padding, each thread then
// computes outputs from LDS.  HBM-bound: each input and output element is
// read / written once.

#define DW_LDS_FLOATS 8192

struct DwK {
  const float* x;
  const float* w;
  const float* bias;
  const float* res;
  float* y;
  int64_t c, h, w_, kh, kw, sh, sw, ph, pw, oh, ow;
  int64_t y_ctotal, y_coff, y_up;
  int tw, th, rt, ct, tiles_x;
  Act act;
};

template <int KH, int KW>
__global__ __launch_bounds__(256) void depthwise_kernel(DwK p) {
  __shared__ float tile[DW_LDS_FLOATS];
  const int tid = threadIdx.x;
  const int64_t plane_id = blockIdx.y;  // n * c + ch
  const int64_t ch = plane_id % p.c;
  const int tyb = blockIdx.x / p.tiles_x, txb = blockIdx.x - tyb * p.tiles_x;
  const int64_t oy0 = (int64_t)tyb * p.th, ox0 = (int64_t)txb * p.tw;
  const int64_t iy0 = oy0 * p.sh - p.ph, ix0 = ox0 * p.sw - p.pw;
  const float* xp = p.x + plane_id * p.h * p.w_;
  const int tot = p.rt * p.ct;
  for (int idx = tid; idx < tot; idx += 256) {
    int ry = idx / p.ct, rx = idx - ry * p.ct;
    int64_t iy = iy0 + ry, ix = ix0 + rx;
    float v = 0.0f;
    if (iy >= 0 && iy < p.h && ix >= 0 && ix < p.w_) v = xp[iy * p.w_ + ix];
    tile[idx] = v;
  }
  float wr[KH * KW];
#pragma unroll
  for (int i = 0; i < KH * KW; i++) wr[i] = p.w[ch * KH * KW + i];
  const float bv = p.bias ? p.bias[ch] : 0.0f;
  __syncthreads();
  const int64_t bn = plane_id / p.c;
  const int64_t yoh = p.oh * p.y_up, yow = p.ow * p.y_up;
  float* yb = p.y + ((bn * p.y_ctotal + p.y_coff + ch) * yoh) * yow;
  const int npx = p.th * p.tw;
  for (int pix = tid; pix < npx; pix += 256) {
    int py = pix / p.tw, px = pix - py * p.tw;
    int64_t oy = oy0 + py, ox = ox0 + px;
    if (oy >= p.oh || ox >= p.ow) continue;
    const float* base = tile + py * p.sh * p.ct + px * p.sw;
    float acc = 0.0f;
#pragma unroll
    for (int ky = 0; ky < KH; ky++)
#pragma unroll
      for (int kx = 0; kx < KW; kx++) acc = __builtin_fmaf(wr[ky * KW + kx], base[ky * p.ct + kx], acc);
    float v = acc + bv;
    v = act_apply(v, p.act);
    if (p.res) v = v + p.res[(plane_id * p.oh + oy) * p.ow + ox];
    for (int dy = 0; dy < p.y_up; dy++)
      for (int dx = 0; dx < p.y_up; dx++) yb[(oy * p.y_up + dy) * yow + ox * p.y_up + dx] = v;
  }
}

int launch_depthwise(const ConvArgs& a, hipStream_t s) {
  DwK p{};
  p.x = a.x; p.w = a.wt; p.bias = a.bias; p.res = a.res; p.y = a.y;
  p.c = a.c; p.h = a.h; p.w_ = a.w; p.kh = a.kh; p.kw = a.kw; p.sh = a.sh; p.sw = a.sw;
  p.ph = a.ph; p.pw = a.pw; p.oh = a.oh; p.ow = a.ow;
  p.y_ctotal = a.y_ctotal; p.y_coff = a.y_coff; p.y_up = a.y_up;
  p.act = a.act;
  // block of up to 1024 outputs, 64 (or fewer for narrow planes) wide
  p.tw = a.ow >= 64 ? 64 : (a.ow >= 32 ? 32 : 16);
  p.th = 1024 / p.tw;
  if (p.th > a.oh) p.th = (int)a.oh;
  for (;;) {
    p.rt = (int)((p.th - 1) * a.sh + a.kh);
    p.ct = (int)((p.tw - 1) * a.sw + a.kw);
    if ((int64_t)p.rt * p.ct <= DW_LDS_FLOATS) break;
    if (p.th > 1) {
      p.th /= 2;
    } else if (p.tw > 16) {
      p.tw /= 2;
    } else {
      return fail(QPH_EUNSUPPORTED, "depthwise: kernel too large for the LDS tile");
    }
  }
  p.tiles_x = (int)ceil_div(a.ow, p.tw);
  const int64_t tiles = (int64_t)p.tiles_x * ceil_div(a.oh, p.th);
  const int64_t planes = a.n * a.c;
  if (planes > 65535 || tiles > (1ll << 31)) return fail(QPH_EUNSUPPORTED, "depthwise: grid too large");
  dim3 grid((unsigned)tiles, (unsigned)planes);
  if (a.kh == 3 && a.kw == 3)
    hipLaunchKernelGGL((depthwise_kernel<3, 3>), grid, dim3(256), 0, s, p);
  else if (a.kh == 5 && a.kw == 5)
    hipLaunchKernelGGL((depthwise_kernel<5, 5>), grid, dim3(256), 0, s, p);
  else if (a.kh == 7 && a.kw == 7)
    hipLaunchKernelGGL((depthwise_kernel<7, 7>), grid, dim3(256), 0, s, p);
  else
    return fail(QPH_EUNSUPPORTED, "depthwise: kernel sizes 3x3, 5x5, 7x7 only");
  return launch_check("depthwise_kernel");
}

// ----------------------------------------------------------- ConvTranspose
//
// Reference: convtranspose2d (conv.rs:730-804) + convt_row_scalar
// (conv.rs:816-838): out[co][2iy+ky][2ix+kx] = chain over ci ascending of
// fma(x[ci][iy][ix], w[ci][co][ky][kx], acc) from 0; no bias.

__global__ void convt2x2_kernel(const float* __restrict__ x, int64_t c, int64_t h, int64_t w,
                                const float* __restrict__ wt, int64_t m, float* __restrict__ y) {
  const int64_t pix = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t co = blockIdx.y;
  const int64_t bn = blockIdx.z;
  if (pix >= h * w) return;
  const int64_t iy = pix / w, ix = pix - iy * w;
  const float* xn = x + bn * c * h * w + pix;
  float a00 = 0.0f, a01 = 0.0f, a10 = 0.0f, a11 = 0.0f;
  for (int64_t ci = 0; ci < c; ci++) {
    float xv = xn[ci * h * w];
    const float* wc = wt + (ci * m + co) * 4;
    a00 = __builtin_fmaf(xv, wc[0], a00);
    a01 = __builtin_fmaf(xv, wc[1], a01);
    a10 = __builtin_fmaf(xv, wc[2], a10);
    a11 = __builtin_fmaf(xv, wc[3], a11);
  }
  const int64_t ow = 2 * w;
  float* yo = y + ((bn * m + co) * 2 * h + 2 * iy) * ow + 2 * ix;
  yo[0] = a00;
  yo[1] = a01;
  yo[ow] = a10;
  yo[ow + 1] = a11;
}

int launch_convt2x2(const float* x, int64_t n, int64_t c, int64_t h, int64_t w, const float* wt,
                    int64_t m, float* y, hipStream_t s) {
  if (m > 65535 || n > 65535) return fail(QPH_EUNSUPPORTED, "convT: grid too large");
  dim3 grid(ceil_div(h * w, 256), (unsigned)m, (unsigned)n);
  hipLaunchKernelGGL(convt2x2_kernel, grid, dim3(256), 0, s, x, c, h, w, wt, m, y);
  return launch_check("convt2x2_kernel");
}

// Det head tail: ConvT(C->M1) -> ConvT(M1->1) -> Sigmoid in one pass.  One
// thread per input pixel: the 2x2 block of the first ConvT (rounded to f32,
// as the intermediate tensor is) feeds a 2x2 block each of the second, so
// one input pixel produces a 4x4 block of the output.  Weights are read with
// wave-uniform (scalar) loads.
template <int C, int M1>
__global__ __launch_bounds__(256) void convt_pair_sigmoid_kernel(const float* __restrict__ x,
                                                                 int64_t h, int64_t w,
                                                                 const float* __restrict__ w1,
                                                                 const float* __restrict__ w2,
                                                                 float* __restrict__ y) {
  const int64_t pix = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t bn = blockIdx.y;
  if (pix >= h * w) return;
  const int64_t iy = pix / w, ix = pix - iy * w;
  float xv[C];
  const float* xn = x + bn * C * h * w + pix;
#pragma unroll
  for (int ci = 0; ci < C; ci++) xv[ci] = xn[ci * h * w];
  const int64_t ow = 4 * w;
  float* yo = y + (bn * 4 * h + 4 * iy) * ow + 4 * ix;
#pragma unroll
  for (int q = 0; q < 4; q++) {  // (ky, kx) of the first ConvT
    const int ky = q >> 1, kx = q & 1;
    float mid[M1];
#pragma unroll
    for (int co = 0; co < M1; co++) {
      float a = 0.0f;
#pragma unroll
      for (int ci = 0; ci < C; ci++) a = __builtin_fmaf(xv[ci], w1[(ci * M1 + co) * 4 + q], a);
      mid[co] = a;
    }
#pragma unroll
    for (int q2 = 0; q2 < 4; q2++) {
      float a = 0.0f;
#pragma unroll
      for (int co = 0; co < M1; co++) a = __builtin_fmaf(mid[co], w2[co * 4 + q2], a);
      const int oy = 2 * ky + (q2 >> 1), ox = 2 * kx + (q2 & 1);
      yo[oy * ow + ox] = sigmoid1(a);
    }
  }
}

// generic-size fallback of the pair kernel (C, M1 <= 64)
__global__ __launch_bounds__(256) void convt_pair_sigmoid_generic(const float* __restrict__ x,
                                                                  int64_t c, int64_t h, int64_t w,
                                                                  const float* __restrict__ w1,
                                                                  int64_t m1,
                                                                  const float* __restrict__ w2,
                                                                  float* __restrict__ y) {
  const int64_t pix = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t bn = blockIdx.y;
  if (pix >= h * w) return;
  const int64_t iy = pix / w, ix = pix - iy * w;
  const float* xn = x + bn * c * h * w + pix;
  const int64_t ow = 4 * w;
  float* yo = y + (bn * 4 * h + 4 * iy) * ow + 4 * ix;
  float mid[64];
  for (int q = 0; q < 4; q++) {
    const int ky = q >> 1, kx = q & 1;
    for (int64_t co = 0; co < m1; co++) {
      float a = 0.0f;
      for (int64_t ci = 0; ci < c; ci++) a = __builtin_fmaf(xn[ci * h * w], w1[(ci * m1 + co) * 4 + q], a);
      mid[co] = a;
    }
    for (int q2 = 0; q2 < 4; q2++) {
      float a = 0.0f;
      for (int64_t co = 0; co < m1; co++) a = __builtin_fmaf(mid[co], w2[co * 4 + q2], a);
      yo[(2 * ky + (q2 >> 1)) * ow + 2 * kx + (q2 & 1)] = sigmoid1(a);
    }
  }
}

int launch_convt2x2_pair_sigmoid(const float* x, int64_t n, int64_t c, int64_t h, int64_t w,
                                 const float* w1, int64_t m1, const float* w2, float* y,
                                 hipStream_t s) {
  if (n > 65535) return fail(QPH_EUNSUPPORTED, "convT pair: batch too large");
  dim3 grid(ceil_div(h * w, 256), (unsigned)n);
  if (c == 24 && m1 == 24)
    hipLaunchKernelGGL((convt_pair_sigmoid_kernel<24, 24>), grid, dim3(256), 0, s, x, h, w, w1, w2, y);
  else
    hipLaunchKernelGGL(convt_pair_sigmoid_generic, grid, dim3(256), 0, s, x, c, h, w, w1, m1, w2, y);
  return launch_check("convt_pair_sigmoid_kernel");
}

}  // namespace qph
