// The rest of the det / cls / rec operator set around the hot path:
// pooling (global average, max / average), the SE gate's MulAddScale,
// bilinear resize, rank-4 transpose, and the steps either side of the
// networks (det input normalisation, rec line packing, the DB threshold and
// dilation).  All are bandwidth-bound: one thread per output element (or per
// four), coalesced along the fastest output axis, each output written once.
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
// (the reference's Mul-then-Add fallback, the same two roundings).
__global__ __launch_bounds__(256) void mul_add_scale_kernel(const float* __restrict__ f,
                                                            const float* __restrict__ gate,
                                                            const float* __restrict__ r,
                                                            float* __restrict__ out, int64_t c,
                                                            int64_t gmod, int64_t hw,
                                                            int64_t planes, int64_t ctot,
                                                            int64_t coff) {
  const int64_t total = planes * hw;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t p = i / hw, e = i - p * hw;
    const float v = f[i] * gate[p % gmod];
    out[out_plane(p, c, ctot, coff) * hw + e] = v + r[i];
  }
}

int launch_mul_add_scale(const float* f, const float* gate, const float* r, float* out, int64_t c,
                         int64_t gmod, int64_t hw, int64_t planes, int64_t ctot, int64_t coff,
                         hipStream_t s) {
  const int64_t total = planes * hw;
  if (total <= 0) return QPH_OK;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(mul_add_scale_kernel, dim3((unsigned)blocks), dim3(256), 0, s, f, gate, r,
                     out, c, gmod, hw, planes, ctot, coff);
  return launch_check("mul_add_scale_kernel");
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
};

__global__ __launch_bounds__(256) void pool2d_kernel(PoolK p) {
  const int64_t plane = blockIdx.y;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= p.oh * p.ow) return;
  const int64_t oy = idx / p.ow, ox = idx - oy * p.ow;
  const float* xp = p.x + plane * p.h * p.w;
  float v;
  if (p.special) {
    const float* r0 = xp + oy * p.w;
    const bool has_r1 = oy + 1 < p.h;
    const float a = has_r1 ? fmaxf(r0[ox], r0[ox + p.w]) : r0[ox];
    float b = -3.40282347e38f;
    if (ox + 1 < p.w) b = has_r1 ? fmaxf(r0[ox + 1], r0[ox + 1 + p.w]) : r0[ox + 1];
    v = fmaxf(a, b);
  } else {
    float acc = p.max_pool ? -3.4e38f : 0.0f;
    for (int64_t ky = 0; ky < p.kh; ky++) {
      const int64_t iy = oy * p.sh - p.ph + ky;
      if (iy < 0 || iy >= p.h) continue;
      for (int64_t kx = 0; kx < p.kw; kx++) {
        const int64_t ix = ox * p.sw - p.pw + kx;
        if (ix < 0 || ix >= p.w) continue;
        const float t = xp[iy * p.w + ix];
        acc = p.max_pool ? (t > acc ? t : acc) : acc + t;
      }
    }
    v = p.max_pool ? acc : acc / (float)(p.kh * p.kw);
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
  hipLaunchKernelGGL(pool2d_kernel, dim3(ceil_div(p.oh * p.ow, 256), (unsigned)(n * c)),
                     dim3(256), 0, s, p);
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

__global__ __launch_bounds__(256) void resize_bilinear_kernel(BilinearK p) {
  const int64_t plane = blockIdx.y;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= p.oh * p.ow) return;
  const int64_t oy = idx / p.ow, ox = idx - oy * p.ow;
  int64_t y0, y1, x0, x1;
  float ly, lx;
  bilinear_coord(oy, p.oh, p.h, p.align, y0, y1, ly);
  bilinear_coord(ox, p.ow, p.w, p.align, x0, x1, lx);
  const float* r0 = p.x + (plane * p.h + y0) * p.w;
  const float* r1 = p.x + (plane * p.h + y1) * p.w;
  float t = r0[x0] * (1.0f - lx) * (1.0f - ly);
  t = __builtin_fmaf(r0[x1] * lx, 1.0f - ly, t);
  t = __builtin_fmaf(r1[x0] * (1.0f - lx), ly, t);
  p.y[out_plane(plane, p.c, p.ctot, p.coff) * p.oh * p.ow + idx] =
      __builtin_fmaf(r1[x1] * lx, ly, t);
}

int launch_resize_bilinear(const float* x, int64_t n, int64_t c, int64_t h, int64_t w,
                           int64_t oh, int64_t ow, int align, float* y, int64_t ctot,
                           int64_t coff, hipStream_t s) {
  if (n * c > 65535 || oh * ow >= (1ll << 31))
    return fail(QPH_EUNSUPPORTED, "resize_bilinear: grid too large");
  BilinearK p{x, y, c, h, w, oh, ow, ctot, coff, align};
  hipLaunchKernelGGL(resize_bilinear_kernel, dim3(ceil_div(oh * ow, 256), (unsigned)(n * c)),
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
};

__global__ __launch_bounds__(256) void transpose4_kernel(TransposeK p) {
  for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < p.total;
       o += (int64_t)gridDim.x * blockDim.x) {
    int64_t r = o, src = 0;
#pragma unroll
    for (int d = 3; d >= 0; d--) {
      const int64_t i = r % p.ys[d];
      r /= p.ys[d];
      src += i * p.xst[d];
    }
    p.y[o] = p.x[src];
  }
}

int launch_transpose4(const float* x, const int64_t xs[4], const int32_t perm[4], float* y,
                      hipStream_t s) {
  TransposeK p{};
  p.x = x;
  p.y = y;
  int64_t st[4];
  st[3] = 1;
  for (int d = 2; d >= 0; d--) st[d] = st[d + 1] * xs[d + 1];
  for (int d = 0; d < 4; d++) {
    p.ys[d] = xs[perm[d]];
    p.xst[d] = st[perm[d]];
  }
  p.total = xs[0] * xs[1] * xs[2] * xs[3];
  if (p.total <= 0) return QPH_OK;
  int64_t blocks = (p.total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(transpose4_kernel, dim3((unsigned)blocks), dim3(256), 0, s, p);
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
// twelve bytes in (three dwords), four floats out per channel plane.
__global__ __launch_bounds__(256) void det_normalize_kernel(const uint8_t* __restrict__ rgb,
                                                            int64_t h, int64_t w,
                                                            float* __restrict__ out, int vec4) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // pixel quad
  const int64_t wq = (w + 3) / 4;
  const int64_t y = q / wq;
  if (y >= h) return;
  const int64_t x0 = (q - y * wq) * 4;
  const float scale = 1.0f / 255.0f, mean = 0.5f, istd = 1.0f / 0.5f;
  const uint8_t* src = rgb + (y * w + x0) * 3;
  const int n = (int)(w - x0 < 4 ? w - x0 : 4);
  float v[3][4];
#pragma unroll
  for (int k = 0; k < 4; k++)
#pragma unroll
    for (int c = 0; c < 3; c++) {
      const float u = k < n ? (float)src[k * 3 + c] : 0.0f;
      v[c][k] = (u * scale - mean) * istd;
    }
#pragma unroll
  for (int c = 0; c < 3; c++) {
    float* d = out + (c * h + y) * w + x0;
    if (n == 4 && vec4) {
      *(float4*)d = make_float4(v[c][0], v[c][1], v[c][2], v[c][3]);
    } else {
      for (int k = 0; k < n; k++) d[k] = v[c][k];
    }
  }
}

int launch_det_normalize(const uint8_t* rgb, int64_t h, int64_t w, float* out, hipStream_t s) {
  const int64_t quads = h * ((w + 3) / 4);
  if (quads >= (1ll << 40)) return fail(QPH_EUNSUPPORTED, "det_normalize: image too large");
  const int vec4 = (w & 3) == 0 && (uintptr_t)out % 16 == 0;   // 16-byte aligned rows
  hipLaunchKernelGGL(det_normalize_kernel, dim3(ceil_div(quads, 256)), dim3(256), 0, s, rgb, h, w,
                     out, vec4);
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
};

__global__ __launch_bounds__(256) void resize_rgb_u8_kernel(RgbResizeK p, uint8_t* __restrict__ dst) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= p.dw * p.dh) return;
  const int64_t y = idx / p.dw, x = idx - y * p.dw;
  int64_t j0, j1, x0, x1;
  float fy, lx;
  u8_axis(y, p.sy, p.sh, j0, j1, fy);
  u8_axis(x, p.sx, p.sw, x0, x1, lx);
  const uint8_t* r0 = p.src + j0 * p.sw * 3;
  const uint8_t* r1 = p.src + j1 * p.sw * 3;
#pragma unroll
  for (int ch = 0; ch < 3; ch++) dst[idx * 3 + ch] = u8_sample(r0, r1, x0 * 3, x1 * 3, lx, fy, ch);
}

int launch_resize_rgb_u8(const uint8_t* src, int64_t sw, int64_t sh, uint8_t* dst, int64_t dw,
                         int64_t dh, hipStream_t s) {
  RgbResizeK p{src, sw, sh, dw, dh, (float)sw / (float)dw, (float)sh / (float)dh};
  hipLaunchKernelGGL(resize_rgb_u8_kernel, dim3(ceil_div(dw * dh, 256)), dim3(256), 0, s, p, dst);
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

__global__ __launch_bounds__(256) void pack_crop_kernel(PackCropK p) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= p.img_h * p.img_w) return;
  const int64_t y = idx / p.img_w, x = idx - y * p.img_w;
  const int64_t plane = p.img_h * p.img_w;
  float v[3] = {0.0f, 0.0f, 0.0f};
  bool in = false;
  uint8_t u[3];
  if (p.pad_only) {
    const int64_t cy = y - p.y0;
    if (cy >= 0 && cy < p.ch && x < p.cw) {
      in = true;
#pragma unroll
      for (int c = 0; c < 3; c++) u[c] = p.crop[(cy * p.cw + x) * 3 + c];
    }
  } else if (x < p.rw) {
    in = true;
    int64_t j0, j1, x0, x1;
    float fy, lx;
    u8_axis(y, p.sy, p.ch, j0, j1, fy);
    u8_axis(x, p.sx, p.cw, x0, x1, lx);
    const uint8_t* r0 = p.crop + j0 * p.cw * 3;
    const uint8_t* r1 = p.crop + j1 * p.cw * 3;
#pragma unroll
    for (int c = 0; c < 3; c++) u[c] = u8_sample(r0, r1, x0 * 3, x1 * 3, lx, fy, c);
  }
  if (in) {
#pragma unroll
    for (int c = 0; c < 3; c++) v[c] = ((float)u[c] / 255.0f - 0.5f) / 0.5f;
  }
#pragma unroll
  for (int c = 0; c < 3; c++) p.dst[c * plane + idx] = v[c];
}

int launch_pack_crop(const uint8_t* crop, int64_t ch, int64_t cw, int64_t img_h, int64_t img_w,
                     float* dst, int pad_only, hipStream_t s) {
  PackCropK p{};
  p.crop = crop; p.dst = dst; p.ch = ch; p.cw = cw; p.img_h = img_h; p.img_w = img_w;
  p.pad_only = pad_only;
  p.y0 = (img_h - ch) / 2;
  if (!pad_only) {
    const float ratio = (float)cw / (float)ch;
    int64_t rw = (int64_t)__builtin_ceilf((float)img_h * ratio);
    rw = rw > img_w ? img_w : rw;
    p.rw = rw < 1 ? 1 : rw;
    p.sx = (float)cw / (float)p.rw;
    p.sy = (float)ch / (float)img_h;
  }
  hipLaunchKernelGGL(pack_crop_kernel, dim3(ceil_div(img_h * img_w, 256)), dim3(256), 0, s, p);
  return launch_check("pack_crop_kernel");
}

// ------------------------------------------- DB threshold + dilation
//
// qppocr-core/src/pipeline/geometry.rs:287-301 and dilate2x2_max
// (qppocr-kernels/src/resize.rs:219-247): mask = pred > thresh; with
// dilation out[y][x] = max of the in-range masks of rows y - 1, y and
// columns x - 1, x.  One pass: each thread thresholds its own window.
__global__ __launch_bounds__(256) void db_mask_kernel(const float* __restrict__ pred, int64_t h,
                                                      int64_t w, float thresh, int dilate,
                                                      uint8_t* __restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= h * w) return;
  const int64_t y = idx / w, x = idx - y * w;
  uint8_t v = pred[idx] > thresh ? 1 : 0;
  if (dilate) {
    if (x > 0 && pred[idx - 1] > thresh) v = 1;
    if (y > 0) {
      if (pred[idx - w] > thresh) v = 1;
      if (x > 0 && pred[idx - w - 1] > thresh) v = 1;
    }
  }
  out[idx] = v;
}

int launch_db_mask(const float* pred, int64_t h, int64_t w, float thresh, int dilate,
                   uint8_t* out, hipStream_t s) {
  hipLaunchKernelGGL(db_mask_kernel, dim3(ceil_div(h * w, 256)), dim3(256), 0, s, pred, h, w,
                     thresh, dilate, out);
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

QPH_API int qph_db_mask(qph_ctx* ctx, const float* pred, int64_t h, int64_t w, float thresh,
                        int32_t dilate, uint8_t* mask) {
  CTX_CHECK(ctx);
  if (h <= 0 || w <= 0 || !pred || !mask) return fail(QPH_EINVAL, "db_mask: bad argument");
  return launch_db_mask(pred, h, w, thresh, dilate != 0, mask, ctx->stream);
}

}  // extern "C"
