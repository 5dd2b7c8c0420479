// Convolution kernels: implicit-GEMM dense conv on fp32 MFMA, depthwise
// direct conv, 2x2 s2 ConvTranspose (single and the fused det-head pair).
#include <algorithm>

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
// Kernel: a 256-thread workgroup owns MB = 16*WM output channels x a TH x TW
// block of output pixels.  Input channels are taken in chunks (multiples of
// 4): the input halo of the block and the chunk's weights (a k-major repack
// wk[Kpad][Mpad], Kpad = ceil(C/4)*4*T, zero past the real extent) are
// staged in LDS with direct buffer->LDS loads, all of a chunk in flight at
// once; lanes past the image edge or past C use an out-of-range buffer
// offset and read 0, which is the zero padding.  The waves then run
// v_mfma_f32_16x16x4f32 (16 channels x 16 pixels, 4 consecutive k per
// instruction, each k its own rounding, in order) from LDS only.  k advances
// over groups of four input channels: a group holds 4*T k values (T = kh*kw
// taps), i.e. T MFMA k-steps, and the LDS offset of each (step, lane) inside
// a group is a per-lane constant computed once.

#define CONV_LDS_FLOATS 16320  // 63.75 KB per workgroup: halo tile + weight slice

// Group g (blockIdx.y) of an ONNX [group * mg][kk] weight:
// wk[g][k][mo] = w[g * mg + mo][k] for k < kk, mo < mg; zero elsewhere
// (Kpad x Mpad per group).
__global__ void repack_conv_w_kernel(const float* __restrict__ w, int64_t mg, int64_t kk,
                                     int64_t kpad, int64_t mpad, float* __restrict__ wk) {
  int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= kpad * mpad) return;
  const int64_t g = blockIdx.y;
  int64_t k = idx / mpad, mo = idx - k * mpad;
  wk[g * kpad * mpad + idx] = (k < kk && mo < mg) ? w[(g * mg + mo) * kk + k] : 0.0f;
}

static inline int64_t mpad_of(int64_t m) { return (m + 31) / 32 * 32; }
static inline int64_t kpad_of(int64_t cg, int64_t khkw) { return (cg + 3) / 4 * 4 * khkw; }

int64_t dense_conv_wk_floats(int64_t m, int64_t cg, int64_t kh, int64_t kw, int64_t group) {
  return group * kpad_of(cg, kh * kw) * mpad_of(m / group);
}

int launch_repack_conv_w_taps(const float* wt, int64_t m, int64_t cg, int64_t khkw, float* wk,
                              hipStream_t s, int64_t group) {
  if (group < 1 || group > 65535 || m % group) return fail(QPH_EINVAL, "repack: bad group");
  const int64_t mg = m / group;
  int64_t kpad = kpad_of(cg, khkw), mpad = mpad_of(mg);
  int64_t total = kpad * mpad;
  hipLaunchKernelGGL(repack_conv_w_kernel, dim3(ceil_div(total, 256), (unsigned)group), dim3(256),
                     0, s, wt, mg, cg * khkw, kpad, mpad, wk);
  return launch_check("repack_conv_w_kernel");
}

struct DenseConvK {
  const float* x;
  const float* wk;
  const float* bias;
  const float* res;
  float* y;
  // c, m: input / output channels of one group (C/g, M/g); ctot, mtot: of
  // the tensors; group g reads channels [g c, g c + c), writes [g m, g m + m)
  int64_t c, h, w, m, mpad, kpad, kh, kw, sh, sw, ph, pw, oh, ow;
  int64_t ctot, mtot, group;
  int64_t y_ctotal, y_coff, y_up;
  int64_t seed_tile;   // 0: bias rule per output row (implicit GEMM, N = ow);
                       // > 0: im2col tiles of this many rows (N = rows * ow)
  int tw, th;          // pixel block: th rows x tw cols
  int cchunk;          // input channels per LDS fill (multiple of 4)
  int rt, ct;          // halo rows / cols
  int tiles_x;         // pixel blocks along ow
  Act act;
};

// Where the reference seeds the chain with the bias (gemm.rs:7-16, panel
// path): rows in the M % 4 tail of a 32-column panel narrower than 32.  The
// implicit-GEMM branch (conv.rs:595-637) runs one GEMM per output row (N =
// ow, column ox); the im2col branch (conv.rs:639-661, strides other than 1
// and 2) one per tile of seed_tile output rows (N = rows * ow, column
// (oy - tile start) * ow + ox).
__device__ __forceinline__ bool dense_bias_seeded(const DenseConvK& p, int64_t co, int64_t oy,
                                                  int64_t ox) {
  if (co < p.m - p.m % 4) return false;
  int64_t j = ox, n = p.ow;
  if (p.seed_tile > 0) {
    const int64_t t0 = oy / p.seed_tile * p.seed_tile;
    const int64_t rows = p.oh - t0 < p.seed_tile ? p.oh - t0 : p.seed_tile;
    j = (oy - t0) * p.ow + ox;
    n = rows * p.ow;
  }
  return n - ((j >> 5) << 5) < 32;
}

// Writes v to the up x up block of output pixel (oy, ox) (nearest upsample
// by an integer factor); rows as 16-byte stores when up is 4 or 8.
__device__ __forceinline__ void store_replicated(float* yb, int64_t yow, int64_t oy, int64_t ox,
                                                 int up, float v) {
  if (up == 1) {
    yb[oy * yow + ox] = v;
    return;
  }
  for (int dy = 0; dy < up; dy++) {
    float* r = yb + (oy * up + dy) * yow + ox * up;
    if (up % 4 == 0) {
      const float4 q = make_float4(v, v, v, v);
      for (int dx = 0; dx < up; dx += 4) *(float4*)(r + dx) = q;
    } else if (up == 2) {
      *(float2*)r = make_float2(v, v);
    } else {
      for (int dx = 0; dx < up; dx++) r[dx] = v;
    }
  }
}

// WM: waves along M (1: 16 channels, 4 waves along pixels; 2: 32 channels,
// 2 waves along pixels).  NT: 16-pixel MFMA tiles per wave.  T: taps (kh*kw),
// or 0 for any tap count (offsets computed per k-step instead of held in
// registers).  blockIdx.z = batch item * group + group index.
template <int WM, int NT, int T>
__global__ __launch_bounds__(256) void dense_conv_kernel(DenseConvK p) {
  constexpr int MB = 16 * WM;            // output channels per workgroup (4/WM waves along pixels)
  constexpr int TR = T > 0 ? T : 1;      // register arrays of the fixed-tap form
  __shared__ float lds[CONV_LDS_FLOATS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wp = wave / WM;
  const int lg = lane >> 4, l16 = lane & 15;
  const int64_t bn = blockIdx.z / p.group, grp = blockIdx.z - bn * p.group;
  const int taps = T > 0 ? T : (int)(p.kh * p.kw);
  const int64_t mblk0 = (int64_t)blockIdx.y * MB;
  const int64_t m0 = mblk0 + 16 * wm;
  const int tyb = blockIdx.x / p.tiles_x, txb = blockIdx.x - tyb * p.tiles_x;
  const int64_t oy0 = (int64_t)tyb * p.th, ox0 = (int64_t)txb * p.tw;
  const int iy0 = (int)(oy0 * p.sh - p.ph), ix0 = (int)(ox0 * p.sw - p.pw);
  const int plane = p.rt * p.ct;
  const int kw = (int)p.kw;
  const int H = (int)p.h, W = (int)p.w;

  // per-lane pixel offsets into the halo tile for each of this wave's tiles
  int poff[NT];
  bool pval[NT];
  int64_t poy[NT], pox[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    int pix = (wp * NT + t) * 16 + l16;
    int py = pix / p.tw, px = pix - py * p.tw;
    poy[t] = oy0 + py;
    pox[t] = ox0 + px;
    pval[t] = py < p.th && poy[t] < p.oh && pox[t] < p.ow;
    poff[t] = pval[t] ? (int)(py * p.sh * p.ct + px * p.sw) : 0;
  }
  // per-lane offset of k-step s inside a group of four channels:
  // k_local = 4 s + lg -> channel k_local / T, tap k_local % T
  auto step_off = [&](int s) {
    int kl = 4 * s + lg;
    int ci = kl / taps, tap = kl - ci * taps;
    int ky = tap / kw, kx = tap - ky * kw;
    return ci * plane + ky * p.ct + kx;
  };
  int goff[TR];
#pragma unroll
  for (int s = 0; s < TR; s++) goff[s] = T > 0 ? step_off(s) : 0;

  const float* bias_g = p.bias ? p.bias + grp * p.m : nullptr;
  // accumulators (bias-seeded where the reference seeds)
  f32x4 acc[NT];
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int v = 0; v < 4; v++) {
      float s0 = 0.0f;
      int64_t co = m0 + 4 * lg + v;
      if (bias_g && co < p.m && pval[t] && dense_bias_seeded(p, co, poy[t], pox[t]))
        s0 = bias_g[co];
      acc[t][v] = s0;
    }

  // input image (this group's channels) and repacked weights as buffer
  // resources: offsets past the end read as 0
  const float* xn = p.x + (bn * p.ctot + grp * p.c) * p.h * p.w;
  const __amdgpu_buffer_rsrc_t xr =
      __builtin_amdgcn_make_buffer_rsrc((void*)xn, 0, (int)(p.c * p.h * p.w * 4), 0x00020000);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.wk + grp * p.kpad * p.mpad), 0, (int)(p.kpad * p.mpad * 4), 0x00020000);
  const unsigned OOB = 0x80000000u;

  const int cpad = (int)((p.c + 3) / 4 * 4);
  for (int c0 = 0; c0 < cpad; c0 += p.cchunk) {
    const int cc = (cpad - c0) < p.cchunk ? (cpad - c0) : p.cchunk;  // multiple of 4
    float* tile = lds;
    float* wsl = lds + ((cc * plane + 63) & ~63);     // [cc*taps][MB]
    __syncthreads();
    // halo fill: cc channels x rt rows, one buffer->LDS load per 64 columns
    const int nrows = cc * p.rt;
    for (int rr = wave; rr < nrows; rr += 4) {
      const int ci = rr / p.rt, ry = rr - ci * p.rt;
      const int iy = iy0 + ry;
      const bool rowok = c0 + ci < p.c && iy >= 0 && iy < H;
      const unsigned rowbase = (unsigned)(((c0 + ci) * H + iy) * W);
      float* dst = tile + rr * p.ct;
      for (int x0 = 0; x0 < p.ct; x0 += 64) {
        if (lane < p.ct - x0) {
          const int ix = ix0 + x0 + lane;
          const unsigned off =
              (rowok && ix >= 0 && ix < W) ? (rowbase + (unsigned)ix) * 4u : OOB;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              xr, (__attribute__((address_space(3))) void*)(dst + x0), 4, off, 0, 0, 0);
        }
      }
    }
    // weight slice: rows c0*T .. (c0+cc)*T of wk, columns mblk0 .. +MB; one
    // load moves 64/MB consecutive rows
    {
      constexpr int RPL = 64 / MB;   // rows per load
      const int nkr = cc * taps;
      const int kr0 = c0 * taps;
      const int lr = lane / MB, lc = lane - lr * MB;
      for (int r0 = wave * RPL; r0 < nkr; r0 += 4 * RPL) {
        const int kr = r0 + lr;
        const unsigned off = kr < nkr
                                 ? (unsigned)(((int64_t)(kr0 + kr) * p.mpad + mblk0 + lc) * 4)
                                 : OOB;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            wr, (__attribute__((address_space(3))) void*)(wsl + r0 * MB), 4, off, 0, 0, 0);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const float* wl = wsl + 16 * wm + l16;
    for (int q = 0; q < cc / 4; q++) {
      const float* tq = tile + q * 4 * plane;
      const float* wq = wl + q * 4 * taps * MB;
      if constexpr (T > 0) {
        float a[T], b[T][NT];
#pragma unroll
        for (int s = 0; s < T; s++) {
          a[s] = wq[(4 * s + lg) * MB];
#pragma unroll
          for (int t = 0; t < NT; t++) b[s][t] = tq[goff[s] + poff[t]];
        }
#pragma unroll
        for (int s = 0; s < T; s++)
#pragma unroll
          for (int t = 0; t < NT; t++)
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s][t], acc[t], 0, 0, 0);
      } else {
        for (int s = 0; s < taps; s++) {
          const int go = step_off(s);
          const float a = wq[(4 * s + lg) * MB];
          float b[NT];
#pragma unroll
          for (int t = 0; t < NT; t++) b[t] = tq[go + poff[t]];
#pragma unroll
          for (int t = 0; t < NT; t++)
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b[t], acc[t], 0, 0, 0);
        }
      }
    }
  }

  // epilogue: operands (bias, residual) first, then finish and store (the
  // stores may alias the operands as far as the compiler knows)
  const int64_t yoh = p.oh * p.y_up, yow = p.ow * p.y_up;
  float badd[NT][4], rv[NT][4];
  bool hadd[NT][4], ok[NT][4];
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int64_t co = m0 + 4 * lg + v;
      ok[t][v] = pval[t] && co < p.m;
      hadd[t][v] = false;
      badd[t][v] = 0.0f;
      rv[t][v] = 0.0f;
      if (!ok[t][v]) continue;
      if (bias_g && !dense_bias_seeded(p, co, poy[t], pox[t])) {
        badd[t][v] = bias_g[co];
        hadd[t][v] = true;
      }
      if (p.res)
        rv[t][v] = p.res[((bn * p.mtot + grp * p.m + co) * p.oh + poy[t]) * p.ow + pox[t]];
    }
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int v = 0; v < 4; v++) {
      if (!ok[t][v]) continue;
      const int64_t co = m0 + 4 * lg + v;
      float xv = acc[t][v];
      if (hadd[t][v]) xv = xv + badd[t][v];
      xv = act_apply(xv, p.act);
      if (p.res) xv = xv + rv[t][v];
      float* yb = p.y + ((bn * p.y_ctotal + p.y_coff + grp * p.m + co) * yoh) * yow;
      store_replicated(yb, yow, poy[t], pox[t], (int)p.y_up, xv);
    }
}

// ------------------------------------------------------- direct 3x3 conv
//
// The 3x3 dense convs of the det neck/head and the stems (C up to a few
// hundred, M <= 64, any stride and padding): the same k-ascending fma chain
// per output as the implicit-GEMM kernel above (k = (ci, ky, kx), bias after
// the chain or seeded by the same panel rule), with no LDS at all.
//
// One wave owns MT 16-channel blocks x NPX runs of 16 consecutive output
// pixels (row-major over oh x ow) and walks k in groups of four input
// channels (36 k = 9 v_mfma_f32_16x16x4f32 steps).  Lane (n = lane % 16,
// g = lane / 16) supplies k = 4s + g of step s: its input word is read
// straight from HBM / L2 with a buffer load whose per-lane offset is fixed
// for the whole K loop (the buffer base moves by four channels per group),
// and out-of-image taps or channels past C carry an offset past the buffer
// range, which reads 0 -- the zero padding.  Weights come from the k-major
// repack wk[Kpad][Mpad] (one 64-byte row segment per lane group).  The next
// group's operands are loaded into registers while the current group's
// MFMAs run, and every wave is independent (no barriers), so the many waves
// of a launch hide the load latency for each other.

struct DirectConvK {
  const float* x;
  const float* wk;
  const float* bias;
  const float* res;
  float* y;
  int c, h, w, m, mpad, sh, sw, ph, pw, oh, ow;
  int64_t y_ctotal, y_coff, y_up;
  int units_m, units_px, units;
  Act act;
};

// Work unit u (a wave-uniform index) of the conv described by p.
template <int MT, int NPX, int D>
__device__ __forceinline__ void direct3x3_unit(const DirectConvK& p, int u, int lane) {
  const int mu = u % p.units_m, rest = u / p.units_m;
  const int pu = rest % p.units_px, img = rest / p.units_px;
  const int l16 = lane & 15, lg = lane >> 4;
  const int m0 = mu * 16 * MT;
  const int npx = p.oh * p.ow, HW = p.h * p.w;
  const unsigned OOB = 0x80000000u;

  int poy[NPX], pox[NPX];
  bool pval[NPX];
  unsigned voff[NPX][9];
#pragma unroll
  for (int t = 0; t < NPX; t++) {
    const int pix = (pu * NPX + t) * 16 + l16;
    pval[t] = pix < npx;
    poy[t] = pix / p.ow;
    pox[t] = pix - poy[t] * p.ow;
#pragma unroll
    for (int s = 0; s < 9; s++) {
      const int kl = 4 * s + lg, cl = kl / 9, tap = kl - 9 * cl;
      const int ky = tap / 3, kx = tap - 3 * ky;
      const int iy = poy[t] * p.sh - p.ph + ky, ix = pox[t] * p.sw - p.pw + kx;
      const bool ok = pval[t] && iy >= 0 && iy < p.h && ix >= 0 && ix < p.w;
      // offsets of 2^31 and up lie past every range (the image is < 2 GB)
      const int64_t off = ((int64_t)cl * HW + (int64_t)iy * p.w + ix) * 4;
      voff[t][s] = ok && off < (int64_t)OOB ? (unsigned)off : OOB;
    }
  }

  // accumulators, bias-seeded where the reference seeds (M%4 tail rows of a
  // partial 32-column panel of the output row)
  f32x4 acc[MT][NPX];
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
#pragma unroll
    for (int t = 0; t < NPX; t++)
#pragma unroll
      for (int v = 0; v < 4; v++) {
        float s0 = 0.0f;
        const int co = m0 + mt * 16 + 4 * lg + v;
        if (p.bias && co < p.m && pval[t]) {
          const int n0 = (pox[t] >> 5) << 5;
          if ((p.ow - n0) < 32 && co >= p.m - p.m % 4) s0 = p.bias[co];
        }
        acc[mt][t][v] = s0;
      }

  const float* xi = p.x + (int64_t)img * p.c * HW;
  const unsigned woff = (unsigned)(lg * p.mpad + m0 + l16) * 4u;
  const int ng = (p.c + 3) / 4;
  const int w_words = ng * 36 * p.mpad;
  // D register buffers: the loads of groups g+1 .. g+D-1 are in flight
  // while group g's MFMAs run
  float ab[D][MT][9], bb[D][NPX][9];
  auto load = [&](int g, float (&a)[MT][9], float (&b)[NPX][9]) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(xi + (int64_t)g * 4 * HW), 0, (p.c - 4 * g) * HW * 4, 0x00020000);
#pragma unroll
    for (int s = 0; s < 9; s++)
#pragma unroll
      for (int t = 0; t < NPX; t++)
        b[t][s] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff[t][s], 0, 0));
    // weights: the lane part of the offset is fixed, the step part uniform
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.wk + g * 36 * p.mpad), 0, (w_words - g * 36 * p.mpad) * 4, 0x00020000);
#pragma unroll
    for (int s = 0; s < 9; s++)
#pragma unroll
      for (int mt = 0; mt < MT; mt++)
        a[mt][s] = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(wr, woff, (4 * s * p.mpad + mt * 16) * 4, 0));
  };
  auto mma = [&](const float (&a)[MT][9], const float (&b)[NPX][9]) {
#pragma unroll
    for (int s = 0; s < 9; s++)
#pragma unroll
      for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int t = 0; t < NPX; t++)
          acc[mt][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[mt][s], b[t][s], acc[mt][t], 0, 0, 0);
  };

  // Loads are issued unconditionally (groups past the end reload the last
  // group, unused) so that every path has the same loads in flight and the
  // waits before each group's MFMAs stay partial.
#pragma unroll
  for (int j = 0; j < D - 1; j++) load(min(j, ng - 1), ab[j], bb[j]);
  for (int g = 0; g < ng; g += D) {
#pragma unroll
    for (int j = 0; j < D; j++) {
      load(min(g + j + D - 1, ng - 1), ab[(j + D - 1) % D], bb[(j + D - 1) % D]);
      if (g + j < ng) mma(ab[j], bb[j]);
    }
  }

  // epilogue: operands (bias, residual) first, then finish and store
  const int64_t yoh = (int64_t)p.oh * p.y_up, yow = (int64_t)p.ow * p.y_up;
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    float badd[NPX][4], rv[NPX][4];
    bool hadd[NPX][4], ok[NPX][4];
#pragma unroll
    for (int t = 0; t < NPX; t++)
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const int co = m0 + mt * 16 + 4 * lg + v;
        ok[t][v] = pval[t] && co < p.m;
        hadd[t][v] = false;
        badd[t][v] = 0.0f;
        rv[t][v] = 0.0f;
        if (!ok[t][v]) continue;
        if (p.bias) {
          const int n0 = (pox[t] >> 5) << 5;
          const bool seeded = (p.ow - n0) < 32 && co >= p.m - p.m % 4;
          if (!seeded) {
            badd[t][v] = p.bias[co];
            hadd[t][v] = true;
          }
        }
        if (p.res) rv[t][v] = p.res[(((int64_t)img * p.m + co) * p.oh + poy[t]) * p.ow + pox[t]];
      }
#pragma unroll
    for (int t = 0; t < NPX; t++)
#pragma unroll
      for (int v = 0; v < 4; v++) {
        if (!ok[t][v]) continue;
        const int co = m0 + mt * 16 + 4 * lg + v;
        float xv = acc[mt][t][v];
        if (hadd[t][v]) xv = xv + badd[t][v];
        xv = act_apply(xv, p.act);
        if (p.res) xv = xv + rv[t][v];
        float* yb = p.y + (((int64_t)img * p.y_ctotal + p.y_coff + co) * yoh) * yow;
        store_replicated(yb, yow, poy[t], pox[t], (int)p.y_up, xv);
      }
  }
}

template <int MT, int NPX, int D>
__global__ __launch_bounds__(256) void conv3x3_direct_kernel(DirectConvK p) {
  // wave index as a scalar: everything derived from it (image, channel
  // block, buffer bases) stays in SGPRs
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int u = blockIdx.x * 4 + wave;
  if (u >= p.units) return;
  direct3x3_unit<MT, NPX, D>(p, u, lane);
}

// Up to four independent 3x3 convs in one launch (the det neck's four
// smoothing convs, which read different levels and write disjoint channel
// slots of the concat): waves [start[i], start[i+1]) work on conv i.
#define DIRECT_GROUP_MAX 4
struct DirectConvGroup {
  DirectConvK k[DIRECT_GROUP_MAX];
  int start[DIRECT_GROUP_MAX + 1];
  int n;
};

__global__ __launch_bounds__(256) void conv3x3_direct_group_kernel(DirectConvGroup g) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int u = blockIdx.x * 4 + wave;
  if (u >= g.start[g.n]) return;
  if (u < g.start[1]) direct3x3_unit<1, 1, 4>(g.k[0], u, lane);
  else if (u < g.start[2]) direct3x3_unit<1, 1, 4>(g.k[1], u - g.start[1], lane);
  else if (u < g.start[3]) direct3x3_unit<1, 1, 4>(g.k[2], u - g.start[2], lane);
  else direct3x3_unit<1, 1, 4>(g.k[3], u - g.start[3], lane);
}

// ---------------------------------------------- LDS-staged 3x3 conv
//
// Stride 1, pad 1, M <= 32, C a multiple of 8 (the det neck smoothing convs
// and the det head conv, 96 -> 24): the same chain as direct3x3_unit (k =
// ci * 9 + ky * 3 + kx ascending, four per v_mfma_f32_16x16x4f32 step, bias
// after the chain or seeded by the panel rule, then the activation, the
// residual and the replicated store), but with both operands out of LDS.
// A workgroup owns 2 output rows x 32 columns: wave w the 16 pixels of row
// w / 2 from column 16 (w % 2), both 16-channel blocks of M.  K advances in
// chunks of 8 input channels (72 k = 18 steps) through a ring of three LDS
// stages, two chunks in flight while one is multiplied: the chunk's input
// halo (8 x 4 rows x 40 columns from column ox0 - 4, out-of-image words read
// 0 = the zero padding) and its 72 weight rows of the k-major repack (32
// floats each, 16-float halves swapped on rows with k & 2 so that the four k
// rows of one step hit distinct banks) arrive by 16-byte buffer->LDS loads:
// 5 for the halo, 9 for the weights and 2 spare ones (out of range, into a
// spare area) so that every wave issues exactly 4 a chunk and each wait
// counts exactly the chunks still loading.  The image width is a multiple of
// 4, so a 16-byte halo group lies wholly inside or wholly outside a row.
// Each direct3x3_unit step costs two vector-memory loads per lane; here a
// step is three LDS reads and two MFMAs.

#define LC_CC 8                         // input channels per chunk
#define LC_HP 40                        // halo row pitch (4 + 32 + 4 columns)
#define LC_HG 10                        // 16-byte groups per halo row
#define LC_HALO (LC_CC * 4 * LC_HP)     // 1280 floats: 5 loads of 64 groups
#define LC_NST 3                        // ring stages
#define LC_WROWS (LC_CC * 9)            // 72 weight rows per chunk
#define LC_W (LC_WROWS * 32)            // 2304 floats: 9 loads
#define LC_SPARE 512                    // 2 loads' worth of spare words
#define LC_STAGE (LC_HALO + LC_W + LC_SPARE)
#define LC_DMA (LC_STAGE / 256)         // 16 loads per chunk, 4 per wave
#define LC_LEAD 6                       // steps the operand reads run ahead (C = 32)
#define LC_LEAD_RING 2                  // the same in the ring form (C > 32)

// The det head's conv-transpose pair and sigmoid, run in the epilogue of the
// 3x3 conv before it (CVT): w1 [24][24][2][2] and w2 [24][1][2][2] in their
// ONNX layouts, y [n][1][4 oh][4 ow].
struct ConvtEpi {
  const float* w1;
  const float* w2;
  float* y;
};
#define CV_C 24    // channels of the conv output and of the first ConvT
#define CV_HP 28   // LDS pitch of a pixel's 24 conv outputs (16-byte rows)

struct LdsConvGroup {
  DirectConvK k[DIRECT_GROUP_MAX];
  int tiles_x[DIRECT_GROUP_MAX];
  int start[DIRECT_GROUP_MAX + 1];   // start[i] = total for i >= n
  int n;
};

// The ring stages are three __shared__ arrays of their own, picked at compile
// time (the chunk loop is unrolled over the ring): that is what lets the
// compiler tell the loads into one stage from the reads of another and place
// no wait of its own before the operand reads.  The fixed costs around the
// chunk loop are kept short: the first two chunks' loads go out before
// anything else is read (bias terms included), a chunk's operands are all
// read from LDS before its MFMAs (so the reads' latency is paid once a chunk,
// not once a step), and AK (0 none, 2 ReLU, -1 any kind through act_apply)
// keeps the epilogue free of the generic activation switch.
template <int AK, bool ONE, bool CVT = false>
__device__ __forceinline__ void lds_conv_tile(const DirectConvK& p, int tiles_x, int tile,
                                              float* s0, float* s1, float* s2, float* s3,
                                              int wave, int lane,
                                              const ConvtEpi& cv = ConvtEpi{}) {
  // every parameter the loads depend on, fetched in one batch of scalar
  // loads (left alone, the compiler fetches them in dependent rounds as the
  // code first uses them, each round a full kernel-argument load latency)
  __asm__ volatile("" ::"s"(p.x), "s"(p.wk), "s"(p.c), "s"(p.h), "s"(p.w), "s"(p.oh),
                   "s"(p.ow), "s"(p.mpad), "s"(tiles_x), "s"(tile));
  const int l16 = lane & 15, lg = lane >> 4;
  const int per_img = tiles_x * ((p.oh + 1) / 2);
  const int img = tile / per_img, rem = tile - img * per_img;
  const int oy0 = (rem / tiles_x) * 2, ox0 = (rem % tiles_x) * 32;
  const int HW = p.h * p.w;
  const unsigned OOB = 0x80000000u;
  const int r = wave >> 1, c = (wave & 1) * 16 + l16;   // this lane's pixel in the tile
  const int poy = oy0 + r, pox = ox0 + c;
  const bool pval = poy < p.oh && pox < p.ow;

  // chunk-invariant load offsets: load j = wave + 4 q of the chunk brings
  // the 16-byte groups 64 j + lane of the stage (halo groups, then weight
  // groups, then spare ones); the channel / weight-row part of the address
  // is the scalar offset
  unsigned doff[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int gi = 64 * (wave + 4 * q) + lane;
    if (gi < LC_HALO / 4) {
      const int cl = gi / (4 * LC_HG), rem = gi - cl * 4 * LC_HG;
      const int rr = rem / LC_HG, gc = rem - rr * LC_HG;
      const int iy = oy0 - 1 + rr, ix = ox0 - 4 + 4 * gc;
      const bool ok = iy >= 0 && iy < p.h && ix >= 0 && ix < p.w;
      doff[q] = ok ? (unsigned)((cl * HW + iy * p.w + ix) * 4) : OOB;
    } else if (gi < (LC_HALO + LC_W) / 4) {
      const int wg = gi - LC_HALO / 4, kr = wg >> 3;
      const int mc = (4 * (wg & 7)) ^ (((kr >> 1) & 1) << 4);
      doff[q] = (unsigned)((kr * p.mpad + mc) * 4);
    } else {
      doff[q] = OOB;
    }
  }
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.x + (int64_t)img * p.c * HW), 0, p.c * HW * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.wk, 0, p.c * 9 * p.mpad * 4, 0x00020000);
  // The loads are written as inline asm: through the builtin the compiler
  // sees LDS writes in flight and, unable to tell the stage being refilled
  // from the one being read, puts a full vmcnt(0) wait before some chunks'
  // operand reads.  The explicit waits below cover every stage.
  // per-chunk scalar offsets, as values (a field read inside the loop would
  // be re-read from the kernel arguments after every compiler fence)
  const unsigned hstep = __builtin_amdgcn_readfirstlane(LC_CC * HW * 4);
  const unsigned wstep = __builtin_amdgcn_readfirstlane(LC_WROWS * p.mpad * 4);
  auto issue = [&](int ch, float* st) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int j = wave + 4 * q;   // wave-uniform
      const bool halo = j < LC_HALO / 256;
      const unsigned lds = __builtin_amdgcn_readfirstlane(
          (unsigned)(uintptr_t)(__attribute__((address_space(3))) float*)(st + 256 * j));
      const unsigned soff = ch * (halo ? hstep : wstep);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"   // m0 is reserved; nothing else uses it here
      __asm__ volatile(
          "s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds),
          "v"(doff[q]), "s"(halo ? xr : wr), "s"(soff)
          : "m0");
#pragma clang diagnostic pop
    }
  };
  // the bias terms, loaded before the chunks so that the chunk waits below
  // (which count loads in issue order) never wait for them as well.
  // The bias: seeded into the chain where the reference seeds (M%4 tail rows
  // of a partial 32-column panel of the output row), else added after it;
  // -0.0 (the exact additive identity) where nothing is added
  float bld[2][4];
#pragma unroll
  for (int mt = 0; mt < 2; mt++)
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int co = mt * 16 + 4 * lg + v;
      bld[mt][v] = (p.bias && co < p.m) ? p.bias[co] : 0.0f;
    }
  // CVT: this thread's share of the ConvT weights (w1 element tid + 256 j,
  // w2 element tid), loaded before the chunks as the bias is; the epilogue
  // stages them in LDS
  float w1r[CVT ? 9 : 1], w2r = 0.0f;
  if constexpr (CVT) {
    const int tid = wave * 64 + lane;
#pragma unroll
    for (int j = 0; j < 9; j++) w1r[j] = cv.w1[tid + 256 * j];
    if (tid < 4 * CV_C) w2r = cv.w2[tid];
  }

  __asm__ volatile("" ::: "memory");
  const int nch = p.c / LC_CC;   // ONE: exactly 4 (C = 32)
  issue(0, s0);
  if (ONE || nch > 1) issue(1, s1);
  if constexpr (ONE) {
    issue(2, s2);
    issue(3, s3);
  }
  // the bias values are first used here, after every load is out (otherwise
  // the accumulator set-up can be scheduled between the loads, with a wait
  // for the bias loads in front of the later ones)
  __asm__ volatile("" : "+v"(bld[0][0]), "+v"(bld[0][1]), "+v"(bld[0][2]), "+v"(bld[0][3]),
                   "+v"(bld[1][0]), "+v"(bld[1][1]), "+v"(bld[1][2]), "+v"(bld[1][3])::"memory");
  const int n0 = (pox >> 5) << 5;
  const bool tail_panel = (p.ow - n0) < 32;
  const int mtail = p.m - p.m % 4;
  float bterm[2][4];
  f32x4 acc[2];
#pragma unroll
  for (int mt = 0; mt < 2; mt++)
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int co = mt * 16 + 4 * lg + v;
      const bool seeded = p.bias && tail_panel && co >= mtail;
      acc[mt][v] = seeded ? bld[mt][v] : 0.0f;
      bterm[mt][v] = (p.bias && !seeded) ? bld[mt][v] : -0.0f;
    }

  // per-step operand offsets inside a stage: k = 4 s + g of the chunk
  int boff[LC_WROWS / 4];
#pragma unroll
  for (int s = 0; s < LC_WROWS / 4; s++) {
    const int k = 4 * s + lg, cl = k / 9, tap = k - 9 * cl;
    const int ky = tap / 3, kx = tap - 3 * ky;
    boff[s] = cl * 4 * LC_HP + (r + ky) * LC_HP + c + kx + 3;
  }

  constexpr int PER = LC_DMA / 4;   // loads per wave per chunk
  auto stage = [&](auto st) -> float* {
    constexpr int S = decltype(st)::value;
    if constexpr (S == 0) return s0;
    else if constexpr (S == 1) return s1;
    else return s2;
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  // one chunk's 36 MFMAs from stage st
  // In the ring form, where up to three workgroups share a CU and their waves
  // interleave on each SIMD, reads two steps ahead measured faster than six
  // (det head conv 23.4 -> 22.5 us, neck 33.4 -> 32.8 us, trace medians)
  constexpr int LEAD = ONE ? LC_LEAD : LC_LEAD_RING;
  auto mma = [&](const float* st) {
    const float* wst = st + LC_HALO;
    float av[LC_WROWS / 4][2], bv[LC_WROWS / 4];
#pragma unroll
    for (int s = 0; s < LC_WROWS / 4; s++) {
      const int k = 4 * s + lg;
      bv[s] = st[boff[s]];
#pragma unroll
      for (int mt = 0; mt < 2; mt++)
        av[s][mt] = wst[k * 32 + ((mt * 16 + l16) ^ (((k >> 1) & 1) << 4))];
    }
#pragma unroll
    for (int s = 0; s < LC_WROWS / 4; s++)
#pragma unroll
      for (int mt = 0; mt < 2; mt++)
        acc[mt] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[s][mt], bv[s], acc[mt], 0, 0, 0);
    // schedule: the operand reads of the first LEAD steps, then each step's
    // two MFMAs followed by the reads of the step LEAD ahead, so that reads
    // run LEAD steps ahead of their use (left to itself the scheduler reads
    // each step's operands just before its MFMAs)
    __builtin_amdgcn_sched_group_barrier(0x100, 3 * LEAD, 0);
#pragma unroll
    for (int s = LEAD; s < LC_WROWS / 4; s++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * LEAD, 0);
  };
  auto body = [&](auto sti, int ch) {
    constexpr int S = decltype(sti)::value;
    // this chunk in (the next one may still load); then a barrier with no
    // fence, which leaves the loads in flight, after which every wave is
    // done with the stage of chunk ch - 1, refilled with chunk ch + 2
    if (ch + 1 < nch)
      wait_vmcnt<PER>();
    else
      wait_vmcnt<0>();
    __asm__ volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    if (ch + 2 < nch) issue(ch + 2, stage(std::integral_constant<int, (S + 2) % LC_NST>{}));
    mma(stage(sti));
  };
  if constexpr (ONE) {
    // all four chunks loading from the start, each multiplied as soon as
    // every wave's part of it is in (no stage is refilled, so a barrier only
    // publishes the chunk)
    auto arrive = [&](auto left) {
      wait_vmcnt<decltype(left)::value * PER>();
      __asm__ volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_s_barrier();
      __asm__ volatile("" ::: "memory");
    };
    arrive(std::integral_constant<int, 3>{});
    mma(s0);
    arrive(std::integral_constant<int, 2>{});
    mma(s1);
    arrive(std::integral_constant<int, 1>{});
    mma(s2);
    arrive(std::integral_constant<int, 0>{});
    mma(s3);
  } else {
    for (int ch = 0; ch < nch; ch += LC_NST) {
      body(S0{}, ch);
      if (ch + 1 < nch) body(S1{}, ch + 1);
      if (ch + 2 < nch) body(S2{}, ch + 2);
    }
  }

  if constexpr (CVT) {
    // The conv outputs (bias, activation) of this wave's 16 pixels go to LDS,
    // and the ConvT weights, in the two ring stages the last chunk did not
    // use: every wave is past that chunk's barrier, so no wave reads them any
    // more.  The first ConvT is then a 96 x 24 by 24 x 16 product per wave on
    // the MFMAs: row 4 q + v of M tile mt is (tap q, channel 4 mt + v), so that
    // lane (pixel l16, g) ends with the 24 intermediates of its pixel and tap
    // q = g in its registers, each the chain over ci of fma(x[ci], w1[ci][co][q])
    // from 0, in ci order (k = 4 s + g), as convt_pair_sigmoid_kernel chains it.
    // The second ConvT (chain over co) and the sigmoid follow in the lane.
    const int last = (nch - 1) % LC_NST;
    float* fa = last == 0 ? s1 : s0;
    float* fb = last == 2 ? s1 : s2;
    float* hh = fa + wave * 16 * CV_HP;
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const int co = mt * 16 + 4 * lg + v;
        float xv = acc[mt][v] + bterm[mt][v];
        if constexpr (AK == 2)
          xv = relu1(xv);
        else if constexpr (AK < 0)
          xv = act_apply(xv, p.act);
        if (co < CV_C) hh[l16 * CV_HP + co] = xv;
      }
    // A operands in MFMA order [mt][s][lane]: lane g 16 + i of step s, tile mt
    // holds w1[ci = 4 s + g][co = 4 mt + (i & 3)][q = i >> 2]
    float* sa = fb;
    float* sw2 = fb + 4 * CV_C * CV_C;  // [co][q2]
    {
      const int tid = wave * 64 + lane;
#pragma unroll
      for (int j = 0; j < 9; j++) {
        const int i = tid + 256 * j;   // (ci * 24 + co) * 4 + q
        const int ci = i / (4 * CV_C), co = (i >> 2) % CV_C, q = i & 3;
        sa[((co >> 2) * (CV_C / 4) + (ci >> 2)) * 64 + (ci & 3) * 16 + q * 4 + (co & 3)] = w1r[j];
      }
      if (tid < 4 * CV_C) sw2[tid] = w2r;
    }
    __syncthreads();
    // every lane takes part in the products (an idle lane's A row would be
    // lost to every pixel); only the stores are per pixel
    float bx[CV_C / 4];
#pragma unroll
    for (int s = 0; s < CV_C / 4; s++) bx[s] = hh[l16 * CV_HP + 4 * s + lg];
    f32x4 mid[CV_C / 4];
#pragma unroll
    for (int mt = 0; mt < CV_C / 4; mt++) {
      mid[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int s = 0; s < CV_C / 4; s++)
        mid[mt] = __builtin_amdgcn_mfma_f32_16x16x4f32(sa[(mt * (CV_C / 4) + s) * 64 + lane], bx[s],
                                                       mid[mt], 0, 0, 0);
    }
    f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int co = 0; co < CV_C; co++) {
      const f32x4 wv = *(const f32x4*)(sw2 + co * 4);
      const float mv = mid[co >> 2][co & 3];
      o[0] = __builtin_fmaf(mv, wv[0], o[0]);
      o[1] = __builtin_fmaf(mv, wv[1], o[1]);
      o[2] = __builtin_fmaf(mv, wv[2], o[2]);
      o[3] = __builtin_fmaf(mv, wv[3], o[3]);
    }
    if (!pval) return;
    const int ky = lg >> 1, kx = lg & 1;
    const int64_t ow4 = 4 * (int64_t)p.ow;
    float* yo = cv.y + ((int64_t)img * 4 * p.oh + 4 * poy + 2 * ky) * ow4 + 4 * pox + 2 * kx;
    yo[0] = sigmoid1(o[0]);
    yo[1] = sigmoid1(o[1]);
    yo[ow4] = sigmoid1(o[2]);
    yo[ow4 + 1] = sigmoid1(o[3]);
    return;
  }
  // epilogue as in direct3x3_unit; every residual term is read before the
  // first store (a load after a store that may alias the output makes the
  // compiler wait for that store to complete, once per output)
  if (!pval) return;
  const int64_t yoh = (int64_t)p.oh * p.y_up, yow = (int64_t)p.ow * p.y_up;
  float* ybase = p.y + ((int64_t)img * p.y_ctotal + p.y_coff) * yoh * yow;
  const float* rbase = p.res ? p.res + ((int64_t)img * p.m * p.oh + poy) * p.ow + pox : nullptr;
  float outv[2][4];
#pragma unroll
  for (int mt = 0; mt < 2; mt++)
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int co = mt * 16 + 4 * lg + v;
      float xv = acc[mt][v] + bterm[mt][v];
      if constexpr (AK == 2)
        xv = relu1(xv);
      else if constexpr (AK < 0)
        xv = act_apply(xv, p.act);
      if (rbase && co < p.m) xv = xv + rbase[(int64_t)co * p.oh * p.ow];
      outv[mt][v] = xv;
    }
#pragma unroll
  for (int mt = 0; mt < 2; mt++)
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int co = mt * 16 + 4 * lg + v;
      if (co < p.m) store_replicated(ybase + (int64_t)co * yoh * yow, yow, poy, pox, (int)p.y_up,
                                     outv[mt][v]);
    }
}

template <int AK, int NG>
__global__ __launch_bounds__(256) void conv3x3_lds_kernel(LdsConvGroup g) {
  __shared__ __attribute__((aligned(16))) float s0[LC_STAGE], s1[LC_STAGE], s2[LC_STAGE];
  const int lane = threadIdx.x & 63;
  // "& 3" bounds the wave index, so that the LDS offsets of the loads and
  // reads have known ranges
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3;
  const int t = blockIdx.x;   // < start[DIRECT_GROUP_MAX]: the grid is the total
  if constexpr (NG == 1) {
    lds_conv_tile<AK, false>(g.k[0], g.tiles_x[0], t, s0, s1, s2, nullptr, wave, lane);
  } else {
    // the member conv, without branches: start[] is non-decreasing
    const int i = (t >= g.start[1]) + (t >= g.start[2]) + (t >= g.start[3]);
    lds_conv_tile<AK, false>(g.k[i], g.tiles_x[i], t - g.start[i], s0, s1, s2, nullptr, wave,
                             lane);
  }
}

// The det head: a 3x3 conv to 24 channels (lds_conv_tile, one conv) with the
// conv-transpose pair and sigmoid after it in the epilogue; the conv output
// never reaches HBM.
template <int AK>
__global__ __launch_bounds__(256) void conv3x3_lds_convt_kernel(DirectConvK k, int tiles_x,
                                                                ConvtEpi cv) {
  __shared__ __attribute__((aligned(16))) float s0[LC_STAGE], s1[LC_STAGE], s2[LC_STAGE];
  static_assert(4 * 16 * CV_HP <= LC_STAGE && 4 * CV_C * CV_C + 4 * CV_C <= LC_STAGE, "");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3;
  lds_conv_tile<AK, false, true>(k, tiles_x, blockIdx.x, s0, s1, s2, nullptr, wave, lane, cv);
}

// One plain 32-channel conv (no residual, no upsampled store, no activation
// other than ReLU): the whole input halo and all 288 weight rows of a tile
// (four chunks, 64 KB with the spare words) are loaded at once, so the waves
// wait once and meet at one barrier instead of four.  The arguments are
// scalars, 14 dwords, which the dispatch can preload into SGPRs.
template <int AK>
__global__ __launch_bounds__(256) void conv3x3_lds32_kernel(const float* x, const float* wk,
                                                            const float* bias, float* y, int h,
                                                            int w, int m, int tiles_x,
                                                            int y_ctotal, int y_coff) {
  __shared__ __attribute__((aligned(16))) float st[4 * LC_STAGE];
  DirectConvK p{};
  p.x = x; p.wk = wk; p.bias = bias; p.res = nullptr; p.y = y;
  p.c = 32; p.h = h; p.w = w; p.m = m; p.mpad = 32;
  p.sh = 1; p.sw = 1; p.ph = 1; p.pw = 1; p.oh = h; p.ow = w;
  p.y_ctotal = y_ctotal; p.y_coff = y_coff; p.y_up = 1;
  p.act.kind = AK;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3;
  lds_conv_tile<AK, true>(p, tiles_x, blockIdx.x, st, st + LC_STAGE, st + 2 * LC_STAGE,
                          st + 3 * LC_STAGE, wave, lane);
}

static void direct_params(const ConvArgs& a, const float* wk, DirectConvK& p) {
  p = DirectConvK{};
  p.x = a.x; p.wk = wk; p.bias = a.bias; p.res = a.res; p.y = a.y;
  p.c = (int)a.c; p.h = (int)a.h; p.w = (int)a.w; p.m = (int)a.m; p.mpad = (int)mpad_of(a.m);
  p.sh = (int)a.sh; p.sw = (int)a.sw; p.ph = (int)a.ph; p.pw = (int)a.pw;
  p.oh = (int)a.oh; p.ow = (int)a.ow;
  p.y_ctotal = a.y_ctotal; p.y_coff = a.y_coff; p.y_up = a.y_up;
  p.act = a.act;
}

bool direct3x3_eligible(const ConvArgs& a) {
  // strides 1 and 2 along x: the implicit-GEMM branch and its per-row bias
  // rule (other strides take the im2col branch's rule, dense_conv_kernel)
  return a.kh == 3 && a.kw == 3 && a.group == 1 && (a.sw == 1 || a.sw == 2) &&
         a.c * a.h * a.w * 4 < (int64_t)0x80000000 && a.oh * a.ow < (1ll << 30) &&
         kpad_of(a.c, 9) * mpad_of(a.m) * 4 < (int64_t)0x80000000 &&
         (int64_t)ceil_div(a.m, 16) * ceil_div(a.oh * a.ow, 16) * a.n < (1ll << 29);
}

static bool lds3x3_eligible(const ConvArgs& a) {
  return direct3x3_eligible(a) && a.sh == 1 && a.sw == 1 && a.ph == 1 && a.pw == 1 &&
         a.m <= 32 && a.c % LC_CC == 0 && a.c > 0 && mpad_of(a.m) == 32 &&
         a.c * a.h * a.w * 4 < (int64_t)0x80000000 && a.w % 4 == 0 &&
         (uintptr_t)a.x % 16 == 0;
}

static int launch_lds3x3(const ConvArgs* a, int n, hipStream_t s) {
  LdsConvGroup g{};
  g.n = n;
  int64_t total = 0;
  for (int i = 0; i < n; i++) {
    direct_params(a[i], a[i].wk, g.k[i]);
    g.tiles_x[i] = (int)ceil_div(a[i].ow, 32);
    g.start[i] = (int)total;
    total += (int64_t)g.tiles_x[i] * ceil_div(a[i].oh, 2) * a[i].n;
  }
  for (int i = n; i <= DIRECT_GROUP_MAX; i++) g.start[i] = (int)total;
  if (total >= (1ll << 31)) return fail(QPH_EUNSUPPORTED, "conv: grid too large");
  int kind = a[0].act.kind;
  for (int i = 1; i < n; i++)
    if (a[i].act.kind != kind) kind = -1;
  const dim3 grid((unsigned)total);
  if (n == 1 && a[0].c == 32 && (kind == 0 || kind == 2) && !a[0].res && a[0].y_up == 1 &&
      a[0].y_ctotal < (1ll << 31) && a[0].y_coff < (1ll << 31)) {
    const DirectConvK& k = g.k[0];
    if (kind == 0)
      hipLaunchKernelGGL(conv3x3_lds32_kernel<0>, grid, dim3(256), 0, s, k.x, k.wk, k.bias, k.y,
                         k.h, k.w, k.m, g.tiles_x[0], (int)k.y_ctotal, (int)k.y_coff);
    else
      hipLaunchKernelGGL(conv3x3_lds32_kernel<2>, grid, dim3(256), 0, s, k.x, k.wk, k.bias, k.y,
                         k.h, k.w, k.m, g.tiles_x[0], (int)k.y_ctotal, (int)k.y_coff);
    return launch_check("conv3x3_lds32_kernel");
  }
  if (n == 1) {
    if (kind == 0)
      hipLaunchKernelGGL((conv3x3_lds_kernel<0, 1>), grid, dim3(256), 0, s, g);
    else if (kind == 2)
      hipLaunchKernelGGL((conv3x3_lds_kernel<2, 1>), grid, dim3(256), 0, s, g);
    else
      hipLaunchKernelGGL((conv3x3_lds_kernel<-1, 1>), grid, dim3(256), 0, s, g);
  } else {
    if (kind == 0)
      hipLaunchKernelGGL((conv3x3_lds_kernel<0, 4>), grid, dim3(256), 0, s, g);
    else if (kind == 2)
      hipLaunchKernelGGL((conv3x3_lds_kernel<2, 4>), grid, dim3(256), 0, s, g);
    else
      hipLaunchKernelGGL((conv3x3_lds_kernel<-1, 4>), grid, dim3(256), 0, s, g);
  }
  return launch_check("conv3x3_lds_kernel");
}

// The conv of the det head with its conv-transpose pair (24 -> 24 -> 1, 2x2
// stride 2 each) and sigmoid in one launch: a 3x3 conv to 24 channels that
// lds_conv_tile takes, stored plainly (no residual, slot or upsample), ReLU
// or no activation.
bool conv3x3_convt_eligible(const ConvArgs& a) {
  return lds3x3_eligible(a) && a.m == CV_C && !a.res && a.y_up == 1 &&
         (a.y_ctotal == 0 || a.y_ctotal == a.m) && a.y_coff == 0 &&
         (a.act.kind == 0 || a.act.kind == 2) && a.n * 16 * a.oh * a.ow < (1ll << 31);
}

int launch_conv3x3_convt(const ConvArgs& a, const float* w1, const float* w2, float* y,
                         hipStream_t s) {
  if (!a.wk || !conv3x3_convt_eligible(a))
    return fail(QPH_EUNSUPPORTED, "conv + conv-transpose pair: unsupported shape");
  DirectConvK k{};
  direct_params(a, a.wk, k);
  const int tiles_x = (int)ceil_div(a.ow, 32);
  const int64_t total = (int64_t)tiles_x * ceil_div(a.oh, 2) * a.n;
  if (total >= (1ll << 31)) return fail(QPH_EUNSUPPORTED, "conv: grid too large");
  const ConvtEpi cv{w1, w2, y};
  if (a.act.kind == 2)
    hipLaunchKernelGGL(conv3x3_lds_convt_kernel<2>, dim3((unsigned)total), dim3(256), 0, s, k,
                       tiles_x, cv);
  else
    hipLaunchKernelGGL(conv3x3_lds_convt_kernel<0>, dim3((unsigned)total), dim3(256), 0, s, k,
                       tiles_x, cv);
  return launch_check("conv3x3_lds_convt_kernel");
}

int launch_dense_conv_group(const ConvArgs* a, int n, hipStream_t s) {
  if (n < 1 || n > DIRECT_GROUP_MAX) return fail(QPH_EINVAL, "conv group: 1 to 4 convs");
  bool lds = true;
  for (int i = 0; i < n; i++) lds = lds && a[i].wk && lds3x3_eligible(a[i]);
  if (lds) return launch_lds3x3(a, n, s);
  DirectConvGroup g{};
  g.n = n;
  int64_t total = 0;
  for (int i = 0; i < n; i++) {
    if (!a[i].wk || !direct3x3_eligible(a[i]) || a[i].c <= 4)
      return fail(QPH_EUNSUPPORTED, "conv group: member is not a resident direct 3x3 conv");
    direct_params(a[i], a[i].wk, g.k[i]);
    g.k[i].units_m = (int)ceil_div(a[i].m, 16);
    g.k[i].units_px = (int)ceil_div(a[i].oh * a[i].ow, 16);
    g.k[i].units = (int)(g.k[i].units_m * (int64_t)g.k[i].units_px * a[i].n);
    g.start[i] = (int)total;
    total += g.k[i].units;
  }
  for (int i = n; i <= DIRECT_GROUP_MAX; i++) g.start[i] = (int)total;
  if (total >= (1ll << 30)) return fail(QPH_EUNSUPPORTED, "conv group: grid too large");
  hipLaunchKernelGGL(conv3x3_direct_group_kernel, dim3((unsigned)ceil_div(total, 4)), dim3(256),
                     0, s, g);
  return launch_check("conv3x3_direct_group_kernel");
}

// Launches the direct kernel for a 3x3 conv, choosing the per-wave tile so
// that the launch has enough waves to hide load latency.
static int launch_direct3x3(const ConvArgs& a, const float* wk, hipStream_t s) {
  if (lds3x3_eligible(a)) {
    ConvArgs b = a;
    b.wk = wk;
    return launch_lds3x3(&b, 1, s);
  }
  DirectConvK p;
  direct_params(a, wk, p);
  const int64_t npx = a.oh * a.ow;
  auto waves = [&](int mt, int npxu) {
    return (int64_t)ceil_div(a.m, 16 * mt) * ceil_div(npx, 16 * npxu) * a.n;
  };
  int mt = 1, nt = 1;
  if (a.m > 16 && waves(2, 2) >= 4096) { mt = 2; nt = 2; }
  else if (a.m > 16 && waves(2, 1) >= 512) { mt = 2; nt = 1; }   // det head 96->24 at 160x160: 1600
  else if (waves(1, 2) >= 4096) { mt = 1; nt = 2; }
  p.units_m = (int)ceil_div(a.m, 16 * mt);
  p.units_px = (int)ceil_div(npx, 16 * nt);
  const int64_t units = waves(mt, nt);
  if (units >= (1ll << 31) - 4) return fail(QPH_EUNSUPPORTED, "dense conv: grid too large");
  p.units = (int)units;
  dim3 grid((unsigned)ceil_div(units, 4));
  // one group of four channels (the stems): nothing to prefetch
  const bool one = a.c <= 4;
  if (mt == 2 && nt == 2) {
    if (one) hipLaunchKernelGGL((conv3x3_direct_kernel<2, 2, 1>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((conv3x3_direct_kernel<2, 2, 2>), grid, dim3(256), 0, s, p);
  } else if (mt == 2) {
    if (one) hipLaunchKernelGGL((conv3x3_direct_kernel<2, 1, 1>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((conv3x3_direct_kernel<2, 1, 3>), grid, dim3(256), 0, s, p);
  } else if (nt == 2) {
    if (one) hipLaunchKernelGGL((conv3x3_direct_kernel<1, 2, 1>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((conv3x3_direct_kernel<1, 2, 3>), grid, dim3(256), 0, s, p);
  } else {
    if (one) hipLaunchKernelGGL((conv3x3_direct_kernel<1, 1, 1>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((conv3x3_direct_kernel<1, 1, 4>), grid, dim3(256), 0, s, p);
  }
  return launch_check("conv3x3_direct_kernel");
}

template <int T>
static int launch_dense_t(const DenseConvK& p, bool wide_m, dim3 grid, hipStream_t s) {
  if (wide_m)
    hipLaunchKernelGGL((dense_conv_kernel<2, 2, T>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((dense_conv_kernel<1, 2, T>), grid, dim3(256), 0, s, p);
  return launch_check("dense_conv_kernel");
}

// --------------------------------------------------- few input channels
//
// Dense convs with 3 input channels and 16 or 32 outputs (the det and rec
// stems, 3x3 stride 2): one thread per output pixel keeps its C*KH*KW
// input taps in registers and runs the output channels' chains on the VALU,
// four at a time, the weights wave-uniform (scalar loads, ONNX layout).  Per
// element: acc = 0; for k = c*KH*KW + ky*KW + kx ascending: acc = fma(w[m][k],
// x_k, acc) -- the implicit-GEMM chain, taps outside the image giving
// fma(w, 0, acc) -- then + bias (M % 4 == 0: the reference never seeds it),
// then the activation.  The MFMA kernels spend most of their time on
// latency at this size.

struct SmallCK {
  const float* x;
  const float* w;
  const float* bias;
  float* y;
  int h, w_, m, sh, sw, ph, pw, oh, ow;
  Act act;
};

template <int C, int KH, int KW, int M>
__global__ __launch_bounds__(256) void conv_smallc_kernel(SmallCK p) {
  constexpr int K = C * KH * KW;
  // weights transposed to [k][m] in LDS: one broadcast ds_read_b128 gives
  // tap k of four output channels
  __shared__ __attribute__((aligned(16))) float wl[K * M];
  __shared__ float bl[M];
  const int tid = (int)threadIdx.x;
  for (int i = tid; i < K * M; i += 256) {
    const int m = i / K, k = i - m * K;
    wl[k * M + m] = p.w[i];
  }
  if (tid < M) bl[tid] = p.bias ? p.bias[tid] : 0.0f;
  __syncthreads();
  const int npx = p.oh * p.ow;
  const int e = (int)blockIdx.x * 256 + tid;   // pixel of the image
  const int img = (int)blockIdx.y;
  if (e >= npx) return;
  const int oy = e / p.ow, ox = e - oy * p.ow;
  const float* xb = p.x + (int64_t)img * C * p.h * p.w_;
  float xv[K];
#pragma unroll
  for (int c = 0; c < C; c++)
#pragma unroll
    for (int ky = 0; ky < KH; ky++)
#pragma unroll
      for (int kx = 0; kx < KW; kx++) {
        const int iy = oy * p.sh - p.ph + ky, ix = ox * p.sw - p.pw + kx;
        const bool in = iy >= 0 && iy < p.h && ix >= 0 && ix < p.w_;
        xv[(c * KH + ky) * KW + kx] = in ? xb[((int64_t)c * p.h + iy) * p.w_ + ix] : 0.0f;
      }
  float* yb = p.y + (int64_t)img * M * npx + e;
#pragma unroll 2
  for (int m0 = 0; m0 < M; m0 += 4) {
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < K; k++) {
      const f32x4 wv = *(const f32x4*)(wl + k * M + m0);
#pragma unroll
      for (int q = 0; q < 4; q++) acc[q] = __builtin_fmaf(wv[q], xv[k], acc[q]);
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const float v = p.bias ? acc[q] + bl[m0 + q] : acc[q];
      yb[(int64_t)(m0 + q) * npx] = act_apply(v, p.act);
    }
  }
}

static bool smallc_eligible(const ConvArgs& a) {
  return a.group == 1 && a.c == 3 && a.kh == 3 && a.kw == 3 && (a.m == 16 || a.m == 32) &&
         !a.res &&
         a.y_ctotal == a.m && a.y_coff == 0 && a.y_up == 1 && a.oh * a.ow < (1ll << 31) &&
         a.n <= 65535 && a.m * a.oh * a.ow < (1ll << 31);
}

static int launch_smallc(const ConvArgs& a, hipStream_t s) {
  SmallCK p{};
  p.x = a.x; p.w = a.wt; p.bias = a.bias; p.y = a.y;
  p.h = (int)a.h; p.w_ = (int)a.w; p.m = (int)a.m;
  p.sh = (int)a.sh; p.sw = (int)a.sw; p.ph = (int)a.ph; p.pw = (int)a.pw;
  p.oh = (int)a.oh; p.ow = (int)a.ow;
  p.act = a.act;
  dim3 grid(ceil_div(a.oh * a.ow, 256), (unsigned)a.n);
  if (a.m == 16)
    hipLaunchKernelGGL((conv_smallc_kernel<3, 3, 3, 16>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((conv_smallc_kernel<3, 3, 3, 32>), grid, dim3(256), 0, s, p);
  return launch_check("conv_smallc_kernel");
}

// Tile height of the reference's im2col branch (conv.rs:508-524) as it runs
// on one thread: min(oh, max(1, 2^19 / (kk * ow))).  It sets N of each tile
// GEMM and so where the bias is seeded.
static int64_t im2col_tile_rows(const ConvArgs& a) {
  const int64_t kk = a.c / a.group * a.kh * a.kw;
  int64_t t = (int64_t(1) << 19) / std::max<int64_t>(1, kk * a.ow);
  t = std::max<int64_t>(1, t);
  return std::min(t, a.oh);
}

// Launch configuration of the implicit-GEMM kernel (also the validity check
// a session runs at create time).
static int dense_conv_config(const ConvArgs& a, DenseConvK& p, dim3& grid, bool& wide_m) {
  const int64_t khkw = a.kh * a.kw;
  const int64_t g = a.group;
  const int64_t cg = a.c / g, mg = a.m / g;
  p = DenseConvK{};
  p.x = a.x; p.wk = a.wk; p.bias = a.bias; p.res = a.res; p.y = a.y;
  p.c = cg; p.h = a.h; p.w = a.w; p.m = mg; p.mpad = mpad_of(mg);
  p.ctot = a.c; p.mtot = a.m; p.group = g;
  p.kh = a.kh; p.kw = a.kw; p.sh = a.sh; p.sw = a.sw; p.ph = a.ph; p.pw = a.pw;
  p.oh = a.oh; p.ow = a.ow;
  p.y_ctotal = a.y_ctotal; p.y_coff = a.y_coff; p.y_up = a.y_up;
  p.seed_tile = (a.sw == 1 || a.sw == 2) ? 0 : im2col_tile_rows(a);
  p.act = a.act;
  wide_m = mg > 16;
  const int mb = wide_m ? 32 : 16;
  // 2 MFMA tiles per wave; pixels per workgroup: 64 (WM=2) or 128 (WM=1)
  const int pix = wide_m ? 64 : 128;
  p.tw = a.ow >= 32 ? 32 : 16;
  p.th = pix / p.tw;
  p.rt = (int)((p.th - 1) * a.sh + a.kh);
  p.ct = (int)((p.tw - 1) * a.sw + a.kw);
  const int plane = p.rt * p.ct;
  if (p.ct > 128) return fail(QPH_EUNSUPPORTED, "dense conv: halo row wider than 128");
  if (cg * a.h * a.w * 4 >= (int64_t)0x80000000)
    return fail(QPH_EUNSUPPORTED, "dense conv: input image larger than 2 GB");
  // channel chunk (multiple of 4): halo + weight slice within the LDS budget
  const int64_t per4 = 4 * ((int64_t)plane + khkw * mb);
  int64_t groups = (CONV_LDS_FLOATS - 64) / per4;
  const int64_t cpad = (cg + 3) / 4 * 4;
  if (groups <= 0) return fail(QPH_EUNSUPPORTED, "dense conv: kernel too large for the LDS tile");
  if (groups * 4 > cpad) groups = cpad / 4;
  p.cchunk = (int)(4 * groups);
  p.kpad = kpad_of(cg, khkw);
  if (p.kpad * p.mpad * 4 >= (int64_t)0x80000000)
    return fail(QPH_EUNSUPPORTED, "dense conv: weights larger than 2 GB");
  p.tiles_x = (int)ceil_div(a.ow, p.tw);
  const int64_t tiles_y = ceil_div(a.oh, p.th);
  if (a.n * g > 65535 || (int64_t)p.tiles_x * tiles_y >= (1ll << 31))
    return fail(QPH_EUNSUPPORTED, "dense conv: grid too large");
  grid = dim3((unsigned)(p.tiles_x * tiles_y), ceil_div(mg, mb), (unsigned)(a.n * g));
  return QPH_OK;
}

int dense_conv_check(const ConvArgs& a) {
  if (smallc_eligible(a)) return QPH_OK;
  DenseConvK p;
  dim3 grid;
  bool wide_m;
  return dense_conv_config(a, p, grid, wide_m);
}

int launch_dense_conv(const ConvArgs& a, hipStream_t s, float* scratch_wk) {
  if (smallc_eligible(a)) return launch_smallc(a, s);
  const int64_t khkw = a.kh * a.kw;
  const float* wk = a.wk;
  if (!wk) {
    if (!scratch_wk) return fail(QPH_EINVAL, "dense conv: no repacked weights");
    QPH_TRY(launch_repack_conv_w_taps(a.wt, a.m, a.c / a.group, khkw, scratch_wk, s, a.group));
    wk = scratch_wk;
  }
  // 3x3: direct kernel (input and weight buffers within 32-bit offsets)
  if (direct3x3_eligible(a)) return launch_direct3x3(a, wk, s);
  DenseConvK p;
  dim3 grid;
  bool wide_m;
  QPH_TRY(dense_conv_config(a, p, grid, wide_m));
  p.wk = wk;
  switch (khkw) {
    case 9: return launch_dense_t<9>(p, wide_m, grid, s);
    case 25: return launch_dense_t<25>(p, wide_m, grid, s);
    case 4: return launch_dense_t<4>(p, wide_m, grid, s);
    case 1: return launch_dense_t<1>(p, wide_m, grid, s);
    default: return launch_dense_t<0>(p, wide_m, grid, s);
  }
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
  // halo fill: each wave takes whole rows (lanes along x, up to 192 wide),
  // two rows' loads in flight before their stores
  {
    const int lane = tid & 63, wave = tid >> 6;
    for (int r0 = wave * 2; r0 < p.rt; r0 += 8) {
      float v[2][3];
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int ry = r0 + u;
        const int64_t iy = iy0 + ry;
        const bool rowok = ry < p.rt && iy >= 0 && iy < p.h;
#pragma unroll
        for (int hx = 0; hx < 3; hx++) {
          const int rx = lane + 64 * hx;
          const int64_t ix = ix0 + rx;
          v[u][hx] = (rowok && rx < p.ct && ix >= 0 && ix < p.w_) ? xp[iy * p.w_ + ix] : 0.0f;
        }
      }
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int ry = r0 + u;
        if (ry >= p.rt) break;
#pragma unroll
        for (int hx = 0; hx < 3; hx++) {
          const int rx = lane + 64 * hx;
          if (rx < p.ct) tile[ry * p.ct + rx] = v[u][hx];
        }
      }
    }
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

// Tiled depthwise (the HBM-bound NCHW form: cfg-style planes, no residual,
// no upsampled store).  A workgroup is nw waves and one tile of TH x TW
// outputs of a plane; thread t computes PX consecutive outputs of tile row
// t / TPR (TPR = ceil(TW / PX) threads a row, TH = nw * (64 / TPR) rows).
// The tile's input halo (rt x ct floats, zero where it falls outside the
// image) arrives in LDS by buffer->LDS loads, all issued before one wait:
// thread T of load round k brings halo element 64 nw k + T, out-of-image
// elements carry an offset past the buffer and read 0.  Each output keeps the reference chain acc = fma(w, x, acc)
// over ky then kx from 0, + bias, then the activation; its PX outputs share
// the KH halo rows read once from LDS.  AK: 3 = HardSigmoid + Mul inline, 0
// none, -1 any kind through act_apply.
struct DwWaveK {
  const float* x;
  const float* w;
  const float* bias;
  float* y;
  int c, h, w_, sh, ph, pw, oh, ow;
  int th, tw, tpr, rt, ct, tiles_x;
  int64_t y_ctotal, y_coff;
  Act act;
  int vec4;     // 16-byte aligned output rows (float4 stores when PX == 4)
};

template <int KH, int KW, int SW, int PX, int AK>
__global__ __launch_bounds__(256) void depthwise_wave_kernel(DwWaveK p) {
  extern __shared__ float halo[];
  constexpr int NC = (PX - 1) * SW + KW;   // halo columns one thread reads per row
  const int lane = threadIdx.x;            // thread of the workgroup
  const int nthr = blockDim.x;
  const int64_t plane = blockIdx.y;         // n * c + ch
  const int ch = (int)(plane % p.c);
  const int tyb = (int)blockIdx.x / p.tiles_x, txb = (int)blockIdx.x - tyb * p.tiles_x;
  const int oy0 = tyb * p.th, ox0 = txb * p.tw;
  const int iy0 = oy0 * p.sh - p.ph, ix0 = ox0 * SW - p.pw;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.x + plane * p.h * p.w_), 0, p.h * p.w_ * 4, 0x00020000);
  const int nh = p.rt * p.ct;
  const int wbase = lane & ~63;            // this wave's first thread
  for (int e0 = wbase; e0 < nh; e0 += nthr) {
    const int e = e0 + (lane & 63);
    const int ry = e / p.ct, rx = e - ry * p.ct;
    const int iy = iy0 + ry, ix = ix0 + rx;
    const unsigned off = (e < nh && iy >= 0 && iy < p.h && ix >= 0 && ix < p.w_)
                             ? (unsigned)(iy * p.w_ + ix) * 4u
                             : 0x80000000u;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        xr, (__attribute__((address_space(3))) void*)(halo + e0), 4, off, 0, 0, 0);
  }
  float wr[KH * KW];
#pragma unroll
  for (int i = 0; i < KH * KW; i++) wr[i] = p.w[ch * KH * KW + i];
  const float bv = p.bias ? p.bias[ch] : 0.0f;
  __builtin_amdgcn_s_waitcnt(0);   // vmcnt(0), lgkmcnt(0): this wave's part is in LDS
  __asm__ volatile("" ::: "memory");
  if (nthr > 64) __syncthreads();   // and every other wave's
  const int py = lane / p.tpr, g = lane - py * p.tpr;
  const int oy = oy0 + py, oxs = ox0 + g * PX;
  if (py >= p.th || oy >= p.oh || oxs >= p.ow) return;
  float acc[PX];
#pragma unroll
  for (int i = 0; i < PX; i++) acc[i] = 0.0f;
  const float* hb = halo + py * p.sh * p.ct + g * PX * SW;
#pragma unroll
  for (int ky = 0; ky < KH; ky++) {
    float xv[NC];
#pragma unroll
    for (int j = 0; j < NC; j++) xv[j] = hb[ky * p.ct + j];
#pragma unroll
    for (int kx = 0; kx < KW; kx++)
#pragma unroll
      for (int i = 0; i < PX; i++) acc[i] = __builtin_fmaf(wr[ky * KW + kx], xv[i * SW + kx], acc[i]);
  }
  float out[PX];
#pragma unroll
  for (int i = 0; i < PX; i++) {
    float v = acc[i] + bv;
    if constexpr (AK == 3)
      v = v * hsig1(v, p.act.c1, p.act.c2);
    else if constexpr (AK < 0)
      v = act_apply(v, p.act);
    out[i] = v;
  }
  const int64_t bn = plane / p.c;
  float* yr = p.y + ((bn * p.y_ctotal + p.y_coff + ch) * p.oh + oy) * (int64_t)p.ow;
  if (PX == 4 && p.vec4 && oxs + 4 <= p.ow) {
    *(float4*)(yr + oxs) = make_float4(out[0], out[1], out[2], out[3]);
  } else {
#pragma unroll
    for (int i = 0; i < PX; i++)
      if (oxs + i < p.ow) yr[oxs + i] = out[i];
  }
}

template <int KH, int KW, int SW, int PX>
static void launch_dw_wave_ak(const DwWaveK& p, dim3 grid, int nthr, size_t lds, hipStream_t s) {
  if (p.act.kind == 3)
    hipLaunchKernelGGL((depthwise_wave_kernel<KH, KW, SW, PX, 3>), grid, dim3(nthr), lds, s, p);
  else if (p.act.kind == 0)
    hipLaunchKernelGGL((depthwise_wave_kernel<KH, KW, SW, PX, 0>), grid, dim3(nthr), lds, s, p);
  else
    hipLaunchKernelGGL((depthwise_wave_kernel<KH, KW, SW, PX, -1>), grid, dim3(nthr), lds, s, p);
}

template <int KH, int KW, int SW>
static void launch_dw_wave_px(const DwWaveK& p, int px, dim3 grid, int nthr, size_t lds,
                              hipStream_t s) {
  if (px == 4)
    launch_dw_wave_ak<KH, KW, SW, 4>(p, grid, nthr, lds, s);
  else if (px == 2)
    launch_dw_wave_ak<KH, KW, SW, 2>(p, grid, nthr, lds, s);
  else
    launch_dw_wave_ak<KH, KW, SW, 1>(p, grid, nthr, lds, s);
}

// The one-wave form takes 3x3 and 5x5 kernels, x-stride 1 or 2, plain or
// channel-slice outputs without residual or upsampling, offsets in 32 bits.
static bool dw_wave_eligible(const ConvArgs& a) {
  return ((a.kh == 3 && a.kw == 3) || (a.kh == 5 && a.kw == 5)) && (a.sw == 1 || a.sw == 2) &&
         !a.res && a.y_up == 1 && a.h * a.w * 4 < (1ll << 31) && a.oh < (1 << 20) &&
         a.ow < (1 << 20) && a.n * a.c <= 65535;
}

static int launch_depthwise_wave(const ConvArgs& a, hipStream_t s) {
  DwWaveK p{};
  p.x = a.x; p.w = a.wt; p.bias = a.bias; p.y = a.y;
  p.c = (int)a.c; p.h = (int)a.h; p.w_ = (int)a.w; p.sh = (int)a.sh; p.ph = (int)a.ph;
  p.pw = (int)a.pw; p.oh = (int)a.oh; p.ow = (int)a.ow;
  p.y_ctotal = a.y_ctotal; p.y_coff = a.y_coff;
  p.act = a.act;
  const int64_t planes = a.n * a.c;
  // outputs per thread: the most that still leave >= 1024 waves (four per
  // CU) to hide the load latency behind; then waves per workgroup, where
  // >= 4096 waves remain (larger workgroups share their halo rows; on
  // smaller grids the barrier costs more than the shared rows save)
  int px = 1, nw = 1;
  auto waves_of = [&](int cand, int w) {
    const int tw = (int)std::min<int64_t>(a.ow, 16 * cand);
    const int tpr = (tw + cand - 1) / cand;
    const int th = w * (64 / tpr);
    const int64_t tiles = planes * ceil_div(a.ow, tw) * ceil_div(a.oh, th);
    return tiles * std::min<int64_t>(w, ceil_div((int64_t)std::min<int64_t>(th, a.oh) * tpr, 64));
  };
  for (int cand : {4, 2})
    if (waves_of(cand, 1) >= 1024) {
      px = cand;
      break;
    }
  for (int w : {4, 2})
    if (waves_of(px, w) >= 4096 && w * (64 / ((std::min<int64_t>(a.ow, 16 * px) + px - 1) / px)) <= a.oh) {
      nw = w;
      break;
    }
  p.tw = (int)std::min<int64_t>(a.ow, 16 * px);
  p.tpr = (p.tw + px - 1) / px;
  p.th = nw * (64 / p.tpr);
  if (p.th > p.oh) p.th = p.oh;
  p.rt = (p.th - 1) * p.sh + (int)a.kh;
  p.ct = (p.tw - 1) * (int)a.sw + (int)a.kw;
  p.tiles_x = (int)ceil_div(a.ow, p.tw);
  p.vec4 = (a.ow % 4 == 0) && ((uintptr_t)a.y % 16 == 0);
  const int64_t tiles = (int64_t)p.tiles_x * ceil_div(a.oh, p.th);
  // (+64: the last lanes of a row group whose PX outputs run past a narrow
  // tile read up to (PX - 1) * SW floats past the halo, for outputs they
  // never store)
  const size_t lds = (size_t)((p.rt * p.ct + 63) / 64 * 64 + 64) * 4;
  if (tiles >= (1ll << 31) || lds > 64 * 1024)
    return fail(QPH_EUNSUPPORTED, "depthwise: tile outside the one-wave kernel");
  dim3 grid((unsigned)tiles, (unsigned)planes);
  const int k = (int)a.kh, nthr = 64 * nw;
  if (k == 3 && a.sw == 1) launch_dw_wave_px<3, 3, 1>(p, px, grid, nthr, lds, s);
  else if (k == 3) launch_dw_wave_px<3, 3, 2>(p, px, grid, nthr, lds, s);
  else if (a.sw == 1) launch_dw_wave_px<5, 5, 1>(p, px, grid, nthr, lds, s);
  else launch_dw_wave_px<5, 5, 2>(p, px, grid, nthr, lds, s);
  return launch_check("depthwise_wave_kernel");
}

// Depthwise over whole image rows (the HBM-bound NCHW form: cfg-style
// planes whose width is a multiple of 4).  A thread owns 4V adjacent
// outputs of one output row (V 16-byte stores): group gg of a row covers
// outputs [4V gg, 4V gg + 4V), whose own input columns are [4VS gg, 4VS gg +
// 4VS) -- VS 16-byte loads per input row, straight into registers.  A wave
// holds whole output rows, 64 / g of them (g = groups per row), lanes in row
// order, so the K/2 input columns left of a group are the last ones of the
// lane before it and the K/2 + 1 - S right of it the first ones of the lane
// after it: cross-lane shuffles inside the wave, 0 at the image border (the
// zero padding); rows above or below the image read 0 through the buffer
// range check.  A plane takes whole waves, so its channel is the same across
// a wave and the weights and bias come through scalar loads.  Every load is
// issued before the first fma; no LDS, no barrier.  Each output keeps the
// reference chain acc = fma(w, x, acc) over ky then kx from 0 (out-of-image
// taps are fma(w, 0, acc) there, which leave acc unchanged), + bias, then
// the activation.
struct DwRowsK {
  const float* x;
  const float* w;
  const float* bias;
  float* y;
  int c, h, w_, oh, ow;
  int g, rw;         // groups per output row, output rows per wave (rw * g <= 64)
  int wpp;           // waves per plane: ceil(oh / rw)
  int planes;
  int y_ctotal, y_coff;
  Act act;
};

template <int K, int S, int V, int AK>
__global__ __launch_bounds__(256) void depthwise_rows_kernel(DwRowsK p) {
  constexpr int RIN = K;                     // input rows of one output row
  constexpr int NL = K / 2, NR = K / 2 + 1 - S;
  constexpr int OWN = 4 * V * S;             // own input columns of a row
  constexpr int NW = NL + OWN + NR;          // input columns of a row one thread uses
  const int lane = threadIdx.x & 63;
  const unsigned wv = blockIdx.x * 4u + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const unsigned plane = wv / (unsigned)p.wpp;
  if (plane >= (unsigned)p.planes) return;   // whole waves past the last plane
  const int row_in_wave = lane / p.g, gg = lane - row_in_wave * p.g;
  const int oy = (int)(wv - plane * (unsigned)p.wpp) * p.rw + row_in_wave;
  const bool valid = row_in_wave < p.rw && oy < p.oh;
  const int ch = (int)(plane % (unsigned)p.c);
  const int iw = p.w_;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.x + (int64_t)plane * p.h * iw), 0, p.h * iw * 4, 0x00020000);
  const int iy0 = oy * S - NL, ix0 = OWN * gg;
  // the own columns of each input row, every load issued first (lanes past
  // the wave's rows read nothing: an out-of-range offset)
  float xin[RIN][NW];
#pragma unroll
  for (int r = 0; r < RIN; r++) {
    const int iy = iy0 + r;
    const unsigned off =
        (valid && iy >= 0 && iy < p.h) ? (unsigned)(iy * iw + ix0) * 4u : 0x80000000u;
#pragma unroll
    for (int v = 0; v < V * S; v++) {
      const f32x4 q =
          __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 16 * v, 0));
#pragma unroll
      for (int e = 0; e < 4; e++) xin[r][NL + 4 * v + e] = q[e];
    }
  }
  float wr[K * K];
#pragma unroll
  for (int i = 0; i < K * K; i++) wr[i] = p.w[ch * K * K + i];
  const float bv = p.bias ? p.bias[ch] : 0.0f;
  // the neighbours' columns, from the lanes beside this one in the same
  // row, or 0 at the image border
  const bool left_in = gg > 0, right_in = gg + 1 < p.g;
#pragma unroll
  for (int r = 0; r < RIN; r++) {
#pragma unroll
    for (int j = 0; j < NL; j++) {
      const float v = __shfl_up(xin[r][NL + OWN - NL + j], 1, 64);
      xin[r][j] = left_in ? v : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < NR; j++) {
      const float v = __shfl_down(xin[r][NL + j], 1, 64);
      xin[r][NL + OWN + j] = right_in ? v : 0.0f;
    }
  }
  if (!valid) return;
  const int64_t bn = plane / (unsigned)p.c;
  float* yp = p.y + ((bn * p.y_ctotal + p.y_coff + ch) * (int64_t)p.oh + oy) * p.ow + 4 * V * gg;
#pragma unroll
  for (int v = 0; v < V; v++) {
    float out[4];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int i = 4 * v + e;
      float acc = 0.0f;
#pragma unroll
      for (int ky = 0; ky < K; ky++)
#pragma unroll
        for (int kx = 0; kx < K; kx++) acc = __builtin_fmaf(wr[ky * K + kx], xin[ky][S * i + kx], acc);
      float o = acc + bv;
      if constexpr (AK == 3)
        o = o * hsig1(o, p.act.c1, p.act.c2);
      else if constexpr (AK < 0)
        o = act_apply(o, p.act);
      out[e] = o;
    }
    *(f32x4*)(yp + 4 * v) = f32x4{out[0], out[1], out[2], out[3]};
  }
}

// Outputs per thread (4 or 8) for the whole-row form: 0 when a row of
// groups does not fit a wave.  Eight when four would leave a quarter or more
// of a wave's lanes idle and eight fit rows with fewer idle (the 160-wide
// planes: 40 groups of 4 fill 40 lanes, 20 groups of 8 fill 60).
static int dw_rows_v(int64_t ow) {
  if (ow % 4) return 0;
  const int64_t g1 = ow / 4;
  const int64_t idle1 = g1 <= 64 ? 64 - (64 / g1) * g1 : 64;
  if (ow % 8 == 0 && ow / 8 <= 64) {
    const int64_t g2 = ow / 8, idle2 = 64 - (64 / g2) * g2;
    if (idle1 >= 16 && idle2 < idle1) return 2;
  }
  return g1 <= 64 ? 1 : 0;
}

// Whole-row form: k x k kernel (3 or 5) with padding k / 2 on the left and
// top, equal strides 1 or 2, input width = stride * output width, output
// rows of at most 64 groups, 16-byte aligned tensors, plain or channel-slice
// output.
static bool dw_rows_eligible(const ConvArgs& a) {
  auto al16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  return ((a.kh == 3 && a.kw == 3) || (a.kh == 5 && a.kw == 5)) && a.sh == a.sw &&
         (a.sw == 1 || a.sw == 2) && a.ph == a.kh / 2 && a.pw == a.kw / 2 && !a.res &&
         a.y_up == 1 && dw_rows_v(a.ow) > 0 && a.w == a.sw * a.ow && al16(a.x) && al16(a.y) &&
         a.h * a.w * 4 < (1ll << 31) && a.n * a.c < (1ll << 31) &&
         a.n * a.y_ctotal * a.oh * a.ow < (1ll << 40);
}

template <int K, int S, int V>
static void launch_dw_rows_ak(const DwRowsK& p, dim3 grid, hipStream_t s) {
  if (p.act.kind == 3)
    hipLaunchKernelGGL((depthwise_rows_kernel<K, S, V, 3>), grid, dim3(256), 0, s, p);
  else if (p.act.kind == 0)
    hipLaunchKernelGGL((depthwise_rows_kernel<K, S, V, 0>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((depthwise_rows_kernel<K, S, V, -1>), grid, dim3(256), 0, s, p);
}

template <int K, int S>
static void launch_dw_rows_v(const DwRowsK& p, int v, dim3 grid, hipStream_t s) {
  if (v == 2) launch_dw_rows_ak<K, S, 2>(p, grid, s);
  else launch_dw_rows_ak<K, S, 1>(p, grid, s);
}

static int launch_depthwise_rows(const ConvArgs& a, hipStream_t s) {
  DwRowsK p{};
  p.x = a.x; p.w = a.wt; p.bias = a.bias; p.y = a.y;
  p.c = (int)a.c; p.h = (int)a.h; p.w_ = (int)a.w; p.oh = (int)a.oh; p.ow = (int)a.ow;
  const int v = dw_rows_v(a.ow);
  p.g = (int)(a.ow / (4 * v));
  p.rw = 64 / p.g;
  p.y_ctotal = (int)a.y_ctotal; p.y_coff = (int)a.y_coff;
  p.act = a.act;
  const int64_t planes = a.n * a.c;
  p.wpp = (int)ceil_div(a.oh, p.rw);
  p.planes = (int)planes;
  const int64_t blocks = ceil_div(planes * p.wpp, 4);
  if (blocks >= (1ll << 30)) return fail(QPH_EUNSUPPORTED, "depthwise: grid too large");
  const dim3 grid((unsigned)blocks);
  const int k = (int)a.kh;
  if (k == 3 && a.sw == 1) launch_dw_rows_v<3, 1>(p, v, grid, s);
  else if (k == 3) launch_dw_rows_v<3, 2>(p, v, grid, s);
  else if (a.sw == 1) launch_dw_rows_v<5, 1>(p, v, grid, s);
  else launch_dw_rows_v<5, 2>(p, v, grid, s);
  return launch_check("depthwise_rows_kernel");
}

int launch_depthwise(const ConvArgs& a, hipStream_t s) {
  if (dw_rows_eligible(a)) return launch_depthwise_rows(a, s);
  if (dw_wave_eligible(a)) return launch_depthwise_wave(a, s);
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
  if (p.ct > 192) return fail(QPH_EUNSUPPORTED, "depthwise: halo row wider than 192");
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

// Depthwise conv over channel-last tensors, x[n][h][w][c] -> y[n][oh][ow][c]
// (the rec backbone's deeper blocks, whose pointwise half then runs as a
// row-major GEMM): one thread per output element, channels fastest, so a
// wave reads and writes 64 consecutive channels of a pixel.  Same operation
// sequence as depthwise_kernel (out-of-image taps contribute fma(w, 0, acc)).
// C must be a power of two (the rec blocks: 64, 128, 256).

struct DwClK {
  const float* x;
  const float* w;
  const float* bias;
  float* y;
  int n, c, lc, h, w_, sh, sw, ph, pw, oh, ow;   // c = 1 << lc
  Act act;
};

template <int KH, int KW>
__global__ __launch_bounds__(256) void depthwise_cl_kernel(DwClK p) {
  // grid: x over (ox, ch) of one output row, y over (image, oy); C a power
  // of two, so the channel is a mask and the column a shift
  const int row = (int)blockIdx.y;
  const int oy = row % p.oh, img = row / p.oh;
  const int e = (int)blockIdx.x * 256 + (int)threadIdx.x;
  if (e >= p.ow * p.c) return;
  const int ch = e & (p.c - 1), ox = e >> p.lc;
  const float* wp = p.w + ch * KH * KW;
  const float* xb = p.x + (int64_t)img * p.h * p.w_ * p.c + ch;
  float acc = 0.0f;
#pragma unroll
  for (int ky = 0; ky < KH; ky++) {
    const int iy = oy * p.sh - p.ph + ky;
#pragma unroll
    for (int kx = 0; kx < KW; kx++) {
      const int ix = ox * p.sw - p.pw + kx;
      const float xv = (iy >= 0 && iy < p.h && ix >= 0 && ix < p.w_)
                           ? xb[((int64_t)iy * p.w_ + ix) * p.c]
                           : 0.0f;
      acc = __builtin_fmaf(wp[ky * KW + kx], xv, acc);
    }
  }
  const float v = acc + (p.bias ? p.bias[ch] : 0.0f);
  p.y[((int64_t)row * p.ow) * p.c + e] = act_apply(v, p.act);
}

// PX adjacent output columns per thread (stride SW along x, 3x3): the taps
// of the channel sit in registers and the KH rows of (PX - 1) * SW + 3 input
// columns are read once for all PX outputs; each output keeps the chain
// above (acc = fma(w, x, acc) over ky, kx, then + bias, then the
// activation).  AK = 3: HardSigmoid + Mul inline.
template <int SW, int PX, int AK>
__global__ __launch_bounds__(256) void depthwise_cl_px_kernel(DwClK p) {
  constexpr int NC = (PX - 1) * SW + 3;
  const int row = (int)blockIdx.y;
  const int oy = row % p.oh, img = row / p.oh;
  const int ngx = (p.ow + PX - 1) / PX;
  const int e = (int)blockIdx.x * 256 + (int)threadIdx.x;
  if (e >= ngx * p.c) return;
  const int ch = e & (p.c - 1), ox0 = (e >> p.lc) * PX;
  float w[9];
#pragma unroll
  for (int j = 0; j < 9; j++) w[j] = p.w[ch * 9 + j];
  const float bias = p.bias ? p.bias[ch] : 0.0f;
  const float* xb = p.x + (int64_t)img * p.h * p.w_ * p.c + ch;
  float acc[PX];
#pragma unroll
  for (int q = 0; q < PX; q++) acc[q] = 0.0f;
#pragma unroll
  for (int ky = 0; ky < 3; ky++) {
    const int iy = oy * p.sh - p.ph + ky;
    const bool rok = iy >= 0 && iy < p.h;
    float xv[NC];
#pragma unroll
    for (int c2 = 0; c2 < NC; c2++) {
      const int ix = ox0 * SW - p.pw + c2;
      xv[c2] = (rok && ix >= 0 && ix < p.w_) ? xb[((int64_t)iy * p.w_ + ix) * p.c] : 0.0f;
    }
#pragma unroll
    for (int kx = 0; kx < 3; kx++)
#pragma unroll
      for (int q = 0; q < PX; q++) acc[q] = __builtin_fmaf(w[ky * 3 + kx], xv[q * SW + kx], acc[q]);
  }
  float* yb = p.y + ((int64_t)row * p.ow) * p.c + ch;
#pragma unroll
  for (int q = 0; q < PX; q++) {
    if (ox0 + q >= p.ow) break;
    float v = acc[q] + (p.bias ? bias : 0.0f);
    if constexpr (AK == 3) v = v * hsig1(v, p.act.c1, p.act.c2);
    else v = act_apply(v, p.act);
    yb[(int64_t)(ox0 + q) * p.c] = v;
  }
}

template <int SW>
static int launch_dwcl_px(const DwClK& p, hipStream_t s) {
  const int ngx = (p.ow + 3) / 4;
  const dim3 grid(ceil_div((int64_t)ngx * p.c, 256), (unsigned)(p.n * p.oh));
  if (p.act.kind == 3)
    hipLaunchKernelGGL((depthwise_cl_px_kernel<SW, 4, 3>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((depthwise_cl_px_kernel<SW, 4, 0>), grid, dim3(256), 0, s, p);
  return launch_check("depthwise_cl_px_kernel");
}

int launch_depthwise_cl(const ConvArgs& a, hipStream_t s) {
  const int64_t total = a.n * a.oh * a.ow * a.c;
  if (total <= 0) return QPH_OK;
  if (total >= (1ll << 31) || a.n * a.h * a.w * a.c >= (1ll << 31))
    return fail(QPH_EUNSUPPORTED, "depthwise (channel-last): tensor too large");
  if (a.c & (a.c - 1)) return fail(QPH_EUNSUPPORTED, "depthwise (channel-last): C not a power of two");
  if (a.n * a.oh > 65535) return fail(QPH_EUNSUPPORTED, "depthwise (channel-last): grid too large");
  DwClK p{};
  p.x = a.x; p.w = a.wt; p.bias = a.bias; p.y = a.y;
  p.n = (int)a.n; p.c = (int)a.c; p.h = (int)a.h; p.w_ = (int)a.w;
  p.lc = 0;
  while ((1ll << p.lc) < a.c) p.lc++;
  p.sh = (int)a.sh; p.sw = (int)a.sw; p.ph = (int)a.ph; p.pw = (int)a.pw;
  p.oh = (int)a.oh; p.ow = (int)a.ow;
  p.act = a.act;
  if (a.kh == 3 && a.kw == 3 && a.ow >= 8 && (a.sw == 1 || a.sw == 2))
    return a.sw == 1 ? launch_dwcl_px<1>(p, s) : launch_dwcl_px<2>(p, s);
  const dim3 grid(ceil_div(a.ow * a.c, 256), (unsigned)(a.n * a.oh));
  if (a.kh == 3 && a.kw == 3)
    hipLaunchKernelGGL((depthwise_cl_kernel<3, 3>), grid, dim3(256), 0, s, p);
  else if (a.kh == 5 && a.kw == 5)
    hipLaunchKernelGGL((depthwise_cl_kernel<5, 5>), grid, dim3(256), 0, s, p);
  else
    return fail(QPH_EUNSUPPORTED, "depthwise (channel-last): 3x3 and 5x5 only");
  return launch_check("depthwise_cl_kernel");
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

// Det head tail: ConvT(C->M1) -> ConvT(M1->1) -> Sigmoid in one pass.  An
// input pixel's first ConvT gives a 2x2 block of the intermediate (rounded to
// f32, as the intermediate tensor is); each of those four pixels feeds a 2x2
// block of the second, so one input pixel produces a 4x4 output block.  Wave
// q of a workgroup takes tap q = 2ky + kx of the first ConvT for 64 input
// pixels: its weights are then the same for every lane (scalar loads), and
// it writes the 2x2 output block at (2ky, 2kx) of each pixel's 4x4 block.
template <int C, int M1>
__global__ __launch_bounds__(256) void convt_pair_sigmoid_kernel(const float* __restrict__ x,
                                                                 int64_t h, int64_t w,
                                                                 const float* __restrict__ w1,
                                                                 const float* __restrict__ w2,
                                                                 float* __restrict__ y) {
  static_assert(C % 4 == 0, "whole 16-byte weight rows");
  // weights staged per workgroup as [q][co][ci] (w1, ONNX [ci][co][2][2]) and
  // [co][q2] (w2): a wave reads its tap's rows with broadcast 16-byte reads
  __shared__ __attribute__((aligned(16))) float sw1[4 * M1 * C];
  __shared__ __attribute__((aligned(16))) float sw2[M1 * 4];
  for (int i = threadIdx.x; i < C * M1 * 4; i += 256) {
    const int ci = i / (M1 * 4), co = (i >> 2) % M1, tq = i & 3;
    sw1[(tq * M1 + co) * C + ci] = w1[i];
  }
  for (int i = threadIdx.x; i < M1 * 4; i += 256) sw2[i] = w2[i];
  __syncthreads();
  const int q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t hw = h * w;
  const int64_t pix = (int64_t)blockIdx.x * 64 + (threadIdx.x & 63);
  const int64_t bn = blockIdx.y;
  if (pix >= hw) return;
  const int64_t iy = pix / w, ix = pix - iy * w;
  float xv[C];
  const float* xn = x + bn * C * hw + pix;
#pragma unroll
  for (int ci = 0; ci < C; ci++) xv[ci] = xn[ci * hw];
  // first ConvT, tap q: mid[co] = chain over ci of fma(x[ci], w1[ci][co][q], acc)
  float mid[M1];
  const float* wq = sw1 + q * M1 * C;
#pragma unroll
  for (int co = 0; co < M1; co++) {
    float a = 0.0f;
#pragma unroll
    for (int c4 = 0; c4 < C; c4 += 4) {
      const f32x4 wv = *(const f32x4*)(wq + co * C + c4);
      a = __builtin_fmaf(xv[c4], wv[0], a);
      a = __builtin_fmaf(xv[c4 + 1], wv[1], a);
      a = __builtin_fmaf(xv[c4 + 2], wv[2], a);
      a = __builtin_fmaf(xv[c4 + 3], wv[3], a);
    }
    mid[co] = a;
  }
  // second ConvT on that intermediate pixel (chain over co), then Sigmoid
  f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int co = 0; co < M1; co++) {
    const f32x4 wv = *(const f32x4*)(sw2 + co * 4);
    o[0] = __builtin_fmaf(mid[co], wv[0], o[0]);
    o[1] = __builtin_fmaf(mid[co], wv[1], o[1]);
    o[2] = __builtin_fmaf(mid[co], wv[2], o[2]);
    o[3] = __builtin_fmaf(mid[co], wv[3], o[3]);
  }
  const int ky = q >> 1, kx = q & 1;
  const int64_t ow = 4 * w;
  float* yo = y + (bn * 4 * h + 4 * iy + 2 * ky) * ow + 4 * ix + 2 * kx;
  yo[0] = sigmoid1(o[0]);
  yo[1] = sigmoid1(o[1]);
  yo[ow] = sigmoid1(o[2]);
  yo[ow + 1] = sigmoid1(o[3]);
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
  if (c == 24 && m1 == 24) {
    // 64 input pixels per workgroup, one wave per first-ConvT tap
    if (ceil_div(h * w, 64) >= (1ll << 31)) return fail(QPH_EUNSUPPORTED, "convT pair: grid too large");
    dim3 grid((unsigned)ceil_div(h * w, 64), (unsigned)n);
    hipLaunchKernelGGL((convt_pair_sigmoid_kernel<24, 24>), grid, dim3(256), 0, s, x, h, w, w1, w2, y);
  } else {
    dim3 grid(ceil_div(h * w, 256), (unsigned)n);
    hipLaunchKernelGGL(convt_pair_sigmoid_generic, grid, dim3(256), 0, s, x, c, h, w, w1, m1, w2, y);
  }
  return launch_check("convt_pair_sigmoid_kernel");
}

}  // namespace qph
