// The reference's whole-graph plan model (qppocr-gpu/src/plan.rs) on HIP.
//
// The reference's Vulkan and Metal sessions consume a GraphPlan
// (plan.rs:100-156): one arena of u32 words that holds the activations
// NHWC with channels padded to a multiple of 4 (plan.rs:10-17), the
// parameter blocks and the repacked weights (nhwc.rs:28-204), plus a
// dispatch list naming a kernel of the backend's set
// (vulkan/pipeline.rs:84-136) and the word offset of its parameter block.
// This file is the HIP backend's kernel set for those dispatches.
// qph_plan_create copies the static words into a device arena, decodes
// every parameter block once on the host, checks every region a dispatch
// names against the arena, and captures the launches into a HIP graph;
// qph_plan_run replays it.
//
// Numerics: each dispatch computes the CPU operation it stands for with the
// CPU's operation order, so a plan's outputs are bit-identical to the CPU
// executor running the same node sequence:
//  - n_conv / n_conv8: the conv chain in the CPU's k order (channel, ky,
//    kx) with its bias placement (conv.rs:264-661, gemm.rs:7-16), then the
//    activation, then the residual.  The rule needs the real output channel
//    count and the real input channel count, which a parameter block does
//    not carry (only their padded values); they are exact when both are
//    multiples of 4, as in every det and rec conv.
//  - n_conv_dw: acc = fma(w, x, acc) over ky then kx, + bias (conv.rs:461-505).
//  - n_convt: the chain over input channels from 0, + bias, activation.
//  - n_elem / n_channel: the separately rounded IEEE ops of the CPU nodes,
//    exp1-based sigmoid, fma-based HardSigmoid (activation.rs:168-201).
//  - n_reduce_last, n_reduce_hw + n_reduce_fin: f64 means (shape.rs:510-560,
//    pool2d.rs:10-29); the pair is run as one launch.
//  - n_softmax: the reference softmax (activation.rs:321-403);
//    n_exit3_argmax the first strict maximum (rec.rs:46-54).
//  - n_attn_mm: the batched MatMul's k-ascending fma chains (shape.rs:568-698).
// Real-batch early exit: word 0 of the arena holds real_n (plan.rs:587-593);
// the entry, exit3, pool, depthwise, conv, channel, softmax, row-mean
// (n_reduce_last, n_reduce_hw/fin) and batched-matmul (n_attn_mm) launches
// skip batch rows past it as the reference's kernels do; the pointwise
// GEMM dispatches compute the padded rows too (never read).

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <functional>
#include <memory>
#include <string>
#include <type_traits>
#include <vector>

#include "qph_internal.h"

namespace qph {

namespace {

constexpr uint32_t OFF_NONE = 0xFFFFFFFFu;

const char* const kPlanKernels[] = {
    "n_entry",   "n_exit",      "n_exit3",     "n_exit3_argmax", "n_elem",
    "n_channel", "n_conv",      "n_conv8",     "n_conv_dw",      "n_convt",
    "n_pool",    "n_reduce_hw", "n_reduce_fin", "n_reduce_last", "n_resize",
    "n_transpose", "n_transpose_nd", "n_concat_c", "n_softmax",  "n_attn_mm"};
constexpr int kNumPlanKernels = (int)(sizeof(kPlanKernels) / sizeof(kPlanKernels[0]));
enum {
  PK_ENTRY, PK_EXIT, PK_EXIT3, PK_EXIT3_ARGMAX, PK_ELEM, PK_CHANNEL, PK_CONV, PK_CONV8,
  PK_CONV_DW, PK_CONVT, PK_POOL, PK_REDUCE_HW, PK_REDUCE_FIN, PK_REDUCE_LAST, PK_RESIZE,
  PK_TRANSPOSE, PK_TRANSPOSE_ND, PK_CONCAT_C, PK_SOFTMAX, PK_ATTN_MM
};

__device__ __forceinline__ unsigned real_n(const float* arena) {
  return *(const unsigned*)arena;
}

__device__ __forceinline__ float4 act4(float4 v, const Act& a) {
  return make_float4(act_apply(v.x, a), act_apply(v.y, a), act_apply(v.z, a), act_apply(v.w, a));
}

__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

// ------------------------------------------------------------ entry / exit

// f32 NCHW [nb][c][h][w] -> NHWC [nb][h][w][cpad], pad channels 0 (n_entry.comp).
struct EntryK { const float* arena; const float* x; float* y; int64_t nb, c, hw, cp4; };
__global__ __launch_bounds__(256) void plan_entry_kernel(EntryK p) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= p.nb * p.hw) return;
  const int64_t n = gid / p.hw, pos = gid - n * p.hw;
  const unsigned rn = real_n(p.arena);
  if (rn != 0 && n >= rn) return;
  const float* xn = p.x + n * p.c * p.hw + pos;
  float4* yo = (float4*)p.y + gid * p.cp4;
  for (int64_t c4 = 0; c4 < p.cp4; c4++) {
    const int64_t b = c4 * 4;
    float4 v;
    v.x = b + 0 < p.c ? xn[(b + 0) * p.hw] : 0.0f;
    v.y = b + 1 < p.c ? xn[(b + 1) * p.hw] : 0.0f;
    v.z = b + 2 < p.c ? xn[(b + 2) * p.hw] : 0.0f;
    v.w = b + 3 < p.c ? xn[(b + 3) * p.hw] : 0.0f;
    yo[c4] = v;
  }
}

// NHWC -> NCHW, pad channels dropped, optional sigmoid (n_exit.comp).
struct ExitK { const float* x; float* y; int64_t nb, c, hw, cpad; int sigmoid; };
__global__ __launch_bounds__(256) void plan_exit_kernel(ExitK p) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= p.nb * p.hw) return;
  const int64_t n = gid / p.hw, pos = gid - n * p.hw;
  const float* xr = p.x + gid * p.cpad;
  float* yn = p.y + n * p.c * p.hw + pos;
  for (int64_t c = 0; c < p.c; c++) {
    const float v = xr[c];
    yn[c * p.hw] = p.sigmoid ? sigmoid1(v) : v;
  }
}

// rows x cpad -> rows x cols (n_exit3.comp).
struct Exit3K { const float* arena; const float* x; float* y; int64_t rows, cols, cpad, rpb; };
__global__ __launch_bounds__(256) void plan_exit3_kernel(Exit3K p) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= p.rows * p.cols) return;
  const int64_t row = gid / p.cols, col = gid - row * p.cols;
  const unsigned rn = real_n(p.arena);
  if (rn != 0 && row >= (int64_t)rn * p.rpb) return;
  p.y[gid] = p.x[row * p.cpad + col];
}

// ------------------------------------------------------- elementwise ops

// n_elem.comp op codes: 0 relu, 1 sigmoid, 2 hardsigmoid(p1, p2), 3 clip(p1, p2),
// 4 add, 5 mul, 6 + scalar, 7 * scalar, 8 - row value, 9 square, 10 sqrt,
// 11 / row value, 12 sub, 13 div.  One IEEE operation per element, as the
// CPU nodes (elementwise.rs:40-62, activation.rs:168-239).
struct ElemK { const float* a; const float* b; float* y; int64_t nv; int op; float p1, p2; int64_t c4; };

__device__ __forceinline__ float elem1(int op, float a, float b, float p1, float p2) {
  switch (op) {
    case 0: return relu1(a);
    case 1: return sigmoid1(a);
    case 2: return hsig1(a, p1, p2);
    case 3: {  // clip_seg_scalar (activation.rs:223-229)
      const float m = a < p1 ? p1 : a;
      return p2 < m ? p2 : m;
    }
    case 4: case 6: return a + b;
    case 5: case 7: return a * b;
    case 8: case 12: return a - b;
    case 9: return a * a;  // Pow with the constant exponent 2: powf(a, 2) is a * a rounded
    case 10: return __builtin_sqrtf(a);
    default: return a / b;  // 11, 13
  }
}

__global__ __launch_bounds__(256) void plan_elem_kernel(ElemK p) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.nv) return;
  const float4 a = ((const float4*)p.a)[i];
  float4 b = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (p.op == 4 || p.op == 5 || p.op == 12 || p.op == 13) {
    b = ((const float4*)p.b)[i];
  } else if (p.op == 6 || p.op == 7) {
    const float s = p.b[0];
    b = make_float4(s, s, s, s);
  } else if (p.op == 8 || p.op == 11) {
    const float s = p.b[(i / p.c4) * 4];
    b = make_float4(s, s, s, s);
  }
  float4 o;
  o.x = elem1(p.op, a.x, b.x, p.p1, p.p2);
  o.y = elem1(p.op, a.y, b.y, p.p1, p.p2);
  o.z = elem1(p.op, a.z, b.z, p.p1, p.p2);
  o.w = elem1(p.op, a.w, b.w, p.p1, p.p2);
  ((float4*)p.y)[i] = o;
}

// n_channel.comp: per-channel gate broadcast over the feature rows; gate row
// = feature row / hw.  0 a*g, 1 a+g, 2 a*g + r (MulAddScale, two roundings,
// elementwise.rs:134-179), 3 a * hardsigmoid(g), 4 a * sigmoid(g), 5 a*g + r[gate row].
struct ChannelK {
  const float* arena; const float* a; const float* g; const float* r; float* y;
  int64_t nv, c4, hw; int op; float p1, p2;
};
__global__ __launch_bounds__(256) void plan_channel_kernel(ChannelK p) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.nv) return;
  const int64_t c4 = i % p.c4, frow = i / p.c4, grow = frow / p.hw;
  const unsigned rn = real_n(p.arena);
  if (rn != 0 && frow >= (int64_t)rn * p.hw) return;
  const float4 a = ((const float4*)p.a)[i];
  const float4 g = ((const float4*)p.g)[grow * p.c4 + c4];
  float4 o;
  switch (p.op) {
    case 0: o = make_float4(a.x * g.x, a.y * g.y, a.z * g.z, a.w * g.w); break;
    case 1: o = add4(a, g); break;
    case 2: case 5: {
      const float4 r = ((const float4*)p.r)[p.op == 2 ? i : grow * p.c4 + c4];
      o = add4(make_float4(a.x * g.x, a.y * g.y, a.z * g.z, a.w * g.w), r);
      break;
    }
    case 3:
      o = make_float4(a.x * hsig1(g.x, p.p1, p.p2), a.y * hsig1(g.y, p.p1, p.p2),
                      a.z * hsig1(g.z, p.p1, p.p2), a.w * hsig1(g.w, p.p1, p.p2));
      break;
    default:
      o = make_float4(a.x * sigmoid1(g.x), a.y * sigmoid1(g.y), a.z * sigmoid1(g.z),
                      a.w * sigmoid1(g.w));
      break;
  }
  ((float4*)p.y)[i] = o;
}

// ------------------------------------------------------------ dense conv
//
// NHWC conv on v_mfma_f32_16x16x4f32 (16 output channels x 16 pixels per
// block, the weight operand shared by a wave's blocks).  K runs in
// the CPU's order k = c * taps + t (t = ky * kw + kx); the weights are the
// plan's repack w[(t * cin + c) * N + co] (nhwc.rs:28-57).  Out-of-image taps
// and pad channels contribute 0 (the padded channels come last in k, so
// their +0 terms leave the chain as it was).  The bias enters the chain first
// where the CPU seeds it (rule below), else it is added after; then the
// activation; then the residual.
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct ConvK {
  const float* arena; const float* x; const float* w; const float* bias; const float* res;
  float* y;
  int64_t P, N, ow, oh, iw, ih, cin, taps, kw, sh, sw, pt, pl;
  int rule_kind;   // 0 pointwise sgemm (M = N, N = P), 1 implicit GEMM per row, 2 im2col tiles
  int rule_path;   // 0 panel, 1 m-rows (pointwise only)
  int64_t tile;    // im2col tile height
  Act act;
};

// Whether the bias of output channel co at output row oy, column ox is
// seeded into the chain (else added after it): bias_seeded's rule over the
// GEMM the reference runs for the conv's kind (rule_kind 0: pointwise sgemm
// over all P pixels; 1: one implicit GEMM per output row; 2: im2col tiles of
// `tile` output rows).  32-bit arithmetic: the decoder keeps P N, and so
// every index here, below 2^31.
__device__ __forceinline__ bool conv_seeded_at(const ConvK& p, int co, int oy, int ox) {
  const int N = (int)p.N, ow = (int)p.ow;
  const bool mtail = co >= N - N % 4;
  if (p.rule_kind == 0) {
    const int P = (int)p.P, px = oy * ow + ox;
    if (p.rule_path == 1) return px >= P - P % 32;
    return P - (px & ~31) < 32 && mtail;
  }
  if (p.rule_kind == 1) return ow - (ox & ~31) < 32 && mtail;
  const int tile = (int)p.tile, t0 = oy / tile * tile;
  const int n = min(tile, (int)p.oh - t0) * ow, j = (oy - t0) * ow + ox;
  return n - (j & ~31) < 32 && mtail;
}

__device__ __forceinline__ bool conv_seeded(const ConvK& p, int64_t co, int64_t px) {
  const int oy = (int)px / (int)p.ow;
  return conv_seeded_at(p, (int)co, oy, (int)px - oy * (int)p.ow);
}

constexpr int CONV_NB = 2;  // 16-pixel blocks per wave
constexpr int CONV_CS = 8;  // k-steps (4 k each) loaded per batch

// A wave owns 16 output channels x 32 output pixels.  Lane (li = lane % 16,
// kq = lane / 16) supplies k = 4 s + kq of step s; it walks its (channel,
// ky, kx) by +4 in k without divisions.  Operands move in batches of 8
// steps (three words a step per lane), the next batch's loads in flight
// while this batch's MFMAs run.  Index arithmetic is 32-bit (the launcher
// keeps every region below 2^31 words).
__global__ __launch_bounds__(256) void plan_conv_kernel(ConvK p) {
  const int b = blockIdx.y;
  const unsigned rn = real_n(p.arena);
  if (rn != 0 && (unsigned)b >= rn) return;
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int N = (int)p.N, P = (int)p.P, ow = (int)p.ow;
  const int ncob = (N + 15) >> 4;
  const int co0 = (wave % ncob) * 16, px0 = (wave / ncob) * (16 * CONV_NB);
  if (px0 >= P) return;
  const int li = lane & 15, kq = lane >> 4;
  const int co_a = co0 + li;
  const bool co_ok = co_a < N;
  const int cin = (int)p.cin, taps = (int)p.taps, kw = (int)p.kw, kh = taps / kw;
  const int iw = (int)p.iw, ih = (int)p.ih;
  int iy0[CONV_NB], ix0[CONV_NB];
#pragma unroll
  for (int j = 0; j < CONV_NB; j++) {
    const int px = px0 + 16 * j + li;
    const int oy = px / ow, ox = px - oy * ow;
    iy0[j] = px < P ? oy * (int)p.sh - (int)p.pt : -(1 << 30);
    ix0[j] = ox * (int)p.sw - (int)p.pl;
  }
  const float* xb = p.x + (size_t)b * ih * iw * cin;
  f32x4 acc[CONV_NB];
#pragma unroll
  for (int j = 0; j < CONV_NB; j++) {
    const int px = px0 + 16 * j + li;
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int co = co0 + 4 * kq + v;
      acc[j][v] = (p.bias && co < N && px < P && conv_seeded(p, co, px)) ? p.bias[co] : 0.0f;
    }
  }
  // the lane's first k = kq: k = c * taps + ky * kw + kx
  int c = kq / taps, ky = (kq % taps) / kw, kx = (kq % taps) % kw;
  const int steps = cin * taps / 4;
  // operands of CONV_CS steps per batch: a[u] (weight), b[u][j] (pixels)
  auto load_batch = [&](int s0, float (&a)[CONV_CS], float (&bv)[CONV_CS][CONV_NB]) {
#pragma unroll
    for (int u = 0; u < CONV_CS; u++) {
      if (s0 + u >= steps) break;  // wave-uniform
      a[u] = co_ok ? p.w[((ky * kw + kx) * cin + c) * N + co_a] : 0.0f;
#pragma unroll
      for (int j = 0; j < CONV_NB; j++) {
        const int iy = iy0[j] + ky, ix = ix0[j] + kx;
        const bool in = (unsigned)iy < (unsigned)ih && (unsigned)ix < (unsigned)iw;
        bv[u][j] = in ? xb[(iy * iw + ix) * cin + c] : 0.0f;
      }
      kx += 4;
      while (kx >= kw) {
        kx -= kw;
        if (++ky == kh) {
          ky = 0;
          c++;
        }
      }
    }
  };
  auto mma_batch = [&](int s0, const float (&a)[CONV_CS], const float (&bv)[CONV_CS][CONV_NB]) {
#pragma unroll
    for (int u = 0; u < CONV_CS; u++) {
      if (s0 + u >= steps) break;  // wave-uniform: the chain has exactly K terms
#pragma unroll
      for (int j = 0; j < CONV_NB; j++)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u], bv[u][j], acc[j], 0, 0, 0);
    }
  };
  // two batch buffers: the next batch's loads are in flight during this
  // batch's MFMAs
  float a0[CONV_CS], a1[CONV_CS], b0[CONV_CS][CONV_NB], b1[CONV_CS][CONV_NB];
  load_batch(0, a0, b0);
  for (int s0 = 0; s0 < steps; s0 += 2 * CONV_CS) {
    if (s0 + CONV_CS < steps) load_batch(s0 + CONV_CS, a1, b1);
    mma_batch(s0, a0, b0);
    if (s0 + CONV_CS >= steps) break;
    if (s0 + 2 * CONV_CS < steps) load_batch(s0 + 2 * CONV_CS, a0, b0);
    mma_batch(s0 + CONV_CS, a1, b1);
  }
  const int cob = co0 + 4 * kq;  // multiple of 4, N % 4 == 0: the four rows are all in or out
  if (cob >= N) return;
  const float* yres = p.res ? p.res + (size_t)b * P * N : nullptr;
  float* yb = p.y + (size_t)b * P * N;
#pragma unroll
  for (int j = 0; j < CONV_NB; j++) {
    const int px = px0 + 16 * j + li;
    if (px >= P) continue;
    float o[4];
#pragma unroll
    for (int v = 0; v < 4; v++) {
      float x = acc[j][v];
      if (p.bias && !conv_seeded(p, cob + v, px)) x = x + p.bias[cob + v];
      x = act_apply(x, p.act);
      if (yres) x = x + yres[px * N + cob + v];
      o[v] = x;
    }
    *(float4*)(yb + px * N + cob) = make_float4(o[0], o[1], o[2], o[3]);
  }
}

// The same conv for up to CONV_LDS_TAPS taps with the patch matrix staged in
// LDS: a wave owns 16 output channels x 32 pixels (four independent waves a
// workgroup, each with its own patch area); per group
// of 4 input channels it stores, for each tap t and pixel j, the 16-byte
// channel quad x[pixel(j, t)][4g .. 4g + 3] (0 outside the image) at
// slot t * 32 + j, then runs that group's taps steps (k = c * taps + t within
// the group, the CPU's order) with B read from LDS.  The next group's quads
// and weights are loaded into registers while this group's MFMAs run.
constexpr int CONV_LDS_TAPS = 16;
constexpr int CONV_LDS_SLOTS = (CONV_LDS_TAPS * 32 + 63) / 64;  // quads per lane and group

__global__ __launch_bounds__(256) void plan_conv_lds_kernel(ConvK p) {
  extern __shared__ float4 patches[];  // per wave [taps][32]
  const int b = blockIdx.y;
  const unsigned rn = real_n(p.arena);
  if (rn != 0 && (unsigned)b >= rn) return;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int wave = (int)blockIdx.x * 4 + wv;
  const int N = (int)p.N, P = (int)p.P, ow = (int)p.ow;
  const int ncob = (N + 15) >> 4;
  if (wave >= ncob * ((P + 31) >> 5)) return;
  float4* patch = patches + wv * (int)p.taps * 32;
  const int co0 = (wave % ncob) * 16, px0 = (wave / ncob) * 32;
  const int li = lane & 15, kq = lane >> 4;
  const int co_a = co0 + li;
  const bool co_ok = co_a < N;
  const int cin = (int)p.cin, taps = (int)p.taps, kw = (int)p.kw;
  const int iw = (int)p.iw, ih = (int)p.ih;
  const float* xb = p.x + (size_t)b * ih * iw * cin;
  // Index arithmetic without per-lane divisions: pixel px0 + r is output
  // (oy0, ox0) walked r columns on (one wave-uniform division), a tap t is
  // (t / kw, t % kw) walked from 0, and step u's k = 4 u + kq is walked by 4.
  const int oy0 = px0 / ow, ox0 = px0 - oy0 * ow;
  auto pixel = [&](int r, int& oy, int& ox) {
    oy = oy0;
    ox = ox0 + r;
    while (ox >= ow) {
      ox -= ow;
      oy++;
    }
  };
  // the slots this lane fills: q = lane + 64 i -> (t = q / 32, j = q % 32);
  // their input word offsets (channel 0), -1 outside the image
  int soff[CONV_LDS_SLOTS];
  {
    int oy, ox;
    pixel(lane & 31, oy, ox);
    const bool pin = px0 + (lane & 31) < P;
#pragma unroll
    for (int i = 0; i < CONV_LDS_SLOTS; i++) {
      const int t = 2 * i + (lane >> 5);
      soff[i] = -1;
      if (t < taps && pin) {
        int ky = 0, kx = t;
        while (kx >= kw) {
          kx -= kw;
          ky++;
        }
        const int iy = oy * (int)p.sh - (int)p.pt + ky, ix = ox * (int)p.sw - (int)p.pl + kx;
        if ((unsigned)iy < (unsigned)ih && (unsigned)ix < (unsigned)iw) soff[i] = (iy * iw + ix) * cin;
      }
    }
  }
  f32x4 acc[2];
  int poy[2], pox[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int px = px0 + 16 * j + li;
    pixel(16 * j + li, poy[j], pox[j]);
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int co = co0 + 4 * kq + v;
      acc[j][v] = (p.bias && co < N && px < P && conv_seeded_at(p, co, poy[j], pox[j])) ? p.bias[co]
                                                                                        : 0.0f;
    }
  }
  // step u of a group: k = 4 u + kq -> channel c_u = k / taps, tap t_u = k % taps
  int cu[CONV_LDS_TAPS], tu[CONV_LDS_TAPS];
  {
    int c = 0, t = kq;
    while (t >= taps) {
      t -= taps;
      c++;
    }
#pragma unroll
    for (int u = 0; u < CONV_LDS_TAPS; u++) {
      cu[u] = c;
      tu[u] = t;
      t += 4;
      while (t >= taps) {
        t -= taps;
        c++;
      }
    }
  }
  const int groups = cin / 4;
  float4 quad[CONV_LDS_SLOTS];
  float wa[CONV_LDS_TAPS] = {};
  auto load_group = [&](int g) {
#pragma unroll
    for (int i = 0; i < CONV_LDS_SLOTS; i++)
      quad[i] = soff[i] >= 0 ? *(const float4*)(xb + soff[i] + 4 * g)
                             : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
    for (int u = 0; u < CONV_LDS_TAPS; u++) {
      if (u < taps)  // wave-uniform
        wa[u] = co_ok ? p.w[(tu[u] * cin + 4 * g + cu[u]) * N + co_a] : 0.0f;
    }
  };
  load_group(0);
  for (int g = 0; g < groups; g++) {
#pragma unroll
    for (int i = 0; i < CONV_LDS_SLOTS; i++) {
      const int q = lane + 64 * i;
      if (q < taps * 32) patch[q] = quad[i];
    }
    float wc[CONV_LDS_TAPS];
#pragma unroll
    for (int u = 0; u < CONV_LDS_TAPS; u++) wc[u] = wa[u];
    // the patch area is this wave's alone: wave-scope fences order its
    // writes before the reads below and those reads before the next writes
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (g + 1 < groups) load_group(g + 1);
#pragma unroll
    for (int u = 0; u < CONV_LDS_TAPS; u++) {
      if (u < taps) {  // wave-uniform: the chain has exactly the group's terms
        const float* row = (const float*)(patch + tu[u] * 32);
#pragma unroll
        for (int j = 0; j < 2; j++)
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(wc[u], row[(16 * j + li) * 4 + cu[u]], acc[j],
                                                        0, 0, 0);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  const int cob = co0 + 4 * kq;
  if (cob >= N) return;
  const float* yres = p.res ? p.res + (size_t)b * P * N : nullptr;
  float* yb = p.y + (size_t)b * P * N;
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int px = px0 + 16 * j + li;
    if (px >= P) continue;
    float o[4];
#pragma unroll
    for (int v = 0; v < 4; v++) {
      float x = acc[j][v];
      if (p.bias && !conv_seeded_at(p, cob + v, poy[j], pox[j])) x = x + p.bias[cob + v];
      x = act_apply(x, p.act);
      if (yres) x = x + yres[px * N + cob + v];
      o[v] = x;
    }
    *(float4*)(yb + px * N + cob) = make_float4(o[0], o[1], o[2], o[3]);
  }
}

// The conv for 1, 4 or 9 taps with every operand moved by buffer->LDS
// loads (no staging registers) and CONV_DMA_D groups of 4 input channels in
// flight.  Per group a lane issues XQ loads of channel quads (slot
// q = lane + 64 i: tap q / 32, pixel q % 32; outside the image or past the
// slots an offset past the buffer, which reads 0) and WQ loads of weight
// chunks (chunk r = lane + 64 i: row r / 4 = 4 t + c, output channels
// co0 + 4 (r % 4) .. + 3).  Loads are inline asm, so the compiler adds no
// waits of its own; the wait before group g's steps leaves the loads of
// the groups after it outstanding (vmcnt counts in issue order).  A group's
// buffer is refilled only after every LDS read of it has returned (an
// explicit lgkmcnt(0) ahead of the refill).
constexpr int CONV_DMA_D = 4;

template <int TAPS>
struct DmaGeom {
  static constexpr int XQ = (TAPS * 32 + 63) / 64;   // quad loads per lane and group
  static constexpr int WQ = (TAPS * 16 + 63) / 64;   // weight-chunk loads per lane and group
  static constexpr int L = XQ + WQ;
  static constexpr int BUF = (XQ + WQ) * 64;         // float4 per group buffer
};

template <int TAPS>
__global__ __launch_bounds__(64) void plan_conv_dma_kernel(ConvK p) {
  using G = DmaGeom<TAPS>;
  extern __shared__ float4 ring[];  // CONV_DMA_D buffers of G::BUF float4
  const int b = blockIdx.y;
  const unsigned rn = real_n(p.arena);
  if (rn != 0 && (unsigned)b >= rn) return;
  const int lane = threadIdx.x;
  const int N = (int)p.N, P = (int)p.P, ow = (int)p.ow;
  const int ncob = (N + 15) >> 4;
  const int co0 = (blockIdx.x % ncob) * 16, px0 = (blockIdx.x / ncob) * 32;
  const int li = lane & 15, kq = lane >> 4;
  const int cin = (int)p.cin, kw = (int)p.kw;
  const int iw = (int)p.iw, ih = (int)p.ih;
  const unsigned OOB = 0x80000000u;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.x + (size_t)b * ih * iw * cin), 0, ih * iw * cin * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.w, 0, TAPS * cin * N * 4, 0x00020000);
  int xo[G::XQ], wo[G::WQ];   // word offsets at group 0, -1: reads 0
#pragma unroll
  for (int i = 0; i < G::XQ; i++) {
    const int q = lane + 64 * i, t = q >> 5, px = px0 + (q & 31);
    xo[i] = -1;
    if (t < TAPS && px < P) {
      const int oy = px / ow, ox = px - oy * ow;
      const int iy = oy * (int)p.sh - (int)p.pt + t / kw, ix = ox * (int)p.sw - (int)p.pl + t % kw;
      if ((unsigned)iy < (unsigned)ih && (unsigned)ix < (unsigned)iw) xo[i] = (iy * iw + ix) * cin;
    }
  }
#pragma unroll
  for (int i = 0; i < G::WQ; i++) {
    const int r = lane + 64 * i, row = r >> 2, t = row >> 2, c = row & 3, co = co0 + 4 * (r & 3);
    wo[i] = (row < 4 * TAPS && co < N) ? (t * cin + c) * N + co : -1;
  }
  auto issue = [&](int g) {
    float4* buf = ring + (g % CONV_DMA_D) * G::BUF;
#pragma unroll
    for (int i = 0; i < G::L; i++) {
      const bool isx = i < G::XQ;
      const unsigned off = isx ? (xo[i] >= 0 ? (unsigned)((xo[i] + 4 * g) * 4) : OOB)
                               : (wo[i - G::XQ] >= 0 ? (unsigned)((wo[i - G::XQ] + 4 * g * N) * 4) : OOB);
      const unsigned m = __builtin_amdgcn_readfirstlane(
          (unsigned)(uintptr_t)(__attribute__((address_space(3))) float4*)(buf + 64 * i));
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"   // m0 is reserved; nothing else uses it here
      __asm__ volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m),
                       "v"(off), "s"(isx ? xr : wr)
                       : "m0");
#pragma clang diagnostic pop
    }
  };
  f32x4 acc[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int px = px0 + 16 * j + li;
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int co = co0 + 4 * kq + v;
      acc[j][v] = (p.bias && co < N && px < P && conv_seeded(p, co, px)) ? p.bias[co] : 0.0f;
    }
  }
  const int groups = cin / 4;
#pragma unroll
  for (int g = 0; g < CONV_DMA_D - 1; g++)
    if (g < groups) issue(g);
  for (int g = 0; g < groups; g++) {
    // the refill below lands in the buffer group g - 1 read: every LDS
    // read of it must have returned first (lgkmcnt(0); one-wave workgroup,
    // so no other wave reads it)
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __asm__ volatile("" ::: "memory");
    if (g + CONV_DMA_D - 1 < groups) issue(g + CONV_DMA_D - 1);
    const int ahead = min(CONV_DMA_D - 1, groups - 1 - g);   // groups issued after g
    switch (ahead) {
      case 3: wait_vmcnt<3 * G::L>(); break;
      case 2: wait_vmcnt<2 * G::L>(); break;
      case 1: wait_vmcnt<G::L>(); break;
      default: wait_vmcnt<0>(); break;
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");
    const float* xq = (const float*)(ring + (g % CONV_DMA_D) * G::BUF);
    const float* wq = xq + 4 * 64 * G::XQ;
#pragma unroll
    for (int u = 0; u < TAPS; u++) {
      const int k = 4 * u + kq, c = k / TAPS, t = k - c * TAPS;
      const float a = wq[(4 * t + c) * 16 + li];
#pragma unroll
      for (int j = 0; j < 2; j++)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, xq[(t * 32 + 16 * j + li) * 4 + c], acc[j],
                                                      0, 0, 0);
    }
  }
  const int cob = co0 + 4 * kq;
  if (cob >= N) return;
  const float* yres = p.res ? p.res + (size_t)b * P * N : nullptr;
  float* yb = p.y + (size_t)b * P * N;
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int px = px0 + 16 * j + li;
    if (px >= P) continue;
    float o[4];
#pragma unroll
    for (int v = 0; v < 4; v++) {
      float x = acc[j][v];
      if (p.bias && !conv_seeded(p, cob + v, px)) x = x + p.bias[cob + v];
      x = act_apply(x, p.act);
      if (yres) x = x + yres[px * N + cob + v];
      o[v] = x;
    }
    *(float4*)(yb + px * N + cob) = make_float4(o[0], o[1], o[2], o[3]);
  }
}

// The nets' stems: 3x3 convs over 4 (padded) input channels, stride SW, as
// plan_conv_lds_kernel computes them (one group, k = c * 9 + t, the same
// bias rule and epilogue) with the index arithmetic fixed at compile time:
// a wave owns 32 pixels x 16 NCB output channels, its 9 x 32 patch quads in
// its own LDS area; step u's k = 4 u + kq gives c = k / 9 = (57 k) >> 9 and
// t = k - 9 c (exact for k < 64), a tap's row t / 3 = (11 t) >> 5.
template <int SW, int NCB>
__global__ __launch_bounds__(256) void plan_stem_kernel(ConvK p) {
  __shared__ float4 patches[4][9 * 32];
  const int b = blockIdx.y;
  const unsigned rn = real_n(p.arena);
  if (rn != 0 && (unsigned)b >= rn) return;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int wave = (int)blockIdx.x * 4 + wv;
  const int N = (int)p.N, P = (int)p.P, ow = (int)p.ow;
  const int ncob = (N + 16 * NCB - 1) / (16 * NCB);
  if (wave >= ncob * ((P + 31) >> 5)) return;
  float4* patch = patches[wv];
  const int cb = wave % ncob, co0 = cb * 16 * NCB, px0 = (wave / ncob) * 32;
  const int li = lane & 15, kq = lane >> 4;
  const int iw = (int)p.iw, ih = (int)p.ih;
  const float4* xb = (const float4*)p.x + (size_t)b * ih * iw;
  const int oy0 = px0 / ow, ox0 = px0 - oy0 * ow;
  auto pixel = [&](int r, int& oy, int& ox) {
    oy = oy0;
    ox = ox0 + r;
    while (ox >= ow) {
      ox -= ow;
      oy++;
    }
  };
  // patch slots q = lane + 64 i: tap t = 2 i + lane / 32, pixel r = lane % 32
  float4 quad[5];
  {
    int oy, ox;
    pixel(lane & 31, oy, ox);
    const bool pin = px0 + (lane & 31) < P;
#pragma unroll
    for (int i = 0; i < 5; i++) {
      const int t = 2 * i + (lane >> 5), ky = (t * 11) >> 5, kx = t - 3 * ky;
      const int iy = oy * SW - (int)p.pt + ky, ix = ox * SW - (int)p.pl + kx;
      const bool in = t < 9 && pin && (unsigned)iy < (unsigned)ih && (unsigned)ix < (unsigned)iw;
      quad[i] = in ? xb[iy * iw + ix] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
  }
  float a[9][NCB];
#pragma unroll
  for (int u = 0; u < 9; u++) {
    const int k = 4 * u + kq, c = (k * 57) >> 9, t = k - 9 * c;
#pragma unroll
    for (int nb = 0; nb < NCB; nb++) {
      const int co = co0 + 16 * nb + li;
      a[u][nb] = co < N ? p.w[(t * 4 + c) * N + co] : 0.0f;
    }
  }
  f32x4 acc[NCB][2];
  int poy[2], pox[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    pixel(16 * j + li, poy[j], pox[j]);
    const bool pin = px0 + 16 * j + li < P;
#pragma unroll
    for (int nb = 0; nb < NCB; nb++)
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const int co = co0 + 16 * nb + 4 * kq + v;
        acc[nb][j][v] = (p.bias && co < N && pin && conv_seeded_at(p, co, poy[j], pox[j]))
                            ? p.bias[co]
                            : 0.0f;
      }
  }
#pragma unroll
  for (int i = 0; i < 5; i++) {
    const int q = lane + 64 * i;
    if (q < 9 * 32) patch[q] = quad[i];
  }
  // the patch area is this wave's alone: a wave-scope fence orders the
  // writes before the reads
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int u = 0; u < 9; u++) {
    const int k = 4 * u + kq, c = (k * 57) >> 9, t = k - 9 * c;
    const float* row = (const float*)(patch + t * 32);
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const float bv = row[(16 * j + li) * 4 + c];
#pragma unroll
      for (int nb = 0; nb < NCB; nb++)
        acc[nb][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u][nb], bv, acc[nb][j], 0, 0, 0);
    }
  }
  const float* yres = p.res ? p.res + (size_t)b * P * N : nullptr;
  float* yb = p.y + (size_t)b * P * N;
#pragma unroll
  for (int nb = 0; nb < NCB; nb++) {
    const int cob = co0 + 16 * nb + 4 * kq;
    if (cob >= N) continue;
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int px = px0 + 16 * j + li;
      if (px >= P) continue;
      float o[4];
#pragma unroll
      for (int v = 0; v < 4; v++) {
        float x = acc[nb][j][v];
        if (p.bias && !conv_seeded_at(p, cob + v, poy[j], pox[j])) x = x + p.bias[cob + v];
        x = act_apply(x, p.act);
        if (yres) x = x + yres[px * N + cob + v];
        o[v] = x;
      }
      *(float4*)(yb + px * N + cob) = make_float4(o[0], o[1], o[2], o[3]);
    }
  }
}

// 3x3 convs with stride SW in both directions (the det neck and head over
// the NHWC arena): a workgroup of 2 NCB waves owns 32 consecutive output
// pixels of 2 output rows, wave w computing row w / NCB for the 16-channel
// output block w % NCB.  A stage holds HALO_CG groups of 4 input channels:
// per group the HR x HC halo quads the tile reads (input row iy0 + r, column
// ix0 + col, 0 outside the image) and the group's 36 weight rows (t * 4 + c)
// for all output blocks (past N: 0), loaded once for every wave by
// buffer->LDS loads through a HALO_D-deep ring.  The weight rows are stored
// rotated: unit (t, c, block u) of 16 floats at 4 (t NCB + u) + ((t + c + u)
// & 3), so the four k rows of a step (four consecutive k, whose t + c runs
// through four consecutive values) are on four different bank quarters.
// (A channel-planar copy of the halo, which would do the same for the B
// reads, measured no faster and its LDS cost a workgroup per CU.)  Chain order (k = c * 9 + t within a group,
// groups in order), bias rule and epilogue are plan_conv_dma_kernel's, so the
// outputs are the same bits with the halo and weights loaded once per tile
// instead of once per tap and output block.
#define HALO_CG 2   // channel groups per stage
#define HALO_D 3    // DMA ring depth
// steps the operand reads run ahead: with the waves of several workgroups
// interleaving on each SIMD, two measured faster than three or six (the det
// head conv 30.7 -> 29.5 us, the neck group 38.6 -> 37.8 us, trace medians)
#define HALO_LEAD 2
template <int SW, int NCB>
struct HaloGeom {
  static constexpr int W = 2 * NCB;                    // waves
  static constexpr int HR = SW + 3;                    // halo rows (2 output rows)
  static constexpr int HC = 31 * SW + 3;               // halo columns
  static constexpr int HQ = HR * HC;                   // halo quads per group
  static constexpr int HQP = (HALO_CG * HQ + 63) / 64 * 64;   // halo slots (whole loads)
  static constexpr int WG = 144 * NCB;                 // weight quads per group
  static constexpr int L = (HQP + HALO_CG * WG + 64 * W - 1) / (64 * W);   // loads per wave
  static constexpr int BUF = L * 64 * W;               // float4 per ring stage
  static constexpr size_t lds() { return (size_t)HALO_D * BUF * 16; }
};

// Up to four independent such convs of one batch count, one launch: conv m
// takes workgroups [start[m], start[m + 1]) (the det neck's four smoothing
// convs, whose sizes differ 64-fold, so the small ones run beside the large
// one instead of after it).
#define HALO_GROUP_MAX 4
struct HaloGroup {
  ConvK k[HALO_GROUP_MAX];
  int tiles_x[HALO_GROUP_MAX];
  int start[HALO_GROUP_MAX + 1];
};

template <int SW, int NCB>
__device__ __forceinline__ void plan_conv_halo_tile(const ConvK& p, int tiles_x, int tile,
                                                    float4* ring) {
  using G = HaloGeom<SW, NCB>;
  constexpr int L = G::L;
  const int b = blockIdx.y;
  const unsigned rn = real_n(p.arena);
  if (rn != 0 && (unsigned)b >= rn) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int row = wave / NCB, ub = wave - row * NCB, co0 = ub * 16;
  const int N = (int)p.N, ow = (int)p.ow, P = (int)p.P, oh = P / ow;
  const int ty = tile / tiles_x, oy0 = 2 * ty, ox0 = (tile - ty * tiles_x) * 32;
  const int oy = oy0 + row;
  const int li = lane & 15, kq = lane >> 4;
  const int cin = (int)p.cin, iw = (int)p.iw, ih = (int)p.ih;
  const int groups = cin / 4, stages = (groups + HALO_CG - 1) / HALO_CG;
  const int iy0 = oy0 * SW - (int)p.pt, ix0 = ox0 * SW - (int)p.pl;
  const unsigned OOB = 0x80000000u;
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(p.x + (size_t)b * ih * iw * cin), 0, ih * iw * cin * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      (void*)p.w, 0, 9 * cin * N * 4, 0x00020000);
  // this wave's loads: slots 64 (L wave + i) + lane; halo slots [0, HQP),
  // weight slots [HQP, HQP + CG WG): every load is wholly one or the other.
  // off: word offset at stage 0 (-1 reads 0); cg: the slot's channel group
  int off[L], cgs[L];
#pragma unroll
  for (int i = 0; i < L; i++) {
    const int s = 64 * (L * wave + i) + lane;
    off[i] = -1;
    cgs[i] = 0;
    if (s < HALO_CG * G::HQ) {
      const int cg = s / G::HQ, h = s - cg * G::HQ;
      const int r = h / G::HC, col = h - r * G::HC, iy = iy0 + r, ix = ix0 + col;
      cgs[i] = cg;
      if ((unsigned)iy < (unsigned)ih && (unsigned)ix < (unsigned)iw)
        off[i] = (iy * iw + ix) * cin + 4 * cg;
    } else if (s >= G::HQP && s < G::HQP + HALO_CG * G::WG) {
      // rotated weight units: unit position up = 4 (t NCB + u) + ((t + c + u) & 3)
      const int w = s - G::HQP, cg = w / G::WG, w2 = w - cg * G::WG;
      const int up = w2 >> 2, qq = w2 & 3, tu = up >> 2;
      const int t = tu / NCB, u = tu - t * NCB, c = ((up & 3) - t - u) & 3;
      const int co = 16 * u + 4 * qq;
      cgs[i] = cg;
      if (co < N) off[i] = (t * cin + 4 * cg + c) * N + co;
    }
  }
  auto issue = [&](int st) {
    float4* buf = ring + (st % HALO_D) * G::BUF;
#pragma unroll
    for (int i = 0; i < L; i++) {
      const bool isx = 64 * (L * wave + i) < G::HQP;   // wave-uniform
      const bool live = off[i] >= 0 && HALO_CG * st + cgs[i] < groups;
      const unsigned o =
          live ? (unsigned)((off[i] + (isx ? 4 * HALO_CG * st : 4 * HALO_CG * st * N)) * 4) : OOB;
      const unsigned m = __builtin_amdgcn_readfirstlane(
          (unsigned)(uintptr_t)(__attribute__((address_space(3))) float4*)(buf + 64 * (L * wave + i)));
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"   // m0 is reserved; nothing else uses it here
      __asm__ volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m),
                       "v"(o), "s"(isx ? xr : wr)
                       : "m0");
#pragma clang diagnostic pop
    }
  };
  f32x4 acc[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int ox = ox0 + 16 * j + li;
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int co = co0 + 4 * kq + v;
      acc[j][v] = (p.bias && co < N && ox < ow && oy < oh && conv_seeded_at(p, co, oy, ox))
                      ? p.bias[co]
                      : 0.0f;
    }
  }
  // the steps of the first NG channel groups of a stage (k = c * 9 + t
  // within a group): every operand read from LDS first, then two MFMAs a
  // step, the reads HALO_LEAD steps ahead of their use (left to itself the
  // scheduler reads each step's operands just before its MFMAs)
  auto steps = [&](auto ngc, int st) {
    constexpr int NS = 9 * decltype(ngc)::value;
    const float* hq = (const float*)(ring + (st % HALO_D) * G::BUF);
    const float* wq = hq + 4 * G::HQP;
    float av[NS], bv[NS][2];
#pragma unroll
    for (int s = 0; s < NS; s++) {
      const int cg = s / 9, u = s - cg * 9;
      const int k = 4 * u + kq, c = k / 9, t = k - c * 9, ky = t / 3, kx = t - ky * 3;
      av[s] = wq[4 * G::WG * cg + (4 * (t * NCB + ub) + ((t + c + ub) & 3)) * 16 + li];
#pragma unroll
      for (int j = 0; j < 2; j++)
        bv[s][j] = hq[4 * (cg * G::HQ + (row * SW + ky) * G::HC + (16 * j + li) * SW + kx) + c];
    }
#pragma unroll
    for (int s = 0; s < NS; s++)
#pragma unroll
      for (int j = 0; j < 2; j++)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[s], bv[s][j], acc[j], 0, 0, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 3 * HALO_LEAD, 0);
#pragma unroll
    for (int s = HALO_LEAD; s < NS; s++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * HALO_LEAD, 0);
  };
#pragma unroll
  for (int st = 0; st < HALO_D - 1; st++)
    if (st < stages) issue(st);
  for (int st = 0; st < stages; st++) {
    if (st + 1 < stages)   // this wave's loads of st in; st + 1 may load
      wait_vmcnt<L>();
    else
      wait_vmcnt<0>();
    __builtin_amdgcn_s_waitcnt(0xC07F);   // this wave's reads of the previous buffer are back
    __builtin_amdgcn_s_barrier();         // and every wave's; stage st is in for all
    __asm__ volatile("" ::: "memory");
    if (st + HALO_D - 1 < stages) issue(st + HALO_D - 1);   // into the buffer of st - 1
    if (HALO_CG * st + HALO_CG <= groups)
      steps(std::integral_constant<int, HALO_CG>{}, st);
    else
      steps(std::integral_constant<int, 1>{}, st);   // the odd last group
  }
  const int cob = co0 + 4 * kq;
  if (cob >= N || oy >= oh) return;
  const float* yres = p.res ? p.res + (size_t)b * P * N : nullptr;
  float* yb = p.y + (size_t)b * P * N;
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int ox = ox0 + 16 * j + li;
    if (ox >= ow) continue;
    const int px = oy * ow + ox;
    float o[4];
#pragma unroll
    for (int v = 0; v < 4; v++) {
      float x = acc[j][v];
      if (p.bias && !conv_seeded_at(p, cob + v, oy, ox)) x = x + p.bias[cob + v];
      x = act_apply(x, p.act);
      if (yres) x = x + yres[px * N + cob + v];
      o[v] = x;
    }
    *(float4*)(yb + px * N + cob) = make_float4(o[0], o[1], o[2], o[3]);
  }
}

template <int SW, int NCB>
__global__ __launch_bounds__(128 * NCB) void plan_conv_halo_kernel(ConvK p, int tiles_x) {
  extern __shared__ float4 ring[];
  plan_conv_halo_tile<SW, NCB>(p, tiles_x, (int)blockIdx.x, ring);
}

template <int SW, int NCB>
__global__ __launch_bounds__(128 * NCB) void plan_conv_halo_group_kernel(HaloGroup g) {
  extern __shared__ float4 ring[];
  const int t = (int)blockIdx.x;   // < start[HALO_GROUP_MAX]: the grid is the total
  int m = 0;
#pragma unroll
  for (int i = 1; i < HALO_GROUP_MAX; i++) m += t >= g.start[i] ? 1 : 0;
  plan_conv_halo_tile<SW, NCB>(g.k[m], g.tiles_x[m], t - g.start[m], ring);
}

// ------------------------------------------------------ pointwise, small K
// A 1x1 conv with K = 4 KS input channels (16 or 32: the det blocks' first
// pointwise convs and the 32-channel lateral) over the NHWC rows as one GEMM,
// rows = pixels (m = nb P), columns = channels: a wave owns 16 channels x 32
// pixels.  Its 32 input rows arrive by 16-byte loads (consecutive lanes,
// consecutive words) into a wave-private LDS area, read back per step in the
// MFMA layout (lane (li, kq): x[px0 + 16 j + li][4 s + kq], row pitch K + 1
// so the 16 rows of one read are on different banks); the weights
// W[4 s + kq][co0 + li] come straight from memory.  The chain is KS
// v_mfma_f32_16x16x4f32 in k order from +0, then + bias, the activation and
// the residual: gemm_skinny_kernel's chain and epilogue for this shape.
struct PwK {
  const float* x; const float* w; const float* bias; const float* res; float* y;
  int m, n;
  Act act;
};

template <int KS>
__global__ __launch_bounds__(256) void plan_pw_kernel(PwK p) {
  constexpr int K = 4 * KS, RP = K + 1, Q = 32 * KS / 64;   // Q float4 loads per lane
  __shared__ float tile[4][32 * RP];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int wave = (int)blockIdx.x * 4 + wv;
  const int li = lane & 15, kq = lane >> 4;
  const int nco = (p.n + 15) >> 4;
  const int pt = wave / nco, co0 = (wave - pt * nco) * 16, px0 = pt * 32;
  if (px0 >= p.m) return;
  const int N = p.n, M = p.m;
  float* t = tile[wv];
  // the 32 x K input rows: load q covers float4 q * 64 + lane (row r, quad c)
  float4 xv[Q];
#pragma unroll
  for (int q = 0; q < Q; q++) {
    const int f = q * 64 + lane, r = f / KS, c = f - r * KS;
    xv[q] = px0 + r < M ? ((const float4*)p.x)[(px0 + r) * KS + c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  float a[KS];
  const int co = co0 + li;
#pragma unroll
  for (int s = 0; s < KS; s++) a[s] = co < N ? p.w[(4 * s + kq) * N + co] : 0.0f;
  // epilogue terms, their latency under the chain
  const int cob = co0 + 4 * kq;
  float bv[4], rv[2][4];
#pragma unroll
  for (int v = 0; v < 4; v++) bv[v] = p.bias && cob < N ? p.bias[cob + v] : 0.0f;
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int px = px0 + 16 * j + li;
#pragma unroll
    for (int v = 0; v < 4; v++) rv[j][v] = p.res && cob < N && px < M ? p.res[px * N + cob + v] : 0.0f;
  }
#pragma unroll
  for (int q = 0; q < Q; q++) {
    const int f = q * 64 + lane, r = f / KS, c = f - r * KS;
    float* d = t + r * RP + 4 * c;
    d[0] = xv[q].x;
    d[1] = xv[q].y;
    d[2] = xv[q].z;
    d[3] = xv[q].w;
  }
  // the area is this wave's alone: a wave-scope fence orders the writes
  // before the reads
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  f32x4 acc[2];
#pragma unroll
  for (int j = 0; j < 2; j++) acc[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < KS; s++)
#pragma unroll
    for (int j = 0; j < 2; j++)
      acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], t[(16 * j + li) * RP + 4 * s + kq], acc[j],
                                                    0, 0, 0);
  if (cob >= N) return;
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int px = px0 + 16 * j + li;
    if (px >= M) continue;
    float o[4];
#pragma unroll
    for (int v = 0; v < 4; v++) {
      float x = acc[j][v];
      if (p.bias) x = x + bv[v];
      x = act_apply(x, p.act);
      if (p.res) x = x + rv[j][v];
      o[v] = x;
    }
    *(float4*)(p.y + px * N + cob) = make_float4(o[0], o[1], o[2], o[3]);
  }
}

// ------------------------------------------------------------- depthwise
struct DwK {
  const float* arena; const float* x; const float* w; const float* bias; const float* res;
  float* y;
  int64_t P, c4, ow, iw, ih, taps, kw, sh, sw, pt, pl;
  Act act;
};
__global__ __launch_bounds__(256) void plan_dw_kernel(DwK p) {
  const int64_t b = blockIdx.y;
  const unsigned rn = real_n(p.arena);
  if (rn != 0 && b >= rn) return;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= p.P * p.c4) return;
  const int64_t c4 = gid % p.c4, m = gid / p.c4;
  const int64_t oy = m / p.ow, ox = m - oy * p.ow;
  const float4* xb = (const float4*)p.x + b * p.ih * p.iw * p.c4;
  const float4* w4 = (const float4*)p.w;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int64_t t = 0; t < p.taps; t++) {
    const int64_t ky = t / p.kw, kx = t - ky * p.kw;
    const int64_t iy = oy * p.sh - p.pt + ky, ix = ox * p.sw - p.pl + kx;
    float4 xv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (iy >= 0 && iy < p.ih && ix >= 0 && ix < p.iw) xv = xb[(iy * p.iw + ix) * p.c4 + c4];
    const float4 wv = w4[t * p.c4 + c4];
    acc.x = __builtin_fmaf(wv.x, xv.x, acc.x);
    acc.y = __builtin_fmaf(wv.y, xv.y, acc.y);
    acc.z = __builtin_fmaf(wv.z, xv.z, acc.z);
    acc.w = __builtin_fmaf(wv.w, xv.w, acc.w);
  }
  // yc = acc + bv with bv = 0 when there is no bias (conv.rs:461-505)
  const float4 bv = p.bias ? ((const float4*)p.bias)[c4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  float4 o = act4(add4(acc, bv), p.act);
  if (p.res) o = add4(o, ((const float4*)p.res)[b * p.P * p.c4 + gid]);
  ((float4*)p.y)[b * p.P * p.c4 + gid] = o;
}

// The same depthwise with 4 adjacent output pixels of one channel quad per
// thread (KH x KW taps, x-stride SW, any y-stride): the taps' weight quads
// sit in registers and each input row's 3 SW + KW quads are read once for
// the 4 outputs; threads run channel quads fastest (16-byte loads and stores
// of consecutive lanes are contiguous).  Each output's chain is plan_dw_kernel's.
template <int KH, int KW, int SW>
__global__ __launch_bounds__(256) void plan_dw_px_kernel(DwK p) {
  constexpr int NC = 3 * SW + KW;   // input columns a thread reads per row
  const int64_t b = blockIdx.y;
  const unsigned rn = real_n(p.arena);
  if (rn != 0 && b >= rn) return;
  const int64_t ngx = (p.ow + 3) / 4;
  const int64_t oh = p.P / p.ow;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= oh * ngx * p.c4) return;
  const int64_t c4 = gid % p.c4, m = gid / p.c4;
  const int64_t oy = m / ngx, ox0 = (m - oy * ngx) * 4;
  const float4* xb = (const float4*)p.x + b * p.ih * p.iw * p.c4;
  const float4* w4 = (const float4*)p.w;
  float4 wv[KH * KW];
#pragma unroll
  for (int t = 0; t < KH * KW; t++) wv[t] = w4[t * p.c4 + c4];
  float4 acc[4];
#pragma unroll
  for (int q = 0; q < 4; q++) acc[q] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int ky = 0; ky < KH; ky++) {
    const int64_t iy = oy * p.sh - p.pt + ky;
    const bool rok = iy >= 0 && iy < p.ih;
    float4 xv[NC];
#pragma unroll
    for (int cc = 0; cc < NC; cc++) {
      const int64_t ix = ox0 * SW - p.pl + cc;
      xv[cc] = (rok && ix >= 0 && ix < p.iw) ? xb[(iy * p.iw + ix) * p.c4 + c4]
                                             : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int kx = 0; kx < KW; kx++) {
      const float4 w = wv[ky * KW + kx];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const float4 x = xv[q * SW + kx];
        acc[q].x = __builtin_fmaf(w.x, x.x, acc[q].x);
        acc[q].y = __builtin_fmaf(w.y, x.y, acc[q].y);
        acc[q].z = __builtin_fmaf(w.z, x.z, acc[q].z);
        acc[q].w = __builtin_fmaf(w.w, x.w, acc[q].w);
      }
    }
  }
  // yc = acc + bv with bv = 0 when there is no bias (conv.rs:461-505)
  const float4 bv = p.bias ? ((const float4*)p.bias)[c4] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
  for (int q = 0; q < 4; q++) {
    if (ox0 + q >= p.ow) break;
    const int64_t e = (oy * p.ow + ox0 + q) * p.c4 + c4;
    float4 o = act4(add4(acc[q], bv), p.act);
    if (p.res) o = add4(o, ((const float4*)p.res)[b * p.P * p.c4 + e]);
    ((float4*)p.y)[b * p.P * p.c4 + e] = o;
  }
}

// ------------------------------------------------------- conv transpose
// every output pixel from one tap (kh <= sh, kw <= sw): the chain over the
// (padded) input channels from 0, + bias, activation (n_convt.comp layout)
struct ConvtK {
  const float* x; const float* w; const float* bias; float* y;
  int64_t P, nv, ow, iw, ih, cin, sh, sw, kw;
  Act act;
};
__global__ __launch_bounds__(256) void plan_convt_kernel(ConvtK p) {
  const int64_t b = blockIdx.y;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= p.P * p.nv) return;
  const int64_t n4 = gid % p.nv, m = gid / p.nv;
  const int64_t oy = m / p.ow, ox = m - oy * p.ow;
  const int64_t iy = oy / p.sh, ky = oy - iy * p.sh, ix = ox / p.sw, kx = ox - ix * p.sw;
  const int64_t tap = ky * p.kw + kx;
  const float* xr = p.x + (b * p.ih * p.iw + iy * p.iw + ix) * p.cin;
  const float4* w4 = (const float4*)p.w + tap * p.cin * p.nv + n4;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int64_t ci = 0; ci < p.cin; ci++) {
    const float xv = xr[ci];
    const float4 wv = w4[ci * p.nv];
    acc.x = __builtin_fmaf(xv, wv.x, acc.x);
    acc.y = __builtin_fmaf(xv, wv.y, acc.y);
    acc.z = __builtin_fmaf(xv, wv.z, acc.z);
    acc.w = __builtin_fmaf(xv, wv.w, acc.w);
  }
  if (p.bias) acc = add4(acc, ((const float4*)p.bias)[n4]);
  ((float4*)p.y)[b * p.P * p.nv + gid] = act4(acc, p.act);
}

// The det head's tail: an n_convt (2x2, stride 2, CI -> CM channels) whose
// output only a second such n_convt (CM -> at most 4 channels) reads, whose
// output only an n_exit (NHWC -> NCHW, sigmoid or not) reads, in one pass.
// A thread takes one pixel of the middle map: its CM channels by
// plan_convt_kernel's chains (input channels ascending from +0, + bias, the
// activation), then the 2 x 2 output pixels it feeds (the same chains over
// the CM channels) through the exit into NCHW.  A block's threads share the
// tap parity of their middle pixel (blockIdx.y), so every weight a chain
// reads is the same for the whole block (scalar loads).
struct ConvtPairK {
  const float* arena;
  const float* x; const float* w1; const float* b1; const float* w2; const float* b2; float* y;
  int h, w;          // input map; the middle map is 2h x 2w, the output 4h x 4w
  int co2p, c_out;   // second conv's padded channels (weight pitch), exported channels
  Act act1, act2;
  int sigmoid;
};
template <int CI, int CM>
__global__ __launch_bounds__(256) void plan_convt_pair_kernel(ConvtPairK p) {
  const int b = blockIdx.z, py = blockIdx.y >> 1, px = blockIdx.y & 1;
  const unsigned rn = real_n(p.arena);
  if (rn != 0 && (unsigned)b >= rn) return;
  const int t = (int)blockIdx.x * 256 + (int)threadIdx.x;
  if (t >= p.h * p.w) return;
  const int i = t / p.w, j = t - i * p.w;
  float xv[CI];
  const float4* xr = (const float4*)(p.x + ((size_t)(b * p.h + i) * p.w + j) * CI);
#pragma unroll
  for (int q = 0; q < CI / 4; q++) {
    const float4 v = xr[q];
    xv[4 * q] = v.x;
    xv[4 * q + 1] = v.y;
    xv[4 * q + 2] = v.z;
    xv[4 * q + 3] = v.w;
  }
  const float* w1 = p.w1 + (size_t)(py * 2 + px) * CI * CM;   // [tap][ci][CM]
  float m[CM];
#pragma unroll
  for (int c = 0; c < CM; c++) {
    float acc = 0.0f;
#pragma unroll
    for (int ci = 0; ci < CI; ci++) acc = __builtin_fmaf(xv[ci], w1[ci * CM + c], acc);
    if (p.b1) acc = acc + p.b1[c];
    m[c] = act_apply(acc, p.act1);
  }
  const int H2 = 4 * p.h, W2 = 4 * p.w;
  const int my = 2 * i + py, mx = 2 * j + px;
#pragma unroll
  for (int qy = 0; qy < 2; qy++)
#pragma unroll
    for (int qx = 0; qx < 2; qx++) {
      const float* w2 = p.w2 + (size_t)(qy * 2 + qx) * CM * p.co2p;   // [tap][c][co2p]
      const int oy = 2 * my + qy, ox = 2 * mx + qx;
#pragma unroll
      for (int o = 0; o < 4; o++) {
        if (o >= p.c_out) break;
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < CM; c++) acc = __builtin_fmaf(m[c], w2[c * p.co2p + o], acc);
        if (p.b2) acc = acc + p.b2[o];
        acc = act_apply(acc, p.act2);
        p.y[((size_t)(b * p.c_out + o) * H2 + oy) * W2 + ox] = p.sigmoid ? sigmoid1(acc) : acc;
      }
    }
}

// ------------------------------------------------------------------ pool
// pool2d.rs:94-259 on NHWC (see pool2d_kernel for the arithmetic)
struct PoolNK {
  const float* arena; const float* x; float* y;
  int64_t P, c4, ow, iw, ih, kh, kw, sh, sw, pt, pl;
  int max_pool, special;
};
__device__ __forceinline__ float pool_acc(bool mx, float acc, float t) {
  return mx ? (t > acc ? t : acc) : acc + t;
}
__global__ __launch_bounds__(256) void plan_pool_kernel(PoolNK p) {
  const int64_t b = blockIdx.y;
  const unsigned rn = real_n(p.arena);
  if (rn != 0 && b >= rn) return;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= p.P * p.c4) return;
  const int64_t c4 = gid % p.c4, m = gid / p.c4;
  const int64_t oy = m / p.ow, ox = m - oy * p.ow;
  const float4* xb = (const float4*)p.x + b * p.ih * p.iw * p.c4;
  float4 o;
  if (p.special) {  // 2x2 stride 1 SAME_UPPER max (pool2x2_row_scalar, pool2d.rs:242-259)
    const bool r1 = oy + 1 < p.ih;
    const float4 a0 = xb[(oy * p.iw + ox) * p.c4 + c4];
    float4 va = a0;
    if (r1) {
      const float4 a1 = xb[((oy + 1) * p.iw + ox) * p.c4 + c4];
      va = make_float4(fmaxf(a0.x, a1.x), fmaxf(a0.y, a1.y), fmaxf(a0.z, a1.z), fmaxf(a0.w, a1.w));
    }
    float4 vb = make_float4(-3.40282347e38f, -3.40282347e38f, -3.40282347e38f, -3.40282347e38f);
    if (ox + 1 < p.iw) {
      const float4 b0 = xb[(oy * p.iw + ox + 1) * p.c4 + c4];
      vb = b0;
      if (r1) {
        const float4 b1 = xb[((oy + 1) * p.iw + ox + 1) * p.c4 + c4];
        vb = make_float4(fmaxf(b0.x, b1.x), fmaxf(b0.y, b1.y), fmaxf(b0.z, b1.z), fmaxf(b0.w, b1.w));
      }
    }
    o = make_float4(fmaxf(va.x, vb.x), fmaxf(va.y, vb.y), fmaxf(va.z, vb.z), fmaxf(va.w, vb.w));
  } else {
    const bool mx = p.max_pool;
    const float init = mx ? -3.4e38f : 0.0f;
    float4 acc = make_float4(init, init, init, init);
    for (int64_t ky = 0; ky < p.kh; ky++) {
      const int64_t iy = oy * p.sh - p.pt + ky;
      if (iy < 0 || iy >= p.ih) continue;
      for (int64_t kx = 0; kx < p.kw; kx++) {
        const int64_t ix = ox * p.sw - p.pl + kx;
        if (ix < 0 || ix >= p.iw) continue;
        const float4 t = xb[(iy * p.iw + ix) * p.c4 + c4];
        acc = make_float4(pool_acc(mx, acc.x, t.x), pool_acc(mx, acc.y, t.y),
                          pool_acc(mx, acc.z, t.z), pool_acc(mx, acc.w, t.w));
      }
    }
    if (!mx) {
      const float area = (float)(p.kh * p.kw);
      acc = make_float4(acc.x / area, acc.y / area, acc.z / area, acc.w / area);
    }
    o = acc;
  }
  ((float4*)p.y)[b * p.P * p.c4 + gid] = o;
}

// ------------------------------------------------------ nearest resize
// resize.rs:26-57: iy = min((int)((float)oy * (float)H / (float)oh), H - 1)
struct ResizeNK { const float* x; float* y; int64_t P, c4, ow, oh, iw, ih; };
__global__ __launch_bounds__(256) void plan_resize_kernel(ResizeNK p) {
  const int64_t b = blockIdx.y;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= p.P * p.c4) return;
  const int64_t c4 = gid % p.c4, m = gid / p.c4;
  const int64_t oy = m / p.ow, ox = m - oy * p.ow;
  int64_t iy = (int64_t)((float)oy * (float)p.ih / (float)p.oh);
  int64_t ix = (int64_t)((float)ox * (float)p.iw / (float)p.ow);
  if (iy > p.ih - 1) iy = p.ih - 1;
  if (ix > p.iw - 1) ix = p.iw - 1;
  const float4* xb = (const float4*)p.x + b * p.ih * p.iw * p.c4;
  ((float4*)p.y)[b * p.P * p.c4 + gid] = xb[(iy * p.iw + ix) * p.c4 + c4];
}

// plan_resize_kernel's nearest source row (or column) of output o
__device__ __forceinline__ int resize_src(int o, int in, int out) {
  const int i = (int)((float)o * (float)in / (float)out);
  return i > in - 1 ? in - 1 : i;
}

// n_resize (nearest) followed by the n_elem add of its output and another
// tensor, as one pass: y = a + resize(x) (the add commutes bitwise).  32-bit
// indices (the decoder checks the sizes).
struct ResizeAddK { const float* arena; const float4* x; const float4* a; float4* y; int P, c4, ow, oh, iw, ih; };
__global__ __launch_bounds__(256) void plan_resize_add_kernel(ResizeAddK p) {
  const int b = blockIdx.y;
  const unsigned rn = real_n(p.arena);
  if (rn != 0 && (unsigned)b >= rn) return;
  const int gid = (int)blockIdx.x * 256 + (int)threadIdx.x;
  if (gid >= p.P * p.c4) return;
  const int m = gid / p.c4, c4 = gid - m * p.c4;
  const int oy = m / p.ow, ox = m - oy * p.ow;
  const int iy = resize_src(oy, p.ih, p.oh), ix = resize_src(ox, p.iw, p.ow);
  const float4 r = p.x[(b * p.ih * p.iw + iy * p.iw + ix) * p.c4 + c4];
  const float4 v = p.a[b * p.P * p.c4 + gid];
  p.y[b * p.P * p.c4 + gid] = make_float4(v.x + r.x, v.y + r.y, v.z + r.z, v.w + r.w);
}

// n_concat_c whose inputs may be n_resize outputs read through (input i
// with ih[i] > 0 is the resize source of ih[i] x iw[i] pixels, mapped as
// plan_resize_kernel maps it onto the oh x ow output).
struct ConcatUpK {
  float4* y;
  int npx, outc4, n, oh, ow;
  const float4* src[8];
  int c4len[8], ih[8], iw[8];
};
__global__ __launch_bounds__(256) void plan_concat_up_kernel(ConcatUpK p) {
  const int gid = (int)blockIdx.x * 256 + (int)threadIdx.x;
  if (gid >= p.npx * p.outc4) return;
  const int pos = gid / p.outc4, c4 = gid - pos * p.outc4;
  int acc = 0;
  for (int i = 0; i < p.n; i++) {
    if (c4 < acc + p.c4len[i]) {
      int sp = pos;
      if (p.ih[i] > 0) {
        const int hw = p.oh * p.ow, b = pos / hw, r = pos - b * hw;
        const int oy = r / p.ow, ox = r - oy * p.ow;
        sp = (b * p.ih[i] + resize_src(oy, p.ih[i], p.oh)) * p.iw[i] + resize_src(ox, p.iw[i], p.ow);
      }
      p.y[gid] = p.src[i][sp * p.c4len[i] + (c4 - acc)];
      return;
    }
    acc += p.c4len[i];
  }
}

// ------------------------------------------------------ data movement
struct Transpose2K { const float* x; float* y; int64_t r, c; };
__global__ __launch_bounds__(256) void plan_transpose2_kernel(Transpose2K p) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.r * p.c) return;
  const int64_t x = i / p.r, y = i - x * p.r;  // out[x][y] = in[y][x]
  p.y[i] = p.x[y * p.c + x];
}

struct TransposeNK { const float* x; float* y; int64_t total; int rank; int64_t dims[5]; int perm[5]; };
__global__ __launch_bounds__(256) void plan_transpose_nd_kernel(TransposeNK p) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.total) return;
  int64_t oc[5] = {0, 0, 0, 0, 0}, ic[5] = {0, 0, 0, 0, 0};
  int64_t rem = i;
  for (int d = p.rank - 1; d >= 0; d--) {
    const int64_t od = p.dims[p.perm[d]];
    oc[d] = rem % od;
    rem /= od;
  }
  for (int d = 0; d < p.rank; d++) ic[p.perm[d]] = oc[d];
  int64_t src = 0;
  for (int d = 0; d < p.rank; d++) src = src * p.dims[d] + ic[d];
  p.y[i] = p.x[src];
}

// The same permutation in 32-bit index arithmetic (element count below
// 2^31), V consecutive elements a thread: with V = 4 the innermost axis stays
// innermost and is a multiple of 4 (the attention's head split and merge),
// so 4 consecutive output elements are 4 consecutive input elements.  Axis d
// of the output has od[d] units (of V elements) and input stride is[d] units.
struct TransposeFastK { const float* x; float* y; unsigned units; int rank; unsigned od[5], is[5]; };
template <int V>
__global__ __launch_bounds__(256) void plan_transpose_fast_kernel(TransposeFastK p) {
  using T = typename std::conditional<V == 4, float4, float>::type;
  const unsigned i = blockIdx.x * 256u + threadIdx.x;
  if (i >= p.units) return;
  unsigned rem = i, src = 0;
#pragma unroll
  for (int d = 4; d >= 0; d--) {
    if (d >= p.rank) continue;
    const unsigned c = rem % p.od[d];
    rem /= p.od[d];
    src += c * p.is[d];
  }
  ((T*)p.y)[i] = ((const T*)p.x)[src];
}

struct ConcatK { const float* arena; float* y; int64_t hw, outc4; int n; uint32_t src[8]; int64_t c4len[8]; };
__global__ __launch_bounds__(256) void plan_concat_kernel(ConcatK p) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= p.hw * p.outc4) return;
  const int64_t c4 = gid % p.outc4, pos = gid / p.outc4;
  int64_t acc = 0;
  for (int i = 0; i < p.n; i++) {
    if (c4 < acc + p.c4len[i]) {
      const float4* s = (const float4*)(p.arena + p.src[i]);
      ((float4*)p.y)[gid] = s[pos * p.c4len[i] + (c4 - acc)];
      return;
    }
    acc += p.c4len[i];
  }
}

// pad columns [cols, cpad) of rows x cpad set to 0 (n_softmax.comp's tail)
// the softmax output's pad columns (n_softmax.comp writes them in the row's
// pass, so rows past the real batch keep theirs)
struct PadColsK { const float* arena; float* y; int64_t rows, cols, cpad, rpb; };
__global__ __launch_bounds__(256) void plan_pad_cols_kernel(PadColsK p) {
  const int64_t w = p.cpad - p.cols;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= p.rows * w) return;
  const int64_t r = i / w;
  const unsigned rn = real_n(p.arena);
  if (rn != 0 && r >= (int64_t)rn * p.rpb) return;
  p.y[r * p.cpad + p.cols + (i - r * w)] = 0.0f;
}

// word 0 of the arena: the run's real batch count, passed by value
__global__ void plan_set_real_n_kernel(unsigned* arena, unsigned real_n) {
  if (threadIdx.x == 0) arena[0] = real_n;
}

inline unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

// ------------------------------------------------------------ the plan

struct PlanUpload {
  uint32_t off, n;
  const uint32_t* words;
};

}  // namespace qph

struct qph_plan {
  qph_ctx* ctx;
  uint32_t total_words;
  float* arena;
  std::vector<std::function<int(hipStream_t)>> launches;
  std::vector<int32_t> launch_dispatch;  // first dispatch of each launch
  hipGraph_t graph;
  hipGraphExec_t exec;
  bool graph_ready;
  uint32_t in_off;
  int64_t in_numel;
  std::vector<uint32_t> out_off;
  std::vector<int64_t> out_numel;
  uint32_t real_n;
  std::vector<float*> owned;  // transposed weight copies for the resident-weight GEMM
};

namespace qph {
namespace {

struct Decoder {
  qph_plan* pl;
  // dry: validation only (qph_plan_validate, and qph_plan_create before it
  // touches the device): no device memory, nothing copied or launched; the
  // launches recorded into pl are discarded
  bool dry = false;
  std::vector<PlanUpload> ups;  // sorted by offset
  int idx = 0;
  const char* kname = "";
  uint32_t p_off = 0;
  // the dispatch list, what each dispatch reads and writes (word offsets of
  // its regions), the graph outputs, and the dispatches a fused launch took
  const qph_plan_dispatch* disp = nullptr;
  int n_disp = 0;
  std::vector<uint32_t> wr;
  std::vector<std::vector<uint32_t>> rd;
  std::vector<uint32_t> outs;
  std::vector<char> skip;
  // an open group of 3x3 halo convs launched together (first member's
  // position); see join_halo_group
  struct Span { uint64_t lo, hi; };
  struct HaloOpen {
    std::shared_ptr<HaloGroup> g;
    int n = 0, sw = 0, ncb = 0;
    int64_t nb = 0;
    int last = -1;                    // dispatch index of the last member
    std::vector<Span> reads, writes;  // the members' and the dispatches' between them
  };
  HaloOpen halo;
  // n_resize dispatches a later n_concat_c reads through: output region ->
  // source region and geometry
  struct Resized { uint32_t out, src; int64_t nb, ih, iw, oh, ow, c4; };
  std::vector<Resized> resized;

  std::string where() const {
    return "plan dispatch " + std::to_string(idx) + " (" + kname + ", params at word " +
           std::to_string(p_off) + ")";
  }
  // the n words at off from the uploaded static words, or nullptr
  const uint32_t* find(uint32_t off, uint32_t n) const {
    auto it = std::upper_bound(ups.begin(), ups.end(), off,
                               [](uint32_t v, const PlanUpload& u) { return v < u.off; });
    if (it == ups.begin()) return nullptr;
    --it;
    if ((uint64_t)off + n > (uint64_t)it->off + it->n) return nullptr;
    return it->words + (off - it->off);
  }
  // the parameter block [p_off, p_off + n) of the dispatch being decoded
  int params(uint32_t n, const uint32_t** out) {
    *out = find(p_off, n);
    if (!*out)
      return fail(QPH_EINVAL, where() + ": parameter block of " + std::to_string(n) +
                                  " words not uploaded");
    return QPH_OK;
  }
  // dispatch j's parameter block (lookahead), nullptr when j is past the end,
  // is another kernel or has a short block
  const uint32_t* peek(int j, int kernel, uint32_t n) const {
    if (j >= n_disp || disp[j].kernel != kernel || skip[j]) return nullptr;
    return find(disp[j].p_off, n);
  }
  // true when no dispatch after `after` other than those in ok reads a word
  // of [o, o + len) before a later dispatch writes into it, and no graph
  // output lies in it
  bool only_readers(int after, uint32_t o, uint64_t len, std::initializer_list<int> ok) const {
    const uint64_t e = (uint64_t)o + len;
    for (uint32_t g : outs)
      if (g >= o && g < e) return false;
    for (int j = after + 1; j < n_disp; j++) {
      bool reads = false;
      for (uint32_t r : rd[j]) reads = reads || (r >= o && r < e);
      if (reads && std::find(ok.begin(), ok.end(), j) == ok.end()) return false;
      if (wr[j] >= o && wr[j] < e) return true;
    }
    return true;
  }
  // a region of n words at off inside the arena (16-byte aligned for vec4 access)
  int region(uint32_t off, uint64_t n, bool vec4, const char* what) {
    if (off == OFF_NONE || (uint64_t)off + n > pl->total_words)
      return fail(QPH_EINVAL, where() + ": " + what + " [" + std::to_string(off) + ", +" +
                                  std::to_string(n) + ") outside the arena of " +
                                  std::to_string(pl->total_words) + " words");
    if (vec4 && off % 4)
      return fail(QPH_EINVAL, where() + ": " + what + " not 16-byte aligned");
    return QPH_OK;
  }
  // device address of word off (in a dry pass: of an arena based at 256,
  // so alignment tests see what the real 256-byte aligned arena gives)
  float* at(uint32_t off) const {
    const uintptr_t base = dry ? (uintptr_t)256 : (uintptr_t)pl->arena;
    return (float*)(base + (uintptr_t)off * 4);
  }
};

// Word counts of the parameter blocks (the n_*.comp layouts; n_concat_c has
// 4 + 2 per input).
const uint32_t kParamWords[kNumPlanKernels] = {7, 8, 6, 6, 7, 10, 21, 21, 20, 18,
                                               14, 4, 5, 6, 9, 4, 14, 4, 6, 8};

// What dispatch q reads (region start offsets) and writes.
void dispatch_io(const Decoder& d, const qph_plan_dispatch& q, uint32_t* wr,
                 std::vector<uint32_t>* rd) {
  *wr = OFF_NONE;
  rd->clear();
  if (q.kernel < 0 || q.kernel >= kNumPlanKernels) return;
  const uint32_t* w = d.find(q.p_off, kParamWords[q.kernel]);
  if (!w) return;
  auto r = [&](std::initializer_list<int> idx) {
    for (int i : idx)
      if (w[i] != OFF_NONE) rd->push_back(w[i]);
  };
  switch (q.kernel) {
    case PK_ELEM: r({1, 2}); *wr = w[3]; break;
    case PK_CHANNEL: r({1, 2, 3}); *wr = w[4]; break;
    case PK_CONV: case PK_CONV8: r({0, 1, 2, 20}); *wr = w[3]; break;
    case PK_CONV_DW: r({0, 1, 2, 19}); *wr = w[3]; break;
    case PK_CONVT: r({0, 1, 2}); *wr = w[3]; break;
    case PK_ATTN_MM: r({0, 1}); *wr = w[2]; break;
    case PK_CONCAT_C: {
      const uint32_t n = w[2];
      if (n > 8 || !(w = d.find(q.p_off, 4 + 2 * n))) return;
      for (uint32_t i = 0; i < n; i++) rd->push_back(w[4 + 2 * i]);
      *wr = w[0];
      break;
    }
    default: r({0}); *wr = w[1]; break;  // entry, exits, pool, reductions, resize, transposes, softmax
  }
}

// The epilogue of a conv-family launch after absorbing the dispatches that
// only consume its output: act (hardswish from n_elem 2 + n_elem 5 on it),
// a per-column bias (the [V] broadcast n_channel 1 after a MatMul), a
// residual (n_elem 4), and the region the fused launch writes.  Each step is
// the operation the absorbed dispatch performs, in the same order (bias,
// activation, residual), so the values are those of the separate dispatches.
struct Epi {
  uint32_t y;
  Act act;
  uint32_t bias, res;
};

int absorb(Decoder& d, uint64_t len, int64_t cols, bool gemm, Epi* e) {
  int last = d.idx;   // the dispatch whose output e->y is
  for (int j = d.idx + 1; j < d.n_disp; j = last + 1) {
    const uint32_t* w;
    const uint32_t* w2;
    if (e->act.kind == 0 && e->res == OFF_NONE && (w = d.peek(j, PK_ELEM, 7)) && w[0] == 2 &&
        w[1] == e->y && w[4] == len && (w2 = d.peek(j + 1, PK_ELEM, 7)) && w2[0] == 5 &&
        w2[4] == len &&
        ((w2[1] == e->y && w2[2] == w[3]) || (w2[1] == w[3] && w2[2] == e->y)) &&
        d.only_readers(last, e->y, len, {j, j + 1}) && d.only_readers(j, w[3], len, {j + 1})) {
      QPH_TRY(d.region(w2[3], len, true, "fused output"));
      qph_act a{};
      a.kind = QPH_ACT_HARDSWISH;
      std::memcpy(&a.c1, &w[5], 4);
      std::memcpy(&a.c2, &w[6], 4);
      e->act = make_act(&a);
      e->y = w2[3];
      d.skip[j] = d.skip[j + 1] = 1;
      last = j + 1;
      continue;
    }
    if (gemm && e->bias == OFF_NONE && e->act.kind == 0 && e->res == OFF_NONE &&
        (w = d.peek(j, PK_CHANNEL, 10)) && w[0] == 1 && w[1] == e->y && w[5] == len &&
        (int64_t)w[6] == cols && (uint64_t)w[9] * cols == len &&
        d.only_readers(last, e->y, len, {j})) {
      QPH_TRY(d.region(w[2], (uint64_t)cols, true, "fused bias"));
      QPH_TRY(d.region(w[4], len, true, "fused output"));
      e->bias = w[2];
      e->y = w[4];
      d.skip[j] = 1;
      last = j;
      continue;
    }
    if (e->res == OFF_NONE && (w = d.peek(j, PK_ELEM, 7)) && w[0] == 4 && w[4] == len &&
        (w[1] == e->y || w[2] == e->y) && w[1] != w[2] && d.only_readers(last, e->y, len, {j})) {
      const uint32_t other = w[1] == e->y ? w[2] : w[1];
      QPH_TRY(d.region(other, len, true, "fused residual"));
      QPH_TRY(d.region(w[3], len, true, "fused output"));
      e->res = other;
      e->y = w[3];
      d.skip[j] = 1;
      last = j;
    }
    break;  // nothing follows a residual
  }
  return QPH_OK;
}

inline float f32_of(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

// the conv family's act word (plan.rs:1346): 0 none, 1 gelu(c1, c2, c3), 2 relu
int conv_act(Decoder& d, uint32_t act, float c1, float c2, float c3, Act* out) {
  qph_act a{};
  if (act == 0) {
    a.kind = QPH_ACT_NONE;
  } else if (act == 1) {
    a.kind = QPH_ACT_GELU; a.c1 = c1; a.c2 = c2; a.c3 = c3;
  } else if (act == 2) {
    a.kind = QPH_ACT_RELU;
  } else {
    return fail(QPH_EUNSUPPORTED, d.where() + ": activation " + std::to_string(act));
  }
  if (act == 1 && !(c1 != 0.0f)) return fail(QPH_EINVAL, d.where() + ": gelu with c1 = 0");
  if (act != 1) a.c1 = 1.0f;
  *out = make_act(&a);
  return QPH_OK;
}

int add_launch(qph_plan* pl, int dispatch, std::function<int(hipStream_t)> f) {
  pl->launches.push_back(std::move(f));
  pl->launch_dispatch.push_back(dispatch);
  return QPH_OK;
}

struct PendingHw { uint32_t in, scratch; int64_t m, c, nb; };


// A 3x3 halo conv joins the open group (and launches with its first member,
// earlier in the launch order) when: the group has room and the same
// stride, output-block count and batch count; every dispatch since the
// group's last member is an n_resize (the det neck's pattern: smoothing conv,
// upsample, smoothing conv, ...); and none of the regions this conv's launch
// reads (input, weights, bias, residual) overlaps a region written by a
// member or by those n_resize dispatches, nor does the region it writes
// overlap one they read or write.  Its absorbed epilogue moves with it.
bool join_halo_group(Decoder& d, const ConvK& k, int tiles_x, int64_t oh, int sw, int ncb,
                     int64_t nb, const std::vector<Decoder::Span>& rd, const Decoder::Span& wr) {
  Decoder::HaloOpen& h = d.halo;
  if (!h.g || h.n >= HALO_GROUP_MAX || h.sw != sw || h.ncb != ncb || h.nb != nb) return false;
  auto over = [](const Decoder::Span& a, const Decoder::Span& b) { return a.lo < b.hi && b.lo < a.hi; };
  std::vector<Decoder::Span> reads = h.reads, writes = h.writes;
  for (int m = h.last + 1; m < d.idx; m++) {
    const qph_plan_dispatch& q = d.disp[m];
    if (q.kernel == PK_RESIZE && d.skip[(size_t)m]) continue;   // read through by a concat
    const uint32_t* w = q.kernel == PK_RESIZE ? d.find(q.p_off, 9) : nullptr;
    if (!w || d.skip[(size_t)m]) return false;
    const uint64_t nbm = q.groups[1];
    reads.push_back({w[0], w[0] + nbm * w[5] * w[6] * w[3]});
    writes.push_back({w[1], w[1] + nbm * w[2] * w[3]});
  }
  for (const auto& r : rd)
    for (const auto& w : writes)
      if (over(r, w)) return false;
  for (const auto& w : writes)
    if (over(wr, w)) return false;
  for (const auto& r : reads)
    if (over(wr, r)) return false;
  HaloGroup& g = *h.g;
  const int i = h.n++;
  g.k[i] = k;
  g.tiles_x[i] = tiles_x;
  g.start[i + 1] = g.start[i] + (int)((oh + 1) / 2 * tiles_x);
  for (int j = i + 2; j <= HALO_GROUP_MAX; j++) g.start[j] = g.start[i + 1];
  h.reads = reads;
  for (const auto& r : rd) h.reads.push_back(r);
  h.writes = writes;
  h.writes.push_back(wr);
  h.last = d.idx;
  return true;
}

// The attention lowering PlanBuilder writes after the QKV projection
// (plan.rs attention): n_transpose_nd of the [B, T, 3, H, dh] rows to
// [3, B, H, T, dh]; q times the scale (n_elem 7); k transposed per head;
// S = q k^T (n_attn_mm); P = softmax(S) over T; O = P v (n_attn_mm); O
// back to [B, T, H, dh].  When the seven dispatches are exactly that and
// every intermediate is read only inside them, one launch_attention (the
// fused attention over the stored QKV rows: q scaled first, the score and
// output chains over ascending k, the same softmax sequence) writes the
// final rows.  Returns 1 when the pattern does not match (nothing decoded).
int fuse_attention(Decoder& d, const uint32_t* w) {
  const int i = d.idx;
  const int64_t B = w[4], T = w[5], H = w[7], DH = w[8];
  const uint64_t part = (uint64_t)B * H * T * DH;
  const uint32_t t5 = w[1];
  const uint32_t* e = d.peek(i + 1, PK_ELEM, 7);
  const uint32_t* t2 = d.peek(i + 2, PK_TRANSPOSE_ND, 14);
  const uint32_t* m1 = d.peek(i + 3, PK_ATTN_MM, 8);
  const uint32_t* sm = d.peek(i + 4, PK_SOFTMAX, 6);
  const uint32_t* m2 = d.peek(i + 5, PK_ATTN_MM, 8);
  const uint32_t* t3 = d.peek(i + 6, PK_TRANSPOSE_ND, 14);
  if (!e || !t2 || !m1 || !sm || !m2 || !t3) return 1;
  const uint32_t* sc = d.find(e[2], 1);
  auto perm4 = [&](const uint32_t* t, uint32_t a, uint32_t b, uint32_t c, uint32_t e4) {
    return t[2] == part && t[3] == 4 && t[4] == B && t[5] == H && t[6] == T && t[7] == DH &&
           t[9] == a && t[10] == b && t[11] == c && t[12] == e4;
  };
  const bool match =
      sc && e[0] == 7 && e[1] == t5 && e[4] == part && t2[0] == t5 + part && perm4(t2, 0, 1, 3, 2) &&
      m1[0] == e[3] && m1[1] == t2[1] && m1[3] == T && m1[4] == DH && m1[5] == T &&
      m1[6] == (uint64_t)B * H && sm[0] == m1[2] && sm[2] == (uint64_t)B * H * T && sm[3] == T &&
      sm[4] == T && m2[0] == sm[1] && m2[1] == t5 + 2 * part && m2[3] == T && m2[4] == T &&
      m2[5] == DH && m2[6] == (uint64_t)B * H && t3[0] == m2[2] && perm4(t3, 0, 2, 1, 3) &&
      d.only_readers(i, t5, 3 * part, {i + 1, i + 2, i + 5}) &&
      d.only_readers(i + 1, e[3], part, {i + 3}) && d.only_readers(i + 2, t2[1], part, {i + 3}) &&
      d.only_readers(i + 3, m1[2], (uint64_t)B * H * T * T, {i + 4}) &&
      d.only_readers(i + 4, sm[1], (uint64_t)B * H * T * T, {i + 5}) &&
      d.only_readers(i + 5, m2[2], part, {i + 6}) && B * H < (1ll << 31);
  if (!match) return 1;
  QPH_TRY(d.region(t3[1], part, false, "attention output"));
  for (int j = i + 1; j <= i + 6; j++) d.skip[(size_t)j] = 1;
  const float* qkv = d.at(w[0]);
  float* y = d.at(t3[1]);
  const float scale = f32_of(sc[0]);
  return add_launch(d.pl, i, [=](hipStream_t s) {
    return launch_attention(qkv, B, T, H, DH, scale, y, s);
  });
}

int decode_conv(Decoder& d, const qph_plan_dispatch& q) {
  const uint32_t* w;
  QPH_TRY(d.params(21, &w));
  const uint32_t in = w[0], wo = w[1], bo = w[2], out = w[3];
  const int64_t P = w[4], N = w[5], ow = w[6], iw = w[7], ih = w[8], cin = 4 * (int64_t)w[9];
  const int64_t taps = w[10], kw = w[11], sh = w[12], sw = w[13], pt = w[14], pl = w[15];
  const uint32_t ro = w[20];
  const int64_t nb = q.groups[1];
  if (nb < 1 || P < 1 || N < 4 || N % 4 || ow < 1 || P % ow || iw < 1 || ih < 1 || cin < 4 ||
      taps < 1 || kw < 1 || taps % kw || sh < 1 || sw < 1)
    return fail(QPH_EINVAL, d.where() + ": bad conv geometry");
  const int64_t oh = P / ow, kh = taps / kw;
  Act act;
  QPH_TRY(conv_act(d, w[16], f32_of(w[17]), f32_of(w[18]), f32_of(w[19]), &act));
  QPH_TRY(d.region(in, (uint64_t)nb * ih * iw * cin, true, "input"));
  QPH_TRY(d.region(wo, (uint64_t)taps * cin * N, false, "weights"));
  QPH_TRY(d.region(out, (uint64_t)nb * P * N, true, "output"));
  if (bo != OFF_NONE) QPH_TRY(d.region(bo, (uint64_t)N, true, "bias"));
  if (ro != OFF_NONE) QPH_TRY(d.region(ro, (uint64_t)nb * P * N, true, "residual"));
  const float* x = d.at(in);
  const float* wt = d.at(wo);
  const float* bias = bo == OFF_NONE ? nullptr : d.at(bo);
  const float* res = ro == OFF_NONE ? nullptr : d.at(ro);
  float* y = d.at(out);
  // the CPU branch (conv.rs:264, 506-661) and its bias rule
  const bool pointwise = taps == 1 && sh == 1 && sw == 1 && pt == 0 && pl == 0 && oh == ih &&
                         ow == iw;
  ConvK k{};
  k.arena = d.pl->arena; k.x = x; k.w = wt; k.bias = bias; k.res = res; k.y = y;
  k.P = P; k.N = N; k.ow = ow; k.oh = oh; k.iw = iw; k.ih = ih; k.cin = cin; k.taps = taps;
  k.kw = kw; k.sh = sh; k.sw = sw; k.pt = pt; k.pl = pl; k.act = act; k.tile = 1;
  if (pointwise) {
    // 1x1: one sgemm per image, M = N channels, N = P pixels (conv.rs:370-460)
    const double fl = (double)N * (double)P * (double)cin;
    k.rule_kind = 0;
    k.rule_path = (nb > 1 || fl < 2e5 || (P + 31) / 32 >= 2) ? 0 : 1;
    // nothing seeded (panel rule with N % 4 == 0): pixels x channels as one
    // GEMM over the NHWC rows, bias per column after the chain
    const bool seeded_any = bias && k.rule_path == 1 && P % 32 != 0;
    if (!seeded_any) {
      Epi e{out, act, bo, ro};
      QPH_TRY(absorb(d, (uint64_t)nb * P * N, N, true, &e));
      if (!gemm_takes_wide(nb * P, N, 1) && linear_nt_eligible(nb * P, N, cin, cin) &&
          in % 4 == 0) {
        // the session's linear kernel: the weight held transposed ([N][K],
        // k contiguous), made once here on the plan's stream
        float* wt_t = nullptr;
        if (!d.dry) {
          QPH_TRY_HIP(hipMalloc((void**)&wt_t, (size_t)N * cin * 4));
          d.pl->owned.push_back(wt_t);
          QPH_TRY(launch_transpose(wt, cin, N, wt_t, d.pl->ctx->stream));
        }
        LinArgs la{};
        la.a = x; la.lda = cin; la.wt = wt_t; la.c = d.at(e.y);
        la.m = nb * P; la.n = N; la.k = cin;
        la.bias = e.bias == OFF_NONE ? nullptr : d.at(e.bias);
        la.act = e.act;
        la.res = e.res == OFF_NONE ? nullptr : d.at(e.res);
        return add_launch(d.pl, d.idx, [la](hipStream_t s) { return launch_linear_nt(la, s); });
      }
      if ((cin == 16 || cin == 32) && nb * P * N < (1ll << 31) && nb * P * cin < (1ll << 31) &&
          e.y % 4 == 0 && (e.res == OFF_NONE || e.res % 4 == 0)) {
        PwK k{x, wt, e.bias == OFF_NONE ? nullptr : d.at(e.bias),
              e.res == OFF_NONE ? nullptr : d.at(e.res), d.at(e.y), (int)(nb * P), (int)N, e.act};
        const int64_t waves = ((N + 15) / 16) * ((nb * P + 31) / 32);
        const unsigned blocks = (unsigned)((waves + 3) / 4);
        return add_launch(d.pl, d.idx, [k, blocks, cin](hipStream_t s) {
          if (cin == 16)
            hipLaunchKernelGGL(plan_pw_kernel<4>, dim3(blocks), dim3(256), 0, s, k);
          else
            hipLaunchKernelGGL(plan_pw_kernel<8>, dim3(blocks), dim3(256), 0, s, k);
          return launch_check("plan_pw_kernel");
        });
      }
      GemmArgs g{};
      g.a = x; g.lda = cin; g.a_batch = 0;
      g.b = wt; g.ldb = N; g.b_batch = 0;
      g.c = d.at(e.y); g.ldc = N; g.c_batch = 0;
      g.m = nb * P; g.n = N; g.k = cin; g.batch = 1;
      g.bias = e.bias == OFF_NONE ? nullptr : d.at(e.bias);
      g.bias_mode = g.bias ? 2 : 0; g.seed_rule = 0;
      g.act = e.act;
      g.res = e.res == OFF_NONE ? nullptr : d.at(e.res); g.ldr = N; g.r_batch = 0;
      return add_launch(d.pl, d.idx, [g](hipStream_t s) { return launch_gemm(g, s); });
    }
  } else if (sw == 1 || sw == 2) {
    k.rule_kind = 1;  // implicit GEMM, one sgemm per output row (N = ow)
  } else {
    k.rule_kind = 2;  // im2col tiles (conv.rs:639-661), tile height on one thread
    const int64_t kk = cin * kh * kw;
    int64_t tile = ((int64_t)1 << 19) / (kk * ow > 1 ? kk * ow : 1);
    if (tile < 1) tile = 1;
    if (tile > oh) tile = oh;
    k.tile = tile;
  }
  const int64_t waves = ((N + 15) / 16) * ((P + 16 * CONV_NB - 1) / (16 * CONV_NB));
  if (waves / 4 + 1 >= (1ll << 31) || nb > 65535 || ih * iw * cin >= (1ll << 31) ||
      taps * cin * N >= (1ll << 31) || P * N >= (1ll << 31))
    return fail(QPH_EUNSUPPORTED, d.where() + ": conv grid or regions too large");
  Epi e{out, act, bo, ro};
  QPH_TRY(absorb(d, (uint64_t)nb * P * N, N, false, &e));
  k.act = e.act;
  k.res = e.res == OFF_NONE ? nullptr : d.at(e.res);
  k.y = d.at(e.y);
  const int64_t lwaves = ((N + 15) / 16) * ((P + 31) / 32);
  // 3x3 convs with up to four 16-channel output blocks: the halo kernel
  if (kh == 3 && kw == 3 && (sw == 1 || sw == 2) && sh == sw && N <= 64 && cin >= 8 &&
      9 * cin * N * 4 < (1ll << 31) && ih * iw * cin * 4 < (1ll << 31) &&
      oh * ((ow + 31) / 32) < (1ll << 31)) {
    const int tiles_x = (int)((ow + 31) / 32), ncb = (int)((N + 15) / 16);
    // what this conv (with its absorbed epilogue) reads and writes
    using Span = Decoder::Span;
    std::vector<Span> rd{{in, in + (uint64_t)nb * ih * iw * cin}, {wo, wo + (uint64_t)taps * cin * N}};
    if (e.bias != OFF_NONE) rd.push_back({e.bias, e.bias + (uint64_t)N});
    if (e.res != OFF_NONE) rd.push_back({e.res, e.res + (uint64_t)nb * P * N});
    const Span wr{e.y, e.y + (uint64_t)nb * P * N};
    if (join_halo_group(d, k, tiles_x, oh, (int)sw, ncb, nb, rd, wr)) return QPH_OK;
    auto g = std::make_shared<HaloGroup>();
    g->k[0] = k;
    g->tiles_x[0] = tiles_x;
    d.halo = Decoder::HaloOpen{};
    d.halo.g = g;
    d.halo.n = 1;
    d.halo.sw = (int)sw;
    d.halo.ncb = ncb;
    d.halo.nb = nb;
    d.halo.last = d.idx;
    d.halo.reads = rd;
    d.halo.writes = {wr};
    g->start[0] = 0;
    for (int i = 1; i <= HALO_GROUP_MAX; i++) g->start[i] = (int)((oh + 1) / 2 * tiles_x);
    const unsigned nbu = (unsigned)nb;
#define QPH_HALO(S, C)                                                                      \
  if (sw == S && ncb == C)                                                                  \
    return add_launch(d.pl, d.idx, [g, nbu](hipStream_t s) {                                \
      const dim3 grid((unsigned)g->start[HALO_GROUP_MAX], nbu);                             \
      const size_t lds = HaloGeom<S, C>::lds();                                             \
      if (g->start[1] == g->start[HALO_GROUP_MAX])                                          \
        hipLaunchKernelGGL((plan_conv_halo_kernel<S, C>), grid, dim3(128 * C), lds, s,      \
                           g->k[0], g->tiles_x[0]);                                         \
      else                                                                                  \
        hipLaunchKernelGGL((plan_conv_halo_group_kernel<S, C>), grid, dim3(128 * C), lds, s,\
                           *g);                                                             \
      return launch_check("plan_conv_halo_kernel");                                         \
    });
    QPH_HALO(1, 1) QPH_HALO(1, 2) QPH_HALO(1, 3) QPH_HALO(1, 4)
    QPH_HALO(2, 1) QPH_HALO(2, 2) QPH_HALO(2, 3) QPH_HALO(2, 4)
#undef QPH_HALO
  }
  // the ring pays off from two channel groups on (a 3-channel stem has one)
  if ((taps == 1 || taps == 4 || taps == 9) && cin >= 8 && taps * cin * N * 4 < (1ll << 31) &&
      ih * iw * cin * 4 < (1ll << 31) && lwaves < (1ll << 31)) {
    auto go = [k, lwaves, nb](auto fn, size_t lds, hipStream_t s) {
      hipLaunchKernelGGL(fn, dim3((unsigned)lwaves, (unsigned)nb), dim3(64), lds, s, k);
      return launch_check("plan_conv_dma_kernel");
    };
    if (taps == 1)
      return add_launch(d.pl, d.idx, [go](hipStream_t s) {
        return go(plan_conv_dma_kernel<1>, CONV_DMA_D * DmaGeom<1>::BUF * 16, s);
      });
    if (taps == 4)
      return add_launch(d.pl, d.idx, [go](hipStream_t s) {
        return go(plan_conv_dma_kernel<4>, CONV_DMA_D * DmaGeom<4>::BUF * 16, s);
      });
    return add_launch(d.pl, d.idx, [go](hipStream_t s) {
      return go(plan_conv_dma_kernel<9>, CONV_DMA_D * DmaGeom<9>::BUF * 16, s);
    });
  }
  if (kh == 3 && kw == 3 && cin == 4 && sh == sw && (sw == 1 || sw == 2) && ih * iw < (1ll << 31)) {
    const int64_t w2 = ((N + 31) / 32) * ((P + 31) / 32), w1 = ((N + 15) / 16) * ((P + 31) / 32);
    return add_launch(d.pl, d.idx, [k, nb, sw, w1, w2](hipStream_t s) {
      const bool two = k.N > 16;   // both 16-channel blocks in one wave
      const dim3 grid((unsigned)(((two ? w2 : w1) + 3) / 4), (unsigned)nb);
      if (sw == 1 && two) hipLaunchKernelGGL((plan_stem_kernel<1, 2>), grid, dim3(256), 0, s, k);
      else if (sw == 1) hipLaunchKernelGGL((plan_stem_kernel<1, 1>), grid, dim3(256), 0, s, k);
      else if (two) hipLaunchKernelGGL((plan_stem_kernel<2, 2>), grid, dim3(256), 0, s, k);
      else hipLaunchKernelGGL((plan_stem_kernel<2, 1>), grid, dim3(256), 0, s, k);
      return launch_check("plan_stem_kernel");
    });
  }
  if (taps <= CONV_LDS_TAPS) {
    const size_t lds = (size_t)4 * taps * 32 * 16;
    return add_launch(d.pl, d.idx, [k, lwaves, nb, lds](hipStream_t s) {
      hipLaunchKernelGGL(plan_conv_lds_kernel, dim3((unsigned)((lwaves + 3) / 4), (unsigned)nb),
                         dim3(256), lds, s, k);
      return launch_check("plan_conv_lds_kernel");
    });
  }
  return add_launch(d.pl, d.idx, [k, waves, nb](hipStream_t s) {
    hipLaunchKernelGGL(plan_conv_kernel, dim3((unsigned)((waves + 3) / 4), (unsigned)nb),
                       dim3(256), 0, s, k);
    return launch_check("plan_conv_kernel");
  });
}

// The nine dispatches PlanBuilder writes for a LayerNorm over contiguous
// rows, starting at an n_reduce_last (w: its block): mean M = mean(X);
// D = X - M (n_elem 8); SQ = D * D (n_elem 9); V = mean(SQ); VE = V + eps
// (n_elem 6, eps a static word); S = sqrt(VE) (n_elem 10); Y0 = D / S
// (n_elem 11); Y1 = Y0 * gamma (n_channel 0); Y = Y1 + beta (n_channel 1).
// That is layernorm_kernel's operation sequence (the f64 means the
// reference's, each step rounded to f32 in the same order), so when every
// intermediate is read only inside the run and is no graph output, the run
// is one layernorm launch: *folded, the eight dispatches after it skipped.
int fold_layernorm(Decoder& d, const uint32_t* w, bool* folded) {
  *folded = false;
  const uint32_t X = w[0], M = w[1];
  const uint32_t R = w[2], C = w[3];
  if (w[4] != C || C < 4 || C % 4 || C > 4096 || R < 1) return QPH_OK;
  const uint64_t n = (uint64_t)R * C;
  const int i = d.idx;
  const uint32_t* e8 = d.peek(i + 1, PK_ELEM, 7);
  const uint32_t* e9 = d.peek(i + 2, PK_ELEM, 7);
  const uint32_t* r2 = d.peek(i + 3, PK_REDUCE_LAST, 6);
  const uint32_t* e6 = d.peek(i + 4, PK_ELEM, 7);
  const uint32_t* e10 = d.peek(i + 5, PK_ELEM, 7);
  const uint32_t* e11 = d.peek(i + 6, PK_ELEM, 7);
  const uint32_t* c0 = d.peek(i + 7, PK_CHANNEL, 10);
  const uint32_t* c1 = d.peek(i + 8, PK_CHANNEL, 10);
  if (!e8 || !e9 || !r2 || !e6 || !e10 || !e11 || !c0 || !c1) return QPH_OK;
  const uint32_t D = e8[3], SQ = e9[3], V = r2[1], VE = e6[3], S = e10[3], Y0 = e11[3];
  const uint32_t Y1 = c0[4], Y = c1[4], G = c0[2], B = c1[2];
  const bool shape =
      e8[0] == 8 && e8[1] == X && e8[2] == M && e8[4] == n && e8[5] == C / 4 &&
      e9[0] == 9 && e9[1] == D && e9[4] == n &&
      r2[0] == SQ && r2[2] == R && r2[3] == C && r2[4] == C &&
      e6[0] == 6 && e6[1] == V && e6[4] == 4 * R &&
      e10[0] == 10 && e10[1] == VE && e10[4] == 4 * R &&
      e11[0] == 11 && e11[1] == D && e11[2] == S && e11[4] == n && e11[5] == C / 4 &&
      c0[0] == 0 && c0[1] == Y0 && c0[3] == OFF_NONE && c0[5] == n && c0[6] == C && c0[9] == R &&
      c1[0] == 1 && c1[1] == Y1 && c1[3] == OFF_NONE && c1[5] == n && c1[6] == C && c1[9] == R;
  if (!shape) return QPH_OK;
  const uint32_t* eps_w = d.find(e6[2], 1);
  if (!eps_w) return QPH_OK;   // eps not a static word: the dispatches one by one
  // intermediates read only inside the run (and no graph output)
  if (!d.only_readers(i, M, 4ull * R, {i + 1}) || !d.only_readers(i + 1, D, n, {i + 2, i + 6}) ||
      !d.only_readers(i + 2, SQ, n, {i + 3}) || !d.only_readers(i + 3, V, 4ull * R, {i + 4}) ||
      !d.only_readers(i + 4, VE, 4ull * R, {i + 5}) || !d.only_readers(i + 5, S, 4ull * R, {i + 6}) ||
      !d.only_readers(i + 6, Y0, n, {i + 7}) || !d.only_readers(i + 7, Y1, n, {i + 8}))
    return QPH_OK;
  QPH_TRY(d.region(X, n, true, "LayerNorm input"));
  QPH_TRY(d.region(Y, n, true, "LayerNorm output"));
  QPH_TRY(d.region(G, C, true, "LayerNorm gamma"));
  QPH_TRY(d.region(B, C, true, "LayerNorm beta"));
  float eps;
  std::memcpy(&eps, eps_w, 4);
  const float* x = d.at(X);
  const float* g = d.at(G);
  const float* b = d.at(B);
  float* y = d.at(Y);
  for (int j = i + 1; j <= i + 8; j++) d.skip[(size_t)j] = 1;
  *folded = true;
  return add_launch(d.pl, d.idx, [=](hipStream_t s) {
    return launch_layernorm(x, g, b, eps, R, C, y, s);
  });
}

int decode(Decoder& d, const qph_plan_dispatch& q, std::vector<PendingHw>& pending) {
  qph_plan* pl = d.pl;
  const uint32_t* w = nullptr;
  switch (q.kernel) {
    case PK_ENTRY: {
      QPH_TRY(d.params(7, &w));
      const int64_t nb = w[2], c = w[3], h = w[4], wd = w[5], cp = w[6];
      if (nb < 1 || c < 1 || h < 1 || wd < 1 || cp < c || cp % 4)
        return fail(QPH_EINVAL, d.where() + ": bad entry shape");
      QPH_TRY(d.region(w[0], (uint64_t)nb * c * h * wd, false, "input"));
      QPH_TRY(d.region(w[1], (uint64_t)nb * h * wd * cp, true, "output"));
      EntryK k{pl->arena, d.at(w[0]), d.at(w[1]), nb, c, h * wd, cp / 4};
      return add_launch(pl, d.idx, [k](hipStream_t s) {
        hipLaunchKernelGGL(plan_entry_kernel, dim3(blocks_for(k.nb * k.hw)), dim3(256), 0, s, k);
        return launch_check("plan_entry_kernel");
      });
    }
    case PK_EXIT: {
      QPH_TRY(d.params(8, &w));
      const int64_t nb = w[2], c = w[3], h = w[4], wd = w[5], cp = w[6];
      if (nb < 1 || c < 1 || h < 1 || wd < 1 || cp < c || cp % 4 || (w[7] != 0 && w[7] != 4))
        return fail(QPH_EINVAL, d.where() + ": bad exit shape or activation");
      QPH_TRY(d.region(w[0], (uint64_t)nb * h * wd * cp, true, "input"));
      QPH_TRY(d.region(w[1], (uint64_t)nb * c * h * wd, false, "output"));
      ExitK k{d.at(w[0]), d.at(w[1]), nb, c, h * wd, cp, w[7] == 4};
      return add_launch(pl, d.idx, [k](hipStream_t s) {
        hipLaunchKernelGGL(plan_exit_kernel, dim3(blocks_for(k.nb * k.hw)), dim3(256), 0, s, k);
        return launch_check("plan_exit_kernel");
      });
    }
    case PK_EXIT3:
    case PK_EXIT3_ARGMAX: {
      QPH_TRY(d.params(6, &w));
      const int64_t rows = w[2], cols = w[3], cp = w[4], rpb = w[5];
      if (rows < 1 || cols < 1 || cp < cols || rpb < 1)
        return fail(QPH_EINVAL, d.where() + ": bad rows / cols");
      QPH_TRY(d.region(w[0], (uint64_t)rows * cp, false, "input"));
      const float* x = d.at(w[0]);
      float* y = d.at(w[1]);
      if (q.kernel == PK_EXIT3_ARGMAX) {
        QPH_TRY(d.region(w[1], (uint64_t)rows * 2, false, "pairs"));
        if (cols >= (1ll << 31)) return fail(QPH_EUNSUPPORTED, d.where() + ": row too wide");
        return add_launch(pl, d.idx, [=](hipStream_t s) {
          return launch_argmax_pitched(x, rows, cols, cp, y, s);
        });
      }
      QPH_TRY(d.region(w[1], (uint64_t)rows * cols, false, "output"));
      Exit3K k{pl->arena, x, y, rows, cols, cp, rpb};
      return add_launch(pl, d.idx, [k](hipStream_t s) {
        hipLaunchKernelGGL(plan_exit3_kernel, dim3(blocks_for(k.rows * k.cols)), dim3(256), 0, s, k);
        return launch_check("plan_exit3_kernel");
      });
    }
    case PK_ELEM: {
      QPH_TRY(d.params(7, &w));
      const int op = (int)w[0];
      const int64_t n = w[4];
      if (op < 0 || op > 13) return fail(QPH_EUNSUPPORTED, d.where() + ": op " + std::to_string(op));
      if (n < 4 || n % 4) return fail(QPH_EINVAL, d.where() + ": element count not a multiple of 4");
      QPH_TRY(d.region(w[1], (uint64_t)n, true, "input"));
      QPH_TRY(d.region(w[3], (uint64_t)n, true, "output"));
      ElemK k{d.at(w[1]), nullptr, d.at(w[3]), n / 4, op, f32_of(w[5]), f32_of(w[6]), 1};
      if (op == 4 || op == 5 || op == 12 || op == 13) {
        QPH_TRY(d.region(w[2], (uint64_t)n, true, "second input"));
        k.b = d.at(w[2]);
      } else if (op == 6 || op == 7) {
        QPH_TRY(d.region(w[2], 1, false, "scalar"));
        k.b = d.at(w[2]);
      } else if (op == 8 || op == 11) {
        k.c4 = w[5];  // the row's vec4 count, as the bits of p1
        if (k.c4 < 1 || (n / 4) % k.c4)
          return fail(QPH_EINVAL, d.where() + ": row vector width does not divide the tensor");
        QPH_TRY(d.region(w[2], (uint64_t)(n / 4 / k.c4) * 4, true, "row values"));
        k.b = d.at(w[2]);
      }
      return add_launch(pl, d.idx, [k](hipStream_t s) {
        hipLaunchKernelGGL(plan_elem_kernel, dim3(blocks_for(k.nv)), dim3(256), 0, s, k);
        return launch_check("plan_elem_kernel");
      });
    }
    case PK_CHANNEL: {
      QPH_TRY(d.params(10, &w));
      const int op = (int)w[0];
      const int64_t n = w[5], cp = w[6], hw = w[9];
      if (op < 0 || op > 5) return fail(QPH_EUNSUPPORTED, d.where() + ": op " + std::to_string(op));
      if (n < 4 || n % 4 || cp < 4 || cp % 4 || (n / 4) % (cp / 4) || hw < 1)
        return fail(QPH_EINVAL, d.where() + ": bad channel broadcast shape");
      const int64_t frows = n / cp, grows = (frows - 1) / hw + 1;
      QPH_TRY(d.region(w[1], (uint64_t)n, true, "input"));
      QPH_TRY(d.region(w[2], (uint64_t)grows * cp, true, "gate"));
      QPH_TRY(d.region(w[4], (uint64_t)n, true, "output"));
      ChannelK k{pl->arena, d.at(w[1]), d.at(w[2]), nullptr, d.at(w[4]), n / 4, cp / 4, hw, op,
                 f32_of(w[7]), f32_of(w[8])};
      if (op == 2) {
        QPH_TRY(d.region(w[3], (uint64_t)n, true, "residual"));
        k.r = d.at(w[3]);
      } else if (op == 5) {
        QPH_TRY(d.region(w[3], (uint64_t)grows * cp, true, "shift"));
        k.r = d.at(w[3]);
      }
      return add_launch(pl, d.idx, [k](hipStream_t s) {
        hipLaunchKernelGGL(plan_channel_kernel, dim3(blocks_for(k.nv)), dim3(256), 0, s, k);
        return launch_check("plan_channel_kernel");
      });
    }
    case PK_CONV:
    case PK_CONV8:
      return decode_conv(d, q);
    case PK_CONV_DW: {
      QPH_TRY(d.params(20, &w));
      const int64_t P = w[4], C = w[5], ow = w[6], iw = w[7], ih = w[8], taps = w[9], kw = w[10];
      const int64_t sh = w[11], sw = w[12], pt = w[13], pl_ = w[14];
      const int64_t nb = q.groups[1];
      if (nb < 1 || nb > 65535 || P < 1 || C < 4 || C % 4 || ow < 1 || P % ow || iw < 1 ||
          ih < 1 || taps < 1 || kw < 1 || taps % kw || sh < 1 || sw < 1)
        return fail(QPH_EINVAL, d.where() + ": bad depthwise geometry");
      Act act;
      QPH_TRY(conv_act(d, w[15], f32_of(w[16]), f32_of(w[17]), f32_of(w[18]), &act));
      QPH_TRY(d.region(w[0], (uint64_t)nb * ih * iw * C, true, "input"));
      QPH_TRY(d.region(w[1], (uint64_t)taps * C, true, "weights"));
      QPH_TRY(d.region(w[3], (uint64_t)nb * P * C, true, "output"));
      if (w[2] != OFF_NONE) QPH_TRY(d.region(w[2], (uint64_t)C, true, "bias"));
      if (w[19] != OFF_NONE) QPH_TRY(d.region(w[19], (uint64_t)nb * P * C, true, "residual"));
      Epi e{w[3], act, OFF_NONE, w[19]};
      QPH_TRY(absorb(d, (uint64_t)nb * P * C, C, false, &e));
      DwK k{pl->arena, d.at(w[0]), d.at(w[1]), w[2] == OFF_NONE ? nullptr : d.at(w[2]),
            e.res == OFF_NONE ? nullptr : d.at(e.res), d.at(e.y),
            P, C / 4, ow, iw, ih, taps, kw, sh, sw, pt, pl_, e.act};
      const int64_t kh = taps / kw;
      if (((kh == 3 && kw == 3) || (kh == 5 && kw == 5)) && (sw == 1 || sw == 2)) {
        const int64_t threads = (P / ow) * ((ow + 3) / 4) * (C / 4);
        return add_launch(pl, d.idx, [k, nb, threads, kh, sw](hipStream_t s) {
          const dim3 grid(blocks_for(threads), (unsigned)nb);
          if (kh == 3 && sw == 1) hipLaunchKernelGGL((plan_dw_px_kernel<3, 3, 1>), grid, dim3(256), 0, s, k);
          else if (kh == 3) hipLaunchKernelGGL((plan_dw_px_kernel<3, 3, 2>), grid, dim3(256), 0, s, k);
          else if (sw == 1) hipLaunchKernelGGL((plan_dw_px_kernel<5, 5, 1>), grid, dim3(256), 0, s, k);
          else hipLaunchKernelGGL((plan_dw_px_kernel<5, 5, 2>), grid, dim3(256), 0, s, k);
          return launch_check("plan_dw_px_kernel");
        });
      }
      return add_launch(pl, d.idx, [k, nb](hipStream_t s) {
        hipLaunchKernelGGL(plan_dw_kernel, dim3(blocks_for(k.P * k.c4), (unsigned)nb), dim3(256), 0,
                           s, k);
        return launch_check("plan_dw_kernel");
      });
    }
    case PK_CONVT: {
      QPH_TRY(d.params(18, &w));
      const int64_t P = w[4], N = w[5], ow = w[6], iw = w[7], ih = w[8], cin = w[9];
      const int64_t sh = w[11], sw = w[12], kw = w[13];
      const int64_t nb = q.groups[1];
      if (nb < 1 || nb > 65535 || P < 1 || N < 4 || N % 4 || ow < 1 || P % ow || iw < 1 ||
          ih < 1 || cin < 4 || cin % 4 || (int64_t)w[10] * 4 != cin || sh < 1 || sw < 1 ||
          kw < 1 || kw > sw || P / ow > ih * sh || ow > iw * sw)
        return fail(QPH_EINVAL, d.where() + ": bad conv-transpose geometry");
      Act act;
      QPH_TRY(conv_act(d, w[14], f32_of(w[15]), f32_of(w[16]), f32_of(w[17]), &act));
      const int64_t max_tap = (sh - 1) * kw + (sw - 1);
      QPH_TRY(d.region(w[0], (uint64_t)nb * ih * iw * cin, false, "input"));
      QPH_TRY(d.region(w[1], (uint64_t)(max_tap + 1) * cin * N, true, "weights"));
      QPH_TRY(d.region(w[3], (uint64_t)nb * P * N, true, "output"));
      if (w[2] != OFF_NONE) QPH_TRY(d.region(w[2], (uint64_t)N, true, "bias"));
      ConvtK k{d.at(w[0]), d.at(w[1]), w[2] == OFF_NONE ? nullptr : d.at(w[2]), d.at(w[3]),
               P, N / 4, ow, iw, ih, cin, sh, sw, kw, act};
      // a second 2x2 stride-2 conv-transpose and an n_exit after it, each
      // the only reader of what it reads: one pass (plan_convt_pair_kernel)
      const uint32_t* w2 = d.peek(d.idx + 1, PK_CONVT, 18);
      const uint32_t* ex = d.peek(d.idx + 2, PK_EXIT, 8);
      const bool twice = sh == 2 && sw == 2 && kw == 2 && P == 4 * ih * iw && ow == 2 * iw;
      if (twice && cin == 24 && N == 24 && w2 && ex && w2[0] == w[3] && w2[9] == (uint32_t)N &&
          w2[11] == 2 && w2[12] == 2 && w2[13] == 2 && w2[8] == (uint32_t)(2 * ih) &&
          w2[7] == (uint32_t)ow && w2[4] == 16ull * ih * iw && w2[6] == 4ull * iw && w2[5] == 4 &&
          d.disp[d.idx + 1].groups[1] == (uint32_t)nb && ex[0] == w2[3] && ex[2] == (uint32_t)nb &&
          ex[4] == 4ull * ih && ex[5] == 4ull * iw && ex[6] == 4 && ex[3] >= 1 && ex[3] <= 4 &&
          nb * 16 * ih * iw < (1ll << 31) && (w[0] % 4) == 0 &&
          d.only_readers(d.idx, w[3], (uint64_t)nb * P * N, {d.idx + 1}) &&
          d.only_readers(d.idx + 1, w2[3], (uint64_t)nb * w2[4] * 4, {d.idx + 2})) {
        Act act2;
        QPH_TRY(conv_act(d, w2[14], f32_of(w2[15]), f32_of(w2[16]), f32_of(w2[17]), &act2));
        QPH_TRY(d.region(w2[1], 4ull * N * 4, true, "second weights"));
        if (w2[2] != OFF_NONE) QPH_TRY(d.region(w2[2], 4, true, "second bias"));
        QPH_TRY(d.region(ex[1], (uint64_t)nb * ex[3] * 16 * ih * iw, false, "output"));
        d.skip[(size_t)d.idx + 1] = 1;
        d.skip[(size_t)d.idx + 2] = 1;
        ConvtPairK f{pl->arena, d.at(w[0]), d.at(w[1]), k.bias, d.at(w2[1]),
                     w2[2] == OFF_NONE ? nullptr : d.at(w2[2]), d.at(ex[1]), (int)ih, (int)iw, 4,
                     (int)ex[3], act, act2, ex[7] == 4};
        return add_launch(pl, d.idx, [f, nb](hipStream_t s) {
          const dim3 grid((unsigned)((f.h * f.w + 255) / 256), 4, (unsigned)nb);
          hipLaunchKernelGGL((plan_convt_pair_kernel<24, 24>), grid, dim3(256), 0, s, f);
          return launch_check("plan_convt_pair_kernel");
        });
      }
      return add_launch(pl, d.idx, [k, nb](hipStream_t s) {
        hipLaunchKernelGGL(plan_convt_kernel, dim3(blocks_for(k.P * k.nv), (unsigned)nb), dim3(256),
                           0, s, k);
        return launch_check("plan_convt_kernel");
      });
    }
    case PK_POOL: {
      QPH_TRY(d.params(14, &w));
      const int64_t P = w[2], C = w[3], ow = w[4], iw = w[5], ih = w[6], kh = w[7], kw = w[8];
      const int64_t sh = w[9], sw = w[10], pt = w[11], pl_ = w[12];
      const int64_t nb = q.groups[1];
      if (nb < 1 || nb > 65535 || P < 1 || C < 4 || C % 4 || ow < 1 || P % ow || iw < 1 ||
          ih < 1 || kh < 1 || kw < 1 || sh < 1 || sw < 1)
        return fail(QPH_EINVAL, d.where() + ": bad pool geometry");
      QPH_TRY(d.region(w[0], (uint64_t)nb * ih * iw * C, true, "input"));
      QPH_TRY(d.region(w[1], (uint64_t)nb * P * C, true, "output"));
      PoolNK k{pl->arena, d.at(w[0]), d.at(w[1]), P, C / 4, ow, iw, ih, kh, kw, sh, sw, pt, pl_,
               w[13] != 0, 0};
      k.special = k.max_pool && kh == 2 && kw == 2 && sh == 1 && sw == 1 && pt == 0 && pl_ == 0 &&
                  P / ow == ih && ow == iw;
      return add_launch(pl, d.idx, [k, nb](hipStream_t s) {
        hipLaunchKernelGGL(plan_pool_kernel, dim3(blocks_for(k.P * k.c4), (unsigned)nb), dim3(256),
                           0, s, k);
        return launch_check("plan_pool_kernel");
      });
    }
    case PK_REDUCE_HW: {
      QPH_TRY(d.params(4, &w));
      const int64_t m = w[2], c = w[3], nb = q.groups[1];
      if (nb < 1 || m < 1 || c < 4 || c % 4) return fail(QPH_EINVAL, d.where() + ": bad reduce shape");
      QPH_TRY(d.region(w[0], (uint64_t)nb * m * c, true, "input"));
      pending.push_back({w[0], w[1], m, c, nb});
      return QPH_OK;  // runs with its n_reduce_fin
    }
    case PK_REDUCE_FIN: {
      QPH_TRY(d.params(5, &w));
      const uint32_t scratch = w[0], out = w[1];
      const int64_t c = w[3], m = w[4], nb = q.groups[0];
      auto it = std::find_if(pending.begin(), pending.end(),
                             [&](const PendingHw& h) { return h.scratch == scratch; });
      if (it == pending.end() || it->c != c || it->m != m || it->nb != nb)
        return fail(QPH_EUNSUPPORTED, d.where() + ": no matching n_reduce_hw before it");
      QPH_TRY(d.region(out, (uint64_t)nb * c, true, "output"));
      const float* x = d.at(it->in);
      float* y = d.at(out);
      pending.erase(it);
      // GlobalAveragePool: channel c of image b is the mean over the P
      // pixels x[(b * P + p) * C + c]
      const unsigned* rn = (const unsigned*)d.at(0);
      return add_launch(pl, d.idx, [=](hipStream_t s) {
        return launch_reduce_mean_rows(x, nb * c, m, c, m * c, 1, c, y, 1, s, rn, c);
      });
    }
    case PK_REDUCE_LAST: {
      QPH_TRY(d.params(6, &w));
      const int64_t rows = w[2], cols = w[3], cp = w[4];
      if (rows < 1 || cols < 1 || cp < cols) return fail(QPH_EINVAL, d.where() + ": bad rows / cols");
      bool folded = false;
      QPH_TRY(fold_layernorm(d, w, &folded));
      if (folded) return QPH_OK;
      QPH_TRY(d.region(w[0], (uint64_t)rows * cp, false, "input"));
      QPH_TRY(d.region(w[1], (uint64_t)rows * 4, false, "output"));
      const float* x = d.at(w[0]);
      float* y = d.at(w[1]);
      const unsigned* rn = (const unsigned*)d.at(0);
      const int64_t rpb = w[5];
      return add_launch(pl, d.idx, [=](hipStream_t s) {
        return launch_reduce_mean_rows(x, rows, cols, rows, 0, cp, 1, y, 4, s, rn, rpb);
      });
    }
    case PK_RESIZE: {
      QPH_TRY(d.params(9, &w));
      const int64_t P = w[2], C = w[3], ow = w[4], iw = w[5], ih = w[6], nb = q.groups[1];
      if (nb < 1 || nb > 65535 || P < 1 || C < 4 || C % 4 || ow < 1 || P % ow || iw < 1 || ih < 1)
        return fail(QPH_EINVAL, d.where() + ": bad resize geometry");
      QPH_TRY(d.region(w[0], (uint64_t)nb * ih * iw * C, true, "input"));
      QPH_TRY(d.region(w[1], (uint64_t)nb * P * C, true, "output"));
      const uint32_t S = w[0], R = w[1];
      const uint64_t len = (uint64_t)nb * P * C, slen = (uint64_t)nb * ih * iw * C;
      const bool small = len < (1ull << 31) && slen < (1ull << 31);
      auto hits = [](uint32_t o, uint32_t lo, uint64_t n) { return o >= lo && (uint64_t)o < lo + n; };
      // (a) the next dispatch adds the resized map to another tensor of its
      // size, and is its only reader: one pass (the FPN's top-down adds)
      const uint32_t* e = d.peek(d.idx + 1, PK_ELEM, 7);
      if (small && e && e[0] == 4 && e[4] == len && ((e[1] == R) != (e[2] == R)) &&
          d.only_readers(d.idx, R, len, {d.idx + 1}) && !hits(e[3], S, slen) &&
          !hits(S, e[3], len)) {
        const uint32_t Y = e[1] == R ? e[2] : e[1];
        QPH_TRY(d.region(Y, len, true, "addend"));
        QPH_TRY(d.region(e[3], len, true, "sum"));
        d.skip[(size_t)d.idx + 1] = 1;
        ResizeAddK k{pl->arena, (const float4*)d.at(S), (const float4*)d.at(Y), (float4*)d.at(e[3]), (int)P,
                     (int)(C / 4), (int)ow, (int)(P / ow), (int)iw, (int)ih};
        return add_launch(pl, d.idx, [k, nb](hipStream_t s) {
          hipLaunchKernelGGL(plan_resize_add_kernel, dim3(blocks_for((int64_t)k.P * k.c4), (unsigned)nb),
                             dim3(256), 0, s, k);
          return launch_check("plan_resize_add_kernel");
        });
      }
      // (b) a later n_concat_c is the only reader of the resized map, and
      // nothing writes the source or the map before it: the concat reads the
      // source through the same mapping (the det neck's upsampled maps)
      for (int j = d.idx + 1; small && j < d.n_disp && j <= d.idx + 16; j++) {
        if (d.wr[(size_t)j] != OFF_NONE && (hits(d.wr[(size_t)j], S, slen) || hits(d.wr[(size_t)j], R, len)))
          break;
        if (d.disp[j].kernel != PK_CONCAT_C || d.skip[(size_t)j]) continue;
        const uint32_t* c = d.find(d.disp[j].p_off, 4);
        if (!c || c[2] < 1 || c[2] > 8 || c[1] != (uint64_t)nb * P) break;
        const uint32_t* cw = d.find(d.disp[j].p_off, 4 + 2 * c[2]);
        bool reads = false;
        for (uint32_t i = 0; cw && i < c[2]; i++) reads = reads || (cw[4 + 2 * i] == R && cw[5 + 2 * i] == C / 4);
        if (reads && d.only_readers(d.idx, R, len, {j})) {
          d.resized.push_back({R, S, nb, ih, iw, P / ow, ow, C / 4});
          d.skip[(size_t)d.idx] = 1;
          return QPH_OK;
        }
        break;
      }
      ResizeNK k{d.at(w[0]), d.at(w[1]), P, C / 4, ow, P / ow, iw, ih};
      return add_launch(pl, d.idx, [k, nb](hipStream_t s) {
        hipLaunchKernelGGL(plan_resize_kernel, dim3(blocks_for(k.P * k.c4), (unsigned)nb),
                           dim3(256), 0, s, k);
        return launch_check("plan_resize_kernel");
      });
    }
    case PK_TRANSPOSE: {
      QPH_TRY(d.params(4, &w));
      const int64_t r = w[2], c = w[3];
      if (r < 1 || c < 1) return fail(QPH_EINVAL, d.where() + ": empty transpose");
      QPH_TRY(d.region(w[0], (uint64_t)r * c, false, "input"));
      QPH_TRY(d.region(w[1], (uint64_t)r * c, false, "output"));
      Transpose2K k{d.at(w[0]), d.at(w[1]), r, c};
      return add_launch(pl, d.idx, [k](hipStream_t s) {
        hipLaunchKernelGGL(plan_transpose2_kernel, dim3(blocks_for(k.r * k.c)), dim3(256), 0, s, k);
        return launch_check("plan_transpose2_kernel");
      });
    }
    case PK_TRANSPOSE_ND: {
      QPH_TRY(d.params(14, &w));
      TransposeNK k{};
      k.total = w[2];
      k.rank = (int)w[3];
      if (k.rank < 1 || k.rank > 5) return fail(QPH_EINVAL, d.where() + ": rank outside 1..5");
      int64_t prod = 1;
      bool seen[5] = {false, false, false, false, false};
      for (int i = 0; i < k.rank; i++) {
        k.dims[i] = w[4 + i];
        k.perm[i] = (int)w[9 + i];
        if (k.dims[i] < 1 || k.perm[i] < 0 || k.perm[i] >= k.rank || seen[k.perm[i]])
          return fail(QPH_EINVAL, d.where() + ": bad dims / permutation");
        seen[k.perm[i]] = true;
        prod *= k.dims[i];
      }
      if (prod != k.total || k.total < 1) return fail(QPH_EINVAL, d.where() + ": total != product");
      QPH_TRY(d.region(w[0], (uint64_t)k.total, false, "input"));
      QPH_TRY(d.region(w[1], (uint64_t)k.total, false, "output"));
      k.x = d.at(w[0]);
      k.y = d.at(w[1]);
      if (k.rank == 5 && k.perm[0] == 2 && k.perm[1] == 0 && k.perm[2] == 3 && k.perm[3] == 1 &&
          k.perm[4] == 4 && k.dims[2] == 3) {
        int rc = fuse_attention(d, w);
        if (rc != 1) return rc;   // 1: not the attention pattern
      }
      if (k.total < (1ll << 31)) {
        const int r = k.rank;
        const bool v4 = k.perm[r - 1] == r - 1 && k.dims[r - 1] % 4 == 0 && w[0] % 4 == 0 &&
                        w[1] % 4 == 0;
        const int V = v4 ? 4 : 1;
        TransposeFastK f{};
        f.x = k.x; f.y = k.y; f.rank = r; f.units = (unsigned)(k.total / V);
        int64_t stride[5];
        stride[r - 1] = 1;
        for (int i = r - 2; i >= 0; i--) stride[i] = stride[i + 1] * k.dims[i + 1];
        for (int i = 0; i < r; i++) {
          f.od[i] = (unsigned)(k.dims[k.perm[i]] / (i == r - 1 ? V : 1));
          f.is[i] = (unsigned)(stride[k.perm[i]] / (k.perm[i] == r - 1 ? 1 : V));
        }
        return add_launch(pl, d.idx, [f, v4](hipStream_t s) {
          const dim3 grid((f.units + 255) / 256);
          if (v4)
            hipLaunchKernelGGL(plan_transpose_fast_kernel<4>, grid, dim3(256), 0, s, f);
          else
            hipLaunchKernelGGL(plan_transpose_fast_kernel<1>, grid, dim3(256), 0, s, f);
          return launch_check("plan_transpose_fast_kernel");
        });
      }
      return add_launch(pl, d.idx, [k](hipStream_t s) {
        hipLaunchKernelGGL(plan_transpose_nd_kernel, dim3(blocks_for(k.total)), dim3(256), 0, s, k);
        return launch_check("plan_transpose_nd_kernel");
      });
    }
    case PK_CONCAT_C: {
      QPH_TRY(d.params(4, &w));
      const int64_t hw = w[1], n = w[2], outc4 = w[3];
      if (hw < 1 || n < 1 || n > 8 || outc4 < 1)
        return fail(QPH_EINVAL, d.where() + ": bad concat (1 to 8 inputs)");
      QPH_TRY(d.params(4 + 2 * (uint32_t)n, &w));
      ConcatK k{};
      k.arena = pl->arena; k.hw = hw; k.outc4 = outc4; k.n = (int)n;
      int64_t sum = 0;
      for (int i = 0; i < n; i++) {
        k.src[i] = w[4 + 2 * i];
        k.c4len[i] = w[5 + 2 * i];
        if (k.c4len[i] < 1) return fail(QPH_EINVAL, d.where() + ": empty concat input");
        QPH_TRY(d.region(k.src[i], (uint64_t)hw * k.c4len[i] * 4, true, "concat input"));
        sum += k.c4len[i];
      }
      if (sum != outc4) return fail(QPH_EINVAL, d.where() + ": input channels do not sum to the output's");
      QPH_TRY(d.region(w[0], (uint64_t)hw * outc4 * 4, true, "output"));
      k.y = d.at(w[0]);
      // inputs that are n_resize outputs read through (see PK_RESIZE)
      ConcatUpK u{};
      bool up = false;
      u.y = (float4*)k.y; u.npx = (int)hw; u.outc4 = (int)outc4; u.n = (int)n;
      for (int i = 0; i < n; i++) {
        u.src[i] = (const float4*)d.at(k.src[i]);
        u.c4len[i] = (int)k.c4len[i];
        for (const auto& r : d.resized) {
          if (r.out != k.src[i]) continue;
          if ((up && (u.oh != r.oh || u.ow != r.ow)) || r.nb * r.oh * r.ow != hw || r.c4 != k.c4len[i])
            return fail(QPH_EINVAL, d.where() + ": read-through input geometry");
          up = true;
          u.oh = (int)r.oh; u.ow = (int)r.ow;
          u.src[i] = (const float4*)d.at(r.src);
          u.ih[i] = (int)r.ih; u.iw[i] = (int)r.iw;
        }
      }
      if (up && hw * outc4 >= (1ll << 31))
        return fail(QPH_EUNSUPPORTED, d.where() + ": read-through concat too large");
      if (up)
        return add_launch(pl, d.idx, [u](hipStream_t s) {
          hipLaunchKernelGGL(plan_concat_up_kernel, dim3(blocks_for((int64_t)u.npx * u.outc4)), dim3(256),
                             0, s, u);
          return launch_check("plan_concat_up_kernel");
        });
      return add_launch(pl, d.idx, [k](hipStream_t s) {
        hipLaunchKernelGGL(plan_concat_kernel, dim3(blocks_for(k.hw * k.outc4)), dim3(256), 0, s, k);
        return launch_check("plan_concat_kernel");
      });
    }
    case PK_SOFTMAX: {
      QPH_TRY(d.params(6, &w));
      const int64_t rows = w[2], cols = w[3], cp = w[4];
      if (rows < 1 || cols < 1 || cp < cols) return fail(QPH_EINVAL, d.where() + ": bad rows / cols");
      QPH_TRY(d.region(w[0], (uint64_t)rows * cp, false, "input"));
      QPH_TRY(d.region(w[1], (uint64_t)rows * cp, false, "output"));
      const float* x = d.at(w[0]);
      float* y = d.at(w[1]);
      if (x != y && (uint64_t)w[1] < (uint64_t)w[0] + rows * cp &&
          (uint64_t)w[0] < (uint64_t)w[1] + rows * cp)
        return fail(QPH_EUNSUPPORTED, d.where() + ": input and output overlap");
      // the first maximum of each row in the same pass when an
      // n_exit3_argmax of this output follows (after n_exit3 reads of it):
      // the softmax kernels take it from the probabilities they store
      // When that argmax is the probabilities' only reader (no n_exit3 of
      // them, no graph output in them: the rec plan's pairs exit), they are
      // not stored at all, nor their padding columns (wide rows only, whose
      // kernels take a null output).
      float* pairs = nullptr;
      bool dead = false;
      for (int j = d.idx + 1; j < d.n_disp; j++) {
        const uint32_t* e3 = d.peek(j, PK_EXIT3, 6);
        const uint32_t* am = d.peek(j, PK_EXIT3_ARGMAX, 6);
        if (e3 && e3[0] == w[1] && ((uint64_t)e3[1] >= (uint64_t)w[1] + rows * cp ||
                                    (uint64_t)e3[1] + (uint64_t)e3[2] * e3[3] <= w[1]))
          continue;
        if (am && am[0] == w[1] && am[2] == rows && am[3] == cols && am[4] == cp) {
          QPH_TRY(d.region(am[1], (uint64_t)rows * 2, false, "pairs"));
          pairs = d.at(am[1]);
          d.skip[j] = 1;
          dead = cols > 128 && d.only_readers(d.idx, w[1], (uint64_t)rows * cp, {j});
        }
        break;
      }
      const unsigned* rn = (const unsigned*)d.at(0);
      const int64_t rpb = w[5];
      PadColsK pk{d.at(0), y, rows, cols, cp, rpb};
      return add_launch(pl, d.idx, [=](hipStream_t s) {
        QPH_TRY(launch_softmax_pitched(x, rows, cols, cp, dead ? nullptr : y, cp, pairs, s, rn,
                                       rpb));
        if (dead || cp == cols) return QPH_OK;
        hipLaunchKernelGGL(plan_pad_cols_kernel, dim3(blocks_for(rows * (cp - cols))), dim3(256),
                           0, s, pk);
        return launch_check("plan_pad_cols_kernel");
      });
    }
    case PK_ATTN_MM: {
      QPH_TRY(d.params(8, &w));
      const int64_t m = w[3], kk = w[4], n = w[5], batch = w[6];
      if (m < 1 || kk < 1 || n < 1 || batch < 1 || batch > 65535)
        return fail(QPH_EINVAL, d.where() + ": bad batched matmul shape");
      QPH_TRY(d.region(w[0], (uint64_t)batch * m * kk, false, "A"));
      QPH_TRY(d.region(w[1], (uint64_t)batch * kk * n, false, "B"));
      QPH_TRY(d.region(w[2], (uint64_t)batch * m * n, false, "output"));
      GemmArgs g{};
      g.a = d.at(w[0]); g.lda = kk; g.a_batch = m * kk;
      g.b = d.at(w[1]); g.ldb = n; g.b_batch = kk * n;
      g.c = d.at(w[2]); g.ldc = n; g.c_batch = m * n;
      g.m = m; g.n = n; g.k = kk; g.batch = batch;
      g.bias = nullptr; g.bias_mode = 0; g.seed_rule = 0;
      g.act = make_act(nullptr);
      // batch items past real_n x heads skipped (n_attn_mm.comp)
      g.rn = (const unsigned*)d.at(0); g.rn_per = w[7];
      return add_launch(pl, d.idx, [g](hipStream_t s) { return launch_gemm(g, s); });
    }
    default:
      return fail(QPH_EUNSUPPORTED, d.where() + ": kernel id " + std::to_string(q.kernel) +
                                        " is not in the HIP kernel set");
  }
}

int capture_plan(qph_plan* pl) {
  hipStream_t s = pl->ctx->stream;
  QPH_TRY_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
  int rc = QPH_OK;
  for (size_t i = 0; i < pl->launches.size() && rc == QPH_OK; i++) {
    rc = pl->launches[i](s);
    if (rc != QPH_OK)
      rc = fail(rc, "plan dispatch " + std::to_string(pl->launch_dispatch[i]) + ": " +
                        qph_last_error());
  }
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(s, &g);
  if (rc != QPH_OK) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  QPH_TRY_HIP(e);
  e = hipGraphInstantiate(&pl->exec, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g);
    return hip_check(e, "hipGraphInstantiate");
  }
  pl->graph = g;
  pl->graph_ready = true;
  return QPH_OK;
}

// The spec's checks that need no device, its uploads sorted into d.ups.
int check_spec(const qph_plan_spec* spec, Decoder& d) {
  if (spec->total_words < 1 || spec->n_dispatches < 1 || spec->n_uploads < 0 ||
      (spec->n_uploads && !spec->uploads) || !spec->dispatches || spec->n_outputs < 1 ||
      !spec->out_offs || !spec->out_numel || spec->in_numel < 1)
    return fail(QPH_EINVAL, "plan_create: empty plan");
  if ((uint64_t)spec->in_f32_off + (uint64_t)spec->in_numel > spec->total_words)
    return fail(QPH_EINVAL, "plan_create: the input region is outside the arena");
  for (int32_t o = 0; o < spec->n_outputs; o++)
    if (spec->out_numel[o] < 1 ||
        (uint64_t)spec->out_offs[o] + (uint64_t)spec->out_numel[o] > spec->total_words)
      return fail(QPH_EINVAL, "plan_create: output " + std::to_string(o) + " is outside the arena");
  for (int32_t u = 0; u < spec->n_uploads; u++) {
    const qph_plan_upload& up = spec->uploads[u];
    if (up.n_words == 0) continue;
    if (!up.words || (uint64_t)up.off + up.n_words > spec->total_words)
      return fail(QPH_EINVAL, "plan_create: upload " + std::to_string(u) + " is outside the arena");
    d.ups.push_back({up.off, up.n_words, up.words});
  }
  std::sort(d.ups.begin(), d.ups.end(),
            [](const PlanUpload& a, const PlanUpload& b) { return a.off < b.off; });
  for (size_t u = 1; u < d.ups.size(); u++)
    if ((uint64_t)d.ups[u - 1].off + d.ups[u - 1].n > d.ups[u].off)
      return fail(QPH_EINVAL, "plan_create: uploads overlap");
  return QPH_OK;
}

// Decodes every dispatch of the spec into launches on d.pl (consumer
// folding included); every parameter block and region is checked here.
int decode_all(Decoder& d, const qph_plan_spec* spec) {
  d.disp = spec->dispatches;
  d.n_disp = spec->n_dispatches;
  d.wr.assign((size_t)d.n_disp, OFF_NONE);
  d.rd.assign((size_t)d.n_disp, {});
  d.skip.assign((size_t)d.n_disp, 0);
  d.outs.assign(spec->out_offs, spec->out_offs + spec->n_outputs);
  for (int32_t i = 0; i < d.n_disp; i++) dispatch_io(d, d.disp[i], &d.wr[i], &d.rd[i]);
  std::vector<PendingHw> pending;
  for (int32_t i = 0; i < spec->n_dispatches; i++) {
    const qph_plan_dispatch& q = spec->dispatches[i];
    if (d.skip[i]) continue;  // taken into an earlier dispatch's launch
    d.idx = i;
    d.kname = (q.kernel >= 0 && q.kernel < kNumPlanKernels) ? kPlanKernels[q.kernel] : "?";
    d.p_off = q.p_off;
    QPH_TRY(decode(d, q, pending));
  }
  if (!pending.empty())
    return fail(QPH_EUNSUPPORTED, "plan_create: an n_reduce_hw without its n_reduce_fin");
  return QPH_OK;
}

// A dry decode: no context, no device.
int validate_plan(const qph_plan_spec* spec) {
  Decoder d;
  QPH_TRY(check_spec(spec, d));
  qph_plan tmp{};
  tmp.ctx = nullptr;
  tmp.arena = nullptr;
  tmp.total_words = spec->total_words;
  d.pl = &tmp;
  d.dry = true;
  return decode_all(d, spec);
}

void release_plan(qph_plan* pl) {
  if (!pl) return;
  if (pl->ctx) (void)hipStreamSynchronize(pl->ctx->stream);
  if (pl->graph_ready) {
    (void)hipGraphExecDestroy(pl->exec);
    (void)hipGraphDestroy(pl->graph);
  }
  if (pl->arena) (void)hipFree(pl->arena);
  for (float* p : pl->owned) (void)hipFree(p);
  delete pl;
}

}  // namespace
}  // namespace qph

using namespace qph;

extern "C" {

QPH_API int qph_plan_kernel_id(const char* name) {
  if (!name) return fail(QPH_EINVAL, "plan_kernel_id: NULL name");
  for (int i = 0; i < kNumPlanKernels; i++)
    if (std::strcmp(name, kPlanKernels[i]) == 0) return i;
  return fail(QPH_EUNSUPPORTED, std::string("plan kernel ") + name + " is not in the HIP kernel set");
}

QPH_API int qph_plan_validate(const qph_plan_spec* spec) {
  if (!spec) return fail(QPH_EINVAL, "plan_validate: NULL argument");
  return validate_plan(spec);
}

QPH_API int qph_plan_create(qph_ctx* ctx, const qph_plan_spec* spec, qph_plan** out) {
  if (!ctx || !spec || !out) return fail(QPH_EINVAL, "plan_create: NULL argument");
  *out = nullptr;
  // every block and region is checked before anything touches the device
  QPH_TRY(validate_plan(spec));
  Decoder d;
  QPH_TRY(check_spec(spec, d));

  qph_plan* pl = new qph_plan();
  pl->ctx = ctx;
  pl->total_words = spec->total_words;
  pl->arena = nullptr;
  pl->graph_ready = false;
  pl->in_off = spec->in_f32_off;
  pl->in_numel = spec->in_numel;
  pl->out_off.assign(spec->out_offs, spec->out_offs + spec->n_outputs);
  pl->out_numel.assign(spec->out_numel, spec->out_numel + spec->n_outputs);
  pl->real_n = 0;
  d.pl = pl;
  auto bail = [&](int rc) {
    release_plan(pl);
    return rc;
  };
  int rc = hip_check(hipSetDevice(ctx->device), "hipSetDevice");
  if (rc) return bail(rc);
  rc = hip_check(hipMalloc((void**)&pl->arena, (size_t)spec->total_words * 4), "hipMalloc(plan arena)");
  if (rc) return bail(rc);
  rc = hip_check(hipMemset(pl->arena, 0, (size_t)spec->total_words * 4), "hipMemset(plan arena)");
  if (rc) return bail(rc);
  for (const PlanUpload& up : d.ups) {
    rc = hip_check(hipMemcpy(pl->arena + up.off, up.words, (size_t)up.n * 4, hipMemcpyHostToDevice),
                   "hipMemcpy(plan upload)");
    if (rc) return bail(rc);
  }
  rc = decode_all(d, spec);
  if (rc) return bail(rc);
  rc = capture_plan(pl);
  if (rc) return bail(rc);
  *out = pl;
  return QPH_OK;
}

QPH_API int qph_plan_destroy(qph_plan* pl) {
  release_plan(pl);
  return QPH_OK;
}

QPH_API int qph_plan_set_real_n(qph_plan* pl, uint32_t real_n) {
  if (!pl) return fail(QPH_EINVAL, "plan_set_real_n: NULL plan");
  pl->real_n = real_n;
  return QPH_OK;
}

QPH_API int qph_plan_run(qph_plan* pl, const float* input, int32_t input_is_device,
                         float* const* outputs_host) {
  if (!pl) return fail(QPH_EINVAL, "plan_run: NULL plan");
  hipStream_t s = pl->ctx->stream;
  // word 0: the real batch rows of this run (0 = all), written before the
  // graph by a kernel that takes the value as an argument (stream-ordered,
  // no host buffer for a later qph_plan_set_real_n to race with)
  hipLaunchKernelGGL(plan_set_real_n_kernel, dim3(1), dim3(64), 0, s, (unsigned*)pl->arena,
                     pl->real_n);
  QPH_TRY(launch_check("plan_set_real_n_kernel"));
  if (input)
    QPH_TRY_HIP(hipMemcpyAsync(pl->arena + pl->in_off, input, (size_t)pl->in_numel * 4,
                               input_is_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, s));
  QPH_TRY_HIP(hipGraphLaunch(pl->exec, s));
  if (outputs_host) {
    for (size_t o = 0; o < pl->out_off.size(); o++) {
      if (!outputs_host[o]) continue;
      QPH_TRY_HIP(hipMemcpyAsync(outputs_host[o], pl->arena + pl->out_off[o],
                                 (size_t)pl->out_numel[o] * 4, hipMemcpyDeviceToHost, s));
    }
    QPH_TRY_HIP(hipStreamSynchronize(s));
  }
  return QPH_OK;
}

QPH_API int qph_plan_arena(qph_plan* pl, float** dev, int64_t* words) {
  if (!pl) return fail(QPH_EINVAL, "plan_arena: NULL plan");
  if (dev) *dev = pl->arena;
  if (words) *words = pl->total_words;
  return QPH_OK;
}

QPH_API int qph_plan_launches(qph_plan* pl, int32_t* n) {
  if (!pl || !n) return fail(QPH_EINVAL, "plan_launches: NULL argument");
  *n = (int32_t)pl->launches.size();
  return QPH_OK;
}

}  // extern "C"
