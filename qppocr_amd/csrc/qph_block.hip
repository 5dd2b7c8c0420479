// Fused backbone block: depthwise conv (+ bias + activation) straight into
// the pointwise 1x1 conv (+ bias + activation), one launch, the depthwise
// output never written to HBM.
//
// Reference: the two Conv nodes of a block (qppocr-core/src/executor.rs:
// 433-652), each followed by its HardSigmoid + Mul pair (746-758, 885-951):
// depthwise as conv.rs:461-505 / x86.rs:994-1060 (acc = 0; for ky, kx:
// acc = fma(w, xpad, acc); y = acc + bias), pointwise as the 1x1 GEMM path
// conv.rs:264-460 (k = input channel ascending, bias after the chain or
// seeded by the same placement rule).  Every element keeps those operation
// sequences; only where the intermediate lives changes.
//
// A workgroup owns 16 consecutive output pixels of one output row of one
// image and a 64-channel slice of M (one 16-channel block per wave).
// Phase 1: one burst of buffer->LDS loads brings the input halo of those
// pixels for all C channels (KH rows x (15*sw + KW) columns, rows padded to
// a multiple of 4 columns; out-of-image taps carry an out-of-range offset
// and read 0, the zero padding) and the k-major weight rows of the slice.
// Phase 2: the depthwise outputs of all C channels for the 16 pixels into
// LDS (t[c][16]); a thread computes PX adjacent pixels of one channel with
// that channel's taps in registers and reads each halo row once (16-byte
// reads where PX * sw is a multiple of 4; the channel pitch is 4 mod 64
// floats, so 16 lanes on 16 channels cover the 64 banks once).
// Phase 3: each wave runs the pointwise chain of its 16 channels with
// v_mfma_f32_16x16x4f32, both operands from LDS.  LDS is sized per launch.
//
// With the stem in front (STEM, the first block of both nets: stem conv
// 3 -> C, 3x3 stride 2 pad 1, then a 3x3 stride-2 pad-1 depthwise), the halo
// is not loaded but computed: phase 1 brings the 3 x 7 x 67 input pixels the
// tile's 3 x 33 stem outputs read (3 x 11 x 67 for 5 x 33 when a workgroup
// owns two output rows, as the launcher picks when one-row workgroups would
// not all be resident at once; the stem row the two rows share is then
// computed once), phase S runs the stem chains on
// v_mfma_f32_16x16x4f32 (16 stem pixels x 16 channels a block, k = c*9 +
// ky*3 + kx ascending after one leading 0 * 0 term, so each output is the
// reference's chain acc = 0; acc = fma(w, x, acc) exactly; taps outside the
// image read 0), adds the bias, applies the activation and writes the halo,
// with exact zeros where the depthwise reads its own zero padding.  The stem
// output never reaches HBM.  Reference for the stem: the Conv node of
// qppocr-core/src/executor.rs:433-652 over conv.rs:264-460 (the implicit
// GEMM; bias after the chain), its HardSigmoid + Mul pair as above.
#include "qph_internal.h"

namespace qph {

typedef float f32x4 __attribute__((ext_vector_type(4)));

#define DWPW_MAX_C 256
#define DWPW_MAX_HALO 20480   // floats of input halo per workgroup (80 KB)
#define DWPW_MSLICE 64        // output channels per workgroup

struct DwPwK {
  const float* x;
  const float* wd;
  const float* bd;
  int c, h, w, sh, sw, ph, pw, oh, ow;
  Act act_d;
  const float* wk;   // pointwise weights, k-major [cpad][mpad], zero-padded
  const float* bp;
  int m, mpad, cpad, seed_rule;
  Act act_p;
  float* y;
  int trans_out;
  int ct;            // halo row pitch: 15 * sw + kw rounded up to 4
  int ctr;           // halo columns read from the image: 15 * sw + kw
  int tiles_x;       // 16-pixel tiles per output row
  int slices;        // 64-channel slices of M
  int halo, wrows;   // LDS floats of the halo and of the weight slice
  int wdl_pad;       // LDS floats of the depthwise weights (rounded to 64)
  int pcp;           // LDS floats per channel of the halo (KH * ct rounded to 64, + 4)
  // stem (STEM launches only)
  const float* xin;
  const float* wst;
  const float* bst;
  int hin, win;
  Act act_s;
  int xvec;          // stem input in 16-byte chunks (region column 0 one left)
};

// Stem tile of a launch whose workgroups own R output rows (R = 1 or 2):
// the depthwise (3x3, stride 2) reads 2R + 1 stem rows x 33 stem columns,
// which the stem (3x3, stride 2) computes from an input region of 3
// channels x (4R + 3) rows x 67 columns, rows 68 floats apart (a row
// arrives as a 64-lane load and a 3-lane load: only active lanes write LDS;
// or, when the input width is a multiple of 4, as 17 aligned 16-byte chunks
// starting one column further left).  The halo rows are CT = 36 floats
// apart; a channel's pitch PCP holds its 2R + 1 rows and the spare words
// where the pixels past the tile of the last 16-pixel block land, and is
// 4 or 60 mod 64 (16 lanes reading 16 consecutive channels hit distinct
// banks).  At one row, 124 floats keep a 16-channel det stem workgroup
// within 16 KB of LDS (what the rec head GEMM leaves free on a CU).
template <int R>
struct StemGeom {
  static constexpr int RR = 4 * R + 3;
  static constexpr int RP = 68;
  static constexpr int IN = 3 * RR * RP;
  static constexpr int ROWS = 2 * R + 1;
  static constexpr int PX = ROWS * 33;
  static constexpr int PB = (PX + 15) / 16;
  static constexpr int CT = 36;
  static constexpr int PCP = R == 1 ? 124 : 196;
  static_assert(ROWS * CT + (PB * 16 - PX) <= PCP && (PCP % 64 == 4 || PCP % 64 == 60), "stem halo pitch");
};
#define ST_K 28            // 27 taps after one leading zero term

// Halo geometry of the 16-byte load path (VEC: left padding KW / 2, image
// width a multiple of 4, 16-byte aligned tensors).  A halo row starts at the
// 4-aligned column SHIFT columns left of the tile's first tap, so every
// 16-byte chunk of it is wholly inside or wholly outside the image; CT
// columns a row (a multiple of 4), CPR chunks a row, CH chunks a channel
// (odd: a channel pitch of 4 mod 8 words puts the 16-byte reads of 16
// consecutive channels on 16 disjoint groups of 4 banks).  Channels are
// contiguous, so one 64-lane load fills 64 consecutive chunks.
template <int KH, int KW, int SW>
struct VecGeom {
  static constexpr int SHIFT = (4 - (KW / 2) % 4) % 4;
  static constexpr int CT = (SHIFT + 15 * SW + KW + 3) / 4 * 4;
  static constexpr int CPR = CT / 4;
  static constexpr int CH = KH * CPR + ((KH * CPR) % 2 == 0 ? 1 : 0);
  static constexpr int PITCH = 4 * CH;
};

// AK = 3: every activation of the launch is the HardSigmoid + Mul pair
// (both nets' blocks), applied inline; AK = 0: any, through act_apply
template <int AK>
__device__ __forceinline__ float act_k(float v, const Act& a) {
  if constexpr (AK == 3) return v * hsig1(v, a.c1, a.c2);
  else return act_apply(v, a);
}

template <int KH, int KW, int SW, int PX, bool STEM, int AK, bool VEC, int R>
__global__ __launch_bounds__(256) void dwpw_kernel(DwPwK p) {
  static_assert(!(STEM && VEC), "the stem computes its halo");
  static_assert(R == 1 || (STEM && R == 2), "two output rows a workgroup: stem launches only");
  using SG = StemGeom<R>;
  extern __shared__ float lds[];
  float* halo = lds;                 // [c][KH][ct]
  float* wsl = lds + p.halo;         // [cpad][64]
  float* t = wsl + p.wrows;          // [cpad][R][16]
  // depthwise weights [c][KH*KW], then bias [c]; STEM: after the halo (no
  // weight slice), t aliasing the input region instead
  float* wdl = STEM ? wsl : t + p.cpad * 16 * R;
  // STEM: depthwise bias [c] after its weights, input region [3][4R + 3][68],
  // stem weights [c][27] (28 c floats of room), stem bias [c]
  float* xin = wdl + p.wdl_pad + (STEM ? (p.c + 3) / 4 * 4 : (p.c + 63) / 64 * 64);
  // (phase 2 writes t only after the barrier that ends phase S, the last
  // reader of the input region)
  if constexpr (STEM) t = xin;
  float* wsm = xin + SG::IN;
  float* bsm = wsm + ST_K * p.c;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int img = blockIdx.z;
  const int slice = blockIdx.y;
  // STEM (one 64-channel slice, cpad = 16 PX): this lane's pointwise A terms
  // W[m = 16 wave + l][k = 4 s + g] of the k-major repack, loaded first so
  // that their latency hides under phase 1; read by phase 3 from registers
  constexpr int WS = STEM ? 4 * PX : 1;
  // the pointwise bias of this lane's four output channels, loaded now
  // (latency under phase 1)
  float bpre[4];
#pragma unroll
  for (int v = 0; v < 4; v++) {
    const int mo = (slice * 4 + wave) * 16 + 4 * (lane >> 4) + v;
    bpre[v] = (p.bp && mo < p.m) ? p.bp[mo] : 0.0f;
  }
  float wreg[WS];
  if constexpr (STEM) {
    const int col = wave * 16 + (lane & 15);
#pragma unroll
    for (int u = 0; u < WS; u++)
      wreg[u] = col < p.mpad ? p.wk[(4 * u + (lane >> 4)) * p.mpad + col] : 0.0f;
  }
  // this workgroup's output rows oy .. oy + R - 1 (rows past the map are
  // computed from zeros and not stored)
  const int ob = blockIdx.x / p.tiles_x;
  const int oy = ob * R;
  const int ox0 = (blockIdx.x - ob * p.tiles_x) * 16;
  const int64_t plane = (int64_t)p.h * p.w;
  const unsigned OOB = 0x80000000u;

  // phase 1: halo and weight slice, all loads in flight at once
  {
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.x + (int64_t)img * p.c * plane), 0, (int)(p.c * plane * 4), 0x00020000);
    // lane -> a fixed (row, column) of a channel's halo (one or two loads
    // per channel); the channel moves the scalar offset only, so the loop
    // issues no vector instructions.  Out-of-image taps keep an
    // out-of-range vector offset (read 0) whatever the scalar offset.
    const int iy0 = oy * p.sh - p.ph, ix0 = ox0 * p.sw - p.pw;
    if constexpr (STEM) {
      // input rows 2 * iy0 - 1 .., columns 2 * ix0 - 1 .. (the stem is
      // stride 2, pad 1); a row per (channel, region row), columns 0-63
      // and 64-66
      const int64_t iplane = (int64_t)p.hin * p.win;
      const __amdgpu_buffer_rsrc_t ir = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(p.xin + (int64_t)img * 3 * iplane), 0, (int)(3 * iplane * 4), 0x00020000);
      const int jy0 = 2 * iy0 - 1, jx0 = 2 * ix0 - 1;
      // stem weights in their ONNX layout [c][27] and the bias (27 c and c
      // floats: whole 16-byte chunks, c being 16 or 32)
      const int nws = 27 * p.c;
      const __amdgpu_buffer_rsrc_t swr =
          __builtin_amdgcn_make_buffer_rsrc((void*)p.wst, 0, nws * 4, 0x00020000);
      if (p.xvec) {
        // chunk q: region row q / 17 (channel, row), columns jx0 - 1 + 4 (q % 17)
        // .. + 3, wholly inside or outside the image (width % 4 == 0)
        for (int q0 = wave * 64; q0 < 3 * SG::RR * 17; q0 += 256) {
          const int q = q0 + lane, cr = q / 17, j = q - 17 * cr;
          const int c = cr / SG::RR, iy = jy0 + cr - c * SG::RR, ix = jx0 - 1 + 4 * j;
          const bool ok = iy >= 0 && iy < p.hin && ix >= 0 && ix < p.win;
          if (q < 3 * SG::RR * 17)
            lds_load16(ir, xin + 4 * q0, ok ? (unsigned)(((c * p.hin + iy) * p.win + ix) * 4) : OOB, 0);
        }
        for (int base = wave * 256; base < nws; base += 1024)
          if (base + 4 * lane < nws) lds_load16(swr, wsm + base, (unsigned)(base + 4 * lane) * 4u, 0);
        if (p.bst && wave == 0 && 4 * lane < p.c) {
          const __amdgpu_buffer_rsrc_t sbr =
              __builtin_amdgcn_make_buffer_rsrc((void*)p.bst, 0, p.c * 4, 0x00020000);
          lds_load16(sbr, bsm, (unsigned)lane * 16u, 0);
        }
      } else {
        for (int cr = wave; cr < 3 * SG::RR; cr += 4) {
          const int c = cr / SG::RR, rr = cr - c * SG::RR;
          const int iy = jy0 + rr;
#pragma unroll
          for (int j = 0; j < 2; j++) {
            const int col = 64 * j + lane, ix = jx0 + col;
            const bool ok = iy >= 0 && iy < p.hin && ix >= 0 && ix < p.win;
            if (j == 0 || lane < 3)
              __builtin_amdgcn_raw_ptr_buffer_load_lds(
                  ir, (__attribute__((address_space(3))) void*)(xin + cr * SG::RP + 64 * j), 4,
                  ok ? (unsigned)(((c * p.hin + iy) * p.win + ix) * 4) : OOB, 0, 0, 0);
          }
        }
        for (int base = wave * 64; base < nws; base += 256)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              swr, (__attribute__((address_space(3))) void*)(wsm + base), 4,
              (unsigned)(base + lane) * 4u, 0, 0, 0);
        if (p.bst && wave == 0) {
          const __amdgpu_buffer_rsrc_t sbr =
              __builtin_amdgcn_make_buffer_rsrc((void*)p.bst, 0, p.c * 4, 0x00020000);
          if (lane < p.c)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(sbr, (__attribute__((address_space(3))) void*)bsm,
                                                     4, (unsigned)lane * 4u, 0, 0, 0);
        }
      }
    } else if constexpr (VEC) {
      // chunk q of the [c][CH] halo: channel q / CH, row (q % CH) / CPR,
      // columns ix0 - SHIFT + 4 ((q % CH) % CPR) .. + 3; chunks outside the
      // image (and the odd channel's spare chunk) carry an out-of-range
      // offset and read 0; lanes past the last chunk stay inactive
      using G = VecGeom<KH, KW, SW>;
      const int ix0a = ix0 - G::SHIFT;
      const int nch = p.c * G::CH;
      for (int q0 = wave * 64; q0 < nch; q0 += 256) {
        const int q = q0 + lane;
        const int ci = q / G::CH, rem = q - ci * G::CH;
        const int r = rem / G::CPR, j = rem - r * G::CPR;
        const int iy = iy0 + r, ix = ix0a + 4 * j;
        const bool ok = r < KH && iy >= 0 && iy < p.h && ix >= 0 && ix < p.w;
        if (q < nch)
          lds_load16(xr, halo + 4 * q0, ok ? (unsigned)((ci * (int)plane + iy * p.w + ix) * 4) : OOB,
                     0);
      }
    } else {
      const int per_c = KH * p.ct;
      unsigned voff[2];
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int q = 64 * j + lane;
        const int r = q / p.ct, col = q - r * p.ct;
        const int iy = iy0 + r, ix = ix0 + col;
        const bool ok = q < per_c && col < p.ctr && iy >= 0 && iy < p.h && ix >= 0 && ix < p.w;
        voff[j] = ok ? (unsigned)((iy * p.w + ix) * 4) : OOB;
      }
      for (int ci = wave; ci < p.c; ci += 4) {
        const int soff = (int)(ci * plane * 4);
#pragma unroll
        for (int j = 0; j < 2; j++)
          if (64 * j < per_c)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                xr, (__attribute__((address_space(3))) void*)(halo + ci * p.pcp + 64 * j), 4,
                voff[j], soff, 0, 0);
      }
    }
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)p.wk, 0, p.cpad * p.mpad * 4, 0x00020000);
    const int m0 = slice * DWPW_MSLICE;
    // weight row k holds column j of the slice at j ^ (16 (k % 4)), so that
    // phase 3's four row groups read four disjoint groups of 16 banks
    // (a wave's rows k = wave + 4 i all have k % 4 == wave)
    const int wcol = m0 + (lane ^ (16 * wave));
    const unsigned woff = wcol < p.mpad ? (unsigned)(wcol * 4) : OOB;
    const int nwd = p.c * KH * KW;
    const __amdgpu_buffer_rsrc_t dwr =
        __builtin_amdgcn_make_buffer_rsrc((void*)p.wd, 0, nwd * 4, 0x00020000);
    if constexpr (VEC) {
      // 16-byte chunks: the weight rows k (16 chunks of the slice each;
      // mpad is a multiple of 32, so a chunk is wholly inside or outside
      // it; chunk j of row k lands at j ^ (4 (k % 4))), the depthwise
      // weights and bias (c % 4 == 0: whole chunks)
      for (int q0 = wave * 64; q0 < p.cpad * 16; q0 += 256) {
        const int q = q0 + lane, col = m0 + 4 * ((q & 15) ^ (4 * ((q >> 4) & 3)));
        lds_load16(wr, wsl + 4 * q0, col < p.mpad ? (unsigned)(((q >> 4) * p.mpad + col) * 4) : OOB, 0);
      }
      for (int base = wave * 256; base < nwd; base += 1024)
        if (base + 4 * lane < nwd) lds_load16(dwr, wdl + base, (unsigned)(base + 4 * lane) * 4u, 0);
      if (p.bd) {
        const __amdgpu_buffer_rsrc_t br =
            __builtin_amdgcn_make_buffer_rsrc((void*)p.bd, 0, p.c * 4, 0x00020000);
        for (int base = wave * 256; base < p.c; base += 1024)
          if (base + 4 * lane < p.c)
            lds_load16(br, wdl + p.wdl_pad + base, (unsigned)(base + 4 * lane) * 4u, 0);
      }
    } else {
      // (STEM: the pointwise weights go to registers below, not to LDS)
      for (int k = wave; k < (STEM ? 0 : p.cpad); k += 4)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            wr, (__attribute__((address_space(3))) void*)(wsl + k * 64), 4, woff,
            k * p.mpad * 4, 0, 0);
      // depthwise weights and bias (contiguous [c][KH*KW] and [c])
      for (int base = wave * 64; base < nwd; base += 256)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            dwr, (__attribute__((address_space(3))) void*)(wdl + base), 4,
            (unsigned)(base + lane) * 4u, 0, 0, 0);
      if (p.bd) {
        const __amdgpu_buffer_rsrc_t br =
            __builtin_amdgcn_make_buffer_rsrc((void*)p.bd, 0, p.c * 4, 0x00020000);
        for (int base = wave * 64; base < p.c; base += 256)
          if (base + lane < p.c)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                br, (__attribute__((address_space(3))) void*)(wdl + p.wdl_pad + base), 4,
                (unsigned)(base + lane) * 4u, 0, 0, 0);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // phase S: the stem outputs of the halo, pixel block pb (16 stem pixels)
  // per wave task, all channel blocks cb (16 channels each) of that block in
  // the task; lane (g, l) feeds stem pixel 16 pb + l's tap k' = 4 s + g and
  // takes outputs (pixel 16 pb + 4 g + v, channel 16 cb + l)
  if constexpr (STEM) {
    const int l16 = lane & 15, lg = lane >> 4;
    const int sy0 = oy * p.sh - p.ph, sx0 = ox0 * p.sw - p.pw;
    constexpr int NCB = 2;          // channel blocks: c is 16 or 32
    const int ncb = p.c >> 4;
    // tap offsets in the input region, k = k' - 1 = c * 9 + ky * 3 + kx
    // (-1: the leading zero term)
    int koff[ST_K / 4];
#pragma unroll
    for (int s = 0; s < ST_K / 4; s++) {
      const int k = 4 * s + lg - 1;
      const int c = k / 9, ky = (k - 9 * c) / 3, kx = k - 9 * c - 3 * ky;
      koff[s] = k < 0 ? -1 : (c * SG::RR + ky) * SG::RP + kx + p.xvec;
    }
    // this lane's weights and bias of every channel block, read once:
    // weight (k', channel) = w[ch][k' - 1], 0 for the leading term (27
    // words apart over the 16 channels: no bank conflict); the words read
    // for absent blocks or the leading term are in bounds and unused
    float bw[NCB][ST_K / 4], bb[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; cb++) {
#pragma unroll
      for (int s = 0; s < ST_K / 4; s++)
        bw[cb][s] = wsm[cb < ncb && koff[s] >= 0 ? (cb * 16 + l16) * 27 + 4 * s + lg - 1 : 0];
      bb[cb] = bsm[cb * 16 + l16];
    }
#pragma unroll
    for (int cb = 0; cb < NCB; cb++)
#pragma unroll
      for (int s = 0; s < ST_K / 4; s++) bw[cb][s] = koff[s] >= 0 ? bw[cb][s] : 0.0f;
    for (int pb = wave; pb < SG::PB; pb += 4) {
      const int q = pb * 16 + l16;
      const bool qok = q < SG::PX;
      const int qr = q / 33, qc = q - 33 * qr;
      const int poff = 2 * qr * SG::RP + 2 * qc;
      // the input operands, one LDS round trip (the leading term and pixels
      // past the tile read word 0 and select 0)
      float a[ST_K / 4];
#pragma unroll
      for (int s = 0; s < ST_K / 4; s++) a[s] = xin[koff[s] >= 0 && qok ? koff[s] + poff : 0];
      // this lane's four output pixels: halo offset, inside the stem map
      // (outside: the depthwise's zero padding).  Pixels past the tile (the
      // last block's, in row 2R + 1) land in the channel pitch's spare
      // words, which the depthwise never reads.
      int hoff[4];
      bool inmap[4];
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const int qo = pb * 16 + 4 * lg + v;
        const int ro = qo / 33, co = qo - 33 * ro;
        const int sy = sy0 + ro, sx = sx0 + co;
        hoff[v] = ro * SG::CT + co;
        inmap[v] = sy >= 0 && sy < p.h && sx >= 0 && sx < p.w;
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int s = 0; s < ST_K / 4; s++) a[s] = koff[s] >= 0 && qok ? a[s] : 0.0f;
      f32x4 acc[NCB];
#pragma unroll
      for (int cb = 0; cb < NCB; cb++) {
        acc[cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if (cb < ncb) {
#pragma unroll
          for (int s = 0; s < ST_K / 4; s++)
            acc[cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], bw[cb][s], acc[cb], 0, 0, 0);
        }
      }
#pragma unroll
      for (int cb = 0; cb < NCB; cb++) {
        if (cb < ncb) {
          float* hc = halo + (cb * 16 + l16) * SG::PCP;
#pragma unroll
          for (int v = 0; v < 4; v++) {
            const float y = act_k<AK>(p.bst ? acc[cb][v] + bb[cb] : acc[cb][v], p.act_s);
            hc[hoff[v]] = inmap[v] ? y : 0.0f;
          }
        }
      }
    }
    __syncthreads();
  }

  // phase 2: depthwise outputs of every channel for the 16 pixels of each of
  // the R rows; task e = (part, channel): row rw = part / (16 / PX), pixels
  // pp * PX .. pp * PX + PX - 1 of it (pp = part % (16 / PX)), channel ci
  const int npx = p.oh * p.ow;
  {
    // halo columns of a task's row, from its 16-byte aligned start (the
    // first tap SH columns in)
    constexpr int SH = VEC ? VecGeom<KH, KW, SW>::SHIFT : 0;
    constexpr int NC = SH + (PX - 1) * SW + KW;
    constexpr bool V4 = (PX * SW) % 4 == 0;  // row start 16-byte aligned
    constexpr int NV = (NC + 3) / 4;
    constexpr int NR = V4 ? 4 * NV : NC;
    const int ntask = p.cpad * (16 / PX) * R;
    for (int e = tid; e < ntask; e += 256) {
      const int part = e / p.cpad;
      const int ci = e - part * p.cpad;
      const int rw = R == 1 ? 0 : part / (16 / PX);
      const int px0 = (part - rw * (16 / PX)) * PX;
      float acc[PX];
#pragma unroll
      for (int q = 0; q < PX; q++) acc[q] = 0.0f;
      if (ci < p.c) {
        float wv[KH * KW];
        const float* wp = wdl + ci * KH * KW;
#pragma unroll
        for (int j = 0; j < KH * KW; j++) wv[j] = wp[j];
        const float* hp = halo + ci * (VEC ? VecGeom<KH, KW, SW>::PITCH : p.pcp) +
                          rw * p.sh * (VEC ? VecGeom<KH, KW, SW>::CT : p.ct) + px0 * SW;
        // every row read before the first FMA (one LDS round trip)
        float r[KH][NR];
#pragma unroll
        for (int ky = 0; ky < KH; ky++) {
          const float* rp = hp + ky * (VEC ? VecGeom<KH, KW, SW>::CT : p.ct);
          if constexpr (V4) {
            // only the words the taps use (SH .. NC - 1): 16-byte reads of
            // whole aligned chunks, single words at either end (a partly
            // dead 16-byte destination would let its registers be reused
            // under the pending read, and the compiler then waits)
#pragma unroll
            for (int v = 0; v < NV; v++) {
              if (4 * v >= SH && 4 * v + 4 <= NC) {
                const f32x4 t4 = *(const f32x4*)(rp + 4 * v);
                r[ky][4 * v] = t4[0];
                r[ky][4 * v + 1] = t4[1];
                r[ky][4 * v + 2] = t4[2];
                r[ky][4 * v + 3] = t4[3];
              } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                  if (4 * v + e >= SH && 4 * v + e < NC) r[ky][4 * v + e] = rp[4 * v + e];
              }
            }
          } else {
#pragma unroll
            for (int j = SH; j < NC; j++) r[ky][j] = rp[j];
          }
        }
        __builtin_amdgcn_sched_barrier(0);   // keep the reads ahead of the FMAs
#pragma unroll
        for (int ky = 0; ky < KH; ky++)
#pragma unroll
          for (int kx = 0; kx < KW; kx++)
#pragma unroll
            for (int q = 0; q < PX; q++)
              acc[q] = __builtin_fmaf(wv[ky * KW + kx], r[ky][SH + q * SW + kx], acc[q]);
      }
      // the bias read once (in bounds for every ci < cpad), the outputs
      // past the image or the channels select 0
      const float bdv = p.bd ? wdl[p.wdl_pad + ci] : 0.0f;
      float o[PX];
#pragma unroll
      for (int q = 0; q < PX; q++) {
        const float v = act_k<AK>(acc[q] + bdv, p.act_d);
        o[q] = (ci < p.c && ox0 + px0 + q < p.ow) ? v : 0.0f;
      }
      float* tp = t + ci * 16 * R + rw * 16 + px0;
      if constexpr (PX % 4 == 0) {
#pragma unroll
        for (int q = 0; q < PX; q += 4) *(f32x4*)(tp + q) = f32x4{o[q], o[q + 1], o[q + 2], o[q + 3]};
      } else {
#pragma unroll
        for (int q = 0; q < PX; q++) tp[q] = o[q];
      }
    }
  }
  __syncthreads();

  // phase 3: pointwise chain of this wave's 16 channels, for each of the R rows
  const int l16 = lane & 15, lg = lane >> 4;
  const int mb = slice * 4 + wave;            // 16-channel block index
  if (mb * 16 >= p.m) return;
  for (int rw = 0; rw < R; rw++) {
    const int px = (oy + rw) * p.ow + ox0 + l16;
    const bool pok = ox0 + l16 < p.ow && oy + rw < p.oh;
    f32x4 acc;
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int mo = mb * 16 + 4 * lg + v;
      float s0 = 0.0f;
      if (p.bp && mo < p.m && pok && bias_seeded(p.seed_rule, mo, px, p.m, npx)) s0 = bpre[v];
      acc[v] = s0;
    }
    const float* al = wsl + lg * 64 + ((wave * 16 + l16) ^ (16 * lg));   // swizzled rows
    const float* bl = t + lg * 16 * R + rw * 16 + l16;
    const int nsteps = p.cpad >> 2;
    int s = 0;
    if constexpr (STEM) {
#pragma unroll
      for (int u = 0; u < WS; u++)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wreg[u], bl[u * 64 * R], acc, 0, 0, 0);
      s = nsteps;
    }
    // (the LDS-fed chain below: R = 1 launches only)
    if (!STEM && s + 4 <= nsteps) {
      // groups of 4 steps in two register sets: the next group's operands
      // are read before this group's MFMAs (a group past the end re-reads
      // the current one: in bounds, unused)
      float a0[4], b0[4], a1[4], b1[4];
      auto ld = [&](float* a, float* b, const float* ap, const float* bp) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
          a[u] = ap[u * 256];
          b[u] = bp[u * 64];
        }
      };
      auto mm = [&](const float* a, const float* b) {
#pragma unroll
        for (int u = 0; u < 4; u++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u], b[u], acc, 0, 0, 0);
      };
      const float* ap = al;
      const float* bp = bl;
      ld(a0, b0, ap, bp);
      for (; s + 8 <= nsteps; s += 8) {
        ld(a1, b1, ap + 1024, bp + 256);
        mm(a0, b0);
        const int nx = s + 12 <= nsteps ? 2 : 1;
        ld(a0, b0, ap + nx * 1024, bp + nx * 256);
        mm(a1, b1);
        // reads of the next group ahead of each group's MFMAs
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        ap += 2048;
        bp += 512;
      }
      if (s + 4 <= nsteps) {
        mm(a0, b0);
        s += 4;
      }
    }
    for (; !STEM && s < nsteps; s++)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(al[s * 256], bl[s * 64], acc, 0, 0, 0);

    // epilogue: bias terms first, then finish and store
    float badd[4];
    bool hadd[4];
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int mo = mb * 16 + 4 * lg + v;
      hadd[v] = p.bp && mo < p.m && pok && !bias_seeded(p.seed_rule, mo, px, p.m, npx);
      badd[v] = hadd[v] ? bpre[v] : 0.0f;
    }
    if (!pok) continue;
    float r[4];
#pragma unroll
    for (int v = 0; v < 4; v++) {
      r[v] = acc[v];
      if (hadd[v]) r[v] = r[v] + badd[v];
      r[v] = act_k<AK>(r[v], p.act_p);
    }
    const int mo0 = mb * 16 + 4 * lg;
    // channel-last: this lane's four channels of the pixel are adjacent, one
    // 16-byte store when they are all inside M and 16-byte aligned
    if (p.trans_out && mo0 + 3 < p.m && p.m % 4 == 0 && ((uintptr_t)p.y & 15) == 0) {
      *(f32x4*)(p.y + ((int64_t)img * npx + px) * p.m + mo0) = f32x4{r[0], r[1], r[2], r[3]};
      continue;
    }
#pragma unroll
    for (int v = 0; v < 4; v++) {
      const int mo = mo0 + v;
      if (mo >= p.m) continue;
      if (p.trans_out)
        p.y[((int64_t)img * npx + px) * p.m + mo] = r[v];
      else
        p.y[((int64_t)img * p.m + mo) * npx + px] = r[v];
    }
  }
}

// Register-fed form of the same block, for the 16-byte path's shapes with
// C = 4 NS channels (NS = 4, 8, 16 or 32): the same tile (16 output pixels of a
// row, a 64-channel slice of M) and the same arithmetic, with only the
// depthwise outputs in LDS (C x 16 floats, at most 8 KB, where dwpw_kernel
// stages the whole input halo and weight slice: 40-115 KB).  A workgroup
// this small fits beside other kernels' workgroups on a CU, for instance
// beside the rec head GEMM (144 KB of LDS a CU) when the det and rec graphs
// run concurrently.
//  - First, each lane loads its NS pointwise A operands W[k = 4 s + g][m]
//    (the k-major repack, m = this wave's 16-channel block + l16) into
//    registers; their latency runs under the depthwise phase.
//  - Depthwise: task (channel ci, quarter part) computes the 4 outputs
//    part * 4 .. + 3 of the tile for channel ci.  Its window is the KH input
//    rows x 3 aligned 16-byte chunks starting 4 columns left of its first
//    output's first tap (so the first tap sits SHIFT = 4 - KW / 2 words in),
//    loaded straight into registers; a chunk is wholly inside or outside
//    the image (width % 4 == 0), outside ones read 0 through the buffer
//    range check, which is the zero padding.  The taps and bias come from
//    memory.  Lanes 4 ci + part: one load instruction touches 16 channels'
//    rows, four consecutive chunks each.  acc = fma(w, x, acc) over ky then
//    kx from 0, + bias, activation; outputs past the image store 0.
//  - One barrier; each wave then runs the chain of its 16 output channels
//    over k = 4 s + g ascending on v_mfma_f32_16x16x4f32, the B operands
//    read from LDS, and stores as dwpw_kernel does.
#define DWPW_REG_MAXC 128

template <int KH, int KW, int SW, int NS, int AK>
__global__ __launch_bounds__(256) void dwpw_reg_kernel(DwPwK p) {
  constexpr int C = 4 * NS;
  constexpr int PX = 4;
  constexpr int SHIFT = 4 - KW / 2;
  constexpr int NC = SHIFT + (PX - 1) * SW + KW;
  constexpr int NV = (NC + 3) / 4;
  static_assert(C <= DWPW_REG_MAXC && NV == 3, "");
  __shared__ __attribute__((aligned(16))) float t[C * 16];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, lg = lane >> 4;
  const int img = blockIdx.z, slice = blockIdx.y;
  const int oy = blockIdx.x / p.tiles_x;
  const int ox0 = (blockIdx.x - oy * p.tiles_x) * 16;
  const int mb = slice * 4 + wave;            // 16-channel block index
  const unsigned OOB = 0x80000000u;

  // pointwise A operands and this lane's four bias terms, issued first
  float wa[NS];
  {
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)p.wk, 0, C * p.mpad * 4, 0x00020000);
    const int col = mb * 16 + l16;
    const unsigned vo = col < p.mpad ? (unsigned)(lg * p.mpad + col) * 4u : OOB;
#pragma unroll
    for (int s = 0; s < NS; s++)
      wa[s] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(wr, vo, 16 * s * p.mpad, 0));
  }
  float bpre[4];
#pragma unroll
  for (int v = 0; v < 4; v++) {
    const int mo = mb * 16 + 4 * lg + v;
    bpre[v] = (p.bp && mo < p.m) ? p.bp[mo] : 0.0f;
  }

  // depthwise phase
  {
    const int64_t plane = (int64_t)p.h * p.w;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.x + (int64_t)img * C * plane), 0, (int)(C * plane * 4), 0x00020000);
    const int iy0 = oy * p.sh - p.ph;
#pragma unroll
    for (int e0 = 0; e0 < 4 * C; e0 += 256) {
      const int e = e0 + tid;
      if (4 * C % 256 != 0 && e >= 4 * C) break;
      const int ci = e >> 2, part = e & 3;
      const int px0 = part * PX;
      const int wx = (ox0 + px0) * SW - 4;    // window column 0 (a multiple of 4)
      float r[KH][4 * NV];
#pragma unroll
      for (int ky = 0; ky < KH; ky++) {
        const int iy = iy0 + ky;
        const bool rok = iy >= 0 && iy < p.h;
#pragma unroll
        for (int v = 0; v < NV; v++) {
          const int ix = wx + 4 * v;
          const unsigned off =
              rok && ix >= 0 && ix < p.w ? (unsigned)((ci * (int)plane + iy * p.w + ix) * 4) : OOB;
          const f32x4 q =
              __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
#pragma unroll
          for (int j = 0; j < 4; j++) r[ky][4 * v + j] = q[j];
        }
      }
      float wv[KH * KW];
      const float* wp = p.wd + ci * KH * KW;
#pragma unroll
      for (int j = 0; j < KH * KW; j++) wv[j] = wp[j];
      const float bdv = p.bd ? p.bd[ci] : 0.0f;
      float acc[PX];
#pragma unroll
      for (int q = 0; q < PX; q++) acc[q] = 0.0f;
#pragma unroll
      for (int ky = 0; ky < KH; ky++)
#pragma unroll
        for (int kx = 0; kx < KW; kx++)
#pragma unroll
          for (int q = 0; q < PX; q++)
            acc[q] = __builtin_fmaf(wv[ky * KW + kx], r[ky][SHIFT + q * SW + kx], acc[q]);
      float o[PX];
#pragma unroll
      for (int q = 0; q < PX; q++) {
        const float v = act_k<AK>(acc[q] + bdv, p.act_d);
        o[q] = ox0 + px0 + q < p.ow ? v : 0.0f;
      }
      *(f32x4*)(t + ci * 16 + px0) = f32x4{o[0], o[1], o[2], o[3]};
    }
  }
  __syncthreads();

  // pointwise chain of this wave's 16 channels
  if (mb * 16 >= p.m) return;
  const int npx = p.oh * p.ow;
  const int px = oy * p.ow + ox0 + l16;
  const bool pok = ox0 + l16 < p.ow;
  float bv[NS];
#pragma unroll
  for (int s = 0; s < NS; s++) bv[s] = t[(4 * s + lg) * 16 + l16];
  f32x4 acc;
#pragma unroll
  for (int v = 0; v < 4; v++) {
    const int mo = mb * 16 + 4 * lg + v;
    float s0 = 0.0f;
    if (p.bp && mo < p.m && pok && bias_seeded(p.seed_rule, mo, px, p.m, npx)) s0 = bpre[v];
    acc[v] = s0;
  }
#pragma unroll
  for (int s = 0; s < NS; s++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[s], bv[s], acc, 0, 0, 0);

  float badd[4];
  bool hadd[4];
#pragma unroll
  for (int v = 0; v < 4; v++) {
    const int mo = mb * 16 + 4 * lg + v;
    hadd[v] = p.bp && mo < p.m && pok && !bias_seeded(p.seed_rule, mo, px, p.m, npx);
    badd[v] = hadd[v] ? bpre[v] : 0.0f;
  }
  if (!pok) return;
  float r[4];
#pragma unroll
  for (int v = 0; v < 4; v++) {
    r[v] = acc[v];
    if (hadd[v]) r[v] = r[v] + badd[v];
    r[v] = act_k<AK>(r[v], p.act_p);
  }
  const int mo0 = mb * 16 + 4 * lg;
  if (p.trans_out && mo0 + 3 < p.m && p.m % 4 == 0 && ((uintptr_t)p.y & 15) == 0) {
    *(f32x4*)(p.y + ((int64_t)img * npx + px) * p.m + mo0) = f32x4{r[0], r[1], r[2], r[3]};
    return;
  }
#pragma unroll
  for (int v = 0; v < 4; v++) {
    const int mo = mo0 + v;
    if (mo >= p.m) continue;
    if (p.trans_out)
      p.y[((int64_t)img * npx + px) * p.m + mo] = r[v];
    else
      p.y[((int64_t)img * p.m + mo) * npx + px] = r[v];
  }
}

// halo row pitch: 15 * sw + KW columns rounded up to 4 (16-byte rows)
static int halo_ct(const DwPwArgs& a) { return (int)((15 * a.sw + a.kw + 3) / 4 * 4); }
// halo per channel: KH rows, in one or two loads
static int halo_per_c(const DwPwArgs& a) { return (int)(a.kh * halo_ct(a)); }
// channel pitch 4 mod 64 floats: 16 lanes reading 16 consecutive channels
// 16 bytes each hit the 64 banks once
static int halo_pcp(const DwPwArgs& a) { return (halo_per_c(a) + 63) / 64 * 64 + 4; }
static int halo_floats(const DwPwArgs& a) { return (int)(a.c * halo_pcp(a)); }
// pixels per depthwise task: about one task per thread
static int dw_px(int64_t cpad) { return cpad >= 128 ? 8 : cpad >= 64 ? 4 : cpad >= 32 ? 2 : 1; }

// LDS of a (non-stem) launch with `halo` floats of input halo: halo,
// k-major pointwise weight slice, depthwise outputs, depthwise weights and
// bias (the layout launch_dwpw sizes)
static int64_t dwpw_lds_bytes(const DwPwArgs& a, int64_t halo) {
  const int64_t cpad = (a.c + 3) / 4 * 4;
  return (halo + cpad * 64 + cpad * 16 + (a.c * a.kh * a.kw + 63) / 64 * 64 + (a.c + 63) / 64 * 64) *
         4;
}

// (5x5 taps with x-stride 1 only: the 5x5 kernel instances are stride-1)
bool dwpw_eligible(const DwPwArgs& a) {
  return ((a.kh == 3 && a.kw == 3 && (a.sw == 1 || a.sw == 2)) ||
          (a.kh == 5 && a.kw == 5 && a.sw == 1)) &&
         a.c > 0 && a.c <= DWPW_MAX_C && a.m > 0 && a.n <= 65535 &&
         halo_per_c(a) <= 128 && halo_floats(a) <= DWPW_MAX_HALO &&
         dwpw_lds_bytes(a, halo_floats(a)) <= 160 * 1024 &&
         a.c * a.h * a.w * 4 < (int64_t)0x80000000 && a.oh * a.ow < (1ll << 30) &&
         (a.m + 31) / 32 * 32 * ((a.c + 3) / 4 * 4) * 4 < (1ll << 31);
}

template <int KH, int KW, int SW, int PX, bool STEM, int AK, bool VEC, int R>
static int launch_dwpw_a(dim3 grid, size_t lds, const DwPwK& p, hipStream_t s) {
  // the widest halo row read of a task stays inside its row
  static_assert(VEC || (16 - PX) * SW + 4 * (((PX - 1) * SW + KW + 3) / 4) <=
                           (15 * SW + KW + 3) / 4 * 4 + 4,
                "depthwise row reads past the halo row");
  static_assert(!VEC || (16 - PX) * SW +
                            ((PX * SW) % 4 == 0
                                 ? 4 * ((VecGeom<KH, KW, SW>::SHIFT + (PX - 1) * SW + KW + 3) / 4)
                                 : VecGeom<KH, KW, SW>::SHIFT + (PX - 1) * SW + KW) <=
                            VecGeom<KH, KW, SW>::CT,
                "depthwise row reads past the halo row");
  QPH_TRY(allow_full_lds((const void*)dwpw_kernel<KH, KW, SW, PX, STEM, AK, VEC, R>));
  hipLaunchKernelGGL((dwpw_kernel<KH, KW, SW, PX, STEM, AK, VEC, R>), grid, dim3(256), lds, s, p);
  return launch_check("dwpw_kernel");
}

template <int KH, int KW, int SW, int PX, bool STEM = false, bool VEC = false, int R = 1>
static int launch_dwpw_t(dim3 grid, size_t lds, const DwPwK& p, hipStream_t s) {
  const bool hs = p.act_d.kind == 3 && p.act_p.kind == 3 && (!STEM || p.act_s.kind == 3);
  return hs ? launch_dwpw_a<KH, KW, SW, PX, STEM, 3, VEC, R>(grid, lds, p, s)
            : launch_dwpw_a<KH, KW, SW, PX, STEM, 0, VEC, R>(grid, lds, p, s);
}

template <int KH, int KW, int SW, bool VEC>
static int launch_dwpw_px(int px, dim3 grid, size_t lds, const DwPwK& p, hipStream_t s) {
  switch (px) {
    case 8: return launch_dwpw_t<KH, KW, SW, 8, false, VEC>(grid, lds, p, s);
    case 4: return launch_dwpw_t<KH, KW, SW, 4, false, VEC>(grid, lds, p, s);
    case 2: return launch_dwpw_t<KH, KW, SW, 2, false, VEC>(grid, lds, p, s);
    default: return launch_dwpw_t<KH, KW, SW, 1, false, VEC>(grid, lds, p, s);
  }
}

template <int KH, int KW, int SW>
static int launch_dwpw_v(bool vec, int px, dim3 grid, size_t lds, const DwPwK& p, hipStream_t s) {
  return vec ? launch_dwpw_px<KH, KW, SW, true>(px, grid, lds, p, s)
             : launch_dwpw_px<KH, KW, SW, false>(px, grid, lds, p, s);
}

// the 16-byte load path: left padding KW / 2 (the halo geometry assumes
// it), whole 16-byte chunks of image rows and of the weight arrays, 16-byte
// aligned tensors
static bool dwpw_vec(const DwPwArgs& a) {
  auto al = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
  return !a.stem && a.pw == a.kw / 2 && a.w % 4 == 0 && a.c % 4 == 0 && al(a.x) && al(a.wd) &&
         (!a.bd || al(a.bd)) && al(a.wk);
}

// the register-fed form: the 16-byte path with C = 16, 32, 64 or 128
static bool dwpw_reg_ok(const DwPwArgs& a) {
  return a.c == 16 || a.c == 32 || a.c == 64 || a.c == 128;
}

template <int KH, int KW, int SW, int NS>
static int launch_dwpw_reg_t(dim3 grid, const DwPwK& p, hipStream_t s) {
  if (p.act_d.kind == 3 && p.act_p.kind == 3)
    hipLaunchKernelGGL((dwpw_reg_kernel<KH, KW, SW, NS, 3>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((dwpw_reg_kernel<KH, KW, SW, NS, 0>), grid, dim3(256), 0, s, p);
  return launch_check("dwpw_reg_kernel");
}

template <int KH, int KW, int SW>
static int launch_dwpw_reg(int64_t c, dim3 grid, const DwPwK& p, hipStream_t s) {
  if (c == 16) return launch_dwpw_reg_t<KH, KW, SW, 4>(grid, p, s);
  if (c == 32) return launch_dwpw_reg_t<KH, KW, SW, 8>(grid, p, s);
  if (c == 64) return launch_dwpw_reg_t<KH, KW, SW, 16>(grid, p, s);
  return launch_dwpw_reg_t<KH, KW, SW, 32>(grid, p, s);
}

bool dwpw_stem_eligible(const DwPwArgs& a) {
  return a.stem && a.xin && a.wst && (a.c == 16 || a.c == 32) && a.kh == 3 && a.kw == 3 &&
         a.sh == 2 && a.sw == 2 && a.ph == 1 && a.pw == 1 && a.h == (a.hin - 1) / 2 + 1 &&
         a.w == (a.win - 1) / 2 + 1 && 3 * a.hin * a.win * 4 < (int64_t)0x80000000;
}

int launch_dwpw(const DwPwArgs& a, hipStream_t s) {
  if (!dwpw_eligible(a) || !a.wk) return fail(QPH_EUNSUPPORTED, "dw+pw block: unsupported shape");
  DwPwK p{};
  p.x = a.x; p.wd = a.wd; p.bd = a.bd;
  p.c = (int)a.c; p.h = (int)a.h; p.w = (int)a.w; p.sh = (int)a.sh; p.sw = (int)a.sw;
  p.ph = (int)a.ph; p.pw = (int)a.pw; p.oh = (int)a.oh; p.ow = (int)a.ow;
  p.act_d = a.act_d;
  p.wk = a.wk; p.bp = a.bp;
  p.m = (int)a.m; p.mpad = (int)((a.m + 31) / 32 * 32); p.cpad = (int)((a.c + 3) / 4 * 4);
  p.seed_rule = a.seed_rule;
  p.act_p = a.act_p;
  p.y = a.y; p.trans_out = a.trans_out;
  p.ct = halo_ct(a);
  p.ctr = (int)(15 * a.sw + a.kw);
  p.tiles_x = (int)ceil_div(a.ow, 16);
  p.slices = (int)ceil_div(a.m, DWPW_MSLICE);
  p.pcp = halo_pcp(a);
  p.halo = halo_floats(a);
  p.wrows = p.cpad * 64;
  p.wdl_pad = (int)((a.c * a.kh * a.kw + 63) / 64 * 64);
  size_t lds = (size_t)dwpw_lds_bytes(a, p.halo);
  const int64_t tiles = (int64_t)p.tiles_x * a.oh;
  if (tiles >= (1ll << 31)) return fail(QPH_EUNSUPPORTED, "dw+pw block: grid too large");
  dim3 grid((unsigned)tiles, (unsigned)p.slices, (unsigned)a.n);
  const int px = dw_px(p.cpad);
  if (a.stem) {
    if (!dwpw_stem_eligible(a)) return fail(QPH_EUNSUPPORTED, "stem + dw + pw block: unsupported shape");
    p.xin = a.xin; p.wst = a.wst; p.bst = a.bst; p.act_s = a.act_s;
    p.hin = (int)a.hin; p.win = (int)a.win;
    auto al16 = [](const void* q) { return ((uintptr_t)q & 15) == 0; };
    p.xvec = a.win % 4 == 0 && al16(a.xin) && al16(a.wst) && (!a.bst || al16(a.bst));
    if (p.cpad != 16 * px || p.slices != 1)
      return fail(QPH_EUNSUPPORTED, "stem + dw + pw block: unsupported shape");
    // the stem phase writes the halo with this row pitch as a constant
    if (p.ct != StemGeom<1>::CT || StemGeom<2>::CT != StemGeom<1>::CT)
      return fail(QPH_EUNSUPPORTED, "stem + dw + pw block: halo pitch");
    p.wrows = 0;   // pointwise weights in registers
    // LDS of the launch at R output rows a workgroup (t inside the input
    // region: cpad 16 R <= 1024 floats, below the region's 1428 / 2244)
    auto stem_lds = [&](int pcp, int in, int r) -> size_t {
      if (p.cpad * 16 * r > in) return SIZE_MAX;
      return (size_t)(p.c * pcp + p.wdl_pad + (p.c + 3) / 4 * 4 + in + ST_K * p.c + (p.c + 3) / 4 * 4) * 4;
    };
    const size_t lds1 = stem_lds(StemGeom<1>::PCP, StemGeom<1>::IN, 1);
    const size_t lds2 = stem_lds(StemGeom<2>::PCP, StemGeom<2>::IN, 2);
    if (lds1 > 160 * 1024 || lds2 > 160 * 1024)
      return fail(QPH_EUNSUPPORTED, "stem + dw + pw block: LDS");
    // two output rows a workgroup when one-row workgroups would not all be
    // resident at once (by LDS): the stem row the two rows share is
    // computed once and the launch has half the workgroups, so the rec
    // stem (1920 one-row workgroups of 27 KB) runs in one round instead of
    // two; the det stem (1600 of 17 KB) already fits and keeps one row
    int cus = 0;
    QPH_TRY(device_cus(nullptr, &cus));
    const int64_t wg1 = (int64_t)p.tiles_x * a.oh * a.n;
    const bool two = wg1 > (int64_t)(160 * 1024 / lds1) * cus;
    const int R = two ? 2 : 1;
    p.pcp = two ? StemGeom<2>::PCP : StemGeom<1>::PCP;
    p.halo = p.c * p.pcp;
    lds = two ? lds2 : lds1;
    grid.x = (unsigned)(p.tiles_x * ceil_div(a.oh, R));
    // cpad 16 -> 1 pixel per depthwise task, 32 -> 2
    if (two) {
      if (px == 2) return launch_dwpw_t<3, 3, 2, 2, true, false, 2>(grid, lds, p, s);
      return launch_dwpw_t<3, 3, 2, 1, true, false, 2>(grid, lds, p, s);
    }
    if (px == 2) return launch_dwpw_t<3, 3, 2, 2, true, false, 1>(grid, lds, p, s);
    return launch_dwpw_t<3, 3, 2, 1, true, false, 1>(grid, lds, p, s);
  }
  if (dwpw_vec(a) && dwpw_reg_ok(a)) {
    if (a.kh == 5) return launch_dwpw_reg<5, 5, 1>(a.c, grid, p, s);
    if (a.sw == 1) return launch_dwpw_reg<3, 3, 1>(a.c, grid, p, s);
    return launch_dwpw_reg<3, 3, 2>(a.c, grid, p, s);
  }
  // the 16-byte path's halo: whole chunks, channels contiguous
  const int vch = a.kh == 5 ? VecGeom<5, 5, 1>::CH : a.sw == 1 ? VecGeom<3, 3, 1>::CH
                                                              : VecGeom<3, 3, 2>::CH;
  const bool vec = dwpw_vec(a) && a.c * 4 * vch <= DWPW_MAX_HALO &&
                   dwpw_lds_bytes(a, a.c * 4 * vch) <= 160 * 1024;
  if (vec) {
    lds -= (size_t)p.halo * 4;
    p.halo = (int)a.c * 4 * vch;
    lds += (size_t)p.halo * 4;
  }
  if (a.kh == 5) return launch_dwpw_v<5, 5, 1>(vec, px, grid, lds, p, s);
  if (a.sw == 1) return launch_dwpw_v<3, 3, 1>(vec, px, grid, lds, p, s);
  return launch_dwpw_v<3, 3, 2>(vec, px, grid, lds, p, s);
}

}  // namespace qph
