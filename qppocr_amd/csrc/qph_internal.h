// Internal declarations shared by the qppocr HIP library's translation units.
//
// Numerics contract: every kernel reproduces the qppocr-kernels CPU operation
// sequence for each output element (same fma chains in the same k order,
// same separately-rounded multiplies/adds, same exp/erf polynomials), so the
// results are bit-identical to the CPU path.  All device code is compiled
// with -ffp-contract=off so that a*b+c is never fused unless written as fmaf,
// and with f32 denormals flushed, as the CPU executor runs with FTZ|DAZ
// (qppocr-kernels/src/par.rs:229-256).  fp32 MFMA on gfx950 accumulates each
// product in k order with one rounding per product, i.e. an MFMA k-chain is a
// chain of fmaf calls.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include <string>

#include "../../include/qppocr_hip.h"

namespace qph {

// ----------------------------------------------------------------- errors

void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
// Checks a HIP return code; on failure records the message and returns QPH_EHIP.
int hip_check(hipError_t e, const char* what);

#define QPH_TRY_HIP(expr)                                  \
  do {                                                     \
    int _rc = ::qph::hip_check((expr), #expr);             \
    if (_rc != QPH_OK) return _rc;                         \
  } while (0)

#define QPH_TRY(expr)               \
  do {                              \
    int _rc = (expr);               \
    if (_rc != QPH_OK) return _rc;  \
  } while (0)

// After a kernel launch: report launch-configuration errors.
int launch_check(const char* kernel);

}  // namespace qph

struct qph_ctx {
  int device;
  hipStream_t stream;
  bool own_stream;
  void* ws;         // scratch for standalone operator calls (repacked weights, masks)
  size_t ws_bytes;
  float* noalloc_wk;  // device address of this device's fixed repack array (qph_conv2d_noalloc)
};

namespace qph {

// Grows the context scratch to at least `bytes` (synchronises the stream
// before releasing a smaller buffer) and returns it.
int ctx_workspace(qph_ctx* ctx, size_t bytes, void** out);

// Activation kinds (qph_act.kind): 0 none, 1 gelu(c1,c2,c3), 2 relu,
// 3 hardswish(alpha=c1, beta=c2), 4 sigmoid, 5 hardsigmoid(alpha=c1, beta=c2),
// 6 clip(lo=c1, hi=c2), 7 the Add / Clip / Mul / Div hardswish (c1, c2, c3).

// exp1: qppocr-kernels/src/activation.rs:28-47 (x86.rs:28-57).
__device__ __forceinline__ float exp1(float x) {
  const float LN2_HI = 0.6931472f;
  const float LN2_LO = -2.9802322e-8f;
  const float INV_LN2 = 1.442695f;
  x = fminf(x, 88.0f);
  x = fmaxf(x, -88.0f);
  float kf = __builtin_rintf(x * INV_LN2);
  float r = __builtin_fmaf(-kf, LN2_HI, x);
  r = __builtin_fmaf(-kf, LN2_LO, r);
  float p = 1.0f / 720.0f;
  p = __builtin_fmaf(p, r, 1.0f / 120.0f);
  p = __builtin_fmaf(p, r, 1.0f / 24.0f);
  p = __builtin_fmaf(p, r, 1.0f / 6.0f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ki = (int)kf + 127;
  return __uint_as_float((unsigned)ki << 23) * p;
}

// erf1: qppocr-kernels/src/activation.rs:53-66 (A&S 7.1.26).
__device__ __forceinline__ float erf1(float x) {
  float ax = __uint_as_float(__float_as_uint(x) & 0x7fffffffu);
  float t = 1.0f / __builtin_fmaf(0.3275911f, ax, 1.0f);
  float p = 1.0614054f;
  p = __builtin_fmaf(p, t, -1.453152027f);
  p = __builtin_fmaf(p, t, 1.421413741f);
  p = __builtin_fmaf(p, t, -0.284496736f);
  p = __builtin_fmaf(p, t, 0.2548296f);
  p = p * t;
  float e = exp1(ax * (0.0f - ax));
  float r = __builtin_fmaf(-p, e, 1.0f);
  return __uint_as_float(__float_as_uint(r) | (__float_as_uint(x) & 0x80000000u));
}

// relu: activation.rs:232-239 (NaN -> 0).
__device__ __forceinline__ float relu1(float v) { return v > 0.0f ? v : 0.0f; }

// hardsigmoid: activation.rs:168-187.
__device__ __forceinline__ float hsig1(float x, float alpha, float beta) {
  float v = __builtin_fmaf(x, alpha, beta);
  return v < 0.0f ? 0.0f : (v > 1.0f ? 1.0f : v);
}

// clip: activation.rs:221-229, the comparison chain (NaN passes through).
__device__ __forceinline__ float clip1(float v, float lo, float hi) {
  const float m = v < lo ? lo : v;
  return hi < m ? hi : m;
}

// sigmoid: activation.rs:196-201 (true division).
__device__ __forceinline__ float sigmoid1(float x) { return 1.0f / (1.0f + exp1(-x)); }

// gelu: activation.rs:209-215, (c3*x) * (erf1(x*inv_c1) + c2).
__device__ __forceinline__ float gelu1(float v, float inv_c1, float c2, float c3) {
  return c3 * v * (erf1(v * inv_c1) + c2);
}

struct Act {
  int kind;
  float c1, c2, c3, inv_c1;
};

__device__ __forceinline__ float act_apply(float v, const Act& a) {
  switch (a.kind) {
    case 1: return gelu1(v, a.inv_c1, a.c2, a.c3);
    case 2: return relu1(v);
    case 3: return v * hsig1(v, a.c1, a.c2);  // HardSigmoid node then Mul node
    case 4: return sigmoid1(v);
    case 5: return hsig1(v, a.c1, a.c2);      // HardSigmoid node alone (the SE gate)
    case 6: return clip1(v, a.c1, a.c2);      // Clip node
    case 7: {                                 // Add(c1), Clip(0, c2), Mul(x), Div(c3) nodes
      const float t = clip1(v + a.c1, 0.0f, a.c2);
      return (v * t) / a.c3;
    }
    default: return v;
  }
}

inline Act make_act(const qph_act* a) {
  Act r;
  if (!a) {
    r.kind = 0; r.c1 = 1.0f; r.c2 = 0.0f; r.c3 = 0.0f;
  } else {
    r.kind = a->kind; r.c1 = a->c1; r.c2 = a->c2; r.c3 = a->c3;
  }
  r.inv_c1 = 1.0f / r.c1;  // host f32 division: same value as the reference's 1.0f32 / c1
  return r;
}

inline bool act_valid(const qph_act* a) { return !a || (a->kind >= 0 && a->kind <= 7); }

// The conv the reference runs as a plain GEMM over X[C][H*W] (conv.rs:264):
// 1x1, stride 1, one group; padding excluded (X is then not that matrix).
inline bool conv_is_pointwise(const int64_t ws[4], const qph_conv_params& p) {
  return p.group == 1 && ws[2] == 1 && ws[3] == 1 && p.sh == 1 && p.sw == 1 && p.ph == 0 &&
         p.pw == 0 && p.peh == 0 && p.pew == 0;
}

// -------------------------------------------------------- launch helpers

inline unsigned ceil_div(int64_t a, int64_t b) { return (unsigned)((a + b - 1) / b); }

// Internal launchers shared between the operator entry points and the
// session runner.  All pointers are device pointers; shapes were validated
// by the caller.

struct GemmArgs {
  const float* a; int64_t lda; int64_t a_batch;   // A[M][K], row stride lda
  const float* b; int64_t ldb; int64_t b_batch;   // B[K][N], row stride ldb
  float* c; int64_t ldc; int64_t c_batch;         // C[M][N] (or C^T when trans_out)
  int64_t m, n, k, batch;
  const float* bias; int bias_mode;               // 0 none, 1 per row (M), 2 per column (N)
  int seed_rule;                                  // reference bias placement: 0 panel, 1 m-rows
  Act act;
  const float* res; int64_t ldr; int64_t r_batch;  // residual, same layout as C
  int res_up;                                      // 0 same shape; 2 = nearest 2x of a coarse map
  int64_t up_w, up_cw;                             // output / coarse image width (res_up)
  int trans_out;                                   // store C^T: c[j*ldc + i]
  float* part;                                     // fused head: per-block argmax partials
  // real-batch early exit (plan path): batch items bz >= *rn * rn_per are
  // skipped when rn is set and *rn != 0 (the pointwise and skinny kernels)
  const unsigned* rn; int64_t rn_per;
};
int launch_gemm(const GemmArgs& g, hipStream_t s);
// The GEMM of a pointwise (1x1, stride 1, no padding, one group) conv of x
// [n][C][H][W] with w [M][C]: everything but residual, placement and store
// layout (plain rows), as conv_dispatch sets it up.
void pointwise_gemm_args(const float* x, const int64_t xs[4], const float* w,
                         const int64_t ws[4], const float* bias, const Act& a, float* y,
                         GemmArgs* out);
// Up to three pointwise GEMMs (no residual) that each take one-block
// pointwise tiles, as one launch (pw_group_eligible says which can).
bool pw_group_eligible(const GemmArgs& g);
int launch_pw_group(const GemmArgs* g, int n, hipStream_t s);
// FPN top-down on the level-3 maps: in4 = t4 + up2(in5), in3 = t3 + up2(in4)
// (nearest 2x, each Add rounded, as the laterals' residual epilogues do);
// per batch item c planes of h3 x w3 (in4 h3/2 x w3/2, in5 h3/4 x w3/4).
int launch_fpn_topdown(const float* t4, const float* in5, const float* t3, float* in4, float* in3,
                       int64_t n, int64_t c, int64_t h3, int64_t w3, hipStream_t s);
// The rec head with the softmax-argmax fused into the GEMM (pairs only):
// (max, first index, exp1 sum) per row and 64-column block into part
// (head_argmax_part_floats floats), then the pairs.  Values within ~1e-6
// of the unfused path's, not bit-identical (hardware exp2; the exp sum is
// taken per block and rescaled); indices are the first maximum of the logits.
bool head_argmax_eligible(int64_t m, int64_t n, int64_t k, int64_t lda, int64_t ldb);
int64_t head_argmax_part_floats(int64_t m, int64_t n);
int launch_head_argmax(const float* x, int64_t m, int64_t k, const float* w, int64_t ldb,
                       int64_t n, const float* bias, float* part, float* pairs, hipStream_t s);

// The session's linears: C[M][N] = act(A[M][K] * Wt[N][K]^T + bias) (+ res),
// Wt the weight held transposed (k contiguous).
struct LinArgs {
  const float* a; int64_t lda;
  const float* wt;
  float* c;
  int64_t m, n, k;
  const float* bias;          // per column, or NULL
  Act act;
  const float* res;           // [M][N], or NULL
  int bias_seed;              // 1: the bias starts each chain instead of following it
};
bool linear_nt_eligible(int64_t m, int64_t n, int64_t k, int64_t lda);
// the rec QKV linear (x [batch * t][k] . Wt[3 heads dh][k]^T + bias) and
// the attention after it in one launch; wt is the linear's resident
// transposed weight
bool qkv_attention_eligible(int64_t batch, int64_t t, int64_t heads, int64_t dh, int64_t k);
int launch_qkv_attention(const float* x, const float* wt, const float* bias, int64_t batch,
                         int64_t t, int64_t heads, int64_t dh, int64_t k, float scale, float* out,
                         hipStream_t s);
int launch_linear_nt(const LinArgs& g, hipStream_t s);
// true when launch_gemm takes the 128x128 persistent kernel for this shape
bool gemm_takes_wide(int64_t m, int64_t n, int64_t batch);
// wt[j][i] = w[i][j] for a [k][n] row-major w
int launch_transpose(const float* w, int64_t k, int64_t n, float* wt, hipStream_t s);

// 16-byte buffer->LDS load: lane L's four words land at dst + 4L.  (A plain
// function, so that only the device compile checks the builtin's size.)
__device__ __forceinline__ void lds_load16(__amdgpu_buffer_rsrc_t r, float* dst, unsigned voff,
                                           int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)dst, 16,
                                           voff, soff, 0, 0);
}

// s_waitcnt that waits until at most N vector-memory operations of this
// wave are outstanding (N < 64); the export and LDS/scalar counters are left
// at their maxima (no wait).  Encoding: vmcnt bits [3:0] and [15:14].
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (0xF << 8));
}

// Reference bias placement (gemm.rs:7-16): rule 0 (panel kernel): seeded
// when row is in the M%4 tail and the 32-column panel is partial; rule 1
// (m-rows kernel): seeded for columns j >= n - n%32.
__device__ __forceinline__ bool bias_seeded(int rule, int64_t i, int64_t j, int64_t m, int64_t n) {
  if (rule == 1) return j >= n - n % 32;
  int64_t n0 = (j >> 5) << 5;
  return (n - n0) < 32 && i >= m - m % 4;
}

struct ConvArgs {
  const float* x; int64_t n, c, h, w;
  const float* wt;     // ONNX layout [M][C/g][kh][kw]
  const float* wk;     // optional repacked k-major weights [Kpad][Mpad] (NULL: built per call)
  const float* bias;
  int64_t m, kh, kw, sh, sw, ph, pw, oh, ow, group;
  Act act;
  const float* res;    // residual, same layout as y
  float* y;            // y[N][M][oh][ow] when y_cstride == 0 (default NCHW)
  // optional strided placement of the output: channel slice of a larger
  // tensor (y_ctotal channels, offset y_coff) and nearest upsample by y_up.
  int64_t y_ctotal, y_coff, y_up;
};
// plan != NULL: a dense conv with resident weights is not launched; its
// arguments are returned in *plan (other conv kinds fail with EUNSUPPORTED).
// fixed_wk (fixed_floats long), when not NULL, takes the repacked weights of
// a standalone dense conv instead of the context scratch (nothing allocated).
int conv_dispatch(qph_ctx* ctx, const float* x, const int64_t xs[4], const float* w,
                  const float* wk_resident, const int64_t ws[4], const float* bias,
                  const qph_conv_params* p, const qph_act* act, const qph_conv_epilogue* ep,
                  float* y, ConvArgs* plan = nullptr, float* fixed_wk = nullptr,
                  int64_t fixed_floats = 0);
int launch_dense_conv(const ConvArgs& a, hipStream_t s, float* scratch_wk);
// Depthwise conv (+ bias + act) feeding a 1x1 conv (+ bias + act) in one
// kernel; wk = the 1x1 weights repacked k-major [ceil(C/4)*4][ceil(M/32)*32].
struct DwPwArgs {
  const float* x; int64_t n, c, h, w;
  const float* wd; const float* bd;
  int64_t kh, kw, sh, sw, ph, pw, oh, ow;
  Act act_d;
  const float* wk; const float* bp;
  int64_t m;
  int seed_rule;
  Act act_p;
  int trans_out;
  float* y;
  // stem in front (stem != 0): x is then the stem's output, never stored;
  // the kernel computes it from xin ([n][3][hin][win]) with the 3x3
  // stride-2 pad-1 conv wst ([c][3][3][3]) + bst, then act_s
  int stem;
  const float* xin; int64_t hin, win;
  const float* wst; const float* bst;
  Act act_s;
};
// Lets kernel fn take up to the whole 160 KB of a CU's LDS as dynamic
// shared memory; the attribute is set once per kernel and device.
int allow_full_lds(const void* fn);
// Compute units of the current device and the resident workgroups per CU of
// kernel fn at `block` threads (no dynamic LDS), each queried once per
// device (and kernel) and cached; safe to call from several host threads.
int device_cus(int* dev_out, int* cus);
int kernel_occupancy(const void* fn, int block, int* occ);
bool dwpw_eligible(const DwPwArgs& a);
// the stem conv that can run inside the dw + pw launch of a (3 -> a.c
// channels, 3x3, stride 2, pad 1, into a 3x3 stride-2 pad-1 depthwise)
bool dwpw_stem_eligible(const DwPwArgs& a);
int launch_dwpw(const DwPwArgs& a, hipStream_t s);
// 3x3 convs the direct kernel takes; up to four independent ones in one launch
bool direct3x3_eligible(const ConvArgs& a);
int launch_dense_conv_group(const ConvArgs* a, int n, hipStream_t s);
// A 3x3 conv to 24 channels with the det head's conv-transpose pair (w1
// [24][24][2][2], w2 [24][1][2][2]) and sigmoid in its epilogue: y [n][1][4
// oh][4 ow]; the conv output is never stored.  a as conv_dispatch plans it
// (resident weights).
bool conv3x3_convt_eligible(const ConvArgs& a);
int launch_conv3x3_convt(const ConvArgs& a, const float* w1, const float* w2, float* y,
                         hipStream_t s);
int launch_depthwise(const ConvArgs& a, hipStream_t s);
// depthwise conv with x and y channel-last ([n][h][w][c]); 3x3 and 5x5
int launch_depthwise_cl(const ConvArgs& a, hipStream_t s);
int64_t dense_conv_wk_floats(int64_t m, int64_t cg, int64_t kh, int64_t kw, int64_t group = 1);
// Per group, wk[Kpad][Mpad] k-major copy of that group's rows of an ONNX
// [M][cg][kh][kw] weight, Kpad = ceil(cg/4)*4*khkw, Mpad = ceil(M/g/32)*32,
// zero-filled past the real extent; groups follow each other.
int launch_repack_conv_w_taps(const float* wt, int64_t m, int64_t cg, int64_t khkw, float* wk,
                              hipStream_t s, int64_t group = 1);
// The implicit-GEMM launch checks of a dense (or grouped) conv, no launch.
int dense_conv_check(const ConvArgs& a);

int launch_convt2x2(const float* x, int64_t n, int64_t c, int64_t h, int64_t w, const float* wt,
                    int64_t m, float* y, hipStream_t s);
int launch_convt2x2_pair_sigmoid(const float* x, int64_t n, int64_t c, int64_t h, int64_t w,
                                 const float* w1, int64_t m1, const float* w2, float* y,
                                 hipStream_t s);
int launch_layernorm(const float* x, const float* gamma, const float* beta, float eps,
                     int64_t rows, int64_t cols, float* y, hipStream_t s);
int launch_softmax_rows(float* t, int64_t rows, int64_t cols, hipStream_t s);
int launch_softmax_argmax(const float* logits, int64_t rows, int64_t cols, int64_t ld,
                          float* probs, float* pairs, hipStream_t s);
int launch_argmax(const float* probs, int64_t rows, int64_t cols, float* pairs, hipStream_t s);
int launch_argmax_pitched(const float* probs, int64_t rows, int64_t cols, int64_t ld,
                          float* pairs, hipStream_t s);
// logits rows ld floats apart, probabilities rows ldo floats apart (either may be NULL)
// rn (plan path): rows >= *rn * rpb are skipped when *rn != 0
int launch_softmax_pitched(const float* logits, int64_t rows, int64_t cols, int64_t ld,
                           float* probs, int64_t ldo, float* pairs, hipStream_t s,
                           const unsigned* rn = nullptr, int64_t rpb = 0);
int launch_attention(const float* qkv, int64_t batch, int64_t t, int64_t heads, int64_t dh,
                     float scale, float* out, hipStream_t s);
int launch_attention_generic(const float* qkv, int64_t batch, int64_t t, int64_t heads,
                             int64_t dh, float scale, float* out, hipStream_t s);
int launch_elementwise_act(const float* x, float* y, int64_t n, const Act& a, hipStream_t s);
// y = x op b (mode 0, same element count), x op sv (mode 1) or sv op x
// (mode 2); op 0 add, 1 sub, 2 mul, 3 div
int launch_binary_out(const float* x, const float* b, float sv, float* y, int64_t n, int op,
                      int mode, hipStream_t s);
int launch_resize_nearest(const float* x, int64_t nc, int64_t h, int64_t w, int64_t oh,
                          int64_t ow, float* y, hipStream_t s);
int launch_binary(float* a, const float* b, int64_t rows, int64_t cols, int op, int bmode,
                  hipStream_t s);
int launch_mask_pairs(float* pairs, int64_t batch, int64_t t, const int32_t* t_valid,
                      hipStream_t s);
// reduce_mean over the last axis (also GlobalAveragePool: rows = N*C planes)
int launch_reduce_mean(const float* x, int64_t rows, int64_t cols, float* out, hipStream_t s);
// row r's element j at x[(r / rpg) * gstride + (r % rpg) * rstride + j * estride],
// its mean to out[r * ostride] (ostride 4: the row's other three words set to 0)
// rn (plan path): rows >= *rn * rpb are skipped when *rn != 0
int launch_reduce_mean_rows(const float* x, int64_t rows, int64_t cols, int64_t rpg,
                            int64_t gstride, int64_t rstride, int64_t estride, float* out,
                            int64_t ostride, hipStream_t s, const unsigned* rn = nullptr,
                            int64_t rpb = 0);

// qph_aux.hip.  ctot / coff: the output is channels [coff, coff + c) of a
// tensor with ctot channels (ctot = c, coff = 0 for a plain output).
int launch_mul_add_scale(const float* f, const float* gate, const float* r, float* out, int64_t c,
                         int64_t gmod, int64_t hw, int64_t planes, int64_t ctot, int64_t coff,
                         hipStream_t s);
void pool2d_out_hw(int64_t h, int64_t w, int64_t kh, int64_t kw, int64_t sh, int64_t sw,
                   int64_t ph, int64_t pw, int64_t peh, int64_t pew, int64_t* oh, int64_t* ow);
int launch_pool2d(const float* x, int64_t n, int64_t c, int64_t h, int64_t w, int64_t kh,
                  int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t peh,
                  int64_t pew, int max_pool, float* y, int64_t ctot, int64_t coff, hipStream_t s);
int launch_resize_bilinear(const float* x, int64_t n, int64_t c, int64_t h, int64_t w,
                           int64_t oh, int64_t ow, int align, float* y, int64_t ctot,
                           int64_t coff, hipStream_t s);
int launch_transpose4(const float* x, const int64_t xs[4], const int32_t perm[4], float* y,
                      hipStream_t s);
int launch_copy_slot(const float* x, float* y, int64_t c, int64_t hw, int64_t planes,
                     int64_t ctot, int64_t coff, hipStream_t s);
int launch_det_normalize(const uint8_t* rgb, int64_t h, int64_t w, float* out, hipStream_t s);
int launch_resize_rgb_u8(const uint8_t* src, int64_t sw, int64_t sh, uint8_t* dst, int64_t dw,
                         int64_t dh, hipStream_t s);
int launch_pack_crop(const uint8_t* crop, int64_t ch, int64_t cw, int64_t img_h, int64_t img_w,
                     float* dst, int pad_only, hipStream_t s);
int launch_db_mask(const float* pred, int64_t h, int64_t w, float thresh, int dilate,
                   uint8_t* out, hipStream_t s);

}  // namespace qph
