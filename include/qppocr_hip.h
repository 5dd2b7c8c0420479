/*
 * qppocr_hip.h -- C ABI of the MI355X (gfx950) HIP backend for the
 * qppocr-kernels operator set and the det/rec session built on it.
 *
 * Plain C99 types only.  Every call returns an int status: QPH_OK (0) or a
 * negative code; qph_last_error() returns the message of the calling
 * thread's last failure.  Nothing aborts or throws across this boundary.
 * Tensor pointers are device pointers unless a name says _host.  Layouts are
 * the reference's: contiguous row-major NCHW activations, ONNX weight layouts.
 * A context owns one HIP stream; every operator call is enqueued on it
 * (asynchronous with respect to the host; qph_sync waits).
 *
 * Numerics: outputs are bit-identical to the qppocr-kernels CPU path for the
 * same inputs (same fma chains in the same order, same polynomial exp/erf).
 */
#ifndef QPPOCR_HIP_H
#define QPPOCR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define QPH_API __attribute__((visibility("default")))
#else
#define QPH_API
#endif

/* status codes (mirror qppocr-core/src/error.rs:343-353: Graph / Device errors) */
#define QPH_OK 0
#define QPH_EINVAL -1        /* bad shape / argument (Error::Graph) */
#define QPH_EHIP -2          /* HIP runtime failure (Error::Device) */
#define QPH_EUNSUPPORTED -3  /* operator form the backend does not implement */
#define QPH_ENOMEM -4

/* ------------------------------------------------------------- context */

typedef struct qph_ctx qph_ctx;

/* Device context + stream: the DeviceContext analogue
 * (qppocr-core/src/device.rs:83-101).  device = HIP device ordinal. */
QPH_API int qph_ctx_create(int device, qph_ctx** out);
QPH_API int qph_ctx_destroy(qph_ctx* ctx);
/* Use an external HIP stream (e.g. a framework's current stream) instead of
 * the context's own; NULL restores the context's stream. */
QPH_API int qph_ctx_set_stream(qph_ctx* ctx, void* hip_stream);
QPH_API void* qph_ctx_stream(qph_ctx* ctx);
/* Bytes of device scratch the context has allocated for standalone operator
 * calls (it grows on demand with hipMalloc; 0 until a call needs it).  No
 * counterpart in the reference; for tests of the allocation-free entry
 * point and for memory accounting. */
QPH_API int qph_ctx_scratch_bytes(qph_ctx* ctx, size_t* bytes);
QPH_API int qph_sync(qph_ctx* ctx);
/* Thread-local message of the last failed call (empty string if none). */
QPH_API const char* qph_last_error(void);
QPH_API const char* qph_version(void);

/* device memory (the library never frees caller memory) */
QPH_API int qph_malloc(qph_ctx* ctx, void** ptr, size_t bytes);
QPH_API int qph_free(qph_ctx* ctx, void* ptr);
QPH_API int qph_memcpy_h2d(qph_ctx* ctx, void* dst, const void* src_host, size_t bytes);
QPH_API int qph_memcpy_d2h(qph_ctx* ctx, void* dst_host, const void* src, size_t bytes);
/* Fills bytes with (value & 0xff), asynchronously on the context stream, by a
 * kernel (never hipMemsetAsync), so it may be recorded into a captured
 * graph. */
QPH_API int qph_memset(qph_ctx* ctx, void* dst, int value, size_t bytes);

/* ------------------------------------------------------------ operators */

/* ConvParams (qppocr-kernels/src/conv.rs:124-143). */
typedef struct {
  int64_t sh, sw;   /* stride */
  int64_t ph, pw;   /* begin padding */
  int64_t peh, pew; /* end padding */
  int64_t dh, dw;   /* dilation (must be 1, conv.rs:149) */
  int64_t group;
} qph_conv_params;

/* Activation folded into a producer: superset of
 * qppocr-kernels/src/activation.rs:75-95 (None | Gelu(c1,c2,c3) | Relu) plus
 * the HardSigmoid+Mul pair (hardswish, alpha=c1 beta=c2; executor.rs:746-758)
 * and Sigmoid (executor.rs:737-745), each with the standalone op's arithmetic. */
#define QPH_ACT_NONE 0
#define QPH_ACT_GELU 1
#define QPH_ACT_RELU 2
#define QPH_ACT_HARDSWISH 3
#define QPH_ACT_SIGMOID 4
#define QPH_ACT_HARDSIGMOID 5  /* HardSigmoid node alone (alpha = c1, beta = c2): the SE gate */
/* Clip node (executor.rs:779-807, activation.rs:221-229): m = x < c1 ? c1 : x,
 * then c2 < m ? c2 : m (lo = c1, hi = c2; NaN passes through). */
#define QPH_ACT_CLIP 6
/* The Add / Clip / Mul / Div export form of hardswish, each node rounding
 * to f32 as the reference's separate nodes do (elementwise.rs:350-363 for
 * the scalar Add and Div): t = x + c1, t = clip(t, +0.0, c2), t = x * t,
 * y = t / c3. */
#define QPH_ACT_HARDSWISH_CLIP 7
typedef struct {
  int32_t kind;
  float c1, c2, c3;
} qph_act;

/* conv2d_out_shape (qppocr-kernels/src/conv.rs:146-156). */
QPH_API int qph_conv2d_out_shape(const int64_t xs[4], const int64_t ws[4],
                                 const qph_conv_params* p, int64_t ys[4]);

/* conv2d_res_into (qppocr-kernels/src/conv.rs:222-715): y = act(conv(x, w) +
 * bias) (+ residual).  Dispatch as the reference: 1x1 s1 g1 -> GEMM,
 * depthwise (g > 1, C/g == 1) -> direct, else implicit GEMM.  bias,
 * residual and act may be NULL.  ys_out (may be NULL) receives the shape. */
QPH_API int qph_conv2d(qph_ctx* ctx, const float* x, const int64_t xs[4], const float* w,
                       const int64_t ws[4], const float* bias, const qph_conv_params* p,
                       const qph_act* act, const float* residual, float* y, int64_t ys_out[4]);

/* Allocation-free qph_conv2d (same arguments, same results).  No counterpart
 * in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  qph_conv2d repacks a dense conv's weights into the context's
 * scratch, which it grows with hipMalloc; this form repacks them into a fixed
 * device array of QPH_NOALLOC_WK_FLOATS floats (4 MiB per GPU, held until
 * the process ends) and refuses (QPH_EUNSUPPORTED) a conv whose repacked
 * weights need more: group * ceil(C/g/4)*4*kh*kw * ceil(M/g/32)*32 floats.
 * Every call on one GPU uses that GPU's one array: calls that overlap on a
 * GPU (from several streams or threads) race; calls on one stream are
 * ordered.  1x1 and depthwise convs use no scratch either way. */
#define QPH_NOALLOC_WK_FLOATS 1048576
QPH_API int qph_conv2d_noalloc(qph_ctx* ctx, const float* x, const int64_t xs[4],
                               const float* w, const int64_t ws[4], const float* bias,
                               const qph_conv_params* p, const qph_act* act,
                               const float* residual, float* y, int64_t ys_out[4]);

/* Epilogue placement for the fused det neck (no reference counterpart as one
 * call; it is the reference's Conv -> Resize(nearest) -> Add / Concat node
 * sequence, qppocr-core/src/executor.rs:433-652, 885-951, 1889-1916, with
 * identical per-element arithmetic):
 *   res_up   residual is a coarse map at half resolution, added via nearest
 *            2x upsample (resize.rs:26-57 with oh = 2h); 0 = same shape.
 *   y_ctotal/y_coff  write into channels [y_coff, y_coff+M) of a tensor with
 *            y_ctotal channels (Concat along C); 0/0 = plain output.
 *   y_up     replicate each output pixel y_up x y_up times (nearest upsample
 *            of the result by an integer factor); 1 = none.
 *   trans_out (1x1 only) store the output as [N][oh*ow][M] (the rec
 *            backbone's [B,C,1,T] -> [B,T,C] reshape/transpose). */
typedef struct {
  const float* residual;
  int32_t res_up;
  int64_t y_ctotal, y_coff, y_up;
  int32_t trans_out;
} qph_conv_epilogue;
QPH_API int qph_conv2d_ex(qph_ctx* ctx, const float* x, const int64_t xs[4], const float* w,
                          const int64_t ws[4], const float* bias, const qph_conv_params* p,
                          const qph_act* act, const qph_conv_epilogue* ep, float* y);

/* convtranspose2d, 2x2 s2 p0 only, no bias (qppocr-kernels/src/conv.rs:730-804).
 * w: ONNX [Ci, Co, 2, 2]. */
QPH_API int qph_convtranspose2d(qph_ctx* ctx, const float* x, const int64_t xs[4],
                                const float* w, const int64_t ws[4], int64_t sh, int64_t sw,
                                int64_t ph, int64_t pw, float* y, int64_t ys_out[4]);
/* Two chained 2x2 s2 ConvTranspose nodes then Sigmoid in one pass (the det
 * head tail: executor.rs:654-687 twice, then executor.rs:737-745).
 * w1 [C, M1, 2, 2], w2 [M1, 1, 2, 2]; y [N, 1, 4H, 4W]. */
QPH_API int qph_convt2x2_pair_sigmoid(qph_ctx* ctx, const float* x, const int64_t xs[4],
                                      const float* w1, const int64_t w1s[4], const float* w2,
                                      const int64_t w2s[4], float* y);

/* sgemm / sgemm_res (qppocr-kernels/src/gemm.rs:37-70): C[M,N] (row stride
 * ldc) = A[M,K] B[K,N], bias per row placed as the reference does, then act,
 * then += residual (C's layout).  serial selects the reference's serial panel
 * path (sgemm_serial*, gemm.rs:138-168) for the bias-placement rule. */
QPH_API int qph_sgemm(qph_ctx* ctx, const float* a, const float* b, float* c, int64_t m,
                      int64_t n, int64_t k, int64_t ldc, const float* bias, const qph_act* act,
                      const float* residual, int32_t serial);

/* MatMul (qppocr-kernels/src/shape.rs:568-698) for a [batch, M, K] x b
 * [K, N] (b_shared = 1) or b [batch, K, N]; no bias. */
QPH_API int qph_matmul(qph_ctx* ctx, const float* a, const float* b, float* out, int64_t batch,
                       int64_t m, int64_t k, int64_t n, int32_t b_shared);

/* The rec linear: MatMul x[R,K] . w[K,N] then Add(bias[N]) then act then
 * Add(residual[R,N]) (executor.rs:1559-1580 MatMul, 885-951 Add,
 * 759-768 FusedGelu) in one kernel. */
QPH_API int qph_linear(qph_ctx* ctx, const float* x, const float* w, const float* bias,
                       int64_t rows, int64_t k, int64_t n, const qph_act* act,
                       const float* residual, float* y);

/* LayerNorm as the exported ReduceMean/Sub/Pow/ReduceMean/Add/Sqrt/Div/Mul/Add
 * chain over the last axis (shape.rs:510-560 f64 means, elementwise.rs). */
QPH_API int qph_layernorm(qph_ctx* ctx, const float* x, const float* gamma, const float* beta,
                          float eps, int64_t rows, int64_t cols, float* y);

/* softmax_last_dim in place (qppocr-kernels/src/activation.rs:321-403). */
QPH_API int qph_softmax_last_dim(qph_ctx* ctx, float* t, int64_t rows, int64_t inner);

/* Row softmax then per-row argmax, the rec head's Softmax node followed by
 * the CTC argmax (activation.rs:321-403; qppocr-core/src/pipeline/rec.rs:34-90).
 * probs may be NULL (pairs only); pairs[2r] = max prob, pairs[2r+1] = index
 * as u32 bits stored in an f32 slot (device.rs:160-165). */
QPH_API int qph_softmax_argmax(qph_ctx* ctx, const float* logits, int64_t rows, int64_t cols,
                               float* probs, float* pairs);

/* The rec head MatMul + Add(bias) + Softmax + CTC argmax in one GEMM whose
 * epilogue keeps, per row and 64-column block, the logits' max, the first
 * column holding it and the sum of exp1(v - max); a second kernel combines
 * the blocks into pairs[2r] = 1 / sum (the max's probability) and
 * pairs[2r+1] = index as u32 bits.  The logits never reach memory (no single
 * reference kernel does this; the reference's Metal n_head_argmax,
 * qppocr-gpu/src/plan.rs:316-340, fuses only Softmax + argmax).  x [rows, k],
 * w [k, n] (ONNX MatMul layout), bias [n] or NULL.  Not bit-identical to
 * qph_linear + qph_softmax_argmax: the exponentials come from the hardware
 * exp2 and the sum is taken per block and rescaled, so values agree to
 * ~1e-6 relative (the tolerance of the pairs is 1e-4); the index is
 * the first maximum of the logits, which differs from the first maximum of
 * the rounded probabilities only where two logits lie within a few ulps.
 * Needs k % 16 == 0 and x 16-byte aligned with rows k floats apart. */
QPH_API int qph_linear_softmax_argmax(qph_ctx* ctx, const float* x, const float* w,
                                      const float* bias, int64_t rows, int64_t k, int64_t n,
                                      float* pairs);

/* CTC greedy argmax over probabilities (rec.rs:46-54): first strict max,
 * ties to the lowest index.  t_valid (may be NULL) masks steps t >= t_valid[b]
 * of batch item b (rows = batch * t_len) to (0, blank). */
QPH_API int qph_ctc_argmax(qph_ctx* ctx, const float* probs, int64_t batch, int64_t t_len,
                           int64_t cols, const int32_t* t_valid_host, float* pairs);

/* Multi-head self-attention core of the rec encoder on a packed qkv
 * [B, T, 3, heads, dh] (the QKV MatMul output): q*scale, q.k^T, Softmax,
 * .v, transposed back to [B, T, heads*dh] (shape.rs:664-697 small matmul
 * path, activation.rs:321-403). */
QPH_API int qph_attention(qph_ctx* ctx, const float* qkv, int64_t batch, int64_t t,
                          int64_t heads, int64_t dh, float scale, float* out);

/* Standalone activations (activation.rs:232-276; executor.rs:732-768). */
QPH_API int qph_activation(qph_ctx* ctx, const float* x, float* y, int64_t n,
                           const qph_act* act);
/* HardSigmoid(alpha, beta) node (activation.rs:243-251). */
QPH_API int qph_hardsigmoid(qph_ctx* ctx, const float* x, float* y, int64_t n, float alpha,
                            float beta);
/* resize_nearest (qppocr-kernels/src/resize.rs:8-57). */
QPH_API int qph_resize_nearest(qph_ctx* ctx, const float* x, int64_t nc, int64_t h, int64_t w,
                               int64_t oh, int64_t ow, float* y);
/* Broadcast binary op in place on a[rows, cols] (elementwise.rs:185-298):
 * op 0 add, 1 sub, 2 mul, 3 div; bmode 0 = b[rows] (per row), 1 = b[cols]
 * (per column), 2 = scalar b[0], 3 = same shape. */
QPH_API int qph_binary_inplace(qph_ctx* ctx, float* a, const float* b, int64_t rows,
                               int64_t cols, int32_t op, int32_t bmode);
/* reduce_mean over the last axis (shape.rs:510-560, f64 accumulation). */
QPH_API int qph_reduce_mean_last(qph_ctx* ctx, const float* x, int64_t rows, int64_t cols,
                                 float* out);

/* ------------------------------------ pooling, SE gate, resize, layout */

/* global_avg_pool (qppocr-kernels/src/pool2d.rs:10-29): x [N, C, H, W] ->
 * out [N, C] (f64 sum per plane in order, (sum / (H*W)) as f32). */
QPH_API int qph_global_avg_pool(qph_ctx* ctx, const float* x, int64_t n, int64_t c,
                                int64_t hw, float* out);
/* mul_add_scale (elementwise.rs:134-179), the SE block's gated residual
 * Add(Mul(feature, gate), residual) as fused by optimize.rs:429-497:
 * out = feature * gate[channel] + residual, each op rounded; feature,
 * residual and out [N, C, hw]. */
QPH_API int qph_mul_add_scale(qph_ctx* ctx, const float* feature, const float* gate,
                              const float* residual, int64_t n, int64_t c, int64_t hw,
                              float* out);
/* pool2d (pool2d.rs:51-236): max (max_pool = 1) or average (padding counted
 * in the divisor) over kh x kw windows; pads ph/pw begin, peh/pew end.
 * ys_out (may be NULL) receives [N, C, oh, ow], oh = (H + ph + peh - kh) /
 * sh + 1. */
QPH_API int qph_pool2d(qph_ctx* ctx, const float* x, const int64_t xs[4], int64_t kh,
                       int64_t kw, int64_t sh, int64_t sw, int64_t ph, int64_t pw, int64_t peh,
                       int64_t pew, int32_t max_pool, float* y, int64_t ys_out[4]);
/* resize_bilinear (resize.rs:60-142) over the last two axes of [nc, h, w]. */
QPH_API int qph_resize_bilinear(qph_ctx* ctx, const float* x, int64_t nc, int64_t h, int64_t w,
                                int64_t oh, int64_t ow, int32_t align_corners, float* y);
/* Rank-4 Transpose: y's dimension d is x's dimension perm[d]. */
QPH_API int qph_transpose(qph_ctx* ctx, const float* x, const int64_t xs[4],
                          const int32_t perm[4], float* y);

/* ------------------------------------ steps either side of the networks */

/* det input (qppocr-core/src/pipeline/engine.rs:959-982): u8 RGB
 * [h, w, 3] -> f32 [1, 3, h, w], v = u8 * (1/255), (v - 0.5) * (1/0.5). */
QPH_API int qph_det_normalize_u8(qph_ctx* ctx, const uint8_t* rgb, int64_t h, int64_t w,
                                 float* out);
/* resize_bilinear_rgb_u8 (resize.rs:153-209): u8 RGB [sh, sw, 3] ->
 * [dh, dw, 3]. */
QPH_API int qph_resize_bilinear_rgb_u8(qph_ctx* ctx, const uint8_t* src, int64_t sw, int64_t sh,
                                       uint8_t* dst, int64_t dw, int64_t dh);
/* pack_crop (qppocr-core/src/pipeline/crop.rs:153-190): a u8 RGB crop
 * [ch, cw, 3] into one f32 [3, img_h, img_w] slot of a rec batch (resized
 * to img_h x clamp(ceil(img_h * cw / ch), 1, img_w), or centred at its own
 * size when pad_only), (u8 / 255 - 0.5) / 0.5; the rest of the slot is 0. */
QPH_API int qph_pack_crop(qph_ctx* ctx, const uint8_t* crop, int64_t ch, int64_t cw,
                          int64_t img_h, int64_t img_w, int32_t pad_only, float* dst);
/* A whole rec batch: crops[i] (device u8 RGB [ch[i], cw[i], 3]) into slot i
 * of dst [n, 3, img_h, img_w] exactly as qph_pack_crop with pad_only[i]; one
 * launch per 64 lines, the line descriptors in the kernel arguments.  The
 * arrays are host memory, the crops and dst device memory.  Replaces the
 * per-line pack loop that fills a rec batch
 * (qppocr-core/src/pipeline/engine.rs:1413-1431). */
QPH_API int qph_pack_crops(qph_ctx* ctx, int32_t n, const uint8_t* const* crops,
                           const int64_t* ch, const int64_t* cw, const int32_t* pad_only,
                           int64_t img_h, int64_t img_w, float* dst);
/* DB post front end (geometry.rs:287-301, resize.rs:219-247): mask =
 * pred > thresh (u8 0/1), then (dilate != 0) the 2x2 dilation with anchor
 * (1, 1), out-of-range samples ignored. */
QPH_API int qph_db_mask(qph_ctx* ctx, const float* pred, int64_t h, int64_t w, float thresh,
                        int32_t dilate, uint8_t* mask);

/* ------------------------------------------------------------- session */

/* A static det or rec graph (the optimised graph the DeviceContext receives,
 * qppocr-core/src/device.rs:83-101) as a node list over numbered tensors.
 * Tensor 0 is the graph input; the node list is topologically ordered. */
#define QPH_OP_CONV 1          /* x -> y; w, bias; qph_conv_params; act; epilogue fields */
#define QPH_OP_CONVT_PAIR_SIG 2 /* x -> y; w (first ConvT), w2 (second ConvT); then sigmoid */
#define QPH_OP_LINEAR 3        /* x [R,K] -> y [R,N]; w [K,N]; bias [N]; act; residual tensor */
#define QPH_OP_LAYERNORM 4     /* x -> y; w = gamma, bias = beta; eps */
#define QPH_OP_ATTENTION 5     /* qkv -> y; heads, dh, scale */
#define QPH_OP_SOFTMAX_ARGMAX 6 /* logits -> probs (y, optional) and pairs (y2) */
#define QPH_OP_CONVT 7         /* x -> y; w [Ci, Co, 2, 2] */
#define QPH_OP_ACT 8           /* x -> y; act */
#define QPH_OP_GAP 9           /* GlobalAveragePool: x [N,C,H,W] -> y [N,C,1,1] */
#define QPH_OP_MUL_ADD_SCALE 10 /* y = in * in3 (gate [C] or [N,C]) + in2 (in2 = -1: the
                                  gate Mul alone); y_ctotal/y_coff */
#define QPH_OP_POOL 11         /* ws = {max?, 0, kh, kw}; cp strides and pads; y_ctotal/y_coff */
#define QPH_OP_RESIZE 12       /* ws = {mode 0 nearest | 1 bilinear, align_corners, 0, 0};
                                  output size from the tensor table; y_ctotal/y_coff (bilinear) */
#define QPH_OP_TRANSPOSE 13    /* rank-4 permutation ws = {perm0..3} */
#define QPH_OP_COPY_SLOT 14    /* x -> channels [y_coff, y_coff + C) of y (a Concat slot) */
#define QPH_OP_BINARY 15       /* y = x op in2 (same element count), or with in2 = -1 the
                                  one-element broadcast: y = x op scale (ws[1] = 0) or
                                  y = scale op x (ws[1] = 1); ws[0] = op: 0 Add, 1 Sub,
                                  2 Mul, 3 Div (elementwise.rs:185-298, 350-363) */

typedef struct {
  int32_t op;
  int32_t in;       /* input tensor id */
  int32_t in2;      /* residual / second input tensor id, -1 if none */
  int32_t out;      /* output tensor id */
  int32_t out2;     /* second output tensor id (pairs), -1 if none */
  int32_t w, bias, w2;  /* weight indices, -1 if none */
  int64_t ws[4];    /* weight shape of w */
  int64_t w2s[4];   /* weight shape of w2 */
  qph_conv_params cp;
  qph_act act;
  int32_t res_up;
  int32_t trans_out;
  int64_t y_ctotal, y_coff, y_up;
  int64_t heads, dh;
  float eps, scale;
  int32_t in3;      /* third input tensor id (the MulAddScale gate), -1 if none */
} qph_node;

/* Tensor table: shape per tensor id (rank 4, unused trailing dims = 1).
 * alias[i] >= 0 makes tensor i share tensor alias[i]'s storage (Concat
 * slots written through y_ctotal/y_coff). */
typedef struct {
  int32_t n_tensors;
  const int64_t* shapes;  /* n_tensors * 4 */
  const int32_t* alias;   /* n_tensors, -1 = own storage */
  int32_t n_nodes;
  const qph_node* nodes;
  int32_t n_weights;
  const int64_t* weight_sizes;  /* floats per weight */
  int32_t n_outputs;
  const int32_t* outputs;       /* graph output tensor ids */
  int32_t flags;                /* QPH_NET_* */
} qph_net_spec;

/* Every node its own launch: no shared launch of independent 3x3 convs, no
 * depthwise + 1x1 (+ stem) fusion, no QKV linear + attention launch, no
 * channel-last rec blocks (per-op measurement and debugging; the results
 * are the same bits). */
#define QPH_NET_SEPARATE_LAUNCHES 1
/* A linear whose output only the pairs-only softmax argmax right after it
 * reads (the rec head) runs as one GEMM with the softmax argmax in its
 * epilogue; the logits are never stored (qph_linear_softmax_argmax).  Pairs
 * within float rounding of the unfused path, not bit-identical. */
#define QPH_NET_FUSED_HEAD 2

typedef struct qph_net qph_net;

/* create_session (device.rs:88-101): validates every node (unsupported ->
 * QPH_EUNSUPPORTED naming the node), copies the weights to device memory
 * owned by the net, plans the fusions and the activation arena, and
 * captures the kernel sequence into a HIP graph, so that a graph the
 * kernels cannot run fails here rather than at the first run. */
QPH_API int qph_net_create(qph_ctx* ctx, const qph_net_spec* spec,
                           const float* const* weights_host, qph_net** out);
QPH_API int qph_net_destroy(qph_net* net);
/* DeviceSession::run (device.rs:130): input from the host (or device when
 * input_is_device; NULL keeps the input tensor as it is), the net's HIP
 * graph replayed, outputs copied to the host buffers (sizes from the
 * tensor table) unless outputs_host is NULL. */
QPH_API int qph_net_run(qph_net* net, const float* input, int32_t input_is_device,
                        float* const* outputs_host);
/* Deferred runs (DeviceSession::run_deferred + DeferredRun::complete,
 * device.rs:105-110, 166-176): batch k+1 is packed and submitted while batch
 * k runs.  qph_net_staging returns the net's pinned host buffer (allocated
 * on first use with hipHostMalloc, owned by the net) for the input
 * (slot -1) or output `slot`; a caller that writes its input there and
 * reads its outputs from there needs no pageable copies.
 * qph_net_run_async enqueues, on the context stream: the input upload from
 * its staging buffer (flags & QPH_RUN_UPLOAD; otherwise the input tensor is
 * used as it is), the graph, and the output downloads into their staging
 * buffers (flags & QPH_RUN_DOWNLOAD), then returns.  qph_net_complete waits
 * for all of it.  As in the reference, one net has one run in flight: a
 * second qph_net_run_async before qph_net_complete is refused (the buffers
 * are shared); qph_net_run completes a pending run first. */
#define QPH_RUN_UPLOAD 1
#define QPH_RUN_DOWNLOAD 2
/* Real batch count (the plan model's params[0] slot, qppocr-gpu/src/plan.rs:
 * 587-593, which the GPU sessions write before a run padded to
 * DeviceSession::batch_grain, qppocr-core/src/device.rs:139-157): the runs
 * that follow compute batch items 0 .. real_n - 1 only, 1 <= real_n <= the
 * input's batch dimension.  Every kernel of such a run is launched over the
 * real items alone (a HIP graph per distinct count, captured by this call
 * the first time the count is set), the input upload and the output
 * downloads of qph_net_run / qph_net_run_async move real_n items, and
 * batch items past real_n keep stale contents.  Requires every tensor
 * derived from the input to keep the batch as its first dimension
 * (QPH_EUNSUPPORTED otherwise); refused while a deferred run is in flight.
 * qph_net_real_n reads the current count and the batch dimension. */
QPH_API int qph_net_set_real_n(qph_net* net, int32_t real_n);
QPH_API int qph_net_real_n(qph_net* net, int32_t* real_n, int32_t* batch);
QPH_API int qph_net_staging(qph_net* net, int32_t slot, float** host, int64_t* numel);
QPH_API int qph_net_run_async(qph_net* net, int32_t flags);
QPH_API int qph_net_complete(qph_net* net);
/* Device pointer of a tensor of the net (valid until destroy).  Tensors that
 * a fused launch consumes inside itself are never written: a depthwise
 * output inside a depthwise + 1x1 block and a stem output inside the first
 * block keep stale arena storage; the QKV output of a linear + attention
 * launch and a fused head's logits have none, and asking for them returns
 * QPH_EINVAL. */
QPH_API int qph_net_tensor(qph_net* net, int32_t id, float** dev_ptr, int64_t* numel);
/* Average device time (ms) of each node over the runs since the last reset
 * when profiling is on (events around each node; graph replay disabled).
 * A launch that covers several nodes (a depthwise + 1x1 block, a stem conv
 * run inside the first block, a group of independent 3x3 convs, a QKV
 * linear + attention) is booked on its first node; the nodes it covers
 * read only the event overhead. */
QPH_API int qph_net_set_profiling(qph_net* net, int32_t on);
QPH_API int qph_net_node_times(qph_net* net, double* ms_per_node, int32_t n);

/* The launch sequence of a run, for profilers matching kernel traces to
 * nodes: launch j covers nodes first[j] .. first[j] + nodes[j] - 1 and
 * issues kernels[j] kernels (the fused rec head: 2; every other launch: 1).
 * Fills at most cap entries of each non-NULL array and stores the number of
 * launches in *n_launches.  No counterpart in the reference (whose executor
 * runs node by node); for profiling tools. */
QPH_API int qph_net_plan(qph_net* net, int32_t* first, int32_t* nodes, int32_t* kernels,
                         int32_t cap, int32_t* n_launches);

/* ------------------------------------------------------------------------
 * Sessions over the reference's plan model (qppocr-gpu/src/plan.rs): the
 * GraphPlan a PlanBuilder produces for one input shape (plan.rs:100-156) is
 * handed over as plain arrays and run by the HIP kernel set of the Vulkan
 * backend's dispatch contracts (vulkan/pipeline.rs:84-136, the shaders
 * qppocr-gpu/shaders/n_*.comp).  The arena holds u32 words: activations NHWC
 * with channels padded to a multiple of 4, parameter blocks, weights
 * repacked by nhwc.rs; word 0 is the real batch count (plan.rs:587-593).
 * Each dispatch computes the CPU operation it stands for in the CPU's
 * operation order, so outputs are bit-identical to the CPU executor running
 * the same node sequence (the conv bias rule assumes channel counts that
 * are multiples of 4; a parameter block carries only the padded ones).
 * ---------------------------------------------------------------------- */

/* One static segment (GraphPlan.uploads and .upload_init entries). */
typedef struct qph_plan_upload {
  uint32_t off;           /* word offset in the arena */
  uint32_t n_words;
  const uint32_t* words;  /* host; read during qph_plan_create only */
} qph_plan_upload;

/* One Dispatch (plan.rs:84-107): kernel = qph_plan_kernel_id(Dispatch.kernel). */
typedef struct qph_plan_dispatch {
  int32_t kernel;
  uint32_t p_off;         /* word offset of the parameter block */
  uint32_t groups[3];     /* the dispatch grid; groups[1] carries the batch of the
                             conv / pool / resize family, groups[0] that of n_reduce_fin */
} qph_plan_dispatch;

typedef struct qph_plan_spec {
  uint32_t total_words;                 /* GraphPlan.total_words */
  int32_t n_uploads;
  const qph_plan_upload* uploads;
  int32_t n_dispatches;
  const qph_plan_dispatch* dispatches;  /* in execution order */
  uint32_t in_f32_off;                  /* GraphPlan.in_f32_off: the NCHW f32 input */
  int64_t in_numel;
  int32_t n_outputs;                    /* GraphPlan.out_offs */
  const uint32_t* out_offs;
  const int64_t* out_numel;             /* words per output ((value, index) pairs: rows * 2) */
} qph_plan_spec;

typedef struct qph_plan qph_plan;

/* KernelSet lookup by Dispatch.kernel name (vulkan/pipeline.rs:84-136):
 * the id, or QPH_EUNSUPPORTED for a kernel outside the set (the Metal-only
 * n_conv8_mma*, n_conv8h, n_conv_dw_tile, n_convt4w, n_head_argmax). */
QPH_API int qph_plan_kernel_id(const char* name);
/* The session's load step (vulkan/session.rs): decodes every parameter
 * block on the host first (refusing regions outside the arena, unknown
 * kernels and malformed blocks with the dispatch's index, before any device
 * call), then allocates the arena, writes the uploads and captures the
 * launches into a HIP graph. */
QPH_API int qph_plan_create(qph_ctx* ctx, const qph_plan_spec* spec, qph_plan** out);
/* The checks of qph_plan_create alone, on the host: no context and no
 * device are needed (QPH_OK, or the error qph_plan_create would return for
 * a malformed plan).  No counterpart in the reference, whose load step
 * builds the device objects as it goes; for loaders that vet a plan first. */
QPH_API int qph_plan_validate(const qph_plan_spec* spec);
QPH_API int qph_plan_destroy(qph_plan* plan);
/* real_n for the following runs (0 = every batch row): the reference's run
 * writes it to word 0 before each submit. */
QPH_API int qph_plan_set_real_n(qph_plan* plan, uint32_t real_n);
/* One run: real_n to word 0, input (numel = in_numel) to in_f32_off, the
 * dispatches, then the outputs to the host buffers (NULL entries skipped)
 * and a sync; without outputs the run is only enqueued on the context's
 * stream.  input NULL: the arena's input region is used as it is.  Runs of
 * one plan share its arena: calls on one plan must not overlap. */
QPH_API int qph_plan_run(qph_plan* plan, const float* input, int32_t input_is_device,
                         float* const* outputs_host);
/* The device arena (valid until destroy), for reading any region. */
QPH_API int qph_plan_arena(qph_plan* plan, float** dev, int64_t* words);
/* Number of launches the decoded plan issues per run (an n_reduce_hw and
 * its n_reduce_fin are one).  No counterpart in the reference. */
QPH_API int qph_plan_launches(qph_plan* plan, int32_t* n);

#ifdef __cplusplus
}
#endif

#endif /* QPPOCR_HIP_H */
