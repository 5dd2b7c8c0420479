// Context, memory, error reporting and the operator entry points of the C ABI
// (shape validation and kernel selection; the kernels live in the other
// translation units).
#include <cstdio>
#include <cstring>
#include <string>

#include <map>
#include <mutex>
#include <set>
#include <tuple>
#include <utility>

#include "qph_internal.h"

namespace qph {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}

int hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return QPH_OK;
  return fail(QPH_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

int launch_check(const char* kernel) {
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) return QPH_OK;
  return fail(QPH_EHIP, std::string("launch ") + kernel + ": " + hipGetErrorString(e));
}

int ctx_workspace(qph_ctx* ctx, size_t bytes, void** out) {
  if (bytes <= ctx->ws_bytes && ctx->ws) {
    *out = ctx->ws;
    return QPH_OK;
  }
  if (ctx->ws) {
    QPH_TRY_HIP(hipStreamSynchronize(ctx->stream));
    QPH_TRY_HIP(hipFree(ctx->ws));
    ctx->ws = nullptr;
    ctx->ws_bytes = 0;
  }
  size_t sz = bytes < (1u << 20) ? (1u << 20) : bytes;
  hipError_t e = hipMalloc(&ctx->ws, sz);
  if (e != hipSuccess) {
    ctx->ws = nullptr;
    return hip_check(e, "hipMalloc(workspace)");
  }
  ctx->ws_bytes = sz;
  *out = ctx->ws;
  return QPH_OK;
}

// The allocation-free conv entry point's device array: room for the k-major
// repacked weights of one dense conv, one copy per GPU for the life of the
// process.  Host code never uses this name as an address (on the host it is
// only a stand-in): the device address comes from hipGetSymbolAddress,
// looked up once per device with that device current, at context creation.
static __device__ __align__(256) float scratch[QPH_NOALLOC_WK_FLOATS];

static int scratch_address(int device, float** out) {
  static std::mutex mu;
  static std::map<int, float*> addr;
  std::lock_guard<std::mutex> lock(mu);
  auto it = addr.find(device);
  if (it != addr.end()) {
    *out = it->second;
    return QPH_OK;
  }
  void* p = nullptr;
  QPH_TRY_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
  if (!p) return fail(QPH_EHIP, "hipGetSymbolAddress(scratch) returned NULL");
  addr[device] = (float*)p;
  *out = (float*)p;
  return QPH_OK;
}

}  // namespace qph

using namespace qph;

#define CTX_CHECK(ctx) \
  if (!(ctx)) return fail(QPH_EINVAL, "null context")

// Fills `head` (< 16) bytes, `body16` 16-byte words and `tail` (< 16) bytes
// with the byte of v4 (replicated four times).
__global__ __launch_bounds__(256) void fill_bytes_kernel(unsigned char* head, size_t nhead,
                                                         uint4* body, size_t body16,
                                                         unsigned char* tail, size_t ntail,
                                                         unsigned v4) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * 256;
  for (size_t k = i; k < body16; k += stride) body[k] = make_uint4(v4, v4, v4, v4);
  if (i < nhead) head[i] = (unsigned char)v4;
  if (i < ntail) tail[i] = (unsigned char)v4;
}

extern "C" {

QPH_API const char* qph_last_error(void) { return g_last_error.c_str(); }
QPH_API const char* qph_version(void) { return "qppocr-hip 0.1 gfx950"; }

QPH_API int qph_ctx_create(int device, qph_ctx** out) {
  if (!out) return fail(QPH_EINVAL, "qph_ctx_create: out is NULL");
  *out = nullptr;
  int count = 0;
  QPH_TRY_HIP(hipGetDeviceCount(&count));
  if (device < 0 || device >= count)
    return fail(QPH_EINVAL, "qph_ctx_create: device " + std::to_string(device) + " of " +
                                std::to_string(count));
  QPH_TRY_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  QPH_TRY_HIP(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(QPH_EUNSUPPORTED, std::string("qph_ctx_create: device is ") + prop.gcnArchName +
                                      ", this library is built for gfx950 only");
  float* fixed_wk = nullptr;
  QPH_TRY(scratch_address(device, &fixed_wk));   // device is current
  qph_ctx* c = new qph_ctx;
  c->device = device;
  c->own_stream = true;
  c->ws = nullptr;
  c->ws_bytes = 0;
  c->noalloc_wk = fixed_wk;
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return hip_check(e, "hipStreamCreateWithFlags");
  }
  *out = c;
  return QPH_OK;
}

QPH_API int qph_ctx_destroy(qph_ctx* ctx) {
  if (!ctx) return QPH_OK;
  int rc = hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  if (ctx->ws) {
    int r2 = hip_check(hipFree(ctx->ws), "hipFree(workspace)");
    if (rc == QPH_OK) rc = r2;
  }
  if (ctx->own_stream) {
    int r2 = hip_check(hipStreamDestroy(ctx->stream), "hipStreamDestroy");
    if (rc == QPH_OK) rc = r2;
  }
  delete ctx;
  return rc;
}

QPH_API int qph_ctx_set_stream(qph_ctx* ctx, void* stream) {
  CTX_CHECK(ctx);
  if (ctx->own_stream) QPH_TRY_HIP(hipStreamDestroy(ctx->stream));
  if (stream) {
    ctx->stream = (hipStream_t)stream;
    ctx->own_stream = false;
  } else {
    QPH_TRY_HIP(hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking));
    ctx->own_stream = true;
  }
  return QPH_OK;
}

QPH_API void* qph_ctx_stream(qph_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

QPH_API int qph_ctx_scratch_bytes(qph_ctx* ctx, size_t* bytes) {
  CTX_CHECK(ctx);
  if (!bytes) return fail(QPH_EINVAL, "ctx_scratch_bytes: NULL argument");
  *bytes = ctx->ws_bytes;
  return QPH_OK;
}

QPH_API int qph_sync(qph_ctx* ctx) {
  CTX_CHECK(ctx);
  QPH_TRY_HIP(hipStreamSynchronize(ctx->stream));
  return QPH_OK;
}

QPH_API int qph_malloc(qph_ctx* ctx, void** ptr, size_t bytes) {
  CTX_CHECK(ctx);
  if (!ptr) return fail(QPH_EINVAL, "qph_malloc: ptr is NULL");
  QPH_TRY_HIP(hipSetDevice(ctx->device));
  hipError_t e = hipMalloc(ptr, bytes ? bytes : 1);
  if (e == hipErrorOutOfMemory) return fail(QPH_ENOMEM, "qph_malloc: out of device memory");
  return hip_check(e, "hipMalloc");
}

QPH_API int qph_free(qph_ctx* ctx, void* ptr) {
  CTX_CHECK(ctx);
  if (!ptr) return QPH_OK;
  QPH_TRY_HIP(hipStreamSynchronize(ctx->stream));
  return hip_check(hipFree(ptr), "hipFree");
}

QPH_API int qph_memcpy_h2d(qph_ctx* ctx, void* dst, const void* src, size_t bytes) {
  CTX_CHECK(ctx);
  QPH_TRY_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  return hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

QPH_API int qph_memcpy_d2h(qph_ctx* ctx, void* dst, const void* src, size_t bytes) {
  CTX_CHECK(ctx);
  QPH_TRY_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  return hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

QPH_API int qph_memset(qph_ctx* ctx, void* dst, int value, size_t bytes) {
  CTX_CHECK(ctx);
  if (!bytes) return QPH_OK;
  if (!dst) return fail(QPH_EINVAL, "memset: NULL destination");
  // a fill kernel, not hipMemsetAsync: a caller may capture the context
  // stream into a graph, and memset nodes are kept out of graphs
  unsigned char* p = (unsigned char*)dst;
  const size_t head = std::min(bytes, (size_t)((16 - (uintptr_t)p % 16) % 16));
  const size_t body16 = (bytes - head) / 16;
  const size_t tail = bytes - head - body16 * 16;
  const unsigned b = (unsigned)value & 0xffu;
  const size_t blocks = std::max<size_t>(1, std::min<size_t>((body16 + 255) / 256, 8192));
  hipLaunchKernelGGL(fill_bytes_kernel, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, p, head,
                     (uint4*)(p + head), body16, p + head + body16 * 16, tail,
                     b | (b << 8) | (b << 16) | (b << 24));
  return launch_check("fill_bytes_kernel");
}

// ------------------------------------------------------------------ conv

QPH_API int qph_conv2d_out_shape(const int64_t xs[4], const int64_t ws[4],
                                 const qph_conv_params* p, int64_t ys[4]) {
  if (!xs || !ws || !p || !ys) return fail(QPH_EINVAL, "conv2d_out_shape: NULL argument");
  for (int i = 0; i < 4; i++)
    if (xs[i] <= 0 || ws[i] <= 0)
      return fail(QPH_EINVAL, "conv2d_out_shape: non-positive dimension");
  if (p->dh != 1 || p->dw != 1) return fail(QPH_EUNSUPPORTED, "conv2d: dilation not supported");
  if (p->sh <= 0 || p->sw <= 0 || p->ph < 0 || p->pw < 0 || p->peh < 0 || p->pew < 0 ||
      p->group <= 0)
    return fail(QPH_EINVAL, "conv2d: bad stride/padding/group");
  if (p->group * ws[1] != xs[1]) return fail(QPH_EINVAL, "conv group mismatch");
  if (ws[0] % p->group != 0) return fail(QPH_EINVAL, "conv out channels % group");
  int64_t oh = (xs[2] + p->ph + p->peh - ws[2]) / p->sh + 1;
  int64_t ow = (xs[3] + p->pw + p->pew - ws[3]) / p->sw + 1;
  if (xs[2] + p->ph + p->peh < ws[2] || xs[3] + p->pw + p->pew < ws[3] || oh <= 0 || ow <= 0)
    return fail(QPH_EINVAL, "conv output empty");
  ys[0] = xs[0];
  ys[1] = ws[0];
  ys[2] = oh;
  ys[3] = ow;
  return QPH_OK;
}

}  // extern "C"

namespace qph {
int allow_full_lds(const void* fn) {
  static std::mutex mu;
  static std::set<std::pair<const void*, int>> done;
  int dev = 0;
  QPH_TRY_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  if (done.count({fn, dev})) return QPH_OK;
  QPH_TRY_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
  done.insert({fn, dev});
  return QPH_OK;
}

int device_cus(int* dev_out, int* cus) {
  static std::mutex mu;
  static std::map<int, int> cache;
  int dev = 0;
  QPH_TRY_HIP(hipGetDevice(&dev));
  if (dev_out) *dev_out = dev;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find(dev);
  if (it != cache.end()) {
    *cus = it->second;
    return QPH_OK;
  }
  int v = 0;
  QPH_TRY_HIP(hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev));
  if (v <= 0) return fail(QPH_EHIP, "device reports no compute units");
  cache[dev] = v;
  *cus = v;
  return QPH_OK;
}

int kernel_occupancy(const void* fn, int block, int* occ) {
  static std::mutex mu;
  static std::map<std::tuple<const void*, int, int>, int> cache;
  int dev = 0;
  QPH_TRY_HIP(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lock(mu);
  const auto key = std::make_tuple(fn, block, dev);
  auto it = cache.find(key);
  if (it != cache.end()) {
    *occ = it->second;
    return QPH_OK;
  }
  int v = 0;
  QPH_TRY_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&v, fn, block, 0));
  if (v <= 0) return fail(QPH_EHIP, "kernel does not fit a compute unit");
  cache[key] = v;
  *occ = v;
  return QPH_OK;
}

// The GEMM of a pointwise conv (the reference's 1x1 branch, conv.rs:264-460):
// Y[n][M][HW] = W[M][C] X[n][C][HW] over the batch, column-major-free rows,
// with the reference's bias placement rule; no residual, plain store.
void pointwise_gemm_args(const float* x, const int64_t xs[4], const float* w,
                         const int64_t ws[4], const float* bias, const Act& a, float* y,
                         GemmArgs* out) {
  const int64_t n = xs[0], c = xs[1], hw = xs[2] * xs[3], m = ws[0];
  GemmArgs gm{};
  gm.a = w; gm.lda = c; gm.a_batch = 0;
  gm.b = x; gm.ldb = hw; gm.b_batch = c * hw;
  gm.c = y; gm.ldc = hw; gm.c_batch = m * hw;
  gm.m = m; gm.n = hw; gm.k = c; gm.batch = n;
  gm.bias = bias; gm.bias_mode = bias ? 1 : 0;
  // 1x1 path of conv.rs:370-460: N > 1 runs the serial panel kernel per
  // chunk; N == 1 runs sgemm_res, whose rule depends on the shape.
  const double fl = (double)m * (double)hw * (double)c;
  gm.seed_rule = (n > 1 || fl < 2e5 || (hw + 31) / 32 >= 2) ? 0 : 1;
  gm.act = a;
  *out = gm;
}

// Validates a conv node and launches its kernel.  wk: resident k-major
// repacked weights of a dense conv (NULL: repacked into the context scratch).
int conv_dispatch(qph_ctx* ctx, const float* x, const int64_t xs[4], const float* w,
                  const float* wk_resident, const int64_t ws[4], const float* bias,
                  const qph_conv_params* p, const qph_act* act, const qph_conv_epilogue* ep,
                  float* y, ConvArgs* plan, float* fixed_wk, int64_t fixed_floats) {
  CTX_CHECK(ctx);
  if (!x || !w || !y) return fail(QPH_EINVAL, "conv2d: NULL tensor");
  if (!act_valid(act)) return fail(QPH_EINVAL, "conv2d: bad activation kind");
  int64_t ys[4];
  QPH_TRY(qph_conv2d_out_shape(xs, ws, p, ys));
  const int64_t n = xs[0], c = xs[1], h = xs[2], wd = xs[3];
  const int64_t m = ws[0], cg = ws[1], kh = ws[2], kw = ws[3];
  const int64_t g = p->group;
  const int64_t oh = ys[2], ow = ys[3];
  // the reference's 1x1 branch (conv.rs:264) reads X as a dense [C][oh*ow]
  // matrix, which holds only without padding; a padded 1x1 conv is an
  // ordinary conv and takes the implicit-GEMM branch here
  const bool pointwise = conv_is_pointwise(ws, *p);
  const bool depthwise = g > 1 && cg == 1;
  const float* res = ep ? ep->residual : nullptr;
  int res_up = ep ? ep->res_up : 0;
  int64_t y_ctotal = ep && ep->y_ctotal ? ep->y_ctotal : m;
  int64_t y_coff = ep ? ep->y_coff : 0;
  int64_t y_up = ep && ep->y_up ? ep->y_up : 1;
  int trans = ep ? ep->trans_out : 0;
  if (res_up != 0 && res_up != 2) return fail(QPH_EINVAL, "conv2d: res_up must be 0 or 2");
  if (y_up < 1 || y_coff < 0 || y_coff + m > y_ctotal)
    return fail(QPH_EINVAL, "conv2d: bad output placement");
  if (res_up == 2 && ((oh & 1) || (ow & 1)))
    return fail(QPH_EINVAL, "conv2d: upsample-add needs even output size");
  if (res_up == 2 && oh * ow >= (1ll << 32))
    return fail(QPH_EUNSUPPORTED, "conv2d: upsample-add map past 2^32 pixels");
  const bool plain_out = y_ctotal == m && y_coff == 0 && y_up == 1;
  Act a = make_act(act);

  if (plan && (pointwise || depthwise || g != 1 || !wk_resident))
    return fail(QPH_EUNSUPPORTED, "conv2d: only resident dense convs are planned");
  if (pointwise) {
    if (!plain_out) return fail(QPH_EUNSUPPORTED, "conv2d 1x1: channel-slice output not supported");
    if (trans && res_up) return fail(QPH_EUNSUPPORTED, "conv2d 1x1: trans_out with res_up");
    GemmArgs gm{};
    pointwise_gemm_args(x, xs, w, ws, bias, a, y, &gm);
    gm.ldc = trans ? m : oh * ow;
    gm.res = res;
    gm.ldr = res_up ? (oh / 2) * (ow / 2) : oh * ow;
    gm.r_batch = m * gm.ldr;
    gm.res_up = res_up;
    gm.up_w = ow;
    gm.up_cw = ow / 2;
    gm.trans_out = trans;
    return launch_gemm(gm, ctx->stream);
  }
  if (trans) return fail(QPH_EUNSUPPORTED, "conv2d: trans_out only for 1x1");
  if (res_up) return fail(QPH_EUNSUPPORTED, "conv2d: upsample-add only for 1x1");
  ConvArgs ca{};
  ca.x = x; ca.n = n; ca.c = c; ca.h = h; ca.w = wd;
  ca.wt = w; ca.wk = nullptr; ca.bias = bias;
  ca.m = m; ca.kh = kh; ca.kw = kw; ca.sh = p->sh; ca.sw = p->sw; ca.ph = p->ph; ca.pw = p->pw;
  ca.oh = oh; ca.ow = ow; ca.group = g;
  ca.act = a; ca.res = res; ca.y = y;
  ca.y_ctotal = y_ctotal; ca.y_coff = y_coff; ca.y_up = y_up;
  // depthwise (conv.rs:461-505) with one output per channel; a channel
  // multiplier (M = k C) is a grouped conv with C/g = 1 and goes the general way
  if (depthwise && m == c) return launch_depthwise(ca, ctx->stream);
  if (res && !plain_out) return fail(QPH_EUNSUPPORTED, "conv2d: residual with placed output");
  if (wk_resident) {
    ca.wk = wk_resident;
    if (plan) {
      *plan = ca;
      return QPH_OK;
    }
    return launch_dense_conv(ca, ctx->stream, nullptr);
  }
  // standalone call: k-major repacked weights go to the fixed array or the
  // context scratch
  int64_t nwk = dense_conv_wk_floats(m, cg, kh, kw, g);
  if (fixed_wk) {
    if (nwk > fixed_floats)
      return fail(QPH_EUNSUPPORTED,
                  "conv2d_noalloc: the repacked weights need " + std::to_string(nwk) +
                      " floats, the fixed device array holds " + std::to_string(fixed_floats));
    return launch_dense_conv(ca, ctx->stream, fixed_wk);
  }
  void* wk = nullptr;
  QPH_TRY(ctx_workspace(ctx, (size_t)nwk * 4, &wk));
  return launch_dense_conv(ca, ctx->stream, (float*)wk);
}
}  // namespace qph

extern "C" {

QPH_API int qph_conv2d(qph_ctx* ctx, const float* x, const int64_t xs[4], const float* w,
                       const int64_t ws[4], const float* bias, const qph_conv_params* p,
                       const qph_act* act, const float* residual, float* y, int64_t ys_out[4]) {
  if (ys_out) QPH_TRY(qph_conv2d_out_shape(xs, ws, p, ys_out));
  qph_conv_epilogue ep{};
  ep.residual = residual;
  return conv_dispatch(ctx, x, xs, w, nullptr, ws, bias, p, act, &ep, y);
}

QPH_API int qph_conv2d_noalloc(qph_ctx* ctx, const float* x, const int64_t xs[4], const float* w,
                               const int64_t ws[4], const float* bias, const qph_conv_params* p,
                               const qph_act* act, const float* residual, float* y,
                               int64_t ys_out[4]) {
  CTX_CHECK(ctx);
  if (ys_out) QPH_TRY(qph_conv2d_out_shape(xs, ws, p, ys_out));
  qph_conv_epilogue ep{};
  ep.residual = residual;
  return conv_dispatch(ctx, x, xs, w, nullptr, ws, bias, p, act, &ep, y, nullptr,
                       ctx->noalloc_wk, QPH_NOALLOC_WK_FLOATS);
}

QPH_API int qph_conv2d_ex(qph_ctx* ctx, const float* x, const int64_t xs[4], const float* w,
                          const int64_t ws[4], const float* bias, const qph_conv_params* p,
                          const qph_act* act, const qph_conv_epilogue* ep, float* y) {
  return conv_dispatch(ctx, x, xs, w, nullptr, ws, bias, p, act, ep, y);
}

QPH_API int qph_convtranspose2d(qph_ctx* ctx, const float* x, const int64_t xs[4],
                                const float* w, const int64_t ws[4], int64_t sh, int64_t sw,
                                int64_t ph, int64_t pw, float* y, int64_t ys_out[4]) {
  CTX_CHECK(ctx);
  if (!x || !w || !y || !xs || !ws) return fail(QPH_EINVAL, "convtranspose2d: NULL argument");
  if (ws[0] != xs[1]) return fail(QPH_EINVAL, "convT weight C_in mismatch");
  if (ws[2] != 2 || ws[3] != 2 || sh != 2 || sw != 2 || ph != 0 || pw != 0)
    return fail(QPH_EUNSUPPORTED, "convtranspose: only 2x2 s2 p0 supported");
  for (int i = 0; i < 4; i++)
    if (xs[i] <= 0 || ws[i] <= 0) return fail(QPH_EINVAL, "convtranspose2d: empty tensor");
  if (ys_out) {
    ys_out[0] = xs[0]; ys_out[1] = ws[1]; ys_out[2] = 2 * xs[2]; ys_out[3] = 2 * xs[3];
  }
  return launch_convt2x2(x, xs[0], xs[1], xs[2], xs[3], w, ws[1], y, ctx->stream);
}

QPH_API int qph_convt2x2_pair_sigmoid(qph_ctx* ctx, const float* x, const int64_t xs[4],
                                      const float* w1, const int64_t w1s[4], const float* w2,
                                      const int64_t w2s[4], float* y) {
  CTX_CHECK(ctx);
  if (!x || !w1 || !w2 || !y) return fail(QPH_EINVAL, "convt pair: NULL argument");
  if (w1s[0] != xs[1] || w1s[2] != 2 || w1s[3] != 2 || w2s[0] != w1s[1] || w2s[1] != 1 ||
      w2s[2] != 2 || w2s[3] != 2)
    return fail(QPH_EUNSUPPORTED, "convt pair: needs w1 [C,M,2,2], w2 [M,1,2,2]");
  if (xs[1] > 64 || w1s[1] > 64) return fail(QPH_EUNSUPPORTED, "convt pair: C and M must be <= 64");
  return launch_convt2x2_pair_sigmoid(x, xs[0], xs[1], xs[2], xs[3], w1, w1s[1], w2, y,
                                      ctx->stream);
}

// ------------------------------------------------------------------ GEMM

QPH_API int qph_sgemm(qph_ctx* ctx, const float* a, const float* b, float* c, int64_t m,
                      int64_t n, int64_t k, int64_t ldc, const float* bias, const qph_act* act,
                      const float* residual, int32_t serial) {
  CTX_CHECK(ctx);
  if (m == 0 || n == 0 || k == 0) return QPH_OK;  // gemm.rs:236-238
  if (m < 0 || n < 0 || k < 0 || ldc < n) return fail(QPH_EINVAL, "sgemm: ldc < n or bad dims");
  if (!a || !b || !c) return fail(QPH_EINVAL, "sgemm: NULL operand");
  if (!act_valid(act)) return fail(QPH_EINVAL, "sgemm: bad activation kind");
  GemmArgs g{};
  g.a = a; g.lda = k; g.b = b; g.ldb = n; g.c = c; g.ldc = ldc;
  g.m = m; g.n = n; g.k = k; g.batch = 1;
  g.bias = bias; g.bias_mode = bias ? 1 : 0;
  double fl = (double)m * (double)n * (double)k;
  g.seed_rule = (serial || fl < 2e5 || (n + 31) / 32 >= 2) ? 0 : 1;
  g.act = make_act(act);
  g.res = residual; g.ldr = ldc;
  return launch_gemm(g, ctx->stream);
}

QPH_API int qph_matmul(qph_ctx* ctx, const float* a, const float* b, float* out, int64_t batch,
                       int64_t m, int64_t k, int64_t n, int32_t b_shared) {
  CTX_CHECK(ctx);
  if (batch <= 0 || m <= 0 || k <= 0 || n <= 0) return fail(QPH_EINVAL, "matmul: bad dims");
  if (!a || !b || !out) return fail(QPH_EINVAL, "matmul: NULL operand");
  GemmArgs g{};
  g.a = a; g.lda = k; g.a_batch = m * k;
  g.b = b; g.ldb = n; g.b_batch = b_shared ? 0 : k * n;
  g.c = out; g.ldc = n; g.c_batch = m * n;
  g.m = m; g.n = n; g.k = k; g.batch = batch;
  g.act = make_act(nullptr);
  if (b_shared) {  // shape.rs:621-662 folds the batch into M
    g.m = batch * m; g.batch = 1; g.a_batch = 0; g.c_batch = 0;
  }
  return launch_gemm(g, ctx->stream);
}

QPH_API int qph_linear(qph_ctx* ctx, const float* x, const float* w, const float* bias,
                       int64_t rows, int64_t k, int64_t n, const qph_act* act,
                       const float* residual, float* y) {
  CTX_CHECK(ctx);
  if (rows <= 0 || k <= 0 || n <= 0) return fail(QPH_EINVAL, "linear: bad dims");
  if (!x || !w || !y) return fail(QPH_EINVAL, "linear: NULL operand");
  if (!act_valid(act)) return fail(QPH_EINVAL, "linear: bad activation kind");
  GemmArgs g{};
  g.a = x; g.lda = k; g.b = w; g.ldb = n; g.c = y; g.ldc = n;
  g.m = rows; g.n = n; g.k = k; g.batch = 1;
  g.bias = bias; g.bias_mode = bias ? 2 : 0;
  g.act = make_act(act);
  g.res = residual; g.ldr = n;
  return launch_gemm(g, ctx->stream);
}

// ------------------------------------------------------------ row kernels

QPH_API int qph_layernorm(qph_ctx* ctx, const float* x, const float* gamma, const float* beta,
                          float eps, int64_t rows, int64_t cols, float* y) {
  CTX_CHECK(ctx);
  if (rows <= 0 || cols <= 0 || !x || !gamma || !beta || !y)
    return fail(QPH_EINVAL, "layernorm: bad argument");
  if (cols > 4096) return fail(QPH_EUNSUPPORTED, "layernorm: cols > 4096");
  return launch_layernorm(x, gamma, beta, eps, rows, cols, y, ctx->stream);
}

QPH_API int qph_softmax_last_dim(qph_ctx* ctx, float* t, int64_t rows, int64_t inner) {
  CTX_CHECK(ctx);
  if (rows <= 0 || inner <= 0 || !t) return fail(QPH_EINVAL, "softmax: bad argument");
  return launch_softmax_rows(t, rows, inner, ctx->stream);
}

QPH_API int qph_softmax_argmax(qph_ctx* ctx, const float* logits, int64_t rows, int64_t cols,
                               float* probs, float* pairs) {
  CTX_CHECK(ctx);
  if (rows <= 0 || cols <= 0 || !logits || !pairs)
    return fail(QPH_EINVAL, "softmax_argmax: bad argument");
  if (cols >= (1ll << 31)) return fail(QPH_EUNSUPPORTED, "softmax_argmax: cols >= 2^31");
  return launch_softmax_argmax(logits, rows, cols, cols, probs, pairs, ctx->stream);
}

QPH_API int qph_linear_softmax_argmax(qph_ctx* ctx, const float* x, const float* w,
                                      const float* bias, int64_t rows, int64_t k, int64_t n,
                                      float* pairs) {
  CTX_CHECK(ctx);
  if (rows <= 0 || k <= 0 || n <= 0 || !x || !w || !pairs)
    return fail(QPH_EINVAL, "linear_softmax_argmax: bad argument");
  if (!head_argmax_eligible(rows, n, k, k, n))
    return fail(QPH_EUNSUPPORTED, "linear_softmax_argmax: needs k % 16 == 0, operands < 2 GB");
  void* part = nullptr;
  QPH_TRY(ctx_workspace(ctx, (size_t)head_argmax_part_floats(rows, n) * 4, &part));
  return launch_head_argmax(x, rows, k, w, n, n, bias, (float*)part, pairs, ctx->stream);
}

QPH_API int qph_ctc_argmax(qph_ctx* ctx, const float* probs, int64_t batch, int64_t t_len,
                           int64_t cols, const int32_t* t_valid_host, float* pairs) {
  CTX_CHECK(ctx);
  if (batch <= 0 || t_len <= 0 || cols <= 0 || !probs || !pairs)
    return fail(QPH_EINVAL, "ctc_argmax: bad argument");
  QPH_TRY(launch_argmax(probs, batch * t_len, cols, pairs, ctx->stream));
  if (!t_valid_host) return QPH_OK;
  void* dv = nullptr;
  QPH_TRY(ctx_workspace(ctx, (size_t)batch * 4, &dv));
  QPH_TRY_HIP(hipMemcpyAsync(dv, t_valid_host, (size_t)batch * 4, hipMemcpyHostToDevice,
                             ctx->stream));
  QPH_TRY(launch_mask_pairs(pairs, batch, t_len, (const int32_t*)dv, ctx->stream));
  // the host array may be released as soon as this call returns
  return hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

QPH_API int qph_attention(qph_ctx* ctx, const float* qkv, int64_t batch, int64_t t,
                          int64_t heads, int64_t dh, float scale, float* out) {
  CTX_CHECK(ctx);
  if (batch <= 0 || t <= 0 || heads <= 0 || dh <= 0 || !qkv || !out)
    return fail(QPH_EINVAL, "attention: bad argument");
  if (dh > 64 || t > 256) return fail(QPH_EUNSUPPORTED, "attention: needs dh <= 64, t <= 256");
  return launch_attention(qkv, batch, t, heads, dh, scale, out, ctx->stream);
}

QPH_API int qph_activation(qph_ctx* ctx, const float* x, float* y, int64_t n, const qph_act* act) {
  CTX_CHECK(ctx);
  if (n < 0 || (n > 0 && (!x || !y))) return fail(QPH_EINVAL, "activation: bad argument");
  if (!act_valid(act)) return fail(QPH_EINVAL, "activation: bad kind");
  if (n == 0) return QPH_OK;
  return launch_elementwise_act(x, y, n, make_act(act), ctx->stream);
}

QPH_API int qph_hardsigmoid(qph_ctx* ctx, const float* x, float* y, int64_t n, float alpha,
                            float beta) {
  CTX_CHECK(ctx);
  if (n < 0 || (n > 0 && (!x || !y))) return fail(QPH_EINVAL, "hardsigmoid: bad argument");
  if (n == 0) return QPH_OK;
  Act a{};
  a.kind = 5;  // bare HardSigmoid (internal kind)
  a.c1 = alpha;
  a.c2 = beta;
  a.inv_c1 = 1.0f;
  return launch_elementwise_act(x, y, n, a, ctx->stream);
}

QPH_API int qph_resize_nearest(qph_ctx* ctx, const float* x, int64_t nc, int64_t h, int64_t w,
                               int64_t oh, int64_t ow, float* y) {
  CTX_CHECK(ctx);
  if (nc <= 0 || h <= 0 || w <= 0 || oh <= 0 || ow <= 0 || !x || !y)
    return fail(QPH_EINVAL, "resize_nearest: bad argument");
  return launch_resize_nearest(x, nc, h, w, oh, ow, y, ctx->stream);
}

QPH_API int qph_binary_inplace(qph_ctx* ctx, float* a, const float* b, int64_t rows,
                               int64_t cols, int32_t op, int32_t bmode) {
  CTX_CHECK(ctx);
  if (rows <= 0 || cols <= 0 || !a || !b || op < 0 || op > 3 || bmode < 0 || bmode > 3)
    return fail(QPH_EINVAL, "binary: bad argument");
  return launch_binary(a, b, rows, cols, op, bmode, ctx->stream);
}

}  // extern "C"
