// Session: a static det/rec graph resident on the device, run as one HIP
// graph replay per call.  This is the DeviceSession side of the boundary
// (qppocr-core/src/device.rs:83-176): weights are moved to the device once at
// create time, every node is validated then (unsupported -> error naming the
// node, no silent fallback, device.rs:88-94), and each run is one host call.
#include <cstring>
#include <string>
#include <vector>

#include "qph_internal.h"

using namespace qph;

struct qph_net {
  qph_ctx* ctx;
  std::vector<qph_node> nodes;
  std::vector<int64_t> shapes_full;  // 4 per tensor, as created
  std::vector<int64_t> shapes;   // 4 per tensor, batch dimension cut to real_n
  std::vector<bool> batch_major; // per tensor: derived from the input, batch outermost
  int64_t batch;                 // the input's batch dimension (the net's capacity)
  int64_t real_n;                // batch items the next run computes (1..batch)
  std::vector<int32_t> alias;
  std::vector<int32_t> outputs;
  std::vector<float*> weights;   // device copies
  std::vector<float*> wk;        // per node: resident repacked dense-conv weights (or NULL)
  std::vector<ConvArgs> plan;    // per node: launch arguments of a dense 3x3 conv
  std::vector<int> group_len;    // > 1: first of that many independent 3x3 convs, one launch
  std::vector<bool> convt_fused; // 3x3 conv node i and its conv-transpose pair i + 1, one launch
  std::vector<int> absorb_after; // nodes after node i done in its launch's epilogue (0 or 4)
  std::vector<bool> fpn;         // node i starts four FPN laterals run as three launches
  std::vector<float*> fpn_tmp;   // per such node: the raw level-4 and level-3 laterals
  std::vector<float*> fpn_t4, fpn_t3;
  std::vector<DwPwArgs> dwpw;    // per node: fused depthwise + pointwise launch
  std::vector<bool> fused;       // node i runs dwpw[i] (and node i + 1, and i + 2 for a stem, with it)
  std::vector<float*> wt;        // per linear node: resident transposed weight Wt[N][K] (or NULL)
  std::vector<bool> cl_dw;       // depthwise conv node run channel-last (in and out)
  std::vector<bool> cl_pw;       // 1x1 conv node run as a row-major GEMM, channel-last in and out
  std::vector<bool> cl_out;      // 1x1 conv node storing channel-last (trans_out) for a cl_dw reader
  std::vector<bool> head;        // linear node i and the pairs-only softmax i + 1 run fused
  std::vector<bool> qa_fused;    // linear node i (QKV) and attention node i + 1, one launch
  std::vector<float*> head_part; // per fused head: its per-block argmax partials
  std::vector<bool> nostore;     // per tensor: never materialised (inside one fused launch)
  std::vector<float*> tptr;      // per tensor device pointer
  std::vector<int64_t> pitch;    // per tensor: padded row pitch in floats (0: contiguous)
  char* arena;
  size_t arena_bytes;
  std::vector<hipGraph_t> graphs;     // per real_n (index 1..batch): captured on first use
  std::vector<hipGraphExec_t> execs;
  bool profiling;
  std::vector<hipEvent_t> ev;
  std::vector<double> node_ms;
  int64_t prof_runs;
  // deferred runs: pinned host staging of the input and of each output
  float* in_stage;
  std::vector<float*> out_stage;
  hipEvent_t done;
  bool inflight;
};

// Elements of a tensor in the current run (batch-major tensors hold
// real_n batch items) and of its storage.
static int64_t numel_of(const qph_net* net, int32_t id) {
  const int64_t* s = &net->shapes[4 * (size_t)id];
  return s[0] * s[1] * s[2] * s[3];
}

static int64_t numel_full(const qph_net* net, int32_t id) {
  const int64_t* s = &net->shapes_full[4 * (size_t)id];
  return s[0] * s[1] * s[2] * s[3];
}

static std::string node_name(size_t i, const qph_node& n) {
  return "node " + std::to_string(i) + " (op " + std::to_string(n.op) + ")";
}

static int check_tensor(const qph_net* net, int32_t id, bool optional, size_t i, const qph_node& n,
                        const char* what) {
  if (id < 0 && optional) return QPH_OK;
  if (id < 0 || id >= (int32_t)net->tptr.size())
    return fail(QPH_EINVAL, node_name(i, n) + ": bad " + what + " tensor id");
  return QPH_OK;
}

// The 1x1 path's bias-placement rule for n batch items of px pixels
// (qppocr-kernels/src/conv.rs:264-460, as conv_dispatch picks it): 0 = the
// bias after the chain everywhere, 1 = the N == 1 panel / m-rows rule.
static int pw_seed_rule(int64_t n, int64_t m, int64_t px, int64_t c) {
  const double fl = (double)m * (double)px * (double)c;
  return (n > 1 || fl < 2e5 || (px + 31) / 32 >= 2) ? 0 : 1;
}

// Linear node i over its resident transposed weight.
static LinArgs lin_args(const qph_net* net, size_t i) {
  const qph_node& n = net->nodes[i];
  LinArgs g{};
  g.a = net->tptr[n.in];
  g.lda = n.ws[0];
  g.wt = net->wt[i];
  g.c = net->tptr[n.out];
  g.k = n.ws[0];
  g.n = n.ws[1];
  g.m = numel_of(net, n.in) / g.k;
  g.bias = n.bias >= 0 ? net->weights[n.bias] : nullptr;
  g.act = make_act(&n.act);
  g.res = n.in2 >= 0 ? net->tptr[n.in2] : nullptr;
  return g;
}

// Launches node i on the context stream.
static int run_node(qph_net* net, size_t i) {
  const qph_node& n = net->nodes[i];
  qph_ctx* ctx = net->ctx;
  hipStream_t s = ctx->stream;
  const int64_t* xs = &net->shapes[4 * (size_t)n.in];
  float* x = net->tptr[n.in];
  float* y = n.out >= 0 ? net->tptr[n.out] : nullptr;
  const float* w = n.w >= 0 ? net->weights[n.w] : nullptr;
  const float* bias = n.bias >= 0 ? net->weights[n.bias] : nullptr;
  const float* w2 = n.w2 >= 0 ? net->weights[n.w2] : nullptr;
  const float* res = n.in2 >= 0 ? net->tptr[n.in2] : nullptr;
  switch (n.op) {
    case QPH_OP_CONV: {
      if (net->cl_dw[i]) {
        ConvArgs a{};
        a.x = x; a.n = xs[0]; a.c = xs[1]; a.h = xs[2]; a.w = xs[3];
        a.wt = w; a.bias = bias;
        a.m = n.ws[0]; a.kh = n.ws[2]; a.kw = n.ws[3];
        a.sh = n.cp.sh; a.sw = n.cp.sw; a.ph = n.cp.ph; a.pw = n.cp.pw;
        const int64_t* ys = &net->shapes[4 * (size_t)n.out];
        a.oh = ys[2]; a.ow = ys[3];
        a.act = make_act(&n.act);
        a.y = y;
        return launch_depthwise_cl(a, s);
      }
      if (net->cl_pw[i]) {
        // y[n * h * w][M] = act(x[n * h * w][C] . W[M][C]^T + bias)
        LinArgs g{};
        g.a = x; g.lda = n.ws[1]; g.wt = w; g.c = y;
        g.m = xs[0] * xs[2] * xs[3]; g.n = n.ws[0]; g.k = n.ws[1];
        g.bias = bias; g.act = make_act(&n.act); g.res = nullptr;
        // the m-rows rule (one batch item of at most 32 pixels, as a run at
        // real_n = 1 can be) seeds the chain with the bias for the pixels
        // past the last full 32-pixel block: all of them below 32 pixels
        const int64_t px = xs[2] * xs[3];
        g.bias_seed = bias && pw_seed_rule(xs[0], g.n, px, g.k) == 1 && px < 32;
        return launch_linear_nt(g, s);
      }
      qph_conv_epilogue ep{};
      ep.residual = res;
      ep.res_up = n.res_up;
      ep.y_ctotal = n.y_ctotal;
      ep.y_coff = n.y_coff;
      ep.y_up = n.y_up;
      ep.trans_out = n.trans_out || net->cl_out[i];
      return conv_dispatch(ctx, x, xs, w, net->wk[i], n.ws, bias, &n.cp, &n.act, &ep, y);
    }
    case QPH_OP_CONVT_PAIR_SIG:
      return launch_convt2x2_pair_sigmoid(x, xs[0], xs[1], xs[2], xs[3], w, n.ws[1], w2, y, s);
    case QPH_OP_CONVT:
      return launch_convt2x2(x, xs[0], xs[1], xs[2], xs[3], w, n.ws[1], y, s);
    case QPH_OP_LINEAR: {
      const int64_t k = n.ws[0], nn = n.ws[1];
      const int64_t rows = numel_of(net, n.in) / k;
      if (net->wt[i]) return launch_linear_nt(lin_args(net, i), s);
      GemmArgs g{};
      // weights resident with rows padded to a multiple of 4 floats
      g.a = x; g.lda = k; g.b = net->wk[i] ? net->wk[i] : w; g.ldb = (nn + 3) / 4 * 4;
      if (!net->wk[i]) g.ldb = nn;
      g.c = y; g.ldc = net->pitch[n.out] ? net->pitch[n.out] : nn;
      g.m = rows; g.n = nn; g.k = k; g.batch = 1;
      g.bias = bias; g.bias_mode = bias ? 2 : 0;
      g.act = make_act(&n.act);
      g.res = res; g.ldr = nn;
      return launch_gemm(g, s);
    }
    case QPH_OP_LAYERNORM: {
      const int64_t cols = n.ws[0];
      return launch_layernorm(x, w, bias, n.eps, numel_of(net, n.in) / cols, cols, y, s);
    }
    case QPH_OP_ATTENTION:
      return launch_attention(x, xs[0], xs[1], n.heads, n.dh, n.scale, y, s);
    case QPH_OP_SOFTMAX_ARGMAX: {
      const int64_t c = n.ws[0];  // row width
      float* pairs = n.out2 >= 0 ? net->tptr[n.out2] : nullptr;
      return launch_softmax_argmax(x, numel_of(net, n.in) / c, c,
                                   net->pitch[n.in] ? net->pitch[n.in] : c, y, pairs, s);
    }
    case QPH_OP_ACT:
      return launch_elementwise_act(x, y, numel_of(net, n.in), make_act(&n.act), s);
    case QPH_OP_GAP:
      return launch_reduce_mean(x, xs[0] * xs[1], xs[2] * xs[3], y, s);
    case QPH_OP_MUL_ADD_SCALE: {
      // gate per channel ([C]) or per batch item and channel ([N, C])
      const int64_t c = xs[1], planes = xs[0] * xs[1];
      const float* gate = net->tptr[n.in3];
      const int64_t gmod = numel_of(net, n.in3) == c ? c : planes;
      return launch_mul_add_scale(x, gate, res, y, c, gmod, xs[2] * xs[3], planes,
                                  n.y_ctotal ? n.y_ctotal : c, n.y_coff, s);
    }
    case QPH_OP_POOL:
      return launch_pool2d(x, xs[0], xs[1], xs[2], xs[3], n.ws[2], n.ws[3], n.cp.sh, n.cp.sw,
                           n.cp.ph, n.cp.pw, n.cp.peh, n.cp.pew, n.ws[0] != 0, y,
                           n.y_ctotal ? n.y_ctotal : xs[1], n.y_coff, s);
    case QPH_OP_RESIZE: {
      const int64_t* ys = &net->shapes[4 * (size_t)n.out];
      if (n.ws[0] == 0)
        return launch_resize_nearest(x, xs[0] * xs[1], xs[2], xs[3], ys[2], ys[3], y, s);
      return launch_resize_bilinear(x, xs[0], xs[1], xs[2], xs[3], ys[2], ys[3], n.ws[1] != 0, y,
                                    n.y_ctotal ? n.y_ctotal : xs[1], n.y_coff, s);
    }
    case QPH_OP_TRANSPOSE: {
      const int32_t perm[4] = {(int32_t)n.ws[0], (int32_t)n.ws[1], (int32_t)n.ws[2],
                               (int32_t)n.ws[3]};
      return launch_transpose4(x, xs, perm, y, s);
    }
    case QPH_OP_COPY_SLOT:
      return launch_copy_slot(x, y, xs[1], xs[2] * xs[3], xs[0] * xs[1], n.y_ctotal, n.y_coff, s);
    case QPH_OP_BINARY:
      return launch_binary_out(x, n.in2 >= 0 ? net->tptr[n.in2] : nullptr, n.scale, y,
                               numel_of(net, n.in), (int)n.ws[0],
                               n.in2 >= 0 ? 0 : (n.ws[1] ? 2 : 1), s);
    default:
      return fail(QPH_EUNSUPPORTED, node_name(i, n) + ": unknown op");
  }
}

static int32_t storage_of(const qph_net* net, int32_t t) {
  return t >= 0 && net->alias[(size_t)t] >= 0 ? net->alias[(size_t)t] : t;
}

// A linear on the 128x128 path whose output only a softmax_argmax reads
// (the rec head, N = 18709) keeps its rows 32 floats (128 bytes) apart: every
// 32-column segment of the GEMM's stores is then one whole cache line instead
// of parts of two.  Runs before the arena is laid out; ids are range-checked
// here because the nodes are validated later.
// With QPH_NET_FUSED_HEAD: a linear read only by the pairs-only softmax
// argmax right after it (the rec head) runs as one GEMM whose epilogue keeps
// per-block (max, index, exp sum) partials; its logits are never stored.
// Runs before the arena is laid out (ids range-checked here: the nodes are
// validated later).
static void plan_fused_head(qph_net* net, int32_t flags) {
  const size_t nn = net->nodes.size(), nt = net->tptr.size();
  net->head.assign(nn, false);
  net->head_part.assign(nn, nullptr);
  net->nostore.assign(nt, false);
  if (!(flags & QPH_NET_FUSED_HEAD)) return;
  auto ok = [&](int32_t t) { return t >= 0 && (size_t)t < nt; };
  for (size_t i = 0; i + 1 < nn; i++) {
    const qph_node& q = net->nodes[i];
    const qph_node& r = net->nodes[i + 1];
    if (q.op != QPH_OP_LINEAR || r.op != QPH_OP_SOFTMAX_ARGMAX || !ok(q.out) || !ok(q.in) ||
        !ok(r.out2) || r.out >= 0 || r.in != q.out || q.in2 >= 0 || q.act.kind != QPH_ACT_NONE ||
        q.ws[0] <= 0 || q.ws[1] <= 0 || r.ws[0] != q.ws[1])
      continue;
    const int32_t t = q.out;
    if (net->alias[(size_t)t] >= 0) continue;
    bool single = true;
    for (size_t t2 = 0; t2 < nt; t2++) single = single && net->alias[t2] != t;
    for (size_t j = 0; j < nn; j++)
      if (j != i + 1)
        single = single && net->nodes[j].in != t && net->nodes[j].in2 != t &&
                 net->nodes[j].in3 != t;
    for (int32_t o : net->outputs) single = single && o != t;
    const int64_t rows = numel_of(net, q.in) / q.ws[0];
    if (!single || numel_of(net, q.in) % q.ws[0] ||
        !head_argmax_eligible(rows, q.ws[1], q.ws[0], q.ws[0], (q.ws[1] + 3) / 4 * 4))
      continue;
    net->head[i] = true;
    net->nostore[(size_t)t] = true;
  }
}

// A linear read only by the attention right after it (the rec QKV
// projection), with no activation or residual, whose output is the
// attention's q, k, v of head dimension 32 over T <= 64 rows (T % 4 == 0)
// and whose K is a multiple of 64 up to 256: both run as one launch
// (qkv_attention_kernel), the QKV tensor never stored.  The linear keeps
// its resident transposed weight (same rule as the resident-weight
// linears).  Runs after plan_pitch (both tensors contiguous) and before
// the arena is laid out.
static void plan_qkv_attention(qph_net* net, int32_t flags) {
  const size_t nn = net->nodes.size(), nt = net->tptr.size();
  net->qa_fused.assign(nn, false);
  if (flags & QPH_NET_SEPARATE_LAUNCHES) return;
  auto ok = [&](int32_t t) { return t >= 0 && (size_t)t < nt; };
  for (size_t i = 0; i + 1 < nn; i++) {
    const qph_node& q = net->nodes[i];
    const qph_node& r = net->nodes[i + 1];
    if (q.op != QPH_OP_LINEAR || r.op != QPH_OP_ATTENTION || !ok(q.in) || !ok(q.out) ||
        !ok(r.out) || r.in != q.out || q.in2 >= 0 || q.act.kind != QPH_ACT_NONE ||
        q.ws[0] <= 0 || q.ws[1] != 3 * (int64_t)r.heads * r.dh || net->head[i])
      continue;
    const int32_t t = q.out;
    const int64_t* xs = &net->shapes[4 * (size_t)t];
    const int64_t k = q.ws[0], rows = numel_of(net, q.in) / k;
    if (net->alias[(size_t)t] >= 0 || net->alias[(size_t)q.in] >= 0 || net->pitch[(size_t)t] ||
        net->pitch[(size_t)q.in] || numel_of(net, q.in) % k || xs[2] * xs[3] != q.ws[1] ||
        rows != xs[0] * xs[1])
      continue;
    bool single = true;
    for (size_t t2 = 0; t2 < nt; t2++) single = single && net->alias[t2] != t;
    for (size_t j = 0; j < nn; j++)
      if (j != i + 1)
        single = single && net->nodes[j].in != t && net->nodes[j].in2 != t &&
                 net->nodes[j].in3 != t;
    for (int32_t o : net->outputs) single = single && o != t;
    if (!single || gemm_takes_wide(rows, q.ws[1], 1) || !linear_nt_eligible(rows, q.ws[1], k, k) ||
        !qkv_attention_eligible(xs[0], xs[1], r.heads, r.dh, k))
      continue;
    net->qa_fused[i] = true;
    net->nostore[(size_t)t] = true;
  }
}

static void plan_pitch(qph_net* net) {
  const size_t nt = net->tptr.size();
  net->pitch.assign(nt, 0);
  std::vector<int> readers(nt, 0);
  std::vector<bool> aliased(nt, false);
  auto ok = [&](int32_t t) { return t >= 0 && (size_t)t < nt; };
  for (size_t t = 0; t < nt; t++)
    if (net->alias[t] >= 0 && (size_t)net->alias[t] < nt) aliased[(size_t)net->alias[t]] = true;
  for (const qph_node& n : net->nodes) {
    if (ok(n.in)) readers[(size_t)storage_of(net, n.in)]++;
    if (ok(n.in2)) readers[(size_t)storage_of(net, n.in2)]++;
    if (ok(n.in3)) readers[(size_t)storage_of(net, n.in3)]++;
  }
  for (int32_t o : net->outputs)
    if (ok(o)) readers[(size_t)storage_of(net, o)] += 1 << 20;   // outputs stay contiguous
  for (const qph_node& q : net->nodes) {
    if (q.op != QPH_OP_LINEAR || !ok(q.out) || !ok(q.in) || q.ws[0] <= 0) continue;
    const int32_t t = q.out;
    const int64_t nn = q.ws[1], rows = numel_of(net, q.in) / q.ws[0];
    if (net->alias[(size_t)t] >= 0 || aliased[(size_t)t] || readers[(size_t)t] != 1) continue;
    if (nn % 32 == 0 || !gemm_takes_wide(rows, nn, 1) || numel_of(net, t) != rows * nn) continue;
    bool soft = false;
    for (const qph_node& r : net->nodes)
      soft = soft || (r.in == t && r.op == QPH_OP_SOFTMAX_ARGMAX && r.ws[0] == nn);
    if (soft) net->pitch[(size_t)t] = (nn + 31) / 32 * 32;
  }
}

// The Add / Clip / Mul / Div export form of hardswish after a conv or
// linear with no activation, residual or placed output:
//   X = P(...); T1 = X + a; T2 = Clip(T1, +0.0, hi); T3 = X * T2; Y = T3 / d
// as the five consecutive nodes i .. i + 4, with X, T1, T2 and T3 read only
// inside the chain: node i then writes Y with activation kind 7 (the same
// four roundings in its epilogue) and the four nodes after it launch
// nothing.  Rewrites node i before the other planners see it.
static void plan_hardswish_clip(qph_net* net) {
  const size_t nn = net->nodes.size(), nt = net->tptr.size();
  net->absorb_after.assign(nn, 0);
  std::vector<int> readers(nt, 0);
  std::vector<bool> aliased(nt, false);
  for (const qph_node& n : net->nodes)
    for (int32_t t : {n.in, n.in2, n.in3})
      if (t >= 0) readers[(size_t)t]++;
  for (int32_t o : net->outputs) readers[(size_t)o] += 1000;
  for (size_t t = 0; t < nt; t++)
    if (net->alias[t] >= 0) aliased[t] = aliased[(size_t)net->alias[t]] = true;
  auto plain = [&](int32_t t) { return t >= 0 && !aliased[(size_t)t]; };
  for (size_t i = 0; i + 4 < nn; i++) {
    qph_node& p = net->nodes[i];
    const qph_node& a = net->nodes[i + 1];
    const qph_node& c = net->nodes[i + 2];
    const qph_node& m = net->nodes[i + 3];
    const qph_node& d = net->nodes[i + 4];
    if ((p.op != QPH_OP_CONV && p.op != QPH_OP_LINEAR) || p.act.kind != QPH_ACT_NONE ||
        p.in2 >= 0 || p.y_ctotal || p.y_coff || (p.y_up && p.y_up != 1) || p.trans_out ||
        net->head[i] || net->qa_fused[i])
      continue;
    const int32_t x = p.out;
    if (a.op != QPH_OP_BINARY || a.ws[0] != 0 || a.in != x || a.in2 >= 0) continue;
    if (c.op != QPH_OP_ACT || c.act.kind != QPH_ACT_CLIP || c.in != a.out ||
        __builtin_bit_cast(uint32_t, c.act.c1) != 0u)
      continue;
    if (m.op != QPH_OP_BINARY || m.ws[0] != 2 || m.in2 < 0 ||
        !((m.in == x && m.in2 == c.out) || (m.in == c.out && m.in2 == x)))
      continue;
    if (d.op != QPH_OP_BINARY || d.ws[0] != 3 || d.in != m.out || d.in2 >= 0 || d.ws[1] != 0)
      continue;
    const int32_t y = d.out;
    if (!plain(x) || !plain(a.out) || !plain(c.out) || !plain(m.out) || !plain(y) ||
        readers[(size_t)x] != 2 || readers[(size_t)a.out] != 1 || readers[(size_t)c.out] != 1 ||
        readers[(size_t)m.out] != 1)
      continue;
    bool same = true;
    for (int k = 0; k < 4; k++)
      same = same && net->shapes[4 * (size_t)x + k] == net->shapes[4 * (size_t)y + k];
    if (!same) continue;
    p.act.kind = QPH_ACT_HARDSWISH_CLIP;
    p.act.c1 = a.scale;
    p.act.c2 = c.act.c2;
    p.act.c3 = d.scale;
    p.out = y;
    net->absorb_after[i] = 4;
    i += 4;
  }
}

// Consecutive dense 3x3 convs (up to four) of which none reads another's
// output run as one launch of the direct kernel: the det neck's smoothing
// convs at 20, 40, 80 and 160 px each leave most of the chip idle alone.
static void plan_conv_groups(qph_net* net) {
  const size_t nn = net->nodes.size();
  net->plan.assign(nn, ConvArgs{});
  net->group_len.assign(nn, 1);
  std::vector<bool> ok(nn, false);
  for (size_t i = 0; i < nn; i++) {
    const qph_node& n = net->nodes[i];
    if (n.op != QPH_OP_CONV || !net->wk[i] || n.ws[2] != 3 || n.ws[3] != 3 || n.cp.group != 1)
      continue;
    qph_conv_epilogue ep{};
    ep.residual = n.in2 >= 0 ? net->tptr[n.in2] : nullptr;
    ep.res_up = n.res_up;
    ep.y_ctotal = n.y_ctotal;
    ep.y_coff = n.y_coff;
    ep.y_up = n.y_up;
    ep.trans_out = n.trans_out;
    ConvArgs pl{};
    const float* bias = n.bias >= 0 ? net->weights[n.bias] : nullptr;
    if (conv_dispatch(net->ctx, net->tptr[n.in], &net->shapes[4 * (size_t)n.in],
                      net->weights[n.w], net->wk[i], n.ws, bias, &n.cp, &n.act, &ep,
                      net->tptr[n.out], &pl) != QPH_OK)
      continue;
    if (!direct3x3_eligible(pl) || pl.c <= 4) continue;
    net->plan[i] = pl;
    ok[i] = true;
  }
  auto reads_output_of = [&](size_t a, size_t b) {
    const qph_node& na = net->nodes[a];
    const int32_t out = storage_of(net, net->nodes[b].out);
    return storage_of(net, na.in) == out || (na.in2 >= 0 && storage_of(net, na.in2) == out);
  };
  for (size_t i = 0; i < nn;) {
    size_t j = i;
    if (ok[i]) {
      j = i + 1;
      while (j < nn && j - i < 4 && ok[j]) {
        bool indep = true;
        for (size_t k = i; k < j && indep; k++)
          indep = !reads_output_of(j, k) && !reads_output_of(k, j);
        if (!indep) break;
        j++;
      }
      if (j - i >= 2) net->group_len[i] = (int)(j - i);
    }
    i = j > i ? j : i + 1;
  }
}

// A single 3x3 conv whose output only the conv-transpose pair after it reads
// (the det head: conv 96 -> 24, ReLU, then ConvT -> ConvT -> Sigmoid): one
// launch, the pair in the conv's epilogue (launch_conv3x3_convt).
static void plan_conv_convt(qph_net* net) {
  const size_t nn = net->nodes.size();
  net->convt_fused.assign(nn, false);
  std::vector<bool> grouped(nn, false);
  for (size_t i = 0; i < nn; i++)
    for (int k = 1; k < net->group_len[i] && i + (size_t)k < nn; k++) grouped[i + (size_t)k] = true;
  std::vector<int> readers(net->tptr.size(), 0);
  for (const qph_node& n : net->nodes) {
    readers[(size_t)storage_of(net, n.in)]++;
    if (n.in2 >= 0) readers[(size_t)storage_of(net, n.in2)]++;
    if (n.in3 >= 0) readers[(size_t)storage_of(net, n.in3)]++;
  }
  for (int32_t o : net->outputs) readers[(size_t)storage_of(net, o)]++;
  for (size_t i = 0; i + 1 < nn; i++) {
    const qph_node& d = net->nodes[i];
    const qph_node& q = net->nodes[i + 1];
    if (d.op != QPH_OP_CONV || q.op != QPH_OP_CONVT_PAIR_SIG || !net->plan[i].wk) continue;
    if (net->group_len[i] > 1 || grouped[i]) continue;
    if (storage_of(net, d.out) != d.out || storage_of(net, q.in) != d.out ||
        readers[(size_t)d.out] != 1)
      continue;
    const int64_t* xs = &net->shapes[4 * (size_t)q.in];
    if (xs[1] != 24 || q.ws[1] != 24 || q.w2 < 0) continue;
    if (!conv3x3_convt_eligible(net->plan[i])) continue;
    net->convt_fused[i] = true;
  }
}

// The deeper backbone blocks of the rec net (64..256 channels over a few
// rows of pixels) run channel-last: the depthwise conv as
// depthwise_cl_kernel, the 1x1 conv as a row-major GEMM (linear_nt_kernel:
// rows = pixels, k = channels; the ONNX [M][C][1][1] weight is already
// k-contiguous).  The fused kernel reloads every channel's halo for each
// 64-channel slice and the weight slice for each 16-pixel tile, which at
// these shapes costs far more than the intermediate round trip.
// Structure: a chain of (depthwise -> 1x1) blocks ending in a 1x1 conv that
// stores [n][pixels][M] (trans_out), every intermediate read only by the
// next node; the 1x1 conv feeding the chain's first depthwise stores
// channel-last too (trans_out).  A 1x1 conv joins only if its bias comes
// after the chain (rule 0 with M % 4 == 0: no seeded accumulators, as in the
// linear epilogue) and linear_nt_kernel takes the shape (C % 64 == 0).
static void plan_cl(qph_net* net) {
  const size_t nn = net->nodes.size(), nt = net->tptr.size();
  net->cl_dw.assign(nn, false);
  net->cl_pw.assign(nn, false);
  net->cl_out.assign(nn, false);
  std::vector<int> readers(nt, 0);
  for (const qph_node& n : net->nodes) {
    readers[(size_t)storage_of(net, n.in)]++;
    if (n.in2 >= 0) readers[(size_t)storage_of(net, n.in2)]++;
    if (n.in3 >= 0) readers[(size_t)storage_of(net, n.in3)]++;
  }
  for (int32_t o : net->outputs) readers[(size_t)storage_of(net, o)] += 1 << 20;
  auto producer = [&](int32_t t) {
    for (size_t i = 0; i < nn; i++)
      if (net->nodes[i].out == t) return (int)i;
    return -1;
  };
  auto plain_out = [&](const qph_node& q) {
    return q.in2 < 0 && q.res_up == 0 && (q.y_ctotal == 0 || q.y_ctotal == q.ws[0]) &&
           q.y_coff == 0 && q.y_up <= 1;
  };
  auto single = [&](int32_t t) { return storage_of(net, t) == t && readers[(size_t)t] == 1; };
  auto is_pw = [&](const qph_node& q) {
    return q.op == QPH_OP_CONV && q.cp.group == 1 && q.ws[2] == 1 && q.ws[3] == 1 &&
           q.cp.sh == 1 && q.cp.sw == 1 && q.cp.ph == 0 && q.cp.pw == 0 && q.cp.peh == 0 &&
           q.cp.pew == 0 && plain_out(q);
  };
  auto is_dw = [&](const qph_node& d) {
    const int64_t* xs = &net->shapes[4 * (size_t)d.in];
    const int64_t* ys = &net->shapes[4 * (size_t)d.out];
    return d.op == QPH_OP_CONV && d.cp.group > 1 && d.ws[1] == 1 && d.ws[0] == xs[1] &&
           (xs[1] & (xs[1] - 1)) == 0 && ys[0] * ys[2] <= 65535 &&
           d.cp.group == xs[1] && ((d.ws[2] == 3 && d.ws[3] == 3) || (d.ws[2] == 5 && d.ws[3] == 5)) &&
           d.trans_out == 0 && plain_out(d);
  };
  auto pw_ok = [&](const qph_node& q) {
    const int64_t* xs = &net->shapes[4 * (size_t)q.in];
    const int64_t m = q.ws[0], c = q.ws[1], px = xs[2] * xs[3];
    // (a run over one batch item, real_n = 1, may need the m-rows rule:
    // run_node seeds the chains then, see below)
    return pw_seed_rule(xs[0], m, px, c) == 0 && m % 4 == 0 &&
           linear_nt_eligible(xs[0] * px, m, c, c);
  };
  for (size_t e = 0; e < nn; e++) {
    const qph_node& last = net->nodes[e];
    if (!is_pw(last) || !last.trans_out || !pw_ok(last)) continue;
    // walk back: blocks (dw[k], pw[k]), pw[0] = e; feeder = the 1x1 conv
    // before the chain's first depthwise
    std::vector<int> dws, pws;
    int p = (int)e, feeder = -1;
    while (true) {
      const int d = producer(net->nodes[(size_t)p].in);
      if (d < 0 || !is_dw(net->nodes[(size_t)d]) || !single(net->nodes[(size_t)d].out)) break;
      const int x = producer(net->nodes[(size_t)d].in);
      if (x < 0 || !is_pw(net->nodes[(size_t)x]) || net->nodes[(size_t)x].trans_out ||
          !single(net->nodes[(size_t)x].out))
        break;
      dws.push_back(d);
      pws.push_back(p);
      if (!pw_ok(net->nodes[(size_t)x])) {
        feeder = x;
        break;
      }
      p = x;
      feeder = x;
    }
    // the last block taken needs its depthwise input channel-last: the
    // feeder stores it so; a chain whose walk stopped on a 1x1 conv that
    // joined as a block gives that conv back as the feeder
    if (!dws.empty() && feeder >= 0 && feeder == pws.back()) {
      dws.pop_back();
      pws.pop_back();
    }
    if (dws.empty() || feeder < 0) continue;
    for (size_t k = 0; k < dws.size(); k++) {
      net->cl_dw[(size_t)dws[k]] = true;
      net->cl_pw[(size_t)pws[k]] = true;
    }
    net->cl_out[(size_t)feeder] = true;
  }
}

// Depthwise conv node i feeding 1x1 conv node i + 1 (the backbone blocks):
// one launch, the depthwise output kept on chip.  Needs plain outputs (the
// 1x1 may store transposed), no residuals, and no other reader of the
// intermediate tensor.  The 1x1 weights are repacked k-major here.
static int plan_dwpw(qph_net* net) {
  const size_t nn = net->nodes.size();
  net->dwpw.assign(nn, DwPwArgs{});
  net->fused.assign(nn, false);
  std::vector<int> readers(net->tptr.size(), 0);
  for (const qph_node& n : net->nodes) {
    readers[(size_t)storage_of(net, n.in)]++;
    if (n.in2 >= 0) readers[(size_t)storage_of(net, n.in2)]++;
    if (n.in3 >= 0) readers[(size_t)storage_of(net, n.in3)]++;
  }
  for (int32_t o : net->outputs) readers[(size_t)storage_of(net, o)]++;
  for (size_t i = 0; i + 1 < nn; i++) {
    if (i > 0 && net->fused[i - 1]) continue;
    const qph_node& d = net->nodes[i];
    const qph_node& q = net->nodes[i + 1];
    if (d.op != QPH_OP_CONV || q.op != QPH_OP_CONV) continue;
    const int64_t* xs = &net->shapes[4 * (size_t)d.in];
    const bool dw = d.cp.group > 1 && d.ws[1] == 1 && d.ws[0] == xs[1] && d.cp.group == xs[1] &&
                    d.in2 < 0 && d.res_up == 0 && d.trans_out == 0 &&
                    (d.y_ctotal == 0 || d.y_ctotal == d.ws[0]) && d.y_coff == 0 && d.y_up <= 1;
    const bool pw = q.cp.group == 1 && q.ws[2] == 1 && q.ws[3] == 1 && q.cp.sh == 1 &&
                    q.cp.sw == 1 && q.cp.ph == 0 && q.cp.pw == 0 && q.cp.peh == 0 &&
                    q.cp.pew == 0 && q.in2 < 0 && q.res_up == 0 &&
                    (q.y_ctotal == 0 || q.y_ctotal == q.ws[0]) && q.y_coff == 0 && q.y_up <= 1;
    if (!dw || !pw || q.in != d.out || q.ws[1] != d.ws[0]) continue;
    if (net->cl_dw[i] || net->cl_pw[i + 1]) continue;
    if (storage_of(net, d.out) != d.out || readers[(size_t)d.out] != 1) continue;
    int64_t ys[4];
    if (qph_conv2d_out_shape(xs, d.ws, &d.cp, ys) != QPH_OK) continue;
    DwPwArgs f{};
    f.x = net->tptr[d.in]; f.n = xs[0]; f.c = xs[1]; f.h = xs[2]; f.w = xs[3];
    f.wd = net->weights[d.w]; f.bd = d.bias >= 0 ? net->weights[d.bias] : nullptr;
    f.kh = d.ws[2]; f.kw = d.ws[3]; f.sh = d.cp.sh; f.sw = d.cp.sw; f.ph = d.cp.ph; f.pw = d.cp.pw;
    f.oh = ys[2]; f.ow = ys[3];
    f.act_d = make_act(&d.act);
    f.bp = q.bias >= 0 ? net->weights[q.bias] : nullptr;
    f.m = q.ws[0];
    // the 1x1 path's bias-placement rule (as conv_dispatch picks it)
    f.seed_rule = pw_seed_rule(f.n, f.m, f.oh * f.ow, f.c);
    f.act_p = make_act(&q.act);
    f.trans_out = q.trans_out || net->cl_out[i + 1];
    f.y = net->tptr[q.out];
    if (!dwpw_eligible(f)) continue;
    // the stem conv in front (3 -> c channels, 3x3 stride 2 pad 1), its
    // output read by this depthwise only: computed inside the launch
    size_t at = i;
    if (i > 0 && storage_of(net, d.in) == d.in && readers[(size_t)d.in] == 1 &&
        !(i > 1 && net->fused[i - 2])) {
      const qph_node& st = net->nodes[i - 1];
      const int64_t* ss = &net->shapes[4 * (size_t)st.in];
      const bool sok = st.op == QPH_OP_CONV && st.out == d.in && st.cp.group == 1 && ss[1] == 3 &&
                       st.ws[1] == 3 && st.ws[0] == f.c && st.ws[2] == 3 && st.ws[3] == 3 &&
                       st.cp.sh == 2 && st.cp.sw == 2 && st.cp.ph == 1 && st.cp.pw == 1 &&
                       st.cp.dh <= 1 && st.cp.dw <= 1 && st.in2 < 0 && st.res_up == 0 &&
                       st.trans_out == 0 && !net->cl_out[i - 1] &&
                       (st.y_ctotal == 0 || st.y_ctotal == st.ws[0]) && st.y_coff == 0 &&
                       st.y_up <= 1 && net->group_len[i - 1] <= 1;
      if (sok) {
        DwPwArgs g = f;
        g.stem = 1;
        g.xin = net->tptr[st.in]; g.hin = ss[2]; g.win = ss[3];
        g.wst = net->weights[st.w]; g.bst = st.bias >= 0 ? net->weights[st.bias] : nullptr;
        g.act_s = make_act(&st.act);
        if (ss[0] == f.n && dwpw_stem_eligible(g)) {
          f = g;
          at = i - 1;
        }
      }
    }
    float* wk = nullptr;
    QPH_TRY(hip_check(hipMalloc((void**)&wk, (size_t)dense_conv_wk_floats(f.m, f.c, 1, 1) * 4),
                      "hipMalloc(repacked 1x1 weight)"));
    net->wk[i + 1] = wk;
    QPH_TRY(launch_repack_conv_w_taps(net->weights[q.w], f.m, f.c, 1, wk, net->ctx->stream));
    f.wk = wk;
    net->dwpw[at] = f;
    net->fused[at] = true;
  }
  return QPH_OK;
}

// The output of node i is [n, c, h, w], or channels [y_coff, y_coff + c) of a
// [n, y_ctotal, h, w] tensor (a Concat slot).
static int check_slot(const qph_net* net, size_t i, const qph_node& q, int64_t n, int64_t c,
                      int64_t h, int64_t w) {
  const int64_t* ys = &net->shapes[4 * (size_t)q.out];
  const int64_t ct = q.y_ctotal ? q.y_ctotal : c;
  if (q.y_coff < 0 || q.y_coff + c > ct || ys[0] != n || ys[1] != ct || ys[2] != h || ys[3] != w)
    return fail(QPH_EINVAL, node_name(i, q) + ": output shape / Concat slot mismatch");
  return QPH_OK;
}

static int validate_node(qph_net* net, size_t i, const int64_t* wsizes, int32_t nw) {
  const qph_node& n = net->nodes[i];
  QPH_TRY(check_tensor(net, n.in, false, i, n, "input"));
  // a softmax node may export pairs only (out = -1, the rec_argmax_pairs
  // exit of device.rs:160-165)
  QPH_TRY(check_tensor(net, n.out, n.op == QPH_OP_SOFTMAX_ARGMAX, i, n, "output"));
  QPH_TRY(check_tensor(net, n.in2, true, i, n, "second input"));
  QPH_TRY(check_tensor(net, n.in3, true, i, n, "third input"));
  QPH_TRY(check_tensor(net, n.out2, true, i, n, "second output"));
  for (int32_t wi : {n.w, n.bias, n.w2})
    if (wi >= nw) return fail(QPH_EINVAL, node_name(i, n) + ": bad weight index");
  if (!act_valid(&n.act)) return fail(QPH_EINVAL, node_name(i, n) + ": bad activation");
  const int64_t* xs = &net->shapes[4 * (size_t)n.in];
  const int64_t* ys = &net->shapes[4 * (size_t)n.out];
  auto wsize = [&](int32_t wi) { return wi >= 0 ? wsizes[wi] : (int64_t)-1; };
  switch (n.op) {
    case QPH_OP_CONV: {
      if (n.w < 0) return fail(QPH_EINVAL, node_name(i, n) + ": conv without weight");
      int64_t os[4];
      int rc = qph_conv2d_out_shape(xs, n.ws, &n.cp, os);
      if (rc) return fail(rc, node_name(i, n) + ": " + qph_last_error());
      if (wsize(n.w) != n.ws[0] * n.ws[1] * n.ws[2] * n.ws[3])
        return fail(QPH_EINVAL, node_name(i, n) + ": weight size mismatch");
      if (n.bias >= 0 && wsize(n.bias) != n.ws[0])
        return fail(QPH_EINVAL, node_name(i, n) + ": bias size mismatch");
      const int64_t up = n.y_up ? n.y_up : 1;
      const int64_t ctot = n.y_ctotal ? n.y_ctotal : os[1];
      int64_t want[4] = {os[0], ctot, os[2] * up, os[3] * up};
      if (n.trans_out) {
        if (numel_of(net, n.out) != os[0] * os[1] * os[2] * os[3])
          return fail(QPH_EINVAL, node_name(i, n) + ": output size mismatch");
      } else {
        for (int d = 0; d < 4; d++)
          if (ys[d] != want[d])
            return fail(QPH_EINVAL, node_name(i, n) + ": output shape mismatch");
      }
      if (n.in2 >= 0) {
        const int64_t* rs = &net->shapes[4 * (size_t)n.in2];
        int64_t f = n.res_up == 2 ? 2 : 1;
        if (rs[0] != os[0] || rs[1] != os[1] || rs[2] * f != os[2] || rs[3] * f != os[3])
          return fail(QPH_EINVAL, node_name(i, n) + ": residual shape mismatch");
      }
      return QPH_OK;
    }
    case QPH_OP_CONVT_PAIR_SIG:
    case QPH_OP_CONVT: {
      if (n.w < 0 || n.ws[0] != xs[1] || n.ws[2] != 2 || n.ws[3] != 2)
        return fail(QPH_EUNSUPPORTED, node_name(i, n) + ": ConvTranspose needs [C,M,2,2]");
      int64_t f = 2, m = n.ws[1];
      if (n.op == QPH_OP_CONVT_PAIR_SIG) {
        if (n.w2 < 0 || n.w2s[0] != n.ws[1] || n.w2s[1] != 1 || n.w2s[2] != 2 || n.w2s[3] != 2)
          return fail(QPH_EUNSUPPORTED, node_name(i, n) + ": second ConvTranspose needs [M,1,2,2]");
        if (xs[1] > 64 || n.ws[1] > 64)
          return fail(QPH_EUNSUPPORTED, node_name(i, n) + ": ConvT pair needs C, M <= 64");
        f = 4;
        m = 1;
      }
      if (ys[0] != xs[0] || ys[1] != m || ys[2] != f * xs[2] || ys[3] != f * xs[3])
        return fail(QPH_EINVAL, node_name(i, n) + ": output shape mismatch");
      return QPH_OK;
    }
    case QPH_OP_LINEAR: {
      if (n.w < 0 || wsize(n.w) != n.ws[0] * n.ws[1])
        return fail(QPH_EINVAL, node_name(i, n) + ": linear weight [K,N] mismatch");
      if (numel_of(net, n.in) % n.ws[0])
        return fail(QPH_EINVAL, node_name(i, n) + ": input not a multiple of K");
      int64_t rows = numel_of(net, n.in) / n.ws[0];
      if (numel_of(net, n.out) != rows * n.ws[1])
        return fail(QPH_EINVAL, node_name(i, n) + ": output size mismatch");
      if (n.bias >= 0 && wsize(n.bias) != n.ws[1])
        return fail(QPH_EINVAL, node_name(i, n) + ": bias size mismatch");
      if (n.in2 >= 0 && numel_of(net, n.in2) != rows * n.ws[1])
        return fail(QPH_EINVAL, node_name(i, n) + ": residual size mismatch");
      return QPH_OK;
    }
    case QPH_OP_LAYERNORM:
      if (n.w < 0 || n.bias < 0 || n.ws[0] <= 0 || wsize(n.w) != n.ws[0] ||
          wsize(n.bias) != n.ws[0] || numel_of(net, n.in) % n.ws[0] ||
          numel_of(net, n.out) != numel_of(net, n.in))
        return fail(QPH_EINVAL, node_name(i, n) + ": layernorm shapes");
      if (n.ws[0] > 4096)
        return fail(QPH_EUNSUPPORTED, node_name(i, n) + ": layernorm rows wider than 4096");
      return QPH_OK;
    case QPH_OP_ATTENTION:
      if (xs[2] * xs[3] != 3 * n.heads * n.dh || n.dh > 64 || xs[1] > 256 ||
          numel_of(net, n.out) != xs[0] * xs[1] * n.heads * n.dh)
        return fail(QPH_EINVAL, node_name(i, n) + ": attention shapes");
      if ((2 * xs[1] * (n.dh + 1) + 4 * (xs[1] + n.dh)) * 4 > 64 * 1024)
        return fail(QPH_EUNSUPPORTED, node_name(i, n) + ": attention too large for LDS");
      return QPH_OK;
    case QPH_OP_SOFTMAX_ARGMAX:
      if (n.out < 0 && n.out2 < 0)
        return fail(QPH_EINVAL, node_name(i, n) + ": softmax without an output");
      if (n.ws[0] <= 0 || n.ws[0] >= (1ll << 31) || numel_of(net, n.in) % n.ws[0] ||
          (n.out >= 0 && numel_of(net, n.out) != numel_of(net, n.in)))
        return fail(QPH_EINVAL, node_name(i, n) + ": softmax row width / probs size");
      if (n.out2 >= 0 && numel_of(net, n.out2) != 2 * (numel_of(net, n.in) / n.ws[0]))
        return fail(QPH_EINVAL, node_name(i, n) + ": pairs size mismatch");
      return QPH_OK;
    case QPH_OP_ACT:
      if (numel_of(net, n.out) != numel_of(net, n.in))
        return fail(QPH_EINVAL, node_name(i, n) + ": size mismatch");
      return QPH_OK;
    case QPH_OP_GAP:
      if (ys[0] != xs[0] || ys[1] != xs[1] || ys[2] != 1 || ys[3] != 1)
        return fail(QPH_EINVAL, node_name(i, n) + ": GlobalAveragePool output must be [N,C,1,1]");
      return QPH_OK;
    case QPH_OP_MUL_ADD_SCALE: {
      QPH_TRY(check_tensor(net, n.in3, false, i, n, "gate"));
      // in2 = -1: the gate Mul alone (an SE block without a residual)
      const int64_t g = numel_of(net, n.in3);
      if ((n.in2 >= 0 && numel_of(net, n.in2) != numel_of(net, n.in)) ||
          (g != xs[1] && g != xs[0] * xs[1]))
        return fail(QPH_EINVAL, node_name(i, n) + ": MulAddScale shapes");
      QPH_TRY(check_slot(net, i, n, xs[0], xs[1], xs[2], xs[3]));
      return QPH_OK;
    }
    case QPH_OP_POOL: {
      if (n.ws[2] <= 0 || n.ws[3] <= 0 || n.cp.sh <= 0 || n.cp.sw <= 0 || n.cp.ph < 0 ||
          n.cp.pw < 0 || n.cp.peh < 0 || n.cp.pew < 0)
        return fail(QPH_EINVAL, node_name(i, n) + ": pool window");
      int64_t oh, ow;
      pool2d_out_hw(xs[2], xs[3], n.ws[2], n.ws[3], n.cp.sh, n.cp.sw, n.cp.ph, n.cp.pw, n.cp.peh,
                    n.cp.pew, &oh, &ow);
      QPH_TRY(check_slot(net, i, n, xs[0], xs[1], oh, ow));
      return QPH_OK;
    }
    case QPH_OP_RESIZE:
      if (n.ws[0] != 0 && n.ws[0] != 1)
        return fail(QPH_EUNSUPPORTED, node_name(i, n) + ": resize mode must be nearest or bilinear");
      if (n.ws[0] == 0 && (n.y_ctotal || n.y_coff))
        return fail(QPH_EUNSUPPORTED, node_name(i, n) + ": nearest resize into a Concat slot");
      QPH_TRY(check_slot(net, i, n, xs[0], xs[1], ys[2], ys[3]));
      return QPH_OK;
    case QPH_OP_TRANSPOSE: {
      int seen = 0;
      for (int d = 0; d < 4; d++) {
        if (n.ws[d] < 0 || n.ws[d] > 3 || (seen >> n.ws[d]) & 1)
          return fail(QPH_EINVAL, node_name(i, n) + ": perm is not a permutation of 0..3");
        seen |= 1 << n.ws[d];
        if (ys[d] != xs[n.ws[d]])
          return fail(QPH_EINVAL, node_name(i, n) + ": transpose output shape");
      }
      return QPH_OK;
    }
    case QPH_OP_COPY_SLOT:
      if (!n.y_ctotal) return fail(QPH_EINVAL, node_name(i, n) + ": copy slot needs y_ctotal");
      QPH_TRY(check_slot(net, i, n, xs[0], xs[1], xs[2], xs[3]));
      return QPH_OK;
    case QPH_OP_BINARY:
      // Pow (op 4) goes through libm powf on the reference's CPU path
      // (elementwise.rs:32-34), with ulp-level differences across libms
      if (n.ws[0] < 0 || n.ws[0] > 3)
        return fail(QPH_EUNSUPPORTED, node_name(i, n) + ": binary op must be Add, Sub, Mul or Div");
      if (n.ws[1] != 0 && n.ws[1] != 1)
        return fail(QPH_EINVAL, node_name(i, n) + ": ws[1] (scalar first) must be 0 or 1");
      if ((n.in2 >= 0 && numel_of(net, n.in2) != numel_of(net, n.in)) ||
          numel_of(net, n.out) != numel_of(net, n.in))
        return fail(QPH_EINVAL, node_name(i, n) + ": binary operands and output differ in size");
      if (n.y_ctotal || n.y_coff)
        return fail(QPH_EUNSUPPORTED, node_name(i, n) + ": binary op into a Concat slot");
      return QPH_OK;
    default:
      return fail(QPH_EUNSUPPORTED, node_name(i, n) + ": unsupported op");
  }
}

// Every node in order, fused launches where planned.  With profiling on,
// an event precedes each node; the nodes a fused launch covers after its
// first get their events right after it (so their time reads 0).
// The FPN top-down laterals: four consecutive 1x1 convs to the same M with
// no activation, L5 = conv(C5), L4 = conv(C4) + up2(L5), L3 = conv(C3) +
// up2(L4), L2 = conv(C2) + up2(L3), each a plain single-node launch.  The
// three coarse GEMMs do not depend on one another without their residuals:
// one grouped launch computes conv(C5) into L5 and conv(C4), conv(C3) into
// net-owned buffers, one elementwise pass forms L4 and L3 (the same Adds),
// and L2 runs as before.  Three launches instead of four, the coarse GEMMs
// side by side instead of one after another.  (L2's GEMM forming its
// residual from the raw laterals itself, with the elementwise pass in its
// launch, made two launches but a slower step with two pages in flight.)
static int plan_fpn(qph_net* net) {
  const size_t nn = net->nodes.size();
  net->fpn.assign(nn, false);
  // nodes that start a single-node launch in run_all's stepping
  std::vector<bool> single(nn, false);
  for (size_t i = 0; i < nn;) {
    size_t step = 1;
    if (net->group_len[i] > 1) step = (size_t)net->group_len[i];
    else if (net->head[i] || net->convt_fused[i] || net->qa_fused[i]) step = 2;
    else if (net->fused[i]) step = net->dwpw[i].stem ? 3 : 2;
    step += (size_t)net->absorb_after[i + step - 1];
    single[i] = step == 1 && !net->cl_dw[i] && !net->cl_pw[i] && !net->cl_out[i];
    i += step;
  }
  auto lateral = [&](size_t i) {
    const qph_node& n = net->nodes[i];
    return n.op == QPH_OP_CONV && single[i] && conv_is_pointwise(n.ws, n.cp) &&
           n.cp.group == 1 && n.act.kind == QPH_ACT_NONE && !n.y_ctotal && !n.y_coff &&
           (!n.y_up || n.y_up == 1) && !n.trans_out && n.bias >= 0 &&
           storage_of(net, n.out) == n.out && net->alias[(size_t)n.out] < 0;
  };
  for (size_t i = 0; i + 3 < nn; i++) {
    bool ok = true;
    for (size_t k = 0; k < 4 && ok; k++) ok = lateral(i + k);
    if (!ok) continue;
    const qph_node* q[4] = {&net->nodes[i], &net->nodes[i + 1], &net->nodes[i + 2],
                            &net->nodes[i + 3]};
    if (q[0]->in2 >= 0) continue;
    for (int k = 1; k < 4 && ok; k++)
      ok = q[k]->in2 == q[k - 1]->out && q[k]->res_up == 2 && q[k]->ws[0] == q[0]->ws[0];
    if (!ok) continue;
    const int64_t* s3 = &net->shapes[4 * (size_t)q[2]->out];
    if (s3[2] % 4 || s3[3] % 4) continue;
    // the grouped GEMMs at the full batch take the pointwise group kernel
    for (int k = 0; k < 3 && ok; k++) {
      GemmArgs g{};
      const qph_node& n = *q[k];
      Act a = make_act(&n.act);
      pointwise_gemm_args(net->tptr[n.in], &net->shapes_full[4 * (size_t)n.in],
                          net->weights[n.w], n.ws, net->weights[n.bias], a, net->tptr[n.out], &g);
      ok = pw_group_eligible(g);
    }
    if (!ok) continue;
    float* t4 = nullptr;
    float* t3 = nullptr;
    QPH_TRY(hip_check(hipMalloc((void**)&t4, (size_t)numel_of(net, q[1]->out) * 4), "hipMalloc(fpn)"));
    net->fpn_tmp.push_back(t4);
    QPH_TRY(hip_check(hipMalloc((void**)&t3, (size_t)numel_of(net, q[2]->out) * 4), "hipMalloc(fpn)"));
    net->fpn_tmp.push_back(t3);
    net->fpn[i] = true;
    net->fpn_t4.resize(nn, nullptr);
    net->fpn_t3.resize(nn, nullptr);
    net->fpn_t4[i] = t4;
    net->fpn_t3[i] = t3;
    i += 3;
  }
  return QPH_OK;
}

static int run_fpn(qph_net* net, size_t i) {
  hipStream_t s = net->ctx->stream;
  const qph_node* q[4] = {&net->nodes[i], &net->nodes[i + 1], &net->nodes[i + 2],
                          &net->nodes[i + 3]};
  float* t4 = net->fpn_t4[i];
  float* t3 = net->fpn_t3[i];
  float* outs[3] = {net->tptr[q[0]->out], t4, t3};
  GemmArgs g[3];
  for (int k = 0; k < 3; k++) {
    const qph_node& n = *q[k];
    Act a = make_act(&n.act);
    pointwise_gemm_args(net->tptr[n.in], &net->shapes[4 * (size_t)n.in], net->weights[n.w], n.ws,
                        net->weights[n.bias], a, outs[k], &g[k]);
  }
  int rc = launch_pw_group(g, 3, s);
  if (rc != QPH_OK) return fail(rc, node_name(i, *q[0]) + ": " + qph_last_error());
  const int64_t* s3 = &net->shapes[4 * (size_t)q[2]->out];
  rc = launch_fpn_topdown(t4, net->tptr[q[0]->out], t3, net->tptr[q[1]->out],
                          net->tptr[q[2]->out], s3[0], s3[1], s3[2], s3[3], s);
  if (rc != QPH_OK) return fail(rc, node_name(i + 1, *q[1]) + ": " + qph_last_error());
  rc = run_node(net, i + 3);
  if (rc != QPH_OK) return fail(rc, node_name(i + 3, *q[3]) + ": " + qph_last_error());
  return QPH_OK;
}

static int run_all(qph_net* net) {
  hipStream_t s = net->ctx->stream;
  const size_t nn = net->nodes.size();
  for (size_t i = 0; i < nn;) {
    if (net->profiling) QPH_TRY_HIP(hipEventRecord(net->ev[i], s));
    size_t step = 1;
    if (net->group_len[i] > 1) {
      ConvArgs grp[4];
      for (int k = 0; k < net->group_len[i] && k < 4; k++) {
        grp[k] = net->plan[i + (size_t)k];
        grp[k].n = net->real_n;
      }
      QPH_TRY(launch_dense_conv_group(grp, net->group_len[i], s));
      step = (size_t)net->group_len[i];
    } else if (net->head[i]) {
      const qph_node& q = net->nodes[i];
      const qph_node& r = net->nodes[i + 1];
      const int64_t k = q.ws[0], nn = q.ws[1];
      const float* w = net->wk[i] ? net->wk[i] : net->weights[q.w];
      const int64_t ldb = net->wk[i] ? (nn + 3) / 4 * 4 : nn;
      const int rc = launch_head_argmax(net->tptr[q.in], numel_of(net, q.in) / k, k, w, ldb, nn,
                                        q.bias >= 0 ? net->weights[q.bias] : nullptr,
                                        net->head_part[i], net->tptr[r.out2], s);
      if (rc != QPH_OK) return fail(rc, node_name(i, q) + ": " + qph_last_error());
      step = 2;
    } else if (net->fpn[i]) {
      QPH_TRY(run_fpn(net, i));
      step = 4;
    } else if (net->convt_fused[i]) {
      const qph_node& q = net->nodes[i + 1];
      ConvArgs a = net->plan[i];
      a.n = net->real_n;
      const int rc = launch_conv3x3_convt(a, net->weights[q.w], net->weights[q.w2],
                                          net->tptr[q.out], s);
      if (rc != QPH_OK) return fail(rc, node_name(i, net->nodes[i]) + ": " + qph_last_error());
      step = 2;
    } else if (net->fused[i]) {
      DwPwArgs f = net->dwpw[i];
      f.n = net->real_n;
      f.seed_rule = pw_seed_rule(f.n, f.m, f.oh * f.ow, f.c);
      QPH_TRY(launch_dwpw(f, s));
      step = net->dwpw[i].stem ? 3 : 2;
    } else if (net->qa_fused[i]) {
      const qph_node& q = net->nodes[i];
      const qph_node& r = net->nodes[i + 1];
      const int64_t* xs = &net->shapes[4 * (size_t)q.out];
      const int rc = launch_qkv_attention(net->tptr[q.in], net->wt[i],
                                          q.bias >= 0 ? net->weights[q.bias] : nullptr, xs[0],
                                          xs[1], r.heads, r.dh, q.ws[0], r.scale,
                                          net->tptr[r.out], s);
      if (rc != QPH_OK) return fail(rc, node_name(i, q) + ": " + qph_last_error());
      step = 2;
    } else {
      const int rc = run_node(net, i);
      if (rc != QPH_OK) return fail(rc, node_name(i, net->nodes[i]) + ": " + qph_last_error());
    }
    step += (size_t)net->absorb_after[i + step - 1];
    if (net->profiling)
      for (size_t k = i + 1; k < i + step; k++) QPH_TRY_HIP(hipEventRecord(net->ev[k], s));
    i += step;
  }
  return QPH_OK;
}

// Records the whole kernel sequence for the current real_n into a HIP
// graph (nothing executes).  Every launcher validates its arguments as it
// records, so a node that no kernel takes fails here, at create time (or
// at the first run with a new real_n), naming the node.
static int capture(qph_net* net) {
  hipStream_t s = net->ctx->stream;
  const size_t r = (size_t)net->real_n;
  QPH_TRY_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
  int rc = run_all(net);
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(s, &g);
  if (rc != QPH_OK) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  QPH_TRY_HIP(e);
  hipGraphExec_t x = nullptr;
  e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g);
    return hip_check(e, "hipGraphInstantiate");
  }
  net->graphs[r] = g;
  net->execs[r] = x;
  return QPH_OK;
}

// The graph of the current real_n, captured on first use.
static int launch_graph(qph_net* net) {
  const size_t r = (size_t)net->real_n;
  if (!net->execs[r]) QPH_TRY(capture(net));
  QPH_TRY_HIP(hipGraphLaunch(net->execs[r], net->ctx->stream));
  return QPH_OK;
}

// Batch-major tensors: the input, and every output of a node that reads a
// batch-major tensor (each op maps batch item b of its inputs to batch
// item b of its outputs).  A run over real_n items cuts their first
// dimension to real_n; that is a batch cut only when the first dimension
// is the batch, which real_n requires of every batch-major tensor.
static void mark_batch_major(qph_net* net) {
  const size_t nt = net->shapes_full.size() / 4;
  net->batch_major.assign(nt, false);
  net->batch_major[0] = true;
  auto bm = [&](int32_t t) { return t >= 0 && (size_t)t < nt && net->batch_major[(size_t)t]; };
  for (const qph_node& n : net->nodes) {
    if (!(bm(n.in) || bm(n.in2) || bm(n.in3))) continue;
    if (n.out >= 0 && (size_t)n.out < nt) net->batch_major[(size_t)n.out] = true;
    if (n.out2 >= 0 && (size_t)n.out2 < nt) net->batch_major[(size_t)n.out2] = true;
  }
  for (size_t t = 0; t < nt; t++)
    if (net->alias[t] >= 0 && (size_t)net->alias[t] < nt && net->batch_major[t])
      net->batch_major[(size_t)net->alias[t]] = true;
}

static void set_eff_shapes(qph_net* net) {
  net->shapes = net->shapes_full;
  for (size_t t = 0; t < net->batch_major.size(); t++)
    if (net->batch_major[t]) net->shapes[4 * t] = net->real_n;
}

static void release(qph_net* net) {
  if (!net) return;
  (void)hipStreamSynchronize(net->ctx->stream);
  for (size_t r = 0; r < net->execs.size(); r++) {
    if (net->execs[r]) (void)hipGraphExecDestroy(net->execs[r]);
    if (net->graphs[r]) (void)hipGraphDestroy(net->graphs[r]);
  }
  for (auto e : net->ev) (void)hipEventDestroy(e);
  if (net->done) (void)hipEventDestroy(net->done);
  if (net->in_stage) (void)hipHostFree(net->in_stage);
  for (float* p : net->out_stage)
    if (p) (void)hipHostFree(p);
  for (float* p : net->weights) (void)hipFree(p);
  for (float* p : net->wk)
    if (p) (void)hipFree(p);
  for (float* p : net->head_part)
    if (p) (void)hipFree(p);
  for (float* p : net->fpn_tmp)
    if (p) (void)hipFree(p);
  for (float* p : net->wt)
    if (p) (void)hipFree(p);
  if (net->arena) (void)hipFree(net->arena);
  delete net;
}

extern "C" {

QPH_API int qph_net_create(qph_ctx* ctx, const qph_net_spec* spec,
                           const float* const* weights_host, qph_net** out) {
  if (!spec || !out) return fail(QPH_EINVAL, "net_create: NULL argument");
  *out = nullptr;
  // the spec is checked before anything touches the device
  if (spec->n_tensors <= 0 || spec->n_nodes <= 0 || !spec->shapes || !spec->nodes)
    return fail(QPH_EINVAL, "net_create: empty graph");
  if (spec->n_weights > 0 && (!weights_host || !spec->weight_sizes))
    return fail(QPH_EINVAL, "net_create: missing weights");
  if (spec->n_outputs < 0 || (spec->n_outputs > 0 && !spec->outputs))
    return fail(QPH_EINVAL, "net_create: missing output list");
  for (int32_t o = 0; o < spec->n_outputs; o++)
    if (spec->outputs[o] < 0 || spec->outputs[o] >= spec->n_tensors)
      return fail(QPH_EINVAL, "net_create: output " + std::to_string(o) + " names tensor " +
                                  std::to_string(spec->outputs[o]) + " of " +
                                  std::to_string(spec->n_tensors));
  for (int32_t wi = 0; wi < spec->n_weights; wi++)
    if (spec->weight_sizes[wi] < 0 || (spec->weight_sizes[wi] > 0 && !weights_host[wi]))
      return fail(QPH_EINVAL, "net_create: weight " + std::to_string(wi) + " missing");
  if (!ctx) return fail(QPH_EINVAL, "net_create: NULL context");
  qph_net* net = new qph_net();
  net->ctx = ctx;
  net->arena = nullptr;
  net->arena_bytes = 0;
  net->profiling = false;
  net->prof_runs = 0;
  net->in_stage = nullptr;
  net->done = nullptr;
  net->inflight = false;
  net->nodes.assign(spec->nodes, spec->nodes + spec->n_nodes);
  net->shapes_full.assign(spec->shapes, spec->shapes + 4 * (size_t)spec->n_tensors);
  net->shapes = net->shapes_full;
  net->batch = net->shapes_full[0];
  net->real_n = net->batch;
  net->alias.assign((size_t)spec->n_tensors, -1);
  if (spec->alias) net->alias.assign(spec->alias, spec->alias + spec->n_tensors);
  if (spec->n_outputs > 0 && spec->outputs)
    net->outputs.assign(spec->outputs, spec->outputs + spec->n_outputs);
  net->out_stage.assign(net->outputs.size(), nullptr);
  net->tptr.assign((size_t)spec->n_tensors, nullptr);
  net->wk.assign(net->nodes.size(), nullptr);
  net->wt.assign(net->nodes.size(), nullptr);
  int rc = QPH_OK;
  auto bail = [&](int code) {
    std::string msg = qph_last_error();
    release(net);
    set_error(msg);
    return code;
  };
  // tensors: one arena, 256-byte aligned slots; aliases share their target
  for (int32_t t = 0; t < spec->n_tensors; t++) {
    for (int d = 0; d < 4; d++)
      if (net->shapes[4 * t + d] <= 0) {
        fail(QPH_EINVAL, "net_create: tensor " + std::to_string(t) + " has an empty shape");
        return bail(QPH_EINVAL);
      }
    int32_t a = net->alias[t];
    if (a >= spec->n_tensors || a == t || (a >= 0 && net->alias[a] >= 0)) {
      fail(QPH_EINVAL, "net_create: bad alias of tensor " + std::to_string(t));
      return bail(QPH_EINVAL);
    }
  }
  if (net->batch <= 0 || net->batch > (1 << 20)) {
    fail(QPH_EINVAL, "net_create: input batch dimension out of range");
    return bail(QPH_EINVAL);
  }
  mark_batch_major(net);
  net->graphs.assign((size_t)net->batch + 1, nullptr);
  net->execs.assign((size_t)net->batch + 1, nullptr);
  plan_fused_head(net, spec->flags);
  plan_pitch(net);
  plan_qkv_attention(net, spec->flags);
  std::vector<size_t> off((size_t)spec->n_tensors, 0);
  for (int32_t t = 0; t < spec->n_tensors; t++) {
    if (net->alias[t] >= 0) continue;
    off[t] = net->arena_bytes;
    if (net->nostore[(size_t)t]) continue;
    int64_t words = numel_of(net, t);
    if (net->pitch[(size_t)t]) {
      const qph_node* q = nullptr;
      for (const qph_node& n : net->nodes)
        if (n.out == t) q = &n;
      words = numel_of(net, q->in) / q->ws[0] * net->pitch[(size_t)t];
    }
    net->arena_bytes += ((size_t)words * 4 + 255) / 256 * 256;
  }
  rc = hip_check(hipMalloc((void**)&net->arena, net->arena_bytes), "hipMalloc(arena)");
  if (rc) return bail(rc);
  for (int32_t t = 0; t < spec->n_tensors; t++) {
    int32_t a = net->alias[t] >= 0 ? net->alias[t] : t;
    net->tptr[t] = (float*)(net->arena + off[a]);
  }
  // weights
  for (int32_t wi = 0; wi < spec->n_weights; wi++) {
    float* d = nullptr;
    size_t bytes = (size_t)spec->weight_sizes[wi] * 4;
    rc = hip_check(hipMalloc((void**)&d, bytes ? bytes : 4), "hipMalloc(weight)");
    if (rc) return bail(rc);
    net->weights.push_back(d);
    if (bytes) {
      rc = hip_check(hipMemcpy(d, weights_host[wi], bytes, hipMemcpyHostToDevice), "hipMemcpy(weight)");
      if (rc) return bail(rc);
    }
  }
  for (size_t i = 0; i < net->nodes.size(); i++) {
    rc = validate_node(net, i, spec->weight_sizes, spec->n_weights);
    if (rc) return bail(rc);
    const qph_node& n = net->nodes[i];
    // dense and grouped convs keep k-major repacked weights (the depthwise
    // kernel reads the ONNX layout as it is)
    const bool dense = n.op == QPH_OP_CONV && !conv_is_pointwise(n.ws, n.cp) &&
                       !(n.cp.group > 1 && n.ws[1] == 1 && n.ws[0] == n.cp.group);
    if (dense) {
      float* d = nullptr;
      const size_t bytes =
          (size_t)dense_conv_wk_floats(n.ws[0], n.ws[1], n.ws[2], n.ws[3], n.cp.group) * 4;
      rc = hip_check(hipMalloc((void**)&d, bytes), "hipMalloc(repacked weight)");
      if (rc) return bail(rc);
      net->wk[i] = d;
      rc = launch_repack_conv_w_taps(net->weights[n.w], n.ws[0], n.ws[1], n.ws[2] * n.ws[3], d,
                                     ctx->stream, n.cp.group);
      if (rc) return bail(rc);
    }
    if (n.op == QPH_OP_LINEAR) {
      // below the 128x128 size: weight kept transposed for linear_nt_kernel
      const int64_t k = n.ws[0], nn = n.ws[1], rows = numel_of(net, n.in) / k;
      if (!gemm_takes_wide(rows, nn, 1) && linear_nt_eligible(rows, nn, k, k)) {
        float* d = nullptr;
        rc = hip_check(hipMalloc((void**)&d, (size_t)(k * nn) * 4), "hipMalloc(transposed weight)");
        if (rc) return bail(rc);
        net->wt[i] = d;
        rc = launch_transpose(net->weights[n.w], k, nn, d, ctx->stream);
        if (rc) return bail(rc);
        continue;
      }
    }
    if (n.op == QPH_OP_LINEAR && n.ws[1] % 4 != 0) {
      // [K][N] -> [K][N4] with zero columns past N (16-byte aligned rows)
      const int64_t k = n.ws[0], nn = n.ws[1], n4 = (nn + 3) / 4 * 4;
      float* d = nullptr;
      rc = hip_check(hipMalloc((void**)&d, (size_t)(k * n4) * 4), "hipMalloc(padded weight)");
      if (rc) return bail(rc);
      net->wk[i] = d;
      rc = hip_check(hipMemset2DAsync(d, (size_t)n4 * 4, 0, (size_t)n4 * 4, (size_t)k, ctx->stream),
                     "hipMemset2DAsync");
      if (rc == QPH_OK)
        rc = hip_check(hipMemcpy2DAsync(d, (size_t)n4 * 4, net->weights[n.w], (size_t)nn * 4,
                                        (size_t)nn * 4, (size_t)k, hipMemcpyDeviceToDevice,
                                        ctx->stream),
                       "hipMemcpy2DAsync");
      if (rc) return bail(rc);
    }
  }
  const size_t nn = net->nodes.size();
  for (size_t i = 0; i < nn; i++) {
    if (!net->head[i]) continue;
    const qph_node& q = net->nodes[i];
    const int64_t rows = numel_of(net, q.in) / q.ws[0];
    float* d = nullptr;
    rc = hip_check(hipMalloc((void**)&d, (size_t)head_argmax_part_floats(rows, q.ws[1]) * 4),
                   "hipMalloc(head partials)");
    if (rc) return bail(rc);
    net->head_part[i] = d;
  }
  if (spec->flags & QPH_NET_SEPARATE_LAUNCHES) {
    net->plan.assign(nn, ConvArgs{});
    net->group_len.assign(nn, 1);
    net->convt_fused.assign(nn, false);
    net->absorb_after.assign(nn, 0);
    net->fpn.assign(nn, false);
    net->cl_dw.assign(nn, false);
    net->cl_pw.assign(nn, false);
    net->cl_out.assign(nn, false);
    net->dwpw.assign(nn, DwPwArgs{});
    net->fused.assign(nn, false);
  } else {
    plan_hardswish_clip(net);
    plan_conv_groups(net);
    plan_conv_convt(net);
    plan_cl(net);
    rc = plan_dwpw(net);
    if (rc) return bail(rc);
    rc = plan_fpn(net);
    if (rc) return bail(rc);
  }
  rc = hip_check(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
  if (rc) return bail(rc);
  rc = capture(net);
  if (rc) return bail(rc);
  *out = net;
  return QPH_OK;
}

QPH_API int qph_net_destroy(qph_net* net) {
  release(net);
  return QPH_OK;
}

QPH_API int qph_net_tensor(qph_net* net, int32_t id, float** dev_ptr, int64_t* numel) {
  if (!net || id < 0 || id >= (int32_t)net->tptr.size())
    return fail(QPH_EINVAL, "net_tensor: bad tensor id");
  // a tensor consumed inside one fused launch (a fused head's logits, the
  // QKV output of a linear + attention launch) owns no arena bytes: its
  // pointer would name the next tensor's storage
  if (net->nostore[(size_t)id])
    return fail(QPH_EINVAL, "net_tensor: tensor is internal to a fused launch and never stored");
  if (dev_ptr) *dev_ptr = net->tptr[id];
  if (numel) *numel = numel_full(net, id);
  return QPH_OK;
}

QPH_API int qph_net_set_profiling(qph_net* net, int32_t on) {
  if (!net) return fail(QPH_EINVAL, "net_set_profiling: NULL net");
  net->profiling = on != 0;
  net->prof_runs = 0;
  net->node_ms.assign(net->nodes.size(), 0.0);
  if (net->profiling && net->ev.empty()) {
    net->ev.resize(net->nodes.size() + 1);
    for (auto& e : net->ev) QPH_TRY_HIP(hipEventCreate(&e));
  }
  return QPH_OK;
}

QPH_API int qph_net_node_times(qph_net* net, double* ms, int32_t n) {
  if (!net || !ms) return fail(QPH_EINVAL, "net_node_times: NULL argument");
  for (int32_t i = 0; i < n && i < (int32_t)net->node_ms.size(); i++)
    ms[i] = net->prof_runs ? net->node_ms[i] / (double)net->prof_runs : 0.0;
  return QPH_OK;
}

QPH_API int qph_net_plan(qph_net* net, int32_t* first, int32_t* nodes, int32_t* kernels,
                         int32_t cap, int32_t* n_launches) {
  if (!net || !n_launches) return fail(QPH_EINVAL, "net_plan: NULL argument");
  // the stepping of run_all: one launch per plain node, one per fused
  // block / dense group / conv + conv-transpose pair / fused head (the head
  // is two kernels) / QKV linear + attention, each also covering the
  // elementwise nodes folded into its epilogue; the four FPN laterals are
  // three kernels
  int32_t n = 0;
  const size_t nn = net->nodes.size();
  for (size_t i = 0; i < nn; n++) {
    size_t step = 1;
    int32_t nk = 1;
    if (net->group_len[i] > 1) step = (size_t)net->group_len[i];
    else if (net->head[i]) step = 2, nk = 2;
    else if (net->fused[i]) step = net->dwpw[i].stem ? 3 : 2;
    else if (net->convt_fused[i]) step = 2;
    else if (net->qa_fused[i]) step = 2;
    else if (net->fpn[i]) step = 4, nk = 3;
    step += (size_t)net->absorb_after[i + step - 1];
    if (n < cap) {
      if (first) first[n] = (int32_t)i;
      if (nodes) nodes[n] = (int32_t)step;
      if (kernels) kernels[n] = nk;
    }
    i += step;
  }
  *n_launches = n;
  return QPH_OK;
}

QPH_API int qph_net_set_real_n(qph_net* net, int32_t real_n) {
  if (!net) return fail(QPH_EINVAL, "net_set_real_n: NULL net");
  if (real_n < 1 || real_n > net->batch)
    return fail(QPH_EINVAL, "net_set_real_n: " + std::to_string(real_n) + " outside 1.." +
                                std::to_string(net->batch));
  if (net->inflight)
    return fail(QPH_EINVAL, "net_set_real_n: the previous run of this net is not complete");
  if (real_n == net->real_n) return QPH_OK;
  for (size_t t = 0; t < net->batch_major.size(); t++)
    if (net->batch_major[t] && net->shapes_full[4 * t] != net->batch)
      return fail(QPH_EUNSUPPORTED, "net_set_real_n: tensor " + std::to_string(t) +
                                        " does not keep the batch as its first dimension");
  const int64_t prev = net->real_n;
  net->real_n = real_n;
  set_eff_shapes(net);
  // capture now, so a failure names its node here and the first run with
  // this count pays no capture time
  const int rc = net->execs[(size_t)real_n] ? QPH_OK : capture(net);
  if (rc != QPH_OK) {
    const std::string msg = qph_last_error();
    net->real_n = prev;
    set_eff_shapes(net);
    return fail(rc, msg);
  }
  return QPH_OK;
}

QPH_API int qph_net_real_n(qph_net* net, int32_t* real_n, int32_t* batch) {
  if (!net) return fail(QPH_EINVAL, "net_real_n: NULL net");
  if (real_n) *real_n = (int32_t)net->real_n;
  if (batch) *batch = (int32_t)net->batch;
  return QPH_OK;
}

QPH_API int qph_net_staging(qph_net* net, int32_t slot, float** host, int64_t* numel) {
  if (!net || !host) return fail(QPH_EINVAL, "net_staging: NULL argument");
  if (slot < -1 || slot >= (int32_t)net->outputs.size())
    return fail(QPH_EINVAL, "net_staging: slot " + std::to_string(slot) + " of " +
                                std::to_string(net->outputs.size()) + " outputs");
  const int32_t id = slot < 0 ? 0 : net->outputs[(size_t)slot];
  float*& buf = slot < 0 ? net->in_stage : net->out_stage[(size_t)slot];
  if (!buf) {
    QPH_TRY_HIP(hipSetDevice(net->ctx->device));
    void* p = nullptr;
    QPH_TRY_HIP(hipHostMalloc(&p, (size_t)numel_full(net, id) * 4, hipHostMallocDefault));
    buf = (float*)p;
  }
  *host = buf;
  if (numel) *numel = numel_full(net, id);
  return QPH_OK;
}

QPH_API int qph_net_run_async(qph_net* net, int32_t flags) {
  if (!net) return fail(QPH_EINVAL, "net_run_async: NULL net");
  if (net->inflight)
    return fail(QPH_EINVAL, "net_run_async: the previous run of this net is not complete");
  if (net->profiling) return fail(QPH_EINVAL, "net_run_async: profiling is on");
  hipStream_t s = net->ctx->stream;
  if ((flags & QPH_RUN_UPLOAD) && !net->in_stage)
    return fail(QPH_EINVAL, "net_run_async: no input staging buffer (qph_net_staging -1)");
  if (flags & QPH_RUN_DOWNLOAD)
    for (size_t o = 0; o < net->outputs.size(); o++)
      if (!net->out_stage[o])
        return fail(QPH_EINVAL, "net_run_async: output " + std::to_string(o) +
                                    " has no staging buffer");
  if (!net->done) QPH_TRY_HIP(hipEventCreateWithFlags(&net->done, hipEventDisableTiming));
  if (flags & QPH_RUN_UPLOAD)
    QPH_TRY_HIP(hipMemcpyAsync(net->tptr[0], net->in_stage, (size_t)numel_of(net, 0) * 4,
                               hipMemcpyHostToDevice, s));
  QPH_TRY(launch_graph(net));
  if (flags & QPH_RUN_DOWNLOAD)
    for (size_t o = 0; o < net->outputs.size(); o++) {
      const int32_t id = net->outputs[o];
      QPH_TRY_HIP(hipMemcpyAsync(net->out_stage[o], net->tptr[id], (size_t)numel_of(net, id) * 4,
                                 hipMemcpyDeviceToHost, s));
    }
  QPH_TRY_HIP(hipEventRecord(net->done, s));
  net->inflight = true;
  return QPH_OK;
}

QPH_API int qph_net_complete(qph_net* net) {
  if (!net) return fail(QPH_EINVAL, "net_complete: NULL net");
  if (!net->inflight) return QPH_OK;
  net->inflight = false;
  return hip_check(hipEventSynchronize(net->done), "hipEventSynchronize");
}

QPH_API int qph_net_run(qph_net* net, const float* input, int32_t input_is_device,
                        float* const* outputs_host) {
  if (!net) return fail(QPH_EINVAL, "net_run: NULL net");
  if (net->inflight) QPH_TRY(qph_net_complete(net));
  hipStream_t s = net->ctx->stream;
  if (input) {
    size_t bytes = (size_t)numel_of(net, 0) * 4;
    QPH_TRY_HIP(hipMemcpyAsync(net->tptr[0], input, bytes,
                               input_is_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, s));
  }
  if (net->profiling) {
    QPH_TRY(run_all(net));
    QPH_TRY_HIP(hipEventRecord(net->ev[net->nodes.size()], s));
    QPH_TRY_HIP(hipEventSynchronize(net->ev[net->nodes.size()]));
    for (size_t i = 0; i < net->nodes.size(); i++) {
      float ms = 0.0f;
      QPH_TRY_HIP(hipEventElapsedTime(&ms, net->ev[i], net->ev[i + 1]));
      net->node_ms[i] += ms;
    }
    net->prof_runs++;
  } else {
    QPH_TRY(launch_graph(net));
  }
  if (outputs_host) {
    for (size_t o = 0; o < net->outputs.size(); o++) {
      if (!outputs_host[o]) continue;
      int32_t id = net->outputs[o];
      QPH_TRY_HIP(hipMemcpyAsync(outputs_host[o], net->tptr[id], (size_t)numel_of(net, id) * 4,
                                 hipMemcpyDeviceToHost, s));
    }
    QPH_TRY_HIP(hipStreamSynchronize(s));
  }
  return QPH_OK;
}

}  // extern "C"
