"""Sessions over the reference's plan model on the GPU (qph_plan_*): every
dispatch contract of the Vulkan kernel set (qppocr-gpu/shaders/n_*.comp)
against the CPU oracle's operation, with parameter blocks laid out as
PlanBuilder writes them (qppocr-gpu/src/plan.rs), and whole det / rec plans
against the oracle's graph run.  Bit-exact throughout."""
import math

import numpy as np
import pytest

from conftest import assert_bitexact

pytestmark = pytest.mark.gpu

OFF_NONE = 0xFFFFFFFF


def nhwc(x, cp=None):
    """NCHW [n, c, h, w] -> NHWC words [n, h, w, cpad] (pad channels 0)."""
    n, c, h, w = x.shape
    cp = cp or (c + 3) // 4 * 4
    out = np.zeros((n, h, w, cp), np.float32)
    out[..., :c] = x.transpose(0, 2, 3, 1)
    return out


class MiniPlan:
    """A hand-built GraphPlan: regions, parameter blocks and dispatches."""

    def __init__(self):
        from qppocr_amd import plan
        self.P = plan
        self.p = plan.GraphPlan()
        self.words = 0
        self.static(np.array([0], np.uint32))           # word 0: real_n
        self.p.in_f32_off = self.alloc(4)
        self.p.in_shape = (4,)

    def alloc(self, n):
        off = self.words
        self.words += max(4, (int(n) + 3) // 4 * 4)
        return off

    def static(self, a):
        a = np.ascontiguousarray(a)
        w = a.view(np.uint32).reshape(-1) if a.dtype != np.uint32 else a.reshape(-1)
        off = self.alloc(w.size)
        self.p.uploads.append((off, np.ascontiguousarray(w)))
        return off

    def dispatch(self, kernel, params, groups=(1, 1, 1)):
        pw = np.array([p if isinstance(p, (int, np.integer)) else self.P.f32_bits(p) for p in params],
                      dtype=np.uint32)
        self.p.dispatches.append((kernel, self.static(pw), tuple(groups), -1))

    def output(self, off, numel, shape):
        self.p.outputs.append((off, int(numel), tuple(shape)))

    def run(self, real_n=0):
        from qppocr_amd import plan
        self.p.total_words = self.words
        s = plan.HipPlanSession(self.p)
        try:
            return s.run(None, real_n=real_n)
        finally:
            s.close()


def rng(seed):
    return np.random.default_rng(seed)


def rnd(r, shape, scale=1.0):
    return (r.standard_normal(shape) * scale).astype(np.float32)


# ---------------------------------------------------------------- conv family

CONV_CASES = [
    # n, c, h, w, m, kh, kw, (sh, sw), (ph, pw, peh, pew), bias, act, residual
    (1, 8, 12, 12, 16, 3, 3, (1, 1), (1, 1, 1, 1), True, "relu", False),    # implicit GEMM rule
    (1, 3, 17, 15, 16, 3, 3, (2, 2), (1, 1, 1, 1), True, "none", False),    # stem: C 3 -> pad 4
    (1, 32, 20, 20, 24, 1, 1, (1, 1), (0, 0, 0, 0), True, "gelu", True),    # pointwise on the GEMM
    (1, 256, 4, 4, 64, 1, 1, (1, 1), (0, 0, 0, 0), True, "none", False),    # pointwise, m-rows: all seeded
    (2, 12, 9, 11, 20, 3, 3, (1, 1), (1, 1, 1, 1), True, "none", True),     # batch 2 + residual
    (1, 8, 17, 19, 12, 5, 5, (3, 3), (2, 2, 2, 2), True, "relu", False),    # x-stride 3: im2col tiles
    (1, 16, 10, 10, 8, 1, 1, (2, 2), (0, 0, 0, 0), True, "none", False),    # 1x1 stride 2: general
    (1, 8, 7, 8, 4, 2, 2, (1, 1), (0, 0, 1, 1), False, "none", False),      # SAME_UPPER 2x2, no bias
    (3, 20, 6, 6, 36, 3, 3, (1, 1), (1, 1, 1, 1), True, "gelu", False),     # N odd vec4 count: n_conv
    # the 3x3 halo tiles (2 output rows, 2 channel groups a stage): stride 2
    # with an odd row count; 4 output blocks, 5 stages through the 3-deep
    # ring, 3 column tiles; stride 2 with 3 blocks, an odd group count, no bias
    (1, 16, 21, 19, 24, 3, 3, (2, 2), (1, 1, 1, 1), True, "relu", False),
    (2, 40, 13, 70, 64, 3, 3, (1, 1), (1, 1, 1, 1), True, "none", True),
    (1, 28, 23, 66, 48, 3, 3, (2, 2), (1, 1, 1, 1), False, "gelu", False),
    # pointwise with 16 input channels (register-operand kernel): batch 2,
    # a row count off the 32-pixel tiles, residual; and without bias
    (2, 16, 9, 13, 40, 1, 1, (1, 1), (0, 0, 0, 0), True, "relu", True),
    (1, 16, 12, 12, 20, 1, 1, (1, 1), (0, 0, 0, 0), False, "none", False),
    # stems (3x3 over 4 padded channels): 32 outputs in one wave, stride 1,
    # batch 2 + residual; 40 outputs (a partial second wave), stride 2
    (2, 3, 11, 37, 32, 3, 3, (1, 1), (1, 1, 1, 1), True, "relu", True),
    (1, 4, 20, 21, 40, 3, 3, (2, 2), (1, 1, 1, 1), False, "gelu", False),
]


@pytest.mark.parametrize("case", CONV_CASES, ids=lambda c: f"{c[1]}to{c[4]}_k{c[5]}x{c[6]}_s{c[7][1]}_{c[10]}")
def test_plan_conv(gpu, oracle, case):
    from qppocr_amd import plan
    n, c, h, w, m, kh, kw, (sh, sw), pads, has_b, act, has_r = case
    O = oracle
    r = rng(n * 100003 + c * 1009 + h * 101 + m * 13 + kh * 7 + sw)
    x = rnd(r, (n, c, h, w))
    wt = rnd(r, (m, c, kh, kw), 1.0 / math.sqrt(c * kh * kw))
    b = rnd(r, (m,), 0.1) if has_b else None
    p = O.conv_params(sh, sw, pads[0], pads[1], pads[2], pads[3])
    oh = (h + pads[0] + pads[2] - kh) // sh + 1
    ow = (w + pads[1] + pads[3] - kw) // sw + 1
    res = rnd(r, (n, m, oh, ow)) if has_r else None
    code = {"none": O.ACT_NONE, "relu": O.ACT_RELU, "gelu": O.ACT_GELU}[act]
    ref = O.conv2d(x, wt, b, p, code, res)
    cp, mp = plan.cpad4(c), plan.cpad4(m)
    mp_ = MiniPlan()
    xo = mp_.static(nhwc(x))
    wo = mp_.static(np.concatenate([plan.repack_conv_w(wt, m, c, kh, kw), np.zeros(32, np.uint32)]))
    bo = mp_.static(plan.conv_bias(b, m)) if has_b else OFF_NONE
    ro = mp_.static(nhwc(res)) if has_r else OFF_NONE
    yo = mp_.alloc(n * oh * ow * mp)
    kname = "n_conv8" if (mp // 4) % 2 == 0 else "n_conv"
    mp_.dispatch(kname, [xo, wo, bo, yo, oh * ow, mp, ow, w, h, cp // 4, kh * kw, kw, sh, sw,
                         pads[0], pads[1], {"none": 0, "gelu": 1, "relu": 2}[act], *plan.GELU_C, ro],
                 (1, n, 1))
    mp_.output(yo, n * oh * ow * mp, (n, oh, ow, mp))
    print(f"plan conv {case}", flush=True)
    got = mp_.run()[0]
    assert_bitexact(got, nhwc(ref), "conv")


@pytest.mark.parametrize("dependent", [False, True])
def test_plan_halo_convs_share_a_launch(gpu, oracle, dependent):
    """Two 9-tap convs with 24 outputs (the det neck's smoothing shape) with an
    n_resize between them run as one launch when the second reads nothing
    the resize or the first writes; when the second reads the first's output
    it keeps its own launch.  Bit-exact against the oracle either way."""
    from qppocr_amd import plan as P
    O = oracle
    r = rng(91 + int(dependent))
    c, m, h1, h2 = 32, 24, 20, 40
    x1 = rnd(r, (1, c, h1, h1))
    x2 = rnd(r, (1, c, h2, h2))
    w1 = rnd(r, (m, c, 3, 3), 1.0 / math.sqrt(c * 9))
    w2 = rnd(r, (m, m if dependent else c, 3, 3), 1.0 / math.sqrt(c * 9))
    b1, b2 = rnd(r, (m,), 0.1), rnd(r, (m,), 0.1)
    p = O.conv_params(1, 1, 1, 1, 1, 1)
    ref1 = O.conv2d(x1, w1, b1, p, O.ACT_RELU)
    ref2 = O.conv2d(ref1 if dependent else x2, w2, b2, p, O.ACT_NONE)
    up = O.resize_nearest(ref1, 2 * h1, 2 * h1)
    mp = MiniPlan()
    x1o, x2o = mp.static(nhwc(x1)), mp.static(nhwc(x2))
    w1o = mp.static(np.concatenate([P.repack_conv_w(w1, m, c, 3, 3), np.zeros(32, np.uint32)]))
    c2 = m if dependent else c
    w2o = mp.static(np.concatenate([P.repack_conv_w(w2, m, c2, 3, 3), np.zeros(32, np.uint32)]))
    b1o, b2o = mp.static(P.conv_bias(b1, m)), mp.static(P.conv_bias(b2, m))
    y1o = mp.alloc(h1 * h1 * m)
    upo = mp.alloc(4 * h1 * h1 * m)
    hi = h1 if dependent else h2
    y2o = mp.alloc(hi * hi * m)
    mp.dispatch("n_conv8", [x1o, w1o, b1o, y1o, h1 * h1, m, h1, h1, h1, c // 4, 9, 3, 1, 1, 1, 1,
                            2, *P.GELU_C, OFF_NONE], (1, 1, 1))
    mp.dispatch("n_resize", [y1o, upo, 4 * h1 * h1, m, 2 * h1, h1, h1, float(np.float32(0.5)),
                             float(np.float32(0.5))], (1, 1, 1))
    mp.dispatch("n_conv8", [y1o if dependent else x2o, w2o, b2o, y2o, hi * hi, m, hi, hi, hi,
                            c2 // 4, 9, 3, 1, 1, 1, 1, 0, *P.GELU_C, OFF_NONE], (1, 1, 1))
    mp.output(y2o, hi * hi * m, (1, hi, hi, m))
    mp.output(upo, 4 * h1 * h1 * m, (1, 2 * h1, 2 * h1, m))
    mp.p.total_words = mp.words
    sess = P.HipPlanSession(mp.p)
    try:
        got2, gotup = sess.run(None)
        assert sess.launches() == (3 if dependent else 2)
    finally:
        sess.close()
    assert_bitexact(got2, nhwc(ref2), "second conv")
    assert_bitexact(gotup, nhwc(up), "upsampled first conv")


DW_CASES = [
    # n, c, h, w, k, (sh, sw), (pt, pl, pb, pr), bias, act, residual
    (1, 16, 13, 12, 3, (1, 1), (1, 1, 1, 1), True, "none", False),
    (2, 12, 11, 14, 5, (2, 2), (2, 2, 2, 2), True, "relu", True),
    (1, 8, 6, 40, 3, (3, 1), (0, 1, 0, 1), False, "gelu", False),   # rec block 4 geometry
]


@pytest.mark.parametrize("case", DW_CASES, ids=lambda c: f"c{c[1]}_k{c[4]}_s{c[5][0]}{c[5][1]}_{c[8]}")
def test_plan_conv_dw(gpu, oracle, case):
    from qppocr_amd import plan
    n, c, h, w, k, (sh, sw), pads, has_b, act, has_r = case
    O = oracle
    r = rng(7 + c + k)
    x = rnd(r, (n, c, h, w))
    wt = rnd(r, (c, 1, k, k), 1.0 / k)
    b = rnd(r, (c,), 0.1) if has_b else None
    p = O.conv_params(sh, sw, pads[0], pads[1], pads[2], pads[3], group=c)
    ref = O.conv2d(x, wt, b, p)
    if act == "relu":
        ref = O.relu_inplace(ref.copy())
    elif act == "gelu":
        ref = O.gelu_inplace(ref.copy())
    oh, ow = ref.shape[2:]
    res = rnd(r, ref.shape) if has_r else None
    if has_r:
        ref = O.binary_flat(ref, res, 0)
    mp = MiniPlan()
    xo = mp.static(nhwc(x))
    wo = mp.static(plan.repack_dw_w(wt, c, k, k))
    bo = mp.static(plan.conv_bias(b, c)) if has_b else OFF_NONE
    ro = mp.static(nhwc(res)) if has_r else OFF_NONE
    cp = plan.cpad4(c)
    yo = mp.alloc(n * oh * ow * cp)
    mp.dispatch("n_conv_dw", [xo, wo, bo, yo, oh * ow, cp, ow, w, h, k * k, k, sh, sw, pads[0],
                              pads[1], {"none": 0, "gelu": 1, "relu": 2}[act], *plan.GELU_C, ro],
                (1, n, 1))
    mp.output(yo, n * oh * ow * cp, (n, oh, ow, cp))
    print(f"plan dw {case}", flush=True)
    assert_bitexact(mp.run()[0], nhwc(ref), "depthwise")


@pytest.mark.parametrize("ci,co", [(24, 24), (24, 1), (6, 10)])
def test_plan_convt(gpu, oracle, ci, co):
    from qppocr_amd import plan
    r = rng(ci * 31 + co)
    n, h, w = 2, 5, 7
    x = rnd(r, (n, ci, h, w))
    wt = rnd(r, (ci, co, 2, 2), 0.3)
    ref = oracle.convtranspose2d(x, wt)
    cip, cop = plan.cpad4(ci), plan.cpad4(co)
    mp = MiniPlan()
    xo = mp.static(nhwc(x))
    wo = mp.static(plan.repack_convt_w(wt, ci, co, 2, 2))
    yo = mp.alloc(n * 4 * h * w * cop)
    mp.dispatch("n_convt", [xo, wo, OFF_NONE, yo, 4 * h * w, cop, 2 * w, w, h, cip, cip // 4, 2, 2,
                            2, 0, *plan.GELU_C], (1, n, 1))
    mp.output(yo, n * 4 * h * w * cop, (n, 2 * h, 2 * w, cop))
    print(f"plan convt {ci}->{co}", flush=True)
    assert_bitexact(mp.run()[0], nhwc(ref), "conv transpose")


@pytest.mark.parametrize("sig", [True, False])
def test_plan_convt_pair_exit_fused(gpu, oracle, sig):
    """n_convt 24 -> 24, n_convt 24 -> 1 and the n_exit after them (the det
    head's tail) run as one pass; bit-exact against the oracle's two
    conv-transposes and sigmoid."""
    from qppocr_amd import plan
    r = rng(41 + sig)
    n, h, w = 2, 5, 6
    x = rnd(r, (n, 24, h, w))
    w1 = rnd(r, (24, 24, 2, 2), 0.3)
    w2 = rnd(r, (24, 1, 2, 2), 0.3)
    t2 = oracle.convtranspose2d(oracle.convtranspose2d(x, w1), w2)
    ref = oracle.sigmoid_tensor(t2) if sig else t2
    mp = MiniPlan()
    xo = mp.static(nhwc(x))
    wo1 = mp.static(plan.repack_convt_w(w1, 24, 24, 2, 2))
    wo2 = mp.static(plan.repack_convt_w(w2, 24, 1, 2, 2))
    y1 = mp.alloc(n * 4 * h * w * 24)
    mp.dispatch("n_convt", [xo, wo1, OFF_NONE, y1, 4 * h * w, 24, 2 * w, w, h, 24, 6, 2, 2, 2, 0,
                            *plan.GELU_C], (1, n, 1))
    y2 = mp.alloc(n * 16 * h * w * 4)
    mp.dispatch("n_convt", [y1, wo2, OFF_NONE, y2, 16 * h * w, 4, 4 * w, 2 * w, 2 * h, 24, 6, 2, 2, 2,
                            0, *plan.GELU_C], (1, n, 1))
    out = mp.alloc(n * 16 * h * w)
    mp.dispatch("n_exit", [y2, out, n, 1, 4 * h, 4 * w, 4, 4 if sig else 0])
    mp.output(out, n * 16 * h * w, (n, 1, 4 * h, 4 * w))
    mp.p.total_words = mp.words
    s = plan.HipPlanSession(mp.p)
    try:
        assert s.launches() == 1
        (got,) = s.run(None)
    finally:
        s.close()
    assert_bitexact(got, ref, "conv-transpose pair + exit")


def test_plan_real_n_skips_padded_batch_rows(gpu, oracle):
    """Word 0 (real_n) stops the conv at the real batch (plan.rs:587-593):
    the padded batch item's output keeps what the arena held."""
    from qppocr_amd import plan
    O = oracle
    r = rng(5)
    n, c, h, w, m = 3, 8, 6, 6, 8
    x = rnd(r, (n, c, h, w))
    wt = rnd(r, (m, c, 3, 3), 0.2)
    ref = O.conv2d(x, wt, None, O.conv_params(1, 1, 1, 1))
    mp = MiniPlan()
    xo = mp.static(nhwc(x))
    wo = mp.static(np.concatenate([plan.repack_conv_w(wt, m, c, 3, 3), np.zeros(32, np.uint32)]))
    sentinel = np.full(n * h * w * m, 7.0, np.float32)
    yo = mp.static(sentinel)
    mp.dispatch("n_conv8", [xo, wo, OFF_NONE, yo, h * w, m, w, w, h, 2, 9, 3, 1, 1, 1, 1, 0,
                            *plan.GELU_C, OFF_NONE], (1, n, 1))
    mp.output(yo, n * h * w * m, (n, h, w, m))
    got = mp.run(real_n=2)[0]
    assert_bitexact(got[:2], nhwc(ref)[:2], "real rows")
    assert np.all(got[2] == 7.0)


def test_plan_real_n_in_fused_launches(gpu, oracle):
    """real_n in the launches that take over several dispatches: the
    resize + add pass and the conv-transpose pair + exit stop at the real
    batch; the real items equal the oracle, the padded item's outputs keep
    what the arena held."""
    from qppocr_amd import plan
    r = rng(17)
    n, h, w = 3, 4, 5
    a = rnd(r, (n, 2, 3, 8))
    y = rnd(r, (n, 4, 6, 8))
    x = rnd(r, (n, 24, h, w))
    w1 = rnd(r, (24, 24, 2, 2), 0.3)
    w2 = rnd(r, (24, 1, 2, 2), 0.3)
    ref_t = oracle.sigmoid_tensor(oracle.convtranspose2d(oracle.convtranspose2d(x, w1), w2))
    mp = MiniPlan()
    ao, yo = mp.static(a), mp.static(y)
    ra = mp.alloc(n * 4 * 6 * 8)
    mp.dispatch("n_resize", [ao, ra, 4 * 6, 8, 6, 3, 2, 0.5, 0.5], (1, n, 1))
    so = mp.static(np.full(n * 4 * 6 * 8, 7.0, np.float32))
    mp.dispatch("n_elem", [4, ra, yo, so, n * 4 * 6 * 8, 0.0, 0.0])
    xo = mp.static(nhwc(x))
    wo1 = mp.static(plan.repack_convt_w(w1, 24, 24, 2, 2))
    wo2 = mp.static(plan.repack_convt_w(w2, 24, 1, 2, 2))
    t1 = mp.alloc(n * 4 * h * w * 24)
    mp.dispatch("n_convt", [xo, wo1, OFF_NONE, t1, 4 * h * w, 24, 2 * w, w, h, 24, 6, 2, 2, 2, 0,
                            *plan.GELU_C], (1, n, 1))
    t2 = mp.alloc(n * 16 * h * w * 4)
    mp.dispatch("n_convt", [t1, wo2, OFF_NONE, t2, 16 * h * w, 4, 4 * w, 2 * w, 2 * h, 24, 6, 2, 2, 2,
                            0, *plan.GELU_C], (1, n, 1))
    out = mp.static(np.full(n * 16 * h * w, 7.0, np.float32))
    mp.dispatch("n_exit", [t2, out, n, 1, 4 * h, 4 * w, 4, 4])
    mp.output(so, n * 4 * 6 * 8, (n, 4, 6, 8))
    mp.output(out, n * 16 * h * w, (n, 1, 4 * h, 4 * w))
    got_s, got_t = mp.run(real_n=2)
    assert_bitexact(got_s[:2], (_resize_ref(a, 4, 6) + y)[:2], "resize + add, real items")
    assert np.all(got_s[2] == 7.0)
    assert_bitexact(got_t[:2], ref_t[:2], "conv-transpose pair, real items")
    assert np.all(got_t[2] == 7.0)


# -------------------------------------------------------- pool / resize / reductions

POOL_CASES = [  # kh, kw, sh, sw, pads (t, l, b, r), max
    (3, 3, 2, 2, (1, 1, 1, 1), True),
    (2, 2, 2, 2, (0, 0, 0, 0), False),
    (2, 2, 1, 1, (0, 0, 1, 1), True),      # SAME_UPPER 2x2 stride 1 (pool2x2_row_scalar)
    (3, 3, 1, 1, (1, 1, 1, 1), False),
]


@pytest.mark.parametrize("case", POOL_CASES)
def test_plan_pool(gpu, oracle, case):
    kh, kw, sh, sw, (pt, pl, pb, pr), mx = case
    r = rng(kh * 10 + sh)
    n, c, h, w = 2, 8, 9, 10
    x = rnd(r, (n, c, h, w))
    ref = oracle.pool2d(x, kh, kw, sh, sw, pt, pl, pb, pr, mx)
    oh, ow = ref.shape[2:]
    mp = MiniPlan()
    xo = mp.static(nhwc(x))
    yo = mp.alloc(n * oh * ow * c)
    mp.dispatch("n_pool", [xo, yo, oh * ow, c, ow, w, h, kh, kw, sh, sw, pt, pl, int(mx)], (1, n, 1))
    mp.output(yo, n * oh * ow * c, (n, oh, ow, c))
    assert_bitexact(mp.run()[0], nhwc(ref), "pool")


@pytest.mark.parametrize("ih,iw,oh,ow", [(5, 6, 10, 12), (5, 7, 12, 9), (8, 8, 3, 5)])
def test_plan_resize_nearest(gpu, oracle, ih, iw, oh, ow):
    r = rng(ih * oh)
    n, c = 2, 12
    x = rnd(r, (n, c, ih, iw))
    ref = oracle.resize_nearest(x, oh, ow)
    mp = MiniPlan()
    xo = mp.static(nhwc(x))
    yo = mp.alloc(n * oh * ow * c)
    mp.dispatch("n_resize", [xo, yo, oh * ow, c, ow, iw, ih, float(np.float32(ih / oh)),
                             float(np.float32(iw / ow))], (1, n, 1))
    mp.output(yo, n * oh * ow * c, (n, oh, ow, c))
    assert_bitexact(mp.run()[0], nhwc(ref), "resize")


def test_plan_global_average_pool(gpu, oracle):
    """n_reduce_hw + n_reduce_fin: one exact f64 mean per image and channel."""
    r = rng(11)
    n, c, h, w = 3, 20, 33, 35
    x = rnd(r, (n, c, h, w)) + 3.0
    ref = oracle.global_avg_pool(x).reshape(n, c)
    mp = MiniPlan()
    xo = mp.static(nhwc(x))
    scratch = mp.alloc(n * ((h * w + 1023) // 1024) * c)
    yo = mp.alloc(n * c)
    mp.dispatch("n_reduce_hw", [xo, scratch, h * w, c], ((h * w + 1023) // 1024, n, 1))
    mp.dispatch("n_reduce_fin", [scratch, yo, (h * w + 1023) // 1024, c, h * w], (n, 1, 1))
    mp.output(yo, n * c, (n, c))
    assert_bitexact(mp.run()[0], ref, "global average pool")


def test_plan_reduce_last_and_row_ops(gpu, oracle):
    """n_reduce_last (rows x cpad storage, [rows, 4] out) and the row-vector
    sub / div of the LayerNorm chain."""
    r = rng(12)
    rows, cols, cp = 37, 30, 32
    x = np.zeros((rows, cp), np.float32)
    x[:, :cols] = rnd(r, (rows, cols)) + 1.0
    mean = oracle.reduce_mean_last(x[:, :cols])
    mp = MiniPlan()
    xo = mp.static(x)
    mo = mp.alloc(rows * 4)
    mp.dispatch("n_reduce_last", [xo, mo, rows, cols, cp, rows], (rows, 1, 1))
    so = mp.alloc(rows * cp)
    mp.dispatch("n_elem", [8, xo, mo, so, rows * cp, cp // 4, 0.0])
    do = mp.alloc(rows * cp)
    mp.dispatch("n_elem", [11, xo, mo, do, rows * cp, cp // 4, 0.0])
    mp.output(mo, rows * 4, (rows, 4))
    mp.output(so, rows * cp, (rows, cp))
    mp.output(do, rows * cp, (rows, cp))
    m4, sub, div = mp.run()
    assert_bitexact(m4[:, 0], mean, "row means")
    assert np.all(m4[:, 1:] == 0.0)
    assert_bitexact(sub, oracle.binary_bcast(x, mean, rows, cp, 1, 0), "x - mean")
    assert_bitexact(div, oracle.binary_bcast(x, mean, rows, cp, 3, 0), "x / mean")


@pytest.mark.parametrize("export_d", [False, True])
def test_plan_layernorm_run_folds_into_one_launch(gpu, oracle, export_d):
    """The nine dispatches PlanBuilder writes for a LayerNorm (n_reduce_last,
    n_elem 8 / 9, n_reduce_last, n_elem 6 / 10 / 11, n_channel 0 / 1) run as
    one LayerNorm launch when no intermediate is read elsewhere, and as nine
    launches when one is (here x - mean, exported as a graph output); the
    bits are the oracle's LayerNorm either way.  Rows 0 and 5 hold a huge
    cancelling pair (their means take the sequential sum)."""
    from qppocr_amd import plan as P
    r = rng(13)
    rows, cols, eps = 37, 256, 1e-6
    x = (rnd(r, (rows, cols)) + 0.5).astype(np.float32)
    x[0, 3], x[0, 7] = 1e15, -1e15
    x[5, 9], x[5, 200] = -1e18, 1e18
    g = (1.0 + rnd(r, (cols,), 0.1)).astype(np.float32)
    bt = rnd(r, (cols,), 0.1)
    mp = MiniPlan()
    xo, go, bo = mp.static(x), mp.static(g), mp.static(bt)
    eo = mp.static(np.array([eps], np.float32))
    mo, vo, veo, so = (mp.alloc(rows * 4) for _ in range(4))
    do, sqo, y0, y1, yo = (mp.alloc(rows * cols) for _ in range(5))
    n = rows * cols
    mp.dispatch("n_reduce_last", [xo, mo, rows, cols, cols, rows], (rows, 1, 1))
    mp.dispatch("n_elem", [8, xo, mo, do, n, cols // 4, 0.0])
    mp.dispatch("n_elem", [9, do, OFF_NONE, sqo, n, 0.0, 0.0])
    mp.dispatch("n_reduce_last", [sqo, vo, rows, cols, cols, rows], (rows, 1, 1))
    mp.dispatch("n_elem", [6, vo, eo, veo, 4 * rows, 0.0, 0.0])
    mp.dispatch("n_elem", [10, veo, OFF_NONE, so, 4 * rows, 0.0, 0.0])
    mp.dispatch("n_elem", [11, do, so, y0, n, cols // 4, 0.0])
    mp.dispatch("n_channel", [0, y0, go, OFF_NONE, y1, n, cols, 0.0, 0.0, rows])
    mp.dispatch("n_channel", [1, y1, bo, OFF_NONE, yo, n, cols, 0.0, 0.0, rows])
    mp.output(yo, n, (rows, cols))
    if export_d:
        mp.output(do, n, (rows, cols))
    mp.p.total_words = mp.words
    sess = P.HipPlanSession(mp.p)
    try:
        outs = sess.run(None)
        assert sess.launches() == (9 if export_d else 1)
    finally:
        sess.close()
    ref = oracle.layernorm(x, g, bt, eps)
    assert_bitexact(outs[0], ref, "plan LayerNorm")
    if export_d:
        mean = oracle.reduce_mean_last(x)
        assert_bitexact(outs[1], oracle.binary_bcast(x, mean, rows, cols, 1, 0), "x - mean")


ELEM_UNARY = [(0, None), (1, None), (2, (0.2, 0.5)), (2, (1.0 / 6.0, 0.5)), (3, (-0.5, 0.7)),
              (9, None), (10, None)]


@pytest.mark.parametrize("op,pp", ELEM_UNARY, ids=lambda v: str(v))
def test_plan_elem_unary(gpu, oracle, op, pp):
    r = rng(20 + op)
    n = 4 * 333
    x = rnd(r, (n,), 2.0)
    if op == 10:
        x = np.abs(x)
    O = oracle
    ref = {0: lambda: O.relu_inplace(x.copy()), 1: lambda: O.sigmoid_tensor(x),
           2: lambda: O.hardsigmoid(x, *pp), 3: lambda: O.clip_inplace(x.copy(), *pp),
           9: lambda: x * x, 10: lambda: np.sqrt(x)}[op]()
    mp = MiniPlan()
    xo = mp.static(x)
    yo = mp.alloc(n)
    p1, p2 = pp if pp else (0.0, 0.0)
    mp.dispatch("n_elem", [op, xo, OFF_NONE, yo, n, p1, p2])
    mp.output(yo, n, (n,))
    assert_bitexact(mp.run()[0], ref, f"elem op {op}")


@pytest.mark.parametrize("op", [4, 5, 12, 13, 6, 7])
def test_plan_elem_binary(gpu, oracle, op):
    r = rng(40 + op)
    n = 4 * 257
    a = rnd(r, (n,))
    b = rnd(r, (n,)) + 0.5
    s = np.float32(r.standard_normal())
    O = oracle
    code = {4: 0, 5: 2, 12: 1, 13: 3, 6: 0, 7: 2}[op]
    if op in (6, 7):
        ref = O.binary_bcast(a.reshape(1, n), np.array([s], np.float32), 1, n, code, 2).reshape(n)
    else:
        ref = O.binary_flat(a, b, code)
    mp = MiniPlan()
    ao = mp.static(a)
    bo = mp.static(np.array([s, 0, 0, 0], np.float32) if op in (6, 7) else b)
    yo = mp.alloc(n)
    mp.dispatch("n_elem", [op, ao, bo, yo, n, 0.0, 0.0])
    mp.output(yo, n, (n,))
    assert_bitexact(mp.run()[0], ref, f"elem op {op}")


@pytest.mark.parametrize("op", [0, 1, 2, 3, 4, 5])
def test_plan_channel(gpu, oracle, op):
    """n_channel with two gate rows (one per batch item: hw = rows / 2)."""
    O = oracle
    r = rng(60 + op)
    frows, cp = 24, 12
    a = rnd(r, (frows, cp))
    g = rnd(r, (2, cp))
    rr = rnd(r, (frows, cp))
    sh = rnd(r, (2, cp))
    gate = np.repeat(g, frows // 2, axis=0)
    shift = np.repeat(sh, frows // 2, axis=0)
    if op == 0:
        ref = O.binary_flat(a, gate, 2)
    elif op == 1:
        ref = O.binary_flat(a, gate, 0)
    elif op == 2:
        ref = O.binary_flat(O.binary_flat(a, gate, 2), rr, 0)
    elif op == 3:
        ref = O.binary_flat(a, O.hardsigmoid(gate, 0.2, 0.5), 2)
    elif op == 4:
        ref = O.binary_flat(a, O.sigmoid_tensor(gate), 2)
    else:
        ref = O.binary_flat(O.binary_flat(a, gate, 2), shift, 0)
    mp = MiniPlan()
    ao = mp.static(a)
    go = mp.static(g)
    ro = mp.static(rr) if op == 2 else (mp.static(sh) if op == 5 else OFF_NONE)
    yo = mp.alloc(frows * cp)
    mp.dispatch("n_channel", [op, ao, go, ro, yo, frows * cp, cp, 0.2, 0.5, frows // 2])
    mp.output(yo, frows * cp, (frows, cp))
    assert_bitexact(mp.run()[0], ref, f"channel op {op}")


# ------------------------------------------------------ softmax / argmax / matmul

@pytest.mark.parametrize("rows,cols", [(6, 30), (5, 18709), (3, 25001)])
def test_plan_softmax_and_argmax_exits(gpu, oracle, rows, cols):
    """n_softmax over rows x cpad (pad columns written 0), n_exit3 and
    n_exit3_argmax on its output."""
    r = rng(cols)
    cp = (cols + 3) // 4 * 4
    x = np.zeros((rows, cp), np.float32)
    x[:, :cols] = rnd(r, (rows, cols), 3.0)
    x[:, cols:] = 99.0                       # pad columns never read
    ref = x[:, :cols].copy()
    oracle.softmax_last_dim(ref, cols)
    pairs = oracle.ctc_argmax(ref)
    mp = MiniPlan()
    xo = mp.static(x)
    po = mp.static(np.full(rows * cp, 5.0, np.float32))
    mp.dispatch("n_softmax", [xo, po, rows, cols, cp, rows], (rows, 1, 1))
    eo = mp.alloc(rows * cols)
    mp.dispatch("n_exit3", [po, eo, rows, cols, cp, rows], (1, 1, 1))
    ao = mp.alloc(rows * 2)
    mp.dispatch("n_exit3_argmax", [po, ao, rows, cols, cp, rows], (rows, 1, 1))
    mp.output(po, rows * cp, (rows, cp))
    mp.output(eo, rows * cols, (rows, cols))
    mp.output(ao, rows * 2, (rows, 2))
    p, e, a = mp.run()
    assert_bitexact(p[:, :cols], ref, "softmax")
    assert np.all(p[:, cols:] == 0.0)
    assert_bitexact(e, ref, "exit3")
    assert_bitexact(a, pairs, "pairs")


@pytest.mark.parametrize("rows,cols", [(5, 18709), (4, 300)])
def test_plan_softmax_pairs_only(gpu, oracle, rows, cols):
    """n_softmax whose output only an n_exit3_argmax reads (the rec plan's
    pairs exit): the pairs bit-exact, the probabilities left unwritten."""
    from qppocr_amd import plan
    r = rng(cols + 1)
    cp = (cols + 3) // 4 * 4
    x = np.zeros((rows, cp), np.float32)
    x[:, :cols] = rnd(r, (rows, cols), 3.0)
    ref = x[:, :cols].copy()
    oracle.softmax_last_dim(ref, cols)
    pairs = oracle.ctc_argmax(ref)
    mp = MiniPlan()
    xo = mp.static(x)
    po = mp.static(np.full(rows * cp, 5.0, np.float32))
    mp.dispatch("n_softmax", [xo, po, rows, cols, cp, rows], (rows, 1, 1))
    ao = mp.alloc(rows * 2)
    mp.dispatch("n_exit3_argmax", [po, ao, rows, cols, cp, rows], (rows, 1, 1))
    mp.output(ao, rows * 2, (rows, 2))
    mp.p.total_words = mp.words
    s = plan.HipPlanSession(mp.p)
    try:
        (a,) = s.run(None)
        left = s.read(po, rows * cp)
    finally:
        s.close()
    assert_bitexact(a, pairs, "pairs")
    assert np.all(left == 5.0)


def test_plan_attn_mm(gpu, oracle):
    r = rng(77)
    b, heads, t, dh = 2, 3, 12, 8
    a = rnd(r, (b, heads, t, dh))
    k = rnd(r, (b, heads, dh, t))
    ref = oracle.matmul(a, k)
    mp = MiniPlan()
    ao = mp.static(a)
    ko = mp.static(k)
    yo = mp.alloc(b * heads * t * t)
    mp.dispatch("n_attn_mm", [ao, ko, yo, t, dh, t, b * heads, heads], (1, b * heads * t, 1))
    mp.output(yo, b * heads * t * t, (b, heads, t, t))
    assert_bitexact(mp.run()[0], ref, "batched matmul")


@pytest.mark.parametrize("kind", ["softmax30", "softmax18709", "softmax20000", "softmax25001",
                                  "reduce_last", "gap", "attn_qk", "attn_pv"])
def test_plan_real_n_row_kernels(gpu, oracle, kind):
    """Word 0 (real_n) also stops the softmax, the row means (n_reduce_last,
    n_reduce_hw + n_reduce_fin) and the batched matmul (n_attn_mm) at the
    real batch, as n_softmax / n_reduce_last / n_reduce_fin / n_attn_mm.comp
    exit early: 3 batch items, real_n 1; the real rows bit-exact, the
    padded items' outputs keep what the arena held."""
    O = oracle
    r = rng(len(kind))
    mp = MiniPlan()
    n = 3
    S = 5.0
    if kind.startswith("softmax"):
        cols = int(kind[7:])
        rpb = 2
        rows = n * rpb
        cp = (cols + 3) // 4 * 4
        x = np.zeros((rows, cp), np.float32)
        x[:, :cols] = rnd(r, (rows, cols), 3.0)
        ref = x[:rpb, :cols].copy()
        O.softmax_last_dim(ref, cols)
        xo = mp.static(x)
        yo = mp.static(np.full(rows * cp, S, np.float32))
        mp.dispatch("n_softmax", [xo, yo, rows, cols, cp, rpb], (rows, 1, 1))
        mp.output(yo, rows * cp, (rows, cp))
        got = mp.run(real_n=1)[0]
        assert_bitexact(got[:rpb, :cols], ref, "real rows")
        assert np.all(got[rpb:] == S)
    elif kind == "reduce_last":
        rpb, cols, cp = 12, 30, 32
        rows = n * rpb
        x = np.zeros((rows, cp), np.float32)
        x[:, :cols] = rnd(r, (rows, cols)) + 1.0
        mean = O.reduce_mean_last(x[:rpb, :cols])
        xo = mp.static(x)
        mo = mp.static(np.full(rows * 4, S, np.float32))
        mp.dispatch("n_reduce_last", [xo, mo, rows, cols, cp, rpb], (rows, 1, 1))
        mp.output(mo, rows * 4, (rows, 4))
        got = mp.run(real_n=1)[0]
        assert_bitexact(got[:rpb, 0], mean, "real row means")
        assert np.all(got[rpb:] == S)
    elif kind == "gap":
        c, h, w = 20, 33, 35
        x = rnd(r, (n, c, h, w)) + 3.0
        ref = O.global_avg_pool(x[:1]).reshape(1, c)
        xo = mp.static(nhwc(x))
        scratch = mp.alloc(n * ((h * w + 1023) // 1024) * c)
        yo = mp.static(np.full(n * c, S, np.float32))
        mp.dispatch("n_reduce_hw", [xo, scratch, h * w, c], ((h * w + 1023) // 1024, n, 1))
        mp.dispatch("n_reduce_fin", [scratch, yo, (h * w + 1023) // 1024, c, h * w], (n, 1, 1))
        mp.output(yo, n * c, (n, c))
        got = mp.run(real_n=1)[0]
        assert_bitexact(got[:1], ref, "real image")
        assert np.all(got[1:] == S)
    else:
        heads, t, dh = 3, 12, 32 if kind == "attn_qk" else 8
        kk, nn = (dh, t) if kind == "attn_qk" else (t, dh)
        a = rnd(r, (n, heads, t, kk))
        bm = rnd(r, (n, heads, kk, nn))
        ref = O.matmul(a[:1], bm[:1])
        ao = mp.static(a)
        bo = mp.static(bm)
        yo = mp.static(np.full(n * heads * t * nn, S, np.float32))
        mp.dispatch("n_attn_mm", [ao, bo, yo, t, kk, nn, n * heads, heads], (1, n * heads * t, 1))
        mp.output(yo, n * heads * t * nn, (n, heads, t, nn))
        got = mp.run(real_n=1)[0]
        assert_bitexact(got[:1], ref, "real batch item")
        assert np.all(got[1:] == S)


# ------------------------------------------------------------- data movement

def test_plan_entry_exit_and_concat(gpu, oracle):
    """n_entry (NCHW -> NHWC), n_concat_c of two segments, n_exit with and
    without the fused sigmoid, n_transpose and n_transpose_nd."""
    r = rng(90)
    n, c1, c2, h, w = 2, 5, 8, 3, 4
    x1 = rnd(r, (n, c1, h, w))
    x2 = rnd(r, (n, c2, h, w))
    mp = MiniPlan()
    i1 = mp.static(x1)
    e1 = mp.alloc(n * h * w * 8)
    mp.dispatch("n_entry", [i1, e1, n, c1, h, w, 8])
    e2 = mp.static(nhwc(x2))
    cat = mp.alloc(n * h * w * 16)
    mp.dispatch("n_concat_c", [cat, n * h * w, 2, 4, e1, 2, e2, 2])
    o1 = mp.alloc(n * 16 * h * w)
    mp.dispatch("n_exit", [cat, o1, n, 16, h, w, 16, 0])
    o2 = mp.alloc(n * 16 * h * w)
    mp.dispatch("n_exit", [cat, o2, n, 16, h, w, 16, 4])
    t2 = mp.alloc(n * 16 * h * w)
    mp.dispatch("n_transpose", [o1, t2, n * 16, h * w])
    t5 = mp.alloc(n * 16 * h * w)
    mp.dispatch("n_transpose_nd", [o1, t5, n * 16 * h * w, 4, n, 16, h, w, 0, 2, 0, 3, 1, 0])
    for off, shape in [(e1, (n, h, w, 8)), (o1, (n, 16, h, w)), (o2, (n, 16, h, w)),
                       (t2, (h * w, n * 16)), (t5, (h, n, w, 16))]:
        mp.output(off, int(np.prod(shape)), shape)
    got = mp.run()
    xp1 = np.zeros((n, 8, h, w), np.float32)
    xp1[:, :c1] = x1
    cat_ref = np.concatenate([xp1, x2], 1)   # channels 5..7: x1's pad channels (0)
    assert_bitexact(got[0], nhwc(x1, 8), "entry")
    assert_bitexact(got[1], cat_ref, "concat + exit")
    assert_bitexact(got[2], oracle.sigmoid_tensor(cat_ref), "exit sigmoid")
    assert_bitexact(got[3], cat_ref.reshape(n * 16, h * w).T, "transpose")
    assert_bitexact(got[4], cat_ref.transpose(2, 0, 3, 1), "transpose nd")


def _resize_ref(x, oh, ow):
    """plan_resize_kernel's nearest map on NHWC x [n, h, w, c]."""
    n, h, w, c = x.shape
    iy = np.minimum((np.arange(oh, dtype=np.float32) * np.float32(h) / np.float32(oh)).astype(np.int64), h - 1)
    ix = np.minimum((np.arange(ow, dtype=np.float32) * np.float32(w) / np.float32(ow)).astype(np.int64), w - 1)
    return x[:, iy][:, :, ix]


@pytest.mark.parametrize("order,export_resized", [(0, False), (1, False), (0, True)])
def test_plan_resize_fusions(gpu, oracle, order, export_resized):
    """n_resize + n_elem add (either operand order) as one pass, and resizes
    that only an n_concat_c reads, read through by it (the det neck); with
    a resized map also exported, the resizes run as dispatched.  Every
    output equals numpy's nearest resize, add and concat."""
    from qppocr_amd import plan
    r = rng(5 + order + 2 * export_resized)
    n = 2
    a = rnd(r, (n, 5, 7, 8))            # coarse map, 8 channels
    y = rnd(r, (n, 10, 14, 8))          # fine lateral
    c1 = rnd(r, (n, 3, 4, 4))           # concat inputs: two coarse, one full size
    c2 = rnd(r, (n, 6, 7, 4))
    c3 = rnd(r, (n, 12, 14, 4))
    mp = MiniPlan()
    ao, yo = mp.static(a), mp.static(y)
    o1, o2, o3 = mp.static(c1), mp.static(c2), mp.static(c3)
    ra = mp.alloc(n * 10 * 14 * 8)
    mp.dispatch("n_resize", [ao, ra, 10 * 14, 8, 14, 7, 5, 0.5, 0.5], (1, n, 1))
    so = mp.alloc(n * 10 * 14 * 8)
    mp.dispatch("n_elem", [4, ra, yo, so, n * 10 * 14 * 8, 0.0, 0.0] if order == 0 else
                [4, yo, ra, so, n * 10 * 14 * 8, 0.0, 0.0])
    r1 = mp.alloc(n * 12 * 14 * 4)
    mp.dispatch("n_resize", [o1, r1, 12 * 14, 4, 14, 4, 3, 0.25, 0.25], (1, n, 1))
    r2 = mp.alloc(n * 12 * 14 * 4)
    mp.dispatch("n_resize", [o2, r2, 12 * 14, 4, 14, 7, 6, 0.5, 0.5], (1, n, 1))
    cat = mp.alloc(n * 12 * 14 * 12)
    mp.dispatch("n_concat_c", [cat, n * 12 * 14, 3, 3, r1, 1, r2, 1, o3, 1])
    mp.output(so, n * 10 * 14 * 8, (n, 10, 14, 8))
    mp.output(cat, n * 12 * 14 * 12, (n, 12, 14, 12))
    if export_resized:
        mp.output(r1, n * 12 * 14 * 4, (n, 12, 14, 4))
    got = mp.run()
    assert_bitexact(got[0], _resize_ref(a, 10, 14) + y, "resize + add")
    cat_ref = np.concatenate([_resize_ref(c1, 12, 14), _resize_ref(c2, 12, 14), c3], -1)
    assert_bitexact(got[1], cat_ref, "concat of resized maps")
    if export_resized:
        assert_bitexact(got[2], _resize_ref(c1, 12, 14), "exported resize")


@pytest.mark.parametrize("dims,perm", [
    ((2, 5, 3, 4, 8), (2, 0, 3, 1, 4)),    # innermost axis kept, 4 | 8: 16-byte moves
    ((3, 7, 12), (1, 0, 2)),
    ((2, 3, 5, 6, 7), (4, 2, 0, 1, 3)),    # innermost axis moved: element moves
    ((4, 9, 5), (2, 1, 0)),
])
def test_plan_transpose_nd_paths(gpu, oracle, dims, perm):
    """n_transpose_nd against numpy's transpose on both of the kernel's paths."""
    r = rng(sum(dims) * 7 + perm[0])
    x = rnd(r, dims)
    mp = MiniPlan()
    xo = mp.static(x)
    yo = mp.alloc(x.size)
    dd = list(dims) + [1] * (5 - len(dims))
    pp = list(perm) + [0] * (5 - len(perm))
    mp.dispatch("n_transpose_nd", [xo, yo, x.size, len(dims), *dd, *pp])
    ref = np.ascontiguousarray(x.transpose(perm))
    mp.output(yo, x.size, ref.shape)
    (got,) = mp.run()
    assert_bitexact(got, ref, "transpose nd")


# ------------------------------------------------------------------ fusion

@pytest.mark.parametrize("export_conv", [False, True])
def test_plan_epilogue_fusion_respects_readers(gpu, oracle, export_conv):
    """Conv -> HardSigmoid -> Mul -> Add(residual) and MatMul -> Add(bias):
    the session folds the consumers into the producer's epilogue only when
    nothing else reads the intermediate regions; exporting the conv output
    keeps the three conv launches apart.  Same values either way."""
    from qppocr_amd import plan
    O = oracle
    r = rng(123)
    n, c, h, w, m = 1, 8, 10, 12, 16
    x = rnd(r, (n, c, h, w))
    wt = rnd(r, (m, c, 3, 3), 0.2)
    b = rnd(r, (m,), 0.1)
    res = rnd(r, (n, m, h, w))
    conv = O.conv2d(x, wt, b, O.conv_params(1, 1, 1, 1))
    hs = O.hardsigmoid(conv, 1.0 / 6.0, 0.5)
    ref = O.binary_flat(O.binary_flat(conv, hs, 2), res, 0)
    rows, k, nn = 20, 12, 20
    a = rnd(r, (rows, k))
    bm = rnd(r, (k, nn), 0.3)
    bb = rnd(r, (nn,), 0.1)
    mm_ref = O.binary_bcast(O.matmul(a, bm), bb, rows, nn, 0, 1)
    mp = MiniPlan()
    xo = mp.static(nhwc(x))
    wo = mp.static(np.concatenate([plan.repack_conv_w(wt, m, c, 3, 3), np.zeros(32, np.uint32)]))
    bo = mp.static(plan.conv_bias(b, m))
    ro = mp.static(nhwc(res))
    words = n * h * w * m
    co = mp.alloc(words)
    mp.dispatch("n_conv8", [xo, wo, bo, co, h * w, m, w, w, h, 2, 9, 3, 1, 1, 1, 1, 0,
                            *plan.GELU_C, OFF_NONE], (1, n, 1))
    ho = mp.alloc(words)
    mp.dispatch("n_elem", [2, co, OFF_NONE, ho, words, 1.0 / 6.0, 0.5])
    mo = mp.alloc(words)
    mp.dispatch("n_elem", [5, co, ho, mo, words, 0.0, 0.0])
    yo = mp.alloc(words)
    mp.dispatch("n_elem", [4, ro, mo, yo, words, 0.0, 0.0])
    ao = mp.static(a)
    bmo = mp.static(np.concatenate([plan.repack_conv_w(bm.T, nn, k, 1, 1), np.zeros(32, np.uint32)]))
    mmo = mp.alloc(rows * nn)
    mp.dispatch("n_conv8", [ao, bmo, OFF_NONE, mmo, rows, nn, rows, rows, 1, k // 4, 1, 1, 1, 1, 0,
                            0, 0, *plan.GELU_C, OFF_NONE], (1, 1, 1))
    bvo = mp.static(plan.vector_nhwc(bb))
    mbo = mp.alloc(rows * nn)
    mp.dispatch("n_channel", [1, mmo, bvo, OFF_NONE, mbo, rows * nn, nn, 0.0, 0.0, rows])
    mp.output(yo, words, (n, h, w, m))
    mp.output(mbo, rows * nn, (rows, nn))
    if export_conv:
        mp.output(co, words, (n, h, w, m))
    mp.p.total_words = mp.words
    s = plan.HipPlanSession(mp.p)
    got = s.run(None)
    launches = s.launches()
    s.close()
    assert launches == (5 if export_conv else 2)
    assert_bitexact(got[0], nhwc(ref), "conv + hardswish + residual")
    assert_bitexact(got[1], mm_ref, "matmul + bias")
    if export_conv:
        assert_bitexact(got[2], nhwc(conv), "conv output")


# ------------------------------------------------------------------- checks

def test_plan_create_refuses_bad_plans(gpu):
    from qppocr_amd import _lib
    with pytest.raises(_lib.QphError, match="not in the HIP kernel set"):
        _lib.check(_lib.load().qph_plan_kernel_id(b"n_conv8_mma"))
    mp = MiniPlan()
    xo = mp.alloc(16)
    mp.dispatch("n_elem", [0, xo, OFF_NONE, xo + 1000, 16, 0.0, 0.0])   # output past the arena
    mp.output(xo, 16, (16,))
    with pytest.raises(_lib.QphError, match="outside the arena"):
        mp.run()
    mp = MiniPlan()
    xo = mp.alloc(16)
    mp.dispatch("n_reduce_fin", [xo, xo, 1, 4, 4], (1, 1, 1))         # no n_reduce_hw before it
    mp.output(xo, 4, (4,))
    with pytest.raises(_lib.QphError, match="n_reduce_hw"):
        mp.run()


# -------------------------------------------------------------- whole graphs

def test_plan_det_graph(gpu, oracle):
    """The det graph (stem, dw/pw blocks, FPN, concat, head, ConvT pair +
    Sigmoid) planned as PlanBuilder lowers it, run on the HIP kernel set:
    bit-exact against the oracle's run of the same graph."""
    from oracle import nets as onets
    from qppocr_amd import nets, plan
    g, x = nets.build_det(2, 96, 64)
    pl = plan.build_plan(g)
    print("plan det", len(pl.dispatches), "dispatches", flush=True)
    s = plan.HipPlanSession(pl)
    got = s.run(x)
    assert s.launches() < len(pl.dispatches)     # hardswish / residual epilogues absorbed
    s.close()
    ref = onets.run_graph(g, x)
    assert_bitexact(got[0], ref[0], "det map")


@pytest.mark.parametrize("probs", [True, False])
def test_plan_rec_graph(gpu, oracle, probs):
    """The rec graph (stem, blocks, two encoder layers with the LayerNorm
    chain and attention, CTC head) planned and run; probabilities and the
    (value, index) pairs bit-exact against the oracle."""
    from oracle import nets as onets
    from qppocr_amd import nets, plan
    g, x = nets.build_rec(3, 2, 160, probs=probs)
    pl = plan.build_plan(g)
    print("plan rec", len(pl.dispatches), "dispatches", flush=True)
    s = plan.HipPlanSession(pl)
    got = s.run(x)
    s.close()
    ref = onets.run_graph(g, x)
    for i, (a, b) in enumerate(zip(got, ref)):
        assert_bitexact(a, b, f"output {i}")


def test_plan_rec_padded_batch_real_n(gpu, oracle):
    """A rec plan built for a padded batch of 3 run with real_n = 2 (the
    reference session's batch grain, vulkan/session.rs:283-296): the two
    real items' pairs equal the oracle's run of the 2-item graph; the padded
    item holds garbage and is never read."""
    from oracle import nets as onets
    from qppocr_amd import nets, plan
    x2, r = nets.rec_input(3, 2, 48, 160)
    ws = nets.rec_weights(r)
    g2 = nets.build_rec_graph(ws, 2, 160, probs=False)
    g3 = nets.build_rec_graph(ws, 3, 160, probs=False)
    x3 = np.concatenate([x2, np.full((1, 3, 48, 160), 1e30, np.float32)], 0)
    s = plan.HipPlanSession(plan.build_plan(g3))
    got = s.run(x3, real_n=2)[0]
    s.close()
    ref = onets.run_graph(g2, x2)[0]
    assert_bitexact(got[:2], ref, "pairs of the real items")
