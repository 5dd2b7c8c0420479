"""Pins the CPU oracle (plain-C restatement of the qppocr-kernels CPU path).

Against: the known-answer data of the reference's own tests
(tests/golden/reference_known_answers.json, each entry citing its source),
the reference tests' f64 brute-force checks re-run with the reference's own
xorshift64* data, closed-form arithmetic cases chosen so that a plausible
transcription mistake (wrong accumulation order, bias added at the wrong
place, wrong tie rule) gives a different exact answer, and float64
library routines (numpy, torch on the CPU).
"""
import json
import math
import os

import numpy as np
import pytest

from conftest import XorShift, rel_check

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                   "reference_known_answers.json")))


def ref_conv_f64(x, w, b, sh, sw, ph, pw, group, peh=None, pew=None):
    """f64 NCHW conv with groups (the reference's ref_conv, kernels.rs:94-141)."""
    peh = ph if peh is None else peh
    pew = pw if pew is None else pew
    n, c, h, wd = x.shape
    m, cg, kh, kw = w.shape
    oh = (h + ph + peh - kh) // sh + 1
    ow = (wd + pw + pew - kw) // sw + 1
    xp = np.zeros((n, c, h + ph + peh + sh * 2, wd + pw + pew + sw * 2), np.float64)
    xp[:, :, ph:ph + h, pw:pw + wd] = x
    mg = m // group
    y = np.zeros((n, m, oh, ow), np.float64)
    for g in range(group):
        xs = xp[:, g * cg:(g + 1) * cg]
        for ky in range(kh):
            for kx in range(kw):
                patch = xs[:, :, ky:ky + sh * oh:sh, kx:kx + sw * ow:sw]   # n, cg, oh, ow
                wt = w[g * mg:(g + 1) * mg, :, ky, kx].astype(np.float64)    # mg, cg
                y[:, g * mg:(g + 1) * mg] += np.einsum("mc,nchw->nmhw", wt, patch)
    if b is not None:
        y += b.astype(np.float64)[None, :, None, None]
    return y


# ------------------------------------------------------- exp / erf polynomials

def test_erf_known_values(oracle):
    g = GOLD["erf_table"]
    for x, r in g["points"]:
        assert abs(float(oracle.erf1(x)) - r) < g["tol"], (x, oracle.erf1(x), r)


def test_exp_relative_error_sweep(oracle):
    g = GOLD["exp_sweep"]
    x = np.float32(g["start"])
    step = np.float32(g["step"])
    n = 0
    while x <= g["stop"]:
        got = float(oracle.exp1(x))
        ref = math.exp(float(x))
        assert abs(got - ref) / max(ref, 1e-30) < g["rel_tol"], (x, got)
        x = np.float32(x + step)
        n += 1
    assert n > 2000


def test_exp_saturation_and_erf_odd(oracle):
    for a, b in GOLD["exp_saturation"]["pairs"]:
        assert oracle.exp1(a) == oracle.exp1(b)
    for v in GOLD["erf_odd"]["values"]:
        a = np.float32(oracle.erf1(-v)).view(np.uint32)
        b = np.float32(-oracle.erf1(v)).view(np.uint32)
        assert a == b, v
    # exp1(0) is exactly 1 (kf = 0, r = 0, Horner gives 1)
    assert oracle.exp1(0.0) == np.float32(1.0)


# -------------------------------------------------------------- activations

def test_activations_vs_f64(oracle):
    """kernels.rs:1038-1141 on the reference's own 4096 xorshift values."""
    tol = GOLD["activation_tolerances"]
    rng = XorShift(int(GOLD["rng"]["kernels_seed"], 16))
    x = rng.fill((4096,))
    xd = x.astype(np.float64)
    relu = oracle.relu_inplace(x.copy())
    want = np.where(x > 0, x, np.float32(0))
    assert (relu.view(np.uint32) == want.view(np.uint32)).all()
    sig = oracle.sigmoid_tensor(x)
    assert np.abs(sig - 1 / (1 + np.exp(-xd))).max() < tol["sigmoid"]
    hs = oracle.hardsigmoid(x, np.float32(1 / 6), np.float32(0.5))
    a = np.float32(1 / 6)
    assert np.abs(hs - np.clip(xd * float(a) + 0.5, 0, 1)).max() < tol["hardsigmoid"]
    gl = oracle.gelu_inplace(x.copy(), 1.4142135, 1.0, 0.5)
    ax = np.abs(xd / 1.4142135)
    tt = 1 / (0.3275911 * ax + 1)
    poly = tt * ((((1.061405429 * tt - 1.453152027) * tt + 1.421413741) * tt - 0.284496736) * tt
                 + 0.254829592)
    er = 1 - poly * np.exp(-ax * ax)
    er = np.where(xd < 0, -er, er)
    assert np.abs(gl - 0.5 * xd * (er + 1)).max() < tol["gelu"]
    ei = oracle.erf_inplace(x.copy())
    assert (ei == np.array([oracle.erf1(v) for v in x[:256]] + list(ei[256:]))).all()
    cl = oracle.clip_inplace(x.copy(), -0.3, 0.7)
    lo, hi = np.float32(-0.3), np.float32(0.7)
    want = np.where(x < lo, lo, np.where(hi < x, hi, x))
    assert (cl.view(np.uint32) == want.view(np.uint32)).all()


def test_binary_scalar_both_orders(oracle):
    """The one-element broadcast of binary_op (elementwise.rs:350-363): each
    op is the IEEE single op with the scalar on the side asked for (a
    swapped Sub or Div operand fails), as numpy's float32 ops give it."""
    rng = np.random.default_rng(5)
    x = rng.normal(0, 2, 4099).astype(np.float32)
    x[::9] = 0.0
    s = np.float32(-1.375)
    with np.errstate(divide="ignore", invalid="ignore"):
        for op, f in enumerate((np.add, np.subtract, np.multiply, np.divide)):
            for first in (False, True):
                got = oracle.binary_scalar(x, s, op, scalar_first=first)
                want = f(s, x) if first else f(x, s)
                assert want.dtype == np.float32
                assert (got.view(np.uint32) == want.view(np.uint32)).all(), (op, first)
    assert not (oracle.binary_scalar(x, s, 1, True) == oracle.binary_scalar(x, s, 1, False)).all()


def test_hardswish_clip_chain_order(oracle):
    """The oracle executor runs the Add(3) / Clip(0, 6) / Mul / Div(6) form as
    four nodes, each rounding to f32: (x * clip(x + 3)) / 6, which differs
    from x * (clip(x + 3) / 6) and from the HardSigmoid + Mul form on some
    inputs, so the order of the roundings is what is checked."""
    from oracle import nets as onets
    rng = np.random.default_rng(6)
    x = rng.normal(0, 3, 20000).astype(np.float32)
    y = onets._act_nodes(x.copy(), (onets.ACT_HARDSWISH_CLIP, 3.0, 6.0, 6.0))
    t = np.minimum(np.maximum(x + np.float32(3), np.float32(0)), np.float32(6))
    want = (x * t) / np.float32(6)
    assert (y == want).all()
    other = x * (t / np.float32(6))
    assert (y != other).any()
    hs = onets._act_nodes(x.copy(), oracle.ACT_HARDSWISH)
    assert (y != hs).any()


def test_softmax_invariants(oracle):
    tol = GOLD["activation_tolerances"]
    rng = XorShift(int(GOLD["rng"]["kernels_seed"], 16))
    t = rng.fill((37, 13))
    oracle.softmax_last_dim(t, 13)
    assert np.abs(t.astype(np.float64).sum(1) - 1).max() < tol["softmax_rowsum"]
    t4 = rng.fill((4, 4))
    orig = t4.astype(np.float64).copy()
    oracle.softmax_last_dim(t4, 4)
    e = np.exp(orig - orig.max(1, keepdims=True))
    assert np.abs(t4 - e / e.sum(1, keepdims=True)).max() < tol["softmax4"]
    # wide rows (the rec head width) against f64
    w = (np.random.default_rng(0).standard_normal((8, 18709)) * 3).astype(np.float32)
    p = oracle.softmax_last_dim(w.copy(), 18709)
    e = np.exp(w.astype(np.float64) - w.max(1, keepdims=True))
    rel_check(p, e / e.sum(1, keepdims=True))


def test_hardswish_closed_forms(oracle):
    x = np.array([3.0, 4.5, 100.0, -3.0, -7.0, 0.0], np.float32)
    hs = oracle.binary_flat(x, oracle.hardsigmoid(x), 2)
    assert (hs[:3] == x[:3]).all() and (hs[3:] == 0).all()
    s = oracle.sigmoid_tensor(np.array([-50.0, 0.0, 50.0], np.float32))
    assert 0 < s[0] < 1e-20 and s[1] == 0.5 and s[2] == 1.0


# -------------------------------------------------------------------- conv

@pytest.mark.parametrize("case", GOLD["conv_cases"]["cases"], ids=lambda c: c[0])
def test_conv_cases_vs_f64(oracle, case):
    name, n, c, m, h, w, kh, kw, sh, sw, ph, pw, group, has_b = case
    rng = XorShift(int(GOLD["rng"]["kernels_seed"], 16))
    x = rng.fill((n, c, h, w))
    wt = rng.fill((m, c // group, kh, kw))
    b = rng.fill((m,)) if has_b else None
    y = oracle.conv2d(x, wt, b, oracle.conv_params(sh, sw, ph, pw, group=group))
    rel_check(y, ref_conv_f64(x, wt, b, sh, sw, ph, pw, group))


def test_conv_vs_torch_f64(oracle):
    torch = pytest.importorskip("torch")
    F = torch.nn.functional
    rng = np.random.default_rng(1)
    for (c, m, k, s, g) in [(3, 16, 3, 2, 1), (32, 32, 3, 1, 1), (64, 64, 5, 2, 64), (16, 32, 1, 1, 1)]:
        x = rng.standard_normal((2, c, 23, 19)).astype(np.float32)
        w = rng.standard_normal((m, c // g, k, k)).astype(np.float32)
        b = rng.standard_normal(m).astype(np.float32)
        y = oracle.conv2d(x, w, b, oracle.conv_params(s, s, k // 2, k // 2, group=g))
        ref = F.conv2d(torch.from_numpy(x).double(), torch.from_numpy(w).double(),
                       torch.from_numpy(b).double(), stride=s, padding=k // 2, groups=g).numpy()
        rel_check(y, ref)


def test_depthwise_end_pad_closed_form(oracle):
    """kernels.rs:594-635: end padding larger than begin padding."""
    x = np.ones((1, 4, 1, 1), np.float32)
    w = np.zeros((4, 1, 3, 3), np.float32)
    for o in range(4):
        w[o, 0, 0, 0] = 10.0 + o
    b = np.arange(4, dtype=np.float32)
    y = oracle.conv2d(x, w, b, oracle.conv_params(1, 1, 0, 0, 2, 2, group=4))
    assert y.shape == (1, 4, 1, 1)
    assert (y.ravel() == np.array(GOLD["depthwise_end_pad"]["expected"], np.float32)).all()


def test_conv_accumulation_order(oracle):
    """The implicit-GEMM k order is ch -> ky -> kx (conv.rs:595-615) and the
    depthwise order is ky outer, kx inner (conv.rs:45-71).  With terms 2^24,
    1, 1 the f32 chain gives 2^24 when 2^24 comes first and 2^24 + 2 when it
    comes last, so the two orders give different exact answers."""
    big = np.float32(2.0 ** 24)
    # dense: 2^24 at (ch0, ky2, kx2) = k 8, ones at (ch1, ky0, kx0/kx1) = k 9, 10
    x = np.ones((1, 2, 3, 3), np.float32)
    w = np.zeros((1, 2, 3, 3), np.float32)
    w[0, 0, 2, 2] = big
    w[0, 1, 0, 0] = 1
    w[0, 1, 0, 1] = 1
    y = oracle.conv2d(x, w, None, oracle.conv_params(1, 1, 0, 0))
    assert y.ravel()[0] == big            # ch-major: 2^24 + 1 + 1 rounds back to 2^24
    # depthwise: 2^24 at (ky0, kx2), ones at (ky1, kx0), (ky1, kx1)
    x = np.ones((1, 1, 3, 3), np.float32)
    w = np.zeros((1, 1, 3, 3), np.float32)
    w[0, 0, 0, 2] = big
    w[0, 0, 1, 0] = 1
    w[0, 0, 1, 1] = 1
    y = oracle.conv2d(x, w, None, oracle.conv_params(1, 1, 0, 0, group=1))
    assert y.ravel()[0] == big
    w2 = np.zeros((2, 1, 3, 3), np.float32)
    w2[:] = w
    y = oracle.conv2d(np.ones((1, 2, 3, 3), np.float32), w2, None,
                      oracle.conv_params(1, 1, 0, 0, group=2))
    assert (y.ravel() == big).all()
    # a bias-first chain would give 2^24 + 2 here; the reference adds it last
    y = oracle.conv2d(np.ones((1, 2, 3, 3), np.float32), w2, np.ones(2, np.float32),
                      oracle.conv_params(1, 1, 0, 0, group=2))
    assert (y.ravel() == big).all()


def _im2col_seed_pattern(oh, ow, tile):
    """Columns the reference's im2col branch seeds with the bias in an M%4
    tail row: tiles of `tile` output rows, N = rows * ow per tile GEMM, the
    panel rule over the tile's flattened columns (gemm.rs:7-16)."""
    pat = np.zeros((oh, ow), bool)
    for oy0 in range(0, oh, tile):
        rows = min(tile, oh - oy0)
        n = rows * ow
        for j in range(n):
            if n - (j // 32) * 32 < 32:
                pat[oy0 + j // ow, j % ow] = True
    return pat


@pytest.mark.parametrize("shape", [(31, 31, 1, 2), (301, 301, 7, 16)],
                         ids=["one tile", "tiles of 6 rows"])
def test_conv_im2col_bias_placement(oracle, shape):
    """x-stride 3 runs the im2col branch (conv.rs:639-661): one sgemm per
    tile of rows with N = rows * ow, so the M%4-tail seeding follows the
    tile's flattened columns, not each output row.  Chain 1, then 2^24,
    bias 1: seeded gives 2^24 + 2, added after gives 2^24 -- the pattern of
    2^24 + 2 in the tail row (row 4 of 5) shows where the bias went."""
    h, w, k, cg = shape
    big = np.float32(2.0 ** 24)
    x = np.ones((1, cg, h, w), np.float32)
    x[0, 1] = big
    wt = np.zeros((5, cg, k, k), np.float32)
    wt[:, 0, 0, 0] = 1            # k index 0
    wt[:, 1, 0, 0] = 1            # k index k*k (channel 1, tap 0): after it
    y = oracle.conv2d(x, wt, np.ones(5, np.float32), oracle.conv_params(3, 3, 0, 0))
    oh, ow = y.shape[2:]
    kk = cg * k * k
    tile = min(oh, max(1, (1 << 19) // (kk * ow)))
    if k == 7:
        assert tile == 6 and oh == 99       # several tiles, last one partial
    pat = _im2col_seed_pattern(oh, ow, tile)
    assert (y[0, :4] == big).all()
    assert (y[0, 4][pat] == big + 2).all() and (y[0, 4][~pat] == big).all()
    # the per-row rule of the implicit-GEMM branch would differ here
    per_row = np.ones((oh, ow), bool) if ow < 32 else None
    if per_row is not None:
        assert (pat != per_row).any()


def test_conv_general_forms_vs_f64(oracle):
    """Convs outside the reference test list that the dispatcher must still
    run as convolutions: x-stride 3 (im2col branch), a padded 1x1 conv, a
    depthwise conv with channel multiplier 2 (general branch), a 7x7 and a
    2x3 dense kernel, and groups with several channels each."""
    rng = XorShift(int(GOLD["rng"]["kernels_seed"], 16))
    cases = [  # n, c, m, h, w, kh, kw, sh, sw, ph, pw, group
        (1, 8, 12, 31, 29, 3, 3, 3, 3, 1, 1, 1),
        (2, 6, 10, 20, 22, 5, 5, 1, 3, 2, 2, 2),
        (1, 8, 13, 12, 14, 1, 1, 1, 1, 1, 2, 1),
        (1, 8, 16, 17, 19, 3, 3, 1, 1, 1, 1, 8),
        (1, 5, 7, 23, 21, 7, 7, 2, 2, 3, 3, 1),
        (1, 6, 9, 15, 18, 2, 3, 1, 2, 0, 1, 3),
    ]
    for n, c, m, h, w, kh, kw, sh, sw, ph, pw, g in cases:
        x = rng.fill((n, c, h, w))
        wt = rng.fill((m, c // g, kh, kw))
        b = rng.fill((m,))
        y = oracle.conv2d(x, wt, b, oracle.conv_params(sh, sw, ph, pw, group=g))
        rel_check(y, ref_conv_f64(x, wt, b, sh, sw, ph, pw, g))


# -------------------------------------------------------------------- sgemm

def test_sgemm_shapes_vs_f64(oracle):
    rng = XorShift(int(GOLD["rng"]["kernels_seed"], 16))
    for m, n, k in GOLD["sgemm_shapes"]["shapes"]:
        if m * n * k > 3e6:
            rng2 = np.random.default_rng(m + n + k)
            a = rng2.uniform(-1, 1, (m, k)).astype(np.float32)
            b = rng2.uniform(-1, 1, (k, n)).astype(np.float32)
            bias = rng2.uniform(-1, 1, m).astype(np.float32)
        else:
            a = rng.fill((m, k))
            b = rng.fill((k, n))
            bias = rng.fill((m,))
        c = oracle.sgemm(a, b, m, n, k, bias)
        rel_check(c, a.astype(np.float64) @ b + bias[:, None].astype(np.float64))


def test_sgemm_bias_placement(oracle):
    """gemm.rs:7-16.  Row chain 1, then 2^24, plus bias 1: adding the bias after
    the chain gives 2^24; seeding the chain with it gives 2^24 + 2."""
    big = 2.0 ** 24

    def run(m, n, k, serial=False):
        a = np.zeros((m, k), np.float32)
        a[:, :2] = 1
        b = np.zeros((k, n), np.float32)
        b[0] = 1
        b[1] = big
        return oracle.sgemm(a, b, m, n, k, np.ones(m, np.float32), serial=serial)

    c = run(5, 5, 2)            # panel path, partial panel: row 4 is the M%4 tail
    assert (c[:4] == big).all() and (c[4] == big + 2).all()
    c = run(5, 40, 2)           # full first panel: tail row seeded only past column 32
    assert (c[4, :32] == big).all() and (c[4, 32:] == big + 2).all()
    c = run(64, 16, 4000)       # parallel m-rows path (n <= 32): every column seeded
    assert oracle.sgemm_path(64, 16, 4000) == 1
    assert (c == big + 2).all()
    c = run(64, 16, 4000, serial=True)   # serial panel path: no tail rows (64 % 4 == 0)
    assert (c == big).all()
    c = run(8, 64, 3)           # full panels, M % 4 == 0: never seeded
    assert (c == big).all()


# ----------------------------------------------------- matmul / LN / reduce

def test_matmul_vs_f64(oracle):
    rng = XorShift(int(GOLD["rng"]["kernels_seed"], 16))
    a = rng.fill(tuple(GOLD["matmul"]["a_shape"]))
    b = rng.fill(tuple(GOLD["matmul"]["b_shape"]))
    rel_check(oracle.matmul(a, b), a.astype(np.float64) @ b)
    a = rng.fill((3, 40, 32))
    b = rng.fill((3, 32, 40))
    rel_check(oracle.matmul(a, b), np.matmul(a.astype(np.float64), b))


def test_reduce_mean_exact(oracle):
    rng = XorShift(int(GOLD["rng"]["kernels_seed"], 16))
    x = rng.fill((2, 3, 4, 5))
    got = oracle.reduce_mean_last(x.reshape(6, 20))
    want = np.array([np.float32(x.reshape(6, 20)[i].astype(np.float64).sum() / 20.0)
                     for i in range(6)])
    assert (got == want).all()


def test_reduce_mean_sequential_order(oracle):
    """shape.rs:551-557 sums each row in ascending order in f64.  Row
    [2^60, -2^60, 1 x 254]: in that order the ones survive (sum 254); a
    pairwise or lane-strided order adds them to +-2^60 first, where they are
    lost (|2^60| has an f64 ulp of 256)."""
    row = np.ones(256, np.float32)
    row[0], row[1] = 2.0 ** 60, -(2.0 ** 60)
    x = np.stack([row, row[::-1].copy()])
    got = oracle.reduce_mean_last(x)
    for i in range(2):
        s = 0.0
        for v in x[i]:
            s += float(v)
        assert got[i] == np.float32(s / 256)
    assert got[0] == np.float32(254 / 256)
    # the strided (64-lane) order would give something else entirely
    lanes = [sum(float(v) for v in row[l::64]) for l in range(64)]
    assert np.float32(sum(lanes) / 256) != got[0]


def test_layernorm_vs_f64_and_pow_square(oracle):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((64, 256)) * 2 + 1).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(256)).astype(np.float32)
    b = (0.1 * rng.standard_normal(256)).astype(np.float32)
    y = oracle.layernorm(x, g, b, 1e-6)
    xd = x.astype(np.float64)
    mu = xd.mean(1, keepdims=True)
    var = ((xd - mu) ** 2).mean(1, keepdims=True)
    ref = (xd - mu) / np.sqrt(var + 1e-6) * g + b
    rel_check(y, ref, tol=2e-6)
    # The LayerNorm's Pow(2) is the correctly rounded square (the reference GPU
    # plan's lowering).  The CPU executor's runtime libm powf (the Pow node of
    # binary_op) is within one ulp of it and equal for nearly every input.
    d = (rng.standard_normal(200000) * 3).astype(np.float32)
    sq = oracle.binary_flat(d, np.full_like(d, 2.0), 4)
    exact = (d.astype(np.float64) ** 2).astype(np.float32)
    assert (exact == d * d).all()
    ulps = np.abs(sq.view(np.int32).astype(np.int64) - exact.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1 and (ulps > 0).mean() < 0.005
    # the chain uses the square: a row whose squares libm would round differently
    one = np.zeros((1, 256), np.float32)
    one[0, :128] = d[:128]
    one[0, 128:] = -d[:128]
    y1 = oracle.layernorm(one, np.ones(256, np.float32), np.zeros(256, np.float32), 1e-6)
    mu = np.float32(one[0].astype(np.float64).sum() / 256)
    dd = one[0] - mu
    var = np.float32((dd * dd).astype(np.float64).sum() / 256)
    sd = np.sqrt(np.float32(var + np.float32(1e-6)), dtype=np.float32)
    assert (y1[0] == (dd / sd) * np.float32(1) + np.float32(0)).all()


# ----------------------------------------------------- convT / resize / CTC

def test_convtranspose_vs_f64(oracle):
    rng = XorShift(int(GOLD["rng"]["kernels_seed"], 16))
    n, c, h, w = GOLD["convtranspose"]["x_shape"]
    m = GOLD["convtranspose"]["m"]
    x = rng.fill((n, c, h, w))
    wt = rng.fill((c, m, 2, 2))
    y = oracle.convtranspose2d(x, wt)
    xd = x.astype(np.float64)
    ref = np.einsum("nchw,cmyx->nmhywx", xd, wt.astype(np.float64)).reshape(n, m, 2 * h, 2 * w)
    assert y.shape == ref.shape
    assert (np.abs(y - ref) / np.maximum(np.abs(ref), 1e-6)).max() < 1e-5


def test_convtranspose_vs_torch(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(4)
    x = rng.standard_normal((1, 24, 9, 11)).astype(np.float32)
    w = rng.standard_normal((24, 24, 2, 2)).astype(np.float32)
    ref = torch.nn.functional.conv_transpose2d(torch.from_numpy(x).double(),
                                               torch.from_numpy(w).double(), stride=2).numpy()
    rel_check(oracle.convtranspose2d(x, w), ref)


def test_resize_nearest_exact(oracle):
    rng = XorShift(int(GOLD["rng"]["kernels_seed"], 16))
    n, c, h, w = GOLD["resize_nearest"]["x_shape"]
    oh, ow = GOLD["resize_nearest"]["out"]
    x = rng.fill((n, c, h, w))
    y = oracle.resize_nearest(x, oh, ow)
    for oy in range(oh):
        iy = min(int(np.float32(oy) * np.float32(h) / np.float32(oh)), h - 1)
        for ox in range(ow):
            ix = min(int(np.float32(ox) * np.float32(w) / np.float32(ow)), w - 1)
            assert (y[:, :, oy, ox] == x[:, :, iy, ix]).all()
    # exact 2x: index oy >> 1
    y2 = oracle.resize_nearest(x, 2 * h, 2 * w)
    assert (y2 == x.repeat(2, 2).repeat(2, 3)).all()


def test_ctc_argmax_and_collapse(oracle):
    for row, want in GOLD["ctc"]["argmax_rows"]:
        pairs = oracle.ctc_argmax(np.array([row], np.float32))
        assert oracle.pairs_ids(pairs)[0] == want
        assert pairs[0, 0] == np.float32(max(row))
    for ids, want in GOLD["ctc"]["collapse"]:
        pairs = np.zeros((len(ids), 2), np.float32)
        pairs[:, 0] = 0.5
        pairs[:, 1] = np.array(ids, np.uint32).view(np.float32)
        got, conf = oracle.ctc_collapse(pairs, len(ids))
        assert list(got) == want
        assert conf == (0.5 if want else 0.0)


# ------------------------------------------------------------ whole graphs

def test_det_graph_invariants(oracle):
    from qppocr_amd import nets
    from oracle import nets as onets
    g, x = nets.build_det(2, 64, 64)
    out = onets.run_graph(g, x)[0]
    assert out.shape == (1, 1, 64, 64)
    assert (out > 0).all() and (out < 1).all()


def test_rec_graph_invariants(oracle):
    from qppocr_amd import nets
    from oracle import nets as onets
    g, x = nets.build_rec(3, 2, 160)
    probs, pairs = onets.run_graph(g, x)
    assert probs.shape == (2, 20, nets.REC_CLASSES) and pairs.shape == (2, 20, 2)
    assert np.abs(probs.astype(np.float64).sum(-1) - 1).max() < 1e-4
    ids = oracle.pairs_ids(pairs)
    assert (ids == probs.argmax(-1)).all()
    assert (pairs[..., 0] == probs.max(-1)).all()


def test_gemm_tiles_match_scalar_form(oracle):
    """The oracle's AVX2 6 x 16 GEMM tiles against its scalar form, bit for
    bit (the reference's own AVX2-vs-scalar discipline, bitexact.rs):
    sgemm on both bias paths with ragged edges, matmul, and convs on the
    implicit-GEMM and im2col branches."""
    rng = np.random.default_rng(31)

    def both(fn):
        oracle.set_scalar(False)
        a = fn()
        oracle.set_scalar(True)
        try:
            b = fn()
        finally:
            oracle.set_scalar(False)
        return a, b

    for m, n, k, serial in [(37, 150, 70, False), (64, 16, 4000, False), (13, 333, 9, True),
                            (6, 16, 5, False), (100, 40, 256, True)]:
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal((k, n)).astype(np.float32)
        bias = rng.standard_normal(m).astype(np.float32)
        x, y = both(lambda: oracle.sgemm(a, b, m, n, k, bias, act=oracle.ACT_RELU, serial=serial))
        assert (x == y).all(), (m, n, k)
    a = rng.standard_normal((3, 50, 70)).astype(np.float32)
    b = rng.standard_normal((70, 130)).astype(np.float32)
    x, y = both(lambda: oracle.matmul(a, b))
    assert (x == y).all()
    b3 = rng.standard_normal((3, 70, 45)).astype(np.float32)
    x, y = both(lambda: oracle.matmul(a, b3))
    assert (x == y).all()
    t = (rng.standard_normal((9, 1003)) * 30).astype(np.float32)
    x, y = both(lambda: oracle.softmax_last_dim(t.copy(), 1003))
    assert (x == y).all()
    v = np.concatenate([(rng.standard_normal(8 * 4096) * 40).astype(np.float32),
                        np.array([88.5, -88.5, 100, -100, 0, -0.0, 1e-30, 87.9], np.float32)])
    got = np.concatenate([oracle.exp1x8(v[i:i + 8]) for i in range(0, v.size, 8)])
    want = np.array([oracle.exp1(float(e)) for e in v], np.float32)
    assert (got == want).all()
    for (c, m, k, s, g) in [(16, 22, 3, 1, 1), (12, 18, 5, 2, 3), (8, 13, 3, 3, 1)]:
        xin = rng.standard_normal((2, c, 29, 37)).astype(np.float32)
        w = rng.standard_normal((m, c // g, k, k)).astype(np.float32)
        bias = rng.standard_normal(m).astype(np.float32)
        p = oracle.conv_params(s, s, k // 2, k // 2, group=g)
        x, y = both(lambda: oracle.conv2d(xin, w, bias, p, oracle.ACT_RELU))
        assert (x == y).all(), (c, m, k, s, g)


# ---------------------------------------- pooling / SE / resize / pre-post

def test_pool_and_resize_reference_cases(oracle):
    """The reference's pool_and_resize_tests (kernels.rs:1143-1258) on its
    own xorshift data: 2x2 s1 SAME_UPPER max pool against the clamped
    brute force (exact), 3x3 s2 p1 avg pool against f64 / 9 (1e-5), global
    average pool against the f64 sum in order (exact), bilinear 33 x 47 in
    both coordinate modes against f64 (1e-4)."""
    rng = XorShift(int(GOLD["rng"]["kernels_seed"], 16))
    n, c, h, w = 2, 3, 20, 30
    x = rng.fill((n, c, h, w))
    y = oracle.pool2d(x, 2, 2, 1, 1, 0, 0, 1, 1, True)
    assert y.shape == (n, c, h, w)
    iy = np.minimum(np.arange(h)[:, None] + np.array([0, 1])[None], h - 1)
    ix = np.minimum(np.arange(w)[:, None] + np.array([0, 1])[None], w - 1)
    want = np.maximum.reduce([x[:, :, iy[:, a]][:, :, :, ix[:, b]] for a in (0, 1)
                              for b in (0, 1)])
    assert (y == want).all()
    y = oracle.pool2d(x, 3, 3, 2, 2, 1, 1, 1, 1, False)
    oh, ow = (20 + 2 - 3) // 2 + 1, (30 + 2 - 3) // 2 + 1
    assert y.shape == (n, c, oh, ow)
    xp = np.zeros((n, c, h + 2, w + 2))
    xp[:, :, 1:1 + h, 1:1 + w] = x
    s = sum(xp[:, :, ky:ky + 2 * oh:2, kx:kx + 2 * ow:2] for ky in range(3) for kx in range(3))
    assert np.abs(y - (s / 9.0)).max() < 1e-5
    g = oracle.global_avg_pool(x)
    for i in range(n * c):
        acc = 0.0
        for v in x.reshape(n * c, -1)[i]:
            acc += float(v)
        assert g.ravel()[i] == np.float32(acc / (h * w))
    for align in (False, True):
        y = oracle.resize_bilinear(x, 33, 47, align)

        def coords(no, ni):
            i = np.arange(no, dtype=np.float64)
            v = i * (ni - 1) / (no - 1) if align else np.maximum((i + 0.5) * ni / no - 0.5, 0)
            i0 = np.clip(np.floor(v), 0, ni - 1).astype(int)
            return i0, np.minimum(i0 + 1, ni - 1), v - i0
        y0, y1, fy = coords(33, h)
        x0, x1, fx = coords(47, w)
        xd = x.astype(np.float64)
        fy, fx = fy[:, None], fx[None, :]
        want = (xd[:, :, y0][:, :, :, x0] * (1 - fx) * (1 - fy) +
                xd[:, :, y0][:, :, :, x1] * fx * (1 - fy) +
                xd[:, :, y1][:, :, :, x0] * (1 - fx) * fy + xd[:, :, y1][:, :, :, x1] * fx * fy)
        assert np.abs(y - want).max() < 1e-4


def test_pool_and_bilinear_vs_torch(oracle):
    """Independent library cross-check: torch's max / avg pooling (padding
    counted in the average's divisor) and half-pixel bilinear interpolation."""
    torch = pytest.importorskip("torch")
    F = torch.nn.functional
    rng = np.random.default_rng(41)
    x = rng.standard_normal((2, 5, 23, 31)).astype(np.float32)
    t = torch.from_numpy(x).double()
    y = oracle.pool2d(x, 3, 3, 2, 2, 1, 1, 1, 1, True)
    assert (y == F.max_pool2d(t, 3, 2, 1).float().numpy()).all()
    y = oracle.pool2d(x, 2, 2, 2, 2, 0, 0, 0, 0, False)
    rel_check(y, F.avg_pool2d(t, 2, 2).numpy(), tol=1e-6)
    y = oracle.pool2d(x, 3, 3, 1, 1, 1, 1, 1, 1, False)
    rel_check(y, F.avg_pool2d(t, 3, 1, 1, count_include_pad=True).numpy(), tol=1e-6)
    for oh, ow in [(46, 62), (11, 17), (23, 31)]:
        y = oracle.resize_bilinear(x, oh, ow)
        rel_check(y, F.interpolate(t, (oh, ow), mode="bilinear", align_corners=False).numpy(),
                  tol=1e-5)
    y = oracle.resize_bilinear(x, 40, 50, True)
    rel_check(y, F.interpolate(t, (40, 50), mode="bilinear", align_corners=True).numpy(), tol=1e-5)


def test_mul_add_scale_and_transpose(oracle):
    """f * gate + r with the Mul and Add each rounded (elementwise.rs:134-179):
    numpy float32 does exactly that; a fused multiply-add differs on this data."""
    rng = np.random.default_rng(42)
    f = rng.standard_normal((2, 6, 7, 9)).astype(np.float32)
    gate = rng.random(6).astype(np.float32)
    r = rng.standard_normal(f.shape).astype(np.float32)
    out = oracle.mul_add_scale(f, gate, r)
    want = f * gate[None, :, None, None] + r
    assert (out == want).all()
    fused = (f.astype(np.float64) * gate[None, :, None, None] + r).astype(np.float32)
    assert (fused != want).any()
    x = rng.standard_normal((2, 3, 4, 5)).astype(np.float32)
    for perm in [(0, 2, 3, 1), (0, 3, 1, 2), (3, 2, 1, 0), (0, 1, 2, 3)]:
        assert (oracle.transpose4(x, perm) == x.transpose(perm)).all()


def _fma_f32(a, b, c):
    """fma on float32 inputs via float64: exact here (u8 x weight products
    and their sums fit 53 bits), then one rounding to float32."""
    return (a.astype(np.float64) * b + c).astype(np.float32)


def _resize_u8_restated(src, dw, dh):
    """The scalar formula of the reference's resize test (rsz_par.rs:6-41)."""
    sh, sw = src.shape[:2]
    sx, sy = np.float32(sw) / np.float32(dw), np.float32(sh) / np.float32(dh)

    def axis(n_out, n_in, s):
        v = np.maximum((np.arange(n_out, dtype=np.float32) + np.float32(0.5)) * s - np.float32(0.5),
                       np.float32(0))
        i0 = np.minimum(v.astype(np.int64), n_in - 1)
        return i0, np.minimum(i0 + 1, n_in - 1), (v - i0.astype(np.float32)).astype(np.float32)
    x0, x1, fx = axis(dw, sw, sx)
    y0, y1, fy = axis(dh, sh, sy)
    s = src.astype(np.float32)
    lx, ly = fx[None, :, None], fy[:, None, None]
    one = np.float32(1)
    p00, p01 = s[y0][:, x0], s[y0][:, x1]
    p10, p11 = s[y1][:, x0], s[y1][:, x1]
    t = (p00 * (one - lx)) * (one - ly)
    t = _fma_f32(p01 * lx, one - ly, t)
    t = _fma_f32(p10 * (one - lx), ly, t)
    v = _fma_f32(p11 * lx, ly, t) + np.float32(0.5)
    return np.clip(v, 0, 255).astype(np.uint8)


def test_resize_rgb_u8_and_pack_crop(oracle):
    """u8 bilinear resize against the reference test's scalar formula on its
    source pattern (rsz_par.rs:42-52), then pack_crop (crop.rs:153-190):
    width ceil(img_h * w / h) clamped to img_w, (u8 / 255 - 0.5) / 0.5 by
    true divisions, zeros past the resized width; and the pad_only branch."""
    sw, sh = 848, 816
    src = (np.arange(sw * sh * 3, dtype=np.int64) * 7919 % 256).astype(np.uint8).reshape(sh, sw, 3)
    for dw, dh in [(400, 48), (17, 33), (832, 832)]:
        assert (oracle.resize_bilinear_rgb_u8(src, dw, dh) == _resize_u8_restated(src, dw, dh)).all()
    crop = src[100:154, 20:330]                     # 54 x 310
    dst = oracle.pack_crop(crop, 48, 320)
    rw = min(int(np.ceil(np.float32(48) * (np.float32(310) / np.float32(54)))), 320)
    assert rw == 276
    r = _resize_u8_restated(crop, rw, 48).astype(np.float32)
    want = (r / np.float32(255) - np.float32(0.5)) / np.float32(0.5)
    assert (dst[:, :, :rw] == want.transpose(2, 0, 1)).all()
    assert (dst[:, :, rw:] == 0).all()
    crop = src[:40, :500]
    dst = oracle.pack_crop(crop, 48, 320, pad_only=True)
    v = (crop[:, :320].astype(np.float32) / np.float32(255) - np.float32(0.5)) / np.float32(0.5)
    assert (dst[:, 4:44, :] == v.transpose(2, 0, 1)).all()
    assert (dst[:, :4] == 0).all() and (dst[:, 44:] == 0).all()


def test_det_normalize_and_db_mask(oracle):
    """det input normalisation (engine.rs:959-982) in float32 steps; DB
    threshold + 2x2 dilation against the reference test's brute force
    (rsz_par.rs:55-84) on its mask pattern, thresholded at 0.5."""
    rng = np.random.default_rng(43)
    rgb = rng.integers(0, 256, (37, 53, 3)).astype(np.uint8)
    got = oracle.det_normalize(rgb)
    v = rgb.astype(np.float32) * (np.float32(1) / np.float32(255))
    want = ((v - np.float32(0.5)) * (np.float32(1) / np.float32(0.5))).transpose(2, 0, 1)[None]
    assert (got == want).all()
    for h, w in [(37, 129), (1, 1), (5, 300), (300, 5), (832, 832)]:
        i = np.arange(h * w, dtype=np.uint64)
        mask = (((i * np.uint64(2654435761)) >> np.uint64(24)) % np.uint64(256)).astype(np.uint8) % 3
        pred = mask.reshape(h, w).astype(np.float32)
        binm = (pred > 0.5).astype(np.uint8)
        want = binm.copy()
        want[1:] = np.maximum(want[1:], binm[:-1])
        want2 = want.copy()
        want2[:, 1:] = np.maximum(want[:, 1:], want[:, :-1])
        assert (oracle.db_mask(pred, 0.5) == want2).all(), (h, w)
        assert (oracle.db_mask(pred, 0.5, dilate=False) == binm).all()
