"""Parity of every HIP operator with the CPU oracle (bit-exact), through the C ABI.

The oracle restates the qppocr-kernels CPU arithmetic; the HIP kernels keep
each element's operation sequence, so outputs must be identical element for
element.  Shapes follow the reference's own kernel test cases
(qppocr-kernels/tests/kernels.rs:162-590, 638-683, 1038-1141, 1143-1260,
1422-1467).
"""
import json
import math
import os
import zlib

import numpy as np
import pytest

from conftest import assert_bitexact, baseline_tol_check

pytestmark = pytest.mark.gpu

# The reference's own conv cases (qppocr-kernels/tests/kernels.rs:162-590:
# name, n, c, m, h, w, kh, kw, sh, sw, ph, pw, group, bias), grouped ones
# included, then forms outside that list the dispatcher must still run as
# convolutions: x-stride 3 (the im2col branch), a padded 1x1 conv, a
# depthwise conv with channel multiplier 2, 7x7 and 2x3 dense kernels, a
# 96 -> 24 neck conv, M % 4 tails and batches.
GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden",
                                   "reference_known_answers.json")))
CONV_CASES = [tuple(c) for c in GOLD["conv_cases"]["cases"]] + [
    ("3x3 s3 p1 (im2col)", 1, 8, 12, 31, 29, 3, 3, 3, 3, 1, 1, 1, True),
    ("grouped g=2 5x5 s[1,3]", 2, 6, 10, 20, 22, 5, 5, 1, 3, 2, 2, 2, True),
    ("1x1 padded", 1, 8, 13, 12, 14, 1, 1, 1, 1, 1, 2, 1, True),
    ("depthwise multiplier 2", 1, 8, 16, 17, 19, 3, 3, 1, 1, 1, 1, 8, True),
    ("7x7 s2 p3", 1, 5, 7, 23, 21, 7, 7, 2, 2, 3, 3, 1, True),
    ("2x3 s[1,2] g=3", 1, 6, 9, 15, 18, 2, 3, 1, 2, 0, 1, 3, True),
    ("grouped g=4 s3", 1, 16, 24, 32, 32, 3, 3, 3, 3, 1, 1, 4, True),
    ("3x3 s1 p1", 1, 3, 16, 64, 64, 3, 3, 1, 1, 1, 1, 1, True),
    ("depthwise 3x3 s1 p1 on 1x1", 1, 4, 4, 1, 1, 3, 3, 1, 1, 1, 1, 4, False),
    ("dense 96->24 3x3 (neck)", 1, 96, 24, 20, 20, 3, 3, 1, 1, 1, 1, 1, True),
    ("dense 32->40 3x3 wide M", 2, 32, 40, 19, 37, 3, 3, 1, 1, 1, 1, 1, True),
    ("M=3 3x3 (all tail)", 1, 4, 3, 16, 16, 3, 3, 1, 1, 1, 1, 1, True),
    ("1x1 batch=3 M%4", 3, 20, 13, 7, 9, 1, 1, 1, 1, 0, 0, 1, True),
    # the LDS-staged 3x3 kernels: one-shot 32 channels with seeded tail rows
    # in a partial panel, a ring of 5 chunks, and a width that is not a
    # multiple of 4 (direct kernel)
    ("lds 32->30 3x3 tail panel", 2, 32, 30, 20, 36, 3, 3, 1, 1, 1, 1, 1, True),
    ("lds ring 40->20 3x3", 1, 40, 20, 12, 44, 3, 3, 1, 1, 1, 1, 1, True),
    ("3x3 32->32 w%4 != 0", 1, 32, 32, 10, 30, 3, 3, 1, 1, 1, 1, 1, True),
]


def _seed(name):
    """Stable per-case seed (str hashes change with PYTHONHASHSEED)."""
    return zlib.crc32(name.encode())


def _t(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def _n(t):
    return t.detach().cpu().numpy()


@pytest.mark.parametrize("case", CONV_CASES, ids=[c[0] for c in CONV_CASES])
@pytest.mark.parametrize("act", [0, 2, 3])
def test_conv2d(gpu, oracle, case, act):
    torch = gpu
    from qppocr_amd import ops
    name, n, c, m, h, w, kh, kw, sh, sw, ph, pw, g, has_b = case
    rng = np.random.default_rng(_seed(name))
    x = rng.uniform(-1, 1, (n, c, h, w)).astype(np.float32)
    wt = rng.uniform(-1, 1, (m, c // g, kh, kw)).astype(np.float32)
    b = rng.uniform(-1, 1, (m,)).astype(np.float32) if has_b else None
    params = oracle.conv_params(sh, sw, ph, pw, group=g)
    # the reference graph fuses only ReLU into group-1 convs; hardswish is the
    # HardSigmoid + Mul pair applied to the conv output
    y_ref = oracle.conv2d(x, wt, b, params, act if act != 3 else 0)
    if act == 3:
        y_ref = oracle.binary_flat(y_ref, oracle.hardsigmoid(y_ref), 2)
    y = ops.conv2d(_t(torch, x), _t(torch, wt), None if b is None else _t(torch, b),
                   ops.conv_params(sh, sw, ph, pw, group=g), act)
    assert_bitexact(_n(y), y_ref, name)


def test_conv2d_residual(gpu, oracle):
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(5)
    for (c, m, k, s, g) in [(8, 16, 3, 1, 1), (16, 32, 1, 1, 1), (24, 24, 5, 1, 24)]:
        x = rng.standard_normal((2, c, 21, 23)).astype(np.float32)
        wt = rng.standard_normal((m, c // g, k, k)).astype(np.float32)
        b = rng.standard_normal((m,)).astype(np.float32)
        p = oracle.conv_params(s, s, k // 2, k // 2, group=g)
        ys = oracle.conv_out_shape(x.shape, wt.shape, p)
        r = rng.standard_normal(ys).astype(np.float32)
        act = 2 if g == 1 else 0
        y_ref = oracle.conv2d(x, wt, b, p, act, residual=r)
        y = ops.conv2d(_t(torch, x), _t(torch, wt), _t(torch, b),
                       ops.conv_params(s, s, k // 2, k // 2, group=g), act, residual=_t(torch, r))
        assert_bitexact(_n(y), y_ref, f"residual c{c} m{m} k{k} g{g}")


def test_conv1x1_upsample_add_and_transposed_out(gpu, oracle):
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(6)
    x = rng.standard_normal((1, 32, 20, 20)).astype(np.float32)
    wt = rng.standard_normal((96, 32, 1, 1)).astype(np.float32)
    b = rng.standard_normal((96,)).astype(np.float32)
    coarse = rng.standard_normal((1, 96, 10, 10)).astype(np.float32)
    y_ref = oracle.conv2d(x, wt, b)
    y_ref = oracle.binary_flat(y_ref, oracle.resize_nearest(coarse, 20, 20), 0)
    y = ops.conv2d(_t(torch, x), _t(torch, wt), _t(torch, b), residual=_t(torch, coarse), res_up=2)
    assert_bitexact(_n(y), y_ref, "lateral + up2")
    # [B, C, 1, T] -> [B, T, C]
    x = rng.standard_normal((4, 64, 1, 40)).astype(np.float32)
    wt = rng.standard_normal((48, 64, 1, 1)).astype(np.float32)
    y_ref = oracle.conv2d(x, wt, b[:48], act=0)
    y_ref = oracle.binary_flat(y_ref, oracle.hardsigmoid(y_ref), 2)
    y_ref = y_ref.reshape(4, 48, 40).transpose(0, 2, 1)
    y = ops.conv2d(_t(torch, x), _t(torch, wt), _t(torch, b[:48]), act_kind=3, trans_out=True)
    assert_bitexact(_n(y), y_ref, "trans_out")


def test_conv3x3_placed_output(gpu, oracle):
    """Smoothing conv written upsampled into a channel slot of the neck concat."""
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(7)
    out = torch.full((1, 96, 40, 40), float("nan"), device="cuda")
    ref = np.zeros((1, 96, 40, 40), dtype=np.float32)
    for slot, hw in enumerate([5, 10, 20, 40]):
        x = rng.standard_normal((1, 96, hw, hw)).astype(np.float32)
        wt = rng.standard_normal((24, 96, 3, 3)).astype(np.float32)
        b = rng.standard_normal((24,)).astype(np.float32)
        y = oracle.conv2d(x, wt, b, oracle.conv_params(1, 1, 1, 1))
        ref[:, 24 * slot:24 * slot + 24] = oracle.resize_nearest(y, 40, 40)
        ops.conv2d(_t(torch, x), _t(torch, wt), _t(torch, b), ops.conv_params(1, 1, 1, 1),
                   out=out, y_ctotal=96, y_coff=24 * slot, y_up=40 // hw)
    assert_bitexact(_n(out), ref, "concat slots")


# Depthwise convs at the shapes of the depthwise workloads (3x3 / 5x5, stride
# 1 / 2, + hardswish) and two ragged planes large enough for the tiled kernel
# to take four-wave workgroups (partial last tile in both directions).
DW_CASES = [
    ("dw3 s1 C64 160", 64, 160, 160, 3, 1),
    ("dw3 s2 C128 80", 128, 80, 80, 3, 2),
    ("dw5 s1 C256 40", 256, 40, 40, 5, 1),
    ("dw5 s2 C256 40", 256, 40, 40, 5, 2),
    ("dw3 s1 C64 130x150 (4 waves)", 64, 130, 150, 3, 1),
    ("dw5 s2 C256 120 (4 waves)", 256, 120, 120, 5, 2),
    ("dw3 s2 C8 9x300", 8, 9, 300, 3, 2),
]


@pytest.mark.parametrize("case", DW_CASES, ids=[c[0] for c in DW_CASES])
def test_depthwise_shapes(gpu, oracle, case):
    torch = gpu
    from qppocr_amd import ops
    name, c, h, w, k, s = case
    rng = np.random.default_rng(_seed(name))
    x = rng.uniform(-1, 1, (1, c, h, w)).astype(np.float32)
    wt = rng.uniform(-1, 1, (c, 1, k, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (c,)).astype(np.float32)
    y_ref = oracle.conv2d(x, wt, b, oracle.conv_params(s, s, k // 2, k // 2, group=c))
    y_ref = oracle.binary_flat(y_ref, oracle.hardsigmoid(y_ref), 2)
    y = ops.conv2d(_t(torch, x), _t(torch, wt), _t(torch, b),
                   ops.conv_params(s, s, k // 2, k // 2, group=c), 3)
    assert_bitexact(_n(y), y_ref, name)


# 3x3 convs on the direct kernel: each per-wave tile shape (16/32 channels x
# 16/32 pixels), a channel count that ends inside a group of four, M with a
# partial last block and a bias-seeded M%4 tail (partial 32-column panel),
# stride (2, 1) with uneven padding.
DIRECT_CASES = [
    # n, c, m, h, w, sh, sw, ph, pw, peh, pew
    (1, 96, 24, 40, 40, 1, 1, 1, 1, 1, 1),
    (2, 5, 22, 37, 40, 1, 1, 1, 1, 1, 1),
    (2, 32, 32, 128, 128, 1, 1, 1, 1, 1, 1),
    (8, 8, 32, 128, 128, 1, 1, 1, 1, 1, 1),
    (8, 8, 16, 128, 128, 1, 1, 1, 1, 1, 1),
    # LDS-staged kernel (stride 1, pad 1, C % 8 == 0, M <= 32): two chunks with
    # bias-seeded rows (M % 4 tail, partial last 32-column panel) and partial
    # tiles; three chunks, M = 8, odd sizes; five chunks (the ring wraps)
    (1, 16, 22, 19, 45, 1, 1, 1, 1, 1, 1),
    (2, 24, 8, 9, 70, 1, 1, 1, 1, 1, 1),
    (1, 40, 32, 7, 33, 1, 1, 1, 1, 1, 1),
    (8, 3, 16, 128, 128, 2, 2, 1, 1, 1, 1),
    (3, 12, 40, 33, 47, 2, 1, 0, 1, 2, 0),
    # 3 input channels, M % 4 == 0: the VALU kernel (odd sizes, asymmetric pads)
    (3, 3, 32, 47, 81, 2, 2, 1, 1, 1, 1),
    (2, 3, 20, 30, 33, 1, 2, 0, 1, 2, 0),
    (1, 3, 22, 17, 19, 2, 2, 1, 1, 1, 1),   # M % 4 != 0: MFMA path
]


@pytest.mark.parametrize("case", DIRECT_CASES, ids=[str(c) for c in DIRECT_CASES])
def test_conv3x3_direct_tiles(gpu, oracle, case):
    torch = gpu
    from qppocr_amd import ops
    n, c, m, h, w, sh, sw, ph, pw, peh, pew = case
    rng = np.random.default_rng(sum(case))
    x = rng.standard_normal((n, c, h, w)).astype(np.float32)
    wt = rng.standard_normal((m, c, 3, 3)).astype(np.float32)
    b = rng.standard_normal((m,)).astype(np.float32)
    y_ref = oracle.conv2d(x, wt, b, oracle.conv_params(sh, sw, ph, pw, peh, pew), 2)
    y = ops.conv2d(_t(torch, x), _t(torch, wt), _t(torch, b),
                   ops.conv_params(sh, sw, ph, pw, peh, pew), 2)
    assert_bitexact(_n(y), y_ref, f"direct 3x3 {case}")


@pytest.mark.parametrize("shape", [(31, 31, 1, 2), (301, 301, 7, 16)],
                         ids=["one tile", "tiles of 6 rows"])
def test_conv_im2col_bias_placement(gpu, oracle, shape):
    """x-stride 3: the reference's im2col branch seeds the M%4 tail rows by
    the tile's flattened columns (conv.rs:639-661).  Chain 1 then 2^24 with
    bias 1 gives 2^24 + 2 where seeded and 2^24 where added after."""
    torch = gpu
    from qppocr_amd import ops
    h, w, k, cg = shape
    big = np.float32(2.0 ** 24)
    x = np.ones((1, cg, h, w), np.float32)
    x[0, 1] = big
    wt = np.zeros((5, cg, k, k), np.float32)
    wt[:, 0, 0, 0] = 1
    wt[:, 1, 0, 0] = 1
    b = np.ones(5, np.float32)
    y_ref = oracle.conv2d(x, wt, b, oracle.conv_params(3, 3, 0, 0))
    y = _n(ops.conv2d(_t(torch, x), _t(torch, wt), _t(torch, b), ops.conv_params(3, 3, 0, 0)))
    assert_bitexact(y, y_ref, f"im2col seeding {shape}")
    assert (y[0, 4] == big + 2).any() and (y[0, 4] == big).any()


# the last eleven take the pointwise kernel (M <= 128, K % 16 == 0, N % 4 ==
# 0): the det lateral shapes, an M % 4 tail with partial panels, 7 and 8
# row blocks, one block, wide ones where a wave takes 8, 6 or 2 blocks, and
# small grids with every slab in flight (a 16-stage ring wrapping over 32
# slabs; 8 stages for 5 slabs)
SGEMM_SHAPES = [(1, 1, 1), (64, 64, 64), (1, 500, 300), (17, 33, 129), (256, 96, 384),
                (1, 368, 368 * 9), (17, 713, 77), (5, 37, 13),
                (96, 400, 256), (96, 25600, 32), (100, 1600, 128), (128, 6400, 64),
                (13, 100, 48), (7, 36, 16), (128, 32768, 16), (96, 33024, 32), (32, 32768, 48),
                (64, 256, 512), (48, 96, 80)]


@pytest.mark.parametrize("mnk", SGEMM_SHAPES, ids=[f"{m}x{n}x{k}" for m, n, k in SGEMM_SHAPES])
@pytest.mark.parametrize("serial", [False, True])
def test_sgemm(gpu, oracle, mnk, serial):
    torch = gpu
    from qppocr_amd import ops
    m, n, k = mnk
    rng = np.random.default_rng(m * 1000 + n + k)
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    bias = rng.uniform(-1, 1, (m,)).astype(np.float32)
    c_ref = oracle.sgemm(a, b, m, n, k, bias, serial=serial)
    c = ops.sgemm(_t(torch, a), _t(torch, b), m, n, k, _t(torch, bias), serial=serial)
    assert_bitexact(_n(c), c_ref, f"sgemm {mnk}")
    ref64 = a.astype(np.float64) @ b + bias[:, None]
    from conftest import rel_check
    rel_check(_n(c), ref64)


def test_sgemm_bias_placement(gpu, oracle):
    """Bias seeded vs added after the chain: with a = [1, 1], b rows [1], [2^24]
    and bias 1, the after-chain order gives 2^24 and the seeded order 2^24 + 2."""
    torch = gpu
    from qppocr_amd import ops
    for (m, n, k) in [(5, 5, 2), (64, 16, 4000)]:
        a = np.zeros((m, k), np.float32)
        a[:, :2] = 1.0
        b = np.zeros((k, n), np.float32)
        b[0] = 1.0
        b[1] = 2.0 ** 24
        bias = np.ones(m, np.float32)
        c_ref = oracle.sgemm(a, b, m, n, k, bias)
        c = _n(ops.sgemm(_t(torch, a), _t(torch, b), m, n, k, _t(torch, bias)))
        assert_bitexact(c, c_ref, f"bias placement {m}x{n}x{k}")


def test_linear_epilogues(gpu, oracle):
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(11)
    for (rows, k, n, act, res) in [(1280, 256, 768, 0, False), (1280, 256, 1024, 1, False),
                                   (1280, 1024, 256, 0, True), (37, 256, 18709, 0, False),
                                   (100, 77, 130, 2, True)]:
        x = rng.standard_normal((rows, k)).astype(np.float32)
        w = (rng.standard_normal((k, n)) * math.sqrt(2 / k)).astype(np.float32)
        b = (rng.standard_normal((n,)) * 0.1).astype(np.float32)
        r = rng.standard_normal((rows, n)).astype(np.float32) if res else None
        y_ref = oracle.matmul(x, w)
        y_ref = oracle.binary_bcast(y_ref, b, rows, n, 0, 1)
        if act == 1:
            y_ref = oracle.gelu_inplace(y_ref)
        elif act == 2:
            y_ref = oracle.relu_inplace(y_ref)
        if res:
            y_ref = oracle.binary_flat(y_ref, r, 0)
        y = ops.linear(_t(torch, x), _t(torch, w), _t(torch, b), act,
                       None if r is None else _t(torch, r))
        assert_bitexact(_n(y), y_ref, f"linear {rows}x{k}x{n}")


def test_gemm_wide_tiles(gpu, oracle):
    """Shapes with >= 512 128x128 tiles take the persistent wide-tile kernel:
    ragged M / N edges, unpadded odd ldb, both bias-seeding rules (row bias),
    GELU + residual epilogue, batched B, and K not a multiple of 16 (which
    falls back to the 128x128 staged kernel); plain ones (column bias or
    none) take the one-wave kernel, with its row-store epilogue when the
    rows come in whole 64-row blocks and 16-byte aligned, batched too."""
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(21)
    for (m, n, k, serial) in [(1300, 6500, 48, False), (1300, 6500, 48, True),
                              (1290, 6531, 50, False)]:
        a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
        b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
        bias = rng.uniform(-1, 1, (m,)).astype(np.float32)
        c_ref = oracle.sgemm(a, b, m, n, k, bias, serial=serial)
        c = ops.sgemm(_t(torch, a), _t(torch, b), m, n, k, _t(torch, bias), serial=serial)
        assert_bitexact(_n(c), c_ref, f"wide sgemm {m}x{n}x{k} serial={serial}")
    # (1280, 32, 8196): column bias only, whole 64-row blocks, rows 16-byte
    # aligned -- the one-wave kernel with its row-store epilogue
    for (rows, k, n, act, res) in [(1290, 32, 8195, 0, False), (1280, 64, 8200, 1, True),
                                   (1280, 32, 8196, 0, False)]:
        x = rng.standard_normal((rows, k)).astype(np.float32)
        w = (rng.standard_normal((k, n)) * math.sqrt(2 / k)).astype(np.float32)
        b = (rng.standard_normal((n,)) * 0.1).astype(np.float32)
        r = rng.standard_normal((rows, n)).astype(np.float32) if res else None
        y_ref = oracle.binary_bcast(oracle.matmul(x, w), b, rows, n, 0, 1)
        if act == 1:
            y_ref = oracle.gelu_inplace(y_ref)
        if res:
            y_ref = oracle.binary_flat(y_ref, r, 0)
        y = ops.linear(_t(torch, x), _t(torch, w), _t(torch, b), act,
                       None if r is None else _t(torch, r))
        assert_bitexact(_n(y), y_ref, f"wide linear {rows}x{k}x{n} act={act}")
    # both plain, so the one-wave kernel; the second with whole 64-row blocks
    # and 16-byte rows, so its row-store epilogue
    for (bt, m, k, n) in [(6, 300, 32, 4100), (6, 320, 32, 4100)]:
        a = rng.uniform(-1, 1, (bt, m, k)).astype(np.float32)
        b = rng.uniform(-1, 1, (bt, k, n)).astype(np.float32)
        assert_bitexact(_n(ops.matmul(_t(torch, a), _t(torch, b))), oracle.matmul(a, b),
                        f"wide batched matmul {bt}x{m}x{k}x{n}")


def test_matmul_batched(gpu, oracle):
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(12)
    a = rng.uniform(-1, 1, (2, 3, 40, 80)).astype(np.float32)   # kernels.rs shape_op_tests
    b = rng.uniform(-1, 1, (80, 101)).astype(np.float32)
    assert_bitexact(_n(ops.matmul(_t(torch, a), _t(torch, b))), oracle.matmul(a, b), "shared B")
    a = rng.uniform(-1, 1, (16, 40, 32)).astype(np.float32)
    b = rng.uniform(-1, 1, (16, 32, 40)).astype(np.float32)
    assert_bitexact(_n(ops.matmul(_t(torch, a), _t(torch, b))), oracle.matmul(a, b), "batched B")


@pytest.mark.parametrize("inner", [1, 4, 7, 8, 13, 40, 100, 4099, 18709, 19007, 19008, 19009, 20480, 40000])
def test_softmax_last_dim(gpu, oracle, inner):
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(inner)
    rows = 37
    t = (rng.standard_normal((rows, inner)) * 3).astype(np.float32)
    ref = oracle.softmax_last_dim(t.copy(), inner)
    g = _t(torch, t)
    ops.softmax_last_dim(g, inner)
    assert_bitexact(_n(g), ref, f"softmax {inner}")


def test_softmax_argmax_and_ties(gpu, oracle):
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(13)
    logits = (rng.standard_normal((64, 18709)) * 2).astype(np.float32)
    logits[3, 100] = logits[3, 50] = 40.0        # tie: lowest index wins
    logits[5, :] = 0.0                           # all equal: index 0
    logits[7, 18708] = 30.0                      # last column
    probs, pairs = ops.softmax_argmax(_t(torch, logits))
    p_ref = oracle.softmax_last_dim(logits.copy(), 18709)
    pr_ref = oracle.ctc_argmax(p_ref)
    assert_bitexact(_n(probs), p_ref, "probs")
    assert_bitexact(_n(pairs)[:, 0], pr_ref[:, 0], "pair values")
    ids = ops.pairs_ids(pairs).cpu().numpy()
    ids_ref = oracle.pairs_ids(pr_ref)
    assert (ids == ids_ref).all()
    assert ids[3] == 50 and ids[5] == 0 and ids[7] == 18708


@pytest.mark.parametrize("shape", [(1280, 256, 18709), (100, 256, 18709), (37, 64, 1001),
                                   (130, 32, 70)], ids=lambda s: "x".join(map(str, s)))
def test_linear_softmax_argmax_fused(gpu, oracle, shape):
    """The fused head (GEMM + softmax + argmax, logits never stored) against
    the oracle's MatMul, Add, Softmax, argmax under the pairs tolerance rule:
    values within 1e-4, ids equal except at top-2 logit gaps below 1e-4.
    Planted exact ties and a maximum in the last, partial column block."""
    torch = gpu
    from conftest import pairs_tolerance_check
    from qppocr_amd import ops
    rows, k, n = shape
    rng = np.random.default_rng(rows + n)
    x = rng.standard_normal((rows, k)).astype(np.float32)
    w = (rng.standard_normal((k, n)) * math.sqrt(2 / k)).astype(np.float32)
    b = (rng.standard_normal(n) * 0.1).astype(np.float32)
    x[2] = 0.0                   # row 2: every logit is its bias, and
    w[:, 3] = w[:, n // 2] = 0.0
    b[3] = b[n // 2] = 60.0      # ... two equal maxima: the first wins
    x[1] = 0.0                   # row 1: the max in the last, partial column block
    x[1, 0] = 1.0
    w[0, n - 1] = 100.0
    logits = oracle.binary_bcast(oracle.matmul(x, w), b, rows, n, 0, 1)
    ref = oracle.ctc_argmax(oracle.softmax_last_dim(logits.copy(), n))
    pairs = _n(ops.linear_softmax_argmax(_t(torch, x), _t(torch, w), _t(torch, b)))
    nd = pairs_tolerance_check(pairs, ref, logits)
    ids = pairs[:, 1].copy().view(np.uint32)
    assert ids[2] == 3 and ids[1] == n - 1
    assert nd <= max(1, rows // 100)
    rel = np.abs(pairs[:, 0].astype(np.float64) - ref[:, 0]) / np.abs(ref[:, 0])
    assert rel.max() < 1e-5, rel.max()


@pytest.mark.parametrize("cols", [18709, 19500, 40000, 7])
def test_softmax_argmax_pairs_only(gpu, oracle, cols):
    """probs = NULL: pairs only (rec_argmax_pairs, device.rs:160-165), the
    same pairs as the full path, on every row-width kernel."""
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(cols)
    logits = (rng.standard_normal((40, cols)) * 2).astype(np.float32)
    logits[3, 1], logits[3, 5] = 30.0, 30.0
    none, pairs = ops.softmax_argmax(_t(torch, logits), probs=False)
    assert none is None
    ref = oracle.ctc_argmax(oracle.softmax_last_dim(logits.copy(), cols))
    assert_bitexact(_n(pairs)[:, 0], ref[:, 0], "pair values")
    assert (ops.pairs_ids(pairs).cpu().numpy() == oracle.pairs_ids(ref)).all()


def test_ctc_argmax_masked(gpu, oracle):
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(14)
    probs = rng.random((4, 20, 97)).astype(np.float32)
    probs[0, 2, 10] = probs[0, 2, 20] = 2.0
    tv = [20, 10, 0, 5]
    pairs = _n(ops.ctc_argmax(_t(torch, probs), tv))
    ref = oracle.ctc_argmax(probs)
    ids = pairs[..., 1].copy().view(np.uint32)
    ids_ref = ref[..., 1].copy().view(np.uint32)
    for b in range(4):
        assert (ids[b, :tv[b]] == ids_ref[b, :tv[b]]).all()
        assert (ids[b, tv[b]:] == 0).all()
    assert ids[0, 2] == 10


def test_layernorm(gpu, oracle):
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(15)
    for rows, cols in [(1280, 256), (7, 33), (3, 1000)]:
        x = (rng.standard_normal((rows, cols)) * 2 + 0.5).astype(np.float32)
        g = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
        b = (0.1 * rng.standard_normal(cols)).astype(np.float32)
        ref = oracle.layernorm(x, g, b, 1e-6)
        y = ops.layernorm(_t(torch, x), _t(torch, g), _t(torch, b), 1e-6)
        assert_bitexact(_n(y), ref, f"layernorm {rows}x{cols}")


def test_row_sums_wide_span(gpu, oracle):
    """f64 row sums where the order changes the value: the reference's
    ascending sequential sum (shape.rs:551-557) must come out, not a tree
    sum.  Rows [2^60, -2^60, 1, ...] (sequential: the ones survive) next to
    ordinary rows and rows with a 2^30 magnitude span."""
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(22)
    rows, cols = 512, 256
    x = (rng.standard_normal((rows, cols)) * 2).astype(np.float32)
    x[::4, 0], x[::4, 1] = 2.0 ** 60, -(2.0 ** 60)
    x[1::4] *= np.exp2(rng.integers(-15, 15, (rows // 4, cols))).astype(np.float32)
    x[2::4, 5] = 3.0e38
    mean = _n(ops.reduce_mean_last(_t(torch, x)))
    assert_bitexact(mean, oracle.reduce_mean_last(x), "reduce_mean wide span")
    assert mean[0] != 0.0
    g = np.ones(cols, np.float32)
    b = np.zeros(cols, np.float32)
    xs = x.copy()
    xs[2::4, 5] = 1.0       # keep the squares finite
    ref = oracle.layernorm(xs, g, b, 1e-6)
    got = _n(ops.layernorm(_t(torch, xs), _t(torch, g), _t(torch, b), 1e-6))
    assert_bitexact(got, ref, "layernorm wide span")


@pytest.mark.parametrize("t", [40, 20, 5, 13, 64, 160])
def test_attention(gpu, oracle, t):
    torch = gpu
    from qppocr_amd import ops, nets
    from oracle import nets as onets
    rng = np.random.default_rng(t)
    b, heads, dh = 3, 8, 32
    qkv = rng.standard_normal((b, t, 3 * heads * dh)).astype(np.float32)
    g = nets.Graph((b, t, 3 * heads * dh))
    o = g.attention(0, heads, dh, 1.0 / math.sqrt(dh))
    g.outputs = [o]
    ref = onets.run_graph(g, qkv)[0].reshape(b, t, heads * dh)
    y = ops.attention(_t(torch, qkv), heads, dh, 1.0 / math.sqrt(dh))
    assert_bitexact(_n(y), ref, f"attention T={t}")


def test_convtranspose(gpu, oracle):
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(16)
    x = rng.uniform(-1, 1, (2, 24, 17, 19)).astype(np.float32)
    w1 = rng.uniform(-1, 1, (24, 24, 2, 2)).astype(np.float32)
    w2 = rng.uniform(-1, 1, (24, 1, 2, 2)).astype(np.float32)
    y1 = oracle.convtranspose2d(x, w1)
    assert_bitexact(_n(ops.convtranspose2d(_t(torch, x), _t(torch, w1))), y1, "convT")
    ref = oracle.sigmoid_tensor(oracle.convtranspose2d(y1, w2))
    got = _n(ops.convt_pair_sigmoid(_t(torch, x), _t(torch, w1), _t(torch, w2)))
    assert_bitexact(got, ref, "convT pair + sigmoid")
    # generic-size path of the pair kernel
    x = rng.uniform(-1, 1, (1, 5, 6, 7)).astype(np.float32)
    w1 = rng.uniform(-1, 1, (5, 3, 2, 2)).astype(np.float32)
    w2 = rng.uniform(-1, 1, (3, 1, 2, 2)).astype(np.float32)
    ref = oracle.sigmoid_tensor(oracle.convtranspose2d(oracle.convtranspose2d(x, w1), w2))
    got = _n(ops.convt_pair_sigmoid(_t(torch, x), _t(torch, w1), _t(torch, w2)))
    assert_bitexact(got, ref, "convT pair generic")


def test_elementwise_activations(gpu, oracle):
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(17)
    x = rng.uniform(-1, 1, 4096).astype(np.float32)
    special = np.array([0.0, -0.0, 3.0, -3.0, 88.0, -88.0, 100.0, -100.0, 1e-30, -1e-30, 6.0,
                        -6.0, 1e6, -1e6], np.float32)
    x = np.concatenate([x, x * 10, special])
    gx = _t(torch, x)
    assert_bitexact(_n(ops.sigmoid_tensor(gx)), oracle.sigmoid_tensor(x), "sigmoid")
    assert_bitexact(_n(ops.hardsigmoid(gx)), oracle.hardsigmoid(x), "hardsigmoid")
    assert_bitexact(_n(ops.relu_inplace(gx.clone())), oracle.relu_inplace(x.copy()), "relu")
    assert_bitexact(_n(ops.gelu_inplace(gx.clone())), oracle.gelu_inplace(x.copy()), "gelu")
    hs = oracle.binary_flat(x, oracle.hardsigmoid(x), 2)
    assert_bitexact(_n(ops.activation(gx, 3)), hs, "hardswish")
    # erf1 through GELU with c1 = 1, c2 = 0, c3 = 1: y = v * erf1(v), exact
    # for powers of two; the reference's erf table (activation.rs:474-488)
    pts = GOLD["erf_table"]["points"]
    v = np.array([p[0] for p in pts], np.float32)
    y = _n(ops.gelu_inplace(_t(torch, v), 1.0, 0.0, 1.0))
    assert_bitexact(y, oracle.gelu_inplace(v.copy(), 1.0, 0.0, 1.0), "gelu c=(1,0,1)")
    for (xv, ev), yv in zip(pts, y):
        if xv == 0.0:
            assert yv == 0.0
            continue
        erf_gpu = float(yv) / xv
        exact = math.frexp(xv)[0] == 0.5
        tol = GOLD["erf_table"]["tol"] + (0.0 if exact else 2.0 ** -23)
        assert abs(erf_gpu - ev) <= tol, (xv, erf_gpu, ev)


def test_resize_nearest(gpu, oracle):
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(18)
    x = rng.uniform(-1, 1, (2, 3, 20, 30)).astype(np.float32)   # kernels.rs:1203-1219
    for oh, ow in [(33, 47), (40, 60), (10, 15)]:
        assert_bitexact(_n(ops.resize_nearest(_t(torch, x), oh, ow)),
                        oracle.resize_nearest(x, oh, ow), f"resize {oh}x{ow}")


def test_reduce_mean_and_binary(gpu, oracle):
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(19)
    x = rng.standard_normal((100, 256)).astype(np.float32)
    assert_bitexact(_n(ops.reduce_mean_last(_t(torch, x))), oracle.reduce_mean_last(x), "mean")
    b = rng.standard_normal(256).astype(np.float32)
    for op in range(4):
        got = _n(ops.binary_inplace(_t(torch, x), _t(torch, b), op, 1))
        assert_bitexact(got, oracle.binary_bcast(x, b, 100, 256, op, 1), f"binary {op}")

