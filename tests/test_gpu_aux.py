"""Parity of the operators around the hot path (pooling, the SE gate's
MulAddScale, bilinear resize, transpose, Concat slots) and of the steps
either side of the networks (det input normalisation, rec pack_crop, the DB
threshold + dilation) with the CPU oracle, bit for bit, through the C ABI.
Shapes follow the reference's own tests (qppocr-kernels/tests/kernels.rs:
1143-1258, tests/rsz_par.rs)."""
import numpy as np
import pytest

from conftest import XorShift, assert_bitexact

pytestmark = pytest.mark.gpu


def _t(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _n(t):
    return t.detach().cpu().numpy()


POOL_CASES = [  # (k, stride, pad (ph, pw, peh, pew), max)
    ((2, 2), (1, 1), (0, 0, 1, 1), True),      # 2x2 s1 SAME_UPPER (the v6 det MaxPool)
    ((3, 3), (2, 2), (1, 1, 1, 1), False),     # kernels.rs:1169
    ((3, 3), (2, 2), (1, 1, 1, 1), True),
    ((2, 2), (2, 2), (0, 0, 0, 0), False),
    ((3, 2), (1, 2), (1, 0, 2, 1), True),
    ((2, 2), (2, 2), (0, 0, 0, 0), True),      # 2x2 s2: paired column loads on even widths
    ((2, 2), (2, 2), (1, 0, 1, 0), True),      # ... with padded rows
    ((2, 2), (2, 2), (1, 0, 0, 0), False),
]


@pytest.mark.parametrize("case", POOL_CASES, ids=[str(c) for c in POOL_CASES])
def test_pool2d(gpu, oracle, case):
    torch = gpu
    from qppocr_amd import ops
    k, s, pad, mx = case
    rng = XorShift(0x243F6A8885A308D3)
    for shape in [(2, 3, 20, 30), (1, 2, 9, 31)]:   # even and odd widths
        x = rng.fill(shape)
        want = oracle.pool2d(x, k[0], k[1], s[0], s[1], *pad, mx)
        assert_bitexact(_n(ops.pool2d(_t(torch, x), k, s, pad, mx)), want, f"pool {case} {shape}")


def test_global_avg_pool_and_mul_add_scale(gpu, oracle):
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(51)
    x = rng.standard_normal((2, 40, 23, 37)).astype(np.float32)
    x[0, 3, 0, 0] = 2.0 ** 40                 # a plane whose f64 sum order matters
    x[0, 3, 0, 1] = -(2.0 ** 40)
    assert_bitexact(_n(ops.global_avg_pool(_t(torch, x))), oracle.global_avg_pool(x), "GAP")
    gate = rng.random(40).astype(np.float32)
    r = rng.standard_normal(x.shape).astype(np.float32)
    assert_bitexact(_n(ops.mul_add_scale(_t(torch, x), _t(torch, gate), _t(torch, r))),
                    oracle.mul_add_scale(x, gate, r), "mul_add_scale")


@pytest.mark.parametrize("align", [False, True])
def test_resize_bilinear_and_transpose(gpu, oracle, align):
    torch = gpu
    from qppocr_amd import ops
    rng = XorShift(0x243F6A8885A308D3)
    x = rng.fill((2, 3, 20, 30))
    for oh, ow in [(33, 47), (10, 15), (40, 60), (1, 1)]:
        assert_bitexact(_n(ops.resize_bilinear(_t(torch, x), oh, ow, align)),
                        oracle.resize_bilinear(x, oh, ow, align), f"bilinear {oh}x{ow}")
    for perm in [(0, 2, 3, 1), (0, 3, 1, 2), (3, 2, 1, 0)]:
        assert_bitexact(_n(ops.transpose(_t(torch, x), perm)), oracle.transpose4(x, perm),
                        f"transpose {perm}")


def test_transpose_every_permutation(gpu):
    """All 24 rank-4 permutations on shapes with ragged 64-tiles: the tiled
    path (input axis 3 moved) and the element path, against numpy's
    transpose (a copy, so equality is exact)."""
    import itertools
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(53)
    for shape in [(3, 70, 5, 130), (1, 96, 40, 72), (2, 1, 65, 1)]:
        x = rng.standard_normal(shape).astype(np.float32)
        gx = _t(torch, x)
        for perm in itertools.permutations(range(4)):
            got = _n(ops.transpose(gx, perm))
            assert np.array_equal(got, np.transpose(x, perm)), (shape, perm)


def test_det_normalize_resize_u8_pack_crop(gpu, oracle):
    torch = gpu
    from qppocr_amd import ops
    sw, sh = 848, 816                              # the reference test's source (rsz_par.rs:42)
    src = (np.arange(sw * sh * 3, dtype=np.int64) * 7919 % 256).astype(np.uint8).reshape(sh, sw, 3)
    gsrc = _t(torch, src)
    for dw, dh in [(832, 832), (400, 48), (960, 1216), (17, 33)]:
        got = _n(ops.resize_bilinear_rgb_u8(gsrc, dw, dh))
        assert (got == oracle.resize_bilinear_rgb_u8(src, dw, dh)).all(), (dw, dh)
    rgb = src[:301, :417]
    assert_bitexact(_n(ops.det_normalize_u8(_t(torch, rgb))), oracle.det_normalize(rgb), "det norm")
    assert_bitexact(_n(ops.det_normalize_u8(_t(torch, src[:64, :128]))),
                    oracle.det_normalize(src[:64, :128]), "det norm (vector stores)")
    for (y0, y1, x0, x1, pad_only) in [(100, 154, 20, 330, False), (0, 40, 0, 500, True),
                                        (10, 58, 5, 1900 // 4, False), (7, 20, 3, 900, False),
                                        (0, 48, 0, 200, True)]:
        crop = np.ascontiguousarray(src[y0:y1, x0:x1])
        got = _n(ops.pack_crop(_t(torch, crop), 48, 320, pad_only))
        assert_bitexact(got, oracle.pack_crop(crop, 48, 320, pad_only), f"pack_crop {y0, x1}")


def test_pack_crops_batch(gpu, oracle):
    """A 70-line rec batch (two launches: 64 + 6 lines) of crops that are
    resized (tall, wide and clamped at img_w, 1x1) or centred (pad_only),
    bit-exact per line against the oracle's pack_crop and against the
    one-line entry point; a pad_only crop taller than img_h is refused."""
    torch = gpu
    from qppocr_amd import _lib, ops
    rng = np.random.default_rng(54)
    shapes = [(54, 310), (40, 500), (1, 1), (48, 200), (30, 40), (7, 900), (20, 64)]
    crops, pads = [], []
    for i in range(70):
        ch, cw = shapes[i % len(shapes)]
        pad = ch <= 48 and i % 3 == 0
        crops.append(rng.integers(0, 256, (ch, cw, 3), dtype=np.uint8))
        pads.append(pad)
    gcrops = [_t(torch, c) for c in crops]
    got = _n(ops.pack_crops(gcrops, 48, 320, pads))
    assert got.shape == (70, 3, 48, 320)
    for i, (c, pad) in enumerate(zip(crops, pads)):
        assert_bitexact(got[i], oracle.pack_crop(c, 48, 320, pad), f"line {i} pad {pad}")
        assert np.array_equal(got[i], _n(ops.pack_crop(gcrops[i], 48, 320, pad)))
    with pytest.raises(_lib.QphError, match="taller"):
        ops.pack_crops([gcrops[0]], 48, 320, [True])


def test_db_mask(gpu, oracle):
    torch = gpu
    from qppocr_amd import ops
    for h, w in [(832, 832), (37, 129), (1, 1), (5, 300), (300, 5)]:
        i = np.arange(h * w, dtype=np.uint64)
        m = (((i * np.uint64(2654435761)) >> np.uint64(24)) % np.uint64(256)).astype(np.uint8) % 3
        pred = (m.reshape(h, w).astype(np.float32) * 0.4).astype(np.float32)   # 0, 0.4, 0.8
        for dil in (True, False):
            got = _n(ops.db_mask(_t(torch, pred), 0.3, dil))
            assert (got == oracle.db_mask(pred, 0.3, dil)).all(), (h, w, dil)


def test_session_se_block_concat_slots(gpu, oracle):
    """A PP-OCRv6-style gated block through the session against the oracle's
    node-by-node run: conv, depthwise, the SE path (GlobalAveragePool, 1x1 +
    ReLU, 1x1 + HardSigmoid) into MulAddScale with a residual, written into a
    Concat slot; a 2x2 s1 SAME_UPPER MaxPool and a bilinear Resize into the
    other slots; the graph input copied into the last; then a Transpose."""
    from qppocr_amd import nets
    from qppocr_amd._lib import ACT_HARDSIGMOID, ACT_RELU, ACT_HARDSWISH
    from oracle import nets as onets
    r = nets.WeightRng(52)
    g = nets.Graph((2, 16, 24, 28))
    x = r.uniform((2, 16, 24, 28), -1, 1)
    w1 = g.weight(r.kaiming((32, 16, 3, 3), 144))
    b1 = g.weight(r.normal((32,), 0.1))
    a = g.conv(0, w1, b1, pad=(1, 1, 1, 1), act=ACT_HARDSWISH)
    wd = g.weight(r.kaiming((32, 1, 5, 5), 25))
    bd = g.weight(r.normal((32,), 0.1))
    d = g.conv(a, wd, bd, pad=(2, 2, 2, 2), group=32, act=ACT_HARDSWISH)
    gp = g.global_avg_pool(d)
    ws1 = g.weight(r.kaiming((8, 32, 1, 1), 32))
    bs1 = g.weight(r.normal((8,), 0.1))
    s1 = g.conv(gp, ws1, bs1, act=ACT_RELU)
    ws2 = g.weight(r.kaiming((32, 8, 1, 1), 8))
    bs2 = g.weight(r.normal((32,), 0.1))
    gate = g.conv(s1, ws2, bs2, act=ACT_HARDSIGMOID)
    cat = g.tensor((2, 32 + 32 + 32 + 16, 24, 28))
    g.mul_add_scale(d, gate, a, out=cat, y_ctotal=112, y_coff=0)
    g.pool(a, (2, 2), (1, 1), (0, 0, 1, 1), True, out=cat, y_ctotal=112, y_coff=32)
    small = g.pool(a, (2, 2), (2, 2), (0, 0, 0, 0), False)
    g.resize(small, 24, 28, bilinear=True, out=cat, y_ctotal=112, y_coff=64)
    g.copy_slot(0, cat, 112, 96)
    t = g.transpose(cat, (0, 2, 3, 1))
    g.outputs = [cat, t]
    sess = nets.HipSession(g)
    outs = sess.run(x)
    refs = onets.run_graph(g, x)
    assert_bitexact(outs[0], refs[0], "concat tensor")
    assert_bitexact(outs[1], refs[1], "transposed")
    sess.close()


def test_mean_of_long_rows(gpu, oracle):
    """Rows of 1024 terms and more take one workgroup per row: 16-byte loads
    (GAP planes of 96x96, rows of 4096) or scalar ones (rows of 1027, not
    16-byte aligned), with rows whose tree sum could round differently
    (2^60 cancellations, a 2^30 magnitude span, a 3e38 term, denormals) and
    so take the sequential sum."""
    torch = gpu
    from qppocr_amd import ops
    rng = np.random.default_rng(52)
    x = rng.standard_normal((2, 6, 96, 96)).astype(np.float32)
    x[0, 1, 0, :2] = 2.0 ** 60, -(2.0 ** 60)
    x[0, 2] *= np.exp2(rng.integers(-15, 15, (96, 96))).astype(np.float32)
    x[1, 3, 5, 7] = 3.0e38
    x[1, 4, :3, :5] = np.float32(1e-40)
    assert_bitexact(_n(ops.global_avg_pool(_t(torch, x))), oracle.global_avg_pool(x), "GAP 96^2")
    for rows, cols in [(5, 1027), (3, 4096), (2, 1024)]:
        y = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
        y[0, 0], y[0, 1] = 2.0 ** 60, -(2.0 ** 60)    # sequential: cancel, the rest survive
        got = _n(ops.reduce_mean_last(_t(torch, y)))
        assert_bitexact(got, oracle.reduce_mean_last(y), f"mean {rows}x{cols}")
        assert got[0] != 0.0


def test_aux_ops_graph_replays_match_eager(gpu):
    """The benchmark's aux leg (bench.aux_specs) captures these C-ABI calls
    into a graph on a caller's stream: each replay, with eager work and a
    synchronisation between replays, reproduces the eager output exactly."""
    torch = gpu
    import ctypes

    import bench
    from qppocr_amd import ops
    lib = ops._lib.load()
    ctx = ops.new_context(0)
    st = torch.cuda.Stream()
    ops.check(lib.qph_ctx_set_stream(ctx, ctypes.c_void_p(st.cuda_stream)))
    try:
        torch.manual_seed(7)
        for name, _, _, make, call, _, _, _ in bench.aux_specs(torch, lib, ctx):
            print("aux graph case", name, flush=True)
            s = make()                       # the last tensor of a set is the output
            torch.cuda.synchronize()
            with torch.cuda.stream(st):
                ops.check(call(s))
            st.synchronize()
            want = s[-1].clone()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=st):
                ops.check(call(s))
            for rep in range(3):
                s[-1].fill_(77 if s[-1].dtype == torch.uint8 else float("nan"))
                torch.cuda.synchronize()
                with torch.cuda.stream(st):
                    g.replay()
                st.synchronize()
                assert torch.equal(s[-1], want), (name, rep)
            del g, s, want
    finally:
        ops.check(lib.qph_ctx_set_stream(ctx, None))
        ops.close_context(ctx)


def test_memset_fill_kernel_eager_and_captured(gpu):
    """qph_memset fills exactly the bytes asked for (unaligned start and
    length, the 16-byte body and both ends) with value & 0xff, eagerly and
    when recorded into a captured graph (replayed three times with eager
    work in between)."""
    torch = gpu
    import ctypes

    from qppocr_amd import ops
    lib = ops._lib.load()
    ctx = ops.new_context(0)
    st = torch.cuda.Stream()
    ops.check(lib.qph_ctx_set_stream(ctx, ctypes.c_void_p(st.cuda_stream)))
    try:
        buf = torch.zeros(70000, dtype=torch.uint8, device="cuda")
        base = buf.data_ptr()
        for off, n, v in [(3, 1000, 0x1A5), (0, 64, 7), (5, 9, 255), (16, 65536, 0), (1, 1, 3)]:
            print(f"memset off {off} bytes {n} value {v}", flush=True)
            buf.fill_(0xEE)
            torch.cuda.synchronize()
            ops.check(lib.qph_memset(ctx, ctypes.c_void_p(base + off), v, n))
            st.synchronize()
            h = buf.cpu().numpy()
            assert (h[off:off + n] == (v & 0xff)).all()
            assert (h[:off] == 0xEE).all() and (h[off + n:] == 0xEE).all()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=st):
            ops.check(lib.qph_memset(ctx, ctypes.c_void_p(base + 7), 0x42, 33333))
        for rep in range(3):
            buf.fill_(0x11)
            torch.cuda.synchronize()
            with torch.cuda.stream(st):
                g.replay()
            st.synchronize()
            h = buf.cpu().numpy()
            assert (h[7:7 + 33333] == 0x42).all() and (h[:7] == 0x11).all(), rep
            assert (h[7 + 33333:] == 0x11).all(), rep
        del g
    finally:
        ops.check(lib.qph_ctx_set_stream(ctx, None))
        ops.close_context(ctx)
