"""qph_conv2d_noalloc (the allocation-free form of qph_conv2d) against
qph_conv2d itself, through the C ABI: two calls in a row, the second on a
smaller input, bit for bit; and the size limit of its fixed device array."""
import ctypes

import numpy as np
import pytest

from conftest import assert_bitexact

pytestmark = pytest.mark.gpu


def _call(lib, fn, ctx, torch, x, w, b, params, act, res):
    from qppocr_amd import ops
    from qppocr_amd._lib import i64arr
    ys = ops.conv2d_out_shape(tuple(x.shape), tuple(w.shape), params)
    y = torch.full(ys, float("nan"), device="cuda")
    torch.cuda.synchronize()
    rc = getattr(lib, fn)(ctx, ctypes.c_void_p(x.data_ptr()), i64arr(x.shape),
                          ctypes.c_void_p(w.data_ptr()), i64arr(w.shape),
                          None if b is None else ctypes.c_void_p(b.data_ptr()),
                          ctypes.byref(params), ctypes.byref(act),
                          None if res is None else ctypes.c_void_p(res.data_ptr()),
                          ctypes.c_void_p(y.data_ptr()), None)
    if rc == 0:
        rc = lib.qph_sync(ctx)
    return rc, y


def test_conv2d_noalloc_matches_conv2d(gpu):
    torch = gpu
    from qppocr_amd import _lib, ops
    lib = _lib.load()
    ctx = ops.context(0)
    rng = np.random.default_rng(71)
    # (n, c, m, h, w, k, stride, pad, group, residual): a dense 3x3 conv, then
    # a smaller grouped 5x5 one (the array keeps the first call's repack; the
    # second must overwrite what it reads), then 1x1 and depthwise forms
    cases = [(2, 64, 96, 40, 44, 3, 1, 1, 1, True), (1, 12, 18, 21, 17, 5, 2, 2, 3, False),
             (1, 16, 24, 20, 20, 1, 1, 0, 1, False), (1, 32, 32, 30, 30, 3, 1, 1, 32, False)]
    for n, c, m, h, w, k, s, p, g, has_res in cases:
        print(f"noalloc conv n{n} c{c} m{m} {h}x{w} k{k} s{s} g{g}", flush=True)
        x = torch.from_numpy(rng.standard_normal((n, c, h, w)).astype(np.float32)).cuda()
        wt = torch.from_numpy(rng.standard_normal((m, c // g, k, k)).astype(np.float32)).cuda()
        b = torch.from_numpy(rng.standard_normal(m).astype(np.float32)).cuda()
        params = ops.conv_params(s, s, p, p, group=g)
        ys = ops.conv2d_out_shape(tuple(x.shape), tuple(wt.shape), params)
        res = (torch.from_numpy(rng.standard_normal(ys).astype(np.float32)).cuda()
               if has_res else None)
        act = ops.act(2 if g == 1 else 0)
        rc1, y1 = _call(lib, "qph_conv2d", ctx, torch, x, wt, b, params, act, res)
        rc2, y2 = _call(lib, "qph_conv2d_noalloc", ctx, torch, x, wt, b, params, act, res)
        assert rc1 == 0 and rc2 == 0, lib.qph_last_error()
        assert_bitexact(y2.cpu().numpy(), y1.cpu().numpy(), f"noalloc {n, c, m, k, g}")


def test_conv2d_noalloc_refuses_oversize_weights(gpu):
    torch = gpu
    from qppocr_amd import _lib, ops
    lib = _lib.load()
    ctx = ops.context(0)
    # 512 -> 512 3x3: 4608 x 512 floats repacked, past the 2^20 of the array
    x = torch.zeros((1, 512, 8, 8), device="cuda")
    wt = torch.zeros((512, 512, 3, 3), device="cuda")
    rc, _ = _call(lib, "qph_conv2d_noalloc", ctx, torch, x, wt, None, ops.conv_params(1, 1, 1, 1),
                  ops.act(0), None)
    assert rc == -3 and b"fixed device array" in lib.qph_last_error()
    assert 512 * 9 * 512 > _lib.NOALLOC_WK_FLOATS


def test_conv2d_noalloc_allocates_nothing(gpu):
    """On a fresh context, qph_conv2d_noalloc called before any qph_conv2d
    leaves the context's hipMalloc-grown scratch at 0 bytes (so it cannot
    have fallen back to it), and still matches qph_conv2d bit for bit; the
    qph_conv2d call that follows does grow the scratch (the query sees it)."""
    torch = gpu
    from qppocr_amd import _lib, ops
    lib = _lib.load()
    ctx = ops.new_context(0)
    try:
        def scratch():
            v = ctypes.c_size_t()
            assert lib.qph_ctx_scratch_bytes(ctx, ctypes.byref(v)) == 0
            return v.value
        rng = np.random.default_rng(72)
        x = torch.from_numpy(rng.standard_normal((1, 48, 36, 40)).astype(np.float32)).cuda()
        wt = torch.from_numpy(rng.standard_normal((64, 48, 3, 3)).astype(np.float32)).cuda()
        b = torch.from_numpy(rng.standard_normal(64).astype(np.float32)).cuda()
        params = ops.conv_params(1, 1, 1, 1)
        print("noalloc on a fresh context: dense 3x3 48->64 36x40", flush=True)
        assert scratch() == 0
        rc2, y2 = _call(lib, "qph_conv2d_noalloc", ctx, torch, x, wt, b, params, ops.act(2), None)
        assert rc2 == 0, lib.qph_last_error()
        assert scratch() == 0
        rc1, y1 = _call(lib, "qph_conv2d", ctx, torch, x, wt, b, params, ops.act(2), None)
        assert rc1 == 0, lib.qph_last_error()
        assert scratch() > 0
        assert_bitexact(y2.cpu().numpy(), y1.cpu().numpy(), "noalloc on a fresh context")
    finally:
        ops.close_context(ctx)
