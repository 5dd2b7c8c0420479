"""CPU oracle: ctypes binding of oracle/qpo.c (plain-C restatement of the
qppocr-kernels CPU arithmetic).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, by __graft_entry__.smoke() and
by bench.py's cpu_baseline leg, always as the checker or the timed CPU
baseline, never as the product path.  The product (qppocr_amd) never imports
this module.

Function names follow the reference operator API (qppocr-kernels/src/lib.rs:28-40):
conv2d, sgemm, softmax_last_dim, gelu_inplace, hardsigmoid, sigmoid_tensor,
relu_inplace, reduce_mean (last axis), matmul, convtranspose2d,
resize_nearest, plus the CTC argmax of qppocr-core/src/pipeline/rec.rs.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libqpo.so")
_lib = None

ACT_NONE, ACT_GELU, ACT_RELU, ACT_HARDSWISH, ACT_SIGMOID = 0, 1, 2, 3, 4
HS_ALPHA = np.float32(1.0 / 6.0)
HS_BETA = np.float32(0.5)
GELU_C = (np.float32(1.4142135), np.float32(1.0), np.float32(0.5))


def build():
    """Compile qpo.c into oracle/libqpo.so (gcc, no GPU needed)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        F = ctypes.c_float
        I = ctypes.c_int
        sig = {
            "qpo_threads": ([], I),
            "qpo_set_threads": ([I], None),
            "qpo_set_scalar": ([I], None),
            "qpo_exp1x8": ([P, P], None),
            "qpo_exp1": ([F], F),
            "qpo_erf1": ([F], F),
            "qpo_relu_inplace": ([P, I64], None),
            "qpo_hardsigmoid": ([P, P, I64, F, F], None),
            "qpo_sigmoid": ([P, P, I64], None),
            "qpo_gelu_inplace": ([P, I64, F, F, F], None),
            "qpo_erf_inplace": ([P, I64], None),
            "qpo_clip_inplace": ([P, I64, F, F], None),
            "qpo_softmax_last_dim": ([P, I64, I64], None),
            "qpo_sgemm_path": ([I64, I64, I64, I], I),
            "qpo_sgemm": ([P, P, P, I64, I64, I64, I64, P, I, F, F, F, P, I], None),
            "qpo_conv2d_out_shape": ([P, P, P, P], I),
            "qpo_conv2d": ([P, P, P, P, P, P, I, F, F, F, P, P, P], I),
            "qpo_convtranspose2x2": ([P, P, P, P, P], I),
            "qpo_resize_nearest": ([P, I64, I64, I64, I64, I64, P], None),
            "qpo_binary_flat": ([P, P, I64, I], None),
            "qpo_binary_bcast": ([P, P, I64, I64, I, I], None),
            "qpo_binary_scalar": ([P, I64, F, I, I, P], None),
            "qpo_reduce_mean_last": ([P, I64, I64, P], None),
            "qpo_sqrt_inplace": ([P, I64], None),
            "qpo_layernorm_chain": ([P, P, P, F, I64, I64, P], None),
            "qpo_matmul": ([P, P, P, I64, I64, I64, I64, I, I], None),
            "qpo_ctc_argmax": ([P, I64, I64, P], None),
            "qpo_global_avg_pool": ([P, I64, I64, P], None),
            "qpo_mul_add_scale": ([P, P, P, P, I64, I64, I64], None),
            "qpo_pool2d_out_hw": ([I64] * 10 + [P, P], None),
            "qpo_pool2d": ([P] + [I64] * 12 + [I, P], None),
            "qpo_resize_bilinear": ([P, I64, I64, I64, I64, I64, I, P], None),
            "qpo_transpose4": ([P, P, P, P], None),
            "qpo_det_normalize": ([P, I64, I64, P], None),
            "qpo_resize_bilinear_rgb_u8": ([P, I64, I64, P, I64, I64], None),
            "qpo_pack_crop": ([P, I64, I64, I64, I64, P, I], None),
            "qpo_db_mask": ([P, I64, I64, F, I, P], None),
            "qpo_ctc_collapse": ([P, I64, P, P], I64),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _i64(seq):
    return np.ascontiguousarray(np.asarray(seq, dtype=np.int64))


def threads():
    return lib().qpo_threads()


def set_threads(n):
    lib().qpo_set_threads(int(n))


def exp1x8(x):
    """exp1 on eight lanes at once (the AVX2 form)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(8)
    y = np.empty(8, np.float32)
    lib().qpo_exp1x8(_p(x), _p(y))
    return y


def set_scalar(on):
    """Every GEMM and softmax in the scalar form (the AVX2 forms give the
    same bits)."""
    lib().qpo_set_scalar(int(bool(on)))


def exp1(x):
    return np.float32(lib().qpo_exp1(float(np.float32(x))))


def erf1(x):
    return np.float32(lib().qpo_erf1(float(np.float32(x))))


def relu_inplace(t):
    lib().qpo_relu_inplace(_p(t), t.size)
    return t


def hardsigmoid(x, alpha=HS_ALPHA, beta=HS_BETA):
    x = _f32(x)
    y = np.empty_like(x)
    lib().qpo_hardsigmoid(_p(x), _p(y), x.size, float(alpha), float(beta))
    return y


def sigmoid_tensor(x):
    x = _f32(x)
    y = np.empty_like(x)
    lib().qpo_sigmoid(_p(x), _p(y), x.size)
    return y


def gelu_inplace(t, c1=GELU_C[0], c2=GELU_C[1], c3=GELU_C[2]):
    lib().qpo_gelu_inplace(_p(t), t.size, float(c1), float(c2), float(c3))
    return t


def erf_inplace(t):
    lib().qpo_erf_inplace(_p(t), t.size)
    return t


def clip_inplace(t, lo, hi):
    lib().qpo_clip_inplace(_p(t), t.size, float(lo), float(hi))
    return t


def softmax_last_dim(t, inner):
    assert t.size % inner == 0
    lib().qpo_softmax_last_dim(_p(t), t.size // inner, inner)
    return t


def sgemm_path(m, n, k, serial=False):
    return lib().qpo_sgemm_path(m, n, k, int(serial))


def sgemm(a, b, m, n, k, bias=None, act=ACT_NONE, residual=None, serial=False):
    """C[M,N] = A[M,K] B[K,N] (+bias per row, reference placement) -> act -> +residual."""
    a = _f32(a)
    b = _f32(b)
    c = np.empty((m, n), dtype=np.float32)
    bias = None if bias is None else _f32(bias)
    residual = None if residual is None else _f32(residual)
    c1, c2, c3 = act_params(act)
    lib().qpo_sgemm(_p(a), _p(b), _p(c), m, n, k, n, _p(bias), act, c1, c2, c3,
                    _p(residual), int(serial))
    return c


def act_params(act):
    """(c1, c2, c3) of an act kind: GELU's (sqrt2, 1, 0.5) (executor.rs:759-768),
    hardswish's HardSigmoid (alpha 1/6, beta 0.5) (activation.rs:243-251)."""
    if act == ACT_GELU:
        return tuple(float(v) for v in GELU_C)
    if act == ACT_HARDSWISH:
        return float(HS_ALPHA), float(HS_BETA), 0.0
    return 1.0, 0.0, 0.0


def conv_out_shape(xs, ws, params):
    ys = np.zeros(4, dtype=np.int64)
    rc = lib().qpo_conv2d_out_shape(_p(_i64(xs)), _p(_i64(ws)), _p(_i64(params)), _p(ys))
    if rc:
        raise ValueError(f"conv2d_out_shape: bad shapes {xs} {ws} {params} ({rc})")
    return tuple(int(v) for v in ys)


def conv_params(sh=1, sw=1, ph=0, pw=0, peh=None, pew=None, group=1):
    """ConvParams (qppocr-kernels/src/conv.rs:124-143) as the int64[9] the C side takes."""
    return [sh, sw, ph, pw, ph if peh is None else peh, pw if pew is None else pew, 1, 1, group]


def conv2d(x, w, bias=None, params=None, act=ACT_NONE, residual=None):
    """conv2d_res (qppocr-kernels/src/conv.rs:183-211): x NCHW, w [M, C/g, kh, kw]."""
    x = _f32(x)
    w = _f32(w)
    params = conv_params() if params is None else params
    ys = conv_out_shape(x.shape, w.shape, params)
    y = np.empty(ys, dtype=np.float32)
    bias = None if bias is None else _f32(bias)
    residual = None if residual is None else _f32(residual)
    c1, c2, c3 = act_params(act)
    rc = lib().qpo_conv2d(_p(x), _p(_i64(x.shape)), _p(w), _p(_i64(w.shape)), _p(bias),
                          _p(_i64(params)), act, c1, c2, c3, _p(residual), _p(y), None)
    if rc:
        raise ValueError(f"qpo_conv2d failed ({rc})")
    return y


def convtranspose2d(x, w):
    """convtranspose2d 2x2 s2 p0, no bias (qppocr-kernels/src/conv.rs:730-804)."""
    x = _f32(x)
    w = _f32(w)
    n, c, h, wd = x.shape
    y = np.empty((n, w.shape[1], 2 * h, 2 * wd), dtype=np.float32)
    rc = lib().qpo_convtranspose2x2(_p(x), _p(_i64(x.shape)), _p(w), _p(_i64(w.shape)), _p(y))
    if rc:
        raise ValueError("convtranspose2d: only 2x2 s2 p0 supported")
    return y


def resize_nearest(x, oh, ow):
    x = _f32(x)
    n, c, h, w = x.shape
    y = np.empty((n, c, oh, ow), dtype=np.float32)
    lib().qpo_resize_nearest(_p(x), n * c, h, w, oh, ow, _p(y))
    return y


def binary_flat(a, b, op):
    a = _f32(a).copy()
    b = _f32(b)
    assert a.size == b.size
    lib().qpo_binary_flat(_p(a), _p(b), a.size, op)
    return a


def binary_scalar(x, s, op, scalar_first=False):
    """y = x op s, or s op x (the one-element broadcast of binary_op)."""
    x = _f32(x)
    y = np.empty_like(x)
    lib().qpo_binary_scalar(_p(x), x.size, float(np.float32(s)), op, int(bool(scalar_first)), _p(y))
    return y


def binary_bcast(a, b, rows, cols, op, bmode):
    a = _f32(a).copy()
    b = _f32(b)
    lib().qpo_binary_bcast(_p(a), _p(b), rows, cols, op, bmode)
    return a


def reduce_mean_last(x):
    x = _f32(x)
    cols = x.shape[-1]
    rows = x.size // cols
    out = np.empty(x.shape[:-1], dtype=np.float32)
    lib().qpo_reduce_mean_last(_p(x), rows, cols, _p(out))
    return out


def layernorm(x, gamma, beta, eps):
    x = _f32(x)
    cols = x.shape[-1]
    y = np.empty_like(x)
    lib().qpo_layernorm_chain(_p(x), _p(_f32(gamma)), _p(_f32(beta)), float(eps),
                              x.size // cols, cols, _p(y))
    return y


def matmul(a, b):
    """Batched matmul (qppocr-kernels/src/shape.rs:568-698) for a [..., M, K] x b [..., K, N]
    where b is rank 2 (shared) or has a's batch dims."""
    a = _f32(a)
    b = _f32(b)
    m, k = a.shape[-2:]
    k2, n = b.shape[-2:]
    assert k == k2
    batch = int(np.prod(a.shape[:-2])) if a.ndim > 2 else 1
    b_shared = b.ndim == 2
    if not b_shared:
        assert int(np.prod(b.shape[:-2])) == batch
    out = np.empty(a.shape[:-2] + (m, n), dtype=np.float32)
    lib().qpo_matmul(_p(a), _p(b), _p(out), batch, m, k, n, 0, int(b_shared))
    return out


def ctc_argmax(probs):
    """(value, index-bits) pairs per row: qppocr-core/src/pipeline/rec.rs:34-90."""
    probs = _f32(probs)
    cols = probs.shape[-1]
    rows = probs.size // cols
    pairs = np.empty((rows, 2), dtype=np.float32)
    lib().qpo_ctc_argmax(_p(probs), rows, cols, _p(pairs))
    return pairs.reshape(probs.shape[:-1] + (2,))


def pairs_ids(pairs):
    """Index half of a pairs array as int32 (f32 bits -> u32)."""
    return np.ascontiguousarray(pairs[..., 1]).view(np.uint32).astype(np.int32)


def ctc_collapse(pairs, t_len):
    pairs = _f32(pairs).reshape(-1, 2)
    ids = np.empty(max(t_len, 1), dtype=np.int32)
    conf = np.zeros(1, dtype=np.float32)
    cnt = lib().qpo_ctc_collapse(_p(pairs), t_len, _p(ids), _p(conf))
    return ids[:cnt].copy(), float(conf[0])


# ------------------------------------------------------ pooling / SE / resize

def global_avg_pool(x):
    """[N, C, H, W] -> [N, C, 1, 1] (pool2d.rs:10-29, f64 sum in order)."""
    x = _f32(x)
    n, c = x.shape[:2]
    out = np.empty((n, c, 1, 1), np.float32)
    lib().qpo_global_avg_pool(_p(x), n * c, x.size // (n * c), _p(out))
    return out


def mul_add_scale(f, gate, r):
    """f * gate[c] + r per channel plane (elementwise.rs:134-179)."""
    f, gate, r = _f32(f), _f32(gate), _f32(r)
    c = gate.size
    hw = f.size // (f.shape[0] * f.shape[1])
    out = np.empty_like(f)
    lib().qpo_mul_add_scale(_p(f), _p(gate), _p(r), _p(out), c, hw, f.size)
    return out


def pool2d(x, kh, kw, sh, sw, ph, pw, peh, pew, max_pool):
    """pool2d (pool2d.rs:51-236); returns [N, C, oh, ow]."""
    x = _f32(x)
    n, c, h, w = x.shape
    oh, ow = ctypes.c_int64(), ctypes.c_int64()
    lib().qpo_pool2d_out_hw(h, w, kh, kw, sh, sw, ph, pw, peh, pew, ctypes.byref(oh),
                            ctypes.byref(ow))
    y = np.empty((n, c, oh.value, ow.value), np.float32)
    lib().qpo_pool2d(_p(x), n, c, h, w, kh, kw, sh, sw, ph, pw, peh, pew, int(max_pool), _p(y))
    return y


def resize_bilinear(x, oh, ow, align_corners=False):
    """resize_bilinear (resize.rs:60-142) over the last two axes."""
    x = _f32(x)
    h, w = x.shape[-2:]
    nc = x.size // (h * w)
    y = np.empty(x.shape[:-2] + (oh, ow), np.float32)
    lib().qpo_resize_bilinear(_p(x), nc, h, w, oh, ow, int(bool(align_corners)), _p(y))
    return y


def transpose4(x, perm):
    x = _f32(x)
    xs = _i64(x.shape)
    pm = _i64(perm)
    y = np.empty(tuple(x.shape[p] for p in perm), np.float32)
    lib().qpo_transpose4(_p(x), _p(xs), _p(pm), _p(y))
    return y


def det_normalize(rgb):
    """u8 [H, W, 3] -> f32 [1, 3, H, W] (engine.rs:959-982)."""
    rgb = np.ascontiguousarray(rgb, np.uint8)
    h, w = rgb.shape[:2]
    out = np.empty((1, 3, h, w), np.float32)
    lib().qpo_det_normalize(_p(rgb), h, w, _p(out))
    return out


def resize_bilinear_rgb_u8(src, dw, dh):
    """u8 [sh, sw, 3] -> u8 [dh, dw, 3] (resize.rs:153-209)."""
    src = np.ascontiguousarray(src, np.uint8)
    sh, sw = src.shape[:2]
    dst = np.empty((dh, dw, 3), np.uint8)
    lib().qpo_resize_bilinear_rgb_u8(_p(src), sw, sh, _p(dst), dw, dh)
    return dst


def pack_crop(crop, img_h, img_w, pad_only=False):
    """u8 crop [ch, cw, 3] -> f32 [3, img_h, img_w] slot (crop.rs:153-190)."""
    crop = np.ascontiguousarray(crop, np.uint8)
    ch, cw = crop.shape[:2]
    dst = np.zeros((3, img_h, img_w), np.float32)
    lib().qpo_pack_crop(_p(crop), ch, cw, img_h, img_w, _p(dst), int(bool(pad_only)))
    return dst


def db_mask(pred, thresh, dilate=True):
    """DB threshold then 2x2 dilation (geometry.rs:287-301, resize.rs:219-247)."""
    pred = _f32(pred)
    h, w = pred.shape[-2:]
    out = np.empty((h, w), np.uint8)
    lib().qpo_db_mask(_p(pred), h, w, float(thresh), int(bool(dilate)), _p(out))
    return out
