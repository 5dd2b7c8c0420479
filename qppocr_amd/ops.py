"""Operator API of the HIP backend, mirroring the qppocr-kernels public functions
(qppocr-kernels/src/lib.rs:28-40): conv2d / conv2d_res, convtranspose2d,
sgemm / sgemm_res, matmul, softmax_last_dim, gelu_inplace, hardsigmoid,
sigmoid_tensor, relu_inplace, reduce_mean (last axis), resize_nearest, and the
CTC argmax of qppocr-core/src/pipeline/rec.rs.

Tensors are torch tensors on a ROCm device (torch is only the device-memory
plumbing here); every call goes through the C ABI of libqppocr_hip.so.  Calls
are synchronous with respect to torch's current stream: the stream is drained
before the library's own stream runs the kernel, and the library stream is
drained before returning.  Errors raise QphError (no silent fallback).
"""
import ctypes

import torch

from . import _lib
from ._lib import (ACT_GELU, ACT_HARDSWISH, ACT_NONE, ACT_RELU, ACT_SIGMOID, Act, ConvEpilogue,
                   ConvParams, check, i64arr)

HS_ALPHA = 1.0 / 6.0   # HardSigmoid alpha of the hardswish pair (activation.rs:243-251)
HS_BETA = 0.5
GELU_C = (1.4142135, 1.0, 0.5)  # FusedGelu defaults (executor.rs:759-768)

_ctx = {}


def context(device=0):
    """The library context (DeviceContext analogue) of a HIP device."""
    if device not in _ctx:
        lib = _lib.load()
        p = ctypes.c_void_p()
        check(lib.qph_ctx_create(int(device), ctypes.byref(p)))
        _ctx[device] = p
    return _ctx[device]


def new_context(device=0):
    """A further context of a HIP device, with its own stream: sessions on
    different contexts run concurrently (e.g. det of one page while rec of
    the previous page).  Destroy it with close_context."""
    lib = _lib.load()
    p = ctypes.c_void_p()
    check(lib.qph_ctx_create(int(device), ctypes.byref(p)))
    return p


def close_context(ctx):
    check(_lib.load().qph_ctx_destroy(ctx))


def _dev(t):
    return t.device.index if t.device.index is not None else torch.cuda.current_device()


def _ptr(t):
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("qppocr_amd ops take device tensors")
    if t.dtype != torch.float32:
        raise ValueError("qppocr_amd ops take float32 tensors")
    if not t.is_contiguous():
        raise ValueError("qppocr_amd ops take contiguous tensors")
    return ctypes.c_void_p(t.data_ptr())


class _Call:
    """Orders a library call after torch's pending work and waits for it."""

    def __init__(self, device):
        self.device = device
        self.ctx = context(device)

    def __enter__(self):
        torch.cuda.current_stream(self.device).synchronize()
        return self.ctx

    def __exit__(self, *exc):
        if exc[0] is None:
            check(_lib.load().qph_sync(self.ctx))
        return False


def act(kind=ACT_NONE):
    if kind == ACT_GELU:
        return Act(ACT_GELU, *GELU_C)
    if kind == ACT_HARDSWISH:
        return Act(ACT_HARDSWISH, HS_ALPHA, HS_BETA, 0.0)
    return Act(kind, 1.0, 0.0, 0.0)


def conv_params(sh=1, sw=1, ph=0, pw=0, peh=None, pew=None, group=1):
    return ConvParams(sh, sw, ph, pw, ph if peh is None else peh, pw if pew is None else pew,
                      1, 1, group)


def conv2d_out_shape(x_shape, w_shape, p):
    ys = (_lib.I64 * 4)()
    check(_lib.load().qph_conv2d_out_shape(i64arr(x_shape), i64arr(w_shape), ctypes.byref(p), ys))
    return tuple(int(v) for v in ys)


def conv2d(x, w, bias=None, params=None, act_kind=ACT_NONE, residual=None, out=None,
           res_up=0, y_ctotal=0, y_coff=0, y_up=1, trans_out=False):
    """conv2d_res (qppocr-kernels/src/conv.rs:183-211) with the fused epilogue
    options of qph_conv2d_ex."""
    params = conv_params() if params is None else params
    ys = conv2d_out_shape(x.shape, w.shape, params)
    if out is None:
        if trans_out:
            out = torch.empty((ys[0], ys[2] * ys[3], ys[1]), device=x.device)
        elif y_ctotal or y_up != 1:
            raise ValueError("placed output needs an explicit out tensor")
        else:
            out = torch.empty(ys, device=x.device)
    ep = ConvEpilogue(None if residual is None else residual.data_ptr(), res_up, y_ctotal, y_coff,
                      y_up, int(bool(trans_out)))
    a = act(act_kind)
    with _Call(_dev(x)) as ctx:
        check(_lib.load().qph_conv2d_ex(ctx, _ptr(x), i64arr(x.shape), _ptr(w), i64arr(w.shape),
                                        _ptr(bias), ctypes.byref(params), ctypes.byref(a),
                                        ctypes.byref(ep), _ptr(out)))
    return out


def convtranspose2d(x, w):
    """convtranspose2d, 2x2 s2 p0, no bias (qppocr-kernels/src/conv.rs:730-804)."""
    n, c, h, wd = x.shape
    out = torch.empty((n, w.shape[1], 2 * h, 2 * wd), device=x.device)
    with _Call(_dev(x)) as ctx:
        check(_lib.load().qph_convtranspose2d(ctx, _ptr(x), i64arr(x.shape), _ptr(w),
                                              i64arr(w.shape), 2, 2, 0, 0, _ptr(out), None))
    return out


def convt_pair_sigmoid(x, w1, w2):
    n, c, h, wd = x.shape
    out = torch.empty((n, 1, 4 * h, 4 * wd), device=x.device)
    with _Call(_dev(x)) as ctx:
        check(_lib.load().qph_convt2x2_pair_sigmoid(ctx, _ptr(x), i64arr(x.shape), _ptr(w1),
                                                    i64arr(w1.shape), _ptr(w2), i64arr(w2.shape),
                                                    _ptr(out)))
    return out


def sgemm(a, b, m, n, k, bias=None, act_kind=ACT_NONE, residual=None, serial=False):
    """sgemm / sgemm_res (qppocr-kernels/src/gemm.rs:37-70): C[M,N] = A[M,K] B[K,N]."""
    c = torch.empty((m, n), device=a.device)
    ac = act(act_kind)
    with _Call(_dev(a)) as ctx:
        check(_lib.load().qph_sgemm(ctx, _ptr(a), _ptr(b), _ptr(c), m, n, k, n, _ptr(bias),
                                    ctypes.byref(ac), _ptr(residual), int(bool(serial))))
    return c


def matmul(a, b):
    """MatMul (qppocr-kernels/src/shape.rs:568-698): a [..., M, K] x b [K, N] or [..., K, N]."""
    m, k = a.shape[-2:]
    n = b.shape[-1]
    batch = 1
    for d in a.shape[:-2]:
        batch *= d
    shared = b.dim() == 2
    out = torch.empty(tuple(a.shape[:-2]) + (m, n), device=a.device)
    with _Call(_dev(a)) as ctx:
        check(_lib.load().qph_matmul(ctx, _ptr(a), _ptr(b), _ptr(out), batch, m, k, n,
                                     int(shared)))
    return out


def linear(x, w, bias=None, act_kind=ACT_NONE, residual=None):
    """MatMul x[..., K] . w[K, N] -> Add(bias) -> act -> Add(residual)."""
    k, n = w.shape
    rows = x.numel() // k
    y = torch.empty(tuple(x.shape[:-1]) + (n,), device=x.device)
    ac = act(act_kind)
    with _Call(_dev(x)) as ctx:
        check(_lib.load().qph_linear(ctx, _ptr(x), _ptr(w), _ptr(bias), rows, k, n,
                                     ctypes.byref(ac), _ptr(residual), _ptr(y)))
    return y


def layernorm(x, gamma, beta, eps):
    cols = x.shape[-1]
    y = torch.empty_like(x)
    with _Call(_dev(x)) as ctx:
        check(_lib.load().qph_layernorm(ctx, _ptr(x), _ptr(gamma), _ptr(beta), float(eps),
                                        x.numel() // cols, cols, _ptr(y)))
    return y


def softmax_last_dim(t, inner):
    """In place (qppocr-kernels/src/activation.rs:321-334)."""
    with _Call(_dev(t)) as ctx:
        check(_lib.load().qph_softmax_last_dim(ctx, _ptr(t), t.numel() // inner, inner))
    return t


def softmax_argmax(logits, probs=True):
    """Row softmax + argmax pairs; probs=False exports the pairs only (the
    rec_argmax_pairs exit, qppocr-core/src/device.rs:160-165) and returns
    (None, pairs)."""
    cols = logits.shape[-1]
    rows = logits.numel() // cols
    pr = torch.empty_like(logits) if probs else None
    pairs = torch.empty(tuple(logits.shape[:-1]) + (2,), device=logits.device)
    with _Call(_dev(logits)) as ctx:
        check(_lib.load().qph_softmax_argmax(ctx, _ptr(logits), rows, cols,
                                             _ptr(pr) if probs else None, _ptr(pairs)))
    return pr, pairs


def linear_softmax_argmax(x, w, bias=None):
    """The fused rec head: MatMul + Add(bias) + Softmax + argmax pairs in one
    GEMM (logits never stored).  x [..., K], w [K, N]; returns pairs
    [..., 2].  Values agree with the unfused path to float rounding."""
    k, n = w.shape
    rows = x.numel() // k
    pairs = torch.empty(tuple(x.shape[:-1]) + (2,), device=x.device)
    with _Call(_dev(x)) as ctx:
        check(_lib.load().qph_linear_softmax_argmax(ctx, _ptr(x), _ptr(w), _ptr(bias), rows, k, n,
                                                    _ptr(pairs)))
    return pairs


def ctc_argmax(probs, t_valid=None):
    """(value, index-bits) per step; probs [B, T, C] (rec.rs:34-90)."""
    b, t, c = probs.shape
    pairs = torch.empty((b, t, 2), device=probs.device)
    tv = None
    if t_valid is not None:
        arr = (ctypes.c_int32 * b)(*[int(v) for v in t_valid])
        tv = ctypes.cast(arr, ctypes.c_void_p)
    with _Call(_dev(probs)) as ctx:
        check(_lib.load().qph_ctc_argmax(ctx, _ptr(probs), b, t, c, tv, _ptr(pairs)))
    return pairs


def attention(qkv, heads, dh, scale):
    b, t = qkv.shape[0], qkv.shape[1]
    out = torch.empty((b, t, heads * dh), device=qkv.device)
    with _Call(_dev(qkv)) as ctx:
        check(_lib.load().qph_attention(ctx, _ptr(qkv), b, t, heads, dh, float(scale), _ptr(out)))
    return out


def activation(x, act_kind):
    y = torch.empty_like(x)
    ac = act(act_kind)
    with _Call(_dev(x)) as ctx:
        check(_lib.load().qph_activation(ctx, _ptr(x), _ptr(y), x.numel(), ctypes.byref(ac)))
    return y


def relu_inplace(t):
    ac = act(ACT_RELU)
    with _Call(_dev(t)) as ctx:
        check(_lib.load().qph_activation(ctx, _ptr(t), _ptr(t), t.numel(), ctypes.byref(ac)))
    return t


def gelu_inplace(t, c1=GELU_C[0], c2=GELU_C[1], c3=GELU_C[2]):
    ac = Act(ACT_GELU, c1, c2, c3)
    with _Call(_dev(t)) as ctx:
        check(_lib.load().qph_activation(ctx, _ptr(t), _ptr(t), t.numel(), ctypes.byref(ac)))
    return t


def sigmoid_tensor(x):
    return activation(x, ACT_SIGMOID)


def hardsigmoid(x, alpha=HS_ALPHA, beta=HS_BETA):
    y = torch.empty_like(x)
    with _Call(_dev(x)) as ctx:
        check(_lib.load().qph_hardsigmoid(ctx, _ptr(x), _ptr(y), x.numel(), float(alpha),
                                          float(beta)))
    return y


def resize_nearest(x, oh, ow):
    n, c, h, w = x.shape
    y = torch.empty((n, c, oh, ow), device=x.device)
    with _Call(_dev(x)) as ctx:
        check(_lib.load().qph_resize_nearest(ctx, _ptr(x), n * c, h, w, oh, ow, _ptr(y)))
    return y


def binary_inplace(a, b, op, bmode):
    cols = a.shape[-1]
    with _Call(_dev(a)) as ctx:
        check(_lib.load().qph_binary_inplace(ctx, _ptr(a), _ptr(b), a.numel() // cols, cols, op,
                                             bmode))
    return a


def reduce_mean_last(x):
    cols = x.shape[-1]
    out = torch.empty(x.shape[:-1], device=x.device)
    with _Call(_dev(x)) as ctx:
        check(_lib.load().qph_reduce_mean_last(ctx, _ptr(x), x.numel() // cols, cols, _ptr(out)))
    return out


def pairs_ids(pairs):
    """Index half of a pairs tensor as int64 (f32 bits -> u32)."""
    return pairs[..., 1].contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF


# ------------------------------------------- pooling / SE gate / resize / layout

def _ptr_any(t):
    """Device pointer of a contiguous tensor of any dtype (u8 images)."""
    if not t.is_cuda or not t.is_contiguous():
        raise ValueError("qppocr_amd ops take contiguous device tensors")
    return ctypes.c_void_p(t.data_ptr())


def global_avg_pool(x):
    """global_avg_pool (qppocr-kernels/src/pool2d.rs:10-29): [N,C,H,W] -> [N,C,1,1]."""
    n, c, h, w = x.shape
    out = torch.empty((n, c, 1, 1), device=x.device)
    with _Call(_dev(x)) as ctx:
        check(_lib.load().qph_global_avg_pool(ctx, _ptr(x), n, c, h * w, _ptr(out)))
    return out


def mul_add_scale(feature, gate, residual):
    """mul_add_scale (elementwise.rs:134-179): feature * gate[c] + residual."""
    n, c, h, w = feature.shape
    out = torch.empty_like(feature)
    with _Call(_dev(feature)) as ctx:
        check(_lib.load().qph_mul_add_scale(ctx, _ptr(feature), _ptr(gate), _ptr(residual), n, c,
                                            h * w, _ptr(out)))
    return out


def pool2d(x, k, stride, pad=(0, 0, 0, 0), max_pool=True):
    """pool2d (pool2d.rs:51-236); pad = (ph, pw, peh, pew)."""
    n, c, h, w = x.shape
    kh, kw = k
    sh, sw = stride
    ph, pw, peh, pew = pad
    oh = max(h + ph + peh - kh, 0) // sh + 1
    ow = max(w + pw + pew - kw, 0) // sw + 1
    y = torch.empty((n, c, oh, ow), device=x.device)
    ys = (_lib.I64 * 4)()
    with _Call(_dev(x)) as ctx:
        check(_lib.load().qph_pool2d(ctx, _ptr(x), i64arr(x.shape), kh, kw, sh, sw, ph, pw, peh,
                                     pew, int(bool(max_pool)), _ptr(y), ys))
    assert tuple(ys) == (n, c, oh, ow)
    return y


def resize_bilinear(x, oh, ow, align_corners=False):
    """resize_bilinear (resize.rs:60-142) over the last two axes."""
    h, w = x.shape[-2:]
    nc = x.numel() // (h * w)
    y = torch.empty(tuple(x.shape[:-2]) + (oh, ow), device=x.device)
    with _Call(_dev(x)) as ctx:
        check(_lib.load().qph_resize_bilinear(ctx, _ptr(x), nc, h, w, oh, ow,
                                              int(bool(align_corners)), _ptr(y)))
    return y


def transpose(x, perm):
    """Rank-4 Transpose."""
    y = torch.empty(tuple(x.shape[p] for p in perm), device=x.device)
    pm = (_lib.I32 * 4)(*perm)
    with _Call(_dev(x)) as ctx:
        check(_lib.load().qph_transpose(ctx, _ptr(x), i64arr(x.shape), pm, _ptr(y)))
    return y


def det_normalize_u8(rgb):
    """det input (engine.rs:959-982): u8 [H, W, 3] -> f32 [1, 3, H, W]."""
    h, w = rgb.shape[:2]
    out = torch.empty((1, 3, h, w), device=rgb.device)
    with _Call(_dev(rgb)) as ctx:
        check(_lib.load().qph_det_normalize_u8(ctx, _ptr_any(rgb), h, w, _ptr(out)))
    return out


def resize_bilinear_rgb_u8(src, dw, dh):
    """resize_bilinear_rgb_u8 (resize.rs:153-209): u8 [sh, sw, 3] -> [dh, dw, 3]."""
    sh, sw = src.shape[:2]
    dst = torch.empty((dh, dw, 3), dtype=torch.uint8, device=src.device)
    with _Call(_dev(src)) as ctx:
        check(_lib.load().qph_resize_bilinear_rgb_u8(ctx, _ptr_any(src), sw, sh, _ptr_any(dst),
                                                     dw, dh))
    return dst


def pack_crop(crop, img_h, img_w, pad_only=False, out=None):
    """pack_crop (crop.rs:153-190): u8 crop [ch, cw, 3] -> f32 [3, img_h, img_w]."""
    ch, cw = crop.shape[:2]
    if out is None:
        out = torch.empty((3, img_h, img_w), device=crop.device)
    with _Call(_dev(crop)) as ctx:
        check(_lib.load().qph_pack_crop(ctx, _ptr_any(crop), ch, cw, img_h, img_w,
                                        int(bool(pad_only)), _ptr(out)))
    return out


def pack_crops(crops, img_h, img_w, pad_only=None, out=None):
    """A rec batch in one launch per 64 lines (engine.rs:1413-1431 packs it
    line by line): u8 crops [ch, cw, 3] -> f32 [n, 3, img_h, img_w], line i
    as pack_crop(crops[i], img_h, img_w, pad_only[i])."""
    n = len(crops)
    for c in crops:
        if c.dtype != torch.uint8 or c.dim() != 3 or c.shape[2] != 3:
            raise ValueError("pack_crops takes u8 [ch, cw, 3] crops")
    if pad_only is None:
        pad_only = [False] * n
    if out is None:
        out = torch.empty((n, 3, img_h, img_w), device=crops[0].device)
    ptrs = (ctypes.c_void_p * n)(*[_ptr_any(c).value for c in crops])
    ch = (_lib.I64 * n)(*[c.shape[0] for c in crops])
    cw = (_lib.I64 * n)(*[c.shape[1] for c in crops])
    po = (_lib.I32 * n)(*[int(bool(p)) for p in pad_only])
    with _Call(_dev(crops[0])) as ctx:
        check(_lib.load().qph_pack_crops(ctx, n, ptrs, ch, cw, po, img_h, img_w, _ptr(out)))
    return out


def db_mask(pred, thresh, dilate=True):
    """DB threshold + 2x2 dilation (geometry.rs:287-301, resize.rs:219-247)."""
    h, w = pred.shape[-2:]
    out = torch.empty((h, w), dtype=torch.uint8, device=pred.device)
    with _Call(_dev(pred)) as ctx:
        check(_lib.load().qph_db_mask(ctx, _ptr(pred), h, w, float(thresh), int(bool(dilate)),
                                      _ptr_any(out)))
    return out
