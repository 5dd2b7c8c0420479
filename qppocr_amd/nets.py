"""Static det / rec graphs of the synthetic OCR workloads and the session that
runs them on the HIP backend.

A Graph is the node list the DeviceContext receives after load-time
optimisation (qppocr-core/src/device.rs:83-101): numbered tensors, nodes
topologically ordered, weights in creation order.  Fusions follow the
reference graph optimiser where it has one (ReLU/GELU into group-1 conv,
qppocr-core/src/graph/optimize.rs:337-427; conv + residual,
optimize.rs:662-772; BN folded into the conv bias, optimize.rs:512-653) and
fold the remaining producer/consumer pairs into kernel epilogues with
per-element arithmetic identical to the separate nodes (HardSigmoid+Mul,
Resize(nearest)+Add, Resize+Concat, Reshape/Transpose).

Det (1 x 3 x H x W): stem conv3x3 s2 3->16 hardswish; blocks 2..12 each
dw(k, s) + hardswish -> pw 1x1 + hardswish with channels 16->32->64->128->256,
stride 2 at blocks 2, 4, 6, 12, 5x5 depthwise in blocks 9-11; FPN (C2..C5 =
outputs of blocks 3, 5, 11, 12) with 1x1 laterals to 96, nearest-2x
upsample-add top-down, 3x3 smoothing 96->24 per level, nearest upsample to
H/4 and concat [p5, p4, p3, p2] -> 96; head conv3x3 96->24 + ReLU, ConvT 2x2
s2 24->24, ConvT 2x2 s2 24->1 (bias-free, as the CPU ConvTranspose,
qppocr-kernels/src/conv.rs:730-740), Sigmoid -> 1 x 1 x H x W.

Rec (B x 3 x 48 x W): stem conv3x3 s2 3->32 hardswish; dw+pw blocks with dw
strides (2,2), (2,2), (2,1), (3,1) (the last with padding (0,1)) and
channels 32->64->128->256->256, giving [B, 256, 1, W/8] -> [B, W/8, 256];
two pre-LN encoder blocks (LN eps 1e-6, 8 heads x 32, q scale 1/sqrt(32),
MLP 256->1024 GELU ->256, residuals); head linear 256->18709, Softmax, CTC
argmax pairs.
"""
import ctypes
import math

import numpy as np

from . import _lib
from ._lib import (ACT_CLIP, ACT_GELU, ACT_HARDSIGMOID, ACT_HARDSWISH, ACT_HARDSWISH_CLIP,
                   ACT_NONE, ACT_RELU, BIN_ADD, BIN_DIV, BIN_MUL, NET_FUSED_HEAD,
                   NET_SEPARATE_LAUNCHES, Act,
                   ConvParams, Node, NetSpec,
                   OP_ACT, OP_ATTENTION, OP_BINARY, OP_CONV, OP_CONVT, OP_CONVT_PAIR_SIG,
                   OP_COPY_SLOT,
                   OP_GAP, OP_LAYERNORM, OP_LINEAR, OP_MUL_ADD_SCALE, OP_POOL, OP_RESIZE,
                   OP_SOFTMAX_ARGMAX, OP_TRANSPOSE, check)

HS = (1.0 / 6.0, 0.5, 0.0)
GELU_C = (1.4142135, 1.0, 0.5)
REC_CLASSES = 18709   # 18,708 dictionary entries + blank
REC_DIM, REC_HEADS, REC_DH, REC_MLP = 256, 8, 32, 1024
LN_EPS = 1e-6


def _act(kind):
    if isinstance(kind, tuple):          # (kind, c1, c2, c3): the Clip forms
        return Act(*kind)
    if kind in (ACT_HARDSWISH, ACT_HARDSIGMOID):
        return Act(kind, *HS)
    if kind == ACT_GELU:
        return Act(kind, *GELU_C)
    return Act(kind, 1.0, 0.0, 0.0)


class Graph:
    """Node list over numbered tensors plus the weights, in creation order."""

    def __init__(self, input_shape):
        self.shapes = []     # padded to rank 4 (the C tensor table)
        self.lshapes = []    # logical shapes
        self.alias = []
        self.nodes = []      # dicts (also read by the CPU oracle's executor)
        self.weights = []    # numpy float32 arrays
        self.outputs = []
        self.flags = 0       # QPH_NET_* session flags
        self.tensor(input_shape)

    # -------------------------------------------------------------- tensors
    def tensor(self, shape, alias=-1):
        s = [int(v) for v in shape] + [1] * (4 - len(shape))
        self.shapes.append(s)
        self.lshapes.append(tuple(int(v) for v in shape))
        self.alias.append(alias)
        return len(self.shapes) - 1

    def weight(self, arr):
        self.weights.append(np.ascontiguousarray(arr, dtype=np.float32))
        return len(self.weights) - 1

    def numel(self, t):
        return int(np.prod(self.shapes[t]))

    # ---------------------------------------------------------------- nodes
    def conv(self, x, w, b, stride=(1, 1), pad=(0, 0, 0, 0), group=1, act=ACT_NONE,
             residual=-1, res_up=0, out=None, y_ctotal=0, y_coff=0, y_up=1, trans_out=False):
        """Conv node (weights: ONNX [M, C/g, kh, kw]); pad = (ph, pw, peh, pew)."""
        n, c, h, wd = self.shapes[x]
        m, cg, kh, kw = self.weights[w].shape
        sh, sw = stride
        ph, pw, peh, pew = pad
        oh = (h + ph + peh - kh) // sh + 1
        ow = (wd + pw + pew - kw) // sw + 1
        if out is None:
            out = self.tensor((n, oh * ow, m) if trans_out else (n, m, oh, ow))
        self.nodes.append(dict(op=OP_CONV, inp=x, in2=residual, out=out, out2=-1, w=w, bias=b,
                               w2=-1, ws=(m, cg, kh, kw), w2s=(0, 0, 0, 0),
                               cp=(sh, sw, ph, pw, peh, pew, 1, 1, group), act=act, res_up=res_up,
                               trans_out=int(trans_out), y_ctotal=y_ctotal, y_coff=y_coff,
                               y_up=y_up, heads=0, dh=0, eps=0.0, scale=0.0))
        return out

    def convt_pair_sigmoid(self, x, w1, w2):
        n, c, h, wd = self.shapes[x]
        out = self.tensor((n, 1, 4 * h, 4 * wd))
        self.nodes.append(dict(op=OP_CONVT_PAIR_SIG, inp=x, in2=-1, out=out, out2=-1, w=w1,
                               bias=-1, w2=w2, ws=self.weights[w1].shape,
                               w2s=self.weights[w2].shape, cp=(1,) * 9, act=ACT_NONE, res_up=0,
                               trans_out=0, y_ctotal=0, y_coff=0, y_up=1, heads=0, dh=0, eps=0.0,
                               scale=0.0))
        return out

    def linear(self, x, w, b, act=ACT_NONE, residual=-1):
        k, nn = self.weights[w].shape
        rows = self.numel(x) // k
        s = self.shapes[x]
        out = self.tensor((s[0], rows // s[0], nn))
        self.nodes.append(dict(op=OP_LINEAR, inp=x, in2=residual, out=out, out2=-1, w=w, bias=b,
                               w2=-1, ws=(k, nn, 1, 1), w2s=(0, 0, 0, 0), cp=(1,) * 9, act=act,
                               res_up=0, trans_out=0, y_ctotal=0, y_coff=0, y_up=1, heads=0, dh=0,
                               eps=0.0, scale=0.0))
        return out

    def layernorm(self, x, g, b, eps):
        cols = self.weights[g].shape[0]
        out = self.tensor(self.lshapes[x])
        self.nodes.append(dict(op=OP_LAYERNORM, inp=x, in2=-1, out=out, out2=-1, w=g, bias=b,
                               w2=-1, ws=(cols, 1, 1, 1), w2s=(0, 0, 0, 0), cp=(1,) * 9,
                               act=ACT_NONE, res_up=0, trans_out=0, y_ctotal=0, y_coff=0, y_up=1,
                               heads=0, dh=0, eps=eps, scale=0.0))
        return out

    def attention(self, qkv, heads, dh, scale):
        b, t = self.shapes[qkv][0], self.shapes[qkv][1]
        out = self.tensor((b, t, heads * dh))
        self.nodes.append(dict(op=OP_ATTENTION, inp=qkv, in2=-1, out=out, out2=-1, w=-1, bias=-1,
                               w2=-1, ws=(0, 0, 0, 0), w2s=(0, 0, 0, 0), cp=(1,) * 9,
                               act=ACT_NONE, res_up=0, trans_out=0, y_ctotal=0, y_coff=0, y_up=1,
                               heads=heads, dh=dh, eps=0.0, scale=scale))
        return out

    def softmax_argmax(self, logits, cols, probs=True):
        """Softmax over rows of `cols` then per-row argmax pairs; probs=False
        exports the pairs only (rec_argmax_pairs, device.rs:160-165) and
        returns (-1, pairs)."""
        s = self.shapes[logits]
        probs = self.tensor(self.lshapes[logits]) if probs else -1
        rows = self.numel(logits) // cols
        pairs = self.tensor((s[0], rows // s[0], 2))
        self.nodes.append(dict(op=OP_SOFTMAX_ARGMAX, inp=logits, in2=-1, out=probs, out2=pairs,
                               w=-1, bias=-1, w2=-1, ws=(cols, 1, 1, 1), w2s=(0, 0, 0, 0),
                               cp=(1,) * 9, act=ACT_NONE, res_up=0, trans_out=0, y_ctotal=0,
                               y_coff=0, y_up=1, heads=0, dh=0, eps=0.0, scale=0.0))
        return probs, pairs

    # ---------------------------------------------- pooling / SE / layout
    def _node(self, op, x, out, **kw):
        d = dict(op=op, inp=x, in2=-1, in3=-1, out=out, out2=-1, w=-1, bias=-1, w2=-1,
                 ws=(0, 0, 0, 0), w2s=(0, 0, 0, 0), cp=(1, 1, 0, 0, 0, 0, 1, 1, 1), act=ACT_NONE,
                 res_up=0, trans_out=0, y_ctotal=0, y_coff=0, y_up=1, heads=0, dh=0, eps=0.0,
                 scale=0.0)
        d.update(kw)
        self.nodes.append(d)
        return out

    def act(self, x, act):
        """A standalone activation node (act: a kind or (kind, c1, c2, c3))."""
        return self._node(OP_ACT, x, self.tensor(self.lshapes[x]), act=act)

    def clip(self, x, lo, hi):
        """Clip node (executor.rs:779-807): lo / hi as the node's min / max."""
        return self.act(x, (ACT_CLIP, float(lo), float(hi), 0.0))

    def binary(self, x, op, other=-1, scalar=0.0, scalar_first=False):
        """Add / Sub / Mul / Div node: x op other (same element count), or with
        other = -1 the one-element broadcast x op scalar (scalar op x when
        scalar_first)."""
        return self._node(OP_BINARY, x, self.tensor(self.lshapes[x]), in2=other,
                          ws=(int(op), int(bool(scalar_first)), 0, 0), scale=float(scalar))

    def hardswish_clip(self, x):
        """The Add(3) / Clip(0, 6) / Mul / Div(6) export form of hardswish."""
        t = self.clip(self.binary(x, BIN_ADD, scalar=3.0), 0.0, 6.0)
        return self.binary(self.binary(x, BIN_MUL, other=t), BIN_DIV, scalar=6.0)

    def global_avg_pool(self, x):
        """GlobalAveragePool [N, C, H, W] -> [N, C, 1, 1] (pool2d.rs:10-29)."""
        n, c = self.shapes[x][:2]
        return self._node(OP_GAP, x, self.tensor((n, c, 1, 1)))

    def mul_add_scale(self, feature, gate, residual, out=None, y_ctotal=0, y_coff=0):
        """MulAddScale (optimize.rs:429-497): feature * gate + residual (residual
        -1: the gate Mul alone); out / y_ctotal / y_coff place it in a Concat
        slot."""
        n, c, h, w = self.shapes[feature]
        out = self.tensor((n, c, h, w)) if out is None else out
        return self._node(OP_MUL_ADD_SCALE, feature, out, in2=residual, in3=gate,
                          y_ctotal=y_ctotal, y_coff=y_coff)

    def pool(self, x, k, stride, pad=(0, 0, 0, 0), max_pool=True, out=None, y_ctotal=0,
             y_coff=0):
        """MaxPool / AveragePool (pool2d.rs:51-236); pad = (ph, pw, peh, pew)."""
        n, c, h, w = self.shapes[x]
        kh, kw = k
        sh, sw = stride
        ph, pw, peh, pew = pad
        oh = max(h + ph + peh - kh, 0) // sh + 1
        ow = max(w + pw + pew - kw, 0) // sw + 1
        out = self.tensor((n, c, oh, ow)) if out is None else out
        return self._node(OP_POOL, x, out, ws=(int(max_pool), 0, kh, kw),
                          cp=(sh, sw, ph, pw, peh, pew, 1, 1, 1), y_ctotal=y_ctotal, y_coff=y_coff)

    def resize(self, x, oh, ow, bilinear=True, align_corners=False, out=None, y_ctotal=0,
               y_coff=0):
        """Resize: nearest (resize.rs:8-57) or bilinear (resize.rs:60-142)."""
        n, c = self.shapes[x][:2]
        out = self.tensor((n, c, oh, ow)) if out is None else out
        return self._node(OP_RESIZE, x, out, ws=(int(bilinear), int(align_corners), 0, 0),
                          y_ctotal=y_ctotal, y_coff=y_coff)

    def transpose(self, x, perm):
        """Rank-4 Transpose: output dimension d is input dimension perm[d]."""
        s = self.shapes[x]
        return self._node(OP_TRANSPOSE, x, self.tensor(tuple(s[p] for p in perm)),
                          ws=tuple(int(p) for p in perm))

    def copy_slot(self, x, out, y_ctotal, y_coff):
        """A Concat input no producer writes in place, copied into its slot."""
        return self._node(OP_COPY_SLOT, x, out, y_ctotal=y_ctotal, y_coff=y_coff)

    # ------------------------------------------------------------ C struct
    def to_c(self):
        nt = len(self.shapes)
        shapes = (ctypes.c_int64 * (4 * nt))(*[v for s in self.shapes for v in s])
        alias = (ctypes.c_int32 * nt)(*self.alias)
        nodes = (Node * len(self.nodes))()
        for i, d in enumerate(self.nodes):
            nd = nodes[i]
            nd.op, nd.in_, nd.in2, nd.out, nd.out2 = d["op"], d["inp"], d["in2"], d["out"], d["out2"]
            nd.w, nd.bias, nd.w2 = d["w"], d["bias"], d["w2"]
            for j in range(4):
                nd.ws[j] = int(d["ws"][j])
                nd.w2s[j] = int(d["w2s"][j])
            nd.cp = ConvParams(*d["cp"])
            nd.act = _act(d["act"])
            nd.res_up, nd.trans_out = d["res_up"], d["trans_out"]
            nd.y_ctotal, nd.y_coff, nd.y_up = d["y_ctotal"], d["y_coff"], d["y_up"]
            nd.heads, nd.dh, nd.eps, nd.scale = d["heads"], d["dh"], d["eps"], d["scale"]
            nd.in3 = d.get("in3", -1)
        wsizes = (ctypes.c_int64 * max(1, len(self.weights)))(*[w.size for w in self.weights])
        outs = (ctypes.c_int32 * max(1, len(self.outputs)))(*self.outputs)
        spec = NetSpec(nt, shapes, alias, len(self.nodes), nodes, len(self.weights), wsizes,
                       len(self.outputs), outs, self.flags)
        keep = (shapes, alias, nodes, wsizes, outs)
        return spec, keep


# ------------------------------------------------------------------ weights

class WeightRng:
    """Seeded synthetic weights: numpy PCG64; Kaiming-normal N(0, sqrt(2/fan_in))
    conv/linear weights, N(0, 0.1) biases (BN folded in), drawn in graph order."""

    def __init__(self, seed):
        self.rng = np.random.Generator(np.random.PCG64(seed))

    def uniform(self, shape, lo=0.0, hi=1.0):
        u = self.rng.random(size=shape, dtype=np.float32)
        return (u * np.float32(hi - lo) + np.float32(lo)).astype(np.float32)

    def normal(self, shape, std):
        return (self.rng.standard_normal(size=shape, dtype=np.float32) * np.float32(std)).astype(
            np.float32)

    def kaiming(self, shape, fan_in):
        return self.normal(shape, math.sqrt(2.0 / fan_in))


def det_input(seed, h=640, w=640):
    """U[0,1) image normalised as the det pre-processing does:
    (v - 0.5) * (1 / 0.5) (qppocr-core/src/pipeline/engine.rs:966-979)."""
    r = WeightRng(seed)
    u = r.uniform((1, 3, h, w))
    x = ((u - np.float32(0.5)) * np.float32(1.0 / 0.5)).astype(np.float32)
    return x, r


DET_BLOCKS = [  # (dw kernel, stride, cin, cout) for blocks 2..12
    (3, 2, 16, 32), (3, 1, 32, 32), (3, 2, 32, 64), (3, 1, 64, 64), (3, 2, 64, 128),
    (3, 1, 128, 128), (3, 1, 128, 128), (5, 1, 128, 128), (5, 1, 128, 128), (5, 1, 128, 128),
    (3, 2, 128, 256),
]


def build_det(seed=2, h=640, w=640):
    """Det graph and its input; weights drawn after the input from the same stream."""
    x_in, r = det_input(seed, h, w)
    g = Graph((1, 3, h, w))
    # stem
    ws = g.weight(r.kaiming((16, 3, 3, 3), 27))
    bs = g.weight(r.normal((16,), 0.1))
    x = g.conv(0, ws, bs, stride=(2, 2), pad=(1, 1, 1, 1), act=ACT_HARDSWISH)
    feats = {}
    for bi, (k, s, cin, cout) in enumerate(DET_BLOCKS, start=2):
        wd = g.weight(r.kaiming((cin, 1, k, k), k * k))
        bd = g.weight(r.normal((cin,), 0.1))
        x = g.conv(x, wd, bd, stride=(s, s), pad=(k // 2,) * 4, group=cin, act=ACT_HARDSWISH)
        wp = g.weight(r.kaiming((cout, cin, 1, 1), cin))
        bp = g.weight(r.normal((cout,), 0.1))
        x = g.conv(x, wp, bp, act=ACT_HARDSWISH)
        feats[bi] = x
    c2, c3, c4, c5 = feats[3], feats[5], feats[11], feats[12]

    def lat(c, cin, coarse):
        wl = g.weight(r.kaiming((96, cin, 1, 1), cin))
        bl = g.weight(r.normal((96,), 0.1))
        if coarse < 0:
            return g.conv(c, wl, bl)
        return g.conv(c, wl, bl, residual=coarse, res_up=2)

    in5 = lat(c5, 256, -1)
    in4 = lat(c4, 128, in5)
    in3 = lat(c3, 64, in4)
    in2 = lat(c2, 32, in3)
    fh, fw = g.shapes[in2][2], g.shapes[in2][3]
    fuse = g.tensor((1, 96, fh, fw))
    for slot, (src, up) in enumerate([(in5, 8), (in4, 4), (in3, 2), (in2, 1)]):
        wsm = g.weight(r.kaiming((24, 96, 3, 3), 96 * 9))
        bsm = g.weight(r.normal((24,), 0.1))
        g.conv(src, wsm, bsm, pad=(1, 1, 1, 1), out=fuse, y_ctotal=96, y_coff=24 * slot, y_up=up)
    wh = g.weight(r.kaiming((24, 96, 3, 3), 96 * 9))
    bh = g.weight(r.normal((24,), 0.1))
    hh = g.conv(fuse, wh, bh, pad=(1, 1, 1, 1), act=ACT_RELU)
    wt1 = g.weight(r.kaiming((24, 24, 2, 2), 24 * 4))
    wt2 = g.weight(r.kaiming((24, 1, 2, 2), 24 * 4))
    prob = g.convt_pair_sigmoid(hh, wt1, wt2)
    g.outputs = [prob]
    return g, x_in


def rec_input(seed, batch=32, h=48, w=320):
    r = WeightRng(seed)
    x = r.uniform((batch, 3, h, w), -1.0, 1.0)
    return x, r


REC_BLOCKS = [  # (dw stride, dw padding (ph, pw, peh, pew), cin, cout)
    ((2, 2), (1, 1, 1, 1), 32, 64), ((2, 2), (1, 1, 1, 1), 64, 128),
    ((2, 1), (1, 1, 1, 1), 128, 256), ((3, 1), (0, 1, 0, 1), 256, 256),
]


def rec_weights(r):
    """All rec weights in graph order (shape-independent of the input)."""
    ws = [r.kaiming((32, 3, 3, 3), 27), r.normal((32,), 0.1)]
    for _, _, cin, cout in REC_BLOCKS:
        ws += [r.kaiming((cin, 1, 3, 3), 9), r.normal((cin,), 0.1),
               r.kaiming((cout, cin, 1, 1), cin), r.normal((cout,), 0.1)]
    d = REC_DIM
    for _ in range(2):
        ws += [(1.0 + r.normal((d,), 0.1)).astype(np.float32), r.normal((d,), 0.1),
               r.kaiming((d, 3 * d), d), r.normal((3 * d,), 0.1),
               r.kaiming((d, d), d), r.normal((d,), 0.1),
               (1.0 + r.normal((d,), 0.1)).astype(np.float32), r.normal((d,), 0.1),
               r.kaiming((d, REC_MLP), d), r.normal((REC_MLP,), 0.1),
               r.kaiming((REC_MLP, d), REC_MLP), r.normal((d,), 0.1)]
    ws += [r.kaiming((d, REC_CLASSES), d), r.normal((REC_CLASSES,), 0.1)]
    return ws


def build_rec_graph(weights, batch, w, h=48, probs=True, fused_head=False):
    """Rec graph for a [batch, 3, h, w] input over the weights of rec_weights().
    probs=False: the head exports the (val, idx) pairs only, the GPU
    sessions' CTC exit (rec_argmax_pairs, device.rs:160-165).  fused_head:
    pairs only, and the session runs the head linear + softmax argmax as one
    GEMM (QPH_NET_FUSED_HEAD; pairs to float rounding, not bit-exact)."""
    if fused_head:
        probs = False
    it = iter(weights)
    g = Graph((batch, 3, h, w))
    nw = lambda: g.weight(next(it))  # noqa: E731
    ws, bs = nw(), nw()
    x = g.conv(0, ws, bs, stride=(2, 2), pad=(1, 1, 1, 1), act=ACT_HARDSWISH)
    for i, (st, pad, cin, cout) in enumerate(REC_BLOCKS):
        wd, bd = nw(), nw()
        x = g.conv(x, wd, bd, stride=st, pad=pad, group=cin, act=ACT_HARDSWISH)
        wp, bp = nw(), nw()
        last = i == len(REC_BLOCKS) - 1
        x = g.conv(x, wp, bp, act=ACT_HARDSWISH, trans_out=last)
    for _ in range(2):
        g1, b1 = nw(), nw()
        hdn = g.layernorm(x, g1, b1, LN_EPS)
        wq, bq = nw(), nw()
        qkv = g.linear(hdn, wq, bq)
        att = g.attention(qkv, REC_HEADS, REC_DH, 1.0 / math.sqrt(REC_DH))
        wo, bo = nw(), nw()
        x = g.linear(att, wo, bo, residual=x)
        g2, b2 = nw(), nw()
        hdn = g.layernorm(x, g2, b2, LN_EPS)
        w1, b1m = nw(), nw()
        mm = g.linear(hdn, w1, b1m, act=ACT_GELU)
        w2, b2m = nw(), nw()
        x = g.linear(mm, w2, b2m, residual=x)
    wh, bh = nw(), nw()
    logits = g.linear(x, wh, bh)
    pr, pairs = g.softmax_argmax(logits, REC_CLASSES, probs)
    g.outputs = [pr, pairs] if probs else [pairs]
    if fused_head:
        g.flags |= NET_FUSED_HEAD
    return g


def build_rec(seed=3, batch=32, w=320, h=48, probs=True, fused_head=False):
    x_in, r = rec_input(seed, batch, h, w)
    g = build_rec_graph(rec_weights(r), batch, w, h, probs, fused_head)
    return g, x_in


# ------------------------------------------------------------------- cls

CLS_H, CLS_W = 48, 192   # the cls canvas (PipelineConfig cls_height / cls_width, config.rs:156)
CLS_BLOCKS = [  # (dw kernel, stride, cin, cout, SE gate on the depthwise output)
    (3, 1, 16, 32, False), (3, 2, 32, 64, False), (3, 1, 64, 64, False),
    (3, 2, 64, 128, False), (3, 1, 128, 128, False), (5, 2, 128, 256, True),
    (5, 1, 256, 256, True),
]
CLS_LAST = 1280          # the 1x1 conv after the last GlobalAveragePool
CLS_CLASSES = 2          # 0 and 180 degrees


def cls_input(seed, batch=32, h=CLS_H, w=CLS_W):
    r = WeightRng(seed)
    x = r.uniform((batch, 3, h, w), -1.0, 1.0)
    return x, r


def cls_weights(r):
    """All cls weights in graph order (shape-independent of the batch)."""
    ws = [r.kaiming((16, 3, 3, 3), 27), r.normal((16,), 0.1)]
    for k, _, cin, cout, se in CLS_BLOCKS:
        ws += [r.kaiming((cin, 1, k, k), k * k), r.normal((cin,), 0.1)]
        if se:
            ws += [r.kaiming((cin // 4, cin, 1, 1), cin), r.normal((cin // 4,), 0.1),
                   r.kaiming((cin, cin // 4, 1, 1), cin // 4), r.normal((cin,), 0.1)]
        ws += [r.kaiming((cout, cin, 1, 1), cin), r.normal((cout,), 0.1)]
    c = CLS_BLOCKS[-1][3]
    ws += [r.kaiming((CLS_LAST, c, 1, 1), c), r.normal((CLS_LAST,), 0.1),
           r.kaiming((CLS_LAST, CLS_CLASSES), CLS_LAST), r.normal((CLS_CLASSES,), 0.1)]
    return ws


def build_cls_graph(weights, batch, h=CLS_H, w=CLS_W):
    """Text-line orientation classifier (the engine's cls stage,
    qppocr-core/src/pipeline/engine.rs:1294-1380) on [batch, 3, h, w]: a
    PP-LCNet-style backbone (stem conv 3x3 s2 + hardswish; depthwise +
    pointwise blocks, the last two with an SE gate on the depthwise output:
    GlobalAveragePool, 1x1 + ReLU, 1x1 + HardSigmoid, Mul), then
    GlobalAveragePool, a 1x1 conv to 1280 + hardswish, the linear to 2
    classes and the row softmax: [batch, 2] probabilities."""
    it = iter(weights)
    g = Graph((batch, 3, h, w))
    nw = lambda: g.weight(next(it))  # noqa: E731
    ws, bs = nw(), nw()
    x = g.conv(0, ws, bs, stride=(2, 2), pad=(1, 1, 1, 1), act=ACT_HARDSWISH)
    for k, s, cin, cout, se in CLS_BLOCKS:
        wd, bd = nw(), nw()
        x = g.conv(x, wd, bd, stride=(s, s), pad=(k // 2,) * 4, group=cin, act=ACT_HARDSWISH)
        if se:
            w1, b1, w2, b2 = nw(), nw(), nw(), nw()
            gp = g.global_avg_pool(x)
            gate = g.conv(g.conv(gp, w1, b1, act=ACT_RELU), w2, b2, act=ACT_HARDSIGMOID)
            x = g.mul_add_scale(x, gate, -1)
        wp, bp = nw(), nw()
        x = g.conv(x, wp, bp, act=ACT_HARDSWISH)
    wl, bl = nw(), nw()
    x = g.conv(g.global_avg_pool(x), wl, bl, act=ACT_HARDSWISH)
    wf, bf = nw(), nw()
    logits = g.linear(x, wf, bf)
    probs, _ = g.softmax_argmax(logits, CLS_CLASSES)
    g.outputs = [probs]
    return g


def build_cls(seed=5, batch=32, h=CLS_H, w=CLS_W):
    x_in, r = cls_input(seed, batch, h, w)
    return build_cls_graph(cls_weights(r), batch, h, w), x_in


def node_cost(g, d):
    """Algorithmic work of one node: (flops, bytes, bound).  flops = 2 x MACs
    of the mathematical op (activations not counted); bytes = compulsory fp32
    traffic, each input, weight and output counted once (an output written
    up x up times by a fused nearest upsample counts at its written size).
    bound: "mfma" for conv / linear / attention products, "hbm" otherwise."""
    f32 = 4
    op = d["op"]
    if op == OP_CONV:
        n = g.shapes[d["inp"]][0]
        m, cg, kh, kw = d["ws"]
        sh, sw, ph, pw, peh, pew = d["cp"][:6]
        group = d["cp"][8]
        h, w = g.shapes[d["inp"]][2], g.shapes[d["inp"]][3]
        oh = (h + ph + peh - kh) // sh + 1
        ow = (w + pw + pew - kw) // sw + 1
        fl = 2 * n * m * cg * kh * kw * oh * ow
        by = g.numel(d["inp"]) + m * cg * kh * kw + (m if d["bias"] >= 0 else 0)
        by += n * m * oh * ow * d["y_up"] ** 2
        if d["in2"] >= 0:
            by += g.numel(d["in2"])
        bound = "hbm" if group > 1 and cg == 1 else "mfma"
        return fl, by * f32, bound
    if op == OP_LINEAR:
        k, nn = d["ws"][0], d["ws"][1]
        rows = g.numel(d["inp"]) // k
        by = rows * k + k * nn + nn + rows * nn + (rows * nn if d["in2"] >= 0 else 0)
        return 2 * rows * k * nn, by * f32, "mfma"
    if op == OP_ATTENTION:
        b, t = g.shapes[d["inp"]][0], g.shapes[d["inp"]][1]
        hd = d["heads"] * d["dh"]
        return 2 * 2 * b * d["heads"] * t * t * d["dh"], (b * t * 3 * hd + b * t * hd) * f32, "mfma"
    if op == OP_CONVT_PAIR_SIG:
        n, c, h, w = g.shapes[d["inp"]]
        m1 = d["ws"][1]
        fl = 2 * n * h * w * 4 * (c * m1 + m1 * 4)
        by = g.numel(d["inp"]) + c * m1 * 4 + m1 * 4 + n * 16 * h * w
        return fl, by * f32, "hbm"
    if op == OP_CONVT:
        n, c, h, w = g.shapes[d["inp"]]
        m1 = d["ws"][1]
        return 2 * n * h * w * 4 * c * m1, (g.numel(d["inp"]) + c * m1 * 4 + n * m1 * 4 * h * w) * f32, "hbm"
    if op == OP_SOFTMAX_ARGMAX:
        cols = d["ws"][0]
        rows = g.numel(d["inp"]) // cols
        probs = rows * cols if d["out"] >= 0 else 0
        return 0, (rows * cols + probs + 2 * rows) * f32, "hbm"
    if op == OP_LAYERNORM:
        cols = d["ws"][0]
        return 0, (2 * g.numel(d["inp"]) + 2 * cols) * f32, "hbm"
    if op == OP_GAP:
        n, c = g.shapes[d["inp"]][:2]
        return 0, (g.numel(d["inp"]) + n * c) * f32, "hbm"
    if op == OP_MUL_ADD_SCALE:
        tensors = 3 if d["in2"] >= 0 else 2
        return 0, (tensors * g.numel(d["inp"]) + g.numel(d["in3"])) * f32, "hbm"
    if op == OP_BINARY:
        tensors = 3 if d["in2"] >= 0 else 2
        return 0, tensors * g.numel(d["inp"]) * f32, "hbm"
    if op in (OP_POOL, OP_RESIZE, OP_COPY_SLOT):
        n = g.shapes[d["inp"]][0]
        c = g.shapes[d["inp"]][1]
        oh, ow = g.shapes[d["out"]][2:]
        return 0, (g.numel(d["inp"]) + n * c * oh * ow) * f32, "hbm"
    return 0, 2 * g.numel(d["inp"]) * f32, "hbm"


def flops(g):
    """Algorithmic FLOPs of a graph: 2 x MACs of conv / linear / attention matmuls."""
    return sum(node_cost(g, d)[0] for d in g.nodes)


# ------------------------------------------------------------------ session

class HipSession:
    """DeviceSession over the HIP backend (qppocr-core/src/device.rs:125-176):
    created once per graph (weights resident), run(input) -> outputs.  The
    rec graph exports both the probability tensor and the (val, idx) argmax
    pairs (rec_argmax_pairs, device.rs:160-165)."""

    def __init__(self, graph, device=0, ctx=None):
        """ctx: the context (and so the stream) to run on; default: the
        device's shared context (ops.context)."""
        from . import ops
        self.lib = _lib.load()
        self.ctx = ctx if ctx is not None else ops.context(device)
        self.graph = graph
        spec, self._keep = graph.to_c()
        self._spec = spec
        warr = (ctypes.c_void_p * max(1, len(graph.weights)))(
            *[w.ctypes.data_as(ctypes.c_void_p).value for w in graph.weights])
        p = ctypes.c_void_p()
        check(self.lib.qph_net_create(self.ctx, ctypes.byref(spec), warr, ctypes.byref(p)))
        self.net = p

    @property
    def batch(self):
        """The input's batch dimension: the most batch items a run computes."""
        return self.graph.lshapes[0][0]

    @property
    def real_n(self):
        r, b = ctypes.c_int32(), ctypes.c_int32()
        check(self.lib.qph_net_real_n(self.net, ctypes.byref(r), ctypes.byref(b)))
        return r.value

    def set_real_n(self, n):
        """Real batch count of the runs that follow (the plan model's
        params[0], qppocr-gpu/src/plan.rs:587-593): batch items past it are
        neither uploaded, computed nor downloaded."""
        check(self.lib.qph_net_set_real_n(self.net, int(n)))

    def run(self, x, outputs=True):
        """x: numpy input (host) or a device pointer int; returns numpy outputs.
        A host input with fewer batch items than the net holds (a batch
        padded to the session's grain) sets the real count to its length
        first; outputs then hold the real items only."""
        if isinstance(x, np.ndarray):
            x = np.ascontiguousarray(x, dtype=np.float32)
            full = self.graph.lshapes[0]
            if x.shape[1:] == tuple(full[1:]) and 1 <= x.shape[0] <= full[0]:
                if x.shape[0] != self.real_n:
                    self.set_real_n(x.shape[0])
            else:
                assert x.size == self.graph.numel(0)
            inp, is_dev = x.ctypes.data_as(ctypes.c_void_p), 0
        elif x is None:
            inp, is_dev = None, 1
        else:
            inp, is_dev = ctypes.c_void_p(int(x)), 1
        outs = None
        optr = None
        if outputs:
            rn = self.real_n
            outs = [np.empty((rn,) + tuple(self.graph.lshapes[t][1:]), dtype=np.float32)
                    for t in self.graph.outputs]
            optr = (ctypes.c_void_p * len(outs))(*[o.ctypes.data_as(ctypes.c_void_p).value for o in outs])
        check(self.lib.qph_net_run(self.net, inp, is_dev, optr))
        return outs

    def staging(self, slot):
        """Pinned host buffer of the input (slot -1) or of output `slot`, as a
        numpy view (owned by the session; valid until close)."""
        p = ctypes.c_void_p()
        n = ctypes.c_int64()
        check(self.lib.qph_net_staging(self.net, slot, ctypes.byref(p), ctypes.byref(n)))
        shape = self.graph.lshapes[0 if slot < 0 else self.graph.outputs[slot]]
        buf = (ctypes.c_float * n.value).from_address(p.value)
        return np.frombuffer(buf, dtype=np.float32).reshape(shape)

    def run_async(self, upload=True, download=True):
        """run_deferred (device.rs:172): enqueue input upload (from the input
        staging buffer), the graph and the output downloads (into the output
        staging buffers); complete() waits."""
        flags = (_lib.RUN_UPLOAD if upload else 0) | (_lib.RUN_DOWNLOAD if download else 0)
        check(self.lib.qph_net_run_async(self.net, flags))

    def complete(self):
        check(self.lib.qph_net_complete(self.net))

    def tensor_ptr(self, tid):
        p = ctypes.c_void_p()
        n = ctypes.c_int64()
        check(self.lib.qph_net_tensor(self.net, tid, ctypes.byref(p), ctypes.byref(n)))
        return p.value, n.value

    def sync(self):
        check(self.lib.qph_sync(self.ctx))

    def set_profiling(self, on):
        check(self.lib.qph_net_set_profiling(self.net, int(on)))

    def node_times(self):
        n = len(self.graph.nodes)
        arr = (ctypes.c_double * n)()
        check(self.lib.qph_net_node_times(self.net, arr, n))
        return list(arr)

    def plan(self):
        """The launch sequence of a run: (first node, nodes covered, kernels
        issued) per launch."""
        n = len(self.graph.nodes)
        first, nodes, kern = ((ctypes.c_int32 * n)() for _ in range(3))
        cnt = ctypes.c_int32()
        check(self.lib.qph_net_plan(self.net, first, nodes, kern, n, ctypes.byref(cnt)))
        return [(first[j], nodes[j], kern[j]) for j in range(cnt.value)]

    def close(self):
        if self.net:
            self.lib.qph_net_destroy(self.net)
            self.net = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
