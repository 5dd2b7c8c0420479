"""Plans in the reference's plan model (qppocr-gpu/src/plan.rs) for this
package's graphs, and the session that runs them on the HIP kernel set.

The reference's PlanBuilder (plan.rs:547-2480) turns an optimised ONNX graph
and an input shape into a GraphPlan: one arena of u32 words (activations
NHWC with channels padded to a multiple of 4, parameter blocks, repacked
weights) and a dispatch list naming kernels of the backend's set.  The
Vulkan and Metal sessions consume that plan; HipPlanSession hands it to
qph_plan_create (the HIP kernel set of the same dispatch contracts).

PlanWriter lowers a nets.Graph (the det and rec graphs) to the dispatches
PlanBuilder emits in its Vulkan configuration for the node sequence that
graph stands for:
  Conv -> n_conv / n_conv8 (plan.rs:1353-1600; depthwise -> n_conv_dw),
  HardSigmoid + Mul after it -> n_elem 2 then n_elem 5 (plan.rs:2117-2218),
  Conv -> Resize -> Add (FPN) -> n_resize + n_elem 4, Concat -> n_concat_c,
  ConvTranspose -> n_convt (plan.rs:1645-1705), graph-output Sigmoid fused
  into n_exit (act 4), MatMul with a constant B -> n_conv8 over the rows
  (plan.rs:1873-2025) + Add bias as the [V] broadcast n_channel 1, the
  LayerNorm chain -> n_reduce_last / n_elem 8, 9, 6, 10, 11 / n_channel 0, 1,
  attention -> n_transpose_nd, n_elem 7, n_attn_mm, n_softmax (plan.rs:2026-
  2055), the CTC head -> n_softmax + n_exit3_argmax (plan.rs:1014).
One departure: a MatMul followed by GELU has no plan lowering in the
reference (GELU is a conv activation there, plan.rs:1346); it is written as
the conv form, the MatMul dispatch carrying the bias and act 1.

The arena is laid out by one bump allocator (16-byte aligned regions, no
reuse), word 0 first (real_n, plan.rs:587-593).
"""
import ctypes
import struct

import numpy as np

from . import _lib
from ._lib import (ACT_GELU, ACT_HARDSWISH, ACT_NONE, ACT_RELU, OP_ATTENTION, OP_CONV,
                   OP_CONVT_PAIR_SIG, OP_LAYERNORM, OP_LINEAR, OP_SOFTMAX_ARGMAX, check)

OFF_NONE = 0xFFFFFFFF
MMA_W_TAIL = 32          # words appended to every conv / MatMul weight blob (nhwc.rs)
HS_ALPHA, HS_BETA = 1.0 / 6.0, 0.5
GELU_C = (1.4142135, 1.0, 0.5)


def cpad4(c):
    """nhwc.rs:cpad4 -- channels padded to a multiple of 4."""
    return (int(c) + 3) // 4 * 4


def f32_bits(v):
    return struct.unpack("<I", struct.pack("<f", float(v)))[0]


def _words(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def repack_conv_w(w, co, cin, kh, kw):
    """nhwc.rs:repack_conv_w: word (t * cip + ci) * cop + o = w[o, ci, ky, kx]
    (t = ky * kw + kx), zero past the real channels."""
    cop, cip = cpad4(co), cpad4(cin)
    v = np.zeros((kh * kw, cip, cop), dtype=np.float32)
    v[:, :cin, :co] = np.asarray(w, np.float32).reshape(co, cin, kh * kw).transpose(2, 1, 0)
    return _words(v.reshape(-1))


def repack_dw_w(w, c, kh, kw):
    """nhwc.rs:repack_dw_w: word t * cp + ch = w[ch, 0, ky, kx]."""
    v = np.zeros((kh * kw, cpad4(c)), dtype=np.float32)
    v[:, :c] = np.asarray(w, np.float32).reshape(c, kh * kw).T
    return _words(v.reshape(-1))


def repack_convt_w(w, ci, co, kh, kw):
    """nhwc.rs:repack_convt_w: word (t * cip + i) * cop + o = w[i, o, ky, kx]."""
    v = np.zeros((kh * kw, cpad4(ci), cpad4(co)), dtype=np.float32)
    v[:, :ci, :co] = np.asarray(w, np.float32).reshape(ci, co, kh * kw).transpose(2, 0, 1)
    return _words(v.reshape(-1))


def conv_bias(b, co):
    """nhwc.rs:conv_bias: the bias padded to cpad4(co) words."""
    v = np.zeros(cpad4(co), dtype=np.float32)
    v[:co] = b
    return _words(v)


def vector_nhwc(v):
    """nhwc.rs:init_to_nhwc of a rank-1 tensor [V] (taken as [1, V, 1, 1]) or a
    scalar: cpad4(V) words."""
    v = np.asarray(v, np.float32).reshape(-1)
    out = np.zeros(cpad4(v.size), dtype=np.float32)
    out[:v.size] = v
    return _words(out)


class GraphPlan:
    """plan.rs:GraphPlan as plain data."""

    def __init__(self):
        self.total_words = 0
        self.uploads = []        # (word offset, uint32 array)
        self.dispatches = []     # (kernel name, parameter block offset, groups, node index)
        self.in_f32_off = 0
        self.in_shape = ()
        self.outputs = []        # (word offset, numel, shape)

    def params_of(self, i):
        """The parameter words of dispatch i (for tests)."""
        p_off = self.dispatches[i][1]
        for off, w in self.uploads:
            if off == p_off:
                return w
        raise KeyError(p_off)


def _div256(t):
    return (int(t) + 255) // 256


class PlanWriter:
    """Lowers a nets.Graph to a GraphPlan (see the module docstring)."""

    def __init__(self, graph):
        self.g = graph
        self.plan = GraphPlan()
        self.words = 0
        self.loc = {}            # tensor id -> word offset of its storage
        self.concat = {}         # concat tensor id -> list of (c_off, src_off, c)
        rn = self._static(np.array([1], dtype=np.uint32))
        assert rn == 0
        self.node = -1

    # ------------------------------------------------------------ arena
    def _alloc(self, n):
        off = self.words
        self.words += max(4, (int(n) + 3) // 4 * 4)
        return off

    def _static(self, words):
        words = np.ascontiguousarray(words, dtype=np.uint32)
        off = self._alloc(words.size)
        self.plan.uploads.append((off, words))
        return off

    def _emit(self, kernel, params, groups):
        pw = np.array([p if isinstance(p, (int, np.integer)) else f32_bits(p) for p in params],
                      dtype=np.uint32)
        p_off = self._static(pw)
        self.plan.dispatches.append((kernel, p_off, tuple(int(v) for v in groups), self.node))
        return p_off

    # ---------------------------------------------------------- helpers
    def _nhwc(self, t):
        n, c, h, w = self.g.shapes[t]
        return n, c, h, w, cpad4(c)

    def _rows(self, t, cols):
        """Rank-3 (and rank-4 [B, 1, T, C] conv) tensors stored as rows x cpad4(cols)."""
        rows = self.g.numel(t) // cols
        return rows, cpad4(cols)

    def _elem(self, op, a, n, b=OFF_NONE, p1=0.0, p2=0.0):
        out = self._alloc(n)
        self._emit("n_elem", [op, a, b, out, n, p1, p2], [_div256(n // 4), 1, 1])
        return out

    def _hardswish(self, x, n):
        hs = self._elem(2, x, n, p1=HS_ALPHA, p2=HS_BETA)
        return self._elem(5, x, n, b=hs)

    def _resize(self, x, nb, cp, ih, iw, oh, ow):
        out = self._alloc(nb * oh * ow * cp)
        sy, sx = np.float32(ih / oh), np.float32(iw / ow)   # host-side f64 ratios (plan.rs:1806-1838)
        self._emit("n_resize", [x, out, oh * ow, cp, ow, iw, ih, float(sy), float(sx)],
                   [_div256(oh * ow * cp // 4), nb, 1])
        return out

    # -------------------------------------------------------------- nodes
    def _conv(self, d):
        g = self.g
        n, c, h, w, cip = self._nhwc(d["inp"])
        m, cg, kh, kw = d["ws"]
        sh, sw, ph, pw, peh, pew = d["cp"][:6]
        group = d["cp"][8]
        oh = (h + ph + peh - kh) // sh + 1
        ow = (w + pw + pew - kw) // sw + 1
        x = self.loc[d["inp"]]
        wt = g.weights[d["w"]]
        bias = g.weights[d["bias"]] if d["bias"] >= 0 else None
        act = d["act"]
        fused_act = {ACT_NONE: 0, ACT_RELU: 2, ACT_GELU: 1}.get(act, 0)
        cop = cpad4(m)
        out = self._alloc(n * oh * ow * cop)
        if group == 1:
            w_off = self._static(np.concatenate([repack_conv_w(wt, m, c, kh, kw),
                                                 np.zeros(MMA_W_TAIL, np.uint32)]))
            b_off = self._static(conv_bias(bias, m)) if bias is not None else OFF_NONE
            nv = cop // 4
            kname = "n_conv8" if nv % 2 == 0 else "n_conv"
            tiles = -(-(oh * ow) // 4) * (nv // 2 if nv % 2 == 0 else nv)
            self._emit(kname, [x, w_off, b_off, out, oh * ow, cop, ow, w, h, cip // 4, kh * kw, kw,
                               sh, sw, ph, pw, fused_act, *GELU_C, OFF_NONE],
                       [_div256(tiles), n, 1])
        elif group == c and m == c and cg == 1:
            w_off = self._static(repack_dw_w(wt, c, kh, kw))
            b_off = self._static(conv_bias(bias, m)) if bias is not None else OFF_NONE
            self._emit("n_conv_dw", [x, w_off, b_off, out, oh * ow, cop, ow, w, h, kh * kw, kw,
                                     sh, sw, ph, pw, 0, *GELU_C, OFF_NONE],
                       [_div256(oh * ow * cop // 4), n, 1])
            fused_act = 0
        else:
            raise ValueError("plan: grouped conv is not lowered")
        y = out
        words = n * oh * ow * cop
        if act == ACT_HARDSWISH:
            y = self._hardswish(y, words)
        elif act != ACT_NONE and fused_act == 0:
            y = self._elem({ACT_RELU: 0}[act], y, words)
        if d["in2"] >= 0:
            r = self.loc[d["in2"]]
            if d["res_up"] == 2:
                rn, rc, rh, rw, rcp = self._nhwc(d["in2"])
                r = self._resize(r, rn, rcp, rh, rw, oh, ow)
            y = self._elem(4, y, words, b=r)
        if d["y_ctotal"]:
            up = d["y_up"]
            if up != 1:
                y = self._resize(y, n, cop, oh, ow, oh * up, ow * up)
            slots = self.concat.setdefault(d["out"], [])
            slots.append((d["y_coff"], y, m))
            if sum(s[2] for s in slots) == d["y_ctotal"]:
                self._concat(d["out"], sorted(slots))
        else:
            self.loc[d["out"]] = y

    def _concat(self, t, slots):
        n, c, h, w, cp = self._nhwc(t)
        out = self._alloc(n * h * w * cp)
        params = [out, n * h * w, len(slots), cp // 4]
        for _, src, m in slots:
            params += [src, cpad4(m) // 4]
        self._emit("n_concat_c", params, [_div256(n * h * w * cp // 4), 1, 1])
        self.loc[t] = out

    def _convt(self, x, n, ci, h, w, wt, co):
        cop, cip = cpad4(co), cpad4(ci)
        w_off = self._static(repack_convt_w(wt, ci, co, 2, 2))
        oh, ow = 2 * h, 2 * w
        out = self._alloc(n * oh * ow * cop)
        self._emit("n_convt", [x, w_off, OFF_NONE, out, oh * ow, cop, ow, w, h, cip, cip // 4, 2, 2,
                               2, 0, *GELU_C],
                   [_div256(oh * ow * cop // 4), n, 1])
        return out

    def _convt_pair_sigmoid(self, d):
        g = self.g
        n, c, h, w, _ = self._nhwc(d["inp"])
        w1, w2 = g.weights[d["w"]], g.weights[d["w2"]]
        m1, m2 = w1.shape[1], w2.shape[1]
        y = self._convt(self.loc[d["inp"]], n, c, h, w, w1, m1)
        y = self._convt(y, n, m1, 2 * h, 2 * w, w2, m2)
        # the Sigmoid of a graph output runs in n_exit (act 4, n_exit.comp)
        self.loc[d["out"]] = ("sigmoid", y)

    def _linear(self, d):
        g = self.g
        k, nn = d["ws"][0], d["ws"][1]
        rows, kp = self._rows(d["inp"], k)
        cols = cpad4(nn)
        x = self.loc[d["inp"]]
        wt = g.weights[d["w"]]
        bias = g.weights[d["bias"]] if d["bias"] >= 0 else None
        w_off = self._static(np.concatenate([repack_conv_w(wt.T, nn, k, 1, 1),
                                             np.zeros(MMA_W_TAIL, np.uint32)]))
        gelu = d["act"] == ACT_GELU
        b_off = self._static(conv_bias(bias, nn)) if (gelu and bias is not None) else OFF_NONE
        out = self._alloc(rows * cols)
        nv = cols // 4
        kname = "n_conv8" if nv % 2 == 0 else "n_conv"
        tiles = -(-rows // 4) * (nv // 2 if nv % 2 == 0 else nv)
        self._emit(kname, [x, w_off, b_off, out, rows, cols, rows, rows, 1, kp // 4, 1, 1, 1, 1, 0,
                           0, 1 if gelu else 0, *GELU_C, OFF_NONE], [_div256(tiles), 1, 1])
        y = out
        if bias is not None and not gelu:
            bv = self._static(vector_nhwc(bias))
            o2 = self._alloc(rows * cols)
            self._emit("n_channel", [1, y, bv, OFF_NONE, o2, rows * cols, cols, 0.0, 0.0, rows],
                       [_div256(rows * cols // 4), 1, 1])
            y = o2
        if d["act"] not in (ACT_NONE, ACT_GELU):
            raise ValueError("plan: linear activation is not lowered")
        if d["in2"] >= 0:
            y = self._elem(4, y, rows * cols, b=self.loc[d["in2"]])
        self.loc[d["out"]] = y

    def _layernorm(self, d):
        g = self.g
        cols = d["ws"][0]
        rows, cp = self._rows(d["inp"], cols)
        batch = g.shapes[d["inp"]][0]
        x = self.loc[d["inp"]]
        n = rows * cp
        c4 = cp // 4          # p1 carries the row's vec4 count as raw bits (plan.rs:2209-2214)

        def mean(src):
            out = self._alloc(rows * 4)
            self._emit("n_reduce_last", [src, out, rows, cols, cp, rows // batch], [rows, 1, 1])
            return out
        mu = mean(x)
        dv = self._elem(8, x, n, b=mu, p1=c4)
        sq = self._elem(9, dv, n)
        var = mean(sq)
        eps = self._static(vector_nhwc([d["eps"]]))
        ve = self._elem(6, var, rows * 4, b=eps)
        sd = self._elem(10, ve, rows * 4)
        q = self._elem(11, dv, n, b=sd, p1=c4)
        gm = self._static(vector_nhwc(g.weights[d["w"]]))
        bt = self._static(vector_nhwc(g.weights[d["bias"]]))
        o1 = self._alloc(n)
        self._emit("n_channel", [0, q, gm, OFF_NONE, o1, n, cp, 0.0, 0.0, rows], [_div256(n // 4), 1, 1])
        o2 = self._alloc(n)
        self._emit("n_channel", [1, o1, bt, OFF_NONE, o2, n, cp, 0.0, 0.0, rows], [_div256(n // 4), 1, 1])
        self.loc[d["out"]] = o2

    def _attention(self, d):
        g = self.g
        b, t = g.shapes[d["inp"]][0], g.shapes[d["inp"]][1]
        H, dh = d["heads"], d["dh"]
        hd = H * dh
        if cpad4(3 * hd) != 3 * hd or cpad4(hd) != hd:
            raise ValueError("plan: attention widths must be multiples of 4")
        qkv = self.loc[d["inp"]]
        total = b * t * 3 * hd
        t5 = self._alloc(total)
        self._emit("n_transpose_nd", [qkv, t5, total, 5, b, t, 3, H, dh, 2, 0, 3, 1, 4],
                   [_div256(total), 1, 1])
        part = b * H * t * dh
        q, k, v = t5, t5 + part, t5 + 2 * part
        sc = self._static(vector_nhwc([d["scale"]]))
        qs = self._elem(7, q, part, b=sc)
        kt = self._alloc(part)
        self._emit("n_transpose_nd", [k, kt, part, 4, b, H, t, dh, 0, 0, 1, 3, 2, 0],
                   [_div256(part), 1, 1])
        s = self._alloc(b * H * t * t)
        self._emit("n_attn_mm", [qs, kt, s, t, dh, t, b * H, H], [1, b * H * t, 1])
        p = self._alloc(b * H * t * t)
        self._emit("n_softmax", [s, p, b * H * t, t, t, H * t], [b * H * t, 1, 1])
        o = self._alloc(part)
        self._emit("n_attn_mm", [p, v, o, t, t, dh, b * H, H], [1, b * H * t, 1])
        y = self._alloc(part)
        self._emit("n_transpose_nd", [o, y, part, 4, b, H, t, dh, 0, 0, 2, 1, 3, 0],
                   [_div256(part), 1, 1])
        self.loc[d["out"]] = y

    def _softmax_argmax(self, d):
        g = self.g
        cols = d["ws"][0]
        rows, cp = self._rows(d["inp"], cols)
        batch = g.shapes[d["inp"]][0]
        p = self._alloc(rows * cp)
        self._emit("n_softmax", [self.loc[d["inp"]], p, rows, cols, cp, rows // batch], [rows, 1, 1])
        if d["out"] >= 0:
            self.loc[d["out"]] = ("probs", p, rows, cols, cp, rows // batch)
        self.loc[d["out2"]] = ("pairs", p, rows, cols, cp, rows // batch)

    # ---------------------------------------------------------------- build
    def build(self):
        g = self.g
        shp = g.shapes[0]
        nb, c, h, w = shp
        cp = cpad4(c)
        self.plan.in_shape = tuple(g.lshapes[0])
        self.plan.in_f32_off = self._alloc(nb * c * h * w)
        x = self._alloc(nb * h * w * cp)
        self._emit("n_entry", [self.plan.in_f32_off, x, nb, c, h, w, cp], [_div256(nb * h * w), 1, 1])
        self.loc[0] = x
        lower = {OP_CONV: self._conv, OP_LINEAR: self._linear, OP_LAYERNORM: self._layernorm,
                 OP_ATTENTION: self._attention, OP_SOFTMAX_ARGMAX: self._softmax_argmax,
                 OP_CONVT_PAIR_SIG: self._convt_pair_sigmoid}
        for i, d in enumerate(g.nodes):
            if d["op"] not in lower:
                raise ValueError(f"plan: node {i} op {d['op']} is not lowered")
            self.node = i
            lower[d["op"]](d)
        self.node = -1
        for t in g.outputs:
            self._exit(t)
        self.plan.total_words = self.words
        return self.plan

    def _exit(self, t):
        g = self.g
        loc = self.loc[t]
        shape = g.lshapes[t]
        numel = int(np.prod(shape))
        if isinstance(loc, tuple) and loc[0] == "pairs":
            _, p, rows, cols, cp, rpb = loc
            out = self._alloc(rows * 2)
            self._emit("n_exit3_argmax", [p, out, rows, cols, cp, rpb], [rows, 1, 1])
        elif isinstance(loc, tuple) and loc[0] == "probs":
            _, p, rows, cols, cp, rpb = loc
            out = self._alloc(rows * cols)
            self._emit("n_exit3", [p, out, rows, cols, cp, rpb], [_div256(rows * cols), 1, 1])
        else:
            sig = isinstance(loc, tuple) and loc[0] == "sigmoid"
            src = loc[1] if sig else loc
            n, c, h, w = g.shapes[t]
            out = self._alloc(numel)
            self._emit("n_exit", [src, out, n, c, h, w, cpad4(c), 4 if sig else 0],
                       [_div256(n * h * w), 1, 1])
        self.plan.outputs.append((out, numel, shape))


def build_plan(graph):
    return PlanWriter(graph).build()


def plan_spec(plan, lib=None):
    """The qph_plan_spec of a GraphPlan and the buffers it points into (keep
    both alive while the spec is used)."""
    lib = lib or _lib.load()
    ups = [(off, np.ascontiguousarray(w, dtype=np.uint32)) for off, w in plan.uploads]
    uarr = (_lib.PlanUpload * len(ups))()
    for i, (off, w) in enumerate(ups):
        uarr[i].off = off
        uarr[i].n_words = w.size
        uarr[i].words = w.ctypes.data_as(ctypes.c_void_p)
    darr = (_lib.PlanDispatch * len(plan.dispatches))()
    for i, (name, p_off, groups, _) in enumerate(plan.dispatches):
        kid = lib.qph_plan_kernel_id(name.encode())
        if kid < 0:
            check(kid)
        darr[i].kernel = kid
        darr[i].p_off = p_off
        for j in range(3):
            darr[i].groups[j] = groups[j]
    offs = (ctypes.c_uint32 * len(plan.outputs))(*[o[0] for o in plan.outputs])
    nums = (ctypes.c_int64 * len(plan.outputs))(*[o[1] for o in plan.outputs])
    spec = _lib.PlanSpec(plan.total_words, len(ups), uarr, len(plan.dispatches), darr,
                         plan.in_f32_off, int(np.prod(plan.in_shape)), len(plan.outputs), offs,
                         nums)
    return spec, (ups, uarr, darr, offs, nums)


def validate_plan(plan):
    """qph_plan_validate: every check of the load step, on the host (raises
    QphError naming the dispatch for a malformed plan)."""
    lib = _lib.load()
    spec, keep = plan_spec(plan, lib)
    check(lib.qph_plan_validate(ctypes.byref(spec)))
    del keep


class HipPlanSession:
    """A session over a GraphPlan: the reference's Vulkan / Metal session load
    and run steps (vulkan/session.rs) on the HIP kernel set (qph_plan_*)."""

    def __init__(self, plan, device=0, ctx=None):
        from . import ops
        self.lib = _lib.load()
        self.ctx = ctx if ctx is not None else ops.context(device)
        self.plan = plan
        spec, self._keep = plan_spec(plan, self.lib)
        p = ctypes.c_void_p()
        check(self.lib.qph_plan_create(self.ctx, ctypes.byref(spec), ctypes.byref(p)))
        self.handle = p

    def run(self, x, outputs=True, real_n=0):
        """x: numpy input (host) or None (reuse the arena's input); returns the
        outputs as numpy arrays (pairs as float32 [value, index bits])."""
        check(self.lib.qph_plan_set_real_n(self.handle, int(real_n)))
        inp, is_dev = None, 1
        if x is not None:
            x = np.ascontiguousarray(x, dtype=np.float32)
            assert x.size == int(np.prod(self.plan.in_shape))
            inp, is_dev = x.ctypes.data_as(ctypes.c_void_p), 0
        outs, optr = None, None
        if outputs:
            outs = [np.empty(shape, dtype=np.float32) for _, _, shape in self.plan.outputs]
            optr = (ctypes.c_void_p * len(outs))(*[o.ctypes.data_as(ctypes.c_void_p).value
                                                     for o in outs])
        check(self.lib.qph_plan_run(self.handle, inp, is_dev, optr))
        return outs

    def launches(self):
        n = ctypes.c_int32()
        check(self.lib.qph_plan_launches(self.handle, ctypes.byref(n)))
        return n.value

    def arena(self):
        p, n = ctypes.c_void_p(), ctypes.c_int64()
        check(self.lib.qph_plan_arena(self.handle, ctypes.byref(p), ctypes.byref(n)))
        return p.value, n.value

    def read(self, off, n):
        """n words of the arena at word offset off (device -> host)."""
        base, _ = self.arena()
        out = np.empty(n, dtype=np.float32)
        check(self.lib.qph_memcpy_d2h(self.ctx, out.ctypes.data_as(ctypes.c_void_p),
                                      ctypes.c_void_p(base + 4 * off), 4 * n))
        check(self.lib.qph_sync(self.ctx))
        return out

    def close(self):
        if getattr(self, "handle", None):
            self.lib.qph_plan_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
