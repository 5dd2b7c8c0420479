"""Session elementwise nodes on the GPU against the CPU oracle: the Add / Sub /
Mul / Div node (qppocr-kernels/src/elementwise.rs:185-298, its one-element
fast path elementwise.rs:350-363), the Clip node (qppocr-core/src/executor.rs:
779-807, activation.rs:221-229) and the Add / Clip / Mul / Div export form of
hardswish, folded into the epilogue of the conv or linear before it.

Bar: bit-exact (every element equal, NaNs at the same places).
"""
import numpy as np
import pytest

from conftest import assert_bitexact

pytestmark = pytest.mark.gpu


def _run(g, x, build1=None):
    """Runs g on x through the session and the oracle (bit-exact, and a
    replay); with build1 (the same graph at batch 1), also real_n 1 against
    the oracle's one-item graph."""
    from qppocr_amd import nets
    from oracle import nets as onets
    sess = nets.HipSession(g)
    launches = sess.plan()
    got = sess.run(x)
    ref = onets.run_graph(g, x)
    for i, (a, b) in enumerate(zip(got, ref)):
        assert_bitexact(a, b, f"output {i}")
    again = sess.run(x)
    for i, (a, b) in enumerate(zip(again, got)):
        assert_bitexact(a, b, f"replay output {i}")
    if build1 is not None:
        got1 = sess.run(x[:1])
        ref1 = onets.run_graph(build1(), x[:1])
        for i, (a, b) in enumerate(zip(got1, ref1)):
            assert_bitexact(a, b, f"real_n 1 output {i}")
    sess.close()
    return launches


@pytest.mark.parametrize("shape", [(2, 8, 10, 12), (1, 3, 7, 5)], ids=["vec4", "ragged"])
def test_session_binary_nodes(gpu, oracle, shape):
    """Every op in both operand orders, scalar and same-shape, including
    zero divisors (signed infinities), on a 16-byte and a ragged size."""
    from qppocr_amd import nets

    def build(n):
        g = nets.Graph((n,) + shape[1:])
        outs = []
        for op in range(4):
            outs.append(g.binary(0, op, scalar=0.375))
            outs.append(g.binary(0, op, scalar=-1.25, scalar_first=True))
        prod = g.binary(outs[0], 2, other=outs[3])
        outs.append(prod)
        outs.append(g.binary(prod, 1, other=0))
        outs.append(g.binary(0, 3, other=outs[6]))
        g.outputs = outs
        return g

    g = build(shape[0])
    x = nets.WeightRng(21).normal(shape, 1.5)
    x.flat[::7] = 0.0
    print(f"binary nodes {shape}", flush=True)
    launches = _run(g, x, (lambda: build(1)) if shape[0] > 1 else None)
    assert len(launches) == len(g.nodes)


def test_session_clip_nodes(gpu, oracle):
    """Clip with NaN and infinities passing through, and Clip as a conv and
    linear activation (the reference runs it as the node after them)."""
    from qppocr_amd import nets
    r = nets.WeightRng(22)
    shape = (1, 16, 12, 20)
    g = nets.Graph(shape)
    x = r.normal(shape, 2.0)
    x.flat[::11] = np.nan
    x.flat[5::13] = np.inf
    x.flat[7::17] = -np.inf
    c0 = g.clip(0, -0.5, 1.25)
    w = g.weight(r.kaiming((24, 16, 3, 3), 144))
    b = g.weight(r.normal((24,), 0.1))
    xc = g.act(0, (nets.ACT_CLIP, -6.0, 6.0, 0.0))   # finite input for the conv
    c1 = g.conv(xc, w, b, pad=(1, 1, 1, 1), act=(nets.ACT_CLIP, 0.0, 0.75, 0.0))
    wl = g.weight(r.kaiming((20, 40), 20))
    bl = g.weight(r.normal((40,), 0.1))
    c2 = g.linear(xc, wl, bl, act=(nets.ACT_CLIP, -0.25, 0.5, 0.0))
    g.outputs = [c0, c1, c2]
    print("clip nodes and clip epilogues", flush=True)
    _run(g, x)


HSW_CASES = [
    # producer, shared (X also read elsewhere), separate launches
    ("conv3x3", False, False),
    ("conv1x1", False, False),
    ("depthwise", False, False),
    ("linear", False, False),
    ("dwpw", False, False),       # depthwise + 1x1 block: the fold rides on the block's launch
    ("conv3x3", True, False),
    ("conv3x3", False, True),
]


@pytest.mark.parametrize("case", HSW_CASES, ids=lambda c: f"{c[0]}-{int(c[1])}{int(c[2])}")
def test_session_hardswish_clip_fold(gpu, oracle, case):
    """X = producer; X + 3 -> Clip(0, 6) -> X * t -> t / 6: one launch when only
    the chain reads X and its intermediates (the producer's epilogue does the
    four roundings), five otherwise; bit-exact either way."""
    from qppocr_amd import nets
    prod, shared, separate = case
    shape = (2, 16, 14, 20)

    def build(n):
        r = nets.WeightRng(23)
        g = nets.Graph((n,) + shape[1:])
        if prod == "conv3x3":
            w = g.weight(r.kaiming((24, 16, 3, 3), 144))
            b = g.weight(r.normal((24,), 0.1))
            t = g.conv(0, w, b, pad=(1, 1, 1, 1))
        elif prod == "conv1x1":
            w = g.weight(r.kaiming((32, 16, 1, 1), 16))
            b = g.weight(r.normal((32,), 0.1))
            t = g.conv(0, w, b)
        elif prod == "depthwise":
            w = g.weight(r.kaiming((16, 1, 3, 3), 9))
            b = g.weight(r.normal((16,), 0.1))
            t = g.conv(0, w, b, stride=(2, 2), pad=(1, 1, 1, 1), group=16)
        elif prod == "dwpw":
            wd = g.weight(r.kaiming((16, 1, 3, 3), 9))
            bd = g.weight(r.normal((16,), 0.1))
            d = g.conv(0, wd, bd, pad=(1, 1, 1, 1), group=16, act=nets.ACT_HARDSWISH)
            w = g.weight(r.kaiming((32, 16, 1, 1), 16))
            b = g.weight(r.normal((32,), 0.1))
            t = g.conv(d, w, b)
        else:
            w = g.weight(r.kaiming((20, 48), 20))
            b = g.weight(r.normal((48,), 0.1))
            t = g.linear(0, w, b)
        y = g.hardswish_clip(t)
        g.outputs = [y, t] if shared else [y]
        if separate:
            g.flags |= nets.NET_SEPARATE_LAUNCHES
        return g

    g = build(2)
    x = nets.WeightRng(24).normal(shape, 3.0)
    print(f"hardswish clip form after {case}", flush=True)
    launches = _run(g, x, lambda: build(1))
    if prod == "dwpw":   # one launch: the block (two nodes) and the four folded nodes
        assert launches == [(0, 6, 1)], launches
        return
    assert ((0, 5, 1) in launches) == (not shared and not separate), launches
    assert len(launches) == (1 if (0, 5, 1) in launches else 5)
