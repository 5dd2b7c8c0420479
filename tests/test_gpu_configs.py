"""End-to-end parity of the five workloads on the GPU against the CPU oracle.

Bar: bit-exact fp32 outputs (every element equal) and identical CTC argmax
ids; the fp32 tolerance (1e-4 relative / 1e-5 absolute, argmax ids equal
except where the top-2 logit gap is below 1e-4) is checked as well, so a
future kernel that trades exactness for speed still has a stated bar.
"""
import math

import numpy as np
import pytest

from conftest import assert_bitexact, baseline_tol_check

pytestmark = pytest.mark.gpu


def _t(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def test_cfg1_conv3x3_bias_relu(gpu, oracle):
    torch = gpu
    from qppocr_amd import configs, ops
    x, w, b = configs.cfg1(0)
    print("cfg1 conv3x3 32->32 160x160 bias+relu", flush=True)
    y = ops.conv2d(_t(torch, x), _t(torch, w), _t(torch, b), ops.conv_params(1, 1, 1, 1), 2)
    ref = oracle.conv2d(x, w, b, oracle.conv_params(1, 1, 1, 1), oracle.ACT_RELU)
    got = y.cpu().numpy()
    baseline_tol_check(got, ref)
    assert_bitexact(got, ref, "cfg1")


@pytest.mark.parametrize("case", range(4))
def test_cfg2_depthwise_hardswish(gpu, oracle, case):
    torch = gpu
    from qppocr_amd import configs, ops
    x, w, b, k, s = configs.cfg2(1)[case]
    print(f"cfg2 case {case}: C{x.shape[1]} {x.shape[2]}^2 k{k} s{s}", flush=True)
    c = x.shape[1]
    y = ops.conv2d(_t(torch, x), _t(torch, w), _t(torch, b),
                   ops.conv_params(s, s, k // 2, k // 2, group=c), 3)
    ref = oracle.conv2d(x, w, b, oracle.conv_params(s, s, k // 2, k // 2, group=c))
    ref = oracle.binary_flat(ref, oracle.hardsigmoid(ref), 2)
    got = y.cpu().numpy()
    baseline_tol_check(got, ref)
    assert_bitexact(got, ref, f"cfg2[{case}]")


def test_cfg3_det_net(gpu, oracle):
    from qppocr_amd import nets
    from oracle import nets as onets
    g, x = nets.build_det(2, 640, 640)
    print("cfg3 det 1x3x640x640", flush=True)
    sess = nets.HipSession(g)
    out = sess.run(x)[0]
    ref = onets.run_graph(g, x)[0]
    baseline_tol_check(out, ref)
    assert_bitexact(out, ref, "det prob map")
    out2 = sess.run(x)[0]   # graph replay gives the same bits
    assert_bitexact(out2, out, "det replay")
    sess.close()


def _ids(pairs):
    return np.ascontiguousarray(pairs[..., 1]).view(np.uint32)


def test_cfg4_rec_net(gpu, oracle):
    from qppocr_amd import nets
    from oracle import nets as onets
    g, x = nets.build_rec(3, 32, 320)
    print("cfg4 rec 32x3x48x320", flush=True)
    sess = nets.HipSession(g)
    probs, pairs = sess.run(x)
    probs_ref, pairs_ref = onets.run_graph(g, x)
    baseline_tol_check(probs, probs_ref)
    assert_bitexact(probs, probs_ref, "rec probs")
    assert (_ids(pairs) == _ids(pairs_ref)).all()
    assert_bitexact(pairs[..., 0], pairs_ref[..., 0], "rec pair values")
    probs2, pairs2 = sess.run(x)
    assert_bitexact(probs2, probs, "rec replay")
    sess.close()


def test_cls_net(gpu, oracle):
    """The cls stage's net (engine.rs:1294-1380) over a 42-line page in the
    stage's batches of 32 (cls_batches): the second batch of 10 lines runs on
    the same 32-item session through real_n.  Probabilities bit-exact against
    the oracle's run of a net of the batch's own size, and the same flip
    decisions (cls_decisions)."""
    from qppocr_amd import nets, pipeline
    from oracle import nets as onets
    r = nets.WeightRng(5)
    cw = nets.cls_weights(r)
    x42 = r.uniform((42, 3, nets.CLS_H, nets.CLS_W), -1.0, 1.0)
    print("cls 32x3x48x192 net, lines 0..32 then real_n 10", flush=True)
    sess = nets.HipSession(nets.build_cls_graph(cw, 32))
    for b, e in pipeline.cls_batches(42):
        (probs,) = sess.run(x42[b:e])
        (ref,) = onets.run_graph(nets.build_cls_graph(cw, e - b), x42[b:e])
        assert probs.shape == ref.shape
        assert_bitexact(probs, ref, f"cls probabilities, lines {b}..{e}")
        flip, conf = pipeline.cls_decisions(probs)
        flip_r, conf_r = pipeline.cls_decisions(ref)
        assert (flip == flip_r).all() and (conf == conf_r).all()
    sess.close()


def test_rec_pairs_only_and_deferred_runs(gpu, oracle):
    """The rec graph with the pairs-only head (rec_argmax_pairs,
    device.rs:160-165) gives the same pairs as the full graph and the
    oracle; deferred runs (run_deferred / complete, device.rs:105-110,
    166-176) through the pinned staging buffers give the same bits, and a
    second deferred run before complete is refused."""
    from qppocr_amd import nets
    from qppocr_amd._lib import QphError
    from oracle import nets as onets
    g, x = nets.build_rec(3, 8, 240, probs=False)
    assert len(g.outputs) == 1
    print("rec 8x3x48x240 pairs only", flush=True)
    sess = nets.HipSession(g)
    (pairs,) = sess.run(x)
    (pairs_ref,) = onets.run_graph(g, x)
    assert (_ids(pairs) == _ids(pairs_ref)).all()
    assert_bitexact(pairs[..., 0], pairs_ref[..., 0], "pairs-only values")
    xin = sess.staging(-1)
    out = sess.staging(0)
    out[:] = np.nan
    xin[:] = x
    sess.run_async()
    with pytest.raises(QphError):
        sess.run_async()
    sess.complete()
    assert_bitexact(out, pairs, "deferred run pairs")
    x2 = np.ascontiguousarray(x[::-1])
    xin[:] = x2
    sess.run_async()
    sess.complete()
    (pairs2_ref,) = onets.run_graph(g, x2)
    assert (_ids(out) == _ids(pairs2_ref)).all()
    sess.close()


@pytest.mark.parametrize("batch,width", [(32, 320), (5, 160), (19, 480)])
def test_rec_fused_head(gpu, oracle, batch, width):
    """The rec graph with QPH_NET_FUSED_HEAD (head GEMM + softmax argmax in
    one kernel, logits never stored) against the oracle's full graph under
    the pairs tolerance rule; every node before the head is bit-exact already."""
    from conftest import pairs_tolerance_check
    from qppocr_amd import nets
    from oracle import nets as onets
    g, x = nets.build_rec(3, batch, width, fused_head=True)
    print(f"rec {batch}x3x48x{width} fused head", flush=True)
    sess = nets.HipSession(g)
    (pairs,) = sess.run(x)
    outs, T = onets.run_graph(g, x, keep=True)
    logits = T[g.nodes[-2]["out"]]
    pairs_tolerance_check(pairs, outs[0], logits)
    (pairs2,) = sess.run(x)
    assert_bitexact(pairs2, pairs, "fused head replay")
    sess.close()


def _d2h(sess, tid):
    import ctypes
    ptr, n = sess.tensor_ptr(tid)
    host = np.empty(n, dtype=np.float32)
    sess.sync()
    assert sess.lib.qph_memcpy_d2h(sess.ctx, host.ctypes.data_as(ctypes.c_void_p),
                                   ctypes.c_void_p(ptr), n * 4) == 0
    return host


def test_rec_real_n_padded_batch(gpu, oracle):
    """A 64-row rec net run with real_n (the plan model's params[0],
    qppocr-gpu/src/plan.rs:587-593; DeviceSession::batch_grain,
    qppocr-core/src/device.rs:139-157): 37 real lines give the oracle's bits
    for a 37-line batch, the 27 padded items are neither uploaded nor
    computed (their input and output rows keep the previous full run's
    contents), real_n = 1 gives the oracle's 1-line batch, and the 64-item
    graph still gives its earlier bits afterwards."""
    from qppocr_amd import nets
    from oracle import nets as onets
    r = nets.WeightRng(3)
    rw = nets.rec_weights(r)
    x64 = r.uniform((64, 3, 48, 160), -1.0, 1.0)
    x37 = r.uniform((37, 3, 48, 160), -1.0, 1.0)
    g = nets.build_rec_graph(rw, 64, 160)
    print("rec 64x3x48x160 net, full run then real_n 37 / 1 / 64", flush=True)
    sess = nets.HipSession(g)
    assert sess.batch == 64 and sess.real_n == 64
    probs64, pairs64 = sess.run(x64)
    probs, pairs = sess.run(x37)
    assert sess.real_n == 37 and probs.shape[0] == 37 and pairs.shape[0] == 37
    g37 = nets.build_rec_graph(rw, 37, 160)
    probs_ref, pairs_ref = onets.run_graph(g37, x37)
    assert_bitexact(probs, probs_ref, "real_n 37 probs")
    assert (_ids(pairs) == _ids(pairs_ref)).all()
    assert_bitexact(pairs[..., 0], pairs_ref[..., 0], "real_n 37 pair values")
    # padded items untouched: input rows 37.. hold x64's, outputs the full run's
    dev_in = _d2h(sess, 0).reshape(x64.shape)
    assert_bitexact(dev_in[:37], x37, "uploaded real rows")
    assert_bitexact(dev_in[37:], x64[37:], "padded input rows not uploaded")
    dev_pairs = _d2h(sess, g.outputs[1]).reshape(pairs64.shape)
    assert_bitexact(dev_pairs[37:], pairs64[37:], "padded pair rows not computed")
    dev_probs = _d2h(sess, g.outputs[0]).reshape(probs64.shape)
    assert_bitexact(dev_probs[37:], probs64[37:], "padded prob rows not computed")
    probs1, pairs1 = sess.run(x37[:1])
    g1 = nets.build_rec_graph(rw, 1, 160)
    probs1_ref, pairs1_ref = onets.run_graph(g1, x37[:1])
    assert_bitexact(probs1, probs1_ref, "real_n 1 probs")
    assert (_ids(pairs1) == _ids(pairs1_ref)).all()
    again64, _ = sess.run(x64)
    assert_bitexact(again64, probs64, "64-item graph after real_n runs")
    ref64 = onets.run_graph(g, x64)[0]
    assert_bitexact(probs64, ref64, "full 64-item run")
    sess.close()


def test_rec_real_n_fused_head_and_refusals(gpu, oracle):
    """The fused-head 64-row net at real_n 37 under the pairs tolerance rule
    against the oracle's 37-line graph; out-of-range counts and a count
    change while a deferred run is in flight are refused."""
    from conftest import pairs_tolerance_check
    from qppocr_amd import nets
    from qppocr_amd._lib import QphError
    from oracle import nets as onets
    r = nets.WeightRng(5)
    rw = nets.rec_weights(r)
    x37 = r.uniform((37, 3, 48, 160), -1.0, 1.0)
    g = nets.build_rec_graph(rw, 64, 160, fused_head=True)
    print("rec 64x3x48x160 fused head, real_n 37", flush=True)
    sess = nets.HipSession(g)
    (pairs,) = sess.run(x37)
    g37 = nets.build_rec_graph(rw, 37, 160, probs=False)
    outs, T = onets.run_graph(g37, x37, keep=True)
    pairs_tolerance_check(pairs, outs[0], T[g37.nodes[-2]["out"]])
    for bad in (0, 65, -1):
        with pytest.raises(QphError):
            sess.set_real_n(bad)
    assert sess.real_n == 37
    xin = sess.staging(-1)
    out = sess.staging(0)
    xin[:37] = x37
    sess.run_async()
    with pytest.raises(QphError):
        sess.set_real_n(12)
    sess.complete()
    assert_bitexact(out[:37], pairs, "deferred run at real_n 37")
    sess.close()


def test_cfg5_engine_batching(gpu, oracle):
    """The mixed page's lines batched as the reference engine batches them
    for a GPU session (width spans of 64, 64 lines a forward, widths rounded
    to 64; engine.rs:1211-1290, 1413-1422) and run on 64-row nets with
    real_n: every batch's pairs bit-exact with the oracle's graph of exactly
    that batch, and the decoded lines equal to the oracle's collapse."""
    from qppocr_amd import pipeline
    from oracle import nets as onets
    det_g, det_x, rw, lines, widths = pipeline.mixed_page(4, 1536, 128)
    print("cfg5 engine batching: 128 lines on 64-row nets", flush=True)
    page = pipeline.PageRunner(det_g, det_x, rw, lines, widths, engine=True)
    assert all(len(idx) <= 64 and bw % 64 == 0 for bw, idx in page.plan)
    page.upload()
    page.run()
    page.sync()
    got = page.rec_pairs()
    decoded = page.decode()
    for bw, idx, g, sess, x in page.rec:
        assert sess.batch == 64 and sess.real_n == len(idx)
        print(f"engine rec batch {len(idx)}x{bw}", flush=True)
        gb = pipeline.build_rec_graph(rw, len(idx), bw, pipeline.REC_H, probs=False)
        pairs_ref = onets.run_graph(gb, x)[-1]
        for b, i in enumerate(idx):
            assert (_ids(got[i]) == _ids(pairs_ref[b])).all(), f"line {i}"
            assert_bitexact(got[i][..., 0], pairs_ref[b][..., 0], f"line {i} values")
            t_valid = int(widths[i]) // pipeline.REC_STRIDE
            ref_ids, _ = oracle.ctc_collapse(pairs_ref[b][:t_valid], t_valid)
            assert decoded[i][0] == [int(v) for v in ref_ids], f"line {i} ids"
    page.close()


def test_cfg5_mixed_page(gpu, oracle):
    """det 1536^2 + 128 rec lines in width buckets, CTC masked past w/8:
    det map and every batch's pairs bit-exact with the oracle, and each
    line's decoded ids equal to the oracle's collapse of the oracle pairs."""
    from qppocr_amd import pipeline
    from oracle import nets as onets
    det_g, det_x, rw, lines, widths = pipeline.mixed_page(4, 1536, 128)
    print("cfg5 det 1536^2 + 128 lines", flush=True)
    page = pipeline.PageRunner(det_g, det_x, rw, lines, widths)
    page.upload()
    page.run()
    page.sync()
    det_ref = onets.run_graph(det_g, det_x)[0]
    assert_bitexact(page.det_map(), det_ref, "cfg5 det map")
    got = page.rec_pairs()
    decoded = page.decode()
    for bw, idx, g, _, x in page.rec:
        print(f"cfg5 rec batch {len(idx)}x{bw}", flush=True)
        pairs_ref = onets.run_graph(g, x)[-1]
        for b, i in enumerate(idx):
            assert (_ids(got[i]) == _ids(pairs_ref[b])).all(), f"line {i}"
            assert_bitexact(got[i][..., 0], pairs_ref[b][..., 0], f"line {i} values")
            t_valid = int(widths[i]) // pipeline.REC_STRIDE
            ref_ids, ref_conf = oracle.ctc_collapse(pairs_ref[b][:t_valid], t_valid)
            assert decoded[i][0] == [int(v) for v in ref_ids], f"line {i} ids"
            assert np.float32(decoded[i][1]) == np.float32(ref_conf)
    page.close()


def test_cfg5_mixed_page_fused_head(gpu, oracle):
    """The mixed page with fused rec heads (the benchmarked form): every
    batch's pairs under the pairs tolerance rule against the oracle's full graph,
    and the decoded lines equal to the oracle's wherever no id changed."""
    from conftest import pairs_tolerance_check
    from qppocr_amd import pipeline
    from oracle import nets as onets
    det_g, det_x, rw, lines, widths = pipeline.mixed_page(4, 1536, 128)
    print("cfg5 fused heads: det 1536^2 + 128 lines", flush=True)
    page = pipeline.PageRunner(det_g, det_x, rw, lines, widths, fused_head=True)
    page.upload()
    page.run()
    page.sync()
    got = page.rec_pairs()
    decoded = page.decode()
    for bw, idx, g, _, x in page.rec:
        print(f"cfg5 fused rec batch {len(idx)}x{bw}", flush=True)
        outs, T = onets.run_graph(g, x, keep=True)
        pairs_ref, logits = outs[-1], T[g.nodes[-2]["out"]]
        mine = np.stack([got[i] for i in idx])
        changed = pairs_tolerance_check(mine, pairs_ref, logits)
        for b, i in enumerate(idx):
            if (_ids(got[i]) == _ids(pairs_ref[b])).all():
                t_valid = int(widths[i]) // pipeline.REC_STRIDE
                ref_ids, _ = oracle.ctc_collapse(pairs_ref[b][:t_valid], t_valid)
                assert decoded[i][0] == [int(v) for v in ref_ids], f"line {i} ids"
        print(f"  steps with a near-tie id change: {changed}", flush=True)
    page.close()


def test_session_fusion_rules(gpu, oracle):
    """The session fuses a depthwise conv into the following 1x1 conv only
    when nothing else reads the intermediate: here one block's intermediate
    is also a graph output (kept separate), the next block is fused, and
    four independent 3x3 convs share one launch; everything bit-exact."""
    from qppocr_amd import nets
    from oracle import nets as onets
    r = nets.WeightRng(11)
    g = nets.Graph((2, 16, 24, 40))
    wd = g.weight(r.kaiming((16, 1, 3, 3), 9))
    bd = g.weight(r.normal((16,), 0.1))
    t1 = g.conv(0, wd, bd, pad=(1, 1, 1, 1), group=16, act=nets.ACT_HARDSWISH)
    wp = g.weight(r.kaiming((32, 16, 1, 1), 16))
    bp = g.weight(r.normal((32,), 0.1))
    y1 = g.conv(t1, wp, bp, act=nets.ACT_HARDSWISH)
    wd2 = g.weight(r.kaiming((32, 1, 5, 5), 25))
    bd2 = g.weight(r.normal((32,), 0.1))
    t2 = g.conv(y1, wd2, bd2, stride=(2, 2), pad=(2, 2, 2, 2), group=32, act=nets.ACT_HARDSWISH)
    wp2 = g.weight(r.kaiming((48, 32, 1, 1), 32))
    bp2 = g.weight(r.normal((48,), 0.1))
    y2 = g.conv(t2, wp2, bp2, act=nets.ACT_HARDSWISH)
    outs = [t1, y2]
    for k in range(4):
        w3 = g.weight(r.kaiming((8, 48, 3, 3), 48 * 9))
        b3 = g.weight(r.normal((8,), 0.1))
        outs.append(g.conv(y2, w3, b3, pad=(1, 1, 1, 1), act=nets.ACT_RELU))
    g.outputs = outs
    x = r.normal((2, 16, 24, 40), 1.0)
    sess = nets.HipSession(g)
    got = sess.run(x)
    ref = onets.run_graph(g, x)
    for i, (a, b) in enumerate(zip(got, ref)):
        assert_bitexact(a, b, f"output {i}")
    sess.close()


CONVT_CASES = [
    # batch, c, h, w, conv activation, conv output also a graph output, fused
    (1, 96, 40, 64, "relu", False, True),    # the det head's shape, 12 chunks of 8 channels
    (2, 8, 13, 20, "relu", False, True),     # one chunk, odd rows, a partial 32-column tile
    (1, 16, 9, 44, "none", False, True),     # two chunks, no activation
    (3, 24, 6, 36, "relu", False, True),     # three chunks
    (1, 32, 10, 12, "relu", True, False),    # the conv output is read twice: two launches
    (2, 40, 7, 18, "relu", False, False),    # width not a multiple of 4: the plain conv path
]


@pytest.mark.parametrize("case", CONVT_CASES, ids=lambda c: "x".join(map(str, c[:4])) + f"-{c[4]}{c[5]}")
def test_session_conv_convt_pair(gpu, oracle, case):
    """The det head (3x3 conv to 24 channels, ReLU, then ConvTranspose 2x2
    24 -> 24, ConvTranspose 2x2 24 -> 1, Sigmoid; DBHead as the det graph
    holds it) runs as one launch when only the pair reads the conv output:
    bit-exact against the oracle's conv, ConvT, ConvT and sigmoid, and, with
    real_n below the batch, the oracle's bits for the real items."""
    from qppocr_amd import nets
    from oracle import nets as onets
    n, c, h, w, act, shared, fused = case
    r = nets.WeightRng(17)
    g = nets.Graph((n, c, h, w))
    wc = g.weight(r.kaiming((24, c, 3, 3), 9 * c))
    bc = g.weight(r.normal((24,), 0.1))
    kind = nets.ACT_RELU if act == "relu" else nets.ACT_NONE
    t = g.conv(0, wc, bc, pad=(1, 1, 1, 1), act=kind)
    w1 = g.weight(r.kaiming((24, 24, 2, 2), 24))
    w2 = g.weight(r.kaiming((24, 1, 2, 2), 24))
    y = g.convt_pair_sigmoid(t, w1, w2)
    g.outputs = [y, t] if shared else [y]
    x = r.normal((n, c, h, w), 1.0)
    print(f"conv + ConvT pair {case}", flush=True)
    sess = nets.HipSession(g)
    launches = sess.plan()
    assert ((0, 2, 1) in launches) == fused, launches
    got = sess.run(x)
    ref = onets.run_graph(g, x)
    for i, (a, b) in enumerate(zip(got, ref)):
        assert_bitexact(a, b, f"output {i}")
    if n > 1:
        x1 = r.normal((1, c, h, w), 1.0)
        got1 = sess.run(x1)[0]
        g1 = nets.Graph((1, c, h, w))
        for arr in g.weights:
            g1.weight(arr)
        t1 = g1.conv(0, wc, bc, pad=(1, 1, 1, 1), act=kind)
        g1.outputs = [g1.convt_pair_sigmoid(t1, w1, w2)]
        assert_bitexact(got1, onets.run_graph(g1, x1)[0], "real_n 1")
    sess.close()


FPN_CASES = [
    # batch, level-2 side (h, w), channels of C2..C5, M, a lateral with ReLU (not fused)
    (1, (32, 40), (16, 32, 48, 64), 32, False),
    (2, (16, 32), (32, 64, 128, 256), 96, False),
    (1, (32, 40), (16, 32, 48, 64), 32, True),
]


@pytest.mark.parametrize("case", FPN_CASES, ids=lambda c: f"n{c[0]}-{c[1][0]}x{c[1][1]}-m{c[3]}-{int(c[4])}")
def test_session_fpn_laterals(gpu, oracle, case):
    """The det FPN's four 1x1 laterals with their nearest-2x top-down Adds
    (L5 = conv(C5), Lk = conv(Ck) + up2(Lk+1)) run as the grouped coarse
    GEMMs, the top-down pass and the fine lateral: one plan entry of four
    nodes and three kernels; every level bit-exact against the oracle, and
    with real_n 1 on a batch of 2 the oracle's one-item bits."""
    from qppocr_amd import nets
    from qppocr_amd._lib import ACT_RELU
    from oracle import nets as onets
    n, (h, w), cs, m, relu = case

    def build(batch, r):
        g = nets.Graph((batch, cs[0], h, w))
        feats = [0]
        for k in range(1, 4):
            wc = g.weight(r.kaiming((cs[k], cs[k - 1], 3, 3), 9 * cs[k - 1]))
            bc = g.weight(r.normal((cs[k],), 0.1))
            feats.append(g.conv(feats[-1], wc, bc, stride=(2, 2), pad=(1, 1, 1, 1)))
        lat = -1
        outs = []
        for k in (3, 2, 1, 0):
            wl = g.weight(r.kaiming((m, cs[k], 1, 1), cs[k]))
            bl = g.weight(r.normal((m,), 0.1))
            act = ACT_RELU if (relu and k == 1) else nets.ACT_NONE
            lat = g.conv(feats[k], wl, bl, residual=lat, res_up=2 if lat >= 0 else 0, act=act)
            outs.append(lat)
        g.outputs = outs
        return g

    g = build(n, nets.WeightRng(31))
    x = nets.WeightRng(32).normal((n, cs[0], h, w), 1.0)
    print(f"fpn laterals {case}", flush=True)
    sess = nets.HipSession(g)
    assert ((3, 4, 3) in sess.plan()) == (not relu), sess.plan()
    got = sess.run(x)
    ref = onets.run_graph(g, x)
    for lvl, (a, b) in enumerate(zip(got, ref)):
        assert_bitexact(a, b, f"level {5 - lvl}")
    if n > 1:
        got1 = sess.run(x[:1])
        ref1 = onets.run_graph(build(1, nets.WeightRng(31)), x[:1])
        for lvl, (a, b) in enumerate(zip(got1, ref1)):
            assert_bitexact(a, b, f"real_n 1 level {5 - lvl}")
    sess.close()


LINEAR_CASES = [
    # rows, k, n, layernorm in front, activation, residual, LN output also an output
    (1280, 256, 768, True, "none", False, False),   # rec QKV: 4 slabs
    (1280, 1024, 256, False, "none", True, False),  # rec MLP down: 16 slabs + residual
    (1280, 256, 1024, True, "gelu", False, False),  # rec MLP up + GELU
    (70, 64, 40, False, "gelu", True, False),        # ragged rows / columns, 1 slab
    (33, 192, 96, True, "none", True, False),        # 3 slabs, run-time slab loop
    (64, 128, 200, True, "none", False, True),       # 2 slabs
    (50, 320, 64, True, "gelu", False, False),       # 5 slabs
    (96, 448, 37, False, "none", True, False),       # 7 slabs, odd N
    (70, 64, 40, True, "none", False, False),        # 1 slab, ragged rows
    (40, 128, 96, True, "gelu", True, False),        # 2 slabs
]


@pytest.mark.parametrize("case", LINEAR_CASES, ids=lambda c: "x".join(map(str, c[:3])) + f"-{c[3]}{c[4]}{c[5]}{c[6]}")
def test_session_linear_shapes(gpu, oracle, case):
    """Session linears below the 128x128 size run over a transposed resident
    weight (linear_nt_kernel): ragged rows and columns, 1..16 slabs of 64
    (compile-time and run-time slab loops), GELU and residual epilogues,
    after a LayerNorm or not; bit-exact against the oracle."""
    from qppocr_amd import nets
    from oracle import nets as onets
    rows, k, n, ln, act, res, ln_out = case
    r = nets.WeightRng(rows * 7 + k + n)
    g = nets.Graph((1, rows, k))
    x = 0
    outs = []
    if ln:
        gam = g.weight((1.0 + r.normal((k,), 0.1)).astype(np.float32))
        bet = g.weight(r.normal((k,), 0.1))
        x = g.layernorm(0, gam, bet, nets.LN_EPS)
        if ln_out:
            outs.append(x)
    resid = -1
    if res:
        w0 = g.weight(r.kaiming((k, n), k))
        b0 = g.weight(r.normal((n,), 0.1))
        resid = g.linear(0, w0, b0)
        outs.append(resid)
    w = g.weight(r.kaiming((k, n), k))
    b = g.weight(r.normal((n,), 0.1))
    y = g.linear(x, w, b, act=nets.ACT_GELU if act == "gelu" else nets.ACT_NONE, residual=resid)
    g.outputs = outs + [y]
    xin = r.normal((1, rows, k), 1.0)
    sess = nets.HipSession(g)
    got = sess.run(xin)
    ref = onets.run_graph(g, xin)
    for i, (a, bb) in enumerate(zip(got, ref)):
        assert_bitexact(a, bb, f"output {i}")
    sess.close()


QKV_ATTN_CASES = [
    # batch, T, K, heads, bias
    (2, 40, 256, 8, True),    # the rec encoder's shape (one launch for both nodes)
    (3, 64, 128, 4, True),    # 64 rows: four 16-row blocks, three output blocks a wave
    (1, 12, 64, 2, False),    # one K slab, one row block, no bias
    (2, 36, 192, 8, True),    # three slabs, partial last row block
    (2, 30, 256, 8, True),    # T % 4 != 0: the linear and the attention apart
    (1, 40, 320, 8, True),    # K = 320: the linear and the attention apart
]


@pytest.mark.parametrize("case", QKV_ATTN_CASES, ids=lambda c: "x".join(map(str, c[:4])) + ("b" if c[4] else ""))
def test_session_qkv_attention(gpu, oracle, case):
    """A linear read only by the attention after it (head dimension 32,
    T <= 64, T % 4 == 0, K a multiple of 64 up to 256) runs with it as one
    launch, the QKV tensor never stored; other shapes run the two nodes
    apart.  Bit-exact against the oracle either way."""
    from qppocr_amd import _lib, nets
    from oracle import nets as onets
    b, t, k, heads, has_b = case
    dh = 32
    r = nets.WeightRng(b * 1000 + t * 10 + k + heads)
    g = nets.Graph((b, t, k))
    w = g.weight(r.kaiming((k, 3 * heads * dh), k))
    bias = g.weight(r.normal((3 * heads * dh,), 0.1)) if has_b else -1
    qkv = g.linear(0, w, bias)
    o = g.attention(qkv, heads, dh, 1.0 / math.sqrt(dh))
    g.outputs = [o]
    x = r.normal((b, t, k), 1.0)
    print(f"qkv + attention {case}", flush=True)
    sess = nets.HipSession(g)
    got = sess.run(x)
    ref = onets.run_graph(g, x)
    assert_bitexact(got[0], ref[0], "attention output")
    fused = t % 4 == 0 and k <= 256
    assert (sess.plan()[0][1] == 2) == fused
    if fused:   # the QKV tensor has no storage to hand out
        with pytest.raises(_lib.QphError, match="never stored"):
            sess.tensor_ptr(qkv)
    else:
        assert sess.tensor_ptr(qkv)[1] == b * t * 3 * heads * dh
    sess.close()


def test_session_layernorm_linear_sequential_rows(gpu, oracle):
    """LayerNorm (K = 256) then a linear: rows with a huge cancelling pair
    (+-1e15, +-1e18) make the shuffle-tree f64 sums of the mean unprovable,
    so those rows take the sequential sum; a constant row and a
    large-offset row beside ordinary ones; bit-exact against the oracle."""
    from qppocr_amd import nets
    from oracle import nets as onets
    r = nets.WeightRng(41)
    rows, k, n = 96, 256, 64
    g = nets.Graph((1, rows, k))
    gam = g.weight((1.0 + r.normal((k,), 0.1)).astype(np.float32))
    bet = g.weight(r.normal((k,), 0.1))
    x = g.layernorm(0, gam, bet, nets.LN_EPS)
    w = g.weight(r.kaiming((k, n), k))
    b = g.weight(r.normal((n,), 0.1))
    y = g.linear(x, w, b)
    g.outputs = [y]
    xin = r.normal((1, rows, k), 1.0)
    xin[0, 3, 7], xin[0, 3, 200] = 1e15, -1e15
    xin[0, 17, 0], xin[0, 17, 255] = -1e18, 1e18
    xin[0, 40, :] = 1e7 + r.normal((k,), 1e-3)
    xin[0, 41, :] = 3.0
    sess = nets.HipSession(g)
    got = sess.run(xin)
    ref = onets.run_graph(g, xin)
    assert_bitexact(got[0], ref[0], "layernorm + linear")
    sess.close()


STEM_CASES = [
    # n, h, w, stem channels, pw channels, activations (stem, dw, pw), stem bias, stem output read elsewhere
    (2, 30, 50, 16, 24, ("relu", "none", "relu"), False, False),   # odd sizes, generic activations
    (1, 48, 100, 32, 64, ("hs", "hs", "hs"), True, False),         # rec-like, partial last tile
    (1, 48, 100, 32, 64, ("hs", "hs", "hs"), True, True),          # stem output also an output: not fused
    (3, 7, 9, 16, 16, ("hs", "hs", "hs"), True, False),            # tiny maps
    (1, 44, 64, 32, 64, ("hs", "hs", "hs"), True, False),          # odd output height: a tile's second row past the map
    (2, 42, 70, 16, 32, ("relu", "hs", "relu"), True, False),      # odd output height, width % 4 != 0 (one-word loads)
    # enough workgroups that one-row tiles would not all be resident: two output rows a workgroup
    (32, 44, 300, 32, 64, ("hs", "hs", "hs"), True, False),        # rec-like, odd output height, partial tiles
    (16, 64, 640, 16, 32, ("hs", "hs", "hs"), True, False),        # det-like, 16 stem channels
]


@pytest.mark.parametrize("case", STEM_CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}-{c[3]}-{c[4]}-{c[5][0]}-{c[6]}{c[7]}")
def test_session_stem_fusion(gpu, oracle, case):
    """A 3-channel 3x3 stride-2 stem conv in front of a 3x3 stride-2
    depthwise + 1x1 block runs inside the block's launch (its output
    computed in LDS, never stored) unless something else reads it: odd
    map sizes, partial tiles, no stem bias, generic and hardswish
    activations; bit-exact against the oracle."""
    from qppocr_amd import nets
    from oracle import nets as onets
    n, h, w, cs, m, acts, sbias, shared = case
    kind = {"relu": nets.ACT_RELU, "none": nets.ACT_NONE, "hs": nets.ACT_HARDSWISH}
    r = nets.WeightRng(n * 131 + h * 7 + w + cs + m)
    g = nets.Graph((n, 3, h, w))
    ws = g.weight(r.kaiming((cs, 3, 3, 3), 27))
    bs = g.weight(r.normal((cs,), 0.1)) if sbias else -1
    s0 = g.conv(0, ws, bs, stride=(2, 2), pad=(1, 1, 1, 1), act=kind[acts[0]])
    wd = g.weight(r.kaiming((cs, 1, 3, 3), 9))
    bd = g.weight(r.normal((cs,), 0.1))
    t = g.conv(s0, wd, bd, stride=(2, 2), pad=(1, 1, 1, 1), group=cs, act=kind[acts[1]])
    wp = g.weight(r.kaiming((m, cs, 1, 1), cs))
    bp = g.weight(r.normal((m,), 0.1))
    y = g.conv(t, wp, bp, act=kind[acts[2]])
    g.outputs = [s0, y] if shared else [y]
    x = r.normal((n, 3, h, w), 1.0)
    sess = nets.HipSession(g)
    got = sess.run(x)
    ref = onets.run_graph(g, x)
    for i, (a, b) in enumerate(zip(got, ref)):
        assert_bitexact(a, b, f"output {i}")
    sess.close()


BLOCK_CASES = [
    # n, c, h, w, depthwise kernel, stride, pad, pointwise channels, activation
    (1, 128, 40, 40, 3, 1, 1, 128, "hs"),   # det block 7: 16-byte loads, 8 px a task
    (1, 128, 40, 40, 5, 1, 2, 128, "hs"),   # det block 9: 5x5
    (1, 128, 40, 40, 3, 2, 1, 256, "hs"),   # det block 12: stride 2, four 64-channel slices
    (2, 64, 23, 44, 3, 1, 1, 96, "hs"),     # partial tiles and slice, odd height
    (1, 32, 30, 36, 3, 2, 1, 64, "hs"),     # stride 2, 2 px a task, partial tile
    (1, 16, 17, 20, 3, 1, 1, 32, "relu"),   # register-fed, C = 16, generic activations
    (1, 16, 17, 22, 3, 1, 1, 32, "relu"),   # width % 4 != 0: one-word loads, 1 px a task
    (1, 64, 24, 48, 5, 1, 2, 64, "hs"),     # 5x5, 4 px a task
    (1, 64, 20, 42, 3, 1, 1, 64, "hs"),     # width % 4 != 0: one-word loads
    (1, 30, 20, 40, 3, 1, 1, 40, "hs"),     # channels % 4 != 0: one-word loads
    (1, 32, 20, 40, 3, 1, 0, 32, "hs"),     # no padding: one-word loads
    (1, 32, 40, 64, 3, 1, 1, 32, "relu"),   # register-fed form, generic activations
    (1, 64, 26, 36, 3, 2, 1, 128, "hs"),    # register-fed, stride 2, partial tile (18 wide)
    (1, 64, 24, 48, 5, 2, 2, 64, "hs"),     # 5x5 stride 2: depthwise and 1x1 as two launches
]


@pytest.mark.parametrize("case", BLOCK_CASES, ids=lambda c: "-".join(map(str, c)))
def test_session_block_paths(gpu, oracle, case):
    """Depthwise + 1x1 blocks fused into one launch: the register-fed form
    (C = 32, 64, 128 on the 16-byte path) and both halo load paths of the
    LDS form (16-byte chunks when the width and channel count are multiples
    of 4 and the padding is k // 2; one-word loads otherwise), 1 to 8
    pixels a depthwise task, 3x3 and 5x5, strides 1 and 2, partial tiles
    and channel slices, and a 5x5 stride-2 pair (not fused); bit-exact
    against the oracle."""
    from qppocr_amd import nets
    from oracle import nets as onets
    n, c, h, w, k, st, pad, m, act = case
    kind = nets.ACT_RELU if act == "relu" else nets.ACT_HARDSWISH
    r = nets.WeightRng(n * 17 + c * 5 + h + w + k + m)
    g = nets.Graph((n, c, h, w))
    wd = g.weight(r.kaiming((c, 1, k, k), k * k))
    bd = g.weight(r.normal((c,), 0.1))
    t = g.conv(0, wd, bd, stride=(st, st), pad=(pad,) * 4, group=c, act=kind)
    wp = g.weight(r.kaiming((m, c, 1, 1), c))
    bp = g.weight(r.normal((m,), 0.1))
    y = g.conv(t, wp, bp, act=kind)
    g.outputs = [y]
    x = r.uniform((n, c, h, w), -1.0, 1.0)
    print(f"block {case}", flush=True)
    sess = nets.HipSession(g)
    got = sess.run(x)
    ref = onets.run_graph(g, x)
    assert_bitexact(got[0], ref[0], "block output")
    sess.close()


@pytest.mark.parametrize("m", [64, 30])
def test_session_block_channel_last_out(gpu, oracle, m):
    """A register-fed depthwise + 1x1 block (C = 64, 16-byte path) whose 1x1
    conv stores channel-last: 16-byte stores of four channels when M % 4 == 0,
    one word a channel otherwise; bit-exact against the oracle."""
    from qppocr_amd import nets
    from oracle import nets as onets
    r = nets.WeightRng(41 + m)
    g = nets.Graph((2, 64, 20, 40))
    wd = g.weight(r.kaiming((64, 1, 3, 3), 9))
    bd = g.weight(r.normal((64,), 0.1))
    t = g.conv(0, wd, bd, stride=(1, 1), pad=(1, 1, 1, 1), group=64, act=nets.ACT_HARDSWISH)
    wp = g.weight(r.kaiming((m, 64, 1, 1), 64))
    bp = g.weight(r.normal((m,), 0.1))
    y = g.conv(t, wp, bp, act=nets.ACT_HARDSWISH, trans_out=True)
    g.outputs = [y]
    x = r.uniform((2, 64, 20, 40), -1.0, 1.0)
    sess = nets.HipSession(g)
    got = sess.run(x)
    ref = onets.run_graph(g, x)
    assert_bitexact(got[0], ref[0], "channel-last block output")
    sess.close()


def test_session_channel_last_chain_px(gpu, oracle):
    """Channel-last depthwise with four outputs per thread: x-stride 2 and 1
    at odd output widths (19), and a ReLU depthwise (the generic activation
    path next to the inline HardSigmoid + Mul); bit-exact against the
    oracle."""
    from qppocr_amd import nets
    from oracle import nets as onets
    r = nets.WeightRng(29)
    g = nets.Graph((3, 3, 20, 75))
    ws = g.weight(r.kaiming((32, 3, 3, 3), 27))
    bs = g.weight(r.normal((32,), 0.1))
    x = g.conv(0, ws, bs, stride=(2, 2), pad=(1, 1, 1, 1), act=nets.ACT_HARDSWISH)
    blocks = [  # (dw stride, dw activation, cin, cout)
        ((1, 1), nets.ACT_HARDSWISH, 32, 64), ((2, 2), nets.ACT_HARDSWISH, 64, 128),
        ((1, 1), nets.ACT_RELU, 128, 128),
    ]
    for i, (st, act, cin, cout) in enumerate(blocks):
        wd = g.weight(r.kaiming((cin, 1, 3, 3), 9))
        bd = g.weight(r.normal((cin,), 0.1))
        x = g.conv(x, wd, bd, stride=st, pad=(1, 1, 1, 1), group=cin, act=act)
        wp = g.weight(r.kaiming((cout, cin, 1, 1), cin))
        bp = g.weight(r.normal((cout,), 0.1))
        x = g.conv(x, wp, bp, act=nets.ACT_HARDSWISH, trans_out=i == len(blocks) - 1)
    g.outputs = [x]
    xin = r.uniform((3, 3, 20, 75), -1.0, 1.0)
    sess = nets.HipSession(g)
    got = sess.run(xin)
    ref = onets.run_graph(g, xin)
    assert_bitexact(got[0], ref[0], "chain output")
    sess.close()


def test_session_channel_last_blocks_wide(gpu, oracle):
    """Channel-last depthwise + 1x1 blocks over wide rows (105 and 53
    columns), C = 64, 128, 256, x-stride 2 at C = 128, and a ReLU depthwise
    next to the inline HardSigmoid + Mul; bit-exact against the oracle."""
    from qppocr_amd import nets
    from oracle import nets as onets
    r = nets.WeightRng(53)
    g = nets.Graph((2, 3, 16, 420))
    ws = g.weight(r.kaiming((32, 3, 3, 3), 27))
    bs = g.weight(r.normal((32,), 0.1))
    x = g.conv(0, ws, bs, stride=(2, 2), pad=(1, 1, 1, 1), act=nets.ACT_HARDSWISH)
    blocks = [  # (dw stride, dw activation, cin, cout)
        ((1, 1), nets.ACT_HARDSWISH, 32, 64), ((2, 2), nets.ACT_HARDSWISH, 64, 128),
        ((1, 2), nets.ACT_RELU, 128, 256), ((1, 1), nets.ACT_HARDSWISH, 256, 256),
    ]
    for i, (st, act, cin, cout) in enumerate(blocks):
        wd = g.weight(r.kaiming((cin, 1, 3, 3), 9))
        bd = g.weight(r.normal((cin,), 0.1))
        x = g.conv(x, wd, bd, stride=st, pad=(1, 1, 1, 1), group=cin, act=act)
        wp = g.weight(r.kaiming((cout, cin, 1, 1), cin))
        bp = g.weight(r.normal((cout,), 0.1))
        x = g.conv(x, wp, bp, act=nets.ACT_HARDSWISH, trans_out=i == len(blocks) - 1)
    g.outputs = [x]
    xin = r.uniform((2, 3, 16, 420), -1.0, 1.0)
    sess = nets.HipSession(g)
    got = sess.run(xin)
    ref = onets.run_graph(g, xin)
    assert_bitexact(got[0], ref[0], "chain output")
    sess.close()


def test_session_channel_last_chain(gpu, oracle):
    """A chain of depthwise -> 1x1 blocks ending in a 1x1 conv that stores
    [n][pixels][M] runs channel-last (depthwise_cl_kernel + the 1x1 convs as
    row-major GEMMs) from the first block whose 1x1 conv has C % 64 == 0;
    the block before it (C = 32) stays fused and stores channel-last.
    Strides (2,2), (2,1), (3,1), a 5x5 depthwise and an odd width; bit-exact
    against the oracle."""
    from qppocr_amd import nets
    from oracle import nets as onets
    r = nets.WeightRng(23)
    g = nets.Graph((2, 3, 24, 41))
    ws = g.weight(r.kaiming((32, 3, 3, 3), 27))
    bs = g.weight(r.normal((32,), 0.1))
    x = g.conv(0, ws, bs, stride=(2, 2), pad=(1, 1, 1, 1), act=nets.ACT_HARDSWISH)
    blocks = [  # (dw kernel, stride, pad, cin, cout)
        (3, (1, 1), (1, 1, 1, 1), 32, 64), (3, (2, 1), (1, 1, 1, 1), 64, 128),
        (5, (1, 1), (2, 2, 2, 2), 128, 64), (3, (3, 1), (0, 1, 0, 1), 64, 128),
    ]
    for i, (k, st, pad, cin, cout) in enumerate(blocks):
        wd = g.weight(r.kaiming((cin, 1, k, k), k * k))
        bd = g.weight(r.normal((cin,), 0.1))
        x = g.conv(x, wd, bd, stride=st, pad=pad, group=cin, act=nets.ACT_HARDSWISH)
        wp = g.weight(r.kaiming((cout, cin, 1, 1), cin))
        bp = g.weight(r.normal((cout,), 0.1))
        x = g.conv(x, wp, bp, act=nets.ACT_HARDSWISH, trans_out=i == len(blocks) - 1)
    g.outputs = [x]
    xin = r.uniform((2, 3, 24, 41), -1.0, 1.0)
    sess = nets.HipSession(g)
    got = sess.run(xin)
    ref = onets.run_graph(g, xin)
    assert_bitexact(got[0], ref[0], "chain output")
    sess.close()
