"""The plan-model host side without a GPU: the nhwc.rs weight layouts, the
plan writer's dispatch lists and parameter blocks for the det and rec
graphs, and the HIP kernel set's name table."""
import numpy as np
import pytest

from qppocr_amd import nets, plan

# parameter block length per kernel (the n_*.comp layouts, plan.rs)
PARAM_WORDS = {"n_entry": 7, "n_exit": 8, "n_exit3": 6, "n_exit3_argmax": 6, "n_elem": 7,
               "n_channel": 10, "n_conv": 21, "n_conv8": 21, "n_conv_dw": 20, "n_convt": 18,
               "n_pool": 14, "n_reduce_hw": 4, "n_reduce_fin": 5, "n_reduce_last": 6,
               "n_resize": 9, "n_transpose": 4, "n_transpose_nd": 14, "n_softmax": 6,
               "n_attn_mm": 8}


def f32(words):
    return np.asarray(words, np.uint32).view(np.float32)


def test_repack_conv_w_layout():
    """nhwc.rs:28-57: element (((t * cin4v + ci4) * 4 + ci % 4) * nv + n4) * 4 + l
    holds w[n4 * 4 + l, ci, ky, kx]; channels past the real ones are 0."""
    r = np.random.default_rng(0)
    co, cin, kh, kw = 6, 5, 3, 2
    w = r.standard_normal((co, cin, kh, kw)).astype(np.float32)
    v = f32(plan.repack_conv_w(w, co, cin, kh, kw))
    cin4v, nv = 2, 2
    assert v.size == kh * kw * cin4v * 4 * nv * 4
    for t in range(kh * kw):
        ky, kx = divmod(t, kw)
        for ci in range(8):
            for o in range(8):
                idx = (((t * cin4v + ci // 4) * 4 + ci % 4) * nv + o // 4) * 4 + o % 4
                want = w[o, ci, ky, kx] if (ci < cin and o < co) else 0.0
                assert v[idx] == want


def test_repack_dw_and_convt_layouts():
    r = np.random.default_rng(1)
    c, kh, kw = 7, 3, 3
    w = r.standard_normal((c, 1, kh, kw)).astype(np.float32)
    v = f32(plan.repack_dw_w(w, c, kh, kw))
    for t in range(9):
        for ch in range(8):
            want = w[ch, 0, t // 3, t % 3] if ch < c else 0.0
            assert v[(t * 2 + ch // 4) * 4 + ch % 4] == want     # nhwc.rs:161-179
    ci, co = 5, 3
    wt = r.standard_normal((ci, co, 2, 2)).astype(np.float32)
    v = f32(plan.repack_convt_w(wt, ci, co, 2, 2))
    for t in range(4):
        for i in range(8):
            for o in range(4):
                want = wt[i, o, t // 2, t % 2] if (i < ci and o < co) else 0.0
                assert v[((t * 8 + i) * 1 + o // 4) * 4 + o % 4] == want   # nhwc.rs:181-202
    b = f32(plan.conv_bias(np.arange(5, dtype=np.float32), 5))
    assert b.tolist() == [0, 1, 2, 3, 4, 0, 0, 0]


def test_matmul_weight_repack_is_k_major():
    """A MatMul's constant B [K, N] goes through repack_conv_w of B^T as a
    1x1 conv (plan.rs:1905-1925): word k * cpad4(N) + j = B[k, j], which is
    the row-major [K, Npad] operand the GEMM reads."""
    r = np.random.default_rng(2)
    k, n = 6, 10
    b = r.standard_normal((k, n)).astype(np.float32)
    v = f32(plan.repack_conv_w(b.T, n, k, 1, 1)).reshape(8, 12)
    assert np.array_equal(v[:k, :n], b)
    assert not v[k:].any() and not v[:, n:].any()


def _check_plan(pl):
    """Every parameter block has its kernel's length and names regions in
    the arena; uploads do not overlap; word 0 is real_n."""
    spans = sorted((off, off + w.size) for off, w in pl.uploads)
    assert spans[0] == (0, 1)
    for (a0, a1), (b0, _) in zip(spans, spans[1:]):
        assert a1 <= b0
    assert spans[-1][1] <= pl.total_words
    for i, (name, p_off, groups, _) in enumerate(pl.dispatches):
        w = pl.params_of(i)
        if name == "n_concat_c":
            assert w.size == 4 + 2 * int(w[2])
        else:
            assert w.size == PARAM_WORDS[name], name
        assert groups[1] >= 1 and groups[0] >= 1
    for off, numel, shape in pl.outputs:
        assert off + numel <= pl.total_words and numel == int(np.prod(shape))


def test_det_plan_structure():
    g, _ = nets.build_det(2, 96, 64)
    pl = plan.build_plan(g)
    _check_plan(pl)
    names = [d[0] for d in pl.dispatches]
    assert names[0] == "n_entry" and names[-1] == "n_exit"
    assert names.count("n_convt") == 2 and names.count("n_concat_c") == 1
    # the det output's Sigmoid runs in the exit (act 4)
    assert pl.params_of(len(names) - 1)[7] == 4
    convs = [i for i, n in enumerate(names) if n in ("n_conv", "n_conv8", "n_conv_dw")]
    assert len(convs) == sum(1 for d in g.nodes if d["op"] == nets.OP_CONV)


def test_rec_plan_structure():
    g, _ = nets.build_rec(3, 2, 160, probs=False)
    pl = plan.build_plan(g)
    _check_plan(pl)
    names = [d[0] for d in pl.dispatches]
    assert names[-1] == "n_exit3_argmax"
    assert names.count("n_reduce_last") == 8          # two LayerNorms per layer, two layers
    assert names.count("n_attn_mm") == 4 and names.count("n_softmax") == 3
    # the head: MatMul over 2 * 20 rows into cpad4(18709) columns, bias as n_channel 1
    head = max(i for i, n in enumerate(names) if n == "n_conv8")
    w = pl.params_of(head)
    assert (w[4], w[5], w[9]) == (40, 18712, 64)
    assert names[head + 1] == "n_channel" and pl.params_of(head + 1)[0] == 1


@pytest.fixture(scope="module")
def lib():
    from qppocr_amd import _lib
    return _lib.load()


def test_kernel_set_names(lib):
    """Every kernel the Vulkan backend registers has an id; the Metal-only
    variants are refused (vulkan/pipeline.rs:84-136)."""
    ids = [lib.qph_plan_kernel_id(n.encode()) for n in PARAM_WORDS] + \
          [lib.qph_plan_kernel_id(b"n_concat_c")]
    assert all(i >= 0 for i in ids) and len(set(ids)) == len(ids) == 20
    for n in (b"n_conv8_mma", b"n_conv8h", b"n_head_argmax", b"n_convt4w", b"n_conv_dw_tile"):
        assert lib.qph_plan_kernel_id(n) < 0


# ------------------------------------------------------ host-side validation

class _Plan:
    """A small hand-built GraphPlan (word 0 = real_n, a 4-word input)."""

    def __init__(self):
        self.p = plan.GraphPlan()
        self.words = 0
        self.static(np.array([0], np.uint32))
        self.p.in_f32_off = self.alloc(4)
        self.p.in_shape = (4,)

    def alloc(self, n):
        off = self.words
        self.words += max(4, (int(n) + 3) // 4 * 4)
        return off

    def static(self, w):
        w = np.ascontiguousarray(w, np.uint32).reshape(-1)
        off = self.alloc(w.size)
        self.p.uploads.append((off, w))
        return off

    def dispatch(self, kernel, params, groups=(1, 1, 1)):
        pw = np.array([v if isinstance(v, (int, np.integer)) else plan.f32_bits(v) for v in params],
                      np.uint32)
        self.p.dispatches.append((kernel, self.static(pw), tuple(groups), -1))

    def done(self, out_off, numel):
        self.p.outputs.append((out_off, int(numel), (int(numel),)))
        self.p.total_words = self.words
        return self.p


OFF_NONE = 0xFFFFFFFF


def test_validate_accepts_the_written_plans(lib):
    """qph_plan_validate (no context, no device) passes the det and rec plans
    the writer produces, the checks qph_plan_create runs first."""
    plan.validate_plan(plan.build_plan(nets.build_det(2, 96, 64)[0]))
    plan.validate_plan(plan.build_plan(nets.build_rec(3, 2, 160, probs=False)[0]))
    mp = _Plan()
    x = mp.alloc(16)
    mp.dispatch("n_elem", [0, x, OFF_NONE, x, 16, 0.0, 0.0])
    plan.validate_plan(mp.done(x, 16))


def test_validate_refuses_malformed_plans(lib):
    """Malformed plans are refused on the host, naming what is wrong: a
    region past the arena, a misaligned vec4 region, a parameter block that
    was never uploaded, an n_reduce_fin with no n_reduce_hw before it, an
    output or input outside the arena, overlapping uploads."""
    from qppocr_amd import _lib

    def refused(p, match):
        with pytest.raises(_lib.QphError, match=match):
            plan.validate_plan(p)

    mp = _Plan()
    x = mp.alloc(16)
    mp.dispatch("n_elem", [0, x, OFF_NONE, x + 1000, 16, 0.0, 0.0])
    refused(mp.done(x, 16), "outside the arena")
    mp = _Plan()
    x = mp.alloc(16)
    mp.dispatch("n_elem", [0, x + 1, OFF_NONE, x, 12, 0.0, 0.0])
    refused(mp.done(x, 16), "16-byte aligned")
    mp = _Plan()
    x = mp.alloc(16)
    mp.p.dispatches.append(("n_elem", mp.alloc(8), (1, 1, 1), -1))   # block never uploaded
    refused(mp.done(x, 16), "not uploaded")
    mp = _Plan()
    x = mp.alloc(16)
    mp.dispatch("n_reduce_fin", [x, x, 1, 4, 4])
    refused(mp.done(x, 4), "n_reduce_hw")
    mp = _Plan()
    x = mp.alloc(16)
    mp.dispatch("n_elem", [0, x, OFF_NONE, x, 16, 0.0, 0.0])
    p = mp.done(x, 16)
    p.outputs[0] = (p.total_words - 4, 16, (16,))
    refused(p, "output 0 is outside")
    mp = _Plan()
    x = mp.alloc(16)
    mp.dispatch("n_elem", [0, x, OFF_NONE, x, 16, 0.0, 0.0])
    p = mp.done(x, 16)
    p.in_f32_off = p.total_words - 2
    refused(p, "input region")
    mp = _Plan()
    x = mp.alloc(16)
    mp.dispatch("n_elem", [0, x, OFF_NONE, x, 16, 0.0, 0.0])
    p = mp.done(x, 16)
    p.uploads.append((p.uploads[-1][0] + 2, np.zeros(4, np.uint32)))
    refused(p, "overlap")
