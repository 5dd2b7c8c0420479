"""Host side of the page pipeline (no GPU): the CTC collapse of the (val, idx)
pairs (qppocr-core/src/pipeline/rec.rs:82-115) and the width bucketing of
the rec lines."""
import numpy as np


def test_ctc_decode_pairs_matches_oracle_collapse(oracle):
    """Host CTC collapse of the pipeline (rec.rs:82-115) against the oracle's
    C collapse on the same pairs, including masked lengths and all-blank rows."""
    from qppocr_amd.pipeline import ctc_decode_pairs
    rng = np.random.default_rng(9)
    for t_len, vocab in [(40, 5), (160, 3), (7, 1), (1, 2)]:
        vals = rng.random(t_len).astype(np.float32)
        idx = rng.integers(0, vocab, t_len).astype(np.uint32)
        pairs = np.stack([vals, idx.view(np.float32)], axis=1)
        for t_valid in sorted({t_len, max(1, t_len // 2), 1}):
            ids, conf = ctc_decode_pairs(pairs, t_valid)
            ref_ids, ref_conf = oracle.ctc_collapse(pairs[:t_valid], t_valid)
            assert ids == [int(v) for v in ref_ids]
            assert np.float32(conf) == np.float32(ref_conf)


def test_bucket_plan():
    from qppocr_amd.pipeline import bucket_plan
    widths = [80, 160, 161, 320, 1280, 87, 1279] + [400] * 70
    plan = bucket_plan(widths, 160, 64)
    seen = sorted(i for _, idx in plan for i in idx)
    assert seen == list(range(len(widths)))
    for bw, idx in plan:
        assert bw % 160 == 0 and 0 < len(idx) <= 64
        assert all(bw - 160 < widths[i] <= bw for i in idx)
    assert [len(idx) for bw, idx in plan if bw == 480] == [64, 6]


def test_engine_batches_follow_the_engine_grouping():
    """engine_batches restates the reference engine's rec grouping for a GPU
    session (qppocr-core/src/pipeline/engine.rs:1240-1290, 1413-1422): lines
    in width order, a group closed when it holds `chunk` lines or its next
    line is more than `grain` px wider than its first, batch width = widest
    line (at least 16) rounded up to the grain."""
    from qppocr_amd.pipeline import engine_batches
    widths = [300, 80, 100, 144, 145, 1280, 1216, 90, 80]
    b = engine_batches(widths, grain=64, chunk=64)
    # sorted: 80(1) 80(8) 90(7) 100(2) 144(3) | 145(4) 300(0) ... spans <= 64 from the first
    assert b[0] == (192, [1, 8, 7, 2, 3])     # 144 - 80 = 64 joins; 145 - 80 = 65 does not
    assert b[1] == (192, [4])                  # 145 -> 192; 300 - 145 > 64
    assert b[2] == (320, [0])
    assert b[3] == (1280, [6, 5])              # 1280 - 1216 = 64
    assert sum(len(i) for _, i in b) == len(widths)
    # the chunk limit cuts a long run of equal widths
    b = engine_batches([200] * 150, grain=64, chunk=64)
    assert [len(i) for _, i in b] == [64, 64, 22] and all(w == 256 for w, _ in b)
    # grain 1: raw widths, min width 16
    assert engine_batches([8, 33], grain=1, chunk=4) == [(16, [0]), (33, [1])]
    # every line once, widths multiples of 64, spans within the grain
    rng = np.random.default_rng(4)
    ws = rng.choice(np.arange(80, 1281, 8), size=128)
    b = engine_batches(ws)
    seen = sorted(i for _, idx in b for i in idx)
    assert seen == list(range(128))
    for w, idx in b:
        assert w % 64 == 0 and len(idx) <= 64
        assert max(ws[idx]) - min(ws[idx]) <= 64 and w >= max(ws[idx]) and w - max(ws[idx]) < 64


def test_rec_session_hooks():
    """The engine-facing rec session reports the reference GPU sessions'
    batching hooks (device.rs:139-165, vulkan/session.rs:2010-2033) and maps a
    batch to the net of its grain-padded size (nothing touches a GPU)."""
    from qppocr_amd.pipeline import HipRecSession
    s = HipRecSession(weights=None)
    assert not s.prefers_host_parallelism()
    assert s.bucket_grain() == 64 and s.batch_grain() == 64 and s.rec_chunk() == 64
    assert s.rec_argmax_pairs()


def test_cls_batches_and_decisions():
    """The cls stage's batching (consecutive runs of 32 lines, the last one
    shorter and not padded; engine.rs:1313-1324) and decision rule (flip when
    p1 > p0 and p1 >= cls_thresh 0.9; confidence max(p0, p1);
    engine.rs:1375-1380)."""
    from qppocr_amd import pipeline
    assert pipeline.cls_batches(42) == [(0, 32), (32, 42)]
    assert pipeline.cls_batches(32) == [(0, 32)]
    assert pipeline.cls_batches(0) == []
    assert pipeline.cls_batches(5, per=2) == [(0, 2), (2, 4), (4, 5)]
    p = np.array([[0.05, 0.95], [0.5, 0.5], [0.1, 0.9], [0.95, 0.05], [0.2, 0.8],
                  [0.9, 0.9]], dtype=np.float32)
    flip, conf = pipeline.cls_decisions(p)
    assert flip.tolist() == [True, False, True, False, False, False]
    assert conf.dtype == np.float32
    assert (conf == np.array([0.95, 0.5, 0.9, 0.95, 0.8, 0.9], dtype=np.float32)).all()
    assert pipeline.cls_decisions(p, thresh=0.96)[0].tolist() == [False] * 6
