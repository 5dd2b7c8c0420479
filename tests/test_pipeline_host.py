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
