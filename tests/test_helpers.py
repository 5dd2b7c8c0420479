"""The test suite's own comparison helpers (CPU only)."""
import numpy as np
import pytest

from conftest import assert_bitexact, baseline_tol_check


def test_baseline_tolerance_helper():
    """|g - r| <= max(1e-4 |r|, 1e-5): inside passes, outside fails."""
    baseline_tol_check(np.array([1.0, 0.0]), np.array([1.00005, 5e-6]))
    with pytest.raises(AssertionError):
        baseline_tol_check(np.array([1.0, 0.0]), np.array([1.0002, 0.0]))
    with pytest.raises(AssertionError):
        baseline_tol_check(np.array([0.0]), np.array([2e-5]))


def test_bitexact_helper():
    assert_bitexact(np.array([0.0, np.nan, 1.0], np.float32), np.array([-0.0, np.nan, 1.0], np.float32))
    with pytest.raises(BaseException):
        assert_bitexact(np.array([1.0], np.float32), np.array([np.nextafter(np.float32(1), 2)]))


def test_pairs_tolerance_helper():
    """ids may differ only at near-ties of the logits; values within 1e-4."""
    from conftest import pairs_tolerance_check

    def pr(vals, ids):
        p = np.zeros((len(vals), 2), np.float32)
        p[:, 0] = vals
        p[:, 1] = np.array(ids, np.uint32).view(np.float32)
        return p
    logits = np.array([[0.0, 5.0, 5.0 - 1e-6], [3.0, 1.0, 0.0]], np.float32)
    ref = pr([0.5, 0.8], [1, 0])
    assert pairs_tolerance_check(pr([0.50001, 0.8], [2, 0]), ref, logits) == 1
    with pytest.raises(AssertionError):
        pairs_tolerance_check(pr([0.5, 0.8], [1, 1]), ref, logits)    # gap 2: not a tie
    with pytest.raises(AssertionError):
        pairs_tolerance_check(pr([0.51, 0.8], [1, 0]), ref, logits)   # value off by 2%
