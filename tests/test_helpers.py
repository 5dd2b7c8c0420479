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
