import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def gpu():
    """torch + the HIP library on device 0; fails loudly when either is missing."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    from qppocr_amd import _lib, ops
    _lib.load()
    ops.context(0)
    return torch


class XorShift:
    """xorshift64* stream of the reference kernel tests
    (qppocr-kernels/tests/kernels.rs:29-49): values in [-1, 1)."""

    def __init__(self, seed=0x243F6A8885A308D3):
        self.s = seed

    def next_f32(self):
        m = (1 << 64) - 1
        s = self.s
        s ^= s >> 12
        s ^= (s << 25) & m
        s ^= s >> 27
        self.s = s
        v = (s * 0x2545F4914F6CDD1D) & m
        return np.float32(((v >> 40) - (1 << 23)) / float(1 << 23))

    def fill(self, shape):
        n = int(np.prod(shape))
        return np.array([self.next_f32() for _ in range(n)], dtype=np.float32).reshape(shape)


def rel_check(got, ref, tol=1e-5):
    """The reference's acceptance check (kernels.rs:51-77): max|diff| / max|ref| < tol."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    mx = np.abs(got - ref).max() if got.size else 0.0
    scale = max(np.abs(ref).max() if ref.size else 0.0, 1e-6)
    assert mx / scale < tol, f"max diff {mx:.3e} (rel {mx / scale:.2e})"


def baseline_tol_check(got, ref):
    """Elementwise |g - r| <= max(1e-4 |r|, 1e-5) (the fp32 tolerance of the path)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    bad = np.abs(got - ref) > np.maximum(1e-4 * np.abs(ref), 1e-5)
    assert not bad.any(), f"{bad.sum()} elements outside 1e-4 rel / 1e-5 abs"


def assert_bitexact(got, ref, name=""):
    """Value equality of every element (+0 == -0; NaNs must coincide)."""
    got = np.asarray(got, dtype=np.float32)
    ref = np.asarray(ref, dtype=np.float32)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    nan_g, nan_r = np.isnan(got), np.isnan(ref)
    assert (nan_g == nan_r).all(), f"{name}: NaN pattern differs"
    neq = (got != ref) & ~nan_g
    if neq.any():
        idx = np.argwhere(neq)[0]
        d = np.abs(got.astype(np.float64) - ref).max()
        pytest.fail(f"{name}: {neq.sum()} / {got.size} elements differ; first at {tuple(idx)}: "
                    f"{got[tuple(idx)]!r} vs {ref[tuple(idx)]!r}; max |diff| {d:.3e}")


def pairs_tolerance_check(pairs, pairs_ref, logits_ref):
    """The tolerance rule for the CTC argmax exit: values within 1e-4
    relative (1e-5 absolute near zero) of the reference's, ids identical
    except where the top-2 logit gap of the step is below 1e-4.  Returns the
    number of steps whose ids differ (all of them near-ties)."""
    pairs = np.asarray(pairs, np.float32).reshape(-1, 2)
    pairs_ref = np.asarray(pairs_ref, np.float32).reshape(-1, 2)
    logits = np.asarray(logits_ref, np.float32).reshape(pairs.shape[0], -1)
    baseline_tol_check(pairs[:, 0], pairs_ref[:, 0])
    ids = np.ascontiguousarray(pairs[:, 1]).view(np.uint32)
    ids_ref = np.ascontiguousarray(pairs_ref[:, 1]).view(np.uint32)
    diff = np.nonzero(ids != ids_ref)[0]
    if diff.size:
        top2 = -np.sort(-logits[diff], axis=1)[:, :2].astype(np.float64)
        gap = top2[:, 0] - top2[:, 1]
        assert (gap < 1e-4).all(), f"ids differ at steps {diff[gap >= 1e-4][:8]} (gaps {gap.max()})"
    return int(diff.size)
