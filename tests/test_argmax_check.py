"""The downstream-argmax checker used by the GPU parity tests (CPU only)."""
import numpy as np
import pytest

from tests.gpu_util import _projection, assert_argmax_agrees


def test_identical_and_small_noise_pass():
    rng = np.random.default_rng(0)
    want = rng.standard_normal((64, 256)).astype(np.float32)
    assert assert_argmax_agrees(want, want) == 0
    assert_argmax_agrees(want + rng.standard_normal(want.shape).astype(np.float32) * 1e-6, want)


def test_near_tie_flip_is_allowed_and_real_flip_is_not():
    rng = np.random.default_rng(1)
    W = _projection(256)
    want = rng.standard_normal((8, 256))
    # row 0: push the output along (W_b - W_a) until the oracle's top two classes nearly tie, then
    # add an error just large enough to flip them: a near tie, allowed
    lw = want @ W
    a, b = np.argsort(lw[0])[-1], np.argsort(lw[0])[-2]
    d = W[:, b] - W[:, a]
    want[0] += d * (lw[0, a] - lw[0, b] - 1e-4) / (d @ d)
    got = want.copy()
    r = np.random.default_rng(2).standard_normal(256) * 1e-4
    r -= d * (r @ d) / (d @ d)             # error component that leaves the two classes' gap alone
    got[0] += d * 2e-4 / (d @ d) + r
    assert assert_argmax_agrees(got, want) == 1
    # row 1: a wide-margin row moved far enough to change its argmax: must fail
    got2 = want.copy()
    lw1 = want[1] @ W
    a1, b1 = np.argsort(lw1)[-1], np.argsort(lw1)[-2]
    d1 = W[:, b1] - W[:, a1]
    got2[1] += d1 * 2.0 * (lw1[a1] - lw1[b1]) / (d1 @ d1)
    with pytest.raises(AssertionError):
        assert_argmax_agrees(got2, want)
