"""The tolerance checker of the parity tests must reject the errors it is there to catch (CPU only)."""
import numpy as np
import pytest

from helpers import ATOL, assert_close


def test_accepts_f16_rounding():
    rng = np.random.default_rng(0)
    ref = rng.standard_normal((4, 128))
    got = ref.astype(np.float16).astype(np.float64)
    assert_close(got, ref, 64)


@pytest.mark.parametrize("delta", [3e-3, 5e-2])
def test_rejects_an_abs_error(delta):
    ref = np.zeros((2, 128))
    got = ref.copy()
    got[1, 70] = delta
    with pytest.raises(AssertionError):
        assert_close(got, ref, 64)


def test_rejects_a_relative_error_on_large_values():
    ref = np.full((1, 64), 10.0)
    got = ref.copy()
    got[0, 3] = 10.0 * (1 + 2e-2)
    with pytest.raises(AssertionError):
        assert_close(got, ref, 64)


def test_rejects_nan():
    ref = np.zeros((1, 64))
    got = ref.copy()
    got[0, 0] = np.nan
    with pytest.raises(AssertionError):
        assert_close(got, ref, 64)


def test_rejects_an_lse_error():
    ref = np.zeros((1, 64))
    with pytest.raises(AssertionError):
        assert_close(ref, ref, 64, "", np.array([[1.0]]), np.array([[1.0 + 2e-3]]))
    assert ATOL == 2e-3
