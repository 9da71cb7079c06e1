"""The tolerance check the parity tests use rejects what it must: a NaN where
the reference is finite fails, as does any element past the bound; matching
infinities and NaN against NaN pass."""
import numpy as np
import pytest

from tests.helpers import assert_close


def test_nan_against_a_number_fails():
    with pytest.raises(AssertionError):
        assert_close(np.array([1.0, np.nan]), np.array([1.0, 2.0]), atol=1e-2, rtol=1e-2)


def test_out_of_bound_fails_and_within_passes():
    with pytest.raises(AssertionError):
        assert_close(np.array([1.0, 2.1]), np.array([1.0, 2.0]), atol=1e-2, rtol=1e-2)
    assert_close(np.array([1.0, 2.01]), np.array([1.0, 2.0]), atol=1e-2, rtol=1e-2)


def test_matching_specials_pass():
    assert_close(np.array([np.inf, -np.inf, np.nan]), np.array([np.inf, -np.inf, np.nan]),
                 atol=0.0, rtol=0.0)
    with pytest.raises(AssertionError):
        assert_close(np.array([np.inf]), np.array([-np.inf]), atol=1e-2, rtol=1e-2)
