"""CPU checks of the fused-attention bar of the GPU tests
(conftest.check_against_reference): the exception to the reference bar is
taken only where the reference itself misses the bar against the exact
result, and planted mistakes fail it."""
import numpy as np
import pytest

from conftest import check_against_reference


def arrays(seed=0, n=(4, 128)):
    rng = np.random.default_rng(seed)
    exact = rng.standard_normal(n) * 3
    return exact


def test_plain_bar_holds():
    exact = arrays()
    ref = exact + 3e-5
    got = exact - 3e-5
    assert check_against_reference(got, ref, exact)[0] == "reference"


def test_exception_taken_where_reference_misses_the_bar():
    exact = arrays(1)
    ref = exact.copy()
    ref[1, 7] += 5e-3                 # the reference's lost weight sum
    got = exact + 2e-5
    mode, e_gr, e_re, e_ge = check_against_reference(got, ref, exact)
    assert mode == "exact" and e_re == pytest.approx(5e-3) and e_ge <= 2.1e-5


def test_wrong_result_fails_where_reference_is_accurate():
    exact = arrays(2)
    ref = exact + 1e-6
    got = exact.copy()
    got[3, 100] += 2e-3               # a planted mistake
    with pytest.raises(AssertionError, match="although the reference meets it"):
        check_against_reference(got, ref, exact)


def test_wrong_result_fails_even_when_reference_misses_the_bar():
    exact = arrays(3)
    ref = exact.copy()
    ref[0, 0] += 5e-3
    got = exact.copy()
    got[2, 5] += 5e-4                 # wrong elsewhere: not excused
    with pytest.raises(AssertionError, match="against the exact result"):
        check_against_reference(got, ref, exact)


def test_nan_is_never_close():
    exact = arrays(4)
    got = exact.copy()
    got[0, 1] = np.nan
    with pytest.raises(AssertionError):
        check_against_reference(got, exact.copy(), exact)
