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
    mode, e_gr, e_re, e_ge, n, ref_bar = check_against_reference(got, ref, exact)
    assert mode == "exact" and n == 1 and e_re == pytest.approx(5e-3) and e_ge <= 2.1e-5
    assert ref_bar > 1


def test_exception_taken_where_reference_is_at_the_edge_of_the_bar():
    # the reference 0.99 of the bar above exact, got a fifth of the bar below
    exact = arrays(5)
    ref = exact.copy()
    got = exact.copy()
    bar = 1e-4 + 1e-5 * abs(exact[3, 105])
    ref[3, 105] += 0.99 * bar
    got[3, 105] -= 0.2 * bar
    mode, e_gr, e_re, e_ge, n, ref_bar = check_against_reference(got, ref, exact)
    assert mode == "exact" and n == 1 and ref_bar < 1


def test_less_accurate_than_reference_not_excused():
    # got and ref on either side of exact, got the farther: not excused
    exact = arrays(6)
    ref = exact.copy()
    got = exact.copy()
    bar = 1e-4 + 1e-5 * abs(exact[0, 9])
    ref[0, 9] += 0.5 * bar
    got[0, 9] -= 0.6 * bar
    with pytest.raises(AssertionError, match="not closer to the exact"):
        check_against_reference(got, ref, exact)


def test_wrong_result_fails_where_reference_is_accurate():
    exact = arrays(2)
    ref = exact + 1e-6
    got = exact.copy()
    got[3, 100] += 2e-3               # a planted mistake
    with pytest.raises(AssertionError, match="not closer to the exact"):
        check_against_reference(got, ref, exact)


def test_wrong_result_fails_even_when_reference_misses_the_bar():
    exact = arrays(3)
    ref = exact.copy()
    ref[0, 0] += 5e-3
    got = exact.copy()
    got[2, 5] += 5e-4                 # wrong elsewhere: not excused
    with pytest.raises(AssertionError, match="not closer to the exact"):
        check_against_reference(got, ref, exact)


def test_wrong_result_within_reference_error_still_held_to_exact():
    # got closer to exact than a very wrong reference, but outside the bar
    # of exact: not excused
    exact = arrays(7)
    ref = exact.copy()
    ref[1, 1] += 1e-2
    got = exact.copy()
    got[1, 1] += 5e-3
    with pytest.raises(AssertionError, match="against the exact result"):
        check_against_reference(got, ref, exact)


def test_nan_is_never_close():
    exact = arrays(4)
    got = exact.copy()
    got[0, 1] = np.nan
    with pytest.raises(AssertionError):
        check_against_reference(got, exact.copy(), exact)
