"""bench.py's interleaved A/B (DequantGEMVBenchmark.swift:220-286): the sign
test's normal approximation and the alternating sample order.  CPU only."""
import math
import os
import sys

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import pytest  # noqa: E402
from scipy.stats import binomtest, norm  # noqa: E402

import bench  # noqa: E402


def test_sign_test_needs_eight_pairs():
    # ABResult.signTestP: a 4-of-4 result is NaN (chance gives it one time in eight)
    assert math.isnan(bench.sign_test_p([1.1, 1.2, 1.3, 1.05]))
    assert math.isnan(bench.sign_test_p([1.1] * 7))
    assert not math.isnan(bench.sign_test_p([1.1] * 8))


@pytest.mark.parametrize("n,wins", [(40, 20), (40, 30), (40, 40), (12, 3), (9, 9)])
def test_sign_test_is_two_sided_normal_approximation(n, wins):
    ratios = [1.5] * wins + [0.5] * (n - wins)
    z = abs(wins - n / 2) / (math.sqrt(n) / 2)
    assert bench.sign_test_p(ratios) == pytest.approx(2 * norm.sf(z), rel=1e-12, abs=1e-300)
    # symmetric: B losing as often is as significant
    assert bench.sign_test_p([1 / r for r in ratios]) == pytest.approx(bench.sign_test_p(ratios))
    # and close to the exact binomial test where the approximation holds
    if n >= 40:
        exact = binomtest(wins, n, 0.5).pvalue
        assert bench.sign_test_p(ratios) == pytest.approx(exact, abs=0.02)


def test_ties_count_as_no_win():
    assert bench.sign_test_p([1.0] * 10) == pytest.approx(2 * norm.sf(math.sqrt(10)))


def test_interleaved_order_and_ratios():
    calls = []

    def a(i):
        calls.append(("a", i))
        return 2e-6

    def b(i):
        calls.append(("b", i))
        return 1e-6 if i % 4 else 4e-6      # B twice as fast, except every fourth pair

    r = bench.interleaved_ab(a, b, 8)
    # the side that runs first alternates, so neither keeps the warmer slot
    assert calls == [("a", 0), ("b", 0), ("b", 1), ("a", 1), ("a", 2), ("b", 2), ("b", 3), ("a", 3),
                     ("a", 4), ("b", 4), ("b", 5), ("a", 5), ("a", 6), ("b", 6), ("b", 7), ("a", 7)]
    # ratio = B throughput / A throughput
    assert r["ratios"] == [0.5, 2.0, 2.0, 2.0, 0.5, 2.0, 2.0, 2.0]
    assert r["median_ratio"] == 2.0 and r["b_wins"] == 6 and r["pairs"] == 8
    assert r["a_median_us"] == 2.0 and r["b_median_us"] == 1.0
    assert r["sign_test_p"] == pytest.approx(2 * norm.sf(abs(6 - 4) / (math.sqrt(8) / 2)))


def test_ab_spec_parsing():
    assert bench.parse_ab("GODWIT_DECODE_LAYER=0") == {"GODWIT_DECODE_LAYER": "0"}
    assert bench.parse_ab("GODWIT_PREFILL_ABOVE=8, GODWIT_SELF_GROUP_TOKENS=0") == {
        "GODWIT_PREFILL_ABOVE": "8", "GODWIT_SELF_GROUP_TOKENS": "0"}
    for bad in ("DECODE_LAYER=0", "GODWIT_DECODE_LAYER", "HOME=/"):
        with pytest.raises(SystemExit):
            bench.parse_ab(bad)
