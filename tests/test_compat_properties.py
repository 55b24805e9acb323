"""Properties of the selector's ranking rule, checked on random timings (hypothesis, CPU only).

The rule (Popcorn's `core/policy.py:150-172`, restated in `popcorn_amd.compat.selection`): among
the timings at the nearest comparable recorded configuration, the implementation with the lowest
median time wins, torch's time being the median of the reference times; when the runner-up is
within the indifference margin of the winner, the call goes to torch. Distances add |log2| gaps of
each dimension (values below 1 count as 1) and 10 when the batch extents differ.
"""

import math
import statistics
from types import SimpleNamespace

from hypothesis import given, settings
from hypothesis import strategies as st

from popcorn_amd.compat.selection import INDIFFERENCE, Timing, distance, fastest, rank

IMPLS = ("a", "b", "c")
times = st.floats(min_value=1e-3, max_value=1e3, allow_nan=False, allow_infinity=False)


def _timing(impl, n, ms, ref_ms, batch=(), device="gpu"):
    return Timing(impl, device, False, {"n": n}, tuple(batch), "float32", {}, frozenset(), ms, ref_ms)


def _call(n, batch=(), device="gpu"):
    config = {"dims": {"n": n}, "batch": list(batch), "dtype": "float32", "args": {}, "present": []}
    return SimpleNamespace(config=config, device_name=device, grad=False)


timing_lists = st.lists(st.tuples(st.sampled_from(IMPLS), times, times), min_size=1, max_size=12)


@settings(max_examples=300, deadline=None)
@given(timing_lists)
def test_fastest_is_the_lowest_median_unless_the_runner_up_is_within_the_margin(entries):
    timings = [_timing(impl, 64, ms, ref) for impl, ms, ref in entries]
    medians = {"torch": statistics.median(ref for _, _, ref in entries)}
    for impl in {impl for impl, _, _ in entries}:
        medians[impl] = statistics.median(ms for i, ms, _ in entries if i == impl)
    order = sorted(medians, key=lambda name: (medians[name], name))
    winner = fastest(timings)
    assert winner in medians
    if medians[order[1]] <= medians[order[0]] * (1 + INDIFFERENCE):
        assert winner == "torch"
    else:
        assert medians[winner] == medians[order[0]]
    # a zero margin never declares a tie unless two medians are equal
    exact = fastest(timings, margin=0.0)
    if medians[order[1]] > medians[order[0]]:
        assert medians[exact] == medians[order[0]]


@settings(max_examples=300, deadline=None)
@given(st.integers(min_value=0, max_value=1 << 20), st.integers(min_value=0, max_value=1 << 20),
       st.lists(st.integers(1, 8), max_size=2), st.lists(st.integers(1, 8), max_size=2))
def test_distance_is_the_log2_gap_plus_ten_for_another_batch(n, m, batch_a, batch_b):
    d = distance(_call(n, batch_a).config, _timing("a", m, 1.0, 1.0, batch_b))
    want = abs(math.log2(max(1, n)) - math.log2(max(1, m))) + (10.0 if list(batch_a) != list(batch_b) else 0.0)
    assert d >= 0 and math.isclose(d, want, rel_tol=1e-12, abs_tol=1e-12)
    # symmetric in the two configurations
    assert math.isclose(d, distance(_call(m, batch_b).config, _timing("a", n, 1.0, 1.0, batch_a)), abs_tol=1e-12)


powers = st.integers(0, 12).map(lambda e: 2 ** e)  # exact log2 gaps, so ties between sizes are exact


@settings(max_examples=200, deadline=None)
@given(st.lists(st.tuples(st.sampled_from(IMPLS), powers, times, times), min_size=1, max_size=10), powers)
def test_rank_decides_at_the_nearest_recorded_size_only(entries, n):
    timings = [_timing(impl, size, ms, ref) for impl, size, ms, ref in entries]
    names = list(IMPLS) + ["torch"]
    got = rank(names, _call(n), timings)
    gaps = [abs(math.log2(size) - math.log2(n)) for _, size, _, _ in entries]
    nearest = min(gaps)
    pool = [t for t, gap in zip(timings, gaps) if gap == nearest]
    assert got == fastest(pool)
    # timings on another device are never comparable
    assert rank(names, _call(n, device="other"), timings) is None


@settings(max_examples=100, deadline=None)
@given(timing_lists)
def test_rank_only_returns_a_name_it_was_offered(entries):
    timings = [_timing(impl, 64, ms, ref) for impl, ms, ref in entries]
    got = rank(["a", "torch"], _call(64), timings)
    assert got in ("a", "torch", None)
    if not any(impl == "a" for impl, _, _ in entries):
        # only torch's reference times remain: torch, the sole candidate in the pool of "a" rows, has none
        assert got is None
