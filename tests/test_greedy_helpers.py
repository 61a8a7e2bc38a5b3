"""The greedy-comparison helper of the GPU tests, checked on the CPU with
hand-made token sequences: a difference is accepted only at a near-tie, and
the comparison then continues against the oracle's sequence from the GPU's
pick instead of stopping there."""
import pytest

from gpu_util import compare_greedy


def _cont(table):
    """An oracle continuation from a table {prefix: (tokens, margins)}."""
    def resume(prefix, k):
        toks, mar = table[tuple(prefix)]
        return toks[:k], mar[:k]
    return resume


def test_identical_sequences_compare_every_step():
    assert compare_greedy([1, 2, 3], [1, 2, 3], [0.5, 0.5, 0.5], "same") == 3


def test_a_difference_at_a_clear_margin_fails():
    with pytest.raises(AssertionError, match="step 1"):
        compare_greedy([1, 9, 3], [1, 2, 3], [0.5, 0.5, 0.5], "clear")


def test_a_near_tie_continues_against_the_forced_oracle():
    # step 1 is a near-tie; from the GPU's pick 9 the oracle continues 7, 8
    resume = _cont({(1, 9): ([7, 8], [0.3, 0.3])})
    assert compare_greedy([1, 9, 7, 8], [1, 2, 3, 4], [0.5, 1e-4, 0.5, 0.5], "tie", resume=resume) == 1


def test_a_mismatch_after_the_forced_step_still_fails():
    resume = _cont({(1, 9): ([7, 8], [0.3, 0.3])})
    with pytest.raises(AssertionError, match="step 3"):
        compare_greedy([1, 9, 7, 5], [1, 2, 3, 4], [0.5, 1e-4, 0.5, 0.5], "tie then miss", resume=resume)


def test_a_near_tie_without_a_continuation_fails():
    with pytest.raises(AssertionError, match="no oracle continuation"):
        compare_greedy([1, 9], [1, 2], [0.5, 1e-4], "no resume")


def test_length_mismatch_fails():
    with pytest.raises(AssertionError, match="tokens"):
        compare_greedy([1, 2], [1, 2, 3], [0.5, 0.5, 0.5], "short")
