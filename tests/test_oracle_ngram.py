"""The n-gram guard's oracle, pinned without the reference (MAX is absent here).

* hand-worked cases: tests/test_kernels_ngram.py:62-69's spot checks, whose answers follow from the
  processor's definition by hand;
* the two formulations agree: the reference processor over the whole sequence with a window
  (ngram_block.mojo:5-15) and the op's per-id scan over the windowed history
  (ngram_block.mojo:112-146), on random sequences with planted repeats;
* the op only touches banned entries, and leaves ids outside the vocabulary alone.
"""

from __future__ import annotations

import numpy as np
import pytest


def test_hand_worked_cases(oracle) -> None:
    b = oracle.ngram_banned
    assert b([1, 2, 3], 3, 10) == set()            # the prefix's own occurrence never bans
    assert b([1, 2, 3, 1, 2], 3, 10) == {3}
    assert b([1, 2, 3, 1, 2], 3, 2) == set()       # out of the window
    assert b([1, 2], 3, 10) == set()               # too short for one n-gram
    assert b([4, 5, 6], 1, 2) == {5, 6}            # n == 1 bans every id in the window
    assert b([7, 8, 9], 0, 5) == set() and b([7, 8, 9], -2, 5) == set()
    assert b([5, 5, 5, 5], 2, 10) == {5}
    assert b([1, 2, 9, 1, 2, 8, 1, 2], 3, 10) == {9, 8}  # every earlier occurrence of the prefix bans


@pytest.mark.parametrize("seed", range(6))
def test_whole_sequence_and_windowed_forms_agree(oracle, seed) -> None:
    rng = np.random.default_rng(seed)
    vocab = 12
    for _ in range(40):
        length = int(rng.integers(1, 60))
        seq = [int(v) for v in rng.integers(0, vocab, length)]
        if length > 8 and rng.random() < 0.5:  # plant a repeat of the tail
            k = int(rng.integers(2, 6))
            at = int(rng.integers(0, length - k))
            seq[at:at + k] = seq[-k:]
        window = int(rng.integers(1, 70))
        n = int(rng.integers(-1, 8))
        history = seq[-window:]
        want = oracle.ngram_banned(seq, n, window)
        assert oracle.ngram_banned(history, n, len(history)) == want
        assert oracle.ngram_banned_per_id(history, n, vocab) == want


def test_op_sets_only_banned_ids_in_range(oracle) -> None:
    rng = np.random.default_rng(3)
    logits = rng.standard_normal((2, 10)).astype(np.float32)
    history = np.array([[1, 2, 3, 1, 2], [4, 40, -3, 4, 40]], np.int32)
    out = oracle.ngram_block(logits, history, 2)
    # row 0: prefix (2,) recurs at 1 -> bans 3; row 1: prefix (40,) recurs -> bans -3 (outside, ignored)
    assert out[0, 3] == oracle.NGRAM_BLOCKED and np.array_equal(np.delete(out[0], 3), np.delete(logits[0], 3))
    assert np.array_equal(out[1], logits[1])
    assert np.array_equal(oracle.ngram_block(logits[0], history[0], 3), out[0])  # rank 1 == row 0 here
