"""GPU parity of ``ngram_block`` (the n-gram logit guard) against the oracle: integer work, so every
row bans exactly the oracle's set (to the kernel's BLOCKED) and returns every other logit bit for bit.

The cases are tests/test_kernels_ngram.py's: four histories the guard treats differently (a planted
repeat inside the window, distinct ids, period 10, a repeat outside the window), n = 1, 3, 35 over
B rows in one call, rows that do not mix, n < 1 and short histories as pass-throughs, the real
shape (B = 8 x 129 280), and the one-row form.  Sequences are drawn by this file's own generator.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _gpu import n, t

pytestmark = pytest.mark.gpu

WINDOW = 128
VOCAB = 4096
REAL_VOCAB = 129280


def _distinct(rng, count, vocab):
    return [int(i) for i in rng.permutation(vocab)[:count]]


def _rows(vocab: int, seed: int = 0) -> list[list[int]]:
    """0: filler(60) + motif(40) + filler(20) + motif(40); 1: distinct ids; 2: period 10;
    3: motif(40) + filler(150) + motif(40) (the earlier motif outside the last 128 ids)."""
    rng = np.random.default_rng(seed)
    ids = _distinct(rng, 310, vocab)
    planted = ids[:60] + ids[60:100] + ids[100:120] + ids[60:100]
    unique = _distinct(rng, 200, vocab)
    period = [int(i) for i in rng.integers(0, vocab, size=10)] * 20
    far = ids[120:160] + ids[160:310] + ids[120:160]
    return [planted, unique, period, far]


def _history(seq, window=WINDOW):
    return np.asarray(seq[-window:], dtype=np.int32)


def _ops():
    import uocr_moe

    return uocr_moe.ops


def _check(oracle, got, logits, seq, ngram, label):
    want = oracle.ngram_banned(seq, ngram, WINDOW)
    banned = {int(i) for i in np.flatnonzero(got == oracle.NGRAM_BLOCKED)}
    assert banned == want, f"{label}: n={ngram} banned {sorted(banned)[:8]}, oracle {sorted(want)[:8]}"
    keep = np.ones(got.shape[0], bool)
    keep[list(banned)] = False
    assert np.array_equal(got[keep].view(np.uint32), logits[keep].view(np.uint32)), label
    return banned


@pytest.mark.parametrize("ngram", [1, 3, 35])
def test_each_row_bans_what_the_oracle_bans(oracle, ngram) -> None:
    seqs = _rows(VOCAB)
    logits = np.random.default_rng(5).standard_normal((4, VOCAB)).astype(np.float32)
    hist = np.stack([_history(s) for s in seqs])
    got = n(_ops().ngram_block(t(logits), t(hist), t(np.array([ngram], np.int32))))
    assert np.array_equal(got, oracle.ngram_block(logits, hist, ngram))
    banned = [_check(oracle, got[b], logits[b], seqs[b], ngram, f"row {b}") for b in range(4)]
    if ngram == 1:
        assert all(banned[b] == set(seqs[b][-WINDOW:]) for b in range(4))
    else:
        assert banned[0] and banned[2] and not banned[1] and not banned[3]
    if ngram == 35:
        assert banned[0] == {seqs[0][100]}


def test_rows_do_not_mix() -> None:
    seqs = _rows(VOCAB)
    logits = np.tile(np.random.default_rng(6).standard_normal(VOCAB).astype(np.float32), (4, 1))
    hist = np.stack([_history(s) for s in seqs])
    order = [2, 3, 0, 1]
    straight = n(_ops().ngram_block(t(logits), t(hist), 3))
    swapped = n(_ops().ngram_block(t(logits), t(hist[order]), 3))
    assert np.array_equal(swapped, straight[order])
    assert not np.array_equal(straight[0], straight[2])


@pytest.mark.parametrize("ngram", [0, -1, WINDOW + 1])
def test_pass_through_cases(ngram) -> None:
    """n < 1 (the guard switched off, any history, zeros included) and a history shorter than n."""
    seqs = _rows(VOCAB)
    logits = np.random.default_rng(7).standard_normal((4, VOCAB)).astype(np.float32)
    hist = np.stack([_history(s) for s in seqs])
    for h in (hist, np.zeros_like(hist)):
        assert np.array_equal(n(_ops().ngram_block(t(logits), t(h), ngram)), logits)


@pytest.mark.parametrize("ngram", [1, 35])
def test_the_real_shape_b8(oracle, ngram) -> None:
    seqs = _rows(REAL_VOCAB, seed=11) + _rows(REAL_VOCAB, seed=13)
    logits = np.random.default_rng(12).standard_normal((8, REAL_VOCAB)).astype(np.float32)
    hist = np.stack([_history(s) for s in seqs])
    got = n(_ops().ngram_block(t(logits), t(hist), ngram))
    for b in range(8):
        _check(oracle, got[b], logits[b], seqs[b], ngram, f"row {b}")


@pytest.mark.parametrize("ngram", [1, 3, 35])
def test_one_row_form_in_place_and_odd_vocab(oracle, ngram) -> None:
    """Rank 1 equals row b of the rank-2 call; in place (result = logits) gives the same bits; a
    vocabulary that is not a multiple of 4 (the one-column path) too."""
    seqs = _rows(VOCAB)
    logits = np.random.default_rng(9).standard_normal((4, VOCAB)).astype(np.float32)
    hist = np.stack([_history(s) for s in seqs])
    rows = n(_ops().ngram_block(t(logits), t(hist), ngram))
    for b in range(4):
        one = n(_ops().ngram_block(t(logits[b]), t(hist[b]), ngram))
        assert np.array_equal(one, rows[b])
    inplace = t(logits)
    _ops().ngram_block(inplace, t(hist), ngram, out=inplace)
    assert np.array_equal(n(inplace), rows)
    odd = np.ascontiguousarray(logits[:, : VOCAB - 3])
    assert np.array_equal(n(_ops().ngram_block(t(odd), t(hist), ngram)), oracle.ngram_block(odd, hist, ngram))


def test_refusals() -> None:
    import uocr_moe

    ops = _ops()
    logits = torch.zeros((2, 16), device="cuda:0")
    hist = torch.zeros((2, 4), dtype=torch.int32, device="cuda:0")
    with pytest.raises(uocr_moe.UocrError, match="history and logits disagree on the row count"):
        ops.ngram_block(logits, hist[:1], 2)
    with pytest.raises(uocr_moe.UocrError, match="`ngram` must be a single int32"):
        ops.ngram_block(logits, hist, torch.zeros(2, dtype=torch.int32, device="cuda:0"))
    with pytest.raises(uocr_moe.UocrError, match="history is empty"):
        ops.ngram_block(logits, hist[:, :0], 2)
    with pytest.raises(uocr_moe.UocrError, match="logits and output disagree on shape"):
        ops.ngram_block(logits, hist, 2, out=torch.zeros((2, 15), device="cuda:0"))
