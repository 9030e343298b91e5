"""The prefill grouping's row placement, restated on the CPU: rows grouped by expert, in row order.

``csrc/route.hip``'s ``k_group_scatter_hist`` runs one workgroup of 256 threads per counting block
(``block_tokens`` tokens, ``block_tokens * topk`` rows).  Each workgroup sums the blocks' per-expert
counts into group starts and its own cursor per expert (the rows of that expert in earlier
blocks), then places its rows 256 a pass: a row's place is its expert's cursor, plus the lanes
below it in its wave with the same expert (one ballot per bit of the expert id, then a count of
the lower set bits), plus that expert's rows in the pass's earlier waves; the cursors then advance
by the pass's rows per expert.  Rows past the block's end take key 64, which no row has.

If this is right, ``group_rows`` is the stable argsort of the expert ids and ``inv`` its inverse.
Planted mistakes (counting the lane itself, leaving out the earlier waves, not advancing the
cursors) must fail the same check.
"""

from __future__ import annotations

import numpy as np
import pytest

WAVE, THREADS = 64, 256


def place_rows(ids: np.ndarray, E: int, topk: int, block_tokens: int, mistake: str = "") -> np.ndarray:
    """Positions of every row (``inv``) as the kernel computes them, one counting block at a time."""
    R = ids.size
    T = R // topk
    blocks = (T + block_tokens - 1) // block_tokens
    rows_per_block = block_tokens * topk
    hist = np.zeros((blocks, E), np.int64)
    for b in range(blocks):
        hist[b] = np.bincount(ids[b * rows_per_block:(b + 1) * rows_per_block], minlength=E)
    tot = hist.sum(axis=0)
    start = np.concatenate([[0], np.cumsum(tot)[:-1]])
    inv = np.full(R, -1, np.int64)
    for b in range(blocks):
        cursor = start + hist[:b].sum(axis=0)
        r0 = b * rows_per_block
        nr = min(R - r0, rows_per_block)
        for c0 in range(0, nr, THREADS):
            key = np.full(THREADS, 64, np.int64)  # lanes past the rows
            n = min(THREADS, nr - c0)
            key[:n] = ids[r0 + c0:r0 + c0 + n]
            wcnt = np.zeros((THREADS // WAVE, 65), np.int64)
            below = np.zeros(THREADS, np.int64)
            for w in range(THREADS // WAVE):
                k = key[w * WAVE:(w + 1) * WAVE]
                for lane in range(WAVE):
                    same = k == k[lane]  # the ballots over the key's 7 bits
                    below[w * WAVE + lane] = same[:lane + 1].sum() if mistake == "self" else same[:lane].sum()
                wcnt[w] = np.bincount(k, minlength=65)
            for tid in range(n):
                w, e = tid // WAVE, key[tid]
                earlier = 0 if mistake == "waves" else wcnt[:w, e].sum()
                inv[r0 + c0 + tid] = cursor[e] + below[tid] + earlier
            if mistake != "cursor":
                cursor = cursor + wcnt[:, :E].sum(axis=0)
    return inv


def expected(ids: np.ndarray) -> np.ndarray:
    order = np.argsort(ids, kind="stable")
    inv = np.empty_like(order)
    inv[order] = np.arange(order.size)
    return inv


def _ids(T: int, topk: int, E: int, seed: int, skew: bool) -> np.ndarray:
    rng = np.random.default_rng(seed)
    if skew:  # most rows on a few experts, as under Zipf routing
        p = 1.0 / np.arange(1, E + 1) ** 1.2
        return rng.choice(E, size=T * topk, p=p / p.sum())
    return rng.integers(0, E, size=T * topk)


@pytest.mark.parametrize(("T", "topk", "E", "skew"), [
    (2048, 6, 64, False), (2049, 6, 64, True), (2100, 20, 64, False), (4096, 6, 64, True), (2111, 6, 40, False),
])
def test_ballot_ranks_give_row_order(T: int, topk: int, E: int, skew: bool) -> None:
    ids = _ids(T, topk, E, T + topk, skew)
    assert np.array_equal(place_rows(ids, E, topk, 16), expected(ids))


def test_fused_routing_blocks() -> None:
    # the T < 2048 routing counts 4-token blocks: one pass of 24 rows a block at top-k 6
    ids = _ids(512, 6, 64, 7, True)
    assert np.array_equal(place_rows(ids, 64, 6, 4), expected(ids))


@pytest.mark.parametrize("mistake", ["self", "waves", "cursor"])
def test_planted_mistakes_fail(mistake: str) -> None:
    # 20 x 16 = 320 rows a block: two passes, four waves in the first
    ids = _ids(2100, 20, 64, 3, False)
    assert not np.array_equal(place_rows(ids, 64, 20, 16, mistake), expected(ids))
