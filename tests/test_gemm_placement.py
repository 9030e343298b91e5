"""The grouped GEMM's tile placements, restated on the CPU: every tile of a launch is run exactly once.

``csrc/gemm.hip`` places a launch's tiles two ways (``walk_balanced`` and ``walk_classes``); a tile
placed twice would be computed twice (the same bits, so no output test notices the waste), and a tile
placed nowhere would leave its rows unwritten.  This restates the balanced placement's arithmetic --
the groups ranked by rows (``make_seq``), the routed sequence cut into 8 equal-cost ranges
(``seq_below``, ``group_below``, ``below``), the shared row tiles in 8 runs, and each workgroup's walk
(``walk_of``: two rounds, the second reversed, or rounds in order) -- and checks, for skewed and
adversarial routings and the served shapes, that the walks of all 8 x 64 workgroups cover every tile
of both problems exactly once with rows inside the tile's group.  Planted mistakes (shared runs of
rtb // 8 row tiles each, which drop the remainder; the second round not reversed) must fail it.
"""

from __future__ import annotations

import numpy as np
import pytest

BK = 64
XCDS = 8


def tile_cost(K: int, int8: bool, nact: int) -> int:
    """``tile_cost``: per 64-k step 100 + 35 per active block (int8) or 65 + 36 (bf16), plus 600."""
    return (K // BK) * ((100 + 35 * nact) if int8 else (65 + 36 * nact)) + 600


def row_tiles(count: int, BM: int) -> tuple[int, int, int]:
    """``row_tiles_of``: row tiles, whether the last is partial, and its active 32-row blocks."""
    rt = (count + BM - 1) // BM
    rem = count - (rt - 1) * BM
    part = 1 if (count > 0 and rem < BM) else 0
    return rt, part, ((rem + 31) >> 5) if part else 0


def below(t: int, c: int) -> int:
    """Tiles of cost c whose midpoints lie below t: (2i + 1) c < 2t."""
    return (2 * t - c + 2 * c - 1) // (2 * c) if 2 * t > c else 0


def group_below(K, int8, BM, rt, part, apart, nt, t):
    cf = tile_cost(K, int8, BM // 32)
    full = nt * (rt - part) * cf
    if t <= full:
        return below(t, cf)
    return nt * (rt - part) + (min(nt, below(t - full, tile_cost(K, int8, apart))) if part else 0)


def balanced_walks(counts, M, nta, ntb, Ka, int8=True, J=64, planted_runs=False, planted_order=False):
    """Every workgroup's tiles under the balanced placement, as (problem, group, row tile, column)."""
    BMA, BMB, L = (128 if int8 else 64), 64, 64
    cnt = [counts[l] if l < len(counts) else 0 for l in range(L)]
    # the rank of each group, most rows first, ties in group order
    rank = [sum(1 for k in range(L) if cnt[k] > cnt[l] or (cnt[k] == cnt[l] and k < l)) for l in range(L)]
    qc, qg = [0] * L, [0] * L
    for l in range(L):
        qc[rank[l]], qg[rank[l]] = cnt[l], l
    tiles, costs = [], []
    for p in range(L):
        rt, part, apart = row_tiles(qc[p], BMA)
        tiles.append(nta * rt)
        costs.append(nta * ((rt - part) * tile_cost(Ka, int8, BMA // 32) + (tile_cost(Ka, int8, apart) if part else 0)))
    tp = np.concatenate([[0], np.cumsum(tiles)[:-1]]).tolist()
    cp = np.concatenate([[0], np.cumsum(costs)[:-1]]).tolist()
    ta, ca = sum(tiles), sum(costs)

    def seq_below(t):
        if t <= 0:
            return 0
        if t >= ca:
            return ta
        g = sum(1 for p in range(L) if qc[p] > 0 and cp[p] <= t) - 1
        rt, part, apart = row_tiles(qc[g], BMA)
        return tp[g] + group_below(Ka, int8, BMA, rt, part, apart, nta, t - cp[g])

    walks = []
    rtb = (M + BMB - 1) // BMB
    for x in range(XCDS):
        b0, b1 = rtb * x // XCDS, rtb * (x + 1) // XCDS
        if planted_runs:
            b0, b1 = x * (rtb // XCDS), (x + 1) * (rtb // XCDS)
        nsh = (b1 - b0) * ntb
        s0, s1 = seq_below(ca * x // XCDS), seq_below(ca * (x + 1) // XCDS)
        n = nsh + s1 - s0
        two = n <= 2 * J
        for j in range(J):
            items = []
            count = ((1 if j < n else 0) + (1 if 2 * J - 1 - j < n else 0)) if two else max(0, (n - j + J - 1) // J)
            for k in range(count):
                it = (2 * J - 1 - j) if (two and k == 1 and not planted_order) else j + k * J
                if it >= n:
                    continue
                if it >= nsh:
                    i = it - nsh + s0
                    g = sum(1 for p in range(L) if qc[p] > 0 and tp[p] <= i) - 1
                    local = i - tp[g]
                    mt, c = local // nta, local % nta
                    rows = min(BMA, qc[g] - mt * BMA)
                    items.append(("a", qg[g], mt, c, rows))
                else:
                    mt = b0 + it // ntb
                    c = it - (mt - b0) * ntb
                    rows = min(BMB, M - mt * BMB)
                    items.append(("b", 0, mt, c, rows))
            walks.append(items)
    want = {("a", g, mt, c) for g, n_rows in enumerate(counts) for mt in range(row_tiles(n_rows, BMA)[0])
            for c in range(nta)}
    want |= {("b", 0, mt, c) for mt in range(rtb) for c in range(ntb)}
    return walks, want


def covers_once(walks, want) -> bool:
    seen = [it[:4] for w in walks for it in w]
    return len(seen) == len(set(seen)) and set(seen) == want and all(it[4] > 0 for w in walks for it in w)


def _zipf_counts(rng, T: int, topk: int = 6, E: int = 64) -> list[int]:
    w = 1.0 / np.arange(1, E + 1) ** 1.1
    rng.shuffle(w)
    return np.bincount(rng.choice(E, size=T * topk, p=w / w.sum()), minlength=E).tolist()


@pytest.mark.parametrize("T", [512, 2048, 4096])
@pytest.mark.parametrize("proj", ["gate_up", "down"])
def test_balanced_placement_runs_every_tile_once(T: int, proj: str) -> None:
    nta, ntb, Ka = (7, 14, 1280) if proj == "gate_up" else (5, 5, 896)
    rng = np.random.default_rng(T + len(proj))
    for counts in (_zipf_counts(rng, T), [T] * 6 + [0] * 58, [T * 6 // 64] * 64, [1] * 64):
        walks, want = balanced_walks(counts, T, nta, ntb, Ka)
        assert covers_once(walks, want), (T, proj, counts[:8])


def test_balanced_placement_balances_the_xcds() -> None:
    """Skewed routing at T=4096: every XCD's estimated cost is within 10 % of the mean (the round-robin
    unit deal it replaced left them up to 2x apart)."""
    rng = np.random.default_rng(7)
    counts = _zipf_counts(rng, 4096)
    walks, _ = balanced_walks(counts, 4096, 5, 5, 896)
    per_xcd = []
    for x in range(XCDS):
        cost = 0
        for items in walks[x * 64:(x + 1) * 64]:
            for prob, _g, _mt, _c, rows in items:
                nact = (rows + 31) >> 5
                cost += tile_cost(896, True, nact) if prob == "a" else tile_cost(1792, False, nact)
        per_xcd.append(cost)
    mean = np.mean(per_xcd)
    assert max(per_xcd) <= 1.1 * mean and min(per_xcd) >= 0.9 * mean, per_xcd


def test_random_shapes_run_every_tile_once() -> None:
    rng = np.random.default_rng(3)
    for _ in range(60):
        ng = int(rng.integers(0, 65))
        counts = [int(rng.choice([1, 5, 31, 32, 33, 100, 127, 128, 129, 500, 3000])) if rng.random() < 0.5
                  else int(rng.integers(1, 4000)) for _ in range(ng)]
        M = int(rng.choice([0, 1, 63, 64, 65, 512, 4096]))
        nta, ntb, Ka = ((7, 14, 1280), (5, 5, 896))[int(rng.integers(0, 2))]
        walks, want = balanced_walks(counts, M, nta, ntb, Ka, int8=bool(rng.random() < 0.7))
        assert covers_once(walks, want)


def test_planted_mistakes_fail() -> None:
    """Shared runs of equal length (rtb // 8 each) lose the remainder row tiles; an unreversed second
    round repeats list entries: the same check catches both."""
    rng = np.random.default_rng(11)
    counts = _zipf_counts(rng, 4096)
    assert covers_once(*balanced_walks(counts, 4000, 7, 14, 1280))
    assert not covers_once(*balanced_walks(counts, 4000, 7, 14, 1280, planted_runs=True))
    counts = _zipf_counts(rng, 512)
    assert not covers_once(*balanced_walks(counts, 512, 7, 14, 1280, planted_order=True))
