"""The router-logits kernels' work placement, restated on the CPU: every logit and every bf16 row of x
is produced exactly once.

``csrc/route.hip``'s ``k_logits_ring`` (T >= 2048, E = 64, H = 1280) maps workgroup b to token block
``tb = (b // 8 // neb) * 8 + b % 8`` and expert block ``eb = (b // 8) % neb`` (the expert blocks of a
token block on one XCD), wave w of it to tokens ``(4 tb + w) * TW ..`` and, inside the wave, slot t to
token ``t0 + (t + 2 eb) % TW``; the waves of expert block eb write the bf16 copy of their slots 0 and
1.  The grid is padded to whole rounds of 8 token blocks.  ``k_logits_topk`` (T < 2048) gives wave w
of workgroup b the four experts ``4 ((w + b) % 16) ..``.  A logit computed twice would be written
twice with the same bits (no output test notices), and one computed nowhere would leave stale
memory; these checks catch both, and planted mistakes must fail them.
"""

from __future__ import annotations

from collections import Counter

import pytest

XCDS = 8
TW, EW, E = 8, 16, 64


def ring_work(T: int, rot_step: int = 2, padded: bool = True):
    """(logit writes, xb row writes) of one k_logits_ring launch: Counters over (token, expert) and token."""
    neb = (E + EW - 1) // EW
    ntb = (T + 4 * TW - 1) // (4 * TW)
    rounds = (ntb + XCDS - 1) // XCDS if padded else ntb // XCDS
    grid = XCDS * rounds * neb
    logits, rows = Counter(), Counter()
    for b in range(grid):
        slot = b // XCDS
        tb = (slot // neb) * XCDS + b % XCDS
        eb = slot % neb
        e0 = eb * EW
        for w in range(4):
            t0 = (tb * 4 + w) * TW
            if t0 >= T or e0 >= E:
                continue
            rot = rot_step * eb
            for t in range(TW):
                tok = t0 + (t + rot) % TW
                if t < 2:
                    rows[min(tok, T - 1)] += 1  # a slot past the end stores row T - 1 again
                if tok < T:
                    for e in range(EW):
                        if e0 + e < E:
                            logits[(tok, e0 + e)] += 1
    return logits, rows


def ring_complete(T: int, **kw) -> bool:
    logits, rows = ring_work(T, **kw)
    every = all(logits[(t, e)] == 1 for t in range(T) for e in range(E)) and len(logits) == T * E
    # every row written at least once, and more than once only for the last row (the same value)
    rows_ok = all(rows[t] >= 1 for t in range(T)) and all(rows[t] == 1 for t in range(T - 1))
    return every and rows_ok


@pytest.mark.parametrize("T", [2048, 2049, 2080, 3000, 4096, 4097, 8191])
def test_ring_computes_every_logit_once(T: int) -> None:
    assert ring_complete(T)


def test_ring_places_a_token_blocks_expert_blocks_on_one_xcd() -> None:
    neb = E // EW
    ntb = 4096 // (4 * TW)
    xcd_of = {}
    for b in range(XCDS * ((ntb + XCDS - 1) // XCDS) * neb):
        slot = b // XCDS
        tb = (slot // neb) * XCDS + b % XCDS
        xcd_of.setdefault(tb, set()).add(b % XCDS)
    assert all(len(x) == 1 for x in xcd_of.values()) and len(xcd_of) == ntb


def test_ring_planted_mistakes_fail() -> None:
    # rotating by eb instead of 2 eb leaves tokens 2 eb + 1 of some blocks without their bf16 row
    assert not ring_complete(4096, rot_step=1)
    # a grid cut to whole rounds drops the last token blocks when they do not fill a round
    assert not ring_complete(2080, padded=False)


def test_fused_router_rotation_covers_every_expert_once() -> None:
    for b in range(300):
        quads = Counter(4 * ((w + b) % 16) for w in range(16))
        assert sorted(quads) == list(range(0, 64, 4)) and set(quads.values()) == {1}
