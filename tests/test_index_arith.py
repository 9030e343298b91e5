"""The persistent decode kernel's integer divisions by launch parameters, checked on the CPU.

``csrc/decode.hip`` replaces two kinds of integer division by cheaper forms whose exactness holds only over
ranges:

* ``task_div(x, m)`` = ``mulhi(x, m)`` with ``m = ceil(2^32 / d)`` from the host (``uocr_moe.cpp``'s
  ``magic``; 0 for ``d = 1``, where the kernel returns ``x``), in the task list's decoding and the stacked
  kernel's x polls;
* ``small_div(x, inv)`` = ``(int)(((float)x + 0.5f) * inv)`` with ``inv = 1/d`` as the host's correctly
  rounded float, or the hardware reciprocal ``v_rcp_f32`` (within 1 ulp) for the row's token.

Every divisor and every dividend that a layer admitted by ``fused_eligible`` (``uocr_moe.cpp``: B <= 8,
top_k <= 8, B * top_k <= 64, E <= 64, hidden / ffn / shared_ffn multiples of 128 up to 2048) can produce
is enumerated from the layout arithmetic of ``fused_layout`` (restated below, ``decode.hip``), and each
(x, d) pair is checked against Python's integer division, exhaustively.  The layout restated here is a
superset of what the kernel takes (the LDS bound of ``fused_eligible`` is not applied), so every admitted
pair is covered.
"""

from __future__ import annotations

import numpy as np
import pytest

WIDTHS = range(128, 2049, 128)  # hidden, ffn, shared_ffn: multiples of 128 up to 2048


def _magic(d: int) -> int:
    """The host's multiplier: ceil(2^32 / d), 0 for d <= 1."""
    return 0 if d <= 1 else ((1 << 32) + d - 1) // d


def _task_div(x: np.ndarray, d: int) -> np.ndarray:
    """The kernel's ``task_div``: the high 32 bits of the 64-bit product, or x itself when m = 0."""
    m = _magic(d)
    if m == 0:
        return x.astype(np.int64)
    return ((x.astype(np.uint64) * np.uint64(m)) >> np.uint64(32)).astype(np.int64)


def _small_div(x: np.ndarray, inv: np.float32) -> np.ndarray:
    """The kernel's ``small_div`` in float32 arithmetic (no contraction): truncation of (x + 1/2) * inv."""
    xf = x.astype(np.float32) + np.float32(0.5)
    return (xf * np.float32(inv)).astype(np.int64)


def _layout(B: int, H: int, F: int, Fs: int, sub: int) -> dict:
    """The task layout of ``fused_layout`` (decode.hip) for one layer shape."""
    gh, gf, gfs = H // 128, F // 128, Fs // 128
    c_gu = 64 // (2 * gh)
    c_dn = 64 // gf
    return {
        "gh": gh, "gf": gf, "gfs": gfs,
        "per_e_gu": -(-F // (c_gu * sub)), "per_e_dn": -(-H // c_dn),
        "cb_fs": Fs // 64, "cb_h": H // 64,
    }


def _admitted_pairs() -> dict[int, int]:
    """Divisor -> the largest dividend any admitted layer gives ``task_div`` (the division sites of
    ``task_at`` and the stacked x poll in decode.hip)."""
    need: dict[int, int] = {}

    def note(d: int, xmax: int) -> None:
        need[d] = max(need.get(d, -1), xmax)

    for B in range(1, 9):
        for topk in range(1, 9):
            if B * topk > 64:
                continue
            slots = min(64, B * topk)  # distinct selected experts, at most E <= 64
            for H in WIDTHS:
                for F in WIDTHS:
                    for Fs in WIDTHS:
                        for int8 in (False, True):
                            sub = 2 if int8 and B >= 4 else 1
                            L = _layout(B, H, F, Fs, sub)
                            note(2 * L["gh"], L["cb_fs"] * 2 * L["gh"] - 1)  # shared gate/up: chunk block
                            note(L["gh"], 2 * L["gh"] - 1)  # its projection
                            note(L["per_e_gu"], slots * L["per_e_gu"] - 1)  # routed gate/up: expert slot
                            note(B, max(L["cb_fs"], L["cb_h"]) * B - 1)  # shared folds and combines: token
                            note(L["gfs"], L["cb_h"] * L["gfs"] - 1)  # shared down: column block
                            note(L["per_e_dn"], slots * L["per_e_dn"] - 1)  # routed down: expert slot
                            note(H, B * H - 1)  # stacked x poll: element -> token row
    return need


def test_task_div_is_exact_over_every_admitted_pair() -> None:
    need = _admitted_pairs()
    assert len(need) > 20 and max(need) == 2048
    checked = 0
    for d, xmax in sorted(need.items()):
        x = np.arange(xmax + 1, dtype=np.int64)
        got = _task_div(x, d)
        bad = np.nonzero(got != x // d)[0]
        assert bad.size == 0, f"task_div({int(x[bad[0]])}, {d}) = {int(got[bad[0]])}, want {int(x[bad[0]]) // d}"
        checked += x.size
    assert checked > 10_000


def test_task_div_bound_of_the_header() -> None:
    """The header's stated range (x < 2^20 with d < 2^12) holds at its corners, and the multiplier is the
    ceiling the kernel expects."""
    for d in (2, 3, 7, 100, 1000, 4095):
        x = np.concatenate([np.arange(4096), np.arange((1 << 20) - 4096, 1 << 20)]).astype(np.int64)
        assert np.array_equal(_task_div(x, d), x // d), d
        assert _magic(d) * d >= 1 << 32 and (_magic(d) - 1) * d < 1 << 32
    assert _magic(1) == 0 and np.array_equal(_task_div(np.arange(10), 1), np.arange(10))


def test_task_div_planted_wrong_multiplier_fails() -> None:
    """A floor instead of a ceiling (a plausible mistake in ``magic``) is caught by the same check."""
    d = 7
    x = np.arange(1 << 12, dtype=np.int64)
    floor_m = (1 << 32) // d
    got = ((x.astype(np.uint64) * np.uint64(floor_m)) >> np.uint64(32)).astype(np.int64)
    assert not np.array_equal(got, x // d)


@pytest.mark.parametrize("ulps", [0, -1, 1])
def test_small_div_is_exact_below_2_16(ulps: int) -> None:
    """``small_div`` for every x < 2^16 and d <= 64 (the kernel divides lane and row indices below 64 by
    gh, gf <= 16 and top_k <= 8), with inv the correctly rounded 1/d and one ulp either side (the hardware
    reciprocal's error)."""
    x = np.arange(1 << 16, dtype=np.int64)
    for d in range(1, 65):
        inv = np.float32(1.0) / np.float32(d)
        if ulps:
            inv = np.nextafter(inv, np.float32(np.inf if ulps > 0 else 0.0), dtype=np.float32)
        got = _small_div(x, inv)
        bad = np.nonzero(got != x // d)[0]
        assert bad.size == 0, f"small_div({int(x[bad[0]])}, 1/{d} {ulps:+d} ulp) = {int(got[bad[0]])}"


def test_small_div_without_the_half_fails() -> None:
    """Dropping the +1/2 (a plausible mistake) gives wrong quotients at exact multiples, which the check
    above would catch."""
    x = np.arange(64, dtype=np.int64)
    inv = np.nextafter(np.float32(1.0) / np.float32(3), np.float32(0.0), dtype=np.float32)
    got = (x.astype(np.float32) * inv).astype(np.int64)
    assert not np.array_equal(got, x // 3)
