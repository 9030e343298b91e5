"""The oracle's quantiser against the reference's hand-derived golden micro-tensor.

The golden values (``tests/golden/quantize_golden.json``) are the reference's own
known answers (tools/quantize_int8.py:787-870): RNE ties, the +-127 edges, an
all-zero group taking scale 1.0, a scale that is not a power of two, and a value
that underflows to 0. The random cases check the properties the format fixes
(tools/quantize_int8.py:54-70): |q| <= 127, the group amax maps to +-127, and
|q*scale - w| <= scale/2.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden" / "quantize_golden.json"


def _golden():
    g = json.loads(GOLDEN.read_text())
    w = np.zeros(g["shape"], np.float32)
    q = np.zeros(g["shape"], np.int8)
    for row, col, value, expect in g["nonzero"]:
        w[row, col] = value
        q[row, col] = expect
    scales = np.array([[float.fromhex(v) for v in row] for row in g["scales_hex"]], np.float32)
    return w, q, scales, g["group"]


def test_golden_micro_tensor(oracle) -> None:
    w, want_q, want_s, group = _golden()
    q, s = oracle.quantize_per_group(w, group)
    assert np.array_equal(s.view(np.uint32), want_s.view(np.uint32)), (s, want_s)
    assert np.array_equal(q, want_q), np.argwhere(q != want_q)


def test_golden_has_the_documented_edge_cases() -> None:
    w, q, s, _ = _golden()
    assert s[0, 1] == 1.0 and not np.any(w[0, 128:])  # zero group -> scale 1.0, q 0
    assert s[1, 0] != 2.0 ** np.round(np.log2(s[1, 0]))  # a non power of two scale
    assert q[0, 3] == 0 and q[0, 4] == 2  # 0.5 and 1.5 ties to even


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_groups_hold_the_format_invariants(oracle, seed: int) -> None:
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((16, 384)) * 10.0 ** rng.uniform(-4, 1, size=(16, 1))).astype(np.float32)
    w[3, 128:256] = 0.0
    q, s = oracle.quantize_per_group(w, 128)
    assert q.min() >= -127
    grouped = w.reshape(16, 3, 128)
    amax = np.abs(grouped).max(axis=2)
    assert np.array_equal(s, np.where(amax == 0, np.float32(1), amax / np.float32(127)).astype(np.float32))
    qg = q.reshape(16, 3, 128).astype(np.int32)
    at_amax = np.abs(grouped) == amax[..., None]
    assert np.all(np.abs(qg[at_amax & (amax[..., None] > 0)]) == 127)
    err = np.abs(qg * s[..., None].astype(np.float64) - grouped)
    assert np.all(err <= s[..., None] * (0.5 + 1e-6))
    assert not np.any(q[3, 128:256]) and s[3, 1] == 1.0


def test_refuses_a_partial_group(oracle) -> None:
    with pytest.raises(ValueError):
        oracle.quantize_per_group(np.zeros((2, 100), np.float32), 128)
