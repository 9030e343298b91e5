"""The oracle's MoE decode layer against the float64 layer closed form.

Bars from the reference's module tests (tests/test_decoder_int8.py:740-807):
cosine >= 0.99999 and rel <= 1e-4 against the float64 evaluation of the exact
int8 math (``q * scale``, softmax, top-6, SwiGLU, shared experts); the B = 8
rows bitwise their one-row values. The small shape is the reference's own
(hidden 256, ffn 128, 8 experts, top-6, 2 shared; tests/test_decoder_int8.py:95-105),
the large one the served layer (hidden 1280, ffn 896, 64 experts).
"""

from __future__ import annotations

import numpy as np
import pytest


@pytest.fixture(scope="module")
def small_layers(oracle):
    return {
        int8: oracle.make_layer(19, E=8, H=256, F=128, int8=int8, std=0.05, router_std=0.1)
        for int8 in (True, False)
    }


@pytest.fixture(scope="module")
def full_int8_layer(oracle):
    return oracle.make_layer(1, int8=True)


@pytest.mark.parametrize("int8", [True, False], ids=["int8", "bf16"])
def test_small_layer_exact_orders_match_float64(oracle, small_layers, int8: bool) -> None:
    layer = small_layers[int8]
    x = np.random.default_rng(23).standard_normal((8, 256)).astype(np.float32)
    out, ids, wts = oracle.moe_decode_exact(x, layer)
    exact = oracle.moe_layer_f64(x, layer, ids, wts)
    assert min(oracle.cosine(out[i], exact[i]) for i in range(8)) >= 0.99999
    assert oracle.rel_err(out, exact) <= 1e-4
    single = np.concatenate([oracle.moe_decode_exact(x[i : i + 1], layer)[0] for i in range(8)])
    assert np.array_equal(out, single)
    ref = oracle.moe_decode_refdecomp(x, layer)
    assert oracle.rel_err(ref, exact) <= 1e-4


def test_small_layer_gate_agrees_with_float64(oracle, small_layers) -> None:
    layer = small_layers[True]
    x = np.random.default_rng(24).standard_normal((64, 256)).astype(np.float32)
    _, ids, _ = oracle.moe_decode_exact(x, layer)
    ids64, _, probs = oracle.gate_f64(x, layer.router)
    ordered = -np.sort(-probs, axis=1)
    clear = (ordered[:, 5] - ordered[:, 6]) > 1e-5 * ordered[:, 0]
    assert np.array_equal(np.sort(ids[clear], 1), np.sort(ids64[clear], 1))


@pytest.mark.parametrize("B", [1, 8])
def test_full_int8_layer_matches_float64(oracle, full_int8_layer, B: int) -> None:
    x = oracle.rmsnorm_rows(np.random.default_rng(100 + B), B, 1280)
    out, ids, wts = oracle.moe_decode_exact(x, full_int8_layer)
    exact = oracle.moe_layer_f64(x, full_int8_layer, ids, wts)
    assert min(oracle.cosine(out[i], exact[i]) for i in range(B)) >= 0.99999
    assert oracle.rel_err(out, exact) <= 1e-4
    ref = oracle.moe_decode_refdecomp(x, full_int8_layer)
    assert oracle.rel_err(ref, out) <= 1e-5
    if B > 1:
        single = np.concatenate([oracle.moe_decode_exact(x[i : i + 1], full_int8_layer)[0] for i in range(B)])
        assert np.array_equal(out, single)


def test_a_wrong_expert_breaks_the_float64_match(oracle, small_layers) -> None:
    """A transposed id pair (expert swapped) must fail the layer bar."""
    layer = small_layers[True]
    x = np.random.default_rng(25).standard_normal((2, 256)).astype(np.float32)
    out, ids, wts = oracle.moe_decode_exact(x, layer)
    bad = ids.copy()
    bad[0, 0], bad[0, 5] = ids[0, 5], ids[0, 0]
    assert oracle.rel_err(out, oracle.moe_layer_f64(x, layer, bad, wts)) > 1e-3


@pytest.mark.parametrize("int8", [True, False], ids=["int8", "bf16"])
def test_grouped_float64_layer_equals_the_per_token_form(oracle, small_layers, int8: bool) -> None:
    """The expert-batched float64 layer (used at prefill sizes) is the per-token closed form up to float64
    rounding, with either dequantisation, and on a row subset; a planted wrong routing weight breaks it."""
    layer = small_layers[int8]
    x = np.random.default_rng(26).standard_normal((40, 256)).astype(np.float32)
    ids, wts = oracle.moe_gate(x, layer.router, 6)
    for bf in (False, True):
        per_token = oracle.moe_layer_f64(x, layer, ids, wts, bf16_dequant=bf)
        grouped = oracle.moe_layer_f64_grouped(x, layer, ids, wts, bf16_dequant=bf)
        assert oracle.rel_err(grouped, per_token) <= 1e-12
        rows = np.array([3, 0, 39, 17])
        sub = oracle.moe_layer_f64_grouped(x, layer, ids, wts, bf16_dequant=bf, rows=rows)
        assert oracle.rel_err(sub, per_token[rows]) <= 1e-12
    bad = wts.copy()
    bad[5, 2] *= 1.5
    assert oracle.rel_err(oracle.moe_layer_f64_grouped(x, layer, ids, bad), oracle.moe_layer_f64(x, layer, ids, wts)) > 1e-4
