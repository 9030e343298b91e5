"""The CPU oracle's op restatements pinned against closed forms and the reference's known answers.

Cases follow the reference's kernel tests (tests/test_kernels_int8.py,
tests/test_kernels_bf16.py, tests/test_kernels_dense_bf16.py): small adversarial
shapes, scales over four decades, ids from ``[-2, E + 2)`` so rows share and
clamp, one-hot weights with exact answers, zero groups, ``k = 0``.

Independent checks per function:
* ``moe_int8_qmv``: float64 closed form at 1e-6, and bitwise a float64-emulated
  fma chain in the base order (the reference's own ``_qmv_base_order_fp32``
  method, tests/test_kernels_int8.py:165-197);
* bf16 GEMVs: float64 at 1e-5, one-hot rows exact, zero weights exactly zero;
* ``int8_dequant_expert``: bitwise the numpy closed form;
* ``uexp``/``silu``: libm within 2 ulp on a dense sweep;
* gate: float64 softmax + stable argsort (ids equal away from near-ties).
"""

from __future__ import annotations

from collections import Counter

import numpy as np
import pytest

E, N, K, GROUPS = 5, 8, 128, 4
G = K // GROUPS
K_SHORT = 32


def _rand_int8(seed: int, k: int = 6, kdim: int = K):
    """tests/test_kernels_int8.py:211-221."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((k, kdim)).astype(np.float32)
    ids = rng.integers(0, E, size=k).astype(np.int32)
    w = rng.integers(-127, 128, size=(E, N, kdim)).astype(np.int8)
    scales = (10.0 ** rng.uniform(-3.0, 1.0, size=(E, N, GROUPS))).astype(np.float32)
    return x, ids, w, scales


def _fma32(a, b, c):
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(np.float32)


def _qmv_base_order_emulated(O, x, ids, w, scales):
    """fp32 in the base operation order with each fma emulated in float64."""
    k = x.shape[0]
    num_experts, n, kdim = w.shape
    groups = scales.shape[2]
    gsize = kdim // groups
    out = np.empty((k, n), np.float32)
    for s in range(k):
        e = O.clamp(ids[s], num_experts)
        wf = w[e].astype(np.float32)
        acc = np.zeros(n, np.float32)
        for g in range(groups):
            gsum = np.zeros(n, np.float32)
            for kk in range(g * gsize, (g + 1) * gsize):
                gsum = _fma32(wf[:, kk], x[s, kk], gsum)
            acc = _fma32(scales[e, :, g], gsum, acc)
        out[s] = acc
    return out


# ----------------------------------------------------------------------------- int8 qmv


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_int8_qmv_random(oracle, seed: int) -> None:
    x, ids, w, scales = _rand_int8(seed)
    assert oracle.rel_err(oracle.moe_int8_qmv(x, ids, w, scales), oracle.qmv_int8_f64(x, ids, w, scales)) <= 1e-6


@pytest.mark.parametrize("kdim", [K, K_SHORT], ids=["G32", "G8"])
@pytest.mark.parametrize("k", [1, 6, 48])
def test_int8_qmv_bits_are_the_base_order(oracle, k: int, kdim: int) -> None:
    x, _, w, scales = _rand_int8(12 + k, k=k, kdim=kdim)
    ids = np.random.default_rng(90 + k).integers(-2, E + 2, size=k).astype(np.int32)
    out = oracle.moe_int8_qmv(x, ids, w, scales)
    want = _qmv_base_order_emulated(oracle, x, ids, w, scales)
    assert np.array_equal(out.view(np.uint32), want.view(np.uint32))


def test_int8_qmv_a_dropped_fma_fails_the_base_order_check(oracle) -> None:
    """The emulated chain detects a chain that rounds the product on its own."""
    x, ids, w, scales = _rand_int8(5, k=6)
    want = _qmv_base_order_emulated(oracle, x, ids, w, scales)
    e = ids[0]
    wf = w[e].astype(np.float32)
    acc = np.zeros(N, np.float32)
    for g in range(GROUPS):
        gsum = np.zeros(N, np.float32)
        for kk in range(g * G, (g + 1) * G):
            gsum = (gsum + (wf[:, kk] * x[0, kk]).astype(np.float32)).astype(np.float32)
        acc = _fma32(scales[e, :, g], gsum, acc)
    assert np.count_nonzero(acc.view(np.uint32) != want[0].view(np.uint32)) > 0


@pytest.mark.parametrize("k", [1, 6, 12, 24, 48])
def test_int8_qmv_rows_sharing_experts_are_their_lone_values(oracle, k: int) -> None:
    x, _, w, scales = _rand_int8(40 + k, k=k)
    ids = np.random.default_rng(80 + k).integers(-2, E + 2, size=k).astype(np.int32)
    if k >= 24:
        assert max(Counter(ids.tolist()).values()) > 4
    out = oracle.moe_int8_qmv(x, ids, w, scales)
    assert oracle.rel_err(out, oracle.qmv_int8_f64(x, ids, w, scales)) <= 1e-6
    for s in range(k):
        assert np.array_equal(out[s : s + 1], oracle.moe_int8_qmv(x[s : s + 1], ids[s : s + 1], w, scales)), s


def test_int8_qmv_clamp_zero_groups_sentinels(oracle) -> None:
    x, _, w, scales = _rand_int8(7)
    raw = np.array([-1, E, E + 2, -100, 2, 4], np.int32)
    assert np.array_equal(oracle.moe_int8_qmv(x, raw, w, scales), oracle.moe_int8_qmv(x, np.clip(raw, 0, E - 1), w, scales))
    x, ids, w, scales = _rand_int8(5)
    w, scales = w.copy(), scales.copy()
    w[:, :, G : 2 * G] = 0
    scales[:, :, 2] = 0.0
    assert oracle.rel_err(oracle.moe_int8_qmv(x, ids, w, scales), oracle.qmv_int8_f64(x, ids, w, scales)) <= 1e-6
    assert not np.any(oracle.moe_int8_qmv(x, ids, np.zeros_like(w), scales))
    # group boundary sentinels (tests/test_kernels_int8.py:373-385)
    x = np.arange(1, K + 1, dtype=np.float32)[None, :].repeat(2, axis=0)
    ids = np.array([0, E - 1], np.int32)
    w = np.zeros((E, N, K), np.int8)
    w[:, :, ::G] = 1
    w[:, :, G - 1 :: G] = 1
    scales = np.ascontiguousarray(np.broadcast_to((10.0 ** np.arange(GROUPS, dtype=np.float32))[None, None, :], (E, N, GROUPS)))
    got = oracle.moe_int8_qmv(x, ids, w, scales)
    want = sum(10.0**g * ((g * G + 1) + (g * G + G)) for g in range(GROUPS))
    assert np.all(got == np.float32(want))


def test_int8_qmv_zero_rows(oracle) -> None:
    _, _, w, scales = _rand_int8(13)
    assert oracle.moe_int8_qmv(np.zeros((0, K), np.float32), np.zeros(0, np.int32), w, scales).shape == (0, N)


# ----------------------------------------------------------------------------- dequant


def test_int8_dequant_every_expert_and_clamp(oracle) -> None:
    _, _, w, scales = _rand_int8(8)
    scales = scales.copy()
    scales[:, :, 1] = 0.0
    for e in list(range(E)) + [-3, E + 7]:
        ec = oracle.clamp(e, E)
        want = oracle.bf16_bits(w[ec].astype(np.float32) * np.repeat(scales[ec], G, axis=1))
        got = oracle.int8_dequant_expert(w, scales, e)
        assert np.array_equal(got, want), e
    assert np.any(oracle.int8_dequant_expert(w, scales, 2)[:, G : 2 * G] == 0x8000)  # -0.0 kept


def test_int8_dequant_k30_groups_of_6(oracle) -> None:
    rng = np.random.default_rng(15)
    w = rng.integers(-127, 128, size=(E, N, 30)).astype(np.int8)
    scales = (10.0 ** rng.uniform(-3.0, 1.0, size=(E, N, 5))).astype(np.float32)
    for e in (0, E - 1):
        want = oracle.bf16_bits(w[e].astype(np.float32) * np.repeat(scales[e], 6, axis=1))
        assert np.array_equal(oracle.int8_dequant_expert(w, scales, e), want)


# ----------------------------------------------------------------------------- bf16 qmv


def _rand_bf16(O, seed: int, k: int = 6, kdim: int = 32, num_experts: int = E, n: int = N):
    """tests/test_kernels_bf16.py:125-133."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((k, kdim)).astype(np.float32)
    ids = rng.integers(0, num_experts, size=k).astype(np.int32)
    magnitude = 10.0 ** rng.uniform(-3.0, 1.0, size=(num_experts, n, kdim))
    w = (magnitude * rng.choice([-1.0, 1.0], size=magnitude.shape)).astype(np.float32)
    return x, ids, O.bf16_bits(w)


@pytest.mark.parametrize("fn", ["moe_bf16_qmv_ref", "moe_bf16_qmv_chunked"])
@pytest.mark.parametrize("kdim", [32, 30, 1280])
def test_bf16_qmv_against_float64(oracle, fn: str, kdim: int) -> None:
    for seed in range(3):
        x, ids, w = _rand_bf16(oracle, seed, kdim=kdim)
        ids = np.random.default_rng(80 + seed).integers(-2, E + 2, size=6).astype(np.int32)
        got = getattr(oracle, fn)(x, ids, w)
        assert oracle.rel_err(got, oracle.qmv_bf16_f64(x, ids, w)) <= 1e-5


@pytest.mark.parametrize("fn", ["moe_bf16_qmv_ref", "moe_bf16_qmv_chunked"])
def test_bf16_qmv_one_hot_and_zero(oracle, fn: str) -> None:
    k, kdim = 6, 32
    x = (np.arange(k * kdim, dtype=np.float32).reshape(k, kdim) + 1.0) * np.float32(0.5)
    ids = np.array([4, 0, 2, 3, 1, 4], np.int32)
    w = np.zeros((E, N, kdim), np.float32)
    for e in range(E):
        for n in range(N):
            w[e, n, (n + 3 * e) % kdim] = 1.0
    want = np.array([[x[s, (n + 3 * ids[s]) % kdim] for n in range(N)] for s in range(k)], np.float32)
    assert np.array_equal(getattr(oracle, fn)(x, ids, oracle.bf16_bits(w)), want)
    assert not np.any(getattr(oracle, fn)(x, ids, np.zeros((E, N, kdim), np.uint16)))


# ----------------------------------------------------------------------------- dense bf16 qmv


def _rand_dense(O, seed: int, m: int, n: int, k: int):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    magnitude = 10.0 ** rng.uniform(-3.0, 1.0, size=(n, k))
    return x, O.kblocked(O.bf16_bits((magnitude * rng.choice([-1.0, 1.0], size=(n, k))).astype(np.float32)))


@pytest.mark.parametrize(("m", "n", "k"), [(1, 24, 64), (5, 24, 64), (8, 40, 96), (13, 7, 32), (3, 33, 1280)])
def test_dense_against_float64_every_tile(oracle, m: int, n: int, k: int) -> None:
    x, w = _rand_dense(oracle, m * 1000 + n + k, m, n, k)
    ref = oracle.dense_f64(x, w)
    alone = np.concatenate([oracle.dense_bf16_qmv_ref(x[r : r + 1], w, 1) for r in range(m)])
    for tile in range(1, 9):
        got = oracle.dense_bf16_qmv_ref(x, w, tile)
        assert oracle.rel_err(got, ref) <= 1e-5, tile
        assert np.array_equal(got, alone), tile
    assert oracle.rel_err(oracle.dense_bf16_qmv_chunked(x, w), ref) <= 1e-5


def test_dense_one_hot(oracle) -> None:
    m, n, k = 6, 24, 64
    x = (np.arange(m * k, dtype=np.float32).reshape(m, k) + 1.0) * np.float32(0.5)
    w = np.zeros((n, k), np.float32)
    for row in range(n):
        w[row, (3 * row + 1) % k] = 1.0
    want = np.array([[x[r, (3 * c + 1) % k] for c in range(n)] for r in range(m)], np.float32)
    wk = oracle.kblocked(oracle.bf16_bits(w))
    for tile in range(1, 9):
        assert np.array_equal(oracle.dense_bf16_qmv_ref(x, wk, tile), want)
    assert np.array_equal(oracle.dense_bf16_qmv_chunked(x, wk), want)


# ----------------------------------------------------------------------------- bf16 bits, exp, silu


def test_bf16_rne_ties_and_specials(oracle) -> None:
    import torch

    rng = np.random.default_rng(0)
    bits = np.concatenate([
        rng.integers(0, 2**32, size=200000, dtype=np.uint64).astype(np.uint32),
        (np.arange(65536, dtype=np.uint32) << 16) | 0x8000,  # exact ties
        (np.arange(65536, dtype=np.uint32) << 16) | 0x7FFF,
        (np.arange(65536, dtype=np.uint32) << 16) | 0x8001,
    ])
    vals = bits.view(np.float32)
    finite = ~np.isnan(vals)
    got = oracle.bf16_bits(vals)
    want = torch.from_numpy(vals[finite].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got[finite], want)
    assert np.all(got[~finite] == 0x7FC0)
    c = oracle.lib()
    for v in vals[:2000]:
        assert c.or_bf16_rne(float(v)) == oracle.bf16_bits(np.array([v], np.float32))[0]


def _ulp_diff(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    return np.abs(ia - ib)


def test_uexp_within_two_ulp_of_libm(oracle) -> None:
    x = np.concatenate([np.linspace(-87.0, 88.7, 2_000_001, dtype=np.float32),
                        np.random.default_rng(1).uniform(-20, 20, 200000).astype(np.float32),
                        np.array([0.0, -0.0, 1e-30, -1e-30], np.float32)])
    got = oracle.uexp_array(x)
    want = np.exp(x.astype(np.float64)).astype(np.float32)
    assert int(_ulp_diff(got, want).max()) <= 2
    assert oracle.uexp(0.0) == 1.0 and oracle.uexp(-200.0) == 0.0 and np.isinf(oracle.uexp(100.0))


def test_silu_matches_its_closed_form(oracle) -> None:
    x = np.linspace(-30, 30, 600001, dtype=np.float32)
    got = oracle.silu_array(x).astype(np.float64)
    want = x.astype(np.float64) / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) <= 4e-7
    assert oracle.silu(-200.0) == 0.0 and oracle.silu(0.0) == 0.0


# ----------------------------------------------------------------------------- gate


def test_dot_tree64_against_float64(oracle) -> None:
    rng = np.random.default_rng(3)
    for k in (1, 63, 64, 65, 1280, 1792):
        a = rng.standard_normal(k).astype(np.float32)
        b = rng.standard_normal(k).astype(np.float32)
        want = float(a.astype(np.float64) @ b.astype(np.float64))
        assert abs(oracle.dot_tree64(a, b) - want) <= 1e-6 * max(1.0, float(np.abs(a) @ np.abs(b)))


@pytest.mark.parametrize(("E_", "H"), [(64, 1280), (8, 256), (5, 64)])
def test_gate_matches_float64_softmax_topk(oracle, E_: int, H: int) -> None:
    rng = np.random.default_rng(E_ + H)
    topk = min(6, E_)
    x = rng.standard_normal((300, H)).astype(np.float32)
    router = (rng.standard_normal((E_, H)) * 0.1).astype(np.float32)
    ids, wts = oracle.moe_gate(x, router, topk)
    ids64, wts64, probs = oracle.gate_f64(x, router, topk)
    ordered = -np.sort(-probs, axis=1)
    gap = ordered[:, topk - 1] - ordered[:, topk] if E_ > topk else np.ones(len(x))
    clear = gap > 1e-5 * ordered[:, 0]
    assert clear.mean() > 0.9
    assert np.array_equal(np.sort(ids[clear], axis=1), np.sort(ids64[clear], axis=1))
    assert np.max(np.abs(wts - np.take_along_axis(probs, ids.astype(np.int64), axis=1))) <= 1e-6
    assert np.all(np.diff(wts, axis=1) <= 0)  # score order


def test_gate_ties_go_to_the_lower_id(oracle) -> None:
    x = np.ones((1, 64), np.float32)
    router = np.zeros((8, 64), np.float32)
    router[[1, 5, 6], :] = 0.01
    ids, wts = oracle.moe_gate(x, router, 6)
    assert ids[0].tolist() == [1, 5, 6, 0, 2, 3]
    assert wts[0, 0] == wts[0, 1] == wts[0, 2]


def test_gate_renormalise_flag(oracle) -> None:
    rng = np.random.default_rng(9)
    x = rng.standard_normal((10, 128)).astype(np.float32)
    router = (rng.standard_normal((16, 128)) * 0.2).astype(np.float32)
    _, w = oracle.moe_gate(x, router, 6, renorm=True)
    assert np.allclose(w.sum(axis=1), 1.0, atol=1e-6)
