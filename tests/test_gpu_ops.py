"""GPU parity of the reference's custom ops against the CPU oracle.

Cases mirror the reference's kernel tests (tests/test_kernels_int8.py,
tests/test_kernels_bf16.py, tests/test_kernels_dense_bf16.py), including their
real-shape smokes ([64,896,1280] / [64,1280,896] at k = 6 and 48, seeds
20260909+k and 20261003+k).  Bars:
* moe_int8_qmv, int8_dequant_expert: bit-exact against the oracle (which is
  itself pinned to the reference's operation order and closed forms);
* moe_bf16_qmv, dense_bf16_qmv: bit-exact against the oracle's chunked order,
  and within the reference's 1e-5 of float64 (the reference pins these by
  tolerance only);
* every row bitwise its value computed alone (batch invariance).
"""

from __future__ import annotations

from collections import Counter

import numpy as np
import pytest
import torch

from _gpu import bits_equal, differ, n, t

pytestmark = pytest.mark.gpu

E, N, K, GROUPS = 5, 8, 128, 4
G = K // GROUPS


@pytest.fixture(scope="module")
def ops():
    import uocr_moe

    return uocr_moe


def _rand_int8(seed, k=6, kdim=K, e=E, n_=N, groups=GROUPS):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((k, kdim)).astype(np.float32)
    ids = rng.integers(0, e, size=k).astype(np.int32)
    w = rng.integers(-127, 128, size=(e, n_, kdim)).astype(np.int8)
    scales = (10.0 ** rng.uniform(-3.0, 1.0, size=(e, n_, groups))).astype(np.float32)
    return x, ids, w, scales


def _qmv8(ops, x, ids, w, s):
    return n(ops.moe_int8_qmv(t(x), t(ids), t(w), t(s)))


# ----------------------------------------------------------------------------- moe_int8_qmv


@pytest.mark.parametrize("kdim", [K, 32], ids=["G32", "G8"])
@pytest.mark.parametrize("k", [1, 6, 48])
def test_int8_qmv_bits(ops, oracle, k, kdim) -> None:
    x, _, w, s = _rand_int8(12 + k, k=k, kdim=kdim)
    ids = np.random.default_rng(90 + k).integers(-2, E + 2, size=k).astype(np.int32)
    got = _qmv8(ops, x, ids, w, s)
    want = oracle.moe_int8_qmv(x, ids, w, s)
    print(f"[uocr] int8 qmv k={k} K={kdim}: {differ(got, want)} of {got.size} differ")
    assert bits_equal(got, want)
    assert oracle.rel_err(got, oracle.qmv_int8_f64(x, ids, w, s)) <= 1e-6


@pytest.mark.parametrize("k", [1, 6, 12, 24, 48])
def test_int8_qmv_rows_sharing_experts_are_their_lone_values(ops, oracle, k) -> None:
    x, _, w, s = _rand_int8(40 + k, k=k)
    ids = np.random.default_rng(80 + k).integers(-2, E + 2, size=k).astype(np.int32)
    if k == 48:  # expert groups wider than one 8-row tile
        assert max(Counter(np.clip(ids, 0, E - 1).tolist()).values()) > 8
    out = _qmv8(ops, x, ids, w, s)
    assert bits_equal(out, oracle.moe_int8_qmv(x, ids, w, s))
    for r in range(k):
        assert bits_equal(out[r : r + 1], _qmv8(ops, x[r : r + 1], ids[r : r + 1], w, s)), r


def test_int8_qmv_edges(ops, oracle) -> None:
    # amax edge (tests/test_kernels_int8.py:320-327)
    x, ids, _, s = _rand_int8(4)
    w = np.ascontiguousarray(np.broadcast_to(np.where(np.arange(K) % 2 == 0, 127, -127).astype(np.int8), (E, N, K)))
    assert bits_equal(_qmv8(ops, x, ids, w, s), oracle.moe_int8_qmv(x, ids, w, s))
    # zero groups and zero scales (330-341)
    x, ids, w, s = _rand_int8(5)
    w, s = w.copy(), s.copy()
    w[:, :, G : 2 * G] = 0
    s[:, :, 2] = 0.0
    assert bits_equal(_qmv8(ops, x, ids, w, s), oracle.moe_int8_qmv(x, ids, w, s))
    assert not np.any(_qmv8(ops, x, ids, np.zeros_like(w), s))
    # permutations, repeats, one expert for all (344-358)
    x, _, w, s = _rand_int8(6)
    for ids in (np.array([4, 2, 0, 1, 3, 2]), np.array([3] * 6), np.array([0, 1, 2, 3, 4, 0])):
        ids = ids.astype(np.int32)
        assert bits_equal(_qmv8(ops, x, ids, w, s), oracle.moe_int8_qmv(x, ids, w, s))
    assert np.max(np.abs(_qmv8(ops, x, np.zeros(6, np.int32), w, s) - _qmv8(ops, x, np.full(6, 4, np.int32), w, s))) > 0
    # clamp (361-370)
    x, _, w, s = _rand_int8(7)
    raw = np.array([-1, E, E + 2, -100, 2, 4], np.int32)
    assert bits_equal(_qmv8(ops, x, raw, w, s), _qmv8(ops, x, np.clip(raw, 0, E - 1).astype(np.int32), w, s))
    # group boundary sentinels (373-385)
    x = np.arange(1, K + 1, dtype=np.float32)[None, :].repeat(2, axis=0)
    ids = np.array([0, E - 1], np.int32)
    w = np.zeros((E, N, K), np.int8)
    w[:, :, ::G] = 1
    w[:, :, G - 1 :: G] = 1
    s = np.ascontiguousarray(np.broadcast_to((10.0 ** np.arange(GROUPS, dtype=np.float32))[None, None, :], (E, N, GROUPS)))
    assert bits_equal(_qmv8(ops, x, ids, w, s), oracle.moe_int8_qmv(x, ids, w, s))


def test_int8_qmv_zero_rows(ops) -> None:
    _, _, w, s = _rand_int8(13)
    out = ops.moe_int8_qmv(torch.zeros((0, K), device="cuda:0"), torch.zeros(0, dtype=torch.int32, device="cuda:0"),
                           t(w), t(s))
    assert tuple(out.shape) == (0, N)


def test_int8_qmv_refuses_a_group_miscount(ops) -> None:
    with pytest.raises(Exception, match=r"moe_int8_qmv: K must be a multiple of the group count"):
        ops.moe_int8_qmv(torch.zeros((2, 32), device="cuda:0"), torch.zeros(2, dtype=torch.int32, device="cuda:0"),
                         torch.zeros((3, 4, 32), dtype=torch.int8, device="cuda:0"),
                         torch.zeros((3, 4, 5), device="cuda:0"))


@pytest.mark.parametrize("k", [6, 48], ids=["decode", "decode_b8"])
@pytest.mark.parametrize(("n_", "kdim"), [(896, 1280), (1280, 896)], ids=["gate_up", "down"])
def test_int8_real_shape(ops, oracle, n_, kdim, k) -> None:
    """tests/test_kernels_int8.py:468-513: 64 experts, G = 128, ids from a 28-expert pool."""
    rng = np.random.default_rng(20260909 + k)
    x = rng.standard_normal((k, kdim)).astype(np.float32)
    pool = rng.permutation(64)[:28]
    ids = np.concatenate([rng.choice(pool, 6, replace=False) for _ in range(k // 6)]).astype(np.int32)
    w = rng.integers(-127, 128, size=(64, n_, kdim)).astype(np.int8)
    s = rng.uniform(1e-3, 3e-2, size=(64, n_, kdim // 128)).astype(np.float32)
    got = _qmv8(ops, x, ids, w, s)
    want = oracle.moe_int8_qmv(x, ids, w, s)
    print(f"[uocr] real-shape int8 qmv [64,{n_},{kdim}] k={k}: {differ(got, want)} differ")
    assert bits_equal(got, want)
    if k > 6:
        for b in range(0, k, 6):
            assert bits_equal(got[b : b + 6], _qmv8(ops, x[b : b + 6], ids[b : b + 6], w, s)), b
    else:
        e = int(ids[0])
        assert np.array_equal(n(ops.int8_dequant_expert(t(w), t(s), t(np.array([e], np.int32)))),
                              oracle.int8_dequant_expert(w, s, e))


# ----------------------------------------------------------------------------- int8_dequant_expert


def test_dequant_every_expert_clamp_and_zero_scale(ops, oracle) -> None:
    _, _, w, s = _rand_int8(8)
    s = s.copy()
    s[:, :, 1] = 0.0
    wt, st = t(w), t(s)
    for e in list(range(E)) + [-3, E, E + 7]:
        got = n(ops.int8_dequant_expert(wt, st, t(np.array([e], np.int32))))
        assert np.array_equal(got, oracle.int8_dequant_expert(w, s, e)), e
    assert np.any(n(ops.int8_dequant_expert(wt, st, t(np.array([2], np.int32))))[:, G : 2 * G] == 0x8000)
    f32 = n(ops.int8_dequant_expert(wt, st, t(np.array([1], np.int32)), dtype=torch.float32))
    assert bits_equal(f32, w[1].astype(np.float32) * np.repeat(s[1], G, axis=1))


def test_dequant_k30_groups_of_6(ops, oracle) -> None:
    rng = np.random.default_rng(15)
    w = rng.integers(-127, 128, size=(E, N, 30)).astype(np.int8)
    s = (10.0 ** rng.uniform(-3.0, 1.0, size=(E, N, 5))).astype(np.float32)
    for e in (0, E - 1):
        assert np.array_equal(n(ops.int8_dequant_expert(t(w), t(s), t(np.array([e], np.int32)))),
                              oracle.int8_dequant_expert(w, s, e))


def test_dequant_every_rounding_case(ops, oracle) -> None:
    """All 255 int8 values against scales whose products hit RNE ties and large exponents."""
    q = np.arange(-127, 128, dtype=np.int8)
    rng = np.random.default_rng(2)
    scales = np.concatenate([rng.uniform(1e-4, 4.0, 126), [1.0 + 2.0**-8, 1.0 + 3 * 2.0**-9, 2.0**-20, 3e30]])
    w = np.ascontiguousarray(np.broadcast_to(q, (1, len(scales), 255))).astype(np.int8)
    w = np.ascontiguousarray(np.concatenate([w, np.zeros((1, len(scales), 1), np.int8)], axis=2))  # K = 256
    s = np.repeat(scales.astype(np.float32)[None, :, None], 2, axis=2)
    got = n(ops.int8_dequant_expert(t(w), t(s), t(np.array([0], np.int32))))
    assert np.array_equal(got, oracle.int8_dequant_expert(w, s, 0))


# ----------------------------------------------------------------------------- moe_bf16_qmv


def _rand_bf16(oracle, seed, k=6, kdim=32, e=E, n_=N):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((k, kdim)).astype(np.float32)
    ids = rng.integers(0, e, size=k).astype(np.int32)
    mag = 10.0 ** rng.uniform(-3.0, 1.0, size=(e, n_, kdim))
    return x, ids, oracle.bf16_bits((mag * rng.choice([-1.0, 1.0], size=mag.shape)).astype(np.float32))


def _qmv16(ops, x, ids, w):
    return n(ops.moe_bf16_qmv(t(x), t(ids), t(w)))


@pytest.mark.parametrize("kdim", [32, 30, 1280, 896])
@pytest.mark.parametrize("k", [1, 6, 48])
def test_bf16_qmv_bits_and_tolerance(ops, oracle, k, kdim) -> None:
    x, _, w = _rand_bf16(oracle, 100 + k + kdim, k=k, kdim=kdim)
    ids = np.random.default_rng(80 + k).integers(-2, E + 2, size=k).astype(np.int32)
    got = _qmv16(ops, x, ids, w)
    assert bits_equal(got, oracle.moe_bf16_qmv_chunked(x, ids, w))
    assert oracle.rel_err(got, oracle.qmv_bf16_f64(x, ids, w)) <= 1e-5
    for r in range(0, k, max(1, k // 6)):
        assert bits_equal(got[r : r + 1], _qmv16(ops, x[r : r + 1], ids[r : r + 1], w)), r


def test_bf16_qmv_one_hot_zero_and_empty(ops, oracle) -> None:
    k, kdim = 6, 32
    x = (np.arange(k * kdim, dtype=np.float32).reshape(k, kdim) + 1.0) * np.float32(0.5)
    ids = np.array([4, 0, 2, 3, 1, 4], np.int32)
    w = np.zeros((E, N, kdim), np.float32)
    for e in range(E):
        for c in range(N):
            w[e, c, (c + 3 * e) % kdim] = 1.0
    want = np.array([[x[s, (c + 3 * ids[s]) % kdim] for c in range(N)] for s in range(k)], np.float32)
    assert np.array_equal(_qmv16(ops, x, ids, oracle.bf16_bits(w)), want)
    assert not np.any(_qmv16(ops, x, ids, np.zeros((E, N, kdim), np.uint16)))
    out = ops.moe_bf16_qmv(torch.zeros((0, kdim), device="cuda:0"), torch.zeros(0, dtype=torch.int32, device="cuda:0"),
                           t(np.zeros((E, N, kdim), np.uint16)))
    assert tuple(out.shape) == (0, N)


@pytest.mark.parametrize("k", [6, 48])
@pytest.mark.parametrize(("n_", "kdim"), [(896, 1280), (1280, 896)], ids=["gate_up", "down"])
def test_bf16_real_shape(ops, oracle, n_, kdim, k) -> None:
    rng = np.random.default_rng(20261003 + k)
    x = rng.standard_normal((k, kdim)).astype(np.float32)
    pool = rng.permutation(64)[:28]
    ids = np.concatenate([rng.choice(pool, 6, replace=False) for _ in range(k // 6)]).astype(np.int32)
    w = oracle.bf16_bits((0.05 * rng.standard_normal((64, n_, kdim))).astype(np.float32))
    got = _qmv16(ops, x, ids, w)
    assert bits_equal(got, oracle.moe_bf16_qmv_chunked(x, ids, w))
    assert oracle.rel_err(got, oracle.qmv_bf16_f64(x, ids, w)) <= 1e-5


# ----------------------------------------------------------------------------- dense_bf16_qmv


def _rand_dense(oracle, seed, m, n_, k):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((m, k)).astype(np.float32)
    mag = 10.0 ** rng.uniform(-3.0, 1.0, size=(n_, k))
    return x, oracle.kblocked(oracle.bf16_bits((mag * rng.choice([-1.0, 1.0], size=(n_, k))).astype(np.float32)))


@pytest.mark.parametrize(("m", "n_", "k"), [(1, 24, 64), (5, 24, 64), (8, 40, 96), (13, 7, 32), (9, 1792, 1280),
                                            (3, 1280, 1792), (2, 3840, 1280), (1, 129, 6848), (2, 1280, 6848),
                                            (8, 1280, 1280), (4, 3840, 1280), (6, 1280, 6848), (7, 13696, 1280),
                                            (5, 100, 1008)])
def test_dense_every_tile(ops, oracle, m, n_, k) -> None:
    x, w = _rand_dense(oracle, m * 1000 + n_ + k, m, n_, k)
    want = oracle.dense_bf16_qmv_chunked(x, w)
    alone = np.concatenate([n(ops.dense_bf16_qmv(t(x[r : r + 1]), t(w), tile=1)) for r in range(m)])
    for tile in range(1, 9):
        got = n(ops.dense_bf16_qmv(t(x), t(w), tile=tile))
        assert bits_equal(got, want), tile
        assert bits_equal(got, alone), tile
    assert oracle.rel_err(want, oracle.dense_f64(x, w)) <= 1e-5


def test_dense_eight_rows_in_graph_replays(ops, oracle) -> None:
    """8 rows of a 1280-wide projection, captured three times in a graph: replays, with eager calls between
    them, give the eager bits every time."""
    x, w = _rand_dense(oracle, 77, 8, 1280, 1280)
    xg, wg = t(x), t(w)
    eager = n(ops.dense_bf16_qmv(xg, wg))
    assert bits_equal(eager, oracle.dense_bf16_qmv_chunked(x, w))
    out = torch.empty((8, 1280), device="cuda:0")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.dense_bf16_qmv(xg, wg, out=out)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(3):
            ops.dense_bf16_qmv(xg, wg, out=out)
    for _ in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert bits_equal(n(out), eager)
        assert bits_equal(n(ops.dense_bf16_qmv(xg, wg)), eager)


def test_dense_one_hot_zero_and_empty(ops, oracle) -> None:
    m, n_, k = 6, 24, 64
    x = (np.arange(m * k, dtype=np.float32).reshape(m, k) + 1.0) * np.float32(0.5)
    w = np.zeros((n_, k), np.float32)
    for row in range(n_):
        w[row, (3 * row + 1) % k] = 1.0
    want = np.array([[x[r, (3 * c + 1) % k] for c in range(n_)] for r in range(m)], np.float32)
    wk = t(oracle.kblocked(oracle.bf16_bits(w)))
    for tile in range(1, 9):
        assert np.array_equal(n(ops.dense_bf16_qmv(t(x), wk, tile=tile)), want)
    assert not np.any(n(ops.dense_bf16_qmv(t(x), torch.zeros_like(wk))))
    assert tuple(ops.dense_bf16_qmv(torch.zeros((0, k), device="cuda:0"), wk).shape) == (0, n_)


def test_dense_column_slice_activation(ops, oracle) -> None:
    """tests/test_kernels_dense_bf16.py:121-133: a strided view gives the packed bits."""
    xw = np.random.default_rng(7).standard_normal((6, 67)).astype(np.float32)
    _, w = _rand_dense(oracle, 8, 6, 24, 64)
    view = t(xw)[:, 1:65]
    assert not view.is_contiguous()
    got = n(ops.dense_bf16_qmv(view, t(w), tile=4))
    assert bits_equal(got, n(ops.dense_bf16_qmv(t(np.ascontiguousarray(xw[:, 1:65])), t(w), tile=4)))


@pytest.mark.parametrize(("n_", "k"), [(1280, 1280), (6848, 1280), (1280, 6848), (1792, 1280), (1280, 1792),
                                        (129280, 1280)],
                         ids=["attention", "dense_gate_up", "dense_down", "shared_gate_up", "shared_down", "lm_head"])
def test_dense_real_shapes(ops, oracle, n_, k) -> None:
    """tests/test_kernels_dense_bf16.py:203-223 at M = 1 and 8; lm_head's width is tests/test_dense_tile.py:20."""
    for m in (1, 8):
        rng = np.random.default_rng(n_ + k + m)
        x = rng.standard_normal((m, k)).astype(np.float32)
        w = oracle.kblocked(oracle.bf16_bits((rng.standard_normal((n_, k), dtype=np.float32) * np.float32(0.05))))
        got = n(ops.dense_bf16_qmv(t(x), t(w)))
        assert bits_equal(got, oracle.dense_bf16_qmv_chunked(x, w))
        assert np.all(np.isfinite(got)) and np.any(got)


def test_custom_dispatch(ops, oracle) -> None:
    x, ids, w, s = _rand_int8(3)
    [out] = ops.custom("moe_int8_qmv", values=[t(x), t(ids), t(w), t(s)])
    assert bits_equal(n(out), oracle.moe_int8_qmv(x, ids, w, s))
    logits = np.random.default_rng(4).standard_normal((2, 64)).astype(np.float32)
    hist = np.array([[1, 2, 3, 1, 2], [5, 6, 7, 8, 9]], np.int32)
    [guarded] = ops.custom("ngram_block", values=[t(logits), t(hist), t(np.array([3], np.int32))])
    assert np.array_equal(n(guarded), oracle.ngram_block(logits, hist, 3))
    with pytest.raises(KeyError):
        ops.custom("flash_attention_ragged", values=[])
