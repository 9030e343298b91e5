"""The paged decode attention's oracle (oracle.paged_decode_attention), pinned without the reference
(MAX is absent here) by what does not share its formulation:

* torch's ``scaled_dot_product_attention`` in float64 over each request's rows laid out contiguously,
  with the pool filled from those rows page by page (whole-page copies, kv_cache.py:133-152's seeding)
  rather than row by row through the lookup table, and the new row substituted at the write index as
  the reference's test chain does (tests/test_kv_cache.py:339-349);
* closed forms: one attended row gives that row's value exactly (the padding row of
  tests/test_kv_cache.py:431-433); equal keys give the mean of the values;
* rows at or past ``attend_len`` do not matter, and the store changes exactly the written slots.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

P = 128
HEADS, D = 3, 128
SCALE = 1.0 / math.sqrt(D)


def _pool_from_requests(rng, requests, pages, layers, null_fill=0.0):
    """A pool holding each request's contiguous rows ``(pages list, K [L, n, h, D], V)`` page by page."""
    pool = rng.standard_normal((pages, 2, layers, P, HEADS, D)).astype(np.float32)
    pool[-1] = null_fill
    for page_list, keys, values in requests:
        for j, page in enumerate(page_list):
            pool[page, 0, :, :, :, :] = keys[:, j * P:(j + 1) * P]
            pool[page, 1, :, :, :, :] = values[:, j * P:(j + 1) * P]
    return pool


def _lookup(page_lists, cols, null):
    lut = np.full((len(page_lists), cols), null, np.uint32)
    for b, pl in enumerate(page_lists):
        lut[b, :len(pl)] = pl
    return lut


def _sdpa64(q, k, v, scale):
    """torch's attention, float64: q [h, D], k/v [n, h, D] -> [h, D]."""
    qt = torch.from_numpy(q.astype(np.float64))[:, None, :]            # [h, 1, D]
    kt = torch.from_numpy(k.astype(np.float64)).permute(1, 0, 2)        # [h, n, D]
    vt = torch.from_numpy(v.astype(np.float64)).permute(1, 0, 2)
    out = torch.nn.functional.scaled_dot_product_attention(qt, kt.contiguous(), vt.contiguous(), scale=scale)
    return out[:, 0, :].numpy()


@pytest.mark.parametrize("layer", [0, 2])
def test_matches_library_attention_over_contiguous_rows(oracle, layer) -> None:
    rng = np.random.default_rng(layer)
    layers, pages = 3, 9
    # (pages, attend_len, write_index): an append across a page edge, a ring overwrite, a short append
    shapes = [([4, 1, 6], 300, 299), ([7, 0, 3], 330, 140), ([5], 2, 1)]
    reqs = []
    for page_list, _, _ in shapes:
        n = len(page_list) * P
        reqs.append((page_list, rng.standard_normal((layers, n, HEADS, D)).astype(np.float32),
                     rng.standard_normal((layers, n, HEADS, D)).astype(np.float32)))
    pool = _pool_from_requests(rng, reqs, pages, layers)
    B = len(shapes)
    q, k_new, v_new = (rng.standard_normal((B, HEADS, D)).astype(np.float32) for _ in range(3))
    lut = _lookup([s[0] for s in shapes], 3, pages - 1)
    attend = np.array([s[1] - 1 for s in shapes], np.uint32)
    write = np.array([s[2] for s in shapes], np.uint32)
    out, after = oracle.paged_decode_attention(q, k_new, v_new, pool, lut, attend, write, layer, SCALE)
    for b, (page_list, keys, values) in enumerate(reqs):
        n, w = shapes[b][1], shapes[b][2]
        k = keys[layer, :n].copy()
        v = values[layer, :n].copy()
        k[w], v[w] = k_new[b], v_new[b]
        want = _sdpa64(q[b], k, v, SCALE)
        assert np.max(np.abs(out[b] - want)) <= 1e-12 * np.max(np.abs(want))
        page, slot = page_list[w // P], w % P
        assert np.array_equal(after[page, 0, layer, slot], k_new[b])
        assert np.array_equal(after[page, 1, layer, slot], v_new[b])
        after[page, :, layer, slot] = pool[page, :, layer, slot]
    assert np.array_equal(after, pool), "the store wrote outside the write slots"


def test_closed_forms(oracle) -> None:
    rng = np.random.default_rng(7)
    pool = rng.standard_normal((3, 2, 1, P, HEADS, D)).astype(np.float32)
    q, k_new, v_new = (rng.standard_normal((2, HEADS, D)).astype(np.float32) for _ in range(3))
    lut = np.array([[2, 2], [0, 1]], np.uint32)
    # row 0: the padding row (one row, written at the null page's slot 0): its value, exactly
    # row 1: every key equal -> uniform weights -> the mean of the values
    pool[0, 0, 0, :] = pool[0, 0, 0, 0]
    pool[1, 0, 0, :] = pool[0, 0, 0, 0]
    k_new[1] = pool[0, 0, 0, 0]
    out, _ = oracle.paged_decode_attention(q, k_new, v_new, pool, lut, np.array([0, 199], np.uint32),
                                           np.array([0, 150], np.uint32), 0, SCALE)
    assert np.array_equal(out[0], v_new[0].astype(np.float64))
    values = np.concatenate([pool[0, 1, 0], pool[1, 1, 0]])[:200].astype(np.float64)
    values[150] = v_new[1]
    np.testing.assert_allclose(out[1], values.mean(axis=0), rtol=0, atol=1e-12)


def test_rows_past_attend_len_do_not_matter(oracle) -> None:
    rng = np.random.default_rng(9)
    pool = rng.standard_normal((4, 2, 2, P, HEADS, D)).astype(np.float32)
    q, k_new, v_new = (rng.standard_normal((1, HEADS, D)).astype(np.float32) for _ in range(3))
    lut = np.array([[1, 0, 2]], np.uint32)
    args = (lut, np.array([129], np.uint32), np.array([129], np.uint32), 1, SCALE)
    base, _ = oracle.paged_decode_attention(q, k_new, v_new, pool, *args)
    planted = pool.copy()
    planted[0, :, 1, 2:] = 1e4      # logical rows 130.. of page 0
    planted[2, :, 1] = -1e4          # the third page, never reached
    planted[1, :, 0] = 1e4           # another layer
    again, _ = oracle.paged_decode_attention(q, k_new, v_new, planted, *args)
    assert np.array_equal(base, again)
    planted[0, 0, 1, 0] = 1e4        # logical row 128 is attended
    moved, _ = oracle.paged_decode_attention(q, k_new, v_new, planted, *args)
    assert not np.array_equal(base, moved)
