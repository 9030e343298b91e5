"""GPU parity of ``paged_decode_attention`` (unlimited_ocr_max/decoder.py:425-437) against the oracle,
through the C ABI, at the reference's bar (tests/test_kv_cache.py:395-445): the output within 1e-5
relative to the float64 chain, a padding row within 1e-6 of its own value, and the store bitwise --
exactly the written slots move.

Cases: the reference test's rows (an append at row 409, a ring overwrite at row 300, a short append,
a padding row on the null page) at the real head dims (10 x 128) on a shuffled pool, at layers 0 and
2 of 3; attend lengths 1, 5, 128, 129, 640 across page and split edges; a 256-row page; the reference's
walk of two requests through warm-up and two full wraps of a 40-slot ring (tests/test_kv_cache.py:447-);
the caller's workspace and output, uint32 metadata, and the refusals.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from _gpu import n, t

pytestmark = pytest.mark.gpu

HEADS, D = 10, 128
SCALE = 1.0 / math.sqrt(D)
LAYERS, OP_LAYERS = 3, (0, 2)


def _ops():
    import uocr_moe

    return uocr_moe


def _relative(got, want) -> float:
    return float(np.max(np.abs(got.astype(np.float64) - want)) / np.max(np.abs(want)))


def _shuffled_pages(rng, pages: int, sizes: list[int]) -> list[list[int]]:
    """Hands out ``sizes`` pages per request from a shuffled free list (the last page is the null page)."""
    free = [int(p) for p in rng.permutation(pages - 1)]
    out = []
    for k in sizes:
        out.append(free[:k])
        free = free[k:]
    return out


def _lookup(page_lists, cols, null):
    lut = np.full((len(page_lists), cols), null, np.uint32)
    for b, pl in enumerate(page_lists):
        lut[b, :len(pl)] = pl
    return lut


def _step(pool_gpu, lut, attend_len, write, q, k_new, v_new, layer, *, out=None, workspace=None):
    uocr = _ops()
    kv = uocr.PagedKv(kv_blocks=pool_gpu, lookup_table=t(lut.view(np.int32)),
                      attend_lengths=t((np.asarray(attend_len, np.uint32) - 1).view(np.int32)),
                      attend_max=int(max(attend_len)), write_index=t(np.asarray(write, np.uint32).view(np.int32)))
    assert int(lut.max()) < pool_gpu.shape[0] and max(write) < lut.shape[1] * pool_gpu.shape[3]
    return uocr.paged_decode_attention(t(q), t(k_new), t(v_new), kv=kv, layer_idx=layer, scale=SCALE, out=out,
                                       workspace=workspace)


def _run_and_check(oracle, rng, pool, page_lists, attend_len, write, padding_rows=()):
    """Both op layers in turn on one pool; every row checked, then the pool bitwise."""
    B = len(attend_len)
    cols = max(len(p) for p in page_lists) + 1
    lut = _lookup(page_lists, cols, pool.shape[0] - 1)
    q, k_new, v_new = (rng.standard_normal((B, HEADS, D)).astype(np.float32) for _ in range(3))
    gpu_pool = t(pool)
    expect = pool
    for layer in OP_LAYERS:
        got = n(_step(gpu_pool, lut, attend_len, write, q, k_new, v_new, layer))
        want, expect = oracle.paged_decode_attention(q, k_new, v_new, expect, lut,
                                                     np.asarray(attend_len, np.uint32) - 1,
                                                     np.asarray(write, np.uint32), layer, SCALE)
        for b in range(B):
            if b in padding_rows:
                assert _relative(got[b], v_new[b].astype(np.float64)) <= 1e-6, (layer, b)
            else:
                assert _relative(got[b], want[b]) <= 1e-5, (layer, b, attend_len[b], _relative(got[b], want[b]))
    after = n(gpu_pool)
    assert np.array_equal(after.view(np.uint32), expect.view(np.uint32)), "the pool differs from the oracle's store"
    moved = np.argwhere(np.any(after != pool, axis=(4, 5)))
    allowed = {(int(lut[b, write[b] // pool.shape[3]]), kv, layer, write[b] % pool.shape[3])
               for b in range(B) for kv in (0, 1) for layer in OP_LAYERS}
    assert {tuple(int(v) for v in m) for m in moved} <= allowed, "the store wrote outside the rows' write slots"
    return got


#: (prefill, window, attend_len, write_index) of the reference test's rows (tests/test_kv_cache.py:380-388)
_APPEND = (282, 128, 410, 409)
_OVERWRITE = (277, 128, 405, 300)
_SHORT = (1, 128, 2, 1)


@pytest.mark.parametrize(("rows", "padding"), [([_APPEND], 0), ([_OVERWRITE], 0), ([_APPEND, _OVERWRITE, _SHORT], 1)],
                         ids=["b1-append", "b1-overwrite", "b4"])
def test_reference_rows(oracle, rows, padding) -> None:
    rng = np.random.default_rng(11 + len(rows) + padding)
    pages = 16
    pool = rng.standard_normal((pages, 2, LAYERS, 128, HEADS, D)).astype(np.float32)
    page_lists = _shuffled_pages(rng, pages, [math.ceil((p + w) / 128) for p, w, _, _ in rows])
    assert sorted(sum(page_lists, [])) != sum(page_lists, [])
    page_lists += [[]] * padding
    attend = [r[2] for r in rows] + [1] * padding
    write = [r[3] for r in rows] + [0] * padding
    _run_and_check(oracle, rng, pool, page_lists, attend, write, padding_rows=range(len(rows), len(rows) + padding))


@pytest.mark.parametrize("page_size", [128, 256])
def test_attend_lengths_across_page_and_split_edges(oracle, page_size) -> None:
    rng = np.random.default_rng(page_size)
    attend = [1, 5, 128, 129, 640, 257, 300]
    write = [0, 4, 127, 128, 639, 100, 0]      # appends, then two ring overwrites
    sizes = [math.ceil(640 / page_size) + 1] * len(attend)
    pages = sum(sizes) + 1
    pool = rng.standard_normal((pages, 2, LAYERS, page_size, HEADS, D)).astype(np.float32)
    _run_and_check(oracle, rng, pool, _shuffled_pages(rng, pages, sizes), attend, write)


def test_two_requests_walk_two_ring_wraps(oracle) -> None:
    """Prefixes of 100 and 120 rows, a 40-slot ring, two padding rows: warm-up appends, then two full wraps
    of in-place overwrites.  Each step runs layers 0 and 2; its output must be the float64 chain over the
    ring as a plain array keeps it (tests/test_kv_cache.py:211-245), and the pool's rows that ring's."""
    rng = np.random.default_rng(13)
    window, prefixes, pages = 40, (100, 120), 5
    pool = np.zeros((pages, 2, LAYERS, 128, HEADS, D), np.float32)
    page_lists = _shuffled_pages(rng, pages, [2, 2])
    rings = []
    for b, prefill in enumerate(prefixes):
        rows = rng.standard_normal((2, LAYERS, 2 * 128, HEADS, D)).astype(np.float32)  # the two pages' rows
        rows[:, :, prefill:] = 0.0
        for j, page in enumerate(page_lists[b]):
            pool[page] = rows[:, :, j * 128:(j + 1) * 128]
        rings.append({"rows": rows, "prefill": prefill, "length": prefill, "ring_pos": 0})
    gpu_pool = t(pool)
    lut = _lookup(page_lists + [[], []], 3, pages - 1)

    def write_index(r):  # kv_cache.py:89-94
        return r["length"] if r["length"] < r["prefill"] + window else r["prefill"] + r["ring_pos"]

    for step in range(window + 2 * window):
        write = [write_index(r) for r in rings] + [0, 0]
        attend = [max(r["length"], w + 1) for r, w in zip(rings, write)] + [1, 1]  # kv_cache.py:96-99
        q, k_new, v_new = (rng.standard_normal((4, HEADS, D)).astype(np.float32) for _ in range(3))
        for layer in OP_LAYERS:
            got = n(_step(gpu_pool, lut, attend, write, q, k_new, v_new, layer))
            for b, r in enumerate(rings):
                keys = r["rows"][0, layer, :attend[b]].astype(np.float64).copy()
                vals = r["rows"][1, layer, :attend[b]].astype(np.float64).copy()
                keys[write[b]], vals[write[b]] = k_new[b], v_new[b]
                s = np.einsum("hd,lhd->hl", q[b].astype(np.float64), keys) * SCALE
                w = np.exp(s - s.max(axis=-1, keepdims=True))
                w /= w.sum(axis=-1, keepdims=True)
                assert _relative(got[b], np.einsum("hl,lhd->hd", w, vals)) <= 1e-5, (step, layer, b)
            for b in (2, 3):
                assert _relative(got[b], v_new[b].astype(np.float64)) <= 1e-6
        for b, r in enumerate(rings):  # kv_cache.py:118-124: the ring advances
            r["rows"][0, :, write[b]] = k_new[b]
            r["rows"][1, :, write[b]] = v_new[b]
            if write[b] == r["length"]:
                r["length"] += 1
            else:
                r["ring_pos"] = (r["ring_pos"] + 1) % window
        if step % 20 == 19:
            after = n(gpu_pool)
            for b, r in enumerate(rings):
                held = np.concatenate([after[p] for p in page_lists[b]], axis=2)  # [2, L, rows, h, D]
                for layer in OP_LAYERS:
                    m = r["length"]
                    assert np.array_equal(held[:, layer, :m], r["rows"][:, layer, :m]), (step, b, layer)
    assert [r["ring_pos"] for r in rings] == [0, 0] and [r["length"] for r in rings] == [140, 160]


def test_caller_workspace_output_and_uint32_metadata(oracle) -> None:
    uocr = _ops()
    from uocr_moe import _lib

    rng = np.random.default_rng(3)
    pool = rng.standard_normal((11, 2, LAYERS, 128, HEADS, D)).astype(np.float32)
    page_lists = _shuffled_pages(rng, 11, [5, 5])
    lut = _lookup(page_lists, 6, 10)
    attend, write = [640, 333], [639, 200]
    q, k_new, v_new = (rng.standard_normal((2, HEADS, D)).astype(np.float32) for _ in range(3))
    own = n(_step(t(pool), lut, attend, write, q, k_new, v_new, 1))
    need = _lib.load().uocr_paged_attention_workspace_bytes(2, HEADS, 640)
    assert need == 2 * HEADS * 5 * (D + 4) * 4
    ws = torch.empty(need // 4, dtype=torch.float32, device="cuda:0")
    out = torch.full((2, HEADS, D), float("nan"), device="cuda:0")
    gpu_pool = t(pool)
    u32 = lambda a: t(np.asarray(a, np.uint32).view(np.int32)).view(torch.uint32)  # noqa: E731
    kv = uocr.PagedKv(kv_blocks=gpu_pool, lookup_table=u32(lut), attend_lengths=u32(np.array(attend) - 1),
                      attend_max=640, write_index=u32(write))
    got = uocr.paged_decode_attention(t(q), t(k_new), t(v_new), kv=kv, layer_idx=1, scale=SCALE, out=out,
                                      workspace=ws)
    assert got.data_ptr() == out.data_ptr()
    assert np.array_equal(n(out).view(np.uint32), own.view(np.uint32)), "the result depends on the workspace"
    small = torch.empty(need // 4 - 4, dtype=torch.float32, device="cuda:0")
    with pytest.raises(uocr.UocrError, match="workspace of .* bytes is smaller than the .* needed"):
        uocr.paged_decode_attention(t(q), t(k_new), t(v_new), kv=kv, layer_idx=1, scale=SCALE, workspace=small)


def test_refusals() -> None:
    uocr = _ops()
    dev = "cuda:0"
    pool = torch.zeros((3, 2, 2, 128, 2, 128), device=dev)
    meta = dict(lookup_table=torch.zeros((1, 2), dtype=torch.int32, device=dev),
                attend_lengths=torch.zeros(1, dtype=torch.int32, device=dev), attend_max=1,
                write_index=torch.zeros(1, dtype=torch.int32, device=dev))
    q = torch.zeros((1, 2, 128), device=dev)
    with pytest.raises(uocr.UocrError, match=r"layer 2 is not in the pool's 2 layers"):
        uocr.paged_decode_attention(q, q, q, kv=uocr.PagedKv(kv_blocks=pool, **meta), layer_idx=2, scale=1.0)
    with pytest.raises(uocr.UocrError, match=r"attend_max 257 is not in \[1, 256\]"):
        uocr.paged_decode_attention(q, q, q, kv=uocr.PagedKv(kv_blocks=pool, **{**meta, "attend_max": 257}),
                                    layer_idx=0, scale=1.0)
    bad = torch.zeros((3, 2, 2, 64, 2, 128), device=dev)
    with pytest.raises(uocr.UocrError, match="page_size must be a positive multiple of 128"):
        uocr.paged_decode_attention(q, q, q, kv=uocr.PagedKv(kv_blocks=bad, **meta), layer_idx=0, scale=1.0)
    with pytest.raises(ValueError, match="does not hold"):
        uocr.paged_decode_attention(q[:, :1], q[:, :1], q[:, :1], kv=uocr.PagedKv(kv_blocks=pool, **meta),
                                    layer_idx=0, scale=1.0)
    with pytest.raises(ValueError, match="not for 2 rows"):
        q2 = torch.zeros((2, 2, 128), device=dev)
        uocr.paged_decode_attention(q2, q2, q2, kv=uocr.PagedKv(kv_blocks=pool, **meta), layer_idx=0, scale=1.0)


def test_more_pairs_than_counters_merge_in_a_second_launch(oracle) -> None:
    """6560 rows x 10 heads (past the 65 536 (row, head) counters of the in-kernel merge) take the
    two-launch path; the same rows in two calls of 3280 take the in-kernel merge: the outputs agree bit for
    bit, and sampled rows match the oracle.  Every row attends 129..328 rows of three shared pages and
    stores its new row on a fourth page that nobody attends (rows there overwrite each other)."""
    rng = np.random.default_rng(21)
    rows, pages = 6560, 5
    pool = rng.standard_normal((pages, 2, 1, 128, HEADS, D)).astype(np.float32)
    lut = np.tile(np.array([[0, 1, 2, 3]], np.uint32), (rows, 1))
    attend = [129 + b % 200 for b in range(rows)]
    write = [3 * 128 + b % 128 for b in range(rows)]
    q, k_new, v_new = (rng.standard_normal((rows, HEADS, D)).astype(np.float32) for _ in range(3))
    whole = n(_step(t(pool), lut, attend, write, q, k_new, v_new, 0))
    halves = []
    for lo in (0, rows // 2):
        sl = slice(lo, lo + rows // 2)
        halves.append(n(_step(t(pool), lut[sl], attend[sl], write[sl], q[sl], k_new[sl], v_new[sl], 0)))
    assert np.array_equal(whole.view(np.uint32), np.concatenate(halves).view(np.uint32))
    pick = rng.choice(rows, 48, replace=False)
    want, _ = oracle.paged_decode_attention(q[pick], k_new[pick], v_new[pick], pool, lut[pick],
                                            np.asarray(attend, np.uint32)[pick] - 1, np.asarray(write)[pick], 0,
                                            SCALE)
    for i, b in enumerate(pick):
        assert _relative(whole[b], want[i]) <= 1e-5, b


def test_graph_replays_match_eager() -> None:
    """Three layers' calls captured in a graph (the merge counters are the device's, allocated by the eager
    call first); each of several replays, with eager work between them, gives the eager bits."""
    uocr = _ops()
    rng = np.random.default_rng(23)
    pool = rng.standard_normal((11, 2, LAYERS, 128, HEADS, D)).astype(np.float32)
    page_lists = _shuffled_pages(rng, 11, [5, 5])
    lut = _lookup(page_lists, 6, 10)
    attend, write = [640, 333], [639, 200]
    q, k_new, v_new = (t(rng.standard_normal((2, HEADS, D)).astype(np.float32)) for _ in range(3))
    gpu_pool = t(pool)
    kv = uocr.PagedKv(kv_blocks=gpu_pool, lookup_table=t(lut.view(np.int32)),
                      attend_lengths=t(np.asarray(attend, np.int32) - 1), attend_max=640,
                      write_index=t(np.asarray(write, np.int32)))
    outs = [torch.empty((2, HEADS, D), device="cuda:0") for _ in range(LAYERS)]
    from uocr_moe import _lib

    ws = torch.empty(_lib.load().uocr_paged_attention_workspace_bytes(2, HEADS, 640) // 4, device="cuda:0")

    def run():  # a captured call brings its workspace (the library's own may allocate)
        for layer in range(LAYERS):
            uocr.paged_decode_attention(q, k_new, v_new, kv=kv, layer_idx=layer, scale=SCALE, out=outs[layer],
                                        workspace=ws)

    run()
    eager = [n(o) for o in outs]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    for rep in range(4):
        for o in outs:
            o.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for layer in range(LAYERS):
            assert np.array_equal(n(outs[layer]).view(np.uint32), eager[layer].view(np.uint32)), (rep, layer)
        run()  # eager work between the replays
        torch.cuda.synchronize()
