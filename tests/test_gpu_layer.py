"""GPU parity of the MoE block (gate, decode layer, prefill layer) against the CPU oracle.

* gate: ids and weights bitwise the oracle's ``or_moe_gate`` (which is pinned to
  the float64 softmax + stable argsort); ties go to the lower id.
* decode (``MoE.decode_rows``): bitwise the oracle's ``or_moe_decode_exact``, and
  within the reference's module bars of the float64 layer (cosine >= 0.99999,
  rel <= 1e-4; tests/test_decoder_int8.py:740-807); rows bitwise their one-row
  values.
* prefill (``MoE.__call__``): expert ids bitwise the oracle gate; output within
  max relative error 1e-2 of the float64 layer on the reference's prefill
  weights, ``bf16_rne(f32(q) * scale)`` (the int8 path's int8_dequant_expert values;
  decoder.py:568-584) -- the north-star tolerance for the bf16-MFMA layer.
  Shapes: the served layer (64 experts, 1280/896, 2 shared) at T = 64, 512 and
  2048 on RMS-normalised rows (near-uniform routing), and T = 512 with the
  adversarial routing (all tokens on experts 0-5).  The benchmark's skewed
  workloads (Zipf routing at T = 512 and 4096, the T = 4096 adversarial case)
  and the chained 11-layer decode are in test_gpu_configs.py.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _gpu import DEV, bits_equal, differ, moe_for, n, t

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def small(oracle):
    return {i8: oracle.make_layer(19, E=8, H=256, F=128, int8=i8, std=0.05, router_std=0.1) for i8 in (True, False)}


@pytest.fixture(scope="module")
def full_int8(oracle):
    return oracle.make_layer(1, int8=True)


@pytest.fixture(scope="module")
def full_bf16(oracle):
    return oracle.make_layer(2, int8=False)


# ----------------------------------------------------------------------------- gate


@pytest.mark.parametrize("T", [1, 8, 64, 300, 2049, 2111, 4096])
def test_gate_bitwise(oracle, T) -> None:
    from uocr_moe import gate

    rng = np.random.default_rng(T)
    x = oracle.rmsnorm_rows(rng, T, 1280)
    router = oracle.bf16_values(oracle.bf16_bits(rng.standard_normal((64, 1280), dtype=np.float32) * np.float32(0.02)))
    idx, wts = gate(t(x), t(router), 6)
    ids_o, wts_o = oracle.moe_gate(x, router, 6)
    assert np.array_equal(n(idx), ids_o.astype(np.int64))
    assert bits_equal(n(wts), wts_o)


@pytest.mark.parametrize(("T", "H", "E"), [(3, 100, 64), (20, 100, 40), (5, 2112, 64), (20, 2112, 40)])
def test_gate_general_widths(oracle, T, H, E) -> None:
    """H that is not a multiple of 64, or above 2048, takes the general logits kernel (lanes past H add +0;
    4 tokens x 1 expert or 16 x 4 per wave); E = 40 leaves part of the last expert block empty."""
    from uocr_moe import gate

    rng = np.random.default_rng(T * 7 + H)
    x = oracle.rmsnorm_rows(rng, T, H)
    router = rng.standard_normal((E, H), dtype=np.float32) * np.float32(0.05)
    idx, wts = gate(t(x), t(router), 6)
    ids_o, wts_o = oracle.moe_gate(x, router, 6)
    assert np.array_equal(n(idx), ids_o.astype(np.int64))
    assert bits_equal(n(wts), wts_o)


def test_gate_ties_and_renorm(oracle) -> None:
    from uocr_moe import gate

    x = np.ones((2, 64), np.float32)
    router = np.zeros((8, 64), np.float32)
    router[[1, 5, 6], :] = 0.01
    idx, wts = gate(t(x), t(router), 6)
    assert n(idx)[0].tolist() == [1, 5, 6, 0, 2, 3]
    idx, wts = gate(t(x), t(router), 6, renormalize=True)
    _, w_o = oracle.moe_gate(x, router, 6, renorm=True)
    assert bits_equal(n(wts), w_o)


# ----------------------------------------------------------------------------- decode


@pytest.fixture(params=["fused", "multi"])
def decode_path(request, monkeypatch):
    """The persistent one-kernel decode (B <= 8) and the multi-kernel decode: same bits."""
    if request.param == "multi":
        monkeypatch.setenv("UOCR_MOE_DECODE", "multi")
    else:
        monkeypatch.delenv("UOCR_MOE_DECODE", raising=False)
    yield request.param
    if request.param == "fused":
        from uocr_moe import _lib

        assert _lib.fused_errors() == 0


@pytest.mark.parametrize("int8", [True, False], ids=["int8", "bf16"])
def test_decode_small_layer_bitwise(oracle, small, int8, decode_path) -> None:
    layer = small[int8]
    moe = moe_for(layer)
    x = np.random.default_rng(23).standard_normal((8, 256)).astype(np.float32)
    out, ids, wts = moe.decode_rows(t(x), routing=True)
    want, ids_o, wts_o = oracle.moe_decode_exact(x, layer)
    print(f"[uocr] decode small {'int8' if int8 else 'bf16'} {decode_path}: {differ(n(out), want)} differ")
    assert np.array_equal(n(ids), ids_o) and bits_equal(n(wts), wts_o)
    assert bits_equal(n(out), want)


@pytest.mark.parametrize("B", [1, 2, 3, 8])  # 1 and 2 take the shared-first task order
def test_decode_full_int8_bitwise(oracle, full_int8, B, decode_path) -> None:
    moe = moe_for(full_int8)
    x = oracle.rmsnorm_rows(np.random.default_rng(100 + B), B, 1280)
    out, ids, wts = moe.decode_rows(t(x), routing=True)
    got = n(out)
    want, ids_o, wts_o = oracle.moe_decode_exact(x, full_int8)
    print(f"[uocr] decode int8 B={B} {decode_path}: {differ(got, want)} of {got.size} differ")
    assert np.array_equal(n(ids), ids_o)
    assert bits_equal(got, want)
    exact = oracle.moe_layer_f64(x, full_int8, ids_o, wts_o)
    assert min(oracle.cosine(got[i], exact[i]) for i in range(B)) >= 0.99999
    assert oracle.rel_err(got, exact) <= 1e-4
    if B > 1:
        single = np.concatenate([n(moe.decode_rows(t(x[i : i + 1]))) for i in range(B)])
        assert bits_equal(got, single)


def test_decode_routing_ties(oracle, full_int8, decode_path) -> None:
    """Equal router logits on the decode path: token 0 has two pairs of tied experts (3 = 9 and
    20 = 40, identical router rows) on top, token 1 is all zeros (all 64 logits tie: experts 0-5),
    token 2 has none; ids, weights and outputs bitwise the oracle's (ties to the lower id)."""
    import dataclasses

    x = oracle.rmsnorm_rows(np.random.default_rng(31), 3, 1280)
    x[0, 0] = 10.0
    x[1, :] = 0.0
    router = full_int8.router.copy()
    router[:, 0] = 0.0
    router[[3, 20], 0] = 1.0
    router[9] = router[3]
    router[40] = router[20]
    tied = dataclasses.replace(full_int8, router=np.ascontiguousarray(router))
    moe = moe_for(tied)
    for B in (1, 3):
        out, ids, wts = moe.decode_rows(t(x[:B]), routing=True)
        want, ids_o, wts_o = oracle.moe_decode_exact(x[:B], tied)
        assert np.array_equal(n(ids), ids_o) and bits_equal(n(wts), wts_o)
        assert bits_equal(n(out), want)
    assert ids_o[0, :4].tolist() == [3, 9, 20, 40]
    assert ids_o[1].tolist() == [0, 1, 2, 3, 4, 5]


@pytest.mark.parametrize("B", [1, 2, 8])
def test_decode_full_bf16_bitwise(oracle, full_bf16, B, decode_path) -> None:
    moe = moe_for(full_bf16)
    x = oracle.rmsnorm_rows(np.random.default_rng(200 + B), B, 1280)
    got = n(moe.decode_rows(t(x)))
    want, ids_o, wts_o = oracle.moe_decode_exact(x, full_bf16)
    assert bits_equal(got, want)
    exact = oracle.moe_layer_f64(x, full_bf16, ids_o, wts_o)
    assert oracle.rel_err(got, exact) <= 1e-4


def test_decode_repeated_calls_and_graph_replays(oracle, small) -> None:
    """The persistent kernel leaves its control words clean: back-to-back launches, eager and
    captured in a HIP graph replayed several times with eager work between replays, all bitwise."""
    layer = small[True]
    moe = moe_for(layer)
    xs = [np.random.default_rng(60 + i).standard_normal((1 + i % 8, 256)).astype(np.float32) for i in range(12)]
    want = [oracle.moe_decode_exact(x, layer)[0] for x in xs]
    for x, w in zip(xs, want):
        assert bits_equal(n(moe.decode_rows(t(x))), w)
    xg = t(xs[3])
    ws = moe.workspace(xg.shape[0], prefill=False)
    moe.decode_rows(xg, workspace=ws)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outg = moe.decode_rows(xg, workspace=ws)
    for _ in range(4):
        graph.replay()
        assert bits_equal(n(outg), want[3])
        assert bits_equal(n(moe.decode_rows(t(xs[5]))), want[5])
    from uocr_moe import _lib

    assert _lib.fused_errors() == 0


def test_decode_batch_of_64_and_workspace(oracle, small) -> None:
    layer = small[True]
    moe = moe_for(layer)
    x = np.random.default_rng(5).standard_normal((64, 256)).astype(np.float32)
    ws = moe.workspace(64, prefill=False)
    got = n(moe.decode_rows(t(x), workspace=ws))
    assert bits_equal(got, oracle.moe_decode_exact(x, layer)[0])
    with pytest.raises(Exception, match="rows must be in"):
        moe.decode_rows(t(np.zeros((65, 256), np.float32)))


# ----------------------------------------------------------------------------- prefill


@pytest.mark.parametrize(("which", "T"), [("int8", 64), ("int8", 512), ("bf16", 512)])
def test_prefill_matches_float64(oracle, full_int8, full_bf16, which, T) -> None:
    layer = full_int8 if which == "int8" else full_bf16
    moe = moe_for(layer)
    x = oracle.rmsnorm_rows(np.random.default_rng(300 + T), T, 1280)
    out, ids, wts = moe(t(x), routing=True)
    ids_o, wts_o = oracle.moe_gate(x, layer.router, 6)
    assert np.array_equal(n(ids), ids_o) and bits_equal(n(wts), wts_o)
    got = n(out)
    ref = oracle.moe_layer_f64(x, layer, ids_o, wts_o, bf16_dequant=True)
    rel = oracle.rel_err(got, ref)
    print(f"[uocr] prefill {which} T={T}: rel {rel:.3e}, min cos {min(oracle.cosine(got[i], ref[i]) for i in range(T)):.6f}")
    assert rel <= 1e-2
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize(("int8", "group", "H", "F", "T"),
                         [(True, 64, 384, 256, 40), (True, 256, 512, 256, 200), (False, 128, 384, 384, 130),
                          (True, 64, 1024, 1024, 70), (True, 64, 1280, 256, 90)],
                         ids=["int8-G64-H384", "int8-G256-H512", "bf16-H384", "int8-G64-16groups", "int8-G64-20groups"])
def test_prefill_small_shapes(oracle, int8, group, H, F, T) -> None:
    """Column tiles that overhang N (down N = 384 against 256-column tiles), scale groups of 64 and 256, short
    and partial row tiles; 16 scale groups per weight row (the most a tile keeps in LDS) and 20 (gate/up on the
    fragment-load kernel, down on the LDS-staged one)."""
    layer = oracle.make_layer(40 + H + group, E=8, H=H, F=F, n_shared=1, int8=int8, std=0.05, router_std=0.1,
                              group=group)
    moe = moe_for(layer)
    x = oracle.rmsnorm_rows(np.random.default_rng(500 + T), T, H)
    out, ids, wts = moe(t(x), routing=True)
    ids_o, wts_o = oracle.moe_gate(x, layer.router, 6)
    assert np.array_equal(n(ids), ids_o)
    got = n(out)
    ref = oracle.moe_layer_f64(x, layer, ids_o, wts_o, bf16_dequant=True)
    rel = oracle.rel_err(got, ref)
    print(f"[uocr] prefill small int8={int8} G={group} H={H} F={F} T={T}: rel {rel:.3e}")
    assert rel <= 1e-2


@pytest.mark.parametrize(("T", "topk"), [(2048, 6), (2100, 20)])
def test_prefill_many_tokens_small_layer(oracle, T, topk) -> None:
    """T >= 2048 routes through the top-k counting launch (16 tokens a block) and the shared scatter;
    top-k 20 gives 320 rows a block, which the scatter ranks in two passes of 256 (a narrow layer, so the
    logits take the general tile kernel)."""
    layer = oracle.make_layer(70 + topk, E=64, H=256, F=256, n_shared=1, topk=topk, int8=True, std=0.05,
                              router_std=0.1)
    moe = moe_for(layer)
    x = oracle.rmsnorm_rows(np.random.default_rng(900 + T), T, 256)
    out, ids, wts = moe(t(x), routing=True)
    ids_o, wts_o = oracle.moe_gate(x, layer.router, topk)
    assert np.array_equal(n(ids), ids_o)
    assert bits_equal(n(wts), wts_o)
    got = n(out)
    ref = oracle.moe_layer_f64(x, layer, ids_o, wts_o, bf16_dequant=True)
    rel = oracle.rel_err(got, ref)
    print(f"[uocr] prefill small E=64 H=256 T={T} top-k {topk}: rel {rel:.3e}")
    assert rel <= 1e-2


def test_prefill_128_row_tiles(oracle, full_int8) -> None:
    """T = 2048 (12288 routed rows): the launch runs 128-row tiles."""
    moe = moe_for(full_int8)
    x = oracle.rmsnorm_rows(np.random.default_rng(2048), 2048, 1280)
    out, ids, wts = moe(t(x), routing=True)
    ids_o, wts_o = oracle.moe_gate(x, full_int8.router, 6)
    assert np.array_equal(n(ids), ids_o)
    got = n(out)
    ref = oracle.moe_layer_f64(x, full_int8, ids_o, wts_o, bf16_dequant=True)
    rel = oracle.rel_err(got, ref)
    print(f"[uocr] prefill int8 T=2048: rel {rel:.3e}")
    assert rel <= 1e-2


def test_prefill_adversarial_routing(oracle, full_int8) -> None:
    """Router logits +10 on experts 0-5 for every token: six groups of all T tokens."""
    import dataclasses

    x = oracle.rmsnorm_rows(np.random.default_rng(7), 512, 1280)
    x[:, 0] = 10.0
    router = full_int8.router.copy()
    router[:, 0] = 0.0
    router[:6, 0] = 1.0
    adv = dataclasses.replace(full_int8, router=np.ascontiguousarray(router))
    moe = moe_for(adv)
    out, ids, wts = moe(t(x), routing=True)
    ids_o, wts_o = oracle.moe_gate(x, adv.router, 6)
    assert np.array_equal(n(ids), ids_o)
    assert np.all(np.sort(ids_o, axis=1) == np.arange(6)[None, :])
    got = n(out)
    ref = oracle.moe_layer_f64(x, adv, ids_o, wts_o, bf16_dequant=True)
    assert oracle.rel_err(got, ref) <= 1e-2


@pytest.mark.parametrize("which", ["int8", "bf16"])
def test_prefill_every_tile_class(oracle, full_int8, full_bf16, which) -> None:
    """Token groups steered onto chosen expert sets give experts 100, 127, 27, 50 and 70 rows: partial row
    tiles of every active-block count for 128-row tiles (4, 4, 1, 2, 3) and 64-row tiles (2, 2, 1, 2, 1),
    each computed once."""
    import dataclasses

    layer = full_int8 if which == "int8" else full_bf16
    sizes = [100, 27, 50, 70]
    sets = [np.arange(0, 6), np.arange(3, 9), np.arange(9, 15), np.arange(15, 21)]
    T = sum(sizes)
    x = oracle.rmsnorm_rows(np.random.default_rng(11), T, 1280)
    router = layer.router.copy()
    x[:, 1:5] = 0.0
    router[:, 1:5] = 0.0
    start = 0
    for gi, (n_, st) in enumerate(zip(sizes, sets)):
        x[start:start + n_, 1 + gi] = 10.0
        router[st, 1 + gi] = 1.0
        start += n_
    steered = dataclasses.replace(layer, router=np.ascontiguousarray(router))
    moe = moe_for(steered)
    out, ids, wts = moe(t(x), routing=True)
    ids_o, wts_o = oracle.moe_gate(x, steered.router, 6)
    assert np.array_equal(n(ids), ids_o)
    counts = np.bincount(ids_o.ravel(), minlength=64)
    assert sorted(set(counts[:21].tolist())) == [27, 50, 70, 100, 127]
    got = n(out)
    ref = oracle.moe_layer_f64(x, steered, ids_o, wts_o, bf16_dequant=True)
    rel = oracle.rel_err(got, ref)
    print(f"[uocr] prefill {which} steered groups: rel {rel:.3e}")
    assert rel <= 1e-2
    assert min(oracle.cosine(got[i], ref[i]) for i in range(T)) > 0.999


def test_prefill_rows_do_not_depend_on_the_batch(oracle, full_int8) -> None:
    """A token's prefill output does not depend on which tokens share its call (row-independent tiles)."""
    moe = moe_for(full_int8)
    x = oracle.rmsnorm_rows(np.random.default_rng(9), 96, 1280)
    whole = n(moe(t(x)))
    part = n(moe(t(x[:40])))
    assert bits_equal(whole[:40], part)


@pytest.mark.parametrize("T", [512, 2048])
def test_prefill_graph_replays(oracle, full_int8, T) -> None:
    """The prefill's routing counters are cleared inside its own launches (no memset in a graph): the layer
    captured in a HIP graph, replayed several times with another eager prefill between the replays, gives
    the eager bits every time.  T = 512 takes the one-launch routing, T = 2048 the many-workgroup counts."""
    moe = moe_for(full_int8)
    rng = np.random.default_rng(T)
    x = oracle.rmsnorm_rows(rng, T, 1280)
    x2 = oracle.rmsnorm_rows(rng, T // 2, 1280)
    ws = moe.workspace(T, prefill=True)
    xg = t(x)
    want = n(moe(xg, workspace=ws))
    want2 = n(moe(t(x2)))
    assert bits_equal(n(moe(xg, workspace=ws)), want)  # deterministic back to back
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        moe(xg, workspace=ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outg = moe(xg, workspace=ws)
    for _ in range(3):
        outg.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert bits_equal(n(outg), want)
        assert bits_equal(n(moe(t(x2))), want2)


def test_unaligned_output_pointer(oracle, small) -> None:
    """The C entry points accept an out pointer that is only 4-byte aligned (the combine's one-column path):
    same bits as an aligned buffer, for the prefill and the multi-kernel decode (B = 40)."""
    import ctypes

    from uocr_moe import _lib
    from uocr_moe.ops import _stream

    layer = small[True]
    moe = moe_for(layer)
    T, H = 40, 256
    x = t(oracle.rmsnorm_rows(np.random.default_rng(77), T, H))
    for entry, prefill, ref in (("uocr_moe_forward", True, moe(x)), ("uocr_moe_decode_rows", False, moe.decode_rows(x))):
        buf = torch.zeros(T * H + 1, dtype=torch.float32, device=x.device)
        ws = moe.workspace(T, prefill)
        _lib.call(entry, buf.data_ptr() + 4, x.data_ptr(), T, H, ctypes.byref(moe._layer), None, None, ws.data_ptr(),
                  ws.numel(), _stream(x))
        assert bits_equal(n(buf[1:].view(T, H)), n(ref)), entry


def test_decode_failure_is_loud_and_recoverable(oracle, small, monkeypatch) -> None:
    """The persistent kernel's bounded waits, forced to fail from the host (a spin limit of 0: every wait
    gives up at its first check), end the launch normally with NaN outputs and the error word set; later
    launches on the slot write NaN until ``fused_errors`` reports and clears it; the next launch is bitwise
    the oracle again."""
    from uocr_moe import _lib

    layer = small[True]
    moe = moe_for(layer)
    x = np.random.default_rng(31).standard_normal((4, 256)).astype(np.float32)
    want = oracle.moe_decode_exact(x, layer)[0]
    flag = torch.full((1,), 7, dtype=torch.int32, device=DEV)
    assert bits_equal(n(moe.decode_rows(t(x), status=flag)), want)
    assert int(flag.item()) == 0
    assert _lib.fused_errors() == 0
    monkeypatch.setenv("UOCR_MOE_SPIN_LIMIT", "0")
    failed = n(moe.decode_rows(t(x), status=flag))
    monkeypatch.delenv("UOCR_MOE_SPIN_LIMIT")
    assert np.isnan(failed).all()
    assert int(flag.item()) == 1  # seen in the caller's buffer, stream-ordered, no fused_errors call
    assert np.isnan(n(moe.decode_rows(t(x), status=flag))).all()  # the slot stays poisoned
    assert int(flag.item()) == 1
    assert _lib.fused_errors() == 1  # reported, and cleared
    assert bits_equal(n(moe.decode_rows(t(x), status=flag)), want)
    assert int(flag.item()) == 0
    assert _lib.fused_errors() == 0


def test_decode_on_many_streams(oracle, small) -> None:
    """Each stream owns its control slot (no sharing past a first chunk of slots); eager persistent launches
    on different streams are ordered, so each keeps the whole device: all bitwise the oracle."""
    from uocr_moe import _lib

    layer = small[True]
    moe = moe_for(layer)
    xs = [np.random.default_rng(400 + i).standard_normal((1 + i % 8, 256)).astype(np.float32) for i in range(10)]
    want = [oracle.moe_decode_exact(x, layer)[0] for x in xs]
    streams = [torch.cuda.Stream() for _ in range(10)]
    outs = []
    for rep in range(2):
        for s, x in zip(streams, xs):
            with torch.cuda.stream(s):
                outs.append(moe.decode_rows(t(x)))
    torch.cuda.synchronize()
    for i, o in enumerate(outs):
        assert bits_equal(n(o), want[i % 10]), i
    for s in streams:
        assert _lib.fused_errors(s.cuda_stream) == 0
