"""GPU parity of the MoE block on the benchmark's own workloads, which stress the routing and tile paths.

* Prefill T = 512 with Zipf-skewed routing: the bench's inputs (``bench.zipf_prefill_inputs``: N(0, 1)
  rows whose constant feature carries a per-expert Zipf(1.1) bias through the router), so that a few
  experts take hundreds of rows and others none; int8 and bf16 experts.
* Prefill T = 4096 (8 prompts of 512), int8, with the same Zipf routing and with the adversarial routing
  (router logits +10 on experts 0-5: six groups of all 4096 rows, the 128-row tile path).
* The 11-layer int8 decode stack at B = 8: 11 independently seeded full-size layers (the bench's layers),
  chained through the residual stream (``x <- x + moe_l(x)``), each layer bitwise the oracle's
  ``or_moe_decode_exact`` applied to the same chain.
* Inputs at any alignment: x and the weight stacks as storage-offset views give the aligned call's bits
  (the reference picks its load path by alignment with the same bits, unlimited_ocr_max/kernels/loads.mojo:59-89,
  tests/test_kernels_int8.py:270-283).

Bars: expert ids bitwise the oracle gate for every row; prefill output within max relative error 1e-2 of
the float64 layer on ``bf16_rne(f32(q) * scale)`` weights (the reference's prefill values, decoder.py:568-584;
tests/test_decoder_int8.py:740-925 hold the layer to tolerances); decode bitwise.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from _gpu import DEV, bits_equal, differ, moe_for, n, t

pytestmark = pytest.mark.gpu


def _zipf_layer(oracle, layer, T: int, seed: int):
    """The bench's Zipf inputs for ``layer``: x (numpy) and the layer with the bias in its router column 0."""
    import bench

    g = torch.Generator(device=DEV).manual_seed(seed)
    x, bias = bench.zipf_prefill_inputs(g, T, DEV, seed)
    router = layer.router.copy()
    router[:, 0] = n(bias)
    return n(x), dataclasses.replace(layer, router=np.ascontiguousarray(router))


def _prefill_check(oracle, layer, x, label: str, rows=None) -> np.ndarray:
    moe = moe_for(layer)
    out, ids, wts = moe(t(x), routing=True)
    ids_o, wts_o = oracle.moe_gate(x, layer.router, layer.topk)
    assert np.array_equal(n(ids), ids_o), f"{label}: expert ids differ"
    assert bits_equal(n(wts), wts_o), f"{label}: routing weights differ"
    got = n(out)
    assert np.all(np.isfinite(got))
    ref = oracle.moe_layer_f64_grouped(x, layer, ids_o, wts_o, bf16_dequant=True, rows=rows)
    rel = oracle.rel_err(got if rows is None else got[rows], ref)
    hist = np.bincount(ids_o.ravel(), minlength=layer.gate.shape[0])
    print(f"[uocr] {label}: rel {rel:.3e}; rows per expert max {hist.max()}, empty experts {(hist == 0).sum()}")
    assert rel <= 1e-2
    return hist


@pytest.fixture(scope="module")
def full_int8(oracle):
    return oracle.make_layer(1, int8=True)


@pytest.fixture(scope="module")
def full_bf16(oracle):
    return oracle.make_layer(2, int8=False)


@pytest.mark.parametrize("which", ["int8", "bf16"])
def test_prefill_t512_zipf(oracle, full_int8, full_bf16, which) -> None:
    x, layer = _zipf_layer(oracle, full_int8 if which == "int8" else full_bf16, 512, 512)
    hist = _prefill_check(oracle, layer, x, f"prefill {which} T=512 Zipf")
    assert hist.max() > 100 and (hist == 0).sum() >= 4, hist  # the skew the workload asks for: idle experts


def test_prefill_t4096_zipf(oracle, full_int8) -> None:
    x, layer = _zipf_layer(oracle, full_int8, 4096, 4096)
    hist = _prefill_check(oracle, layer, x, "prefill int8 T=4096 Zipf")
    assert hist.max() > 1000


def test_prefill_t2049_partial_token_block(oracle, full_int8) -> None:
    """T = 2049 (Zipf): the T >= 2048 router logits kernel's last token block holds one token, its
    padding slots repeat that row, and its expert blocks each write their share of the bf16 x rows
    (a missing or misplaced row would change those tokens' outputs beyond the bar)."""
    x, layer = _zipf_layer(oracle, full_int8, 2049, 2049)
    hist = _prefill_check(oracle, layer, x, "prefill int8 T=2049 Zipf")
    assert hist.sum() == 2049 * 6


def test_prefill_t4096_adversarial(oracle, full_int8) -> None:
    """All 4096 tokens on experts 0-5 (bias +10 through the constant feature): six 4096-row groups."""
    x, layer = _zipf_layer(oracle, full_int8, 4096, 4097)
    router = layer.router.copy()
    router[:, 0] = 0.0
    router[:6, 0] = 10.0
    adv = dataclasses.replace(layer, router=np.ascontiguousarray(router))
    hist = _prefill_check(oracle, adv, x, "prefill int8 T=4096 adversarial")
    assert hist[:6].tolist() == [4096] * 6 and hist[6:].sum() == 0


def test_decode_eleven_layers_chained_b8(oracle) -> None:
    """The MoE stack of one decode step: 11 full-size int8 layers at B = 8, x <- x + moe_l(x), bitwise the
    oracle layer by layer (routing differs per layer; every layer's weights are its own)."""
    import bench

    layers = [bench.make_layer(1000 + i, True, DEV) for i in range(bench.LAYERS)]
    x0 = oracle.rmsnorm_rows(np.random.default_rng(811), 8, 1280)
    xg = t(x0)
    xh = x0.copy()
    for i, (moe, w) in enumerate(layers):
        y, ids, _ = moe.decode_rows(xg, routing=True)
        host = oracle.MoeWeights(
            router=n(w["gate.gate_score.weight"]), gate=n(w["experts.gate_proj"]), up=n(w["experts.up_proj"]),
            down=n(w["experts.down_proj"]), gate_s=n(w["experts.gate_proj_scales"]),
            up_s=n(w["experts.up_proj_scales"]), down_s=n(w["experts.down_proj_scales"]),
            sh_gate=n(w["shared_experts.gate_proj.weight"]), sh_up=n(w["shared_experts.up_proj.weight"]),
            sh_down=n(w["shared_experts.down_proj.weight"]))
        want, ids_o, _ = oracle.moe_decode_exact(xh, host)
        got = n(y)
        print(f"[uocr] chained layer {i}: {len(np.unique(ids_o))} experts, {differ(got, want)} outputs differ")
        assert np.array_equal(n(ids), ids_o), f"layer {i}: expert ids differ"
        assert bits_equal(got, want), f"layer {i}"
        xg = xg + y
        xh = (xh + want).astype(np.float32)
        assert bits_equal(n(xg), xh)
    from uocr_moe import _lib

    assert _lib.fused_errors() == 0


def _offset_copy(a: torch.Tensor, shift: int) -> torch.Tensor:
    """``a`` copied into a buffer ``shift`` elements past a 256-byte-aligned start: same values, data pointer
    off 16-byte alignment (a storage-offset view, as a caller's packed slice of a larger buffer would be)."""
    buf = torch.empty(a.numel() + shift, dtype=a.dtype, device=a.device)
    view = buf[shift:].view(a.shape)
    view.copy_(a)
    assert view.data_ptr() % 16 != 0 and view.is_contiguous()
    return view


@pytest.mark.parametrize(("int8", "T"), [(True, 64), (True, 1), (True, 8), (False, 8)],
                         ids=["int8-T64", "int8-T1", "int8-T8", "bf16-T8"])
def test_misaligned_inputs_give_the_aligned_bits(oracle, full_int8, full_bf16, int8, T) -> None:
    from uocr_moe import MoE

    layer = full_int8 if int8 else full_bf16
    moe = moe_for(layer)
    weights = {}
    for p in ("gate_proj", "up_proj", "down_proj"):
        weights[f"experts.{p}"] = _offset_copy(moe.stacks[p], 1)
        weights[f"shared_experts.{p}.weight"] = _offset_copy(moe.shared[p], 1)
        if int8:
            weights[f"experts.{p}_scales"] = _offset_copy(moe.scales[p], 1)
    weights["gate.gate_score.weight"] = _offset_copy(moe.router, 1)
    mis = MoE(moe.config, weights)
    x = oracle.rmsnorm_rows(np.random.default_rng(900 + T), T, 1280)
    xg = _offset_copy(t(x), 1)
    for entry in ("prefill", "decode"):
        run = (lambda m, v: m(v)) if entry == "prefill" else (lambda m, v: m.decode_rows(v))
        want = n(run(moe, t(x)))
        got = n(run(mis, xg))
        print(f"[uocr] misaligned {entry} int8={int8} T={T}: {differ(got, want)} differ")
        assert bits_equal(got, want), entry


def test_strided_out_is_refused(oracle) -> None:
    """An ``out=`` view that is not contiguous would be replaced by a packed temporary and never written:
    the op refuses it instead."""
    import uocr_moe

    logits = torch.zeros((4, 64), device=DEV)
    hist = torch.zeros((4, 8), dtype=torch.int32, device=DEV)
    strided = torch.zeros((64, 4), device=DEV).t()
    with pytest.raises(ValueError, match="must be contiguous"):
        uocr_moe.ngram_block(logits, hist, 2, out=strided)
    ok = torch.full((4, 64), 7.0, device=DEV)
    uocr_moe.ngram_block(logits, hist, 2, out=ok)
    assert torch.equal(ok, uocr_moe.ngram_block(logits, hist, 2))
