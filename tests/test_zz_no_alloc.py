"""The allocation-free decode entry, ``uocr_moe_decode_rows_static``, against ``uocr_moe_decode_rows``.

Both are called through the C ABI on the same inputs; the static entry's scratch is one device array per
GPU (no hipMalloc), so consecutive calls share it.  Checked bitwise, two calls in a row with the second on
fewer rows, for the persistent kernel (rows <= 8, int8 and bf16 layers) and the multi-kernel path
(rows > 8), then once more after the other path has used the scratch; routing outputs too.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from _gpu import DEV, bits_equal, differ, moe_for, n, t

pytestmark = pytest.mark.gpu


def _static(moe, x: torch.Tensor, routing: bool = False):
    from uocr_moe import _lib
    from uocr_moe.ops import _stream

    rows, hidden = x.shape
    out = torch.full_like(x, float("nan"))
    ids = wts = None
    if routing:
        k = moe.config.num_experts_per_tok
        ids = torch.full((rows, k), -1, dtype=torch.int32, device=x.device)
        wts = torch.full((rows, k), float("nan"), dtype=torch.float32, device=x.device)
    _lib.call("uocr_moe_decode_rows_static", out.data_ptr(), x.data_ptr(), rows, hidden, ctypes.byref(moe._layer),
              None if ids is None else ids.data_ptr(), None if wts is None else wts.data_ptr(), _stream(x))
    return (out, ids, wts) if routing else out


@pytest.fixture(scope="module")
def layers(oracle):
    return {"int8": oracle.make_layer(1, int8=True), "bf16": oracle.make_layer(2, int8=False),
            "small": oracle.make_layer(19, E=8, H=256, F=128, int8=True, std=0.05, router_std=0.1)}


@pytest.mark.parametrize(("which", "first", "second"),
                         [("int8", 8, 3), ("int8", 1, 1), ("bf16", 8, 2), ("int8", 40, 12), ("small", 64, 9)])
def test_static_entry_matches_decode_rows(oracle, layers, which, first, second) -> None:
    moe = moe_for(layers[which])
    H = moe.config.hidden_size
    rng = np.random.default_rng(first * 100 + second)
    for rows in (first, second):
        x = t(oracle.rmsnorm_rows(rng, rows, H))
        want, ids_w, wts_w = moe.decode_rows(x, routing=True)
        got, ids, wts = _static(moe, x, routing=True)
        print(f"[uocr] static decode {which} rows={rows}: {differ(n(got), n(want))} differ")
        assert bits_equal(n(got), n(want))
        assert torch.equal(ids, ids_w) and bits_equal(n(wts), n(wts_w))
    from uocr_moe import _lib

    assert _lib.fused_errors() == 0


def test_static_entry_after_the_other_path(oracle, layers) -> None:
    """Persistent, then multi-kernel, then persistent again on the shared scratch, with an oracle check."""
    moe = moe_for(layers["int8"])
    rng = np.random.default_rng(77)
    for rows in (4, 24, 2):
        xh = oracle.rmsnorm_rows(rng, rows, 1280)
        got = n(_static(moe, t(xh)))
        want = oracle.moe_decode_exact(xh, layers["int8"])[0]
        assert bits_equal(got, want), rows


def test_static_entry_refuses_beyond_its_scratch(oracle, layers) -> None:
    from uocr_moe import UocrError, _lib
    from uocr_moe.ops import _stream

    moe = moe_for(layers["int8"])
    x = torch.zeros((65, 1280), device=DEV)
    with pytest.raises(UocrError, match="rows must be in"):
        _lib.call("uocr_moe_decode_rows_static", x.data_ptr(), x.data_ptr(), 65, 1280, ctypes.byref(moe._layer),
                  None, None, _stream(x))


def test_static_entry_refuses_a_workspace_beyond_its_scratch(oracle, layers) -> None:
    """A layer the persistent kernel does not take (64 rows, top-8 of 8 experts, widths 2048) needs more than
    the 7 MiB multi-kernel part of the static scratch: refused with the size before anything is enqueued;
    the next static call is still bitwise decode_rows."""
    from uocr_moe import UocrError, _lib
    from uocr_moe.ops import _stream

    E, H, F, Fs, k, G = 8, 2048, 2048, 4096, 8, 128
    dev = DEV
    # every buffer the layer names exists at full size (never read: the call is refused first)
    w = {name: torch.empty(shape, dtype=dt, device=dev) for name, shape, dt in (
        ("router", (E, H), torch.float32), ("gate", (E, F, H), torch.int8), ("up", (E, F, H), torch.int8),
        ("down", (E, H, F), torch.int8), ("gs", (E, F, H // G), torch.float32), ("us", (E, F, H // G), torch.float32),
        ("ds", (E, H, F // G), torch.float32), ("sg", (Fs, H), torch.bfloat16), ("su", (Fs, H), torch.bfloat16),
        ("sd", (H, Fs), torch.bfloat16))}
    L = _lib.Layer(num_experts=E, hidden=H, ffn=F, shared_ffn=Fs, top_k=k, group=G, int8=1, renormalize=0,
                   router=w["router"].data_ptr(), gate_proj=w["gate"].data_ptr(), up_proj=w["up"].data_ptr(),
                   down_proj=w["down"].data_ptr(), gate_proj_scales=w["gs"].data_ptr(),
                   up_proj_scales=w["us"].data_ptr(), down_proj_scales=w["ds"].data_ptr(),
                   shared_gate=w["sg"].data_ptr(), shared_up=w["su"].data_ptr(), shared_down=w["sd"].data_ptr())
    x = torch.zeros((64, H), device=dev)
    out = torch.zeros_like(x)
    with pytest.raises(UocrError, match="need [0-9]+ bytes of scratch"):
        _lib.call("uocr_moe_decode_rows_static", out.data_ptr(), x.data_ptr(), 64, H, ctypes.byref(L), None, None,
                  _stream(x))
    moe = moe_for(layers["small"])
    xs = t(oracle.rmsnorm_rows(np.random.default_rng(91), 5, 256))
    assert bits_equal(n(_static(moe, xs)), n(moe.decode_rows(xs)))
