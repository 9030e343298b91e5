"""GPU parity of the stacked decode (``uocr_moe.decode_stack``): the MoE blocks of consecutive layers
chained through the residual stream in one persistent launch give the same bits as chaining
``MoE.decode_rows`` (``x <- x + moe_l(x)``), whose layers are bitwise the oracle's
``or_moe_decode_exact`` (test_gpu_configs.py holds that check for the 11 full-size layers).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _gpu import DEV, bits_equal, differ, moe_for, n, t

pytestmark = pytest.mark.gpu


def _chain(moes, x: torch.Tensor) -> torch.Tensor:
    for m in moes:
        x = x + m.decode_rows(x)
    return x


@pytest.mark.parametrize("int8", [True, False], ids=["int8", "bf16"])
@pytest.mark.parametrize("B", [1, 3, 8])
def test_stack_matches_chained_decode_small(oracle, int8, B) -> None:
    from uocr_moe import _lib, decode_stack

    moes = [moe_for(oracle.make_layer(40 + i, E=64, H=256, F=128, int8=int8, std=0.05, router_std=0.1))
            for i in range(4)]
    x = t(oracle.rmsnorm_rows(np.random.default_rng(70 + B), B, 256))
    want = n(_chain(moes, x))
    got = n(decode_stack(moes, x))
    print(f"[uocr] stack of 4 small {'int8' if int8 else 'bf16'} layers, B={B}: {differ(got, want)} outputs differ")
    assert bits_equal(got, want)
    # the stack of one layer is one residual step
    one = n(decode_stack(moes[:1], x))
    assert bits_equal(one, n(x + moes[0].decode_rows(x)))
    assert _lib.fused_errors() == 0


@pytest.mark.parametrize("B", [1, 8])
def test_stack_eleven_full_int8_layers(B) -> None:
    """The MoE stack of one decode step (11 full-size int8 layers, each with its own weights): one
    launch, bitwise the chain of decode_rows calls; then repeated launches (the epoch advancing) and
    launches with another batch on the same stream keep the bits."""
    import bench
    from uocr_moe import _lib, decode_stack

    moes = [bench.make_layer(1000 + i, True, DEV)[0] for i in range(bench.LAYERS)]
    g = torch.Generator(device=DEV).manual_seed(90 + B)
    x = bench.rmsnorm_rows(g, B, DEV)
    want = n(_chain(moes, x))
    for _ in range(3):
        got = n(decode_stack(moes, x))
        print(f"[uocr] stack of 11 full int8 layers, B={B}: {differ(got, want)} outputs differ")
        assert bits_equal(got, want)
    other = bench.rmsnorm_rows(g, 9 - B, DEV)
    assert bits_equal(n(decode_stack(moes, other)), n(_chain(moes, other)))
    assert bits_equal(n(decode_stack(moes, x)), want)
    assert _lib.fused_errors() == 0


def test_stack_recovers_after_a_failed_launch(oracle, monkeypatch) -> None:
    """A stacked launch whose bounded waits are forced to fail from the host (a spin limit of 0; every
    kernel still ends normally) reports through the stream-ordered status flag and ``fused_errors``;
    after the reset, more stacked launches than ran before the failure (their launch tags climbing past
    every tag the failed and earlier launches left in the arenas) are each bitwise the chained calls."""
    from uocr_moe import _lib, decode_stack

    moes = [moe_for(oracle.make_layer(60 + i, E=64, H=256, F=128, int8=True, std=0.05, router_std=0.1))
            for i in range(3)]
    xs = [t(oracle.rmsnorm_rows(np.random.default_rng(600 + i), 1 + i % 4, 256)) for i in range(4)]
    wants = [n(_chain(moes, x)) for x in xs]
    flag = torch.full((1,), 7, dtype=torch.int32, device=DEV)
    k = 3
    for i in range(k):
        assert bits_equal(n(decode_stack(moes, xs[i % 4], status=flag)), wants[i % 4])
        assert int(flag.item()) == 0
    monkeypatch.setenv("UOCR_MOE_SPIN_LIMIT", "0")
    failed = n(decode_stack(moes, xs[0], status=flag))
    monkeypatch.delenv("UOCR_MOE_SPIN_LIMIT")
    assert np.isnan(failed).all()
    assert int(flag.item()) == 1
    assert _lib.fused_errors() == 1
    for i in range(2 * k + 2):
        got = n(decode_stack(moes, xs[i % 4], status=flag))
        assert bits_equal(got, wants[i % 4]), (i, differ(got, wants[i % 4]))
        assert int(flag.item()) == 0
    assert _lib.fused_errors() == 0


def test_stack_refusals(oracle) -> None:
    from uocr_moe import UocrError, decode_stack

    a = moe_for(oracle.make_layer(50, E=64, H=256, F=128, int8=True, std=0.05, router_std=0.1))
    b = moe_for(oracle.make_layer(51, E=64, H=256, F=256, int8=True, std=0.05, router_std=0.1))
    c = moe_for(oracle.make_layer(52, E=64, H=256, F=128, int8=False, std=0.05, router_std=0.1))
    x = t(oracle.rmsnorm_rows(np.random.default_rng(5), 2, 256))
    with pytest.raises(UocrError, match="differs in shape or kind"):
        decode_stack([a, b], x)
    with pytest.raises(UocrError, match="differs in shape or kind"):
        decode_stack([a, c], x)
    with pytest.raises(UocrError, match="n_layers"):
        decode_stack([a] * 13, x)
    x9 = t(oracle.rmsnorm_rows(np.random.default_rng(6), 9, 256))
    with pytest.raises(UocrError, match="rows"):
        decode_stack([a, a], x9)
