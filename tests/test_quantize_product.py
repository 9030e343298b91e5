"""The product's quantiser, ``uocr_moe.quantize_per_group`` (which builds every synthetic int8 layer the
benchmark times), bitwise the reference's format.

* The reference's hand-derived golden micro-tensor (tools/quantize_int8.py:787-870): RNE ties, the +-127
  edges, an all-zero group taking scale 1.0, a scale that is not a power of two.
* Bitwise the oracle's ``or_quantize_per_group`` (itself pinned to that golden) on random groups of widely
  varying magnitude, on values placed exactly on rounding ties, on zero groups and on [E, N, K] stacks.
* The reference's refusals: a partial trailing group, and NaN or Inf (tools/quantize_int8.py:309-312).
* At the served stack shape [64, 896, 1280], bitwise the oracle.

The quantiser is a HIP kernel (``uocr_quantize_per_group``): its inputs live on the GPU, so every case but
the host-side shape refusals runs under ``-m gpu``.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from test_oracle_quantize import _golden


def _q(w: np.ndarray, group: int, device: str = "cuda:0"):
    import uocr_moe

    q, s = uocr_moe.quantize_per_group(torch.from_numpy(np.ascontiguousarray(w)).to(device), group)
    return q.cpu().numpy(), s.cpu().numpy()


@pytest.mark.gpu
def test_golden_micro_tensor() -> None:
    w, want_q, want_s, group = _golden()
    q, s = _q(w, group)
    assert q.dtype == np.int8 and s.dtype == np.float32
    assert np.array_equal(s.view(np.uint32), want_s.view(np.uint32))
    assert np.array_equal(q, want_q), np.argwhere(q != want_q)


def _random_groups(seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((32, 512)) * 10.0 ** rng.uniform(-6, 2, size=(32, 1))).astype(np.float32)
    w[5, 128:256] = 0.0
    w[6, :128] = -0.0
    # exact ties: amax 127 -> scale 1.0, so k + 0.5 lands halfway between two integers
    w[7, :128] = np.float32(127.0)
    w[7, 1:128] = (np.arange(127) - 63).astype(np.float32) + np.float32(0.5)
    return w


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_bitwise_the_oracle_on_random_groups(oracle, seed: int) -> None:
    w = _random_groups(seed)
    q, s = _q(w, 128)
    q_o, s_o = oracle.quantize_per_group(w, 128)
    assert np.array_equal(s.view(np.uint32), s_o.view(np.uint32))
    assert np.array_equal(q, q_o), np.argwhere(q != q_o)[:8]
    assert q[7, 1:5].tolist() == [-62, -62, -60, -60]  # -62.5 -> -62, -61.5 -> -62, ... (half to even)


@pytest.mark.gpu
def test_bitwise_the_oracle_on_a_stack(oracle) -> None:
    rng = np.random.default_rng(7)
    stack = (rng.standard_normal((4, 24, 256)) * 0.02).astype(np.float32)
    q, s = _q(stack, 64)
    q_o, s_o = oracle.quantize_stack(stack, 64)
    assert q.shape == (4, 24, 256) and s.shape == (4, 24, 4)
    assert np.array_equal(q, q_o) and np.array_equal(s.view(np.uint32), s_o.view(np.uint32))


def test_host_side_refusals() -> None:
    """Refused before anything touches a device: a partial trailing group, and a tensor off the GPU."""
    import uocr_moe

    with pytest.raises(ValueError, match="not divisible by the group size"):
        uocr_moe.quantize_per_group(torch.zeros((2, 100)), 128)
    with pytest.raises(ValueError, match="must be on the GPU"):
        uocr_moe.quantize_per_group(torch.zeros((2, 128)), 128)


@pytest.mark.gpu
def test_refuses_nan_and_inf() -> None:
    for bad in (np.nan, np.inf, -np.inf):
        w = np.zeros((2, 128), np.float32)
        w[1, 7] = bad
        with pytest.raises(ValueError, match="NaN or Inf"):
            _q(w, 128)


@pytest.mark.gpu
def test_served_stack_on_the_gpu(oracle) -> None:
    """[64, 896, 1280] bf16 N(0, 0.02) weights quantised on the device, bitwise the oracle."""
    g = torch.Generator(device="cuda:0").manual_seed(31)
    w = (torch.randn((64, 896, 1280), generator=g, device="cuda:0") * 0.02).to(torch.bfloat16)
    import uocr_moe

    q, s = uocr_moe.quantize_per_group(w, 128)
    q_o, s_o = oracle.quantize_stack(w.float().cpu().numpy(), 128)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_o.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), q_o)
