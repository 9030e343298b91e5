"""The checkpoint mapping (uocr_moe.checkpoint; unlimited_ocr_max/weight_adapters.py:121-292): a
per-expert safetensors file in the reference's names becomes the served layer, byte for byte, and
malformed files fail with the reference's reasons.  CPU tests, plus one GPU test that builds the MoE
from such a checkpoint and compares its decode and prefill bits with the directly built layer's."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import uocr_moe
from uocr_moe.checkpoint import WeightMappingError, is_int8_checkpoint, moe_layer_weights

LAYER = 3


def _bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def _unblock(kb: np.ndarray) -> np.ndarray:
    """[K/16, N, 16] -> [N, K]."""
    k16, n, b = kb.shape
    return np.ascontiguousarray(kb.transpose(1, 0, 2).reshape(n, k16 * b))


def checkpoint_of(layer, *, prefix: str = "model.") -> dict[str, torch.Tensor]:
    """The oracle's layer written the way the reference's checkpoints hold it: one tensor per expert."""
    p = f"{prefix}layers.{LAYER}.mlp."
    ck = {p + "gate.weight": torch.from_numpy(layer.router).to(torch.bfloat16)}
    for proj, stack, sc in (("gate_proj", layer.gate, layer.gate_s), ("up_proj", layer.up, layer.up_s),
                            ("down_proj", layer.down, layer.down_s)):
        for e in range(stack.shape[0]):
            w = torch.from_numpy(stack[e].copy()) if layer.int8 else _bf16(stack[e])
            ck[f"{p}experts.{e}.{proj}.weight"] = w
            if layer.int8:
                ck[f"{p}experts.{e}.{proj}.weight_scales"] = torch.from_numpy(sc[e].copy())
    for proj, kb in (("gate_proj", layer.sh_gate), ("up_proj", layer.sh_up), ("down_proj", layer.sh_down)):
        ck[f"{p}shared_experts.{proj}.weight"] = _bf16(_unblock(kb))
    ck["model.layers.4.mlp.gate.weight"] = torch.zeros(2, 2)  # another layer's tensors are left alone
    return ck


@pytest.fixture(scope="module")
def small(oracle):
    return {i8: oracle.make_layer(31, E=4, H=256, F=128, n_shared=2, topk=2, int8=i8, std=0.05, router_std=0.1)
            for i8 in (True, False)}


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.contiguous()
    return (t.view(torch.int16) if t.dtype == torch.bfloat16 else t).numpy().view(np.uint8)


@pytest.mark.parametrize("int8", [True, False], ids=["int8", "bf16"])
@pytest.mark.parametrize("prefix", ["model.", ""])
def test_round_trip_through_a_safetensors_file(small, tmp_path, int8, prefix) -> None:
    from safetensors.torch import save_file

    layer = small[int8]
    path = tmp_path / "moe.safetensors"
    save_file(checkpoint_of(layer, prefix=prefix), str(path))
    w, got_int8 = moe_layer_weights(uocr_moe.load_safetensors(path), LAYER, num_experts=4)
    assert got_int8 == int8
    assert np.array_equal(w["gate.gate_score.weight"].numpy(), layer.router)
    for proj, stack in (("gate_proj", layer.gate), ("up_proj", layer.up), ("down_proj", layer.down)):
        assert np.array_equal(_bits(w[f"experts.{proj}"]), stack.view(np.uint8))
    if int8:
        for proj, sc in (("gate_proj", layer.gate_s), ("up_proj", layer.up_s), ("down_proj", layer.down_s)):
            assert np.array_equal(w[f"experts.{proj}_scales"].numpy(), sc)
    else:
        assert not any(k.endswith("_scales") for k in w)
    for proj, kb in (("gate_proj", layer.sh_gate), ("up_proj", layer.sh_up), ("down_proj", layer.sh_down)):
        assert np.array_equal(_bits(w[f"shared_experts.{proj}.weight"]), kb.view(np.uint8))


def test_expert_gaps_counts_dtypes_and_shapes_are_errors(small) -> None:
    ck = checkpoint_of(small[True])
    p = f"model.layers.{LAYER}.mlp.experts."
    gap = {k: v for k, v in ck.items() if not k.startswith(p + "1.")}
    with pytest.raises(WeightMappingError, match="expert indices must be 0..n-1 with no gaps"):
        moe_layer_weights(gap, LAYER, num_experts=4)
    with pytest.raises(WeightMappingError, match="expected 5 experts, got 4"):
        moe_layer_weights(ck, LAYER, num_experts=5)
    shape = dict(ck)
    shape[p + "2.up_proj.weight"] = shape[p + "2.up_proj.weight"][:, :128].contiguous()
    with pytest.raises(WeightMappingError, match="disagree on shape"):
        moe_layer_weights(shape, LAYER, num_experts=4)
    bf = checkpoint_of(small[False])
    mixed = dict(bf)
    mixed[p + "0.gate_proj.weight"] = mixed[p + "0.gate_proj.weight"].float()
    with pytest.raises(WeightMappingError, match="disagree on dtype"):
        moe_layer_weights(mixed, LAYER, num_experts=4)
    with pytest.raises(WeightMappingError, match="gate.weight: not in the checkpoint"):
        moe_layer_weights({k: v for k, v in ck.items() if not k.endswith("mlp.gate.weight")}, LAYER, num_experts=4)


def test_half_quantized_files_are_errors(small) -> None:
    """weight_adapters.py:186-219: every way of mixing the two forms is refused, with its reason."""
    ck = checkpoint_of(small[True])
    p = f"model.layers.{LAYER}.mlp.experts."
    no_scales = {k: v for k, v in ck.items() if not k.endswith("_scales")}
    with pytest.raises(WeightMappingError, match="int8 expert weights without weight_scales"):
        is_int8_checkpoint(no_scales)
    one_missing = {k: v for k, v in ck.items() if k != p + "3.down_proj.weight_scales"}
    with pytest.raises(WeightMappingError, match="half-quantized checkpoint: no weight_scales for"):
        is_int8_checkpoint(one_missing)
    orphan = {k: v for k, v in ck.items() if k != p + "2.gate_proj.weight"}
    with pytest.raises(WeightMappingError, match="weight_scales without an expert weight"):
        is_int8_checkpoint(orphan)
    bf = checkpoint_of(small[False])
    bf[p + "0.gate_proj.weight_scales"] = ck[p + "0.gate_proj.weight_scales"]
    with pytest.raises(WeightMappingError, match="not int8"):
        is_int8_checkpoint(bf)
    assert is_int8_checkpoint(ck) and not is_int8_checkpoint(checkpoint_of(small[False]))


@pytest.mark.gpu
def test_moe_from_checkpoint_decodes_like_the_direct_layer(oracle, small) -> None:
    from _gpu import bits_equal, moe_for, n, t

    for int8 in (True, False):
        layer = small[int8]
        direct = moe_for(layer)
        loaded = uocr_moe.moe_from_checkpoint(checkpoint_of(layer), LAYER, num_experts=4, top_k=layer.topk)
        x = t(oracle.rmsnorm_rows(np.random.default_rng(5), 3, 256))
        assert bits_equal(n(loaded.decode_rows(x)), n(direct.decode_rows(x)))
        assert bits_equal(n(loaded(x)), n(direct(x)))


def test_stack_refusals_name_the_stack_in_the_reference_format(small) -> None:
    """The texts tests/test_weight_adapters.py:120-147 match: the stack's name, then the reason with the
    offending dtypes, shapes or counts listed in sorted order."""
    p = f"model.layers.{LAYER}.mlp.experts."
    bf = checkpoint_of(small[False])
    mixed = dict(bf)
    mixed[p + "2.up_proj.weight"] = mixed[p + "2.up_proj.weight"].float()
    with pytest.raises(WeightMappingError) as info:
        moe_layer_weights(mixed, LAYER, num_experts=4)
    assert str(info.value) == f"layers.{LAYER}.mlp.experts.up_proj: the experts disagree on dtype: ['bfloat16', 'float32']"
    half = dict(bf)
    half[p + "2.up_proj.weight"] = half[p + "2.up_proj.weight"][:, :128].contiguous()
    with pytest.raises(WeightMappingError) as info:
        moe_layer_weights(half, LAYER, num_experts=4)
    assert str(info.value) == f"layers.{LAYER}.mlp.experts.up_proj: the experts disagree on shape: [(128, 128), (128, 256)]"
    ck = checkpoint_of(small[True])
    short = {k: v for k, v in ck.items() if not k.startswith(p + "3.")}
    with pytest.raises(WeightMappingError) as info:
        moe_layer_weights(short, LAYER, num_experts=4)
    assert str(info.value) == f"layers.{LAYER}.mlp.experts.gate_proj: expected 4 experts, got 3"
    gap = {k: v for k, v in ck.items() if not k.startswith(p + "0.")}
    with pytest.raises(WeightMappingError) as info:
        moe_layer_weights(gap, LAYER, num_experts=4)
    assert str(info.value) == (f"layers.{LAYER}.mlp.experts.gate_proj: expert indices must be 0..n-1 with no gaps, "
                               "got [1, 2, 3]")


def test_form_refusals_list_the_offenders(small) -> None:
    """The four half-quantized refusals list the offending tensors by their checkpoint names (the first 20,
    sorted), scales named with their suffix."""
    p = f"model.layers.{LAYER}.mlp.experts."
    ck = checkpoint_of(small[True])
    orphan = {k: v for k, v in ck.items() if k not in (p + "2.gate_proj.weight", p + "0.up_proj.weight")}
    with pytest.raises(WeightMappingError) as info:
        is_int8_checkpoint(orphan)
    assert str(info.value) == ("weight_scales without an expert weight to scale: "
                               f"['{p}0.up_proj.weight_scales', '{p}2.gate_proj.weight_scales']")
    bare = {k: v for k, v in ck.items() if k != p + "1.down_proj.weight_scales"}
    with pytest.raises(WeightMappingError) as info:
        is_int8_checkpoint(bare, LAYER)
    assert str(info.value) == f"half-quantized checkpoint: no weight_scales for ['{p}1.down_proj.weight']"
    assert not is_int8_checkpoint(ck, LAYER + 1)  # another layer holds no experts: nothing to judge
