"""Checkpoint tensors -> one MoE layer's weights (unlimited_ocr_max/weight_adapters.py:121-292, the MoE part).

The reference's checkpoints hold every routed expert as its own tensor and the
projections un-blocked; :class:`~uocr_moe.moe.MoE` takes the served layout.
This module maps one ``model.layers.{L}.mlp`` from the first to the second:

* ``…mlp.gate.weight`` ``[E, H]`` (bf16 on disk) -> ``gate.gate_score.weight``
  fp32, the router the reference serves in fp32 (decoder.py:19-22,227-229);
* ``…mlp.experts.{j}.{gate,up,down}_proj.weight`` ``[N, K]`` -> one
  ``experts.<proj>`` stack ``[E, N, K]`` in ascending expert index
  (weight_adapters.py:121-166), int8 or bf16 as stored;
* ``…weight_scales`` fp32 ``[N, K / 128]`` next to int8 weights ->
  ``experts.<proj>_scales`` ``[E, N, K / 128]`` (the int8 form);
* ``…mlp.shared_experts.<proj>.weight`` bf16 ``[N, K]`` -> K-blocked
  ``[K / 16, N, 16]`` (weight_adapters.py:222-233).

The checks are the reference's: expert indices ``0..n-1`` with no gaps and
exactly ``num_experts`` of them, one dtype and one shape per stack, and a
half-quantized file (scales for some experts but not all, int8 weights with no
scales, scales next to non-int8 weights) is an error, never a guess
(weight_adapters.py:186-219).  Names with or without the ``model.`` prefix are
accepted, as the reference matches both (weight_adapters.py:169-178).
"""

from __future__ import annotations

import re
from collections.abc import Mapping
from pathlib import Path

import torch

from .moe import ROUTED, MoE, MoeConfig
from .ops import kblocked

__all__ = ["WeightMappingError", "is_int8_checkpoint", "load_safetensors", "moe_from_checkpoint", "moe_layer_weights"]

_EXPERT_RE = re.compile(
    r"^(?:model\.)?layers\.(?P<layer>\d+)\.mlp\.experts\.(?P<expert>\d+)\."
    r"(?P<proj>gate_proj|up_proj|down_proj)\.weight(?P<scales>_scales)?$"
)


class WeightMappingError(RuntimeError):
    """The checkpoint's MoE tensors do not line up with one served layer."""


def load_safetensors(path: str | Path) -> dict[str, torch.Tensor]:
    """Every tensor of a safetensors file, on the CPU (bf16 stays bf16)."""
    from safetensors.torch import load_file

    return load_file(str(path), device="cpu")


def _expert_tensors(checkpoint: Mapping[str, torch.Tensor], layer: int | None = None):
    """``(weights, scales)`` keyed by ``(layer, expert, proj)``."""
    weights: dict[tuple[int, int, str], torch.Tensor] = {}
    scales: dict[tuple[int, int, str], torch.Tensor] = {}
    for name, value in checkpoint.items():
        m = _EXPERT_RE.match(name)
        if m is None or (layer is not None and int(m["layer"]) != layer):
            continue
        key = (int(m["layer"]), int(m["expert"]), m["proj"])
        (scales if m["scales"] else weights)[key] = value
    return weights, scales


def _names(keys, suffix: str = "") -> list[str]:
    return [f"model.layers.{l}.mlp.experts.{e}.{p}.weight{suffix}" for l, e, p in sorted(keys)[:20]]


def is_int8_checkpoint(checkpoint: Mapping[str, torch.Tensor], layer: int | None = None) -> bool:
    """Whether the routed experts are int8 with per-group ``weight_scales`` (False for the bf16 form)."""
    weights, scales = _expert_tensors(checkpoint, layer)
    quantized = {k for k, v in weights.items() if v.dtype == torch.int8}
    if not scales:
        if quantized:
            raise WeightMappingError(f"int8 expert weights without weight_scales: {_names(quantized)}")
        return False
    orphans = set(scales) - set(weights)
    if orphans:
        raise WeightMappingError(f"weight_scales without an expert weight to scale: {_names(orphans, '_scales')}")
    unquantized = set(weights) - quantized
    if unquantized:
        found = sorted({str(weights[k].dtype).removeprefix("torch.") for k in unquantized})
        raise WeightMappingError(
            f"weight_scales are present but these expert weights are {found}, not int8: {_names(unquantized)}")
    bare = set(weights) - set(scales)
    if bare:
        raise WeightMappingError(f"half-quantized checkpoint: no weight_scales for {_names(bare)}")
    return True


def _stack(stacked: str, members: dict[int, torch.Tensor], num_experts: int) -> torch.Tensor:
    """``members`` (expert index -> tensor) as one tensor in ascending index, with the reference's checks."""
    indices = sorted(members)
    if indices != list(range(len(indices))):
        raise WeightMappingError(f"{stacked}: expert indices must be 0..n-1 with no gaps, got {indices}")
    if len(indices) != num_experts:
        raise WeightMappingError(f"{stacked}: expected {num_experts} experts, got {len(indices)}")
    dtypes = {members[j].dtype for j in indices}
    if len(dtypes) != 1:
        found = sorted(str(d).removeprefix("torch.") for d in dtypes)
        raise WeightMappingError(f"{stacked}: the experts disagree on dtype: {found}")
    shapes = {tuple(members[j].shape) for j in indices}
    if len(shapes) != 1:
        raise WeightMappingError(f"{stacked}: the experts disagree on shape: {sorted(shapes)}")
    return torch.stack([members[j] for j in indices]).contiguous()


def _tensor(checkpoint: Mapping[str, torch.Tensor], layer: int, suffix: str) -> torch.Tensor:
    for name in (f"model.layers.{layer}.mlp.{suffix}", f"layers.{layer}.mlp.{suffix}"):
        if name in checkpoint:
            return checkpoint[name]
    raise WeightMappingError(f"model.layers.{layer}.mlp.{suffix}: not in the checkpoint")


def moe_layer_weights(checkpoint: Mapping[str, torch.Tensor], layer: int, *,
                      num_experts: int) -> tuple[dict[str, torch.Tensor], bool]:
    """Layer ``layer``'s MoE tensors under :class:`MoE`'s names, and whether its experts are int8."""
    int8 = is_int8_checkpoint(checkpoint, layer)
    weights, scales = _expert_tensors(checkpoint, layer)
    if not weights:
        raise WeightMappingError(f"model.layers.{layer}.mlp.experts: no expert weights in the checkpoint")
    out: dict[str, torch.Tensor] = {"gate.gate_score.weight": _tensor(checkpoint, layer, "gate.weight").float()}
    for proj in ROUTED:
        stacked = f"layers.{layer}.mlp.experts.{proj}"
        out[f"experts.{proj}"] = _stack(stacked, {e: v for (_, e, p), v in weights.items() if p == proj}, num_experts)
        if int8:
            out[f"experts.{proj}_scales"] = _stack(
                stacked + "_scales", {e: v for (_, e, p), v in scales.items() if p == proj}, num_experts).float()
    for proj in ROUTED:
        w = _tensor(checkpoint, layer, f"shared_experts.{proj}.weight")
        if w.dim() != 2:
            raise WeightMappingError(f"model.layers.{layer}.mlp.shared_experts.{proj}.weight: expected [N, K], "
                                     f"got shape {tuple(w.shape)}")
        out[f"shared_experts.{proj}.weight"] = kblocked(w.to(torch.bfloat16))
    return out, int8


def moe_from_checkpoint(checkpoint: Mapping[str, torch.Tensor], layer: int, *, num_experts: int = 64,
                        top_k: int = 6, renormalize: bool = False, device: str | torch.device = "cuda:0") -> MoE:
    """The :class:`MoE` of ``model.layers.{layer}.mlp``; the shapes give H, F, the shared width and the group."""
    w, int8 = moe_layer_weights(checkpoint, layer, num_experts=num_experts)
    E, F, H = w["experts.gate_proj"].shape
    fs = w["shared_experts.gate_proj.weight"].shape[1]
    if fs % F:
        raise WeightMappingError(f"layer {layer}: shared width {fs} is not a multiple of the expert width {F}")
    group = H // w["experts.gate_proj_scales"].shape[2] if int8 else 128
    cfg = MoeConfig(hidden_size=H, moe_intermediate_size=F, n_routed_experts=E, num_experts_per_tok=top_k,
                    n_shared_experts=fs // F, int8_experts=int8, group_size=group, renormalize=renormalize)
    return MoE(cfg, {k: v.to(device) for k, v in w.items()})
