"""Checkpoint tensors -> one MoE layer's served weights (the MoE part of unlimited_ocr_max/weight_adapters.py).

A checkpoint in the reference's layout holds every routed expert projection as
its own ``[N, K]`` tensor, and the shared-expert projections un-blocked.
:class:`~uocr_moe.moe.MoE` takes the served layout instead:

==========================================================  ==========================================
checkpoint (``model.`` prefix optional)                     served (:class:`MoE` names)
==========================================================  ==========================================
``layers.L.mlp.gate.weight`` ``[E, H]`` (bf16 on disk)      ``gate.gate_score.weight`` fp32
``layers.L.mlp.experts.j.<proj>.weight`` ``[N, K]``         ``experts.<proj>`` ``[E, N, K]``, j ascending
``layers.L.mlp.experts.j.<proj>.weight_scales``             ``experts.<proj>_scales`` ``[E, N, K/G]`` fp32
``layers.L.mlp.shared_experts.<proj>.weight`` ``[N, K]``    K-blocked ``[K/16, N, 16]`` bf16
==========================================================  ==========================================

How it is read.  One pass over the checkpoint's names takes a census of the
layer: a slot per (projection, expert index) holding that expert's weight and,
on an int8 file, its scales.  Two ordered rule tables then judge the census;
the first rule that finds offenders raises :class:`WeightMappingError` with its
message, so a malformed file is refused for one named reason, never read as a
guess:

* the form rules decide int8 vs bf16 and refuse a half-quantized file (int8
  weights without scales, scales without a weight, scales next to non-int8
  weights, weights without scales while others have them) --
  weight_adapters.py:186-219 states the same four refusals;
* the stack rules check each of the six stacks (three projections, weights and
  scales): expert indices 0..n-1 without gaps, exactly ``num_experts`` of them,
  one dtype and one shape -- weight_adapters.py:121-163.

The refusal texts are the reference's (its tests match them:
tests/test_weight_adapters.py:124-222), and so is their order of precedence.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping
from dataclasses import dataclass
from pathlib import Path

import torch

from .moe import ROUTED, MoE, MoeConfig
from .ops import kblocked

__all__ = ["WeightMappingError", "is_int8_checkpoint", "load_safetensors", "moe_from_checkpoint", "moe_layer_weights"]


class WeightMappingError(RuntimeError):
    """The checkpoint's MoE tensors do not line up with one served layer."""


def load_safetensors(path: str | Path) -> dict[str, torch.Tensor]:
    """Every tensor of a safetensors file, on the CPU (bf16 stays bf16)."""
    from safetensors.torch import load_file

    return load_file(str(path), device="cpu")


# ----------------------------------------------------------------------------- the census


def _routed_part(name: str) -> tuple[int, int, str, bool] | None:
    """``(layer, expert, proj, is_scales)`` of a routed-expert tensor name, else None."""
    parts = name.split(".")
    if parts and parts[0] == "model":
        parts = parts[1:]
    if len(parts) != 7 or parts[0] != "layers" or parts[2:4] != ["mlp", "experts"]:
        return None
    layer, expert, proj, leaf = parts[1], parts[4], parts[5], parts[6]
    if not (layer.isdigit() and expert.isdigit()) or proj not in ROUTED or leaf not in ("weight", "weight_scales"):
        return None
    return int(layer), int(expert), proj, leaf == "weight_scales"


@dataclass
class _Slot:
    """One expert's projection: its weight and (int8 form) its scales, as found."""

    weight: torch.Tensor | None = None
    scales: torch.Tensor | None = None


class _Census:
    """Every routed-expert tensor of one layer (or of all layers: ``layer=None``), in one pass."""

    def __init__(self, checkpoint: Mapping[str, torch.Tensor], layer: int | None) -> None:
        self.slots: dict[tuple[int, int, str], _Slot] = {}
        for name, value in checkpoint.items():
            part = _routed_part(name)
            if part is None or (layer is not None and part[0] != layer):
                continue
            slot = self.slots.setdefault(part[:3], _Slot())
            if part[3]:
                slot.scales = value
            else:
                slot.weight = value

    def keys(self, pick: Callable[[_Slot], bool]) -> list[tuple[int, int, str]]:
        return sorted(k for k, s in self.slots.items() if pick(s))

    @property
    def any_scales(self) -> bool:
        return any(s.scales is not None for s in self.slots.values())


def _listed(keys: list[tuple[int, int, str]], suffix: str = "") -> list[str]:
    """At most 20 offenders, named as the checkpoint names them."""
    return [f"model.layers.{l}.mlp.experts.{e}.{p}.weight{suffix}" for l, e, p in keys[:20]]


def _dtype(t: torch.Tensor) -> str:
    return str(t.dtype).removeprefix("torch.")


def _is_int8(s: _Slot) -> bool:
    return s.weight is not None and s.weight.dtype == torch.int8


# The form rules, in order: (offenders of a census, message); the census is int8
# when it has scales and no rule fires, bf16 when it has none.
_FORM_RULES: tuple[tuple[Callable[[_Census], list], Callable[[_Census, list], str]], ...] = (
    (lambda c: [] if c.any_scales else c.keys(_is_int8),
     lambda c, ks: f"int8 expert weights without weight_scales: {_listed(ks)}"),
    (lambda c: c.keys(lambda s: s.scales is not None and s.weight is None) if c.any_scales else [],
     lambda c, ks: f"weight_scales without an expert weight to scale: {_listed(ks, '_scales')}"),
    (lambda c: c.keys(lambda s: s.weight is not None and not _is_int8(s)) if c.any_scales else [],
     lambda c, ks: "weight_scales are present but these expert weights are "
                   f"{sorted({_dtype(c.slots[k].weight) for k in ks})}, not int8: {_listed(ks)}"),
    (lambda c: c.keys(lambda s: s.weight is not None and s.scales is None) if c.any_scales else [],
     lambda c, ks: f"half-quantized checkpoint: no weight_scales for {_listed(ks)}"),
)


def _judge_form(census: _Census) -> bool:
    for offenders, message in _FORM_RULES:
        found = offenders(census)
        if found:
            raise WeightMappingError(message(census, found))
    return census.any_scales


def is_int8_checkpoint(checkpoint: Mapping[str, torch.Tensor], layer: int | None = None) -> bool:
    """Whether the routed experts are int8 with per-group ``weight_scales`` (False for the bf16 form);
    a half-quantized file raises :class:`WeightMappingError`."""
    return _judge_form(_Census(checkpoint, layer))


# ----------------------------------------------------------------------------- the stacks


# The stack rules, in order, over ``members`` (expert index -> tensor): a failing
# predicate raises with the message, prefixed by the stack's name.
_STACK_RULES: tuple[tuple[Callable[[dict, int], bool], Callable[[dict, int], str]], ...] = (
    (lambda m, n: sorted(m) == list(range(len(m))),
     lambda m, n: f"expert indices must be 0..n-1 with no gaps, got {sorted(m)}"),
    (lambda m, n: len(m) == n,
     lambda m, n: f"expected {n} experts, got {len(m)}"),
    (lambda m, n: len({t.dtype for t in m.values()}) == 1,
     lambda m, n: f"the experts disagree on dtype: {sorted({_dtype(t) for t in m.values()})}"),
    (lambda m, n: len({tuple(t.shape) for t in m.values()}) == 1,
     lambda m, n: f"the experts disagree on shape: {sorted({tuple(t.shape) for t in m.values()})}"),
)


def _stacked(name: str, members: dict[int, torch.Tensor], num_experts: int) -> torch.Tensor:
    for holds, message in _STACK_RULES:
        if not holds(members, num_experts):
            raise WeightMappingError(f"{name}: {message(members, num_experts)}")
    return torch.stack([members[j] for j in range(num_experts)]).contiguous()


def _mlp_tensor(checkpoint: Mapping[str, torch.Tensor], layer: int, leaf: str) -> torch.Tensor:
    for prefix in ("model.", ""):
        t = checkpoint.get(f"{prefix}layers.{layer}.mlp.{leaf}")
        if t is not None:
            return t
    raise WeightMappingError(f"model.layers.{layer}.mlp.{leaf}: not in the checkpoint")


def moe_layer_weights(checkpoint: Mapping[str, torch.Tensor], layer: int, *,
                      num_experts: int) -> tuple[dict[str, torch.Tensor], bool]:
    """Layer ``layer``'s MoE tensors under :class:`MoE`'s names, and whether its experts are int8."""
    census = _Census(checkpoint, layer)
    int8 = _judge_form(census)
    if not census.slots:
        raise WeightMappingError(f"model.layers.{layer}.mlp.experts: no expert weights in the checkpoint")
    served: dict[str, torch.Tensor] = {"gate.gate_score.weight": _mlp_tensor(checkpoint, layer, "gate.weight").float()}
    parts = ("weight", "scales") if int8 else ("weight",)
    for proj in ROUTED:
        for part in parts:
            members = {e: getattr(s, part) for (_, e, p), s in census.slots.items()
                       if p == proj and getattr(s, part) is not None}
            suffix = "_scales" if part == "scales" else ""
            stack = _stacked(f"layers.{layer}.mlp.experts.{proj}{suffix}", members, num_experts)
            served[f"experts.{proj}{suffix}"] = stack.float() if part == "scales" else stack
    for proj in ROUTED:
        w = _mlp_tensor(checkpoint, layer, f"shared_experts.{proj}.weight")
        if w.dim() != 2:
            raise WeightMappingError(f"model.layers.{layer}.mlp.shared_experts.{proj}.weight: expected [N, K], "
                                     f"got shape {tuple(w.shape)}")
        served[f"shared_experts.{proj}.weight"] = kblocked(w.to(torch.bfloat16))
    return served, int8


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
