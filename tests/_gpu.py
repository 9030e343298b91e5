"""Helpers shared by the GPU tests: moving oracle-side numpy data onto the GPU and back."""

from __future__ import annotations

import numpy as np
import torch

DEV = "cuda:0"


def t(a: np.ndarray) -> torch.Tensor:
    """numpy -> GPU tensor; uint16 arrays become bfloat16 (bit patterns kept)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).to(DEV).view(torch.bfloat16)
    return torch.from_numpy(a).to(DEV)


def n(x: torch.Tensor) -> np.ndarray:
    """GPU tensor -> numpy; bfloat16 becomes uint16 bit patterns."""
    torch.cuda.synchronize()
    if x.dtype == torch.bfloat16:
        return x.view(torch.int16).cpu().numpy().view(np.uint16)
    return x.cpu().numpy()


def layer_weights(layer) -> dict[str, torch.Tensor]:
    """An oracle ``MoeWeights`` as the reference's state-dict names on the GPU."""
    w = {
        "gate.gate_score.weight": t(layer.router),
        "experts.gate_proj": t(layer.gate),
        "experts.up_proj": t(layer.up),
        "experts.down_proj": t(layer.down),
        "shared_experts.gate_proj.weight": t(layer.sh_gate),
        "shared_experts.up_proj.weight": t(layer.sh_up),
        "shared_experts.down_proj.weight": t(layer.sh_down),
    }
    if layer.int8:
        w["experts.gate_proj_scales"] = t(layer.gate_s)
        w["experts.up_proj_scales"] = t(layer.up_s)
        w["experts.down_proj_scales"] = t(layer.down_s)
    return w


def moe_for(layer):
    from uocr_moe import MoE, MoeConfig

    E, H, F, Fs = layer.dims
    cfg = MoeConfig(hidden_size=H, moe_intermediate_size=F, n_routed_experts=E, num_experts_per_tok=layer.topk,
                    n_shared_experts=Fs // F, int8_experts=layer.int8, group_size=layer.group,
                    renormalize=layer.renorm)
    return MoE(cfg, layer_weights(layer))


def bits_equal(a: np.ndarray, b: np.ndarray) -> bool:
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def differ(a: np.ndarray, b: np.ndarray) -> int:
    return int(np.count_nonzero(np.ascontiguousarray(a).view(np.uint32) != np.ascontiguousarray(b).view(np.uint32)))
