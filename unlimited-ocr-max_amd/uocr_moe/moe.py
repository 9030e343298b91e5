"""The MoE block (unlimited_ocr_max/decoder.py:500-667) on the HIP library.

:class:`MoE` holds one layer's weights under the reference's state-dict names
(``StackedExperts.__init__``, decoder.py:297-313; ``MoEGate``, decoder.py:500-514;
``GatedMlp``, decoder.py:264-278)::

    gate.gate_score.weight            fp32 [E, H]           (the fp32-resident router)
    experts.gate_proj / up_proj       [E, F, H]  int8 or bf16
    experts.down_proj                 [E, H, F]  int8 or bf16
    experts.<proj>_scales             fp32 [E, N, K/128]    (int8 only)
    shared_experts.gate_proj.weight   bf16 K-blocked [H/16, Fs, 16]
    shared_experts.up_proj.weight     bf16 K-blocked [H/16, Fs, 16]
    shared_experts.down_proj.weight   bf16 K-blocked [Fs/16, H, 16]

and runs the two entry points of the reference's module:
:meth:`MoE.decode_rows` (decoder.py:641-655; the batched decode step, B <= 64
rows, bitwise the CPU oracle) and :meth:`MoE.__call__` (decoder.py:657-667;
the prefill, as a grouped GEMM on the bf16 matrix cores).  The gate is
softmax over all experts then top-k with no renormalisation
(model_config.py:149-150) unless ``renormalize=True``.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from .ops import INT8_GROUP_SIZE, KBLOCK, _gpu, _stream

ROUTED = ("gate_proj", "up_proj", "down_proj")


@dataclass(frozen=True)
class MoeConfig:
    """The MoE fields of the reference's DecoderConfig (model_config.py:52-63,166-168)."""

    hidden_size: int = 1280
    moe_intermediate_size: int = 896
    n_routed_experts: int = 64
    num_experts_per_tok: int = 6
    n_shared_experts: int = 2
    int8_experts: bool = True
    group_size: int = INT8_GROUP_SIZE
    renormalize: bool = False

    @property
    def shared_experts_dim(self) -> int:
        return self.n_shared_experts * self.moe_intermediate_size


class MoE:
    """One MoE layer: weights on the GPU, the decode and prefill entry points."""

    def __init__(self, config: MoeConfig, weights: dict[str, torch.Tensor]) -> None:
        self.config = config
        c = config
        E, H, F, Fs = c.n_routed_experts, c.hidden_size, c.moe_intermediate_size, c.shared_experts_dim
        op = "MoE"
        wdt = torch.int8 if c.int8_experts else torch.bfloat16
        self.router = _gpu(op, "gate.gate_score.weight", weights["gate.gate_score.weight"], torch.float32, 2)
        self.stacks = {p: _gpu(op, f"experts.{p}", weights[f"experts.{p}"], wdt, 3) for p in ROUTED}
        self.scales = (
            {p: _gpu(op, f"experts.{p}_scales", weights[f"experts.{p}_scales"], torch.float32, 3) for p in ROUTED}
            if c.int8_experts else {}
        )
        self.shared = {
            p: _gpu(op, f"shared_experts.{p}.weight", weights[f"shared_experts.{p}.weight"], torch.bfloat16, 3)
            for p in ROUTED
        }
        expect = {
            "gate.gate_score.weight": (self.router, (E, H)),
            "experts.gate_proj": (self.stacks["gate_proj"], (E, F, H)),
            "experts.up_proj": (self.stacks["up_proj"], (E, F, H)),
            "experts.down_proj": (self.stacks["down_proj"], (E, H, F)),
            "shared_experts.gate_proj.weight": (self.shared["gate_proj"], (H // KBLOCK, Fs, KBLOCK)),
            "shared_experts.up_proj.weight": (self.shared["up_proj"], (H // KBLOCK, Fs, KBLOCK)),
            "shared_experts.down_proj.weight": (self.shared["down_proj"], (Fs // KBLOCK, H, KBLOCK)),
        }
        if c.int8_experts:
            G = c.group_size
            expect.update({
                "experts.gate_proj_scales": (self.scales["gate_proj"], (E, F, H // G)),
                "experts.up_proj_scales": (self.scales["up_proj"], (E, F, H // G)),
                "experts.down_proj_scales": (self.scales["down_proj"], (E, H, F // G)),
            })
        for name, (t, shape) in expect.items():
            if tuple(t.shape) != shape:
                raise ValueError(f"MoE: {name} has shape {tuple(t.shape)}, expected {shape}")
        self._layer = _lib.Layer(
            E, H, F, Fs, c.num_experts_per_tok, c.group_size, int(c.int8_experts), int(c.renormalize),
            self.router.data_ptr(),
            self.stacks["gate_proj"].data_ptr(), self.stacks["up_proj"].data_ptr(), self.stacks["down_proj"].data_ptr(),
            self.scales["gate_proj"].data_ptr() if c.int8_experts else None,
            self.scales["up_proj"].data_ptr() if c.int8_experts else None,
            self.scales["down_proj"].data_ptr() if c.int8_experts else None,
            self.shared["gate_proj"].data_ptr(), self.shared["up_proj"].data_ptr(), self.shared["down_proj"].data_ptr(),
        )

    @property
    def device(self) -> torch.device:
        return self.router.device

    def workspace_bytes(self, rows: int, prefill: bool) -> int:
        return int(_lib.load().uocr_moe_workspace_bytes(ctypes.byref(self._layer), rows, int(prefill)))

    def workspace(self, rows: int, prefill: bool) -> torch.Tensor:
        """A workspace for ``rows`` tokens, from torch's allocator (stream-ordered)."""
        return torch.empty(self.workspace_bytes(rows, prefill), dtype=torch.uint8, device=self.device)

    def _run(self, entry: str, x: torch.Tensor, prefill: bool, workspace: torch.Tensor | None,
             routing: bool) -> torch.Tensor | tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        x = _gpu(entry, "x", x, torch.float32, 2)
        rows = int(x.shape[0])
        out = torch.empty_like(x)
        ids = wts = None
        if routing:
            ids = torch.empty((rows, self.config.num_experts_per_tok), dtype=torch.int32, device=x.device)
            wts = torch.empty((rows, self.config.num_experts_per_tok), dtype=torch.float32, device=x.device)
        if workspace is None:
            workspace = self.workspace(rows, prefill)
        _lib.call(entry, out.data_ptr(), x.data_ptr(), rows, x.shape[1], ctypes.byref(self._layer),
                  None if ids is None else ids.data_ptr(), None if wts is None else wts.data_ptr(),
                  workspace.data_ptr(), workspace.numel(), _stream(x))
        return (out, ids, wts) if routing else out

    def decode_rows(self, x: torch.Tensor, *, workspace: torch.Tensor | None = None, routing: bool = False,
                    status: torch.Tensor | None = None):
        """MoE.decode_rows (decoder.py:641-655): row ``b`` of ``x [B, H]`` is request ``b``'s token.

        ``status`` (optional, an int32 device tensor of at least one element) receives, in stream order
        after the launch, 1 if the persistent decode kernel's bounded waits ran out on this stream (its
        outputs are then NaN) and 0 otherwise; no synchronisation (see :func:`fused_status`)."""
        out = self._run("uocr_moe_decode_rows", x, False, workspace, routing)
        if status is not None:
            fused_status(status)
        return out

    def __call__(self, x: torch.Tensor, *, workspace: torch.Tensor | None = None, routing: bool = False):
        """MoE.__call__ (decoder.py:657-667): the prefill over ``x [seq, H]``."""
        return self._run("uocr_moe_forward", x, True, workspace, routing)

    def gate(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """MoEGate.__call__ (decoder.py:509-514): ``(indices int64 [T,k], weights fp32 [T,k])`` in score order."""
        return gate(x, self.router, self.config.num_experts_per_tok, renormalize=self.config.renormalize)


def decode_stack(layers: "list[MoE]", x: torch.Tensor, *, status: torch.Tensor | None = None) -> torch.Tensor:
    """The MoE blocks of consecutive decoder layers on the residual stream, one launch:
    ``x_{l+1} = x_l + layers[l].decode_rows(x_l)`` (the adds of decoder.py:709 with the attention
    taken out), returning ``x_n``; the same bits as chaining ``decode_rows``.  Up to 12 layers of
    one shape and kind, ``x [B, H]`` with B <= 8.  ``status`` as for :meth:`MoE.decode_rows`."""
    op = "uocr_moe_decode_stack"
    x = _gpu(op, "x", x, torch.float32, 2)
    if not layers:
        raise ValueError(f"{op}: no layers")
    out = torch.empty_like(x)
    ptrs = (ctypes.POINTER(_lib.Layer) * len(layers))(*[ctypes.pointer(m._layer) for m in layers])
    _lib.call(op, out.data_ptr(), x.data_ptr(), int(x.shape[0]), int(x.shape[1]), ptrs, len(layers), _stream(x))
    if status is not None:
        fused_status(status)
    return out


def fused_status(flag: torch.Tensor) -> torch.Tensor:
    """Writes ``flag[0]`` on the device, in stream order: 1 if a persistent decode launch on the current
    stream (or on the device's static scratch) ran out of its bounded waits, else 0.  Nothing is
    synchronised or cleared (``uocr_moe._lib.fused_errors`` reports with a sync and resets the slot);
    the reference's ops fail on the host only (kernels/moe_int8.mojo:194-210)."""
    op = "uocr_moe_fused_status"
    if not (flag.is_cuda and flag.dtype == torch.int32 and flag.numel() >= 1 and flag.is_contiguous()):
        raise ValueError(f"{op}: flag must be a contiguous int32 device tensor of at least one element")
    _lib.call(op, flag.data_ptr(), _stream(flag))
    return flag


def gate(x: torch.Tensor, router: torch.Tensor, top_k: int, *, renormalize: bool = False):
    """Softmax over the experts, then top-k in score order, ties to the lower id."""
    op = "uocr_moe_gate"
    x = _gpu(op, "x", x, torch.float32, 2)
    router = _gpu(op, "router", router, torch.float32, 2)
    T, H = x.shape
    if router.shape[1] != H:
        raise ValueError(f"{op}: x and the router disagree on hidden")
    idx = torch.empty((T, top_k), dtype=torch.int64, device=x.device)
    wts = torch.empty((T, top_k), dtype=torch.float32, device=x.device)
    ws = torch.empty(max(1, T * router.shape[0] * 4 + 256), dtype=torch.uint8, device=x.device)
    _lib.call(op, idx.data_ptr(), wts.data_ptr(), x.data_ptr(), T, H, router.data_ptr(), router.shape[0], top_k,
              int(renormalize), ws.data_ptr(), ws.numel(), _stream(x))
    return idx, wts
