"""The decoder's decode step on the HIP library: ``UnlimitedOcrDecoder.decode`` / ``DecoderLayer.decode`` /
``Attention.decode`` / ``GatedMlp.decode_rows`` (unlimited_ocr_max/decoder.py:264-276,478-495,670-800).

Per layer, for ``B`` rows (one token of each of ``B`` requests):

* ``input_layernorm`` (with the previous layer's residual add fused in: :func:`ops.rms_norm`, or, at
  one or two rows, inside the q/k/v projection: :func:`ops.rms_norm_dense_bf16_qmv`);
* one ``dense_bf16_qmv`` over the q, k and v projections at once (their K-blocked weights side by side
  along N, the reference's three ``Projection.decode_rows`` calls in one launch);
* :func:`ops.paged_decode_attention_qkv`: RoPE of q and k at each row's position and the paged attention
  (stores the new k/v rows, attends each row's own pages) in one launch, with the bits of
  :func:`ops.rope` followed by :func:`ops.paged_decode_attention`;
* ``o_proj``, then ``post_attention_layernorm`` with the attention residual fused in;
* the MoE block (:meth:`uocr_moe.MoE.decode_rows`) or, for the first ``first_k_dense_replace`` layers,
  the dense gated MLP (one gate+up ``dense_bf16_qmv``, :func:`ops.swiglu`, ``down``).

The final ``norm`` adds the last layer's output.  Every step is a HIP kernel of this library; torch holds
the tensors and orders the launches on the current stream.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from . import ops
from .moe import MoE, MoeConfig


@dataclass(frozen=True)
class DecoderConfig:
    """The decoder fields the decode step reads (unlimited_ocr_max/model_config.py:66-175)."""

    hidden_size: int = 1280
    num_attention_heads: int = 10
    num_hidden_layers: int = 12
    intermediate_size: int = 6848
    first_k_dense_replace: int = 1
    vocab_size: int = 129280
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    moe: MoeConfig = field(default_factory=MoeConfig)

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    def is_moe_layer(self, layer_idx: int) -> bool:
        if not 0 <= layer_idx < self.num_hidden_layers:
            raise IndexError(f"layer_idx {layer_idx} out of range")
        return self.moe.n_routed_experts > 0 and layer_idx >= self.first_k_dense_replace


def rope_tables(*, head_dim: int, seq_len: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """``(cos, sin) [seq_len, head_dim]`` float32, as the reference builds them (decoder.py:115-123)."""
    exponent = np.arange(0, head_dim, 2, dtype=np.int64).astype(np.float32)
    inv_freq = (1.0 / (np.float32(theta) ** (exponent / np.float32(head_dim)))).astype(np.float32)
    positions = np.arange(seq_len, dtype=np.int64).astype(np.float32)
    freqs = positions[:, None] * inv_freq[None, :]
    emb = np.concatenate([freqs, freqs], axis=-1).astype(np.float32)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def _kb_cat(*weights: torch.Tensor) -> torch.Tensor:
    """K-blocked ``[K/16, N_i, 16]`` weights side by side along N: one projection of ``sum N_i`` outputs."""
    return torch.cat(weights, dim=1).contiguous()


class DecoderLayer:
    """One layer's weights on the GPU (the checkpoint's names under ``layers.{i}.``) and its decode step."""

    def __init__(self, config: DecoderConfig, layer_idx: int, weights: dict[str, torch.Tensor]) -> None:
        self.config = config
        self.layer_idx = layer_idx
        p = f"layers.{layer_idx}."
        a = p + "self_attn."
        self.qkv = _kb_cat(*(weights[f"{a}{n}_proj.weight"] for n in "qkv"))
        self.o_proj = weights[f"{a}o_proj.weight"].contiguous()
        self.input_norm = weights[p + "input_layernorm.weight"].float().contiguous()
        self.post_norm = weights[p + "post_attention_layernorm.weight"].float().contiguous()
        m = p + "mlp."
        if config.is_moe_layer(layer_idx):
            self.moe = MoE(config.moe, {k[len(m):]: v for k, v in weights.items() if k.startswith(m)})
            self.gate_up = self.down = None
        else:
            self.moe = None
            self.gate_up = _kb_cat(weights[m + "gate_proj.weight"], weights[m + "up_proj.weight"])
            self.down = weights[m + "down_proj.weight"].contiguous()

    def decode(self, x: torch.Tensor, delta: torch.Tensor | None, *, positions: torch.Tensor, cos: torch.Tensor,
               sin: torch.Tensor, kv: ops.PagedKv, scale: float, spare: torch.Tensor | None = None,
               moe_workspace: torch.Tensor | None = None,
               attn_workspace: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """``x [B, hidden]`` is the residual stream; ``delta`` the previous layer's output, added to it before
        this layer's input norm.  Returns ``(this layer's output, the buffer that now holds the stream)``.

        Without ``spare`` the add is in place (``x``) and the norm a launch of its own; with ``spare`` (rows
        <= :data:`ops.NORM_DENSE_MAX_ROWS`) the norm runs inside the q/k/v projection and the sum lands in
        ``spare`` -- the same bits either way."""
        c = self.config
        rows, heads = x.shape[0], c.num_attention_heads
        if spare is not None:
            qkv = ops.rms_norm_dense_bf16_qmv(x, self.input_norm, c.rms_norm_eps, self.qkv, residual=delta,
                                              x_out=None if delta is None else spare)
            x = x if delta is None else spare
        else:
            normed = ops.rms_norm(x, self.input_norm, c.rms_norm_eps, residual=delta)
            qkv = ops.dense_bf16_qmv(normed, self.qkv)
        attended = ops.paged_decode_attention_qkv(qkv, positions, cos, sin, heads=heads, kv=kv,
                                                  layer_idx=self.layer_idx, scale=scale, workspace=attn_workspace)
        attn_out = ops.dense_bf16_qmv(attended.view(rows, c.hidden_size), self.o_proj)
        normed = ops.rms_norm(x, self.post_norm, c.rms_norm_eps, residual=attn_out)
        if self.moe is not None:
            return self.moe.decode_rows(normed, workspace=moe_workspace), x
        return ops.dense_bf16_qmv(ops.swiglu(ops.dense_bf16_qmv(normed, self.gate_up)), self.down), x


class Decoder:
    """``UnlimitedOcrDecoder``'s decode step (decoder.py:777-800) over the checkpoint's names (without the
    ``model.`` prefix): ``layers.{i}.*``, ``norm.weight``, ``lm_head.weight`` (K-blocked bf16)."""

    def __init__(self, config: DecoderConfig, weights: dict[str, torch.Tensor], *, max_seq_len: int) -> None:
        self.config = config
        self.layers = [DecoderLayer(config, i, weights) for i in range(config.num_hidden_layers)]
        self.norm = weights["norm.weight"].float().contiguous()
        self.lm_head = weights["lm_head.weight"].contiguous()
        dev = self.norm.device
        cos, sin = rope_tables(head_dim=config.head_dim, seq_len=max_seq_len, theta=config.rope_theta)
        self.cos = torch.from_numpy(cos).to(dev)
        self.sin = torch.from_numpy(sin).to(dev)
        self.scale = 1.0 / float(np.sqrt(config.head_dim))

    def decode(self, hidden: torch.Tensor, *, positions: torch.Tensor, kv: ops.PagedKv,
               moe_workspace: torch.Tensor | None = None, attn_workspace: torch.Tensor | None = None,
               scratch: torch.Tensor | None = None, fuse_norm: bool = True) -> torch.Tensor:
        """One token for each of ``B`` requests: ``hidden [B, hidden]`` (used, with ``scratch`` of the same
        shape, to hold the residual stream: its contents afterwards are unspecified), ``positions`` int32
        ``[B]``; every layer stores its new k/v rows through ``kv``.  Returns the final norm of the last
        hidden state, ``[B, hidden]``.  At ``B <=`` :data:`ops.NORM_DENSE_MAX_ROWS` the input norms run
        inside the q/k/v projections (``fuse_norm=False`` keeps them apart; the bits are the same)."""
        fused = fuse_norm and hidden.shape[0] <= ops.NORM_DENSE_MAX_ROWS
        if fused and scratch is None:
            scratch = torch.empty_like(hidden)
        cur, delta = hidden, None
        for layer in self.layers:
            spare = (scratch if cur is hidden else hidden) if fused else None
            delta, cur = layer.decode(cur, delta, positions=positions, cos=self.cos, sin=self.sin, kv=kv,
                                      scale=self.scale, spare=spare, moe_workspace=moe_workspace,
                                      attn_workspace=attn_workspace)
        return ops.rms_norm(cur, self.norm, self.config.rms_norm_eps, residual=delta)

    def logits_rows(self, normed: torch.Tensor) -> torch.Tensor:
        """``lm_head`` over every row, fp32 ``[B, vocab]`` (decoder.py:802-804)."""
        return ops.dense_bf16_qmv(normed, self.lm_head)
