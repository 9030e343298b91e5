"""uocr_moe: the DeepSeek-V2 routed-expert MoE block of unlimited-ocr-max on MI355X (gfx950).

The product is the HIP library ``libuocr_moe.so`` behind a C ABI
(``include/uocr_moe.h``); this package is its Python host side, mirroring the
reference's op names (:mod:`uocr_moe.ops`) and MoE module (:mod:`uocr_moe.moe`),
plus the ops either side of the block on the decode path (RMSNorm, RoPE, the
paged decode attention, the dense projections and lm_head GEMV, the n-gram
guard) and the decode step they make up (:mod:`uocr_moe.decoder`).
"""

from ._lib import LIB_PATH, UocrError
from .checkpoint import WeightMappingError, load_safetensors, moe_from_checkpoint, moe_layer_weights
from .decoder import Decoder, DecoderConfig, DecoderLayer, rope_tables
from .moe import MoE, MoeConfig, decode_stack, fused_status, gate
from .ops import (
    PagedKv,
    custom,
    dense_bf16_qmv,
    int8_dequant_expert,
    kblocked,
    moe_bf16_qmv,
    moe_int8_qmv,
    ngram_block,
    paged_decode_attention,
    paged_decode_attention_qkv,
    quantize_per_group,
    rms_norm,
    rms_norm_dense_bf16_qmv,
    rope,
    swiglu,
)

__all__ = [
    "Decoder",
    "DecoderConfig",
    "DecoderLayer",
    "LIB_PATH",
    "MoE",
    "MoeConfig",
    "PagedKv",
    "UocrError",
    "WeightMappingError",
    "custom",
    "decode_stack",
    "dense_bf16_qmv",
    "fused_status",
    "gate",
    "int8_dequant_expert",
    "kblocked",
    "load_safetensors",
    "moe_bf16_qmv",
    "moe_from_checkpoint",
    "moe_int8_qmv",
    "moe_layer_weights",
    "ngram_block",
    "paged_decode_attention",
    "paged_decode_attention_qkv",
    "quantize_per_group",
    "rms_norm",
    "rms_norm_dense_bf16_qmv",
    "rope",
    "rope_tables",
    "swiglu",
]
