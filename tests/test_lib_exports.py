"""The HIP library loads, exports every entry point ``include/uocr_moe.h`` declares, and
refuses mis-shaped calls with the reference's messages before touching the GPU.

No compute is launched here (no GPU needed): each refused call fails in the
host-side shape checks, which run before anything is enqueued
(unlimited_ocr_max/kernels/moe_int8.mojo:194-210, moe_bf16.mojo:276-285,
dense_bf16.mojo:130-144, moe_int8.mojo:280-296).
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "uocr_moe.h"


def _declared() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(uocr_\w+)\s*\(", text)))


def test_header_declares_the_entry_points() -> None:
    names = _declared()
    for want in ("uocr_moe_int8_qmv", "uocr_moe_bf16_qmv", "uocr_int8_dequant_expert", "uocr_dense_bf16_qmv",
                 "uocr_moe_gate", "uocr_moe_decode_rows", "uocr_moe_forward", "uocr_ngram_block",
                 "uocr_paged_decode_attention", "uocr_paged_attention_workspace_bytes", "uocr_rms_norm", "uocr_rope",
                 "uocr_swiglu", "uocr_paged_decode_attention_qkv", "uocr_rms_norm_dense_bf16_qmv"):
        assert want in names


def test_library_exports_every_declared_symbol() -> None:
    from uocr_moe import _lib

    lib = _lib.load()
    for name in _declared():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, name
    assert lib.uocr_moe_abi_version() == 1


def _err(name: str, *args) -> str:
    from uocr_moe import _lib

    with pytest.raises(_lib.UocrError) as info:
        _lib.call(name, *args)
    return str(info.value)


@pytest.mark.parametrize(
    ("dims", "message"),
    [
        ((2, 4, 3, 32, 2, 3, 4, 32, 3, 4, 4), "moe_int8_qmv: x and output disagree on k"),
        ((2, 4, 2, 32, 3, 3, 4, 32, 3, 4, 4), "moe_int8_qmv: expert_ids and output disagree on k"),
        ((2, 4, 2, 32, 2, 3, 5, 32, 3, 5, 4), "moe_int8_qmv: w and output disagree on N"),
        ((2, 4, 2, 24, 2, 3, 4, 32, 3, 4, 4), "moe_int8_qmv: w and x disagree on K"),
        ((2, 4, 2, 32, 2, 0, 4, 32, 0, 4, 4), "moe_int8_qmv: the expert stack is empty"),
        ((2, 4, 2, 32, 2, 3, 4, 32, 2, 4, 4), "moe_int8_qmv: scales and w disagree on E"),
        ((2, 4, 2, 32, 2, 3, 4, 32, 3, 5, 4), "moe_int8_qmv: scales and w disagree on N"),
        ((2, 4, 2, 32, 2, 3, 4, 32, 3, 4, 5), "moe_int8_qmv: K must be a multiple of the group count"),
        ((2, 4, 2, 32, 2, 3, 4, 32, 3, 4, 0), "moe_int8_qmv: K must be a multiple of the group count"),
    ],
)
def test_int8_qmv_refusals(dims, message: str) -> None:
    rk, rn, xk, xK, ik, we, wn, wK, se, sn, sg = dims
    got = _err("uocr_moe_int8_qmv", None, rk, rn, None, xk, xK, None, ik, None, we, wn, wK, None, se, sn, sg, None)
    assert got == message


def test_bf16_qmv_refusals() -> None:
    assert _err("uocr_moe_bf16_qmv", None, 2, 4, None, 2, 24, None, 2, None, 3, 4, 32, None) == \
        "moe_bf16_qmv: w and x disagree on K"
    assert _err("uocr_moe_bf16_qmv", None, 2, 4, None, 2, 32, None, 2, None, 0, 4, 32, None) == \
        "moe_bf16_qmv: the expert stack is empty"


def test_dequant_refusals() -> None:
    assert _err("uocr_int8_dequant_expert", None, 4, 32, 0, None, 3, 4, 32, None, 3, 4, 5, None, 1, None) == \
        "int8_dequant_expert: K must be a multiple of the group count"
    assert _err("uocr_int8_dequant_expert", None, 4, 32, 0, None, 3, 4, 32, None, 3, 4, 4, None, 2, None) == \
        "int8_dequant_expert: `expert_idx` must be a single int32"


def test_dense_refusals() -> None:
    assert _err("uocr_dense_bf16_qmv", None, 2, 4, None, 2, 24, None, 2, 4, 16, 1, None) == \
        "dense_bf16_qmv: w and x disagree on K"
    assert _err("uocr_dense_bf16_qmv", None, 2, 4, None, 2, 32, None, 4, 4, 8, 1, None) == \
        "dense_bf16_qmv: w is not K-blocked by KBLOCK"
    assert _err("uocr_dense_bf16_qmv", None, 2, 4, None, 2, 32, None, 2, 4, 16, 0, None) == \
        "dense_bf16_qmv: tile must be >= 1"


def test_ngram_refusals() -> None:
    """unlimited_ocr_max/kernels/ngram_block.mojo:85-99."""
    # (result rows, vocab, logits rows, vocab, history rows, length, ngram count)
    cases = [
        ((2, 16, 2, 15, 2, 4, 1), "ngram_block: logits and output disagree on shape"),
        ((2, 16, 2, 16, 1, 4, 1), "ngram_block: history and logits disagree on the row count"),
        ((2, 16, 2, 16, 2, 4, 2), "ngram_block: `ngram` must be a single int32"),
        ((2, 16, 2, 16, 2, 0, 1), "ngram_block: history is empty"),
        ((2, 16, 2, 16, 2, 8193, 1), "ngram_block: history longer than 8192 ids"),
    ]
    for (rr, rv, lr, lv, hr, hl, nl), message in cases:
        assert _err("uocr_ngram_block", None, rr, rv, None, lr, lv, None, hr, hl, None, nl, None) == message


def test_paged_attention_refusals_and_workspace_size() -> None:
    """The host checks of uocr_paged_decode_attention, before anything is enqueued."""
    from uocr_moe import _lib

    def call(rows=1, heads=10, head_dim=128, pages=3, layers=2, page_size=128, layer=0, cols=2, attend_max=1):
        return _err("uocr_paged_decode_attention", None, None, None, None, rows, heads, head_dim, None, pages, layers,
                    page_size, layer, None, cols, None, attend_max, None, 1.0, None, 0, None)

    assert call(head_dim=64) == "paged_decode_attention: head_dim must be 128, got 64"
    assert call(page_size=64) == "paged_decode_attention: page_size must be a positive multiple of 128"
    assert call(page_size=192) == "paged_decode_attention: page_size must be a positive multiple of 128"
    assert call(layer=2) == "paged_decode_attention: layer 2 is not in the pool's 2 layers"
    assert call(layer=-1) == "paged_decode_attention: layer -1 is not in the pool's 2 layers"
    assert call(attend_max=257) == \
        "paged_decode_attention: attend_max 257 is not in [1, 256], the rows the lookup table addresses"
    assert call(attend_max=0).startswith("paged_decode_attention: attend_max 0 is not in")
    assert call(rows=65536) == "paged_decode_attention: rows must be in [0, 65535] and heads in [1, 65535]"
    assert call() == "paged_decode_attention: a tensor is missing"
    lib = _lib.load()
    assert lib.uocr_paged_attention_workspace_bytes(8, 10, 640) == 8 * 10 * 5 * 132 * 4
    assert lib.uocr_paged_attention_workspace_bytes(1, 10, 129) == 10 * 2 * 132 * 4
    assert lib.uocr_paged_attention_workspace_bytes(1, 10, 0) == 0


def test_decoder_step_refusals() -> None:
    """The host checks of uocr_rms_norm, uocr_rope and uocr_swiglu, before anything is enqueued."""
    assert _err("uocr_rms_norm", None, None, None, None, None, 2, 0, 1e-6, None) == "rms_norm: bad shape [2, 0]"
    assert _err("uocr_rms_norm", None, None, None, None, None, 2, 8, -1.0, None) == "rms_norm: eps must be >= 0"
    assert _err("uocr_rms_norm", None, None, None, None, None, 2, 8, 1e-6, None) == \
        "rms_norm: a tensor is missing"

    def rope(heads=2, head_dim=8, stride=16, table_rows=4, table_dim=8):
        return _err("uocr_rope", None, None, None, None, None, None, 3, heads, head_dim, stride, None, None, None,
                    table_rows, table_dim, None)

    assert rope(head_dim=7, table_dim=7) == "rope: head_dim must be even for RoPE"
    assert rope(table_dim=16) == "rope: the cos/sin tables are 16 wide, not head_dim 8"
    assert rope(stride=15) == "rope: input rows 15 floats apart overlap rows of 16"
    assert rope(table_rows=0) == "rope: bad shape"
    assert rope() == "rope: a tensor is missing"
    def qkv(stride=3840, table_dim=128, rows=1):
        return _err("uocr_paged_decode_attention_qkv", None, None, rows, 10, 128, stride, None, None, None, 16,
                    table_dim, None, 3, 2, 128, 0, None, 2, None, 1, None, 1.0, None, 0, None)

    assert qkv(stride=3839) == "paged_decode_attention_qkv: qkv rows 3839 floats apart overlap rows of 3840"
    assert qkv(table_dim=64) == "paged_decode_attention_qkv: the cos/sin tables are 64 wide, not head_dim 128"
    assert qkv() == "paged_decode_attention_qkv: a tensor is missing"
    def nd(m=2, n=3840, k=1280, blocks=80):
        return _err("uocr_rms_norm_dense_bf16_qmv", None, m, n, None, m, k, None, None, None, 1e-6, None, blocks, n,
                    16, None)

    assert nd(m=3) == "rms_norm_dense_bf16_qmv: takes at most 2 rows, N < 16384 and K <= 2048"
    assert nd(n=16384) == "rms_norm_dense_bf16_qmv: takes at most 2 rows, N < 16384 and K <= 2048"
    assert nd(k=4096, blocks=256) == "rms_norm_dense_bf16_qmv: takes at most 2 rows, N < 16384 and K <= 2048"
    assert nd(blocks=79) == "rms_norm_dense_bf16_qmv: w and x disagree on K"
    assert nd() == "rms_norm_dense_bf16_qmv: a tensor is missing"
    assert _err("uocr_swiglu", None, None, 2, 0, None) == "swiglu: bad shape [2, 0]"
    assert _err("uocr_swiglu", None, None, 2, 4, None) == "swiglu: a tensor is missing"


def test_layer_refusals() -> None:
    from uocr_moe import _lib

    layer = _lib.Layer(65, 1280, 896, 1792, 6, 128, 1, 0)
    msg = _err("uocr_moe_decode_rows", None, None, 1, 1280, ctypes.byref(layer), None, None, None, 0, None)
    assert msg == "uocr_moe_decode_rows: num_experts must be in [1, 64]"
    layer = _lib.Layer(64, 1280, 896, 1792, 6, 128, 1, 0)
    msg = _err("uocr_moe_forward", None, None, 1, 1024, ctypes.byref(layer), None, None, None, 0, None)
    assert msg == "uocr_moe_forward: x and the layer disagree on hidden"


def test_quantize_refusals() -> None:
    """tools/quantize_int8.py:306-308: a partial trailing group is refused, not quantised."""
    assert _err("uocr_quantize_per_group", 8, 8, 8, 0, 2, 100, 128, None) == \
        "quantize_per_group: K=100 is not divisible by the group size 128"
    assert "bad group size" in _err("uocr_quantize_per_group", 8, 8, 8, 0, 2, 128, 0, None)


def test_static_decode_refuses_beyond_its_scratch() -> None:
    """The allocation-free decode refuses, before any device call, a call whose multi-kernel workspace would
    not fit its static scratch (64 rows of a layer 2048 wide)."""
    from uocr_moe import _lib

    fake = 4096  # never dereferenced: the call is refused on the host
    layer = _lib.Layer(64, 2048, 2048, 2048, 6, 128, 0, 0, fake, fake, fake, fake, None, None, None, fake, fake, fake)
    msg = _err("uocr_moe_decode_rows_static", None, None, 64, 2048, ctypes.byref(layer), None, None, None)
    assert msg.startswith("uocr_moe_decode_rows_static: 64 rows of this layer need ") and "more than the" in msg
    msg = _err("uocr_moe_decode_rows_static", None, None, 65, 2048, ctypes.byref(layer), None, None, None)
    assert msg == "uocr_moe_decode_rows_static: rows must be in [0, 64]"


def test_fused_status_refuses_a_missing_flag() -> None:
    """The stream-ordered error flag entry refuses a null flag before any device call."""
    assert _err("uocr_moe_fused_status", None, None) == "uocr_moe_fused_status: no flag"
