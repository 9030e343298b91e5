"""The reference's custom ops on PyTorch-ROCm tensors, through the HIP library.

Names, argument order, dtypes, output shapes and error messages follow the
reference's MAX ops (``unlimited_ocr_max/kernels/*.mojo``) as its graph code
stages them (``unlimited_ocr_max/decoder.py:166-184,325-330,355-366``):

=====================  ===================================================  ==================
op                     values                                               result
=====================  ===================================================  ==================
moe_int8_qmv           x f32 [k,K], expert_ids i32 [k], w i8 [E,N,K],       f32 [k,N]
                       scales f32 [E,N,K/G]
moe_bf16_qmv           x f32 [k,K], expert_ids i32 [k], w bf16 [E,N,K]      f32 [k,N]
int8_dequant_expert    w i8 [E,N,K], scales f32 [E,N,K/G], expert_idx i32   bf16 (or f32) [N,K]
                       [1]
dense_bf16_qmv         x f32 [M,K], w bf16 [K/16,N,16]; parameter ``tile``  f32 [M,N]
ngram_block            logits f32 [B,V], history i32 [B,W], ngram i32 [1]   f32 [B,V]
=====================  ===================================================  ==================

:func:`paged_decode_attention` (decoder.py:425-437) takes its page pool and
step metadata as a :class:`PagedKv`.

:func:`custom` dispatches by symbol like ``ops.custom(symbol, values=...)``.
Inputs must be GPU tensors; non-contiguous views are packed first (the
reference reads strided inputs with the same bits as packed ones).  An
``out=`` tensor is written in place and must be contiguous.  Work is
enqueued on the current torch stream.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import _lib

KBLOCK = 16
INT8_GROUP_SIZE = 128
#: The fewest work items the reference's tile rule leaves a dense_bf16_qmv call
#: (unlimited_ocr_max/decoder.py:141).
DENSE_MIN_ITEMS = 2048


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _gpu(op: str, name: str, t: torch.Tensor, dtype: torch.dtype, rank: int) -> torch.Tensor:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{op}: {name} must be a torch.Tensor, got {type(t).__name__}")
    if t.dtype != dtype:
        raise TypeError(f"{op}: {name} must be {dtype}, got {t.dtype}")
    if t.dim() != rank:
        raise ValueError(f"{op}: {name} must be rank {rank}, got shape {tuple(t.shape)}")
    if t.device.type != "cuda":
        raise ValueError(f"{op}: {name} must be on the GPU, got {t.device}")
    return t.contiguous()


def _out(op: str, name: str, t: torch.Tensor, dtype: torch.dtype, rank: int) -> torch.Tensor:
    """An output tensor: checked like an input, and written in place, so it must be contiguous (a packed
    copy would take the result and leave the caller's tensor unchanged)."""
    _gpu(op, name, t, dtype, rank)
    if not t.is_contiguous():
        raise ValueError(f"{op}: {name} must be contiguous (the result is written into it in place)")
    return t


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _rows_per_read(rows: int, out_dim: int) -> int:
    """The reference's tile rule for dense_bf16_qmv (unlimited_ocr_max/decoder.py:144-163); 1 for no rows."""
    if rows <= 0:
        return 1
    tiles = 1
    while True:
        tile = math.ceil(rows / tiles)
        if tile == 1 or out_dim * math.ceil(rows / tile) >= DENSE_MIN_ITEMS:
            return tile
        tiles += 1


def moe_int8_qmv(x, expert_ids, w, scales, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """``out[s,n] = sum_g scales[e,n,g] * sum_{kk in g} f32(w[e,n,kk]) * x[s,kk]``, ``e = clamp(expert_ids[s])``.

    unlimited_ocr_max/kernels/moe_int8.mojo:181-258, bitwise its operation order.
    """
    op = "moe_int8_qmv"
    x = _gpu(op, "x", x, torch.float32, 2)
    expert_ids = _gpu(op, "expert_ids", expert_ids, torch.int32, 1)
    w = _gpu(op, "w", w, torch.int8, 3)
    scales = _gpu(op, "scales", scales, torch.float32, 3)
    if out is None:
        out = torch.empty((x.shape[0], w.shape[1]), dtype=torch.float32, device=x.device)
    out = _out(op, "result", out, torch.float32, 2)
    _lib.call("uocr_moe_int8_qmv", out.data_ptr(), out.shape[0], out.shape[1], x.data_ptr(), x.shape[0], x.shape[1],
              expert_ids.data_ptr(), expert_ids.shape[0], w.data_ptr(), *w.shape, scales.data_ptr(), *scales.shape,
              _stream(x))
    return out


def moe_bf16_qmv(x, expert_ids, w, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """``out[s,n] = sum_kk f32(w[e,n,kk]) * x[s,kk]`` (unlimited_ocr_max/kernels/moe_bf16.mojo:264-345)."""
    op = "moe_bf16_qmv"
    x = _gpu(op, "x", x, torch.float32, 2)
    expert_ids = _gpu(op, "expert_ids", expert_ids, torch.int32, 1)
    w = _gpu(op, "w", w, torch.bfloat16, 3)
    if out is None:
        out = torch.empty((x.shape[0], w.shape[1]), dtype=torch.float32, device=x.device)
    out = _out(op, "result", out, torch.float32, 2)
    _lib.call("uocr_moe_bf16_qmv", out.data_ptr(), out.shape[0], out.shape[1], x.data_ptr(), x.shape[0], x.shape[1],
              expert_ids.data_ptr(), expert_ids.shape[0], w.data_ptr(), *w.shape, _stream(x))
    return out


def int8_dequant_expert(w, scales, expert_idx, *, dtype: torch.dtype = torch.bfloat16,
                        out: torch.Tensor | None = None) -> torch.Tensor:
    """Expert ``clamp(expert_idx[0])`` as ``round(f32(q) * scale)`` in ``dtype`` [N, K]
    (unlimited_ocr_max/kernels/moe_int8.mojo:261-342)."""
    op = "int8_dequant_expert"
    w = _gpu(op, "w", w, torch.int8, 3)
    scales = _gpu(op, "scales", scales, torch.float32, 3)
    expert_idx = _gpu(op, "expert_idx", expert_idx, torch.int32, 1)
    if out is None:
        if dtype not in (torch.bfloat16, torch.float32):
            raise TypeError(f"{op}: the result must be bfloat16 or float32, got {dtype}")
        out = torch.empty((w.shape[1], w.shape[2]), dtype=dtype, device=w.device)
    if out.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError(f"{op}: the result must be bfloat16 or float32, got {out.dtype}")
    out = _out(op, "result", out, out.dtype, 2)
    _lib.call("uocr_int8_dequant_expert", out.data_ptr(), out.shape[0], out.shape[1], int(out.dtype == torch.float32),
              w.data_ptr(), *w.shape, scales.data_ptr(), *scales.shape, expert_idx.data_ptr(), expert_idx.shape[0],
              _stream(w))
    return out


def dense_bf16_qmv(x, w, *, tile: int | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """``x @ W.T`` for a K-blocked bf16 ``w [K/16, N, 16]`` (unlimited_ocr_max/kernels/dense_bf16.mojo:119-158).

    ``tile`` defaults to the reference's :func:`_rows_per_read`; a row's bits do not depend on it.
    """
    op = "dense_bf16_qmv"
    x = _gpu(op, "x", x, torch.float32, 2)
    w = _gpu(op, "w", w, torch.bfloat16, 3)
    if tile is None:
        tile = _rows_per_read(int(x.shape[0]), int(w.shape[1]))
    if out is None:
        out = torch.empty((x.shape[0], w.shape[1]), dtype=torch.float32, device=x.device)
    out = _out(op, "result", out, torch.float32, 2)
    _lib.call("uocr_dense_bf16_qmv", out.data_ptr(), out.shape[0], out.shape[1], x.data_ptr(), x.shape[0], x.shape[1],
              w.data_ptr(), *w.shape, int(tile), _stream(x))
    return out


#: The value a banned logit is set to (unlimited_ocr_max/kernels/ngram_block.mojo:49): finite, below every logit.
NGRAM_BLOCKED = -3.0e38


def ngram_block(logits, history, ngram, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """The no-repeat-n-gram guard (unlimited_ocr_max/kernels/ngram_block.mojo:1-151).

    ``logits [V]`` with ``history [H]`` (one row), or ``logits [B, V]`` with ``history [B, H]``: row ``b``
    against row ``b``'s last ids only.  ``ngram`` is an int32 ``[1]`` tensor on the GPU (read on the device,
    as the reference's) or a Python int.  Banned ids become :data:`NGRAM_BLOCKED`; ``out`` may be ``logits``.
    """
    op = "ngram_block"
    if not isinstance(logits, torch.Tensor) or logits.dim() not in (1, 2):
        raise ValueError(f"{op} takes one row (V,) or B rows (B, V)")
    rank = logits.dim()
    logits = _gpu(op, "logits", logits, torch.float32, rank)
    history = _gpu(op, "history", history, torch.int32, rank)
    if isinstance(ngram, int):
        ngram = torch.tensor([ngram], dtype=torch.int32, device=logits.device)
    ngram = _gpu(op, "ngram", ngram, torch.int32, 1)
    if out is None:
        out = torch.empty_like(logits)
    out = _out(op, "result", out, torch.float32, rank)
    rows = 1 if rank == 1 else int(logits.shape[0])
    hrows = 1 if rank == 1 else int(history.shape[0])
    orows = 1 if rank == 1 else int(out.shape[0])
    _lib.call("uocr_ngram_block", out.data_ptr(), orows, out.shape[-1], logits.data_ptr(), rows, logits.shape[-1],
              history.data_ptr(), hrows, history.shape[-1], ngram.data_ptr(), ngram.shape[0], _stream(logits))
    return out


def rms_norm(x, gamma, eps: float, *, residual=None, out: torch.Tensor | None = None,
             x_out: torch.Tensor | None = None):
    """``RmsNorm`` (unlimited_ocr_max/decoder.py:252-261) over the rows of ``x [rows, dim]`` with an fp32
    ``gamma [dim]``.  Given ``residual``, the residual add before it (decoder.py:702-709):
    ``v = x + residual`` is written to ``x_out`` (default: ``x`` itself, in place) and the norm of ``v``
    is returned.  ``x`` must then be contiguous."""
    op = "rms_norm"
    if residual is not None and not x.is_contiguous():
        raise ValueError(f"{op}: x must be contiguous when the residual is added in place")
    x = _gpu(op, "x", x, torch.float32, 2)
    gamma = _gpu(op, "gamma", gamma, torch.float32, 1)
    if gamma.shape[0] != x.shape[1]:
        raise ValueError(f"{op}: gamma has {gamma.shape[0]} entries for rows of {x.shape[1]}")
    if residual is not None:
        residual = _gpu(op, "residual", residual, torch.float32, 2)
        if residual.shape != x.shape:
            raise ValueError(f"{op}: residual {tuple(residual.shape)} and x {tuple(x.shape)} disagree")
        x_out = x if x_out is None else _gpu(op, "x_out", x_out, torch.float32, 2)
        if x_out.shape != x.shape or not x_out.is_contiguous():
            raise ValueError(f"{op}: x_out must be a contiguous {tuple(x.shape)} tensor")
    if out is None:
        out = torch.empty_like(x)
    out = _out(op, "out", out, torch.float32, 2)
    if out.shape != x.shape:
        raise ValueError(f"{op}: out must be {tuple(x.shape)}")
    _lib.call("uocr_rms_norm", out.data_ptr(), _ptr(x_out), x.data_ptr(), _ptr(residual), gamma.data_ptr(),
              x.shape[0], x.shape[1], float(eps), _stream(x))
    return out


def _rows_view(op: str, name: str, t, like=None) -> torch.Tensor:
    """A ``[rows, heads, D]`` fp32 GPU view whose heads and elements are packed (rows may be strided)."""
    if not isinstance(t, torch.Tensor) or t.dtype != torch.float32 or t.dim() != 3 or t.device.type != "cuda":
        raise ValueError(f"{op}: {name} must be an fp32 [rows, heads, head_dim] GPU tensor")
    if t.stride(2) != 1 or t.stride(1) != t.shape[2]:
        t = t.contiguous()
    if like is not None and (t.shape != like.shape or t.stride(0) != like.stride(0)):
        raise ValueError(f"{op}: {name} {tuple(t.shape)} (row stride {t.stride(0)}) does not match "
                         f"{tuple(like.shape)} (row stride {like.stride(0)})")
    return t


#: The fused norm + projection takes at most this many rows (and K <= 2048, N < 16384).
NORM_DENSE_MAX_ROWS = 2


def rms_norm_dense_bf16_qmv(x, gamma, eps: float, w, *, residual=None, x_out=None,
                            out: torch.Tensor | None = None) -> torch.Tensor:
    """:func:`rms_norm` then :func:`dense_bf16_qmv` in one launch, with their bits, for decode rows
    (at most :data:`NORM_DENSE_MAX_ROWS`): ``rmsnorm(x + residual) * gamma @ W^T``.  With ``residual``,
    ``x + residual`` is written to ``x_out``, which must be another buffer than ``x`` and ``residual``."""
    op = "rms_norm_dense_bf16_qmv"
    x = _gpu(op, "x", x, torch.float32, 2)
    gamma = _gpu(op, "gamma", gamma, torch.float32, 1)
    w = _gpu(op, "w", w, torch.bfloat16, 3)
    if residual is not None:
        residual = _gpu(op, "residual", residual, torch.float32, 2)
        if x_out is None:
            raise ValueError(f"{op}: a residual add needs x_out")
        if residual.shape != x.shape or tuple(x_out.shape) != tuple(x.shape) or not x_out.is_contiguous():
            raise ValueError(f"{op}: residual and x_out must be contiguous {tuple(x.shape)} tensors")
    if out is None:
        out = torch.empty((x.shape[0], w.shape[1]), device=x.device, dtype=torch.float32)
    out = _out(op, "result", out, torch.float32, 2)
    _lib.call("uocr_rms_norm_dense_bf16_qmv", out.data_ptr(), out.shape[0], out.shape[1], x.data_ptr(), x.shape[0],
              x.shape[1], _ptr(residual), _ptr(x_out), gamma.data_ptr(), float(eps), w.data_ptr(), w.shape[0],
              w.shape[1], w.shape[2], _stream(x))
    return out


def rope(q, k, positions, cos_table, sin_table, *, v=None, q_out=None, k_out=None, v_out=None):
    """``Attention._rope`` on the decode rows (decoder.py:459-462,487-491) with the cos / sin rows gathered
    at ``positions`` (``rope_rows``, decoder.py:766-775): ``q``, ``k`` ``[rows, heads, head_dim]`` (``k``
    may be ``None``; rows may be strided, as the thirds of one fused q/k/v projection are), ``positions``
    int32 ``[rows]``, tables ``[table_rows, head_dim]``.  ``v``, when given, is copied to a packed
    ``v_out``.  Returns ``(q_out, k_out, v_out)``, packed; ``q_out=q`` rotates a packed ``q`` in place."""
    op = "rope"
    q = _rows_view(op, "q", q)
    k = None if k is None else _rows_view(op, "k", k, q)
    v = None if v is None else _rows_view(op, "v", v, q)
    positions = _gpu(op, "positions", positions, torch.int32, 1)
    if positions.shape[0] != q.shape[0]:
        raise ValueError(f"{op}: {positions.shape[0]} positions for {q.shape[0]} rows")
    cos_table = _gpu(op, "cos_table", cos_table, torch.float32, 2)
    sin_table = _gpu(op, "sin_table", sin_table, torch.float32, 2)
    if cos_table.shape != sin_table.shape:
        raise ValueError(f"{op}: the cos and sin tables disagree on shape")
    shape = tuple(q.shape)

    def packed(name, t, src):
        if src is None:
            return None
        t = torch.empty(shape, device=q.device, dtype=torch.float32) if t is None else t
        if not isinstance(t, torch.Tensor) or tuple(t.shape) != shape or not t.is_contiguous() or \
                t.dtype != torch.float32:
            raise ValueError(f"{op}: {name} must be a contiguous fp32 {shape} tensor")
        return t

    q_out, k_out, v_out = packed("q_out", q_out, q), packed("k_out", k_out, k), packed("v_out", v_out, v)
    _lib.call("uocr_rope", q_out.data_ptr(), _ptr(k_out), _ptr(v_out), q.data_ptr(), _ptr(k), _ptr(v), shape[0],
              shape[1], shape[2], q.stride(0), positions.data_ptr(), cos_table.data_ptr(), sin_table.data_ptr(),
              cos_table.shape[0], cos_table.shape[1], _stream(q))
    return q_out, k_out, v_out


def swiglu(gate_up, *, out: torch.Tensor | None = None) -> torch.Tensor:
    """``silu(gate) * up`` of ``GatedMlp.decode_rows`` (decoder.py:274-276) over one gate+up projection's
    output ``[rows, 2 * ffn]`` (gate columns first); returns ``[rows, ffn]``."""
    op = "swiglu"
    gate_up = _gpu(op, "gate_up", gate_up, torch.float32, 2)
    if gate_up.shape[1] % 2:
        raise ValueError(f"{op}: gate_up must hold 2 * ffn columns, got {gate_up.shape[1]}")
    ffn = gate_up.shape[1] // 2
    if out is None:
        out = torch.empty((gate_up.shape[0], ffn), device=gate_up.device, dtype=torch.float32)
    out = _out(op, "out", out, torch.float32, 2)
    if tuple(out.shape) != (gate_up.shape[0], ffn):
        raise ValueError(f"{op}: out must be {(gate_up.shape[0], ffn)}")
    _lib.call("uocr_swiglu", out.data_ptr(), gate_up.data_ptr(), gate_up.shape[0], ffn, _stream(gate_up))
    return out


@dataclass(frozen=True)
class PagedKv:
    """One decode step's view of the KV page pool: the pool and the step's metadata, as the reference's
    ``PagedKv`` / ``PagedStep`` hold them (unlimited_ocr_max/decoder.py:407-422,
    unlimited_ocr_max/kv_cache.py:169-207).

    ``kv_blocks`` f32 ``[pages, 2, layers, page_size, heads, head_dim]`` (its last page the null page);
    ``lookup_table`` ``[B, cols]``, ``attend_lengths`` ``[B]`` (``attend_len - 1``, the attention's cache
    lengths) and ``write_index`` ``[B]`` (the store's), int32 or uint32 on the GPU; ``attend_max`` the
    largest ``attend_len``, a host int.
    """

    kv_blocks: torch.Tensor
    lookup_table: torch.Tensor
    attend_lengths: torch.Tensor
    attend_max: int
    write_index: torch.Tensor


def _u32(op: str, name: str, t: torch.Tensor, rank: int) -> torch.Tensor:
    if isinstance(t, torch.Tensor) and t.dtype == torch.uint32:
        return _gpu(op, name, t.view(torch.int32), torch.int32, rank)
    return _gpu(op, name, t, torch.int32, rank)


def paged_decode_attention(q, k_new, v_new, *, kv: PagedKv, layer_idx: int, scale: float,
                           out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Store each row's new k/v at its write index, then attend each row over its own rows
    (unlimited_ocr_max/decoder.py:425-437).

    ``q`` / ``k_new`` / ``v_new`` are post-RoPE f32 ``[B, heads, head_dim]``, row ``b`` for request ``b``;
    returns ``[B, heads, head_dim]``, row ``b`` attended over its logical rows ``[0, attend_lengths[b] + 1)``
    of layer ``layer_idx``, logical row ``r`` being slot ``r % page_size`` of page
    ``lookup_table[b, r // page_size]``.  ``kv.kv_blocks`` is written in place (it must be contiguous).
    """
    op = "paged_decode_attention"
    q = _gpu(op, "q", q, torch.float32, 3)
    k_new = _gpu(op, "k_new", k_new, torch.float32, 3)
    v_new = _gpu(op, "v_new", v_new, torch.float32, 3)
    if k_new.shape != q.shape or v_new.shape != q.shape:
        raise ValueError(f"{op}: q, k_new and v_new disagree on shape: {tuple(q.shape)}, {tuple(k_new.shape)}, "
                         f"{tuple(v_new.shape)}")
    blocks = kv.kv_blocks
    if not isinstance(blocks, torch.Tensor) or blocks.dtype != torch.float32 or blocks.dim() != 6:
        raise ValueError(f"{op}: kv_blocks must be f32 [pages, 2, layers, page_size, heads, head_dim]")
    if blocks.device.type != "cuda" or not blocks.is_contiguous():
        raise ValueError(f"{op}: kv_blocks must be a contiguous GPU tensor (it is written in place)")
    pages, two, layers, page_size, heads, head_dim = blocks.shape
    rows = int(q.shape[0])
    if two != 2 or (heads, head_dim) != tuple(q.shape[1:]):
        raise ValueError(f"{op}: kv_blocks {tuple(blocks.shape)} does not hold [.., 2, .., .., heads, head_dim] "
                         f"of q {tuple(q.shape)}")
    lookup = _u32(op, "lookup_table", kv.lookup_table, 2)
    attend = _u32(op, "attend_lengths", kv.attend_lengths, 1)
    write = _u32(op, "write_index", kv.write_index, 1)
    if lookup.shape[0] != rows or attend.shape[0] != rows or write.shape[0] != rows:
        raise ValueError(f"{op}: the step metadata is not for {rows} rows")
    if out is None:
        out = torch.empty_like(q)
    out = _out(op, "out", out, torch.float32, 3)
    if out.shape != q.shape:
        raise ValueError(f"{op}: out must be {tuple(q.shape)}, got {tuple(out.shape)}")
    ws, ws_bytes = (None, 0) if workspace is None else (workspace.data_ptr(), workspace.numel() * workspace.element_size())
    _lib.call("uocr_paged_decode_attention", out.data_ptr(), q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), rows,
              heads, head_dim, blocks.data_ptr(), pages, layers, page_size, int(layer_idx), lookup.data_ptr(),
              lookup.shape[1], attend.data_ptr(), int(kv.attend_max), write.data_ptr(), float(scale), ws, ws_bytes,
              _stream(q))
    return out


def paged_decode_attention_qkv(qkv, positions, cos_table, sin_table, *, heads: int, kv: PagedKv, layer_idx: int,
                               scale: float, out: torch.Tensor | None = None,
                               workspace: torch.Tensor | None = None) -> torch.Tensor:
    """:func:`rope` of q and k followed by :func:`paged_decode_attention`, in one launch and with the same
    bits: ``qkv [B, 3 * heads * head_dim]`` (q, k, v side by side, q and k before RoPE; rows may be
    strided) is one fused projection's output (unlimited_ocr_max/decoder.py:487-492 with :425-437)."""
    op = "paged_decode_attention_qkv"
    if not isinstance(qkv, torch.Tensor) or qkv.dtype != torch.float32 or qkv.dim() != 2 or qkv.device.type != "cuda":
        raise ValueError(f"{op}: qkv must be an fp32 [rows, 3 * heads * head_dim] GPU tensor")
    if qkv.stride(1) != 1:
        qkv = qkv.contiguous()
    rows, width = qkv.shape
    if width % (3 * heads):
        raise ValueError(f"{op}: qkv width {width} is not 3 x {heads} heads")
    head_dim = width // (3 * heads)
    positions = _gpu(op, "positions", positions, torch.int32, 1)
    cos_table = _gpu(op, "cos_table", cos_table, torch.float32, 2)
    sin_table = _gpu(op, "sin_table", sin_table, torch.float32, 2)
    if positions.shape[0] != rows or cos_table.shape != sin_table.shape:
        raise ValueError(f"{op}: positions or the cos/sin tables do not fit {rows} rows")
    blocks = kv.kv_blocks
    if not isinstance(blocks, torch.Tensor) or blocks.dtype != torch.float32 or blocks.dim() != 6 or \
            blocks.device.type != "cuda" or not blocks.is_contiguous():
        raise ValueError(f"{op}: kv_blocks must be a contiguous f32 [pages, 2, layers, page_size, heads, head_dim]")
    pages, two, layers, page_size, bh, bd = blocks.shape
    if two != 2 or (bh, bd) != (heads, head_dim):
        raise ValueError(f"{op}: kv_blocks {tuple(blocks.shape)} does not hold {heads} heads of {head_dim}")
    lookup = _u32(op, "lookup_table", kv.lookup_table, 2)
    attend = _u32(op, "attend_lengths", kv.attend_lengths, 1)
    write = _u32(op, "write_index", kv.write_index, 1)
    if lookup.shape[0] != rows or attend.shape[0] != rows or write.shape[0] != rows:
        raise ValueError(f"{op}: the step metadata is not for {rows} rows")
    if out is None:
        out = torch.empty((rows, heads, head_dim), device=qkv.device, dtype=torch.float32)
    out = _out(op, "out", out, torch.float32, 3)
    ws, ws_bytes = (None, 0) if workspace is None else (workspace.data_ptr(), workspace.numel() * workspace.element_size())
    _lib.call("uocr_paged_decode_attention_qkv", out.data_ptr(), qkv.data_ptr(), rows, heads, head_dim, qkv.stride(0),
              positions.data_ptr(), cos_table.data_ptr(), sin_table.data_ptr(), cos_table.shape[0],
              cos_table.shape[1], blocks.data_ptr(), pages, layers, page_size, int(layer_idx), lookup.data_ptr(),
              lookup.shape[1], attend.data_ptr(), int(kv.attend_max), write.data_ptr(), float(scale), ws, ws_bytes,
              _stream(qkv))
    return out


_OPS = {
    "moe_int8_qmv": moe_int8_qmv,
    "moe_bf16_qmv": moe_bf16_qmv,
    "int8_dequant_expert": int8_dequant_expert,
    "dense_bf16_qmv": dense_bf16_qmv,
    "ngram_block": ngram_block,
}


def custom(symbol: str, values: list, out: torch.Tensor | None = None, parameters: dict | None = None) -> list:
    """``ops.custom(symbol, values=[...])``-style dispatch; returns ``[result]``."""
    if symbol not in _OPS:
        raise KeyError(f"unknown custom op {symbol!r}; known: {sorted(_OPS)}")
    kwargs = dict(parameters or {})
    if out is not None:
        kwargs["out"] = out
    return [_OPS[symbol](*values, **kwargs)]


def kblocked(weight: torch.Tensor) -> torch.Tensor:
    """``W [N, K]`` as ``[K/16, N, 16]`` (unlimited_ocr_max/weight_adapters.py:222-233)."""
    n, k = weight.shape
    if k % KBLOCK:
        raise ValueError(f"a K-blocked projection needs K to be a multiple of {KBLOCK}, got shape {tuple(weight.shape)}")
    return weight.reshape(n, k // KBLOCK, KBLOCK).permute(1, 0, 2).contiguous()


def quantize_per_group(w: torch.Tensor, group: int = INT8_GROUP_SIZE) -> tuple[torch.Tensor, torch.Tensor]:
    """Symmetric per-group int8 of a GPU tensor ``[..., K]`` along K (tools/quantize_int8.py:54-70,298-329):
    ``scale = amax/127`` (1.0 for an all-zero group), ``q = clip(rint(w/scale), -127, 127)``, in fp32 with
    correctly rounded divisions (bitwise the reference's numpy) -> ``(int8 [..., K], fp32 [..., K/group])``.
    bf16 and fp32 weights are read as they are; other float dtypes are converted to fp32 first."""
    op = "quantize_per_group"
    if not isinstance(w, torch.Tensor) or w.dim() < 1:
        raise TypeError(f"{op}: w must be a torch.Tensor of rank >= 1")
    k = int(w.shape[-1])
    if k % group:
        raise ValueError(f"K={k} is not divisible by the group size {group}")
    if w.dtype not in (torch.bfloat16, torch.float32):
        w = w.float()
    w = _gpu(op, "w", w, w.dtype, w.dim())
    if not bool(torch.isfinite(w).all()):
        raise ValueError("weight holds NaN or Inf; refusing to quantise it")
    q = torch.empty(w.shape, dtype=torch.int8, device=w.device)
    scales = torch.empty((*w.shape[:-1], k // group), dtype=torch.float32, device=w.device)
    rows = w.numel() // k if k else 0
    _lib.call("uocr_quantize_per_group", q.data_ptr(), scales.data_ptr(), w.data_ptr(), int(w.dtype == torch.bfloat16),
              rows, k, group, _stream(w))
    return q, scales
