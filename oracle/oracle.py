"""ctypes front end of the CPU oracle (``oracle/liboracle.so``) plus its float64 closed forms.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py``, as the checker or the timed CPU baseline.
The product never imports it.

Arrays cross as numpy; bf16 tensors travel as their ``uint16`` bit patterns.
"""

from __future__ import annotations

import ctypes
import subprocess
from dataclasses import dataclass
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64


def build(force: bool = False) -> Path:
    """Compile ``liboracle.so`` with the committed Makefile (host compiler only)."""
    args = ["make", "-C", str(HERE)] + (["-B"] if force else [])
    subprocess.run(args, check=True, stdout=subprocess.DEVNULL)
    return LIB_PATH


class _Layer(ctypes.Structure):
    _fields_ = [
        ("E", _i64), ("H", _i64), ("F", _i64), ("Fs", _i64), ("topk", _i64), ("group", _i64),
        ("int8", ctypes.c_int), ("renorm", ctypes.c_int),
        ("router", ctypes.c_void_p),
        ("gate_w", ctypes.c_void_p), ("up_w", ctypes.c_void_p), ("down_w", ctypes.c_void_p),
        ("gate_s", ctypes.c_void_p), ("up_s", ctypes.c_void_p), ("down_s", ctypes.c_void_p),
        ("sh_gate", ctypes.c_void_p), ("sh_up", ctypes.c_void_p), ("sh_down", ctypes.c_void_p),
    ]


_LIB = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.or_bf16_rne.argtypes = [ctypes.c_float]
        L.or_bf16_rne.restype = ctypes.c_uint16
        L.or_uexp.argtypes = [ctypes.c_float]
        L.or_uexp.restype = ctypes.c_float
        L.or_silu.argtypes = [ctypes.c_float]
        L.or_silu.restype = ctypes.c_float
        L.or_uexp_array.argtypes = [_f32p, _f32p, _i64]
        L.or_silu_array.argtypes = [_f32p, _f32p, _i64]
        L.or_threads.argtypes = [ctypes.c_int]
        L.or_threads.restype = ctypes.c_int
        L.or_quantize_per_group.argtypes = [_f32p, _i64, _i64, _i64, _i8p, _f32p]
        L.or_moe_int8_qmv.argtypes = [_f32p, _f32p, _i32p, _i8p, _f32p, _i64, _i64, _i64, _i64, _i64, ctypes.c_int]
        L.or_moe_bf16_qmv_ref.argtypes = [_f32p, _f32p, _i32p, _u16p, _i64, _i64, _i64, _i64, ctypes.c_int]
        L.or_moe_bf16_qmv_chunked.argtypes = [_f32p, _f32p, _i32p, _u16p, _i64, _i64, _i64, _i64, ctypes.c_int]
        L.or_dense_bf16_qmv_ref.argtypes = [_f32p, _f32p, _u16p, _i64, _i64, _i64, _i64, ctypes.c_int]
        L.or_dense_bf16_qmv_chunked.argtypes = [_f32p, _f32p, _u16p, _i64, _i64, _i64, ctypes.c_int]
        L.or_int8_dequant_expert.argtypes = [_u16p, _i8p, _f32p, ctypes.c_int32, _i64, _i64, _i64, _i64]
        L.or_dot_tree64.argtypes = [_f32p, _f32p, _i64]
        L.or_dot_tree64.restype = ctypes.c_float
        L.or_moe_gate.argtypes = [_i32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64, ctypes.c_int]
        L.or_moe_decode_exact.argtypes = [_f32p, _i32p, _f32p, _f32p, _i64, ctypes.POINTER(_Layer), ctypes.c_int]
        L.or_moe_decode_refdecomp.argtypes = [_f32p, _f32p, _i64, ctypes.POINTER(_Layer), ctypes.c_int]
        _LIB = L
    return _LIB


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ValueError(f"oracle {what} failed with code {rc}")


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------------------
# bf16 bits (unlimited_ocr_max/bf16.py:110-136; tests/_harness.py:36-49)
# ---------------------------------------------------------------------------


def bf16_bits(values: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round-to-nearest-even, NaN to 0x7FC0 (numpy twin of ``or_bf16_rne``)."""
    bits = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32)
    carry = ((bits & np.uint32(0xFFFF)) + ((bits >> 16) & np.uint32(1)) + np.uint32(0x7FFF)) >> 16
    out = ((bits >> 16) + carry).astype(np.uint16)
    nan = np.isnan(np.asarray(values, dtype=np.float32))
    out[nan] = 0x7FC0
    return out


def bf16_values(bits: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def clamp(e: int, num_experts: int) -> int:
    return min(max(int(e), 0), num_experts - 1)


def kblocked(w_bits: np.ndarray, kblock: int = 16) -> np.ndarray:
    """``W [N, K]`` as ``[K/16, N, 16]`` (unlimited_ocr_max/weight_adapters.py:222-233)."""
    n, k = w_bits.shape
    if k % kblock:
        raise ValueError(f"K={k} is not a multiple of {kblock}")
    return np.ascontiguousarray(w_bits.reshape(n, k // kblock, kblock).transpose(1, 0, 2))


def unkblocked(w_kb: np.ndarray) -> np.ndarray:
    kb, n, width = w_kb.shape
    return np.ascontiguousarray(w_kb.transpose(1, 0, 2).reshape(n, kb * width))


# ---------------------------------------------------------------------------
# scalar functions
# ---------------------------------------------------------------------------


def uexp(x: float) -> float:
    return float(lib().or_uexp(float(x)))


def silu(x: float) -> float:
    return float(lib().or_silu(float(x)))


def uexp_array(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty_like(x)
    lib().or_uexp_array(out, x, x.size)
    return out


def silu_array(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty_like(x)
    lib().or_silu_array(out, x, x.size)
    return out


def threads(n: int = 0) -> int:
    return int(lib().or_threads(n))


# ---------------------------------------------------------------------------
# quantiser (tools/quantize_int8.py:298-329)
# ---------------------------------------------------------------------------


def quantize_per_group(w: np.ndarray, group: int = 128) -> tuple[np.ndarray, np.ndarray]:
    w = _c(w, np.float32)
    n, k = w.shape
    q = np.empty((n, k), np.int8)
    s = np.empty((n, k // group), np.float32)
    _check(lib().or_quantize_per_group(w, n, k, group, q, s), "quantize_per_group")
    return q, s


def quantize_stack(w: np.ndarray, group: int = 128) -> tuple[np.ndarray, np.ndarray]:
    """A ``[E, N, K]`` fp32 stack quantised expert by expert."""
    e, n, k = w.shape
    q, s = quantize_per_group(w.reshape(e * n, k), group)
    return q.reshape(e, n, k), s.reshape(e, n, k // group)


# ---------------------------------------------------------------------------
# the reference's ops
# ---------------------------------------------------------------------------


def moe_int8_qmv(x, ids, w, scales, threads: int = 0) -> np.ndarray:
    x, ids, w, scales = _c(x, np.float32), _c(ids, np.int32), _c(w, np.int8), _c(scales, np.float32)
    k, K = x.shape
    E, N, _ = w.shape
    out = np.zeros((k, N), np.float32)
    _check(lib().or_moe_int8_qmv(out, x, ids, w, scales, k, E, N, K, scales.shape[2], threads), "moe_int8_qmv")
    return out


def moe_bf16_qmv_ref(x, ids, w_bits, threads: int = 0) -> np.ndarray:
    x, ids, w = _c(x, np.float32), _c(ids, np.int32), _c(w_bits, np.uint16)
    k, K = x.shape
    E, N, _ = w.shape
    out = np.zeros((k, N), np.float32)
    _check(lib().or_moe_bf16_qmv_ref(out, x, ids, w, k, E, N, K, threads), "moe_bf16_qmv_ref")
    return out


def moe_bf16_qmv_chunked(x, ids, w_bits, threads: int = 0) -> np.ndarray:
    x, ids, w = _c(x, np.float32), _c(ids, np.int32), _c(w_bits, np.uint16)
    k, K = x.shape
    E, N, _ = w.shape
    out = np.zeros((k, N), np.float32)
    _check(lib().or_moe_bf16_qmv_chunked(out, x, ids, w, k, E, N, K, threads), "moe_bf16_qmv_chunked")
    return out


def dense_bf16_qmv_ref(x, w_kb, tile: int, threads: int = 0) -> np.ndarray:
    x, w = _c(x, np.float32), _c(w_kb, np.uint16)
    M, K = x.shape
    N = w.shape[1]
    out = np.zeros((M, N), np.float32)
    _check(lib().or_dense_bf16_qmv_ref(out, x, w, M, N, K, tile, threads), "dense_bf16_qmv_ref")
    return out


def dense_bf16_qmv_chunked(x, w_kb, threads: int = 0) -> np.ndarray:
    x, w = _c(x, np.float32), _c(w_kb, np.uint16)
    M, K = x.shape
    N = w.shape[1]
    out = np.zeros((M, N), np.float32)
    _check(lib().or_dense_bf16_qmv_chunked(out, x, w, M, N, K, threads), "dense_bf16_qmv_chunked")
    return out


def int8_dequant_expert(w, scales, idx: int) -> np.ndarray:
    w, scales = _c(w, np.int8), _c(scales, np.float32)
    E, N, K = w.shape
    out = np.zeros((N, K), np.uint16)
    _check(lib().or_int8_dequant_expert(out, w, scales, int(idx), E, N, K, scales.shape[2]), "int8_dequant_expert")
    return out


def dot_tree64(a, b) -> float:
    a, b = _c(a, np.float32), _c(b, np.float32)
    return float(lib().or_dot_tree64(a, b, a.shape[0]))


def moe_gate(x, router, topk: int = 6, renorm: bool = False) -> tuple[np.ndarray, np.ndarray]:
    x, router = _c(x, np.float32), _c(router, np.float32)
    T, H = x.shape
    E = router.shape[0]
    ids = np.zeros((T, topk), np.int32)
    wts = np.zeros((T, topk), np.float32)
    _check(lib().or_moe_gate(ids, wts, x, router, T, E, H, topk, int(renorm)), "moe_gate")
    return ids, wts


# ---------------------------------------------------------------------------
# one MoE layer's weights
# ---------------------------------------------------------------------------


@dataclass
class MoeWeights:
    """One MoE layer as numpy arrays, in the reference's declared layouts.

    Routed stacks ``[E, F, H]`` / ``[E, F, H]`` / ``[E, H, F]``: int8 with fp32
    scales ``[E, N, K/group]`` when ``int8``, else bf16 bit patterns (uint16).
    Shared experts bf16 bits K-blocked ``[H/16, Fs, 16]`` / ``[H/16, Fs, 16]`` /
    ``[Fs/16, H, 16]``; router fp32 ``[E, H]``.
    """

    router: np.ndarray
    gate: np.ndarray
    up: np.ndarray
    down: np.ndarray
    sh_gate: np.ndarray
    sh_up: np.ndarray
    sh_down: np.ndarray
    gate_s: np.ndarray | None = None
    up_s: np.ndarray | None = None
    down_s: np.ndarray | None = None
    topk: int = 6
    group: int = 128
    renorm: bool = False

    @property
    def int8(self) -> bool:
        return self.gate.dtype == np.int8

    @property
    def dims(self) -> tuple[int, int, int, int]:
        E, F, H = self.gate.shape
        return E, H, F, self.sh_gate.shape[1]

    def _struct(self) -> _Layer:
        E, H, F, Fs = self.dims
        keep = [_c(self.router, np.float32), self.gate, self.up, self.down, self.sh_gate, self.sh_up, self.sh_down]
        if self.int8:
            keep += [_c(self.gate_s, np.float32), _c(self.up_s, np.float32), _c(self.down_s, np.float32)]
        for a in keep:
            if not a.flags.c_contiguous:
                raise ValueError("layer arrays must be C-contiguous")
        ptr = lambda a: a.ctypes.data  # noqa: E731
        s = _Layer(E, H, F, Fs, self.topk, self.group, int(self.int8), int(self.renorm), ptr(keep[0]),
                   ptr(self.gate), ptr(self.up), ptr(self.down),
                   ptr(keep[7]) if self.int8 else None, ptr(keep[8]) if self.int8 else None,
                   ptr(keep[9]) if self.int8 else None,
                   ptr(self.sh_gate), ptr(self.sh_up), ptr(self.sh_down))
        s._keep = keep  # keep the buffers alive with the struct
        return s


def moe_decode_exact(x, layer: MoeWeights, threads: int = 0):
    """``(out, ids, weights)`` of the decode layer in the HIP path's exact orders."""
    x = _c(x, np.float32)
    B, H = x.shape
    out = np.zeros((B, H), np.float32)
    ids = np.zeros((B, layer.topk), np.int32)
    wts = np.zeros((B, layer.topk), np.float32)
    s = layer._struct()
    _check(lib().or_moe_decode_exact(out, ids, wts, x, B, ctypes.byref(s), threads), "moe_decode_exact")
    return out, ids, wts


def moe_decode_refdecomp(x, layer: MoeWeights, threads: int = 0) -> np.ndarray:
    """The decode layer in the reference's own CPU decomposition (the timed CPU baseline)."""
    x = _c(x, np.float32)
    B, H = x.shape
    out = np.zeros((B, H), np.float32)
    s = layer._struct()
    _check(lib().or_moe_decode_refdecomp(out, x, B, ctypes.byref(s), threads), "moe_decode_refdecomp")
    return out


# ---------------------------------------------------------------------------
# float64 closed forms
# ---------------------------------------------------------------------------


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """``max |got - ref| / max |ref|`` in float64 (tests/_harness.py:52-58)."""
    got64, ref64 = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    denom = float(np.max(np.abs(ref64))) if ref64.size else 0.0
    if ref64.size == 0:
        return 0.0
    if denom == 0.0:
        return float(np.max(np.abs(got64)))
    return float(np.max(np.abs(got64 - ref64)) / denom)


def cosine(a: np.ndarray, b: np.ndarray) -> float:
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def qmv_int8_f64(x, ids, w, scales) -> np.ndarray:
    """tests/test_kernels_int8.py:150-162, ids clamped."""
    xf, wf, sf = (np.asarray(a, np.float64) for a in (x, w, scales))
    k = x.shape[0]
    E, N, K = w.shape
    groups = scales.shape[2]
    out = np.empty((k, N), np.float64)
    for s in range(k):
        e = clamp(ids[s], E)
        gsums = (wf[e] * xf[s]).reshape(N, groups, K // groups).sum(axis=2)
        out[s] = (sf[e] * gsums).sum(axis=1)
    return out


def qmv_bf16_f64(x, ids, w_bits) -> np.ndarray:
    """tests/test_kernels_bf16.py:118-122, ids clamped."""
    xf, wf = np.asarray(x, np.float64), bf16_values(w_bits).astype(np.float64)
    E = w_bits.shape[0]
    if x.shape[0] == 0:
        return np.zeros((0, w_bits.shape[1]))
    return np.stack([wf[clamp(ids[s], E)] @ xf[s] for s in range(x.shape[0])])


def dense_f64(x, w_kb) -> np.ndarray:
    """tests/test_kernels_dense_bf16.py:86-87 on the K-blocked weight."""
    return np.asarray(x, np.float64) @ bf16_values(unkblocked(w_kb)).astype(np.float64).T


def _silu64(a: np.ndarray) -> np.ndarray:
    return a / (1.0 + np.exp(-a))


def gate_f64(x, router, topk: int = 6, renorm: bool = False):
    """``(ids, weights, probs)``: float64 softmax and stable-argsort top-k (tests/test_decoder_int8.py:724-727)."""
    logits = np.asarray(x, np.float64) @ np.asarray(router, np.float64).T
    probs = np.exp(logits - logits.max(axis=1, keepdims=True))
    probs /= probs.sum(axis=1, keepdims=True)
    ids = np.argsort(-probs, axis=1, kind="stable")[:, :topk]
    wts = np.take_along_axis(probs, ids, axis=1)
    if renorm:
        wts = wts / wts.sum(axis=1, keepdims=True)
    return ids.astype(np.int32), wts, probs


def routed_stacks_f64(layer: MoeWeights, bf16_dequant: bool = False) -> list[np.ndarray]:
    """The three routed stacks' values in float64: exact ``q * scale`` (decode's arithmetic,
    tests/test_decoder_int8.py:709-711) or, with ``bf16_dequant``, ``bf16_rne(f32(q)*scale)``
    (the prefill's, unlimited_ocr_max/kernels/moe_int8.mojo:340)."""
    out = []
    for w, s in ((layer.gate, layer.gate_s), (layer.up, layer.up_s), (layer.down, layer.down_s)):
        if layer.int8:
            g = w.shape[2] // s.shape[2]
            if bf16_dequant:
                v = w.astype(np.float32) * np.repeat(s.astype(np.float32), g, axis=2)
                out.append(bf16_values(bf16_bits(v)).astype(np.float64))
            else:
                out.append(w.astype(np.float64) * np.repeat(s.astype(np.float64), g, axis=2))
        else:
            out.append(bf16_values(w).astype(np.float64))
    return out


def moe_layer_f64(x, layer: MoeWeights, ids=None, wts=None, bf16_dequant: bool = False) -> np.ndarray:
    """The MoE layer in float64 (tests/test_decoder_int8.py:720-732), every token independently.

    ``ids``/``wts`` default to the float64 gate; pass the oracle gate's to compare
    the expert math alone (so that a near-tie in the 6th place cannot swap an expert).
    """
    xf = np.asarray(x, np.float64)
    if ids is None:
        ids, wts, _ = gate_f64(x, layer.router, layer.topk, layer.renorm)
    wts = np.asarray(wts, np.float64)
    gate, up, down = routed_stacks_f64(layer, bf16_dequant)
    sg, su, sd = (bf16_values(unkblocked(w)).astype(np.float64) for w in (layer.sh_gate, layer.sh_up, layer.sh_down))
    out = np.zeros_like(xf)
    for t in range(xf.shape[0]):
        routed = np.zeros(xf.shape[1])
        for j in range(ids.shape[1]):
            e = int(ids[t, j])
            routed += wts[t, j] * (down[e] @ (_silu64(gate[e] @ xf[t]) * (up[e] @ xf[t])))
        out[t] = routed + sd @ (_silu64(sg @ xf[t]) * (su @ xf[t]))
    return out


def moe_layer_f64_grouped(x, layer: MoeWeights, ids, wts, bf16_dequant: bool = False,
                          rows: np.ndarray | None = None) -> np.ndarray:
    """:func:`moe_layer_f64` with each expert's tokens batched into one float64 matmul (same closed form,
    other summation order; for prefill-sized T).  ``rows`` restricts the result to those token rows."""
    xf = np.asarray(x, np.float64)
    ids = np.asarray(ids)
    wts = np.asarray(wts, np.float64)
    if rows is not None:
        xf, ids, wts = xf[rows], ids[rows], wts[rows]
    gate, up, down = routed_stacks_f64(layer, bf16_dequant)
    sg, su, sd = (bf16_values(unkblocked(w)).astype(np.float64) for w in (layer.sh_gate, layer.sh_up, layer.sh_down))
    out = (_silu64(xf @ sg.T) * (xf @ su.T)) @ sd.T
    for e in np.unique(ids):
        tok, slot = np.nonzero(ids == e)
        xe = xf[tok]
        y = (_silu64(xe @ gate[e].T) * (xe @ up[e].T)) @ down[e].T
        np.add.at(out, tok, wts[tok, slot][:, None] * y)
    return out


# ---------------------------------------------------------------------------
# the n-gram guard (unlimited_ocr_max/kernels/ngram_block.mojo)
# ---------------------------------------------------------------------------

#: ngram_block.mojo:49, as the float32 it lands in.
NGRAM_BLOCKED = np.float32(-3.0e38)


def ngram_banned(sequence, ngram_size: int, window: int) -> set[int]:
    """The reference processor's banned ids, over the WHOLE sequence with an explicit window
    (``SlidingWindowNoRepeatNgramProcessor`` as restated in ngram_block.mojo:5-15)."""
    ids = [int(i) for i in sequence]
    if ngram_size < 1 or len(ids) < ngram_size:
        return set()
    search_start = max(0, len(ids) - window)
    search_end = len(ids) - ngram_size + 1
    prefix = tuple(ids[len(ids) - (ngram_size - 1):]) if ngram_size > 1 else ()  # sequence[-0:] is all of it
    banned: set[int] = set()
    for idx in range(search_start, search_end):
        gram = ids[idx: idx + ngram_size]
        if ngram_size == 1 or tuple(gram[:-1]) == prefix:
            banned.add(gram[-1])
    return banned


def ngram_banned_per_id(history, ngram_size: int, vocab: int) -> set[int]:
    """The same set as the op's work items compute it (ngram_block.mojo:112-146): for every vocabulary id,
    a scan of every start of the windowed history.  Brute force, for small vocabularies."""
    h = [int(i) for i in history]
    if ngram_size < 1 or len(h) < ngram_size:
        return set()
    prefix_len = ngram_size - 1
    starts = len(h) - ngram_size + 1
    prefix_at = len(h) - prefix_len
    out = set()
    for token in range(vocab):
        for start in range(starts):
            if h[start + prefix_len] != token:
                continue
            if all(h[start + j] == h[prefix_at + j] for j in range(prefix_len)):
                out.add(token)
                break
    return out


def ngram_block(logits: np.ndarray, history: np.ndarray, ngram_size: int) -> np.ndarray:
    """The op: ``logits [V]`` / ``[B, V]`` with row b's banned ids (from history row b, the row's last
    ids) set to :data:`NGRAM_BLOCKED`; ids outside ``[0, V)`` ban nothing."""
    out = np.array(logits, dtype=np.float32, copy=True)
    rows = out.reshape(-1, out.shape[-1])
    hist = np.asarray(history).reshape(rows.shape[0], -1)
    for b in range(rows.shape[0]):
        banned = [v for v in ngram_banned(hist[b], ngram_size, hist.shape[1]) if 0 <= v < rows.shape[1]]
        rows[b, banned] = NGRAM_BLOCKED
    return out


# ---------------------------------------------------------------------------
# paged decode attention (unlimited_ocr_max/decoder.py:425-437 over kv_cache.py's pool)
# ---------------------------------------------------------------------------


def paged_row(kv_blocks: np.ndarray, lookup_row: np.ndarray, r: int, kv: int, layer: int) -> np.ndarray:
    """Logical row ``r`` of one request, ``[heads, D]``: slot ``r % P`` of page ``lookup_row[r // P]``
    (kv_cache.py:17-19) in ``kv_blocks [pages, 2, layers, P, heads, D]``."""
    P = kv_blocks.shape[3]
    return kv_blocks[int(lookup_row[r // P]), kv, layer, r % P]


def paged_decode_attention(q, k_new, v_new, kv_blocks, lookup, attend_lengths, write_index, layer: int,
                           scale: float) -> tuple[np.ndarray, np.ndarray]:
    """``(out float64 [B, heads, D], the pool after the store)``.

    The store (store_k/v_cache_ragged at ``write_index``, decoder.py:434-435) on a copy of the pool, then
    per row ``b`` the chain the reference's test holds the op to (tests/test_kv_cache.py:339-349): the
    rows ``[0, attend_lengths[b] + 1)``, read back through the lookup table, ``softmax(q k^T * scale) @ v``
    in float64.  Rows are stored in order, so two rows that write one slot leave the later row's values,
    and row ``b`` reads the pool after every store.
    """
    pool = np.array(kv_blocks, dtype=np.float32, copy=True)
    B = q.shape[0]
    P = pool.shape[3]
    for b in range(B):
        w = int(write_index[b])
        page = int(lookup[b, w // P])
        pool[page, 0, layer, w % P] = k_new[b]
        pool[page, 1, layer, w % P] = v_new[b]
    out = np.zeros(q.shape, np.float64)
    for b in range(B):
        n = int(attend_lengths[b]) + 1
        k = np.stack([paged_row(pool, lookup[b], r, 0, layer) for r in range(n)]).astype(np.float64)  # [n, h, D]
        v = np.stack([paged_row(pool, lookup[b], r, 1, layer) for r in range(n)]).astype(np.float64)
        scores = np.einsum("hd,lhd->hl", q[b].astype(np.float64), k) * scale
        weights = np.exp(scores - scores.max(axis=-1, keepdims=True))
        weights /= weights.sum(axis=-1, keepdims=True)
        out[b] = np.einsum("hl,lhd->hd", weights, v)
    return out, pool


# ---------------------------------------------------------------------------
# the decoder layer's per-row steps (unlimited_ocr_max/decoder.py)
# ---------------------------------------------------------------------------


def rms_norm(x, gamma, eps: float, residual=None) -> tuple[np.ndarray, np.ndarray]:
    """``(out float64, v float32)``: ``v = x + residual`` in fp32 (or ``x``), then ``RmsNorm``
    (decoder.py:252-261) in float64: ``v / sqrt(mean(v^2) + eps) * gamma``."""
    v = np.asarray(x, np.float32)
    if residual is not None:
        v = (v + np.asarray(residual, np.float32)).astype(np.float32)
    v64 = v.astype(np.float64)
    r = 1.0 / np.sqrt(np.mean(v64 * v64, axis=-1, keepdims=True) + eps)
    return v64 * r * np.asarray(gamma, np.float64), v


def rope_tables(*, head_dim: int, seq_len: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """``(cos, sin) [seq_len, head_dim]`` in float32 as the reference builds them (decoder.py:115-123):
    inverse frequencies ``1 / theta^(2i/D)``, angles ``position * inv_freq``, duplicated halves."""
    exponent = np.arange(0, head_dim, 2, dtype=np.int64).astype(np.float32)
    inv_freq = (1.0 / (np.float32(theta) ** (exponent / np.float32(head_dim)))).astype(np.float32)
    angles = np.arange(seq_len, dtype=np.int64).astype(np.float32)[:, None] * inv_freq[None, :]
    emb = np.concatenate([angles, angles], axis=-1).astype(np.float32)
    return np.cos(emb).astype(np.float32), np.sin(emb).astype(np.float32)


def rope(x, positions, cos_t, sin_t) -> np.ndarray:
    """``Attention._rope`` (decoder.py:459-462) on ``x [rows, heads, D]`` with row ``b`` at
    ``positions[b]``: ``x * cos + rotate_half(x) * sin`` in float32, each product and the sum rounded
    (numpy's elementwise float32)."""
    x = np.asarray(x, np.float32)
    half = x.shape[-1] // 2
    rotated = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    c = np.asarray(cos_t, np.float32)[np.asarray(positions)][:, None, :]
    s = np.asarray(sin_t, np.float32)[np.asarray(positions)][:, None, :]
    return (x * c + rotated * s).astype(np.float32)


def swiglu(gate_up) -> np.ndarray:
    """``silu(gate) * up`` (decoder.py:274-276) over ``[rows, 2F]``, with the oracle's fp32 silu."""
    gu = np.asarray(gate_up, np.float32)
    f = gu.shape[-1] // 2
    return (silu_array(np.ascontiguousarray(gu[..., :f])) * gu[..., f:]).astype(np.float32)


# ---------------------------------------------------------------------------
# synthetic layers
# ---------------------------------------------------------------------------


def make_layer(seed: int, *, E: int = 64, H: int = 1280, F: int = 896, n_shared: int = 2, topk: int = 6,
               int8: bool = True, std: float = 0.02, router_std: float = 0.02, group: int = 128) -> MoeWeights:
    """One layer of seeded ``N(0, std)`` weights rounded to bf16, int8-quantised per group when ``int8``.

    Draw order: router, gate, up, down stacks, shared gate, up, down.
    """
    rng = np.random.default_rng(seed)
    Fs = n_shared * F
    router = bf16_values(bf16_bits(rng.standard_normal((E, H), dtype=np.float32) * np.float32(router_std)))
    stacks = []
    for shape in ((E, F, H), (E, F, H), (E, H, F)):
        stacks.append(bf16_bits(rng.standard_normal(shape, dtype=np.float32) * np.float32(std)))
    shared = []
    for n, k in ((Fs, H), (Fs, H), (H, Fs)):
        shared.append(kblocked(bf16_bits(rng.standard_normal((n, k), dtype=np.float32) * np.float32(std))))
    kw = dict(router=np.ascontiguousarray(router), sh_gate=shared[0], sh_up=shared[1], sh_down=shared[2],
              topk=topk, group=group)
    if not int8:
        return MoeWeights(gate=stacks[0], up=stacks[1], down=stacks[2], **kw)
    q = [quantize_stack(bf16_values(s), group) for s in stacks]
    return MoeWeights(gate=q[0][0], up=q[1][0], down=q[2][0], gate_s=q[0][1], up_s=q[1][1], down_s=q[2][1], **kw)


def rmsnorm_rows(rng: np.random.Generator, rows: int, dim: int) -> np.ndarray:
    """``rows`` of N(0, 1) normalised to unit RMS (RMSNorm with gamma = 1)."""
    x = rng.standard_normal((rows, dim), dtype=np.float32)
    rms = np.sqrt(np.mean(x.astype(np.float64) ** 2, axis=1, keepdims=True) + 1e-6)
    return (x / rms).astype(np.float32)

