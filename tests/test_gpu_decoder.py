"""GPU parity of the decoder-step ops and of the decode step they make up, through the C ABI.

* ``rms_norm`` (with and without the fused residual add, in place, rows of 1280 and of 100):
  within 1e-6 relative of the float64 norm; the residual sum is bitwise the fp32 sum.
* ``rope``: bitwise the oracle's float32 (numpy elementwise) at positions 0, 1, 255, 639 and one past the
  table (clamped into it), from the strided thirds of a fused q/k/v buffer; v copied bitwise.
* ``swiglu``: bitwise the oracle's fp32 silu times up.
* ``Decoder.decode``: a 3-layer decoder at the real attention and hidden sizes (10 heads x 128; layer 0
  dense, layers 1-2 int8 MoE with 8 experts), two requests with seeded KV pages, two decode steps; the
  final norm and the logits within 1e-4 relative of the oracle's chain in float64 (dense projections,
  paged attention, MoE layer and norms of the oracle), and every layer's new k/v rows stored.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from _gpu import layer_weights, n, t

pytestmark = pytest.mark.gpu


def _ops():
    import uocr_moe

    return uocr_moe


def _rel(got, want) -> float:
    return float(np.max(np.abs(np.asarray(got, np.float64) - want)) / np.max(np.abs(want)))


@pytest.mark.parametrize("dim", [1280, 100])
@pytest.mark.parametrize("resid", [False, True])
def test_rms_norm(oracle, dim, resid) -> None:
    rng = np.random.default_rng(dim + resid)
    x = rng.standard_normal((8, dim)).astype(np.float32)
    d = rng.standard_normal((8, dim)).astype(np.float32) if resid else None
    g = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
    want, v = oracle.rms_norm(x, g, 1e-6, residual=d)
    xg = t(x)
    got = _ops().rms_norm(xg, t(g), 1e-6, residual=None if d is None else t(d))
    assert _rel(n(got), want) <= 1e-6
    assert np.array_equal(n(xg).view(np.uint32), v.view(np.uint32))  # in place: x + residual (or x)


def test_rope_from_a_fused_qkv_buffer(oracle) -> None:
    rng = np.random.default_rng(5)
    B, H, D, seq = 5, 10, 128, 640
    cos_t, sin_t = oracle.rope_tables(head_dim=D, seq_len=seq, theta=10000.0)
    qkv = rng.standard_normal((B, 3, H, D)).astype(np.float32)
    pos = np.array([0, 1, 255, 639, 640], np.int32)  # the last one past the table: clamped to 639
    g = t(qkv)
    q, k, v = _ops().rope(g[:, 0], g[:, 1], t(pos), t(cos_t), t(sin_t), v=g[:, 2])
    clamped = np.minimum(pos, seq - 1)
    assert np.array_equal(n(q).view(np.uint32), oracle.rope(qkv[:, 0], clamped, cos_t, sin_t).view(np.uint32))
    assert np.array_equal(n(k).view(np.uint32), oracle.rope(qkv[:, 1], clamped, cos_t, sin_t).view(np.uint32))
    assert np.array_equal(n(v).view(np.uint32), qkv[:, 2].view(np.uint32))
    inplace = t(np.ascontiguousarray(qkv[:, 0]))
    _ops().rope(inplace, None, t(pos), t(cos_t), t(sin_t), q_out=inplace)
    assert np.array_equal(n(inplace), n(q))


@pytest.mark.parametrize("B", [1, 3])
def test_attention_with_rope_in_the_kernel_equals_rope_then_attention(oracle, B) -> None:
    """``paged_decode_attention_qkv`` (RoPE of q and k inside the attention kernel, read from a fused
    projection's output) gives the bits of ``rope`` followed by ``paged_decode_attention``: the output and
    every pool word."""
    uocr = _ops()
    rng = np.random.default_rng(30 + B)
    H, D, P, layers, seq = 10, 128, 128, 2, 1024
    cos_t, sin_t = oracle.rope_tables(head_dim=D, seq_len=seq, theta=10000.0)
    pages = 4 * B + 1
    pool = rng.standard_normal((pages, 2, layers, P, H, D)).astype(np.float32)
    perm = rng.permutation(pages - 1)
    lut = np.full((B, 5), pages - 1, np.uint32)
    lut[:, :4] = perm[: 4 * B].reshape(B, 4)
    attend = np.array([300, 129, 512][:B], np.uint32)
    write = np.array([299, 60, 511][:B], np.uint32)  # appends and a ring overwrite
    pos = np.array([299, 900, 511][:B], np.int32)
    # the fused projection's output, rows 64 floats wider than q, k and v (a strided view)
    g = t(rng.standard_normal((B, 3 * H * D + 64)).astype(np.float32))[:, : 3 * H * D]

    def kv_of(gpu_pool):
        return uocr.PagedKv(kv_blocks=gpu_pool, lookup_table=t(lut.view(np.int32)),
                            attend_lengths=t((attend - 1).view(np.int32)), attend_max=int(attend.max()),
                            write_index=t(write.view(np.int32)))

    cos_g, sin_g, pos_g = t(cos_t), t(sin_t), t(pos)
    two = t(pool)
    q, k, v = uocr.rope(g[:, : H * D].view(B, H, D), g[:, H * D: 2 * H * D].view(B, H, D), pos_g, cos_g, sin_g,
                        v=g[:, 2 * H * D:].view(B, H, D))
    want = n(uocr.paged_decode_attention(q, k, v, kv=kv_of(two), layer_idx=1, scale=1 / math.sqrt(D)))
    one = t(pool)
    got = n(uocr.paged_decode_attention_qkv(g, pos_g, cos_g, sin_g, heads=H, kv=kv_of(one), layer_idx=1,
                                            scale=1 / math.sqrt(D)))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(n(one).view(np.uint32), n(two).view(np.uint32))


@pytest.mark.parametrize("rows", [1, 2])
@pytest.mark.parametrize("resid", [False, True])
def test_norm_inside_the_projection_equals_norm_then_projection(oracle, rows, resid) -> None:
    uocr = _ops()
    rng = np.random.default_rng(40 + rows + resid)
    x = rng.standard_normal((rows, 1280)).astype(np.float32)
    d = rng.standard_normal((rows, 1280)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(1280)).astype(np.float32)
    w = t(_bf16_kb(rng, 3840, 1280, 0.03))
    x_out = torch.full((rows, 1280), float("nan"), device="cuda:0")
    got = uocr.rms_norm_dense_bf16_qmv(t(x), t(g), 1e-6, w, residual=t(d) if resid else None,
                                       x_out=x_out if resid else None)
    xs = t(x)
    want = uocr.dense_bf16_qmv(uocr.rms_norm(xs, t(g), 1e-6, residual=t(d) if resid else None), w)
    assert np.array_equal(n(got).view(np.uint32), n(want).view(np.uint32))
    if resid:
        assert np.array_equal(n(x_out).view(np.uint32), n(xs).view(np.uint32))
        with pytest.raises(uocr.UocrError, match="must not overlap"):
            xg = t(x)
            uocr.rms_norm_dense_bf16_qmv(xg, t(g), 1e-6, w, residual=t(d), x_out=xg)


def test_swiglu(oracle) -> None:
    rng = np.random.default_rng(6)
    gu = (4 * rng.standard_normal((8, 2 * 6848))).astype(np.float32)
    got = n(_ops().swiglu(t(gu)))
    assert np.array_equal(got.view(np.uint32), oracle.swiglu(gu).view(np.uint32))


def test_refusals() -> None:
    uocr = _ops()
    dev = "cuda:0"
    x = torch.zeros((2, 16), device=dev)
    with pytest.raises(ValueError, match="gamma has 8 entries"):
        uocr.rms_norm(x, torch.ones(8, device=dev), 1e-6)
    q = torch.zeros((2, 2, 6), device=dev)
    with pytest.raises(uocr.UocrError, match="the cos/sin tables are 8 wide, not head_dim 6"):
        uocr.rope(q, q, torch.zeros(2, dtype=torch.int32, device=dev), torch.zeros((4, 8), device=dev),
                  torch.zeros((4, 8), device=dev))
    with pytest.raises(ValueError, match="2 \\* ffn columns"):
        uocr.swiglu(torch.zeros((2, 5), device=dev))


# ---------------------------------------------------------------------------- the decode step

LAYERS, HID, HEADS, D, FFN, VOCAB, E = 3, 1280, 10, 128, 256, 64, 8
P = 128


def _bf16_kb(rng, n_out, k_in, std):
    """A K-blocked bf16 projection weight (bits) of N(0, std)."""
    from oracle import oracle as O

    return O.kblocked(O.bf16_bits(rng.standard_normal((n_out, k_in)).astype(np.float32) * np.float32(std)))


def _decoder_weights(oracle, seed=7):
    rng = np.random.default_rng(seed)
    w, moes = {}, {}
    for i in range(LAYERS):
        p = f"layers.{i}."
        for name in "qkvo":
            w[f"{p}self_attn.{name}_proj.weight"] = _bf16_kb(rng, HID, HID, 0.03)
        w[p + "input_layernorm.weight"] = (1 + 0.1 * rng.standard_normal(HID)).astype(np.float32)
        w[p + "post_attention_layernorm.weight"] = (1 + 0.1 * rng.standard_normal(HID)).astype(np.float32)
        if i == 0:
            w[p + "mlp.gate_proj.weight"] = _bf16_kb(rng, FFN, HID, 0.03)
            w[p + "mlp.up_proj.weight"] = _bf16_kb(rng, FFN, HID, 0.03)
            w[p + "mlp.down_proj.weight"] = _bf16_kb(rng, HID, FFN, 0.03)
        else:
            moes[i] = oracle.make_layer(100 + i, E=E, H=HID, F=128, n_shared=2, topk=6, int8=True, std=0.03,
                                        router_std=0.05)
    w["norm.weight"] = (1 + 0.1 * rng.standard_normal(HID)).astype(np.float32)
    w["lm_head.weight"] = _bf16_kb(rng, VOCAB, HID, 0.03)
    return w, moes


def _oracle_step(oracle, w, moes, pool, lut, attend, write, pos, hidden, cos_t, sin_t):
    """The decode step as the oracle's float64 chain; returns (normed, logits, pool after the stores)."""
    x = hidden.astype(np.float64)
    delta = None
    scale = 1.0 / math.sqrt(D)
    B = x.shape[0]
    for i in range(LAYERS):
        p = f"layers.{i}."
        if delta is not None:
            x = x + delta
        normed = _norm64(x, w[p + "input_layernorm.weight"])
        q, k, v = (oracle.dense_f64(normed, w[f"{p}self_attn.{c}_proj.weight"]).reshape(B, HEADS, D) for c in "qkv")
        q = _rope64(q, pos, cos_t, sin_t)
        k = _rope64(k, pos, cos_t, sin_t)
        att, pool = oracle.paged_decode_attention(q.astype(np.float32), k.astype(np.float32), v.astype(np.float32),
                                                  pool, lut, attend - 1, write, i, scale)
        x = x + oracle.dense_f64(att.reshape(B, HID), w[p + "self_attn.o_proj.weight"])
        normed = _norm64(x, w[p + "post_attention_layernorm.weight"])
        if i == 0:
            g = oracle.dense_f64(normed, w[p + "mlp.gate_proj.weight"])
            u = oracle.dense_f64(normed, w[p + "mlp.up_proj.weight"])
            delta = oracle.dense_f64(g / (1 + np.exp(-g)) * u, w[p + "mlp.down_proj.weight"])
        else:
            delta = oracle.moe_layer_f64(normed, moes[i])
    out = _norm64(x + delta, w["norm.weight"])
    return out, oracle.dense_f64(out, w["lm_head.weight"]), pool


def _norm64(x, g):
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 1e-6) * g.astype(np.float64)


def _rope64(x, pos, cos_t, sin_t):
    half = D // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return x * cos_t[pos][:, None, :].astype(np.float64) + rot * sin_t[pos][:, None, :].astype(np.float64)


def test_decoder_decode_step_matches_the_oracle_chain(oracle) -> None:
    import uocr_moe

    w, moes = _decoder_weights(oracle)
    gw = {}
    for k, v in w.items():
        gw[k] = t(v)
    for i, layer in moes.items():
        gw.update({f"layers.{i}.mlp.{k}": v for k, v in layer_weights(layer).items()})
    cfg = uocr_moe.DecoderConfig(hidden_size=HID, num_attention_heads=HEADS, num_hidden_layers=LAYERS,
                                 intermediate_size=FFN, first_k_dense_replace=1, vocab_size=VOCAB,
                                 moe=uocr_moe.MoeConfig(hidden_size=HID, moe_intermediate_size=128,
                                                        n_routed_experts=E, num_experts_per_tok=6,
                                                        n_shared_experts=2, int8_experts=True))
    seq = 1024
    dec = uocr_moe.Decoder(cfg, gw, max_seq_len=seq)
    cos_t, sin_t = oracle.rope_tables(head_dim=D, seq_len=seq, theta=10000.0)
    rng = np.random.default_rng(8)
    pages = 6
    pool = (0.5 * rng.standard_normal((pages, 2, LAYERS, P, HEADS, D))).astype(np.float32)
    lut = np.array([[3, 0, 5], [1, 4, 5]], np.uint32)  # page 5 is the null page
    gpu_pool = t(pool)
    for step, (attend, write) in enumerate([([40, 200], [39, 199]), ([41, 201], [40, 200])]):
        attend, write = np.array(attend, np.uint32), np.array(write, np.uint32)
        pos = write.astype(np.int32)
        hidden = rng.standard_normal((2, HID)).astype(np.float32)
        kv = uocr_moe.PagedKv(kv_blocks=gpu_pool, lookup_table=t(lut.view(np.int32)),
                              attend_lengths=t((attend - 1).view(np.int32)), attend_max=int(attend.max()),
                              write_index=t(write.view(np.int32)))
        apart_pool = gpu_pool.clone()
        apart = dec.decode(t(hidden), positions=t(pos), kv=uocr_moe.PagedKv(
            kv_blocks=apart_pool, lookup_table=kv.lookup_table, attend_lengths=kv.attend_lengths,
            attend_max=kv.attend_max, write_index=kv.write_index), fuse_norm=False)
        normed = dec.decode(t(hidden), positions=t(pos), kv=kv)
        assert np.array_equal(n(normed).view(np.uint32), n(apart).view(np.uint32))  # the fused norms: same bits
        logits = dec.logits_rows(normed)
        want_n, want_l, pool = _oracle_step(oracle, w, moes, pool, lut, attend, write, pos, hidden, cos_t, sin_t)
        assert _rel(n(normed), want_n) <= 1e-4, (step, _rel(n(normed), want_n))
        assert _rel(n(logits), want_l) <= 1e-4, (step, _rel(n(logits), want_l))
        after = n(gpu_pool)
        for b in range(2):
            page, slot = lut[b, write[b] // P], write[b] % P
            for layer in range(LAYERS):
                np.testing.assert_allclose(after[page, :, layer, slot], pool[page, :, layer, slot], rtol=1e-4,
                                           atol=1e-5)
        pool = after  # continue from the GPU's stored rows
