"""The decoder-step oracle pieces (oracle.rms_norm, rope, rope_tables, swiglu), pinned without the
reference (MAX is absent here) by what does not share their formulation:

* ``rms_norm``: torch's ``rms_norm`` in float64; a constant row normalises to ``sign * gamma`` (up to
  eps); the residual add is the fp32 sum;
* ``rope``: the rotation of each pair ``(x[d], x[d + D/2])`` by the angle ``position * inv_freq[d]`` as a
  complex product, in float64; position 0 is the identity, bit for bit; rotations keep pair norms;
* ``rope_tables``: ``cos`` / ``sin`` of ``position / theta^(2i/D)`` in float64 (within the fp32 rounding
  of the angle), and the package's own table builder gives the same bits;
* ``swiglu``: ``g / (1 + exp(-g)) * u`` in float64 within a few fp32 ulp; silu(0) = 0.
"""

from __future__ import annotations

import numpy as np
import torch


def test_rms_norm_against_torch_and_closed_forms(oracle) -> None:
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 1280)).astype(np.float32)
    d = rng.standard_normal((5, 1280)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(1280)).astype(np.float32)
    out, v = oracle.rms_norm(x, g, 1e-6, residual=d)
    assert np.array_equal(v, (x + d).astype(np.float32))
    want = torch.nn.functional.rms_norm(torch.from_numpy(v.astype(np.float64)), (1280,),
                                        torch.from_numpy(g.astype(np.float64)), eps=1e-6).numpy()
    np.testing.assert_allclose(out, want, rtol=1e-12, atol=0)
    const = np.full((2, 1280), 3.0, np.float32)
    const[1] = -0.5
    out, _ = oracle.rms_norm(const, g, 0.0)
    np.testing.assert_allclose(out, np.sign(const) * g, rtol=1e-12)


def test_rope_is_a_complex_rotation(oracle) -> None:
    rng = np.random.default_rng(2)
    D, seq = 128, 700
    cos_t, sin_t = oracle.rope_tables(head_dim=D, seq_len=seq, theta=10000.0)
    x = rng.standard_normal((4, 10, D)).astype(np.float32)
    pos = np.array([0, 1, 255, 699])
    got = oracle.rope(x, pos, cos_t, sin_t)
    assert np.array_equal(got[0], x[0])  # position 0: cos 1, sin 0
    half = D // 2
    z = x[..., :half].astype(np.float64) + 1j * x[..., half:].astype(np.float64)
    ang = cos_t[pos][:, None, :half].astype(np.float64) + 1j * sin_t[pos][:, None, :half].astype(np.float64)
    rot = z * ang
    want = np.concatenate([rot.real, rot.imag], axis=-1)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)
    np.testing.assert_allclose(np.abs(got[..., :half] + 1j * got[..., half:]), np.abs(z), rtol=2e-6)


def test_rope_tables_closed_form_and_the_package_builder(oracle) -> None:
    from uocr_moe.decoder import rope_tables

    D, seq, theta = 128, 1024, 10000.0
    cos_t, sin_t = oracle.rope_tables(head_dim=D, seq_len=seq, theta=theta)
    inv = 1.0 / theta ** (np.arange(0, D, 2) / D)
    ang = np.arange(seq)[:, None] * inv[None, :]
    # the angle is rounded to fp32 (|error| <= 2^-24 * |angle| plus the inv_freq rounding)
    tol = 4 * np.finfo(np.float32).eps * (np.abs(ang) + 1.0)
    assert np.all(np.abs(cos_t[:, :D // 2] - np.cos(ang)) <= tol)
    assert np.all(np.abs(sin_t[:, :D // 2] - np.sin(ang)) <= tol)
    assert np.array_equal(cos_t[:, :D // 2], cos_t[:, D // 2:]) and np.all(cos_t[0] == 1) and np.all(sin_t[0] == 0)
    pc, ps = rope_tables(head_dim=D, seq_len=seq, theta=theta)
    assert np.array_equal(pc, cos_t) and np.array_equal(ps, sin_t)


def test_swiglu(oracle) -> None:
    rng = np.random.default_rng(3)
    gu = (4 * rng.standard_normal((3, 2 * 300))).astype(np.float32)
    gu[0, 0] = 0.0
    got = oracle.swiglu(gu)
    g, u = gu[:, :300].astype(np.float64), gu[:, 300:].astype(np.float64)
    want = g / (1 + np.exp(-g)) * u
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-30)
    assert got[0, 0] == 0.0
