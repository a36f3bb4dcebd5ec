"""Pins of oracle/engine.py (its PINNED_BY list), on the CPU."""

import math

import numpy as np

import oracle.engine as OE
from oracle.moe import silu


def test_rms_norm_constant_row_and_scale_invariance():
    w = np.linspace(0.5, 1.5, 128)
    for c in (-3.0, 1e-3, 7.5):
        got = OE.rms_norm_f16(np.full((1, 128), c), w, 1e-6)
        want = (np.sign(c) * w / math.sqrt(1.0 + 1e-6 / (c * c))).astype(np.float16)
        np.testing.assert_array_equal(got[0], want)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((3, 256))
    a = OE.rms_norm_f16(x, w[:1].repeat(256), 0.0)
    b = OE.rms_norm_f16(x * 1024.0, w[:1].repeat(256), 0.0)
    np.testing.assert_array_equal(a, b)


def test_rms_norm_textbook():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4, 512))
    w = rng.uniform(0.5, 1.5, 512)
    rms = np.linalg.norm(x, axis=1, keepdims=True) / math.sqrt(512)
    want = (x / np.sqrt(rms ** 2 + 1e-5) * w).astype(np.float16)
    np.testing.assert_array_equal(OE.rms_norm_f16(x, w, 1e-5), want)


def test_mlp_dense_structure():
    """A zero down product leaves h; the down product enters linearly; with identity gate/up
    maps the SwiGLU of the normed rows comes out."""
    rng = np.random.default_rng(2)
    H = I = 64
    h = rng.standard_normal((3, H))
    w = np.ones(H)
    G = rng.standard_normal((2 * I, H)) * 0.1
    D = rng.standard_normal((H, I)) * 0.1
    gu = lambda xn: xn.astype(np.float64) @ G.T                       # noqa: E731
    np.testing.assert_array_equal(OE.mlp_dense_f64(h, w, 1e-6, gu, lambda a: np.zeros((a.shape[0], H)), I), h)
    one = OE.mlp_dense_f64(h, w, 1e-6, gu, lambda a: a.astype(np.float64) @ D.T, I) - h
    two = OE.mlp_dense_f64(h, w, 1e-6, gu, lambda a: a.astype(np.float64) @ (2 * D).T, I) - h
    np.testing.assert_allclose(two, 2 * one, rtol=1e-9, atol=1e-12)
    ident = lambda xn: np.concatenate([xn, xn], axis=1).astype(np.float64)    # noqa: E731
    got = OE.mlp_dense_f64(h, w, 1e-6, ident, lambda a: a.astype(np.float64), I) - h
    xn = OE.rms_norm_f16(h, w, 1e-6).astype(np.float64)
    np.testing.assert_allclose(got, (silu(xn) * xn).astype(np.float16).astype(np.float64), rtol=1e-9, atol=1e-12)


def test_top_k_brute_force():
    rng = np.random.default_rng(3)
    x = rng.integers(-5, 5, 300).astype(np.float32)
    x[rng.random(300) < 0.1] = np.nan
    order = sorted((i for i in range(300) if not np.isnan(x[i])), key=lambda i: (-float(x[i]), i))
    for k in (1, 10, 300, 400):
        ids, vals = OE.top_k(x, k)
        assert list(ids) == order[:k]
        np.testing.assert_array_equal(vals, x[order[:k]])
    assert len(OE.top_k(np.full(4, np.nan, np.float32), 2)[0]) == 0
