"""Pins of the oracle's leaf statistics (h3/htrc_flat_triton.py:55-85) against the float64
teaching reference's exact leaf identities (src/htrc_reference/model.py:35-49): with the
scaled centre c = scale * mu,
    lz = log_mass(c),  g = scale * gradient(c),  vb = value(c),
and closed forms for degenerate leaves.  A dropped scale, a transposed operand or a sign
error in the softmax fails these.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import bf16, flat_i8, htrc_ref

D = 128


def _data(nt, nk, seed):
    rng = np.random.default_rng(seed)
    mu = (rng.standard_normal((nt, D)) * 1.5).astype(np.float32)
    k = bf16.from_f32((rng.standard_normal((nk, D)) * 1.5).astype(np.float32))
    v = bf16.from_f32(rng.standard_normal((nk, D)).astype(np.float32))
    return mu, k, v


@pytest.mark.parametrize("leaf", [16, 64, 128])
def test_stats_equal_exact_leaf_identities(leaf):
    nt, nk = 3, 4 * leaf
    scale = 1.0 / math.sqrt(D)
    mu, k, v = _data(nt, nk, leaf)
    g8, sg, vb, lz = flat_i8.stats(mu, k, v, leaf, scale)
    kf, vf = bf16.to_f32(k).astype(np.float64), bf16.to_f32(v).astype(np.float64)
    for t in range(nt):
        for l in range(nk // leaf):
            sl = slice(l * leaf, (l + 1) * leaf)
            ex = htrc_ref.leaf_stats(kf[sl], vf[sl], scale * mu[t].astype(np.float64))
            assert abs(lz[t, l] - ex.log_mass) <= 2e-5 * (1 + abs(ex.log_mass))
            g = scale * ex.gradient
            am = np.abs(g).max()
            # int8 g: dequantised within half a step (+ fp32 slack) of the exact gradient
            np.testing.assert_allclose(sg[t, l], am / 127, rtol=1e-5)
            assert np.abs(g8[t, l] * np.float64(sg[t, l]) - g).max() <= 0.5 * sg[t, l] * (1 + 1e-3)
            assert np.abs(g8[t, l]).max() == 127
            # vb: bf16 rounding of the exact value mean
            np.testing.assert_allclose(bf16.to_f32(vb[t, l]), ex.value, rtol=2 ** -8, atol=1e-6)


def test_identical_keys_give_uniform_weights():
    leaf, scale = 64, 1.0 / math.sqrt(D)
    rng = np.random.default_rng(1)
    key = bf16.from_f32((rng.standard_normal(D)).astype(np.float32))
    k = np.tile(key, (leaf, 1))
    v = bf16.from_f32(rng.standard_normal((leaf, D)).astype(np.float32))
    mu = rng.standard_normal((1, D)).astype(np.float32)
    g8, sg, vb, lz = flat_i8.stats(mu, k, v, leaf, scale)
    a = float(mu[0].astype(np.float64) @ bf16.to_f32(key).astype(np.float64) * scale)
    assert abs(lz[0, 0] - (a + math.log(leaf))) < 1e-4
    g = scale * bf16.to_f32(key).astype(np.float64)
    assert np.abs(g8[0, 0] * np.float64(sg[0, 0]) - g).max() <= 0.5 * sg[0, 0] * 1.001
    np.testing.assert_allclose(bf16.to_f32(vb[0, 0]), bf16.to_f32(v).astype(np.float64).mean(0), rtol=2 ** -8,
                               atol=1e-6)


def test_single_token_leaf():
    scale = 0.25
    rng = np.random.default_rng(2)
    k = bf16.from_f32(rng.standard_normal((5, D)).astype(np.float32))
    v = bf16.from_f32(rng.standard_normal((5, D)).astype(np.float32))
    mu = rng.standard_normal((2, D)).astype(np.float32)
    g8, sg, vb, lz = flat_i8.stats(mu, k, v, 1, scale)
    kf = bf16.to_f32(k).astype(np.float64)
    np.testing.assert_allclose(lz, (mu.astype(np.float64) @ kf.T) * scale, rtol=1e-6, atol=1e-6)
    assert np.array_equal(vb, np.broadcast_to(v, vb.shape))      # w = 1 exactly: vb is v
    np.testing.assert_allclose(g8 * sg[..., None].astype(np.float64), np.broadcast_to(scale * kf, g8.shape),
                               atol=float(sg.max()) * 0.51)


def test_zero_gradient_floor():
    """g = 0 (all-zero keys): am floors at 1e-30, g8 = 0, lz = log(leaf)."""
    leaf = 16
    k = np.zeros((leaf, D), np.uint16)
    v = bf16.from_f32(np.ones((leaf, D), np.float32))
    mu = np.ones((1, D), np.float32)
    g8, sg, vb, lz = flat_i8.stats(mu, k, v, leaf, 0.1)
    assert np.all(g8 == 0)
    assert sg[0, 0] == np.float32(np.float32(1e-30) * np.float32(flat_i8.r127()))
    assert abs(lz[0, 0] - math.log(leaf)) < 1e-6
    assert np.all(bf16.to_f32(vb) == 1.0)
