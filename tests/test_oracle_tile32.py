"""Pins of the oracle at 32-row tiles (tile=32, the runner's mode "max",
h3/htrc_flat_runner.py:52; _tiles h3/htrc_flat.py:142-156 with tile = 32):

* tile centres: exact on integer-valued rows, the last partial tile over its real rows only;
* every 64-row tile made of two equal 32-row halves (values on a 1/16 grid): the 32-row
  centres equal the 64-row centres exactly, so the state is each 64-row tile's state twice,
  the routing is each 64-row tile's twice and out / logZ equal the 64-row path bit for bit;
* all leaves exact: the output does not depend on the tile size (the same near tokens in
  the same order for every row).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import bf16, flat_i8

D = 128


def _kv(nk, seed):
    rng = np.random.default_rng(seed)
    c = rng.standard_normal((nk // 64, D)) * 1.5
    k = bf16.from_f32((np.repeat(c, 64, 0) + 0.5 * rng.standard_normal((nk, D))).astype(np.float32))
    v = bf16.from_f32(rng.standard_normal((nk, D)).astype(np.float32))
    return k, v


@pytest.mark.parametrize("n", [32 * 7, 32 * 7 + 5, 1, 33])
def test_tile32_centres_exact_on_integer_rows(n):
    rng = np.random.default_rng(n)
    q = rng.integers(-60, 61, size=(n, D)).astype(np.float32)
    mu = flat_i8.tile_centres(q, 32)
    assert mu.shape == (-(-n // 32), D)
    for t in range(mu.shape[0]):
        rows = q[32 * t: min(n, 32 * t + 32)].astype(np.float64)
        assert np.array_equal(mu[t], (rows.sum(0) / rows.shape[0]).astype(np.float32))


@pytest.mark.parametrize("leaf,ex,stride", [(64, 4, 1), (16, 24, 1), (32, 8, 2)])
def test_equal_halves_make_tile32_the_tile64_path(leaf, ex, stride):
    rng = np.random.default_rng(leaf + ex)
    nt64 = 9
    halves = np.round(rng.standard_normal((nt64, 32, D)) * 16) / 16
    q = np.concatenate([halves, halves], axis=1).reshape(-1, D).astype(np.float32)
    k, v = _kv(64 * 24, leaf)
    a = flat_i8.flat_i8(q, k, v, tile=32, leaf=leaf, exact_leaves=ex, splits=2, bn=64, sel_stride=stride)
    b = flat_i8.flat_i8(q, k, v, tile=64, leaf=leaf, exact_leaves=ex, splits=2, bn=64, sel_stride=stride)
    assert np.array_equal(a["mu"], np.repeat(b["mu"], 2, 0))
    assert np.array_equal(a["g8"], np.repeat(b["g8"], 2, 0)) and np.array_equal(a["lz"], np.repeat(b["lz"], 2, 0))
    assert np.array_equal(a["idx"], np.repeat(b["idx"], 2, 0))
    assert np.array_equal(a["out"], b["out"]) and np.array_equal(a["logz"], b["logz"])


def test_all_leaves_exact_output_does_not_depend_on_tile():
    rng = np.random.default_rng(3)
    n = 32 * 11 + 9
    q = bf16.from_f32(rng.standard_normal((n, D)).astype(np.float32))
    k, v = _kv(64 * 8, 4)
    a = flat_i8.flat_i8(q, k, v, tile=32, leaf=64, exact_leaves=8, splits=1, bn=64)
    b = flat_i8.flat_i8(q, k, v, tile=64, leaf=64, exact_leaves=8, splits=1, bn=64)
    assert np.array_equal(a["out"], b["out"]) and np.array_equal(a["logz"], b["logz"])
