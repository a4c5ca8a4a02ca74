"""Pins of the NumPy restatement of the reference's torch backend _flat
(h3/htrc_flat.py:279-388), the CPU path bench.py times:
  all leaves exact -> dense attention; one query per tile with no exact leaves -> dense
  attention (the far field is exact at the centre, both for lin and iso curvature);
  tile_chunk does not change the result; ragged tiles and key tails.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import flat_fp32


def _data(n, m, d=64, seed=0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((n, d)).astype(np.float32), (rng.standard_normal((m, d)) * 1.2).astype(np.float32),
            rng.standard_normal((m, d)).astype(np.float32))


@pytest.mark.parametrize("select", ["max", "bound"])
def test_all_leaves_exact_is_dense(select):
    q, k, v = _data(300, 512)
    out, lz = flat_fp32.flat_fp32(q, k, v, tile=64, exact_leaves=512 // 16, leaf=16, select=select,
                                  return_logz=True)
    ref, rlz = flat_fp32.dense(q, k, v)
    assert np.linalg.norm(out - ref) / np.linalg.norm(ref) < 1e-5
    assert np.abs(lz - rlz).max() < 1e-4


@pytest.mark.parametrize("curvature", ["lin", "iso"])
def test_one_query_per_tile_far_field_is_exact(curvature):
    q, k, v = _data(40, 256, seed=1)
    out = flat_fp32.flat_fp32(q, k, v, tile=1, exact_leaves=0, leaf=32, curvature=curvature, tile_chunk=7)
    ref, _ = flat_fp32.dense(q, k, v)
    assert np.linalg.norm(out - ref) / np.linalg.norm(ref) < 1e-5


def test_tile_chunk_invariance_and_tail():
    q, k, v = _data(333, 520, seed=2)                  # 520 = 32 leaves of 16 + 8 tail keys
    a = flat_fp32.flat_fp32(q, k, v, tile=64, exact_leaves=5, leaf=16, tile_chunk=1)
    b = flat_fp32.flat_fp32(q, k, v, tile=64, exact_leaves=5, leaf=16, tile_chunk=32)
    assert np.linalg.norm(a - b) / np.linalg.norm(b) < 1e-6          # BLAS blocking only
    full = flat_fp32.flat_fp32(q, k, v, tile=64, exact_leaves=32, leaf=16)
    ref, _ = flat_fp32.dense(q, k, v)
    assert np.linalg.norm(full - ref) / np.linalg.norm(ref) < 1e-5   # tail keys are always exact


def test_tiles_slice_matches_full_run():
    q, k, v = _data(256, 256, seed=3)
    full = flat_fp32.flat_fp32(q, k, v, tile=64, exact_leaves=3, leaf=16)
    part = flat_fp32.flat_fp32(q, k, v, tile=64, exact_leaves=3, leaf=16, tiles=slice(1, 3))
    assert np.allclose(part[64:192], full[64:192], rtol=1e-5, atol=1e-6) and np.all(part[:64] == 0)


def test_validation():
    q, k, v = _data(8, 32)
    with pytest.raises(ValueError):
        flat_fp32.flat_fp32(q, k, v, select="nope")
    with pytest.raises(ValueError):
        flat_fp32.flat_fp32(q, k, v, curvature="quad")
    with pytest.raises(ValueError):
        flat_fp32.flat_fp32(q, k[:8], v[:8], leaf=16)
