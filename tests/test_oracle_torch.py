"""Pins of the torch-CPU restatement of the reference's torch backend _flat (h3/htrc_flat.py:279-388),
the CPU operator bench.py times as ``cpu_baseline``:
  equal to the NumPy restatement flat_fp32 within fp32 rounding (out and logZ, lin / iso curvature,
  max / bound select, ragged tiles, tail keys, tile windows); all leaves exact -> dense attention;
  one query per tile with no exact leaves -> dense attention.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import flat_fp32, flat_torch


def _data(n, m, d=64, seed=0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((n, d)).astype(np.float32), (rng.standard_normal((m, d)) * 1.2).astype(np.float32),
            rng.standard_normal((m, d)).astype(np.float32))


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("curvature,select", [("lin", "max"), ("iso", "max"), ("lin", "bound")])
def test_equals_numpy_restatement(curvature, select):
    q, k, v = _data(333, 520, seed=4)                 # ragged last tile, 32 leaves of 16 + 8 tail keys
    kw = dict(tile=64, exact_leaves=5, leaf=16, curvature=curvature, select=select, tile_chunk=3, return_logz=True)
    o1, z1 = flat_torch.flat_torch(q, k, v, **kw)
    o2, z2 = flat_fp32.flat_fp32(q, k, v, **kw)
    assert isinstance(o1, torch.Tensor) and o1.dtype == torch.float32 and tuple(o1.shape) == (333, 64)
    assert _rel(o1.numpy(), o2) < 1e-5
    assert np.abs(z1.numpy() - z2).max() < 1e-4


def test_all_leaves_exact_is_dense():
    q, k, v = _data(300, 512, seed=5)
    out, lz = flat_torch.flat_torch(q, k, v, tile=64, exact_leaves=32, leaf=16, return_logz=True)
    ref, rlz = flat_fp32.dense(q, k, v)
    assert _rel(out.numpy(), ref) < 1e-5 and np.abs(lz.numpy() - rlz).max() < 1e-4


@pytest.mark.parametrize("curvature", ["lin", "iso"])
def test_one_query_per_tile_far_field_is_exact(curvature):
    q, k, v = _data(40, 256, seed=6)
    out = flat_torch.flat_torch(q, k, v, tile=1, exact_leaves=0, leaf=32, curvature=curvature, tile_chunk=7)
    ref, _ = flat_fp32.dense(q, k, v)
    assert _rel(out.numpy(), ref) < 1e-5


def test_windows_and_tile_slices():
    q, k, v = _data(256, 256, seed=7)
    full = flat_torch.flat_torch(q, k, v, tile=64, exact_leaves=3, leaf=16, tile_chunk=4)
    one = flat_torch.flat_torch(q, k, v, tile=64, exact_leaves=3, leaf=16, tile_chunk=1)
    assert _rel(one.numpy(), full.numpy()) < 1e-6
    part = flat_torch.flat_torch(q, k, v, tile=64, exact_leaves=3, leaf=16, tiles=slice(1, 3))
    assert torch.allclose(part[64:192], full[64:192], rtol=1e-5, atol=1e-6) and not part[:64].any()


def test_validation():
    q, k, v = _data(8, 32)
    with pytest.raises(ValueError):
        flat_torch.flat_torch(q, k, v, select="nope")
    with pytest.raises(ValueError):
        flat_torch.flat_torch(q, k, v, curvature="quad")
    with pytest.raises(ValueError):
        flat_torch.flat_torch(q, k[:8], v[:8], leaf=16)
