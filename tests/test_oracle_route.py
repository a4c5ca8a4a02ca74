"""Pins of the oracle's routing and attention stages:

* select (h3/htrc_flat_triton.py:214-254): brute force with NumPy int64 matmuls; the
  centred-rows invariant (dq = 0 gives SEL = lz).
* top-k (h3/htrc_flat.py:262-265): brute force by a stable argsort; sink forcing.
* tile + merge (h3/htrc_flat_triton.py:88-273):
  (i)  all leaves exact  -> dense softmax attention over the int8 scores, bf16 V;
  (ii) constant tiles (q = mu) with no exact leaves -> dense attention at the centre
       (the far field is exact at the expansion point: flat analogue of
       tests/test_reference.py:30-35);
  (iii) splits / block sizes agree to fp32 rounding; (iv) all far leaves excluded.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import bf16, flat_i8, flat_fp32

D = 128


def _clustered(n, seed, runs=None):
    rng = np.random.default_rng(seed)
    runs = runs or max(1, n // 64)
    c = rng.standard_normal((runs, D)) * 1.5
    rid = np.minimum(np.arange(n) // 64, runs - 1)
    q = bf16.from_f32((c[rid] + 0.5 * rng.standard_normal((n, D))).astype(np.float32))
    k = bf16.from_f32((c[rid] + 0.5 * rng.standard_normal((n, D))).astype(np.float32))
    v = bf16.from_f32(rng.standard_normal((n, D)).astype(np.float32))
    return q, k, v


def test_select_brute_force_and_centred_invariant():
    q, k, v = _clustered(1024, 0)
    st = flat_i8.flat_i8(q, k, v, tile=64, leaf=64, exact_leaves=4)
    nt, nb, _ = st["g8"].shape
    for stride in (1, 2, 8):
        sel = flat_i8.select(st["dq8"], st["sdq"], 64, st["g8"], st["sg"], st["lz"], stride)
        dots = np.einsum("trd,tld->trl", st["dq8"].reshape(nt, 64, D)[:, ::stride].astype(np.int64),
                         st["g8"].astype(np.int64))
        sc = dots.astype(np.float32) * (st["sdq"].reshape(nt, 64)[:, ::stride, None] * st["sg"][:, None, :])
        bf = sc.max(1) + st["lz"]
        assert np.array_equal(sel.view(np.uint32), bf.astype(np.float32).view(np.uint32))
    # q rows all equal to the centre: dq8 = 0 -> SEL = lz exactly
    zero = np.zeros_like(st["dq8"])
    sel0 = flat_i8.select(zero, st["sdq"], 64, st["g8"], st["sg"], st["lz"], 1)
    assert np.array_equal(sel0, st["lz"])


@pytest.mark.parametrize("kx,sink", [(5, 0), (16, 3), (64, 0), (1, 1)])
def test_topk_brute_force(kx, sink):
    rng = np.random.default_rng(kx)
    sel = rng.standard_normal((40, 64)).astype(np.float32)
    sel[:, ::5] = 0.5                                           # ties across the boundary
    idx, excl = flat_i8.topk(sel, kx, sink)
    for t in range(sel.shape[0]):
        x = sel[t].copy()
        x[:sink] = np.inf
        order = np.argsort(-x.astype(np.float64), kind="stable")[:kx]
        assert np.array_equal(idx[t], np.sort(order))
        assert excl[t].sum() == kx and np.all(excl[t, idx[t]] == 1)
        assert np.all(idx[t, :min(sink, kx)] == np.arange(min(sink, kx)))


def _dense_int8(st, n, scale):
    """Dense attention over the int8 scores float(q8.k8) * (sq * ks * scale) with bf16 V (float64)."""
    s = (st["q8"][:n].astype(np.int64) @ st["k8"].astype(np.int64).T).astype(np.float64)
    s *= st["sq"][:n, None].astype(np.float64) * st["ks"][None, :].astype(np.float64) * scale
    m = s.max(1, keepdims=True)
    e = np.exp(s - m)
    z = e.sum(1, keepdims=True)
    return e @ bf16.to_f32(st["v"]).astype(np.float64) / z, (np.log(z) + m)[:, 0]


@pytest.mark.parametrize("leaf,splits", [(64, 4), (32, 3), (16, 1)])
def test_all_leaves_exact_is_dense_int8_attention(leaf, splits):
    n = 1000
    q, k, v = _clustered(1024, leaf)
    q = q[:n]
    nb = 1024 // leaf
    scale = 1 / math.sqrt(D)
    st = flat_i8.flat_i8(q, k, v, tile=64, leaf=leaf, exact_leaves=nb, splits=splits, bn=64)
    assert st["excl"].all()
    ref, lz = _dense_int8(st, n, scale)
    rel = np.linalg.norm(st["out"] - ref) / np.linalg.norm(ref)
    assert rel < 4e-3                                           # bf16 rounding of p only
    assert np.abs(st["logz"] - lz).max() < 2e-5 * (1 + np.abs(lz).max())
    # and int8 Q/K stays within a few percent of exact fp32 attention
    dense, dlz = flat_fp32.dense(bf16.to_f32(q), bf16.to_f32(k), bf16.to_f32(v))
    assert np.linalg.norm(st["out"] - dense) / np.linalg.norm(dense) < 0.05


def test_centre_collapse_far_field_is_exact():
    """Every tile's rows equal its centre: dq = 0, far logit = lz, far value = vb; with no
    exact leaves the output is softmax attention at the centre (up to bf16 of vb and p)."""
    rng = np.random.default_rng(5)
    nt, nk, leaf = 4, 1024, 64
    cen = bf16.round_f32((rng.standard_normal((nt, D)) * 0.7).astype(np.float32))
    q = np.repeat(cen, 64, 0)
    k = bf16.from_f32((rng.standard_normal((nk, D)) * 1.5).astype(np.float32))
    v = bf16.from_f32(rng.standard_normal((nk, D)).astype(np.float32))
    st = flat_i8.flat_i8(q, k, v, tile=64, leaf=leaf, exact_leaves=0, splits=2, bn=64)
    assert np.all(st["dq8"] == 0)
    dense, dlz = flat_fp32.dense(cen, bf16.to_f32(k), bf16.to_f32(v))
    out = st["out"].reshape(nt, 64, D)
    for t in range(nt):
        ref = np.broadcast_to(dense[t], out[t].shape)
        assert np.linalg.norm(out[t] - ref) / np.linalg.norm(ref) < 5e-3
        assert np.abs(st["logz"].reshape(nt, 64)[t] - dlz[t]).max() < 1e-4 * (1 + abs(dlz[t]))


def test_splits_and_blocks_agree():
    q, k, v = _clustered(2048, 3)
    outs = []
    for splits, bn in ((1, 64), (2, 64), (4, 32), (8, 128), (3, 64)):
        st = flat_i8.flat_i8(q, k, v, tile=64, leaf=64, exact_leaves=6, splits=splits, bn=bn)
        outs.append((st["out"], st["logz"], st["idx"]))
    for o, l, i in outs[1:]:
        assert np.array_equal(i, outs[0][2])
        assert np.linalg.norm(o - outs[0][0]) / np.linalg.norm(outs[0][0]) < 5e-3
        assert np.abs(l - outs[0][1]).max() < 1e-5 * (1 + np.abs(l).max())


def test_merge_single_split_is_normalisation():
    rng = np.random.default_rng(9)
    pm = rng.standard_normal((2, 1, 64)).astype(np.float32)
    pl = (rng.random((2, 1, 64)) + 0.5).astype(np.float32)
    pacc = rng.standard_normal((2, 1, 64, D)).astype(np.float32)
    out, logz = flat_i8.merge(pm, pl, pacc)
    np.testing.assert_array_equal(out, (pacc[:, 0] / pl[:, 0, :, None]).reshape(128, D))
    np.testing.assert_allclose(logz, (pm[:, 0] + np.log(pl[:, 0])).reshape(-1), rtol=1e-6, atol=1e-6)


def test_merge_empty_split():
    pm = np.full((1, 2, 64), -np.inf, np.float32)
    pm[0, 1] = 1.0
    pl = np.zeros((1, 2, 64), np.float32)
    pl[0, 1] = 2.0
    pacc = np.zeros((1, 2, 64, D), np.float32)
    pacc[0, 1] = 4.0
    out, logz = flat_i8.merge(pm, pl, pacc)
    assert np.all(out == 2.0)
    np.testing.assert_allclose(logz, 1.0 + math.log(2.0), rtol=1e-6)


def test_split_lengths():
    assert flat_i8.split(1008, 4, 64) == 256
    assert flat_i8.split(2048, 4, 64) == 512
    assert flat_i8.split(10, 4, 64) == 64
    assert flat_i8.split(0, 4, 32) == 32
