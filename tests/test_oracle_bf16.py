"""Pins of the oracle's bf16 state store (store="bf16", h3/htrc_flat_triton.py:65-72, 132-153,
165-184, 214-254 with the 16-bit state and FP8 = 0):

* the stored state equals the float64 teaching reference's exact leaf identities
  (src/htrc_reference/model.py:35-49) within half a bf16 step, and lz within fp32 rounding;
* select: brute force in float64 (every bf16 x bf16 product is exact in fp32); centred rows
  give lz;
* tile: all leaves exact -> dense attention over bf16 q.k scores; rows at their centre with
  no exact leaves -> dense attention at the centre within the bf16 rounding of vb, closer
  than the fp8 store gets.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import bf16, flat_fp32, flat_i8, htrc_ref

D = 128


@pytest.mark.parametrize("leaf", [16, 64])
def test_bf16_state_rounds_the_exact_leaf_identities(leaf):
    rng = np.random.default_rng(leaf + 1)
    nt, nk, scale = 3, 4 * leaf, 1 / math.sqrt(D)
    mu = (rng.standard_normal((nt, D)) * 1.5).astype(np.float32)
    k = bf16.from_f32((rng.standard_normal((nk, D)) * 1.5).astype(np.float32))
    v = bf16.from_f32(rng.standard_normal((nk, D)).astype(np.float32))
    g16, vb16, lz = flat_i8.stats_bf16(mu, k, v, leaf, scale)
    kf, vf = bf16.to_f32(k).astype(np.float64), bf16.to_f32(v).astype(np.float64)
    for t in range(nt):
        for l in range(nk // leaf):
            sl = slice(l * leaf, (l + 1) * leaf)
            ex = htrc_ref.leaf_stats(kf[sl], vf[sl], scale * mu[t].astype(np.float64))
            assert abs(lz[t, l] - ex.log_mass) <= 2e-5 * (1 + abs(ex.log_mass))
            g = scale * ex.gradient
            gd = bf16.to_f32(g16[t, l]).astype(np.float64)
            vd = bf16.to_f32(vb16[t, l]).astype(np.float64)
            # half a bf16 step (2^-8 relative) plus the fp32 error of the accumulated moments
            assert np.all(np.abs(gd - g) <= np.abs(g) * 2 ** -8 * 1.01 + 1e-6 * np.abs(g).max())
            assert np.all(np.abs(vd - ex.value) <= np.abs(ex.value) * 2 ** -8 * 1.01 + 1e-6 * np.abs(ex.value).max())


def _clustered(n, seed):
    rng = np.random.default_rng(seed)
    runs = max(1, n // 64)
    c = rng.standard_normal((runs, D)) * 1.5
    rid = np.minimum(np.arange(n) // 64, runs - 1)
    q = bf16.from_f32((c[rid] + 0.5 * rng.standard_normal((n, D))).astype(np.float32))
    k = bf16.from_f32((c[rid] + 0.5 * rng.standard_normal((n, D))).astype(np.float32))
    v = bf16.from_f32(rng.standard_normal((n, D)).astype(np.float32))
    return q, k, v


def test_bf16_operands_are_bf16_roundings():
    q, k, v = _clustered(320, 2)
    q = q[:300]
    st = flat_i8.flat_i8(q, k, v, tile=64, leaf=64, exact_leaves=2, store="bf16")
    qf = bf16.to_f32(q)
    rows = qf[np.minimum(np.arange(st["q16"].shape[0]), 299)]
    assert np.array_equal(st["q16"], bf16.from_f32(rows))
    dq = rows - st["mu"][np.arange(rows.shape[0]) // 64]
    assert np.array_equal(st["dq16"], bf16.from_f32(dq.astype(np.float32)))


def test_select_bf16_brute_force_and_centred_rows():
    q, k, v = _clustered(1024, 3)
    st = flat_i8.flat_i8(q, k, v, tile=64, leaf=64, exact_leaves=4, store="bf16")
    nt, nb, _ = st["g16"].shape
    dq = bf16.to_f32(st["dq16"]).astype(np.float64).reshape(nt, 64, D)
    g = bf16.to_f32(st["g16"]).astype(np.float64)
    for stride in (1, 4):
        sel = flat_i8.select_bf16(st["dq16"], 64, st["g16"], st["lz"], stride)
        want = np.einsum("trd,tld->trl", dq[:, ::stride], g).max(1) + st["lz"]
        np.testing.assert_allclose(sel, want, rtol=1e-5, atol=1e-5)
    zero = np.zeros_like(st["dq16"])
    assert np.array_equal(flat_i8.select_bf16(zero, 64, st["g16"], st["lz"], 1), st["lz"])


@pytest.mark.parametrize("leaf,splits", [(64, 4), (32, 1)])
def test_bf16_all_leaves_exact_is_dense_bf16_attention(leaf, splits):
    n = 1000
    q, k, v = _clustered(1024, leaf)
    q = q[:n]
    nb = 1024 // leaf
    scale = 1 / math.sqrt(D)
    st = flat_i8.flat_i8(q, k, v, tile=64, leaf=leaf, exact_leaves=nb, splits=splits, bn=64, store="bf16")
    assert st["excl"].all()
    qf, kf, vf = (bf16.to_f32(x).astype(np.float64) for x in (q, k, v))
    s = qf @ kf.T * scale
    m = s.max(1, keepdims=True)
    e = np.exp(s - m)
    ref = e @ vf / e.sum(1, keepdims=True)
    assert np.linalg.norm(st["out"] - ref) / np.linalg.norm(ref) < 4e-3          # bf16 rounding of p only
    assert np.abs(st["logz"] - (np.log(e.sum(1)) + m[:, 0])).max() < 2e-5 * (1 + np.abs(m).max())


def test_bf16_centre_collapse_far_field_beats_fp8():
    """Rows at their tile's centre with no exact leaves: softmax attention at the centre up to
    the bf16 rounding of vb and p, and nearer to it than the fp8 store."""
    rng = np.random.default_rng(5)
    nt, nk, leaf = 4, 1024, 64
    cen = bf16.round_f32((rng.standard_normal((nt, D)) * 0.7).astype(np.float32))
    q = np.repeat(cen, 64, 0)
    k = bf16.from_f32((rng.standard_normal((nk, D)) * 1.5).astype(np.float32))
    v = bf16.from_f32(rng.standard_normal((nk, D)).astype(np.float32))
    st = flat_i8.flat_i8(q, k, v, tile=64, leaf=leaf, exact_leaves=0, splits=2, bn=64, store="bf16")
    f8 = flat_i8.flat_i8(q, k, v, tile=64, leaf=leaf, exact_leaves=0, splits=2, bn=64, store="fp8")
    assert np.all(st["dq16"] == 0)
    dense, dlz = flat_fp32.dense(cen, bf16.to_f32(k), bf16.to_f32(v))
    out, o8 = st["out"].reshape(nt, 64, D), f8["out"].reshape(nt, 64, D)
    for t in range(nt):
        ref = np.broadcast_to(dense[t], out[t].shape)
        e16 = np.linalg.norm(out[t] - ref) / np.linalg.norm(ref)
        assert e16 < 1e-2
        assert e16 < np.linalg.norm(o8[t] - ref) / np.linalg.norm(ref)
        assert np.abs(st["logz"].reshape(nt, 64)[t] - dlz[t]).max() < 1e-4 * (1 + abs(dlz[t]))


def test_bf16_group_path_runs_and_matches_group_one_on_exact_leaves():
    q, k, v = _clustered(64 * 6, 9)
    a = flat_i8.flat_i8(q, k, v, tile=64, leaf=64, exact_leaves=6, group=2, store="bf16")
    b = flat_i8.flat_i8(q, k, v, tile=64, leaf=64, exact_leaves=6, group=1, store="bf16")
    assert np.array_equal(a["out"], b["out"]) and np.array_equal(a["logz"], b["logz"])
