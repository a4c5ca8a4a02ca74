"""Pins of the oracle's shared tile centres (kern["group"], h3/htrc_flat.py:223-231):

* group centres: exact on integer-valued rows (every partial sum representable), and the
  mean of the padded rows (last row repeated, last tile repeated) within fp32 rounding of
  a float64 mean;
* the group path equals the per-tile path run with each tile's centre replaced by its
  group's centre, SEL the elementwise max over the group's tiles and every tile of a group
  given the group's near set: bit for bit (select's group max, the tile kernel's state and
  near-set row t // G);
* tiles that repeat within each group: the group path equals the plain per-tile path;
* all leaves exact: the output does not depend on the centres at all.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import bf16, flat_i8

D = 128


def _data(n, nk, seed):
    rng = np.random.default_rng(seed)
    runs = max(1, nk // 64)
    c = rng.standard_normal((runs, D)) * 1.5
    rq = np.minimum(np.arange(n) * runs // n, runs - 1)
    rk = np.arange(nk) // 64
    q = (c[rq] + 0.5 * rng.standard_normal((n, D))).astype(np.float32)
    k = bf16.from_f32((c[rk] + 0.5 * rng.standard_normal((nk, D))).astype(np.float32))
    v = bf16.from_f32(rng.standard_normal((nk, D)).astype(np.float32))
    return q, k, v


def _padded_rows(q, tile, group):
    n = q.shape[0]
    nt = -(-n // tile)
    ng = -(-nt // group)
    rows = []
    for g in range(ng):
        for j in range(group * tile):
            t = min(g * group + j // tile, nt - 1)
            rows.append(min(t * tile + j % tile, n - 1))
    return np.asarray(rows).reshape(ng, group * tile)


@pytest.mark.parametrize("n,group", [(64 * 8, 2), (64 * 7 + 5, 2), (64 * 10 + 1, 4), (64 * 3, 8)])
def test_group_centres_are_means_of_padded_rows(n, group):
    rng = np.random.default_rng(n + group)
    qi = rng.integers(-50, 51, size=(n, D)).astype(np.float32)   # integer rows: sums are exact
    mu = flat_i8.group_centres(qi, 64, group)
    rows = _padded_rows(qi, 64, group)
    want = qi[rows].astype(np.float64).sum(1) / (group * 64)
    assert np.array_equal(mu, want.astype(np.float32))
    q = rng.standard_normal((n, D)).astype(np.float32)
    mu = flat_i8.group_centres(q, 64, group)
    want = q[rows].astype(np.float64).mean(1)
    assert np.abs(mu - want).max() <= 1e-5 * max(1.0, np.abs(want).max())


@pytest.mark.parametrize("n,group,stride", [(64 * 8, 2, 1), (64 * 9 + 17, 4, 1), (64 * 6, 3, 4)])
def test_group_path_equals_per_tile_path_with_group_centres(n, group, stride):
    q, k, v = _data(n, 64 * 24, n)
    leaf, ex, scale = 64, 5, 1 / math.sqrt(D)
    st = flat_i8.flat_i8(q, k, v, tile=64, leaf=leaf, exact_leaves=ex, splits=2, bn=64,
                         sel_stride=stride, group=group)
    nt = -(-n // 64)
    rep = np.minimum(np.arange(nt) // group, st["mu"].shape[0] - 1)
    mu_t = st["mu"][rep]                                          # each tile gets its group's centre
    q8, sq, dq8, sdq = flat_i8.pack_q(q, 64, mu_t, 1)
    for a, b in ((q8, st["q8"]), (sq, st["sq"]), (dq8, st["dq8"]), (sdq, st["sdq"])):
        assert np.array_equal(a, b)
    g8, sg, vb, lz = flat_i8.stats(mu_t, k, v, leaf, scale)
    assert np.array_equal(g8, st["g8"][rep]) and np.array_equal(vb, st["vb"][rep])
    sel_t = flat_i8.select(dq8, sdq, 64, g8, sg, lz, stride)
    ng = st["mu"].shape[0]
    sel_g = np.stack([sel_t[g * group: min(nt, (g + 1) * group)].max(0) for g in range(ng)])
    assert np.array_equal(sel_g.view(np.uint32), st["sel"].view(np.uint32))
    pt = {"q8": q8, "sq": sq, "dq8": dq8, "sdq": sdq, "g8": g8, "sg": sg, "vb": vb, "lz": lz,
          "k8": st["k8"], "ks": st["ks"], "v": st["v"], "idx": st["idx"][rep], "excl": st["excl"][rep]}
    pm, pl, pacc = flat_i8.tile_partials(pt, tile=64, leaf=leaf, scale=scale, splits=2, bn=64)
    out, logz = flat_i8.merge(pm, pl, pacc)
    assert np.array_equal(out[:n], st["out"]) and np.array_equal(logz[:n], st["logz"])


def test_repeated_tiles_make_the_group_path_the_tile_path():
    """Every group's tiles are copies of one 64-row block with values on a 1/16 grid, so the
    group centre equals each tile's centre exactly; the state, routing and output are those
    of the plain per-tile operator."""
    rng = np.random.default_rng(7)
    group, ngr = 4, 3
    blocks = np.round(rng.standard_normal((ngr, 64, D)) * 16) / 16
    q = np.repeat(blocks, group, axis=0).reshape(-1, D).astype(np.float32)
    _, k, v = _data(64, 64 * 16, 8)
    a = flat_i8.flat_i8(q, k, v, tile=64, leaf=64, exact_leaves=3, group=group)
    b = flat_i8.flat_i8(q, k, v, tile=64, leaf=64, exact_leaves=3, group=1)
    assert np.array_equal(a["mu"], b["mu"][::group])
    assert np.array_equal(a["g8"], b["g8"][::group]) and np.array_equal(a["idx"], b["idx"][::group])
    assert np.array_equal(a["out"], b["out"]) and np.array_equal(a["logz"], b["logz"])


def test_all_leaves_exact_output_does_not_depend_on_centres():
    q, k, v = _data(64 * 6 + 9, 64 * 8, 3)
    outs = [flat_i8.flat_i8(q, k, v, tile=64, leaf=64, exact_leaves=8, group=g)["out"] for g in (1, 2, 3)]
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
