"""Pins of the oracle's k-means query order (h3/htrc_flat.py:47-61):

* the sample positions are torch's device ``linspace(0, n - 1, m).round()`` (float32,
  elementwise from both ends; the GPU suite compares with torch.linspace on the device —
  torch's CPU kernel builds its upper half from vector bases and differs in the last bit):
  here, within fp32 rounding of the exact i (n - 1) / (m - 1) and equal to its rounding
  away from half-integer ties, with both ends exact;
* on data whose nearest-centre margins are wide at every Lloyd step (checked), the oracle's
  permutation equals the reference's algorithm run with torch's library routines in float64
  (cdist, index_add_, where, stable argsort), so the iteration count, the update of empty
  centres and the stable order are all fixed by the reference;
* the order is a permutation, grouped by nearest centre, and stable within a centre.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import flat_i8

D = 128


def _torch_kmeans_f64(q, clusters, sample, iters):
    """h3/htrc_flat.py:47-61 with float64 tensors; also the smallest relative margin between
    the nearest and second-nearest centre seen by any assignment."""
    n = q.shape[0]
    x = torch.from_numpy(q).double()
    m = min(sample, n)
    idx = torch.tensor([flat_i8.linspace_round(n - 1, m, i) for i in range(m)])       # device linspace
    s = x.index_select(0, idx)
    c = s[torch.tensor([flat_i8.linspace_round(m - 1, clusters, j) for j in range(clusters)])].clone()
    margin = np.inf

    def nearest(pts):
        nonlocal margin
        dist = torch.cdist(pts, c)
        if clusters > 1:
            two = dist.topk(2, dim=1, largest=False).values
            margin = min(margin, float(((two[:, 1] - two[:, 0]) / two[:, 1].clamp_min(1e-30)).min()))
        return dist.argmin(1)

    for _ in range(iters):
        a = nearest(s)
        sums = torch.zeros_like(c).index_add_(0, a, s)
        cnt = torch.zeros((clusters,), dtype=s.dtype).index_add_(0, a, torch.ones_like(a, dtype=s.dtype))
        c = torch.where((cnt > 0)[:, None], sums / cnt.clamp_min(1.0)[:, None], c)
    assign = nearest(x)
    return torch.argsort(assign, stable=True).numpy(), assign.numpy(), margin


def _planted(n, k, seed, spread=4.0, noise=0.3, sample=None):
    """Rows of k planted clusters in random order; with ``sample`` given, the rows the k initial
    centres are taken from carry labels 0..k-1, one centre per planted cluster."""
    rng = np.random.default_rng(seed)
    means = rng.standard_normal((k, D)) * spread
    lab = rng.integers(0, k, size=n)
    if sample is not None:
        m = min(sample, n)
        for j in range(k):
            lab[flat_i8.linspace_round(n - 1, m, flat_i8.linspace_round(m - 1, k, j))] = j
    return (means[lab] + noise * rng.standard_normal((n, D))).astype(np.float32), lab


@pytest.mark.parametrize("n,m", [(64512, 4096), (4096, 4096), (5000, 4096), (1000, 33), (100, 7), (77, 1),
                                 (124992, 4096), (64512, 32)])
def test_sample_positions_round_the_exact_grid(n, m):
    got = np.array([flat_i8.linspace_round(n - 1, m, i) for i in range(m)])
    assert got[0] == 0 and got[-1] == (n - 1 if m > 1 else 0)
    if m == 1:
        return
    exact = np.arange(m, dtype=np.float64) * (n - 1) / (m - 1)
    assert np.abs(got - exact).max() <= 0.5 + 1e-3 * (n - 1) / (m - 1) + 1e-6
    far = np.abs(exact - np.floor(exact) - 0.5) > 1e-5 * max(1.0, n)     # not next to a half-integer tie
    assert np.array_equal(got[far], np.rint(exact[far]).astype(np.int64))


@pytest.mark.parametrize("n,clusters,sample,iters,seed", [
    (3000, 32, 4096, 8, 0),         # sample = all rows
    (9000, 32, 1024, 8, 1),         # strided sample
    (2000, 12, 500, 3, 2),
    (5000, 64, 4096, 1, 3),
    (777, 7, 64, 0, 4),             # no Lloyd step: the initial centres order the rows
])
def test_order_equals_reference_algorithm_in_float64(n, clusters, sample, iters, seed):
    q, lab = _planted(n, clusters, seed, sample=sample)
    want, assign, margin = _torch_kmeans_f64(q, clusters, sample, iters)
    assert margin > 1e-2, f"test premise: nearest-centre margin {margin:.2e} too small"
    assert np.array_equal(assign, lab)                   # premise: the planted partition
    got = flat_i8.kmeans_order(q, clusters, sample, iters)
    assert np.array_equal(got, want)


def test_permutation_grouped_and_stable():
    """Clustered rows (not well separated): whatever the fp32 assignment, the order is a
    permutation whose blocks of one nearest centre keep row order, and the first rows of
    consecutive blocks follow the centre order."""
    q, _ = _planted(4000, 64, 7, spread=1.5, noise=0.5)
    perm = flat_i8.kmeans_order(q, 32, 4096, 8)
    assert np.array_equal(np.sort(perm), np.arange(q.shape[0]))
    # empty centres keep their initial position, so every centre is some sample row; the fp32
    # assignment is recovered here by re-running the oracle on the permuted rows' own order:
    # within a block the indices increase, so the number of descents bounds the blocks
    descents = int((np.diff(perm) < 0).sum())
    assert descents <= 31


def test_more_centres_than_rows_and_single_row():
    q, _ = _planted(10, 3, 9)
    perm = flat_i8.kmeans_order(q, 32, 4096, 8)
    assert np.array_equal(np.sort(perm), np.arange(10))
    assert np.array_equal(flat_i8.kmeans_order(q[:1], 32, 4096, 8), [0])


def test_lloyd_step_moves_a_blob():
    """Blobs A (-10), B (-2) and a large C (+10) on one axis; the two initial centres come
    from A and B.  Before any step B and C share a centre; after one update that centre sits
    near C and B moves over to A's.  The oracle follows the float64 reference algorithm for
    0, 1 and 3 steps, and 0 and 1 steps order the rows differently."""
    rng = np.random.default_rng(11)
    n, m = 1200, 4096
    pos = np.where(np.arange(n) < 200, -10.0, np.where(np.arange(n) < 400, -2.0, 10.0))
    rng.shuffle(pos)
    pos[flat_i8.linspace_round(n - 1, n, flat_i8.linspace_round(n - 1, 2, 0))] = -10.0
    pos[flat_i8.linspace_round(n - 1, n, flat_i8.linspace_round(n - 1, 2, 1))] = -2.0
    q = (0.1 * rng.standard_normal((n, D))).astype(np.float32)
    q[:, 0] += pos.astype(np.float32)
    got = {}
    for iters in (0, 1, 3):
        want, assign, margin = _torch_kmeans_f64(q, 2, m, iters)
        assert margin > 5e-2, f"premise: margin {margin:.2e}"
        got[iters] = flat_i8.kmeans_order(q, 2, m, iters)
        assert np.array_equal(got[iters], want)
    assert not np.array_equal(got[0], got[1])
