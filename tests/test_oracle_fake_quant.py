"""Pins of the fake-quant restatement (oracle/fake_quant.py; h3/htrc_flat.py:68-96) by what the
formats fix independently of the formula: every output is a grid point times the group scale,
the grid point is the nearest one to x / s (brute force over the grid, in float64) with the
format's tie rule, the group maximum lands on the top of the grid, groups are independent,
and the e4m3 grid comes from torch's own float8_e4m3fn decode."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.fake_quant import fake_quant

E4M3 = np.unique(np.abs(torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn)
                         .float().numpy()))
E4M3 = E4M3[np.isfinite(E4M3)].astype(np.float64)                  # 0 .. 448, every finite magnitude


def _scale(x, fmt, group):
    d = x.shape[-1]
    gsz = d if not group else group
    y = x.reshape(*x.shape[:-1], d // gsz, gsz)
    amax = np.maximum(np.abs(y).max(-1, keepdims=True), np.float32(1e-20)).astype(np.float32)
    qmax = {"int8": 127.0, "int4": 7.0, "fp8": 448.0, "fp4": 6.0}[fmt]
    return y, (amax / np.float32(qmax)).astype(np.float32)


def _data(seed, rows=64, d=128):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, d)) * np.exp2(rng.integers(-8, 9, (rows, 1)))).astype(np.float32)
    x[3, :16] = 0.0                                                  # an all-zero group
    x[5, 7] = -0.0
    return x


@pytest.mark.parametrize("fmt,group", [("int8", 0), ("int8", 32), ("int4", 0), ("int4", 16)])
def test_int_formats_nearest_integer_step(fmt, group):
    x = _data(1)
    out = fake_quant(x, fmt, group)
    y, sc = _scale(x, fmt, group)
    o = out.reshape(y.shape).astype(np.float64)
    qmax = 127 if fmt == "int8" else 7
    r = np.rint(o / sc)                                              # the integer the output encodes
    assert np.array_equal((r.astype(np.float32) * sc).astype(np.float32), out.reshape(y.shape))
    assert np.abs(r).max() <= qmax
    t = y.astype(np.float64) / sc                                    # exact quotient
    err = np.abs(t - r)
    assert np.all(err <= 0.5 + 1e-6)
    ties = np.isclose(err, 0.5, rtol=0, atol=1e-9)
    assert np.all(r[ties] % 2 == 0)                                  # nearest even at a tie
    top = np.abs(y).argmax(-1)[..., None]
    big = np.take_along_axis(np.abs(r), top, -1)
    nz = np.take_along_axis(np.abs(y), top, -1) > 0
    assert np.all(big[nz] == qmax)                                   # the group maximum hits the top code


def test_int8_exact_ties_round_to_even():
    x = np.zeros((1, 128), np.float32)
    x[0, 0] = 127.0                                                  # s = 1: quotients are the values
    x[0, 1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, 126.5, -2.5, 3.5]
    out = fake_quant(x, "int8")
    assert out[0, :9].tolist() == [127.0, 0.0, 2.0, 2.0, -0.0, -2.0, 126.0, -2.0, 4.0]


def test_fp8_nearest_e4m3_value():
    x = _data(2)
    out = fake_quant(x, "fp8", 0)
    y, sc = _scale(x, "fp8", 0)
    t = np.abs(y.astype(np.float64) / sc)
    # brute force: nearest finite e4m3 magnitude, ties to the even code (the grid index parity)
    dist = np.abs(t[..., None] - E4M3)
    best = dist.min(-1, keepdims=True)
    cand = dist == best
    idx = np.where(cand.sum(-1) > 1, np.argmax(cand & (np.arange(E4M3.size) % 2 == 0), -1), np.argmin(dist, -1))
    want = (np.sign(y) * E4M3[idx]).astype(np.float32)
    assert np.array_equal((want * sc).astype(np.float32), out.reshape(y.shape))


def test_fp4_nearest_grid_value_ties_down():
    x = _data(3)
    grid = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
    out = fake_quant(x, "fp4")                                       # default group 16
    y, sc = _scale(x, "fp4", 16)
    t = np.abs(y.astype(np.float64) / sc)
    dist = np.abs(t[..., None] - grid)
    idx = np.argmin(dist + 1e-12 * np.arange(grid.size), -1)         # ties to the lower magnitude
    want = (np.where(y > 0, 1.0, np.where(y < 0, -1.0, 0.0)) * grid[idx]).astype(np.float32)
    assert np.array_equal((want * sc).astype(np.float32), out.reshape(y.shape))
    z = np.zeros((1, 16), np.float32)
    z[0, :8] = [6.0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]         # every threshold, s = 1
    assert fake_quant(z, "fp4")[0, :8].tolist() == [6.0, 0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0]


@pytest.mark.parametrize("fmt", ["int8", "int4", "fp8", "fp4"])
def test_groups_are_independent_and_zero_groups_stay_zero(fmt):
    x = _data(4)
    a = fake_quant(x, fmt, 32)
    x2 = x.copy()
    x2[:, 32:64] *= 1000.0
    b = fake_quant(x2, fmt, 32)
    keep = np.ones(128, bool)
    keep[32:64] = False
    assert np.array_equal(a[:, keep], b[:, keep])
    assert np.array_equal(fake_quant(x, fmt, 0 if fmt != "fp4" else 16)[3, :16], np.zeros(16, np.float32))


def test_errors():
    with pytest.raises(ValueError, match="divide"):
        fake_quant(np.zeros((2, 128), np.float32), "int8", 48)
    with pytest.raises(ValueError, match="unknown quant format"):
        fake_quant(np.zeros((2, 128), np.float32), "int2", 0)


# ---- select="bound" (oracle flat_i8.bound_select; h3/htrc_flat.py:255-257)

def _bound_case(seed, n, tile, group, nb=12):
    from oracle import bf16, flat_i8
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((n, 128)).astype(np.float32)
    mu = flat_i8.tile_centres(q, tile) if group == 1 else flat_i8.group_centres(q, tile, group)
    g16 = bf16.from_f32(rng.standard_normal((mu.shape[0], nb, 128)).astype(np.float32))
    lz = rng.standard_normal((mu.shape[0], nb)).astype(np.float32)
    return q, mu, g16, lz, flat_i8.bound_select(q, tile, mu, g16, lz, group)


@pytest.mark.parametrize("n,tile,group", [(640, 64, 1), (600, 64, 1), (330, 32, 3), (1000, 64, 4)])
def test_bound_select_against_float64_norms(n, tile, group):
    """SEL = lz + r ||g||: r the largest distance of the group's (padded) rows from the centre and
    ||g|| the leaf slope norm, both against float64 norms; padding repeats real rows, so r is the
    maximum over the group's real rows."""
    from oracle import bf16
    q, mu, g16, lz, sel = _bound_case(n + tile + group, n, tile, group)
    nt = -(-n // tile)
    gnorm = np.linalg.norm(bf16.to_f32(g16).astype(np.float64), axis=-1)
    for gi in range(mu.shape[0]):
        t0, t1 = gi * group, min(nt, (gi + 1) * group)
        rows = np.arange(t0 * tile, min(n, t1 * tile))
        r = np.linalg.norm(q[rows].astype(np.float64) - mu[gi].astype(np.float64), axis=-1).max()
        want = lz[gi].astype(np.float64) + r * gnorm[gi]
        assert np.allclose(sel[gi], want, rtol=2e-6, atol=2e-6 * (1 + np.abs(want).max()))


def test_bound_select_rows_at_the_centre_give_lz():
    from oracle import bf16, flat_i8
    # integer rows: the 64-row sums and the centre are exact, so every row sits on its centre
    q = np.repeat(np.random.default_rng(3).integers(-8, 9, (1, 128)).astype(np.float32), 128, 0)
    mu = flat_i8.tile_centres(q, 64)
    g16 = bf16.from_f32(np.ones((2, 5, 128), np.float32))
    lz = np.arange(10, dtype=np.float32).reshape(2, 5)
    assert np.array_equal(flat_i8.bound_select(q, 64, mu, g16, lz), lz)
