"""The fp32-dot oracle (oracle/flat_f32.py) pinned on the CPU: its TF32 rounding against an
independent float64 rounding, its IEEE fp32 operator against the reference's torch backend
(oracle/flat_fp32.py, h3/htrc_flat.py:279-388) and against dense attention, and its bf16 store
against the fp32 store's state rounded to bf16."""
from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import bf16, flat_f32, flat_fp32


def _tf32_by_value(x: np.ndarray) -> np.ndarray:
    """TF32 rounding from the values: the two neighbours on the 11-significant-bit grid of |x|'s
    binade, the nearer one, ties to the larger magnitude (float64 arithmetic)."""
    out = np.empty_like(x, dtype=np.float64)
    for i, xv in enumerate(x.astype(np.float64)):
        if not np.isfinite(xv) or xv == 0.0:
            out[i] = xv
            continue
        a = abs(xv)
        e = max(math.floor(math.log2(a)), -126)
        while 2.0 ** e > a:            # guard the log's rounding
            e -= 1
        while 2.0 ** (e + 1) <= a:
            e += 1
        ulp = 2.0 ** (max(e, -126) - 10)
        lo = math.floor(a / ulp) * ulp
        hi = lo + ulp
        r = hi if (a - lo) >= (hi - a) else lo
        out[i] = math.copysign(r, xv)
    return out


def test_tf32_rounding_known_values():
    one = np.float32(1.0)
    x = np.array([1.0, 1 + 2 ** -11, -(1 + 2 ** -11), 1 + 2 ** -11 - 2 ** -23, 1 + 3 * 2 ** -11,
                  np.nextafter(np.float32(2), np.float32(0)), np.inf, -np.inf, 0.0, -0.0], np.float32)
    want = np.array([1.0, 1 + 2 ** -10, -(1 + 2 ** -10), 1.0, 1 + 2 ** -9, 2.0, np.inf, -np.inf, 0.0, -0.0],
                    np.float32)
    got = flat_f32.tf32_rna(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.isnan(flat_f32.tf32_rna(np.array([np.nan], np.float32)))[0]
    # the largest finite fp32 rounds up past the largest TF32 value: infinity
    big = np.array([np.finfo(np.float32).max], np.float32)
    assert np.isinf(flat_f32.tf32_rna(big))[0]
    assert one == flat_f32.tf32_rna(np.array([one]))[0]


def test_tf32_rounding_matches_value_rounding():
    rng = np.random.default_rng(3)
    bits = rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x) & (np.abs(x) < np.float32(3e38))]
    # ties: the exact halfway points, both signs, several binades
    base = rng.integers(0, 2 ** 10, 500).astype(np.float64)
    ties = ((1024 + base + 0.5) * 2.0 ** rng.integers(-20, 20, 500)).astype(np.float32)
    x = np.concatenate([x, ties, -ties])
    got = flat_f32.tf32_rna(x).astype(np.float64)
    want = _tf32_by_value(x)
    assert np.array_equal(got, want)


def _data(n, nk, d, seed):
    rng = np.random.default_rng(seed)
    cent = rng.normal(0, 1.5, (16, d))
    q = cent[rng.integers(0, 16, n)] + rng.normal(0, 0.5, (n, d))
    k = cent[np.repeat(rng.integers(0, 16, nk // 64), 64)] + rng.normal(0, 0.5, (nk, d))
    v = rng.normal(0, 1, (nk, d))
    r = lambda a: bf16.round_f32(a.astype(np.float32))
    return r(q), r(k), r(v)


def _rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("leaf,ex", [(64, 4), (32, 6)])
def test_fp32_store_equals_the_torch_backend(leaf, ex):
    q, k, v = _data(512, 2048, 64, seed=leaf)
    st = flat_f32.flat_f32(q, k, v, tile=64, leaf=leaf, exact_leaves=ex)
    ref, lzr = flat_fp32.flat_fp32(q, k, v, tile=64, exact_leaves=ex, leaf=leaf, return_logz=True)
    # same near sets by construction on this data (no near-ties): fp32 rounding apart
    assert _rel(st["out"], ref) < 1e-5
    assert np.abs(st["logz"] - lzr).max() < 1e-4


def test_all_leaves_near_is_dense_attention():
    q, k, v = _data(256, 1024, 64, seed=5)
    st = flat_f32.flat_f32(q, k, v, tile=64, leaf=64, exact_leaves=16)
    out, lz = flat_fp32.dense(q, k, v)
    assert _rel(st["out"], out) < 1e-6
    assert np.abs(st["logz"] - lz).max() < 1e-5


def test_bf16_store_is_the_rounded_fp32_state():
    q, k, v = _data(256, 1024, 64, seed=7)
    a = flat_f32.flat_f32(q, k, v, leaf=64, exact_leaves=3)
    b = flat_f32.flat_f32(q, k, v, leaf=64, exact_leaves=3, store="bf16")
    assert np.array_equal(b["g"], bf16.round_f32(a["g"])) and np.array_equal(b["vb"], bf16.round_f32(a["vb"]))
    assert np.array_equal(b["lz"], a["lz"])
    # the routing and output from that state: a bf16 rounding away from the fp32 ones
    assert _rel(b["out"], a["out"]) < 1e-2


def test_tf32_operands_change_results_at_tf32_level():
    q, k, v = _data(256, 1024, 64, seed=9)
    a = flat_f32.flat_f32(q, k, v, leaf=64, exact_leaves=3)
    b = flat_f32.flat_f32(q, k, v, leaf=64, exact_leaves=3, prec="tf32")
    r = _rel(b["out"], a["out"])
    assert 1e-7 < r < 2e-3


def _stats_inputs(seed=0, nt=8, nk=1024, d=128):
    rng = np.random.default_rng(seed)
    cent = rng.normal(0, 1.5, (16, d))
    mu = (cent[rng.integers(0, 16, nt)] + rng.normal(0, 0.5, (nt, d))).astype(np.float32)
    k = cent[np.repeat(rng.integers(0, 16, nk // 64), 64)] + rng.normal(0, 0.5, (nk, d))
    v = rng.normal(0, 1, (nk, d))
    return mu, bf16.from_f32(k.astype(np.float32)), bf16.from_f32(v.astype(np.float32))


def test_tf32_statistics_of_the_c_oracle_equal_the_numpy_restatement():
    """The C oracle's leaf statistics with prec="tf32" (every store: the reference's leaf_stats
    takes PREC for all of them) against flat_f32.stats at TF32: lz within fp32 noise where IEEE
    and TF32 differ by ~1e-3 (the centre's rounding), g8 within half a code, and the bf16 store's
    g bits equal to the restatement's bf16 rounding except at fp32-noise ties, where the IEEE
    restatement's differ in 1.4% of entries (the weights' rounding)."""
    from oracle import flat_i8
    mu, kb, vb = _stats_inputs()
    leaf, sc = 64, 1 / math.sqrt(128)
    kf, vf = bf16.to_f32(kb), bf16.to_f32(vb)
    g_t, vb_t, lz_t = flat_f32.stats(mu, kf, vf, leaf, sc, "tf32")
    g_i, _, lz_i = flat_f32.stats(mu, kf, vf, leaf, sc, "ieee")
    assert np.abs(lz_t - lz_i).max() > 3e-4                       # the two precisions do differ
    g8, sg, vb16, lz = flat_i8.stats(mu, kb, vb, leaf, sc, "tf32")
    assert np.abs(lz - lz_t).max() <= 2e-5
    assert np.all(np.abs(g8 * sg[..., None].astype(np.float64) - g_t) <= 0.501 * sg[..., None])
    # vb: half a bf16 step (plus fp32 noise where a row's sum cancels), but for the few weights
    # whose fp32 values straddle a TF32 rounding point in the two restatements (2^-11 of a weight)
    far = np.abs(bf16.to_f32(vb16) - vb_t) > 2.0 ** -8 * np.abs(vb_t) + 1e-5
    assert far.mean() <= 0.01, far.mean()
    g16, _, lz16 = flat_i8.stats_bf16(mu, kb, vb, leaf, sc, "tf32")
    assert np.array_equal(lz16, lz)
    flips_t = (g16 != bf16.from_f32(g_t.astype(np.float32))).mean()
    flips_i = (g16 != bf16.from_f32(g_i.astype(np.float32))).mean()
    assert flips_t <= 0.002 and flips_i >= 0.005, (flips_t, flips_i)    # measured 1.2e-4 and 1.4e-2
    g8f, sgf, vb8, svf, lzf = flat_i8.stats_fp8(mu, kb, vb, leaf, sc, "tf32")
    assert np.array_equal(lzf, lz)
    # ieee stays the default
    assert np.array_equal(flat_i8.stats(mu, kb, vb, leaf, sc)[3], flat_i8.stats(mu, kb, vb, leaf, sc, "ieee")[3])
