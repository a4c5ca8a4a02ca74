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
