"""The reference's own unit tests (tests/test_reference.py:13-51), restated against the
oracle's float64 restatement of src/htrc_reference/model.py, plus BASELINE configuration 1.

Same fixture as the reference: default_rng(1107), k [128, 8], v [128, 5], c = 0.2 N(0, I),
d = 0.1 N(0, I) (tests/test_reference.py:7-11).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import htrc_ref


@pytest.fixture()
def fx():
    rng = np.random.default_rng(1107)
    k = rng.normal(size=(128, 8))
    v = rng.normal(size=(128, 5))
    c = rng.normal(size=8) * 0.2
    d = rng.normal(size=8) * 0.1
    return k, v, c, d


def test_parent_identities_are_exact(fx):
    """tests/test_reference.py:13-19"""
    k, v, c, _ = fx
    full = htrc_ref.leaf_stats(k, v, c)
    merged = htrc_ref.merge([htrc_ref.leaf_stats(k[i:i + 16], v[i:i + 16], c) for i in range(0, 128, 16)])
    assert abs(full.log_mass - merged.log_mass) < 1e-12
    for f in ("gradient", "hessian", "value", "value_jacobian"):
        np.testing.assert_allclose(getattr(full, f), getattr(merged, f), atol=1e-12)


def test_value_jacobian_finite_difference(fx):
    """tests/test_reference.py:21-28"""
    k, v, c, d = fx
    ref = htrc_ref.leaf_stats(k, v, c)
    u = d / np.linalg.norm(d)
    eps = 1e-5
    fd = (htrc_ref.exact_attention(k, v, c + eps * u) - htrc_ref.exact_attention(k, v, c - eps * u)) / (2 * eps)
    np.testing.assert_allclose(fd, ref.value_jacobian @ u, atol=1e-9, rtol=1e-8)


def test_gradient_and_hessian_finite_difference(fx):
    """The log-mass gradient and Hessian are the derivatives of log-sum-exp (model.py:42-47)."""
    k, v, c, d = fx
    ref = htrc_ref.leaf_stats(k, v, c)
    u = d / np.linalg.norm(d)
    eps = 1e-4
    lp = htrc_ref.exact_log_partition(k, c + eps * u)
    lm = htrc_ref.exact_log_partition(k, c - eps * u)
    l0 = htrc_ref.exact_log_partition(k, c)
    assert abs((lp - lm) / (2 * eps) - ref.gradient @ u) < 1e-8
    assert abs((lp - 2 * l0 + lm) / eps ** 2 - u @ ref.hessian @ u) < 1e-5


def test_at_centroid_root_collapse_is_exact(fx):
    """tests/test_reference.py:30-35"""
    k, v, c, _ = fx
    roots = htrc_ref.forest(k, v, c)
    approx, meta = htrc_ref.evaluate(k, v, c, c, roots)
    np.testing.assert_allclose(approx, htrc_ref.exact_attention(k, v, c), atol=1e-12)
    assert meta["exact_leaves"] == 0


def test_open_all_exact_leaves_is_exact(fx):
    """tests/test_reference.py:37-43"""
    k, v, c, d = fx
    roots = htrc_ref.forest(k, v, c)
    approx, meta = htrc_ref.evaluate(k, v, c + d, c, roots, opening_threshold=0)
    np.testing.assert_allclose(approx, htrc_ref.exact_attention(k, v, c + d), atol=1e-12)
    assert meta["exact_leaves"] == 8


def test_shapes_and_threshold_validation(fx):
    """tests/test_reference.py:45-51"""
    k, v, c, d = fx
    roots = htrc_ref.forest(k, v, c)
    out, info = htrc_ref.evaluate(k, v, c + d, c, roots, opening_threshold=0.01)
    assert out.shape == (5,)
    assert info["visited_nodes"] >= 1
    with pytest.raises(ValueError):
        htrc_ref.evaluate(k, v, c, c, roots, opening_threshold=-1)


def test_forest_structure(fx):
    k, v, c, _ = fx
    roots = htrc_ref.forest(k, v, c, leaf_size=16, fanout=4)
    assert len(roots) == 2                                        # 8 leaves -> 2 parents of 4
    assert all(len(r.children) == 4 for r in roots)
    with pytest.raises(ValueError):
        htrc_ref.forest(k, v, c, leaf_size=0)
    with pytest.raises(ValueError):
        htrc_ref.leaf_stats(k[:0], v[:0], c)


def test_config1_small_sample():
    """BASELINE configuration 1 (float64, 1024 q x 4096 k, d 64, leaves of 64, fanout 4) on
    the first queries.  Opening threshold 0 opens every leaf, so the result is exact
    attention; at the default 0.01 the Taylor-2 log-partition stays within a few 1e-3."""
    exact = htrc_ref.config1(seed=0, query_limit=4, opening_threshold=0.0)
    assert exact["rel_l2_max"] < 1e-10 and exact["logz_abs_max"] < 1e-10
    assert exact["exact_leaves_mean"] == 64
    r = htrc_ref.config1(seed=0, query_limit=8)
    assert r["queries"] == 8 and 0 < r["exact_leaves_mean"] < 64
    assert r["logz_abs_max"] < 0.02
    assert np.isfinite(r["rel_l2_max"]) and r["rel_l2_max"] < 1.0
