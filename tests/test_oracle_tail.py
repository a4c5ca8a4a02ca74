"""Pins of the oracle's tail merge (h3/htrc_flat_triton.py:187-207 for <= 16 tail keys, bf16
operands; :381-388 for more, fp32): the result must be one softmax over the main keys and the
tail keys.  The main part is given as an exact dense partial, so the merged output must equal
dense attention over the concatenated keys, computed directly in float64."""
from __future__ import annotations

import math

import numpy as np

from oracle import bf16, flat_i8

D = 128


def _dense(q, k, v, scale):
    s = (q.astype(np.float64) @ k.T.astype(np.float64)) * scale
    m = s.max(axis=1)
    p = np.exp(s - m[:, None])
    z = p.sum(axis=1)
    return (p @ v.astype(np.float64)) / z[:, None], m + np.log(z)


def _bf(x):
    return bf16.round_f32(x.astype(np.float32))


def test_fp32_tail_equals_dense_over_all_keys():
    rng = np.random.default_rng(0)
    q = rng.standard_normal((96, D)).astype(np.float32)
    k1, v1 = rng.standard_normal((200, D)).astype(np.float32), rng.standard_normal((200, D)).astype(np.float32)
    k2, v2 = rng.standard_normal((24, D)).astype(np.float32), rng.standard_normal((24, D)).astype(np.float32)
    scale = 1 / math.sqrt(D)
    o1, z1 = _dense(q, k1, v1, scale)
    out, logz = flat_i8.tail_merge(o1.astype(np.float32), z1.astype(np.float32), q, k2, v2, scale)
    want, wz = _dense(q, np.concatenate([k1, k2]), np.concatenate([v1, v2]), scale)
    assert np.abs(out - want).max() <= 2e-6 * np.abs(want).max()
    assert np.abs(logz - wz).max() <= 2e-5


def test_bf16_tail_with_equal_scores_is_exact():
    """Seven identical bf16 tail keys: every p is exactly 1, so the bf16 rounding of q, k, v and
    p is exact and the merge must match dense attention over all keys."""
    rng = np.random.default_rng(1)
    q = _bf(rng.standard_normal((64, D)))
    k1, v1 = _bf(rng.standard_normal((128, D))), _bf(rng.standard_normal((128, D)))
    k2 = np.repeat(_bf(rng.standard_normal((1, D))), 7, axis=0)
    v2 = _bf(rng.standard_normal((7, D)))
    scale = 0.0625
    o1, z1 = _dense(q, k1, v1, scale)
    out, logz = flat_i8.tail_merge(o1.astype(np.float32), z1.astype(np.float32), q, k2, v2, scale)
    want, wz = _dense(q, np.concatenate([k1, k2]), np.concatenate([v1, v2]), scale)
    assert np.abs(out - want).max() <= 2e-6 * np.abs(want).max()
    assert np.abs(logz - wz).max() <= 2e-5


def test_empty_main_part_gives_tail_softmax():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((32, D)).astype(np.float32)
    k2, v2 = rng.standard_normal((40, D)).astype(np.float32), rng.standard_normal((40, D)).astype(np.float32)
    out, logz = flat_i8.tail_merge(np.zeros((32, D), np.float32), np.full(32, -np.inf, np.float32), q, k2, v2, 0.1)
    want, wz = _dense(q, k2, v2, 0.1)
    assert np.abs(out - want).max() <= 2e-6 * np.abs(want).max()
    assert np.abs(logz - wz).max() <= 2e-5


def test_short_tail_rounds_to_bf16():
    """<= 16 tail keys go through bf16 (the reference's in-kernel tail block): on inputs that are
    not bf16 values the result moves by about bf16 rounding, and no more."""
    rng = np.random.default_rng(3)
    q = rng.standard_normal((64, D)).astype(np.float32)
    k2, v2 = rng.standard_normal((8, D)).astype(np.float32), rng.standard_normal((8, D)).astype(np.float32)
    base = (np.zeros((64, D), np.float32), np.full(64, -np.inf, np.float32))
    out, _ = flat_i8.tail_merge(*base, q, k2, v2, 0.1)
    exact, _ = _dense(q, k2, v2, 0.1)
    err = np.abs(out - exact).max() / np.abs(exact).max()
    assert 1e-5 < err < 2e-2
