"""Pins of the oracle's fp8 state store (store="fp8", h3/htrc_flat_triton.py:65-72, 132-153,
165-184, 214-254 with FP8 = 1):

* e4m3 codes and values equal torch's own float8_e4m3fn conversion (every code; values at,
  between and around every grid point), fp16 codes numpy's float16;
* the stored state dequantises to the float64 teaching reference's exact leaf identities
  within half an e4m3 step (src/htrc_reference/model.py:35-49);
* select: brute force in float64 (every fp16 x e4m3 product is exact); centred rows give lz;
* tile: all leaves exact -> dense attention over bf16 q.k scores; rows at their centre with
  no exact leaves -> dense attention at the centre within the e4m3 rounding of vb.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import bf16, flat_fp32, flat_i8, htrc_ref

D = 128


def test_e4m3_codes_equal_torch():
    codes = np.arange(256, dtype=np.uint8)
    vals = torch.from_numpy(codes.copy()).view(torch.float8_e4m3fn).float().numpy()
    ours = flat_i8.e4m3_to_f32(codes)
    fin = np.isfinite(vals)
    assert np.array_equal(ours[fin], vals[fin]) and np.all(np.isnan(ours[~fin]))
    grid = np.unique(np.abs(vals[fin]))
    mids = (grid[1:] + grid[:-1]) / 2
    rng = np.random.default_rng(0)
    x = np.concatenate([grid, mids, np.nextafter(mids, 0), np.nextafter(mids, 1),
                        rng.standard_normal(20000) * 30, rng.standard_normal(5000) * 1e-3]).astype(np.float32)
    x = x[np.abs(x) <= 448]
    x = np.concatenate([x, -x])
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(flat_i8.f32_to_e4m3(x), want)
    assert flat_i8.f32_to_e4m3(np.float32([500.0, -1e9]))[0] == 0x7E       # saturates at 448


def test_f16_codes_equal_numpy():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(20000) * 100, rng.standard_normal(5000) * 1e-5,
                        np.float32([6.1035156e-05, 65504, 65519, 2.0 ** -24, 1.5 * 2.0 ** -24])]).astype(np.float32)
    x = np.concatenate([x, -x])
    assert np.array_equal(flat_i8.f32_to_f16(x), x.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("leaf", [16, 64])
def test_fp8_state_dequantises_to_exact_leaf_identities(leaf):
    rng = np.random.default_rng(leaf)
    nt, nk, scale = 3, 4 * leaf, 1 / math.sqrt(D)
    mu = (rng.standard_normal((nt, D)) * 1.5).astype(np.float32)
    k = bf16.from_f32((rng.standard_normal((nk, D)) * 1.5).astype(np.float32))
    v = bf16.from_f32(rng.standard_normal((nk, D)).astype(np.float32))
    g8, sg, vb8, sv, lz = flat_i8.stats_fp8(mu, k, v, leaf, scale)
    kf, vf = bf16.to_f32(k).astype(np.float64), bf16.to_f32(v).astype(np.float64)
    for t in range(nt):
        for l in range(nk // leaf):
            sl = slice(l * leaf, (l + 1) * leaf)
            ex = htrc_ref.leaf_stats(kf[sl], vf[sl], scale * mu[t].astype(np.float64))
            assert abs(lz[t, l] - ex.log_mass) <= 2e-5 * (1 + abs(ex.log_mass))
            g = scale * ex.gradient
            np.testing.assert_allclose(sg[t, l], np.abs(g).max() / 448, rtol=1e-5)
            np.testing.assert_allclose(sv[t, l], np.abs(ex.value).max() / 448, rtol=1e-5)
            gd = flat_i8.e4m3_to_f32(g8[t, l]).astype(np.float64) * sg[t, l]
            vd = flat_i8.e4m3_to_f32(vb8[t, l]).astype(np.float64) * sv[t, l]
            # half a step of e4m3 (2^-4 relative) above its subnormal floor (2^-10 of the scale)
            assert np.all(np.abs(gd - g) <= np.maximum(np.abs(g) * 2 ** -4, 2 ** -10 * 448 * sg[t, l]) * 1.01)
            assert np.all(np.abs(vd - ex.value) <= np.maximum(np.abs(ex.value) * 2 ** -4, 2 ** -10 * 448 * sv[t, l]) * 1.01)
            assert np.abs(flat_i8.e4m3_to_f32(g8[t, l])).max() == 448


def _clustered(n, seed):
    rng = np.random.default_rng(seed)
    runs = max(1, n // 64)
    c = rng.standard_normal((runs, D)) * 1.5
    rid = np.minimum(np.arange(n) // 64, runs - 1)
    q = bf16.from_f32((c[rid] + 0.5 * rng.standard_normal((n, D))).astype(np.float32))
    k = bf16.from_f32((c[rid] + 0.5 * rng.standard_normal((n, D))).astype(np.float32))
    v = bf16.from_f32(rng.standard_normal((n, D)).astype(np.float32))
    return q, k, v


def test_select_fp8_brute_force_and_centred_rows():
    q, k, v = _clustered(1024, 3)
    st = flat_i8.flat_i8(q, k, v, tile=64, leaf=64, exact_leaves=4, store="fp8")
    nt, nb, _ = st["g8"].shape
    dq = st["dq16"].view(np.float16).astype(np.float64).reshape(nt, 64, D)
    g = flat_i8.e4m3_to_f32(st["g8"]).astype(np.float64)
    for stride in (1, 4):
        sel = flat_i8.select_fp8(st["dq16"], 64, st["g8"], st["sg"], st["lz"], stride)
        want = np.einsum("trd,tld->trl", dq[:, ::stride], g).max(1) * st["sg"] + st["lz"]
        np.testing.assert_allclose(sel, want, rtol=1e-5, atol=1e-5)
    zero = np.zeros_like(st["dq16"])
    assert np.array_equal(flat_i8.select_fp8(zero, 64, st["g8"], st["sg"], st["lz"], 1), st["lz"])


@pytest.mark.parametrize("leaf,splits", [(64, 4), (32, 1)])
def test_fp8_all_leaves_exact_is_dense_bf16_attention(leaf, splits):
    n = 1000
    q, k, v = _clustered(1024, leaf)
    q = q[:n]
    nb = 1024 // leaf
    scale = 1 / math.sqrt(D)
    st = flat_i8.flat_i8(q, k, v, tile=64, leaf=leaf, exact_leaves=nb, splits=splits, bn=64, store="fp8")
    assert st["excl"].all()
    qf, kf, vf = (bf16.to_f32(x).astype(np.float64) for x in (q, k, v))
    s = qf @ kf.T * scale
    m = s.max(1, keepdims=True)
    e = np.exp(s - m)
    ref = e @ vf / e.sum(1, keepdims=True)
    assert np.linalg.norm(st["out"] - ref) / np.linalg.norm(ref) < 4e-3          # bf16 rounding of p only
    assert np.abs(st["logz"] - (np.log(e.sum(1)) + m[:, 0])).max() < 2e-5 * (1 + np.abs(m).max())


def test_fp8_centre_collapse_far_field():
    """Rows at their tile's centre with no exact leaves: softmax attention at the centre, up to
    the e4m3 rounding of vb (and fp16 of p sv)."""
    rng = np.random.default_rng(5)
    nt, nk, leaf = 4, 1024, 64
    cen = bf16.round_f32((rng.standard_normal((nt, D)) * 0.7).astype(np.float32))
    q = np.repeat(cen, 64, 0)
    k = bf16.from_f32((rng.standard_normal((nk, D)) * 1.5).astype(np.float32))
    v = bf16.from_f32(rng.standard_normal((nk, D)).astype(np.float32))
    st = flat_i8.flat_i8(q, k, v, tile=64, leaf=leaf, exact_leaves=0, splits=2, bn=64, store="fp8")
    assert np.all(st["dq16"] == 0)
    dense, dlz = flat_fp32.dense(cen, bf16.to_f32(k), bf16.to_f32(v))
    out = st["out"].reshape(nt, 64, D)
    for t in range(nt):
        ref = np.broadcast_to(dense[t], out[t].shape)
        assert np.linalg.norm(out[t] - ref) / np.linalg.norm(ref) < 4e-2
        assert np.abs(st["logz"].reshape(nt, 64)[t] - dlz[t]).max() < 1e-4 * (1 + abs(dlz[t]))
