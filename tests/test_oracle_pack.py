"""Pins of the oracle's pack stage (K int8, tile centres, Q / dQ int8) by closed-form
properties -- rounding to nearest, the tie rules of the reference, the amax element
mapping to +-127, scale floors -- over every finite bf16 bit pattern.

Reference: h3/htrc_flat.py:216-218 (K: round half to even), h3/htrc_flat_triton.py:111-117
(Q/dQ: fp32 x +- 0.5 then truncation), h3/htrc_flat.py:142-156 (tile centres).
"""
from __future__ import annotations

import struct

import numpy as np
import pytest

from oracle import bf16, flat_i8

D = 128


def _finite_bf16_patterns():
    b = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = bf16.to_f32(b)
    return b[np.isfinite(f)]


def test_r127_constant():
    assert struct.unpack("<I", struct.pack("<f", flat_i8.r127()))[0] == 0x3C010204
    assert np.float32(flat_i8.r127()) == np.float32(1.0 / 127.0)


def _rows_with_amax(vals: np.ndarray, amax_bits: int) -> np.ndarray:
    """Rows of D bf16 patterns: element 0 fixes amax, the rest are test values (|v| <= amax)."""
    amax = bf16.to_f32(np.array([amax_bits], np.uint16))[0]
    v = vals[np.abs(bf16.to_f32(vals)) <= amax]
    n = -(-v.size // (D - 1))
    rows = np.zeros((n, D), np.uint16)
    flat = np.zeros(n * (D - 1), np.uint16)
    flat[: v.size] = v
    rows[:, 1:] = flat.reshape(n, D - 1)
    rows[:, 0] = amax_bits
    rows[1::2, 0] = amax_bits | 0x8000          # negative amax element on odd rows
    return rows


@pytest.mark.parametrize("amax", [1.0, 3.0, 0.0078125, 1.0e5, 2.0 ** -120])
def test_pack_k_exhaustive_rounding(amax):
    amax_bits = int(bf16.from_f32(np.array([amax], np.float32))[0])
    rows = _rows_with_amax(_finite_bf16_patterns(), amax_bits)
    k8, ks = flat_i8.pack_k(rows)
    x = bf16.to_f32(rows)
    a = np.float32(bf16.to_f32(np.array([amax_bits], np.uint16))[0])
    s = max(np.float32(a * np.float32(flat_i8.r127())), np.float32(1e-20))
    assert np.all(ks == s)
    q = (x.astype(np.float64) / np.float64(s))                    # exact ratio, no fp32 rounding
    k8i = k8.astype(np.float64)
    assert np.all(np.abs(k8i) <= 127)
    if s > np.float32(1e-20):
        assert np.all(np.abs(k8[:, 0].astype(np.int32)) == 127)    # amax element -> +-127
    r32 = (x / s).astype(np.float32)                               # the fp32 quotient the pack rounds
    err = np.abs(r32.astype(np.float64) - k8i)
    assert np.all(err <= 0.5)                                      # nearest
    tie = err == 0.5
    assert np.all(k8[tie] % 2 == 0)                                # ties to even
    assert np.all(np.abs(q - k8i) <= 0.5 + 1e-5)


def test_pack_k_zero_row_and_tiny():
    rows = np.zeros((3, D), np.uint16)
    rows[1, 5] = bf16.from_f32(np.array([1e-30], np.float32))[0]
    rows[2] = bf16.from_f32(np.linspace(-1e-19, 1e-19, D).astype(np.float32))
    k8, ks = flat_i8.pack_k(rows)
    assert np.all(ks[:2] == np.float32(1e-20))
    assert np.all(k8[0] == 0) and np.all(k8[1] == 0)
    assert ks[2] == np.float32(1e-20)                              # 1e-19 / 127 < 1e-20: the floor applies
    assert np.abs(k8[2]).max() == 10                               # 1e-19 / 1e-20 = 10


def _pack_q_rows(rows_f32: np.ndarray):
    n = rows_f32.shape[0]
    mu = flat_i8.tile_centres(rows_f32, 64)
    return mu, flat_i8.pack_q(rows_f32, 64, mu)


@pytest.mark.parametrize("amax", [1.0, 127.0, 0.5, 6.0e3])
def test_pack_q_exhaustive_rounding(amax):
    amax_bits = int(bf16.from_f32(np.array([amax], np.float32))[0])
    rows = bf16.to_f32(_rows_with_amax(_finite_bf16_patterns(), amax_bits))
    mu, (q8, sq, dq8, sdq) = _pack_q_rows(rows)
    n = rows.shape[0]
    a = bf16.to_f32(np.array([amax_bits], np.uint16))[0]
    s = np.maximum(np.float32(a * np.float32(flat_i8.r127())), np.float32(1e-20))
    assert np.all(sq[:n] == s)
    r32 = (rows / s).astype(np.float32).astype(np.float64)
    qi = q8[:n].astype(np.float64)
    err = np.abs(r32 - qi)
    assert np.all(np.abs(qi) <= 127)
    assert np.all(err <= 0.5 + 1e-12)
    tie = err == 0.5
    assert np.all(np.abs(qi[tie]) > np.abs(r32[tie]))             # ties away from zero
    assert np.all(np.abs(q8[:n, 0].astype(np.int32)) == 127)
    # dq = q - mu uses the same rounding on the centred rows
    t = np.arange(n) // 64
    dq = (rows - mu[t]).astype(np.float32)
    ad = np.abs(dq).max(1)
    sd = np.maximum((ad * np.float32(flat_i8.r127())).astype(np.float32), np.float32(1e-20))
    assert np.all(sdq[:n] == sd)
    rd = (dq / sd[:, None]).astype(np.float32).astype(np.float64)
    ed = np.abs(rd - dq8[:n].astype(np.float64))
    assert np.all(ed <= 0.5 + 1e-12)


def test_pack_q_rounds_049999997_up():
    """trunc(x + 0.5) in fp32 sends 0.49999997 to 1 (x + 0.5 rounds to 1.0): the reference's rule."""
    row = np.zeros((1, D), np.float32)
    row[0, 0] = 127.0                       # scale = 127 * fp32(1/127) = 1.0 exactly
    row[0, 1] = np.float32(0.49999997)
    row[0, 2] = np.float32(-0.49999997)
    row[0, 3] = np.float32(0.5)
    row[0, 4] = np.float32(-2.5)
    row[0, 5] = np.float32(0.49999994)      # 0.49999994 + 0.5 = 0.99999994: stays below 1
    _, (q8, sq, _, _) = _pack_q_rows(row)
    assert sq[0] == np.float32(1.0)
    assert list(q8[0, :6]) == [127, 1, -1, 1, -3, 0]


def test_tile_centres_real_rows_only_and_padding():
    rng = np.random.default_rng(0)
    n = 100
    q = rng.standard_normal((n, D)).astype(np.float32)
    q[64:] += 10.0 * np.arange(36, dtype=np.float32)[:, None]        # last tile rows very different
    mu = flat_i8.tile_centres(q, 64)
    assert mu.shape == (2, D)
    np.testing.assert_allclose(mu[0], q[:64].astype(np.float64).mean(0), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(mu[1], q[64:].astype(np.float64).mean(0), rtol=1e-5, atol=1e-5)
    q8, sq, dq8, sdq = flat_i8.pack_q(q, 64, mu)
    assert q8.shape == (128, D)
    for p in range(n, 128):                                        # pad rows repeat the last real row
        assert np.array_equal(q8[p], q8[n - 1]) and sq[p] == sq[n - 1]
        assert np.array_equal(dq8[p], dq8[n - 1]) and sdq[p] == sdq[n - 1]


def test_tile_centre_of_constant_tile_is_exact():
    # short-mantissa values: every partial sum of the 64 copies is exact in fp32
    q = np.tile((np.round(np.linspace(-3, 3, D) * 8) / 8).astype(np.float32), (64, 1))
    mu = flat_i8.tile_centres(q, 64)
    assert np.array_equal(mu[0], q[0])
    _, _, dq8, sdq = flat_i8.pack_q(q, 64, mu)
    assert np.all(dq8 == 0) and np.all(sdq == np.float32(1e-20))
