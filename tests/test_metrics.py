"""Closed-form cases of the error-structure report (tools/compare_h3_error_structure.py:45-64)."""
from __future__ import annotations

import math

import pytest
import torch

from htrc_amd.metrics import metrics


def _ref(n=512, d=128, seed=0, zero_mean=True):
    r = torch.randn((n, d), generator=torch.Generator().manual_seed(seed), dtype=torch.float64)
    if zero_mean:
        r = r - r.mean(0, keepdim=True)
    return r.float()


def test_exact_output():
    r = _ref()
    m = metrics(r.clone(), r)
    assert m["err"] == 0 and m["rows30"] == 0 and m["rows50"] == 0 and m["rowp99"] == 0
    assert m["gain"] == pytest.approx(1.0, abs=1e-6) and m["cos"] == pytest.approx(1.0, abs=1e-6)


def test_uniform_scaling():
    """out = 1.2 ref: every row's error is exactly 20 %, gain 1.2, cosine 1, and the error
    (0.2 ref) has the zero token mean of ref: no bias, neighbouring errors as correlated as ref."""
    r = _ref()
    m = metrics(1.2 * r, r)
    assert m["err"] == pytest.approx(20.0, rel=1e-5)
    assert m["rows30"] == 0 and m["rowp99"] == pytest.approx(20.0, rel=1e-5)
    assert m["gain"] == pytest.approx(1.2, rel=1e-6) and m["cos"] == pytest.approx(1.0, abs=1e-6)
    assert m["bias"] == pytest.approx(0.0, abs=1e-6)
    un = r / r.norm(dim=1, keepdim=True)
    assert m["corr1"] == pytest.approx(float((un[1:] * un[:-1]).sum(1).mean()), abs=1e-5)


def test_constant_offset_is_all_bias_and_fully_correlated():
    r = _ref()
    c = torch.randn(128, generator=torch.Generator().manual_seed(3))
    m = metrics(r + c, r)
    assert m["bias"] == pytest.approx(100.0, rel=1e-4)
    assert m["corr1"] == pytest.approx(1.0, abs=1e-5)


def test_alternating_error_grain():
    """e_t = (-1)^t u: neighbouring error vectors are opposite (corr1 = -1) and the token
    mean is zero for an even row count (bias 0)."""
    r = _ref()
    u = torch.randn(128, generator=torch.Generator().manual_seed(4))
    sgn = torch.tensor([(-1.0) ** t for t in range(r.shape[0])])[:, None]
    m = metrics(r + sgn * u, r)
    assert m["corr1"] == pytest.approx(-1.0, abs=1e-5)
    assert m["bias"] == pytest.approx(0.0, abs=1e-4)


def test_row_thresholds():
    """Rows 0..9 of 100 damaged by 40 % (> 30, < 50), rows 10..14 by 60 %."""
    r = _ref(100)
    o = r.clone()
    o[:10] *= 1.4
    o[10:15] *= 1.6
    m = metrics(o, r)
    assert m["rows30"] == pytest.approx(15.0) and m["rows50"] == pytest.approx(5.0)
    e = math.sqrt(float((0.4 * r[:10]).square().sum() + (0.6 * r[10:15]).square().sum()) / float(r.square().sum()))
    assert m["err"] == pytest.approx(100 * e, rel=1e-5)
