"""CPU restatement of the reference's fake quantisation -- test infrastructure only.

fake_quant (h3/htrc_flat.py:68-96): x [..., D] round-trips through int8 / int4 / fp8 (e4m3fn) /
fp4 (e2m1) with one symmetric scale per group of `group` consecutive values of a row (group 0:
the whole row; fp4 defaults to 16).  Every operation is one IEEE fp32 operation, as the torch
ops are: s = max(max|x|, 1e-20) / qmax; int: rint(x / s) (nearest even) clamped to +-qmax,
times s; fp8: the e4m3fn code of x / s clamped to +-448 (nearest even), decoded, times s; fp4:
the e2m1 magnitude chosen by the thresholds (h3/htrc_flat.py:64-65; torch.bucketize: a value
on a threshold takes the lower magnitude) with x's sign (sign(0) = 0), times s.
"""
from __future__ import annotations

import numpy as np

from . import flat_i8

FP4 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], np.float32)
FP4_THR = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], np.float32)
QMAX = {"int8": 127.0, "int4": 7.0, "fp8": 448.0, "fp4": 6.0}


def fake_quant(x, fmt: str, group: int = 0) -> np.ndarray:
    x = np.asarray(x, np.float32)
    d = x.shape[-1]
    if fmt == "fp4" and not group:
        group = 16
    gsz = d if not group else int(group)
    if d % gsz:
        raise ValueError("quant group must divide the feature size")
    if fmt not in QMAX:
        raise ValueError(f"unknown quant format {fmt}")
    y = x.reshape(*x.shape[:-1], d // gsz, gsz)
    amax = np.maximum(np.abs(y).max(-1, keepdims=True), np.float32(1e-20)).astype(np.float32)
    qmax = np.float32(QMAX[fmt])
    sc = (amax / qmax).astype(np.float32)
    t = (y / sc).astype(np.float32)
    if fmt in ("int8", "int4"):
        r = np.clip(np.rint(t), -qmax, qmax).astype(np.float32)
    elif fmt == "fp8":
        codes = flat_i8.f32_to_e4m3(np.clip(t, -448.0, 448.0).astype(np.float32))
        r = flat_i8.e4m3_to_f32(codes).astype(np.float32)
    else:
        idx = np.searchsorted(FP4_THR, np.abs(t), side="left")     # thresholds strictly below |t|
        sgn = np.where(y > 0, np.float32(1.0), np.where(y < 0, np.float32(-1.0), np.float32(0.0)))  # sign(0) = +0
        r = (sgn * FP4[idx]).astype(np.float32)
    return (r * sc).astype(np.float32).reshape(x.shape)
