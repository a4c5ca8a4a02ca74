"""Error structure of an approximate attention output against a reference output.

The same report as the reference's ``metrics(out, ref)``
(tools/compare_h3_error_structure.py:45-64), so numbers from either side compare directly.
``out`` and ``ref`` are [rows, D] (any float dtype, any device); rows are query tokens in
sequence order.  Percentages are in percent.

  err     relative L2 of the whole output
  rows30  share of rows whose own relative error exceeds 30 %   (rows50: 50 %)
  rowp99  99th percentile of the per-row relative error (on at most ~200k evenly spaced rows)
  bias    share of the error energy in the token-mean error (systematic drift vs noise)
  corr1   mean cosine between the error vectors of neighbouring rows (blur ~1, grain ~0)
  gain    |out| / |ref|
  cos     cosine between out and ref over all rows
"""
from __future__ import annotations

import torch


def metrics(out: torch.Tensor, ref: torch.Tensor) -> dict:
    o = out.float()
    r = ref.float()
    if o.shape != r.shape or o.dim() != 2:
        raise ValueError("out and ref must be [rows, D] of one shape")
    err = o - r
    e_norm, r_norm, o_norm = err.norm(), r.norm(), o.norm()
    row_err = err.norm(dim=1) / r.norm(dim=1).clamp_min(1e-9)
    mean_err = err.mean(dim=0)
    bias = mean_err.square().sum() * err.shape[0] / err.square().sum().clamp_min(1e-12)
    unit = err / err.norm(dim=1, keepdim=True).clamp_min(1e-9)
    corr1 = (unit[1:] * unit[:-1]).sum(dim=1).mean()
    step = max(1, row_err.numel() // 200000)
    return {
        "err": float(e_norm / r_norm) * 100,
        "rows30": float((row_err > 0.3).float().mean()) * 100,
        "rows50": float((row_err > 0.5).float().mean()) * 100,
        "rowp99": float(torch.quantile(row_err[::step], 0.99)) * 100,
        "bias": float(bias) * 100,
        "corr1": float(corr1),
        "gain": float(o_norm / r_norm),
        "cos": float((o * r).sum() / (o_norm * r_norm)),
    }
