"""NumPy fp32 restatement of the reference's torch backend ``_flat`` -- TEST INFRASTRUCTURE ONLY.

Follows h3/htrc_flat.py:279-388 (order="seq"; curvature "lin" or "iso"; select
"max" or "bound"): per chunk of tiles the exact leaf cumulants at the tile
centres, the linear far-field logits, the top-k near leaves replaced by their
exact tokens, and a shared-max merge.  No int8 anywhere; selection uses the fp32
far logits.  This is the reference's CPU path, timed as ``cpu_baseline`` by
bench.py, and it carries the fp32 invariants (all leaves exact = dense
attention; one query per tile with no exact leaves = dense attention).
"""
from __future__ import annotations

import math

import numpy as np


def _logsumexp(a: np.ndarray, axis: int) -> np.ndarray:
    m = a.max(axis=axis, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0).astype(a.dtype)
    return (np.log(np.exp(a - m).sum(axis=axis, keepdims=True)) + m).squeeze(axis)


def _softmax(a: np.ndarray, axis: int) -> np.ndarray:
    e = np.exp(a - a.max(axis=axis, keepdims=True))
    return e / e.sum(axis=axis, keepdims=True)


def _topk_idx(x: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest per row (ties to the lower index), ascending."""
    order = np.argsort(-x, axis=-1, kind="stable")[..., :k]
    return np.sort(order, axis=-1)


def flat_fp32(q, k, v, *, tile: int = 64, exact_leaves: int = 64, curvature: str = "lin",
              tile_chunk: int = 32, leaf: int = 16, scale: float | None = None,
              select: str = "max", tiles: slice | None = None, return_logz: bool = False):
    """q [N,D], k/v [M,D] float arrays -> out [N,D] float32 (h3/htrc_flat.py:279-388).
    ``tiles`` restricts the computation to a slice of query tiles (rows outside are
    left at zero); bench.py uses it to time a bounded sample."""
    if select not in ("max", "bound"):
        raise ValueError("select must be max or bound")
    if curvature not in ("lin", "iso"):
        raise ValueError("curvature must be lin or iso")
    q = np.asarray(q, dtype=np.float32)
    k = np.asarray(k, dtype=np.float32)
    v = np.asarray(v, dtype=np.float32)
    n, d = q.shape
    scale = np.float32(1.0 / math.sqrt(d) if scale is None else scale)
    m = k.shape[0]
    nb = m // leaf
    pre = nb * leaf
    if nb <= 0:
        raise ValueError("flat attention needs at least one full leaf")
    kf, vf = np.ascontiguousarray(k[:pre]), np.ascontiguousarray(v[:pre])
    k3, v3 = kf.reshape(nb, leaf, d), vf.reshape(nb, leaf, d)
    tail = m - pre
    kt, vt = (k[pre:], v[pre:]) if tail else (None, None)
    kn2 = (k3 * k3).sum(-1) if curvature == "iso" else None
    nt = -(-n // tile)
    npad = nt * tile
    qs = q
    valid = np.ones((npad,), np.float32)
    if npad > n:
        qs = np.concatenate([q, np.repeat(q[-1:], npad - n, 0)], 0)
        valid[n:] = 0.0
    qt = qs.reshape(nt, tile, d)
    vw = valid.reshape(nt, tile)
    mu = (qt * vw[..., None]).sum(1) / vw.sum(1, keepdims=True)
    kx_n = min(int(exact_leaves), nb)
    out = np.zeros((npad, d), np.float32)
    logz = np.zeros((npad,), np.float32)
    ar = np.arange(leaf)
    sel_tiles = range(nt) if tiles is None else range(*tiles.indices(nt))
    t_lo, t_hi = sel_tiles.start, sel_tiles.stop
    for t0 in range(t_lo, t_hi, tile_chunk):
        t1 = min(t_hi, t0 + tile_chunk)
        tc = t1 - t0
        mu_c, q_c = mu[t0:t1], qt[t0:t1]
        a = ((mu_c @ kf.T) * scale).reshape(tc, nb, leaf)
        lz = _logsumexp(a, -1)
        w = _softmax(a, -1)
        wb = w.transpose(1, 0, 2)
        g = np.matmul(wb, k3) * scale                         # [nb, tc, d]
        vb = np.matmul(wb, v3)
        dq = q_c - mu_c[:, None, :]
        lg = np.matmul(dq, g.transpose(1, 2, 0)) + lz[:, None, :]   # [tc, T, nb]
        if curvature == "iso":
            tr = (w * kn2[None]).sum(-1) * (scale * scale) - np.square(g).sum(-1).T
            lg += (0.5 / d) * np.maximum(tr, 0.0)[:, None, :] * np.square(dq).sum(-1)[:, :, None]
        if kx_n > 0:
            if select == "bound":
                r = np.linalg.norm(dq, axis=-1).max(1)
                sel = lz + r[:, None] * np.linalg.norm(g, axis=-1).T
            else:
                sel = lg.max(1)
            idx = _topk_idx(sel, kx_n)
            np.put_along_axis(lg, np.broadcast_to(idx[:, None, :], (tc, tile, kx_n)), -np.inf, axis=2)
        mf = lg.max(-1)
        mfs = np.where(np.isfinite(mf), mf, 0.0).astype(np.float32)
        p = np.exp(lg - mfs[..., None])
        zf = p.sum(-1)
        nf = np.matmul(p, vb.transpose(1, 0, 2))
        parts_k, parts_v = [], []
        if kx_n > 0:
            tok = (idx[..., None] * leaf + ar).reshape(tc, kx_n * leaf)
            parts_k.append(kf[tok])
            parts_v.append(vf[tok])
        if tail:
            parts_k.append(np.broadcast_to(kt[None], (tc,) + kt.shape))
            parts_v.append(np.broadcast_to(vt[None], (tc,) + vt.shape))
        if parts_k:
            kx = np.concatenate(parts_k, 1) if len(parts_k) > 1 else parts_k[0]
            vx = np.concatenate(parts_v, 1) if len(parts_v) > 1 else parts_v[0]
            le = np.matmul(q_c, kx.transpose(0, 2, 1)) * scale
            me = le.max(-1)
            pe = np.exp(le - me[..., None])
            ze = pe.sum(-1)
            ne = np.matmul(pe, vx)
            mm = np.maximum(mf, me)
            af, ae = np.exp(mf - mm), np.exp(me - mm)
            num = nf * af[..., None] + ne * ae[..., None]
            den = zf * af + ze * ae
        else:
            mm, num, den = mfs, nf, zf
        out[t0 * tile:t1 * tile] = (num / np.maximum(den, 1e-30)[..., None]).reshape(tc * tile, d)
        with np.errstate(divide="ignore"):
            logz[t0 * tile:t1 * tile] = (mm + np.log(den)).reshape(-1)
    if return_logz:
        return out[:n], logz[:n]
    return out[:n]


def dense(q, k, v, scale: float | None = None):
    """Exact softmax attention in float64 -> (out [N,D], logz [N])."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    s = (1.0 / math.sqrt(q.shape[1]) if scale is None else scale) * (q @ k.T)
    m = s.max(-1, keepdims=True)
    e = np.exp(s - m)
    z = e.sum(-1, keepdims=True)
    return e @ v / z, (np.log(z) + m)[:, 0]
